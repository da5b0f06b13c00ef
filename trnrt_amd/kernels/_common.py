"""Argument checks shared by the operator wrappers: device tensors only (the HIP path is the only path), the
dtypes and layouts the C ABI expects, and the current HIP stream."""

from __future__ import annotations

import torch

FP8 = torch.float8_e4m3fn  # OCP e4m3fn: gfx950's FP8 and the reference's CPU cache dtype (model_runner.py:54-70)


def on_gpu(*ts: torch.Tensor | None) -> torch.device:
    """The common GPU device of the tensors; RuntimeError for host tensors (there is no CPU path)."""
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                "trnrt_amd DSA kernels run on the GPU only (libdsa_gfx950.so); got a tensor on " + str(t.device)
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise ValueError("no tensor arguments")
    return dev


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def need(t: torch.Tensor, name: str, dtype: torch.dtype | tuple, shape: tuple | None = None) -> torch.Tensor:
    """t itself if it has the dtype (one of), shape (None entries free) and is contiguous; ValueError otherwise."""
    dts = dtype if isinstance(dtype, tuple) else (dtype,)
    if t.dtype not in dts:
        raise ValueError(f"{name}: dtype {t.dtype}, expected {' or '.join(map(str, dts))}")
    if shape is not None:
        if t.dim() != len(shape) or any(s is not None and s != d for s, d in zip(shape, t.shape)):
            raise ValueError(f"{name}: shape {tuple(t.shape)}, expected {shape}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    return t


def as_bf16(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.bfloat16 and t.is_contiguous() else t.to(torch.bfloat16).contiguous()


def as_i32(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.int32 and t.is_contiguous() else t.to(torch.int32).contiguous()


def as_f32(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.float32 and t.is_contiguous() else t.float().contiguous()


def fp8_bytes(t: torch.Tensor, name: str) -> torch.Tensor:
    """The e4m3fn cache as a contiguous tensor (float8_e4m3fn or its uint8 bit pattern)."""
    if t.dtype not in (FP8, torch.uint8):
        raise ValueError(f"{name}: dtype {t.dtype}, expected float8_e4m3fn (or its uint8 bits)")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    return t


# Zero-filled workspaces kept per (device, stream, use) and reused by the functional surfaces when the caller passes
# none: every call leaves the regions that must start at zero at zero again, so one zero fill serves every later call
# on the same stream (calls on one stream never overlap; each stream has its own). A call needing more grows it: a
# new zero-filled buffer on the same stream (the old one returns to torch's stream-ordered allocator).
_WORKSPACES: dict = {}


def cached_workspace(device: torch.device, nbytes: int, use: str) -> torch.Tensor:
    """A zero-filled uint8 device buffer of at least nbytes for `use` on the current stream of `device`."""
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream_ptr(device), use)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = zeroed_workspace(max(int(nbytes), 256), device)
        _WORKSPACES[key] = ws
    return ws


def zeroed_workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """A new uint8 device buffer of nbytes (a multiple of 256) zero-filled by the library's dsa_workspace_clear on the
    current stream, which also records it as zero, so its first call does not fill it again."""
    from .. import _lib

    n = (int(nbytes) + 255) // 256 * 256
    ws = torch.empty(n, dtype=torch.uint8, device=device)
    _lib.check(_lib.lib().dsa_workspace_clear(ws.data_ptr(), n, stream_ptr(device)), "dsa_workspace_clear")
    return ws
