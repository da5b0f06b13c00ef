"""Shared helpers of the GPU parity tests."""

import sys

import torch


def say(*a):
    """Names the case before a GPU step (flushed, so a crash still shows which case ran)."""
    print(*a, flush=True)
    sys.stdout.flush()


def row_rel_err(got: torch.Tensor, ref: torch.Tensor, live: torch.Tensor) -> float:
    """max over rows of max|got - ref| / max|ref| over the live entries (the reference's error form,
    trnrt tests/test_dsa_index.py:100)."""
    worst = 0.0
    for r in range(ref.shape[0]):
        m = live[r]
        if not m.any():
            continue
        d = (got[r][m] - ref[r][m]).abs().max() / ref[r][m].abs().max().clamp(min=1e-30)
        worst = max(worst, float(d))
    return worst


def assert_attention_close(out: torch.Tensor, ref: torch.Tensor, tol: float = 2e-2):
    """The north star's bound for the bf16 attention output: within tol absolute + tol relative."""
    torch.testing.assert_close(out.float().cpu(), ref.float().cpu(), atol=tol, rtol=tol)


def launched_kernels(step) -> list:
    """Names of the library kernels one call of step() launches, in order (the library's timing hooks,
    dsa_timing_begin / dsa_timing_end, with HIP events from the runtime)."""
    import ctypes

    from trnrt_amd import _lib

    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
    pairs = 16
    evs = []
    for _ in range(2 * pairs):
        e = ctypes.c_void_p()
        assert hip.hipEventCreate(ctypes.byref(e)) == 0
        evs.append(e)
    arr = (ctypes.c_void_p * (2 * pairs))(*[e.value for e in evs])
    lib = _lib.lib()
    lib.dsa_timing_begin(arr, pairs)
    try:
        step()
    finally:
        n = lib.dsa_timing_end()
    names = [lib.dsa_timing_kernel_name(k).decode() for k in range(min(n, pairs))]
    torch.cuda.synchronize()
    for e in evs:
        hip.hipEventDestroy(e.value)
    return names
