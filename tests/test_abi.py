"""The C ABI on the CPU host (no GPU calls): the library loads, exports every entry point include/dsa_gfx950.h
declares with the ctypes signatures the binding uses, and rejects bad arguments on the host before any launch."""

import ctypes
import os
import re

import pytest

from trnrt_amd import _lib

HERE = os.path.dirname(os.path.abspath(__file__))
HEADER = os.path.join(os.path.dirname(HERE), "include", "dsa_gfx950.h")


def declared() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?\w+[\s\*]+(dsa_\w+)\s*\(", text, flags=re.M)


def test_header_and_binding_agree():
    names = declared()
    assert len(names) >= 11
    assert sorted(names) == sorted(_lib.SIGNATURES), "every declared entry point has a ctypes signature and back"


def test_library_exports_every_symbol():
    lib = _lib.lib()
    for name in declared():
        assert hasattr(lib, name), name
    assert lib.dsa_abi_version() == _lib.ABI_VERSION


def test_one_hip_runtime_when_the_library_is_loaded_first():
    """Opening the library before anything imported torch, then importing torch, leaves one HIP runtime in the
    process (torch's): the loader imports torch first, so the library binds to torch's libamdhip64 instead of
    pulling in ROCm's copy beside it. A fresh interpreter, since this one has torch loaded already."""
    import subprocess
    import sys
    code = ("import re, sys; sys.path.insert(0, %r); from trnrt_amd import _lib; _lib.lib(); import torch; "
            "print(len(set(re.findall(r'\\S*libamdhip64\\S*', open('/proc/self/maps').read()))))"
            % os.path.dirname(HERE))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    assert r.stdout.strip().splitlines()[-1] == "1"


def test_status_strings():
    lib = _lib.lib()
    for s in (0, -1, -2, -3, -4, -99):
        assert lib.dsa_strerror(s)


def test_layer_status_checks_its_outputs():
    # null output pointers are refused before any HIP call
    lib = _lib.lib()
    assert lib.dsa_layer_status(ctypes.c_void_p(16), None, None, 0, None) == _lib.DSA_EINVAL


def test_host_side_argument_checks():
    lib = _lib.lib()
    null = None
    # null pointers and bad sizes are refused before any HIP call
    assert lib.dsa_indexer_decode(null, null, null, null, null, null, null, null, 1, 64, 128, 1, 64, 2, 64, null) == -1
    p = ctypes.c_void_p(16)  # never dereferenced: every call below fails its host checks
    assert lib.dsa_indexer_decode(p, p, p, p, p, p, null, p, 1, 64, 96, 1, 64, 2, 64, null) == -2  # D != 128
    assert lib.dsa_indexer_decode(p, p, p, p, p, p, null, p, 1, 64, 128, 1, 48, 2, 48, null) == -2  # page 48
    assert lib.dsa_indexer_decode(p, p, p, p, p, p, null, p, 1, 65, 128, 1, 64, 2, 64, null) == -2  # Hi 65
    assert lib.dsa_indexer_decode(p, p, p, p, p, p, null, p, 1, 64, 128, 1, 64, 2, 128, null) == -1  # stride > cap
    assert lib.dsa_topk(p, null, p, p, null, 0, 1, 100, 100, 0, 1, null) == -1  # keep 0
    assert lib.dsa_topk(p, p, p, p, null, 0, 2, 1 << 20, 1 << 20, 2048, 1, null) == -3  # no workspace
    assert lib.dsa_topk(p, p, p, p, p, 100, 2, 4096, 4096, 2048, 1, null) == -3  # workspace too small
    assert lib.dsa_workspace_clear(ctypes.c_void_p(8), 64, null) == -1  # misaligned
    assert lib.dsa_topk(p, p, p, p, null, 0, 2, 1 << 20, 1 << 20, 2048, 0, null) == -2  # long rows need vis_only
    # sparse MLA: exactly one slot form, 576 / 512 widths, heads in 16s
    args = [p, p, p, p, p, p, p, p, p, null, p, null, 0, 1, 16, 576, 512, 64, 4, 64, 8, 0.1, 1, null]
    assert lib.dsa_sparse_mla_decode(*args) == -1  # both forms given
    args2 = list(args)
    args2[6], args2[7] = None, None
    args2[14] = 24
    assert lib.dsa_sparse_mla_decode(*args2) == -2  # 24 heads
    args3 = list(args)
    args3[6], args3[7] = None, None
    args3[24 - 9] = 640
    assert lib.dsa_sparse_mla_decode(*args3) == -2  # Dqk 640


def test_supported_and_workspace():
    lib = _lib.lib()
    assert lib.dsa_topk_supported(32768, 2048, 1) == 1
    assert lib.dsa_topk_supported(1 << 20, 2048, 1) == 1
    assert lib.dsa_topk_supported(1 << 20, 2048, 0) == 0
    # one level: the histograms, the per-row meta and the candidate lists
    assert 8 * 4096 * 4 + 8 * 16 * 2048 * 4 <= _lib.workspace_bytes(_lib.DSA_WS_TOPK, 8, 64, 2048, 32768) < 2 << 20
    assert _lib.workspace_bytes(_lib.DSA_WS_TOPK, 4, 64, 2048, 1 << 20) > 4 * (1 << 20) // 64 * 4
    sp = lib.dsa_default_splits(8, 64, 2048)
    assert 1 <= sp <= 32
    ws = _lib.workspace_bytes(_lib.DSA_WS_ATTENTION, 8, 64, 2048, 0, 0)
    assert ws >= (8 * sp * 64 * 512 * 4 if sp > 1 else 0)


def test_check_maps_status_to_the_reference_exceptions():
    with pytest.raises(ValueError):
        _lib.check(-1, "x")
    with pytest.raises(NotImplementedError):
        _lib.check(-2, "x")
    with pytest.raises(RuntimeError):
        _lib.check(-4, "x")
    _lib.check(0, "x")


def test_prefill_host_checks():
    lib = _lib.lib()
    p = ctypes.c_void_p(16)
    null = None
    assert lib.dsa_indexer_prefill(p, p, p, p, p, null, 4, 64, 128, 100, 100, 0.1, null) == -1  # no output
    assert lib.dsa_indexer_prefill(p, p, p, p, p, p, 4, 64, 128, 100, 99, 0.1, null) == -1  # stride < P
    assert lib.dsa_indexer_prefill(p, p, p, p, p, p, 4, 64, 128, 100, 100, 0.0, null) == -1  # scale 0
    assert lib.dsa_indexer_prefill(p, p, p, p, p, p, 4, 65, 128, 100, 100, 0.1, null) == -2  # Hi 65
    assert lib.dsa_indexer_prefill(p, p, p, p, p, p, 4, 64, 64, 100, 100, 0.1, null) == -2  # D 64
    assert lib.dsa_indexer_prefill(p, p, p, p, p, p, 0, 64, 128, 100, 100, 0.1, null) == 0  # nothing to do
    assert lib.dsa_indexer_prefill_fp8(p, p, p, p, p, p, null, 4, 64, 128, 100, 100, 0.1, null) == -1  # no output
    assert lib.dsa_indexer_prefill_fp8(p, null, p, p, p, p, p, 4, 64, 128, 100, 100, 0.1, null) == -1  # no q scale
    assert lib.dsa_indexer_prefill_fp8(p, p, p, p, p, p, p, 4, 64, 96, 100, 100, 0.1, null) == -2  # D 96
    assert lib.dsa_indexer_prefill_fp8(p, p, p, p, p, p, p, 0, 64, 128, 100, 100, 0.1, null) == 0


def test_cache_write_host_checks():
    lib = _lib.lib()
    p = ctypes.c_void_p(16)
    null = None
    assert lib.dsa_cache_write(p, 0, p, p, null, 4, 576, 100, 1, 448.0, null) == -1  # per-token without a scale
    assert lib.dsa_cache_write(p, 0, p, p, p, 4, 576, 100, 1, 500.0, null) == -1  # fp8_max above 448
    assert lib.dsa_cache_write(p, 0, p, p, p, 4, 20, 100, 1, 448.0, null) == -2  # width not a multiple of 8
    assert lib.dsa_cache_write(p, 0, p, p, p, 4, 1032, 100, 1, 448.0, null) == -2  # width above 1024
    assert lib.dsa_cache_write(p, 0, p, p, p, 0, 576, 100, 1, 448.0, null) == 0  # nothing to do


def test_prefill_select_and_pooled_layer_host_checks():
    """Argument checks of dsa_prefill_select and dsa_pooled_decode_layer, which return before any launch."""
    lib = _lib.lib()
    p = ctypes.c_void_p(16)
    null = None
    ws = lib.dsa_prefill_select_workspace_bytes(4, 67584, 67584, 2048, 0, 0)
    assert ws > 0 and lib.dsa_prefill_select_workspace_bytes(4, 0, 0, 2048, 0, 0) == 0
    assert lib.dsa_prefill_select_workspace_bytes(4, 67584, 67583, 2048, 0, 0) == 0  # stride < P
    big = ctypes.c_size_t(ws)
    args = lambda **k: dict(dict(q=p, qs=p, w=p, k=p, ks=p, npool=p, sc=p, pools=p, cnt=p, vals=p, ws=p, wsb=big, N=4,
                                 Hi=64, D=128, P=67584, stride=67584, keep=2048, scale=0.1, tile=0), **k)

    def call(a):
        return lib.dsa_prefill_select(a["q"], a["qs"], a["w"], a["k"], a["ks"], a["npool"], a["sc"], a["pools"],
                                      a["cnt"], a["vals"], a["ws"], a["wsb"], a["N"], a["Hi"], a["D"], a["P"],
                                      a["stride"], a["keep"], a["scale"], a["tile"], null)

    assert call(args(vals=null)) == -1  # no output
    assert call(args(stride=67583)) == -1  # stride < P
    assert call(args(scale=0.0)) == -1
    assert call(args(tile=-1)) == -1
    assert call(args(Hi=65)) == -2
    assert call(args(D=64)) == -2
    assert call(args(wsb=ctypes.c_size_t(ws - 1))) == -3  # workspace too small
    # the memory-bounded form (scores null) holds its score tiles in the workspace
    own = lib.dsa_prefill_select_workspace_bytes(4, 67584, 67584, 2048, 0, 1)
    assert own >= ws + 4 * 67584 * 4
    assert call(args(sc=null)) == -3
    assert call(args(N=0)) == 0
    pw = lib.dsa_pooled_workspace_bytes(8, 64, 512, 8192, 4, 0)
    assert pw > 0 and lib.dsa_pooled_workspace_bytes(8, 64, 512, 8192, 1, 0) == 0
    pwb = ctypes.c_size_t(pw)

    def layer(kp=4, H=64, Dqk=512, page_size=64, wsb=pwb, B=8, table=p):
        return lib.dsa_pooled_decode_layer(p, p, p, p, p, p, table, p, p, p, p, p, p, p, p, wsb, B, 32, H, Dqk, 512,
                                           page_size, 4097, kp, 512, 0.0625, 0, null)

    assert layer(table=null) == -1
    assert layer(kp=3) == -2 and layer(kp=1) == -2 and layer(page_size=66) == -2
    assert layer(H=40) == -2 and layer(Dqk=256) == -2
    assert layer(wsb=ctypes.c_size_t(pw - 1)) == -3
    assert layer(B=0) == 0
