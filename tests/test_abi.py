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


def test_status_strings():
    lib = _lib.lib()
    for s in (0, -1, -2, -3, -4, -99):
        assert lib.dsa_strerror(s)


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
