"""The decode workspace's barrier block (csrc/dsa_common.h, csrc/dsa_fused.hip), checked without a GPU: per XCD
WS_SYNC_LINES 128-byte lines, word 0 of each a copy of the XCD's barrier counter, the status words in the first line,
the whole block WS_SYNC_BYTES at the workspace's start. Every arrival and every exit adds to all copies (lanes 0 ..
WS_SYNC_LINES - 1 of the workgroup, one copy each) and each workgroup polls and reads its base from copy j mod
WS_SYNC_LINES, so the copies hold equal values between launches; the GPU tests read the block with the layout named
here."""

import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
COMMON = (ROOT / "trnrt_amd" / "csrc" / "dsa_common.h").read_text()
FUSED = (ROOT / "trnrt_amd" / "csrc" / "dsa_fused.hip").read_text()


def _const(name: str) -> str:
    m = re.search(rf"constexpr int {name} = ([^;]+);", COMMON)
    assert m, name
    return m.group(1)


def test_block_layout():
    lines, line_words = int(_const("WS_SYNC_LINES")), int(_const("WS_SYNC_LINE_WORDS"))
    assert line_words * 4 == 128  # a copy per 128-byte line
    assert _const("WS_SYNC_WORDS") == "WS_SYNC_LINE_WORDS * WS_SYNC_LINES"
    assert _const("WS_SYNC_BYTES") == "8 * 4 * WS_SYNC_WORDS"
    assert int(_const("WS_SYNC_GAVE_UP")) < line_words and int(_const("WS_SYNC_TWO_EXCHANGE")) < line_words
    gpu = (ROOT / "tests" / "test_gpu_fused.py").read_text()
    assert f"SYNC_LINES, LINE_WORDS = {lines}, {line_words}" in gpu


def test_every_copy_counted():
    body = FUSED[FUSED.index("__device__ __forceinline__ FuSync fu_sync_begin"):FUSED.index("// Block-wide over 512")]
    assert "w + WS_SYNC_LINE_WORDS * (j % WS_SYNC_LINES)" in body  # the copy this workgroup polls
    # the arrival (fu_barrier) and the exit's remaining arrivals (fu_exit) go to every copy, one lane each
    assert body.count("if (threadIdx.x < WS_SYNC_LINES)") == 2
    assert body.count("sy.w + WS_SYNC_LINE_WORDS * threadIdx.x") == 2
    assert "unsigned* ctr = sy.rep;" in body
    # every kernel with these barriers picks its copy by its workgroup index within the XCD
    assert FUSED.count("fu_sync_begin(a.sync + x * WS_SYNC_WORDS, j)") == FUSED.count("fu_sync_begin(") - 1
