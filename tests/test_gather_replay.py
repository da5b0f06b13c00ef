"""A CPU replay of the attention gather's lane indexing in csrc/dsa_fused.hip (`fu_attend`), for every slot count of
the three FuAtt forms the library instantiates (16 heads x 576-byte rows, 32 x 576, and the pooled 32 x 512 with its
tail rows): each wave's loads k = wave, wave + 8, ... while 64 k < padded x KPIECES, lane l of load k filling 16 bytes
of the row tile at 1024 k + 16 l from row u / KPIECES, piece u % KPIECES of unit u = 64 k + l, the row and piece
advanced per load as the kernel advances them (by DR rows and DP pieces, with a carry). Checked: the stepped
(row, piece) equals the division's, every lane's row is inside the split's padded rows (whose slot ids the split's
list holds) and inside the tile's CAP rows, the piece read is inside the cache row, the LDS bytes written stay
inside the row tile, and NI loads per lane cover every load of the split. A load with lanes past the padded rows would read slot ids past the written list and load
from outside the cache, the fault this replay once found. The constants are read from the source, so a change there
is replayed here."""

import re
from pathlib import Path

import pytest

SRC = Path(__file__).resolve().parents[1] / "trnrt_amd" / "csrc" / "dsa_fused.hip"


def _const(text: str, name: str) -> int:
    m = re.search(rf"constexpr int [^;]*\b{name} = ([^,;]+)[,;]", text)
    assert m, name
    expr = m.group(1)
    return int(eval(expr, {}, CONSTS))  # the constants are integer expressions of earlier ones


CONSTS: dict = {}


def _load_consts():
    text = SRC.read_text()
    common = (SRC.parent / "dsa_common.h").read_text()
    CONSTS["WAVE"] = _const(common, "WAVE")
    for name in ("FU_THREADS", "FU_CH", "FU_DQK"):
        CONSTS[name] = _const(text, name)
    CONSTS["FU_WAVES"] = CONSTS["FU_THREADS"] // CONSTS["WAVE"]
    # the struct's own formulas must be the ones replayed below
    assert "static constexpr int SPLIT = 4096 / HPW;" in text
    assert "static constexpr int CAP = SPLIT + (XT ? FU_CH : 0);" in text
    assert "static constexpr int KPIECES = PIECES + 1;" in text
    assert "const int padded = (n_slots + FU_CH - 1) / FU_CH * FU_CH;" in text
    assert "constexpr int NI = (AT::CAP * KPIECES + FU_THREADS - 1) / FU_THREADS;" in text
    assert "sl[i] = slot_l[min(row, AT::CAP - 1)];" in text
    assert "const int k = wave + FU_WAVES * i;\n      if (k * WAVE < units) {" in text
    assert "const uint8_t* src = a.kv + (size_t)sl[i] * DQK + 16 * min(pc, PIECES - 1);" in text
    # the issue loop steps the piece alone (pc += DP, less KPIECES on a carry), as the slot loop steps it
    assert "      pc += DP;\n      if (pc >= KPIECES) pc -= KPIECES;\n" in text
    assert "(__attribute__((address_space(3))) void*)(kt + 1024 * k), 16, 0, 0);" in text
    return CONSTS


# (HPW, DQK, XT): the instances the library launches (decode_fused_kernel, decode_attend_kernel and its pooled form)
FORMS = [(16, 576, False), (32, 576, False), (32, 512, True)]


@pytest.mark.parametrize("hpw,dqk,xt", FORMS)
def test_gather_lanes_stay_inside_the_padded_rows(hpw, dqk, xt):
    c = _load_consts()
    WAVE, WAVES, CH = c["WAVE"], c["FU_WAVES"], c["FU_CH"]
    split = 4096 // hpw
    cap = split + (CH if xt else 0)
    pieces = dqk // 16
    kpieces = pieces + 1
    krow = 16 * kpieces
    tile_bytes = cap * krow  # the rows' LDS, before the slot list / P at L_P
    DR, DP = WAVES * WAVE // kpieces, WAVES * WAVE % kpieces
    for n_slots in range(1, cap + 1):
        padded = (n_slots + CH - 1) // CH * CH
        assert padded <= cap, (n_slots, padded, cap)
        units = padded * kpieces
        assert units % WAVE == 0, f"a padded split's pieces do not fill whole loads ({n_slots} slots)"
        ni = (cap * kpieces + WAVES * WAVE - 1) // (WAVES * WAVE)  # NI: loads per lane at most
        loads = 0
        for wave in range(WAVES):
            for lane in range(WAVE):
                row, pc = (WAVE * wave + lane) // kpieces, (WAVE * wave + lane) % kpieces
                pc0 = pc
                for i in range(ni):
                    k = wave + WAVES * i
                    assert 0 <= min(row, cap - 1) < cap  # the slot read, taken for every i
                    if k * WAVE < units:
                        u = WAVE * k + lane
                        assert (row, pc) == divmod(u, kpieces), (n_slots, wave, lane, k)
                        assert row < padded and row < cap, f"{n_slots} slots: lane {lane} of load {k} reads row {row}"
                        assert 0 <= min(pc, pieces - 1) < pieces
                        assert 1024 * k + 16 * lane + 16 <= tile_bytes, f"{n_slots} slots: LDS past the row tile"
                        loads += lane == 0
                    # the issue loop's piece, stepped without the row: the same sequence
                    assert pc == (pc0 + DP * i) % kpieces
                    row += DR
                    pc += DP
                    if pc >= kpieces:
                        pc -= kpieces
                        row += 1
        assert loads == units // WAVE, f"{n_slots} slots: {loads} loads for {units // WAVE} (NI too small)"


def test_an_odd_padding_would_be_caught():
    """The replay's own check: padding a split to 32 rows (the faulting form) leaves lanes past the padded rows for
    some slot count of the pooled form, which the row check above would report."""
    c = _load_consts()
    WAVE = c["WAVE"]
    kpieces = 512 // 16 + 1
    bad = [n for n in range(1, 193) if ((n + 31) // 32 * 32 * kpieces) % WAVE]
    assert bad, "padding to 32 rows should leave partial loads"
