"""A CPU replay of the long-row indexer's even work split in csrc/dsa_indexer.hip (`indexer_decode_long_kernel` with
TW = 0, launched by `launch_indexer_long_v`): G workgroups of 4 waves share the batch's live tiles (32-key tiles holding
a position below the row's length), cw = ceil(T / (4 (G - B))) tiles a wave, row b taking ceil(T_b / 4 cw) workgroups
in row order, and the tiles past each row's length are shared out ceil(Q / G) a workgroup, each tail tile's row found
by a binary search over the rows' tail offsets. Checked over ragged, empty, full and odd-stride batches: every live
tile of every row is scored by exactly one wave, no wave holds more than the 64 tiles its page-id lanes and tile
maxima hold, the workgroups that take rows fit in the grid, every tail tile is written exactly once, and no tile is
both. The host's grid formula and the kernel's expressions are checked to be the ones replayed."""

import random
from pathlib import Path

import pytest

SRC = Path(__file__).resolve().parents[1] / "trnrt_amd" / "csrc" / "dsa_indexer.hip"
TILE, WAVES, TW_MAX, MAXB = 32, 4, 64, 256


def test_source_matches_replay():
    text = SRC.read_text()
    for expr in (
        "const int cw = max((T + 4 * (G - B) - 1) / (4 * (G - B)), 1);",
        "const int mt = (Tt + 4 * cw - 1) / (4 * cw);",
        "wrow[1] = (g - Mt) * 4 * cw;",
        "n_live = n_t = max(min(cw, bal[IL_BAL_MAXB + b] - tw0), 0);",
        "tw0 = wrow[1] + wave * cw;",
        "const int qg = (Q + G - 1) / G, u0 = g * qg, u1 = min(u0 + qg, Q);",
        "const int tile = bal[IL_BAL_MAXB + lo] + (u - bal[lo]);",
        "const long need = B + ((long)B * tiles_row + IDX_WAVES * IL_TW_MAX - 1) / (IDX_WAVES * IL_TW_MAX);",
        "const long G = need > 2L * num_cu ? need : 2L * num_cu;",
    ):
        assert expr in text, expr


def _grid(B: int, stride: int, num_cu: int) -> int:
    tiles_row = (stride + TILE - 1) // TILE
    need = B + (B * tiles_row + WAVES * TW_MAX - 1) // (WAVES * TW_MAX)
    return max(need, 2 * num_cu)


def _replay(lengths: list[int], stride: int, num_cu: int = 256):
    B = len(lengths)
    assert B <= MAXB
    G = _grid(B, stride, num_cu)
    tiles_row = (stride + TILE - 1) // TILE
    Tb = [min((min(max(L, 0), stride) + TILE - 1) // TILE, tiles_row) for L in lengths]
    T = sum(Tb)
    cw = max((T + 4 * (G - B) - 1) // (4 * (G - B)), 1)
    assert cw <= TW_MAX
    mt = [(t + 4 * cw - 1) // (4 * cw) for t in Tb]
    Mt = [sum(mt[:i]) for i in range(B)]
    assert sum(mt) <= G
    Pt = [tiles_row - t for t in Tb]
    Ut = [sum(Pt[:i]) for i in range(B)]
    Q = sum(Pt)
    scored = [[0] * tiles_row for _ in range(B)]
    tail = [[0] * tiles_row for _ in range(B)]
    qg = (Q + G - 1) // G
    for g in range(G):
        u0, u1 = g * qg, min(g * qg + qg, Q)
        for u in range(u0, u1):
            lo, hi = 0, B - 1
            while lo < hi:
                mid = (lo + hi + 1) >> 1
                if Ut[mid] <= u:
                    lo = mid
                else:
                    hi = mid - 1
            tile = Tb[lo] + (u - Ut[lo])
            assert Tb[lo] <= tile < tiles_row
            tail[lo][tile] += 1
        rows = [t for t in range(B) if Mt[t] <= g < Mt[t] + mt[t]]
        assert len(rows) <= 1
        if not rows:
            continue
        b = rows[0]
        first = (g - Mt[b]) * 4 * cw
        for wave in range(WAVES):
            tw0 = first + wave * cw
            n = max(min(cw, Tb[b] - tw0), 0)
            assert n <= TW_MAX
            for i in range(n):
                scored[b][tw0 + i] += 1
    for b in range(B):
        for t in range(tiles_row):
            live = t < Tb[b]
            assert scored[b][t] == (1 if live else 0), (b, t)
            assert tail[b][t] == (0 if live else 1), (b, t)
    return G, cw


@pytest.mark.parametrize("seed", range(6))
def test_split_ragged(seed):
    rnd = random.Random(seed)
    stride = rnd.choice([131072, 65540, 40000 + 4 * rnd.randrange(1000)])
    B = rnd.choice([1, 3, 12, 37])
    lengths = [rnd.randrange(0, stride + 1) for _ in range(B)]
    _replay(lengths, stride)


def test_split_config3_shape():
    lengths = [60535, 63048, 100500, 39786, 72509, 75768, 91015, 111039, 124575, 10867, 70236, 35922]
    G, cw = _replay(lengths, 131072)
    assert G == 512 and cw == 14


def test_split_full_and_empty_rows():
    _replay([1 << 20] * 4, 1 << 20)  # config 4: 64 tiles a wave, as the fixed split
    _replay([0] * 5, 70000)  # nothing live: tails only
    _replay([0, 70000, 0, 1, 33], 70000)
    _replay([70001] * 3, 70001)  # a partial last tile (stride not a multiple of 32)


def test_split_max_rows():
    rnd = random.Random(7)
    _replay([rnd.randrange(0, 40001) for _ in range(MAXB)], 40000, num_cu=256)
    _replay([40000] * MAXB, 40000, num_cu=256)  # the grid grows past 2 per CU to keep 64 tiles a wave
