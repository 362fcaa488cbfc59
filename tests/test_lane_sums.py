"""CPU check of the transposed lane reduction `lane_sums` / `lane_rank_offset` (csrc/mm_common.h)
that the P/Q kernels use for their R coupling sums over a channel's LPR lanes.

The test decodes the DPP controls the header names (quad_perm, row_half_mirror, row_mirror) into
lane permutations, derives each lane's rank order t ^ c_k from the stage rule (a lane and its
partner at transposed stage j hold each other's halves of every 2^(log2 R - j)-block swapped; the
symmetric stages pair lanes with the same order), simulates the kernel's stages on symbolic
partials -- the transposed adds, the symmetric adds and the gather -- and requires that every lane
ends with the complete sum of rank t ^ c_k at position t. The packed c_k tables and stage controls
written in the header must be the ones derived here."""
import pathlib
import re

import pytest

HEADER = pathlib.Path(__file__).resolve().parents[1] / "motif-mamba_amd" / "csrc" / "mm_common.h"

# DPP controls of the stages, outermost first (kLaneStage<LPR, J> in the header).
STAGES = {16: [0x140, 0x141, 0x4E, 0xB1], 8: [0x141, 0x4E, 0xB1], 4: [0x1B, 0xB1]}


def dpp_source(ctrl, lane):
    """The lane whose value `lane` reads under a DPP control (GCN/CDNA encoding)."""
    row, j = lane - lane % 16, lane % 16
    if ctrl <= 0xFF:                                  # quad_perm: 2-bit source per lane of a quad
        return row + (j - j % 4) + ((ctrl >> (2 * (j % 4))) & 3)
    if ctrl == 0x140:                                 # row_mirror
        return row + 15 - j
    if ctrl == 0x141:                                 # row_half_mirror
        return row + (j // 8) * 8 + 7 - j % 8
    raise ValueError(hex(ctrl))


def test_dpp_controls_are_involutions_inside_the_group():
    for lpr, ctrls in STAGES.items():
        for c in ctrls:
            for lane in range(64):
                src = dpp_source(c, lane)
                assert dpp_source(c, src) == lane
                assert src // lpr == lane // lpr, (lpr, hex(c), lane)   # stays inside the channel's lanes


def derive_offsets(lpr, r):
    m = r.bit_length() - 1
    ctrls = STAGES[lpr]
    order = {0: list(range(r))}
    changed = True
    while changed:
        changed = False
        for i in list(order):
            for j, c in enumerate(ctrls):
                k = dpp_source(c, i)
                if j >= m:
                    want = list(order[i])
                else:
                    blk = r >> j
                    want = []
                    for b0 in range(0, r, blk):
                        seg = order[i][b0:b0 + blk]
                        want += seg[blk // 2:] + seg[:blk // 2]
                if k in order:
                    assert order[k] == want, (lpr, r, i, k)
                else:
                    order[k] = want
                    changed = True
    assert sorted(order) == list(range(lpr))
    offs = [order[i][0] for i in range(lpr)]
    for i in range(lpr):
        assert order[i] == [t ^ offs[i] for t in range(r)]      # the order is t ^ c_k
    return offs


def simulate(lpr, r, offs):
    """The kernel's stages on symbolic partials {(lane, rank)}; returns each lane's final x[]."""
    m = r.bit_length() - 1
    ctrls = STAGES[lpr]
    x = [[frozenset([(i, t ^ offs[i])]) for t in range(r)] for i in range(lpr)]
    for j in range(m):                                # transposed stages
        n = r >> j
        x = [[x[i][t] | x[dpp_source(ctrls[j], i)][n // 2 + t] for t in range(n // 2)] for i in range(lpr)]
    for j in range(m, len(ctrls)):                    # symmetric stages
        x = [[x[i][0] | x[dpp_source(ctrls[j], i)][0]] for i in range(lpr)]
    for i_stage in range(m):                          # gather: x[t + h] = partner's x[t]
        j, h = m - 1 - i_stage, 1 << i_stage
        x = [x[i] + [x[dpp_source(ctrls[j], i)][t] for t in range(h)] for i in range(lpr)]
    return x


CASES = [(lpr, r) for lpr in (4, 8, 16) for r in (2, 4, 8) if r <= lpr]


@pytest.mark.parametrize("lpr,r", CASES)
def test_every_lane_gets_every_total_in_its_order(lpr, r):
    offs = derive_offsets(lpr, r)
    x = simulate(lpr, r, offs)
    for i in range(lpr):
        assert len(x[i]) == r
        for t in range(r):
            assert x[i][t] == frozenset((lane, t ^ offs[i]) for lane in range(lpr)), (lpr, r, i, t)


def test_a_wrong_order_fails():
    """The check is not vacuous: swapping two lanes' offsets breaks some total."""
    offs = derive_offsets(8, 4)
    bad = list(offs)
    bad[2], bad[4] = bad[4], bad[2]
    x = simulate(8, 4, bad)
    ok = all(x[i][t] == frozenset((lane, t ^ bad[i]) for lane in range(8)) for i in range(8) for t in range(4))
    assert not ok


def test_header_tables_match():
    text = HEADER.read_text()
    for lpr, r in CASES:
        packed = sum(c << (4 * k) for k, c in enumerate(derive_offsets(lpr, r)))
        assert re.search(rf"0x{packed:x}ull", text, re.IGNORECASE), (lpr, r, hex(packed))
    stage_src = text[text.index("constexpr int kLaneStage"):text.index("template <int LPR, int R>\n__device__ __forceinline__ int lane_rank_offset")]
    # kLaneStage lists the controls of 16, 8 and 4 lanes in that order, outermost stage first.
    got = [int(h, 16) for h in re.findall(r"0x[0-9A-Fa-f]+", stage_src)]
    assert got == STAGES[16] + STAGES[8] + STAGES[4], [hex(v) for v in got]
