"""Host-side grouped schedule of the Block-ELL gather GEMM (tmac_bell_group_schedule).

The grouped forward kernel sums each output block over the schedule's steps
where that output is active; parity with the gather kernel (same sums in the
same order) rests on the properties checked here: every member's active steps
are exactly its own list, ascending, with the right value block; every output
block appears in exactly one group; unions are ascending and groups longest
first; the pad member of a short last group is never active.
"""
import ctypes
from pathlib import Path

import numpy as np
import pytest

from titans_core.kernels import _lib
from titans_core.kernels.block_ell import BlockELLPattern

GOLDEN = Path(__file__).resolve().parent / "golden"


def schedule(col_idx, n_bcol, direction, group):
    n_brow, width = col_idx.shape
    n_out = n_bcol if direction == 0 else n_brow
    ng = (n_out + group - 1) // group
    cap = n_brow * width
    gp = np.zeros(ng + 1, np.int32)
    go = np.zeros(ng * group, np.int32)
    st = np.zeros(cap * (1 + group), np.int32)
    a, b = ctypes.c_int(), ctypes.c_int()
    rc = _lib.lib().tmac_bell_group_schedule(np.ascontiguousarray(col_idx, np.int32).ctypes.data,
                                             n_brow, n_bcol, width, direction, group, gp.ctypes.data,
                                             go.ctypes.data, st.ctypes.data, cap, ctypes.byref(a),
                                             ctypes.byref(b))
    assert rc == 0
    assert a.value == ng
    return gp, go, st[: b.value * (1 + group)].reshape(-1, 1 + group)


def lists(col_idx, n_bcol, direction):
    """Per output block: [(input block, value block)] ascending, from the definition."""
    n_brow, width = col_idx.shape
    if direction == 0:
        out = [[] for _ in range(n_bcol)]
        for r in range(n_brow):
            for s, c in enumerate(col_idx[r]):
                out[c].append((r, r * width + s))
    else:
        out = [[(int(c), r * width + s) for s, c in enumerate(col_idx[r])] for r in range(n_brow)]
    return out


CASES = [(40, 160, 40), (10, 40, 20), (40, 10, 5), (3, 5, 2), (7, 9, 3), (1, 1, 1), (70, 4, 3),
         (5, 161, 17)]


@pytest.mark.parametrize("n_brow,n_bcol,width", CASES)
@pytest.mark.parametrize("direction", [0, 1])
@pytest.mark.parametrize("group", [2, 4])
def test_schedule_properties(n_brow, n_bcol, width, direction, group):
    pat = BlockELLPattern.sample(n_brow * 7 + width, n_brow, n_bcol, width)
    gp, go, st = schedule(pat.col_idx, n_bcol, direction, group)
    want = lists(pat.col_idx, n_bcol, direction)
    seen = []
    lens = np.diff(gp)
    assert np.all(lens[:-1] >= lens[1:]), "groups are not longest first"
    for g in range(len(gp) - 1):
        rows = st[gp[g]:gp[g + 1]]
        assert np.all(np.diff(rows[:, 0]) > 0), "union not ascending"
        assert np.all((rows[:, 1:] >= 0).any(axis=1)), "a step with no active member"
        for j in range(group):
            o = go[g * group + j]
            if o < 0:
                assert np.all(rows[:, 1 + j] < 0), "pad member active"
                continue
            seen.append(o)
            act = rows[rows[:, 1 + j] >= 0][:, [0, 1 + j]]
            assert [tuple(map(int, x)) for x in act] == want[o], f"member {o} steps differ from its list"
    n_out = n_bcol if direction == 0 else n_brow
    assert sorted(seen) == list(range(n_out))
    # the union size is the number of distinct inputs of the group
    for g in range(len(gp) - 1):
        members = [o for o in go[g * group:(g + 1) * group] if o >= 0]
        assert lens[g] == len({i for o in members for i, _ in want[o]})


def test_config2_pair_unions():
    """Config 2's committed pattern: pairing cuts the activation-tile copies of a
    row tile from 1600 (one per stored block) to 1172 union steps (841 in fours);
    the steps still carry all 1600 blocks."""
    ci = np.load(GOLDEN / "bell_col_idx_cfg2.npy")
    gp, go, st = schedule(ci, 160, 0, 2)
    assert len(st) == 1172
    assert int((st[:, 1:] >= 0).sum()) == 1600
    gp4, _, st4 = schedule(ci, 160, 0, 4)
    assert len(st4) == 841


def test_schedule_errors():
    L = _lib.lib()
    ci = np.array([[0, 2], [1, 2]], np.int32)
    buf = np.zeros(64, np.int32)
    a, b = ctypes.c_int(), ctypes.c_int()

    def call(col=ci, n_bcol=3, direction=0, group=2, cap=4, null=False):
        return L.tmac_bell_group_schedule(col.ctypes.data, col.shape[0], n_bcol, col.shape[1], direction,
                                          group, buf.ctypes.data, None if null else buf.ctypes.data,
                                          buf.ctypes.data, cap, ctypes.byref(a), ctypes.byref(b))

    assert call() == 0
    assert call(group=3) == -8
    assert call(direction=2) == -8
    assert call(null=True) == -1
    assert call(cap=1) == -7
    assert call(col=np.array([[2, 0], [1, 2]], np.int32)) == -3  # unsorted row
    assert call(n_bcol=2) == -3                                   # index out of range


def tile_order(gp, M):
    n = ctypes.c_int()
    L = _lib.lib()
    assert L.tmac_bell_group_tile_order(gp.ctypes.data, len(gp) - 1, M, None, 0, ctypes.byref(n)) == 0
    out = np.full(n.value, 7, np.int32)
    assert L.tmac_bell_group_tile_order(gp.ctypes.data, len(gp) - 1, M, out.ctypes.data, n.value,
                                        ctypes.byref(n)) == 0
    return out


@pytest.mark.parametrize("M", [1, 511, 512, 8192, 17920, 32768])
@pytest.mark.parametrize("pat_case", ["cfg2", (10, 40, 20), (40, 10, 5), (3, 5, 2)])
def test_tile_order_properties(M, pat_case):
    """The balanced order is a per-XCD permutation of the launch's tiles laid out in
    rounds of n_slots (holes -1): every tile exactly once, in its own XCD's range, at
    most one per slot and round; its makespan (steps + 2 per tile) never exceeds the
    round-robin deal's."""
    if pat_case == "cfg2":
        ci, n_bcol = np.load(GOLDEN / "bell_col_idx_cfg2.npy"), 160
    else:
        n_brow, n_bcol, width = pat_case
        ci = BlockELLPattern.sample(1, n_brow, n_bcol, width).col_idx
    gp, _, _ = schedule(ci, n_bcol, 0, 2)
    ng = len(gp) - 1
    n_tiles = -(-M // 512) * ng
    per_xcd = -(-n_tiles // 8)
    n_slots = min(per_xcd, 32)
    n_rounds = -(-per_xcd // n_slots)
    order = tile_order(gp, M)
    assert order.shape == (8 * n_rounds * n_slots,)
    lay = order.reshape(8, n_rounds, n_slots)
    cost = lambda t: int(gp[t % ng + 1] - gp[t % ng]) + 2  # noqa: E731
    for x in range(8):
        got = lay[x][lay[x] >= 0]
        want = np.arange(x * per_xcd, min(n_tiles, (x + 1) * per_xcd))
        assert sorted(got.tolist()) == want.tolist()
        assert (lay[x] >= -1).all()
        load = [sum(cost(t) for t in lay[x][:, s] if t >= 0) for s in range(n_slots)]
        rr = [sum(cost(t) for t in want[s::n_slots]) for s in range(n_slots)]
        assert max(load) <= max(rr)


def test_tile_order_errors():
    L = _lib.lib()
    gp = np.array([0, 5, 3], np.int32)  # decreasing offsets
    n = ctypes.c_int()
    assert L.tmac_bell_group_tile_order(gp.ctypes.data, 2, 100, None, 0, ctypes.byref(n)) == -8
    gp = np.array([0, 5, 9], np.int32)
    assert L.tmac_bell_group_tile_order(gp.ctypes.data, 2, 0, None, 0, ctypes.byref(n)) == -2
    assert L.tmac_bell_group_tile_order(None, 2, 100, None, 0, ctypes.byref(n)) == -1
    assert L.tmac_bell_group_tile_order(gp.ctypes.data, 2, 100, None, 0, ctypes.byref(n)) == 0
    out = np.zeros(n.value, np.int32)
    assert L.tmac_bell_group_tile_order(gp.ctypes.data, 2, 100, out.ctypes.data, n.value - 1,
                                        ctypes.byref(n)) == -7
