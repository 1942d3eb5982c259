"""Pins of oracle.masks: known answers, closed forms and brute force on small S."""
import itertools

import numpy as np
import pytest

from oracle import masks as om

# Known answers (allowed pairs; non-empty / full / partial 64x64 tiles) computed
# for the configurations this path runs at.
KNOWN_BAND = [
    # S, w, Np, pairs, nonempty, full, partial
    (4096, 512, 16, 2_027_248, 595, 420, 175),
    (4112, 512, 16, 2_035_712, 605, 420, 185),
    (512, 256, 16, 102_768, 33, 18, 15),
    (560, 512, 16, 156_704, 45, 28, 17),
]


@pytest.mark.parametrize("S,w,Np,pairs,ne,full,part", KNOWN_BAND)
def test_band_known_answers(S, w, Np, pairs, ne, full, part):
    m = om.band_mask(S, w, Np)
    assert m.shape == (S, S) and m.dtype == bool
    assert int(m.sum()) == pairs
    k = om.tile_kinds(m, 64, 64)
    assert (int((k > 0).sum()), int((k == 1).sum()), int((k == 2).sum())) == (ne, full, part)


def test_blockwin_known_answers():
    m = om.blockwin_mask(4096, 512, 64, 16)
    assert int(m.sum()) == 2_204_536
    assert int((m != om.band_mask(4096, 512, 16)).sum()) == 177_288
    assert int(om.blockwin_mask(560, 512, 64, 16).sum()) == 165_904


def brute_band(S, w, Np, causal):
    m = np.zeros((S, S), dtype=bool)
    for i in range(S):
        for j in range(S):
            if j < Np:
                m[i, j] = True
            elif i >= Np and abs(i - j) <= w and (not causal or j <= i):
                m[i, j] = True
    return m


@pytest.mark.parametrize("S,w,Np,causal", [
    (1, 0, 0, True), (5, 0, 0, True), (9, 2, 3, True), (9, 2, 3, False), (17, 40, 4, True),
    (17, 40, 4, False), (33, 7, 0, False), (40, 1, 39, True), (64, 16, 8, True), (70, 0, 5, False)])
def test_band_brute_force(S, w, Np, causal):
    assert np.array_equal(om.band_mask(S, w, Np, causal), brute_band(S, w, Np, causal))


@pytest.mark.parametrize("S,w,Np", [(s, w, n) for s in (1, 2, 7, 65, 300) for w in (0, 1, 5, 64, 1000)
                                     for n in (0, 1, 3) if n < s])
def test_band_closed_form_and_row_counts(S, w, Np):
    m = om.band_mask(S, w, Np)
    assert int(m.sum()) == om.band_pair_count(S, w, Np)
    rows = m.sum(axis=1)
    want = [Np if i < Np else Np + min(i - Np, w) + 1 for i in range(S)]
    assert rows.tolist() == want


def test_band_value_errors():
    with pytest.raises(ValueError):
        om.band_mask(16, 4, 16)
    with pytest.raises(ValueError):
        om.band_mask(16, -1, 0)


def intervals_blockwin(S, w, bs, Np, causal):
    """Second statement of the block-window mask: per-row intervals."""
    m = np.zeros((S, S), dtype=bool)
    for i in range(S):
        if i < Np:
            m[i, :] = True
            continue
        m[i, :Np] = True
        r = i - Np
        b0 = (r // bs) * bs
        lo = max(0, b0 - w)
        hi = r + 1 if causal else min(b0 + bs, S - Np)
        m[i, Np + lo:Np + hi] = True
    return m


@pytest.mark.parametrize("S,w,bs,Np,causal", [
    (1, 0, 4, 0, True), (30, 8, 4, 3, True), (30, 8, 4, 3, False), (100, 64, 16, 16, True),
    (100, 5, 64, 0, False), (129, 64, 64, 1, True), (300, 128, 32, 20, False)])
def test_blockwin_loop_matches_intervals(S, w, bs, Np, causal):
    assert np.array_equal(om.blockwin_mask(S, w, bs, Np, causal), intervals_blockwin(S, w, bs, Np, causal))


def brute_tiles(m, tq, tk):
    S = m.shape[0]
    nq, nk = -(-S // tq), -(-S // tk)
    out = np.zeros((nq, nk), dtype=np.uint8)
    for a in range(nq):
        for b in range(nk):
            cnt = 0
            for i in range(a * tq, a * tq + tq):
                for j in range(b * tk, b * tk + tk):
                    if i < S and j < S and m[i, j]:
                        cnt += 1
            out[a, b] = 0 if cnt == 0 else (1 if cnt == tq * tk else 2)
    return out


@pytest.mark.parametrize("S,w,Np,tq,tk", [(40, 5, 3, 8, 8), (41, 5, 3, 8, 16), (100, 20, 10, 32, 16),
                                          (70, 70, 0, 16, 64)])
def test_tile_kinds_brute_force(S, w, Np, tq, tk):
    m = om.band_mask(S, w, Np)
    assert np.array_equal(om.tile_kinds(m, tq, tk), brute_tiles(m, tq, tk))


def test_schedule_covers_every_nonempty_subtile_once():
    S, w, Np = 700, 200, 16
    m = om.band_mask(S, w, Np)
    rp, ent = om.schedule(m, 128, 32, 64)
    kinds32 = om.tile_kinds(m, 32, 64)
    seen = np.zeros_like(kinds32)
    for qb in range(len(rp) - 1):
        kts = [int(e) & 0xffff for e in ent[rp[qb]:rp[qb + 1]]]
        assert kts == sorted(kts) and len(set(kts)) == len(kts)
        for e in ent[rp[qb]:rp[qb + 1]]:
            e = int(e) & 0xffffffff
            kt = e & 0xffff
            for j in range(4):
                qs = qb * 4 + j
                k = (e >> (16 + 2 * j)) & 3
                if qs < kinds32.shape[0]:
                    assert k == kinds32[qs, kt]
                    seen[qs, kt] = k
                else:
                    assert k == 0
    assert np.array_equal(seen, kinds32)
