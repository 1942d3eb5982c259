"""The C-ABI library on the CPU: it loads, exports every symbol include/tmac.h
declares, its host index construction is bit-exact with the oracle, and its
device entry points reject bad arguments before touching any device memory."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from oracle import block_ell as ob
from oracle import masks as om
from titans_core.kernels import _lib
from titans_core.kernels.block_ell import BlockELLPattern
from titans_core.kernels.window_attn import tile_kinds, work_list, work_list_kv

HEADER = Path(__file__).resolve().parents[1] / "include" / "tmac.h"
GOLDEN = Path(__file__).resolve().parent / "golden"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tmac_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(lib):
    names = declared_symbols()
    assert len(names) >= 12
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES or n in ("tmac_status_string", "tmac_wattn_mask_workspace"), \
            f"{n} has no ctypes signature"
    assert lib.tmac_abi_version() == _lib.ABI_VERSION


def test_status_strings(lib):
    for code in range(0, -9, -1):
        s = lib.tmac_status_string(code).decode()
        assert s and s != "unknown tmac status"
    assert lib.tmac_status_string(-99).decode() == "unknown tmac status"


@pytest.mark.parametrize("seed,n_brow,n_bcol,width", [(0, 40, 160, 40), (4, 10, 40, 20), (1, 1, 1, 1),
                                                      (123456789, 17, 33, 32), (2**64 - 1, 5, 9, 9)])
def test_sampler_and_transpose_bit_exact(seed, n_brow, n_bcol, width):
    pat = BlockELLPattern.sample(seed, n_brow, n_bcol, width)
    ci = ob.sample_col_idx(seed, n_brow, n_bcol, width)
    assert np.array_equal(pat.col_idx, ci)
    for got, want in zip((pat.t_ptr, pat.t_row, pat.t_vblk, pat.order), ob.transpose(ci, n_bcol)):
        assert np.array_equal(got, want)


def test_sampler_matches_golden():
    assert np.array_equal(BlockELLPattern.sample(0, 40, 160, 40).col_idx,
                          np.load(GOLDEN / "bell_col_idx_cfg2.npy"))
    assert np.array_equal(BlockELLPattern.sample(4, 10, 40, 20).col_idx,
                          np.load(GOLDEN / "bell_col_idx_cfg4.npy"))


@pytest.mark.parametrize("ci", [[[0, 0]], [[2, 1]], [[0, 4]], [[-1, 2]]])
def test_pattern_validation_rejects(ci):
    with pytest.raises(ValueError):
        BlockELLPattern(np.array(ci, dtype=np.int32), 4)


def test_sampler_shape_errors(lib):
    buf = np.zeros(4, dtype=np.int32)
    assert lib.tmac_bell_sample_col_idx(0, 1, 3, 4, buf.ctypes.data) == -2
    assert lib.tmac_bell_sample_col_idx(0, 1, 3, 1, None) == -1


CASES = [(4096, 512, 16, True, "band", 64), (4112, 512, 16, True, "band", 64), (560, 512, 16, True, "band", 64),
         (300, 64, 0, False, "band", 64), (1, 0, 0, True, "band", 64), (129, 3, 128, True, "band", 64),
         (4096, 512, 16, True, "blockwin", 64), (333, 128, 5, False, "blockwin", 32),
         (250, 0, 1, True, "blockwin", 64)]


@pytest.mark.parametrize("S,w,Np,causal,pattern,bs", CASES)
def test_tile_kinds_bit_exact(S, w, Np, causal, pattern, bs):
    m = om.make_mask(S, w, Np, causal, pattern, bs)
    for tq, tk in [(64, 64), (32, 64), (128, 64), (16, 32)]:
        assert np.array_equal(tile_kinds(S, w, Np, causal, pattern, bs, tq, tk), om.tile_kinds(m, tq, tk))


@pytest.mark.parametrize("S,w,Np,causal,pattern,bs", CASES)
def test_work_list_bit_exact(S, w, Np, causal, pattern, bs):
    m = om.make_mask(S, w, Np, causal, pattern, bs)
    rp, ent = work_list(S, w, Np, causal, pattern, bs)
    rp2, ent2 = om.schedule(m, 128, 32, 64)
    assert np.array_equal(rp, rp2) and np.array_equal(ent, ent2)


@pytest.mark.parametrize("S,w,Np,causal,pattern,bs", CASES)
def test_work_list_kv_bit_exact(S, w, Np, causal, pattern, bs):
    m = om.make_mask(S, w, Np, causal, pattern, bs)
    cp, ent = work_list_kv(S, w, Np, causal, pattern, bs)
    cp2, ent2 = om.schedule_kv(m, 128, 32, 64)
    assert np.array_equal(cp, cp2) and np.array_equal(ent, ent2)


@pytest.mark.parametrize("S,w,Np,causal,pattern,bs", [(700, 200, 16, True, "band", 64),
                                                      (333, 40, 5, False, "blockwin", 32)])
def test_work_list_kv_covers_every_allowed_pair_once(S, w, Np, causal, pattern, bs):
    """Every allowed (query, key) pair lies in exactly one listed (key slice, query tile)
    of its key block whose kind is non-zero, and full slices hold only allowed pairs."""
    m = om.make_mask(S, w, Np, causal, pattern, bs)
    cp, ent = work_list_kv(S, w, Np, causal, pattern, bs)
    cover = np.zeros((S, S), dtype=np.int32)
    for kb in range(len(cp) - 1):
        qts = [int(e) & 0xffff for e in ent[cp[kb]:cp[kb + 1]]]
        assert qts == sorted(qts) and len(set(qts)) == len(qts)
        for e in ent[cp[kb]:cp[kb + 1]]:
            e = int(e) & 0xffffffff
            qt = e & 0xffff
            for j in range(4):
                kind = (e >> (16 + 2 * j)) & 3
                k0 = kb * 128 + 32 * j
                blk = m[qt * 64:qt * 64 + 64, k0:k0 + 32]
                if kind == 0:
                    assert not blk.any()
                    continue
                if kind == 1:
                    assert blk.shape == (64, 32) and blk.all()
                cover[qt * 64:qt * 64 + 64, k0:k0 + 32] += 1
    assert np.array_equal(cover[m], np.ones(int(m.sum()), dtype=np.int32))


def test_work_list_kv_shape_errors(lib):
    cp = np.zeros(40, dtype=np.int32)
    n = ctypes.c_int(0)
    for kb, sc in [(128, 48), (512, 32), (0, 32)]:
        assert lib.tmac_wattn_schedule_kv(4096, 512, 16, 1, 0, 64, kb, sc, cp.ctypes.data, None, 0,
                                          ctypes.byref(n)) == -2


SPAN_CASES = CASES + [(300, 5000, 7, False, "band", 64), (300, 10**9, 7, True, "blockwin", 48),
                      (129, 0, 0, False, "blockwin", 1), (65, 3, 65, True, "blockwin", 8),
                      (1, 0, 0, True, "band", 64), (200, 63, 5, False, "blockwin", 200)]


@pytest.mark.parametrize("S,w,Np,causal,pattern,bs", SPAN_CASES)
def test_mask_spans_bit_exact(lib, S, w, Np, causal, pattern, bs):
    """The per-row and per-key intervals the kernels test on partial tiles reproduce
    the oracle mask and its transpose exactly."""
    rows = np.zeros(3 * S, dtype=np.int32)
    cols = np.zeros(3 * S, dtype=np.int32)
    code = 0 if pattern == "band" else 1
    assert lib.tmac_wattn_mask_spans(S, w, Np, int(causal), code, bs, rows.ctypes.data,
                                     cols.ctypes.data) == 0
    m = om.make_mask(S, w, Np, causal, pattern, bs)
    idx = np.arange(S)

    def expand(sp):
        np_, lo, hi = sp.reshape(S, 3).T
        return (idx[None, :] < np_[:, None]) | ((idx[None, :] >= lo[:, None]) & (idx[None, :] <= hi[:, None]))

    assert np.array_equal(expand(rows), m)
    assert np.array_equal(expand(cols), m.T)


def test_tile_map_golden():
    assert np.array_equal(tile_kinds(4096, 512, 16), np.load(GOLDEN / "wattn_tiles_cfg3.npy"))
    g = np.load(GOLDEN / "wattn_worklist_cfg3.npz")
    rp, ent = work_list(4096, 512, 16)
    assert np.array_equal(rp, g["row_ptr"]) and np.array_equal(ent, g["entries"])


def test_tile_map_value_errors():
    with pytest.raises(ValueError):
        tile_kinds(16, 4, 16)
    with pytest.raises(ValueError):
        tile_kinds(16, -1, 0)
    with pytest.raises(ValueError):
        work_list(64, 8, 0, pattern="nope")


def test_schedule_capacity_error(lib):
    rp = np.zeros(33, dtype=np.int32)
    ent = np.zeros(3, dtype=np.int32)
    n = ctypes.c_int(0)
    rc = lib.tmac_wattn_schedule(4096, 512, 16, 1, 0, 64, 128, 32, rp.ctypes.data, ent.ctypes.data, 3,
                                 ctypes.byref(n))
    assert rc == -7


# Device entry points: argument errors come back before any device access, so
# these run without a GPU. Fake pointers are never dereferenced on these paths.
FAKE = ctypes.c_void_p(1 << 20)
MISALIGNED = ctypes.c_void_p((1 << 20) + 2)


def test_bell_fwd_argument_errors(lib):
    ok = [FAKE, 2560, FAKE, FAKE, FAKE, FAKE, FAKE, None, FAKE, 10240, 8192, 40, 160, 40, 1, 0, None]
    assert lib.tmac_bell_fwd(*[None if i == 0 else a for i, a in enumerate(ok)]) == -1
    bad = list(ok); bad[13] = 161
    assert lib.tmac_bell_fwd(*bad) == -2          # width > n_bcol
    bad = list(ok); bad[14] = 9
    assert lib.tmac_bell_fwd(*bad) == -4          # unknown dtype
    bad = list(ok); bad[14] = 0; bad[1] = 2562
    assert lib.tmac_bell_fwd(*bad) == -5          # fp32: ldx in whole 16-byte vectors
    bad = list(ok); bad[15] = 7
    assert lib.tmac_bell_fwd(*bad) == -8          # unknown epilogue
    bad = list(ok); bad[1] = 2000
    assert lib.tmac_bell_fwd(*bad) == -2          # ldx < K
    bad = list(ok); bad[0] = MISALIGNED
    assert lib.tmac_bell_fwd(*bad) == -5
    bad = list(ok); bad[1] = 2564
    assert lib.tmac_bell_fwd(*bad) == -5          # ldx not a multiple of 8


def test_bias_grad_argument_errors(lib):
    """tmac_bell_bias_grad rejects bad arguments before any launch (no GPU needed)."""
    ws = ctypes.c_size_t(0)
    assert lib.tmac_bell_gelu_bwd_workspace(32768, 640, ctypes.byref(ws)) == 0
    g = [FAKE, 640, FAKE, FAKE, ws.value, 32768, 640, 1, None]
    for i, code in ((0, -1), (2, -1), (3, -1)):
        bad = list(g); bad[i] = None
        assert lib.tmac_bell_bias_grad(*bad) == code
    bad = list(g); bad[6] = 644
    assert lib.tmac_bell_bias_grad(*bad) == -2           # N % 8
    bad = list(g); bad[1] = 600
    assert lib.tmac_bell_bias_grad(*bad) == -2           # pitch < N
    bad = list(g); bad[5] = -1
    assert lib.tmac_bell_bias_grad(*bad) == -2
    bad = list(g); bad[7] = 7
    assert lib.tmac_bell_bias_grad(*bad) == -4           # not a dtype
    bad = list(g); bad[7] = 0; bad[6] = 642
    assert lib.tmac_bell_bias_grad(*bad) == -2           # fp32: N % 4
    bad = list(g); bad[4] = ws.value - 1
    assert lib.tmac_bell_bias_grad(*bad) == -6
    bad = list(g); bad[0] = MISALIGNED
    assert lib.tmac_bell_bias_grad(*bad) == -5


def test_fused_gelu_argument_errors(lib):
    """tmac_bell_fwd_gelu_aux and tmac_bell_gelu_bwd reject bad arguments before
    any launch (no GPU needed)."""
    ok = [FAKE, 2560, FAKE, FAKE, FAKE, FAKE, FAKE, None, FAKE, 10240, FAKE, 10240, 8192, 40, 160, 40,
          1, None]
    bad = list(ok); bad[10] = None
    assert lib.tmac_bell_fwd_gelu_aux(*bad) == -1        # Z required
    bad = list(ok); bad[16] = 7
    assert lib.tmac_bell_fwd_gelu_aux(*bad) == -4        # not a dtype
    bad = list(ok); bad[11] = 10200
    assert lib.tmac_bell_fwd_gelu_aux(*bad) == -2        # ldz < N
    bad = list(ok); bad[10] = MISALIGNED
    assert lib.tmac_bell_fwd_gelu_aux(*bad) == -5
    ws = ctypes.c_size_t(0)
    assert lib.tmac_bell_gelu_bwd_workspace(32768, 2560, ctypes.byref(ws)) == 0
    assert ws.value == 256 * 2560 * 4                    # 256 row parts of fp32 column sums
    assert lib.tmac_bell_gelu_bwd_workspace(-1, 2560, ctypes.byref(ws)) == -2
    g = [FAKE, 2560, FAKE, 2560, FAKE, 2560, FAKE, FAKE, ws.value, 32768, 2560, 1, None]
    bad = list(g); bad[0] = None
    assert lib.tmac_bell_gelu_bwd(*bad) == -1
    bad = list(g); bad[7] = None
    assert lib.tmac_bell_gelu_bwd(*bad) == -1            # bias gradient needs the workspace
    bad = list(g); bad[10] = 2564
    assert lib.tmac_bell_gelu_bwd(*bad) == -2            # N % 8
    bad = list(g); bad[11] = 7
    assert lib.tmac_bell_gelu_bwd(*bad) == -4            # not a dtype
    bad = list(g); bad[11] = 0; bad[10] = 2562
    assert lib.tmac_bell_gelu_bwd(*bad) == -2            # fp32: N % 4
    bad = list(g); bad[8] = ws.value - 1
    assert lib.tmac_bell_gelu_bwd(*bad) == -6
    bad = list(g); bad[1] = 2568
    bad[4] = MISALIGNED
    assert lib.tmac_bell_gelu_bwd(*bad) == -5


def test_bell_dx_and_sddmm_argument_errors(lib):
    assert lib.tmac_bell_dx(FAKE, 2560, FAKE, FAKE, FAKE, 640, 0, 10, 40, 20, 1, None) == -2
    assert lib.tmac_bell_dx(FAKE, 2560, FAKE, FAKE, FAKE, 640, 100, 10, 40, 20, 3, None) == -4
    assert lib.tmac_bell_dx(FAKE, 2562, FAKE, FAKE, FAKE, 640, 100, 10, 40, 20, 0, None) == -5
    ws = ctypes.c_size_t(0)
    assert lib.tmac_bell_sddmm_workspace(32768, 10, 40, 20, ctypes.byref(ws)) == 0 and ws.value > 0
    args = [FAKE, 640, FAKE, 2560, FAKE, FAKE, 0, FAKE, ws.value - 1, 32768, 10, 40, 20, 1, None]
    assert lib.tmac_bell_sddmm(*args) == -6      # workspace too small
    args[8] = ws.value; args[6] = 5
    assert lib.tmac_bell_sddmm(*args) == -4      # unknown output dtype


def test_wattn_fwd_argument_errors(lib):
    st = (ctypes.c_int64 * 3)(4096 * 1920, 64, 1920)
    base = [FAKE, st, FAKE, st, FAKE, st, FAKE, st, None, 8, 10, 4096, 64, 512, 16, 1, 0, 64, 0.125,
            FAKE, FAKE, FAKE, 0, 1, None]
    for dh in (0, 16, 48, 96, 256):
        a = list(base); a[12] = dh
        assert lib.tmac_wattn_fwd(*a) == -2       # head_dim must be 32, 64 or 128
    a = list(base); a[14] = 4096
    assert lib.tmac_wattn_fwd(*a) == -8           # n_persistent >= S
    a = list(base); a[13] = -1
    assert lib.tmac_wattn_fwd(*a) == -8           # negative window
    a = list(base); a[23] = 9
    assert lib.tmac_wattn_fwd(*a) == -4
    a = list(base); a[22] = 33
    assert lib.tmac_wattn_fwd(*a) == -8           # more leading blocks than 128-row blocks
    a = list(base); a[21] = None
    assert lib.tmac_wattn_fwd(*a) == -1
    a = list(base); a[1] = (ctypes.c_int64 * 3)(4096 * 1920, 60, 1920)
    assert lib.tmac_wattn_fwd(*a) == -5           # head stride not 16-byte aligned
    a = list(base); a[19] = None
    assert lib.tmac_wattn_fwd(*a) == -1


def test_wattn_bwd_argument_errors(lib):
    st = (ctypes.c_int64 * 3)(4096 * 1920, 64, 1920)
    base = [FAKE, st, FAKE, st, FAKE, st, FAKE, st, FAKE, st, FAKE, FAKE, FAKE, st, FAKE, st,
            FAKE, st, 8, 10, 4096, 64, 512, 16, 1, 0, 64, 0.125, FAKE, FAKE, FAKE, 1,
            FAKE, FAKE, FAKE, 1, 1, None]
    for dh in (0, 16, 48, 96, 256):
        a = list(base); a[21] = dh
        assert lib.tmac_wattn_bwd(*a) == -2       # head_dim must be 32, 64 or 128
    a = list(base); a[36] = 9
    assert lib.tmac_wattn_bwd(*a) == -4           # unknown dtype
    a = list(base); a[36] = 0; a[1] = (ctypes.c_int64 * 3)(4096 * 1920, 64, 1922)
    assert lib.tmac_wattn_bwd(*a) == -5           # fp32: strides in whole 16-byte vectors
    a = list(base); a[23] = 4096
    assert lib.tmac_wattn_bwd(*a) == -8           # n_persistent >= S (band)
    a = list(base); a[35] = -1
    assert lib.tmac_wattn_bwd(*a) == -8
    a = list(base); a[13] = (ctypes.c_int64 * 3)(4096 * 1920, 64, 1921)
    assert lib.tmac_wattn_bwd(*a) == -5           # dQ token stride not a multiple of 8
    a = list(base); a[11] = None
    assert lib.tmac_wattn_bwd(*a) == -1           # delta workspace
    a = list(base); a[34] = None
    assert lib.tmac_wattn_bwd(*a) == -1


def test_launch_order():
    from titans_core.kernels.window_attn import launch_order
    order, lead = launch_order(np.array([0, 3, 4, 20, 23, 26, 27], dtype=np.int32))
    # lengths 3, 1, 16, 3, 3, 1 (mean 4.5): longest first, ties by block index
    assert order.tolist() == [2, 0, 3, 4, 1, 5] and lead == 1
    order, lead = launch_order(np.array([0, 5, 10, 15], dtype=np.int32))
    assert order.tolist() == [0, 1, 2] and lead == 0
    rp, _ = work_list(4096, 512, 16, True, "blockwin", 64)
    order, lead = launch_order(rp)
    assert order[0] == 0 and lead == 1 and sorted(order.tolist()) == list(range(32))
    with pytest.raises(ValueError):
        launch_order(np.array([0, 3, 2], dtype=np.int32))


def test_dwconv_argument_errors(lib):
    # in, ld_in, w, out, ld_out, B, T, C, ksize, dtype, stream
    ok = [FAKE, 1920, FAKE, FAKE, 1920, 8, 4096, 1920, 4, 1, None]
    bad = list(ok); bad[0] = None
    assert lib.tmac_dwconv_causal(*bad) == -1
    bad = list(ok); bad[8] = 9
    assert lib.tmac_dwconv_causal(*bad) == -8      # ksize above 8
    bad = list(ok); bad[7] = 1921
    assert lib.tmac_dwconv_causal(*bad) == -2      # C not a multiple of the 16-byte vector
    bad = list(ok); bad[1] = 1000
    assert lib.tmac_dwconv_causal(*bad) == -2      # row stride < C
    bad = list(ok); bad[0] = MISALIGNED
    assert lib.tmac_dwconv_causal(*bad) == -5
    bad = list(ok); bad[9] = 7
    assert lib.tmac_dwconv_causal(*bad) == -4


def test_only_persistent_tokens_allowed_for_blockwin_only():
    k = tile_kinds(24, 8, 24, True, "blockwin", 16, tq=8, tk=8)
    assert k.shape == (3, 3) and (k == 1).all()     # every pair allowed
    with pytest.raises(ValueError):
        tile_kinds(24, 8, 24, True, "band", 64)


@pytest.mark.parametrize("S,w,Np,pattern", [(4096, 512, 16, 0), (333, 128, 5, 1), (1, 0, 0, 0)])
def test_work_lists_exact_and_short_capacity(lib, S, w, Np, pattern):
    """Each work list fills a buffer of exactly its length, reports the length with a
    NULL buffer, and refuses a buffer one entry short (TMAC_ERR_CAPACITY) without writing
    past it (the sanitizer run of this file checks the writes)."""
    n_b = -(-S // 128)
    for fn in (lib.tmac_wattn_schedule, lib.tmac_wattn_schedule_kv):
        ptr = np.zeros(n_b + 1, dtype=np.int32)
        n = ctypes.c_int(-1)
        assert fn(S, w, Np, 1, pattern, 64, 128, 32, ptr.ctypes.data, None, 0, ctypes.byref(n)) == 0
        total = n.value
        assert total == ptr[-1] and total > 0
        exact = np.full(total, -1, dtype=np.int32)
        assert fn(S, w, Np, 1, pattern, 64, 128, 32, ptr.ctypes.data, exact.ctypes.data, total,
                  ctypes.byref(n)) == 0
        assert (exact >= 0).all() and n.value == total
        short = np.zeros(max(total - 1, 1), dtype=np.int32)
        rc = fn(S, w, Np, 1, pattern, 64, 128, 32, ptr.ctypes.data, short.ctypes.data, total - 1,
                ctypes.byref(n))
        assert rc == -7, rc


def test_transpose_rejects_malformed_indices(lib):
    out = [np.zeros(n, dtype=np.int32) for n in (5, 8, 8, 4)]
    ptrs = [a.ctypes.data for a in out]
    for ci in ([[0, 1], [2, 4]], [[1, 1], [0, 2]], [[2, 1], [0, 3]], [[0, -1], [1, 2]]):
        ci = np.array(ci, dtype=np.int32)
        assert lib.tmac_bell_transpose(ci.ctypes.data, 2, 4, 2, *ptrs) == -3
    ci = np.array([[0, 1], [2, 3]], dtype=np.int32)
    assert lib.tmac_bell_transpose(ci.ctypes.data, 2, 4, 2, None, *ptrs[1:]) == -1
    assert lib.tmac_bell_validate(ci.ctypes.data, 70000, 70000, 40000) == -2   # n_brow * width > 2^31 - 1
    assert lib.tmac_bell_sample_col_idx(0, 70000, 70000, 40000, ci.ctypes.data) == -2


def test_mask_spans_and_launch_order_edges(lib):
    rows = np.zeros(3, dtype=np.int32)
    cols = np.zeros(3, dtype=np.int32)
    assert lib.tmac_wattn_mask_spans(1, 0, 0, 1, 0, 64, rows.ctypes.data, cols.ctypes.data) == 0
    assert rows.tolist() == [0, 0, 0] and cols.tolist() == [0, 0, 0]
    assert lib.tmac_wattn_mask_spans(1, 0, 0, 1, 0, 64, None, cols.ctypes.data) == -1
    assert lib.tmac_wattn_mask_spans(0, 0, 0, 1, 0, 64, rows.ctypes.data, cols.ctypes.data) == -2
    ptr = np.array([0], dtype=np.int32)
    order = np.zeros(1, dtype=np.int32)
    lead = ctypes.c_int(-1)
    rc = lib.tmac_wattn_launch_order(ptr.ctypes.data, 0, order.ctypes.data, ctypes.byref(lead))
    assert rc in (0, -2)


def test_mask_workspace_size(lib):
    for S, mb, mh in [(1, 1, 1), (4096, 1, 1), (4096, 4, 10), (300, 2, 1), (129, 1, 3)]:
        n = lib.tmac_wattn_mask_workspace(S, mb, mh)
        n_b, n_t = -(-S // 128), -(-S // 64)
        rows = mb * mh * n_b
        bitmaps = 2 * mb * mh * n_b * 128 * n_t * 8
        assert n % 256 == 0
        # two launch orders, kinds (1 byte) and entries (4 bytes) per list row and tile,
        # counts, bitmaps; each part 256-byte aligned
        assert n >= 8 * n_b + 2 * rows * n_t * (1 + 4) + 2 * rows * 4 + bitmaps
        assert n <= 8 * n_b + 2 * rows * n_t * (1 + 4) + 2 * rows * 4 + bitmaps + 4 * 256
    for bad in [(0, 1, 1), (64, 0, 1), (64, 1, 0), (-5, 1, 1)]:
        assert lib.tmac_wattn_mask_workspace(*bad) == 0


def _opts(**kw):
    from titans_core.kernels.window_attn import AttnOpts
    o = AttnOpts()
    for k, v in kw.items():
        if k == "mask_strides":
            o.mask_strides[0], o.mask_strides[1], o.mask_strides[2] = v
        else:
            setattr(o, k, v)
    return o


def test_wattn_ex_option_errors(lib):
    """Option checks of tmac_wattn_fwd_ex / _bwd_ex / _mask_lists (nothing is launched)."""
    st = (ctypes.c_int64 * 3)(4096 * 1920, 64, 1920)
    S = 4096
    fwd = [FAKE, st, FAKE, st, FAKE, st, FAKE, st, None, 8, 10, S, 64, 512, 16, 1, 0, 64, 0.125,
           FAKE, FAKE, FAKE, 0, 1, None]
    bwd = [FAKE, st, FAKE, st, FAKE, st, FAKE, st, FAKE, st, FAKE, FAKE, FAKE, st, FAKE, st,
           FAKE, st, 8, 10, S, 64, 512, 16, 1, 0, 64, 0.125, FAKE, FAKE, FAKE, 1,
           FAKE, FAKE, FAKE, 1, 1, None]
    ws_ok = lib.tmac_wattn_mask_workspace(S, 1, 1)
    good_mask = dict(d_mask=1 << 20, mask_format=0, mask_batch=1, mask_heads=1,
                     mask_strides=(0, 0, S), d_mask_ws=1 << 24, mask_ws_bytes=ws_ok)
    cases = [
        (dict(dropout_p=1.0), -8), (dict(dropout_p=-0.1), -8), (dict(dropout_p=float("nan")), -8),
        (dict(good_mask, mask_format=7), -4),
        (dict(good_mask, mask_batch=3), -2), (dict(good_mask, mask_heads=4), -2),
        (dict(good_mask, mask_strides=(0, 0, S - 1)), -2),
        (dict(good_mask, mask_strides=(-1, 0, S)), -2),
        (dict(good_mask, d_mask_ws=None), -6), (dict(good_mask, mask_ws_bytes=ws_ok - 1), -6),
        (dict(good_mask, d_mask_ws=(1 << 24) + 16), -5),
        (dict(good_mask, mask_format=1, d_mask=(1 << 20) + 2), -5),
    ]
    for kw, want in cases:
        o = _opts(**kw)
        assert lib.tmac_wattn_fwd_ex(*fwd, ctypes.byref(o)) == want, kw
        assert lib.tmac_wattn_bwd_ex(*bwd, ctypes.byref(o)) == want, kw
    # with a mask the pattern arguments are not checked, but the rest still is
    o = _opts(**dict(good_mask, dropout_p=2.0))
    a = list(fwd); a[14] = S   # n_persistent = S: invalid for the band pattern, unused here
    assert lib.tmac_wattn_fwd_ex(*a, ctypes.byref(o)) == -8   # the dropout_p
    a = list(fwd); a[12] = 48
    assert lib.tmac_wattn_fwd_ex(*a, ctypes.byref(_opts(**good_mask))) == -2
    # without a mask the schedule arrays are required
    a = list(bwd); a[28] = None
    assert lib.tmac_wattn_bwd_ex(*a, ctypes.byref(_opts())) == -1
    # tmac_wattn_mask_lists
    assert lib.tmac_wattn_mask_lists(None, S, None) == -1
    assert lib.tmac_wattn_mask_lists(ctypes.byref(_opts()), S, None) == -1
    assert lib.tmac_wattn_mask_lists(ctypes.byref(_opts(**good_mask)), 0, None) == -2
    assert lib.tmac_wattn_mask_lists(ctypes.byref(_opts(**dict(good_mask, mask_format=5))),
                                     S, None) == -4
    assert lib.tmac_wattn_mask_lists(ctypes.byref(_opts(**dict(good_mask, mask_ws_bytes=8))),
                                     S, None) == -6
