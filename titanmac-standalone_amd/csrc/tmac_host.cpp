// Host-side index construction for the TitanMAC sparse hot path: Block-ELL
// sampling / validation / transposition and the attention tile maps.
// Everything here is plain integer work on host memory; the results are copied
// to the device once per pattern by the caller and cached.

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <vector>

#include "../../include/tmac.h"
#include "tmac_device.h"

extern "C" int tmac_abi_version(void) { return TMAC_ABI_VERSION; }

extern "C" const char* tmac_status_string(int code) {
  switch (code) {
    case TMAC_OK: return "ok";
    case TMAC_ERR_NULL: return "a required pointer is NULL";
    case TMAC_ERR_SHAPE: return "invalid or inconsistent shape";
    case TMAC_ERR_INDEX: return "Block-ELL index out of range, duplicated or unsorted";
    case TMAC_ERR_DTYPE: return "unsupported dtype";
    case TMAC_ERR_ALIGN: return "pointer or stride not 16-byte aligned for vector loads";
    case TMAC_ERR_WORKSPACE: return "workspace missing or too small";
    case TMAC_ERR_CAPACITY: return "output array too small";
    case TMAC_ERR_VALUE: return "argument value outside its domain";
    case TMAC_ERR_TOO_LARGE: return "sizes exceed the static scratch of an allocation-free entry point";
    default: break;
  }
  if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
  return "unknown tmac status";
}

// ---------------------------------------------------------------------------
// Block-ELL index
// ---------------------------------------------------------------------------

namespace {

// splitmix64 (Steele, Lea, Flood 2014; public-domain reference by S. Vigna).
struct SplitMix64 {
  uint64_t s;
  uint64_t next() {
    s += 0x9E3779B97F4A7C15ull;
    uint64_t z = s;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  }
  // Uniform integer in [0, n), n >= 1: reject draws below 2^64 mod n so every
  // residue class has the same number of accepted values.
  uint64_t bounded(uint64_t n) {
    const uint64_t threshold = (0ull - n) % n;
    for (;;) {
      const uint64_t x = next();
      if (x >= threshold) return x % n;
    }
  }
};

}  // namespace

extern "C" int tmac_bell_sample_col_idx(uint64_t seed, int n_brow, int n_bcol, int width,
                                        int32_t* h_col_idx) {
  if (!h_col_idx) return TMAC_ERR_NULL;
  if (n_brow <= 0 || n_bcol <= 0 || width <= 0 || width > n_bcol) return TMAC_ERR_SHAPE;
  if (static_cast<int64_t>(n_brow) * width > INT32_MAX) return TMAC_ERR_SHAPE;
  SplitMix64 rng{seed};
  std::vector<int32_t> perm(n_bcol);
  for (int r = 0; r < n_brow; ++r) {
    for (int c = 0; c < n_bcol; ++c) perm[c] = c;
    for (int i = 0; i < width; ++i) {
      const int j = i + static_cast<int>(rng.bounded(static_cast<uint64_t>(n_bcol - i)));
      std::swap(perm[i], perm[j]);
    }
    int32_t* row = h_col_idx + static_cast<size_t>(r) * width;
    std::copy(perm.begin(), perm.begin() + width, row);
    std::sort(row, row + width);
  }
  return TMAC_OK;
}

extern "C" int tmac_bell_validate(const int32_t* h_col_idx, int n_brow, int n_bcol, int width) {
  if (!h_col_idx) return TMAC_ERR_NULL;
  if (n_brow <= 0 || n_bcol <= 0 || width <= 0 || width > n_bcol) return TMAC_ERR_SHAPE;
  // entry indices (r * width + s) are ints in the transposed index and the kernels
  if (static_cast<int64_t>(n_brow) * width > INT32_MAX) return TMAC_ERR_SHAPE;
  for (int r = 0; r < n_brow; ++r) {
    const int32_t* row = h_col_idx + static_cast<size_t>(r) * width;
    for (int s = 0; s < width; ++s) {
      if (row[s] < 0 || row[s] >= n_bcol) return TMAC_ERR_INDEX;
      if (s > 0 && row[s] <= row[s - 1]) return TMAC_ERR_INDEX;
    }
  }
  return TMAC_OK;
}

extern "C" int tmac_bell_transpose(const int32_t* h_col_idx, int n_brow, int n_bcol, int width,
                                   int32_t* h_t_ptr, int32_t* h_t_row, int32_t* h_t_vblk,
                                   int32_t* h_order) {
  if (!h_t_ptr || !h_t_row || !h_t_vblk || !h_order) return TMAC_ERR_NULL;
  const int st = tmac_bell_validate(h_col_idx, n_brow, n_bcol, width);
  if (st != TMAC_OK) return st;
  std::vector<int32_t> count(n_bcol, 0);
  for (int e = 0; e < n_brow * width; ++e) ++count[h_col_idx[e]];
  h_t_ptr[0] = 0;
  for (int c = 0; c < n_bcol; ++c) h_t_ptr[c + 1] = h_t_ptr[c] + count[c];
  std::vector<int32_t> fill(h_t_ptr, h_t_ptr + n_bcol);
  // Rows ascending, so every column's list comes out ordered by block-row.
  for (int r = 0; r < n_brow; ++r) {
    for (int s = 0; s < width; ++s) {
      const int c = h_col_idx[r * width + s];
      const int e = fill[c]++;
      h_t_row[e] = r;
      h_t_vblk[e] = r * width + s;
    }
  }
  for (int c = 0; c < n_bcol; ++c) h_order[c] = c;
  std::stable_sort(h_order, h_order + n_bcol,
                   [&](int32_t a, int32_t b) { return count[a] > count[b]; });
  return TMAC_OK;
}

extern "C" int tmac_bell_group_schedule(const int32_t* h_col_idx, int n_brow, int n_bcol,
                                        int width, int dir, int group, int32_t* h_grp_ptr,
                                        int32_t* h_grp_out, int32_t* h_steps, int capacity,
                                        int* n_groups, int* n_steps) {
  if (!h_grp_ptr || !h_grp_out || !h_steps || !n_groups || !n_steps) return TMAC_ERR_NULL;
  if (dir != 0 && dir != 1) return TMAC_ERR_VALUE;
  if (group != 2 && group != 4) return TMAC_ERR_VALUE;
  const int st = tmac_bell_validate(h_col_idx, n_brow, n_bcol, width);
  if (st != TMAC_OK) return st;
  // Lists of (input block, value block) per output block, ascending by input:
  // forward (dir 0): output block-column c, inputs = the block-rows holding a
  // block in c; dX (dir 1): output block-row r, inputs = col_idx[r].
  const int n_out = dir == 0 ? n_bcol : n_brow;
  const int n_in = dir == 0 ? n_brow : n_bcol;
  std::vector<std::vector<std::pair<int32_t, int32_t>>> lists(n_out);
  for (int r = 0; r < n_brow; ++r)
    for (int s = 0; s < width; ++s) {
      const int c = h_col_idx[static_cast<size_t>(r) * width + s];
      if (dir == 0)
        lists[c].push_back({r, r * width + s});
      else
        lists[r].push_back({c, r * width + s});
    }
  // Input sets as bitsets, for the overlap counts of the greedy grouping.
  const int words = (n_in + 63) / 64;
  std::vector<uint64_t> bits(static_cast<size_t>(n_out) * words, 0);
  for (int o = 0; o < n_out; ++o)
    for (const auto& e : lists[o]) bits[static_cast<size_t>(o) * words + e.first / 64] |= 1ull << (e.first % 64);
  auto popc = [](uint64_t x) { return __builtin_popcountll(x); };
  // Greedy grouping: seed = the longest remaining list (lowest index on ties);
  // then, until the group is full, add the remaining output sharing the most
  // inputs with the group's union (fewest new inputs, then lowest index, on ties).
  std::vector<char> used(n_out, 0);
  std::vector<std::vector<int>> groups;
  std::vector<uint64_t> uni(words);
  int left = n_out;
  while (left > 0) {
    int seed = -1;
    for (int o = 0; o < n_out; ++o)
      if (!used[o] && (seed < 0 || lists[o].size() > lists[seed].size())) seed = o;
    used[seed] = 1;
    --left;
    std::vector<int> g{seed};
    std::copy(bits.begin() + static_cast<size_t>(seed) * words,
              bits.begin() + static_cast<size_t>(seed + 1) * words, uni.begin());
    while (static_cast<int>(g.size()) < group && left > 0) {
      int best = -1, best_sh = -1, best_new = 0;
      for (int o = 0; o < n_out; ++o) {
        if (used[o]) continue;
        int sh = 0, nw = 0;
        for (int w = 0; w < words; ++w) {
          const uint64_t b = bits[static_cast<size_t>(o) * words + w];
          sh += popc(b & uni[w]);
          nw += popc(b & ~uni[w]);
        }
        if (sh > best_sh || (sh == best_sh && nw < best_new)) {
          best = o;
          best_sh = sh;
          best_new = nw;
        }
      }
      used[best] = 1;
      --left;
      g.push_back(best);
      for (int w = 0; w < words; ++w) uni[w] |= bits[static_cast<size_t>(best) * words + w];
    }
    groups.push_back(std::move(g));
  }
  // Union length of each group; groups are launched longest first.
  const int ng = static_cast<int>(groups.size());
  std::vector<int> ulen(ng);
  for (int gi = 0; gi < ng; ++gi) {
    std::fill(uni.begin(), uni.end(), 0);
    for (int o : groups[gi])
      for (int w = 0; w < words; ++w) uni[w] |= bits[static_cast<size_t>(o) * words + w];
    int n = 0;
    for (int w = 0; w < words; ++w) n += popc(uni[w]);
    ulen[gi] = n;
  }
  std::vector<int> gorder(ng);
  for (int gi = 0; gi < ng; ++gi) gorder[gi] = gi;
  std::stable_sort(gorder.begin(), gorder.end(), [&](int a, int b) { return ulen[a] > ulen[b]; });
  // Steps: the group's union in ascending input order, each with the value
  // block of every member that holds that input (or -1). A member's active
  // steps are then exactly its own list in its own order.
  const int rec = 1 + group;
  int count = 0;
  std::vector<int32_t> vb(static_cast<size_t>(n_in) * group);
  h_grp_ptr[0] = 0;
  for (int k = 0; k < ng; ++k) {
    const std::vector<int>& g = groups[gorder[k]];
    std::fill(vb.begin(), vb.end(), -1);
    for (int j = 0; j < group; ++j) {
      const int o = j < static_cast<int>(g.size()) ? g[j] : -1;
      h_grp_out[static_cast<size_t>(k) * group + j] = o;
      if (o < 0) continue;
      for (const auto& e : lists[o]) vb[static_cast<size_t>(e.first) * group + j] = e.second;
    }
    for (int i = 0; i < n_in; ++i) {
      bool any = false;
      for (int j = 0; j < group; ++j) any |= vb[static_cast<size_t>(i) * group + j] >= 0;
      if (!any) continue;
      if (count >= capacity) return TMAC_ERR_CAPACITY;
      int32_t* out = h_steps + static_cast<size_t>(count) * rec;
      out[0] = i;
      for (int j = 0; j < group; ++j) out[1 + j] = vb[static_cast<size_t>(i) * group + j];
      ++count;
    }
    h_grp_ptr[k + 1] = count;
  }
  *n_groups = ng;
  *n_steps = count;
  return TMAC_OK;
}

extern "C" int tmac_bell_group_tile_order(const int32_t* h_grp_ptr, int n_groups, int M,
                                          int32_t* h_order, int capacity, int* n_entries) {
  if (!h_grp_ptr || !n_entries) return TMAC_ERR_NULL;
  if (n_groups <= 0 || M <= 0) return TMAC_ERR_SHAPE;
  for (int g = 0; g < n_groups; ++g)
    if (h_grp_ptr[g + 1] < h_grp_ptr[g]) return TMAC_ERR_VALUE;
  // the grouped launcher's split: 8 XCD ranges of per_xcd consecutive tiles
  // (tile = m_tile * n_groups + group), min(per_xcd, 32) persistent slots each
  const int64_t n_mtiles = (static_cast<int64_t>(M) + TMAC_BELL_GROUP_ROWS - 1) / TMAC_BELL_GROUP_ROWS;
  const int64_t n_tiles = n_mtiles * n_groups;
  if (n_tiles > (1ll << 30)) return TMAC_ERR_SHAPE;
  const int per_xcd = static_cast<int>((n_tiles + 7) / 8);
  const int n_slots = per_xcd < TMAC_BELL_GROUP_SLOTS ? per_xcd : TMAC_BELL_GROUP_SLOTS;
  const int n_rounds = (per_xcd + n_slots - 1) / n_slots;
  const int64_t total = 8ll * n_rounds * n_slots;
  *n_entries = static_cast<int>(total);
  if (!h_order) return TMAC_OK;
  if (capacity < total) return TMAC_ERR_CAPACITY;
  std::fill(h_order, h_order + total, -1);
  // Per XCD, round by round, the round's tiles are those of the round-robin
  // deal (the next n_slots of the XCD's range, so the tiles that run together,
  // and share the L2, stay the same); longest first (steps plus a fixed cost for
  // the prologue and epilogue; ties by tile index), they go to the slots in
  // ascending order of their load so far (ties by slot).
  constexpr int64_t kTileCost = 2;
  std::vector<int> tiles, slots(n_slots);
  std::vector<int64_t> load(n_slots);
  auto cost = [&](int t) {
    const int g = t % n_groups;
    return static_cast<int64_t>(h_grp_ptr[g + 1] - h_grp_ptr[g]) + kTileCost;
  };
  for (int x = 0; x < 8; ++x) {
    const int64_t t0 = static_cast<int64_t>(x) * per_xcd;
    const int64_t t1 = std::min<int64_t>(n_tiles, t0 + per_xcd);
    std::fill(load.begin(), load.end(), 0);
    for (int r = 0; r < n_rounds; ++r) {
      tiles.clear();
      for (int64_t t = t0 + static_cast<int64_t>(r) * n_slots; t < t1 && tiles.size() < static_cast<size_t>(n_slots); ++t)
        tiles.push_back(static_cast<int>(t));
      std::stable_sort(tiles.begin(), tiles.end(), [&](int a, int b) { return cost(a) > cost(b); });
      for (int j = 0; j < n_slots; ++j) slots[j] = j;
      std::stable_sort(slots.begin(), slots.end(), [&](int a, int b) { return load[a] < load[b]; });
      for (size_t j = 0; j < tiles.size(); ++j) {
        const int sl = slots[j];
        h_order[(static_cast<int64_t>(x) * n_rounds + r) * n_slots + sl] = tiles[j];
        load[sl] += cost(tiles[j]);
      }
    }
    // keep the round-robin deal where the greedy one is not better
    std::vector<int64_t> rr(n_slots, 0);
    for (int64_t t = t0; t < t1; ++t) rr[(t - t0) % n_slots] += cost(static_cast<int>(t));
    if (*std::max_element(load.begin(), load.end()) > *std::max_element(rr.begin(), rr.end())) {
      for (int r = 0; r < n_rounds; ++r)
        for (int sl = 0; sl < n_slots; ++sl) {
          const int64_t t = t0 + static_cast<int64_t>(r) * n_slots + sl;
          h_order[(static_cast<int64_t>(x) * n_rounds + r) * n_slots + sl] = t < t1 ? static_cast<int>(t) : -1;
        }
    }
  }
  return TMAC_OK;
}

// ---------------------------------------------------------------------------
// Attention tile maps
// ---------------------------------------------------------------------------

namespace {

struct RowSpan {
  // Allowed key columns of one query row: [0, a_end) ∪ [b_lo, b_hi).
  int a_end;
  int b_lo, b_hi;
};

// Allowed key set of row i, written as at most two half-open intervals.
// Band (attn/windowed_attention.py:97-152):
//   persistent rows (i < Np) see the persistent columns only (:115-132);
//   sequence rows see the persistent columns (:118) and, among sequence
//   columns, |i - j| <= w (:136-141) intersected with j <= i when causal (:144-150).
// Blockwin (attn/block_sparse_attention.py:277-334), r = i - Np, b0 = bs*floor(r/bs):
//   persistent rows see every key (:277-285);
//   sequence rows see the persistent keys (:305) and sequence keys c = j - Np in
//   [max(0, b0 - w), r] when causal (:299-301, :156-161), or
//   [max(0, b0 - w), min(b0 + bs, S - Np)) when not (:299-300, causal_mask=None).
RowSpan row_span(int i, int S, int w, int Np, bool causal, int pattern, int bs) {
  RowSpan sp{Np, 0, 0};
  if (i < Np) {
    if (pattern == TMAC_PATTERN_BLOCKWIN) sp.a_end = S;
    return sp;
  }
  if (pattern == TMAC_PATTERN_BAND) {
    const long lo = std::max<long>(Np, static_cast<long>(i) - w);
    const long hi = causal ? static_cast<long>(i) + 1
                           : std::min<long>(S, static_cast<long>(i) + w + 1);
    sp.b_lo = static_cast<int>(lo);
    sp.b_hi = static_cast<int>(hi);
  } else {
    const int r = i - Np;
    const int b0 = (r / bs) * bs;
    const int c_lo = std::max(0, b0 - w);
    const int c_hi = causal ? r + 1 : std::min(b0 + bs, S - Np);
    sp.b_lo = Np + c_lo;
    sp.b_hi = Np + c_hi;
  }
  return sp;
}

// Number of allowed keys of a row inside [k0, k1).
inline int span_count(const RowSpan& sp, int k0, int k1) {
  int n = 0;
  const int a1 = std::min(sp.a_end, k1);
  if (a1 > k0) n += a1 - k0;
  const int b0 = std::max(sp.b_lo, k0), b1 = std::min(sp.b_hi, k1);
  if (b1 > b0) {
    // Remove any overlap with the first interval so nothing is counted twice.
    const int ov0 = std::max(b0, k0), ov1 = std::min(b1, std::min(sp.a_end, k1));
    n += (b1 - b0) - std::max(0, ov1 - ov0);
  }
  return n;
}

int check_mask_args(int S, int window, int n_persistent, int pattern, int block_size) {
  if (S <= 0) return TMAC_ERR_SHAPE;
  if (n_persistent < 0) return TMAC_ERR_VALUE;
  // build_band_mask raises for n_persistent >= S (windowed_attention.py:97-100);
  // BlockSparseAttention accepts a sequence made only of persistent tokens.
  if (n_persistent > S || (pattern == TMAC_PATTERN_BAND && n_persistent == S)) return TMAC_ERR_VALUE;
  if (window < 0) return TMAC_ERR_VALUE;         // windowed_attention.py:102-103
  if (pattern != TMAC_PATTERN_BAND && pattern != TMAC_PATTERN_BLOCKWIN) return TMAC_ERR_VALUE;
  if (pattern == TMAC_PATTERN_BLOCKWIN && block_size <= 0) return TMAC_ERR_VALUE;
  return TMAC_OK;
}

// Kind of the tile rows [q0, q1) x keys [k0, k1) (both clipped to S by the
// caller's padding rule: padded positions count as masked).
uint8_t tile_kind(const std::vector<RowSpan>& spans, int S, int q0, int q1, int k0, int k1) {
  const int tile_rows = q1 - q0, tile_cols = k1 - k0;
  const int qe = std::min(q1, S), ke = std::min(k1, S);
  long allowed = 0;
  if (qe > q0 && ke > k0)
    for (int i = q0; i < qe; ++i) allowed += span_count(spans[i], k0, ke);
  if (allowed == 0) return 0;
  if (allowed == static_cast<long>(tile_rows) * tile_cols) return 1;
  return 2;
}

}  // namespace

extern "C" int tmac_wattn_tile_kinds(int S, int window, int n_persistent, int causal,
                                     int pattern, int block_size, int tq, int tk,
                                     uint8_t* h_kind) {
  if (!h_kind) return TMAC_ERR_NULL;
  int st = check_mask_args(S, window, n_persistent, pattern, block_size);
  if (st != TMAC_OK) return st;
  if (tq <= 0 || tk <= 0) return TMAC_ERR_SHAPE;
  std::vector<RowSpan> spans(S);
  for (int i = 0; i < S; ++i)
    spans[i] = row_span(i, S, window, n_persistent, causal != 0, pattern, block_size);
  const int n_qt = (S + tq - 1) / tq, n_kt = (S + tk - 1) / tk;
  for (int qt = 0; qt < n_qt; ++qt)
    for (int kt = 0; kt < n_kt; ++kt)
      h_kind[static_cast<size_t>(qt) * n_kt + kt] =
          tile_kind(spans, S, qt * tq, qt * tq + tq, kt * tk, kt * tk + tk);
  return TMAC_OK;
}

extern "C" int tmac_wattn_schedule(int S, int window, int n_persistent, int causal,
                                   int pattern, int block_size, int q_block, int sub_rows,
                                   int32_t* h_row_ptr, int32_t* h_entries, int capacity,
                                   int* n_entries) {
  if (!h_row_ptr || !n_entries) return TMAC_ERR_NULL;
  int st = check_mask_args(S, window, n_persistent, pattern, block_size);
  if (st != TMAC_OK) return st;
  if (q_block <= 0 || sub_rows <= 0 || q_block % sub_rows != 0 || q_block / sub_rows > 8)
    return TMAC_ERR_SHAPE;
  const int n_sub = q_block / sub_rows;
  const int n_qb = (S + q_block - 1) / q_block;
  const int n_kt = (S + TMAC_BLOCK - 1) / TMAC_BLOCK;
  if (n_kt > 0xffff) return TMAC_ERR_SHAPE;
  std::vector<RowSpan> spans(S);
  for (int i = 0; i < S; ++i)
    spans[i] = row_span(i, S, window, n_persistent, causal != 0, pattern, block_size);
  int count = 0;
  h_row_ptr[0] = 0;
  for (int qb = 0; qb < n_qb; ++qb) {
    for (int kt = 0; kt < n_kt; ++kt) {
      uint32_t kinds = 0;
      for (int j = 0; j < n_sub; ++j) {
        const int q0 = qb * q_block + j * sub_rows;
        const uint8_t k = tile_kind(spans, S, q0, q0 + sub_rows, kt * TMAC_BLOCK,
                                    kt * TMAC_BLOCK + TMAC_BLOCK);
        kinds |= static_cast<uint32_t>(k) << (2 * j);
      }
      if (kinds == 0) continue;
      if (h_entries) {
        if (count >= capacity) return TMAC_ERR_CAPACITY;
        h_entries[count] = static_cast<int32_t>(static_cast<uint32_t>(kt) | (kinds << 16));
      }
      ++count;
    }
    h_row_ptr[qb + 1] = count;
  }
  *n_entries = count;
  return TMAC_OK;
}

extern "C" int tmac_wattn_schedule_kv(int S, int window, int n_persistent, int causal,
                                      int pattern, int block_size, int k_block, int sub_cols,
                                      int32_t* h_col_ptr, int32_t* h_entries, int capacity,
                                      int* n_entries) {
  if (!h_col_ptr || !n_entries) return TMAC_ERR_NULL;
  int st = check_mask_args(S, window, n_persistent, pattern, block_size);
  if (st != TMAC_OK) return st;
  if (k_block <= 0 || sub_cols <= 0 || k_block % sub_cols != 0 || k_block / sub_cols > 8)
    return TMAC_ERR_SHAPE;
  const int n_sub = k_block / sub_cols;
  const int n_kb = (S + k_block - 1) / k_block;
  const int n_qt = (S + TMAC_BLOCK - 1) / TMAC_BLOCK;
  if (n_qt > 0xffff) return TMAC_ERR_SHAPE;
  std::vector<RowSpan> spans(S);
  for (int i = 0; i < S; ++i)
    spans[i] = row_span(i, S, window, n_persistent, causal != 0, pattern, block_size);
  int count = 0;
  h_col_ptr[0] = 0;
  for (int kb = 0; kb < n_kb; ++kb) {
    for (int qt = 0; qt < n_qt; ++qt) {
      uint32_t kinds = 0;
      for (int j = 0; j < n_sub; ++j) {
        const int k0 = kb * k_block + j * sub_cols;
        const uint8_t k = tile_kind(spans, S, qt * TMAC_BLOCK, qt * TMAC_BLOCK + TMAC_BLOCK, k0,
                                    k0 + sub_cols);
        kinds |= static_cast<uint32_t>(k) << (2 * j);
      }
      if (kinds == 0) continue;
      if (h_entries) {
        if (count >= capacity) return TMAC_ERR_CAPACITY;
        h_entries[count] = static_cast<int32_t>(static_cast<uint32_t>(qt) | (kinds << 16));
      }
      ++count;
    }
    h_col_ptr[kb + 1] = count;
  }
  *n_entries = count;
  return TMAC_OK;
}

extern "C" int tmac_wattn_launch_order(const int32_t* h_ptr, int n_blocks, int32_t* h_order,
                                       int* n_lead) {
  if (!h_ptr || !h_order || !n_lead) return TMAC_ERR_NULL;
  if (n_blocks <= 0) return TMAC_ERR_SHAPE;
  std::vector<int64_t> len(n_blocks);
  int64_t total = 0;
  for (int i = 0; i < n_blocks; ++i) {
    len[i] = static_cast<int64_t>(h_ptr[i + 1]) - h_ptr[i];
    if (len[i] < 0) return TMAC_ERR_VALUE;
    total += len[i];
  }
  for (int i = 0; i < n_blocks; ++i) h_order[i] = i;
  std::stable_sort(h_order, h_order + n_blocks,
                   [&](int32_t a, int32_t b) { return len[a] > len[b]; });
  // A block is "leading" when its list is at least twice the mean length.
  int lead = 0;
  while (lead < n_blocks && len[h_order[lead]] * n_blocks >= 2 * total && total > 0) ++lead;
  *n_lead = lead;
  return TMAC_OK;
}

extern "C" int tmac_wattn_mask_spans(int S, int window, int n_persistent, int causal, int pattern,
                                     int block_size, int32_t* h_rows, int32_t* h_cols) {
  if (!h_rows || !h_cols) return TMAC_ERR_NULL;
  int st = check_mask_args(S, window, n_persistent, pattern, block_size);
  if (st != TMAC_OK) return st;
  const tmac::MaskParams mp{S, std::min(window, S), n_persistent, causal ? 1 : 0, pattern,
                            block_size};
  for (int i = 0; i < S; ++i) {
    const tmac::Span r = tmac::mask_row_span(mp, i), c = tmac::mask_col_span(mp, i);
    h_rows[3 * i] = r.np;
    h_rows[3 * i + 1] = r.lo;
    h_rows[3 * i + 2] = r.hi;
    h_cols[3 * i] = c.np;
    h_cols[3 * i + 1] = c.lo;
    h_cols[3 * i + 2] = c.hi;
  }
  return TMAC_OK;
}
