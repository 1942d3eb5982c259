// Windowed + persistent-token attention forward for gfx950 (MI355X).
//
// O = softmax(Q·Kᵀ·scale + mask)·V where the mask is the band pattern of
// build_band_mask (attn/windowed_attention.py:97-152) or the block-window
// pattern of BlockSparseAttention (attn/block_sparse_attention.py:277-334).
// Only key tiles with at least one allowed pair are visited; the host builds
// that work list once per (S, pattern) (tmac_wattn_schedule).
//
// 16-bit path (bf16 / fp16): a workgroup of 4 waves owns 128 query rows of
// one (batch, head); wave w owns rows 32w..32w+31. For each listed 64-key tile
// the K and V tiles are staged once in LDS (double-buffered, register
// prefetch of the next tile) and every wave whose 32-row slice is not empty
// against the tile
//   1. computes Sᵀ = K·Qᵀ (keys x queries) with v_mfma_f32_32x32x16: K rows
//      are the A operand (16-byte LDS reads), the wave's Q rows sit in
//      registers as the B operand for the whole kernel;
//   2. applies the element mask only on tiles classified partial;
//   3. runs the online softmax in fp32. In the Sᵀ layout every lane holds one
//      query row, so row max and row sum need a single exchange between lanes
//      l and l+32;
//   4. computes Oᵀ += Vᵀ·Pᵀ: the probabilities stay in registers as the B
//      operand (their accumulator layout already is a valid operand layout,
//      with the key order permuted), and Vᵀ comes from the row-major V tile
//      through ds_read_b64_tr_b16 in the same permuted key order.
// The output keeps one query row per lane, so normalisation needs no exchange.
//
// fp32 path (fp32 modules): the same structure on v_mfma_f32_32x32x2_f32,
// fp32 products and sums (wattn_fwd_f32m_kernel).

#include <math.h>

#include <initializer_list>
#include <mutex>

#include "tmac_device.h"

using namespace tmac;

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Masking of a partial 32-wide half tile: v[j] keeps its score where bit
// 8(j/4) + j%4 of w is set, else -inf. w holds this lane's 32 positions of the
// half tile, shifted to the lane's origin. The bit, moved to the sign and
// shifted back, is an all-ones or zero mask that selects between the score and
// -inf bit by bit (two instructions per element).
__device__ __forceinline__ void apply_bits(f32x16& v, uint32_t w) {
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int bit = 8 * (j >> 2) + (j & 3);
    const uint32_t keep = static_cast<uint32_t>(static_cast<int32_t>(w << (31 - bit)) >> 31);
    v[j] = __uint_as_float((__float_as_uint(v[j]) & keep) | (0xff800000u & ~keep));
  }
}

// Bits [0, n) of a 32-bit word (none for n <= 0, all for n >= 32).
__device__ __forceinline__ uint32_t below32(int n) {
  return n <= 0 ? 0u : (n >= 32 ? ~0u : (1u << n) - 1u);
}

// Bit t (t < 32) set iff position o + t lies in the span: t < np - o, or
// lo - o <= t <= hi - o. Built once per half tile for apply_bits.
__device__ __forceinline__ uint32_t span_bits32(const Span& s, int o) {
  return below32(s.np - o) | (below32(s.hi - o + 1) & ~below32(s.lo - o));
}

// Register operands loaded once before a tile loop (this lane's Q, K or V rows)
// are handed through an empty asm statement, so the compiler waits for their
// loads there, once. Otherwise the loop's entry state (these loads pending) and
// back edge (the next tile's prefetch pending) merge, and it waits for the
// prefetch before the first MFMA of every tile.
__device__ __forceinline__ void settle(u32x4& v) { asm volatile("" : "+v"(v)); }

// Row log-sum-exp in log2 units for the backward. A row that a caller's mask
// masks fully has lse = -inf (and output 0): it gets +inf, so each of its
// probabilities exp2(s - l2) is 0 (also for s = -inf).
template <bool CM>
__device__ __forceinline__ float lse_log2(float lse) {
  const float l2 = lse * kLog2e;
  if constexpr (CM) return lse == -INFINITY ? INFINITY : l2;
  return l2;
}

// 64-row tiles of head dimension D (32, 64 or 128) in LDS: rows padded to
// D + 8 elements, so the 16-byte row reads of 16 consecutive rows and the
// transpose reads of 4 rows hit distinct banks. 256 threads stage one tile in
// D / 32 passes of 16-byte chunks (D / 8 chunks per row, 2048 / D rows a pass).
template <int D>
struct Tile {
  static_assert(D == 32 || D == 64 || D == 128, "head dimension 32, 64 or 128");
  static constexpr int kP = D + 8;        // row pitch, elements
  static constexpr int kElems = 64 * kP;  // one tile
  static constexpr int kCpr = D / 8;      // 16-byte chunks per row
  static constexpr int kRpp = 256 / kCpr; // rows per staging pass
  static constexpr int kPasses = D / 32;  // staging passes per tile
  static constexpr int kKk = D / 16;      // MFMA k-steps over the head dimension
  static constexpr int kDt = D / 32;      // 32-wide head-dimension tiles of an output
};

// Four workgroups per CU at D <= 64 (at most 128 VGPRs, 36 KB of LDS each); with
// dropout or a bool mask three (their extra state would spill at 128 VGPRs); two at
// D = 128 and with an additive mask (whose bias path takes about 180 VGPRs).
//
// FEAT (kFeatMask, kFeatDrop, kFeatBool bits, tmac_device.h): with kFeatMask the caller's mask
// tensor replaces the pattern (work lists built from it on the device, partial
// slices masked element by element from the tensor, scores kept in log2 units
// with the mask's bias added); with kFeatDrop each probability that enters O·V is
// kept with probability 1 - p and scaled by 1 / (1 - p) (Philox draws), while the
// row sum takes the undropped probabilities (dropout follows the softmax).
template <int DT, int D, int FEAT = 0>
__global__ __launch_bounds__(256, D > 64 ? 2
                                  : FEAT == 0 ? 4
                                  : ((FEAT & kFeatMask) && !(FEAT & kFeatBool)) ? 2 : 3)
void wattn_fwd_mfma_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
    uint16_t* __restrict__ O, float* __restrict__ lse, int64_t qsb, int64_t qsh, int64_t qss,
    int64_t ksb, int64_t ksh, int64_t kss, int64_t vsb, int64_t vsh, int64_t vss, int64_t osb,
    int64_t osh, int64_t oss, int H, MaskParams mp, float scale_log2,
    const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ entries,
    const int32_t* __restrict__ order, WorkMap wm, AttnX ax) {
  constexpr bool CM = (FEAT & kFeatMask) != 0, DR = (FEAT & kFeatDrop) != 0;
  using T = Tile<D>;
  // [buffer][K, V] 64 x D tiles.
  __shared__ __attribute__((aligned(16))) uint16_t smem[4 * T::kElems];

  int bh, qb;
  if (!work_item(wm, order, bh, qb)) return;
  const int b = bh / H, hd = bh - b * H;
  const int S = mp.S;

  const int tid = threadIdx.x;
  // The wave index is uniform; saying so keeps the tile kinds and their branches scalar.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int l32 = lane & 31, h = lane >> 5;
  const int grp = (lane >> 4) & 1;
  const int q_row = qb * 128 + wave * 32 + l32;  // this lane's query row
  const Span span = mask_row_span(mp, q_row);    // its allowed keys (partial tiles only)

  const uint16_t* Kbh = K + b * ksb + hd * ksh;
  const uint16_t* Vbh = V + b * vsb + hd * vsh;

  // Q rows as the B operand of Sᵀ = K·Qᵀ: lane holds Q[row][16kk + 8h .. +8].
  u32x4 qf[T::kKk];
  {
    const uint16_t* qp = Q + b * qsb + hd * qsh + static_cast<int64_t>(min(q_row, S - 1)) * qss + 8 * h;
#pragma unroll
    for (int kk = 0; kk < T::kKk; ++kk) qf[kk] = ldg16(qp + 16 * kk);
#pragma unroll
    for (int kk = 0; kk < T::kKk; ++kk) settle(qf[kk]);
  }

  int e0, e1, mrow = 0;
  if constexpr (CM) {
    mrow = mask_row(ax, b, hd);
    const int row = mrow * ((S + 127) >> 7) + qb;
    e0 = row * ax.cap;
    e1 = e0 + ax.cnt[row];
  } else {
    e0 = row_ptr[qb];
    e1 = row_ptr[qb + 1];
  }
  // Scores enter the softmax as st * sc: raw scores times scale·log2e, or, with a
  // caller's mask, already in log2 units (sc = 1).
  const float sc = CM ? 1.f : scale_log2;
  // caller's mask: this row's allowed-key bits of the current and the next tile
  uint64_t wb = 0, wb_next = 0;

  // K/V tile staging: T::kPasses 16-byte chunks of each tile per thread (rows
  // r0 + pass * T::kRpp, chunk tid % T::kCpr). Offsets within a tile are fixed per
  // thread; only the last tile of a sequence whose length is not a multiple of 64
  // needs its rows clamped.
  u32x4 pre[2 * T::kPasses];
  const int r0 = tid / T::kCpr, c8 = (tid % T::kCpr) * 8;
  int64_t koff[T::kPasses], voff[T::kPasses];
#pragma unroll
  for (int p = 0; p < T::kPasses; ++p) {
    koff[p] = static_cast<int64_t>(r0 + p * T::kRpp) * kss + c8;
    voff[p] = static_cast<int64_t>(r0 + p * T::kRpp) * vss + c8;
  }
  auto gload = [&](int kt) __attribute__((always_inline)) {
    if (kt * 64 + 64 <= S) {
      const uint16_t* kb = Kbh + static_cast<int64_t>(kt) * 64 * kss;
      const uint16_t* vb = Vbh + static_cast<int64_t>(kt) * 64 * vss;
#pragma unroll
      for (int p = 0; p < T::kPasses; ++p) {
        pre[p] = ldg16(kb + koff[p]);
        pre[T::kPasses + p] = ldg16(vb + voff[p]);
      }
    } else {
#pragma unroll
      for (int p = 0; p < T::kPasses; ++p) {
        const int key = min(kt * 64 + r0 + p * T::kRpp, S - 1);  // rows past S: always masked
        pre[p] = ldg16(Kbh + key * kss + c8);
        pre[T::kPasses + p] = ldg16(Vbh + key * vss + c8);
      }
    }
  };
  auto sstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int p = 0; p < T::kPasses; ++p) {
      const int off = (r0 + p * T::kRpp) * T::kP + c8;
      sts16(smem + (2 * buf) * T::kElems + off, pre[p]);
      sts16(smem + (2 * buf + 1) * T::kElems + off, pre[T::kPasses + p]);
    }
  };

  f32x16 ot[T::kDt];
#pragma unroll
  for (int dt = 0; dt < T::kDt; ++dt) ot[dt] = f32x16{};
  // Online softmax with a lazily moved reference: P = exp2(S·c − m_ref) with c =
  // scale·log2e, and m_ref (scaled units) moves, rescaling O and the row sum, only
  // when a tile's row maximum exceeds it by more than kTau. P then stays <= 2^kTau,
  // which neither the 16-bit P operand (relative rounding) nor the fp32 sums mind,
  // and the 32 accumulator multiplies run only on the rare tiles that move it.
  constexpr float kTau = 8.f;
  float m_ref = -INFINITY, l_run = 0.f;

  if (e0 < e1) {
    gload(entries[e0] & 0xffff);
    if constexpr (CM) wb = mask_word(ax, mrow, q_row, entries[e0] & 0xffff, S);
    sstore(0);
  }
  __syncthreads();
  int buf = 0;
  for (int e = e0; e < e1; ++e) {
    const int ent = entries[e];
    const int kt = ent & 0xffff;
    const int kind = (ent >> (16 + 2 * wave)) & 3;
    const bool more = e + 1 < e1;
    if (more) {
      gload(entries[e + 1] & 0xffff);
      if constexpr (CM) wb_next = mask_word(ax, mrow, q_row, entries[e + 1] & 0xffff, S);
    }

    if (kind != 0) {
      const uint16_t* kt_lds = smem + (2 * buf) * T::kElems;
      const uint16_t* vt_lds = smem + (2 * buf + 1) * T::kElems;
      f32x16 st[2];
      st[0] = f32x16{};
      st[1] = f32x16{};
#pragma unroll
      for (int kk = 0; kk < T::kKk; ++kk)
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
          const u32x4 a = lds16(kt_lds + (32 * kh + l32) * T::kP + 16 * kk + 8 * h);
          st[kh] = Mfma<DT>::run(a, qf[kk], st[kh]);
        }
      // st[kh][j] = S[q_row][key], key = kt*64 + 32kh + 8(j/4) + 4h + j%4 (raw
      // scores; scale_log2 > 0, so the row maximum commutes with the scaling).
      if constexpr (CM) {
        // log2 units; partial slices take -inf from the mask's bits (kind 2) or
        // add the mask's bias element by element (kind 3)
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) st[kh] *= scale_log2;
        if (kind == 2) {
          const uint64_t w = wb >> (4 * h);
          apply_bits(st[0], static_cast<uint32_t>(w));
          apply_bits(st[1], static_cast<uint32_t>(w >> 32));
        } else if (!(FEAT & kFeatBool) && kind == 3) {
#pragma unroll
          for (int kh = 0; kh < 2; ++kh)
#pragma unroll
            for (int j = 0; j < 16; ++j) {
              const int key = kt * 64 + 32 * kh + 8 * (j >> 2) + 4 * h + (j & 3);
              st[kh][j] += mask_bias(ax, b, hd, q_row, key, S) * kLog2e;
            }
        }
      } else if (kind == 2) {
        // key - (kt*64 + 32kh + 4h) is 8(j/4) + j%4: the span as bits from this
        // lane's origin in each half
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) apply_bits(st[kh], span_bits32(span, kt * 64 + 32 * kh + 4 * h));
      }
      float mx = -INFINITY;
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int j = 0; j < 16; ++j) mx = fmaxf(mx, st[kh][j]);
      mx = xor32_max(mx) * sc;
      const bool move = mx > m_ref + kTau;  // false while the row is fully masked
      if (__builtin_amdgcn_ballot_w64(move)) {
        // lanes that keep their reference scale by 1 (also when it is still -inf)
        const float alpha = move ? __builtin_amdgcn_exp2f(m_ref - mx) : 1.f;  // 0 from -inf
        const float m_new = move ? mx : m_ref;
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < T::kDt; ++dt) ot[dt] *= alpha;
        m_ref = m_new;
      }
      const float m_use = (m_ref == -INFINITY) ? 0.f : m_ref;

      // Pᵀ as the B operand, 16 keys per MFMA: k-step ks covers keys
      // 16ks..16ks+15 and lane t-th value is key 16ks + 8(t/4) + 4h + t%4. The
      // row sum stays in fp32, in four chains started by the first k-step.
      u32x4 pb[4];
      float r4[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int kh = ks >> 1, j0 = 8 * (ks & 1);
        // dropout factors of the 8 keys: 16ks + 4h + 0..3 and 16ks + 8 + 4h + 0..3
        float z[8] = {1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f};
        if constexpr (DR) drop_row8(ax, bh, q_row, kt * 64 + 16 * ks, h, z);
        uint32_t w[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float p0 = __builtin_amdgcn_exp2f(fmaf(st[kh][j0 + 2 * t], sc, -m_use));
          const float p1 = __builtin_amdgcn_exp2f(fmaf(st[kh][j0 + 2 * t + 1], sc, -m_use));
          if constexpr (DR)
            w[t] = Mfma<DT>::pack2(p0 * z[2 * t], p1 * z[2 * t + 1]);
          else
            w[t] = Mfma<DT>::pack2(p0, p1);
          r4[t] = ks == 0 ? p0 + p1 : r4[t] + (p0 + p1);
        }
        pb[ks] = u32x4{w[0], w[1], w[2], w[3]};
      }
      l_run += xor32_add((r4[0] + r4[1]) + (r4[2] + r4[3]));
      // Vᵀ as the A operand in the same key order: rows 16ks + 4h + 0..3, then
      // 16ks + 8 + 4h + 0..3 of the V tile, column dh = 32dt + lane%32.
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int dt = 0; dt < T::kDt; ++dt) {
          const u32x4 va = lds_read_tr4x2<T::kP>(vt_lds, 16 * ks + 4 * h, 16 * ks + 8 + 4 * h,
                                                 32 * dt + 16 * grp, lane);
          ot[dt] = Mfma<DT>::run(va, pb[ks], ot[dt]);
        }
    }
    if (more) sstore(buf ^ 1);
    if constexpr (CM) wb = wb_next;
    __syncthreads();
    buf ^= 1;
  }

  if (q_row >= S) return;
  const float inv_l = l_run > 0.f ? 1.f / l_run : 0.f;
  uint16_t* op = O + b * osb + hd * osh + static_cast<int64_t>(q_row) * oss;
  // ot[dt][j] = O[q_row][32dt + 8(j/4) + 4h + j%4]: four consecutive dh per j/4.
#pragma unroll
  for (int dt = 0; dt < T::kDt; ++dt)
#pragma unroll
    for (int jg = 0; jg < 4; ++jg) {
      u32x2 packed;
      packed.x = Mfma<DT>::pack2(ot[dt][4 * jg] * inv_l, ot[dt][4 * jg + 1] * inv_l);
      packed.y = Mfma<DT>::pack2(ot[dt][4 * jg + 2] * inv_l, ot[dt][4 * jg + 3] * inv_l);
      *reinterpret_cast<u32x2*>(op + 32 * dt + 8 * jg + 4 * h) = packed;
    }
  if (lse && h == 0)
    lse[(static_cast<int64_t>(b) * H + hd) * S + q_row] = (m_ref + __log2f(l_run)) * kLn2;
}

// fp32 path on the matrix cores (head dimension 32, 64 or 128): the structure of
// wattn_fwd_mfma_kernel with v_mfma_f32_32x32x2_f32
// (fp32 products and sums). A workgroup of 4 waves owns 128 query rows, wave w
// rows 32w..32w+31, and per listed 64-key tile:
//   - Sᵀ = K·Qᵀ: an MFMA k-step sums two head dimensions, one per lane half
//     (k-step s: dimension s in lanes 0-31, D/2 + s in lanes 32-63). Each lane
//     holds the D/2 contiguous dimensions of its query row that its half
//     needs, pre-multiplied by scale·log2e (B operand), and reads the same
//     slice of a key row from LDS in 16-byte chunks (A operand);
//   - masking and the online softmax as in the 16-bit kernel (same accumulator
//     layout: lane = query row, keys 32kh + 8(j/4) + 4h + j%4);
//   - Oᵀ += Vᵀ·Pᵀ with k-steps over key pairs: k-step s of key half kh takes
//     key 32kh + 8(s/4) + 4h + s%4 in lane half h, where the Sᵀ accumulator
//     left that lane's probability, so Pᵀ is used in place and Vᵀ is one
//     4-byte LDS read per lane and k-step.
// K and V tiles are staged with rows padded to D + 4 floats, double-buffered
// with a register prefetch of the next tile (two workgroups per CU; one at head
// dimension 128, where LDS and the register file hold one). FEAT as for the 16-bit kernel: the
// caller's mask from its device work lists (scores in log2 units, partial slices
// from the allowed-pair bits or the mask's bias), dropout factors on the P·V
// operand while the row sum takes the undropped probabilities.
template <int D, int FEAT = 0>
__global__ __launch_bounds__(256, D > 64 ? 1 : 2) void wattn_fwd_f32m_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    float* __restrict__ O, float* __restrict__ lse, int64_t qsb, int64_t qsh, int64_t qss,
    int64_t ksb, int64_t ksh, int64_t kss, int64_t vsb, int64_t vsh, int64_t vss, int64_t osb,
    int64_t osh, int64_t oss, int H, MaskParams mp, float scale_log2,
    const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ entries,
    const int32_t* __restrict__ order, WorkMap wm, AttnX ax) {
  static_assert(D == 32 || D == 64 || D == 128, "head dimension 32, 64 or 128");
  constexpr bool CM = (FEAT & kFeatMask) != 0, DR = (FEAT & kFeatDrop) != 0;
  constexpr int kP = D + 4;           // row pitch, floats
  constexpr int kTile = 64 * kP;      // one staged tile, floats
  constexpr int kHalf = D / 2;        // Sᵀ k-steps; dimensions per lane
  constexpr int kDt = D / 32;         // 32-wide dimension tiles of O
  constexpr int kC4 = D / 4;          // 16-byte chunks per row
  constexpr int kRpp = 256 / kC4;     // rows per staging pass
  constexpr int kPasses = 64 / kRpp;  // staging passes per tile
  // [buffer][K, V] 64 x D tiles
  __shared__ __attribute__((aligned(16))) float smem[4 * kTile];

  int bh, qb;
  if (!work_item(wm, order, bh, qb)) return;
  const int b = bh / H, hd = bh - b * H;
  const int S = mp.S;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int l32 = lane & 31, h = lane >> 5;
  const int q_row = qb * 128 + wave * 32 + l32;
  const Span span = mask_row_span(mp, q_row);

  const float* Kbh = K + b * ksb + hd * ksh;
  const float* Vbh = V + b * vsb + hd * vsh;

  float qf[kHalf];
  {
    const float* qp = Q + b * qsb + hd * qsh + static_cast<int64_t>(min(q_row, S - 1)) * qss + h * kHalf;
#pragma unroll
    for (int c = 0; c < kHalf; c += 4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(qp + c);
      qf[c] = v.x * scale_log2;
      qf[c + 1] = v.y * scale_log2;
      qf[c + 2] = v.z * scale_log2;
      qf[c + 3] = v.w * scale_log2;
    }
  }
  int e0, e1, mrow = 0;
  if constexpr (CM) {
    mrow = mask_row(ax, b, hd);
    const int row = mrow * ((S + 127) >> 7) + qb;
    e0 = row * ax.cap;
    e1 = e0 + ax.cnt[row];
  } else {
    e0 = row_ptr[qb];
    e1 = row_ptr[qb + 1];
  }
  uint64_t wb = 0, wb_next = 0;  // caller's mask: this row's allowed-key bits, two tiles

  // Staging: pass p moves row r0 + p * kRpp, chunk tid % kC4, of both tiles.
  f32x4 pre[2 * kPasses];
  const int r0 = tid / kC4, c4 = (tid % kC4) * 4;
  auto gload = [&](int kt) __attribute__((always_inline)) {
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int key = min(kt * 64 + r0 + p * kRpp, S - 1);  // rows past S: always masked
      pre[p] = *reinterpret_cast<const f32x4*>(Kbh + key * kss + c4);
      pre[kPasses + p] = *reinterpret_cast<const f32x4*>(Vbh + key * vss + c4);
    }
  };
  auto sstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int off = (r0 + p * kRpp) * kP + c4;
      *reinterpret_cast<f32x4*>(smem + (2 * buf) * kTile + off) = pre[p];
      *reinterpret_cast<f32x4*>(smem + (2 * buf + 1) * kTile + off) = pre[kPasses + p];
    }
  };

  f32x16 ot[kDt];
#pragma unroll
  for (int dt = 0; dt < kDt; ++dt) ot[dt] = f32x16{};
  constexpr float kTau = 8.f;  // lazy reference, as in the 16-bit kernel
  float m_ref = -INFINITY, l_run = 0.f;

  if (e0 < e1) {
    gload(entries[e0] & 0xffff);
    if constexpr (CM) wb = mask_word(ax, mrow, q_row, entries[e0] & 0xffff, S);
    sstore(0);
  }
  __syncthreads();
  int buf = 0;
  for (int e = e0; e < e1; ++e) {
    const int ent = entries[e];
    const int kt = ent & 0xffff;
    const int kind = (ent >> (16 + 2 * wave)) & 3;
    const bool more = e + 1 < e1;
    if (more) {
      gload(entries[e + 1] & 0xffff);
      if constexpr (CM) wb_next = mask_word(ax, mrow, q_row, entries[e + 1] & 0xffff, S);
    }

    if (kind != 0) {
      const float* kt_lds = smem + (2 * buf) * kTile;
      const float* vt_lds = smem + (2 * buf + 1) * kTile;
      f32x16 st[2];
      st[0] = f32x16{};
      st[1] = f32x16{};
#pragma unroll
      for (int c = 0; c < kHalf; c += 4) {
        f32x4 a4[2];
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
          a4[kh] = *reinterpret_cast<const f32x4*>(kt_lds + (32 * kh + l32) * kP + h * kHalf + c);
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int kh = 0; kh < 2; ++kh)
            st[kh] = __builtin_amdgcn_mfma_f32_32x32x2f32(a4[kh][t], qf[c + t], st[kh], 0, 0, 0);
      }
      // st[kh][j] = S[q_row][key]·scale·log2e, key = kt*64 + 32kh + 8(j/4) + 4h + j%4
      if constexpr (CM) {
        if (kind == 2) {
          const uint64_t w = wb >> (4 * h);
          apply_bits(st[0], static_cast<uint32_t>(w));
          apply_bits(st[1], static_cast<uint32_t>(w >> 32));
        } else if (!(FEAT & kFeatBool) && kind == 3) {
#pragma unroll
          for (int kh = 0; kh < 2; ++kh)
#pragma unroll
            for (int j = 0; j < 16; ++j) {
              const int key = kt * 64 + 32 * kh + 8 * (j >> 2) + 4 * h + (j & 3);
              st[kh][j] += mask_bias(ax, b, hd, q_row, key, S) * kLog2e;
            }
        }
      } else if (kind == 2) {
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) apply_bits(st[kh], span_bits32(span, kt * 64 + 32 * kh + 4 * h));
      }
      float mx = -INFINITY;
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int j = 0; j < 16; ++j) mx = fmaxf(mx, st[kh][j]);
      mx = xor32_max(mx);
      const bool move = mx > m_ref + kTau;  // false while the row is fully masked
      if (__builtin_amdgcn_ballot_w64(move)) {
        const float alpha = move ? __builtin_amdgcn_exp2f(m_ref - mx) : 1.f;  // 0 from -inf
        const float m_new = move ? mx : m_ref;
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < kDt; ++dt) ot[dt] *= alpha;
        m_ref = m_new;
      }
      const float m_use = (m_ref == -INFINITY) ? 0.f : m_ref;
      float r4[4];
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const float p = __builtin_amdgcn_exp2f(st[kh][j] - m_use);
          st[kh][j] = p;
          r4[j & 3] = (kh == 0 && j < 4) ? p : r4[j & 3] + p;
        }
      l_run += xor32_add((r4[0] + r4[1]) + (r4[2] + r4[3]));
      if constexpr (DR) {
        // P ⊙ Z for O: elements 8m + t and 8m + 4 + t are keys 16m + 4h + t and
        // 16m + 8 + 4h + t of the half
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
#pragma unroll
          for (int m = 0; m < 2; ++m) {
            float z8[8];
            drop_row8(ax, bh, q_row, kt * 64 + 32 * kh + 16 * m, h, z8);
#pragma unroll
            for (int t = 0; t < 8; ++t) st[kh][8 * m + t] *= z8[t];
          }
      }
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int s = 0; s < 16; ++s) {
          const int key = 32 * kh + 8 * (s >> 2) + 4 * h + (s & 3);
#pragma unroll
          for (int dt = 0; dt < kDt; ++dt)
            ot[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vt_lds[key * kP + 32 * dt + l32], st[kh][s],
                                                          ot[dt], 0, 0, 0);
        }
    }
    if (more) sstore(buf ^ 1);
    if constexpr (CM) wb = wb_next;
    __syncthreads();
    buf ^= 1;
  }

  if (q_row >= S) return;
  const float inv_l = l_run > 0.f ? 1.f / l_run : 0.f;
  float* op = O + b * osb + hd * osh + static_cast<int64_t>(q_row) * oss;
  // ot[dt][j] = O[q_row][32dt + 8(j/4) + 4h + j%4]: four consecutive dimensions per j/4.
#pragma unroll
  for (int dt = 0; dt < kDt; ++dt)
#pragma unroll
    for (int jg = 0; jg < 4; ++jg)
      *reinterpret_cast<f32x4*>(op + 32 * dt + 8 * jg + 4 * h) =
          f32x4{ot[dt][4 * jg] * inv_l, ot[dt][4 * jg + 1] * inv_l, ot[dt][4 * jg + 2] * inv_l,
                ot[dt][4 * jg + 3] * inv_l};
  if (lse && h == 0)
    lse[(static_cast<int64_t>(b) * H + hd) * S + q_row] = (m_ref + __log2f(l_run)) * kLn2;
}

// ---------------------------------------------------------------------------
// Backward (16-bit MFMA path). With P = softmax(S) recomputed from the
// forward's log-sum-exp, Δ = rowsum(dO ⊙ O):
//   dV = Pᵀ·dO,  dS = P ⊙ (dO·Vᵀ − Δ),  dK = scale·dSᵀ·Q,  dQ = scale·dS·K.
// Two kernels, no atomics (results are deterministic): wattn_bwd_q_kernel owns
// 128 queries, walks the forward's work list and also writes Δ of its rows;
// then wattn_bwd_kv_kernel owns 128 keys and walks the query tiles that touch
// them (key-major work list, tmac_wattn_schedule_kv). Both recompute S and dP
// with MFMAs.
// ---------------------------------------------------------------------------

// Packs accumulator values v[j0 + 2t], v[j0 + 2t + 1] (t = 0..3) into one
// 16-bit MFMA operand (eight values, in the permuted key/query order of the
// 32x32 accumulator layout).
template <int DT>
__device__ __forceinline__ u32x4 pack8(const f32x16& v, int j0) {
  uint32_t w[4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
    w[t] = Mfma<DT>::pack2(v[j0 + 2 * t], v[j0 + 2 * t + 1]);
  return u32x4{w[0], w[1], w[2], w[3]};
}

// Stores the transposed accumulators acc[dt] (lane = row `row`, entries
// 32dt + 8(j/4) + 4h + j%4 of the 32*NDT columns) into row `row` of a 16-bit
// tensor, multiplied by `mul`: four consecutive columns per 8-byte store.
template <int DT, int NDT>
__device__ __forceinline__ void store_row(uint16_t* rowp, const f32x16 (&acc)[NDT], float mul,
                                          int h) {
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int jg = 0; jg < 4; ++jg) {
      u32x2 packed;
      packed.x = Mfma<DT>::pack2(acc[dt][4 * jg] * mul, acc[dt][4 * jg + 1] * mul);
      packed.y = Mfma<DT>::pack2(acc[dt][4 * jg + 2] * mul, acc[dt][4 * jg + 3] * mul);
      *reinterpret_cast<u32x2*>(rowp + 32 * dt + 8 * jg + 4 * h) = packed;
    }
}

// −Δ of the queries of a 32-query half in accumulator order (element j: row
// 32qh + 8(j/4) + 4h + j%4 of the tile), from the staged −Δ values: the initial
// dP accumulator, so the MFMAs produce dP − Δ.
__device__ __forceinline__ f32x16 neg_delta_acc(const float* ndl_l, int qh, int h) {
  f32x16 r;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const f32x4 d4 = *reinterpret_cast<const f32x4*>(ndl_l + 32 * qh + 8 * g + 4 * h);
    r[4 * g] = d4.x;
    r[4 * g + 1] = d4.y;
    r[4 * g + 2] = d4.z;
    r[4 * g + 3] = d4.w;
  }
  return r;
}

// The vector-ALU and dV/dK part of one 32-query half of a listed tile, for
// the wave's 32 keys (both dK/dV kernels). s holds S of the half (scaled to
// log2 units by sc), element j for query q0 + 8(j/4) + j%4 with q0 = qbase +
// 32qh + 4h; lse_l and ndl_l hold LSE·log2e and −Δ of the tile's 64 queries.
// dp holds dP − Δ (its accumulator started from neg_delta_acc), or, with
// kFeatDrop, dP. Forms P and dS in place (with kFeatDrop, P ⊙ Z for dV and
// P ⊙ (Z ⊙ dP − Δ)), then dVᵀ += dOᵀ·P and dKᵀ += Qᵀ·dS, dOᵀ and Qᵀ taken by
// tr(tile, r0, r1, c0), a transpose read of rows r0..r0+3 and r1..r1+3 at
// column c0 of the staged tile, in the accumulator's permuted query order.
template <int DT, int D, bool DR, class TrRead>
__device__ __forceinline__ void kv_half_update(f32x16& s, f32x16& dp, float sc, const float* lse_l,
                                               const float* ndl_l, int qh, int qbase, int h,
                                               int grp, int lane, int key, int bh,
                                               const AttnX& ax, const uint16_t* q_lds,
                                               const uint16_t* g_lds, f32x16 (&dkt)[D / 32],
                                               f32x16 (&dvt)[D / 32], TrRead tr) {
  // rows 32qh + 8g + 4h + 0..3 of the tile: LSE·log2e (and −Δ) as one 16-byte read each
  uint32_t kq2[2] = {0u, 0u};  // keep bits of query groups (0, 1) and (2, 3)
  if constexpr (DR) {
#pragma unroll
    for (int g2 = 0; g2 < 2; ++g2) {
      const int qa = qbase + 32 * qh + 16 * g2 + 4 * h;
      kq2[g2] = keep_octet2(ax, bh, qa, qa + 8, key, lane & 7);
    }
  }
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const f32x4 l4 = *reinterpret_cast<const f32x4*>(lse_l + 32 * qh + 8 * g + 4 * h);
    const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
    if constexpr (DR) {
      const f32x4 d4 = *reinterpret_cast<const f32x4*>(ndl_l + 32 * qh + 8 * g + 4 * h);
      const float nd[4] = {d4.x, d4.y, d4.z, d4.w};
      const uint32_t kq = kq2[g >> 1] >> (16 * (g & 1));
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int j = 4 * g + t;
        const float pj = __builtin_amdgcn_exp2f(fmaf(s[j], sc, -lv[t]));
        const float z = ((kq >> (4 * t)) & 1u) ? ax.keep_scale : 0.f;
        s[j] = pj * z;
        dp[j] = pj * fmaf(z, dp[j], nd[t]);
      }
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int j = 4 * g + t;
        const float pj = __builtin_amdgcn_exp2f(fmaf(s[j], sc, -lv[t]));
        s[j] = pj;
        dp[j] *= pj;
      }
    }
  }
  // dVᵀ[d][key] += Σ_q dO[q][d] P[q][key]; dKᵀ[d][key] += Σ_q Q[q][d] dS[q][key].
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const u32x4 pb = pack8<DT>(s, 8 * ks);
    const u32x4 db = pack8<DT>(dp, 8 * ks);
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
      const int rr = 32 * qh + 16 * ks + 4 * h;
      const u32x4 ga = tr(g_lds, rr, rr + 8, 32 * dt + 16 * grp);
      const u32x4 qa = tr(q_lds, rr, rr + 8, 32 * dt + 16 * grp);
      dvt[dt] = Mfma<DT>::run(ga, pb, dvt[dt]);
      dkt[dt] = Mfma<DT>::run(qa, db, dkt[dt]);
    }
  }
}

// dK, dV. Workgroup = (b, h, 128 keys); wave w owns keys 32w..32w+31 of the
// block, held in registers as the B operands of S = Q·Kᵀ and dP = dO·Vᵀ
// (lane = key). Per listed 64-query tile, Q and dO (plus LSE and Δ of those
// queries) are staged in LDS; for each 32-query half the wave computes S and dP
// (lane = key, 16 queries per lane), P = exp2(S·c − LSE·log2e) and dS, then
// dVᵀ += dOᵀ·P and dKᵀ += Qᵀ·dS, with dOᵀ and Qᵀ read by transpose reads in the
// accumulator's permuted query order and P, dS packed straight from registers.
// FEAT as for the forward: with kFeatDrop, dV takes the dropped probabilities
// P ⊙ Z and dS = P ⊙ (Z ⊙ dP − Δ) (Z the forward's factors, redrawn from the seed).
template <int DT, int D, int FEAT = 0>
__global__ __launch_bounds__(256, D > 64 ? 1 : 2) void wattn_bwd_kv_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
    const uint16_t* __restrict__ dO, const float* __restrict__ lse, const float* __restrict__ delta,
    uint16_t* __restrict__ dK, uint16_t* __restrict__ dV, int64_t qsb, int64_t qsh, int64_t qss,
    int64_t ksb, int64_t ksh, int64_t kss, int64_t vsb, int64_t vsh, int64_t vss, int64_t gsb,
    int64_t gsh, int64_t gss, int64_t dksb, int64_t dksh, int64_t dkss, int64_t dvsb,
    int64_t dvsh, int64_t dvss, int H, MaskParams mp, float scale, float scale_log2,
    const int32_t* __restrict__ col_ptr, const int32_t* __restrict__ entries,
    const int32_t* __restrict__ order, WorkMap wm, AttnX ax) {
  constexpr bool CM = (FEAT & kFeatMask) != 0, DR = (FEAT & kFeatDrop) != 0;
  using T = Tile<D>;
  // [buffer][Q, dO] 64 x D tiles, then [buffer] LSE·log2e and −Δ of the 64 queries.
  __shared__ __attribute__((aligned(16))) uint16_t smem[4 * T::kElems];
  __shared__ __attribute__((aligned(16))) float stat[2][2][64];

  int bh, kb;
  if (!work_item(wm, order, bh, kb)) return;
  const int b = bh / H, hd = bh - b * H;
  const int S = mp.S;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;  // uniform
  const int l32 = lane & 31, h = lane >> 5;
  const int grp = (lane >> 4) & 1;
  const int key = kb * 128 + wave * 32 + l32;  // this lane's key
  const Span span = mask_col_span(mp, key);     // the queries that see it (partial tiles only)

  u32x4 kf[T::kKk], vf[T::kKk];
  {
    const int kc = min(key, S - 1);
    const uint16_t* kp = K + b * ksb + hd * ksh + static_cast<int64_t>(kc) * kss + 8 * h;
    const uint16_t* vp = V + b * vsb + hd * vsh + static_cast<int64_t>(kc) * vss + 8 * h;
#pragma unroll
    for (int kk = 0; kk < T::kKk; ++kk) {
      kf[kk] = ldg16(kp + 16 * kk);
      vf[kk] = ldg16(vp + 16 * kk);
    }
#pragma unroll
    for (int kk = 0; kk < T::kKk; ++kk) {
      settle(kf[kk]);
      settle(vf[kk]);
    }
  }
  const uint16_t* Qbh = Q + b * qsb + hd * qsh;
  const uint16_t* Gbh = dO + b * gsb + hd * gsh;
  const float* lse_bh = lse + static_cast<int64_t>(bh) * S;
  const float* dl_bh = delta + static_cast<int64_t>(bh) * S;

  int e0, e1, mrow = 0;
  if constexpr (CM) {
    mrow = mask_row(ax, b, hd);
    const int row = mrow * ((S + 127) >> 7) + kb;
    e0 = row * ax.cap;
    e1 = e0 + ax.cnt[row];
  } else {
    e0 = col_ptr[kb];
    e1 = col_ptr[kb + 1];
  }
  const float sc = CM ? 1.f : scale_log2;

  u32x4 pre[2 * T::kPasses];
  float st_pre = 0.f;
  const int r0 = tid / T::kCpr, c8 = (tid % T::kCpr) * 8;
  int64_t qoff[T::kPasses], goff[T::kPasses];
#pragma unroll
  for (int p = 0; p < T::kPasses; ++p) {
    qoff[p] = static_cast<int64_t>(r0 + p * T::kRpp) * qss + c8;
    goff[p] = static_cast<int64_t>(r0 + p * T::kRpp) * gss + c8;
  }
  auto gload = [&](int qt) __attribute__((always_inline)) {
    if (qt * 64 + 64 <= S) {
      const uint16_t* qb = Qbh + static_cast<int64_t>(qt) * 64 * qss;
      const uint16_t* gb = Gbh + static_cast<int64_t>(qt) * 64 * gss;
#pragma unroll
      for (int p = 0; p < T::kPasses; ++p) {
        pre[p] = ldg16(qb + qoff[p]);
        pre[T::kPasses + p] = ldg16(gb + goff[p]);
      }
    } else {
#pragma unroll
      for (int p = 0; p < T::kPasses; ++p) {
        const int qr = min(qt * 64 + r0 + p * T::kRpp, S - 1);  // rows past S: always masked
        pre[p] = ldg16(Qbh + qr * qss + c8);
        pre[T::kPasses + p] = ldg16(Gbh + qr * gss + c8);
      }
    }
    // LSE (threads 0-63) and Δ (64-127) of the tile's queries, loaded raw by every
    // thread (threads 128-255 repeat them): an unconditional load that nothing
    // consumes until sstore, so no wait lands here.
    st_pre = ((tid & 64) ? dl_bh : lse_bh)[min(qt * 64 + (tid & 63), S - 1)];
  };
  auto sstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int p = 0; p < T::kPasses; ++p) {
      const int off = (r0 + p * T::kRpp) * T::kP + c8;
      sts16(smem + (2 * buf) * T::kElems + off, pre[p]);
      sts16(smem + (2 * buf + 1) * T::kElems + off, pre[T::kPasses + p]);
    }
    if (tid < 128) stat[buf][tid >> 6][tid & 63] = tid < 64 ? lse_log2<CM>(st_pre) : -st_pre;
  };

  f32x16 dkt[T::kDt], dvt[T::kDt];
#pragma unroll
  for (int dt = 0; dt < T::kDt; ++dt) {
    dkt[dt] = f32x16{};
    dvt[dt] = f32x16{};
  }

  uint64_t wb = 0, wb_next = 0;  // caller's mask: allowed-query bits of this key, two tiles
  if (e0 < e1) {
    gload(entries[e0] & 0xffff);
    if constexpr (CM) wb = mask_word(ax, mrow, key, entries[e0] & 0xffff, S);
    sstore(0);
  }
  __syncthreads();
  int buf = 0;
  for (int e = e0; e < e1; ++e) {
    const int ent = entries[e];
    const int qt = ent & 0xffff;
    const int kind = (ent >> (16 + 2 * wave)) & 3;
    const bool more = e + 1 < e1;
    if (more) {
      gload(entries[e + 1] & 0xffff);
      if constexpr (CM) wb_next = mask_word(ax, mrow, key, entries[e + 1] & 0xffff, S);
    }

    if (kind != 0) {
      const uint16_t* q_lds = smem + (2 * buf) * T::kElems;
      const uint16_t* g_lds = smem + (2 * buf + 1) * T::kElems;
#pragma unroll
      for (int qh = 0; qh < 2; ++qh) {
        f32x16 s = f32x16{};
        f32x16 dp = DR ? f32x16{} : neg_delta_acc(&stat[buf][1][0], qh, h);
#pragma unroll
        for (int kk = 0; kk < T::kKk; ++kk) {
          const u32x4 qa = lds16(q_lds + (32 * qh + l32) * T::kP + 16 * kk + 8 * h);
          const u32x4 ga = lds16(g_lds + (32 * qh + l32) * T::kP + 16 * kk + 8 * h);
          s = Mfma<DT>::run(qa, kf[kk], s);
          dp = Mfma<DT>::run(ga, vf[kk], dp);
        }
        // s[j] = S[query][key], query = qt*64 + 32qh + 8(j/4) + 4h + j%4. The
        // span bounds move to this lane's origin (qt*64 + 32qh + 4h), so each
        // test compares a per-element constant with them.
        if constexpr (CM) {
          s *= scale_log2;
          if (kind == 2) {
            apply_bits(s, static_cast<uint32_t>((wb >> (4 * h)) >> (32 * qh)));
          } else if (!(FEAT & kFeatBool) && kind == 3) {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
              const int qr = qt * 64 + 32 * qh + 8 * (j >> 2) + 4 * h + (j & 3);
              s[j] += mask_bias(ax, b, hd, qr, key, S) * kLog2e;
            }
          }
        } else if (kind == 2) {
          apply_bits(s, span_bits32(span, qt * 64 + 32 * qh + 4 * h));
        }
        kv_half_update<DT, D, DR>(s, dp, sc, &stat[buf][0][0], &stat[buf][1][0], qh, qt * 64, h,
                                  grp, lane, key, bh, ax, q_lds, g_lds, dkt, dvt,
                                  [&](const uint16_t* t, int r0, int r1, int c0) {
                                    return lds_read_tr4x2<T::kP>(t, r0, r1, c0, lane);
                                  });
      }
    }
    if (more) sstore(buf ^ 1);
    if constexpr (CM) wb = wb_next;
    __syncthreads();
    buf ^= 1;
  }

  if (key >= S) return;
  store_row<DT, T::kDt>(dK + b * dksb + hd * dksh + static_cast<int64_t>(key) * dkss, dkt, scale, h);
  store_row<DT, T::kDt>(dV + b * dvsb + hd * dvsh + static_cast<int64_t>(key) * dvss, dvt, 1.f, h);
}

// dK, dV at head dimension 64 (every FEAT; a caller's mask word of the next
// tile is loaded during the current one): the work of wattn_bwd_kv_kernel, with
// the query tiles copied HBM/L2 -> LDS by
// global_load_lds into a ring of four stages, three tiles ahead of the math,
// one barrier per tile. Stage = Q and dO tiles (64 rows of 128 bytes, chunks
// swizzled by swz64: conflict-free for the S/dP operands' 16-byte row reads and
// the dK/dV operands' transpose reads), then LSE·log2e and −Δ of the 64 queries.
// Wave w copies Q and dO rows 16w..16w+15 (two 8-row instructions each); wave 2
// also copies the 64 LSE values and wave 3 the 64 Δ values, each converting
// its values in place once they have landed. Rows past S read row S-1 (always
// masked).
constexpr int kKvStages = 4;
constexpr int kKvTileB = 64 * 128;             // one 64x64 16-bit tile, bytes
constexpr int kKvStageB = 2 * kKvTileB + 512;  // Q, dO, LSE·log2e, Δ

template <int DT, int FEAT = 0>
__global__ __launch_bounds__(256, 2) void wattn_bwd_kv64_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
    const uint16_t* __restrict__ dO, const float* __restrict__ lse, const float* __restrict__ delta,
    uint16_t* __restrict__ dK, uint16_t* __restrict__ dV, int64_t qsb, int64_t qsh, int64_t qss,
    int64_t ksb, int64_t ksh, int64_t kss, int64_t vsb, int64_t vsh, int64_t vss, int64_t gsb,
    int64_t gsh, int64_t gss, int64_t dksb, int64_t dksh, int64_t dkss, int64_t dvsb,
    int64_t dvsh, int64_t dvss, int H, MaskParams mp, float scale, float scale_log2,
    const int32_t* __restrict__ col_ptr, const int32_t* __restrict__ entries,
    const int32_t* __restrict__ order, WorkMap wm, AttnX ax) {
  constexpr int D = 64;
  constexpr bool CM = (FEAT & kFeatMask) != 0, DR = (FEAT & kFeatDrop) != 0;
  using T = Tile<D>;
  __shared__ __attribute__((aligned(16))) uint16_t ring[kKvStages * kKvStageB / 2];

  int bh, kb;
  if (!work_item(wm, order, bh, kb)) return;
  const int b = bh / H, hd = bh - b * H;
  const int S = mp.S;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;  // uniform
  const int l32 = lane & 31, h = lane >> 5;
  const int grp = (lane >> 4) & 1;
  const int key = kb * 128 + wave * 32 + l32;  // this lane's key
  const Span span = mask_col_span(mp, key);     // the queries that see it (partial tiles only)

  u32x4 kf[T::kKk], vf[T::kKk];
  {
    const int kc = min(key, S - 1);
    const uint16_t* kp = K + b * ksb + hd * ksh + static_cast<int64_t>(kc) * kss + 8 * h;
    const uint16_t* vp = V + b * vsb + hd * vsh + static_cast<int64_t>(kc) * vss + 8 * h;
#pragma unroll
    for (int kk = 0; kk < T::kKk; ++kk) {
      kf[kk] = ldg16(kp + 16 * kk);
      vf[kk] = ldg16(vp + 16 * kk);
    }
#pragma unroll
    for (int kk = 0; kk < T::kKk; ++kk) {
      settle(kf[kk]);
      settle(vf[kk]);
    }
  }
  const uint16_t* Qbh = Q + b * qsb + hd * qsh;
  const uint16_t* Gbh = dO + b * gsb + hd * gsh;
  const float* lse_bh = lse + static_cast<int64_t>(bh) * S;
  const float* dl_bh = delta + static_cast<int64_t>(bh) * S;
  int e0, e1, mrow = 0;
  if constexpr (CM) {
    mrow = mask_row(ax, b, hd);
    const int row = mrow * ((S + 127) >> 7) + kb;
    e0 = row * ax.cap;
    e1 = e0 + ax.cnt[row];
  } else {
    e0 = col_ptr[kb];
    e1 = col_ptr[kb + 1];
  }
  const int n = e1 - e0;
  // caller's mask: allowed-query bits of this key in the current and the next tile
  uint64_t wb = 0, wb_next = 0;
  if constexpr (CM) {
    if (n > 0) wb = mask_word(ax, mrow, key, entries[e0] & 0xffff, S);
  }

  // Copies: this wave's rows of Q and dO, chunk positions as for swz64 (lane L
  // of an instruction covering rows R..R+7 fills chunk position L & 7 of row
  // R + L / 8 with the global chunk the swizzle stores there).
  const int drow = lane >> 3, dpos = lane & 7;
  int crow[2];
  uint32_t cchunk[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    crow[j] = 16 * wave + 8 * j + drow;
    const int a = (crow[j] >> 1) & 7;
    cchunk[j] = 16u * static_cast<uint32_t>(dpos ^ (((a & 1) << 2) | (a >> 1)));
  }
  const uint32_t ring0 = lds_offset(ring);
  auto issue = [&](int idx) __attribute__((always_inline)) {
    const int qt = entries[e0 + idx] & 0xffff;
    const uint32_t st = ring0 + static_cast<uint32_t>((idx % kKvStages) * kKvStageB);
    const int lim = S - 1 - qt * 64;  // rows beyond this one read it instead
    const uint16_t* qb = Qbh + static_cast<int64_t>(qt) * 64 * qss;
    const uint16_t* gb = Gbh + static_cast<int64_t>(qt) * 64 * gss;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t r = static_cast<uint32_t>(min(crow[j], lim));
      dma_lds16(qb, r * static_cast<uint32_t>(2 * qss) + cchunk[j], st + (16 * wave + 8 * j) * 128);
      dma_lds16(gb, r * static_cast<uint32_t>(2 * gss) + cchunk[j],
                st + kKvTileB + (16 * wave + 8 * j) * 128);
    }
    if (wave >= 2) {
      const float* sb = wave == 2 ? lse_bh : dl_bh;
      dma_lds4(sb, 4u * static_cast<uint32_t>(min(qt * 64 + lane, S - 1)),
               st + 2 * kKvTileB + (wave - 2) * 256);
    }
  };

  f32x16 dkt[T::kDt], dvt[T::kDt];
#pragma unroll
  for (int dt = 0; dt < T::kDt; ++dt) {
    dkt[dt] = f32x16{};
    dvt[dt] = f32x16{};
  }

  for (int i = 0; i < kKvStages - 1 && i < n; ++i) issue(i);
  for (int i = 0; i < n; ++i) {
    // this wave's copies of tile i have landed when at most those of the (up
    // to kKvStages - 2) later tiles already issued are outstanding: four copies
    // per tile for waves 0-1, five for waves 2-3
    const int later = min(kKvStages - 2, n - 1 - i);
    if (wave >= 2) {
      if (later == 2) asm volatile("s_waitcnt vmcnt(10)" ::: "memory");
      else if (later == 1) asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
      else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else {
      if (later == 2) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
      else if (later == 1) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
      else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    const uint16_t* st = ring + (i % kKvStages) * (kKvStageB / 2);
    float* lse2 = reinterpret_cast<float*>(const_cast<uint16_t*>(st) + 2 * (kKvTileB / 2));
    if (wave >= 2) {
      // LSE -> LSE·log2e (wave 2) and Δ -> −Δ (wave 3), in place (this wave's
      // copy has landed)
      float* v = lse2 + 64 * (wave - 2) + lane;
      *v = wave == 2 ? lse_log2<CM>(*v) : -*v;
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    // every wave's copies of tile i are in LDS (and converted), and every wave
    // is done reading the stage the next copies overwrite (tile i-1's)
    asm volatile("s_barrier" ::: "memory");
    if (i + kKvStages - 1 < n) issue(i + kKvStages - 1);

    const int ent = entries[e0 + i];
    const int qt = ent & 0xffff;
    const int kind = (ent >> (16 + 2 * wave)) & 3;
    if constexpr (CM) {
      if (i + 1 < n) wb_next = mask_word(ax, mrow, key, entries[e0 + i + 1] & 0xffff, S);
    }
    if (kind != 0) {
      const uint16_t* q_lds = st;
      const uint16_t* g_lds = st + kKvTileB / 2;
      const float* lse_l = lse2;
      const float* ndl_l = lse2 + 64;
      // S and dP of both 32-query halves first: the second half's MFMAs run
      // while the first half's softmax is on the vector ALU.
      f32x16 s2[2], dp2[2];
#pragma unroll
      for (int qh = 0; qh < 2; ++qh) {
        s2[qh] = f32x16{};
        dp2[qh] = DR ? f32x16{} : neg_delta_acc(ndl_l, qh, h);
#pragma unroll
        for (int kk = 0; kk < T::kKk; ++kk) {
          const u32x4 qa = lds16(q_lds + swz64(32 * qh + l32, 2 * kk + h));
          const u32x4 ga = lds16(g_lds + swz64(32 * qh + l32, 2 * kk + h));
          s2[qh] = Mfma<DT>::run(qa, kf[kk], s2[qh]);
          dp2[qh] = Mfma<DT>::run(ga, vf[kk], dp2[qh]);
        }
      }
      // s2[qh][j] = S[query][key], query = qt*64 + 32qh + 8(j/4) + 4h + j%4
      if constexpr (CM) {
        // log2 units; partial slices take -inf from the mask's bits (kind 2) or
        // add the mask's bias element by element (kind 3)
#pragma unroll
        for (int qh = 0; qh < 2; ++qh) s2[qh] *= scale_log2;
        if (kind == 2) {
#pragma unroll
          for (int qh = 0; qh < 2; ++qh)
            apply_bits(s2[qh], static_cast<uint32_t>((wb >> (4 * h)) >> (32 * qh)));
        } else if (!(FEAT & kFeatBool) && kind == 3) {
#pragma unroll
          for (int qh = 0; qh < 2; ++qh)
#pragma unroll
            for (int j = 0; j < 16; ++j) {
              const int qr = qt * 64 + 32 * qh + 8 * (j >> 2) + 4 * h + (j & 3);
              s2[qh][j] += mask_bias(ax, b, hd, qr, key, S) * kLog2e;
            }
        }
      } else if (kind == 2) {
#pragma unroll
        for (int qh = 0; qh < 2; ++qh) apply_bits(s2[qh], span_bits32(span, qt * 64 + 32 * qh + 4 * h));
      }
#pragma unroll
      for (int qh = 0; qh < 2; ++qh) {
        f32x16& s = s2[qh];
        f32x16& dp = dp2[qh];
        kv_half_update<DT, D, DR>(s, dp, CM ? 1.f : scale_log2, lse_l, ndl_l, qh, qt * 64, h, grp, lane, key,
                                  bh, ax, q_lds, g_lds, dkt, dvt,
                                  [&](const uint16_t* t, int r0, int r1, int c0) {
                                    return lds_read_tr4x2_swz64(t, r0, r1, c0, lane);
                                  });
      }
    }
    if constexpr (CM) wb = wb_next;
  }

  if (key >= S) return;
  store_row<DT, T::kDt>(dK + b * dksb + hd * dksh + static_cast<int64_t>(key) * dkss, dkt, scale, h);
  store_row<DT, T::kDt>(dV + b * dvsb + hd * dvsh + static_cast<int64_t>(key) * dvss, dvt, 1.f, h);
}

// dQ. Workgroup = (b, h, 128 queries) as in the forward; wave w owns queries
// 32w..32w+31, Q and dO rows in registers (B operands of Sᵀ = K·Qᵀ and
// dPᵀ = V·dOᵀ, lane = query). Per listed 64-key tile (the forward's work list),
// K and V are staged in LDS; the wave computes Sᵀ, dPᵀ, P and dSᵀ (lane = query,
// 16 keys per lane), then dQᵀ += Kᵀ·dSᵀ with Kᵀ read by transpose reads in the
// accumulator's permuted key order.
// FEAT as for the forward: with kFeatDrop, dS = P ⊙ (Z ⊙ dP − Δ).
// Three workgroups per CU at D ≤ 64 (≤ 168 VGPRs): the caller-mask variants
// would otherwise take 169–174 and drop to two; with mask and dropout the cap
// costs four spilled VGPRs and still runs faster.
// RING (D = 64, plain): K and V go HBM/L2 -> LDS with global_load_lds into two
// unpadded swz64 stages, one tile ahead, so no staging registers are needed and
// four workgroups fit per CU (≤ 128 VGPRs, 32 KB of LDS).
template <int DT, int D, int FEAT = 0, bool RING = false>
__global__ __launch_bounds__(256, RING ? 4 : (D > 64 ? 1 : 3)) void wattn_bwd_q_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
    const uint16_t* __restrict__ dO, const uint16_t* __restrict__ O, int64_t osb, int64_t osh,
    int64_t oss, const float* __restrict__ lse, float* __restrict__ delta,
    uint16_t* __restrict__ dQ, int64_t qsb, int64_t qsh, int64_t qss, int64_t ksb, int64_t ksh,
    int64_t kss, int64_t vsb, int64_t vsh, int64_t vss, int64_t gsb, int64_t gsh, int64_t gss,
    int64_t dqsb, int64_t dqsh, int64_t dqss, int H, MaskParams mp, float scale,
    float scale_log2, const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ entries,
    const int32_t* __restrict__ order, WorkMap wm, AttnX ax) {
  constexpr bool CM = (FEAT & kFeatMask) != 0, DR = (FEAT & kFeatDrop) != 0;
  using T = Tile<D>;
  static_assert(!RING || D == 64, "the copy ring stages 64-wide tiles");
  // [buffer][K, V] 64 x D tiles: padded rows, or with RING unpadded swz64 tiles
  constexpr int kTileE = RING ? 64 * 64 : T::kElems;
  __shared__ __attribute__((aligned(16))) uint16_t smem[4 * kTileE];

  int bh, qb;
  if (!work_item(wm, order, bh, qb)) return;
  const int b = bh / H, hd = bh - b * H;
  const int S = mp.S;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;  // uniform
  const int l32 = lane & 31, h = lane >> 5;
  const int grp = (lane >> 4) & 1;
  const int q_row = qb * 128 + wave * 32 + l32;
  const Span span = mask_row_span(mp, q_row);

  u32x4 qf[T::kKk], gf[T::kKk];
  {
    const int qc = min(q_row, S - 1);
    const uint16_t* qp = Q + b * qsb + hd * qsh + static_cast<int64_t>(qc) * qss + 8 * h;
    const uint16_t* gp = dO + b * gsb + hd * gsh + static_cast<int64_t>(qc) * gss + 8 * h;
#pragma unroll
    for (int kk = 0; kk < T::kKk; ++kk) {
      qf[kk] = ldg16(qp + 16 * kk);
      gf[kk] = ldg16(gp + 16 * kk);
    }
#pragma unroll
    for (int kk = 0; kk < T::kKk; ++kk) {
      settle(qf[kk]);
      settle(gf[kk]);
    }
  }
  const float l2 = lse_log2<CM>(lse[static_cast<int64_t>(bh) * S + min(q_row, S - 1)]);
  // Δ = rowsum(dO ⊙ O) of this row in fp32: this lane's half of the head dims
  // (the dO chunks it holds), then lane ^ 32's half. Written for the dK/dV
  // kernel, which runs after this one.
  float dl;
  {
    const uint16_t* op = O + b * osb + hd * osh + static_cast<int64_t>(min(q_row, S - 1)) * oss + 8 * h;
    float acc = 0.f;
#pragma unroll
    for (int kk = 0; kk < T::kKk; ++kk) {
      const u32x4 o = ldg16(op + 16 * kk);
      const uint32_t ow[4] = {o.x, o.y, o.z, o.w};
      const uint32_t gw[4] = {gf[kk].x, gf[kk].y, gf[kk].z, gf[kk].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc = fmaf(Mfma<DT>::to_f32(static_cast<uint16_t>(ow[i] & 0xffff)),
                   Mfma<DT>::to_f32(static_cast<uint16_t>(gw[i] & 0xffff)), acc);
        acc = fmaf(Mfma<DT>::to_f32(static_cast<uint16_t>(ow[i] >> 16)),
                   Mfma<DT>::to_f32(static_cast<uint16_t>(gw[i] >> 16)), acc);
      }
    }
    dl = xor32_add(acc);
    if (h == 0 && q_row < S) delta[static_cast<int64_t>(bh) * S + q_row] = dl;
  }
  const uint16_t* Kbh = K + b * ksb + hd * ksh;
  const uint16_t* Vbh = V + b * vsb + hd * vsh;
  int e0, e1, mrow = 0;
  if constexpr (CM) {
    mrow = mask_row(ax, b, hd);
    const int row = mrow * ((S + 127) >> 7) + qb;
    e0 = row * ax.cap;
    e1 = e0 + ax.cnt[row];
  } else {
    e0 = row_ptr[qb];
    e1 = row_ptr[qb + 1];
  }
  const float sc = CM ? 1.f : scale_log2;

  u32x4 pre[RING ? 1 : 2 * T::kPasses];
  const int r0 = tid / T::kCpr, c8 = (tid % T::kCpr) * 8;
  int64_t koff[T::kPasses], voff[T::kPasses];
  if constexpr (!RING) {
#pragma unroll
    for (int p = 0; p < T::kPasses; ++p) {
      koff[p] = static_cast<int64_t>(r0 + p * T::kRpp) * kss + c8;
      voff[p] = static_cast<int64_t>(r0 + p * T::kRpp) * vss + c8;
    }
  }
  // RING: this wave's 16 rows of the K and V tiles go HBM/L2 -> LDS with
  // global_load_lds (two 8-row instructions each, chunk positions as for swz64),
  // rows past S reading row S - 1; four copies per wave and tile.
  const int drow = lane >> 3, dpos = lane & 7;
  int crow[2];
  uint32_t cchunk[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    crow[j] = 16 * wave + 8 * j + drow;
    const int a = (crow[j] >> 1) & 7;
    cchunk[j] = 16u * static_cast<uint32_t>(dpos ^ (((a & 1) << 2) | (a >> 1)));
  }
  const uint32_t smem0 = lds_offset(smem);
  auto issue = [&](int kt, int bf) __attribute__((always_inline)) {
    const int lim = S - 1 - kt * 64;
    const uint16_t* kb = Kbh + static_cast<int64_t>(kt) * 64 * kss;
    const uint16_t* vb = Vbh + static_cast<int64_t>(kt) * 64 * vss;
    const uint32_t st = smem0 + static_cast<uint32_t>(2 * bf * kTileE * 2);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t r = static_cast<uint32_t>(min(crow[j], lim));
      dma_lds16(kb, r * static_cast<uint32_t>(2 * kss) + cchunk[j], st + (16 * wave + 8 * j) * 128);
      dma_lds16(vb, r * static_cast<uint32_t>(2 * vss) + cchunk[j],
                st + kTileE * 2 + (16 * wave + 8 * j) * 128);
    }
  };
  auto gload = [&](int kt) __attribute__((always_inline)) {
    if (kt * 64 + 64 <= S) {
      const uint16_t* kb = Kbh + static_cast<int64_t>(kt) * 64 * kss;
      const uint16_t* vb = Vbh + static_cast<int64_t>(kt) * 64 * vss;
#pragma unroll
      for (int p = 0; p < T::kPasses; ++p) {
        pre[p] = ldg16(kb + koff[p]);
        pre[T::kPasses + p] = ldg16(vb + voff[p]);
      }
    } else {
#pragma unroll
      for (int p = 0; p < T::kPasses; ++p) {
        const int kr = min(kt * 64 + r0 + p * T::kRpp, S - 1);  // rows past S: always masked
        pre[p] = ldg16(Kbh + kr * kss + c8);
        pre[T::kPasses + p] = ldg16(Vbh + kr * vss + c8);
      }
    }
  };
  auto sstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int p = 0; p < T::kPasses; ++p) {
      const int off = (r0 + p * T::kRpp) * T::kP + c8;
      sts16(smem + (2 * buf) * kTileE + off, pre[p]);
      sts16(smem + (2 * buf + 1) * kTileE + off, pre[T::kPasses + p]);
    }
  };

  f32x16 dqt[T::kDt];
#pragma unroll
  for (int dt = 0; dt < T::kDt; ++dt) dqt[dt] = f32x16{};

  uint64_t wb = 0, wb_next = 0;  // caller's mask: allowed-key bits of this row, two tiles
  if constexpr (RING) {
    if (e0 < e1) issue(entries[e0] & 0xffff, 0);
  } else {
    if (e0 < e1) {
      gload(entries[e0] & 0xffff);
      if constexpr (CM) wb = mask_word(ax, mrow, q_row, entries[e0] & 0xffff, S);
      sstore(0);
    }
    __syncthreads();
  }
  // K (or V) row r, 16-byte chunk c of a staged tile
  auto tile_off = [&](int r, int c) __attribute__((always_inline)) {
    if constexpr (RING) return swz64(r, c);
    else return r * T::kP + 8 * c;
  };
  int buf = 0;
  for (int e = e0; e < e1; ++e) {
    const int ent = entries[e];
    const int kt = ent & 0xffff;
    const int kind = (ent >> (16 + 2 * wave)) & 3;
    const bool more = e + 1 < e1;
    if constexpr (RING) {
      // this wave's copies of tile e have landed; after the barrier every wave's
      // have, and every wave is done with tile e - 1, whose buffer the next copies fill
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      asm volatile("s_barrier" ::: "memory");
      if (more) issue(entries[e + 1] & 0xffff, buf ^ 1);
    } else if (more) {
      gload(entries[e + 1] & 0xffff);
      if constexpr (CM) wb_next = mask_word(ax, mrow, q_row, entries[e + 1] & 0xffff, S);
    }

    if (kind != 0) {
      const uint16_t* k_lds = smem + (2 * buf) * kTileE;
      const uint16_t* v_lds = smem + (2 * buf + 1) * kTileE;
      // One 32-key half at a time (s, dp: 32 VGPRs instead of 64).
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
        f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
        for (int kk = 0; kk < T::kKk; ++kk) {
          const u32x4 ka = lds16(k_lds + tile_off(32 * kh + l32, 2 * kk + h));
          const u32x4 va = lds16(v_lds + tile_off(32 * kh + l32, 2 * kk + h));
          s = Mfma<DT>::run(ka, qf[kk], s);
          dp = Mfma<DT>::run(va, gf[kk], dp);
        }
        // s[j] = S[q_row][key], key = kt*64 + 32kh + 8(j/4) + 4h + j%4; the span
        // bounds move to this lane's origin (kt*64 + 4h).
        if constexpr (CM) {
          s *= scale_log2;
          if (kind == 2) {
            apply_bits(s, static_cast<uint32_t>((wb >> (4 * h)) >> (32 * kh)));
          } else if (!(FEAT & kFeatBool) && kind == 3) {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
              const int key = kt * 64 + 32 * kh + 8 * (j >> 2) + 4 * h + (j & 3);
              s[j] += mask_bias(ax, b, hd, q_row, key, S) * kLog2e;
            }
          }
        } else if (kind == 2) {
          apply_bits(s, span_bits32(span, kt * 64 + 32 * kh + 4 * h));
        }
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          // elements 8m + t and 8m + 4 + t: keys 16m + 4h + t and 16m + 8 + 4h + t of the half
          float z[8] = {1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f};
          if constexpr (DR) drop_row8(ax, bh, q_row, kt * 64 + 32 * kh + 16 * m, h, z);
#pragma unroll
          for (int t = 0; t < 8; ++t) {
            const int j = 8 * m + t;
            const float pj = __builtin_amdgcn_exp2f(fmaf(s[j], sc, -l2));
            dp[j] = DR ? pj * (z[t] * dp[j] - dl) : pj * (dp[j] - dl);
          }
        }
        if constexpr ((FEAT & kFeatDBias) != 0) {
          {
            float ds[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) ds[j] = dp[j];
            store_dbias(ax.dbias, bh, S, q_row, kt * 64 + 32 * kh + 4 * h, ds);
          }
        }
        // dQᵀ[d][q] += Σ_key K[key][d] dS[q][key], 16 keys per MFMA.
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
          const int ks = 2 * kh + k2;
          const u32x4 db = pack8<DT>(dp, 8 * k2);
#pragma unroll
          for (int dt = 0; dt < T::kDt; ++dt) {
            u32x4 ka;
            if constexpr (RING)
              ka = lds_read_tr4x2_swz64(k_lds, 16 * ks + 4 * h, 16 * ks + 8 + 4 * h, 32 * dt + 16 * grp,
                                        lane);
            else
              ka = lds_read_tr4x2<T::kP>(k_lds, 16 * ks + 4 * h, 16 * ks + 8 + 4 * h,
                                         32 * dt + 16 * grp, lane);
            dqt[dt] = Mfma<DT>::run(ka, db, dqt[dt]);
          }
        }
      }
    }
    if constexpr (!RING) {
      if (more) sstore(buf ^ 1);
      if constexpr (CM) wb = wb_next;
      __syncthreads();
    }
    buf ^= 1;
  }

  if (q_row >= S) return;
  store_row<DT, T::kDt>(dQ + b * dqsb + hd * dqsh + static_cast<int64_t>(q_row) * dqss, dqt, scale, h);
}

// fp32 backward. Δ[b, h, q] = Σ_d dO · O, D/8 lanes per row (eight elements
// each), for every head dimension.
template <int D>
__global__ __launch_bounds__(256) void wattn_bwd_delta_f32_kernel(
    const float* __restrict__ O, const float* __restrict__ dO, float* __restrict__ delta,
    int64_t osb, int64_t osh, int64_t oss, int64_t gsb, int64_t gsh, int64_t gss, int H, int S,
    int64_t n_rows) {
  constexpr int kLpr = D / 8;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (256 / kLpr) + threadIdx.x / kLpr;
  const int ch = threadIdx.x % kLpr;
  float acc = 0.f;
  if (row < n_rows) {
    const int64_t bh = row / S;
    const int q = static_cast<int>(row - bh * S);
    const int b = static_cast<int>(bh / H), hd = static_cast<int>(bh - static_cast<int64_t>(b) * H);
    const float* op = O + b * osb + hd * osh + static_cast<int64_t>(q) * oss + 8 * ch;
    const float* gp = dO + b * gsb + hd * gsh + static_cast<int64_t>(q) * gss + 8 * ch;
#pragma unroll
    for (int i = 0; i < 8; i += 4) {
      const f32x4 o = *reinterpret_cast<const f32x4*>(op + i);
      const f32x4 g = *reinterpret_cast<const f32x4*>(gp + i);
      acc = fmaf(o.x, g.x, fmaf(o.y, g.y, fmaf(o.z, g.z, fmaf(o.w, g.w, acc))));
    }
  }
#pragma unroll
  for (int o = 1; o < kLpr; o <<= 1) acc += __shfl_xor(acc, o);
  if (row < n_rows && ch == 0) delta[row] = acc;
}

// fp32 backward on the matrix cores (head dimension 32, 64 or 128; Δ from
// wattn_bwd_delta_f32_kernel; FEAT as for the 16-bit kernels). The layouts of
// wattn_fwd_f32m_kernel: a v_mfma_f32_32x32x2_f32 k-step sums two head
// dimensions, one per lane half, for the score-like products (each lane holds
// the D/2 dimensions of its row that its half needs, the other operand comes
// from LDS in 16-byte row chunks), and two keys or queries, one per lane half,
// for the gradient products (the probability or dS the accumulator left in the
// lane is the B operand in place; the staged tile gives a 4-byte read per lane).
//
// dQ: the forward's work list; wave w owns queries 32w..32w+31 of the
// 128-query block, Q·scale·log2e and dO rows in registers. Per listed key tile
// and 32-key half: Sᵀ = K·Qᵀ and dPᵀ = V·dOᵀ, P = exp2(Sᵀ − LSE·log2e),
// dSᵀ = P ⊙ (dPᵀ − Δ) (with dropout P ⊙ (Z ⊙ dPᵀ − Δ)), dQᵀ += Kᵀ·dSᵀ.
template <int D, int FEAT = 0>
__global__ __launch_bounds__(256, D > 64 ? 1 : 2) void wattn_bwd_q_f32m_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ dO, const float* __restrict__ lse, const float* __restrict__ delta,
    float* __restrict__ dQ, int64_t qsb, int64_t qsh, int64_t qss, int64_t ksb, int64_t ksh,
    int64_t kss, int64_t vsb, int64_t vsh, int64_t vss, int64_t gsb, int64_t gsh, int64_t gss,
    int64_t dqsb, int64_t dqsh, int64_t dqss, int H, MaskParams mp, float scale,
    float scale_log2, const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ entries,
    const int32_t* __restrict__ order, WorkMap wm, AttnX ax) {
  static_assert(D == 32 || D == 64 || D == 128, "head dimension 32, 64 or 128");
  constexpr bool CM = (FEAT & kFeatMask) != 0, DR = (FEAT & kFeatDrop) != 0;
  constexpr int kP = D + 4, kTile = 64 * kP, kHalf = D / 2, kDt = D / 32;
  constexpr int kC4 = D / 4, kRpp = 256 / kC4, kPasses = 64 / kRpp;
  __shared__ __attribute__((aligned(16))) float smem[4 * kTile];  // [buffer][K, V]

  int bh, qb;
  if (!work_item(wm, order, bh, qb)) return;
  const int b = bh / H, hd = bh - b * H;
  const int S = mp.S;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int l32 = lane & 31, h = lane >> 5;
  const int q_row = qb * 128 + wave * 32 + l32;
  const int qc = min(q_row, S - 1);
  const Span span = mask_row_span(mp, q_row);

  float qf[kHalf], gf[kHalf];
  {
    const float* qp = Q + b * qsb + hd * qsh + static_cast<int64_t>(qc) * qss + h * kHalf;
    const float* gp = dO + b * gsb + hd * gsh + static_cast<int64_t>(qc) * gss + h * kHalf;
#pragma unroll
    for (int c = 0; c < kHalf; c += 4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(qp + c);
      const f32x4 w = *reinterpret_cast<const f32x4*>(gp + c);
      qf[c] = v.x * scale_log2;
      qf[c + 1] = v.y * scale_log2;
      qf[c + 2] = v.z * scale_log2;
      qf[c + 3] = v.w * scale_log2;
      gf[c] = w.x;
      gf[c + 1] = w.y;
      gf[c + 2] = w.z;
      gf[c + 3] = w.w;
    }
  }
  const float l2 = lse_log2<CM>(lse[static_cast<int64_t>(bh) * S + qc]);
  const float dl = delta[static_cast<int64_t>(bh) * S + qc];
  const float* Kbh = K + b * ksb + hd * ksh;
  const float* Vbh = V + b * vsb + hd * vsh;
  int e0, e1, mrow = 0;
  if constexpr (CM) {
    mrow = mask_row(ax, b, hd);
    const int row = mrow * ((S + 127) >> 7) + qb;
    e0 = row * ax.cap;
    e1 = e0 + ax.cnt[row];
  } else {
    e0 = row_ptr[qb];
    e1 = row_ptr[qb + 1];
  }
  uint64_t wb = 0, wb_next = 0;  // caller's mask: this row's allowed-key bits, two tiles

  f32x4 pre[2 * kPasses];
  const int r0 = tid / kC4, c4 = (tid % kC4) * 4;
  auto gload = [&](int kt) __attribute__((always_inline)) {
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int key = min(kt * 64 + r0 + p * kRpp, S - 1);  // rows past S: always masked
      pre[p] = *reinterpret_cast<const f32x4*>(Kbh + key * kss + c4);
      pre[kPasses + p] = *reinterpret_cast<const f32x4*>(Vbh + key * vss + c4);
    }
  };
  auto sstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int off = (r0 + p * kRpp) * kP + c4;
      *reinterpret_cast<f32x4*>(smem + (2 * buf) * kTile + off) = pre[p];
      *reinterpret_cast<f32x4*>(smem + (2 * buf + 1) * kTile + off) = pre[kPasses + p];
    }
  };

  f32x16 dqt[kDt];
#pragma unroll
  for (int dt = 0; dt < kDt; ++dt) dqt[dt] = f32x16{};
  if (e0 < e1) {
    gload(entries[e0] & 0xffff);
    if constexpr (CM) wb = mask_word(ax, mrow, q_row, entries[e0] & 0xffff, S);
    sstore(0);
  }
  __syncthreads();
  int buf = 0;
  for (int e = e0; e < e1; ++e) {
    const int ent = entries[e];
    const int kt = ent & 0xffff;
    const int kind = (ent >> (16 + 2 * wave)) & 3;
    const bool more = e + 1 < e1;
    if (more) {
      gload(entries[e + 1] & 0xffff);
      if constexpr (CM) wb_next = mask_word(ax, mrow, q_row, entries[e + 1] & 0xffff, S);
    }
    if (kind != 0) {
      const float* kt_lds = smem + (2 * buf) * kTile;
      const float* vt_lds = smem + (2 * buf + 1) * kTile;
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
        f32x16 st = f32x16{}, dpt = f32x16{};
#pragma unroll
        for (int c = 0; c < kHalf; c += 4) {
          const f32x4 ka = *reinterpret_cast<const f32x4*>(kt_lds + (32 * kh + l32) * kP + h * kHalf + c);
          const f32x4 va = *reinterpret_cast<const f32x4*>(vt_lds + (32 * kh + l32) * kP + h * kHalf + c);
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            st = __builtin_amdgcn_mfma_f32_32x32x2f32(ka[t], qf[c + t], st, 0, 0, 0);
            dpt = __builtin_amdgcn_mfma_f32_32x32x2f32(va[t], gf[c + t], dpt, 0, 0, 0);
          }
        }
        // st[j]: key kt*64 + 32kh + 8(j/4) + 4h + j%4 of this lane's query
        if constexpr (CM) {
          if (kind == 2) {
            apply_bits(st, static_cast<uint32_t>((wb >> (4 * h)) >> (32 * kh)));
          } else if (!(FEAT & kFeatBool) && kind == 3) {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
              const int key = kt * 64 + 32 * kh + 8 * (j >> 2) + 4 * h + (j & 3);
              st[j] += mask_bias(ax, b, hd, q_row, key, S) * kLog2e;
            }
          }
        } else if (kind == 2) {
          apply_bits(st, span_bits32(span, kt * 64 + 32 * kh + 4 * h));
        }
        if constexpr (DR) {
#pragma unroll
          for (int m = 0; m < 2; ++m) {
            float z8[8];
            drop_row8(ax, bh, q_row, kt * 64 + 32 * kh + 16 * m, h, z8);
#pragma unroll
            for (int t = 0; t < 8; ++t)
              st[8 * m + t] = __builtin_amdgcn_exp2f(st[8 * m + t] - l2) * (z8[t] * dpt[8 * m + t] - dl);
          }
        } else {
#pragma unroll
          for (int j = 0; j < 16; ++j)
            st[j] = __builtin_amdgcn_exp2f(st[j] - l2) * (dpt[j] - dl);
        }
        if constexpr ((FEAT & kFeatDBias) != 0) {
          {
            float ds[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) ds[j] = st[j];
            store_dbias(ax.dbias, bh, S, q_row, kt * 64 + 32 * kh + 4 * h, ds);
          }
        }
#pragma unroll
        for (int s = 0; s < 16; ++s) {
          const int key = 32 * kh + 8 * (s >> 2) + 4 * h + (s & 3);
#pragma unroll
          for (int dt = 0; dt < kDt; ++dt)
            dqt[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(kt_lds[key * kP + 32 * dt + l32], st[s],
                                                           dqt[dt], 0, 0, 0);
        }
      }
    }
    if (more) sstore(buf ^ 1);
    if constexpr (CM) wb = wb_next;
    __syncthreads();
    buf ^= 1;
  }
  if (q_row >= S) return;
  float* op = dQ + b * dqsb + hd * dqsh + static_cast<int64_t>(q_row) * dqss;
#pragma unroll
  for (int dt = 0; dt < kDt; ++dt)
#pragma unroll
    for (int jg = 0; jg < 4; ++jg)
      *reinterpret_cast<f32x4*>(op + 32 * dt + 8 * jg + 4 * h) =
          f32x4{dqt[dt][4 * jg] * scale, dqt[dt][4 * jg + 1] * scale, dqt[dt][4 * jg + 2] * scale,
                dqt[dt][4 * jg + 3] * scale};
}

// dK, dV: the key-major work list; wave w owns keys 32w..32w+31 of the 128-key
// block, K·scale·log2e and V rows in registers. Per listed query tile, Q, dO,
// LSE·log2e and Δ of its 64 queries are staged in LDS; per 32-query half:
// S = Q·Kᵀ and dP = dO·Vᵀ (lane = key, element j = query 32qh + 8(j/4) + 4h +
// j%4), P = exp2(S − LSE·log2e), dS = P ⊙ (dP − Δ), dVᵀ += dOᵀ·P and
// dKᵀ += Qᵀ·dS; with dropout dV takes P ⊙ Z and dS = P ⊙ (Z ⊙ dP − Δ).
template <int D, int FEAT = 0>
__global__ __launch_bounds__(256, D > 64 ? 1 : 2) void wattn_bwd_kv_f32m_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ dO, const float* __restrict__ lse, const float* __restrict__ delta,
    float* __restrict__ dK, float* __restrict__ dV, int64_t qsb, int64_t qsh, int64_t qss,
    int64_t ksb, int64_t ksh, int64_t kss, int64_t vsb, int64_t vsh, int64_t vss, int64_t gsb,
    int64_t gsh, int64_t gss, int64_t dksb, int64_t dksh, int64_t dkss, int64_t dvsb,
    int64_t dvsh, int64_t dvss, int H, MaskParams mp, float scale, float scale_log2,
    const int32_t* __restrict__ col_ptr, const int32_t* __restrict__ entries,
    const int32_t* __restrict__ order, WorkMap wm, AttnX ax) {
  static_assert(D == 32 || D == 64 || D == 128, "head dimension 32, 64 or 128");
  constexpr bool CM = (FEAT & kFeatMask) != 0, DR = (FEAT & kFeatDrop) != 0;
  constexpr int kP = D + 4, kTile = 64 * kP, kHalf = D / 2, kDt = D / 32;
  constexpr int kC4 = D / 4, kRpp = 256 / kC4, kPasses = 64 / kRpp;
  // [buffer][Q, dO] tiles, then [buffer][LSE·log2e, Δ] of the 64 queries
  __shared__ __attribute__((aligned(16))) float smem[4 * kTile];
  __shared__ __attribute__((aligned(16))) float stat[2][2][64];

  int bh, kb;
  if (!work_item(wm, order, bh, kb)) return;
  const int b = bh / H, hd = bh - b * H;
  const int S = mp.S;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int l32 = lane & 31, h = lane >> 5;
  const int key = kb * 128 + wave * 32 + l32;
  const int kc = min(key, S - 1);
  const Span span = mask_col_span(mp, key);

  float kf[kHalf], vf[kHalf];
  {
    const float* kp = K + b * ksb + hd * ksh + static_cast<int64_t>(kc) * kss + h * kHalf;
    const float* vp = V + b * vsb + hd * vsh + static_cast<int64_t>(kc) * vss + h * kHalf;
#pragma unroll
    for (int c = 0; c < kHalf; c += 4) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(kp + c);
      const f32x4 w = *reinterpret_cast<const f32x4*>(vp + c);
      kf[c] = a.x * scale_log2;
      kf[c + 1] = a.y * scale_log2;
      kf[c + 2] = a.z * scale_log2;
      kf[c + 3] = a.w * scale_log2;
      vf[c] = w.x;
      vf[c + 1] = w.y;
      vf[c + 2] = w.z;
      vf[c + 3] = w.w;
    }
  }
  const float* Qbh = Q + b * qsb + hd * qsh;
  const float* Gbh = dO + b * gsb + hd * gsh;
  const float* lse_bh = lse + static_cast<int64_t>(bh) * S;
  const float* dl_bh = delta + static_cast<int64_t>(bh) * S;
  int e0, e1, mrow = 0;
  if constexpr (CM) {
    mrow = mask_row(ax, b, hd);
    const int row = mrow * ((S + 127) >> 7) + kb;
    e0 = row * ax.cap;
    e1 = e0 + ax.cnt[row];
  } else {
    e0 = col_ptr[kb];
    e1 = col_ptr[kb + 1];
  }
  uint64_t wb = 0, wb_next = 0;  // caller's mask: allowed-query bits of this key, two tiles

  f32x4 pre[2 * kPasses];
  float st_pre = 0.f;
  const int r0 = tid / kC4, c4 = (tid % kC4) * 4;
  auto gload = [&](int qt) __attribute__((always_inline)) {
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int qr = min(qt * 64 + r0 + p * kRpp, S - 1);  // rows past S: always masked
      pre[p] = *reinterpret_cast<const f32x4*>(Qbh + qr * qss + c4);
      pre[kPasses + p] = *reinterpret_cast<const f32x4*>(Gbh + qr * gss + c4);
    }
    // LSE (threads 0-63) and Δ (64-127) of the tile's queries
    st_pre = ((tid & 64) ? dl_bh : lse_bh)[min(qt * 64 + (tid & 63), S - 1)];
  };
  auto sstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int off = (r0 + p * kRpp) * kP + c4;
      *reinterpret_cast<f32x4*>(smem + (2 * buf) * kTile + off) = pre[p];
      *reinterpret_cast<f32x4*>(smem + (2 * buf + 1) * kTile + off) = pre[kPasses + p];
    }
    if (tid < 128) stat[buf][tid >> 6][tid & 63] = tid < 64 ? lse_log2<CM>(st_pre) : st_pre;
  };

  f32x16 dkt[kDt], dvt[kDt];
#pragma unroll
  for (int dt = 0; dt < kDt; ++dt) {
    dkt[dt] = f32x16{};
    dvt[dt] = f32x16{};
  }
  if (e0 < e1) {
    gload(entries[e0] & 0xffff);
    if constexpr (CM) wb = mask_word(ax, mrow, key, entries[e0] & 0xffff, S);
    sstore(0);
  }
  __syncthreads();
  int buf = 0;
  for (int e = e0; e < e1; ++e) {
    const int ent = entries[e];
    const int qt = ent & 0xffff;
    const int kind = (ent >> (16 + 2 * wave)) & 3;
    const bool more = e + 1 < e1;
    if (more) {
      gload(entries[e + 1] & 0xffff);
      if constexpr (CM) wb_next = mask_word(ax, mrow, key, entries[e + 1] & 0xffff, S);
    }
    if (kind != 0) {
      const float* q_lds = smem + (2 * buf) * kTile;
      const float* g_lds = smem + (2 * buf + 1) * kTile;
      const float* l2_l = &stat[buf][0][0];
      const float* dl_l = &stat[buf][1][0];
#pragma unroll
      for (int qh = 0; qh < 2; ++qh) {
        f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
        for (int c = 0; c < kHalf; c += 4) {
          const f32x4 qa = *reinterpret_cast<const f32x4*>(q_lds + (32 * qh + l32) * kP + h * kHalf + c);
          const f32x4 ga = *reinterpret_cast<const f32x4*>(g_lds + (32 * qh + l32) * kP + h * kHalf + c);
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            s = __builtin_amdgcn_mfma_f32_32x32x2f32(qa[t], kf[c + t], s, 0, 0, 0);
            dp = __builtin_amdgcn_mfma_f32_32x32x2f32(ga[t], vf[c + t], dp, 0, 0, 0);
          }
        }
        // s[j]: query qt*64 + 32qh + 8(j/4) + 4h + j%4 of this lane's key
        if constexpr (CM) {
          if (kind == 2) {
            apply_bits(s, static_cast<uint32_t>((wb >> (4 * h)) >> (32 * qh)));
          } else if (!(FEAT & kFeatBool) && kind == 3) {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
              const int qr = qt * 64 + 32 * qh + 8 * (j >> 2) + 4 * h + (j & 3);
              s[j] += mask_bias(ax, b, hd, qr, key, S) * kLog2e;
            }
          }
        } else if (kind == 2) {
          apply_bits(s, span_bits32(span, qt * 64 + 32 * qh + 4 * h));
        }
        uint32_t kq2[2] = {0u, 0u};  // keep bits of query groups (0, 1) and (2, 3)
        if constexpr (DR) {
#pragma unroll
          for (int g2 = 0; g2 < 2; ++g2) {
            const int qa = qt * 64 + 32 * qh + 16 * g2 + 4 * h;
            kq2[g2] = keep_octet2(ax, bh, qa, qa + 8, key, lane & 7);
          }
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 l4 = *reinterpret_cast<const f32x4*>(l2_l + 32 * qh + 8 * g + 4 * h);
          const f32x4 d4 = *reinterpret_cast<const f32x4*>(dl_l + 32 * qh + 8 * g + 4 * h);
          uint32_t kq = 0;
          if constexpr (DR) kq = kq2[g >> 1] >> (16 * (g & 1));
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const float pj = __builtin_amdgcn_exp2f(s[4 * g + t] - l4[t]);
            if constexpr (DR) {
              const float z = ((kq >> (4 * t)) & 1u) ? ax.keep_scale : 0.f;
              s[4 * g + t] = pj * z;
              dp[4 * g + t] = pj * (z * dp[4 * g + t] - d4[t]);
            } else {
              s[4 * g + t] = pj;
              dp[4 * g + t] = pj * (dp[4 * g + t] - d4[t]);
            }
          }
        }
#pragma unroll
        for (int k2 = 0; k2 < 16; ++k2) {
          const int qr = 32 * qh + 8 * (k2 >> 2) + 4 * h + (k2 & 3);
#pragma unroll
          for (int dt = 0; dt < kDt; ++dt) {
            dvt[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(g_lds[qr * kP + 32 * dt + l32], s[k2],
                                                           dvt[dt], 0, 0, 0);
            dkt[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(q_lds[qr * kP + 32 * dt + l32], dp[k2],
                                                           dkt[dt], 0, 0, 0);
          }
        }
      }
    }
    if (more) sstore(buf ^ 1);
    if constexpr (CM) wb = wb_next;
    __syncthreads();
    buf ^= 1;
  }
  if (key >= S) return;
  float* dkp = dK + b * dksb + hd * dksh + static_cast<int64_t>(key) * dkss;
  float* dvp = dV + b * dvsb + hd * dvsh + static_cast<int64_t>(key) * dvss;
  // dkt[dt][j] = dKᵀ[32dt + 8(j/4) + 4h + j%4][key]: four consecutive dimensions per j/4
#pragma unroll
  for (int dt = 0; dt < kDt; ++dt)
#pragma unroll
    for (int jg = 0; jg < 4; ++jg) {
      const int d0 = 32 * dt + 8 * jg + 4 * h;
      *reinterpret_cast<f32x4*>(dkp + d0) =
          f32x4{dkt[dt][4 * jg] * scale, dkt[dt][4 * jg + 1] * scale, dkt[dt][4 * jg + 2] * scale,
                dkt[dt][4 * jg + 3] * scale};
      *reinterpret_cast<f32x4*>(dvp + d0) =
          f32x4{dvt[dt][4 * jg], dvt[dt][4 * jg + 1], dvt[dt][4 * jg + 2], dvt[dt][4 * jg + 3]};
    }
}

// Work lists of a caller's mask (kFeatMask), built on the device in three launches.
//
// 1. wattn_mask_kinds_kernel: one workgroup per (mask row mr, 128x128 square
//    (query block i, key block j)); wave w reads the square's 32 query rows
//    32w..32w+31, lane l the keys l and 64 + l of each, so every mask byte (or
//    float) is read once, 64 consecutive keys per wave load. It writes
//    - the allowed-pair bitmaps: bits_q word (mr, query q, key tile t) has bit
//      i for key 64t + i (one ballot per row and tile), bits_kv word (mr, key k,
//      query tile u) bit i for query 64u + i (each lane gathers 32 rows of its
//      key, and two waves fill the two halves of a word);
//    - for each 32x32 sub-block three flags: some pair allowed, every pair
//      allowed with bias 0, some allowed pair with a nonzero bias; from them
//      kinds_q[(mr * n_b + i) * n_t + t] for the key tiles t = 2j, 2j + 1 and
//      kinds_kv[(mr * n_b + j) * n_t + u] for the query tiles u = 2i, 2i + 1,
//      2 bits per 32-wide slice of the block (query slices for the query-major
//      lists, key slices for the key-major ones): 0 nothing allowed, 1 all
//      allowed with bias 0, 2 some allowed and all of those with bias 0 (the
//      kernels mask from the bitmap), 3 some nonzero bias (the kernels read it).
//    Positions at or past S count as masked.
// 2. wattn_mask_compact_kernel: one wave per list row (query-major rows, then
//    key-major rows): entries[row * n_t + c] = t | kinds << 16 for the tiles t
//    with a nonzero kind, t ascending, and cnt[row] = their number.
__global__ __launch_bounds__(256) void wattn_mask_kinds_kernel(AttnX ax, int S, int n_b, int n_t,
                                                               uint8_t* __restrict__ kinds_q,
                                                               uint8_t* __restrict__ kinds_kv,
                                                               uint64_t* __restrict__ bits_q,
                                                               uint32_t* __restrict__ bits_kv) {
  __shared__ uint32_t flags[4];  // per wave: (any, all, nonzero) bits of its four sub-blocks
  const int j = blockIdx.x, i = blockIdx.y, mr = blockIdx.z;
  const int bm = mr / ax.MH, hm = mr - bm * ax.MH;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int64_t rows = static_cast<int64_t>(n_b) * 128;  // bitmap rows per mask row
  bool any0 = false, all0 = true, nz0 = false, any1 = false, all1 = true, nz1 = false;
  uint32_t col0 = 0, col1 = 0;    // this lane's keys: allowed bits of the 32 rows
  uint64_t row0 = 0, row1 = 0;    // lane r < 32: allowed bits of row r, key tiles 2j, 2j + 1
  const int k0 = j * 128 + lane, k1 = k0 + 64;
#pragma unroll 8
  for (int r = 0; r < 32; ++r) {
    const int q = i * 128 + 32 * wave + r;
    const float v0 = mask_bias(ax, bm, hm, q, k0, S);
    const float v1 = mask_bias(ax, bm, hm, q, k1, S);
    const bool a0 = !(v0 == -INFINITY), a1 = !(v1 == -INFINITY);
    any0 |= a0;
    all0 &= (v0 == 0.f);
    nz0 |= a0 & (v0 != 0.f);
    any1 |= a1;
    all1 &= (v1 == 0.f);
    nz1 |= a1 & (v1 != 0.f);
    col0 |= static_cast<uint32_t>(a0) << r;
    col1 |= static_cast<uint32_t>(a1) << r;
    const uint64_t w0 = __ballot(a0), w1 = __ballot(a1);
    if (lane == r) {
      row0 = w0;
      row1 = w1;
    }
  }
  // bitmaps
  const int t0 = 2 * j, u = 2 * i + (wave >> 1);
  if (lane < 32) {
    uint64_t* dst = bits_q + (mr * rows + i * 128 + 32 * wave + lane) * n_t + t0;
    dst[0] = row0;
    if (t0 + 1 < n_t) dst[1] = row1;
  }
  if (u < n_t) {
    // the 32-bit half (wave & 1) of word (mr, key, u)
    bits_kv[2 * ((mr * rows + k0) * n_t + u) + (wave & 1)] = col0;
    bits_kv[2 * ((mr * rows + k1) * n_t + u) + (wave & 1)] = col1;
  }
  // sub-block c (key columns 32c..32c+31 of the square) of this wave's 32 rows
  const uint64_t ba0 = __ballot(any0), bl0 = __ballot(all0), bn0 = __ballot(nz0);
  const uint64_t ba1 = __ballot(any1), bl1 = __ballot(all1), bn1 = __ballot(nz1);
  if (lane == 0) {
    auto lo = [](uint64_t m) { return static_cast<uint32_t>(m & 0xffffffffull); };
    auto hi = [](uint64_t m) { return static_cast<uint32_t>(m >> 32); };
    uint32_t f = 0;
    f |= (lo(ba0) != 0) << 0 | (hi(ba0) != 0) << 1 | (lo(ba1) != 0) << 2 | (hi(ba1) != 0) << 3;
    f |= (lo(bl0) == ~0u) << 4 | (hi(bl0) == ~0u) << 5 | (lo(bl1) == ~0u) << 6 |
         (hi(bl1) == ~0u) << 7;
    f |= (lo(bn0) != 0) << 8 | (hi(bn0) != 0) << 9 | (lo(bn1) != 0) << 10 | (hi(bn1) != 0) << 11;
    flags[wave] = f;
  }
  __syncthreads();
  if (tid < 4) {
    // tid 0, 1: query-major kinds of key tile 2j + tid; tid 2, 3: key-major kinds
    // of query tile 2i + tid - 2.
    const int h = tid & 1;
    uint32_t kb = 0;
    for (int sl = 0; sl < 4; ++sl) {
      bool any, all, nz;
      if (tid < 2) {  // query slice sl, sub-blocks (sl, 2h), (sl, 2h + 1)
        const uint32_t f = flags[sl];
        any = ((f >> (2 * h)) & 3) != 0;
        all = ((f >> (4 + 2 * h)) & 3) == 3;
        nz = ((f >> (8 + 2 * h)) & 3) != 0;
      } else {  // key slice sl, sub-blocks (2h, sl), (2h + 1, sl)
        const uint32_t f0 = flags[2 * h], f1 = flags[2 * h + 1];
        any = ((f0 >> sl) & 1) | ((f1 >> sl) & 1);
        all = ((f0 >> (4 + sl)) & 1) & ((f1 >> (4 + sl)) & 1);
        nz = ((f0 >> (8 + sl)) & 1) | ((f1 >> (8 + sl)) & 1);
      }
      kb |= static_cast<uint32_t>(!any ? 0 : (all ? 1 : (nz ? 3 : 2))) << (2 * sl);
    }
    if (tid < 2) {
      const int t = 2 * j + h;
      if (t < n_t) kinds_q[(static_cast<int64_t>(mr) * n_b + i) * n_t + t] = static_cast<uint8_t>(kb);
    } else {
      const int uu = 2 * i + h;
      if (uu < n_t) kinds_kv[(static_cast<int64_t>(mr) * n_b + j) * n_t + uu] = static_cast<uint8_t>(kb);
    }
  }
}

__global__ __launch_bounds__(256) void wattn_mask_compact_kernel(
    const uint8_t* __restrict__ kinds, int n_rows, int n_t, int32_t* __restrict__ entries,
    int32_t* __restrict__ cnt) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  const uint8_t* kr = kinds + static_cast<int64_t>(row) * n_t;
  int32_t* er = entries + static_cast<int64_t>(row) * n_t;
  int count = 0;
  for (int t0 = 0; t0 < n_t; t0 += 64) {
    const int t = t0 + lane;
    const int kb = t < n_t ? kr[t] : 0;
    const uint64_t m = __ballot(kb != 0);
    if (kb != 0) {
      const int before = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0));
      er[count + before] = t | (kb << 16);
    }
    count += __popcll(m);
  }
  if (lane == 0) cnt[row] = count;
}

// 3. wattn_mask_order_kernel: the launch order of each orientation (workgroup 0:
//    query-major, 1: key-major): blocks by list length, longest first (ties by
//    block index), the length of a block being its largest over the first
//    kOrderRows mask rows; rank r launches order[r] of every head, and rank 0 of
//    all heads goes first (one lead rank, as in the host schedule). Up to
//    kOrderBlocks blocks (S <= 65536); beyond that the order is the identity.
constexpr int kOrderBlocks = 512, kOrderRows = 64;

__global__ __launch_bounds__(256) void wattn_mask_order_kernel(const int32_t* __restrict__ cnt,
                                                               int n_mr, int n_b,
                                                               int32_t* __restrict__ order) {
  __shared__ int len[kOrderBlocks];
  const int side = blockIdx.x;
  const int32_t* c = cnt + static_cast<int64_t>(side) * n_mr * n_b;
  int32_t* o = order + side * n_b;
  if (n_b > kOrderBlocks) {
    for (int b = threadIdx.x; b < n_b; b += 256) o[b] = b;
    return;
  }
  const int rows = min(n_mr, kOrderRows);
  for (int b = threadIdx.x; b < n_b; b += 256) {
    int m = 0;
    for (int r = 0; r < rows; ++r) m = max(m, c[static_cast<int64_t>(r) * n_b + b]);
    len[b] = m;
  }
  __syncthreads();
  for (int b = threadIdx.x; b < n_b; b += 256) {
    const int lb = len[b];
    int rank = 0;
    for (int b2 = 0; b2 < n_b; ++b2) rank += (len[b2] > lb) | ((len[b2] == lb) & (b2 < b));
    o[rank] = b;
  }
}

// Byte offsets of the parts of a mask workspace (each 256-byte aligned): the
// launch orders, query-major then key-major; the tile kinds, query-major rows
// then key-major rows; the entries, same order; the counts, same order.
struct MaskWs {
  size_t order, kinds_q, kinds_kv, ent_q, ent_kv, cnt_q, cnt_kv, bits_q, bits_kv, total;
  int64_t rows;  // list rows of each orientation: mask rows x blocks
};
inline MaskWs mask_ws_layout(int S, int mask_batch, int mask_heads) {
  auto up = [](size_t x) { return (x + 255) & ~static_cast<size_t>(255); };
  const size_t n_b = (S + 127) / 128, n_t = (S + 63) / 64;
  const size_t rows = static_cast<size_t>(mask_batch) * mask_heads * n_b;
  MaskWs w;
  w.rows = static_cast<int64_t>(rows);
  w.order = 0;  // query-major, then key-major at order + n_b * 4
  w.kinds_q = up(2 * n_b * 4);
  w.kinds_kv = w.kinds_q + rows * n_t;
  w.ent_q = w.kinds_q + up(2 * rows * n_t);
  w.ent_kv = w.ent_q + rows * n_t * 4;
  w.cnt_q = w.ent_q + up(2 * rows * n_t * 4);
  w.cnt_kv = w.cnt_q + rows * 4;
  // bitmaps: one 64-bit word per (mask row, position padded to 128, tile)
  const size_t words = static_cast<size_t>(mask_batch) * mask_heads * n_b * 128 * n_t;
  w.bits_q = w.cnt_q + up(2 * rows * 4);
  w.bits_kv = w.bits_q + words * 8;
  w.total = w.bits_kv + words * 8;
  return w;
}

// Checks the options of the *_ex entry points and fills the kernels' AttnX (with
// the query-major counts; the caller switches to the key-major ones). feat gets the
// kFeat bits.
int make_attn_x(const tmac_attn_opts* o, int B, int H, int S, AttnX* x, int* feat) {
  *x = AttnX{};
  *feat = 0;
  x->keep_scale = 1.f;
  if (!o) return TMAC_OK;
  if (!(o->dropout_p >= 0.f && o->dropout_p < 1.f)) return TMAC_ERR_VALUE;
  if (o->dropout_p > 0.f) {
    *feat |= kFeatDrop;
    // 16-bit draws: dropped below floor(p * 2^16); kept ones scaled by the inverse
    // of the exact keep probability
    const double th = floor(static_cast<double>(o->dropout_p) * 65536.0);
    x->thresh = th >= 65535.0 ? 65535u : static_cast<uint32_t>(th);
    x->keep_scale = 65536.f / static_cast<float>(65536u - x->thresh);
    x->seed0 = static_cast<uint32_t>(o->dropout_seed);
    x->seed1 = static_cast<uint32_t>(o->dropout_seed >> 32);
  }
  if (o->d_mask_grad) {
    // a gradient exists for an additive mask only
    if (!o->d_mask || o->mask_format != TMAC_MASK_ADD_F32) return TMAC_ERR_VALUE;
    if (reinterpret_cast<uintptr_t>(o->d_mask_grad) & 3u) return TMAC_ERR_ALIGN;
    x->dbias = o->d_mask_grad;
    *feat |= kFeatDBias;
  }
  if (o->d_mask) {
    if (o->mask_format != TMAC_MASK_BOOL && o->mask_format != TMAC_MASK_ADD_F32) return TMAC_ERR_DTYPE;
    if (!(o->mask_batch == 1 || o->mask_batch == B) || !(o->mask_heads == 1 || o->mask_heads == H))
      return TMAC_ERR_SHAPE;
    for (int i = 0; i < 3; ++i)
      if (o->mask_strides[i] < 0) return TMAC_ERR_SHAPE;
    if (o->mask_strides[2] < S) return TMAC_ERR_SHAPE;
    if (o->mask_format == TMAC_MASK_ADD_F32 && (reinterpret_cast<uintptr_t>(o->d_mask) & 3u))
      return TMAC_ERR_ALIGN;
    const MaskWs w = mask_ws_layout(S, o->mask_batch, o->mask_heads);
    if (!o->d_mask_ws || o->mask_ws_bytes < w.total) return TMAC_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(o->d_mask_ws) & 255u) return TMAC_ERR_ALIGN;
    *feat |= kFeatMask;
    if (o->mask_format == TMAC_MASK_BOOL) *feat |= kFeatBool;
    x->mask = o->d_mask;
    x->fmt = o->mask_format;
    x->msb = o->mask_strides[0];
    x->msh = o->mask_strides[1];
    x->msq = o->mask_strides[2];
    x->mb1 = o->mask_batch == 1;
    x->mh1 = o->mask_heads == 1;
    x->MH = o->mask_heads;
    x->cnt = reinterpret_cast<const int32_t*>(static_cast<const char*>(o->d_mask_ws) + w.cnt_q);
    x->cap = (S + 63) / 64;
    x->bits = reinterpret_cast<const uint64_t*>(static_cast<const char*>(o->d_mask_ws) + w.bits_q);
  }
  return TMAC_OK;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Launch map and grid size for n_bh heads x n_blk blocks with the n_lead
// heaviest blocks of each head launched first.
inline WorkMap make_work_map(int n_bh, int n_blk, int n_lead, unsigned* grid) {
  WorkMap m;
  m.n_bh = n_bh;
  m.n_blk = n_blk;
  m.n_lead = n_lead;
  m.lead_pad = (n_bh * n_lead + 7) & ~7;
  m.per_xcd = (n_bh * (n_blk - n_lead) + 7) / 8;
  *grid = static_cast<unsigned>(m.lead_pad + 8 * m.per_xcd);
  return m;
}

// Arguments of one attention launch (forward or backward), gathered so the
// kernels can be dispatched over dtype, head dimension and feature bits.
struct AttnLaunch {
  const void *Q, *K, *V, *O, *dO;
  void *Out, *dQ, *dK, *dV;
  float* lse_out;
  const float* lse;
  float* delta;
  const int64_t *qs, *ks, *vs, *os, *gs, *dqs, *dks, *dvs;
  int B, H, S, dh, dtype;
  MaskParams mp;
  float scale, scale_log2;
  const int32_t *row_ptr, *entries, *order, *col_ptr, *entries_kv, *order_kv;
  WorkMap wm_q, wm_kv;
  unsigned grid_q, grid_kv;
  AttnX ax_q, ax_kv;  // the caller's mask with the query-major / key-major counts
  hipStream_t s;
};

template <int D, int FEAT>
void launch_fwd(const AttnLaunch& a) {
  const int64_t *qs = a.qs, *ks = a.ks, *vs = a.vs, *os = a.os;
  if (a.dtype == TMAC_F32) {
    hipLaunchKernelGGL((wattn_fwd_f32m_kernel<D, FEAT>), dim3(a.grid_q), dim3(256), 0, a.s,
                       static_cast<const float*>(a.Q), static_cast<const float*>(a.K),
                       static_cast<const float*>(a.V), static_cast<float*>(a.Out), a.lse_out,
                       qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2], os[0], os[1],
                       os[2], a.H, a.mp, a.scale_log2, a.row_ptr, a.entries, a.order, a.wm_q,
                       a.ax_q);
  } else if (a.dtype == TMAC_BF16) {
    hipLaunchKernelGGL((wattn_fwd_mfma_kernel<TMAC_BF16, D, FEAT>), dim3(a.grid_q), dim3(256), 0,
                       a.s, static_cast<const uint16_t*>(a.Q), static_cast<const uint16_t*>(a.K),
                       static_cast<const uint16_t*>(a.V), static_cast<uint16_t*>(a.Out),
                       a.lse_out, qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2],
                       os[0], os[1], os[2], a.H, a.mp, a.scale_log2, a.row_ptr, a.entries,
                       a.order, a.wm_q, a.ax_q);
  } else {
    hipLaunchKernelGGL((wattn_fwd_mfma_kernel<TMAC_F16, D, FEAT>), dim3(a.grid_q), dim3(256), 0,
                       a.s, static_cast<const uint16_t*>(a.Q), static_cast<const uint16_t*>(a.K),
                       static_cast<const uint16_t*>(a.V), static_cast<uint16_t*>(a.Out),
                       a.lse_out, qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2],
                       os[0], os[1], os[2], a.H, a.mp, a.scale_log2, a.row_ptr, a.entries,
                       a.order, a.wm_q, a.ax_q);
  }
}

// Backward, 16-bit MFMA kernels: dQ (which also writes the row sums Δ), then dK/dV.
template <int DT, int D, int FEAT>
void launch_bwd_mfma(const AttnLaunch& a) {
  const int64_t *qs = a.qs, *ks = a.ks, *vs = a.vs, *os = a.os, *gs = a.gs, *dqs = a.dqs,
                *dks = a.dks, *dvs = a.dvs;
  const auto* Q = static_cast<const uint16_t*>(a.Q);
  const auto* K = static_cast<const uint16_t*>(a.K);
  const auto* V = static_cast<const uint16_t*>(a.V);
  const auto* O = static_cast<const uint16_t*>(a.O);
  const auto* G = static_cast<const uint16_t*>(a.dO);
  // The dQ copy ring addresses 64 rows of K and V with 32-bit byte offsets.
  bool ring = false;
  if constexpr (D == 64 && FEAT == 0) ring = ks[2] <= (1ll << 25) && vs[2] <= (1ll << 25);
#define TMAC_BWD_Q(RG)                                                                              \
  hipLaunchKernelGGL((wattn_bwd_q_kernel<DT, D, FEAT, RG>), dim3(a.grid_q), dim3(256), 0, a.s, Q, K, \
                     V, G, O, os[0], os[1], os[2], a.lse, a.delta, static_cast<uint16_t*>(a.dQ),    \
                     qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2], gs[0], gs[1],  \
                     gs[2], dqs[0], dqs[1], dqs[2], a.H, a.mp, a.scale, a.scale_log2, a.row_ptr,   \
                     a.entries, a.order, a.wm_q, a.ax_q)
  if constexpr (D == 64 && FEAT == 0) {
    if (ring) TMAC_BWD_Q(true);
    else TMAC_BWD_Q(false);
  } else {
    TMAC_BWD_Q(false);
  }
#undef TMAC_BWD_Q
  // The copy-ring kernel addresses 64 rows of Q and dO with 32-bit byte offsets.
  if constexpr (D == 64) {
    if (qs[2] <= (1ll << 25) && gs[2] <= (1ll << 25)) {
      hipLaunchKernelGGL((wattn_bwd_kv64_kernel<DT, (FEAT & ~kFeatDBias)>), dim3(a.grid_kv), dim3(256), 0, a.s, Q,
                         K, V, G, a.lse, a.delta, static_cast<uint16_t*>(a.dK),
                         static_cast<uint16_t*>(a.dV), qs[0], qs[1], qs[2], ks[0], ks[1], ks[2],
                         vs[0], vs[1], vs[2], gs[0], gs[1], gs[2], dks[0], dks[1], dks[2], dvs[0],
                         dvs[1], dvs[2], a.H, a.mp, a.scale, a.scale_log2, a.col_ptr,
                         a.entries_kv, a.order_kv, a.wm_kv, a.ax_kv);
      return;
    }
  }
  hipLaunchKernelGGL((wattn_bwd_kv_kernel<DT, D, (FEAT & ~kFeatDBias)>), dim3(a.grid_kv), dim3(256), 0, a.s, Q, K,
                     V, G, a.lse, a.delta, static_cast<uint16_t*>(a.dK),
                     static_cast<uint16_t*>(a.dV), qs[0], qs[1], qs[2], ks[0], ks[1], ks[2],
                     vs[0], vs[1], vs[2], gs[0], gs[1], gs[2], dks[0], dks[1], dks[2], dvs[0],
                     dvs[1], dvs[2], a.H, a.mp, a.scale, a.scale_log2, a.col_ptr, a.entries_kv,
                     a.order_kv, a.wm_kv, a.ax_kv);
}

// Backward, fp32 MFMA kernels (v_mfma_f32_32x32x2_f32): Δ, then dK/dV, then dQ.
template <int D, int FEAT>
void launch_bwd_f32(const AttnLaunch& a) {
  const int64_t *qs = a.qs, *ks = a.ks, *vs = a.vs, *os = a.os, *gs = a.gs, *dqs = a.dqs,
                *dks = a.dks, *dvs = a.dvs;
  const auto* Q = static_cast<const float*>(a.Q);
  const auto* K = static_cast<const float*>(a.K);
  const auto* V = static_cast<const float*>(a.V);
  const auto* O = static_cast<const float*>(a.O);
  const auto* G = static_cast<const float*>(a.dO);
  const int64_t n_rows = static_cast<int64_t>(a.B) * a.H * a.S;
  const unsigned dgrid = static_cast<unsigned>((n_rows * D + 2047) / 2048);
  hipLaunchKernelGGL((wattn_bwd_delta_f32_kernel<D>), dim3(dgrid), dim3(256), 0, a.s, O, G,
                     a.delta, os[0], os[1], os[2], gs[0], gs[1], gs[2], a.H, a.S, n_rows);
  hipLaunchKernelGGL((wattn_bwd_kv_f32m_kernel<D, (FEAT & ~kFeatDBias)>), dim3(a.grid_kv), dim3(256), 0, a.s, Q, K,
                     V, G, a.lse, a.delta, static_cast<float*>(a.dK), static_cast<float*>(a.dV),
                     qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2], gs[0], gs[1],
                     gs[2], dks[0], dks[1], dks[2], dvs[0], dvs[1], dvs[2], a.H, a.mp, a.scale,
                     a.scale_log2, a.col_ptr, a.entries_kv, a.order_kv, a.wm_kv, a.ax_kv);
  hipLaunchKernelGGL((wattn_bwd_q_f32m_kernel<D, FEAT>), dim3(a.grid_q), dim3(256), 0, a.s, Q, K, V,
                     G, a.lse, a.delta, static_cast<float*>(a.dQ), qs[0], qs[1], qs[2], ks[0],
                     ks[1], ks[2], vs[0], vs[1], vs[2], gs[0], gs[1], gs[2], dqs[0], dqs[1],
                     dqs[2], a.H, a.mp, a.scale, a.scale_log2, a.row_ptr, a.entries, a.order,
                     a.wm_q, a.ax_q);
}

template <int FEAT>
void dispatch(const AttnLaunch& a, bool bwd) {
  const int d = a.dh;
  if (!bwd) {
    constexpr int F = FEAT & ~kFeatDBias;  // the forward writes no gradient
    if (d == 32) launch_fwd<32, F>(a);
    else if (d == 64) launch_fwd<64, F>(a);
    else launch_fwd<128, F>(a);
  } else if (a.dtype == TMAC_F32) {
    if (d == 32) launch_bwd_f32<32, FEAT>(a);
    else if (d == 64) launch_bwd_f32<64, FEAT>(a);
    else launch_bwd_f32<128, FEAT>(a);
  } else if (a.dtype == TMAC_BF16) {
    if (d == 32) launch_bwd_mfma<TMAC_BF16, 32, FEAT>(a);
    else if (d == 64) launch_bwd_mfma<TMAC_BF16, 64, FEAT>(a);
    else launch_bwd_mfma<TMAC_BF16, 128, FEAT>(a);
  } else {
    if (d == 32) launch_bwd_mfma<TMAC_F16, 32, FEAT>(a);
    else if (d == 64) launch_bwd_mfma<TMAC_F16, 64, FEAT>(a);
    else launch_bwd_mfma<TMAC_F16, 128, FEAT>(a);
  }
}

// Checks shared by the forward and backward: sizes, dtype, strides, pointer
// alignment, and (without a caller's mask) the pattern's arguments.
int check_common(int B, int H, int S, int dh, int window, int n_persistent, int pattern,
                 int block_size, float scale, int dtype, bool masked,
                 std::initializer_list<const int64_t*> strides,
                 std::initializer_list<const void*> ptrs) {
  if (B <= 0 || H <= 0 || S <= 0) return TMAC_ERR_SHAPE;
  if (dh != 32 && dh != 64 && dh != 128) return TMAC_ERR_SHAPE;
  if (!masked) {
    if (pattern != TMAC_PATTERN_BAND && pattern != TMAC_PATTERN_BLOCKWIN) return TMAC_ERR_VALUE;
    if (n_persistent < 0 || window < 0 || n_persistent > S) return TMAC_ERR_VALUE;
    if (pattern == TMAC_PATTERN_BAND && n_persistent == S) return TMAC_ERR_VALUE;
    if (pattern == TMAC_PATTERN_BLOCKWIN && block_size <= 0) return TMAC_ERR_VALUE;
  }
  if (!(scale > 0.f)) return TMAC_ERR_VALUE;
  if (dtype != TMAC_F32 && dtype != TMAC_BF16 && dtype != TMAC_F16) return TMAC_ERR_DTYPE;
  const int vec = dtype == TMAC_F32 ? 4 : 8;  // elements per 16-byte vector
  for (const int64_t* st : strides)
    for (int i = 0; i < 3; ++i)
      if (st[i] < 0 || st[i] % vec) return TMAC_ERR_ALIGN;
  for (const void* p : ptrs)
    if (!aligned16(p)) return TMAC_ERR_ALIGN;
  if (static_cast<int64_t>(B) * H * ((S + 127) / 128) > (1ll << 30)) return TMAC_ERR_SHAPE;
  return TMAC_OK;
}

// Fills the pattern / mask part of a launch: work lists, launch maps, AttnX.
int setup_lists(AttnLaunch& a, const tmac_attn_opts* opts, int window, int n_persistent,
                int causal, int pattern, int block_size, const int32_t* row_ptr,
                const int32_t* entries, const int32_t* order, int n_lead,
                const int32_t* col_ptr, const int32_t* entries_kv, const int32_t* order_kv,
                int n_lead_kv, int* feat) {
  const int n_qb = (a.S + 127) / 128;  // 128-query blocks (fwd, dQ) and 128-key blocks (dK, dV)
  const int st = make_attn_x(opts, a.B, a.H, a.S, &a.ax_q, feat);
  if (st != TMAC_OK) return st;
  a.ax_kv = a.ax_q;
  a.mp = MaskParams{a.S, min(window, a.S), n_persistent, causal ? 1 : 0, pattern, block_size};
  if (*feat & kFeatMask) {
    const MaskWs w = mask_ws_layout(a.S, opts->mask_batch, opts->mask_heads);
    const char* ws = static_cast<const char*>(opts->d_mask_ws);
    a.ax_kv.cnt = reinterpret_cast<const int32_t*>(ws + w.cnt_kv);
    a.ax_kv.bits = reinterpret_cast<const uint64_t*>(ws + w.bits_kv);
    a.entries = reinterpret_cast<const int32_t*>(ws + w.ent_q);
    a.entries_kv = reinterpret_cast<const int32_t*>(ws + w.ent_kv);
    a.order = reinterpret_cast<const int32_t*>(ws + w.order);
    a.order_kv = a.order + n_qb;
    a.row_ptr = a.col_ptr = nullptr;
    n_lead = n_lead_kv = 1;  // the longest list of every head first (wattn_mask_order_kernel)
    a.mp = MaskParams{a.S, a.S, 0, 0, TMAC_PATTERN_BAND, 1};
  } else {
    if (!row_ptr || !entries || !order) return TMAC_ERR_NULL;
    a.row_ptr = row_ptr;
    a.entries = entries;
    a.order = order;
    a.col_ptr = col_ptr;
    a.entries_kv = entries_kv;
    a.order_kv = order_kv;
  }
  if (n_lead < 0 || n_lead > n_qb || n_lead_kv < 0 || n_lead_kv > n_qb) return TMAC_ERR_VALUE;
  a.wm_q = make_work_map(a.B * a.H, n_qb, n_lead, &a.grid_q);
  a.wm_kv = make_work_map(a.B * a.H, n_qb, n_lead_kv, &a.grid_kv);
  return TMAC_OK;
}

int launch_status(const AttnLaunch& a, int feat, bool bwd) {
  switch (feat) {
    case 0: dispatch<0>(a, bwd); break;
    case kFeatMask: dispatch<kFeatMask>(a, bwd); break;
    case kFeatDrop: dispatch<kFeatDrop>(a, bwd); break;
    case kFeatMask | kFeatDrop: dispatch<kFeatMask | kFeatDrop>(a, bwd); break;
    case kFeatMask | kFeatBool: dispatch<kFeatMask | kFeatBool>(a, bwd); break;
    case kFeatMask | kFeatDBias: dispatch<kFeatMask | kFeatDBias>(a, bwd); break;
    case kFeatMask | kFeatDrop | kFeatDBias: dispatch<kFeatMask | kFeatDrop | kFeatDBias>(a, bwd); break;
    default: dispatch<kFeatMask | kFeatDrop | kFeatBool>(a, bwd); break;
  }
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? TMAC_OK : static_cast<int>(err);
}

int wattn_fwd_impl(const void* d_Q, const int64_t q_strides[3], const void* d_K,
                   const int64_t k_strides[3], const void* d_V, const int64_t v_strides[3],
                   void* d_O, const int64_t o_strides[3], float* d_lse, int B, int H, int S,
                   int dh, int window, int n_persistent, int causal, int pattern, int block_size,
                   float scale, const int32_t* d_row_ptr, const int32_t* d_entries,
                   const int32_t* d_order, int n_lead, int dtype, void* stream,
                   const tmac_attn_opts* opts) {
  if (!d_Q || !d_K || !d_V || !d_O || !q_strides || !k_strides || !v_strides || !o_strides)
    return TMAC_ERR_NULL;
  const bool masked = opts && opts->d_mask;
  int st = check_common(B, H, S, dh, window, n_persistent, pattern, block_size, scale, dtype,
                        masked, {q_strides, k_strides, v_strides, o_strides},
                        {d_Q, d_K, d_V, d_O});
  if (st != TMAC_OK) return st;
  AttnLaunch a{};
  a.Q = d_Q;
  a.K = d_K;
  a.V = d_V;
  a.Out = d_O;
  a.lse_out = d_lse;
  a.qs = q_strides;
  a.ks = k_strides;
  a.vs = v_strides;
  a.os = o_strides;
  a.B = B;
  a.H = H;
  a.S = S;
  a.dh = dh;
  a.dtype = dtype;
  a.scale = scale;
  a.scale_log2 = scale * kLog2e;
  a.s = static_cast<hipStream_t>(stream);
  int feat = 0;
  st = setup_lists(a, opts, window, n_persistent, causal, pattern, block_size, d_row_ptr,
                   d_entries, d_order, n_lead, nullptr, nullptr, nullptr, 0, &feat);
  if (st != TMAC_OK) return st;
  return launch_status(a, feat & ~kFeatDBias, false);  // the forward writes no gradient
}

}  // namespace

extern "C" int tmac_wattn_fwd(const void* d_Q, const int64_t q_strides[3], const void* d_K,
                              const int64_t k_strides[3], const void* d_V,
                              const int64_t v_strides[3], void* d_O, const int64_t o_strides[3],
                              float* d_lse, int B, int H, int S, int dh, int window,
                              int n_persistent, int causal, int pattern, int block_size,
                              float scale, const int32_t* d_row_ptr, const int32_t* d_entries,
                              const int32_t* d_order, int n_lead, int dtype, void* stream) {
  return wattn_fwd_impl(d_Q, q_strides, d_K, k_strides, d_V, v_strides, d_O, o_strides, d_lse, B,
                        H, S, dh, window, n_persistent, causal, pattern, block_size, scale,
                        d_row_ptr, d_entries, d_order, n_lead, dtype, stream, nullptr);
}

extern "C" int tmac_wattn_fwd_ex(const void* d_Q, const int64_t q_strides[3], const void* d_K,
                                 const int64_t k_strides[3], const void* d_V,
                                 const int64_t v_strides[3], void* d_O,
                                 const int64_t o_strides[3], float* d_lse, int B, int H, int S,
                                 int dh, int window, int n_persistent, int causal, int pattern,
                                 int block_size, float scale, const int32_t* d_row_ptr,
                                 const int32_t* d_entries, const int32_t* d_order, int n_lead,
                                 int dtype, void* stream, const tmac_attn_opts* opts) {
  return wattn_fwd_impl(d_Q, q_strides, d_K, k_strides, d_V, v_strides, d_O, o_strides, d_lse, B,
                        H, S, dh, window, n_persistent, causal, pattern, block_size, scale,
                        d_row_ptr, d_entries, d_order, n_lead, dtype, stream, opts);
}

extern "C" size_t tmac_wattn_mask_workspace(int S, int mask_batch, int mask_heads) {
  if (S <= 0 || mask_batch <= 0 || mask_heads <= 0) return 0;
  return mask_ws_layout(S, mask_batch, mask_heads).total;
}

namespace {

// out[r][e] = sum over the (b, h) served by mask row r = (mb, mh) of
// ds[b][h][e], e < n (= S * S), in ascending b then h. Four elements per thread.
__global__ __launch_bounds__(256) void wattn_mask_grad_reduce_kernel(
    const float* __restrict__ ds, float* __restrict__ out, int64_t n, int B, int H, int mb1,
    int mh1) {
  const int r = blockIdx.y;  // mask row
  const int MH = mh1 ? 1 : H;
  const int rb = r / MH, rh = r - rb * MH;
  const int b0 = mb1 ? 0 : rb, b1 = mb1 ? B : rb + 1;
  const int h0 = mh1 ? 0 : rh, h1 = mh1 ? H : rh + 1;
  const int64_t e = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (e >= n) return;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int b = b0; b < b1; ++b)
    for (int hd = h0; hd < h1; ++hd) {
      const float* src = ds + (static_cast<int64_t>(b) * H + hd) * n + e;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (e + i < n) acc[i] += src[i];
    }
  float* dst = out + static_cast<int64_t>(r) * n + e;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (e + i < n) dst[i] = acc[i];
}

}  // namespace

extern "C" int tmac_wattn_mask_grad_reduce(const float* d_ds, int B, int H, int S, int mask_batch,
                                           int mask_heads, float* d_out, void* stream) {
  if (!d_ds || !d_out) return TMAC_ERR_NULL;
  if (B <= 0 || H <= 0 || S <= 0) return TMAC_ERR_SHAPE;
  if (!(mask_batch == 1 || mask_batch == B) || !(mask_heads == 1 || mask_heads == H))
    return TMAC_ERR_SHAPE;
  const int64_t n = static_cast<int64_t>(S) * S;
  const int64_t rows = static_cast<int64_t>(mask_batch) * mask_heads;
  const int64_t blocks = (n + 1023) / 1024;
  if (rows > 65535 || blocks > (1ll << 31) - 1) return TMAC_ERR_SHAPE;
  const float* out_end = d_out + rows * n;
  const float* ds_end = d_ds + static_cast<int64_t>(B) * H * n;
  if (d_out < ds_end && d_ds < out_end) return TMAC_ERR_VALUE;  // overlapping buffers
  hipLaunchKernelGGL(wattn_mask_grad_reduce_kernel,
                     dim3(static_cast<unsigned>(blocks), static_cast<unsigned>(rows)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), d_ds, d_out, n, B, H,
                     mask_batch == 1 && B > 1 ? 1 : 0, mask_heads == 1 && H > 1 ? 1 : 0);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? TMAC_OK : static_cast<int>(err);
}

extern "C" int tmac_wattn_mask_lists(const tmac_attn_opts* opts, int S, void* stream) {
  if (!opts || !opts->d_mask || !opts->d_mask_ws) return TMAC_ERR_NULL;
  if (S <= 0 || opts->mask_batch <= 0 || opts->mask_heads <= 0) return TMAC_ERR_SHAPE;
  const int n_b = (S + 127) / 128, n_t = (S + 63) / 64;
  const int64_t n_mr = static_cast<int64_t>(opts->mask_batch) * opts->mask_heads;
  if (n_mr > 65535 || n_b > 65535 || n_mr * n_b > (1ll << 29)) return TMAC_ERR_SHAPE;  // grid y, z
  AttnX x;
  int feat = 0;
  const int st = make_attn_x(opts, opts->mask_batch, opts->mask_heads, S, &x, &feat);
  if (st != TMAC_OK) return st;
  const MaskWs w = mask_ws_layout(S, opts->mask_batch, opts->mask_heads);
  char* ws = static_cast<char*>(opts->d_mask_ws);
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto* kinds_q = reinterpret_cast<uint8_t*>(ws + w.kinds_q);
  hipLaunchKernelGGL(wattn_mask_kinds_kernel, dim3(n_b, n_b, static_cast<unsigned>(n_mr)),
                     dim3(256), 0, s, x, S, n_b, n_t, kinds_q,
                     reinterpret_cast<uint8_t*>(ws + w.kinds_kv),
                     reinterpret_cast<uint64_t*>(ws + w.bits_q),
                     reinterpret_cast<uint32_t*>(ws + w.bits_kv));
  const int64_t n_rows = 2 * w.rows;  // query-major rows, then key-major rows
  hipLaunchKernelGGL(wattn_mask_compact_kernel, dim3(static_cast<unsigned>((n_rows + 3) / 4)),
                     dim3(256), 0, s, kinds_q, static_cast<int>(n_rows), n_t,
                     reinterpret_cast<int32_t*>(ws + w.ent_q),
                     reinterpret_cast<int32_t*>(ws + w.cnt_q));
  hipLaunchKernelGGL(wattn_mask_order_kernel, dim3(2), dim3(256), 0, s,
                     reinterpret_cast<const int32_t*>(ws + w.cnt_q), static_cast<int>(n_mr), n_b,
                     reinterpret_cast<int32_t*>(ws + w.order));
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? TMAC_OK : static_cast<int>(err);
}

namespace {

// Shared body of tmac_wattn_bwd, tmac_wattn_bwd_ex and tmac_wattn_bwd_noalloc:
// d_delta is the fp32 [B, H, S] row-sum buffer (the caller's workspace, or the
// static scratch).
int wattn_bwd_impl(const void* d_Q, const int64_t q_strides[3], const void* d_K,
                   const int64_t k_strides[3], const void* d_V, const int64_t v_strides[3],
                   const void* d_O, const int64_t o_strides[3], const void* d_dO,
                   const int64_t do_strides[3], const float* d_lse, float* d_delta, void* d_dQ,
                   const int64_t dq_strides[3], void* d_dK, const int64_t dk_strides[3],
                   void* d_dV, const int64_t dv_strides[3], int B, int H, int S, int dh,
                   int window, int n_persistent, int causal, int pattern, int block_size,
                   float scale, const int32_t* d_row_ptr, const int32_t* d_entries,
                   const int32_t* d_order, int n_lead, const int32_t* d_col_ptr,
                   const int32_t* d_entries_kv, const int32_t* d_order_kv, int n_lead_kv,
                   int dtype, void* stream, const tmac_attn_opts* opts) {
  if (!d_Q || !d_K || !d_V || !d_O || !d_dO || !d_lse || !d_delta || !d_dQ || !d_dK || !d_dV ||
      !q_strides || !k_strides || !v_strides || !o_strides || !do_strides || !dq_strides ||
      !dk_strides || !dv_strides)
    return TMAC_ERR_NULL;
  const bool masked = opts && opts->d_mask;
  if (!masked && (!d_row_ptr || !d_entries || !d_order || !d_col_ptr || !d_entries_kv ||
                  !d_order_kv))
    return TMAC_ERR_NULL;
  int st = check_common(B, H, S, dh, window, n_persistent, pattern, block_size, scale, dtype,
                        masked,
                        {q_strides, k_strides, v_strides, o_strides, do_strides, dq_strides,
                         dk_strides, dv_strides},
                        {d_Q, d_K, d_V, d_O, d_dO, d_dQ, d_dK, d_dV});
  if (st != TMAC_OK) return st;
  AttnLaunch a{};
  a.Q = d_Q;
  a.K = d_K;
  a.V = d_V;
  a.O = d_O;
  a.dO = d_dO;
  a.dQ = d_dQ;
  a.dK = d_dK;
  a.dV = d_dV;
  a.lse = d_lse;
  a.delta = d_delta;
  a.qs = q_strides;
  a.ks = k_strides;
  a.vs = v_strides;
  a.os = o_strides;
  a.gs = do_strides;
  a.dqs = dq_strides;
  a.dks = dk_strides;
  a.dvs = dv_strides;
  a.B = B;
  a.H = H;
  a.S = S;
  a.dh = dh;
  a.dtype = dtype;
  a.scale = scale;
  a.scale_log2 = scale * kLog2e;
  a.s = static_cast<hipStream_t>(stream);
  int feat = 0;
  st = setup_lists(a, opts, window, n_persistent, causal, pattern, block_size, d_row_ptr,
                   d_entries, d_order, n_lead, d_col_ptr, d_entries_kv, d_order_kv, n_lead_kv,
                   &feat);
  if (st != TMAC_OK) return st;
  return launch_status(a, feat, true);
}

// Row sums of the allocation-free backward: a file-scope device array, one copy
// per GPU, of TMAC_WATTN_BWD_SCRATCH_ROWS floats (16 MiB). Host code never
// passes `scratch` itself to a kernel (in host code the name is a host-side
// stand-in, not a device address): it passes the address hipGetSymbolAddress
// returns for the current device.
__device__ __align__(256) float scratch[TMAC_WATTN_BWD_SCRATCH_ROWS];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up once per device
// (with that device current) and kept; nullptr with *err set on failure.
float* scratch_on_current_device(int* err) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    *err = static_cast<int>(e);
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    *err = TMAC_ERR_VALUE;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      *err = e != hipSuccess ? static_cast<int>(e) : TMAC_ERR_NULL;
      return nullptr;
    }
    g_scratch_ptr[dev] = static_cast<float*>(ptr);
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" int tmac_wattn_bwd(const void* d_Q, const int64_t q_strides[3], const void* d_K,
                              const int64_t k_strides[3], const void* d_V,
                              const int64_t v_strides[3], const void* d_O,
                              const int64_t o_strides[3], const void* d_dO,
                              const int64_t do_strides[3], const float* d_lse, float* d_delta,
                              void* d_dQ, const int64_t dq_strides[3], void* d_dK,
                              const int64_t dk_strides[3], void* d_dV,
                              const int64_t dv_strides[3], int B, int H, int S, int dh, int window,
                              int n_persistent, int causal, int pattern, int block_size,
                              float scale, const int32_t* d_row_ptr, const int32_t* d_entries,
                              const int32_t* d_order, int n_lead, const int32_t* d_col_ptr,
                              const int32_t* d_entries_kv, const int32_t* d_order_kv,
                              int n_lead_kv, int dtype, void* stream) {
  return wattn_bwd_impl(d_Q, q_strides, d_K, k_strides, d_V, v_strides, d_O, o_strides, d_dO,
                        do_strides, d_lse, d_delta, d_dQ, dq_strides, d_dK, dk_strides, d_dV,
                        dv_strides, B, H, S, dh, window, n_persistent, causal, pattern, block_size,
                        scale, d_row_ptr, d_entries, d_order, n_lead, d_col_ptr, d_entries_kv,
                        d_order_kv, n_lead_kv, dtype, stream, nullptr);
}

extern "C" int tmac_wattn_bwd_ex(
    const void* d_Q, const int64_t q_strides[3], const void* d_K, const int64_t k_strides[3],
    const void* d_V, const int64_t v_strides[3], const void* d_O, const int64_t o_strides[3],
    const void* d_dO, const int64_t do_strides[3], const float* d_lse, float* d_delta, void* d_dQ,
    const int64_t dq_strides[3], void* d_dK, const int64_t dk_strides[3], void* d_dV,
    const int64_t dv_strides[3], int B, int H, int S, int dh, int window, int n_persistent,
    int causal, int pattern, int block_size, float scale, const int32_t* d_row_ptr,
    const int32_t* d_entries, const int32_t* d_order, int n_lead, const int32_t* d_col_ptr,
    const int32_t* d_entries_kv, const int32_t* d_order_kv, int n_lead_kv, int dtype,
    void* stream, const tmac_attn_opts* opts) {
  return wattn_bwd_impl(d_Q, q_strides, d_K, k_strides, d_V, v_strides, d_O, o_strides, d_dO,
                        do_strides, d_lse, d_delta, d_dQ, dq_strides, d_dK, dk_strides, d_dV,
                        dv_strides, B, H, S, dh, window, n_persistent, causal, pattern, block_size,
                        scale, d_row_ptr, d_entries, d_order, n_lead, d_col_ptr, d_entries_kv,
                        d_order_kv, n_lead_kv, dtype, stream, opts);
}

extern "C" int tmac_wattn_bwd_noalloc(
    const void* d_Q, const int64_t q_strides[3], const void* d_K, const int64_t k_strides[3],
    const void* d_V, const int64_t v_strides[3], const void* d_O, const int64_t o_strides[3],
    const void* d_dO, const int64_t do_strides[3], const float* d_lse, void* d_dQ,
    const int64_t dq_strides[3], void* d_dK, const int64_t dk_strides[3], void* d_dV,
    const int64_t dv_strides[3], int B, int H, int S, int dh, int window, int n_persistent,
    int causal, int pattern, int block_size, float scale, const int32_t* d_row_ptr,
    const int32_t* d_entries, const int32_t* d_order, int n_lead, const int32_t* d_col_ptr,
    const int32_t* d_entries_kv, const int32_t* d_order_kv, int n_lead_kv, int dtype,
    void* stream) {
  if (B <= 0 || H <= 0 || S <= 0) return TMAC_ERR_SHAPE;
  if (static_cast<int64_t>(B) * H * S > TMAC_WATTN_BWD_SCRATCH_ROWS) return TMAC_ERR_TOO_LARGE;
  // The scratch array is looked up for the current device; a stream of another
  // device would run the kernels there against this device's array.
  if (stream) {
    int cur = -1;
    hipDevice_t sdev = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e == hipSuccess) e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev);
    if (e != hipSuccess) return static_cast<int>(e);
    if (static_cast<int>(sdev) != cur) return TMAC_ERR_VALUE;
  }
  int err = TMAC_OK;
  float* delta = scratch_on_current_device(&err);
  if (!delta) return err;
  // every row of delta is written by the row-sum kernel before it is read: no clearing
  return wattn_bwd_impl(d_Q, q_strides, d_K, k_strides, d_V, v_strides, d_O, o_strides, d_dO,
                        do_strides, d_lse, delta, d_dQ, dq_strides, d_dK, dk_strides, d_dV,
                        dv_strides, B, H, S, dh, window, n_persistent, causal, pattern, block_size,
                        scale, d_row_ptr, d_entries, d_order, n_lead, d_col_ptr, d_entries_kv,
                        d_order_kv, n_lead_kv, dtype, stream, nullptr);
}
