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
// fp32 path: the exact-precision variant used by fp32 modules. One thread per
// query row (128 rows per workgroup), K/V tiles staged in LDS as fp32, plain
// FMA arithmetic, same work list and the same online softmax.

#include <math.h>

#include "tmac_device.h"

using namespace tmac;

namespace {

struct MaskParams {
  int S, window, Np, causal, pattern, bs;
};

// The effective mask, element by element (see tmac_wattn_tile_kinds for the
// reference citations of each clause).
__device__ __forceinline__ bool allowed(const MaskParams& p, int i, int j) {
  if (i >= p.S || j >= p.S) return false;
  if (i < p.Np) return p.pattern == TMAC_PATTERN_BLOCKWIN || j < p.Np;
  if (j < p.Np) return true;
  if (p.pattern == TMAC_PATTERN_BAND) {
    if (j < i - p.window) return false;
    return p.causal ? j <= i : j <= i + p.window;
  }
  const int r = i - p.Np, c = j - p.Np;
  const int b0 = (r / p.bs) * p.bs;
  if (c < b0 - p.window) return false;
  return p.causal ? c <= r : c < min(b0 + p.bs, p.S - p.Np);
}

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

template <int DT>
__global__ __launch_bounds__(256, 2) void wattn_fwd_mfma_kernel(
    const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
    uint16_t* __restrict__ O, float* __restrict__ lse, int64_t qsb, int64_t qsh, int64_t qss,
    int64_t ksb, int64_t ksh, int64_t kss, int64_t vsb, int64_t vsh, int64_t vss, int64_t osb,
    int64_t osh, int64_t oss, int H, MaskParams mp, float scale_log2,
    const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ entries, int n_qb,
    int n_work, int per_xcd) {
  // [buffer][K, V] 64x64 tiles.
  __shared__ __attribute__((aligned(16))) uint16_t smem[4 * kTileElems];

  const int logical = xcd_logical_id(per_xcd);
  if (logical >= n_work) return;
  const int bh = logical / n_qb;
  const int qb = n_qb - 1 - (logical - bh * n_qb);  // later blocks have longer lists: start them first
  const int b = bh / H, hd = bh - b * H;
  const int S = mp.S;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, h = lane >> 5;
  const int grp = (lane >> 4) & 1;
  const int q_row = qb * 128 + wave * 32 + l32;  // this lane's query row

  const uint16_t* Kbh = K + b * ksb + hd * ksh;
  const uint16_t* Vbh = V + b * vsb + hd * vsh;

  // Q rows as the B operand of Sᵀ = K·Qᵀ: lane holds Q[row][16kk + 8h .. +8].
  u32x4 qf[4];
  {
    const uint16_t* qp = Q + b * qsb + hd * qsh + static_cast<int64_t>(min(q_row, S - 1)) * qss + 8 * h;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) qf[kk] = ldg16(qp + 16 * kk);
  }

  const int e0 = row_ptr[qb], e1 = row_ptr[qb + 1];

  // K/V tile staging: 2 x 512 chunks of 16 bytes, 4 per thread.
  u32x4 pre[4];
  auto gload = [&](int kt) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int row = (tid >> 3) + 32 * (p & 1);
      const int key = min(kt * 64 + row, S - 1);  // rows past S: valid memory, always masked
      const uint16_t* src = (p < 2 ? Kbh + key * kss : Vbh + key * vss) + (tid & 7) * 8;
      pre[p] = ldg16(src);
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int row = (tid >> 3) + 32 * (p & 1);
      sts16(smem + (2 * buf + (p >> 1)) * kTileElems + row * kPitch + (tid & 7) * 8, pre[p]);
    }
  };

  f32x16 ot[2];
  ot[0] = f32x16{};
  ot[1] = f32x16{};
  float m_run = -INFINITY, l_run = 0.f;

  if (e0 < e1) {
    gload(entries[e0] & 0xffff);
    sstore(0);
  }
  __syncthreads();
  int buf = 0;
  for (int e = e0; e < e1; ++e) {
    const int ent = entries[e];
    const int kt = ent & 0xffff;
    const int kind = (ent >> (16 + 2 * wave)) & 3;
    const bool more = e + 1 < e1;
    if (more) gload(entries[e + 1] & 0xffff);

    if (kind != 0) {
      const uint16_t* kt_lds = smem + (2 * buf) * kTileElems;
      const uint16_t* vt_lds = smem + (2 * buf + 1) * kTileElems;
      f32x16 st[2];
      st[0] = f32x16{};
      st[1] = f32x16{};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
          const u32x4 a = lds16(kt_lds + (32 * kh + l32) * kPitch + 16 * kk + 8 * h);
          st[kh] = Mfma<DT>::run(a, qf[kk], st[kh]);
        }
      // st[kh][j] = S[q_row][key], key = kt*64 + 32kh + 8(j/4) + 4h + j%4.
      float mx = -INFINITY;
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          float x = st[kh][j] * scale_log2;
          if (kind == 2) {
            const int key = kt * 64 + 32 * kh + 8 * (j >> 2) + 4 * h + (j & 3);
            if (!allowed(mp, q_row, key)) x = -INFINITY;
          }
          st[kh][j] = x;
          mx = fmaxf(mx, x);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run, mx);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;  // row fully masked so far
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
      float rs = 0.f;
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const float pj = __builtin_amdgcn_exp2f(st[kh][j] - m_use);
          st[kh][j] = pj;
          rs += pj;
        }
      rs += __shfl_xor(rs, 32);
      l_run = l_run * alpha + rs;
      m_run = m_new;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) ot[dt] *= alpha;

      // Pᵀ as the B operand, 16 keys per MFMA: k-step ks covers keys
      // 16ks..16ks+15 and lane t-th value is key 16ks + 8(t/4) + 4h + t%4.
      u32x4 pb[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int kh = ks >> 1, j0 = 8 * (ks & 1);
        uint32_t w[4];
#pragma unroll
        for (int t = 0; t < 4; ++t)
          w[t] = static_cast<uint32_t>(Mfma<DT>::from_f32(st[kh][j0 + 2 * t])) |
                 (static_cast<uint32_t>(Mfma<DT>::from_f32(st[kh][j0 + 2 * t + 1])) << 16);
        pb[ks] = u32x4{w[0], w[1], w[2], w[3]};
      }
      // Vᵀ as the A operand in the same key order: rows 16ks + 4h + 0..3, then
      // 16ks + 8 + 4h + 0..3 of the V tile, column dh = 32dt + lane%32.
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) {
          const u32x4 va = lds_read_tr4x2(vt_lds, 16 * ks + 4 * h, 16 * ks + 8 + 4 * h,
                                          32 * dt + 16 * grp, lane);
          ot[dt] = Mfma<DT>::run(va, pb[ks], ot[dt]);
        }
    }
    if (more) sstore(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }

  if (q_row >= S) return;
  const float inv_l = l_run > 0.f ? 1.f / l_run : 0.f;
  uint16_t* op = O + b * osb + hd * osh + static_cast<int64_t>(q_row) * oss;
  // ot[dt][j] = O[q_row][32dt + 8(j/4) + 4h + j%4]: four consecutive dh per j/4.
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int jg = 0; jg < 4; ++jg) {
      u32x2 packed;
      packed.x = static_cast<uint32_t>(Mfma<DT>::from_f32(ot[dt][4 * jg] * inv_l)) |
                 (static_cast<uint32_t>(Mfma<DT>::from_f32(ot[dt][4 * jg + 1] * inv_l)) << 16);
      packed.y = static_cast<uint32_t>(Mfma<DT>::from_f32(ot[dt][4 * jg + 2] * inv_l)) |
                 (static_cast<uint32_t>(Mfma<DT>::from_f32(ot[dt][4 * jg + 3] * inv_l)) << 16);
      *reinterpret_cast<u32x2*>(op + 32 * dt + 8 * jg + 4 * h) = packed;
    }
  if (lse && h == 0)
    lse[(static_cast<int64_t>(b) * H + hd) * S + q_row] = (m_run + __log2f(l_run)) * kLn2;
}

// fp32 path: one query row per thread, 128 rows per workgroup (2 waves).
__global__ __launch_bounds__(128) void wattn_fwd_f32_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    float* __restrict__ O, float* __restrict__ lse, int64_t qsb, int64_t qsh, int64_t qss,
    int64_t ksb, int64_t ksh, int64_t kss, int64_t vsb, int64_t vsh, int64_t vss, int64_t osb,
    int64_t osh, int64_t oss, int H, MaskParams mp, float scale_log2,
    const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ entries, int n_qb,
    int n_work, int per_xcd) {
  __shared__ __attribute__((aligned(16))) float kt_lds[64 * 64];
  __shared__ __attribute__((aligned(16))) float vt_lds[64 * 64];

  const int logical = xcd_logical_id(per_xcd);
  if (logical >= n_work) return;
  const int bh = logical / n_qb;
  const int qb = n_qb - 1 - (logical - bh * n_qb);
  const int b = bh / H, hd = bh - b * H;
  const int S = mp.S;
  const int tid = threadIdx.x;
  const int q_row = qb * 128 + tid;
  const int sub = tid >> 5;  // 32-row slice of this thread

  float q[64], o[64];
  {
    const float* qp = Q + b * qsb + hd * qsh + static_cast<int64_t>(min(q_row, S - 1)) * qss;
#pragma unroll
    for (int d = 0; d < 64; d += 4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(qp + d);
      q[d] = v.x * scale_log2;
      q[d + 1] = v.y * scale_log2;
      q[d + 2] = v.z * scale_log2;
      q[d + 3] = v.w * scale_log2;
    }
  }
#pragma unroll
  for (int d = 0; d < 64; ++d) o[d] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  const float* Kbh = K + b * ksb + hd * ksh;
  const float* Vbh = V + b * vsb + hd * vsh;
  const int e0 = row_ptr[qb], e1 = row_ptr[qb + 1];
  for (int e = e0; e < e1; ++e) {
    const int ent = entries[e];
    const int kt = ent & 0xffff;
    __syncthreads();
    // 64 rows x 16 chunks of 16 bytes per tile; 8 chunks per thread per tile.
    for (int c = tid; c < 64 * 16; c += 128) {
      const int row = c >> 4, col = (c & 15) * 4;
      const int key = min(kt * 64 + row, S - 1);
      *reinterpret_cast<f32x4*>(kt_lds + row * 64 + col) =
          *reinterpret_cast<const f32x4*>(Kbh + key * kss + col);
      *reinterpret_cast<f32x4*>(vt_lds + row * 64 + col) =
          *reinterpret_cast<const f32x4*>(Vbh + key * vss + col);
    }
    __syncthreads();
    const int kind = (ent >> (16 + 2 * sub)) & 3;
    if (kind == 0) continue;
    float s[64];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 64; ++j) {
      float acc = 0.f;
#pragma unroll
      for (int d = 0; d < 64; ++d) acc = fmaf(q[d], kt_lds[j * 64 + d], acc);
      if (kind == 2 && !allowed(mp, q_row, kt * 64 + j)) acc = -INFINITY;
      s[j] = acc;
      mx = fmaxf(mx, acc);
    }
    const float m_new = fmaxf(m_run, mx);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = exp2f(m_run - m_use);
    l_run *= alpha;
#pragma unroll
    for (int d = 0; d < 64; ++d) o[d] *= alpha;
#pragma unroll
    for (int j = 0; j < 64; ++j) {
      const float pj = exp2f(s[j] - m_use);
      l_run += pj;
#pragma unroll
      for (int d = 0; d < 64; ++d) o[d] = fmaf(pj, vt_lds[j * 64 + d], o[d]);
    }
    m_run = m_new;
  }
  if (q_row >= S) return;
  const float inv_l = l_run > 0.f ? 1.f / l_run : 0.f;
  float* op = O + b * osb + hd * osh + static_cast<int64_t>(q_row) * oss;
#pragma unroll
  for (int d = 0; d < 64; d += 4)
    *reinterpret_cast<f32x4*>(op + d) =
        f32x4{o[d] * inv_l, o[d + 1] * inv_l, o[d + 2] * inv_l, o[d + 3] * inv_l};
  if (lse) lse[(static_cast<int64_t>(b) * H + hd) * S + q_row] = (m_run + log2f(l_run)) * kLn2;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" int tmac_wattn_fwd(const void* d_Q, const int64_t q_strides[3], const void* d_K,
                              const int64_t k_strides[3], const void* d_V,
                              const int64_t v_strides[3], void* d_O, const int64_t o_strides[3],
                              float* d_lse, int B, int H, int S, int dh, int window,
                              int n_persistent, int causal, int pattern, int block_size,
                              float scale, const int32_t* d_row_ptr, const int32_t* d_entries,
                              int dtype, void* stream) {
  if (!d_Q || !d_K || !d_V || !d_O || !q_strides || !k_strides || !v_strides || !o_strides ||
      !d_row_ptr || !d_entries)
    return TMAC_ERR_NULL;
  if (B <= 0 || H <= 0 || S <= 0) return TMAC_ERR_SHAPE;
  if (dh != 64) return TMAC_ERR_SHAPE;
  if (pattern != TMAC_PATTERN_BAND && pattern != TMAC_PATTERN_BLOCKWIN) return TMAC_ERR_VALUE;
  if (n_persistent < 0 || window < 0 || n_persistent > S) return TMAC_ERR_VALUE;
  if (pattern == TMAC_PATTERN_BAND && n_persistent == S) return TMAC_ERR_VALUE;
  if (pattern == TMAC_PATTERN_BLOCKWIN && block_size <= 0) return TMAC_ERR_VALUE;
  if (!(scale > 0.f)) return TMAC_ERR_VALUE;
  if (dtype != TMAC_F32 && dtype != TMAC_BF16 && dtype != TMAC_F16) return TMAC_ERR_DTYPE;
  const int vec = dtype == TMAC_F32 ? 4 : 8;  // elements per 16-byte vector
  const int64_t* all[4] = {q_strides, k_strides, v_strides, o_strides};
  for (const int64_t* st : all)
    for (int i = 0; i < 3; ++i)
      if (st[i] < 0 || st[i] % vec) return TMAC_ERR_ALIGN;
  if (!aligned16(d_Q) || !aligned16(d_K) || !aligned16(d_V) || !aligned16(d_O))
    return TMAC_ERR_ALIGN;

  const int n_qb = (S + 127) / 128;
  const int64_t n_work = static_cast<int64_t>(B) * H * n_qb;
  if (n_work > (1ll << 30)) return TMAC_ERR_SHAPE;
  const int per_xcd = static_cast<int>((n_work + 7) / 8);
  const MaskParams mp{S, window, n_persistent, causal ? 1 : 0, pattern, block_size};
  const float scale_log2 = scale * kLog2e;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t* qs = q_strides;
  const int64_t* ks = k_strides;
  const int64_t* vs = v_strides;
  const int64_t* os = o_strides;
  if (dtype == TMAC_F32) {
    hipLaunchKernelGGL(wattn_fwd_f32_kernel, dim3(8 * per_xcd), dim3(128), 0, s,
                       static_cast<const float*>(d_Q), static_cast<const float*>(d_K),
                       static_cast<const float*>(d_V), static_cast<float*>(d_O), d_lse, qs[0],
                       qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2], os[0], os[1], os[2],
                       H, mp, scale_log2, d_row_ptr, d_entries, n_qb, static_cast<int>(n_work),
                       per_xcd);
  } else if (dtype == TMAC_BF16) {
    hipLaunchKernelGGL((wattn_fwd_mfma_kernel<TMAC_BF16>), dim3(8 * per_xcd), dim3(256), 0, s,
                       static_cast<const uint16_t*>(d_Q), static_cast<const uint16_t*>(d_K),
                       static_cast<const uint16_t*>(d_V), static_cast<uint16_t*>(d_O), d_lse,
                       qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2], os[0], os[1],
                       os[2], H, mp, scale_log2, d_row_ptr, d_entries, n_qb,
                       static_cast<int>(n_work), per_xcd);
  } else {
    hipLaunchKernelGGL((wattn_fwd_mfma_kernel<TMAC_F16>), dim3(8 * per_xcd), dim3(256), 0, s,
                       static_cast<const uint16_t*>(d_Q), static_cast<const uint16_t*>(d_K),
                       static_cast<const uint16_t*>(d_V), static_cast<uint16_t*>(d_O), d_lse,
                       qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2], os[0], os[1],
                       os[2], H, mp, scale_log2, d_row_ptr, d_entries, n_qb,
                       static_cast<int>(n_work), per_xcd);
  }
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? TMAC_OK : static_cast<int>(err);
}
