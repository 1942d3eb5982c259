// Causal depthwise 1-D convolution over the sequence axis, for gfx950.
//
//   out[b, t, c] = Σ_{j=0}^{k-1} w[c, j] · in[b, t - (k-1) + j, c]   (in[b, <0, c] = 0)
//
// This is what BlockSparseAttention applies to q, k and v after the fused
// projection: nn.Conv1d(d, d, k, padding=k-1, groups=d, bias=False) on the
// [B, d, T] transpose, trimmed to the first T outputs
// (attn/block_sparse_attention.py:87-98, 227-241). Here it runs directly on
// the [B, T, C] activation layout (C = 3d: q, k and v channels in one launch),
// so no transposes are needed.
//
// Memory-bound stencil: each thread owns one 16-byte vector of channels and a
// chunk of 64 consecutive positions, keeps a window of input rows in registers
// (fp32), loads the rows in groups of 4 before using them (four loads in
// flight per thread) and writes each output row once; consecutive threads read
// consecutive 16-byte pieces of a row, so every row is read with full
// coalescing. The halo (k-1 rows before the chunk) is the only re-read.

#include "tmac_device.h"

using namespace tmac;

namespace {

constexpr int kChunk = 64;  // positions per thread
constexpr int kGroup = 4;   // rows loaded together before use (memory-level parallelism)

template <int DT>
struct Vec;

template <>
struct Vec<TMAC_F32> {
  static constexpr int N = 4;
  static __device__ __forceinline__ void load(const void* p, float (&v)[4]) {
    const f32x4 x = *reinterpret_cast<const f32x4*>(p);
    v[0] = x.x;
    v[1] = x.y;
    v[2] = x.z;
    v[3] = x.w;
  }
  static __device__ __forceinline__ void store(void* p, const float (&v)[4]) {
    *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
  }
};

template <int DT16>
struct Vec16 {
  static constexpr int N = 8;
  static __device__ __forceinline__ void load(const void* p, float (&v)[8]) {
    const u32x4 x = *reinterpret_cast<const u32x4*>(p);
    const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = Mfma<DT16>::to_f32(static_cast<uint16_t>(w[i] & 0xffff));
      v[2 * i + 1] = Mfma<DT16>::to_f32(static_cast<uint16_t>(w[i] >> 16));
    }
  }
  static __device__ __forceinline__ void store(void* p, const float (&v)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = Mfma<DT16>::pack2(v[2 * i], v[2 * i + 1]);
    *reinterpret_cast<u32x4*>(p) = u32x4{w[0], w[1], w[2], w[3]};
  }
};
template <>
struct Vec<TMAC_BF16> : Vec16<TMAC_BF16> {};
template <>
struct Vec<TMAC_F16> : Vec16<TMAC_F16> {};

// Row `row` of a [rows, ld] buffer when `ok`, else zeros, without a branch: the
// load always reads a valid row (row 0 when not ok), so a group of these stays
// in flight together instead of each waiting behind its own branch.
template <int DT, int NN>
__device__ __forceinline__ void load_or_zero(const uint8_t* base, int64_t row_bytes, int row,
                                             bool ok, float (&v)[NN]) {
  Vec<DT>::load(base + static_cast<int64_t>(ok ? row : 0) * row_bytes, v);
#pragma unroll
  for (int e = 0; e < NN; ++e) v[e] = ok ? v[e] : 0.f;
}

template <int DT, int KS>
__global__ __launch_bounds__(256) void dwconv_causal_kernel(const uint8_t* __restrict__ in,
                                                            int64_t ld_in, const uint8_t* __restrict__ w,
                                                            uint8_t* __restrict__ out, int64_t ld_out,
                                                            int T, int C, int n_chunks) {
  using V = Vec<DT>;
  constexpr int N = V::N;
  constexpr int E = DT == TMAC_F32 ? 4 : 2;  // bytes per element
  constexpr int W = KS - 1 + kGroup;         // window rows
  const int vc = blockIdx.y * 256 + threadIdx.x;
  if (vc * N >= C) return;
  const int b = blockIdx.x / n_chunks;
  const int t0 = (blockIdx.x - b * n_chunks) * kChunk;
  const int t1 = min(t0 + kChunk, T);
  const int c0 = vc * N;

  // Taps of this thread's channels: wt[j][i] = w[c0 + i][j] (weights are
  // [C, KS], so the KS taps of one channel are contiguous).
  float wt[KS][N];
#pragma unroll
  for (int i = 0; i < N; ++i)
#pragma unroll
    for (int j = 0; j < KS; ++j) {
      const uint8_t* p = w + (static_cast<int64_t>(c0 + i) * KS + j) * E;
      if constexpr (DT == TMAC_F32)
        wt[j][i] = *reinterpret_cast<const float*>(p);
      else
        wt[j][i] = Mfma<DT>::to_f32(*reinterpret_cast<const uint16_t*>(p));
    }

  const uint8_t* ib = in + (static_cast<int64_t>(b) * T) * ld_in * E + static_cast<int64_t>(c0) * E;
  uint8_t* ob = out + (static_cast<int64_t>(b) * T) * ld_out * E + static_cast<int64_t>(c0) * E;
  // win[i] holds input row t - (KS-1) + i for the group of rows t .. t + kGroup - 1.
  float win[W][N];
  const int64_t rb_in = ld_in * E;
#pragma unroll
  for (int i = 0; i < KS - 1; ++i) {
    const int t = t0 - (KS - 1) + i;
    load_or_zero<DT>(ib, rb_in, t, t >= 0, win[i]);
  }
  for (int t = t0; t < t1; t += kGroup) {
    // the group's kGroup input rows are loaded before any is used
#pragma unroll
    for (int u = 0; u < kGroup; ++u) load_or_zero<DT>(ib, rb_in, t + u, t + u < t1, win[KS - 1 + u]);
#pragma unroll
    for (int u = 0; u < kGroup; ++u) {
      if (t + u < t1) {
        float o[N];
#pragma unroll
        for (int e = 0; e < N; ++e) {
          float acc = 0.f;
#pragma unroll
          for (int j = 0; j < KS; ++j) acc = fmaf(wt[j][e], win[u + j][e], acc);
          o[e] = acc;
        }
        V::store(ob + static_cast<int64_t>(t + u) * ld_out * E, o);
      }
    }
    // move down, lowest slot first (the slots overlap when KS - 1 > kGroup)
#pragma unroll
    for (int i = 0; i < KS - 1; ++i)
#pragma unroll
      for (int e = 0; e < N; ++e) win[i][e] = win[kGroup + i][e];
  }
}

template <int DT>
int launch_dwconv(const void* d_in, int64_t ld_in, const void* d_w, void* d_out, int64_t ld_out,
                  int B, int T, int C, int ks, hipStream_t s) {
  constexpr int N = Vec<DT>::N;
  const int n_vec = C / N;
  const int n_chunks = (T + kChunk - 1) / kChunk;
  const int64_t gx = static_cast<int64_t>(B) * n_chunks;
  const int gy = (n_vec + 255) / 256;
  if (gx > (1ll << 31) - 1 || gy > 65535) return TMAC_ERR_SHAPE;
  const dim3 grid(static_cast<unsigned>(gx), gy);
  const auto* in = static_cast<const uint8_t*>(d_in);
  const auto* w = static_cast<const uint8_t*>(d_w);
  auto* out = static_cast<uint8_t*>(d_out);
#define TMAC_DWCONV_CASE(KS)                                                                   \
  case KS:                                                                                     \
    hipLaunchKernelGGL((dwconv_causal_kernel<DT, KS>), grid, dim3(256), 0, s, in, ld_in, w, out, \
                       ld_out, T, C, n_chunks);                                                \
    break;
  switch (ks) {
    TMAC_DWCONV_CASE(1)
    TMAC_DWCONV_CASE(2)
    TMAC_DWCONV_CASE(3)
    TMAC_DWCONV_CASE(4)
    TMAC_DWCONV_CASE(5)
    TMAC_DWCONV_CASE(6)
    TMAC_DWCONV_CASE(7)
    TMAC_DWCONV_CASE(8)
    default:
      return TMAC_ERR_VALUE;
  }
#undef TMAC_DWCONV_CASE
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? TMAC_OK : static_cast<int>(err);
}

// Backward, one pass over d_out and the input:
//   d_in[b, t, c] = Σ_j w[c, j] · d_out[b, t + (k-1) - j, c]   (d_out[b, >= T, c] = 0)
//   dw[c, j]     = Σ_{b, t} d_out[b, t, c] · in[b, t - (k-1) + j, c]
// Each thread owns one 16-byte vector of channels and a chunk of 64 positions,
// walks the chunk from its end in groups of 4 rows with register windows of
// the d_out rows from t on and the input rows up to t, writes each d_in row
// once and its chunk's partial dw (fp32, tap-major) to one workspace row.
// column_sum_kernel then sums the partials of every (c, j) in a fixed order,
// so dw is deterministic.
template <int DT, int KS>
__global__ __launch_bounds__(256) void dwconv_causal_bwd_kernel(
    const uint8_t* __restrict__ dout, int64_t ld_dout, const uint8_t* __restrict__ in,
    int64_t ld_in, const uint8_t* __restrict__ w, uint8_t* __restrict__ din, int64_t ld_din,
    float* __restrict__ partial, int T, int C, int n_chunks) {
  using V = Vec<DT>;
  constexpr int N = V::N;
  constexpr int E = DT == TMAC_F32 ? 4 : 2;
  constexpr int W = KS - 1 + kGroup;
  const int vc = blockIdx.y * 256 + threadIdx.x;
  if (vc * N >= C) return;
  const int b = blockIdx.x / n_chunks;
  const int chunk = blockIdx.x - b * n_chunks;
  const int t0 = chunk * kChunk;
  const int t1 = min(t0 + kChunk, T);
  const int c0 = vc * N;

  float wt[KS][N];
#pragma unroll
  for (int i = 0; i < N; ++i)
#pragma unroll
    for (int j = 0; j < KS; ++j) {
      const uint8_t* p = w + (static_cast<int64_t>(c0 + i) * KS + j) * E;
      if constexpr (DT == TMAC_F32)
        wt[j][i] = *reinterpret_cast<const float*>(p);
      else
        wt[j][i] = Mfma<DT>::to_f32(*reinterpret_cast<const uint16_t*>(p));
    }

  const int64_t row0 = static_cast<int64_t>(b) * T;
  const uint8_t* gb = dout + row0 * ld_dout * E + static_cast<int64_t>(c0) * E;
  const uint8_t* ib = in + row0 * ld_in * E + static_cast<int64_t>(c0) * E;
  uint8_t* db = din + row0 * ld_din * E + static_cast<int64_t>(c0) * E;

  // Groups of kGroup rows t0 + gU .. t0 + gU + kGroup - 1, walked from the top.
  // For the group with first row tb: gw[i] = d_out row tb + i and
  // xw[i] = input row tb - (KS-1) + i, i < W. The KS-1 rows one group shares
  // with the next lower one move from the bottom of the windows to the top.
  float gw[W][N], xw[W][N], dw[KS][N];
  const int n_groups = (t1 - t0 + kGroup - 1) / kGroup;
  int tb = t0 + (n_groups - 1) * kGroup;
  const int64_t rb_g = ld_dout * E, rb_in = ld_in * E;
#pragma unroll
  for (int i = kGroup; i < W; ++i) {
    const int tg = tb + i, tx = tb - (KS - 1) + i;
    load_or_zero<DT>(gb, rb_g, tg, tg < T, gw[i]);
    load_or_zero<DT>(ib, rb_in, tx, tx >= 0 && tx < t1, xw[i]);
  }
#pragma unroll
  for (int j = 0; j < KS; ++j)
#pragma unroll
    for (int e = 0; e < N; ++e) dw[j][e] = 0.f;
  for (; tb >= t0; tb -= kGroup) {
#pragma unroll
    for (int u = 0; u < kGroup; ++u) {
      const int tg = tb + u, tx = tb - (KS - 1) + u;  // d_out rows in [t1, T) are the next chunk's
      load_or_zero<DT>(gb, rb_g, tg, tg < T, gw[u]);
      load_or_zero<DT>(ib, rb_in, tx, tx >= 0 && tx < t1, xw[u]);
    }
#pragma unroll
    for (int u = 0; u < kGroup; ++u) {
      if (tb + u < t1) {
        float o[N];
#pragma unroll
        for (int e = 0; e < N; ++e) {
          float acc = 0.f;
#pragma unroll
          for (int j = 0; j < KS; ++j) {
            acc = fmaf(wt[j][e], gw[u + KS - 1 - j][e], acc);
            dw[j][e] = fmaf(gw[u][e], xw[u + j][e], dw[j][e]);
          }
          o[e] = acc;
        }
        V::store(db + static_cast<int64_t>(tb + u) * ld_din * E, o);
      }
    }
    // move up, highest slot first (the slots overlap when KS - 1 > kGroup)
#pragma unroll
    for (int i = KS - 2; i >= 0; --i)
#pragma unroll
      for (int e = 0; e < N; ++e) {
        gw[kGroup + i][e] = gw[i][e];
        xw[kGroup + i][e] = xw[i][e];
      }
  }
  // partial[(b * n_chunks + chunk)][j][c]: for each tap, consecutive threads
  // write consecutive 16-byte pieces (coalesced); the reduction transposes to [c][j].
  float* pp = partial + static_cast<int64_t>(blockIdx.x) * C * KS + c0;
#pragma unroll
  for (int j = 0; j < KS; ++j)
#pragma unroll
    for (int i = 0; i < N; i += 4)
      *reinterpret_cast<f32x4*>(pp + static_cast<int64_t>(j) * C + i) =
          f32x4{dw[j][i], dw[j][i + 1], dw[j][i + 2], dw[j][i + 3]};
}

template <int DT>
int launch_dwconv_bwd(const void* d_dout, int64_t ld_dout, const void* d_in, int64_t ld_in,
                      const void* d_w, void* d_din, int64_t ld_din, float* d_dw, float* ws, int B,
                      int T, int C, int ks, hipStream_t s) {
  constexpr int N = Vec<DT>::N;
  const int n_vec = C / N;
  const int n_chunks = (T + kChunk - 1) / kChunk;
  const int64_t gx = static_cast<int64_t>(B) * n_chunks;
  const int gy = (n_vec + 255) / 256;
  if (gx > (1ll << 31) - 1 || gy > 65535) return TMAC_ERR_SHAPE;
  const dim3 grid(static_cast<unsigned>(gx), gy);
  const auto* g = static_cast<const uint8_t*>(d_dout);
  const auto* in = static_cast<const uint8_t*>(d_in);
  const auto* w = static_cast<const uint8_t*>(d_w);
  auto* din = static_cast<uint8_t*>(d_din);
#define TMAC_DWCONV_BWD_CASE(KS)                                                              \
  case KS:                                                                                    \
    hipLaunchKernelGGL((dwconv_causal_bwd_kernel<DT, KS>), grid, dim3(256), 0, s, g, ld_dout, \
                       in, ld_in, w, din, ld_din, ws, T, C, n_chunks);                        \
    break;
  switch (ks) {
    TMAC_DWCONV_BWD_CASE(1)
    TMAC_DWCONV_BWD_CASE(2)
    TMAC_DWCONV_BWD_CASE(3)
    TMAC_DWCONV_BWD_CASE(4)
    TMAC_DWCONV_BWD_CASE(5)
    TMAC_DWCONV_BWD_CASE(6)
    TMAC_DWCONV_BWD_CASE(7)
    TMAC_DWCONV_BWD_CASE(8)
    default:
      return TMAC_ERR_VALUE;
  }
#undef TMAC_DWCONV_BWD_CASE
  const int64_t n_elem = static_cast<int64_t>(C) * ks;
  hipLaunchKernelGGL(column_sum_kernel, dim3(static_cast<unsigned>((n_elem + 63) / 64)), dim3(256), 0,
                     s, ws, d_dw, n_elem, static_cast<int>(gx), static_cast<int64_t>(C));
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? TMAC_OK : static_cast<int>(err);
}

size_t dwconv_bwd_ws_bytes(int B, int T, int C, int ks) {
  const int64_t n_chunks = (T + kChunk - 1) / kChunk;
  return static_cast<size_t>(B) * n_chunks * C * ks * sizeof(float);
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" int tmac_dwconv_causal(const void* d_in, int64_t ld_in, const void* d_w, void* d_out,
                                  int64_t ld_out, int B, int T, int C, int ksize, int dtype,
                                  void* stream) {
  if (!d_in || !d_w || !d_out) return TMAC_ERR_NULL;
  if (B <= 0 || T <= 0 || C <= 0) return TMAC_ERR_SHAPE;
  if (ksize < 1 || ksize > 8) return TMAC_ERR_VALUE;
  if (dtype != TMAC_F32 && dtype != TMAC_BF16 && dtype != TMAC_F16) return TMAC_ERR_DTYPE;
  const int vec = dtype == TMAC_F32 ? 4 : 8;
  if (C % vec || ld_in < C || ld_out < C) return TMAC_ERR_SHAPE;
  if ((ld_in % vec) || (ld_out % vec) || !aligned16(d_in) || !aligned16(d_out)) return TMAC_ERR_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == TMAC_F32) return launch_dwconv<TMAC_F32>(d_in, ld_in, d_w, d_out, ld_out, B, T, C, ksize, s);
  if (dtype == TMAC_BF16) return launch_dwconv<TMAC_BF16>(d_in, ld_in, d_w, d_out, ld_out, B, T, C, ksize, s);
  return launch_dwconv<TMAC_F16>(d_in, ld_in, d_w, d_out, ld_out, B, T, C, ksize, s);
}

extern "C" int tmac_dwconv_causal_bwd_workspace(int B, int T, int C, int ksize, size_t* ws_bytes) {
  if (!ws_bytes) return TMAC_ERR_NULL;
  if (B <= 0 || T <= 0 || C <= 0) return TMAC_ERR_SHAPE;
  if (ksize < 1 || ksize > 8) return TMAC_ERR_VALUE;
  *ws_bytes = dwconv_bwd_ws_bytes(B, T, C, ksize);
  return TMAC_OK;
}

extern "C" int tmac_dwconv_causal_bwd(const void* d_dout, int64_t ld_dout, const void* d_in,
                                      int64_t ld_in, const void* d_w, void* d_din, int64_t ld_din,
                                      float* d_dw, void* d_ws, size_t ws_bytes, int B, int T, int C,
                                      int ksize, int dtype, void* stream) {
  if (!d_dout || !d_in || !d_w || !d_din || !d_dw) return TMAC_ERR_NULL;
  if (B <= 0 || T <= 0 || C <= 0) return TMAC_ERR_SHAPE;
  if (ksize < 1 || ksize > 8) return TMAC_ERR_VALUE;
  if (dtype != TMAC_F32 && dtype != TMAC_BF16 && dtype != TMAC_F16) return TMAC_ERR_DTYPE;
  const int vec = dtype == TMAC_F32 ? 4 : 8;
  if (C % vec || ld_dout < C || ld_in < C || ld_din < C) return TMAC_ERR_SHAPE;
  if ((ld_dout % vec) || (ld_in % vec) || (ld_din % vec) || !aligned16(d_dout) || !aligned16(d_in) ||
      !aligned16(d_din))
    return TMAC_ERR_ALIGN;
  if (!d_ws || ws_bytes < dwconv_bwd_ws_bytes(B, T, C, ksize)) return TMAC_ERR_WORKSPACE;
  float* ws = static_cast<float*>(d_ws);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == TMAC_F32)
    return launch_dwconv_bwd<TMAC_F32>(d_dout, ld_dout, d_in, ld_in, d_w, d_din, ld_din, d_dw, ws, B,
                                       T, C, ksize, s);
  if (dtype == TMAC_BF16)
    return launch_dwconv_bwd<TMAC_BF16>(d_dout, ld_dout, d_in, ld_in, d_w, d_din, ld_din, d_dw, ws,
                                        B, T, C, ksize, s);
  return launch_dwconv_bwd<TMAC_F16>(d_dout, ld_dout, d_in, ld_in, d_w, d_din, ld_din, d_dw, ws, B,
                                     T, C, ksize, s);
}
