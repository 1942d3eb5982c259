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
// chunk of 64 consecutive positions, keeps the last k input rows in registers
// (fp32) and writes each output row once; consecutive threads read consecutive
// 16-byte pieces of a row, so every row is read with full coalescing. The
// halo (k-1 rows before the chunk) is the only re-read.

#include "tmac_device.h"

using namespace tmac;

namespace {

constexpr int kChunk = 64;  // positions per thread

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
      w[i] = static_cast<uint32_t>(Mfma<DT16>::from_f32(v[2 * i])) |
             (static_cast<uint32_t>(Mfma<DT16>::from_f32(v[2 * i + 1])) << 16);
    *reinterpret_cast<u32x4*>(p) = u32x4{w[0], w[1], w[2], w[3]};
  }
};
template <>
struct Vec<TMAC_BF16> : Vec16<TMAC_BF16> {};
template <>
struct Vec<TMAC_F16> : Vec16<TMAC_F16> {};

template <int DT, int KS>
__global__ __launch_bounds__(256) void dwconv_causal_kernel(const uint8_t* __restrict__ in,
                                                            int64_t ld_in, const uint8_t* __restrict__ w,
                                                            uint8_t* __restrict__ out, int64_t ld_out,
                                                            int T, int C, int n_chunks) {
  using V = Vec<DT>;
  constexpr int N = V::N;
  constexpr int E = DT == TMAC_F32 ? 4 : 2;  // bytes per element
  const int vc = blockIdx.y * 256 + threadIdx.x;
  if (vc * N >= C) return;
  const int b = blockIdx.x / n_chunks;
  const int t0 = (blockIdx.x - b * n_chunks) * kChunk;
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
  // ring[j] holds input row t - (KS-1) + j for the row t being produced.
  float ring[KS][N];
#pragma unroll
  for (int j = 0; j < KS - 1; ++j) {
    const int t = t0 - (KS - 1) + j;
    if (t >= 0)
      V::load(ib + static_cast<int64_t>(t) * ld_in * E, ring[j]);
    else
#pragma unroll
      for (int i = 0; i < N; ++i) ring[j][i] = 0.f;
  }
  const int t1 = min(t0 + kChunk, T);
  for (int t = t0; t < t1; ++t) {
    V::load(ib + static_cast<int64_t>(t) * ld_in * E, ring[KS - 1]);
    float o[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < KS; ++j) acc = fmaf(wt[j][i], ring[j][i], acc);
      o[i] = acc;
    }
    V::store(ob + static_cast<int64_t>(t) * ld_out * E, o);
#pragma unroll
    for (int j = 0; j < KS - 1; ++j)
#pragma unroll
      for (int i = 0; i < N; ++i) ring[j][i] = ring[j + 1][i];
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
// walks the chunk from its end with register rings of the k d_out rows
// starting at t and of the k input rows ending at t, writes each d_in row once
// and its chunk's partial dw (fp32 [N channels][k]) to one workspace row.
// dwconv_wgrad_reduce_kernel then sums the partials of every (c, j) in chunk
// order, so dw is deterministic.
template <int DT, int KS>
__global__ __launch_bounds__(256) void dwconv_causal_bwd_kernel(
    const uint8_t* __restrict__ dout, int64_t ld_dout, const uint8_t* __restrict__ in,
    int64_t ld_in, const uint8_t* __restrict__ w, uint8_t* __restrict__ din, int64_t ld_din,
    float* __restrict__ partial, int T, int C, int n_chunks) {
  using V = Vec<DT>;
  constexpr int N = V::N;
  constexpr int E = DT == TMAC_F32 ? 4 : 2;
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

  // g[j] = d_out row t + j (g[0] loaded per step); x[j] = input row t - (KS-1) + j;
  // set up for t = t1 - 1.
  float g[KS][N], x[KS][N], dw[KS][N];
#pragma unroll
  for (int j = 0; j < KS; ++j) {
    const int tg = t1 - 1 + j;
    if (j > 0 && tg < T)
      V::load(gb + static_cast<int64_t>(tg) * ld_dout * E, g[j]);
    else
#pragma unroll
      for (int i = 0; i < N; ++i) g[j][i] = 0.f;
    const int tx = t1 - KS + j;
    if (tx >= 0)
      V::load(ib + static_cast<int64_t>(tx) * ld_in * E, x[j]);
    else
#pragma unroll
      for (int i = 0; i < N; ++i) x[j][i] = 0.f;
#pragma unroll
    for (int i = 0; i < N; ++i) dw[j][i] = 0.f;
  }
  for (int t = t1 - 1; t >= t0; --t) {
    V::load(gb + static_cast<int64_t>(t) * ld_dout * E, g[0]);
    float o[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < KS; ++j) {
        acc = fmaf(wt[j][i], g[KS - 1 - j][i], acc);
        dw[j][i] = fmaf(g[0][i], x[j][i], dw[j][i]);
      }
      o[i] = acc;
    }
    V::store(db + static_cast<int64_t>(t) * ld_din * E, o);
    // step to t - 1: d_out rows move up one slot, input rows down one slot and
    // input row t - KS enters at the bottom
#pragma unroll
    for (int j = KS - 1; j > 0; --j)
#pragma unroll
      for (int i = 0; i < N; ++i) g[j][i] = g[j - 1][i];
#pragma unroll
    for (int j = KS - 1; j > 0; --j)
#pragma unroll
      for (int i = 0; i < N; ++i) x[j][i] = x[j - 1][i];
    const int tx = t - KS;
    if (tx >= 0 && t > t0)
      V::load(ib + static_cast<int64_t>(tx) * ld_in * E, x[0]);
    else
#pragma unroll
      for (int i = 0; i < N; ++i) x[0][i] = 0.f;
  }
  // partial[(b * n_chunks + chunk)][c][j], contiguous N*KS floats per thread
  float* pp = partial + (static_cast<int64_t>(blockIdx.x) * C + c0) * KS;
#pragma unroll
  for (int i = 0; i < N; ++i)
#pragma unroll
    for (int j = 0; j < KS; ++j) pp[i * KS + j] = dw[j][i];
}

// dw[e] = Σ_p partial[p][e] over p = 0..P-1 in order, e = c * KS + j; fp32.
__global__ __launch_bounds__(256) void dwconv_wgrad_reduce_kernel(const float* __restrict__ partial,
                                                                  float* __restrict__ dw,
                                                                  int64_t n_elem, int P) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= n_elem) return;
  float acc = 0.f;
  for (int p = 0; p < P; ++p) acc += partial[static_cast<int64_t>(p) * n_elem + e];
  dw[e] = acc;
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
  hipLaunchKernelGGL(dwconv_wgrad_reduce_kernel, dim3(static_cast<unsigned>((n_elem + 255) / 256)),
                     dim3(256), 0, s, ws, d_dw, n_elem, static_cast<int>(gx));
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
