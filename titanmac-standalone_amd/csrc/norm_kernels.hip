// RMSNorm over the last dimension, for gfx950.
//
//   y[m, :] = x[m, :] · r[m] · scale,   r[m] = 1 / sqrt(mean(x[m, :]²) + eps)
//
// TitanBlock's pre-norms (blocks/norms.py:44-62, used at blocks/titan_block.py
// :46-47,91,96). Memory-bound: one wave per row, each lane owning 16-byte
// vectors of the row (8 16-bit or 4 fp32 elements) in registers, fp32
// arithmetic, rows of up to 4096 elements. The backward
//   dx = r·(g ⊙ scale) − x · r³ · mean(g ⊙ scale ⊙ x),   dscale = Σ_m g ⊙ x · r
// writes each workgroup's partial dscale row (64 rows of x) to a workspace and
// sums the partial rows in a fixed order, so dscale is deterministic.

#include "tmac_device.h"

using namespace tmac;

namespace {

constexpr int kRowsPerWave = 16;  // backward: rows per wave; 64 rows per dscale partial

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

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// NV: vectors per lane held in registers (D <= 64 * NV * N).
template <int DT, int NV>
__global__ __launch_bounds__(256) void rmsnorm_fwd_kernel(const uint8_t* __restrict__ x,
                                                         int64_t ldx,
                                                         const uint8_t* __restrict__ scale,
                                                         uint8_t* __restrict__ y, int64_t ldy,
                                                         float* __restrict__ rstd, int M, int D,
                                                         float eps) {
  using V = Vec<DT>;
  constexpr int N = V::N;
  constexpr int E = DT == TMAC_F32 ? 4 : 2;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= M) return;
  const int n_vec = D / N;
  const uint8_t* xr = x + static_cast<int64_t>(row) * ldx * E;
  float v[NV][N];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = lane + 64 * i;
    if (c < n_vec) {
      V::load(xr + static_cast<int64_t>(c) * N * E, v[i]);
#pragma unroll
      for (int e = 0; e < N; ++e) ss = fmaf(v[i][e], v[i][e], ss);
    }
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(D) + eps);
  if (rstd && lane == 0) rstd[row] = r;
  uint8_t* yr = y + static_cast<int64_t>(row) * ldy * E;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = lane + 64 * i;
    if (c < n_vec) {
      float s[N], o[N];
      V::load(scale + static_cast<int64_t>(c) * N * E, s);
#pragma unroll
      for (int e = 0; e < N; ++e) o[e] = v[i][e] * r * s[e];
      V::store(yr + static_cast<int64_t>(c) * N * E, o);
    }
  }
}

// Backward: workgroup b owns rows [64b, 64b + 64), wave w of it rows
// 64b + 16w .. +16, walked with the next row's loads issued before the current
// row's arithmetic. The four waves' Σ g ⊙ x · r are added through LDS in wave
// order into partial[b][:]. Dynamic LDS: 3 * D floats.
template <int DT, int NV>
__global__ __launch_bounds__(256) void rmsnorm_bwd_kernel(
    const uint8_t* __restrict__ g, int64_t ldg, const uint8_t* __restrict__ x, int64_t ldx,
    const uint8_t* __restrict__ scale, const float* __restrict__ rstd, uint8_t* __restrict__ dx,
    int64_t lddx, float* __restrict__ partial, int M, int D) {
  using V = Vec<DT>;
  constexpr int N = V::N;
  constexpr int E = DT == TMAC_F32 ? 4 : 2;
  extern __shared__ float red[];  // [3][D]: waves 1..3
  const int w = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int n_vec = D / N;
  const int r0 = blockIdx.x * (4 * kRowsPerWave) + w * kRowsPerWave;
  const int r1 = min(r0 + kRowsPerWave, M);  // r0 >= r1: no rows, but the wave still joins the barrier
  float sc[NV][N], ds[NV][N];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = lane + 64 * i;
#pragma unroll
    for (int e = 0; e < N; ++e) ds[i][e] = 0.f;
    if (c < n_vec)
      V::load(scale + static_cast<int64_t>(c) * N * E, sc[i]);
    else
#pragma unroll
      for (int e = 0; e < N; ++e) sc[i][e] = 0.f;
  }
  float gv[NV][N], xv[NV][N];
  auto load_row = [&](int row, float (&gg)[NV][N], float (&xx)[NV][N])
      __attribute__((always_inline)) {
    const uint8_t* gr = g + static_cast<int64_t>(row) * ldg * E;
    const uint8_t* xr = x + static_cast<int64_t>(row) * ldx * E;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = lane + 64 * i;
      if (c < n_vec) {
        V::load(gr + static_cast<int64_t>(c) * N * E, gg[i]);
        V::load(xr + static_cast<int64_t>(c) * N * E, xx[i]);
      }
    }
  };
  if (r0 < r1) load_row(r0, gv, xv);
  for (int row = r0; row < r1; ++row) {
    float gn[NV][N], xn[NV][N];
    if (row + 1 < r1) load_row(row + 1, gn, xn);
    const float r = rstd[row];
    float dot = 0.f;  // Σ g ⊙ scale ⊙ x
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = lane + 64 * i;
      if (c < n_vec) {
#pragma unroll
        for (int e = 0; e < N; ++e) {
          dot = fmaf(gv[i][e] * sc[i][e], xv[i][e], dot);
          ds[i][e] = fmaf(gv[i][e] * xv[i][e], r, ds[i][e]);
        }
      }
    }
    dot = wave_sum(dot);
    const float k = r * r * r * dot / static_cast<float>(D);
    uint8_t* dr = dx + static_cast<int64_t>(row) * lddx * E;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = lane + 64 * i;
      if (c < n_vec) {
        float o[N];
#pragma unroll
        for (int e = 0; e < N; ++e) o[e] = r * gv[i][e] * sc[i][e] - xv[i][e] * k;
        V::store(dr + static_cast<int64_t>(c) * N * E, o);
      }
    }
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int e = 0; e < N; ++e) {
        gv[i][e] = gn[i][e];
        xv[i][e] = xn[i][e];
      }
  }
  if (w > 0) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = lane + 64 * i;
      if (c < n_vec)
#pragma unroll
        for (int e = 0; e < N; ++e) red[(w - 1) * D + c * N + e] = ds[i][e];
    }
  }
  __syncthreads();
  if (w == 0) {
    float* pr = partial + static_cast<int64_t>(blockIdx.x) * D;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = lane + 64 * i;
      if (c < n_vec)
#pragma unroll
        for (int e = 0; e < N; ++e) {
          const int d = c * N + e;
          pr[d] = ((ds[i][e] + red[d]) + red[D + d]) + red[2 * D + d];
        }
    }
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

constexpr int kMaxD = 4096;  // rows are held in registers: at most 16 fp32 / 8 16-bit vectors per lane

// Vectors per lane the kernels are instantiated for (1, 2, 4, 8, 16).
inline int nv_for(int n_vec) {
  const int need = (n_vec + 63) / 64;
  return need <= 1 ? 1 : need <= 2 ? 2 : need <= 4 ? 4 : need <= 8 ? 8 : 16;
}

int check_common(int M, int D, int dtype) {
  if (M <= 0 || D <= 0 || D > kMaxD) return TMAC_ERR_SHAPE;
  if (dtype != TMAC_F32 && dtype != TMAC_BF16 && dtype != TMAC_F16) return TMAC_ERR_DTYPE;
  const int vec = dtype == TMAC_F32 ? 4 : 8;
  if (D % vec) return TMAC_ERR_SHAPE;
  return TMAC_OK;
}

template <int DT>
void launch_fwd(const void* x, int64_t ldx, const void* scale, void* y, int64_t ldy, float* rstd,
                int M, int D, float eps, hipStream_t s) {
  const int nv = nv_for(D / Vec<DT>::N);
  const dim3 grid(static_cast<unsigned>((M + 3) / 4));
  const auto* xp = static_cast<const uint8_t*>(x);
  const auto* sp = static_cast<const uint8_t*>(scale);
  auto* yp = static_cast<uint8_t*>(y);
#define TMAC_RMS_FWD(NVV)                                                                         \
  hipLaunchKernelGGL((rmsnorm_fwd_kernel<DT, NVV>), grid, dim3(256), 0, s, xp, ldx, sp, yp, ldy, \
                     rstd, M, D, eps)
  switch (nv) {
    case 1: TMAC_RMS_FWD(1); break;
    case 2: TMAC_RMS_FWD(2); break;
    case 4: TMAC_RMS_FWD(4); break;
    default:
      if constexpr (Vec<DT>::N == 4) {
        if (nv == 16) {
          TMAC_RMS_FWD(16);
          break;
        }
      }
      TMAC_RMS_FWD(8);
      break;
  }
#undef TMAC_RMS_FWD
}

template <int DT>
void launch_bwd(const void* g, int64_t ldg, const void* x, int64_t ldx, const void* scale,
                const float* rstd, void* dx, int64_t lddx, float* dscale, float* ws, int M, int D,
                hipStream_t s) {
  const int nv = nv_for(D / Vec<DT>::N);
  const int n_blocks = (M + 4 * kRowsPerWave - 1) / (4 * kRowsPerWave);
  const dim3 grid(static_cast<unsigned>(n_blocks));
  const size_t shmem = 3 * static_cast<size_t>(D) * sizeof(float);
  const auto* gp = static_cast<const uint8_t*>(g);
  const auto* xp = static_cast<const uint8_t*>(x);
  const auto* sp = static_cast<const uint8_t*>(scale);
  auto* dp = static_cast<uint8_t*>(dx);
#define TMAC_RMS_BWD(NVV)                                                                          \
  hipLaunchKernelGGL((rmsnorm_bwd_kernel<DT, NVV>), grid, dim3(256), shmem, s, gp, ldg, xp, ldx, sp, \
                     rstd, dp, lddx, ws, M, D)
  switch (nv) {
    case 1: TMAC_RMS_BWD(1); break;
    case 2: TMAC_RMS_BWD(2); break;
    case 4: TMAC_RMS_BWD(4); break;
    default:
      if constexpr (Vec<DT>::N == 4) {
        if (nv == 16) {
          TMAC_RMS_BWD(16);
          break;
        }
      }
      TMAC_RMS_BWD(8);
      break;
  }
#undef TMAC_RMS_BWD
  hipLaunchKernelGGL(column_sum_kernel, dim3(static_cast<unsigned>((D + 63) / 64)), dim3(256), 0, s,
                     ws, dscale, static_cast<int64_t>(D), n_blocks, int64_t{0});
}

}  // namespace

extern "C" int tmac_rmsnorm_fwd(const void* d_x, int64_t ldx, const void* d_scale, void* d_y,
                                int64_t ldy, float* d_rstd, int M, int D, float eps, int dtype,
                                void* stream) {
  if (!d_x || !d_scale || !d_y) return TMAC_ERR_NULL;
  int st = check_common(M, D, dtype);
  if (st != TMAC_OK) return st;
  if (!(eps >= 0.f)) return TMAC_ERR_VALUE;
  const int vec = dtype == TMAC_F32 ? 4 : 8;
  if (ldx < D || ldy < D) return TMAC_ERR_SHAPE;
  if (ldx % vec || ldy % vec || !aligned16(d_x) || !aligned16(d_y) || !aligned16(d_scale))
    return TMAC_ERR_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == TMAC_F32)
    launch_fwd<TMAC_F32>(d_x, ldx, d_scale, d_y, ldy, d_rstd, M, D, eps, s);
  else if (dtype == TMAC_BF16)
    launch_fwd<TMAC_BF16>(d_x, ldx, d_scale, d_y, ldy, d_rstd, M, D, eps, s);
  else
    launch_fwd<TMAC_F16>(d_x, ldx, d_scale, d_y, ldy, d_rstd, M, D, eps, s);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? TMAC_OK : static_cast<int>(err);
}

extern "C" int tmac_rmsnorm_bwd_workspace(int M, int D, size_t* ws_bytes) {
  if (!ws_bytes) return TMAC_ERR_NULL;
  if (M <= 0 || D <= 0) return TMAC_ERR_SHAPE;
  *ws_bytes = static_cast<size_t>((M + 4 * kRowsPerWave - 1) / (4 * kRowsPerWave)) * D * sizeof(float);
  return TMAC_OK;
}

extern "C" int tmac_rmsnorm_bwd(const void* d_dy, int64_t lddy, const void* d_x, int64_t ldx,
                                const void* d_scale, const float* d_rstd, void* d_dx, int64_t lddx,
                                float* d_dscale, void* d_ws, size_t ws_bytes, int M, int D,
                                int dtype, void* stream) {
  if (!d_dy || !d_x || !d_scale || !d_rstd || !d_dx || !d_dscale) return TMAC_ERR_NULL;
  int st = check_common(M, D, dtype);
  if (st != TMAC_OK) return st;
  const int vec = dtype == TMAC_F32 ? 4 : 8;
  if (lddy < D || ldx < D || lddx < D) return TMAC_ERR_SHAPE;
  if (lddy % vec || ldx % vec || lddx % vec || !aligned16(d_dy) || !aligned16(d_x) ||
      !aligned16(d_dx) || !aligned16(d_scale))
    return TMAC_ERR_ALIGN;
  size_t need = 0;
  tmac_rmsnorm_bwd_workspace(M, D, &need);
  if (!d_ws || ws_bytes < need) return TMAC_ERR_WORKSPACE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* ws = static_cast<float*>(d_ws);
  if (dtype == TMAC_F32)
    launch_bwd<TMAC_F32>(d_dy, lddy, d_x, ldx, d_scale, d_rstd, d_dx, lddx, d_dscale, ws, M, D, s);
  else if (dtype == TMAC_BF16)
    launch_bwd<TMAC_BF16>(d_dy, lddy, d_x, ldx, d_scale, d_rstd, d_dx, lddx, d_dscale, ws, M, D, s);
  else
    launch_bwd<TMAC_F16>(d_dy, lddy, d_x, ldx, d_scale, d_rstd, d_dx, lddx, d_dscale, ws, M, D, s);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? TMAC_OK : static_cast<int>(err);
}
