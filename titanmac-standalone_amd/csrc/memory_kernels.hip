// Titans neural-memory update for gfx950: the gradient-norm clip, momentum and
// forgetting steps over all memory-MLP parameters, and the two elementwise
// steps of the memory MLP's hand-written backward.
//
//   norm = ||g||₂ over every tensor;  g' = g · scale(norm)
//   S ← η·S − θ·g';   W ← (1 − α)·W + S
//
// NeuralMemory.update (memory/neural_memory.py:386-434) flattens the MLP
// gradients into a cache, computes the norm, branches on the host twice (clip,
// NaN/Inf check), then runs five in-place passes plus a copy of the parameters
// into and out of a flat cache. fused_clip_momentum_update
// (kernels/memory_mlp.py:51-154) fuses the last two steps per tensor but still
// needs the norm first. Here it is two launches and no host synchronisation:
//
// 1. mem_sumsq_kernel: each workgroup sums g² (fp32) and counts non-finite
//    entries over its 256·per_thread 4-element chunks of one tensor and writes
//    one partial pair;
// 2. mem_update_kernel: every workgroup re-adds all partials in the same fixed
//    order (a few KB from L2), so all of them see the same norm bit for bit;
//    then each updates its own chunks: reads g, S, W once, writes S, W (and, if
//    given, a mirror copy of W and the clipped g). α and η are device scalars,
//    so the gates never come back to the host.
//
// Workgroups never straddle tensors: the host lays the workgroups out tensor by
// tensor, so each one finds its tensor with a uniform loop over at most 16
// entries. Memory-bound: 20 bytes per fp32 parameter (12 read, 8 written).

#include <math.h>

#include "tmac_device.h"

using namespace tmac;

namespace {

constexpr int kThreads = 256;
constexpr int kMaxTensors = TMAC_MEM_MAX_TENSORS;
constexpr int kMaxPartials = 512;  // workgroups (= partials) per launch at most: 2 per CU

struct TensorTable {
  void* g[kMaxTensors];
  void* s[kMaxTensors];
  void* w[kMaxTensors];
  void* c[kMaxTensors];             // mirror of the updated W, or null
  int64_t n[kMaxTensors];           // elements
  int wg_start[kMaxTensors + 1];    // first workgroup of each tensor
  int vec[kMaxTensors];             // 1: all of the tensor's pointers allow 4-element vectors
  int n_tensors;
  int per_thread;                   // 4-element chunks per thread
};

template <int DT>
struct Elem;

template <>
struct Elem<TMAC_F32> {
  static __device__ __forceinline__ void load4(const void* p, int64_t i, float (&v)[4]) {
    const f32x4 x = *reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + i);
    v[0] = x.x;
    v[1] = x.y;
    v[2] = x.z;
    v[3] = x.w;
  }
  static __device__ __forceinline__ void store4(void* p, int64_t i, const float (&v)[4]) {
    *reinterpret_cast<f32x4*>(static_cast<float*>(p) + i) = f32x4{v[0], v[1], v[2], v[3]};
  }
  static __device__ __forceinline__ float load1(const void* p, int64_t i) {
    return static_cast<const float*>(p)[i];
  }
  static __device__ __forceinline__ void store1(void* p, int64_t i, float v) {
    static_cast<float*>(p)[i] = v;
  }
};

template <int DT16>
struct Elem16 {
  static __device__ __forceinline__ void load4(const void* p, int64_t i, float (&v)[4]) {
    const u32x2 x = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(p) + i);
    v[0] = Mfma<DT16>::to_f32(static_cast<uint16_t>(x.x & 0xffff));
    v[1] = Mfma<DT16>::to_f32(static_cast<uint16_t>(x.x >> 16));
    v[2] = Mfma<DT16>::to_f32(static_cast<uint16_t>(x.y & 0xffff));
    v[3] = Mfma<DT16>::to_f32(static_cast<uint16_t>(x.y >> 16));
  }
  static __device__ __forceinline__ void store4(void* p, int64_t i, const float (&v)[4]) {
    *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(p) + i) =
        u32x2{Mfma<DT16>::pack2(v[0], v[1]), Mfma<DT16>::pack2(v[2], v[3])};
  }
  static __device__ __forceinline__ float load1(const void* p, int64_t i) {
    return Mfma<DT16>::to_f32(static_cast<const uint16_t*>(p)[i]);
  }
  static __device__ __forceinline__ void store1(void* p, int64_t i, float v) {
    static_cast<uint16_t*>(p)[i] = Mfma<DT16>::from_f32(v);
  }
};
template <>
struct Elem<TMAC_BF16> : Elem16<TMAC_BF16> {};
template <>
struct Elem<TMAC_F16> : Elem16<TMAC_F16> {};

// The tensor that workgroup `wg` belongs to (uniform across the workgroup).
__device__ __forceinline__ int tensor_of(const TensorTable& t, int wg) {
  int k = 0;
#pragma unroll
  for (int i = 1; i < kMaxTensors; ++i)
    if (i < t.n_tensors && wg >= t.wg_start[i]) k = i;
  return k;
}

// a[k] for a uniform k without indexing the kernel-argument array dynamically.
template <typename T, int N>
__device__ __forceinline__ T pick(const T (&a)[N], int k) {
  T r = a[0];
#pragma unroll
  for (int i = 1; i < N; ++i)
    if (i == k) r = a[i];
  return r;
}

// Sum over the workgroup; every thread gets the total.
template <typename T>
__device__ __forceinline__ T block_sum(T v, T* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int wave = threadIdx.x / 64;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

template <int DT>
__global__ __launch_bounds__(kThreads) void mem_sumsq_kernel(TensorTable t, float* part_sq,
                                                             uint32_t* part_bad) {
  using E = Elem<DT>;
  __shared__ float red_f[4];
  __shared__ uint32_t red_u[4];
  const int k = tensor_of(t, blockIdx.x);
  const void* g = pick(t.g, k);
  const int64_t n = pick(t.n, k);
  const bool vec = pick(t.vec, k) != 0;
  const int64_t chunk0 = static_cast<int64_t>(blockIdx.x - pick(t.wg_start, k)) * kThreads * t.per_thread;
  float acc = 0.f;
  uint32_t bad = 0;
  for (int j = 0; j < t.per_thread; ++j) {
    const int64_t e = 4 * (chunk0 + static_cast<int64_t>(j) * kThreads + threadIdx.x);
    if (e >= n) break;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (vec && e + 4 <= n) {
      E::load4(g, e, v);
    } else {
      for (int i = 0; i < 4 && e + i < n; ++i) v[i] = E::load1(g, e + i);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc += v[i] * v[i];
      bad += isfinite(v[i]) ? 0u : 1u;
    }
  }
  acc = block_sum(acc, red_f);
  bad = block_sum(bad, red_u);
  if (threadIdx.x == 0) {
    part_sq[blockIdx.x] = acc;
    part_bad[blockIdx.x] = bad;
  }
}

template <int DT>
__global__ __launch_bounds__(kThreads) void mem_update_kernel(
    TensorTable t, const float* __restrict__ part_sq, const uint32_t* __restrict__ part_bad,
    int n_part, const float* __restrict__ alpha_p, const float* __restrict__ eta_p,
    const float* __restrict__ norm_p, float theta, float max_norm, int mode,
    float* __restrict__ stats) {
  using E = Elem<DT>;
  __shared__ float red_f[4];
  __shared__ uint32_t red_u[4];
  float norm;
  uint32_t bad;
  if (norm_p) {  // the caller's norm (fused_clip_momentum_update takes it as an argument)
    norm = *norm_p;
    bad = isfinite(norm) ? 0u : 1u;
  } else {
    // Fixed-order re-add of the partials: thread i takes i, i + 256, ...
    float sq = 0.f;
    bad = 0;
    for (int i = threadIdx.x; i < n_part; i += kThreads) {
      sq += part_sq[i];
      bad += part_bad[i];
    }
    sq = block_sum(sq, red_f);
    bad = block_sum(bad, red_u);
    norm = sqrtf(sq);
  }
  float scale;
  bool skip, clipped;
  if (mode == TMAC_MEM_CLIP_MEMORY) {
    // NeuralMemory.update: scale by max_norm / norm only when norm > max_norm,
    // skip the whole update when any gradient is NaN or Inf.
    clipped = norm > max_norm;
    scale = clipped ? max_norm / norm : 1.f;
    skip = bad != 0;
  } else {
    // fused_clip_momentum_update: clamp(max_norm / (norm + 1e-8), max = 1), a NaN
    // ratio stays NaN as torch.clamp leaves it.
    const float r = max_norm / (norm + 1e-8f);
    scale = r > 1.f ? 1.f : r;
    clipped = r < 1.f;
    skip = false;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    stats[0] = norm;
    stats[1] = scale;
    stats[2] = skip ? 1.f : 0.f;
    stats[3] = clipped ? 1.f : 0.f;
  }
  if (skip) return;
  const float alpha = *alpha_p;
  const float eta = *eta_p;
  const float keep = 1.f - alpha;
  const bool write_g = mode == TMAC_MEM_CLIP_MEMORY && clipped;

  const int k = tensor_of(t, blockIdx.x);
  void* g = pick(t.g, k);
  void* s = pick(t.s, k);
  void* w = pick(t.w, k);
  void* c = pick(t.c, k);
  const int64_t n = pick(t.n, k);
  const bool vec = pick(t.vec, k) != 0;
  const int64_t chunk0 = static_cast<int64_t>(blockIdx.x - pick(t.wg_start, k)) * kThreads * t.per_thread;
  for (int j = 0; j < t.per_thread; ++j) {
    const int64_t e = 4 * (chunk0 + static_cast<int64_t>(j) * kThreads + threadIdx.x);
    if (e >= n) break;
    if (vec && e + 4 <= n) {
      float gv[4], sv[4], wv[4];
      E::load4(g, e, gv);
      E::load4(s, e, sv);
      E::load4(w, e, wv);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        gv[i] *= scale;
        sv[i] = eta * sv[i] - theta * gv[i];
        wv[i] = keep * wv[i] + sv[i];
      }
      E::store4(s, e, sv);
      E::store4(w, e, wv);
      if (c) E::store4(c, e, wv);
      if (write_g) E::store4(g, e, gv);
    } else {
      for (int i = 0; i < 4 && e + i < n; ++i) {
        const float gi = E::load1(g, e + i) * scale;
        const float si = eta * E::load1(s, e + i) - theta * gi;
        const float wi = keep * E::load1(w, e + i) + si;
        E::store1(s, e + i, si);
        E::store1(w, e + i, wi);
        if (c) E::store1(c, e + i, wi);
        if (write_g) E::store1(g, e + i, gi);
      }
    }
  }
}

// Elementwise: 4 elements per thread, the tail element by element.
template <int DT>
__global__ __launch_bounds__(kThreads) void silu_bwd_kernel(const void* __restrict__ dh,
                                                            const void* __restrict__ z,
                                                            void* __restrict__ dz, int64_t n,
                                                            int vec) {
  using E = Elem<DT>;
  const int64_t e = 4 * (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x);
  if (e >= n) return;
  if (vec && e + 4 <= n) {
    float a[4], b[4];
    E::load4(dh, e, a);
    E::load4(z, e, b);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float sg = 1.f / (1.f + expf(-b[i]));
      a[i] *= sg * (1.f + b[i] * (1.f - sg));
    }
    E::store4(dz, e, a);
  } else {
    for (int i = 0; i < 4 && e + i < n; ++i) {
      const float zi = E::load1(z, e + i);
      const float sg = 1.f / (1.f + expf(-zi));
      E::store1(dz, e + i, E::load1(dh, e + i) * sg * (1.f + zi * (1.f - sg)));
    }
  }
}

template <int DT>
__global__ __launch_bounds__(kThreads) void mse_grad_kernel(const void* __restrict__ y,
                                                            const void* __restrict__ v,
                                                            void* __restrict__ dy, int64_t n,
                                                            float coef, int vec) {
  using E = Elem<DT>;
  const int64_t e = 4 * (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x);
  if (e >= n) return;
  if (vec && e + 4 <= n) {
    float a[4], b[4];
    E::load4(y, e, a);
    E::load4(v, e, b);
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = coef * (a[i] - b[i]);
    E::store4(dy, e, a);
  } else {
    for (int i = 0; i < 4 && e + i < n; ++i)
      E::store1(dy, e + i, coef * (E::load1(y, e + i) - E::load1(v, e + i)));
  }
}

int elem_bytes(int dtype) { return dtype == TMAC_F32 ? 4 : 2; }

bool vec_aligned(const void* p, int dtype) {
  return p == nullptr || (reinterpret_cast<uintptr_t>(p) % (4 * elem_bytes(dtype))) == 0;
}

// Chunks per thread so that the partial count stays within kMaxPartials.
int per_thread_for(const int64_t* sizes, int n) {
  for (int pt = 1;; pt *= 2) {
    int64_t wgs = 0;
    for (int i = 0; i < n; ++i) wgs += (sizes[i] + 4LL * kThreads * pt - 1) / (4LL * kThreads * pt);
    if (wgs <= kMaxPartials) return pt;
  }
}

int64_t n_workgroups(const int64_t* sizes, int n, int pt) {
  int64_t wgs = 0;
  for (int i = 0; i < n; ++i) wgs += (sizes[i] + 4LL * kThreads * pt - 1) / (4LL * kThreads * pt);
  return wgs;
}

int check_dtype(int dtype) {
  return dtype == TMAC_F32 || dtype == TMAC_BF16 || dtype == TMAC_F16 ? TMAC_OK : TMAC_ERR_DTYPE;
}

}  // namespace

extern "C" int tmac_mem_update_workspace(const int64_t* sizes, int n_tensors, size_t* ws_bytes) {
  if (!sizes || !ws_bytes) return TMAC_ERR_NULL;
  if (n_tensors <= 0 || n_tensors > kMaxTensors) return TMAC_ERR_SHAPE;
  for (int i = 0; i < n_tensors; ++i)
    if (sizes[i] <= 0) return TMAC_ERR_SHAPE;
  const int pt = per_thread_for(sizes, n_tensors);
  *ws_bytes = static_cast<size_t>(n_workgroups(sizes, n_tensors, pt)) * 8;
  return TMAC_OK;
}

extern "C" int tmac_mem_update(void* const* d_grads, void* const* d_moms, void* const* d_weights,
                               void* const* d_mirrors, const int64_t* sizes, int n_tensors,
                               const float* d_alpha, const float* d_eta, const float* d_norm,
                               float theta, float max_norm, int mode, float* d_stats, void* d_ws,
                               size_t ws_bytes, int dtype, void* stream) {
  if (!d_grads || !d_moms || !d_weights || !sizes || !d_alpha || !d_eta || !d_stats)
    return TMAC_ERR_NULL;
  if (!d_norm && !d_ws) return TMAC_ERR_WORKSPACE;
  if (check_dtype(dtype) != TMAC_OK) return TMAC_ERR_DTYPE;
  if (n_tensors <= 0 || n_tensors > kMaxTensors) return TMAC_ERR_SHAPE;
  if (mode != TMAC_MEM_CLIP_MEMORY && mode != TMAC_MEM_CLIP_KERNEL) return TMAC_ERR_VALUE;
  if (!(max_norm > 0.f) || !isfinite(theta)) return TMAC_ERR_VALUE;
  TensorTable t = {};
  const int pt = per_thread_for(sizes, n_tensors);
  int wg = 0;
  for (int i = 0; i < n_tensors; ++i) {
    if (sizes[i] <= 0) return TMAC_ERR_SHAPE;
    if (!d_grads[i] || !d_moms[i] || !d_weights[i]) return TMAC_ERR_NULL;
    t.g[i] = d_grads[i];
    t.s[i] = d_moms[i];
    t.w[i] = d_weights[i];
    t.c[i] = d_mirrors ? d_mirrors[i] : nullptr;
    t.n[i] = sizes[i];
    t.vec[i] = vec_aligned(t.g[i], dtype) && vec_aligned(t.s[i], dtype) &&
               vec_aligned(t.w[i], dtype) && vec_aligned(t.c[i], dtype);
    t.wg_start[i] = wg;
    wg += static_cast<int>((sizes[i] + 4LL * kThreads * pt - 1) / (4LL * kThreads * pt));
  }
  t.wg_start[n_tensors] = wg;
  t.n_tensors = n_tensors;
  t.per_thread = pt;
  if (!d_norm && ws_bytes < static_cast<size_t>(wg) * 8) return TMAC_ERR_WORKSPACE;
  if (!d_norm && (reinterpret_cast<uintptr_t>(d_ws) & 3u)) return TMAC_ERR_ALIGN;
  auto* part_sq = static_cast<float*>(d_ws);
  auto* part_bad = d_norm ? nullptr : reinterpret_cast<uint32_t*>(part_sq + wg);
  hipStream_t s = static_cast<hipStream_t>(stream);
#define TMAC_MEM_UPDATE(DTV)                                                                    \
  do {                                                                                          \
    if (!d_norm)                                                                                \
      hipLaunchKernelGGL(mem_sumsq_kernel<DTV>, dim3(wg), dim3(kThreads), 0, s, t, part_sq,     \
                         part_bad);                                                             \
    hipLaunchKernelGGL(mem_update_kernel<DTV>, dim3(wg), dim3(kThreads), 0, s, t, part_sq,      \
                       part_bad, wg, d_alpha, d_eta, d_norm, theta, max_norm, mode, d_stats);   \
  } while (0)
  if (dtype == TMAC_F32)
    TMAC_MEM_UPDATE(TMAC_F32);
  else if (dtype == TMAC_BF16)
    TMAC_MEM_UPDATE(TMAC_BF16);
  else
    TMAC_MEM_UPDATE(TMAC_F16);
#undef TMAC_MEM_UPDATE
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? TMAC_OK : static_cast<int>(err);
}

extern "C" int tmac_silu_bwd(const void* d_dh, const void* d_z, void* d_dz, int64_t n, int dtype,
                             void* stream) {
  if (!d_dh || !d_z || !d_dz) return TMAC_ERR_NULL;
  if (check_dtype(dtype) != TMAC_OK) return TMAC_ERR_DTYPE;
  if (n <= 0) return TMAC_ERR_SHAPE;
  const int vec = vec_aligned(d_dh, dtype) && vec_aligned(d_z, dtype) && vec_aligned(d_dz, dtype);
  const unsigned grid = static_cast<unsigned>((n + 4 * kThreads - 1) / (4 * kThreads));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == TMAC_F32)
    hipLaunchKernelGGL(silu_bwd_kernel<TMAC_F32>, dim3(grid), dim3(kThreads), 0, s, d_dh, d_z,
                       d_dz, n, vec);
  else if (dtype == TMAC_BF16)
    hipLaunchKernelGGL(silu_bwd_kernel<TMAC_BF16>, dim3(grid), dim3(kThreads), 0, s, d_dh, d_z,
                       d_dz, n, vec);
  else
    hipLaunchKernelGGL(silu_bwd_kernel<TMAC_F16>, dim3(grid), dim3(kThreads), 0, s, d_dh, d_z,
                       d_dz, n, vec);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? TMAC_OK : static_cast<int>(err);
}

extern "C" int tmac_mse_grad(const void* d_y, const void* d_v, void* d_dy, int64_t n, float coef,
                             int dtype, void* stream) {
  if (!d_y || !d_v || !d_dy) return TMAC_ERR_NULL;
  if (check_dtype(dtype) != TMAC_OK) return TMAC_ERR_DTYPE;
  if (n <= 0) return TMAC_ERR_SHAPE;
  const int vec = vec_aligned(d_y, dtype) && vec_aligned(d_v, dtype) && vec_aligned(d_dy, dtype);
  const unsigned grid = static_cast<unsigned>((n + 4 * kThreads - 1) / (4 * kThreads));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == TMAC_F32)
    hipLaunchKernelGGL(mse_grad_kernel<TMAC_F32>, dim3(grid), dim3(kThreads), 0, s, d_y, d_v,
                       d_dy, n, coef, vec);
  else if (dtype == TMAC_BF16)
    hipLaunchKernelGGL(mse_grad_kernel<TMAC_BF16>, dim3(grid), dim3(kThreads), 0, s, d_y, d_v,
                       d_dy, n, coef, vec);
  else
    hipLaunchKernelGGL(mse_grad_kernel<TMAC_F16>, dim3(grid), dim3(kThreads), 0, s, d_y, d_v,
                       d_dy, n, coef, vec);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? TMAC_OK : static_cast<int>(err);
}
