// Block-ELL block-sparse GEMM kernels for gfx950 (MI355X).
//
//   forward  Y[M, N]  = X[M, K] · W          (tmac_bell_fwd)
//   input    dX[M, K] = dY[M, N] · Wᵀ        (tmac_bell_dx)
//   weight   dW[r, s] = X[:, r]ᵀ · dY[:, c]  on W's non-zero blocks only (tmac_bell_sddmm)
//
// W is Block-ELL with 64x64 blocks, stored row-major inside each block in W's
// own orientation (vals[blk][kk][nn]).
//
// Forward and dX are one gather GEMM. A workgroup (4 waves) owns a 256-row by
// 64-column output tile and walks that tile's list of non-zero blocks:
//   - forward: output block-column c; list = the block-rows holding a block in
//     column c (transposed index, precomputed on the host), reduction over K;
//   - dX: output block-row r; list = row r's own width blocks, reduction over N.
// Each wave owns 64 rows. Per list entry the workgroup loads the 256x64
// activation tile (X or dY) and the 64x64 weight block with coalesced 16-byte
// loads (eight lanes per 128-byte row: a lane-per-row load pattern would cost
// the L1 one tag lookup per lane), stages both in LDS (the activation tile
// XOR-swizzled, the weight block padded) and feeds the MFMAs from there. The
// next entry's tiles are loaded into registers during the current entry's
// math. The weight block is the A operand: read with ds_read_b64_tr_b16 for the
// forward (W is N-contiguous but the reduction runs over K) and with plain
// 16-byte reads for dX (reduction over N).
// The MFMA computes the transposed tile Cᵀ[n][m], so each lane ends up with
// four consecutive output columns per row; the tile is packed through LDS and
// written with full 128-byte row segments.
//
// Workgroups are numbered so each XCD works through whole 256-row slabs of the
// activations (all output block-columns of a slab, longest list first): the
// running workgroups of one XCD then share the slab in that XCD's L2.
//
// SDDMM: a workgroup owns one block-row r, four of its slots (one per wave)
// and a contiguous range of M. Per 64-row step it stages X[m, 64r:+64] and the
// four dY[m, 64c:+64] tiles in LDS and reads both MFMA operands with transpose
// reads (the reduction runs over M, the rows). Partial sums per M-range go to a
// workspace and a second kernel adds them in a fixed order, so the result is
// deterministic.

#include "tmac_device.h"

using namespace tmac;

namespace {

constexpr int kBM = 256;        // output rows per gather-GEMM workgroup (4 waves x 64)
constexpr int kMaxList = 1024;  // longest block list of one output block (checked on the host)

// Activation tile of the gather GEMM in LDS: kBM rows of 64 16-bit values
// (128 bytes) without padding. The 16-byte chunk c of row r sits at chunk
// position c ^ ((r >> 1) & 7): a 16-lane phase of the operand reads (16
// consecutive rows, one chunk each) then covers all 64 banks once, and each
// 8-row group written by one store instruction stays a contiguous 1 KB.
__device__ __forceinline__ int xswz(int row, int chunk) {
  return row * 64 + ((chunk ^ ((row >> 1) & 7)) << 3);
}

template <int DT, bool FWD>
__global__ __launch_bounds__(256, 3) void bell_gemm_kernel(
    const uint16_t* __restrict__ A, int64_t lda, const uint16_t* __restrict__ vals,
    const int32_t* __restrict__ t_ptr, const int32_t* __restrict__ in_blk,
    const int32_t* __restrict__ t_vblk, const int32_t* __restrict__ order,
    const uint16_t* __restrict__ bias, int epi, uint16_t* __restrict__ Y, int64_t ldy, int M,
    int n_out, int width, int n_mtiles, int per_xcd) {
  // Main loop: the activation tile (kBM x 64, swizzled) and the weight tile
  // (64 x kPitch). Epilogue: four per-wave 64x64 staging tiles over the same
  // memory.
  constexpr int kXElems = kBM * 64;
  __shared__ __attribute__((aligned(16))) uint16_t smem[kXElems + kTileElems];
  // The workgroup's list of non-zero blocks, copied once: activation block
  // index and weight block index per entry.
  __shared__ int32_t s_in[kMaxList];
  __shared__ int32_t s_vb[kMaxList];
  uint16_t* const xt = smem;
  uint16_t* const wt = smem + kXElems;

  const int logical = xcd_logical_id(per_xcd);
  if (logical >= n_mtiles * n_out) return;
  const int mtile = logical / n_out;
  const int oi = logical - mtile * n_out;
  const int ob = FWD ? order[oi] : oi;
  const int e0 = FWD ? t_ptr[ob] : ob * width;
  const int e1 = FWD ? t_ptr[ob + 1] : e0 + width;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, h = lane >> 5;
  const int grp = (lane >> 4) & 1;  // which 16-column half of a 32-wide MFMA tile
  const int m_tile0 = mtile * kBM;
  const int m_base = m_tile0 + wave * 64;

  for (int i = tid; i < e1 - e0; i += 256) {
    s_in[i] = in_blk[e0 + i];
    s_vb[i] = FWD ? t_vblk[e0 + i] : e0 + i;
  }

  // Coalesced tile loads: thread t moves 16-byte chunk (t & 7) of rows
  // 32j + (t >> 3), j = 0..7, of the activation tile, and of rows t >> 3 and
  // 32 + (t >> 3) of the weight block. Rows past M are clamped onto row M-1:
  // they load valid memory and their results are never stored.
  const int lrow = tid >> 3, lch = tid & 7;
  const uint16_t* xsrc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
    xsrc[j] = A + static_cast<int64_t>(min(m_tile0 + 32 * j + lrow, M - 1)) * lda + 8 * lch;
  u32x4 xr[8], wr[2];
  auto gload = [&](int i) {
    const int64_t col = static_cast<int64_t>(s_in[i]) * 64;
    const uint16_t* wsrc = vals + static_cast<int64_t>(s_vb[i]) * 4096 + tid * 8;
    wr[0] = ldg16(wsrc);
    wr[1] = ldg16(wsrc + 2048);
#pragma unroll
    for (int j = 0; j < 8; ++j) xr[j] = ldg16(xsrc[j] + col);
  };
  auto sstore = [&]() {
#pragma unroll
    for (int j = 0; j < 8; ++j) sts16(xt + xswz(32 * j + lrow, lch), xr[j]);
    sts16(wt + lrow * kPitch + lch * 8, wr[0]);
    sts16(wt + (32 + lrow) * kPitch + lch * 8, wr[1]);
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = f32x16{};

  // MFMA operands of k-step kk: the wave's activation rows (B operand, 16-byte
  // reads of the swizzled tile) and the weight block (A operand: transpose
  // reads for the forward, where W is N-contiguous but the reduction runs over
  // K; plain 16-byte reads for dX, whose reduction runs over N).
  auto read_ops = [&](u32x4(&xa)[2], u32x4(&wf)[2], int kk) {
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) xa[mi] = lds16(xt + xswz(wave * 64 + 32 * mi + l32, 2 * kk + h));
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) {
      if constexpr (FWD)
        wf[ni] = lds_read_tr8(wt, 16 * kk + 8 * h, 32 * ni + 16 * grp, lane);
      else
        wf[ni] = lds16(wt + (32 * ni + l32) * kPitch + 16 * kk + 8 * h);
    }
  };
  // The reads of k-step kk+1 are issued before the MFMAs of k-step kk, and
  // the scheduling group barriers keep that order.
  auto compute = [&]() {
    u32x4 xa[2][2], wf[2][2];
    read_ops(xa[0], wf[0], 0);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      if (kk + 1 < 4) read_ops(xa[(kk + 1) & 1], wf[(kk + 1) & 1], kk + 1);
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
          acc[mi][ni] = Mfma<DT>::run(wf[kk & 1][ni], xa[kk & 1][mi], acc[mi][ni]);
    }
    constexpr int kDs = FWD ? 6 : 4;  // LDS read instructions per k-step
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * kDs, 0);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
      if (kk + 2 < 4) __builtin_amdgcn_sched_group_barrier(0x100, kDs, 0);
    }
  };

  // One LDS copy of the tiles: entry i+1's tiles are loaded into registers
  // while entry i is computed, then written once every wave is done reading.
  __syncthreads();  // index lists visible
  const int n = e1 - e0;
  if (n > 0) {
    gload(0);
    sstore();
    __syncthreads();
    for (int i = 0; i < n; ++i) {
      const bool more = i + 1 < n;
      if (more) gload(i + 1);
      __builtin_amdgcn_sched_barrier(0);
      compute();
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
      if (more) {
        sstore();
        __syncthreads();
      }
    }
  }

  // Epilogue: bias, activation, conversion, then pack through this wave's LDS
  // staging tile and store 128-byte row segments.
  uint16_t* stage = smem + wave * kTileElems;
  const int64_t col0 = static_cast<int64_t>(ob) * 64;
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
#pragma unroll
      for (int jg = 0; jg < 4; ++jg) {
        const int n_loc = 32 * ni + 8 * jg + 4 * h;
        float v[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] = acc[mi][ni][4 * jg + t];
        if (bias) {
          const u32x2 b2 = *reinterpret_cast<const u32x2*>(bias + col0 + n_loc);
          v[0] += Mfma<DT>::to_f32(static_cast<uint16_t>(b2.x & 0xffff));
          v[1] += Mfma<DT>::to_f32(static_cast<uint16_t>(b2.x >> 16));
          v[2] += Mfma<DT>::to_f32(static_cast<uint16_t>(b2.y & 0xffff));
          v[3] += Mfma<DT>::to_f32(static_cast<uint16_t>(b2.y >> 16));
        }
        if (epi == TMAC_EPI_GELU) {
#pragma unroll
          for (int t = 0; t < 4; ++t) v[t] = gelu_erf(v[t]);
        }
        u32x2 packed;
        packed.x = static_cast<uint32_t>(Mfma<DT>::from_f32(v[0])) |
                   (static_cast<uint32_t>(Mfma<DT>::from_f32(v[1])) << 16);
        packed.y = static_cast<uint32_t>(Mfma<DT>::from_f32(v[2])) |
                   (static_cast<uint32_t>(Mfma<DT>::from_f32(v[3])) << 16);
        *reinterpret_cast<u32x2*>(stage + (32 * mi + l32) * kPitch + n_loc) = packed;
      }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int row = it * 8 + (lane >> 3), ch = lane & 7;
    const int grow = m_base + row;
    if (grow < M) stg16(Y + static_cast<int64_t>(grow) * ldy + col0 + ch * 8, lds16(stage + row * kPitch + ch * 8));
  }
}

template <int DT>
__global__ __launch_bounds__(256, 2) void bell_sddmm_kernel(
    const uint16_t* __restrict__ X, int64_t ldx, const uint16_t* __restrict__ dY, int64_t lddy,
    const int32_t* __restrict__ col_idx, float* __restrict__ part, int M, int n_brow, int width,
    int n_sgroups, int rows_per_split, int n_splits, int per_xcd) {
  // Tile 0: X[m0:m0+64, 64r:64r+64]; tiles 1..4: dY[m0:m0+64, 64c_w:64c_w+64].
  __shared__ __attribute__((aligned(16))) uint16_t smem[5 * kTileElems];

  const int per_split = n_brow * n_sgroups;
  const int logical = xcd_logical_id(per_xcd);
  if (logical >= n_splits * per_split) return;
  const int split = logical / per_split;
  const int rem = logical - split * per_split;
  const int r = rem / n_sgroups;
  const int sg = rem - r * n_sgroups;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, h = lane >> 5;
  const int grp = (lane >> 4) & 1;
  const int s = sg * 4 + wave;
  const bool active = s < width;

  // Block-columns of the four staged dY tiles; slots past the row's width
  // repeat the last valid one (loaded, never used).
  int cblk[4];
#pragma unroll
  for (int w = 0; w < 4; ++w) cblk[w] = col_idx[r * width + min(sg * 4 + w, width - 1)];

  const int m_begin = split * rows_per_split;
  const int m_end = min(M, m_begin + rows_per_split);

  // 5 tiles x 64 rows x 8 chunks of 16 bytes = 10 chunks per thread; chunk
  // p of this thread belongs to tile p/2, row (tid/8) + 32*(p%2), column chunk tid%8.
  u32x4 pre[10];
  auto gload = [&](int m0) {
#pragma unroll
    for (int p = 0; p < 10; ++p) {
      const int t = p >> 1;
      const int row = (tid >> 3) + 32 * (p & 1);
      const int ch = tid & 7;
      const int m = m0 + row;
      if (m < m_end) {
        const uint16_t* src = (t == 0)
                                  ? X + static_cast<int64_t>(m) * ldx + 64 * r + ch * 8
                                  : dY + static_cast<int64_t>(m) * lddy + 64 * cblk[t - 1] + ch * 8;
        pre[p] = ldg16(src);
      } else {
        pre[p] = u32x4{0u, 0u, 0u, 0u};  // rows past the range contribute zero
      }
    }
  };
  auto sstore = [&]() {
#pragma unroll
    for (int p = 0; p < 10; ++p) {
      const int t = p >> 1;
      const int row = (tid >> 3) + 32 * (p & 1);
      sts16(smem + t * kTileElems + row * kPitch + (tid & 7) * 8, pre[p]);
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int ki = 0; ki < 2; ++ki)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) acc[ki][ni] = f32x16{};

  const uint16_t* xt = smem;
  const uint16_t* dyt = smem + (1 + wave) * kTileElems;

  gload(m_begin);
  sstore();
  __syncthreads();
  for (int m0 = m_begin; m0 < m_end; m0 += 64) {
    const bool more = m0 + 64 < m_end;
    if (more) gload(m0 + 64);
    if (active) {
#pragma unroll
      for (int ms = 0; ms < 4; ++ms) {
        u32x4 af[2], bf[2];
#pragma unroll
        for (int ki = 0; ki < 2; ++ki) af[ki] = lds_read_tr8(xt, 16 * ms + 8 * h, 32 * ki + 16 * grp, lane);
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) bf[ni] = lds_read_tr8(dyt, 16 * ms + 8 * h, 32 * ni + 16 * grp, lane);
#pragma unroll
        for (int ki = 0; ki < 2; ++ki)
#pragma unroll
          for (int ni = 0; ni < 2; ++ni) acc[ki][ni] = Mfma<DT>::run(af[ki], bf[ni], acc[ki][ni]);
      }
    }
    __syncthreads();
    if (more) {
      sstore();
      __syncthreads();
    }
  }

  if (!active) return;
  float* dst = part + (static_cast<int64_t>(split) * n_brow * width + r * width + s) * 4096;
#pragma unroll
  for (int ki = 0; ki < 2; ++ki)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int kk = 32 * ki + 8 * (j >> 2) + 4 * h + (j & 3);
        dst[kk * 64 + 32 * ni + l32] = acc[ki][ni][j];
      }
}

// dvals[i] = Σ_split part[split][i], splits added in ascending order.
template <int OUT>
__global__ __launch_bounds__(256) void bell_sddmm_reduce_kernel(const float* __restrict__ part,
                                                                void* __restrict__ out,
                                                                int64_t n_elem, int n_splits) {
  const int64_t i4 = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (i4 >= n_elem) return;
  f32x4 s = *reinterpret_cast<const f32x4*>(part + i4);
  for (int k = 1; k < n_splits; ++k) s += *reinterpret_cast<const f32x4*>(part + k * n_elem + i4);
  if constexpr (OUT == TMAC_F32) {
    *reinterpret_cast<f32x4*>(static_cast<float*>(out) + i4) = s;
  } else {
    u32x2 packed;
    packed.x = static_cast<uint32_t>(Mfma<OUT>::from_f32(s.x)) |
               (static_cast<uint32_t>(Mfma<OUT>::from_f32(s.y)) << 16);
    packed.y = static_cast<uint32_t>(Mfma<OUT>::from_f32(s.z)) |
               (static_cast<uint32_t>(Mfma<OUT>::from_f32(s.w)) << 16);
    *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(out) + i4) = packed;
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_bell_shape(int M, int n_brow, int n_bcol, int width) {
  if (M <= 0 || n_brow <= 0 || n_bcol <= 0 || width <= 0 || width > n_bcol) return TMAC_ERR_SHAPE;
  if (static_cast<int64_t>(n_brow) * width * 4096 > (static_cast<int64_t>(1) << 31)) return TMAC_ERR_SHAPE;
  return TMAC_OK;
}

int launch_status() {
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? TMAC_OK : static_cast<int>(err);
}

// Split of the SDDMM reduction over M: enough workgroups to cover the chip
// about twice, rows per split a multiple of 64.
void sddmm_split(int M, int n_brow, int width, int* n_splits, int* rows_per_split) {
  const int n_sg = (width + 3) / 4;
  const int base = n_brow * n_sg;
  const int m_steps = (M + 63) / 64;
  int want = (512 + base - 1) / base;
  if (want < 1) want = 1;
  if (want > m_steps) want = m_steps;
  const int steps_per = (m_steps + want - 1) / want;
  *rows_per_split = steps_per * 64;
  *n_splits = (M + *rows_per_split - 1) / *rows_per_split;
}

}  // namespace

extern "C" int tmac_bell_fwd(const void* d_X, int64_t ldx, const void* d_vals,
                             const int32_t* d_t_ptr, const int32_t* d_t_row,
                             const int32_t* d_t_vblk, const int32_t* d_order, const void* d_bias,
                             void* d_Y, int64_t ldy, int M, int n_brow, int n_bcol, int width,
                             int dtype, int epi, void* stream) {
  if (!d_X || !d_vals || !d_t_ptr || !d_t_row || !d_t_vblk || !d_order || !d_Y) return TMAC_ERR_NULL;
  int st = check_bell_shape(M, n_brow, n_bcol, width);
  if (st != TMAC_OK) return st;
  if (dtype != TMAC_BF16 && dtype != TMAC_F16) return TMAC_ERR_DTYPE;
  if (epi != TMAC_EPI_NONE && epi != TMAC_EPI_GELU) return TMAC_ERR_VALUE;
  if (n_brow > kMaxList) return TMAC_ERR_SHAPE;  // a column's list has up to n_brow entries
  const int64_t K = 64ll * n_brow, N = 64ll * n_bcol;
  if (ldx < K || ldy < N) return TMAC_ERR_SHAPE;
  if (!aligned16(d_X) || !aligned16(d_vals) || !aligned16(d_Y) || (ldx % 8) || (ldy % 8))
    return TMAC_ERR_ALIGN;
  if (d_bias && !aligned16(d_bias)) return TMAC_ERR_ALIGN;
  const int n_mtiles = (M + kBM - 1) / kBM;
  const int64_t total = static_cast<int64_t>(n_mtiles) * n_bcol;
  if (total > (1ll << 30)) return TMAC_ERR_SHAPE;
  const int per_xcd = static_cast<int>((total + 7) / 8);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const auto* X = static_cast<const uint16_t*>(d_X);
  const auto* V = static_cast<const uint16_t*>(d_vals);
  const auto* b = static_cast<const uint16_t*>(d_bias);
  auto* Y = static_cast<uint16_t*>(d_Y);
  if (dtype == TMAC_BF16)
    hipLaunchKernelGGL((bell_gemm_kernel<TMAC_BF16, true>), dim3(8 * per_xcd), dim3(256), 0, s, X,
                       ldx, V, d_t_ptr, d_t_row, d_t_vblk, d_order, b, epi, Y, ldy, M, n_bcol, width,
                       n_mtiles, per_xcd);
  else
    hipLaunchKernelGGL((bell_gemm_kernel<TMAC_F16, true>), dim3(8 * per_xcd), dim3(256), 0, s, X,
                       ldx, V, d_t_ptr, d_t_row, d_t_vblk, d_order, b, epi, Y, ldy, M, n_bcol, width,
                       n_mtiles, per_xcd);
  return launch_status();
}

extern "C" int tmac_bell_dx(const void* d_dY, int64_t lddy, const void* d_vals,
                            const int32_t* d_col_idx, void* d_dX, int64_t lddx, int M, int n_brow,
                            int n_bcol, int width, int dtype, void* stream) {
  if (!d_dY || !d_vals || !d_col_idx || !d_dX) return TMAC_ERR_NULL;
  int st = check_bell_shape(M, n_brow, n_bcol, width);
  if (st != TMAC_OK) return st;
  if (dtype != TMAC_BF16 && dtype != TMAC_F16) return TMAC_ERR_DTYPE;
  if (width > kMaxList) return TMAC_ERR_SHAPE;
  const int64_t K = 64ll * n_brow, N = 64ll * n_bcol;
  if (lddy < N || lddx < K) return TMAC_ERR_SHAPE;
  if (!aligned16(d_dY) || !aligned16(d_vals) || !aligned16(d_dX) || (lddy % 8) || (lddx % 8))
    return TMAC_ERR_ALIGN;
  const int n_mtiles = (M + kBM - 1) / kBM;
  const int64_t total = static_cast<int64_t>(n_mtiles) * n_brow;
  if (total > (1ll << 30)) return TMAC_ERR_SHAPE;
  const int per_xcd = static_cast<int>((total + 7) / 8);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const auto* dY = static_cast<const uint16_t*>(d_dY);
  const auto* V = static_cast<const uint16_t*>(d_vals);
  auto* dX = static_cast<uint16_t*>(d_dX);
  if (dtype == TMAC_BF16)
    hipLaunchKernelGGL((bell_gemm_kernel<TMAC_BF16, false>), dim3(8 * per_xcd), dim3(256), 0, s,
                       dY, lddy, V, nullptr, d_col_idx, nullptr, nullptr, nullptr, 0, dX, lddx, M,
                       n_brow, width, n_mtiles, per_xcd);
  else
    hipLaunchKernelGGL((bell_gemm_kernel<TMAC_F16, false>), dim3(8 * per_xcd), dim3(256), 0, s,
                       dY, lddy, V, nullptr, d_col_idx, nullptr, nullptr, nullptr, 0, dX, lddx, M,
                       n_brow, width, n_mtiles, per_xcd);
  return launch_status();
}

extern "C" int tmac_bell_sddmm_workspace(int M, int n_brow, int n_bcol, int width,
                                         size_t* ws_bytes) {
  if (!ws_bytes) return TMAC_ERR_NULL;
  int st = check_bell_shape(M, n_brow, n_bcol, width);
  if (st != TMAC_OK) return st;
  int n_splits, rows_per_split;
  sddmm_split(M, n_brow, width, &n_splits, &rows_per_split);
  *ws_bytes = static_cast<size_t>(n_splits) * n_brow * width * 4096 * sizeof(float);
  return TMAC_OK;
}

extern "C" int tmac_bell_sddmm(const void* d_X, int64_t ldx, const void* d_dY, int64_t lddy,
                               const int32_t* d_col_idx, void* d_dvals, int dvals_dtype,
                               void* d_ws, size_t ws_bytes, int M, int n_brow, int n_bcol,
                               int width, int dtype, void* stream) {
  if (!d_X || !d_dY || !d_col_idx || !d_dvals) return TMAC_ERR_NULL;
  int st = check_bell_shape(M, n_brow, n_bcol, width);
  if (st != TMAC_OK) return st;
  if (dtype != TMAC_BF16 && dtype != TMAC_F16) return TMAC_ERR_DTYPE;
  if (dvals_dtype != TMAC_F32 && dvals_dtype != TMAC_BF16 && dvals_dtype != TMAC_F16)
    return TMAC_ERR_DTYPE;
  const int64_t K = 64ll * n_brow, N = 64ll * n_bcol;
  if (ldx < K || lddy < N) return TMAC_ERR_SHAPE;
  if (!aligned16(d_X) || !aligned16(d_dY) || !aligned16(d_dvals) || (ldx % 8) || (lddy % 8))
    return TMAC_ERR_ALIGN;
  int n_splits, rows_per_split;
  sddmm_split(M, n_brow, width, &n_splits, &rows_per_split);
  const size_t need = static_cast<size_t>(n_splits) * n_brow * width * 4096 * sizeof(float);
  if (!d_ws || ws_bytes < need) return TMAC_ERR_WORKSPACE;
  if (!aligned16(d_ws)) return TMAC_ERR_ALIGN;
  const int n_sg = (width + 3) / 4;
  const int64_t total = static_cast<int64_t>(n_splits) * n_brow * n_sg;
  const int per_xcd = static_cast<int>((total + 7) / 8);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const auto* X = static_cast<const uint16_t*>(d_X);
  const auto* dY = static_cast<const uint16_t*>(d_dY);
  float* part = static_cast<float*>(d_ws);
  if (dtype == TMAC_BF16)
    hipLaunchKernelGGL((bell_sddmm_kernel<TMAC_BF16>), dim3(8 * per_xcd), dim3(256), 0, s, X, ldx,
                       dY, lddy, d_col_idx, part, M, n_brow, width, n_sg, rows_per_split, n_splits,
                       per_xcd);
  else
    hipLaunchKernelGGL((bell_sddmm_kernel<TMAC_F16>), dim3(8 * per_xcd), dim3(256), 0, s, X, ldx,
                       dY, lddy, d_col_idx, part, M, n_brow, width, n_sg, rows_per_split, n_splits,
                       per_xcd);
  st = launch_status();
  if (st != TMAC_OK) return st;
  const int64_t n_elem = static_cast<int64_t>(n_brow) * width * 4096;
  const int grid = static_cast<int>((n_elem / 4 + 255) / 256);
  if (dvals_dtype == TMAC_F32)
    hipLaunchKernelGGL((bell_sddmm_reduce_kernel<TMAC_F32>), dim3(grid), dim3(256), 0, s, part,
                       d_dvals, n_elem, n_splits);
  else if (dvals_dtype == TMAC_BF16)
    hipLaunchKernelGGL((bell_sddmm_reduce_kernel<TMAC_BF16>), dim3(grid), dim3(256), 0, s, part,
                       d_dvals, n_elem, n_splits);
  else
    hipLaunchKernelGGL((bell_sddmm_reduce_kernel<TMAC_F16>), dim3(grid), dim3(256), 0, s, part,
                       d_dvals, n_elem, n_splits);
  return launch_status();
}
