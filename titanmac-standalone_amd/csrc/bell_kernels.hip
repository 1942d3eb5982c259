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
// and the weight block XOR-swizzled) and feeds the MFMAs from there. The
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
// With at most 64 rows the forward runs bell_fwd_small_kernel instead: one
// workgroup per block-column whose four waves split the column's list.
//
// SDDMM: a workgroup owns one block-row r, four of its slots (one per wave)
// and a contiguous range of M. Per 32-row step it needs X[m, 64r:+64] and the
// four dY[m, 64c:+64] tiles (20 KB), copied HBM/L2 -> LDS with global_load_lds
// into a four-stage ring three steps ahead of the math (one barrier per step),
// and reads both MFMA operands with transpose reads (the reduction runs over M,
// the rows). Partial sums per M-range go to a workspace and a second kernel
// adds them in a fixed order, so the result is deterministic.

#include "tmac_device.h"

using namespace tmac;

namespace {

constexpr int kBM = 256;        // output rows per gather-GEMM workgroup (4 waves x 64)

// LDS tiles of the gather GEMM, 64 16-bit values (128 bytes) per row without
// padding; 16-byte chunks are XOR-swizzled for the 64 four-byte banks.
//   activation tile (kBM rows): chunk c of row r at c ^ ((r >> 1) & 7), so a
//     16-lane phase of the operand reads (16 consecutive rows, one chunk each)
//     covers all 64 banks once;
//   weight block (64 rows): swz64 (tmac_device.h), conflict-free both for the
//     forward's transpose reads and for dX's 16-byte row reads.
// Every 16-lane phase of the tile stores writes 256 contiguous bytes.
__device__ __forceinline__ int xswz(int row, int chunk) {
  return row * 64 + ((chunk ^ ((row >> 1) & 7)) << 3);
}

// Transpose read of rows r0..r0+7 (r0 a multiple of 8) x 16 columns of a
// swz64 tile: lane (lane % 16) of each 16-lane group receives column
// c0 + lane % 16 of those rows, as one MFMA operand (see lds_read_tr8).
__device__ __forceinline__ u32x4 lds_read_tr8_swz64(const uint16_t* tile, int r0, int c0, int lane) {
  return lds_read_tr4x2_swz64(tile, r0, r0 + 4, c0, lane);
}

typedef __attribute__((address_space(3))) void lds_void;

// 16-byte store marked non-temporal (streamed past the caches' normal
// replacement), for outputs no kernel of the same launch reads again.
__device__ __forceinline__ void stg16_nt(uint16_t* p, u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// Direct HBM/L2 -> LDS copy of 1 KB: lane L of the wave moves the 16 bytes at
// src (its own address) to lds_base + 16 L. lds_base must be wave-uniform.
__device__ __forceinline__ void dma16(const uint16_t* src, uint16_t* lds_base) {
  __builtin_amdgcn_global_load_lds(src, (lds_void*)(lds_base), 16, 0, 0);
}

template <int DT, bool FWD>
__global__ __launch_bounds__(256, 2) void bell_gemm_kernel(
    const uint16_t* __restrict__ A, int64_t lda, const uint16_t* __restrict__ vals,
    const int32_t* __restrict__ t_ptr, const int32_t* __restrict__ in_blk,
    const int32_t* __restrict__ t_vblk, const int32_t* __restrict__ order,
    const uint16_t* __restrict__ bias, int epi, uint16_t* __restrict__ Y, int64_t ldy,
    uint16_t* __restrict__ Z, int64_t ldz, int M, int n_out, int width, int n_mtiles, int per_xcd) {
  // Two buffers, each the activation tile (kBM x 64, xswz) and the weight
  // block (64 x 64, swz64); the epilogue's four per-wave 64x64 staging tiles
  // (pitch kPitch) reuse the same memory.
  // The buffers are separate arrays so the compiler can tell that copies into
  // one do not alias reads of the other (and does not wait for them).
  constexpr int kXElems = kBM * 64;
  constexpr int kBufElems = kXElems + 4096;
  static_assert(kBufElems >= 4 * kTileElems, "staging tiles must fit");
  __shared__ __attribute__((aligned(16))) uint16_t smem0[kBufElems];
  __shared__ __attribute__((aligned(16))) uint16_t smem1[kBufElems];

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

  // Tile copies, eight 1 KB wave instructions for the wave's own 64
  // activation rows and two for rows 16w..16w+15 of the weight block. Lane L
  // of an instruction covering rows R..R+7 fills LDS chunk position L & 7 of
  // row R + L / 8, so it fetches the global chunk that the swizzle stores
  // there; the eight lanes of a row still read its 128 bytes contiguously.
  // Activation rows past M are clamped onto row M-1 (valid memory, results
  // never stored).
  const int drow = lane >> 3, dpos = lane & 7;
  const uint16_t* xsrc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int row = wave * 64 + 8 * j + drow;
    const int chunk = dpos ^ ((row >> 1) & 7);
    xsrc[j] = A + static_cast<int64_t>(min(m_tile0 + row, M - 1)) * lda + 8 * chunk;
  }
  int woff[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int row = wave * 16 + 8 * j + drow;
    const int a = (row >> 1) & 7;
    woff[j] = row * 64 + 8 * (dpos ^ (((a & 1) << 2) | (a >> 1)));
  }
  auto dma_tiles = [&](int blk_in, int blk_w, uint16_t* buf) {
    const int64_t col = static_cast<int64_t>(blk_in) * 64;
#pragma unroll
    for (int j = 0; j < 8; ++j) dma16(xsrc[j] + col, buf + (wave * 64 + 8 * j) * 64);
    const uint16_t* wsrc = vals + static_cast<int64_t>(blk_w) * 4096;
#pragma unroll
    for (int j = 0; j < 2; ++j) dma16(wsrc + woff[j], buf + kXElems + (wave * 16 + 8 * j) * 64);
  };
  // Block indices of the list, 64 entries at a time in a VGPR pair (lane L
  // holds entry base + L) and taken out with readlane: loads issued after the
  // tile copies cannot use the scalar cache, and a vector load there would
  // make the next wait cover the copies too. Indices are fetched right after
  // a barrier, when no copy is in flight, so a window reload (once per 64
  // entries) waits only for itself.
  const int n_list = e1 - e0;
  int win_base = 0, win_in = 0, win_w = 0;
  auto load_window = [&](int base) {
    win_base = base;
    const int i = min(base + lane, n_list - 1);
    win_in = in_blk[e0 + i];
    win_w = FWD ? t_vblk[e0 + i] : e0 + i;
  };
  auto fetch_idx = [&](int i, int& bin, int& bw) {
    if (i - win_base >= 64) load_window(i & ~63);
    bin = __builtin_amdgcn_readlane(win_in, i - win_base);
    bw = __builtin_amdgcn_readlane(win_w, i - win_base);
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
  auto read_ops = [&](u32x4(&xa)[2], u32x4(&wf)[2], const uint16_t* buf, int kk) {
    const uint16_t* wt = buf + kXElems;
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) xa[mi] = lds16(buf + xswz(wave * 64 + 32 * mi + l32, 2 * kk + h));
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) {
      if constexpr (FWD)
        wf[ni] = lds_read_tr8_swz64(wt, 16 * kk + 8 * h, 32 * ni + 16 * grp, lane);
      else
        wf[ni] = lds16(wt + swz64(32 * ni + l32, 2 * kk + h));
    }
  };
  // The reads of k-step kk+1 are issued before the MFMAs of k-step kk, and
  // the scheduling group barriers keep that order.
  auto compute = [&](const uint16_t* buf) {
    u32x4 xa[2][2], wf[2][2];
    read_ops(xa[0], wf[0], buf, 0);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      if (kk + 1 < 4) read_ops(xa[(kk + 1) & 1], wf[(kk + 1) & 1], buf, kk + 1);
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

  // Double-buffered pipeline with one barrier per list entry: the copies of
  // entry i+1 fly into the idle buffer while entry i is computed; the barrier
  // (which waits for this wave's copies) then publishes the new buffer and
  // retires the old one.
  const int n = e1 - e0;
  if (n > 0) {
    int bin, bw;
    load_window(0);
    fetch_idx(0, bin, bw);
    dma_tiles(bin, bw, smem0);
    __syncthreads();
    int i = 0;
    for (; i + 1 < n; i += 2) {
      // entry i from buffer 0 while entry i+1 flies into buffer 1
      fetch_idx(i + 1, bin, bw);
      __builtin_amdgcn_sched_barrier(0);
      dma_tiles(bin, bw, smem1);
      __builtin_amdgcn_sched_barrier(0);
      compute(smem0);
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
      // entry i+1 from buffer 1 while entry i+2 (if any) flies into buffer 0
      if (i + 2 < n) {
        fetch_idx(i + 2, bin, bw);
        __builtin_amdgcn_sched_barrier(0);
        dma_tiles(bin, bw, smem0);
      }
      __builtin_amdgcn_sched_barrier(0);
      compute(smem1);
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
    }
    if (i < n) {
      compute(smem0);
      __syncthreads();
    }
  }

  // Epilogue: bias, activation, conversion, then pack through this wave's LDS
  // staging tile and store 128-byte row segments. With Z (forward only), the
  // pre-activation goes to Z as well, through a second staging tile.
  uint16_t* stage = smem0 + wave * kTileElems;
  uint16_t* stage_z = smem1 + wave * kTileElems;
  const int64_t col0 = static_cast<int64_t>(ob) * 64;
  // the bias values of this lane's 32 columns, all eight loads in flight at once
  u32x2 bb[2][4] = {};
  if (bias) {
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
#pragma unroll
      for (int jg = 0; jg < 4; ++jg)
        bb[ni][jg] = *reinterpret_cast<const u32x2*>(bias + col0 + 32 * ni + 8 * jg + 4 * h);
  }
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
          const u32x2 b2 = bb[ni][jg];
          v[0] += Mfma<DT>::to_f32(static_cast<uint16_t>(b2.x & 0xffff));
          v[1] += Mfma<DT>::to_f32(static_cast<uint16_t>(b2.x >> 16));
          v[2] += Mfma<DT>::to_f32(static_cast<uint16_t>(b2.y & 0xffff));
          v[3] += Mfma<DT>::to_f32(static_cast<uint16_t>(b2.y >> 16));
        }
        if (Z) {
          u32x2 pz;
          pz.x = Mfma<DT>::pack2(v[0], v[1]);
          pz.y = Mfma<DT>::pack2(v[2], v[3]);
          *reinterpret_cast<u32x2*>(stage_z + (32 * mi + l32) * kPitch + n_loc) = pz;
        }
        if (epi == TMAC_EPI_GELU) {
#pragma unroll
          for (int t = 0; t < 4; ++t) v[t] = gelu_erf(v[t]);
        }
        u32x2 packed;
        packed.x = Mfma<DT>::pack2(v[0], v[1]);
        packed.y = Mfma<DT>::pack2(v[2], v[3]);
        *reinterpret_cast<u32x2*>(stage + (32 * mi + l32) * kPitch + n_loc) = packed;
      }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int row = it * 8 + (lane >> 3), ch = lane & 7;
    const int grow = m_base + row;
    if (grow < M) {
      stg16_nt(Y + static_cast<int64_t>(grow) * ldy + col0 + ch * 8, lds16(stage + row * kPitch + ch * 8));
      if (Z) stg16_nt(Z + static_cast<int64_t>(grow) * ldz + col0 + ch * 8, lds16(stage_z + row * kPitch + ch * 8));
    }
  }
}

// Grouped gather GEMM, forward (16-bit). bell_gemm_kernel copies an activation
// tile once per stored weight block, i.e. once for every output block-column
// that uses it, and those L2 -> LDS copies (2.1 GB at config 2) are what bound
// it. Here the output block-columns are grouped in pairs on the host so that the
// two members share many block-rows (tmac_bell_group_schedule), and a workgroup
// walks the union of the pair's lists, ascending by block-row: per union step
// the activation tile is copied once and used by each member holding a block
// there. A member's active steps are its own list in its own order, so each
// output is summed exactly as in bell_gemm_kernel (bitwise-identical results).
//
// Tiles are 512 rows by 2 block-columns, 4R waves per member (R = 1 or 2):
// wave w owns rows (128 / R)(w % 4R) .. +128/R - 1 of member w / 4R (4/R x 2
// MFMA tiles, 32/R MFMAs per step), so every SIMD holds waves of both members
// and gets the same MFMA work per step. R = 2 (16 waves, 128 VGPRs, four per
// SIMD) runs the plain forward: the waves cover each other's LDS and copy
// latency, so operands are read just before their MFMAs; R = 1 (8 waves, two per
// SIMD, operands for k-step kk + 1 read before the MFMAs of kk) runs the bias /
// GELU / Z epilogue, whose registers do not fit 128.
//
// Copies: global_load_lds (1 KB per wave instruction, eight lanes per 128-byte
// row) written as assembly with an SGPR base and per-lane 32-bit offsets fixed
// for the tile, into a two-stage ring (activation tile 64 KB + two weight
// slots 16 KB per stage, all of LDS). Each wave copies 64/R rows of the
// activation tile and, when its member is active, 16/R rows of that member's
// weight block; the next step's copies go out right after the barrier that
// opens a step, and each wave waits for its own copies with an exact vmcnt
// before the next barrier.
//
// Persistent: workgroup b runs on XCD b % 8 and walks that XCD's share of the
// logical tiles (slab-major, longest group first), in the host's balanced
// order (tmac_bell_group_tile_order) when given, else round-robin. After a tile's
// last step it issues the next tile's first copies and only then converts and
// stores the finished tile, staged through the activation stage the next tile
// does not use yet, so the stores drain while the next tile computes.
constexpr int kGM = TMAC_BELL_GROUP_ROWS;  // output rows per grouped tile
static_assert(kGM == 512, "the grouped kernel's waves cover 512 rows");

// s_waitcnt vmcnt(n) for a run-time n in 0..31 (exact); larger n waits for 31.
__device__ __forceinline__ void wait_vm_upto31(int n) {
  switch (n) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(1)" ::: "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(2)" ::: "memory"); break;
    case 3: asm volatile("s_waitcnt vmcnt(3)" ::: "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
    case 5: asm volatile("s_waitcnt vmcnt(5)" ::: "memory"); break;
    case 6: asm volatile("s_waitcnt vmcnt(6)" ::: "memory"); break;
    case 7: asm volatile("s_waitcnt vmcnt(7)" ::: "memory"); break;
    case 8: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
    case 9: asm volatile("s_waitcnt vmcnt(9)" ::: "memory"); break;
    case 10: asm volatile("s_waitcnt vmcnt(10)" ::: "memory"); break;
    case 11: asm volatile("s_waitcnt vmcnt(11)" ::: "memory"); break;
    case 12: asm volatile("s_waitcnt vmcnt(12)" ::: "memory"); break;
    case 13: asm volatile("s_waitcnt vmcnt(13)" ::: "memory"); break;
    case 14: asm volatile("s_waitcnt vmcnt(14)" ::: "memory"); break;
    case 15: asm volatile("s_waitcnt vmcnt(15)" ::: "memory"); break;
    case 16: asm volatile("s_waitcnt vmcnt(16)" ::: "memory"); break;
    case 17: asm volatile("s_waitcnt vmcnt(17)" ::: "memory"); break;
    case 18: asm volatile("s_waitcnt vmcnt(18)" ::: "memory"); break;
    case 19: asm volatile("s_waitcnt vmcnt(19)" ::: "memory"); break;
    case 20: asm volatile("s_waitcnt vmcnt(20)" ::: "memory"); break;
    case 21: asm volatile("s_waitcnt vmcnt(21)" ::: "memory"); break;
    case 22: asm volatile("s_waitcnt vmcnt(22)" ::: "memory"); break;
    case 23: asm volatile("s_waitcnt vmcnt(23)" ::: "memory"); break;
    case 24: asm volatile("s_waitcnt vmcnt(24)" ::: "memory"); break;
    case 25: asm volatile("s_waitcnt vmcnt(25)" ::: "memory"); break;
    case 26: asm volatile("s_waitcnt vmcnt(26)" ::: "memory"); break;
    case 27: asm volatile("s_waitcnt vmcnt(27)" ::: "memory"); break;
    case 28: asm volatile("s_waitcnt vmcnt(28)" ::: "memory"); break;
    case 29: asm volatile("s_waitcnt vmcnt(29)" ::: "memory"); break;
    case 30: asm volatile("s_waitcnt vmcnt(30)" ::: "memory"); break;
    case 31: asm volatile("s_waitcnt vmcnt(31)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(31)" ::: "memory"); break;
  }
}

template <int DT, bool EPI, int R>
__global__ __launch_bounds__(512 * R, 1) void bell_ggemm_kernel(
    const uint16_t* __restrict__ A, int64_t lda, const uint16_t* __restrict__ vals,
    const int32_t* __restrict__ grp_ptr, const int32_t* __restrict__ grp_out,
    const int32_t* __restrict__ steps, const uint16_t* __restrict__ bias, int epi,
    uint16_t* __restrict__ Y, int64_t ldy, uint16_t* __restrict__ Z, int64_t ldz, int M,
    int n_groups, int n_tiles, int per_xcd, const int32_t* __restrict__ order, int n_rounds) {
  constexpr int G = 2;                   // members per group
  constexpr int NQ = 4 * R;              // waves per member, each on kGM / NQ rows
  constexpr int RW = kGM / NQ;           // output rows per wave (128 or 64)
  constexpr int MI = RW / 32;            // 32-row MFMA tiles per wave
  constexpr int XI = 8 / R;              // 8-row activation copies per wave and step
  constexpr int WI = 2 / R;              // 8-row weight copies per wave and step
  constexpr int kX = kGM * 64;           // activation tile, 16-bit elements (64 KB)
  constexpr int kW = G * 4096;           // weight slots of a stage (16 KB)
  constexpr int kRec = 1 + G;            // step record: block-row, G value blocks (-1: none)
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * kX + 2 * kW];

  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3, n_slots = gridDim.x >> 3;
  const int t_end = min(n_tiles, (xcd + 1) * per_xcd);
  // This slot's tiles, round by round: the host's balanced order (entry (xcd *
  // n_rounds + round) * n_slots + slot; -1 or out of range: none that round), or
  // tiles xcd * per_xcd + slot + round * n_slots of the XCD's range.
  auto tile_of = [&](int r) {
    if (order) {
      const int t = order[(xcd * n_rounds + r) * n_slots + slot];
      return t >= 0 && t < n_tiles ? t : -1;
    }
    const int t = xcd * per_xcd + slot + r * n_slots;
    return t < t_end ? t : -1;
  };
  auto next_tile = [&](int& r) {  // first tile at round >= r (r advanced to it), or -1
    for (; r < n_rounds; ++r) {
      const int t = tile_of(r);
      if (t >= 0) return t;
    }
    return -1;
  };
  int rnd = 0;
  int t = next_tile(rnd);
  if (t < 0) return;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int q = wave % NQ, mem = wave / NQ;
  const int l32 = lane & 31, h = lane >> 5;
  const int grp = (lane >> 4) & 1;  // which 16-column half of a 32-wide MFMA tile
  const int drow = lane >> 3, dpos = lane & 7;
  // Per-lane copy offsets (bytes). Lane L of an instruction covering rows
  // R..R+7 fills LDS chunk position L & 7 of row R + L / 8 and fetches the
  // global chunk that the swizzle stores there.
  uint32_t woff[WI];
#pragma unroll
  for (int j = 0; j < WI; ++j) {
    const int row = 8 * WI * q + 8 * j + drow;
    const int a = (row >> 1) & 7;
    woff[j] = static_cast<uint32_t>(row * 128 + 16 * (dpos ^ (((a & 1) << 2) | (a >> 1))));
  }
  const uint32_t lds0 = lds_offset(smem);

  // the current tile
  int mtile = t / n_groups, gi = t - (t / n_groups) * n_groups;
  int n_steps = grp_ptr[gi + 1] - grp_ptr[gi];
  const int32_t* rec0 = steps + static_cast<int64_t>(grp_ptr[gi]) * kRec;
  int m_tile0 = mtile * kGM;
  // activation rows past M read row M-1 (valid memory, results never stored)
  uint32_t xoff[XI];
  auto set_xoff = [&]() {
    const int last = M - 1 - m_tile0;
#pragma unroll
    for (int j = 0; j < XI; ++j) {
      const int row = 8 * XI * wave + 8 * j + drow;
      const int chunk = dpos ^ ((row >> 1) & 7);
      xoff[j] = static_cast<uint32_t>(min(row, last)) * static_cast<uint32_t>(2 * lda) +
                16u * static_cast<uint32_t>(chunk);
    }
  };
  set_xoff();

  // Step records of the current tile in VGPRs, 64 steps per window (lane L
  // holds step 64k + L), read with readlane: no memory access on the per-step
  // path. Two windows are resident, since the look-ahead crosses into the next.
  int win_in0 = 0, win_in1 = 0, win_vb0 = -1, win_vb1 = -1;
  auto load_window = [&](int k) {
    const int j = min(64 * k + lane, n_steps - 1);
    const int a = rec0[j * kRec], b = rec0[j * kRec + 1 + mem];
    if (k & 1) {
      win_in1 = a;
      win_vb1 = b;
    } else {
      win_in0 = a;
      win_vb0 = b;
    }
  };
  auto step_in = [&](int i) {
    return __builtin_amdgcn_readlane((i & 64) ? win_in1 : win_in0, i & 63);
  };
  // this wave's member's value block at step i (-1: the member has none there)
  auto own_vb = [&](int i) {
    return __builtin_amdgcn_readlane((i & 64) ? win_vb1 : win_vb0, i & 63);
  };
  // copies of step i of the current tile into ring stage gs & 1
  auto issue = [&](int i, int gs) {
    const uint32_t sx = lds0 + static_cast<uint32_t>((gs & 1) * kX * 2);
    const uint16_t* xb = A + static_cast<int64_t>(m_tile0) * lda + static_cast<int64_t>(step_in(i)) * 64;
#pragma unroll
    for (int j = 0; j < XI; ++j) dma_lds16(xb, xoff[j], sx + (8 * XI * wave + 8 * j) * 128);
    const int vb = own_vb(i);
    if (vb >= 0) {
      const uint32_t sw = lds0 + static_cast<uint32_t>((2 * kX + (gs & 1) * kW + mem * 4096) * 2);
      const uint16_t* wb = vals + static_cast<int64_t>(vb) * 4096;
#pragma unroll
      for (int j = 0; j < WI; ++j) dma_lds16(wb, woff[j], sw + (8 * WI * q + 8 * j) * 128);
    }
  };

  f32x16 acc[MI][2];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = f32x16{};
  // MFMA operands of k-step kk: the wave's activation rows (B operand, 16-byte
  // reads of the swizzled tile) and its member's weight block (A operand,
  // transpose reads: W is N-contiguous but the reduction runs over K).
  auto read_ops = [&](u32x4(&xa)[MI], u32x4(&wf)[2], const uint16_t* xt, const uint16_t* wt, int kk) {
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) xa[mi] = lds16(xt + xswz(RW * q + 32 * mi + l32, 2 * kk + h));
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) wf[ni] = lds_read_tr8_swz64(wt, 16 * kk + 8 * h, 32 * ni + 16 * grp, lane);
  };
  // operand reads of k-step kk + 1 are issued before the MFMAs of k-step kk
  auto compute = [&](const uint16_t* xt, const uint16_t* wt) {
    if constexpr (R == 1) {
      u32x4 xa[2][MI], wf[2][2];
      read_ops(xa[0], wf[0], xt, wt, 0);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        if (kk + 1 < 4) read_ops(xa[(kk + 1) & 1], wf[(kk + 1) & 1], xt, wt, kk + 1);
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
#pragma unroll
          for (int ni = 0; ni < 2; ++ni)
            acc[mi][ni] = Mfma<DT>::run(wf[kk & 1][ni], xa[kk & 1][mi], acc[mi][ni]);
      }
    } else {
      // four waves per SIMD cover each other's LDS latency: no operand double buffer
      u32x4 xa[MI], wf[2];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        read_ops(xa, wf, xt, wt, kk);
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
#pragma unroll
          for (int ni = 0; ni < 2; ++ni)
            acc[mi][ni] = Mfma<DT>::run(wf[ni], xa[mi], acc[mi][ni]);
      }
    }
  };

  int gs = 0;       // steps this workgroup has walked (ring parity)
  int pending = 0;  // this wave's stores issued after the current tile's first copies
  if (n_steps > 0) {
    load_window(0);
    if (n_steps > 64) load_window(1);
    issue(0, 0);
  }
  for (;;) {
    for (int i = 0; i < n_steps; ++i) {
      // entering window k >= 1: fetch window k + 1 into the slot of window k - 1
      if ((i & 63) == 0 && i > 0 && i + 64 < n_steps) load_window((i >> 6) + 1);
      // This wave's copies of step i have landed once at most the previous
      // tile's stores (step 0 only) are outstanding behind them: copies and
      // stores complete in issue order.
      wait_vm_upto31(i == 0 ? pending : 0);
      // every wave's copies of step i are in LDS, and every wave is done with
      // step i - 1, whose stage the next copies overwrite
      asm volatile("s_barrier" ::: "memory");
      if (i + 1 < n_steps) issue(i + 1, gs + i + 1);
      if (own_vb(i) >= 0) compute(smem + ((gs + i) & 1) * kX, smem + 2 * kX + ((gs + i) & 1) * kW + mem * 4096);
    }
    gs += n_steps;
    const int ob = grp_out[gi * G + mem];
    const int m_out = m_tile0 + RW * q;
    const int64_t col0 = static_cast<int64_t>(ob) * 64;
    // The bias of this lane's 32 columns, loaded and waited for before the
    // next tile's copies are issued, so that no wait on it covers them.
    u32x2 bb[2][4] = {};
    if (EPI && bias && ob >= 0) {
#pragma unroll
      for (int ni = 0; ni < 2; ++ni)
#pragma unroll
        for (int jg = 0; jg < 4; ++jg)
          bb[ni][jg] = *reinterpret_cast<const u32x2*>(bias + col0 + 32 * ni + 8 * jg + 4 * h);
      asm volatile("" ::"v"(bb[0][0]), "v"(bb[0][1]), "v"(bb[0][2]), "v"(bb[0][3]), "v"(bb[1][0]),
                   "v"(bb[1][1]), "v"(bb[1][2]), "v"(bb[1][3]));
    }
    // every wave is done with the ring before the next tile's copies go in
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    asm volatile("s_barrier" ::: "memory");
    ++rnd;
    const int t_next = next_tile(rnd);
    const bool more = t_next >= 0;
    if (more) {
      t = t_next;
      mtile = t / n_groups;
      gi = t - mtile * n_groups;
      n_steps = grp_ptr[gi + 1] - grp_ptr[gi];
      rec0 = steps + static_cast<int64_t>(grp_ptr[gi]) * kRec;
      m_tile0 = mtile * kGM;
      set_xoff();
      if (n_steps > 0) {
        load_window(0);
        if (n_steps > 64) load_window(1);
        issue(0, gs);
      }
    }
    // Epilogue of the finished tile (block-column ob, rows m_out..m_out+127),
    // one 32-row MFMA tile at a time: bias and activation in place, conversion,
    // then through this wave's 4 KB of staging (32 rows x 64, chunks
    // XOR-swizzled by row) in the activation stage the next tile's first step
    // does not use, and out as 128-byte row segments. A store instruction is
    // issued (and counted) only when some of its rows are in range.
    uint16_t* stage = smem + ((gs + 1) & 1) * kX + wave * 2048;
    int n_st = 0;
    if (ob >= 0) {
      // The staging offsets below depend on the lane only; formed from these
      // copies (the empty asm hides that they are loop-invariant), they are
      // computed here per tile instead of being held in registers, or spilled,
      // across the step loop.
      int el = lane;
      asm volatile("" : "+v"(el));
      const int el32 = el & 31, eh = el >> 5;
      auto stage_store = [&](const f32x16(&v)[2], int mi, uint16_t* out, int64_t ld) {
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
          for (int jg = 0; jg < 4; ++jg) {
            u32x2 packed;
            packed.x = Mfma<DT>::pack2(v[ni][4 * jg], v[ni][4 * jg + 1]);
            packed.y = Mfma<DT>::pack2(v[ni][4 * jg + 2], v[ni][4 * jg + 3]);
            const int chunk = 4 * ni + jg;
            *reinterpret_cast<u32x2*>(stage + el32 * 64 + ((chunk ^ (el32 & 7)) << 3) + 4 * eh) = packed;
          }
#pragma unroll
        for (int it = 0; it < 4; ++it) {
          const int base = m_out + 32 * mi + 8 * it;
          if (base < M) {
            const int row = 8 * it + (el >> 3), ch = el & 7;
            const u32x4 v4 = lds16(stage + row * 64 + ((ch ^ (row & 7)) << 3));
            if (base + (lane >> 3) < M)
              stg16_nt(out + static_cast<int64_t>(base + (lane >> 3)) * ld + col0 + ch * 8, v4);
            n_st += 1;
          }
        }
      };
#pragma unroll
      for (int mi = 0; mi < MI; ++mi) {
        if (EPI && bias) {
#pragma unroll
          for (int ni = 0; ni < 2; ++ni)
#pragma unroll
            for (int jg = 0; jg < 4; ++jg) {
              const u32x2 b2 = bb[ni][jg];
              acc[mi][ni][4 * jg] += Mfma<DT>::to_f32(static_cast<uint16_t>(b2.x & 0xffff));
              acc[mi][ni][4 * jg + 1] += Mfma<DT>::to_f32(static_cast<uint16_t>(b2.x >> 16));
              acc[mi][ni][4 * jg + 2] += Mfma<DT>::to_f32(static_cast<uint16_t>(b2.y & 0xffff));
              acc[mi][ni][4 * jg + 3] += Mfma<DT>::to_f32(static_cast<uint16_t>(b2.y >> 16));
            }
        }
        if (EPI && Z) stage_store(acc[mi], mi, Z, ldz);
        if (EPI && epi == TMAC_EPI_GELU) {
#pragma unroll
          for (int ni = 0; ni < 2; ++ni)
#pragma unroll
            for (int j = 0; j < 16; ++j) acc[mi][ni][j] = gelu_erf(acc[mi][ni][j]);
        }
        stage_store(acc[mi], mi, Y, ldy);
      }
    }
    if (!more) break;
    pending = n_st;
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = f32x16{};
  }
}

// Forward for few rows (M <= kSmallM: decoding, small batches). The gather GEMM
// above gives such a call one 256-row tile per block-column and walks each list
// one entry at a time, so it pays one memory latency per entry whatever M is.
// Here one workgroup owns block-column c (all M <= 64 rows) and its four waves
// split c's list: wave w takes entries w, w + 4, ..., each wave with two LDS
// stages of its own (64-row activation tile + weight block, both swizzled as
// above), so up to eight entries' copies are in flight per workgroup and the
// waves never wait for each other. Each wave accumulates a full 64x64 partial
// tile; the partials are added through LDS in wave order (deterministic), and
// wave 0 runs the epilogue. Activation rows past M are clamped onto row M-1.
constexpr int kSmallM = 64;

template <int DT>
__global__ __launch_bounds__(256) void bell_fwd_small_kernel(
    const uint16_t* __restrict__ A, int64_t lda, const uint16_t* __restrict__ vals,
    const int32_t* __restrict__ t_ptr, const int32_t* __restrict__ t_row,
    const int32_t* __restrict__ t_vblk, const uint16_t* __restrict__ bias, int epi,
    uint16_t* __restrict__ Y, int64_t ldy, uint16_t* __restrict__ Z, int64_t ldz, int M) {
  // Per wave and stage: activation tile (64 x 64, xswz) then weight block
  // (64 x 64, swz64). Separate arrays per stage, so the compiler can tell the
  // copies into one stage from the reads of the other.
  __shared__ __attribute__((aligned(16))) uint16_t st0[4][8192];
  __shared__ __attribute__((aligned(16))) uint16_t st1[4][8192];

  const int ob = blockIdx.x;
  const int e0 = t_ptr[ob], e1 = t_ptr[ob + 1];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int l32 = lane & 31, h = lane >> 5;
  const int grp = (lane >> 4) & 1;
  const int drow = lane >> 3, dpos = lane & 7;

  // Copy addressing as in bell_gemm_kernel: lane L of the instruction for rows
  // 8j..8j+7 fills chunk position L & 7 of row 8j + L / 8.
  const uint16_t* xsrc[8];
  int woff[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int row = 8 * j + drow;
    const int a = (row >> 1) & 7;
    xsrc[j] = A + static_cast<int64_t>(min(row, M - 1)) * lda + 8 * (dpos ^ a);
    woff[j] = row * 64 + 8 * (dpos ^ (((a & 1) << 2) | (a >> 1)));
  }
  auto dma_tiles = [&](int e, uint16_t* buf) {
    const int64_t col = static_cast<int64_t>(t_row[e]) * 64;
    const uint16_t* wsrc = vals + static_cast<int64_t>(t_vblk[e]) * 4096;
#pragma unroll
    for (int j = 0; j < 8; ++j) dma16(xsrc[j] + col, buf + 8 * j * 64);
#pragma unroll
    for (int j = 0; j < 8; ++j) dma16(wsrc + woff[j], buf + 4096 + 8 * j * 64);
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = f32x16{};
  auto compute = [&](const uint16_t* buf) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      u32x4 xa[2], wf[2];
#pragma unroll
      for (int mi = 0; mi < 2; ++mi) xa[mi] = lds16(buf + xswz(32 * mi + l32, 2 * kk + h));
#pragma unroll
      for (int ni = 0; ni < 2; ++ni) wf[ni] = lds_read_tr8_swz64(buf + 4096, 16 * kk + 8 * h, 32 * ni + 16 * grp, lane);
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = Mfma<DT>::run(wf[ni], xa[mi], acc[mi][ni]);
    }
  };

  // This wave's entries e0 + wave + 4i, two at a time: both copies are issued
  // before either is computed.
  uint16_t* b0 = st0[wave];
  uint16_t* b1 = st1[wave];
  for (int e = e0 + wave; e < e1; e += 8) {
    const bool two = e + 4 < e1;
    dma_tiles(e, b0);
    if (two) dma_tiles(e + 4, b1);
    __builtin_amdgcn_sched_barrier(0);
    compute(b0);
    if (two) compute(b1);
    __builtin_amdgcn_sched_barrier(0);
  }

  // Partial tiles of waves 1..3 through LDS (fp32, lane-major: conflict-free),
  // added to wave 0's in wave order.
  __syncthreads();
  float* red = reinterpret_cast<float*>(&st0[0][0]);  // 3 x 64 x 64 floats = 48 KB
  if (wave > 0) {
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
      for (int ni = 0; ni < 2; ++ni)
#pragma unroll
        for (int j = 0; j < 16; ++j)
          red[((wave - 1) * 64 + (mi * 2 + ni) * 16 + j) * 64 + lane] = acc[mi][ni][j];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < 3; ++w)
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
      for (int ni = 0; ni < 2; ++ni)
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[mi][ni][j] += red[(w * 64 + (mi * 2 + ni) * 16 + j) * 64 + lane];

  // Epilogue as in bell_gemm_kernel, for wave 0's 64 rows (staging tiles in
  // stage-1 memory, which no wave touches any more).
  uint16_t* stage = &st1[0][0];
  uint16_t* stage_z = &st1[1][0];
  const int64_t col0 = static_cast<int64_t>(ob) * 64;
  // the bias values of this lane's 32 columns, all eight loads in flight at once
  u32x2 bb[2][4] = {};
  if (bias) {
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
#pragma unroll
      for (int jg = 0; jg < 4; ++jg)
        bb[ni][jg] = *reinterpret_cast<const u32x2*>(bias + col0 + 32 * ni + 8 * jg + 4 * h);
  }
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
          const u32x2 b2 = bb[ni][jg];
          v[0] += Mfma<DT>::to_f32(static_cast<uint16_t>(b2.x & 0xffff));
          v[1] += Mfma<DT>::to_f32(static_cast<uint16_t>(b2.x >> 16));
          v[2] += Mfma<DT>::to_f32(static_cast<uint16_t>(b2.y & 0xffff));
          v[3] += Mfma<DT>::to_f32(static_cast<uint16_t>(b2.y >> 16));
        }
        if (Z) {
          u32x2 pz;
          pz.x = Mfma<DT>::pack2(v[0], v[1]);
          pz.y = Mfma<DT>::pack2(v[2], v[3]);
          *reinterpret_cast<u32x2*>(stage_z + (32 * mi + l32) * kPitch + n_loc) = pz;
        }
        if (epi == TMAC_EPI_GELU) {
#pragma unroll
          for (int t = 0; t < 4; ++t) v[t] = gelu_erf(v[t]);
        }
        u32x2 packed;
        packed.x = Mfma<DT>::pack2(v[0], v[1]);
        packed.y = Mfma<DT>::pack2(v[2], v[3]);
        *reinterpret_cast<u32x2*>(stage + (32 * mi + l32) * kPitch + n_loc) = packed;
      }
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int row = it * 8 + (lane >> 3), ch = lane & 7;
    if (row < M) {
      stg16(Y + static_cast<int64_t>(row) * ldy + col0 + ch * 8, lds16(stage + row * kPitch + ch * 8));
      if (Z) stg16(Z + static_cast<int64_t>(row) * ldz + col0 + ch * 8, lds16(stage_z + row * kPitch + ch * 8));
    }
  }
}

// s_waitcnt vmcnt(n) for n in {0, 5, 10}; the other counters are left alone.
__device__ __forceinline__ void wait_vm(int n) {
  if (n >= 10)
    asm volatile("s_waitcnt vmcnt(10)" ::: "memory");
  else if (n >= 5)
    asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
  else
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

constexpr int kSdRows = 32;            // M rows per SDDMM step
constexpr int kSdStages = 4;           // LDS ring depth (three steps of copies in flight)
constexpr int kSdTile = kSdRows * 64;  // one 32x64 tile, 16-bit elements
constexpr int kSdStage = 5 * kSdTile;  // X tile + four dY tiles (20 KB)

template <int DT>
__global__ __launch_bounds__(256, 2) void bell_sddmm_kernel(
    const uint16_t* __restrict__ X, int64_t ldx, const uint16_t* __restrict__ dY, int64_t lddy,
    const int32_t* __restrict__ col_idx, float* __restrict__ part, int M, int n_brow, int width,
    int n_sgroups, int rows_per_split, int n_splits, int per_xcd) {
  // Ring of four stages; stage = X[m:m+32, 64r:+64] then dY[m:m+32, 64c_w:+64]
  // for w = 0..3, each tile 32 rows of 64 elements, chunks swizzled as swz64.
  __shared__ __attribute__((aligned(16))) uint16_t ring[kSdStages * kSdStage];

  const int per_split = n_brow * n_sgroups;
  const int logical = xcd_logical_id(per_xcd);
  if (logical >= n_splits * per_split) return;
  const int split = logical / per_split;
  const int rem = logical - split * per_split;
  const int r = rem / n_sgroups;
  const int sg = rem - r * n_sgroups;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int h = lane >> 5, grp = (lane >> 4) & 1, l32 = lane & 31;
  const int s = sg * 4 + wave;
  const bool active = s < width;
  // this wave's block-column; a slot past the row's width repeats the last one
  // (copied, never used)
  const int cw = col_idx[r * width + min(s, width - 1)];

  const int m_begin = split * rows_per_split;
  const int m_end = min(M, m_begin + rows_per_split);
  const int n_steps = (m_end - m_begin + kSdRows - 1) / kSdRows;

  // Copies per step and wave: its own dY tile (four 8-row instructions) and
  // rows 8w..8w+7 of the X tile. Lane L of an instruction covering rows
  // R..R+7 fills chunk position L & 7 of row R + L / 8 and fetches the global
  // chunk the swizzle stores there; the eight lanes of a row read 128
  // contiguous bytes. A lane's byte offsets from the step's first row are the
  // same for every step; rows past M (last step of the matrix only) read row
  // M-1, valid memory, and are zeroed in LDS once the copies have landed.
  const int drow = lane >> 3, dpos = lane & 7;
  auto swz_chunk = [](int row, int pos) {
    const int a = (row >> 1) & 7;
    return pos ^ (((a & 1) << 2) | (a >> 1));
  };
  const int xrow = 8 * wave + drow;
  const uint32_t xcol = 2u * (64 * r + 8 * swz_chunk(xrow, dpos));
  uint32_t ycol[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) ycol[j] = 2u * (64 * cw + 8 * swz_chunk(8 * j + drow, dpos));
  const uint32_t ring0 = lds_offset(ring);
  auto issue = [&](int step) {
    const int m0 = m_begin + step * kSdRows;
    const uint32_t st = ring0 + static_cast<uint32_t>((step % kSdStages) * kSdStage * 2);
    const uint16_t* xb = X + static_cast<int64_t>(m0) * ldx;
    const uint16_t* yb = dY + static_cast<int64_t>(m0) * lddy;
    const int lim = M - 1 - m0;  // rows beyond this one read it instead
    dma_lds16(xb, static_cast<uint32_t>(min(xrow, lim)) * static_cast<uint32_t>(2 * ldx) + xcol,
                 st + 8 * wave * 128);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      dma_lds16(yb, static_cast<uint32_t>(min(8 * j + drow, lim)) * static_cast<uint32_t>(2 * lddy) + ycol[j],
                   st + (1 + wave) * kSdTile * 2 + 8 * j * 128);
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int ki = 0; ki < 2; ++ki)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) acc[ki][ni] = f32x16{};

  for (int i = 0; i < kSdStages - 1 && i < n_steps; ++i) issue(i);
  for (int i = 0; i < n_steps; ++i) {
    // this wave's copies of step i have landed when at most those of the
    // (up to kSdStages - 2) later steps already issued are outstanding
    wait_vm(5 * min(kSdStages - 2, n_steps - 1 - i));
    const int m0 = m_begin + i * kSdRows;
    uint16_t* st = ring + (i % kSdStages) * kSdStage;
    if (m0 + kSdRows > m_end) {
      // rows past the range contribute zero: each wave clears the rows it copied
      const int valid = m_end - m0;
      if (xrow >= valid) sts16(st + xrow * 64 + 8 * dpos, u32x4{0u, 0u, 0u, 0u});
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (8 * j + drow >= valid)
          sts16(st + (1 + wave) * kSdTile + (8 * j + drow) * 64 + 8 * dpos, u32x4{0u, 0u, 0u, 0u});
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    // every wave's copies of step i are in LDS, and every wave is done reading
    // the stage the next copies overwrite (step i-1's)
    asm volatile("s_barrier" ::: "memory");
    if (i + kSdStages - 1 < n_steps) issue(i + kSdStages - 1);
    if (active) {
      const uint16_t* xt = st;
      const uint16_t* dyt = st + (1 + wave) * kSdTile;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        u32x4 af[2], bf[2];
#pragma unroll
        for (int ki = 0; ki < 2; ++ki) af[ki] = lds_read_tr8_swz64(xt, 16 * ks + 8 * h, 32 * ki + 16 * grp, lane);
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) bf[ni] = lds_read_tr8_swz64(dyt, 16 * ks + 8 * h, 32 * ni + 16 * grp, lane);
#pragma unroll
        for (int ki = 0; ki < 2; ++ki)
#pragma unroll
          for (int ni = 0; ni < 2; ++ni) acc[ki][ni] = Mfma<DT>::run(af[ki], bf[ni], acc[ki][ni]);
      }
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

// ---------------------------------------------------------------------------
// fp32 path (fp32 modules without autocast): the same three products on
// v_mfma_f32_32x32x2_f32, fp32 products and fp32 accumulation.
//
// Gather GEMM (forward and dX): a workgroup owns a 128-row by 64-column output
// tile and walks the same list as the 16-bit kernel. Per list entry it stages
// the 128x64 activation tile (row-major) and the weight block as Bᵀ ([n][k]:
// transposed while staging for the forward, as stored for dX) in LDS, rows
// padded to 68 floats so the 16-byte reads of 16 consecutive rows hit all 64
// banks once; the next entry's tiles are prefetched into registers during the
// current entry's math. Wave w computes output rows 32w..32w+31 against both
// 32-column halves. An MFMA step sums k = 4u + q (lanes 0-31) and 32 + 4u + q
// (lanes 32-63), so each lane's operands for four steps are one 16-byte read
// of its own row.
constexpr int kBMf = 128;  // output rows per fp32 workgroup (4 waves x 32)
constexpr int kPf = 68;    // LDS row pitch of the fp32 tiles, floats

__device__ __forceinline__ f32x16 mfma_f32(float a, float b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

template <bool FWD>
__global__ __launch_bounds__(256, 2) void bell_gemm_f32_kernel(
    const float* __restrict__ A, int64_t lda, const float* __restrict__ vals,
    const int32_t* __restrict__ t_ptr, const int32_t* __restrict__ in_blk,
    const int32_t* __restrict__ t_vblk, const int32_t* __restrict__ order,
    const float* __restrict__ bias, int epi, float* __restrict__ Y, int64_t ldy,
    float* __restrict__ Z, int64_t ldz, int M, int n_out, int width, int n_mtiles, int per_xcd) {
  __shared__ __attribute__((aligned(16))) float xs[kBMf * kPf];  // activation tile [m][k]
  __shared__ __attribute__((aligned(16))) float ws[64 * kPf];    // weight block as Bᵀ [n][k]

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
  const int m0 = mtile * kBMf;

  // Staging: activation rows 16p + tid/16 (p = 0..7), 16-byte chunk tid % 16 (16
  // threads per 256-byte row); weight block: dX rows 16p + tid/16 as they are,
  // forward rows kk = tid % 64 with chunk tid/64 + 4p, written transposed.
  const int srow = tid >> 4, schunk = tid & 15;
  int64_t xoff[8];
#pragma unroll
  for (int p = 0; p < 8; ++p)
    xoff[p] = static_cast<int64_t>(min(m0 + 16 * p + srow, M - 1)) * lda + 4 * schunk;
  f32x4 px[8], pw[4];
  auto gload = [&](int e) __attribute__((always_inline)) {
    const float* xb = A + static_cast<int64_t>(in_blk[e]) * 64;
    const float* wb = vals + static_cast<int64_t>(FWD ? t_vblk[e] : e) * 4096;
#pragma unroll
    for (int p = 0; p < 8; ++p) px[p] = *reinterpret_cast<const f32x4*>(xb + xoff[p]);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      if constexpr (FWD)
        pw[p] = *reinterpret_cast<const f32x4*>(wb + (tid & 63) * 64 + 4 * ((tid >> 6) + 4 * p));
      else
        pw[p] = *reinterpret_cast<const f32x4*>(wb + (16 * p + srow) * 64 + 4 * schunk);
    }
  };
  auto sstore = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int p = 0; p < 8; ++p)
      *reinterpret_cast<f32x4*>(xs + (16 * p + srow) * kPf + 4 * schunk) = px[p];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      if constexpr (FWD) {
        const int kk = tid & 63, n0 = 4 * ((tid >> 6) + 4 * p);
        ws[(n0 + 0) * kPf + kk] = pw[p].x;
        ws[(n0 + 1) * kPf + kk] = pw[p].y;
        ws[(n0 + 2) * kPf + kk] = pw[p].z;
        ws[(n0 + 3) * kPf + kk] = pw[p].w;
      } else {
        *reinterpret_cast<f32x4*>(ws + (16 * p + srow) * kPf + 4 * schunk) = pw[p];
      }
    }
  };

  f32x16 acc[2];
  acc[0] = f32x16{};
  acc[1] = f32x16{};
  if (e0 < e1) gload(e0);
  const float* xa = xs + (32 * wave + l32) * kPf + 32 * h;
  const float* wa0 = ws + l32 * kPf + 32 * h;
  const float* wa1 = ws + (32 + l32) * kPf + 32 * h;
  for (int e = e0; e < e1; ++e) {
    __syncthreads();  // the previous entry's reads of xs / ws are done
    sstore();
    __syncthreads();
    if (e + 1 < e1) gload(e + 1);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(xa + 4 * u);
      const f32x4 b0 = *reinterpret_cast<const f32x4*>(wa0 + 4 * u);
      const f32x4 b1 = *reinterpret_cast<const f32x4*>(wa1 + 4 * u);
      acc[0] = mfma_f32(a.x, b0.x, acc[0]);
      acc[1] = mfma_f32(a.x, b1.x, acc[1]);
      acc[0] = mfma_f32(a.y, b0.y, acc[0]);
      acc[1] = mfma_f32(a.y, b1.y, acc[1]);
      acc[0] = mfma_f32(a.z, b0.z, acc[0]);
      acc[1] = mfma_f32(a.z, b1.z, acc[1]);
      acc[0] = mfma_f32(a.w, b0.w, acc[0]);
      acc[1] = mfma_f32(a.w, b1.w, acc[1]);
    }
  }

  // acc[ct][j] = out[m0 + 32w + 8(j/4) + 4h + j%4][64 ob + 32 ct + l32]
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    const int col = 64 * ob + 32 * ct + l32;
    const float bv = bias ? bias[col] : 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int row = m0 + 32 * wave + 8 * (j >> 2) + 4 * h + (j & 3);
      if (row >= M) continue;
      float v = acc[ct][j] + bv;
      if (Z) Z[static_cast<int64_t>(row) * ldz + col] = v;  // pre-activation (training)
      if (epi == TMAC_EPI_GELU) v = 0.5f * v * (1.f + erff(v * 0.70710678118654752f));
      Y[static_cast<int64_t>(row) * ldy + col] = v;
    }
  }
}

// fp32 SDDMM: the work split of bell_sddmm_kernel (a workgroup per M-range,
// block-row r and four slots, wave w on slot 4 sg + w). Per 32-row step the
// workgroup stages X[m:m+32, 64r:+64] and each wave its own dY[m:m+32, 64c:+64]
// in LDS (rows past the range are zero); the wave's 64x64 block is four 32x32
// MFMA tiles, an MFMA step summing rows m + 2s (lanes 0-31) and m + 2s + 1
// (lanes 32-63). Partial sums go to the workspace as in the 16-bit kernel.
__global__ __launch_bounds__(256, 2) void bell_sddmm_f32_kernel(
    const float* __restrict__ X, int64_t ldx, const float* __restrict__ dY, int64_t lddy,
    const int32_t* __restrict__ col_idx, float* __restrict__ part, int M, int n_brow, int width,
    int n_sgroups, int rows_per_split, int n_splits, int per_xcd) {
  __shared__ __attribute__((aligned(16))) float xs[32 * 64];
  __shared__ __attribute__((aligned(16))) float ds[4][32 * 64];

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
  const int s = sg * 4 + wave;
  const bool active = s < width;
  const int c = col_idx[r * width + min(s, width - 1)];  // inactive waves stage a valid tile
  const int m_lo = split * rows_per_split;
  const int m_hi = min(M, m_lo + rows_per_split);

  // X: rows tid/16 and 16 + tid/16, chunk tid % 16; dY: the wave's lanes, rows
  // 4p + lane/16 (p = 0..7), chunk lane % 16.
  const int xr = tid >> 4, xc = tid & 15, dr = lane >> 4, dc = lane & 15;
  f32x4 px[2], pd[8];
  auto gload = [&](int m) __attribute__((always_inline)) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int row = m + 16 * p + xr;
      const f32x4 v = *reinterpret_cast<const f32x4*>(
          X + static_cast<int64_t>(min(row, M - 1)) * ldx + 64 * r + 4 * xc);
      px[p] = row < m_hi ? v : f32x4{};
    }
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const int row = min(m + 4 * p + dr, M - 1);
      pd[p] = *reinterpret_cast<const f32x4*>(dY + static_cast<int64_t>(row) * lddy + 64 * c + 4 * dc);
    }
  };
  auto sstore = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int p = 0; p < 2; ++p) *reinterpret_cast<f32x4*>(xs + (16 * p + xr) * 64 + 4 * xc) = px[p];
#pragma unroll
    for (int p = 0; p < 8; ++p)
      *reinterpret_cast<f32x4*>(ds[wave] + (4 * p + dr) * 64 + 4 * dc) = pd[p];
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = f32x16{};
  if (m_lo < m_hi) gload(m_lo);
  for (int m = m_lo; m < m_hi; m += 32) {
    __syncthreads();
    sstore();
    __syncthreads();
    if (m + 32 < m_hi) gload(m + 32);
    const float* dsw = ds[wave];
#pragma unroll
    for (int st = 0; st < 16; ++st) {
      const int row = 2 * st + h;
      const float a0 = xs[row * 64 + l32], a1 = xs[row * 64 + 32 + l32];
      const float b0 = dsw[row * 64 + l32], b1 = dsw[row * 64 + 32 + l32];
      acc[0][0] = mfma_f32(a0, b0, acc[0][0]);
      acc[0][1] = mfma_f32(a0, b1, acc[0][1]);
      acc[1][0] = mfma_f32(a1, b0, acc[1][0]);
      acc[1][1] = mfma_f32(a1, b1, acc[1][1]);
    }
  }

  if (!active) return;
  float* dst = part + (static_cast<int64_t>(split) * n_brow * width + r * width + s) * 4096;
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int kk = 32 * a + 8 * (j >> 2) + 4 * h + (j & 3);
        dst[kk * 64 + 32 * b + l32] = acc[a][b][j];
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
    packed.x = Mfma<OUT>::pack2(s.x, s.y);
    packed.y = Mfma<OUT>::pack2(s.z, s.w);
    *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(out) + i4) = packed;
  }
}

// GELU backward with the bias gradient's partial sums (fc1 of an MLP in
// training): gZ = gA ⊙ gelu_erf_grad(Z) for [M, N] 16-bit rows (N a multiple
// of 8), and with part non-null part[p][n] = the sum of the stored (rounded)
// gZ[m][n] over the rows of part p (rows p·R .. p·R + R - 1). Workgroup = 512
// columns x 4 waves: each wave reads 1 KB of one row per instruction (lane =
// 8 columns) and walks rows w, w + 4, ... of the part; the 4 waves' sums are
// added through LDS in a fixed order, and column_sum_kernel adds the parts in
// a fixed order: deterministic for given (M, N). Grid (ceil(N / 512), parts).
constexpr int kGeluParts = 256;  // at most this many row parts

template <int DT, bool GELU = true>
__global__ __launch_bounds__(256) void bell_gelu_bwd_kernel(
    const uint16_t* __restrict__ gA, int64_t lda, const uint16_t* __restrict__ Z, int64_t ldz,
    uint16_t* __restrict__ gZ, int64_t ldg, float* __restrict__ part, int M, int N,
    int rows_per_part) {
  __shared__ float red[4][512];
  const int cg = threadIdx.x & 63, rl = threadIdx.x >> 6;
  const int col = blockIdx.x * 512 + cg * 8;
  const int r0 = blockIdx.y * rows_per_part;
  const int r1 = min(M, r0 + rows_per_part);
  float acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k] = 0.f;
  if (col < N) {
    // four rows per pass, their eight loads issued together (rows past the
    // part read its last row, valid memory, and are computed but neither
    // stored nor summed)
    for (int r = r0 + rl; r < r1; r += 16) {
      u32x4 a[4], z[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int rr = min(r + 4 * u, r1 - 1);
        a[u] = ldg16(gA + static_cast<int64_t>(rr) * lda + col);
        if constexpr (GELU) z[u] = ldg16(Z + static_cast<int64_t>(rr) * ldz + col);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const bool valid = r + 4 * u < r1;
        if constexpr (!GELU) {
          // column sums of the gradient itself (a plain bias gradient)
          const uint32_t aw[4] = {a[u].x, a[u].y, a[u].z, a[u].w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            acc[2 * i] += valid ? Mfma<DT>::to_f32(static_cast<uint16_t>(aw[i] & 0xffff)) : 0.f;
            acc[2 * i + 1] += valid ? Mfma<DT>::to_f32(static_cast<uint16_t>(aw[i] >> 16)) : 0.f;
          }
          continue;
        }
        const uint32_t aw[4] = {a[u].x, a[u].y, a[u].z, a[u].w};
        const uint32_t zw[4] = {z[u].x, z[u].y, z[u].z, z[u].w};
        uint32_t ow[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float g0 = Mfma<DT>::to_f32(static_cast<uint16_t>(aw[i] & 0xffff)) *
                           gelu_erf_grad(Mfma<DT>::to_f32(static_cast<uint16_t>(zw[i] & 0xffff)));
          const float g1 = Mfma<DT>::to_f32(static_cast<uint16_t>(aw[i] >> 16)) *
                           gelu_erf_grad(Mfma<DT>::to_f32(static_cast<uint16_t>(zw[i] >> 16)));
          ow[i] = Mfma<DT>::pack2(g0, g1);
          acc[2 * i] += valid ? Mfma<DT>::to_f32(static_cast<uint16_t>(ow[i] & 0xffff)) : 0.f;
          acc[2 * i + 1] += valid ? Mfma<DT>::to_f32(static_cast<uint16_t>(ow[i] >> 16)) : 0.f;
        }
        if (valid) stg16(gZ + static_cast<int64_t>(r + 4 * u) * ldg + col, u32x4{ow[0], ow[1], ow[2], ow[3]});
      }
    }
  }
  if (!part) return;
#pragma unroll
  for (int k = 0; k < 8; ++k) red[rl][cg * 8 + k] = acc[k];
  __syncthreads();
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int cl = threadIdx.x + 256 * h;
    const int c = blockIdx.x * 512 + cl;
    if (c < N) part[static_cast<int64_t>(blockIdx.y) * N + c] = ((red[0][cl] + red[1][cl]) + red[2][cl]) + red[3][cl];
  }
}

// d/dx of the exact erf GELU, 0.5 (1 + erf(x/√2)) + x exp(-x²/2) / √(2π), with the
// device library's erff and expf: the fp32 form (the forward's fp32 epilogue uses
// erff as well).
__device__ __forceinline__ float gelu_grad_f32(float x) {
  return fmaf(x * 0.39894228040143268f, expf(-0.5f * x * x),
              0.5f * (1.0f + erff(x * 0.70710678118654752f)));
}

// fp32 form of bell_gelu_bwd_kernel: lane = 4 columns (16 bytes), workgroup =
// 256 columns x 4 waves, the same row walk and fixed-order sums (of gZ as
// stored, here unrounded fp32). Grid (ceil(N / 256), parts).
template <bool GELU = true>
__global__ __launch_bounds__(256) void bell_gelu_bwd_f32_kernel(
    const float* __restrict__ gA, int64_t lda, const float* __restrict__ Z, int64_t ldz,
    float* __restrict__ gZ, int64_t ldg, float* __restrict__ part, int M, int N,
    int rows_per_part) {
  __shared__ float red[4][256];
  const int cg = threadIdx.x & 63, rl = threadIdx.x >> 6;
  const int col = blockIdx.x * 256 + cg * 4;
  const int r0 = blockIdx.y * rows_per_part;
  const int r1 = min(M, r0 + rows_per_part);
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  if (col < N) {
    for (int r = r0 + rl; r < r1; r += 16) {
      f32x4 a[4], z[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int rr = min(r + 4 * u, r1 - 1);
        a[u] = *reinterpret_cast<const f32x4*>(gA + static_cast<int64_t>(rr) * lda + col);
        if constexpr (GELU) z[u] = *reinterpret_cast<const f32x4*>(Z + static_cast<int64_t>(rr) * ldz + col);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const bool valid = r + 4 * u < r1;
        f32x4 g = a[u];
        if constexpr (GELU) {
#pragma unroll
          for (int i = 0; i < 4; ++i) g[i] = a[u][i] * gelu_grad_f32(z[u][i]);
          if (valid) *reinterpret_cast<f32x4*>(gZ + static_cast<int64_t>(r + 4 * u) * ldg + col) = g;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] += valid ? g[i] : 0.f;
      }
    }
  }
  if (!part) return;
#pragma unroll
  for (int k = 0; k < 4; ++k) red[rl][cg * 4 + k] = acc[k];
  __syncthreads();
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c < N)
    part[static_cast<int64_t>(blockIdx.y) * N + c] =
        ((red[0][threadIdx.x] + red[1][threadIdx.x]) + red[2][threadIdx.x]) + red[3][threadIdx.x];
}

// Row parts of bell_gelu_bwd_kernel: about 128 rows each, at most kGeluParts.
void gelu_parts(int M, int* n_parts, int* rows_per_part) {
  int p = (M + 127) / 128;
  p = p < 1 ? 1 : (p > kGeluParts ? kGeluParts : p);
  *n_parts = p;
  *rows_per_part = (M + p - 1) / p;
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

// Split of the SDDMM reduction over M, rows per split a multiple of 64. The
// 16-bit kernel (two workgroups per CU) takes as many splits as fit the 512
// slots of one wave of workgroups, so no workgroup waits for a second round;
// the fp32 kernel (four per CU) about 512 workgroups or a few more.
void sddmm_split(int M, int n_brow, int width, bool f32, int* n_splits, int* rows_per_split) {
  const int n_sg = (width + 3) / 4;
  const int base = n_brow * n_sg;
  const int m_steps = (M + 63) / 64;
  int want = f32 ? (512 + base - 1) / base : 512 / base;
  if (want < 1) want = 1;
  if (want > m_steps) want = m_steps;
  const int steps_per = (m_steps + want - 1) / want;
  *rows_per_split = steps_per * 64;
  *n_splits = (M + *rows_per_split - 1) / *rows_per_split;
}

// Workspace of tmac_bell_sddmm: the partial sums of the larger of the two
// kernels' splits (one size for every dtype).
size_t sddmm_ws_bytes(int M, int n_brow, int width) {
  int n32, n16, rows_per_split;
  sddmm_split(M, n_brow, width, true, &n32, &rows_per_split);
  sddmm_split(M, n_brow, width, false, &n16, &rows_per_split);
  return static_cast<size_t>(n32 > n16 ? n32 : n16) * n_brow * width * 4096 * sizeof(float);
}

}  // namespace

namespace {

// tmac_bell_fwd, and with d_Z (16-bit, epi GELU) tmac_bell_fwd_gelu_aux.
int bell_fwd_impl(const void* d_X, int64_t ldx, const void* d_vals, const int32_t* d_t_ptr,
                  const int32_t* d_t_row, const int32_t* d_t_vblk, const int32_t* d_order,
                  const void* d_bias, void* d_Y, int64_t ldy, void* d_Z, int64_t ldz, int M,
                  int n_brow, int n_bcol, int width, int dtype, int epi, void* stream) {
  if (!d_X || !d_vals || !d_t_ptr || !d_t_row || !d_t_vblk || !d_order || !d_Y) return TMAC_ERR_NULL;
  int st = check_bell_shape(M, n_brow, n_bcol, width);
  if (st != TMAC_OK) return st;
  if (dtype != TMAC_BF16 && dtype != TMAC_F16 && dtype != TMAC_F32) return TMAC_ERR_DTYPE;
  if (epi != TMAC_EPI_NONE && epi != TMAC_EPI_GELU) return TMAC_ERR_VALUE;
  const int64_t K = 64ll * n_brow, N = 64ll * n_bcol;
  if (ldx < K || ldy < N || (d_Z && ldz < N)) return TMAC_ERR_SHAPE;
  const int vec = dtype == TMAC_F32 ? 4 : 8;  // elements per 16 bytes
  if (!aligned16(d_X) || !aligned16(d_vals) || !aligned16(d_Y) || (ldx % vec) || (ldy % vec))
    return TMAC_ERR_ALIGN;
  if (d_bias && !aligned16(d_bias)) return TMAC_ERR_ALIGN;
  if (d_Z && (!aligned16(d_Z) || (ldz % vec))) return TMAC_ERR_ALIGN;
  if (dtype == TMAC_F32) {
    const int n_mt = (M + kBMf - 1) / kBMf;
    const int64_t tot = static_cast<int64_t>(n_mt) * n_bcol;
    if (tot > (1ll << 30)) return TMAC_ERR_SHAPE;
    const int pxcd = static_cast<int>((tot + 7) / 8);
    hipLaunchKernelGGL((bell_gemm_f32_kernel<true>), dim3(8 * pxcd), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const float*>(d_X), ldx,
                       static_cast<const float*>(d_vals), d_t_ptr, d_t_row, d_t_vblk, d_order,
                       static_cast<const float*>(d_bias), epi, static_cast<float*>(d_Y), ldy,
                       static_cast<float*>(d_Z), ldz, M, n_bcol, width, n_mt, pxcd);
    return launch_status();
  }
  const int n_mtiles = (M + kBM - 1) / kBM;
  const int64_t total = static_cast<int64_t>(n_mtiles) * n_bcol;
  if (total > (1ll << 30)) return TMAC_ERR_SHAPE;
  const int per_xcd = static_cast<int>((total + 7) / 8);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const auto* X = static_cast<const uint16_t*>(d_X);
  const auto* V = static_cast<const uint16_t*>(d_vals);
  const auto* b = static_cast<const uint16_t*>(d_bias);
  auto* Y = static_cast<uint16_t*>(d_Y);
  auto* Z = static_cast<uint16_t*>(d_Z);
  if (M <= kSmallM) {
    if (dtype == TMAC_BF16)
      hipLaunchKernelGGL((bell_fwd_small_kernel<TMAC_BF16>), dim3(n_bcol), dim3(256), 0, s, X, ldx, V,
                         d_t_ptr, d_t_row, d_t_vblk, b, epi, Y, ldy, Z, ldz, M);
    else
      hipLaunchKernelGGL((bell_fwd_small_kernel<TMAC_F16>), dim3(n_bcol), dim3(256), 0, s, X, ldx, V,
                         d_t_ptr, d_t_row, d_t_vblk, b, epi, Y, ldy, Z, ldz, M);
    return launch_status();
  }
  if (dtype == TMAC_BF16)
    hipLaunchKernelGGL((bell_gemm_kernel<TMAC_BF16, true>), dim3(8 * per_xcd), dim3(256), 0, s, X,
                       ldx, V, d_t_ptr, d_t_row, d_t_vblk, d_order, b, epi, Y, ldy, Z, ldz, M, n_bcol,
                       width, n_mtiles, per_xcd);
  else
    hipLaunchKernelGGL((bell_gemm_kernel<TMAC_F16, true>), dim3(8 * per_xcd), dim3(256), 0, s, X,
                       ldx, V, d_t_ptr, d_t_row, d_t_vblk, d_order, b, epi, Y, ldy, Z, ldz, M, n_bcol,
                       width, n_mtiles, per_xcd);
  return launch_status();
}

}  // namespace

extern "C" int tmac_bell_fwd(const void* d_X, int64_t ldx, const void* d_vals,
                             const int32_t* d_t_ptr, const int32_t* d_t_row,
                             const int32_t* d_t_vblk, const int32_t* d_order, const void* d_bias,
                             void* d_Y, int64_t ldy, int M, int n_brow, int n_bcol, int width,
                             int dtype, int epi, void* stream) {
  return bell_fwd_impl(d_X, ldx, d_vals, d_t_ptr, d_t_row, d_t_vblk, d_order, d_bias, d_Y, ldy,
                       nullptr, 0, M, n_brow, n_bcol, width, dtype, epi, stream);
}

extern "C" int tmac_bell_fwd_gelu_aux(const void* d_X, int64_t ldx, const void* d_vals,
                                      const int32_t* d_t_ptr, const int32_t* d_t_row,
                                      const int32_t* d_t_vblk, const int32_t* d_order,
                                      const void* d_bias, void* d_Y, int64_t ldy, void* d_Z,
                                      int64_t ldz, int M, int n_brow, int n_bcol, int width,
                                      int dtype, void* stream) {
  if (!d_Z) return TMAC_ERR_NULL;
  return bell_fwd_impl(d_X, ldx, d_vals, d_t_ptr, d_t_row, d_t_vblk, d_order, d_bias, d_Y, ldy,
                       d_Z, ldz, M, n_brow, n_bcol, width, dtype, TMAC_EPI_GELU, stream);
}

namespace {

// Launch of the grouped forward: one persistent workgroup per CU (at most 32
// per XCD), fewer when there are fewer tiles.
int bell_fwd_grouped_impl(const void* d_A, int64_t lda, const void* d_vals, const int32_t* d_grp_ptr,
                          const int32_t* d_grp_out, const int32_t* d_steps, int n_groups, int group,
                          const int32_t* d_order, int order_len, const void* d_bias, int epi,
                          void* d_Y, int64_t ldy, void* d_Z, int64_t ldz, int M, int n_brow,
                          int n_bcol, int width, int dtype, void* stream) {
  if (!d_A || !d_vals || !d_grp_ptr || !d_grp_out || !d_steps || !d_Y) return TMAC_ERR_NULL;
  int st = check_bell_shape(M, n_brow, n_bcol, width);
  if (st != TMAC_OK) return st;
  if (dtype != TMAC_BF16 && dtype != TMAC_F16) return TMAC_ERR_DTYPE;
  if (group != 2) return TMAC_ERR_VALUE;
  if (epi != TMAC_EPI_NONE && epi != TMAC_EPI_GELU) return TMAC_ERR_VALUE;
  if (n_groups != (n_bcol + group - 1) / group) return TMAC_ERR_SHAPE;
  const int64_t K = 64ll * n_brow, N = 64ll * n_bcol;
  if (lda < K || ldy < N || (d_Z && ldz < N)) return TMAC_ERR_SHAPE;
  // the copies address 512 activation rows with 32-bit byte offsets
  if (lda > (1ll << 22)) return TMAC_ERR_SHAPE;
  if (!aligned16(d_A) || !aligned16(d_vals) || !aligned16(d_Y) || (lda % 8) || (ldy % 8))
    return TMAC_ERR_ALIGN;
  if (d_bias && !aligned16(d_bias)) return TMAC_ERR_ALIGN;
  if (d_Z && (!aligned16(d_Z) || (ldz % 8))) return TMAC_ERR_ALIGN;
  if (M == 0) return TMAC_OK;
  const int n_mtiles = (M + kGM - 1) / kGM;
  const int64_t total = static_cast<int64_t>(n_mtiles) * n_groups;
  if (total > (1ll << 30)) return TMAC_ERR_SHAPE;
  const int per_xcd = static_cast<int>((total + 7) / 8);
  const int n_slots = per_xcd < TMAC_BELL_GROUP_SLOTS ? per_xcd : TMAC_BELL_GROUP_SLOTS;
  const int n_rounds = (per_xcd + n_slots - 1) / n_slots;
  // the balanced order must be tmac_bell_group_tile_order's for this launch
  if (d_order && static_cast<int64_t>(order_len) != 8ll * n_rounds * n_slots) return TMAC_ERR_SHAPE;
  const int grid = 8 * n_slots;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const auto* A = static_cast<const uint16_t*>(d_A);
  const auto* V = static_cast<const uint16_t*>(d_vals);
  const auto* b = static_cast<const uint16_t*>(d_bias);
  auto* Y = static_cast<uint16_t*>(d_Y);
  auto* Z = static_cast<uint16_t*>(d_Z);
  // the epilogue's bias / activation / Z code is compiled only where used
  const bool epi_any = b || Z || epi != TMAC_EPI_NONE;
#define TMAC_GG_LAUNCH(DT, E, R)                                                                    \
  hipLaunchKernelGGL((bell_ggemm_kernel<DT, E, R>), dim3(grid), dim3(512 * R), 0, s, A, lda, V, d_grp_ptr, \
                     d_grp_out, d_steps, b, epi, Y, ldy, Z, ldz, M, n_groups,                      \
                     static_cast<int>(total), per_xcd, d_order, n_rounds)
  // Without an epilogue: 16 waves (64 rows each, 128 VGPRs, four waves per SIMD to
  // cover each other's LDS and copy latency). The bias / GELU / Z epilogue needs more
  // registers than that allows without spilling: 8 waves of 128 rows.
  if (dtype == TMAC_BF16) {
    if (epi_any)
      TMAC_GG_LAUNCH(TMAC_BF16, true, 1);
    else
      TMAC_GG_LAUNCH(TMAC_BF16, false, 2);
  } else {
    if (epi_any)
      TMAC_GG_LAUNCH(TMAC_F16, true, 1);
    else
      TMAC_GG_LAUNCH(TMAC_F16, false, 2);
  }
#undef TMAC_GG_LAUNCH
  return launch_status();
}

}  // namespace

extern "C" int tmac_bell_fwd_grouped(const void* d_X, int64_t ldx, const void* d_vals,
                                     const int32_t* d_grp_ptr, const int32_t* d_grp_out,
                                     const int32_t* d_steps, int n_groups, int group,
                                     const int32_t* d_tile_order, int tile_order_len,
                                     const void* d_bias, void* d_Y, int64_t ldy, int M, int n_brow,
                                     int n_bcol, int width, int dtype, int epi, void* stream) {
  return bell_fwd_grouped_impl(d_X, ldx, d_vals, d_grp_ptr, d_grp_out, d_steps, n_groups, group,
                               d_tile_order, tile_order_len, d_bias, epi, d_Y, ldy, nullptr, 0, M,
                               n_brow, n_bcol, width, dtype, stream);
}

extern "C" int tmac_bell_fwd_grouped_gelu_aux(const void* d_X, int64_t ldx, const void* d_vals,
                                              const int32_t* d_grp_ptr, const int32_t* d_grp_out,
                                              const int32_t* d_steps, int n_groups, int group,
                                              const int32_t* d_tile_order, int tile_order_len,
                                              const void* d_bias, void* d_Y, int64_t ldy, void* d_Z,
                                              int64_t ldz, int M, int n_brow, int n_bcol, int width,
                                              int dtype, void* stream) {
  if (!d_Z) return TMAC_ERR_NULL;
  return bell_fwd_grouped_impl(d_X, ldx, d_vals, d_grp_ptr, d_grp_out, d_steps, n_groups, group,
                               d_tile_order, tile_order_len, d_bias, TMAC_EPI_GELU, d_Y, ldy, d_Z,
                               ldz, M, n_brow, n_bcol, width, dtype, stream);
}

extern "C" int tmac_bell_dx(const void* d_dY, int64_t lddy, const void* d_vals,
                            const int32_t* d_col_idx, void* d_dX, int64_t lddx, int M, int n_brow,
                            int n_bcol, int width, int dtype, void* stream) {
  if (!d_dY || !d_vals || !d_col_idx || !d_dX) return TMAC_ERR_NULL;
  int st = check_bell_shape(M, n_brow, n_bcol, width);
  if (st != TMAC_OK) return st;
  if (dtype != TMAC_BF16 && dtype != TMAC_F16 && dtype != TMAC_F32) return TMAC_ERR_DTYPE;
  const int64_t K = 64ll * n_brow, N = 64ll * n_bcol;
  if (lddy < N || lddx < K) return TMAC_ERR_SHAPE;
  const int vec = dtype == TMAC_F32 ? 4 : 8;
  if (!aligned16(d_dY) || !aligned16(d_vals) || !aligned16(d_dX) || (lddy % vec) || (lddx % vec))
    return TMAC_ERR_ALIGN;
  if (dtype == TMAC_F32) {
    const int n_mt = (M + kBMf - 1) / kBMf;
    const int64_t tot = static_cast<int64_t>(n_mt) * n_brow;
    if (tot > (1ll << 30)) return TMAC_ERR_SHAPE;
    const int pxcd = static_cast<int>((tot + 7) / 8);
    hipLaunchKernelGGL((bell_gemm_f32_kernel<false>), dim3(8 * pxcd), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const float*>(d_dY), lddy,
                       static_cast<const float*>(d_vals), nullptr, d_col_idx, nullptr, nullptr,
                       nullptr, 0, static_cast<float*>(d_dX), lddx, nullptr, 0, M, n_brow, width,
                       n_mt, pxcd);
    return launch_status();
  }
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
                       dY, lddy, V, nullptr, d_col_idx, nullptr, nullptr, nullptr, 0, dX, lddx, nullptr,
                       0, M, n_brow, width, n_mtiles, per_xcd);
  else
    hipLaunchKernelGGL((bell_gemm_kernel<TMAC_F16, false>), dim3(8 * per_xcd), dim3(256), 0, s,
                       dY, lddy, V, nullptr, d_col_idx, nullptr, nullptr, nullptr, 0, dX, lddx, nullptr,
                       0, M, n_brow, width, n_mtiles, per_xcd);
  return launch_status();
}

extern "C" int tmac_bell_sddmm_workspace(int M, int n_brow, int n_bcol, int width,
                                         size_t* ws_bytes) {
  if (!ws_bytes) return TMAC_ERR_NULL;
  int st = check_bell_shape(M, n_brow, n_bcol, width);
  if (st != TMAC_OK) return st;
  *ws_bytes = sddmm_ws_bytes(M, n_brow, width);
  return TMAC_OK;
}

extern "C" int tmac_bell_sddmm(const void* d_X, int64_t ldx, const void* d_dY, int64_t lddy,
                               const int32_t* d_col_idx, void* d_dvals, int dvals_dtype,
                               void* d_ws, size_t ws_bytes, int M, int n_brow, int n_bcol,
                               int width, int dtype, void* stream) {
  if (!d_X || !d_dY || !d_col_idx || !d_dvals) return TMAC_ERR_NULL;
  int st = check_bell_shape(M, n_brow, n_bcol, width);
  if (st != TMAC_OK) return st;
  if (dtype != TMAC_BF16 && dtype != TMAC_F16 && dtype != TMAC_F32) return TMAC_ERR_DTYPE;
  if (dvals_dtype != TMAC_F32 && dvals_dtype != TMAC_BF16 && dvals_dtype != TMAC_F16)
    return TMAC_ERR_DTYPE;
  const int64_t K = 64ll * n_brow, N = 64ll * n_bcol;
  if (ldx < K || lddy < N) return TMAC_ERR_SHAPE;
  const int vec = dtype == TMAC_F32 ? 4 : 8;
  if (!aligned16(d_X) || !aligned16(d_dY) || !aligned16(d_dvals) || (ldx % vec) || (lddy % vec))
    return TMAC_ERR_ALIGN;
  int n_splits, rows_per_split;
  sddmm_split(M, n_brow, width, dtype == TMAC_F32, &n_splits, &rows_per_split);
  if (!d_ws || ws_bytes < sddmm_ws_bytes(M, n_brow, width)) return TMAC_ERR_WORKSPACE;
  if (!aligned16(d_ws)) return TMAC_ERR_ALIGN;
  // the 16-bit kernel addresses 32 rows of X and dY with 32-bit byte offsets
  if (dtype != TMAC_F32 && (ldx > (1ll << 25) || lddy > (1ll << 25))) return TMAC_ERR_SHAPE;
  const int n_sg = (width + 3) / 4;
  const int64_t total = static_cast<int64_t>(n_splits) * n_brow * n_sg;
  const int per_xcd = static_cast<int>((total + 7) / 8);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const auto* X = static_cast<const uint16_t*>(d_X);
  const auto* dY = static_cast<const uint16_t*>(d_dY);
  float* part = static_cast<float*>(d_ws);
  if (dtype == TMAC_F32)
    hipLaunchKernelGGL(bell_sddmm_f32_kernel, dim3(8 * per_xcd), dim3(256), 0, s,
                       static_cast<const float*>(d_X), ldx, static_cast<const float*>(d_dY), lddy,
                       d_col_idx, part, M, n_brow, width, n_sg, rows_per_split, n_splits, per_xcd);
  else if (dtype == TMAC_BF16)
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

extern "C" int tmac_bell_gelu_bwd_workspace(int M, int N, size_t* ws_bytes) {
  if (!ws_bytes) return TMAC_ERR_NULL;
  if (M < 0 || N <= 0) return TMAC_ERR_SHAPE;
  int n_parts, rows;
  gelu_parts(M, &n_parts, &rows);
  *ws_bytes = static_cast<size_t>(n_parts) * N * sizeof(float);
  return TMAC_OK;
}

extern "C" int tmac_bell_gelu_bwd(const void* d_gA, int64_t ldga, const void* d_Z, int64_t ldz,
                                  void* d_gZ, int64_t ldgz, float* d_dbias, void* d_ws,
                                  size_t ws_bytes, int M, int N, int dtype, void* stream) {
  // with M = 0 the row operands are not read (empty tensors may pass null)
  if ((M > 0 && (!d_gA || !d_Z || !d_gZ)) || (d_dbias && !d_ws)) return TMAC_ERR_NULL;
  if (dtype != TMAC_BF16 && dtype != TMAC_F16 && dtype != TMAC_F32) return TMAC_ERR_DTYPE;
  const int vec = dtype == TMAC_F32 ? 4 : 8;  // elements per 16 bytes
  if (M < 0 || N <= 0 || (N % vec) || ldga < N || ldz < N || ldgz < N) return TMAC_ERR_SHAPE;
  if (!aligned16(d_gA) || !aligned16(d_Z) || !aligned16(d_gZ) || (ldga % vec) || (ldz % vec) ||
      (ldgz % vec))
    return TMAC_ERR_ALIGN;
  int n_parts, rows;
  gelu_parts(M, &n_parts, &rows);
  float* part = nullptr;
  if (d_dbias) {
    if (ws_bytes < static_cast<size_t>(n_parts) * N * sizeof(float)) return TMAC_ERR_WORKSPACE;
    if (!aligned16(d_ws)) return TMAC_ERR_ALIGN;
    part = static_cast<float*>(d_ws);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (M > 0 && dtype == TMAC_F32) {
    const dim3 grid(static_cast<unsigned>((N + 255) / 256), static_cast<unsigned>(n_parts));
    hipLaunchKernelGGL(bell_gelu_bwd_f32_kernel<true>, grid, dim3(256), 0, s,
                       static_cast<const float*>(d_gA), ldga, static_cast<const float*>(d_Z), ldz,
                       static_cast<float*>(d_gZ), ldgz, part, M, N, rows);
    const int st = launch_status();
    if (st != TMAC_OK) return st;
  } else if (M > 0) {
    const dim3 grid(static_cast<unsigned>((N + 511) / 512), static_cast<unsigned>(n_parts));
    const auto* gA = static_cast<const uint16_t*>(d_gA);
    const auto* Z = static_cast<const uint16_t*>(d_Z);
    auto* gZ = static_cast<uint16_t*>(d_gZ);
    if (dtype == TMAC_BF16)
      hipLaunchKernelGGL((bell_gelu_bwd_kernel<TMAC_BF16>), grid, dim3(256), 0, s, gA, ldga, Z, ldz,
                         gZ, ldgz, part, M, N, rows);
    else
      hipLaunchKernelGGL((bell_gelu_bwd_kernel<TMAC_F16>), grid, dim3(256), 0, s, gA, ldga, Z, ldz,
                         gZ, ldgz, part, M, N, rows);
    const int st = launch_status();
    if (st != TMAC_OK) return st;
  }
  if (d_dbias) {
    // with M = 0 there are no partials: the sums over zero parts are 0
    hipLaunchKernelGGL(column_sum_kernel, dim3(static_cast<unsigned>((N + 63) / 64)), dim3(256), 0, s,
                       part, d_dbias, static_cast<int64_t>(N), M > 0 ? n_parts : 0, int64_t{0});
    return launch_status();
  }
  return TMAC_OK;
}

extern "C" int tmac_bell_bias_grad(const void* d_gY, int64_t ldgy, float* d_dbias, void* d_ws,
                                   size_t ws_bytes, int M, int N, int dtype, void* stream) {
  if ((M > 0 && !d_gY) || !d_dbias || !d_ws) return TMAC_ERR_NULL;
  if (dtype != TMAC_BF16 && dtype != TMAC_F16 && dtype != TMAC_F32) return TMAC_ERR_DTYPE;
  const int vec = dtype == TMAC_F32 ? 4 : 8;  // elements per 16 bytes
  if (M < 0 || N <= 0 || (N % vec) || ldgy < N) return TMAC_ERR_SHAPE;
  if (!aligned16(d_gY) || (ldgy % vec) || !aligned16(d_ws)) return TMAC_ERR_ALIGN;
  int n_parts, rows;
  gelu_parts(M, &n_parts, &rows);
  if (ws_bytes < static_cast<size_t>(n_parts) * N * sizeof(float)) return TMAC_ERR_WORKSPACE;
  auto* part = static_cast<float*>(d_ws);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (M > 0 && dtype == TMAC_F32) {
    const dim3 grid(static_cast<unsigned>((N + 255) / 256), static_cast<unsigned>(n_parts));
    hipLaunchKernelGGL(bell_gelu_bwd_f32_kernel<false>, grid, dim3(256), 0, s,
                       static_cast<const float*>(d_gY), ldgy, nullptr, int64_t{0}, nullptr, int64_t{0},
                       part, M, N, rows);
    const int st = launch_status();
    if (st != TMAC_OK) return st;
  } else if (M > 0) {
    const dim3 grid(static_cast<unsigned>((N + 511) / 512), static_cast<unsigned>(n_parts));
    const auto* gY = static_cast<const uint16_t*>(d_gY);
    if (dtype == TMAC_BF16)
      hipLaunchKernelGGL((bell_gelu_bwd_kernel<TMAC_BF16, false>), grid, dim3(256), 0, s, gY, ldgy,
                         nullptr, int64_t{0}, nullptr, int64_t{0}, part, M, N, rows);
    else
      hipLaunchKernelGGL((bell_gelu_bwd_kernel<TMAC_F16, false>), grid, dim3(256), 0, s, gY, ldgy,
                         nullptr, int64_t{0}, nullptr, int64_t{0}, part, M, N, rows);
    const int st = launch_status();
    if (st != TMAC_OK) return st;
  }
  hipLaunchKernelGGL(column_sum_kernel, dim3(static_cast<unsigned>((N + 63) / 64)), dim3(256), 0, s,
                     part, d_dbias, static_cast<int64_t>(N), M > 0 ? n_parts : 0, int64_t{0});
  return launch_status();
}
