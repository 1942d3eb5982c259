// Device-side building blocks shared by the gfx950 kernels: vector types, the
// 32x32x16 MFMA wrappers, LDS transpose reads and conversions.
//
// Lane layouts of v_mfma_f32_32x32x16_{bf16,f16} (wave64, h = lane / 32):
//   A operand (32 x 16):  lane holds A[lane % 32][8h + t], t = 0..7
//   B operand (16 x 32):  lane holds B[8h + t][lane % 32], t = 0..7
//   C/D (32 x 32, fp32):  lane holds C[8(j/4) + 4h + j%4][lane % 32], j = 0..15
//
// ds_read_b64_tr_b16 (gfx950): inside each group of 16 lanes, lane i receives
// element (i % 4) of the 8-byte chunks addressed by lanes 4j + i/4, j = 0..3.
// Pointing lane i' of the group at row (r0 + i'/4), column (c0 + 4*(i'%4)) of a
// row-major 16-bit tile therefore hands lane i the column (c0 + i) entries of
// rows r0..r0+3: a 4x16 tile read transposed.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tmac.h"

namespace tmac {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// Row pitch of every 64-wide 16-bit tile staged in LDS: 64 elements plus 8 of
// padding (144 bytes), so eight consecutive rows start in eight different
// 16-byte bank groups and both the row reads (16 B per lane over 32 rows) and
// the transpose reads (8 rows x 64 B) proceed without bank conflicts.
constexpr int kPitch = 72;
constexpr int kTileElems = 64 * kPitch;  // one 64x64 tile, in 16-bit elements

template <int DT>
struct Mfma;

template <>
struct Mfma<TMAC_BF16> {
  static __device__ __forceinline__ f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t from_f32(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
  }
  static __device__ __forceinline__ float to_f32(uint16_t x) {
    return __uint_as_float(static_cast<uint32_t>(x) << 16);
  }
  // lo | hi << 16, both rounded to nearest even: one v_cvt_pk_bf16_f32.
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
  }
};

template <>
struct Mfma<TMAC_F16> {
  static __device__ __forceinline__ f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t from_f32(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
  }
  static __device__ __forceinline__ float to_f32(uint16_t x) {
    return static_cast<float>(__builtin_bit_cast(_Float16, x));
  }
  // lo | hi << 16, both rounded to nearest even.
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, f16x2_t));
  }
};

// x combined with the value of lane (lane ^ 32), identical in both lanes: one
// v_permlane32_swap of x with itself puts x[l] and x[l ^ 32] in the two results
// (in an order that depends on the half), and max and + are commutative.
__device__ __forceinline__ float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_add(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Eight 16-bit values of column (c0 + lane%16 of the 16-lane group) from rows
// r0..r0+7 of a row-major LDS tile with pitch kPitch, as one MFMA operand:
// two transpose reads, rows r0..r0+3 then r0+4..r0+7. The caller passes the
// tile base offset by the lane's own group (r0 row, c0 column already chosen).
__device__ __forceinline__ u32x4 lds_read_tr8(const uint16_t* tile, int r0, int c0, int lane) {
  const int i = lane & 15;
  const uint16_t* p = tile + (r0 + (i >> 2)) * kPitch + c0 + 4 * (i & 3);
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + 4 * kPitch));
  const u32x2 l2 = __builtin_bit_cast(u32x2, lo);
  const u32x2 h2 = __builtin_bit_cast(u32x2, hi);
  return u32x4{l2.x, l2.y, h2.x, h2.y};
}

// Same as lds_read_tr8 but the two 4-row groups are independent
// (rows r0..r0+3 and r1..r1+3), in a tile of row pitch P elements.
template <int P = kPitch>
__device__ __forceinline__ u32x4 lds_read_tr4x2(const uint16_t* tile, int r0, int r1, int c0,
                                                int lane) {
  const int i = lane & 15;
  const uint16_t* p0 = tile + (r0 + (i >> 2)) * P + c0 + 4 * (i & 3);
  const uint16_t* p1 = tile + (r1 + (i >> 2)) * P + c0 + 4 * (i & 3);
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p0));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p1));
  const u32x2 l2 = __builtin_bit_cast(u32x2, lo);
  const u32x2 h2 = __builtin_bit_cast(u32x2, hi);
  return u32x4{l2.x, l2.y, h2.x, h2.y};
}

__device__ __forceinline__ u32x4 ldg16(const uint16_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void stg16(uint16_t* p, u32x4 v) {
  *reinterpret_cast<u32x4*>(p) = v;
}
__device__ __forceinline__ u32x4 lds16(const uint16_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void sts16(uint16_t* p, u32x4 v) {
  *reinterpret_cast<u32x4*>(p) = v;
}

// Element offset of 16-byte chunk `chunk` of row `row` in an LDS tile of 64
// 16-bit values (128 bytes) per row, chunks XOR-swizzled: chunk c of row r at
// c ^ w((r >> 1) & 7), w(a) = ((a & 1) << 2) | (a >> 1). Conflict-free for the
// 64 four-byte banks both for transpose reads (4 consecutive rows x 64 bytes
// per 32-lane phase) and for 16-byte row reads (16 consecutive rows per phase).
__device__ __forceinline__ int swz64(int row, int chunk) {
  const int a = (row >> 1) & 7;
  return row * 64 + ((chunk ^ (((a & 1) << 2) | (a >> 1))) << 3);
}

// lds_read_tr4x2 for a swz64 tile: rows r0..r0+3 and r1..r1+3 (multiples of
// 4) at column c0 + lane%16 of the 16-lane group.
__device__ __forceinline__ u32x4 lds_read_tr4x2_swz64(const uint16_t* tile, int r0, int r1, int c0,
                                                      int lane) {
  const int i = lane & 15;
  const int col = c0 + 4 * (i & 3);
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_i16x4*)(tile + swz64(r0 + (i >> 2), col >> 3) + (col & 7)));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_i16x4*)(tile + swz64(r1 + (i >> 2), col >> 3) + (col & 7)));
  const u32x2 l2 = __builtin_bit_cast(u32x2, lo);
  const u32x2 h2 = __builtin_bit_cast(u32x2, hi);
  return u32x4{l2.x, l2.y, h2.x, h2.y};
}

// LDS address (byte offset in the workgroup's LDS) of a __shared__ pointer.
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)(p)));
}

// HBM/L2 -> LDS copies with global_load_lds: lane L moves the bytes at
// base + voff (base wave-uniform, in SGPRs; voff this lane's byte offset) to
// LDS byte lds_byte + size * L (lds_byte wave-uniform). 16 bytes per lane
// (1 KB per wave instruction) or 4 (256 bytes). Written as assembly so the
// compiler does not track them: a kernel using these waits for them itself
// with exact vmcnt values (loads complete in issue order), and the compiler's
// own waits, which would cover every copy in flight, stay out of its loop.
__device__ __forceinline__ void dma_lds16(const void* base, uint32_t voff, uint32_t lds_byte) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds_byte), "v"(voff),
               "s"(base)
               : "memory", "m0");
}
__device__ __forceinline__ void dma_lds4(const void* base, uint32_t voff, uint32_t lds_byte) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2" ::"s"(lds_byte), "v"(voff),
               "s"(base)
               : "memory", "m0");
}

// Workgroup id remapped so that consecutive logical ids run on the same XCD:
// the hardware hands workgroup b to XCD b % 8, so logical = (b % 8) * per_xcd +
// b / 8 keeps each XCD on one contiguous slice of the logical work order (and
// its L2 on one slice of the data). Grids are padded to 8 * per_xcd.
__device__ __forceinline__ int xcd_logical_id(int per_xcd) {
  const int b = blockIdx.x;
  return (b & 7) * per_xcd + (b >> 3);
}

// Mask of the windowed attention. window is clamped to S by the host (any
// window >= S gives the same mask), so index arithmetic stays in int range.
struct MaskParams {
  int S, window, Np, causal, pattern, bs;
};

// A set of indices x in [0, S): x < np, or lo <= x <= hi.
struct Span {
  int np, lo, hi;
};

__host__ __device__ inline bool span_has(const Span& s, int x) {
  return (x < s.np) | ((x >= s.lo) & (x <= s.hi));
}

// Keys that query row i attends to.
// Band (attn/windowed_attention.py:97-152): persistent rows (i < Np) see the
// persistent keys only; sequence rows see the persistent keys and the
// sequence keys j with i - w <= j <= i (causal) or |i - j| <= w.
// Block window (attn/block_sparse_attention.py:277-334), r = i - Np,
// b0 = bs * floor(r / bs): persistent rows see every key; sequence rows see
// the persistent keys and sequence keys c = j - Np in [max(0, b0 - w), r]
// (causal) or [max(0, b0 - w), min(b0 + bs, S - Np) - 1].
// Rows i >= S (tile padding) see nothing.
__host__ __device__ inline Span mask_row_span(const MaskParams& p, int i) {
  Span s{0, 1, 0};
  if (i >= p.S) return s;
  s.np = p.Np;
  if (i < p.Np) {
    if (p.pattern == TMAC_PATTERN_BLOCKWIN) {
      s.lo = 0;
      s.hi = p.S - 1;
    }
    return s;
  }
  if (p.pattern == TMAC_PATTERN_BAND) {
    s.lo = i - p.window > p.Np ? i - p.window : p.Np;
    s.hi = p.causal ? i : (i + p.window < p.S - 1 ? i + p.window : p.S - 1);
  } else {
    const int r = i - p.Np, b0 = (r / p.bs) * p.bs;
    s.lo = p.Np + (b0 - p.window > 0 ? b0 - p.window : 0);
    const int end = b0 + p.bs < p.S - p.Np ? b0 + p.bs : p.S - p.Np;
    s.hi = p.Np + (p.causal ? r : end - 1);
  }
  return s;
}

// Query rows that attend to key j: the transpose of mask_row_span.
// Band: a persistent key is seen by every row; a sequence key j by the sequence
// rows i with j <= i <= j + w (causal) or |i - j| <= w.
// Block window: every key is seen by the persistent rows; a persistent key by
// every row; a sequence key c = j - Np by the sequence rows r = i - Np with
// c <= r (causal) or floor(c / bs) * bs <= r (not causal), and
// floor(r / bs) <= floor((c + w) / bs).
__host__ __device__ inline Span mask_col_span(const MaskParams& p, int j) {
  Span s{0, 1, 0};
  if (j >= p.S) return s;
  if (p.pattern == TMAC_PATTERN_BAND) {
    if (j < p.Np) {
      s.lo = 0;
      s.hi = p.S - 1;
    } else {
      const int a = p.causal ? j : j - p.window;
      s.lo = a > p.Np ? a : p.Np;
      s.hi = j + p.window < p.S - 1 ? j + p.window : p.S - 1;
    }
    return s;
  }
  s.np = p.Np;
  if (j < p.Np) {
    s.lo = p.Np;
    s.hi = p.S - 1;
    return s;
  }
  const int c = j - p.Np;
  const int r_lo = p.causal ? c : (c / p.bs) * p.bs;
  const int r_hi = ((c + p.window) / p.bs + 1) * p.bs - 1;
  s.lo = p.Np + r_lo;
  s.hi = p.Np + r_hi < p.S - 1 ? p.Np + r_hi : p.S - 1;
  return s;
}

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as
// 1, 2, 3", SC 2011): ten rounds of a keyed bijection on a 128-bit counter; the
// multipliers and Weyl increments are the paper's. Attention dropout makes one
// call per (query, group of 8 keys, batch*head): counter {key / 8, query, bh, 0},
// key {seed low, seed high}; the call's four words give eight 16-bit draws, key k
// taking bits 16 (k % 2) .. 16 (k % 2) + 15 of word (k % 8) / 2, and (query, key)
// is kept iff its draw >= floor(p * 2^16) (drop_row8, keep_octet2).
struct U32x4 {
  uint32_t x, y, z, w;
};
// 64-bit product of two 32-bit values. On the device one v_mad_u64_u32 gives
// both halves; left to itself the compiler emits v_mul_hi_u32 and v_mul_lo_u32,
// two quarter-rate instructions, for the same product.
__host__ __device__ inline uint64_t mul_wide_u32(uint32_t a, uint32_t m) {
#if defined(__HIP_DEVICE_COMPILE__)
  uint64_t p, carry;  // carry: the instruction's carry-out (an SGPR pair), unused
  asm("v_mad_u64_u32 %0, %1, %2, %3, 0" : "=v"(p), "=s"(carry) : "v"(a), "s"(m));
  return p;
#else
  return static_cast<uint64_t>(a) * m;
#endif
}
__host__ __device__ inline U32x4 philox4x32_10(U32x4 c, uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = mul_wide_u32(c.x, 0xD2511F53u);
    const uint64_t p1 = mul_wide_u32(c.z, 0xCD9E8D57u);
    const uint32_t hi0 = static_cast<uint32_t>(p0 >> 32), lo0 = static_cast<uint32_t>(p0);
    const uint32_t hi1 = static_cast<uint32_t>(p1 >> 32), lo1 = static_cast<uint32_t>(p1);
    c = U32x4{hi1 ^ c.y ^ k0, lo1, hi0 ^ c.w ^ k1, lo0};
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return c;
}

// Extra features of the attention kernels (template flag bits): a caller's mask
// tensor instead of the band / block-window pattern (kFeatMask), attention dropout
// (kFeatDrop).
// kFeatBool (with kFeatMask): the mask is boolean, so no slice takes a bias
// (kind 3) and the kernels leave that path out; it holds about 20 VGPRs.
constexpr int kFeatMask = 1, kFeatDrop = 2, kFeatBool = 4;
// the dQ kernels also write dS, the gradient of an additive mask (AttnX::dbias)
constexpr int kFeatDBias = 8;

struct AttnX {
  const void* mask;      // TMAC_MASK_BOOL: uint8 (0 = masked); TMAC_MASK_ADD_F32: fp32 added to the scores
  int fmt;
  int64_t msb, msh, msq; // element strides of the mask's batch, head, query dims (key stride 1)
  int mb1, mh1, MH;      // batch / head dims of size 1 (broadcast); number of mask heads
  const int32_t* cnt;    // custom work lists: entries of each list row
  int cap;               // entries a list row can hold (row r starts at r * cap) = 64-wide tiles
  const uint64_t* bits;  // allowed-pair bitmap: word (mask row, position, tile) holds 64 bits,
                         // one per position of the other axis in that tile
  uint32_t seed0, seed1; // dropout seed
  uint32_t thresh;       // dropped when the 16-bit draw is below thresh (= floor(p * 2^16))
  float keep_scale;      // 2^16 / (2^16 - thresh): the inverse of the keep probability
  float* dbias;          // additive mask's gradient: dS as fp32 [B*H, S, S] (backward; may be null)
};

// dS of this lane's query row q and keys k0 + 8g + (0..3), g = 0..3 (the
// lane's 16 accumulator elements of a 32-key half), into the fp32 [B*H, S, S]
// gradient of an additive mask; rows and keys past S are skipped.
__device__ __forceinline__ void store_dbias(float* __restrict__ dbias, int bh, int S, int q, int k0,
                                            const float (&ds)[16]) {
  if (q >= S) return;
  float* row = dbias + (static_cast<int64_t>(bh) * S + q) * S;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int k = k0 + 8 * (j >> 2) + (j & 3);
    if (k < S) row[k] = ds[j];
  }
}

// Row of the custom work lists of (b, head): the mask's own (batch, head) row.
__device__ __forceinline__ int mask_row(const AttnX& x, int b, int hd) {
  return (x.mb1 ? 0 : b) * x.MH + (x.mh1 ? 0 : hd);
}

// Bitmap word of list position r (a query for the query-major bitmap, a key for the
// key-major one) against 64-wide tile t of the other axis, in mask row mrow; bit i
// is position 64t + i. Rows are padded to a multiple of 128.
__device__ __forceinline__ uint64_t mask_word(const AttnX& x, int mrow, int r, int t, int S) {
  const int64_t rows = static_cast<int64_t>((S + 127) >> 7) << 7;
  return x.bits[(mrow * rows + r) * x.cap + t];
}

// Natural-log bias the caller's mask adds to score (q, k): 0 or -inf for a bool
// mask; positions at or past S are masked.
__device__ __forceinline__ float mask_bias(const AttnX& x, int b, int hd, int q, int k, int S) {
  if (q >= S || k >= S) return -INFINITY;
  const int64_t off = (x.mb1 ? 0 : static_cast<int64_t>(b) * x.msb) +
                      (x.mh1 ? 0 : static_cast<int64_t>(hd) * x.msh) +
                      static_cast<int64_t>(q) * x.msq + k;
  if (x.fmt == TMAC_MASK_BOOL) return static_cast<const uint8_t*>(x.mask)[off] ? 0.f : -INFINITY;
  return static_cast<const float*>(x.mask)[off];
}

// Dropout decisions. Pair (bh, q, k) is kept iff the 16-bit draw k % 8 of
// Philox4x32-10 at counter {k / 8, q, bh, 0} (draw i = bits 16(i % 2).. of word
// i / 2) is at least thresh: one call decides eight consecutive keys of a row.
//
// Dropout factors (keep_scale or 0) of a lane that holds query q and, of the 16
// keys base .. base + 15 (base a multiple of 16), the keys base + 4h + t and
// base + 8 + 4h + t, t = 0..3, where lane l ^ 32 holds the same query and the
// other four of each eight (h = lane / 32): z[t] and z[4 + t]. Lane half h draws
// the eight keys base + 8h .. +7 and hands the other half the two words of draws
// it needs, so each call serves eight decisions.
__device__ __forceinline__ void drop_row8(const AttnX& x, int bh, int q, int base, int h,
                                          float (&z)[8]) {
  const U32x4 r = philox4x32_10(U32x4{static_cast<uint32_t>((base >> 3) + h),
                                      static_cast<uint32_t>(q), static_cast<uint32_t>(bh), 0u},
                                x.seed0, x.seed1);
  // words 0, 1 hold the draws of keys +0..3 of a group, words 2, 3 those of +4..7:
  // half 0 keeps words 0, 1 of group 0 and sends 2, 3; half 1 keeps words 2, 3 of
  // group 1 and sends 0, 1
  const uint32_t keep_a = h ? r.z : r.x, keep_b = h ? r.w : r.y;
  const uint32_t recv_a = static_cast<uint32_t>(__shfl_xor(static_cast<int>(h ? r.x : r.z), 32));
  const uint32_t recv_b = static_cast<uint32_t>(__shfl_xor(static_cast<int>(h ? r.y : r.w), 32));
  const uint32_t w[4] = {h ? recv_a : keep_a, h ? recv_b : keep_b,   // keys base + 4h + 0..3
                         h ? keep_a : recv_a, h ? keep_b : recv_b};  // keys base + 8 + 4h + 0..3
#pragma unroll
  for (int i = 0; i < 8; ++i)
    z[i] = ((w[i >> 1] >> (16 * (i & 1))) & 0xffffu) >= x.thresh ? x.keep_scale : 0.f;
}
// Keep bits of a lane that holds key k and two groups of four queries, qa..qa+3
// and qb..qb+3 (multiples of 4), where the eight lanes of its octet (lane & ~7 ..
// +7, all active, j = lane & 7 = k & 7) hold the eight keys of k's group with the
// same qa, qb: bit 4t of the result is the decision of (qa + t, k), bit 16 + 4t
// that of (qb + t, k). Lane j draws k's group at query qa + j (j < 4) or
// qb + j - 4 (j >= 4), so the octet's eight calls cover its 64 decisions. A lane
// of the lower quad (keys +0..3) needs words 0 and 1 of every draw, one of the
// upper quad words 2 and 3: each lane hands the other quad's two words to its
// partner lane j ^ 4, and DPP broadcasts within the quad spread them.
__device__ __forceinline__ uint32_t keep_octet2(const AttnX& x, int bh, int qa, int qb, int k, int j) {
  const int q = j < 4 ? qa + j : qb + j - 4;
  const U32x4 r = philox4x32_10(U32x4{static_cast<uint32_t>(k >> 3), static_cast<uint32_t>(q),
                                      static_cast<uint32_t>(bh), 0u},
                                x.seed0, x.seed1);
  const bool upper = j >= 4;
  const int own0 = static_cast<int>(upper ? r.z : r.x), own1 = static_cast<int>(upper ? r.w : r.y);
  const int cross0 = __shfl_xor(static_cast<int>(upper ? r.x : r.z), 4);
  const int cross1 = __shfl_xor(static_cast<int>(upper ? r.y : r.w), 4);
  const int sh = 16 * (j & 1);
  const bool second = (j & 2) != 0;  // this lane's draw is in the second of its two words
  auto bit = [&](int w0, int w1) {
    const uint32_t w = static_cast<uint32_t>(second ? w1 : w0);
    return static_cast<uint32_t>(((w >> sh) & 0xffffu) >= x.thresh);
  };
  // quad lane t of this lane's own quad drew group (upper ? b : a); via the
  // exchange, the same lane holds the other quad's lane t draw, group (upper ? a : b)
  uint32_t own = 0, other = 0;
#define TMAC_OCTET_T(t, ctl)                                                                     \
  own |= bit(__builtin_amdgcn_mov_dpp(own0, ctl, 0xf, 0xf, false),                               \
             __builtin_amdgcn_mov_dpp(own1, ctl, 0xf, 0xf, false)) << (4 * (t));                  \
  other |= bit(__builtin_amdgcn_mov_dpp(cross0, ctl, 0xf, 0xf, false),                           \
               __builtin_amdgcn_mov_dpp(cross1, ctl, 0xf, 0xf, false)) << (4 * (t));
  TMAC_OCTET_T(0, 0x00)
  TMAC_OCTET_T(1, 0x55)
  TMAC_OCTET_T(2, 0xaa)
  TMAC_OCTET_T(3, 0xff)
#undef TMAC_OCTET_T
  const uint32_t ga = upper ? other : own, gb = upper ? own : other;
  return ga | (gb << 16);
}

// Launch map of a per-(b, h) block work list whose lists differ in length.
// order[0..n_blk) names the blocks heaviest (longest list) first. Workgroup ids
// [0, n_bh * n_lead) take the n_lead heaviest blocks of every (b, h), so they
// start first and consecutive ids spread them over the XCDs; ids from lead_pad
// (n_bh * n_lead rounded up to 8) on take the remaining blocks (b, h)-major,
// each XCD on one contiguous slice as in xcd_logical_id, so that neighbouring
// blocks of one head, which share tiles, meet in that XCD's L2.
struct WorkMap {
  int n_bh, n_blk, n_lead, lead_pad, per_xcd;
};

// (bh, block) of this workgroup; false for a padding workgroup.
__device__ __forceinline__ bool work_item(const WorkMap& m, const int32_t* __restrict__ order,
                                          int& bh, int& blk) {
  const int b = blockIdx.x;
  int rank;
  if (b < m.lead_pad) {
    if (b >= m.n_bh * m.n_lead) return false;
    rank = b / m.n_bh;
    bh = b - rank * m.n_bh;
  } else {
    const int r = b - m.lead_pad;
    const int logical = (r & 7) * m.per_xcd + (r >> 3);
    const int rest = m.n_blk - m.n_lead;
    if (rest <= 0 || logical >= m.n_bh * rest) return false;
    bh = logical / rest;
    rank = m.n_lead + (logical - bh * rest);
  }
  blk = min(max(order[rank], 0), m.n_blk - 1);
  return true;
}

// out[o(e)] = Σ_{p < P} part[p * n + e] for e < n (fp32 partial sums of a
// weight gradient), o(e) = e, or with inner > 0 the transpose of an
// [n / inner, inner] row-major column index: o(e) = (e % inner) * (n / inner)
// + e / inner. Workgroup = 64 consecutive columns x 4 waves; wave w sums
// rows p ≡ w (mod 4) into 8 independent accumulators (rows p ≡ w + 4j
// (mod 32)), so each lane keeps 8 loads in flight, and the 32 partial sums of
// a column are added through LDS in a fixed order: deterministic for given
// (n, P). Launch with grid ceil(n / 64), 256 threads.
static __global__ __launch_bounds__(256) void column_sum_kernel(const float* __restrict__ part,
                                                                float* __restrict__ out,
                                                                int64_t n, int P, int64_t inner) {
  __shared__ float red[4][8][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 64 + lane;
  float acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.f;
  if (e < n) {
    int p = w;
    for (; p + 28 < P; p += 32) {
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] += part[static_cast<int64_t>(p + 4 * j) * n + e];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (p + 4 * j < P) acc[j] += part[static_cast<int64_t>(p + 4 * j) * n + e];
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) red[w][j][lane] = acc[j];
  __syncthreads();
  if (w == 0 && e < n) {
    float t = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int ww = 0; ww < 4; ++ww) t += red[ww][j][lane];
    out[inner > 0 ? (e % inner) * (n / inner) + e / inner : e] = t;
  }
}

__device__ __forceinline__ float gelu_erf(float x) {
  // erf by Abramowitz & Stegun, Handbook of Mathematical Functions, formula 7.1.26
  // (Hastings' approximation, |error| <= 1.5e-7 on erf):
  //   erf(z) = 1 - t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) exp(-z^2), t = 1 / (1 + p z),
  // for z >= 0, odd in z. Over |x| <= 12 the GELU it gives is within 5e-7 of the
  // exact one (absolute), far below the 16-bit rounding of the outputs it feeds,
  // at about a dozen instructions with one reciprocal and one exp2.
  const float z = x * 0.70710678118654752440f;
  const float az = fabsf(z);
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, az, 1.0f));
  float poly = fmaf(1.061405429f, t, -1.453152027f);
  poly = fmaf(poly, t, 1.421413741f);
  poly = fmaf(poly, t, -0.284496736f);
  poly = fmaf(poly, t, 0.254829592f) * t;
  const float e = __builtin_amdgcn_exp2f(-(az * az) * 1.4426950408889634f);
  const float erf_z = copysignf(fmaf(-poly, e, 1.0f), z);
  return 0.5f * x * (1.0f + erf_z);
}

// d/dx of gelu_erf: Φ(x) + x φ(x) = 0.5 (1 + erf(x/√2)) + x exp(-x²/2) / √(2π),
// with the same erf approximation (the exp2 term is exp(-x²/2) itself).
__device__ __forceinline__ float gelu_erf_grad(float x) {
  const float z = x * 0.70710678118654752440f;
  const float az = fabsf(z);
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, az, 1.0f));
  float poly = fmaf(1.061405429f, t, -1.453152027f);
  poly = fmaf(poly, t, 1.421413741f);
  poly = fmaf(poly, t, -0.284496736f);
  poly = fmaf(poly, t, 0.254829592f) * t;
  const float e = __builtin_amdgcn_exp2f(-(az * az) * 1.4426950408889634f);
  const float erf_z = copysignf(fmaf(-poly, e, 1.0f), z);
  return fmaf(x * 0.39894228040143268f, e, 0.5f * (1.0f + erf_z));
}

}  // namespace tmac
