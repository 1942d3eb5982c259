/*
 * tmac.h — C ABI of the TitanMAC sparse hot path for MI355X (gfx950).
 *
 * Two operations live behind this boundary:
 *   - the Block-ELL block-sparse GEMM (forward Y = X·W, dX = dY·Wᵀ, and the
 *     dW SDDMM restricted to W's non-zero blocks), which replaces the dense
 *     nn.Linear calls of the TitanMAC MLP;
 *   - windowed + persistent-token attention computed tile-sparsely, which
 *     replaces the masked F.scaled_dot_product_attention call of
 *     WindowedAttention.
 *
 * The reference (bigwolfeman/TitanMAC-Standalone) is pure Python and has no
 * FFI of its own; each entry point below cites the reference call it stands in
 * for. Paths are relative to the reference checkout.
 *
 * Conventions
 *   - Every pointer named d_* is a device pointer owned by the caller. The
 *     library never allocates, frees or synchronises the device.
 *   - Every pointer named h_* is a host pointer.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *   - Return value: 0 on success, a negative tmac_status on an argument error
 *     (nothing was launched), a positive hipError_t if a launch failed.
 *   - Strides and leading dimensions are in elements, not bytes.
 *   - Block-ELL layout (block size bs = 64):
 *       W has logical shape [K, N]; n_brow = K/64 block-rows, n_bcol = N/64
 *       block-columns. Each block-row r keeps `width` non-zero blocks whose
 *       block-column indices col_idx[r*width + s] are strictly increasing.
 *       vals[(r*width + s)*4096 + kk*64 + nn] = W[64*r + kk][64*col_idx[r][s] + nn]
 *       (each block row-major in W's own orientation).
 */
#ifndef TMAC_H
#define TMAC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TMAC_ABI_VERSION 8
#define TMAC_BLOCK 64

typedef enum {
  TMAC_OK = 0,
  TMAC_ERR_NULL = -1,      /* a required pointer is NULL */
  TMAC_ERR_SHAPE = -2,     /* a size is non-positive, not a multiple of 64, or inconsistent */
  TMAC_ERR_INDEX = -3,     /* a Block-ELL index is out of range, duplicated or unsorted */
  TMAC_ERR_DTYPE = -4,     /* unsupported dtype code */
  TMAC_ERR_ALIGN = -5,     /* a pointer or stride breaks the 16-byte vector-load alignment */
  TMAC_ERR_WORKSPACE = -6, /* workspace missing or smaller than required */
  TMAC_ERR_CAPACITY = -7,  /* an output array is too small */
  TMAC_ERR_VALUE = -8,     /* an argument value is outside its domain (reference raises ValueError) */
  TMAC_ERR_TOO_LARGE = -9  /* sizes exceed the static scratch of an allocation-free entry point */
} tmac_status;

typedef enum { TMAC_F32 = 0, TMAC_BF16 = 1, TMAC_F16 = 2 } tmac_dtype;

/* Epilogue of the forward GEMM (fused into the store). */
typedef enum { TMAC_EPI_NONE = 0, TMAC_EPI_GELU = 1 } tmac_epilogue;

/* Attention masking pattern. */
typedef enum {
  TMAC_PATTERN_BAND = 0,    /* build_band_mask: attn/windowed_attention.py:97-152 */
  TMAC_PATTERN_BLOCKWIN = 1 /* BlockSparseAttention: attn/block_sparse_attention.py:277-334 */
} tmac_pattern;

/* Format of a caller's attention mask (tmac_attn_opts.mask_format). */
typedef enum {
  TMAC_MASK_BOOL = 0,    /* uint8, nonzero = attend (the reference's bool mask) */
  TMAC_MASK_ADD_F32 = 1  /* fp32 added to the scaled scores (the reference's additive mask; -inf = masked) */
} tmac_mask_format;

/* Human-readable text for a return code (negative tmac_status or positive hipError_t). */
const char* tmac_status_string(int code);

/* ABI version compiled into the library (TMAC_ABI_VERSION). */
int tmac_abi_version(void);

/* ------------------------------------------------------------------------- */
/* Block-ELL index construction (host).                                       */
/* The reference has no Block-ELL code; its MLP is dense nn.Linear             */
/* (blocks/mlp.py:36,39). These build the sparsity pattern that replaces it.   */
/* ------------------------------------------------------------------------- */

/* Seeded sampler: for each block-row, in order, draw `width` distinct
 * block-columns by a partial Fisher-Yates shuffle driven by one splitmix64
 * stream started at `seed` (unbiased bounded draws by rejection), then sort the
 * row ascending. h_col_idx has n_brow*width entries. */
int tmac_bell_sample_col_idx(uint64_t seed, int n_brow, int n_bcol, int width,
                             int32_t* h_col_idx);

/* Check every index is in [0, n_bcol) and each row is strictly increasing. */
int tmac_bell_validate(const int32_t* h_col_idx, int n_brow, int n_bcol, int width);

/* Transposed (block-column-major) index used by the forward gather:
 * for block-column c, entries e in [t_ptr[c], t_ptr[c+1]) list the block-rows
 * t_row[e] (ascending) holding a non-zero block in column c, and
 * t_vblk[e] = t_row[e]*width + slot, the block's index into vals.
 * h_order receives the block-columns sorted by entry count, descending, ties by
 * column ascending (the forward kernel's longest-first schedule).
 * Sizes: t_ptr n_bcol+1, t_row and t_vblk n_brow*width, order n_bcol. */
int tmac_bell_transpose(const int32_t* h_col_idx, int n_brow, int n_bcol, int width,
                        int32_t* h_t_ptr, int32_t* h_t_row, int32_t* h_t_vblk,
                        int32_t* h_order);

/* Grouped schedule of the gather GEMM (host, deterministic). The output blocks
 * (block-columns for dir = 0, the forward; block-rows for dir = 1, dX) are
 * grouped `group` at a time (2 or 4) so that the members share many list
 * entries: greedily, each group seeded by the longest remaining list (lowest
 * index on ties) and filled with the remaining output sharing the most entries
 * with the group so far (then fewest new entries, then lowest index). A
 * group's steps are the union of its members' lists, ascending by input block;
 * step record = {input block, value block of member 0 .. group-1 or -1}, so a
 * member's active steps are its own list in its own order. Groups are listed
 * longest first. Output: h_grp_ptr [n_groups + 1] (step offsets), h_grp_out
 * [n_groups * group] (member output blocks, -1 pads the last group), h_steps
 * [capacity * (1 + group)]; capacity >= n_brow * width always suffices.
 * n_groups = ceil(n_out / group). No counterpart in the reference (its MLP is
 * dense); it serves tmac_bell_fwd_grouped. */
int tmac_bell_group_schedule(const int32_t* h_col_idx, int n_brow, int n_bcol, int width, int dir,
                             int group, int32_t* h_grp_ptr, int32_t* h_grp_out, int32_t* h_steps,
                             int capacity, int* n_groups, int* n_steps);

/* Geometry of the grouped forward's launch: output rows per tile, and
 * persistent workgroups per XCD (8 XCDs). */
#define TMAC_BELL_GROUP_ROWS 512
#define TMAC_BELL_GROUP_SLOTS 32

/* Balanced tile order for tmac_bell_fwd_grouped (host, deterministic). The
 * launch splits the tiles (tile = m_tile * n_groups + group, m_tile of
 * TMAC_BELL_GROUP_ROWS rows) into 8 XCD ranges of per_xcd = ceil(n_tiles / 8)
 * consecutive tiles, each served by n_slots = min(per_xcd, TMAC_BELL_GROUP_SLOTS)
 * persistent workgroups in n_rounds = ceil(per_xcd / n_slots) rounds. Per XCD,
 * each round keeps the round-robin deal's tiles (the next n_slots of the range,
 * so the tiles that run together, and share the L2, stay the same), but hands
 * them out longest first (union steps + 2) to the slots with the least work so
 * far; an XCD whose deal that does not improve keeps the round-robin one.
 * h_order[(xcd * n_rounds + round) * n_slots + slot] = tile, or -1. With h_order == NULL only *n_entries (= 8 * n_rounds * n_slots)
 * is computed. h_grp_ptr: tmac_bell_group_schedule's output for the pattern.
 * No counterpart in the reference. */
int tmac_bell_group_tile_order(const int32_t* h_grp_ptr, int n_groups, int M, int32_t* h_order,
                               int capacity, int* n_entries);

/* ------------------------------------------------------------------------- */
/* Block-ELL kernels (device).                                                */
/* ------------------------------------------------------------------------- */

/* Forward: Y[M, N] = epilogue(X[M, K] · W + bias), fp32 accumulation.
 * Replaces the dense `self.fc1(x)` / `self.fc2(hidden)` calls of
 * MLPBlock.forward (blocks/mlp.py:58,64; bias from nn.Linear, :36,39) and, with
 * epi = TMAC_EPI_GELU, also the erf GELU between them (blocks/mlp.py:42,61).
 * X, Y row-major with leading dimensions ldx, ldy; bias (nullable) has N
 * entries of the same dtype. dtype: TMAC_BF16 or TMAC_F16 (16-bit MFMA), or
 * TMAC_F32 (fp32 MFMA, for fp32 modules outside autocast; ldx, ldy multiples
 * of 4). K = 64*n_brow, N = 64*n_bcol; M >= 1 arbitrary (16-bit with M <= 64
 * runs a few-row kernel that splits each block-column's list over four waves).
 * t_ptr/t_row/t_vblk/order: device copies of tmac_bell_transpose's output. */
int tmac_bell_fwd(const void* d_X, int64_t ldx, const void* d_vals,
                  const int32_t* d_t_ptr, const int32_t* d_t_row,
                  const int32_t* d_t_vblk, const int32_t* d_order,
                  const void* d_bias, void* d_Y, int64_t ldy,
                  int M, int n_brow, int n_bcol, int width,
                  int dtype, int epi, void* stream);

/* Forward of fc1 with the erf GELU in training: Y = gelu(Z) and Z = X·W + bias
 * (the pre-activation, kept for tmac_bell_gelu_bwd), both written by the
 * forward kernel's epilogue, so the activation costs no pass of its own.
 * Replaces `self.fc1(x)` followed by `self.activation(hidden)` of
 * MLPBlock.forward when gradients are recorded (blocks/mlp.py:58,61). As
 * tmac_bell_fwd with epi = TMAC_EPI_GELU, plus Z [M, N] with leading dimension
 * ldz; any dtype of tmac_bell_fwd (16-bit: Z and Y rounded from the same fp32
 * value; TMAC_F32: Z and Y in fp32, the GELU with the device library's erff). */
int tmac_bell_fwd_gelu_aux(const void* d_X, int64_t ldx, const void* d_vals,
                           const int32_t* d_t_ptr, const int32_t* d_t_row,
                           const int32_t* d_t_vblk, const int32_t* d_order,
                           const void* d_bias, void* d_Y, int64_t ldy, void* d_Z, int64_t ldz,
                           int M, int n_brow, int n_bcol, int width, int dtype, void* stream);

/* The same forward as tmac_bell_fwd (replacing `self.fc1(x)` / `self.fc2(hidden)`
 * of MLPBlock.forward, blocks/mlp.py:58,64) through the grouped schedule:
 * pairs of block-columns sharing many block-rows, one activation-tile copy per
 * union step instead of one per stored block (-30% copied bytes at config 2),
 * persistent 512-row tiles. Bitwise-identical to tmac_bell_fwd (each output is
 * summed over its own list in the same order). 16-bit only; group must be 2;
 * d_grp_ptr/d_grp_out/d_steps: device copies of tmac_bell_group_schedule(dir 0,
 * group 2); ldx <= 2^22. Faster than tmac_bell_fwd once ceil(M/512) *
 * n_groups fills the GPU (>= 256 tiles); the Python wrapper chooses.
 * d_tile_order (nullable): a device copy of tmac_bell_group_tile_order(same
 * grp_ptr, same M), tile_order_len its n_entries (TMAC_ERR_SHAPE if another
 * length); which workgroup computes which tile changes, the results do not.
 * NULL: tiles in round-robin order within each XCD range. */
int tmac_bell_fwd_grouped(const void* d_X, int64_t ldx, const void* d_vals,
                          const int32_t* d_grp_ptr, const int32_t* d_grp_out,
                          const int32_t* d_steps, int n_groups, int group,
                          const int32_t* d_tile_order, int tile_order_len, const void* d_bias,
                          void* d_Y, int64_t ldy, int M, int n_brow, int n_bcol, int width,
                          int dtype, int epi, void* stream);

/* tmac_bell_fwd_gelu_aux through the grouped schedule (Y = gelu(Z), Z kept). */
int tmac_bell_fwd_grouped_gelu_aux(const void* d_X, int64_t ldx, const void* d_vals,
                                   const int32_t* d_grp_ptr, const int32_t* d_grp_out,
                                   const int32_t* d_steps, int n_groups, int group,
                                   const int32_t* d_tile_order, int tile_order_len,
                                   const void* d_bias, void* d_Y, int64_t ldy, void* d_Z,
                                   int64_t ldz, int M, int n_brow, int n_bcol, int width,
                                   int dtype, void* stream);

/* Bytes of device workspace tmac_bell_gelu_bwd needs for the bias gradient. */
int tmac_bell_gelu_bwd_workspace(int M, int N, size_t* ws_bytes);

/* GELU backward and bias gradient of fc1, one pass over the gradient:
 * gZ = gA ⊙ GELU'(Z) (erf form) for [M, N] row-major operands with leading
 * dimensions (N and the pitches multiples of 16 bytes: 8 elements for 16-bit,
 * 4 for fp32), and with d_dbias non-null dbias[n] = Σ_m gZ[m][n] in fp32 (of
 * gZ as stored, summed in a fixed order: deterministic; 0 when M = 0).
 * Replaces autograd's backward of nn.GELU and the bias gradient of fc1 in
 * MLPBlock's backward (blocks/mlp.py:58,61). d_ws: tmac_bell_gelu_bwd_workspace
 * bytes (needed with d_dbias only; the row operands may be null when M = 0).
 * dtype: TMAC_BF16, TMAC_F16 or TMAC_F32. */
int tmac_bell_gelu_bwd(const void* d_gA, int64_t ldga, const void* d_Z, int64_t ldz, void* d_gZ,
                       int64_t ldgz, float* d_dbias, void* d_ws, size_t ws_bytes, int M, int N,
                       int dtype, void* stream);

/* Bias gradient of a Block-ELL linear without activation (fc2):
 * dbias[n] = Σ_m gY[m][n] in fp32 over a [M, N] row-major gradient (N and the
 * pitch multiples of 16 bytes), summed in a fixed order (deterministic; 0 when
 * M = 0). Replaces the bias gradient of F.linear in MLPBlock's backward
 * (blocks/mlp.py:64). d_ws: tmac_bell_gelu_bwd_workspace(M, N) bytes. dtype:
 * TMAC_BF16, TMAC_F16 or TMAC_F32. */
int tmac_bell_bias_grad(const void* d_gY, int64_t ldgy, float* d_dbias, void* d_ws,
                        size_t ws_bytes, int M, int N, int dtype, void* stream);

/* Input gradient: dX[M, K] = dY[M, N] · Wᵀ, fp32 accumulation.
 * Replaces autograd's grad_input of F.linear in the MLP backward
 * (loss.backward() at train_titanmac_nested.py:462 through blocks/mlp.py:58,64).
 * For block-row r: dX[:, 64r:64r+64] = Σ_s dY[:, 64·col_idx[r][s] + :] · W[r,s]ᵀ.
 * d_col_idx: device copy of the row-major index. dtype as for tmac_bell_fwd. */
int tmac_bell_dx(const void* d_dY, int64_t lddy, const void* d_vals,
                 const int32_t* d_col_idx, void* d_dX, int64_t lddx,
                 int M, int n_brow, int n_bcol, int width, int dtype, void* stream);

/* Bytes of device workspace tmac_bell_sddmm needs for these sizes. */
int tmac_bell_sddmm_workspace(int M, int n_brow, int n_bcol, int width,
                              size_t* ws_bytes);

/* Weight gradient on the non-zero blocks only (SDDMM):
 * dvals[r][s][kk][nn] = Σ_m X[m][64r+kk] · dY[m][64·col_idx[r][s]+nn].
 * Replaces autograd's grad_weight = dYᵀ·X of F.linear (blocks/mlp.py:58,64),
 * restricted to the Block-ELL pattern. The M reduction is split across
 * workgroups and summed in a fixed order, so results are deterministic.
 * dvals_dtype: TMAC_F32, TMAC_BF16 or TMAC_F16 (inputs, dtype: TMAC_BF16,
 * TMAC_F16 or TMAC_F32). ws_bytes >= tmac_bell_sddmm_workspace(...) (else
 * TMAC_ERR_WORKSPACE); 16-bit inputs need ldx, lddy <= 2^25 (else TMAC_ERR_SHAPE). */
int tmac_bell_sddmm(const void* d_X, int64_t ldx, const void* d_dY, int64_t lddy,
                    const int32_t* d_col_idx, void* d_dvals, int dvals_dtype,
                    void* d_ws, size_t ws_bytes,
                    int M, int n_brow, int n_bcol, int width, int dtype, void* stream);

/* ------------------------------------------------------------------------- */
/* Windowed attention (host tile maps + device kernel).                       */
/* ------------------------------------------------------------------------- */

/* Per-tile classification of the attention mask: kind[qt*n_kt + kt] is
 * 0 (no allowed pair), 1 (every pair allowed) or 2 (some allowed) for the
 * tq × tk tile (qt, kt); positions at or beyond S count as masked.
 * The mask is build_band_mask (attn/windowed_attention.py:97-152) for
 * TMAC_PATTERN_BAND and the effective mask of BlockSparseAttention
 * (attn/block_sparse_attention.py:277-334, block size `block_size`) for
 * TMAC_PATTERN_BLOCKWIN. Raises TMAC_ERR_VALUE where build_band_mask raises
 * ValueError (n_persistent >= S, window < 0); the block-window pattern also
 * accepts n_persistent == S (a sequence of persistent tokens only), as
 * BlockSparseAttention does (attn/block_sparse_attention.py:250-267). */
int tmac_wattn_tile_kinds(int S, int window, int n_persistent, int causal,
                          int pattern, int block_size, int tq, int tk,
                          uint8_t* h_kind);

/* Work list of the attention kernel: for query block qb (q_block rows),
 * entries e in [row_ptr[qb], row_ptr[qb+1]) name every 64-wide key tile with at
 * least one allowed pair for the block, ascending. entries[e] & 0xffff is the
 * key-tile index; bits 16+2j..17+2j hold the kind (0/1/2 as above) of the
 * j-th `sub_rows`-row slice of the block against that tile.
 * q_block must be a multiple of sub_rows and q_block/sub_rows <= 8.
 * With h_entries == NULL only *n_entries is computed. */
int tmac_wattn_schedule(int S, int window, int n_persistent, int causal,
                        int pattern, int block_size, int q_block, int sub_rows,
                        int32_t* h_row_ptr, int32_t* h_entries, int capacity,
                        int* n_entries);

/* Key-major work list of the attention backward (dK, dV): for key block kb
 * (k_block keys), entries e in [col_ptr[kb], col_ptr[kb+1]) name every 64-row
 * query tile with at least one allowed pair for the block, ascending.
 * entries[e] & 0xffff is the query-tile index; bits 16+2j..17+2j hold the kind
 * (0/1/2 as in tmac_wattn_tile_kinds) of the query tile against the j-th
 * `sub_cols`-key slice of the block. k_block must be a multiple of sub_cols and
 * k_block/sub_cols <= 8. With h_entries == NULL only *n_entries is computed. */
int tmac_wattn_schedule_kv(int S, int window, int n_persistent, int causal,
                           int pattern, int block_size, int k_block, int sub_cols,
                           int32_t* h_col_ptr, int32_t* h_entries, int capacity,
                           int* n_entries);

/* The mask as the attention kernels evaluate it on partial tiles: for each
 * query row i, h_rows[3i..3i+2] = (np, lo, hi) such that i attends to key j
 * iff j < np or lo <= j <= hi; for each key j, h_cols[3j..3j+2] = (np, lo, hi)
 * such that query i attends to j iff i < np or lo <= i <= hi (the transpose,
 * used by the backward's dK/dV kernel). Same masks and errors as
 * tmac_wattn_tile_kinds; h_rows and h_cols hold 3*S entries each. */
int tmac_wattn_mask_spans(int S, int window, int n_persistent, int causal,
                          int pattern, int block_size, int32_t* h_rows,
                          int32_t* h_cols);

/* Launch order of a work list (tmac_wattn_schedule's row_ptr or
 * tmac_wattn_schedule_kv's col_ptr, n_blocks + 1 entries): h_order[0..n_blocks)
 * lists the blocks by list length, longest first (ties by block index), and
 * *n_lead counts the leading blocks whose list is at least twice the mean
 * length (the blocks of persistent tokens, which meet every key or query).
 * The attention kernels launch those n_lead blocks of every (batch, head)
 * first and spread over the XCDs, then the rest (batch, head)-major, so that
 * the longest workgroups do not start last. No counterpart in the reference
 * (the dense SDPA has no work list). */
int tmac_wattn_launch_order(const int32_t* h_ptr, int n_blocks, int32_t* h_order,
                            int* n_lead);

/* Attention forward: O = softmax(Q·Kᵀ·scale + mask)·V over the allowed pairs
 * only, fp32 accumulation and online softmax. Replaces
 * F.scaled_dot_product_attention(q, k, v, attn_mask=additive band mask,
 * is_causal=False) in WindowedAttention.forward
 * (attn/windowed_attention.py:306-323), including the per-call mask
 * conversion (:311-315).
 * Q, K, V, O: [B, H, S, dh] addressed by strides (batch, head, seq) in
 * elements, last dimension contiguous, so the chunked views of the fused qkv
 * projection (:295-304) are taken without a copy. dh: 32, 64 or 128
 * (d_model / n_heads of the reference's configs).
 * lse (nullable): fp32 [B, H, S], natural-log log-sum-exp of each row.
 * row_ptr/entries: device copies of tmac_wattn_schedule's output built with
 * q_block = 128, sub_rows = 32; order/n_lead: device copy of
 * tmac_wattn_launch_order of that row_ptr, and its lead count.
 * dtype: TMAC_BF16 / TMAC_F16 (16-bit MFMA kernels) or TMAC_F32 (fp32 MFMA kernels,
 * v_mfma_f32_32x32x2_f32). */
int tmac_wattn_fwd(const void* d_Q, const int64_t q_strides[3],
                   const void* d_K, const int64_t k_strides[3],
                   const void* d_V, const int64_t v_strides[3],
                   void* d_O, const int64_t o_strides[3], float* d_lse,
                   int B, int H, int S, int dh, int window, int n_persistent,
                   int causal, int pattern, int block_size, float scale,
                   const int32_t* d_row_ptr, const int32_t* d_entries,
                   const int32_t* d_order, int n_lead, int dtype, void* stream);

/* Attention backward: given dO, recomputes P = exp(Q·Kᵀ·scale − lse) on the
 * allowed pairs and writes
 *   dV = Pᵀ·dO,  dS = P ⊙ (dO·Vᵀ − rowsum(dO ⊙ O)),
 *   dK = scale · dSᵀ·Q,  dQ = scale · dS·K.
 * Replaces the autograd backward of the masked SDPA call in
 * WindowedAttention.forward (attn/windowed_attention.py:318-323) and of
 * BlockSparseAttention's per-block matmul/softmax loop
 * (attn/block_sparse_attention.py:277-334). Launches on `stream`, no atomics:
 * results are deterministic (16-bit: dQ, which also writes the row sums, then
 * dK/dV; fp32: row sums, dK/dV, dQ).
 * Q, K, V, O, dO, dQ, dK, dV: [B, H, S, dh] addressed by strides as in
 * tmac_wattn_fwd; dQ, dK, dV must not overlap each other or the inputs.
 * lse: fp32 [B, H, S] from tmac_wattn_fwd of the same Q, K, V and mask.
 * delta: fp32 [B, H, S] workspace (overwritten).
 * row_ptr/entries/order/n_lead: as for tmac_wattn_fwd;
 * col_ptr/entries_kv: tmac_wattn_schedule_kv with k_block = 128,
 * sub_cols = 32, order_kv/n_lead_kv: tmac_wattn_launch_order of col_ptr
 * (device copies). dtype: TMAC_BF16 / TMAC_F16 (16-bit MFMA kernels) or TMAC_F32
 * (fp32 MFMA kernels, for fp32 modules); dh: 32, 64 or 128 (the Python wrapper
 * zero-pads other head dimensions up to 128). */
int tmac_wattn_bwd(const void* d_Q, const int64_t q_strides[3],
                   const void* d_K, const int64_t k_strides[3],
                   const void* d_V, const int64_t v_strides[3],
                   const void* d_O, const int64_t o_strides[3],
                   const void* d_dO, const int64_t do_strides[3],
                   const float* d_lse, float* d_delta,
                   void* d_dQ, const int64_t dq_strides[3],
                   void* d_dK, const int64_t dk_strides[3],
                   void* d_dV, const int64_t dv_strides[3],
                   int B, int H, int S, int dh, int window, int n_persistent,
                   int causal, int pattern, int block_size, float scale,
                   const int32_t* d_row_ptr, const int32_t* d_entries,
                   const int32_t* d_order, int n_lead,
                   const int32_t* d_col_ptr, const int32_t* d_entries_kv,
                   const int32_t* d_order_kv, int n_lead_kv,
                   int dtype, void* stream);

/* Options of tmac_wattn_fwd_ex / tmac_wattn_bwd_ex: a caller's attention mask
 * and attention dropout. A zero-initialised struct (or a NULL pointer) means
 * neither: the calls then equal tmac_wattn_fwd / tmac_wattn_bwd bit for bit. */
typedef struct {
  /* Caller's mask, replacing the pattern arguments (window, n_persistent,
   * causal, pattern, block_size and the schedule arrays are then ignored and
   * may be NULL), as WindowedAttention.forward's attn_mask replaces its band
   * mask (attn/windowed_attention.py:307-315). [mask_batch, mask_heads, S, S]
   * with element strides mask_strides (batch, head, query; keys contiguous);
   * mask_batch is 1 (broadcast) or B, mask_heads 1 or H. NULL: no mask. A
   * query row with no allowed key gets output 0, lse -inf and gradients 0. */
  const void* d_mask;
  int mask_format;          /* tmac_mask_format; fp32 masks 4-byte aligned */
  int mask_batch, mask_heads;
  int64_t mask_strides[3];  /* mask_strides[2] >= S */
  /* Work lists of the mask: tmac_wattn_mask_workspace(S, mask_batch,
   * mask_heads) bytes, 256-byte aligned, filled by tmac_wattn_mask_lists from
   * this mask (on the stream, before the attention calls that use it). */
  void* d_mask_ws;
  size_t mask_ws_bytes;
  /* Attention dropout after the softmax, F.scaled_dot_product_attention's
   * dropout_p (attn/windowed_attention.py:318-323) and
   * BlockSparseAttention's F.dropout of the weights
   * (attn/block_sparse_attention.py:196-197): each probability of (b, h, q, k)
   * is kept with probability 1 - p (to within 2^-16) and scaled by the
   * inverse of its keep probability; the row sums (lse) use the undropped
   * probabilities. The keep decision is a 16-bit draw of Philox 4x32-10
   * (Salmon et al., SC 2011) at counter {k / 8, q, b * H + h, 0} under key
   * {seed low 32 bits, seed high 32 bits}: draw k % 8 (bits 16 * (k % 2) ..
   * of word (k % 8) / 2), kept iff draw >= t = floor(p * 2^16), and kept
   * entries are scaled by 2^16 / (2^16 - t). The same seed gives the same mask
   * in forward and backward. 0 <= p < 1. */
  float dropout_p;
  uint64_t dropout_seed;
  /* Gradient of an additive mask (tmac_wattn_bwd_ex only; NULL: none), as
   * F.scaled_dot_product_attention differentiates a float attn_mask
   * (attn/windowed_attention.py:311-323): the backward writes, as fp32 into
   * d_mask_grad [B, H, S, S] (contiguous), dS[b, h, q, k] = dL/d(score) of
   * every pair in a 64-key tile that holds an allowed pair of q's 32-row slice;
   * the other entries (all-masked tiles, whose gradient is 0) are not written,
   * so the caller zero-fills the buffer first. Summing over broadcast mask
   * dimensions: tmac_wattn_mask_grad_reduce. TMAC_MASK_ADD_F32 masks only
   * (a bool mask, or no mask, with d_mask_grad returns TMAC_ERR_VALUE). */
  float* d_mask_grad;
} tmac_attn_opts;

/* The gradient of a broadcast additive mask from tmac_wattn_bwd_ex's per-head
 * d_mask_grad: d_out[mb][mh][q][k] = sum over the (b, h) that mask row
 * (mb, mh) serves of d_ds[b][h][q][k], in ascending b, then h (a fixed order:
 * the same bits on every call). mask_batch is 1 or B, mask_heads 1 or H; d_out
 * [mask_batch, mask_heads, S, S] fp32, contiguous; d_out may not overlap d_ds.
 * No counterpart in the reference (autograd sums the broadcast dimensions of
 * SDPA's mask gradient). */
int tmac_wattn_mask_grad_reduce(const float* d_ds, int B, int H, int S, int mask_batch,
                                int mask_heads, float* d_out, void* stream);

/* Bytes of the work-list workspace of a mask of [mask_batch, mask_heads, S, S];
 * 0 for a non-positive argument. No counterpart in the reference (which masks
 * dense scores): lists of the 64-wide tiles each 128-row block visits. */
size_t tmac_wattn_mask_workspace(int S, int mask_batch, int mask_heads);

/* Builds the work lists of opts->d_mask into opts->d_mask_ws on `stream`
 * (device work only, no host synchronisation): per (mask row, 128-query
 * block) the 64-key tiles holding an allowed pair, and per (mask row,
 * 128-key block) the 64-query tiles, each with a 2-bit kind per 32-wide
 * slice (0 none allowed, 1 all allowed with bias 0, 2 mixed). Run it once per
 * mask; forward and backward calls with that mask then reuse the lists. */
int tmac_wattn_mask_lists(const tmac_attn_opts* opts, int S, void* stream);

/* tmac_wattn_fwd with options (tmac_attn_opts): a caller's mask and/or
 * dropout. Same kernels, templated on the options. */
int tmac_wattn_fwd_ex(const void* d_Q, const int64_t q_strides[3],
                      const void* d_K, const int64_t k_strides[3],
                      const void* d_V, const int64_t v_strides[3],
                      void* d_O, const int64_t o_strides[3], float* d_lse,
                      int B, int H, int S, int dh, int window, int n_persistent,
                      int causal, int pattern, int block_size, float scale,
                      const int32_t* d_row_ptr, const int32_t* d_entries,
                      const int32_t* d_order, int n_lead, int dtype, void* stream,
                      const tmac_attn_opts* opts);

/* tmac_wattn_bwd with options; the options (mask, dropout_p, dropout_seed)
 * must be those of the forward whose lse is passed. With dropout, P·Z (Z the
 * keep-and-scale factors) replaces P in dV = (P·Z)ᵀ·dO and
 * dS = P ⊙ (Z ⊙ dO·Vᵀ − rowsum(dO ⊙ O)). */
int tmac_wattn_bwd_ex(const void* d_Q, const int64_t q_strides[3],
                      const void* d_K, const int64_t k_strides[3],
                      const void* d_V, const int64_t v_strides[3],
                      const void* d_O, const int64_t o_strides[3],
                      const void* d_dO, const int64_t do_strides[3],
                      const float* d_lse, float* d_delta,
                      void* d_dQ, const int64_t dq_strides[3],
                      void* d_dK, const int64_t dk_strides[3],
                      void* d_dV, const int64_t dv_strides[3],
                      int B, int H, int S, int dh, int window, int n_persistent,
                      int causal, int pattern, int block_size, float scale,
                      const int32_t* d_row_ptr, const int32_t* d_entries,
                      const int32_t* d_order, int n_lead,
                      const int32_t* d_col_ptr, const int32_t* d_entries_kv,
                      const int32_t* d_order_kv, int n_lead_kv,
                      int dtype, void* stream, const tmac_attn_opts* opts);

/* Rows of the static scratch of tmac_wattn_bwd_noalloc (B*H*S at most). */
#define TMAC_WATTN_BWD_SCRATCH_ROWS (4 * 1024 * 1024)

/* tmac_wattn_bwd without the delta workspace argument: the fp32 row sums go to a
 * static device array inside the library (16 MiB per GPU, held until the
 * process ends), so the call allocates nothing and needs no workspace from the
 * caller. No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving or
 * training loops, harnesses that forbid hipMalloc). Same arguments, kernels and
 * results (bit for bit) as tmac_wattn_bwd. Returns TMAC_ERR_TOO_LARGE when
 * B*H*S > TMAC_WATTN_BWD_SCRATCH_ROWS (nothing launched). Every call on one GPU
 * shares that GPU's scratch: calls that overlap on one GPU (concurrent streams,
 * threads) race and must be serialised by the caller. The scratch's device
 * address is looked up once per device, on the first call with that device
 * current; the stream must belong to the current device (a stream of another
 * device returns TMAC_ERR_VALUE, nothing launched). */
int tmac_wattn_bwd_noalloc(const void* d_Q, const int64_t q_strides[3],
                           const void* d_K, const int64_t k_strides[3],
                           const void* d_V, const int64_t v_strides[3],
                           const void* d_O, const int64_t o_strides[3],
                           const void* d_dO, const int64_t do_strides[3],
                           const float* d_lse,
                           void* d_dQ, const int64_t dq_strides[3],
                           void* d_dK, const int64_t dk_strides[3],
                           void* d_dV, const int64_t dv_strides[3],
                           int B, int H, int S, int dh, int window, int n_persistent,
                           int causal, int pattern, int block_size, float scale,
                           const int32_t* d_row_ptr, const int32_t* d_entries,
                           const int32_t* d_order, int n_lead,
                           const int32_t* d_col_ptr, const int32_t* d_entries_kv,
                           const int32_t* d_order_kv, int n_lead_kv,
                           int dtype, void* stream);

/* ------------------------------------------------------------------------- */
/* Causal depthwise convolution (device).                                     */
/* ------------------------------------------------------------------------- */

/* out[b, t, c] = Σ_{j<ksize} w[c][j] · in[b, t - (ksize-1) + j, c], with rows
 * before t = 0 taken as zero; fp32 accumulation, output in the input dtype.
 * Replaces BlockSparseAttention's causal depthwise Conv1d on q, k and v
 * (nn.Conv1d(d, d, ksize, padding=ksize-1, groups=d, bias=False) on the
 * [B, d, T] transpose, trimmed to T outputs: attn/block_sparse_attention.py
 * :87-98, :227-241), on the [B, T, C] layout without transposes; q, k and v
 * go through one launch as C = 3d channels of the fused projection.
 * in / out: [B, T, C] with row strides ld_in / ld_out (elements; batch stride
 * T * ld); w: [C, ksize] in the same dtype. 1 <= ksize <= 8; C and the row
 * strides multiples of 8 (16-bit) or 4 (fp32); in and out 16-byte aligned and
 * not overlapping. dtype: TMAC_F32, TMAC_BF16 or TMAC_F16. */
int tmac_dwconv_causal(const void* d_in, int64_t ld_in, const void* d_w, void* d_out,
                       int64_t ld_out, int B, int T, int C, int ksize, int dtype, void* stream);

/* Bytes of device workspace tmac_dwconv_causal_bwd needs for these sizes. */
int tmac_dwconv_causal_bwd_workspace(int B, int T, int C, int ksize, size_t* ws_bytes);

/* Backward of tmac_dwconv_causal:
 *   d_in[b, t, c] = Σ_j w[c][j] · d_out[b, t + (ksize-1) - j, c]  (rows past T zero)
 *   dw[c][j]     = Σ_{b, t} d_out[b, t, c] · in[b, t - (ksize-1) + j, c]
 * Replaces autograd's input and weight gradients of the three depthwise
 * Conv1d calls of BlockSparseAttention (attn/block_sparse_attention.py
 * :234-236). d_out, in, d_in: [B, T, C] with row strides ld_dout, ld_in,
 * ld_din, same dtype and alignment rules as tmac_dwconv_causal; w: [C, ksize]
 * in that dtype; dw: fp32 [C, ksize], overwritten (not accumulated). The
 * weight gradient is summed per 64-position chunk into the workspace, then
 * over the chunks in a fixed order, so it is deterministic. */
int tmac_dwconv_causal_bwd(const void* d_dout, int64_t ld_dout, const void* d_in,
                           int64_t ld_in, const void* d_w, void* d_din, int64_t ld_din,
                           float* d_dw, void* d_ws, size_t ws_bytes, int B, int T, int C,
                           int ksize, int dtype, void* stream);

/* ------------------------------------------------------------------------- */
/* RMSNorm (device).                                                          */
/* ------------------------------------------------------------------------- */

/* y[m, :] = x[m, :] · r[m] · scale,  r[m] = 1 / sqrt(mean(x[m, :]²) + eps),
 * fp32 arithmetic, y in the input dtype. Replaces RMSNorm.forward
 * (blocks/norms.py:44-62), TitanBlock's two pre-norms
 * (blocks/titan_block.py:46-47,91,96). x, y: [M, D] with row strides ldx, ldy;
 * scale: [D] in the same dtype; rstd (nullable): fp32 [M] receives r (what the
 * backward needs). 1 <= D <= 4096, D and the row strides multiples of 8
 * (16-bit) or 4 (fp32); pointers 16-byte aligned. dtype: TMAC_F32, TMAC_BF16
 * or TMAC_F16. */
int tmac_rmsnorm_fwd(const void* d_x, int64_t ldx, const void* d_scale, void* d_y,
                     int64_t ldy, float* d_rstd, int M, int D, float eps, int dtype,
                     void* stream);

/* Bytes of device workspace tmac_rmsnorm_bwd needs for these sizes. */
int tmac_rmsnorm_bwd_workspace(int M, int D, size_t* ws_bytes);

/* Backward of tmac_rmsnorm_fwd (autograd of blocks/norms.py:58-62):
 *   dx = r·(dy ⊙ scale) − x · r³ · mean(dy ⊙ scale ⊙ x),
 *   dscale = Σ_m dy[m, :] ⊙ x[m, :] · r[m]  (fp32 [D], overwritten).
 * rstd from the forward. dscale is summed per 64 rows into the workspace, then
 * over those partials in a fixed order, so it is deterministic. */
int tmac_rmsnorm_bwd(const void* d_dy, int64_t lddy, const void* d_x, int64_t ldx,
                     const void* d_scale, const float* d_rstd, void* d_dx, int64_t lddx,
                     float* d_dscale, void* d_ws, size_t ws_bytes, int M, int D, int dtype,
                     void* stream);

/* ------------------------------------------------------------------------- */
/* Titans neural memory: update of the memory MLP (device).                   */
/* ------------------------------------------------------------------------- */

#define TMAC_MEM_MAX_TENSORS 16

/* Clip rule of tmac_mem_update. */
typedef enum {
  /* NeuralMemory.update (memory/neural_memory.py:391-409): scale = max_norm/norm
   * only when norm > max_norm (the clipped gradient is written back into the
   * gradient tensors, as the reference's in-place mul_ does); the whole update
   * is skipped when any gradient is NaN or Inf. */
  TMAC_MEM_CLIP_MEMORY = 0,
  /* fused_clip_momentum_update (kernels/memory_mlp.py:129-131): scale =
   * min(1, max_norm / (norm + 1e-8)), never skipped, gradients left as they are. */
  TMAC_MEM_CLIP_KERNEL = 1
} tmac_mem_clip_mode;

/* Bytes of device workspace tmac_mem_update needs for these tensor sizes
 * (8 bytes per workgroup of the launch; at most 4 KB). */
int tmac_mem_update_workspace(const int64_t* sizes, int n_tensors, size_t* ws_bytes);

/* The Titans memory step over n_tensors (<= TMAC_MEM_MAX_TENSORS) parameter
 * tensors, elementwise on tensor i's sizes[i] contiguous elements:
 *   norm = ||g||₂ over all tensors, g' = g · scale(norm, mode),
 *   S ← η·S − θ·g',  W ← (1 − α)·W + S,  mirror (if given) ← W.
 * Replaces NeuralMemory.update's flatten / norm / clip / NaN check / momentum /
 * parameter steps (memory/neural_memory.py:386-434) and the Triton
 * fused_clip_momentum_update with its norm (kernels/memory_mlp.py:51-154,
 * 233-252). Two launches on `stream`, no host synchronisation: α (forget gate)
 * and η (decay gate) are read from device scalars d_alpha, d_eta (fp32).
 * d_grads/d_moms/d_weights/d_mirrors: host arrays of n_tensors device pointers
 * (d_mirrors and its entries nullable), all of `dtype` (TMAC_F32/BF16/F16,
 * fp32 arithmetic). d_norm (nullable): a device fp32 norm to use instead of
 * computing ||g|| (fused_clip_momentum_update's grad_norm argument); then one
 * launch and no workspace, and in TMAC_MEM_CLIP_MEMORY mode the skip test is
 * "norm not finite". d_stats: fp32 [4] receives norm, scale, skipped (0/1),
 * clipped (0/1). The norm is summed per workgroup and re-added in a fixed
 * order: deterministic. Calls that share a workspace must not overlap. */
int tmac_mem_update(void* const* d_grads, void* const* d_moms, void* const* d_weights,
                    void* const* d_mirrors, const int64_t* sizes, int n_tensors,
                    const float* d_alpha, const float* d_eta, const float* d_norm, float theta,
                    float max_norm, int mode, float* d_stats, void* d_ws, size_t ws_bytes,
                    int dtype, void* stream);

/* dz = dh · σ(z)·(1 + z·(1 − σ(z))) over n contiguous elements: the SiLU
 * backward of the memory MLP's hand-written gradient (silu_backward,
 * kernels/memory_mlp.py:28-44, memory/manual_backward.py:26-41). */
int tmac_silu_bwd(const void* d_dh, const void* d_z, void* d_dz, int64_t n, int dtype,
                  void* stream);

/* dy = coef · (y − v) over n contiguous elements: the MSE gradient that starts
 * the memory MLP's backward, coef = 2 / numel (kernels/memory_mlp.py:215-218). */
int tmac_mse_grad(const void* d_y, const void* d_v, void* d_dy, int64_t n, float coef, int dtype,
                  void* stream);

#ifdef __cplusplus
}
#endif
#endif /* TMAC_H */
