/*
 * polylora_hip.h — C ABI of the MI355X (gfx950) multi-LoRA SGMV library.
 *
 * Every entry point is `extern "C"`, takes plain pointers, sizes and a
 * hipStream_t (passed as `void*`), enqueues asynchronously on that stream and
 * returns 0 on success or a nonzero PL_ERR_* code; `pl_last_error()` returns
 * the message of the last failure on the calling thread.  No entry point
 * allocates device memory: every buffer is owned by the caller.
 *
 * Reference interfaces replaced (Knowledgator/PolyLoRA, paths relative to the
 * repository root):
 *   pl_sgmv_lora_a_ref  <- src/polylora/sgmv.py:141-175  sgmv_lora_a_fwd
 *   pl_sgmv_lora_b_ref  <- src/polylora/sgmv.py:278-328  sgmv_lora_b_fwd
 *   pl_sgmv_ref_workspace_bytes
 *                          (size of their MFMA path's workspace; the Triton
 *                          kernels of the reference allocate nothing)
 *   pl_sgmv_lora_a_ref_parts, pl_sgmv_lora_b_ref_parts, pl_sgmv_ref_part_bytes
 *                       <- the same two calls with the plan and the
 *                          repacked weights kept by the caller across calls
 *   pl_plan_build       <- src/polylora/sgmv.py:29-61    _build_flat_schedule
 *                          (one device-side plan per forward instead of a
 *                          host-synchronising schedule per layer)
 *   pl_sgmv_shrink      <- src/polylora/sgmv.py:63-138   _sgmv_lora_a_kernel
 *   pl_shrink_planes, pl_shrink_workspace_bytes
 *                          (sizes of the shrink -> expand workspace)
 *   pl_sgmv_expand      <- src/polylora/sgmv.py:178-275  _sgmv_lora_b_kernel
 *   pl_sgmv_shrink_stacked, pl_sgmv_expand_stacked
 *                       <- the same for sibling Linears in one launch each
 *                          (sgmv.py:141-175 stack_num reads x once)
 *   pl_lora_apply       <- src/polylora/layers.py:42-53  (shrink then expand,
 *                          the LoRA half of MultiLoraLinear.forward)
 *   pl_lora_decode_stacked <- src/polylora/sgmv.py:63-138 and :178-275 in one
 *                          launch for decode-sized batches (the pair of
 *                          Triton kernels of layers.py:45-53, split-K with a
 *                          hand-off inside the launch)
 *   pl_decode_counter_ints (size of its hand-off counters)
 *   pl_lora_fused       <- src/polylora/sgmv.py:63-138 and :178-275 in one
 *                          launch (both Triton kernels of layers.py:45-53)
 *   pl_lora_fused_stacked <- the same for sibling Linears in one launch
 *                          (sgmv.py:141-175 stack_num reads x once)
 *   pl_slot_upload      <- src/polylora/cache.py:119-150 _load_adapter_into_slot
 *                          (host->device copy of one adapter into a slot)
 *   pl_host_copy_async  <- the same for an image in pageable memory: its
 *                          copy into page-locked staging, in stream order
 *   pl_check_right_padded <- src/polylora/context.py:37-45 assert_right_padded
 */
#ifndef POLYLORA_HIP_H
#define POLYLORA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types of x, y and the adapter weights */
enum pl_dtype { PL_F32 = 0, PL_BF16 = 1, PL_F16 = 2 };

/* epilogue rounding order of the expand (scale and add-back) */
enum pl_epilogue {
  /* layers.py:127-128: d = T(acc); d = T(d * T(scale)); y = T(y + d) */
  PL_EPI_FALLBACK = 0,
  /* sgmv.py:268-275:   y = T(T(acc * scale) + y) */
  PL_EPI_TRITON = 1
};

enum pl_status {
  PL_OK = 0,
  PL_ERR_ARG = 1,     /* invalid argument (null pointer, bad size, bad dtype) */
  PL_ERR_ALIGN = 2,   /* shape or pointer alignment not supported by the tiled path */
  PL_ERR_LAUNCH = 3,  /* kernel launch or HIP runtime failure */
  PL_ERR_LIMIT = 4    /* a size exceeds a documented maximum */
};

/* One entry per (slot, module) of the slot table, 32 bytes.  The table is a
 * device array laid out [num_slots][num_modules].  Slot 0 is the base
 * adapter and always has rank 0.  `a_off` points (bytes from the arena base)
 * at the adapter's A for this module, an [rank][in_features] matrix; `b_off`
 * points at B, an [out_features][rank8] matrix where rank8 = rank rounded up
 * to a multiple of 8 and columns rank..rank8-1 are 0.  Both are stored in
 * MFMA blocks: an [R][C] matrix is cut into tiles of 16 rows (the last tile
 * has rt = min(16, R - 16t) rows), and each tile is stored as its column
 * blocks of W = 64 bytes (32 bf16/f16 or 16 f32 elements; the last block is
 * wb = min(W, C - sW) wide), one after the other, each row-major:
 *   element (i, c) at 16*t*C + s*rt*W + (i % 16)*wb + (c - s*W),
 *   t = i / 16, s = c / W.
 * A 16-row x 64-byte MFMA operand load then reads contiguous memory.  For
 * C <= W (e.g. B of ranks up to 32 in bf16) this is plain row-major.
 * Replaces the per-module A/B/ranks/scales tensors of cache.py:37-58. */
typedef struct pl_slot_entry {
  int32_t rank;
  float scale;  /* lora_alpha / rank, fp32 (store.py:252) */
  int32_t rank8;
  int32_t reserved;
  int64_t a_off;
  int64_t b_off;
} pl_slot_entry;

/* One group of at most `group_tokens` tokens that all use the same slot.
 * `start` indexes the sorted token list written by pl_plan_build. */
typedef struct pl_group {
  int32_t slot;
  int32_t start;
  int32_t len;
  int32_t reserved;
} pl_group;

/* Modules one pl_sgmv_shrink_stacked launch can serve. */
#define PL_MAX_STACKED_MODULES 4

/* Maximum slot count accepted by pl_plan_build (slot 0 included). */
#define PL_MAX_SLOTS 4096
/* Token-group sizes of a plan: short groups for short adapter segments
 * (decode), long groups for long segments (prefill).  The tiled kernels are
 * called with the group size of the plan they walk. */
#define PL_GROUP_TOKENS_SHORT 16
#define PL_GROUP_TOKENS_LONG 64

/* Library version (major*10000 + minor*100 + patch). */
int pl_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* pl_last_error(void);

/* 1 if `ptr` is a device (or managed) pointer visible to the current HIP
 * device, 0 if not, negative on a runtime error.  Used at load time to check
 * that the caller's allocator and this library share one HIP runtime. */
int pl_is_device_pointer(const void* ptr);

/* Group records a plan for `rows` rows of `row_len` tokens over `num_slots`
 * slots needs: at most n = ceil(rows*row_len/group_tokens) + num_slots - 1
 * groups, placed below 8 * ceil(n / 8). */
int64_t pl_plan_group_capacity(int32_t rows, int32_t row_len, int32_t num_slots,
                               int32_t group_tokens);

/* Build the per-forward adapter-major plan on the device.
 *   row_slot[rows]  int32 slot of each row (weight_indices, cache.py:77-84)
 *   seq_lens[rows]  int32 valid length of each row; the row contributes
 *                   min(max(seq_len,0), row_len) tokens (layers.py:127 slicing)
 *   group_tokens    16 or 64: tokens per group at most
 *   tok[rows*row_len]          out: token indices (row*row_len + m), grouped by slot
 *   groups[group_cap]          out: pl_group records
 *   meta[4]                    out: {num_groups, num_tokens, group_tokens,
 *                                    positions = 8 * ceil(num_groups / 8)}
 * Rows with slot 0, slot >= num_slots, slot < 0 or length 0 are skipped.
 * Token order inside one slot is unspecified; every consumer is order-free.
 * Placement: the kernels give the work of the record at position p to XCD
 * p % 8, so the slot-major list of the n groups is cut into 8 contiguous
 * chunks, chunk x = groups [x*n/8, (x+1)*n/8), and the i-th group of chunk
 * x is stored at position 8*i + x: an adapter's groups share one or two XCDs'
 * L2.  Every other record below group_cap is empty (slot 0, length 0).
 *
 * Plan inputs of the kernels.  Every entry point below that takes tok,
 * groups and meta (pl_sgmv_shrink(_stacked), pl_sgmv_expand(_stacked),
 * pl_lora_apply, pl_lora_fused(_stacked), pl_lora_decode_stacked) reads
 * them as pl_plan_build or pl_plan_build_active wrote them: it walks the
 * group positions below meta[3] (records past the groups in use are empty)
 * and gives position p to XCD p % 8.  A plan built another way must follow
 * that format, meta[3] included: with meta[3] = 0 no group is read and the
 * call adds no LoRA delta. */
int pl_plan_build(const int32_t* row_slot, const int32_t* seq_lens, int32_t rows,
                  int32_t row_len, int32_t num_slots, int32_t group_tokens, int32_t* tok,
                  pl_group* groups, int32_t* meta, int64_t group_cap, void* stream);

/* pl_plan_build for one module's launches: rows whose slot s has
 * slot_active[s * active_stride] <= 0 (e.g. the module's rank column of the
 * slot table, which is 0 for slots whose adapter lacks the module) are left
 * out like base rows, so they take no group positions and the groups of the
 * slots with work are spread evenly over the XCDs.  Such a plan serves only
 * launches for which those rows need no work. */
int pl_plan_build_active(const int32_t* row_slot, const int32_t* seq_lens, int32_t rows,
                         int32_t row_len, int32_t num_slots, const int32_t* slot_active,
                         int64_t active_stride, int32_t group_tokens, int32_t* tok,
                         pl_group* groups, int32_t* meta, int64_t group_cap, void* stream);

/* Number of K splits pl_sgmv_shrink uses for a requested count: the K range
 * is cut into at most k_splits pieces of whole MFMA steps. */
int32_t pl_shrink_planes(int32_t dtype, int32_t K, int32_t k_splits, int32_t group_tokens);

/* Bytes of the workspace `ws` that pl_sgmv_shrink / pl_lora_apply need for
 * these sizes: fp32 partial planes [planes][tmp_rows][ldt]. */
int64_t pl_shrink_workspace_bytes(int32_t dtype, int32_t K, int32_t k_splits,
                                  int32_t group_tokens, int64_t tmp_rows, int32_t ldt);

/* Shrink: planes[c][p][j] = sum_{k in split c} x[tok[p]][k] * A_slot[j][k]
 * for every planned token position p, j < rank(slot, module) and split
 * c < pl_shrink_planes(dtype, K, k_splits).  fp32 accumulation, plain stores
 * (no atomics); entries outside (p, j < rank) are not written and nothing
 * needs clearing between calls.
 *   x [*, ldx] of dtype; K = in_features
 *   tok, groups, meta, group_cap: a plan of pl_plan_build or
 *     pl_plan_build_active (group positions below meta[3] are read)
 *   group_tokens: the group size the plan was built with (16 or 64)
 *   ws / ws_bytes: at least pl_shrink_workspace_bytes(...) bytes
 *   tmp_rows >= the plan's token count; ldt a multiple of 8 and >= every
 *     rank8 of this module.
 * Requires K % 8 == 0 (bf16/f16) or K % 4 == 0 (f32) and 16-byte aligned x
 * rows and arena parts; otherwise returns PL_ERR_ALIGN. */
int pl_sgmv_shrink(int32_t dtype, const void* x, int64_t ldx, int32_t K, const void* arena,
                   const pl_slot_entry* table, int32_t num_modules, int32_t module,
                   const int32_t* tok, const pl_group* groups, const int32_t* meta,
                   int64_t group_cap, int32_t group_tokens, void* ws, int64_t ws_bytes,
                   int32_t ldt, int64_t tmp_rows, int32_t k_splits, void* stream);

/* Shrink for up to PL_MAX_STACKED_MODULES wrapped Linears that read the same
 * x (e.g. q/k/v or gate/up projections): one launch, x read once per group
 * and split, module j's planes written to its own workspace ws[j] (each at
 * least pl_shrink_workspace_bytes(...) bytes and distinct).  modules[] and
 * ws[] are host arrays of n_modules entries; every other argument is as for
 * pl_sgmv_shrink, which is this call with one module.  No counterpart in the
 * reference, whose sgmv_lora_a_fwd (sgmv.py:141-175) serves one weight
 * tensor per call (its stack_num packs modules along N instead). */
int pl_sgmv_shrink_stacked(int32_t dtype, const void* x, int64_t ldx, int32_t K, const void* arena,
                           const pl_slot_entry* table, int32_t num_modules, int32_t n_modules,
                           const int32_t* modules, void* const* ws, const int32_t* tok,
                           const pl_group* groups, const int32_t* meta, int64_t group_cap,
                           int32_t group_tokens, int64_t ws_bytes, int32_t ldt, int64_t tmp_rows,
                           int32_t k_splits, void* stream);

/* Expand: y[tok[p]][n] = T(y + d), d = scale * sum_{j<rank} T(sum_c
 * planes[c][p][j]) * B_slot[n][j] rounded in the order of `epilogue`; the
 * `planes` partial sums the shrink left in `ws` are added in split order, so
 * results are bitwise reproducible.  y [*, ldy] of dtype; requires
 * N % 8 == 0 (bf16/f16) or N % 4 == 0 (f32) and 16-byte aligned y rows.
 * The plan (tok, groups, meta, group_cap) is the one the shrink walked, in
 * the format of pl_plan_build. */
int pl_sgmv_expand(int32_t dtype, const void* ws, int32_t ldt, int64_t tmp_rows, int32_t planes,
                   const void* arena, const pl_slot_entry* table, int32_t num_modules,
                   int32_t module, const int32_t* tok, const pl_group* groups,
                   const int32_t* meta, int64_t group_cap, int32_t group_tokens, void* y,
                   int64_t ldy, int32_t N, int32_t epilogue, void* stream);

/* Expand for up to PL_MAX_STACKED_MODULES modules in one launch: module i
 * reads the planes in ws[i] (left by a shrink of the same plan, K split and
 * ldt, e.g. pl_sgmv_shrink_stacked) and adds its delta into y[i] [*, ldy[i]]
 * of N[i] columns, each as pl_sgmv_expand would.  For sibling Linears whose
 * base outputs all exist before any of them is read (q/k/v, gate/up). */
int pl_sgmv_expand_stacked(int32_t dtype, void* const* ws, int32_t ldt, int64_t tmp_rows,
                           int32_t planes, const void* arena, const pl_slot_entry* table,
                           int32_t num_modules, int32_t n_modules, const int32_t* modules,
                           const int32_t* tok, const pl_group* groups, const int32_t* meta,
                           int64_t group_cap, int32_t group_tokens, void* const* y,
                           const int64_t* ldy, const int32_t* N, int32_t epilogue, void* stream);

/* Shrink and expand of 1..PL_MAX_STACKED_MODULES sibling Linears in ONE
 * launch, for plans of 16-token groups (decode): module modules[i] adds the
 * LoRA delta of x [*, ldx] (K columns) into y[i] [*, ldy[i]] of N[i]
 * columns, bitwise equal to pl_sgmv_shrink_stacked followed by
 * pl_sgmv_expand_stacked with the same ws, k_splits and epilogue.  The
 * shrink workgroups come first in the grid and write their fp32 partial
 * planes to ws[i] with agent-scope stores; each expand workgroup waits until
 * every shrink workgroup of its (group, module) has arrived on a counter in
 * `counters`, then reads the planes.  ldt must be a multiple of 32 here (so
 * that no 128-byte line of the planes holds rows of two groups).  `counters`
 * holds counter_ints >= pl_decode_counter_ints(group_cap, n_modules) int32s,
 * must be all zero before the first call and is all zero again after each
 * call whose waits all end in time (the last reader of each counter resets
 * it), so it is reused call after call without a clear; calls that share it
 * must not overlap (one stream).  A wait gives up after spin_limit (>= 1)
 * polls of its counter and then sets counters[0] (the status word) to 1:
 * the results of that call are undefined, and a shrink workgroup that
 * arrives after the wait gave up can leave its counter above zero, so the
 * caller must zero all counter_ints words (with no call in flight) before
 * the next call; otherwise the status word stays 0.  Every other argument
 * is as for pl_sgmv_shrink_stacked and pl_sgmv_expand_stacked. */
int pl_lora_decode_stacked(int32_t dtype, const void* x, int64_t ldx, int32_t K, const void* arena,
                           const pl_slot_entry* table, int32_t num_modules, int32_t n_modules,
                           const int32_t* modules, void* const* ws, const int32_t* tok,
                           const pl_group* groups, const int32_t* meta, int64_t group_cap,
                           int32_t group_tokens, int64_t ws_bytes, int32_t ldt, int64_t tmp_rows,
                           int32_t k_splits, void* const* y, const int64_t* ldy, const int32_t* N,
                           int32_t epilogue, int32_t* counters, int64_t counter_ints,
                           int32_t spin_limit, void* stream);

/* int32 words of hand-off counters pl_lora_decode_stacked needs: 64 per
 * counter (one 256-byte line each), for the status and group_cap * n_modules
 * counters. */
int64_t pl_decode_counter_ints(int64_t group_cap, int32_t n_modules);

/* Shrink followed by expand on one stream (one call per wrapped Linear),
 * over a plan in the format of pl_plan_build. */
int pl_lora_apply(int32_t dtype, const void* x, int64_t ldx, int32_t K, void* y, int64_t ldy,
                  int32_t N, const void* arena, const pl_slot_entry* table,
                  int32_t num_modules, int32_t module, const int32_t* tok,
                  const pl_group* groups, const int32_t* meta, int64_t group_cap,
                  int32_t group_tokens, void* ws, int64_t ws_bytes, int32_t ldt,
                  int64_t tmp_rows, int32_t k_splits, int32_t epilogue, void* stream);

/* Fused shrink + expand in one launch for long adapter segments: one
 * workgroup per (16-token tile of a plan group, column slice) computes
 * t = T(x·Aᵀ) over all of K and then y[tok[p]][n] = T(y + d) over its
 * columns, d rounded in the order of `epilogue`.  No workspace.  Takes slot
 * ranks up to 64 (ldt, the table's rank capacity, must be <= 64), 1..8
 * column slices per tile (each slice recomputes the tile's shrink; more
 * slices, more workgroups), the alignment rules of the tiled path, and a
 * plan of 16- or 64-token groups in the format of pl_plan_build (positions
 * below meta[3] are read).  Pays off when groups are full (many
 * tokens per adapter); for a few tokens per adapter (decode) use
 * pl_sgmv_shrink + pl_sgmv_expand, which split K and N over many
 * workgroups. */
int pl_lora_fused(int32_t dtype, const void* x, int64_t ldx, int32_t K, void* y, int64_t ldy,
                  int32_t N, const void* arena, const pl_slot_entry* table, int32_t num_modules,
                  int32_t module, int32_t ldt, const int32_t* tok, const pl_group* groups,
                  const int32_t* meta, int64_t group_cap, int32_t group_tokens, int32_t slices,
                  int32_t epilogue, void* stream);

/* pl_lora_fused for 1..PL_MAX_STACKED_MODULES sibling Linears fed the same
 * x [*, ldx] (K columns): module modules[i] adds into y[i] [*, ldy[i]] of
 * N[i] columns.  A tile's modules run side by side on one XCD, so its x rows
 * come from HBM once and from that XCD's L2 for the other modules.  modules,
 * y, ldy and N are host arrays of n_modules entries; every other argument
 * is as for pl_lora_fused. */
int pl_lora_fused_stacked(int32_t dtype, const void* x, int64_t ldx, int32_t K, int32_t n_modules,
                          const int32_t* modules, void* const* y, const int64_t* ldy,
                          const int32_t* N, const void* arena, const pl_slot_entry* table,
                          int32_t num_modules, int32_t ldt, const int32_t* tok,
                          const pl_group* groups, const int32_t* meta, int64_t group_cap,
                          int32_t group_tokens, int32_t slices, int32_t epilogue, void* stream);

/* Row-based LoRA on the slot arena for shapes the tiled path rejects
 * (any K, N, strides, alignment).  Writes y[b*row_len+m] for m < seq_len[b].
 * Rows whose slot is <= 0 or >= num_slots get no LoRA.  tmp is
 * [rows*row_len][ldt] fp32 scratch with ldt >= the largest rank. */
int pl_lora_apply_rows(int32_t dtype, const void* x, int64_t ldx, int32_t K, void* y,
                       int64_t ldy, int32_t N, const void* arena, const pl_slot_entry* table,
                       int32_t num_slots, int32_t num_modules, int32_t module,
                       const int32_t* row_slot,
                       const int32_t* seq_lens, int32_t rows, int32_t row_len, float* tmp,
                       int32_t ldt, int32_t epilogue, void* stream);

/* Workspace bytes of the MFMA path of pl_sgmv_lora_a_ref (which = 0: K =
 * in_features, n = n_max) or pl_sgmv_lora_b_ref (which = 1: K = k_max, n =
 * N) for these sizes, or 0 when that path does not take the shape (K of the
 * shrink or N of the expand not a whole number of 16-byte chunks, n_max or
 * k_max above 64, more than PL_MAX_SLOTS - 1 adapters, or an empty call):
 * then the row kernels run and no workspace is needed. */
int64_t pl_sgmv_ref_workspace_bytes(int32_t dtype, int32_t which, int32_t B, int32_t M, int32_t K,
                                    int32_t n, int32_t num_adapters);

/* Reference-layout shrink (sgmv.py:141-175): out[b][m][n] = T(sum_k x[b][m][k] *
 * w[widx[b]][k][n]) for m < min(seq_lens[b], M), n < min(ranks[widx[b]] *
 * stack_num, n_max); every other element of out is left as it was (the
 * reference allocates it with torch.empty).  x [B][M][K] contiguous; w
 * [num_adapters][K][n_max] with element strides; out [B][M][n_max]
 * contiguous.  Rows with widx outside [0, num_adapters) are skipped.
 * With a 256-byte aligned workspace of at least
 * pl_sgmv_ref_workspace_bytes(dtype, 0, ...) bytes (when that is nonzero)
 * and a 16-byte aligned x, the call runs on the MFMA path: one launch
 * repacks the weights of every adapter some row uses into the slot arena's
 * block layout inside the workspace (reading the reference layout with
 * consecutive lanes on consecutive elements) and builds the device plan
 * that groups the rows by adapter, then the tiled shrink writes out, its
 * last K split of each 16-token tile summing the splits in the same launch
 * (2 launches; with 64-token groups a finish kernel sums them, 3 launches;
 * no host synchronisation); with long adapter segments (B*M >= 1024 and >=
 * 64 rows per adapter, K <= 16384) one launch of the fused kernel's shrink
 * phase writes out instead (2 launches).  Otherwise, or with a null
 * workspace, one wave per token row computes it.  A workspace that is too
 * small or misaligned is an error (PL_ERR_ARG). */
int pl_sgmv_lora_a_ref(int32_t dtype, const void* x, int32_t B, int32_t M, int32_t K,
                       const void* w, int64_t w_s0, int64_t w_s1, int64_t w_s2,
                       int32_t num_adapters, int32_t n_max,
                       const int32_t* seq_lens, const int32_t* weight_indices,
                       const int32_t* lora_ranks, int32_t stack_num, void* out,
                       void* workspace, int64_t workspace_bytes, void* stream);

/* Reference-layout expand (sgmv.py:278-328): out[b][m][n] = T(T(scale * sum_{k<rank}
 * x[b][m][k] * w[widx[b]][k][n]) + out[b][m][n]) for m < min(seq_lens[b], M),
 * rank = min(ranks[widx[b]], k_max) > 0.  x [B][M][k_max] contiguous; w
 * [num_adapters][k_max][N] with element strides; out [B][M][N] contiguous
 * (updated in place).  Rows with widx outside [0, num_adapters) are
 * skipped.  Workspace and paths as for pl_sgmv_lora_a_ref (which = 1; the
 * MFMA path needs a 16-byte aligned out), except that after the repack +
 * plan launch one launch reads x directly and adds the scaled delta into
 * out: the short expand (one workgroup per 16-token group and column
 * chunk) where the shrink would take the split kernels, the fused kernel's
 * expand phase for long adapter segments or 64-token groups. */
int pl_sgmv_lora_b_ref(int32_t dtype, const void* x, int32_t B, int32_t M, int32_t k_max,
                       const void* w, int64_t w_s0, int64_t w_s1, int64_t w_s2,
                       int32_t num_adapters, int32_t N,
                       const int32_t* seq_lens, const int32_t* weight_indices,
                       const int32_t* lora_ranks, const float* scalings, void* out,
                       void* workspace, int64_t workspace_bytes, void* stream);

/* The operator API's MFMA path in three caller-kept parts (codes for
 * pl_sgmv_ref_part_bytes):
 *   PL_REF_PART_PLAN     the plan (meta, group records, token list) and the
 *                        counters with which the split shrink's last K
 *                        split of each tile finishes it in the same launch
 *                        (zeroed by every plan build, left zero by every
 *                        call; so calls that share a plan part must not
 *                        overlap).  It depends on weight_indices, seq_lens, B, M and
 *                        num_adapters only (not on ranks, weights or
 *                        which), so one plan built by any call serves the
 *                        shrink and the expand of every module that shares
 *                        them.
 *   PL_REF_PART_WEIGHTS  per-adapter pack marks, the slot table and the
 *                        weights repacked into the MFMA block layout.  It
 *                        depends on w, lora_ranks, stack_num (shrink) and
 *                        scalings (expand).
 *   PL_REF_PART_SCRATCH  the fp32 planes of one call (0 bytes when the
 *                        fused kernel's phase serves the shape).
 * Build flags of a call:
 *   PL_REF_BUILD_PLAN    build the plan into the plan part.
 *   PL_REF_PACK_USED     write the slot table and repack every adapter that
 *                        some row's weight index names.
 *   PL_REF_PACK_ALL      write the slot table and repack every adapter.
 *   PL_REF_KEEP_PACKED   with a PACK flag: skip adapters the weights part
 *                        marks as packed by an earlier call and mark the
 *                        ones this call packs with `epoch`.  The marks, the
 *                        first align256(4 * num_adapters) bytes of the
 *                        weights part (align256 rounds up to a multiple of
 *                        256), must be zero before its first such call, and
 *                        `epoch` must be >= 1 and differ from every earlier
 *                        call's on that part (a counter).
 * A call without flags reads the plan and weights parts as earlier calls
 * left them: the caller must rebuild them (with the flags, after zeroing
 * the marks again) whenever what they depend on changes.  The first call on
 * a part must build it (PL_REF_BUILD_PLAN for a plan part, a PACK flag for a
 * weights part): the kernels read offsets and lengths from the parts without
 * checking them, so a part that no call has built is read as garbage. */
#define PL_REF_PART_PLAN 0
#define PL_REF_PART_WEIGHTS 1
#define PL_REF_PART_SCRATCH 2
#define PL_REF_BUILD_PLAN 1
#define PL_REF_PACK_USED 2
#define PL_REF_PACK_ALL 4
#define PL_REF_KEEP_PACKED 8

/* Bytes of one part of the MFMA path of pl_sgmv_lora_a_ref_parts (which =
 * 0, K = in_features, n = n_max) or pl_sgmv_lora_b_ref_parts (which = 1, K
 * = k_max, n = N), or 0 for every part when that path does not take the
 * shape (as pl_sgmv_ref_workspace_bytes). */
int64_t pl_sgmv_ref_part_bytes(int32_t dtype, int32_t which, int32_t B, int32_t M, int32_t K,
                               int32_t n, int32_t num_adapters, int32_t part);

/* pl_sgmv_lora_a_ref with the plan, weights and scratch parts given
 * separately (each 256-byte aligned and at least pl_sgmv_ref_part_bytes
 * long; scratch may be NULL when its size is 0) and the build flags above:
 * results are bit for bit those of pl_sgmv_lora_a_ref once the parts hold
 * what the flags build.  Launches step 1 (table, plan, repack) only when a
 * flag asks for it.  Shapes the MFMA path does not take run the row
 * kernels and leave the parts alone.  Calls that share a part must be
 * ordered (one stream). */
int pl_sgmv_lora_a_ref_parts(int32_t dtype, const void* x, int32_t B, int32_t M, int32_t K,
                             const void* w, int64_t w_s0, int64_t w_s1, int64_t w_s2,
                             int32_t num_adapters, int32_t n_max, const int32_t* seq_lens,
                             const int32_t* weight_indices, const int32_t* lora_ranks,
                             int32_t stack_num, void* out, void* plan, int64_t plan_bytes,
                             void* weights, int64_t weights_bytes, void* scratch,
                             int64_t scratch_bytes, int32_t flags, int32_t epoch, void* stream);

/* pl_sgmv_lora_b_ref with separate parts and build flags, as
 * pl_sgmv_lora_a_ref_parts. */
int pl_sgmv_lora_b_ref_parts(int32_t dtype, const void* x, int32_t B, int32_t M, int32_t k_max,
                             const void* w, int64_t w_s0, int64_t w_s1, int64_t w_s2,
                             int32_t num_adapters, int32_t N, const int32_t* seq_lens,
                             const int32_t* weight_indices, const int32_t* lora_ranks,
                             const float* scalings, void* out, void* plan, int64_t plan_bytes,
                             void* weights, int64_t weights_bytes, void* scratch,
                             int64_t scratch_bytes, int32_t flags, int32_t epoch, void* stream);

/* Bytes of the static device scratch behind pl_lora_apply_noalloc. */
#define PL_NOALLOC_SCRATCH_BYTES (32 << 20)

/* pl_plan_build followed by pl_lora_apply in one call that allocates
 * nothing.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  The plan (meta, group records,
 * token list) and the shrink's fp32 planes live in a static device array of
 * PL_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends; the caller
 * passes only inputs and outputs: x, y, the slot arena and table, and the
 * int32 row -> slot map and row lengths of pl_plan_build.  A call needs
 *   256 + align256(16 * pl_plan_group_capacity(rows, row_len, num_slots,
 *   group_tokens)) + align256(4 * max(1, rows * row_len))
 *   + pl_shrink_workspace_bytes(dtype, K, k_splits, group_tokens,
 *   max(1, rows * row_len), ldt)
 * bytes of it (align256 rounds up to a multiple of 256); larger calls return
 * PL_ERR_LIMIT.  Every call on one GPU uses that GPU's one array and leaves
 * its contents behind (nothing in it needs clearing: each call writes every
 * byte it reads), so calls that overlap on one GPU (other streams, or other
 * threads without ordering) race.  Results equal pl_plan_build +
 * pl_lora_apply with the same group_tokens and k_splits bit for bit. */
int pl_lora_apply_noalloc(int32_t dtype, const void* x, int64_t ldx, int32_t K, void* y,
                          int64_t ldy, int32_t N, const void* arena, const pl_slot_entry* table,
                          int32_t num_modules, int32_t module, const int32_t* row_slot,
                          const int32_t* seq_lens, int32_t rows, int32_t row_len,
                          int32_t num_slots, int32_t group_tokens, int32_t ldt,
                          int32_t k_splits, int32_t epilogue, void* stream);

/* Page-locked host memory of exactly nbytes for adapter slot images (host
 * side of cache.py:119-150's uploads: the source of pl_slot_upload), or NULL
 * (with pl_last_error set and the runtime's error state cleared) when the
 * system refuses; pl_host_free releases it. */
void* pl_host_alloc(int64_t nbytes);
int pl_host_free(void* ptr);

/* Copy one packed adapter (host, pinned) into its slot region and its table
 * row into the slot table, both asynchronously on `stream`. */
int pl_slot_upload(void* arena_dst, const void* host_src, int64_t nbytes, void* table_dst,
                   const void* table_src, int64_t table_bytes, void* stream);

/* Host -> host copy of nbytes run in `stream`'s order as a host function
 * (split over up to 8 threads), for an adapter image held in pageable memory:
 * its copy into a page-locked staging buffer that a pl_slot_upload queued
 * behind it (on this stream, or on another after an event) reads.  The
 * caller never waits; dst and src stay valid until the stream has passed
 * the copy. */
int pl_host_copy_async(void* dst, const void* src, int64_t nbytes, void* stream);

/* flag[0] |= 1 if (mask[b][s] != 0) != (s < seq_lens[b]) for any element.
 * mask_dtype: 0 int64, 1 int32, 2 uint8/bool, 3 f32, 4 bf16, 5 f16. */
int pl_check_right_padded(const void* mask, int32_t mask_dtype, int32_t B, int32_t S,
                          const int32_t* seq_lens, int32_t* flag, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* POLYLORA_HIP_H */
