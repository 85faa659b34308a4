// Shared device/host helpers of the gfx950 multi-LoRA SGMV library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/polylora_hip.h"

typedef __bf16 pl_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 pl_f16x8 __attribute__((ext_vector_type(8)));
typedef float pl_f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t pl_u32x4 __attribute__((ext_vector_type(4)));

// Element traits.  E = elements per 16-byte chunk, the unit every lane loads.
template <int DT>
struct pl_traits;
template <>
struct pl_traits<PL_F32> {
  typedef float T;
  typedef float T4 __attribute__((ext_vector_type(4)));
  typedef float T8 __attribute__((ext_vector_type(8)));
  enum { E = 4 };
};
template <>
struct pl_traits<PL_BF16> {
  typedef __bf16 T;
  typedef __bf16 T4 __attribute__((ext_vector_type(4)));
  typedef __bf16 T8 __attribute__((ext_vector_type(8)));
  enum { E = 8 };
};
template <>
struct pl_traits<PL_F16> {
  typedef _Float16 T;
  typedef _Float16 T4 __attribute__((ext_vector_type(4)));
  typedef _Float16 T8 __attribute__((ext_vector_type(8)));
  enum { E = 8 };
};

// Round an fp32 value to the element type (round-to-nearest-even) and back.
template <int DT>
__device__ __forceinline__ float pl_round(float v) {
  typedef typename pl_traits<DT>::T T;
  return (float)(T)v;
}

// Expand epilogue: the scaled delta added to the base output, y = T(y + d), with
//   fallback order (layers.py:127-128): d = T(T(acc) * T(scale))
//   triton order   (sgmv.py:268-275):   d = T(acc * scale)
// pl_delta returns d (exactly representable in the element type).
template <int DT>
__device__ __forceinline__ float pl_delta(float acc, float scale, float scale_t, int mode) {
  if (mode == PL_EPI_FALLBACK) return pl_round<DT>(pl_round<DT>(acc) * scale_t);
  return pl_round<DT>(acc * scale);
}

template <int DT>
__device__ __forceinline__ float pl_epilogue(float acc, float y, float scale, float scale_t,
                                             int mode) {
  return pl_round<DT>(y + pl_delta<DT>(acc, scale, scale_t, mode));
}

__device__ __forceinline__ pl_u32x4 pl_ld16(const void* p) {
  return *reinterpret_cast<const pl_u32x4*>(p);
}

// Workgroups go to the GPU's 8 XCDs round-robin by block index, and each XCD
// has its own L2.  pl_xcd_map gives every work item of the plan group at
// position g to XCD g % 8, so the group's rereads (x rows, A and B) hit that
// XCD's L2; the plan places an adapter's groups at positions of one XCD (or
// two), in 8 balanced chunks of its slot-major group list (pl_plan_build).
// The grid is 8 * ceil(group_cap / 8) * per_group blocks; a block whose group
// is past group_cap, or empty, does nothing.
constexpr int kXcds = 8;
struct pl_xcd_slot {
  int g;  // plan group
  int j;  // work item within the group, 0 .. per_group-1
};
__device__ __forceinline__ pl_xcd_slot pl_xcd_map(int per_group) {
  const int x = (int)(blockIdx.x % kXcds);
  const int s = (int)(blockIdx.x / kXcds);
  const int gq = s / per_group;
  return {gq * kXcds + x, s - gq * per_group};
}
// A launch of `blocks` workgroups of `threads` threads fits a grid
// dimension: the dispatch packet counts work-items in 32 bits.
static inline bool pl_grid_fits(int64_t blocks, int threads) {
  return blocks >= 0 && blocks <= (int64_t)0xffffffffLL / threads;
}
static inline int64_t pl_xcd_grid(int64_t group_cap, int64_t per_group) {
  return (group_cap + kXcds - 1) / kXcds * kXcds * per_group;
}

// Slot arena layout of a module's A ([rank][K]) and B ([N][rank8]): MFMA
// blocks.  An [R][C] matrix is cut into tiles of 16 rows (rt = min(16,
// R - 16t) in tile t) and each tile is stored as its column blocks of W =
// 64 bytes (wb = min(W, C - sW) wide), one after the other, row-major:
//   element (i, c) at 16*t*C + s*rt*W + (i % 16)*wb + (c - s*W),
// t = i / 16, s = c / W.  A wave's 16-row x 64-byte operand load (lane
// (li, lg): row 16t + li, columns sW + lg*E .. +E) reads rt*wb contiguous
// elements.  With c0 = sW the block of tile t starts at 16*t*C + c0*rt.
template <int DT>
__device__ __forceinline__ int64_t pl_tile_off(int i, int c, int R, int C) {
  constexpr int W = 4 * pl_traits<DT>::E;
  const int t = i >> 4;
  const int rt = min(16, R - (t << 4));
  const int c0 = c - c % W;
  const int wb = min(W, C - c0);
  return (int64_t)(t << 4) * C + (int64_t)c0 * rt + (i & 15) * wb + (c - c0);
}

// Sixteen zero bytes in device memory: the source of every masked-off lane.
static __device__ __attribute__((aligned(16))) uint32_t pl_zero16[4];

// Branch-free guarded load: lanes with !ok read pl_zero16 instead of p.  The
// guard only selects an address, so no exec-masked branch and no select on
// the loaded value: the compiler can keep a wave's loads in flight together.
__device__ __forceinline__ pl_u32x4 pl_ld16_or0(const void* p, bool ok) {
  return pl_ld16(ok ? p : static_cast<const void*>(pl_zero16));
}

// Streaming (non-temporal) forms for data a launch touches once: activations
// x and outputs y.  On gfx950 they mark the line non-temporal, so a read or a
// read-modify-write stream does not fill the XCD's L2 with lines no workgroup
// reads again (the adapter weights, which other tiles reread, stay cached),
// and written lines leave no dirty L2 state to write back when the kernel
// ends.  Measured on MI355X for the isolated op (T=4096, K=N=4096): fused
// kernel 21.5 -> 18.3 us with x, y loads and y stores all non-temporal;
// non-temporal y stores alone gave nothing and y loads alone were slower.
__device__ __forceinline__ pl_u32x4 pl_ld16_nt_or0(const void* p, bool ok) {
  return __builtin_nontemporal_load(
      reinterpret_cast<const pl_u32x4*>(ok ? p : static_cast<const void*>(pl_zero16)));
}
__device__ __forceinline__ void pl_st16_nt(void* p, pl_u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<pl_u32x4*>(p));
}

// One 16-byte chunk per lane on each operand of a 16x16 MFMA tile, fp32
// accumulate.  Lane l supplies row (l % 16) of the A operand and column
// (l % 16) of the B operand; its chunk covers the reduction slots owned by
// lane group l / 16.  bf16/f16: one 16x16x32 MFMA (8 elements per lane).
// f32: four 16x16x4 MFMAs, element i of both chunks feeding MFMA i.  Both
// operands use the same lane -> reduction-index map, so any consistent
// assignment of k to (lane group, element) yields the same contraction.
template <int DT>
__device__ __forceinline__ pl_f32x4 pl_mfma_chunk(pl_u32x4 a, pl_u32x4 b, pl_f32x4 c);

template <>
__device__ __forceinline__ pl_f32x4 pl_mfma_chunk<PL_BF16>(pl_u32x4 a, pl_u32x4 b,
                                                           pl_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(pl_bf16x8, a),
                                                 __builtin_bit_cast(pl_bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ pl_f32x4 pl_mfma_chunk<PL_F16>(pl_u32x4 a, pl_u32x4 b,
                                                          pl_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(pl_f16x8, a),
                                                __builtin_bit_cast(pl_f16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ pl_f32x4 pl_mfma_chunk<PL_F32>(pl_u32x4 a, pl_u32x4 b, pl_f32x4 c) {
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.x), __uint_as_float(b.x), c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.y), __uint_as_float(b.y), c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.z), __uint_as_float(b.z), c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.w), __uint_as_float(b.w), c, 0, 0, 0);
  return c;
}

// ---------------------------------------------------------------- host side
void pl_set_error(const char* fmt, ...);
int pl_launch_status(const char* what);

static inline int pl_elem_size(int dtype) { return dtype == PL_F32 ? 4 : 2; }
static inline int pl_chunk_elems(int dtype) { return dtype == PL_F32 ? 4 : 8; }

// One phase of the fused kernel (sgmv_fused.hip) over a one-module slot
// table (module 0), one column slice, for the reference-layout operator API:
//   PL_FUSED_SHRINK: y[tok][c] = T(sum_k x[tok][k] * A[c][k]) for c below the
//     slot's rank (the rest of the row is not written); N and ldy describe y.
//   PL_FUSED_EXPAND: y[tok] += the expand of the intermediate x[tok][0..rank)
//     (model dtype, row stride ldx; K is unused), the columns cut into
//     `slices` ranges of their own workgroups (1 to 8; the shrink takes 1).
// Operands are checked by the caller.
enum { PL_FUSED_FULL = 0, PL_FUSED_SHRINK = 1, PL_FUSED_EXPAND = 2 };
int pl_fused_phase(int mode, int32_t dtype, const void* x, int64_t ldx, int32_t K, void* y,
                   int64_t ldy, int32_t N, const void* arena, const pl_slot_entry* table,
                   int32_t ldt, const int32_t* tok, const pl_group* groups, const int32_t* meta,
                   int64_t group_cap, int32_t group_tokens, int32_t slices, int32_t epilogue,
                   void* stream);

// MFMA path of the reference-layout operator API (sgmv_refop.hip).  Both
// return PL_REFOP_DECLINED, having launched nothing, when there is neither a
// workspace nor parts, or the shape is not one the tiled kernels take; the
// caller then runs the row kernels.  With parts == nullptr the workspace of
// pl_sgmv_ref_workspace_bytes bytes is split into the three parts and the
// call builds the plan and packs the adapters its rows use.
constexpr int PL_REFOP_DECLINED = -100;
struct pl_refop_parts {
  void* plan;
  int64_t plan_bytes;
  void* weights;
  int64_t weights_bytes;
  void* scratch;
  int64_t scratch_bytes;
  int32_t flags;  // PL_REF_* build flags
  int32_t epoch;
};
// pl_sgmv_shrink for one module (table column 0) of a plan of 16-token
// groups, with each (group, rank pass) finished inside the launch: the last
// of its K splits to store its plane writes out[tok][j] = T(sum of the planes
// in split order) for j below the slot's rank and n_max, as a separate pass
// over the planes would, and nothing else of out.  counters: counter_ints >=
// group_cap * rank passes (ldt / 32 at most 2) * PL_FINISH_COUNTER_INTS
// int32s, all zero, and all zero again when the launch has run.  Returns
// PL_REFOP_DECLINED, having launched nothing, for plans of 64-token groups,
// ldt not a multiple of 32 (each 128-byte line of the planes must hold one
// row's ranks of one rank pass) or too few counters.
constexpr int PL_FINISH_COUNTER_INTS = 16;  // int32s per counter: 64 bytes
int pl_shrink_finish_launch(int32_t dtype, const void* x, int64_t ldx, int32_t K,
                            const void* arena, const pl_slot_entry* table, const int32_t* tok,
                            const pl_group* groups, const int32_t* meta, int64_t group_cap,
                            int32_t group_tokens, void* ws, int64_t ws_bytes, int32_t ldt,
                            int64_t tmp_rows, int32_t k_splits, int32_t* counters,
                            int64_t counter_ints, void* out, int32_t n_max, void* stream);

// The short expand (16-token groups) staging the caller's model-dtype
// intermediate inter[token][ldi] instead of split planes, for the operator
// API's expand: one workgroup per (group, 256- or 128-column chunk).  Returns
// PL_REFOP_DECLINED for arguments it does not take (the caller then runs
// another kernel); ranks in the slot table must not exceed ldi.
int pl_expand_inter_launch(int32_t dtype, const void* inter, int64_t ldi, const void* arena,
                           const pl_slot_entry* table, const int32_t* tok, const pl_group* groups,
                           const int32_t* meta, int64_t group_cap, int32_t group_tokens, void* y,
                           int64_t ldy, int32_t N, int32_t ldt, int32_t epilogue, void* stream);
int pl_refop_shrink(int32_t dtype, const void* x, int32_t B, int32_t M, int32_t K, const void* w,
                    int64_t w_s0, int64_t w_s1, int64_t w_s2, int32_t num_adapters,
                    int32_t n_max, const int32_t* seq_lens, const int32_t* weight_indices,
                    const int32_t* lora_ranks, int32_t stack_num, void* out, void* workspace,
                    int64_t workspace_bytes, const pl_refop_parts* parts, void* stream);
int pl_refop_expand(int32_t dtype, const void* x, int32_t B, int32_t M, int32_t k_max,
                    const void* w, int64_t w_s0, int64_t w_s1, int64_t w_s2,
                    int32_t num_adapters, int32_t N, const int32_t* seq_lens,
                    const int32_t* weight_indices, const int32_t* lora_ranks,
                    const float* scalings, void* out, void* workspace, int64_t workspace_bytes,
                    const pl_refop_parts* parts, void* stream);
