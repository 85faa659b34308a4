// MFMA path behind the reference-layout operator API (sgmv_lora_a_fwd and
// sgmv_lora_b_fwd, sgmv.py:141-175 and :278-328).
//
// Those calls take adapter weights in the reference's own slot layout
// (w [num_adapters][k][n] with any element strides) and a per-row adapter
// index, and pass the LoRA intermediate between them as a model-dtype tensor
// [B][M][n].  A call works in three caller-provided parts of device memory:
//
//   plan     the plan over (B rows of M tokens): meta, group records, token
//            list.  It depends only on the adapter index, the row lengths
//            and B, M, num_adapters, so one plan serves the shrink and the
//            expand of every module of a forward.
//   weights  per-adapter pack marks, the slot table (rank, scale, offsets)
//            and the adapters' weights repacked into the MFMA block layout
//            of the slot arena (A as [rank][K], B as [N][rank8]).  It
//            depends on w, the ranks, the scalings and stack_num.
//   scratch  the fp32 split planes of a shrink (the expand needs none).
//
// The build flags say what a call must (re)build; a caller that keeps the
// plan and weights parts across calls (keyed on what they depend on)
// passes none of them and skips step 1:
//
//   1. pl_refop_prep (only with PL_REF_BUILD_PLAN or a PL_REF_PACK_* flag):
//      workgroup (0, 0) writes the slot table and builds the plan straight
//      from the adapter index (adapter i -> slot i + 1, an index out of
//      range -> slot 0); the workgroups of row y = s + 1 repack adapter s:
//      with PL_REF_PACK_USED only when some row uses it, with
//      PL_REF_PACK_ALL always, and with PL_REF_KEEP_PACKED not when the
//      weights part marks it packed at an earlier call.  Each repack unit
//      reads a 64-row x 4-block panel of the reference layout with
//      consecutive lanes on consecutive elements of its fastest dimension,
//      transposes it through LDS and writes 16 whole MFMA blocks.  Ranks,
//      scales and indices stay on the device: no host synchronisation.
//   2. shrink: the split shrink into fp32 planes, and out[b][m][n] = T(sum
//      of the planes) for n < rank * stack_num written by the last K split
//      of each tile to finish, in the same launch (pl_shrink_finish_launch,
//      16-token groups; its counters live in the plan part, zeroed by every
//      plan build and left zero by every launch); with 64-token groups a
//      second launch (pl_refop_finish) sums the planes; with long adapter
//      segments (at least 1024 rows and 64 per adapter)
//      one launch of the fused kernel's shrink phase (pl_fused_phase)
//      instead reduces each 16-token tile in LDS and writes T(sum) straight
//      into out.  expand: one launch that stages the caller's model-dtype
//      intermediate in LDS (zero past each row's rank) and adds
//      T(scale * sum) into the output in the reference's rounding order:
//      where the shrink took the split kernels (16-token groups), the short
//      expand reading the intermediate by token (pl_expand_inter_launch);
//      with long segments, the fused kernel's expand phase, its columns cut
//      into slices so that the launch has about 1024 workgroups.  (On the
//      Llama-3-8B decode layer, 256 rows over 64 adapters, the fused shrink
//      phase took 18.8 us against 13.6 us for the split shrink and its
//      finish, so short segments keep the split shrink; the short expand
//      there takes 4.5-13.2 us per module against 5.8-14.3 us for the fused
//      expand phase.)
//
// The plan gives every row with an adapter index in range its slot, rank 0
// or not: every kernel of step 2 returns at once for a slot whose table
// rank is 0, so those rows are left alone as the reference's kernels leave
// them.  Shapes the tiled kernels do not take (K or N not a whole number of
// 16-byte chunks, ranks above 64, misaligned pointers) fall back to the row
// kernels of sgmv_rows.hip.
#include <algorithm>
#include <type_traits>

#include "pl_common.h"
#include "pl_plan_body.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxRefRank = 64;  // rank capacity of the repacked slots (the tiled kernels' tested range)
constexpr int kPackRows = 64;    // destination rows of one repack unit (4 MFMA tiles)
constexpr int kPackBlocks = 4;   // 64-byte column blocks of one repack unit
constexpr int kPackGridCap = 16; // repack workgroups per adapter (each loops over its units)
constexpr int kMaxPlanes = 16;   // split planes a shrink writes at most (pl_shrink_planes)

int64_t align256(int64_t v) { return (v + 255) & ~(int64_t)255; }
int32_t round8(int32_t v) { return (v + 7) & ~7; }

struct refop_layout {
  int32_t group_tokens;
  int64_t group_cap;
  int32_t ldt;        // rank capacity of a slot, a multiple of 8
  int32_t pldt;       // row stride of the split shrink's planes, a multiple of 32
  int32_t k_splits;   // shrink planes requested
  int32_t planes;     // planes the shrink writes (1 for the expand)
  int64_t tokens;     // B * M
  int64_t slot_bytes;
  // byte offsets inside the plan part
  int64_t meta, groups, tok, counters, plan_bytes;
  int64_t counter_ints;  // the shrink's finish counters (pl_shrink_finish_launch)
  // byte offsets inside the weights part
  int64_t marks, table, arena, weights_bytes;
  int64_t scratch_bytes;  // the planes
  int64_t total;          // one workspace holding the three parts in this order
};

// which: 0 = shrink (K = in_features, n = n_max), 1 = expand (K = k_max, n = N).
bool refop_plan_layout(int32_t dtype, int which, int32_t B, int32_t M, int32_t K, int32_t n,
                       int32_t num_adapters, refop_layout& L) {
  if (dtype != PL_F32 && dtype != PL_BF16 && dtype != PL_F16) return false;
  if (B <= 0 || M <= 0 || K <= 0 || n <= 0 || num_adapters <= 0) return false;
  if (num_adapters + 1 > PL_MAX_SLOTS) return false;
  const int64_t T = (int64_t)B * M;
  if (T > 0x7fffffffLL) return false;
  const int E = pl_chunk_elems(dtype);
  const int es = pl_elem_size(dtype);
  const int32_t rank_cap = which == 0 ? n : K;  // n_max, or k_max
  const int32_t width = which == 0 ? K : n;     // K of the shrink, N of the expand
  if (rank_cap > kMaxRefRank || width % E != 0) return false;
  L.tokens = T;
  L.group_tokens = (T >= 8192 && T > (int64_t)32 * num_adapters) ? PL_GROUP_TOKENS_LONG
                                                                  : PL_GROUP_TOKENS_SHORT;
  L.group_cap = pl_plan_group_capacity(B, M, num_adapters + 1, L.group_tokens);
  if (L.group_cap < 1) L.group_cap = 1;
  L.ldt = round8(rank_cap);
  // the split shrink planes' row stride: whole 128-byte lines, as its
  // in-launch finish needs
  L.pldt = (rank_cap + 31) & ~31;
  if (which == 0) {
    const int64_t by_k = (K + 1023) / 1024;
    const int64_t by_groups = (2048 + L.group_cap - 1) / L.group_cap;
    L.k_splits = (int32_t)std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>(8, by_k), by_groups));
    L.planes = pl_shrink_planes(dtype, K, L.k_splits, L.group_tokens);
    if (L.planes < 1) return false;
    L.slot_bytes = align256((int64_t)rank_cap * K * es);
  } else {
    L.k_splits = 1;
    L.planes = 0;  // the fused expand phase reads the intermediate directly
    L.slot_bytes = align256((int64_t)n * L.ldt * es);
  }
  int64_t o = 0;
  L.meta = o;
  o += 256;
  L.groups = o;
  o += align256(16 * L.group_cap);
  L.tok = o;
  o += align256(4 * T);
  // counters of the split shrink's in-launch finish: one per (group, rank
  // pass), at most 2 passes of 32 ranks for slots of up to 64; the same size
  // for the shrink and the expand, so that their plans stay interchangeable
  L.counters = o;
  L.counter_ints = L.group_cap * 2 * PL_FINISH_COUNTER_INTS;
  o += align256(4 * L.counter_ints);
  L.plan_bytes = o;
  o = 0;
  L.marks = o;
  o += align256(4 * (int64_t)num_adapters);
  L.table = o;
  o += align256((int64_t)sizeof(pl_slot_entry) * (num_adapters + 1));
  L.arena = o;
  o += L.slot_bytes * num_adapters;
  L.weights_bytes = o;
  L.scratch_bytes = align256((int64_t)L.planes * T * L.pldt * 4);
  L.total = L.plan_bytes + L.weights_bytes + L.scratch_bytes;
  return true;
}

enum { kPackNone = 0, kPackUsed = 1, kPackAll = 2 };

struct refop_prep_args {
  const void* w;
  int64_t s0, s1, s2;  // element strides of w [num_adapters][k][n]
  int32_t num_adapters;
  int32_t which;       // 0: A [rank][K] from w[s][k][r]; 1: B [N][rank8] from w[s][r][n]
  int32_t width;       // K (shrink) or N (expand)
  int32_t rank_cap;    // n_max (shrink) or k_max (expand)
  int32_t stack_num;   // shrink: rank * stack_num columns per row
  const int32_t* ranks;
  const float* scalings;  // expand only
  const int32_t* widx;
  char* arena;
  int64_t slot_bytes;
  pl_slot_entry* table;
  int32_t* marks;      // marks[s]: call epoch at which adapter s was packed, 0 = never
  int32_t build_plan;
  int32_t pack;        // kPackNone, kPackUsed or kPackAll
  int32_t keep;        // consult and update marks
  int32_t epoch;
  // the plan
  const int32_t* seq_lens;
  int32_t B, M;
  int32_t group_tokens;
  int64_t group_cap;
  int32_t* tok;
  pl_group* groups;
  int32_t* meta;
  int32_t* counters;  // zeroed with every plan build
  int64_t counter_ints;
};

// Rank a slot holds for adapter s: rank * stack_num columns of the shrink,
// rank rows of the expand, clamped to the weight tensor's extent.
__device__ __forceinline__ int pl_refop_rank(const refop_prep_args& a, int s) {
  const int64_t r = (int64_t)a.ranks[s] * (a.which == 0 ? a.stack_num : 1);
  return (int)(r < 0 ? 0 : (r > a.rank_cap ? a.rank_cap : r));
}

// One repack unit of adapter s: destination rows [i0, i0 + 64) and columns
// [c0, c0 + 4W) of its [R][C] matrix (A [r][K]: i = rank, c = k; B
// [N][rank8]: i = n, c = rank), element (i, c) = w[s][c][i] in the
// reference layout (zero for c >= r in B).  Reads: lane l of a wave takes
// row i0 + l, so a wave reads 64 consecutive elements of the source's
// i-dimension (its fastest for the reference's contiguous tensors) at one
// c.  Writes: the unit's 16 destination blocks (4 row tiles x 4 column
// blocks), each rt * wb contiguous elements, consecutive threads on
// consecutive elements.
template <int DT>
__device__ __forceinline__ void pl_refop_pack_unit(const refop_prep_args& a, int s, int r, int R,
                                                   int C, int i0, int c0,
                                                   typename pl_traits<DT>::T* tile) {
  typedef typename pl_traits<DT>::T T;
  constexpr int W = 4 * pl_traits<DT>::E;  // elements of a 64-byte column block
  constexpr int UC = kPackBlocks * W;      // columns of a unit
  constexpr int LD = UC + 4 / (int)sizeof(T);  // row stride: an odd number of words
  constexpr int kColsPerPass = kPlanThreads / kPackRows;
  const int tid = threadIdx.x;
  const int i_off = tid & (kPackRows - 1);
  const int cq = tid / kPackRows;
  const int i = i0 + i_off;
  const int c_lim = a.which == 0 ? C : min(C, r);  // B's columns r..rank8-1 are zero
  const T* __restrict__ w = reinterpret_cast<const T*>(a.w) + (int64_t)s * a.s0;
  T v[UC / kColsPerPass];
#pragma unroll
  for (int k = 0; k < UC / kColsPerPass; ++k) {
    const int c = c0 + cq + k * kColsPerPass;
    v[k] = (i < R && c < c_lim) ? w[(int64_t)c * a.s1 + (int64_t)i * a.s2] : (T)0.f;
  }
#pragma unroll
  for (int k = 0; k < UC / kColsPerPass; ++k) tile[i_off * LD + cq + k * kColsPerPass] = v[k];
  __syncthreads();
  T* __restrict__ dst = reinterpret_cast<T*>(a.arena + (int64_t)s * a.slot_bytes);
  constexpr int kBlockElems = 16 * W;
  for (int f = tid; f < 4 * kPackBlocks * kBlockElems; f += kPlanThreads) {
    const int blk = f / kBlockElems;  // tile-major: a tile's column blocks are adjacent in memory
    const int e = f - blk * kBlockElems;
    const int tt = blk / kPackBlocks;
    const int cb = blk - tt * kPackBlocks;
    const int t16 = i0 + 16 * tt;
    const int cs = c0 + cb * W;
    if (t16 >= R || cs >= C) continue;
    const int rt = min(16, R - t16);
    const int wb = min(W, C - cs);
    if (e >= rt * wb) continue;
    const int row = e / wb;
    const int col = e - row * wb;
    dst[(int64_t)t16 * C + (int64_t)cs * rt + e] = tile[(16 * tt + row) * LD + cb * W + col];
  }
  __syncthreads();  // the tile is reused by the next unit
}

// Grid: y = 0, x = 0 writes the slot table (when packing) and builds the
// plan (when asked); the other workgroups of row y = 0 have nothing to do.
// y = s + 1 repacks adapter s, the x workgroups striding over its units.
template <int DT>
__global__ __launch_bounds__(kPlanThreads) void pl_refop_prep(refop_prep_args a) {
  typedef typename pl_traits<DT>::T T;
  constexpr int W = 4 * pl_traits<DT>::E;
  __shared__ T tile[kPackRows * (kPackBlocks * W + 4 / (int)sizeof(T))];
  if (blockIdx.y == 0) {
    if (blockIdx.x != 0) return;
    if (a.pack != kPackNone) {
      for (int e = threadIdx.x; e <= a.num_adapters; e += kPlanThreads) {
        pl_slot_entry en;
        en.rank = 0;
        en.scale = 0.f;
        en.rank8 = 0;
        en.reserved = 0;
        en.a_off = 0;
        en.b_off = 0;
        if (e > 0) {
          const int r = pl_refop_rank(a, e - 1);
          en.rank = r;
          en.scale = a.which == 1 ? a.scalings[e - 1] : 1.f;
          en.rank8 = (r + 7) & ~7;
          en.a_off = (int64_t)(e - 1) * a.slot_bytes;
          en.b_off = en.a_off;
        }
        a.table[e] = en;
      }
    }
    if (a.build_plan) {
      // a new plan starts the shrink's finish counters at zero (each launch
      // leaves them zero again)
      for (int64_t i = threadIdx.x; i < a.counter_ints; i += kPlanThreads) a.counters[i] = 0;
      pl_plan_body<true>(a.widx, a.num_adapters, a.seq_lens, a.B, a.M, a.num_adapters + 1,
                         nullptr, 0, a.group_tokens, a.tok, a.groups, a.meta, a.group_cap);
    }
    return;
  }
  const int s = blockIdx.y - 1;
  if (a.keep) {
    // packed at an earlier call: skip.  Within this call every workgroup of
    // s reads 0 or this call's epoch and packs its units.
    const int prev = a.marks[s];
    if (prev != 0 && prev != a.epoch) return;
  }
  const int r = pl_refop_rank(a, s);
  if (r == 0) {
    if (a.keep && blockIdx.x == 0 && threadIdx.x == 0) a.marks[s] = a.epoch;  // nothing to pack
    return;
  }
  if (a.pack == kPackUsed) {
    int used = 0;
    for (int b = threadIdx.x; b < a.B; b += kPlanThreads) used |= a.widx[b] == s;
    if (!__syncthreads_or(used)) return;
  }
  // the slot's matrix [R][C]: A [r][K], B [N][rank8]
  const int R = a.which == 0 ? r : a.width;
  const int C = a.which == 0 ? a.width : ((r + 7) & ~7);
  const int nc = (C + kPackBlocks * W - 1) / (kPackBlocks * W);
  const int units = (R + kPackRows - 1) / kPackRows * nc;
  for (int u = blockIdx.x; u < units; u += gridDim.x) {
    const int q = u / nc;
    pl_refop_pack_unit<DT>(a, s, r, R, C, q * kPackRows, (u - q * nc) * kPackBlocks * W, tile);
  }
  if (a.keep && threadIdx.x == 0) a.marks[s] = a.epoch;
}

// out[tok[p]][n] = T(sum of the planes at (p, n)) for n below the slot's rank:
// one workgroup per plan group record.
template <int DT>
__global__ __launch_bounds__(kThreads) void pl_refop_finish(const float* __restrict__ planes,
                                                            int64_t plane, int32_t n_planes,
                                                            int32_t ldt,
                                                            const pl_group* __restrict__ groups,
                                                            const int32_t* __restrict__ tok,
                                                            const pl_slot_entry* __restrict__ table,
                                                            int32_t n_max, void* __restrict__ out) {
  typedef typename pl_traits<DT>::T T;
  const pl_group g = groups[blockIdx.x];
  if (g.len <= 0 || g.slot <= 0) return;
  const int r = table[g.slot].rank;
  if (r <= 0) return;
  for (int idx = threadIdx.x; idx < g.len * r; idx += kThreads) {
    const int i = idx / r;
    const int n = idx - i * r;
    const int64_t p = (int64_t)g.start + i;
    // every plane's load before the first add (an index past the last plane
    // reads the last one again): one round trip, not one per plane
    const float* src = planes + p * ldt + n;
    float v[kMaxPlanes];
#pragma unroll
    for (int c = 0; c < kMaxPlanes; ++c) v[c] = src[(int64_t)min(c, n_planes - 1) * plane];
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < kMaxPlanes; ++c)
      if (c < n_planes) acc += v[c];
    reinterpret_cast<T*>(out)[(int64_t)tok[p] * n_max + n] = (T)acc;
  }
}

template <typename F>
void refop_dispatch(int32_t dtype, F&& launch) {
  switch (dtype) {
    case PL_BF16: launch(std::integral_constant<int, PL_BF16>()); break;
    case PL_F16: launch(std::integral_constant<int, PL_F16>()); break;
    default: launch(std::integral_constant<int, PL_F32>()); break;
  }
}

bool aligned256(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 255) == 0; }

// Long adapter segments (the fused kernel's regime, as sgmv.fused_ok picks it
// on the forward path): one workgroup per 16-token tile does the whole
// reduction of a call and hands the result straight to the caller's tensor,
// with no split planes and no finish or gather launch.  Few tokens per
// adapter keep the split kernels, which spread each adapter's weights over
// many more workgroups.
bool refop_fused(const refop_layout& L, int32_t num_adapters, int32_t K) {
  return L.tokens >= 1024 && L.tokens >= (int64_t)64 * num_adapters && K <= 16384;
}

// Column slices of the fused kernel's expand phase.  The phase recomputes
// nothing per slice (the intermediate comes from the caller), so slices only
// add workgroups: about 1024 keep every CU busy with a few waves each (one
// per 16-token tile left most CUs with one workgroup), and each slice keeps
// at least 512 columns, one 128-column step per wave.
int refop_expand_slices(const refop_layout& L, int32_t N) {
  const int64_t tiles = std::max<int64_t>(1, L.group_cap * (L.group_tokens / 16));
  const int64_t want = (1024 + tiles - 1) / tiles;
  const int64_t most = std::max<int64_t>(1, N / 512);
  return (int)std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>(want, most), 8));
}

// The three parts of a call: the caller's, or one workspace split in order
// plan | weights | scratch with the flags of a call that keeps nothing.
// Returns PL_OK, PL_ERR_ARG for parts that are too small, misaligned or
// missing, or PL_REFOP_DECLINED when there is nothing to work in.
int refop_parts(const refop_layout& L, bool fused, void* workspace, int64_t workspace_bytes,
                const pl_refop_parts* parts, const char* what, pl_refop_parts& P) {
  if (parts == nullptr) {
    if (!workspace) return PL_REFOP_DECLINED;
    if (!aligned256(workspace) || workspace_bytes < L.total) {
      pl_set_error("%s workspace: %lld bytes at %p, this call needs %lld 256-byte aligned", what,
                   (long long)workspace_bytes, workspace, (long long)L.total);
      return PL_ERR_ARG;
    }
    char* ws = reinterpret_cast<char*>(workspace);
    P.plan = ws;
    P.plan_bytes = L.plan_bytes;
    P.weights = ws + L.plan_bytes;
    P.weights_bytes = L.weights_bytes;
    P.scratch = ws + L.plan_bytes + L.weights_bytes;
    P.scratch_bytes = L.scratch_bytes;
    P.flags = PL_REF_BUILD_PLAN | PL_REF_PACK_USED;
    P.epoch = 0;
    return PL_OK;
  }
  P = *parts;
  const bool scratch_ok =
      fused || (P.scratch && aligned256(P.scratch) && P.scratch_bytes >= L.scratch_bytes);
  if (!P.plan || !aligned256(P.plan) || P.plan_bytes < L.plan_bytes || !P.weights ||
      !aligned256(P.weights) || P.weights_bytes < L.weights_bytes || !scratch_ok) {
    pl_set_error("%s parts: plan %lld bytes at %p, weights %lld at %p, scratch %lld at %p; this "
                 "call needs %lld, %lld and %lld, each 256-byte aligned",
                 what, (long long)P.plan_bytes, P.plan, (long long)P.weights_bytes, P.weights,
                 (long long)P.scratch_bytes, P.scratch, (long long)L.plan_bytes,
                 (long long)L.weights_bytes, fused ? 0LL : (long long)L.scratch_bytes);
    return PL_ERR_ARG;
  }
  const int32_t known = PL_REF_BUILD_PLAN | PL_REF_PACK_USED | PL_REF_PACK_ALL | PL_REF_KEEP_PACKED;
  if ((P.flags & ~known) != 0 || ((P.flags & PL_REF_KEEP_PACKED) && P.epoch < 1)) {
    pl_set_error("%s: build flags 0x%x / epoch %d (PL_REF_KEEP_PACKED needs an epoch >= 1)", what,
                 P.flags, P.epoch);
    return PL_ERR_ARG;
  }
  return PL_OK;
}

// Step 1 (pl_refop_prep) when the flags ask for any of it.  The layout fixes
// the plan's sizes: group_tokens 16 or 64, num_adapters + 1 <= PL_MAX_SLOTS
// slots, B * M < 2^31 tokens and group_cap at the bound of
// pl_plan_group_capacity, the checks pl_plan_build makes.
int refop_prep(int32_t dtype, const refop_layout& L, const pl_refop_parts& P, const void* w,
               int64_t s0, int64_t s1, int64_t s2, int32_t num_adapters, int which, int32_t width,
               int32_t rank_cap, int32_t stack_num, const int32_t* ranks, const float* scalings,
               const int32_t* widx, int32_t B, int32_t M, const int32_t* seq_lens, hipStream_t s) {
  refop_prep_args a;
  a.build_plan = (P.flags & PL_REF_BUILD_PLAN) ? 1 : 0;
  a.pack = (P.flags & PL_REF_PACK_ALL) ? kPackAll : (P.flags & PL_REF_PACK_USED) ? kPackUsed
                                                                                  : kPackNone;
  if (!a.build_plan && a.pack == kPackNone) return PL_OK;
  a.keep = (P.flags & PL_REF_KEEP_PACKED) ? 1 : 0;
  a.epoch = P.epoch;
  a.w = w;
  a.s0 = s0;
  a.s1 = s1;
  a.s2 = s2;
  a.num_adapters = num_adapters;
  a.which = which;
  a.width = width;
  a.rank_cap = rank_cap;
  a.stack_num = stack_num;
  a.ranks = ranks;
  a.scalings = scalings;
  a.widx = widx;
  char* wp = reinterpret_cast<char*>(P.weights);
  char* pp = reinterpret_cast<char*>(P.plan);
  a.arena = wp + L.arena;
  a.slot_bytes = L.slot_bytes;
  a.table = reinterpret_cast<pl_slot_entry*>(wp + L.table);
  a.marks = reinterpret_cast<int32_t*>(wp + L.marks);
  a.seq_lens = seq_lens;
  a.B = B;
  a.M = M;
  a.group_tokens = L.group_tokens;
  a.group_cap = L.group_cap;
  a.tok = reinterpret_cast<int32_t*>(pp + L.tok);
  a.groups = reinterpret_cast<pl_group*>(pp + L.groups);
  a.meta = reinterpret_cast<int32_t*>(pp + L.meta);
  a.counters = reinterpret_cast<int32_t*>(pp + L.counters);
  a.counter_ints = L.counter_ints;
  // repack units of the largest matrix an adapter can have (rank = rank_cap)
  const int W = 4 * pl_chunk_elems(dtype);
  const int64_t Rmax = which == 0 ? rank_cap : width;
  const int64_t Cmax = which == 0 ? width : round8(rank_cap);
  const int64_t units = (Rmax + kPackRows - 1) / kPackRows *
                        ((Cmax + kPackBlocks * W - 1) / (kPackBlocks * W));
  const int64_t gx = a.pack == kPackNone ? 1 : std::min<int64_t>(units, kPackGridCap);
  const int gy = a.pack == kPackNone ? 1 : num_adapters + 1;
  refop_dispatch(dtype, [&](auto dt) {
    hipLaunchKernelGGL(pl_refop_prep<decltype(dt)::value>, dim3((unsigned)gx, gy),
                       dim3(kPlanThreads), 0, s, a);
  });
  return pl_launch_status("pl_refop_prep");
}

}  // namespace

extern "C" int64_t pl_sgmv_ref_workspace_bytes(int32_t dtype, int32_t which, int32_t B, int32_t M,
                                               int32_t K, int32_t n, int32_t num_adapters) {
  refop_layout L;
  if (which != 0 && which != 1) return 0;
  return refop_plan_layout(dtype, which, B, M, K, n, num_adapters, L) ? L.total : 0;
}

extern "C" int64_t pl_sgmv_ref_part_bytes(int32_t dtype, int32_t which, int32_t B, int32_t M,
                                          int32_t K, int32_t n, int32_t num_adapters,
                                          int32_t part) {
  refop_layout L;
  if (which != 0 && which != 1) return 0;
  if (!refop_plan_layout(dtype, which, B, M, K, n, num_adapters, L)) return 0;
  switch (part) {
    case PL_REF_PART_PLAN: return L.plan_bytes;
    case PL_REF_PART_WEIGHTS: return L.weights_bytes;
    case PL_REF_PART_SCRATCH:
      return which == 1 || refop_fused(L, num_adapters, K) ? 0 : L.scratch_bytes;
    default: return 0;
  }
}

int pl_refop_shrink(int32_t dtype, const void* x, int32_t B, int32_t M, int32_t K, const void* w,
                    int64_t w_s0, int64_t w_s1, int64_t w_s2, int32_t num_adapters,
                    int32_t n_max, const int32_t* seq_lens, const int32_t* weight_indices,
                    const int32_t* lora_ranks, int32_t stack_num, void* out, void* workspace,
                    int64_t workspace_bytes, const pl_refop_parts* parts, void* stream) {
  refop_layout L;
  if (!refop_plan_layout(dtype, 0, B, M, K, n_max, num_adapters, L) ||
      (reinterpret_cast<uintptr_t>(x) & 15) != 0)
    return PL_REFOP_DECLINED;
  const bool fused = refop_fused(L, num_adapters, K);
  pl_refop_parts P;
  int st = refop_parts(L, fused, workspace, workspace_bytes, parts, "sgmv_lora_a", P);
  if (st) return st;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  st = refop_prep(dtype, L, P, w, w_s0, w_s1, w_s2, num_adapters, 0, K, n_max, stack_num,
                  lora_ranks, nullptr, weight_indices, B, M, seq_lens, s);
  if (st) return st;
  char* pp = reinterpret_cast<char*>(P.plan);
  char* wp = reinterpret_cast<char*>(P.weights);
  int32_t* meta = reinterpret_cast<int32_t*>(pp + L.meta);
  pl_group* groups = reinterpret_cast<pl_group*>(pp + L.groups);
  int32_t* tok = reinterpret_cast<int32_t*>(pp + L.tok);
  const pl_slot_entry* table = reinterpret_cast<const pl_slot_entry*>(wp + L.table);
  if (fused)
    return pl_fused_phase(PL_FUSED_SHRINK, dtype, x, K, K, out, n_max, n_max, wp + L.arena, table,
                          L.ldt, tok, groups, meta, L.group_cap, L.group_tokens, 1, PL_EPI_FALLBACK,
                          stream);
  float* planes = reinterpret_cast<float*>(P.scratch);
  // 16-token groups: the last K split of each tile writes its intermediate
  // in the same launch
  st = pl_shrink_finish_launch(dtype, x, K, K, wp + L.arena, table, tok, groups, meta, L.group_cap,
                               L.group_tokens, planes, L.scratch_bytes, L.pldt, L.tokens,
                               L.k_splits, reinterpret_cast<int32_t*>(pp + L.counters),
                               L.counter_ints, out, n_max, stream);
  if (st != PL_REFOP_DECLINED) return st;
  st = pl_sgmv_shrink(dtype, x, K, K, wp + L.arena, table, 1, 0, tok, groups, meta, L.group_cap,
                      L.group_tokens, planes, L.scratch_bytes, L.pldt, L.tokens, L.k_splits,
                      stream);
  if (st) return st;
  refop_dispatch(dtype, [&](auto dt) {
    hipLaunchKernelGGL(pl_refop_finish<decltype(dt)::value>, dim3((unsigned)L.group_cap),
                       dim3(kThreads), 0, s, planes, L.tokens * L.pldt, L.planes, L.pldt, groups, tok,
                       table, n_max, out);
  });
  return pl_launch_status("pl_refop_finish");
}

int pl_refop_expand(int32_t dtype, const void* x, int32_t B, int32_t M, int32_t k_max,
                    const void* w, int64_t w_s0, int64_t w_s1, int64_t w_s2,
                    int32_t num_adapters, int32_t N, const int32_t* seq_lens,
                    const int32_t* weight_indices, const int32_t* lora_ranks,
                    const float* scalings, void* out, void* workspace, int64_t workspace_bytes,
                    const pl_refop_parts* parts, void* stream) {
  refop_layout L;
  if (!refop_plan_layout(dtype, 1, B, M, k_max, N, num_adapters, L) ||
      (reinterpret_cast<uintptr_t>(out) & 15) != 0)
    return PL_REFOP_DECLINED;
  pl_refop_parts P;
  int st = refop_parts(L, true, workspace, workspace_bytes, parts, "sgmv_lora_b", P);
  if (st) return st;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  st = refop_prep(dtype, L, P, w, w_s0, w_s1, w_s2, num_adapters, 1, N, k_max, 1, lora_ranks,
                  scalings, weight_indices, B, M, seq_lens, s);
  if (st) return st;
  char* pp = reinterpret_cast<char*>(P.plan);
  char* wp = reinterpret_cast<char*>(P.weights);
  int32_t* meta = reinterpret_cast<int32_t*>(pp + L.meta);
  pl_group* groups = reinterpret_cast<pl_group*>(pp + L.groups);
  int32_t* tok = reinterpret_cast<int32_t*>(pp + L.tok);
  const pl_slot_entry* table = reinterpret_cast<const pl_slot_entry*>(wp + L.table);
  // Few tokens per adapter (the shrink took the split kernels) with 16-token
  // groups: the short expand staging the caller's intermediate, one workgroup
  // per group and 256-column chunk (decode layer: 133.5 -> 125.5 us of
  // kernels for its 7 pairs).  Long segments keep the fused kernel's expand
  // phase, whose non-temporal y stores leave no dirty lines behind (the short
  // expand there: 15.9 -> 18.4 us, and the next call's shrink 10.3 -> 12.3 us);
  // so do 64-token groups and calls the short expand declines.
  if (L.group_tokens == PL_GROUP_TOKENS_SHORT && !refop_fused(L, num_adapters, k_max)) {
    st = pl_expand_inter_launch(dtype, x, k_max, wp + L.arena, table, tok, groups, meta, L.group_cap,
                                L.group_tokens, out, N, N, L.ldt, PL_EPI_TRITON, stream);
    if (st != PL_REFOP_DECLINED) return st;
  }
  return pl_fused_phase(PL_FUSED_EXPAND, dtype, x, k_max, k_max, out, N, N, wp + L.arena, table,
                        L.ldt, tok, groups, meta, L.group_cap, L.group_tokens,
                        refop_expand_slices(L, N), PL_EPI_TRITON, stream);
}
