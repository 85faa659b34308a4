// MFMA path behind the reference-layout operator API (sgmv_lora_a_fwd and
// sgmv_lora_b_fwd, sgmv.py:141-175 and :278-328).
//
// Those calls take adapter weights in the reference's own slot layout
// (w [num_adapters][k][n] with any element strides) and a per-row adapter
// index, and pass the LoRA intermediate between them as a model-dtype tensor
// [B][M][n].  Each call here runs two or three launches on the caller's
// stream, all inside a caller-provided workspace:
//
//   1. pl_refop_prep_plan: workgroup (0, 0) writes the slot table and builds
//      the plan over (B rows of M tokens) straight from the adapter index
//      (adapter i -> slot i+1; rows whose adapter index is out of range or
//      whose rank is 0 get slot 0 and are left alone, as the reference's
//      kernels skip them); the other workgroups repack the adapters'
//      weights into the MFMA block layout of the slot arena (A as [rank][K],
//      B as [N][rank8]).  Ranks, scales and indices stay on the device: no
//      host synchronisation.
//   2. shrink: pl_sgmv_shrink into fp32 split planes, then pl_refop_finish
//      writes out[b][m][n] = T(sum of the planes) for n < rank * stack_num;
//      expand: pl_refop_gather loads the model-dtype intermediate into one
//      fp32 plane (zero past each row's rank), then pl_sgmv_expand adds
//      T(scale * sum) into the output in the reference's rounding order.
//      With long adapter segments (at least 1024 rows and 64 per adapter)
//      step 2 is one launch of a phase of the fused kernel instead
//      (pl_fused_phase): the shrink reduces each 16-token tile in LDS and
//      writes T(sum) straight into out, the expand stages the caller's
//      intermediate in LDS and adds the deltas into out.
//
// The repack reads every adapter's weights once per call (the reference's
// weight tensor is the caller's, and may change between calls); for the
// 16-adapter, rank-16, K = N = 4096 case that is 2 MB per call against 26 to
// 52 MB of activations.  Shapes the tiled kernels do not take (K or N not a
// whole number of 16-byte chunks, ranks above 64, misaligned pointers) fall
// back to the row kernels of sgmv_rows.hip.
#include <algorithm>
#include <type_traits>

#include "pl_common.h"
#include "pl_plan_body.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxRefRank = 64;  // rank capacity of the repacked slots (the tiled kernels' tested range)

int64_t align256(int64_t v) { return (v + 255) & ~(int64_t)255; }
int32_t round8(int32_t v) { return (v + 7) & ~7; }

struct refop_layout {
  int32_t group_tokens;
  int64_t group_cap;
  int32_t ldt;        // rank capacity of a slot, a multiple of 8
  int32_t k_splits;   // shrink planes requested
  int32_t planes;     // planes the shrink writes (1 for the expand)
  int64_t tokens;     // B * M
  int64_t slot_bytes;
  // byte offsets inside the workspace
  int64_t meta, groups, tok, table, arena, plane, total;
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
  if (which == 0) {
    const int64_t by_k = (K + 1023) / 1024;
    const int64_t by_groups = (2048 + L.group_cap - 1) / L.group_cap;
    L.k_splits = (int32_t)std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>(8, by_k), by_groups));
    L.planes = pl_shrink_planes(dtype, K, L.k_splits, L.group_tokens);
    if (L.planes < 1) return false;
    L.slot_bytes = align256((int64_t)rank_cap * K * es);
  } else {
    L.k_splits = 1;
    L.planes = 1;
    L.slot_bytes = align256((int64_t)n * L.ldt * es);
  }
  int64_t o = 0;
  L.meta = o;
  o += 256;
  L.groups = o;
  o += align256(16 * L.group_cap);
  L.tok = o;
  o += align256(4 * T);
  L.table = o;
  o += align256((int64_t)sizeof(pl_slot_entry) * (num_adapters + 1));
  L.arena = o;
  o += L.slot_bytes * num_adapters;
  L.plane = o;
  o += align256((int64_t)L.planes * T * L.ldt * 4);
  L.total = o;
  return true;
}

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
  // the plan
  const int32_t* seq_lens;
  int32_t B, M;
  int32_t group_tokens;
  int64_t group_cap;
  int32_t* tok;
  pl_group* groups;
  int32_t* meta;
};

// Rank a slot holds for adapter s: rank * stack_num columns of the shrink,
// rank rows of the expand, clamped to the weight tensor's extent.
__device__ __forceinline__ int pl_refop_rank(const refop_prep_args& a, int s) {
  const int64_t r = (int64_t)a.ranks[s] * (a.which == 0 ? a.stack_num : 1);
  return (int)(r < 0 ? 0 : (r > a.rank_cap ? a.rank_cap : r));
}

// Grid: y = 0, x = 0 writes the slot table and builds the plan (the other
// workgroups of row y = 0 have nothing to do); y = s + 1 repacks adapter s,
// x covering its matrix.  The plan's slot for row b is adapter widx[b] + 1
// when widx[b] is in range and ranks[widx[b]] > 0 (the same test as
// pl_refop_rank(a, widx[b]) > 0, since stack_num >= 1 and rank_cap >= 1).
template <int DT>
__global__ __launch_bounds__(kPlanThreads) void pl_refop_prep_plan(refop_prep_args a) {
  typedef typename pl_traits<DT>::T T;
  if (blockIdx.y == 0) {
    if (blockIdx.x != 0) return;
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
    pl_plan_body<true>(a.widx, a.ranks, a.num_adapters, a.seq_lens, a.B, a.M, a.num_adapters + 1,
                       nullptr, 0, a.group_tokens, a.tok, a.groups, a.meta, a.group_cap);
    return;
  }
  const int s = blockIdx.y - 1;
  const int64_t e = (int64_t)blockIdx.x * kPlanThreads + threadIdx.x;
  const int r = pl_refop_rank(a, s);
  if (r == 0) return;
  // the slot's matrix [R][C] in logical order, columns fastest: A [r][K], B [N][rank8]
  const int R = a.which == 0 ? r : a.width;
  const int C = a.which == 0 ? a.width : ((r + 7) & ~7);
  if (e >= (int64_t)R * C) return;
  const int i = (int)(e / C);
  const int c = (int)(e - (int64_t)i * C);
  const T* w = reinterpret_cast<const T*>(a.w) + (int64_t)s * a.s0;
  T v;
  if (a.which == 0) {
    v = w[(int64_t)c * a.s1 + (int64_t)i * a.s2];  // A[r=i][k=c] = w[s][k][r]
  } else {
    v = c < r ? w[(int64_t)c * a.s1 + (int64_t)i * a.s2] : (T)0.f;  // B[n=i][j=c] = w[s][j][n]
  }
  T* dst = reinterpret_cast<T*>(a.arena + (int64_t)s * a.slot_bytes);
  dst[pl_tile_off<DT>(i, c, R, C)] = v;
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
    float acc = 0.f;
    for (int c = 0; c < n_planes; ++c) acc += planes[c * plane + p * ldt + n];
    reinterpret_cast<T*>(out)[(int64_t)tok[p] * n_max + n] = (T)acc;
  }
}

// plane[p][j] = x[tok[p]][j] for j below the slot's rank, 0 up to ldt: one
// workgroup per plan group record.
template <int DT>
__global__ __launch_bounds__(kThreads) void pl_refop_gather(const void* __restrict__ x,
                                                            int32_t k_max, int32_t ldt,
                                                            const pl_group* __restrict__ groups,
                                                            const int32_t* __restrict__ tok,
                                                            const pl_slot_entry* __restrict__ table,
                                                            float* __restrict__ plane) {
  typedef typename pl_traits<DT>::T T;
  const pl_group g = groups[blockIdx.x];
  if (g.len <= 0 || g.slot <= 0) return;
  const int r = table[g.slot].rank;
  for (int idx = threadIdx.x; idx < g.len * ldt; idx += kThreads) {
    const int i = idx / ldt;
    const int j = idx - i * ldt;
    const int64_t p = (int64_t)g.start + i;
    float v = 0.f;
    if (j < r) v = (float)reinterpret_cast<const T*>(x)[(int64_t)tok[p] * k_max + j];
    plane[p * ldt + j] = v;
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

// The slot table, the plan and the repacked weights (pl_refop_prep_plan).
// The layout fixes the plan's sizes: group_tokens 16 or 64, num_adapters + 1
// <= PL_MAX_SLOTS slots, B * M < 2^31 tokens and group_cap at the bound of
// pl_plan_group_capacity, the checks pl_plan_build makes.
int refop_prep(int32_t dtype, const refop_layout& L, char* ws, const void* w, int64_t s0,
               int64_t s1, int64_t s2, int32_t num_adapters, int which, int32_t width,
               int32_t rank_cap, int32_t stack_num, const int32_t* ranks, const float* scalings,
               const int32_t* widx, int32_t B, int32_t M, const int32_t* seq_lens, hipStream_t s) {
  refop_prep_args a;
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
  a.arena = ws + L.arena;
  a.slot_bytes = L.slot_bytes;
  a.table = reinterpret_cast<pl_slot_entry*>(ws + L.table);
  a.seq_lens = seq_lens;
  a.B = B;
  a.M = M;
  a.group_tokens = L.group_tokens;
  a.group_cap = L.group_cap;
  a.tok = reinterpret_cast<int32_t*>(ws + L.tok);
  a.groups = reinterpret_cast<pl_group*>(ws + L.groups);
  a.meta = reinterpret_cast<int32_t*>(ws + L.meta);
  const int64_t mat = which == 0 ? (int64_t)rank_cap * width : (int64_t)width * round8(rank_cap);
  const int64_t gx = (mat + kPlanThreads - 1) / kPlanThreads;
  if (!pl_grid_fits(gx, kPlanThreads)) {
    pl_set_error("reference-layout repack grid too large");
    return PL_ERR_LIMIT;
  }
  refop_dispatch(dtype, [&](auto dt) {
    hipLaunchKernelGGL(pl_refop_prep_plan<decltype(dt)::value>,
                       dim3((unsigned)gx, num_adapters + 1), dim3(kPlanThreads), 0, s, a);
  });
  return pl_launch_status("pl_refop_prep_plan");
}

}  // namespace

extern "C" int64_t pl_sgmv_ref_workspace_bytes(int32_t dtype, int32_t which, int32_t B, int32_t M,
                                               int32_t K, int32_t n, int32_t num_adapters) {
  refop_layout L;
  if (which != 0 && which != 1) return 0;
  return refop_plan_layout(dtype, which, B, M, K, n, num_adapters, L) ? L.total : 0;
}

int pl_refop_shrink(int32_t dtype, const void* x, int32_t B, int32_t M, int32_t K, const void* w,
                    int64_t w_s0, int64_t w_s1, int64_t w_s2, int32_t num_adapters,
                    int32_t n_max, const int32_t* seq_lens, const int32_t* weight_indices,
                    const int32_t* lora_ranks, int32_t stack_num, void* out, void* workspace,
                    int64_t workspace_bytes, void* stream) {
  refop_layout L;
  if (!workspace || !refop_plan_layout(dtype, 0, B, M, K, n_max, num_adapters, L) ||
      (reinterpret_cast<uintptr_t>(x) & 15) != 0)
    return PL_REFOP_DECLINED;
  if (!aligned256(workspace) || workspace_bytes < L.total) {
    pl_set_error("sgmv_lora_a workspace: %lld bytes at %p, this call needs %lld 256-byte aligned",
                 (long long)workspace_bytes, workspace, (long long)L.total);
    return PL_ERR_ARG;
  }
  char* ws = reinterpret_cast<char*>(workspace);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int st = refop_prep(dtype, L, ws, w, w_s0, w_s1, w_s2, num_adapters, 0, K, n_max, stack_num,
                      lora_ranks, nullptr, weight_indices, B, M, seq_lens, s);
  if (st) return st;
  int32_t* meta = reinterpret_cast<int32_t*>(ws + L.meta);
  pl_group* groups = reinterpret_cast<pl_group*>(ws + L.groups);
  int32_t* tok = reinterpret_cast<int32_t*>(ws + L.tok);
  const pl_slot_entry* table = reinterpret_cast<const pl_slot_entry*>(ws + L.table);
  float* planes = reinterpret_cast<float*>(ws + L.plane);
  if (refop_fused(L, num_adapters, K))
    return pl_fused_phase(PL_FUSED_SHRINK, dtype, x, K, K, out, n_max, n_max, ws + L.arena, table,
                          L.ldt, tok, groups, meta, L.group_cap, L.group_tokens, PL_EPI_FALLBACK,
                          stream);
  st = pl_sgmv_shrink(dtype, x, K, K, ws + L.arena, table, 1, 0, tok, groups, meta, L.group_cap,
                      L.group_tokens, planes, L.total - L.plane, L.ldt, L.tokens, L.k_splits,
                      stream);
  if (st) return st;
  refop_dispatch(dtype, [&](auto dt) {
    hipLaunchKernelGGL(pl_refop_finish<decltype(dt)::value>, dim3((unsigned)L.group_cap),
                       dim3(kThreads), 0, s, planes, L.tokens * L.ldt, L.planes, L.ldt, groups, tok,
                       table, n_max, out);
  });
  return pl_launch_status("pl_refop_finish");
}

int pl_refop_expand(int32_t dtype, const void* x, int32_t B, int32_t M, int32_t k_max,
                    const void* w, int64_t w_s0, int64_t w_s1, int64_t w_s2,
                    int32_t num_adapters, int32_t N, const int32_t* seq_lens,
                    const int32_t* weight_indices, const int32_t* lora_ranks,
                    const float* scalings, void* out, void* workspace, int64_t workspace_bytes,
                    void* stream) {
  refop_layout L;
  if (!workspace || !refop_plan_layout(dtype, 1, B, M, k_max, N, num_adapters, L) ||
      (reinterpret_cast<uintptr_t>(out) & 15) != 0)
    return PL_REFOP_DECLINED;
  if (!aligned256(workspace) || workspace_bytes < L.total) {
    pl_set_error("sgmv_lora_b workspace: %lld bytes at %p, this call needs %lld 256-byte aligned",
                 (long long)workspace_bytes, workspace, (long long)L.total);
    return PL_ERR_ARG;
  }
  char* ws = reinterpret_cast<char*>(workspace);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int st = refop_prep(dtype, L, ws, w, w_s0, w_s1, w_s2, num_adapters, 1, N, k_max, 1, lora_ranks,
                      scalings, weight_indices, B, M, seq_lens, s);
  if (st) return st;
  int32_t* meta = reinterpret_cast<int32_t*>(ws + L.meta);
  pl_group* groups = reinterpret_cast<pl_group*>(ws + L.groups);
  int32_t* tok = reinterpret_cast<int32_t*>(ws + L.tok);
  const pl_slot_entry* table = reinterpret_cast<const pl_slot_entry*>(ws + L.table);
  float* plane = reinterpret_cast<float*>(ws + L.plane);
  if (refop_fused(L, num_adapters, k_max))
    return pl_fused_phase(PL_FUSED_EXPAND, dtype, x, k_max, k_max, out, N, N, ws + L.arena, table,
                          L.ldt, tok, groups, meta, L.group_cap, L.group_tokens, PL_EPI_TRITON,
                          stream);
  refop_dispatch(dtype, [&](auto dt) {
    hipLaunchKernelGGL(pl_refop_gather<decltype(dt)::value>, dim3((unsigned)L.group_cap),
                       dim3(kThreads), 0, s, x, k_max, L.ldt, groups, tok, table, plane);
  });
  st = pl_launch_status("pl_refop_gather");
  if (st) return st;
  return pl_sgmv_expand(dtype, plane, L.ldt, L.tokens, 1, ws + L.arena, table, 1, 0, tok, groups,
                        meta, L.group_cap, L.group_tokens, out, N, N, PL_EPI_TRITON, stream);
}
