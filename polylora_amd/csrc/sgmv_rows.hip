// Row-based SGMV kernels: any shape, stride and alignment.
//
// They serve two callers: the reference-layout operator API
// (sgmv_lora_a_fwd / sgmv_lora_b_fwd, sgmv.py:141-175 and :278-328, weights
// [slots][k][n] with arbitrary strides) where its MFMA path (sgmv_refop.hip)
// declines the shape or gets no workspace, and MultiLoraLinear shapes the
// tiled kernels reject (K or N not a multiple of the 16-byte chunk,
// unaligned rows).  Throughput is not their goal; the tiled kernels carry
// the hot path.
//
// Shrink: one wave per token row; lanes stride K, each rank column is a
// wave-wide dot product finished with a butterfly reduction.
// Expand: one thread per output element; loop over the adapter's rank.
// Every kernel skips rows whose slot index is outside [0, num_slots), so a
// corrupt row map cannot read outside the weight tensors.
#include "pl_common.h"

namespace {

// Weight access for the reference layout [slot][k][n] (element strides).
struct pl_ref_layout {
  const void* w;
  int64_t s0, s1, s2;
  int32_t num_slots;
};

template <int DT>
__device__ __forceinline__ float pl_ld(const void* p, int64_t i) {
  typedef typename pl_traits<DT>::T T;
  return (float)reinterpret_cast<const T*>(p)[i];
}

__device__ __forceinline__ float pl_wave_sum(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d);
  return v;
}

// ---- reference layout -----------------------------------------------------

template <int DT>
__global__ __launch_bounds__(256) void pl_ref_shrink(const void* __restrict__ x, int32_t B,
                                                     int32_t M, int32_t K, pl_ref_layout w,
                                                     int32_t n_max,
                                                     const int32_t* __restrict__ seq_lens,
                                                     const int32_t* __restrict__ widx,
                                                     const int32_t* __restrict__ ranks,
                                                     int32_t stack_num, void* __restrict__ out) {
  typedef typename pl_traits<DT>::T T;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= (int64_t)B * M) return;
  const int b = (int)(row / M);
  const int m = (int)(row - (int64_t)b * M);
  if (m >= seq_lens[b]) return;
  const int s = widx[b];
  if (s < 0 || s >= w.num_slots) return;
  const int n_eff = min(ranks[s] * stack_num, n_max);
  const int64_t xb = row * K;
  const int64_t wb = (int64_t)s * w.s0;
  for (int n = 0; n < n_eff; ++n) {
    float acc = 0.f;
    for (int k = lane; k < K; k += 64)
      acc += pl_ld<DT>(x, xb + k) * pl_ld<DT>(w.w, wb + (int64_t)k * w.s1 + (int64_t)n * w.s2);
    acc = pl_wave_sum(acc);
    if (lane == 0) reinterpret_cast<T*>(out)[row * n_max + n] = (T)acc;
  }
}

template <int DT>
__global__ __launch_bounds__(256) void pl_ref_expand(const void* __restrict__ x, int32_t B,
                                                     int32_t M, int32_t k_max, pl_ref_layout w,
                                                     int32_t N,
                                                     const int32_t* __restrict__ seq_lens,
                                                     const int32_t* __restrict__ widx,
                                                     const int32_t* __restrict__ ranks,
                                                     const float* __restrict__ scalings,
                                                     void* __restrict__ out, int32_t nblk) {
  typedef typename pl_traits<DT>::T T;
  const int64_t row = blockIdx.x / nblk;
  const int n = (int)(blockIdx.x - row * nblk) * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const int b = (int)(row / M);
  const int m = (int)(row - (int64_t)b * M);
  if (m >= seq_lens[b]) return;
  const int s = widx[b];
  if (s < 0 || s >= w.num_slots) return;
  const int rank = min(ranks[s], k_max);
  if (rank <= 0) return;
  const int64_t xb = row * k_max;
  const int64_t wb = (int64_t)s * w.s0 + (int64_t)n * w.s2;
  float acc = 0.f;
  for (int k = 0; k < rank; ++k) acc += pl_ld<DT>(x, xb + k) * pl_ld<DT>(w.w, wb + (int64_t)k * w.s1);
  T* o = reinterpret_cast<T*>(out) + row * N + n;
  const float scale = scalings[s];
  *o = (T)pl_epilogue<DT>(acc, (float)*o, scale, pl_round<DT>(scale), PL_EPI_TRITON);
}

// ---- slot arena layout ------------------------------------------------------

struct pl_rows_args {
  const void* x;
  int64_t ldx;
  int32_t K;
  void* y;
  int64_t ldy;
  int32_t N;
  const char* arena;
  const pl_slot_entry* table;
  int32_t num_slots;
  int32_t num_modules;
  int32_t module;
  const int32_t* row_slot;
  const int32_t* seq_lens;
  int32_t rows;
  int32_t row_len;
  float* tmp;
  int32_t ldt;
  int32_t epilogue;
  int32_t nblk;
};

// Slot-table entry of token t's row, or nullptr when the token gets no LoRA.
__device__ __forceinline__ const pl_slot_entry* pl_row_entry(const pl_rows_args& a, int64_t t) {
  const int b = (int)(t / a.row_len);
  const int m = (int)(t - (int64_t)b * a.row_len);
  if (m >= a.seq_lens[b]) return nullptr;
  const int s = a.row_slot[b];
  if (s <= 0 || s >= a.num_slots) return nullptr;
  const pl_slot_entry* e = a.table + (int64_t)s * a.num_modules + a.module;
  return e->rank > 0 ? e : nullptr;
}

template <int DT>
__global__ __launch_bounds__(256) void pl_rows_shrink(pl_rows_args a) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= (int64_t)a.rows * a.row_len) return;
  const pl_slot_entry* e = pl_row_entry(a, t);
  if (e == nullptr) return;
  const int rank = min(e->rank, a.ldt);
  const void* A = a.arena + e->a_off;
  for (int j = 0; j < rank; ++j) {
    float acc = 0.f;
    for (int k = lane; k < a.K; k += 64)
      acc += pl_ld<DT>(a.x, t * a.ldx + k) * pl_ld<DT>(A, pl_tile_off<DT>(j, k, e->rank, a.K));
    acc = pl_wave_sum(acc);
    if (lane == 0) a.tmp[t * a.ldt + j] = acc;
  }
}

template <int DT>
__global__ __launch_bounds__(256) void pl_rows_expand(pl_rows_args a) {
  typedef typename pl_traits<DT>::T T;
  const int64_t t = blockIdx.x / a.nblk;
  const int n = (int)(blockIdx.x - t * a.nblk) * blockDim.x + threadIdx.x;
  if (n >= a.N) return;
  const pl_slot_entry* e = pl_row_entry(a, t);
  if (e == nullptr) return;
  const int rank = min(e->rank, a.ldt);
  const int r8 = e->rank8;
  const void* Bc = a.arena + e->b_off;
  float acc = 0.f;
  for (int j = 0; j < rank; ++j)
    acc += pl_round<DT>(a.tmp[t * a.ldt + j]) * pl_ld<DT>(Bc, pl_tile_off<DT>(n, j, a.N, r8));
  T* o = reinterpret_cast<T*>(a.y) + t * a.ldy + n;
  *o = (T)pl_epilogue<DT>(acc, (float)*o, e->scale, pl_round<DT>(e->scale), a.epilogue);
}

bool valid_dtype(int32_t dtype) { return dtype == PL_F32 || dtype == PL_BF16 || dtype == PL_F16; }

// Instantiate `launch<DT>()` for the runtime dtype code.
template <typename F>
void pl_dispatch(int32_t dtype, F&& launch) {
  switch (dtype) {
    case PL_BF16: launch(std::integral_constant<int, PL_BF16>()); break;
    case PL_F16: launch(std::integral_constant<int, PL_F16>()); break;
    default: launch(std::integral_constant<int, PL_F32>()); break;
  }
}

// The shrink of the operator API: the MFMA path in the parts given (or in
// one workspace), else one wave per token row.
int ref_a(int32_t dtype, const void* x, int32_t B, int32_t M, int32_t K, const void* w,
          int64_t w_s0, int64_t w_s1, int64_t w_s2, int32_t num_adapters, int32_t n_max,
          const int32_t* seq_lens, const int32_t* weight_indices, const int32_t* lora_ranks,
          int32_t stack_num, void* out, void* workspace, int64_t workspace_bytes,
          const pl_refop_parts* parts, void* stream) {
  if (!valid_dtype(dtype)) {
    pl_set_error("unsupported dtype code %d", dtype);
    return PL_ERR_ARG;
  }
  if (B < 0 || M < 0 || K < 0 || n_max < 0 || stack_num < 1 || num_adapters < 0) {
    pl_set_error("pl_sgmv_lora_a_ref: bad sizes");
    return PL_ERR_ARG;
  }
  const int64_t rows = (int64_t)B * M;
  if (rows == 0 || n_max == 0 || num_adapters == 0) return PL_OK;
  if (!x || !w || !seq_lens || !weight_indices || !lora_ranks || !out) {
    pl_set_error("pl_sgmv_lora_a_ref: null pointer");
    return PL_ERR_ARG;
  }
  const int fast = pl_refop_shrink(dtype, x, B, M, K, w, w_s0, w_s1, w_s2, num_adapters, n_max,
                                   seq_lens, weight_indices, lora_ranks, stack_num, out, workspace,
                                   workspace_bytes, parts, stream);
  if (fast != PL_REFOP_DECLINED) return fast;
  const int64_t grid = (rows + 3) / 4;
  if (!pl_grid_fits(grid, 256)) {
    pl_set_error("pl_sgmv_lora_a_ref: too many rows");
    return PL_ERR_LIMIT;
  }
  const pl_ref_layout L{w, w_s0, w_s1, w_s2, num_adapters};
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  pl_dispatch(dtype, [&](auto dt) {
    hipLaunchKernelGGL(pl_ref_shrink<decltype(dt)::value>, dim3((unsigned)grid), dim3(256), 0, s, x,
                       B, M, K, L, n_max, seq_lens, weight_indices, lora_ranks, stack_num, out);
  });
  return pl_launch_status("pl_sgmv_lora_a_ref");
}

// The expand of the operator API, as ref_a.
int ref_b(int32_t dtype, const void* x, int32_t B, int32_t M, int32_t k_max, const void* w,
          int64_t w_s0, int64_t w_s1, int64_t w_s2, int32_t num_adapters, int32_t N,
          const int32_t* seq_lens, const int32_t* weight_indices, const int32_t* lora_ranks,
          const float* scalings, void* out, void* workspace, int64_t workspace_bytes,
          const pl_refop_parts* parts, void* stream) {
  if (!valid_dtype(dtype)) {
    pl_set_error("unsupported dtype code %d", dtype);
    return PL_ERR_ARG;
  }
  if (B < 0 || M < 0 || k_max < 0 || N < 0 || num_adapters < 0) {
    pl_set_error("pl_sgmv_lora_b_ref: bad sizes");
    return PL_ERR_ARG;
  }
  const int64_t rows = (int64_t)B * M;
  if (rows == 0 || N == 0 || num_adapters == 0) return PL_OK;
  if (!x || !w || !seq_lens || !weight_indices || !lora_ranks || !scalings || !out) {
    pl_set_error("pl_sgmv_lora_b_ref: null pointer");
    return PL_ERR_ARG;
  }
  const int fast = pl_refop_expand(dtype, x, B, M, k_max, w, w_s0, w_s1, w_s2, num_adapters, N,
                                   seq_lens, weight_indices, lora_ranks, scalings, out, workspace,
                                   workspace_bytes, parts, stream);
  if (fast != PL_REFOP_DECLINED) return fast;
  const int32_t nblk = (N + 255) / 256;
  if (!pl_grid_fits(rows * nblk, 256)) {
    pl_set_error("pl_sgmv_lora_b_ref: grid too large");
    return PL_ERR_LIMIT;
  }
  const pl_ref_layout L{w, w_s0, w_s1, w_s2, num_adapters};
  const dim3 grid((unsigned)(rows * nblk));
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  pl_dispatch(dtype, [&](auto dt) {
    hipLaunchKernelGGL(pl_ref_expand<decltype(dt)::value>, grid, dim3(256), 0, s, x, B, M, k_max,
                       L, N, seq_lens, weight_indices, lora_ranks, scalings, out, nblk);
  });
  return pl_launch_status("pl_sgmv_lora_b_ref");
}

pl_refop_parts make_parts(void* plan, int64_t plan_bytes, void* weights, int64_t weights_bytes,
                          void* scratch, int64_t scratch_bytes, int32_t flags, int32_t epoch) {
  pl_refop_parts P;
  P.plan = plan;
  P.plan_bytes = plan_bytes;
  P.weights = weights;
  P.weights_bytes = weights_bytes;
  P.scratch = scratch;
  P.scratch_bytes = scratch_bytes;
  P.flags = flags;
  P.epoch = epoch;
  return P;
}

}  // namespace

extern "C" int pl_sgmv_lora_a_ref(int32_t dtype, const void* x, int32_t B, int32_t M, int32_t K,
                                  const void* w, int64_t w_s0, int64_t w_s1, int64_t w_s2,
                                  int32_t num_adapters, int32_t n_max, const int32_t* seq_lens,
                                  const int32_t* weight_indices, const int32_t* lora_ranks,
                                  int32_t stack_num, void* out, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
  return ref_a(dtype, x, B, M, K, w, w_s0, w_s1, w_s2, num_adapters, n_max, seq_lens,
               weight_indices, lora_ranks, stack_num, out, workspace, workspace_bytes, nullptr,
               stream);
}

extern "C" int pl_sgmv_lora_b_ref(int32_t dtype, const void* x, int32_t B, int32_t M,
                                  int32_t k_max, const void* w, int64_t w_s0, int64_t w_s1,
                                  int64_t w_s2, int32_t num_adapters, int32_t N,
                                  const int32_t* seq_lens, const int32_t* weight_indices,
                                  const int32_t* lora_ranks, const float* scalings, void* out,
                                  void* workspace, int64_t workspace_bytes, void* stream) {
  return ref_b(dtype, x, B, M, k_max, w, w_s0, w_s1, w_s2, num_adapters, N, seq_lens,
               weight_indices, lora_ranks, scalings, out, workspace, workspace_bytes, nullptr,
               stream);
}

extern "C" int pl_sgmv_lora_a_ref_parts(int32_t dtype, const void* x, int32_t B, int32_t M,
                                        int32_t K, const void* w, int64_t w_s0, int64_t w_s1,
                                        int64_t w_s2, int32_t num_adapters, int32_t n_max,
                                        const int32_t* seq_lens, const int32_t* weight_indices,
                                        const int32_t* lora_ranks, int32_t stack_num, void* out,
                                        void* plan, int64_t plan_bytes, void* weights,
                                        int64_t weights_bytes, void* scratch,
                                        int64_t scratch_bytes, int32_t flags, int32_t epoch,
                                        void* stream) {
  const pl_refop_parts P =
      make_parts(plan, plan_bytes, weights, weights_bytes, scratch, scratch_bytes, flags, epoch);
  return ref_a(dtype, x, B, M, K, w, w_s0, w_s1, w_s2, num_adapters, n_max, seq_lens,
               weight_indices, lora_ranks, stack_num, out, nullptr, 0, &P, stream);
}

extern "C" int pl_sgmv_lora_b_ref_parts(int32_t dtype, const void* x, int32_t B, int32_t M,
                                        int32_t k_max, const void* w, int64_t w_s0, int64_t w_s1,
                                        int64_t w_s2, int32_t num_adapters, int32_t N,
                                        const int32_t* seq_lens, const int32_t* weight_indices,
                                        const int32_t* lora_ranks, const float* scalings,
                                        void* out, void* plan, int64_t plan_bytes, void* weights,
                                        int64_t weights_bytes, void* scratch,
                                        int64_t scratch_bytes, int32_t flags, int32_t epoch,
                                        void* stream) {
  const pl_refop_parts P =
      make_parts(plan, plan_bytes, weights, weights_bytes, scratch, scratch_bytes, flags, epoch);
  return ref_b(dtype, x, B, M, k_max, w, w_s0, w_s1, w_s2, num_adapters, N, seq_lens,
               weight_indices, lora_ranks, scalings, out, nullptr, 0, &P, stream);
}

extern "C" int pl_lora_apply_rows(int32_t dtype, const void* x, int64_t ldx, int32_t K, void* y,
                                  int64_t ldy, int32_t N, const void* arena,
                                  const pl_slot_entry* table, int32_t num_slots,
                                  int32_t num_modules, int32_t module, const int32_t* row_slot,
                                  const int32_t* seq_lens, int32_t rows, int32_t row_len,
                                  float* tmp, int32_t ldt, int32_t epilogue, void* stream) {
  if (!valid_dtype(dtype)) {
    pl_set_error("unsupported dtype code %d", dtype);
    return PL_ERR_ARG;
  }
  if (rows < 0 || row_len < 0 || K <= 0 || N <= 0 || ldx < K || ldy < N || ldt <= 0 ||
      num_slots < 1 || num_slots > PL_MAX_SLOTS || num_modules <= 0 || module < 0 ||
      module >= num_modules) {
    pl_set_error("pl_lora_apply_rows: bad sizes");
    return PL_ERR_ARG;
  }
  if (epilogue != PL_EPI_FALLBACK && epilogue != PL_EPI_TRITON) {
    pl_set_error("bad epilogue mode %d", epilogue);
    return PL_ERR_ARG;
  }
  const int64_t T = (int64_t)rows * row_len;
  if (T == 0) return PL_OK;
  if (!x || !y || !arena || !table || !row_slot || !seq_lens || !tmp) {
    pl_set_error("pl_lora_apply_rows: null pointer");
    return PL_ERR_ARG;
  }
  const int32_t nblk = (N + 255) / 256;
  if (!pl_grid_fits(T * nblk, 256)) {
    pl_set_error("pl_lora_apply_rows: grid too large");
    return PL_ERR_LIMIT;
  }
  pl_rows_args a;
  a.x = x;
  a.ldx = ldx;
  a.K = K;
  a.y = y;
  a.ldy = ldy;
  a.N = N;
  a.arena = reinterpret_cast<const char*>(arena);
  a.table = table;
  a.num_slots = num_slots;
  a.num_modules = num_modules;
  a.module = module;
  a.row_slot = row_slot;
  a.seq_lens = seq_lens;
  a.rows = rows;
  a.row_len = row_len;
  a.tmp = tmp;
  a.ldt = ldt;
  a.epilogue = epilogue;
  a.nblk = nblk;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 g1((unsigned)((T + 3) / 4));
  const dim3 g2((unsigned)(T * nblk));
  pl_dispatch(dtype, [&](auto dt) {
    hipLaunchKernelGGL(pl_rows_shrink<decltype(dt)::value>, g1, dim3(256), 0, s, a);
    hipLaunchKernelGGL(pl_rows_expand<decltype(dt)::value>, g2, dim3(256), 0, s, a);
  });
  return pl_launch_status("pl_lora_apply_rows");
}
