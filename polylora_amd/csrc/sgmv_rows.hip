// Row-based SGMV kernels: any shape, stride and alignment.
//
// They serve two callers: the reference-layout operator API
// (sgmv_lora_a_fwd / sgmv_lora_b_fwd, sgmv.py:141-175 and :278-328, weights
// [slots][k][n] with arbitrary strides) and MultiLoraLinear shapes the tiled
// kernels reject (K or N not a multiple of the 16-byte chunk, unaligned rows).
// Throughput is not their goal; the tiled kernels carry the hot path.
//
// Shrink: one wave per token row; lanes stride K, each rank column is a
// wave-wide dot product finished with a butterfly reduction.
// Expand: one thread per output element; loop over the adapter's rank.
#include "pl_common.h"

namespace {

// Weight access for the two layouts.
struct pl_ref_layout {
  const void* w;
  int64_t s0, s1, s2;  // element strides of [slot][k][n]
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

template <int DT>
__global__ __launch_bounds__(256) void pl_rows_shrink(
    const void* __restrict__ x, int64_t ldx, int32_t K, const char* __restrict__ arena,
    const pl_slot_entry* __restrict__ table, int32_t num_modules, int32_t module,
    const int32_t* __restrict__ row_slot, const int32_t* __restrict__ seq_lens, int32_t rows,
    int32_t row_len, float* __restrict__ tmp, int32_t ldt) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= (int64_t)rows * row_len) return;
  const int b = (int)(t / row_len);
  const int m = (int)(t - (int64_t)b * row_len);
  if (m >= seq_lens[b]) return;
  const int s = row_slot[b];
  if (s <= 0) return;
  const pl_slot_entry e = table[(int64_t)s * num_modules + module];
  if (e.rank <= 0) return;
  const void* A = arena + e.a_off;
  for (int j = 0; j < e.rank; ++j) {
    float acc = 0.f;
    for (int k = lane; k < K; k += 64)
      acc += pl_ld<DT>(x, t * ldx + k) * pl_ld<DT>(A, (int64_t)j * K + k);
    acc = pl_wave_sum(acc);
    if (lane == 0) tmp[t * ldt + j] = acc;
  }
}

template <int DT>
__global__ __launch_bounds__(256) void pl_rows_expand(
    const float* __restrict__ tmp, int32_t ldt, const char* __restrict__ arena,
    const pl_slot_entry* __restrict__ table, int32_t num_modules, int32_t module,
    const int32_t* __restrict__ row_slot, const int32_t* __restrict__ seq_lens,
    int32_t row_len, void* __restrict__ y, int64_t ldy, int32_t N, int32_t epilogue,
    int32_t nblk) {
  typedef typename pl_traits<DT>::T T;
  const int64_t t = blockIdx.x / nblk;
  const int n = (int)(blockIdx.x - t * nblk) * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const int b = (int)(t / row_len);
  const int m = (int)(t - (int64_t)b * row_len);
  if (m >= seq_lens[b]) return;
  const int s = row_slot[b];
  if (s <= 0) return;
  const pl_slot_entry e = table[(int64_t)s * num_modules + module];
  if (e.rank <= 0) return;
  const void* Bc = arena + e.b_off;
  float acc = 0.f;
  for (int j = 0; j < e.rank; ++j)
    acc += pl_round<DT>(tmp[t * ldt + j]) * pl_ld<DT>(Bc, (int64_t)n * e.rank8 + j);
  T* o = reinterpret_cast<T*>(y) + t * ldy + n;
  *o = (T)pl_epilogue<DT>(acc, (float)*o, e.scale, pl_round<DT>(e.scale), epilogue);
}

bool valid_dtype(int32_t dtype) { return dtype == PL_F32 || dtype == PL_BF16 || dtype == PL_F16; }

}  // namespace

extern "C" int pl_sgmv_lora_a_ref(int32_t dtype, const void* x, int32_t B, int32_t M, int32_t K,
                                  const void* w, int64_t w_s0, int64_t w_s1, int64_t w_s2,
                                  int32_t n_max, const int32_t* seq_lens,
                                  const int32_t* weight_indices, const int32_t* lora_ranks,
                                  int32_t stack_num, void* out, void* stream) {
  if (!valid_dtype(dtype)) {
    pl_set_error("unsupported dtype code %d", dtype);
    return PL_ERR_ARG;
  }
  if (B < 0 || M < 0 || K < 0 || n_max < 0 || stack_num < 1) {
    pl_set_error("pl_sgmv_lora_a_ref: bad sizes");
    return PL_ERR_ARG;
  }
  const int64_t rows = (int64_t)B * M;
  if (rows == 0 || n_max == 0) return PL_OK;
  if (!x || !w || !seq_lens || !weight_indices || !lora_ranks || !out) {
    pl_set_error("pl_sgmv_lora_a_ref: null pointer");
    return PL_ERR_ARG;
  }
  const int64_t grid = (rows + 3) / 4;
  if (grid > 0x7fffffffLL) {
    pl_set_error("pl_sgmv_lora_a_ref: too many rows");
    return PL_ERR_LIMIT;
  }
  pl_ref_layout L{w, w_s0, w_s1, w_s2};
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (dtype) {
    case PL_BF16:
      hipLaunchKernelGGL(pl_ref_shrink<PL_BF16>, dim3((unsigned)grid), dim3(256), 0, s, x, B, M, K,
                         L, n_max, seq_lens, weight_indices, lora_ranks, stack_num, out);
      break;
    case PL_F16:
      hipLaunchKernelGGL(pl_ref_shrink<PL_F16>, dim3((unsigned)grid), dim3(256), 0, s, x, B, M, K,
                         L, n_max, seq_lens, weight_indices, lora_ranks, stack_num, out);
      break;
    default:
      hipLaunchKernelGGL(pl_ref_shrink<PL_F32>, dim3((unsigned)grid), dim3(256), 0, s, x, B, M, K,
                         L, n_max, seq_lens, weight_indices, lora_ranks, stack_num, out);
  }
  return pl_launch_status("pl_sgmv_lora_a_ref");
}

extern "C" int pl_sgmv_lora_b_ref(int32_t dtype, const void* x, int32_t B, int32_t M,
                                  int32_t k_max, const void* w, int64_t w_s0, int64_t w_s1,
                                  int64_t w_s2, int32_t N, const int32_t* seq_lens,
                                  const int32_t* weight_indices, const int32_t* lora_ranks,
                                  const float* scalings, void* out, void* stream) {
  if (!valid_dtype(dtype)) {
    pl_set_error("unsupported dtype code %d", dtype);
    return PL_ERR_ARG;
  }
  if (B < 0 || M < 0 || k_max < 0 || N < 0) {
    pl_set_error("pl_sgmv_lora_b_ref: bad sizes");
    return PL_ERR_ARG;
  }
  const int64_t rows = (int64_t)B * M;
  if (rows == 0 || N == 0) return PL_OK;
  if (!x || !w || !seq_lens || !weight_indices || !lora_ranks || !scalings || !out) {
    pl_set_error("pl_sgmv_lora_b_ref: null pointer");
    return PL_ERR_ARG;
  }
  const int32_t nblk = (N + 255) / 256;
  if (rows * nblk > 0x7fffffffLL) {
    pl_set_error("pl_sgmv_lora_b_ref: grid too large");
    return PL_ERR_LIMIT;
  }
  pl_ref_layout L{w, w_s0, w_s1, w_s2};
  dim3 grid((unsigned)(rows * nblk));
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (dtype) {
    case PL_BF16:
      hipLaunchKernelGGL(pl_ref_expand<PL_BF16>, grid, dim3(256), 0, s, x, B, M, k_max, L, N,
                         seq_lens, weight_indices, lora_ranks, scalings, out, nblk);
      break;
    case PL_F16:
      hipLaunchKernelGGL(pl_ref_expand<PL_F16>, grid, dim3(256), 0, s, x, B, M, k_max, L, N,
                         seq_lens, weight_indices, lora_ranks, scalings, out, nblk);
      break;
    default:
      hipLaunchKernelGGL(pl_ref_expand<PL_F32>, grid, dim3(256), 0, s, x, B, M, k_max, L, N,
                         seq_lens, weight_indices, lora_ranks, scalings, out, nblk);
  }
  return pl_launch_status("pl_sgmv_lora_b_ref");
}

extern "C" int pl_lora_apply_rows(int32_t dtype, const void* x, int64_t ldx, int32_t K, void* y,
                                  int64_t ldy, int32_t N, const void* arena,
                                  const pl_slot_entry* table, int32_t num_modules,
                                  int32_t module, const int32_t* row_slot,
                                  const int32_t* seq_lens, int32_t rows, int32_t row_len,
                                  float* tmp, int32_t ldt, int32_t epilogue, void* stream) {
  if (!valid_dtype(dtype)) {
    pl_set_error("unsupported dtype code %d", dtype);
    return PL_ERR_ARG;
  }
  if (rows < 0 || row_len < 0 || K <= 0 || N <= 0 || ldx < K || ldy < N || ldt <= 0 ||
      num_modules <= 0 || module < 0 || module >= num_modules) {
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
  if (T * nblk > 0x7fffffffLL) {
    pl_set_error("pl_lora_apply_rows: grid too large");
    return PL_ERR_LIMIT;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const char* ar = reinterpret_cast<const char*>(arena);
  dim3 g1((unsigned)((T + 3) / 4));
  dim3 g2((unsigned)(T * nblk));
  switch (dtype) {
    case PL_BF16:
      hipLaunchKernelGGL(pl_rows_shrink<PL_BF16>, g1, dim3(256), 0, s, x, ldx, K, ar, table,
                         num_modules, module, row_slot, seq_lens, rows, row_len, tmp, ldt);
      hipLaunchKernelGGL(pl_rows_expand<PL_BF16>, g2, dim3(256), 0, s, tmp, ldt, ar, table,
                         num_modules, module, row_slot, seq_lens, row_len, y, ldy, N, epilogue, nblk);
      break;
    case PL_F16:
      hipLaunchKernelGGL(pl_rows_shrink<PL_F16>, g1, dim3(256), 0, s, x, ldx, K, ar, table,
                         num_modules, module, row_slot, seq_lens, rows, row_len, tmp, ldt);
      hipLaunchKernelGGL(pl_rows_expand<PL_F16>, g2, dim3(256), 0, s, tmp, ldt, ar, table,
                         num_modules, module, row_slot, seq_lens, row_len, y, ldy, N, epilogue, nblk);
      break;
    default:
      hipLaunchKernelGGL(pl_rows_shrink<PL_F32>, g1, dim3(256), 0, s, x, ldx, K, ar, table,
                         num_modules, module, row_slot, seq_lens, rows, row_len, tmp, ldt);
      hipLaunchKernelGGL(pl_rows_expand<PL_F32>, g2, dim3(256), 0, s, tmp, ldt, ar, table,
                         num_modules, module, row_slot, seq_lens, row_len, y, ldy, N, epilogue, nblk);
  }
  return pl_launch_status("pl_lora_apply_rows");
}
