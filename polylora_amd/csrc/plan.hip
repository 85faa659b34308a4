// Device-side per-forward plan (pl_plan_build): the kernel around the plan
// body of pl_plan_body.h, the group-capacity bound, and the right-padding
// check of an attention mask.
#include "pl_plan_body.h"

namespace {

__global__ __launch_bounds__(kPlanThreads) void pl_plan_kernel(
    const int32_t* __restrict__ row_slot, const int32_t* __restrict__ seq_lens, int32_t rows,
    int32_t row_len, int32_t num_slots, const int32_t* __restrict__ active, int64_t active_stride,
    int32_t group_tokens, int32_t* __restrict__ tok, pl_group* __restrict__ groups,
    int32_t* __restrict__ meta, int64_t group_cap) {
  pl_plan_body<false>(row_slot, 0, seq_lens, rows, row_len, num_slots, active,
                      active_stride, group_tokens, tok, groups, meta, group_cap);
}

template <typename M>
__device__ __forceinline__ bool pl_mask_on(const void* mask, int64_t i) {
  return reinterpret_cast<const M*>(mask)[i] != M(0);
}

__global__ __launch_bounds__(256) void pl_right_pad_kernel(const void* __restrict__ mask,
                                                           int32_t mask_dtype, int32_t B,
                                                           int32_t S,
                                                           const int32_t* __restrict__ seq_lens,
                                                           int32_t* __restrict__ flag) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)B * S) return;
  const int b = (int)(i / S);
  const int s = (int)(i - (int64_t)b * S);
  bool on;
  switch (mask_dtype) {
    case 0: on = pl_mask_on<int64_t>(mask, i); break;
    case 1: on = pl_mask_on<int32_t>(mask, i); break;
    case 2: on = pl_mask_on<uint8_t>(mask, i); break;
    case 3: on = pl_mask_on<float>(mask, i); break;
    case 4: on = (reinterpret_cast<const uint16_t*>(mask)[i] & 0x7fffu) != 0; break;
    default: on = (reinterpret_cast<const uint16_t*>(mask)[i] & 0x7fffu) != 0; break;
  }
  const bool expect = s < seq_lens[b];
  if (on != expect) *flag = 1;  // every writer stores the same value
}

}  // namespace

extern "C" int64_t pl_plan_group_capacity(int32_t rows, int32_t row_len, int32_t num_slots,
                                          int32_t group_tokens) {
  if (rows < 0 || row_len < 0 || num_slots < 1 || group_tokens < 1) return 0;
  const int64_t t = (int64_t)rows * row_len;
  // at most ceil(t/G) + num_slots - 1 groups, placed below 8 * ceil(groups / 8)
  const int64_t n = (t + group_tokens - 1) / group_tokens + (num_slots - 1);
  return (n + 7) / 8 * 8;
}

namespace {

int plan_build(const int32_t* row_slot, const int32_t* seq_lens, int32_t rows, int32_t row_len,
               int32_t num_slots, const int32_t* active, int64_t active_stride,
               int32_t group_tokens, int32_t* tok, pl_group* groups, int32_t* meta,
               int64_t group_cap, void* stream) {
  if (!meta || (rows > 0 && (!row_slot || !seq_lens || !tok || !groups))) {
    pl_set_error("pl_plan_build: null pointer");
    return PL_ERR_ARG;
  }
  if (rows < 0 || row_len < 0 || num_slots < 1) {
    pl_set_error("pl_plan_build: bad sizes rows=%d row_len=%d num_slots=%d", rows, row_len,
                 num_slots);
    return PL_ERR_ARG;
  }
  if (active != nullptr && active_stride < 0) {
    pl_set_error("pl_plan_build: negative stride of the active-slot vector");
    return PL_ERR_ARG;
  }
  if (group_tokens != 16 && group_tokens != 64) {
    pl_set_error("pl_plan_build: group_tokens must be 16 or 64 (got %d)", group_tokens);
    return PL_ERR_ARG;
  }
  if (num_slots > PL_MAX_SLOTS) {
    pl_set_error("pl_plan_build: %d slots exceed the maximum of %d", num_slots, PL_MAX_SLOTS);
    return PL_ERR_LIMIT;
  }
  if ((int64_t)rows * row_len > 0x7fffffffLL) {
    pl_set_error("pl_plan_build: rows*row_len exceeds 2^31-1");
    return PL_ERR_LIMIT;
  }
  if (group_cap < pl_plan_group_capacity(rows, row_len, num_slots, group_tokens)) {
    pl_set_error("pl_plan_build: group capacity %lld below the bound %lld", (long long)group_cap,
                 (long long)pl_plan_group_capacity(rows, row_len, num_slots, group_tokens));
    return PL_ERR_ARG;
  }
  hipLaunchKernelGGL(pl_plan_kernel, dim3(1), dim3(kPlanThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), row_slot, seq_lens, rows, row_len,
                     num_slots, active, active_stride, group_tokens, tok, groups, meta, group_cap);
  return pl_launch_status("pl_plan_build");
}

}  // namespace

extern "C" int pl_plan_build(const int32_t* row_slot, const int32_t* seq_lens, int32_t rows,
                             int32_t row_len, int32_t num_slots, int32_t group_tokens,
                             int32_t* tok, pl_group* groups, int32_t* meta, int64_t group_cap,
                             void* stream) {
  return plan_build(row_slot, seq_lens, rows, row_len, num_slots, nullptr, 0, group_tokens, tok,
                    groups, meta, group_cap, stream);
}

extern "C" int pl_plan_build_active(const int32_t* row_slot, const int32_t* seq_lens,
                                    int32_t rows, int32_t row_len, int32_t num_slots,
                                    const int32_t* slot_active, int64_t active_stride,
                                    int32_t group_tokens, int32_t* tok, pl_group* groups,
                                    int32_t* meta, int64_t group_cap, void* stream) {
  if (!slot_active) {
    pl_set_error("pl_plan_build_active: null active-slot vector");
    return PL_ERR_ARG;
  }
  return plan_build(row_slot, seq_lens, rows, row_len, num_slots, slot_active, active_stride,
                    group_tokens, tok, groups, meta, group_cap, stream);
}

extern "C" int pl_check_right_padded(const void* mask, int32_t mask_dtype, int32_t B, int32_t S,
                                     const int32_t* seq_lens, int32_t* flag, void* stream) {
  if (!flag || (B > 0 && S > 0 && (!mask || !seq_lens))) {
    pl_set_error("pl_check_right_padded: null pointer");
    return PL_ERR_ARG;
  }
  if (B < 0 || S < 0 || mask_dtype < 0 || mask_dtype > 5) {
    pl_set_error("pl_check_right_padded: bad arguments");
    return PL_ERR_ARG;
  }
  const int64_t n = (int64_t)B * S;
  if (n == 0) return PL_OK;
  const int64_t grid = (n + 255) / 256;
  if (!pl_grid_fits(grid, 256)) {
    pl_set_error("pl_check_right_padded: mask too large");
    return PL_ERR_LIMIT;
  }
  hipLaunchKernelGGL(pl_right_pad_kernel, dim3((unsigned)grid), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), mask, mask_dtype, B, S, seq_lens,
                     flag);
  return pl_launch_status("pl_check_right_padded");
}
