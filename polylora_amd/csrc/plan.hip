// Device-side per-forward plan: rows -> adapter-major token groups.
//
// Replaces the per-layer host schedule of sgmv.py:29-61 (two host syncs per
// wrapped Linear) with one single-workgroup kernel per forward whose output
// every wrapped Linear of that forward shares.  A row b with slot s > 0 and
// length L = min(max(seq_len, 0), row_len) contributes the L tokens
// b*row_len + m, m < L (the slicing x[b, :seq_len] of layers.py:127).
//
// Steps: per-slot token counts (LDS atomics), one block-wide exclusive scan
// of counts and of group counts, group emission (one thread per group), then
// the token indices of each row are copied to the slot's segment (one thread
// per row for rows of up to 16 tokens, one wave per row for longer ones).  Row order inside a
// segment follows LDS atomic order and is not fixed; no consumer depends on
// it.
//
// Group placement.  Kernels give the work items of the group at position p
// to XCD p % 8 (workgroups are dealt to the 8 XCDs round-robin).  The plan
// puts the slot-major group list in 8 contiguous chunks, chunk x = groups
// [x*n/8, (x+1)*n/8) of the n groups, and the i-th group of chunk x at
// position 8*i + x, so an adapter's groups share one XCD's L2 (or two, where
// a chunk boundary splits it) instead of all eight, and its A and B come
// from HBM about once per launch.  Positions below 8*ceil(n/8) that get no
// group, and the rest of the capacity, hold empty records (slot 0, length 0).
#include "pl_common.h"

namespace {

constexpr int kPlanThreads = 1024;
// Rows a plan thread keeps in registers: the first kPlanThreads * kPlanCached
// rows are read once, with all of a thread's loads in flight together, and
// serve both passes over the rows.  Rows beyond them are read per pass.
constexpr int kPlanCached = 8;

// Sum over the wave of v (0 <= v < 2^bits) and over the lanes below this
// one, from one ballot per bit: independent instructions, where a shuffle
// scan is a chain of LDS permutes.
__device__ __forceinline__ void pl_wave_sum(int v, int bits, int& excl, int& total) {
  const uint64_t below = __lanemask_lt();
  excl = 0;
  total = 0;
  for (int b = 0; b < bits; ++b) {
    const uint64_t m = __ballot((v >> b) & 1);
    total += __popcll(m) << b;
    excl += __popcll(m & below) << b;
  }
}

// Bits that hold any row length up to row_len.
__device__ __forceinline__ int pl_len_bits(int row_len) { return 32 - __clz(row_len | 1); }

// Inclusive prefix sum over the 64 lanes of a wave with DPP moves (register
// to register, no LDS): a Hillis-Steele scan inside each row of 16 lanes
// (row_shr 1, 2, 4, 8; lanes whose source lies before the row add 0), then
// lane 15 of rows 0 and 2 into rows 1 and 3 (row_bcast:15) and lane 31
// into rows 2 and 3 (row_bcast:31).
__device__ __forceinline__ int pl_wave_scan_incl(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15, rows 1 and 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31, rows 2 and 3
  return v;
}

// Slot and clamped length of row b, or slot 0 for a row that gets no tokens
// (its slot is 0, out of range or inactive, or its length is 0).
__device__ __forceinline__ void pl_plan_row(const int32_t* __restrict__ row_slot,
                                            const int32_t* __restrict__ seq_lens, int b,
                                            int row_len, int S, const uint8_t* act, int& s,
                                            int& L) {
  s = row_slot[b];
  L = seq_lens[b];
  L = L < 0 ? 0 : (L > row_len ? row_len : L);
  if (s <= 0 || s >= S || L <= 0 || !act[s]) s = 0;
}

// First slot-major group index of XCD chunk x (x = 0..8) of n groups.
__device__ __forceinline__ int pl_chunk_lo(int x, int n) { return (int)(((int64_t)x * n) / 8); }

// Position of slot-major group gi among n groups (see "Group placement").
__device__ __forceinline__ int64_t pl_plan_position(int gi, int n) {
  int x = 7;
  while (x > 0 && pl_chunk_lo(x, n) > gi) --x;
  return (int64_t)(gi - pl_chunk_lo(x, n)) * 8 + x;
}

__device__ __forceinline__ bool pl_plan_position_used(int64_t p, int n) {
  const int x = (int)(p & 7);
  const int64_t i = p >> 3;
  return pl_chunk_lo(x, n) + i < pl_chunk_lo(x + 1, n);
}

// Positions a plan of n groups spans: 8 * ceil(n / 8).
__device__ __forceinline__ int pl_plan_positions(int n) { return (n + 7) / 8 * 8; }

__global__ __launch_bounds__(kPlanThreads) void pl_plan_kernel(
    const int32_t* __restrict__ row_slot, const int32_t* __restrict__ seq_lens, int32_t rows,
    int32_t row_len, int32_t num_slots, const int32_t* __restrict__ active, int64_t active_stride,
    int32_t group_tokens, int32_t* __restrict__ tok, pl_group* __restrict__ groups,
    int32_t* __restrict__ meta, int64_t group_cap) {
  // 16-byte aligned: each thread reads its 4 counters and writes its 4
  // offsets with one LDS access (a stride-4 word access conflicts 8 ways)
  __shared__ __attribute__((aligned(16))) int32_t cnt[PL_MAX_SLOTS];
  __shared__ uint8_t act[PL_MAX_SLOTS];  // slot s has work (active[s * stride] > 0, or no vector)
  __shared__ __attribute__((aligned(16))) int32_t off[PL_MAX_SLOTS];
  __shared__ __attribute__((aligned(16))) int32_t goff[PL_MAX_SLOTS];
  __shared__ int32_t wsum[2][kPlanThreads / 64];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int S = num_slots;

  for (int s = tid; s < S; s += kPlanThreads) {
    cnt[s] = 0;
    act[s] = active == nullptr || active[(int64_t)s * active_stride] > 0;
  }
  // this thread's cached rows tid + q * kPlanThreads: all loads first
  int rs[kPlanCached], rl[kPlanCached];
#pragma unroll
  for (int q = 0; q < kPlanCached; ++q) {
    const int b = tid + q * kPlanThreads;
    rs[q] = 0;
    rl[q] = 0;
    if (b < rows) {
      rs[q] = row_slot[b];
      rl[q] = seq_lens[b];
    }
  }
  __syncthreads();  // act[] is complete
#pragma unroll
  for (int q = 0; q < kPlanCached; ++q) {
    int L = rl[q];
    L = L < 0 ? 0 : (L > row_len ? row_len : L);
    if (rs[q] <= 0 || rs[q] >= S || L <= 0 || !act[rs[q]]) rs[q] = 0;
    rl[q] = L;
  }

  // A wave whose rows all use one slot (a batch sorted by adapter) adds
  // them with one atomic: 64 lanes adding to one LDS counter serialize
  // (4096 rows sorted by slot: 3.3 us, shuffled: 1.0 us).
  const int len_bits = pl_len_bits(row_len);
#pragma unroll
  for (int q = 0; q < kPlanCached; ++q) {
    if (__ballot(rs[q] > 0) == 0) continue;  // wave-uniform
    const int k0 = __builtin_amdgcn_readfirstlane(rs[q]);
    if (__all(rs[q] == k0)) {
      int excl, total;
      pl_wave_sum(rl[q], len_bits, excl, total);
      if (lane == 0) atomicAdd(&cnt[k0], total);
    } else if (rs[q] > 0) {
      atomicAdd(&cnt[rs[q]], rl[q]);
    }
  }
  for (int b = tid + kPlanCached * kPlanThreads; b < rows; b += kPlanThreads) {
    int s, L;
    pl_plan_row(row_slot, seq_lens, b, row_len, S, act, s, L);
    if (s > 0) atomicAdd(&cnt[s], L);
  }
  __syncthreads();

  // Each thread owns 4 consecutive slots (PL_MAX_SLOTS == 4 * kPlanThreads);
  // counters past the slot count were never cleared and are not used.
  static_assert(PL_MAX_SLOTS == 4 * kPlanThreads, "four slots per plan thread");
  const int4 c4 = reinterpret_cast<const int4*>(cnt)[tid];
  const int cq[4] = {c4.x, c4.y, c4.z, c4.w};
  int loc_t[4], loc_g[4];
  int st = 0, sg = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int c = tid * 4 + q < S ? cq[q] : 0;
    loc_t[q] = st;
    loc_g[q] = sg;
    st += c;
    sg += (c + group_tokens - 1) / group_tokens;
  }
  const int it = pl_wave_scan_incl(st);
  const int ig = pl_wave_scan_incl(sg);
  if (lane == 63) {
    wsum[0][wave] = it;
    wsum[1][wave] = ig;
  }
  __syncthreads();
  int wt = 0, wg = 0, tt = 0, tg = 0;
  for (int w = 0; w < kPlanThreads / 64; ++w) {
    if (w < wave) {
      wt += wsum[0][w];
      wg += wsum[1][w];
    }
    tt += wsum[0][w];
    tg += wsum[1][w];
  }
  const int ex_t = wt + it - st;
  const int ex_g = wg + ig - sg;
  // entries past the slot count are written too (never read)
  reinterpret_cast<int4*>(off)[tid] =
      make_int4(ex_t + loc_t[0], ex_t + loc_t[1], ex_t + loc_t[2], ex_t + loc_t[3]);
  reinterpret_cast<int4*>(goff)[tid] =
      make_int4(ex_g + loc_g[0], ex_g + loc_g[1], ex_g + loc_g[2], ex_g + loc_g[3]);
  if (tid == 0) {
    meta[0] = tg;
    meta[1] = tt;
    meta[2] = group_tokens;
    meta[3] = pl_plan_positions(tg);
  }
  __syncthreads();

  // One thread per group (a slot can have hundreds): the group's slot is
  // the last s with goff[s] <= gi (a slot with no groups shares its goff
  // with the next slot, so the last such s is the one that has groups).
  for (int gi = tid; gi < tg; gi += kPlanThreads) {
    int lo = 0, hi = S - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (goff[mid] <= gi)
        lo = mid;
      else
        hi = mid - 1;
    }
    const int q = gi - goff[lo];
    const int64_t p = pl_plan_position(gi, tg);
    if (p < group_cap) {
      pl_group gr;
      gr.slot = lo;
      gr.start = off[lo] + q * group_tokens;
      gr.len = min(group_tokens, cnt[lo] - q * group_tokens);
      gr.reserved = 0;
      groups[p] = gr;
    }
  }
  // Every other position up to the capacity holds an empty group (slot 0,
  // length 0), so a kernel may read any record below group_cap without first
  // reading meta.
  for (int64_t p = tid; p < group_cap; p += kPlanThreads) {
    if (!pl_plan_position_used(p, tg)) {
      pl_group gr;
      gr.slot = 0;
      gr.start = 0;
      gr.len = 0;
      gr.reserved = 0;
      groups[p] = gr;
    }
  }
  __syncthreads();
  for (int s = tid; s < S; s += kPlanThreads) cnt[s] = 0;  // reused as fill counters
  __syncthreads();
  // the token list holds rows * row_len entries; a position outside it is
  // never written (the offsets above keep every token inside it)
  const int64_t cap = (int64_t)rows * row_len;

  if (row_len <= 16) {
    // short rows (decode, flattened tokens): one thread per row
#pragma unroll
    for (int q = 0; q < kPlanCached; ++q) {
      if (__ballot(rs[q] > 0) == 0) continue;  // wave-uniform
      const int k0 = __builtin_amdgcn_readfirstlane(rs[q]);
      int p = 0;
      if (__all(rs[q] == k0)) {
        int excl, total;
        pl_wave_sum(rl[q], len_bits, excl, total);
        int p0 = 0;
        if (lane == 0) p0 = off[k0] + atomicAdd(&cnt[k0], total);
        p = __builtin_amdgcn_readfirstlane(p0) + excl;
      } else if (rs[q] > 0) {
        p = off[rs[q]] + atomicAdd(&cnt[rs[q]], rl[q]);
      }
      if (rs[q] > 0) {
        const int base = (tid + q * kPlanThreads) * row_len;
        for (int m = 0; m < rl[q]; ++m)
          if (p + m < cap) tok[p + m] = base + m;
      }
    }
    for (int b = tid + kPlanCached * kPlanThreads; b < rows; b += kPlanThreads) {
      int s, L;
      pl_plan_row(row_slot, seq_lens, b, row_len, S, act, s, L);
      if (s > 0) {
        const int p = off[s] + atomicAdd(&cnt[s], L);
        const int base = b * row_len;
        for (int m = 0; m < L; ++m)
          if (p + m < cap) tok[p + m] = base + m;
      }
    }
  } else {
    // long rows (prefill): one wave per row
    for (int b = wave; b < rows; b += kPlanThreads / 64) {
      int s, L;
      pl_plan_row(row_slot, seq_lens, b, row_len, S, act, s, L);
      if (s > 0) {
        int p = 0;
        if (lane == 0) p = off[s] + atomicAdd(&cnt[s], L);
        p = __shfl(p, 0);
        const int base = b * row_len;
        for (int m = lane; m < L; m += 64)
          if (p + m < cap) tok[p + m] = base + m;
      }
    }
  }
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
  if (grid > 0x7fffffffLL) {
    pl_set_error("pl_check_right_padded: mask too large");
    return PL_ERR_LIMIT;
  }
  hipLaunchKernelGGL(pl_right_pad_kernel, dim3((unsigned)grid), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), mask, mask_dtype, B, S, seq_lens,
                     flag);
  return pl_launch_status("pl_check_right_padded");
}
