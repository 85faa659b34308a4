// Plan-building code shared by the plan kernel (plan.hip) and the
// reference-layout operator path (sgmv_refop.hip).
//
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
// per row for rows of up to 16 tokens, one wave per row for longer ones; a
// second set of LDS counters places them, so this step needs no barrier
// after the emission).  Row order inside a segment follows LDS atomic order
// and is not fixed; no consumer depends on it.
//
// Group placement.  Kernels give the work items of the group at position p
// to XCD p % 8 (workgroups are dealt to the 8 XCDs round-robin).  The plan
// puts the slot-major group list in 8 contiguous chunks, chunk x = groups
// [x*n/8, (x+1)*n/8) of the n groups, and the i-th group of chunk x at
// position 8*i + x, so an adapter's groups share one XCD's L2 (or two, where
// a chunk boundary splits it) instead of all eight, and its A and B come
// from HBM about once per launch.  Positions below 8*ceil(n/8) that get no
// group, and the rest of the capacity, hold empty records (slot 0, length 0).
#pragma once

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

// Where a row's slot comes from: a row -> slot map (pl_plan_build,
// ADAPTER_ROWS false: rows[b]), or a per-row adapter index as the
// reference's operator API passes it (ADAPTER_ROWS true: adapter i = rows[b]
// -> slot i + 1; an index outside [0, num_adapters) -> slot 0, and slot
// i + 1 is active only when ranks[i] > 0, so an adapter of rank 0 gets no
// tokens either).  The pointer stays a plain restrict parameter so that the
// token stores are known not to alias it.
template <bool ADAPTER_ROWS>
__device__ __forceinline__ int pl_row_slot(const int32_t* __restrict__ rows, int num_adapters,
                                           int b) {
  if constexpr (ADAPTER_ROWS) {
    const int w = rows[b];
    return w >= 0 && w < num_adapters ? w + 1 : 0;
  } else {
    return rows[b];
  }
}

// Slot and clamped length of row b, or slot 0 for a row that gets no tokens
// (its slot is 0, out of range or inactive, or its length is 0).
template <bool ADAPTER_ROWS>
__device__ __forceinline__ void pl_plan_row(const int32_t* __restrict__ row_src, int num_adapters,
                                            const int32_t* __restrict__ seq_lens, int b,
                                            int row_len, int S, const uint8_t* act, int& s,
                                            int& L) {
  s = pl_row_slot<ADAPTER_ROWS>(row_src, num_adapters, b);
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

// The plan, built by one workgroup of kPlanThreads threads.  row_src and
// num_adapters as for pl_row_slot; with ADAPTER_ROWS, slot s > 0 is active
// when ranks[s - 1] > 0 (active is then unused), otherwise when there is no
// active vector or active[s * active_stride] > 0.
template <bool ADAPTER_ROWS>
__device__ __forceinline__ void pl_plan_body(
    const int32_t* __restrict__ row_src, const int32_t* __restrict__ ranks, int32_t num_adapters,
    const int32_t* __restrict__ seq_lens, int32_t rows,
    int32_t row_len, int32_t num_slots, const int32_t* __restrict__ active, int64_t active_stride,
    int32_t group_tokens, int32_t* __restrict__ tok, pl_group* __restrict__ groups,
    int32_t* __restrict__ meta, int64_t group_cap) {
  // 16-byte aligned: each thread reads its 4 counters and writes its 4
  // offsets with one LDS access (a stride-4 word access conflicts 8 ways)
  __shared__ __attribute__((aligned(16))) int32_t cnt[PL_MAX_SLOTS];
  __shared__ uint8_t act[PL_MAX_SLOTS];  // slot s has work (active[s * stride] > 0, or no vector)
  __shared__ __attribute__((aligned(16))) int32_t off[PL_MAX_SLOTS];
  __shared__ __attribute__((aligned(16))) int32_t goff[PL_MAX_SLOTS];
  __shared__ int32_t fill[PL_MAX_SLOTS];  // tokens placed per slot by the scatter
  __shared__ int32_t wsum[2][kPlanThreads / 64];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int S = num_slots;

  for (int s = tid; s < S; s += kPlanThreads) {
    cnt[s] = 0;
    fill[s] = 0;
    if constexpr (ADAPTER_ROWS)
      act[s] = s > 0 && ranks[s - 1] > 0;
    else
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
      rs[q] = pl_row_slot<ADAPTER_ROWS>(row_src, num_adapters, b);
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
    pl_plan_row<ADAPTER_ROWS>(row_src, num_adapters, seq_lens, b, row_len, S, act, s, L);
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
  int ex_t, ex_g, tt, tg;
  if (S <= 4 * 64) {
    // every count is in wave 0's slots: its scan is the whole prefix, and
    // the totals reach the other waves through LDS at the barrier below
    ex_t = it - st;
    ex_g = ig - sg;
    tt = __shfl(it, 63);
    tg = __shfl(ig, 63);
    if (tid == 63) {
      wsum[0][0] = it;
      wsum[1][0] = ig;
    }
  } else {
    if (lane == 63) {
      wsum[0][wave] = it;
      wsum[1][wave] = ig;
    }
    __syncthreads();
    int wt = 0, wg = 0;
    tt = 0;
    tg = 0;
    for (int w = 0; w < kPlanThreads / 64; ++w) {
      if (w < wave) {
        wt += wsum[0][w];
        wg += wsum[1][w];
      }
      tt += wsum[0][w];
      tg += wsum[1][w];
    }
    ex_t = wt + it - st;
    ex_g = wg + ig - sg;
  }
  // entries past the slot count are written too (never read); with at most
  // 256 slots the other waves' entries are past it
  if (S > 4 * 64 || wave == 0) {
    reinterpret_cast<int4*>(off)[tid] =
        make_int4(ex_t + loc_t[0], ex_t + loc_t[1], ex_t + loc_t[2], ex_t + loc_t[3]);
    reinterpret_cast<int4*>(goff)[tid] =
        make_int4(ex_g + loc_g[0], ex_g + loc_g[1], ex_g + loc_g[2], ex_g + loc_g[3]);
  }
  if (tid == 0) {
    meta[0] = tg;
    meta[1] = tt;
    meta[2] = group_tokens;
    meta[3] = pl_plan_positions(tg);
  }
  __syncthreads();
  if (S <= 4 * 64) {
    tt = wsum[0][0];
    tg = wsum[1][0];
  }

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
  // the scatter reads off[] (complete since the last barrier) and fill[]
  // (cleared before the first one), so it needs no barrier after the groups
  // are written.  The token list holds rows * row_len entries; a position
  // outside it is never written (the offsets above keep every token inside)
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
        if (lane == 0) p0 = off[k0] + atomicAdd(&fill[k0], total);
        p = __builtin_amdgcn_readfirstlane(p0) + excl;
      } else if (rs[q] > 0) {
        p = off[rs[q]] + atomicAdd(&fill[rs[q]], rl[q]);
      }
      if (rs[q] > 0) {
        const int base = (tid + q * kPlanThreads) * row_len;
        for (int m = 0; m < rl[q]; ++m)
          if (p + m < cap) tok[p + m] = base + m;
      }
    }
    for (int b = tid + kPlanCached * kPlanThreads; b < rows; b += kPlanThreads) {
      int s, L;
      pl_plan_row<ADAPTER_ROWS>(row_src, num_adapters, seq_lens, b, row_len, S, act, s, L);
      if (s > 0) {
        const int p = off[s] + atomicAdd(&fill[s], L);
        const int base = b * row_len;
        for (int m = 0; m < L; ++m)
          if (p + m < cap) tok[p + m] = base + m;
      }
    }
  } else {
    // long rows (prefill): one wave per row
    for (int b = wave; b < rows; b += kPlanThreads / 64) {
      int s, L;
      pl_plan_row<ADAPTER_ROWS>(row_src, num_adapters, seq_lens, b, row_len, S, act, s, L);
      if (s > 0) {
        int p = 0;
        if (lane == 0) p = off[s] + atomicAdd(&fill[s], L);
        p = __shfl(p, 0);
        const int base = b * row_len;
        for (int m = lane; m < L; m += 64)
          if (p + m < cap) tok[p + m] = base + m;
      }
    }
  }
}

}  // namespace
