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
// Steps: per-slot token counts (LDS atomics), one exclusive scan of counts
// and of group counts, group emission (one thread per group), then the token
// indices of each row are written to the slot's segment (one thread per 4
// rows for rows of up to 16 tokens, one wave per row for longer ones; a
// second set of LDS counters places them, so this step needs no barrier
// after the emission).  Row order inside a segment follows LDS atomic order and is not
// fixed; no consumer depends on it.
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
// -> slot i + 1; an index outside [0, num_adapters) -> slot 0).  The plan
// does not look at ranks: an adapter of rank 0 gets its groups like any
// other, and every kernel that consumes the plan returns at once for a slot
// whose table entry has rank 0, so one plan serves every module of a
// forward, whatever each module's ranks.  The pointer stays a plain
// restrict parameter so that the token stores are known not to alias it.
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

// A plan thread takes kPlanRun consecutive rows per pass (one 16-byte load
// of each input array where they are aligned); kPlanChunk rows per pass of
// the workgroup.  The first pass's rows stay in registers for the scatter.
constexpr int kPlanRun = 4;
constexpr int kPlanChunk = kPlanThreads * kPlanRun;

// Slots and lengths of rows b0 .. b0 + 3 (rows > 0; indices past the last
// row are clamped to it, and masked by pl_plan_mask4).
template <bool ADAPTER_ROWS>
__device__ __forceinline__ void pl_plan_load4(const int32_t* __restrict__ row_src, int num_adapters,
                                              const int32_t* __restrict__ seq_lens, int b0,
                                              int rows, bool vec, int (&s)[kPlanRun],
                                              int (&L)[kPlanRun]) {
  if (vec && b0 + kPlanRun <= rows) {
    const int4 a = *reinterpret_cast<const int4*>(row_src + b0);
    const int4 l = *reinterpret_cast<const int4*>(seq_lens + b0);
    s[0] = a.x, s[1] = a.y, s[2] = a.z, s[3] = a.w;
    L[0] = l.x, L[1] = l.y, L[2] = l.z, L[3] = l.w;
    if constexpr (ADAPTER_ROWS) {
#pragma unroll
      for (int i = 0; i < kPlanRun; ++i) s[i] = s[i] >= 0 && s[i] < num_adapters ? s[i] + 1 : 0;
    }
  } else {
#pragma unroll
    for (int i = 0; i < kPlanRun; ++i) {
      const int b = min(b0 + i, rows - 1);
      s[i] = pl_row_slot<ADAPTER_ROWS>(row_src, num_adapters, b);
      L[i] = seq_lens[b];
    }
  }
}

// Clamp lengths to [0, row_len]; slot 0 for a row that gets no tokens (past
// the last row, slot 0 or out of range, inactive, or length 0).
__device__ __forceinline__ void pl_plan_mask4(int b0, int rows, int row_len, int S,
                                              const uint8_t* act, int (&s)[kPlanRun],
                                              int (&L)[kPlanRun]) {
  uint8_t on[kPlanRun];
#pragma unroll
  for (int i = 0; i < kPlanRun; ++i) on[i] = act[s[i] > 0 && s[i] < S ? s[i] : 0];
#pragma unroll
  for (int i = 0; i < kPlanRun; ++i) {
    const int l = L[i] < 0 ? 0 : (L[i] > row_len ? row_len : L[i]);
    s[i] = b0 + i < rows && l > 0 && on[i] ? s[i] : 0;
    L[i] = l;
  }
}

// Slot shared by every row of this wave's pass (all 4 * 64 rows), or 0.
__device__ __forceinline__ int pl_plan_wave_slot(const int (&s)[kPlanRun]) {
  const int k0 = __builtin_amdgcn_readfirstlane(s[0]);
  bool same = true;
#pragma unroll
  for (int i = 0; i < kPlanRun; ++i) same = same && s[i] == k0;
  return k0 > 0 && __all(same) ? k0 : 0;
}

// Claim places for this thread's rows in per-slot counters ctr: pos[i] is
// row i's first place counted from the slot's counter's start.  One atomic
// per wave when the wave's rows share one slot (64 lanes adding to one LDS
// counter serialize), else one per run of equal slots in the thread's rows.
// With CLAIM false only the counts are added.
template <bool CLAIM>
__device__ __forceinline__ void pl_plan_claim4(const int (&s)[kPlanRun], const int (&L)[kPlanRun],
                                               int lane, int32_t* ctr, int (&pos)[kPlanRun]) {
  const int k = pl_plan_wave_slot(s);
  if (k > 0) {
    int t = 0;
#pragma unroll
    for (int i = 0; i < kPlanRun; ++i) t += L[i];
    const int incl = pl_wave_scan_incl(t);
    if constexpr (CLAIM) {
      int p0 = 0;
      if (lane == 63) p0 = atomicAdd(&ctr[k], incl);  // lane 63 holds the wave's total
      int p = __builtin_amdgcn_readlane(p0, 63) + incl - t;
#pragma unroll
      for (int i = 0; i < kPlanRun; ++i) {
        pos[i] = p;
        p += L[i];
      }
    } else if (lane == 63) {
      atomicAdd(&ctr[k], incl);
    }
  } else {
    int first = 0, acc = 0;
#pragma unroll
    for (int i = 0; i <= kPlanRun; ++i) {
      if (i == kPlanRun || (i > 0 && s[i] != s[i - 1])) {
        if (s[i - 1] > 0) {
          if constexpr (CLAIM) {
            int p = atomicAdd(&ctr[s[i - 1]], acc);
            for (int j = first; j < i; ++j) {
              pos[j] = p;
              p += L[j];
            }
          } else {
            atomicAdd(&ctr[s[i - 1]], acc);
          }
        }
        first = i;
        acc = 0;
      }
      if (i < kPlanRun) acc += L[i];
    }
  }
}

// Token indices b * row_len + m, m < L, of this thread's rows (of at most 16
// tokens) from place base[slot] + pos[i] of the token list, which holds cap
// entries; a place outside it is never written.
__device__ __forceinline__ void pl_plan_store4(const int (&s)[kPlanRun], const int (&L)[kPlanRun],
                                               const int (&pos)[kPlanRun], int b0, int row_len,
                                               const int32_t* base, int32_t* __restrict__ tok,
                                               int64_t cap) {
#pragma unroll
  for (int i = 0; i < kPlanRun; ++i) {
    if (s[i] > 0) {
      const int p = base[s[i]] + pos[i];
      const int t = (b0 + i) * row_len;
      for (int m = 0; m < L[i]; ++m)
        if (p + m < cap) tok[p + m] = t + m;
    }
  }
}

// The plan, built by one workgroup of kPlanThreads threads.  row_src and
// num_adapters as for pl_row_slot; slot s > 0 is active when there is no
// active vector or active[s * active_stride] > 0.
//
// All of it runs on one CU, whose four SIMDs issue one wave64 instruction
// per 4 cycles each, so the cost is the waves' instruction count: a thread
// takes 4 consecutive rows, a wave whose rows share one slot claims its
// counts and places with one atomic, and only the waves that have rows,
// slots or groups run each step.
template <bool ADAPTER_ROWS>
__device__ __forceinline__ void pl_plan_body(
    const int32_t* __restrict__ row_src, int32_t num_adapters,
    const int32_t* __restrict__ seq_lens, int32_t rows,
    int32_t row_len, int32_t num_slots, const int32_t* __restrict__ active, int64_t active_stride,
    int32_t group_tokens, int32_t* __restrict__ tok, pl_group* __restrict__ groups,
    int32_t* __restrict__ meta, int64_t group_cap) {
  // 16-byte aligned: each thread reads or writes its 4 slots' words with one
  // LDS access (a stride-4 word access conflicts 8 ways)
  __shared__ __attribute__((aligned(16))) int32_t cnt[PL_MAX_SLOTS];
  __shared__ __attribute__((aligned(16))) uint8_t act[PL_MAX_SLOTS];  // slot s has work
  __shared__ __attribute__((aligned(16))) int32_t off[PL_MAX_SLOTS];
  __shared__ __attribute__((aligned(16))) int32_t goff[PL_MAX_SLOTS];
  __shared__ __attribute__((aligned(16))) int32_t fill[PL_MAX_SLOTS];  // tokens placed per slot
  __shared__ int32_t wsum[2][kPlanThreads / 64];
  static_assert(PL_MAX_SLOTS == 4 * kPlanThreads, "four slots per plan thread");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int S = num_slots;
  const bool owns_slots = 4 * tid < S;  // this thread's slots 4 * tid .. 4 * tid + 3
  const int b0 = kPlanRun * tid;        // this thread's first row of the first pass
  const bool vec = ((reinterpret_cast<uintptr_t>(row_src) | reinterpret_cast<uintptr_t>(seq_lens)) & 15) == 0;

  // Global reads first, all in flight together: the first pass's rows and
  // the activity of the thread's slots.  The row steps run whole waves (they
  // use cross-lane operations): a wave with any row in a pass takes part,
  // and its lanes past the last row have no rows (pl_plan_mask4).
  const bool wave_rows = wave * 64 * kPlanRun < rows;
  int rs[kPlanRun], rl[kPlanRun];
  if (wave_rows) {
    pl_plan_load4<ADAPTER_ROWS>(row_src, num_adapters, seq_lens, b0, rows, vec, rs, rl);
  } else {
#pragma unroll
    for (int i = 0; i < kPlanRun; ++i) rs[i] = rl[i] = 0;
  }
  if (owns_slots) {
    int av[4] = {1, 1, 1, 1};
    if (active != nullptr) {
#pragma unroll
      for (int j = 0; j < 4; ++j) av[j] = active[(int64_t)min(4 * tid + j, S - 1) * active_stride];
    }
    reinterpret_cast<int4*>(cnt)[tid] = make_int4(0, 0, 0, 0);
    reinterpret_cast<int4*>(fill)[tid] = make_int4(0, 0, 0, 0);
    uint32_t a4 = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int s = 4 * tid + j;
      a4 |= (uint32_t)(s > 0 && s < S && av[j] > 0) << (8 * j);  // slot 0 (base) never has work
    }
    reinterpret_cast<uint32_t*>(act)[tid] = a4;
  }
  __syncthreads();  // act[] is complete, the counters are clear

  int unused[kPlanRun];
  if (wave_rows) {
    pl_plan_mask4(b0, rows, row_len, S, act, rs, rl);
    pl_plan_claim4<false>(rs, rl, lane, cnt, unused);
  }
  for (int c0 = kPlanChunk; c0 < rows; c0 += kPlanChunk) {
    if (c0 + wave * 64 * kPlanRun >= rows) break;  // wave-uniform
    int s[kPlanRun], L[kPlanRun];
    pl_plan_load4<ADAPTER_ROWS>(row_src, num_adapters, seq_lens, c0 + b0, rows, vec, s, L);
    pl_plan_mask4(c0 + b0, rows, row_len, S, act, s, L);
    pl_plan_claim4<false>(s, L, lane, cnt, unused);
  }
  __syncthreads();

  // Exclusive prefix over slots of token counts and of group counts.  With
  // at most 256 slots every count is in wave 0's slots and wave 0 alone
  // scans them; the totals reach the other waves through wsum.
  const bool one_wave = S <= 4 * 64;
  if (!one_wave || wave == 0) {
    const int4 c4 = reinterpret_cast<const int4*>(cnt)[tid];
    const int cq[4] = {c4.x, c4.y, c4.z, c4.w};
    int loc_t[4], loc_g[4];
    int st = 0, sg = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int cc = tid * 4 + q < S ? cq[q] : 0;
      loc_t[q] = st;
      loc_g[q] = sg;
      st += cc;
      sg += (cc + group_tokens - 1) / group_tokens;
    }
    const int it = pl_wave_scan_incl(st);
    const int ig = pl_wave_scan_incl(sg);
    int ex_t = it - st, ex_g = ig - sg;
    if (lane == 63) {
      wsum[0][wave] = it;
      wsum[1][wave] = ig;
    }
    if (!one_wave) {
      __syncthreads();
      for (int w = 0; w < wave; ++w) {
        ex_t += wsum[0][w];
        ex_g += wsum[1][w];
      }
    }
    // entries past the slot count are written too (never read)
    reinterpret_cast<int4*>(off)[tid] =
        make_int4(ex_t + loc_t[0], ex_t + loc_t[1], ex_t + loc_t[2], ex_t + loc_t[3]);
    reinterpret_cast<int4*>(goff)[tid] =
        make_int4(ex_g + loc_g[0], ex_g + loc_g[1], ex_g + loc_g[2], ex_g + loc_g[3]);
  }
  __syncthreads();
  int tt = 0, tg = 0;
  for (int w = 0; w < (one_wave ? 1 : kPlanThreads / 64); ++w) {
    tt += wsum[0][w];
    tg += wsum[1][w];
  }
  if (tid == 0) {
    meta[0] = tg;
    meta[1] = tt;
    meta[2] = group_tokens;
    meta[3] = pl_plan_positions(tg);
  }

  // One thread per group (a slot can have hundreds): the group's slot is
  // the last s with goff[s] <= gi (a slot with no groups shares its goff
  // with the next slot, so the last such s is the one that has groups).
  // Groups go to the highest threads first: the first waves hold the rows
  // (all of them in decode), so emission and scatter run on different waves.
  for (int gi = kPlanThreads - 1 - tid; gi < tg; gi += kPlanThreads) {
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
    // short rows (decode, flattened tokens): a thread's 4 rows at a time
    if (wave_rows) {
      int pos[kPlanRun] = {0, 0, 0, 0};
      pl_plan_claim4<true>(rs, rl, lane, fill, pos);
      pl_plan_store4(rs, rl, pos, b0, row_len, off, tok, cap);
    }
    for (int c0 = kPlanChunk; c0 < rows; c0 += kPlanChunk) {
      if (c0 + wave * 64 * kPlanRun >= rows) break;  // wave-uniform
      int s[kPlanRun], L[kPlanRun], pos[kPlanRun] = {0, 0, 0, 0};
      pl_plan_load4<ADAPTER_ROWS>(row_src, num_adapters, seq_lens, c0 + b0, rows, vec, s, L);
      pl_plan_mask4(c0 + b0, rows, row_len, S, act, s, L);
      pl_plan_claim4<true>(s, L, lane, fill, pos);
      pl_plan_store4(s, L, pos, c0 + b0, row_len, off, tok, cap);
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
