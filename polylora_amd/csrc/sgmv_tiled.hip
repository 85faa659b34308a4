// Adapter-major tiled SGMV kernels for gfx950 (MFMA 16x16, wave64).
//
// Every kernel walks the plan written by pl_plan_build: a list of groups of
// at most G tokens that share one slot, G = 16 (decode and small batches) or
// 64 (large batches of long segments).  A token's result never depends on
// which other tokens share its group, so the plan's order inside a slot is
// free.
//
// Shrink (replaces sgmv.py:63-138).  16-token groups: pl_shrink_short, one
// workgroup per (group, 64- or 32-rank pass, K split, module).  64-token groups:
// pl_shrink_long, one workgroup per (group, K split, module), each A chunk
// feeding the group's four row tiles.  In both, the four waves split the
// split's K range, 16x16 MFMA tiles [tokens x ranks] accumulate in fp32, the
// four wave partials are summed in LDS in a fixed order, and the workgroup
// stores its sum with plain stores into its own fp32 plane
// planes[split][position][rank].
//
// Expand (replaces sgmv.py:178-275): pl_expand_short, one workgroup per
// (group, column chunk of 256 bf16/f16 or 128 f32 output columns, 16-token
// sub-tile).  The planes of the sub-tile's tokens are summed in split order
// and rounded once to the model dtype, staged in LDS, and multiplied with B
// on the transposed tile [columns x tokens], so that B (stored [out][rank8],
// rank contiguous) is read in contiguous 16-byte rank chunks.  Split-K
// therefore needs no atomics, no cross-workgroup signalling and no cleared
// buffers: results are bitwise reproducible and every launch can be recorded
// in a HIP graph.  The scaled, rounded delta goes through LDS to the
// row-major layout of y, and the fused add-back reads and writes y once with
// 16-byte accesses (512 contiguous bytes per row).
//
// Adapter weights (A in the short shrink, B in the expand) are read with
// non-temporal loads: a decode launch reads each adapter's A and B about once, and
// keeping them out of the L2 leaves it to x and the split planes, which many
// workgroups reread (decode sequence of a Llama-3-8B layer, 47 adapters:
// 87.4 -> 83.8 us; non-temporal x or plane loads made it slower).  The long
// shrink keeps A cached: every 64-token group of a slot rereads it.
//
// Latency is what these launches are short of, so every kernel issues a
// wave's loads together before their first use: guards select an address
// (masked lanes read a zero page) instead of branching around a load, and
// scheduling barriers keep the compiler from interleaving the loads with
// the MFMAs that consume them.
#include <mutex>

#include "pl_common.h"

namespace {

constexpr int kWaves = 4;

// Modules one shrink launch serves: wrapped Linears fed the same input x.
constexpr int kMaxJobs = PL_MAX_STACKED_MODULES;

struct pl_shrink_args {
  const void* x;
  int64_t ldx;
  int32_t K;
  int32_t kw;  // K per wave, a multiple of the step span
  const char* arena;
  const pl_slot_entry* table;
  int32_t num_modules;
  int32_t n_jobs;                // modules served, 1..kMaxJobs
  int32_t module[kMaxJobs];      // table column of each served module
  float* planes[kMaxJobs];       // its fp32 planes [k_splits][tmp_rows][ldt]
  const int32_t* tok;
  const pl_group* groups;
  const int32_t* meta;
  int32_t ldt;
  int32_t k_splits;
  int32_t rank_passes;  // rank passes per (group, split) of the short shrink
  int32_t rank_tiles;   // 16-rank tiles per short-shrink pass (2 or 4)
  int32_t sub;          // 16-token sub-tiles per plan group (1 or 4)
  int64_t plane;        // floats between split planes
};

struct pl_expand_args {
  int32_t ldt;
  int32_t k_splits;
  int64_t plane;
  const char* arena;
  const pl_slot_entry* table;
  int32_t num_modules;
  const int32_t* tok;
  const pl_group* groups;
  const int32_t* meta;
  int32_t epilogue;
  int32_t sub;                    // 16-token sub-tiles per plan group (1 or 4)
  int32_t n_jobs;                 // modules written, 1..kMaxJobs
  int32_t n_chunks;               // column chunks of all jobs together
  int32_t chunk0[kMaxJobs];       // first chunk of each job
  int32_t module[kMaxJobs];       // table column of each job's module
  const float* planes[kMaxJobs];  // its shrink planes
  void* y[kMaxJobs];              // its output
  int64_t ldy[kMaxJobs];
  int32_t N[kMaxJobs];
  const void* inter;  // the caller's model-dtype intermediate [tokens][ldi] (pl_expand_inter_launch)
  int64_t ldi;
};

// Columns of y one expand wave owns: 128 bytes of each row (64 for 2-byte
// types, 32 for fp32), so that a workgroup's tile row is 512 bytes; the 256
// threads read and write the tile's y rows 16 bytes at a time, kYLanes
// lanes per row.
constexpr int kExpandWaveBytes = 128;
template <int DT>
struct pl_expand_shape {
  typedef typename pl_traits<DT>::T T;
  enum { kColsWave = kExpandWaveBytes / (int)sizeof(T) };
  enum { kCT = kColsWave / 16 };
  enum { kChunk = kWaves * kColsWave };
  enum { kPad = 16 / (int)sizeof(T) };  // 16 bytes of LDS row padding
  enum { kLdsRow = kChunk + kPad };
  enum { kYLanes = kChunk * (int)sizeof(T) / 16 };  // lanes per y row
  enum { kYRowsPerPass = 256 / kYLanes };          // y rows per pass of the workgroup
};

// ------------------------------------------------------------ short groups
// Groups of at most 16 tokens (decode: a handful of rows per adapter) move
// little data per workgroup, so these kernels are built for latency: all of
// a step's loads are issued before its first MFMA.
//
// Shrink: one workgroup per (group, pass of 64 or 32 ranks, K split, served
// module); passes beyond the slot's rank exit before loading anything.  The
// four waves split the split's K range (256 each for a split of 1024) and
// their partials are summed in LDS in a fixed order, as in pl_shrink_tiled.
// A step is 2 chunks (64 K per lane group) of the four rank tiles, so a wave
// walks its K range in a few short steps with 70 VGPRs (48 for 32-rank
// passes); seven waves per SIMD
// then hide each other's latency better than fewer waves holding their whole
// K range in flight (measured on MI355X, decode shapes: 8 chunks per step,
// 120 VGPRs, 4 waves per SIMD: q_proj 5.9 us, down_proj 14.2 us; 2 chunks:
// 5.5 and 13.5 us).  One 64-rank pass reads the group's x rows once for all
// of a slot's ranks (32-rank passes read them twice for rank 64): decode
// gate/up shrink 8.1 -> 6.8 us, down_proj 11.8 -> 10.5 us; tiles past the
// rank multiply zeros.  A launch that would have fewer than
// kShortWideMinBlocks workgroups at 64 ranks (o_proj in decode: 320) keeps
// 32-rank passes (6.95 against 7.7 us).
//
// Expand: one workgroup per (group, 256-column chunk).  The shrink planes of
// the group's tokens are summed once per workgroup (all planes' loads in
// flight together), rounded to T and staged in LDS as [token][rank]; B and
// the y rows are loaded at the same time.
constexpr int kShortCC = 2;      // 16-byte chunks per lane per shrink step
// Short-shrink passes cover 64 ranks (4 tiles) when the launch still has at
// least kShortWideMinBlocks workgroups, else 32 (more, smaller workgroups).
constexpr int kShortWideMinBlocks = 512;
constexpr int kShortMaxPlanes = 16;
// Ranks staged in LDS per expand pass (RB): 32 when the shrink left at most
// 4 planes and the launch has at least kExpandNarrowMinBlocks workgroups,
// else 64.  Measured on MI355X (decode, Llama-8B shapes, 4 planes): the
// narrower block frees B registers (90 instead of 104 VGPRs), and the q/k/v
// expand (1920 workgroups) went from 7.3 to 6.3 us, gate/up (8960) from 21.7
// to 20.0 us, while o_proj (1280) is faster with one 64-rank pass (5.3
// against 5.5 us); with 8 planes (down_proj) the 64-rank block stays faster
// (5.9 against 6.6 us).
constexpr int kExpandNarrowMinBlocks = 1536;

// One-launch shrink -> expand hand-off of the decode path
// (pl_lora_decode_stacked): the shrink workgroups come first in the grid, and
// an expand workgroup of (group, module) starts on the group's planes once
// every shrink workgroup of that (group, module) has arrived.
//
// Visibility across the XCDs' separate L2s without a device-wide fence (an
// L2 write-back and invalidate): the planes are written with agent-scope
// stores, which write through the writer's L2; each shrink workgroup arrives
// with one agent-scope atomic add on its (group, module) counter, after all
// of its stores are acknowledged; an expand wave reads the counter at agent
// scope (its first load, then polls) and only then loads the planes, with
// ordinary loads.  Those cannot hit a stale line: every plane row is whole
// 128-byte lines (ldt a multiple of 32), so no line holds rows of two
// groups; a group's lines are read only after all of its writers have
// arrived; and each launch starts with the L2s invalidated, as every kernel
// launch does.
//
// Progress: workgroups are dispatched in block order on each XCD, so every
// shrink workgroup has started before any expand workgroup waits, and a
// shrink workgroup waits on nothing: each wait ends.  The wait is also
// bounded by spin_limit polls; a wait that runs out sets the status word
// (counters[0]) to 1 and goes on with whatever planes it finds.  The last
// expand workgroup of a (group, module) puts its counter back to 0, so the
// counters start every launch at zero without a clear (and the launch can be
// recorded in a HIP graph).
//
// Measured on MI355X (decode layer of a Llama-3-8B shape, 256 rows, 47
// adapters): with every counter in one cache line, the polls and arrivals
// queued on one memory channel and the launches took 4x the split pair; a
// workgroup-wide wait (thread 0 polls, then a barrier) put one more round
// trip on every expand workgroup's path; agent-scope plane loads another.
// Each counter (and the status word) has a 256-byte line of its own: the
// polls and arrivals of different (group, module)s then go to different
// memory channels instead of queueing on one line.
constexpr int kCounterStride = 64;  // int32s per counter
struct pl_handoff {
  int32_t* counters;   // status at [0], counter i at [(1 + i) * kCounterStride]
  int32_t n_shrink;    // shrink workgroups at the start of the grid
  int32_t arrivals;    // shrink workgroups per (group, module): planes x rank passes
  int32_t spin_limit;  // polls before a wait gives up
};

__device__ __forceinline__ void pl_store_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// s_waitcnt vmcnt(0) with the other counters left alone (gfx9 encoding:
// expcnt 7, lgkmcnt 15): this thread's stores are acknowledged.
__device__ __forceinline__ void pl_wait_stores() { __builtin_amdgcn_s_waitcnt(0x0F70); }

__device__ __forceinline__ int32_t* pl_counter(const pl_handoff& h, int counter) {
  return h.counters + (int64_t)(1 + counter) * kCounterStride;
}

__device__ __forceinline__ void pl_handoff_arrive(const pl_handoff& h, int counter) {
  __hip_atomic_fetch_add(pl_counter(h, counter), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Each wave on its own: `seen` is the counter as first read; while fewer
// than h.arrivals shrink workgroups have arrived, poll it again (the value is
// the same in every lane, so the loop is uniform).  No barrier: a wave goes
// on to its plane loads as soon as it has seen every arrival.
__device__ __forceinline__ void pl_handoff_wait_wave(const pl_handoff& h, int counter, int seen) {
  int polls = 0;
  while (__builtin_amdgcn_readfirstlane(seen) < h.arrivals) {
    if (++polls > h.spin_limit) {
      if ((threadIdx.x & 63) == 0)
        __hip_atomic_store(h.counters, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
    __builtin_amdgcn_s_sleep(8);
    seen = __hip_atomic_load(pl_counter(h, counter), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Departure, once every thread of the workgroup has read its planes (after a
// barrier that follows the last plane read): thread 0 counts it, and the
// last of the (group, module)'s `consumers` resets the counter.  The add is
// issued by pl_handoff_depart and its result checked by pl_handoff_reset at
// the very end of the workgroup, so its round trip overlaps the epilogue.
__device__ __forceinline__ int pl_handoff_depart(const pl_handoff& h, int counter) {
  int old = -1;
  if (threadIdx.x == 0)
    old = __hip_atomic_fetch_add(pl_counter(h, counter), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return old;
}

__device__ __forceinline__ void pl_handoff_reset(const pl_handoff& h, int counter, int old,
                                                 int consumers) {
  if (threadIdx.x == 0 && old == h.arrivals + consumers - 1)
    __hip_atomic_store(pl_counter(h, counter), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int JT>
constexpr int pl_shrink_short_lds() {
  return kWaves * JT * 64 * (int)sizeof(pl_f32x4);
}

// What a short-shrink workgroup does with its partial sums: store them as
// the split planes (plain), store them for the decode launch's expand and
// arrive on the hand-off counter (handoff), or store them, arrive on the
// (group, rank pass) counter and, as the last of the K splits to arrive, sum
// the planes and write the model-dtype intermediate (finish).
enum { kShrinkPlain = 0, kShrinkHandoff = 1, kShrinkFinish = 2 };

// The finish mode's counters and output: counter (g * rank_passes + rp) at
// [(g * rank_passes + rp) * PL_FINISH_COUNTER_INTS], zero before the launch
// and zero again after it (its last arrival resets it); out [tokens][n_max].
struct pl_shrink_finish {
  int32_t* counters;
  void* out;
  int32_t n_max;
};

template <int DT, int JT, int MODE>
__device__ __forceinline__ void pl_shrink_short_body(const pl_shrink_args& a, int block,
                                                     char* smem, const pl_handoff& h,
                                                     const pl_shrink_finish& fin) {
  typedef typename pl_traits<DT>::T T;
  constexpr int E = pl_traits<DT>::E;
  constexpr int kInstr = 4 * E;
  constexpr int kStep = kShortCC * kInstr;
  constexpr int kShortRanks = 16 * JT;
  pl_f32x4 (*red)[JT][64] = reinterpret_cast<pl_f32x4 (*)[JT][64]>(smem);

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;

  // block -> (group g, K split c, rank pass rp, served module job); blocks
  // that read the same x rows are adjacent
  const int job = block % a.n_jobs;
  int rest = block / a.n_jobs;
  const int rp = rest % a.rank_passes;
  rest /= a.rank_passes;
  const int c = rest % a.k_splits;
  const int g = rest / a.k_splits;
  // the group count and the group record load together (every record below
  // the capacity is readable); the record is used only for g below the count
  const int n_groups = a.meta[3];  // positions in use (the plan spreads groups over them)
  const pl_group grp = a.groups[g];
  const int len = min(grp.len, 16);  // the host pairs 16-token groups with this kernel
  if (g >= n_groups || len <= 0) return;
  const pl_slot_entry e = a.table[(int64_t)grp.slot * a.num_modules + a.module[job]];
  const int rank = min(e.rank, a.ldt);  // the host guarantees rank <= ldt
  const int rb = rp * kShortRanks;
  if (rb >= rank) {
    // a pass past the rank stores nothing; with a hand-off it still arrives
    // (the expand waits for every pass of a slot that has this module)
    if constexpr (MODE == kShrinkHandoff)
      if (tid == 0 && rank > 0) pl_handoff_arrive(h, g * a.n_jobs + job);
    return;
  }
  const int K = a.K;
  const T* __restrict__ x = reinterpret_cast<const T*>(a.x);
  const T* __restrict__ A = reinterpret_cast<const T*>(a.arena + e.a_off);
  float* __restrict__ out = a.planes[job] + (int64_t)c * a.plane;

  // Every load below is unconditional (pl_ld16_or0), so a wave's loads are
  // all in flight before its first MFMA.  The token index loads first; A,
  // which does not need it, issues next, and only then x, whose addresses
  // wait for the index (the load counter retires in order).
  const bool xok = li < len;
  const int xt = a.tok[grp.start + min(li, len - 1)];
  const int k0 = (c * kWaves + wave) * a.kw;
  const int k1 = min(K, k0 + a.kw);

  pl_f32x4 acc[JT];
#pragma unroll
  for (int jt = 0; jt < JT; ++jt) acc[jt] = pl_f32x4{0.f, 0.f, 0.f, 0.f};

  auto step = [&](int kb) {
    // chunk cc of lane (li, lg) covers k = kb + cc*kInstr + lg*E .. +E
    pl_u32x4 xf[kShortCC];
    pl_u32x4 af[JT][kShortCC];
#pragma unroll
    for (int jt = 0; jt < JT; ++jt) {
      // rank tile of A's MFMA blocks (rt rows): the block of columns k
      // starts at t0*K + k*rt and is wb wide
      const int t0 = rb + jt * 16;
      const int rt = min(16, rank - t0);
#pragma unroll
      for (int cc = 0; cc < kShortCC; ++cc) {
        const int k = kb + cc * kInstr;
        const int wb = min(kInstr, K - k);
        af[jt][cc] = pl_ld16_nt_or0(A + (int64_t)t0 * K + (int64_t)k * rt + li * wb + lg * E,
                                 li < rt && k + lg * E < k1);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    const T* xrow = x + (int64_t)xt * a.ldx + lg * E;
#pragma unroll
    for (int cc = 0; cc < kShortCC; ++cc) {
      const int k = kb + cc * kInstr;
      xf[cc] = pl_ld16_or0(xrow + k, xok && k + lg * E < k1);
    }
    // keep the scheduler from interleaving the loads above with the MFMAs
    // below (it would wait on each load in turn)
    __builtin_amdgcn_sched_barrier(0);
    // no rank guard here: a guard would let the compiler sink the second
    // tile's loads behind the first tile's MFMAs; a tile past the rank
    // multiplies zeros
#pragma unroll
    for (int jt = 0; jt < JT; ++jt)
#pragma unroll
      for (int cc = 0; cc < kShortCC; ++cc)
        acc[jt] = pl_mfma_chunk<DT>(xf[cc], af[jt][cc], acc[jt]);
  };
  // The first step is peeled and unguarded (a wave with no K range reads
  // only zeros), so nothing that needs the index can be placed ahead of the
  // first A loads.
  step(k0);
  for (int kb = k0 + kStep; kb < k1; kb += kStep) step(kb);

  // Sum the four wave partials of each tile in a fixed order; acc[jt][v]
  // holds tile element (token 4*lg+v, rank rb + jt*16 + li).
#pragma unroll
  for (int jt = 0; jt < JT; ++jt) red[wave][jt][lane] = acc[jt];
  __syncthreads();
  if (tid < JT * 64) {
    const int jt = tid >> 6;
    const int l = tid & 63;
    const pl_f32x4 s = red[0][jt][l] + red[1][jt][l] + red[2][jt][l] + red[3][jt][l];
    const int j = rb + jt * 16 + (l & 15);
    if (j < rank) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int prow = (l >> 4) * 4 + v;
        if (prow < len) {
          if constexpr (MODE != kShrinkPlain)
            pl_store_agent(out + (int64_t)(grp.start + prow) * a.ldt + j, s[v]);
          else
            out[(int64_t)(grp.start + prow) * a.ldt + j] = s[v];
        }
      }
    }
  }
  if constexpr (MODE == kShrinkHandoff) {
    pl_wait_stores();  // this thread's planes have reached the agent's coherence point
    __syncthreads();   // ... and every other thread's
    if (tid == 0) pl_handoff_arrive(h, g * a.n_jobs + job);
  }
  if constexpr (MODE == kShrinkFinish) {
    pl_wait_stores();  // this thread's planes have reached the agent's coherence point
    __syncthreads();   // ... and every other thread's; red[] is no longer read
    int* last = reinterpret_cast<int*>(smem);
    if (tid == 0) {
      int32_t* ctr = fin.counters + (int64_t)(g * a.rank_passes + rp) * PL_FINISH_COUNTER_INTS;
      const int old = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int is_last = old == a.k_splits - 1;
      if (is_last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *last = is_last;
    }
    __syncthreads();
    if (!*last) return;
    // The last of the tile's K splits: T(sum of the planes in split order)
    // for its rows and this pass's ranks, as a separate pass over the planes
    // would write it.  Ordinary loads see every split's stores: with ldt a
    // multiple of 32 each 128-byte line of a plane holds this pass's ranks of
    // one row only, so its one writer is that plane's workgroup of this
    // (group, rank pass), which stored it through its L2 before arriving;
    // this XCD's L2 can hold the line only from that writer's own stores,
    // since each launch starts with the L2s invalidated and no other
    // workgroup reads it.
    // Every plane's load is issued before the first add (an index past the
    // last plane reads the last one again), so the sum waits one round trip,
    // not one per plane.
    const float* __restrict__ planes = a.planes[job];
    T* __restrict__ o = reinterpret_cast<T*>(fin.out);
    for (int idx = tid; idx < len * kShortRanks; idx += 256) {
      const int i = idx / kShortRanks;
      const int j = rb + (idx - i * kShortRanks);
      if (j >= rank || j >= fin.n_max) continue;
      const int64_t p = grp.start + i;
      const float* src = planes + p * a.ldt + j;
      float v[kShortMaxPlanes];
#pragma unroll
      for (int q = 0; q < kShortMaxPlanes; ++q) v[q] = src[(int64_t)min(q, a.k_splits - 1) * a.plane];
      float acc = 0.f;
#pragma unroll
      for (int q = 0; q < kShortMaxPlanes; ++q)
        if (q < a.k_splits) acc += v[q];
      o[(int64_t)a.tok[p] * fin.n_max + j] = (T)acc;
    }
  }
}

template <int DT, int JT>
__global__ __launch_bounds__(256, 2) void pl_shrink_short(pl_shrink_args a) {
  __shared__ __attribute__((aligned(16))) char smem[pl_shrink_short_lds<JT>()];
  pl_shrink_short_body<DT, JT, kShrinkPlain>(a, blockIdx.x, smem, pl_handoff{}, pl_shrink_finish{});
}

// pl_shrink_short whose last K split of each (group, rank pass) also writes
// the tile's model-dtype intermediate (pl_shrink_finish_launch).
template <int DT, int JT>
__global__ __launch_bounds__(256, 2) void pl_shrink_short_finish(pl_shrink_args a,
                                                                 pl_shrink_finish f) {
  __shared__ __attribute__((aligned(16))) char smem[pl_shrink_short_lds<JT>()];
  pl_shrink_short_body<DT, JT, kShrinkFinish>(a, blockIdx.x, smem, pl_handoff{}, f);
}

// Long-group shrink (64-token groups, e.g. prefill): one workgroup per
// (group, K split, served module).  Each wave takes a quarter of the split's
// K range for all four 16-token row tiles, so every A chunk it loads feeds
// four MFMAs; the four wave partials are summed in LDS in a fixed order.
// The K loop is double-buffered: the loads of step s+1 are in flight while
// step s runs on the MFMA.
constexpr int kLongCC = 2;  // 16-byte chunks per lane per step
constexpr int kLongJT = 2;  // 16-rank tiles per pass
constexpr int kLongRT = 4;  // 16-token row tiles per group

template <int DT>
__global__ __launch_bounds__(256, 2) void pl_shrink_long(pl_shrink_args a) {
  typedef typename pl_traits<DT>::T T;
  constexpr int E = pl_traits<DT>::E;
  constexpr int kInstr = 4 * E;
  constexpr int kStep = kLongCC * kInstr;
  constexpr int kTiles = kLongRT * kLongJT;
  __shared__ pl_f32x4 red[kWaves][kWaves][64];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;

  // block -> (group g, split c, served module job); the modules of one
  // (group, split) are adjacent so their shared x rows are fetched together
  const int job = blockIdx.x % a.n_jobs;
  const int gc = blockIdx.x / a.n_jobs;
  const int g = gc / a.k_splits;
  const int c = gc - g * a.k_splits;
  const int n_groups = a.meta[3];  // positions in use (the plan spreads groups over them)
  const pl_group grp = a.groups[g];
  const int len = min(grp.len, 16 * kLongRT);  // the host pairs 64-token groups with this kernel
  if (g >= n_groups || len <= 0) return;
  const pl_slot_entry e = a.table[(int64_t)grp.slot * a.num_modules + a.module[job]];
  const int rank = min(e.rank, a.ldt);  // the host guarantees rank <= ldt
  if (rank <= 0) return;
  const int nrt = (len + 15) >> 4;
  const int K = a.K;
  const T* __restrict__ x = reinterpret_cast<const T*>(a.x);
  const T* __restrict__ A = reinterpret_cast<const T*>(a.arena + e.a_off);
  float* __restrict__ out = a.planes[job] + (int64_t)c * a.plane;

  bool xok[kLongRT];
  int xt[kLongRT];
#pragma unroll
  for (int rt = 0; rt < kLongRT; ++rt) {
    xok[rt] = rt * 16 + li < len;
    xt[rt] = a.tok[grp.start + min(rt * 16 + li, len - 1)];
  }
  const int k0 = (c * kWaves + wave) * a.kw;
  const int k1 = min(K, k0 + a.kw);

  for (int rb = 0; rb < rank; rb += 16 * kLongJT) {
    pl_f32x4 acc[kLongRT][kLongJT];
#pragma unroll
    for (int rt = 0; rt < kLongRT; ++rt)
#pragma unroll
      for (int jt = 0; jt < kLongJT; ++jt) acc[rt][jt] = pl_f32x4{0.f, 0.f, 0.f, 0.f};

    // chunk cc of lane (li, lg) covers k = kb + cc*kInstr + lg*E .. +E
    auto load = [&](pl_u32x4 (&xf)[kLongRT][kLongCC], pl_u32x4 (&af)[kLongJT][kLongCC], int kb) {
#pragma unroll
      for (int jt = 0; jt < kLongJT; ++jt) {
        const int t0 = rb + jt * 16;
        const int rt = min(16, rank - t0);
#pragma unroll
        for (int cc = 0; cc < kLongCC; ++cc) {
          const int k = kb + cc * kInstr;
          const int wb = min(kInstr, K - k);
          af[jt][cc] = pl_ld16_or0(A + (int64_t)t0 * K + (int64_t)k * rt + li * wb + lg * E,
                                   li < rt && k + lg * E < k1);
        }
      }
#pragma unroll
      for (int rt = 0; rt < kLongRT; ++rt) {
        const T* xrow = x + (int64_t)xt[rt] * a.ldx + lg * E;
#pragma unroll
        for (int cc = 0; cc < kLongCC; ++cc) {
          const int k = kb + cc * kInstr;
          xf[rt][cc] = pl_ld16_or0(xrow + k, xok[rt] && k + lg * E < k1);
        }
      }
    };
    auto mfma = [&](const pl_u32x4 (&xf)[kLongRT][kLongCC], const pl_u32x4 (&af)[kLongJT][kLongCC]) {
#pragma unroll
      for (int rt = 0; rt < kLongRT; ++rt)
#pragma unroll
        for (int jt = 0; jt < kLongJT; ++jt)
#pragma unroll
          for (int cc = 0; cc < kLongCC; ++cc)
            acc[rt][jt] = pl_mfma_chunk<DT>(xf[rt][cc], af[jt][cc], acc[rt][jt]);
    };
    // steps past k1 load only zeros; no guard, so no branch splits the
    // loads of a step from each other
    pl_u32x4 xa[kLongRT][kLongCC], aa[kLongJT][kLongCC];
    pl_u32x4 xb[kLongRT][kLongCC], ab[kLongJT][kLongCC];
    load(xa, aa, k0);
    for (int kb = k0; kb < k1; kb += 2 * kStep) {
      load(xb, ab, kb + kStep);
      __builtin_amdgcn_sched_barrier(0);
      mfma(xa, aa);
      load(xa, aa, kb + 2 * kStep);
      __builtin_amdgcn_sched_barrier(0);
      mfma(xb, ab);
    }

    // Sum the four wave partials of each tile in a fixed order, four tiles
    // (one per finishing wave) at a time.  acc[rt][jt][v] holds tile element
    // (row 4*lg+v, column li); tile index = rt*JT + jt.
#pragma unroll
    for (int t0 = 0; t0 < kTiles; t0 += kWaves) {
      if (t0 / kLongJT < nrt) {
        __syncthreads();
#pragma unroll
        for (int q = 0; q < kWaves; ++q) {
          const int t = t0 + q;
          red[wave][q][lane] = acc[t / kLongJT][t % kLongJT];
        }
        __syncthreads();
        const int t = t0 + wave;  // tile this wave finishes
        const int rt = t / kLongJT;
        const int j = rb + (t % kLongJT) * 16 + li;
        const pl_f32x4 sum = red[0][wave][lane] + red[1][wave][lane] + red[2][wave][lane] +
                             red[3][wave][lane];
        if (j < rank && rt < nrt) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int prow = rt * 16 + lg * 4 + v;
            if (prow < len) out[(int64_t)(grp.start + prow) * a.ldt + j] = sum[v];
          }
        }
      }
    }
  }
}

// INTER: the intermediate is the caller's model-dtype tensor a.inter, row
// (token) stride a.ldi, staged as it is (it already holds T(x·A)), instead
// of the sum of the split planes; otherwise the same work, the same MFMA
// order and the same epilogue.
template <int DT, int PMAX, int RB, bool INTER = false>
__global__ __launch_bounds__(256, 2) void pl_expand_short(pl_expand_args a) {
  typedef typename pl_traits<DT>::T T;
  typedef typename pl_traits<DT>::T4 T4;
  typedef typename pl_traits<DT>::T8 T8;
  typedef pl_expand_shape<DT> S;
  constexpr int E = pl_traits<DT>::E;
  constexpr int kStep = 4 * E;                        // rank slots per MFMA step
  constexpr int kRB = RB;                             // ranks per staged block
  constexpr int kSteps = kRB / kStep;                 // MFMA steps per staged rank block
  constexpr int kTRow = kRB + S::kPad;                // LDS row of the staged intermediate
  constexpr int kYPer = 16 / S::kYRowsPerPass;        // y rows per thread
  __shared__ __attribute__((aligned(16))) T tt[16 * kTRow];
  __shared__ __attribute__((aligned(16))) T delta[16 * S::kLdsRow];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;

  // block -> (group g, column chunk c of module job, 16-token sub-tile rt);
  // the sub-tiles of one chunk, which read the same B rows, are adjacent
  const int rt = blockIdx.x % a.sub;
  const int gc = blockIdx.x / a.sub;
  const int g = gc / a.n_chunks;
  const int cg = gc - g * a.n_chunks;
  int job = 0;
#pragma unroll
  for (int j = 1; j < kMaxJobs; ++j)
    if (j < a.n_jobs && cg >= a.chunk0[j]) job = j;
  const int c = cg - a.chunk0[job];
  // the group count and the group record load together (every record below
  // the capacity is readable); the record is used only for g below the count
  const int n_groups = a.meta[3];  // positions in use (the plan spreads groups over them)
  pl_group grp = a.groups[g];
  grp.start += rt * 16;
  const int len = min(grp.len - rt * 16, 16);
  if (g >= n_groups || len <= 0) return;
  const pl_slot_entry e = a.table[(int64_t)grp.slot * a.num_modules + a.module[job]];
  const int rank = min(e.rank, a.ldt);  // the host guarantees rank <= ldt
  if (rank <= 0) return;
  const int r8 = e.rank8;
  const int N = a.N[job];
  const int n_base = c * S::kChunk;
  const float scale = e.scale;
  const float scale_t = pl_round<DT>(scale);
  const int n0 = n_base + wave * S::kColsWave;
  const T* __restrict__ Bc = reinterpret_cast<const T*>(a.arena + e.b_off);

  // Load order: the y rows' token indices, then B and the planes of the
  // first rank block, then the y rows (their addresses need the indices).
  // The load counter retires in order, so waiting for the indices does not
  // wait for B or the planes.
  const int yq = tid % S::kYLanes;
  const int yr0 = tid / S::kYLanes;
  const int ycol = n_base + yq * E;
  T* __restrict__ y = reinterpret_cast<T*>(a.y[job]);
  int yt[kYPer];
#pragma unroll
  for (int i = 0; i < kYPer; ++i) yt[i] = a.tok[grp.start + min(yr0 + S::kYRowsPerPass * i, len - 1)];

  // planes -> staged intermediate: thread (token sp, ranks rb + sq .. +4);
  // the waves past the 16 tokens' rows stage nothing and load no planes
  constexpr int kStageLanes = kRB / 4;  // threads per token row
  constexpr int kStageThreads = 16 * kStageLanes;
  static_assert(kStageThreads <= 256 && kStageThreads % 64 == 0, "whole waves stage a rank block");
  const bool stager = kStageThreads == 256 || wave * 64 < kStageThreads;  // wave-uniform
  const int sp = tid / kStageLanes;
  const int sq = (tid % kStageLanes) * 4;
  const float* srow = a.planes[job] + (int64_t)(grp.start + (sp < len ? sp : 0)) * a.ldt;
  // INTER: the stager's row is token tok[grp.start + sp] of the intermediate
  int st_tok = 0;
  if constexpr (INTER) st_tok = a.tok[grp.start + min(sp, len - 1)];

  pl_u32x4 bf[kSteps][S::kCT];
  pl_u32x4 pv[PMAX];
  T4 iv;
  // B rows n0 + ct*16 + li and the planes of ranks rb .. rb+63
  auto load_block = [&](int rb) {
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      // B's MFMA blocks: the 16-column tile at nb (nt columns), rank block
      // j0 (wb wide) starts at nb*r8 + j0*nt
      const int j0 = rb + s * kStep;
      const int wb = min(kStep, r8 - j0);
#pragma unroll
      for (int ct = 0; ct < S::kCT; ++ct) {
        const int nb = n0 + ct * 16;
        const int nt = min(16, N - nb);
        bf[s][ct] = pl_ld16_nt_or0(Bc + (int64_t)nb * r8 + (int64_t)j0 * nt + li * wb + lg * E,
                                li < nt && j0 + lg * E < r8);
      }
    }
    // PMAX loads per thread, the plane index clamped to the last plane;
    // only the first k_splits are summed
    if (stager) {
      const int jr = rb + sq;
      if constexpr (INTER) {
        // four elements of the token's row (the row stride need not keep
        // them 8-byte aligned); ranks past the slot's rank read as zeros
        const T* ip = reinterpret_cast<const T*>(a.inter) + (int64_t)st_tok * a.ldi + jr;
#pragma unroll
        for (int i = 0; i < 4; ++i) iv[i] = (sp < len && jr + i < rank) ? ip[i] : (T)0.f;
      } else {
        const bool sok = sp < len && jr < rank;
        const float* sbase = srow + jr;
#pragma unroll
        for (int q = 0; q < PMAX; ++q)
          pv[q] = pl_ld16_or0(sbase + (int64_t)min(q, a.k_splits - 1) * a.plane, sok);
      }
    }
  };

  // delta^T tiles [columns x tokens]: acc[ct][v] = delta(column n0 + ct*16 + 4*lg + v, token li)
  pl_f32x4 acc[S::kCT];
#pragma unroll
  for (int ct = 0; ct < S::kCT; ++ct) acc[ct] = pl_f32x4{0.f, 0.f, 0.f, 0.f};
  // planes summed in split order, masked at the rank, rounded once to T,
  // staged in LDS and multiplied with B
  auto use_block = [&](int rb) {
    if (rb > 0) __syncthreads();  // the previous rank block's MFMA reads are done
    if (stager) {
      const int jr = rb + sq;
      const bool sok = sp < len && jr < rank;
      T4 tv;
      if constexpr (INTER) {
        tv = iv;
      } else {
        pl_f32x4 sum = __builtin_bit_cast(pl_f32x4, pv[0]);
#pragma unroll
        for (int q = 1; q < PMAX; ++q)
          if (q < a.k_splits) sum += __builtin_bit_cast(pl_f32x4, pv[q]);
#pragma unroll
        for (int i = 0; i < 4; ++i) tv[i] = (T)((sok && jr + i < rank) ? sum[i] : 0.f);
      }
      *reinterpret_cast<T4*>(tt + sp * kTRow + sq) = tv;
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      if (rb + s * kStep < r8) {
        const pl_u32x4 tf = *reinterpret_cast<const pl_u32x4*>(tt + li * kTRow + s * kStep + lg * E);
#pragma unroll
        for (int ct = 0; ct < S::kCT; ++ct) acc[ct] = pl_mfma_chunk<DT>(bf[s][ct], tf, acc[ct]);
      }
    }
  };

  load_block(0);
  __builtin_amdgcn_sched_barrier(0);  // B and plane loads issue before the y loads
  pl_u32x4 yv[kYPer];
  T* yptr[kYPer];
#pragma unroll
  for (int i = 0; i < kYPer; ++i) {
    const int r = yr0 + S::kYRowsPerPass * i;
    yptr[i] = (r < len && ycol < N) ? y + (int64_t)yt[i] * a.ldy[job] + ycol : nullptr;
    yv[i] = pl_ld16_or0(yptr[i], yptr[i] != nullptr);
  }
  __builtin_amdgcn_sched_barrier(0);  // every load above is in flight before the first use
  use_block(0);
  for (int rb = kRB; rb < r8; rb += kRB) {
    load_block(rb);
    __builtin_amdgcn_sched_barrier(0);
    use_block(rb);
  }

  // scale and round in the epilogue's order, stage in LDS as [token][column]
  T* drow = delta + li * S::kLdsRow + wave * S::kColsWave;
#pragma unroll
  for (int ct = 0; ct < S::kCT; ++ct) {
    T4 d;
#pragma unroll
    for (int v = 0; v < 4; ++v) d[v] = (T)pl_delta<DT>(acc[ct][v], scale, scale_t, a.epilogue);
    *reinterpret_cast<T4*>(drow + ct * 16 + lg * 4) = d;
  }
  __syncthreads();

  // y = T(y + delta) with full-width stores
#pragma unroll
  for (int i = 0; i < kYPer; ++i) {
    if (yptr[i] != nullptr) {
      const int r = yr0 + S::kYRowsPerPass * i;
      const pl_u32x4 dv = *reinterpret_cast<const pl_u32x4*>(delta + r * S::kLdsRow + yq * E);
      if constexpr (E == 8) {
        T8 yy = __builtin_bit_cast(T8, yv[i]);
        const T8 dd = __builtin_bit_cast(T8, dv);
#pragma unroll
        for (int q = 0; q < 8; ++q) yy[q] = (T)((float)yy[q] + (float)dd[q]);
        *reinterpret_cast<pl_u32x4*>(yptr[i]) = __builtin_bit_cast(pl_u32x4, yy);
      } else {
        pl_f32x4 yy = __builtin_bit_cast(pl_f32x4, yv[i]);
        yy += __builtin_bit_cast(pl_f32x4, dv);
        *reinterpret_cast<pl_f32x4*>(yptr[i]) = yy;
      }
    }
  }
}

template <int DT, int RB>
constexpr int pl_expand_short_lds() {
  typedef pl_expand_shape<DT> S;
  return (16 * (RB + S::kPad) + 16 * S::kLdsRow) * (int)sizeof(typename pl_traits<DT>::T);
}

// pl_expand_short with the hand-off of pl_lora_decode_stacked: the same work
// per workgroup, but the counter is read first, B and the y rows load before
// the wait for it, the planes after it, and the workgroup departs once its
// planes are staged.  (Kept apart from
// pl_expand_short: compiled as a shared function body, the plain kernel took
// 97 instead of 90 VGPRs, one wave per SIMD fewer.)
template <int DT, int PMAX, int RB>
__device__ __forceinline__ void pl_expand_handoff_body(const pl_expand_args& a, int block,
                                                       char* smem, const pl_handoff& h) {
  typedef typename pl_traits<DT>::T T;
  typedef typename pl_traits<DT>::T4 T4;
  typedef typename pl_traits<DT>::T8 T8;
  typedef pl_expand_shape<DT> S;
  constexpr int E = pl_traits<DT>::E;
  constexpr int kStep = 4 * E;                        // rank slots per MFMA step
  constexpr int kRB = RB;                             // ranks per staged block
  constexpr int kSteps = kRB / kStep;                 // MFMA steps per staged rank block
  constexpr int kTRow = kRB + S::kPad;                // LDS row of the staged intermediate
  constexpr int kYPer = 16 / S::kYRowsPerPass;        // y rows per thread
  T* tt = reinterpret_cast<T*>(smem);                 // [16][kTRow]
  T* delta = tt + 16 * kTRow;                         // [16][S::kLdsRow]

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;

  // block -> (group g, column chunk c of module job, 16-token sub-tile rt);
  // the sub-tiles of one chunk, which read the same B rows, are adjacent
  const int rt = block % a.sub;
  const int gc = block / a.sub;
  const int g = gc / a.n_chunks;
  const int cg = gc - g * a.n_chunks;
  int job = 0;
#pragma unroll
  for (int j = 1; j < kMaxJobs; ++j)
    if (j < a.n_jobs && cg >= a.chunk0[j]) job = j;
  const int c = cg - a.chunk0[job];
  // the (group, module) counter's first read is this workgroup's first load:
  // it is back by the time B and the y rows are in flight, so a workgroup
  // that starts after the shrink has finished does not wait a round trip
  const int counter = g * a.n_jobs + job;
  const int seen = __hip_atomic_load(pl_counter(h, counter), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // the group count and the group record load together (every record below
  // the capacity is readable); the record is used only for g below the count
  const int n_groups = a.meta[3];  // positions in use (the plan spreads groups over them)
  pl_group grp = a.groups[g];
  grp.start += rt * 16;
  const int len = min(grp.len - rt * 16, 16);
  if (g >= n_groups || len <= 0) return;
  const pl_slot_entry e = a.table[(int64_t)grp.slot * a.num_modules + a.module[job]];
  const int rank = min(e.rank, a.ldt);  // the host guarantees rank <= ldt
  if (rank <= 0) return;
  const int r8 = e.rank8;
  const int N = a.N[job];
  const int n_base = c * S::kChunk;
  const float scale = e.scale;
  const float scale_t = pl_round<DT>(scale);
  const int n0 = n_base + wave * S::kColsWave;
  const T* __restrict__ Bc = reinterpret_cast<const T*>(a.arena + e.b_off);

  // Load order: the y rows' token indices, then B and the planes of the
  // first rank block, then the y rows (their addresses need the indices).
  // The load counter retires in order, so waiting for the indices does not
  // wait for B or the planes.
  const int yq = tid % S::kYLanes;
  const int yr0 = tid / S::kYLanes;
  const int ycol = n_base + yq * E;
  T* __restrict__ y = reinterpret_cast<T*>(a.y[job]);
  int yt[kYPer];
#pragma unroll
  for (int i = 0; i < kYPer; ++i) yt[i] = a.tok[grp.start + min(yr0 + S::kYRowsPerPass * i, len - 1)];

  // planes -> staged intermediate: thread (token sp, ranks rb + sq .. +4);
  // the waves past the 16 tokens' rows stage nothing and load no planes
  constexpr int kStageLanes = kRB / 4;  // threads per token row
  constexpr int kStageThreads = 16 * kStageLanes;
  static_assert(kStageThreads <= 256 && kStageThreads % 64 == 0, "whole waves stage a rank block");
  const bool stager = kStageThreads == 256 || wave * 64 < kStageThreads;  // wave-uniform
  const int sp = tid / kStageLanes;
  const int sq = (tid % kStageLanes) * 4;
  const float* srow = a.planes[job] + (int64_t)(grp.start + (sp < len ? sp : 0)) * a.ldt;

  pl_u32x4 bf[kSteps][S::kCT];
  pl_u32x4 pv[PMAX];
  // B rows n0 + ct*16 + li and the planes of ranks rb .. rb+RB-1
  auto load_b = [&](int rb) {
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      // B's MFMA blocks: the 16-column tile at nb (nt columns), rank block
      // j0 (wb wide) starts at nb*r8 + j0*nt
      const int j0 = rb + s * kStep;
      const int wb = min(kStep, r8 - j0);
#pragma unroll
      for (int ct = 0; ct < S::kCT; ++ct) {
        const int nb = n0 + ct * 16;
        const int nt = min(16, N - nb);
        bf[s][ct] = pl_ld16_nt_or0(Bc + (int64_t)nb * r8 + (int64_t)j0 * nt + li * wb + lg * E,
                                li < nt && j0 + lg * E < r8);
      }
    }
  };
  // PMAX loads per thread, the plane index clamped to the last plane; only
  // the first k_splits are summed
  auto load_p = [&](int rb) {
    if (stager) {
      const int jr = rb + sq;
      const bool sok = sp < len && jr < rank;
      const float* sbase = srow + jr;
#pragma unroll
      for (int q = 0; q < PMAX; ++q)
        pv[q] = pl_ld16_or0(sbase + (int64_t)min(q, a.k_splits - 1) * a.plane, sok);
    }
  };
  auto load_block = [&](int rb) {
    load_b(rb);
    load_p(rb);
  };

  // delta^T tiles [columns x tokens]: acc[ct][v] = delta(column n0 + ct*16 + 4*lg + v, token li)
  pl_f32x4 acc[S::kCT];
#pragma unroll
  for (int ct = 0; ct < S::kCT; ++ct) acc[ct] = pl_f32x4{0.f, 0.f, 0.f, 0.f};
  // planes summed in split order, masked at the rank, rounded once to T,
  // staged in LDS and multiplied with B
  auto use_block = [&](int rb) {
    if (rb > 0) __syncthreads();  // the previous rank block's MFMA reads are done
    if (stager) {
      const int jr = rb + sq;
      const bool sok = sp < len && jr < rank;
      pl_f32x4 sum = __builtin_bit_cast(pl_f32x4, pv[0]);
#pragma unroll
      for (int q = 1; q < PMAX; ++q)
        if (q < a.k_splits) sum += __builtin_bit_cast(pl_f32x4, pv[q]);
      T4 tv;
#pragma unroll
      for (int i = 0; i < 4; ++i) tv[i] = (T)((sok && jr + i < rank) ? sum[i] : 0.f);
      *reinterpret_cast<T4*>(tt + sp * kTRow + sq) = tv;
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      if (rb + s * kStep < r8) {
        const pl_u32x4 tf = *reinterpret_cast<const pl_u32x4*>(tt + li * kTRow + s * kStep + lg * E);
#pragma unroll
        for (int ct = 0; ct < S::kCT; ++ct) acc[ct] = pl_mfma_chunk<DT>(bf[s][ct], tf, acc[ct]);
      }
    }
  };

  pl_u32x4 yv[kYPer];
  T* yptr[kYPer];
  auto load_y = [&]() {
#pragma unroll
    for (int i = 0; i < kYPer; ++i) {
      const int r = yr0 + S::kYRowsPerPass * i;
      yptr[i] = (r < len && ycol < N) ? y + (int64_t)yt[i] * a.ldy[job] + ycol : nullptr;
      yv[i] = pl_ld16_or0(yptr[i], yptr[i] != nullptr);
    }
  };
  // B and y do not depend on the shrink: they load while the planes are awaited
  load_b(0);
  load_y();
  pl_handoff_wait_wave(h, counter, seen);
  load_p(0);
  __builtin_amdgcn_sched_barrier(0);  // every load above is in flight before the first use
  use_block(0);
  for (int rb = kRB; rb < r8; rb += kRB) {
    load_block(rb);
    __builtin_amdgcn_sched_barrier(0);
    use_block(rb);
  }

  // scale and round in the epilogue's order, stage in LDS as [token][column]
  T* drow = delta + li * S::kLdsRow + wave * S::kColsWave;
#pragma unroll
  for (int ct = 0; ct < S::kCT; ++ct) {
    T4 d;
#pragma unroll
    for (int v = 0; v < 4; ++v) d[v] = (T)pl_delta<DT>(acc[ct][v], scale, scale_t, a.epilogue);
    *reinterpret_cast<T4*>(drow + ct * 16 + lg * 4) = d;
  }
  __syncthreads();
  // y = T(y + delta), all rows in registers first (every y load is then
  // complete, so the departure below is the only access left in flight)
  pl_u32x4 yo[kYPer];
#pragma unroll
  for (int i = 0; i < kYPer; ++i) {
    const int r = yr0 + S::kYRowsPerPass * i;
    const pl_u32x4 dv = *reinterpret_cast<const pl_u32x4*>(delta + min(r, 15) * S::kLdsRow + yq * E);
    if constexpr (E == 8) {
      T8 yy = __builtin_bit_cast(T8, yv[i]);
      const T8 dd = __builtin_bit_cast(T8, dv);
#pragma unroll
      for (int q = 0; q < 8; ++q) yy[q] = (T)((float)yy[q] + (float)dd[q]);
      yo[i] = __builtin_bit_cast(pl_u32x4, yy);
    } else {
      pl_f32x4 yy = __builtin_bit_cast(pl_f32x4, yv[i]);
      yy += __builtin_bit_cast(pl_f32x4, dv);
      yo[i] = __builtin_bit_cast(pl_u32x4, yy);
    }
  }
  // every wave is past its last plane read (the staging of the last rank block)
  const int departed = pl_handoff_depart(h, counter);
#pragma unroll
  for (int i = 0; i < kYPer; ++i)
    if (yptr[i] != nullptr) *reinterpret_cast<pl_u32x4*>(yptr[i]) = yo[i];
  const int chunks = (job + 1 < a.n_jobs ? a.chunk0[job + 1] : a.n_chunks) - a.chunk0[job];
  pl_handoff_reset(h, counter, departed, chunks * a.sub);
}

// Shrink and expand of the decode path in one launch (see pl_handoff): the
// first h.n_shrink workgroups are pl_shrink_short's, the rest
// pl_expand_short's, sharing one LDS buffer.
// The 4-plane, 32-rank-block form (the big decode expands: q/k/v, gate/up)
// is held to 96 VGPRs, five waves per SIMD like the plain expand it replaces
// (90 VGPRs); the others would spill at that size.
template <int PMAX, int RB>
constexpr int pl_decode_min_blocks() {
  return PMAX == 4 && RB == 32 ? 5 : 2;
}

template <int DT, int JT, int PMAX, int RB>
__global__ __launch_bounds__(256, (pl_decode_min_blocks<PMAX, RB>())) void pl_decode_fused(
    pl_shrink_args sa, pl_expand_args ea,
                                                         pl_handoff h) {
  constexpr int kLds = pl_shrink_short_lds<JT>() > pl_expand_short_lds<DT, RB>()
                           ? pl_shrink_short_lds<JT>()
                           : pl_expand_short_lds<DT, RB>();
  __shared__ __attribute__((aligned(16))) char smem[kLds];
  const int b = (int)blockIdx.x;
  if (b < h.n_shrink)
    pl_shrink_short_body<DT, JT, kShrinkHandoff>(sa, b, smem, h, pl_shrink_finish{});
  else
    pl_expand_handoff_body<DT, PMAX, RB>(ea, b - h.n_shrink, smem, h);
}

template <int DT>
int launch_shrink(const pl_shrink_args& a, int64_t group_cap, hipStream_t stream) {
  if (a.sub == 1) {
    const int64_t grid = group_cap * a.k_splits * a.rank_passes * a.n_jobs;
    if (grid <= 0) return PL_OK;
    if (a.rank_tiles == 4)
      hipLaunchKernelGGL((pl_shrink_short<DT, 4>), dim3((unsigned)grid), dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((pl_shrink_short<DT, 2>), dim3((unsigned)grid), dim3(256), 0, stream, a);
  } else {
    const int64_t grid = group_cap * a.k_splits * a.n_jobs;
    if (grid <= 0) return PL_OK;
    hipLaunchKernelGGL((pl_shrink_long<DT>), dim3((unsigned)grid), dim3(256), 0, stream, a);
  }
  return pl_launch_status("pl_sgmv_shrink");
}

template <int DT>
int launch_expand(const pl_expand_args& a, int64_t group_cap, hipStream_t stream) {
  const int64_t grid = group_cap * a.n_chunks * a.sub;
  if (grid <= 0) return PL_OK;
  if (a.k_splits <= 4 && grid >= kExpandNarrowMinBlocks)
    hipLaunchKernelGGL((pl_expand_short<DT, 4, 32>), dim3((unsigned)grid), dim3(256), 0, stream, a);
  else if (a.k_splits <= 4)
    hipLaunchKernelGGL((pl_expand_short<DT, 4, 64>), dim3((unsigned)grid), dim3(256), 0, stream, a);
  else if (a.k_splits <= 8)
    hipLaunchKernelGGL((pl_expand_short<DT, 8, 64>), dim3((unsigned)grid), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((pl_expand_short<DT, kShortMaxPlanes, 64>), dim3((unsigned)grid),
                       dim3(256), 0, stream, a);
  return pl_launch_status("pl_sgmv_expand");
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <int DT, int JT>
int launch_decode_jt(const pl_shrink_args& sa, const pl_expand_args& ea, const pl_handoff& h,
                     int64_t expand_grid, hipStream_t stream) {
  const dim3 grid((unsigned)(h.n_shrink + expand_grid));
  if (ea.k_splits <= 4 && expand_grid >= kExpandNarrowMinBlocks)
    hipLaunchKernelGGL((pl_decode_fused<DT, JT, 4, 32>), grid, dim3(256), 0, stream, sa, ea, h);
  else if (ea.k_splits <= 4)
    hipLaunchKernelGGL((pl_decode_fused<DT, JT, 4, 64>), grid, dim3(256), 0, stream, sa, ea, h);
  else if (ea.k_splits <= 8)
    hipLaunchKernelGGL((pl_decode_fused<DT, JT, 8, 64>), grid, dim3(256), 0, stream, sa, ea, h);
  else
    hipLaunchKernelGGL((pl_decode_fused<DT, JT, kShortMaxPlanes, 64>), grid, dim3(256), 0, stream,
                       sa, ea, h);
  return pl_launch_status("pl_lora_decode_stacked");
}

template <int DT>
int launch_decode(const pl_shrink_args& sa, const pl_expand_args& ea, pl_handoff h,
                  int64_t group_cap, hipStream_t stream) {
  const int64_t expand_grid = group_cap * ea.n_chunks * ea.sub;
  if (h.n_shrink + expand_grid <= 0) return PL_OK;
  if (sa.rank_tiles == 4) return launch_decode_jt<DT, 4>(sa, ea, h, expand_grid, stream);
  return launch_decode_jt<DT, 2>(sa, ea, h, expand_grid, stream);
}


int check_common(int32_t dtype, const void* arena, const pl_slot_entry* table,
                 int32_t num_modules, int32_t module, const int32_t* tok,
                 const pl_group* groups, const int32_t* meta, int64_t group_cap,
                 int32_t group_tokens) {
  if (dtype != PL_F32 && dtype != PL_BF16 && dtype != PL_F16) {
    pl_set_error("unsupported dtype code %d", dtype);
    return PL_ERR_ARG;
  }
  if (!arena || !table || !tok || !groups || !meta) {
    pl_set_error("null arena/table/plan pointer");
    return PL_ERR_ARG;
  }
  if (num_modules <= 0 || module < 0 || module >= num_modules) {
    pl_set_error("module index %d out of range [0, %d)", module, num_modules);
    return PL_ERR_ARG;
  }
  if (group_cap < 0 || group_cap > (int64_t)1 << 24) {
    pl_set_error("group capacity %lld out of range", (long long)group_cap);
    return PL_ERR_LIMIT;
  }
  if (group_tokens != 16 && group_tokens != 64) {
    pl_set_error("group_tokens must be 16 or 64 (got %d)", group_tokens);
    return PL_ERR_ARG;
  }
  if (!aligned16(arena)) {
    pl_set_error("arena base is not 16-byte aligned");
    return PL_ERR_ALIGN;
  }
  return PL_OK;
}

// K per wave for a requested split count: a multiple of the wave step.  The
// short-group expand sums at most kShortMaxPlanes planes, so 16-token groups
// take at most that many splits.
int64_t shrink_kw(int32_t dtype, int32_t K, int32_t k_splits, int32_t group_tokens) {
  const int cc = group_tokens == 16 ? kShortCC : kLongCC;
  k_splits = k_splits < kShortMaxPlanes ? k_splits : kShortMaxPlanes;
  const int64_t step = (int64_t)cc * 4 * pl_chunk_elems(dtype);
  const int64_t per_split = (K + (int64_t)k_splits - 1) / k_splits;
  const int64_t kw = (per_split + kWaves - 1) / kWaves;
  return (kw + step - 1) / step * step;
}

int32_t shrink_planes(int32_t dtype, int32_t K, int32_t k_splits, int32_t group_tokens) {
  const int64_t kw = shrink_kw(dtype, K, k_splits, group_tokens);
  return (int32_t)((K + kWaves * kw - 1) / (kWaves * kw));
}

// Workspace of the shrink -> expand hand-off: fp32 planes [planes][tmp_rows][ldt].
int64_t workspace_bytes(int32_t planes, int64_t tmp_rows, int32_t ldt) {
  return (int64_t)planes * tmp_rows * ldt * 4;
}

int check_ws(const void* ws, int32_t ldt, int64_t tmp_rows) {
  if (!ws) {
    pl_set_error("null workspace pointer");
    return PL_ERR_ARG;
  }
  if (ldt <= 0 || (ldt & 7) != 0 || tmp_rows < 0) {
    pl_set_error("workspace needs ldt a positive multiple of 8 (got %d) and tmp_rows >= 0", ldt);
    return PL_ERR_ARG;
  }
  if (!aligned16(ws)) {
    pl_set_error("workspace is not 16-byte aligned");
    return PL_ERR_ALIGN;
  }
  return PL_OK;
}

int prepare_shrink(pl_shrink_args& a, int32_t dtype, const void* x, int64_t ldx, int32_t K,
                   const void* arena, const pl_slot_entry* table, int32_t num_modules,
                   int32_t n_jobs, const int32_t* modules, void* const* ws, const int32_t* tok,
                   const pl_group* groups, const int32_t* meta, int64_t group_cap,
                   int32_t group_tokens, int64_t ws_bytes, int32_t ldt, int64_t tmp_rows,
                   int32_t k_splits) {
  if (n_jobs < 1 || n_jobs > kMaxJobs || !modules || !ws) {
    pl_set_error("shrink serves 1..%d modules (got %d) with one workspace each", kMaxJobs, n_jobs);
    return PL_ERR_ARG;
  }
  int st = PL_OK;
  for (int j = 0; j < n_jobs; ++j) {
    st = check_common(dtype, arena, table, num_modules, modules[j], tok, groups, meta, group_cap,
                      group_tokens);
    if (st) return st;
    if ((st = check_ws(ws[j], ldt, tmp_rows))) return st;
    for (int i = 0; i < j; ++i)
      if (ws[i] == ws[j]) {
        pl_set_error("each module of a stacked shrink needs its own workspace");
        return PL_ERR_ARG;
      }
  }
  const int E = pl_chunk_elems(dtype);
  const int es = pl_elem_size(dtype);
  if (!x) {
    pl_set_error("null x pointer");
    return PL_ERR_ARG;
  }
  if (K <= 0 || ldx < K || k_splits < 1 || k_splits > 4096) {
    pl_set_error("bad shrink sizes K=%d ldx=%lld k_splits=%d", K, (long long)ldx, k_splits);
    return PL_ERR_ARG;
  }
  if (K % E != 0 || (ldx * es) % 16 != 0 || !aligned16(x)) {
    pl_set_error("shrink needs K %% %d == 0 and 16-byte aligned x rows", E);
    return PL_ERR_ALIGN;
  }
  const int32_t planes = shrink_planes(dtype, K, k_splits, group_tokens);
  const int32_t rank_tiles = group_cap * planes * n_jobs >= kShortWideMinBlocks ? 4 : 2;
  const int32_t rank_passes = (ldt + 16 * rank_tiles - 1) / (16 * rank_tiles);
  const int32_t sub = group_tokens / 16;
  if (!pl_grid_fits(group_cap * planes * rank_passes * sub * n_jobs, 256)) {
    pl_set_error("shrink grid too large");
    return PL_ERR_LIMIT;
  }
  if (ws_bytes < workspace_bytes(planes, tmp_rows, ldt)) {
    pl_set_error("workspace of %lld bytes is below the %lld this call needs", (long long)ws_bytes,
                 (long long)workspace_bytes(planes, tmp_rows, ldt));
    return PL_ERR_ARG;
  }
  a.x = x;
  a.ldx = ldx;
  a.K = K;
  a.kw = (int32_t)shrink_kw(dtype, K, k_splits, group_tokens);
  a.arena = reinterpret_cast<const char*>(arena);
  a.table = table;
  a.num_modules = num_modules;
  a.n_jobs = n_jobs;
  for (int j = 0; j < kMaxJobs; ++j) {
    a.module[j] = j < n_jobs ? modules[j] : 0;
    a.planes[j] = j < n_jobs ? reinterpret_cast<float*>(ws[j]) : nullptr;
  }
  a.tok = tok;
  a.groups = groups;
  a.meta = meta;
  a.ldt = ldt;
  a.k_splits = planes;
  a.rank_passes = rank_passes;
  a.rank_tiles = rank_tiles;
  a.sub = sub;
  a.plane = tmp_rows * ldt;
  return PL_OK;
}

int prepare_expand(pl_expand_args& a, int32_t dtype, void* const* ws, int32_t ldt,
                   int64_t tmp_rows, int32_t planes, const void* arena,
                   const pl_slot_entry* table, int32_t num_modules, int32_t n_jobs,
                   const int32_t* modules, const int32_t* tok, const pl_group* groups,
                   const int32_t* meta, int64_t group_cap, int32_t group_tokens, void* const* y,
                   const int64_t* ldy, const int32_t* N, int32_t epilogue) {
  if (n_jobs < 1 || n_jobs > kMaxJobs || !modules || !ws || !y || !ldy || !N) {
    pl_set_error("expand serves 1..%d modules (got %d), each with its workspace, y, ldy and N",
                 kMaxJobs, n_jobs);
    return PL_ERR_ARG;
  }
  const int E = pl_chunk_elems(dtype);
  const int es = pl_elem_size(dtype);
  const int chunk = dtype == PL_F32 ? (int)pl_expand_shape<PL_F32>::kChunk
                                    : (int)pl_expand_shape<PL_BF16>::kChunk;
  int64_t n_chunks = 0;
  for (int j = 0; j < n_jobs; ++j) {
    int st = check_common(dtype, arena, table, num_modules, modules[j], tok, groups, meta,
                          group_cap, group_tokens);
    if (st) return st;
    if ((st = check_ws(ws[j], ldt, tmp_rows))) return st;
    if (!y[j]) {
      pl_set_error("null y pointer");
      return PL_ERR_ARG;
    }
    if (N[j] <= 0 || ldy[j] < N[j]) {
      pl_set_error("bad expand sizes N=%d ldy=%lld", N[j], (long long)ldy[j]);
      return PL_ERR_ARG;
    }
    if (N[j] % E != 0 || (ldy[j] * es) % 16 != 0 || !aligned16(y[j])) {
      pl_set_error("expand needs N %% %d == 0 and 16-byte aligned y rows", E);
      return PL_ERR_ALIGN;
    }
    a.chunk0[j] = (int32_t)n_chunks;
    n_chunks += (N[j] + chunk - 1) / chunk;
  }
  if (planes < 1 || planes > kShortMaxPlanes) {
    pl_set_error("the expand sums 1..%d shrink planes (got %d)", kShortMaxPlanes, planes);
    return PL_ERR_ARG;
  }
  if (epilogue != PL_EPI_FALLBACK && epilogue != PL_EPI_TRITON) {
    pl_set_error("bad epilogue mode %d", epilogue);
    return PL_ERR_ARG;
  }
  if (!pl_grid_fits(group_cap * n_chunks * (group_tokens / 16), 256)) {
    pl_set_error("expand grid too large");
    return PL_ERR_LIMIT;
  }
  a.ldt = ldt;
  a.k_splits = planes;
  a.plane = tmp_rows * ldt;
  a.inter = nullptr;
  a.ldi = 0;
  a.arena = reinterpret_cast<const char*>(arena);
  a.table = table;
  a.num_modules = num_modules;
  a.tok = tok;
  a.groups = groups;
  a.meta = meta;
  a.epilogue = epilogue;
  a.sub = group_tokens / 16;
  a.n_jobs = n_jobs;
  a.n_chunks = (int32_t)n_chunks;
  for (int j = 0; j < kMaxJobs; ++j) {
    const bool on = j < n_jobs;
    if (!on) a.chunk0[j] = (int32_t)n_chunks;
    a.module[j] = on ? modules[j] : 0;
    a.planes[j] = on ? reinterpret_cast<const float*>(ws[j]) : nullptr;
    a.y[j] = on ? y[j] : nullptr;
    a.ldy[j] = on ? ldy[j] : 0;
    a.N[j] = on ? N[j] : 0;
  }
  return PL_OK;
}

int dispatch_shrink(int32_t dtype, const pl_shrink_args& a, int64_t group_cap, hipStream_t s) {
  switch (dtype) {
    case PL_BF16: return launch_shrink<PL_BF16>(a, group_cap, s);
    case PL_F16: return launch_shrink<PL_F16>(a, group_cap, s);
    default: return launch_shrink<PL_F32>(a, group_cap, s);
  }
}

template <int DT>
void launch_shrink_finish(const pl_shrink_args& a, const pl_shrink_finish& f, int64_t grid,
                          hipStream_t s) {
  if (a.rank_tiles == 4)
    hipLaunchKernelGGL((pl_shrink_short_finish<DT, 4>), dim3((unsigned)grid), dim3(256), 0, s, a, f);
  else
    hipLaunchKernelGGL((pl_shrink_short_finish<DT, 2>), dim3((unsigned)grid), dim3(256), 0, s, a, f);
}

int dispatch_expand(int32_t dtype, const pl_expand_args& a, int64_t group_cap, hipStream_t s) {
  switch (dtype) {
    case PL_BF16: return launch_expand<PL_BF16>(a, group_cap, s);
    case PL_F16: return launch_expand<PL_F16>(a, group_cap, s);
    default: return launch_expand<PL_F32>(a, group_cap, s);
  }
}

}  // namespace

extern "C" int32_t pl_shrink_planes(int32_t dtype, int32_t K, int32_t k_splits,
                                    int32_t group_tokens) {
  if (K <= 0 || k_splits < 1 || (group_tokens != 16 && group_tokens != 64)) return 0;
  return shrink_planes(dtype, K, k_splits, group_tokens);
}

extern "C" int64_t pl_shrink_workspace_bytes(int32_t dtype, int32_t K, int32_t k_splits,
                                             int32_t group_tokens, int64_t tmp_rows,
                                             int32_t ldt) {
  if (K <= 0 || k_splits < 1 || tmp_rows < 0 || ldt <= 0 ||
      (group_tokens != 16 && group_tokens != 64))
    return 0;
  return workspace_bytes(shrink_planes(dtype, K, k_splits, group_tokens), tmp_rows, ldt);
}

extern "C" int pl_sgmv_shrink(int32_t dtype, const void* x, int64_t ldx, int32_t K,
                              const void* arena, const pl_slot_entry* table,
                              int32_t num_modules, int32_t module, const int32_t* tok,
                              const pl_group* groups, const int32_t* meta, int64_t group_cap,
                              int32_t group_tokens, void* ws, int64_t ws_bytes, int32_t ldt,
                              int64_t tmp_rows, int32_t k_splits, void* stream) {
  return pl_sgmv_shrink_stacked(dtype, x, ldx, K, arena, table, num_modules, 1, &module, &ws,
                                tok, groups, meta, group_cap, group_tokens, ws_bytes, ldt,
                                tmp_rows, k_splits, stream);
}

int pl_shrink_finish_launch(int32_t dtype, const void* x, int64_t ldx, int32_t K,
                            const void* arena, const pl_slot_entry* table, const int32_t* tok,
                            const pl_group* groups, const int32_t* meta, int64_t group_cap,
                            int32_t group_tokens, void* ws, int64_t ws_bytes, int32_t ldt,
                            int64_t tmp_rows, int32_t k_splits, int32_t* counters,
                            int64_t counter_ints, void* out, int32_t n_max, void* stream) {
  if (group_tokens != PL_GROUP_TOKENS_SHORT || !counters || !out || n_max < 1 || ldt % 32 != 0)
    return PL_REFOP_DECLINED;
  pl_shrink_args a;
  const int32_t module = 0;
  int st = prepare_shrink(a, dtype, x, ldx, K, arena, table, 1, 1, &module, &ws, tok, groups, meta,
                          group_cap, group_tokens, ws_bytes, ldt, tmp_rows, k_splits);
  if (st) return st;
  if (a.sub != 1 || group_cap * a.rank_passes * PL_FINISH_COUNTER_INTS > counter_ints)
    return PL_REFOP_DECLINED;
  const int64_t grid = group_cap * a.k_splits * a.rank_passes;
  if (grid <= 0) return PL_OK;
  const pl_shrink_finish f{counters, out, n_max};
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (dtype) {
    case PL_BF16: launch_shrink_finish<PL_BF16>(a, f, grid, s); break;
    case PL_F16: launch_shrink_finish<PL_F16>(a, f, grid, s); break;
    default: launch_shrink_finish<PL_F32>(a, f, grid, s); break;
  }
  return pl_launch_status("pl_sgmv_shrink (finish)");
}

int pl_expand_inter_launch(int32_t dtype, const void* inter, int64_t ldi, const void* arena,
                           const pl_slot_entry* table, const int32_t* tok, const pl_group* groups,
                           const int32_t* meta, int64_t group_cap, int32_t group_tokens, void* y,
                           int64_t ldy, int32_t N, int32_t ldt, int32_t epilogue, void* stream) {
  const int E = pl_chunk_elems(dtype);
  const int es = pl_elem_size(dtype);
  if (group_tokens != PL_GROUP_TOKENS_SHORT || !inter || !y || !arena || !table || !tok ||
      !groups || !meta || ldi < 1 || N < 1 || ldy < N || ldt < 1 || group_cap < 1 ||
      group_cap > ((int64_t)1 << 24) || N % E != 0 || (ldy * es) % 16 != 0 || !aligned16(y) ||
      !aligned16(arena) || (epilogue != PL_EPI_FALLBACK && epilogue != PL_EPI_TRITON))
    return PL_REFOP_DECLINED;
  const int chunk = dtype == PL_F32 ? (int)pl_expand_shape<PL_F32>::kChunk
                                    : (int)pl_expand_shape<PL_BF16>::kChunk;
  const int64_t n_chunks = (N + chunk - 1) / chunk;
  const int64_t grid = group_cap * n_chunks;
  if (!pl_grid_fits(grid, 256)) return PL_REFOP_DECLINED;
  pl_expand_args a;
  a.ldt = ldt;
  a.k_splits = 1;
  a.plane = 0;
  a.arena = reinterpret_cast<const char*>(arena);
  a.table = table;
  a.num_modules = 1;
  a.tok = tok;
  a.groups = groups;
  a.meta = meta;
  a.epilogue = epilogue;
  a.sub = 1;
  a.n_jobs = 1;
  a.n_chunks = (int32_t)n_chunks;
  for (int j = 0; j < kMaxJobs; ++j) {
    const bool on = j == 0;
    a.chunk0[j] = on ? 0 : (int32_t)n_chunks;
    a.module[j] = 0;
    a.planes[j] = nullptr;
    a.y[j] = on ? y : nullptr;
    a.ldy[j] = on ? ldy : 0;
    a.N[j] = on ? N : 0;
  }
  a.inter = inter;
  a.ldi = ldi;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 g((unsigned)grid);
  switch (dtype) {
    case PL_BF16: hipLaunchKernelGGL((pl_expand_short<PL_BF16, 1, 64, true>), g, dim3(256), 0, s, a); break;
    case PL_F16: hipLaunchKernelGGL((pl_expand_short<PL_F16, 1, 64, true>), g, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((pl_expand_short<PL_F32, 1, 64, true>), g, dim3(256), 0, s, a); break;
  }
  return pl_launch_status("pl_sgmv_lora_b (short expand)");
}

extern "C" int pl_sgmv_shrink_stacked(int32_t dtype, const void* x, int64_t ldx, int32_t K,
                                      const void* arena, const pl_slot_entry* table,
                                      int32_t num_modules, int32_t n_modules,
                                      const int32_t* modules, void* const* ws,
                                      const int32_t* tok, const pl_group* groups,
                                      const int32_t* meta, int64_t group_cap,
                                      int32_t group_tokens, int64_t ws_bytes, int32_t ldt,
                                      int64_t tmp_rows, int32_t k_splits, void* stream) {
  pl_shrink_args a;
  int st = prepare_shrink(a, dtype, x, ldx, K, arena, table, num_modules, n_modules, modules, ws,
                          tok, groups, meta, group_cap, group_tokens, ws_bytes, ldt, tmp_rows,
                          k_splits);
  if (st) return st;
  return dispatch_shrink(dtype, a, group_cap, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int pl_sgmv_expand(int32_t dtype, const void* ws, int32_t ldt, int64_t tmp_rows,
                              int32_t planes, const void* arena, const pl_slot_entry* table,
                              int32_t num_modules, int32_t module, const int32_t* tok,
                              const pl_group* groups, const int32_t* meta, int64_t group_cap,
                              int32_t group_tokens, void* y, int64_t ldy, int32_t N,
                              int32_t epilogue, void* stream) {
  void* wsp = const_cast<void*>(ws);
  return pl_sgmv_expand_stacked(dtype, &wsp, ldt, tmp_rows, planes, arena, table, num_modules, 1,
                                &module, tok, groups, meta, group_cap, group_tokens, &y, &ldy, &N,
                                epilogue, stream);
}

extern "C" int pl_sgmv_expand_stacked(int32_t dtype, void* const* ws, int32_t ldt,
                                      int64_t tmp_rows, int32_t planes, const void* arena,
                                      const pl_slot_entry* table, int32_t num_modules,
                                      int32_t n_modules, const int32_t* modules,
                                      const int32_t* tok, const pl_group* groups,
                                      const int32_t* meta, int64_t group_cap,
                                      int32_t group_tokens, void* const* y, const int64_t* ldy,
                                      const int32_t* N, int32_t epilogue, void* stream) {
  pl_expand_args a;
  int st = prepare_expand(a, dtype, ws, ldt, tmp_rows, planes, arena, table, num_modules,
                          n_modules, modules, tok, groups, meta, group_cap, group_tokens, y, ldy, N,
                          epilogue);
  if (st) return st;
  return dispatch_expand(dtype, a, group_cap, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int pl_lora_apply(int32_t dtype, const void* x, int64_t ldx, int32_t K, void* y,
                             int64_t ldy, int32_t N, const void* arena,
                             const pl_slot_entry* table, int32_t num_modules, int32_t module,
                             const int32_t* tok, const pl_group* groups, const int32_t* meta,
                             int64_t group_cap, int32_t group_tokens, void* ws, int64_t ws_bytes,
                             int32_t ldt, int64_t tmp_rows, int32_t k_splits, int32_t epilogue,
                             void* stream) {
  pl_shrink_args sa;
  pl_expand_args ea;
  int st = prepare_shrink(sa, dtype, x, ldx, K, arena, table, num_modules, 1, &module, &ws, tok,
                          groups, meta, group_cap, group_tokens, ws_bytes, ldt, tmp_rows, k_splits);
  if (st) return st;
  st = prepare_expand(ea, dtype, &ws, ldt, tmp_rows, sa.k_splits, arena, table, num_modules, 1,
                      &module, tok, groups, meta, group_cap, group_tokens, &y, &ldy, &N, epilogue);
  if (st) return st;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  st = dispatch_shrink(dtype, sa, group_cap, s);
  if (st) return st;
  return dispatch_expand(dtype, ea, group_cap, s);
}

extern "C" int64_t pl_decode_counter_ints(int64_t group_cap, int32_t n_modules) {
  if (group_cap < 0 || n_modules < 1 || n_modules > kMaxJobs) return 0;
  return (1 + group_cap * n_modules) * kCounterStride;
}

extern "C" int pl_lora_decode_stacked(int32_t dtype, const void* x, int64_t ldx, int32_t K,
                                      const void* arena, const pl_slot_entry* table,
                                      int32_t num_modules, int32_t n_modules,
                                      const int32_t* modules, void* const* ws,
                                      const int32_t* tok, const pl_group* groups,
                                      const int32_t* meta, int64_t group_cap,
                                      int32_t group_tokens, int64_t ws_bytes, int32_t ldt,
                                      int64_t tmp_rows, int32_t k_splits, void* const* y,
                                      const int64_t* ldy, const int32_t* N, int32_t epilogue,
                                      int32_t* counters, int64_t counter_ints,
                                      int32_t spin_limit, void* stream) {
  if (group_tokens != 16) {
    pl_set_error("pl_lora_decode_stacked: plans of 16-token groups only (got %d)", group_tokens);
    return PL_ERR_ARG;
  }
  if (ldt % 32 != 0) {
    // every plane row is then whole 128-byte lines, so no line holds rows of
    // two groups and the planes can be read through the L2 (see pl_handoff)
    pl_set_error("pl_lora_decode_stacked: ldt must be a multiple of 32 (got %d)", ldt);
    return PL_ERR_ARG;
  }
  pl_shrink_args sa;
  int st = prepare_shrink(sa, dtype, x, ldx, K, arena, table, num_modules, n_modules, modules, ws,
                          tok, groups, meta, group_cap, group_tokens, ws_bytes, ldt, tmp_rows,
                          k_splits);
  if (st) return st;
  pl_expand_args ea;
  st = prepare_expand(ea, dtype, ws, ldt, tmp_rows, sa.k_splits, arena, table, num_modules,
                      n_modules, modules, tok, groups, meta, group_cap, group_tokens, y, ldy, N,
                      epilogue);
  if (st) return st;
  if (!counters || (reinterpret_cast<uintptr_t>(counters) & 3u) != 0) {
    pl_set_error("pl_lora_decode_stacked: null or misaligned hand-off counters");
    return PL_ERR_ARG;
  }
  if (counter_ints < pl_decode_counter_ints(group_cap, n_modules)) {
    pl_set_error("pl_lora_decode_stacked: %lld hand-off counters, %lld needed", (long long)counter_ints,
                 (long long)pl_decode_counter_ints(group_cap, n_modules));
    return PL_ERR_ARG;
  }
  if (spin_limit < 1) {
    pl_set_error("pl_lora_decode_stacked: spin_limit must be positive");
    return PL_ERR_ARG;
  }
  const int64_t n_shrink = group_cap * sa.k_splits * sa.rank_passes * n_modules;
  const int64_t n_expand = group_cap * ea.n_chunks * ea.sub;
  if (!pl_grid_fits(n_shrink + n_expand, 256) || n_shrink > 0x7fffffff) {
    pl_set_error("pl_lora_decode_stacked: grid too large");
    return PL_ERR_LIMIT;
  }
  pl_handoff h;
  h.counters = counters;
  h.n_shrink = (int32_t)n_shrink;
  h.arrivals = sa.k_splits * sa.rank_passes;
  h.spin_limit = spin_limit;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (dtype) {
    case PL_BF16: return launch_decode<PL_BF16>(sa, ea, h, group_cap, s);
    case PL_F16: return launch_decode<PL_F16>(sa, ea, h, group_cap, s);
    default: return launch_decode<PL_F32>(sa, ea, h, group_cap, s);
  }
}

// ---------------------------------------------------------------------------
// pl_lora_apply_noalloc: pl_plan_build + pl_lora_apply for callers that
// cannot allocate device memory.  The plan (meta, groups, token list) and
// the shrink -> expand planes live in `scratch`, a static device array of
// PL_NOALLOC_SCRATCH_BYTES that every GPU the library runs on holds until the
// process ends.  Host code never passes `scratch` itself to a kernel: on
// the host that name is only a stand-in for the symbol, so each device's
// address is looked up once with hipGetSymbolAddress (with that device
// current) and that pointer is what the kernels receive.  Nothing in the
// array needs clearing: every byte a kernel reads was written earlier in
// the same call (plan records up to the capacity, planes of planned tokens
// and ranks).  All calls on one GPU share its array, so calls that overlap
// on one GPU (different streams, or threads without ordering) race.
static __device__ __align__(256) unsigned char scratch[PL_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kScratchMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchMaxDevices] = {};

int64_t align256(int64_t n) { return (n + 255) / 256 * 256; }

// Device address of `scratch` on the device `stream` belongs to.
int scratch_address(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t err = hipStreamGetDevice(stream, &dev);
  if (err != hipSuccess) {
    pl_set_error("pl_lora_apply_noalloc: hipStreamGetDevice: %s", hipGetErrorString(err));
    return PL_ERR_LAUNCH;
  }
  if (dev < 0 || dev >= kScratchMaxDevices) {
    pl_set_error("pl_lora_apply_noalloc: device %d beyond the %d supported", dev,
                 kScratchMaxDevices);
    return PL_ERR_LIMIT;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int prev = -1;
    if ((err = hipGetDevice(&prev)) != hipSuccess || (err = hipSetDevice(dev)) != hipSuccess) {
      pl_set_error("pl_lora_apply_noalloc: selecting device %d: %s", dev, hipGetErrorString(err));
      return PL_ERR_LAUNCH;
    }
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    const hipError_t back = hipSetDevice(prev);
    if (err != hipSuccess || !p) {
      pl_set_error("pl_lora_apply_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                   hipGetErrorString(err));
      return PL_ERR_LAUNCH;
    }
    if (back != hipSuccess) {
      pl_set_error("pl_lora_apply_noalloc: restoring device %d: %s", prev,
                   hipGetErrorString(back));
      return PL_ERR_LAUNCH;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return PL_OK;
}

// Scratch bytes a call needs: meta (256), the group records, the token list
// and the shrink planes, each part 256-byte aligned; -1 for bad sizes.
int64_t noalloc_bytes(int32_t dtype, int32_t rows, int32_t row_len, int32_t num_slots,
                      int32_t group_tokens, int32_t K, int32_t ldt, int32_t k_splits) {
  if (rows < 0 || row_len < 0 || num_slots < 1 || K <= 0 || ldt <= 0 || k_splits < 1 ||
      (group_tokens != 16 && group_tokens != 64))
    return -1;
  const int64_t tokens = (int64_t)rows * row_len;
  const int64_t tmp_rows = tokens > 0 ? tokens : 1;
  const int64_t cap = pl_plan_group_capacity(rows, row_len, num_slots, group_tokens);
  return 256 + align256((cap > 0 ? cap : 1) * (int64_t)sizeof(pl_group)) +
         align256(tmp_rows * 4) +
         workspace_bytes(shrink_planes(dtype, K, k_splits, group_tokens), tmp_rows, ldt);
}

}  // namespace

extern "C" int pl_lora_apply_noalloc(int32_t dtype, const void* x, int64_t ldx, int32_t K, void* y,
                                     int64_t ldy, int32_t N, const void* arena,
                                     const pl_slot_entry* table, int32_t num_modules,
                                     int32_t module, const int32_t* row_slot,
                                     const int32_t* seq_lens, int32_t rows, int32_t row_len,
                                     int32_t num_slots, int32_t group_tokens, int32_t ldt,
                                     int32_t k_splits, int32_t epilogue, void* stream) {
  const int64_t need = noalloc_bytes(dtype, rows, row_len, num_slots, group_tokens, K, ldt,
                                    k_splits);
  if (need < 0) {
    pl_set_error("pl_lora_apply_noalloc: bad sizes rows=%d row_len=%d num_slots=%d "
                 "group_tokens=%d K=%d ldt=%d k_splits=%d",
                 rows, row_len, num_slots, group_tokens, K, ldt, k_splits);
    return PL_ERR_ARG;
  }
  if (need > (int64_t)PL_NOALLOC_SCRATCH_BYTES) {
    pl_set_error("pl_lora_apply_noalloc: this call needs %lld bytes of scratch; the library's "
                 "static scratch holds %lld (use pl_plan_build + pl_lora_apply with caller "
                 "buffers for larger batches)",
                 (long long)need, (long long)PL_NOALLOC_SCRATCH_BYTES);
    return PL_ERR_LIMIT;
  }
  if (rows > 0 && (!row_slot || !seq_lens)) {
    pl_set_error("pl_lora_apply_noalloc: null row_slot / seq_lens");
    return PL_ERR_ARG;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  void* base = nullptr;
  int st = scratch_address(s, &base);
  if (st) return st;
  const int64_t tokens = (int64_t)rows * row_len;
  const int64_t tmp_rows = tokens > 0 ? tokens : 1;
  int64_t group_cap = pl_plan_group_capacity(rows, row_len, num_slots, group_tokens);
  if (group_cap < 1) group_cap = 1;
  char* p = reinterpret_cast<char*>(base);
  int32_t* meta = reinterpret_cast<int32_t*>(p);
  pl_group* groups = reinterpret_cast<pl_group*>(p + 256);
  int32_t* tok = reinterpret_cast<int32_t*>(p + 256 + align256(group_cap * sizeof(pl_group)));
  void* ws = p + 256 + align256(group_cap * sizeof(pl_group)) + align256(tmp_rows * 4);
  const int64_t ws_bytes = (int64_t)PL_NOALLOC_SCRATCH_BYTES - (reinterpret_cast<char*>(ws) - p);
  // validate every operand before anything is enqueued
  pl_shrink_args sa;
  pl_expand_args ea;
  st = prepare_shrink(sa, dtype, x, ldx, K, arena, table, num_modules, 1, &module, &ws, tok,
                      groups, meta, group_cap, group_tokens, ws_bytes, ldt, tmp_rows, k_splits);
  if (st) return st;
  st = prepare_expand(ea, dtype, &ws, ldt, tmp_rows, sa.k_splits, arena, table, num_modules, 1,
                      &module, tok, groups, meta, group_cap, group_tokens, &y, &ldy, &N, epilogue);
  if (st) return st;
  st = pl_plan_build(row_slot, seq_lens, rows, row_len, num_slots, group_tokens, tok, groups, meta,
                     group_cap, stream);
  if (st) return st;
  st = dispatch_shrink(dtype, sa, group_cap, s);
  if (st) return st;
  return dispatch_expand(dtype, ea, group_cap, s);
}
