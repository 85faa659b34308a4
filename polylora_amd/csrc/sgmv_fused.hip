// Fused shrink + expand for long adapter segments (prefill, large batches of
// few adapters), gfx950.
//
// One workgroup per (16-token tile of a plan group, slice of the output
// columns, served module).  Its four waves split K and accumulate x·Aᵀ for
// the tile in 16x16 MFMA tiles (fp32), the four partials are summed in LDS
// in a fixed order and rounded once to the model dtype (the reference's
// t = T(x @ A[:, :r]), layers.py:127), and then each wave streams its share
// of the slice's columns: B rows and y rows of the next step (128 columns,
// 64 at rank 64 or fp32) are in flight while the MFMA, the epilogue (the
// expand's rounding order) and the 16-byte read-modify-write of y run on
// the current ones.  The first step's loads, which need nothing from the
// shrink, issue before the partials are reduced.  The intermediate never
// leaves the workgroup, so there is one launch per wrapped Linear (or per
// set of sibling Linears fed the same x), no workspace and no split-K
// partial sums; results are bitwise reproducible.
//
// y is streamed with non-temporal loads and stores (each byte is touched once
// per launch), and so is x when only one workgroup reads each x row (one
// module, one column slice); A and B, which every tile of a slot rereads, go
// through the caches normally.
//
// A tile's slices (column ranges) and modules all recompute or share the
// same x rows; they run on one XCD (workgroups are dealt to the 8 XCDs
// round-robin by index), so x and A are fetched from HBM once and reread
// from that XCD's L2.
//
// Ranks up to 64 (4 tiles of 16) are held in registers; the kernel is
// instantiated for at most 1, 2 or 4 rank tiles and each group runs the
// narrowest body that covers its slot's rank.
#include <type_traits>

#include "pl_common.h"

namespace {

constexpr int kFWaves = 4;
constexpr int kFThreads = 64 * kFWaves;
constexpr int kFCC = 4;         // 16-byte chunks per lane per shrink step
constexpr int kFColsMax = 128;  // output columns per wave per expand step (at most)
constexpr int kFStages = 2;     // expand steps in flight per wave
constexpr int kFRankMax = 64;   // largest rank the fused kernel takes

// Columns per wave per expand step: as wide as the registers allow for the
// rank tiles in play (B's rank chunks and y's rows of kFStages steps are
// held at once).
template <int DT, int JT>
constexpr int pl_fused_cols() {
  return (JT >= 4 || (DT == PL_F32 && JT >= 2)) ? 64 : kFColsMax;
}
constexpr int kFSliceMax = 8;   // column slices per tile
constexpr int kFJobs = PL_MAX_STACKED_MODULES;  // sibling modules one launch serves

struct pl_fused_args {
  const void* x;
  int64_t ldx;
  int32_t K;
  int32_t kw;  // K per wave, a multiple of the shrink step
  const char* arena;
  const pl_slot_entry* table;
  int32_t num_modules;
  const int32_t* tok;
  const pl_group* groups;
  const int32_t* meta;
  int32_t group_cap;
  int32_t sub;     // 16-token tiles per plan group (1 or 4)
  int32_t slices;  // column slices per tile
  int32_t epilogue;
  int32_t n_jobs;  // modules served, 1..kFJobs, all fed the same x
  int32_t module[kFJobs];  // table column of each served module
  void* y[kFJobs];
  int64_t ldy[kFJobs];
  int32_t N[kFJobs];
  int32_t nw[kFJobs];  // columns per wave, a multiple of kFColsMax
};

template <int DT>
struct pl_fused_lds {
  typedef typename pl_traits<DT>::T T;
  enum { kPad = DT == PL_F32 ? 4 : 8 };  // 16 bytes of row padding
  enum { kTRow = kFRankMax + kPad };     // staged intermediate [token][rank]
  enum { kDRow = kFColsMax + kPad };     // per-wave delta tile [token][column]
  enum { kXRow = 256 / (int)sizeof(T) + kPad };  // per-wave x tile [token][one step's K]
};

constexpr int kFXLoads = 4;  // x loads per lane per shrink step (4 rows of 256 bytes each)

template <int DT, int JT, bool XNT, int MODE = PL_FUSED_FULL>
__device__ __forceinline__ void pl_fused_body(const pl_fused_args& a, const pl_group& grp, int len,
                                              const int (&xtok)[kFXLoads],
                                              const pl_slot_entry& e, int rank, int job, int slice,
                                              pl_f32x4 (*red)[4][64],
                                              typename pl_traits<DT>::T* tt,
                                              typename pl_traits<DT>::T* dbuf,
                                              typename pl_traits<DT>::T* xtile) {
  typedef typename pl_traits<DT>::T T;
  typedef typename pl_traits<DT>::T4 T4;
  typedef typename pl_traits<DT>::T8 T8;
  typedef pl_fused_lds<DT> L;
  constexpr int E = pl_traits<DT>::E;
  constexpr int kInstr = 4 * E;              // K covered by one wave load
  constexpr int kStep = kFCC * kInstr;       // K covered by one shrink step
  constexpr int kXLoads = kFXLoads;
  static_assert(kStep * (int)sizeof(T) == 256, "one shrink step spans 256 bytes of each x row");
  constexpr int kRStep = 4 * E;              // ranks per expand MFMA step
  constexpr int kRSteps = (16 * JT + kRStep - 1) / kRStep;
  constexpr int kCols = pl_fused_cols<DT, JT>();
  constexpr int kCT = kCols / 16;            // 16-column MFMA tiles per expand step
  constexpr int kYLanes = kCols * (int)sizeof(T) / 16;  // lanes per y row of a step
  constexpr int kYRows = 64 / kYLanes;       // y rows one wave load covers
  constexpr int kYLoads = 16 / kYRows;       // loads per lane for the 16 rows

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int K = a.K;
  const int N = a.N[job];

  // ---- shrink: t[token][j] = sum_k x[token][k] * A[j][k] over this wave's K quarter
  const T* __restrict__ x = reinterpret_cast<const T*>(a.x);
  const T* __restrict__ A = reinterpret_cast<const T*>(a.arena + e.a_off);
  // x is loaded in whole 128-byte lines: load i of a step brings rows
  // 4i .. 4i+3, lane l taking row 4i + l/16 (token xtok[i]) and 16-byte
  // piece l%16 of the step's 256 bytes; the wave's LDS tile then hands each
  // lane its MFMA operand chunks (row li, pieces cc*4 + lg)
  const int xr = lane >> 4;
  const int xp = lane & 15;
  const T* xrow[kXLoads];
  bool xok[kXLoads];
#pragma unroll
  for (int i = 0; i < kXLoads; ++i) {
    xok[i] = xr + 4 * i < len;
    xrow[i] = x + (int64_t)xtok[i] * a.ldx + xp * E;
  }
  T* __restrict__ xw = xtile + wave * 16 * L::kXRow;
  // y rows of the expand, addressed now so that their token indices are not
  // a round trip between the two phases
  T* __restrict__ y = reinterpret_cast<T*>(a.y[job]);
  const int64_t ldy = a.ldy[job];
  const int yq = lane % kYLanes;
  const int yr0 = lane / kYLanes;
  T* yrow[kYLoads];
  bool yok[kYLoads];
#pragma unroll
  for (int i = 0; i < kYLoads; ++i) {
    const int r = yr0 + kYRows * i;
    yok[i] = r < len;
    // the y rows are the x rows when a step's y row spans 16 lanes
    int t;
    if constexpr (kYRows == 4 && kYLoads == kFXLoads)
      t = xtok[i];
    else
      t = a.tok[grp.start + min(r, len - 1)];
    yrow[i] = y + (int64_t)t * ldy + yq * E;
  }
  const int k0 = wave * a.kw;
  const int k1 = min(K, k0 + a.kw);

  pl_f32x4 acc[JT];
#pragma unroll
  for (int jt = 0; jt < JT; ++jt) acc[jt] = pl_f32x4{0.f, 0.f, 0.f, 0.f};
  auto load_k = [&](pl_u32x4 (&xf)[kXLoads], pl_u32x4 (&af)[JT][kFCC], int kb) {
#pragma unroll
    for (int jt = 0; jt < JT; ++jt) {
      // rank tile of A's MFMA blocks (rt rows): the block of columns k
      // starts at t0*K + k*rt and is wb wide
      const int t0 = jt * 16;
      const int rt = min(16, rank - t0);
#pragma unroll
      for (int cc = 0; cc < kFCC; ++cc) {
        const int k = kb + cc * kInstr;
        const int wb = min(kInstr, K - k);
        af[jt][cc] = pl_ld16_or0(A + (int64_t)t0 * K + (int64_t)k * rt + li * wb + lg * E,
                                 li < rt && k + lg * E < k1);
      }
    }
#pragma unroll
    for (int i = 0; i < kXLoads; ++i) {
      // streamed when no other workgroup of the launch reads these x rows
      if constexpr (XNT)
        xf[i] = pl_ld16_nt_or0(xrow[i] + kb, xok[i] && kb + xp * E < k1);
      else
        xf[i] = pl_ld16_or0(xrow[i] + kb, xok[i] && kb + xp * E < k1);
    }
  };
  auto mfma_k = [&](const pl_u32x4 (&xf)[kXLoads], const pl_u32x4 (&af)[JT][kFCC]) {
    // through the wave's LDS tile into the MFMA layout (one wave writes and
    // reads it, and LDS accesses of a wave complete in order)
#pragma unroll
    for (int i = 0; i < kXLoads; ++i)
      *reinterpret_cast<pl_u32x4*>(xw + (xr + 4 * i) * L::kXRow + xp * E) = xf[i];
    pl_u32x4 xm[kFCC];
#pragma unroll
    for (int cc = 0; cc < kFCC; ++cc)
      xm[cc] = *reinterpret_cast<const pl_u32x4*>(xw + li * L::kXRow + cc * kInstr + lg * E);
#pragma unroll
    for (int jt = 0; jt < JT; ++jt)
#pragma unroll
      for (int cc = 0; cc < kFCC; ++cc) acc[jt] = pl_mfma_chunk<DT>(xm[cc], af[jt][cc], acc[jt]);
  };
  if constexpr (MODE == PL_FUSED_EXPAND) {
    // the intermediate comes from the caller: x[token][0 .. rank), model
    // dtype, row stride ldx; zeros past the rank and past the tile's tokens.
    // Thread (row 4*wave + lg, ranks 4*li .. +3): the row's token index is
    // xtok[wave] (row lg + 4*wave), already loaded, so the four element
    // loads go out together
    static_assert(kFThreads == 16 * 16 && kFRankMax == 4 * 16, "one thread per row and 4 ranks");
    const int r = 4 * wave + lg;
    const int j0 = 4 * li;
    int t = xtok[0];
#pragma unroll
    for (int i = 1; i < kFXLoads; ++i)
      if (wave == i) t = xtok[i];
    const T* xr = x + (int64_t)t * a.ldx;
    T4 v;
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = (r < len && j0 + q < rank) ? xr[j0 + q] : (T)0.f;
    *reinterpret_cast<T4*>(tt + r * L::kTRow + j0) = v;
  } else {
    // double-buffered K loop over pairs of steps; the last pair is peeled
    // so that no loads past k1 are left in flight when the shrink ends (its
    // second step may lie past k1 and then loads only zeros)
    pl_u32x4 xa[kXLoads], aa[JT][kFCC], xb[kXLoads], ab[JT][kFCC];
    load_k(xa, aa, k0);
    // the staged intermediate's ranks past the reduced tiles must read as
    // zeros (the reduction below writes ranks 0 .. 16*JT-1)
    for (int i = tid; i < 16 * L::kTRow; i += kFThreads) tt[i] = (T)0.f;
    int kb = k0;
    for (; kb + 2 * kStep < k1; kb += 2 * kStep) {
      load_k(xb, ab, kb + kStep);
      __builtin_amdgcn_sched_barrier(0);
      mfma_k(xa, aa);
      load_k(xa, aa, kb + 2 * kStep);
      __builtin_amdgcn_sched_barrier(0);
      mfma_k(xb, ab);
    }
    if (kb < k1) {
      load_k(xb, ab, kb + kStep);
      __builtin_amdgcn_sched_barrier(0);
      mfma_k(xa, aa);
      __builtin_amdgcn_sched_barrier(0);
      mfma_k(xb, ab);
    }
  }

  // ---- expand set-up; its first steps' loads need nothing from the shrink
  // and are issued before the partials are reduced
  const int c0 = (slice * kFWaves + wave) * a.nw[job];
  const int c1 = min(N, c0 + a.nw[job]);
  const int r8 = e.rank8;
  const T* __restrict__ Bc = reinterpret_cast<const T*>(a.arena + e.b_off);
  T* __restrict__ dw = dbuf + wave * 16 * L::kDRow;
  auto load_n = [&](pl_u32x4 (&bf)[kRSteps][kCT], pl_u32x4 (&yv)[kYLoads], int cb) {
#pragma unroll
    for (int s = 0; s < kRSteps; ++s) {
      // B's MFMA blocks: the 16-column tile at nb (nt columns), rank block
      // j0 (wb wide) starts at nb*r8 + j0*nt
      const int j0 = s * kRStep;
      const int wb = min(kRStep, r8 - j0);
#pragma unroll
      for (int ct = 0; ct < kCT; ++ct) {
        const int nb = cb + ct * 16;
        const int nt = min(16, N - nb);
        bf[s][ct] = pl_ld16_or0(Bc + (int64_t)nb * r8 + (int64_t)j0 * nt + li * wb + lg * E,
                                nb + li < c1 && j0 + lg * E < r8);
      }
    }
#pragma unroll
    for (int i = 0; i < kYLoads; ++i)
      yv[i] = pl_ld16_nt_or0(yrow[i] + cb, yok[i] && cb + yq * E < c1);
  };
  // a ring of kFStages steps: the loads of the next kFStages-1 steps are in
  // flight while one is applied; steps past c1 load only zeros
  pl_u32x4 bring[kFStages][kRSteps][kCT], yring[kFStages][kYLoads];
  if constexpr (MODE != PL_FUSED_SHRINK) {
#pragma unroll
    for (int st = 0; st < kFStages - 1; ++st) load_n(bring[st], yring[st], c0 + st * kCols);
  }

  if constexpr (MODE == PL_FUSED_EXPAND) {
    __syncthreads();  // the staged intermediate is complete
  } else {
    // the four wave partials summed in a fixed order, rounded once to T;
    // acc[jt][v] holds (token 4*lg+v, rank jt*16+li)
#pragma unroll
    for (int jt = 0; jt < JT; ++jt) red[wave][jt][lane] = acc[jt];
    __syncthreads();
    if (tid < JT * 64) {
      const int jt = tid >> 6;
      const int l = tid & 63;
      pl_f32x4 s = red[0][jt][l];
#pragma unroll
      for (int w = 1; w < kFWaves; ++w) s += red[w][jt][l];
      const int j = jt * 16 + (l & 15);
#pragma unroll
      for (int v = 0; v < 4; ++v) tt[((l >> 4) * 4 + v) * L::kTRow + j] = (T)(j < rank ? s[v] : 0.f);
    }
    __syncthreads();
  }
  if constexpr (MODE == PL_FUSED_SHRINK) {
    // the rounded intermediate to y[token][0 .. rank); nothing else is
    // written.  Thread (row 4*wave + lg, ranks 4*li .. +3), the row's token
    // index from the prologue's registers (xtok[wave] holds row lg + 4*wave)
    const int r = 4 * wave + lg;
    const int j0 = 4 * li;
    if (r < len) {
      int t = xtok[0];
#pragma unroll
      for (int i = 1; i < kFXLoads; ++i)
        if (wave == i) t = xtok[i];
      const T4 v = *reinterpret_cast<const T4*>(tt + r * L::kTRow + j0);
      T* yr = y + (int64_t)t * ldy;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (j0 + q < rank) yr[j0 + q] = v[q];
    }
    return;
  }

  // ---- expand over this wave's columns
  const float scale = e.scale;
  const float scale_t = pl_round<DT>(scale);

  pl_u32x4 tf[kRSteps];  // MFMA operand: (token li, ranks s*kRStep + lg*E ..)
#pragma unroll
  for (int s = 0; s < kRSteps; ++s)
    tf[s] = *reinterpret_cast<const pl_u32x4*>(tt + li * L::kTRow + s * kRStep + lg * E);

  auto apply_n = [&](const pl_u32x4 (&bf)[kRSteps][kCT], const pl_u32x4 (&yv)[kYLoads], int cb) {
    pl_f32x4 d[kCT];
#pragma unroll
    for (int ct = 0; ct < kCT; ++ct) d[ct] = pl_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < kRSteps; ++s)
#pragma unroll
      for (int ct = 0; ct < kCT; ++ct) d[ct] = pl_mfma_chunk<DT>(bf[s][ct], tf[s], d[ct]);
    // d[ct][v] = delta(column cb + ct*16 + 4*lg + v, token li): scale and round,
    // then through this wave's LDS tile to the row-major layout of y
#pragma unroll
    for (int ct = 0; ct < kCT; ++ct) {
      T4 dd;
#pragma unroll
      for (int v = 0; v < 4; ++v) dd[v] = (T)pl_delta<DT>(d[ct][v], scale, scale_t, a.epilogue);
      *reinterpret_cast<T4*>(dw + li * L::kDRow + ct * 16 + lg * 4) = dd;
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
    for (int i = 0; i < kYLoads; ++i) {
      const int r = yr0 + kYRows * i;
      const pl_u32x4 dv = *reinterpret_cast<const pl_u32x4*>(dw + r * L::kDRow + yq * E);
      if (yok[i] && cb + yq * E < c1) {
        if constexpr (E == 8) {
          T8 yy = __builtin_bit_cast(T8, yv[i]);
          const T8 dd = __builtin_bit_cast(T8, dv);
#pragma unroll
          for (int q = 0; q < 8; ++q) yy[q] = (T)((float)yy[q] + (float)dd[q]);
          pl_st16_nt(yrow[i] + cb, __builtin_bit_cast(pl_u32x4, yy));
        } else {
          pl_f32x4 yy = __builtin_bit_cast(pl_f32x4, yv[i]);
          yy += __builtin_bit_cast(pl_f32x4, dv);
          pl_st16_nt(yrow[i] + cb, __builtin_bit_cast(pl_u32x4, yy));
        }
      }
    }
    // the next step rewrites the tile only after these reads (in-order LDS)
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  };
  for (int cb = c0; cb < c1; cb += kFStages * kCols) {
#pragma unroll
    for (int st = 0; st < kFStages; ++st) {
      constexpr int kAhead = kFStages - 1;
      const int nx = (st + kAhead) % kFStages;
      load_n(bring[nx], yring[nx], cb + (st + kAhead) * kCols);
      __builtin_amdgcn_sched_barrier(0);
      apply_n(bring[st], yring[st], cb + st * kCols);
    }
  }
}

template <int DT, int JTMAX, bool XNT, int MODE = PL_FUSED_FULL>
__global__ __launch_bounds__(kFThreads, 2) void pl_lora_fused_tile(pl_fused_args a) {
  typedef typename pl_traits<DT>::T T;
  typedef pl_fused_lds<DT> L;
  __shared__ pl_f32x4 red[kFWaves][4][64];
  __shared__ __attribute__((aligned(16))) T tt[16 * L::kTRow];
  __shared__ __attribute__((aligned(16))) T dbuf[kFWaves * 16 * L::kDRow];
  __shared__ __attribute__((aligned(16))) T xtile[kFWaves * 16 * L::kXRow];

  // block -> (group g, 16-token tile rt, column slice, served module job); a
  // group's work items go to one XCD, the modules of one tile and slice are
  // adjacent (they read the same x rows, which the later ones find in that
  // XCD's L2), and the groups are dealt to the XCDs in turn
  const pl_xcd_slot ws = pl_xcd_map(a.n_jobs * a.sub * a.slices);
  const int g = ws.g;
  if (g >= a.group_cap) return;
  const int job = ws.j % a.n_jobs;
  const int ts = ws.j / a.n_jobs;
  const int rt = ts / a.slices;
  const int slice = ts - rt * a.slices;
  const int n_groups = a.meta[3];  // positions in use (the plan spreads groups over them)
  pl_group grp = a.groups[g];
  grp.start += rt * 16;
  const int len = min(grp.len - rt * 16, 16);
  if (g >= n_groups || len <= 0) return;
  // token indices of this lane's x rows (rows lane/16 + 4i), fetched in the
  // same round trip as the slot entry: the asm statement takes them before
  // the rank test, so the compiler cannot sink their loads behind it
  int xtok[kFXLoads];
#pragma unroll
  for (int i = 0; i < kFXLoads; ++i)
    xtok[i] = a.tok[grp.start + min((int)(threadIdx.x & 63) / 16 + 4 * i, len - 1)];
  const pl_slot_entry e = a.table[(int64_t)grp.slot * a.num_modules + a.module[job]];
  asm volatile("" ::"v"(xtok[0]), "v"(xtok[1]), "v"(xtok[2]), "v"(xtok[3]));
  const int rank = min(e.rank, kFRankMax);  // the host guarantees rank <= kFRankMax
  if (rank <= 0) return;

  const int jt = (rank + 15) >> 4;
  if (JTMAX == 1 || jt == 1)
    pl_fused_body<DT, 1, XNT, MODE>(a, grp, len, xtok, e, rank, job, slice, red, tt, dbuf, xtile);
  else if (JTMAX == 2 || jt == 2)
    pl_fused_body<DT, 2 < JTMAX ? 2 : JTMAX, XNT, MODE>(a, grp, len, xtok, e, rank, job, slice, red,
                                                        tt, dbuf, xtile);
  else
    pl_fused_body<DT, JTMAX, XNT, MODE>(a, grp, len, xtok, e, rank, job, slice, red, tt, dbuf,
                                        xtile);
}

template <int DT, bool XNT>
void launch_fused_x(const pl_fused_args& a, int jtmax, dim3 grid, hipStream_t stream) {
  if (jtmax <= 1)
    hipLaunchKernelGGL((pl_lora_fused_tile<DT, 1, XNT>), grid, dim3(kFThreads), 0, stream, a);
  else if (jtmax == 2)
    hipLaunchKernelGGL((pl_lora_fused_tile<DT, 2, XNT>), grid, dim3(kFThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((pl_lora_fused_tile<DT, 4, XNT>), grid, dim3(kFThreads), 0, stream, a);
}

template <int DT>
int launch_fused(const pl_fused_args& a, int jtmax, hipStream_t stream) {
  const dim3 grid((unsigned)pl_xcd_grid(a.group_cap, (int64_t)a.n_jobs * a.sub * a.slices));
  // x is streamed (non-temporal) only when each tile's x rows have one reader:
  // sibling modules and column slices of a tile reread them from L2.  Prefill
  // (q/k/v and gate/up stacked) lost 2 ms per forward with x streamed.
  if (a.n_jobs == 1 && a.slices == 1)
    launch_fused_x<DT, true>(a, jtmax, grid, stream);
  else
    launch_fused_x<DT, false>(a, jtmax, grid, stream);
  return pl_launch_status("pl_lora_fused");
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" int pl_lora_fused_stacked(int32_t dtype, const void* x, int64_t ldx, int32_t K,
                                     int32_t n_modules, const int32_t* modules, void* const* y,
                                     const int64_t* ldy, const int32_t* N, const void* arena,
                                     const pl_slot_entry* table, int32_t num_modules, int32_t ldt,
                                     const int32_t* tok, const pl_group* groups,
                                     const int32_t* meta, int64_t group_cap, int32_t group_tokens,
                                     int32_t slices, int32_t epilogue, void* stream) {
  if (dtype != PL_F32 && dtype != PL_BF16 && dtype != PL_F16) {
    pl_set_error("unsupported dtype code %d", dtype);
    return PL_ERR_ARG;
  }
  if (!x || !arena || !table || !tok || !groups || !meta || !modules || !y || !ldy || !N) {
    pl_set_error("pl_lora_fused: null pointer");
    return PL_ERR_ARG;
  }
  if (n_modules < 1 || n_modules > kFJobs) {
    pl_set_error("pl_lora_fused serves 1..%d modules (got %d)", kFJobs, n_modules);
    return PL_ERR_ARG;
  }
  if (group_tokens != PL_GROUP_TOKENS_SHORT && group_tokens != PL_GROUP_TOKENS_LONG) {
    pl_set_error("group_tokens must be 16 or 64 (got %d)", group_tokens);
    return PL_ERR_ARG;
  }
  if (ldt <= 0 || ldt > kFRankMax) {
    pl_set_error("pl_lora_fused takes ranks up to %d (slot rank capacity %d)", kFRankMax, ldt);
    return PL_ERR_LIMIT;
  }
  if (slices < 1 || slices > kFSliceMax) {
    pl_set_error("pl_lora_fused: slices must be in [1, %d] (got %d)", kFSliceMax, slices);
    return PL_ERR_ARG;
  }
  if (epilogue != PL_EPI_FALLBACK && epilogue != PL_EPI_TRITON) {
    pl_set_error("bad epilogue mode %d", epilogue);
    return PL_ERR_ARG;
  }
  const int E = dtype == PL_F32 ? 4 : 8;
  const int es = dtype == PL_F32 ? 4 : 2;
  if (K <= 0 || ldx < K || K % E != 0 || (ldx * es) % 16 != 0 || !aligned16(x) ||
      !aligned16(arena)) {
    pl_set_error("pl_lora_fused needs K > 0, a multiple of %d, and 16-byte aligned x rows "
                 "(K=%d ldx=%lld)", E, K, (long long)ldx);
    return PL_ERR_ALIGN;
  }
  if (group_cap < 0 || group_cap > (int64_t)1 << 24) {
    pl_set_error("group capacity %lld out of range", (long long)group_cap);
    return PL_ERR_LIMIT;
  }
  pl_fused_args a;
  for (int j = 0; j < n_modules; ++j) {
    if (num_modules <= 0 || modules[j] < 0 || modules[j] >= num_modules) {
      pl_set_error("module index %d out of range [0, %d)", modules[j], num_modules);
      return PL_ERR_ARG;
    }
    if (!y[j] || N[j] <= 0 || ldy[j] < N[j]) {
      pl_set_error("bad fused output %d: N=%d ldy=%lld", j, N[j], (long long)ldy[j]);
      return PL_ERR_ARG;
    }
    if (N[j] % E != 0 || (ldy[j] * es) % 16 != 0 || !aligned16(y[j])) {
      pl_set_error("pl_lora_fused needs N a multiple of %d and 16-byte aligned y rows", E);
      return PL_ERR_ALIGN;
    }
    a.module[j] = modules[j];
    a.y[j] = y[j];
    a.ldy[j] = ldy[j];
    a.N[j] = N[j];
    const int64_t per_wave =
        ((int64_t)N[j] + (int64_t)slices * kFWaves - 1) / ((int64_t)slices * kFWaves);
    a.nw[j] = (int32_t)((per_wave + kFColsMax - 1) / kFColsMax * kFColsMax);
  }
  if (!pl_grid_fits(pl_xcd_grid(group_cap, (int64_t)n_modules * (group_tokens / 16) * slices),
                    kFThreads)) {
    pl_set_error("pl_lora_fused: grid of %lld groups too large", (long long)group_cap);
    return PL_ERR_LIMIT;
  }
  if (group_cap == 0) return PL_OK;
  a.x = x;
  a.ldx = ldx;
  a.K = K;
  const int64_t step = (int64_t)kFCC * 4 * E;
  const int64_t kq = (K + kFWaves - 1) / kFWaves;
  a.kw = (int32_t)((kq + step - 1) / step * step);
  a.arena = reinterpret_cast<const char*>(arena);
  a.table = table;
  a.num_modules = num_modules;
  a.tok = tok;
  a.groups = groups;
  a.meta = meta;
  a.group_cap = (int32_t)group_cap;
  a.sub = group_tokens / 16;
  a.slices = slices;
  a.epilogue = epilogue;
  a.n_jobs = n_modules;
  const int jtmax = (ldt + 15) / 16;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (dtype) {
    case PL_BF16: return launch_fused<PL_BF16>(a, jtmax, s);
    case PL_F16: return launch_fused<PL_F16>(a, jtmax, s);
    default: return launch_fused<PL_F32>(a, jtmax, s);
  }
}

namespace {

template <int DT, int MODE>
void launch_phase(const pl_fused_args& a, int jtmax, hipStream_t stream) {
  const dim3 grid((unsigned)pl_xcd_grid(a.group_cap, (int64_t)a.sub * a.slices));
  if (jtmax <= 1)
    hipLaunchKernelGGL((pl_lora_fused_tile<DT, 1, false, MODE>), grid, dim3(kFThreads), 0, stream, a);
  else if (jtmax == 2)
    hipLaunchKernelGGL((pl_lora_fused_tile<DT, 2, false, MODE>), grid, dim3(kFThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((pl_lora_fused_tile<DT, 4, false, MODE>), grid, dim3(kFThreads), 0, stream, a);
}

}  // namespace

int pl_fused_phase(int mode, int32_t dtype, const void* x, int64_t ldx, int32_t K, void* y,
                   int64_t ldy, int32_t N, const void* arena, const pl_slot_entry* table,
                   int32_t ldt, const int32_t* tok, const pl_group* groups, const int32_t* meta,
                   int64_t group_cap, int32_t group_tokens, int32_t slices, int32_t epilogue,
                   void* stream) {
  if ((mode != PL_FUSED_SHRINK && mode != PL_FUSED_EXPAND) || ldt <= 0 || ldt > kFRankMax ||
      group_cap < 1 || group_cap > ((int64_t)1 << 24) || K <= 0 || N <= 0 ||
      (group_tokens != PL_GROUP_TOKENS_SHORT && group_tokens != PL_GROUP_TOKENS_LONG) ||
      slices < 1 || slices > kFSliceMax || (mode == PL_FUSED_SHRINK && slices != 1)) {
    pl_set_error("pl_fused_phase: bad arguments");
    return PL_ERR_ARG;
  }
  if (!pl_grid_fits(pl_xcd_grid(group_cap, (int64_t)(group_tokens / 16) * slices), kFThreads)) {
    pl_set_error("pl_fused_phase: grid of %lld groups too large", (long long)group_cap);
    return PL_ERR_LIMIT;
  }
  const int E = dtype == PL_F32 ? 4 : 8;
  pl_fused_args a;
  a.x = x;
  a.ldx = ldx;
  a.K = K;
  const int64_t step = (int64_t)kFCC * 4 * E;
  const int64_t kq = (K + kFWaves - 1) / kFWaves;
  a.kw = (int32_t)((kq + step - 1) / step * step);
  a.arena = reinterpret_cast<const char*>(arena);
  a.table = table;
  a.num_modules = 1;
  a.tok = tok;
  a.groups = groups;
  a.meta = meta;
  a.group_cap = (int32_t)group_cap;
  a.sub = group_tokens / 16;
  a.slices = slices;
  a.epilogue = epilogue;
  a.n_jobs = 1;
  a.module[0] = 0;
  a.y[0] = y;
  a.ldy[0] = ldy;
  a.N[0] = N;
  const int64_t per_wave = ((int64_t)N + (int64_t)slices * kFWaves - 1) / ((int64_t)slices * kFWaves);
  a.nw[0] = (int32_t)((per_wave + kFColsMax - 1) / kFColsMax * kFColsMax);
  const int jtmax = (ldt + 15) / 16;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  auto go = [&](auto dt) {
    constexpr int D = decltype(dt)::value;
    if (mode == PL_FUSED_SHRINK)
      launch_phase<D, PL_FUSED_SHRINK>(a, jtmax, s);
    else
      launch_phase<D, PL_FUSED_EXPAND>(a, jtmax, s);
  };
  switch (dtype) {
    case PL_BF16: go(std::integral_constant<int, PL_BF16>()); break;
    case PL_F16: go(std::integral_constant<int, PL_F16>()); break;
    default: go(std::integral_constant<int, PL_F32>()); break;
  }
  return pl_launch_status(mode == PL_FUSED_SHRINK ? "pl_fused_phase(shrink)" : "pl_fused_phase(expand)");
}

extern "C" int pl_lora_fused(int32_t dtype, const void* x, int64_t ldx, int32_t K, void* y,
                             int64_t ldy, int32_t N, const void* arena, const pl_slot_entry* table,
                             int32_t num_modules, int32_t module, int32_t ldt, const int32_t* tok,
                             const pl_group* groups, const int32_t* meta, int64_t group_cap,
                             int32_t group_tokens, int32_t slices, int32_t epilogue, void* stream) {
  return pl_lora_fused_stacked(dtype, x, ldx, K, 1, &module, &y, &ldy, &N, arena, table,
                               num_modules, ldt, tok, groups, meta, group_cap, group_tokens, slices,
                               epilogue, stream);
}
