// Adapter-major tiled SGMV kernels for gfx950 (MFMA 16x16, wave64).
//
// Both kernels walk the plan written by pl_plan_build: a list of groups of
// at most G tokens that share one slot, G = 16 * RT with RT = 1 (short
// adapter segments, e.g. decode) or RT = 4 (long segments, e.g. prefill).
// RT is a template parameter so that registers are sized for the group:
// short segments get more K and more ranks in flight per wave instead of
// accumulators for rows that do not exist.  A token's result never depends
// on which other tokens share its group, so the plan's order inside a slot
// is free.
//
// Shrink (replaces sgmv.py:63-138): one workgroup per (group, K split).  Its
// four waves split the split's K range; per step each lane loads CC 16-byte
// chunks of one token row of x and of one rank row of A, and the four lanes
// that share a row read 64 contiguous bytes per load.  16x16 MFMA tiles
// [tokens x ranks] accumulate in fp32 (16*JT ranks per pass), the four wave
// partials are summed in LDS in a fixed order, and the block stores its sum
// with plain stores into its own fp32 plane planes[split][position][rank].
//
// Expand (replaces sgmv.py:178-275): one workgroup per (group, column chunk
// of 256 bf16/f16 or 128 f32 output columns), one 16-token row tile at a
// time.  The intermediate is the shrink planes summed in split order (four
// planes' loads in flight together) and rounded once to the model dtype; the
// MFMA runs on the transposed tile [columns x tokens] so that B (stored
// [out][rank8], rank contiguous) and the planes (rank contiguous) are both
// read in contiguous 16-byte rank chunks.  Split-K therefore needs no
// atomics, no cross-workgroup signalling and no cleared buffers: results are
// bitwise reproducible and every launch can be recorded in a HIP graph.
// The scaled, rounded delta goes through LDS to the row-major layout of y,
// and the fused add-back reads and writes y once with 16-byte accesses (512
// contiguous bytes per row).  With RT = 1 the y rows are loaded up front, in
// parallel with B.  Registers stay at or below 128 per lane so that four
// workgroups share a CU and hide each other's memory latency.
#include "pl_common.h"

namespace {

constexpr int kWaves = 4;
constexpr int kYRowsPerPass = 8;  // 256 threads, 32 lanes per tile row

// Shrink shape per row-tile count: CC 16-byte chunks per lane per step and
// JT 16-rank column tiles per pass.
template <int RT>
struct pl_shrink_shape;
template <>
struct pl_shrink_shape<1> {
  enum { CC = 4, JT = 4 };
};
template <>
struct pl_shrink_shape<4> {
  enum { CC = 2, JT = 2 };
};

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
  int64_t plane;  // floats between split planes
};

struct pl_expand_args {
  const float* planes;
  int32_t ldt;
  int32_t k_splits;
  int64_t plane;
  const char* arena;
  const pl_slot_entry* table;
  int32_t num_modules;
  int32_t module;
  const int32_t* tok;
  const pl_group* groups;
  const int32_t* meta;
  void* y;
  int64_t ldy;
  int32_t N;
  int32_t n_chunks;
  int32_t epilogue;
};

// Columns of y one expand wave owns: 64 for 2-byte types, 32 for fp32, so
// that a block's tile row is always 512 bytes.
template <int DT>
struct pl_expand_shape {
  enum { kColsWave = DT == PL_F32 ? 32 : 64 };
  enum { kCT = kColsWave / 16 };
  enum { kChunk = kWaves * kColsWave };
  enum { kPad = DT == PL_F32 ? 4 : 8 };  // 16 bytes of LDS row padding
  enum { kLdsRow = kChunk + kPad };
};

template <int DT, int RT>
__global__ __launch_bounds__(256, 4) void pl_shrink_tiled(pl_shrink_args a) {
  typedef typename pl_traits<DT>::T T;
  typedef pl_shrink_shape<RT> S;
  constexpr int E = pl_traits<DT>::E;
  constexpr int kInstr = 4 * E;          // k covered by one wave load (4 lane groups)
  constexpr int kStep = S::CC * kInstr;  // k covered by one wave step
  constexpr int kSlots = RT * S::JT;     // 16x16 tiles per pass
  __shared__ pl_f32x4 red[kWaves][kWaves][64];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;

  // block -> (group g, split c, served module job); the modules of one
  // (group, split) are adjacent so their shared x rows are fetched together
  const int job = blockIdx.x % a.n_jobs;
  const int gc = blockIdx.x / a.n_jobs;
  const int g = gc / a.k_splits;
  const int c = gc - g * a.k_splits;
  if (g >= a.meta[0]) return;
  const pl_group grp = a.groups[g];
  const pl_slot_entry e = a.table[(int64_t)grp.slot * a.num_modules + a.module[job]];
  const int rank = min(e.rank, a.ldt);  // the host guarantees rank <= ldt
  if (rank <= 0) return;
  const int len = min(grp.len, 16 * RT);  // the host pairs the plan's group size with RT
  const int nrt = (len + 15) >> 4;
  const int K = a.K;
  const T* __restrict__ x = reinterpret_cast<const T*>(a.x);
  const T* __restrict__ A = reinterpret_cast<const T*>(a.arena + e.a_off);
  float* __restrict__ out = a.planes[job] + (int64_t)c * a.plane;

  const T* xrow[RT];
  bool xok[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int p = rt * 16 + li;
    xok[rt] = p < len;
    const int t = xok[rt] ? a.tok[grp.start + p] : 0;
    xrow[rt] = x + (int64_t)t * a.ldx + lg * E;
  }
  const int k0 = (c * kWaves + wave) * a.kw;
  const int k1 = min(K, k0 + a.kw);

  for (int rb = 0; rb < rank; rb += 16 * S::JT) {
    pl_f32x4 acc[RT][S::JT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int jt = 0; jt < S::JT; ++jt) acc[rt][jt] = pl_f32x4{0.f, 0.f, 0.f, 0.f};

    for (int kb = k0; kb < k1; kb += kStep) {
      // chunk cc of lane (li, lg) covers k = kb + cc*kInstr + lg*E .. +E
      pl_u32x4 xf[RT][S::CC];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int cc = 0; cc < S::CC; ++cc) {
          const int k = kb + cc * kInstr;
          pl_u32x4 v = {0u, 0u, 0u, 0u};
          if (xok[rt] && k + lg * E < k1) v = pl_ld16(xrow[rt] + k);
          xf[rt][cc] = v;
        }
#pragma unroll
      for (int jt = 0; jt < S::JT; ++jt) {
        if (rb + jt * 16 < rank) {
          const int j = rb + jt * 16 + li;
          const T* arow = A + (int64_t)j * K + lg * E;
          pl_u32x4 af[S::CC];
#pragma unroll
          for (int cc = 0; cc < S::CC; ++cc) {
            const int k = kb + cc * kInstr;
            pl_u32x4 v = {0u, 0u, 0u, 0u};
            if (j < rank && k + lg * E < k1) v = pl_ld16(arow + k);
            af[cc] = v;
          }
#pragma unroll
          for (int rt = 0; rt < RT; ++rt)
            if (rt < nrt)
#pragma unroll
              for (int cc = 0; cc < S::CC; ++cc)
                acc[rt][jt] = pl_mfma_chunk<DT>(xf[rt][cc], af[cc], acc[rt][jt]);
        }
      }
    }

    // Sum the four wave partials of each tile in a fixed order, four tiles
    // (one per finishing wave) at a time.  acc[rt][jt][v] holds tile element
    // (row 4*lg+v, column li); tile index = rt*JT + jt.
#pragma unroll
    for (int t0 = 0; t0 < kSlots; t0 += kWaves) {
      if (t0 / S::JT < nrt) {
        __syncthreads();
#pragma unroll
        for (int q = 0; q < kWaves; ++q) {
          const int t = t0 + q;
          red[wave][q][lane] = acc[t / S::JT][t % S::JT];
        }
        __syncthreads();
        const int t = t0 + wave;  // tile this wave finishes
        const int rt = t / S::JT;
        const int j = rb + (t % S::JT) * 16 + li;
        const pl_f32x4 s = red[0][wave][lane] + red[1][wave][lane] + red[2][wave][lane] +
                           red[3][wave][lane];
        if (j < rank && rt < nrt) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int prow = rt * 16 + lg * 4 + v;
            if (prow < len) out[(int64_t)(grp.start + prow) * a.ldt + j] = s[v];
          }
        }
      }
    }
  }
}

// Intermediate chunk of one token for an MFMA operand: planes summed in split
// order, entries at or beyond `rank` zero, rounded once to T.  Four planes'
// loads are issued before any of them is added.
template <int DT, int E>
__device__ __forceinline__ pl_u32x4 pl_sum_planes(const float* __restrict__ src, int64_t plane,
                                                  int planes, int jl, int rank) {
  typedef typename pl_traits<DT>::T T;
  typedef typename pl_traits<DT>::T8 T8;
  pl_f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = {0.f, 0.f, 0.f, 0.f};
  int q = 0;
  for (; q + 4 <= planes; q += 4) {
    pl_f32x4 l[4], h[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      l[u] = *reinterpret_cast<const pl_f32x4*>(src + (q + u) * plane);
      if constexpr (E == 8) h[u] = *reinterpret_cast<const pl_f32x4*>(src + (q + u) * plane + 4);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      lo += l[u];
      if constexpr (E == 8) hi += h[u];
    }
  }
  for (; q < planes; ++q) {
    lo += *reinterpret_cast<const pl_f32x4*>(src + q * plane);
    if constexpr (E == 8) hi += *reinterpret_cast<const pl_f32x4*>(src + q * plane + 4);
  }
  if constexpr (E == 8) {
    T8 h8;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      h8[i] = (T)((jl + i < rank) ? lo[i] : 0.f);
      h8[i + 4] = (T)((jl + i + 4 < rank) ? hi[i] : 0.f);
    }
    return __builtin_bit_cast(pl_u32x4, h8);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) lo[i] = (jl + i < rank) ? lo[i] : 0.f;
    return __builtin_bit_cast(pl_u32x4, lo);
  }
}

template <int DT, int RT>
__global__ __launch_bounds__(256, 4) void pl_expand_tiled(pl_expand_args a) {
  typedef typename pl_traits<DT>::T T;
  typedef typename pl_traits<DT>::T4 T4;
  typedef typename pl_traits<DT>::T8 T8;
  typedef pl_expand_shape<DT> S;
  constexpr int E = pl_traits<DT>::E;
  constexpr int kStep = 4 * E;  // rank slots per MFMA step
  constexpr int kRows = 16 * RT;
  constexpr int kYPer = kRows / kYRowsPerPass;  // y rows per thread
  __shared__ __attribute__((aligned(16))) T delta[kRows * S::kLdsRow];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;

  const int g = blockIdx.x / a.n_chunks;
  const int c = blockIdx.x - g * a.n_chunks;
  if (g >= a.meta[0]) return;
  const pl_group grp = a.groups[g];
  const pl_slot_entry e = a.table[(int64_t)grp.slot * a.num_modules + a.module];
  const int rank = min(e.rank, a.ldt);  // the host guarantees rank <= ldt
  if (rank <= 0) return;
  const int r8 = e.rank8;
  const int N = a.N;
  const int n_base = c * S::kChunk;
  const int len = min(grp.len, kRows);  // the host pairs the plan's group size with RT
  const int nrt = (len + 15) >> 4;
  const float scale = e.scale;
  const float scale_t = pl_round<DT>(scale);
  const int n0 = n_base + wave * S::kColsWave;
  const T* __restrict__ Bc = reinterpret_cast<const T*>(a.arena + e.b_off);

  // y tile rows of this thread: rows t/32 + 8*i, columns (t%32)*E .. +E.
  const int yq = tid & 31;
  const int yr0 = tid >> 5;
  const int ycol = n_base + yq * E;
  T* __restrict__ y = reinterpret_cast<T*>(a.y);
  pl_u32x4 yv[kYPer];
  T* yptr[kYPer];
#pragma unroll
  for (int i = 0; i < kYPer; ++i) {
    const int r = yr0 + kYRowsPerPass * i;
    yptr[i] = (r < len && ycol < N) ? y + (int64_t)a.tok[grp.start + r] * a.ldy + ycol : nullptr;
    yv[i] = pl_u32x4{0u, 0u, 0u, 0u};
    if (RT == 1 && yptr[i] != nullptr) yv[i] = pl_ld16(yptr[i]);  // short tiles: load y early
  }

  // 1. delta^T tiles [columns x tokens] on the MFMA, one 16-token row tile at
  // a time; acc[ct][v] = delta(column n0 + ct*16 + 4*lg + v, token rt*16 + li).
  for (int rt = 0; rt < nrt; ++rt) {
    const int p = rt * 16 + li;
    const bool tok_ok = p < len;
    const float* prow = a.planes + (int64_t)(grp.start + (tok_ok ? p : 0)) * a.ldt;
    pl_f32x4 acc[S::kCT];
#pragma unroll
    for (int ct = 0; ct < S::kCT; ++ct) acc[ct] = pl_f32x4{0.f, 0.f, 0.f, 0.f};
    for (int j0 = 0; j0 < r8; j0 += kStep) {
      const int jl = j0 + lg * E;
      pl_u32x4 bf[S::kCT];
#pragma unroll
      for (int ct = 0; ct < S::kCT; ++ct) {
        const int n = n0 + ct * 16 + li;
        bf[ct] = pl_u32x4{0u, 0u, 0u, 0u};
        if (n < N && jl < r8) bf[ct] = pl_ld16(Bc + (int64_t)n * r8 + jl);
      }
      pl_u32x4 tf = {0u, 0u, 0u, 0u};
      if (tok_ok && jl < rank) tf = pl_sum_planes<DT, E>(prow + jl, a.plane, a.k_splits, jl, rank);
#pragma unroll
      for (int ct = 0; ct < S::kCT; ++ct) acc[ct] = pl_mfma_chunk<DT>(bf[ct], tf, acc[ct]);
    }
    // 2. scale and round in the epilogue's order, stage in LDS as [token][column]
    T* drow = delta + p * S::kLdsRow + wave * S::kColsWave;
#pragma unroll
    for (int ct = 0; ct < S::kCT; ++ct) {
      T4 d;
#pragma unroll
      for (int v = 0; v < 4; ++v) d[v] = (T)pl_delta<DT>(acc[ct][v], scale, scale_t, a.epilogue);
      *reinterpret_cast<T4*>(drow + ct * 16 + lg * 4) = d;
    }
  }
  __syncthreads();

  // 3. y = T(y + delta) with full-width stores.
  if (RT != 1) {
#pragma unroll
    for (int i = 0; i < kYPer; ++i)
      if (yptr[i] != nullptr) yv[i] = pl_ld16(yptr[i]);
  }
#pragma unroll
  for (int i = 0; i < kYPer; ++i) {
    if (yptr[i] != nullptr) {
      const int r = yr0 + kYRowsPerPass * i;
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

template <int DT, int RT>
int launch_shrink(const pl_shrink_args& a, int64_t group_cap, hipStream_t stream) {
  const int64_t grid = group_cap * a.k_splits * a.n_jobs;
  if (grid <= 0) return PL_OK;
  hipLaunchKernelGGL((pl_shrink_tiled<DT, RT>), dim3((unsigned)grid), dim3(256), 0, stream, a);
  return pl_launch_status("pl_sgmv_shrink");
}

template <int DT, int RT>
int launch_expand(const pl_expand_args& a, int64_t group_cap, hipStream_t stream) {
  const int64_t grid = group_cap * a.n_chunks;
  if (grid <= 0) return PL_OK;
  hipLaunchKernelGGL((pl_expand_tiled<DT, RT>), dim3((unsigned)grid), dim3(256), 0, stream, a);
  return pl_launch_status("pl_sgmv_expand");
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

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

// K per wave for a requested split count: a multiple of the wave step.
int64_t shrink_kw(int32_t dtype, int32_t K, int32_t k_splits, int32_t group_tokens) {
  const int cc = group_tokens == 16 ? pl_shrink_shape<1>::CC : pl_shrink_shape<4>::CC;
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
  if (group_cap * planes * n_jobs > 0x7fffffffLL) {
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
  a.plane = tmp_rows * ldt;
  return PL_OK;
}

int prepare_expand(pl_expand_args& a, int32_t dtype, const void* ws, int32_t ldt,
                   int64_t tmp_rows, int32_t planes, const void* arena,
                   const pl_slot_entry* table, int32_t num_modules, int32_t module,
                   const int32_t* tok, const pl_group* groups, const int32_t* meta,
                   int64_t group_cap, int32_t group_tokens, void* y, int64_t ldy, int32_t N,
                   int32_t epilogue) {
  int st = check_common(dtype, arena, table, num_modules, module, tok, groups, meta, group_cap,
                        group_tokens);
  if (st) return st;
  if ((st = check_ws(ws, ldt, tmp_rows))) return st;
  const int E = pl_chunk_elems(dtype);
  const int es = pl_elem_size(dtype);
  if (!y) {
    pl_set_error("null y pointer");
    return PL_ERR_ARG;
  }
  if (N <= 0 || ldy < N || planes < 1 || planes > 4096) {
    pl_set_error("bad expand sizes N=%d ldy=%lld planes=%d", N, (long long)ldy, planes);
    return PL_ERR_ARG;
  }
  if (epilogue != PL_EPI_FALLBACK && epilogue != PL_EPI_TRITON) {
    pl_set_error("bad epilogue mode %d", epilogue);
    return PL_ERR_ARG;
  }
  if (N % E != 0 || (ldy * es) % 16 != 0 || !aligned16(y)) {
    pl_set_error("expand needs N %% %d == 0 and 16-byte aligned y rows", E);
    return PL_ERR_ALIGN;
  }
  const int chunk = 4 * (dtype == PL_F32 ? 32 : 64);
  const int64_t n_chunks = (N + chunk - 1) / chunk;
  if (group_cap * n_chunks > 0x7fffffffLL) {
    pl_set_error("expand grid too large");
    return PL_ERR_LIMIT;
  }
  a.planes = reinterpret_cast<const float*>(ws);
  a.ldt = ldt;
  a.k_splits = planes;
  a.plane = tmp_rows * ldt;
  a.arena = reinterpret_cast<const char*>(arena);
  a.table = table;
  a.num_modules = num_modules;
  a.module = module;
  a.tok = tok;
  a.groups = groups;
  a.meta = meta;
  a.y = y;
  a.ldy = ldy;
  a.N = N;
  a.n_chunks = (int32_t)n_chunks;
  a.epilogue = epilogue;
  return PL_OK;
}

template <int RT>
int dispatch_shrink_rt(int32_t dtype, const pl_shrink_args& a, int64_t group_cap,
                       hipStream_t s) {
  switch (dtype) {
    case PL_BF16: return launch_shrink<PL_BF16, RT>(a, group_cap, s);
    case PL_F16: return launch_shrink<PL_F16, RT>(a, group_cap, s);
    default: return launch_shrink<PL_F32, RT>(a, group_cap, s);
  }
}

template <int RT>
int dispatch_expand_rt(int32_t dtype, const pl_expand_args& a, int64_t group_cap,
                       hipStream_t s) {
  switch (dtype) {
    case PL_BF16: return launch_expand<PL_BF16, RT>(a, group_cap, s);
    case PL_F16: return launch_expand<PL_F16, RT>(a, group_cap, s);
    default: return launch_expand<PL_F32, RT>(a, group_cap, s);
  }
}

int dispatch_shrink(int32_t dtype, int32_t group_tokens, const pl_shrink_args& a,
                    int64_t group_cap, hipStream_t s) {
  return group_tokens == 16 ? dispatch_shrink_rt<1>(dtype, a, group_cap, s)
                            : dispatch_shrink_rt<4>(dtype, a, group_cap, s);
}

int dispatch_expand(int32_t dtype, int32_t group_tokens, const pl_expand_args& a,
                    int64_t group_cap, hipStream_t s) {
  return group_tokens == 16 ? dispatch_expand_rt<1>(dtype, a, group_cap, s)
                            : dispatch_expand_rt<4>(dtype, a, group_cap, s);
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
  return dispatch_shrink(dtype, group_tokens, a, group_cap, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int pl_sgmv_expand(int32_t dtype, const void* ws, int32_t ldt, int64_t tmp_rows,
                              int32_t planes, const void* arena, const pl_slot_entry* table,
                              int32_t num_modules, int32_t module, const int32_t* tok,
                              const pl_group* groups, const int32_t* meta, int64_t group_cap,
                              int32_t group_tokens, void* y, int64_t ldy, int32_t N,
                              int32_t epilogue, void* stream) {
  pl_expand_args a;
  int st = prepare_expand(a, dtype, ws, ldt, tmp_rows, planes, arena, table, num_modules, module,
                          tok, groups, meta, group_cap, group_tokens, y, ldy, N, epilogue);
  if (st) return st;
  return dispatch_expand(dtype, group_tokens, a, group_cap, reinterpret_cast<hipStream_t>(stream));
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
  st = prepare_expand(ea, dtype, ws, ldt, tmp_rows, sa.k_splits, arena, table, num_modules,
                      module, tok, groups, meta, group_cap, group_tokens, y, ldy, N, epilogue);
  if (st) return st;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  st = dispatch_shrink(dtype, group_tokens, sa, group_cap, s);
  if (st) return st;
  return dispatch_expand(dtype, group_tokens, ea, group_cap, s);
}
