// Adapter-major tiled SGMV kernels for gfx950 (MFMA 16x16, wave64).
//
// Both kernels walk the plan written by pl_plan_build: a list of groups of
// at most 64 tokens that share one slot.  A token's result never depends on
// which other tokens share its group, so the plan's order inside a slot is
// free.
//
// Shrink (replaces sgmv.py:63-138): one workgroup per (group, K-chunk).  Its
// four waves split the chunk along K; each lane streams 64 contiguous bytes
// of one token row of x and of one rank row of A per step, feeding 16x16
// MFMA tiles [tokens x ranks].  The four wave partials are summed in LDS in
// a fixed order, then stored (one K-chunk) or added atomically (split-K) to
// the fp32 intermediate tmp[position][rank].
//
// Expand (replaces sgmv.py:178-275): one workgroup per (group, 256 output
// columns), each wave owns 64 columns.  The MFMA computes the transposed
// tile [columns x tokens] so that B (stored [out][rank8], rank contiguous)
// and tmp (stored [position][ldt], rank contiguous) are both read as 16-byte
// rank chunks, and every lane ends up with 4 consecutive output columns of
// one token for the fused scale + add-back read-modify-write of y.
#include "pl_common.h"

namespace {

constexpr int kWaves = 4;
constexpr int kChunksPerLane = 4;  // 64 contiguous bytes per lane per step

struct pl_shrink_args {
  const void* x;
  int64_t ldx;
  int32_t K;
  int32_t kw;  // K per wave, multiple of the step span
  const char* arena;
  const pl_slot_entry* table;
  int32_t num_modules;
  int32_t module;
  const int32_t* tok;
  const pl_group* groups;
  const int32_t* meta;
  float* tmp;
  int32_t ldt;
  int32_t k_splits;
  int32_t atomic;
  float* zero_ptr;
  int64_t zero_count;
};

struct pl_expand_args {
  const float* tmp;
  int32_t ldt;
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

template <int DT>
__global__ __launch_bounds__(256) void pl_shrink_tiled(pl_shrink_args a) {
  typedef typename pl_traits<DT>::T T;
  constexpr int E = pl_traits<DT>::E;
  constexpr int kLaneSpan = kChunksPerLane * E;  // k covered by one lane per step
  constexpr int kStep = 4 * kLaneSpan;           // k covered by one wave per step
  __shared__ pl_f32x4 red[kWaves][4][64];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;

  if (a.zero_ptr != nullptr) {
    pl_f32x4* z = reinterpret_cast<pl_f32x4*>(a.zero_ptr);
    const int64_t n4 = a.zero_count >> 2;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + tid; i < n4; i += stride)
      z[i] = pl_f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const int g = blockIdx.x / a.k_splits;
  const int c = blockIdx.x - g * a.k_splits;
  if (g >= a.meta[0]) return;
  const pl_group grp = a.groups[g];
  const pl_slot_entry e = a.table[(int64_t)grp.slot * a.num_modules + a.module];
  const int rank = min(e.rank, a.ldt);  // the host guarantees rank <= ldt
  if (rank <= 0) return;
  const int len = grp.len;
  const int nrt = (len + 15) >> 4;
  const int K = a.K;
  const T* __restrict__ x = reinterpret_cast<const T*>(a.x);
  const T* __restrict__ A = reinterpret_cast<const T*>(a.arena + e.a_off);

  const T* xrow[4];
  bool xok[4];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) {
    const int p = rt * 16 + li;
    xok[rt] = p < len;
    const int t = xok[rt] ? a.tok[grp.start + p] : 0;
    xrow[rt] = x + (int64_t)t * a.ldx;
  }
  const int k0 = (c * kWaves + wave) * a.kw;
  const int k1 = min(K, k0 + a.kw);

  for (int rb = 0; rb < rank; rb += 64) {
    pl_f32x4 acc[4][4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) acc[rt][jt] = pl_f32x4{0.f, 0.f, 0.f, 0.f};

    for (int kb = k0; kb < k1; kb += kStep) {
      const int kl = kb + lg * kLaneSpan;
      pl_u32x4 xf[4][kChunksPerLane];
#pragma unroll
      for (int rt = 0; rt < 4; ++rt)
#pragma unroll
        for (int cc = 0; cc < kChunksPerLane; ++cc) {
          const int k = kl + cc * E;
          pl_u32x4 v = {0u, 0u, 0u, 0u};
          if (xok[rt] && k < k1) v = pl_ld16(xrow[rt] + k);
          xf[rt][cc] = v;
        }
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        if (rb + jt * 16 < rank) {
          const int j = rb + jt * 16 + li;
          pl_u32x4 af[kChunksPerLane];
#pragma unroll
          for (int cc = 0; cc < kChunksPerLane; ++cc) {
            const int k = kl + cc * E;
            pl_u32x4 v = {0u, 0u, 0u, 0u};
            if (j < rank && k < k1) v = pl_ld16(A + (int64_t)j * K + k);
            af[cc] = v;
          }
#pragma unroll
          for (int rt = 0; rt < 4; ++rt)
            if (rt < nrt)
#pragma unroll
              for (int cc = 0; cc < kChunksPerLane; ++cc)
                acc[rt][jt] = pl_mfma_chunk<DT>(xf[rt][cc], af[cc], acc[rt][jt]);
        }
      }
    }

    // Sum the four wave partials of each row tile in a fixed order.
    // acc[rt][jt][v] holds tile element (row 4*lg+v, column li).
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      if (rt < nrt) {
        __syncthreads();
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) red[wave][jt][lane] = acc[rt][jt];
        __syncthreads();
        const int jt = wave;  // thread (wave, lane) finishes tile column block jt
        const int j = rb + jt * 16 + li;
        const pl_f32x4 s = red[0][jt][lane] + red[1][jt][lane] + red[2][jt][lane] +
                           red[3][jt][lane];
        if (j < rank) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int prow = rt * 16 + lg * 4 + v;
            if (prow < len) {
              float* dst = a.tmp + (int64_t)(grp.start + prow) * a.ldt + j;
              if (a.atomic)
                atomicAdd(dst, s[v]);
              else
                *dst = s[v];
            }
          }
        }
      }
    }
  }
}

template <int DT>
__global__ __launch_bounds__(256) void pl_expand_tiled(pl_expand_args a) {
  typedef typename pl_traits<DT>::T T;
  typedef typename pl_traits<DT>::T4 T4;
  typedef typename pl_traits<DT>::T8 T8;
  constexpr int E = pl_traits<DT>::E;
  constexpr int kStep = 4 * E;  // rank slots per MFMA step

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
  const int n0 = c * 256 + wave * 64;
  if (n0 >= N) return;
  const int len = grp.len;
  const int nrt = (len + 15) >> 4;
  const T* __restrict__ Bc = reinterpret_cast<const T*>(a.arena + e.b_off);

  int trow[4];
  bool tok_ok[4];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) {
    const int p = rt * 16 + li;
    tok_ok[rt] = p < len;
    trow[rt] = grp.start + (tok_ok[rt] ? p : 0);
  }

  pl_f32x4 acc[4][4];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) acc[rt][ct] = pl_f32x4{0.f, 0.f, 0.f, 0.f};

  for (int j0 = 0; j0 < r8; j0 += kStep) {
    const int jl = j0 + lg * E;
    pl_u32x4 tf[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      pl_u32x4 v = {0u, 0u, 0u, 0u};
      if (tok_ok[rt] && jl < rank) {
        const float* src = a.tmp + (int64_t)trow[rt] * a.ldt + jl;
        if constexpr (E == 8) {
          const pl_f32x4 lo = *reinterpret_cast<const pl_f32x4*>(src);
          const pl_f32x4 hi = *reinterpret_cast<const pl_f32x4*>(src + 4);
          T8 h;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            h[i] = (T)((jl + i < rank) ? lo[i] : 0.f);
            h[i + 4] = (T)((jl + i + 4 < rank) ? hi[i] : 0.f);
          }
          v = __builtin_bit_cast(pl_u32x4, h);
        } else {
          pl_f32x4 f = *reinterpret_cast<const pl_f32x4*>(src);
#pragma unroll
          for (int i = 0; i < 4; ++i) f[i] = (jl + i < rank) ? f[i] : 0.f;
          v = __builtin_bit_cast(pl_u32x4, f);
        }
      }
      tf[rt] = v;
    }
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const int n = n0 + ct * 16 + li;
      pl_u32x4 bf = {0u, 0u, 0u, 0u};
      if (n < N && jl < r8) bf = pl_ld16(Bc + (int64_t)n * r8 + jl);
#pragma unroll
      for (int rt = 0; rt < 4; ++rt)
        if (rt < nrt) acc[rt][ct] = pl_mfma_chunk<DT>(bf, tf[rt], acc[rt][ct]);
    }
  }

  // acc[rt][ct][v] = delta(column n0 + ct*16 + 4*lg + v, token row rt*16 + li)
  const float scale = e.scale;
  const float scale_t = pl_round<DT>(scale);
  T* __restrict__ y = reinterpret_cast<T*>(a.y);
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) {
    if (rt < nrt && tok_ok[rt]) {
      const int t = a.tok[trow[rt]];
      T* yrow = y + (int64_t)t * a.ldy;
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        const int nb = n0 + ct * 16 + lg * 4;
        if (nb < N) {
          T4 yv = *reinterpret_cast<const T4*>(yrow + nb);
#pragma unroll
          for (int v = 0; v < 4; ++v)
            yv[v] = (T)pl_epilogue<DT>(acc[rt][ct][v], (float)yv[v], scale, scale_t, a.epilogue);
          *reinterpret_cast<T4*>(yrow + nb) = yv;
        }
      }
    }
  }
}

template <int DT>
int launch_shrink(const pl_shrink_args& a, int64_t group_cap, hipStream_t stream) {
  const int64_t grid = group_cap * a.k_splits;
  if (grid <= 0) return PL_OK;
  hipLaunchKernelGGL(pl_shrink_tiled<DT>, dim3((unsigned)grid), dim3(256), 0, stream, a);
  return pl_launch_status("pl_sgmv_shrink");
}

template <int DT>
int launch_expand(const pl_expand_args& a, int64_t group_cap, hipStream_t stream) {
  const int64_t grid = group_cap * a.n_chunks;
  if (grid <= 0) return PL_OK;
  hipLaunchKernelGGL(pl_expand_tiled<DT>, dim3((unsigned)grid), dim3(256), 0, stream, a);
  return pl_launch_status("pl_sgmv_expand");
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_common(int32_t dtype, const void* arena, const pl_slot_entry* table,
                 int32_t num_modules, int32_t module, const int32_t* tok,
                 const pl_group* groups, const int32_t* meta, int64_t group_cap) {
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
  if (!aligned16(arena)) {
    pl_set_error("arena base is not 16-byte aligned");
    return PL_ERR_ALIGN;
  }
  return PL_OK;
}

int prepare_shrink(pl_shrink_args& a, int32_t dtype, const void* x, int64_t ldx, int32_t K,
                   const void* arena, const pl_slot_entry* table, int32_t num_modules,
                   int32_t module, const int32_t* tok, const pl_group* groups,
                   const int32_t* meta, int64_t group_cap, float* tmp, int32_t ldt,
                   int32_t k_splits, float* zero_ptr, int64_t zero_count) {
  int st = check_common(dtype, arena, table, num_modules, module, tok, groups, meta, group_cap);
  if (st) return st;
  const int E = pl_chunk_elems(dtype);
  const int es = pl_elem_size(dtype);
  if (!x || !tmp) {
    pl_set_error("null x or tmp pointer");
    return PL_ERR_ARG;
  }
  if (K <= 0 || ldx < K || ldt <= 0 || (ldt & 7) != 0 || k_splits < 1) {
    pl_set_error("bad shrink sizes K=%d ldx=%lld ldt=%d k_splits=%d", K, (long long)ldx, ldt,
                 k_splits);
    return PL_ERR_ARG;
  }
  if (K % E != 0 || (ldx * es) % 16 != 0 || !aligned16(x) || !aligned16(tmp)) {
    pl_set_error("shrink needs K %% %d == 0 and 16-byte aligned rows", E);
    return PL_ERR_ALIGN;
  }
  if (zero_ptr && ((zero_count & 3) != 0 || !aligned16(zero_ptr) || zero_count < 0)) {
    pl_set_error("zero buffer must be 16-byte aligned with a multiple of 4 floats");
    return PL_ERR_ARG;
  }
  const int step = 16 * E;  // k per wave per step
  const int64_t per_split = (K + (int64_t)k_splits - 1) / k_splits;
  int64_t kw = (per_split + kWaves - 1) / kWaves;
  kw = (kw + step - 1) / step * step;
  const int64_t eff_splits = (K + kWaves * kw - 1) / (kWaves * kw);
  a.x = x;
  a.ldx = ldx;
  a.K = K;
  a.kw = (int32_t)kw;
  a.arena = reinterpret_cast<const char*>(arena);
  a.table = table;
  a.num_modules = num_modules;
  a.module = module;
  a.tok = tok;
  a.groups = groups;
  a.meta = meta;
  a.tmp = tmp;
  a.ldt = ldt;
  a.k_splits = (int32_t)eff_splits;
  a.atomic = k_splits > 1 ? 1 : 0;
  a.zero_ptr = zero_count > 0 ? zero_ptr : nullptr;
  a.zero_count = zero_count;
  if (group_cap * eff_splits > 0x7fffffffLL) {
    pl_set_error("shrink grid too large");
    return PL_ERR_LIMIT;
  }
  return PL_OK;
}

int prepare_expand(pl_expand_args& a, int32_t dtype, const float* tmp, int32_t ldt,
                   const void* arena, const pl_slot_entry* table, int32_t num_modules,
                   int32_t module, const int32_t* tok, const pl_group* groups,
                   const int32_t* meta, int64_t group_cap, void* y, int64_t ldy, int32_t N,
                   int32_t epilogue) {
  int st = check_common(dtype, arena, table, num_modules, module, tok, groups, meta, group_cap);
  if (st) return st;
  const int es = pl_elem_size(dtype);
  if (!y || !tmp) {
    pl_set_error("null y or tmp pointer");
    return PL_ERR_ARG;
  }
  if (N <= 0 || ldy < N || ldt <= 0 || (ldt & 7) != 0) {
    pl_set_error("bad expand sizes N=%d ldy=%lld ldt=%d", N, (long long)ldy, ldt);
    return PL_ERR_ARG;
  }
  if (epilogue != PL_EPI_FALLBACK && epilogue != PL_EPI_TRITON) {
    pl_set_error("bad epilogue mode %d", epilogue);
    return PL_ERR_ARG;
  }
  if (N % 4 != 0 || (ldy % 4) != 0 || (reinterpret_cast<uintptr_t>(y) % (4 * es)) != 0 ||
      !aligned16(tmp)) {
    pl_set_error("expand needs N %% 4 == 0 and %d-byte aligned y rows", 4 * es);
    return PL_ERR_ALIGN;
  }
  const int64_t n_chunks = (N + 255) / 256;
  if (group_cap * n_chunks > 0x7fffffffLL) {
    pl_set_error("expand grid too large");
    return PL_ERR_LIMIT;
  }
  a.tmp = tmp;
  a.ldt = ldt;
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

int dispatch_shrink(int32_t dtype, const pl_shrink_args& a, int64_t group_cap,
                    hipStream_t s) {
  switch (dtype) {
    case PL_BF16: return launch_shrink<PL_BF16>(a, group_cap, s);
    case PL_F16: return launch_shrink<PL_F16>(a, group_cap, s);
    default: return launch_shrink<PL_F32>(a, group_cap, s);
  }
}

int dispatch_expand(int32_t dtype, const pl_expand_args& a, int64_t group_cap,
                    hipStream_t s) {
  switch (dtype) {
    case PL_BF16: return launch_expand<PL_BF16>(a, group_cap, s);
    case PL_F16: return launch_expand<PL_F16>(a, group_cap, s);
    default: return launch_expand<PL_F32>(a, group_cap, s);
  }
}

}  // namespace

extern "C" int pl_sgmv_shrink(int32_t dtype, const void* x, int64_t ldx, int32_t K,
                              const void* arena, const pl_slot_entry* table,
                              int32_t num_modules, int32_t module, const int32_t* tok,
                              const pl_group* groups, const int32_t* meta, int64_t group_cap,
                              float* tmp, int32_t ldt, int32_t k_splits, float* zero_ptr,
                              int64_t zero_count, void* stream) {
  pl_shrink_args a;
  int st = prepare_shrink(a, dtype, x, ldx, K, arena, table, num_modules, module, tok, groups,
                          meta, group_cap, tmp, ldt, k_splits, zero_ptr, zero_count);
  if (st) return st;
  return dispatch_shrink(dtype, a, group_cap, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int pl_sgmv_expand(int32_t dtype, const float* tmp, int32_t ldt, const void* arena,
                              const pl_slot_entry* table, int32_t num_modules, int32_t module,
                              const int32_t* tok, const pl_group* groups, const int32_t* meta,
                              int64_t group_cap, void* y, int64_t ldy, int32_t N,
                              int32_t epilogue, void* stream) {
  pl_expand_args a;
  int st = prepare_expand(a, dtype, tmp, ldt, arena, table, num_modules, module, tok, groups,
                          meta, group_cap, y, ldy, N, epilogue);
  if (st) return st;
  return dispatch_expand(dtype, a, group_cap, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int pl_lora_apply(int32_t dtype, const void* x, int64_t ldx, int32_t K, void* y,
                             int64_t ldy, int32_t N, const void* arena,
                             const pl_slot_entry* table, int32_t num_modules, int32_t module,
                             const int32_t* tok, const pl_group* groups, const int32_t* meta,
                             int64_t group_cap, float* tmp, int32_t ldt, int32_t k_splits,
                             float* zero_ptr, int64_t zero_count, int32_t epilogue,
                             void* stream) {
  pl_shrink_args sa;
  pl_expand_args ea;
  int st = prepare_shrink(sa, dtype, x, ldx, K, arena, table, num_modules, module, tok, groups,
                          meta, group_cap, tmp, ldt, k_splits, zero_ptr, zero_count);
  if (st) return st;
  st = prepare_expand(ea, dtype, tmp, ldt, arena, table, num_modules, module, tok, groups, meta,
                      group_cap, y, ldy, N, epilogue);
  if (st) return st;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  st = dispatch_shrink(dtype, sa, group_cap, s);
  if (st) return st;
  return dispatch_expand(dtype, ea, group_cap, s);
}
