// DynamicSlice / DynamicUpdateSlice windows and XLA scatter (ScatterSum / Max /
// Min), the device side of function.go:1571-1621 and gather.go:441-640.
//
// The window starts are run-time values (integer scalars in device memory), so
// each thread reads them (uniform loads) and clamps them to [0, dim - window]
// the way XLA defines DynamicSlice / DynamicUpdateSlice.
//
// Scatter combines each update element into the output with a vector-memory
// atomic: one thread per update element, windows whose start does not fit the
// operand skipped whole (XLA's rule).  fp32 / fp64 / 32- and 64-bit integers
// combine in place; 16-bit floats accumulate in an fp32 copy of the operand and
// 8/16-bit integers in an int32 copy (converted back afterwards), so a sum of
// many bf16 updates is rounded once instead of once per update.
#include <hip/hip_runtime.h>

#include <atomic>
#include <type_traits>

#include "common.h"
#include "graph.h"

namespace ghip {

namespace {

__device__ __forceinline__ int64_t load_index(const void* p, int dt) {
  switch (dt) {
    case GHIP_DTYPE_INT8: return *static_cast<const int8_t*>(p);
    case GHIP_DTYPE_INT16: return *static_cast<const int16_t*>(p);
    case GHIP_DTYPE_INT32: return *static_cast<const int32_t*>(p);
    case GHIP_DTYPE_UINT8: return *static_cast<const uint8_t*>(p);
    case GHIP_DTYPE_UINT16: return *static_cast<const uint16_t*>(p);
    case GHIP_DTYPE_UINT32: return *static_cast<const uint32_t*>(p);
    case GHIP_DTYPE_UINT64: {
      const uint64_t u = *static_cast<const uint64_t*>(p);
      return u > 0x7fffffffffffffffull ? INT64_MAX : static_cast<int64_t>(u);
    }
    default: return *static_cast<const int64_t*>(p);
  }
}

// Window copy between `src` and `dst`: thread i handles window element i (row
// major over d.win); the window sits at the clamped starts on the `at_dst` side
// (DynamicUpdateSlice) or the source side (DynamicSlice).
template <typename T>
__global__ void __launch_bounds__(256) window_copy_kernel(const T* __restrict__ src, T* __restrict__ dst, DynDesc d,
                                                          int64_t n, int at_dst) {
  int64_t start[kMaxRank];
#pragma unroll
  for (int k = 0; k < kMaxRank; ++k) {
    if (k >= d.rank) break;
    int64_t s = load_index(d.start[k], d.sdt[k]);
    const int64_t hi = d.dims[k] - d.win[k];
    start[k] = s < 0 ? 0 : (s > hi ? hi : s);
  }
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256) {
    int64_t q = i, so = 0, dof = 0;
    for (int k = d.rank - 1; k >= 0; --k) {
      const int64_t c = q % d.win[k];
      q /= d.win[k];
      so += (at_dst ? c : start[k] + c) * d.sst[k];
      dof += (at_dst ? start[k] + c : c) * d.dst[k];
    }
    dst[dof] = src[so];
  }
}

// ---------------------------------------------------------------- combiners
__device__ __forceinline__ float max_nan(float a, float b) { return (a != a || b != b) ? __builtin_nanf("") : (a > b ? a : b); }
__device__ __forceinline__ float min_nan(float a, float b) { return (a != a || b != b) ? __builtin_nanf("") : (a < b ? a : b); }
__device__ __forceinline__ double max_nan(double a, double b) { return (a != a || b != b) ? __builtin_nan("") : (a > b ? a : b); }
__device__ __forceinline__ double min_nan(double a, double b) { return (a != a || b != b) ? __builtin_nan("") : (a < b ? a : b); }

// Compare-and-swap loop for float max / min (no native NaN-propagating atomic).
template <typename F, typename U, bool MAX>
__device__ __forceinline__ void cas_minmax(F* p, F v) {
  U* a = reinterpret_cast<U*>(p);
  U old = __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  while (true) {
    const F cur = __builtin_bit_cast(F, old);
    const F nv = MAX ? max_nan(cur, v) : min_nan(cur, v);
    const U nb = __builtin_bit_cast(U, nv);
    if (nb == old) return;
    const U prev = atomicCAS(a, old, nb);
    if (prev == old) return;
    old = prev;
  }
}

template <typename A>
__device__ __forceinline__ void combine(A* p, A v, int mode) {
  if constexpr (std::is_same_v<A, float>) {
    if (mode == GHIP_SCATTER_SUM) unsafeAtomicAdd(p, v);
    else if (mode == GHIP_SCATTER_MAX) cas_minmax<float, unsigned int, true>(p, v);
    else cas_minmax<float, unsigned int, false>(p, v);
  } else if constexpr (std::is_same_v<A, double>) {
    if (mode == GHIP_SCATTER_SUM) unsafeAtomicAdd(p, v);
    else if (mode == GHIP_SCATTER_MAX) cas_minmax<double, unsigned long long, true>(p, v);
    else cas_minmax<double, unsigned long long, false>(p, v);
  } else if constexpr (std::is_same_v<A, long long>) {  // two's complement: add as unsigned
    if (mode == GHIP_SCATTER_SUM) atomicAdd(reinterpret_cast<unsigned long long*>(p), static_cast<unsigned long long>(v));
    else if (mode == GHIP_SCATTER_MAX) atomicMax(p, v);
    else atomicMin(p, v);
  } else {
    if (mode == GHIP_SCATTER_SUM) atomicAdd(p, v);
    else if (mode == GHIP_SCATTER_MAX) atomicMax(p, v);
    else atomicMin(p, v);
  }
}

// Update element -> accumulator value.
template <typename U, typename A>
__device__ __forceinline__ A widen(U u) {
  if constexpr (std::is_same_v<U, bf16_t>) return bf16_to_f32(u.bits);
  else if constexpr (std::is_same_v<U, _Float16>) return static_cast<float>(u);
  else return static_cast<A>(u);
}

// One thread per update element (row major over the update dims).
template <typename U, typename A>
__global__ void __launch_bounds__(256) scatter_kernel(const U* __restrict__ upd, const void* __restrict__ idx, A* acc,
                                                      ScatterDesc d, int64_t n, int mode) {
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256) {
    int64_t q = i, uo = 0, io = 0;
    int64_t w[kMaxRank];
#pragma unroll
    for (int k = 0; k < kMaxRank; ++k) w[k] = 0;
    for (int k = d.ur - 1; k >= 0; --k) {
      const int64_t c = q % d.udims[k];
      q /= d.udims[k];
      uo += c * d.ust[k];
      if (d.uwin_od[k] >= 0) w[d.uwin_od[k]] = c;
      else io += c * d.ibatch_st[k];
    }
    int64_t start[kMaxRank];
#pragma unroll
    for (int k = 0; k < kMaxRank; ++k) start[k] = 0;
    const char* ip = static_cast<const char*>(idx);
    const int ies = d.idx_es;
    for (int k = 0; k < d.nidx; ++k) start[d.sato[k]] = load_index(ip + (io + k * d.ivec_st) * ies, d.idx_dt);
    bool ok = true;
    for (int k = 0; k < d.r; ++k) ok = ok && start[k] >= 0 && start[k] <= d.odims[k] - d.wsize[k];
    if (!ok) continue;
    int64_t oo = 0;
    for (int k = 0; k < d.r; ++k) oo += (start[k] + w[k]) * d.ost[k];
    combine<A>(acc + oo, widen<U, A>(upd[uo]), mode);
  }
}

template <typename S, typename D>
__global__ void __launch_bounds__(256) convert_kernel(const S* __restrict__ src, D* __restrict__ dst, CopyDesc d,
                                                      int64_t n) {
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256) {
    int64_t q = i, so = 0;
    for (int k = d.rank - 1; k >= 0; --k) {
      so += (q % d.dims[k]) * d.sst[k];
      q /= d.dims[k];
    }
    if constexpr (std::is_same_v<S, bf16_t>) dst[i] = bf16_to_f32(src[so].bits);
    else if constexpr (std::is_same_v<D, bf16_t>) dst[i] = bf16_t{f32_to_bf16(src[so])};
    else dst[i] = static_cast<D>(src[so]);
  }
}

// Contiguous source: 8 elements per thread with vector loads and stores.
template <typename S, typename D>
__global__ void __launch_bounds__(256) convert_vec_kernel(const S* __restrict__ src, D* __restrict__ dst, int64_t groups) {
  struct alignas(8 * sizeof(S)) VS { S x[8]; };
  struct alignas(8 * sizeof(D)) VD { D x[8]; };
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < groups; i += static_cast<int64_t>(gridDim.x) * 256) {
    const VS v = reinterpret_cast<const VS*>(src)[i];
    VD w;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if constexpr (std::is_same_v<S, bf16_t>) w.x[e] = bf16_to_f32(v.x[e].bits);
      else if constexpr (std::is_same_v<D, bf16_t>) w.x[e] = bf16_t{f32_to_bf16(v.x[e])};
      else w.x[e] = static_cast<D>(v.x[e]);
    }
    reinterpret_cast<VD*>(dst)[i] = w;
  }
}

// ---------------------------------------------------------------- row scatter-add
// Embedding-gradient form (scatter along axis 0 of a [V, D] operand, one id per
// update row, whole rows): deterministic.  One workgroup sorts the update rows
// by table row, stably (LSD radix passes of 8 bits over keys row << 14 | pos kept
// in LDS; ranks inside a pass from wave ballots), so each table row's updates
// form a segment in their original order; then one workgroup per segment folds
// them into the row in that order, in fp32, rounding once:
// out[id] = (((out[id] + u_p1) + u_p2) + ...).
constexpr int kSortThreads = 1024;
constexpr int kSortWaves = kSortThreads / 64;
constexpr int kPosBits = 14;  // positions < kScatterRowsMax = 2^14

__device__ __forceinline__ unsigned long long lanemask_lt() {
  const int lane = threadIdx.x & 63;
  return lane ? (~0ull >> (64 - lane)) : 0ull;
}

// Lanes of the wave whose (active) digit equals this lane's.
__device__ __forceinline__ unsigned long long digit_peers(int dg, bool act) {
  unsigned long long peers = __ballot(act);
#pragma unroll
  for (int bit = 0; bit < 8; ++bit) {
    const unsigned long long bal = __ballot((dg >> bit) & 1);
    peers &= ((dg >> bit) & 1) ? bal : ~bal;
  }
  return peers;
}

// keys_out[n]: sorted (row << 14 | pos); seg[n + 2]: segment starts, then at
// seg[n] the segment count and at seg[n + 1] the number of in-range keys.
struct RowSortArgs {
  const void* ids;
  int id_dt;
  int64_t id_stride;
  int n, V, passes;
  int* keys_out;
  int* seg;
};

__device__ __forceinline__ void row_sort_body(const RowSortArgs& a) {
  __shared__ unsigned ka[kScatterRowsMax], kb[kScatterRowsMax];
  __shared__ int hist[kSortWaves][256];
  __shared__ int part[kSortThreads];
  const int n = a.n, V = a.V, passes = a.passes;
  int* keys_out = a.keys_out;
  int* seg = a.seg;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const char* ip = static_cast<const char*>(a.ids);
  const int es = a.id_dt == GHIP_DTYPE_INT64 ? 8 : 4;
  {
    // All of this thread's ids are loaded before any is stored, so the loads overlap.
    constexpr int kPer = kScatterRowsMax / kSortThreads;
    int64_t idv[kPer];
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int i = t + q * kSortThreads;
      idv[q] = i < n ? load_index(ip + static_cast<int64_t>(i) * a.id_stride * es, a.id_dt) : 0;
    }
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int i = t + q * kSortThreads;
      const int64_t id = idv[q];
      const unsigned row = (id < 0 || id >= V) ? static_cast<unsigned>(V) : static_cast<unsigned>(id);
      if (i < n) ka[i] = (row << kPosBits) | static_cast<unsigned>(i);
    }
  }
  __syncthreads();
  const int chunk = (n + kSortWaves - 1) / kSortWaves;
  const int beg = w * chunk, end = beg + chunk < n ? beg + chunk : n;
  unsigned* src = ka;
  unsigned* dst = kb;
  for (int p = 0; p < passes; ++p) {
    const int sh = kPosBits + 8 * p;
    for (int d = lane; d < 256; d += 64) hist[w][d] = 0;
    __syncthreads();
    for (int b0 = beg; b0 < end; b0 += 64) {  // count, per wave
      const int i = b0 + lane;
      const bool act = i < end;
      const int dg = act ? static_cast<int>((src[i] >> sh) & 255u) : 0;
      const unsigned long long peers = digit_peers(dg, act);
      if (act && (peers & lanemask_lt()) == 0) hist[w][dg] += __popcll(peers);
    }
    __syncthreads();
    // Bin t's start: exclusive scan over the digit totals (threads 0..255), then
    // each wave's run inside the bin in wave order.
    int tot = 0;
    if (t < 256)
      for (int ww = 0; ww < kSortWaves; ++ww) tot += hist[ww][t];
    part[t] = tot;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
      const int v = (t < 256 && t >= off) ? part[t - off] : 0;
      __syncthreads();
      part[t] += v;
      __syncthreads();
    }
    if (t < 256) {
      int base = part[t] - tot;
      for (int ww = 0; ww < kSortWaves; ++ww) {
        const int h = hist[ww][t];
        hist[ww][t] = base;
        base += h;
      }
    }
    __syncthreads();
    for (int b0 = beg; b0 < end; b0 += 64) {  // stable scatter, per wave in order
      const int i = b0 + lane;
      const bool act = i < end;
      const unsigned k = act ? src[i] : 0u;
      const int dg = static_cast<int>((k >> sh) & 255u);
      const unsigned long long peers = digit_peers(dg, act);
      const int rank = __popcll(peers & lanemask_lt());
      if (act) dst[hist[w][dg] + rank] = k;
      __builtin_amdgcn_wave_barrier();
      if (act && rank == 0) hist[w][dg] += __popcll(peers);
      __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();
    unsigned* tmp = src;
    src = dst;
    dst = tmp;
  }
  // Segment starts: in-range keys whose row differs from the previous key's.
  const int per = (n + kSortThreads - 1) / kSortThreads;
  const int lo = t * per, hi = lo + per < n ? lo + per : n;
  auto row_of = [&](int i) { return static_cast<int>(src[i] >> kPosBits); };
  int cnt = 0;
  for (int i = lo; i < hi; ++i) cnt += row_of(i) < V && (i == 0 || row_of(i) != row_of(i - 1));
  part[t] = cnt;
  __syncthreads();
  for (int off = 1; off < kSortThreads; off <<= 1) {
    const int v = t >= off ? part[t - off] : 0;
    __syncthreads();
    part[t] += v;
    __syncthreads();
  }
  int o = part[t] - cnt;
  for (int i = lo; i < hi; ++i) {
    const int r = row_of(i);
    if (r < V && (i == 0 || r != row_of(i - 1))) seg[o++] = i;
    if (r < V && (i + 1 == n || row_of(i + 1) >= V)) seg[n + 1] = i + 1;
    keys_out[i] = static_cast<int>(src[i]);
  }
  if (t == kSortThreads - 1) {
    seg[n] = part[t];
    if (part[t] == 0) seg[n + 1] = 0;
  }
}

__global__ void __launch_bounds__(kSortThreads) row_sort_kernel(RowSortArgs a) { row_sort_body(a); }

// Workgroup 0 sorts; the others copy the (contiguous) operand into the output
// meanwhile, 16 bytes per thread per step.
__global__ void __launch_bounds__(kSortThreads) row_sort_copy_kernel(RowSortArgs a, const uint4* __restrict__ src,
                                                                     uint4* __restrict__ dst, int64_t n16) {
  if (blockIdx.x == 0) {
    row_sort_body(a);
    return;
  }
  const int64_t stride = static_cast<int64_t>(gridDim.x - 1) * kSortThreads;
  int64_t i = static_cast<int64_t>(blockIdx.x - 1) * kSortThreads + threadIdx.x;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const uint4 v0 = src[i], v1 = src[i + stride], v2 = src[i + 2 * stride], v3 = src[i + 3 * stride];
    dst[i] = v0;
    dst[i + stride] = v1;
    dst[i + 2 * stride] = v2;
    dst[i + 3 * stride] = v3;
  }
  for (; i < n16; i += stride) dst[i] = src[i];
}

template <typename T>
__device__ __forceinline__ float to_f(T v) {
  if constexpr (std::is_same_v<T, bf16_t>) return bf16_to_f32(v.bits);
  else return static_cast<float>(v);
}
template <typename T>
__device__ __forceinline__ T from_f(float v) {
  if constexpr (std::is_same_v<T, bf16_t>) return bf16_t{f32_to_bf16(v)};
  else return static_cast<T>(v);
}

// One workgroup per segment; VEC: 8 consecutive columns per thread (16- or
// 32-byte accesses), else one column per thread.
template <typename T, bool VEC>
__global__ void __launch_bounds__(256) row_fold_kernel(const T* __restrict__ upd, int64_t upd_row, T* __restrict__ out,
                                                       int64_t D, const int* __restrict__ keys,
                                                       const int* __restrict__ seg, int n) {
  struct alignas(8 * sizeof(T)) V8 { T x[8]; };
  const int nseg = seg[n];
  for (int sgi = blockIdx.x; sgi < nseg; sgi += gridDim.x) {
    const int b = seg[sgi], e = sgi + 1 < nseg ? seg[sgi + 1] : seg[n + 1];
    const int64_t row = static_cast<int64_t>(static_cast<unsigned>(keys[b]) >> kPosBits);
    T* o = out + row * D;
    if constexpr (VEC) {
      for (int64_t c = threadIdx.x * 8ll; c < D; c += 256 * 8) {
        const V8 ov = *reinterpret_cast<const V8*>(o + c);
        float acc[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) acc[q] = to_f(ov.x[q]);
        for (int r = b; r < e; ++r) {
          const int64_t pos = keys[r] & ((1 << kPosBits) - 1);
          if (pos >= n) continue;  // cannot happen for keys the sort wrote; keeps reads in bounds
          const V8 uv = *reinterpret_cast<const V8*>(upd + pos * upd_row + c);
#pragma unroll
          for (int q = 0; q < 8; ++q) acc[q] += to_f(uv.x[q]);
        }
        V8 w;
#pragma unroll
        for (int q = 0; q < 8; ++q) w.x[q] = from_f<T>(acc[q]);
        *reinterpret_cast<V8*>(o + c) = w;
      }
    } else {
      for (int64_t c = threadIdx.x; c < D; c += 256) {
        float acc = to_f(o[c]);
        for (int r = b; r < e; ++r) {
          const int64_t pos = keys[r] & ((1 << kPosBits) - 1);
          if (pos < n) acc += to_f(upd[pos * upd_row + c]);
        }
        o[c] = from_f<T>(acc);
      }
    }
  }
}

unsigned grid_for(int64_t n) {
  int64_t g = (n + 255) / 256;
  if (g > 16384) g = 16384;
  return static_cast<unsigned>(g < 1 ? 1 : g);
}

}  // namespace

int launch_window_copy(int elem_bytes, const void* src, void* dst, const DynDesc& d, int at_dst, hipStream_t s,
                       GHipError* err) {
  int64_t n = 1;
  for (int k = 0; k < d.rank; ++k) n *= d.win[k];
  if (n == 0) return GHIP_OK;
  const unsigned g = grid_for(n);
  switch (elem_bytes) {
    case 1: hipLaunchKernelGGL(window_copy_kernel<uint8_t>, dim3(g), dim3(256), 0, s, static_cast<const uint8_t*>(src), static_cast<uint8_t*>(dst), d, n, at_dst); break;
    case 2: hipLaunchKernelGGL(window_copy_kernel<uint16_t>, dim3(g), dim3(256), 0, s, static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst), d, n, at_dst); break;
    case 4: hipLaunchKernelGGL(window_copy_kernel<uint32_t>, dim3(g), dim3(256), 0, s, static_cast<const uint32_t*>(src), static_cast<uint32_t*>(dst), d, n, at_dst); break;
    case 8: hipLaunchKernelGGL(window_copy_kernel<uint64_t>, dim3(g), dim3(256), 0, s, static_cast<const uint64_t*>(src), static_cast<uint64_t*>(dst), d, n, at_dst); break;
    default: return set_error(err, GHIP_ERR_UNSUPPORTED, "window copy: element size %d", elem_bytes);
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GHIP_OK : check_hip(e, err, "window copy launch");
}

int scatter_acc_dtype(int dt) {
  switch (dt) {
    case GHIP_DTYPE_BFLOAT16: case GHIP_DTYPE_FLOAT16: return GHIP_DTYPE_FLOAT32;
    case GHIP_DTYPE_INT8: case GHIP_DTYPE_INT16: case GHIP_DTYPE_UINT8: case GHIP_DTYPE_UINT16: return GHIP_DTYPE_INT32;
    default: return dt;
  }
}

int launch_scatter(int dtype, int mode, const void* updates, const void* indices, void* acc, const ScatterDesc& d,
                   hipStream_t s, GHipError* err) {
  int64_t n = 1;
  for (int k = 0; k < d.ur; ++k) n *= d.udims[k];
  if (n == 0) return GHIP_OK;
  const unsigned g = grid_for(n);
#define GHIP_SCATTER(U, A)                                                                                        \
  hipLaunchKernelGGL((scatter_kernel<U, A>), dim3(g), dim3(256), 0, s, static_cast<const U*>(updates), indices, \
                     static_cast<A*>(acc), d, n, mode)
  switch (dtype) {
    case GHIP_DTYPE_FLOAT32: GHIP_SCATTER(float, float); break;
    case GHIP_DTYPE_FLOAT64: GHIP_SCATTER(double, double); break;
    case GHIP_DTYPE_BFLOAT16: GHIP_SCATTER(bf16_t, float); break;
    case GHIP_DTYPE_FLOAT16: GHIP_SCATTER(_Float16, float); break;
    case GHIP_DTYPE_INT32: GHIP_SCATTER(int32_t, int); break;
    case GHIP_DTYPE_UINT32: GHIP_SCATTER(uint32_t, unsigned int); break;
    case GHIP_DTYPE_INT64: GHIP_SCATTER(int64_t, long long); break;
    case GHIP_DTYPE_UINT64: GHIP_SCATTER(uint64_t, unsigned long long); break;
    case GHIP_DTYPE_INT8: GHIP_SCATTER(int8_t, int); break;
    case GHIP_DTYPE_INT16: GHIP_SCATTER(int16_t, int); break;
    case GHIP_DTYPE_UINT8: GHIP_SCATTER(uint8_t, int); break;
    case GHIP_DTYPE_UINT16: GHIP_SCATTER(uint16_t, int); break;
    default: return set_error(err, GHIP_ERR_UNSUPPORTED, "scatter: dtype %s", dtype_name(dtype));
  }
#undef GHIP_SCATTER
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GHIP_OK : check_hip(e, err, "scatter launch");
}

int launch_convert(int src_dt, int dst_dt, const void* src, void* dst, const CopyDesc& d, hipStream_t s,
                   GHipError* err) {
  int64_t n = 1;
  for (int k = 0; k < d.rank; ++k) n *= d.dims[k];
  if (n == 0) return GHIP_OK;
  // Vector path: contiguous source, whole 8-element groups, aligned bases.
  bool contiguous = true;
  int64_t acc = 1;
  for (int k = d.rank - 1; k >= 0; --k) {
    contiguous = contiguous && (d.dims[k] == 1 || d.sst[k] == acc);
    acc *= d.dims[k];
  }
  const int ss = dtype_size(src_dt), ds = dtype_size(dst_dt);
  const bool vec = contiguous && n % 8 == 0 && reinterpret_cast<uintptr_t>(src) % (8 * ss) == 0 &&
                   reinterpret_cast<uintptr_t>(dst) % (8 * ds) == 0;
  const unsigned g = grid_for(vec ? n / 8 : n);
#define GHIP_CONVERT(S, D)                                                                                         \
  do {                                                                                                             \
    if (vec)                                                                                                       \
      hipLaunchKernelGGL((convert_vec_kernel<S, D>), dim3(g), dim3(256), 0, s, static_cast<const S*>(src),         \
                         static_cast<D*>(dst), n / 8);                                                             \
    else                                                                                                           \
      hipLaunchKernelGGL((convert_kernel<S, D>), dim3(g), dim3(256), 0, s, static_cast<const S*>(src),             \
                         static_cast<D*>(dst), d, n);                                                              \
  } while (0)
  if (src_dt == GHIP_DTYPE_BFLOAT16 && dst_dt == GHIP_DTYPE_FLOAT32) GHIP_CONVERT(bf16_t, float);
  else if (src_dt == GHIP_DTYPE_FLOAT32 && dst_dt == GHIP_DTYPE_BFLOAT16) GHIP_CONVERT(float, bf16_t);
  else if (src_dt == GHIP_DTYPE_FLOAT16 && dst_dt == GHIP_DTYPE_FLOAT32) GHIP_CONVERT(_Float16, float);
  else if (src_dt == GHIP_DTYPE_FLOAT32 && dst_dt == GHIP_DTYPE_FLOAT16) GHIP_CONVERT(float, _Float16);
  else if (src_dt == GHIP_DTYPE_INT8 && dst_dt == GHIP_DTYPE_INT32) GHIP_CONVERT(int8_t, int);
  else if (src_dt == GHIP_DTYPE_INT16 && dst_dt == GHIP_DTYPE_INT32) GHIP_CONVERT(int16_t, int);
  else if (src_dt == GHIP_DTYPE_UINT8 && dst_dt == GHIP_DTYPE_INT32) GHIP_CONVERT(uint8_t, int);
  else if (src_dt == GHIP_DTYPE_UINT16 && dst_dt == GHIP_DTYPE_INT32) GHIP_CONVERT(uint16_t, int);
  else if (src_dt == GHIP_DTYPE_INT32 && dst_dt == GHIP_DTYPE_INT8) GHIP_CONVERT(int, int8_t);
  else if (src_dt == GHIP_DTYPE_INT32 && dst_dt == GHIP_DTYPE_INT16) GHIP_CONVERT(int, int16_t);
  else if (src_dt == GHIP_DTYPE_INT32 && dst_dt == GHIP_DTYPE_UINT8) GHIP_CONVERT(int, uint8_t);
  else if (src_dt == GHIP_DTYPE_INT32 && dst_dt == GHIP_DTYPE_UINT16) GHIP_CONVERT(int, uint16_t);
  else return set_error(err, GHIP_ERR_UNSUPPORTED, "convert %s -> %s", dtype_name(src_dt), dtype_name(dst_dt));
#undef GHIP_CONVERT
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GHIP_OK : check_hip(e, err, "convert launch");
}

int launch_scatter_rows(int dtype, const void* updates, int64_t upd_row, const void* ids, int id_dt, int64_t id_stride,
                        int64_t n, void* out, int64_t V, int64_t D, void* scratch, const void* copy_src, hipStream_t s,
                        GHipError* err) {
  const int64_t table_bytes = V * D * dtype_size(dtype);
  if (n == 0 || D == 0) {
    if (copy_src && table_bytes) {
      const hipError_t ce = hipMemcpyAsync(out, copy_src, table_bytes, hipMemcpyDeviceToDevice, s);
      if (ce != hipSuccess) return check_hip(ce, err, "table copy");
    }
    return GHIP_OK;
  }
  if (n > kScatterRowsMax || V > kScatterRowsMaxTable)
    return set_error(err, GHIP_ERR_INVALID_ARG, "row scatter: %lld rows / table of %lld rows", (long long)n, (long long)V);
  int passes = 0;
  while ((V >> (8 * passes)) > 0) ++passes;  // cover the row values 0..V (V: out of range)
  auto* keys = static_cast<int*>(scratch);
  int* seg = keys + n;
  const RowSortArgs sa{ids, id_dt, id_stride, static_cast<int>(n), static_cast<int>(V), passes, keys, seg};
  if (copy_src) {
    if (table_bytes % 16 || reinterpret_cast<uintptr_t>(copy_src) % 16 || reinterpret_cast<uintptr_t>(out) % 16)
      return set_error(err, GHIP_ERR_INVALID_ARG, "row scatter: table copy needs 16-byte alignment");
    // One workgroup per CU (each holds the sort's LDS): the sort on one, the copy on the rest.
    static std::atomic<int> cus_of[64];  // per device; 0 = not queried yet
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    int cus = cus_of[dev].load(std::memory_order_relaxed);
    if (cus == 0) {
      if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 2) cus = 256;
      cus_of[dev].store(cus, std::memory_order_relaxed);
    }
    hipLaunchKernelGGL(row_sort_copy_kernel, dim3(cus), dim3(kSortThreads), 0, s, sa, static_cast<const uint4*>(copy_src),
                       static_cast<uint4*>(out), table_bytes / 16);
  } else {
    hipLaunchKernelGGL(row_sort_kernel, dim3(1), dim3(kSortThreads), 0, s, sa);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return check_hip(e, err, "row sort launch");
  const unsigned g = static_cast<unsigned>(n);
#define GHIP_FOLD(T)                                                                                                    \
  do {                                                                                                                 \
    const bool vec = D % 8 == 0 && upd_row % 8 == 0 && reinterpret_cast<uintptr_t>(updates) % (8 * sizeof(T)) == 0 &&  \
                     reinterpret_cast<uintptr_t>(out) % (8 * sizeof(T)) == 0;                                          \
    if (vec)                                                                                                           \
      hipLaunchKernelGGL((row_fold_kernel<T, true>), dim3(g), dim3(256), 0, s, static_cast<const T*>(updates), upd_row, \
                         static_cast<T*>(out), D, keys, seg, static_cast<int>(n));                                     \
    else                                                                                                               \
      hipLaunchKernelGGL((row_fold_kernel<T, false>), dim3(g), dim3(256), 0, s, static_cast<const T*>(updates),        \
                         upd_row, static_cast<T*>(out), D, keys, seg, static_cast<int>(n));                            \
  } while (0)
  switch (dtype) {
    case GHIP_DTYPE_FLOAT32: GHIP_FOLD(float); break;
    case GHIP_DTYPE_BFLOAT16: GHIP_FOLD(bf16_t); break;
    case GHIP_DTYPE_FLOAT16: GHIP_FOLD(_Float16); break;
    default: return set_error(err, GHIP_ERR_UNSUPPORTED, "row scatter: dtype %s", dtype_name(dtype));
  }
#undef GHIP_FOLD
  e = hipGetLastError();
  return e == hipSuccess ? GHIP_OK : check_hip(e, err, "row fold launch");
}

}  // namespace ghip
