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

}  // namespace ghip
