// Integer / indexing kernels: argmin/argmax, iota, and the embedding-gather entry
// point (its kernel is the graph Gather's, in k_generic.hip).
// All three are bit-exact by construction (copies and integer arithmetic).
#include <limits>
#include <type_traits>

#include "common.h"
#include "graph.h"

namespace ghip {

// ---------------------------------------------------------------------------
// ArgMin / ArgMax along the middle axis of [outer, n, inner].
// One thread per (outer, inner) output when inner > 1 (adjacent threads read
// adjacent columns: coalesced); one wave per row when inner == 1.
// Order: for floating point, NaN beats everything (first NaN wins); among numbers
// the extreme value wins and ties keep the lowest index.  Values compare in V:
// fp32 for the float dtypes (bf16 / f16 widen exactly), int64 / uint64 for the
// signed / unsigned integers.
// ---------------------------------------------------------------------------
template <typename T> struct ArgV { using type = float; };
template <> struct ArgV<int8_t> { using type = int64_t; };
template <> struct ArgV<int16_t> { using type = int64_t; };
template <> struct ArgV<int32_t> { using type = int64_t; };
template <> struct ArgV<int64_t> { using type = int64_t; };
template <> struct ArgV<uint8_t> { using type = uint64_t; };
template <> struct ArgV<uint16_t> { using type = uint64_t; };
template <> struct ArgV<uint32_t> { using type = uint64_t; };
template <> struct ArgV<uint64_t> { using type = uint64_t; };

template <typename T> __device__ __forceinline__ typename ArgV<T>::type arg_load(const T* p) { return *p; }
template <> __device__ __forceinline__ float arg_load<bf16_t>(const bf16_t* p) { return Elem<bf16_t>::load1(p); }
template <> __device__ __forceinline__ float arg_load<f16_t>(const f16_t* p) { return Elem<f16_t>::load1(p); }

template <typename V>
struct ArgBest {
  V v;
  int64_t i;
};
template <typename V>
__device__ __forceinline__ ArgBest<V> arg_pick(ArgBest<V> a, ArgBest<V> b, bool is_min) {
  // Returns the better of a and b (a and b from disjoint index sets).
  if constexpr (std::is_floating_point<V>::value) {
    const bool an = isnan(a.v), bn = isnan(b.v);
    if (an || bn) {
      if (an && bn) return a.i <= b.i ? a : b;
      return an ? a : b;
    }
  }
  if (a.v == b.v) return a.i <= b.i ? a : b;
  const bool a_better = is_min ? (a.v < b.v) : (a.v > b.v);
  return a_better ? a : b;
}
// Start value of a wave's search: worse than or equal to every element.
template <typename V>
__device__ __forceinline__ V arg_sentinel(bool is_min) {
  if constexpr (std::is_floating_point<V>::value) return is_min ? INFINITY : -INFINITY;
  else return is_min ? std::numeric_limits<V>::max() : std::numeric_limits<V>::lowest();
}
template <typename V>
__device__ __forceinline__ V shfl_xor_v(V v, int off) {
  if constexpr (sizeof(V) == 8) {
    return __builtin_bit_cast(V, __shfl_xor(__builtin_bit_cast(int64_t, v), off, 64));
  } else {
    return __shfl_xor(v, off, 64);
  }
}
template <typename T, typename O>
__global__ __launch_bounds__(256) void argminmax_cols_kernel(const T* __restrict__ x, int64_t outer,
                                                             int64_t n, int64_t inner, int is_min,
                                                             O* __restrict__ out) {
  using V = typename ArgV<T>::type;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= outer * inner) return;
  const int64_t o = t / inner, j = t % inner;
  const T* xr = x + o * n * inner + j;
  ArgBest<V> best{arg_load(xr), 0};
  for (int64_t i = 1; i < n; ++i) best = arg_pick(best, ArgBest<V>{arg_load(xr + i * inner), i}, is_min);
  out[t] = static_cast<O>(best.i);
}
template <typename T, typename O>
__global__ __launch_bounds__(256) void argminmax_rows_kernel(const T* __restrict__ x, int64_t rows,
                                                             int64_t n, int is_min,
                                                             O* __restrict__ out) {
  using V = typename ArgV<T>::type;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;
  if (r >= rows) return;
  const int lane = threadIdx.x % kWave;
  const T* xr = x + r * n;
  ArgBest<V> best{arg_sentinel<V>(is_min), INT64_MAX};
  for (int64_t c = lane; c < n; c += kWave) best = arg_pick(best, ArgBest<V>{arg_load(xr + c), c}, is_min);
  // The sentinel (index INT64_MAX) only survives in lanes that saw no element;
  // a real element equal to it ties and wins on its lower index.
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    ArgBest<V> o{shfl_xor_v(best.v, off), __shfl_xor(best.i, off, 64)};
    best = arg_pick(best, o, is_min);
  }
  if (lane == 0) out[r] = static_cast<O>(best.i);
}

// ---------------------------------------------------------------------------
// Iota.
// ---------------------------------------------------------------------------
template <typename O>
__global__ __launch_bounds__(256) void iota_kernel(O* __restrict__ out, int64_t total, int64_t n,
                                                   int64_t inner) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= total) return;
  out[t] = static_cast<O>((t / inner) % n);
}

template <>
__global__ __launch_bounds__(256) void iota_kernel<bf16_t>(bf16_t* __restrict__ out, int64_t total,
                                                           int64_t n, int64_t inner) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= total) return;
  out[t].bits = f32_to_bf16(static_cast<float>((t / inner) % n));
}

static inline unsigned blocks_for(int64_t work, int per_block) {
  return static_cast<unsigned>((work + per_block - 1) / per_block);
}

}  // namespace ghip

using namespace ghip;

extern "C" int ghip_gather_rows(const void* table, int64_t V, int64_t row_bytes,
                                const int32_t* ids, int64_t n, void* out, void* stream,
                                GHipError* err) {
  if (V <= 0 || row_bytes <= 0 || n < 0)
    return set_error(err, GHIP_ERR_INVALID_ARG, "gather_rows: bad sizes V=%lld row_bytes=%lld n=%lld",
                     (long long)V, (long long)row_bytes, (long long)n);
  if (n == 0) return GHIP_OK;
  if (!table || !ids || !out) return set_error(err, GHIP_ERR_INVALID_ARG, "gather_rows: null pointer");
  // The graph's Gather kernel (k_generic.hip): one wave per row, clamped ids.
  return launch_gather_rows(table, V, row_bytes, ids, GHIP_DTYPE_INT32, n, out, static_cast<hipStream_t>(stream),
                            err);
}

template <typename T, typename O>
static hipError_t launch_arg(const void* x, int64_t outer, int64_t n, int64_t inner, int is_min,
                             void* out, hipStream_t s) {
  if (inner == 1) {
    hipLaunchKernelGGL((argminmax_rows_kernel<T, O>), dim3(blocks_for(outer, 4)), dim3(256), 0, s,
                       static_cast<const T*>(x), outer, n, is_min, static_cast<O*>(out));
  } else {
    hipLaunchKernelGGL((argminmax_cols_kernel<T, O>), dim3(blocks_for(outer * inner, 256)),
                       dim3(256), 0, s, static_cast<const T*>(x), outer, n, inner, is_min,
                       static_cast<O*>(out));
  }
  return hipGetLastError();
}

extern "C" int ghip_argminmax(int dtype, const void* x, int64_t outer, int64_t n, int64_t inner,
                              int is_min, int out_dtype, void* out, void* stream, GHipError* err) {
  if (outer < 0 || n <= 0 || inner < 0)
    return set_error(err, GHIP_ERR_INVALID_ARG, "argminmax: reduced axis must be non-empty");
  if (outer * inner == 0) return GHIP_OK;
  if (!x || !out) return set_error(err, GHIP_ERR_INVALID_ARG, "argminmax: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  const bool o32 = out_dtype == GHIP_DTYPE_INT32, o64 = out_dtype == GHIP_DTYPE_INT64;
  if (!o32 && !o64) return set_error(err, GHIP_ERR_UNSUPPORTED, "argminmax: output dtype %d", out_dtype);
  auto go = [&](auto tag) {
    using T = decltype(tag);
    return o32 ? launch_arg<T, int32_t>(x, outer, n, inner, is_min, out, s)
               : launch_arg<T, int64_t>(x, outer, n, inner, is_min, out, s);
  };
  switch (dtype) {
    case GHIP_DTYPE_FLOAT32: e = go(float{}); break;
    case GHIP_DTYPE_BFLOAT16: e = go(bf16_t{}); break;
    case GHIP_DTYPE_FLOAT16: e = go(f16_t{}); break;
    case GHIP_DTYPE_INT8: e = go(int8_t{}); break;
    case GHIP_DTYPE_INT16: e = go(int16_t{}); break;
    case GHIP_DTYPE_INT32: e = go(int32_t{}); break;
    case GHIP_DTYPE_INT64: e = go(int64_t{}); break;
    case GHIP_DTYPE_UINT8: e = go(uint8_t{}); break;
    case GHIP_DTYPE_UINT16: e = go(uint16_t{}); break;
    case GHIP_DTYPE_UINT32: e = go(uint32_t{}); break;
    case GHIP_DTYPE_UINT64: e = go(uint64_t{}); break;
    default: return set_error(err, GHIP_ERR_UNSUPPORTED, "argminmax: input dtype %d", dtype);
  }
  GHIP_CHECK(e, err);
  return GHIP_OK;
}

extern "C" int ghip_iota(int dtype, void* out, int64_t outer, int64_t n, int64_t inner, void* stream,
                         GHipError* err) {
  if (outer < 0 || n < 0 || inner < 0) return set_error(err, GHIP_ERR_INVALID_ARG, "iota: negative size");
  const int64_t total = outer * n * inner;
  if (total == 0) return GHIP_OK;
  if (!out) return set_error(err, GHIP_ERR_INVALID_ARG, "iota: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned g = blocks_for(total, 256);
  switch (dtype) {
    case GHIP_DTYPE_INT32:
      hipLaunchKernelGGL(iota_kernel<int32_t>, dim3(g), dim3(256), 0, s, static_cast<int32_t*>(out), total, n, inner);
      break;
    case GHIP_DTYPE_INT64:
      hipLaunchKernelGGL(iota_kernel<int64_t>, dim3(g), dim3(256), 0, s, static_cast<int64_t*>(out), total, n, inner);
      break;
    case GHIP_DTYPE_FLOAT32:
      hipLaunchKernelGGL(iota_kernel<float>, dim3(g), dim3(256), 0, s, static_cast<float*>(out), total, n, inner);
      break;
    case GHIP_DTYPE_BFLOAT16:
      hipLaunchKernelGGL(iota_kernel<bf16_t>, dim3(g), dim3(256), 0, s, static_cast<bf16_t*>(out), total, n, inner);
      break;
    default:
      return set_error(err, GHIP_ERR_UNSUPPORTED, "iota: dtype %d", dtype);
  }
  GHIP_CHECK(hipGetLastError(), err);
  return GHIP_OK;
}
