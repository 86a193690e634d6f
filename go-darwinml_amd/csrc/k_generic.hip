// Generic kernels the graph lowering falls back to: strided copy (materialises
// transposes, broadcasts, slices, concatenations), reductions over arbitrary
// axes, and the row gather with int32/int64 ids.
#include "common.h"
#include "graph.h"

namespace ghip {

// ---------------------------------------------------------------------------
// Strided copy: one element per thread per grid-stride step; elements of 1, 2,
// 4, 8 or 16 bytes.  When the innermost source and destination strides are 1
// the caller may widen the element (see launch_strided_copy).
// ---------------------------------------------------------------------------
template <typename E>
__global__ __launch_bounds__(256) void strided_copy_kernel(const E* __restrict__ src, E* __restrict__ dst,
                                                           CopyDesc d, int64_t total) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    int64_t r = i, so = 0, dof = 0;
    for (int k = d.rank - 1; k >= 0; --k) {
      const int64_t idx = r % d.dims[k];
      r /= d.dims[k];
      so += idx * d.sst[k];
      dof += idx * d.dst[k];
    }
    dst[dof] = src[so];
  }
}

// Dense copy of n 16-byte vectors: each thread moves kPer vectors, all loads
// issued before the stores, nontemporal both ways (the data is streamed once).
constexpr int kCopyPer = 4;
typedef unsigned u32x4_nt __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void copy_dense16_kernel(const u32x4_nt* __restrict__ src,
                                                          u32x4_nt* __restrict__ dst, int64_t n) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (256 * kCopyPer) + threadIdx.x;
  u32x4_nt v[kCopyPer];
#pragma unroll
  for (int k = 0; k < kCopyPer; ++k)
    if (base + k * 256 < n) v[k] = __builtin_nontemporal_load(src + base + k * 256);
#pragma unroll
  for (int k = 0; k < kCopyPer; ++k)
    if (base + k * 256 < n) __builtin_nontemporal_store(v[k], dst + base + k * 256);
}

static unsigned grid_for(int64_t total) {
  int64_t g = (total + 255) / 256;
  if (g > 65536) g = 65536;
  return static_cast<unsigned>(g < 1 ? 1 : g);
}

int launch_strided_copy(int elem_bytes, const void* src, void* dst, const CopyDesc& din,
                        hipStream_t s, GHipError* err) {
  // Drop unit axes and merge an axis into the next one when both sides step
  // through them as one run (stride[k] == stride[k+1] * dims[k+1]): fewer
  // divisions per element, and a dense copy becomes rank 1.
  CopyDesc d;
  d.rank = 0;
  int64_t total = 1;
  for (int k = 0; k < din.rank; ++k) {
    total *= din.dims[k];
    if (din.dims[k] == 1) continue;
    if (d.rank > 0 && d.sst[d.rank - 1] == din.sst[k] * din.dims[k] && d.dst[d.rank - 1] == din.dst[k] * din.dims[k]) {
      d.dims[d.rank - 1] *= din.dims[k];
      d.sst[d.rank - 1] = din.sst[k];
      d.dst[d.rank - 1] = din.dst[k];
      continue;
    }
    d.dims[d.rank] = din.dims[k];
    d.sst[d.rank] = din.sst[k];
    d.dst[d.rank] = din.dst[k];
    ++d.rank;
  }
  if (total == 0) return GHIP_OK;
  if (d.rank == 0) {  // a single element
    d.rank = 1;
    d.dims[0] = 1;
    d.sst[0] = d.dst[0] = 1;
  }
  // Dense on both sides: 16-byte vectors when the size and both bases allow.
  if (d.rank == 1 && d.sst[0] == 1 && d.dst[0] == 1) {
    const int64_t bytes = total * elem_bytes;
    if (bytes % 16 == 0 && reinterpret_cast<uintptr_t>(src) % 16 == 0 && reinterpret_cast<uintptr_t>(dst) % 16 == 0) {
      const int64_t n = bytes / 16;
      const int64_t g = (n + 256 * kCopyPer - 1) / (256 * kCopyPer);
      if (g > 0x7fffffffLL) return set_error(err, GHIP_ERR_INVALID_ARG, "copy: too large");
      hipLaunchKernelGGL(copy_dense16_kernel, dim3(static_cast<unsigned>(g)), dim3(256), 0, s,
                         static_cast<const u32x4_nt*>(src), static_cast<u32x4_nt*>(dst), n);
      GHIP_CHECK(hipGetLastError(), err);
      return GHIP_OK;
    }
  }
  // Widen the element when the innermost axis is unit-stride on both sides and
  // its extent, both base pointers and all other strides allow it.
  int eb = elem_bytes;
  if (d.rank > 0 && d.sst[d.rank - 1] == 1 && d.dst[d.rank - 1] == 1) {
    while (eb < 16) {
      const int f = 2;
      const int64_t inner = d.dims[d.rank - 1];
      bool ok = inner % f == 0 && (reinterpret_cast<uintptr_t>(src) % (eb * f)) == 0 &&
                (reinterpret_cast<uintptr_t>(dst) % (eb * f)) == 0;
      for (int k = 0; ok && k < d.rank - 1; ++k) ok = d.sst[k] % f == 0 && d.dst[k] % f == 0;
      if (!ok) break;
      d.dims[d.rank - 1] /= f;
      for (int k = 0; k < d.rank - 1; ++k) {
        d.sst[k] /= f;
        d.dst[k] /= f;
      }
      eb *= f;
      total /= f;
    }
  }
  const unsigned g = grid_for(total);
  switch (eb) {
    case 1: hipLaunchKernelGGL(strided_copy_kernel<uint8_t>, dim3(g), dim3(256), 0, s, (const uint8_t*)src, (uint8_t*)dst, d, total); break;
    case 2: hipLaunchKernelGGL(strided_copy_kernel<uint16_t>, dim3(g), dim3(256), 0, s, (const uint16_t*)src, (uint16_t*)dst, d, total); break;
    case 4: hipLaunchKernelGGL(strided_copy_kernel<uint32_t>, dim3(g), dim3(256), 0, s, (const uint32_t*)src, (uint32_t*)dst, d, total); break;
    case 8: hipLaunchKernelGGL(strided_copy_kernel<uint2>, dim3(g), dim3(256), 0, s, (const uint2*)src, (uint2*)dst, d, total); break;
    case 16: hipLaunchKernelGGL(strided_copy_kernel<uint4>, dim3(g), dim3(256), 0, s, (const uint4*)src, (uint4*)dst, d, total); break;
    default: return set_error(err, GHIP_ERR_INVALID_ARG, "strided copy: element size %d", eb);
  }
  GHIP_CHECK(hipGetLastError(), err);
  return GHIP_OK;
}

// ---------------------------------------------------------------------------
// Reductions.  Accumulator: fp32 for fp32/bf16/fp16, fp64 for fp64, int64 /
// uint64 for integers.  One wave per output when the reduced extent is >= 64
// (lanes stride the reduced index space, then a butterfly), else one thread per
// output.
// ---------------------------------------------------------------------------
template <typename T> struct RAcc { using type = float; };
template <> struct RAcc<double> { using type = double; };
template <> struct RAcc<int8_t> { using type = int64_t; };
template <> struct RAcc<int16_t> { using type = int64_t; };
template <> struct RAcc<int32_t> { using type = int64_t; };
template <> struct RAcc<int64_t> { using type = int64_t; };
template <> struct RAcc<uint8_t> { using type = uint64_t; };
template <> struct RAcc<uint16_t> { using type = uint64_t; };
template <> struct RAcc<uint32_t> { using type = uint64_t; };
template <> struct RAcc<uint64_t> { using type = uint64_t; };

template <typename T> __device__ __forceinline__ typename RAcc<T>::type rload(const T* p) { return *p; }
template <> __device__ __forceinline__ float rload<bf16_t>(const bf16_t* p) { return bf16_to_f32(p->bits); }
template <> __device__ __forceinline__ float rload<_Float16>(const _Float16* p) { return static_cast<float>(*p); }

template <typename T> __device__ __forceinline__ void rstore(T* p, typename RAcc<T>::type v) { *p = static_cast<T>(v); }
template <> __device__ __forceinline__ void rstore<bf16_t>(bf16_t* p, float v) { p->bits = f32_to_bf16(v); }
template <> __device__ __forceinline__ void rstore<_Float16>(_Float16* p, float v) { *p = static_cast<_Float16>(v); }

template <typename A>
__device__ __forceinline__ A rcombine(A a, A b, int op) {
  switch (op) {
    case GHIP_REDUCE_SUM: return a + b;
    case GHIP_REDUCE_PRODUCT: return a * b;
    case GHIP_REDUCE_MAX: return (a > b || a != a) ? a : b;  // NaN propagates
    default: return (a < b || a != a) ? a : b;
  }
}

template <typename A>
__device__ __forceinline__ A rinit(int op) {
  switch (op) {
    case GHIP_REDUCE_SUM: return A(0);
    case GHIP_REDUCE_PRODUCT: return A(1);
    case GHIP_REDUCE_MAX:
      if constexpr (std::is_floating_point<A>::value) return -INFINITY;
      else return std::numeric_limits<A>::lowest();
    default:
      if constexpr (std::is_floating_point<A>::value) return INFINITY;
      else return std::numeric_limits<A>::max();
  }
}

__device__ __forceinline__ int64_t offset_of(int64_t i, int rank, const int64_t* dims, const int64_t* st) {
  int64_t off = 0;
  for (int k = rank - 1; k >= 0; --k) {
    off += (i % dims[k]) * st[k];
    i /= dims[k];
  }
  return off;
}

template <typename T>
__global__ __launch_bounds__(256) void reduce_thread_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                                            ReduceDesc d, int64_t osize, int64_t rsize,
                                                            int op) {
  using A = typename RAcc<T>::type;
  const int64_t o = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (o >= osize) return;
  const T* base = src + offset_of(o, d.orank, d.odims, d.ost);
  A acc = rinit<A>(op);
  for (int64_t r = 0; r < rsize; ++r) acc = rcombine<A>(acc, rload(base + offset_of(r, d.rrank, d.rdims, d.rst)), op);
  rstore(dst + o, acc);
}

template <typename A>
__device__ __forceinline__ A shfl_xor_any(A v, int off) {
  if constexpr (sizeof(A) == 8) {
    int64_t bits = __builtin_bit_cast(int64_t, v);
    bits = __shfl_xor(bits, off, 64);
    return __builtin_bit_cast(A, bits);
  } else {
    return __shfl_xor(v, off, 64);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void reduce_wave_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                                          ReduceDesc d, int64_t osize, int64_t rsize,
                                                          int op) {
  using A = typename RAcc<T>::type;
  const int64_t o = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / 64;
  if (o >= osize) return;
  const int lane = threadIdx.x % 64;
  const T* base = src + offset_of(o, d.orank, d.odims, d.ost);
  A acc = rinit<A>(op);
  for (int64_t r = lane; r < rsize; r += 64) acc = rcombine<A>(acc, rload(base + offset_of(r, d.rrank, d.rdims, d.rst)), op);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc = rcombine<A>(acc, shfl_xor_any(acc, off), op);
  if (lane == 0) rstore(dst + o, acc);
}

template <typename T>
static hipError_t launch_reduce_t(const void* src, const ReduceDesc& d, void* dst, int op, hipStream_t s) {
  int64_t osize = 1, rsize = 1;
  for (int k = 0; k < d.orank; ++k) osize *= d.odims[k];
  for (int k = 0; k < d.rrank; ++k) rsize *= d.rdims[k];
  if (osize == 0) return hipSuccess;
  if (rsize >= 64) {
    hipLaunchKernelGGL(reduce_wave_kernel<T>, dim3(static_cast<unsigned>((osize + 3) / 4)), dim3(256), 0, s,
                       static_cast<const T*>(src), static_cast<T*>(dst), d, osize, rsize, op);
  } else {
    hipLaunchKernelGGL(reduce_thread_kernel<T>, dim3(static_cast<unsigned>((osize + 255) / 256)), dim3(256), 0, s,
                       static_cast<const T*>(src), static_cast<T*>(dst), d, osize, rsize, op);
  }
  return hipGetLastError();
}

int launch_reduce(int dtype, int op, const void* src, const ReduceDesc& d, void* dst, hipStream_t s,
                  GHipError* err) {
  hipError_t e;
  switch (dtype) {
    case GHIP_DTYPE_FLOAT32: e = launch_reduce_t<float>(src, d, dst, op, s); break;
    case GHIP_DTYPE_BFLOAT16: e = launch_reduce_t<bf16_t>(src, d, dst, op, s); break;
    case GHIP_DTYPE_FLOAT16: e = launch_reduce_t<_Float16>(src, d, dst, op, s); break;
    case GHIP_DTYPE_FLOAT64: e = launch_reduce_t<double>(src, d, dst, op, s); break;
    case GHIP_DTYPE_INT8: e = launch_reduce_t<int8_t>(src, d, dst, op, s); break;
    case GHIP_DTYPE_INT16: e = launch_reduce_t<int16_t>(src, d, dst, op, s); break;
    case GHIP_DTYPE_INT32: e = launch_reduce_t<int32_t>(src, d, dst, op, s); break;
    case GHIP_DTYPE_INT64: e = launch_reduce_t<int64_t>(src, d, dst, op, s); break;
    case GHIP_DTYPE_UINT8: e = launch_reduce_t<uint8_t>(src, d, dst, op, s); break;
    case GHIP_DTYPE_UINT16: e = launch_reduce_t<uint16_t>(src, d, dst, op, s); break;
    case GHIP_DTYPE_UINT32: e = launch_reduce_t<uint32_t>(src, d, dst, op, s); break;
    case GHIP_DTYPE_UINT64: e = launch_reduce_t<uint64_t>(src, d, dst, op, s); break;
    default: return set_error(err, GHIP_ERR_UNSUPPORTED, "reduce: dtype %d", dtype);
  }
  GHIP_CHECK(e, err);
  return GHIP_OK;
}

// ---------------------------------------------------------------------------
// Row gather with int32 / int64 ids (the public ghip_gather_rows takes int32).
// ---------------------------------------------------------------------------
// One wave per output row.  A wave issues the loads of up to 4 vectors per lane
// (a 4 KiB bf16 row of 2048 values at 16-byte vectors) before their stores, so a
// row's reads are in flight together.  ids and n are the first kernel arguments
// (preloaded into SGPRs, -amdgpu-kernarg-preload-count for this file): the id
// load, on which every row load depends, is issued without a kernel-argument fetch.
template <typename V, typename I>
__global__ __launch_bounds__(256) void gather_any_kernel(const I* __restrict__ ids, int64_t n,
                                                         const V* __restrict__ table, int64_t nrows,
                                                         int64_t row_vecs, V* __restrict__ out) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / 64;
  if (r >= n) return;
  const int lane = threadIdx.x % 64;
  int64_t id = static_cast<int64_t>(ids[r]);
  id = id < 0 ? 0 : (id > nrows - 1 ? nrows - 1 : id);
  const V* srcp = table + id * row_vecs;
  V* dstp = out + r * row_vecs;
  int64_t c0 = 0;
  for (; c0 + 4 * 64 <= row_vecs; c0 += 4 * 64) {
    const V a0 = srcp[c0 + lane], a1 = srcp[c0 + 64 + lane], a2 = srcp[c0 + 128 + lane], a3 = srcp[c0 + 192 + lane];
    dstp[c0 + lane] = a0;
    dstp[c0 + 64 + lane] = a1;
    dstp[c0 + 128 + lane] = a2;
    dstp[c0 + 192 + lane] = a3;
  }
  for (int64_t c = c0 + lane; c < row_vecs; c += 64) dstp[c] = srcp[c];
}

template <typename I>
static hipError_t gather_t(const void* table, int64_t V_, int64_t row_bytes, const I* ids, int64_t n,
                           void* out, hipStream_t s) {
  const unsigned grid = static_cast<unsigned>((n + 3) / 4);
  auto al = [](const void* p, unsigned a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; };
  if (row_bytes % 16 == 0 && al(table, 16) && al(out, 16))
    hipLaunchKernelGGL((gather_any_kernel<uint4, I>), dim3(grid), dim3(256), 0, s, ids, n, (const uint4*)table, V_,
                       row_bytes / 16, (uint4*)out);
  else if (row_bytes % 4 == 0 && al(table, 4) && al(out, 4))
    hipLaunchKernelGGL((gather_any_kernel<uint32_t, I>), dim3(grid), dim3(256), 0, s, ids, n, (const uint32_t*)table,
                       V_, row_bytes / 4, (uint32_t*)out);
  else
    hipLaunchKernelGGL((gather_any_kernel<uint8_t, I>), dim3(grid), dim3(256), 0, s, ids, n, (const uint8_t*)table, V_,
                       row_bytes, (uint8_t*)out);
  return hipGetLastError();
}

int launch_gather_rows(const void* table, int64_t V_, int64_t row_bytes, const void* ids, int id_dtype,
                       int64_t n, void* out, hipStream_t s, GHipError* err) {
  if (n == 0) return GHIP_OK;
  hipError_t e;
  switch (id_dtype) {
    case GHIP_DTYPE_INT32: e = gather_t(table, V_, row_bytes, static_cast<const int32_t*>(ids), n, out, s); break;
    case GHIP_DTYPE_INT64: e = gather_t(table, V_, row_bytes, static_cast<const int64_t*>(ids), n, out, s); break;
    case GHIP_DTYPE_UINT32: e = gather_t(table, V_, row_bytes, static_cast<const uint32_t*>(ids), n, out, s); break;
    case GHIP_DTYPE_INT16: e = gather_t(table, V_, row_bytes, static_cast<const int16_t*>(ids), n, out, s); break;
    case GHIP_DTYPE_INT8: e = gather_t(table, V_, row_bytes, static_cast<const int8_t*>(ids), n, out, s); break;
    case GHIP_DTYPE_UINT8: e = gather_t(table, V_, row_bytes, static_cast<const uint8_t*>(ids), n, out, s); break;
    case GHIP_DTYPE_UINT16: e = gather_t(table, V_, row_bytes, static_cast<const uint16_t*>(ids), n, out, s); break;
    default: return set_error(err, GHIP_ERR_UNSUPPORTED, "gather: index dtype %s", dtype_name(id_dtype));
  }
  GHIP_CHECK(e, err);
  return GHIP_OK;
}

}  // namespace ghip

extern "C" int ghip_copy_strided(int elem_bytes, const void* src, void* dst, int rank, const int64_t* dims,
                                 const int64_t* src_strides, const int64_t* dst_strides, void* stream,
                                 GHipError* err) {
  using namespace ghip;
  if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8 && elem_bytes != 16)
    return set_error(err, GHIP_ERR_INVALID_ARG, "copy: element size %d", elem_bytes);
  if (rank < 0 || rank > kMaxRank) return set_error(err, GHIP_ERR_INVALID_ARG, "copy: rank %d", rank);
  if (rank > 0 && (!dims || !src_strides || !dst_strides))
    return set_error(err, GHIP_ERR_INVALID_ARG, "copy: null dims or strides");
  CopyDesc d;
  d.rank = rank;
  int64_t total = 1;
  for (int k = 0; k < rank; ++k) {
    if (dims[k] < 0) return set_error(err, GHIP_ERR_INVALID_ARG, "copy: negative size");
    d.dims[k] = dims[k];
    d.sst[k] = src_strides[k];
    d.dst[k] = dst_strides[k];
    total *= dims[k];
  }
  if (total == 0) return GHIP_OK;
  if (!src || !dst) return set_error(err, GHIP_ERR_INVALID_ARG, "copy: null pointer");
  return launch_strided_copy(elem_bytes, src, dst, d, static_cast<hipStream_t>(stream), err);
}
