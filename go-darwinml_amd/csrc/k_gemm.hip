// Batched GEMM for DotGeneral: c[b] = a[b] (M x K) * b[b] (K x N), fp32 accumulate.
//
// bf16 path (the MFMA path the metric is quoted on): the core lives in
// gemm_bf16_dev.h (shared with the Compile-time generated epilogue GEMMs); the
// kernels here instantiate it with a plain store epilogue.
// fp32 path: v_mfma_f32_32x32x2f32 with MN-major LDS tiles (one float per lane).
// Anything the vector paths cannot address (odd strides, unaligned bases,
// negative strides, > 2 GiB per batch slice) runs a generic LDS-tiled kernel.
#include "common.h"
#include "gemm_bf16_dev.h"

namespace ghip {

template <typename OutT>
__device__ __forceinline__ void store_out(OutT* p, float v);
template <>
__device__ __forceinline__ void store_out<float>(float* p, float v) { *p = v; }
template <>
__device__ __forceinline__ void store_out<bf16_t>(bf16_t* p, float v) { p->bits = f32_to_bf16(v); }

// Epilogue of the precompiled bf16 kernels: store 4 adjacent outputs, one 8-byte
// (bf16) / 16-byte (fp32) store when the row allows it.
template <typename OutT>
struct StoreEpi {
  struct Pre {};
  OutT* c;
  int64_t sc_b, sc_m, N;
  int vec;
  template <bool FULL>
  __device__ __forceinline__ void prefetch(int64_t, int64_t, int64_t, Pre&) const {}
  template <bool FULL>
  __device__ __forceinline__ void store(int64_t bb, int64_t m, int64_t n, const float* v, const float*,
                                        const Pre&) const {
    OutT* dst = c + bb * sc_b + m * sc_m + n;
    if (vec && (FULL || n + 3 < N)) {
      if constexpr (sizeof(OutT) == 2) {
        *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
      } else {
        *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (n + e < N) store_out<OutT>(dst + e, v[e]);
    }
  }
};

template <int BM, int BN, int WM, int WN, bool A_K, bool B_K, typename OutT>
__global__ __launch_bounds__(WM* WN * 64, 1) void gemm_bf16_kernel(GemmParams p) {
  const StoreEpi<OutT> epi{static_cast<OutT*>(p.c), p.sc_b, p.sc_m, p.N, p.vec_c};
  gemm_bf16_body<BM, BN, WM, WN, A_K, B_K, 1>(p, epi);
}

// ---------------------------------------------------------------------------
// fp32 MFMA path: 128x128x32 tiles, 4 waves (2x2, 64x64 each),
// v_mfma_f32_32x32x2f32.  LDS tiles are MN-major [k][row] so a fragment read is
// 32 consecutive floats.
// ---------------------------------------------------------------------------
constexpr int kBK32 = 32;

template <int R, int T, bool KCONTIG>
struct TileLoaderF32 {
  // K-contiguous: float4 along k for one row; LD = R + 1 (scalar LDS writes).
  // MN-contiguous: float4 along rows for one k; LD = R + 4 (vector LDS writes).
  static constexpr int kLD = KCONTIG ? R + 1 : R + 4;
  static constexpr int kUnits = R * kBK32 / 4;
  static constexpr int kPer = (kUnits + T - 1) / T;
  float4 r[kPer];

  __device__ __forceinline__ void load(const float* base, int64_t s_row, int64_t s_k,
                                       int64_t rows_left, int64_t k_left, int tid) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int u = tid + i * T;
      if constexpr (KCONTIG) {
        const int row = u / (kBK32 / 4), kc = u % (kBK32 / 4);
        const bool ok = u < kUnits && row < rows_left && kc * 4 < k_left;
        r[i] = ok ? *reinterpret_cast<const float4*>(base + row * s_row + kc * 4)
                  : make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        const int rg = u % (R / 4), k = u / (R / 4);
        const bool ok = u < kUnits && rg * 4 < rows_left && k < k_left;
        r[i] = ok ? *reinterpret_cast<const float4*>(base + k * s_k + rg * 4)
                  : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
  }
  __device__ __forceinline__ void store(float* lds, int tid) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int u = tid + i * T;
      if (u >= kUnits) continue;
      if constexpr (KCONTIG) {
        const int row = u / (kBK32 / 4), kc = u % (kBK32 / 4);
        lds[(kc * 4 + 0) * kLD + row] = r[i].x;
        lds[(kc * 4 + 1) * kLD + row] = r[i].y;
        lds[(kc * 4 + 2) * kLD + row] = r[i].z;
        lds[(kc * 4 + 3) * kLD + row] = r[i].w;
      } else {
        const int rg = u % (R / 4), k = u / (R / 4);
        *reinterpret_cast<float4*>(lds + k * kLD + rg * 4) = r[i];
      }
    }
  }
};

template <bool A_K, bool B_K, typename OutT>
__global__ __launch_bounds__(256) void gemm_f32_kernel(GemmParams p) {
  constexpr int BM = 128, BN = 128, T = 256, WN = 2;
  constexpr int TM = 64, TN = 64, FM = 2, FN = 2;
  using LA = TileLoaderF32<BM, T, A_K>;
  using LB = TileLoaderF32<BN, T, B_K>;
  constexpr int SA = kBK32 * LA::kLD, SB = kBK32 * LB::kLD;
  __shared__ __attribute__((aligned(16))) float lds[2][SA + SB];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  int64_t bb;
  int tm, tn;
  map_tile(blockIdx.x, p.batch * p.tiles_m * p.tiles_n, p.tiles_m, p.tiles_n, bb, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;
  const float* A = static_cast<const float*>(p.a) + bb * p.sa_b + m0 * p.sa_m;
  const float* B = static_cast<const float*>(p.b) + bb * p.sb_b + n0 * p.sb_n;
  LA la;
  LB lb;
  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int KT = static_cast<int>((p.K + kBK32 - 1) / kBK32);
  la.load(A, p.sa_m, p.sa_k, p.M - m0, p.K, tid);
  lb.load(B, p.sb_n, p.sb_k, p.N - n0, p.K, tid);
  la.store(lds[0], tid);
  lb.store(lds[0] + SA, tid);
  __syncthreads();
  const int frow = lane & 31, kk = lane >> 5;
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < KT;
    if (more) {
      const int64_t k0 = static_cast<int64_t>(kt + 1) * kBK32;
      la.load(A + k0 * p.sa_k, p.sa_m, p.sa_k, p.M - m0, p.K - k0, tid);
      lb.load(B + k0 * p.sb_k, p.sb_n, p.sb_k, p.N - n0, p.K - k0, tid);
    }
    const float* As = lds[cur];
    const float* Bs = lds[cur] + SA;
#pragma unroll
    for (int s = 0; s < kBK32 / 2; ++s) {
      const int k = s * 2 + kk;
      float af[FM], bfv[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) af[i] = As[k * LA::kLD + wm * TM + i * 32 + frow];
#pragma unroll
      for (int j = 0; j < FN; ++j) bfv[j] = Bs[k * LB::kLD + wn * TN + j * 32 + frow];
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i], bfv[j], acc[i][j], 0, 0, 0);
    }
    if (more) {
      la.store(lds[cur ^ 1], tid);
      lb.store(lds[cur ^ 1] + SA, tid);
    }
    __syncthreads();
  }
  OutT* C = static_cast<OutT*>(p.c) + bb * p.sc_b;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int64_t col = n0 + wn * TN + j * 32 + frow;
      if (col >= p.N) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t row = m0 + wm * TM + i * 32 + (v >> 2) * 8 + kk * 4 + (v & 3);
        if (row < p.M) store_out<OutT>(C + row * p.sc_m + col, acc[i][j][v]);
      }
    }
}

// ---------------------------------------------------------------------------
// Generic fallback: 16x16 output tiles, arbitrary strides, scalar loads.
// ---------------------------------------------------------------------------
template <typename InT, typename OutT>
__global__ __launch_bounds__(256) void gemm_generic_kernel(GemmParams p) {
  __shared__ float As[16][17], Bs[16][17];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int64_t bb = blockIdx.z;
  const int64_t m = static_cast<int64_t>(blockIdx.y) * 16 + ty;
  const int64_t n = static_cast<int64_t>(blockIdx.x) * 16 + tx;
  const InT* A = static_cast<const InT*>(p.a) + bb * p.sa_b;
  const InT* B = static_cast<const InT*>(p.b) + bb * p.sb_b;
  float acc = 0.f;
  for (int64_t k0 = 0; k0 < p.K; k0 += 16) {
    const int64_t am = static_cast<int64_t>(blockIdx.y) * 16 + ty, ak = k0 + tx;
    As[ty][tx] = (am < p.M && ak < p.K) ? Elem<InT>::load1(A + am * p.sa_m + ak * p.sa_k) : 0.f;
    const int64_t bk = k0 + ty, bn = static_cast<int64_t>(blockIdx.x) * 16 + tx;
    Bs[ty][tx] = (bk < p.K && bn < p.N) ? Elem<InT>::load1(B + bk * p.sb_k + bn * p.sb_n) : 0.f;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; ++k) acc += As[ty][k] * Bs[k][tx];
    __syncthreads();
  }
  if (m < p.M && n < p.N) store_out<OutT>(static_cast<OutT*>(p.c) + bb * p.sc_b + m * p.sc_m + n, acc);
}

// ---------------------------------------------------------------------------
// Host dispatch.
// ---------------------------------------------------------------------------
static inline bool al16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

template <int BM, int BN, int WM, int WN, typename OutT>
static hipError_t launch_bf16(GemmParams p, bool a_k, bool b_k, hipStream_t s) {
  p.tiles_m = static_cast<int>((p.M + BM - 1) / BM);
  p.tiles_n = static_cast<int>((p.N + BN - 1) / BN);
  const int64_t blocks = p.batch * p.tiles_m * p.tiles_n;
  const dim3 grid(static_cast<unsigned>(blocks)), block(WM * WN * 64);
  if (a_k && b_k) hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WM, WN, true, true, OutT>), grid, block, 0, s, p);
  else if (a_k) hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WM, WN, true, false, OutT>), grid, block, 0, s, p);
  else if (b_k) hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WM, WN, false, true, OutT>), grid, block, 0, s, p);
  else hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WM, WN, false, false, OutT>), grid, block, 0, s, p);
  return hipGetLastError();
}

template <typename OutT>
static hipError_t launch_f32(GemmParams p, bool a_k, bool b_k, hipStream_t s) {
  p.tiles_m = static_cast<int>((p.M + 127) / 128);
  p.tiles_n = static_cast<int>((p.N + 127) / 128);
  const dim3 grid(static_cast<unsigned>(p.batch * p.tiles_m * p.tiles_n)), block(256);
  if (a_k && b_k) hipLaunchKernelGGL((gemm_f32_kernel<true, true, OutT>), grid, block, 0, s, p);
  else if (a_k) hipLaunchKernelGGL((gemm_f32_kernel<true, false, OutT>), grid, block, 0, s, p);
  else if (b_k) hipLaunchKernelGGL((gemm_f32_kernel<false, true, OutT>), grid, block, 0, s, p);
  else hipLaunchKernelGGL((gemm_f32_kernel<false, false, OutT>), grid, block, 0, s, p);
  return hipGetLastError();
}

template <typename InT, typename OutT>
static hipError_t launch_generic(const GemmParams& p, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((p.N + 15) / 16), static_cast<unsigned>((p.M + 15) / 16),
                  static_cast<unsigned>(p.batch));
  hipLaunchKernelGGL((gemm_generic_kernel<InT, OutT>), grid, dim3(256), 0, s, p);
  return hipGetLastError();
}

// Operand majorness for the vector paths: returns 1 for K-contiguous, 0 for
// MN-contiguous, -1 when neither vector layout can address the operand.
static int majorness(const void* base, int64_t s_b, int64_t s_mn, int64_t s_k, int64_t MN,
                     int64_t K, int vec, int64_t batch) {
  if (!al16(base)) return -1;
  const bool b_ok = batch == 1 || s_b % vec == 0;
  if (s_k == 1 && K % vec == 0 && (MN == 1 || s_mn % vec == 0) && b_ok) return 1;
  if (s_mn == 1 && MN % vec == 0 && (K == 1 || s_k % vec == 0) && b_ok) return 0;
  return -1;
}

// Bytes spanned by one batch slice of an operand with non-negative strides.
static int64_t slice_bytes(int64_t rows, int64_t s_row, int64_t K, int64_t s_k, int64_t es) {
  return ((rows - 1) * s_row + (K - 1) * s_k + 1) * es;
}

template <typename OutT>
static hipError_t dispatch_bf16(GemmParams p, hipStream_t s) {
  const int ma = majorness(p.a, p.sa_b, p.sa_m, p.sa_k, p.M, p.K, 8, p.batch);
  const int mb = majorness(p.b, p.sb_b, p.sb_n, p.sb_k, p.N, p.K, 8, p.batch);
  const bool nonneg = p.sa_b >= 0 && p.sa_m >= 0 && p.sa_k >= 0 && p.sb_b >= 0 && p.sb_k >= 0 &&
                      p.sb_n >= 0;
  const int64_t ea = slice_bytes(p.M, p.sa_m, p.K, p.sa_k, 2);
  const int64_t eb = slice_bytes(p.N, p.sb_n, p.K, p.sb_k, 2);
  if (ma < 0 || mb < 0 || !nonneg || ea >= (int64_t{1} << 31) || eb >= (int64_t{1} << 31))
    return launch_generic<bf16_t, OutT>(p, s);
  p.a_extent = static_cast<uint32_t>(ea);
  p.b_extent = static_cast<uint32_t>(eb);
  p.vec_c = (p.sc_m % 4 == 0) && (p.sc_b % 4 == 0 || p.batch == 1) &&
            (reinterpret_cast<uintptr_t>(p.c) % (4 * sizeof(OutT)) == 0);
  const int64_t t256 = p.batch * ((p.M + 255) / 256) * ((p.N + 255) / 256);
  if (p.M >= 256 && p.N >= 256 && t256 >= 128) return launch_bf16<256, 256, 2, 4, OutT>(p, ma, mb, s);
  if (p.M >= 256 && p.N >= 128) return launch_bf16<256, 128, 2, 2, OutT>(p, ma, mb, s);
  return launch_bf16<128, 128, 2, 2, OutT>(p, ma, mb, s);
}

template <typename OutT>
static hipError_t dispatch_f32(GemmParams p, hipStream_t s) {
  const int ma = majorness(p.a, p.sa_b, p.sa_m, p.sa_k, p.M, p.K, 4, p.batch);
  const int mb = majorness(p.b, p.sb_b, p.sb_n, p.sb_k, p.N, p.K, 4, p.batch);
  if (ma < 0 || mb < 0) return launch_generic<float, OutT>(p, s);
  return launch_f32<OutT>(p, ma, mb, s);
}

}  // namespace ghip

using namespace ghip;

extern "C" int ghip_gemm_batched(int ab_dtype, int c_dtype, int64_t batch, int64_t M, int64_t N,
                                 int64_t K, const void* a, int64_t sa_b, int64_t sa_m,
                                 int64_t sa_k, const void* b, int64_t sb_b, int64_t sb_k,
                                 int64_t sb_n, void* c, int64_t sc_b, int64_t sc_m, int64_t sc_n,
                                 void* stream, GHipError* err) {
  if (batch < 0 || M < 0 || N < 0 || K < 0)
    return set_error(err, GHIP_ERR_INVALID_ARG, "gemm_batched: negative size");
  if (sc_n != 1) return set_error(err, GHIP_ERR_INVALID_ARG, "gemm_batched: sc_n must be 1");
  if (batch == 0 || M == 0 || N == 0) return GHIP_OK;
  if (!c || (K > 0 && (!a || !b))) return set_error(err, GHIP_ERR_INVALID_ARG, "gemm_batched: null pointer");
  const int64_t tiles = batch * ((M + 127) / 128) * ((N + 127) / 128);
  if (tiles > 0x7fffffffLL || batch > 65535)
    return set_error(err, GHIP_ERR_INVALID_ARG, "gemm_batched: problem too large");
  GemmParams p{};
  p.a = a; p.b = b; p.c = c;
  p.sa_b = sa_b; p.sa_m = sa_m; p.sa_k = sa_k;
  p.sb_b = sb_b; p.sb_k = sb_k; p.sb_n = sb_n;
  p.sc_b = sc_b; p.sc_m = sc_m;
  p.batch = batch; p.M = M; p.N = N; p.K = K;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (ab_dtype == GHIP_DTYPE_BFLOAT16) {
    if (c_dtype == GHIP_DTYPE_BFLOAT16) e = dispatch_bf16<bf16_t>(p, s);
    else if (c_dtype == GHIP_DTYPE_FLOAT32) e = dispatch_bf16<float>(p, s);
    else return set_error(err, GHIP_ERR_UNSUPPORTED, "gemm_batched: output dtype %d", c_dtype);
  } else if (ab_dtype == GHIP_DTYPE_FLOAT32) {
    if (c_dtype == GHIP_DTYPE_FLOAT32) e = dispatch_f32<float>(p, s);
    else if (c_dtype == GHIP_DTYPE_BFLOAT16) e = dispatch_f32<bf16_t>(p, s);
    else return set_error(err, GHIP_ERR_UNSUPPORTED, "gemm_batched: output dtype %d", c_dtype);
  } else {
    return set_error(err, GHIP_ERR_UNSUPPORTED, "gemm_batched: input dtype %d", ab_dtype);
  }
  GHIP_CHECK(e, err);
  return GHIP_OK;
}
