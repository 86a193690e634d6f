// Batched GEMM for DotGeneral: c[b] = a[b] (M x K) * b[b] (K x N), fp32 accumulate.
//
// bf16 / f16 path (the MFMA path the metric is quoted on): the cores live in
// gemm_bf16_dev.h (shared with the Compile-time generated epilogue GEMMs); the
// kernels here instantiate them with a plain store epilogue.  Grids of more than
// 128 256 x 256 tiles run the 256 x 256 cores (A K- / B N-contiguous: the 4-wave
// 16x16x32 core; B K-contiguous: the 8-wave 64-deep 16x16x32 core; both
// MN-contiguous: the 4-wave 32-deep core); smaller grids the 4-wave 128 x 128
// 32x32x16 core, two workgroups per CU.
// fp32 path: v_mfma_f32_32x32x2f32 over LDS-DMA tiles (below).
// Anything the vector paths cannot address (odd strides, unaligned bases,
// negative strides, a row stride of 4M elements (bf16) / 2M (fp32) or more) runs
// a generic LDS-tiled kernel.  Operand slices may exceed 4 GiB: each tile's
// buffer descriptors are based at the tile (gemm_rows_fit, left_bytes).
#include "gemm_kernels.h"

namespace ghip {


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

template <int BM, int BN, int WM, int WN, typename InT, typename OutT>
static hipError_t launch_bf16(GemmParams p, bool a_k, bool b_k, hipStream_t s) {
  p.tiles_m = static_cast<int>((p.M + BM - 1) / BM);
  p.tiles_n = static_cast<int>((p.N + BN - 1) / BN);
  const int64_t blocks = p.batch * p.tiles_m * p.tiles_n;
  const dim3 grid(static_cast<unsigned>(blocks)), block(WM * WN * 64);
  if (a_k && b_k) hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WM, WN, true, true, InT, OutT>), grid, block, 0, s, p);
  else if (a_k) hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WM, WN, true, false, InT, OutT>), grid, block, 0, s, p);
  else if (b_k) hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WM, WN, false, true, InT, OutT>), grid, block, 0, s, p);
  else hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WM, WN, false, false, InT, OutT>), grid, block, 0, s, p);
  return hipGetLastError();
}



// Sum of the s fp32 partial products of a split contraction (gemm_k_split),
// ws[j][m][n] (dense [M, N] each), in split order j = 0, 1, .., s - 1, rounded
// once to the output c[m * sc_m + n].  V4: a thread takes 4 consecutive n of one
// row (N % 4 == 0: one 16-byte load per partial; vec_out: one store); else one
// element.
template <typename OutT, bool V4>
__global__ __launch_bounds__(256) void gemm_split_sum_kernel(const float* __restrict__ ws, OutT* __restrict__ c,
                                                             int64_t M, int64_t N, int64_t sc_m, int s, int vec_out) {
  const int64_t slice = M * N;
  constexpr int W = V4 ? 4 : 1;
  const int64_t nw = N / W;
  const int64_t groups = M * nw;
  for (int64_t g = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; g < groups;
       g += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t m = g / nw, n = (g % nw) * W;
    const float* src = ws + m * N + n;
    OutT* dst = c + m * sc_m + n;
    if constexpr (V4) {
      // Every partial's load is issued before the first add (one memory latency
      // per thread, not s); the adds then run in split order.
      float4 v[kGemmMaxSplit];
#pragma unroll
      for (int j = 0; j < kGemmMaxSplit; ++j)
        if (j < s) v[j] = *reinterpret_cast<const float4*>(src + j * slice);
      float4 acc = v[0];
#pragma unroll
      for (int j = 1; j < kGemmMaxSplit; ++j)
        if (j < s) {
          acc.x += v[j].x;
          acc.y += v[j].y;
          acc.z += v[j].z;
          acc.w += v[j].w;
        }
      if (vec_out) {
        if constexpr (__is_same(OutT, float)) {
          *reinterpret_cast<float4*>(dst) = acc;
        } else if constexpr (__is_same(OutT, bf16_t)) {
          *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(acc.x, acc.y), pack_bf16x2(acc.z, acc.w));
        } else {
          *reinterpret_cast<uint2*>(dst) = make_uint2(pack_f16x2(acc.x, acc.y), pack_f16x2(acc.z, acc.w));
        }
      } else {
        store_out<OutT>(dst, acc.x);
        store_out<OutT>(dst + 1, acc.y);
        store_out<OutT>(dst + 2, acc.z);
        store_out<OutT>(dst + 3, acc.w);
      }
    } else {
      float acc = src[0];
      for (int j = 1; j < s; ++j) acc += src[j * slice];
      store_out<OutT>(dst, acc);
    }
  }
}

// The same core for a K-contiguous A only (the two B layouts): tiles of 32 rows,
// whose A tile is too short for the MN-contiguous DMA pattern.
template <int BM, int BN, int WM, int WN, typename InT, typename OutT>
static hipError_t launch_bf16_ak(GemmParams p, bool b_k, hipStream_t s) {
  p.tiles_m = static_cast<int>((p.M + BM - 1) / BM);
  p.tiles_n = static_cast<int>((p.N + BN - 1) / BN);
  const int64_t blocks = p.batch * p.tiles_m * p.tiles_n;
  const dim3 grid(static_cast<unsigned>(blocks)), block(WM * WN * 64);
  if (b_k) hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WM, WN, true, true, InT, OutT>), grid, block, 0, s, p);
  else hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WM, WN, true, false, InT, OutT>), grid, block, 0, s, p);
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

// Workspace of a split contraction (16-byte aligned, large enough: checked by the
// entry points); ptr null: no split.
struct GemmWs {
  float* ptr = nullptr;
  int64_t bytes = 0;
};

// A split contraction (gemm_k_split): the s ranges of kc steps run as s "batches"
// of the 128 x 128 core (16-bit operands: the 32x32x16 core; fp32: the fp32 MFMA
// core; range j: a + j kc sa_k, b + j kc sb_k) writing fp32 partials into the
// workspace, then gemm_split_sum_kernel adds them in range order.
template <typename InT>
static hipError_t launch_split_partials(const GemmParams& p, int ma, int mb, const GemmSplit& sp, float* ws,
                                        hipStream_t s) {
  constexpr int64_t es = sizeof(InT);
  GemmParams q = p;
  q.batch = sp.s;
  q.K = sp.kc;
  q.sa_b = sp.kc * p.sa_k;
  q.sb_b = sp.kc * p.sb_k;
  q.c = ws;
  q.sc_b = p.M * p.N;
  q.sc_m = p.N;
  const int64_t ea = slice_bytes(p.M, p.sa_m, sp.kc, p.sa_k, es);
  const int64_t eb = slice_bytes(p.N, p.sb_n, sp.kc, p.sb_k, es);
  q.a_extent = static_cast<uint32_t>(ea);
  q.b_extent = static_cast<uint32_t>(eb);
  q.a_extent64 = ea;
  q.b_extent64 = eb;
  q.vec_c = p.N % 4 == 0;
  if constexpr (es == 4) {
    // At most 32 rows: 32 x 128 fp32 tiles (four waves of 32 x 32), a quarter of
    // the 128-row tile's MFMA work, which the slow fp32 MFMAs feel.  Same MFMA and k
    // order per accumulator: the same bits.
    if (p.M <= 32) return launch_f32<32, 128, 1, 4, float>(q, ma == 1, mb == 1, s);
    return launch_f32<128, 128, 2, 2, float>(q, ma == 1, mb == 1, s);
  } else {
    // At most 32 rows (decoding) and A K-contiguous: 32 x 128 tiles (four waves of
    // 32 x 32), a quarter of the 128-row tile's wasted MFMA work and LDS, more
    // workgroups resident per CU: 4-13% faster at [16, 1024..14336, 4096..14336]
    // (graph-replayed A/B).  Same MFMA and k order per accumulator: the same bits.
    if (p.M <= 32 && ma == 1) return launch_bf16_ak<32, 128, 1, 4, InT, float>(q, mb == 1, s);
    return launch_bf16<128, 128, 2, 2, InT, float>(q, ma == 1, mb == 1, s);
  }
}

template <typename InT, typename OutT>
static hipError_t launch_split(const GemmParams& p, int ma, int mb, const GemmSplit& sp, float* ws, hipStream_t s) {
  const hipError_t e = launch_split_partials<InT>(p, ma, mb, sp, ws, s);
  if (e != hipSuccess) return e;
  const bool v4 = p.N % 4 == 0;
  const int64_t groups = p.M * (v4 ? p.N / 4 : p.N);
  const int64_t blocks = (groups + 255) / 256 < 4096 ? (groups + 255) / 256 : 4096;
  const int vec_out = p.sc_m % 4 == 0 && reinterpret_cast<uintptr_t>(p.c) % (4 * sizeof(OutT)) == 0;
  OutT* c = static_cast<OutT*>(p.c);
  if (v4)
    hipLaunchKernelGGL((gemm_split_sum_kernel<OutT, true>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, ws,
                       c, p.M, p.N, p.sc_m, sp.s, vec_out);
  else
    hipLaunchKernelGGL((gemm_split_sum_kernel<OutT, false>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, ws,
                       c, p.M, p.N, p.sc_m, sp.s, vec_out);
  return hipGetLastError();
}

template <typename InT, typename OutT>
static hipError_t dispatch_bf16(GemmParams p, hipStream_t s, GemmWs ws = {}) {
  const int ma = majorness(p.a, p.sa_b, p.sa_m, p.sa_k, p.M, p.K, 8, p.batch);
  const int mb = majorness(p.b, p.sb_b, p.sb_n, p.sb_k, p.N, p.K, 8, p.batch);
  const bool nonneg = p.sa_b >= 0 && p.sa_m >= 0 && p.sa_k >= 0 && p.sb_b >= 0 && p.sb_k >= 0 &&
                      p.sb_n >= 0;
  const int64_t ea = slice_bytes(p.M, p.sa_m, p.K, p.sa_k, 2);
  const int64_t eb = slice_bytes(p.N, p.sb_n, p.K, p.sb_k, 2);
  const int64_t t256 = p.batch * ((p.M + 255) / 256) * ((p.N + 255) / 256);
  // Slices of 2 GiB or more: the 256 x 256 cores' 64-bit-records forms.
  const bool big = ea >= (int64_t{1} << 31) || eb >= (int64_t{1} << 31);
  const bool big_ok = p.M >= 256 && p.N >= 256 && t256 >= 128;
  if (ma < 0 || mb < 0 || !nonneg || !gemm_rows_fit(p.sa_m, p.sa_k, 2) || !gemm_rows_fit(p.sb_n, p.sb_k, 2) ||
      (big && !big_ok))
    return launch_generic<InT, OutT>(p, s);
  p.a_extent = big ? 0u : static_cast<uint32_t>(ea);
  p.b_extent = big ? 0u : static_cast<uint32_t>(eb);
  p.a_extent64 = ea;
  p.b_extent64 = eb;
  constexpr int64_t kV = 16 / sizeof(OutT);  // elements per 16-byte store
  p.vec_c = (p.sc_m % kV == 0) && (p.sc_b % kV == 0 || p.batch == 1) &&
            (reinterpret_cast<uintptr_t>(p.c) % 16 == 0);
  if (big) return launch_bf16_4w<true, InT, OutT>(p, ma, mb, s);
  // Few tiles and a long contraction, with a workspace: the contraction split.
  if (ws.ptr) {
    const GemmSplit sp = gemm_k_split(p.batch, p.M, p.N, p.K, 2);
    if (sp.s > 1 && gemm_split_bytes(sp, p.M, p.N) <= ws.bytes) return launch_split<InT, OutT>(p, ma, mb, sp, ws.ptr, s);
  }
  // Grids of more than 128 256 x 256 tiles: the 256 x 256 cores (one workgroup per
  // CU).  Up to 128 such tiles they would leave half the 256 CUs or more idle, and
  // the 128 x 128 core (two workgroups per CU, so up to 512 tiles in one round) is
  // faster in every layout: 11-33% at 128 tiles ([2048,4096,4096], [8192,1024,2048]),
  // 12-43% against the 256 x 128 core below that (A/B, one box).  All cores give
  // the same bits.
  if (p.M >= 256 && p.N >= 256 && t256 > 128) return launch_bf16_4w<false, InT, OutT>(p, ma, mb, s);
  return launch_bf16<128, 128, 2, 2, InT, OutT>(p, ma, mb, s);
}

// G products A.B_g -> C_g sharing A (same sizes and strides): one launch of G x
// tiles workgroups on the 4-wave core when A is K-contiguous and every B_g is
// MN-contiguous (the layouts of x . W); otherwise one dispatch per product.  Each
// product's result is the one the stand-alone dispatch would give (the same core
// and k order).
template <typename InT, typename OutT>
static hipError_t dispatch_grouped(GemmParams p, int G, const void* const* b, void* const* c, hipStream_t s,
                                   GemmWs ws = {}) {
  bool ok = majorness(p.a, 0, p.sa_m, p.sa_k, p.M, p.K, 8, 1) == 1 && p.sa_m >= 0 && p.sa_k >= 0 &&
            p.sb_k >= 0 && p.sb_n >= 0;
  for (int g = 0; g < G && ok; ++g) ok = majorness(b[g], 0, p.sb_n, p.sb_k, p.N, p.K, 8, 1) == 0;
  const int64_t ea = slice_bytes(p.M, p.sa_m, p.K, p.sa_k, 2);
  const int64_t eb = slice_bytes(p.N, p.sb_n, p.K, p.sb_k, 2);
  const int64_t tiles = ((p.M + 255) / 256) * ((p.N + 255) / 256);
  ok = ok && ea < (int64_t{1} << 31) && eb < (int64_t{1} << 31) && p.M >= 256 && p.N >= 256 && G * tiles >= 128;
  // Products the stand-alone entry splits (given the workspace) run as that split,
  // one after another in the same workspace, so each keeps the stand-alone bits.
  if (ws.ptr && gemm_k_split(1, p.M, p.N, p.K, 2).s > 1) ok = false;
  if (!ok) {
    for (int g = 0; g < G; ++g) {
      GemmParams q = p;
      q.batch = 1;
      q.b = b[g];
      q.c = c[g];
      const hipError_t e = dispatch_bf16<InT, OutT>(q, s, ws);
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
  p.a_extent = static_cast<uint32_t>(ea);
  p.b_extent = static_cast<uint32_t>(eb);
  constexpr int64_t kV = 16 / sizeof(OutT);
  p.vec_c = p.sc_m % kV == 0;
  for (int g = 0; g < G; ++g) p.vec_c = p.vec_c && reinterpret_cast<uintptr_t>(c[g]) % 16 == 0;
  p.batch = G;
  p.sa_b = p.sb_b = p.sc_b = 0;
  p.groups = G;
  for (int g = 0; g < kGemmMaxGroups; ++g) {
    p.b_g[g] = b[g < G ? g : 0];
    p.c_g[g] = c[g < G ? g : 0];
  }
  p.b = b[0];
  p.c = c[0];
  p.tiles_m = static_cast<int>((p.M + 255) / 256);
  p.tiles_n = static_cast<int>((p.N + 255) / 256);
  hipLaunchKernelGGL((gemm_bf16_kernel4km_grouped<InT, OutT>), dim3(static_cast<unsigned>(G * tiles)), dim3(256), 0,
                     s, p);
  return hipGetLastError();
}

template <typename OutT>
static hipError_t dispatch_f32(GemmParams p, hipStream_t s, GemmWs ws = {}) {
  const int ma = majorness(p.a, p.sa_b, p.sa_m, p.sa_k, p.M, p.K, 4, p.batch);
  const int mb = majorness(p.b, p.sb_b, p.sb_n, p.sb_k, p.N, p.K, 4, p.batch);
  const bool nonneg = p.sa_b >= 0 && p.sa_m >= 0 && p.sa_k >= 0 && p.sb_b >= 0 && p.sb_k >= 0 &&
                      p.sb_n >= 0;
  const int64_t ea = slice_bytes(p.M, p.sa_m, p.K, p.sa_k, 4);
  const int64_t eb = slice_bytes(p.N, p.sb_n, p.K, p.sb_k, 4);
  const int64_t t256 = p.batch * ((p.M + 255) / 256) * ((p.N + 255) / 256);
  const bool grid256 = p.M >= 256 && p.N >= 256 && t256 >= 128;
  const bool big = ea >= (int64_t{1} << 31) || eb >= (int64_t{1} << 31);
  if (ma < 0 || mb < 0 || !nonneg || !gemm_rows_fit(p.sa_m, p.sa_k, 4) || !gemm_rows_fit(p.sb_n, p.sb_k, 4) ||
      (big && !grid256))
    return launch_generic<float, OutT>(p, s);
  p.a_extent = big ? 0u : static_cast<uint32_t>(ea);
  p.b_extent = big ? 0u : static_cast<uint32_t>(eb);
  p.a_extent64 = ea;
  p.b_extent64 = eb;
  p.vec_c = (p.sc_m % 4 == 0) && (p.sc_b % 4 == 0 || p.batch == 1) &&
            (reinterpret_cast<uintptr_t>(p.c) % (4 * sizeof(OutT)) == 0);
  if (big) return launch_f32<256, 256, 2, 4, OutT, true>(p, ma, mb, s);
  // Few tiles and a long contraction, with a workspace: the contraction split.
  if (ws.ptr) {
    const GemmSplit sp = gemm_k_split(p.batch, p.M, p.N, p.K, 4);
    if (sp.s > 1 && gemm_split_bytes(sp, p.M, p.N) <= ws.bytes) return launch_split<float, OutT>(p, ma, mb, sp, ws.ptr, s);
  }
  // The 8-wave 256 x 256 fp32 core only from one full round of its tiles: below
  // that the 4-wave 128 x 128 core (two workgroups per CU) is faster, 1.9x at 128
  // tiles of 256 x 256 ([2048,4096,4096]), 1.3x at 144 and 192, even at 256.
  if (p.M >= 256 && p.N >= 256 && t256 >= 256) return launch_f32<256, 256, 2, 4, OutT>(p, ma, mb, s);
  return launch_f32<128, 128, 2, 2, OutT>(p, ma, mb, s);
}

int gemm_split_partials(int ab_dtype, int64_t M, int64_t N, int64_t K, const void* a, int64_t sa_m, int64_t sa_k,
                        const void* b, int64_t sb_k, int64_t sb_n, float* ws, int64_t ws_bytes, int s, void* stream,
                        GHipError* err) {
  if (ab_dtype != GHIP_DTYPE_BFLOAT16 && ab_dtype != GHIP_DTYPE_FLOAT16)
    return set_error(err, GHIP_ERR_INVALID_ARG, "gemm_split_partials: 16-bit operands only");
  if (M <= 0 || N <= 0 || K <= 0 || !a || !b || !ws)
    return set_error(err, GHIP_ERR_INVALID_ARG, "gemm_split_partials: empty product or null pointer");
  GemmParams p{};
  p.a = a;
  p.b = b;
  p.sa_m = sa_m; p.sa_k = sa_k;
  p.sb_k = sb_k; p.sb_n = sb_n;
  p.batch = 1; p.M = M; p.N = N; p.K = K;
  const int ma = majorness(a, 0, sa_m, sa_k, M, K, 8, 1);
  const int mb = majorness(b, 0, sb_n, sb_k, N, K, 8, 1);
  const bool ok = ma >= 0 && mb >= 0 && sa_m >= 0 && sa_k >= 0 && sb_k >= 0 && sb_n >= 0 &&
                  gemm_rows_fit(sa_m, sa_k, 2) && gemm_rows_fit(sb_n, sb_k, 2) &&
                  slice_bytes(M, sa_m, K, sa_k, 2) < (int64_t{1} << 31) && slice_bytes(N, sb_n, K, sb_k, 2) < (int64_t{1} << 31);
  const GemmSplit sp = gemm_k_split(1, M, N, K, 2);
  if (!ok || sp.s != s)
    return set_error(err, GHIP_ERR_STATE, "gemm_split_partials: the product does not take a %d-range split", s);
  if (ws_bytes < gemm_split_bytes(sp, M, N) || reinterpret_cast<uintptr_t>(ws) % 16 != 0)
    return set_error(err, GHIP_ERR_INVALID_ARG, "gemm_split_partials: workspace too small or misaligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const hipError_t e = ab_dtype == GHIP_DTYPE_BFLOAT16 ? launch_split_partials<bf16_t>(p, ma, mb, sp, ws, st)
                                                       : launch_split_partials<f16_t>(p, ma, mb, sp, ws, st);
  GHIP_CHECK(e, err);
  return GHIP_OK;
}

}  // namespace ghip

using namespace ghip;

// Workspace bytes a split of this product needs (0: never split): 16-bit operands
// only.
static int64_t split_ws_bytes(int ab_dtype, int64_t batch, int64_t M, int64_t N, int64_t K) {
  const int es = ab_dtype == GHIP_DTYPE_FLOAT32 ? 4
                 : (ab_dtype == GHIP_DTYPE_BFLOAT16 || ab_dtype == GHIP_DTYPE_FLOAT16) ? 2 : 0;
  if (es == 0) return 0;
  return gemm_split_bytes(gemm_k_split(batch, M, N, K, es), M, N);
}

// A workspace given for a product that splits must hold the split's partials and
// be 16-byte aligned.
static int check_split_ws(const char* who, int64_t need, const void* workspace, int64_t workspace_bytes,
                          GHipError* err) {
  if (!workspace || need == 0) return GHIP_OK;
  if (workspace_bytes < need)
    return set_error(err, GHIP_ERR_INVALID_ARG, "%s: workspace of %lld bytes, %lld needed", who,
                     static_cast<long long>(workspace_bytes), static_cast<long long>(need));
  if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0)
    return set_error(err, GHIP_ERR_INVALID_ARG, "%s: workspace must be 16-byte aligned", who);
  return GHIP_OK;
}

extern "C" int64_t ghip_gemm_workspace_bytes(int ab_dtype, int c_dtype, int64_t batch, int64_t M, int64_t N,
                                             int64_t K) {
  (void)c_dtype;
  if (batch < 0 || M < 0 || N < 0 || K < 0) return 0;
  return split_ws_bytes(ab_dtype, batch, M, N, K);
}

extern "C" int ghip_gemm_batched(int ab_dtype, int c_dtype, int64_t batch, int64_t M, int64_t N,
                                 int64_t K, const void* a, int64_t sa_b, int64_t sa_m,
                                 int64_t sa_k, const void* b, int64_t sb_b, int64_t sb_k,
                                 int64_t sb_n, void* c, int64_t sc_b, int64_t sc_m, int64_t sc_n,
                                 void* stream, GHipError* err) {
  return ghip_gemm_batched_ws(ab_dtype, c_dtype, batch, M, N, K, a, sa_b, sa_m, sa_k, b, sb_b, sb_k, sb_n, c, sc_b,
                              sc_m, sc_n, nullptr, 0, stream, err);
}

extern "C" int ghip_gemm_batched_ws(int ab_dtype, int c_dtype, int64_t batch, int64_t M, int64_t N,
                                    int64_t K, const void* a, int64_t sa_b, int64_t sa_m,
                                    int64_t sa_k, const void* b, int64_t sb_b, int64_t sb_k,
                                    int64_t sb_n, void* c, int64_t sc_b, int64_t sc_m, int64_t sc_n,
                                    void* workspace, int64_t workspace_bytes, void* stream, GHipError* err) {
  if (batch < 0 || M < 0 || N < 0 || K < 0)
    return set_error(err, GHIP_ERR_INVALID_ARG, "gemm_batched: negative size");
  if (sc_n != 1) return set_error(err, GHIP_ERR_INVALID_ARG, "gemm_batched: sc_n must be 1");
  if (batch == 0 || M == 0 || N == 0) return GHIP_OK;
  if (!c || (K > 0 && (!a || !b))) return set_error(err, GHIP_ERR_INVALID_ARG, "gemm_batched: null pointer");
  const int64_t tiles = batch * ((M + 127) / 128) * ((N + 127) / 128);
  if (tiles > 0x7fffffffLL || batch > 65535)
    return set_error(err, GHIP_ERR_INVALID_ARG, "gemm_batched: problem too large");
  const int rc = check_split_ws("gemm_batched", split_ws_bytes(ab_dtype, batch, M, N, K), workspace, workspace_bytes, err);
  if (rc != GHIP_OK) return rc;
  GemmWs ws;
  ws.ptr = static_cast<float*>(workspace);
  ws.bytes = workspace ? workspace_bytes : 0;
  GemmParams p{};
  p.a = a; p.b = b; p.c = c;
  p.sa_b = sa_b; p.sa_m = sa_m; p.sa_k = sa_k;
  p.sb_b = sb_b; p.sb_k = sb_k; p.sb_n = sb_n;
  p.sc_b = sc_b; p.sc_m = sc_m;
  p.batch = batch; p.M = M; p.N = N; p.K = K;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (ab_dtype == GHIP_DTYPE_BFLOAT16) {
    if (c_dtype == GHIP_DTYPE_BFLOAT16) e = dispatch_bf16<bf16_t, bf16_t>(p, s, ws);
    else if (c_dtype == GHIP_DTYPE_FLOAT32) e = dispatch_bf16<bf16_t, float>(p, s, ws);
    else return set_error(err, GHIP_ERR_UNSUPPORTED, "gemm_batched: output dtype %d", c_dtype);
  } else if (ab_dtype == GHIP_DTYPE_FLOAT16) {
    if (c_dtype == GHIP_DTYPE_FLOAT16) e = dispatch_bf16<f16_t, f16_t>(p, s, ws);
    else if (c_dtype == GHIP_DTYPE_FLOAT32) e = dispatch_bf16<f16_t, float>(p, s, ws);
    else return set_error(err, GHIP_ERR_UNSUPPORTED, "gemm_batched: output dtype %d", c_dtype);
  } else if (ab_dtype == GHIP_DTYPE_FLOAT32) {
    if (c_dtype == GHIP_DTYPE_FLOAT32) e = dispatch_f32<float>(p, s, ws);
    else if (c_dtype == GHIP_DTYPE_BFLOAT16) e = dispatch_f32<bf16_t>(p, s, ws);
    else return set_error(err, GHIP_ERR_UNSUPPORTED, "gemm_batched: output dtype %d", c_dtype);
  } else {
    return set_error(err, GHIP_ERR_UNSUPPORTED, "gemm_batched: input dtype %d", ab_dtype);
  }
  GHIP_CHECK(e, err);
  return GHIP_OK;
}

extern "C" int ghip_gemm_grouped(int ab_dtype, int c_dtype, int groups, int64_t M, int64_t N, int64_t K,
                                 const void* a, int64_t sa_m, int64_t sa_k, const void* const* b, int64_t sb_k,
                                 int64_t sb_n, void* const* c, int64_t sc_m, void* stream, GHipError* err) {
  return ghip_gemm_grouped_ws(ab_dtype, c_dtype, groups, M, N, K, a, sa_m, sa_k, b, sb_k, sb_n, c, sc_m, nullptr, 0,
                              stream, err);
}

extern "C" int ghip_gemm_grouped_ws(int ab_dtype, int c_dtype, int groups, int64_t M, int64_t N, int64_t K,
                                    const void* a, int64_t sa_m, int64_t sa_k, const void* const* b, int64_t sb_k,
                                    int64_t sb_n, void* const* c, int64_t sc_m, void* workspace,
                                    int64_t workspace_bytes, void* stream, GHipError* err) {
  if (groups < 1 || groups > kGemmMaxGroups)
    return set_error(err, GHIP_ERR_INVALID_ARG, "gemm_grouped: groups must be 1..%d", kGemmMaxGroups);
  if (M < 0 || N < 0 || K < 0) return set_error(err, GHIP_ERR_INVALID_ARG, "gemm_grouped: negative size");
  if (M == 0 || N == 0) return GHIP_OK;
  if (!b || !c) return set_error(err, GHIP_ERR_INVALID_ARG, "gemm_grouped: null pointer array");
  for (int g = 0; g < groups; ++g)
    if (!c[g] || (K > 0 && (!a || !b[g]))) return set_error(err, GHIP_ERR_INVALID_ARG, "gemm_grouped: null pointer");
  const bool in16 = ab_dtype == GHIP_DTYPE_BFLOAT16 || ab_dtype == GHIP_DTYPE_FLOAT16;
  if (!in16 || K == 0 || (c_dtype != ab_dtype && c_dtype != GHIP_DTYPE_FLOAT32)) {
    // fp32 operands, an empty contraction or an output dtype the batched entry
    // rejects: product by product.
    for (int g = 0; g < groups; ++g) {
      const int rc = ghip_gemm_batched_ws(ab_dtype, c_dtype, 1, M, N, K, a, 0, sa_m, sa_k, b[g], 0, sb_k, sb_n, c[g],
                                          0, sc_m, 1, workspace, workspace_bytes, stream, err);
      if (rc != GHIP_OK) return rc;
    }
    return GHIP_OK;
  }
  if (((M + 127) / 128) * ((N + 127) / 128) > 0x7fffffffLL / groups)
    return set_error(err, GHIP_ERR_INVALID_ARG, "gemm_grouped: problem too large");
  const int rc = check_split_ws("gemm_grouped", split_ws_bytes(ab_dtype, 1, M, N, K), workspace, workspace_bytes, err);
  if (rc != GHIP_OK) return rc;
  GemmWs ws;
  ws.ptr = static_cast<float*>(workspace);
  ws.bytes = workspace ? workspace_bytes : 0;
  GemmParams p{};
  p.a = a;
  p.sa_m = sa_m; p.sa_k = sa_k;
  p.sb_k = sb_k; p.sb_n = sb_n;
  p.sc_m = sc_m;
  p.batch = 1; p.M = M; p.N = N; p.K = K;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (ab_dtype == GHIP_DTYPE_BFLOAT16)
    e = c_dtype == GHIP_DTYPE_FLOAT32 ? dispatch_grouped<bf16_t, float>(p, groups, b, c, s, ws)
                                      : dispatch_grouped<bf16_t, bf16_t>(p, groups, b, c, s, ws);
  else
    e = c_dtype == GHIP_DTYPE_FLOAT32 ? dispatch_grouped<f16_t, float>(p, groups, b, c, s, ws)
                                      : dispatch_grouped<f16_t, f16_t>(p, groups, b, c, s, ws);
  GHIP_CHECK(e, err);
  return GHIP_OK;
}
