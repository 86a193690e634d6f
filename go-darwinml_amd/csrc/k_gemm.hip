// Batched GEMM for DotGeneral: c[b] = a[b] (M x K) * b[b] (K x N), fp32 accumulate.
//
// bf16 path (the MFMA path the metric is quoted on):
//   * v_mfma_f32_32x32x16_bf16 (gfx950): every lane feeds 8 consecutive-k bf16 of
//     one row (A) / one column (B), so both operand tiles live in LDS K-major:
//     tile[row][64 k] with the 16-byte chunk index XOR-swizzled by (row & 7); a
//     fragment read is one ds_read_b128 per lane and 8 consecutive lanes hit 8
//     different chunks (no bank conflicts).
//   * K-contiguous operands are copied to LDS with 16-byte loads/stores.
//     MN-contiguous operands (e.g. rhs [K, N] row-major, the DotGeneral config)
//     are loaded as 4(k) x 8(mn) blocks with 16-byte loads and transposed in
//     registers (byte permutes) into four-k 8-byte LDS stores — no transpose pass
//     over HBM, unlike the reference's two materialized rhs transposes
//     (dotgeneral.go:116-145).
//   * Two LDS stages: the global loads of k-tile t+1 are in flight while the MFMAs
//     of tile t run; one barrier per k-tile.
//   * Workgroup -> tile mapping is XCD-aware: consecutive workgroup ids land on
//     different XCDs (round robin), so ids are remapped to give each XCD a
//     contiguous run of tiles, ordered in GROUP_M-row groups for L2 reuse.
// fp32 path: v_mfma_f32_32x32x2f32 with MN-major LDS tiles (one float per lane).
// Anything the vector paths cannot address (odd strides, unaligned bases) runs a
// generic LDS-tiled kernel.
#include "common.h"

namespace ghip {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

struct GemmParams {
  const void* a;
  const void* b;
  void* c;
  int64_t sa_b, sa_m, sa_k;
  int64_t sb_b, sb_k, sb_n;
  int64_t sc_b, sc_m;
  int64_t batch, M, N, K;
  int tiles_m, tiles_n;
};

template <typename OutT>
__device__ __forceinline__ void store_out(OutT* p, float v);
template <>
__device__ __forceinline__ void store_out<float>(float* p, float v) { *p = v; }
template <>
__device__ __forceinline__ void store_out<bf16_t>(bf16_t* p, float v) { p->bits = f32_to_bf16(v); }

// Maps a linear workgroup id to (batch, tile_m, tile_n).
__device__ __forceinline__ void map_tile(int64_t bid, int64_t total, int tiles_m, int tiles_n,
                                         int64_t& bb, int& tm, int& tn) {
  constexpr int kXcd = 8;
  constexpr int kGroupM = 8;
  if (total % kXcd == 0) bid = (bid % kXcd) * (total / kXcd) + bid / kXcd;
  const int64_t per_batch = static_cast<int64_t>(tiles_m) * tiles_n;
  bb = bid / per_batch;
  const int t = static_cast<int>(bid % per_batch);
  const int group = t / (kGroupM * tiles_n);
  const int first_m = group * kGroupM;
  const int gsize = min(tiles_m - first_m, kGroupM);
  const int in_group = t % (kGroupM * tiles_n);
  tm = first_m + in_group % gsize;
  tn = in_group / gsize;
}

// ---------------------------------------------------------------------------
// bf16 operand tile loader: R rows (m or n) x 64 k, LDS layout [R][64] K-major,
// 16-byte chunks swizzled by (row & 7).
// ---------------------------------------------------------------------------
constexpr int kBK = 64;

__device__ __forceinline__ int swz(int row, int chunk) { return (chunk ^ (row & 7)); }

template <int R, int T, bool KCONTIG>
struct TileLoader {
  // K-contiguous: R*8 chunks of 16 B.  MN-contiguous: (64/4)*(R/8) blocks of
  // 4 k-rows x 8 mn (four 16 B loads each).
  static constexpr int kUnits = KCONTIG ? R * 8 : (kBK / 4) * (R / 8);
  static constexpr int kPer = (kUnits + T - 1) / T;
  static constexpr int kRegs = KCONTIG ? kPer : kPer * 4;
  uint4 r[kRegs];

  // base: operand pointer at (row0, k0) of this tile for batch bb.
  // s_row / s_k: element strides; rows_left / k_left: valid extent from (row0,k0).
  __device__ __forceinline__ void load(const uint16_t* base, int64_t s_row, int64_t s_k,
                                       int64_t rows_left, int64_t k_left, int tid) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int u = tid + i * T;
      if constexpr (KCONTIG) {
        const int row = u >> 3, kc = u & 7;
        const bool ok = (u < kUnits) && row < rows_left && kc * 8 < k_left;
        r[i] = ok ? *reinterpret_cast<const uint4*>(base + row * s_row + kc * 8)
                  : make_uint4(0, 0, 0, 0);
      } else {
        const int rg = u % (R / 8), kg = u / (R / 8);
        const bool rok = (u < kUnits) && rg * 8 < rows_left;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int k = kg * 4 + j;
          const bool ok = rok && k < k_left;
          r[i * 4 + j] = ok ? *reinterpret_cast<const uint4*>(base + k * s_k + rg * 8)
                            : make_uint4(0, 0, 0, 0);
        }
      }
    }
  }

  __device__ __forceinline__ void store(uint16_t* lds, int tid) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int u = tid + i * T;
      if (u >= kUnits) continue;
      if constexpr (KCONTIG) {
        const int row = u >> 3, kc = u & 7;
        *reinterpret_cast<uint4*>(lds + row * kBK + swz(row, kc) * 8) = r[i];
      } else {
        const int rg = u % (R / 8), kg = u / (R / 8);
        const uint32_t w0[4] = {r[i * 4 + 0].x, r[i * 4 + 0].y, r[i * 4 + 0].z, r[i * 4 + 0].w};
        const uint32_t w1[4] = {r[i * 4 + 1].x, r[i * 4 + 1].y, r[i * 4 + 1].z, r[i * 4 + 1].w};
        const uint32_t w2[4] = {r[i * 4 + 2].x, r[i * 4 + 2].y, r[i * 4 + 2].z, r[i * 4 + 2].w};
        const uint32_t w3[4] = {r[i * 4 + 3].x, r[i * 4 + 3].y, r[i * 4 + 3].z, r[i * 4 + 3].w};
        const int kc = kg >> 1, half = kg & 1;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          // Column e of the 4x8 block: k = kg*4 .. kg*4+3 of row rg*8+e.
          const int d = e >> 1;
          uint32_t lo, hi;
          if (e & 1) {
            lo = (w0[d] >> 16) | (w1[d] & 0xffff0000u);
            hi = (w2[d] >> 16) | (w3[d] & 0xffff0000u);
          } else {
            lo = (w0[d] & 0xffffu) | (w1[d] << 16);
            hi = (w2[d] & 0xffffu) | (w3[d] << 16);
          }
          const int row = rg * 8 + e;
          *reinterpret_cast<uint2*>(lds + row * kBK + swz(row, kc) * 8 + half * 4) =
              make_uint2(lo, hi);
        }
      }
    }
  }
};

template <int BM, int BN, int WM, int WN, bool A_K, bool B_K, typename OutT>
__global__ __launch_bounds__(WM * WN * 64) void gemm_bf16_kernel(GemmParams p) {
  constexpr int T = WM * WN * 64;
  constexpr int TM = BM / WM, TN = BN / WN;  // wave tile
  constexpr int FM = TM / 32, FN = TN / 32;  // 32x32 MFMA blocks per wave
  static_assert(FM >= 1 && FN >= 1, "wave tile too small");
  __shared__ __attribute__((aligned(16))) uint16_t lds[2][(BM + BN) * kBK];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  int64_t bb;
  int tm, tn;
  const int64_t total = p.batch * p.tiles_m * p.tiles_n;
  map_tile(blockIdx.x, total, p.tiles_m, p.tiles_n, bb, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;

  const uint16_t* A = static_cast<const uint16_t*>(p.a) + bb * p.sa_b + m0 * p.sa_m;
  const uint16_t* B = static_cast<const uint16_t*>(p.b) + bb * p.sb_b + n0 * p.sb_n;
  const int64_t s_am = p.sa_m, s_ak = p.sa_k;
  const int64_t rows_a = p.M - m0, rows_b = p.N - n0;

  TileLoader<BM, T, A_K> la;
  TileLoader<BN, T, B_K> lb;

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int KT = static_cast<int>((p.K + kBK - 1) / kBK);
  la.load(A, s_am, s_ak, rows_a, p.K, tid);
  lb.load(B, p.sb_n, p.sb_k, rows_b, p.K, tid);
  la.store(lds[0], tid);
  lb.store(lds[0] + BM * kBK, tid);
  __syncthreads();

  const int frow = lane & 31;  // row (A) / column (B) inside a 32-block
  const int kgrp = lane >> 5;  // which 8-k half of a 16-k MFMA step

  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < KT;
    if (more) {
      const int64_t k0 = static_cast<int64_t>(kt + 1) * kBK;
      la.load(A + k0 * s_ak, s_am, s_ak, rows_a, p.K - k0, tid);
      lb.load(B + k0 * p.sb_k, p.sb_n, p.sb_k, rows_b, p.K - k0, tid);
    }
    const uint16_t* As = lds[cur];
    const uint16_t* Bs = lds[cur] + BM * kBK;
#pragma unroll
    for (int s = 0; s < kBK / 16; ++s) {
      const int kc = s * 2 + kgrp;
      bf16x8_t af[FM], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int row = wm * TM + i * 32 + frow;
        uint4 v = *reinterpret_cast<const uint4*>(As + row * kBK + swz(row, kc) * 8);
        af[i] = __builtin_bit_cast(bf16x8_t, v);
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int row = wn * TN + j * 32 + frow;
        uint4 v = *reinterpret_cast<const uint4*>(Bs + row * kBK + swz(row, kc) * 8);
        bfr[j] = __builtin_bit_cast(bf16x8_t, v);
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (more) {
      la.store(lds[cur ^ 1], tid);
      lb.store(lds[cur ^ 1] + BM * kBK, tid);
    }
    __syncthreads();
  }

  // Epilogue: acc[i][j][v] is C[row, col] with col = lane % 32 and
  // row = (v / 4) * 8 + (lane / 32) * 4 + v % 4 inside the 32x32 block.
  OutT* C = static_cast<OutT*>(p.c) + bb * p.sc_b;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int64_t col = n0 + wn * TN + j * 32 + frow;
      if (col >= p.N) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t row = m0 + wm * TM + i * 32 + (v >> 2) * 8 + kgrp * 4 + (v & 3);
        if (row < p.M) store_out<OutT>(C + row * p.sc_m + col, acc[i][j][v]);
      }
    }
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

template <typename OutT>
static hipError_t dispatch_bf16(GemmParams p, hipStream_t s) {
  const int ma = majorness(p.a, p.sa_b, p.sa_m, p.sa_k, p.M, p.K, 8, p.batch);
  const int mb = majorness(p.b, p.sb_b, p.sb_n, p.sb_k, p.N, p.K, 8, p.batch);
  if (ma < 0 || mb < 0) return launch_generic<bf16_t, OutT>(p, s);
  const int64_t t256 = p.batch * ((p.M + 255) / 256) * ((p.N + 255) / 256);
  const int64_t t256x128 = p.batch * ((p.M + 255) / 256) * ((p.N + 127) / 128);
  if (p.M >= 256 && p.N >= 256 && t256 >= 256) return launch_bf16<256, 256, 2, 4, OutT>(p, ma, mb, s);
  if (p.M >= 256 && t256x128 >= 256) return launch_bf16<256, 128, 4, 2, OutT>(p, ma, mb, s);
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
