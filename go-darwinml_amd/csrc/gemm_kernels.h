// Kernel templates of the precompiled DotGeneral path (k_gemm.hip) and the
// launchers of its 256 x 256 cores, shared with k_gemm_big.hip, which
// instantiates the 64-bit-records forms (BIG = true) for operand slices of 2 GiB
// or more in a translation unit of its own.
#pragma once
#include "common.h"
#include "gemm_bf16_dev.h"

namespace ghip {

template <typename OutT>
__device__ __forceinline__ void store_out(OutT* p, float v);
template <>
__device__ __forceinline__ void store_out<float>(float* p, float v) { *p = v; }
template <>
__device__ __forceinline__ void store_out<bf16_t>(bf16_t* p, float v) { p->bits = f32_to_bf16(v); }
template <>
__device__ __forceinline__ void store_out<f16_t>(f16_t* p, float v) { p->bits = f32_to_f16(v); }

// Epilogue of the precompiled bf16 kernels: the output value itself is staged
// (bf16 bits or fp32) and a row chunk is one 16-byte store.
template <typename OutT>
struct StoreEpi;
// 16-bit outputs (bf16 / f16): the staged value is the output's bits.
template <typename OutT>
struct StoreEpi16 {
  using Stage = uint16_t;
  struct Pre {};
  OutT* c;
  int64_t sc_b, sc_m, N;
  int vec;
  __device__ __forceinline__ static Stage stage(float v) {
    if constexpr (sizeof(OutT) == 2 && __is_same(OutT, f16_t)) return f32_to_f16(v);
    else return f32_to_bf16(v);
  }
  template <bool FULL>
  __device__ __forceinline__ void prefetch(int64_t, int64_t, int64_t, Pre&) const {}
  template <bool FULL>
  __device__ __forceinline__ void store(int64_t bb, int64_t m, int64_t n, const Stage* v, const Stage*,
                                        const Pre&) const {
    uint16_t* dst = reinterpret_cast<uint16_t*>(c + bb * sc_b + m * sc_m + n);
    if (vec && (FULL || n + 7 < N)) {
      *reinterpret_cast<uint4*>(dst) = make_uint4(v[0] | (uint32_t(v[1]) << 16), v[2] | (uint32_t(v[3]) << 16),
                                                 v[4] | (uint32_t(v[5]) << 16), v[6] | (uint32_t(v[7]) << 16));
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (FULL || n + e < N) dst[e] = v[e];
    }
  }
};
template <>
struct StoreEpi<bf16_t> : StoreEpi16<bf16_t> {};
template <>
struct StoreEpi<f16_t> : StoreEpi16<f16_t> {};
template <>
struct StoreEpi<float> {
  using Stage = float;
  struct Pre {};
  float* c;
  int64_t sc_b, sc_m, N;
  int vec;
  __device__ __forceinline__ static Stage stage(float v) { return v; }
  template <bool FULL>
  __device__ __forceinline__ void prefetch(int64_t, int64_t, int64_t, Pre&) const {}
  template <bool FULL>
  __device__ __forceinline__ void store(int64_t bb, int64_t m, int64_t n, const Stage* v, const Stage*,
                                        const Pre&) const {
    float* dst = c + bb * sc_b + m * sc_m + n;
    if (vec && (FULL || n + 3 < N)) {
      *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (FULL || n + e < N) dst[e] = v[e];
    }
  }
};

template <typename OutT>
__device__ __forceinline__ StoreEpi<OutT> store_epi(const GemmParams& p) {
  StoreEpi<OutT> e;
  e.c = static_cast<OutT*>(p.c);
  e.sc_b = p.sc_b;
  e.sc_m = p.sc_m;
  e.N = p.N;
  e.vec = p.vec_c;
  return e;
}

// 16-bit inputs: bf16, or f16 (InT = f16_t selects the f16 MFMA).
template <int BM, int BN, int WM, int WN, bool A_K, bool B_K, typename InT, typename OutT>
__global__ __launch_bounds__(WM* WN * 64, 1) void gemm_bf16_kernel(GemmParams p) {
  const StoreEpi<OutT> epi = store_epi<OutT>(p);
  gemm_bf16_body<BM, BN, WM, WN, A_K, B_K, 1, StoreEpi<OutT>, __is_same(InT, f16_t)>(p, epi);
}
// The 4-wave 256 x 256 16x16x32 core for A K-contiguous, B MN-contiguous (128 x 128
// waves, AGPR accumulators).
template <typename InT, typename OutT, bool BIG = false>
__global__ __launch_bounds__(256, 1) void gemm_bf16_kernel4km(GemmParams p) {
  const StoreEpi<OutT> epi = store_epi<OutT>(p);
  gemm_bf16_body4km<StoreEpi<OutT>, __is_same(InT, f16_t), 1, BIG>(p, epi);
}
// Products sharing A, one per "batch" index g of the grid (gemm_bf16_kernel4km's
// core): the output base of tile group g is c_g[g].
template <typename OutT>
struct GroupStoreEpi : StoreEpi<OutT> {
  void* cg[kGemmMaxGroups];
  template <bool FULL>
  __device__ __forceinline__ void store(int64_t bb, int64_t m, int64_t n, const typename StoreEpi<OutT>::Stage* v,
                                        const typename StoreEpi<OutT>::Stage* v1,
                                        const typename StoreEpi<OutT>::Pre& pre) const {
    StoreEpi<OutT> e = *this;
    e.c = static_cast<OutT*>(pick_group(cg, bb));
    e.template store<FULL>(0, m, n, v, v1, pre);
  }
};
template <typename InT, typename OutT>
__global__ __launch_bounds__(256, 1) void gemm_bf16_kernel4km_grouped(GemmParams p) {
  GroupStoreEpi<OutT> epi;
  static_cast<StoreEpi<OutT>&>(epi) = store_epi<OutT>(p);
#pragma unroll
  for (int g = 0; g < kGemmMaxGroups; ++g) epi.cg[g] = p.c_g[g];
  gemm_bf16_body4km<GroupStoreEpi<OutT>, __is_same(InT, f16_t)>(p, epi);
}
// The 4-wave 256 x 256 core for both operands MN-contiguous (32-deep, four stages).
template <typename InT, typename OutT, bool BIG = false>
__global__ __launch_bounds__(256, 1) void gemm_bf16_kernel4mn(GemmParams p) {
  const StoreEpi<OutT> epi = store_epi<OutT>(p);
  gemm_bf16_body4mn<StoreEpi<OutT>, __is_same(InT, f16_t), BIG>(p, epi);
}
// The 8-wave 256 x 256 16x16x32 core for B K-contiguous layouts (64-deep, two stages).
template <bool A_K, bool B_K, typename InT, typename OutT, bool BIG = false>
__global__ __launch_bounds__(512, 1) void gemm_bf16_kernel8x(GemmParams p) {
  const StoreEpi<OutT> epi = store_epi<OutT>(p);
  gemm_bf16_body8x<A_K, B_K, StoreEpi<OutT>, __is_same(InT, f16_t), 1, BIG>(p, epi);
}

// ---------------------------------------------------------------------------
// fp32 MFMA path: v_mfma_f32_32x32x2f32, 32-deep k-tiles by buffer_load ... lds
// (two stages), operands swapped like the bf16 path so a lane stores 4 adjacent
// columns.  K-contiguous tiles are [rows][32 k] with 16-byte chunks XOR-swizzled
// per row; one ds_read_b128 hands a lane the 4 k of 4 consecutive MFMA steps
// (lanes 0-31 take k = 8g + e, lanes 32-63 k = 8g + 4 + e at step e: both operands
// use the same k order, so the contraction is unchanged).  MN-contiguous tiles
// stay [32 k][rows] and are read one k per step (ds_read_b32, 128 contiguous
// bytes per half-wave).
// ---------------------------------------------------------------------------
constexpr int kBK32 = 32;

// 32-bit LDS address form of dma16 (the generic-pointer form costs SGPRs here).
// m0 is set and consumed inside this one asm statement, and no compiler-generated
// code in these kernels reads or writes m0 (none appears in their ISA apart from
// these pairs), so clang's warning that a reserved-register clobber is not
// preserved does not apply here.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16_la(i32x4_t rsrc, uint32_t la, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               ::"s"(la), "v"(voff), "s"(rsrc) : "memory", "m0");
}
#pragma clang diagnostic pop

// R rows x 32 k fp32 tile, split over NW waves in 1 KiB DMA instructions.
template <int R, bool KC, int NW>
struct TileF32 {
  static constexpr int kInstr = R * kBK32 * 4 / 1024;
  static constexpr int kPerWave = kInstr / NW;
  static_assert(kInstr % NW == 0, "tile must split evenly over waves");
  static_assert(KC || (R >= 16 && R <= 256), "MN-major: 1..4 k-rows per instruction");
  uint32_t voff[kPerWave];
  int rowv[kPerWave], kv[kPerWave];  // first row / k each lane's chunk holds

  __device__ __forceinline__ void init(int wave, int lane, int64_t s_mn, int64_t s_k) {
#pragma unroll
    for (int i = 0; i < kPerWave; ++i) {
      const int blk = wave * kPerWave + i;
      if constexpr (KC) {  // 8 rows of 8 chunks per instruction; slot pc holds chunk pc ^ (r & 7)
        const int r = blk * 8 + lane / 8, c = (lane % 8) ^ (r & 7);
        rowv[i] = r;
        kv[i] = c * 4;
        voff[i] = static_cast<uint32_t>((r * s_mn + c * 4) * 4);
      } else {
        constexpr int kCPR = R / 4, kRPI = 64 / kCPR;  // chunks per k-row, k-rows per instruction
        const int k = blk * kRPI + lane / kCPR, ch = lane % kCPR;
        rowv[i] = ch * 4;
        kv[i] = k;
        voff[i] = static_cast<uint32_t>((k * s_k + ch * 4) * 4);
      }
    }
  }
  __device__ __forceinline__ void issue(i32x4_t rs, uint32_t lds, int wave, bool full, int rows_left,
                                        int k_left) const {
#pragma unroll
    for (int i = 0; i < kPerWave; ++i) {
      const bool ok = rowv[i] < rows_left && kv[i] < k_left;
      dma16_la(rs, lds + (wave * kPerWave + i) * 1024, (full || ok) ? voff[i] : kOffOOB);
    }
  }
};

// K-contiguous fragment, group g (k 8g .. 8g+7) of the 32-row block at rbase.
__device__ __forceinline__ float4 frag_f32_kc(const float* lds, int rbase, int g, int lane) {
  const int r = rbase + (lane & 31);
  const int c = (2 * g + (lane >> 5)) ^ (r & 7);
  return *reinterpret_cast<const float4*>(lds + r * kBK32 + c * 4);
}
// MN-contiguous fragment at step e of group g.
template <int R>
__device__ __forceinline__ float frag_f32_mn(const float* lds, int rbase, int g, int e, int lane) {
  return lds[(8 * g + 4 * (lane >> 5) + e) * R + rbase + (lane & 31)];
}
__device__ __forceinline__ float f4_at(const float4& v, int e) {
  return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
}

template <int BM, int BN, int WM, int WN, bool A_K, bool B_K, typename OutT, bool BIG = false>
__global__ __launch_bounds__(WM* WN * 64, (WM * WN == 4 ? 2 : 1)) void gemm_f32_kernel(GemmParams p) {
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;
  using TA = TileF32<BM, A_K, NW>;
  using TB = TileF32<BN, B_K, NW>;
  constexpr int LPW = TA::kPerWave + TB::kPerWave;
  constexpr int SA = BM * kBK32, SB = BN * kBK32;  // floats per stage
  __shared__ __attribute__((aligned(1024))) float smem[2][SA + SB];
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((GHIP_LDS void*)&smem[0][0]));

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;
  int64_t bb;
  int tm, tn;
  map_tile(blockIdx.x, p.batch * p.tiles_m * p.tiles_n, p.tiles_m, p.tiles_n, bb, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;
  const float* A0 = static_cast<const float*>(p.a) + bb * p.sa_b + m0 * p.sa_m;
  const float* B0 = static_cast<const float*>(p.b) + bb * p.sb_b + n0 * p.sb_n;
  const auto a_left0 = ExtSel<BIG>::a(p, m0 * p.sa_m * 4);
  const auto b_left0 = ExtSel<BIG>::b(p, n0 * p.sb_n * 4);
  TA ta;
  TB tb;
  ta.init(wave, lane, p.sa_m, p.sa_k);
  tb.init(wave, lane, p.sb_n, p.sb_k);
  const int rows_a = static_cast<int>(p.M - m0 < BM ? p.M - m0 : BM);
  const int rows_b = static_cast<int>(p.N - n0 < BN ? p.N - n0 : BN);
  const bool mn_full = m0 + BM <= p.M && n0 + BN <= p.N;
  const int KT = static_cast<int>((p.K + kBK32 - 1) / kBK32);

  auto issue = [&](int kt, int st) {
    const int64_t k0 = static_cast<int64_t>(kt) * kBK32;
    const int k_left = static_cast<int>(p.K - k0 < kBK32 ? p.K - k0 : kBK32);
    const bool full = mn_full && k_left == kBK32;
    const uint32_t la = lds0 + static_cast<uint32_t>(st) * (SA + SB) * 4;
    ta.issue(make_rsrc(A0 + k0 * p.sa_k, a_left0.at(k0 * p.sa_k * 4)), la, wave, full,
             rows_a, k_left);
    tb.issue(make_rsrc(B0 + k0 * p.sb_k, b_left0.at(k0 * p.sb_k * 4)), la + SA * 4, wave,
             full, rows_b, k_left);
  };

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  auto compute = [&](int st) {
    const float* As = &smem[st][0];
    const float* Bs = &smem[st][SA];
#pragma unroll
    for (int g = 0; g < kBK32 / 8; ++g) {
      float4 a4[FM], b4[FN];
      if constexpr (A_K) {
#pragma unroll
        for (int i = 0; i < FM; ++i) a4[i] = frag_f32_kc(As, wm * TM + i * 32, g, lane);
      }
      if constexpr (B_K) {
#pragma unroll
        for (int j = 0; j < FN; ++j) b4[j] = frag_f32_kc(Bs, wn * TN + j * 32, g, lane);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float af[FM], bf[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
          af[i] = A_K ? f4_at(a4[i], e) : frag_f32_mn<BM>(As, wm * TM + i * 32, g, e, lane);
#pragma unroll
        for (int j = 0; j < FN; ++j)
          bf[j] = B_K ? f4_at(b4[j], e) : frag_f32_mn<BN>(Bs, wn * TN + j * 32, g, e, lane);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(bf[j], af[i], acc[i][j], 0, 0, 0);
      }
    }
  };

  // Prologue: tiles 0 and 1 in flight, wait for tile 0.
  issue(0, 0);
  if (KT > 1) {
    issue(1, 1);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(LPW) : "memory");
  } else {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int st = kt & 1;
    compute(st);
    // Every wave is done with stage st and tile kt+1 has landed; tile kt+2 refills st.
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (kt + 2 < KT) issue(kt + 2, st);
  }

  // acc[i][j]: lane l, value v -> row m = l % 32 of block i, columns
  // n = (v / 4) * 8 + (l / 32) * 4 + v % 4 of block j.
  OutT* C = static_cast<OutT*>(p.c) + bb * p.sc_b;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int64_t m = m0 + wm * TM + i * 32 + (lane & 31);
    if (m >= p.M) continue;
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t n = n0 + wn * TN + j * 32 + q * 8 + (lane >> 5) * 4;
        if (n >= p.N) continue;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[i][j][q * 4 + e];
        OutT* dst = C + m * p.sc_m + n;
        if (p.vec_c && n + 3 < p.N) {
          if constexpr (sizeof(OutT) == 2)
            *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
          else
            *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < p.N) store_out<OutT>(dst + e, v[e]);
        }
      }
  }
}

// The 256 x 256 cores (grids of >= 128 tiles).  BIG: the 64-bit-records
// instantiations (operand slices of 2 GiB or more), instantiated in k_gemm_big.hip.
template <bool BIG, typename InT, typename OutT>
hipError_t launch_bf16_4w(GemmParams p, bool a_k, bool b_k, hipStream_t s) {
  p.tiles_m = static_cast<int>((p.M + 255) / 256);
  p.tiles_n = static_cast<int>((p.N + 255) / 256);
  const dim3 grid(static_cast<unsigned>(p.batch * p.tiles_m * p.tiles_n));
  if (a_k && b_k) hipLaunchKernelGGL((gemm_bf16_kernel8x<true, true, InT, OutT, BIG>), grid, dim3(512), 0, s, p);
  else if (a_k) hipLaunchKernelGGL((gemm_bf16_kernel4km<InT, OutT, BIG>), grid, dim3(256), 0, s, p);
  else if (b_k) hipLaunchKernelGGL((gemm_bf16_kernel8x<false, true, InT, OutT, BIG>), grid, dim3(512), 0, s, p);
  else hipLaunchKernelGGL((gemm_bf16_kernel4mn<InT, OutT, BIG>), grid, dim3(256), 0, s, p);
  return hipGetLastError();
}

template <int BM, int BN, int WM, int WN, typename OutT, bool BIG = false>
hipError_t launch_f32(GemmParams p, bool a_k, bool b_k, hipStream_t s) {
  p.tiles_m = static_cast<int>((p.M + BM - 1) / BM);
  p.tiles_n = static_cast<int>((p.N + BN - 1) / BN);
  const dim3 grid(static_cast<unsigned>(p.batch * p.tiles_m * p.tiles_n)), block(WM * WN * 64);
  if (a_k && b_k) hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, WM, WN, true, true, OutT, BIG>), grid, block, 0, s, p);
  else if (a_k) hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, WM, WN, true, false, OutT, BIG>), grid, block, 0, s, p);
  else if (b_k) hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, WM, WN, false, true, OutT, BIG>), grid, block, 0, s, p);
  else hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, WM, WN, false, false, OutT, BIG>), grid, block, 0, s, p);
  return hipGetLastError();
}

extern template hipError_t launch_bf16_4w<true, bf16_t, bf16_t>(GemmParams, bool, bool, hipStream_t);
extern template hipError_t launch_bf16_4w<true, bf16_t, float>(GemmParams, bool, bool, hipStream_t);
extern template hipError_t launch_bf16_4w<true, f16_t, f16_t>(GemmParams, bool, bool, hipStream_t);
extern template hipError_t launch_bf16_4w<true, f16_t, float>(GemmParams, bool, bool, hipStream_t);
extern template hipError_t launch_f32<256, 256, 2, 4, float, true>(GemmParams, bool, bool, hipStream_t);
extern template hipError_t launch_f32<256, 256, 2, 4, bf16_t, true>(GemmParams, bool, bool, hipStream_t);

}  // namespace ghip
