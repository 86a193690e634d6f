// Batched GEMM for DotGeneral: c[b] = a[b] (M x K) * b[b] (K x N), fp32 accumulate.
//
// bf16 path (the MFMA path the metric is quoted on), gfx950:
//   * v_mfma_f32_32x32x16_bf16.  Each lane feeds 8 consecutive-k bf16 of one
//     row of A / one column of B.  The MFMA is issued with the operands swapped
//     (B fragment first), so each lane's accumulators hold 4 consecutive output
//     columns and the epilogue stores 8 bytes (bf16) / 16 bytes (fp32) per lane.
//   * Global -> LDS without a VGPR round trip: buffer_load_dwordx4 ... lds puts
//     16 bytes per lane straight into LDS.  Out-of-range lanes are given an
//     offset past the buffer's end and read zeros, which pads ragged M/N/K edges.
//   * K-contiguous operand tiles live in LDS as [rows][64 k] with 16-byte chunks
//     XOR-swizzled per row; fragments are one ds_read_b128 per lane.
//     MN-contiguous operand tiles (e.g. rhs [K, N] row-major, the DotGeneral
//     config) stay [64 k][rows] as in memory and are read with the gfx950
//     transpose read ds_read_b64_tr_b16, so no transpose ever touches HBM or
//     VGPRs (the reference materializes two rhs transposes, dotgeneral.go:116-145).
//     Both swizzles are bank-conflict free for 8- and 16-lane LDS phases.
//   * Two LDS stages of 64-deep k-tiles: the loads of tile t+2 are issued right
//     after the barrier that retires tile t, so one tile of MFMA work covers the
//     load latency.  The loads are issued as inline asm so the compiler does not
//     wait on them before unrelated LDS reads; waits are explicit.
//   * Workgroup -> tile mapping is XCD-aware: consecutive workgroup ids land on
//     different XCDs (round robin), so ids are remapped to give each XCD a
//     contiguous run of tiles, ordered in GROUP_M-row groups for L2 reuse.
// fp32 path: v_mfma_f32_32x32x2f32 with MN-major LDS tiles (one float per lane).
// Anything the vector paths cannot address (odd strides, unaligned bases,
// negative strides, > 2 GiB per batch slice) runs a generic LDS-tiled kernel.
#include "common.h"

#define GHIP_LDS __attribute__((address_space(3)))

namespace ghip {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));

struct GemmParams {
  const void* a;
  const void* b;
  void* c;
  int64_t sa_b, sa_m, sa_k;
  int64_t sb_b, sb_k, sb_n;
  int64_t sc_b, sc_m;
  int64_t batch, M, N, K;
  int tiles_m, tiles_n;
  uint32_t a_extent, b_extent;  // bytes addressable from one batch slice's base
  int vec_c;                    // C rows allow 4-element vector stores
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
// bf16 operand tiles: R rows (m for A, n for B) x 64 k, loaded into LDS by
// buffer_load ... lds.
// ---------------------------------------------------------------------------
constexpr int kBK = 64;
constexpr uint32_t kOffOOB = 0x80000000u;  // past any buffer this path accepts

// K-contiguous LDS tile [R][64]: 16-byte chunk kc of row r sits at slot
// kc ^ swz_k(r), so 8 (or 16) consecutive rows reading the same kc land in
// distinct 16-byte bank groups of a 128-byte (or 256-byte) bank period.
__device__ __forceinline__ int swz_k(int r) { return (r & 7) ^ ((r >> 3) & 1); }
// MN-contiguous LDS tile [64][R]: chunk j of k-row k sits at slot j ^ swz_n(k),
// swz_n = {0, 6, 10, 12}[k & 3] (a nibble table): the 4 k-rows x 32 bytes read
// by 16 lanes of a transpose read, and the 4 x 64 bytes read by 32 lanes, land
// in distinct bank groups.
__device__ __forceinline__ int swz_n(int k) { return (0xCA60u >> ((k & 3) * 4)) & 15u; }

// Raw buffer descriptor (stride 0): reads at byte offsets >= `bytes` return 0.
__device__ __forceinline__ i32x4_t make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  i32x4_t r;
  r.x = __builtin_amdgcn_readfirstlane(static_cast<int>(b));
  r.y = __builtin_amdgcn_readfirstlane(static_cast<int>((b >> 32) & 0xffff));
  r.z = __builtin_amdgcn_readfirstlane(static_cast<int>(bytes));
  r.w = 0x00020000;
  return r;
}

// 16 bytes per lane from buffer offset voff straight into LDS at lds + lane*16.
__device__ __forceinline__ void dma16(i32x4_t rsrc, const void* lds, uint32_t voff) {
  const uint32_t la = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((GHIP_LDS const void*)lds));
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               ::"s"(__builtin_amdgcn_readfirstlane(la)), "v"(voff), "s"(rsrc)
               : "memory", "m0");
}

// Wave-instruction i of a wave fills LDS bytes [blk*1024, blk*1024 + 1024),
// blk = wave * kPerWave + i; lane l writes bytes l*16 .. l*16+15 of that block, so
// the swizzle is applied by choosing which global chunk each lane fetches.
template <int R, bool KC, int NW>
struct OperandTile {
  static constexpr int kInstr = R * kBK * 2 / 1024;
  static constexpr int kPerWave = kInstr / NW;
  static_assert(kInstr % NW == 0 && kPerWave % 2 == 0, "tile must split evenly over waves");
  static constexpr int kCPR = KC ? kBK / 8 : R / 8;  // 16-byte chunks per LDS row
  static constexpr int kRPI = 64 / kCPR;             // LDS rows per instruction
  static_assert(KC || R >= 128, "MN-major tiles need >= 16 chunks per LDS row");

  // The swizzle depends on the parity of the instruction only: byte offsets of
  // this lane's chunk for even / odd i; instruction i adds (i & ~1) * step.
  uint32_t voff[2];
  uint32_t step;
  int mn_valid;

  __device__ __forceinline__ static int row_of(int wave, int i, int lane) {
    return (wave * kPerWave + i) * kRPI + lane / kCPR;
  }
  __device__ __forceinline__ static int chunk_of(int wave, int i, int lane) {
    const int r = row_of(wave, i, lane);
    return KC ? (lane % kCPR) ^ swz_k(r) : (lane % kCPR) ^ swz_n(r);
  }
  // s_mn / s_k: element strides of the operand along its rows (m or n) and k.
  __device__ __forceinline__ void init(int wave, int lane, int64_t s_mn, int64_t s_k, int64_t valid) {
    mn_valid = valid > R ? R : static_cast<int>(valid);
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      const int r = row_of(wave, par, lane);
      const int c = chunk_of(wave, par, lane);
      voff[par] = KC ? static_cast<uint32_t>((r * s_mn + c * 8) * 2)
                     : static_cast<uint32_t>((r * s_k + c * 8) * 2);
    }
    step = static_cast<uint32_t>(kRPI * (KC ? s_mn : s_k) * 2);
  }
  // full: the whole tile lies inside the operand; otherwise out-of-range rows and
  // k-chunks read zeros.
  __device__ __forceinline__ void issue(i32x4_t rs, uint16_t* lds, int wave, int lane, bool full,
                                        int k_left) const {
#pragma unroll
    for (int i = 0; i < kPerWave; ++i) {
      const uint32_t v = voff[i & 1] + static_cast<uint32_t>(i & ~1) * step;
      const int r = row_of(wave, i, lane);
      const int c = chunk_of(wave, i, lane);
      const bool ok = KC ? (r < mn_valid && c * 8 < k_left) : (r < k_left && c * 8 < mn_valid);
      dma16(rs, lds + (wave * kPerWave + i) * 512, (full || ok) ? v : kOffOOB);
    }
  }
};

// Fragment of a 32-row (A) / 32-column (B) block for k16 step s: lane l gets 8
// consecutive k (8*(l/32) .. +8) of row/column l % 32.
__device__ __forceinline__ bf16x8_t frag_kc(const uint16_t* lds, int rbase, int s, int lane) {
  const int row = rbase + (lane & 31);
  const int slot = (2 * s + (lane >> 5)) ^ swz_k(row);
  return *reinterpret_cast<const bf16x8_t*>(lds + row * kBK + slot * 8);
}
// Same fragment from an MN-major tile: ds_read_b64_tr_b16 hands lane j of each
// 16-lane group element j of the four 4-element rows its group points at, so
// lanes address 4 k-rows x 16 columns and receive 4 consecutive k of one column.
template <int R>
__device__ __forceinline__ bf16x8_t frag_mn(const uint16_t* lds, int nbase, int s, int lane) {
  const int kl = 16 * s + 8 * (lane >> 5) + ((lane & 15) >> 2);
  const int nl = nbase + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  const uint16_t* p0 = lds + kl * R + (((nl >> 3) ^ swz_n(kl)) * 8) + (nl & 7);
  const uint16_t* p1 = p0 + 4 * R;  // k + 4 keeps k & 3, hence the swizzle
  bf16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((GHIP_LDS bf16x4_t*)(p0));
  bf16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((GHIP_LDS bf16x4_t*)(p1));
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

template <int BM, int BN, int WM, int WN, bool A_K, bool B_K, typename OutT>
__global__ __launch_bounds__(WM* WN * 64, 1) void gemm_bf16_kernel(GemmParams p) {
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;  // wave tile
  constexpr int FM = TM / 32, FN = TN / 32;  // 32x32 MFMA blocks per wave
  constexpr int NS = kBK / 16;               // k16 steps per k-tile
  using TA = OperandTile<BM, A_K, NW>;
  using TB = OperandTile<BN, B_K, NW>;
  constexpr int LPW = TA::kPerWave + TB::kPerWave;  // loads per wave per k-tile
  __shared__ __attribute__((aligned(1024))) uint16_t sa[2][BM * kBK];
  __shared__ __attribute__((aligned(1024))) uint16_t sb[2][BN * kBK];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;

  int64_t bb;
  int tm, tn;
  map_tile(blockIdx.x, p.batch * p.tiles_m * p.tiles_n, p.tiles_m, p.tiles_n, bb, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;
  const uint16_t* A0 = static_cast<const uint16_t*>(p.a) + bb * p.sa_b + m0 * p.sa_m;
  const uint16_t* B0 = static_cast<const uint16_t*>(p.b) + bb * p.sb_b + n0 * p.sb_n;
  const uint32_t a_left0 = p.a_extent - static_cast<uint32_t>(m0 * p.sa_m * 2);
  const uint32_t b_left0 = p.b_extent - static_cast<uint32_t>(n0 * p.sb_n * 2);

  TA ta;
  TB tb;
  ta.init(wave, lane, p.sa_m, p.sa_k, p.M - m0);
  tb.init(wave, lane, p.sb_n, p.sb_k, p.N - n0);
  const bool mn_full = m0 + BM <= p.M && n0 + BN <= p.N;
  const int KT = static_cast<int>((p.K + kBK - 1) / kBK);

  auto issue = [&](int kt, int st) {
    const int64_t k0 = static_cast<int64_t>(kt) * kBK;
    const int k_left = static_cast<int>(p.K - k0 < kBK ? p.K - k0 : kBK);
    const bool full = mn_full && k_left == kBK;
    ta.issue(make_rsrc(A0 + k0 * p.sa_k, a_left0 - static_cast<uint32_t>(k0 * p.sa_k * 2)), sa[st],
             wave, lane, full, k_left);
    tb.issue(make_rsrc(B0 + k0 * p.sb_k, b_left0 - static_cast<uint32_t>(k0 * p.sb_k * 2)), sb[st],
             wave, lane, full, k_left);
  };

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  bf16x8_t fa[2][FM], fb[2][FN];
  auto read = [&](int st, int s, int buf) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
      fa[buf][i] = A_K ? frag_kc(sa[st], wm * TM + i * 32, s, lane)
                       : frag_mn<BM>(sa[st], wm * TM + i * 32, s, lane);
#pragma unroll
    for (int j = 0; j < FN; ++j)
      fb[buf][j] = B_K ? frag_kc(sb[st], wn * TN + j * 32, s, lane)
                       : frag_mn<BN>(sb[st], wn * TN + j * 32, s, lane);
  };
  auto mfma = [&](int buf) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[buf][j], fa[buf][i], acc[i][j], 0, 0, 0);
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
  read(0, 0, 0);

  // Tile kt lives in stage kt & 1.  At its last k16 step: wait for tile kt+1,
  // barrier (everyone has finished reading stage kt & 1), refill that stage with
  // tile kt+2, fetch step 0 of tile kt+1, then run the last MFMAs of tile kt.
  auto tile = [&](int kt, int st) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int buf = s & 1;
      if (s + 1 < NS) {
        read(st, s + 1, buf ^ 1);
      } else {
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (kt + 2 < KT) issue(kt + 2, st);
        if (kt + 1 < KT) read(st ^ 1, 0, buf ^ 1);
      }
      mfma(buf);
    }
  };
  for (int kt = 0; kt < KT; kt += 2) {
    tile(kt, 0);
    if (kt + 1 < KT) tile(kt + 1, 1);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // acc[i][j] holds the transposed 32x32 block: lane l, value v ->
  // row m = l % 32, columns n = (v / 4) * 8 + (l / 32) * 4 + v % 4.
  OutT* C = static_cast<OutT*>(p.c) + bb * p.sc_b;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int64_t m = m0 + wm * TM + i * 32 + (lane & 31);
    if (m >= p.M) continue;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t n = n0 + wn * TN + j * 32 + q * 8 + (lane >> 5) * 4;
        OutT* dst = C + m * p.sc_m + n;
        if (p.vec_c && n + 3 < p.N) {
          if constexpr (sizeof(OutT) == 2) {
            *reinterpret_cast<uint2*>(dst) =
                make_uint2(pack_bf16x2(acc[i][j][q * 4 + 0], acc[i][j][q * 4 + 1]),
                           pack_bf16x2(acc[i][j][q * 4 + 2], acc[i][j][q * 4 + 3]));
          } else {
            *reinterpret_cast<float4*>(dst) = make_float4(acc[i][j][q * 4 + 0], acc[i][j][q * 4 + 1],
                                                          acc[i][j][q * 4 + 2], acc[i][j][q * 4 + 3]);
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < p.N) store_out<OutT>(dst + e, acc[i][j][q * 4 + e]);
        }
      }
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
