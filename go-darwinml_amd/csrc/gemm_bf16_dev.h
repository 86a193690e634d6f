// bf16 MFMA GEMM core for gfx950 (device code only).
//
// Shared by the precompiled DotGeneral kernels (k_gemm.hip, epilogue = plain
// store) and by GEMMs whose epilogue is generated at graph Compile time
// (graph_lower.cpp embeds this file's text and compiles it with hipRTC together
// with the generated elementwise epilogue), so both run the same main loop.
//
//   * v_mfma_f32_32x32x16_bf16.  Each lane feeds 8 consecutive-k bf16 of one
//     row of A / one column of B.  The MFMA is issued with the operands swapped
//     (B fragment first), so each lane's accumulators hold 4 consecutive output
//     columns and the epilogue handles 4 adjacent outputs per call.
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
//   * NB = 2 computes two products that share the left operand, A.B and A.B1
//     (B1 has B's strides), in one pass: the A tile is loaded once for both, and
//     the epilogue receives both results for the same output element (a gated
//     activation such as SiLU(x.Wg) * (x.Wu) never writes its two halves).
#ifndef GHIP_GEMM_BF16_DEV_H
#define GHIP_GEMM_BF16_DEV_H

#if defined(__HIPCC_RTC__)
typedef __hip_internal::int64_t int64_t;
typedef __hip_internal::uint64_t uint64_t;
typedef __hip_internal::uint32_t uint32_t;
typedef __hip_internal::uint16_t uint16_t;
#else
#include <hip/hip_runtime.h>
#include <stdint.h>
#endif

#ifndef GHIP_LDS
#define GHIP_LDS __attribute__((address_space(3)))
#endif

namespace ghip {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
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
  uint32_t a_extent, b_extent;  // bytes addressable from one batch slice's base (< 2 GiB)
  int vec_c;                    // C rows allow 4-element vector stores
  const void* b1;               // second right operand (NB = 2), B's strides and extent
  // Grouped launch (4-wave K-contiguous-A core): groups > 0 products A.B_g -> C_g
  // sharing A, one per "batch" index g; b_g / c_g replace b + g sb_b / c + g sc_b.
  int groups;
  const void* b_g[4];
  void* c_g[4];
  // Slices of 2 GiB or more (the BIG instantiations): their byte extents.
  int64_t a_extent64, b_extent64;
};
constexpr int kGemmMaxGroups = 4;

// A tile's DMA reads at most 256 rows of an operand (m or n rows of a K-contiguous
// operand, k rows of an MN-contiguous one) from a descriptor based at the tile and
// k step, at byte offsets that must stay below 2 GiB; s_mn / s_k are element
// strides, es the element size.  The operand slice itself may be of any size.
__host__ __device__ inline bool gemm_rows_fit(int64_t s_mn, int64_t s_k, int64_t es) {
  const int64_t s = s_mn > s_k ? s_mn : s_k;
  return s >= 0 && (s * 256 + 256) * es < (int64_t{1} << 31);
}

#if !defined(__HIPCC_RTC__)
// Contraction split for products whose grid leaves most of the chip idle.  s
// ranges of kc = K / s contraction steps (kc a multiple of 64) run as s slices of
// one grid, each writing its fp32 partial product; a second kernel sums the s
// partials in split order and rounds once.  s = 1: no split.  The rule is a cost
// model fitted to split-count sweeps (graph-replayed launches, one box): a 128 x
// 128 tile takes ~2 us plus ~14.6 ns per contraction step with 16-bit operands,
// latency-bound, so two workgroups per CU each keep that pace (512 slots); with
// fp32 operands ~65 ns a step, which is already ~80% of a CU's fp32 MFMA rate, so
// only one tile per CU counts (256 slots).  A split grid cannot beat the operands'
// own read time (A + B at ~5 TB/s), and the partials cost s x M x N x 8 bytes
// (written, then read by the sum) at ~3 TB/s plus ~2 us for the summing launch; a
// split must save 15%, and a range keeps at least 128 steps.  es: the operands'
// element size (2 or 4).  One batch only.
struct GemmSplit {
  int s;
  int64_t kc;
};
constexpr int kGemmMaxSplit = 16;
inline GemmSplit gemm_k_split(int64_t batch, int64_t M, int64_t N, int64_t K, int es) {
  GemmSplit r{1, K};
  if (batch != 1 || M <= 0 || N <= 0 || K < 1024 || (es != 2 && es != 4)) return r;
  const int64_t t = ((M + 127) / 128) * ((N + 127) / 128);
  const int64_t slots = es == 4 ? 256 : 512;
  if (2 * t > slots) return r;
  const int64_t kc_min = 128;
  const double step_us = es == 4 ? 0.065 : 0.0146;
  int64_t smax = slots / t;
  if (smax > K / kc_min) smax = K / kc_min;
  if (smax > kGemmMaxSplit) smax = kGemmMaxSplit;
  const double floor_us = static_cast<double>(M * K + K * N) * es / 5e6;
  auto cost = [&](int64_t s) {
    const double k_us = 2.0 + static_cast<double>(K / s) * step_us;
    const double part_us = s > 1 ? static_cast<double>(s) * M * N * 8 / 3e6 + 2.0 : 0.0;
    return (k_us > floor_us ? k_us : floor_us) + part_us;
  };
  double best = 0.85 * cost(1);
  for (int64_t s = 2; s <= smax; ++s) {
    if (K % (s * 64) != 0) continue;
    const double c = cost(s);
    if (c < best) {
      best = c;
      r.s = static_cast<int>(s);
      r.kc = K / s;
    }
  }
  return r;
}
// Workspace bytes of a split (0 for s = 1): s fp32 partial products [M, N].
inline int64_t gemm_split_bytes(const GemmSplit& sp, int64_t M, int64_t N) {
  return sp.s > 1 ? static_cast<int64_t>(sp.s) * M * N * 4 : 0;
}
#endif

// Generated epilogues read up to kEpiMaxIn extra operands, each addressed as
// in[k] + bb * s_b[k] + m * s_m[k] + n * s_n[k] (elements), and write `out`
// ([batch, M, N] with strides so_b, so_m, 1).
constexpr int kEpiMaxIn = 6;
struct EpiArgs {
  const void* in[kEpiMaxIn];
  int64_t s_b[kEpiMaxIn], s_m[kEpiMaxIn], s_n[kEpiMaxIn];
  int vin[kEpiMaxIn];  // operand k allows 4-element vector loads (unit n stride, aligned)
  void* out;
  int64_t so_b, so_m, N;
  int vec;  // out rows allow 4-element vector stores
};

#if defined(__HIP__) || defined(__HIPCC_RTC__)
// (The structs above are also used by host-only translation units.)

// ptrs[g] for a wave-uniform g < kGemmMaxGroups, by selects (an indexed read of a
// kernel-argument array would be copied to scratch memory first).
template <typename P>
__device__ __forceinline__ P pick_group(const P (&ptrs)[kGemmMaxGroups], int64_t g) {
  return g == 0 ? ptrs[0] : g == 1 ? ptrs[1] : g == 2 ? ptrs[2] : ptrs[3];
}

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
// Variant for 16x16x32 fragments, whose transpose reads cover k-rows k..k+3 and
// k+8..k+11 of the same 16 columns in one half-wave: bit 3 of k also flips bit 1 of
// the slot, so those 8 row pieces (2 chunks each) fill all 16 slots of a 256-byte
// bank period.
__device__ __forceinline__ int swz_n2(int k) { return swz_n(k) ^ (((k >> 3) & 1) << 1); }

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

// Records of a descriptor based `left` bytes before the end of an operand slice:
// the rest of the slice, capped at kOffOOB.  A slice may span more than 4 GiB; a
// tile's loads stay below 2 GiB from the descriptor's base (gemm_rows_fit), so
// the cap cuts nothing a tile reads and a masked lane's kOffOOB still reads zeros.
__device__ __forceinline__ uint32_t left_bytes(int64_t left) {
  return left <= 0 ? 0u : left >= static_cast<int64_t>(kOffOOB) ? kOffOOB : static_cast<uint32_t>(left);
}

// Records of the descriptors a tile bases at its rows and k step, from the bytes
// of the operand slice left after the tile's base.  Ext32 (BIG = false: slices
// below 2 GiB) keeps the arithmetic in 32 bits; Ext64 (BIG = true: any slice)
// subtracts in 64 bits and caps with left_bytes.  They are separate
// instantiations because Ext64's extra scalar registers made the 32-bit cases'
// cores spill SGPRs (1.5-9% slower, measured).
struct Ext32 {
  uint32_t left;
  __device__ __forceinline__ Ext32(uint32_t extent, int64_t used) : left(extent - static_cast<uint32_t>(used)) {}
  __device__ __forceinline__ uint32_t at(int64_t d) const { return left - static_cast<uint32_t>(d); }
};
struct Ext64 {
  int64_t left;
  __device__ __forceinline__ Ext64(int64_t extent, int64_t used) : left(extent - used) {}
  __device__ __forceinline__ uint32_t at(int64_t d) const { return left_bytes(left - d); }
};
template <bool BIG>
struct ExtSel {
  __device__ __forceinline__ static Ext32 a(const GemmParams& p, int64_t used) { return Ext32(p.a_extent, used); }
  __device__ __forceinline__ static Ext32 b(const GemmParams& p, int64_t used) { return Ext32(p.b_extent, used); }
};
template <>
struct ExtSel<true> {
  __device__ __forceinline__ static Ext64 a(const GemmParams& p, int64_t used) { return Ext64(p.a_extent64, used); }
  __device__ __forceinline__ static Ext64 b(const GemmParams& p, int64_t used) { return Ext64(p.b_extent64, used); }
};

// 16 bytes per lane from buffer offset voff straight into LDS byte address
// la + lane*16 (la wave-uniform; a 32-bit LDS address, so no generic-pointer
// conversion is needed per load).
// m0 is set and consumed inside this one asm statement, and no compiler-generated
// code in these kernels reads or writes m0 (none appears in their ISA apart from
// these pairs), so clang's warning that a reserved-register clobber is not
// preserved does not apply here.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(i32x4_t rsrc, uint32_t la, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               ::"s"(la), "v"(voff), "s"(rsrc) : "memory", "m0");
}
#pragma clang diagnostic pop

// Wave-instruction i of a wave fills LDS bytes [blk*1024, blk*1024 + 1024),
// blk = wave * kPerWave + i; lane l writes bytes l*16 .. l*16+15 of that block, so
// the swizzle is applied by choosing which global chunk each lane fetches.
// BK: k-depth of the tile (64; MN-contiguous tiles may also be 32 deep).  L16: the
// tile is read as 16x16x32 fragments: an MN-contiguous tile uses swz_n2 instead of
// swz_n; a K-contiguous one is laid out so that a fragment read has the access
// pattern of a 32x32x16 one (see KC16 below).
//
// IL (interleaved, KC16 tiles of four waves): instruction i of wave w fills the 1 KiB
// block i * NW + w instead of w * kPerWave + i, so the NW waves' instruction i
// together fill the 32-row group i (NW * kRPI == 32) and a wave's instructions
// step through the groups, 32 operand rows apart.
template <int R, bool KC, int NW, int BK = kBK, bool L16 = false, bool IL = false>
struct OperandTile {
  static_assert(BK == kBK || (!KC && BK == 32), "32-deep tiles are MN-contiguous only");
  static constexpr int kInstr = R * BK * 2 / 1024;
  static constexpr int kPerWave = kInstr / NW;
  // An even share repeats the swizzle every two instructions; a share of one uses
  // voff[0] alone.
  static_assert(kInstr % NW == 0 && (kPerWave % 2 == 0 || kPerWave == 1), "tile must split evenly over waves");
  static constexpr int kCPR = KC ? BK / 8 : R / 8;  // 16-byte chunks per LDS row
  static constexpr int kRPI = 64 / kCPR;             // LDS rows per instruction
  static_assert(KC || R >= 128, "MN-major tiles need >= 16 chunks per LDS row");
  static_assert(!IL || (KC && L16 && NW * kRPI == 32), "interleaved: KC16 tiles whose waves fill 32 rows");
  // 1 KiB LDS block written by instruction i of `wave`.
  __device__ __forceinline__ static int block(int wave, int i) { return IL ? i * NW + wave : wave * kPerWave + i; }
  // KC16: K-contiguous [R][64] tile for 16x16x32 fragments.  A 16x16x32 fragment
  // (16 rows x 4 k-chunks) read from a plain [R][64] tile puts lanes l and l + 16 on
  // the same row, which the LDS serves with 2-way bank conflicts (measured: 4
  // conflict cycles per ds_read_b128).  So LDS row rho, chunk slot q ^ swz_k(rho)
  // holds operand row m = 32 (rho / 32) + 16 (q / 4) + (rho % 32) / 2 and k-chunk
  // kc = 4 ((q / 2) % 2) + 2 (q % 2) + rho % 2: the fragment of 16-row block b at k32
  // step s is read as lane l -> LDS row 32 (b / 2) + 2 (l % 16) + (l / 16) % 2, chunk
  // 4 (b % 2) + 2 s + l / 32 (32 distinct rows per chunk, measured conflict-free),
  // and each load instruction (8 LDS rows) still fetches 8 whole 128-byte rows.
  static constexpr bool KC16 = KC && L16;
  static_assert(!KC16 || (R % 32 == 0 && (IL || 32 % (kPerWave * kRPI) == 0)),
                "KC16: a wave's loads stay inside one 32-row group (or interleave)");

  // Byte offsets of this lane's chunk.  The swizzle depends on the parity of the
  // instruction only: even / odd i; instruction i adds (i & ~1) * step, step being
  // kRPI operand rows (in the KC16 layout instruction i + 2 holds the operand rows
  // 8 further on, so kRPI / 2).
  static constexpr int kNV = 2;
  uint32_t voff[kNV];
  uint32_t step;
  int mn_valid;

  __device__ __forceinline__ static int lds_row(int wave, int i, int lane) {
    return block(wave, i) * kRPI + lane / kCPR;
  }
  // Operand row (m / n for K-contiguous tiles, k for MN-contiguous ones) and
  // 16-byte chunk that the lane fetches in instruction i.
  __device__ __forceinline__ static int row_of(int wave, int i, int lane) {
    const int rho = lds_row(wave, i, lane);
    if constexpr (KC16) {
      const int q = (lane % kCPR) ^ swz_k(rho);
      return 32 * (rho / 32) + 16 * (q / 4) + (rho % 32) / 2;
    } else {
      return rho;
    }
  }
  __device__ __forceinline__ static int chunk_of(int wave, int i, int lane) {
    const int rho = lds_row(wave, i, lane);
    if constexpr (KC16) {
      const int q = (lane % kCPR) ^ swz_k(rho);
      return 4 * ((q / 2) % 2) + 2 * (q % 2) + rho % 2;
    } else {
      return KC ? (lane % kCPR) ^ swz_k(rho) : (lane % kCPR) ^ (L16 ? swz_n2(rho) : swz_n(rho));
    }
  }
  // s_mn / s_k: element strides of the operand along its rows (m or n) and k.
  __device__ __forceinline__ void init(int wave, int lane, int64_t s_mn, int64_t s_k, int64_t valid) {
    mn_valid = valid > R ? R : static_cast<int>(valid);
#pragma unroll
    for (int par = 0; par < kNV; ++par) {
      const int r = row_of(wave, par, lane);
      const int c = chunk_of(wave, par, lane);
      voff[par] = KC ? static_cast<uint32_t>((r * s_mn + c * 8) * 2)
                     : static_cast<uint32_t>((r * s_k + c * 8) * 2);
    }
    step = static_cast<uint32_t>((IL ? 32 : KC16 ? kRPI / 2 : kRPI) * (KC ? s_mn : s_k) * 2);
  }
  __device__ __forceinline__ uint32_t off(int i) const {
    if constexpr (IL) return voff[0] + static_cast<uint32_t>(i) * step;
    else return voff[i & 1] + static_cast<uint32_t>(i & ~1) * step;
  }
  // Instruction i of this wave's share (see issue()).
  template <bool FULL>
  __device__ __forceinline__ void issue_one(i32x4_t rs, uint32_t lds, int wave, int lane, int k_left, int i) const {
    const uint32_t v = off(i);
    if constexpr (FULL) {
      dma16(rs, lds + block(wave, i) * 1024, v);
    } else {
      const int r = row_of(wave, i, lane);
      const int c = chunk_of(wave, i, lane);
      const bool ok = KC ? (r < mn_valid && c * 8 < k_left) : (r < k_left && c * 8 < mn_valid);
      dma16(rs, lds + block(wave, i) * 1024, ok ? v : kOffOOB);
    }
  }
  // lds: LDS byte address of the tile.  FULL: the whole tile lies inside the
  // operand (no per-lane masks); otherwise out-of-range rows and k-chunks read
  // zeros.
  template <bool FULL>
  __device__ __forceinline__ void issue(i32x4_t rs, uint32_t lds, int wave, int lane, int k_left) const {
#pragma unroll
    for (int i = 0; i < kPerWave; ++i) {
      const uint32_t v = off(i);
      if constexpr (FULL) {
        dma16(rs, lds + block(wave, i) * 1024, v);
      } else {
        const int r = row_of(wave, i, lane);
        const int c = chunk_of(wave, i, lane);
        const bool ok = KC ? (r < mn_valid && c * 8 < k_left) : (r < k_left && c * 8 < mn_valid);
        dma16(rs, lds + block(wave, i) * 1024, ok ? v : kOffOOB);
      }
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

// Half h (k + 0..3 or k + 4..7) of frag_mn's fragment: one transpose read.
template <int R>
__device__ __forceinline__ bf16x4_t frag_mn_half(const uint16_t* lds, int nbase, int s, int lane, int h) {
  const int kl = 16 * s + 8 * (lane >> 5) + ((lane & 15) >> 2);
  const int nl = nbase + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  const uint16_t* p0 = lds + kl * R + (((nl >> 3) ^ swz_n(kl)) * 8) + (nl & 7) + h * 4 * R;
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((GHIP_LDS bf16x4_t*)(p0));
}

template <bool B>
struct BoolC {
  static constexpr bool value = B;
};
template <int V>
struct IntC {
  static constexpr int value = V;
};

// One 32x32x16 MFMA on 16-bit operands held as raw bits: bf16, or IEEE f16 when
// F16 (the same operand layout; gfx950 has both instructions).
template <bool F16>
__device__ __forceinline__ f32x16_t mma16(const bf16x8_t& a, const bf16x8_t& b, const f32x16_t& c) {
  if constexpr (F16) {
    typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
}

// One 16x16x32 MFMA (bf16, or f16 when F16) accumulating in place.  Lane l of a
// and b holds k 8 (l / 16) .. +8 of row / column l % 16; lane l of c holds rows
// 4 (l / 16) .. +4 of column l % 16.  Written as inline asm: with the builtin the
// register allocator moves 4-register accumulators between MFMAs (dst != srcC) and
// spills a 128 x 64 wave tile at two waves per SIMD.  The compiler then does not
// see these as MFMAs, so the callers keep the MFMA data hazards themselves:
//   * operands come from LDS reads only, waited for with explicit lgkmcnt waits;
//   * accumulators are written only by these MFMAs (zeroed by VALU long before the
//     first one), and read only after mfma_drain();
//   * overwriting an operand register right after the MFMA that reads it is
//     allowed without wait states (the compiler emits that pattern itself for the
//     builtin MFMAs).
template <bool F16>
__device__ __forceinline__ void mma16x32(f32x4_t& c, const bf16x8_t& a, const bf16x8_t& b) {
  if constexpr (F16)
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
  else
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
}
// Waits out the last inline-asm MFMAs' result latency (32 wait states, more than an
// 8-pass MFMA needs before a VALU or memory instruction reads its result) and
// passes every accumulator through an empty volatile asm ordered after the wait, so
// nothing that reads them is scheduled before it.
template <int FM, int FN>
__device__ __forceinline__ void mfma_drain(f32x4_t (&acc)[FM][FN]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) asm volatile("" : "+v"(acc[i][j]));
}

// sched_barrier(0): the machine scheduler moves nothing across this point, so
// the source order of MFMAs, LDS reads and loads is the issue order.
__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

// Epilogue through LDS, shared by all cores.  acc[i][j] holds the transposed
// 32x32 block of wave (wm, wn): lane l, value v -> row m = l % 32, columns
// n = (v / 4) * 8 + (l / 32) * 4 + v % 4 (16x16 blocks, f32x4_t: row l % 16,
// columns 4 (l / 16) + v), so storing it directly writes 16 bytes
// into each of 32 rows per instruction.  Instead the tile is staged in LDS (as
// Epi::Stage values, 16-byte chunk c of row r at slot c ^ (r % chunks-per-row))
// and read back row-wise: each lane takes CH = 16 / sizeof(Stage) consecutive
// columns of one row, so a wave instruction covers whole rows.  Tiles whose stage
// exceeds the main loop's LDS take 2 passes of half the rows.  The epilogue's own
// operands for the next row chunk are fetched (prefetch) before the current chunk
// is stored.
template <int BM, int BN, int WM, int WN, int NB, class Epi, int kLdsHalfwords, class AccV, int FM, int FNB>
__device__ __forceinline__ void tile_epilogue(const GemmParams& p, const Epi& epi, uint16_t (&smem)[kLdsHalfwords],
                                              const AccV (&acc)[FM][FNB], int64_t bb, int64_t m0, int64_t n0,
                                              bool mn_full, int lane, int wm, int wn) {
  constexpr int kLdsBytes = kLdsHalfwords * 2;
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int MB = sizeof(AccV) == 64 ? 32 : 16;  // MFMA block: 32x32 (f32x16_t) or 16x16 (f32x4_t)
  static_assert(sizeof(AccV) == 64 || sizeof(AccV) == 16, "accumulator block");
  constexpr int FN = TN / MB;
  constexpr int NQ = MB == 32 ? 4 : 1;  // 4-value column runs per block and lane
  static_assert(FM == TM / MB && FNB == NB * FN, "accumulator shape");
  using Stage = typename Epi::Stage;
  constexpr int ES = sizeof(Stage);
  constexpr int CH = 16 / ES;
  constexpr int kStageBytes = NB * BM * BN * ES;
  constexpr int P = kStageBytes <= kLdsBytes ? 1 : 2;  // passes
  static_assert(kStageBytes <= P * kLdsBytes && BM % (32 * P) == 0,
                "stage must fit the LDS in at most 2 passes of whole 32-row blocks");
  constexpr int PR = BM / P;          // rows per pass
  constexpr int CPR = BN * ES / 16;   // 16-byte chunks per staged row (per product)
  constexpr int NT = NW * 64;
  static_assert((CPR & (CPR - 1)) == 0 && NT % CPR == 0 && PR % (NT / CPR) == 0, "row-chunk split");
  constexpr int RPI = NT / CPR;  // rows per read iteration
  constexpr int NIT = PR / RPI;  // read iterations per pass
  Stage* stg = reinterpret_cast<Stage*>(smem);
  auto slot = [](int r, int c) { return c ^ (r & (CPR - 1)); };

  auto epilogue = [&](auto full_c) {
    constexpr bool FULL = decltype(full_c)::value;
#pragma unroll
    for (int pass = 0; pass < P; ++pass) {
      // LDS is free: every wave has finished its main-loop reads (or the
      // previous pass's row reads).
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __syncthreads();
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int r = wm * TM + i * MB + (lane & (MB - 1));
        if ((wm * TM + i * MB) / PR != pass) continue;  // uniform over the wave
        const int rl = r - pass * PR;
#pragma unroll
        for (int h = 0; h < NB; ++h)
#pragma unroll
          for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
              const int n = MB == 32 ? wn * TN + j * 32 + q * 8 + (lane >> 5) * 4 : wn * TN + j * 16 + (lane >> 4) * 4;
              Stage w[4];
#pragma unroll
              for (int e = 0; e < 4; ++e) w[e] = Epi::stage(acc[i][h * FN + j][q * 4 + e]);
              const int c = n * ES / 16, off = (n * ES) % 16;
              char* dst = reinterpret_cast<char*>(stg + (h * PR + rl) * BN) + slot(rl, c) * 16 + off;
              if constexpr (ES == 2) {
                struct __attribute__((aligned(8))) W8 { Stage x[4]; };
                *reinterpret_cast<W8*>(dst) = W8{{w[0], w[1], w[2], w[3]}};
              } else {
                struct __attribute__((aligned(16))) W16 { Stage x[4]; };
                *reinterpret_cast<W16*>(dst) = W16{{w[0], w[1], w[2], w[3]}};
              }
            }
      }
      __syncthreads();
      const int t = threadIdx.x;
      const int cl = t % CPR;
      const int64_t n = n0 + cl * CH;
      typename Epi::Pre pre[2];
      auto row_of = [&](int it) { return pass * PR + it * RPI + t / CPR; };
      if (FULL || m0 + row_of(0) < p.M) epi.template prefetch<FULL>(bb, m0 + row_of(0), n, pre[0]);
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        if (it + 1 < NIT && (FULL || m0 + row_of(it + 1) < p.M))
          epi.template prefetch<FULL>(bb, m0 + row_of(it + 1), n, pre[(it + 1) & 1]);
        const int rl = it * RPI + t / CPR;
        const int64_t m = m0 + pass * PR + rl;
        if (!FULL && m >= p.M) continue;
        Stage v0[CH], v1[CH];
        struct __attribute__((aligned(16))) C16 { Stage x[CH]; };
        const C16 a0 = *reinterpret_cast<const C16*>(reinterpret_cast<const char*>(stg + rl * BN) + slot(rl, cl) * 16);
        const C16 a1 = *reinterpret_cast<const C16*>(reinterpret_cast<const char*>(stg + ((NB - 1) * PR + rl) * BN) +
                                                     slot(rl, cl) * 16);
#pragma unroll
        for (int e = 0; e < CH; ++e) {
          v0[e] = a0.x[e];
          v1[e] = a1.x[e];
        }
        epi.template store<FULL>(bb, m, n, v0, v1, pre[it & 1]);
      }
    }
  };
  if (mn_full) epilogue(BoolC<true>{});
  else epilogue(BoolC<false>{});
}

// One BM x BN output tile per workgroup of WM x WN waves.  The epilogue functor:
//   Stage                        how one product value is held in LDS (uint16_t:
//                                bf16 bits; float: fp32)
//   static Stage stage(float)    fp32 accumulator -> staged value
//   Pre, prefetch<FULL>(bb, m, n, Pre&)
//                                loads the epilogue's own operands for a row chunk
//   store<FULL>(bb, m, n, const Stage* v0, const Stage* v1, const Pre&)
//                                finishes CH = 16 / sizeof(Stage) consecutive
//                                outputs (bb, m, n .. n+CH-1) of row m < M: v0 from
//                                A.B, v1 from A.B1 when NB == 2 (else v1 == v0);
//                                FULL: the whole tile lies inside the output (no
//                                column bounds), else columns >= N are ignored.
template <int BM, int BN, int WM, int WN, bool A_K, bool B_K, int NB, class Epi, bool F16 = false, bool BIG = false>
__device__ __forceinline__ void gemm_bf16_body(const GemmParams& p, const Epi& epi) {
  static_assert(NB == 1 || NB == 2, "one or two right operands");
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;  // wave tile (per right operand)
  constexpr int FM = TM / 32, FN = TN / 32;  // 32x32 MFMA blocks per wave
  constexpr int NS = kBK / 16;               // k16 steps per k-tile
  using TA = OperandTile<BM, A_K, NW>;
  using TB = OperandTile<BN, B_K, NW>;
  constexpr int LPW = TA::kPerWave + NB * TB::kPerWave;  // loads per wave per k-tile
  // Two stages of the A and B tiles; after the main loop the same memory stages
  // the output tile for the epilogue.
  constexpr int kLdsBytes = 2 * BM * kBK * 2 + 2 * NB * BN * kBK * 2;
  __shared__ __attribute__((aligned(1024))) uint16_t smem[kLdsBytes / 2];
  uint16_t(*sa)[BM * kBK] = reinterpret_cast<uint16_t(*)[BM * kBK]>(smem);
  uint16_t(*sb)[NB * BN * kBK] = reinterpret_cast<uint16_t(*)[NB * BN * kBK]>(smem + 2 * BM * kBK);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;

  int64_t bb;
  int tm, tn;
  map_tile(blockIdx.x, p.batch * p.tiles_m * p.tiles_n, p.tiles_m, p.tiles_n, bb, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;
  const uint16_t* A0 = static_cast<const uint16_t*>(p.a) + bb * p.sa_b + m0 * p.sa_m;
  const uint16_t* B0 = static_cast<const uint16_t*>(p.b) + bb * p.sb_b + n0 * p.sb_n;
  const uint16_t* B1 = static_cast<const uint16_t*>(NB == 2 ? p.b1 : p.b) + bb * p.sb_b + n0 * p.sb_n;
  const auto a_left0 = ExtSel<BIG>::a(p, m0 * p.sa_m * 2);
  const auto b_left0 = ExtSel<BIG>::b(p, n0 * p.sb_n * 2);

  TA ta;
  TB tb;
  ta.init(wave, lane, p.sa_m, p.sa_k, p.M - m0);
  tb.init(wave, lane, p.sb_n, p.sb_k, p.N - n0);
  const bool mn_full = m0 + BM <= p.M && n0 + BN <= p.N;
  const int KT = static_cast<int>((p.K + kBK - 1) / kBK);

  const uint32_t lds_a = static_cast<uint32_t>(reinterpret_cast<uint64_t>((GHIP_LDS void*)smem));
  const uint32_t lds_b = lds_a + 2 * BM * kBK * 2;
  auto issue = [&](int kt, int st) {
    const int64_t k0 = static_cast<int64_t>(kt) * kBK;
    const int k_left = static_cast<int>(p.K - k0 < kBK ? p.K - k0 : kBK);
    const uint32_t b_left = b_left0.at(k0 * p.sb_k * 2);
    const i32x4_t ra = make_rsrc(A0 + k0 * p.sa_k, a_left0.at(k0 * p.sa_k * 2));
    const i32x4_t rb = make_rsrc(B0 + k0 * p.sb_k, b_left);
    const uint32_t la = lds_a + st * (BM * kBK * 2), lb = lds_b + st * (NB * BN * kBK * 2);
    if (mn_full && k_left == kBK) {
      ta.template issue<true>(ra, la, wave, lane, k_left);
      tb.template issue<true>(rb, lb, wave, lane, k_left);
      if constexpr (NB == 2) tb.template issue<true>(make_rsrc(B1 + k0 * p.sb_k, b_left), lb + BN * kBK * 2, wave, lane, k_left);
    } else {
      ta.template issue<false>(ra, la, wave, lane, k_left);
      tb.template issue<false>(rb, lb, wave, lane, k_left);
      if constexpr (NB == 2)
        tb.template issue<false>(make_rsrc(B1 + k0 * p.sb_k, b_left), lb + BN * kBK * 2, wave, lane, k_left);
    }
  };

  f32x16_t acc[FM][NB * FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < NB * FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  bf16x8_t fa[2][FM], fb[2][NB * FN];
  auto read = [&](int st, int s, int buf) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
      fa[buf][i] = A_K ? frag_kc(sa[st], wm * TM + i * 32, s, lane)
                       : frag_mn<BM>(sa[st], wm * TM + i * 32, s, lane);
#pragma unroll
    for (int h = 0; h < NB; ++h)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        fb[buf][h * FN + j] = B_K ? frag_kc(sb[st] + h * BN * kBK, wn * TN + j * 32, s, lane)
                                  : frag_mn<BN>(sb[st] + h * BN * kBK, wn * TN + j * 32, s, lane);
  };
  auto mfma = [&](int buf) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < NB * FN; ++j)
        acc[i][j] = mma16<F16>(fb[buf][j], fa[buf][i], acc[i][j]);
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

  tile_epilogue<BM, BN, WM, WN, NB>(p, epi, smem, acc, bb, m0, n0, mn_full, lane, wm, wn);
}


// 4-wave core for both operands MN-contiguous (A [K, M], B [K, N] in memory, e.g.
// a weight gradient X^T . dY): one 256 x 256 tile per workgroup of 2 x 2 waves, each
// a 128 x 128 sub-tile (16 32x32 blocks, 256 accumulators per lane, one wave per
// SIMD, which reads a third less LDS per MFMA than 128 x 64 waves).  With one wave
// per SIMD nothing hides a stall, so the issue order is fixed by sched_fence(): the
// MFMAs of a k16 step alternate with the LDS reads of the next step's fragments;
// in the last step of a k-tile half the MFMAs run, then the wait and the barrier,
// then the other half carry the refill loads and the next tile's first reads.
// 32-deep k-tiles in four LDS stages (128 KiB).
// At the barrier that retires tile kt its stage takes tile kt+4, so three tiles of
// MFMA work cover a load; the steady state (every tile has a successor and a tile
// four ahead) runs without runtime branches.  Measured 5% faster than the 64-deep,
// two-stage core for this layout (K-contiguous rows would fetch half cache lines per
// 32-deep tile, which is why the other layouts keep 64).  Bit-identical to the other
// cores: same MFMA, same k order per accumulator.
template <class Epi, bool F16 = false, bool BIG = false>
__device__ __forceinline__ void gemm_bf16_body4mn(const GemmParams& p, const Epi& epi) {
  constexpr int BM = 256, BN = 256, WM = 2, WN = 2, BK = 32, S = 4;
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;
  constexpr int NS = BK / 16;
  using TA = OperandTile<BM, false, NW, BK>;
  using TB = OperandTile<BN, false, NW, BK>;
  constexpr int ND = TA::kPerWave + TB::kPerWave;  // loads per wave per k-tile
  constexpr int kSA = BM * BK * 2, kSB = BN * BK * 2;  // bytes per stage
  constexpr int kLdsBytes = S * (kSA + kSB);
  __shared__ __attribute__((aligned(1024))) uint16_t smem[kLdsBytes / 2];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;

  int64_t bb;
  int tm, tn;
  map_tile(blockIdx.x, p.batch * p.tiles_m * p.tiles_n, p.tiles_m, p.tiles_n, bb, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;
  const uint16_t* A0 = static_cast<const uint16_t*>(p.a) + bb * p.sa_b + m0 * p.sa_m;
  const uint16_t* B0 = static_cast<const uint16_t*>(p.b) + bb * p.sb_b + n0 * p.sb_n;
  const auto a_left0 = ExtSel<BIG>::a(p, m0 * p.sa_m * 2);
  const auto b_left0 = ExtSel<BIG>::b(p, n0 * p.sb_n * 2);

  TA ta;
  TB tb;
  ta.init(wave, lane, p.sa_m, p.sa_k, p.M - m0);
  tb.init(wave, lane, p.sb_n, p.sb_k, p.N - n0);
  const bool mn_full = m0 + BM <= p.M && n0 + BN <= p.N;
  const int KT = static_cast<int>((p.K + BK - 1) / BK);
  const uint32_t lds_a = static_cast<uint32_t>(reinterpret_cast<uint64_t>((GHIP_LDS void*)smem));
  const uint32_t lds_b = lds_a + S * kSA;
  const uint16_t* sA = smem;
  const uint16_t* sB = smem + S * kSA / 2;

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // Fragments [buffer][block][half], two transpose reads per fragment.
  bf16x4_t fa[2][FM][2], fb[2][FN][2];
  constexpr int NR = 2 * (FM + FN);  // LDS reads per k16 step
  auto read_op = [&](int st, int s, int nb, int r) {
    const int blk = r / 4, q = r % 4;
    if (q < 2) fa[nb][blk][q] = frag_mn_half<BM>(sA + st * (kSA / 2), wm * TM + blk * 32, s, lane, q);
    else fb[nb][blk][q - 2] = frag_mn_half<BN>(sB + st * (kSB / 2), wn * TN + blk * 32, s, lane, q - 2);
  };
  auto mfma_op = [&](int b, int k) {
    constexpr int ord[16][2] = {{0, 0}, {0, 1}, {1, 0}, {1, 1}, {0, 2}, {1, 2}, {2, 0}, {2, 1},
                                {2, 2}, {0, 3}, {1, 3}, {2, 3}, {3, 0}, {3, 1}, {3, 2}, {3, 3}};
    const int i = ord[k][0], j = ord[k][1];
    const bf16x8_t av = __builtin_shufflevector(fa[b][i][0], fa[b][i][1], 0, 1, 2, 3, 4, 5, 6, 7);
    const bf16x8_t bv = __builtin_shufflevector(fb[b][j][0], fb[b][j][1], 0, 1, 2, 3, 4, 5, 6, 7);
    acc[i][j] = mma16<F16>(bv, av, acc[i][j]);
  };
  // Wait until at most n k-tiles of this wave's loads are in flight (n wave-uniform).
  auto wait_tiles = [&](int n) {
    if (n >= 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * ND) : "memory");
    else if (n == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(ND) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  };

  auto run = [&](auto full_c) {
    constexpr bool FULL = decltype(full_c)::value;
    auto dma = [&](int kt, int st, int d) {
      const int64_t k0 = static_cast<int64_t>(kt) * BK;
      const int k_left = static_cast<int>(p.K - k0 < BK ? p.K - k0 : BK);
      if (d < TA::kPerWave) {
        const i32x4_t ra = make_rsrc(A0 + k0 * p.sa_k, a_left0.at(k0 * p.sa_k * 2));
        ta.template issue_one<FULL>(ra, lds_a + st * kSA, wave, lane, k_left, d);
      } else {
        const i32x4_t rb = make_rsrc(B0 + k0 * p.sb_k, b_left0.at(k0 * p.sb_k * 2));
        tb.template issue_one<FULL>(rb, lds_b + st * kSB, wave, lane, k_left, d - TA::kPerWave);
      }
    };
    // Prologue: tiles 0 .. S-1 in flight, wait for tile 0.
#pragma unroll
    for (int t = 0; t < S; ++t)
      if (t < KT) {
#pragma unroll
        for (int d = 0; d < ND; ++d) dma(t, t, d);
      }
    wait_tiles(min(S, KT) - 1);
    __syncthreads();
#pragma unroll
    for (int r = 0; r < NR; ++r) read_op(0, 0, 0, r);

    // Tile kt in stage ST; STEADY: tiles kt+1 and kt+S exist (no runtime checks).
    auto tile = [&](int kt, auto st_c, auto steady_c) {
      constexpr int ST = decltype(st_c)::value;
      constexpr int SN = (ST + 1) % S;
      constexpr bool STEADY = decltype(steady_c)::value;
      const bool nx = STEADY || kt + 1 < KT, dm = STEADY || kt + S < KT;
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int b = s & 1;
        if (s + 1 < NS) {
#pragma unroll
          for (int k = 0; k < 16; ++k) {
            mfma_op(b, k);
            if (k < NR) read_op(ST, s + 1, b ^ 1, k);
            sched_fence();
          }
        } else {
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            mfma_op(b, k);
            sched_fence();
          }
          // Tile kt+1 has landed (tiles kt+2 .. kt+S-1 may still be in flight) and
          // every wave is done reading stage ST, so tile kt+S may refill it.
          if (nx) {
            if constexpr (STEADY) asm volatile("s_waitcnt vmcnt(%0)" ::"n"((S - 2) * ND) : "memory");
            else wait_tiles(min(S - 2, KT - kt - 2));
            __syncthreads();
          }
          sched_fence();
#pragma unroll
          for (int k = 8; k < 16; ++k) {
            mfma_op(b, k);
            const int x = k - 8;
            if (dm) {
#pragma unroll
              for (int d = x * ND / 8; d < (x + 1) * ND / 8; ++d) dma(kt + S, ST, d);
            }
            if (nx) {
#pragma unroll
              for (int r = x * NR / 8; r < (x + 1) * NR / 8; ++r) read_op(SN, 0, b ^ 1, r);
            }
            sched_fence();
          }
        }
      }
    };
    int kt = 0;
    for (; kt + 2 * S - 1 < KT; kt += S) {
      tile(kt, IntC<0>{}, BoolC<true>{});
      tile(kt + 1, IntC<1>{}, BoolC<true>{});
      tile(kt + 2, IntC<2>{}, BoolC<true>{});
      tile(kt + 3, IntC<3>{}, BoolC<true>{});
    }
    for (; kt < KT; kt += S) {
      tile(kt, IntC<0>{}, BoolC<false>{});
      if (kt + 1 < KT) tile(kt + 1, IntC<1>{}, BoolC<false>{});
      if (kt + 2 < KT) tile(kt + 2, IntC<2>{}, BoolC<false>{});
      if (kt + 3 < KT) tile(kt + 3, IntC<3>{}, BoolC<false>{});
    }
  };
  if (mn_full && (p.K % BK) == 0) run(BoolC<true>{});
  else run(BoolC<false>{});
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  tile_epilogue<BM, BN, WM, WN, 1>(p, epi, smem, acc, bb, m0, n0, mn_full, lane, wm, wn);
}

// 8-wave core for A K-contiguous and B MN-contiguous (the DotGeneral config, x . W
// with W [K, N] row-major): one 256 x 256 tile per workgroup of 2 x 4 waves (128 x 64
// each, two waves per SIMD), k-steps of 32 with B in four 32-deep LDS stages and A in
// two 64-deep "super-tile" stages (a K-contiguous row of 32 k would fetch half cache
// lines).  B tile kt's stage takes tile kt+4 at the barrier that starts tile kt; the
// A stage of super-tile j (tiles 2j, 2j+1) takes super-tile j+2 at the barrier that
// starts tile 2j+1.  Issue order per barrier: A (at odd tiles), then B; so at the
// barrier of an odd kt, tile kt+1 is complete once all but B kt+2, kt+3 have landed
// (vmcnt 2 NB), at an even kt all but those and A super-tile kt/2+1 (vmcnt 2 NB + NA).
//
// 16x16x32 MFMAs (32 per tile and wave): under the board's power limit the part
// clocks ~10-15% higher running them than 32x32x16 MFMAs of the same work (one
// 16x16 accumulator block moves a quarter of the accumulator data per product), and
// the products come out bit-identical.  A tile's fragments are in registers when it
// starts; its MFMAs run row block by row block, each block's A fragment refilled for
// tile kt+1 right after its last MFMA, and B's in the last block, so one set of
// fragments (48 VGPRs) serves both tiles.  B stages sit below A in LDS, so every
// fragment read is one base register plus an immediate offset.
//
// NP = 2 computes A.B and A.B1 (two products sharing A) on a 256 x (2 x 128) tile:
// each B stage holds the 128 columns of B, then those of B1, and a wave's 128 x 64
// sub-tile is 32 columns of each, so the epilogue finds both values of an output in
// one lane.
template <class Epi, bool F16 = false, int NP = 1, bool BIG = false>
__device__ __forceinline__ void gemm_bf16_body8km(const GemmParams& p, const Epi& epi) {
  static_assert(NP == 1 || NP == 2, "one or two right operands");
  constexpr int BM = 256, BN = 256 / NP, WM = 2, WN = 4, BK = 32;  // BN: per product
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 16, FN = TN / 16, FB = NP * FN;  // 16x16 blocks per wave
  using TA = OperandTile<BM, true, NW, 2 * BK, true>;
  using TB = OperandTile<BN, false, NW, BK, true>;
  constexpr int NA = TA::kPerWave;       // A loads per wave per super-tile
  constexpr int NB = NP * TB::kPerWave;  // B loads per wave per tile
  constexpr int kSA = BM * 2 * BK * 2, kSB1 = BN * BK * 2, kSB = NP * kSB1;  // bytes per stage
  constexpr int kLdsBytes = 4 * kSB + 2 * kSA;
  static_assert(4 * kSB <= 65536 && kSA + TM * 2 * BK * 2 <= 65536, "fragment offsets fit the 16-bit immediate");
  __shared__ __attribute__((aligned(1024))) uint16_t smem[kLdsBytes / 2];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;

  int64_t bb;
  int tm, tn;
  map_tile(blockIdx.x, p.batch * p.tiles_m * p.tiles_n, p.tiles_m, p.tiles_n, bb, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;
  const uint16_t* A0 = static_cast<const uint16_t*>(p.a) + bb * p.sa_b + m0 * p.sa_m;
  const uint16_t* B0 = (NP == 1 && p.groups ? static_cast<const uint16_t*>(pick_group(p.b_g, bb))
                                             : static_cast<const uint16_t*>(p.b) + bb * p.sb_b) +
                       n0 * p.sb_n;
  const uint16_t* B1 = static_cast<const uint16_t*>(NP == 2 ? p.b1 : p.b) + bb * p.sb_b + n0 * p.sb_n;
  const auto a_left0 = ExtSel<BIG>::a(p, m0 * p.sa_m * 2);
  const auto b_left0 = ExtSel<BIG>::b(p, n0 * p.sb_n * 2);

  TA ta;
  TB tb;
  ta.init(wave, lane, p.sa_m, p.sa_k, p.M - m0);
  tb.init(wave, lane, p.sb_n, p.sb_k, p.N - n0);
  const bool mn_full = m0 + BM <= p.M && n0 + BN <= p.N;
  const int KT = static_cast<int>((p.K + BK - 1) / BK);  // 32-deep tiles
  const int KS = (KT + 1) / 2;                             // 64-deep A super-tiles
  const uint32_t lds_b = static_cast<uint32_t>(reinterpret_cast<uint64_t>((GHIP_LDS void*)smem));
  const uint32_t lds_a = lds_b + 4 * kSB;

  f32x4_t acc[FM][FB];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FB; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[i][j][v] = 0.f;

  // Per-lane LDS base pointers (address space 3, so stage and block offsets fold
  // into the reads' immediate offsets): A per block parity and k32 step as (0, 1)
  // of a super-tile (the KC16 layout: lane l reads LDS row 32 (b / 2) + 2 (l % 16) +
  // (l / 16) % 2, chunk 4 (b % 2) + 2 as + l / 32 for block b), B per column block (the swizzle
  // mixes the block's chunk bits; lane l: column l % 16 of the block, k-rows
  // 8 (l / 16) + (l % 16) / 4 and + 4 for the two transpose reads).
  typedef GHIP_LDS const uint16_t* lds_p;
  lds_p const lds0 = (lds_p)((GHIP_LDS void*)smem);
  lds_p abase[2][2], bbase[FN];
#pragma unroll
  for (int par = 0; par < 2; ++par)
#pragma unroll
    for (int as = 0; as < 2; ++as) {
      const int rho = wm * TM + 2 * (lane & 15) + ((lane >> 4) & 1);
      abase[par][as] = lds0 + 2 * kSB + rho * (2 * BK) + (((4 * par + 2 * as + (lane >> 5)) ^ swz_k(rho)) * 8);
    }
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int kl = 8 * (lane >> 4) + ((lane & 15) >> 2);
    const int nl = wn * TN + j * 16 + 4 * (lane & 3);
    bbase[j] = lds0 + kl * BN + (((nl >> 3) ^ swz_n2(kl)) * 8) + (nl & 7);
  }
  bf16x8_t fa[FM], fb[FB];
  auto read_a = [&](int i, int sa, int as) {  // row block i from A stage sa, k32 step as
    fa[i] = *(GHIP_LDS const bf16x8_t*)(abase[i & 1][as] + sa * (kSA / 2) + (i >> 1) * 32 * (2 * BK));
  };
  auto read_b = [&](int jj, int sb) {  // column block jj (product jj / FN) from B stage sb
    lds_p p0 = bbase[jj % FN] + sb * (kSB / 2) + (jj / FN) * (kSB1 / 2);
    const bf16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((GHIP_LDS bf16x4_t*)(p0));
    const bf16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((GHIP_LDS bf16x4_t*)(p0 + 4 * BN));
    fb[jj] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  };

  auto run = [&](auto full_c) {
    constexpr bool FULL = decltype(full_c)::value;
    auto issue_a = [&](int j) {  // A super-tile j (k 64j ..) into A stage j % 2
      if (j < KS) {
        const int64_t k0 = static_cast<int64_t>(j) * 2 * BK;
        const int k_left = static_cast<int>(p.K - k0 < 2 * BK ? p.K - k0 : 2 * BK);
        const i32x4_t ra = make_rsrc(A0 + k0 * p.sa_k, a_left0.at(k0 * p.sa_k * 2));
#pragma unroll
        for (int d = 0; d < NA; ++d) ta.template issue_one<FULL>(ra, lds_a + (j & 1) * kSA, wave, lane, k_left, d);
      }
    };
    auto issue_b = [&](int t) {  // B tile t into B stage t % 4
      if (t < KT) {
        const int64_t k0 = static_cast<int64_t>(t) * BK;
        const int k_left = static_cast<int>(p.K - k0 < BK ? p.K - k0 : BK);
        const uint32_t b_left = b_left0.at(k0 * p.sb_k * 2);
        const i32x4_t rb = make_rsrc(B0 + k0 * p.sb_k, b_left);
#pragma unroll
        for (int d = 0; d < TB::kPerWave; ++d)
          tb.template issue_one<FULL>(rb, lds_b + (t & 3) * kSB, wave, lane, k_left, d);
        if constexpr (NP == 2) {
          const i32x4_t rb1 = make_rsrc(B1 + k0 * p.sb_k, b_left);
#pragma unroll
          for (int d = 0; d < TB::kPerWave; ++d)
            tb.template issue_one<FULL>(rb1, lds_b + (t & 3) * kSB + kSB1, wave, lane, k_left, d);
        }
      }
    };
    // Prologue in the steady state's issue order (as if barriers -4 .. -1 had run).
    issue_b(0);
    issue_a(0);
    issue_b(1);
    issue_b(2);
    issue_a(1);
    issue_b(3);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
#pragma unroll
    for (int j = 0; j < FB; ++j) read_b(j, 0);
#pragma unroll
    for (int i = 0; i < FM; ++i) read_a(i, 0, 0);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

    // Tile kt (B stage ST = kt % 4, A stage ST / 2, k32 step ST % 2 of the
    // super-tile), fragments in registers.  STEADY: tiles kt+1 and kt+4 exist.
    auto tile = [&](int kt, auto st_c, auto steady_c) {
      constexpr int ST = decltype(st_c)::value;
      constexpr int SN = (ST + 1) % 4;
      constexpr bool STEADY = decltype(steady_c)::value;
      const bool nx = STEADY || kt + 1 < KT;
      if (nx) {
        if constexpr (STEADY) {
          if constexpr (ST % 2 == 1)
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(%0)" ::"n"(2 * NB) : "memory");
          else
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(%0)" ::"n"(2 * NB + NA) : "memory");
        } else {
          asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(0)" ::: "memory");
        }
        // Every wave holds tile kt's fragments: its B stage (and after an odd kt
        // its A stage) is free; tile kt+1 is visible to all.
        __syncthreads();
        if constexpr (ST % 2 == 1) {
          if (STEADY || (kt + 3) / 2 < KS) issue_a(kt / 2 + 2);
        }
        if (STEADY || kt + 4 < KT) issue_b(kt + 4);
      }
#pragma unroll
      for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FB; ++j) {
          mma16x32<F16>(acc[i][j], fb[j], fa[i]);
          if (i == FM - 1 && nx) read_b(j, SN);
        }
        if (nx) read_a(i, SN / 2, SN % 2);
      }
    };
    int kt = 0;
    for (; kt + 7 < KT; kt += 4) {
      tile(kt, IntC<0>{}, BoolC<true>{});
      tile(kt + 1, IntC<1>{}, BoolC<true>{});
      tile(kt + 2, IntC<2>{}, BoolC<true>{});
      tile(kt + 3, IntC<3>{}, BoolC<true>{});
    }
    for (; kt < KT; kt += 4) {
      tile(kt, IntC<0>{}, BoolC<false>{});
      if (kt + 1 < KT) tile(kt + 1, IntC<1>{}, BoolC<false>{});
      if (kt + 2 < KT) tile(kt + 2, IntC<2>{}, BoolC<false>{});
      if (kt + 3 < KT) tile(kt + 3, IntC<3>{}, BoolC<false>{});
    }
  };
  if (mn_full && (p.K % (2 * BK)) == 0) run(BoolC<true>{});
  else run(BoolC<false>{});
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  mfma_drain(acc);

  tile_epilogue<BM, BN, WM, WN, NP>(p, epi, smem, acc, bb, m0, n0, mn_full, lane, wm, wn);
}

// One 16x16x32 MFMA accumulating in place in AGPRs (the 4-wave cores keep 256
// accumulators a lane); otherwise as mma16x32.
template <bool F16>
__device__ __forceinline__ void mma16x32a(f32x4_t& c, const bf16x8_t& a, const bf16x8_t& b) {
  if constexpr (F16)
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
  else
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}
template <int FM, int FN>
__device__ __forceinline__ void mfma_drain_a(f32x4_t (&acc)[FM][FN]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) asm volatile("" : "+a"(acc[i][j]));
}

// 4-wave core for A K-contiguous and B MN-contiguous (the DotGeneral config): one
// 256 x 256 tile per workgroup of 2 x 2 waves, each 128 x 128 (64 16x16x32 MFMAs per
// k32 step, 256 accumulators a lane in AGPRs, one wave per SIMD).  A wave reads 16
// fragments per 64 MFMAs from LDS, a third less than the 8-wave core's 128 x 64
// waves (12 per 32), for the same DMA traffic; under the board's power limit the
// LDS bytes are energy the MFMAs do not get.
//
// LDS staging as in gemm_bf16_body8km (B in four 32-deep stages, A in two 64-deep
// super-tile stages; the A DMA interleaves the waves so each instruction fills one
// 32-row group).  With one wave per SIMD nothing hides a stall, so the issue order is
// fixed (sched_fence) and no wait sits where the MFMA queue would drain:
//   * tile kt's fragments are in registers when it starts (A rolling: fa[i] is
//     refilled for tile kt+1 right after row block i's last MFMA; B double-buffered);
//   * the wait and barrier of tile kt come after its first two row blocks: by then
//     this wave's reads of stage kt (issued during tile kt-1) have completed, and
//     the wait for tile kt+1's DMA (issued three tiles earlier) is normally a no-op;
//   * after the barrier, stage kt takes tile kt+4 (and an odd kt's A stage the
//     super-tile two ahead) by DMA spread over the remaining MFMAs, and tile kt+1's
//     B fragments are read, two per row block.
// DMA issue order per tile is A (odd tiles) then B, as in gemm_bf16_body8km, so the
// same vmcnt counts hold.  Bit-identical to the other cores (same MFMA, same k order
// per accumulator).
//
// NP = 2 computes A.B and A.B1 (two products sharing A) on a 256 x (2 x 128) tile,
// as gemm_bf16_body8km does: each B stage holds 128 columns of B, then those of B1,
// and a wave's 128 x 128 sub-tile is 64 columns of each.
template <class Epi, bool F16 = false, int NP = 1, bool BIG = false>
__device__ __forceinline__ void gemm_bf16_body4km(const GemmParams& p, const Epi& epi) {
  static_assert(NP == 1 || NP == 2, "one or two right operands");
  constexpr int BM = 256, BN = 256 / NP, WM = 2, WN = 2, BK = 32;  // BN: per product
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 16, FN = TN / 16, FB = NP * FN;  // 8 x 8 blocks of 16 x 16
  using TA = OperandTile<BM, true, NW, 2 * BK, true, true>;
  using TB = OperandTile<BN, false, NW, BK, true>;
  constexpr int NA = TA::kPerWave;          // A loads per wave per super-tile (8)
  constexpr int NBP = TB::kPerWave;         // B loads per wave per tile and product
  constexpr int NB = NP * NBP;              // B loads per wave per tile (4)
  constexpr int kSA = BM * 2 * BK * 2, kSB1 = BN * BK * 2, kSB = NP * kSB1;  // bytes per stage
  constexpr int kLdsBytes = 4 * kSB + 2 * kSA;
  static_assert(4 * kSB <= 65536 && kSA + TM * 2 * BK * 2 <= 65536, "fragment offsets fit the 16-bit immediate");
  static_assert(NA + NB <= 12 && FM == 8 && FB == 8, "DMA slots of one tile");
  __shared__ __attribute__((aligned(1024))) uint16_t smem[kLdsBytes / 2];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;

  int64_t bb;
  int tm, tn;
  map_tile(blockIdx.x, p.batch * p.tiles_m * p.tiles_n, p.tiles_m, p.tiles_n, bb, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;
  const uint16_t* A0 = static_cast<const uint16_t*>(p.a) + bb * p.sa_b + m0 * p.sa_m;
  const uint16_t* B0 = (NP == 1 && p.groups ? static_cast<const uint16_t*>(pick_group(p.b_g, bb))
                                             : static_cast<const uint16_t*>(p.b) + bb * p.sb_b) +
                       n0 * p.sb_n;
  const uint16_t* B1 = static_cast<const uint16_t*>(NP == 2 ? p.b1 : p.b) + bb * p.sb_b + n0 * p.sb_n;
  const auto a_left0 = ExtSel<BIG>::a(p, m0 * p.sa_m * 2);
  const auto b_left0 = ExtSel<BIG>::b(p, n0 * p.sb_n * 2);

  TA ta;
  TB tb;
  ta.init(wave, lane, p.sa_m, p.sa_k, p.M - m0);
  tb.init(wave, lane, p.sb_n, p.sb_k, p.N - n0);
  const bool mn_full = m0 + BM <= p.M && n0 + BN <= p.N;
  const int KT = static_cast<int>((p.K + BK - 1) / BK);  // 32-deep tiles
  const int KS = (KT + 1) / 2;                             // 64-deep A super-tiles
  const uint32_t lds_b = static_cast<uint32_t>(reinterpret_cast<uint64_t>((GHIP_LDS void*)smem));
  const uint32_t lds_a = lds_b + 4 * kSB;

  f32x4_t acc[FM][FB];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FB; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[i][j][v] = 0.f;

  // Per-lane LDS base pointers, as in gemm_bf16_body8km.
  typedef GHIP_LDS const uint16_t* lds_p;
  lds_p const lds0 = (lds_p)((GHIP_LDS void*)smem);
  lds_p abase[2][2], bbase[FN];
#pragma unroll
  for (int par = 0; par < 2; ++par)
#pragma unroll
    for (int as = 0; as < 2; ++as) {
      const int rho = wm * TM + 2 * (lane & 15) + ((lane >> 4) & 1);
      abase[par][as] = lds0 + 2 * kSB + rho * (2 * BK) + (((4 * par + 2 * as + (lane >> 5)) ^ swz_k(rho)) * 8);
    }
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int kl = 8 * (lane >> 4) + ((lane & 15) >> 2);
    const int nl = wn * TN + j * 16 + 4 * (lane & 3);
    bbase[j] = lds0 + kl * BN + (((nl >> 3) ^ swz_n2(kl)) * 8) + (nl & 7);
  }
  bf16x8_t fa[FM], fb[2][FB];
  auto read_a = [&](int i, int sa, int as) {  // row block i from A stage sa, k32 step as
    fa[i] = *(GHIP_LDS const bf16x8_t*)(abase[i & 1][as] + sa * (kSA / 2) + (i >> 1) * 32 * (2 * BK));
  };
  auto read_b = [&](int buf, int jj, int sb) {  // column block jj (product jj / FN) from B stage sb
    lds_p p0 = bbase[jj % FN] + sb * (kSB / 2) + (jj / FN) * (kSB1 / 2);
    const bf16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((GHIP_LDS bf16x4_t*)(p0));
    const bf16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((GHIP_LDS bf16x4_t*)(p0 + 4 * BN));
    fb[buf][jj] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  };

  auto run = [&](auto full_c) {
    constexpr bool FULL = decltype(full_c)::value;
    auto dma_a = [&](int j, int d) {  // instruction d of A super-tile j (k 64j ..) into A stage j % 2
      const int64_t k0 = static_cast<int64_t>(j) * 2 * BK;
      const int k_left = static_cast<int>(p.K - k0 < 2 * BK ? p.K - k0 : 2 * BK);
      const i32x4_t ra = make_rsrc(A0 + k0 * p.sa_k, a_left0.at(k0 * p.sa_k * 2));
      ta.template issue_one<FULL>(ra, lds_a + (j & 1) * kSA, wave, lane, k_left, d);
    };
    auto dma_b = [&](int t, int d) {  // instruction d of B tile t into B stage t % 4 (d / NBP: product)
      const int64_t k0 = static_cast<int64_t>(t) * BK;
      const int k_left = static_cast<int>(p.K - k0 < BK ? p.K - k0 : BK);
      const uint16_t* Bp = (NP == 2 && d >= NBP) ? B1 : B0;
      const i32x4_t rb = make_rsrc(Bp + k0 * p.sb_k, b_left0.at(k0 * p.sb_k * 2));
      tb.template issue_one<FULL>(rb, lds_b + (t & 3) * kSB + (d / NBP) * kSB1, wave, lane, k_left, d % NBP);
    };
    auto issue_a = [&](int j) {
      if (j < KS) {
#pragma unroll
        for (int d = 0; d < NA; ++d) dma_a(j, d);
      }
    };
    auto issue_b = [&](int t) {
      if (t < KT) {
#pragma unroll
        for (int d = 0; d < NB; ++d) dma_b(t, d);
      }
    };
    // Prologue in the steady state's issue order (as if barriers -4 .. -1 had run).
    issue_b(0);
    issue_a(0);
    issue_b(1);
    issue_b(2);
    issue_a(1);
    issue_b(3);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
#pragma unroll
    for (int j = 0; j < FB; ++j) read_b(0, j, 0);
#pragma unroll
    for (int i = 0; i < FM; ++i) read_a(i, 0, 0);

    // Tile kt (B stage ST = kt % 4, A stage ST / 2, k32 step ST % 2 of the
    // super-tile; B fragments in fb[ST % 2]).  STEADY: tiles kt+1 and kt+4 exist.
    auto tile = [&](int kt, auto st_c, auto steady_c) {
      constexpr int ST = decltype(st_c)::value;
      constexpr int SN = (ST + 1) % 4;
      constexpr int CB = ST & 1;
      constexpr bool STEADY = decltype(steady_c)::value;
      const bool nx = STEADY || kt + 1 < KT;
      const bool do_b = STEADY || kt + 4 < KT;
      const bool do_a = ST % 2 == 1 && (STEADY || (kt + 3) / 2 < KS);
      constexpr int ND = (ST % 2 == 1 ? NA : 0) + NB;  // DMA instructions of this tile
#pragma unroll
      for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FB; ++j) {
          mma16x32a<F16>(acc[i][j], fb[CB][j], fa[i]);
          if (i >= 2 && nx) {
            // After the barrier: one DMA instruction every 4th MFMA, tile kt+1's B
            // fragments two per row block (rows 2-5).
            const int q = (i - 2) * FB + j;  // 0 .. 47
            if (q % 4 == 0 && q / 4 < ND) {
              const int d = q / 4;
              if (ST % 2 == 1 && d < NA) {
                if (do_a) dma_a(kt / 2 + 2, d);
              } else if (do_b) {
                dma_b(kt + 4, ST % 2 == 1 ? d - NA : d);
              }
            }
            if (q % 4 == 2 && q / 4 < FB) read_b(CB ^ 1, q / 4, SN);
          }
          sched_fence();
        }
        if (i == 1 && nx) {
          // Tile kt+1 has landed (this wave's loads, then everyone's through the
          // barrier), and every wave has finished reading stage ST (its fragments
          // were read during tile kt-1), which may now be refilled.
          if constexpr (STEADY) {
            if constexpr (ST % 2 == 1)
              asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(%0)" ::"n"(2 * NB) : "memory");
            else
              asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(%0)" ::"n"(2 * NB + NA) : "memory");
          } else {
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(0)" ::: "memory");
          }
          __syncthreads();
          read_a(0, SN / 2, SN % 2);
          read_a(1, SN / 2, SN % 2);
          sched_fence();
        }
        if (i >= 2 && nx) {
          read_a(i, SN / 2, SN % 2);
          sched_fence();
        }
      }
    };
    int kt = 0;
    for (; kt + 7 < KT; kt += 4) {
      tile(kt, IntC<0>{}, BoolC<true>{});
      tile(kt + 1, IntC<1>{}, BoolC<true>{});
      tile(kt + 2, IntC<2>{}, BoolC<true>{});
      tile(kt + 3, IntC<3>{}, BoolC<true>{});
    }
    for (; kt < KT; kt += 4) {
      tile(kt, IntC<0>{}, BoolC<false>{});
      if (kt + 1 < KT) tile(kt + 1, IntC<1>{}, BoolC<false>{});
      if (kt + 2 < KT) tile(kt + 2, IntC<2>{}, BoolC<false>{});
      if (kt + 3 < KT) tile(kt + 3, IntC<3>{}, BoolC<false>{});
    }
  };
  if (mn_full && (p.K % (2 * BK)) == 0) run(BoolC<true>{});
  else run(BoolC<false>{});
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  mfma_drain_a(acc);

  tile_epilogue<BM, BN, WM, WN, NP>(p, epi, smem, acc, bb, m0, n0, mn_full, lane, wm, wn);
}

// 8-wave 16x16x32 core for any operand layout (the A K-contiguous / B MN-contiguous
// one has its own deeper pipeline, gemm_bf16_body8km): one 256 x 256 tile (256 x
// (2 x 128) for NP = 2, as there) per workgroup of 2 x 4 waves, 64-deep k-tiles in
// two LDS stages, two k32 steps per tile.  Fragments roll as in gemm_bf16_body8km:
// step 0 of tile kt reads step 1 of the same stage; then wait for tile kt+1, barrier
// (stage kt % 2 is free), refill it with tile kt+2, and step 1 reads step 0 of tile
// kt+1.  MN-contiguous tiles use swz_n2.  Bit-identical to the other cores; in one
// process at the config shape 2-3% faster than the 4-wave 32x32x16 cores for B
// K-contiguous layouts (and 4-6% on [8192,2048].[2048,2048]), 4-5% faster than the
// 8-wave 32x32x16 64-deep core for two products and heavy epilogues, 4% slower than
// the 4-wave 32-deep core when both operands are MN-contiguous.
template <bool A_K, bool B_K, class Epi, bool F16 = false, int NP = 1, bool BIG = false>
__device__ __forceinline__ void gemm_bf16_body8x(const GemmParams& p, const Epi& epi) {
  static_assert(NP == 1 || NP == 2, "one or two right operands");
  constexpr int BM = 256, BN = 256 / NP, WM = 2, WN = 4, BK = kBK;
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 16, FN = TN / 16, FB = NP * FN;
  using TA = OperandTile<BM, A_K, NW, BK, true>;
  using TB = OperandTile<BN, B_K, NW, BK, true>;
  constexpr int kSA = BM * BK * 2, kSB1 = BN * BK * 2, kSB = NP * kSB1;  // bytes per stage
  constexpr int kLdsBytes = 2 * kSA + 2 * kSB;
  __shared__ __attribute__((aligned(1024))) uint16_t smem[kLdsBytes / 2];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;

  int64_t bb;
  int tm, tn;
  map_tile(blockIdx.x, p.batch * p.tiles_m * p.tiles_n, p.tiles_m, p.tiles_n, bb, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn) * BN;
  const uint16_t* A0 = static_cast<const uint16_t*>(p.a) + bb * p.sa_b + m0 * p.sa_m;
  const uint16_t* B0 = (NP == 1 && p.groups ? static_cast<const uint16_t*>(pick_group(p.b_g, bb))
                                             : static_cast<const uint16_t*>(p.b) + bb * p.sb_b) +
                       n0 * p.sb_n;
  const uint16_t* B1 = static_cast<const uint16_t*>(NP == 2 ? p.b1 : p.b) + bb * p.sb_b + n0 * p.sb_n;
  const auto a_left0 = ExtSel<BIG>::a(p, m0 * p.sa_m * 2);
  const auto b_left0 = ExtSel<BIG>::b(p, n0 * p.sb_n * 2);

  TA ta;
  TB tb;
  ta.init(wave, lane, p.sa_m, p.sa_k, p.M - m0);
  tb.init(wave, lane, p.sb_n, p.sb_k, p.N - n0);
  const bool mn_full = m0 + BM <= p.M && n0 + BN <= p.N;
  const int KT = static_cast<int>((p.K + BK - 1) / BK);
  const uint32_t lds_a = static_cast<uint32_t>(reinterpret_cast<uint64_t>((GHIP_LDS void*)smem));
  const uint32_t lds_b = lds_a + 2 * kSA;

  f32x4_t acc[FM][FB];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FB; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[i][j][v] = 0.f;

  typedef GHIP_LDS const uint16_t* lds_p;
  lds_p const ldsA = (lds_p)((GHIP_LDS void*)smem);
  lds_p const ldsB = ldsA + kSA;  // halfwords: after the two A stages
  // Per-lane LDS base pointers (address space 3, so stage, step and block offsets
  // fold into the reads' immediate offsets): a K-contiguous operand (KC16 layout)
  // has one per block parity and k32 step (lane l reads LDS row 32 (b / 2) +
  // 2 (l % 16) + (l / 16) % 2, chunk 4 (b % 2) + 2 s + l / 32 for block b), an
  // MN-contiguous one ([64][R]) one
  // per block (the swizzle mixes the block's chunk bits; lane l: column l % 16,
  // k-rows 8 (l / 16) + (l % 16) / 4 and + 4).
  constexpr int NBA = A_K ? 4 : FM, NBB = B_K ? 4 : FN;
  lds_p abase[NBA], bbase[NBB];
#pragma unroll
  for (int q = 0; q < NBA; ++q) {
    if constexpr (A_K) {
      const int rho = wm * TM + 2 * (lane & 15) + ((lane >> 4) & 1);
      abase[q] = ldsA + rho * BK + (((4 * (q >> 1) + 2 * (q & 1) + (lane >> 5)) ^ swz_k(rho)) * 8);
    } else {
      const int kl = 8 * (lane >> 4) + ((lane & 15) >> 2);
      const int nl = wm * TM + q * 16 + 4 * (lane & 3);
      abase[q] = ldsA + kl * BM + (((nl >> 3) ^ swz_n2(kl)) * 8) + (nl & 7);
    }
  }
#pragma unroll
  for (int q = 0; q < NBB; ++q) {
    if constexpr (B_K) {
      const int rho = wn * TN + 2 * (lane & 15) + ((lane >> 4) & 1);
      bbase[q] = ldsB + rho * BK + (((4 * (q >> 1) + 2 * (q & 1) + (lane >> 5)) ^ swz_k(rho)) * 8);
    } else {
      const int kl = 8 * (lane >> 4) + ((lane & 15) >> 2);
      const int nl = wn * TN + q * 16 + 4 * (lane & 3);
      bbase[q] = ldsB + kl * BN + (((nl >> 3) ^ swz_n2(kl)) * 8) + (nl & 7);
    }
  }
  bf16x8_t fa[FM], fb[FB];
  auto rd_tr = [](lds_p p0, int R) {
    const bf16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((GHIP_LDS bf16x4_t*)(p0));
    const bf16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((GHIP_LDS bf16x4_t*)(p0 + 4 * R));
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  };
  // block i of A / jj of B at k32 step s (0, 1) of stage st
  auto read_a = [&](int i, int st, int s) {
    if constexpr (A_K) fa[i] = *(GHIP_LDS const bf16x8_t*)(abase[2 * (i & 1) + s] + st * (kSA / 2) + (i >> 1) * 32 * BK);
    else fa[i] = rd_tr(abase[i] + st * (kSA / 2) + s * 32 * BM, BM);
  };
  auto read_b = [&](int jj, int st, int s) {
    const int h = jj / FN, j = jj % FN;
    if constexpr (B_K)
      fb[jj] = *(GHIP_LDS const bf16x8_t*)(bbase[2 * (j & 1) + s] + st * (kSB / 2) + h * (kSB1 / 2) + (j >> 1) * 32 * BK);
    else fb[jj] = rd_tr(bbase[j] + st * (kSB / 2) + h * (kSB1 / 2) + s * 32 * BN, BN);
  };

  auto run = [&](auto full_c) {
    constexpr bool FULL = decltype(full_c)::value;
    auto issue = [&](int kt, int st) {
      const int64_t k0 = static_cast<int64_t>(kt) * BK;
      const int k_left = static_cast<int>(p.K - k0 < BK ? p.K - k0 : BK);
      const i32x4_t ra = make_rsrc(A0 + k0 * p.sa_k, a_left0.at(k0 * p.sa_k * 2));
#pragma unroll
      for (int d = 0; d < TA::kPerWave; ++d) ta.template issue_one<FULL>(ra, lds_a + st * kSA, wave, lane, k_left, d);
      const uint32_t b_left = b_left0.at(k0 * p.sb_k * 2);
      const i32x4_t rb = make_rsrc(B0 + k0 * p.sb_k, b_left);
#pragma unroll
      for (int d = 0; d < TB::kPerWave; ++d) tb.template issue_one<FULL>(rb, lds_b + st * kSB, wave, lane, k_left, d);
      if constexpr (NP == 2) {
        const i32x4_t rb1 = make_rsrc(B1 + k0 * p.sb_k, b_left);
#pragma unroll
        for (int d = 0; d < TB::kPerWave; ++d)
          tb.template issue_one<FULL>(rb1, lds_b + st * kSB + kSB1, wave, lane, k_left, d);
      }
    };
    issue(0, 0);
    if (KT > 1) issue(1, 1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
#pragma unroll
    for (int j = 0; j < FB; ++j) read_b(j, 0, 0);
#pragma unroll
    for (int i = 0; i < FM; ++i) read_a(i, 0, 0);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

    // MFMAs of the fragments in registers, reading (row block by row block, B in
    // the last one) the fragments of k32 step s of stage st when rd.
    auto step = [&](bool rd, int st, int s) {
#pragma unroll
      for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FB; ++j) {
          mma16x32<F16>(acc[i][j], fb[j], fa[i]);
          if (i == FM - 1 && rd) read_b(j, st, s);
        }
        if (rd) read_a(i, st, s);
      }
    };
    // Tile kt in stage ST: step 0 (reading step 1 of ST), then wait for tile kt+1,
    // barrier (stage ST is free: every wave holds step 1's fragments), refill ST
    // with tile kt+2, step 1 (reading step 0 of tile kt+1).
    auto tile = [&](int kt, auto st_c) {
      constexpr int ST = decltype(st_c)::value;
      const bool nx = kt + 1 < KT;
      step(true, ST, 1);
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(0)" ::: "memory");
      if (nx) {
        __syncthreads();
        if (kt + 2 < KT) issue(kt + 2, ST);
      }
      step(nx, ST ^ 1, 0);
    };
    for (int kt = 0; kt < KT; kt += 2) {
      tile(kt, IntC<0>{});
      if (kt + 1 < KT) tile(kt + 1, IntC<1>{});
    }
  };
  if (mn_full && (p.K % BK) == 0) run(BoolC<true>{});
  else run(BoolC<false>{});
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  mfma_drain(acc);
  tile_epilogue<BM, BN, WM, WN, NP>(p, epi, smem, acc, bb, m0, n0, mn_full, lane, wm, wn);
}

#endif  // __HIP__ || __HIPCC_RTC__

}  // namespace ghip

#endif  // GHIP_GEMM_BF16_DEV_H
