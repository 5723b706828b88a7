// Large-M kernel: LDS double-buffered MFMA GEMM for gfx950.
//
//   C[M][N] = epilogue( sum_k A[m][k] * B[n][k] )
//
// Workgroup tile BM x BN, K tile 128.  WM x WN waves; each wave owns a (BM/WM) x (BN/WN)
// block of 16x16 MFMA tiles.  Operands go global -> LDS with the gfx950 LDS-DMA load
// (buffer_load_dwordx4 ... lds: each lane fetches 16 bytes from its own offset and the wave
// writes 64 x 16 contiguous bytes of LDS), so no registers are spent on staging.  Two LDS
// stages (ping/pong): while the MFMAs consume one stage the DMA of the next K tile fills
// the other.  One barrier per K tile.  The grid is persistent (about one workgroup per CU
// slot); each workgroup walks its tiles as one continuous pipeline.
//
// LDS per stage:
//   A: row-major [BM][128 B]; the 16-byte chunk c of row r sits at chunk slot
//      c ^ ((r >> 1) & 7).  One DMA instruction fills 8 rows (1 KB): lane l brings the
//      chunk that belongs in slot (l % 8) of row (l / 8), so each wave load reads eight
//      whole 128-byte row segments of A, and the 16 lanes that later read one chunk column
//      of 16 consecutive rows hit 16 distinct 16-byte bank groups (64 banks x 4 B).
//   B: the preshuffled bytes copied verbatim: per 16-column block a 2 KB run
//      [chunk 0..7][col 0..15][16 B] (INT4: 1 KB [chunk][col][8 B]); lanes that read one
//      chunk read 256 (128) contiguous bytes.
//   Scales of the K tile, when the kernel has per-K-tile scales (blockscale, MXFP4), after B:
//      they travel with the tile through the same DMA and barrier, so no separate vector
//      memory load has to be waited for inside a step (such a wait would also drain the
//      next step's DMA, which vector memory counters track in issue order).
//      Blockscale: A's BM fp32 scales of the tile (x_scale_t[kt][m0..], 4-byte DMA, since
//      those rows need not be 16-byte aligned), then w_scale[n/128][kt] of each 128-column
//      block.  MXFP4: the 256-byte lane-word block of every 32-row group of A, then of every
//      32-column group of B (16-byte DMA).
#pragma once
#include "gemm_common.h"

#ifndef FLY_SCHED
#define FLY_SCHED 1
#endif
#ifndef FLY_GROUP_M
#define FLY_GROUP_M 8
#endif
#ifndef FLY_ROLES
#define FLY_ROLES 1
#endif

namespace flygemm {

template <int BM, int BN, int WM, int WN, int KIND>
struct MainCfg {
  static constexpr int NW = WM * WN;
  static constexpr int NT = NW * 64;
  static constexpr int TM = BM / WM;
  static constexpr int TN = BN / WN;
  static constexpr int MR = TM / 16;
  static constexpr int NR = TN / 16;
  static constexpr int A_BYTES = BM * KT;
  static constexpr int B_BLK = (KIND == KIND_INT4) ? 1024 : 2048;  // bytes per 16 cols per K tile
  static constexpr int B_BYTES = (BN / 16) * B_BLK;
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int A_DMA = A_BYTES / 1024 / NW;  // 1 KB DMA instructions per wave per tile
  static constexpr int B_DMA = B_BYTES / 1024 / NW;
  // LDS stages: three for the 4-wave tiles of at most 64x128 outputs (short steps) and for the
  // 8-wave 128x256 / 256x128 tiles (3 x 48 KB plus scales fits the 160 KB), else two.
  // Measured on MI355X: the third stage saves 4-18% on the 4-wave tiles for fp8/int8 shapes
  // from 128x4096x4096 to 1024x7168x7168 and 10-25% on the 8-wave ones for fp8, int8, bf16,
  // MXFP4 and blockscale (1024x7168x7168 fp8 with 128x256 tiles: 58.3 us against 70.9), but
  // costs 12-15% on int4 (W4A8 256x14336x4096 with 64x128 tiles, 1024x14336x4096 with
  // 256x128), whose half-size B steps are not waiting on their DMA.
  static constexpr int NS =
      (KIND != KIND_INT4 && ((NW == 4 && BM * BN <= 64 * 128) || (NW == 8 && BM * BN == 256 * 128))) ? 3 : 2;
  static constexpr int DMA_PER_STEP = A_DMA + B_DMA;  // per wave, scale DMAs not counted
  static_assert(TM % 16 == 0 && TN % 16 == 0, "wave tile must be a multiple of 16");
  static_assert(A_BYTES % (1024 * NW) == 0 && B_BYTES % (1024 * NW) == 0, "tile not divisible into wave DMAs");
};

// Tile index -> (tile_m, tile_n).  Workgroups are handed to the 8 XCDs round-robin, and a
// persistent workgroup b visits tiles b, b + G, ... with G a multiple of 8, so tile t runs
// on XCD t % 8.  The remap gives each XCD a contiguous range of logical ids, and the
// grouped order walks GROUP_M tile-rows at a time so tiles in flight together share A rows
// and B columns in that XCD's L2.
__device__ __forceinline__ void tile_coords(int t, int ntiles, int nbm, int& bm, int& bn) {
  const int nbn = ntiles / nbm;
  if ((ntiles & 7) == 0) t = (t & 7) * (ntiles >> 3) + (t >> 3);
  constexpr int GROUP_M = FLY_GROUP_M;
  const int per_group = GROUP_M * nbn;
  const int g = t / per_group;
  const int first_m = g * GROUP_M;
  const int gsz = min(nbm - first_m, GROUP_M);
  const int r = t - g * per_group;
  bm = first_m + r % gsz;
  bn = r / gsz;
}

// Raw buffer descriptor over [base, base + bytes) as four SGPR words: base, stride 0,
// num_records = bytes, dword3 0x00020000 (32-bit data format, the gfx9 setting for untyped raw
// buffer access).  Loads past num_records return zero; stores past it are dropped.
typedef int sgpr4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ sgpr4 buf_desc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  return sgpr4{(int)(uint32_t)a, (int)((uint32_t)(a >> 32) & 0xFFFF), (int)bytes, 0x00020000};
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, bytes, 0x00020000);
}

// LDS-DMA loads (gfx950 buffer_load ... lds): lane l reads 16 (4) bytes at voffset(l) + soffset
// of the buffer and the wave writes them to LDS base + 16*l (4*l); lanes past the buffer write
// zeros.  They are issued as inline assembly on purpose: the compiler then does not treat them
// as LDS writes that a later LDS read of the *other* stage might alias (it cannot tell the two
// stages apart and would wait for every outstanding load, including the DMA just issued).  The
// kernels wait for them explicitly (vector memory counter) before the barrier that publishes a
// stage.  M0 carries the LDS base; nothing else in these kernels uses M0.
__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)p);
}
__device__ __forceinline__ void dma16(sgpr4 desc, uint8_t* lds_wave_base, uint32_t voffset, uint32_t soffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               ::"s"(lds_addr(lds_wave_base)), "v"(voffset), "s"(desc), "s"(soffset)
               : "memory", "m0");
}
__device__ __forceinline__ void dma4(sgpr4 desc, uint8_t* lds_wave_base, uint32_t voffset, uint32_t soffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds"
               ::"s"(lds_addr(lds_wave_base)), "v"(voffset), "s"(desc), "s"(soffset)
               : "memory", "m0");
}

// Waits go through __builtin_amdgcn_s_waitcnt rather than inline assembly: the compiler's
// own wait insertion accounts for them.  It does not see waits written as inline assembly, and
// would then assume a step's LDS-DMA still pending when that stage is read and wait for every
// outstanding load -- including the next step's DMA, issued just before.
// gfx9 encoding: vmcnt bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8].
template <int VM, int LGKM = 15>
__device__ __forceinline__ void waitcnt() {
  static_assert(VM >= 0 && VM <= 63 && LGKM >= 0 && LGKM <= 15, "counter range");
  __builtin_amdgcn_s_waitcnt((VM & 15) | ((VM >> 4) << 14) | (7 << 4) | (LGKM << 8));
}

__device__ __forceinline__ void wait_dma() { waitcnt<0>(); }

// Wait until at most N vector memory operations of this wave are outstanding.
template <int N>
__device__ __forceinline__ void wait_vmem_leaving() {
  waitcnt<(N < 63 ? N : 63)>();
}

// Workgroup barrier without a memory fence (__syncthreads() adds one that waits for every
// outstanding vector memory operation): this wave's LDS reads have completed, and the empty
// "memory" assembly keeps the compiler from moving LDS or buffer accesses across it.
__device__ __forceinline__ void workgroup_barrier() {
  waitcnt<63, 0>();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// KSUB: K tiles per pipeline step (two-stage ring only).  With 2, each LDS stage holds two
// 128-byte K tiles and a step waits for, and multiplies, both: half the barriers and twice the
// bytes in flight per wait, for tiles whose steps are short next to the DMA latency.
template <int BM, int BN, int WM, int WN, int KIND, int EPI, bool OUT_BF16, int KSUB = 1>
__global__ void __launch_bounds__(WM * WN * 64, 1) gemm_main_kernel(GemmArgs p) {
  using C = MainCfg<BM, BN, WM, WN, KIND>;
  static_assert(KSUB == 1 || (KSUB == 2 && C::NS == 2 && EPI != EPI_BLOCK && KIND != KIND_FP4),
                "two K tiles per step: two-stage ring, no per-K-tile scales");
  constexpr int MR = C::MR, NR = C::NR, NW = C::NW;
  // per-K-tile scale regions of a stage, in whole DMA instructions: 1 KB (16-byte lanes) for
  // MXFP4, 256 bytes (4-byte lanes) for blockscale
  constexpr int SC_INSTR = KIND == KIND_FP4 ? 1024 : 256;
  constexpr int SA_BYTES = KIND == KIND_FP4 ? (BM / 32 * 256 + 1023) / 1024 * 1024
                                            : (EPI == EPI_BLOCK ? (BM * 4 + 255) / 256 * 256 : 0);
  constexpr int SB_BYTES = KIND == KIND_FP4 ? (BN / 32 * 256 + 1023) / 1024 * 1024 : (EPI == EPI_BLOCK ? 256 : 0);
  constexpr int SA_DMA = SA_BYTES / SC_INSTR, SB_DMA = SB_BYTES / SC_INSTR;
  static_assert(EPI != EPI_BLOCK || BN / 128 <= 64, "one w_scale per lane");
  constexpr int STAGE = C::STAGE + SA_BYTES + SB_BYTES;  // one K tile
  __shared__ __attribute__((aligned(1024))) uint8_t lds0[STAGE * KSUB];
  __shared__ __attribute__((aligned(1024))) uint8_t lds1[STAGE * KSUB];

  const int M = p.M, N = p.N, K = p.K;
  const int nbm = (M + BM - 1) / BM;
  const int nbn = (N + BN - 1) / BN;
  const int ntiles = nbm * nbn;
  // K (bytes) is a multiple of 64: the last K tile holds half a tile when K % 128 == 64
  // (never for blockscale and MXFP4, whose scale blocks span whole K tiles)
  constexpr bool kHalfOk = KIND != KIND_FP4 && EPI != EPI_BLOCK;
  const int nk = (K + KT - 1) / KT;
  const bool half_k = kHalfOk && (K % KT) != 0;
  const int nblk_max = N / 16 - 1;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN;
  const int wn = wave % WN;
  const int l16 = lane & 15;
  const int lq = lane >> 4;  // 0..3

  // Staged epilogue (2-byte outputs, see epilogue_staged below): each wave's rows go through an
  // LDS stage in two halves, then whole 128-byte lines are stored.  Not where its registers
  // would spill (more than 4 column blocks per wave, or the blockscale epilogue's partials next
  // to 32 accumulator tiles), nor for 64-column tiles, whose 128-byte rows gain less than the
  // two barriers cost (256x4096x4096 fp8 on 64x64 tiles 13.9 us staged against 13.6 direct).
  constexpr int RB = BN * 2, CPR = RB / 16, HR = C::TM / 2, HMR = MR / 2;
  constexpr bool kStage = EPI != EPI_RAW && MR % 2 == 0 && NR <= 4 && BN >= 128 && !(EPI == EPI_BLOCK && MR * NR >= 32) &&
                          BM / 2 * RB <= C::STAGE && (BM / 2 * CPR) % C::NT == 0;
  // Split roles (8-wave tiles on the two-stage ring with the staged epilogue): waves NW/2..NW-1
  // issue every LDS-DMA, waves 0..NW/2-1 every epilogue store.  A wave's wait for its DMA
  // (vector memory counter, retired in issue order) then never includes stores, so a tile's
  // output write drains while the next tile's first K steps run instead of stalling the
  // second one.  Graph-timed on MI355X, split against shared roles: FP8 8192^3 395.5 us against
  // 408, fp8 9728x8192x8320 476 against 498, int8 9728x8192x8320 496 against 517, bf16
  // 5120x5120x8320 364 against 380, bf16 8192^3 781 against 813; level with one tile per CU
  // (int8 4096^3 59.0 against 59.1); int4 9728x8192x8320 0.7% slower (kept shared there).
  constexpr bool ROLES = FLY_ROLES && C::NS == 2 && NW == 8 && kStage && KSUB == 1 && KIND != KIND_INT4;
  constexpr int DW = ROLES ? NW / 2 : NW;              // waves that issue DMA
  const int dwave = ROLES ? wave - NW / 2 : wave;      // this wave's index among them (< 0: none)
  constexpr int A_DMA_W = C::A_DMA * NW / DW, B_DMA_W = C::B_DMA * NW / DW;  // per DMA wave

  // ---- DMA addressing ----
  // A: buffer resource over the rows still ahead of this K tile; the per-lane VGPR offset
  // carries the row, so rows >= M fall outside num_records and read as zero.  The swizzled
  // chunk depends only on the row inside the tile (tile rows start at multiples of 16).
  // B: one resource over the whole buffer; the 16-column block offset is wave-uniform
  // (SGPR soffset), column blocks past N are clamped to the last one.
  // A half K tile (the last one when K % 128 == 64 bytes) loads its upper 64 bytes -- A
  // chunks 4-7, the upper KB of each B block (int4: its lanes 32-63) -- from an offset past
  // every buffer, so the range check writes zeros there and those MFMA halves add nothing
  // (va0h / vbh; 0x80000000 plus any row offset stays past the 2^31-byte operands).
  constexpr uint32_t kPast = 0x80000000u;
  uint32_t va0[A_DMA_W], va0h[A_DMA_W];
#pragma unroll
  for (int j = 0; j < A_DMA_W; ++j) {
    const int rloc = (dwave + j * DW) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((rloc >> 1) & 7);
    va0[j] = (uint32_t)rloc * (uint32_t)K + (uint32_t)(c * 16);
    va0h[j] = (kHalfOk && c >= 4) ? kPast : va0[j];
  }
  constexpr int PARTS = C::B_BLK / 1024;
  const uint32_t vb = (uint32_t)lane * 16u;
  const uint32_t vbh = (kHalfOk && PARTS == 1 && lane >= 32) ? kPast : vb;
  const int b_bytes = (KIND == KIND_INT4) ? (N / 2) * K : N * K;
  const sgpr4 rsrc_b = buf_desc(p.b, (uint32_t)b_bytes);

  // scale arrays: MXFP4 [round_up(M, 32) / 32][K tiles][64 lanes] words of A and
  // [N / 32][K tiles][64] of B; blockscale x_scale_t [K tiles][M] and w_scale [ceil(N/128)][K tiles]
  const int sa_bytes = KIND == KIND_FP4 ? (M + 31) / 32 * nk * 256 : nk * M * 4;
  const int sb_bytes = KIND == KIND_FP4 ? N / 32 * nk * 256 : (N + 127) / 128 * nk * 4;
  const sgpr4 rsrc_sa = buf_desc(p.sa, (SA_DMA + SB_DMA > 0) ? (uint32_t)sa_bytes : 0u);
  const sgpr4 rsrc_sb = buf_desc(p.sb, (SA_DMA + SB_DMA > 0) ? (uint32_t)sb_bytes : 0u);

  // one K tile kt into the stage region s; a K tile past the end (the second K tile of a last
  // step with KSUB = 2 and an odd K tile count) reads zeros: an empty A range, B lanes past
  // the buffer
  auto issue_tile = [&](uint8_t* s, int m0, int n0, int kt) {
    if (ROLES && dwave < 0) return;  // a store wave
    const bool live = KSUB == 1 || kt < nk;
    const sgpr4 rsrc_a = buf_desc(p.a + (size_t)(live ? kt : 0) * KT, live ? (uint32_t)(M * K - kt * KT) : 0u);
    const uint32_t mo = (uint32_t)m0 * (uint32_t)K;
    const bool half = half_k && kt == nk - 1;
#pragma unroll
    for (int j = 0; j < A_DMA_W; ++j) dma16(rsrc_a, s + (dwave + j * DW) * 1024, (half ? va0h[j] : va0[j]) + mo, 0);
#pragma unroll
    for (int j = 0; j < B_DMA_W; ++j) {
      const int q = dwave + j * DW;
      const int nb = min(n0 / 16 + q / PARTS, nblk_max);
      const uint32_t so = (uint32_t)nb * (uint32_t)(C::B_BLK / KT) * (uint32_t)K + (uint32_t)((q % PARTS) * 1024) +
                          (uint32_t)(live ? kt : 0) * C::B_BLK;
      const uint32_t vo = !live ? kPast : (!half ? vb : (PARTS == 1 ? vbh : (q % PARTS == 1 ? kPast : vb)));
      dma16(rsrc_b, s + C::A_BYTES + q * 1024, vo, __builtin_amdgcn_readfirstlane(so));
    }
    // this K tile's scales: scale instruction q = wave, wave + NW, ... (q < SA_DMA: A region,
    // then B region); indices past the arrays are clamped
    if constexpr (SA_DMA + SB_DMA > 0) {
      uint8_t* sc = s + C::STAGE;
#pragma unroll
      for (int j = 0; j < (SA_DMA + SB_DMA + DW - 1) / DW; ++j) {
        const int q = dwave + j * DW;
        if (q < SA_DMA) {
          if constexpr (KIND == KIND_FP4) {
            const uint32_t b = (uint32_t)q * 1024u + (uint32_t)lane * 16u;  // byte in the region
            const int r1 = min(m0 / 32 + (int)(b >> 8), (M + 31) / 32 - 1);
            dma16(rsrc_sa, sc + q * 1024, ((uint32_t)r1 * (uint32_t)nk * 64u) * 4u + (b & 255u), (uint32_t)kt * 256u);
          } else {
            // x_scale_t[kt][m0 + 64q + lane]; rows past M read the next values or zeros
            dma4(rsrc_sa, sc + q * 256, ((uint32_t)kt * (uint32_t)M + (uint32_t)(m0 + q * 64 + lane)) * 4u, 0);
          }
        } else if (q < SA_DMA + SB_DMA) {
          const int qb = q - SA_DMA;
          if constexpr (KIND == KIND_FP4) {
            const uint32_t b = (uint32_t)qb * 1024u + (uint32_t)lane * 16u;
            const int c1 = min(n0 / 32 + (int)(b >> 8), N / 32 - 1);
            dma16(rsrc_sb, sc + SA_BYTES + qb * 1024, ((uint32_t)c1 * (uint32_t)nk * 64u) * 4u + (b & 255u),
                  (uint32_t)kt * 256u);
          } else {
            // lane l < BN/128: w_scale[n0/128 + l][kt]; the other lanes repeat lane 0's
            // address (one cache line for the wave instead of 64 scattered ones)
            const int nb = min(n0 / 128 + (lane < (BN + 127) / 128 ? lane : 0), (N - 1) / 128);
            dma4(rsrc_sb, sc + SA_BYTES, ((uint32_t)nb * (uint32_t)nk + (uint32_t)kt) * 4u, 0);
          }
        }
      }
    }
  };
  // one pipeline step (KSUB K tiles) into stage s
  auto issue = [&](uint8_t* s, int m0, int n0, int step_k) {
#pragma unroll
    for (int u = 0; u < KSUB; ++u) issue_tile(s + u * STAGE, m0, n0, step_k * KSUB + u);
  };

  typedef typename std::conditional<kind_float_acc(KIND), f32x4, i32x4>::type AccT;
  AccT acc[MR][NR];
  // per-token / per-channel scaling (not applied to 16-bit inputs, whose scale pointers may be
  // null, nor to MXFP4, whose block scales are applied by the MFMA)
  constexpr bool kScaled = EPI == EPI_ROWCOL && !kind_unscaled(KIND);

  // A fragment of MFMA row mi: lane holds 16-byte chunks lq and lq+4 of its row
  auto load_a = [&](const uint8_t* sA, int mi, i32x4& lo, i32x4& hi) {
    const int row = wm * C::TM + mi * 16 + l16;
    const int sw = (row >> 1) & 7;
    lo = *(const i32x4*)(sA + row * KT + ((lq ^ sw) << 4));
    hi = *(const i32x4*)(sA + row * KT + (((lq + 4) ^ sw) << 4));
  };

  // Blockscale: the 128-deep MFMA of row mi goes into a zeroed partial, which is added to the
  // accumulator scaled by sa * sb one row later, after the next row's MFMAs have been issued,
  // so the FMAs never wait on the MFMA that produced their operand.  Two partial sets
  // alternate between rows (MR is even).  The last row's partial waits for the next K tile:
  // it is added after that tile's first MFMAs (with the factors pend_s kept from its own
  // tile), or before the epilogue, so the end of a step never waits on its last MFMAs.
  static_assert(EPI != EPI_BLOCK || MR % 2 == 0, "blockscale alternates two partial sets over an even MR");
  f32x4 part[2][NR];
  float pend_s[NR];
  auto flush_pending = [&]() {
#pragma unroll
    for (int ni = 0; ni < NR; ++ni) {
      const f32x4 pv = part[(MR - 1) & 1][ni];
      acc[MR - 1][ni].x = __builtin_fmaf(pv.x, pend_s[ni], acc[MR - 1][ni].x);
      acc[MR - 1][ni].y = __builtin_fmaf(pv.y, pend_s[ni], acc[MR - 1][ni].y);
      acc[MR - 1][ni].z = __builtin_fmaf(pv.z, pend_s[ni], acc[MR - 1][ni].z);
      acc[MR - 1][ni].w = __builtin_fmaf(pv.w, pend_s[ni], acc[MR - 1][ni].w);
    }
  };

  // One K tile.  The A fragment of row mi+1 is requested before the MFMAs of row mi are
  // issued, so its LDS latency hides behind NR MFMAs.  B is the MFMA's first operand, so
  // each accumulator tile holds C transposed (see the epilogue).  `pending`: the previous K
  // tile of this output tile left its last blockscale row to add.
  auto compute = [&](const uint8_t* sA, bool pending) {
    const uint8_t* sB = sA + C::A_BYTES;
    const uint8_t* sS = sA + C::STAGE;  // this K tile's scales
    // blockscale: this lane's row scale per row block, the column-block scale per tile column;
    // MXFP4: this lane's scale word per 32-row / 32-column group
    constexpr int MQ = (MR + 1) / 2, NQ = (NR + 1) / 2;
    float sa_t[MR], sb_t[NR];
    uint32_t fa_t[MQ], fb_t[NQ];
    if constexpr (EPI == EPI_BLOCK) {
#pragma unroll
      for (int mi = 0; mi < MR; ++mi) sa_t[mi] = *(const float*)(sS + (wm * C::TM + mi * 16 + l16) * 4);
#pragma unroll
      for (int ni = 0; ni < NR; ++ni) sb_t[ni] = *(const float*)(sS + SA_BYTES + ((wn * C::TN + ni * 16) / 128) * 4);
    }
    if constexpr (KIND == KIND_FP4) {
#pragma unroll
      for (int q = 0; q < MQ; ++q) fa_t[q] = *(const uint32_t*)(sS + (wm * C::TM / 32 + q) * 256 + lane * 4);
#pragma unroll
      for (int q = 0; q < NQ; ++q) fb_t[q] = *(const uint32_t*)(sS + SA_BYTES + (wn * C::TN / 32 + q) * 256 + lane * 4);
    }
    i32x4 alo, ahi;
    load_a(sA, 0, alo, ahi);
    if constexpr (KIND == KIND_FP8) {
      i32x8 bf[NR];
#pragma unroll
      for (int ni = 0; ni < NR; ++ni) {
        const int off = (wn * NR + ni) * 2048 + lq * 256 + l16 * 16;
        const i32x4 lo = *(const i32x4*)(sB + off);
        const i32x4 hi = *(const i32x4*)(sB + off + 1024);
        bf[ni] = i32x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      }
    auto scale_row = [&](int mi) {
#pragma unroll
      for (int ni = 0; ni < NR; ++ni) {
        const f32x4 pv = part[mi & 1][ni];
        const float s = sa_t[mi] * sb_t[ni];
        acc[mi][ni].x = __builtin_fmaf(pv.x, s, acc[mi][ni].x);
        acc[mi][ni].y = __builtin_fmaf(pv.y, s, acc[mi][ni].y);
        acc[mi][ni].z = __builtin_fmaf(pv.z, s, acc[mi][ni].z);
        acc[mi][ni].w = __builtin_fmaf(pv.w, s, acc[mi][ni].w);
      }
    };
#pragma unroll
      for (int mi = 0; mi < MR; ++mi) {
        const i32x8 af = i32x8{alo.x, alo.y, alo.z, alo.w, ahi.x, ahi.y, ahi.z, ahi.w};
        if (mi + 1 < MR) load_a(sA, mi + 1, alo, ahi);
        if constexpr (EPI == EPI_BLOCK) {
#pragma unroll
          for (int ni = 0; ni < NR; ++ni) part[mi & 1][ni] = mfma_fp8(bf[ni], af, f32x4{0.f, 0.f, 0.f, 0.f});
          if (mi > 0)
            scale_row(mi - 1);
          else if (pending)
            flush_pending();
          if (mi + 1 == MR) {
#pragma unroll
            for (int ni = 0; ni < NR; ++ni) pend_s[ni] = sa_t[mi] * sb_t[ni];
          }
        } else {
#if FLY_SCHED
          // the next row's A reads stay ahead of this row's MFMAs
          __builtin_amdgcn_sched_barrier(0);
#endif
#pragma unroll
          for (int ni = 0; ni < NR; ++ni) acc[mi][ni] = mfma_fp8(bf[ni], af, acc[mi][ni]);
#if FLY_SCHED
          __builtin_amdgcn_sched_barrier(0);
#endif
        }
      }
    } else {
      i32x4 bl[NR], bh[NR];
#pragma unroll
      for (int ni = 0; ni < NR; ++ni) {
        if constexpr (KIND == KIND_INT4) {
          const int off = (wn * NR + ni) * 1024 + lq * 128 + l16 * 8;
          bl[ni] = unpack_int4x16(*(const i32x2*)(sB + off));
          bh[ni] = unpack_int4x16(*(const i32x2*)(sB + off + 512));
        } else {
          const int off = (wn * NR + ni) * 2048 + lq * 256 + l16 * 16;
          bl[ni] = *(const i32x4*)(sB + off);
          bh[ni] = *(const i32x4*)(sB + off + 1024);
        }
      }
#pragma unroll
      for (int mi = 0; mi < MR; ++mi) {
        const i32x4 lo = alo, hi = ahi;
        if (mi + 1 < MR) load_a(sA, mi + 1, alo, ahi);
#if FLY_SCHED
        __builtin_amdgcn_sched_barrier(0);
#endif
        // the two 64-byte halves of the K tile go out as two passes over the row's tiles, so
        // the two MFMAs that accumulate into one tile are NR instructions apart
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int ni = 0; ni < NR; ++ni) {
            const i32x4& bq = h ? bh[ni] : bl[ni];
            const i32x4& aq = h ? hi : lo;
            if constexpr (KIND == KIND_FP4) {
              // chunks lq / lq+4 are the 32-element scale blocks of MFMA halves 0 / 1
              const uint32_t sbw = fb_t[ni >> 1] >> (8 * (ni & 1)), saw = fa_t[mi >> 1] >> (8 * (mi & 1));
              acc[mi][ni] = h ? mfma_fp4<1>(bq, aq, acc[mi][ni], sbw, saw) : mfma_fp4<0>(bq, aq, acc[mi][ni], sbw, saw);
            } else {
              acc[mi][ni] = mfma_k64<KIND>(bq, aq, acc[mi][ni]);
            }
          }
        }
#if FLY_SCHED
        __builtin_amdgcn_sched_barrier(0);
#endif
      }
    }
  };

  // ---- epilogue ----
  // B is the MFMA's first operand, so each 16x16 accumulator tile is C transposed: lane
  // (lq, l16) holds row l16, columns 4*lq .. 4*lq+3 -- one 8-byte bf16/fp16 store (16 bytes
  // for raw accumulators) per tile.  Every lane issues exactly MR*NR buffer stores (NSTORE with
  // the staged epilogue below); those outside C get an offset past the buffer end and are
  // dropped by the bounds check, so the number of stores in flight is known when the next tile
  // waits for its first loads.
  constexpr int ESZ = (EPI == EPI_RAW) ? 4 : 2;
  const __amdgpu_buffer_rsrc_t rsrc_c = make_rsrc(p.c, M * N * ESZ);
  // Output stores are non-temporal (cache policy NT) where no later wait of the storing wave
  // covers them: with the split roles, and for a workgroup's last tile.  The output is written
  // once and not read here, and every CU writes its tile at once (4 MB per XCD for a round of
  // 256x256 tiles, an L2's whole capacity).  An NT store takes longer to retire, so where a
  // wave's next DMA wait would cover it (shared roles, more tiles to come) the store is plain.
  // Graph-timed on MI355X against plain stores everywhere: int8 4096^3 52.3 us against 57.1,
  // fp8 blockscale 1024x7168x7168 62.4 against 63.7, W4A8 256x14336x4096 18.8 against 19.3,
  // fp8 8192^3 386 against 391, fp8 5120x5120x8320 178.8 against 180.7; NT on every tile of
  // the shared-role int4 9728x8192x8320 was 12% slower (544 against 486 us).
  constexpr int kStoreNT = 2;
  auto store16 = [&](const i32x4& v, uint32_t off, bool nt) {
    if (nt)
      __builtin_amdgcn_raw_buffer_store_b128(v, rsrc_c, off, 0, kStoreNT);
    else
      __builtin_amdgcn_raw_buffer_store_b128(v, rsrc_c, off, 0, 0);
  };
  auto store8 = [&](const i32x2& v, uint32_t off, bool nt) {
    if (nt)
      __builtin_amdgcn_raw_buffer_store_b64(v, rsrc_c, off, 0, kStoreNT);
    else
      __builtin_amdgcn_raw_buffer_store_b64(v, rsrc_c, off, 0, 0);
  };
  // Staged epilogue (2-byte outputs): in two rounds, each wave's first and then second half of
  // its rows go through the LDS stage `stg` (free once every wave is past the first barrier),
  // then every thread (every thread of the store waves, with split roles) stores 16-byte
  // chunks so that each wave instruction writes whole
  // 128-byte lines (the MFMA layout writes 16 rows x 32 bytes per instruction, which the memory
  // system takes at about 2/3 of the rate of whole lines).  Staged row sr holds row
  // (sr / HR) * TM + h * HR + sr % HR of the tile in round h (HR = TM / 2); its chunk c sits at
  // chunk c ^ (sr % CPR).
  // (the tiles and conditions are in kStage above).  Measured against the direct stores:
  // C3 59.8 us against 62.1, C4 64.4 against 66.0, C5 20.9 against 21.8, T 412 against 418,
  // 1024x7168x7168 fp8 56.3 against 58.0, MXFP4 4096^3 35.5 against 38.5.
  constexpr int SCH = kStage ? (BM / 2 * CPR) / C::NT : 0;
  constexpr int NSTORE = SCH > 0 ? 2 * SCH : MR * NR;   // buffer stores per lane per tile (without roles)
  constexpr int ST_T = ROLES ? C::NT / 2 : C::NT;        // threads that store
  constexpr int SCH_W = ROLES ? 2 * SCH : SCH;           // 16-byte stores per storing thread per half
  auto epilogue_staged = [&](int m0, int n0, uint8_t* stg, bool nt) {
#pragma unroll
    for (int mi = 0; mi < MR; ++mi)
#pragma unroll
      for (int ni = 0; ni < NR; ++ni) acc[mi][ni] = int4_acc<KIND>(acc[mi][ni]);
    float sa_e[MR];
    f32x4 sb_e[NR];
    if constexpr (kScaled) {
#pragma unroll
      for (int mi = 0; mi < MR; ++mi) sa_e[mi] = p.sa[min(m0 + wm * C::TM + mi * 16 + l16, M - 1)];
#pragma unroll
      for (int ni = 0; ni < NR; ++ni)
        sb_e[ni] = *(const f32x4*)(p.sb + min(n0 + wn * C::TN + ni * 16 + lq * 4, N - 4));
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      workgroup_barrier();   // the stage is free: computed from (h == 0) or read out (h == 1)
#pragma unroll
      for (int mh = 0; mh < HMR; ++mh) {
        const int mi = h * HMR + mh;
        const int sr = wm * HR + mh * 16 + l16;
#pragma unroll
        for (int ni = 0; ni < NR; ++ni) {
          const int c = wn * C::TN + ni * 16 + lq * 4;
          float v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            v[q] = (float)acc[mi][ni][q];
            if constexpr (kScaled) v[q] = (v[q] * sa_e[mi]) * sb_e[ni][q];
          }
          *(i32x2*)(stg + sr * RB + (((c >> 3) ^ (sr % CPR)) << 4) + (c & 7) * 2) = pack_out4<OUT_BF16>(v);
        }
      }
      workgroup_barrier();
      __builtin_amdgcn_sched_barrier(0);
      if (ROLES && wave >= NW / 2) continue;  // a DMA wave: the store waves write the lines
#pragma unroll 2
      for (int i = 0; i < SCH_W; ++i) {
        const int cc = tid + i * ST_T;
        const int sr = cc / CPR, ch = cc % CPR;
        const i32x4 val = *(const i32x4*)(stg + sr * RB + ((ch ^ (sr % CPR)) << 4));
        const int row = m0 + (sr / HR) * C::TM + h * HR + sr % HR, col = n0 + ch * 8;
        const uint32_t off = (row < M && col < N) ? ((uint32_t)row * (uint32_t)N + (uint32_t)col) * 2u : 0x80000000u;
        store16(val, off, nt);
      }
    }
  };
  auto epilogue = [&](int m0, int n0, bool nt) {
#pragma unroll
    for (int mi = 0; mi < MR; ++mi)
#pragma unroll
      for (int ni = 0; ni < NR; ++ni) acc[mi][ni] = int4_acc<KIND>(acc[mi][ni]);
    float sa_e[MR];
    f32x4 sb_e[NR];
    if constexpr (kScaled) {
#pragma unroll
      for (int mi = 0; mi < MR; ++mi) sa_e[mi] = p.sa[min(m0 + wm * C::TM + mi * 16 + l16, M - 1)];
#pragma unroll
      for (int ni = 0; ni < NR; ++ni)
        sb_e[ni] = *(const f32x4*)(p.sb + min(n0 + wn * C::TN + ni * 16 + lq * 4, N - 4));
    }
#pragma unroll
    for (int mi = 0; mi < MR; ++mi) {
      const int row = m0 + wm * C::TM + mi * 16 + l16;
#pragma unroll
      for (int ni = 0; ni < NR; ++ni) {
        const int col = n0 + wn * C::TN + ni * 16 + lq * 4;
        const uint32_t off = (row < M && col < N) ? ((uint32_t)row * (uint32_t)N + (uint32_t)col) * ESZ : 0x80000000u;
        if constexpr (EPI == EPI_RAW) {
          store16(__builtin_bit_cast(i32x4, acc[mi][ni]), off, nt);
        } else {
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            v[r] = (float)acc[mi][ni][r];
            if constexpr (kScaled) v[r] = (v[r] * sa_e[mi]) * sb_e[ni][r];
          }
          store8(pack_out4<OUT_BF16>(v), off, nt);
        }
      }
    }
  };

  // ---- persistent loop over this workgroup's tiles, one flattened (tile, K tile) pipeline:
  // the DMA of the next step -- the next K tile, or the first K tile of the next tile -- is
  // in flight while the MFMAs of the current step run, so a tile's first loads overlap the
  // previous tile's last MFMAs and its epilogue.
  const int G = gridDim.x;
  const int nitems = ntiles;
  auto item = [&](int w, int& m0_, int& n0_, int& kb_, int& ke_) {
    int bm, bn;
    tile_coords(w, ntiles, nbm, bm, bn);
    m0_ = bm * BM;
    n0_ = bn * BN;
    kb_ = 0;
    ke_ = (nk + KSUB - 1) / KSUB;  // pipeline steps
  };
  if constexpr (C::NS == 3) {
    // Three LDS stages, the DMA two steps ahead (the 4-wave tiles, whose steps are short
    // enough that one step of lead leaves them waiting on DMA latency).  A step's DMA is
    // complete once no more than the next step's DMA_PER_STEP operations of this wave are
    // outstanding (they retire in issue order); epilogue stores or the extra scale DMAs of
    // some waves may make that wait longer, never too short.  The last issued step waits
    // for everything.
    __shared__ __attribute__((aligned(1024))) uint8_t lds2[STAGE];
    auto ring = [&](int i) -> uint8_t* { return i == 0 ? lds0 : (i == 1 ? lds1 : lds2); };
    int iw = blockIdx.x, ikt = 0, ike = 0;  // the next step to issue: item iw, K tile ikt
    int im0 = 0, in0 = 0;
    if (iw < nitems) item(iw, im0, in0, ikt, ike);
    int issued = 0;
    auto issue_next = [&](int slot) {
      issue(ring(slot), im0, in0, ikt);
      ++issued;
      if (++ikt == ike) {
        iw += G;
        if (iw < nitems) item(iw, im0, in0, ikt, ike);
      }
    };
    if (iw < nitems) issue_next(0);
    if (iw < nitems) issue_next(1);
    int step = 0, slot = 0, last = 0;
    for (int w = blockIdx.x; w < nitems; w += G) {
      int m0, n0, kb, ke;
      item(w, m0, n0, kb, ke);
#pragma unroll
      for (int i = 0; i < MR; ++i)
#pragma unroll
        for (int j = 0; j < NR; ++j) acc[i][j] = AccT{0, 0, 0, 0};
      for (int kt = kb; kt < ke; ++kt, ++step) {
        if (issued > step + 1)
          waitcnt<C::DMA_PER_STEP>();
        else
          wait_dma();
        workgroup_barrier();  // step's stage is published; every wave is done with step-1's
        if (iw < nitems) issue_next(slot == 0 ? 2 : slot - 1);  // the stage step-1 used
        compute(ring(slot), kt != kb);
        last = slot;
        slot = slot == 2 ? 0 : slot + 1;
      }
      if constexpr (EPI == EPI_BLOCK) flush_pending();
      // the last step's stage is written next by the DMA issued after the next step's barrier
      const bool nt = w + G >= nitems;  // this workgroup's last tile
      if constexpr (SCH > 0)
        epilogue_staged(m0, n0, ring(last), nt);
      else
        epilogue(m0, n0, nt);
    }
    return;
  }
  int w = blockIdx.x;
  int m0, n0, kb, ke;
  item(w, m0, n0, kb, ke);
  issue(lds0, m0, n0, kb);
  int step = 0;
  for (; w < nitems; w += G) {
    const int wnext = w + G;
    int nm0 = 0, nn0 = 0, nkb = 0, nke = 0;
    if (wnext < nitems) item(wnext, nm0, nn0, nkb, nke);
#pragma unroll
    for (int i = 0; i < MR; ++i)
#pragma unroll
      for (int j = 0; j < NR; ++j) acc[i][j] = AccT{0, 0, 0, 0};
    for (int kt = kb; kt < ke; ++kt, ++step) {
      // wait for this wave's loads of this step; at a tile's first step the previous
      // tile's MR*NR epilogue stores were issued after them and may still be in flight
      // (vector memory operations retire in issue order).
      if constexpr (ROLES) {
        if (dwave >= 0) wait_dma();  // DMA waves hold no stores; store waves issue no DMA
      } else if (kt == kb && step > 0) {
        wait_vmem_leaving<NSTORE>();
      } else {
        wait_dma();
      }
      // this step's tile has landed; every wave is done with the other stage.  A bare
      // s_barrier: __syncthreads() would add a fence that waits for every outstanding vector
      // memory operation, i.e. also for the previous tile's epilogue stores kept in flight above.
      // The waits this barrier needs are this wave's DMAs (just above) and its LDS reads.
      workgroup_barrier();
      uint8_t* cur = (step & 1) ? lds1 : lds0;
      uint8_t* nxt = (step & 1) ? lds0 : lds1;
      if (kt + 1 < ke)
        issue(nxt, m0, n0, kt + 1);
      else if (wnext < nitems)
        issue(nxt, nm0, nn0, nkb);
#pragma unroll
      for (int u = 0; u < KSUB; ++u) compute(cur + u * STAGE, kt != kb || u > 0);
    }
    if constexpr (EPI == EPI_BLOCK) flush_pending();
    // the stage the last step computed from; the DMA issued after the next step's barrier is the
    // next to write it
    if constexpr (SCH > 0)
      epilogue_staged(m0, n0, (step & 1) ? lds0 : lds1, ROLES || wnext >= nitems);
    else
      epilogue(m0, n0, wnext >= nitems);
    m0 = nm0;
    n0 = nn0;
    kb = nkb;
    ke = nke;
  }
}

}  // namespace flygemm
