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
#pragma once
#include "gemm_common.h"

#ifndef FLY_SCHED
#define FLY_SCHED 1
#endif
#ifndef FLY_GROUP_M
#define FLY_GROUP_M 8
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

typedef __attribute__((address_space(3))) void lds_void;

// Raw buffer resource over [base, base + bytes); dword3 0x00020000 = 32-bit data format,
// the gfx9 setting for untyped raw buffer access.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, bytes, 0x00020000);
}

// One wave-wide LDS-DMA load: lane l reads 16 bytes at voffset(l) + soffset of the buffer
// and the wave writes them to lds_wave_base + 16*l.  Lanes whose voffset lies outside the
// buffer write zeros.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint8_t* lds_wave_base, uint32_t voffset,
                                      uint32_t soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds_wave_base, 16, voffset, soffset, 0, 0);
}

__device__ __forceinline__ void wait_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Wait until at most N (capped at 63, the counter's range) vector memory operations of this
// wave are outstanding.  Values without a case here fall back to waiting for all of them.
template <int N>
__device__ __forceinline__ void wait_vmem_leaving() {
  if constexpr (N >= 63)
    asm volatile("s_waitcnt vmcnt(63)" ::: "memory");
  else if constexpr (N == 32)
    asm volatile("s_waitcnt vmcnt(32)" ::: "memory");
  else if constexpr (N == 16)
    asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
  else if constexpr (N == 8)
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  else
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

template <int BM, int BN, int WM, int WN, int KIND, int EPI, bool OUT_BF16>
__global__ void __launch_bounds__(WM * WN * 64, 1) gemm_main_kernel(GemmArgs p) {
  using C = MainCfg<BM, BN, WM, WN, KIND>;
  constexpr int MR = C::MR, NR = C::NR, NW = C::NW;
  __shared__ __attribute__((aligned(1024))) uint8_t lds0[C::STAGE];
  __shared__ __attribute__((aligned(1024))) uint8_t lds1[C::STAGE];

  const int M = p.M, N = p.N, K = p.K;
  const int nbm = (M + BM - 1) / BM;
  const int nbn = (N + BN - 1) / BN;
  const int ntiles = nbm * nbn;
  const int nk = K / KT;
  const int nblk_max = N / 16 - 1;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN;
  const int wn = wave % WN;
  const int l16 = lane & 15;
  const int lq = lane >> 4;  // 0..3

  // ---- DMA addressing ----
  // A: buffer resource over the rows still ahead of this K tile; the per-lane VGPR offset
  // carries the row, so rows >= M fall outside num_records and read as zero.  The swizzled
  // chunk depends only on the row inside the tile (tile rows start at multiples of 16).
  // B: one resource over the whole buffer; the 16-column block offset is wave-uniform
  // (SGPR soffset), column blocks past N are clamped to the last one.
  uint32_t va0[C::A_DMA];
#pragma unroll
  for (int j = 0; j < C::A_DMA; ++j) {
    const int rloc = (wave + j * NW) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((rloc >> 1) & 7);
    va0[j] = (uint32_t)rloc * (uint32_t)K + (uint32_t)(c * 16);
  }
  constexpr int PARTS = C::B_BLK / 1024;
  const uint32_t vb = (uint32_t)lane * 16u;
  const int b_bytes = (KIND == KIND_INT4) ? (N / 2) * K : N * K;
  const __amdgpu_buffer_rsrc_t rsrc_b = make_rsrc(p.b, b_bytes);

  auto issue = [&](uint8_t* s, int m0, int n0, int kt) {
    const __amdgpu_buffer_rsrc_t rsrc_a = make_rsrc(p.a + (size_t)kt * KT, M * K - kt * KT);
    const uint32_t mo = (uint32_t)m0 * (uint32_t)K;
#pragma unroll
    for (int j = 0; j < C::A_DMA; ++j) dma16(rsrc_a, s + (wave + j * NW) * 1024, va0[j] + mo, 0);
#pragma unroll
    for (int j = 0; j < C::B_DMA; ++j) {
      const int q = wave + j * NW;
      const int nb = min(n0 / 16 + q / PARTS, nblk_max);
      const uint32_t so = (uint32_t)nb * (uint32_t)(C::B_BLK / KT) * (uint32_t)K + (uint32_t)((q % PARTS) * 1024) +
                          (uint32_t)kt * C::B_BLK;
      dma16(rsrc_b, s + C::A_BYTES + q * 1024, vb, __builtin_amdgcn_readfirstlane(so));
    }
  };

  typedef typename std::conditional<kind_float_acc(KIND), f32x4, i32x4>::type AccT;
  AccT acc[MR][NR];
  // per-token / per-channel scaling (not applied to 16-bit inputs, whose scale pointers may be null)
  constexpr bool kScaled = EPI == EPI_ROWCOL && !kind_is_16bit(KIND);

  // blockscale: the A scale of this lane's row in each MFMA row block and the B scale of
  // each 16-column block, for one K tile.  They are loaded one step ahead (into sa_n/sb_n,
  // together with that step's DMA), so the wait at the top of a step covers them too.
  float sa_t[MR], sb_t[NR], sa_n[MR], sb_n[NR];
  auto load_scales = [&](int m0, int n0, int kt) {
    if constexpr (EPI == EPI_BLOCK) {
#pragma unroll
      for (int mi = 0; mi < MR; ++mi)
        sa_n[mi] = p.sa[(size_t)kt * M + min(m0 + wm * C::TM + mi * 16 + l16, M - 1)];
#pragma unroll
      for (int ni = 0; ni < NR; ++ni) {
        const int col = min(n0 + wn * C::TN + ni * 16, N - 1);
        sb_n[ni] = p.sb[(size_t)(col >> 7) * nk + kt];
      }
    }
  };
  auto take_scales = [&]() {
    if constexpr (EPI == EPI_BLOCK) {
#pragma unroll
      for (int mi = 0; mi < MR; ++mi) sa_t[mi] = sa_n[mi];
#pragma unroll
      for (int ni = 0; ni < NR; ++ni) sb_t[ni] = sb_n[ni];
    }
  };

  // A fragment of MFMA row mi: lane holds 16-byte chunks lq and lq+4 of its row
  auto load_a = [&](const uint8_t* sA, int mi, i32x4& lo, i32x4& hi) {
    const int row = wm * C::TM + mi * 16 + l16;
    const int sw = (row >> 1) & 7;
    lo = *(const i32x4*)(sA + row * KT + ((lq ^ sw) << 4));
    hi = *(const i32x4*)(sA + row * KT + (((lq + 4) ^ sw) << 4));
  };

  // One K tile.  The A fragment of row mi+1 is requested before the MFMAs of row mi are
  // issued, so its LDS latency hides behind NR MFMAs.  B is the MFMA's first operand, so
  // each accumulator tile holds C transposed (see the epilogue).
  auto compute = [&](const uint8_t* sA) {
    const uint8_t* sB = sA + C::A_BYTES;
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
#pragma unroll
      for (int mi = 0; mi < MR; ++mi) {
        const i32x8 af = i32x8{alo.x, alo.y, alo.z, alo.w, ahi.x, ahi.y, ahi.z, ahi.w};
        if (mi + 1 < MR) load_a(sA, mi + 1, alo, ahi);
        if constexpr (EPI == EPI_BLOCK) {
#pragma unroll
          for (int ni = 0; ni < NR; ++ni) {
            const f32x4 part = mfma_fp8(bf[ni], af, f32x4{0.f, 0.f, 0.f, 0.f});
            const float s = sa_t[mi] * sb_t[ni];
            acc[mi][ni].x = __builtin_fmaf(part.x, s, acc[mi][ni].x);
            acc[mi][ni].y = __builtin_fmaf(part.y, s, acc[mi][ni].y);
            acc[mi][ni].z = __builtin_fmaf(part.z, s, acc[mi][ni].z);
            acc[mi][ni].w = __builtin_fmaf(part.w, s, acc[mi][ni].w);
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
#pragma unroll
        for (int ni = 0; ni < NR; ++ni) {
          acc[mi][ni] = mfma_k64<KIND>(bl[ni], lo, acc[mi][ni]);
          acc[mi][ni] = mfma_k64<KIND>(bh[ni], hi, acc[mi][ni]);
        }
      }
    }
  };

  // ---- epilogue ----
  // B is the MFMA's first operand, so each 16x16 accumulator tile is C transposed: lane
  // (lq, l16) holds row l16, columns 4*lq .. 4*lq+3 -- one 8-byte bf16/fp16 store (16 bytes
  // for raw accumulators) per tile.  Every lane issues exactly MR*NR buffer stores; those
  // outside C get an offset past the buffer end and are dropped by the bounds check, so the
  // number of stores in flight is known when the next tile waits for its first loads.
  constexpr int ESZ = (EPI == EPI_RAW) ? 4 : 2;
  const __amdgpu_buffer_rsrc_t rsrc_c = make_rsrc(p.c, M * N * ESZ);
  auto epilogue = [&](int m0, int n0) {
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
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, acc[mi][ni]), rsrc_c, off, 0, 0);
        } else {
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            v[r] = (float)acc[mi][ni][r];
            if constexpr (kScaled) v[r] = (v[r] * sa_e[mi]) * sb_e[ni][r];
          }
          __builtin_amdgcn_raw_buffer_store_b64(pack_out4<OUT_BF16>(v), rsrc_c, off, 0, 0);
        }
      }
    }
  };

  // ---- persistent loop over this workgroup's tiles, one flattened (tile, K tile) pipeline:
  // the DMA of the next step -- the next K tile, or the first K tile of the next tile --
  // is in flight while the MFMAs of the current step run, so a tile's first loads overlap
  // the previous tile's last MFMAs and its epilogue.
  const int G = gridDim.x;
  int t = blockIdx.x;
  int bm, bn;
  tile_coords(t, ntiles, nbm, bm, bn);
  int m0 = bm * BM, n0 = bn * BN;
  issue(lds0, m0, n0, 0);
  load_scales(m0, n0, 0);
  int step = 0;
  for (; t < ntiles; t += G) {
    const int tn = t + G;
    int nm0 = 0, nn0 = 0;
    if (tn < ntiles) {
      tile_coords(tn, ntiles, nbm, bm, bn);
      nm0 = bm * BM;
      nn0 = bn * BN;
    }
#pragma unroll
    for (int i = 0; i < MR; ++i)
#pragma unroll
      for (int j = 0; j < NR; ++j) acc[i][j] = AccT{0, 0, 0, 0};
    for (int kt = 0; kt < nk; ++kt, ++step) {
      // wait for this wave's loads of this step; at a tile's first step the previous
      // tile's MR*NR epilogue stores were issued after them and may still be in flight
      // (vector memory operations retire in issue order)
      if (kt == 0 && step > 0)
        wait_vmem_leaving<MR * NR>();
      else
        wait_dma();
      __syncthreads();  // this step's tile has landed; every wave is done with the other stage
      uint8_t* cur = (step & 1) ? lds1 : lds0;
      uint8_t* nxt = (step & 1) ? lds0 : lds1;
      take_scales();
      if (kt + 1 < nk) {
        issue(nxt, m0, n0, kt + 1);
        load_scales(m0, n0, kt + 1);
      } else if (tn < ntiles) {
        issue(nxt, nm0, nn0, 0);
        load_scales(nm0, nn0, 0);
      }
      compute(cur);
    }
    epilogue(m0, n0);
    m0 = nm0;
    n0 = nn0;
  }
}

}  // namespace flygemm
