// Large-M kernel: LDS double-buffered MFMA GEMM for gfx950.
//
//   C[M][N] = epilogue( sum_k A[m][k] * B[n][k] )
//
// Workgroup tile BM x BN, K tile 128.  WM x WN waves; each wave owns a (BM/WM) x (BN/WN)
// block of 16x16 MFMA tiles.  Per K tile every thread moves its share of A and B
// global -> registers (16-byte loads, issued one tile ahead) -> LDS; the next tile's loads
// are in flight while the current tile's MFMAs run.  One barrier per K tile.
//
// LDS per stage:
//   A: row-major [BM][128 B]; the 16-byte chunk c of row r sits at chunk slot
//      c ^ ((r >> 1) & 7), so the 16 lanes that read one chunk column of 16 rows hit
//      16 distinct 16-byte bank groups (64 banks x 4 B), and the 8 threads that write one
//      row write one 128-byte line.
//   B: the preshuffled bytes copied verbatim: per 16-column block a 2 KB run
//      [chunk 0..7][col 0..15][16 B] (INT4: 1 KB [chunk][col][8 B]); lanes that read one
//      chunk read 256 (128) contiguous bytes.
#pragma once
#include "gemm_common.h"

namespace flygemm {

template <int BM, int BN, int WM, int WN, int KIND, int EPI, bool OUT_BF16>
struct MainCfg {
  static constexpr int NT = WM * WN * 64;
  static constexpr int TM = BM / WM;
  static constexpr int TN = BN / WN;
  static constexpr int MR = TM / 16;
  static constexpr int NR = TN / 16;
  static constexpr int A_BYTES = BM * KT;
  static constexpr int B_BLK = (KIND == KIND_INT4) ? 1024 : 2048;  // bytes per 16 cols per K tile
  static constexpr int B_BYTES = (BN / 16) * B_BLK;
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int A_LD = A_BYTES / (NT * 16);
  static constexpr int B_LD = B_BYTES / (NT * 16);
  static constexpr int LDS = 2 * STAGE;
  static_assert(TM % 16 == 0 && TN % 16 == 0, "wave tile must be a multiple of 16");
  static_assert(A_BYTES % (NT * 16) == 0 && B_BYTES % (NT * 16) == 0, "tile not divisible into 16B loads");
};

// Workgroup id -> (tile_m, tile_n).  Workgroups are handed to the 8 XCDs round-robin;
// the remap gives each XCD a contiguous range of logical ids, and the grouped order walks
// GROUP_M tile-rows at a time so neighbouring workgroups share A rows and B columns in L2.
__device__ __forceinline__ void tile_coords(int nbm, int nbn, int& bm, int& bn) {
  const int nblk = nbm * nbn;
  int bid = blockIdx.x;
  if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
  constexpr int GROUP_M = 8;
  const int per_group = GROUP_M * nbn;
  const int g = bid / per_group;
  const int first_m = g * GROUP_M;
  const int gsz = min(nbm - first_m, GROUP_M);
  const int r = bid - g * per_group;
  bm = first_m + r % gsz;
  bn = r / gsz;
}

template <int BM, int BN, int WM, int WN, int KIND, int EPI, bool OUT_BF16>
__global__ void __launch_bounds__(WM * WN * 64, 1) gemm_main_kernel(GemmArgs p) {
  using C = MainCfg<BM, BN, WM, WN, KIND, EPI, OUT_BF16>;
  constexpr int MR = C::MR, NR = C::NR;
  __shared__ __attribute__((aligned(16))) uint8_t smem[C::LDS];

  const int M = p.M, N = p.N, K = p.K;
  const int nbm = (M + BM - 1) / BM;
  const int nbn = (N + BN - 1) / BN;
  int bm, bn;
  tile_coords(nbm, nbn, bm, bn);
  const int m0 = bm * BM;
  const int n0 = bn * BN;
  const int nk = K / KT;
  const int nblk_max = N / 16 - 1;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN;
  const int wn = wave % WN;
  const int l16 = lane & 15;
  const int lq = lane >> 4;  // 0..3

  // ---- global source pointers for this thread's 16-byte pieces (advanced per K tile) ----
  const uint8_t* ga[C::A_LD];
  int la[C::A_LD];
#pragma unroll
  for (int j = 0; j < C::A_LD; ++j) {
    const int q = tid + j * C::NT;
    const int row = q >> 3;
    const int c = q & 7;
    const int grow = min(m0 + row, M - 1);
    ga[j] = p.a + (size_t)grow * K + c * 16;
    la[j] = row * KT + ((c ^ ((row >> 1) & 7)) << 4);
  }
  const uint8_t* gb[C::B_LD];
  int lb[C::B_LD];
  constexpr int CH_PER_BLK = C::B_BLK / 16;
#pragma unroll
  for (int j = 0; j < C::B_LD; ++j) {
    const int q = tid + j * C::NT;
    const int nbl = q / CH_PER_BLK;
    const int w = q % CH_PER_BLK;
    const int nb = min(n0 / 16 + nbl, nblk_max);
    gb[j] = p.b + (size_t)nb * (C::B_BLK / KT) * (size_t)K + w * 16;  // block nb starts at nb*16*K (int4: nb*8*K)
    lb[j] = nbl * C::B_BLK + w * 16;
  }

  i32x4 ra[C::A_LD], rb[C::B_LD];
  auto load_tile = [&](int kt) {
#pragma unroll
    for (int j = 0; j < C::A_LD; ++j) ra[j] = *(const i32x4*)(ga[j] + (size_t)kt * KT);
#pragma unroll
    for (int j = 0; j < C::B_LD; ++j) rb[j] = *(const i32x4*)(gb[j] + (size_t)kt * C::B_BLK);
  };
  auto store_tile = [&](int stage) {
    uint8_t* s = smem + stage * C::STAGE;
#pragma unroll
    for (int j = 0; j < C::A_LD; ++j) *(i32x4*)(s + la[j]) = ra[j];
#pragma unroll
    for (int j = 0; j < C::B_LD; ++j) *(i32x4*)(s + C::A_BYTES + lb[j]) = rb[j];
  };

  typedef typename std::conditional<KIND == KIND_FP8, f32x4, i32x4>::type AccT;
  AccT acc[MR][NR];
#pragma unroll
  for (int i = 0; i < MR; ++i)
#pragma unroll
    for (int j = 0; j < NR; ++j) acc[i][j] = AccT{0, 0, 0, 0};

  // blockscale: per-row A scales (4 rows per mi) and per-column-block B scales
  float sa_cur[MR][4], sb_cur[NR], sa_nxt[MR][4], sb_nxt[NR];
  auto load_scales = [&](int kt, float (&sa_o)[MR][4], float (&sb_o)[NR]) {
    if constexpr (EPI == EPI_BLOCK) {
      const int nkb = nk;
#pragma unroll
      for (int mi = 0; mi < MR; ++mi)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = min(m0 + wm * C::TM + mi * 16 + lq * 4 + i, M - 1);
          sa_o[mi][i] = p.sa[(size_t)kt * M + row];
        }
#pragma unroll
      for (int ni = 0; ni < NR; ++ni) {
        const int col = min(n0 + wn * C::TN + ni * 16, N - 1);
        sb_o[ni] = p.sb[(size_t)(col >> 7) * nkb + kt];
      }
    }
  };

  load_scales(0, sa_cur, sb_cur);
  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = (kt + 1) < nk;
    if (more) {
      load_scales(kt + 1, sa_nxt, sb_nxt);
      load_tile(kt + 1);
    }
    const uint8_t* sA = smem + cur * C::STAGE;
    const uint8_t* sB = sA + C::A_BYTES;

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
        const int row = wm * C::TM + mi * 16 + l16;
        const int sw = (row >> 1) & 7;
        const i32x4 lo = *(const i32x4*)(sA + row * KT + ((lq ^ sw) << 4));
        const i32x4 hi = *(const i32x4*)(sA + row * KT + (((lq + 4) ^ sw) << 4));
        const i32x8 af = i32x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        if constexpr (EPI == EPI_BLOCK) {
#pragma unroll
          for (int ni = 0; ni < NR; ++ni) {
            const f32x4 part = mfma_fp8(af, bf[ni], f32x4{0.f, 0.f, 0.f, 0.f});
            const float s = sb_cur[ni];
            acc[mi][ni].x = __builtin_fmaf(part.x, sa_cur[mi][0] * s, acc[mi][ni].x);
            acc[mi][ni].y = __builtin_fmaf(part.y, sa_cur[mi][1] * s, acc[mi][ni].y);
            acc[mi][ni].z = __builtin_fmaf(part.z, sa_cur[mi][2] * s, acc[mi][ni].z);
            acc[mi][ni].w = __builtin_fmaf(part.w, sa_cur[mi][3] * s, acc[mi][ni].w);
          }
        } else {
#pragma unroll
          for (int ni = 0; ni < NR; ++ni) acc[mi][ni] = mfma_fp8(af, bf[ni], acc[mi][ni]);
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
        const int row = wm * C::TM + mi * 16 + l16;
        const int sw = (row >> 1) & 7;
        const i32x4 lo = *(const i32x4*)(sA + row * KT + ((lq ^ sw) << 4));
        const i32x4 hi = *(const i32x4*)(sA + row * KT + (((lq + 4) ^ sw) << 4));
#pragma unroll
        for (int ni = 0; ni < NR; ++ni) {
          acc[mi][ni] = mfma_i8(lo, bl[ni], acc[mi][ni]);
          acc[mi][ni] = mfma_i8(hi, bh[ni], acc[mi][ni]);
        }
      }
    }

    if (more) {
      store_tile(cur ^ 1);
      if constexpr (EPI == EPI_BLOCK) {
#pragma unroll
        for (int mi = 0; mi < MR; ++mi)
#pragma unroll
          for (int i = 0; i < 4; ++i) sa_cur[mi][i] = sa_nxt[mi][i];
#pragma unroll
        for (int ni = 0; ni < NR; ++ni) sb_cur[ni] = sb_nxt[ni];
      }
    }
    __syncthreads();
  }

  // ---- epilogue: lane holds rows (lq*4 + i), column l16 of every 16x16 tile ----
  typedef typename OutT<OUT_BF16>::type OT;
#pragma unroll
  for (int mi = 0; mi < MR; ++mi) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = m0 + wm * C::TM + mi * 16 + lq * 4 + i;
      if (row >= M) continue;
      float s_a = 1.f;
      if constexpr (EPI == EPI_ROWCOL) s_a = p.sa[row];
#pragma unroll
      for (int ni = 0; ni < NR; ++ni) {
        const int col = n0 + wn * C::TN + ni * 16 + l16;
        if (col >= N) continue;
        const size_t idx = (size_t)row * N + col;
        if constexpr (EPI == EPI_RAW) {
          if constexpr (KIND == KIND_FP8)
            ((float*)p.c)[idx] = acc[mi][ni][i];
          else
            ((int*)p.c)[idx] = acc[mi][ni][i];
        } else {
          float v;
          if constexpr (KIND == KIND_FP8)
            v = acc[mi][ni][i];
          else
            v = (float)acc[mi][ni][i];
          if constexpr (EPI == EPI_ROWCOL) v = (v * s_a) * p.sb[col];
          ((OT*)p.c)[idx] = cvt_out<OUT_BF16>(v);
        }
      }
    }
  }
}

}  // namespace flygemm
