// Small-M (decode) kernel: B is streamed from HBM straight into MFMA operand registers.
//
// For M <= 16*MR the whole of A (a few hundred KB at most) is L2-resident, so the kernel is
// bound by reading B once.  A workgroup owns NBW 16-column blocks and all M rows; its NW
// waves split K (wave w takes K tiles w, w+NW, ...), each wave keeps UNROLL K tiles of
// loads in flight, and the NW partial accumulators are summed through LDS before the
// fused epilogue.  The reduction is inside the workgroup: no workspace, no atomics, and
// the int32 sums stay exact.
//
// Per K tile a lane loads, for every owned 16-column block, the two 16-byte chunks
// (lane/16) and (lane/16)+4 of column (lane%16) -- the preshuffled layout makes each
// wave-wide load one contiguous 1 KB read -- and the matching two chunks of A row
// (lane%16).
#pragma once
#include "gemm_common.h"

namespace flygemm {

template <int MR, int NBW, int NW, int UNROLL, int KIND, int EPI, bool OUT_BF16>
__global__ void __launch_bounds__(NW * 64) gemm_decode_kernel(GemmArgs p) {
  const int M = p.M, N = p.N, K = p.K;
  const int nk = K / KT;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l16 = lane & 15;
  const int lq = lane >> 4;
  const int nblk_max = N / 16 - 1;
  const int nb0 = blockIdx.x * NBW;

  constexpr int B_BLK = (KIND == KIND_INT4) ? 1024 : 2048;
  constexpr size_t B_PER_K = B_BLK / KT;  // bytes of one 16-col block per K element (16 or 8)

  typedef typename std::conditional<KIND == KIND_FP8 || EPI == EPI_BLOCK, f32x4, i32x4>::type AccT;
  AccT acc[MR][NBW];
#pragma unroll
  for (int i = 0; i < MR; ++i)
#pragma unroll
    for (int j = 0; j < NBW; ++j) acc[i][j] = AccT{0, 0, 0, 0};

  const uint8_t* arow[MR];
#pragma unroll
  for (int mi = 0; mi < MR; ++mi) arow[mi] = p.a + (size_t)min(mi * 16 + l16, M - 1) * K;
  const uint8_t* bblk[NBW];
#pragma unroll
  for (int j = 0; j < NBW; ++j) {
    const int nb = min(nb0 + j, nblk_max);
    if constexpr (KIND == KIND_INT4)
      bblk[j] = p.b + (size_t)nb * B_PER_K * K + lq * 128 + l16 * 8;
    else
      bblk[j] = p.b + (size_t)nb * B_PER_K * K + lq * 256 + l16 * 16;
  }

  for (int kt0 = wave; kt0 < nk; kt0 += NW * UNROLL) {
    i32x4 alo[UNROLL][MR], ahi[UNROLL][MR];
    i32x4 blo[UNROLL][NBW], bhi[UNROLL][NBW];
    i32x2 b4lo[UNROLL][NBW], b4hi[UNROLL][NBW];
    // issue all loads of UNROLL K tiles first
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int kt = kt0 + u * NW;
      if (kt < nk) {
#pragma unroll
        for (int j = 0; j < NBW; ++j) {
          if constexpr (KIND == KIND_INT4) {
            const uint8_t* src = bblk[j] + (size_t)kt * B_BLK;
            b4lo[u][j] = __builtin_nontemporal_load((const i32x2*)src);
            b4hi[u][j] = __builtin_nontemporal_load((const i32x2*)(src + 512));
          } else {
            const uint8_t* src = bblk[j] + (size_t)kt * B_BLK;
            blo[u][j] = __builtin_nontemporal_load((const i32x4*)src);
            bhi[u][j] = __builtin_nontemporal_load((const i32x4*)(src + 1024));
          }
        }
#pragma unroll
        for (int mi = 0; mi < MR; ++mi) {
          const uint8_t* src = arow[mi] + (size_t)kt * KT + lq * 16;
          alo[u][mi] = *(const i32x4*)src;
          ahi[u][mi] = *(const i32x4*)(src + 64);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int kt = kt0 + u * NW;
      if (kt < nk) {
        if constexpr (KIND == KIND_FP8) {
#pragma unroll
          for (int mi = 0; mi < MR; ++mi) {
            const i32x8 af = i32x8{alo[u][mi].x, alo[u][mi].y, alo[u][mi].z, alo[u][mi].w,
                                   ahi[u][mi].x, ahi[u][mi].y, ahi[u][mi].z, ahi[u][mi].w};
            float sa4[4] = {0.f, 0.f, 0.f, 0.f};
            if constexpr (EPI == EPI_BLOCK) {
#pragma unroll
              for (int i = 0; i < 4; ++i) sa4[i] = p.sa[(size_t)kt * M + min(mi * 16 + lq * 4 + i, M - 1)];
            }
#pragma unroll
            for (int j = 0; j < NBW; ++j) {
              const i32x8 bf = i32x8{blo[u][j].x, blo[u][j].y, blo[u][j].z, blo[u][j].w,
                                     bhi[u][j].x, bhi[u][j].y, bhi[u][j].z, bhi[u][j].w};
              if constexpr (EPI == EPI_BLOCK) {
                const int col = min((nb0 + j) * 16, N - 1);
                const float s = p.sb[(size_t)(col >> 7) * nk + kt];
                const f32x4 part = mfma_fp8(af, bf, f32x4{0.f, 0.f, 0.f, 0.f});
                acc[mi][j].x = __builtin_fmaf(part.x, sa4[0] * s, acc[mi][j].x);
                acc[mi][j].y = __builtin_fmaf(part.y, sa4[1] * s, acc[mi][j].y);
                acc[mi][j].z = __builtin_fmaf(part.z, sa4[2] * s, acc[mi][j].z);
                acc[mi][j].w = __builtin_fmaf(part.w, sa4[3] * s, acc[mi][j].w);
              } else {
                acc[mi][j] = mfma_fp8(af, bf, acc[mi][j]);
              }
            }
          }
        } else {
#pragma unroll
          for (int j = 0; j < NBW; ++j) {
            i32x4 bl, bh;
            if constexpr (KIND == KIND_INT4) {
              bl = unpack_int4x16(b4lo[u][j]);
              bh = unpack_int4x16(b4hi[u][j]);
            } else {
              bl = blo[u][j];
              bh = bhi[u][j];
            }
#pragma unroll
            for (int mi = 0; mi < MR; ++mi) {
              acc[mi][j] = mfma_i8(alo[u][mi], bl, acc[mi][j]);
              acc[mi][j] = mfma_i8(ahi[u][mi], bh, acc[mi][j]);
            }
          }
        }
      }
    }
  }

  // ---- split-K reduction over the NW waves through LDS ----
  __shared__ __attribute__((aligned(16))) AccT red[NW > 1 ? (NW - 1) : 1][MR * NBW][64];
  if constexpr (NW > 1) {
    if (wave > 0) {
#pragma unroll
      for (int mi = 0; mi < MR; ++mi)
#pragma unroll
        for (int j = 0; j < NBW; ++j) red[wave - 1][mi * NBW + j][lane] = acc[mi][j];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 0; w < NW - 1; ++w)
#pragma unroll
      for (int mi = 0; mi < MR; ++mi)
#pragma unroll
        for (int j = 0; j < NBW; ++j) acc[mi][j] += red[w][mi * NBW + j][lane];
  }

  typedef typename OutT<OUT_BF16>::type OT;
#pragma unroll
  for (int mi = 0; mi < MR; ++mi) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = mi * 16 + lq * 4 + i;
      if (row >= M) continue;
      float s_a = 1.f;
      if constexpr (EPI == EPI_ROWCOL) s_a = p.sa[row];
#pragma unroll
      for (int j = 0; j < NBW; ++j) {
        const int col = (nb0 + j) * 16 + l16;
        if (col >= N) continue;
        const size_t idx = (size_t)row * N + col;
        if constexpr (EPI == EPI_RAW) {
          if constexpr (KIND == KIND_FP8)
            ((float*)p.c)[idx] = acc[mi][j][i];
          else
            ((int*)p.c)[idx] = acc[mi][j][i];
        } else {
          float v;
          if constexpr (KIND == KIND_FP8 || EPI == EPI_BLOCK)
            v = acc[mi][j][i];
          else
            v = (float)acc[mi][j][i];
          if constexpr (EPI == EPI_ROWCOL) v = (v * s_a) * p.sb[col];
          ((OT*)p.c)[idx] = cvt_out<OUT_BF16>(v);
        }
      }
    }
  }
}

}  // namespace flygemm
