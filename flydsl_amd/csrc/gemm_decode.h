// Small-M kernel: B is streamed from HBM straight into MFMA operand registers.
//
// A workgroup owns NBW 16-column blocks and one block of 16*MR rows.  Its NW waves split K
// (wave w takes K tiles w, w+NW, ...), each wave keeps UNROLL-1 K tiles of loads in flight
// ahead of the one it multiplies, and the NW partial accumulators are summed through LDS
// before the fused epilogue.  The K split is reduced inside the workgroup: no workspace, no
// atomics, no second launch, and the int32 sums stay exact.
//
// Decode (M <= 16*MR): one row block, the whole of A (a few hundred KB at most) stays in L2
// and the kernel is bound by reading B once; owning several column blocks per workgroup
// divides the A traffic (one A fragment serves NBW blocks).  Larger M with few output tiles
// (e.g. 128 x 4096): the grid also runs over row blocks, so 256 workgroups can share an output
// that a 64x128 tile would cover with 64.  The row blocks of one column group read the same B
// and are placed on one XCD, next to each other in dispatch order, so B comes from HBM once
// and is re-read from that XCD's L2.
//
// Per K tile a lane loads, for every owned 16-column block, the two 16-byte chunks
// (lane/16) and (lane/16)+4 of column (lane%16) -- the preshuffled layout makes each
// wave-wide load one contiguous 1 KB read, non-temporal when B is read once (NT_B) -- and the
// matching two chunks of A row (lane%16).  As in the large-M kernel, B is the MFMA's first
// operand, so a lane ends with row (lane%16) and four consecutive columns.
//
#pragma once
#include "gemm_common.h"

namespace flygemm {

// B loads: non-temporal (NT_B) when each B byte is read by one workgroup (decode shapes), plain
// when the row blocks of a column group re-read it from L2.
template <bool NT, typename T>
__device__ __forceinline__ T load_b(const T* p) {
  if constexpr (NT)
    return __builtin_nontemporal_load(p);
  else
    return *p;
}

// NW = 4: two workgroups share a CU (at most 256 registers per lane, as for 8 waves), so one
// workgroup's reduction and epilogue run under the other's loads.
template <int MR, int NBW, int NW, int UNROLL, int KIND, int EPI, bool OUT_BF16, bool NT_B = true>
__global__ void __launch_bounds__(NW * 64, 8 / NW) gemm_decode_kernel(GemmArgs p) {
  const int M = p.M, N = p.N, K = p.K;
  // full 128-byte K tiles; K (bytes) is a multiple of 64, and when K % 128 == 64 the last 64
  // bytes form a half tile, taken after the pipeline (see below)
  const int nk = K / KT;
  const bool half_k = (K % KT) != 0;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // Wave-uniform (SGPR) wave index: every branch that guards an MFMA below depends only
  // on it, so the compiler emits scalar branches.  Guarding an MFMA by EXEC masking instead
  // would not skip it (the matrix core computes the whole tile), and a skipped tile's
  // operand registers were never loaded.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15;
  const int lq = lane >> 4;
  const int nblk_max = N / 16 - 1;
  // workgroup -> (row block, column group).  With several row blocks, XCD x (workgroups are
  // dealt to the 8 XCDs round-robin) gets a contiguous range of logical ids, row block
  // fastest, so the row blocks sharing a column group run together on one XCD.
  const int nrb = (M + 16 * MR - 1) / (16 * MR);
  int bid = blockIdx.x;
  const int G = gridDim.x;
  if (nrb > 1 && (G & 7) == 0) bid = (bid & 7) * (G >> 3) + (bid >> 3);
  const int m0 = (bid % nrb) * 16 * MR;
  const int nb0 = (bid / nrb) * NBW;

  constexpr int B_BLK = (KIND == KIND_INT4) ? 1024 : 2048;
  constexpr size_t B_PER_K = B_BLK / KT;  // bytes of one 16-col block per K element (16 or 8)

  typedef typename std::conditional<kind_float_acc(KIND) || EPI == EPI_BLOCK, f32x4, i32x4>::type AccT;
  // per-token / per-channel scaling (not applied to 16-bit inputs, whose scale pointers may be
  // null, nor to MXFP4, whose block scales are applied by the MFMA)
  constexpr bool kScaled = EPI == EPI_ROWCOL && !kind_unscaled(KIND);
  AccT acc[MR][NBW];
#pragma unroll
  for (int i = 0; i < MR; ++i)
#pragma unroll
    for (int j = 0; j < NBW; ++j) acc[i][j] = AccT{0, 0, 0, 0};

  const uint8_t* arow[MR];
#pragma unroll
  for (int mi = 0; mi < MR; ++mi) arow[mi] = p.a + (size_t)min(m0 + mi * 16 + l16, M - 1) * K + lq * 16;
  const uint8_t* bblk[NBW];
#pragma unroll
  for (int j = 0; j < NBW; ++j) {
    const int nb = min(nb0 + j, nblk_max);
    if constexpr (KIND == KIND_INT4)
      bblk[j] = p.b + (size_t)nb * B_PER_K * K + lq * 128 + l16 * 8;
    else
      bblk[j] = p.b + (size_t)nb * B_PER_K * K + lq * 256 + l16 * 16;
  }

  // Rolling pipeline over this wave's K tiles (kt = wave, wave + NW, ...): UNROLL register
  // stages, so the loads of the next UNROLL-1 tiles are in flight while one tile is
  // multiplied; the stage index is a compile-time constant inside the unrolled body.
  struct Stage {
    i32x4 alo[MR], ahi[MR];
    i32x4 blo[NBW], bhi[NBW];
    i32x2 b4lo[NBW], b4hi[NBW];
    float sa[MR], sb[NBW];  // blockscale: this K tile's A scale per row block, B scale per column block
    uint32_t fa[MR], fb[NBW];  // MXFP4: scale words, already shifted to the block's byte pair
  };
  Stage st[UNROLL];
  auto load = [&](Stage& s, int kt) {
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      const uint8_t* src = bblk[j] + (size_t)kt * B_BLK;
      if constexpr (KIND == KIND_INT4) {
        s.b4lo[j] = load_b<NT_B>((const i32x2*)src);
        s.b4hi[j] = load_b<NT_B>((const i32x2*)(src + 512));
      } else {
        s.blo[j] = load_b<NT_B>((const i32x4*)src);
        s.bhi[j] = load_b<NT_B>((const i32x4*)(src + 1024));
      }
    }
#pragma unroll
    for (int mi = 0; mi < MR; ++mi) {
      const uint8_t* src = arow[mi] + (size_t)kt * KT;
      s.alo[mi] = *(const i32x4*)src;
      s.ahi[mi] = *(const i32x4*)(src + 64);
    }
    // blockscale / MXFP4 scales travel with the stage, so their latency hides behind the pipeline
    if constexpr (KIND == KIND_FP4) {
      const uint32_t* wa = (const uint32_t*)p.sa;
      const uint32_t* wb = (const uint32_t*)p.sb;
      // row block r16 = m0/16 + mi is half (r16 & 1) of 32-row scale group r16 / 2
#pragma unroll
      for (int mi = 0; mi < MR; ++mi) {
        const int r16 = (m0 >> 4) + mi;
        s.fa[mi] = wa[((size_t)min(r16 >> 1, (M + 31) / 32 - 1) * nk + kt) * 64 + lane] >> (8 * (r16 & 1));
      }
#pragma unroll
      for (int j = 0; j < NBW; ++j) {
        const int nb = min(nb0 + j, nblk_max);
        s.fb[j] = wb[((size_t)(nb >> 1) * nk + kt) * 64 + lane] >> (8 * (nb & 1));
      }
    }
    if constexpr (EPI == EPI_BLOCK) {
#pragma unroll
      for (int mi = 0; mi < MR; ++mi) s.sa[mi] = p.sa[(size_t)kt * M + min(m0 + mi * 16 + l16, M - 1)];
#pragma unroll
      for (int j = 0; j < NBW; ++j) s.sb[j] = p.sb[(size_t)(min((nb0 + j) * 16, N - 1) >> 7) * nk + kt];
    }
  };
  auto compute = [&](const Stage& s, int kt) {
    auto a_lo = [&](int mi) -> const i32x4& { return s.alo[mi]; };
    auto a_hi = [&](int mi) -> const i32x4& { return s.ahi[mi]; };
    if constexpr (KIND == KIND_FP8) {
#pragma unroll
      for (int mi = 0; mi < MR; ++mi) {
        const i32x4 al = a_lo(mi), ah = a_hi(mi);
        const i32x8 af = i32x8{al.x, al.y, al.z, al.w, ah.x, ah.y, ah.z, ah.w};
        float s_a = 0.f;
        if constexpr (EPI == EPI_BLOCK) s_a = s.sa[mi];
#pragma unroll
        for (int j = 0; j < NBW; ++j) {
          const i32x8 bf = i32x8{s.blo[j].x, s.blo[j].y, s.blo[j].z, s.blo[j].w,
                                 s.bhi[j].x, s.bhi[j].y, s.bhi[j].z, s.bhi[j].w};
          if constexpr (EPI == EPI_BLOCK) {
            const float sc = s_a * s.sb[j];
            const f32x4 part = mfma_fp8(bf, af, f32x4{0.f, 0.f, 0.f, 0.f});
            acc[mi][j].x = __builtin_fmaf(part.x, sc, acc[mi][j].x);
            acc[mi][j].y = __builtin_fmaf(part.y, sc, acc[mi][j].y);
            acc[mi][j].z = __builtin_fmaf(part.z, sc, acc[mi][j].z);
            acc[mi][j].w = __builtin_fmaf(part.w, sc, acc[mi][j].w);
          } else {
            acc[mi][j] = mfma_fp8(bf, af, acc[mi][j]);
          }
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < NBW; ++j) {
        i32x4 bl, bh;
        if constexpr (KIND == KIND_INT4) {
          bl = unpack_int4x16(s.b4lo[j]);
          bh = unpack_int4x16(s.b4hi[j]);
        } else {
          bl = s.blo[j];
          bh = s.bhi[j];
        }
#pragma unroll
        for (int mi = 0; mi < MR; ++mi) {
          if constexpr (KIND == KIND_FP4) {
            acc[mi][j] = mfma_fp4<0>(bl, s.alo[mi], acc[mi][j], s.fb[j], s.fa[mi]);
            acc[mi][j] = mfma_fp4<1>(bh, s.ahi[mi], acc[mi][j], s.fb[j], s.fa[mi]);
          } else {
            acc[mi][j] = mfma_k64<KIND>(bl, a_lo(mi), acc[mi][j]);
            acc[mi][j] = mfma_k64<KIND>(bh, a_hi(mi), acc[mi][j]);
          }
        }
      }
    }
  };

  // The half K tile (index nk), taken first by the wave whose K tiles it continues (nk % NW),
  // before the pipeline's registers are in use: its lower 64 bytes (A chunks 0-3, B chunks 0-3)
  // are loaded and the upper halves are zeros, so the second 64-deep MFMA (and the upper half
  // of the 128-deep fp8 one) adds nothing; nothing past K is read.  Blockscale and MXFP4 take
  // whole K tiles only.
  if constexpr (EPI != EPI_BLOCK && KIND != KIND_FP4) {
    if (half_k && wave == nk % NW) {
      Stage& s = st[0];
#pragma unroll
      for (int j = 0; j < NBW; ++j) {
        const uint8_t* src = bblk[j] + (size_t)nk * B_BLK;
        if constexpr (KIND == KIND_INT4) {
          s.b4lo[j] = load_b<NT_B>((const i32x2*)src);
          s.b4hi[j] = i32x2{0, 0};
        } else {
          s.blo[j] = load_b<NT_B>((const i32x4*)src);
          s.bhi[j] = i32x4{0, 0, 0, 0};
        }
      }
#pragma unroll
      for (int mi = 0; mi < MR; ++mi) {
        const uint8_t* src = arow[mi] + (size_t)nk * KT;
        s.alo[mi] = *(const i32x4*)src;
        s.ahi[mi] = i32x4{0, 0, 0, 0};
      }
      compute(s, nk);
    }
  }
#pragma unroll
  for (int u = 0; u < UNROLL - 1; ++u)
    if (wave + u * NW < nk) load(st[u], wave + u * NW);
  for (int kt0 = wave; kt0 < nk; kt0 += NW * UNROLL) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int kt = kt0 + u * NW;
      const int kl = kt + (UNROLL - 1) * NW;  // the tile whose loads go out now
      if (kl < nk) load(st[(u + UNROLL - 1) % UNROLL], kl);
      if (kt < nk) compute(st[u], kt);
    }
  }

  // ---- split-K reduction over the NW waves through LDS: column block j is summed and
  // written out by wave j % NW ----
  __shared__ __attribute__((aligned(16))) AccT red[NW][MR * NBW][64];
#pragma unroll
  for (int mi = 0; mi < MR; ++mi)
#pragma unroll
    for (int j = 0; j < NBW; ++j) red[wave][mi * NBW + j][lane] = acc[mi][j];
  __syncthreads();

  typedef typename std::conditional<kind_float_acc(KIND) || EPI == EPI_BLOCK, float, int>::type AccE;
#pragma unroll
  for (int j = 0; j < NBW; ++j) {
    if (j % NW != wave) continue;
    const int col = (nb0 + j) * 16 + lq * 4;
    if (col >= N) continue;
    f32x4 sb4 = f32x4{1.f, 1.f, 1.f, 1.f};
    if constexpr (kScaled) sb4 = *(const f32x4*)(p.sb + col);
#pragma unroll
    for (int mi = 0; mi < MR; ++mi) {
      AccT s = red[0][mi * NBW + j][lane];
#pragma unroll
      for (int w = 1; w < NW; ++w) s += red[w][mi * NBW + j][lane];
      s = int4_acc<KIND>(s);
      const int row = m0 + mi * 16 + l16;
      if (row >= M) continue;
      const size_t idx = (size_t)row * N + col;
      if constexpr (EPI == EPI_RAW) {
        *(AccT*)((AccE*)p.c + idx) = s;
      } else {
        float s_a = 1.f;
        if constexpr (kScaled) s_a = p.sa[row];
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          v[r] = (float)s[r];
          if constexpr (kScaled) v[r] = (v[r] * s_a) * sb4[r];
        }
        *(i32x2*)((typename OutT<OUT_BF16>::type*)p.c + idx) = pack_out4<OUT_BF16>(v);
      }
    }
  }
}

}  // namespace flygemm
