// MoE 2-stage GEMM for gfx950: the grouped GEMMs of a mixture-of-experts layer over routing
// metadata sorted by expert (reference kernels/moe_gemm_2stage.py: compile_moe_gemm1 :93-1264,
// compile_moe_gemm2 :1267-2481; semantics tests/kernels/test_ref.py:7-141).
//
// Routing metadata (the reference's moe_sorting, tests/kernels/test_moe_gemm.py:97-162):
//   sorted_token_ids[i] = (slot << 24) | token, grouped by expert, each expert's run padded to
//   a multiple of tile_m with (topk << 24) | tokens; sorted_expert_ids[b] = the expert of rows
//   [b*tile_m, (b+1)*tile_m); sorted_weights[i] = the routing weight of entry i;
//   num_valid_ids[0] = the padded row count (blocks at or past it exit at once).
//
// Stage 1, for each sorted row i of a block with expert e, token t, slot s, and n < I:
//   g = (x[t] . W1[e*2I + n]) * sx[t] * sw1[e*2I + n]
//   u = (x[t] . W1[e*2I + I + n]) * sx[t] * sw1[e*2I + I + n]
//   out1[t][s][n] = silu(g) * u  (* sorted_weights[i] if doweight)
// Stage 2, for n < D:
//   out2[t][n] += (a2[t*topk + s] . W2[e*D + n]) * sa2[t*topk + s] * sw2[e*D + n]
//                 (* sorted_weights[i] if doweight), with global atomics.
// 16-bit inputs carry no scales (the factors are 1).
//
// W1 and W2 are preshuffled like every B operand here.  A rows are gathered by the LDS-DMA:
// each lane's buffer offset names its own row, and padding rows get an offset past the buffer,
// which reads zeros.  One workgroup (4 waves) per (TN-column block, sorted block of TM rows);
// wave w owns columns [w*TN/4, (w+1)*TN/4) of the block for all TM rows (stage 1: of the gate
// and of the up projection).  Two LDS stages, one barrier per 128-byte K tile, LDS layouts as in
// the large-M kernel (gemm_main.h): A rows with the XOR chunk swizzle, B copied verbatim.
#pragma once
#include "gemm_main.h"

namespace flygemm {

struct MoeArgs {
  void* out;
  const uint8_t* a;            // stage 1: x [tokens][K]; stage 2: a2 [tokens*topk][K]  (K in bytes)
  const uint8_t* w;            // preshuffled W1 [E*2I][K] / W2 [E*D][K]
  const float* sa;             // stage 1: [tokens]; stage 2: [tokens*topk]   (unused for 16-bit)
  const float* sw;             // [E*2I] / [E*D]                                 (unused for 16-bit)
  const int32_t* sorted_ids;
  const int32_t* expert_ids;
  const float* sorted_w;
  const int32_t* num_valid;
  int tokens, topk, N, K;      // N: inter_dim (stage 1) or model_dim (stage 2); K in bytes
  int experts;
  int doweight;
  int blocks;                  // sorted blocks (size_expert_ids)
};

// Stage-2 outputs: F16/BF16/F32 accumulate into out[token] with atomics; *_ROWS store each
// route's row out[token*topk + slot] with plain stores (the reduce mode, summed by
// moe_reduce_kernel afterwards).  Stage 1 takes F16 or BF16.
enum MoeOut : int { MOE_OUT_F16 = 0, MOE_OUT_BF16 = 1, MOE_OUT_F32 = 2, MOE_OUT_F16_ROWS = 3, MOE_OUT_BF16_ROWS = 4 };
constexpr bool moe_out_bf16(int o) { return o == MOE_OUT_BF16 || o == MOE_OUT_BF16_ROWS; }

// x * sigmoid(x) = x / (1 + 2^(-x log2 e)) with the hardware exp2 and reciprocal
// (reference moe_gemm_2stage.py:271-281 evaluates it the same way)
__device__ __forceinline__ float silu_f(float x) {
  const float e = __builtin_amdgcn_exp2f(x * -1.4426950408889634f);
  return x * __builtin_amdgcn_rcpf(1.f + e);
}

template <int STAGE, int KIND, int TM, int TN>
struct MoeCfg {
  static constexpr int NW = 4;
  static constexpr int MR = TM / 16;                 // 16-row blocks (every wave covers all rows)
  static constexpr int NR = TN / 64;                 // 16-column blocks per wave
  static constexpr int NB = STAGE == 1 ? 2 : 1;      // weight halves: gate and up in stage 1
  static constexpr int A_BYTES = TM * KT;
  static constexpr int B_BYTES = NB * (TN / 16) * 2048;
  static constexpr int A_DMA = A_BYTES / 1024;       // 1 KB DMA instructions per K tile
  static constexpr int B_DMA = B_BYTES / 1024;
  static constexpr int AQ = (A_DMA + NW - 1) / NW;   // A instructions per wave
  static constexpr int STG = A_BYTES + B_BYTES;
  static_assert(TM % 16 == 0 && TN % 64 == 0 && A_BYTES % 1024 == 0 && B_DMA % NW == 0, "tile shape");
  static_assert(2 * STG <= 160 * 1024, "two stages must fit in LDS");
};

template <int STAGE, int KIND, int TM, int TN, int OUT>
__global__ void __launch_bounds__(256) moe_gemm_kernel(MoeArgs p) {
  using C = MoeCfg<STAGE, KIND, TM, TN>;
  constexpr int NW = C::NW, MR = C::MR, NR = C::NR, NB = C::NB;
  static_assert(KIND == KIND_FP8 || KIND == KIND_INT8 || kind_is_16bit(KIND), "MoE input kinds");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[2][C::STG];

  // Workgroups are dealt to the 8 XCDs round-robin.  Logical tile L (column tile fastest, then
  // sorted block) runs as workgroup (L % chunk) * 8 + L / chunk, i.e. each XCD takes one
  // contiguous range of L, so the consecutive blocks of one expert share that XCD's L2 copy of
  // the expert's weights instead of each XCD fetching them.  The grid has at least 8 * chunk
  // workgroups.
  // Only the tiles of blocks below num_valid_ids are dealt out, so a short routing (decode)
  // still spreads over every XCD.
  const int nv = p.num_valid[0];
  const int ntn = p.N / TN;
  const int V = ntn * min((nv + TM - 1) / TM, p.blocks);
  const int chunk = (V + 7) >> 3;
  const int L = (blockIdx.x & 7) * chunk + (blockIdx.x >> 3);
  if ((int)(blockIdx.x >> 3) >= chunk || L >= V) return;
  const int by = L / ntn;
  const int n0 = (L - by * ntn) * TN;
  const int e = p.expert_ids[by];
  if (e < 0 || e >= p.experts) return;
  const int K = p.K;
  const int nk = K / KT;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lq = lane >> 4;
  const int a_rows = STAGE == 1 ? p.tokens : p.tokens * p.topk;

  // A gather: DMA instruction q fills tile rows 8q .. 8q+7; lane l brings the chunk that
  // belongs in slot l%8 of row 8q + l/8.  Padding entries (token >= tokens) read zeros.
  uint32_t va[C::AQ];
#pragma unroll
  for (int j = 0; j < C::AQ; ++j) {
    const int rloc = min((wave + j * NW) * 8 + (lane >> 3), TM - 1);
    const int id = p.sorted_ids[by * TM + rloc];
    const int t = id & 0xFFFFFF, s = (int)((uint32_t)id >> 24);
    const int row = STAGE == 1 ? t : t * p.topk + s;
    const int c = (lane & 7) ^ ((rloc >> 1) & 7);
    va[j] = (t < p.tokens && s < p.topk) ? (uint32_t)row * (uint32_t)K + (uint32_t)(c * 16) : 0x80000000u;
  }
  const sgpr4 rsrc_a = buf_desc(p.a, (uint32_t)a_rows * (uint32_t)K);
  // this expert's weight rows only (the whole array may exceed 32-bit offsets)
  const int wrows = STAGE == 1 ? 2 * p.N : p.N;
  const sgpr4 rsrc_w = buf_desc(p.w + (size_t)e * (size_t)wrows * (size_t)K, (uint32_t)wrows * (uint32_t)K);
  const uint32_t vb = (uint32_t)lane * 16u;

  auto issue = [&](uint8_t* st, int kt) {
#pragma unroll
    for (int j = 0; j < C::AQ; ++j) {
      const int q = wave + j * NW;
      if (q < C::A_DMA) dma16(rsrc_a, st + q * 1024, va[j], (uint32_t)kt * KT);
    }
#pragma unroll
    for (int j = 0; j < C::B_DMA / NW; ++j) {
      const int q = wave + j * NW;           // 1 KB piece q: local 16-row block q/2, half q%2
      const int lb = q >> 1;                 // blocks [0, TN/16): gate (or W2); then up
      const int nb = lb < TN / 16 ? n0 / 16 + lb : (p.N + n0) / 16 + (lb - TN / 16);
      const uint32_t so = (uint32_t)nb * 16u * (uint32_t)K + (uint32_t)kt * 2048u + (uint32_t)(q & 1) * 1024u;
      dma16(rsrc_w, st + C::A_BYTES + q * 1024, vb, __builtin_amdgcn_readfirstlane(so));
    }
  };

  typedef typename std::conditional<kind_float_acc(KIND), f32x4, i32x4>::type AccT;
  AccT acc[NB][MR][NR];
#pragma unroll
  for (int h = 0; h < NB; ++h)
#pragma unroll
    for (int i = 0; i < MR; ++i)
#pragma unroll
      for (int j = 0; j < NR; ++j) acc[h][i][j] = AccT{0, 0, 0, 0};

  // One K tile: the A fragments of every row block are read once, then each weight fragment
  // is read and applied to all of them.  B is the MFMA's first operand, so each accumulator
  // tile holds its 16x16 block of the output transposed.
  auto compute = [&](const uint8_t* sA) {
    const uint8_t* sB = sA + C::A_BYTES;
    i32x4 alo[MR], ahi[MR];
#pragma unroll
    for (int mi = 0; mi < MR; ++mi) {
      const int row = mi * 16 + l16;
      const int sw = (row >> 1) & 7;
      alo[mi] = *(const i32x4*)(sA + row * KT + ((lq ^ sw) << 4));
      ahi[mi] = *(const i32x4*)(sA + row * KT + (((lq + 4) ^ sw) << 4));
    }
#pragma unroll
    for (int h = 0; h < NB; ++h)
#pragma unroll
      for (int ni = 0; ni < NR; ++ni) {
        const int off = (h * (TN / 16) + wave * NR + ni) * 2048 + lq * 256 + l16 * 16;
        const i32x4 blo = *(const i32x4*)(sB + off);
        const i32x4 bhi = *(const i32x4*)(sB + off + 1024);
        if constexpr (KIND == KIND_FP8) {
          const i32x8 bf = i32x8{blo.x, blo.y, blo.z, blo.w, bhi.x, bhi.y, bhi.z, bhi.w};
#pragma unroll
          for (int mi = 0; mi < MR; ++mi)
            acc[h][mi][ni] = mfma_fp8(bf, i32x8{alo[mi].x, alo[mi].y, alo[mi].z, alo[mi].w, ahi[mi].x, ahi[mi].y,
                                                ahi[mi].z, ahi[mi].w},
                                      acc[h][mi][ni]);
        } else {
#pragma unroll
          for (int mi = 0; mi < MR; ++mi) acc[h][mi][ni] = mfma_k64<KIND>(blo, alo[mi], acc[h][mi][ni]);
#pragma unroll
          for (int mi = 0; mi < MR; ++mi) acc[h][mi][ni] = mfma_k64<KIND>(bhi, ahi[mi], acc[h][mi][ni]);
        }
      }
  };

  issue(lds[0], 0);
  for (int kt = 0; kt < nk; ++kt) {
    wait_dma();
    workgroup_barrier();  // tile kt has landed; every wave is done reading the other stage
    if (kt + 1 < nk) issue(lds[(kt + 1) & 1], kt + 1);
    compute(lds[kt & 1]);
  }

  // ---- epilogue, through LDS so that global writes are row-contiguous ----
  // Phase 1: lane (l16, lq) holds row mi*16 + l16 of the block and columns 4*lq .. 4*lq+3 of
  // each 16-column block; it scales them and writes them to an LDS tile [TM][TN] (padded rows).
  // Phase 2: the workgroup walks the tile row by row, each wave instruction covering 256
  // contiguous bytes of one output row: 16-byte stores (stage 1) or 4-byte atomics (stage 2;
  // fp16/bf16 as packed pairs).  Scattered 4-lane fragments would touch 16 cache lines per
  // instruction, which costs the atomics 8x their useful rate.
  constexpr bool kScaled = !kind_is_16bit(KIND);
  constexpr bool kRows = STAGE == 1 || OUT == MOE_OUT_F16_ROWS || OUT == MOE_OUT_BF16_ROWS;  // plain stores
  constexpr int ESZ = (STAGE == 2 && OUT == MOE_OUT_F32) ? 4 : 2;
  constexpr int RS = TN * ESZ + 16;            // LDS bytes per tile row (padding spreads banks)
  static_assert(TM * RS + TM * 4 <= 2 * C::STG, "output tile fits in the stage buffers");
  uint8_t* ot = &lds[0][0];
  int32_t* rowdst = (int32_t*)(ot + TM * RS);  // destination row per tile row, -1 for padding
  workgroup_barrier();                         // every wave is done with the last K tile
#pragma unroll
  for (int mi = 0; mi < MR; ++mi) {
    const int r = mi * 16 + l16;
    const int i = by * TM + r;
    const int id = p.sorted_ids[i];
    const int t = id & 0xFFFFFF, s = (int)((uint32_t)id >> 24);
    const bool valid = t < p.tokens && s < p.topk;
    if (wave == 0 && lq == 0) rowdst[r] = !valid ? -1 : (kRows ? t * p.topk + s : t);
    const int arow = STAGE == 1 ? t : t * p.topk + s;
    const float sx = kScaled && valid ? p.sa[arow] : 1.f;
    const float rw = p.doweight && valid ? p.sorted_w[i] : 1.f;
#pragma unroll
    for (int ni = 0; ni < NR; ++ni) {
      const int c = (wave * NR + ni) * 16 + lq * 4;
      const int n = n0 + c;
      float v[4];
      if constexpr (STAGE == 1) {
        f32x4 swg = f32x4{1.f, 1.f, 1.f, 1.f}, swu = swg;
        if constexpr (kScaled) {
          swg = *(const f32x4*)(p.sw + (size_t)e * 2 * p.N + n);
          swu = *(const f32x4*)(p.sw + (size_t)e * 2 * p.N + p.N + n);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float g = ((float)acc[0][mi][ni][q] * sx) * swg[q];
          const float u = ((float)acc[1][mi][ni][q] * sx) * swu[q];
          v[q] = silu_f(g) * u;
          if (p.doweight) v[q] *= rw;
        }
      } else {
        f32x4 swd = f32x4{1.f, 1.f, 1.f, 1.f};
        if constexpr (kScaled) swd = *(const f32x4*)(p.sw + (size_t)e * p.N + n);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          v[q] = ((float)acc[0][mi][ni][q] * sx) * swd[q];
          if (p.doweight) v[q] *= rw;
        }
      }
      uint8_t* dst = ot + r * RS + c * ESZ;
      if constexpr (ESZ == 4)
        *(f32x4*)dst = f32x4{v[0], v[1], v[2], v[3]};
      else
        *(i32x2*)dst = pack_out4<moe_out_bf16(OUT)>(v);
    }
  }
  workgroup_barrier();
  if constexpr (kRows) {
    constexpr int CPR = TN * 2 / 16;           // 16-byte chunks per output row
    for (int idx = tid; idx < TM * CPR; idx += 256) {
      const int r = idx / CPR, cc = idx - r * CPR;
      const int d = rowdst[r];
      if (d < 0) continue;
      const i32x4 val = *(const i32x4*)(ot + r * RS + cc * 16);
      *(i32x4*)((uint8_t*)p.out + ((size_t)d * p.N + n0) * 2 + cc * 16) = val;
    }
  } else {
    constexpr int WPR = TN * ESZ / 4;          // 4-byte words per output row
    for (int idx = tid; idx < TM * WPR; idx += 256) {
      const int r = idx / WPR, wd = idx - r * WPR;
      const int d = rowdst[r];
      if (d < 0) continue;
      uint8_t* dst = (uint8_t*)p.out + ((size_t)d * p.N + n0) * ESZ + wd * 4;
      const uint8_t* src = ot + r * RS + wd * 4;
      if constexpr (OUT == MOE_OUT_F32) {
        unsafeAtomicAdd((float*)dst, *(const float*)src);
      } else if constexpr (OUT == MOE_OUT_BF16) {
        typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
        __builtin_amdgcn_global_atomic_fadd_v2bf16((bf16x2*)dst, *(const bf16x2*)src);
      } else {
        typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
        __builtin_amdgcn_global_atomic_fadd_v2f16((f16x2*)dst, *(const f16x2*)src);
      }
    }
  }
}

// Reduce mode, second kernel: y[t][d] = sum over slots k of x[t][k][d] (slots with
// valid_mask[t][k] == 0 skipped when a mask is given), fp32 sums, one 16-byte vector of d per
// thread; x is read once, so it is loaded non-temporally (reference compile_moe_reduction,
// kernels/moe_gemm_2stage.py:2484-2604).  DT: 0 fp16, 1 bf16, 2 fp32.
template <int DT>
__global__ void __launch_bounds__(256) moe_reduce_kernel(void* y, const void* x, const int8_t* mask, int tokens,
                                                         int topk, int D) {
  constexpr int ESZ = DT == 2 ? 4 : 2;
  constexpr int VE = 16 / ESZ;                 // elements per vector
  const int vpr = D / VE;                      // vectors per row
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long)tokens * vpr) return;
  const int t = (int)(idx / vpr), v = (int)(idx - (long)t * vpr);
  float acc[VE];
#pragma unroll
  for (int q = 0; q < VE; ++q) acc[q] = 0.f;
  const i32x4* src = (const i32x4*)x + ((long)t * topk * vpr + v);
  for (int k = 0; k < topk; ++k) {
    if (mask && mask[(long)t * topk + k] == 0) continue;
    const i32x4 w = __builtin_nontemporal_load(src + (long)k * vpr);
    if constexpr (DT == 2) {
      const f32x4 f = __builtin_bit_cast(f32x4, w);
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[q] += f[q];
    } else {
      typedef typename OutT<DT == 1>::type ET;
      typedef ET ET8 __attribute__((ext_vector_type(8)));
      const ET8 h = __builtin_bit_cast(ET8, w);
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[q] += (float)h[q];
    }
  }
  i32x4* dst = (i32x4*)y + idx;
  if constexpr (DT == 2) {
    *dst = __builtin_bit_cast(i32x4, f32x4{acc[0], acc[1], acc[2], acc[3]});
  } else {
    const float lo[4] = {acc[0], acc[1], acc[2], acc[3]}, hi[4] = {acc[4], acc[5], acc[6], acc[7]};
    const i32x2 a = pack_out4<DT == 1>(lo), b = pack_out4<DT == 1>(hi);
    *dst = i32x4{a.x, a.y, b.x, b.y};
  }
}

}  // namespace flygemm
