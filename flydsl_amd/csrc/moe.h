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
};

enum MoeOut : int { MOE_OUT_F16 = 0, MOE_OUT_BF16 = 1, MOE_OUT_F32 = 2 };

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

  // flattened grid: column tile fastest, then sorted block
  const int ntn = p.N / TN;
  const int by = blockIdx.x / ntn;
  const int n0 = (blockIdx.x - by * ntn) * TN;
  if (by * TM >= p.num_valid[0]) return;
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

  // ---- epilogue: lane holds row mi*16 + l16 of the block, columns 4*lq .. 4*lq+3 of each
  // 16-column block ----
  constexpr bool kScaled = !kind_is_16bit(KIND);
#pragma unroll
  for (int mi = 0; mi < MR; ++mi) {
    const int i = by * TM + mi * 16 + l16;
    const int id = p.sorted_ids[i];
    const int t = id & 0xFFFFFF, s = (int)((uint32_t)id >> 24);
    if (t >= p.tokens || s >= p.topk) continue;
    const int arow = STAGE == 1 ? t : t * p.topk + s;
    const float sx = kScaled ? p.sa[arow] : 1.f;
    const float rw = p.doweight ? p.sorted_w[i] : 1.f;
#pragma unroll
    for (int ni = 0; ni < NR; ++ni) {
      const int n = n0 + (wave * NR + ni) * 16 + lq * 4;
      float v[4];
      if constexpr (STAGE == 1) {
        f32x4 swg = f32x4{1.f, 1.f, 1.f, 1.f}, swu = swg;
        if constexpr (kScaled) {
          swg = *(const f32x4*)(p.sw + (size_t)e * 2 * p.N + n);
          swu = *(const f32x4*)(p.sw + (size_t)e * 2 * p.N + p.N + n);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float g = ((float)acc[0][mi][ni][r] * sx) * swg[r];
          const float u = ((float)acc[1][mi][ni][r] * sx) * swu[r];
          v[r] = silu_f(g) * u;
          if (p.doweight) v[r] *= rw;
        }
        const size_t o = ((size_t)t * p.topk + s) * p.N + n;
        if constexpr (OUT == MOE_OUT_BF16)
          *(i32x2*)((__bf16*)p.out + o) = pack_out4<true>(v);
        else
          *(i32x2*)((_Float16*)p.out + o) = pack_out4<false>(v);
      } else {
        f32x4 swd = f32x4{1.f, 1.f, 1.f, 1.f};
        if constexpr (kScaled) swd = *(const f32x4*)(p.sw + (size_t)e * p.N + n);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          v[r] = ((float)acc[0][mi][ni][r] * sx) * swd[r];
          if (p.doweight) v[r] *= rw;
        }
        const size_t o = (size_t)t * p.N + n;
        if constexpr (OUT == MOE_OUT_F32) {
          float* dst = (float*)p.out + o;
#pragma unroll
          for (int r = 0; r < 4; ++r) unsafeAtomicAdd(dst + r, v[r]);
        } else if constexpr (OUT == MOE_OUT_BF16) {
          typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
          bf16x2* dst = (bf16x2*)((__bf16*)p.out + o);
          __builtin_amdgcn_global_atomic_fadd_v2bf16(dst, bf16x2{(__bf16)v[0], (__bf16)v[1]});
          __builtin_amdgcn_global_atomic_fadd_v2bf16(dst + 1, bf16x2{(__bf16)v[2], (__bf16)v[3]});
        } else {
          typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
          f16x2* dst = (f16x2*)((_Float16*)p.out + o);
          __builtin_amdgcn_global_atomic_fadd_v2f16(dst, f16x2{(_Float16)v[0], (_Float16)v[1]});
          __builtin_amdgcn_global_atomic_fadd_v2f16(dst + 1, f16x2{(_Float16)v[2], (_Float16)v[3]});
        }
      }
    }
  }
}

}  // namespace flygemm
