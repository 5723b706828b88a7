// MoE stage 1 (gate/up projection) for gfx950 with the weights streamed straight into registers.
//
// The stage-1 product of the 2-stage MoE GEMM (semantics and routing metadata as moe.h; reference
// kernels/moe_gemm_2stage.py compile_moe_gemm1 :93-1264) for 1-byte (fp8, int8, int8smooth),
// 16-bit (bf16, fp16) and int4 weights with int8 activations (W4A8: the packed preshuffled bytes
// of the dense int4 path, unpacked to int8 in registers).
//
// One workgroup (4 waves) owns a run of up to R routing blocks of one expert (TM * R = 128 rows;
// a block starts a run when its index is a multiple of R or its expert differs from the previous
// block's) and one 64-column tile of the output: 64 gate and 64 up weight rows.  Wave w owns
// output columns [16w, 16w + 16) for all 128 rows, so no weight byte is shared between waves and
// the weights skip LDS: each wave loads its gate and up fragments from the preshuffled weights
// straight into registers (two coalesced loads per 16-column block per 128-byte K step, 1 KB
// each -- 512 bytes for int4 -- each lane's bytes being its MFMA operand), Lb = D - 1 steps ahead
// in D register sets.  Only the
// gathered activation rows, which all four waves read, go global -> LDS by DMA (each lane's
// buffer offset names its own row; padding rows read zeros past the buffer), one step ahead in a
// 2-slot ring.  A workgroup then needs 32 KB of LDS and two share a CU (8 waves, at most 256
// VGPRs each).  The kernel it replaces for these kinds kept the weights in LDS: the weights'
// L2 -> LDS DMA bounded its single-block tiles, and its 128-row tiles, whose two LDS stages
// filled a CU, waited out their loads one workgroup per CU.
//
// Wait discipline.  Loads retire in issue order on one vector memory counter.  A step s issues,
// after its barrier, the A DMA of step s+1, then the weights of step s+Lb, then computes.  The
// A DMA is inline assembly that the compiler does not track; its wait is explicit: at the top
// of step s the only operations issued after A(s) are the weights of step s-1+Lb (LPS of them).
// The compiler waits for a weight set counting only the later weight loads it knows of, so the
// untracked DMAs issued after that set make it also wait for the oldest Lb*AQ operations issued
// after the set: A(s) (already waited for) and some weights of step s+1, issued a step earlier.
// The loop runs whole groups of D steps (the register set of each step is static there and
// every path through a group issues every load); the last nk % D steps form a tail in which the
// weight loads of steps past the end are dead and removed by the compiler, so each tail step
// waits for everything instead.
#pragma once
#include "moe.h"

namespace flygemm {

// f(integral_constant<int, U>) for U = B .. E-1, each call inlined with U a constant
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

template <int KIND, int TM, int R, int D>
__global__ void __launch_bounds__(256, 2) moe_stream_kernel(MoeArgs p) {
  static_assert(KIND == KIND_FP8 || KIND == KIND_INT8 || KIND == KIND_INT4 || kind_is_16bit(KIND),
                "1-byte, 16-bit or int4 weights");
  constexpr bool I4 = KIND == KIND_INT4;
  constexpr uint32_t B_BLK = I4 ? 1024u : 2048u;     // bytes of one 16-row weight block per K step
  constexpr int NW = 4, TN = 64, NB = 2;               // waves, output columns, weight halves
  constexpr int TME = TM * R, MR = TME / 16;           // rows of a run, 16-row blocks
  constexpr int A_BYTES = TME * KT, AQ = A_BYTES / 1024 / NW;
  constexpr int LPS = NB * 2;                          // weight loads per wave per step
  constexpr int Lb = D - 1;
  static_assert(TME % 16 == 0 && A_BYTES % (1024 * NW) == 0 && D >= 3, "tile shape");
  __shared__ __attribute__((aligned(1024))) uint8_t ring[2 * A_BYTES];

  // ---- which run and column tile: logical id L = block * nsplit + column tile (nsplit = N / 64)
  // over the blocks below num_valid_ids, dealt to the 8 XCDs in contiguous ranges, as moe.h ----
  const int nv = p.num_valid[0];
  const int nbv = min((nv + TM - 1) / TM, p.blocks);
  const int V = nbv * p.nsplit;
  const int chunk = (V + 7) >> 3;
  const int L = (blockIdx.x & 7) * chunk + (blockIdx.x >> 3);
  if ((int)(blockIdx.x >> 3) >= chunk || L >= V) return;
  const int b0 = L / p.nsplit;
  const int jt = L - b0 * p.nsplit;
  const int e = p.expert_ids[b0];
  if (e < 0 || e >= p.experts) return;
  const int nblk = moe_run_blocks<R>(p.expert_ids, b0, e, nbv, threadIdx.x & 63);
  if (nblk == 0) return;                       // inside another run
  const int rows_valid = nblk * TM;
  const int K = p.K, nk = K / KT;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lq = lane >> 4;
  const bool a_ts = p.a_token_slot;
  const int a_rows = !a_ts ? p.tokens : p.tokens * p.topk;
  constexpr bool kScaled = !kind_is_16bit(KIND);

  // ---- per-row facts, fixed for the workgroup's life (as moe.h) ----
  // A gather: DMA instruction q fills run rows 8q .. 8q+7; lane l brings the chunk that belongs
  // in slot l%8 of row 8q + l/8 (XOR chunk swizzle of the large-M kernel).
  // (int4 keeps the per-row facts in LDS, below; idr: this lane's rows' ids otherwise)
  constexpr bool kLdsRows = I4;
  uint32_t va[AQ];
  int ida[AQ], idr[kLdsRows ? 1 : MR];
#pragma unroll
  for (int j = 0; j < AQ; ++j)
    ida[j] = p.sorted_ids[b0 * TM + min(min((wave + j * NW) * 8 + (lane >> 3), TME - 1), rows_valid - 1)];
  if constexpr (!kLdsRows) {
#pragma unroll
    for (int mi = 0; mi < MR; ++mi) idr[mi] = p.sorted_ids[b0 * TM + min(mi * 16 + l16, rows_valid - 1)];
  }
#pragma unroll
  for (int j = 0; j < AQ; ++j) {
    const int rloc = min((wave + j * NW) * 8 + (lane >> 3), TME - 1);
    const int id = ida[j];
    const int t = id & 0xFFFFFF, s = (int)((uint32_t)id >> 24);
    const bool ok = rloc < rows_valid && t < p.tokens && s < p.topk;
    const int row = a_ts ? s * p.tokens + t : t;
    const int c = (lane & 7) ^ ((rloc >> 1) & 7);
    va[j] = ok ? (uint32_t)row * (uint32_t)K + (uint32_t)(c * 16) : 0x80000000u;
  }
  // Per-row facts -- activation scale, routing weight, destination (-1: padding) -- and the
  // column scales, read by the epilogue.  int4 keeps them in LDS (row r's by thread r, read
  // after the first step's barrier): 158 instead of 192 VGPRs, so three workgroups share a CU,
  // graph-timed 4-8% faster (DS-TP8 dims, 64-row blocks, 2048 / 8192 / 16384 tokens 89-89.4 /
  // 235-238.5 / 420-422 us against 92.6-93.0 / 248-253 / 455-457, bit-equal).  The other kinds
  // keep them in registers: at three workgroups per CU int8 and bf16 were 5-22% slower and fp8
  // spills.
  __shared__ float s_sx[kLdsRows ? TME : 1], s_rw[kLdsRows ? TME : 1], s_sc[kLdsRows ? NB * TN : 1];
  __shared__ int s_dst[kLdsRows ? TME : 1];
  float sx_r[MR], rw_r[MR];
  int dst_r[MR];
  auto row_facts = [&](int r, int id, float& sxo, float& rwo, int& dsto) __attribute__((always_inline)) {
    const int t = id & 0xFFFFFF, s = (int)((uint32_t)id >> 24);
    const bool ok = r < rows_valid && t < p.tokens && s < p.topk;
    dsto = ok ? t * p.topk + s : -1;
    const int arow = ok ? (a_ts ? s * p.tokens + t : t) : 0;
    const float sxv = kScaled ? p.sa[arow] : 1.f;
    const float rwv = p.doweight ? p.sorted_w[b0 * TM + min(r, rows_valid - 1)] : 1.f;
    sxo = ok ? sxv : 0.f;  // 0 keeps padding rows finite; 1 for unscaled kinds
    rwo = ok ? rwv : 0.f;
  };
  if constexpr (kLdsRows) {
    if (tid < TME)
      row_facts(tid, p.sorted_ids[b0 * TM + min(tid, rows_valid - 1)], s_sx[tid], s_rw[tid], s_dst[tid]);
  } else {
#pragma unroll
    for (int mi = 0; mi < MR; ++mi) row_facts(mi * 16 + l16, idr[mi], sx_r[mi], rw_r[mi], dst_r[mi]);
  }
  const sgpr4 rsrc_a = buf_desc(p.a, (uint32_t)a_rows * (uint32_t)K);
  // this expert's gate/up rows only (the whole array may exceed 32-bit offsets)
  const int wrows = 2 * p.N;
  const uint32_t wrb = I4 ? (uint32_t)K / 2u : (uint32_t)K;   // weight bytes per row
  const __amdgpu_buffer_rsrc_t rsrc_w = make_rsrc(p.w + (size_t)e * (size_t)wrows * wrb, (int)(wrows * wrb));
  const __amdgpu_buffer_rsrc_t rsrc_s = make_rsrc(p.sw + (size_t)e * wrows, kScaled ? wrows * 4 : 0);
  const __amdgpu_buffer_rsrc_t rsrc_o = make_rsrc(p.out, (int)p.out_bytes);

  typedef typename std::conditional<kind_float_acc(KIND), f32x4, i32x4>::type AccT;
  AccT acc[NB][MR];
  typedef typename std::conditional<I4, i32x2, i32x4>::type BT;
  BT bw[D][NB][2];      // weight fragments of D steps: [set][gate/up][K half]
  f32x4 sc[NB];         // this lane's 4 column scales of the gate and of the up half

  // weights of step s into register set U: this wave's gate block (16 rows jt*64 + 16*wave ..)
  // and up block (the same rows + N), B_BLK bytes per K step each in the preshuffled layout
  // (lane (l16, lq) holds K bytes 16*lq .. of its row's first and second 64-byte halves: at
  // 16*lane and 1024 + 16*lane; int4: 8 packed bytes at 128*lq + 8*l16 and 512 past that);
  // steps past the end load zeros from past the buffer
  auto load_b = [&](auto u_tag, int s) __attribute__((always_inline)) {
    constexpr int U = decltype(u_tag)::value;
    const uint32_t past = s < nk ? 0u : 0x80000000u;
    const int kt = s < nk ? s : 0;
#pragma unroll
    for (int h = 0; h < NB; ++h) {
      const int gblk = (h ? p.N / 16 : 0) + jt * (TN / 16) + wave;
      const uint32_t so = (uint32_t)gblk * 16u * wrb + (uint32_t)kt * B_BLK;
      if constexpr (I4) {
        const uint32_t vo = (uint32_t)(lq * 128 + l16 * 8) + past;
        bw[U][h][0] = __builtin_amdgcn_raw_buffer_load_b64(rsrc_w, vo, __builtin_amdgcn_readfirstlane(so), 0);
        bw[U][h][1] = __builtin_amdgcn_raw_buffer_load_b64(rsrc_w, vo, __builtin_amdgcn_readfirstlane(so + 512u), 0);
      } else {
        const uint32_t vo = (uint32_t)lane * 16u + past;
        bw[U][h][0] = __builtin_amdgcn_raw_buffer_load_b128(rsrc_w, vo, __builtin_amdgcn_readfirstlane(so), 0);
        bw[U][h][1] = __builtin_amdgcn_raw_buffer_load_b128(rsrc_w, vo, __builtin_amdgcn_readfirstlane(so + 1024u), 0);
      }
    }
  };
  // A of step s into ring slot s & 1
  auto issue_a = [&](int s) __attribute__((always_inline)) {
    uint8_t* st = ring + (s & 1) * A_BYTES;
#pragma unroll
    for (int j = 0; j < AQ; ++j) dma16(rsrc_a, st + (wave + j * NW) * 1024, va[j], (uint32_t)s * KT);
  };
  // One K step from register set U and the A slot sA: row block by row block, the next row's A
  // fragment read ahead of this row's MFMAs.  B is the MFMA's first operand, so each accumulator
  // tile holds its 16x16 output block transposed.
  auto compute = [&](auto u_tag, const uint8_t* sA) __attribute__((always_inline)) {
    constexpr int U = decltype(u_tag)::value;
    auto load_a = [&](int mi, i32x4& lo, i32x4& hi) __attribute__((always_inline)) {
      const int row = mi * 16 + l16;
      const int sw = (row >> 1) & 7;
      lo = *(const i32x4*)(sA + row * KT + ((lq ^ sw) << 4));
      hi = *(const i32x4*)(sA + row * KT + (((lq + 4) ^ sw) << 4));
    };
    i32x4 alo, ahi;
    load_a(0, alo, ahi);
#pragma unroll
    for (int mi = 0; mi < MR; ++mi) {
      const i32x4 lo = alo, hi = ahi;
      if (mi + 1 < MR) load_a(mi + 1, alo, ahi);
#pragma unroll
      for (int h = 0; h < NB; ++h) {
        i32x4 bl, bh;
        if constexpr (I4) {
          bl = unpack_int4x16(bw[U][h][0]);
          bh = unpack_int4x16(bw[U][h][1]);
        } else {
          bl = bw[U][h][0];
          bh = bw[U][h][1];
        }
        if constexpr (KIND == KIND_FP8) {
          acc[h][mi] = mfma_fp8(__builtin_shufflevector(bl, bh, 0, 1, 2, 3, 4, 5, 6, 7),
                                __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7), acc[h][mi]);
        } else {
          constexpr int MK = I4 ? KIND_INT8 : KIND;   // int4 weights: the int8 MFMA
          acc[h][mi] = mfma_k64<MK>(bl, lo, acc[h][mi]);
          acc[h][mi] = mfma_k64<MK>(bh, hi, acc[h][mi]);
        }
      }
    }
  };

#pragma unroll
  for (int h = 0; h < NB; ++h)
#pragma unroll
    for (int mi = 0; mi < MR; ++mi) acc[h][mi] = AccT{0, 0, 0, 0};
  // prologue: weights of steps 0 .. Lb-1, this lane's column scales, A of step 0 (the first
  // step waits for all of them)
  static_for<0, Lb>([&](auto u) __attribute__((always_inline)) { load_b(u, decltype(u)::value); });
  if constexpr (kLdsRows) {
    if (tid < NB * TN) {
      const uint32_t col = (uint32_t)((tid / TN) * p.N + jt * TN + tid % TN);
      s_sc[tid] = kScaled ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc_s, col * 4u, 0, 0)) : 1.f;
    }
  } else {
#pragma unroll
    for (int h = 0; h < NB; ++h) {
      const uint32_t col = (uint32_t)(h * p.N + jt * TN + wave * 16 + lq * 4);
      sc[h] = kScaled ? __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc_s, col * 4u, 0, 0))
                      : f32x4{1.f, 1.f, 1.f, 1.f};
    }
  }
  issue_a(0);
  // Epilogue: out1[t][s][n] = silu(gate) * up (* routing weight), gate/up = accumulator *
  // activation scale * weight-row scale; lane (l16, lq) holds row mi*16 + l16, columns 4*lq ..
  // 4*lq+3 of this wave's 16; 8-byte row stores, padding rows at an offset past the buffer.  It
  // runs inside the last step: placed after the loop, the fp8 instances spilled 63-70 VGPRs.
  auto epilogue = [&]() __attribute__((always_inline)) {
    const bool obf16 = moe_out_bf16(p.out_mode);
    const int c = jt * TN + wave * 16 + lq * 4;
    if constexpr (kLdsRows) {
#pragma unroll
      for (int h = 0; h < NB; ++h) sc[h] = *(const f32x4*)(s_sc + h * TN + wave * 16 + lq * 4);
    }
#pragma unroll
    for (int mi = 0; mi < MR; ++mi) {
      const int r = mi * 16 + l16;
      const int d = kLdsRows ? s_dst[r] : dst_r[mi];
      const float sxm = kLdsRows ? s_sx[r] : sx_r[mi], rwm = kLdsRows ? s_rw[r] : rw_r[mi];
      float v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float g = ((float)int4_acc<KIND>(acc[0][mi][q]) * sxm) * sc[0][q];
        const float up = ((float)int4_acc<KIND>(acc[1][mi][q]) * sxm) * sc[1][q];
        v[q] = (silu_f(g) * up) * rwm;
      }
      const uint32_t off = d < 0 ? 0xFFFFFFF0u : ((uint32_t)d * (uint32_t)p.N + (uint32_t)c) * 2u;
      const i32x2 pk = obf16 ? pack_out4<true>(v) : pack_out4<false>(v);
      __builtin_amdgcn_raw_buffer_store_b64(pk, rsrc_o, off, 0, 0);
    }
  };
  auto step = [&](auto u_tag, int s, auto tail_tag) __attribute__((always_inline)) {
    constexpr int U = decltype(u_tag)::value;
    if (decltype(tail_tag)::value || s == 0)
      waitcnt<0>();
    else
      waitcnt<LPS>();   // A(s); only the weights of step s-1+Lb were issued after it
    workgroup_barrier();  // A(s) published; every wave is done with slot (s+1) & 1
    if (s + 1 < nk) issue_a(s + 1);
    load_b(std::integral_constant<int, (U + Lb) % D>{}, s + Lb);
    __builtin_amdgcn_sched_barrier(0);   // the loads go out before the MFMAs
    compute(u_tag, ring + (s & 1) * A_BYTES);
    if (s == nk - 1) epilogue();
  };
  int s0 = 0;
  for (; s0 + D <= nk; s0 += D)
    static_for<0, D>([&](auto u) __attribute__((always_inline)) {
      step(u, s0 + decltype(u)::value, std::false_type{});
    });
  static_for<0, D - 1>([&](auto u) __attribute__((always_inline)) {
    if (s0 + decltype(u)::value < nk) step(u, s0 + decltype(u)::value, std::true_type{});
  });
}

}  // namespace flygemm

namespace flygemm {

// MoE stage 2 with per-route row outputs (the reduce mode's GEMM; reference
// kernels/moe_gemm_2stage.py compile_moe_gemm2 :1267-2481 with accumulate = False, summed by
// moe_reduce_kernel) for 1-byte, int4 (with int8 activations) and 16-bit weights and inter_dim of
// NK <= 4 128-byte K steps.
//
// One workgroup (4 waves) owns a run of up to R routing blocks of one expert (TM * R = 128 rows;
// 32 or 64 for the single-block form of routings with few routes per expert) and a range of
// 64-column output tiles (nsplit ranges per run).  The run's gathered A rows -- all NK
// K steps -- go to LDS once and stay there.  Wave w owns output columns [16w, 16w + 16) of each
// tile and loads their weight fragments (NK steps x two coalesced 1 KB loads) and column scales
// straight into registers, one column tile ahead: the loads of tile j+1 are issued before tile
// j's stores, so the compiler's wait for them (vector memory operations retire in issue order)
// never covers a store, and each tile's 16 KB of row stores drain while the next tile computes.
// The epilogue stages the tile through LDS in two rounds of 64 rows (one round for runs of 32
// rows; 16-byte chunk c of row r at chunk c ^ (r % 8)) and stores whole 128-byte row segments.  40 KB of LDS and at most 128 VGPRs
// let four workgroups share a CU.  DS-TP8 prefill (65536 routes, 7168 x 256, fp8), the GEMM and
// the reduction: 438 us against 586 for the single-block kernel with A resident (bit-equal);
// variants measured and not kept: three workgroups per CU with one staging round 453 us, the A
// fragments held in registers (two workgroups per CU) 478, 64-row runs 486-494, 2 / 3 / 6 / 8
// column ranges per run 574 / 470 / 468 / 444.
template <int KIND, int TM, int R, int NK>
__global__ void __launch_bounds__(256, 4) moe_stream2_kernel(MoeArgs p) {
  static_assert(KIND == KIND_FP8 || KIND == KIND_INT8 || KIND == KIND_INT4 || kind_is_16bit(KIND),
                "1-byte, int4 or 16-bit weights");
  constexpr bool I4 = KIND == KIND_INT4;
  constexpr int NW = 4, TN = 64, HALVES = TM * R >= 64 ? 2 : 1;   // staging rounds
  constexpr int TME = TM * R, MR = TME / 16;
  constexpr int A_STEP = TME * KT, AQ = A_STEP / 1024 / NW;
  constexpr int RB = TN * 2;                  // bytes of one output row of the tile
  constexpr int CPR = RB / 16;                // 16-byte chunks per row
  constexpr int HR = TME / HALVES;            // rows staged per round
  constexpr int SCH = HR * CPR / (NW * 64);   // store chunks per thread per round
  static_assert(SCH * NW * 64 == HR * CPR && MR % HALVES == 0 && NK >= 1 && NK <= 4, "tile shape");
  __shared__ __attribute__((aligned(1024))) uint8_t sa_lds[NK * A_STEP];
  __shared__ __attribute__((aligned(1024))) uint8_t stg[HR * RB];

  // ---- which run and column range (as moe.h) ----
  const int nv = p.num_valid[0];
  const int nbv = min((nv + TM - 1) / TM, p.blocks);
  const int V = nbv * p.nsplit;
  const int chunk = (V + 7) >> 3;
  const int L = (blockIdx.x & 7) * chunk + (blockIdx.x >> 3);
  if ((int)(blockIdx.x >> 3) >= chunk || L >= V) return;
  const int b0 = L / p.nsplit;
  const int split = L - b0 * p.nsplit;
  const int e = p.expert_ids[b0];
  if (e < 0 || e >= p.experts) return;
  const int nblk = moe_run_blocks<R>(p.expert_ids, b0, e, nbv, threadIdx.x & 63);
  if (nblk == 0) return;                       // inside another run
  const int rows_valid = nblk * TM;
  const int ntn = p.N / TN;
  const int j0 = split * ntn / p.nsplit, j1 = (split + 1) * ntn / p.nsplit;
  if (j0 >= j1) return;
  const int K = p.K;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lq = lane >> 4;
  const int a_rows = p.tokens * p.topk;
  constexpr bool kScaled = !kind_is_16bit(KIND);

  // ---- the run's A rows, all NK steps, into LDS once (route row t*topk + s; padding rows read
  // zeros past the buffer) ----
  {
    const sgpr4 rsrc_a = buf_desc(p.a, (uint32_t)a_rows * (uint32_t)K);
#pragma unroll
    for (int j = 0; j < AQ; ++j) {
      const int rloc = (wave + j * NW) * 8 + (lane >> 3);
      const int id = p.sorted_ids[b0 * TM + min(rloc, rows_valid - 1)];
      const int t = id & 0xFFFFFF, s = (int)((uint32_t)id >> 24);
      const bool ok = rloc < rows_valid && t < p.tokens && s < p.topk;
      const int c = (lane & 7) ^ ((rloc >> 1) & 7);
      const uint32_t va = ok ? (uint32_t)(t * p.topk + s) * (uint32_t)K + (uint32_t)(c * 16) : 0x80000000u;
#pragma unroll
      for (int kt = 0; kt < NK; ++kt)
        dma16(rsrc_a, sa_lds + kt * A_STEP + (wave + j * NW) * 1024, va, (uint32_t)kt * KT);
    }
  }
  // row factor (activation scale times routing weight) of this lane's rows mi*16 + l16, and the
  // destinations of this thread's store chunks (the same rows for every tile)
  float fr_r[MR];
#pragma unroll
  for (int mi = 0; mi < MR; ++mi) {
    const int r = mi * 16 + l16;
    const int id = p.sorted_ids[b0 * TM + min(r, rows_valid - 1)];
    const int t = id & 0xFFFFFF, s = (int)((uint32_t)id >> 24);
    const bool ok = r < rows_valid && t < p.tokens && s < p.topk;
    const float sxv = kScaled ? p.sa[ok ? t * p.topk + s : 0] : 1.f;
    const float rwv = p.doweight ? p.sorted_w[b0 * TM + min(r, rows_valid - 1)] : 1.f;
    fr_r[mi] = ok ? sxv * rwv : 0.f;
  }
  int dst_c[HALVES][SCH];
#pragma unroll
  for (int h = 0; h < HALVES; ++h)
#pragma unroll
    for (int i = 0; i < SCH; ++i) {
      const int r = h * HR + (tid + i * NW * 64) / CPR;
      const int id = p.sorted_ids[b0 * TM + min(r, rows_valid - 1)];
      const int t = id & 0xFFFFFF, s = (int)((uint32_t)id >> 24);
      const bool ok = r < rows_valid && t < p.tokens && s < p.topk;
      dst_c[h][i] = ok ? t * p.topk + s : -1;
    }
  const uint32_t wrb = I4 ? (uint32_t)K / 2u : (uint32_t)K;   // weight bytes per row (int4: packed)
  const __amdgpu_buffer_rsrc_t rsrc_w = make_rsrc(p.w + (size_t)e * (size_t)p.N * wrb, (int)((uint32_t)p.N * wrb));
  const __amdgpu_buffer_rsrc_t rsrc_s = make_rsrc(p.sw + (size_t)e * p.N, kScaled ? p.N * 4 : 0);
  const __amdgpu_buffer_rsrc_t rsrc_o = make_rsrc(p.out, (int)p.out_bytes);
  const bool obf16 = moe_out_bf16(p.out_mode);

  typedef typename std::conditional<kind_float_acc(KIND), f32x4, i32x4>::type AccT;
  typedef typename std::conditional<I4, i32x2, i32x4>::type BT;
  BT bw[2][NK][2];      // weight fragments of two column tiles: [set][K step][K half]
  f32x4 sc[2];          // this lane's 4 column scales of each
  // column scales and weights of column tile j into set U; every tile issues the same loads (a
  // tile past the range reads zeros from past the buffers), so the compiler's counts hold
  auto load_tile = [&](auto u_tag, int j) __attribute__((always_inline)) {
    constexpr int U = decltype(u_tag)::value;
    const bool live = j < j1;
    const uint32_t past = live ? 0u : 0x80000000u;
    const int jj = live ? j : 0;
    const uint32_t col = (uint32_t)(jj * TN + wave * 16 + lq * 4);
    sc[U] = kScaled ? __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc_s, col * 4u + past, 0, 0))
                    : f32x4{1.f, 1.f, 1.f, 1.f};
    // 16-row weight block per K step: 2048 bytes (int4: 1024 packed, lane (l16, lq) holding 8
    // bytes at 128*lq + 8*l16 and 512 past that, as the stage-1 stream kernel reads them)
    const uint32_t so0 = (uint32_t)(jj * (TN / 16) + wave) * 16u * wrb;
    const uint32_t vo = (I4 ? (uint32_t)(lq * 128 + l16 * 8) : (uint32_t)lane * 16u) + past;
#pragma unroll
    for (int kt = 0; kt < NK; ++kt) {
      if constexpr (I4) {
        const uint32_t so = so0 + (uint32_t)kt * 1024u;
        bw[U][kt][0] = __builtin_amdgcn_raw_buffer_load_b64(rsrc_w, vo, __builtin_amdgcn_readfirstlane(so), 0);
        bw[U][kt][1] = __builtin_amdgcn_raw_buffer_load_b64(rsrc_w, vo, __builtin_amdgcn_readfirstlane(so + 512u), 0);
      } else {
        const uint32_t so = so0 + (uint32_t)kt * 2048u;
        bw[U][kt][0] = __builtin_amdgcn_raw_buffer_load_b128(rsrc_w, vo, __builtin_amdgcn_readfirstlane(so), 0);
        bw[U][kt][1] = __builtin_amdgcn_raw_buffer_load_b128(rsrc_w, vo, __builtin_amdgcn_readfirstlane(so + 1024u), 0);
      }
    }
  };
  auto tile = [&](auto u_tag, int j) __attribute__((always_inline)) {
    constexpr int U = decltype(u_tag)::value;
    load_tile(std::integral_constant<int, U ^ 1>{}, j + 1);   // before this tile's stores
    AccT acc[MR];
#pragma unroll
    for (int mi = 0; mi < MR; ++mi) acc[mi] = AccT{0, 0, 0, 0};
#pragma unroll
    for (int kt = 0; kt < NK; ++kt) {
      const uint8_t* sA = sa_lds + kt * A_STEP;
      i32x4 bl, bh;
      if constexpr (I4) {
        bl = unpack_int4x16(bw[U][kt][0]);
        bh = unpack_int4x16(bw[U][kt][1]);
      } else {
        bl = bw[U][kt][0];
        bh = bw[U][kt][1];
      }
#pragma unroll
      for (int mi = 0; mi < MR; ++mi) {
        const int row = mi * 16 + l16;
        const int sw = (row >> 1) & 7;
        const i32x4 lo = *(const i32x4*)(sA + row * KT + ((lq ^ sw) << 4));
        const i32x4 hi = *(const i32x4*)(sA + row * KT + (((lq + 4) ^ sw) << 4));
        if constexpr (KIND == KIND_FP8) {
          acc[mi] = mfma_fp8(__builtin_shufflevector(bl, bh, 0, 1, 2, 3, 4, 5, 6, 7),
                             __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7), acc[mi]);
        } else {
          constexpr int MK = I4 ? KIND_INT8 : KIND;   // int4 weights: the int8 MFMA
          acc[mi] = mfma_k64<MK>(bl, lo, acc[mi]);
          acc[mi] = mfma_k64<MK>(bh, hi, acc[mi]);
        }
      }
    }
    // epilogue: value = accumulator * column scale * row factor (the order of moe.h's rows)
    const uint32_t n0b = (uint32_t)(j * TN) * 2u;
#pragma unroll
    for (int h = 0; h < HALVES; ++h) {
      workgroup_barrier();   // the staging rows have been read out
#pragma unroll
      for (int mh = 0; mh < MR / HALVES; ++mh) {
        const int mi = h * (MR / HALVES) + mh;
        const int r = mh * 16 + l16;
        const int c = wave * 16 + lq * 4;
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = ((float)int4_acc<KIND>(acc[mi])[q] * sc[U][q]) * fr_r[mi];
        const i32x2 pk = obf16 ? pack_out4<true>(v) : pack_out4<false>(v);
        *(i32x2*)(stg + r * RB + (((c >> 3) ^ (r % CPR)) << 4) + (c & 7) * 2) = pk;
      }
      workgroup_barrier();
#pragma unroll
      for (int i = 0; i < SCH; ++i) {
        const int cc = tid + i * NW * 64;
        const int r = cc / CPR, ch = cc % CPR;
        const i32x4 val = *(const i32x4*)(stg + r * RB + ((ch ^ (r % CPR)) << 4));
        const int d = dst_c[h][i];
        // padding rows: an offset past the buffer (out_bytes <= 0xFFFFFF00) that a 16-byte
        // store cannot wrap
        const uint32_t off = d < 0 ? 0xFFFFFFE0u : (uint32_t)d * (uint32_t)p.N * 2u + n0b + (uint32_t)ch * 16u;
        __builtin_amdgcn_raw_buffer_store_b128(val, rsrc_o, off, 0, 0);
      }
    }
  };
  load_tile(std::integral_constant<int, 0>{}, j0);
  waitcnt<0>();
  workgroup_barrier();   // the A rows are in LDS for every wave
  int j = j0;
  for (; j + 2 <= j1; j += 2) {
    tile(std::integral_constant<int, 0>{}, j);
    tile(std::integral_constant<int, 1>{}, j + 1);
  }
  if (j < j1) tile(std::integral_constant<int, 0>{}, j);
}

}  // namespace flygemm
