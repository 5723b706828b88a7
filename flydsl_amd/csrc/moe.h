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
// Input kinds (reference in_dtype): fp8, int8, bf16, fp16; int8 with slot-major activations
// ("int8smooth": stage-1 x is [topk*tokens][K] with row s*tokens + t and one scale per such row,
// moe_gemm_2stage.py:466-476); int4 weights with int8 activations (W4A8, KIND_INT4: the packed
// preshuffled bytes of the dense int4 path, unpacked to int8 in registers); int4 weights with
// bf16 activations (W4A16, KIND_W4A16: the nibbles converted to bf16 in registers, times a
// per-(32-deep K group, weight row) scale when group scales are given, else the per-row scale
// in the epilogue, as for int8; mfma_preshuffle_pipeline.py:148-222).
//
// W1 and W2 are preshuffled like every B operand here.  A rows are gathered by the LDS-DMA:
// each lane's buffer offset names its own row, and padding rows get an offset past the buffer,
// which reads zeros.  The kernel below (moe_gemm_kernel) keeps A and B in a two-slot LDS ring,
// one barrier per 128-byte K tile, LDS layouts as in the large-M kernel (gemm_main.h): A rows
// with the XOR chunk swizzle, B copied verbatim.  It runs stage 2 (atomics; per-route rows of
// decode-sized routings and of W4A16 / int4 / deeper inter_dim) and stage 1 of W4A16 and of
// blockscale; moe_stream.h holds the kernels that stream the weights into registers (stage 1
// of the other kinds, stage 2 per-route rows of prefill routings).
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
  int nsplit;                  // column ranges per run (workgroups per run)
  int out_mode;                // MoeOut
  uint32_t out_bytes;          // size of out (buffer bounds of the epilogue stores)
  int a_token_slot;            // stage 1: x rows (and sa) per route, slot-major s*tokens + t
  int wgroup;                  // W4A16: 32 = sw holds group scales [E][K/32][rows of W], 0 = per row
};

// Formats of the MoE input kinds.
constexpr bool moe_w_int4(int k) { return k == KIND_INT4 || k == KIND_W4A16; }
constexpr bool moe_a_16bit(int k) { return kind_is_16bit(k) || k == KIND_W4A16; }
// bytes of one 16-column weight block per 128-byte K tile of the activations
constexpr int moe_b_blk(int k) { return k == KIND_W4A16 ? 512 : (k == KIND_INT4 ? 1024 : 2048); }

// Eight packed int4 weights of one 32-bit word (byte j holds element j in its low nibble and
// element j + 4 in its high nibble, the dense int4 packing) -> eight bf16 in element order,
// each times `s` when `scaled`.  The fp32 product becomes bf16 by truncation (its upper 16
// bits), as the reference's conversion does (kernels/mfma_preshuffle_pipeline.py:111-141:
// `bits >> 16` and `bits & 0xFFFF0000`); unscaled nibbles are exact either way.
__device__ __forceinline__ i32x4 int4x8_to_bf16(uint32_t p, float s, bool scaled) {
  uint32_t f[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int off = k < 4 ? 8 * k : 8 * (k - 4) + 4;
    const int v = ((int)(p << (28 - off))) >> 28;   // sign-extended nibble
    f[k] = __builtin_bit_cast(uint32_t, scaled ? (float)v * s : (float)v);
  }
  return i32x4{(int)((f[0] >> 16) | (f[1] & 0xFFFF0000u)), (int)((f[2] >> 16) | (f[3] & 0xFFFF0000u)),
               (int)((f[4] >> 16) | (f[5] & 0xFFFF0000u)), (int)((f[6] >> 16) | (f[7] & 0xFFFF0000u))};
}

// Stage-2 outputs: F16/BF16/F32 accumulate into out[token] with atomics; *_ROWS store each
// route's row out[token*topk + slot] with plain stores (the reduce mode, summed by
// moe_reduce_kernel afterwards).  Stage 1 takes F16 or BF16.
typedef void (*MoeFn)(MoeArgs);
// A kernel of the tables and the workgroup size it was instantiated for (its waves x 64).
struct MoeKernel {
  MoeFn fn;
  int threads;
};

enum MoeOut : int { MOE_OUT_F16 = 0, MOE_OUT_BF16 = 1, MOE_OUT_F32 = 2, MOE_OUT_F16_ROWS = 3, MOE_OUT_BF16_ROWS = 4 };
constexpr bool moe_out_bf16(int o) { return o == MOE_OUT_BF16 || o == MOE_OUT_BF16_ROWS; }

// x * sigmoid(x) = x / (1 + 2^(-x log2 e)) with the hardware exp2 and reciprocal
// (reference moe_gemm_2stage.py:271-281 evaluates it the same way)
__device__ __forceinline__ float silu_f(float x) {
  const float e = __builtin_amdgcn_exp2f(x * -1.4426950408889634f);
  return x * __builtin_amdgcn_rcpf(1.f + e);
}

// Runs of up to R sorted blocks of one expert, counted from the expert's first block (the
// sorting writes an expert's blocks contiguously): the block count of the run starting at
// block b0 (expert e, nbv blocks in use), or 0 when b0 lies inside a run.  Counting from the
// expert's first block rather than from multiples of R gives ceil(blocks / R) runs per expert;
// runs aligned to multiples of R split an expert whose blocks start at an odd position into one
// more run, which streams the expert's weights once more (DS-TP8 prefill, 64-row blocks, R = 2:
// 608 runs against 577).  Every lane reads one expert id behind b0 (and one ahead); the ballots
// make the result uniform over the wave and, all waves reading the same ids, the workgroup.
// Kinds with run tiles of four 64-row blocks for routings with large experts (moe_tiles)
constexpr bool moe_big_kind(int kind) {
  return kind == KIND_FP8 || kind == KIND_INT8 || kind == KIND_BF16 || kind == KIND_F16 || kind == KIND_INT4;
}

template <int R>
__device__ __forceinline__ int moe_run_blocks(const int32_t* expert_ids, int b0, int e, int nbv, int lane) {
  if constexpr (R == 1) {
    return 1;
  } else {
    static_assert(R < 64, "one ballot covers a run");
    int before = 0;                           // blocks of expert e directly before b0
    for (int base = b0;; base -= 64) {
      const int b = base - 1 - lane;
      const bool other = b < 0 || expert_ids[b] != e;
      const uint64_t m = __builtin_amdgcn_ballot_w64(other);
      if (m != 0) {
        before += __builtin_ctzll(m);
        break;
      }
      before += 64;
    }
    if (before % R != 0) return 0;
    const int lim = min(R, nbv - b0);         // blocks b0 .. b0 + lim - 1 may join the run
    const bool other = lane >= lim || expert_ids[b0 + lane] != e;
    return __builtin_ctzll(__builtin_amdgcn_ballot_w64(other) | (1ull << 63));
  }
}

// F32: fp32 output (stage 2 with atomics only); otherwise 2-byte outputs, whose type (fp16 or
// bf16) and mode (rows or atomics) are run-time facts of MoeArgs::out_mode.
template <int STAGE, int KIND, int TM, int R, int TN, int WM, int WN, bool F32, bool SCW = false>
struct MoeCfg {
  static constexpr int NS = 2;                        // LDS ring slots: the DMA runs one step ahead
  static constexpr int NW = WM * WN;                  // waves: WM across the rows, WN across the columns
  static constexpr int TME = TM * R;                  // rows of one run: up to R routing blocks
  static constexpr int TMW = TME / WM;                // rows per wave
  static constexpr int MR = TMW / 16;                 // 16-row blocks per wave
  static constexpr int NR = TN / (16 * WN);           // 16-column blocks per wave and weight half
  static constexpr int NB = STAGE == 1 ? 2 : 1;       // weight halves: gate and up in stage 1
  static constexpr int A_BYTES = TME * KT;            // A part of one LDS slot
  static constexpr int B_BYTES = NB * (TN / 16) * moe_b_blk(KIND);  // B part: NB x TN columns, one K tile
  static constexpr int A_DMA = A_BYTES / 1024;        // 1 KB DMA instructions per K tile
  static constexpr int AQ = (A_DMA + NW - 1) / NW;    // per wave
  static constexpr int B_DMA = B_BYTES / 1024;        // 1 KB DMA instructions per K tile
  static constexpr int BQ = (B_DMA + NW - 1) / NW;    // per wave (some waves one fewer)
  static constexpr int ESZ = F32 ? 4 : 2;
  // epilogue tile row: TN values, then 16 bytes holding the row's destination (the padding also
  // spreads the rows over the LDS banks)
  static constexpr int RS = TN * ESZ + 16;
  // one ring slot: a K step's A and B tiles, and at least 16 rows of the atomic epilogue's
  // staging, which reuses the slot (int4 weights leave the data part small); then, with
  // per-column weight scales (SCW), the column tile's NB x TN fp32 scales, which the tile's
  // last K step brings with its DMA (whole 1 KB instructions) so the epilogue reads them from
  // LDS: a global load of them would be waited for behind the next step's DMA, issued after it
  static constexpr int SLOT_DATA = A_BYTES + B_BYTES > 16 * RS ? A_BYTES + B_BYTES : 16 * RS;
  static constexpr int SC_DMA = SCW ? (NB * TN * 4 + 1023) / 1024 : 0;
  static constexpr int SLOT = SLOT_DATA + SC_DMA * 1024;
  static constexpr int CH = (SLOT_DATA / RS) / 16 * 16 < TME ? (SLOT_DATA / RS) / 16 * 16 : TME;  // rows per chunk
  static constexpr int NCH = (TME + CH - 1) / CH;
  static constexpr int NST = MR * NR;                 // direct row stores per thread per column tile
  static_assert(TM % 16 == 0 && NR >= 1 && TN % (16 * WN) == 0 && TMW % 16 == 0 && A_BYTES % 1024 == 0,
                "tile shape");
  static_assert(B_BYTES % 1024 == 0, "B DMA in whole instructions");
  static_assert(CH >= 16 && NS * SLOT <= 160 * 1024, "LDS budget");
};

// One workgroup (WM x WN waves) per (run, column range): a run is up to R consecutive routing blocks of
// one expert (a block starts a run when its index is a multiple of R or its expert differs from
// the previous block's), so the weight tile of each K step serves up to R*TM rows; the
// workgroup then walks its column tiles and K tiles as one pipeline.
//   Each K step: A (the gathered rows) and B (the expert's preshuffled weight rows of the column
//   tile, gate and up in stage 1) go global -> LDS by DMA into a 2-slot ring, one step ahead.
//   Wave (wm, wn) owns rows [wm*TME/WM, (wm+1)*TME/WM) and columns [wn*TN/WN, (wn+1)*TN/WN) of
//   the tile (of the gate and of the up half in stage 1, so silu(gate) * up pairs in registers).
//   Epilogue at the end of each column tile: row outputs (stage 1, reduce mode) are stored
//   straight from the accumulators; atomic accumulation goes through the slot the last step
//   computed from, in chunks of CH rows, so each wave instruction adds 256 contiguous bytes.
// BS: blockscale (fp8): sa = x scales [K/128][rows of A] (K-block major), sw = weight scales
// [E*wrows/128][K/128] (one per 128x128 block); each K step's MFMA partial is scaled by
// sa[kb][row] * sw[row block of the column][kb] and added to the accumulator (reference
// kernels/moe_blockscale_2stage.py:677-777 for stage 1, :1836-1880 for stage 2).
template <int STAGE, int KIND, int TM, int R, int TN, int WM, int WN, bool F32, bool BS = false>
__global__ void __launch_bounds__(WM * WN * 64) moe_gemm_kernel(MoeArgs p) {
  using C = MoeCfg<STAGE, KIND, TM, R, TN, WM, WN, F32, !kind_is_16bit(KIND) && !BS>;
  constexpr int NW = C::NW, TMW = C::TMW;
  static_assert(!BS || KIND == KIND_FP8, "blockscale is fp8");
  static_assert(STAGE == 2 || !F32, "stage 1 writes 2-byte outputs");
  static_assert(KIND == KIND_FP8 || KIND == KIND_INT8 || kind_is_16bit(KIND) || moe_w_int4(KIND), "MoE input kinds");
  constexpr int MR = C::MR, NR = C::NR, NB = C::NB, TME = C::TME, NT = NW * 64;
  const int mode = p.out_mode;
  const bool rows = STAGE == 1 || mode == MOE_OUT_F16_ROWS || mode == MOE_OUT_BF16_ROWS;
  const bool obf16 = moe_out_bf16(mode);
  __shared__ __attribute__((aligned(1024))) uint8_t ring[C::NS * C::SLOT];
  // Row outputs of tiles of 128+ columns go through the slot the tile's last K step computed
  // from, in two rounds of half of every wave's rows, and leave as 16-byte chunks so each wave
  // instruction writes whole 128-byte lines (the accumulator layout's direct stores cover 16
  // rows x 32 bytes per instruction, which the memory system takes at about 2/3 of the rate of
  // whole lines; these are random rows of the reduce mode's intermediate).  Staged row sr of
  // round h is tile row (sr / HR) * TMW + h * HR + sr % HR; its 16-byte chunk c sits at chunk
  // c ^ (sr % CPR).  NSTR: row stores per lane per tile.
  constexpr int RB = TN * 2, CPR = RB / 16, HR = TMW / 2, HMR = MR / 2;
  // (stage 2 only: stage 1 writes a 2*I-times smaller output, and 128-row stage-1 tiles were
  // 1.7% slower staged; DS-TP8 prefill stage 2 in reduce mode 0.71 ms against 0.77)
  constexpr bool kStageRows = STAGE == 2 && !F32 && MR % 2 == 0 && TN >= 128 && TME / 2 * RB <= C::SLOT_DATA &&
                              (TME / 2 * CPR) % NT == 0;
  constexpr int SCHR = kStageRows ? TME / 2 * CPR / NT : 0;
  constexpr int NSTR = kStageRows ? 2 * SCHR : C::NST;
  __shared__ int sdst[kStageRows ? TME / 2 : 1];   // destinations of the staged rows
  // Stage-2 row outputs with at most two K tiles (`ares`): steps alternate the two slots and
  // every column tile has the same K tiles, so K tile kt's A rows stay in the A part of slot kt
  // (of both slots for a single K tile) after the first column tile (two for a single K tile),
  // and later steps DMA only B.  The row staging then uses the last slot's B part.
  constexpr bool kAres = STAGE == 2 && !F32 && !BS && (!kStageRows || TME / 2 * RB <= C::B_BYTES);

  // ---- which run and which column tiles ----
  // Logical id L = block * nsplit + split over the blocks below num_valid_ids, dealt to the 8
  // XCDs in contiguous ranges (workgroup (L % chunk) * 8 + L / chunk; XCDs take workgroups
  // round-robin), so consecutive runs of one expert share an XCD's L2 copy of its weights.
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
  const int nk = K / KT;
  const bool ares = kAres && rows && nk <= 2;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int rw0 = wm * TMW;    // this wave's first row
  const int l16 = lane & 15, lq = lane >> 4;
  const bool a_ts = STAGE == 1 && p.a_token_slot;
  const int a_rows = STAGE == 1 && !a_ts ? p.tokens : p.tokens * p.topk;
  // per-token activation scales and per-row weight scales in the epilogue: not for 16-bit
  // activations (W4A16 keeps the weight scale unless it has group scales) nor blockscale
  constexpr bool kScaledA = !moe_a_16bit(KIND) && !BS;
  const bool scaled_w = (!kind_is_16bit(KIND) && !BS) && !(KIND == KIND_W4A16 && p.wgroup);

  // ---- per-row facts, fixed for the workgroup's life ----
  // Every load below is unconditional (indices clamped into range, the result masked after), so
  // they all go out before the first wait.
  // A gather: DMA instruction q fills tile rows 8q .. 8q+7; lane l brings the chunk that
  // belongs in slot l%8 of row 8q + l/8.  Padding rows read zeros (offset past the buffer).
  uint32_t va[C::AQ];
  int ida[C::AQ], idr[MR];
#pragma unroll
  for (int j = 0; j < C::AQ; ++j)
    ida[j] = p.sorted_ids[b0 * TM + min(min((wave + j * NW) * 8 + (lane >> 3), TME - 1), rows_valid - 1)];
#pragma unroll
  for (int mi = 0; mi < MR; ++mi) idr[mi] = p.sorted_ids[b0 * TM + min(rw0 + mi * 16 + l16, rows_valid - 1)];
#pragma unroll
  for (int j = 0; j < C::AQ; ++j) {
    const int rloc = min((wave + j * NW) * 8 + (lane >> 3), TME - 1);
    const int id = ida[j];
    const int t = id & 0xFFFFFF, s = (int)((uint32_t)id >> 24);
    const bool ok = rloc < rows_valid && t < p.tokens && s < p.topk;
    const int row = STAGE == 1 ? (a_ts ? s * p.tokens + t : t) : t * p.topk + s;
    const int c = (lane & 7) ^ ((rloc >> 1) & 7);
    va[j] = ok ? (uint32_t)row * (uint32_t)K + (uint32_t)(c * 16) : 0x80000000u;
  }
  // this lane's rows mi*16 + l16: scale, routing weight, destination row (-1: padding)
  float sx_r[MR], rw_r[MR], fr_r[MR];
  int dst_r[MR], arow_r[MR];
#pragma unroll
  for (int mi = 0; mi < MR; ++mi) {
    const int r = rw0 + mi * 16 + l16;
    const int id = idr[mi];
    const int t = id & 0xFFFFFF, s = (int)((uint32_t)id >> 24);
    const bool ok = r < rows_valid && t < p.tokens && s < p.topk;
    dst_r[mi] = !ok ? -1 : (rows ? t * p.topk + s : t);
    const int arow = ok ? (STAGE == 1 ? (a_ts ? s * p.tokens + t : t) : t * p.topk + s) : 0;
    arow_r[mi] = arow;
    const float sxv = kScaledA ? p.sa[arow] : 1.f;
    const float rwv = p.doweight ? p.sorted_w[b0 * TM + min(r, rows_valid - 1)] : 1.f;
    sx_r[mi] = ok ? sxv : 0.f;  // 0 keeps padding rows finite; 1 for unscaled kinds
    rw_r[mi] = ok ? rwv : 0.f;
    fr_r[mi] = sx_r[mi] * rw_r[mi];   // stage 2's row factor (rw_r is 1 without doweight)
  }

  const sgpr4 rsrc_a = buf_desc(p.a, (uint32_t)a_rows * (uint32_t)K);
  // this expert's weight rows only (the whole array may exceed 32-bit offsets)
  const int wrows = STAGE == 1 ? 2 * p.N : p.N;
  // bytes per weight row: K for 1-byte weights of 1-byte activations and 2-byte of 2-byte ones,
  // K/2 for int4 weights of int8 activations, K/4 for int4 weights of bf16 activations
  const uint32_t wrb = KIND == KIND_W4A16 ? (uint32_t)K / 4u : (KIND == KIND_INT4 ? (uint32_t)K / 2u : (uint32_t)K);
  const sgpr4 rsrc_w = buf_desc(p.w + (size_t)e * (size_t)wrows * wrb, (uint32_t)wrows * wrb);
  // this expert's per-column weight scales (gate then up in stage 1)
  const sgpr4 rsrc_s = buf_desc(p.sw + (size_t)e * wrows, (uint32_t)wrows * 4u);
  const uint32_t vb = (uint32_t)lane * 16u;
  // W4A16: one DMA instruction brings two adjacent 16-column blocks, 512 bytes each
  const uint32_t vb_w4 = (uint32_t)(lane & 31) * 16u + (uint32_t)(lane >> 5) * 16u * wrb;

  // DMA of step (column tile jt, K tile kt) into ring slot `slot`: A rows, then the B blocks
  // (local 16-column block lb: gate -- or W2 -- for lb < TN/16, up after), each 2 KB per K tile
  // in the preshuffled layout, copied verbatim.
  auto issue = [&](int jt, int kt, int slot) {
    uint8_t* st = ring + slot * C::SLOT;
    // the guards below are compile-time true when the DMA count divides among the waves (no
    // branches in the step then)
    if (!(ares && jt - j0 >= (nk == 1 ? 2 : 1))) {   // A already resident in this slot
#pragma unroll
      for (int j = 0; j < C::AQ; ++j) {
        const int q = wave + j * NW;
        if (C::A_DMA % NW == 0 || q < C::A_DMA) dma16(rsrc_a, st + q * 1024, va[j], (uint32_t)kt * KT);
      }
    }
    const int n0 = jt * TN;
#pragma unroll
    for (int j = 0; j < C::BQ; ++j) {
      const int q = wave + j * NW;
      if (C::B_DMA % NW != 0 && q >= C::B_DMA) continue;           // wave-uniform
      // local 16-column block lb (gate -- or W2 -- for lb < TN/16, up after) -> global block
      auto gblk = [&](int lb) { return lb < TN / 16 ? n0 / 16 + lb : (p.N + n0) / 16 + (lb - TN / 16); };
      uint32_t so, vo = vb;
      if constexpr (KIND == KIND_W4A16) {     // piece q: blocks 2q and 2q+1 (TN/16 is even)
        so = (uint32_t)gblk(2 * q) * 16u * wrb + (uint32_t)kt * 512u;
        vo = vb_w4;
      } else if constexpr (KIND == KIND_INT4) {  // piece q: block q
        so = (uint32_t)gblk(q) * 16u * wrb + (uint32_t)kt * 1024u;
      } else {                                // piece q: block q/2, half q%2
        so = (uint32_t)gblk(q >> 1) * 16u * wrb + (uint32_t)kt * 2048u + (uint32_t)(q & 1) * 1024u;
      }
      dma16(rsrc_w, st + C::A_BYTES + q * 1024, vo, __builtin_amdgcn_readfirstlane(so));
    }
    // the column tile's weight scales with its last K step, by the last waves (instruction i:
    // scale elements 256i .. 256i+255 of [NB][TN]; lanes past the end bring zeros)
    if constexpr (C::SC_DMA > 0) {
      if (scaled_w && kt == nk - 1) {
#pragma unroll
        for (int i = 0; i < C::SC_DMA; ++i) {
          if (wave != NW - 1 - i) continue;   // wave-uniform
          const int idx = i * 256 + lane * 4;
          const int h = idx / TN, col = idx - h * TN;
          const uint32_t vs = idx < NB * TN ? (uint32_t)(h * p.N + jt * TN + col) * 4u : 0x80000000u;
          dma16(rsrc_s, st + C::SLOT_DATA + i * 1024, vs, 0);
        }
      }
    }
  };

  typedef typename std::conditional<kind_float_acc(KIND), f32x4, i32x4>::type AccT;
  AccT acc[NB][MR][NR];

  // blockscale factors of the current step (bsa_c: this lane's rows, bsw_c: its 16-column
  // blocks) and of the next (bsa_n / bsw_n, loaded before the next step's DMA is issued and
  // copied at that step's top, after its wait -- a copy earlier would wait for the DMA)
  float bsa_c[BS ? MR : 1], bsa_n[BS ? MR : 1], bsw_c[NB][BS ? NR : 1], bsw_n[NB][BS ? NR : 1];
  auto load_bs = [&](int jt, int kt) {
    if constexpr (BS) {
#pragma unroll
      for (int mi = 0; mi < MR; ++mi) bsa_n[mi] = p.sa[kt * a_rows + arow_r[mi]];
#pragma unroll
      for (int h = 0; h < NB; ++h)
#pragma unroll
        for (int ni = 0; ni < NR; ++ni) {
          const int wr = e * wrows + (h ? p.N : 0) + jt * TN + (wn * NR + ni) * 16;
          bsw_n[h][ni] = p.sw[(wr / 128) * nk + kt];
        }
    }
  };

  // W4A16 group scales of the current step and of the next (as the blockscale factors): for
  // each of this lane's weight columns, the scales of the two 32-deep K groups of the step
  float gs_c[NB][NR][2], gs_n[NB][NR][2];
  const int kgroups = K / 64;   // 32-element groups per weight row (K counts bf16 bytes)
  auto load_gs = [&](int jt, int kt) {
    if constexpr (KIND == KIND_W4A16) {
      if (!p.wgroup) return;
#pragma unroll
      for (int h = 0; h < NB; ++h)
#pragma unroll
        for (int ni = 0; ni < NR; ++ni) {
          const int n = (h ? p.N : 0) + jt * TN + (wn * NR + ni) * 16 + l16;
#pragma unroll
          for (int g = 0; g < 2; ++g) gs_n[h][ni][g] = p.sw[((size_t)e * kgroups + 2 * kt + g) * wrows + n];
        }
    }
  };

  // One K tile: this wave's B fragments read once, then row block by row block, the next row's
  // A fragment read ahead of this row's MFMAs.  B is the MFMA's first operand, so each
  // accumulator tile holds its 16x16 output block transposed.
  auto compute = [&](const uint8_t* sA) {
    const uint8_t* sB = sA + C::A_BYTES;
    auto load_a = [&](int mi, i32x4& lo, i32x4& hi) {
      const int row = rw0 + mi * 16 + l16;
      const int sw = (row >> 1) & 7;
      lo = *(const i32x4*)(sA + row * KT + ((lq ^ sw) << 4));
      hi = *(const i32x4*)(sA + row * KT + (((lq + 4) ^ sw) << 4));
    };
    i32x4 bl[NB][NR], bh[NB][NR];
#pragma unroll
    for (int h = 0; h < NB; ++h)
#pragma unroll
      for (int ni = 0; ni < NR; ++ni) {
        const int blk = h * (TN / 16) + wn * NR + ni;
        if constexpr (KIND == KIND_W4A16) {
          // MFMA half j takes elements 32j + 8lq .. +7 of the 64-element step: 4 bytes of
          // 16-element chunk 2j + lq/2 of this column
          const int off = blk * 512 + (lq >> 1) * 128 + l16 * 8 + (lq & 1) * 4;
          const bool gsc = p.wgroup != 0;
          bl[h][ni] = int4x8_to_bf16(*(const uint32_t*)(sB + off), gsc ? gs_c[h][ni][0] : 1.f, gsc);
          bh[h][ni] = int4x8_to_bf16(*(const uint32_t*)(sB + off + 256), gsc ? gs_c[h][ni][1] : 1.f, gsc);
        } else if constexpr (KIND == KIND_INT4) {
          const int off = blk * 1024 + lq * 128 + l16 * 8;
          bl[h][ni] = unpack_int4x16(*(const i32x2*)(sB + off));
          bh[h][ni] = unpack_int4x16(*(const i32x2*)(sB + off + 512));
        } else {
          const int off = blk * 2048 + lq * 256 + l16 * 16;
          bl[h][ni] = *(const i32x4*)(sB + off);
          bh[h][ni] = *(const i32x4*)(sB + off + 1024);
        }
      }
    i32x4 alo, ahi;
    load_a(0, alo, ahi);
#pragma unroll
    for (int mi = 0; mi < MR; ++mi) {
      const i32x4 lo = alo, hi = ahi;
      if (mi + 1 < MR) load_a(mi + 1, alo, ahi);
#pragma unroll
      for (int h = 0; h < NB; ++h)
#pragma unroll
        for (int ni = 0; ni < NR; ++ni) {
          if constexpr (BS) {
            const f32x4 part = mfma_fp8(__builtin_shufflevector(bl[h][ni], bh[h][ni], 0, 1, 2, 3, 4, 5, 6, 7),
                                        __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7),
                                        f32x4{0.f, 0.f, 0.f, 0.f});
            const float sc_k = bsa_c[mi] * bsw_c[h][ni];
            acc[h][mi][ni].x = __builtin_fmaf(part.x, sc_k, acc[h][mi][ni].x);
            acc[h][mi][ni].y = __builtin_fmaf(part.y, sc_k, acc[h][mi][ni].y);
            acc[h][mi][ni].z = __builtin_fmaf(part.z, sc_k, acc[h][mi][ni].z);
            acc[h][mi][ni].w = __builtin_fmaf(part.w, sc_k, acc[h][mi][ni].w);
          } else if constexpr (KIND == KIND_FP8) {
            acc[h][mi][ni] = mfma_fp8(__builtin_shufflevector(bl[h][ni], bh[h][ni], 0, 1, 2, 3, 4, 5, 6, 7),
                                      __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7), acc[h][mi][ni]);
          } else {
            constexpr int MK = KIND == KIND_W4A16 ? KIND_BF16 : KIND;   // int4 weights: int8 or bf16 MFMA
            acc[h][mi][ni] = mfma_k64<MK>(bl[h][ni], lo, acc[h][mi][ni]);
            acc[h][mi][ni] = mfma_k64<MK>(bh[h][ni], hi, acc[h][mi][ni]);
          }
        }
    }
  };


  // Epilogue of column tile jt.  Lane (l16, lq) holds row mi*16 + l16, columns 4*lq .. 4*lq+3
  // of each of its 16-column blocks.  Atomic outputs: through the LDS slot `ot` (free once every
  // wave is past the barrier below), CH rows at a time -- phase 1 writes the scaled values,
  // phase 2 adds them row-contiguously, each wave instruction covering 256 contiguous bytes
  // (scattered 4-lane fragments would touch 16 cache lines per instruction, which costs the
  // atomics 8x their useful rate).
  const __amdgpu_buffer_rsrc_t rsrc_o = make_rsrc(p.out, (int)p.out_bytes);
  // `last`: the slot of the tile's last K step, which holds the column scales after its data;
  // it is next written by a DMA issued after the following step's barrier, so every wave
  // reads it here before any wave can overwrite it.
  auto epilogue = [&](int jt, uint8_t* ot, const uint8_t* last) {
    const int n0 = jt * TN;
    f32x4 sc[NB][NR];
#pragma unroll
    for (int h = 0; h < NB; ++h)
#pragma unroll
      for (int ni = 0; ni < NR; ++ni) {
        sc[h][ni] = f32x4{1.f, 1.f, 1.f, 1.f};
        if constexpr (C::SC_DMA > 0)
          if (scaled_w) sc[h][ni] = *(const f32x4*)(last + C::SLOT_DATA + (h * TN + (wn * NR + ni) * 16 + lq * 4) * 4);
      }
    // Output element (mi, ni, q) before rounding: stage 1 silu(gate) * up of the scaled
    // accumulators, times the routing weight (1 without doweight, an exact factor); stage 2 the
    // accumulator times the column scale and the row factor fr (activation scale times routing
    // weight: two multiplies per element).  Row outputs select the output type on the packed
    // words: instantiating their loop once per type let the compiler hoist the common products
    // above the branch and spill.
    auto value = [&](int mi, int ni, int q) -> float {
      if constexpr (STAGE == 1) {
        const float g = ((float)int4_acc<KIND>(acc[0][mi][ni][q]) * sx_r[mi]) * sc[0][ni][q];
        const float u = ((float)int4_acc<KIND>(acc[1][mi][ni][q]) * sx_r[mi]) * sc[1][ni][q];
        return (silu_f(g) * u) * rw_r[mi];
      } else {
        return ((float)int4_acc<KIND>(acc[0][mi][ni][q]) * sc[0][ni][q]) * fr_r[mi];
      }
    };
    auto pack_sel = [&](const float (&v)[4]) -> i32x2 { return obf16 ? pack_out4<true>(v) : pack_out4<false>(v); };
    if constexpr (kStageRows) {
      if (rows) {
        uint8_t* stg = const_cast<uint8_t*>(last) + (ares ? C::A_BYTES : 0);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          workgroup_barrier();   // the slot is free: computed from (h == 0) or read out (h == 1)
#pragma unroll
          for (int mh = 0; mh < HMR; ++mh) {
            const int mi = h * HMR + mh;
            const int sr = wm * HR + mh * 16 + l16;
#pragma unroll
            for (int ni = 0; ni < NR; ++ni) {
              const int c = (wn * NR + ni) * 16 + lq * 4;
              float v[4];
#pragma unroll
              for (int q = 0; q < 4; ++q) v[q] = value(mi, ni, q);
              *(i32x2*)(stg + sr * RB + (((c >> 3) ^ (sr % CPR)) << 4) + (c & 7) * 2) = pack_sel(v);
            }
            if (wn == 0 && lq == 0) sdst[sr] = dst_r[mi];
          }
          workgroup_barrier();
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll 2
          for (int i = 0; i < SCHR; ++i) {
            const int cc = tid + i * NT;
            const int sr = cc / CPR, ch = cc % CPR;
            const i32x4 val = *(const i32x4*)(stg + sr * RB + ((ch ^ (sr % CPR)) << 4));
            const int d = sdst[sr];
            // padding rows: an offset past the buffer (out_bytes <= 0xFFFFFF00) that a 16-byte
            // store cannot wrap
            const uint32_t off = d < 0 ? 0xFFFFFFE0u : ((uint32_t)d * (uint32_t)p.N + (uint32_t)n0) * 2u + (uint32_t)ch * 16u;
            __builtin_amdgcn_raw_buffer_store_b128(val, rsrc_o, off, 0, 0);
          }
        }
        return;
      }
    }
    if (!F32 && rows) {
      // Row outputs (stage 1, reduce mode): straight from the accumulators, 8 bytes per lane
      // (4 columns of one row), exactly NST buffer stores per thread (padding rows get an
      // offset past the buffer).
      {
#pragma unroll
        for (int mi = 0; mi < MR; ++mi) {
          const int d = dst_r[mi];
          const uint32_t rowoff = d < 0 ? 0xFFFFFFF0u : (uint32_t)d * (uint32_t)p.N * 2u;
#pragma unroll
          for (int ni = 0; ni < NR; ++ni) {
            const int c = (wn * NR + ni) * 16 + lq * 4;
            float v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = value(mi, ni, q);
            const uint32_t off = d < 0 ? rowoff : rowoff + (uint32_t)(n0 + c) * 2u;
            __builtin_amdgcn_raw_buffer_store_b64(pack_sel(v), rsrc_o, off, 0, 0);
          }
        }
      }
      return;
    }
    workgroup_barrier();  // every wave is done computing from the slot
#pragma unroll
    for (int ch = 0; ch < C::NCH; ++ch) {
      if (ch > 0) workgroup_barrier();  // the previous chunk's rows have been read out
      // the staging loop once per output type (here its products do not spill; measured on
      // DS-TP8 prefill stage 2 with atomics: 0.95 ms against 1.09 with the select)
      auto body = [&](auto bf_tag) {
        constexpr bool BF = decltype(bf_tag)::value;
#pragma unroll
        for (int mi = 0; mi < MR; ++mi) {
          if ((rw0 + mi * 16) / C::CH != ch) continue;   // wave-uniform: this row block is in another chunk
          __builtin_amdgcn_sched_barrier(0);
          const int r = rw0 + mi * 16 + l16 - ch * C::CH;
          if (wn == 0 && lq == 0) *(int*)(ot + r * C::RS + TN * C::ESZ) = dst_r[mi];
#pragma unroll
          for (int ni = 0; ni < NR; ++ni) {
            const int c = (wn * NR + ni) * 16 + lq * 4;
            float v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = value(mi, ni, q);
            uint8_t* dst = ot + r * C::RS + c * C::ESZ;
            if constexpr (C::ESZ == 4)
              *(f32x4*)dst = f32x4{v[0], v[1], v[2], v[3]};
            else
              *(i32x2*)dst = pack_out4<BF>(v);
          }
        }
      };
      if (obf16) body(std::true_type{}); else body(std::false_type{});
      workgroup_barrier();
      const int nrows = min(C::CH, TME - ch * C::CH);
      {
        constexpr int WPR = TN * C::ESZ / 4;    // 4-byte words per output row
        for (int idx = tid; idx < nrows * WPR; idx += NT) {
          const int r = idx / WPR, wd = idx - r * WPR;
          const int d = *(const int*)(ot + r * C::RS + TN * C::ESZ);
          if (d < 0) continue;
          uint8_t* dst = (uint8_t*)p.out + ((size_t)d * p.N + n0) * C::ESZ + wd * 4;
          const uint8_t* src = ot + r * C::RS + wd * 4;
          if constexpr (F32) {
            unsafeAtomicAdd((float*)dst, *(const float*)src);
          } else if (obf16) {
            typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
            __builtin_amdgcn_global_atomic_fadd_v2bf16((bf16x2*)dst, *(const bf16x2*)src);
          } else {
            typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
            __builtin_amdgcn_global_atomic_fadd_v2f16((f16x2*)dst, *(const f16x2*)src);
          }
        }
      }
    }
  };

  // ---- the pipeline over (column tile, K tile) steps ----
  // Each step waits for its slot's DMA (issued one step earlier), publishes the slot with the
  // barrier, issues the next step's DMA into the other slot -- the next K tile, or the first of
  // the next column tile -- and computes.  The epilogue's row stores go out after that DMA, so
  // the next step's wait leaves them in flight (vector memory operations retire in issue order).
  int slot = 0;
  bool keep_stores = false;
  load_bs(j0, 0);
  load_gs(j0, 0);
  issue(j0, 0, 0);
  for (int jt = j0; jt < j1; ++jt) {
#pragma unroll
    for (int h = 0; h < NB; ++h)
#pragma unroll
      for (int i = 0; i < MR; ++i)
#pragma unroll
        for (int j = 0; j < NR; ++j) acc[h][i][j] = AccT{0, 0, 0, 0};
    for (int kt = 0; kt < nk; ++kt) {
      if (keep_stores)
        wait_vmem_leaving<NSTR>();
      else
        wait_dma();
      keep_stores = false;
      workgroup_barrier();
      if constexpr (KIND == KIND_W4A16) {
        if (p.wgroup) {
#pragma unroll
          for (int h = 0; h < NB; ++h)
#pragma unroll
            for (int ni = 0; ni < NR; ++ni) {
              gs_c[h][ni][0] = gs_n[h][ni][0];
              gs_c[h][ni][1] = gs_n[h][ni][1];
            }
          if (kt + 1 < nk)
            load_gs(jt, kt + 1);
          else if (jt + 1 < j1)
            load_gs(jt + 1, 0);
        }
      }
      if constexpr (BS) {
#pragma unroll
        for (int mi = 0; mi < MR; ++mi) bsa_c[mi] = bsa_n[mi];
#pragma unroll
        for (int h = 0; h < NB; ++h)
#pragma unroll
          for (int ni = 0; ni < NR; ++ni) bsw_c[h][ni] = bsw_n[h][ni];
        if (kt + 1 < nk)
          load_bs(jt, kt + 1);
        else if (jt + 1 < j1)
          load_bs(jt + 1, 0);
      }
      if (kt + 1 < nk)
        issue(jt, kt + 1, slot ^ 1);
      else if (jt + 1 < j1)
        issue(jt + 1, 0, slot ^ 1);
      compute(ring + slot * C::SLOT);
      slot ^= 1;
    }
    epilogue(jt, ring + (slot ^ 1) * C::SLOT, ring + (slot ^ 1) * C::SLOT);
    keep_stores = rows;
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
  auto add = [&](const i32x4& w) {
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
  };
  if (topk == 8 && !mask) {
    // the common case: all eight slots' loads in flight at once, then the sums in slot order
    // (one load at a time left each thread waiting out the memory latency per slot)
    i32x4 w[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) w[k] = __builtin_nontemporal_load(src + (long)k * vpr);
#pragma unroll
    for (int k = 0; k < 8; ++k) add(w[k]);
  } else {
    for (int k = 0; k < topk; ++k) {
      if (mask && mask[(long)t * topk + k] == 0) continue;
      add(__builtin_nontemporal_load(src + (long)k * vpr));
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
