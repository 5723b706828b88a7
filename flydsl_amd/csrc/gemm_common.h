// Shared device helpers for the gfx950 quantized preshuffle GEMM kernels.
//
// Operand conventions (all kernels):
//   A    row-major [M][K] bytes (fp8 e4m3fn or int8).
//   B    preshuffled bytes: B[n][k] lives at (n/16)*16*K + (k/16)*256 + (n%16)*16 + (k%16)
//        (reference tests/utils.py:76-96 with layout=(16,16); device view
//        kernels/preshuffle_gemm.py:226-241).  INT4 B is that buffer with every 8 bytes
//        packed into 4 (test_preshuffle_gemm.py:165-174): B4[n][k] lives in the byte at
//        (n/16)*8*K + (k/16)*128 + (n%16)*8 + ((k%16)/8)*4 + (k%4), low nibble when
//        (k%8) < 4, high nibble otherwise.
//   K tile = 128 elements.  Within a tile, the 16-byte K chunks c = 0..7 are handed to the
//   MFMA so that lane l carries chunks (l/16) and (l/16)+4 of its row (A) / column (B).
//   A and B use the same chunk assignment, so the dot product over K is exact regardless
//   of how the hardware orders K inside one instruction.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <type_traits>

namespace flygemm {

typedef int   i32x2 __attribute__((ext_vector_type(2)));
typedef int   i32x4 __attribute__((ext_vector_type(4)));
typedef int   i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

enum Kind : int {
  KIND_FP8 = 0, KIND_INT8 = 1, KIND_INT4 = 2, KIND_BF16 = 3, KIND_F16 = 4, KIND_FP4 = 5,
  KIND_W4A16 = 6,  // MoE only: bf16 activations, int4 weights converted to bf16 in registers
};

// 16-bit inputs (bf16 / fp16) run through the same kernels in bytes: K counts bytes (two per
// element), the preshuffled B layout is the 1-byte layout applied to each row's bytes
// (reference tests/utils.py:76-96 with 8 elements per 16-byte chunk), and one
// v_mfma_f32_16x16x32_{bf16,f16} consumes the same 64 bytes of K per row and 16 bytes per
// lane as the int8 16x16x64 instruction.  They are not scaled (kernels/preshuffle_gemm.py:
// 804-806, 874-877).
constexpr bool kind_is_16bit(int k) { return k == KIND_BF16 || k == KIND_F16; }
constexpr bool kind_float_acc(int k) { return k == KIND_FP8 || kind_is_16bit(k) || k == KIND_FP4 || k == KIND_W4A16; }
// kinds whose epilogue applies no per-token / per-channel scale (MXFP4 scales live inside the MFMA)
constexpr bool kind_unscaled(int k) { return kind_is_16bit(k) || k == KIND_FP4; }

// MXFP4 (KIND_FP4): A packed e2m1 [M][K/2] bytes, B the preshuffled packed bytes (the 1-byte
// layout on rows of K/2 bytes), one E8M0 scale per 32 elements of K.  K here counts bytes, so a
// 128-byte K tile holds 256 elements = 8 scale blocks, consumed by two 16x16x128 MFMAs (h = 0,
// 1).  In MFMA h, lane group g = lane/16 supplies the 32 elements of scale block 4h + g, i.e.
// 16-byte chunk 4h + g of the tile, and its scale.  Scales arrive in the reference's shuffled
// order (tests/kernels/utils/fp4_utils.py:624-653): for 32 rows (or columns) r1 and K tile kt,
// lane l reads the 32-bit word (r1 * ktiles + kt) * 64 + l, whose byte 2h + p is the scale of
// 16-row block p (0/1) of the 32 for MFMA h -- the byte the MFMA's op_sel picks.
enum Epi : int {
  EPI_ROWCOL = 0,    // out = (acc * sa[m]) * sb[n]            (per-token / per-channel)
  EPI_BLOCK = 1,     // acc += mfma_block * (sa[kb][m] * sb[n/128][kb]) per 128-K block
  EPI_RAW = 2,       // raw accumulators: int32 (int8/int4) or fp32 (fp8), no scaling
};

constexpr int KT = 128;  // K elements per tile == blockscale K granularity

// E8M0 1.0 in all four byte lanes: the block-scale operand of the gfx950 scaled MFMA
// set to unity, so the instruction is the plain fp8 x fp8 -> fp32 product.
constexpr int kScaleOne = 0x7F7F7F7F;

__device__ __forceinline__ f32x4 mfma_fp8(const i32x8& a, const i32x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, kScaleOne, 0, kScaleOne);
}

__device__ __forceinline__ i32x4 mfma_i8(const i32x4& a, const i32x4& b, const i32x4& c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// One 64-byte-deep MFMA step of the int8 / bf16 / fp16 kinds on 16-byte operand fragments.
template <int KIND, typename AccT>
__device__ __forceinline__ AccT mfma_k64(const i32x4& b, const i32x4& a, const AccT& c) {
  if constexpr (KIND == KIND_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, b), __builtin_bit_cast(bf16x8, a), c, 0, 0, 0);
  else if constexpr (KIND == KIND_F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, b), __builtin_bit_cast(f16x8, a), c, 0, 0, 0);
  else
    return mfma_i8(b, a, c);
}

// v_mfma_scale_f32_16x16x128_f8f6f4 with both operands e2m1 (format 4); an fp4 operand is
// 16 bytes per lane, passed in the low half of the 8-dword operand.  H (0/1) is the MFMA's half
// of the 128-byte K tile; op_sel 2H picks byte 2H of each scale word, so callers pass the word
// shifted right by 8 bits for an odd 16-row (16-column) block, whose scale is byte 2H + 1.
template <int H>
__device__ __forceinline__ f32x4 mfma_fp4(const i32x4& b, const i32x4& a, const f32x4& c, uint32_t sb, uint32_t sa) {
  const i32x8 b8 = i32x8{b.x, b.y, b.z, b.w, 0, 0, 0, 0};
  const i32x8 a8 = i32x8{a.x, a.y, a.z, a.w, 0, 0, 0, 0};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(b8, a8, c, 4, 4, 2 * H, (int)sb, 2 * H, (int)sa);
}

// 8 packed int4 bytes (16 nibbles, little-endian) -> 16 int8 MFMA operands in four dwords: per
// source dword, the low nibbles of its bytes 0..3 first, then the high nibbles (the reference's
// unpack order, kernels/mfma_preshuffle_pipeline.py:277-291).  Each nibble lands in the high
// half of its byte with zeros below, i.e. as the int8 value 16 * n of the signed nibble n (its
// top bit becomes the byte's sign bit): (p << 4) & 0xF0F0F0F0 for the low nibbles,
// p & 0xF0F0F0F0 for the high ones -- three full-rate bit operations per dword, against seven
// for a sign extension in place (which held W4A8 steps back as VALU work next to the MFMAs).
// The int32 accumulators of int4 weights therefore hold 16x the dot product; int4_acc()
// divides it out exactly before anything reads them.  16 * |dot| <= 16 * 128 * 8 * K = 2^14 * K
// stays below 2^31 for K < kInt4KLimit = 2^17, which the entry points check.
__device__ __forceinline__ i32x4 unpack_int4x16(i32x2 p) {
  const uint32_t x = (uint32_t)p.x, y = (uint32_t)p.y;
  return i32x4{(int)((x << 4) & 0xF0F0F0F0u), (int)(x & 0xF0F0F0F0u), (int)((y << 4) & 0xF0F0F0F0u),
               (int)(y & 0xF0F0F0F0u)};
}
constexpr int kInt4KLimit = 131072;

// An accumulator as the dot product: int4 weights' accumulators hold 16x it (exact arithmetic
// shift), every other kind's are unchanged.
template <int KIND, typename T>
__device__ __forceinline__ T int4_acc(T v) {
  if constexpr (KIND == KIND_INT4)
    return v >> 4;
  else
    return v;
}

template <bool BF16>
struct OutT;
template <>
struct OutT<true> { typedef __bf16 type; };
template <>
struct OutT<false> { typedef _Float16 type; };

// fp32 -> output type, round to nearest even.  The value is pinned in a register first:
// otherwise the compiler folds the epilogue's last multiply into the fp16 conversion
// (v_fma_mixlo_f16, one rounding), while the reference rounds the product to fp32 and
// then to fp16.
template <bool BF16>
__device__ __forceinline__ typename OutT<BF16>::type cvt_out(float v) {
  asm volatile("" : "+v"(v));
  return static_cast<typename OutT<BF16>::type>(v);
}

// Four consecutive outputs (fp32) -> one 8-byte store of bf16/fp16 at element idx.
template <bool BF16>
__device__ __forceinline__ void store_out4(void* c, size_t idx, const float (&v)[4]) {
  typedef typename OutT<BF16>::type OT;
  typedef OT OT4 __attribute__((ext_vector_type(4)));
  OT4 o;
  o.x = cvt_out<BF16>(v[0]);
  o.y = cvt_out<BF16>(v[1]);
  o.z = cvt_out<BF16>(v[2]);
  o.w = cvt_out<BF16>(v[3]);
  *(OT4*)((OT*)c + idx) = o;
}

// Four fp32 outputs -> four bf16/fp16 packed in two dwords (for one 8-byte store).
template <bool BF16>
__device__ __forceinline__ i32x2 pack_out4(const float (&v)[4]) {
  typedef typename OutT<BF16>::type OT;
  typedef OT OT4 __attribute__((ext_vector_type(4)));
  OT4 o;
  o.x = cvt_out<BF16>(v[0]);
  o.y = cvt_out<BF16>(v[1]);
  o.z = cvt_out<BF16>(v[2]);
  o.w = cvt_out<BF16>(v[3]);
  return __builtin_bit_cast(i32x2, o);
}

struct GemmArgs {
  void* c;            // output [M][N] bf16/fp16, or int32/fp32 for EPI_RAW
  const uint8_t* a;   // [M][K] (16-bit kinds: K counts bytes)
  const uint8_t* b;   // preshuffled B
  const float* sa;    // EPI_ROWCOL: [M]; EPI_BLOCK: [K/128][M]
  const float* sb;    // EPI_ROWCOL: [N]; EPI_BLOCK: [ceil(N/128)][K/128]
  int M, N, K;
};

}  // namespace flygemm
