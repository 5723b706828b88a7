// C-ABI of the gfx950 quantized preshuffle GEMM library (declarations: include/flygemm.h).
//
// Every entry point validates its arguments on the host, picks a kernel variant (or uses
// the one the caller names), launches asynchronously on the caller's stream and returns 0
// or a nonzero error code; the message of the last failure on the calling thread is
// returned by flygemm_last_error().  Nothing here allocates device memory or synchronizes,
// and every GEMM is one kernel launch.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <map>
#include <mutex>
#include <utility>

#include "../../include/flygemm.h"
#include "abi_error.h"
#include "gemm_decode.h"
#include "gemm_main.h"
#include "quant_rows.h"

using namespace flygemm;

namespace {
thread_local char g_err[512] = "";
}  // namespace

// the one error slot of the library, shared by every translation unit (abi_error.h)
int flygemm::fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

namespace {

typedef void (*KernelFn)(GemmArgs);

// ---- variant table -------------------------------------------------------------------
enum Family { FAM_MAIN = 0, FAM_DECODE = 1 };

struct Shape {
  const char* name;
  int family;
  int bm, bn, threads;  // main: workgroup tile; decode/rows: bm = 16*MR rows, bn = 16*NBW cols
  bool rows;            // row-blocked streaming variant (chosen for M > 64 with few output tiles)
  int ksub;             // main: K tiles per pipeline step
};

// Ordered by preference: the selector takes the first tile that yields enough workgroups.
// (BM, BN, WM, WN, K tiles per step, name suffix).  The two-K-tile steps exist for the
// two-stage tiles without per-K-tile scales (int4 weights on the 4-wave tiles).
#define MAIN_SHAPES(X)       \
  X(256, 256, 2, 4, 1, "")   \
  X(256, 256, 4, 2, 1, "")   \
  X(128, 128, 2, 2, 1, "")   \
  X(64, 128, 1, 4, 1, "")    \
  X(256, 128, 2, 4, 1, "")   \
  X(128, 256, 2, 4, 1, "")   \
  X(256, 64, 4, 1, 1, "")    \
  X(128, 64, 2, 2, 1, "")    \
  X(64, 64, 1, 4, 1, "")     \
  X(64, 128, 1, 4, 2, "_k2") \
  X(64, 64, 1, 4, 2, "_k2")

#define DECODE_SHAPES(X) \
  X(1, 1, 8, 4)          \
  X(1, 2, 8, 4)          \
  X(1, 4, 8, 3)          \
  X(1, 7, 8, 2)          \
  X(1, 5, 8, 3)          \
  X(1, 10, 8, 2)         \
  X(2, 1, 8, 4)          \
  X(2, 2, 8, 3)          \
  X(4, 1, 8, 3)          \
  X(4, 2, 8, 2)          \
  X(8, 1, 8, 2)          \
  X(8, 2, 8, 1)          \
  X(1, 2, 4, 4)          \
  X(1, 4, 4, 4)          \
  X(1, 5, 4, 3)          \
  X(1, 7, 4, 2)          \
  X(2, 2, 4, 4)          \
  X(2, 4, 4, 2)

// The streaming kernel over row blocks (plain B loads: the row blocks of a column group re-read
// B from L2): for M too large for one row block but too small for the tiled kernel to give
// every CU an output tile (e.g. 128 x 4096: 64 tiles of 64x128).  (MR, NBW, waves, unroll).
#define ROW_SHAPES(X) \
  X(1, 4, 8, 3)       \
  X(2, 2, 8, 4)       \
  X(2, 4, 8, 3)

const Shape kShapes[] = {
#define MS(BM, BN, WM, WN, KS, SUF) {"main_" #BM "x" #BN "_w" #WM "x" #WN SUF, FAM_MAIN, BM, BN, WM * WN * 64, false, KS},
    MAIN_SHAPES(MS)
#undef MS
#define DS(MR, NBW, NW, U) {"decode_m" #MR "_nb" #NBW "_w" #NW "_u" #U, FAM_DECODE, 16 * MR, 16 * NBW, NW * 64, false, 1},
        DECODE_SHAPES(DS)
#undef DS
#define RS(MR, NBW, NW, U) {"rows_m" #MR "_nb" #NBW "_w" #NW "_u" #U, FAM_DECODE, 16 * MR, 16 * NBW, NW * 64, true, 1},
            ROW_SHAPES(RS)
#undef RS
};
constexpr int kNumShapes = sizeof(kShapes) / sizeof(kShapes[0]);
#define COUNT(...) +1
constexpr int kFirstDecode = 0 MAIN_SHAPES(COUNT);
constexpr int kFirstRows = kFirstDecode DECODE_SHAPES(COUNT);
#undef COUNT
// Fewer output tiles of 64x128 than the chip has CUs.  At most kRowsMaxTiles: the row-blocked
// streaming kernel (128x4096x4096 fp8 8.8 us; 64x128 tiles 16.0, 64x64 tiles 13.0); up to
// kSmallMaxTiles: 64x64 tiles, twice as many workgroups (graph-timed on MI355X, 64x64 against
// 64x128 and the row-blocked kernel: 96-128 tiles of 64x128 -- 256x4096x4096 fp8 13.2 us against
// 16.0 / 15.9, 128x8192x8192 27.7 against 34.2 / 33.9, 192x4096x4096 13.1 against 16.0 / 15.8,
// 128x7168x2048 int8 8.2 against 10.1 / 10.4, 256x4096x4096 bf16 24.8 against 30.6 / 29.0,
// int4 16.3 against 17.8 / 16.2, 128x7168x7168 blockscale 32.7 against 35.7 / 48.4; at 160 tiles
// 320x4096x4096 16.5 against 16.1, at 224 fp8 256x7168x7168 32.0 against 28.6).  Not for MXFP4.
// Blockscale and MXFP4 keep the row-blocked kernel up to 96 tiles (their 16-row blocks were
// measured against 64x128 only: blockscale 256x2112x7168 25.1 us against 40.6).
constexpr long kRowsMaxTiles = 64;
constexpr long kRowsMaxTiles16 = 96;
constexpr long kSmallMaxTiles = 144;
// Blockscale keeps 64x64 tiles up to 272 tiles of 64x128 (graph-timed on MI355X, 64x64 against
// 64x128: 1024x2112x7168 38.9 us against 42.7, 512x4096x7168 32.5 against 35.0, 256x7168x7168
// 35.6 against 36.4; at 448 tiles, 512x7168x2304, 19.9 against 17.2).
constexpr long kSmallMaxTilesBlock = 272;
constexpr long kMidMaxTiles = 256;
// CUs of an MI355X: the decode selection balances its workgroups over them
constexpr long kCUs = 256;

// The large-M kernel of one table entry.  Two K tiles per step need the two-stage ring and no
// per-K-tile scales; where a kind lacks them (the three-stage 4-wave tiles of fp8, int8 and
// 16-bit inputs, blockscale, MXFP4) the entry runs the one-K-tile kernel of the same tile.
template <int BM, int BN, int WM, int WN, int KS, int KIND, int EPI, bool BF16>
constexpr KernelFn main_fn() {
  if constexpr (KS > 1 && MainCfg<BM, BN, WM, WN, KIND>::NS == 2 && EPI != EPI_BLOCK && KIND != KIND_FP4)
    return gemm_main_kernel<BM, BN, WM, WN, KIND, EPI, BF16, KS>;
  else
    return gemm_main_kernel<BM, BN, WM, WN, KIND, EPI, BF16>;
}

// One row of kernels per (kind, epilogue, output dtype) combination, one column per shape.
template <int KIND, int EPI, bool BF16>
struct KernelRow {
  static const KernelFn* get() {
    static const KernelFn fns[] = {
#define MS(BM, BN, WM, WN, KS, SUF) main_fn<BM, BN, WM, WN, KS, KIND, EPI, BF16>(),
        MAIN_SHAPES(MS)
#undef MS
#define DS(MR, NBW, NW, U) gemm_decode_kernel<MR, NBW, NW, U, KIND, EPI, BF16, true>,
            DECODE_SHAPES(DS)
#undef DS
#define RS(MR, NBW, NW, U) gemm_decode_kernel<MR, NBW, NW, U, KIND, EPI, BF16, false>,
                ROW_SHAPES(RS)
#undef RS
    };
    static_assert(sizeof(fns) / sizeof(fns[0]) == kNumShapes, "variant table mismatch");
    return fns;
  }
};

const KernelFn* kernel_row(int kind, int epi, int out_dtype) {
  const bool bf16 = out_dtype == FLYGEMM_OUT_BF16;
  if (epi == EPI_ROWCOL) {
    if (kind == KIND_FP8) return bf16 ? KernelRow<KIND_FP8, EPI_ROWCOL, true>::get() : KernelRow<KIND_FP8, EPI_ROWCOL, false>::get();
    if (kind == KIND_INT8) return bf16 ? KernelRow<KIND_INT8, EPI_ROWCOL, true>::get() : KernelRow<KIND_INT8, EPI_ROWCOL, false>::get();
    if (kind == KIND_INT4) return bf16 ? KernelRow<KIND_INT4, EPI_ROWCOL, true>::get() : KernelRow<KIND_INT4, EPI_ROWCOL, false>::get();
    if (kind == KIND_BF16) return bf16 ? KernelRow<KIND_BF16, EPI_ROWCOL, true>::get() : KernelRow<KIND_BF16, EPI_ROWCOL, false>::get();
    if (kind == KIND_F16) return bf16 ? KernelRow<KIND_F16, EPI_ROWCOL, true>::get() : KernelRow<KIND_F16, EPI_ROWCOL, false>::get();
    if (kind == KIND_FP4) return bf16 ? KernelRow<KIND_FP4, EPI_ROWCOL, true>::get() : KernelRow<KIND_FP4, EPI_ROWCOL, false>::get();
  } else if (epi == EPI_BLOCK) {
    if (kind == KIND_FP8) return bf16 ? KernelRow<KIND_FP8, EPI_BLOCK, true>::get() : KernelRow<KIND_FP8, EPI_BLOCK, false>::get();
  } else if (epi == EPI_RAW) {
    if (kind == KIND_FP8) return KernelRow<KIND_FP8, EPI_RAW, true>::get();
    if (kind == KIND_INT8) return KernelRow<KIND_INT8, EPI_RAW, true>::get();
    if (kind == KIND_INT4) return KernelRow<KIND_INT4, EPI_RAW, true>::get();
    if (kind == KIND_BF16) return KernelRow<KIND_BF16, EPI_RAW, true>::get();
    if (kind == KIND_F16) return KernelRow<KIND_F16, EPI_RAW, true>::get();
    if (kind == KIND_FP4) return KernelRow<KIND_FP4, EPI_RAW, true>::get();
  }
  return nullptr;
}

// Row-blocked streaming variant for an output too small for the tiled kernel to occupy the
// chip.  Every workgroup of (16*MR) x (16*NBW) outputs reads (16*MR + 16*NBW) * K bytes from L2
// (or HBM), so for 256 workgroups 32x64 blocks move the fewest bytes.  Measured on MI355X
// (kernel time, graph replay): 128x4096x4096 fp8 8.9 us (64x128 tiles: 15.3, 32x32 blocks:
// 13.3), the same shape int8/int4/bf16 8.8/8.9/15.9 against 16.0/17.3/30.2, 200x2048x8192 fp8
// 14.2 against 26.8.  Blockscale and MXFP4 keep MR = 1: their per-tile scales make the 32-row
// block spill registers (blockscale 256x2112x7168: 16x64 blocks 25.1 us, 32x64 37.1, 64x128
// tiles 40.6; MXFP4 128x4096x4096: 9.1 against 10.9).
int select_rows(int M, int N, int kind, int epi) {
  // 16-row blocks also where their workgroups fill the last round over the CUs better than
  // 32-row blocks do (ties: 32 rows; graph-timed: 48x4096x4096 fp8 7.2 us against 9.0 -- 192
  // workgroups against 128 --, int4 6.6 against 8.5, bf16 12.2 against 15.0; 48x7168x2048 fp8
  // 6.8 with 32-row blocks -- 224 workgroups against 336 -- against 8.3; 128x4096x4096 256 or
  // 512 workgroups: 32-row blocks, 8.8 us)
  auto fill = [&](int rows) {
    const long wg = (long)((M + rows - 1) / rows) * ((N + 63) / 64);
    return (double)wg / (double)(((wg + kCUs - 1) / kCUs) * kCUs);
  };
  const int mr = (epi == EPI_BLOCK || kind == KIND_FP4 || fill(16) > fill(32)) ? 1 : 2;
  for (int v = kFirstRows; v < kNumShapes; ++v)
    if (kShapes[v].bm == 16 * mr && kShapes[v].bn == 64) return v;
  return -1;
}

// the main family's one-K-tile variant of a tile shape (-1: none)
int main_shape(int bm, int bn) {
  for (int v = 0; v < kFirstDecode; ++v)
    if (kShapes[v].bm == bm && kShapes[v].bn == bn && kShapes[v].ksub == 1) return v;
  return -1;
}

int select_variant(int M, int N, int K, int kind, int epi) {
  // The decode family up to 32 rows; above that its per-row A traffic grows and the 64x128 tile
  // is faster (and above 16 rows with the blockscale epilogue when N has at least 32 column tiles
  // of 128).  Measured on MI355X for every kind: fp8/int8/int4 (N x K = 28672x8192, 4096x4096,
  // 7168x2048, 14336x4096, 8192x8192), bf16 and MXFP4 (28672x8192, 8192x8192), blockscale
  // (7168x7168, 2112x7168); e.g. 64x28672x8192 fp8 43.8 us against 77.4, bf16 86 against 144,
  // blockscale 64x7168x7168 18.1 against 33.2.  With the 4-wave 32-row forms the decode family
  // also takes 17-32 rows of wide N (graph-timed against the best of the 64x128 / 64x64 tiles:
  // fp8 20x40960x5120 36.5 us against 63.1 for the 256x256 tile the main family gave it,
  // 28x77824x5120 64.8 against 76.4, 32x28672x8192 42.6 against 41.1, 32x25600x4096 22.1 against
  // 21.3; bf16 and int8 alike (bf16 32x25600x4096 41.0 against 38.3); int4 32x28672x8192 28.0
  // against 44.1, 28x77824x5120 43.7 against 40.6).
  const int ncol = (N + 127) / 128;
  const bool tile_small_m = M > 32 || (M > 16 && epi == EPI_BLOCK && ncol >= 32);
  if (M <= 64 && !tile_small_m) {
    // decode family: fewest rows that cover M, then the column blocks per workgroup
    const int rows = M <= 16 ? 16 : (M <= 32 ? 32 : 64);
    const int nblk = N / 16;
    // One 16-row block: the most column blocks per workgroup whose workgroups fill their last
    // round over the 256 CUs to at least 75% -- a partly filled last round runs the tail on a
    // fraction of the chip.  Column groups of 2-7 blocks run in 4-wave workgroups (two share a
    // CU, one's reduction and epilogue under the other's loads), one block in 8 waves; int4
    // keeps 8 waves and alone takes ten blocks (half-size blocks; fp8 with ten spills registers:
    // 77.6 us on 40960x5120); MXFP4 takes at most two (its scale words spill four on 4 waves),
    // on 4 waves only above 256 workgroups.  Graph-timed on MI355X against every variant, 16 x N
    // x K, 12 N x K per kind (10 for blockscale), the rule lands within 5% of the fastest on all
    // but two (blockscale 24576x1536 and 32768x512, 25% / 7%): fp8 40960x5120 33.7 us (5 blocks,
    // 512 workgroups) against 35.4 on 8 waves and 38.6 with 7 blocks (366, the last round 43%
    // full); 77824x5120 62.5 against 65.1; 12288x4096 10.5 with 4 blocks (192 workgroups)
    // against 13.3 with 1 (the former 85% bar); 28672x8192 37.9 either way; int8 alike; bf16
    // 40960x5120 63.0 against 74.0 (the former rule for other kinds), 18432x7168 41.3 against
    // 58.1; MXFP4 24576x8192 18.9 against 23.4; blockscale 36864x7168 41.9 against 61.1,
    // 18432x7168 22.3 against 31.1; int4 40960x5120 19.3 with 10 blocks, its 4-wave forms level
    // or up to 11% slower.  32-row blocks follow the same rule with 1, 2 or 4 blocks (int4 too,
    // in 4 waves: 32x28672x8192 28.0 us on 4 blocks against 39.1 on 2 in 8 waves; fp8
    // 32x14336x4096 12.6 against 16.4, 32x12288x4096 11.7 against 15.9, 32x7168x2048 5.8 against
    // 7.9).  Without a choice that fills 75% (few columns), the rule below.
    if (rows <= 32) {
      int best = -1;
      for (int v = kFirstDecode; v < kFirstRows; ++v) {
        if (kShapes[v].bm != rows) continue;
        const int nbw = kShapes[v].bn / 16;
        const bool four = kShapes[v].threads == 256;
        const long wg = (nblk + nbw - 1) / nbw;
        bool ok;
        if (kind == KIND_INT4 && rows == 16)
          ok = !four;
        else if (kind == KIND_FP4)
          ok = nbw <= 2 && four == (nbw == 2 && wg > kCUs);
        else
          ok = nbw != 10 && four == (nbw > 1);
        if (!ok) continue;
        const long rounds = (wg + kCUs - 1) / kCUs;
        if (wg * 100 >= rounds * kCUs * 75 && (best < 0 || nbw > kShapes[best].bn / 16)) best = v;
      }
      if (best >= 0) return best;
    }
    // otherwise the most column blocks per workgroup that still leaves about one workgroup per CU
    int best = -1;
    for (int v = kFirstDecode; v < kFirstRows; ++v) {
      if (kShapes[v].bm != rows) continue;
      const int nbw = kShapes[v].bn / 16;
      if (kind == KIND_FP4 && nbw > 4) continue;  // MXFP4's scale words push 7 blocks past the register file
      if (nbw == 5 || nbw == 10) continue;        // these and the 4-wave forms serve the 16-row rule
      if (kShapes[v].threads == 256) continue;
      // int4 blocks carry half the bytes: 4 blocks per workgroup beat 2 even at 224 workgroups
      // (16x14336x4096: 7.6 us against 8.5)
      const int min_wg = kind == KIND_INT4 ? 200 : 240;
      if (best < 0 || (nblk / nbw >= min_wg && nbw > kShapes[best].bn / 16)) best = v;
    }
    return best;
  }
  // main family: the first tile in a measured preference list that gives enough workgroups
  // to occupy the chip (256 CUs) and not too many.  Without the blockscale epilogue 256x256
  // wins from about 160 tiles (1536x8192x8192: 88 us against 110 for 128x256; 512x28672x8192:
  // 113 against 166), the three-stage 128x256 tile with 200-256 tiles (1024x7168x7168: fp8
  // 58.3 us against 62.3 for 128x128, int8 59.1 against 62.4, bf16 107.7 against 118.0, MXFP4
  // 34.7 against 36.1; 1024x8192x8192 fp8 69.8 against 74.0) except for int4 (two stages
  // there), 128x128 when it gives more than one tile per CU (272+: at 256 tiles the 64x128
  // tile is still 3-25% faster, at 280-512 tiles 128x128 is 4-40% faster), and the 4-wave
  // 64x128 tile (two resident per CU) below that.
  struct Pref {
    int bm, bn, threads, min_wg, max_wg;
    bool int4;  // also for int4 weights
  };
  static const Pref kRowcol[] = {{256, 256, 512, 160, 1 << 30, true},
                                 {128, 256, 512, 200, 256, false},
                                 {128, 128, 256, 272, 1 << 30, true},
                                 {64, 128, 256, 0, 1 << 30, true}};
  // blockscale (measured on M = 128-4096 with N x K = 7168x7168, 2112x7168, 3072x1536,
  // 24576x1536): 256x256 from 160 tiles (4096x24576x1536: 196 us against 231 for 256x128;
  // 1536x7168x7168, 168 tiles: 107 against 110 for 128x128 and 121 for 128x256), then with
  // 160-256 tiles the three-stage 128x256 when N is a multiple of 256 (1024x7168x7168: 66.2 us
  // against 70.2 for 256x128; 2048x3072x1536: 19.4 against 20.4), 128x128 from 240.
  // Re-measured against 128x128 as well (graph-timed, the tiles forced): with K of at least 4096
  // 256x256 from 160 tiles also between one and two per CU (4096x7168x7168, 448 tiles: 220.8 us
  // against 246.8 for 256x128), and 128x128 before 256x128 (4096x2112x7168: 102.8 against
  // 120.1); with shorter K the three-stage 128x256 from 160 tiles whatever the count
  // (1536x24576x1536: 72.0 against 102.9 for 256x256, 1024x24576x1536 45.8 against 49.1 for
  // 256x128, 8192x7168x2048 132.9 against 156.4, 4096x3072x1536 29.9 against 41.6) -- and with
  // few rows 64-row tiles rather than 256-row ones (48x24576x1536: 10.7 against 16.6).
  static const Pref kBlock[] = {{256, 256, 512, 160, 1 << 30, true},
                                {128, 256, 512, 160, 256, true},
                                {128, 128, 256, 240, 1 << 30, true},
                                {64, 128, 256, 0, 1 << 30, true}};
  static const Pref kBlockShortK[] = {{128, 256, 512, 160, 1 << 30, true},
                                      {128, 128, 256, 240, 1 << 30, true},
                                      {64, 128, 256, 0, 1 << 30, true}};
  // int4 weights with few output tiles (at most 512 of 64x128): two K tiles per pipeline step.
  // A 4-wave tile's step moves little, so a step waits on DMA latency rather than bandwidth;
  // two K tiles per stage halve the waits (graph-timed on MI355X, int4 M x N x K with t 64x128
  // tiles: 64x64 tiles with two K tiles per step against the table's choice -- 64x14336x4096
  // (t = 112) 12.7 us against 17.5, 128x7168x8192 (112) 20.5 against 30.7, 256x4096x4096 (128)
  // 11.9 against 16.8, 128x14336x4096 (224) 14.1 against 18.3, 256x8192x4096 (256) 13.9 against
  // 18.4, 320x8192x8192 (320) 33.3 against 38.0; 64x128 tiles with two K tiles per step from 353
  // to 512 tiles with K of at least 8192: 256x14336x8192 (448) 39.4 against 47.7, while at K =
  // 4096 the one-K-tile 64x128 is level or faster (256x14336x4096: 19.6 against 19.7,
  // 384x8192x4096: 19.1 against 19.7); at most 64 tiles the row-blocked kernel stays faster:
  // 128x4096x4096 8.5 against 11.5)
  if (kind == KIND_INT4 && epi != EPI_BLOCK) {
    const long t128 = (long)((M + 63) / 64) * ((N + 127) / 128);
    auto find = [](int bm, int bn, int ks) {
      for (int v = 0; v < kFirstDecode; ++v)
        if (kShapes[v].bm == bm && kShapes[v].bn == bn && kShapes[v].ksub == ks) return v;
      return -1;
    };
    if (t128 > kRowsMaxTiles && t128 <= 352) return find(64, 64, 2);
    if (t128 > 352 && t128 <= 512 && K >= 8192) return find(64, 128, 2);
  }
  const bool bs_short = epi == EPI_BLOCK && K < 4096;
  const Pref* list = epi == EPI_BLOCK ? (bs_short ? kBlockShortK : kBlock) : kRowcol;
  const int n = epi == EPI_BLOCK ? (bs_short ? 3 : 4) : 4;
  for (int i = 0; i < n; ++i) {
    if (kind == KIND_INT4 && !list[i].int4) continue;
    if (epi == EPI_BLOCK && list[i].bm == 128 && list[i].bn == 256 && N % 256 != 0) continue;
    // one 128x256 tile per CU needs long K to amortise its fill and epilogue: below 32 K tiles
    // (4096 bytes) 128x128 is faster (fp8 1024x7168 with K = 1536 / 2048 / 3072: 15.1 / 18.2 /
    // 24.7 us against 16.1 / 19.2 / 25.7; int8 K = 2048 19.2 against 20.0; bf16 K = 1024 18.2
    // against 19.3; from K = 4096 bytes 128x256 wins: fp8 32.8 against 35.7, bf16 K = 2048
    // 34.3 against 36.6).  Not for MXFP4, whose K bytes hold two elements (7168 elements,
    // 3584 bytes: 34.7 us against 36.1 for 128x128).
    if (epi != EPI_BLOCK && kind != KIND_FP4 && list[i].bm == 128 && list[i].bn == 256 && K < 4096) continue;
    const long wg = (long)((M + list[i].bm - 1) / list[i].bm) * ((N + list[i].bn - 1) / list[i].bn);
    if (wg < list[i].min_wg || wg > list[i].max_wg) continue;
    // int4 weights: 256x256 only from about 2.5 tiles per CU; below that 128x128 (graph-timed, int4:
    // 4096x4096x4096, 256 tiles of 256x256, 60.5 us against 70.9; 1024x14336x4096 58.0 against
    // 66.5; 2048x8192x8192 113.4 against 123.6; 4096x8192x8192 (512) 227.8 against 241.7;
    // 2048x7168x2048 33.9 against 47.4; from 600 tiles 256x256 wins: 8192^3 445.9 against 453.5,
    // 1536x28672x8192 (672) 300 against 327, 9728x8192x8320 508 against 547, 4096x28672x8192
    // 726 against 816)
    // -- except with one round of them and B far larger than A (N >= 16M), where two row blocks
    // read B half as often as 128x128's four (int4 x 28672 x 8192: 512 rows 109.6 us against 119.8,
    // 384 rows 102.6 against 107.0; with 768 rows, 336 tiles, 197.9 against 169.8)
    if (kind == KIND_INT4 && list[i].bm == 256 && list[i].bn == 256 && wg < 600 && !(wg <= kCUs && N >= 16L * M))
      continue;
    // int4 with 129-192 rows: 64x128 rather than 128x128 (three row blocks cover 192 rows, two of
    // 128 leave a quarter or more idle; x 28672 x 8192: 160 / 192 rows 55.2 / 55.9 us against
    // 58.5 / 59.3; 256 rows 69.3 against 64.2)
    if (kind == KIND_INT4 && epi != EPI_BLOCK && list[i].bm == 128 && list[i].bn == 128 && M > 128 && M <= 192)
      return main_shape(64, 128);
    // the last resort (64x128) leaves CUs idle with few tiles: the row-blocked streaming kernel
    // or 64x64 tiles spread the output over more CUs instead
    const long rows_max = (epi == EPI_BLOCK || kind == KIND_FP4) ? kRowsMaxTiles16 : kRowsMaxTiles;
    if (list[i].min_wg == 0 && wg <= rows_max) return select_rows(M, N, kind, epi);
    if (list[i].min_wg == 0 && wg <= (epi == EPI_BLOCK ? kSmallMaxTilesBlock : kSmallMaxTiles) && kind != KIND_FP4)
      for (int v = 0; v < kFirstDecode; ++v)
        if (kShapes[v].bm == 64 && kShapes[v].bn == 64) return v;
    // up to 256 such tiles and at least 384 rows: the same number of 128x64 tiles (graph-timed,
    // against 64x128: fp8 512x4096x7168 26.5 us against 27.7, 512x3072x7168 25.6 against 26.9,
    // 512x2560x8192 28.8 against 30.1, 384x5120x7168 27.3 against 28.0, 768x2112x4096 16.5
    // against 17.1, int8 512x4096x4096 16.7 against 17.3, bf16 30.6 against 31.5; at 256 rows
    // level or up to 2% slower; int4 10% slower), not for blockscale nor MXFP4
    if (list[i].min_wg == 0 && wg <= kMidMaxTiles && M >= 384 && epi != EPI_BLOCK && kind != KIND_INT4 &&
        kind != KIND_FP4 && (long)((M + 127) / 128) * ((N + 63) / 64) <= wg)
      return main_shape(128, 64);
    // 129-192 rows (two 128-row blocks against three of 64), or 65-128 rows with at least 96 MB
    // of B (which 64-row tiles read twice, past what the 256 MB last-level cache keeps): 128x64
    // tiles too (graph-timed against 64x128: fp8 144 / 160 / 192 x 14336 x 4096 24.4 / 24.1 /
    // 25.9 us against 26.7 / 27.1 / 27.9, int8 alike, bf16 43.8 / 44.7 / 48.1 against 52.8 /
    // 53.8 / 55.7, x 8192 x 8192 level to 4% faster; fp8 80 / 96 / 112 x 28672 x 8192 55.4 /
    // 58.0 / 60.3 against 57.3 / 60.2 / 62.6, bf16 107.0 / 111.0 / 115.6 against 113.3 / 118.2 /
    // 122.7; at 224-256 rows level or slower).  Not int4 nor MXFP4 (64x128 faster there at 160
    // and 192 rows: 14.4 / 14.5 us against 15.8 / 16.1), nor blockscale.
    // Above 192 rows the same holds for K of at least 8192 bytes (fp8 320 / 384 / 512 x 8192 x
    // 8192 48.5 / 51.5 / 54.8 against 49.8 / 53.4 / 56.1, bf16 92.4 / 97.1 / 100.1 against 95.1
    // / 102.5 / 106.5; bf16 x 4096 x 4096, 320-1024 rows, 3-7% faster), not for shorter K (fp8
    // 640x4096x4096 24.3 against 21.6, x 7168 x 2048 6-18% slower).  All of it where B
    // dominates, N >= 4M: with N near M the 64x128 tile is faster (bf16 1536x2112x7168 68.8
    // against 79.1).
    if (list[i].min_wg == 0 && epi != EPI_BLOCK && kind != KIND_INT4 && kind != KIND_FP4 && N >= 4L * M &&
        ((M > 128 && M <= 192) || (M > 64 && M <= 128 && (long)N * K >= (96L << 20)) || (M > 192 && K >= 8192)))
      return main_shape(128, 64);
    // 129-256 and 385-512 rows: 256x128 rather than 128x256 -- as many tiles, half the row
    // blocks, so B is read half as often (graph-timed, x 28672 x 8192: fp8 M = 144 / 160 / 192 /
    // 224 / 256 63.5 / 62.6 / 65.1 / 68.7 / 70.0 us against 74.6 / 74.6 / 74.6 / 72.4 / 73.1,
    // int8 alike, bf16 125.5 / 125.9 / 128.3 against 137.2 / 139.9 / 138.3 at 144-192 rows and
    // level at 224-256; fp16 and MXFP4 at 160 rows 128.4 / 37.6 against 141.6 / 42.0;
    // 512x14336x4096 fp8 34.7 against 36.0, bf16 64.9 against 68.9)
    if (epi != EPI_BLOCK && list[i].bm == 128 && list[i].bn == 256 && M > 128 && M <= 512 && ((M + 127) / 128) % 2 == 0)
      return main_shape(256, 128);
    for (int v = 0; v < kFirstDecode; ++v)
      if (kShapes[v].bm == list[i].bm && kShapes[v].bn == list[i].bn && kShapes[v].threads == list[i].threads) return v;
  }
  return -1;
}

// Persistent grid for the large-M kernel: as many workgroups as can be resident at once
// (CUs x workgroups per CU), at most one per tile, and a multiple of 8 when it is smaller
// than the tile count so every workgroup keeps to one XCD's share of the tiles.
// Occupancy is queried once per kernel and cached.
int persistent_grid(KernelFn fn, int threads, long ntiles, int* grid) {
  static std::mutex mu;
  static std::map<std::pair<int, const void*>, int> cache;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(e, "hipGetDevice: %s", hipGetErrorString(e));
  int slots;
  {
    std::lock_guard<std::mutex> lock(mu);
    auto key = std::make_pair(dev, (const void*)fn);
    auto it = cache.find(key);
    if (it == cache.end()) {
      int ncu = 0, per_cu = 0;
      e = hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
      if (e != hipSuccess) return fail(e, "device attribute query: %s", hipGetErrorString(e));
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void*)fn, threads, 0);
      if (e != hipSuccess) return fail(e, "occupancy query: %s", hipGetErrorString(e));
      it = cache.emplace(key, ncu * (per_cu > 0 ? per_cu : 1)).first;
    }
    slots = it->second;
  }
  long g = ntiles <= slots ? ntiles : (slots >= 8 ? slots - slots % 8 : slots);
  *grid = (int)g;
  return 0;
}

int check_common(const void* c, const void* a, const void* b, int M, int N, int K, int variant) {
  if (M < 0 || N <= 0 || K <= 0) return fail(hipErrorInvalidValue, "invalid sizes M=%d N=%d K=%d", M, N, K);
  if (N % 16 != 0) return fail(hipErrorInvalidValue, "N=%d must be a multiple of 16 (preshuffle block)", N);
  if (K % 64 != 0) return fail(hipErrorInvalidValue, "K=%d bytes must be a multiple of 64 (half K tile)", K);
  if ((long)(M + 256) * K >= (1L << 31) || (long)N * K >= (1L << 31) || (long)M * N * 4 >= (1L << 31))
    return fail(hipErrorInvalidValue, "operand too large for 32-bit element offsets (M=%d N=%d K=%d)", M, N, K);
  if (M > 0 && (!c || !a || !b)) return fail(hipErrorInvalidValue, "null tensor pointer");
  if (variant < -1 || variant >= kNumShapes) return fail(hipErrorInvalidValue, "unknown variant %d", variant);
  return 0;
}

// The kernel, grid and work items of one call (M > 0): variant -1 = the library's choice, else
// the index of a variant in the table.
struct Plan {
  int v;
  KernelFn fn;
  int grid, threads;
  long items;
};

int plan_launch(int kind, int epi, int out_dtype, int variant, int M, int N, int K, Plan* pl) {
  const int v = variant >= 0 ? variant : select_variant(M, N, K, kind, epi);
  if (v < 0 || v >= kNumShapes) return fail(hipErrorInvalidValue, "no kernel variant for M=%d N=%d K=%d", M, N, K);
  const Shape& s = kShapes[v];
  const KernelFn* row = kernel_row(kind, epi, out_dtype);
  if (!row) return fail(hipErrorInvalidValue, "unsupported combination kind=%d epilogue=%d", kind, epi);
  pl->v = v;
  pl->fn = row[v];
  pl->threads = s.threads;
  if (s.family == FAM_MAIN) {
    pl->items = (long)((M + s.bm - 1) / s.bm) * ((N + s.bn - 1) / s.bn);
    return persistent_grid(row[v], s.threads, pl->items, &pl->grid);
  }
  // one workgroup per (row block, column group); a decode shape normally has one row block
  const long nrb = (M + s.bm - 1) / s.bm;
  const long ncg = (N / 16 + s.bn / 16 - 1) / (s.bn / 16);
  pl->items = nrb * ncg;
  pl->grid = (int)pl->items;
  return 0;
}

int launch(int kind, int epi, int out_dtype, int variant, const GemmArgs& args, hipStream_t stream) {
  if (kind == KIND_INT4 && args.K >= kInt4KLimit)
    return fail(hipErrorInvalidValue, "K=%d: int4 weights take K < %d (int32 accumulators of 16x the dot product)",
                args.K, kInt4KLimit);
  if (args.M == 0) return 0;
  Plan pl;
  int rc = plan_launch(kind, epi, out_dtype, variant, args.M, args.N, args.K, &pl);
  if (rc) return rc;
  const Shape& s = kShapes[pl.v];
  hipLaunchKernelGGL(pl.fn, dim3(pl.grid), dim3(pl.threads), 0, stream, args);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(e, "launch of %s failed: %s", s.name, hipGetErrorString(e));
  return 0;
}

// ---- per-row quantization ------------------------------------------------------------
typedef void (*QuantFn)(QuantArgs);

// registers-resident variant for rows of up to 1, 2, 4 or 8 slices, streaming beyond
template <int IN, int OUT, int MODE, int NT>
QuantFn quant_fn(int nslices) {
  if (nslices <= 1) return quant_rows_kernel<IN, OUT, MODE, 1, NT>;
  if (nslices <= 2) return quant_rows_kernel<IN, OUT, MODE, 2, NT>;
  if (nslices <= 4) return quant_rows_kernel<IN, OUT, MODE, 4, NT>;
  if (nslices <= 8) return quant_rows_kernel<IN, OUT, MODE, 8, NT>;
  return quant_rows_kernel<IN, OUT, MODE, 0, NT>;
}

template <int IN, int NT>
QuantFn quant_fn_in(int out_dtype, int mode, int nslices) {
  if (out_dtype == QOUT_FP8)
    return mode == QMODE_DIV_NEAREST ? quant_fn<IN, QOUT_FP8, QMODE_DIV_NEAREST, NT>(nslices) : nullptr;
  if (mode == QMODE_RECIP_TRUNC) return quant_fn<IN, QOUT_INT8, QMODE_RECIP_TRUNC, NT>(nslices);
  if (mode == QMODE_DIV_TRUNC) return quant_fn<IN, QOUT_INT8, QMODE_DIV_TRUNC, NT>(nslices);
  if (mode == QMODE_DIV_NEAREST) return quant_fn<IN, QOUT_INT8, QMODE_DIV_NEAREST, NT>(nslices);
  return nullptr;
}

template <int NT>
QuantFn quant_fn_nt(int in_dtype, int out_dtype, int mode, int nslices) {
  return in_dtype == FLYGEMM_QIN_F16    ? quant_fn_in<QIN_F16, NT>(out_dtype, mode, nslices)
         : in_dtype == FLYGEMM_QIN_BF16 ? quant_fn_in<QIN_BF16, NT>(out_dtype, mode, nslices)
                                        : quant_fn_in<QIN_F32, NT>(out_dtype, mode, nslices);
}

// K in bytes for the kernels, which take K tiles of 128 bytes and a last tile of 64 bytes
// (the reference's tile_k * elem_bytes % 64 == 0, kernels/preshuffle_gemm.py:89-93): 16-bit
// inputs have two bytes per element and need K % 32 == 0; returns -1 after setting the error
// for a bad K.
int k_bytes(int in_dtype, int K) {
  if (in_dtype == FLYGEMM_IN_BF16 || in_dtype == FLYGEMM_IN_FP16) {
    if (K <= 0 || K % 32 != 0) {
      fail(hipErrorInvalidValue, "K=%d must be a multiple of 32 for 16-bit inputs (64-byte K tile)", K);
      return -1;
    }
    return 2 * K;
  }
  if (K <= 0 || K % 64 != 0) {
    fail(hipErrorInvalidValue, "K=%d must be a multiple of 64 (64-byte K tile)", K);
    return -1;
  }
  return K;
}

}  // namespace

extern "C" {

int flygemm_preshuffle(void* c, const void* a, const void* b, const float* scale_a, const float* scale_b,
                       int32_t M, int32_t N, int32_t K, int32_t in_dtype, int32_t out_dtype,
                       int32_t variant, void* stream) {
  if (in_dtype < FLYGEMM_IN_FP8 || in_dtype > FLYGEMM_IN_FP16)
    return fail(hipErrorInvalidValue, "in_dtype %d not supported", in_dtype);
  const int kb = k_bytes(in_dtype, K);
  if (kb < 0) return hipErrorInvalidValue;
  int rc = check_common(c, a, b, M, N, kb, variant);
  if (rc) return rc;
  if (out_dtype != FLYGEMM_OUT_BF16 && out_dtype != FLYGEMM_OUT_FP16)
    return fail(hipErrorInvalidValue, "out_dtype %d not supported", out_dtype);
  const bool scaled = in_dtype <= FLYGEMM_IN_INT4;
  if (M > 0 && scaled && (!scale_a || !scale_b)) return fail(hipErrorInvalidValue, "null scale pointer");
  GemmArgs args{c, (const uint8_t*)a, (const uint8_t*)b, scaled ? scale_a : nullptr, scaled ? scale_b : nullptr,
                M, N, kb};
  return launch(in_dtype, EPI_ROWCOL, out_dtype, variant, args, (hipStream_t)stream);
}

int flygemm_blockscale(void* c, const void* a, const void* b, const float* x_scale_t, const float* w_scale,
                       int32_t M, int32_t N, int32_t K, int32_t scale_block_k, int32_t out_dtype,
                       int32_t variant, void* stream) {
  if (scale_block_k != 128) return fail(hipErrorInvalidValue, "scale_block_k=%d: only 128 is supported", scale_block_k);
  if (K <= 0 || K % 128 != 0)
    return fail(hipErrorInvalidValue, "K=%d must be a multiple of scale_block_k=128", K);
  int rc = check_common(c, a, b, M, N, K, variant);
  if (rc) return rc;
  if (out_dtype != FLYGEMM_OUT_BF16 && out_dtype != FLYGEMM_OUT_FP16)
    return fail(hipErrorInvalidValue, "out_dtype %d not supported", out_dtype);
  if (M > 0 && (!x_scale_t || !w_scale)) return fail(hipErrorInvalidValue, "null scale pointer");
  GemmArgs args{c, (const uint8_t*)a, (const uint8_t*)b, x_scale_t, w_scale, M, N, K};
  return launch(KIND_FP8, EPI_BLOCK, out_dtype, variant, args, (hipStream_t)stream);
}

int flygemm_accumulators(void* acc, const void* a, const void* b, int32_t M, int32_t N, int32_t K,
                         int32_t in_dtype, int32_t variant, void* stream) {
  if (in_dtype < FLYGEMM_IN_FP8 || in_dtype > FLYGEMM_IN_FP16)
    return fail(hipErrorInvalidValue, "in_dtype %d not supported", in_dtype);
  const int kb = k_bytes(in_dtype, K);
  if (kb < 0) return hipErrorInvalidValue;
  int rc = check_common(acc, a, b, M, N, kb, variant);
  if (rc) return rc;
  GemmArgs args{acc, (const uint8_t*)a, (const uint8_t*)b, nullptr, nullptr, M, N, kb};
  return launch(in_dtype, EPI_RAW, FLYGEMM_OUT_BF16, variant, args, (hipStream_t)stream);
}

int flygemm_quant_rows(void* out, float* scales, const void* in, int32_t M, int32_t N, int32_t in_dtype,
                       int32_t out_dtype, int32_t mode, void* stream) {
  if (M < 0 || N <= 0) return fail(hipErrorInvalidValue, "invalid sizes M=%d N=%d", M, N);
  if (N % 8 != 0) return fail(hipErrorInvalidValue, "N=%d must be a multiple of 8 (16-byte row vectors)", N);
  if (in_dtype < FLYGEMM_QIN_F16 || in_dtype > FLYGEMM_QIN_F32)
    return fail(hipErrorInvalidValue, "quant in_dtype %d not supported", in_dtype);
  if (out_dtype != FLYGEMM_QOUT_FP8 && out_dtype != FLYGEMM_QOUT_INT8)
    return fail(hipErrorInvalidValue, "quant out_dtype %d not supported", out_dtype);
  if (mode < FLYGEMM_QMODE_RECIP_TRUNC || mode > FLYGEMM_QMODE_DIV_NEAREST)
    return fail(hipErrorInvalidValue, "quant mode %d not supported", mode);
  if (out_dtype == FLYGEMM_QOUT_FP8 && mode != FLYGEMM_QMODE_DIV_NEAREST)
    return fail(hipErrorInvalidValue, "fp8 output rounds to nearest: mode must be FLYGEMM_QMODE_DIV_NEAREST");
  const int esz = in_dtype == FLYGEMM_QIN_F32 ? 4 : 2;
  if ((long)M * N * esz >= (1L << 40)) return fail(hipErrorInvalidValue, "input too large (M=%d N=%d)", M, N);
  if (M == 0) return 0;
  if (!out || !scales || !in) return fail(hipErrorInvalidValue, "null pointer");
  if (((uintptr_t)in & 15) || ((uintptr_t)out & 7) || ((uintptr_t)scales & 3))
    return fail(hipErrorInvalidValue, "misaligned pointer (input needs 16-byte, output 8-byte alignment)");
  const int nt = N >= kQuantWideN ? 2 * kQuantThreads : kQuantThreads;
  const int nslices = (N + nt * 8 - 1) / (nt * 8);
  QuantFn fn = nt == kQuantThreads ? quant_fn_nt<kQuantThreads>(in_dtype, out_dtype, mode, nslices)
                                   : quant_fn_nt<2 * kQuantThreads>(in_dtype, out_dtype, mode, nslices);
  if (!fn) return fail(hipErrorInvalidValue, "unsupported quant combination");
  QuantArgs args{out, scales, in, M, N};
  hipLaunchKernelGGL(fn, dim3(M), dim3(nt), 0, (hipStream_t)stream, args);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(e, "launch of quant_rows failed: %s", hipGetErrorString(e));
  return 0;
}

int flygemm_preshuffle_quant_a(void* c, void* a_q, float* scale_a, const void* x, const void* b, const float* scale_b,
                               int32_t M, int32_t N, int32_t K, int32_t x_dtype, int32_t in_dtype, int32_t mode,
                               int32_t out_dtype, int32_t variant, void* stream) {
  if (in_dtype != FLYGEMM_IN_FP8 && in_dtype != FLYGEMM_IN_INT8 && in_dtype != FLYGEMM_IN_INT4)
    return fail(hipErrorInvalidValue, "in_dtype %d: activations are quantized to fp8 or int8 (in_dtype fp8, int8, int4)",
                in_dtype);
  if (x_dtype < FLYGEMM_QIN_F16 || x_dtype > FLYGEMM_QIN_F32)
    return fail(hipErrorInvalidValue, "x_dtype %d not supported", x_dtype);
  if (mode < FLYGEMM_QMODE_RECIP_TRUNC || mode > FLYGEMM_QMODE_DIV_NEAREST)
    return fail(hipErrorInvalidValue, "quant mode %d not supported", mode);
  if (in_dtype == FLYGEMM_IN_FP8 && mode != FLYGEMM_QMODE_DIV_NEAREST)
    return fail(hipErrorInvalidValue, "fp8 codes round to nearest: mode must be FLYGEMM_QMODE_DIV_NEAREST");
  const int kb = k_bytes(in_dtype, K);
  if (kb < 0) return hipErrorInvalidValue;
  int rc = check_common(c, x, b, M, N, kb, variant);
  if (rc) return rc;
  if (in_dtype == FLYGEMM_IN_INT4 && K >= kInt4KLimit)
    return fail(hipErrorInvalidValue, "K=%d: int4 weights take K < %d (int32 accumulators of 16x the dot product)", K,
                kInt4KLimit);
  if (out_dtype != FLYGEMM_OUT_BF16 && out_dtype != FLYGEMM_OUT_FP16)
    return fail(hipErrorInvalidValue, "out_dtype %d not supported", out_dtype);
  if (M > 0 && !scale_b) return fail(hipErrorInvalidValue, "null scale pointer");
  if (M == 0) return 0;
  if (!a_q || !scale_a)
    return fail(hipErrorInvalidValue, "a_q [M][K] and scale_a [M] are required: the quantization and the GEMM run as two "
                "launches through them");
  if (((uintptr_t)x & 15) || ((uintptr_t)a_q & 7) || ((uintptr_t)scale_a & 3))
    return fail(hipErrorInvalidValue, "misaligned pointer (x needs 16-byte, a_q 8-byte, scale_a 4-byte alignment)");
  const int qout = in_dtype == FLYGEMM_IN_FP8 ? FLYGEMM_QOUT_FP8 : FLYGEMM_QOUT_INT8;
  // Two launches: the quant kernel writes the codes and row scales once, then the GEMM reads
  // them.  A single kernel that quantized A inside the decode GEMM was built and measured on
  // MI355X (graph replay, bf16 activations): every column group's workgroup re-derives the
  // codes and scales of all its rows, work the quant kernel does once, so it never won --
  // int8 16x28672x8192 41.7 us against 41.2 for the pair, 1x7168x2048 7.8 against 5.2, fp8
  // (a true division per element) 77.8 against 42.8 -- and it was removed.
  rc = flygemm_quant_rows(a_q, scale_a, x, M, K, x_dtype, qout, mode, stream);
  if (rc) return rc;
  return flygemm_preshuffle(c, a_q, b, scale_a, scale_b, M, N, K, in_dtype, out_dtype, variant, stream);
}

int flygemm_mxfp4(void* c, const void* a, const void* b, const void* scale_a, const void* scale_b, int32_t M,
                  int32_t N, int32_t K, int32_t out_dtype, int32_t variant, void* stream) {
  if (K <= 0 || K % 256 != 0)
    return fail(hipErrorInvalidValue, "K=%d must be a multiple of 256 (8 scale blocks of 32 per K tile)", K);
  if (N % 32 != 0) return fail(hipErrorInvalidValue, "N=%d must be a multiple of 32 (scale groups)", N);
  int rc = check_common(c, a, b, M, N, K / 2, variant);
  if (rc) return rc;
  if (out_dtype != FLYGEMM_OUT_BF16 && out_dtype != FLYGEMM_OUT_FP16 && out_dtype != FLYGEMM_OUT_F32)
    return fail(hipErrorInvalidValue, "out_dtype %d not supported", out_dtype);
  if (M > 0 && (!scale_a || !scale_b)) return fail(hipErrorInvalidValue, "null scale pointer");
  // the MXFP4 compute reads one scale word per 32-column group of a wave's columns, so the
  // 64x64 tile's 16-column wave tiles are not available here
  if (variant >= 0 && kShapes[variant].family == FAM_MAIN && kShapes[variant].bm == 64 && kShapes[variant].bn == 64)
    return fail(hipErrorInvalidValue, "variant %s is not available for MXFP4 (16-column wave tiles split a scale group)",
                kShapes[variant].name);
  GemmArgs args{c, (const uint8_t*)a, (const uint8_t*)b, (const float*)scale_a, (const float*)scale_b, M, N, K / 2};
  if (out_dtype == FLYGEMM_OUT_F32) return launch(KIND_FP4, EPI_RAW, FLYGEMM_OUT_BF16, variant, args, (hipStream_t)stream);
  return launch(KIND_FP4, EPI_ROWCOL, out_dtype, variant, args, (hipStream_t)stream);
}

int32_t flygemm_num_variants(void) { return kNumShapes; }

const char* flygemm_variant_name(int32_t v) {
  if (v < 0 || v >= kNumShapes) return nullptr;
  return kShapes[v].name;
}

int32_t flygemm_select_variant(int32_t M, int32_t N, int32_t K, int32_t in_dtype, int32_t blockscale) {
  // the kernels count K in bytes: two per element for 16-bit inputs, half for MXFP4
  const int kb = (in_dtype == FLYGEMM_IN_BF16 || in_dtype == FLYGEMM_IN_FP16) ? 2 * K : (in_dtype == FLYGEMM_IN_FP4 ? K / 2 : K);
  return select_variant(M, N, kb, in_dtype, blockscale ? EPI_BLOCK : EPI_ROWCOL);
}

int flygemm_launch_shape(int32_t M, int32_t N, int32_t K, int32_t in_dtype, int32_t blockscale, int32_t variant,
                         int32_t* variant_out, int32_t* grid, int32_t* threads, int32_t* items) {
  if (in_dtype < FLYGEMM_IN_FP8 || in_dtype > FLYGEMM_IN_FP4)
    return fail(hipErrorInvalidValue, "in_dtype %d not supported", in_dtype);
  if (blockscale && in_dtype != FLYGEMM_IN_FP8) return fail(hipErrorInvalidValue, "blockscale takes fp8 inputs");
  if (M <= 0 || N <= 0 || K <= 0) return fail(hipErrorInvalidValue, "invalid sizes M=%d N=%d K=%d", M, N, K);
  if (variant < -1 || variant >= kNumShapes) return fail(hipErrorInvalidValue, "unknown variant %d", variant);
  if (!variant_out || !grid || !threads || !items) return fail(hipErrorInvalidValue, "null output pointer");
  const int kb = (in_dtype == FLYGEMM_IN_BF16 || in_dtype == FLYGEMM_IN_FP16) ? 2 * K : (in_dtype == FLYGEMM_IN_FP4 ? K / 2 : K);
  Plan pl;
  const int rc = plan_launch(in_dtype, blockscale ? EPI_BLOCK : EPI_ROWCOL, FLYGEMM_OUT_BF16, variant, M, N, kb, &pl);
  if (rc) return rc;
  *variant_out = pl.v;
  *grid = pl.grid;
  *threads = pl.threads;
  *items = (int32_t)pl.items;
  return 0;
}

const char* flygemm_last_error(void) { return g_err; }

}  // extern "C"
