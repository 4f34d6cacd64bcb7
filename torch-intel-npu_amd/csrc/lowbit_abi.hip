// C-ABI of liblowbit_hip.so: argument validation, regime dispatch and launches.
// Declarations and contracts: include/lowbit_hip.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cmath>
#include <cstdio>
#include <mutex>
#include <string>

#include "../../include/lowbit_hip.h"
#include "abi_util.h"
#include "fused_launch.h"
#include "lb_stream.h"
#include "lb_gemm.h"
#include "lb_kernels.h"
#include "lb_variants.h"
#include "lb_wide.h"

using namespace lb;
using namespace lb::abi;

namespace {

#ifndef LB_GEMM_FROM_M
#define LB_GEMM_FROM_M 17  // from this many rows, calls with K >= N that no streaming GEMV takes run
#endif                     // on the split-K GEMM (measured faster there up to 32 rows; K < N stays on gemv_kernel)
enum Path { PATH_GEMV = 0, PATH_GEMM = 1, PATH_GENERIC = 2, PATH_ROW = 3, PATH_STREAM = 4, PATH_TILE = 5, PATH_WIDE = 6 };
enum Variant { VAR_PLAIN = 0, VAR_COMPACT = 1, VAR_W8A8 = 2 };
constexpr int kCompactMaxGroups = 32;
constexpr int64_t kW8A8MaxK = 131072;  // |sum| <= K * 128 * 127 stays inside int32

constexpr int kGemvMaxM = 32;
constexpr size_t kGemvLdsBudget = 48 * 1024;

int codes_per_load(int fmt) { return fmt == FMT_FP16 ? 8 : fmt == FMT_INT8 ? 16 : 32; }

struct Plan {
  int path = PATH_GENERIC;
  int variant = VAR_PLAIN;
  size_t xq_off = 0, pieces_off = 0;
  int kg = 1, splits = 1, kslice = 0, kc = 0;
  size_t z_off = 0, z_bytes = 0;
  size_t d_off = 0, d_bytes = 0;
  size_t part_off = 0, part_bytes = 0;
  size_t total = 0;
  bool zeroed = false;  // LB_FLAG_ZEROED_WORKSPACE: [0, LB_ZEROED_WORKSPACE_BYTES) is zero and reserved
};

bool is_pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

int group_shift(int64_t group, int64_t K) {
  if (group == K) return 31;  // one scale per row: index k >> 31 == 0
  int sh = 0;
  while ((int64_t)1 << sh < group) ++sh;
  return sh;
}

// Whether the MFMA fast paths can run these arguments.
bool fast_eligible(int fmt, int64_t K, int64_t group, const void *codes, const void *x, int64_t ldx, int64_t ldw) {
  if (K % 32 != 0) return false;
  if (fmt != FMT_FP16 && !(group == K || (group % 32 == 0 && is_pow2(group)))) return false;
  if (!aligned(codes, 16) || !aligned(x, 16) || ldx % 8 != 0) return false;
  if (fmt == FMT_FP16 && ldw % 8 != 0) return false;
  return true;
}

#ifndef LB_GEMV_TARGET_WAVES
#define LB_GEMV_TARGET_WAVES 4096
#endif
#ifndef LB_GEMV_SPLIT_BELOW
#define LB_GEMV_SPLIT_BELOW 1024  // split K across workgroups only when fewer waves than this
#endif
#ifndef LB_GEMV_MAX_KG
#define LB_GEMV_MAX_KG 4
#endif
#ifndef LB_GEMV_SPLIT
#define LB_GEMV_SPLIT 1
#endif
constexpr int64_t kGemvTargetWaves = LB_GEMV_TARGET_WAVES;

struct GemvShape {
  int kg = 1, splits = 1, kslice = 0, kc = 0;
};

#ifndef LB_GEMV_M_TARGET_WGS
#define LB_GEMV_M_TARGET_WGS 512  // workgroups the several-row GEMV aims for
#endif
#ifndef LB_GEMV_M_MIN_BYTES
#define LB_GEMV_M_MIN_BYTES (2 << 20)  // weights from this size on use the several-row shape
#endif
#ifndef LB_GEMV_M_MIN_M
#define LB_GEMV_M_MIN_M 8              // ... at this many activation rows or more
#endif
constexpr size_t kGemvRowsLds = 64 * 1024;

// Several activation rows, a large weight and too few 64-row tiles to fill the chip: four 16-row
// tiles per workgroup (one per wave, so the staged activations serve 64 weight rows) and K split
// across workgroups, each staging its slice of x once, for ~LB_GEMV_M_TARGET_WGS workgroups with
// at least four 16-byte loads per lane in every slice.
GemvShape gemv_shape_rows(int fmt, int64_t M, int64_t N, int64_t K) {
  GemvShape gs;
  const int cpl = codes_per_load(fmt);
  const int kstep = 4 * cpl;
  const int64_t ksteps = (K + kstep - 1) / kstep;
  const int64_t wg_tiles = (N + 63) / 64;
  const int64_t room = (int64_t)((kGemvRowsLds - 8 * 1024) / 2 / (M + 1)) - 4 * cpl - 8;  // 8 KB for scales
  const int64_t ks_max = std::max<int64_t>(kstep, room / kstep * kstep);
  gs.kg = 1;
  // From 16 rows on, twice the workgroups (shorter K slices): M = 16 4096x14336 29.8 -> 26.1 us, while
  // M = 8 keeps 512 (20.7 us against 24.6 with 1024).
  const int64_t target = M >= 16 ? 2 * LB_GEMV_M_TARGET_WGS : LB_GEMV_M_TARGET_WGS;
  int64_t s = std::max<int64_t>((K + ks_max - 1) / ks_max,
                                std::min<int64_t>((target + wg_tiles - 1) / wg_tiles,
                                                  std::max<int64_t>(1, ksteps / 4)));
  const int64_t ks = round_up((K + s - 1) / s, kstep);
  gs.splits = (int)((K + ks - 1) / ks);
  gs.kslice = (int)ks;
  gs.kc = (int)ks;
  return gs;
}

// In-workgroup K groups (KG) and cross-workgroup splits so the grid holds ~kGemvTargetWaves
// waves while each wave keeps at least one full batch of loads per split.
GemvShape gemv_shape(int fmt, int64_t M, int64_t N, int64_t K, bool allow_split) {
  const int64_t weight_bytes = fmt == FMT_FP16 ? 2 * N * K : fmt == FMT_INT8 ? N * K : N * K / 2;
  if (allow_split && M >= LB_GEMV_M_MIN_M && weight_bytes >= LB_GEMV_M_MIN_BYTES && (N + 63) / 64 < LB_GEMV_M_TARGET_WGS)
    return gemv_shape_rows(fmt, M, N, K);
  GemvShape gs;
  const int kstep = 4 * codes_per_load(fmt);
  const int64_t tiles = (N + 15) / 16;
  const int64_t ksteps = (K + kstep - 1) / kstep;
  int kg = 1;
  const int max_kg = std::min(LB_GEMV_MAX_KG, kGemvWaves);
  while (kg < max_kg && tiles * kg * 2 <= kGemvTargetWaves && ksteps >= 4 * kg) kg *= 2;
  int64_t s = 1;
  if (LB_GEMV_SPLIT && allow_split && tiles * kg < LB_GEMV_SPLIT_BELOW)
    s = std::max<int64_t>(1, std::min<int64_t>((kGemvTargetWaves + tiles * kg - 1) / (tiles * kg),
                                               ksteps / ((int64_t)kg * kGemvBatch)));
  const int64_t ks = round_up((K + s - 1) / s, kstep);
  s = (K + ks - 1) / ks;
  gs.kg = kg;
  gs.splits = (int)s;
  gs.kslice = (int)ks;
  const int64_t budget = (int64_t)(kGemvLdsBudget / 2 / (M + 1)) - 4 * codes_per_load(fmt) - 8;
  const int64_t c = std::max<int64_t>(kstep, budget / kstep * kstep);
  gs.kc = (int)std::min<int64_t>(c, ks);
  return gs;
}

#ifndef LB_GEMM_BM
#define LB_GEMM_BM 128
#endif
#ifndef LB_GEMM_BN
#define LB_GEMM_BN 128
#endif
#ifndef LB_GEMM_BK
#define LB_GEMM_BK 64
#endif
#ifndef LB_GEMM_BIG_MIN
#define LB_GEMM_BIG_MIN 160  // 128 x 128 tiles from this many workgroups
#endif
#ifndef LB_GEMM4_WAVES
#define LB_GEMM4_WAVES 8        // waves per 256 x 256 tile (4: 128 x 128 per wave; 8: 128 x 64)
#endif
#ifndef LB_GEMM4_WM
#define LB_GEMM4_WM 2           // waves along M of a 256 x 256 tile
#endif
#ifndef LB_GEMM_MID_WAVES
#define LB_GEMM_MID_WAVES 8     // waves per 128 x 128 tile ...
#endif
#ifndef LB_GEMM_MID_WM
#define LB_GEMM_MID_WM 2        // ... and along its M
#endif
#ifndef LB_GEMM4_MIN_TILES
#define LB_GEMM4_MIN_TILES 160  // 256 x 256 tiles from this many workgroups
#endif
#ifndef LB_GEMM_TALL_MIN
#define LB_GEMM_TALL_MIN 160  // 256 x 128 tiles (LB_GEMM_TALL_WAVES waves) from this many workgroups ...
#endif
#ifndef LB_GEMM_TALL_WAVES
#define LB_GEMM_TALL_WAVES 8  // 256 x 128 tiles: 8 waves of 64 x 64, or 4 of 128 x 64
#endif
#ifndef LB_GEMM_TALL_MAX
#define LB_GEMM_TALL_MAX 256  // ... up to this many (one workgroup per CU)
#endif
#ifndef LB_GEMM_MID
#define LB_GEMM_MID 1  // 128 x 128 tiles: 1 gemm4_kernel (LB_GEMM_MID_WAVES waves), 0 gemm2_kernel
#endif
#ifndef LB_GEMM_SPLIT_WGS
#define LB_GEMM_SPLIT_WGS 256   // split K while the tile grid has fewer workgroups than this
#endif
#ifndef LB_GEMM_SPLIT_MAX
#define LB_GEMM_SPLIT_MAX 4     // K slices at most
#endif
#ifndef LB_GEMM_SPLIT128_BELOW
#define LB_GEMM_SPLIT128_BELOW 160  // 128 x 128 grids below this many tiles may split along K
#endif
#ifndef LB_GEMM_SPLIT128_TARGET
#define LB_GEMM_SPLIT128_TARGET 256  // workgroups a split 128 x 128 grid aims at (0: as many slices as allowed)
#endif
#ifndef LB_GEMM_SMALL4
#define LB_GEMM_SMALL4 1  // 64 x 64 tiles over k steps of 64: 1 gemm4_kernel, 0 gemm2_kernel
#endif
#ifndef LB_GEMM_SPLIT_LONG_STEPS
#define LB_GEMM_SPLIT_LONG_STEPS 16  // k steps per slice of a split 128 x 128 grid at least
#endif
#ifndef LB_GEMM_SPLIT_MIN_STEPS
#define LB_GEMM_SPLIT_MIN_STEPS 8  // k steps per slice at least
#endif

enum { GEMM_256 = 0, GEMM_128 = 1, GEMM_64 = 2, GEMM_64_K32 = 3, GEMM_256x128 = 4 };
struct GemmShape {
  int kind = GEMM_64;
  int splits = 1;
  int kslice = 0;
};

// Tile kernel and K split of a prefill GEMM:
//   - 256 x 256 tiles (gemm4_kernel) when they nearly fill the CUs;
//   - else 256 x 128 tiles (gemm4_kernel, eight waves of 64 x 64) when they fill the CUs in one round
//     (LB_GEMM_TALL_MIN to LB_GEMM_TALL_MAX workgroups) and the rows past M add at most an eighth;
//   - else 128 x 128 tiles (gemm4_kernel, eight waves of 64 x 32) from LB_GEMM_BIG_MIN workgroups on;
//   - else, for a small 128 x 128 grid (< LB_GEMM_SPLIT128_BELOW tiles) over long rows, 128 x 128
//     tiles split along K into slices of at least LB_GEMM_SPLIT_LONG_STEPS k steps, as few as give
//     LB_GEMM_SPLIT128_TARGET workgroups, when the slices fill the CUs;
//   - else 64 x 64 tiles (k steps of 64 where K allows, else 32), split along K when the grid has
//     fewer than LB_GEMM_SPLIT_WGS workgroups, into slices of at least LB_GEMM_SPLIT_MIN_STEPS
//     k steps, aiming at two workgroups per CU.
// Every split is at most LB_GEMM_SPLIT_MAX slices; the fp32 partials [splits, M, N] go to the
// workspace and splitk_reduce_kernel sums them in a fixed order and applies the epilogue.  The
// launcher recomputes the kind with allow_split = (p.splits > 1), which gives the planned one.
GemmShape gemm_shape(int64_t M, int64_t N, int64_t K, int64_t slices, bool allow_split) {
  GemmShape gs;
  const int64_t huge = ((M + 255) / 256) * ((N + 255) / 256) * slices;
  const int64_t big = ((M + LB_GEMM_BM - 1) / LB_GEMM_BM) * ((N + LB_GEMM_BN - 1) / LB_GEMM_BN) * slices;
  const int64_t small = ((M + 63) / 64) * ((N + 63) / 64) * slices;
  const int64_t tall = ((M + 255) / 256) * ((N + 127) / 128) * slices;
  const bool can_split = allow_split && slices == 1;
  const int64_t s128 = std::min<int64_t>(LB_GEMM_SPLIT_MAX, K / LB_GEMM_BK / LB_GEMM_SPLIT_LONG_STEPS);
  gs.kslice = (int)K;
  int64_t s = 1;
  int bk = K % 64 == 0 ? 64 : 32;
  if (huge >= LB_GEMM4_MIN_TILES && K % 64 == 0) {
    gs.kind = GEMM_256;
  } else if (tall >= LB_GEMM_TALL_MIN && tall <= LB_GEMM_TALL_MAX && K % 64 == 0 &&
             (M + 255) / 256 * 256 * 8 <= 9 * M) {
    gs.kind = GEMM_256x128;
  } else if (big >= LB_GEMM_BIG_MIN && K % LB_GEMM_BK == 0) {
    gs.kind = GEMM_128;
  } else if (can_split && K % LB_GEMM_BK == 0 && big < LB_GEMM_SPLIT128_BELOW && s128 > 1 &&
             big * s128 >= LB_GEMM_BIG_MIN) {
    gs.kind = GEMM_128;
    bk = LB_GEMM_BK;
    s = LB_GEMM_SPLIT128_TARGET > 0
            ? std::max<int64_t>(2, std::min<int64_t>(s128, (LB_GEMM_SPLIT128_TARGET + big - 1) / big))
            : s128;
  } else {
    gs.kind = bk == 64 ? GEMM_64 : GEMM_64_K32;
    if (can_split && small < LB_GEMM_SPLIT_WGS)
      s = std::min<int64_t>(std::min<int64_t>(LB_GEMM_SPLIT_MAX, (2 * LB_GEMM_SPLIT_WGS + small - 1) / small),
                            K / bk / LB_GEMM_SPLIT_MIN_STEPS);
  }
  if (s > 1) {
    const int64_t steps = K / bk;
    const int64_t ks = (steps + s - 1) / s * bk;
    gs.splits = (int)((K + ks - 1) / ks);
    gs.kslice = (int)ks;
  }
  return gs;
}

// One activation row: the single-tile kernel (all of a workgroup's loads in flight at once,
// correction z computed inside each workgroup for K <= kFusedMaxK) needs no workspace.
bool row_eligible(const lb_linear_args *a) {
  if (a->M != 1) return false;
  if (a->K > fused_kmax_limit((int)a->format))  // past the single-tile kernels: the stream kernel only
    return a->rank == 0 && stream_group_span((int)a->format, a->K, a->group_size) != 0;
  if (a->K > kFusedMaxK) {  // long rows: no correction, groups of at least 64 (or one per row)
    const bool dense = a->format == LB_FORMAT_FP16;
    if (a->rank > 0 || !(dense || a->group_size == a->K || a->group_size >= 64)) return false;
  }
  if (a->rank > kFusedMaxRank) return false;
  const int64_t up_ld = a->up_ld == 0 ? a->rank : a->up_ld;
  if (a->rank > 0 && (!aligned(a->down, 16) || !aligned(a->up, 16) || up_ld % 8 != 0)) return false;
  return true;
}

#ifndef LB_STREAM_ROWS_DECODE_MIN_M
#define LB_STREAM_ROWS_DECODE_MIN_M 5  // stream path from this many rows: stream_rows_kernel, below: stream_gemv_kernel
#endif
#ifndef LB_STREAM_ROWS_MIN_BYTES
#define LB_STREAM_ROWS_MIN_BYTES (64ll << 20)  // weights from which 2..16-row calls take stream_gemv_kernel
#endif

#ifndef LB_STREAM_WIDE_MIN_N
#define LB_STREAM_WIDE_MIN_N 32768  // 17..32 rows: stream_wide_kernel needs this many rows to fill the CUs
#endif

// Several activation rows, no correction, a long enough weight the stream kernels take.
bool stream_rows_eligible(const lb_linear_args *a) {
  if (a->rank > 0 || !stream_rows_ok((int)a->format, a->M, a->K, a->group_size)) return false;
  if (a->M > 16 && a->N < LB_STREAM_WIDE_MIN_N) return false;
  const int64_t bytes = a->format == LB_FORMAT_INT8 ? a->N * a->K : a->N * a->K / 2;
  return bytes >= LB_STREAM_ROWS_MIN_BYTES;
}

#ifndef LB_TILE_ROWS
#define LB_TILE_ROWS 1  // 2..16 rows below the streaming sizes: tile_rows_kernel (one workgroup per tile)
#endif
#ifndef LB_TILE_ROWS_MAX_M
#define LB_TILE_ROWS_MAX_M 32  // tile_rows_kernel up to this many activation rows (16 or 32)
#endif
#ifndef LB_TILE_ROWS_MAX_X_BYTES
#define LB_TILE_ROWS_MAX_X_BYTES (32ll << 20)  // activation bytes all tiles stage together, at most
#endif

// Several activation rows, no correction, rows the one-tile kernel stages whole (K <= 4096, and
// K <= 2048 beyond 8 rows), int4 / nf4 / int8 codes.  Every workgroup stages all M rows for its 1,
// 2 or 4 tiles, so the workgroups together read the activations that many times: past
// LB_TILE_ROWS_MAX_X_BYTES of those reads the tiled GEMV, whose workgroups share the staged rows
// over more tiles, measured faster.
// Longer rows go in K slices (tile_rows_slices_for: equal slices of whole 512-code steps and scale
// groups, fp32 partials added in slice order).
int tile_rows_slices(const lb_linear_args *a) {
  const bool per_row = a->format == LB_FORMAT_INT8 && a->group_size == a->K;
  return tile_rows_slices_for((int)a->M, a->N, a->K, a->group_size, per_row);
}

bool tile_rows_eligible(const lb_linear_args *a) {
  if (!LB_TILE_ROWS || a->rank > 0 || a->M < 2 || a->M > LB_TILE_ROWS_MAX_M) return false;
  const int slices = tile_rows_slices(a);
  if (slices < 1) return false;
  const int64_t ks = a->K / slices, tiles = (a->N + 15) / 16, tt = tile_rows_per_wg(tiles * slices, ks, a->M);
  const int64_t wgs = (tiles + tt - 1) / tt * slices;
  if (wgs * a->M * ks * 2 > LB_TILE_ROWS_MAX_X_BYTES) return false;
  // Past 16 rows INT8 stays on the tiled GEMV (per-row 1024x4096 at M = 32: 12.0 against 12.9 us).
  return a->format == LB_FORMAT_INT4 || a->format == LB_FORMAT_NF4 || (a->format == LB_FORMAT_INT8 && a->M <= 16);
}

#ifndef LB_WIDE_MIN_M
#define LB_WIDE_MIN_M 17  // wide_rows_kernel from this many activation rows (up to 32) ...
#endif
#ifndef LB_WIDE_MIN_BYTES
#define LB_WIDE_MIN_BYTES (4ll << 20)  // ... over INT8 weights of at least this many bytes
#endif
#ifndef LB_WIDE_MIN_BYTES_4BIT
#define LB_WIDE_MIN_BYTES_4BIT (16ll << 20)  // ... and INT4 / NF4 weights of at least this many (smaller
                                              // ones measured faster on tile_rows_kernel)
#endif
#ifndef LB_WIDE_MID_M
#define LB_WIDE_MID_M 9  // and from this many rows over INT4 / NF4 weights of LB_WIDE_MID_BYTES up to the
                         // streaming sizes, when the kernel adds its K slices itself
#endif
#ifndef LB_WIDE_MID_BYTES
#define LB_WIDE_MID_BYTES (16ll << 20)
#endif
#ifndef LB_WIDE_TARGET_WGS
#define LB_WIDE_TARGET_WGS 200  // K slices: the fewest that give this many workgroups
#endif
#ifndef LB_WIDE_IN_KERNEL_SLICES
#define LB_WIDE_IN_KERNEL_SLICES 4  // K slices added in the kernel (zeroed workspace) up to this many
#endif
#ifndef LB_WIDE_MAX_SLICES
#define LB_WIDE_MAX_SLICES 16
#endif

// Loads per scale group of wide_rows_kernel (0: per-row INT8), or -1 where its groups do not fit:
// a group is at least two 32-byte pieces of a row (INT4 / NF4 >= 128 codes, INT8 >= 64) and a chunk
// whole groups.
int wide_group_loads(int fmt, int64_t K, int64_t group) {
  if (fmt == FMT_INT8 && group == K) return 0;
  const int bits = fmt == FMT_INT8 ? 8 : 4;
  if (!is_pow2(group) || group * bits / 8 < 64 || wide_chunk_codes(fmt) % group != 0) return -1;
  return (int)(group * bits / 8 / 32);
}

// Whether wide_rows_kernel takes the shape (force flag: this only; the default dispatch adds the
// row count and weight size it is chosen for).
bool wide_shape_ok(const lb_linear_args *a) {
  const int fmt = (int)a->format;
  if ((fmt != FMT_INT4 && fmt != FMT_INT8 && fmt != FMT_NF4) || a->rank > 0 || a->M < 1 || a->M > 32) return false;
  if (a->K % wide_chunk_codes(fmt) != 0 || a->K > 65536) return false;
  if (wide_group_loads(fmt, a->K, a->group_size) < 0) return false;
  return aligned(a->codes, 16) && aligned(a->x, 16) && a->ldx % 8 == 0;
}

int wide_slices(int fmt, int64_t N, int64_t K);

// 17..32 rows over >= 16 MB of INT4 / NF4 or >= 4 MB of INT8; LB_WIDE_MID_M..16 rows over INT4 / NF4
// weights of LB_WIDE_MID_BYTES up to the streaming sizes (which keep larger weights, where they measured
// faster) whose K slices are few enough for the kernel to add (LB_WIDE_IN_KERNEL_SLICES): INT4 g128
// 14336x4096 M = 16 17.5 -> 16.7 us, M = 12 16.8 -> 16.2, NF4 M = 16 20.0 -> 18.7 against
// tile_rows_kernel, which stays faster with more slices or on INT8 (4096x14336 M = 16 17.2 against
// 20.0 us, 8192x4096 9.8 against 12.7, INT8 14336x4096 20.5 against 21.7).
bool wide_eligible(const lb_linear_args *a) {
  if (a->M < LB_WIDE_MID_M || !wide_shape_ok(a)) return false;
  const int64_t bytes = a->format == LB_FORMAT_INT8 ? a->N * a->K : a->N * a->K / 2;
  if (a->M >= LB_WIDE_MIN_M) return bytes >= (a->format == LB_FORMAT_INT8 ? LB_WIDE_MIN_BYTES : LB_WIDE_MIN_BYTES_4BIT);
  return a->format != LB_FORMAT_INT8 && bytes >= LB_WIDE_MID_BYTES && bytes < LB_STREAM_ROWS_MIN_BYTES &&
         wide_slices((int)a->format, a->N, a->K) <= LB_WIDE_IN_KERNEL_SLICES;
}

// K slices of wide_rows_kernel: the fewest dividing the chunk count that give LB_WIDE_TARGET_WGS
// workgroups (row blocks of kWideRows rows x slices), at most LB_WIDE_MAX_SLICES.
int wide_slices(int fmt, int64_t N, int64_t K) {
  const int64_t blocks = (N + kWideRows - 1) / kWideRows, chunks = K / wide_chunk_codes(fmt);
  int best = 1;
  for (int s = 1; s <= LB_WIDE_MAX_SLICES && s <= chunks; ++s) {
    if (chunks % s) continue;
    best = s;
    if (blocks * s >= LB_WIDE_TARGET_WGS) break;
  }
  return best;
}

// Workspace and kernel path of the compact_groups and W8A8 variants.
Plan make_variant_plan(const lb_linear_args *a, int variant) {
  Plan pl;
  pl.variant = variant;
  pl.zeroed = (a->flags & LB_FLAG_ZEROED_WORKSPACE) != 0;
  const int fmt = (int)a->format;
  bool eligible;
  if (variant == VAR_W8A8) {
    eligible = a->K % 64 == 0 && aligned(a->codes, 16) && aligned(a->x, 16) && a->ldx % 8 == 0;
  } else {
    // each group is a product of its own: K_group % 32 == 0 keeps its codes, scales and
    // activations at 16-byte offsets
    eligible = a->group_size % 32 == 0 && aligned(a->codes, 16) && aligned(a->x, 16) && a->ldx % 8 == 0;
  }
  if ((a->flags & LB_FLAG_FORCE_GENERIC) || !eligible) pl.path = PATH_GENERIC;
  else if (a->flags & LB_FLAG_FORCE_GEMM) pl.path = PATH_GEMM;
  else if ((a->flags & LB_FLAG_FORCE_GEMV) || a->M <= kGemvMaxM) pl.path = PATH_GEMV;
  else pl.path = PATH_GEMM;
  size_t off = pl.zeroed ? LB_ZEROED_WORKSPACE_BYTES : 0;
  if (variant == VAR_W8A8 && pl.path != PATH_GENERIC) {
    pl.xq_off = off;
    off = round_up(off + (size_t)a->M * a->K, 256);
  }
  if (variant == VAR_COMPACT) {
    pl.pieces_off = off;
    off = round_up(off + (size_t)(a->K / a->group_size) * a->M * a->N * 2, 256);
    if (pl.path == PATH_GEMV) {
      const GemvShape gs = gemv_shape(fmt, a->M, a->N, a->group_size, false);
      pl.kg = gs.kg;
      pl.kc = gs.kc;
    }
  }
  (void)fmt;
  pl.total = off;
  return pl;
}

Plan make_plan(const lb_linear_args *a, bool eligible) {
  Plan pl;
  const int fmt = (int)a->format;
  pl.zeroed = (a->flags & LB_FLAG_ZEROED_WORKSPACE) != 0;
  if (a->flags & LB_FLAG_FORCE_STREAM) {  // validated: the stream kernel takes the shape
    pl.path = a->M == 1 ? PATH_ROW : PATH_STREAM;
  } else if (a->flags & LB_FLAG_FORCE_WIDE) {  // validated: the wide kernel takes the shape
    pl.path = PATH_WIDE;
  } else if ((a->flags & LB_FLAG_FORCE_GENERIC) || !eligible) {
    pl.path = PATH_GENERIC;
  } else if (a->flags & LB_FLAG_FORCE_GEMM) {
    pl.path = PATH_GEMM;
  } else if (!(a->flags & LB_FLAG_FORCE_GEMV) && wide_eligible(a)) {
    pl.path = PATH_WIDE;
  } else if (!(a->flags & LB_FLAG_FORCE_GEMV) && row_eligible(a)) {
    pl.path = PATH_ROW;
  } else if (!(a->flags & LB_FLAG_FORCE_GEMV) && stream_rows_eligible(a)) {
    pl.path = PATH_STREAM;
  } else if (!(a->flags & LB_FLAG_FORCE_GEMV) && tile_rows_eligible(a)) {
    pl.path = PATH_TILE;
  } else if ((a->flags & LB_FLAG_FORCE_GEMV) || a->M < LB_GEMM_FROM_M || (a->M <= kGemvMaxM && a->K < a->N)) {
    pl.path = PATH_GEMV;
  } else {
    pl.path = PATH_GEMM;
  }
  size_t off = pl.zeroed ? LB_ZEROED_WORKSPACE_BYTES : 0;
  if (a->rank > 0 && pl.path != PATH_ROW) {
    pl.z_off = off;
    pl.z_bytes = (size_t)a->M * a->rank * 2;
    off = round_up(off + pl.z_bytes, 256);
    if (pl.path != PATH_GEMV) {
      pl.d_off = off;
      pl.d_bytes = (size_t)a->M * a->N * 2;
      off = round_up(off + pl.d_bytes, 256);
    }
  }
  if (pl.path == PATH_GEMM) {
    const GemmShape gs = gemm_shape(a->M, a->N, a->K, 1, true);
    pl.splits = gs.splits;
    pl.kslice = gs.kslice;
    if (pl.splits > 1) {
      pl.part_off = off;
      pl.part_bytes = (size_t)pl.splits * a->M * a->N * 4;
      off = round_up(off + pl.part_bytes, 256);
    }
  }
  if (pl.path == PATH_TILE) {
    pl.splits = tile_rows_slices(a);
    pl.kslice = (int)(a->K / pl.splits);
    if (pl.splits > 1) {
      pl.part_off = off;
      pl.part_bytes = (size_t)pl.splits * a->M * a->N * 4;
      off = round_up(off + pl.part_bytes, 256);
    }
  }
  if (pl.path == PATH_WIDE) {
    pl.splits = wide_slices(fmt, a->N, a->K);
    pl.kslice = (int)(a->K / pl.splits);
    if (pl.splits > 1) {
      pl.part_off = off;
      pl.part_bytes = (size_t)pl.splits * a->M * a->N * 4;
      off = round_up(off + pl.part_bytes, 256);
    }
  }
  if (pl.path == PATH_GEMV) {
    const GemvShape gs = gemv_shape(fmt, a->M, a->N, a->K, true);
    pl.kg = gs.kg;
    pl.splits = gs.splits;
    pl.kslice = gs.kslice;
    pl.kc = gs.kc;
    if (pl.splits > 1) {
      pl.part_off = off;
      pl.part_bytes = (size_t)pl.splits * a->M * a->N * 4;
      off = round_up(off + pl.part_bytes, 256);
    }
  }
  pl.total = off;
  return pl;
}

lb_status validate(const lb_linear_args *a, bool check_workspace, Plan *plan) {
  if (!a) return fail(LB_INVALID_ARGUMENT, "lb_linear: args is NULL");
  if (a->struct_size < sizeof(lb_linear_args))
    return fail(LB_INVALID_ARGUMENT, "lb_linear: struct_size %u < %zu", a->struct_size, sizeof(lb_linear_args));
  if (a->format > LB_FORMAT_FP16) return fail(LB_INVALID_ARGUMENT, "lb_linear: unknown format %u", a->format);
  if (a->M <= 0 || a->N <= 0 || a->K <= 0)
    return fail(LB_INVALID_ARGUMENT, "lb_linear: M, N, K must be positive (got %lld, %lld, %lld)",
                (long long)a->M, (long long)a->N, (long long)a->K);
  if (a->M > INT32_MAX || a->N > INT32_MAX || a->K > INT32_MAX || a->M * a->N > (int64_t)1 << 40 ||
      a->N * a->K > (int64_t)1 << 40)
    return fail(LB_UNSUPPORTED, "lb_linear: extents exceed the supported range");
  const bool dense = a->format == LB_FORMAT_FP16;
  if (!dense && (a->group_size < 1 || a->group_size > a->K || a->K % a->group_size != 0))
    return fail(LB_INVALID_ARGUMENT, "lb_linear: group_size %lld must divide K=%lld", (long long)a->group_size,
                (long long)a->K);
  if (!a->codes || !a->x || !a->y || (!dense && !a->scales))
    return fail(LB_INVALID_ARGUMENT, "lb_linear: codes, scales, x and y must be non-NULL");
  if (a->ldx < a->K || a->ldy < a->N)
    return fail(LB_INVALID_ARGUMENT, "lb_linear: ldx >= K and ldy >= N required");
  if (a->rank < 0 || a->rank > std::min(a->N, a->K))
    return fail(LB_INVALID_ARGUMENT, "lb_linear: rank %lld outside 0..min(N,K)", (long long)a->rank);
  const int64_t up_ld = a->up_ld == 0 ? a->rank : a->up_ld;
  if (a->rank > 0 && (!a->down || !a->up || up_ld < a->rank))
    return fail(LB_INVALID_ARGUMENT, "lb_linear: correction needs down, up and up_ld >= rank");
  if (!aligned(a->x, 2) || !aligned(a->y, 2) || (a->scales && !aligned(a->scales, 2)) ||
      (a->bias && !aligned(a->bias, 2)) || (dense && !aligned(a->codes, 2)) ||
      (a->rank > 0 && (!aligned(a->down, 2) || !aligned(a->up, 2))))
    return fail(LB_INVALID_ARGUMENT, "lb_linear: fp16 buffers must be 2-byte aligned");

  const int64_t code_bytes = dense ? a->N * a->K * 2
                             : a->format == LB_FORMAT_INT8 ? a->N * a->K
                                                           : (a->N * a->K + 1) / 2;
  const Range y = range_of(a->y, (size_t)((a->M - 1) * a->ldy + a->N) * 2, "y");
  const Range inputs[] = {
      range_of(a->x, (size_t)((a->M - 1) * a->ldx + a->K) * 2, "x"),
      range_of(a->codes, (size_t)code_bytes, "codes"),
      range_of(a->scales, dense ? 0 : (size_t)(a->N * (a->K / a->group_size) * 2), "scales"),
      range_of(a->bias, a->bias ? (size_t)a->N * 2 : 0, "bias"),
      range_of(a->down, a->rank > 0 ? (size_t)(a->rank * a->K * 2) : 0, "down"),
      range_of(a->up, a->rank > 0 ? (size_t)(((a->N - 1) * up_ld + a->rank) * 2) : 0, "up"),
      range_of(a->workspace, a->workspace ? a->workspace_bytes : 0, "workspace"),
  };
  for (const Range &r : inputs)
    if (overlaps(y, r)) return fail(LB_INVALID_ARGUMENT, "lb_linear: y overlaps %s", r.name);
  for (int i = 0; i < 6; ++i)
    if (overlaps(inputs[6], inputs[i]))
      return fail(LB_INVALID_ARGUMENT, "lb_linear: workspace overlaps %s", inputs[i].name);

  constexpr uint32_t kForce =
      LB_FLAG_FORCE_GEMV | LB_FLAG_FORCE_GEMM | LB_FLAG_FORCE_GENERIC | LB_FLAG_FORCE_STREAM | LB_FLAG_FORCE_WIDE;
  if (a->flags & ~(kForce | LB_FLAG_COMPACT_GROUPS | LB_FLAG_W8A8 | LB_FLAG_ZEROED_WORKSPACE))
    return fail(LB_INVALID_ARGUMENT, "lb_linear: unknown flags 0x%x", a->flags);
  if ((a->flags & LB_FLAG_FORCE_GEMV) && a->M > kGemvMaxM)
    return fail(LB_INVALID_ARGUMENT, "lb_linear: LB_FLAG_FORCE_GEMV needs M <= %d", kGemvMaxM);
  if (__builtin_popcount(a->flags & kForce) > 1)
    return fail(LB_INVALID_ARGUMENT, "lb_linear: at most one LB_FLAG_FORCE_* flag");
  if (a->flags & LB_FLAG_FORCE_STREAM) {
    const bool shape = a->M == 1 ? stream_group_span((int)a->format, a->K, a->group_size) != 0
                                 : stream_rows_ok((int)a->format, a->M, a->K, a->group_size);
    if ((a->flags & (LB_FLAG_COMPACT_GROUPS | LB_FLAG_W8A8)) || a->rank > 0 || !shape || !aligned(a->codes, 16) ||
        !aligned(a->x, 16) || a->ldx % 8 != 0)
      return fail(LB_UNSUPPORTED,
                  "lb_linear: LB_FLAG_FORCE_STREAM needs int4/int8 codes, no correction or variant, 16-byte aligned "
                  "codes/x rows, and M == 1 or 17 <= M <= 32 with K <= 16384 (a multiple of 32 / 16) and groups "
                  "spanning whole 128 / 64-code pieces, or 2 <= M <= 16 with K <= 4096 and longer groups as M grows");
  }
  if ((a->flags & LB_FLAG_FORCE_WIDE) && ((a->flags & (LB_FLAG_COMPACT_GROUPS | LB_FLAG_W8A8)) || !wide_shape_ok(a)))
    return fail(LB_UNSUPPORTED,
                "lb_linear: LB_FLAG_FORCE_WIDE needs int4/nf4/int8 codes, no correction or variant, M <= 32, "
                "16-byte aligned codes/x rows, K a multiple of %d (int4, nf4) / %d (int8) up to 65536, and per-row "
                "int8 or power-of-two groups of at least 128 (int4, nf4) / 64 (int8) codes dividing that",
                wide_chunk_codes(FMT_INT4), wide_chunk_codes(FMT_INT8));
  int variant = VAR_PLAIN;
  if (a->flags & LB_FLAG_W8A8) {
    // reference _activation_scale (torch_npu_lowbit.py:155-166)
    const float s = a->activation_scale;
    int exponent = 0;
    if ((a->flags & LB_FLAG_COMPACT_GROUPS) || a->format != LB_FORMAT_INT8 || a->group_size != a->K)
      return fail(LB_INVALID_ARGUMENT, "lb_linear: W8A8 requires per-channel int8 weights and no compact groups");
    if (!std::isfinite(s) || s < 0x1p-24f || s > 511.0f || std::frexp(s, &exponent) != 0.5f)
      return fail(LB_INVALID_ARGUMENT, "lb_linear: activation_scale must be a power of two in [2^-24, 511]");
    if (a->rank > 0) return fail(LB_UNSUPPORTED, "lb_linear: W8A8 takes no low-rank correction");
    if (a->K > kW8A8MaxK) return fail(LB_UNSUPPORTED, "lb_linear: W8A8 supports K <= %lld", (long long)kW8A8MaxK);
    variant = VAR_W8A8;
  } else if (a->flags & LB_FLAG_COMPACT_GROUPS) {
    if (dense) return fail(LB_INVALID_ARGUMENT, "lb_linear: compact groups need a packed int8/int4/nf4 weight");
    const int64_t groups = a->K / a->group_size;
    if (groups > kCompactMaxGroups)
      return fail(LB_INVALID_ARGUMENT, "lb_linear: compact groups support at most %d groups (got %lld)", kCompactMaxGroups,
                  (long long)groups);
    if (a->rank > 0) return fail(LB_UNSUPPORTED, "lb_linear: compact groups take no low-rank correction");
    if (groups > 1) variant = VAR_COMPACT;  // one group: the default graph (torch_npu_lowbit.py:235)
  }
  if (variant != VAR_PLAIN) {
    *plan = make_variant_plan(a, variant);
    if ((a->flags & (LB_FLAG_FORCE_GEMV | LB_FLAG_FORCE_GEMM)) && plan->path == PATH_GENERIC)
      return fail(LB_UNSUPPORTED, variant == VAR_W8A8
                                      ? "lb_linear: W8A8 MFMA path needs K %% 64 == 0, 16-byte aligned codes/x and ldx %% 8 == 0"
                                      : "lb_linear: compact MFMA path needs group %% 32 == 0, 16-byte aligned codes/x, ldx %% 8 == 0");
  } else {
    const bool eligible = fast_eligible((int)a->format, a->K, dense ? a->K : a->group_size, a->codes, a->x, a->ldx, a->K);
    if ((a->flags & (LB_FLAG_FORCE_GEMV | LB_FLAG_FORCE_GEMM)) && !(a->flags & LB_FLAG_FORCE_GENERIC) && !eligible)
      return fail(LB_UNSUPPORTED,
                  "lb_linear: forced MFMA path needs K %% 32 == 0, group == K or group %% 32 == 0, "
                  "16-byte aligned codes/x and ldx %% 8 == 0");
    *plan = make_plan(a, eligible);
  }
  if (check_workspace && plan->total > 0) {
    if (!a->workspace || a->workspace_bytes < plan->total)
      return fail(LB_INVALID_ARGUMENT, "lb_linear: workspace of %zu bytes required (got %zu)", plan->total,
                  a->workspace ? a->workspace_bytes : (size_t)0);
    if (!aligned(a->workspace, 256)) return fail(LB_INVALID_ARGUMENT, "lb_linear: workspace must be 256-byte aligned");
  }
  return ok();
}

template <int FMT, int MT, int KG, bool SCALED>
void launch_gemv_t(const LinearParams &p, int kc, hipStream_t s) {
  constexpr int rows = 16 * (kGemvWaves / KG);
  const dim3 grid((p.N + rows - 1) / rows, p.splits, p.slices);
  // Staged scales per row: the chunk's groups plus 4 zero entries for tail lanes.
  const int sc_ld = SCALED ? (p.group_shift >= 31 ? 1 : (kc >> p.group_shift) + 2) + 4 : 0;
  const size_t stage = (size_t)(p.M + 1) * (kc + 4 * codes_per_load(FMT) + 8) * 2 + (size_t)rows * sc_ld * 2;
  const size_t reduce = (size_t)(KG - 1) * (kGemvWaves / KG) * MT * 64 * 4 * sizeof(float);
  const size_t lds = (FMT == FMT_NF4 ? 1024 : 0) + std::max(stage, reduce);
  hipLaunchKernelGGL((gemv_kernel<FMT, MT, KG, SCALED>), grid, dim3(kGemvThreads), lds, s, p, kc, sc_ld);
}

template <int FMT, int MT, bool SCALED>
void launch_gemv_kg(const LinearParams &p, int kg, int kc, hipStream_t s) {
  if constexpr (kGemvWaves >= 8) {
    if (kg == 8) return launch_gemv_t<FMT, MT, 8, SCALED>(p, kc, s);
  }
  if (kg == 4)
    launch_gemv_t<FMT, MT, 4, SCALED>(p, kc, s);
  else if (kg == 2)
    launch_gemv_t<FMT, MT, 2, SCALED>(p, kc, s);
  else
    launch_gemv_t<FMT, MT, 1, SCALED>(p, kc, s);
}

template <int FMT, bool SCALED>
void launch_gemv_m(const LinearParams &p, int kg, int kc, hipStream_t s) {
  if (p.M <= 16)
    launch_gemv_kg<FMT, 1, SCALED>(p, kg, kc, s);
  else
    launch_gemv_kg<FMT, 2, SCALED>(p, kg, kc, s);
}

void launch_gemv(int fmt, bool scaled, const LinearParams &p, int kg, int kc, hipStream_t s) {
  switch (fmt) {
    case FMT_INT8:
      scaled ? launch_gemv_m<FMT_INT8, true>(p, kg, kc, s) : launch_gemv_m<FMT_INT8, false>(p, kg, kc, s);
      break;
    case FMT_INT4: launch_gemv_m<FMT_INT4, true>(p, kg, kc, s); break;
    case FMT_NF4: launch_gemv_m<FMT_NF4, true>(p, kg, kc, s); break;
    default: launch_gemv_m<FMT_FP16, false>(p, kg, kc, s); break;
  }
  if (p.splits > 1) {
    const size_t count = (size_t)p.M * p.N;
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s, p);
  }
}

// Launches the GEMM of p (p.splits > 1: grid z runs over the K slices, then the reduction).
template <int FMT, bool SCALED>
void launch_gemm_t(const LinearParams &p, hipStream_t s) {
  constexpr int BM = LB_GEMM_BM, BN = LB_GEMM_BN, BK = LB_GEMM_BK;
  const int kind = gemm_shape(p.M, p.N, p.K, p.slices, p.splits > 1).kind;
  const unsigned gz = (unsigned)(p.splits > 1 ? p.splits : p.slices);
  if (kind == GEMM_256) {
    hipLaunchKernelGGL((gemm4_kernel<FMT, SCALED, LB_GEMM4_WAVES, 256, 256, LB_GEMM4_WM>),
                       dim3((p.N + 255) / 256, (p.M + 255) / 256, gz), dim3(64 * LB_GEMM4_WAVES), 0, s, p);
  } else if (kind == GEMM_256x128) {
    constexpr int TW = LB_GEMM_TALL_WAVES;
    hipLaunchKernelGGL((gemm4_kernel<FMT, SCALED, TW, 256, 128, TW / 2>),
                       dim3((p.N + 127) / 128, (p.M + 255) / 256, gz), dim3(64 * TW), 0, s, p);
  } else if (kind == GEMM_128) {
#if LB_GEMM_MID
    hipLaunchKernelGGL((gemm4_kernel<FMT, SCALED, LB_GEMM_MID_WAVES, BM, BN, LB_GEMM_MID_WM>),
                       dim3((p.N + BN - 1) / BN, (p.M + BM - 1) / BM, gz), dim3(64 * LB_GEMM_MID_WAVES), 0, s, p);
#else
    hipLaunchKernelGGL((gemm2_kernel<FMT, SCALED, BM, BN, BK>), dim3((p.N + BN - 1) / BN, (p.M + BM - 1) / BM, gz),
                       dim3(256), 0, s, p);
#endif
  } else if (kind == GEMM_64) {
#if LB_GEMM_SMALL4
    hipLaunchKernelGGL((gemm4_kernel<FMT, SCALED, 4, 64, 64, 2>), dim3((p.N + 63) / 64, (p.M + 63) / 64, gz), dim3(256),
                       0, s, p);
#else
    hipLaunchKernelGGL((gemm2_kernel<FMT, SCALED, 64, 64, 64>), dim3((p.N + 63) / 64, (p.M + 63) / 64, gz), dim3(256),
                       0, s, p);
#endif
  } else {
    hipLaunchKernelGGL((gemm2_kernel<FMT, SCALED, 64, 64, 32>), dim3((p.N + 63) / 64, (p.M + 63) / 64, gz), dim3(256),
                       0, s, p);
  }
}

void launch_gemm(int fmt, bool scaled, const LinearParams &p, hipStream_t s) {
  switch (fmt) {
    case FMT_INT8: scaled ? launch_gemm_t<FMT_INT8, true>(p, s) : launch_gemm_t<FMT_INT8, false>(p, s); break;
    case FMT_INT4: launch_gemm_t<FMT_INT4, true>(p, s); break;
    case FMT_NF4: launch_gemm_t<FMT_NF4, true>(p, s); break;
    default: launch_gemm_t<FMT_FP16, false>(p, s); break;
  }
  if (p.splits > 1) {
    const size_t count = (size_t)p.M * p.N;
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s, p);
  }
}

void launch_generic(int fmt, const LinearParams &p, hipStream_t s) {
  hipLaunchKernelGGL(generic_kernel, dim3(p.N, (p.M + 7) / 8), dim3(64), 0, s, p, fmt);
}

LinearParams base_params(int fmt, int64_t M, int64_t N, int64_t K, int64_t group, const void *codes,
                         const void *scales, const void *x, int64_t ldx, void *y, int64_t ldy, int64_t ldw) {
  LinearParams p{};
  p.codes = static_cast<const uint8_t *>(codes);
  p.scales = static_cast<const f16 *>(scales);
  p.x = static_cast<const f16 *>(x);
  p.y = static_cast<f16 *>(y);
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  p.group = (int)group;
  p.G = (int)(K / group);
  p.ldx = (int)ldx;
  p.ldy = (int)ldy;
  p.ldw = (int)ldw;
  p.per_row = fmt == FMT_INT8 && group == K;
  p.group_shift = group_shift(group, K);
  p.scales_aligned = aligned(scales, 16);
  p.splits = 1;
  p.kslice = (int)K;
  p.code_ld = (int)(fmt == FMT_FP16 ? ldw * 2 : fmt == FMT_INT8 ? K : K / 2);
  p.slices = 1;
  return p;
}

// Dense fp16 product out[M, N] = fp16(in[M, K] . W[N, K]^T), used for the correction stages.
void dense_fp16(int64_t M, int64_t N, int64_t K, const void *w, int64_t ldw, const void *in, int64_t ld_in,
                void *out, hipStream_t s) {
  LinearParams p = base_params(FMT_FP16, M, N, K, K, w, nullptr, in, ld_in, out, N, ldw);
  const bool eligible = fast_eligible(FMT_FP16, K, K, w, in, ld_in, ldw);
  if (!eligible) {
    launch_generic(FMT_FP16, p, s);
  } else if (M <= kGemvMaxM) {
    const GemvShape gs = gemv_shape(FMT_FP16, M, N, K, false);
    launch_gemv(FMT_FP16, false, p, gs.kg, gs.kc, s);
  } else {
    launch_gemm(FMT_FP16, false, p, s);
  }
}

// W8A8: quantize the activations into the workspace, then the int8 MFMA GEMV / GEMM (or the
// generic kernel, which quantizes as it reads).
void launch_w8a8(const lb_linear_args *a, const Plan &pl, LinearParams p, hipStream_t s) {
  p.act_scale = a->activation_scale;
  if (pl.path == PATH_GENERIC) {
    hipLaunchKernelGGL(generic_w8a8_kernel, dim3(p.N, (p.M + 7) / 8), dim3(64), 0, s, p);
    return;
  }
  p.xq = reinterpret_cast<const int8_t *>(static_cast<uint8_t *>(a->workspace) + pl.xq_off);
  const size_t blocks = (size_t)p.M * (p.K / 8);
  hipLaunchKernelGGL(quantize_rows_kernel, dim3((unsigned)((blocks + 255) / 256)), dim3(256), 0, s, p);
  if (pl.path == PATH_GEMV) {
    const dim3 grid((p.N + 15) / 16);
    if (p.M <= 16)
      hipLaunchKernelGGL(i8_gemv_kernel<1>, grid, dim3(256), 0, s, p);
    else
      hipLaunchKernelGGL(i8_gemv_kernel<2>, grid, dim3(256), 0, s, p);
  } else if (((int64_t)(p.M + 127) / 128) * ((p.N + 127) / 128) >= 256) {
    hipLaunchKernelGGL((i8_gemm_kernel<128, 128>), dim3((p.N + 127) / 128, (p.M + 127) / 128), dim3(256), 0, s, p);
  } else {
    hipLaunchKernelGGL((i8_gemm_kernel<64, 64>), dim3((p.N + 63) / 64, (p.M + 63) / 64), dim3(256), 0, s, p);
  }
}

// compact_groups: the fp16 product of each group into pieces[group, M, N] (the GEMV / GEMM
// kernels on grid slice z = group, or the generic kernel), then the balanced add tree + bias.
void launch_compact(const lb_linear_args *a, const Plan &pl, const LinearParams &p, hipStream_t s) {
  const int fmt = (int)a->format;
  const int groups = (int)(a->K / a->group_size);
  f16 *pieces = reinterpret_cast<f16 *>(static_cast<uint8_t *>(a->workspace) + pl.pieces_off);
  LinearParams q = p;
  q.per_row = 0;  // each piece multiplies by fp16(q*s): the group's Convert + Multiply (:249-251)
  q.bias = nullptr;
  if (pl.path == PATH_GENERIC) {
    hipLaunchKernelGGL(generic_pieces_kernel, dim3(p.N, (p.M + 7) / 8, groups), dim3(64), 0, s, q, fmt, pieces);
  } else {
    const int bits = fmt == FMT_INT8 ? 8 : 4;
    q.K = (int)a->group_size;
    q.group_shift = 31;  // one scale per row of a piece: index k >> 31 == 0
    q.kslice = q.K;
    q.splits = 1;
    q.code_ld = (int)(a->K * bits / 8);
    q.scales_aligned = 0;
    q.y = pieces;
    q.ldy = p.N;
    q.z_x = q.K;
    q.z_codes = q.K * bits / 8;
    q.z_scales = 1;
    q.z_y = (long long)p.M * p.N;
    q.slices = groups;
    if (pl.path == PATH_GEMV)
      launch_gemv(fmt, true, q, pl.kg, pl.kc, s);
    else
      launch_gemm(fmt, true, q, s);
  }
  const size_t count = (size_t)p.M * p.N;
  hipLaunchKernelGGL(compact_tree_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s, p,
                     (const f16 *)pieces, groups);
}


}  // namespace

// Scratch of lb_linear_noalloc: one array per GPU, held by the loaded code object until the process
// ends.  In host code the name `scratch` is only a handle for hipGetSymbolAddress; its device
// address (one per GPU) comes from scratch_address() and is what the kernels receive.
static __device__ __align__(256) uint8_t scratch[LB_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
void *scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the stream's GPU, looked up once per GPU with that GPU current.
lb_status scratch_address(hipStream_t stream, void **out) {
  int dev = -1;
  hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return fail(LB_DEVICE_FAILED, "lb_linear_noalloc: device of the stream: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(LB_UNSUPPORTED, "lb_linear_noalloc: device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (!scratch_ptr[dev]) {
    int current = -1;
    e = hipGetDevice(&current);
    if (e == hipSuccess && current != dev) e = hipSetDevice(dev);
    void *ptr = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (current >= 0 && current != dev) {
      const hipError_t back = hipSetDevice(current);
      if (e == hipSuccess) e = back;
    }
    if (e != hipSuccess || !ptr)
      return fail(LB_DEVICE_FAILED, "lb_linear_noalloc: scratch address on device %d: %s", dev,
                  e != hipSuccess ? hipGetErrorString(e) : "null");
    scratch_ptr[dev] = ptr;
  }
  *out = scratch_ptr[dev];
  return LB_OK;
}

}  // namespace

extern "C" {

int lb_abi_version(void) { return LB_ABI_VERSION; }

const char *lb_status_name(lb_status status) {
  switch (status) {
    case LB_OK: return "LB_OK";
    case LB_INVALID_ARGUMENT: return "LB_INVALID_ARGUMENT";
    case LB_OUT_OF_MEMORY: return "LB_OUT_OF_MEMORY";
    case LB_UNSUPPORTED: return "LB_UNSUPPORTED";
    case LB_DEVICE_FAILED: return "LB_DEVICE_FAILED";
    case LB_INTERNAL: return "LB_INTERNAL";
  }
  return "LB_UNKNOWN_STATUS";
}

const char *lb_last_error(void) { return last_error().c_str(); }

int lb_failed(void) { return failed_state().failed.load(std::memory_order_acquire) ? 1 : 0; }

void lb_mark_failed(const char *reason) { mark_failed(reason ? reason : "reported by the caller"); }

lb_status lb_workspace_bytes(const lb_linear_args *args, size_t *bytes) {
  if (!bytes) return fail(LB_INVALID_ARGUMENT, "lb_workspace_bytes: bytes is NULL");
  Plan plan;
  const lb_status st = validate(args, false, &plan);
  if (st != LB_OK) return st;
  *bytes = plan.total;
  return ok();
}

lb_status lb_linear(const lb_linear_args *a, void *stream) {
  if (const lb_status bad = refuse_if_failed("lb_linear"); bad != LB_OK) return bad;
  Plan plan;
  lb_status st = validate(a, true, &plan);
  if (st != LB_OK) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int fmt = (int)a->format;
  const bool dense = fmt == FMT_FP16;
  LinearParams p = base_params(fmt, a->M, a->N, a->K, dense ? a->K : a->group_size, a->codes, a->scales, a->x,
                               a->ldx, a->y, a->ldy, a->K);
  p.bias = static_cast<const f16 *>(a->bias);
  if (plan.variant == VAR_W8A8) {
    launch_w8a8(a, plan, p, s);
    return launch_status("lb_linear");
  }
  if (plan.variant == VAR_COMPACT) {
    launch_compact(a, plan, p, s);
    return launch_status("lb_linear");
  }
  if (plan.path == PATH_ROW) {
    const bool scaled = !dense && !p.per_row;
    FusedParams fp{};
    fp.x = p.x;
    fp.K = p.K;
    fp.G = p.G;
    fp.group_shift = p.group_shift;
    fp.per_row = p.per_row;
    fp.prologue = PRO_NONE;
    fp.force_stream = (a->flags & LB_FLAG_FORCE_STREAM) != 0;
    const int tiles = (int)((a->N + 15) / 16);
    FusedProblem &q = fp.prob[0];
    q.codes = p.codes;
    q.scales = p.scales;
    q.y = p.y;
    q.bias = p.bias;
    q.N = p.N;
    q.rank = (int)a->rank;
    if (a->rank > 0) {
      q.down = static_cast<const f16 *>(a->down);
      q.up = static_cast<const f16 *>(a->up);
      q.up_ld = (int)(a->up_ld == 0 ? a->rank : a->up_ld);
    }
    for (FusedProblem &r : fp.prob) r.tiles_end = tiles;
    launch_fused(fp, fmt, scaled, a->rank > 0, tiles, s);
    return launch_status("lb_linear");
  }
  if (plan.path == PATH_WIDE) {
    WideParams wp{};
    wp.x = p.x;
    wp.codes = p.codes;
    wp.scales = p.scales;
    wp.y = p.y;
    wp.bias = p.bias;
    wp.M = p.M;
    wp.N = p.N;
    wp.K = p.K;
    wp.G = p.G;
    wp.group_shift = p.group_shift;
    wp.ldx = p.ldx;
    wp.ldy = p.ldy;
    wp.kslice = plan.kslice;
    wp.per_row = p.per_row;
    wp.partial = plan.splits > 1 ? reinterpret_cast<float *>(static_cast<uint8_t *>(a->workspace) + plan.part_off)
                                 : nullptr;
    // With the zeroed counters the kernel adds the slices itself (one counter per 256-row block),
    // up to LB_WIDE_IN_KERNEL_SLICES of them (the adding workgroup reads every slice's partials).
    const bool in_kernel = plan.splits > 1 && plan.splits <= LB_WIDE_IN_KERNEL_SLICES && plan.zeroed && a->N % 4 == 0 &&
                           (a->N + kWideRows - 1) / kWideRows <= (int64_t)(LB_ZEROED_WORKSPACE_BYTES / 4);
    wp.tickets = in_kernel ? static_cast<uint32_t *>(a->workspace) : nullptr;
    launch_wide(wp, fmt, wide_group_loads(fmt, a->K, a->group_size), plan.splits, s);
    if (plan.splits > 1 && !in_kernel) {  // partials [slice, M, N] -> y in slice order (per-row scale, bias)
      p.partial = wp.partial;
      p.splits = plan.splits;
      const size_t count = (size_t)p.M * p.N;
      hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s, p);
    }
    return launch_status("lb_linear");
  }
  if (plan.path == PATH_STREAM || plan.path == PATH_TILE) {
    StreamParams sp{};
    sp.x = p.x;
    sp.codes = p.codes;
    sp.scales = p.scales;
    sp.y = p.y;
    sp.bias = p.bias;
    sp.M = p.M;
    sp.N = p.N;
    sp.K = p.K;
    sp.G = p.G;
    sp.group_shift = p.group_shift;
    sp.ldx = p.ldx;
    sp.ldy = p.ldy;
    sp.tiles = (int)((a->N + 15) / 16);
    if (plan.path == PATH_TILE) {
      bool in_kernel = false;
      if (plan.splits > 1) {  // K slices: fp32 partials, added by the kernel or by a second launch
        const int64_t tt = tile_rows_per_wg((int64_t)sp.tiles * plan.splits, plan.kslice, a->M);
        in_kernel = plan.zeroed && (sp.tiles + tt - 1) / tt <= (int64_t)(LB_ZEROED_WORKSPACE_BYTES / 4);
        sp.kslice = plan.kslice;
        sp.partial = reinterpret_cast<float *>(static_cast<uint8_t *>(a->workspace) + plan.part_off);
        sp.tickets = in_kernel ? static_cast<uint32_t *>(a->workspace) : nullptr;
      }
      launch_tile_rows(sp, fmt, !p.per_row, s);
      if (plan.splits > 1 && !in_kernel) {  // partials [slice, M, N] -> y in slice order (per-row scale, bias)
        p.partial = sp.partial;
        p.splits = plan.splits;
        const size_t count = (size_t)p.M * p.N;
        hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s, p);
      }
    } else if (a->M > 16) launch_stream_wide(sp, fmt, !p.per_row, s);
    else if (a->M >= LB_STREAM_ROWS_DECODE_MIN_M) launch_stream_rows(sp, fmt, !p.per_row, s);
    else launch_stream(sp, fmt, !p.per_row, stream_group_span(fmt, a->K, a->group_size), s);
    return launch_status("lb_linear");
  }
  uint8_t *ws = static_cast<uint8_t *>(a->workspace);
  if (a->rank > 0) {
    const int64_t up_ld = a->up_ld == 0 ? a->rank : a->up_ld;
    f16 *z = reinterpret_cast<f16 *>(ws + plan.z_off);
    // z = fp16(x . V^T)  (reference torch_npu_smollm.py:162, first MatMul of :256)
    dense_fp16(a->M, a->rank, a->K, a->down, a->K, a->x, a->ldx, z, s);
    if (plan.path == PATH_GEMV) {
      p.z = z;
      p.up = static_cast<const f16 *>(a->up);
      p.rank = (int)a->rank;
      p.up_ld = (int)up_ld;
    } else {
      // d = fp16(z . U^T)  (second MatMul of torch_npu_smollm.py:257)
      f16 *d = reinterpret_cast<f16 *>(ws + plan.d_off);
      dense_fp16(a->M, a->N, a->rank, a->up, up_ld, z, a->rank, d, s);
      p.delta = d;
    }
  }
  const bool scaled = !dense && !p.per_row;
  if (plan.path == PATH_GEMV) {
    p.splits = plan.splits;
    p.kslice = plan.kslice;
    p.partial = reinterpret_cast<float *>(ws + plan.part_off);
    launch_gemv(fmt, scaled, p, plan.kg, plan.kc, s);
  } else if (plan.path == PATH_GEMM) {
    p.splits = plan.splits;
    p.kslice = plan.kslice;
    p.partial = reinterpret_cast<float *>(ws + plan.part_off);
    launch_gemm(fmt, scaled, p, s);
  } else {
    launch_generic(fmt, p, s);
  }
  return launch_status("lb_linear");
}

lb_status lb_linear_noalloc(const lb_linear_args *a, void *stream) {
  if (const lb_status bad = refuse_if_failed("lb_linear_noalloc"); bad != LB_OK) return bad;
  if (!a) return fail(LB_INVALID_ARGUMENT, "lb_linear_noalloc: args is NULL");
  if (a->struct_size >= sizeof(lb_linear_args) && (a->workspace || a->workspace_bytes))
    return fail(LB_INVALID_ARGUMENT, "lb_linear_noalloc: workspace must be NULL / 0 (the library holds the scratch)");
  Plan plan;
  const lb_status st = validate(a, false, &plan);
  if (st != LB_OK) return st;
  lb_linear_args b = *a;  // validated: struct_size covers the struct
  b.flags &= ~LB_FLAG_ZEROED_WORKSPACE;  // the shared scratch promises nothing about its contents
  if (b.flags != a->flags) {
    const lb_status again = validate(&b, false, &plan);
    if (again != LB_OK) return again;
  }
  if (plan.total > LB_NOALLOC_SCRATCH_BYTES)
    return fail(LB_INVALID_ARGUMENT, "lb_linear_noalloc: the call needs %zu bytes of scratch; the allocation-free "
                "entry holds %zu (use lb_linear with a workspace)", plan.total, (size_t)LB_NOALLOC_SCRATCH_BYTES);
  if (plan.total > 0) {
    void *ptr = nullptr;
    const lb_status got = scratch_address(static_cast<hipStream_t>(stream), &ptr);
    if (got != LB_OK) return got;
    b.workspace = ptr;
    b.workspace_bytes = LB_NOALLOC_SCRATCH_BYTES;
  }
  return lb_linear(&b, stream);
}

lb_status lb_unpack_codes(uint32_t format, int64_t N, int64_t K, const void *codes, int8_t *out, void *stream) {
  if (const lb_status bad = refuse_if_failed("lb_unpack_codes"); bad != LB_OK) return bad;
  if (format > LB_FORMAT_NF4) return fail(LB_INVALID_ARGUMENT, "lb_unpack_codes: format must be int8/int4/nf4");
  if (N <= 0 || K <= 0 || !codes || !out) return fail(LB_INVALID_ARGUMENT, "lb_unpack_codes: bad arguments");
  const size_t count = (size_t)N * (size_t)K;
  const size_t code_bytes = format == LB_FORMAT_INT8 ? count : (count + 1) / 2;
  if (overlaps(range_of(out, count, "out"), range_of(codes, code_bytes, "codes")))
    return fail(LB_INVALID_ARGUMENT, "lb_unpack_codes: out overlaps codes");
  hipLaunchKernelGGL(unpack_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), (int)format, static_cast<const uint8_t *>(codes), count, out);
  return launch_status("lb_unpack_codes");
}

lb_status lb_dequantize(uint32_t format, int64_t N, int64_t K, int64_t group_size, const void *codes,
                        const void *scales, void *w_out, void *stream) {
  if (const lb_status bad = refuse_if_failed("lb_dequantize"); bad != LB_OK) return bad;
  if (format > LB_FORMAT_NF4) return fail(LB_INVALID_ARGUMENT, "lb_dequantize: format must be int8/int4/nf4");
  if (N <= 0 || K <= 0 || K > INT32_MAX || !codes || !scales || !w_out || group_size < 1 || group_size > K ||
      K % group_size != 0)
    return fail(LB_INVALID_ARGUMENT, "lb_dequantize: bad arguments");
  if (!aligned(scales, 2) || !aligned(w_out, 2))
    return fail(LB_INVALID_ARGUMENT, "lb_dequantize: fp16 buffers must be 2-byte aligned");
  const size_t count = (size_t)N * (size_t)K;
  const size_t code_bytes = format == LB_FORMAT_INT8 ? count : (count + 1) / 2;
  const Range out = range_of(w_out, count * 2, "w_out");
  if (overlaps(out, range_of(codes, code_bytes, "codes")) ||
      overlaps(out, range_of(scales, (size_t)N * (K / group_size) * 2, "scales")))
    return fail(LB_INVALID_ARGUMENT, "lb_dequantize: w_out overlaps an input");
  hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), (int)format, static_cast<const uint8_t *>(codes),
                     static_cast<const f16 *>(scales), (int)K, (int)group_size, (int)(K / group_size), count,
                     static_cast<f16 *>(w_out));
  return launch_status("lb_dequantize");
}

}  // extern "C"
