// Host/device declarations shared by the translation units that launch the fused decode GEMV
// (lb_fused_linear and lb_linear's single-row path).
#pragma once
#include "lb_common.h"

namespace lb {

constexpr int kFusedMaxProblems = 3;
constexpr int kFusedMaxRank = 32;
constexpr int kFusedMaxK = 1536;
enum Prologue { PRO_NONE = 0, PRO_RMSNORM = 1, PRO_SILU_MUL = 2 };

struct FusedProblem {
  const uint8_t *codes;   // packed codes (fp16 weights for FMT_FP16), rows [N, K]
  const f16 *scales;      // [N, G]
  f16 *y;                 // [N]
  const f16 *bias;        // [N] or null
  const f16 *residual;    // [N] or null (may equal y: each element is read and written by one lane)
  const f16 *down;        // V [rank, K] or null
  const f16 *up;          // U [N, up_ld] or null
  int N, rank, up_ld;
  int tiles_end;          // exclusive prefix sum of 16-row tiles over the problems
  int zend;               // exclusive prefix sum of z workgroups over the problems (shared z)
};

// Shared correction activations: a launch with zblocks > 0 starts with that many z workgroups,
// each computing fp16(x'.V^T) for kFusedZRanks ranks of one problem.  Every three z values travel
// in one 64-bit word, zslot[problem][rank / 3], whose low 16 bits are the launch's tag; the tile
// workgroups read their problem's words with 64-bit atomic loads until every tag is current, then
// count themselves on `passed` (64-bit, monotonic).  A launch's tag is (passed / tiles + 1) mod
// 2^16, read by each workgroup at its start: only tile workgroups raise `passed`, each once per
// launch after the wait, so at any workgroup's start it holds launch * tiles plus fewer than
// `tiles`, and no word needs clearing between launches (the previous launch's tag is one behind).
// The wait is bounded: a timeout is recorded in a separate word.
constexpr int kFusedZRanks = 6;                                        // ranks per z workgroup
constexpr int kFusedZWordsPerProblem = (kFusedMaxRank + 2) / 3;        // 11 words hold 32 ranks
constexpr int kFusedZPassedOffset = 384;                               // byte offset of `passed` (u64)
constexpr int kFusedZTimeoutOffset = 392;                              // byte offset of the timeout word
constexpr int kFusedZSpinLimit = 1 << 18;
constexpr unsigned kWaitVmcnt0 = 0x0F70;                               // s_waitcnt vmcnt(0), others free

struct FusedParams {
  int force_stream;       // host-side dispatch only: take stream_gemv_kernel whatever the size
  const f16 *x;           // [K] activation (PRO_SILU_MUL: the gate row)
  const f16 *x2;          // PRO_SILU_MUL: the up row [K]
  const f16 *gamma;       // PRO_RMSNORM: [K]
  float eps;
  int K, G, group_shift, per_row, prologue;
  FusedProblem prob[kFusedMaxProblems];
  uint64_t *zslot;        // shared z words [kFusedMaxProblems][12], then `passed` and the timeout word
  int zblocks;            // z workgroups ahead of the tile workgroups (0: each tile computes z)
};

// Longest K a format's single-tile kernel takes (32 weight loads per lane); beyond
// kFusedMaxK only without a correction and with groups of at least 64 (or one per row).
constexpr int fused_kmax_limit(int format) {
  return format == FMT_FP16 ? 4096 : format == FMT_INT8 ? 8192 : 16384;
}

// Scales per 16-byte-load flush of stream_gemv_kernel for an INT4 / INT8 row of K codes in groups
// of `group` (1, 2 or 4), or 0 when the kernel does not take the shape: K <= 16384 and a multiple
// of the codes per lane load, one group per row or power-of-two groups (the kernel indexes scales
// by a shift), each 4-lane-load piece of a row spanning whole groups.
inline int stream_group_span(int format, long long K, long long group) {
  if (format != FMT_INT4 && format != FMT_INT8) return 0;
  const long long cpl = format == FMT_INT4 ? 32 : 16, cpw = 4 * cpl;
  if (K <= 0 || K > 16384 || K % cpl != 0 || group <= 0 || K % group != 0) return 0;
  if (group == K) return 1;
  if ((group & (group - 1)) != 0) return 0;
  if (group % cpw == 0) return 1;
  if (cpw % group != 0 || group < cpl) return 0;
  return (int)(cpw / group);
}

// Whether the streaming GEMVs take M activation rows (2 <= M <= 32) of such a shape: up to 16 rows
// are staged whole (K <= 4096), and with more rows each MFMA A row of stream_gemv_kernel spans
// more code blocks, so the groups must be longer (INT4: <= 2 groups per 128-code load up to 8
// rows, 1 for 16; INT8: one scale per 64-code load or one per row); 17 .. 32 rows run in
// stream_wide_kernel, which stages K in chunks.
inline bool stream_rows_ok(int format, long long M, long long K, long long group) {
  const int span = stream_group_span(format, K, group);
  if (span == 0 || M < 2 || M > 32) return false;
  if (M > 16) return true;  // stream_wide_kernel: K-outer chunks, the scale looked up per 16-byte load
  if (K > 4096) return false;
  if (format == FMT_INT4) return M <= 8 ? span <= 2 : span == 1;
  return span == 1;
}

// Launches fused_gemv_kernel for `tiles` 16-row tiles (defined with the kernels).
void launch_fused(const FusedParams &p, int format, bool scaled, bool ranked, int tiles, hipStream_t stream);

}  // namespace lb
