// C-ABI of the decode-step entry points (include/lowbit_decode_hip.h): validation and launches.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstring>
#include <map>
#include <vector>

#include "../../include/lowbit_decode_hip.h"
#include "abi_util.h"
#include "lb_decode.h"
#include "lb_layer.h"
#include "lb_line.h"
#include "lb_stream.h"

using namespace lb;
using namespace lb::abi;

namespace {

bool pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

int shift_of(int64_t group, int64_t K) {
  if (group == K) return 31;
  int sh = 0;
  while ((int64_t)1 << sh < group) ++sh;
  return sh;
}

size_t code_bytes(uint32_t format, int64_t N, int64_t K) {
  const int64_t count = N * K;
  return format == LB_FORMAT_FP16 ? (size_t)count * 2 : format == LB_FORMAT_INT8 ? (size_t)count : (size_t)(count + 1) / 2;
}

// Size of the argument struct before the workspace fields (callers built against it pass no workspace).
constexpr size_t kFusedArgsV1 = offsetof(lb_fused_linear_args, workspace);
constexpr size_t kAttnArgsV1 = offsetof(lb_decode_attention_args, workspace);

void *fused_workspace(const lb_fused_linear_args *a) {
  return a->struct_size >= sizeof(lb_fused_linear_args) ? a->workspace : nullptr;
}

lb_status check_fused(const lb_fused_linear_args *a) {
  if (!a) return fail(LB_INVALID_ARGUMENT, "lb_fused_linear: args is NULL");
  if (a->struct_size < kFusedArgsV1)
    return fail(LB_INVALID_ARGUMENT, "lb_fused_linear: struct_size %u < %zu", a->struct_size, kFusedArgsV1);
  if (a->format > LB_FORMAT_FP16) return fail(LB_INVALID_ARGUMENT, "lb_fused_linear: unknown format %u", a->format);
  if (a->K <= 0 || a->K % 32 != 0 || a->K > LB_FUSED_MAX_K)
    return fail(LB_INVALID_ARGUMENT, "lb_fused_linear: K=%lld must be a positive multiple of 32 <= %d",
                (long long)a->K, LB_FUSED_MAX_K);
  const bool dense = a->format == LB_FORMAT_FP16;
  if (!dense) {
    const int64_t g = a->group_size;
    if (!(g == a->K || (pow2(g) && g >= 32 && a->K % g == 0)))
      return fail(LB_INVALID_ARGUMENT, "lb_fused_linear: group_size %lld must be K or a power of two >= 32 dividing K",
                  (long long)g);
  }
  if (a->prologue > LB_PROLOGUE_SILU_MUL) return fail(LB_INVALID_ARGUMENT, "lb_fused_linear: unknown prologue %u", a->prologue);
  if (a->count < 1 || a->count > LB_FUSED_MAX_PROBLEMS)
    return fail(LB_INVALID_ARGUMENT, "lb_fused_linear: count %u outside 1..%d", a->count, LB_FUSED_MAX_PROBLEMS);
  if (!a->x || !aligned(a->x, 16)) return fail(LB_INVALID_ARGUMENT, "lb_fused_linear: x must be non-NULL and 16-byte aligned");
  if (a->prologue == LB_PROLOGUE_SILU_MUL && (!a->x2 || !aligned(a->x2, 16)))
    return fail(LB_INVALID_ARGUMENT, "lb_fused_linear: SILU_MUL needs a 16-byte aligned x2");
  if (a->prologue == LB_PROLOGUE_RMSNORM && (!a->gamma || !aligned(a->gamma, 16) || !std::isfinite(a->eps) || a->eps < 0))
    return fail(LB_INVALID_ARGUMENT, "lb_fused_linear: RMSNORM needs a 16-byte aligned gamma and a finite eps >= 0");

  const size_t kb = (size_t)a->K * 2;
  Range in[4 + 6 * LB_FUSED_MAX_PROBLEMS + 1];
  int nin = 0;
  in[nin++] = range_of(a->x, kb, "x");
  in[nin++] = range_of(a->prologue == LB_PROLOGUE_SILU_MUL ? a->x2 : nullptr, a->prologue == LB_PROLOGUE_SILU_MUL ? kb : 0, "x2");
  in[nin++] = range_of(a->prologue == LB_PROLOGUE_RMSNORM ? a->gamma : nullptr, a->prologue == LB_PROLOGUE_RMSNORM ? kb : 0, "gamma");
  int64_t tiles = 0;
  for (uint32_t i = 0; i < a->count; ++i) {
    const lb_fused_problem &q = a->problems[i];
    if (q.N <= 0 || q.N > ((int64_t)1 << 30))
      return fail(LB_INVALID_ARGUMENT, "lb_fused_linear: problem %u: N=%lld outside 1..2^30", i, (long long)q.N);
    if (!q.codes || !aligned(q.codes, 16) || !q.y || !aligned(q.y, 2) || (!dense && (!q.scales || !aligned(q.scales, 2))))
      return fail(LB_INVALID_ARGUMENT,
                  "lb_fused_linear: problem %u: codes (16-byte aligned), scales and y (2-byte aligned) required", i);
    if ((q.bias && !aligned(q.bias, 2)) || (q.residual && !aligned(q.residual, 2)))
      return fail(LB_INVALID_ARGUMENT, "lb_fused_linear: problem %u: bias/residual must be 2-byte aligned", i);
    if (q.rank < 0 || q.rank > LB_FUSED_MAX_RANK || q.rank > std::min(q.N, a->K))
      return fail(LB_INVALID_ARGUMENT, "lb_fused_linear: problem %u: rank %lld outside 0..%d", i, (long long)q.rank,
                  LB_FUSED_MAX_RANK);
    if (q.rank > 0 && (!q.down || !q.up || !aligned(q.down, 16) || !aligned(q.up, 16) || q.up_ld < q.rank ||
                       q.up_ld % 8 != 0))
      return fail(LB_INVALID_ARGUMENT,
                  "lb_fused_linear: problem %u: correction needs 16-byte aligned down/up and up_ld %% 8 == 0, >= rank", i);
    tiles += (q.N + 15) / 16;
    const int64_t G = dense ? 1 : a->K / a->group_size;
    in[nin++] = range_of(q.codes, code_bytes(a->format, q.N, a->K), "codes");
    in[nin++] = range_of(dense ? nullptr : q.scales, dense ? 0 : (size_t)(q.N * G * 2), "scales");
    in[nin++] = range_of(q.bias, q.bias ? (size_t)q.N * 2 : 0, "bias");
    in[nin++] = range_of(q.rank ? q.down : nullptr, q.rank ? (size_t)(q.rank * a->K * 2) : 0, "down");
    in[nin++] = range_of(q.rank ? q.up : nullptr, q.rank ? (size_t)((q.N - 1) * q.up_ld + q.rank) * 2 : 0, "up");
    in[nin++] = range_of(q.residual != q.y ? q.residual : nullptr, q.residual && q.residual != q.y ? (size_t)q.N * 2 : 0,
                         "residual");
  }
  if (tiles > INT32_MAX) return fail(LB_UNSUPPORTED, "lb_fused_linear: too many rows");
  void *ws = fused_workspace(a);
  if (ws || (a->struct_size >= sizeof(lb_fused_linear_args) && a->workspace_bytes)) {
    if (!ws || !aligned(ws, 256) || a->workspace_bytes < LB_FUSED_WORKSPACE_BYTES)
      return fail(LB_INVALID_ARGUMENT, "lb_fused_linear: workspace must be 256-byte aligned with %d bytes",
                  LB_FUSED_WORKSPACE_BYTES);
    in[nin++] = range_of(ws, LB_FUSED_WORKSPACE_BYTES, "workspace");
    for (int r = 0; r + 1 < nin; ++r)
      if (overlaps(in[nin - 1], in[r])) return fail(LB_INVALID_ARGUMENT, "lb_fused_linear: workspace overlaps %s", in[r].name);
  }
  for (uint32_t i = 0; i < a->count; ++i) {
    const Range y = range_of(a->problems[i].y, (size_t)a->problems[i].N * 2, "y");
    for (int r = 0; r < nin; ++r)
      if (overlaps(y, in[r])) return fail(LB_INVALID_ARGUMENT, "lb_fused_linear: y of problem %u overlaps %s", i, in[r].name);
    for (uint32_t k = i + 1; k < a->count; ++k)
      if (overlaps(y, range_of(a->problems[k].y, (size_t)a->problems[k].N * 2, "y")))
        return fail(LB_INVALID_ARGUMENT, "lb_fused_linear: outputs of problems %u and %u overlap", i, k);
  }
  return ok();
}

// The kernel parameters of a checked lb_fused_linear call (no shared-z workspace) and its tiles.
FusedParams fused_params(const lb_fused_linear_args *a, int *tiles_out) {
  FusedParams p{};
  const bool dense = a->format == LB_FORMAT_FP16;
  p.x = static_cast<const f16 *>(a->x);
  p.x2 = static_cast<const f16 *>(a->x2);
  p.gamma = static_cast<const f16 *>(a->gamma);
  p.eps = a->eps;
  p.K = (int)a->K;
  const int64_t group = dense ? a->K : a->group_size;
  p.G = (int)(a->K / group);
  p.group_shift = shift_of(group, a->K);
  p.per_row = a->format == LB_FORMAT_INT8 && group == a->K;
  p.prologue = (int)a->prologue;
  int tiles = 0;
  for (int i = 0; i < LB_FUSED_MAX_PROBLEMS; ++i) {
    FusedProblem &q = p.prob[i];
    if (i < (int)a->count) {
      const lb_fused_problem &s = a->problems[i];
      q.codes = static_cast<const uint8_t *>(s.codes);
      q.scales = static_cast<const f16 *>(s.scales);
      q.y = static_cast<f16 *>(s.y);
      q.bias = static_cast<const f16 *>(s.bias);
      q.residual = static_cast<const f16 *>(s.residual);
      q.rank = (int)s.rank;
      q.down = s.rank ? static_cast<const f16 *>(s.down) : nullptr;
      q.up = s.rank ? static_cast<const f16 *>(s.up) : nullptr;
      q.up_ld = (int)s.up_ld;
      q.N = (int)s.N;
      tiles += (int)((s.N + 15) / 16);
    }
    q.tiles_end = tiles;  // absent problems own no tiles
  }
  *tiles_out = tiles;
  return p;
}

template <int FMT, bool SCALED, int KMAX, bool RANKED>
void launch_fused_k(const FusedParams &p, int tiles, hipStream_t s) {
  if constexpr (RANKED) {
    if (p.zblocks > 0) {  // z workgroups first: dispatched ahead of every tile workgroup that waits for them
      hipLaunchKernelGGL((fused_gemv_kernel<FMT, SCALED, KMAX, true, true>), dim3(p.zblocks + tiles), dim3(256), 0,
                         s, p);
      return;
    }
  }
  hipLaunchKernelGGL((fused_gemv_kernel<FMT, SCALED, KMAX, RANKED>), dim3(tiles), dim3(256), 0, s, p);
}

// The shortest staged row that holds K: 640 and 1536 (decode shapes), then 4096 / 8192 / 16384
// for one-row calls without a correction, up to the format's limit.
template <int FMT, bool SCALED, bool RANKED>
void launch_fused_r(const FusedParams &p, int tiles, hipStream_t s) {
  constexpr int LIMIT = fused_kmax_limit(FMT);
  if (p.K <= 640) return launch_fused_k<FMT, SCALED, 640, RANKED>(p, tiles, s);
  if (p.K <= kFusedMaxK || RANKED) return launch_fused_k<FMT, SCALED, kFusedMaxK, RANKED>(p, tiles, s);
  if constexpr (!RANKED) {
    if (p.K <= 4096) return launch_fused_k<FMT, SCALED, 4096, false>(p, tiles, s);
    if constexpr (LIMIT >= 8192) {
      if (p.K <= 8192) return launch_fused_k<FMT, SCALED, 8192, false>(p, tiles, s);
    }
    if constexpr (LIMIT >= 16384) return launch_fused_k<FMT, SCALED, 16384, false>(p, tiles, s);
  }
}

#ifndef LB_ROWS_MIN_WGS
#define LB_ROWS_MIN_WGS 512  // rows_gemv_kernel only when it still gives this many workgroups
#endif

template <int FMT, bool SCALED, int KMAX, int RG>
bool launch_rows_k(const FusedParams &p, int tiles, hipStream_t s) {
  constexpr int WSTEP = (4 / RG) * 4 * FormatTraits<FMT>::CPL;
  if constexpr ((KMAX + WSTEP - 1) / WSTEP <= 32) {  // all of a lane's loads fit in registers
    const f16 *aux = p.prologue == PRO_SILU_MUL ? p.x2 : p.gamma;
    hipLaunchKernelGGL((rows_gemv_kernel<FMT, SCALED, KMAX, RG, false>), dim3((tiles + RG - 1) / RG), dim3(256), 0, s,
                       p.prob[0].codes, p.x, p.prob[0].scales, aux, p.prob[0].N, p.K, p.G, p.prologue, p.group_shift, p,
                       HeadNextParams{});
    return true;
  }
  return false;
}

// lb_head_next: rows_gemv_kernel with four tiles per workgroup and the greedy tail (fp16 rows of
// up to 640, INT4 rows of up to 1536; false: not available).
template <int FMT, bool SCALED>
bool launch_head_next_f(const FusedParams &p, const HeadNextParams &hn, int wgs, hipStream_t s) {
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(wgs), dim3(256), 0, s, p.prob[0].codes, p.x, p.prob[0].scales, p.gamma,
                       p.prob[0].N, p.K, p.G, p.prologue, p.group_shift, p, hn);
  };
  if (p.K <= 640) {
    go(rows_gemv_kernel<FMT, SCALED, 640, 4, true>);
    return true;
  }
  if constexpr (FMT == FMT_INT4) {
    go(rows_gemv_kernel<FMT, SCALED, 1536, 4, true>);
    return true;
  }
  return false;
}

// RG tiles per workgroup for the shortest staged row that holds K (false: not available).  Used
// for int4 and fp16 rows of up to 1536 k, where it measured faster than the single-tile kernel
// (int8 and nf4 weights, and longer rows whose loads no longer fit in few registers, did not).
template <int FMT, bool SCALED, int RG>
bool launch_rows(const FusedParams &p, int tiles, hipStream_t s) {
  if constexpr (FMT == FMT_INT8 || FMT == FMT_NF4) return false;
  if (p.K <= 640) return launch_rows_k<FMT, SCALED, 640, RG>(p, tiles, s);
  if (p.K <= 1536) return launch_rows_k<FMT, SCALED, 1536, RG>(p, tiles, s);
  return false;
}

// One tile per workgroup (the four waves split K): the single-tile kernel's arithmetic in the same
// order, with its first loads' operands preloaded, for one problem without a correction.
template <int FMT, bool SCALED>
bool launch_rows1(const FusedParams &p, int tiles, hipStream_t s) {
  constexpr int LIMIT = fused_kmax_limit(FMT);
  if (p.K <= 640) return launch_rows_k<FMT, SCALED, 640, 1>(p, tiles, s);
  if (p.K <= kFusedMaxK) return launch_rows_k<FMT, SCALED, kFusedMaxK, 1>(p, tiles, s);
  if (p.K <= 4096) return launch_rows_k<FMT, SCALED, 4096, 1>(p, tiles, s);
  if constexpr (LIMIT >= 8192) {
    if (p.K <= 8192) return launch_rows_k<FMT, SCALED, 8192, 1>(p, tiles, s);
  }
  if constexpr (LIMIT >= 16384) return launch_rows_k<FMT, SCALED, 16384, 1>(p, tiles, s);
  return false;
}

// stream_gemv_kernel takes one-row INT4 calls with rows longer than LB_STREAM_MIN_K or at least
// LB_STREAM_MIN_BYTES of weights, and INT8 rows longer than the single-tile kernel holds (measured
// on MI355X: otherwise the single-tile kernels, whose workgroups issue every load at once, finish
// first).
#ifndef LB_STREAM_MIN_BYTES
#define LB_STREAM_MIN_BYTES (64ll << 20)
#endif
#ifndef LB_STREAM_MIN_K
#define LB_STREAM_MIN_K 4096
#endif
#ifndef LB_STREAM_WGS_PER_CU
#define LB_STREAM_WGS_PER_CU 4         // persistent workgroups per CU
#endif
#ifndef LB_STREAM_SPLIT_TILES_PER_CU
#define LB_STREAM_SPLIT_TILES_PER_CU 4 // below this many 16-row tiles per CU, split K over the 4 waves
#endif
#ifndef LB_STREAM_PD
#define LB_STREAM_PD 2                 // chunks in flight per wave
#endif
#ifndef LB_STREAM_CH
#define LB_STREAM_CH 8                 // 16-byte loads per lane per chunk (rows longer than 640 codes)
#endif

// Compute units of the current device (cached per device ordinal).
int device_cus() {
  static int cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    cache[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
  }
  return cache[dev];
}

// Waves per persistent workgroup: more rows stage more LDS (fewer workgroups per CU), so their
// workgroups are wider to keep about sixteen waves of loads in flight per CU.
template <int MP, int KSPLIT>
constexpr int stream_waves() { return KSPLIT == 4 || MP <= 4 ? 4 : MP == 8 ? 8 : 16; }

template <int FMT, bool SCALED, int NS, int KMAX, int KSPLIT, int MP>
void launch_stream_k(const StreamParams &p, int grid, hipStream_t s) {
  constexpr int CH = KMAX <= 640 ? (FMT == FMT_INT4 ? 5 : 10) : MP == 1 ? LB_STREAM_CH : 8;
  constexpr int WAVES = stream_waves<MP, KSPLIT>();
  hipLaunchKernelGGL((stream_gemv_kernel<FMT, SCALED, NS, KMAX, CH, LB_STREAM_PD, KSPLIT, MP, WAVES>), dim3(grid),
                     dim3(64 * WAVES), 0, s, p);
}

// LDS bytes of one stream_gemv_kernel workgroup (activation rows, zero region, block sums).
constexpr int stream_lds_bytes(int mp, int kp, int cpl) { return (mp + 1) * kp * 2 + mp * (kp / cpl + 16) * 4; }

// Launch mode and staged length for MP activation rows: K split over one workgroup's waves when
// there are few tiles per CU (and K spans at least 4 chunks), else persistent workgroups.
template <int FMT, bool SCALED, int NS, int MP>
void launch_stream_m(StreamParams p, hipStream_t s) {
  constexpr int CPL = StreamTraits<FMT>::CPL, CPW = 4 * CPL;
  const int cus = device_cus();
  const int kmax = MP > 1 ? 4096 : p.K <= 640 ? 640 : p.K <= 4096 ? 4096 : 16384;
  const int ch = kmax <= 640 ? (FMT == FMT_INT4 ? 5 : 10) : MP == 1 ? LB_STREAM_CH : 8;
  p.chunks = (p.K + ch * CPW - 1) / (ch * CPW);
  if constexpr (MP <= 4) {  // more rows stage too much per workgroup for one tile each
    if (kmax > 640 && p.chunks >= 4 && p.tiles < LB_STREAM_SPLIT_TILES_PER_CU * cus) {
      if (kmax == 4096) launch_stream_k<FMT, SCALED, NS, 4096, 4, MP>(p, p.tiles, s);
      else if constexpr (MP == 1) launch_stream_k<FMT, SCALED, NS, 16384, 4, MP>(p, p.tiles, s);
      return;
    }
  }
  constexpr int WAVES = stream_waves<MP, 1>();
  const int per_cu = std::max(1, std::min(LB_STREAM_WGS_PER_CU * 4 / WAVES, (160 * 1024) / stream_lds_bytes(MP, kmax, CPL)));
  const int grid = std::max(1, std::min((p.tiles + WAVES - 1) / WAVES, cus * per_cu));
  if constexpr (MP == 1) {
    if (kmax == 640) return launch_stream_k<FMT, SCALED, NS, 640, 1, MP>(p, grid, s);
    if (kmax == 16384) return launch_stream_k<FMT, SCALED, NS, 16384, 1, MP>(p, grid, s);
  }
  launch_stream_k<FMT, SCALED, NS, 4096, 1, MP>(p, grid, s);
}

// Activation rows -> MP (the instantiated group spans: any for one row; INT4 up to two groups per
// load for MP <= 8 and one for MP = 16; INT8 groups one per load for MP > 1).
template <int FMT, bool SCALED, int NS>
void launch_stream_ns(const StreamParams &p, hipStream_t s) {
  if (p.M == 1) return launch_stream_m<FMT, SCALED, NS, 1>(p, s);
  if constexpr (NS <= 2 && (FMT == FMT_INT4 || NS == 1)) {
    if (p.M == 2) return launch_stream_m<FMT, SCALED, NS, 2>(p, s);
    if (p.M <= 4) return launch_stream_m<FMT, SCALED, NS, 4>(p, s);
    if (p.M <= 8) return launch_stream_m<FMT, SCALED, NS, 8>(p, s);
    if constexpr (NS == 1) return launch_stream_m<FMT, SCALED, NS, 16>(p, s);
  }
}

template <int FMT, bool SCALED>
void launch_stream_f(const StreamParams &p, int ns, hipStream_t s) {
  if constexpr (!SCALED) {
    launch_stream_ns<FMT, false, 1>(p, s);
  } else {
    if (ns == 1) launch_stream_ns<FMT, true, 1>(p, s);
    else if (ns == 2) launch_stream_ns<FMT, true, 2>(p, s);
    else launch_stream_ns<FMT, true, 4>(p, s);
  }
}

// One problem, one activation row, no prologue or correction, INT4 / INT8 codes with groups that
// stream_gemv_kernel handles (a 4*CPL-code load spans 1, 2 or 4 whole groups), K <= 16384, long
// rows or many weights (above): launched there (false otherwise).
template <int FMT, bool SCALED>
bool try_stream(const FusedParams &p, int tiles, hipStream_t s) {
  if constexpr (FMT != FMT_INT4 && FMT != FMT_INT8) {
    return false;
  } else {
    const FusedProblem &q = p.prob[0];
    if (p.prologue != PRO_NONE || q.rank > 0) return false;
    const int ns = stream_group_span(FMT, p.K, SCALED ? p.K / p.G : p.K);
    if (ns == 0) return false;
    const int64_t weight_bytes = (int64_t)q.N * p.K * StreamTraits<FMT>::BITS / 8;
    // INT8 rows the single-tile kernel holds stay there (it measured faster at every size).
    if (!p.force_stream && p.K <= fused_kmax_limit(FMT) &&
        (FMT == FMT_INT8 || (weight_bytes < LB_STREAM_MIN_BYTES && p.K <= LB_STREAM_MIN_K)))
      return false;
    StreamParams sp{};
    sp.x = p.x;
    sp.codes = q.codes;
    sp.scales = q.scales;
    sp.y = q.y;
    sp.bias = q.bias;
    sp.residual = q.residual;
    sp.M = 1;
    sp.N = q.N;
    sp.K = p.K;
    sp.G = p.G;
    sp.group_shift = p.group_shift;
    sp.ldx = p.K;
    sp.ldy = q.N;
    sp.tiles = tiles;
    launch_stream_f<FMT, SCALED>(sp, ns, s);
    return true;
  }
}

#ifndef LB_LINE_WAVES
#define LB_LINE_WAVES 4  // waves per line_gemv_kernel workgroup: whole row groups of every segment
#endif
#ifndef LB_LINE_FEW_SEGMENTS
#define LB_LINE_FEW_SEGMENTS 4  // rows of at most this many segments: 4 rows per wave (more waves), else 8
#endif

// One problem, one activation row, no prologue or correction, INT4 / INT8 / NF4 codes whose 16-byte lane
// loads each lie in one group (one group per row, or power-of-two groups of at least CPL codes),
// rows of at least one segment (64 lanes x CPL codes) and at most 16: launched in line_gemv_kernel,
// which measured faster than the single-tile, multi-tile and streaming kernels on every such
// shape (MI355X, one-row INT4 g128 and INT8 per-row GEMVs of 1024-128256 rows, K = 2048-14336).
template <int FMT, bool SCALED>
bool try_line(const FusedParams &p, hipStream_t s) {
  if constexpr (FMT != FMT_INT4 && FMT != FMT_INT8 && FMT != FMT_NF4) {
    return false;
  } else {
    constexpr int CPL = LineTraits<FMT>::CPL, SEG = 64 * CPL;
    const FusedProblem &q = p.prob[0];
    if (p.force_stream || p.prologue != PRO_NONE || q.rank > 0 || p.G <= 0 || p.K % p.G != 0) return false;
    const int group = p.K / p.G;
    // NF4 lanes hold the INT4 lane's 32 codes, so the same group spans apply.
    if (p.K < SEG || p.K > kLineMaxWaves * SEG || stream_group_span(FMT == FMT_NF4 ? FMT_INT4 : FMT, p.K, group) == 0 ||
        (group != p.K && group < CPL) || !aligned(q.codes, 16) || !aligned(p.x, 16))
      return false;
    const int nseg = (p.K + SEG - 1) / SEG;
    const int groups = std::max(1, std::min(LB_LINE_WAVES, kLineMaxWaves) / nseg);  // row groups per workgroup
    const int R = nseg <= LB_LINE_FEW_SEGMENTS ? 4 : 8;
    const int rows_wg = groups * R;
    StreamParams sp{};
    sp.y = q.y;
    sp.bias = q.bias;
    sp.residual = q.residual;
    sp.M = 1;
    sp.N = q.N;
    sp.K = p.K;
    sp.G = p.G;
    sp.group_shift = p.group_shift;
    const dim3 grid((q.N + rows_wg - 1) / rows_wg), block(64 * nseg * groups);
    const bool qs = SCALED && group >= 4 * CPL;
    if (R == 4 && qs)
      hipLaunchKernelGGL((line_gemv_kernel<FMT, SCALED, 4, true>), grid, block, 0, s, p.x, q.codes, q.scales, q.N, p.K, p.G,
                         p.group_shift, nseg, groups, sp);
    else if (R == 4)
      hipLaunchKernelGGL((line_gemv_kernel<FMT, SCALED, 4, false>), grid, block, 0, s, p.x, q.codes, q.scales, q.N, p.K,
                         p.G, p.group_shift, nseg, groups, sp);
    else if (qs)
      hipLaunchKernelGGL((line_gemv_kernel<FMT, SCALED, 8, true>), grid, block, 0, s, p.x, q.codes, q.scales, q.N, p.K, p.G,
                         p.group_shift, nseg, groups, sp);
    else
      hipLaunchKernelGGL((line_gemv_kernel<FMT, SCALED, 8, false>), grid, block, 0, s, p.x, q.codes, q.scales, q.N, p.K,
                         p.G, p.group_shift, nseg, groups, sp);
    return true;
  }
}

#ifndef LB_PACK_MIN_ROWS
#define LB_PACK_MIN_ROWS 16384  // INT8: rows (over the problems) from which pack_gemv_kernel takes the call
#endif
#ifndef LB_PACK_ROWS
#define LB_PACK_ROWS 4  // wave-wide loads per pack_gemv_kernel wave from LB_PACK_MIN_ROWS rows on
#endif
#ifndef LB_PACK_SMALL
#define LB_PACK_SMALL 1  // INT4 below LB_PACK_MIN_ROWS rows: pack_gemv_kernel with one load per wave
#endif

template <int FMT, bool SCALED, int R, int NP>
void launch_pack(const FusedParams &p, const PackTable &tab, int waves, bool epi, hipStream_t s) {
  const FusedProblem &q = p.prob[0];
  StreamParams sp{};
  sp.y = q.y;
  sp.bias = q.bias;
  sp.residual = q.residual;
  sp.M = 1;
  sp.N = q.N;
  sp.K = p.K;
  sp.G = p.G;
  sp.group_shift = p.group_shift;
  const dim3 grid((waves + 3) / 4), block(256);
  if (epi)
    hipLaunchKernelGGL((pack_gemv_kernel<FMT, SCALED, R, true, NP>), grid, block, 0, s, p.x, q.codes, q.scales, q.N, p.K,
                       p.G, p.group_shift, sp, tab);
  else
    hipLaunchKernelGGL((pack_gemv_kernel<FMT, SCALED, R, false, NP>), grid, block, 0, s, p.x, q.codes, q.scales, q.N,
                       p.K, p.G, p.group_shift, sp, tab);
}

// One activation row, no prologue or correction, INT4 / INT8 rows of 8 .. 63 16-byte slots
// (shorter than a line_gemv_kernel segment) whose lane loads each lie in one group, one to three
// problems: launched in pack_gemv_kernel (false otherwise).  Four loads per wave from
// LB_PACK_MIN_ROWS rows over the problems on; below that INT4 calls take one load per wave (more,
// shorter waves: the latency of one load and its sum is what such calls cost), INT8 calls decline.
template <int FMT, bool SCALED>
bool try_pack(const FusedParams &p, int tiles, hipStream_t s) {
  if constexpr (FMT != FMT_INT4 && FMT != FMT_INT8) {
    return false;
  } else {
    constexpr int CPL = LineTraits<FMT>::CPL;
    if (p.force_stream || p.prologue != PRO_NONE || p.G <= 0 || p.K % p.G != 0) return false;
    const int np = 1 + (p.prob[0].tiles_end < tiles) + (p.prob[1].tiles_end < tiles);
    const int group = p.K / p.G;
    const int row_bytes = p.K * LineTraits<FMT>::BITS / 8;
    const int slots = row_bytes / 16, per_load = slots > 0 ? 64 / slots : 0;
    if (row_bytes % 16 != 0 || slots < 8 || slots >= 64 || per_load * LB_PACK_ROWS > 64 ||
        stream_group_span(FMT, p.K, group) == 0 || (group != p.K && group < CPL) || !aligned(p.x, 16))
      return false;
    long long rows = 0;
    for (int j = 0; j < np; ++j) {
      const FusedProblem &q = p.prob[j];
      if (q.rank > 0 || q.N < 1 || !aligned(q.codes, 16)) return false;
      rows += q.N;
    }
    const bool big = rows >= LB_PACK_MIN_ROWS;
    if (!big && (FMT != FMT_INT4 || !LB_PACK_SMALL)) return false;
    const int R = big ? LB_PACK_ROWS : 1, per_wave = R * per_load;
    PackTable tab{};
    int waves = 0;
    bool epi = false;
    for (int j = 0; j < np; ++j) {
      const FusedProblem &q = p.prob[j];
      tab.codes[j] = q.codes;
      tab.scales[j] = q.scales;
      tab.y[j] = q.y;
      tab.bias[j] = q.bias;
      tab.residual[j] = q.residual;
      tab.N[j] = q.N;
      waves += (q.N + per_wave - 1) / per_wave;
      tab.wave_end[j] = waves;
      epi = epi || q.bias || q.residual;
    }
    for (int j = np; j < kPackMaxProblems; ++j) tab.wave_end[j] = waves;
    const bool r4 = R == LB_PACK_ROWS;
    switch (np) {
      case 1: r4 ? launch_pack<FMT, SCALED, LB_PACK_ROWS, 1>(p, tab, waves, epi, s)
                 : launch_pack<FMT, SCALED, 1, 1>(p, tab, waves, epi, s); break;
      case 2: r4 ? launch_pack<FMT, SCALED, LB_PACK_ROWS, 2>(p, tab, waves, epi, s)
                 : launch_pack<FMT, SCALED, 1, 2>(p, tab, waves, epi, s); break;
      default: r4 ? launch_pack<FMT, SCALED, LB_PACK_ROWS, 3>(p, tab, waves, epi, s)
                  : launch_pack<FMT, SCALED, 1, 3>(p, tab, waves, epi, s); break;
    }
    return true;
  }
}

// RANKED instantiations carry the correction (V and U loads); the others have none at all.  One
// problem without a correction over many rows runs with several tiles per workgroup, or, when it
// is long enough, in stream_gemv_kernel.
template <int FMT, bool SCALED>
void launch_fused_t(const FusedParams &p, int tiles, bool ranked, hipStream_t s) {
  if (!ranked && p.prob[0].tiles_end == tiles && try_line<FMT, SCALED>(p, s)) return;
  if (!ranked && try_pack<FMT, SCALED>(p, tiles, s)) return;
  if (!ranked && p.prob[0].tiles_end == tiles && try_stream<FMT, SCALED>(p, tiles, s)) return;
  if (!ranked && p.prob[0].tiles_end == tiles) {
    if (tiles / 4 >= LB_ROWS_MIN_WGS && launch_rows<FMT, SCALED, 4>(p, tiles, s)) return;
    if (tiles / 2 >= LB_ROWS_MIN_WGS && launch_rows<FMT, SCALED, 2>(p, tiles, s)) return;
    if (launch_rows1<FMT, SCALED>(p, tiles, s)) return;
  }
  ranked ? launch_fused_r<FMT, SCALED, true>(p, tiles, s) : launch_fused_r<FMT, SCALED, false>(p, tiles, s);
}


}  // namespace

namespace lb {
#ifndef LB_STREAM_ROWS_CH
#define LB_STREAM_ROWS_CH 8  // 16-byte loads per lane per chunk of stream_rows_kernel
#endif

// stream_rows_kernel with the staged row length for K (smaller rows leave LDS for more
// workgroups per CU; a workgroup that fills the CU's LDS alone has sixteen waves).
template <int FMT, bool SCALED, int MP, int KMAX>
void launch_stream_rows_k(const StreamParams &p0, hipStream_t s) {
  constexpr int CH = LB_STREAM_ROWS_CH, PD = 2;
  constexpr int KC = CH * 4 * FormatTraits<FMT>::CPL;
  constexpr int KP = (KMAX + KC - 1) / KC * KC;
  constexpr int LDS = (MP + 1) * KP * 2 + (FMT == FMT_NF4 ? 1024 : 0);
  constexpr int PER_CU = 163840 / LDS < 1 ? 1 : (163840 / LDS > 4 ? 4 : 163840 / LDS);
  constexpr int WAVES = PER_CU == 1 ? 16 : 8;
  StreamParams p = p0;
  p.chunks = (p.K + KC - 1) / KC;
  const int grid = std::min((p.tiles + WAVES - 1) / WAVES, device_cus() * PER_CU);
  hipLaunchKernelGGL((stream_rows_kernel<FMT, SCALED, MP, KMAX, CH, PD, WAVES>), dim3(grid), dim3(64 * WAVES), 0, s, p);
}

template <int FMT, bool SCALED, int MP>
void launch_stream_rows_mp(const StreamParams &p, hipStream_t s) {
  if (p.K <= 1024) launch_stream_rows_k<FMT, SCALED, MP, 1024>(p, s);
  else if (p.K <= 2048) launch_stream_rows_k<FMT, SCALED, MP, 2048>(p, s);
  else launch_stream_rows_k<FMT, SCALED, MP, 4096>(p, s);
}

template <int FMT, bool SCALED>
void launch_stream_rows_f(const StreamParams &p, hipStream_t s) {
  if (p.M <= 8) launch_stream_rows_mp<FMT, SCALED, 8>(p, s);
  else launch_stream_rows_mp<FMT, SCALED, 16>(p, s);
}

void launch_stream_rows(const StreamParams &p, int format, bool scaled, hipStream_t s) {
  if (format == FMT_INT4) launch_stream_rows_f<FMT_INT4, true>(p, s);
  else if (format == FMT_NF4) launch_stream_rows_f<FMT_NF4, true>(p, s);
  else if (scaled) launch_stream_rows_f<FMT_INT8, true>(p, s);
  else launch_stream_rows_f<FMT_INT8, false>(p, s);
}

#ifndef LB_STREAM_WIDE_TPW
#define LB_STREAM_WIDE_TPW 1  // 16-row tiles per wave of stream_wide_kernel
#endif
#ifndef LB_STREAM_WIDE_WAVES
#define LB_STREAM_WIDE_WAVES 8  // waves per workgroup of stream_wide_kernel
#endif

// stream_wide_kernel: chunks of four 16-byte loads per lane per tile.
template <int FMT, bool SCALED>
void launch_stream_wide_f(const StreamParams &p0, hipStream_t s) {
  constexpr int KC = 4 * 4 * FormatTraits<FMT>::CPL;
  constexpr int TPW = LB_STREAM_WIDE_TPW, WAVES = LB_STREAM_WIDE_WAVES;
  StreamParams p = p0;
  p.chunks = (p.K + KC - 1) / KC;
  const int grid = (p.tiles + WAVES * TPW - 1) / (WAVES * TPW);
  hipLaunchKernelGGL((stream_wide_kernel<FMT, SCALED, KC, TPW, WAVES>), dim3(grid), dim3(64 * WAVES), 0, s, p);
}

void launch_stream_wide(const StreamParams &p, int format, bool scaled, hipStream_t s) {
  if (format == FMT_INT4) launch_stream_wide_f<FMT_INT4, true>(p, s);
  else if (format == FMT_NF4) launch_stream_wide_f<FMT_NF4, true>(p, s);
  else if (scaled) launch_stream_wide_f<FMT_INT8, true>(p, s);
  else launch_stream_wide_f<FMT_INT8, false>(p, s);
}

// tile_rows_kernel: TT 16-row tiles per workgroup, the staged row length for K (or the slice).
template <int FMT, bool SCALED, int MP, int TT>
void launch_tile_rows_tt(const StreamParams &p, hipStream_t s) {
  const int slices = p.kslice > 0 ? p.K / p.kslice : 1;
  const dim3 grid(((p.N + 15) / 16 + TT - 1) / TT, slices), block(256 * TT);
#define LB_TILE_ROWS_ARGS p.codes, p.x, p.scales, p.bias, p.M, p.N, p.K, p.G, p.ldx, p
  if constexpr (MP == 32) {  // staged rows of up to 1024 codes (33 rows of them fill the LDS budget)
    if (slices > 1)
      hipLaunchKernelGGL((tile_rows_kernel<FMT, SCALED, 1024, MP, TT, true>), grid, block, 0, s, LB_TILE_ROWS_ARGS);
    else if (p.K <= 640)
      hipLaunchKernelGGL((tile_rows_kernel<FMT, SCALED, 640, MP, TT, false>), grid, block, 0, s, LB_TILE_ROWS_ARGS);
    else
      hipLaunchKernelGGL((tile_rows_kernel<FMT, SCALED, 1024, MP, TT, false>), grid, block, 0, s, LB_TILE_ROWS_ARGS);
  } else if (slices > 1) {
    if (MP == 16 || p.kslice <= 2048)
      hipLaunchKernelGGL((tile_rows_kernel<FMT, SCALED, 2048, MP, TT, true>), grid, block, 0, s, LB_TILE_ROWS_ARGS);
    else if constexpr (MP < 16)
      hipLaunchKernelGGL((tile_rows_kernel<FMT, SCALED, 4096, MP, TT, true>), grid, block, 0, s, LB_TILE_ROWS_ARGS);
  } else if (p.K <= 640) {
    hipLaunchKernelGGL((tile_rows_kernel<FMT, SCALED, 640, MP, TT, false>), grid, block, 0, s, LB_TILE_ROWS_ARGS);
  } else if (MP == 16 || p.K <= 2048) {
    hipLaunchKernelGGL((tile_rows_kernel<FMT, SCALED, 2048, MP, TT, false>), grid, block, 0, s, LB_TILE_ROWS_ARGS);
  } else if constexpr (MP < 16) {
    hipLaunchKernelGGL((tile_rows_kernel<FMT, SCALED, 4096, MP, TT, false>), grid, block, 0, s, LB_TILE_ROWS_ARGS);
  }
#undef LB_TILE_ROWS_ARGS
}

template <int FMT, bool SCALED, int MP>
void launch_tile_rows_mp(const StreamParams &p, hipStream_t s) {
  const int slices = p.kslice > 0 ? p.K / p.kslice : 1;
  const int tt = tile_rows_per_wg((long long)(p.N + 15) / 16 * slices, p.kslice > 0 ? p.kslice : p.K, p.M);
  if (tt == 4) launch_tile_rows_tt<FMT, SCALED, MP, 4>(p, s);
  else if (tt == 2) launch_tile_rows_tt<FMT, SCALED, MP, 2>(p, s);
  else launch_tile_rows_tt<FMT, SCALED, MP, 1>(p, s);
}

template <int FMT, bool SCALED>
void launch_tile_rows_f(const StreamParams &p, hipStream_t s) {
  if (p.M <= 4) launch_tile_rows_mp<FMT, SCALED, 4>(p, s);
  else if (p.M <= 8) launch_tile_rows_mp<FMT, SCALED, 8>(p, s);
  else if (p.M <= 16) launch_tile_rows_mp<FMT, SCALED, 16>(p, s);
  else launch_tile_rows_mp<FMT, SCALED, 32>(p, s);
}

void launch_tile_rows(const StreamParams &p, int format, bool scaled, hipStream_t s) {
  if (format == FMT_INT4) launch_tile_rows_f<FMT_INT4, true>(p, s);
  else if (format == FMT_NF4) launch_tile_rows_f<FMT_NF4, true>(p, s);
  else if (scaled) launch_tile_rows_f<FMT_INT8, true>(p, s);
  else launch_tile_rows_f<FMT_INT8, false>(p, s);
}

void launch_stream(const StreamParams &p, int format, bool scaled, int ns, hipStream_t s) {
  if (format == FMT_INT4) launch_stream_f<FMT_INT4, true>(p, ns, s);
  else if (scaled) launch_stream_f<FMT_INT8, true>(p, ns, s);
  else launch_stream_f<FMT_INT8, false>(p, ns, s);
}

void launch_fused(const FusedParams &p, int format, bool scaled, bool ranked, int tiles, hipStream_t s) {
  switch (format) {
    case FMT_INT8:
      scaled ? launch_fused_t<FMT_INT8, true>(p, tiles, ranked, s) : launch_fused_t<FMT_INT8, false>(p, tiles, ranked, s);
      break;
    case FMT_INT4: launch_fused_t<FMT_INT4, true>(p, tiles, ranked, s); break;
    case FMT_NF4: launch_fused_t<FMT_NF4, true>(p, tiles, ranked, s); break;
    default: launch_fused_t<FMT_FP16, false>(p, tiles, ranked, s); break;
  }
}
}  // namespace lb

extern "C" {

lb_status lb_fused_linear(const lb_fused_linear_args *a, void *stream) {
  if (const lb_status bad = refuse_if_failed("lb_fused_linear"); bad != LB_OK) return bad;
  const lb_status st = check_fused(a);
  if (st != LB_OK) return st;
  int tiles = 0;
  FusedParams p = fused_params(a, &tiles);
  const bool dense = a->format == LB_FORMAT_FP16;
  bool ranked = false;
  for (uint32_t i = 0; i < a->count; ++i) ranked = ranked || a->problems[i].rank > 0;
  void *ws = fused_workspace(a);
  if (ranked && ws) {
    int zb = 0;
    for (int i = 0; i < LB_FUSED_MAX_PROBLEMS; ++i) {
      if (i < (int)a->count) zb += (int)((a->problems[i].rank + kFusedZRanks - 1) / kFusedZRanks);
      p.prob[i].zend = zb;
    }
    p.zblocks = zb;
    p.zslot = static_cast<uint64_t *>(ws);
  }
  launch_fused(p, (int)a->format, !dense && !p.per_row, ranked, tiles, static_cast<hipStream_t>(stream));
  return launch_status("lb_fused_linear");
}

lb_status lb_decode_attention(const lb_decode_attention_args *a, void *stream) {
  if (const lb_status bad = refuse_if_failed("lb_decode_attention"); bad != LB_OK) return bad;
  if (!a) return fail(LB_INVALID_ARGUMENT, "lb_decode_attention: args is NULL");
  if (a->struct_size < kAttnArgsV1)
    return fail(LB_INVALID_ARGUMENT, "lb_decode_attention: struct_size %u < %zu", a->struct_size, kAttnArgsV1);
  if (a->head_dim != kHeadDim) return fail(LB_UNSUPPORTED, "lb_decode_attention: head_dim must be %d", kHeadDim);
  if (a->heads < 1 || a->kv_heads < 1 || a->heads % a->kv_heads != 0 || a->heads > 1024)
    return fail(LB_INVALID_ARGUMENT, "lb_decode_attention: heads must be a multiple of kv_heads (<= 1024)");
  if (a->capacity < 1 || a->capacity > 4096)
    return fail(LB_INVALID_ARGUMENT, "lb_decode_attention: capacity %lld outside 1..4096", (long long)a->capacity);
  if (!a->q || !a->k || !a->v || !a->cos || !a->sin || !a->position || !a->keys || !a->values || !a->out)
    return fail(LB_INVALID_ARGUMENT, "lb_decode_attention: NULL pointer");
  if (!aligned(a->q, 2) || !aligned(a->k, 2) || !aligned(a->v, 2) || !aligned(a->cos, 2) || !aligned(a->sin, 2) ||
      !aligned(a->out, 2) || !aligned(a->position, 8) || !aligned(a->keys, 16) || !aligned(a->values, 16))
    return fail(LB_INVALID_ARGUMENT, "lb_decode_attention: misaligned buffer (keys/values need 16 bytes)");
  if (!std::isfinite(a->scale)) return fail(LB_INVALID_ARGUMENT, "lb_decode_attention: scale must be finite");
  const size_t row = kHeadDim * 2;
  const size_t cache = (size_t)a->kv_heads * a->capacity * row;
  const Range keys = range_of(a->keys, cache, "keys"), values = range_of(a->values, cache, "values");
  const Range out = range_of(a->out, (size_t)a->heads * row, "out");
  const Range in[] = {range_of(a->q, (size_t)a->heads * row, "q"), range_of(a->k, (size_t)a->kv_heads * row, "k"),
                      range_of(a->v, (size_t)a->kv_heads * row, "v"), range_of(a->cos, (size_t)a->capacity * row, "cos"),
                      range_of(a->sin, (size_t)a->capacity * row, "sin"),
                      range_of(a->position, sizeof(int64_t), "position")};
  if (overlaps(keys, values)) return fail(LB_INVALID_ARGUMENT, "lb_decode_attention: keys overlap values");
  for (const Range &r : in) {
    if (overlaps(out, r) || overlaps(keys, r) || overlaps(values, r))
      return fail(LB_INVALID_ARGUMENT, "lb_decode_attention: an output overlaps %s", r.name);
  }
  if (overlaps(out, keys) || overlaps(out, values))
    return fail(LB_INVALID_ARGUMENT, "lb_decode_attention: out overlaps the cache");
  void *ws = a->struct_size >= sizeof(lb_decode_attention_args) ? a->workspace : nullptr;
  const size_t ws_need = LB_ATTN_WORKSPACE_BYTES(a->heads, a->capacity);
  if (ws || (a->struct_size >= sizeof(lb_decode_attention_args) && a->workspace_bytes)) {
    if (!ws || !aligned(ws, 256) || a->workspace_bytes < ws_need)
      return fail(LB_INVALID_ARGUMENT, "lb_decode_attention: workspace must be 256-byte aligned with %zu bytes", ws_need);
    const Range wr = range_of(ws, ws_need, "workspace");
    if (overlaps(wr, out) || overlaps(wr, keys) || overlaps(wr, values))
      return fail(LB_INVALID_ARGUMENT, "lb_decode_attention: workspace overlaps an output");
    for (const Range &r : in)
      if (overlaps(wr, r)) return fail(LB_INVALID_ARGUMENT, "lb_decode_attention: workspace overlaps %s", r.name);
  }
  AttnParams p{};
  p.q = static_cast<const f16 *>(a->q);
  p.k = static_cast<const f16 *>(a->k);
  p.v = static_cast<const f16 *>(a->v);
  p.cos = static_cast<const f16 *>(a->cos);
  p.sin = static_cast<const f16 *>(a->sin);
  p.position = a->position;
  p.keys = static_cast<f16 *>(a->keys);
  p.values = static_cast<f16 *>(a->values);
  p.out = static_cast<f16 *>(a->out);
  p.heads = (int)a->heads;
  p.kv_heads = (int)a->kv_heads;
  p.capacity = (int)a->capacity;
  p.scale = a->scale;
  if (ws && a->heads / a->kv_heads <= kAttnMaxGroup) {
    p.words = static_cast<uint64_t *>(ws);
    p.chunks = (int)((a->capacity + kAttnChunk - 1) / kAttnChunk);
    p.score_wgs = (int)a->kv_heads * p.chunks;
    hipLaunchKernelGGL(split_attention_kernel, dim3((unsigned)(p.score_wgs + a->heads * kAttnDimSlices)), dim3(256),
                       (size_t)a->capacity * sizeof(float), static_cast<hipStream_t>(stream), p);
    return launch_status("lb_decode_attention");
  }
  hipLaunchKernelGGL(decode_attention_kernel, dim3((unsigned)a->heads, kAttnDimSlices), dim3(256),
                     (size_t)a->capacity * sizeof(float),
                     static_cast<hipStream_t>(stream), p);
  return launch_status("lb_decode_attention");
}

lb_status lb_argmax_next(const void *logits, int64_t vocab, const void *embedding, int64_t hidden, void *h_next,
                         int64_t *tokens, int64_t *token, int64_t *position, int64_t limit, void *stream) {
  if (const lb_status bad = refuse_if_failed("lb_argmax_next"); bad != LB_OK) return bad;
  if (!logits || !embedding || !h_next || !tokens || !token || !position)
    return fail(LB_INVALID_ARGUMENT, "lb_argmax_next: NULL pointer");
  if (vocab < 1 || vocab > INT32_MAX / 2 || hidden < 8 || hidden % 8 != 0 || hidden > 65536 || limit < 0 ||
      limit > INT32_MAX)
    return fail(LB_INVALID_ARGUMENT, "lb_argmax_next: vocab >= 1, hidden a positive multiple of 8, limit >= 0");
  if (!aligned(logits, 16) || !aligned(embedding, 16) || !aligned(h_next, 16) || !aligned(tokens, 8) ||
      !aligned(token, 8) || !aligned(position, 8))
    return fail(LB_INVALID_ARGUMENT, "lb_argmax_next: logits/embedding/h_next need 16-byte, indices 8-byte alignment");
  const Range h = range_of(h_next, (size_t)hidden * 2, "h_next");
  const Range outs[] = {h, range_of(tokens, (size_t)limit * 8, "tokens"), range_of(token, 8, "token"),
                        range_of(position, 8, "position")};
  const Range ins[] = {range_of(logits, (size_t)vocab * 2, "logits"),
                       range_of(embedding, (size_t)vocab * hidden * 2, "embedding")};
  for (int i = 0; i < 4; ++i) {
    for (const Range &r : ins)
      if (overlaps(outs[i], r)) return fail(LB_INVALID_ARGUMENT, "lb_argmax_next: %s overlaps %s", outs[i].name, r.name);
    for (int k = i + 1; k < 4; ++k)
      if (overlaps(outs[i], outs[k]))
        return fail(LB_INVALID_ARGUMENT, "lb_argmax_next: %s overlaps %s", outs[i].name, outs[k].name);
  }
  hipLaunchKernelGGL(argmax_next_kernel, dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream),
                     static_cast<const f16 *>(logits), (int)vocab, static_cast<const f16 *>(embedding), (int)hidden,
                     static_cast<f16 *>(h_next), tokens, token, position, (int)limit);
  return launch_status("lb_argmax_next");
}

lb_status lb_head_next(const lb_fused_linear_args *a, const void *embedding, void *h_next, int64_t *tokens,
                       int64_t *token, int64_t *position, int64_t limit, void *stream) {
  if (const lb_status bad = refuse_if_failed("lb_head_next"); bad != LB_OK) return bad;
  if (!a) return fail(LB_INVALID_ARGUMENT, "lb_head_next: args is NULL");
  if (a->struct_size < sizeof(lb_fused_linear_args))
    return fail(LB_INVALID_ARGUMENT, "lb_head_next: struct_size %u < %zu (the workspace fields are required)",
                a->struct_size, sizeof(lb_fused_linear_args));
  const lb_fused_problem &q = a->problems[0];
  if (a->count != 1 || a->prologue != LB_PROLOGUE_RMSNORM || q.rank != 0 || q.bias || q.residual)
    return fail(LB_INVALID_ARGUMENT, "lb_head_next: one problem with the RMSNorm prologue, no correction, bias or residual");
  // The head itself is an lb_fused_linear call; its workspace belongs to the greedy tail here.
  lb_fused_linear_args head = *a;
  head.workspace = nullptr;
  head.workspace_bytes = 0;
  if (const lb_status st = check_fused(&head); st != LB_OK) return st;
  if (a->format != LB_FORMAT_FP16 && a->format != LB_FORMAT_INT4)
    return fail(LB_UNSUPPORTED, "lb_head_next: fp16 or int4 heads only (use lb_fused_linear + lb_argmax_next)");
  if (a->format == LB_FORMAT_FP16 && a->K > 640)
    return fail(LB_UNSUPPORTED, "lb_head_next: fp16 heads of K <= 640 only (use lb_fused_linear + lb_argmax_next)");
  if (!embedding || !h_next || !tokens || !token || !position)
    return fail(LB_INVALID_ARGUMENT, "lb_head_next: NULL pointer");
  if (!aligned(embedding, 16) || !aligned(h_next, 16) || !aligned(tokens, 8) || !aligned(token, 8) ||
      !aligned(position, 8))
    return fail(LB_INVALID_ARGUMENT, "lb_head_next: embedding/h_next need 16-byte, indices 8-byte alignment");
  if (limit < 0 || limit > INT32_MAX) return fail(LB_INVALID_ARGUMENT, "lb_head_next: limit outside 0..2^31-1");
  const int64_t vocab = q.N, hidden = a->K;
  const size_t ws_bytes = LB_HEAD_NEXT_WORKSPACE_BYTES(vocab);
  // The macro counts groups of 8 workgroups of 64 rows (a larger kernel group uses fewer words).
  static_assert(kHeadNextGroup >= 8 && LB_HEAD_NEXT_WORKSPACE_BYTES(64 * 8 * 3) == 16u * 4u,
                "the workspace macro's words cover the kernel's groups");
  if (!a->workspace || !aligned(a->workspace, 256) || a->workspace_bytes < ws_bytes)
    return fail(LB_INVALID_ARGUMENT, "lb_head_next: workspace must be 256-byte aligned with %zu bytes", ws_bytes);
  const Range ins[] = {range_of(a->x, (size_t)hidden * 2, "x"), range_of(a->gamma, (size_t)hidden * 2, "gamma"),
                       range_of(q.codes, code_bytes(a->format, vocab, hidden), "codes"),
                       range_of(q.scales, a->format == LB_FORMAT_FP16 ? 0 : (size_t)(vocab * (hidden / a->group_size) * 2),
                                "scales"),
                       range_of(embedding, (size_t)(vocab * hidden * 2), "embedding")};
  const Range outs[] = {range_of(h_next, (size_t)hidden * 2, "h_next"), range_of(tokens, (size_t)limit * 8, "tokens"),
                        range_of(token, 8, "token"), range_of(position, 8, "position"),
                        range_of(q.y, (size_t)vocab * 2, "logits"), range_of(a->workspace, ws_bytes, "workspace")};
  constexpr int kOuts = sizeof(outs) / sizeof(outs[0]);
  for (int i = 0; i < kOuts; ++i) {
    for (const Range &r : ins)  // h_next may be x itself: every workgroup reads x before the token is known
      if (overlaps(outs[i], r) && !(i == 0 && h_next == a->x && &r == &ins[0]))
        return fail(LB_INVALID_ARGUMENT, "lb_head_next: %s overlaps %s", outs[i].name, r.name);
    for (int k = i + 1; k < kOuts; ++k)
      if (overlaps(outs[i], outs[k]))
        return fail(LB_INVALID_ARGUMENT, "lb_head_next: %s overlaps %s", outs[i].name, outs[k].name);
  }
  int tiles = 0;
  const FusedParams p = fused_params(&head, &tiles);
  const int wgs = (tiles + 3) / 4;
  HeadNextParams hn{};
  hn.ws = static_cast<uint64_t *>(a->workspace);
  hn.embedding = static_cast<const f16 *>(embedding);
  hn.h_next = static_cast<f16 *>(h_next);
  hn.tokens = tokens;
  hn.token = token;
  hn.position = position;
  hn.limit = (int)limit;
  hn.hidden = (int)hidden;
  hn.groups = (wgs + kHeadNextGroup - 1) / kHeadNextGroup;
  hn.vocab = (int)vocab;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const bool launched = a->format == LB_FORMAT_FP16 ? launch_head_next_f<FMT_FP16, false>(p, hn, wgs, s)
                                                    : launch_head_next_f<FMT_INT4, true>(p, hn, wgs, s);
  if (!launched) return fail(LB_UNSUPPORTED, "lb_head_next: no kernel for this shape");
  return launch_status("lb_head_next");
}

}  // extern "C"

namespace {

static_assert(sizeof(LayerWeights) == 256, "LB_DECODE_STACK_TABLE_BYTES assumes 256 bytes per layer");

// Everything of a decode-layer launch but the per-layer tensors: shapes, format, attention,
// workspace layout and the role grid.  `layers` regions of LB_DECODE_LAYER_WORDS words follow the
// workspace header.
struct LayerShape {
  uint32_t format;
  int64_t group_size, hidden, intermediate, heads, kv_heads, capacity, layers;
  void *h;
  float eps, scale;
  const void *cos, *sin;
  const int64_t *position;
  void *workspace;
  size_t workspace_bytes;
};

lb_status check_shape(const char *who, const LayerShape &a, LayerParams *p, Range *in, int &nin) {
  if (a.format > LB_FORMAT_FP16) return fail(LB_INVALID_ARGUMENT, "%s: unknown format %u", who, a.format);
  const int64_t H = a.hidden, I = a.intermediate;
  if (a.heads < 1 || a.kv_heads < 1 || a.heads % a.kv_heads != 0 || a.heads / a.kv_heads > 3 ||
      H != a.heads * kHeadDim || H > 640 || I < 32 || I > kFusedMaxK || I % 32 != 0)
    return fail(LB_INVALID_ARGUMENT,
                "%s: needs hidden = 64 heads <= 640, heads / kv_heads <= 3, intermediate a multiple of 32 <= %d", who,
                kFusedMaxK);
  if (a.capacity < 1 || a.capacity > 4096)
    return fail(LB_INVALID_ARGUMENT, "%s: capacity %lld outside 1..4096", who, (long long)a.capacity);
  if (a.layers < 1 || a.layers > LB_DECODE_STACK_MAX_LAYERS)
    return fail(LB_INVALID_ARGUMENT, "%s: layers %lld outside 1..%d", who, (long long)a.layers, LB_DECODE_STACK_MAX_LAYERS);
  const bool dense = a.format == LB_FORMAT_FP16;
  const int64_t g = a.group_size;
  const bool per_row = a.format == LB_FORMAT_INT8 && g == 0;
  if (!dense && !per_row && !(pow2(g) && g >= 32 && H % g == 0 && I % g == 0))
    return fail(LB_INVALID_ARGUMENT, "%s: group_size %lld must be 0 (int8 per row) or a power of two "
                "(>= 32) dividing hidden and intermediate", who, (long long)g);
  if (!a.h || !aligned(a.h, 16) || !std::isfinite(a.eps) || a.eps < 0)
    return fail(LB_INVALID_ARGUMENT, "%s: h must be 16-byte aligned; eps finite >= 0", who);
  if (!a.cos || !a.sin || !aligned(a.cos, 2) || !aligned(a.sin, 2) || !a.position || !aligned(a.position, 8) ||
      !std::isfinite(a.scale))
    return fail(LB_INVALID_ARGUMENT, "%s: RoPE tables or position NULL or misaligned, or scale not finite", who);
  const size_t need = LB_DECODE_STACK_WORKSPACE_BYTES(H, I, a.kv_heads, a.layers);
  if (!a.workspace || !aligned(a.workspace, 256) || a.workspace_bytes < need)
    return fail(LB_INVALID_ARGUMENT, "%s: workspace must be 256-byte aligned with %zu bytes", who, need);
  const size_t row = kHeadDim * 2;
  in[nin++] = range_of(a.cos, (size_t)a.capacity * row, "cos");
  in[nin++] = range_of(a.sin, (size_t)a.capacity * row, "sin");
  in[nin++] = range_of(a.position, sizeof(int64_t), "position");
  LayerParams q{};
  q.h = static_cast<f16 *>(a.h);
  q.eps = a.eps;
  q.hidden = (int)H;
  q.inter = (int)I;
  q.per_row = per_row;
  const int64_t g1 = dense || per_row ? H : g, g2 = dense || per_row ? I : g;
  q.G1 = (int)(H / g1);
  q.shift1 = shift_of(g1, H);
  q.G2 = (int)(I / g2);
  q.shift2 = shift_of(g2, I);
  q.cos = static_cast<const f16 *>(a.cos);
  q.sin = static_cast<const f16 *>(a.sin);
  q.position = a.position;
  q.heads = (int)a.heads;
  q.kv_heads = (int)a.kv_heads;
  q.capacity = (int)a.capacity;
  q.scale = a.scale;
  q.ws = static_cast<uint64_t *>(a.workspace);
  q.layers = (int)a.layers;
  q.layer_words = (int)LB_DECODE_LAYER_WORDS(H, I, a.kv_heads);
  const int64_t kv = a.kv_heads * kHeadDim;
  q.w_z = 0;
  q.w_qkv = q.w_z + P_COUNT * kLayerZWords;
  q.w_att = q.w_qkv + (int)((H + 2 * kv) / 2);
  q.w_h1 = q.w_att + (int)(H / 2);
  q.w_gu = q.w_h1 + (int)(H / 2);
  q.w_h = q.w_gu + (int)I;
  const int64_t want_n[P_COUNT] = {H, kv, kv, H, I, I, H};
  for (int i = 0; i < P_COUNT; ++i) q.N[i] = (int)want_n[i];
  *p = q;
  return ok();
}

// One layer's tensors: shapes against the launch, ranks and U strides equal to those of the first
// layer (the role grid is shared), into `w`; their byte ranges are appended to `in` / `out`.
lb_status check_weights(const char *who, int layer, uint32_t format, const lb_fused_problem *proj, const void *norm1,
                        const void *norm2, void *keys, void *values, LayerParams *p, LayerWeights *w, Range *in,
                        int &nin, Range *out, int &nout) {
  static const char *names[P_COUNT] = {"q", "k", "v", "o", "gate", "up", "down"};
  const bool dense = format == LB_FORMAT_FP16;
  if (!norm1 || !aligned(norm1, 16) || !norm2 || !aligned(norm2, 16) || !keys || !values || !aligned(keys, 16) ||
      !aligned(values, 16))
    return fail(LB_INVALID_ARGUMENT, "%s: layer %d: norm1, norm2, keys, values must be 16-byte aligned", who, layer);
  const size_t cache = (size_t)p->kv_heads * p->capacity * kHeadDim * 2;
  in[nin++] = range_of(norm1, (size_t)p->hidden * 2, "norm1");
  in[nin++] = range_of(norm2, (size_t)p->hidden * 2, "norm2");
  out[nout++] = range_of(keys, cache, "keys");
  out[nout++] = range_of(values, cache, "values");
  LayerWeights d{};
  for (int i = 0; i < P_COUNT; ++i) {
    const lb_fused_problem &q = proj[i];
    const int64_t K = i == P_DOWN ? p->inter : p->hidden;
    if (q.N != p->N[i])
      return fail(LB_INVALID_ARGUMENT, "%s: layer %d: %s has N=%lld, expected %d", who, layer, names[i], (long long)q.N,
                  p->N[i]);
    if (q.y || q.bias || q.residual)
      return fail(LB_INVALID_ARGUMENT, "%s: layer %d: %s: y, bias and residual must be NULL", who, layer, names[i]);
    if (!q.codes || !aligned(q.codes, 16) || (!dense && (!q.scales || !aligned(q.scales, 2))))
      return fail(LB_INVALID_ARGUMENT, "%s: layer %d: %s: codes (16-byte aligned) and scales required", who, layer,
                  names[i]);
    if (q.rank < 0 || q.rank > LB_FUSED_MAX_RANK)
      return fail(LB_INVALID_ARGUMENT, "%s: layer %d: %s: rank %lld outside 0..32", who, layer, names[i], (long long)q.rank);
    if (q.rank > 0 && (!q.down || !q.up || !aligned(q.down, 16) || !aligned(q.up, 16) || q.up_ld < q.rank ||
                       q.up_ld % 8 != 0))
      return fail(LB_INVALID_ARGUMENT, "%s: layer %d: %s: correction needs 16-byte aligned down/up, up_ld %% 8 == 0", who,
                  layer, names[i]);
    const int up_ld = q.rank ? (int)q.up_ld : 0;
    if (layer == 0) {
      p->rank[i] = (int)q.rank;
      p->up_ld[i] = up_ld;
    } else if (p->rank[i] != (int)q.rank || p->up_ld[i] != up_ld) {
      return fail(LB_INVALID_ARGUMENT, "%s: layer %d: %s: rank and up_ld must equal those of layer 0", who, layer,
                  names[i]);
    }
    const int64_t G = dense ? 1 : p->per_row ? 1 : (i == P_DOWN ? p->G2 : p->G1);
    in[nin++] = range_of(q.codes, code_bytes(format, q.N, K), "codes");
    in[nin++] = range_of(dense ? nullptr : q.scales, dense ? 0 : (size_t)(q.N * G * 2), "scales");
    in[nin++] = range_of(q.rank ? q.down : nullptr, q.rank ? (size_t)(q.rank * K * 2) : 0, "down");
    in[nin++] = range_of(q.rank ? q.up : nullptr, q.rank ? (size_t)((q.N - 1) * q.up_ld + q.rank) * 2 : 0, "up");
    d.codes[i] = static_cast<const uint8_t *>(q.codes);
    d.scales[i] = static_cast<const f16 *>(q.scales);
    d.down[i] = q.rank ? static_cast<const f16 *>(q.down) : nullptr;
    d.up[i] = q.rank ? static_cast<const f16 *>(q.up) : nullptr;
  }
  d.norm1 = static_cast<const f16 *>(norm1);
  d.norm2 = static_cast<const f16 *>(norm2);
  d.keys = static_cast<f16 *>(keys);
  d.values = static_cast<f16 *>(values);
  *w = d;
  return ok();
}

lb_status check_overlaps(const char *who, const Range *in, int nin, const Range *out, int nout) {
  for (int o = 0; o < nout; ++o) {
    for (int r = 0; r < nin; ++r)
      if (overlaps(out[o], in[r])) return fail(LB_INVALID_ARGUMENT, "%s: %s overlaps %s", who, out[o].name, in[r].name);
    for (int r = o + 1; r < nout; ++r)
      if (overlaps(out[o], out[r])) return fail(LB_INVALID_ARGUMENT, "%s: %s overlaps %s", who, out[o].name, out[r].name);
  }
  return ok();
}

// The role grid (T_QKV, ATTN, T_O, T_GU, Z_D, T_D) and the launch's template choice.
void finish_params(LayerParams *p, uint32_t format, int64_t group_size, int *fmt, bool *scaled, bool *ranked) {
  auto zc = [&](int i) { return p->rank[i]; };  // one z workgroup per rank
  auto tc = [&](int i) { return (p->N[i] + 15) / 16; };
  const int counts[R_COUNT] = {tc(P_Q) + tc(P_K) + tc(P_V), p->heads * kAttnDimSlices, tc(P_O),
                               tc(P_GATE) + tc(P_UP), zc(P_DOWN), tc(P_DOWN)};
  int acc = 0;
  for (int r = 0; r < R_COUNT; ++r) p->end[r] = acc += counts[r];
  bool any = false;
  for (int i = 0; i < P_COUNT; ++i) any = any || p->rank[i] > 0;
  *fmt = (int)format;
  *scaled = format != LB_FORMAT_FP16 && !(format == LB_FORMAT_INT8 && group_size == 0);
  *ranked = any;
}

// Dynamic LDS: the largest role (a 1536-long tile: staged row, scales, U rows, reductions, NF4
// table) or the attention (its rows, the P.V partials and one float per cache slot).
size_t layer_smem(const LayerParams &p) { return std::max<size_t>(kLayerTileSmem, 2048 + (size_t)4 * p.capacity); }

template <int FMT, bool SCALED, bool RANKED, bool STACK>
const void *layer_kernel_fn() {
  return reinterpret_cast<const void *>(&decode_layer_kernel<FMT, SCALED, RANKED, STACK>);
}

template <bool STACK>
const void *layer_kernel(int fmt, bool scaled, bool ranked) {
  switch (fmt) {
    case FMT_INT8:
      if (scaled) return ranked ? layer_kernel_fn<FMT_INT8, true, true, STACK>() : layer_kernel_fn<FMT_INT8, true, false, STACK>();
      return ranked ? layer_kernel_fn<FMT_INT8, false, true, STACK>() : layer_kernel_fn<FMT_INT8, false, false, STACK>();
    case FMT_INT4: return ranked ? layer_kernel_fn<FMT_INT4, true, true, STACK>() : layer_kernel_fn<FMT_INT4, true, false, STACK>();
    case FMT_NF4: return ranked ? layer_kernel_fn<FMT_NF4, true, true, STACK>() : layer_kernel_fn<FMT_NF4, true, false, STACK>();
    default: return ranked ? layer_kernel_fn<FMT_FP16, false, true, STACK>() : layer_kernel_fn<FMT_FP16, false, false, STACK>();
  }
}

lb_status launch_layers(const char *who, const void *fn, const LayerParams &p, const LayerWeights *table, hipStream_t s) {
  LayerParams args = p;
  const LayerWeights *tab = table;
  void *kargs[] = {&args, &tab};
  const hipError_t e = hipLaunchKernel(fn, dim3((unsigned)p.end[R_COUNT - 1]), dim3(256), kargs, layer_smem(p), s);
  if (e != hipSuccess) {
    char reason[256];
    snprintf(reason, sizeof reason, "%s: launch failed: %s", who, hipGetErrorString(e));
    mark_failed(reason);
    return fail(LB_DEVICE_FAILED, "%s", reason);
  }
  return launch_status(who);
}

// Tables written by lb_decode_stack_prepare: the bytes, so a later call can verify that its
// arguments describe the same layers, and whether the device holds the stacked grid at once.
struct PreparedTable {
  std::vector<LayerWeights> rows;
  bool resident;
};
std::mutex &table_mutex() {
  static std::mutex m;
  return m;
}
std::map<const void *, PreparedTable> &table_registry() {
  static std::map<const void *, PreparedTable> r;
  return r;
}

lb_status check_stack(const char *who, const lb_decode_stack_args *a, LayerParams *p, std::vector<LayerWeights> *rows,
                      int *fmt, bool *scaled, bool *ranked) {
  if (!a) return fail(LB_INVALID_ARGUMENT, "%s: args is NULL", who);
  if (a->struct_size < sizeof(lb_decode_stack_args))
    return fail(LB_INVALID_ARGUMENT, "%s: struct_size %u < %zu", who, a->struct_size, sizeof(lb_decode_stack_args));
  const LayerShape shape{a->format, a->group_size, a->hidden, a->intermediate, a->heads, a->kv_heads, a->capacity,
                         a->layers, a->h, a->eps, a->scale, a->cos, a->sin, a->position, a->workspace,
                         a->workspace_bytes};
  const int L = a->layers >= 1 && a->layers <= LB_DECODE_STACK_MAX_LAYERS ? (int)a->layers : 1;
  std::vector<Range> in((size_t)L * (2 + 4 * P_COUNT) + 8), out((size_t)L * 2 + 8);
  int nin = 0, nout = 0;
  if (const lb_status st = check_shape(who, shape, p, in.data(), nin); st != LB_OK) return st;
  if (!a->layer) return fail(LB_INVALID_ARGUMENT, "%s: layer array is NULL", who);
  if (!a->table || !aligned(a->table, 256) || a->table_bytes < LB_DECODE_STACK_TABLE_BYTES(a->layers))
    return fail(LB_INVALID_ARGUMENT, "%s: table must be 256-byte aligned with %zu bytes", who,
                (size_t)LB_DECODE_STACK_TABLE_BYTES(a->layers));
  rows->assign((size_t)L, LayerWeights{});
  for (int l = 0; l < L; ++l) {
    const lb_decode_stack_layer &y = a->layer[l];
    if (const lb_status st = check_weights(who, l, a->format, y.proj, y.norm1, y.norm2, y.keys, y.values, p,
                                           &(*rows)[(size_t)l], in.data(), nin, out.data(), nout);
        st != LB_OK)
      return st;
  }
  out[nout++] = range_of(a->h, (size_t)a->hidden * 2, "h");
  out[nout++] = range_of(a->workspace, LB_DECODE_STACK_WORKSPACE_BYTES(a->hidden, a->intermediate, a->kv_heads, a->layers),
                         "workspace");
  out[nout++] = range_of(a->table, LB_DECODE_STACK_TABLE_BYTES(a->layers), "table");
  if (const lb_status st = check_overlaps(who, in.data(), nin, out.data(), nout); st != LB_OK) return st;
  finish_params(p, a->format, a->group_size, fmt, scaled, ranked);
  return ok();
}

}  // namespace

extern "C" lb_status lb_decode_layer(const lb_decode_layer_args *a, void *stream) {
  const char *who = "lb_decode_layer";
  if (const lb_status bad = refuse_if_failed(who); bad != LB_OK) return bad;
  if (!a) return fail(LB_INVALID_ARGUMENT, "%s: args is NULL", who);
  if (a->struct_size < sizeof(lb_decode_layer_args))
    return fail(LB_INVALID_ARGUMENT, "%s: struct_size %u < %zu", who, a->struct_size, sizeof(lb_decode_layer_args));
  const LayerShape shape{a->format, a->group_size, a->hidden, a->intermediate, a->heads, a->kv_heads, a->capacity,
                         1, a->h, a->eps, a->scale, a->cos, a->sin, a->position, a->workspace, a->workspace_bytes};
  Range in[8 + 2 + 4 * P_COUNT], out[8];
  int nin = 0, nout = 0;
  LayerParams p;
  if (const lb_status st = check_shape(who, shape, &p, in, nin); st != LB_OK) return st;
  if (const lb_status st = check_weights(who, 0, a->format, a->proj, a->norm1, a->norm2, a->keys, a->values, &p, &p.w,
                                         in, nin, out, nout);
      st != LB_OK)
    return st;
  out[nout++] = range_of(a->h, (size_t)a->hidden * 2, "h");
  out[nout++] = range_of(a->workspace, LB_DECODE_LAYER_WORKSPACE_BYTES(a->hidden, a->intermediate, a->kv_heads),
                         "workspace");
  if (const lb_status st = check_overlaps(who, in, nin, out, nout); st != LB_OK) return st;
  int fmt;
  bool scaled, ranked;
  finish_params(&p, a->format, a->group_size, &fmt, &scaled, &ranked);
  return launch_layers(who, layer_kernel<false>(fmt, scaled, ranked), p, nullptr, static_cast<hipStream_t>(stream));
}

extern "C" lb_status lb_decode_stack_prepare(const lb_decode_stack_args *a, void *stream) {
  const char *who = "lb_decode_stack_prepare";
  if (const lb_status bad = refuse_if_failed(who); bad != LB_OK) return bad;
  LayerParams p;
  std::vector<LayerWeights> rows;
  int fmt;
  bool scaled, ranked;
  if (const lb_status st = check_stack(who, a, &p, &rows, &fmt, &scaled, &ranked); st != LB_OK) return st;
  // Residency: every workgroup of the stacked grid must be on the device at once.
  // The device is the stream's (the current device for the null stream).
  int device = 0, cus = 0, per_cu = 0;
  const void *fn = layer_kernel<true>(fmt, scaled, ranked);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (hipStreamGetDevice(s, &device) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 256, layer_smem(p)) != hipSuccess)
    return fail(LB_DEVICE_FAILED, "%s: device query failed", who);
  if (hipMemcpyAsync(a->table, rows.data(), rows.size() * sizeof(LayerWeights), hipMemcpyHostToDevice, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess) {
    mark_failed("lb_decode_stack_prepare: table copy failed");
    return fail(LB_DEVICE_FAILED, "%s: table copy failed", who);
  }
  std::lock_guard<std::mutex> lock(table_mutex());
  table_registry()[a->table] = PreparedTable{std::move(rows), (long long)per_cu * cus >= p.end[R_COUNT - 1]};
  return ok();
}

extern "C" lb_status lb_decode_stack(const lb_decode_stack_args *a, void *stream) {
  const char *who = "lb_decode_stack";
  if (const lb_status bad = refuse_if_failed(who); bad != LB_OK) return bad;
  LayerParams p;
  std::vector<LayerWeights> rows;
  int fmt;
  bool scaled, ranked;
  if (const lb_status st = check_stack(who, a, &p, &rows, &fmt, &scaled, &ranked); st != LB_OK) return st;
  {
    std::lock_guard<std::mutex> lock(table_mutex());
    const auto it = table_registry().find(a->table);
    if (it == table_registry().end() || it->second.rows.size() != rows.size() ||
        std::memcmp(it->second.rows.data(), rows.data(), rows.size() * sizeof(LayerWeights)) != 0)
      return fail(LB_INVALID_ARGUMENT, "%s: table was not prepared (lb_decode_stack_prepare) for these layers", who);
    if (!it->second.resident)
      return fail(LB_UNSUPPORTED, "%s: the device cannot hold the %d workgroups of the stacked grid at once", who,
                  p.end[R_COUNT - 1]);
  }
  return launch_layers(who, layer_kernel<true>(fmt, scaled, ranked), p, static_cast<const LayerWeights *>(a->table),
                       static_cast<hipStream_t>(stream));
}

extern "C" lb_status lb_decode_stack_release(const void *table) {
  std::lock_guard<std::mutex> lock(table_mutex());
  if (!table || table_registry().erase(table) == 0)
    return fail(LB_INVALID_ARGUMENT, "lb_decode_stack_release: the table was not prepared");
  return ok();
}

extern "C" lb_status lb_decode_check(const void *workspace, size_t timeout_offset, void *stream, uint32_t *timeouts) {
  const char *who = "lb_decode_check";
  if (timeouts) *timeouts = 0;
  if (const lb_status bad = refuse_if_failed(who); bad != LB_OK) return bad;
  if (!workspace || !aligned(workspace, 256) || timeout_offset % 4 != 0)
    return fail(LB_INVALID_ARGUMENT, "%s: workspace must be 256-byte aligned and the offset a multiple of 4", who);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t word = 0;
  if (hipMemcpyAsync(&word, static_cast<const char *>(workspace) + timeout_offset, sizeof word, hipMemcpyDeviceToHost,
                     s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess) {
    char reason[256];
    snprintf(reason, sizeof reason, "%s: synchronisation failed: %s", who, hipGetErrorString(hipGetLastError()));
    mark_failed(reason);
    return fail(LB_DEVICE_FAILED, "%s", reason);
  }
  if (timeouts) *timeouts = word;
  if (word != 0) {
    mark_failed("a bounded hand-over wait of a decode launch gave up: the outputs of the calls on that workspace are "
                "not valid");
    return fail(LB_DEVICE_FAILED,
                "%s: a bounded hand-over wait gave up (timeout word %u): outputs since are not valid; the library is "
                "now failed",
                who, word);
  }
  return ok();
}
