// gfx950 one-row GEMV over INT4 / INT8 / NF4 weights with lane-linear weight loads:
// y[n] = x . (q * s)[n] (+ bias) (+ residual), the exact-product sums of stream_gemv_kernel.
//
// Layout of the work.  A segment of a row is what one wave-wide 16-byte load covers: 64 lanes x
// CPL codes (2048 INT4 / 1024 INT8 codes, 1 KB).  A wave owns R rows and one segment: its R weight
// loads each read 1 KB of one row contiguously, and a lane's codes sit at the same k in all R
// rows, so the lane loads its activations once (straight into registers, no LDS staging and no
// barrier before the arithmetic) and uses them R times.  A workgroup's waves cover P groups of R
// rows x every segment of K; the segments' row sums meet in LDS once, at the end, and are added
// in segment order.
//
// Arithmetic of a 16-byte load.  The codes enter v_dot2_f32_f16 as the fp16 value of a "magic"
// half-word, the sign-flipped nibble or byte OR-ed under the exponent of 1024:
//   INT4 even codes  0x6400 | (c ^ 8)         = 1032 + q   (activation x)
//   INT4 odd codes   0x6400 | ((c ^ 8) << 4)  = 1152 + 16 q (activation x / 16, nibble in place)
//   INT8             0x6400 | (b ^ 0x80)      = 1152 + q
// so a row's chain sums x (bias + q) over the lane's codes.  The chain starts at -B, B being the
// lane's activations dotted with the biases (computed once, the same for all R rows), which leaves
// sum x q up to fp32 rounding.  NF4 codes enter as the fp16 literals of their byte's two codes
// (the low nibble the even code) from a 256-pair table each workgroup builds in LDS, with no
// bias (line_gemv_kernel only); the lane's CPL codes lie in one group, whose scale multiplies the
// lane's sum (per-row scales multiply the row's total).  The reference's rounding-budget gate
// (torch_npu_lowbit_demo.py:97-106) bounds the distance to its fp16(q * s) weights.
#pragma once
#include "lb_decode.h"
#include "lb_stream.h"

namespace lb {

template <int FMT> struct LineTraits;
template <> struct LineTraits<FMT_INT4> { static constexpr int CPL = 32, BITS = 4, XL = 4; };
template <> struct LineTraits<FMT_INT8> { static constexpr int CPL = 16, BITS = 8, XL = 2; };
template <> struct LineTraits<FMT_NF4> { static constexpr int CPL = 32, BITS = 4, XL = 4; };

constexpr int kLineMaxWaves = 16;  // waves per workgroup (segments x row groups)

// Activation pairs of the lane's codes in the decode's slot order, and the bias sum B.
template <int FMT>
__device__ __forceinline__ float line_pairs(const u4 *xv, h2 *xp) {
  using TR = LineTraits<FMT>;
  float b = 0.0f;
  if constexpr (FMT == FMT_INT4) {
    const h2 even = {(f16)1032.0f, (f16)1032.0f}, odd = {(f16)1152.0f, (f16)1152.0f};
    const h2 sixteenth = {(f16)0.0625f, (f16)0.0625f};
#pragma unroll
    for (int i = 0; i < TR::XL; ++i) {  // load i: codes 8i .. 8i + 7, the weight dword i
      const h8 v = __builtin_bit_cast(h8, xv[i]);
      xp[4 * i + 0] = h2{v[0], v[4]};
      xp[4 * i + 1] = h2{v[1], v[5]} * sixteenth;
      xp[4 * i + 2] = h2{v[2], v[6]};
      xp[4 * i + 3] = h2{v[3], v[7]} * sixteenth;
      b = dot2(xp[4 * i + 0], even, b);
      b = dot2(xp[4 * i + 1], odd, b);
      b = dot2(xp[4 * i + 2], even, b);
      b = dot2(xp[4 * i + 3], odd, b);
    }
  } else if constexpr (FMT == FMT_NF4) {  // natural pairs (codes 2e, 2e + 1 of a byte), no bias
#pragma unroll
    for (int i = 0; i < TR::XL; ++i) {
      const h8 v = __builtin_bit_cast(h8, xv[i]);
#pragma unroll
      for (int e = 0; e < 4; ++e) xp[4 * i + e] = h2{v[2 * e], v[2 * e + 1]};
    }
  } else {
    const h2 bias = {(f16)1152.0f, (f16)1152.0f};
#pragma unroll
    for (int i = 0; i < TR::XL; ++i) {  // load i: codes 8i .. 8i + 7, the weight dwords 2i, 2i + 1
      const h8 v = __builtin_bit_cast(h8, xv[i]);
      xp[4 * i + 0] = h2{v[0], v[2]};
      xp[4 * i + 1] = h2{v[1], v[3]};
      xp[4 * i + 2] = h2{v[4], v[6]};
      xp[4 * i + 3] = h2{v[5], v[7]};
#pragma unroll
      for (int e = 0; e < 4; ++e) b = dot2(xp[4 * i + e], bias, b);
    }
  }
  return b;
}

// Chain of one 16-byte weight load against the lane's activation pairs, starting at acc.  NF4:
// each code byte's pair of fp16 literals from the workgroup's LDS table (all 16 reads issued
// before the chain).
template <int FMT>
__device__ __forceinline__ float line_dot(const u4 &w, const h2 *xp, float acc, const uint32_t *nf4_table) {
  if constexpr (FMT == FMT_NF4) {
    h2 pr[16];
#pragma unroll
    for (int d = 0; d < 4; ++d)
#pragma unroll
      for (int e = 0; e < 4; ++e) pr[4 * d + e] = __builtin_bit_cast(h2, nf4_table[(w[d] >> (8 * e)) & 0xFFu]);
#pragma unroll
    for (int i = 0; i < 16; ++i) acc = dot2(xp[i], pr[i], acc);
    return acc;
  }
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    if constexpr (FMT == FMT_INT4) {  // (nibble ^ 8) under 0x6400: one three-input bit operation each
      const uint32_t a = w[d], u = a >> 8;
      acc = dot2(xp[4 * d + 0], __builtin_bit_cast(h2, (a & 0x000F000Fu) ^ 0x64086408u), acc);  // codes 0, 4
      acc = dot2(xp[4 * d + 1], __builtin_bit_cast(h2, (a & 0x00F000F0u) ^ 0x64806480u), acc);  // codes 1, 5
      acc = dot2(xp[4 * d + 2], __builtin_bit_cast(h2, (u & 0x000F000Fu) ^ 0x64086408u), acc);  // codes 2, 6
      acc = dot2(xp[4 * d + 3], __builtin_bit_cast(h2, (u & 0x00F000F0u) ^ 0x64806480u), acc);  // codes 3, 7
    } else {
      const uint32_t s = w[d] ^ 0x80808080u;
      // v_perm_b32: selector bytes 0-3 pick from the second operand (s), 4-7 from the first.
      acc = dot2(xp[2 * d + 0], __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, s, 0x04020400u)), acc);
      acc = dot2(xp[2 * d + 1], __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, s, 0x04030401u)), acc);
    }
  }
  return acc;
}

// One level of the transposed wave reduction: lanes with bit B of their index clear keep the even
// value of each pair, the others the odd one, and each adds the copy of the value it keeps held by
// lane ^ (1 << B).  Partners always differ in bit B alone, so every row is summed over aligned lane
// blocks in one and the same association (a + b == b + a): the result does not depend on which
// lane of a wave, or which position in its row group, a row falls to.
constexpr int kDppRowRor12 = 0x12C;  // row_ror:12: lane i gets lane i + 4 (mod 16)
template <int B, int NV>
__device__ __forceinline__ void line_fold(float *v, int lane) {
  static_assert(B <= 3, "levels within a row of 16 lanes");
  const bool hi = (lane >> B) & 1;
#pragma unroll
  for (int i = 0; i < NV / 2; ++i) {
    const float keep = hi ? v[2 * i + 1] : v[2 * i];
    const float send = hi ? v[2 * i] : v[2 * i + 1];
    float other;
    if constexpr (B == 0) other = dpp_move<kDppXor1>(send);
    else if constexpr (B == 1) other = dpp_move<kDppXor2>(send);
    else if constexpr (B == 2) {
      // Both moves under the full wave: a select of the two must not become a branch, where a DPP
      // move would read lanes the branch has switched off.
      float down = dpp_move<kDppRowRor4>(send), up = dpp_move<kDppRowRor12>(send);
      asm volatile("" : "+v"(down), "+v"(up));
      other = hi ? down : up;
    }
    else other = dpp_move<kDppRowRor8>(send);  // lane i - 8 (mod 16) is lane i ^ 8
    v[i] = keep + other;
  }
}

// Leading scalar arguments are preloaded into registers at wave launch (the first loads need no
// argument-block read); the epilogue's operands come from `p`.
template <int FMT, bool SCALED, int R, bool QS>
__global__ __launch_bounds__(64 * kLineMaxWaves) void line_gemv_kernel(const f16 *pre_x, const uint8_t *pre_codes,
                                                                       const f16 *pre_scales, int pre_N, int pre_K,
                                                                       int pre_G, int pre_shift, int pre_nseg,
                                                                       int pre_groups, StreamParams p) {
  using TR = LineTraits<FMT>;
  constexpr int CPL = TR::CPL, XL = TR::XL, SEG = 64 * CPL;
  constexpr int kOutOfRange = (int)0x80000000u;
  static_assert(R == 4 || R == 8 || R == 16, "rows per wave");
  __shared__ float part[kLineMaxWaves * R];
  __shared__ uint32_t nf4_table[FMT == FMT_NF4 ? 256 : 1];

  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int nseg = pre_nseg, N = pre_N, K = pre_K;
  const int seg = wave % nseg, rg = wave / nseg;
  const int rows_wg = pre_groups * R;  // pre_groups row groups x nseg segments = the workgroup's waves
  const int n0 = blockIdx.x * rows_wg + rg * R;
  const int rows = min(R, N - n0);  // <= 0 for row groups past N
  const int row_bytes = K * TR::BITS / 8;
  const int k0 = seg * SEG + lane * CPL;
  const bool live = k0 < K;

  // ---- loads: the group scales, the lane's activations, the R weight loads, the epilogue's
  // operands (lanes 0 .. rows_wg - 1 of wave 0) ----
  // QS (groups of at least 4 CPL codes, so a lane quad shares one): a lane scales its quad's sums
  // of rows 4i + lane % 4 (i < R / 4) once two reduction levels have formed them; otherwise it
  // scales its own sum of each row.
  const size_t base_row = rows > 0 ? (size_t)n0 : 0;
  constexpr int NSC = !SCALED ? 1 : QS ? R / 4 : R;
  f16 sc[NSC];
  if constexpr (SCALED) {
    const __amdgpu_buffer_rsrc_t sb =
        buffer_rsrc(pre_scales + base_row * pre_G, rows > 0 ? (size_t)rows * pre_G * 2 : 0);
    const int gi = k0 >> pre_shift;
#pragma unroll
    for (int i = 0; i < NSC; ++i) {
      const int r = QS ? 4 * i + (lane & 3) : i;
      sc[i] = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(sb, live ? (r * pre_G + gi) * 2 : kOutOfRange, 0, 0));
    }
  }
  u4 xv[XL];
  {
    const __amdgpu_buffer_rsrc_t xb = buffer_rsrc(pre_x, (size_t)K * 2);
#pragma unroll
    for (int i = 0; i < XL; ++i)
      xv[i] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(xb, live ? (k0 + 8 * i) * 2 : kOutOfRange, 0, 0));
  }
  u4 w[R];
  {
    const __amdgpu_buffer_rsrc_t wb =
        buffer_rsrc(pre_codes + base_row * row_bytes, rows > 0 ? (size_t)rows * row_bytes : 0);
    const int kb = k0 * TR::BITS / 8;
#pragma unroll
    for (int r = 0; r < R; ++r)
      w[r] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(wb, live ? r * row_bytes + kb : kOutOfRange, 0, 0));
  }
  const int en = blockIdx.x * rows_wg + t;  // the epilogue row of lane t of wave 0
  // Issued by every wave (no branch: a branch join would make wave 0 wait for all its loads here);
  // the lanes that own no output row read nothing.
  const size_t ebytes = (size_t)N * 2;
  const int eoff = wave == 0 && t < rows_wg && en < N ? en * 2 : kOutOfRange;
  const f16 e_bias =
      __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(p.bias, p.bias ? ebytes : 0), eoff, 0, 0));
  const f16 e_res = __builtin_bit_cast(
      f16, __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(p.residual, p.residual ? ebytes : 0), eoff, 0, 0));
  const f16 e_scale =
      SCALED ? (f16)1.0f
             : __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(pre_scales, ebytes), eoff, 0, 0));
  __builtin_amdgcn_sched_barrier(0);  // every load is in flight before the first wait
  if constexpr (FMT == FMT_NF4) {
    build_nf4_pair_table(nf4_table);
    __syncthreads();
  }

  // ---- arithmetic: R chains from -B ----
  h2 xp[4 * XL];
  const float bsum = line_pairs<FMT>(xv, xp);
  float v[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float a = line_dot<FMT>(w[r], xp, -bsum, nf4_table);
    if constexpr (SCALED && !QS) v[r] = (float)sc[r] * a;
    else v[r] = a;
  }

  // ---- row sums: a transposed reduction leaves row r's wave total in lanes r, r + 16, ... ----
  line_fold<0, R>(v, lane);
  line_fold<1, R / 2>(v, lane);
  if constexpr (SCALED && QS) {
#pragma unroll
    for (int i = 0; i < R / 4; ++i) v[i] *= (float)sc[i];
  }
  if constexpr (R >= 8) {
    line_fold<2, R / 4>(v, lane);
  } else {  // one value left: add lane ^ 4's copy (both moves under the full wave, then a select)
    float down = dpp_move<kDppRowRor4>(v[0]), up = dpp_move<kDppRowRor12>(v[0]);
    asm volatile("" : "+v"(down), "+v"(up));
    v[0] += ((lane >> 2) & 1) ? down : up;
  }
  if constexpr (R == 16) line_fold<3, 2>(v, lane);
  else v[0] += dpp_move<kDppRowRor8>(v[0]);
  v[0] += __shfl_xor(v[0], 16, 64);
  v[0] += __shfl_xor(v[0], 32, 64);
  if (lane < R) part[wave * R + lane] = v[0];
  __syncthreads();

  // ---- epilogue: segment sums in segment order, then the reference's staging ----
  if (wave == 0 && t < rows_wg && en < N) {
    const int g = t / R, r = t % R;
    float a = 0.0f;
    for (int s = 0; s < nseg; ++s) a += part[(g * nseg + s) * R + r];
    if constexpr (!SCALED) a *= (float)e_scale;
    f16 h = (f16)a;
    if (p.bias) h = (f16)((float)h + (float)e_bias);
    if (p.residual) h = (f16)((float)e_res + (float)h);
    p.y[en] = h;
  }
}

// Problems of one pack_gemv_kernel launch past the first: weights sharing the activation row, K and
// the group size (q|k|v, gate|up), each over its own range of waves.
constexpr int kPackMaxProblems = 3;
struct PackTable {
  const uint8_t *codes[kPackMaxProblems];
  const f16 *scales[kPackMaxProblems];
  f16 *y[kPackMaxProblems];
  const f16 *bias[kPackMaxProblems];
  const f16 *residual[kPackMaxProblems];
  int N[kPackMaxProblems];
  int wave_end[kPackMaxProblems];  // exclusive prefix sums of the problems' waves
};

// One-row GEMV for rows of at most 64 16-byte slots (up to 2048 INT4 / 1024 INT8 codes, the
// SmolLM shapes): the same lane-linear loads with whole rows packed across a wave's lanes.  A row
// of S slots takes S lanes, so P = 64 / S consecutive rows fill P S lanes of a wave-wide load
// (P S x 16 contiguous bytes; the SmolLM K = 576 INT4 rows: 3 rows in 54 lanes).  Lane l always
// holds slot l % S of its row, so its activations are loaded once and serve all R loads (R P rows
// per wave).  Each lane's partial per load is scaled by its group's scale (groups of at least CPL
// codes).  Where S is even (a multiple of 4), pairs (quads) of neighbouring slot partials are
// added by DPP first: a row's lanes start at an even (4-aligned) lane, so partners stay within
// the row, in the same order for every row.  The sums go to the wave's own LDS rows, contiguous
// per row, and lane q of the wave adds row q's in slot order.  Waves are independent: no barrier.
// Bias and residual loads are compiled in only with EPI (any present).  With NP > 1 problems the
// waves are dealt to the problems by the table's prefix sums (a wave's problem is uniform) and
// the activations are loaded first, while the problem's pointers arrive from the argument block;
// with one problem every pointer of the first loads is a preloaded argument.
template <int FMT, bool SCALED, int R, bool EPI, int NP>
__global__ __launch_bounds__(256) void pack_gemv_kernel(const f16 *pre_x, const uint8_t *pre_codes,
                                                        const f16 *pre_scales, int pre_N, int pre_K, int pre_G,
                                                        int pre_shift, StreamParams p, PackTable tab) {
  using TR = LineTraits<FMT>;
  constexpr int CPL = TR::CPL, XL = TR::XL;
  constexpr int kOutOfRange = (int)0x80000000u;
  constexpr int WAVES = 4;
  static_assert(NP >= 1 && NP <= kPackMaxProblems, "problems per launch");
  __shared__ float part[WAVES][R][64];

  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int K = pre_K;
  const int row_bytes = K * TR::BITS / 8;
  const int S = row_bytes >> 4;        // 16-byte slots per row (1 .. 64)
  const int P = 64 / S;                // rows per wave-wide load
  const int slot = lane % S, ro = lane / S;
  const bool live = ro < P;
  int gw = blockIdx.x * WAVES + wave;  // the wave's index within its problem
  const uint8_t *codes = pre_codes;
  const f16 *scales = pre_scales;
  f16 *y = p.y;
  const f16 *bias = p.bias, *residual = p.residual;
  int N = pre_N;

  // ---- loads: (NP > 1: activations first), scales, activations, epilogue operands, weights ----
  u4 xv[XL];
  auto load_x = [&] {
    const __amdgpu_buffer_rsrc_t xb = buffer_rsrc(pre_x, (size_t)K * 2);
#pragma unroll
    for (int i = 0; i < XL; ++i)
      xv[i] = __builtin_bit_cast(
          u4, __builtin_amdgcn_raw_buffer_load_b128(xb, live ? (slot * CPL + 8 * i) * 2 : kOutOfRange, 0, 0));
  };
  if constexpr (NP > 1) {
    load_x();
    const int j = (gw >= tab.wave_end[0]) + (NP > 2 && gw >= tab.wave_end[1]);
    gw -= j == 0 ? 0 : tab.wave_end[j - 1];
    codes = tab.codes[j];
    scales = tab.scales[j];
    y = tab.y[j];
    bias = tab.bias[j];
    residual = tab.residual[j];
    N = tab.N[j];
  }
  const int n0 = gw * R * P;              // first row of this wave
  const int rows = min(R * P, N - n0);    // <= 0 past N
  const size_t base_row = rows > 0 ? (size_t)n0 : 0;
  f16 sc[SCALED ? R : 1];
  if constexpr (SCALED) {
    const __amdgpu_buffer_rsrc_t sb = buffer_rsrc(scales + base_row * pre_G, rows > 0 ? (size_t)rows * pre_G * 2 : 0);
    const int gi = (slot * CPL) >> pre_shift;
#pragma unroll
    for (int u = 0; u < R; ++u)
      sc[u] = __builtin_bit_cast(
          f16, __builtin_amdgcn_raw_buffer_load_b16(sb, live ? ((u * P + ro) * pre_G + gi) * 2 : kOutOfRange, 0, 0));
  }
  if constexpr (NP == 1) load_x();
  const int en = n0 + lane;  // the epilogue row of lane q < R P
  const size_t ebytes = (size_t)N * 2;
  const int eoff = lane < R * P && en < N ? en * 2 : kOutOfRange;
  f16 e_bias = (f16)0.0f, e_res = (f16)0.0f;
  if constexpr (EPI) {  // an absent operand is an empty buffer (reads zeros)
    e_bias = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(bias, bias ? ebytes : 0), eoff, 0, 0));
    e_res = __builtin_bit_cast(
        f16, __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(residual, residual ? ebytes : 0), eoff, 0, 0));
  }
  const f16 e_scale =
      SCALED ? (f16)1.0f
             : __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(scales, ebytes), eoff, 0, 0));
  u4 w[R];
  {
    const __amdgpu_buffer_rsrc_t wb = buffer_rsrc(codes + base_row * row_bytes, rows > 0 ? (size_t)rows * row_bytes : 0);
#pragma unroll
    for (int u = 0; u < R; ++u)  // rows u P .. u P + P - 1 of the wave, contiguous
      w[u] = __builtin_bit_cast(
          u4, __builtin_amdgcn_raw_buffer_load_b128(wb, live ? u * P * row_bytes + lane * 16 : kOutOfRange, 0, 0));
  }
  __builtin_amdgcn_sched_barrier(0);  // every load is in flight before the first wait

  // ---- arithmetic: one chain per load from -B, scaled by the lane's group scale ----
  h2 xp[4 * XL];
  const float bsum = line_pairs<FMT>(xv, xp);
  const int lg = S % 4 == 0 ? 2 : S % 2 == 0 ? 1 : 0;  // log2 of the slots per LDS sum
#pragma unroll
  for (int u = 0; u < R; ++u) {
    const float a = line_dot<FMT>(w[u], xp, -bsum, nullptr);
    float v = SCALED ? (float)sc[u] * a : a;
    // Both moves under the full wave, then uniform selects.
    const float o1 = dpp_move<kDppXor1>(v);
    v = lg >= 1 ? v + o1 : v;
    const float o2 = dpp_move<kDppXor2>(v);
    v = lg == 2 ? v + o2 : v;
    if ((lane & ((1 << lg) - 1)) == 0) part[wave][u][lane >> lg] = v;
  }

  // ---- row sums: lane q adds row q's sums in slot order (the wave's own LDS rows) ----
  if (lane < R * P && en < N) {
    const int u = lane / P, r = lane % P;
    const float *src = &part[wave][u][(r * S) >> lg];
    float a = 0.0f;
    for (int c = 0; c < (S >> lg); ++c) a += src[c];
    if constexpr (!SCALED) a *= (float)e_scale;
    f16 h = (f16)a;
    if (EPI && bias) h = (f16)((float)h + (float)e_bias);
    if (EPI && residual) h = (f16)((float)e_res + (float)h);
    y[en] = h;
  }
}

}  // namespace lb
