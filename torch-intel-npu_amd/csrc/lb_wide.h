// gfx950 several-row GEMV for 2 .. 32 activation rows over INT4 / INT8 weights:
// y[M, N] = x[M, K] . (q * s)[N, K]^T with every weight code decoded once per launch.
//
// The product runs on v_mfma_f32_32x32x16_f16 with the activation rows as the A operand (32 rows:
// rows past M read a zero row, so M <= 32 costs one MFMA tile) and the decoded weights as the B
// operand (32 weight rows per wave).  A wave owns 32 consecutive weight rows; lane (col, half)
// holds weight row col and reads, per 16-byte load, the half-th 16 bytes of each 32-byte piece of
// the row, so one wave-wide load covers 32 rows x 32 bytes and four consecutive loads a 128-byte
// "position" of every row (256 INT4 / 128 INT8 codes).
//
// INT4 codes enter the MFMA as the fp16 value of a "magic" half-word, the sign-flipped nibble
// under the exponent of 1024 (one three-input bit operation per pair):
//   even codes  (c ^ 8) | 0x6400         = 1032 + q   (activation x)
//   odd codes   ((c ^ 8) << 4) | 0x6400  = 1152 + 16 q (activation x / 16, nibble in place)
// so the product sums x (bias + q).  The bias part, B = the staged activations dotted with the
// biases, is the same for every weight row: the staging computes it per activation row and scale
// group, and the group's MFMA accumulator starts at -B, which leaves sum x q up to fp32 rounding.
// INT8 bytes become the exact q in registers: (b ^ 0x80) | 0x6400 = 1152 + q, then - 1152 (exact
// fp16 arithmetic on small integers).
// Eight codes become the MFMA's eight k slots in the order (0,4,1,5,2,6,3,7) (INT4) or
// (0,2,1,3,4,6,5,7) (INT8); the activations are staged in LDS with the same permutation of every
// 8-element block, so both operands agree on k.  NF4 codes enter as their fp16 literals (no bias).
//
// Scales: a group's integer sums accumulate in their own MFMA accumulator (a group is two or more
// whole loads: 128+ INT4 / 64+ INT8 codes), then acc += s * group_sum in fp32 -- the exact
// x . (q * s) product up to fp32 rounding, whose distance to the reference's fp16(q * s) weights
// the reference's rounding-budget gate bounds (torch_npu_lowbit_demo.py:97-106), as for the other
// exact-q kernels.  Per-row INT8 accumulates all of K and multiplies once (the reference's W8
// value, torch_npu_smollm.py:153-157).
//
// Workgroups of kWideWaves waves own 32 weight rows each and one K slice (grid y), walked in chunks of PC
// positions: the chunk's activations of all M rows are staged once per workgroup in one of two
// LDS stages and serve the four waves; the next chunk's weights (registers) and activations are
// loaded while the current one is computed, one barrier per chunk.  With one slice the workgroup
// writes y; with several it writes fp32 partial sums [slice, M, N] that are added in slice order,
// by splitk_reduce_kernel or, with a zeroed counter per row block, by the row block's last
// workgroup (wide_add_slices).
#pragma once
#include "lb_common.h"

namespace lb {

struct WideParams {
  const f16 *x;           // [M, ldx]
  const uint8_t *codes;   // [N, K * bits / 8]
  const f16 *scales;      // [N, G]
  f16 *y;                 // [M, ldy] (one slice)
  float *partial;         // [slices, M, N] (several slices)
  const f16 *bias;        // [N] or null (one slice)
  int M, N, K, G, group_shift;
  int ldx, ldy;
  int kslice;             // codes per slice, a multiple of the chunk
  int per_row;            // INT8 with one scale per row: the scale multiplies the whole sum
  uint32_t *tickets;      // several slices: one zero counter per row block, the slices added in the
                          // kernel (null: splitk_reduce_kernel adds them in a launch of its own)
};

template <int FMT> struct WideTraits;
template <> struct WideTraits<FMT_INT4> { static constexpr int CPL = 32, BITS = 4; };
template <> struct WideTraits<FMT_INT8> { static constexpr int CPL = 16, BITS = 8; };
template <> struct WideTraits<FMT_NF4> { static constexpr int CPL = 32, BITS = 4; };

#ifndef LB_WIDE_WAVES
#define LB_WIDE_WAVES 8
#endif
constexpr int kWideWaves = LB_WIDE_WAVES;
constexpr int kWideRows = 32 * kWideWaves;  // weight rows per workgroup
constexpr int kWideLoads = 4;               // 16-byte loads per lane per position (128 bytes of a row)

template <int FMT> constexpr int wide_position() { return kWideLoads * 2 * WideTraits<FMT>::CPL; }

#ifndef LB_WIDE_TAIL_BATCH
#define LB_WIDE_TAIL_BATCH 4  // slices whose partials the adding workgroup requests at once
#endif
// The K slices added in the kernel.  Every workgroup of a row block writes its fp32 partial sums
// with system-scope coherent stores (sc0 sc1: written through to memory, as a relaxed system-scope
// atomic store is), waits until they are complete, and counts itself in the block's ticket with a
// returning system-scope atomic.  The workgroup that counts last reads every slice's partials with
// system-scope coherent loads, adds them in slice order starting from 0.0f -- the order and the
// values of splitk_reduce_kernel, so y is the same bit for bit -- applies the epilogue, and returns
// the ticket to zero for the next call.  No workgroup waits for another, and every access to the
// partials is coherent in itself, so no cache-wide write-back or invalidate is needed (agent-scope
// release / acquire fences around the count measured 12-14 us more per call).  The lane (col, half)
// holds rows m = 8 (r / 4) + 4 half + r % 4 of weight row row0 + col; N is a multiple of 4 (the host
// launches this form only then).
__device__ __forceinline__ void wide_add_slices(const WideParams &p, const f16x &acc, int col, int half, int row0,
                                                int rows) {
  constexpr int NT = 64 * kWideWaves;
  constexpr int QUADS = kWideRows / 4;          // 4-row pieces of an activation row in a block
  constexpr int PT = (32 * QUADS + NT - 1) / NT;  // pieces per thread (32 activation rows)
  constexpr int kOutOfRange = (int)0x80000000u;
  __shared__ uint32_t last;
  const int S = gridDim.y;
  const __amdgpu_buffer_rsrc_t pb = buffer_rsrc(p.partial, (size_t)S * p.M * p.N * 4);
  if (col < rows) {
    const int base = blockIdx.y * p.M * p.N + row0 + col;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = 8 * (r >> 2) + 4 * half + (r & 3);
      const float v = acc[r];  // a value first: a bit cast of the vector element itself read element 0
      if (m < p.M) __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), pb, (base + m * p.N) * 4, 0, kSysCoherent);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's partials are written through
  __syncthreads();
  if (threadIdx.x == 0)
    last = __hip_atomic_fetch_add(p.tickets + blockIdx.x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) ==
           (uint32_t)(S - 1);
  __syncthreads();
  if (!last) return;
  if (threadIdx.x == 0) __hip_atomic_store(p.tickets + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  const int nb0 = blockIdx.x * kWideRows;
  const int quads = min(kWideRows, p.N - nb0) / 4;
  f4 sum[PT];
#pragma unroll
  for (int i = 0; i < PT; ++i) sum[i] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  // SB slices' loads in flight per piece; a slice past S reads zeros, and adding +0.0f leaves
  // every sum as it is (a sum that starts at +0.0f is never -0.0f).
  constexpr int SB = LB_WIDE_TAIL_BATCH;
  for (int s0 = 0; s0 < S; s0 += SB) {
    f4 v[PT][SB];
#pragma unroll
    for (int i = 0; i < PT; ++i) {
      const int idx = i * NT + (int)threadIdx.x, m = idx / QUADS, q = idx - m * QUADS;
      const bool live = m < p.M && q < quads;
#pragma unroll
      for (int e = 0; e < SB; ++e) {
        const int off = live && s0 + e < S ? (((s0 + e) * p.M + m) * p.N + nb0 + 4 * q) * 4 : kOutOfRange;
        v[i][e] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(pb, off, 0, kSysCoherent));
      }
    }
#pragma unroll
    for (int i = 0; i < PT; ++i)
#pragma unroll
      for (int e = 0; e < SB; ++e)
#pragma unroll
        for (int c = 0; c < 4; ++c) sum[i][c] += v[i][e][c];
  }
#pragma unroll
  for (int i = 0; i < PT; ++i) {
    const int idx = i * NT + (int)threadIdx.x, m = idx / QUADS, q = idx - m * QUADS;
    if (m >= p.M || q >= quads) continue;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int n = nb0 + 4 * q + c;
      float v = sum[i][c];
      if (p.per_row) v *= (float)p.scales[n];
      f16 h = (f16)v;
      if (p.bias) h = (f16)((float)h + (float)p.bias[n]);
      p.y[(size_t)m * p.ldy + n] = h;
    }
  }
}

// B operand of one 32x32x16 MFMA: the exact codes q of 8 k slots from the 16-byte load w (INT4:
// dword t; INT8: dwords 2t, 2t + 1).
template <int FMT>
__device__ __forceinline__ h8 wide_decode(const u4 &w, int t, const uint32_t *nf4_table) {
  if constexpr (FMT == FMT_NF4) {  // each byte's two fp16 literals from the LDS table, natural order
    const uint32_t v = w[t];
    const h2 p0 = as_h2(nf4_table[v & 0xFFu]), p1 = as_h2(nf4_table[(v >> 8) & 0xFFu]);
    const h2 p2 = as_h2(nf4_table[(v >> 16) & 0xFFu]), p3 = as_h2(nf4_table[v >> 24]);
    return __builtin_shufflevector(__builtin_shufflevector(p0, p1, 0, 1, 2, 3), __builtin_shufflevector(p2, p3, 0, 1, 2, 3),
                                   0, 1, 2, 3, 4, 5, 6, 7);
  }
  uint32_t r[4];
  if constexpr (FMT == FMT_INT4) {
    const uint32_t a = w[t], b = a >> 8;
    r[0] = (a & 0x000F000Fu) ^ 0x64086408u;  // c0, c4: 1032 + q
    r[1] = (a & 0x00F000F0u) ^ 0x64806480u;  // c1, c5: 1152 + 16 q
    r[2] = (b & 0x000F000Fu) ^ 0x64086408u;  // c2, c6
    r[3] = (b & 0x00F000F0u) ^ 0x64806480u;  // c3, c7
  } else {  // INT8: the exact q (the bias removed here; it measured faster than a staged bias)
    const uint32_t a = w[2 * t] ^ 0x80808080u, b = w[2 * t + 1] ^ 0x80808080u;
    r[0] = (a & 0x00FF00FFu) | 0x64006400u;         // b0, b2: 1152 + q
    r[1] = ((a >> 8) & 0x00FF00FFu) | 0x64006400u;  // b1, b3
    r[2] = (b & 0x00FF00FFu) | 0x64006400u;         // b4, b6
    r[3] = ((b >> 8) & 0x00FF00FFu) | 0x64006400u;  // b5, b7
    const h2 bias = {(f16)-1152.0f, (f16)-1152.0f};
    const h2 p0 = as_h2(r[0]) + bias, p1 = as_h2(r[1]) + bias, p2 = as_h2(r[2]) + bias, p3 = as_h2(r[3]) + bias;
    return __builtin_shufflevector(__builtin_shufflevector(p0, p1, 0, 1, 2, 3), __builtin_shufflevector(p2, p3, 0, 1, 2, 3),
                                   0, 1, 2, 3, 4, 5, 6, 7);
  }
  return __builtin_bit_cast(h8, u4{r[0], r[1], r[2], r[3]});
}

// Bias part of one staged INT4 block (slot order) against the magic codes: 1032 for the even
// codes' slots, 1152 for the odd ones (which hold x / 16).
__device__ __forceinline__ float wide_block_bias(const h8 &v) {
  const float even = ((float)v[0] + (float)v[1]) + ((float)v[4] + (float)v[5]);
  const float odd = ((float)v[2] + (float)v[3]) + ((float)v[6] + (float)v[7]);
  return 1032.0f * even + 1152.0f * odd;
}

// Sum over aligned groups of N consecutive lanes (4 .. 64), in every lane of the group; every lane
// active.  DPP: quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror, row_mirror; then lane swaps.
template <int CTRL>
__device__ __forceinline__ float wide_dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
template <int N>
__device__ __forceinline__ float wide_group_sum(float v) {
  static_assert(N == 4 || N == 8 || N == 16 || N == 32 || N == 64, "group of 4 .. 64 lanes");
  v += wide_dpp<0xB1>(v);
  v += wide_dpp<0x4E>(v);
  if constexpr (N >= 8) v += wide_dpp<0x141>(v);
  if constexpr (N >= 16) v += wide_dpp<0x140>(v);
  if constexpr (N >= 32) v += __shfl_xor(v, 16, 64);
  if constexpr (N >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

// Activation block permutation matching wide_decode: slot e holds element perm[e].
// INT4: the odd codes' slots (2, 3, 6, 7) hold x / 16 (exact: a power of two).
template <int FMT>
__device__ __forceinline__ h8 wide_permute(h8 v) {
  if constexpr (FMT == FMT_INT4) {
    h8 p = __builtin_shufflevector(v, v, 0, 4, 1, 5, 2, 6, 3, 7);
    const h2 sixteenth = {(f16)0.0625f, (f16)0.0625f};
    const h2 o0 = h2{p[2], p[3]} * sixteenth, o1 = h2{p[6], p[7]} * sixteenth;
    p[2] = o0[0]; p[3] = o0[1]; p[6] = o1[0]; p[7] = o1[1];
    return p;
  } else if constexpr (FMT == FMT_NF4) {
    return v;
  } else {
    return __builtin_shufflevector(v, v, 0, 2, 1, 3, 4, 6, 5, 7);
  }
}

// GL: loads per scale group (2, 4, 8; 0 for per-row INT8).  PC: positions per chunk.  PD:
// chunks of weights in flight (register buffers; chunk c + PD - 1 is requested while chunk c runs).
// The operands of the first loads come as leading scalar arguments (pre_*, the same values as in
// p), which the build preloads into registers at wave launch: a workgroup dispatched while earlier
// ones flood the memory system would otherwise wait for its argument block before its first load.
template <int FMT, int GL, int PC, int PD>
__global__ __launch_bounds__(64 * kWideWaves) void wide_rows_kernel(const uint8_t *pre_codes, const f16 *pre_x,
                                                                    const f16 *pre_scales, int pre_M, int pre_N,
                                                                    int pre_K, int pre_G, int pre_shift, int pre_ldx,
                                                                    int pre_kslice, WideParams p) {
  constexpr int CPL = WideTraits<FMT>::CPL, BITS = WideTraits<FMT>::BITS;
  constexpr int POS = wide_position<FMT>();  // codes per position
  constexpr int KC = PC * POS;                // codes per chunk
  constexpr int NL = PC * kWideLoads;         // loads per lane per chunk
  constexpr int T8 = CPL / 8;                 // MFMAs per load
  constexpr int LD = KC + 8;                  // staged row stride in halves (+16 bytes: rows spread over banks)
  constexpr int NT = 64 * kWideWaves;
  constexpr int XPIECES = 32 * KC / 8;        // 16-byte activation pieces of a chunk (32 rows)
  constexpr int XP = (XPIECES + NT - 1) / NT; // per thread
  constexpr bool GROUPED = GL > 0;
  constexpr int GPC = GROUPED ? NL / GL : 1;  // scale groups per chunk
  constexpr int kOutOfRange = (int)0x80000000u;
  static_assert(!GROUPED || (NL % GL == 0), "a chunk holds whole groups");
  static_assert(PD >= 2, "at least the next chunk in flight");
  // Staged pieces of one activation row per scale group (INT4, where the bias is staged):
  // consecutive threads hold consecutive pieces of a row, a group aligned to PPG lanes.
  constexpr bool BIASED = FMT == FMT_INT4;
  constexpr int PPG = GROUPED ? GL * 2 * CPL / 8 : KC / 8;  // a load covers 2 CPL codes of a row
  static_assert(!BIASED || GROUPED, "INT4 weights have scale groups");
  static_assert(!BIASED || (PPG <= 64 && NT % (KC / 8) == 0 && (KC / 8) % PPG == 0), "bias groups within a wave");
  __shared__ __align__(16) f16 xs[2 * 32 * LD + LD];  // two stages, then a zero row
  __shared__ __align__(16) float nbs[BIASED ? 2 * GPC * 32 : 4];  // -B per stage, group of the chunk, activation row
  __shared__ uint32_t nf4_table[FMT == FMT_NF4 ? 256 : 1];

  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int col = lane & 31, half = lane >> 5;
  const int row0 = blockIdx.x * kWideRows + wave * 32;  // this wave's first weight row
  const int rows = __builtin_amdgcn_readfirstlane(max(0, min(32, pre_N - row0)));  // scalar: the descriptors stay uniform
  const int kbeg = blockIdx.y * pre_kslice;
  const int chunks = min(pre_kslice, pre_K - kbeg) / KC;
  const int row_bytes = pre_K * BITS / 8;
  const __amdgpu_buffer_rsrc_t wb =
      buffer_rsrc(pre_codes + (size_t)(rows > 0 ? row0 : 0) * row_bytes, (size_t)rows * row_bytes);
  const __amdgpu_buffer_rsrc_t sb =
      buffer_rsrc(pre_scales + (size_t)(rows > 0 ? row0 : 0) * pre_G, GROUPED ? (size_t)rows * pre_G * 2 : 0);
  // Lane's byte offset of load l of a chunk at k: row col, piece 32 * l + 16 * half of the chunk.
  const int lane_off = col * row_bytes + 16 * half;

  struct Buf {
    u4 w[NL];
    uint32_t s[GPC];
  };
  auto issue = [&](Buf &b, int c) {
    const int kb = (kbeg + c * KC) * BITS / 8;
#pragma unroll
    for (int l = 0; l < NL; ++l)
      b.w[l] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(wb, lane_off + kb + 32 * l, 0, 0));
    if constexpr (GROUPED) {
      const int g0 = (kbeg + c * KC) >> pre_shift;
#pragma unroll
      for (int q = 0; q < GPC; ++q)
        b.s[q] = __builtin_amdgcn_raw_buffer_load_b16(sb, (col * pre_G + g0 + q) * 2, 0, 0);
    }
  };
  // Activation pieces of chunk c: piece i = (row m, 8-element block); rows past M are not staged.
  const __amdgpu_buffer_rsrc_t xb = buffer_rsrc(pre_x, ((size_t)(pre_M - 1) * pre_ldx + pre_K) * 2);
  auto load_x = [&](u4 (&xv)[XP], int c) {
#pragma unroll
    for (int i = 0; i < XP; ++i) {
      const int idx = i * NT + t;
      const int m = idx / (KC / 8), blk = idx % (KC / 8);
      const bool live = idx < XPIECES && m < pre_M;
      xv[i] = __builtin_bit_cast(
          u4, __builtin_amdgcn_raw_buffer_load_b128(xb, live ? (m * pre_ldx + kbeg + c * KC + 8 * blk) * 2 : kOutOfRange,
                                                    0, 0));
    }
  };
  // Staged pieces, and each (row, group) bias sum B negated into nbs (every lane takes part in the
  // group sums: pieces past M or the chunk were loaded as zeros).
  auto store_x = [&](const u4 (&xv)[XP], int st) {
#pragma unroll
    for (int i = 0; i < XP; ++i) {
      const int idx = i * NT + t;
      const int m = idx / (KC / 8), blk = idx % (KC / 8);
      const bool live = idx < XPIECES && m < pre_M;
      const h8 v = wide_permute<FMT>(__builtin_bit_cast(h8, xv[i]));
      if (live) *reinterpret_cast<h8 *>(xs + st * 32 * LD + m * LD + 8 * blk) = v;
      if constexpr (BIASED) {
        const float b = wide_group_sum<PPG>(wide_block_bias(v));
        if (live && blk % PPG == 0) nbs[(st * GPC + blk / PPG) * 32 + m] = -b;
      }
    }
  };

  // Loads complete in issue order, so every activation load is issued before the weight loads
  // that may still be in flight when its staging waits for it.
  Buf buf[PD];
  u4 xv[XP];
  if (chunks > 0) load_x(xv, 0);
#pragma unroll
  for (int u = 0; u < PD - 1; ++u)
    if (u < chunks) issue(buf[u], u);
  for (int i = t; i < LD / 8; i += NT) *reinterpret_cast<h8 *>(xs + 2 * 32 * LD + 8 * i) = h8{};
  if constexpr (BIASED) {  // rows past M (never staged) start their groups at 0
    for (int i = t; i < 2 * GPC * 32; i += NT)
      if ((i & 31) >= pre_M) nbs[i] = 0.0f;
  }
  if (chunks > 0) store_x(xv, 0);
  if constexpr (FMT == FMT_NF4) build_nf4_pair_table(nf4_table);  // complete at the barrier below
  __syncthreads();

  // A operand of lane (col, half): activation row col (or the zero row), k piece half.
  const bool arow = col < pre_M;
  const int a_base = (arow ? col * LD : 2 * 32 * LD) + half * CPL;
  f16x acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.0f;

  // The lane's 16 accumulator rows m = 8 (r / 4) + 4 half + r % 4: four runs of 4 consecutive rows.
  auto bias_start = [&](int stage, int grp) {
    f16x c0;
    const float *nb = nbs + (stage * GPC + grp) * 32 + 4 * half;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f4 v = *reinterpret_cast<const f4 *>(nb + 8 * q);
#pragma unroll
      for (int e = 0; e < 4; ++e) c0[4 * q + e] = v[e];
    }
    return c0;
  };
  auto step = [&](Buf &b, int stage) {
    const f16 *xa = xs + a_base + (arow ? stage * 32 * LD : 0);
    f16x part;
#pragma unroll
    for (int l = 0; l < NL; ++l) {
      asm volatile("" : "+v"(b.w[l]));  // decode here, not at the load
#pragma unroll
      for (int q = 0; q < T8; ++q) {
        const h8 bw = wide_decode<FMT>(b.w[l], q, nf4_table);
        const h8 xa8 = *reinterpret_cast<const h8 *>(xa + 2 * CPL * l + 8 * q);
        if constexpr (GROUPED) {
          if (l % GL == 0 && q == 0) {
            f16x start;
            if constexpr (BIASED) {
              start = bias_start(stage, l / GL);
            } else {
#pragma unroll
              for (int r = 0; r < 16; ++r) start[r] = 0.0f;
            }
            part = __builtin_amdgcn_mfma_f32_32x32x16_f16(xa8, bw, start, 0, 0, 0);
          } else {
            part = __builtin_amdgcn_mfma_f32_32x32x16_f16(xa8, bw, part, 0, 0, 0);
          }
        } else {
          acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(xa8, bw, acc, 0, 0, 0);
        }
      }
      if constexpr (GROUPED) {
        if (l % GL == GL - 1) {
          const float s = (float)__builtin_bit_cast(f16, (unsigned short)b.s[l / GL]);
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[r] = __builtin_fmaf(s, part[r], acc[r]);
          __builtin_amdgcn_sched_barrier(0);  // one group's accumulator at a time
        }
      }
    }
  };
  // Chunk c runs from buffer c % PD and stage c % 2; chunk c + 1's activations and chunk c + PD - 1's
  // weights are requested before it, the activations stored into the other stage after it.
  for (int c = 0; c < chunks; c += PD) {
#pragma unroll
    for (int u = 0; u < PD; ++u) {
      const int cc = c + u;
      if (cc < chunks) {
        if (cc + 1 < chunks) load_x(xv, cc + 1);
        if (cc + PD - 1 < chunks) issue(buf[(u + PD - 1) % PD], cc + PD - 1);
        step(buf[u], cc & 1);
        if (cc + 1 < chunks) store_x(xv, (cc + 1) & 1);
        __syncthreads();
      }
    }
  }

  // Lane (col, half) holds rows m = 8 (r / 4) + 4 half + r % 4 of weight row row0 + col.
  const int n = row0 + col;
  if (gridDim.y > 1 && p.tickets) {
    wide_add_slices(p, acc, col, half, row0, rows);
    return;
  }
  if (col >= rows) return;
  if (gridDim.y > 1) {
    float *part = p.partial + (size_t)blockIdx.y * p.M * p.N + n;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = 8 * (r >> 2) + 4 * half + (r & 3);
      if (m < p.M) part[(size_t)m * p.N] = acc[r];
    }
    return;
  }
  const float rs = p.per_row ? (float)p.scales[n] : 1.0f;
  const float bias = p.bias ? (float)p.bias[n] : 0.0f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int m = 8 * (r >> 2) + 4 * half + (r & 3);
    if (m >= p.M) continue;
    f16 h = (f16)(p.per_row ? acc[r] * rs : acc[r]);
    if (p.bias) h = (f16)((float)h + bias);
    p.y[(size_t)m * p.ldy + n] = h;
  }
}

}  // namespace lb

namespace lb {

// Positions per chunk and chunks of weights in flight of the launched kernels (two buffers, the next
// chunk requested while one runs: against three, INT4 g128 M = 32 14336x4096 18.9 -> 18.1 us, M = 24
// 17.7 -> 16.9 us, 4096x14336 22.4 -> 21.8 us, NF4 M = 32 21.9 -> 19.9 us, the head and per-row
// INT8 unchanged; four measured 10-25% slower).
#ifndef LB_WIDE_PD
#define LB_WIDE_PD 2
#endif
constexpr int kWidePC = 2, kWidePD = LB_WIDE_PD;
template <int FMT> constexpr int wide_chunk() { return kWidePC * wide_position<FMT>(); }
inline int wide_chunk_codes(int fmt) { return fmt == FMT_INT8 ? wide_chunk<FMT_INT8>() : wide_chunk<FMT_INT4>(); }

// Launches wide_rows_kernel over ceil(N / 128) x `slices` workgroups; gl: loads per scale group
// (0: per-row INT8).  Defined in wide_abi.hip.
void launch_wide(const WideParams &p, int format, int gl, int slices, hipStream_t stream);

}  // namespace lb
