// One SmolLM decoder layer for one token in one launch (lb_decode_layer).
//
// The five launches of the fused decode step (RMSNorm -> q|k|v, RoPE + attention, o + residual,
// RMSNorm -> gate|up, SiLU * up -> down + residual) become workgroup roles of one grid, in this
// dispatch order:
//
//   T_QKV  q | k | v tiles (16 rows each)            ATTN   RoPE, KV append, attention (head, dims)
//   T_O    o projection + residual                   T_GU   gate | up
//   Z_D    correction activations z of down          T_D    down projection + residual
//
// A tile over K <= 640 computes its problem's correction activations z = fp16(x'.V^T) itself from
// V rows fetched at launch (8 threads per rank); the down projection (K up to 1536) takes z from
// the Z_D workgroups instead, whose V slices stay small.
//
// A role hands its output to later roles through the workspace as tagged 64-bit words (two fp16
// values and the launch's 16-bit tag; the correction activations three to a word), written and
// read with system-scope atomics, which are performed at the memory side past the per-XCD L2s.
// A consumer waits (bounded) on one word of its source, chosen by its workgroup index so the
// consumers of a stage poll different addresses, then reads the words it needs and re-reads any
// whose tag is not yet current.  Every
// workgroup issues its weight, scale, U-row and KV-cache loads at launch, so while it waits its
// data arrives.  A workgroup only ever waits for workgroups of earlier roles, which the hardware
// dispatches before it, so every wait ends.
//
// The launch's tag is (passed / workgroups + 1) mod 2^16: every workgroup reads `passed` at its
// start and raises it once at its end, so at any start it holds launch * workgroups plus fewer
// than `workgroups`, and no word is ever cleared (the previous launch's tag is one behind).
//
// Arithmetic and fp16 rounding points are those of the fused decode kernels (the reference's
// CPU layer, torch_npu_smollm.py:142-193): the prologues, the MFMA products with fp32
// accumulation, z = fp16(x'.V^T), d = fp16(z.U^T), y = fp16(fp16(main) + d), the residual adds,
// and the attention staging of decode_attention_kernel.
#pragma once
#include "lb_decode.h"

namespace lb {

enum LayerRole { R_TQKV, R_ATTN, R_TO, R_TGU, R_ZD, R_TD, R_COUNT };
enum LayerProj { P_Q, P_K, P_V, P_O, P_GATE, P_UP, P_DOWN, P_COUNT };
enum LayerSource { SRC_H, SRC_ATT, SRC_H1, SRC_GU };

// Device addresses of one layer's tensors (read by every role of that layer).
struct LayerWeights {
  const uint8_t *codes[P_COUNT];  // packed codes [N, K] (fp16 weights for FMT_FP16)
  const f16 *scales[P_COUNT];     // [N, G]
  const f16 *down[P_COUNT];       // V [rank, K] or null
  const f16 *up[P_COUNT];         // U [N, up_ld] or null
  const f16 *norm1, *norm2;       // [hidden] RMSNorm weights
  f16 *keys, *values;             // [kv_heads, capacity, 64]
};

struct LayerParams {
  f16 *h;                   // [hidden] residual row: the first layer's input, overwritten by the last layer's output
  float eps;
  int hidden, inter;        // K of q/k/v/o/gate/up, K of down
  int G1, shift1, G2, shift2, per_row;
  int N[P_COUNT], rank[P_COUNT], up_ld[P_COUNT];  // the same in every layer
  const f16 *cos, *sin;     // [capacity, 64]
  const int64_t *position;  // device scalar: the slot of the new token
  int heads, kv_heads, capacity;
  float scale;
  uint64_t *ws;             // workspace words: [0] passed, [1] timeout, then one region per layer
  int layers, layer_words;  // layers of the launch, words per layer region
  int w_z, w_qkv, w_att, w_h1, w_gu, w_h;  // word offsets within a layer's region
  int end[R_COUNT];         // exclusive prefix sums of workgroups per role
  LayerWeights w;           // the layer of a single-layer launch (lb_decode_layer)
};

constexpr int kLayerHeaderWords = 8;

// Entry i of a per-projection array by a chain of selects (i is wave-uniform), so no array of the
// kernel parameters is indexed at run time (which would make the compiler copy them to scratch).
template <class T, int N>
__device__ __forceinline__ T pick(const T (&a)[N], int i) {
  T v = a[0];
#pragma unroll
  for (int q = 1; q < N; ++q) v = i == q ? a[q] : v;
  return v;
}

// Where one layer's words live: its region (word index into the workspace), the next layer's
// region (whose h words receive this layer's output; -1 for the last layer, which writes h), and
// whether the layer input is the plain row h (the first layer) or the previous layer's h words.
struct LayerCtx {
  int lw, nw;
  bool first;
};

constexpr int kLayerSpinLimit = 1 << 18;
constexpr int kLayerZWords = 32;  // z words per problem: one rank per z workgroup and word
constexpr int kLayerTileSmem = 9216;  // dynamic LDS bytes a tile role may use (the launch gives at least this)

__device__ __forceinline__ uint64_t sys_load(const uint64_t *a) {
  return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void sys_store(uint64_t *a, uint64_t v) {
  __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ uint32_t word_tag(uint64_t w) { return (uint32_t)(w & 0xFFFF); }
__device__ __forceinline__ f16 word_half(uint64_t w, int e) {
  return __builtin_bit_cast(f16, (uint16_t)(w >> (16 * (e + 1))));
}
__device__ __forceinline__ uint64_t pair_word(uint32_t tag, f16 a, f16 b) {
  return (uint64_t)tag | ((uint64_t)__builtin_bit_cast(uint16_t, a) << 16) |
         ((uint64_t)__builtin_bit_cast(uint16_t, b) << 32);
}

// The launch's tag from `passed` as read at the workgroup's start.
__device__ __forceinline__ uint32_t layer_tag(const LayerParams &p, uint64_t passed) {
  return (uint32_t)((passed / (uint32_t)p.end[R_COUNT - 1] + 1) & 0xFFFF);
}

__device__ __forceinline__ void layer_timeout(const LayerParams &p) {
  __hip_atomic_store(reinterpret_cast<uint32_t *>(p.ws + 1), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// A word whose tag is current (bounded wait; a timeout is recorded and the stale word returned).
// The retry loop is kept rolled and out of line (unlikely branch), so the straight-line code a
// workgroup executes stays short.
__device__ __forceinline__ uint64_t wait_word(const LayerParams &p, const uint64_t *a, uint32_t tag) {
  uint64_t w = sys_load(a);
  if (__builtin_expect(word_tag(w) != tag, 0)) {
#pragma nounroll
    for (int it = 0; word_tag(w) != tag; ++it) {
      // Give up at the limit, or at once after any wait of the launch timed out (checked every 64
      // polls), so a launch whose waits fail still ends promptly.
      if (it == kLayerSpinLimit || ((it & 63) == 63 && (uint32_t)sys_load(p.ws + 1) != 0u)) {
        layer_timeout(p);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
      w = sys_load(a);
    }
  }
  return w;
}

// Thread 0 waits for the sentinel word, then the whole workgroup proceeds.
__device__ __forceinline__ void wait_sentinel(const LayerParams &p, const uint64_t *a, uint32_t tag) {
  if (threadIdx.x == 0) (void)wait_word(p, a, tag);
  __syncthreads();
}

// The workspace as a buffer over the header and every layer region.
// Built from readfirstlane copies, so the descriptor stays in scalar registers after the
// divergent wait that precedes its use.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t workspace_rsrc(const LayerParams &p) {
  const uint64_t a = reinterpret_cast<uint64_t>(p.ws);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a), hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  const uint32_t words = __builtin_amdgcn_readfirstlane((uint32_t)(kLayerHeaderWords + p.layers * p.layer_words));
  return buffer_rsrc(reinterpret_cast<const uint64_t *>(((uint64_t)hi << 32) | lo), (size_t)words * 8);
}

// Words [word, word + 4) (word even) with two 16-byte loads issued back to back; an offset of
// kOutOfRange reads zeros.
__device__ __forceinline__ void load_words4(__amdgpu_buffer_rsrc_t wb, int byte_off, uint64_t (&w)[4]) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const u4 v = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(wb, byte_off < 0 ? byte_off : byte_off + 16 * h, 0, kSysCoherent));
    w[2 * h] = (uint64_t)v[0] | ((uint64_t)v[1] << 32);
    w[2 * h + 1] = (uint64_t)v[2] | ((uint64_t)v[3] << 32);
  }
}

// Makes the four words current: when any is stale, waits (bounded) for the first stale one, then
// re-reads the four in one round trip (consecutive words come from one producer, so they are
// current together), and only a word still stale after that is waited for on its own.
__device__ __forceinline__ void settle_words4(const LayerParams &p, __amdgpu_buffer_rsrc_t wb, int byte_off,
                                              const uint64_t *a, uint32_t tag, uint64_t (&w)[4]) {
  int first = -1;
#pragma unroll
  for (int q = 3; q >= 0; --q)
    if (word_tag(w[q]) != tag) first = q;
  if (__builtin_expect(first >= 0, 0)) {
    (void)wait_word(p, a + first, tag);
    load_words4(wb, byte_off, w);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (__builtin_expect(word_tag(w[q]) != tag, 0)) w[q] = wait_word(p, a + q, tag);
  }
}

__device__ __forceinline__ h8 words4_to_h8(const uint64_t (&w)[4]) {
  h8 v;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    v[2 * q] = word_half(w[q], 0);
    v[2 * q + 1] = word_half(w[q], 1);
  }
  return v;
}

// The source row of a role's products (K values, 8 per block, thread t holding blocks t + 256 i)
// and the prologue's second row (gamma, or the up half for SiLU-multiply).  Every word of the
// thread is requested at once; a quad with a stale word is re-read once that word is current.
template <int XB>
__device__ __forceinline__ void layer_source_row(const LayerParams &p, int base, int src, int K, uint32_t tag,
                                                 h8 (&xv)[XB], h8 (&av)[XB]) {
  constexpr int kOutOfRange = (int)0x80000000u;
  const int t = threadIdx.x, blocks = K >> 3;
  const int second = base + p.inter / 2;
  const __amdgpu_buffer_rsrc_t wb = workspace_rsrc(p);
  uint64_t wx[XB][4], wa[XB][4];
#pragma unroll
  for (int i = 0; i < XB; ++i) {
    const int b = t + 256 * i;
    load_words4(wb, b < blocks ? (base + 4 * b) * 8 : kOutOfRange, wx[i]);
    if (src == SRC_GU) load_words4(wb, b < blocks ? (second + 4 * b) * 8 : kOutOfRange, wa[i]);
  }
#pragma unroll
  for (int i = 0; i < XB; ++i) {
    const int b = t + 256 * i;
    if (b < blocks) {
      settle_words4(p, wb, (base + 4 * b) * 8, p.ws + base + 4 * b, tag, wx[i]);
      xv[i] = words4_to_h8(wx[i]);
      if (src == SRC_GU) {
        settle_words4(p, wb, (second + 4 * b) * 8, p.ws + second + 4 * b, tag, wa[i]);
        av[i] = words4_to_h8(wa[i]);
      }
    } else {
      xv[i] = h8{};
      if (src == SRC_GU) av[i] = h8{};
    }
  }
}

// The word a consumer of a word source polls before reading the rest: one chosen by the
// workgroup's index, so the consumers of a stage spread their polls over the stage's words
// instead of all polling one address.
__device__ __forceinline__ const uint64_t *source_sentinel(const LayerParams &p, int base, int src) {
  const int words = src == SRC_GU ? p.inter : p.hidden / 2;
  return p.ws + base + (int)((blockIdx.x * 37u) % (unsigned)words);
}

// The word index of a source's region in this layer, or -1 for the plain row h (first layer input).
__device__ __forceinline__ int source_base(const LayerParams &p, const LayerCtx &c, int src) {
  if (src == SRC_H) return c.first ? -1 : c.lw + p.w_h;
  return c.lw + (src == SRC_ATT ? p.w_att : src == SRC_H1 ? p.w_h1 : p.w_gu);
}

__device__ __forceinline__ float layer_inv(int prologue, int K, float eps, float sumsq_total) {
  return prologue == PRO_RMSNORM ? 1.0f / sqrtf(sumsq_total / (float)K + eps) : 1.0f;
}

// RMS of the source row with the fused kernels' order (thread, wave, four waves).
template <int XB>
__device__ __forceinline__ float layer_prologue_inv(int prologue, int K, float eps, const h8 (&xv)[XB], float *wsum) {
  if (prologue != PRO_RMSNORM) return 1.0f;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < XB; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) s += (float)xv[i][e] * (float)xv[i][e];
  s = wave_sum(s);
  if (lane == 0) wsum[wave] = s;
  __syncthreads();
  const float total = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
  return layer_inv(prologue, K, eps, total);
}

__device__ __forceinline__ h8 layer_prologue_apply(int prologue, const h8 &x, const h8 &a, float inv) {
  h8 v;
  if (prologue == PRO_RMSNORM) {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (f16)((float)(f16)((float)x[e] * inv) * (float)a[e]);
  } else if (prologue == PRO_SILU_MUL) {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (f16)((float)(f16)silu_fast((float)x[e]) * (float)a[e]);
  } else {
    v = x;
  }
  return v;
}

// The source, prologue and K of each GEMV role, by its source (a template argument, so every
// role body is compiled for its own source and prologue): q|k|v read h, o the attention output,
// gate|up h1, down (and its z) the gate|up words.
struct RoleShape {
  int src, prologue, K;
  const f16 *gamma;
};
template <int SRC>
__device__ __forceinline__ RoleShape role_shape(const LayerParams &p, const LayerWeights &W) {
  if constexpr (SRC == SRC_H) return {SRC_H, PRO_RMSNORM, p.hidden, W.norm1};
  else if constexpr (SRC == SRC_ATT) return {SRC_ATT, PRO_NONE, p.hidden, nullptr};
  else if constexpr (SRC == SRC_H1) return {SRC_H1, PRO_RMSNORM, p.hidden, W.norm2};
  else return {SRC_GU, PRO_SILU_MUL, p.inter, nullptr};
}

// Loads the plain source row (the layer input h) and the prologue's gamma row, straight-line.
template <int XB>
__device__ __forceinline__ void layer_plain_loads(const LayerParams &p, const LayerCtx &c, const RoleShape &rs,
                                                  h8 (&xv)[XB], h8 (&av)[XB]) {
  constexpr int kOutOfRange = (int)0x80000000u;
  const int t = threadIdx.x, blocks = rs.K >> 3;
  const size_t kb = (size_t)rs.K * 2;
  const __amdgpu_buffer_rsrc_t xbuf = buffer_rsrc(p.h, rs.src == SRC_H && c.first ? kb : 0);
  const __amdgpu_buffer_rsrc_t gbuf = buffer_rsrc(rs.gamma, rs.gamma ? kb : 0);
#pragma unroll
  for (int i = 0; i < XB; ++i) {
    const int b = t + 256 * i;
    xv[i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(xbuf, b < blocks ? b * 16 : kOutOfRange, 0, 0));
    av[i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(gbuf, b < blocks ? b * 16 : kOutOfRange, 0, 0));
  }
}

// ---------------------------------------------------------------- z workgroups
// Rank r of problem pi: z = fp16(x'.V[r]^T), published as one tagged word (z in bits 16..31).
// Thread t holds block t of the source row and of V[r] (K <= 2048), so no staging is needed:
// each thread adds its eight products, the waves reduce on DPP and thread 0 adds the four waves.
template <int KMAX, int SRC>
__device__ __forceinline__ void layer_z_role(const LayerParams &p, const LayerCtx &c, const LayerWeights &W, int pi,
                                             int r, uint64_t passed, float *wsum) {
  constexpr int XB = (KMAX / 8 + 255) / 256;
  static_assert(XB == 1, "one source block per thread");
  constexpr int kOutOfRange = (int)0x80000000u;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const RoleShape rs = role_shape<SRC>(p, W);
  const int K = rs.K, blocks = K >> 3;
  const int zrank = pick(p.rank, pi);
  h8 xv[XB], av[XB];
  layer_plain_loads(p, c, rs, xv, av);
  const __amdgpu_buffer_rsrc_t vbuf = buffer_rsrc(W.down[pi], (size_t)zrank * K * 2);
  u4 vz = __builtin_bit_cast(
      u4, __builtin_amdgcn_raw_buffer_load_b128(vbuf, r < zrank && t < blocks ? (r * K + t * 8) * 2 : kOutOfRange, 0, 0));
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();  // the previous layer's LDS reads are done before this layer writes
  const uint32_t tag = layer_tag(p, passed);
  const int src_base = source_base(p, c, rs.src);
  if (src_base >= 0) {
    h8 gamma_rows[XB];
#pragma unroll
    for (int i = 0; i < XB; ++i) gamma_rows[i] = av[i];
    wait_sentinel(p, source_sentinel(p, src_base, rs.src), tag);
    layer_source_row(p, src_base, rs.src, K, tag, xv, av);
    if (rs.src != SRC_GU) {
#pragma unroll
      for (int i = 0; i < XB; ++i) av[i] = gamma_rows[i];
    }
  }
  const float inv = layer_prologue_inv(rs.prologue, K, p.eps, xv, wsum);
  float acc = 0.0f;
  if (t < blocks) {
    const h8 xx = layer_prologue_apply(rs.prologue, xv[0], av[0], inv);
    asm volatile("" : "+v"(vz));
    const h8 vv = __builtin_bit_cast(h8, vz);
    acc = dot2(pair_of(xx, 0), pair_of(vv, 0), dot2(pair_of(xx, 2), pair_of(vv, 2), 0.0f));
    acc = dot2(pair_of(xx, 1), pair_of(vv, 1), dot2(pair_of(xx, 3), pair_of(vv, 3), acc));
  }
  acc = wave_sum(acc);
  if (rs.prologue == PRO_RMSNORM) __syncthreads();  // wsum held the norm's partial sums
  if (lane == 0) wsum[wave] = acc;
  __syncthreads();
  if (t == 0) {
    const f16 z = r < zrank ? (f16)(((wsum[0] + wsum[1]) + wsum[2]) + wsum[3]) : (f16)0.0f;
    sys_store(p.ws + c.lw + p.w_z + pi * kLayerZWords + r,
              (uint64_t)tag | ((uint64_t)__builtin_bit_cast(uint16_t, z) << 16));
  }
}

// ---------------------------------------------------------------- GEMV tiles
// Rows [n0, n0 + 16) of problem pi, with the fused decode kernel's product and epilogue.  Output:
// q|k|v and gate|up as words, o as the h1 words (after the residual h), down into h (after the
// residual h1).
template <int FMT, bool SCALED, int KMAX, bool RANKED, bool OWN_Z, int SRC>
__device__ __forceinline__ void layer_tile_role(const LayerParams &p, const LayerCtx &c, const LayerWeights &W, int pi,
                                                int n0, uint64_t passed, uint8_t *smem) {
  constexpr int CPL = FormatTraits<FMT>::CPL;
  constexpr int BITS = FormatTraits<FMT>::BITS;
  constexpr int KSTEP = 4 * CPL;
  constexpr int KG = 4;
  constexpr int WSTEP = KG * KSTEP;
  constexpr int D = (KMAX + WSTEP - 1) / WSTEP;
  static_assert(D <= 32, "KMAX too long for this format");
  constexpr int T8 = CPL / 8;
  constexpr int XLD = KMAX + KSTEP + 8;
  constexpr int XB = (KMAX / 8 + 255) / 256;
  constexpr int GMAX = KMAX / FusedGroupMin<KMAX>::value;
  constexpr int SC = SCALED ? (16 * GMAX + 255) / 256 : 0;
  constexpr int VB = OWN_Z ? (KMAX / 8 + 7) / 8 : 0;  // V blocks per thread (8 threads per rank row)
  static_assert(!OWN_Z || RANKED, "own z needs the correction");
  static_assert(XLD * 2 + (SCALED ? 16 * GMAX + 8 : 8) * 2 + 16 * kFusedMaxRank * 2 + 2 * kFusedMaxRank * 2 +
                        ((KG - 1) * 16 + 4) * 4 + 256 * 4 + (OWN_Z ? VB * 64 * 2 : 0) <=
                    kLayerTileSmem,
                "the tile role's LDS exceeds the launch's dynamic LDS");
  static_assert(kFusedMaxRank == 32, "the correction is one 32-deep product");
  constexpr int kOutOfRange = (int)0x80000000u;
  f16 *xs = reinterpret_cast<f16 *>(smem);                                  // [XLD]
  f16 *ss = xs + XLD;                                                       // [16 GMAX + 8]
  f16 *us = ss + (SCALED ? 16 * GMAX + 8 : 8);                              // [16 * 32]
  f16 *zs = us + 16 * kFusedMaxRank;                                        // [32] (a 32-float slot)
  float *red = reinterpret_cast<float *>(zs + 2 * kFusedMaxRank);           // [48]
  float *wsum = red + (KG - 1) * 16;                                        // [4]
  uint32_t *nf4_table = reinterpret_cast<uint32_t *>(wsum + 4);             // [256]
  f16 *xn = reinterpret_cast<f16 *>(nf4_table + 256);                       // [VB * 64] x' in natural order (own z)

  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int j = lane & 15, g = lane >> 4;
  const RoleShape rs = role_shape<SRC>(p, W);
  const int K = rs.K, N = pick(p.N, pi), up_ld = pick(p.up_ld, pi);
  const int G = K == p.hidden ? p.G1 : p.G2;
  const int group_shift = K == p.hidden ? p.shift1 : p.shift2;
  const int rows = min(16, N - n0);
  const int row_bytes = K * BITS / 8;
  const int rank = RANKED ? pick(p.rank, pi) : 0;

  // Wave 0, lane r < rows: the row's per-row scale and (o, first layer) its residual h value.
  const f16 rscale = __builtin_bit_cast(
      f16, __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(W.scales[pi], p.per_row && wave == 0 ? (size_t)N * 2 : 0),
                                                lane < rows ? (n0 + lane) * 2 : kOutOfRange, 0, 0));
  const f16 rres = __builtin_bit_cast(
      f16, __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(p.h, pi == P_O && c.first && wave == 0 ? (size_t)N * 2 : 0),
                                                lane < rows ? (n0 + lane) * 2 : kOutOfRange, 0, 0));
  u4 ureg = {0u, 0u, 0u, 0u};
  if constexpr (RANKED) {
    const int ur = 4 * wave + (lane >> 2), uq = lane & 3;
    const int off = lane < 16 && ur < rows && uq * 8 < rank ? ((n0 + ur) * up_ld + uq * 8) * 2 : kOutOfRange;
    ureg = __builtin_bit_cast(
        u4, __builtin_amdgcn_raw_buffer_load_b128(buffer_rsrc(W.up[pi], rank > 0 ? (size_t)N * up_ld * 2 : 0), off, 0, 0));
  }
  h8 xv[XB], av[XB];
  layer_plain_loads(p, c, rs, xv, av);
  // Own z: thread t holds blocks t % 8 + 8 i of V row t / 8 (zeros past the rank and K).
  const int vr = t >> 3, vpart = t & 7;
  u4 vreg[VB > 0 ? VB : 1];
  if constexpr (OWN_Z) {
    const __amdgpu_buffer_rsrc_t vbuf = buffer_rsrc(W.down[pi], rank > 0 ? (size_t)rank * K * 2 : 0);
#pragma unroll
    for (int i = 0; i < VB; ++i) {
      const int k = (vpart + 8 * i) * 8;
      const int off = vr < rank && k < K ? (vr * K + k) * 2 : kOutOfRange;
      vreg[i] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(vbuf, off, 0, 0));
    }
  }
  f16 sreg[SC > 0 ? SC : 1];
  if constexpr (SCALED) {
    const __amdgpu_buffer_rsrc_t sbuf = buffer_rsrc(W.scales[pi] + (size_t)n0 * G, (size_t)rows * G * 2);
#pragma unroll
    for (int i = 0; i < SC; ++i)
      sreg[i] = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(sbuf, (t + i * 256) * 2, 0, 0));
  }
  const __amdgpu_buffer_rsrc_t wbuf = buffer_rsrc(W.codes[pi] + (size_t)n0 * row_bytes, (size_t)rows * row_bytes);
  u4 w[D];
#pragma unroll
  for (int u = 0; u < D; ++u) {
    const int k = (wave + KG * u) * KSTEP + g * CPL;
    const int off = k < K ? j * row_bytes + k * BITS / 8 : kOutOfRange;
    w[u] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(wbuf, off, 0, 0));
  }
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();  // the previous layer's epilogue has read the LDS this layer overwrites
  const uint32_t tag = layer_tag(p, passed);

  if constexpr (FMT == FMT_NF4) build_nf4_pair_table(nf4_table);
  if constexpr (RANKED) {
    if (lane < 16) stage_u_piece(us + (4 * wave + (lane >> 2)) * kFusedMaxRank + (lane & 3) * 8, ureg, lane & 3, rank);
  }
  if constexpr (SCALED) {
#pragma unroll
    for (int i = 0; i < SC; ++i)
      if (t + i * 256 < 16 * GMAX) ss[t + i * 256] = sreg[i];
    if (t < 8) ss[16 * GMAX + t] = (f16)0.0f;
  }
  // Residual words (o after the first layer: the layer input h; down: h1) are requested with the
  // source row, once its sentinel is current: both are published before the words polled for.
  const int res_base = pi == P_DOWN ? c.lw + p.w_h1 : (pi == P_O && !c.first) ? c.lw + p.w_h : -1;
  uint64_t resw = 0;
  // The source row: the first layer's input (loaded above) or the words of an earlier role.
  const int src_base = source_base(p, c, rs.src);
  if (src_base >= 0) {
    h8 gamma_rows[XB];
#pragma unroll
    for (int i = 0; i < XB; ++i) gamma_rows[i] = av[i];
    wait_sentinel(p, source_sentinel(p, src_base, rs.src), tag);
    if (res_base >= 0 && wave == 0 && lane < rows) resw = sys_load(p.ws + res_base + (n0 + lane) / 2);
    layer_source_row(p, src_base, rs.src, K, tag, xv, av);
    if (rs.src != SRC_GU) {
#pragma unroll
      for (int i = 0; i < XB; ++i) av[i] = gamma_rows[i];
    }
  }
  const float inv = layer_prologue_inv(rs.prologue, K, p.eps, xv, wsum);
  const int blocks = K >> 3;
#pragma unroll
  for (int i = 0; i < XB; ++i) {
    const int b = t + 256 * i;
    if (b < blocks) {
      const h8 v = layer_prologue_apply(rs.prologue, xv[i], av[i], inv);
      *reinterpret_cast<h8 *>(xs + b * 8) = permute_block<FMT>(v);
      if constexpr (OWN_Z) *reinterpret_cast<h8 *>(xn + b * 8) = v;
    }
  }
  // Zeros past K: MFMA lanes read up to KSTEP beyond it, the own z product up to VB * 64.
  for (int b = blocks + t; b * 8 < min(XLD, K + KSTEP + 8); b += 256) *reinterpret_cast<h8 *>(xs + b * 8) = h8{};
  if constexpr (OWN_Z) {
    for (int b = blocks + t; b < VB * 8; b += 256) *reinterpret_cast<h8 *>(xn + b * 8) = h8{};
  }
  __syncthreads();

  // Own z = fp16(x'.V^T) into zs (zero from the rank on), read by the epilogue after the barrier
  // that follows the product: V rows as loaded against the natural-order copy of x'.
  if constexpr (OWN_Z) {
    h8 xx[VB];
#pragma unroll
    for (int i = 0; i < VB; ++i) xx[i] = *reinterpret_cast<const h8 *>(xn + (vpart + 8 * i) * 8);
    float za = 0.0f, zb = 0.0f;
#pragma unroll
    for (int i = 0; i < VB; ++i) {
      asm volatile("" : "+v"(vreg[i]));
      const h8 vv = __builtin_bit_cast(h8, vreg[i]);
      za = dot2(pair_of(xx[i], 0), pair_of(vv, 0), dot2(pair_of(xx[i], 2), pair_of(vv, 2), za));
      zb = dot2(pair_of(xx[i], 1), pair_of(vv, 1), dot2(pair_of(xx[i], 3), pair_of(vv, 3), zb));
    }
    za = sum8(za + zb);
    if (vpart == 0) zs[vr] = vr < rank ? (f16)za : (f16)0.0f;
  }

  f4 acc = {0.f, 0.f, 0.f, 0.f};
  // Every A fragment (and group scale) is read from LDS before the first product, so the reads
  // overlap instead of each waiting behind the previous MFMA.
  const f16 *a0 = xs + g * CPL;
  h8 afr[D][T8];
  f16 gsc[D];
#pragma unroll
  for (int u = 0; u < D; ++u) {
    const int kb = (wave + KG * u) * KSTEP;
#pragma unroll
    for (int q = 0; q < T8; ++q) afr[u][q] = kb < K ? *reinterpret_cast<const h8 *>(a0 + kb + 8 * q) : h8{};
    gsc[u] = (f16)1.0f;
    if constexpr (SCALED) {
      if (kb < K) gsc[u] = ss[j * G + ((kb + g * CPL) >> group_shift)];
    }
  }
#pragma unroll
  for (int u = 0; u < D; ++u) {
    const int kb = (wave + KG * u) * KSTEP;
    asm volatile("" : "+v"(w[u]));
    const h2 s2 = {gsc[u], gsc[u]};
#pragma unroll
    for (int q = 0; q < T8; ++q) {
      const h8 b = decode8<FMT, !SCALED>(w[u], q, s2, nf4_table);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(afr[u][q], b, acc, 0, 0, 0);
    }
  }
  if (wave > 0 && g == 0) red[(wave - 1) * 16 + j] = acc[0];
  __syncthreads();
  if (wave != 0) return;

  // ---- epilogue: wave 0; lane j < rows owns row n0 + j ----
  if constexpr (RANKED && !OWN_Z) {
    if (rank > 0) {
      const uint64_t *zw = p.ws + c.lw + p.w_z + pi * kLayerZWords;
      if (lane < kFusedMaxRank)  // every zs entry, zero from rank on
        zs[lane] = lane < rank ? word_half(wait_word(p, zw + lane, tag), 0) : (f16)0.0f;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
    }
  }
  // Residuals: o adds the layer input h (plain in the first layer, else the h words), down adds
  // h1; the words requested above are final by now (what this tile read depends on them), so the
  // bounded re-read is a formality.
  f16 residual = rres;
  if (res_base >= 0 && lane < rows) {
    if (word_tag(resw) != tag) resw = wait_word(p, p.ws + res_base + (n0 + lane) / 2, tag);
    residual = word_half(resw, (n0 + lane) & 1);
  }
  float sum = ((acc[0] + red[j]) + red[16 + j]) + red[32 + j];
  if (p.per_row) sum *= (float)rscale;
  f16 hv = (f16)sum;
  if (RANKED && rank > 0) {
    // d = z.U[row]^T as one 32-deep product: lane (g, j) brings ranks [8g, 8g + 8) of z (the A
    // rows, all alike) and of U row j; both are zero from the rank on.  Lane (0, j) gets row j.
    const h8 zfr = *reinterpret_cast<const h8 *>(zs + 8 * g);
    const h8 ufr = *reinterpret_cast<const h8 *>(us + j * kFusedMaxRank + 8 * g);
    const float d = __builtin_amdgcn_mfma_f32_16x16x32_f16(zfr, ufr, f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0)[0];
    hv = (f16)((float)hv + (float)(f16)d);
  }
  if (pi == P_O || pi == P_DOWN) hv = (f16)((float)residual + (float)hv);
  const f16 next = __builtin_bit_cast(f16, (uint16_t)dpp_move<kDppRowShl1>((int)__builtin_bit_cast(uint16_t, hv)));
  if (g != 0 || j >= rows) return;
  if (pi == P_DOWN && c.nw < 0) {  // the last layer's output: the plain row h
    p.h[n0 + j] = hv;
    return;
  }
  if (j & 1) return;
  int region, off = 0;
  if (pi <= P_V) {
    region = c.lw + p.w_qkv;
    off = pi == P_Q ? 0 : pi == P_K ? p.N[P_Q] : p.N[P_Q] + p.N[P_K];
  } else if (pi == P_O) {
    region = c.lw + p.w_h1;
  } else if (pi == P_DOWN) {
    region = c.nw + p.w_h;  // the next layer's input
  } else {
    region = c.lw + p.w_gu;
    off = pi == P_GATE ? 0 : p.inter;
  }
  sys_store(p.ws + region + (off + n0 + j) / 2, pair_word(tag, hv, next));
}

// ---------------------------------------------------------------- attention
#ifndef LB_ATTN_FAST_EXP
#define LB_ATTN_FAST_EXP 1  // the hardware exponential (v_exp_f32) in the softmax
#endif
__device__ __forceinline__ float attn_exp(float x) {
  if constexpr (LB_ATTN_FAST_EXP) return __expf(x);
  else return expf(x);
}

// Query head h, output dims [d0, d0 + kSliceDims): the staging of decode_attention_kernel on q, k
// and v rows read from the q|k|v words; the output dims are published as att words.
__device__ __forceinline__ void layer_attention_role(const LayerParams &p, const LayerCtx &c, const LayerWeights &W,
                                                     int idx, uint64_t passed, uint8_t *smem) {
  f16 *qs = reinterpret_cast<f16 *>(smem);               // [64] raw, then rotated
  f16 *kn = qs + kHeadDim;                               // [64]
  f16 *vn = kn + kHeadDim;                               // [64]
  f16 *raw = vn + kHeadDim;                              // [128] raw q and k rows
  float *wred = reinterpret_cast<float *>(raw + 2 * kHeadDim);  // [8] wave maxima, then wave sums
  float *pv = wred + 8;                                  // [kPvPartials * kSliceDims]
  float *sc = pv + kPvPartials * kSliceDims;             // [capacity]
  constexpr int kOutOfRange = (int)0x80000000u;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int h = idx / kAttnDimSlices;
  const int d0 = (idx % kAttnDimSlices) * kSliceDims;
  const int group = p.heads / p.kv_heads;
  const int kvh = h / group;
  const int pos = (int)p.position[0];
  const bool valid = pos >= 0 && pos < p.capacity;
  const int cpos = valid ? pos : 0;
  const size_t head_base = (size_t)kvh * p.capacity * kHeadDim;
  // Cached rows (slots below pos) and the RoPE row, issued before the wait for q, k, v.
  const __amdgpu_buffer_rsrc_t kbuf = buffer_rsrc(W.keys + head_base, valid ? (size_t)pos * kHeadDim * 2 : 0);
  const __amdgpu_buffer_rsrc_t vbuf = buffer_rsrc(W.values + head_base, valid ? (size_t)pos * kHeadDim * 2 : 0);
  const int blk = t % kSliceBlocks, part = t / kSliceBlocks;
  u4 kreg[kScoreSlots][kHeadDim / 8];
  u4 vreg[kValueSlots];
  auto load_keys = [&](int base) {
#pragma unroll
    for (int i = 0; i < kScoreSlots; ++i) {
      const int s = base + t + 256 * i;
#pragma unroll
      for (int b = 0; b < kHeadDim / 8; ++b)
        kreg[i][b] = __builtin_bit_cast(
            u4, __builtin_amdgcn_raw_buffer_load_b128(kbuf, s < pos ? (s * kHeadDim + 8 * b) * 2 : kOutOfRange, 0, 0));
    }
  };
  auto load_values = [&](int base) {
#pragma unroll
    for (int i = 0; i < kValueSlots; ++i) {
      const int s = base + part + kAttnParts * i;
      vreg[i] = __builtin_bit_cast(
          u4, __builtin_amdgcn_raw_buffer_load_b128(vbuf, s < pos ? (s * kHeadDim + d0 + 8 * blk) * 2 : kOutOfRange, 0, 0));
    }
  };
  load_keys(0);
  load_values(0);
  const int d = lane;
  const __amdgpu_buffer_rsrc_t cbuf = buffer_rsrc(p.cos + (size_t)cpos * kHeadDim, wave < 2 ? kHeadDim * 2 : 0);
  const __amdgpu_buffer_rsrc_t snbuf = buffer_rsrc(p.sin + (size_t)cpos * kHeadDim, wave < 2 ? kHeadDim * 2 : 0);
  const f16 cv = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(cbuf, d * 2, 0, 0));
  const f16 sv = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(snbuf, d * 2, 0, 0));
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();  // the previous layer's LDS reads are done before this layer writes
  const uint32_t tag = layer_tag(p, passed);

  // q of head h, k and v of KV head kvh: 96 words from the q|k|v region.
  const int nq = p.N[P_Q], nk = p.N[P_K];
  const uint64_t *qkv = p.ws + c.lw + p.w_qkv;
  wait_sentinel(p, qkv + (nq + nk + (kvh + 1) * kHeadDim) / 2 - 1, tag);
  if (t < 3 * kHeadDim / 2) {
    const int part3 = t / (kHeadDim / 2), wi = t % (kHeadDim / 2);
    const int first = part3 == 0 ? h * kHeadDim : part3 == 1 ? nq + kvh * kHeadDim : nq + nk + kvh * kHeadDim;
    const uint64_t word = wait_word(p, qkv + first / 2 + wi, tag);
    f16 *dst = part3 == 0 ? raw : part3 == 1 ? raw + kHeadDim : vn;
    dst[2 * wi] = word_half(word, 0);
    dst[2 * wi + 1] = word_half(word, 1);
  }
  __syncthreads();
  if (wave < 2) {
    const f16 *src = raw + wave * kHeadDim;
    const float x0 = (float)src[d], x1 = (float)src[d ^ 32];
    const float rot = d < 32 ? -x1 : x1;
    const f16 r = rope_element(x0, rot, (float)cv, (float)sv);
    if (wave == 0) qs[d] = r; else kn[d] = r;
  }
  __syncthreads();
  if (!valid) {
    if (t < kSliceDims) {
      f16 nan = (f16)__builtin_nanf("");
      if ((t & 1) == 0)
        sys_store(p.ws + c.lw + p.w_att + (h * kHeadDim + d0 + t) / 2, pair_word(tag, nan, nan));
    }
    return;
  }
  h8 qreg[kHeadDim / 8];
#pragma unroll
  for (int b = 0; b < kHeadDim / 8; ++b) qreg[b] = *reinterpret_cast<const h8 *>(qs + 8 * b);
  // Scores of the first round's slots (t + 256 i) stay in registers; later rounds go through sc.
  // The new key (slot pos, written to the cache by this launch) is read from LDS by the one lane
  // that owns it, after the cached ones.
  float scv[kScoreSlots];
  float lmax = -INFINITY;
  for (int base = 0; base <= pos; base += 256 * kScoreSlots) {
    if (base > 0) load_keys(base);
#pragma unroll
    for (int i = 0; i < kScoreSlots; ++i) {
      const int s = base + t + 256 * i;
      if (base + 256 * i > pos) break;
      float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
      for (int b = 0; b < kHeadDim / 8; ++b) {
        asm volatile("" : "+v"(kreg[i][b]));
        const h8 qq = qreg[b];
        const h8 kk = __builtin_bit_cast(h8, kreg[i][b]);
        acc0 = dot2(pair_of(qq, 0), pair_of(kk, 0), dot2(pair_of(qq, 2), pair_of(kk, 2), acc0));
        acc1 = dot2(pair_of(qq, 1), pair_of(kk, 1), dot2(pair_of(qq, 3), pair_of(kk, 3), acc1));
      }
      if (s == pos) {
        acc0 = acc1 = 0.0f;
#pragma unroll
        for (int b = 0; b < kHeadDim / 8; ++b) {
          const h8 qq = qreg[b];
          const h8 kk = *reinterpret_cast<const h8 *>(kn + 8 * b);
          acc0 = dot2(pair_of(qq, 0), pair_of(kk, 0), dot2(pair_of(qq, 2), pair_of(kk, 2), acc0));
          acc1 = dot2(pair_of(qq, 1), pair_of(kk, 1), dot2(pair_of(qq, 3), pair_of(kk, 3), acc1));
        }
      }
      const float v = (float)(f16)((float)(f16)(acc0 + acc1) * p.scale);
      if (base == 0) scv[i] = v;
      else if (s <= pos) sc[s] = v;
      if (s <= pos) lmax = fmaxf(lmax, v);
    }
  }
  // Softmax with one exchange between the waves: each wave takes its exponentials against its own
  // maximum and sums them; after one barrier every thread rescales by exp(wave max - max) (0 for a
  // wave without keys) and divides by the rescaled total, added in wave order.
  lmax = wave_max(lmax);
  float ev[kScoreSlots];
  float lsum = 0.0f;
#pragma unroll
  for (int i = 0; i < kScoreSlots; ++i) {
    ev[i] = 0.0f;
    if (t + 256 * i <= pos) {
      ev[i] = attn_exp(scv[i] - lmax);
      lsum += ev[i];
    }
  }
  for (int s = t + 256 * kScoreSlots; s <= pos; s += 256) {
    const float e = attn_exp(sc[s] - lmax);
    sc[s] = e;
    lsum += e;
  }
  lsum = wave_sum(lsum);
  if (lane == 0) {
    wred[wave] = lmax;
    wred[4 + wave] = lsum;
  }
  __syncthreads();
  const float m = fmaxf(fmaxf(wred[0], wred[1]), fmaxf(wred[2], wred[3]));
  float total = 0.0f;
#pragma unroll
  for (int w = 0; w < 4; ++w) total += wred[4 + w] * attn_exp(wred[w] - m);
  const float f = attn_exp(lmax - m) / total;
#pragma unroll
  for (int i = 0; i < kScoreSlots; ++i)
    if (t + 256 * i <= pos) sc[t + 256 * i] = (float)(f16)(ev[i] * f);
  for (int s = t + 256 * kScoreSlots; s <= pos; s += 256) sc[s] = (float)(f16)(sc[s] * f);
  __syncthreads();

  float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const h8 vnew = *reinterpret_cast<const h8 *>(vn + d0 + 8 * blk);  // the new value row's block
  for (int base = 0; base <= pos; base += kAttnParts * kValueSlots) {
    if (base > 0) load_values(base);
#pragma unroll
    for (int i = 0; i < kValueSlots; ++i) {
      const int s = base + part + kAttnParts * i;
      if (base + kAttnParts * i > pos) break;
      asm volatile("" : "+v"(vreg[i]));
      const h8 vv = s == pos ? vnew : __builtin_bit_cast(h8, vreg[i]);
      const float pr = s <= pos ? sc[min(s, pos)] : 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] += pr * (float)vv[e];
    }
  }
  pv_row_partials(o, pv, lane, wave);
  __syncthreads();
  if (t < kSliceDims && (t & 1) == 0) {
    const f16 a = (f16)pv_total(pv, t), b = (f16)pv_total(pv, t + 1);
    sys_store(p.ws + c.lw + p.w_att + (h * kHeadDim + d0 + t) / 2, pair_word(tag, a, b));
  }
  // The KV append (the first dim slice of the first query head of each KV group) comes last: the
  // load counter also counts stores, so a store issued before the scores would make their wait
  // for the cached rows wait for the store's round trip as well.  No workgroup of this launch
  // reads the slot (each uses its own copy of the new row).
  if (h % group == 0 && idx % kAttnDimSlices == 0 && t < 2 * kHeadDim) {
    const int dd = t & 63;
    f16 *dst = (t < kHeadDim ? W.keys : W.values) + head_base + (size_t)pos * kHeadDim + dd;
    *dst = t < kHeadDim ? kn[dd] : vn[dd];
  }
}

// ---------------------------------------------------------------- the kernel
// One layer (STACK false: the weights in the parameters) or p.layers layers (STACK true: the
// weights in `table`, one entry per layer) per launch.  In a stacked launch every workgroup keeps
// its role through all layers: after finishing its part of layer l it issues the loads of layer
// l + 1 and waits there, so weights are fetched while earlier stages run, and layer l + 1's
// inputs arrive as the h words of layer l's down tiles.  A workgroup then also waits for
// workgroups dispatched after it (the previous layer's later roles), so a stacked grid must be
// resident all at once: the host launches it only when the device holds every workgroup
// together, and the bounded waits end the launch (with a timeout recorded) should it not.
template <int FMT, bool SCALED, bool RANKED, bool STACK>
__global__ __launch_bounds__(256) void decode_layer_kernel(LayerParams p, const LayerWeights *__restrict__ table) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ float wsum[4];
  const int b = blockIdx.x;
  const uint64_t passed = sys_load(p.ws);  // waited for only where a role first needs the tag
  const int role = b < p.end[R_TQKV] ? R_TQKV : b < p.end[R_ATTN] ? R_ATTN : b < p.end[R_TO] ? R_TO
                   : b < p.end[R_TGU] ? R_TGU : b < p.end[R_ZD] ? R_ZD : R_TD;
  const int i = b - (role == R_TQKV ? 0 : role == R_ATTN ? p.end[R_TQKV] : role == R_TO ? p.end[R_ATTN]
                     : role == R_TGU ? p.end[R_TO] : role == R_ZD ? p.end[R_TGU] : p.end[R_ZD]);
  // Tile workgroups of q|k|v and gate|up: the problem and first row from the per-problem counts.
  auto tile_of = [&](int p0, int count, int &pi, int &n0) {
    pi = p0;
    int ti = i;
    for (int q = 0; q < count - 1; ++q) {
      const int n = (pick(p.N, pi) + 15) / 16;
      if (ti < n) break;
      ti -= n;
      ++pi;
    }
    n0 = ti * 16;
  };
  // Each role runs its own loop over the layers (one layer unless STACK), so the compiler keeps
  // one role's values live at a time; every role body is specialised for its problems.
  const int layers = STACK ? p.layers : 1;
  auto each_layer = [&](auto &&body) {
    for (int l = 0; l < layers; ++l) {
      const LayerCtx c{kLayerHeaderWords + l * p.layer_words,
                       l + 1 < layers ? kLayerHeaderWords + (l + 1) * p.layer_words : -1, l == 0};
      if constexpr (STACK) body(c, table[l]);
      else body(c, p.w);
    }
  };
  int pi = 0, n0 = 0;
  switch (role) {
    case R_TQKV:
      tile_of(P_Q, 3, pi, n0);
      each_layer([&](const LayerCtx &c, const LayerWeights &W) {
        layer_tile_role<FMT, SCALED, 640, RANKED, RANKED, SRC_H>(p, c, W, pi, n0, passed, smem);
      });
      break;
    case R_ATTN:
      each_layer([&](const LayerCtx &c, const LayerWeights &W) { layer_attention_role(p, c, W, i, passed, smem); });
      break;
    case R_TO:
      each_layer([&](const LayerCtx &c, const LayerWeights &W) {
        layer_tile_role<FMT, SCALED, 640, RANKED, RANKED, SRC_ATT>(p, c, W, P_O, i * 16, passed, smem);
      });
      break;
    case R_TGU:
      tile_of(P_GATE, 2, pi, n0);
      each_layer([&](const LayerCtx &c, const LayerWeights &W) {
        layer_tile_role<FMT, SCALED, 640, RANKED, RANKED, SRC_H1>(p, c, W, pi, n0, passed, smem);
      });
      break;
    case R_ZD:
      each_layer([&](const LayerCtx &c, const LayerWeights &W) { layer_z_role<kFusedMaxK, SRC_GU>(p, c, W, P_DOWN, i, passed, wsum); });
      break;
    default:
      each_layer([&](const LayerCtx &c, const LayerWeights &W) {
        layer_tile_role<FMT, SCALED, kFusedMaxK, RANKED, false, SRC_GU>(p, c, W, P_DOWN, i * 16, passed, smem);
      });
      break;
  }
  // Every workgroup counts itself once, after all of its work (thread 0 of wave 0 runs every role
  // to its end).
  if (threadIdx.x == 0) __hip_atomic_fetch_add(p.ws, (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

}  // namespace lb
