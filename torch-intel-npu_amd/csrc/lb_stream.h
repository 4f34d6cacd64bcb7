// gfx950 streaming GEMV for up to 16 activation rows over long INT4 / INT8 weight matrices (the
// tied head, the Llama-shaped projections): y[M, N] = x[M, K] . (q * s)[N, K]^T, scales applied
// to exact integer-code sums.
//
// Weight decode without per-weight arithmetic.  A code enters the MFMA as the fp16 value of a
// "magic" half-word: the (sign-flipped) nibble or byte is OR-ed under the exponent of 1024, so the
// B operand costs one bit operation per pair of codes and nothing else:
//   INT4 even codes  0x6400 | (c ^ 8)         = 1032 + q
//   INT4 odd codes   0x6400 | ((c ^ 8) << 4)  = 1152 + 16 q   (the nibble decoded where it sits)
//   INT8             0x6400 | (b ^ 0x80)      = 1152 + b
// The activations are staged with the matching slot permutation, odd INT4 codes' activations
// divided by 16, so every product is x * (bias + q).  The bias part is removed per 32-code (INT4)
// or 16-code (INT8) block with the staged activations' block sums, and the block's group scale is
// applied to the fp32 difference: y = sum_blocks s_block * (sum x (bias + q) - bias-sum), i.e. the
// exact x . (q * s) product up to fp32 rounding (the reference's rounding-budget gate,
// torch_npu_lowbit_demo.py:97-106, bounds the distance to its fp16(q * s) weights).
//
// Per-block sums come from the MFMA's 16 A rows: with MP (1, 2, 4, 8 or 16) activation rows, each
// activation row owns R = 16 / MP A rows, and A row (m, r) is activation row m masked to the
// blocks it accumulates (lanes read a zero region of LDS where their row is inactive):
//   R >= 4  one 32/16-code block each: a flush window covers R / 4 loads (any group >= a block);
//   R == 2  two blocks (half of a 16-byte load's four lane groups): groups >= 2 blocks;
//   R == 1  all four blocks of a load: groups >= 4 blocks.
// The 16 x 16 result is flushed (scaled, bias removed, accumulated in fp32) once per window.
//
// A wave streams 16-row tiles chunk by chunk (CH 16-byte loads per lane per chunk, PD chunks in
// flight); the activation rows, a zero region and the block sums are staged in LDS once per
// workgroup.  KSPLIT = 1: persistent waves, each owning whole tiles; KSPLIT = 4: one tile per
// workgroup, the four waves taking interleaved chunks and reducing through LDS.
#pragma once
#include "fused_launch.h"

namespace lb {

template <int FMT> struct StreamTraits;
template <> struct StreamTraits<FMT_INT4> { static constexpr int CPL = 32, BITS = 4, T8 = 4; };
template <> struct StreamTraits<FMT_INT8> { static constexpr int CPL = 16, BITS = 8, T8 = 2; };

struct StreamParams {
  const f16 *x;           // [M, ldx]
  const uint8_t *codes;   // [N, K * bits / 8]
  const f16 *scales;      // [N, G]
  f16 *y;                 // [M, ldy]
  const f16 *bias;        // [N] or null
  const f16 *residual;    // [N] or null (may equal y; M == 1 only)
  int M, N, K, G, group_shift;
  int ldx, ldy;
  int tiles, chunks;      // 16-row tiles; chunks per tile row
  int kslice;             // tile_rows_kernel over K slices (grid y): codes per slice (0: none)
  float *partial;         // K slices: fp32 partial sums [slices, M, N]
  uint32_t *tickets;      // K slices: one zero counter per workgroup column, the slices added in the
                          // kernel (null: splitk_reduce_kernel adds them in a launch of its own)
};

// Slot permutation of an 8-code group, the activation factor and the bias of each slot.
template <int FMT> struct StreamSlots;
template <> struct StreamSlots<FMT_INT4> {
  static constexpr int perm[8] = {0, 4, 1, 5, 2, 6, 3, 7};
  static constexpr float factor[8] = {1.f, 1.f, 0.0625f, 0.0625f, 1.f, 1.f, 0.0625f, 0.0625f};
  static constexpr float bias[8] = {1032.f, 1032.f, 1152.f, 1152.f, 1032.f, 1032.f, 1152.f, 1152.f};
};
template <> struct StreamSlots<FMT_INT8> {
  static constexpr int perm[8] = {0, 2, 1, 3, 4, 6, 5, 7};
  static constexpr float factor[8] = {1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f};
  static constexpr float bias[8] = {1152.f, 1152.f, 1152.f, 1152.f, 1152.f, 1152.f, 1152.f, 1152.f};
};

// B operand q of an MFMA from the 16-byte load w: INT4 dword q = 8 codes, INT8 dwords 2q, 2q + 1.
template <int FMT>
__device__ __forceinline__ h8 stream_decode(const u4 &w, int q) {
  u4 v;
  if constexpr (FMT == FMT_INT4) {
    const uint32_t a = w[q], t = a >> 8;
    v[0] = (a & 0x000F000Fu) ^ 0x64086408u;  // c0, c4: 1032 + q
    v[1] = (a & 0x00F000F0u) ^ 0x64806480u;  // c1, c5: 1152 + 16 q
    v[2] = (t & 0x000F000Fu) ^ 0x64086408u;  // c2, c6
    v[3] = (t & 0x00F000F0u) ^ 0x64806480u;  // c3, c7
  } else {
    const uint32_t a = w[2 * q], b = w[2 * q + 1];
    v[0] = (a & 0x00FF00FFu) ^ 0x64806480u;         // b0, b2: 1152 + b
    v[1] = ((a >> 8) & 0x00FF00FFu) ^ 0x64806480u;  // b1, b3
    v[2] = (b & 0x00FF00FFu) ^ 0x64806480u;         // b4, b6
    v[3] = ((b >> 8) & 0x00FF00FFu) ^ 0x64806480u;  // b5, b7
  }
  return __builtin_bit_cast(h8, v);
}

// Geometry of the A-row assignment for MP activation rows (see the file comment).
template <int MP, int NS, int CH>
struct StreamGeom {
  static_assert(MP == 1 || MP == 2 || MP == 4 || MP == 8 || MP == 16, "MP is a power of two <= 16");
  static constexpr int R = 16 / MP;                 // A rows per activation row
  static constexpr int WL = R >= 4 ? R / 4 : 1;     // loads per flush window
  static constexpr int BPR = R >= 4 ? 1 : 4 / R;    // blocks per A row
  static constexpr int NMR = R >= 4 ? 1 : 4 / R;    // activation rows a lane flushes
  static constexpr int NSL = NS;                    // scales a lane reads per window (one load's groups)
  static constexpr int WIN = (CH + WL - 1) / WL;    // flush windows per chunk
  static_assert(R >= 4 || NS <= 4 / BPR, "groups must cover an A row's blocks");
};

template <int CH, int NSL, int WIN, bool SCALED>
struct StreamBuf {
  u4 w[CH];
  f16 s[SCALED ? WIN * NSL : 1];
  f16 e[3];                // bias, residual, per-row scale of the lane's row (KSPLIT = 1)
};

template <int FMT, bool SCALED, int NS, int KMAX, int CH, int PD, int KSPLIT, int MP, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void stream_gemv_kernel(StreamParams p) {
  using TR = StreamTraits<FMT>;
  using SL = StreamSlots<FMT>;
  using GE = StreamGeom<MP, NS, CH>;
  constexpr int R = GE::R, WL = GE::WL, BPR = GE::BPR, NMR = GE::NMR, NSL = GE::NSL, WIN = GE::WIN;
  using Buf = StreamBuf<CH, NSL, WIN, SCALED>;
  constexpr int CPL = TR::CPL, CPW = 4 * CPL, BITS = TR::BITS, T8 = TR::T8;
  constexpr int KC = CH * CPW;                       // codes per chunk
  constexpr int KP = (KMAX + KC - 1) / KC * KC;      // staged row length
  constexpr int NB = KP / 8;                         // 8-code groups of a staged row
  constexpr int XBLD = KP / CPL + 16;                // block sums per staged row (zero tail)
  constexpr int kOutOfRange = (int)0x80000000u;
  static_assert(KSPLIT == 1 || (KSPLIT == 4 && WAVES == 4), "KSPLIT is 1, or 4 with four waves");
  constexpr int NT = 64 * WAVES;
  __shared__ __align__(16) f16 xs[MP * KP];
  __shared__ __align__(16) f16 xz[KP];
  __shared__ __align__(16) float xb[MP * XBLD];
  __shared__ float red[KSPLIT > 1 ? 3 * 64 * NMR : 1];

  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int K = p.K, C = p.chunks;
  const int row_bytes = K * BITS / 8;

  // ---- loads of one chunk: the lane's flush scales and epilogue operands first (a window's flush
  // then waits only for its own weights), then the CH weight loads ----
  auto issue = [&](Buf &b, int tile, int chunk) {
    const int n0 = tile * 16;
    const int rows = tile < p.tiles ? min(16, p.N - n0) : 0;
    if constexpr (SCALED) {
      const __amdgpu_buffer_rsrc_t sb =
          buffer_rsrc(p.scales + (size_t)(rows > 0 ? n0 : 0) * p.G, (size_t)rows * p.G * 2);
#pragma unroll
      for (int w = 0; w < WIN; ++w) {
        const int u = w * WL + (R >= 4 ? (4 * g % R) / 4 : 0);  // the load this lane flushes
        const int kb = (chunk * CH + u) * CPW;
#pragma unroll
        for (int r = 0; r < NSL; ++r) {
          const int kk = kb + r * (CPW / NS);
          const int off = (u < CH && kk < K) ? (j * p.G + (kk >> p.group_shift)) * 2 : kOutOfRange;
          b.s[w * NSL + r] = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(sb, off, 0, 0));
        }
      }
    }
    if constexpr (KSPLIT == 1) {
      const int eoff = j < rows ? (n0 + j) * 2 : kOutOfRange;
      const size_t nb = (size_t)p.N * 2;
      b.e[0] = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(p.bias, p.bias ? nb : 0), eoff, 0, 0));
      b.e[1] = __builtin_bit_cast(
          f16, __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(p.residual, p.residual ? nb : 0), eoff, 0, 0));
      b.e[2] = SCALED ? (f16)1.0f
                      : __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(p.scales, nb), eoff, 0, 0));
    }
    const __amdgpu_buffer_rsrc_t wb =
        buffer_rsrc(p.codes + (size_t)(rows > 0 ? n0 : 0) * row_bytes, (size_t)rows * row_bytes);
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int k = (chunk * CH + u) * CPW + g * CPL;
      const int off = k < K ? j * row_bytes + k * BITS / 8 : kOutOfRange;
      b.w[u] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(wb, off, 0, 0));
    }
  };

  // Work list of this wave: (tile, chunk) items.
  int it_tile, it_chunk, c_tile, c_chunk, items;
  if constexpr (KSPLIT == 1) {
    const int gw = blockIdx.x * WAVES + wave, W = gridDim.x * WAVES;
    it_tile = c_tile = gw;
    it_chunk = c_chunk = 0;
    items = gw < p.tiles ? ((p.tiles - 1 - gw) / W + 1) * C : 0;
  } else {
    it_tile = c_tile = blockIdx.x;
    it_chunk = c_chunk = wave;
    items = wave < C ? (C - 1 - wave) / 4 + 1 : 0;
  }
  auto advance = [&](int &tile, int &chunk) {
    if constexpr (KSPLIT == 1) {
      if (++chunk == C) { chunk = 0; tile += gridDim.x * WAVES; }
    } else {
      chunk += 4;
    }
  };

  Buf buf[PD];
#pragma unroll
  for (int s = 0; s < PD - 1; ++s) {
    issue(buf[s], it_tile, it_chunk);
    advance(it_tile, it_chunk);
  }
  // Epilogue operands of the single tile (KSPLIT = 4): lanes 0..15 of wave 0.
  f16 ek[3] = {(f16)0.0f, (f16)0.0f, (f16)1.0f};
  if constexpr (KSPLIT == 4) {
    const int n0 = blockIdx.x * 16;
    const int eoff = (wave == 0 && n0 + j < p.N) ? (n0 + j) * 2 : kOutOfRange;
    const size_t nb = (size_t)p.N * 2;
    ek[0] = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(p.bias, p.bias ? nb : 0), eoff, 0, 0));
    ek[1] = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(p.residual, p.residual ? nb : 0), eoff, 0, 0));
    if constexpr (!SCALED)
      ek[2] = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(p.scales, nb), eoff, 0, 0));
  }

  // ---- stage the activation rows (slot order, factors), the zero region and the block bias sums.
  // Rows m >= M are not staged (no lane reads them); their block sums are zero.  Loads go out XU
  // per thread at a time, so a batch costs one memory round trip. ----
  {
    constexpr int TOTAL = MP * NB;
    constexpr int ITER = (TOTAL + NT - 1) / NT;
    constexpr int XU = ITER < 8 ? ITER : 8;
    for (int base = 0; base < ITER; base += XU) {  // uniform trip counts: the shuffles see every lane
      h8 xv[XU];
#pragma unroll
      for (int i = 0; i < XU; ++i) {
        const int idx = (base + i) * NT + t;
        const int m = idx / NB, b = idx - m * NB;
        const bool live = base + i < ITER && idx < TOTAL && m < p.M && 8 * b < K;
        xv[i] = __builtin_bit_cast(
            h8, __builtin_amdgcn_raw_buffer_load_b128(buffer_rsrc(p.x + (size_t)(live ? m : 0) * p.ldx, (size_t)K * 2),
                                                      live ? b * 16 : kOutOfRange, 0, 0));
      }
#pragma unroll
      for (int i = 0; i < XU; ++i) {
        const int idx = (base + i) * NT + t;
        const int m = idx / NB, b = idx - m * NB;
        const bool live = idx < TOTAL && m < p.M;
        h8 v;
        float bsum = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          v[e] = (f16)((float)xv[i][SL::perm[e]] * SL::factor[e]);
          bsum += (float)v[e] * SL::bias[e];
        }
        bsum += __shfl_xor(bsum, 1, 64);
        if constexpr (CPL == 32) bsum += __shfl_xor(bsum, 2, 64);
        if (base + i < ITER && idx < TOTAL) {
          if (live) *reinterpret_cast<h8 *>(xs + m * KP + 8 * b) = v;
          if (m == 0) *reinterpret_cast<h8 *>(xz + 8 * b) = h8{};
          if (b % (CPL / 8) == 0) xb[m * XBLD + b / (CPL / 8)] = live ? bsum : 0.0f;
        }
      }
    }
    for (int idx = t; idx < MP * 16; idx += NT) xb[(idx / 16) * XBLD + KP / CPL + idx % 16] = 0.0f;
  }
  __syncthreads();

  // A operand of load position v (0 .. WL-1) of a window: lane (j, g) is A row j = (m, r) with
  // m = j / R, r = j % R, active when m < M and (R >= 4) r == 4 v + g or (R < 4) r == g / BPR.
  const f16 *abase[WL];
  {
    const int m = j / R, r = j % R;
#pragma unroll
    for (int v = 0; v < WL; ++v) {
      const bool active = m < p.M && (R >= 4 ? r == 4 * v + g : r == g / BPR);
      abase[v] = (active ? xs + m * KP : xz) + g * CPL;
    }
  }

  float tot[NMR];
#pragma unroll
  for (int i = 0; i < NMR; ++i) tot[i] = 0.0f;
  auto consume = [&](Buf &b, int chunk) {
#pragma unroll
    for (int w = 0; w < WIN; ++w) {
      const int k0 = (chunk * CH + w * WL) * CPW;  // first code of the window (uniform)
      if (k0 >= K) break;
      f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int v = 0; v < WL; ++v) {
        const int u = w * WL + v;
        if (u >= CH) break;
        const int kb = k0 + v * CPW;
        if (kb >= K) break;
        asm volatile("" : "+v"(b.w[u]));  // decode here, not at the load
        const f16 *ap = abase[v] + kb;
#pragma unroll
        for (int q = 0; q < T8; ++q) {
          const h8 a = *reinterpret_cast<const h8 *>(ap + 8 * q);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, stream_decode<FMT>(b.w[u], q), acc, 0, 0, 0);
        }
      }
      // Lane (j, g) holds A rows 4g + r' (r' = 0..3) of output row j.
      if constexpr (R >= 4) {
        const int v = (4 * g % R) / 4;           // the window load of these rows
        const int m = 4 * g / R;                 // their activation row
        const f4 bias = *reinterpret_cast<const f4 *>(xb + m * XBLD + (k0 + v * CPW) / CPL);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float s;
          if constexpr (SCALED) s = (float)b.s[w * NSL + (r * NS) / 4];
          else s = (w * WL + v < CH) ? 1.0f : 0.0f;
          tot[0] += s * (acc[r] - bias[r]);
        }
      } else {
#pragma unroll
        for (int mi = 0; mi < NMR; ++mi) {
          const int m = 4 * g / R + mi;
          const f4 bias4 = *reinterpret_cast<const f4 *>(xb + m * XBLD + k0 / CPL);
#pragma unroll
          for (int rr = 0; rr < R; ++rr) {
            float bias = 0.0f;
#pragma unroll
            for (int q = 0; q < BPR; ++q) bias += bias4[rr * BPR + q];
            const float s = SCALED ? (float)b.s[w * NSL + (rr * BPR * NS) / 4] : 1.0f;
            tot[mi] += s * (acc[mi * R + rr] - bias);
          }
        }
      }
    }
  };
  // Final row sums of a tile: lanes of one activation row are reduced (R >= 8), then the owners
  // write y[m, n0 + j] with the reference's epilogue staging.
  auto finish = [&](float *v, const f16 *e, int n0) -> void {
    if constexpr (R >= 8) v[0] += __shfl_xor(v[0], 16, 64);
    if constexpr (R >= 16) v[0] += __shfl_xor(v[0], 32, 64);
    const bool owner = R >= 4 ? (4 * g % R) == 0 : true;
    if (!owner || n0 + j >= p.N) return;
#pragma unroll
    for (int mi = 0; mi < NMR; ++mi) {
      const int m = 4 * g / R + mi;
      if (m >= p.M) continue;
      float a = v[mi];
      if constexpr (!SCALED) a *= (float)e[2];
      f16 h = (f16)a;
      if (p.bias) h = (f16)((float)h + (float)e[0]);
      if (p.residual) h = (f16)((float)e[1] + (float)h);
      p.y[(size_t)m * p.ldy + n0 + j] = h;
    }
  };

  for (int done = 0; done < items; done += PD) {
#pragma unroll
    for (int s = 0; s < PD; ++s) {
      issue(buf[(s + PD - 1) % PD], it_tile, it_chunk);
      advance(it_tile, it_chunk);
      if (done + s < items) {
        consume(buf[s], c_chunk);
        if constexpr (KSPLIT == 1) {
          if (c_chunk == C - 1) {
            finish(tot, buf[s].e, c_tile * 16);
#pragma unroll
            for (int i = 0; i < NMR; ++i) tot[i] = 0.0f;
          }
        }
        advance(c_tile, c_chunk);
      }
    }
  }
  if constexpr (KSPLIT == 4) {
    if (wave > 0) {
#pragma unroll
      for (int i = 0; i < NMR; ++i) red[((wave - 1) * 64 + lane) * NMR + i] = tot[i];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int i = 0; i < NMR; ++i)
        tot[i] = ((tot[i] + red[lane * NMR + i]) + red[(64 + lane) * NMR + i]) + red[(128 + lane) * NMR + i];
      finish(tot, ek, blockIdx.x * 16);
    }
  }
}

// Streaming GEMV for 2 .. MP activation rows (MP = 8 or 16) with the reference's weights: each
// code is decoded to fp16(q * s) in registers (decode8, as in the single-tile kernels), so the
// MFMA accumulates the whole row of a tile and nothing is flushed before the tile's end:
// y[m, n] = fp16(sum_k x[m, k] * fp16(q[n, k] * s)) (+ bias), the products the other GEMV paths
// form.  A rows 0 .. M-1 are the activation rows (staged in the decode8 slot order); rows M .. 15
// read a zero row.  A wave streams 16-row tiles chunk by chunk (CH 16-byte loads per lane per
// chunk, PD chunks in flight), persistent over the grid like stream_gemv_kernel; a lane's 16-byte
// load holds CPL codes of one group (groups are >= 32 codes, powers of two, or one per row).
template <int FMT, bool SCALED, int MP, int KMAX, int CH, int PD, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void stream_rows_kernel(StreamParams p) {
  constexpr int CPL = FormatTraits<FMT>::CPL, BITS = FormatTraits<FMT>::BITS, T8 = CPL / 8;
  constexpr int CPW = 4 * CPL;                       // codes per load position (four lane groups)
  constexpr int KC = CH * CPW;                       // codes per chunk
  constexpr int KP = (KMAX + KC - 1) / KC * KC;      // staged row length (zero past K)
  constexpr int NB = KP / 8;                         // 8-code blocks of a staged row
  constexpr int NT = 64 * WAVES;
  constexpr int kOutOfRange = (int)0x80000000u;
  static_assert(MP == 8 || MP == 16, "MP is 8 or 16");
  __shared__ __align__(16) f16 xs[(MP + 1) * KP];    // activation rows 0 .. MP-1, then a zero row
  __shared__ uint32_t nf4_table[FMT == FMT_NF4 ? 256 : 1];

  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int K = p.K, C = p.chunks;
  const int row_bytes = K * BITS / 8;

  // fp16 operands are kept as 32-bit words (raw bits): arrays of 16-bit values would be packed
  // through scratch memory.
  struct Buf {
    u4 w[CH];
    uint32_t s[SCALED ? CH : 1];
    uint32_t e[2];  // bias and per-row scale of row n0 + j
  };
  // Loads of one chunk: the scales and epilogue operands first, then the CH weight loads.
  auto issue = [&](Buf &b, int tile, int chunk) {
    const int n0 = tile * 16;
    const int rows = tile < p.tiles ? min(16, p.N - n0) : 0;
    if constexpr (SCALED) {
      const __amdgpu_buffer_rsrc_t sb =
          buffer_rsrc(p.scales + (size_t)(rows > 0 ? n0 : 0) * p.G, (size_t)rows * p.G * 2);
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        const int k = (chunk * CH + u) * CPW + g * CPL;
        const int off = k < K ? (j * p.G + (k >> p.group_shift)) * 2 : kOutOfRange;
        b.s[u] = __builtin_amdgcn_raw_buffer_load_b16(sb, off, 0, 0);
      }
    }
    const int eoff = j < rows ? (n0 + j) * 2 : kOutOfRange;
    const size_t nb = (size_t)p.N * 2;
    b.e[0] = __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(p.bias, p.bias ? nb : 0), eoff, 0, 0);
    b.e[1] = SCALED ? 0u : __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(p.scales, nb), eoff, 0, 0);
    const __amdgpu_buffer_rsrc_t wb =
        buffer_rsrc(p.codes + (size_t)(rows > 0 ? n0 : 0) * row_bytes, (size_t)rows * row_bytes);
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int k = (chunk * CH + u) * CPW + g * CPL;
      const int off = k < K ? j * row_bytes + k * BITS / 8 : kOutOfRange;
      b.w[u] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(wb, off, 0, 0));
    }
  };

  // Work list of this wave: (tile, chunk) items, tiles gw, gw + W, ...
  const int gw = blockIdx.x * WAVES + wave, W = gridDim.x * WAVES;
  int it_tile = gw, it_chunk = 0, c_tile = gw, c_chunk = 0;
  const int items = gw < p.tiles ? ((p.tiles - 1 - gw) / W + 1) * C : 0;
  auto advance = [&](int &tile, int &chunk) {
    if (++chunk == C) { chunk = 0; tile += W; }
  };

  Buf buf[PD];
#pragma unroll
  for (int s = 0; s < PD - 1; ++s) {
    issue(buf[s], it_tile, it_chunk);
    advance(it_tile, it_chunk);
  }

  // ---- stage the activation rows in the decode8 slot order, and the zero row.  Loads go out XU
  // per thread at a time, so a batch costs one memory round trip. ----
  {
    constexpr int TOTAL = (MP + 1) * NB;
    constexpr int ITER = (TOTAL + NT - 1) / NT;
    constexpr int XU = ITER < 8 ? ITER : 8;
    for (int base = 0; base < ITER; base += XU) {
      h8 xv[XU];
#pragma unroll
      for (int i = 0; i < XU; ++i) {
        const int idx = (base + i) * NT + t;
        const int m = idx / NB, b = idx - m * NB;
        const bool live = base + i < ITER && idx < TOTAL && m < p.M && 8 * b < K;
        xv[i] = __builtin_bit_cast(
            h8, __builtin_amdgcn_raw_buffer_load_b128(buffer_rsrc(p.x + (size_t)(live ? m : 0) * p.ldx, (size_t)K * 2),
                                                      live ? b * 16 : kOutOfRange, 0, 0));
      }
#pragma unroll
      for (int i = 0; i < XU; ++i) {
        const int idx = (base + i) * NT + t;
        const int m = idx / NB, b = idx - m * NB;
        if (base + i < ITER && idx < TOTAL && (m < p.M || m == MP))
          *reinterpret_cast<h8 *>(xs + m * KP + 8 * b) = permute_block<FMT>(xv[i]);
      }
    }
  }
  if constexpr (FMT == FMT_NF4) build_nf4_pair_table(nf4_table);
  __syncthreads();

  const f16 *abase = xs + (j < p.M ? j : MP) * KP + g * CPL;
  f4 acc = {0.f, 0.f, 0.f, 0.f};
  auto consume = [&](Buf &b, int chunk) {
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int kb = (chunk * CH + u) * CPW;
      if (kb >= K) break;  // wave-uniform
      asm volatile("" : "+v"(b.w[u]));  // decode here, not at the load
      h2 s2 = {(f16)1.0f, (f16)1.0f};
      if constexpr (SCALED) {
        const f16 sv = __builtin_bit_cast(f16, (unsigned short)b.s[u]);
        s2 = h2{sv, sv};
      }
#pragma unroll
      for (int q = 0; q < T8; ++q) {
        const h8 a = *reinterpret_cast<const h8 *>(abase + kb + 8 * q);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, decode8<FMT, !SCALED>(b.w[u], q, s2, nf4_table), acc, 0, 0, 0);
      }
    }
  };
  // Lane (j, g) holds rows 4g .. 4g+3 (activation rows) of column j (weight row n0 + j).
  auto finish = [&](uint32_t ebits, uint32_t rbits, int n0) {
    const f16 ebias = __builtin_bit_cast(f16, (unsigned short)ebits);
    const f16 erow = __builtin_bit_cast(f16, (unsigned short)rbits);
    if (n0 + j < p.N) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 4 * g + r;
        if (m >= p.M) continue;
        float v = acc[r];
        if constexpr (!SCALED) v *= (float)erow;
        f16 h = (f16)v;
        if (p.bias) h = (f16)((float)h + (float)ebias);
        p.y[(size_t)m * p.ldy + n0 + j] = h;
      }
    }
    acc = f4{0.f, 0.f, 0.f, 0.f};
  };

  for (int done = 0; done < items; done += PD) {
#pragma unroll
    for (int s = 0; s < PD; ++s) {
      issue(buf[(s + PD - 1) % PD], it_tile, it_chunk);
      advance(it_tile, it_chunk);
      if (done + s < items) {
        consume(buf[s], c_chunk);
        if (c_chunk == C - 1) finish(buf[s].e[0], buf[s].e[1], c_tile * 16);
        advance(c_tile, c_chunk);
      }
    }
  }
}

// Streaming GEMV for 17 .. 32 activation rows (two 16-row halves of the MFMA A operand) with the
// reference's weights fp16(q * s) decoded in registers; each decoded B fragment feeds both halves.
// 32 staged rows of a long K do not fit in LDS, so the loop is K-outer: a workgroup owns WAVES *
// TPW consecutive 16-row tiles (TPW per wave, accumulators in registers) and walks K in chunks of
// KC codes; per chunk every row's KC activations are staged in one of two LDS stages (the next
// chunk's weights and activations are loaded during the current chunk), one barrier per chunk.
// A rows past M read a zero row.
template <int FMT, bool SCALED, int KC, int TPW, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void stream_wide_kernel(StreamParams p) {
  constexpr int CPL = FormatTraits<FMT>::CPL, BITS = FormatTraits<FMT>::BITS, T8 = CPL / 8;
  constexpr int CPW = 4 * CPL;                       // codes per load position (four lane groups)
  constexpr int CH = KC / CPW;                       // loads per lane per tile per chunk
  constexpr int NT = 64 * WAVES;
  constexpr int XCH = 32 * KC / 8;                   // 16-byte activation pieces per stage
  constexpr int XP = (XCH + NT - 1) / NT;            // per thread
  constexpr int kOutOfRange = (int)0x80000000u;
  static_assert(KC % CPW == 0 && CH >= 1, "chunk of whole loads");
  __shared__ __align__(16) f16 xs[2 * 32 * KC + KC];  // two stages of 32 rows, then a zero row
  __shared__ uint32_t nf4_table[FMT == FMT_NF4 ? 256 : 1];

  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int K = p.K, C = p.chunks;
  const int row_bytes = K * BITS / 8;
  const int tile0 = (blockIdx.x * WAVES + wave) * TPW;  // this wave's first tile

  // fp16 operands are kept as 32-bit words (raw bits): arrays of 16-bit values would be packed
  // through scratch memory.
  struct Buf {
    u4 w[TPW][CH];
    uint32_t s[TPW][SCALED ? CH : 1];
  };
  auto issue = [&](Buf &b, int chunk) {
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) {
      const int n0 = (tile0 + tt) * 16;
      const int rows = tile0 + tt < p.tiles ? min(16, p.N - n0) : 0;
      if constexpr (SCALED) {
        const __amdgpu_buffer_rsrc_t sb =
            buffer_rsrc(p.scales + (size_t)(rows > 0 ? n0 : 0) * p.G, (size_t)rows * p.G * 2);
#pragma unroll
        for (int u = 0; u < CH; ++u) {
          const int k = chunk * KC + u * CPW + g * CPL;
          b.s[tt][u] = __builtin_amdgcn_raw_buffer_load_b16(sb, k < K ? (j * p.G + (k >> p.group_shift)) * 2 : kOutOfRange, 0, 0);
        }
      }
      const __amdgpu_buffer_rsrc_t wb =
          buffer_rsrc(p.codes + (size_t)(rows > 0 ? n0 : 0) * row_bytes, (size_t)rows * row_bytes);
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        const int k = chunk * KC + u * CPW + g * CPL;
        b.w[tt][u] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(wb, k < K ? j * row_bytes + k * BITS / 8 : kOutOfRange, 0, 0));
      }
    }
  };
  // Activation pieces of a chunk: piece i = (row m, 8-code block b); rows past M and codes past K
  // read zeros.
  auto load_x = [&](h8 (&xv)[XP], int chunk) {
#pragma unroll
    for (int i = 0; i < XP; ++i) {
      const int idx = i * NT + t;
      const int m = idx / (KC / 8), b = idx % (KC / 8);
      const int k = chunk * KC + 8 * b;
      const bool live = idx < XCH && m < p.M && k < K;
      xv[i] = __builtin_bit_cast(
          h8, __builtin_amdgcn_raw_buffer_load_b128(buffer_rsrc(p.x + (size_t)(live ? m : 0) * p.ldx, (size_t)K * 2),
                                                    live ? k * 2 : kOutOfRange, 0, 0));
    }
  };
  auto store_x = [&](const h8 (&xv)[XP], int st) {
#pragma unroll
    for (int i = 0; i < XP; ++i) {
      const int idx = i * NT + t;
      if (idx < XCH) *reinterpret_cast<h8 *>(xs + st * 32 * KC + idx * 8) = permute_block<FMT>(xv[i]);
    }
  };

  Buf buf[2];
  h8 xv[XP];
  issue(buf[0], 0);
  load_x(xv, 0);
  for (int i = t; i < KC / 8; i += NT) *reinterpret_cast<h8 *>(xs + 2 * 32 * KC + i * 8) = h8{};
  if constexpr (FMT == FMT_NF4) build_nf4_pair_table(nf4_table);
  store_x(xv, 0);
  __syncthreads();

  f4 acc[TPW][2];
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt) acc[tt][0] = acc[tt][1] = f4{0.f, 0.f, 0.f, 0.f};
  // A operand of lane (j, g) for the two row halves: rows j and 16 + j (or the zero row).
  const int a_lo = (j < p.M ? j * KC : 2 * 32 * KC) + g * CPL;
  const int a_hi = (16 + j < p.M ? (16 + j) * KC : 2 * 32 * KC) + g * CPL;

  auto step = [&](auto stage) {
    constexpr int ST = decltype(stage)::value;
    Buf &b = buf[ST];
    const int sx = ST * 32 * KC;  // this stage's activation offset (rows past M use the zero row)
    const f16 *alo = xs + a_lo + (j < p.M ? sx : 0);
    const f16 *ahi = xs + a_hi + (16 + j < p.M ? sx : 0);
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) {
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        asm volatile("" : "+v"(b.w[tt][u]));  // decode here, not at the load
        h2 s2 = {(f16)1.0f, (f16)1.0f};
        if constexpr (SCALED) {
          const f16 sv = __builtin_bit_cast(f16, (unsigned short)b.s[tt][u]);
          s2 = h2{sv, sv};
        }
#pragma unroll
        for (int q = 0; q < T8; ++q) {
          const h8 bw = decode8<FMT, !SCALED>(b.w[tt][u], q, s2, nf4_table);
          const h8 x0 = *reinterpret_cast<const h8 *>(alo + u * CPW + 8 * q);
          const h8 x1 = *reinterpret_cast<const h8 *>(ahi + u * CPW + 8 * q);
          acc[tt][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x0, bw, acc[tt][0], 0, 0, 0);
          acc[tt][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x1, bw, acc[tt][1], 0, 0, 0);
        }
      }
    }
  };
  // Chunk c uses stage c % 2; chunk c + 1 is loaded meanwhile and stored into the other stage.
  for (int c = 0; c < C; c += 2) {
    if (c + 1 < C) {
      issue(buf[1], c + 1);
      load_x(xv, c + 1);
    }
    step(std::integral_constant<int, 0>{});
    if (c + 1 < C) store_x(xv, 1);
    __syncthreads();
    if (c + 1 >= C) break;
    if (c + 2 < C) {
      issue(buf[0], c + 2);
      load_x(xv, c + 2);
    }
    step(std::integral_constant<int, 1>{});
    if (c + 2 < C) store_x(xv, 0);
    __syncthreads();
  }

  // Lane (j, g) holds rows h * 16 + 4g .. + 3 of column j (weight row n0 + j) in acc[tt][h].
#pragma unroll
  for (int tt = 0; tt < TPW; ++tt) {
    const int n0 = (tile0 + tt) * 16;
    if (tile0 + tt >= p.tiles || n0 + j >= p.N) continue;
    const float rs = SCALED ? 1.0f : (float)p.scales[n0 + j];
    const float bias = p.bias ? (float)p.bias[n0 + j] : 0.0f;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 16 * h + 4 * g + r;
        if (m >= p.M) continue;
        f16 y = (f16)(acc[tt][h][r] * rs);
        if (p.bias) y = (f16)((float)y + bias);
        p.y[(size_t)m * p.ldy + n0 + j] = y;
      }
  }
}

// Launches stream_wide_kernel for 17 <= p.M <= 32 rows.
void launch_stream_wide(const StreamParams &p, int format, bool scaled, hipStream_t stream);

// Element e of a SLICED workgroup's tiles (tile e / (16 M), activation row (e / 16) % M, column
// e % 16): the slices' partials added in slice order from 0.0f, then the epilogue.
template <int TT, bool SCALED>
__device__ __forceinline__ void tile_rows_slice_sum(const StreamParams &p, __amdgpu_buffer_rsrc_t pb, int e, int M, int N,
                                                    int S) {
  constexpr int kOutOfRange = (int)0x80000000u;
  constexpr int SMAX = 8;  // slices whose partials are requested at once
  const int tl = e / (16 * M), m = (e / 16) - tl * M, n = (blockIdx.x * TT + tl) * 16 + (e & 15);
  const bool live = tl < TT && n < N;
  float sum = 0.0f;
  for (int s0 = 0; s0 < S; s0 += SMAX) {
    float v[SMAX];
#pragma unroll
    for (int q = 0; q < SMAX; ++q) {
      const int off = live && s0 + q < S ? (((s0 + q) * M + m) * N + n) * 4 : kOutOfRange;
      v[q] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(pb, off, 0, kSysCoherent));
    }
    // a slice past S reads +0.0f, which leaves the sum as it is (a sum that starts at +0.0f is
    // never -0.0f)
#pragma unroll
    for (int q = 0; q < SMAX; ++q) sum += v[q];
  }
  if (!live) return;
  if constexpr (!SCALED) {
    sum *= (float)p.scales[n];  // per-row INT8: the row's scale
    // the fp32 product, then fp16 (two roundings, as splitk_reduce_kernel), not one mixed-precision
    // multiply rounding straight to fp16
    asm volatile("" : "+v"(sum));
  }
  f16 h = (f16)sum;
  if (p.bias) h = (f16)((float)h + (float)p.bias[n]);
  p.y[(size_t)m * p.ldy + n] = h;
}

// End of a SLICED tile_rows_kernel workgroup (every thread calls it).  Wave 0 of each tile adds the
// other waves' sums (red, the order of the unsliced kernel) and writes the tile's fp32 partials of
// its slice.  Without tickets that is all (splitk_reduce_kernel follows).  With them the partials are
// written with system-scope coherent stores (as wide_add_slices does), and the workgroup counts itself
// in its tile column's ticket with a returning system-scope atomic once every wave's stores are
// complete; the one that counts last (gridDim.y - 1) reads the column's partials with coherent loads,
// adds the slices in slice order from 0.0f (splitk_reduce_kernel's order and values: the same y bit
// for bit), applies the epilogue (per-row scale, fp16, bias) and returns the ticket to zero.  No
// workgroup waits for another.
template <int TT, bool SCALED, int MH>
__device__ __forceinline__ void tile_rows_slices(const StreamParams &p, f4 (&acc)[MH], const float *red, int wave,
                                                 int lane, int n0, int rows, int M, int N) {
  constexpr int kOutOfRange = (int)0x80000000u;
  __shared__ uint32_t last;
  const int S = gridDim.y, j = lane & 15, g = lane >> 4;
  const bool through = p.tickets != nullptr;
  const __amdgpu_buffer_rsrc_t pb = buffer_rsrc(p.partial, (size_t)S * M * N * 4);
  if (wave == 0) {
#pragma unroll
    for (int h = 0; h < MH; ++h)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        acc[h][r] = ((acc[h][r] + red[(h * 64 + lane) * 4 + r]) + red[((MH + h) * 64 + lane) * 4 + r]) +
                    red[((2 * MH + h) * 64 + lane) * 4 + r];
    if (j < rows) {
#pragma unroll
      for (int hr = 0; hr < 4 * MH; ++hr) {
        const int m = 16 * (hr / 4) + 4 * g + hr % 4;
        const float v = acc[hr / 4][hr % 4];
        const int off = m < M ? ((blockIdx.y * M + m) * N + n0 + j) * 4 : kOutOfRange;
        if (through) __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), pb, off, 0, kSysCoherent);
        else __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), pb, off, 0, 0);
      }
    }
  }
  if (!through) return;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's partials are written through
  __syncthreads();
  if (threadIdx.x == 0)
    last = __hip_atomic_fetch_add(p.tickets + blockIdx.x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) ==
           (uint32_t)(S - 1);
  __syncthreads();
  if (!last) return;
  if (threadIdx.x == 0) __hip_atomic_store(p.tickets + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  // Every element of the workgroup's tiles (up to 32 rows: two elements per thread).
  for (int e = threadIdx.x; e < TT * 16 * M; e += 256 * TT)
    tile_rows_slice_sum<TT, SCALED>(p, pb, e, M, N, S);
}

// TT 16-row tiles per workgroup for 2 .. MP activation rows (MP = 4, 8, 16, or 32 as two 16-row
// MFMA A operands against each decoded weight fragment), the multi-row
// form of the single-tile one-row kernels: four waves per tile split K (wave 4 i + w of tile i
// takes k steps w, w + 4, ...), every weight load of a lane is issued straight-line before the
// first wait (up to 32 x 16 bytes), the M activation rows are staged once per workgroup in LDS in
// the decode8 slot order (zero from K on, and a zero row that A rows past M read) and serve its TT
// tiles, the scales of each tile's 16 rows too.  The reference's weights fp16(q * s) (decode8);
// each tile's four partial sums are added in a fixed order through LDS.
// y[m, n] = fp16(sum) (* per-row scale before rounding for per-row int8) (+ bias, fp16).
// The operands of the first loads come as leading scalar arguments (pre_*, the same values as in
// p), which the build preloads into registers at wave launch, so a workgroup dispatched while
// earlier ones flood the memory system issues its loads without waiting for its argument block.
// SLICED: rows longer than KMAX are cut into p.kslice-code slices (grid y; a slice is whole scale
// groups), each staged and summed as above into fp32 partials [slice, M, N]; with p.tickets the
// last workgroup of a tile column to count itself adds the slices in slice order (as
// splitk_reduce_kernel does otherwise) and writes y.
template <int FMT, bool SCALED, int KMAX, int MP, int TT, bool SLICED>
__global__ __launch_bounds__(256 * TT) void tile_rows_kernel(const uint8_t *pre_codes, const f16 *pre_x,
                                                             const f16 *pre_scales, const f16 *pre_bias, int pre_M,
                                                             int pre_N, int pre_K, int pre_G, int pre_ldx,
                                                             StreamParams p) {
  constexpr int CPL = FormatTraits<FMT>::CPL, BITS = FormatTraits<FMT>::BITS, T8 = CPL / 8;
  constexpr int KSTEP = 4 * CPL, KG = 4, WSTEP = KG * KSTEP;
  constexpr int D = (KMAX + WSTEP - 1) / WSTEP;      // weight loads per lane
  static_assert(D <= 32, "KMAX too long for one tile per workgroup");
  constexpr int XLD = KMAX + KSTEP + 8;              // staged row pitch (halves)
  constexpr int NBR = KMAX / 8;                      // 8-code blocks per staged row
  constexpr int NT = 256 * TT;                       // threads of the workgroup
  constexpr int XT = (MP * NBR + NT - 1) / NT;       // activation loads per thread
  static_assert(XT <= 16, "the staged rows are loaded in one batch");
  constexpr int GMAX = KMAX / 32;                    // groups per row at most (groups >= 32)
  constexpr int SC = SCALED ? (16 * GMAX + 255) / 256 : 0;
  constexpr int kOutOfRange = (int)0x80000000u;
  static_assert(MP == 4 || MP == 8 || MP == 16 || MP == 32, "MP is 4, 8, 16 or 32");
  constexpr int MH = MP > 16 ? 2 : 1;                // 16-row halves of the activation rows (MFMA A operands)
  // Four tiles per workgroup (1024 threads) measured slower with the preloaded operands: there the
  // argument block is read as before (the leading arguments are then unused and not preloaded).
  constexpr bool PRE = TT < 4;
  const uint8_t *const codes_ = PRE ? pre_codes : p.codes;
  const f16 *const x_ = PRE ? pre_x : p.x;
  const f16 *const scales_ = PRE ? pre_scales : p.scales;
  const f16 *const bias_ = PRE ? pre_bias : p.bias;
  const int M_ = PRE ? pre_M : p.M, N_ = PRE ? pre_N : p.N, G_ = PRE ? pre_G : p.G, ldx_ = PRE ? pre_ldx : p.ldx;
  __shared__ __align__(16) f16 xs[(MP + 1) * XLD];   // MP rows, then the zero row
  __shared__ __align__(16) f16 ss[TT][SCALED ? 16 * GMAX + 8 : 8];
  __shared__ float red[TT][(KG - 1) * 64 * 4 * MH];
  __shared__ uint32_t nf4_table[FMT == FMT_NF4 ? 256 : 1];

  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane((t >> 6) & 3);    // k split within the tile
  const int tile = __builtin_amdgcn_readfirstlane(t >> 8);          // tile of the workgroup
  const int tt = t & 255;                                           // thread within the tile
  const int j = lane & 15, g = lane >> 4;
  const int K = PRE ? pre_K : p.K;
  const int n0 = (blockIdx.x * TT + tile) * 16;
  const int rows = min(16, N_ - n0);  // <= 0: the tile lies past N (no loads, no stores)
  const int row_bytes = K * BITS / 8;
  // This workgroup's codes of each row: [kbeg, kbeg + KS) (the whole row unless SLICED), and the
  // scale groups of that range staged per row (GS; g0 the first).
  const int kbeg = SLICED ? (int)blockIdx.y * p.kslice : 0;
  const int KS = SLICED ? p.kslice : K;
  const int GS = SLICED && SCALED ? KS >> p.group_shift : G_;
  const int g0 = SLICED && SCALED ? kbeg >> p.group_shift : 0;
  const int blocks = KS >> 3;

  // Epilogue operands of row n0 + j (lanes of group 0): bias, per-row scale.
  const int eoff = g == 0 && j < rows ? (n0 + j) * 2 : kOutOfRange;
  const size_t nb = (size_t)N_ * 2;
  const uint32_t ebias = __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(bias_, bias_ ? nb : 0), eoff, 0, 0);
  const uint32_t erow = SCALED ? 0u : __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(scales_, nb), eoff, 0, 0);
  // Activation rows, issued before the weights (a wait for them leaves the weights in flight):
  // piece i = (row m, 8-code block b); blocks past K read zeros.
  h8 xv[XT];
#pragma unroll
  for (int i = 0; i < XT; ++i) {
    const int idx = i * NT + t;
    const int m = idx / NBR, b = idx - m * NBR;
    const bool live = m < M_ && b < blocks;
    xv[i] = __builtin_bit_cast(
        h8, __builtin_amdgcn_raw_buffer_load_b128(buffer_rsrc(x_ + (size_t)(live ? m : 0) * ldx_ + kbeg, (size_t)KS * 2),
                                                  live ? b * 16 : kOutOfRange, 0, 0));
  }
  // Scales of the tile's rows (16 x G halves), weights of this wave's k steps.
  uint32_t sreg[SC > 0 ? SC : 1];
  if constexpr (SCALED) {
    const __amdgpu_buffer_rsrc_t sb =
        buffer_rsrc(scales_ + (size_t)(rows > 0 ? n0 : 0) * G_, (size_t)max(rows, 0) * G_ * 2);
#pragma unroll
    for (int i = 0; i < SC; ++i) {
      const int e = tt + 256 * i;  // staged entry: row e / GS, group e % GS of the slice
      int off = e * 2;
      if constexpr (SLICED) {
        const int r = e / GS;
        off = e < 16 * GS ? (r * G_ + g0 + (e - r * GS)) * 2 : kOutOfRange;
      }
      sreg[i] = __builtin_amdgcn_raw_buffer_load_b16(sb, off, 0, 0);
    }
  }
  const __amdgpu_buffer_rsrc_t wb =
      buffer_rsrc(codes_ + (size_t)(rows > 0 ? n0 : 0) * row_bytes, (size_t)max(rows, 0) * row_bytes);
  u4 w[D];
#pragma unroll
  for (int u = 0; u < D; ++u) {
    const int k = (wave + KG * u) * KSTEP + g * CPL;
    w[u] = __builtin_bit_cast(
        u4, __builtin_amdgcn_raw_buffer_load_b128(wb, k < KS ? j * row_bytes + (kbeg + k) * BITS / 8 : kOutOfRange, 0, 0));
  }
  __builtin_amdgcn_sched_barrier(0);  // no use of the loaded data is scheduled above this point
#pragma unroll
  for (int i = 0; i < XT; ++i) {
    const int idx = i * NT + t;
    const int m = idx / NBR, b = idx - m * NBR;
    if (m < p.M) *reinterpret_cast<h8 *>(xs + m * XLD + 8 * b) = permute_block<FMT>(xv[i]);
  }
  // Zero tails (k from KMAX on) of the staged rows and the whole zero row.
  for (int i = t; i < MP * ((XLD - KMAX) / 8); i += NT) {
    const int m = i / ((XLD - KMAX) / 8), b = i - m * ((XLD - KMAX) / 8);
    if (m < p.M) *reinterpret_cast<h8 *>(xs + m * XLD + KMAX + 8 * b) = h8{};
  }
  for (int i = t; i < XLD / 8; i += NT) *reinterpret_cast<h8 *>(xs + MP * XLD + 8 * i) = h8{};
  if constexpr (SCALED) {
#pragma unroll
    for (int i = 0; i < SC; ++i)
      if (tt + 256 * i < 16 * GMAX) ss[tile][tt + 256 * i] = __builtin_bit_cast(f16, (unsigned short)sreg[i]);
    if (tt < 8) ss[tile][16 * GMAX + tt] = (f16)0.0f;
  }
  if constexpr (FMT == FMT_NF4) build_nf4_pair_table(nf4_table);
  __syncthreads();

  f4 acc[MH];
#pragma unroll
  for (int h = 0; h < MH; ++h) acc[h] = f4{0.f, 0.f, 0.f, 0.f};
  const f16 *a0 = xs + (j < p.M ? j : MP) * XLD + g * CPL;
  const f16 *a1 = xs + (MH > 1 && j + 16 < p.M ? j + 16 : MP) * XLD + g * CPL;
#pragma unroll
  for (int u = 0; u < D; ++u) {
    const int kb = (wave + KG * u) * KSTEP;
    if (kb >= KS) break;  // wave-uniform
    asm volatile("" : "+v"(w[u]));  // decode here, not at the load
    h2 s2 = {(f16)1.0f, (f16)1.0f};
    if constexpr (SCALED) {
      // past the row (or slice) the scale is zero (index past the row's groups reads the next row or
      // the pad, and the codes there are zero: only the zero scale makes fp16(q * s) zero for every format)
      const f16 sc = kb + g * CPL < KS ? ss[tile][j * GS + ((kb + g * CPL) >> p.group_shift)] : (f16)0.0f;
      s2 = h2{sc, sc};
    }
#pragma unroll
    for (int q = 0; q < T8; ++q) {
      const h8 bw = decode8<FMT, !SCALED>(w[u], q, s2, nf4_table);
      acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const h8 *>(a0 + kb + 8 * q), bw, acc[0], 0, 0, 0);
      if constexpr (MH > 1)
        acc[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const h8 *>(a1 + kb + 8 * q), bw, acc[1], 0, 0, 0);
    }
  }
  // Partial sums of waves 1..3 of each tile through LDS; its wave 0 adds them in order and writes it.
  if (wave > 0) {
#pragma unroll
    for (int h = 0; h < MH; ++h)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[tile][(((wave - 1) * MH + h) * 64 + lane) * 4 + r] = acc[h][r];
  }
  __syncthreads();
  if constexpr (SLICED) {
    tile_rows_slices<TT, SCALED, MH>(p, acc, red[tile], wave, lane, n0, rows, M_, N_);
    return;
  }
  if (wave > 0) return;
#pragma unroll
  for (int h = 0; h < MH; ++h)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      acc[h][r] = ((acc[h][r] + red[tile][(h * 64 + lane) * 4 + r]) + red[tile][((MH + h) * 64 + lane) * 4 + r]) +
                  red[tile][((2 * MH + h) * 64 + lane) * 4 + r];
  // Lane (j, g) holds rows 16 h + 4g .. + 3 of column j (weight row n0 + j) in acc[h].  The bias /
  // per-row scale of column j sit in lane j (group 0).
  const f16 bias = __builtin_bit_cast(f16, (unsigned short)__shfl((int)ebias, j, 64));
  const f16 rowscale = __builtin_bit_cast(f16, (unsigned short)__shfl((int)erow, j, 64));
  if (j >= rows) return;
#pragma unroll
  for (int hr = 0; hr < 4 * MH; ++hr) {
    const int m = 16 * (hr / 4) + 4 * g + hr % 4;
    if (m >= p.M) continue;
    float v = acc[hr / 4][hr % 4];
    if constexpr (!SCALED) v *= (float)rowscale;
    f16 h = (f16)v;
    if (p.bias) h = (f16)((float)h + (float)bias);
    p.y[(size_t)m * p.ldy + n0 + j] = h;
  }
}

#ifndef LB_TILE_ROWS_MIN_WGS
#define LB_TILE_ROWS_MIN_WGS 224  // tile_rows_kernel groups 4 (or 2) tiles per workgroup while this many remain
#endif
#ifndef LB_TILE_ROWS_FEW_ROWS
#define LB_TILE_ROWS_FEW_ROWS 4  // calls of at most this many activation rows ...
#endif
#ifndef LB_TILE_ROWS_MIN_WGS_FEW
#define LB_TILE_ROWS_MIN_WGS_FEW 256  // ... keep this many workgroups instead
#endif
#ifndef LB_TILE_ROWS_SHORT_K
#define LB_TILE_ROWS_SHORT_K 1024  // rows of at most this many codes take at most 2 tiles per workgroup
#endif
// Tiles per tile_rows_kernel workgroup for `tiles` 16-row tiles of K codes and M activation rows:
// the staged activation rows are shared by more tiles as long as the grid keeps LB_TILE_ROWS_MIN_WGS
// workgroups (LB_TILE_ROWS_MIN_WGS_FEW for up to LB_TILE_ROWS_FEW_ROWS rows, which stage little:
// INT4 14336x4096 as 448 workgroups of two tiles instead of 224 of four, M = 2 11.6 -> 10.5 us,
// M = 4 11.9 -> 10.9 us, where M = 8 measured 12.3 -> 13.8 us); four tiles only over long rows
// (short ones stage little, and two tiles with preloaded operands measured faster: the 49152x576
// head at M = 4 8.9 -> 7.3 us, at M = 16 10.1 -> 9.3 us).
inline int tile_rows_per_wg(long long tiles, long long K, long long M) {
  const long long min_wgs = M <= LB_TILE_ROWS_FEW_ROWS ? LB_TILE_ROWS_MIN_WGS_FEW : LB_TILE_ROWS_MIN_WGS;
  if (K > LB_TILE_ROWS_SHORT_K && tiles >= 4ll * min_wgs) return 4;
  return tiles >= 2ll * min_wgs ? 2 : 1;
}

// K slices of tile_rows_kernel for rows longer than it stages whole (4096 codes up to 8
// activation rows, 2048 up to 16, 1024 up to 32): the fewest, at most 16, that cut K into equal slices of whole
// 512-code steps and whole scale groups (any length for per-row scales); 0 when there is no such
// cut.  Rows that fit stay whole (1), unless there are fewer than LB_TILE_ROWS_FEW_TILES tiles: then
// the fewest slices of at least 1024 codes, at most 8, that give 256 tile slices (or the most there
// are), so more CUs share the weights (1024x4096 at M = 8: 6.9 -> 6.5 us, M = 2 6.6 -> 5.8 us).
#ifndef LB_TILE_ROWS_KMAX8
#define LB_TILE_ROWS_KMAX8 4096  // longest row tile_rows_kernel stages whole for up to 8 activation rows
#endif
#ifndef LB_TILE_ROWS_KMAX16
#define LB_TILE_ROWS_KMAX16 2048  // ... for 9..16 rows
#endif
#ifndef LB_TILE_ROWS_KMAX32
#define LB_TILE_ROWS_KMAX32 1024  // ... and for 17..32 rows
#endif
static_assert(LB_TILE_ROWS_KMAX8 <= 4096 && LB_TILE_ROWS_KMAX16 <= 2048 && LB_TILE_ROWS_KMAX32 <= 1024,
              "the staged lengths the launches instantiate");
#ifndef LB_TILE_ROWS_FEW_TILES
#define LB_TILE_ROWS_FEW_TILES 128  // rows that fit are sliced too (slices of >= 1024 codes) while the tiles number fewer than this
#endif
inline int tile_rows_slices_for(int M, long long N, long long K, long long group, bool per_row) {
  const long long kmax = M <= 8 ? LB_TILE_ROWS_KMAX8 : M <= 16 ? LB_TILE_ROWS_KMAX16 : LB_TILE_ROWS_KMAX32;
  if (K <= kmax) {
    const long long tiles = (N + 15) / 16;
    int best = 1;
    for (int s = 2; s <= 8 && tiles < LB_TILE_ROWS_FEW_TILES; ++s) {
      if (K % s) continue;
      const long long ks = K / s;
      if (ks < 1024 || ks % 512 != 0 || (!per_row && ks % group != 0)) continue;
      best = s;
      if (tiles * s >= 256) break;
    }
    return best;
  }
  for (int s = 2; s <= 16; ++s) {
    if (K % s) continue;
    const long long ks = K / s;
    if (ks <= kmax && ks % 512 == 0 && (per_row || ks % group == 0)) return s;
  }
  return 0;
}

// Launches tile_rows_kernel for 2 <= p.M <= 16 rows with M * K <= 32768 (K <= 4096), or over K
// slices of p.kslice codes (p.kslice > 0, the count from tile_rows_slices_for, fp32 partials in
// p.partial; with p.tickets the kernel adds them, else the caller launches splitk_reduce_kernel):
// the staged rows are loaded in one batch of at most 16 loads per thread.
void launch_tile_rows(const StreamParams &p, int format, bool scaled, hipStream_t stream);

// Launches stream_rows_kernel for 2 <= p.M <= 16 rows (K <= 4096, groups of at least 32 codes
// that are powers of two, or one per row).
void launch_stream_rows(const StreamParams &p, int format, bool scaled, hipStream_t stream);

// Launches stream_gemv_kernel for p.M <= 16 rows (defined with the decode launchers); `ns` is
// stream_group_span of the shape, and stream_rows_ok must hold for p.M > 1.
void launch_stream(const StreamParams &p, int format, bool scaled, int ns, hipStream_t stream);

}  // namespace lb
