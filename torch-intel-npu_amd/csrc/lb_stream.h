// gfx950 streaming GEMV for one activation row over long INT4 / INT8 weight matrices (the tied
// head, the Llama-shaped projections): y[N] = x[K] . (q * s)[N, K]^T, scales applied to exact
// integer-code sums.
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
// Per-block sums come from the MFMA rows that a one-row product leaves unused: MFMA A row i is the
// activation masked to one block (lanes read a zero region of LDS where their row is inactive), so
// the 16 x 16 result holds 16 block partials per output row, flushed every window of 4 loads.
//
// A wave streams 16-row tiles chunk by chunk (CH 16-byte loads per lane per chunk, PD chunks in
// flight); the activation row, its zero twin and the block sums are staged in LDS once per
// workgroup.  KSPLIT = 1: persistent waves, each owning whole tiles; KSPLIT = 4: one tile per
// workgroup, the four waves taking interleaved chunks and reducing through LDS.
#pragma once
#include "fused_launch.h"

namespace lb {

template <int FMT> struct StreamTraits;
template <> struct StreamTraits<FMT_INT4> { static constexpr int CPL = 32, BITS = 4, T8 = 4; };
template <> struct StreamTraits<FMT_INT8> { static constexpr int CPL = 16, BITS = 8, T8 = 2; };

struct StreamParams {
  const f16 *x;           // [K]
  const uint8_t *codes;   // [N, K * bits / 8]
  const f16 *scales;      // [N, G]
  f16 *y;                 // [N]
  const f16 *bias;        // [N] or null
  const f16 *residual;    // [N] or null (may equal y)
  int N, K, G, group_shift;
  int tiles, chunks;      // 16-row tiles; chunks per tile row
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

// NS: scales a lane reads per flush (the groups one 4*CPL-code load spans: 1, 2 or 4).
template <int CH, int NS, bool SCALED>
struct StreamBuf {
  static constexpr int WIN = (CH + 3) / 4;
  u4 w[CH];
  f16 s[SCALED ? WIN * NS : 1];
  f16 e[3];                // bias, residual, per-row scale of the lane's row (KSPLIT = 1)
};

template <int FMT, bool SCALED, int NS, int KMAX, int CH, int PD, int KSPLIT>
__global__ __launch_bounds__(256) void stream_gemv_kernel(StreamParams p) {
  using TR = StreamTraits<FMT>;
  using SL = StreamSlots<FMT>;
  using Buf = StreamBuf<CH, NS, SCALED>;
  constexpr int CPL = TR::CPL, CPW = 4 * CPL, BITS = TR::BITS, T8 = TR::T8;
  constexpr int KC = CH * CPW;                       // codes per chunk
  constexpr int KP = (KMAX + KC - 1) / KC * KC;      // staged row length
  constexpr int WIN = Buf::WIN;                      // flush windows per chunk
  constexpr int NB = KP / 8;                         // 8-code groups of the staged row
  constexpr int XPER = (NB + 255) / 256;
  constexpr int kOutOfRange = (int)0x80000000u;
  static_assert(KSPLIT == 1 || KSPLIT == 4, "KSPLIT is 1 or 4");
  __shared__ __align__(16) f16 xs[KP];
  __shared__ __align__(16) f16 xz[KP];
  __shared__ __align__(16) float xb[KP / CPL + 16];
  __shared__ float red[KSPLIT > 1 ? 3 * 16 : 1];

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
        const int u = 4 * w + g;  // the load whose blocks this lane flushes
        const int kb = (chunk * CH + u) * CPW;
#pragma unroll
        for (int r = 0; r < NS; ++r) {
          const int kk = kb + r * (CPW / NS);
          const int off = (u < CH && kk < K) ? (j * p.G + (kk >> p.group_shift)) * 2 : kOutOfRange;
          b.s[w * NS + r] = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(sb, off, 0, 0));
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
    const int gw = blockIdx.x * 4 + wave, W = gridDim.x * 4;
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
      if (++chunk == C) { chunk = 0; tile += gridDim.x * 4; }
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
    const int eoff = (wave == 0 && g == 0 && n0 + j < p.N) ? (n0 + j) * 2 : kOutOfRange;
    const size_t nb = (size_t)p.N * 2;
    ek[0] = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(p.bias, p.bias ? nb : 0), eoff, 0, 0));
    ek[1] = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(p.residual, p.residual ? nb : 0), eoff, 0, 0));
    if constexpr (!SCALED)
      ek[2] = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(p.scales, nb), eoff, 0, 0));
  }

  // ---- stage the activation row (slot order, factors), its zero twin and the block bias sums ----
  {
    const __amdgpu_buffer_rsrc_t xbuf = buffer_rsrc(p.x, (size_t)K * 2);
    h8 xv[XPER];
#pragma unroll
    for (int i = 0; i < XPER; ++i) {
      const int b = t + 256 * i;
      xv[i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(xbuf, b < NB ? b * 16 : kOutOfRange, 0, 0));
    }
#pragma unroll
    for (int i = 0; i < XPER; ++i) {
      const int b = t + 256 * i;
      h8 v;
      float bsum = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[e] = (f16)((float)xv[i][SL::perm[e]] * SL::factor[e]);
        bsum += (float)v[e] * SL::bias[e];
      }
      bsum += __shfl_xor(bsum, 1, 64);
      if constexpr (CPL == 32) bsum += __shfl_xor(bsum, 2, 64);
      if (b < NB) {
        *reinterpret_cast<h8 *>(xs + 8 * b) = v;
        *reinterpret_cast<h8 *>(xz + 8 * b) = h8{};
        if (b % (CPL / 8) == 0) xb[b / (CPL / 8)] = bsum;
      }
    }
    if (t < 16) xb[KP / CPL + t] = 0.0f;
  }
  __syncthreads();

  // A operand of load position u' (0..3) of a window: lane (j, g) is row j of the MFMA A matrix and
  // is active for position u' when j == 4 u' + g; inactive lanes read zeros.
  const f16 *abase[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) abase[v] = (j == 4 * v + g ? xs : xz) + g * CPL;

  float tot = 0.0f;
  auto consume = [&](Buf &b, int chunk) {
#pragma unroll
    for (int w = 0; w < WIN; ++w) {
      const int k0 = (chunk * CH + 4 * w) * CPW;  // first code of the window (uniform)
      if (k0 >= K) break;
      f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int u = 4 * w + v;
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
      // Lane (j, g) holds rows 4g + r: the blocks r of the window's load g.
      const f4 bias = *reinterpret_cast<const f4 *>(xb + (k0 + g * CPW) / CPL);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float s;
        if constexpr (SCALED) s = (float)b.s[w * NS + (r * NS) / 4];
        else s = (4 * w + g < CH) ? 1.0f : 0.0f;
        tot += s * (acc[r] - bias[r]);
      }
    }
  };
  auto finish = [&](float v, const f16 *e, int n0) -> void {
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    if (g == 0 && n0 + j < p.N) {
      if constexpr (!SCALED) v *= (float)e[2];
      f16 h = (f16)v;
      if (p.bias) h = (f16)((float)h + (float)e[0]);
      if (p.residual) h = (f16)((float)e[1] + (float)h);
      p.y[n0 + j] = h;
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
            tot = 0.0f;
          }
        }
        advance(c_tile, c_chunk);
      }
    }
  }
  if constexpr (KSPLIT == 4) {
    float v = tot;
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    if (wave > 0 && g == 0) red[(wave - 1) * 16 + j] = v;
    __syncthreads();
    if (wave == 0) {
      if (g == 0) v = ((v + red[j]) + red[16 + j]) + red[32 + j];
      else v = 0.0f;
      // finish() reduces over the lane groups again: only lanes g == 0 carry the sum
      finish(v, ek, blockIdx.x * 16);
    }
  }
}

}  // namespace lb
