// gfx950 kernels of the low-bit linear path.
//
//   gemv_kernel    decode regime (M <= 32): packed rows streamed with 16-byte loads,
//                  dequantized in registers, multiplied on v_mfma_f32_16x16x32_f16 with
//                  the activations as the (zero padded) A operand; optional split-K.
//   (the prefill GEMM, gemm2_kernel, is in lb_gemm.h)
//   generic_kernel any shape / group size (odd K, rows starting mid-byte, groups < 32).
//   unpack_kernel, dequant_kernel   bit-exact decode used by tests and by callers that
//                  want the reference's dequantized fp16 weights on device.
#pragma once
#include "lb_common.h"

namespace lb {

// Tuning knobs of the decode GEMV (compile-time; the shipped values are the defaults).
#ifndef LB_GEMV_WAVES
#define LB_GEMV_WAVES 4    // waves per workgroup
#endif
#ifndef LB_GEMV_BATCH
#define LB_GEMV_BATCH 8    // 16-byte loads per lane in one batch
#endif
#ifndef LB_GEMV_DOUBLE
#define LB_GEMV_DOUBLE 1   // double-buffer batches in registers
#endif
constexpr int kGemvWaves = LB_GEMV_WAVES;
constexpr int kGemvThreads = 64 * kGemvWaves;
constexpr int kGemvBatch = LB_GEMV_BATCH;
constexpr bool kGemvDouble = LB_GEMV_DOUBLE != 0;

// One batch of kGemvBatch 16-byte weight loads per lane, with their scales.
struct GemvBatch {
  u4 w[kGemvBatch];
  h2 s[kGemvBatch];
};

// Decode-regime GEMV.  The waves of a workgroup form RG row groups x KG k groups:
// wave (rg, kg) owns weight rows n0 + 16 rg .. +15 (the MFMA N dimension) and every KG-th
// k-step of the workgroup's K range; lane (j, g) streams row n0 + 16 rg + j at
// k = kb + g*CPL with 16-byte buffer loads.  Rows past N and bytes past the weight buffer
// read as zero (buffer bounds), so no load is predicated or clamped.  Activations
// (M <= 32 rows) are the A operand, staged per k-chunk in LDS with the format's slot
// permutation, followed by 4*CPL zeros per row and one all-zero row that lanes with
// m >= M read; A is therefore zero wherever k is outside the chunk, and every A read is
// unconditional.  Register batches are double-buffered and the first batch is issued
// before the activations are staged.  The KG partial sums are reduced through LDS; with
// split-K (gridDim.y > 1) fp32 partials go to the workspace and splitk_reduce_kernel
// finishes.
template <int FMT, int MT, int KG, bool SCALED>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(LinearParams p, int KC, int sc_ld) {
  constexpr int CPL = FormatTraits<FMT>::CPL;
  constexpr int BITS = FormatTraits<FMT>::BITS;
  constexpr int KSTEP = 4 * CPL;      // k covered by one wave-wide 16-byte load
  constexpr int WSTEP = KG * KSTEP;   // k distance between one wave's consecutive loads
  constexpr int T8 = CPL / 8;         // MFMAs per lane load
  constexpr int RG = kGemvWaves / KG;
  constexpr int ROWS = 16 * RG;
  constexpr int D = kGemvBatch;
  constexpr int PAD = 4 * CPL;        // zero tail after each staged activation row
  extern __shared__ __align__(16) unsigned char smem[];
  uint32_t *nf4_table = reinterpret_cast<uint32_t *>(smem);
  unsigned char *dyn = smem + (FMT == FMT_NF4 ? 1024 : 0);
  f16 *xs = reinterpret_cast<f16 *>(dyn);
  const int xs_ld = KC + PAD + 8;  // +16 bytes per row spreads the A rows over the banks
  // Scales of this workgroup's rows for the current chunk: ROWS x sc_ld halves, zero padded
  // (rows past N and the 4 entries after the chunk's last group read as zero).
  f16 *ss = xs + (p.M + 1) * xs_ld;
  select_slice(p);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // scalar: loop control stays uniform
  const int rg = wave % RG, kg = wave / RG;
  const int j = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * ROWS;
  const int n = n0 + rg * 16 + j;
  const int ks = blockIdx.y * p.kslice;
  const int ke = min(p.K, ks + p.kslice);
  const size_t row_bytes = (size_t)p.code_ld;
  // Buffer views start at this workgroup's first row, so offsets stay 32-bit.
  const __amdgpu_buffer_rsrc_t wbuf =
      buffer_rsrc(p.codes + (size_t)n0 * row_bytes, (size_t)(p.N - n0) * row_bytes);
  const int wrow = (rg * 16 + j) * (int)row_bytes;  // byte offset of this lane's row
  const int arow = j < p.M ? j : p.M;                // zero row for m >= M (MT == 1)
  const int arow2 = 16 + j < p.M ? 16 + j : p.M;     // second m tile (MT == 2)

  // Loads past the chunk end are sent to an offset beyond every buffer, which returns zero
  // without touching memory.
  constexpr int kOutOfRange = (int)0x80000000u;
  int sstride = sc_ld, g0 = 0;  // staged scale row stride and first staged group (set by stage)

  // Every batch issues all D loads (no branches, so load counting stays exact); those past
  // the chunk go out of range and cost no memory traffic.
  auto load = [&](GemvBatch &b, int kb, int kend) {
    const int base = wrow + (kb + g * CPL) * BITS / 8;
    const int room = kend - kb - g * CPL;  // load u is in range iff u * WSTEP < room
#pragma unroll
    for (int u = 0; u < D; ++u) {
      const bool ok = u * WSTEP < room;
      b.w[u] = __builtin_bit_cast(
          u4, __builtin_amdgcn_raw_buffer_load_b128(wbuf, (ok ? base : kOutOfRange) + u * WSTEP * BITS / 8, 0, 0));
    }
  };
  // Scales come from LDS when the batch is consumed (gathering them from memory per load
  // costs as much memory-pipeline time as the weights themselves).
  auto scales = [&](GemvBatch &b, int kb) {
    if constexpr (SCALED) {
      const int row = (rg * 16 + j) * sstride - g0;
#pragma unroll
      for (int u = 0; u < D; ++u) {
        const f16 sc = ss[row + ((kb + u * WSTEP + g * CPL) >> p.group_shift)];
        b.s[u] = h2{sc, sc};
      }
    }
  };

  f4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](GemvBatch &b, int kb, int kc, int kend) {
    scales(b, kb);
    const f16 *a0 = xs + arow * xs_ld + (kb - kc) + g * CPL;
    const f16 *a1 = xs + arow2 * xs_ld + (kb - kc) + g * CPL;
#pragma unroll
    for (int u = 0; u < D; ++u) {
      if (kb + u * WSTEP >= kend) break;  // scalar branch: kb, kend are wave-uniform
      h8 a[T8], a2[T8];
#pragma unroll
      for (int t = 0; t < T8; ++t) {  // A operands first: LDS latency overlaps the decode
        a[t] = *reinterpret_cast<const h8 *>(a0 + u * WSTEP + 8 * t);
        if constexpr (MT == 2) a2[t] = *reinterpret_cast<const h8 *>(a1 + u * WSTEP + 8 * t);
      }
#pragma unroll
      for (int t = 0; t < T8; ++t) {
        const h8 bw = decode8<FMT, !SCALED>(b.w[u], t, b.s[u], nf4_table);
        acc[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[t], bw, acc[0], 0, 0, 0);
        if constexpr (MT == 2) acc[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a2[t], bw, acc[1], 0, 0, 0);
      }
    }
  };

  // Scales of this workgroup's rows; when a chunk spans whole rows they are one contiguous
  // block, copied with 16-byte loads.
  const __amdgpu_buffer_rsrc_t sbuf = buffer_rsrc(SCALED ? p.scales + (size_t)n0 * p.G : p.scales,
                                                  SCALED ? (size_t)(p.N - n0) * p.G * 2 : 0);
  GemvBatch ba, bb;

  // Stage the activations (and scales) of [kc, kend) into LDS and issue the chunk's first
  // weight batch.  The first activation/scale block of every thread is loaded before the
  // weight batch so the LDS writes below do not wait behind the weights (loads complete
  // in issue order).
  auto stage = [&](int kc, int kend) {
    const int t = threadIdx.x;
    const int blocks = (kend - kc) >> 3;
    const int xtotal = p.M * blocks;
    g0 = kc >> p.group_shift;
    const int gcount = SCALED ? ((kend - 1) >> p.group_shift) - g0 + 1 : 0;
    const bool dense = SCALED && gcount == p.G && p.scales_aligned;
    sstride = dense ? p.G : sc_ld;
    // Valid scale halves of this workgroup; only whole 16-byte blocks use vector loads (the
    // buffer bounds check zeroes a dword that straddles the end of the scale array).
    const int svalid = dense ? min(ROWS, p.N - n0) * p.G : 0;
    const int stotal = svalid / 8;
    h8 xv = {};
    int xm = 0, xb = 0;
    if (t < xtotal) {
      xm = t / blocks;
      xb = t - xm * blocks;
      xv = *reinterpret_cast<const h8 *>(p.x + (size_t)xm * p.ldx + kc + xb * 8);
    }
    u4 sv = {};
    if (t < stotal) sv = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(sbuf, t * 16, 0, 0));
    load(ba, kc + kg * KSTEP, kend);
    if (t < xtotal) *reinterpret_cast<h8 *>(xs + xm * xs_ld + xb * 8) = permute_block<FMT>(xv);
    for (int idx = t + kGemvThreads; idx < xtotal; idx += kGemvThreads) {
      const int m = idx / blocks, b = idx - m * blocks;
      *reinterpret_cast<h8 *>(xs + m * xs_ld + b * 8) =
          permute_block<FMT>(*reinterpret_cast<const h8 *>(p.x + (size_t)m * p.ldx + kc + b * 8));
    }
    for (int idx = t; idx < p.M * (PAD / 8); idx += kGemvThreads) {  // zero tail after each row
      const int m = idx / (PAD / 8), b = idx - m * (PAD / 8);
      *reinterpret_cast<h8 *>(xs + m * xs_ld + blocks * 8 + b * 8) = h8{};
    }
    if constexpr (SCALED) {
      if (dense) {
        if (t < stotal) *reinterpret_cast<u4 *>(ss + t * 8) = sv;
        for (int idx = t + kGemvThreads; idx < stotal; idx += kGemvThreads)
          *reinterpret_cast<u4 *>(ss + idx * 8) =
              __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(sbuf, idx * 16, 0, 0));
        for (int idx = stotal * 8 + t; idx < ROWS * p.G + 8; idx += kGemvThreads)  // tail, absent rows, pad
          ss[idx] = idx < svalid ? p.scales[(size_t)n0 * p.G + idx] : (f16)0.0f;
      } else {
        for (int idx = t; idx < ROWS * sc_ld; idx += kGemvThreads) {
          const int r = idx / sc_ld, q = idx - r * sc_ld;
          f16 v = (f16)0.0f;
          if (q < gcount && n0 + r < p.N) v = p.scales[(size_t)(n0 + r) * p.G + g0 + q];
          ss[idx] = v;
        }
      }
    }
  };

  if constexpr (FMT == FMT_NF4) build_nf4_pair_table(nf4_table);
  for (int idx = threadIdx.x; idx < xs_ld / 8; idx += kGemvThreads)
    *reinterpret_cast<h8 *>(xs + p.M * xs_ld + idx * 8) = h8{};  // the zero row
  for (int kc = ks; kc < ke; kc += KC) {
    const int kend = min(ke, kc + KC);
    if (kc != ks) __syncthreads();  // every wave is done with the previous chunk
    stage(kc, kend);
    __syncthreads();
    if constexpr (kGemvDouble) {
      for (int kb = kc + kg * KSTEP;;) {  // ba holds the batch at kb
        const int kb2 = kb + D * WSTEP;
        if (kb2 < kend) load(bb, kb2, kend);
        compute(ba, kb, kc, kend);
        if (kb2 >= kend) break;
        const int kb3 = kb2 + D * WSTEP;
        if (kb3 < kend) load(ba, kb3, kend);
        compute(bb, kb2, kc, kend);
        if (kb3 >= kend) break;
        kb = kb3;
      }
    } else {
      for (int kb = kc + kg * KSTEP; kb < kend; kb += D * WSTEP) {
        if (kb != kc + kg * KSTEP) load(ba, kb, kend);
        compute(ba, kb, kc, kend);
      }
    }
  }

  if constexpr (KG > 1) {
    // Reduce the KG k-group partials of each row group through LDS (reusing xs).
    float *red = reinterpret_cast<float *>(dyn);
    __syncthreads();
    if (kg > 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        *reinterpret_cast<f4 *>(red + ((((kg - 1) * RG + rg) * MT + mt) * 64 + lane) * 4) = acc[mt];
    }
    __syncthreads();
    if (kg > 0) return;
#pragma unroll
    for (int q = 1; q < KG; ++q)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        acc[mt] += *reinterpret_cast<const f4 *>(red + ((((q - 1) * RG + rg) * MT + mt) * 64 + lane) * 4);
  }

  // D layout of the 16x16 MFMA: lane (j, g) holds rows m = 4g + r of column j.
  if (n >= p.N) return;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = mt * 16 + 4 * g + r;
      if (m >= p.M) continue;
      if (p.splits == 1)
        store_output(p, m, n, acc[mt][r]);
      else
        p.partial[((size_t)blockIdx.y * p.M + m) * p.N + n] = acc[mt][r];
    }
}

// Sums split-K partials in a fixed order (deterministic) and applies the epilogue.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(LinearParams p) {
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (size_t)p.M * p.N) return;
  const int m = (int)(idx / p.N), n = (int)(idx % p.N);
  float s = 0.0f;
  for (int sp = 0; sp < p.splits; ++sp) s += p.partial[((size_t)sp * p.M + m) * p.N + n];
  store_output(p, m, n, s);
}

// Natural-order (k ascending) fp16 decode of one dword of codes for LDS staging.
template <int FMT, bool SCALED>
__device__ __forceinline__ h8 decode8_natural(uint32_t w0, uint32_t w1, h2 s2, const uint32_t *nf4_table) {
  h2 p[4];
  if constexpr (FMT == FMT_INT4) {
    int4_pairs(w0, p);  // (c0,c2),(c4,c6),(c1,c3),(c5,c7)
    h2 q0 = {p[0].x, p[2].x}, q1 = {p[0].y, p[2].y}, q2 = {p[1].x, p[3].x}, q3 = {p[1].y, p[3].y};
    p[0] = q0; p[1] = q1; p[2] = q2; p[3] = q3;
  } else if constexpr (FMT == FMT_NF4) {
    p[0] = as_h2(nf4_table[w0 & 0xFFu]);
    p[1] = as_h2(nf4_table[(w0 >> 8) & 0xFFu]);
    p[2] = as_h2(nf4_table[(w0 >> 16) & 0xFFu]);
    p[3] = as_h2(nf4_table[w0 >> 24]);
  } else {  // INT8: two dwords
    h2 a[2], b[2];
    int8_pairs(w0, a);  // (b0,b2),(b1,b3)
    int8_pairs(w1, b);
    p[0] = h2{a[0].x, a[1].x}; p[1] = h2{a[0].y, a[1].y};
    p[2] = h2{b[0].x, b[1].x}; p[3] = h2{b[0].y, b[1].y};
  }
  if (SCALED) { p[0] *= s2; p[1] *= s2; p[2] *= s2; p[3] *= s2; }
  return __builtin_shufflevector(__builtin_shufflevector(p[0], p[1], 0, 1, 2, 3),
                                 __builtin_shufflevector(p[2], p[3], 0, 1, 2, 3),
                                 0, 1, 2, 3, 4, 5, 6, 7);
}

// Decoded integer value of element (n, k) for the flat packed layout.
__device__ __forceinline__ int decode_code(int fmt, const uint8_t *codes, size_t flat) {
  if (fmt == FMT_INT8) return (int)(int8_t)codes[flat];
  const uint8_t byte = codes[flat >> 1];
  const int c = (flat & 1) ? (byte >> 4) : (byte & 15);
  return fmt == FMT_INT4 ? ((c ^ 8) - 8) : c;
}

// Weight value used by the linear kernels: fp16(q*s) (or q for per-row int8, raw fp16).
__device__ __forceinline__ float weight_value(int fmt, const LinearParams &p, int n, int k) {
  if (fmt == FMT_FP16) return (float)reinterpret_cast<const f16 *>(p.codes)[(size_t)n * p.ldw + k];
  const int q = decode_code(fmt, p.codes, (size_t)n * p.K + k);
  f16 qh;
  if (fmt == FMT_NF4) {
    const float lit[16] = {LB_NF4_LITERALS};
    qh = (f16)lit[q];
  } else {
    qh = (f16)(float)q;
  }
  if (p.per_row) return (float)qh;
  return (float)(f16)(qh * p.scales[(size_t)n * p.G + k / p.group]);
}

// One wave per (row n, 8 activation rows): any shape and group size.
__global__ __launch_bounds__(64) void generic_kernel(LinearParams p, int fmt) {
  const int n = blockIdx.x, m0 = blockIdx.y * 8, lane = threadIdx.x;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
  for (int k = lane; k < p.K; k += 64) {
    const float w = weight_value(fmt, p, n, k);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (m0 + i < p.M) acc[i] += (float)p.x[(size_t)(m0 + i) * p.ldx + k] * w;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc[i] += __shfl_xor(acc[i], off, 64);
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (m0 + i < p.M) store_output(p, m0 + i, n, acc[i]);
  }
}

__global__ __launch_bounds__(256) void unpack_kernel(int fmt, const uint8_t *codes, size_t count, int8_t *out) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < count) out[i] = (int8_t)decode_code(fmt, codes, i);
}

__global__ __launch_bounds__(256) void dequant_kernel(int fmt, const uint8_t *codes, const f16 *scales,
                                                      int K, int group, int G, size_t count, f16 *out) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= count) return;
  const int q = decode_code(fmt, codes, i);
  f16 qh;
  if (fmt == FMT_NF4) {
    const float lit[16] = {LB_NF4_LITERALS};
    qh = (f16)lit[q];
  } else {
    qh = (f16)(float)q;
  }
  const size_t n = i / K;
  const int k = (int)(i - n * K);
  out[i] = qh * scales[n * G + k / group];
}

}  // namespace lb
