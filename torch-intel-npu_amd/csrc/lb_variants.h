// gfx950 kernels of the two optional graph variants of the low-bit linear:
//
//   W8A8 (activation_scale; reference graph torch_npu_lowbit.py:224-231, validated against
//   torch_npu_int8_demo.py:34-51).  Activations are quantized on the power-of-two grid s_x,
//   qx = clip(rint(x / s_x), -128, 127); the int8 weight codes are used as stored; the
//   integer product runs on int8 MFMA (exact int32 sums); the epilogue scales by s_x and the
//   DPU's per-row weight step (fp16(127 s) - fp16(-128 s)) / 255 in fp64 and rounds once.
//     quantize_rows_kernel   x fp16 [M, K] -> qx int8 [M, K] (workspace)
//     i8_gemv_kernel<MT>     M <= 32: 16 weight rows per workgroup, v_mfma_i32_16x16x64_i8
//     i8_gemm_kernel<BM,BN>  M > 32: LDS tiles, v_mfma_i32_32x32x32_i8
//     generic_w8a8_kernel    any shape (K not a multiple of 64, unaligned codes)
//
//   compact_groups (reference torch_npu_lowbit.py:235-256).  One fp16 product per group of K
//   (the GEMV / GEMM kernels on grid slice z = group, or generic_pieces_kernel), then
//   compact_tree_kernel adds the pieces with the reference's balanced fp16 tree and the bias.
#pragma once
#include "lb_kernels.h"

namespace lb {

typedef int i4v __attribute__((ext_vector_type(4)));
typedef int i16v __attribute__((ext_vector_type(16)));

// Correctly rounded fp64 -> fp16: round to odd into fp32 (sticky bit kept in the last place),
// then one RNE to fp16.  fp32 carries 13 more significand bits than fp16, so the second
// rounding sees the exact tie / non-tie status of the first.
__device__ __forceinline__ f16 f64_to_f16(double r) {
  float f = (float)r;
  const double back = (double)f;
  if (back != r && r == r) {
    uint32_t b = __builtin_bit_cast(uint32_t, f);
    if (__builtin_fabs(back) > __builtin_fabs(r)) b -= 1;  // the neighbour toward zero
    f = __builtin_bit_cast(float, b | 1u);
  }
  return (f16)f;
}

// y[m, n] for an exact integer sum: fp16(acc * s_x * step_n), then fp16(y + b).
// step_n = (fp16(127 s_n) - fp16(-128 s_n)) / 255; 127 s_n and -128 s_n are exact in fp32.
__device__ __forceinline__ void store_w8a8(const LinearParams &p, int m, int n, int acc) {
  const float s = (float)p.scales[n];
  const double hi = (double)(f16)(127.0f * s);
  const double lo = (double)(f16)(-128.0f * s);
  const double step = (hi - lo) / 255.0;
  f16 h = f64_to_f16((double)acc * (double)p.act_scale * step);
  if (p.bias) h = (f16)((float)h + (float)p.bias[n]);
  p.y[(size_t)m * p.ldy + n] = h;
}

// clip(rint(x / s_x), -128, 127); x / s_x is exact (s_x a power of two), rint is half-to-even.
__device__ __forceinline__ int quantize_activation(f16 x, float inv_scale) {
  const float q = __builtin_rintf((float)x * inv_scale);
  return (int)fminf(fmaxf(q, -128.0f), 127.0f);
}

// qx[m, k] for K % 8 == 0: one thread per 8 activations.
__global__ __launch_bounds__(256) void quantize_rows_kernel(LinearParams p) {
  const int blocks = p.K >> 3;
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (size_t)p.M * blocks) return;
  const int m = (int)(idx / blocks), b = (int)(idx - (size_t)m * blocks);
  const h8 v = *reinterpret_cast<const h8 *>(p.x + (size_t)m * p.ldx + b * 8);
  const float inv = 1.0f / p.act_scale;  // exact: a power of two
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    lo |= (uint32_t)(quantize_activation(v[e], inv) & 0xFF) << (8 * e);
    hi |= (uint32_t)(quantize_activation(v[e + 4], inv) & 0xFF) << (8 * e);
  }
  *reinterpret_cast<uint2 *>(const_cast<int8_t *>(p.xq) + (size_t)m * p.K + b * 8) = uint2{lo, hi};
}

// W8A8 GEMV, M <= 32 (MT = 1 or 2 tiles of 16 rows of m).  One workgroup (4 waves) per 16 weight
// rows; wave w takes the 64-k steps w, w + 4, ...  Lane (j, g) loads 16 codes of row n0 + j at
// k = 64 s + 16 g (the B operand) and the 16 quantized activations of row m = 16 mt + j at the
// same k (the A operand): A and B use the same (lane group, byte) -> k map, so the MFMA sums
// the right products.  Rows past M or N read zeros (buffer bounds).  K % 64 == 0.
template <int MT>
__global__ __launch_bounds__(256) void i8_gemv_kernel(LinearParams p) {
  constexpr int D = 8;  // steps per batch
  constexpr int kOutOfRange = (int)0x80000000u;
  __shared__ i4v red[3][MT][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int rows = min(16, p.N - n0);
  const int steps = p.K >> 6;
  const __amdgpu_buffer_rsrc_t wbuf = buffer_rsrc(p.codes + (size_t)n0 * p.K, (size_t)rows * p.K);
  const __amdgpu_buffer_rsrc_t xbuf = buffer_rsrc(p.xq, (size_t)p.M * p.K);
  i4v acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = i4v{0, 0, 0, 0};
  for (int s0 = wave; s0 < steps; s0 += 4 * D) {
    i4v b[D], a[D][MT];
#pragma unroll
    for (int u = 0; u < D; ++u) {
      const int s = s0 + 4 * u;
      const int k = s * 64 + 16 * g;
      b[u] = __builtin_bit_cast(i4v, __builtin_amdgcn_raw_buffer_load_b128(wbuf, s < steps ? j * p.K + k : kOutOfRange, 0, 0));
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = 16 * mt + j;
        a[u][mt] = __builtin_bit_cast(
            i4v, __builtin_amdgcn_raw_buffer_load_b128(xbuf, s < steps && m < p.M ? m * p.K + k : kOutOfRange, 0, 0));
      }
    }
#pragma unroll
    for (int u = 0; u < D; ++u) {
      if (s0 + 4 * u >= steps) break;  // wave-uniform
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[u][mt], b[u], acc[mt], 0, 0, 0);
    }
  }
  if (wave > 0) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) red[wave - 1][mt][lane] = acc[mt];
  }
  __syncthreads();
  if (wave > 0) return;
  const int n = n0 + j;
  if (j >= rows) return;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const i4v sum = acc[mt] + red[0][mt][lane] + red[1][mt][lane] + red[2][mt][lane];
    // D layout of the 16x16 MFMA: lane (j, g) holds rows m = 4g + r of column j.
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 16 * mt + 4 * g + r;
      if (m < p.M) store_w8a8(p, m, n, sum[r]);
    }
  }
}

// W8A8 GEMM, M > 32.  256 threads (2 x 2 waves) per BM x BN tile, K steps of 64 bytes; the
// quantized activations and the codes of a step are loaded into registers one step ahead,
// written to LDS (row pitch 80 bytes), and multiplied on v_mfma_i32_32x32x32_i8.  K % 64 == 0.
template <int BM, int BN>
__global__ __launch_bounds__(256) void i8_gemm_kernel(LinearParams p) {
  constexpr int BK = 64, LD = BK + 16;  // bytes
  constexpr int TM = BM / 64, TN = BN / 64;
  constexpr int A_PER = BM * BK / 16 / 256, B_PER = BN * BK / 16 / 256;
  constexpr int kOutOfRange = (int)0x80000000u;
  __shared__ __align__(16) int8_t As[BM * LD];
  __shared__ __align__(16) int8_t Bs[BN * LD];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int bm = blockIdx.y * BM, bn = blockIdx.x * BN;
  const int rows_a = min(BM, p.M - bm), rows_b = min(BN, p.N - bn);
  const __amdgpu_buffer_rsrc_t xbuf = buffer_rsrc(p.xq + (size_t)bm * p.K, rows_a > 0 ? (size_t)rows_a * p.K : 0);
  const __amdgpu_buffer_rsrc_t wbuf = buffer_rsrc(p.codes + (size_t)bn * p.K, rows_b > 0 ? (size_t)rows_b * p.K : 0);
  int a_off[A_PER], b_off[B_PER];
#pragma unroll
  for (int i = 0; i < A_PER; ++i) {
    const int c = tid + 256 * i, r = c >> 2;
    a_off[i] = r < rows_a ? r * p.K + (c & 3) * 16 : kOutOfRange;
  }
#pragma unroll
  for (int i = 0; i < B_PER; ++i) {
    const int c = tid + 256 * i, r = c >> 2;
    b_off[i] = r < rows_b ? r * p.K + (c & 3) * 16 : kOutOfRange;
  }
  i4v ra[A_PER], rb[B_PER];
  auto load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_PER; ++i)
      ra[i] = __builtin_bit_cast(i4v, __builtin_amdgcn_raw_buffer_load_b128(xbuf, a_off[i] + k0, 0, 0));
#pragma unroll
    for (int i = 0; i < B_PER; ++i)
      rb[i] = __builtin_bit_cast(i4v, __builtin_amdgcn_raw_buffer_load_b128(wbuf, b_off[i] + k0, 0, 0));
  };
  i16v acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int jj = 0; jj < TN; ++jj) acc[i][jj] = i16v{};
  load(0);
  for (int k0 = 0; k0 < p.K; k0 += BK) {
    __syncthreads();  // every wave is done with the previous step's tiles
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
      const int c = tid + 256 * i;
      *reinterpret_cast<i4v *>(&As[(c >> 2) * LD + (c & 3) * 16]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      const int c = tid + 256 * i;
      *reinterpret_cast<i4v *>(&Bs[(c >> 2) * LD + (c & 3) * 16]) = rb[i];
    }
    __syncthreads();
    if (k0 + BK < p.K) load(k0 + BK);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 32) {
      i4v a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        a[i] = *reinterpret_cast<const i4v *>(&As[(wm * (BM / 2) + i * 32 + (lane & 31)) * LD + kk + 16 * (lane >> 5)]);
#pragma unroll
      for (int jj = 0; jj < TN; ++jj)
        b[jj] = *reinterpret_cast<const i4v *>(&Bs[(wn * (BN / 2) + jj * 32 + (lane & 31)) * LD + kk + 16 * (lane >> 5)]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int jj = 0; jj < TN; ++jj) acc[i][jj] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[jj], acc[i][jj], 0, 0, 0);
    }
  }
  // D layout of the 32x32 MFMA: lane l, register r -> row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int jj = 0; jj < TN; ++jj) {
      const int n = bn + wn * (BN / 2) + jj * 32 + (lane & 31);
      if (n >= p.N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = bm + wm * (BM / 2) + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m < p.M) store_w8a8(p, m, n, acc[i][jj][r]);
      }
    }
}

// W8A8 for any shape: one wave per (row n, 8 activation rows), integer sums.
__global__ __launch_bounds__(64) void generic_w8a8_kernel(LinearParams p) {
  const int n = blockIdx.x, m0 = blockIdx.y * 8, lane = threadIdx.x;
  const float inv = 1.0f / p.act_scale;
  int acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  const int8_t *w = reinterpret_cast<const int8_t *>(p.codes) + (size_t)n * p.K;
  for (int k = lane; k < p.K; k += 64) {
    const int q = w[k];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (m0 + i < p.M) acc[i] += quantize_activation(p.x[(size_t)(m0 + i) * p.ldx + k], inv) * q;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc[i] += __shfl_xor(acc[i], off, 64);
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (m0 + i < p.M) store_w8a8(p, m0 + i, n, acc[i]);
  }
}

// compact_groups pieces for any shape: grid (N, ceil(M / 8), groups); one wave per (row n,
// 8 activation rows, group z) writes fp16(sum over the group) to pieces[z, m, n].
__global__ __launch_bounds__(64) void generic_pieces_kernel(LinearParams p, int fmt, f16 *pieces) {
  const int n = blockIdx.x, m0 = blockIdx.y * 8, z = blockIdx.z, lane = threadIdx.x;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
  for (int k = z * p.group + lane; k < (z + 1) * p.group; k += 64) {
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
      if (m0 + i < p.M) pieces[((size_t)z * p.M + m0 + i) * p.N + n] = (f16)acc[i];
  }
}

// y[m, n] = fp16(tree(pieces[0..G-1, m, n]) + b): neighbours pair up in each round
// (0+1, 2+3, ...), an odd last piece moves up unpaired (torch_npu_lowbit.py:252-254).
// G <= 32; the rounds are unrolled over fixed slots so every index is a constant.
__global__ __launch_bounds__(256) void compact_tree_kernel(LinearParams p, const f16 *pieces, int groups) {
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (size_t)p.M * p.N) return;
  const int m = (int)(idx / p.N), n = (int)(idx % p.N);
  const size_t plane = (size_t)p.M * p.N;
  f16 v[32];
#pragma unroll
  for (int g = 0; g < 32; ++g) v[g] = g < groups ? pieces[g * plane + idx] : (f16)0.0f;
  int len = groups;
#pragma unroll
  for (int round = 0; round < 5; ++round) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (2 * i + 1 < len) v[i] = (f16)((float)v[2 * i] + (float)v[2 * i + 1]);
      else if (2 * i < len) v[i] = v[2 * i];
    }
    len = (len + 1) >> 1;
  }
  f16 h = v[0];
  if (p.bias) h = (f16)((float)h + (float)p.bias[n]);
  p.y[(size_t)m * p.ldy + n] = h;
}

}  // namespace lb
