// gfx950 kernels of one SmolLM decode step (one sequence, one token).
//
//   rows_gemv_kernel      one-row linear over many rows (no correction): several 16-row tiles per
//                         workgroup share the staged activation row.
//   fused_gemv_kernel     up to three low-bit linears that share one activation row, in one
//                         launch, with the layer's neighbouring element-wise work folded in:
//                         a prologue (RMSNorm, or SiLU(gate) * up) that every workgroup
//                         applies to the row it stages, the rank-r correction z = fp16(x.V^T)
//                         computed inside each workgroup while its weights are in flight, and
//                         an epilogue that adds fp16(z.U^T) and, optionally, a residual.
//   decode_attention_kernel  RoPE of the new query/key row, KV append at the device-held
//                         position, scores, softmax and P.V for one query head.
//   argmax_next_kernel    greedy token of the logits row; writes it, advances the position and
//                         gathers the next input embedding.
//
// Staging (fp16 rounding points) is that of the reference CPU layer, torch_npu_smollm.py:142-193:
// RMSNorm fp16(fp16(x * rsqrt(mean(x^2) + eps)) * gamma); RoPE fp16(fp16(t cos) + fp16(rot(t) sin));
// scores fp16(q.k), fp16(* scale); softmax in fp32 rounded to fp16; P.V fp32 -> fp16;
// MLP fp16(fp16(silu(gate)) * up); residual fp16(x + delta).
#pragma once
#include "fused_launch.h"

namespace lb {

// Cross-lane moves on the VALU's data-parallel primitives (DPP), a few cycles each instead of an
// LDS permute round trip.  Lane layouts (rows of 16 lanes): quad_perm [1,0,3,2] and [2,3,0,1]
// swap neighbours at distance 1 and 2, row_half_mirror maps lane i of each 8 to 7 - i,
// row_mirror lane i of each 16 to 15 - i, row_shl:1 gives lane i the value of lane i + 1 (0 at
// the row's end), row_ror:n the value of lane i - n (mod 16).
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;
constexpr int kDppRowShl1 = 0x101, kDppRowRor4 = 0x124, kDppRowRor8 = 0x128;

template <int CTRL>
__device__ __forceinline__ int dpp_move(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(float, dpp_move<CTRL>(__builtin_bit_cast(int, v)));
}

// Sum over each aligned group of 8 / 16 lanes, the same bits in every lane of the group (each
// step adds two equal-shaped partial sums, in either order the same value).
__device__ __forceinline__ float sum8(float v) {
  v += dpp_move<kDppXor1>(v);
  v += dpp_move<kDppXor2>(v);
  return v + dpp_move<kDppHalfMirror>(v);
}
__device__ __forceinline__ float sum16(float v) {
  v = sum8(v);
  return v + dpp_move<kDppMirror>(v);
}
__device__ __forceinline__ float lane_value(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Whole-wave sum / max (every lane active), wave-uniform: the four row results combined in a
// fixed order.
__device__ __forceinline__ float wave_sum(float v) {
  v = sum16(v);
  return ((lane_value(v, 0) + lane_value(v, 16)) + lane_value(v, 32)) + lane_value(v, 48);
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_move<kDppXor1>(v));
  v = fmaxf(v, dpp_move<kDppXor2>(v));
  v = fmaxf(v, dpp_move<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_move<kDppMirror>(v));
  return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

// 64-bit keys across lanes: the two halves move on DPP / readlane separately.
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_move64(uint64_t v) {
  const uint32_t lo = (uint32_t)dpp_move<CTRL>((int)(uint32_t)v);
  const uint32_t hi = (uint32_t)dpp_move<CTRL>((int)(uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t lane_value64(uint64_t v, int lane) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), lane);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t max64(uint64_t a, uint64_t b) { return a > b ? a : b; }
// Largest key of each row of 16 lanes, in every lane of the row; of the whole wave, wave-uniform.
__device__ __forceinline__ uint64_t row_max64(uint64_t v) {
  v = max64(v, dpp_move64<kDppXor1>(v));
  v = max64(v, dpp_move64<kDppXor2>(v));
  v = max64(v, dpp_move64<kDppHalfMirror>(v));
  return max64(v, dpp_move64<kDppMirror>(v));
}
__device__ __forceinline__ uint64_t wave_max64(uint64_t v) {
  v = row_max64(v);
  return max64(max64(lane_value64(v, 0), lane_value64(v, 16)), max64(lane_value64(v, 32), lane_value64(v, 48)));
}

__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }

// SiLU from the hardware exp2 and reciprocal (about 1 fp32 ulp each; the result is rounded to
// fp16 right after, as in the reference staging).
__device__ __forceinline__ float silu_fast(float v) {
  return v * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(v * -1.4426950408889634f));
}

// c + a.b over fp16 pairs and blocks on v_dot2c_f32_f16 (exact fp16 products, fp32 sums).
__device__ __forceinline__ float dot2(h2 a, h2 b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }
__device__ __forceinline__ h2 pair_of(const h8 &v, int i) { return h2{v[2 * i], v[2 * i + 1]}; }

// Problem pi (0..2, wave-uniform) of a fused launch, selected field by field: a copy chosen by
// index would be kept in scratch memory.
__device__ __forceinline__ FusedProblem problem_of(const FusedParams &p, int pi) {
  const FusedProblem &a = p.prob[0], &b = p.prob[1], &c = p.prob[2];
  FusedProblem r;
#define LB_PICK(f) r.f = pi == 0 ? a.f : (pi == 1 ? b.f : c.f)
  LB_PICK(codes); LB_PICK(scales); LB_PICK(y); LB_PICK(bias); LB_PICK(residual); LB_PICK(down); LB_PICK(up);
  LB_PICK(N); LB_PICK(rank); LB_PICK(up_ld); LB_PICK(tiles_end); LB_PICK(zend);
#undef LB_PICK
  return r;
}

// One rotate-half RoPE element with the reference's three fp16 roundings,
// fp16(fp16(x * c) + fp16(r * s)).  Contraction stays off: once x * c is narrowed to an fp16
// multiply (exact, as both factors are fp16) the compiler would otherwise fuse it with the add
// and drop the first rounding.
__device__ __forceinline__ f16 rope_element(float x, float r, float c, float s) {
#pragma clang fp contract(off)
  const f16 a = (f16)(x * c);
  const f16 b = (f16)(r * s);
  return (f16)((float)a + (float)b);
}

// Smallest group size the KMAX variant stages scales for: KMAX <= 1536 handles group 32, the
// long-K variants (one-row lb_linear calls) need group >= 64.
template <int KMAX> struct FusedGroupMin { static constexpr int value = KMAX <= 1536 ? 32 : 64; };

// The correction term d = sum_r z[r] * U[row][r] (fp32, r in order), eight ranks per step.  zs
// and the staged U row must be zero from rank up to the next multiple of eight.
__device__ __forceinline__ float correction_dot(const float *zs, const f16 *urow, int rank) {
  float d = 0.0f;
#pragma unroll
  for (int r8 = 0; r8 < kFusedMaxRank / 8; ++r8) {
    if (8 * r8 < rank) {
      const h8 u = *reinterpret_cast<const h8 *>(urow + 8 * r8);
      const f4 z0 = *reinterpret_cast<const f4 *>(zs + 8 * r8);
      const f4 z1 = *reinterpret_cast<const f4 *>(zs + 8 * r8 + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) d += z0[e] * (float)u[e];
#pragma unroll
      for (int e = 0; e < 4; ++e) d += z1[e] * (float)u[4 + e];
    }
  }
  return d;
}

// Stages a lane's 8-column piece of a U row (columns 8 uq .. 8 uq + 7), zero from column rank on.
__device__ __forceinline__ void stage_u_piece(f16 *dst, const u4 &piece, int uq, int rank) {
  h8 u = __builtin_bit_cast(h8, piece);
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (8 * uq + e >= rank) u[e] = (f16)0.0f;
  *reinterpret_cast<h8 *>(dst) = u;
}

// The prologue's scale factor: inv = 1 / sqrt(mean(x^2) + eps) for RMSNorm (1 otherwise), summed in
// the same order by every workgroup of a launch (thread, wave, then the four waves), so all of them
// stage the same row.  Contains a workgroup barrier when the prologue is RMSNorm.
template <int XB>
__device__ __forceinline__ float prologue_inv(const FusedParams &p, const h8 (&xv)[XB], float *wsum, int lane, int wave) {
  if (p.prologue != PRO_RMSNORM) return 1.0f;
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < XB; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) s += (float)xv[i][e] * (float)xv[i][e];
  s = wave_sum(s);
  if (lane == 0) wsum[wave] = s;
  __syncthreads();
  const float total = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
  return 1.0f / sqrtf(total / (float)p.K + p.eps);
}

// Eight staged elements of the prologue: RMSNorm fp16(fp16(x * inv) * gamma), SiLU-multiply
// fp16(fp16(silu(x)) * x2), or x itself.
__device__ __forceinline__ h8 prologue_apply(const FusedParams &p, const h8 &x, const h8 &a, float inv) {
  h8 v;
  if (p.prologue == PRO_RMSNORM) {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (f16)((float)(f16)((float)x[e] * inv) * (float)a[e]);
  } else if (p.prologue == PRO_SILU_MUL) {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (f16)((float)(f16)silu((float)x[e]) * (float)a[e]);
  } else {
    v = x;
  }
  return v;
}

// `passed` of a shared-z call, read at the workgroup's start with a system-scope load (performed at
// the memory side, past the per-XCD L2s); shared_z_tag turns it into the launch's tag,
// (passed / tiles + 1) mod 2^16.
__device__ __forceinline__ uint64_t shared_z_passed(const FusedParams &p) {
  return __hip_atomic_load(p.zslot + kFusedZPassedOffset / 8, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ __forceinline__ uint32_t shared_z_tag(const FusedParams &p, uint64_t passed) {
  const uint32_t tiles = (uint32_t)p.prob[kFusedMaxProblems - 1].tiles_end;
  return (uint32_t)((passed / tiles + 1) & 0xFFFF);
}

// One z workgroup of a shared-z launch (blockIdx.x < p.zblocks): ranks [r0, r0 + 6) of one problem,
// z = fp16(x'.V^T) with x' the staged prologue row, published as two tagged 64-bit words with
// system-scope atomic stores.  32 threads per rank row each take every 32nd 16-byte block of it;
// all loads are issued first.
template <int KMAX>
__device__ __forceinline__ void fused_z_block(const FusedParams &p, f16 *xs, float *wsum, f16 *zsh) {
  constexpr int TPR = 32;                             // threads per rank row (8 groups, 6 used)
  constexpr int ZI = (KMAX / 8 + TPR - 1) / TPR;      // 16-byte V loads per thread
  constexpr int XB = (KMAX / 8 + 255) / 256;
  constexpr int kOutOfRange = (int)0x80000000u;
  static_assert(kFusedZRanks <= 256 / TPR, "one thread group per rank");
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int K = p.K, blocks = K >> 3;
  const int b = blockIdx.x;
  const int zp = b < p.prob[0].zend ? 0 : (b < p.prob[1].zend ? 1 : 2);
  const FusedProblem Z = problem_of(p, zp);
  int zfirst = 0;
  if (zp == 1) zfirst = p.prob[0].zend;
  if (zp == 2) zfirst = p.prob[1].zend;
  const int zi = b - zfirst;                          // z workgroup of the problem: words 2 zi, 2 zi + 1
  const int r0 = zi * kFusedZRanks;
  const int rr = t / TPR, li = t % TPR;
  const bool live = rr < kFusedZRanks && r0 + rr < Z.rank;
  const uint64_t passed = shared_z_passed(p);
  const size_t kb = (size_t)K * 2;
  const f16 *aux = p.prologue == PRO_SILU_MUL ? p.x2 : p.gamma;
  const __amdgpu_buffer_rsrc_t abuf = buffer_rsrc(aux, p.prologue == PRO_NONE ? 0 : kb);
  const __amdgpu_buffer_rsrc_t xbuf = buffer_rsrc(p.x, kb);
  h8 av[XB], xv[XB];
#pragma unroll
  for (int i = 0; i < XB; ++i) {
    const int blk = t + 256 * i;
    av[i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(abuf, blk < blocks ? blk * 16 : kOutOfRange, 0, 0));
  }
#pragma unroll
  for (int i = 0; i < XB; ++i) {
    const int blk = t + 256 * i;
    xv[i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(xbuf, blk < blocks ? blk * 16 : kOutOfRange, 0, 0));
  }
  const __amdgpu_buffer_rsrc_t vbuf = buffer_rsrc(Z.down, (size_t)Z.rank * K * 2);
  u4 vz[ZI];
#pragma unroll
  for (int i = 0; i < ZI; ++i) {
    const int blk = li + TPR * i;
    const int off = live && blk < blocks ? ((r0 + rr) * K + blk * 8) * 2 : kOutOfRange;
    vz[i] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(vbuf, off, 0, 0));
  }
  __builtin_amdgcn_sched_barrier(0);
  const float inv = prologue_inv(p, xv, wsum, lane, wave);
#pragma unroll
  for (int i = 0; i < XB; ++i) {
    const int blk = t + 256 * i;
    if (blk < blocks) *reinterpret_cast<h8 *>(xs + blk * 8) = prologue_apply(p, xv[i], av[i], inv);
  }
  __syncthreads();
  float acc = 0.0f, acc2 = 0.0f;
#pragma unroll
  for (int i = 0; i < ZI; ++i) {
    const int blk = li + TPR * i;
    if (blk < blocks) {
      asm volatile("" : "+v"(vz[i]));
      const h8 vv = __builtin_bit_cast(h8, vz[i]);
      const h8 xx = *reinterpret_cast<const h8 *>(xs + blk * 8);
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        acc += (float)xx[e] * (float)vv[e];
        acc2 += (float)xx[e + 1] * (float)vv[e + 1];
      }
    }
  }
  acc += acc2;
#pragma unroll
  for (int off = TPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (li == 0 && rr < kFusedZRanks) zsh[rr] = live ? (f16)acc : (f16)0.0f;
  __syncthreads();
  if (t < 2) {
    const uint64_t word = (uint64_t)shared_z_tag(p, passed) | ((uint64_t)__builtin_bit_cast(uint16_t, zsh[3 * t]) << 16) |
                          ((uint64_t)__builtin_bit_cast(uint16_t, zsh[3 * t + 1]) << 32) |
                          ((uint64_t)__builtin_bit_cast(uint16_t, zsh[3 * t + 2]) << 48);
    __hip_atomic_store(p.zslot + zp * 12 + 2 * zi + t, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

// Tile workgroups of a shared-z launch, wave 0: read the problem's z words (lane w < words holds
// word w) with system-scope 64-bit atomic loads until every tag is the launch's (bounded), unpack
// them to zs[rank] (fp16 values as floats, visible to the whole wave on return), then count the
// workgroup on `passed`.
__device__ __forceinline__ void wait_shared_z(const FusedParams &p, int pi, int rank, uint64_t passed, int lane,
                                              float *zs) {
  const uint32_t tag = shared_z_tag(p, passed);
  const int words = (rank + 2) / 3;
  const uint64_t *slot = p.zslot + pi * 12;
  uint64_t word = 0;
  bool ready = false;
  for (int it = 0; it < kFusedZSpinLimit; ++it) {
    if (lane < words) word = __hip_atomic_load(slot + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    ready = __builtin_amdgcn_ballot_w64(lane < words && (uint32_t)(word & 0xFFFF) != tag) == 0;
    if (ready) break;
    __builtin_amdgcn_s_sleep(1);
  }
  if (lane < kFusedZWordsPerProblem) {  // every zs entry, zero from rank on
#pragma unroll
    for (int e = 0; e < 3; ++e)
      if (3 * lane + e < kFusedMaxRank)
        zs[3 * lane + e] =
            3 * lane + e < rank ? (float)__builtin_bit_cast(f16, (uint16_t)(word >> (16 * (e + 1)))) : 0.0f;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // the LDS writes above precede the wave's reads
  __builtin_amdgcn_wave_barrier();
  if (lane == 0) {
    if (!ready)
      __hip_atomic_store(reinterpret_cast<uint32_t *>(p.zslot) + kFusedZTimeoutOffset / 4, 1u, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_fetch_add(p.zslot + kFusedZPassedOffset / 8, (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

// One workgroup = 4 waves = one 16-row tile of one problem; the waves split K (wave w takes
// k-steps w, w + 4, ...) and are reduced through LDS.  K <= KMAX, so every lane issues all
// of its weight loads (D of them) up front and the activation row is staged once.  Every row
// of the MFMA A operand is the activation row (only row 0 of the result is used), so no zero
// rows are staged.
//
// Every global load is issued, straight-line, before the first wait: the epilogue operands
// (one load per wave), the prologue row, the activation, the scales, V (RANKED only) and the
// weights.  Lanes without data read out of range (zeros).  There are no branches around loads:
// a load under a branch makes the compiler wait for it at the branch's end.
template <int FMT, bool SCALED, int KMAX, bool RANKED, bool SHARED_Z = false>
__global__ __launch_bounds__(256) void fused_gemv_kernel(FusedParams p) {
  constexpr int CPL = FormatTraits<FMT>::CPL;
  constexpr int BITS = FormatTraits<FMT>::BITS;
  constexpr int KSTEP = 4 * CPL;
  constexpr int KG = 4;
  constexpr int WSTEP = KG * KSTEP;
  constexpr int D = (KMAX + WSTEP - 1) / WSTEP;  // weight loads per lane
  static_assert(D <= 32, "KMAX too long for this format");
  constexpr int T8 = CPL / 8;
  constexpr int XLD = KMAX + KSTEP + 8;           // staged row, zero from K to K + KSTEP
  constexpr int XB = (KMAX / 8 + 255) / 256;      // 16-byte activation loads per thread
  constexpr bool OWN_Z = RANKED && !SHARED_Z;     // every workgroup computes z itself
  static_assert(!SHARED_Z || RANKED, "shared z is for ranked launches");
  constexpr int VB = OWN_Z ? KMAX / 64 : 0;       // 16-byte V loads per thread (8 threads per rank row)
  constexpr int GMAX = KMAX / FusedGroupMin<KMAX>::value;  // groups per row at most
  constexpr int SC = SCALED ? (16 * GMAX + 255) / 256 : 0; // staged scales per thread
  constexpr int kOutOfRange = (int)0x80000000u;
  static_assert(!RANKED || KMAX <= kFusedMaxK, "the correction is staged for K <= kFusedMaxK");
  __shared__ __align__(16) f16 xs[XLD];
  __shared__ __align__(16) f16 ss[SCALED ? 16 * GMAX + 8 : 8];
  __shared__ __align__(16) f16 us[RANKED ? 16 * kFusedMaxRank : 8];  // U rows of the tile
  __shared__ f16 es[3 * 16];                      // residual, bias, per-row scale of the tile
  __shared__ __align__(16) float zs[kFusedMaxRank];
  __shared__ float red[(KG - 1) * 16];
  __shared__ float wsum[4];
  __shared__ uint32_t nf4_table[FMT == FMT_NF4 ? 256 : 1];

  if constexpr (SHARED_Z) {
    if ((int)blockIdx.x < p.zblocks) {
      fused_z_block<KMAX>(p, xs, wsum, es);
      return;
    }
  }
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int j = lane & 15, g = lane >> 4;
  const int K = p.K;

  // Problem and tile of this workgroup (wave-uniform selects; no dynamic kernarg indexing).
  const int bid = (int)blockIdx.x - (SHARED_Z ? p.zblocks : 0);
  const int pi = bid < p.prob[0].tiles_end ? 0 : (bid < p.prob[1].tiles_end ? 1 : 2);
  const FusedProblem P = problem_of(p, pi);
  int first = 0;
  if (pi == 1) first = p.prob[0].tiles_end;
  if (pi == 2) first = p.prob[1].tiles_end;
  const int n0 = (bid - first) * 16;
  const int rows = min(16, P.N - n0);
  const int row_bytes = K * BITS / 8;
  const int rank = RANKED ? P.rank : 0;
  uint64_t zpassed = 0;
  if constexpr (SHARED_Z) zpassed = shared_z_passed(p);  // issued with the loads below, used at the epilogue

  // Epilogue operands: wave 0 fetches the residual, wave 1 the bias, wave 2 the per-row
  // scale of the tile's 16 rows (lanes 0..15); absent operands have an empty buffer.
  const f16 *ep = wave == 0 ? P.residual : (wave == 1 ? P.bias : (wave == 2 ? P.scales : nullptr));
  const bool ep_on = wave == 0 ? P.residual != nullptr : (wave == 1 ? P.bias != nullptr : (wave == 2 && p.per_row));
  const f16 ev = __builtin_bit_cast(
      f16, __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(ep, ep_on ? (size_t)P.N * 2 : 0),
                                                lane < rows ? (n0 + lane) * 2 : kOutOfRange, 0, 0));
  // U rows of the tile: wave w, lane l < 16 fetches row 4w + l / 4, halves 8 (l % 4) .. + 7.
  u4 ureg = {0u, 0u, 0u, 0u};
  if constexpr (RANKED) {
    const int ur = 4 * wave + (lane >> 2), uq = lane & 3;
    const int off = lane < 16 && ur < rows && uq * 8 < rank ? ((n0 + ur) * P.up_ld + uq * 8) * 2 : kOutOfRange;
    ureg = __builtin_bit_cast(
        u4, __builtin_amdgcn_raw_buffer_load_b128(buffer_rsrc(P.up, rank > 0 ? (size_t)P.N * P.up_ld * 2 : 0), off, 0, 0));
  }
  // Activation row (and the second row of the prologue: gamma or the up row).
  const int blocks = K >> 3;
  const size_t kb = (size_t)K * 2;
  const f16 *aux = p.prologue == PRO_SILU_MUL ? p.x2 : p.gamma;
  const __amdgpu_buffer_rsrc_t abuf = buffer_rsrc(aux, p.prologue == PRO_NONE ? 0 : kb);
  const __amdgpu_buffer_rsrc_t xbuf = buffer_rsrc(p.x, kb);
  h8 av[XB], xv[XB];
#pragma unroll
  for (int i = 0; i < XB; ++i) {
    const int b = t + 256 * i;
    av[i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(abuf, b < blocks ? b * 16 : kOutOfRange, 0, 0));
  }
#pragma unroll
  for (int i = 0; i < XB; ++i) {
    const int b = t + 256 * i;
    xv[i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(xbuf, b < blocks ? b * 16 : kOutOfRange, 0, 0));
  }
  f16 sreg[SC > 0 ? SC : 1];
  if constexpr (SCALED) {
    const __amdgpu_buffer_rsrc_t sbuf = buffer_rsrc(P.scales + (size_t)n0 * p.G, (size_t)rows * p.G * 2);
#pragma unroll
    for (int i = 0; i < SC; ++i)
      sreg[i] = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(sbuf, (t + i * 256) * 2, 0, 0));
  }
  const int vr = t >> 3, vpart = t & 7;
  u4 vreg[VB > 0 ? VB : 1];
  if constexpr (OWN_Z) {
    const __amdgpu_buffer_rsrc_t vbuf = buffer_rsrc(P.down, (size_t)rank * K * 2);
#pragma unroll
    for (int i = 0; i < VB; ++i) {
      const int k = (vpart + 8 * i) * 8;
      const int off = (vr < rank && k < K) ? (vr * K + k) * 2 : kOutOfRange;
      vreg[i] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(vbuf, off, 0, 0));
    }
  }
  const __amdgpu_buffer_rsrc_t wbuf = buffer_rsrc(P.codes + (size_t)n0 * row_bytes, (size_t)rows * row_bytes);
  u4 w[D];
#pragma unroll
  for (int u = 0; u < D; ++u) {
    const int k = (wave + KG * u) * KSTEP + g * CPL;
    const int off = k < K ? j * row_bytes + k * BITS / 8 : kOutOfRange;
    w[u] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(wbuf, off, 0, 0));
  }
  __builtin_amdgcn_sched_barrier(0);  // no use of the loaded data is scheduled above this point

  // ---- prologue: stage the activation row (fp16, in the format's slot order) ----
  if constexpr (FMT == FMT_NF4) build_nf4_pair_table(nf4_table);
  if (lane < 16 && wave < 3) es[wave * 16 + lane] = ev;
  if constexpr (RANKED) {
    if (lane < 16) stage_u_piece(us + (4 * wave + (lane >> 2)) * kFusedMaxRank + (lane & 3) * 8, ureg, lane & 3, rank);
  }
  const float inv = prologue_inv(p, xv, wsum, lane, wave);
#pragma unroll
  for (int i = 0; i < XB; ++i) {
    const int b = t + 256 * i;
    if (b < blocks) *reinterpret_cast<h8 *>(xs + b * 8) = permute_block<FMT>(prologue_apply(p, xv[i], av[i], inv));
  }
  // Zeros past K: MFMA lanes read up to KSTEP beyond it, the own z product up to KMAX.
  const int zero_end = OWN_Z ? XLD : min(XLD, K + KSTEP + 8);
  for (int b = blocks + t; b * 8 < zero_end; b += 256) *reinterpret_cast<h8 *>(xs + b * 8) = h8{};
  if constexpr (SCALED) {
#pragma unroll
    for (int i = 0; i < SC; ++i)
      if (t + i * 256 < 16 * GMAX) ss[t + i * 256] = sreg[i];
    if (t < 8) ss[16 * GMAX + t] = (f16)0.0f;  // lanes past K of the last row index up to 4 beyond
  }
  __syncthreads();

  // ---- correction activations z = fp16(x . V^T), 8 threads per rank row ----
  if constexpr (OWN_Z) {  // v_dot2 chains, then the 8 threads' sums by DPP
    float za = 0.0f, zb = 0.0f;
#pragma unroll
    for (int i = 0; i < VB; ++i) {
      asm volatile("" : "+v"(vreg[i]));  // V is consumed here, after the barrier, not at its load
      const h8 vv = permute_block<FMT>(__builtin_bit_cast(h8, vreg[i]));
      const h8 xx = *reinterpret_cast<const h8 *>(xs + (vpart + 8 * i) * 8);
      za = dot2(pair_of(xx, 0), pair_of(vv, 0), dot2(pair_of(xx, 2), pair_of(vv, 2), za));
      zb = dot2(pair_of(xx, 1), pair_of(vv, 1), dot2(pair_of(xx, 3), pair_of(vv, 3), zb));
    }
    za = sum8(za + zb);
    if (vpart == 0) zs[vr] = (float)(f16)za;
  }

  // ---- the product on MFMA: every A row is the activation row, B = decoded weights ----
  f4 acc = {0.f, 0.f, 0.f, 0.f};
  const f16 *a0 = xs + g * CPL;
#pragma unroll
  for (int u = 0; u < D; ++u) {
    const int kb = (wave + KG * u) * KSTEP;
    if (kb >= K) break;  // wave-uniform
    asm volatile("" : "+v"(w[u]));  // decode here, not at the load
    h2 s2 = {(f16)1.0f, (f16)1.0f};
    if constexpr (SCALED) {
      const f16 sc = ss[j * p.G + ((kb + g * CPL) >> p.group_shift)];
      s2 = h2{sc, sc};
    }
#pragma unroll
    for (int q = 0; q < T8; ++q) {
      const h8 a = *reinterpret_cast<const h8 *>(a0 + kb + 8 * q);
      const h8 b = decode8<FMT, !SCALED>(w[u], q, s2, nf4_table);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc, 0, 0, 0);
    }
  }
  // Lane (j, g) holds D rows 4g..4g+3 of column j; all rows are equal, row 0 (g == 0) is used.
  if (wave > 0 && g == 0) red[(wave - 1) * 16 + j] = acc[0];
  __syncthreads();
  if constexpr (SHARED_Z) {
    if (wave != 0) return;
    wait_shared_z(p, pi, rank, zpassed, lane, zs);
  }
  const bool writer = wave == 0 && g == 0 && j < rows;
  if (!writer) return;
  float sum = ((acc[0] + red[j]) + red[16 + j]) + red[32 + j];

  // ---- epilogue (reference torch_npu_lowbit.py:262-266, torch_npu_smollm.py:160-163) ----
  if (p.per_row) sum *= (float)es[32 + j];
  f16 h = (f16)sum;
  if (P.bias) h = (f16)((float)h + (float)es[16 + j]);
  if (RANKED && rank > 0) {
    const float d = correction_dot(zs, us + j * kFusedMaxRank, rank);
    h = (f16)((float)h + (float)(f16)d);
  }
  if (P.residual) h = (f16)((float)es[j] + (float)h);
  P.y[n0 + j] = h;
}

// Greedy token folded into the head GEMV (lb_head_next).  A logit v of row n becomes the 64-bit
// key (order(v) << 32) | (2^32 - 1 - n), so the largest key is the largest value at its first row
// (torch.argmax order; -0 ranks with +0); NaN and -inf take key 0, which every other key beats, and
// a result of 0 means token 0, as in argmax_next_kernel.  The workgroups form groups of
// kHeadNextGroup: each raises its group's maximum word to its own largest key, then counts itself
// on the group's counter; the workgroup that completes a group takes the group's maximum (leaving
// 0), raises the total's maximum word and counts itself on the top counter; the one that completes
// that takes the total and writes the token, the position and the next embedding.  Every step is a
// returning system-scope atomic (performed at the memory side, past the per-XCD L2s) issued only
// after the previous one has returned, so a workgroup that sees a counter complete sees every
// maximum raised before it; no workgroup waits for another and no cache is written back or
// invalidated.  Maximum words and counters are set back to zero by the workgroup that completes
// them, so a zeroed workspace is zero again after every call.
#ifndef LB_HEAD_NEXT_GROUP
#define LB_HEAD_NEXT_GROUP 16  // workgroups per first-level group (48 groups for the 49152-row head)
#endif
// LB_HEAD_NEXT_WORKSPACE_BYTES counts groups of 8: larger groups use fewer of its words.
constexpr int kHeadNextGroup = LB_HEAD_NEXT_GROUP;
static_assert(kHeadNextGroup >= 8, "the workspace holds the words of groups of 8");
struct HeadNextParams {
  uint64_t *ws;              // maximum words [groups + 1] (the last one the total's), counters [groups + 1]
  const f16 *embedding;      // [vocab, hidden]
  f16 *h_next;               // [hidden]
  int64_t *tokens, *token, *position;
  int limit, hidden, groups, vocab;
};

__device__ __forceinline__ uint64_t logit_key(float v, int n) {
  if (!(v > -INFINITY)) return 0;
  uint32_t b = __builtin_bit_cast(uint32_t, v);
  if (b == 0x80000000u) b = 0u;
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)b << 32) | (0xFFFFFFFFu - (uint32_t)n);
}

// Lane 0: raise *max_word to key, then count on *counter; returns the counter's previous value.
__device__ __forceinline__ uint64_t head_next_arrive(uint64_t *max_word, uint64_t *counter, uint64_t key) {
  const uint64_t prev = __hip_atomic_fetch_max(max_word, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  asm volatile("" : : "v"(prev) : "memory");  // the maximum has returned before the count is issued
  return __hip_atomic_fetch_add(counter, (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Wave 0 of workgroup `wg` of `wgs`, with the workgroup's largest key `best` (wave-uniform).
__device__ __forceinline__ void head_next_tail(const HeadNextParams &hn, uint64_t best, int lane, int wg, int wgs) {
  uint64_t *maxima = hn.ws, *counters = hn.ws + hn.groups + 1;
  const int grp = wg / kHeadNextGroup;
  const int members = min(kHeadNextGroup, wgs - grp * kHeadNextGroup);
  uint64_t seen = 0, v = 0;
  if (lane == 0) seen = head_next_arrive(maxima + grp, counters + grp, best);
  if ((uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)seen) != (uint32_t)(members - 1)) return;
  if (lane == 0) {
    v = __hip_atomic_exchange(maxima + grp, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(counters + grp, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
  if (hn.groups > 1) {  // a single group's maximum is already the total
    if (lane == 0) seen = head_next_arrive(maxima + hn.groups, counters + hn.groups, v);
    if ((uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)seen) != (uint32_t)(hn.groups - 1)) return;
    if (lane == 0) {
      v = __hip_atomic_exchange(maxima + hn.groups, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      __hip_atomic_store(counters + hn.groups, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
  v = lane_value64(v, 0);
  // A key names a row below vocab; the bound only matters for a workspace that was not zeroed.
  const uint32_t row = 0xFFFFFFFFu - (uint32_t)v;
  const int t = (v == 0 || row >= (uint32_t)hn.vocab) ? 0 : (int)row;
  if (lane == 0) {
    const int64_t pos = hn.position[0];
    if (pos >= 0 && pos < hn.limit) {
      hn.tokens[pos] = t;
      hn.position[0] = pos + 1;
    }
    hn.token[0] = t;
  }
  for (int b = lane; b * 8 < hn.hidden; b += 64)
    *reinterpret_cast<h8 *>(hn.h_next + b * 8) =
        *reinterpret_cast<const h8 *>(hn.embedding + (size_t)t * hn.hidden + b * 8);
}

// One activation row, one problem, no correction, many rows (the long-N one-row linears: a tied
// head, the Llama-shaped projections).  A workgroup holds RG 16-row tiles; wave (rg, kg) computes
// tile rg over the k-steps kg, kg + KG, ... with KG = 4 / RG, so the staged activation row serves
// RG tiles, and with RG = 4 every wave covers all of K and no cross-wave reduction is needed.
// As in fused_gemv_kernel, every global load is issued straight-line before the first wait.  The
// operands of those first loads come as leading scalar arguments, which the build preloads into
// registers at wave launch (-amdgpu-kernarg-preload-count): workgroups dispatched while earlier ones
// flood the memory system with weight requests would otherwise wait microseconds for their
// argument block before issuing a single load.  The epilogue operands (residual, bias, per-row
// scale) are loaded after the weights and staged behind a second barrier.  With NEXT the
// workgroups also pick the greedy token of the row they compute (head_next_tail above).
template <int FMT, bool SCALED, int KMAX, int RG, bool NEXT>
__global__ __launch_bounds__(256) void rows_gemv_kernel(const uint8_t *pre_codes, const f16 *pre_x, const f16 *pre_scales,
                                                        const f16 *pre_aux, int pre_N, int pre_K, int pre_G,
                                                        int pre_prologue, int pre_shift, FusedParams p,
                                                        HeadNextParams hn) {
  constexpr int CPL = FormatTraits<FMT>::CPL;
  constexpr int BITS = FormatTraits<FMT>::BITS;
  constexpr int KSTEP = 4 * CPL;
  constexpr int KG = 4 / RG;
  constexpr int WSTEP = KG * KSTEP;
  constexpr int D = (KMAX + WSTEP - 1) / WSTEP;  // weight loads per lane
  static_assert(D <= 32, "KMAX too long for this tile split");
  constexpr int T8 = CPL / 8;
  constexpr int ROWS = 16 * RG;                   // rows per workgroup
  constexpr int XLD = KMAX + KSTEP + 8;
  constexpr int XB = (KMAX / 8 + 255) / 256;
  constexpr int GMAX = KMAX / FusedGroupMin<KMAX>::value;
  constexpr int SC = SCALED ? (ROWS * GMAX + 255) / 256 : 0;
  constexpr int kOutOfRange = (int)0x80000000u;
  __shared__ __align__(16) f16 xs[XLD];
  __shared__ __align__(16) f16 ss[SCALED ? ROWS * GMAX + 8 : 8];
  __shared__ f16 es[3 * ROWS];                    // residual, bias, per-row scale of the rows
  __shared__ float red[KG > 1 ? (KG - 1) * ROWS : 1];
  __shared__ float wsum[4];
  __shared__ uint32_t nf4_table[FMT == FMT_NF4 ? 256 : 1];
  __shared__ uint64_t wkey[NEXT ? 4 : 1];
  static_assert(!NEXT || RG == 4, "the greedy tail needs every wave to own a whole tile");

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int rg = wave % RG, kg = wave / RG;
  const int j = lane & 15, g = lane >> 4;
  const int K = pre_K;
  const FusedProblem &P = p.prob[0];
  const int w0 = blockIdx.x * ROWS;               // first row of the workgroup
  const int wrows = min(ROWS, pre_N - w0);
  const int n0 = w0 + 16 * rg;                    // first row of this wave's tile
  const int rows = min(16, pre_N - n0);           // <= 0: the tile lies past N (no loads, no stores)
  const int row_bytes = K * BITS / 8;

  // Epilogue operands: wave 0 fetches the residual, wave 1 the bias, wave 2 the per-row scale
  // of the workgroup's rows (lane r < ROWS reads row w0 + r).
  const int blocks = K >> 3;
  const size_t kb_bytes = (size_t)K * 2;
  const __amdgpu_buffer_rsrc_t abuf = buffer_rsrc(pre_aux, pre_prologue == PRO_NONE ? 0 : kb_bytes);
  const __amdgpu_buffer_rsrc_t xbuf = buffer_rsrc(pre_x, kb_bytes);
  h8 av[XB], xv[XB];
#pragma unroll
  for (int i = 0; i < XB; ++i) {
    const int b = t + 256 * i;
    av[i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(abuf, b < blocks ? b * 16 : kOutOfRange, 0, 0));
  }
#pragma unroll
  for (int i = 0; i < XB; ++i) {
    const int b = t + 256 * i;
    xv[i] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(xbuf, b < blocks ? b * 16 : kOutOfRange, 0, 0));
  }
  f16 sreg[SC > 0 ? SC : 1];
  if constexpr (SCALED) {
    const __amdgpu_buffer_rsrc_t sbuf = buffer_rsrc(pre_scales + (size_t)w0 * pre_G, (size_t)max(wrows, 0) * pre_G * 2);
#pragma unroll
    for (int i = 0; i < SC; ++i)
      sreg[i] = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(sbuf, (t + i * 256) * 2, 0, 0));
  }
  const __amdgpu_buffer_rsrc_t wbuf =
      buffer_rsrc(pre_codes + (size_t)max(n0, 0) * row_bytes, rows > 0 ? (size_t)rows * row_bytes : 0);
  u4 w[D];
#pragma unroll
  for (int u = 0; u < D; ++u) {
    const int k = (kg + KG * u) * KSTEP + g * CPL;
    const int off = k < K ? j * row_bytes + k * BITS / 8 : kOutOfRange;
    w[u] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(wbuf, off, 0, 0));
  }
  const f16 *ep = wave == 0 ? P.residual : (wave == 1 ? P.bias : (wave == 2 ? P.scales : nullptr));
  const bool ep_on = wave == 0 ? P.residual != nullptr : (wave == 1 ? P.bias != nullptr : (wave == 2 && p.per_row));
  const f16 ev = __builtin_bit_cast(
      f16, __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(ep, ep_on ? (size_t)pre_N * 2 : 0),
                                                lane < wrows ? (w0 + lane) * 2 : kOutOfRange, 0, 0));
  __builtin_amdgcn_sched_barrier(0);  // no use of the loaded data is scheduled above this point

  if constexpr (FMT == FMT_NF4) build_nf4_pair_table(nf4_table);
  const float inv = prologue_inv(p, xv, wsum, lane, wave);
#pragma unroll
  for (int i = 0; i < XB; ++i) {
    const int b = t + 256 * i;
    if (b < blocks) *reinterpret_cast<h8 *>(xs + b * 8) = permute_block<FMT>(prologue_apply(p, xv[i], av[i], inv));
  }
  for (int b = blocks + t; b * 8 < min(XLD, K + KSTEP + 8); b += 256) *reinterpret_cast<h8 *>(xs + b * 8) = h8{};
  if constexpr (SCALED) {
#pragma unroll
    for (int i = 0; i < SC; ++i)
      if (t + i * 256 < ROWS * GMAX) ss[t + i * 256] = sreg[i];
    if (t < 8) ss[ROWS * GMAX + t] = (f16)0.0f;  // lanes past K of the last row index up to 4 beyond
  }
  __syncthreads();

  f4 acc = {0.f, 0.f, 0.f, 0.f};
  const f16 *a0 = xs + g * CPL;
#pragma unroll
  for (int u = 0; u < D; ++u) {
    const int kb = (kg + KG * u) * KSTEP;
    if (kb >= K) break;  // wave-uniform
    asm volatile("" : "+v"(w[u]));  // decode here, not at the load
    h2 s2 = {(f16)1.0f, (f16)1.0f};
    if constexpr (SCALED) {
      const f16 sc = ss[(rg * 16 + j) * pre_G + ((kb + g * CPL) >> pre_shift)];
      s2 = h2{sc, sc};
    }
#pragma unroll
    for (int q = 0; q < T8; ++q) {
      const h8 a = *reinterpret_cast<const h8 *>(a0 + kb + 8 * q);
      const h8 b = decode8<FMT, !SCALED>(w[u], q, s2, nf4_table);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc, 0, 0, 0);
    }
  }
  // Lane (j, g) holds D rows 4g..4g+3 of column j; all rows are equal, row 0 (g == 0) is used.
  if (wave < 3 && lane < ROWS) es[wave * ROWS + lane] = ev;
  __syncthreads();  // the epilogue operands, loaded after the weights
  float sum = acc[0];
  if constexpr (KG > 1) {
    if (kg > 0 && g == 0) red[(kg - 1) * ROWS + rg * 16 + j] = acc[0];
    __syncthreads();
    if (kg > 0) return;
#pragma unroll
    for (int q = 0; q < KG - 1; ++q) sum += red[q * ROWS + rg * 16 + j];
  }
  // ---- epilogue (reference torch_npu_lowbit.py:262-266, torch_npu_smollm.py:160-163) ----
  auto finish = [&]() {
    const int r = rg * 16 + j;
    if (p.per_row) sum *= (float)es[2 * ROWS + r];
    f16 h = (f16)sum;
    if (P.bias) h = (f16)((float)h + (float)es[ROWS + r]);
    if (P.residual) h = (f16)((float)es[r] + (float)h);
    P.y[n0 + j] = h;
    return h;
  };
  if constexpr (NEXT) {
    // Lanes 0..15 hold the tile's rows: the wave's largest key, then the workgroup's.
    const uint64_t key = (g == 0 && j < rows) ? logit_key((float)finish(), n0 + j) : 0;
    const uint64_t tile_best = row_max64(key);  // every lane active: the DPP moves read lanes 0..15
    if (lane == 0) wkey[wave] = tile_best;
    __syncthreads();
    if (wave != 0) return;
    head_next_tail(hn, max64(max64(wkey[0], wkey[1]), max64(wkey[2], wkey[3])), lane, (int)blockIdx.x,
                   (int)gridDim.x);
  } else {
    if (g != 0 || j >= rows) return;
    finish();
  }
}

struct AttnParams {
  const f16 *q, *k, *v;      // new rows: q [heads, 64], k and v [kv_heads, 64]
  const f16 *cos, *sin;      // [capacity, 64]
  const int64_t *position;   // device scalar: the slot of the new token
  f16 *keys, *values;        // [kv_heads, capacity, 64]
  f16 *out;                  // [heads, 64]
  int heads, kv_heads, capacity;
  float scale;
  // Split form (split_attention_kernel): tagged score words [heads][chunks * 16], then `passed`
  // (u64) and a timeout word; score workgroups first.
  uint64_t *words;
  int chunks;                // position chunks of kAttnChunk per KV head
  int score_wgs;             // kv_heads * chunks
};

constexpr int kHeadDim = 64;
#ifndef LB_ATTN_SLICES
#define LB_ATTN_SLICES 4
#endif
constexpr int kAttnDimSlices = LB_ATTN_SLICES;          // workgroups per query head (grid y)
constexpr int kSliceDims = kHeadDim / kAttnDimSlices;   // output dims per workgroup
constexpr int kSliceBlocks = kSliceDims / 8;            // 16-byte V blocks per slot and workgroup
constexpr int kAttnParts = 256 / kSliceBlocks;          // position partitions of the P.V product
constexpr int kPvPartials = 16;  // P.V partial sums per output dim: one per row of 16 lanes of each wave

// P.V: lane l of a wave holds o[8], the partial products of V block l % kSliceBlocks over its
// positions.  The lanes of one block within each row of 16 are summed on DPP (distance 2 within
// quads, then rotations by 4 and 8), and each row's sums go to pv[(4 wave + row) * kSliceDims + d].
__device__ __forceinline__ void pv_row_partials(float (&o)[8], float *pv, int lane, int wave);
// The output dim d: the 16 row partials added in a fixed order.
__device__ __forceinline__ float pv_total(const float *pv, int d);

constexpr int kScoreSlots = 2;   // K rows per thread per round: 512 slots per round
constexpr int kValueSlots = (384 + kAttnParts - 1) / kAttnParts;  // V blocks per thread per round (>= 384 slots)

__device__ __forceinline__ void pv_row_partials(float (&o)[8], float *pv, int lane, int wave) {
  static_assert(kSliceBlocks == 2, "the DPP steps pair lanes of equal parity");
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    o[e] += dpp_move<kDppXor2>(o[e]);
    o[e] += dpp_move<kDppRowRor4>(o[e]);
    o[e] += dpp_move<kDppRowRor8>(o[e]);
  }
  const int r = lane & 15;
  if (r < kSliceBlocks) {
#pragma unroll
    for (int e = 0; e < 8; ++e) pv[(wave * 4 + (lane >> 4)) * kSliceDims + r * 8 + e] = o[e];
  }
}

__device__ __forceinline__ float pv_total(const float *pv, int d) {
  float r = pv[d];
#pragma unroll
  for (int q = 1; q < kPvPartials; ++q) r += pv[q * kSliceDims + d];
  return r;
}
static_assert(kSliceBlocks >= 1 && kHeadDim % kAttnDimSlices == 0, "attention slices");

// kAttnDimSlices workgroups per query head, each owning kSliceDims of the output dims.  Every
// workgroup of a head computes the same scores and softmax (same data, same order, so the same
// probabilities bit for bit) and P.V for its own dims only, so it reads all cached K rows but a
// quarter of each V row, and no partial result crosses workgroups.  The first slice of the first
// query head of each KV group writes the rotated key and the value into the cache; every
// workgroup uses its own copy of that new row, so no workgroup reads a cache slot another one
// writes.  The cached K and V rows of the first round (slots < 512 and < 384) are loaded before
// anything else, so a step costs one memory round trip plus the on-chip softmax; longer caches
// loop over further rounds.
__global__ __launch_bounds__(256) void decode_attention_kernel(AttnParams p) {
  extern __shared__ float sc[];  // [capacity] scores, then probabilities
  __shared__ __align__(16) f16 qs[kHeadDim], kn[kHeadDim], vn[kHeadDim];
  __shared__ float wred[4];
  __shared__ float pv[4 * kSliceDims];
  constexpr int kOutOfRange = (int)0x80000000u;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);  // scalar: buffer bases below are per wave
  const int h = blockIdx.x;
  const int d0 = (int)blockIdx.y * kSliceDims;  // first output dim of this workgroup
  const int group = p.heads / p.kv_heads;
  const int kvh = h / group;
  const int pos = (int)p.position[0];
  if (pos < 0 || pos >= p.capacity) {
    // No slot for the new row: nothing is read from or written to the cache, and the
    // workgroup's output dims are NaN, so a caller past the capacity sees it in the result.
    if (t < kSliceDims) p.out[h * kHeadDim + d0 + t] = (f16)__builtin_nanf("");
    return;
  }

  // The new rows first: wave 0 reads the query row of head h, wave 1 the key row and wave 2
  // the value row of its KV head (element d and its rotate-half partner d ^ 32), waves 0 and 1
  // the RoPE row pos.
  const int d = lane;
  const f16 *src = wave == 0 ? p.q + h * kHeadDim : (wave == 1 ? p.k : p.v) + kvh * kHeadDim;
  const __amdgpu_buffer_rsrc_t rbuf = buffer_rsrc(src, wave < 3 ? kHeadDim * 2 : 0);
  const __amdgpu_buffer_rsrc_t cbuf = buffer_rsrc(p.cos + (size_t)pos * kHeadDim, wave < 2 ? kHeadDim * 2 : 0);
  const __amdgpu_buffer_rsrc_t snbuf = buffer_rsrc(p.sin + (size_t)pos * kHeadDim, wave < 2 ? kHeadDim * 2 : 0);
  const f16 x0 = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(rbuf, d * 2, 0, 0));
  const f16 x1 = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(rbuf, (d ^ 32) * 2, 0, 0));
  const f16 cv = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(cbuf, d * 2, 0, 0));
  const f16 sv = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(snbuf, d * 2, 0, 0));

  // Cached rows live in slots [0, pos); the buffers end there, so later slots read zero.
  const size_t head_base = (size_t)kvh * p.capacity * kHeadDim;
  const __amdgpu_buffer_rsrc_t kbuf = buffer_rsrc(p.keys + head_base, (size_t)pos * kHeadDim * 2);
  const __amdgpu_buffer_rsrc_t vbuf = buffer_rsrc(p.values + head_base, (size_t)pos * kHeadDim * 2);
  const int blk = t % kSliceBlocks, part = t / kSliceBlocks;
  u4 kreg[kScoreSlots][kHeadDim / 8];
  u4 vreg[kValueSlots];
  // Straight-line loads (a load under a branch is waited for at the branch's end); lanes
  // past the cached slots read out of range (zeros, no memory traffic).
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
  __builtin_amdgcn_sched_barrier(0);

  // RoPE of q and k at row pos (three fp16 roundings); v as given.
  if (wave == 2) {
    vn[d] = x0;
  } else if (wave < 2) {
    const float rot = d < 32 ? -(float)x1 : (float)x1;
    const f16 r = rope_element((float)x0, rot, (float)cv, (float)sv);
    if (wave == 0) qs[d] = r; else kn[d] = r;
  }
  __syncthreads();
  if (h % group == 0 && blockIdx.y == 0 && t < 2 * kHeadDim) {
    const int d = t & 63;
    f16 *dst = (t < kHeadDim ? p.keys : p.values) + head_base + (size_t)pos * kHeadDim + d;
    *dst = t < kHeadDim ? kn[d] : vn[d];
  }

  // scores = fp16(fp16(q . k) * scale) over slots 0..pos
  float lmax = -INFINITY;
  for (int base = 0; base <= pos; base += 256 * kScoreSlots) {
    if (base > 0) load_keys(base);
#pragma unroll
    for (int i = 0; i < kScoreSlots; ++i) {
      const int s = base + t + 256 * i;
      if (base + 256 * i > pos) break;  // wave-uniform
      float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
      for (int b = 0; b < kHeadDim / 8; ++b) {
        asm volatile("" : "+v"(kreg[i][b]));  // consumed here, not at the load
        const h8 qq = *reinterpret_cast<const h8 *>(qs + 8 * b);
        const h8 kk = s == pos ? *reinterpret_cast<const h8 *>(kn + 8 * b) : __builtin_bit_cast(h8, kreg[i][b]);
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          acc0 += (float)qq[e] * (float)kk[e];
          acc1 += (float)qq[e + 1] * (float)kk[e + 1];
        }
      }
      if (s <= pos) {
        const float v = (float)(f16)((float)(f16)(acc0 + acc1) * p.scale);
        sc[s] = v;
        lmax = fmaxf(lmax, v);
      }
    }
  }
  lmax = wave_max(lmax);
  if (lane == 0) wred[wave] = lmax;
  __syncthreads();
  const float m = fmaxf(fmaxf(wred[0], wred[1]), fmaxf(wred[2], wred[3]));
  float lsum = 0.0f;
  for (int s = t; s <= pos; s += 256) {
    const float e = expf(sc[s] - m);
    sc[s] = e;
    lsum += e;
  }
  lsum = wave_sum(lsum);
  __syncthreads();  // every wave has read wred
  if (lane == 0) wred[wave] = lsum;
  __syncthreads();
  const float total = ((wred[0] + wred[1]) + wred[2]) + wred[3];
  for (int s = t; s <= pos; s += 256) sc[s] = (float)(f16)(sc[s] / total);
  __syncthreads();

  // out = fp16(P . V) over this workgroup's dims: thread (blk, part) sums 8 dims over slots part,
  // part + kAttnParts, ...; then the parts of a wave (lane bits above blk) by butterfly, the four
  // waves through LDS, in a fixed order.
  float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int base = 0; base <= pos; base += kAttnParts * kValueSlots) {
    if (base > 0) load_values(base);
#pragma unroll
    for (int i = 0; i < kValueSlots; ++i) {
      const int s = base + part + kAttnParts * i;
      if (base + kAttnParts * i > pos) break;  // wave-uniform
      asm volatile("" : "+v"(vreg[i]));
      const h8 vv = s == pos ? *reinterpret_cast<const h8 *>(vn + d0 + 8 * blk) : __builtin_bit_cast(h8, vreg[i]);
      const float pr = s <= pos ? sc[min(s, pos)] : 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] += pr * (float)vv[e];
    }
  }
#pragma unroll
  for (int off = kSliceBlocks; off < 64; off <<= 1)
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] += __shfl_xor(o[e], off, 64);
  if (lane < kSliceBlocks) {
#pragma unroll
    for (int e = 0; e < 8; ++e) pv[wave * kSliceDims + lane * 8 + e] = o[e];
  }
  __syncthreads();
  if (t < kSliceDims) {
    const float r = ((pv[t] + pv[kSliceDims + t]) + pv[2 * kSliceDims + t]) + pv[3 * kSliceDims + t];
    p.out[h * kHeadDim + d0 + t] = (f16)r;
  }
}

// Split decode attention: the scores and the output in separate workgroups of one launch.
//
// Score workgroups (the first kv_heads * chunks of the grid, so they are dispatched before any
// workgroup that waits for them): KV head kvh, positions [48 c, 48 c + 48) up to the new token's.
// Each applies RoPE to the query rows of the KV group and to the new key, writes the new key and
// value into the cache if its chunk holds the new slot, computes the scores fp16(fp16(q.k) * scale)
// for every query head of the group and publishes them three to a 64-bit word whose low 16 bits
// are the launch's tag (system-scope atomic stores, performed at the memory side).
//
// Output workgroups: query head h, kSliceDims output dims.  Each reads its head's score words with
// system-scope 64-bit atomic loads until every tag is the launch's (bounded), then follows the
// reference staging on the whole row (global max, fp32 sum of exp, probabilities fp16(e / total)),
// and forms fp16(P.V) over its dims from the cached values and the new value row.  The launch tag
// is (passed / output workgroups + 1) mod 2^16, with `passed` raised once per output workgroup
// after its wait, as in the shared-z decode GEMVs.  No workgroup reads a cache slot another writes.
constexpr int kAttnChunk = 48;                          // positions per score workgroup
constexpr int kAttnChunkWords = kAttnChunk / 3;         // score words per head and chunk
constexpr int kAttnMaxGroup = 3;                        // query heads per KV head in the split form
constexpr int kAttnSpinLimit = 1 << 18;

__device__ __forceinline__ uint32_t attn_tag(const AttnParams &p, uint64_t passed) {
  const uint32_t outs = (uint32_t)(p.heads * kAttnDimSlices);
  return (uint32_t)((passed / outs + 1) & 0xFFFF);
}

__device__ __forceinline__ uint64_t *attn_passed(const AttnParams &p) {
  return p.words + (size_t)p.heads * p.chunks * kAttnChunkWords;
}

__device__ __forceinline__ void attention_scores_block(const AttnParams &p, int b) {
  __shared__ __align__(16) f16 qs[kAttnMaxGroup * kHeadDim];
  __shared__ __align__(16) f16 kn[kHeadDim];
  __shared__ float sco[kAttnMaxGroup * kAttnChunk];
  constexpr int kOutOfRange = (int)0x80000000u;
  const int t = threadIdx.x;
  const int group = p.heads / p.kv_heads;
  const int kvh = b / p.chunks, c = b % p.chunks;
  const int c0 = c * kAttnChunk;
  const int pos = (int)p.position[0];
  if (pos < 0 || pos >= p.capacity || c0 > pos) return;  // nothing of this chunk is needed
  const uint64_t passed = __hip_atomic_load(attn_passed(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);

  // New rows: thread t < 64 group reads element d (and its rotate-half partner) of query row
  // kvh * group + t / 64, the next 64 threads the key row; threads 0..63 also the value row.
  const int hh = t >> 6, d = t & 63;
  const bool is_q = hh < group, is_k = hh == group;
  const f16 *src = is_q ? p.q + (size_t)(kvh * group + hh) * kHeadDim : p.k + (size_t)kvh * kHeadDim;
  const __amdgpu_buffer_rsrc_t rbuf = buffer_rsrc(src, is_q || is_k ? kHeadDim * 2 : 0);
  const __amdgpu_buffer_rsrc_t cbuf = buffer_rsrc(p.cos + (size_t)pos * kHeadDim, kHeadDim * 2);
  const __amdgpu_buffer_rsrc_t snbuf = buffer_rsrc(p.sin + (size_t)pos * kHeadDim, kHeadDim * 2);
  const __amdgpu_buffer_rsrc_t vnbuf = buffer_rsrc(p.v + (size_t)kvh * kHeadDim, t < kHeadDim ? kHeadDim * 2 : 0);
  const f16 x0 = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(rbuf, d * 2, 0, 0));
  const f16 x1 = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(rbuf, (d ^ 32) * 2, 0, 0));
  const f16 cv = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(cbuf, d * 2, 0, 0));
  const f16 sv = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(snbuf, d * 2, 0, 0));
  const f16 vnew = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(vnbuf, d * 2, 0, 0));
  // Cached key rows of the chunk (slots below pos): 8 threads per row, 32 rows per pass.
  const size_t head_base = (size_t)kvh * p.capacity * kHeadDim;
  const __amdgpu_buffer_rsrc_t kbuf = buffer_rsrc(p.keys + head_base, (size_t)pos * kHeadDim * 2);
  const int kr = t >> 3, kb = t & 7;
  constexpr int kPasses = (kAttnChunk + 31) / 32;
  u4 kreg[kPasses];
#pragma unroll
  for (int i = 0; i < kPasses; ++i) {
    const int r = kr + 32 * i, s = c0 + r;
    kreg[i] = __builtin_bit_cast(
        u4, __builtin_amdgcn_raw_buffer_load_b128(kbuf, r < kAttnChunk && s < pos ? (s * kHeadDim + 8 * kb) * 2 : kOutOfRange, 0, 0));
  }
  __builtin_amdgcn_sched_barrier(0);

  if (is_q || is_k) {
    const float rot = d < 32 ? -(float)x1 : (float)x1;
    const f16 r = rope_element((float)x0, rot, (float)cv, (float)sv);
    if (is_q) qs[hh * kHeadDim + d] = r; else kn[d] = r;
    if (is_k && pos < c0 + kAttnChunk) p.keys[head_base + (size_t)pos * kHeadDim + d] = r;
  }
  if (t < kHeadDim && pos < c0 + kAttnChunk) p.values[head_base + (size_t)pos * kHeadDim + t] = vnew;
  __syncthreads();

  // Scores: thread (row kr + 32 i, block kb) forms 8-element partial dot products for every query
  // head of the group, summed over the row's 8 threads.
#pragma unroll
  for (int i = 0; i < kPasses; ++i) {
    const int r = kr + 32 * i, s = c0 + r;
    asm volatile("" : "+v"(kreg[i]));
    const h8 kk = s == pos ? *reinterpret_cast<const h8 *>(kn + 8 * kb) : __builtin_bit_cast(h8, kreg[i]);
    for (int q = 0; q < group; ++q) {
      const h8 qq = *reinterpret_cast<const h8 *>(qs + q * kHeadDim + 8 * kb);
      float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        acc0 += (float)qq[e] * (float)kk[e];
        acc1 += (float)qq[e + 1] * (float)kk[e + 1];
      }
      float acc = acc0 + acc1;
      acc += __shfl_xor(acc, 1, 64);
      acc += __shfl_xor(acc, 2, 64);
      acc += __shfl_xor(acc, 4, 64);
      if (kb == 0 && r < kAttnChunk) sco[q * kAttnChunk + r] = (float)(f16)((float)(f16)acc * p.scale);
    }
  }
  __syncthreads();
  if (t < group * kAttnChunkWords) {
    const int q = t / kAttnChunkWords, w = t % kAttnChunkWords;
    uint64_t word = attn_tag(p, passed);
#pragma unroll
    for (int e = 0; e < 3; ++e) {
      const float v = c0 + 3 * w + e <= pos ? sco[q * kAttnChunk + 3 * w + e] : 0.0f;
      word |= (uint64_t)__builtin_bit_cast(uint16_t, (f16)v) << (16 * (e + 1));
    }
    uint64_t *dst = p.words + (size_t)(kvh * group + q) * p.chunks * kAttnChunkWords + c * kAttnChunkWords + w;
    __hip_atomic_store(dst, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

__device__ __forceinline__ void attention_output_block(const AttnParams &p, int idx, float *sc) {
  __shared__ __align__(16) f16 vn[kSliceDims];
  __shared__ float wred[4];
  __shared__ float pv[4 * kSliceDims];
  constexpr int kOutOfRange = (int)0x80000000u;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int h = idx / kAttnDimSlices;
  const int d0 = (idx % kAttnDimSlices) * kSliceDims;
  const int group = p.heads / p.kv_heads;
  const int kvh = h / group;
  const int pos = (int)p.position[0];
  uint64_t *passed_word = attn_passed(p);
  const uint64_t passed = __hip_atomic_load(passed_word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  if (pos < 0 || pos >= p.capacity) {
    if (t < kSliceDims) p.out[h * kHeadDim + d0 + t] = (f16)__builtin_nanf("");
    if (t == 0) __hip_atomic_fetch_add(passed_word, (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    return;
  }
  // Cached value rows of this workgroup's dims (slots below pos) and the new value row.
  const size_t head_base = (size_t)kvh * p.capacity * kHeadDim;
  const __amdgpu_buffer_rsrc_t vbuf = buffer_rsrc(p.values + head_base, (size_t)pos * kHeadDim * 2);
  const int blk = t % kSliceBlocks, part = t / kSliceBlocks;
  u4 vreg[kValueSlots];
  auto load_values = [&](int base) {
#pragma unroll
    for (int i = 0; i < kValueSlots; ++i) {
      const int s = base + part + kAttnParts * i;
      vreg[i] = __builtin_bit_cast(
          u4, __builtin_amdgcn_raw_buffer_load_b128(vbuf, s < pos ? (s * kHeadDim + d0 + 8 * blk) * 2 : kOutOfRange, 0, 0));
    }
  };
  load_values(0);
  const __amdgpu_buffer_rsrc_t vnbuf = buffer_rsrc(p.v + (size_t)kvh * kHeadDim + d0, t < kSliceDims ? kSliceDims * 2 : 0);
  const f16 vnew = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(vnbuf, t * 2, 0, 0));
  __builtin_amdgcn_sched_barrier(0);
  if (t < kSliceDims) vn[t] = vnew;

  // The head's scores: word w holds slots 3 w .. 3 w + 2 (chunk w / 16 of its head).
  const uint32_t tag = attn_tag(p, passed);
  const int words = pos / 3 + 1;
  const uint64_t *hw = p.words + (size_t)h * p.chunks * kAttnChunkWords;
  bool late = false;
  for (int w = t; w < words; w += 256) {
    uint64_t word = 0;
    int it = 0;
    for (; it < kAttnSpinLimit; ++it) {
      word = __hip_atomic_load(hw + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      if ((uint32_t)(word & 0xFFFF) == tag) break;
      __builtin_amdgcn_s_sleep(1);
    }
    late = late || it == kAttnSpinLimit;
#pragma unroll
    for (int e = 0; e < 3; ++e)
      if (3 * w + e <= pos) sc[3 * w + e] = (float)__builtin_bit_cast(f16, (uint16_t)(word >> (16 * (e + 1))));
  }
  if (late)
    __hip_atomic_store(reinterpret_cast<uint32_t *>(passed_word + 1), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  __syncthreads();
  if (t == 0) __hip_atomic_fetch_add(passed_word, (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);

  // Reference staging over slots 0..pos: global max, fp32 sum of exp, probabilities fp16(e / total).
  float lmax = -INFINITY;
  for (int s = t; s <= pos; s += 256) lmax = fmaxf(lmax, sc[s]);
  lmax = wave_max(lmax);
  if (lane == 0) wred[wave] = lmax;
  __syncthreads();
  const float m = fmaxf(fmaxf(wred[0], wred[1]), fmaxf(wred[2], wred[3]));
  float lsum = 0.0f;
  for (int s = t; s <= pos; s += 256) {
    const float e = expf(sc[s] - m);
    sc[s] = e;
    lsum += e;
  }
  lsum = wave_sum(lsum);
  __syncthreads();  // every wave has read wred
  if (lane == 0) wred[wave] = lsum;
  __syncthreads();
  const float total = ((wred[0] + wred[1]) + wred[2]) + wred[3];
  for (int s = t; s <= pos; s += 256) sc[s] = (float)(f16)(sc[s] / total);
  __syncthreads();

  // out = fp16(P . V) over this workgroup's dims, as in decode_attention_kernel.
  float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int base = 0; base <= pos; base += kAttnParts * kValueSlots) {
    if (base > 0) load_values(base);
#pragma unroll
    for (int i = 0; i < kValueSlots; ++i) {
      const int s = base + part + kAttnParts * i;
      if (base + kAttnParts * i > pos) break;  // wave-uniform
      asm volatile("" : "+v"(vreg[i]));
      const h8 vv = s == pos ? *reinterpret_cast<const h8 *>(vn + 8 * blk) : __builtin_bit_cast(h8, vreg[i]);
      const float pr = s <= pos ? sc[min(s, pos)] : 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] += pr * (float)vv[e];
    }
  }
#pragma unroll
  for (int off = kSliceBlocks; off < 64; off <<= 1)
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] += __shfl_xor(o[e], off, 64);
  if (lane < kSliceBlocks) {
#pragma unroll
    for (int e = 0; e < 8; ++e) pv[wave * kSliceDims + lane * 8 + e] = o[e];
  }
  __syncthreads();
  if (t < kSliceDims) {
    const float r = ((pv[t] + pv[kSliceDims + t]) + pv[2 * kSliceDims + t]) + pv[3 * kSliceDims + t];
    p.out[h * kHeadDim + d0 + t] = (f16)r;
  }
}

__global__ __launch_bounds__(256) void split_attention_kernel(AttnParams p) {
  extern __shared__ float sc[];  // [capacity] scores, then probabilities (output workgroups)
  if ((int)blockIdx.x < p.score_wgs) attention_scores_block(p, (int)blockIdx.x);
  else attention_output_block(p, (int)blockIdx.x - p.score_wgs, sc);
}

// Greedy next token: first index of the largest logit (torch.argmax order), written to
// tokens[position] and token; the position advances by one and h receives the token's
// embedding row.  One workgroup of 1024 threads.
__global__ __launch_bounds__(1024) void argmax_next_kernel(const f16 *logits, int vocab, const f16 *embedding,
                                                           int hidden, f16 *h, int64_t *tokens, int64_t *token,
                                                           int64_t *position, int limit) {
  __shared__ float bv[16];
  __shared__ int bi[16];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  constexpr int kOutOfRange = (int)0x80000000u;
  constexpr int kLoads = 6;  // 16-byte loads per thread per round: 49152 logits per round
  float best = -INFINITY;
  int idx = 0x7fffffff;
  const int full = vocab >> 3;  // whole 8-logit blocks; the tail is read element by element
  const __amdgpu_buffer_rsrc_t lbuf = buffer_rsrc(logits, (size_t)full * 16);
  for (int base = 0; base < full; base += 1024 * kLoads) {
    u4 v[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int b = base + t + 1024 * i;
      v[i] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(lbuf, b < full ? b * 16 : kOutOfRange, 0, 0));
    }
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int b = base + t + 1024 * i;
      const h8 h8v = __builtin_bit_cast(h8, v[i]);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (b < full && (float)h8v[e] > best) { best = (float)h8v[e]; idx = b * 8 + e; }
    }
  }
  for (int i = full * 8 + t; i < vocab; i += 1024)
    if ((float)logits[i] > best) { best = (float)logits[i]; idx = i; }
  if (idx == 0x7fffffff) idx = vocab;  // a thread with no element (or only -inf) loses every tie below
  // (value, index) pairs reduced by the larger value, then the smaller index: a total order, so the
  // result does not depend on the order of the steps.  Within each row of 16 lanes on DPP moves,
  // then over the four rows and the sixteen waves.
  auto take = [](float &bv_, int &bi_, float ov, int oi) {
    if (ov > bv_ || (ov == bv_ && oi < bi_)) { bv_ = ov; bi_ = oi; }
  };
  auto row_best = [&](float &bv_, int &bi_) {
    take(bv_, bi_, dpp_move<kDppXor1>(bv_), dpp_move<kDppXor1>(bi_));
    take(bv_, bi_, dpp_move<kDppXor2>(bv_), dpp_move<kDppXor2>(bi_));
    take(bv_, bi_, dpp_move<kDppHalfMirror>(bv_), dpp_move<kDppHalfMirror>(bi_));
    take(bv_, bi_, dpp_move<kDppMirror>(bv_), dpp_move<kDppMirror>(bi_));
  };
  row_best(best, idx);
#pragma unroll
  for (int r = 16; r < 64; r += 16)
    take(best, idx, lane_value(best, r), __builtin_amdgcn_readlane(idx, r));
  if (lane == 0) { bv[wave] = best; bi[wave] = idx; }
  __syncthreads();
  if (wave != 0) return;
  // Wave 0: the sixteen wave results (lanes 16..63 hold copies that lose every comparison), the
  // token's bookkeeping, then the next input embedding.
  best = lane < 16 ? bv[lane] : -INFINITY;
  idx = lane < 16 ? bi[lane] : 0x7fffffff;
  row_best(best, idx);
  int i0 = __builtin_amdgcn_readfirstlane(idx);
  if (i0 >= vocab) i0 = 0;  // every logit -inf: torch.argmax returns 0
  if (lane == 0) {
    const int64_t pos = position[0];
    if (pos >= 0 && pos < limit) {
      tokens[pos] = i0;
      position[0] = pos + 1;
    }
    token[0] = i0;
  }
  for (int b = lane; b * 8 < hidden; b += 64)
    *reinterpret_cast<h8 *>(h + b * 8) = *reinterpret_cast<const h8 *>(embedding + (size_t)i0 * hidden + b * 8);
}

}  // namespace lb
