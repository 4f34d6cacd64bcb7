// gfx950 prefill GEMM of the low-bit linear path: y[M,N] = x[M,K] . dequant(W)[N,K]^T.
//
// 256 threads (2 x 2 waves) per BM x BN tile; each wave owns a (BM/2) x (BN/2) block of
// v_mfma_f32_32x32x16_f16 tiles.  K advances in steps of BK = 64:
//   - the activations (fp16) and the packed weights of a step are fetched with 16-byte buffer
//     loads two steps ahead into registers (rows past M or N, and k past K, read zeros);
//   - the weights are decoded to fp16 (fp16(q*s), or q for per-row int8) once per tile and
//     written with the activations into one of two LDS buffers (gfx950 has 160 KB of LDS per
//     workgroup, so both buffers of a 128 x 128 tile fit);
//   - one barrier per step separates the MFMAs on buffer s % 2 from the writes of step s + 1
//     into the other buffer.
// The loop is unrolled by two so each register stage keeps its own registers (a loaded
// register is never copied before its load completes).  The epilogue is the linear path's
// (store_output): per-row scale, fp16, bias, correction; with split-K the fp32 sums of each
// K slice go to p.partial and splitk_reduce_kernel applies it.
#pragma once
#include <type_traits>
#include <utility>

#include "lb_kernels.h"

namespace lb {

#ifndef LB_GEMM_IGLP
#define LB_GEMM_IGLP 0
#endif
// LDS swizzle of gemm4_kernel: row r stores chunk c at c ^ LB_G4_SWZ(r).  Rows are 128 bytes, so
// two consecutive rows cover the 64 banks once; with the shift of 1 the 16 rows a 16-byte access
// serves together land on distinct (row parity, chunk) bank groups.
#ifndef LB_GEMM4_SWZ_SHIFT
#define LB_GEMM4_SWZ_SHIFT 1  // chunk c ^ ((r >> 1) & 7): conflict-free 16-row groups over 64 LDS banks
#endif
#define LB_G4_SWZ(r) (((r) >> LB_GEMM4_SWZ_SHIFT) & 7)
#ifndef LB_GEMM4_SCHED
#define LB_GEMM4_SCHED 1  // interleave each MFMA with a share of the step's other instructions
#endif
#ifndef LB_GEMM4_ADMA
#define LB_GEMM4_ADMA 1  // activations straight from memory to LDS (buffer_load ... lds)
#endif
#ifndef LB_GEMM4_SCHED_VALU
#define LB_GEMM4_SCHED_VALU 0  // VALU instructions after each MFMA (0: by block size, below)
#endif
#ifndef LB_GEMM4_SCHED_DSR
#define LB_GEMM4_SCHED_DSR 0  // LDS reads after each MFMA (0: 2 with eight or more waves, else 1)
#endif
#ifndef LB_GEMM_IGLP_VALU
#define LB_GEMM_IGLP_VALU 4
#endif

template <int FMT, int BM, int BN, int BK>
struct G2Traits {
  static constexpr int BITS = FormatTraits<FMT>::BITS;
  static constexpr int A_CHUNKS = BM * BK * 2 / 16;              // 16-byte chunks of the A tile
  static constexpr int B_CHUNKS = BN * BK * BITS / 8 / 16;       // of the packed B tile
  static constexpr int A_PER = (A_CHUNKS + 255) / 256;
  static constexpr int B_PER = (B_CHUNKS + 255) / 256;
  static constexpr int CODES = 16 * 8 / BITS;                    // codes per 16-byte chunk
  static constexpr int CHUNKS_PER_ROW = BK / CODES;              // B chunks per row per step
  static constexpr int A_PER_ROW = BK / 8;                       // A chunks per row per step
};

template <int FMT, int BM, int BN, int BK>
struct G2Stage {
  u4 a[G2Traits<FMT, BM, BN, BK>::A_PER];
  u4 b[G2Traits<FMT, BM, BN, BK>::B_PER];
  f16 s[G2Traits<FMT, BM, BN, BK>::B_PER];
};

// K % BK == 0 (the dispatcher guarantees it): no step reads past K.
template <int FMT, bool SCALED, int BM, int BN, int BK>
__global__ __launch_bounds__(256) void gemm2_kernel(LinearParams p) {
  using T = G2Traits<FMT, BM, BN, BK>;
  using Stage = G2Stage<FMT, BM, BN, BK>;
  constexpr int LD = BK + 8;                 // LDS row pitch in halves: rows start on different banks
  constexpr int TM = BM / 64, TN = BN / 64;  // 32x32 MFMA tiles per wave along M and N
  constexpr int CPC = T::CODES;              // codes per B chunk
  constexpr int kOutOfRange = (int)0x80000000u;
  __shared__ __align__(16) f16 As[2][BM * LD];
  __shared__ __align__(16) f16 Bs[2][BN * LD];
  __shared__ uint32_t nf4_table[FMT == FMT_NF4 ? 256 : 1];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int bm = blockIdx.y * BM, bn = blockIdx.x * BN;
  if constexpr (FMT == FMT_NF4) build_nf4_pair_table(nf4_table);
  select_slice(p);

  const int rows_a = min(BM, p.M - bm), rows_b = min(BN, p.N - bn);
  const size_t row_bytes = (size_t)p.code_ld;
  // Buffer views start at the tile's first row; rows past M / N are out of range (zeros).
  const __amdgpu_buffer_rsrc_t xbuf =
      buffer_rsrc(p.x + (size_t)bm * p.ldx, rows_a > 0 ? ((size_t)(rows_a - 1) * p.ldx + p.K) * 2 : 0);
  const __amdgpu_buffer_rsrc_t wbuf = buffer_rsrc(p.codes + (size_t)bn * row_bytes, (size_t)rows_b * row_bytes);
  const __amdgpu_buffer_rsrc_t sbuf =
      buffer_rsrc(SCALED ? p.scales + (size_t)bn * p.G : p.scales, SCALED ? (size_t)rows_b * p.G * 2 : 0);

  // Per-thread byte offsets of its chunks at k = 0 (out of range for rows past M / N); a step
  // adds its k offset.  The out-of-range offset plus any k stays out of range (unsigned).
  int a_off[T::A_PER], b_off[T::B_PER], s_off[T::B_PER];
#pragma unroll
  for (int i = 0; i < T::A_PER; ++i) {
    const int c = tid + 256 * i;
    const int r = c / T::A_PER_ROW, k = (c % T::A_PER_ROW) * 8;
    a_off[i] = c < T::A_CHUNKS && r < rows_a ? (r * p.ldx + k) * 2 : kOutOfRange;
  }
#pragma unroll
  for (int i = 0; i < T::B_PER; ++i) {
    const int c = tid + 256 * i;
    const int r = c / T::CHUNKS_PER_ROW, k = (c % T::CHUNKS_PER_ROW) * CPC;
    const bool ok = c < T::B_CHUNKS && r < rows_b;
    b_off[i] = ok ? (int)(r * row_bytes) + k * T::BITS / 8 : kOutOfRange;
    s_off[i] = ok ? r * p.G * 2 : kOutOfRange;
  }
  auto load = [&](Stage &st, int k0) {
#pragma unroll
    for (int i = 0; i < T::A_PER; ++i)
      st.a[i] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(xbuf, a_off[i] + k0 * 2, 0, 0));
#pragma unroll
    for (int i = 0; i < T::B_PER; ++i) {
      st.b[i] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(wbuf, b_off[i] + k0 * T::BITS / 8, 0, 0));
      if constexpr (SCALED)  // a chunk lies inside one group (group >= 32 >= codes per chunk)
        st.s[i] = __builtin_bit_cast(
            f16, __builtin_amdgcn_raw_buffer_load_b16(
                     sbuf, s_off[i] + (((k0 + (tid % T::CHUNKS_PER_ROW) * CPC) >> p.group_shift) << 1), 0, 0));
    }
  };
  // Chunk guards are compile-time when the chunk counts are whole multiples of the 256 threads:
  // a runtime guard would split the step into basic blocks and keep the decode from being
  // scheduled among the MFMAs.
  auto store = [&](Stage &st, int buf) {
#pragma unroll
    for (int i = 0; i < T::A_PER; ++i) {
      const int c = tid + 256 * i;
      asm volatile("" : "+v"(st.a[i]));
      if (T::A_CHUNKS % 256 == 0 || c < T::A_CHUNKS)
        *reinterpret_cast<u4 *>(&As[buf][(c / T::A_PER_ROW) * LD + (c % T::A_PER_ROW) * 8]) = st.a[i];
    }
#pragma unroll
    for (int i = 0; i < T::B_PER; ++i) {
      const int c = tid + 256 * i;
      asm volatile("" : "+v"(st.b[i]));
      if (T::B_CHUNKS % 256 != 0 && c >= T::B_CHUNKS) continue;
      const int r = c / T::CHUNKS_PER_ROW, kk = (c % T::CHUNKS_PER_ROW) * CPC;
      f16 *dst = &Bs[buf][r * LD + kk];
      const h2 s2 = SCALED ? h2{st.s[i], st.s[i]} : h2{(f16)1.0f, (f16)1.0f};
      if constexpr (T::BITS == 4) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<h8 *>(dst + 8 * q) = decode8_natural<FMT, SCALED>(st.b[i][q], 0u, s2, nf4_table);
      } else if constexpr (T::BITS == 8) {
        *reinterpret_cast<h8 *>(dst) = decode8_natural<FMT, SCALED>(st.b[i][0], st.b[i][1], s2, nf4_table);
        *reinterpret_cast<h8 *>(dst + 8) = decode8_natural<FMT, SCALED>(st.b[i][2], st.b[i][3], s2, nf4_table);
      } else {
        *reinterpret_cast<u4 *>(dst) = st.b[i];
      }
    }
  };

  f16x acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int jj = 0; jj < TN; ++jj)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][jj][r] = 0.0f;

  auto compute = [&](int buf) {
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      h8 a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        a[i] = *reinterpret_cast<const h8 *>(&As[buf][(wm * (BM / 2) + i * 32 + (lane & 31)) * LD + kk + 8 * (lane >> 5)]);
#pragma unroll
      for (int jj = 0; jj < TN; ++jj)
        b[jj] = *reinterpret_cast<const h8 *>(&Bs[buf][(wn * (BN / 2) + jj * 32 + (lane & 31)) * LD + kk + 8 * (lane >> 5)]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int jj = 0; jj < TN; ++jj)
          acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[jj], acc[i][jj], 0, 0, 0);
    }
  };

  // Scheduling hint for one step: spread the decode VALU work and the LDS traffic of the next
  // step between the MFMAs (they use different units and have no data dependences).
  auto interleave = [&]() {
#if LB_GEMM_IGLP
    constexpr int MFMAS = TM * TN * (BK / 16);
#pragma unroll
    for (int i = 0; i < MFMAS; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // one LDS read
      __builtin_amdgcn_sched_group_barrier(0x002, LB_GEMM_IGLP_VALU, 0);  // VALU
    }
#endif
  };

  // Step s computes on buffer s % 2; the register stage holding step s + 1 (loaded two steps
  // earlier) is decoded into the other buffer, and step s + 3 is loaded into the stage just
  // emptied.  Loads are unconditional (steps past K read out of range): the waits stay exact.
  // Loads of steps past the last one re-read the last step (in range, unused).  With split-K
  // (p.splits > 1, grid z = split) the workgroup covers k in [z * kslice, z * kslice + kslice).
  const int kbeg = p.splits > 1 ? (int)blockIdx.z * p.kslice : 0;
  const int steps = (min(p.K, kbeg + (p.splits > 1 ? p.kslice : p.K)) - kbeg) / BK;
  const int klast = kbeg + (steps - 1) * BK;
  Stage r0, r1;
  load(r0, kbeg);
  load(r1, min(kbeg + BK, klast));
  // Every entry of the NF4 table (each written by one thread) before the first decode reads it.
  if constexpr (FMT == FMT_NF4) __syncthreads();
  store(r0, 0);
  load(r0, min(kbeg + 2 * BK, klast));
  __syncthreads();
  int s = 0;
  for (; s + 2 <= steps; s += 2) {
    compute(0);                 // step s; r1 = step s + 1, r0 = step s + 2
    store(r1, 1);
    load(r1, min(kbeg + (s + 3) * BK, klast));
    interleave();
    __syncthreads();
    compute(1);                 // step s + 1; r0 = step s + 2, r1 = step s + 3
    store(r0, 0);
    load(r0, min(kbeg + (s + 4) * BK, klast));
    interleave();
    __syncthreads();
  }
  if (s < steps) compute(0);    // odd step count: the last step is in buffer 0

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
        if (m >= p.M) continue;
        if (p.splits > 1) p.partial[((size_t)blockIdx.z * p.M + m) * p.N + n] = acc[i][jj][r];
        else store_output(p, m, n, acc[i][jj][r]);
      }
    }
}

typedef uint32_t u2w __attribute__((ext_vector_type(2)));

// Calls f(std::integral_constant<int, i>) for i = 0 .. N-1 (compile-time indices, so register
// arrays indexed by them stay in registers).
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// BM x BN prefill GEMM (BM, BN = 128 or 256) with WAVES = 4 or 8 waves in a WM x (WAVES / WM)
// grid; a wave owns a (BM / WM) x (BN / (WAVES / WM)) block of v_mfma_f32_32x32x16_f16 tiles
// (TM x TN), whose fp32 accumulators live in AGPRs.  Per K step of 64 and 16-deep substep, a wave
// reads TM A and TN B fragments for its TM TN MFMAs.  LDS holds two stages of A (fp16 activations)
// and B (decoded fp16 weights), BM (BN) rows x 64 halves each, without padding: the 16-byte chunk c
// of row r is stored at chunk c ^ LB_G4_SWZ(r), so the rows of a fragment read hit distinct banks.
// The next step's activations go straight from memory to the other LDS stage (buffer_load ...
// lds; the two stages are separate arrays so the compiler sees no alias with the stage being
// read), issued at the start of the step and complete before its closing barrier; the packed
// weights of the step after it are loaded into registers and decoded into the other B stage
// between the MFMA groups.  Each MFMA of a substep is followed by a share of the other work (one or,
// with eight waves, two LDS reads, up to 8 VALU, one LDS write, one global load:
// sched_group_barrier), so the MFMA pipe
// is fed while the decode and the transfers proceed.  Fragment reads of substep kk + 1 are issued
// before the MFMAs of substep kk.  With split-K (p.splits > 1, grid z = split) a workgroup covers
// k in [z * kslice, z * kslice + kslice) and writes fp32 sums to p.partial.
template <int FMT, bool SCALED, int WAVES, int BM = 256, int BN = 256, int WM = 2>
__global__ __launch_bounds__(64 * WAVES) void gemm4_kernel(LinearParams p) {
  constexpr int BK = 64;
  constexpr int NT = 64 * WAVES;
  constexpr int WN = WAVES / WM;                    // waves along N
  constexpr int WROWS = BM / WM;                    // rows per wave
  constexpr int TM = WROWS / 32;                    // 32-row MFMA tiles per wave
  constexpr int WCOLS = BN / WN;                    // columns per wave
  constexpr int TN = WCOLS / 32;                    // 32-column MFMA tiles per wave
  constexpr int BITS = FormatTraits<FMT>::BITS;
  // Packed B chunks of 16 bytes, or of 8 where 16-byte chunks would leave threads without one
  // (4-bit codes, BN * 2 < NT): every thread then decodes an equal share.
  constexpr int CB = BN * (BK * BITS / 8 / 16) < NT ? 8 : 16;
  constexpr int CODES = CB * 8 / BITS;              // codes per B chunk
  constexpr int B_ROW_CHUNKS = BK / CODES;          // packed chunks per B row per step
  constexpr int B_PER = BN * B_ROW_CHUNKS / NT;     // packed B chunks per thread per step
  constexpr int A_PER = BM * (BK / 8) / NT;         // A chunks per thread per step
  constexpr int STAGE_A = BM * BK, STAGE_B = BN * BK;  // halves per operand per stage
  constexpr int kOutOfRange = (int)0x80000000u;
  // VALU instructions placed after each MFMA: blocks of 8+ MFMA tiles spread the decode thinly,
  // smaller blocks (fewer MFMAs per substep) take it in larger shares.
  constexpr int SCHED_VALU =
      LB_GEMM4_SCHED_VALU > 0 ? LB_GEMM4_SCHED_VALU : (TM * TN >= 8 ? (WAVES >= 8 ? 8 : 4) : 16);
  // LDS reads placed after each MFMA: two with eight waves (1-4% on the 256-wide tiles), one with four.
  constexpr int SCHED_DSR = LB_GEMM4_SCHED_DSR > 0 ? LB_GEMM4_SCHED_DSR : (WAVES >= 8 ? 2 : 1);
  static_assert((WAVES == 4 || WAVES == 8 || WAVES == 16) && WAVES % WM == 0 && TM >= 1 && TN >= 1 && B_PER >= 1 &&
                    A_PER >= 1 && BN * B_ROW_CHUNKS % NT == 0 && BM * (BK / 8) % NT == 0 && (CB == 16 || BITS == 4),
                "tile constants");
  // The two activation stages are separate arrays, so the compiler sees that a transfer into one
  // does not alias reads of the other.
  __shared__ __align__(16) f16 As0[STAGE_A];
  __shared__ __align__(16) f16 As1[STAGE_A];
  __shared__ __align__(16) f16 Bs[2 * STAGE_B];
  __shared__ uint32_t nf4_table[FMT == FMT_NF4 ? 256 : 1];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int bm = blockIdx.y * BM, bn = blockIdx.x * BN;
  if constexpr (FMT == FMT_NF4) build_nf4_pair_table(nf4_table);
  select_slice(p);

  const int rows_a = min(BM, p.M - bm), rows_b = min(BN, p.N - bn);
  const int row_bytes = p.code_ld;
  const __amdgpu_buffer_rsrc_t xbuf =
      buffer_rsrc(p.x + (size_t)bm * p.ldx, rows_a > 0 ? ((size_t)(rows_a - 1) * p.ldx + p.K) * 2 : 0);
  const __amdgpu_buffer_rsrc_t wbuf = buffer_rsrc(p.codes + (size_t)bn * row_bytes, (size_t)rows_b * row_bytes);
  const __amdgpu_buffer_rsrc_t sbuf =
      buffer_rsrc(SCALED ? p.scales + (size_t)bn * p.G : p.scales, SCALED ? (size_t)rows_b * p.G * 2 : 0);

  // Global byte offsets at k = 0 and LDS slots of this thread's chunks.
  int a_off[A_PER], a_lds[A_PER], b_off[B_PER], s_off[B_PER], b_row[B_PER], b_code[B_PER];
#pragma unroll
  for (int i = 0; i < A_PER; ++i) {
    const int c = tid + NT * i, r = c >> 3, lc = c & 7;
    a_off[i] = r < rows_a ? (r * p.ldx + 8 * lc) * 2 : kOutOfRange;
    a_lds[i] = r * BK + 8 * (lc ^ LB_G4_SWZ(r));
  }
#pragma unroll
  for (int i = 0; i < B_PER; ++i) {
    const int c = tid + NT * i, r = c / B_ROW_CHUNKS, kc = (c % B_ROW_CHUNKS) * CODES;
    const bool ok = r < rows_b;
    b_off[i] = ok ? r * row_bytes + kc * BITS / 8 : kOutOfRange;
    s_off[i] = ok ? r * p.G * 2 : kOutOfRange;
    b_row[i] = r;
    b_code[i] = kc;
  }
  u4 ra[A_PER], rb[B_PER];
  f16 rs[B_PER];
  auto load = [&](int k0) {
#if !LB_GEMM4_ADMA
#pragma unroll
    for (int i = 0; i < A_PER; ++i)
      ra[i] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(xbuf, a_off[i] + k0 * 2, 0, 0));
#endif
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      if constexpr (CB == 16) {
        rb[i] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(wbuf, b_off[i] + k0 * BITS / 8, 0, 0));
      } else {
        const u2w h = __builtin_bit_cast(u2w, __builtin_amdgcn_raw_buffer_load_b64(wbuf, b_off[i] + k0 * BITS / 8, 0, 0));
        rb[i] = u4{h[0], h[1], 0u, 0u};
      }
      if constexpr (SCALED)
        rs[i] = __builtin_bit_cast(
            f16, __builtin_amdgcn_raw_buffer_load_b16(sbuf, s_off[i] + (((k0 + b_code[i]) >> p.group_shift) << 1), 0, 0));
    }
  };
  auto astage = [&](auto st) -> f16 * {
    if constexpr (decltype(st)::value == 0) return As0;
    else return As1;
  };
  auto store_a = [&](auto st) {
    f16 *dst = astage(st);
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
      asm volatile("" : "+v"(ra[i]));
      *reinterpret_cast<u4 *>(dst + a_lds[i]) = ra[i];
    }
  };
#if LB_GEMM4_ADMA
  // Activations straight to LDS (buffer_load ... lds): block i of a stage is the 1 KB of rows
  // 8i .. 8i+7; lane L of the wave writes its chunk position L & 7 of row 8i + L / 8, so it loads
  // the row's chunk (L & 7) ^ swizzle(row).  Wave w moves blocks w, w + WAVES, ...
  constexpr int ABLK = BM / 8 / WAVES;  // 1 KB blocks per wave per stage
  int adma_off[ABLK];
#pragma unroll
  for (int i = 0; i < ABLK; ++i) {
    const int r = 8 * (wave + WAVES * i) + (lane >> 3), pc = lane & 7;
    adma_off[i] = r < rows_a ? (r * p.ldx + 8 * (pc ^ LB_G4_SWZ(r))) * 2 : kOutOfRange;
  }
  auto dma_a = [&](auto st, int k0) {
#if defined(__HIP_DEVICE_COMPILE__)  // the LDS address space exists in the device pass only
#pragma unroll
    for (int i = 0; i < ABLK; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          xbuf, (__attribute__((address_space(3))) void *)(astage(st) + (wave + WAVES * i) * 512), 16,
          adma_off[i] + k0 * 2, 0, 0, 0);
#endif
  };
#endif
  auto store_b = [&](int st) {
    f16 *dst = Bs + st * STAGE_B;
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      asm volatile("" : "+v"(rb[i]));
      const int r = b_row[i];
      const h2 s2 = SCALED ? h2{rs[i], rs[i]} : h2{(f16)1.0f, (f16)1.0f};
      constexpr int HALF_CHUNKS = CODES / 8;  // LDS chunks one packed chunk decodes to
#pragma unroll
      for (int q = 0; q < HALF_CHUNKS; ++q) {
        const int lc = b_code[i] / 8 + q;
        h8 v;
        if constexpr (BITS == 4) v = decode8_natural<FMT, SCALED>(rb[i][q], 0u, s2, nf4_table);
        else if constexpr (BITS == 8) v = decode8_natural<FMT, SCALED>(rb[i][2 * q], rb[i][2 * q + 1], s2, nf4_table);
        else v = __builtin_bit_cast(h8, rb[i]);
        *reinterpret_cast<h8 *>(dst + r * BK + 8 * (lc ^ LB_G4_SWZ(r))) = v;
      }
    }
  };

  f16x acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int jj = 0; jj < TN; ++jj)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][jj][r] = 0.0f;

  // Fragment reads: lane row fr = lane & 31 of a tile at logical chunk 2 kk + lane / 32.  Every
  // tile row is fr plus a tile base that is a multiple of 32 (wave block offsets and 32-row MFMA
  // tiles), so while 32 is a multiple of 8 << LB_GEMM4_SWZ_SHIFT the swizzle LB_G4_SWZ(row) equals
  // LB_G4_SWZ(fr): a per-lane constant, and a read is a per-lane base plus compile-time offsets
  // (tile, stage) and one of four chunk offsets.
  static_assert(LB_GEMM4_SWZ_SHIFT >= 0 && LB_GEMM4_SWZ_SHIFT <= 2 && WROWS % 32 == 0 && WCOLS % 32 == 0,
                "fragment swizzle needs tile bases that are multiples of 8 << LB_GEMM4_SWZ_SHIFT");
  const int fr = lane & 31, fh = lane >> 5;
  int koff[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) koff[kk] = 8 * ((2 * kk + fh) ^ LB_G4_SWZ(fr));
  const int a_lane = (wm * WROWS + fr) * BK;
  const f16 *b_lane = Bs + (wn * WCOLS + fr) * BK;

  const int kbeg = p.splits > 1 ? (int)blockIdx.z * p.kslice : 0;
  const int steps = (min(p.K, kbeg + (p.splits > 1 ? p.kslice : p.K)) - kbeg) / BK;
#if LB_GEMM4_ADMA
  // vmcnt-only wait: all but the last n vector-memory operations of this wave are complete.
  auto wait_vm = [](auto n) {
    constexpr int N = decltype(n)::value;
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
  };
  dma_a(std::integral_constant<int, 0>{}, kbeg);
  __builtin_amdgcn_sched_barrier(0);
  load(kbeg);
  // Every entry of the NF4 table (each written by one thread) before the first decode reads it.
  if constexpr (FMT == FMT_NF4) __syncthreads();
  store_b(0);
  load(kbeg + min(1, steps - 1) * BK);
  wait_vm(std::integral_constant<int, 0>{});
#else
  load(kbeg);
  store_a(std::integral_constant<int, 0>{});
  if constexpr (FMT == FMT_NF4) __syncthreads();  // the NF4 table before the first decode
  store_b(0);
  if (steps > 1) load(kbeg + BK);
#endif
  __syncthreads();
  // One K step on LDS stage ST (compile-time, so every LDS offset is an immediate).
  auto step = [&](auto stage, int s) {
    constexpr int ST = decltype(stage)::value;
    const f16 *a_base = astage(stage) + a_lane;
    const f16 *b_base = b_lane + ST * STAGE_B;
    h8 fa[2][TM], fb[2][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) fa[0][i] = *reinterpret_cast<const h8 *>(a_base + i * 32 * BK + koff[0]);
#pragma unroll
    for (int jj = 0; jj < TN; ++jj) fb[0][jj] = *reinterpret_cast<const h8 *>(b_base + jj * 32 * BK + koff[0]);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int cur = kk & 1;
      if (kk < 3) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
          fa[cur ^ 1][i] = *reinterpret_cast<const h8 *>(a_base + i * 32 * BK + koff[kk + 1]);
#pragma unroll
        for (int jj = 0; jj < TN; ++jj)
          fb[cur ^ 1][jj] = *reinterpret_cast<const h8 *>(b_base + jj * 32 * BK + koff[kk + 1]);
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int jj = 0; jj < TN; ++jj)
          acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[cur][i], fb[cur][jj], acc[i][jj], 0, 0, 0);
      // The next step's operands go to the other stage between the MFMA groups.
#if LB_GEMM4_ADMA
      // Activations of step s + 1 go straight to the other stage (free since the last barrier);
      // packed weights of step s + 2 to registers.  Past the last step both re-read it (in range).
      if (kk == 0) {
        dma_a(std::integral_constant<int, ST ^ 1>{}, kbeg + min(s + 1, steps - 1) * BK);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (kk == 2) {
        store_b(ST ^ 1);
        load(kbeg + min(s + 2, steps - 1) * BK);
      }
#if LB_GEMM4_SCHED
#pragma unroll
      for (int i = 0; i < TM * TN; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                  // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, SCHED_DSR, 0);            // LDS reads
        __builtin_amdgcn_sched_group_barrier(0x002, SCHED_VALU, 0);  // VALU
        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);                  // one LDS write
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                  // one global load
      }
#endif
#elif LB_GEMM4_SCHED
      // One basic block per step (past the last step the loads re-read the last step, in range,
      // and the stores fill the idle stage), and each MFMA followed by a share of the other work.
      if (kk == 1) store_a(std::integral_constant<int, ST ^ 1>{});
      if (kk == 2) {
        store_b(ST ^ 1);
        load(kbeg + min(s + 2, steps - 1) * BK);
      }
#pragma unroll
      for (int i = 0; i < TM * TN; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                  // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                  // one LDS read
        __builtin_amdgcn_sched_group_barrier(0x002, SCHED_VALU, 0);  // VALU
        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);                  // one LDS write
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                  // one global load
      }
#else
      if (s + 1 < steps) {
        if (kk == 1) store_a(std::integral_constant<int, ST ^ 1>{});
        if (kk == 2) {
          store_b(ST ^ 1);
          if (s + 2 < steps) load(kbeg + (s + 2) * BK);
        }
      }
#endif
    }
#if LB_GEMM4_ADMA
    // The activations moved this step are complete (only the weight loads issued after them,
    // B_PER codes plus B_PER scales, may be outstanding) before the barrier publishes them.
    wait_vm(std::integral_constant<int, SCALED ? 2 * B_PER : B_PER>{});
#endif
    __syncthreads();
  };
  for (int s = 0; s < steps; s += 2) {
    step(std::integral_constant<int, 0>{}, s);
    if (s + 1 < steps) step(std::integral_constant<int, 1>{}, s + 1);
  }
#if LB_GEMM4_ADMA
  __builtin_amdgcn_s_waitcnt(0);  // no transfer into LDS outlives the loop
#endif

  // D layout of the 32x32 MFMA: lane l, register r -> row 8*(r/4) + 4*(l/32) + r%4, column l%32.
  // Tile indices are compile-time (static_for), so the accumulators stay in AGPRs.
  static_for<TM>([&](auto i) {
    static_for<TN>([&](auto jj) {
      const f16x &v = acc[decltype(i)::value][decltype(jj)::value];
      const int n = bn + wn * WCOLS + decltype(jj)::value * 32 + (lane & 31);
      if (n >= p.N) return;
      const bool split = p.splits > 1;
      const float rs = !split && p.per_row ? (float)p.scales[n] : 1.0f;
      const float b = !split && p.bias ? (float)p.bias[n] : 0.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = bm + wm * WROWS + decltype(i)::value * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m >= p.M) continue;
        if (split) {
          p.partial[((size_t)blockIdx.z * p.M + m) * p.N + n] = v[r];
          continue;
        }
        f16 h = (f16)(v[r] * rs);
        if (p.bias) h = (f16)((float)h + b);
        if (p.delta) h = (f16)((float)h + (float)p.delta[(size_t)m * p.N + n]);
        p.y[(size_t)m * p.ldy + n] = h;
      }
    });
  });
}

}  // namespace lb

