// Shared device helpers for the gfx950 low-bit linear kernels.
//
// Decode rules (reference: torch_npu_lowbit.py:17-21, 67-75):
//   int8  q = stored signed byte
//   int4  q = ((c ^ 8) - 8) for nibble c; flat element 2i is the low nibble of byte i
//   nf4   q = fp16(NF4[c])
//   dequantized weight w = fp16(q * s), one round-to-nearest-even of the exact product.
//
// MFMA operand convention used by every kernel here: for the f16 MFMAs the A and B
// operands use the same (lane / 16 or lane / 32, slot) -> k assignment, so any fixed
// permutation of k inside one 8-element slot group gives the same dot product as long
// as A and B apply it identically.  The unpack routines below therefore emit codes in
// whatever order is cheapest, and the activation staging applies the matching
// permutation (kPerm*).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lb {

typedef _Float16 f16;
typedef f16 h2 __attribute__((ext_vector_type(2)));
typedef f16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

enum Format { FMT_INT8 = 0, FMT_INT4 = 1, FMT_NF4 = 2, FMT_FP16 = 3 };

// fp32 literals of the NormalFloat4 codebook (reference torch_npu_lowbit.py:17-20,
// itself taken from OpenVINO's published nf4.cpp).  The fp16 table is their RNE rounding.
#define LB_NF4_LITERALS                                                              \
  -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,          \
      -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,     \
      0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f,             \
      0.33791524171829224f, 0.44070982933044434f, 0.5626170039176941f,              \
      0.7229568362236023f, 1.0f

__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }
__device__ __forceinline__ uint32_t as_u32(h2 v) { return __builtin_bit_cast(uint32_t, v); }

template <int FMT> struct FormatTraits;
// CPL: codes per 16-byte lane load.  BITS: storage bits per code.
template <> struct FormatTraits<FMT_INT4> { static constexpr int CPL = 32, BITS = 4; };
template <> struct FormatTraits<FMT_NF4>  { static constexpr int CPL = 32, BITS = 4; };
template <> struct FormatTraits<FMT_INT8> { static constexpr int CPL = 16, BITS = 8; };
template <> struct FormatTraits<FMT_FP16> { static constexpr int CPL = 8,  BITS = 16; };

// INT4: one dword (8 nibbles c0..c7, c_i at bits 4i) -> four fp16 pairs holding
// q = (c^8)-8 exactly, in slot order (c0,c2),(c4,c6),(c1,c3),(c5,c7).
// Even / odd nibbles are split into bytes (xor 8 folded in), then v_perm_b32 places each
// byte under the magic 0x64: 0x64bb is the fp16 value 1024 + b, and subtracting 1032 is exact.
__device__ __forceinline__ void int4_pairs(uint32_t w, h2 out[4]) {
  const uint32_t lo = (w & 0x0F0F0F0Fu) ^ 0x08080808u;         // c0 c2 c4 c6
  const uint32_t hi = ((w >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u;  // c1 c3 c5 c7
  const h2 bias = {(f16)-1032.0f, (f16)-1032.0f};
  // v_perm_b32: selector bytes 0-3 pick from the second operand, 4-7 from the first.
  out[0] = as_h2(__builtin_amdgcn_perm(0x64646464u, lo, 0x04010400u)) + bias;
  out[1] = as_h2(__builtin_amdgcn_perm(0x64646464u, lo, 0x04030402u)) + bias;
  out[2] = as_h2(__builtin_amdgcn_perm(0x64646464u, hi, 0x04010400u)) + bias;
  out[3] = as_h2(__builtin_amdgcn_perm(0x64646464u, hi, 0x04030402u)) + bias;
}
// Slot e of an INT4 8-group holds code kPermInt4[e].
__device__ constexpr int kPermInt4[8] = {0, 2, 4, 6, 1, 3, 5, 7};

// INT8: one dword (4 signed bytes b0..b3) -> two fp16 pairs (b0,b2),(b1,b3), exact.
// (b ^ 0x80) in the low mantissa byte of 0x64xx is 1024 + b + 128; subtract 1152.
__device__ __forceinline__ void int8_pairs(uint32_t w, h2 out[2]) {
  const uint32_t t = w ^ 0x80808080u;
  const h2 bias = {(f16)-1152.0f, (f16)-1152.0f};
  // v_perm_b32: selector bytes 0-3 pick from the second operand (t), 4-7 from the first.
  out[0] = as_h2(__builtin_amdgcn_perm(0x64646464u, t, 0x04020400u)) + bias;
  out[1] = as_h2(__builtin_amdgcn_perm(0x64646464u, t, 0x04030401u)) + bias;
}
// Slot e of an INT8 8-group (two dwords) holds code kPermInt8[e].
__device__ constexpr int kPermInt8[8] = {0, 2, 1, 3, 4, 6, 5, 7};

// Permute an 8-element activation block so slot e holds element perm[e].
template <int FMT>
__device__ __forceinline__ h8 permute_block(h8 v) {
  if constexpr (FMT == FMT_INT4) {
    return __builtin_shufflevector(v, v, 0, 2, 4, 6, 1, 3, 5, 7);
  } else if constexpr (FMT == FMT_INT8) {
    return __builtin_shufflevector(v, v, 0, 2, 1, 3, 4, 6, 5, 7);
  } else {
    return v;
  }
}

// NF4 pair table: entry b (a packed byte) = (fp16 NF4[b & 15], fp16 NF4[b >> 4]).
// Built in LDS by each workgroup that needs it.
__device__ __forceinline__ void build_nf4_pair_table(uint32_t *table) {
  const float lit[16] = {LB_NF4_LITERALS};
  for (int b = threadIdx.x; b < 256; b += blockDim.x) {
    h2 v = {(f16)lit[b & 15], (f16)lit[b >> 4]};
    table[b] = as_u32(v);
  }
}

// Decode 8 codes (one MFMA slot group) starting at dword `t8` of a 16-byte lane load
// into an h8 B operand, scaled by s (fp16 multiply, RNE) unless UNSCALED.
// Slot order is the format's kPerm*; FP16 and NF4 use natural order.
template <int FMT, bool UNSCALED>
__device__ __forceinline__ h8 decode8(const u4 &w, int t8, h2 s2, const uint32_t *nf4_table) {
  h8 out;
  if constexpr (FMT == FMT_INT4) {
    h2 p[4];
    int4_pairs(w[t8], p);
    if (!UNSCALED) { p[0] *= s2; p[1] *= s2; p[2] *= s2; p[3] *= s2; }
    out = __builtin_shufflevector(__builtin_shufflevector(p[0], p[1], 0, 1, 2, 3),
                                  __builtin_shufflevector(p[2], p[3], 0, 1, 2, 3),
                                  0, 1, 2, 3, 4, 5, 6, 7);
  } else if constexpr (FMT == FMT_NF4) {
    const uint32_t v = w[t8];
    h2 p[4];
    p[0] = as_h2(nf4_table[v & 0xFFu]);
    p[1] = as_h2(nf4_table[(v >> 8) & 0xFFu]);
    p[2] = as_h2(nf4_table[(v >> 16) & 0xFFu]);
    p[3] = as_h2(nf4_table[v >> 24]);
    if (!UNSCALED) { p[0] *= s2; p[1] *= s2; p[2] *= s2; p[3] *= s2; }
    out = __builtin_shufflevector(__builtin_shufflevector(p[0], p[1], 0, 1, 2, 3),
                                  __builtin_shufflevector(p[2], p[3], 0, 1, 2, 3),
                                  0, 1, 2, 3, 4, 5, 6, 7);
  } else if constexpr (FMT == FMT_INT8) {
    h2 p[4];
    int8_pairs(w[2 * t8], p);
    int8_pairs(w[2 * t8 + 1], p + 2);
    if (!UNSCALED) { p[0] *= s2; p[1] *= s2; p[2] *= s2; p[3] *= s2; }
    out = __builtin_shufflevector(__builtin_shufflevector(p[0], p[1], 0, 1, 2, 3),
                                  __builtin_shufflevector(p[2], p[3], 0, 1, 2, 3),
                                  0, 1, 2, 3, 4, 5, 6, 7);
  } else {
    out = __builtin_bit_cast(h8, w);
  }
  return out;
}

// Raw buffer resource over [base, base + bytes): loads at or beyond `bytes` return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base, size_t bytes) {
  const int records = bytes > 0x7FFFFFF0ull ? 0x7FFFFFF0 : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, records, 0x00020000);
}

// Cache policy of a buffer access performed at the memory side past the per-XCD L2s (sc0 sc1):
// a store is written through before it completes, a load reads what such stores and the
// system-scope atomics wrote, whichever XCD wrote it.
constexpr int kSysCoherent = 17;

// Arguments shared by the linear kernels (device pointers, element strides).
struct LinearParams {
  const uint8_t *codes;   // packed codes, or fp16 weights for FMT_FP16
  const f16 *scales;      // [N, G]
  const f16 *x;           // [M, ldx]
  f16 *y;                 // [M, ldy]
  const f16 *bias;        // [N] or null
  const f16 *z;           // correction activations fp16 [M, rank] (decode epilogue) or null
  const f16 *up;          // U fp16 [N, up_ld] or null
  const f16 *delta;       // precomputed fp16 correction [M, N] (prefill epilogue) or null
  float *partial;         // split-K partial sums [splits, M, N]
  int M, N, K;
  int group, G;           // group size and groups per row
  int ldx, ldy, ldw;      // ldw: row stride (elements) of fp16 weights
  int rank, up_ld;
  int kslice, splits;
  int per_row;            // int8 with one scale per row: scale applied to the fp32 sum
  int group_shift;        // scale index = k >> group_shift (31 when group == K)
  int scales_aligned;     // scales pointer is 16-byte aligned
  int code_ld;            // bytes per weight row (K * bits / 8; 2 * ldw for fp16 weights)
  // Per grid-z-slice offsets (compact groups: slice z computes group z into its own fp16
  // partial output); all zero for a single product.
  int z_x, z_codes, z_scales;
  long long z_y;
  float act_scale;        // W8A8: the activation grid (a power of two)
  const int8_t *xq;       // W8A8: quantized activations [M, K] (row stride K)
  int slices;             // grid z extent (host side: the launchers read it)
};

// Moves p to grid slice blockIdx.z (a no-op when the launch has one slice).
__device__ __forceinline__ void select_slice(LinearParams &p) {
  const int z = blockIdx.z;
  p.x += (size_t)z * p.z_x;
  p.codes += (size_t)z * p.z_codes;
  p.scales += (size_t)z * p.z_scales;
  p.y += (size_t)z * p.z_y;
}

// Epilogue with the reference's staging (torch_npu_lowbit.py:262-266,
// torch_npu_smollm.py:160-163): main -> fp16, + bias -> fp16, + fp16 correction -> fp16.
__device__ __forceinline__ void store_output(const LinearParams &p, int m, int n, float acc) {
  if (p.per_row) acc *= (float)p.scales[n];
  f16 h = (f16)acc;
  if (p.bias) h = (f16)((float)h + (float)p.bias[n]);
  if (p.z) {
    float d = 0.0f;
    const f16 *zr = p.z + (size_t)m * p.rank;
    const f16 *ur = p.up + (size_t)n * p.up_ld;
    for (int j = 0; j < p.rank; ++j) d += (float)zr[j] * (float)ur[j];
    h = (f16)((float)h + (float)(f16)d);
  } else if (p.delta) {
    h = (f16)((float)h + (float)p.delta[(size_t)m * p.N + n]);
  }
  p.y[(size_t)m * p.ldy + n] = h;
}

}  // namespace lb
