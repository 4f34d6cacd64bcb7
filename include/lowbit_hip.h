/*
 * lowbit_hip.h -- C-ABI of liblowbit_hip.so, the MI355X (gfx950) low-bit
 * quantized linear path: W8 per-output-channel, INT4 group-wise and NF4
 * codebook dequant-GEMV/GEMM with an optional fused rank-r low-rank
 * correction y += fp16(fp16(x.V^T).U^T).
 *
 * Conventions (adopted from the reference's native boundary, not its code):
 *   - Status codes keep the numbering of npunlock_status
 *     (reference: npunlock/include/npunlock/error.h:12-26).
 *   - Argument structs are versioned by a leading struct_size, as
 *     graphinfer_* structs are (npunlock/include/npunlock/graphinfer.h:31-198).
 *   - The caller owns every buffer.  All pointers are device pointers except
 *     the argument struct itself.  Buffers are borrowed until the work queued
 *     on `stream` completes; nothing is freed or retained by the library.
 *   - Outputs may not alias inputs (reference: backend.cpp:265-272).
 *   - Calls are asynchronous and ordered on `stream` (a hipStream_t; NULL is
 *     the default stream).  No entry point allocates device memory; scratch
 *     comes from a caller workspace sized by lb_workspace_bytes() (or, for
 *     lb_linear_noalloc, from a library-held array).  Calls that share one
 *     workspace must be ordered (same stream); concurrent calls race.
 *   - On any status other than LB_OK, lb_last_error() returns a thread-local
 *     message describing the failure, valid until the next call on the same
 *     thread.  Argument errors are detected before anything is launched.
 *
 * Packed layouts are exactly the reference's PackedWeight bytes
 * (torch_npu_lowbit.py:24-75):
 *   int8: N*K signed bytes, row-major [N,K].
 *   int4/nf4: ceil(N*K/2) bytes; flat element 2i in the low nibble of byte i,
 *             element 2i+1 in the high nibble (rows are not padded, so for odd
 *             K a row may start mid-byte).
 *   scales: fp16 [N, K/group_size] row-major.
 * Decoded integer value q: int8 as stored; int4 ((c ^ 8) - 8) in [-8,7];
 * nf4 the fp16-rounded codebook entry NF4[c].
 */
#ifndef LOWBIT_HIP_H
#define LOWBIT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LB_ABI_VERSION 6

typedef enum lb_status {
  LB_OK = 0,
  LB_INVALID_ARGUMENT = 1,
  LB_OUT_OF_MEMORY = 2,
  LB_UNSUPPORTED = 5,
  LB_DEVICE_FAILED = 10,
  LB_INTERNAL = 12
} lb_status;

typedef enum lb_format {
  LB_FORMAT_INT8 = 0,
  LB_FORMAT_INT4 = 1,
  LB_FORMAT_NF4 = 2,
  LB_FORMAT_FP16 = 3 /* dense fp16 [N,K] weights (protected projections, tied head); scales unused */
} lb_format;

/* lb_linear_args.flags */
#define LB_FLAG_FORCE_GEMV    0x1u /* decode-regime kernel regardless of M (M <= 32) */
#define LB_FLAG_FORCE_GEMM    0x2u /* prefill-regime MFMA GEMM regardless of M */
#define LB_FLAG_FORCE_GENERIC 0x4u /* shape-agnostic fallback kernel (any N, K, group) */
/* Streaming GEMVs (the kernels one-row calls over >= 64 MB of INT4 weights with rows shorter than
 * 2048 codes, and 2..32-row calls over >= 64 MB, take by themselves) regardless of size: INT4/INT8 codes, no
 * correction or variant, 16-byte aligned codes and x rows, K a multiple of 32 (INT4) or 16 (INT8),
 * groups of one per row or a power of two, each 128-code (INT4) / 64-code (INT8) piece of a row
 * spanning 1, 2 or 4 whole groups; M == 1 or 17 <= M <= 32 with K <= 16384, or 2 <= M <= 16 with
 * K <= 4096 and, as M grows, longer groups (INT4: >= 64 codes up to 8 rows, >= 128 beyond; INT8:
 * >= 64 codes).  Up to 4 rows the sums use the exact q * s weights (the reference's rounding-budget
 * gate bounds the difference to fp16(q * s)); from 5 rows, fp16(q * s).  LB_UNSUPPORTED otherwise.
 * No counterpart in the reference: the path choice is internal there. */
#define LB_FLAG_FORCE_STREAM  0x20u
/* The several-row GEMV on 32x32 MFMA tiles (the kernel 17..32-row calls over >= 16 MB of INT4 / NF4
 * or >= 4 MB of INT8 weights take by themselves, and 9..16-row INT4 / NF4 calls over 16..64 MB split
 * into at most 4 K slices) regardless of size: INT4/NF4/INT8 codes, no
 * correction or variant, M <= 32,
 * 16-byte aligned codes and x rows, K a multiple of 512 (INT4, NF4) / 256 (INT8) up to 65536, and
 * per-row INT8 or power-of-two groups of at least 128 (INT4, NF4) / 64 (INT8) codes dividing that.
 * Sums use the exact q * s weights (NF4: the fp16 literal times the scale; the reference's
 * rounding-budget gate bounds the difference to fp16(q * s)); per-row INT8 multiplies the whole
 * sum by the row scale.  LB_UNSUPPORTED otherwise.
 * No counterpart in the reference: the path choice is internal there. */
#define LB_FLAG_FORCE_WIDE    0x40u
/* One fp16 product per group of K, summed by a balanced fp16 add tree (neighbours pair up,
 * an odd last piece moves up unpaired), then + bias: the compact_groups graph of the
 * reference (torch_npu_lowbit.py:235-256).  At most 32 groups; no correction.  With one
 * group the call is the default linear, as in the reference. */
#define LB_FLAG_COMPACT_GROUPS 0x8u
/* W8A8: int8 per-row weights (group_size == K) and activations quantized on the power-of-two
 * grid activation_scale: qx = clip(rint(x / s_x), -128, 127); the weight grid has the
 * zero point at code 128, step_n = (fp16(127 s_n) - fp16(-128 s_n)) / 255;
 * y = fp16((sum_k qx.qw) * s_x * step_n) with an exact integer sum and one fp64 product,
 * then fp16(y + b).  The FakeQuantize graph of torch_npu_lowbit.py:224-231 as validated by
 * torch_npu_int8_demo.py:34-51.  No correction; K <= 131072. */
#define LB_FLAG_W8A8 0x10u
/* The workspace begins with LB_ZEROED_WORKSPACE_BYTES bytes that are zero, and the caller keeps
 * them for this library: allocate the workspace zeroed once and reuse it.  Every call with this
 * flag places its own scratch after those bytes and, once it has run, leaves them zero again (a
 * launch error leaves the library failed instead).  The GEMVs that split K into slices then add
 * the slices in the kernel, in the last workgroup of each block of output rows (one counter there
 * per block), instead of in a second launch, with the same result bit for bit: the 17..32-row
 * kernel (up to 4 slices, N a multiple of 4 up to 262144) and the 2..16-row one-tile kernel over
 * rows longer than it stages whole (up to 1024 workgroup columns).  lb_workspace_bytes counts the
 * reserved bytes; a call whose plan needs no scratch needs only them.  lb_linear_noalloc ignores
 * the flag.  Calls sharing a workspace must not overlap, as for any workspace.  No counterpart in
 * the reference (its NPU graph owned its intermediates, torch_npu_lowbit.py:189-277). */
#define LB_FLAG_ZEROED_WORKSPACE 0x80u
#define LB_ZEROED_WORKSPACE_BYTES 4096u

typedef struct lb_linear_args {
  uint32_t struct_size;     /* sizeof(lb_linear_args) */
  uint32_t format;          /* lb_format */
  int64_t M, N, K;          /* y[M,N] = x[M,K] . W[N,K]^T */
  int64_t group_size;       /* K % group_size == 0; == K for per-row scales */
  const void *codes;        /* PackedWeight.data bytes (or fp16 [N,K] for LB_FORMAT_FP16) */
  const void *scales;       /* fp16 [N, K/group_size] */
  const void *x;            /* fp16 [M,K], row stride ldx elements */
  int64_t ldx;
  void *y;                  /* fp16 [M,N], row stride ldy elements */
  int64_t ldy;
  const void *bias;         /* fp16 [N] or NULL */
  int64_t rank;             /* 0: no correction */
  const void *down;         /* V fp16 [rank, K] row-major (row stride K) */
  const void *up;           /* U fp16 [N, up_ld], first `rank` columns used */
  int64_t up_ld;            /* row stride of U in elements (0 means rank) */
  void *workspace;          /* caller-owned device scratch */
  size_t workspace_bytes;   /* >= lb_workspace_bytes(args) */
  uint32_t flags;           /* LB_FLAG_* */
  uint32_t reserved;
  float activation_scale;   /* LB_FLAG_W8A8: a power of two in [2^-24, 256] (ignored otherwise) */
  uint32_t reserved2;
} lb_linear_args;

/* ABI version of the loaded library (LB_ABI_VERSION at build time). */
int lb_abi_version(void);

/* Static name of a status, e.g. "LB_INVALID_ARGUMENT". */
const char *lb_status_name(lb_status status);

/* Thread-local description of the last failure on this thread ("" if none). */
const char *lb_last_error(void);

/*
 * Process-wide failed state, the counterpart of the reference's failed context
 * (npunlock-probe/torch-device/backend.cpp:58-60, 280-292, reported as context_failed at :470).
 * A launch that reports a device error marks the library failed; from then on every entry point
 * that enqueues work returns LB_DEVICE_FAILED ("restart the process") without launching.
 * lb_failed() returns 1 in that state.  lb_mark_failed(reason) enters it from the caller's side:
 * the library never synchronises, so a device fault surfaces at the caller's own synchronisation,
 * which reports it here.  The state lasts until the process ends.
 */
int lb_failed(void);
void lb_mark_failed(const char *reason);

/*
 * Bytes of device workspace lb_linear needs for these arguments (0 when none).
 * Host-only; validates args.  Replaces nothing in the reference: the NPU graph
 * owned its intermediates (torch_npu_lowbit.py:189-277).
 */
lb_status lb_workspace_bytes(const lb_linear_args *args, size_t *bytes);

/*
 * y = x . dequant(W)^T [+ bias] [+ fp16(fp16(x.V^T).U^T)], fp32 accumulation,
 * fp16 output with the reference's staging:
 *   main = fp16(acc); with bias: fp16(main + b); with correction:
 *   z = fp16(x.V^T), d = fp16(z.U^T), y = fp16(y + d).
 * Weight values: int8 with per-row scales use the exact product q*s
 * (acc * s in fp32); every other case uses fp16(q*s), the reference's
 * PackedWeight.dequantize() value.  LB_FLAG_COMPACT_GROUPS and LB_FLAG_W8A8 select the
 * reference's compact_groups and activation_scale graphs (see the flags above); their
 * workspace holds the fp16 partials [groups, M, N] or the quantized activations int8 [M, K].
 * Replaces the lowbit_linear graph of weight_graph()
 * (torch_npu_lowbit.py:189-277) executed through _C.run / run_many_impl
 * (npunlock-probe/torch-device/backend.cpp:253-348) and
 * graphinfer_session_infer (npunlock/include/npunlock/graphinfer.h:173-176),
 * plus the correction MatMul/MatMul/Add of the SmolLM linear()
 * (torch_npu_smollm.py:254-258).
 */
lb_status lb_linear(const lb_linear_args *args, void *stream);

/* Scratch held per GPU by the allocation-free entry point below (bytes). */
#define LB_NOALLOC_SCRATCH_BYTES (32u << 20)

/*
 * lb_linear without a caller workspace and without any allocation: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  args->workspace must be NULL and
 * workspace_bytes 0; the scratch a call needs (split-K partials, the correction's z and d,
 * W8A8 activations, compact_groups pieces) comes from a device array of
 * LB_NOALLOC_SCRATCH_BYTES that the library holds on each GPU until the process ends.  A call
 * needing more (lb_workspace_bytes) is refused with LB_INVALID_ARGUMENT before any launch.
 * Same kernels, results and stream ordering as lb_linear.  Every call on one GPU shares that
 * GPU's array and nothing in it needs to start at zero; calls that overlap on one GPU (other
 * streams, other threads) race on it, so order them on one stream.  The first call on a GPU
 * looks the array's address up (making that GPU current for the lookup).
 */
lb_status lb_linear_noalloc(const lb_linear_args *args, void *stream);

/*
 * Bit-exact decode of packed codes to int8 out[N*K] (row-major):
 * int8 -> value, int4 -> ((c ^ 8) - 8), nf4 -> code index c in 0..15.
 * Device counterpart of the Convert(i4/nf4/i8) decode of weight_graph
 * (torch_npu_lowbit.py:216-220) and of the unpack in
 * PackedWeight.dequantize (torch_npu_lowbit.py:69-73).
 */
lb_status lb_unpack_codes(uint32_t format, int64_t N, int64_t K, const void *codes,
                          int8_t *out, void *stream);

/*
 * w[N,K] fp16 = fp16(q * s), bit-identical to PackedWeight.dequantize()
 * (torch_npu_lowbit.py:67-75).
 */
lb_status lb_dequantize(uint32_t format, int64_t N, int64_t K, int64_t group_size,
                        const void *codes, const void *scales, void *w_out, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* LOWBIT_HIP_H */
