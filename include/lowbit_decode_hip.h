/*
 * lowbit_decode_hip.h -- C-ABI of the decode-step entry points of liblowbit_hip.so
 * (MI355X, gfx950): one SmolLM-style decoder token for one sequence, built from a few
 * fused launches instead of one launch per operator.
 *
 * The reference compiles each decoder layer into one NPU graph
 * (torch_npu_smollm.py:195-340, FrozenSmolLayer.graph) and submits 30 of them per token in
 * fenced chains (torch_npu_smollm.py:644-654, torch_intel_npu.py:560-570); its RMSNorm and
 * KV-select steps ran as SHAVE kernels inside that graph
 * (npunlock/tests/fixtures/npu4000/rmsnorm.c, kv_select.c).  These entry points are the
 * pieces of such a layer on the GPU; a caller enqueues them on one stream (and may capture
 * them into a HIP graph -- none of them calls hipMemsetAsync or allocates).
 *
 * Conventions are those of lowbit_hip.h: device pointers, caller-owned buffers,
 * asynchronous stream-ordered calls, lb_status results with lb_last_error().
 * Every activation here is one fp16 row (batch 1, one token).
 */
#ifndef LOWBIT_DECODE_HIP_H
#define LOWBIT_DECODE_HIP_H

#include <stddef.h>
#include <stdint.h>

#include "lowbit_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

#define LB_FUSED_MAX_PROBLEMS 3
#define LB_FUSED_MAX_RANK 32
#define LB_FUSED_MAX_K 1536
#define LB_FUSED_WORKSPACE_BYTES 512

/* lb_fused_linear_args.prologue: what is applied to the activation row before the product */
#define LB_PROLOGUE_NONE 0u     /* x as given */
#define LB_PROLOGUE_RMSNORM 1u  /* fp16(fp16(x * rsqrt(mean(x^2) + eps)) * gamma) (torch_npu_smollm.py:166-168) */
#define LB_PROLOGUE_SILU_MUL 2u /* fp16(fp16(silu(x)) * x2), x = gate row, x2 = up row (torch_npu_smollm.py:188-190) */

typedef struct lb_fused_problem {
  const void *codes;        /* PackedWeight.data bytes, or fp16 [N,K] for LB_FORMAT_FP16; 16-byte aligned */
  const void *scales;       /* fp16 [N, K/group_size] */
  int64_t N;
  void *y;                  /* fp16 [N] */
  const void *bias;         /* fp16 [N] or NULL */
  const void *residual;     /* fp16 [N] or NULL; y = fp16(residual + y) last. May be y itself. */
  int64_t rank;             /* 0..32; 0: no correction */
  const void *down;         /* V fp16 [rank, K], 16-byte aligned */
  const void *up;           /* U fp16 [N, up_ld], 16-byte aligned, up_ld % 8 == 0, up_ld >= rank */
  int64_t up_ld;
} lb_fused_problem;

typedef struct lb_fused_linear_args {
  uint32_t struct_size;     /* sizeof(lb_fused_linear_args) */
  uint32_t format;          /* lb_format, shared by every problem */
  int64_t K;                /* K % 32 == 0, K <= LB_FUSED_MAX_K */
  int64_t group_size;       /* int8: K (per row) or a power of two >= 32; int4/nf4: power of two >= 32 */
  uint32_t prologue;        /* LB_PROLOGUE_* */
  uint32_t count;           /* problems, 1..LB_FUSED_MAX_PROBLEMS */
  const void *x;            /* fp16 [K], 16-byte aligned (SILU_MUL: the gate row) */
  const void *x2;           /* SILU_MUL: the up row fp16 [K] */
  const void *gamma;        /* RMSNORM: fp16 [K] */
  float eps;                /* RMSNORM epsilon */
  uint32_t reserved;
  lb_fused_problem problems[LB_FUSED_MAX_PROBLEMS];
  /* Optional (NULL: every workgroup computes the correction activations z itself).  With a
   * workspace of LB_FUSED_WORKSPACE_BYTES (256-byte aligned, zero before its first use) a call
   * with corrections computes each z = fp16(x'.V^T) once, in workgroups dispatched ahead of the
   * others, which read it after a bounded wait.  A workspace belongs to one call configuration
   * (the same problems and ranks on every call; zero it again before using it for another) and
   * calls sharing it must be ordered (one stream).  Fields absent from a struct whose struct_size
   * ends before them count as NULL / 0. */
  void *workspace;
  size_t workspace_bytes;
} lb_fused_linear_args;

/*
 * For each problem i: y_i = epilogue(x' . dequant(W_i)^T), x' = prologue(x), one launch for
 * all problems.  The epilogue is lb_linear's (scale, fp16, + bias, + fp16(fp16(x'.V^T).U^T))
 * followed by the residual add.  Replaces the per-projection linear() of
 * FrozenSmolLayer.graph with its neighbouring RMSNorm / SiLU-multiply / residual Add
 * (torch_npu_smollm.py:237-259, with the fused RMSNorm of :195-340), for one token.
 * Outputs may not overlap any input except a problem's own residual (same pointer).
 */
lb_status lb_fused_linear(const lb_fused_linear_args *args, void *stream);

typedef struct lb_decode_attention_args {
  uint32_t struct_size;     /* sizeof(lb_decode_attention_args) */
  uint32_t reserved;
  int64_t heads, kv_heads;  /* heads % kv_heads == 0; query head h uses KV head h / (heads / kv_heads) */
  int64_t head_dim;         /* 64 */
  int64_t capacity;         /* KV slots, 1..4096 */
  const void *q;            /* fp16 [heads, 64] new query row (before RoPE) */
  const void *k;            /* fp16 [kv_heads, 64] new key row (before RoPE) */
  const void *v;            /* fp16 [kv_heads, 64] new value row */
  const void *cos, *sin;    /* fp16 [capacity, 64] RoPE tables */
  const int64_t *position;  /* device scalar p: the slot of the new token; outside 0 <= p < capacity the cache is
                               neither read nor written and every element of out is NaN */
  void *keys, *values;      /* fp16 [kv_heads, capacity, 64]; slot p is written */
  void *out;                /* fp16 [heads, 64] */
  float scale;              /* score scale, applied after the fp16 rounding of q.k (0.125 for head_dim 64) */
  uint32_t reserved2;
  /* Optional (NULL: every output workgroup computes the whole score row itself).  With a workspace
   * of LB_ATTN_WORKSPACE_BYTES(heads, capacity) (256-byte aligned, zero before its first use) and
   * heads / kv_heads <= 3, the scores are computed once, by workgroups of 48 cached positions
   * dispatched ahead of the output workgroups, which read them after a bounded wait.  A workspace
   * belongs to one call configuration (same heads and capacity; zero it again before another);
   * calls sharing it must be ordered (one stream).  Fields absent from a struct whose struct_size
   * ends before them count as NULL / 0. */
  void *workspace;
  size_t workspace_bytes;
} lb_decode_attention_args;

/* Workspace of the split attention: tagged score words [heads][ceil(capacity / 48) * 16] (u64),
 * then a launch count (u64) and a timeout word. */
#define LB_ATTN_WORKSPACE_BYTES(heads, capacity) \
  ((size_t)(heads) * (size_t)(((capacity) + 47) / 48) * 128u + 16u)

/*
 * RoPE of q and k at row p, append (k, v) at slot p, causal GQA attention over slots 0..p with
 * the reference staging: scores fp16(q.k) -> fp16(* scale), softmax fp32 -> fp16,
 * out = fp16(P.V) (CPU staging torch_npu_smollm.py:174-182; the device graph's RoPE gather,
 * GQA attention and KV Select, :262-303, :325-329).
 */
lb_status lb_decode_attention(const lb_decode_attention_args *args, void *stream);

/*
 * One decoder layer for one token in one launch: RMSNorm -> q | k | v (+ corrections) -> RoPE, KV
 * append, GQA attention -> o (+ correction) + residual -> RMSNorm -> gate | up (+ corrections) ->
 * SiLU(gate) * up -> down (+ correction) + residual, with the staging of lb_fused_linear and
 * lb_decode_attention.  The counterpart of the reference's one-graph-per-layer decode
 * (torch_npu_smollm.py:195-340, FrozenSmolLayer.graph), replacing the five launches of those
 * entry points with one: each stage runs in workgroups of its own that hand their outputs to the
 * later stages through the workspace (bounded waits), and every workgroup fetches its weights at
 * launch.  Limits: hidden = heads * 64 <= 640, intermediate <= 1536 (multiples of 32),
 * heads / kv_heads <= 3, capacity <= 4096, ranks <= 32, one format and group for all seven
 * projections (group_size 0: int8 per row; otherwise a power of two >= 32 dividing both K).
 */
typedef struct lb_decode_layer_args {
  uint32_t struct_size;        /* sizeof(lb_decode_layer_args) */
  uint32_t format;             /* lb_format of all seven projections */
  int64_t group_size;          /* see above */
  int64_t hidden, intermediate;
  void *h;                     /* fp16 [hidden], 16-byte aligned: the layer input, replaced by its output */
  const void *norm1, *norm2;   /* fp16 [hidden] RMSNorm weights, 16-byte aligned */
  float eps;
  uint32_t reserved;
  lb_fused_problem proj[7];    /* q, k, v, o, gate, up, down: codes, scales, N, rank, down, up, up_ld
                                  (N: hidden, 64 kv_heads, 64 kv_heads, hidden, intermediate,
                                  intermediate, hidden); y, bias and residual must be NULL */
  int64_t heads, kv_heads, capacity;
  const void *cos, *sin;       /* fp16 [capacity, 64] RoPE tables */
  const int64_t *position;     /* device scalar p: the new token's slot (outside 0..capacity-1 the cache is
                                  left alone and the attention output is NaN) */
  void *keys, *values;         /* fp16 [kv_heads, capacity, 64], 16-byte aligned; slot p is written */
  float scale;                 /* attention score scale (0.125) */
  uint32_t reserved2;
  void *workspace;             /* LB_DECODE_LAYER_WORKSPACE_BYTES, 256-byte aligned, zero before its first use;
                                  one per call configuration; calls sharing it must be ordered (one stream) */
  size_t workspace_bytes;
} lb_decode_layer_args;

/* Words of one layer's region of a decode-layer workspace (tagged hand-over words of every stage),
 * and the workspace of one layer: an 8-word header (launch count, timeout word) and one region. */
#define LB_DECODE_LAYER_WORDS(hidden, intermediate, kv_heads)                                              \
  (((size_t)224u + ((size_t)(hidden) + 128u * (size_t)(kv_heads)) / 2u + 3u * (size_t)(hidden) / 2u + \
    (size_t)(intermediate) + 31u) / 32u * 32u)
#define LB_DECODE_LAYER_WORKSPACE_BYTES(hidden, intermediate, kv_heads) \
  ((size_t)8u * (8u + LB_DECODE_LAYER_WORDS(hidden, intermediate, kv_heads)))

lb_status lb_decode_layer(const lb_decode_layer_args *args, void *stream);

/*
 * A whole decoder stack for one token in one launch: the layers of lb_decode_layer one after the
 * other, with the same arithmetic (the output equals `layers` lb_decode_layer calls bit for bit).
 * The counterpart of the reference's per-token chain of layer graphs, submitted in fenced groups
 * (torch_npu_smollm.py:644-654, torch_intel_npu.py:560-570).  Every workgroup keeps its stage
 * through all layers and fetches the next layer's weights while earlier stages run; the grid must
 * be resident on the device all at once (lb_decode_stack returns LB_UNSUPPORTED where the device
 * cannot hold it).  That check is made once, from the kernel's occupancy on the stream's device,
 * at lb_decode_stack_prepare: it cannot see kernels that other streams or processes run on the
 * device at the same time, which can keep part of the grid waiting for compute units.  Its waits
 * then time out (see lb_decode_check), so run the stack without concurrent kernels on the device
 * and check the workspace after use.  All layers share shapes, format, group size and
 * per-projection ranks.
 *
 * lb_decode_stack_prepare validates the arguments and writes the layer table (device addresses of
 * every layer's tensors) into `table`, synchronously on `stream`; it is a set-up call, made once
 * before lb_decode_stack calls (which may be captured into a HIP graph) with the same layers.
 * lb_decode_stack refuses a table that lb_decode_stack_prepare did not write for these layers.
 */
#define LB_DECODE_STACK_MAX_LAYERS 64
#define LB_DECODE_STACK_TABLE_BYTES(layers) ((size_t)(layers) * 256u)
#define LB_DECODE_STACK_WORKSPACE_BYTES(hidden, intermediate, kv_heads, layers) \
  ((size_t)8u * (8u + (size_t)(layers) * LB_DECODE_LAYER_WORDS(hidden, intermediate, kv_heads)))

typedef struct lb_decode_stack_layer {
  const void *norm1, *norm2;   /* fp16 [hidden], 16-byte aligned */
  lb_fused_problem proj[7];    /* as lb_decode_layer_args.proj; rank and up_ld equal in every layer */
  void *keys, *values;         /* fp16 [kv_heads, capacity, 64], 16-byte aligned; slot p is written */
} lb_decode_stack_layer;

typedef struct lb_decode_stack_args {
  uint32_t struct_size;        /* sizeof(lb_decode_stack_args) */
  uint32_t format;             /* lb_format of every projection */
  int64_t group_size;          /* as lb_decode_layer_args.group_size */
  int64_t hidden, intermediate;
  int64_t layers;              /* 1..LB_DECODE_STACK_MAX_LAYERS */
  const lb_decode_stack_layer *layer;  /* host array [layers] */
  void *h;                     /* fp16 [hidden]: the first layer's input, replaced by the last layer's output */
  float eps;
  uint32_t reserved;
  int64_t heads, kv_heads, capacity;
  const void *cos, *sin;       /* fp16 [capacity, 64] RoPE tables */
  const int64_t *position;     /* device scalar p, as lb_decode_layer_args.position */
  float scale;
  uint32_t reserved2;
  void *table;                 /* device, LB_DECODE_STACK_TABLE_BYTES(layers), 256-byte aligned */
  size_t table_bytes;
  void *workspace;             /* LB_DECODE_STACK_WORKSPACE_BYTES, 256-byte aligned, zero before its first use;
                                  one per call configuration; calls sharing it must be ordered (one stream) */
  size_t workspace_bytes;
} lb_decode_stack_args;

lb_status lb_decode_stack_prepare(const lb_decode_stack_args *args, void *stream);
lb_status lb_decode_stack(const lb_decode_stack_args *args, void *stream);

/*
 * Forgets a table written by lb_decode_stack_prepare: a later lb_decode_stack with that table
 * returns LB_INVALID_ARGUMENT until it is prepared again.  Call it before the table's memory is
 * freed, so that a new table allocated at the same address is never taken for the old one.
 * LB_INVALID_ARGUMENT if the table was not prepared.
 */
lb_status lb_decode_stack_release(const void *table);

/*
 * Hand-over health of the calls that use a workspace (lb_fused_linear and lb_decode_attention
 * with a workspace, lb_decode_layer, lb_decode_stack).  Their workgroups hand data to later
 * workgroups of the same launch through tagged words in the workspace, and every wait for such a
 * word is bounded: a wait that gives up sets the workspace's timeout word and the launch goes on
 * with the stale word, so its outputs (and those of every later call on the workspace) are not
 * valid.  A wait gives up only when its producer never ran in time.  The producers are dispatched
 * first and the stacked grid is checked to fit the device at lb_decode_stack_prepare, so this
 * happens only when something else holds the compute units the grid needs -- kernels of other
 * streams or processes running concurrently on the device -- or after a device problem.
 *
 * lb_decode_check synchronises `stream`, then reads the timeout word at byte `timeout_offset` of
 * the workspace (LB_*_TIMEOUT_OFFSET below).  Zero: LB_OK.  Nonzero: the library enters its failed
 * state, as after a launch error (every later call returns LB_DEVICE_FAILED, like the reference's
 * failed context, npunlock-probe/torch-device/backend.cpp:280-292), and the call returns
 * LB_DEVICE_FAILED.  *timeouts (may be NULL) receives the word.  Call it after the calls, or graph
 * replays, whose outputs are about to be used.
 */
#define LB_FUSED_TIMEOUT_OFFSET 392u
#define LB_ATTN_TIMEOUT_OFFSET(heads, capacity) (LB_ATTN_WORKSPACE_BYTES(heads, capacity) - 8u)
#define LB_DECODE_TIMEOUT_OFFSET 8u /* lb_decode_layer and lb_decode_stack workspaces */

lb_status lb_decode_check(const void *workspace, size_t timeout_offset, void *stream, uint32_t *timeouts);

/*
 * Greedy step: t = first index of the largest logit (NaN logits are never chosen);
 * token[0] = t; if 0 <= position[0] < limit: tokens[position[0]] = t and position[0] += 1;
 * h_next = embedding[t] (fp16 [hidden]).  Replaces the host argmax and the next step's embedding
 * lookup of the reference generation loop (torch_npu_smollm_kv_demo.py:229-245,
 * torch_npu_smollm_io.py:45-50).
 */
lb_status lb_argmax_next(const void *logits, int64_t vocab, const void *embedding, int64_t hidden, void *h_next,
                         int64_t *tokens, int64_t *token, int64_t *position, int64_t limit, void *stream);

/* Workspace of lb_head_next for a head of `vocab` rows: room for a 64-bit maximum word and a
 * 64-bit counter per group of 8 workgroups (64 rows each), and one pair for the total (the kernel
 * groups at least 8 workgroups; larger groups use fewer of the words). */
#define LB_HEAD_NEXT_WORKGROUPS(vocab) (((size_t)(vocab) + 63u) / 64u)
#define LB_HEAD_NEXT_WORKSPACE_BYTES(vocab) (16u * ((LB_HEAD_NEXT_WORKGROUPS(vocab) + 7u) / 8u + 1u))

/*
 * Final RMSNorm -> lm_head -> greedy step in one launch: lb_fused_linear(head) followed by
 * lb_argmax_next(head->problems[0].y, vocab = N, embedding, hidden = K, h_next, tokens, token,
 * position, limit), without the second launch: every workgroup reduces its 64 logits to one
 * candidate and the last workgroup to finish picks the token (no workgroup waits for another).
 * The logits are written as lb_fused_linear writes them (the same products and fp32 sums; for
 * heads of fewer than 32768 rows lb_fused_linear may add a row's K slices in another order) and
 * the token is the one lb_argmax_next picks from them.  Replaces the final RMSNorm and tied head
 * (torch_npu_smollm_io.py:52-61) and the host argmax and embedding lookup of the reference
 * generation loop (torch_npu_smollm_kv_demo.py:229-245, torch_npu_smollm_io.py:45-50).
 *   head: one problem (the vocab rows), prologue LB_PROLOGUE_RMSNORM, no correction, bias or
 *         residual; format LB_FORMAT_FP16 with K <= 640 or LB_FORMAT_INT4 (LB_UNSUPPORTED
 *         otherwise: run the two calls).  head->workspace: LB_HEAD_NEXT_WORKSPACE_BYTES(N) bytes,
 *         256-byte aligned, zero before its first use (every call leaves it zero again);
 *         calls sharing it must be ordered (one stream).
 *   h_next may be head->x itself (every workgroup has read x before the token is written).
 */
lb_status lb_head_next(const lb_fused_linear_args *head, const void *embedding, void *h_next, int64_t *tokens,
                       int64_t *token, int64_t *position, int64_t limit, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* LOWBIT_DECODE_HIP_H */
