/*
 * rhizome_gdr.h -- C ABI of the MI355X (gfx950) gated delta-rule library
 * (librhizome_gdr.so).
 *
 * The op, for one head with state S (d_v x d_k, S[i][j] at i*d_k + j,
 * i = value row, j = key column -- the reference layout of
 * crates/ops/src/delta.rs:63):
 *
 *     S_t = alpha_t * S_{t-1} * (I - beta_t k_t k_t^T) + beta_t v_t k_t^T
 *     o_t = S_t q_t
 *
 * Every entry point takes plain pointers and sizes, validates everything it
 * can before touching the GPU, never aborts, and returns an rhz_status.
 * Device pointers are caller-owned device memory; `stream` is a
 * hipStream_t passed as void* (NULL = the default stream).  Launches are
 * asynchronous with respect to the host and stream-ordered.  No entry point
 * allocates device memory: scratch space comes from the caller-provided
 * workspace (size from the matching *_workspace_size query), so the buffers
 * can live at offsets inside a planner arena (crates/plan/src/arena.rs:71,
 * 256-byte aligned).  Results are deterministic (no atomics in any
 * reduction) and batch-invariant: a sequence's outputs do not depend on the
 * other sequences packed with it.
 *
 * Tensor layouts (row-major, dense or packed):
 *   q, k          [tokens, H, d_k]
 *   v, o          [tokens, H, d_v]
 *   gate, beta    [tokens, H]          fp32
 *   states        [seqs, H, d_v, d_k]  fp32
 * Dense batches are the packed layout with tokens = B*T and sequence b at
 * tokens [b*T, (b+1)*T).
 */
#ifndef RHIZOME_GDR_H
#define RHIZOME_GDR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RHZ_GDR_ABI_VERSION 1

/* Status codes.  The Rust wrapper maps INVALID_ARG to
 * rhizome_core::Error::Shape and UNSUPPORTED / WORKSPACE to Error::Invalid
 * (crates/core/src/error.rs:7-28). */
typedef enum rhz_status {
    RHZ_OK = 0,
    RHZ_ERR_INVALID_ARG = 1, /* null pointer, bad dimension or size, bad enum */
    RHZ_ERR_UNSUPPORTED = 2, /* well-formed but not supported (dims, dtype, algo) */
    RHZ_ERR_WORKSPACE = 3,   /* workspace missing, too small or misaligned */
    RHZ_ERR_HIP = 4          /* the HIP runtime reported an error */
} rhz_status;

/* RHZ_F64 is accepted only as the output dtype of rhz_philox_fill. */
typedef enum rhz_dtype { RHZ_F32 = 0, RHZ_BF16 = 1, RHZ_F64 = 2 } rhz_dtype;

/* What `gate` holds: the log-decay g_t = ln(alpha_t) (<= 0), or alpha_t in
 * [0, 1] itself.  alpha_t = 0 forgets the past exactly (delta.rs:348-358). */
typedef enum rhz_gate { RHZ_GATE_LOG_ALPHA = 0, RHZ_GATE_ALPHA = 1 } rhz_gate;

/* Prefill algorithm.  AUTO picks CHUNKED for bf16 and RECURRENT for fp32.
 * RECURRENT: token-sequential fp32 recurrence (the fp32-input path).
 * CHUNKED:   64-token chunks, WY/UT transform on fp16 MFMA with fp32
 *            accumulation and fp32 state (bf16 inputs only, converted to
 *            fp16 on chip).  The state and the corrected values U are
 *            rescaled by powers of two.  The operands formed from q and k
 *            are accurate in the reference's domain (delta.rs:17-20: k
 *            L2-normalised, beta and alpha in [0, 1]; q L2-normalised and
 *            scaled, SPEC.md:53), and the kernel checks it chunk by chunk: a
 *            workgroup that meets a key row with |k|^2 > 1.03125, a beta or
 *            alpha outside [0, 1] or NaN, or an fp16 entry of beta K K^T or
 *            Q K^T (with their decays) that is not finite or of magnitude
 *            65520 or more, recomputes its rows of the state with the fp32
 *            recurrence of RECURRENT inside the same launch.  Every finite
 *            input therefore gets the recurrence's result; such reruns are
 *            slower and are counted by rhz_gdr_exact_reruns.  q elements
 *            below 2^-14 in magnitude are held to 2^-25 absolute (fp16
 *            subnormals).  A log-decay at or below -80 (alpha <= 1.8e-35)
 *            is taken as alpha = 0: the past is forgotten exactly. */
typedef enum rhz_algo { RHZ_ALGO_AUTO = 0, RHZ_ALGO_RECURRENT = 1, RHZ_ALGO_CHUNKED = 2 } rhz_algo;

/* Op identities for rhz_gdr_query_support, named after the plan-level ops
 * OpKind::DeltaScan / OpKind::DeltaStep (crates/plan/src/graph.rs:56-59). */
typedef enum rhz_op {
    RHZ_OP_DELTA_SCAN = 0,     /* "gated_delta_scan_chunked" (graph.rs:124) */
    RHZ_OP_DELTA_STEP = 1,     /* "gated_delta_step" (graph.rs:125) */
    RHZ_OP_DELTA_MULTISTEP = 2 /* gated_delta_multistep (delta.rs:202-230); no plan-level op */
} rhz_op;

/* Prefill over a dense batch or a packed variable-length batch.
 * Replaces, batched over sequences and heads and with a rectangular state,
 * gated_delta_sequential (delta.rs:133-154) and gated_delta_scan_chunked
 * (delta.rs:159-197).  Unlike those two, initial_state is honoured (they
 * reset S at t = 0); pass initial_state = NULL for their behaviour. */
typedef struct rhz_gdr_prefill_args {
    int32_t batch;   /* dense: B;  packed: number of sequences N (>= 1) */
    int32_t seq_len; /* dense: T;  packed: total tokens in the pack (>= 0) */
    int32_t heads;   /* H >= 1 */
    int32_t d_k;     /* 1..256 (RECURRENT), 1..128 (CHUNKED) */
    int32_t d_v;     /* 1..1024 */
    int32_t chunk;   /* requested chunk length >= 1; the result does not depend on it
                        (delta.rs:156-157); CHUNKED computes with 64 */
    int32_t dtype;     /* rhz_dtype of q, k, v and o */
    int32_t gate_kind; /* rhz_gate */
    int32_t algo;      /* rhz_algo */
    const void* q;
    const void* k;
    const void* v;
    const float* gate;
    const float* beta;
    const int32_t* cu_seqlens;  /* device [N+1] non-decreasing token offsets, or NULL for a
                                   dense batch.  Offsets are clamped into [0, seq_len];
                                   decreasing offsets give unspecified (memory-safe)
                                   results. */
    const float* initial_state; /* device [batch, H, d_v, d_k], or NULL for zeros */
    float* final_state;         /* device [batch, H, d_v, d_k], or NULL; may equal
                                   initial_state (the state is then updated in place) */
    void* o;                    /* device [tokens, H, d_v], dtype */
    void* workspace;            /* device scratch, 256-byte aligned */
    size_t workspace_bytes;
} rhz_gdr_prefill_args;

/* One decode position for every (b, h), state updated in place.
 * Replaces gated_delta_step (delta.rs:94-127), batched. */
typedef struct rhz_gdr_decode_args {
    int32_t batch;     /* B >= 1 */
    int32_t heads;     /* H >= 1 */
    int32_t d_k;       /* 1..256 */
    int32_t d_v;       /* 1..1024 */
    int32_t dtype;     /* rhz_dtype of q, k, v and o */
    int32_t gate_kind; /* rhz_gate */
    const void* q;     /* [B, H, d_k] */
    const void* k;     /* [B, H, d_k] */
    const void* v;     /* [B, H, d_v] */
    const float* gate; /* [B, H] */
    const float* beta; /* [B, H] */
    float* state;      /* [B, H, d_v, d_k] fp32, read and written in place */
    void* o;           /* [B, H, d_v] */
} rhz_gdr_decode_args;

/* Up to `steps` consecutive positions for every (b, h) from a given state,
 * returning o and the state after every position (speculative decoding:
 * the snapshot of the last accepted position becomes the new state).
 * Replaces gated_delta_multistep (delta.rs:202-230), batched.  Unlike it,
 * the given state is honoured (the reference resets S at t = 0: pass zeros
 * for its behaviour); a segment change inside the window is a gate of
 * alpha = 0 at that position (RHZ_GATE_ALPHA), which forgets the past
 * exactly as the reference's reset does.  `state` is read only. */
typedef struct rhz_gdr_multistep_args {
    int32_t batch;     /* B >= 1 */
    int32_t steps;     /* positions n, 1..RHZ_MULTISTEP_MAX */
    int32_t heads;     /* H >= 1 */
    int32_t d_k;       /* 1..256 */
    int32_t d_v;       /* 1..1024 */
    int32_t dtype;     /* rhz_dtype of q, k, v and o */
    int32_t gate_kind; /* rhz_gate */
    const void* q;      /* [B, n, H, d_k] */
    const void* k;      /* [B, n, H, d_k] */
    const void* v;      /* [B, n, H, d_v] */
    const float* gate;  /* [B, n, H] */
    const float* beta;  /* [B, n, H] */
    const float* state; /* [B, H, d_v, d_k] fp32, the state before position 0 */
    float* states;      /* [B, n, H, d_v, d_k] fp32 out: the state after each position */
    void* o;            /* [B, n, H, d_v] */
} rhz_gdr_multistep_args;

#define RHZ_MULTISTEP_MAX 64

/* Library identity. */
int32_t rhz_gdr_abi_version(void);

/* Human-readable name of a status code (static storage). */
const char* rhz_status_string(int32_t status);

/* Detail of the last non-OK status returned on the calling thread
 * (thread-local storage, valid until the next call on that thread). */
const char* rhz_last_error(void);

/* Plan-time capability check (R4, SPEC.md:28-30): RHZ_OK when (op, dtype,
 * d_k, d_v, algo) is supported, RHZ_ERR_UNSUPPORTED otherwise, and
 * RHZ_ERR_INVALID_ARG for out-of-range enums or dimensions. */
rhz_status rhz_gdr_query_support(int32_t op, int32_t dtype, int32_t d_k, int32_t d_v,
                                 int32_t algo);

/* Bytes of device workspace rhz_gdr_prefill needs for these arguments
 * (pointers are not read).  0 when none is needed. */
rhz_status rhz_gdr_prefill_workspace_size(const rhz_gdr_prefill_args* args, size_t* bytes);

/* Gated delta-rule prefill (see rhz_gdr_prefill_args). */
rhz_status rhz_gdr_prefill(const rhz_gdr_prefill_args* args, void* stream);

/* rhz_gdr_prefill for callers that cannot allocate device memory: code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  It has no counterpart in the reference.  Same arguments,
 * validation and results as rhz_gdr_prefill, except that `workspace` and
 * `workspace_bytes` are ignored: the only scratch of the prefill (a packed
 * batch's sequence order, 4 bytes per sequence) lives in a static device
 * array of RHZ_NOALLOC_MAX_SEQS entries (256 KiB) that each GPU the library
 * runs on holds until the process ends.  A packed batch of more than
 * RHZ_NOALLOC_MAX_SEQS sequences is rejected with RHZ_ERR_UNSUPPORTED.  The
 * first call on a device looks up that device's copy of the array; no call
 * allocates.  Every call on one GPU shares the array: calls that overlap on
 * one GPU (on different streams, or from threads without ordering) race on
 * it and must be serialised by the caller; a race gives wrong results, not
 * accesses outside the caller's buffers. */
#define RHZ_NOALLOC_MAX_SEQS 65536

rhz_status rhz_gdr_prefill_noalloc(const rhz_gdr_prefill_args* args, void* stream);

/* Diagnostics of the CHUNKED prefill kernel (no counterpart in the
 * reference, whose op is a CPU loop).  The kernel's waves synchronise through
 * LDS counters with bounded waits; a wait that gives up lets the kernel end
 * and is counted on the device.  Blocking: it first waits for all of the
 * current device's outstanding work, on every stream (hipDeviceSynchronize),
 * then writes the device's count to *count and, when reset is nonzero, sets
 * it to zero in the same atomic exchange on the device, so that a count added
 * by a kernel launched meanwhile from another thread is kept for the next
 * read, never lost.  A nonzero count means that some chunked launch since the
 * last reset may have produced wrong results. */
rhz_status rhz_gdr_sync_timeouts(uint32_t* count, int32_t reset);

/* Diagnostics of the fused-prologue chunked kernel, rhz_gdr_local_prefill
 * (no counterpart in the reference, whose op computes in f32 throughout):
 * the number of (workgroup, wave) pairs, counted once per launch, since the
 * last reset whose fp16 MFMA operands formed from q and k on chip -- the
 * blocks of beta K K^T and Q K^T with their decays -- held a NaN, an
 * infinity or a value of magnitude 65520 or more in any chunk.  Its q and k
 * rows are normalised on chip and |q_scale| <= 2^15, so only non-finite
 * projections do that; a nonzero count means that some such launch since
 * the last reset may have produced wrong results.  The plain CHUNKED path
 * recomputes such workgroups exactly instead (rhz_gdr_exact_reruns) and
 * adds nothing here.  Same calling convention as rhz_gdr_sync_timeouts. */
rhz_status rhz_gdr_fp16_range_errors(uint32_t* count, int32_t reset);

/* Diagnostics of the CHUNKED prefill kernel (no counterpart in the
 * reference): the number of workgroups -- one per 32 state rows of a
 * (sequence, head) -- since the last reset whose inputs left the domain of
 * the fp16 operands (see rhz_algo) and which recomputed their rows with the
 * fp32 recurrence in the same launch.  Their results are the recurrence's;
 * a nonzero count only means those launches ran slower.  Same calling
 * convention as rhz_gdr_sync_timeouts. */
rhz_status rhz_gdr_exact_reruns(uint32_t* count, int32_t reset);

/* Test hook (no counterpart in the reference): rhz_gdr_prefill with the
 * CHUNKED kernel's waits bounded at spin_limit polls (>= 1) instead of the
 * built-in 2^20, so that a test can force give-ups and see them counted by
 * rhz_gdr_sync_timeouts.  Same arguments and validation as rhz_gdr_prefill;
 * the results of a call whose waits gave up are unspecified but every access
 * stays inside the caller's buffers. */
rhz_status rhz_gdr_prefill_spin_limit(const rhz_gdr_prefill_args* args, int32_t spin_limit,
                                      void* stream);

/* Gated delta-rule decode step (see rhz_gdr_decode_args). */
rhz_status rhz_gdr_decode_step(const rhz_gdr_decode_args* args, void* stream);

/* Gated delta-rule multistep (see rhz_gdr_multistep_args). */
rhz_status rhz_gdr_multistep(const rhz_gdr_multistep_args* args, void* stream);

/* ---- Local-block prologue and epilogue around the op (SPEC.md:53-63) ---- */

/* Causal depthwise conv1d of width 4 over packed or dense sequences, with a
 * 3-sample carried state per (sequence, channel).  Per channel, the reference
 * step (causal_conv1d_step, delta.rs:232-243) applied along each sequence:
 *     y_t = w[0] x_{t-3} + w[1] x_{t-2} + w[2] x_{t-1} + w[3] x_t + bias
 * where x before the sequence start comes from initial_state (oldest first)
 * or is zero; final_state receives the last three inputs (the state after the
 * last step).  A sequence start resets the conv state as SPEC.md:61-63 asks. */
typedef struct rhz_conv1d_args {
    int32_t batch;    /* dense: B;  packed: number of sequences N (>= 1) */
    int32_t seq_len;  /* dense: T;  packed: total tokens (>= 0) */
    int32_t channels; /* C >= 1 */
    int32_t dtype;    /* rhz_dtype of x and y (RHZ_F32 or RHZ_BF16) */
    const void* x;              /* [tokens, C] */
    const float* weight;        /* [C, 4] */
    const float* bias;          /* [C], or NULL for zero */
    const int32_t* cu_seqlens;  /* [N+1] or NULL (dense) */
    const float* initial_state; /* [batch, C, 3] oldest first, or NULL for zeros */
    float* final_state;         /* [batch, C, 3], or NULL */
    void* y;                    /* [tokens, C], dtype; must not overlap x */
} rhz_conv1d_args;

rhz_status rhz_causal_conv1d(const rhz_conv1d_args* args, void* stream);

/* The op's inputs from the projections (SPEC.md:53-56), per (token, head):
 *     q := l2norm(q) * q_scale,  k := l2norm(k)       (elementwise.rs:125-128)
 *     beta := sigmoid(beta_logit)                     (elementwise.rs:5-12)
 *     g := -softplus(a_log[h]) * softplus(alpha_logit), alpha = exp(g)
 *                                                     (elementwise.rs:36-42)
 * q_out / k_out may alias q_in / k_in.  g is the log-decay that
 * rhz_gdr_prefill / rhz_gdr_decode_step take with RHZ_GATE_LOG_ALPHA. */
typedef struct rhz_gdr_prepare_args {
    int32_t tokens;   /* >= 0 */
    int32_t heads;    /* H >= 1 */
    int32_t d_k;      /* 1..256 */
    int32_t dtype;    /* rhz_dtype of q and k, in and out */
    float q_scale;    /* SPEC.md:53: sqrt(d_k); must be finite */
    const void* q_in;          /* [tokens, H, d_k] */
    const void* k_in;          /* [tokens, H, d_k] */
    void* q_out;               /* [tokens, H, d_k] */
    void* k_out;               /* [tokens, H, d_k] */
    const float* beta_logit;   /* [tokens, H] */
    const float* alpha_logit;  /* [tokens, H] */
    const float* a_log;        /* [H] */
    float* beta;               /* [tokens, H] out */
    float* g;                  /* [tokens, H] out */
} rhz_gdr_prepare_args;

rhz_status rhz_gdr_prepare(const rhz_gdr_prepare_args* args, void* stream);

/* rhz_gdr_prepare fused into the CHUNKED prefill: the Local block's mixer
 * from its projections (SPEC.md:53-56).  `prefill` is as for
 * rhz_gdr_prefill except that q and k are the raw projections, its gate and
 * beta are not read (the logits below replace them) and its gate_kind is
 * ignored.  As the kernel stages each 64-token chunk it applies prepare's
 * maps -- q := l2norm(q) * q_scale, k := l2norm(k),
 * beta := sigmoid(beta_logit), g := -softplus(a_log[h]) softplus(alpha_logit)
 * (elementwise.rs:5-12, 36-42, 125-128) -- in fp32, without prepare's
 * rounding of q and k to bf16, so the prepared q, k, beta and g never go
 * through HBM.  The result is rhz_gdr_prepare followed by rhz_gdr_prefill up
 * to that rounding.  bf16 and the CHUNKED algorithm only (AUTO resolves to
 * it; anything else is RHZ_ERR_UNSUPPORTED); the workspace is the one
 * rhz_gdr_prefill_workspace_size reports for `prefill`.  Because q and k
 * are normalised on chip, every fp16 operand the kernel forms from them is
 * bounded by |q_scale|, which must be at most 2^15 (else
 * RHZ_ERR_UNSUPPORTED): any finite projections are in range.  No
 * counterpart in the reference, whose steps run one after the other on the
 * CPU. */
typedef struct rhz_gdr_local_args {
    rhz_gdr_prefill_args prefill;
    float q_scale;             /* SPEC.md:53: sqrt(d_k); must be finite */
    const float* beta_logit;   /* [tokens, H] */
    const float* alpha_logit;  /* [tokens, H] */
    const float* a_log;        /* [H] */
} rhz_gdr_local_args;

rhz_status rhz_gdr_local_prefill(const rhz_gdr_local_args* args, void* stream);

/* The Local block's prologue in one HBM pass (SPEC.md:53-56): the causal
 * depthwise conv1d of rhz_causal_conv1d (causal_conv1d_step,
 * delta.rs:232-243; width 4, 3-sample carried state, reset at sequence
 * starts) over x = the q, k and v projections side by side, C = heads *
 * (2 d_k + d_v) channels per token (channels [0, H d_k) are q, then k, then
 * v), followed before any rounding by rhz_gdr_prepare's maps: every q row
 * l2-normalised and multiplied by q_scale, every k row l2-normalised
 * (elementwise.rs:125-128), v passed on, beta = sigmoid(beta_logit) and
 * g = -softplus(a_log[h]) softplus(alpha_logit) (elementwise.rs:5-12,
 * 36-42).  The outputs are what rhz_gdr_prefill takes with
 * RHZ_GATE_LOG_ALPHA; they equal rhz_causal_conv1d followed by
 * rhz_gdr_prepare up to the rounding of the convolved q and k to dtype,
 * which this pass skips.  bf16 or fp32; d_k and d_v multiples of 8 (bf16)
 * or 4 (fp32) with d_k / 8 (bf16) or d_k / 4 (fp32) a power of two up to 64
 * (else RHZ_ERR_UNSUPPORTED: use the two calls); x and the q, k, v outputs
 * 16-byte aligned and not overlapping.  No counterpart in the reference,
 * whose steps run one after the other on the CPU. */
typedef struct rhz_gdr_conv_prepare_args {
    int32_t batch;    /* dense: B;  packed: number of sequences N (>= 1) */
    int32_t seq_len;  /* dense: T;  packed: total tokens (>= 0) */
    int32_t heads;    /* H >= 1 */
    int32_t d_k;      /* >= 1 */
    int32_t d_v;      /* >= 1 */
    int32_t dtype;    /* rhz_dtype of x and of the q, k, v outputs */
    float q_scale;    /* SPEC.md:53: sqrt(d_k); must be finite */
    const void* x;              /* [tokens, C] projections, C = H (2 d_k + d_v) */
    const float* weight;        /* [C, 4] */
    const float* bias;          /* [C], or NULL for zero */
    const int32_t* cu_seqlens;  /* [N+1] or NULL (dense) */
    const float* initial_state; /* [batch, C, 3] conv state, oldest first, or NULL */
    float* final_state;         /* [batch, C, 3], or NULL */
    const float* beta_logit;    /* [tokens, H] */
    const float* alpha_logit;   /* [tokens, H] */
    const float* a_log;         /* [H] */
    void* q;                    /* [tokens, H, d_k] out */
    void* k;                    /* [tokens, H, d_k] out */
    void* v;                    /* [tokens, H, d_v] out */
    float* beta;                /* [tokens, H] out */
    float* g;                   /* [tokens, H] out */
} rhz_gdr_conv_prepare_args;

rhz_status rhz_gdr_conv_prepare(const rhz_gdr_conv_prepare_args* args, void* stream);

/* RMSNorm of every row of `dim` values with a learned scale, as the
 * per-head norm of the op's output (groupnorm_heads / rmsnorm,
 * norm.rs:8-13, 48-59): y = x / sqrt(mean(x^2) + eps) * scale.  y may alias
 * x. */
typedef struct rhz_rmsnorm_args {
    int32_t rows;     /* tokens * heads, >= 0 */
    int32_t dim;      /* 1..1024 */
    int32_t dtype;    /* rhz_dtype of x and y */
    float eps;        /* norm.rs:4: 1e-6 */
    const void* x;        /* [rows, dim] */
    const float* scale;   /* [dim] */
    void* y;              /* [rows, dim] */
} rhz_rmsnorm_args;

rhz_status rhz_rmsnorm_heads(const rhz_rmsnorm_args* args, void* stream);

/* Seeded synthetic inputs on the device, from the reference's Philox-4x32-10
 * (crates/ops/src/rng.rs:43-90; elementwise.rs:5-12, 36-42, 125-128).
 * Element e of the output takes normal #e of stream (seed, stream_id): the
 * Box-Muller pair of Philox block e, computed in f64.  Per kind:
 *   RHZ_FILL_NORMAL            mean + std * z
 *   RHZ_FILL_UNIT_ROWS         z, L2-normalised over every run of row_len values
 *                              (mean and std_dev unused; count % row_len == 0)
 *   RHZ_FILL_SIGMOID           sigmoid(mean + std * z)
 *   RHZ_FILL_NEG_SOFTPLUS      -softplus(mean + std * z)
 *   RHZ_FILL_UNIFORM           u = next_f64 #e of the stream (rng.rs:78-82:
 *                              words 2e and 2e + 1), in [0, 1); mean and
 *                              std_dev unused
 * then rounded (f64 -> f32 -> bf16, round to nearest even) to out_dtype
 * (RHZ_F64, RHZ_F32 or RHZ_BF16). */
typedef enum rhz_fill_kind {
    RHZ_FILL_NORMAL = 0,
    RHZ_FILL_UNIT_ROWS = 1,
    RHZ_FILL_SIGMOID = 2,
    RHZ_FILL_NEG_SOFTPLUS = 3,
    RHZ_FILL_UNIFORM = 4
} rhz_fill_kind;

rhz_status rhz_philox_fill(int32_t kind, uint64_t seed, uint64_t stream_id, int64_t count,
                           int32_t row_len, double mean, double std_dev, int32_t out_dtype,
                           void* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RHIZOME_GDR_H */
