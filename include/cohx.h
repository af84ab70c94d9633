/*
 * cohx — MI355X (gfx950) continuous-batching forward step for the Coheryn
 * engine's Qwen2 graph, as a C ABI.
 *
 * Two layers:
 *  1. The device step (cohx_create .. cohx_step): HBM-resident weights, a paged
 *     KV pool, and one call that advances a ragged batch of lanes.  This is what
 *     an `extern "C"` FFI crate binds in place of the engine's CPU kernels
 *     (crates/coheryn-engine/src/inference/batch.rs:117-273 forward_batch,
 *     tensor.rs:302-436 matmul_batch_cooperative, cpu.rs:49-210, quant.rs:175-349).
 *  2. The host mirror of the engine's generation API (cohx_gen_*, cohx_step_batch):
 *     the same state machine as inference/generation.rs:18-394 and the
 *     `BatchModel::step` contract of crates/coheryn-api/src/scheduler/batching.rs:11-21,
 *     so a scheduler written against the reference drives the GPU step unchanged.
 *
 * Every entry point returns a status code (no exceptions cross the ABI) and is
 * single-threaded per context: the caller serializes calls on one context, as
 * the reference scheduler does with its single compute permit
 * (crates/coheryn-api/src/scheduler.rs:201).  Pointers are borrowed for the
 * duration of the call only.
 */
#ifndef COHX_H
#define COHX_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes; classes of crates/coheryn-engine/src/error.rs:6-41. */
enum {
  COHX_OK = 0,
  COHX_INVALID_REQUEST = 1, /* Error::request (bad token, bad batch, bad handle) */
  COHX_INVALID_GGUF = 2,    /* Error::invalid (shapes, non-finite values) */
  COHX_RESOURCE = 3,        /* Error::resource (context / KV pool exhausted) */
  COHX_CANCELLED = 4,       /* ErrorCode::Cancelled */
  COHX_UNSUPPORTED = 5,     /* unsupported dtype / feature */
  COHX_DEAD_END = 6,        /* ErrorCode::ConstraintDeadEnd (empty sampling mask) */
  COHX_DEVICE = 7           /* HIP runtime failure */
};

/* GGML dtypes (gguf.rs:104-128; quant.rs:7-12; BF16 for Qwen3.5).  Qwen2
 * matrices may be F16, Q4_0, Q5_0, Q8_0, Q4_K or Q6_K; vectors are F32. */
enum { COHX_F32 = 0, COHX_F16 = 1, COHX_Q4_0 = 2, COHX_Q5_0 = 6, COHX_Q8_0 = 8, COHX_Q4_K = 12,
       COHX_Q6_K = 14, COHX_BF16 = 30 };
/* cohx_model_desc.weight_dtype for files whose matrices differ in dtype (the
 * engine binds mixed-type files through one graph, docs/QUANTIZATION.md;
 * e.g. a Q4_K_M file holds Q5_0, Q8_0, Q4_K and Q6_K matrices): each matrix
 * takes the dtype of its uploaded tensor.  The parts of a fused matrix
 * (q/k/v, gate/up) must then agree in family: Q8_0 with Q5_0, Q4_K with
 * Q6_K, Q4_0 alone, F16 alone. */
#define COHX_MIXED 0x100u

typedef struct cohx_ctx cohx_ctx;

/* Model and capacity description; the first ten fields are compat.rs:12-23
 * ModelConfig. */
typedef struct {
  uint32_t layers, hidden, intermediate, heads, kv_heads, head_dim, vocabulary, context;
  float rope_base, norm_epsilon;
  uint32_t weight_dtype; /* dtype of every 2-D matrix (COHX_F16, COHX_Q4_0, COHX_Q5_0,
                          * COHX_Q8_0, COHX_Q4_K, COHX_Q6_K), or COHX_MIXED */
  uint32_t tied;         /* 1: logits use token_embd.weight (batch.rs:261-265) */
  uint32_t kv_dtype;     /* 0: f32 KV cache (the engine's, README.md:78) */
  uint32_t max_lanes;    /* lanes per step */
  uint32_t max_rows;     /* packed token rows per step (sum of lane n_tokens) */
  uint32_t max_seqs;     /* live sequences */
  uint32_t max_context;  /* tokens per sequence (<= context) */
  uint32_t kv_pages;     /* KV pool size in pages of COHX_PAGE tokens (0: max_seqs*max_context) */
  uint32_t n_eog;        /* end-of-generation ids (tokenizer.rs:224-236,304-306) */
  uint32_t eog[4];
} cohx_model_desc;

#define COHX_PAGE 16

/* Model::load counterpart (inference.rs:238-297): allocates HBM for weights,
 * the KV pool and per-step workspaces on `device`. */
int cohx_create(const cohx_model_desc *desc, int device, cohx_ctx **out);
void cohx_destroy(cohx_ctx *ctx);
/* Human-readable text of the last failure on this context. */
const char *cohx_last_error(const cohx_ctx *ctx);

/* Model::load from a GGUF file (inference.rs:238-297): the engine's bounded
 * v3 header parser (gguf.rs:304-496), its Qwen2 configuration and graph
 * checks (compat.rs:54-221) and end-of-generation ids (eos, eot and
 * "<|endoftext|>", tokenizer.rs:224-236,304-306), then cohx_create,
 * cohx_upload_tensor of every tensor from a read-only mapping of the file, and
 * cohx_finalize.  desc: in, the capacities (max_lanes, max_rows, max_seqs,
 * max_context, kv_pages; 0 takes 16 lanes, rows = lanes, seqs = lanes,
 * max_context = min(context, 4096)); out, the file's configuration,
 * weight_dtype (one dtype or COHX_MIXED), tied flag and EOG ids.  err (may be
 * NULL) receives the failure's text.  Malformed files fail with
 * COHX_INVALID_GGUF, unsupported ones with COHX_UNSUPPORTED, as the engine
 * classifies them. */
int cohx_load_gguf(const char *path, int device, cohx_model_desc *desc, cohx_ctx **out, char *err,
                   size_t err_cap);
/* The parsing and validation of cohx_load_gguf alone (no device work):
 * fills desc as cohx_load_gguf would. */
int cohx_gguf_inspect(const char *path, cohx_model_desc *desc, char *err, size_t err_cap);

/* Upload one GGUF tensor by name, payload in the file's block layout
 * (gguf.rs:96-103 Tensor; the library repacks into its HBM layout).
 * Names are the engine's (compat.rs:161-221). */
int cohx_upload_tensor(cohx_ctx *ctx, const char *name, uint32_t dtype, uint64_t ne0,
                       uint64_t ne1, const void *data, size_t bytes);
/* Checks that the exact Qwen2 tensor set is present (compat.rs:161-221 graph). */
int cohx_finalize(cohx_ctx *ctx);

/* Sequences: a KV slot map (page table) per session (inference.rs:1019-1055 Kv/Session). */
int cohx_seq_alloc(cohx_ctx *ctx, uint32_t capacity, uint32_t *seq);
/* New sequence sharing `src`'s first `rows` tokens of KV (full pages are shared,
 * a partial last page is copied): the GPU form of prefix reuse
 * (generation.rs:189-202, PrefixCache inference.rs:687-710). */
int cohx_seq_fork(cohx_ctx *ctx, uint32_t src, uint32_t rows, uint32_t capacity, uint32_t *seq);
int cohx_seq_free(cohx_ctx *ctx, uint32_t seq);
int cohx_seq_truncate(cohx_ctx *ctx, uint32_t seq, uint32_t rows);
int cohx_seq_length(const cohx_ctx *ctx, uint32_t seq, uint32_t *rows);
/* The sequence's slot map: physical page of each logical page (-1: none).
 * Returns the number of logical pages (copies at most cap). */
uint32_t cohx_seq_pages(const cohx_ctx *ctx, uint32_t seq, int32_t *out, uint32_t cap);
/* Copy one layer's K (values=0) or V (values=1) rows [0, length) to host,
 * kv_heads*head_dim floats per row. */
int cohx_seq_read_kv(cohx_ctx *ctx, uint32_t seq, uint32_t layer, int values, float *out);
/* The same for rows [first, first + count) only (first + count <= length);
 * copies just the pages those rows occupy.  Test utility; the engine keeps
 * its KV rows in host memory (inference.rs:1019-1043). */
int cohx_seq_read_kv_rows(cohx_ctx *ctx, uint32_t seq, uint32_t layer, int values, uint32_t first,
                          uint32_t count, float *out);
/* Benchmark/test utility with no engine counterpart: fill rows [length, rows)
 * of every layer with seeded values hash(seed, stream, layer, K/V, pos, elem)
 * on the device and set the length to `rows` (rows >= length; on a fresh
 * sequence that is rows [0, rows)).  Appending after a fork leaves the
 * shared prefix pages untouched. */
int cohx_seq_fill_synthetic(cohx_ctx *ctx, uint32_t seq, uint32_t rows, uint64_t seed,
                            uint32_t stream);

/* One lane of a ragged step: n_tokens >= 1 consecutive tokens of one sequence
 * starting at its current length (a decode row or a prefill chunk).
 * start_position must equal that length (the engine's session position,
 * generation.rs:279-317) or be COHX_AT_END, which stands for it. */
#define COHX_AT_END 0xFFFFFFFFu
typedef struct {
  uint32_t seq;
  uint32_t n_tokens;
  const uint32_t *tokens;
  uint32_t start_position;
  uint32_t want_logits; /* 1: copy the last row's logits to cohx_lane_out.logits;
                         * COHX_SKIP_HEAD: see below; 0: argmax only */
} cohx_lane;
/* want_logits value for a lane whose rows only advance its state: no final
 * norm, head or argmax (cohx_lane_out.argmax reads COHX_NO_TOKEN).  Honoured
 * by Qwen3.5 contexts, whose engine computes the head only where
 * cursor + 1 >= len (qwen35/generation.rs:368, execution.rs:586-594);
 * Qwen2 contexts compute the head for every lane (batch.rs:250-266) and treat
 * it as 0. */
#define COHX_SKIP_HEAD 2u
#define COHX_NO_TOKEN 0xFFFFFFFFu

typedef struct {
  uint32_t n_lanes;
  const cohx_lane *lanes;
} cohx_batch;

typedef struct {
  int32_t status;  /* COHX_OK or the lane's own failure (batch.rs:16-29) */
  uint32_t argmax; /* greedy token of the last row, lowest id on ties (sampling.rs:160-173) */
  float *logits;   /* optional caller buffer of `vocabulary` floats, or NULL */
} cohx_lane_out;

typedef struct {
  cohx_lane_out *lanes; /* n_lanes entries */
  uint32_t width;       /* lanes without error (batch.rs:94-97) */
  uint32_t rows;        /* packed token rows */
  uint64_t matrix_bytes;/* weight bytes streamed (BatchStep::matrix_bytes, batch.rs:3-9) */
  uint64_t kv_bytes;    /* KV bytes read + written */
  uint64_t elapsed_ns;
} cohx_step_out;

/* Model::forward_batch counterpart (batch.rs:117-273) over a ragged batch.
 * Shared failures return non-zero; lane failures are reported per lane and
 * never perturb other lanes.  A lane's sequence advances by n_tokens on
 * success. */
int cohx_step(cohx_ctx *ctx, const cohx_batch *batch, cohx_step_out *out);

/* Cooperation with the caller's scheduler during a step (no counterpart
 * needed on a GPU otherwise, since the host only waits while the device
 * computes):
 *  - yield: the engine's WorkYield (multimodal.rs:6; the Qwen3.5 step calls
 *    it between layers, qwen35/execution.rs:306-309, and the scheduler uses it
 *    to release and re-acquire its compute permit, scheduler/batching.rs:
 *    229-239).  Here it is called while the device computes the step, between
 *    polls of the step's completion, so the caller can hand its permit to
 *    other work; it may block.  A non-zero return is the Err of WorkYield
 *    (shared cancellation, shutdown): the call waits for the device, then
 *    fails with COHX_CANCELLED and no lane advances.
 *  - cancel: n_lanes flags (may be NULL), the lanes' Cancellation tokens
 *    (inference.rs:32-68, checked between layers and row tiles,
 *    tensor.rs:361-367).  A lane whose flag is set before the launch is left
 *    out with COHX_CANCELLED (its peers are not perturbed); a Qwen2 lane whose
 *    flag is set by the time the device finishes also reports COHX_CANCELLED
 *    and its sequence does not advance.  A Qwen3.5 step that completed stands
 *    (its recurrent state cannot be rewound); the flag is seen by the next
 *    step. */
typedef struct {
  int (*yield)(void *user);
  void *user;
  const volatile uint32_t *cancel;
} cohx_step_hooks;
/* cohx_step with hooks (NULL: exactly cohx_step). */
int cohx_step_hooked(cohx_ctx *ctx, const cohx_batch *batch, cohx_step_out *out,
                     const cohx_step_hooks *hooks);

/* cohx_step without any device allocation, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference, whose step allocates nothing
 * on a device.  Same inputs, outputs and bits as cohx_step; the step's
 * device scratch (activations, attention partials, argmax keys, the staging
 * of requested logits) comes from one static 64 MiB array per device instead
 * of the context's workspace, and launches are issued directly (no graph).
 * A batch whose scratch would exceed 64 MiB fails with COHX_RESOURCE.  Every
 * call on a device shares that device's array: calls that overlap on one
 * device (from several threads or contexts) race and must be serialized by
 * the caller. */
int cohx_step_noalloc(cohx_ctx *ctx, const cohx_batch *batch, cohx_step_out *out);

/* Packing only (test hook for the bit-exact packer): runs the device packer for
 * `batch` and copies cu_seqlens[n+1], positions[R], slots[R] (page*16 + offset)
 * and lanes[R] back.  Sequences are not advanced. */
int cohx_pack(cohx_ctx *ctx, const cohx_batch *batch, uint32_t *cu_seqlens, uint32_t *positions,
              int64_t *slots, uint32_t *lanes);

/* One matrix on its own (test utility with no engine counterpart, like
 * cohx_pack): `rows` GGUF rows of width K in `dtype` (F16, Q4_0, Q5_0, Q8_0,
 * Q4_K, Q6_K) against n f32 input vectors, through the step's own operand
 * preparation (QuantizedInput::prepare, quant.rs:175-240; binary16 rounding
 * for F16, cpu.rs:37-48) and exact matvec kernels (quant.rs:245-349 dot):
 * out[i*rows + r] = dot(row r, input i).  Optional outputs: act_bytes gets
 * each prepared input in the engine's byte form (Q8_0 34 B per 32 values,
 * Q8_K 292 B per 256, F16 2 B per value), decoded gets the rows as the
 * embedding lookup decodes them (rows*K floats, quant.rs:67-137), status[i]
 * the input's status (COHX_INVALID_GGUF for a non-finite input, scale or
 * result).  Device memory is allocated for the call and released. */
int cohx_matvec(cohx_ctx *ctx, uint32_t dtype, uint32_t rows, uint32_t K, const void *weights, size_t bytes,
                uint32_t n, const float *inputs, float *out, uint8_t *act_bytes, float *decoded,
                int32_t *status);

/* Opt-in per-kernel timing of cohx_step (no engine counterpart; the engine
 * reports only BatchStep byte counts, batch.rs:3-9).  enable=1 clears the
 * counters and starts timing every launch on the context's stream with start
 * and stop events carried in the launches' own dispatch packets (kernel
 * execution time; each timed launch costs a few microseconds more to issue);
 * enable=0 stops.  Each record names a kernel and gives its launches,
 * summed device time and summed algorithmic bytes / flops (the minimum traffic
 * and arithmetic of the operation, independent of how the kernel achieves it). */
typedef struct {
  const char *name;
  uint64_t launches;
  double total_ms;
  double bytes;
  double flops;
} cohx_kernel_stat;
int cohx_profile(cohx_ctx *ctx, int enable);
uint32_t cohx_profile_read(const cohx_ctx *ctx, cohx_kernel_stat *out, uint32_t cap);

/* ---- Qwen3.5 hybrid text model ------------------------------------------- */

/* qwen35/config.rs:6-25 Config plus capacities.  Linear-attention layers carry
 * a causal-conv ring and a gated delta-rule memory per sequence; full-attention
 * layers carry K/V rows. */
typedef struct {
  uint32_t layers, hidden, intermediate, vocabulary;
  uint32_t heads, kv_heads, head_dim; /* full-attention layers */
  uint32_t linear_key_heads, linear_value_heads, linear_key_dim, linear_value_dim;
  uint32_t conv_kernel, rotary_dim, context, tied;
  float epsilon, rope_base;
  uint8_t full_attention[128]; /* layer_types: 1 full_attention, 0 linear_attention */
  uint32_t max_lanes, max_rows, max_seqs, max_context;
  uint32_t n_eog, eog[4];
} cohx_qwen35_desc;

/* qwen35::Model::load counterpart (qwen35/mod.rs:103-193, execution.rs:168-219):
 * HBM for the weights, the per-sequence recurrent state and K/V rows
 * (max_context at most 4096 rows per sequence).  The context then takes:
 *   cohx_upload_tensor: the safetensors tensor set of config.rs:193-309 by name;
 *     matrices BF16 (COHX_BF16), vectors F32 or BF16; conv1d.weight [C][1][K]
 *     as ne0 = K, ne1 = C;
 *   cohx_finalize; cohx_seq_alloc / free / length;
 *   cohx_seq_fork: a full snapshot copy at the source's length (recurrent state
 *     cannot be shared; execution.rs:117-133);
 *   cohx_seq_read_kv: values 0/1 = K/V rows [0, length) of a full-attention
 *     layer, 2 = conv ring [channels][kernel], 3 = delta memory
 *     [value_heads][key_dim][value_dim] of a linear-attention layer;
 *   cohx_step: Graph::forward_batch (execution.rs:257-608) over a ragged batch,
 *     exact; a lane may carry several tokens, processed in order.
 * Other entry points return COHX_UNSUPPORTED on such a context. */
int cohx_create_qwen35(const cohx_qwen35_desc *desc, int device, cohx_ctx **out);

/* ---- host mirror of the engine's generation API ------------------------- */

typedef struct cohx_gen cohx_gen;

/* GenerationOptions (inference.rs:68-108) restricted to the token path. */
typedef struct {
  uint32_t max_tokens;
  float temperature;
  uint32_t top_k;
  float top_p;
  uint64_t seed;
  float repetition_penalty, frequency_penalty, presence_penalty;
  uint32_t n_stop_tokens;
  const uint32_t *stop_tokens;
  uint32_t context; /* session context (0: max_context) */
} cohx_gen_options;

/* BatchStep (batch.rs:3-9). */
typedef struct {
  uint32_t width;
  uint32_t completed_tokens;
  uint64_t matrix_tiles;
  uint64_t matrix_bytes;
} cohx_batch_step;

enum { COHX_FINISH_NONE = 0, COHX_FINISH_STOP = 1, COHX_FINISH_LENGTH = 2,
       COHX_FINISH_CANCELLED = 3 };

/* Model::begin_generation (generation.rs:53-242) from prompt token ids.
 * `prior` (may be NULL) is a finished generation whose KV is reused by
 * longest common token prefix, capped at prompt_len-1 (generation.rs:189-202). */
int cohx_gen_begin(cohx_ctx *ctx, const uint32_t *prompt, uint32_t n_prompt,
                   const cohx_gen_options *options, cohx_gen *prior, cohx_gen **out);
/* Model::step_batch (batch.rs:64-116): one token per lane, 1..=max_lanes lanes. */
int cohx_step_batch(cohx_ctx *ctx, cohx_gen *const *states, uint32_t n, cohx_batch_step *out);
/* cohx_step_batch with the WorkYield hook (see cohx_step_hooks); the states'
 * own cancellation (cohx_gen_cancel, which may be called from any thread while
 * a step runs) is checked before the launch and after the device finishes. */
int cohx_step_batch_hooked(cohx_ctx *ctx, cohx_gen *const *states, uint32_t n, cohx_batch_step *out,
                           int (*yield)(void *user), void *user);
/* Model::step_generation (generation.rs:244-257): the single-lane path. */
int cohx_step_generation(cohx_ctx *ctx, cohx_gen *state);
/* GenerationState::sample (generation.rs:319-394): *token = id or -1 for none. */
int cohx_gen_sample(cohx_gen *state, int64_t *token);
int cohx_gen_needs_forward(const cohx_gen *state);
int cohx_gen_is_finished(const cohx_gen *state);
int cohx_gen_is_prefilling(const cohx_gen *state);
uint32_t cohx_gen_finish_reason(const cohx_gen *state);
/* Generated ids so far; returns the count (copies at most cap). */
uint32_t cohx_gen_tokens(const cohx_gen *state, uint32_t *out, uint32_t cap);
/* Cancellation::cancel for this generation; thread-safe (an atomic flag):
 * the owning thread observes it at its next step, sample or state query. */
void cohx_gen_cancel(cohx_gen *state);
/* GenerationState::compatible (generation.rs:271-275): both states belong to
 * the same context (the engine also requires equal execution settings, which
 * are the context's here). */
int cohx_gen_compatible(const cohx_gen *a, const cohx_gen *b);
void cohx_gen_free(cohx_gen *state);

#ifdef __cplusplus
}
#endif
#endif
