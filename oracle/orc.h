/*
 * CPU ORACLE — test infrastructure only.
 *
 * A plain-C restatement of the Coheryn engine's CPU forward step (Rust,
 * crates/coheryn-engine) used as the parity checker for the HIP path.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it;
 * the product library never links or calls it.
 *
 * Float semantics follow Rust/LLVM on Linux x86-64: no FP contraction
 * (built with -ffp-contract=off), f32::mul_add -> fmaf, round -> roundf,
 * round_ties_even -> rintf, exp/sin/cos/powf -> glibc, f64 sums start at -0.0
 * (Rust's float Sum identity) and run sequentially, half::f16 -> RNE.
 *
 * Parity pins (what checks each function, see tests/test_oracle_*.py):
 *   decode / prepare / dot   fixtures/quantized/kernels.json (100 cases)
 *   rope                     fixtures/quantized/rope.json (12 cases) + closed forms
 *   dot_f32, rms_norm,       closed forms from cpu.rs tests + brute force
 *   round_f16, attention*
 *   f16 conversion           exhaustive against the CPU's F16C instruction
 *   sampler                  fixtures/constraints/sampling-v2.json
 *   forward_batch            batched == individual invariant, zero-weight
 *                            token-0 closed form, EOS stop, tiny-model
 *                            brute-force re-derivation in numpy (f64)
 *   pack                     closed-form prefix sums / page arithmetic
 *   q35 delta step           fixtures/qwen35/operations-v1.json (3 steps, 2e-6)
 *   q35 conv / norm / gates  closed forms from qwen35/kernels.rs tests
 *   q35 partial rope         identity at position 0, untouched tail, f64 closed form
 *   q35 forward              batched == individual, float64 numpy textbook hybrid
 *                            step within tolerance, planted-mistake check
 */
#ifndef ORC_H
#define ORC_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error codes mirror crates/coheryn-engine/src/error.rs ErrorCode classes. */
enum {
  ORC_OK = 0,
  ORC_INVALID_REQUEST = 1,   /* Error::request */
  ORC_INVALID_GGUF = 2,      /* Error::invalid (shape, non-finite) */
  ORC_RESOURCE = 3,          /* Error::resource (context/KV exhausted) */
  ORC_CANCELLED = 4,
  ORC_UNSUPPORTED = 5,
  ORC_DEAD_END = 6           /* ConstraintDeadEnd */
};

/* ---- scalar kernels: quant.rs / cpu.rs ---------------------------------- */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
int orc_row_bytes(uint32_t dtype, size_t width, size_t *out);
int orc_decode(const uint8_t *bytes, size_t nbytes, uint32_t dtype, float *out, size_t n);
float orc_dot_f32(const float *a, const float *b, size_t n);
int orc_round_f16(const float *in, float *out, size_t n);
void orc_rms_norm(const float *x, const float *w, float eps, float *out, size_t n);
void orc_rope(float *x, size_t n, size_t head_dim, size_t position, float base);
void orc_swiglu(float *gate, const float *up, size_t n);
/* QuantizedInput::prepare: writes the canonical activation blocks. */
int orc_prepare(const float *in, size_t n, uint32_t weight_dtype, uint8_t *out, size_t cap,
                size_t *used, uint32_t *kind);
/* quant::dot over one packed row against prepared activation blocks. */
int orc_qdot(const uint8_t *row, size_t row_len, uint32_t dtype, const uint8_t *act,
             uint32_t act_kind, size_t width, float *out);
int orc_attention_rows(const float *q, size_t nq, const float *keys, const float *values,
                       size_t kv_rows, size_t kv_heads, size_t head_dim, float *out);
int orc_attention(const float *q, size_t nq, const float *keys, const float *values,
                  size_t kv_rows, size_t kv_heads, size_t head_dim, float *out);

/* ---- sampler: sampling.rs ------------------------------------------------ */
typedef struct orc_sampler orc_sampler;
int orc_sampler_new(float temperature, uint32_t top_k, float top_p, uint64_t seed,
                    float repetition_penalty, float frequency_penalty,
                    float presence_penalty, orc_sampler **out);
void orc_sampler_free(orc_sampler *s);
int orc_sampler_history(orc_sampler *s, size_t vocabulary, const uint32_t *tokens, size_t n);
int orc_sampler_observe(orc_sampler *s, uint32_t token);
int orc_sampler_sample(orc_sampler *s, const float *logits, size_t n, const uint8_t *allowed,
                       uint32_t *token);

/* ---- Qwen2 model: inference.rs / inference/batch.rs ---------------------- */
typedef struct {
  uint32_t layers, hidden, intermediate, heads, kv_heads, head_dim, vocabulary, context;
  float rope_base, norm_epsilon;
} orc_config;

typedef struct {
  uint32_t dtype;
  uint64_t ne0, ne1; /* GGML order: ne0 = contiguous input width */
  const uint8_t *data;
  uint64_t bytes;
} orc_tensor;

/* Tensor slots per layer, in this order. */
enum {
  ORC_ATTN_NORM = 0, ORC_FFN_NORM, ORC_Q, ORC_K, ORC_V, ORC_QB, ORC_KB, ORC_VB,
  ORC_O, ORC_GATE, ORC_UP, ORC_DOWN, ORC_LAYER_TENSORS
};

typedef struct orc_model orc_model;
typedef struct orc_session orc_session;

/* globals: token_embd, output_norm, output (data==NULL -> tied to token_embd) */
int orc_model_new(const orc_config *c, const orc_tensor *globals, const orc_tensor *layers,
                  int threads, orc_model **out);
void orc_model_free(orc_model *m);
int orc_session_new(const orc_model *m, uint32_t context, orc_session **out);
void orc_session_free(orc_session *s);
uint32_t orc_session_position(const orc_session *s);
/* Truncate a session's KV to `rows` tokens (prefix reuse, generation.rs:189-202). */
int orc_session_truncate(orc_session *s, uint32_t rows);
/* Copy one layer's K or V rows [0, position) out (kv_heads*head_dim floats per row). */
int orc_session_kv(const orc_model *m, const orc_session *s, uint32_t layer, int values,
                   float *out);
/* Seeded synthetic cache value = hash(seed, stream, layer, K/V, position,
 * element) mapped onto multiples of 2^-23 in [-1, 1). */
float orc_synthetic_kv(uint64_t seed, uint32_t stream, uint32_t layer, uint32_t which,
                       uint32_t position, uint32_t element);
/* Rows [position, rows) of every layer take orc_synthetic_kv values (the GPU
 * library's cohx_seq_fill_synthetic contract: appending after a shared prefix
 * keeps the prefix); the position becomes rows. */
int orc_session_fill_synthetic(const orc_model *m, orc_session *s, uint32_t rows, uint64_t seed,
                               uint32_t stream);
const float *orc_session_logits(const orc_session *s);

/* Model::forward_batch over n lanes; errors[i] receives each lane's status.
 * Lanes whose errors[i] != 0 on entry are skipped (already failed). */
int orc_forward_batch(const orc_model *m, orc_session **sessions, const uint32_t *tokens,
                      size_t n, int32_t *errors);
/* Model::forward_row with logits=false on the last layer skipped (prompt rows). */
int orc_forward_row(const orc_model *m, orc_session *s, uint32_t token, int logits);
/* Optional observer: x after each block, per lane (layers*hidden floats). */
int orc_forward_batch_trace(const orc_model *m, orc_session **sessions, const uint32_t *tokens,
                            size_t n, int32_t *errors, float *trace);

/* ---- Qwen3.5 hybrid text model: qwen35/execution.rs, qwen35/kernels.rs ---- */
typedef struct {
  uint32_t layers, hidden, intermediate, vocabulary, heads, kv_heads, head_dim;
  uint32_t key_heads, value_heads, key_dim, value_dim, conv_kernel, rotary_dim, context;
  float epsilon, rope_base;
  uint8_t full[128]; /* 1: full attention, 0: linear attention (config.rs layer_types) */
} orc_q35_config;

/* Tensor slots per layer (unused slots of the other mixer kind stay empty). */
enum {
  ORC_Q35_INPUT_NORM = 0, ORC_Q35_POST_NORM, ORC_Q35_GATE, ORC_Q35_UP, ORC_Q35_DOWN,
  ORC_Q35_Q, ORC_Q35_K, ORC_Q35_V, ORC_Q35_O, ORC_Q35_QNORM, ORC_Q35_KNORM,
  ORC_Q35_QKV, ORC_Q35_Z, ORC_Q35_A, ORC_Q35_B, ORC_Q35_OUT, ORC_Q35_CONV, ORC_Q35_ALOG,
  ORC_Q35_DT, ORC_Q35_NORM, ORC_Q35_LAYER_TENSORS
};

typedef struct orc_q35_model orc_q35_model;
typedef struct orc_q35_session orc_q35_session;

float orc_q35_sigmoid(float x);
float orc_q35_silu(float x);
float orc_q35_softplus(float x);
int orc_q35_norm(const float *in, const float *w, float eps, int zero_centered, float *out,
                 size_t n);
int orc_q35_conv_step(float *history, uint32_t *cursor, size_t channels, size_t kernel,
                      const float *in, const float *w, float *out);
int orc_q35_delta_step(float *memory, size_t heads, size_t key, size_t value, const float *q,
                       const float *k, const float *v, const float *log_decay,
                       const float *beta, float *out);
int orc_q35_partial_rope(float *values, size_t n, size_t head, size_t rotary, size_t position,
                         float base);
/* globals: embed_tokens, final norm, lm_head (data == NULL: tied to embed_tokens).
 * Matrices: dtype 0 (F32) or 30 (BF16), ne0 = input width, ne1 = output rows. */
int orc_q35_model_new(const orc_q35_config *c, const orc_tensor *globals,
                      const orc_tensor *layers, int threads, orc_q35_model **out);
void orc_q35_model_free(orc_q35_model *m);
int orc_q35_session_new(const orc_q35_model *m, uint32_t context, orc_q35_session **out);
void orc_q35_session_free(orc_q35_session *s);
uint32_t orc_q35_session_position(const orc_q35_session *s);
const float *orc_q35_session_logits(const orc_q35_session *s);
int orc_q35_session_state(const orc_q35_model *m, const orc_q35_session *s, uint32_t layer,
                          int which, float *out);
/* One token per lane (logits[i]: compute the vocabulary projection). */
int orc_q35_forward_batch(const orc_q35_model *m, orc_q35_session **sessions,
                          const uint32_t *tokens, const uint8_t *logits, size_t n,
                          int32_t *errors);

/* ---- ragged packer (host restatement of the GPU packing contract) --------- */
/* lanes: n_tokens[i] >= 1, start[i] = first position, page tables row-major
 * [lanes][max_pages] with page_size tokens per page.
 * Outputs: cu_seqlens[n+1], row_position[R], row_slot[R], row_lane[R]. */
int orc_pack(size_t n, const uint32_t *n_tokens, const uint32_t *start, const int32_t *pages,
             uint32_t max_pages, uint32_t page_size, uint32_t *cu_seqlens, uint32_t *row_position,
             int64_t *row_slot, uint32_t *row_lane);

#ifdef __cplusplus
}
#endif
#endif
