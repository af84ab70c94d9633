// Qwen3.5 hybrid text step: device launchers and the per-step views they take
// (not part of the C ABI).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace cohx {

// Row error bit for failures the engine reports as Error::request (norm and
// recurrent-state overflow, qwen35/kernels.rs:4-10,36-47,167-176).
constexpr uint32_t kErrRequest = 8u;

// Widest row the norm kernel stages in LDS.
constexpr int kQ35MaxHidden = 8192;

// Longest sequence slot: the attention kernel keeps a row's scores, prefix
// maxima and rescale factors in LDS (3 floats per key, under 64 KiB).
constexpr int kQ35MaxContext = 4096;

// Attention shapes the kernels stage: heads per KV group (a power of two) and
// head width.
constexpr int kQ35MaxGroup = 16, kQ35MaxHeadDim = 256;

// Lane tables of one step: lane i owns rows [first[i], first[i] + n[i]) of
// sequence seq[i], the first at position start[i].
struct Q35Lanes {
  const uint32_t *first, *n, *seq, *start;
};

// Per-row tables: lane, position and sequence of every packed row.
struct Q35Rows {
  const uint32_t *lane, *pos, *seq;
};

// Matrices live as 16-output tiles: [rows/16][K/8][16][8] binary16-bf16
// words, so a wave's 16 outputs read 256 contiguous bytes per 8 inputs.
inline size_t q35_tiled_index(size_t row, size_t k, size_t K) {
  return (((row / 16) * (K / 8) + k / 8) * 16 + row % 16) * 8 + k % 8;
}

enum Q35Epi { kQ35Store = 0, kQ35Residual = 1, kQ35Argmax = 2, kQ35Swiglu = 3 };

void q35_embed(hipStream_t s, int rows, const uint16_t *embed, const uint32_t *tokens, int H,
               float *x);
// out[r] = norm(x[src ? src[r] : r]) * (w + zc)
void q35_norm(hipStream_t s, int rows, const float *x, int ldx, const uint32_t *src,
              const float *w, int n, float eps, int zc, float *out, int ldo, uint32_t *row_err,
              const uint32_t *err_row);
// out[r][o] (=, +=) sum_k x[r][k] * w[o][k] in f64, k in order; argmax keys
// per 64-output block go to part[r][block] (logits optional).
void q35_matvec(hipStream_t s, int epi, const uint16_t *w, int rows_w, int valid_rows, int K,
                const float *x, int ldx, int R, float *out, int ldo, unsigned long long *part,
                uint32_t *row_err, const uint32_t *err_row);
int q35_matvec_blocks(int rows_w);
// Packed-prefill regime: rows x[rows][K] (stride ldx; K and ldx multiples of
// 4) as bfloat16 pairs hi = bf16(x), lo = bf16(x - hi) into hi/lo[rows][K],
// the operands of q35_gemm_split.
void q35_split_bf16(hipStream_t s, int rows, int K, const float *x, int ldx, uint16_t *hi, uint16_t *lo);
// Packed-prefill regime linear on the matrix cores (gemm.h): out[r][n] (=, or
// += with accumulate) sum_k (hi[r][k] + lo[r][k]) * w[n][k] for n < N, with w
// the tiled matrix the exact matvecs read (q35_tiled_index, K % 64 == 0),
// f32 sums; row_err[r] |= the matvecs' non-finite bit for rows with a
// non-finite output.
void q35_gemm_split(hipStream_t s, bool accumulate, const uint16_t *w, int N, int K, const uint16_t *hi,
                    const uint16_t *lo, int rows, float *out, int ldo, uint32_t *row_err);
// Gate+up and SwiGLU in one launch for few rows: h[r][f] = silu(gate) * up
// with the bits of q35_matvec (gate rows [0, F), up rows [up_off, up_off + F))
// followed by q35_swiglu.  Returns false (nothing launched) where q35_matvec
// would not take its one-chain-per-lane form (more than 64 rows, or few
// enough tiles for the producer/consumer form).
bool q35_matvec_swiglu(hipStream_t s, const uint16_t *w, int up_off, int F, int K, const float *x,
                       int ldx, int R, float *h, int ldh, uint32_t *row_err);
void q35_swiglu(hipStream_t s, int rows, const float *gu, int ldgu, int F, int up_off, float *h,
                int ldh);
void q35_conv(hipStream_t s, int lanes, Q35Lanes L, const float *mix, int ldm, const float *w,
              int C, int K, float *hist, size_t hist_seq, float *out, int ldo, uint32_t *row_err);
bool q35_delta_supported(int key_dim, int value_dim);
// The whole linear-attention mixer (conv, gates, delta rule, output norm x
// SiLU(z)) in one launch per (lane, value head), for conv kernels of at most
// four taps and one key head per value head; hist is the layer's conv ring
// (per-sequence stride hist_seq).
bool q35_linear_fused(int conv_kernel, int key_heads, int value_heads);
void q35_linear(hipStream_t s, int lanes, Q35Lanes L, const float *mix, int ldm, int keys,
                int z_off, int a_off, int b_off, const float *conv_w, int K, float *hist,
                size_t hist_seq, const float *a_log, const float *dt, const float *norm_w,
                int key_heads, int value_heads, int key_dim, int value_dim, float eps,
                float *state, size_t state_seq, float *tgt, int ldt, uint32_t *row_err);
// Gates, the recurrence over each lane's tokens, then the per-head output
// norm times SiLU(z) into tgt (gates: [rows][value_heads], o_raw like tgt).
void q35_delta(hipStream_t s, int rows, int lanes, Q35Lanes L, const float *conv, int ldc, int keys,
               const float *mix, int ldm, int z_off, int a_off, int b_off, const float *a_log,
               const float *dt, const float *norm_w, int key_heads, int value_heads, int key_dim,
               int value_dim, float eps, float *state, size_t state_seq, float4 *gates,
               float *o_raw, float *tgt, int ldt, uint32_t *row_err);
void q35_qk(hipStream_t s, int rows, Q35Rows Rw, const float *mix, int ldm, int k_off, int v_off,
            const float *q_norm, const float *k_norm, int heads, int kv_heads, int D, int rotary,
            float eps, const float2 *rope, float *q, float *z, int ldq, float *kc, float *vc,
            size_t cache_seq, uint32_t *row_err);
// Scores into scores[rows][heads][max_context], then softmax and output.
void q35_attention(hipStream_t s, int rows, Q35Rows Rw, const float *q, const float *z, int ldq,
                   const float *kc, const float *vc, size_t cache_seq, int heads, int kv_heads,
                   int D, int max_context, float *scores, float *out, int ldo);

}  // namespace cohx
