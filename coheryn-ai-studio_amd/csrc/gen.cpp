// Host mirror of the engine's generation API over the GPU step.
//
// GenerationState (crates/coheryn-engine/src/inference/generation.rs:18-394),
// Model::step_batch (inference/batch.rs:64-116) and Sampler
// (crates/coheryn-engine/src/sampling.rs:57-223).  Greedy lanes without
// penalties take the device argmax (lowest id on ties, sampling.rs:160-173)
// and never copy logits; any other sampling setting copies the last row's
// logits and runs the seeded host sampler.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <vector>

#include "internal.h"

using namespace cohx;

namespace {

// ---------------------------------------------------------------------------
// Sampler (sampling.rs:57-223)
// ---------------------------------------------------------------------------
struct Sampler {
  float temperature = 0.0f, top_p = 1.0f;
  uint32_t top_k = 0;
  uint64_t state = 0;
  float rep = 1.0f, freq = 0.0f, pres = 0.0f;
  std::vector<uint32_t> counts;

  bool penalties() const { return rep != 1.0f || freq != 0.0f || pres != 0.0f; }

  int init(const cohx_gen_options &o) {
    temperature = o.temperature;
    top_k = o.top_k;
    top_p = o.top_p;
    state = o.seed;
    rep = o.repetition_penalty;
    freq = o.frequency_penalty;
    pres = o.presence_penalty;
    if (!std::isfinite(temperature) || !(temperature >= 0.0f && temperature <= 2.0f) ||
        !std::isfinite(top_p) || top_p <= 0.0f || top_p > 1.0f)
      return COHX_INVALID_REQUEST;
    if (!std::isfinite(rep) || !(rep >= 0.01f && rep <= 10.0f) || !std::isfinite(freq) ||
        !(freq >= -2.0f && freq <= 2.0f) || !std::isfinite(pres) ||
        !(pres >= -2.0f && pres <= 2.0f))
      return COHX_INVALID_REQUEST;
    return COHX_OK;
  }

  int history(size_t vocabulary) {
    if (top_k > vocabulary) return COHX_INVALID_REQUEST;
    if (penalties()) counts.assign(vocabulary, 0);
    return COHX_OK;
  }

  int observe(uint32_t token) {
    if (!penalties()) return COHX_OK;
    if (token >= counts.size()) return COHX_INVALID_REQUEST;
    if (counts[token] == UINT32_MAX) return COHX_RESOURCE;
    counts[token]++;
    return COHX_OK;
  }

  double random() {  // SplitMix64, sampling.rs:123-130
    state += 0x9e3779b97f4a7c15ULL;
    uint64_t z = state;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return (double)((z ^ (z >> 31)) >> 11) / (double)(1ULL << 53);
  }

  double adjusted(size_t id, float logit) const {
    const uint32_t count = id < counts.size() ? counts[id] : 0;
    double v = (double)logit;
    if (count != 0) {
      v = v < 0.0 ? v * (double)rep : v / (double)rep;
      v -= (double)pres + (double)count * (double)freq;
    }
    return v;
  }

  bool needs_logits() const { return temperature != 0.0f || penalties(); }

  int sample(const float *logits, size_t n, uint32_t *token) {
    if (n == 0) return COHX_INVALID_GGUF;
    for (size_t i = 0; i < n; i++)
      if (!std::isfinite(logits[i])) return COHX_INVALID_GGUF;
    if (top_k > n) return COHX_INVALID_REQUEST;
    if (temperature == 0.0f) {
      size_t best = 0;
      double bv = adjusted(0, logits[0]);
      for (size_t id = 1; id < n; id++) {
        const double v = adjusted(id, logits[id]);
        if (v > bv) {
          best = id;
          bv = v;
        }
      }
      *token = (uint32_t)best;
      return COHX_OK;
    }
    struct Ranked {
      uint32_t id;
      double value;
    };
    std::vector<Ranked> ids(n);
    for (size_t i = 0; i < n; i++) ids[i] = Ranked{(uint32_t)i, adjusted(i, logits[i])};
    auto key = [](double v) {
      int64_t b;
      std::memcpy(&b, &v, 8);
      return b ^ (int64_t)((uint64_t)(b >> 63) >> 1);  // f64::total_cmp order
    };
    auto before = [&](const Ranked &a, const Ranked &b) {
      const int64_t ka = key(a.value), kb = key(b.value);
      if (ka != kb) return ka > kb;
      return a.id < b.id;
    };
    size_t count = n;
    if (top_k > 0 && top_k < n) {
      std::partial_sort(ids.begin(), ids.begin() + top_k, ids.end(), before);
      count = top_k;
    } else {
      std::sort(ids.begin(), ids.end(), before);
    }
    std::vector<double> prob(count);
    const double maximum = ids[0].value;
    for (size_t i = 0; i < count; i++) prob[i] = std::exp((ids[i].value - maximum) / (double)temperature);
    double total = -0.0;
    for (double p : prob) total += p;
    double cumulative = 0.0;
    size_t keep = 0;
    for (size_t i = 0; i < count; i++) {
      cumulative += prob[i] / total;
      keep++;
      if (cumulative >= (double)top_p) break;
    }
    double mass = -0.0;
    for (size_t i = 0; i < keep; i++) mass += prob[i];
    const double threshold = random() * mass;
    cumulative = 0.0;
    for (size_t i = 0; i < keep; i++) {
      cumulative += prob[i];
      if (threshold < cumulative) {
        *token = ids[i].id;
        return COHX_OK;
      }
    }
    *token = ids[keep - 1].id;
    return COHX_OK;
  }
};

}  // namespace

struct cohx_gen {
  cohx_ctx *ctx = nullptr;
  bool has_seq = false;
  uint32_t seq = 0;
  std::vector<uint32_t> prompt;
  std::vector<uint32_t> kv_tokens;  // Session::tokens: ids whose K/V are cached
  size_t cursor = 0, reused = 0;
  int64_t pending = -1;
  Sampler sampler;
  std::vector<uint32_t> ids;
  std::vector<uint32_t> stop_tokens;
  uint32_t max_tokens = 0;
  bool done = false;
  // Cancellation token (set from any thread); the state machine observes it
  // on the owning thread
  std::atomic<bool> cancel{false};
  uint32_t reason = COHX_FINISH_LENGTH;
  int32_t error = COHX_OK;
  std::vector<float> logits;  // last forward's logits (only when the sampler needs them)
  uint32_t argmax = 0;

  bool prefilling() const { return cursor < prompt.size(); }
  bool cancelled() const { return cancel.load(std::memory_order_acquire); }
  // generate_impl (inference.rs:655-664): a decode-phase cancellation
  // finishes the generation with reason Cancelled
  bool finished() const { return done || (cancelled() && !prefilling()); }
  bool needs_forward() const { return !finished() && (prefilling() || pending >= 0); }
};

namespace {

bool is_eog(const cohx_ctx *ctx, uint32_t token) {
  for (uint32_t i = 0; i < ctx->desc.n_eog; i++)
    if (ctx->desc.eog[i] == token) return true;
  return false;
}

// GenerationState::next_token (generation.rs:291-304)
int next_token(cohx_gen *g, uint32_t *token) {
  if (g->error) {
    const int e = g->error;
    g->error = COHX_OK;
    return e;
  }
  if (g->cancelled()) return COHX_CANCELLED;
  if (g->done) return COHX_INVALID_REQUEST;
  if (g->cursor < g->prompt.size()) {
    *token = g->prompt[g->cursor];
    return COHX_OK;
  }
  if (g->pending >= 0) {
    *token = (uint32_t)g->pending;
    return COHX_OK;
  }
  return COHX_INVALID_REQUEST;  // sample existing logits before advancing generation
}

}  // namespace

extern "C" {

int cohx_gen_begin(cohx_ctx *ctx, const uint32_t *prompt, uint32_t n_prompt,
                   const cohx_gen_options *o, cohx_gen *prior, cohx_gen **out) {
  if (!ctx || !out || !o || !prompt || n_prompt == 0) return COHX_INVALID_REQUEST;
  *out = nullptr;
  const cohx_model_desc &d = ctx->desc;
  const uint32_t context = o->context ? o->context : d.max_context;
  if (context == 0 || context > d.max_context)
    return fail(ctx, COHX_INVALID_REQUEST, "requested context exceeds the loaded context limit");
  if (o->max_tokens > context)
    return fail(ctx, COHX_INVALID_REQUEST, "invalid generation length or stop sequences");
  if (o->n_stop_tokens > 16) return fail(ctx, COHX_INVALID_REQUEST, "too many stop tokens");
  for (uint32_t i = 0; i < o->n_stop_tokens; i++)
    if (o->stop_tokens[i] >= d.vocabulary)
      return fail(ctx, COHX_INVALID_REQUEST, "stop_tokens must contain valid token IDs");
  if ((uint64_t)n_prompt + o->max_tokens > context)  // generation.rs:151-161
    return fail(ctx, COHX_INVALID_REQUEST,
                "prompt must be nonempty and prompt plus max_tokens must fit context");
  for (uint32_t i = 0; i < n_prompt; i++)
    if (prompt[i] >= d.vocabulary) return fail(ctx, COHX_INVALID_REQUEST, "token ID outside vocabulary");
  cohx_gen *g = new cohx_gen();
  g->ctx = ctx;
  int rc = g->sampler.init(*o);
  if (!rc) rc = g->sampler.history(d.vocabulary);
  for (uint32_t i = 0; i < n_prompt && !rc; i++) rc = g->sampler.observe(prompt[i]);
  if (rc) {
    delete g;
    return fail(ctx, rc, "invalid sampling settings");
  }
  g->prompt.assign(prompt, prompt + n_prompt);
  g->max_tokens = o->max_tokens;
  g->stop_tokens.assign(o->stop_tokens, o->stop_tokens + o->n_stop_tokens);
  // Prefix reuse (generation.rs:189-202): take over a finished generation's
  // KV, keep the longest common token prefix, capped at prompt_len-1 so the
  // last prompt token is always recomputed.
  // A hybrid (Qwen3.5) context's recurrent state cannot be rewound, so there
  // the prior sequence is taken over only when all of it is such a prefix.
  size_t common = 0;
  if (prior && prior->ctx == ctx && prior->has_seq && prior->finished()) {
    while (common < prior->kv_tokens.size() && common < g->prompt.size() &&
           prior->kv_tokens[common] == g->prompt[common])
      common++;
    common = std::min(common, g->prompt.size() - 1);
  }
  if (prior && prior->ctx == ctx && prior->has_seq && prior->finished() &&
      ctx->seqs[prior->seq].capacity >= context &&
      (!ctx->q35 || common == prior->kv_tokens.size())) {
    g->seq = prior->seq;
    g->has_seq = true;
    prior->has_seq = false;
    rc = cohx_seq_truncate(ctx, g->seq, (uint32_t)common);
    g->kv_tokens.assign(prior->kv_tokens.begin(), prior->kv_tokens.begin() + common);
    g->cursor = g->reused = common;
  } else {
    rc = cohx_seq_alloc(ctx, context, &g->seq);
    g->has_seq = rc == COHX_OK;
  }
  if (rc) {
    cohx_gen_free(g);
    return rc;
  }
  *out = g;
  return COHX_OK;
}

// Model::step_batch (batch.rs:64-116)
int cohx_step_batch(cohx_ctx *ctx, cohx_gen *const *states, uint32_t n, cohx_batch_step *stats) {
  return cohx_step_batch_hooked(ctx, states, n, stats, nullptr, nullptr);
}

int cohx_step_batch_hooked(cohx_ctx *ctx, cohx_gen *const *states, uint32_t n, cohx_batch_step *stats,
                           int (*yield)(void *user), void *user) {
  if (!ctx || !states) return COHX_INVALID_REQUEST;
  if (n == 0 || n > ctx->desc.max_lanes)
    return fail(ctx, COHX_INVALID_REQUEST,
                "batch width must be in 1..=" + std::to_string(ctx->desc.max_lanes));
  for (uint32_t i = 0; i < n; i++)
    if (!states[i] || states[i]->ctx != ctx || !states[i]->has_seq)
      return fail(ctx, COHX_INVALID_REQUEST, "incompatible native generation batch");
  std::vector<uint32_t> tokens(n);
  std::vector<uint8_t> prefilling(n);
  std::vector<cohx_lane> lanes;
  std::vector<uint32_t> lane_of;
  for (uint32_t i = 0; i < n; i++) {
    cohx_gen *g = states[i];
    prefilling[i] = g->prefilling();
    uint32_t tok = 0;
    const int rc = next_token(g, &tok);
    if (rc) {
      g->error = rc;
      continue;
    }
    tokens[i] = tok;
    // Logits are copied only for the row that will be sampled next by a
    // sampler that needs them.
    const bool sampled_next = !(g->cursor + 1 < g->prompt.size());
    cohx_lane ln{};
    ln.seq = g->seq;
    ln.n_tokens = 1;
    ln.tokens = &tokens[i];
    uint32_t len = 0;
    cohx_seq_length(ctx, g->seq, &len);
    ln.start_position = len;
    // Rows that do not end the prompt need no head on a hybrid context
    // (qwen35/generation.rs:368); the Qwen2 graph computes it for every lane.
    ln.want_logits = (sampled_next && g->sampler.needs_logits()) ? 1u
                     : (!sampled_next && ctx->q35)              ? COHX_SKIP_HEAD
                                                                 : 0u;
    if (ln.want_logits == 1u) g->logits.resize(ctx->desc.vocabulary);
    lanes.push_back(ln);
    lane_of.push_back(i);
  }
  uint32_t width = (uint32_t)lanes.size();
  if (stats) *stats = cohx_batch_step{width, 0, 0, 0};
  if (lanes.empty()) return COHX_OK;
  std::vector<cohx_lane_out> outs(lanes.size());
  for (size_t k = 0; k < lanes.size(); k++)
    outs[k].logits = lanes[k].want_logits == 1u ? states[lane_of[k]]->logits.data() : nullptr;
  cohx_batch batch{(uint32_t)lanes.size(), lanes.data()};
  cohx_step_out so{};
  so.lanes = outs.data();
  std::vector<uint32_t> before(lanes.size());
  for (size_t k = 0; k < lanes.size(); k++) before[k] = lanes[k].start_position;
  const cohx_step_hooks hooks{yield, user, nullptr};
  const int rc = cohx_step_hooked(ctx, &batch, &so, yield ? &hooks : nullptr);
  if (rc) {  // shared failure: every participant observes it (batch.rs:98-105)
    for (uint32_t i : lane_of)
      if (!states[i]->error) states[i]->error = rc;
    return COHX_OK;
  }
  uint32_t completed = 0;
  for (size_t k = 0; k < lanes.size(); k++) {
    cohx_gen *g = states[lane_of[k]];
    // cancelled while the device computed: on a Qwen2 context the forward is
    // dropped (the sequence keeps its length), as the engine's check between
    // layers would have stopped it; a Qwen3.5 step stands (its recurrent
    // state cannot be rewound) and the next step observes the token
    if (!outs[k].status && !ctx->q35 && g->cancelled()) {
      cohx_seq_truncate(ctx, g->seq, before[k]);
      outs[k].status = COHX_CANCELLED;
    }
    if (outs[k].status) {
      g->error = outs[k].status;
      continue;
    }
    completed++;
    g->argmax = outs[k].argmax;
    g->kv_tokens.push_back(tokens[lane_of[k]]);
    // GenerationState::forwarded (generation.rs:305-317)
    if (prefilling[lane_of[k]])
      g->cursor++;
    else
      g->pending = -1;
  }
  if (stats) {
    stats->width = width;
    stats->completed_tokens = completed;
    stats->matrix_tiles = 1;
    stats->matrix_bytes = so.matrix_bytes;
  }
  return COHX_OK;
}

int cohx_step_generation(cohx_ctx *ctx, cohx_gen *state) {
  cohx_gen *one[1] = {state};
  cohx_batch_step st;
  int rc = cohx_step_batch(ctx, one, 1, &st);
  if (rc) return rc;
  if (state->error) {
    const int e = state->error;
    state->error = COHX_OK;
    return e;
  }
  return COHX_OK;
}

// GenerationState::sample (generation.rs:319-394)
int cohx_gen_sample(cohx_gen *g, int64_t *token) {
  if (!g || !token) return COHX_INVALID_REQUEST;
  *token = -1;
  if (g->error) {
    const int e = g->error;
    g->error = COHX_OK;
    return e;
  }
  if (g->cancelled()) {
    if (!g->prefilling() && !g->done) {
      g->done = true;
      g->reason = COHX_FINISH_CANCELLED;
    }
    return COHX_CANCELLED;
  }
  if (g->done || g->needs_forward()) return COHX_OK;
  if (g->ids.size() == g->max_tokens) {
    g->done = true;
    return COHX_OK;
  }
  uint32_t tok = g->argmax;
  if (g->sampler.needs_logits()) {
    const int rc = g->sampler.sample(g->logits.data(), g->logits.size(), &tok);
    if (rc) return rc;
  }
  int rc = g->sampler.observe(tok);
  if (rc) return rc;
  g->ids.push_back(tok);
  const bool stop = is_eog(g->ctx, tok) ||
                    std::find(g->stop_tokens.begin(), g->stop_tokens.end(), tok) != g->stop_tokens.end();
  if (stop) {
    g->done = true;
    g->reason = COHX_FINISH_STOP;
    return COHX_OK;
  }
  g->done = g->ids.size() == g->max_tokens;
  if (!g->done) g->pending = tok;
  *token = tok;
  return COHX_OK;
}

int cohx_gen_needs_forward(const cohx_gen *g) { return g && g->needs_forward(); }
int cohx_gen_is_finished(const cohx_gen *g) { return g && g->finished(); }
int cohx_gen_is_prefilling(const cohx_gen *g) { return g && g->prefilling(); }
uint32_t cohx_gen_finish_reason(const cohx_gen *g) {
  if (!g || !g->finished()) return COHX_FINISH_NONE;
  return g->done ? g->reason : (uint32_t)COHX_FINISH_CANCELLED;
}

int cohx_gen_compatible(const cohx_gen *a, const cohx_gen *b) { return a && b && a->ctx == b->ctx; }

uint32_t cohx_gen_tokens(const cohx_gen *g, uint32_t *out, uint32_t cap) {
  if (!g) return 0;
  const uint32_t n = (uint32_t)g->ids.size();
  if (out) std::memcpy(out, g->ids.data(), std::min(n, cap) * sizeof(uint32_t));
  return n;
}

void cohx_gen_cancel(cohx_gen *g) {
  if (g) g->cancel.store(true, std::memory_order_release);
}

void cohx_gen_free(cohx_gen *g) {
  if (!g) return;
  if (g->has_seq && g->ctx) cohx_seq_free(g->ctx, g->seq);
  delete g;
}

}  // extern "C"
