// Host-side generation loop above the C-ABI: the n-gram draft cache and the
// Generator of flare-core/src/generate.rs, driving the device entry points
// (fl_prefill, fl_decode_step / fl_decode_run, fl_verify, fl_decode_step_sample).
//
// Semantics follow generate.rs line by line (cited per function); the one
// structural change is the speculative step: the reference verifies its k
// drafts with k sequential forward_greedy calls (generate.rs:244-312), this
// loop verifies them with ONE fl_verify pass over the same k inputs
// [last, d0, .., d(k-2)] at the same positions.  Pass outputs g[i] are what
// the reference's i-th forward returns, so the accepted tokens, the positions
// and the statistics are the reference's; K/V slots the pass wrote past the
// accepted prefix are rewritten by later steps (positions are tracked here,
// KvCache::truncate_to kv_cache.rs:521-531 is a position reset).
#include <cmath>
#include <cstdint>
#include <cstring>
#include <map>
#include <new>
#include <vector>

#include "../../include/flare_hip.h"

namespace {

// generate.rs:7-13
constexpr size_t kNgramMaxEntries = 10000;
constexpr size_t kMaxDraftTokens = 5;
constexpr int kNgramSizes[3] = {2, 3, 4};

}  // namespace

// NgramCache (generate.rs:37-103).  An ordered map keyed by the context
// n-gram: lookups only ever ask for exact keys, so the map kind does not
// change any result.
struct fl_ngram {
    std::map<std::vector<uint32_t>, std::vector<uint32_t>> table;
    size_t total_entries = 0;

    // evict (generate.rs:96-102): clear everything
    void evict() {
        table.clear();
        total_entries = 0;
    }

    // record (generate.rs:55-75): the n-grams ending at the last token
    void record(const uint32_t *tokens, size_t len) {
        for (int n : kNgramSizes) {
            if (len < (size_t)n + 1) continue;
            const size_t start = len - n - 1;
            std::vector<uint32_t> ctxt(tokens + start, tokens + start + n);
            table[ctxt].push_back(tokens[len - 1]);
            total_entries++;
        }
        if (total_entries > kNgramMaxEntries) evict();
    }

    // record_prompt_ngrams (generate.rs:166-182): every n-gram of the sequence
    void record_all(const uint32_t *tokens, size_t len) {
        for (int n : kNgramSizes) {
            if (len < (size_t)n + 1) continue;
            for (size_t i = 0; i + n + 1 <= len; i++) {
                std::vector<uint32_t> ctxt(tokens + i, tokens + i + n);
                table[ctxt].push_back(tokens[i + n]);
                total_entries++;
            }
        }
        if (total_entries > kNgramMaxEntries) evict();
    }

    // lookup_drafts (generate.rs:79-92): longest n-gram first, the (up to 5)
    // most recent continuations of the first context that is present
    std::vector<uint32_t> lookup(const uint32_t *tokens, size_t len) const {
        for (int k = 2; k >= 0; k--) {
            const int n = kNgramSizes[k];
            if (len < (size_t)n) continue;
            std::vector<uint32_t> ctxt(tokens + len - n, tokens + len);
            auto it = table.find(ctxt);
            if (it != table.end()) {
                const std::vector<uint32_t> &c = it->second;
                const size_t start = c.size() > kMaxDraftTokens ? c.size() - kMaxDraftTokens : 0;
                return std::vector<uint32_t>(c.begin() + start, c.end());
            }
        }
        return {};
    }
};

// Generator (generate.rs:106-560), self-speculation (layer skipping,
// generate.rs:314-403) excluded.
struct fl_generator {
    fl_ctx *ctx = nullptr;
    fl_sampling_params params{};
    std::vector<uint32_t> tokens;
    int position = 0;
    fl_ngram ngram;
    fl_spec_stats stats{};
    int vocab = 0;

    // is_speculative (generate.rs:128-130)
    bool speculative() const { return params.speculative && params.temperature == 0.0f; }
    bool greedy_fused() const { return params.temperature == 0.0f && params.repeat_penalty == 1.0f; }
};

namespace {

// One forward at (last token, position) giving the next token: the fused
// greedy path (forward_greedy) or logits + repeat penalty + temperature +
// sampling (generate.rs:186-238), sampled on the device.
int forward_next(fl_generator *g, float rng_val, uint32_t *out) {
    const uint32_t last = g->tokens.empty() ? 0u : g->tokens.back();
    int32_t t = 0;
    int rc;
    if (g->greedy_fused()) {
        rc = fl_decode_step(g->ctx, last, g->position, nullptr, &t, nullptr);
    } else {
        rc = fl_decode_step_sample(g->ctx, last, g->position, &g->params, g->tokens.data(), (int)g->tokens.size(),
                                   rng_val, &t);
    }
    if (rc) return rc;
    *out = (uint32_t)t;
    return 0;
}

void push_token(fl_generator *g, uint32_t t) {
    g->tokens.push_back(t);
    g->position++;
    if (g->speculative()) g->ngram.record(g->tokens.data(), g->tokens.size());
}

// speculative_step (generate.rs:244-312): up to 5 drafts verified in one
// fl_verify pass (fused greedy path) or sequentially (repeat penalty).
int speculative_step(fl_generator *g, std::vector<uint32_t> &accepted) {
    accepted.clear();
    const std::vector<uint32_t> drafts = g->ngram.lookup(g->tokens.data(), g->tokens.size());
    if (drafts.empty()) return 0;
    g->stats.attempts++;
    g->stats.drafted += drafts.size();
    const size_t k = drafts.size();
    if (g->params.repeat_penalty == 1.0f) {
        // the reference's k forwards see [last, d0, .., d(k-2)] at
        // position, position+1, ...; one pass computes all of them
        std::vector<uint32_t> in(k);
        in[0] = g->tokens.empty() ? 0u : g->tokens.back();
        for (size_t i = 1; i < k; i++) in[i] = drafts[i - 1];
        std::vector<int32_t> out(k);
        const int rc = fl_verify(g->ctx, in.data(), (int)k, g->position, out.data(), nullptr);
        if (rc) return rc;
        for (size_t i = 0; i < k; i++) {
            const uint32_t v = (uint32_t)out[i];
            push_token(g, v);
            accepted.push_back(v);
            if (v != drafts[i]) break;
            g->stats.accepted++;
        }
        return 0;
    }
    for (size_t i = 0; i < k; i++) {
        uint32_t v = 0;
        // greedy over penalized logits (generate.rs:275-285): temperature 0 here
        const int rc = forward_next(g, 0.0f, &v);
        if (rc) return rc;
        push_token(g, v);
        accepted.push_back(v);
        if (v != drafts[i]) break;
        g->stats.accepted++;
    }
    return 0;
}

}  // namespace

extern "C" {

fl_ngram *fl_ngram_create(void) { return new (std::nothrow) fl_ngram(); }
void fl_ngram_destroy(fl_ngram *c) { delete c; }
void fl_ngram_record(fl_ngram *c, const uint32_t *tokens, size_t n) {
    if (c && tokens) c->record(tokens, n);
}
void fl_ngram_record_all(fl_ngram *c, const uint32_t *tokens, size_t n) {
    if (c && tokens) c->record_all(tokens, n);
}
int fl_ngram_lookup(const fl_ngram *c, const uint32_t *tokens, size_t n, uint32_t *out) {
    if (!c || !out || (!tokens && n)) return 0;
    const std::vector<uint32_t> d = c->lookup(tokens, n);
    for (size_t i = 0; i < d.size(); i++) out[i] = d[i];
    return (int)d.size();
}
size_t fl_ngram_entries(const fl_ngram *c) { return c ? c->total_entries : 0; }

void fl_sampling_params_default(fl_sampling_params *p) {
    // SamplingParams::default (flare-core/src/sampling.rs:56-70)
    if (!p) return;
    p->temperature = 0.7f;
    p->top_p = 0.9f;
    p->top_k = 40;
    p->repeat_penalty = 1.1f;
    p->min_p = 0.0f;
    p->speculative = 1;
}

int fl_generator_create(fl_ctx *ctx, const fl_sampling_params *params, fl_generator **out) {
    if (!ctx || !params || !out) return FL_E_INVALID;
    if (!fl_has_weights(ctx)) return FL_E_STATE;
    fl_generator *g = new (std::nothrow) fl_generator();
    if (!g) return FL_E_OOM;
    g->ctx = ctx;
    g->params = *params;
    *out = g;
    return 0;
}

void fl_generator_destroy(fl_generator *g) { delete g; }

int fl_generator_prefill(fl_generator *g, const uint32_t *prompt, int n, float *out_logits) {
    // Generator::prefill (generate.rs:139-163)
    if (!g || (!prompt && n)) return FL_E_INVALID;
    if (n == 0) return 0;
    int32_t t = 0;
    const int rc = fl_prefill(g->ctx, prompt, n, g->position, out_logits, &t, nullptr);
    if (rc) return rc;
    g->tokens.insert(g->tokens.end(), prompt, prompt + n);
    g->position += n;
    if (g->speculative()) g->ngram.record_all(g->tokens.data(), g->tokens.size());
    return 0;
}

int fl_generator_step(fl_generator *g, float rng_val, uint32_t *out_token) {
    // Generator::step (generate.rs:186-238)
    if (!g || !out_token) return FL_E_INVALID;
    uint32_t t = 0;
    const int rc = forward_next(g, rng_val, &t);
    if (rc) return rc;
    push_token(g, t);
    *out_token = t;
    return 0;
}

int fl_generator_generate(fl_generator *g, const uint32_t *prompt, int n_prompt, int max_tokens, int64_t eos,
                          fl_rng_fn rng, void *rng_user, fl_token_fn on_token, void *token_user,
                          uint32_t *out_tokens, int *n_out) {
    // Generator::generate (generate.rs:409-531), n-gram speculation only
    if (!g || !out_tokens || !n_out || max_tokens < 0 || (!prompt && n_prompt)) return FL_E_INVALID;
    *n_out = 0;
    int rc = fl_generator_prefill(g, prompt, n_prompt, nullptr);
    if (rc) return rc;
    int step = 0, n = 0;
    const bool use_spec = g->speculative();
    std::vector<uint32_t> acc;
    while (step < max_tokens) {
        if (use_spec && step > 0) {
            rc = speculative_step(g, acc);
            if (rc) return rc;
            if (!acc.empty()) {
                bool stop = false;
                for (uint32_t t : acc) {
                    out_tokens[n++] = t;
                    if (eos >= 0 && (int64_t)t == eos) { stop = true; break; }
                    if (on_token && !on_token(t, (size_t)step, token_user)) { stop = true; break; }
                    step++;
                    if (step >= max_tokens) { stop = true; break; }
                }
                if (stop) break;
                continue;
            }
        }
        uint32_t t = 0;
        rc = fl_generator_step(g, rng ? rng(rng_user) : 0.0f, &t);
        if (rc) return rc;
        out_tokens[n++] = t;
        if (eos >= 0 && (int64_t)t == eos) break;
        if (on_token && !on_token(t, (size_t)step, token_user)) break;
        step++;
    }
    *n_out = n;
    return 0;
}

int fl_generator_stats(const fl_generator *g, fl_spec_stats *out) {
    if (!g || !out) return FL_E_INVALID;
    *out = g->stats;
    return 0;
}

int fl_generator_position(const fl_generator *g) { return g ? g->position : -1; }

int fl_generator_tokens(const fl_generator *g, uint32_t *out, int cap) {
    if (!g) return FL_E_INVALID;
    const int n = (int)g->tokens.size();
    if (out)
        for (int i = 0; i < n && i < cap; i++) out[i] = g->tokens[i];
    return n;
}

}  // extern "C"
