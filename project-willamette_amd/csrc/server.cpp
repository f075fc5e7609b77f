// Continuous batching on one model: requests join and leave between steps,
// and every step advances all active requests in one ragged batch.
//
// Reference semantics per request: generate_with_cache_and_sampler
// (src/model/generate.rs:195-277) on a cache of its own: the prompt goes into
// the sampler's history, is prefilled in order (generate.rs:151-160 / :235-245),
// then each step samples the next id from the logits of the last token,
// stops at EOS or a stop id, records and observes the id, and forwards it
// unless it is the last one wanted.  Here a step packs, for every active
// request, either its next prompt chunk or its one pending token into a
// single wm_batch_forward-style step; the batch is bit-identical to running
// each request's tokens through forward_with_cache in order, and each
// request samples with its own sampler, so every request's ids equal those
// of wm_generate_with_sampler on its own (or wm_greedy_generate for greedy
// parameters).  The reference has no multi-request driver; this one exists
// so that a serving loop gets MFMA-sized batches.
//
// Scheduling: at most max_seqs requests are active (each owns one cache of
// max_seq_len positions, kept in a pool); waiting requests are admitted in
// submission order.  A step's token budget is step_tokens: every decoding
// request's token first, then prompt chunks in admission order.
#include <algorithm>
#include <deque>
#include <map>
#include <string>
#include <vector>

#include "wm_internal.h"

namespace {

struct srv_req {
    uint64_t id = 0;
    std::vector<uint32_t> prompt;
    uint32_t max_new = 0;
    int64_t eos = -1;
    std::vector<uint32_t> stops;
    wm_sampler *sampler = nullptr;
    bool greedy = false;
    wm_kv_cache *kv = nullptr;
    uint32_t consumed = 0;  // prompt tokens forwarded
    bool has_pending = false;
    uint32_t pending = 0;   // the last sampled id, not yet forwarded
    std::vector<uint32_t> out;
    bool finished = false;
    wm_status status = WM_OK;
    std::string error;
};

bool is_greedy_params(const wm_sampling_params &p) {  // sampler.rs:71-78
    return (p.temperature < 0 ? -p.temperature : p.temperature) < 1e-9f && !p.has_top_k &&
           !p.has_top_p && !p.has_repetition_penalty;
}

}  // namespace

struct wm_server {
    wm_model *m = nullptr;
    uint32_t max_seqs = 0, max_seq_len = 0, step_tokens = 0;
    std::vector<wm_kv_cache *> caches;  // every cache made (at most max_seqs)
    std::vector<wm_kv_cache *> free_caches;
    std::deque<srv_req *> waiting;
    std::vector<srv_req *> active;  // admission order
    std::map<uint64_t, srv_req *> reqs;
    uint64_t next_id = 1;
};

namespace {

void release_cache(wm_server *s, srv_req *r) {
    if (r->kv) {
        wm_kv_cache_rollback(r->kv, 0);
        s->free_caches.push_back(r->kv);
        r->kv = nullptr;
    }
}

void finish(wm_server *s, srv_req *r, wm_status st, const char *msg) {
    r->finished = true;
    r->status = st;
    if (st && msg) r->error = msg;
    release_cache(s, r);
}

// After a successful step over `part` (participants, in batch order, with
// last_rows[i] the final row of participant i): sample for every request
// whose prompt is now consumed.
wm_status after_step(wm_server *s, const std::vector<srv_req *> &part,
                     const std::vector<uint32_t> &last_rows, bool have_next) {
    wm_model *m = s->m;
    wm_ctx *ctx = wm_model_ctx(m);
    std::vector<uint32_t> next(part.size(), 0);
    if (have_next) {
        wm_status st = wm_batch_next_ids(m, (uint32_t)part.size(), next.data());
        if (st) return st;
    }
    const uint32_t vocab = wm_model_cfg(m).vocab_size;
    for (size_t i = 0; i < part.size(); i++) {
        srv_req *r = part[i];
        r->has_pending = false;
        if (r->consumed < r->prompt.size()) continue;  // still prefilling
        if (r->out.size() >= r->max_new) {  // max_new == 0: the prompt alone
            finish(s, r, WM_OK, nullptr);
            continue;
        }
        uint32_t id = 0;
        if (r->greedy) {
            id = next[i];
        } else {
            const float *d_logits = nullptr;
            wm_status st = wm_batch_row_logits(m, last_rows[i], &d_logits);
            if (!st) st = wm_sampler_run(r->sampler, d_logits, vocab, &id);
            if (st) {
                if (st == WM_E_HIP) return st;
                finish(s, r, st, wm_last_error(ctx));
                continue;
            }
        }
        bool stop = r->eos >= 0 && (int64_t)id == r->eos;
        for (uint32_t t : r->stops) stop = stop || t == id;
        if (stop) {
            finish(s, r, WM_OK, nullptr);
            continue;
        }
        r->out.push_back(id);
        wm_sampler_observe(r->sampler, id);
        if (r->out.size() >= r->max_new) {
            finish(s, r, WM_OK, nullptr);  // the last id is not forwarded
        } else {
            r->has_pending = true;
            r->pending = id;
        }
    }
    return WM_OK;
}

// Forward one group of (request, tokens) in one batch; on success the
// requests' positions advance and after_step samples.
wm_status run_group(wm_server *s, const std::vector<srv_req *> &part,
                    const std::vector<uint32_t> &n_new, const std::vector<uint32_t> &toks) {
    std::vector<wm_kv_cache *> kvs(part.size());
    bool any_greedy = false;
    for (size_t i = 0; i < part.size(); i++) {
        kvs[i] = part[i]->kv;
        any_greedy = any_greedy || part[i]->greedy;
    }
    std::vector<uint32_t> last;
    wm_status st = batch_forward_dev(s->m, kvs.data(), (uint32_t)part.size(), n_new.data(),
                                     toks.data(), any_greedy, last);
    if (st) return st;
    for (size_t i = 0; i < part.size(); i++)
        if (!part[i]->has_pending) part[i]->consumed += n_new[i];
    return after_step(s, part, last, any_greedy);
}

}  // namespace

extern "C" {

wm_status wm_server_create(wm_model *m, uint32_t max_seqs, uint32_t max_seq_len, uint32_t step_tokens,
                           wm_server **out) {
    if (!m || !out) return WM_E_ARG;
    wm_ctx *ctx = wm_model_ctx(m);
    *out = nullptr;
    if (!wm_model_batch_ready(m))
        return wm_set_error(ctx, WM_E_STATE, "server: model weights not set or shape not batchable");
    if (max_seqs == 0 || max_seq_len == 0 || step_tokens < max_seqs || step_tokens > 16384)
        return wm_set_error(ctx, WM_E_ARG,
                            "server: need max_seqs >= 1, max_seq_len >= 1, max_seqs <= step_tokens <= 16384");
    if (max_seq_len > wm_model_cfg(m).context_length)
        return wm_set_error(ctx, WM_E_SHAPE, "server: max_seq_len=%u exceeds model context_length=%u",
                            max_seq_len, wm_model_cfg(m).context_length);
    wm_server *s = new wm_server();
    s->m = m;
    s->max_seqs = max_seqs;
    s->max_seq_len = max_seq_len;
    s->step_tokens = step_tokens;
    *out = s;
    return WM_OK;
}

void wm_server_destroy(wm_server *s) {
    if (!s) return;
    for (auto &kv : s->reqs) {
        if (kv.second->sampler) wm_sampler_destroy(kv.second->sampler);
        delete kv.second;
    }
    for (wm_kv_cache *kv : s->caches) wm_kv_cache_destroy(kv);
    delete s;
}

wm_status wm_server_submit(wm_server *s, const uint32_t *prompt, uint32_t n_prompt, uint32_t max_new,
                           int64_t eos, const uint32_t *stop_ids, uint32_t n_stop,
                           const wm_sampling_params *params, uint64_t seed, uint64_t *request_id) {
    if (!s || !params || !request_id || (n_stop && !stop_ids)) return WM_E_ARG;
    wm_ctx *ctx = wm_model_ctx(s->m);
    const wm_model_config &c = wm_model_cfg(s->m);
    if (!prompt || n_prompt == 0)
        return wm_set_error(ctx, WM_E_ARG, "generate_with_cache_and_sampler: prompt_ids must not be empty");
    for (uint32_t i = 0; i < n_prompt; i++)
        if (prompt[i] >= c.vocab_size)
            return wm_set_error(ctx, WM_E_SHAPE,
                                "generate_with_cache_and_sampler: prompt token %u (idx %u) out of vocab range %u",
                                prompt[i], i, c.vocab_size);
    // the final id is returned, not forwarded (generate.rs:283-295)
    if ((uint64_t)n_prompt + (max_new ? max_new - 1 : 0) > s->max_seq_len)
        return wm_set_error(ctx, WM_E_SHAPE,
                            "generate_with_cache_and_sampler: prompt(%u) + generated positions exceed max_seq_len=%u",
                            n_prompt, s->max_seq_len);
    srv_req *r = new srv_req();
    wm_status st = wm_sampler_create(ctx, params, seed, &r->sampler);
    if (st) {
        delete r;
        return st;
    }
    r->id = s->next_id++;
    r->prompt.assign(prompt, prompt + n_prompt);
    r->max_new = max_new;
    r->eos = eos;
    if (n_stop) r->stops.assign(stop_ids, stop_ids + n_stop);
    r->greedy = is_greedy_params(*params);
    for (uint32_t i = 0; i < n_prompt; i++) wm_sampler_observe(r->sampler, prompt[i]);
    s->reqs[r->id] = r;
    s->waiting.push_back(r);
    *request_id = r->id;
    return WM_OK;
}

wm_status wm_server_step(wm_server *s, uint32_t *n_active) {
    if (!s) return WM_E_ARG;
    wm_ctx *ctx = wm_model_ctx(s->m);
    // retire finished requests, admit waiting ones
    s->active.erase(std::remove_if(s->active.begin(), s->active.end(),
                                   [](srv_req *r) { return r->finished; }),
                    s->active.end());
    while (s->active.size() < s->max_seqs && !s->waiting.empty()) {
        srv_req *r = s->waiting.front();
        s->waiting.pop_front();
        if (r->finished) continue;  // released before admission
        if (s->free_caches.empty()) {
            wm_kv_cache *kv = nullptr;
            wm_status st = wm_kv_cache_create(s->m, s->max_seq_len, &kv);
            if (st) {
                s->waiting.push_front(r);
                return st;
            }
            s->caches.push_back(kv);
            s->free_caches.push_back(kv);
        }
        r->kv = s->free_caches.back();
        s->free_caches.pop_back();
        s->active.push_back(r);
    }
    // the step's tokens: decoding requests first, then prompt chunks
    std::vector<srv_req *> part;
    std::vector<uint32_t> n_new, toks;
    uint32_t budget = s->step_tokens;
    for (srv_req *r : s->active)
        if (r->has_pending && budget) {
            part.push_back(r);
            n_new.push_back(1);
            toks.push_back(r->pending);
            budget--;
        }
    for (srv_req *r : s->active) {
        if (r->has_pending || r->consumed >= r->prompt.size() || !budget) continue;
        const uint32_t len = std::min<uint32_t>(budget, (uint32_t)r->prompt.size() - r->consumed);
        part.push_back(r);
        n_new.push_back(len);
        toks.insert(toks.end(), r->prompt.begin() + r->consumed, r->prompt.begin() + r->consumed + len);
        budget -= len;
    }
    if (n_active) *n_active = 0;
    if (part.empty()) return WM_OK;
    wm_status st = run_group(s, part, n_new, toks);
    if (st == WM_E_NONFINITE) {
        // find the failing requests: each one alone (the others' results are
        // those of the shared step, since every request is independent)
        size_t off = 0;
        for (size_t i = 0; i < part.size(); i++) {
            const std::vector<srv_req *> one{part[i]};
            const std::vector<uint32_t> nn{n_new[i]}, tk(toks.begin() + off, toks.begin() + off + n_new[i]);
            off += n_new[i];
            wm_status st1 = run_group(s, one, nn, tk);
            if (st1 == WM_E_NONFINITE) finish(s, part[i], st1, wm_last_error(ctx));
            else if (st1) return st1;
        }
        st = WM_OK;
    }
    if (st) return st;
    uint32_t live = 0;
    for (srv_req *r : s->active) live += !r->finished;
    if (n_active) *n_active = live + (uint32_t)s->waiting.size();
    return WM_OK;
}

wm_status wm_server_result(wm_server *s, uint64_t request_id, uint32_t *out_ids, uint32_t cap,
                           uint32_t *n_out, int *finished) {
    if (!s || !n_out || !finished || (cap && !out_ids)) return WM_E_ARG;
    wm_ctx *ctx = wm_model_ctx(s->m);
    auto it = s->reqs.find(request_id);
    if (it == s->reqs.end())
        return wm_set_error(ctx, WM_E_ARG, "server: no request %llu", (unsigned long long)request_id);
    const srv_req *r = it->second;
    const uint32_t n = (uint32_t)std::min<size_t>(cap, r->out.size());
    std::copy(r->out.begin(), r->out.begin() + n, out_ids);
    *n_out = (uint32_t)r->out.size();
    *finished = r->finished;
    if (r->status) return wm_set_error(ctx, r->status, "%s", r->error.c_str());
    return WM_OK;
}

wm_status wm_server_release(wm_server *s, uint64_t request_id) {
    if (!s) return WM_E_ARG;
    auto it = s->reqs.find(request_id);
    if (it == s->reqs.end())
        return wm_set_error(wm_model_ctx(s->m), WM_E_ARG, "server: no request %llu",
                            (unsigned long long)request_id);
    srv_req *r = it->second;
    release_cache(s, r);
    s->active.erase(std::remove(s->active.begin(), s->active.end(), r), s->active.end());
    s->waiting.erase(std::remove(s->waiting.begin(), s->waiting.end(), r), s->waiting.end());
    if (r->sampler) wm_sampler_destroy(r->sampler);
    delete r;
    s->reqs.erase(it);
    return WM_OK;
}

}  // extern "C"
