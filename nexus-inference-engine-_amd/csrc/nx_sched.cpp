// Request scheduler over the runner's sequence slots: the serving loop of
// Engine::generate (nexus/src/core/engine.cpp:124-184) -- prefill a prompt,
// decode up to max_tokens tokens, stop early -- for many requests at once.
// Requests wait in arrival order; whenever a slot is free and the KV page
// pool can hold the request to its last position (pages reserved per
// request: a model with a shared pool, kv_blocks, holds fewer pages than
// batch * max_seq / 16), the next one is admitted into it (its prompt
// prefilled alone, whatever its length, while the other slots keep their
// sequences), then every active slot decodes in chunks of steps, and a
// request that has its tokens (or emitted its stop token) is retired,
// freeing the slot and its pages for the next one.
#include <algorithm>
#include <deque>
#include <map>
#include <vector>

#include "nx_internal.h"

using nx::fail;

namespace {

struct Request {
    std::vector<int32_t> prompt;
    int max_new = 0, stop = -1;
    int pages = 0;  // KV pages to its last position: (P + max_new - 2) / 16 + 1
    std::vector<int32_t> out;
    int slot = -1;
    bool done = false;
    nx_status err = NX_OK;  // a failed admission: the request is done with this status
};

// Steps per decode call of the scheduler: at most this many, fewer when an
// active request needs fewer tokens.
constexpr int kChunk = 8;

}  // namespace

struct nx_sched {
    nx_model* m = nullptr;
    nx_ctx* ctx = nullptr;
    int batch = 0, max_seq = 0, vocab = 0;
    int pool_pages = 0, reserved = 0;  // pages of the model's pool, reserved by active requests
    std::deque<int> waiting;
    std::vector<int> slot_req;  // request id per slot, -1 = free
    std::map<int, Request> reqs;
    int next_id = 1;
};

namespace {

// Append tokens to request r until it is complete; true when it is.
bool take(Request& r, const int32_t* tok, int n) {
    for (int i = 0; i < n && !r.done; ++i) {
        r.out.push_back(tok[i]);
        if ((int)r.out.size() >= r.max_new || tok[i] == r.stop) r.done = true;
    }
    return r.done;
}

}  // namespace

nx_status nx_sched_create(nx_model* m, nx_sched** out) {
    if (!m || !out) return NX_ERR_INVALID;
    nx_model_config c{};
    nx_status s = nx_model_get_config(m, &c);
    if (s != NX_OK) return s;
    auto* sc = new nx_sched();
    sc->m = m;
    sc->ctx = nx_model_context(m);
    sc->batch = c.batch;
    sc->max_seq = c.max_seq;
    sc->vocab = c.vocab;
    sc->slot_req.assign((size_t)c.batch, -1);
    for (int b = 0; b < c.batch; ++b) (void)nx_model_retire(m, b);
    s = nx_model_kv_pages(m, &sc->pool_pages, nullptr);
    if (s != NX_OK) {
        delete sc;
        return s;
    }
    *out = sc;
    return NX_OK;
}

nx_status nx_sched_destroy(nx_sched* s) {
    if (!s) return NX_ERR_INVALID;
    delete s;
    return NX_OK;
}

nx_status nx_sched_submit(nx_sched* s, const int32_t* prompt, int P, int max_new, int stop, int* id) {
    if (!s || !prompt || !id || P < 1 || max_new < 1) return NX_ERR_INVALID;
    if (P + max_new > s->max_seq)
        return fail(s->ctx, NX_ERR_CAPACITY, "request of %d prompt + %d new tokens exceeds max_seq %d", P, max_new,
                    s->max_seq);
    for (int i = 0; i < P; ++i)
        if (prompt[i] < 0 || prompt[i] >= s->vocab) return fail(s->ctx, NX_ERR_INVALID, "prompt token out of vocabulary");
    Request r;
    r.prompt.assign(prompt, prompt + P);
    r.max_new = max_new;
    r.stop = stop;
    r.pages = (P + max_new - 2) / 16 + 1;
    if (r.pages > s->pool_pages)
        return fail(s->ctx, NX_ERR_CAPACITY, "request of %d pages exceeds the KV pool of %d", r.pages, s->pool_pages);
    const int rid = s->next_id++;
    s->reqs.emplace(rid, std::move(r));
    s->waiting.push_back(rid);
    *id = rid;
    return NX_OK;
}

nx_status nx_sched_step(nx_sched* s, int* n_active, int* n_waiting) {
    if (!s) return NX_ERR_INVALID;
    // admit waiting requests into free slots
    for (int b = 0; b < s->batch && !s->waiting.empty(); ++b) {
        if (s->slot_req[(size_t)b] >= 0) continue;
        const int rid = s->waiting.front();
        Request& r = s->reqs[rid];
        if (s->reserved + r.pages > s->pool_pages) break;  // in arrival order: wait for pages
        int32_t first = 0;
        nx_status st = nx_model_admit(s->m, b, r.prompt.data(), (int)r.prompt.size(), &first);
        // the request leaves the queue either way: admitted, or done with the
        // admission's status (nx_model_admit leaves the slot free on failure;
        // a retry could fail the same way forever in nx_sched_run)
        s->waiting.pop_front();
        if (st != NX_OK) {
            r.done = true;
            r.err = st;
            return st;
        }
        r.slot = b;
        if (take(r, &first, 1)) {
            (void)nx_model_retire(s->m, b);
            r.slot = -1;
        } else {
            s->slot_req[(size_t)b] = rid;
            s->reserved += r.pages;
        }
    }
    // one chunk of decode steps for the active slots
    int need = kChunk, act = 0;
    for (int b = 0; b < s->batch; ++b) {
        const int rid = s->slot_req[(size_t)b];
        if (rid < 0) continue;
        const Request& r = s->reqs[rid];
        need = std::min(need, r.max_new - (int)r.out.size());
        ++act;
    }
    if (act > 0) {
        std::vector<int32_t> tok((size_t)s->batch * need);
        nx_status st = nx_model_decode(s->m, need, tok.data());
        if (st != NX_OK) return st;
        for (int b = 0; b < s->batch; ++b) {
            const int rid = s->slot_req[(size_t)b];
            if (rid < 0) continue;
            Request& r = s->reqs[rid];
            if (take(r, tok.data() + (size_t)b * need, need)) {
                (void)nx_model_retire(s->m, b);
                s->slot_req[(size_t)b] = -1;
                s->reserved -= r.pages;
                r.slot = -1;
            }
        }
    }
    int a = 0;
    for (int rid : s->slot_req) a += rid >= 0;
    if (n_active) *n_active = a;
    if (n_waiting) *n_waiting = (int)s->waiting.size();
    return NX_OK;
}

nx_status nx_sched_run(nx_sched* s) {
    if (!s) return NX_ERR_INVALID;
    int a = 0, w = 0;
    do {
        nx_status st = nx_sched_step(s, &a, &w);
        if (st != NX_OK) return st;
    } while (a > 0 || w > 0);
    return NX_OK;
}

nx_status nx_sched_result(nx_sched* s, int id, int32_t* out, int cap, int* n, int* done) {
    if (!s || !n || !done) return NX_ERR_INVALID;
    auto it = s->reqs.find(id);
    if (it == s->reqs.end()) return fail(s->ctx, NX_ERR_INVALID, "no request %d", id);
    const Request& r = it->second;
    *n = (int)r.out.size();
    *done = r.done ? 1 : 0;
    if (out) std::copy(r.out.begin(), r.out.begin() + std::min(cap, (int)r.out.size()), out);
    if (r.err != NX_OK) return fail(s->ctx, r.err, "request %d failed at admission", id);
    return NX_OK;
}
