// lbt_sched.cpp -- continuous batching of requests over one lbt_batch, greedy
// or drawn by the device sampler with each request's own parameters.
//
// Not in the reference: lb-server runs one request at a time
// (crates/lb-server/src/main.rs:92-100).  A request waits in a FIFO until a
// slot of the batch is free, is prefilled there (its first token is the
// prefill's argmax), then advances one token per step together with every
// other active slot in one batched forward.  Free slots ride along in that
// forward at position 0 (their rows are computed and ignored; their length
// is reset before each step, so they never grow).  Host-side bookkeeping
// only: all model work goes through the lbt_batch entry points.
#include <deque>
#include <map>
#include <vector>

#include "lbt_internal.h"

struct lbt_sched {
    lbt_model* m = nullptr;
    lbt_batch* b = nullptr;
    int slots = 0, cap = 0, vocab = 0;
    struct Req {
        std::vector<uint32_t> prompt;
        size_t max_new = 0;
        uint32_t stop = 0xffffffffu;
        std::vector<uint32_t> out;
        bool done = false;
        // sampled requests: the job's SamplingParams and sampler state
        // (sample.rs:28-35); greedy ones keep temperature 0
        lbt_sample_params sp{0.0f, 1.0f, 0};
        uint64_t state = 1;
    };
    std::map<uint64_t, Req> reqs;
    std::deque<uint64_t> queue;
    std::vector<int64_t> slot_req;  // request id per slot, -1 when free
    uint64_t next_id = 1;
};

namespace {

// A request is finished once it has max_new tokens or emitted its stop token.
bool finished(const lbt_sched::Req& r) {
    return r.out.size() >= r.max_new || (!r.out.empty() && r.out.back() == r.stop);
}

lbt_ctx* ctx_of(lbt_sched* s) { return s ? lbt::model_ctx(s->m) : nullptr; }

}  // namespace

int lbt_sched_new(lbt_model* m, int slots, int cap, lbt_sched** out) {
    if (!m || !out || slots <= 0 || cap <= 1) return lbt::set_err(m ? lbt::model_ctx(m) : nullptr, LBT_E_INVALID, "bad arguments");
    *out = nullptr;
    lbt_batch* b = nullptr;
    int rc = lbt_batch_new(m, slots, cap, &b);
    if (rc) return rc;
    lbt_config c;
    lbt_model_get_config(m, &c);
    lbt_sched* s = new lbt_sched();
    s->m = m;
    s->b = b;
    s->slots = slots;
    s->cap = cap;
    s->vocab = c.vocab_size;
    s->slot_req.assign((size_t)slots, -1);
    *out = s;
    return LBT_OK;
}

void lbt_sched_free(lbt_sched* s) {
    if (!s) return;
    lbt_batch_free(s->b);
    delete s;
}

int lbt_sched_submit(lbt_sched* s, const uint32_t* prompt, size_t n, size_t max_new, uint32_t stop, uint64_t* id) {
    if (!s || !prompt || n == 0 || max_new == 0 || !id) return lbt::set_err(ctx_of(s), LBT_E_INVALID, "bad arguments");
    // the prompt, then max_new - 1 decode steps (the first token is the prefill's)
    if (n > (size_t)s->cap || max_new - 1 > (size_t)s->cap - n)
        return lbt::set_err(ctx_of(s), LBT_E_RANGE, "sched: request exceeds slot capacity");
    for (size_t i = 0; i < n; i++)
        if (prompt[i] >= (uint32_t)s->vocab) return lbt::set_err(ctx_of(s), LBT_E_INVALID, "token id out of range");
    lbt_sched::Req r;
    r.prompt.assign(prompt, prompt + n);
    r.max_new = max_new;
    r.stop = stop;
    *id = s->next_id++;
    s->reqs.emplace(*id, std::move(r));
    s->queue.push_back(*id);
    return LBT_OK;
}

int lbt_sched_submit_sample(lbt_sched* s, const uint32_t* prompt, size_t n, size_t max_new, uint32_t stop,
                            const lbt_sample_params* p, uint64_t seed, uint64_t* id) {
    if (!p) return lbt::set_err(ctx_of(s), LBT_E_INVALID, "bad arguments");
    int rc = lbt_sched_submit(s, prompt, n, max_new, stop, id);
    if (rc) return rc;
    lbt_sched::Req& r = s->reqs[*id];
    r.sp = *p;
    r.state = seed > 1 ? seed : 1;  // Sampler::new: seed.max(1)
    return LBT_OK;
}

int lbt_sched_step(lbt_sched* s, int* pending) {
    if (!s) return LBT_E_INVALID;
    int rc;
    // admission: queued requests into free slots, each prefilled on its own
    for (int k = 0; k < s->slots && !s->queue.empty(); k++) {
        if (s->slot_req[k] >= 0) continue;
        const uint64_t id = s->queue.front();
        lbt_sched::Req& r = s->reqs[id];
        // the request leaves the queue only once its slot holds it: a failed
        // reset or prefill leaves it first in line for the next step
        if ((rc = lbt_batch_reset(s->b, k))) return rc;
        uint32_t first = 0;
        uint64_t st = r.state;
        if ((rc = r.sp.temperature != 0.0f
                      ? lbt_batch_prefill_sample(s->b, k, r.prompt.data(), r.prompt.size(), &r.sp, &st, &first)
                      : lbt_batch_prefill(s->b, k, r.prompt.data(), r.prompt.size(), &first))) {
            lbt_batch_reset(s->b, k);
            return rc;
        }
        s->queue.pop_front();
        r.state = st;
        r.out.push_back(first);
        if (finished(r)) {
            r.done = true;
            lbt_batch_reset(s->b, k);
        } else {
            s->slot_req[k] = (int64_t)id;
        }
    }
    // one batched decode step of the active slots (free slots at position 0)
    bool any = false, sampled = false;
    std::vector<uint32_t> toks((size_t)s->slots, 0), next((size_t)s->slots, 0);
    std::vector<lbt_sample_params> sp((size_t)s->slots, lbt_sample_params{0.0f, 1.0f, 0});
    std::vector<uint64_t> st((size_t)s->slots, 1);
    for (int k = 0; k < s->slots; k++) {
        if (s->slot_req[k] < 0) {
            if ((rc = lbt_batch_reset(s->b, k))) return rc;
            continue;
        }
        any = true;
        const lbt_sched::Req& r = s->reqs[(uint64_t)s->slot_req[k]];
        toks[k] = r.out.back();
        sp[k] = r.sp;
        st[k] = r.state;
        sampled |= r.sp.temperature != 0.0f;
    }
    if (any) {
        // greedy slots ride along in a sampling step at temperature 0 (the argmax)
        if ((rc = sampled ? lbt_batch_forward_sample(s->b, toks.data(), sp.data(), st.data(), next.data())
                          : lbt_batch_forward(s->b, toks.data(), nullptr, next.data())))
            return rc;
        for (int k = 0; k < s->slots; k++) {
            if (s->slot_req[k] < 0) continue;
            lbt_sched::Req& r = s->reqs[(uint64_t)s->slot_req[k]];
            r.state = st[k];
            r.out.push_back(next[k]);
            if (finished(r)) {
                r.done = true;
                s->slot_req[k] = -1;
            }
        }
    }
    if (pending) {
        int p = (int)s->queue.size();
        for (int k = 0; k < s->slots; k++) p += s->slot_req[k] >= 0;
        *pending = p;
    }
    return LBT_OK;
}

int lbt_sched_result(lbt_sched* s, uint64_t id, uint32_t* tokens, size_t cap, size_t* n, int* done) {
    if (!s) return LBT_E_INVALID;
    auto it = s->reqs.find(id);
    if (it == s->reqs.end()) return lbt::set_err(ctx_of(s), LBT_E_INVALID, "sched: unknown request id");
    const lbt_sched::Req& r = it->second;
    if (tokens)
        for (size_t i = 0; i < r.out.size() && i < cap; i++) tokens[i] = r.out[i];
    if (n) *n = r.out.size();
    if (done) *done = r.done ? 1 : 0;
    return LBT_OK;
}

int lbt_sched_release(lbt_sched* s, uint64_t id) {
    if (!s) return LBT_E_INVALID;
    auto it = s->reqs.find(id);
    if (it == s->reqs.end()) return lbt::set_err(ctx_of(s), LBT_E_INVALID, "sched: unknown request id");
    if (!it->second.done) return lbt::set_err(ctx_of(s), LBT_E_INVALID, "sched: request not finished");
    s->reqs.erase(it);
    return LBT_OK;
}
