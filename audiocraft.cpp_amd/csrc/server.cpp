// server.cpp -- the request server of include/mgx.h: many callers, one batched decode.
//
// The reference's HTTP services run one generation at a time: each job thread takes the
// Sessions::gpu() lock for the whole of mg_generate (src/serve/http.h:201-205, 254-255,
// 278-291; tools/musicgen-server.cpp:321-390). Here each caller's mgx_server_generate hands its
// request to one worker thread that owns a slotted batch (runtime.cpp, slots.h) and waits.
// The worker admits queued requests into free slots between rounds of batch steps, so
// requests of different prompt lengths, generation lengths, conditioning lengths, sampling
// parameters and guidance share every step, each computing exactly what mg_generate
// computes for it alone. Progress is reported per loop iteration as the reference's
// ProgressFn is (pipeline.cpp:301), from the worker thread, after the round that ran it.
#include "mgx.h"
#include "slots.h"

#include <algorithm>
#include <chrono>
#include <condition_variable>
#include <deque>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

namespace {

double now_s() {
    using clock = std::chrono::steady_clock;
    return std::chrono::duration<double>(clock::now().time_since_epoch()).count();
}

// One caller's request; it lives on the caller's stack while the caller waits.
struct Job {
    mgx_batch_request req{};
    int n_ctx = 0, prompt_len = 0;
    mgx_progress_fn progress = nullptr;
    void* user = nullptr;
    int32_t* codes = nullptr;
    float *first = nullptr, *steps = nullptr;
    mgx_generate_report* rep = nullptr;
    // worker state
    int slot = -1, start = 0, S = 0, reported = 0;
    double t_open = 0.0, t_first = 0.0;
    // completion (under the server's lock)
    bool done = false;
    int status = MGX_OK;
    std::string error;
};

}  // namespace

struct mgx_server {
    mgx_model* m = nullptr;
    mgx_slots* sl = nullptr;
    mgx_server_config cfg{};
    std::mutex mu;
    std::condition_variable cv_work, cv_done;
    std::deque<Job*> queue;
    std::vector<Job*> active;   // by slot
    bool stop = false;
    int callers = 0;            // callers inside mgx_server_generate
    int fatal = MGX_OK;         // a device failure ends the server: every later request fails
    std::string fatal_msg;
    int64_t steps = 0, slot_steps = 0, served = 0;
    std::thread worker;
};

namespace {

// Completes `j` (the caller wakes up); call with the lock held.
void complete(mgx_server* sv, Job* j, int status, const std::string& msg) {
    j->status = status;
    j->error = msg;
    j->done = true;
    if (status == MGX_OK) ++sv->served;
    sv->cv_done.notify_all();
}

void fail_all(mgx_server* sv, int status, const std::string& msg) {
    for (Job*& j : sv->active)
        if (j) { complete(sv, j, status, msg); j = nullptr; }
    while (!sv->queue.empty()) {
        complete(sv, sv->queue.front(), status, msg);
        sv->queue.pop_front();
    }
}

// Reports loop iterations up to the slot's host position (positions 0..pos-1 are done; the
// loop's first iteration is position start - 1).
void report_progress(Job* j, int processed, double t) {
    const int iters = std::max(0, processed - (j->start - 1));
    if (iters > 0 && j->t_first == 0.0) j->t_first = t;
    for (; j->reported < iters; ++j->reported)
        if (j->progress) j->progress(j->user, j->reported + 1, j->S - j->start);
}

void run(mgx_server* sv) {
    const int n = sv->cfg.slots;
    std::unique_lock<std::mutex> lk(sv->mu);
    for (;;) {
        sv->cv_work.wait(lk, [&] {
            if (sv->stop || !sv->queue.empty()) return true;
            for (Job* j : sv->active)
                if (j) return true;
            return false;
        });
        if (sv->stop) break;
        std::vector<Job*> opening;
        for (int r = 0; r < n && !sv->queue.empty(); ++r)
            if (!sv->active[(size_t)r]) {
                Job* j = sv->queue.front();
                sv->queue.pop_front();
                j->slot = r;
                sv->active[(size_t)r] = j;
                opening.push_back(j);
            }
        lk.unlock();
        int rc = MGX_OK;
        std::string msg;
        std::vector<Job*> refused;
        for (Job* j : opening) {
            const int orc = mgx_internal_slot_open(sv->sl, j->slot, &j->req, j->n_ctx, j->prompt_len);
            if (orc != MGX_OK) {
                if (orc == MGX_ERR_DEVICE) { rc = orc; msg = mgx_last_error(); break; }
                j->error = mgx_last_error();
                j->status = orc;
                refused.push_back(j);
                continue;
            }
            int live = 0, pos = 0;
            mgx_internal_slot_state(sv->sl, j->slot, &live, &pos, &j->start, &j->S);
            j->t_open = now_s();
        }
        // one round: up to steps_per_round steps, ending at the next retirement
        int steps = sv->cfg.steps_per_round, busy = 0;
        if (rc == MGX_OK) {
            for (int r = 0; r < n; ++r) {
                Job* j = sv->active[(size_t)r];
                if (!j || j->status != MGX_OK) continue;
                int live = 0, pos = 0, start = 0, S = 0;
                mgx_internal_slot_state(sv->sl, r, &live, &pos, &start, &S);
                steps = std::min(steps, S - 1 - pos);
                ++busy;
            }
            if (busy > 0) {
                rc = mgx_internal_slots_run(sv->sl, steps);
                if (rc == MGX_OK) rc = mgx_internal_slots_sync(sv->sl);
                if (rc != MGX_OK) msg = mgx_last_error();
            }
        }
        std::vector<Job*> finished;
        if (rc == MGX_OK && busy > 0) {
            const double t = now_s();
            for (int r = 0; r < n; ++r) {
                Job* j = sv->active[(size_t)r];
                if (!j || j->status != MGX_OK) continue;
                int live = 0, pos = 0, start = 0, S = 0;
                mgx_internal_slot_state(sv->sl, r, &live, &pos, &start, &S);
                report_progress(j, live ? pos : S - 1, t);
                if (live) continue;
                const int rrc = mgx_internal_slot_read(sv->sl, r, j->codes, j->first, j->steps);
                if (rrc == MGX_ERR_DEVICE) { rc = rrc; msg = mgx_last_error(); break; }
                if (rrc != MGX_OK) {
                    j->status = rrc;
                    j->error = mgx_last_error();
                } else if (j->rep) {
                    mgx_generate_report& rp = *j->rep;
                    rp.cache_bytes = mgx_internal_slot_cache_bytes(sv->sl);
                    rp.prefill_tokens = j->start;
                    rp.decode_steps = j->S - j->start - 1;
                    rp.forwards = j->S - j->start;
                    rp.prefill_seconds = j->t_first - j->t_open;
                    rp.decode_seconds = t - j->t_first;
                }
                finished.push_back(j);
            }
        }
        lk.lock();
        sv->steps += busy > 0 && rc == MGX_OK ? steps : 0;
        sv->slot_steps += busy > 0 && rc == MGX_OK ? (int64_t)steps * busy : 0;
        for (Job* j : refused) {
            sv->active[(size_t)j->slot] = nullptr;
            complete(sv, j, j->status, j->error);
        }
        for (Job* j : finished) {
            sv->active[(size_t)j->slot] = nullptr;
            complete(sv, j, j->status, j->error);
        }
        if (rc != MGX_OK) {
            sv->fatal = rc;
            sv->fatal_msg = msg;
            fail_all(sv, rc, msg);
        }
    }
    fail_all(sv, MGX_ERR_STATE, "the server was shut down");
}

}  // namespace

extern "C" {

int mgx_server_create(mgx_model* model, const mgx_server_config* cfg, mgx_server** out) {
    if (!model || !cfg || !out) return mgx_internal_set_error(MGX_ERR_INVALID, "null argument");
    *out = nullptr;
    if (cfg->steps_per_round < 0) return mgx_internal_set_error(MGX_ERR_INVALID, "steps_per_round must not be negative");
    mgx_slots* sl = nullptr;
    const int rc = mgx_internal_slots_create(model, cfg->slots, cfg->guided ? 2 : 1, cfg->max_gen_len,
                                             cfg->guided ? cfg->max_ctx : 1, cfg->keep_step_logits, &sl);
    if (rc != MGX_OK) return rc;
    auto* sv = new mgx_server();
    sv->m = model;
    sv->sl = sl;
    sv->cfg = *cfg;
    if (sv->cfg.steps_per_round == 0) sv->cfg.steps_per_round = 16;
    sv->active.assign((size_t)cfg->slots, nullptr);
    sv->worker = std::thread(run, sv);
    *out = sv;
    return MGX_OK;
}

int mgx_server_generate(mgx_server* sv, const float* t5_hidden, int32_t n_ctx, int32_t description_empty,
                        const int32_t* prompt_codes, int32_t prompt_len, const mgx_generate_params* params,
                        mgx_progress_fn progress, void* user, int32_t* codes_out, float* first_logits_out,
                        float* step_logits_out, mgx_generate_report* report) {
    if (!sv || !params || !codes_out || !report) return mgx_internal_set_error(MGX_ERR_INVALID, "null argument");
    if (step_logits_out && !sv->cfg.keep_step_logits)
        return mgx_internal_set_error(MGX_ERR_INVALID, "the server keeps no per-step logits");
    Job j;
    j.req.t5_hidden = t5_hidden;
    j.req.description_empty = description_empty;
    j.req.prompt_codes = prompt_codes;
    j.req.params = *params;
    j.n_ctx = n_ctx;
    j.prompt_len = prompt_len;
    j.progress = progress;
    j.user = user;
    j.codes = codes_out;
    j.first = first_logits_out;
    j.steps = step_logits_out;
    j.rep = report;
    const int crc = mgx_internal_slot_check(sv->sl, &j.req, n_ctx, prompt_len);
    if (crc != MGX_OK) return crc;
    std::unique_lock<std::mutex> lk(sv->mu);
    if (sv->fatal != MGX_OK) return mgx_internal_set_error(sv->fatal, sv->fatal_msg.c_str());
    if (sv->stop) return mgx_internal_set_error(MGX_ERR_STATE, "the server was shut down");
    ++sv->callers;
    sv->queue.push_back(&j);
    sv->cv_work.notify_one();
    sv->cv_done.wait(lk, [&] { return j.done; });
    --sv->callers;
    sv->cv_done.notify_all();
    if (j.status != MGX_OK) return mgx_internal_set_error(j.status, j.error.c_str());
    return MGX_OK;
}

int mgx_server_stats(mgx_server* sv, mgx_server_counters* out) {
    if (!sv || !out) return mgx_internal_set_error(MGX_ERR_INVALID, "null argument");
    std::lock_guard<std::mutex> lk(sv->mu);
    out->steps = sv->steps;
    out->slot_steps = sv->slot_steps;
    out->served = sv->served;
    out->active = 0;
    for (Job* j : sv->active) out->active += j != nullptr;
    out->queued = (int32_t)sv->queue.size();
    return MGX_OK;
}

void mgx_server_destroy(mgx_server* sv) {
    if (!sv) return;
    {
        std::lock_guard<std::mutex> lk(sv->mu);
        sv->stop = true;
    }
    sv->cv_work.notify_all();
    if (sv->worker.joinable()) sv->worker.join();
    {
        // callers still waiting were failed by the worker; let them leave before freeing
        std::unique_lock<std::mutex> lk(sv->mu);
        sv->cv_done.wait(lk, [&] { return sv->callers == 0; });
    }
    mgx_internal_slots_destroy(sv->sl);
    delete sv;
}

}  // extern "C"
