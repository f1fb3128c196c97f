// residency.hip -- the per-token residency loop in native code: device
// routing counters, the policy's decision, asynchronous promotions and the
// publication of the mirrors, the host side moe_dual.cpp runs around the
// fused op (moe_dual.cpp:640-705 publish, 862-880 batch transport, the
// policy callbacks of policy.h:82-104).
//
// After a visible token's layers are queued on the compute stream,
// llapis_residency_token_end:
//   1. hands the promotion engine's finished jobs to the policy
//      (complete_fill / abort_fill; a READY slot marks its layer dirty);
//   2. runs the policy's per-token decision (on_token_end): its
//      fetch_external drains every layer's counters with one kernel on the
//      stream (it writes them to mapped pinned memory and zeroes them), waits
//      for the stream (the only wait of the loop: the token's kernels) and
//      pours them in; stream_expert submits a job and answers FILLING;
//      publish_layer marks the layer dirty;
//   3. publishes the dirty layers' mirrors with one kernel on the compute
//      stream that reads them from mapped pinned staging, so the next token's
//      kernels see them in stream order;
//   4. flushes the engine: the copies start after all of that, on the
//      engine's own stream, and overlap the next token.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../include/llapis_moe.h"
#include "../../include/moert_policy.h"
#include "launch.h"

struct llapis_residency {
    int L = 0, E = 0, K = 0;
    moert_policy * pol = nullptr;
    llapis_xfer * x = nullptr;
    int32_t * counts_dev = nullptr;     // [L][E] routed pairs, then [L][2] hot / other
    int32_t * counts_host = nullptr;    // pinned, mapped
    int32_t * counts_host_dev = nullptr;  // its device address
    hipStream_t cur = nullptr;          // the stream of the token_end in progress (0 is the null stream)
    bool in_call = false;               // inside token_end / refresh: the counters may be drained
    struct Mirrors {
        int32_t * es = nullptr;
        int32_t * se = nullptr;
        int32_t * ss = nullptr;
    };
    std::vector<Mirrors> mirrors;
    std::vector<char> dirty;
    int32_t * staging = nullptr;        // pinned, mapped: every layer's mirrors, [L][E + 2 K]
    const int32_t * staging_dev = nullptr;
    hipEvent_t staged = nullptr;        // after the last publication's copies
    bool staged_used = false;
    hipError_t err = hipSuccess;
    llapis_residency_stats st = {};
};

namespace {

// one launch publishes up to PUB_MAX layers: block b copies entry b's
// exp_slot [E], slot_exp [k] and slot_state [k] from the staging rows
constexpr int PUB_MAX = 64;
struct PubEntry {
    int32_t * es;
    int32_t * se;
    int32_t * ss;
    int64_t off;    // first element of the layer's staging row
    int32_t k;
    int32_t pad;
};
struct PubBatch {
    PubEntry e[PUB_MAX];
    const int32_t * staging;
    int32_t E, K;
};

__global__ __launch_bounds__(256) void k_publish_mirrors(const PubBatch b) {
    const PubEntry & m = b.e[blockIdx.x];
    const int32_t * row = b.staging + m.off;
    for (int i = threadIdx.x; i < b.E; i += blockDim.x) m.es[i] = row[i];
    for (int i = threadIdx.x; i < m.k; i += blockDim.x) {
        m.se[i] = row[b.E + i];
        m.ss[i] = row[b.E + b.K + i];
    }
}

// counters -> mapped pinned memory, then zero
__global__ __launch_bounds__(256) void k_drain_counts(int32_t * __restrict__ counts, int32_t * __restrict__ host,
                                                      int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        host[i] = counts[i];
        counts[i] = 0;
    }
}

double ms_now() {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

thread_local char g_rerr[256];
int32_t rfail(const char * msg) {
    snprintf(g_rerr, sizeof g_rerr, "%s", msg);
    return -1;
}

int32_t cb_stream_expert(void * user, int32_t il, int32_t e, int32_t slot) {
    llapis_residency * r = static_cast<llapis_residency *>(user);
    if (llapis_xfer_submit(r->x, il, e, slot) != 0) return 0;
    ++r->st.submitted;
    return 2;   // accepted asynchronously: FILLING until the copy lands
}

void cb_publish_layer(void * user, int32_t il) {
    llapis_residency * r = static_cast<llapis_residency *>(user);
    if (il >= 0 && il < r->L) r->dirty[il] = 1;
}

// every layer's counters in one copy; waits for the token on the stream
void cb_fetch_external(void * user) {
    llapis_residency * r = static_cast<llapis_residency *>(user);
    if (!r->in_call || r->err != hipSuccess) return;
    const int n = r->L * r->E + 2 * r->L;
    k_drain_counts<<<std::min(16, (n + 255) / 256), 256, 0, r->cur>>>(r->counts_dev, r->counts_host_dev, n);
    hipError_t e = hipGetLastError();
    const double t0 = ms_now();
    if (e == hipSuccess) e = hipStreamSynchronize(r->cur);
    r->st.wait_ms += ms_now() - t0;
    if (e != hipSuccess) {
        (void)hipGetLastError();
        r->err = e;
        return;
    }
    const int32_t * hits = r->counts_host + (size_t)r->L * r->E;
    for (int il = 0; il < r->L; ++il) {
        moert_policy_add_external_counts(r->pol, il, r->counts_host + (size_t)il * r->E, hits[2 * il], hits[2 * il + 1]);
        r->st.hot_pairs += hits[2 * il];
        r->st.cold_pairs += hits[2 * il + 1];
    }
    ++r->st.fetches;
}

// the dirty layers' mirrors, staged and copied in stream order
int32_t publish(llapis_residency * r, hipStream_t s, bool all) {
    if (r->staged_used && hipEventSynchronize(r->staged) != hipSuccess) {
        (void)hipGetLastError();
        return rfail("llapis_residency: staging wait failed");
    }
    const size_t per = (size_t)r->E + 2 * (size_t)r->K;
    bool any = false;
    PubBatch pb;
    pb.staging = r->staging_dev;
    pb.E = r->E;
    pb.K = r->K;
    int nb = 0;
    auto launch = [&]() {
        if (nb == 0) return true;
        k_publish_mirrors<<<nb, 256, 0, s>>>(pb);
        nb = 0;
        return hipGetLastError() == hipSuccess;
    };
    // every capacity first: a refusal leaves all dirty marks in place
    for (int il = 0; il < r->L; ++il) {
        if (!all && !r->dirty[il]) continue;
        const int k = moert_policy_layer_k(r->pol, il);
        if (k < 0 || k > r->K) return rfail("llapis_residency: layer capacity above the runtime's staging");
    }
    for (int il = 0; il < r->L; ++il) {
        if (!all && !r->dirty[il]) continue;
        r->dirty[il] = 0;
        const llapis_residency::Mirrors & m = r->mirrors[il];
        if (!m.es || !m.se || !m.ss) continue;
        const int k = moert_policy_layer_k(r->pol, il);
        int32_t * b = r->staging + (size_t)il * per;
        memcpy(b, moert_policy_exp_slot_view(r->pol, il), (size_t)r->E * 4);
        memcpy(b + r->E, moert_policy_slot_exp_view(r->pol, il), (size_t)k * 4);
        memcpy(b + r->E + r->K, moert_policy_slot_state_view(r->pol, il), (size_t)k * 4);
        pb.e[nb++] = PubEntry{m.es, m.se, m.ss, (int64_t)il * (int64_t)per, k, 0};
        if (nb == PUB_MAX && !launch()) return rfail("llapis_residency: publication launch failed");
        ++r->st.publications;
        any = true;
    }
    if (!launch()) return rfail("llapis_residency: publication launch failed");
    if (any) {
        if (hipEventRecord(r->staged, s) != hipSuccess) {
            (void)hipGetLastError();
            return rfail("llapis_residency: event record failed");
        }
        r->staged_used = true;
    }
    return 0;
}

}  // namespace

extern "C" {

const char * llapis_residency_last_error(void) { return g_rerr; }

llapis_residency * llapis_residency_create(const moert_policy_config * cfg, int32_t copy_wgs) {
    if (!cfg || cfg->n_layers <= 0 || cfg->n_expert <= 0 || cfg->k <= 0) {
        rfail("llapis_residency_create: bad geometry");
        return nullptr;
    }
    int kmax = cfg->k;
    if (cfg->k_per_layer)
        for (int il = 0; il < cfg->n_layers; ++il) kmax = std::max(kmax, cfg->k_per_layer[il]);
    llapis_residency * r = new llapis_residency();
    r->L = cfg->n_layers;
    r->E = cfg->n_expert;
    r->K = kmax;
    moert_policy_callbacks cb = {cb_stream_expert, cb_publish_layer, cb_fetch_external, r};
    r->pol = moert_policy_create(cfg, &cb);
    r->x = r->pol ? llapis_xfer_create(r->L, r->E, r->K, copy_wgs) : nullptr;
    const size_t n = (size_t)r->L * r->E + 2 * (size_t)r->L;
    bool ok = r->pol && r->x && hipMalloc((void **)&r->counts_dev, n * 4) == hipSuccess &&
              hipMemset(r->counts_dev, 0, n * 4) == hipSuccess &&
              hipHostMalloc((void **)&r->counts_host, n * 4, hipHostMallocMapped) == hipSuccess &&
              hipHostGetDevicePointer((void **)&r->counts_host_dev, r->counts_host, 0) == hipSuccess &&
              hipHostMalloc((void **)&r->staging, (size_t)r->L * (r->E + 2 * (size_t)r->K) * 4,
                            hipHostMallocMapped) == hipSuccess &&
              hipHostGetDevicePointer((void **)&r->staging_dev, r->staging, 0) == hipSuccess &&
              hipEventCreateWithFlags(&r->staged, hipEventDisableTiming) == hipSuccess;
    if (!ok) {
        (void)hipGetLastError();
        rfail("llapis_residency_create: policy, engine or device buffers could not be created");
        llapis_residency_free(r);
        return nullptr;
    }
    moert_policy_set_external_observation(r->pol, 1);
    r->mirrors.resize(r->L);
    r->dirty.assign(r->L, 0);
    return r;
}

void llapis_residency_free(llapis_residency * r) {
    if (!r) return;
    if (r->x) llapis_xfer_free(r->x);           // waits for its copies
    if (r->staged) {
        (void)hipEventSynchronize(r->staged);
        (void)hipEventDestroy(r->staged);
    }
    if (r->counts_dev) (void)hipFree(r->counts_dev);
    if (r->counts_host) (void)hipHostFree(r->counts_host);
    if (r->staging) (void)hipHostFree(r->staging);
    if (r->pol) moert_policy_free(r->pol);
    delete r;
}

moert_policy * llapis_residency_policy(llapis_residency * r) { return r ? r->pol : nullptr; }
llapis_xfer * llapis_residency_xfer(llapis_residency * r) { return r ? r->x : nullptr; }

int32_t llapis_residency_set_mirrors(llapis_residency * r, int32_t il, int32_t * exp_slot, int32_t * slot_exp,
                                     int32_t * slot_state) {
    if (!r || il < 0 || il >= r->L || !exp_slot || !slot_exp || !slot_state)
        return rfail("llapis_residency_set_mirrors: bad arguments");
    r->mirrors[il] = {exp_slot, slot_exp, slot_state};
    return 0;
}

int32_t llapis_residency_counters(llapis_residency * r, int32_t il, int32_t ** counts, int32_t ** hits) {
    if (!r || il < 0 || il >= r->L || !counts || !hits) return rfail("llapis_residency_counters: bad arguments");
    *counts = r->counts_dev + (size_t)il * r->E;
    *hits = r->counts_dev + (size_t)r->L * r->E + 2 * (size_t)il;
    return 0;
}

int32_t llapis_residency_publish_all(llapis_residency * r, void * stream) {
    if (!r) return rfail("llapis_residency_publish_all: null runtime");
    return publish(r, (hipStream_t)stream, true);
}

}  // extern "C"

namespace {

// steps 1-4 around one decision: on_token_end (reason < 0) or refresh(reason)
int32_t decide(llapis_residency * r, void * stream, int32_t reason) {
    const double t_in = ms_now(), w_in = r->st.wait_ms;
    hipStream_t s = (hipStream_t)stream;
    // 1. finished promotions
    llapis_xfer_done done[256];
    for (int32_t n; (n = llapis_xfer_take_done(r->x, done, 256)) > 0;) {
        for (int32_t i = 0; i < n; ++i) {
            const llapis_xfer_done & d = done[i];
            if (d.ok ? moert_policy_complete_fill(r->pol, d.il, d.slot, d.e)
                     : moert_policy_abort_fill(r->pol, d.il, d.slot, d.e)) {
                r->dirty[d.il] = 1;
                if (d.ok) ++r->st.completed;
            }
        }
    }
    // 2. the decision (pulls the counters through fetch_external)
    r->cur = s;
    r->in_call = true;
    if (reason < 0) moert_policy_on_token_end(r->pol);
    else moert_policy_refresh(r->pol, reason);
    r->in_call = false;
    if (r->err != hipSuccess) {
        r->err = hipSuccess;
        return rfail("llapis_residency: counter drain failed");
    }
    if (reason < 0) ++r->st.tokens;
    // 3. publication, 4. the copies
    if (publish(r, s, false) != 0) return -1;
    if (llapis_xfer_flush(r->x, stream) != 0) return rfail(llapis_xfer_last_error());
    r->st.host_ms += (ms_now() - t_in) - (r->st.wait_ms - w_in);
    return 0;
}

}  // namespace

extern "C" {

int32_t llapis_residency_token_end(llapis_residency * r, void * stream) {
    if (!r) return rfail("llapis_residency_token_end: null runtime");
    return decide(r, stream, -1);
}

int32_t llapis_residency_refresh(llapis_residency * r, int32_t reason, void * stream) {
    if (!r) return rfail("llapis_residency_refresh: null runtime");
    if (reason < 0) return rfail("llapis_residency_refresh: bad reason");
    return decide(r, stream, reason);
}

void llapis_residency_get_stats(llapis_residency * r, llapis_residency_stats * out) {
    if (!out) return;
    memset(out, 0, sizeof(*out));
    if (r) *out = r->st;
}

}  // extern "C"
