// transfer.hip -- moving expert pages into hot slots.
//
//  * The island's batch transport (moert_cuda_dir_init/async/mark/poll,
//    moert_cuda_publish_h2d, moert_cuda_dir_stats_get; cuda.h:246-272,
//    ffn_moe.cu:521-690): copies are issued at once on a side stream of
//    default priority; completion is an event per mark, polled, never waited
//    for unless asked.  Device and pinned sources are copied in place; a
//    pageable source of at most 4 KiB is staged through a pinned ring, a larger
//    pageable one is refused (the caller copies it itself).  sm_blocks > 0
//    selects the copy kernel below (that many workgroups, so the copies leave
//    the rest of the CUs to the decode kernels) for device sources.
//  * The early-decision gate (moert_cuda_dir_gate, ffn_moe.cu:506-518,
//    693-745): the last MoE op of a layer records an event on the compute
//    stream; a gated copy waits on the host until the decode reached it, then
//    the copy stream waits on that event on the device.
//  * The promotion engine (llapis_xfer_*): the job of moe_xfer plus the
//    memmgr's promote (src/moe_xfer.hpp:55-110, memmgr.h:147-158) when both
//    tiers live in HBM.  flush() issues every pending job's page copies on a
//    side stream as copy kernels of a bounded number of workgroups (one launch
//    per 96 page runs), ordered after everything already queued on the
//    compute stream by an event (this is what the reference's worker thread,
//    read staging and host gate provide); completion is an event per flush,
//    polled by take_done().
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <mutex>
#include <vector>

#include "../../include/llapis_moe.h"
#include "device.h"
#include "launch.h"

using namespace llapis;

#define MOERT_HIP_CHECK(expr)                                                                       \
    do {                                                                                            \
        const hipError_t err_ = (expr);                                                             \
        if (err_ != hipSuccess) {                                                                   \
            fprintf(stderr, "moert/hip: HIP error %s at %s:%d: %s\n", hipGetErrorName(err_), __FILE__, \
                    __LINE__, hipGetErrorString(err_));                                             \
            abort();                                                                                \
        }                                                                                           \
    } while (0)

namespace {

constexpr int COPY_WG = 256;
constexpr int MAX_RUNS = LLAPIS_XFER_MAX_GROUPS;
constexpr int BATCH_RUNS = 96;             // byte runs per launch (kernel arguments < 4 KiB)
constexpr uint64_t CHUNK = 65536;          // bytes one workgroup copies at a time

struct CopyRun {
    const uint8_t * src;
    uint8_t * dst;
    uint64_t n;
};
// Up to BATCH_RUNS runs cut into CHUNK-byte chunks; first[r] is the index of
// run r's first chunk, first[n_runs] the number of chunks.
struct CopyBatch {
    CopyRun run[BATCH_RUNS];
    uint32_t first[BATCH_RUNS + 1];
    int n_runs;
};

// Workgroup w copies chunks w, w + gridDim.x, ... (the grid is the number of
// workgroups the copies may occupy).  A chunk of a 16-byte aligned run whose
// length is a multiple of 16 moves as 128-bit loads, four in flight per lane;
// anything else (a 4-byte scale page) byte by byte.
__global__ __launch_bounds__(COPY_WG) void k_page_copy(const CopyBatch b) {
    const uint32_t total = b.first[b.n_runs];
    for (uint32_t c = blockIdx.x; c < total; c += gridDim.x) {
        int r = 0;
        while (r + 1 < b.n_runs && b.first[r + 1] <= c) ++r;
        const CopyRun run = b.run[r];
        const uint64_t off = (uint64_t)(c - b.first[r]) * CHUNK;
        const uint64_t n = min(CHUNK, run.n - off);
        const uint8_t * src = run.src + off;
        uint8_t * dst = run.dst + off;
        if ((((uintptr_t)src | (uintptr_t)dst | n) & 15) == 0) {
            const dev::u32x4 * s = (const dev::u32x4 *)src;
            dev::u32x4 * d = (dev::u32x4 *)dst;
            const int n16 = (int)(n >> 4);
            int i = threadIdx.x;
            for (; i + 3 * COPY_WG < n16; i += 4 * COPY_WG) {
                const dev::u32x4 a0 = s[i], a1 = s[i + COPY_WG], a2 = s[i + 2 * COPY_WG], a3 = s[i + 3 * COPY_WG];
                d[i] = a0;
                d[i + COPY_WG] = a1;
                d[i + 2 * COPY_WG] = a2;
                d[i + 3 * COPY_WG] = a3;
            }
            for (; i < n16; i += COPY_WG) d[i] = s[i];
        } else {
            for (int i = threadIdx.x; i < (int)n; i += COPY_WG) dst[i] = src[i];
        }
    }
}

enum SrcKind { SRC_PAGEABLE = 0, SRC_PINNED = 1, SRC_DEVICE = 2 };

SrcKind src_kind(const void * p) {
    hipPointerAttribute_t a;
    if (hipPointerGetAttributes(&a, p) != hipSuccess) {
        (void)hipGetLastError();
        return SRC_PAGEABLE;
    }
    if (a.type == hipMemoryTypeDevice || a.type == hipMemoryTypeManaged) return SRC_DEVICE;
    if (a.type == hipMemoryTypeHost) return SRC_PINNED;
    return SRC_PAGEABLE;
}

// Collects runs and launches one copy kernel per BATCH_RUNS of them.
struct Batcher {
    CopyBatch b = {};
    int wgs;
    hipStream_t s;
    hipError_t err = hipSuccess;
    Batcher(int wgs_, hipStream_t s_) : wgs(wgs_), s(s_) {}
    void add(const uint8_t * src, uint8_t * dst, uint64_t n) {
        if (!n) return;
        if (b.n_runs == BATCH_RUNS) (void)launch();
        b.first[b.n_runs + 1] = b.first[b.n_runs] + (uint32_t)((n + CHUNK - 1) / CHUNK);
        b.run[b.n_runs++] = {src, dst, n};
    }
    hipError_t launch() {
        if (b.n_runs > 0 && err == hipSuccess) {
            const uint32_t chunks = b.first[b.n_runs];
            const int grid = (int)std::max<uint32_t>(1, std::min<uint32_t>((uint32_t)wgs, chunks));
            hipLaunchKernelGGL(k_page_copy, dim3(grid), dim3(COPY_WG), 0, s, b);
            err = hipGetLastError();
        }
        b.n_runs = 0;
        b.first[0] = 0;
        return err;
    }
};

// ------------------------------------------------------- batch transport

struct Transport {
    bool on = false;
    int wgs = 0;                 // copy-kernel workgroups (0: hipMemcpyAsync)
    hipStream_t st = nullptr;
    std::mutex mu;
    struct Mark {
        hipEvent_t ev;
        long long id;
    };
    std::deque<Mark> marks;
    long long next_mark = 0, done_upto = -1;
    std::vector<hipEvent_t> ev_pool;
    // pinned ring for small pageable sources: fixed 4 KiB spans, each reused
    // only after the event recorded behind its copy
    static constexpr size_t SPAN = 4096;
    char * ring = nullptr;
    int n_spans = 0, head = 0;
    std::vector<hipEvent_t> span_ev;
    std::vector<bool> span_used;
    std::atomic<long long> async_copies{0}, async_marks{0}, bytes{0}, kernel_copies{0}, ring_copies{0};
    long long ring_waits = 0;
    double ring_wait_ms = 0.0, stage_ms = 0.0;

    hipEvent_t event() {
        if (ev_pool.empty()) {
            hipEvent_t e;
            MOERT_HIP_CHECK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
            return e;
        }
        hipEvent_t e = ev_pool.back();
        ev_pool.pop_back();
        return e;
    }
    // copy n <= SPAN pageable bytes into the next ring span (under mu)
    const void * stage(const void * src, size_t n) {
        const int s = head;
        head = (head + 1) % n_spans;
        if (span_used[s]) {
            const auto t0 = std::chrono::steady_clock::now();
            if (hipEventQuery(span_ev[s]) != hipSuccess) {
                (void)hipGetLastError();
                MOERT_HIP_CHECK(hipEventSynchronize(span_ev[s]));
                ++ring_waits;
                ring_wait_ms += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
            }
        }
        const auto t1 = std::chrono::steady_clock::now();
        memcpy(ring + (size_t)s * SPAN, src, n);
        stage_ms += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t1).count();
        last_span = s;
        return ring + (size_t)s * SPAN;
    }
    int last_span = -1;
} g_dir;

// residency publication: pinned staging grown on demand, its own stream
std::mutex g_pub_mu;
hipStream_t g_pub_st = nullptr;
char * g_pub_pin = nullptr;
size_t g_pub_cap = 0;
std::atomic<long long> g_pub_calls{0}, g_pub_copies{0};

// ------------------------------------------------------------------ gate

struct Gate {
    static constexpr int MAXL = 128;
    bool on = false, per_layer = false;
    int last_layer = -1;
    hipEvent_t ev[MAXL] = {};
    bool recorded[MAXL] = {};
    long long c[MAXL] = {};
    long long armed = 0;
    std::mutex mu;
    std::condition_variable cv;
    long long waits = 0, timeouts = 0;
    double wait_ms = 0.0;
} g_gate;

}  // namespace

namespace llapis {

// Called by moert_ffn_moe after a fire (ffn_moe.cu:1237-1242): the down fire
// of a gated layer records the layer's event and releases the waiters.
void dir_gate_after_fire(int il, int kind, hipStream_t stream) {
    Gate & g = g_gate;
    if (!g.on || kind != 1 || il < 0 || il > g.last_layer || !(g.per_layer || il == g.last_layer)) return;
    MOERT_HIP_CHECK(hipEventRecord(g.ev[il], stream));
    {
        std::lock_guard<std::mutex> lk(g.mu);
        g.recorded[il] = true;
        ++g.c[il];
    }
    g.cv.notify_all();
}

}  // namespace llapis

extern "C" {

int32_t moert_cuda_dir_init(int32_t sm_blocks, int32_t sm_ring_mib, int32_t) {
    Transport & d = g_dir;
    std::lock_guard<std::mutex> lk(d.mu);
    if (d.on) return 1;
    MOERT_HIP_CHECK(hipStreamCreateWithFlags(&d.st, hipStreamNonBlocking));
    d.wgs = sm_blocks > 0 ? std::min<int>(sm_blocks, 1024) : 0;
    const size_t ring_bytes = (size_t)std::max(1, (int)sm_ring_mib) << 20;
    d.n_spans = (int)(ring_bytes / Transport::SPAN);
    MOERT_HIP_CHECK(hipHostMalloc((void **)&d.ring, ring_bytes, hipHostMallocDefault));
    d.span_ev.resize(d.n_spans);
    d.span_used.assign(d.n_spans, false);
    for (auto & e : d.span_ev) MOERT_HIP_CHECK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    d.on = true;
    fprintf(stderr, "moert/hip: batch transport on: copies issued at once on a side stream (%s), completion polled\n",
            d.wgs ? "copy kernel for device sources" : "hipMemcpyAsync");
    return 1;
}

int32_t moert_cuda_dir_async(void * dst_dev, const void * src, uint64_t nbytes) {
    Transport & d = g_dir;
    if (!d.on || !dst_dev || !src || !nbytes) return 0;
    const SrcKind k = src_kind(src);
    if (k == SRC_PAGEABLE && nbytes > Transport::SPAN) return 0;
    std::lock_guard<std::mutex> lk(d.mu);
    if (k == SRC_PAGEABLE) {
        src = d.stage(src, (size_t)nbytes);
        MOERT_HIP_CHECK(hipMemcpyAsync(dst_dev, src, (size_t)nbytes, hipMemcpyHostToDevice, d.st));
        MOERT_HIP_CHECK(hipEventRecord(d.span_ev[d.last_span], d.st));
        d.span_used[d.last_span] = true;
        ++d.ring_copies;
    } else if (k == SRC_DEVICE && d.wgs > 0) {
        Batcher bt(d.wgs, d.st);
        bt.add((const uint8_t *)src, (uint8_t *)dst_dev, nbytes);
        MOERT_HIP_CHECK(bt.launch());
        ++d.kernel_copies;
    } else {
        MOERT_HIP_CHECK(hipMemcpyAsync(dst_dev, src, (size_t)nbytes, hipMemcpyDefault, d.st));
    }
    ++d.async_copies;
    d.bytes += (long long)nbytes;
    return 1;
}

int64_t moert_cuda_dir_mark(void) {
    Transport & d = g_dir;
    if (!d.on) return -1;
    std::lock_guard<std::mutex> lk(d.mu);
    hipEvent_t e = d.event();
    MOERT_HIP_CHECK(hipEventRecord(e, d.st));
    d.marks.push_back({e, d.next_mark});
    ++d.async_marks;
    return d.next_mark++;
}

int64_t moert_cuda_dir_poll(int32_t wait_all) {
    Transport & d = g_dir;
    if (!d.on) return -1;
    std::lock_guard<std::mutex> lk(d.mu);
    if (wait_all) MOERT_HIP_CHECK(hipStreamSynchronize(d.st));
    while (!d.marks.empty()) {
        const hipError_t e = hipEventQuery(d.marks.front().ev);
        if (e == hipErrorNotReady) {
            (void)hipGetLastError();
            break;
        }
        MOERT_HIP_CHECK(e);
        d.done_upto = d.marks.front().id;
        d.ev_pool.push_back(d.marks.front().ev);
        d.marks.pop_front();
    }
    return d.done_upto;
}

int32_t moert_cuda_publish_h2d(int32_t n, void * const * dsts, const void * const * srcs, const uint64_t * sizes) {
    if (n <= 0) return 1;
    std::lock_guard<std::mutex> lk(g_pub_mu);
    if (!g_pub_st) MOERT_HIP_CHECK(hipStreamCreateWithFlags(&g_pub_st, hipStreamNonBlocking));
    size_t tot = 0;
    for (int32_t i = 0; i < n; ++i) tot += ((size_t)sizes[i] + 63) & ~(size_t)63;
    if (tot > g_pub_cap) {
        if (g_pub_pin) MOERT_HIP_CHECK(hipHostFree(g_pub_pin));
        g_pub_cap = std::max(tot, (size_t)256 << 10);
        MOERT_HIP_CHECK(hipHostMalloc((void **)&g_pub_pin, g_pub_cap, hipHostMallocDefault));
    }
    // the views are pageable and may change after the call: stage, copy in
    // stream order, then wait until every copy landed
    size_t off = 0;
    for (int32_t i = 0; i < n; ++i) {
        if (!sizes[i]) continue;
        memcpy(g_pub_pin + off, srcs[i], (size_t)sizes[i]);
        MOERT_HIP_CHECK(hipMemcpyAsync(dsts[i], g_pub_pin + off, (size_t)sizes[i], hipMemcpyHostToDevice, g_pub_st));
        off += ((size_t)sizes[i] + 63) & ~(size_t)63;
    }
    MOERT_HIP_CHECK(hipStreamSynchronize(g_pub_st));
    ++g_pub_calls;
    g_pub_copies += n;
    return 1;
}

void moert_cuda_dir_stats_get(moert_cuda_dir_stats * out) {
    if (!out) return;
    memset(out, 0, sizeof(*out));
    Transport & d = g_dir;
    out->async_copies = d.async_copies.load();
    out->async_marks = d.async_marks.load();
    out->bytes = d.bytes.load();
    out->pub_calls = g_pub_calls.load();
    out->pub_copies = g_pub_copies.load();
    out->sm_copies = d.kernel_copies.load();
    std::lock_guard<std::mutex> lk(d.mu);
    out->sm_ring_copies = d.ring_copies.load();
    out->sm_ring_waits = d.ring_waits;
    out->sm_ring_wait_ms = d.ring_wait_ms;
    out->sm_stage_ms = d.stage_ms;
}

int64_t moert_cuda_dir_gate(int32_t op, int64_t arg) {
    Gate & g = g_gate;
    switch (op) {
        case 0: {  // enable: arg = last MoE layer | per_layer << 16
            const int ll = (int)(arg & 0xffff);
            if (ll < 0 || ll >= Gate::MAXL) return 0;
            std::lock_guard<std::mutex> lk(g.mu);
            for (int l = 0; l <= ll; ++l)
                if (!g.ev[l]) MOERT_HIP_CHECK(hipEventCreateWithFlags(&g.ev[l], hipEventDisableTiming));
            g.last_layer = ll;
            g.per_layer = (arg >> 16) != 0;
            g.on = true;
            return 1;
        }
        case 1: {  // arm: the target a copy decided from now on waits for
            std::lock_guard<std::mutex> lk(g.mu);
            long long m = 0;
            for (int l = 0; l <= g.last_layer; ++l)
                if (g.per_layer || l == g.last_layer) m = std::max(m, g.c[l]);
            g.armed = m + 1;
            return g.armed;
        }
        case 2: {  // wait: arg = layer << 40 | target
            const long long target = arg & ((1LL << 40) - 1);
            int l = (int)(arg >> 40);
            if (!g.on || target <= 0) return 0;
            if (!g.per_layer || l < 0 || l > g.last_layer) l = g.last_layer;
            const auto t0 = std::chrono::steady_clock::now();
            bool rec = false;
            {
                std::unique_lock<std::mutex> lk(g.mu);
                if (!g.cv.wait_for(lk, std::chrono::milliseconds(2000), [&] { return g.c[l] >= target; })) ++g.timeouts;
                rec = g.recorded[l];
                ++g.waits;
                g.wait_ms += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
            }
            if (rec && g_dir.on) MOERT_HIP_CHECK(hipStreamWaitEvent(g_dir.st, g.ev[l], 0));
            return 1;
        }
        case 3: {  // open from the host: the decode returned
            {
                std::lock_guard<std::mutex> lk(g.mu);
                for (int l = 0; l <= g.last_layer; ++l) g.c[l] = std::max(g.c[l], g.armed);
            }
            g.cv.notify_all();
            return 1;
        }
        case 4: {
            std::lock_guard<std::mutex> lk(g.mu);
            if (arg == 0) return g.waits;
            if (arg == 1) return g.timeouts;
            return (int64_t)(g.wait_ms * 1000.0);
        }
        case 5:  // engine source pacing: every source already goes on the copy stream at once
            return 1;
        case 6:
            return 0;
    }
    return 0;
}

}  // extern "C"

// ------------------------------------------------------ promotion engine

struct llapis_xfer {
    int n_layers = 0, n_expert = 0, k_slots = 0, wgs = 0;
    struct Group {
        uint8_t * slab = nullptr;      // slot s at slab + s * bytes
        const uint8_t * src = nullptr; // expert e at src + e * stride
        uint64_t stride = 0, bytes = 0;
        SrcKind kind = SRC_DEVICE;
    };
    std::vector<Group> groups;         // [n_layers][MAX_RUNS]
    hipStream_t st = nullptr;
    hipEvent_t after = nullptr;
    std::mutex mu;
    // the jobs of one flush, finished when ev has completed (next = the
    // first job not yet handed out by take_done)
    struct Batch {
        std::vector<llapis_xfer_done> jobs;
        size_t next;
        hipEvent_t ev;
        bool settled;                  // finished (or failed) before it was queued: no event to query
    };
    std::vector<llapis_xfer_done> pending;
    std::deque<Batch> live;
    long long n_live = 0;              // jobs in live not yet handed out
    std::vector<hipEvent_t> ev_pool;
    llapis_xfer_stats s = {};
    Group & g(int il, int gi) { return groups[(size_t)il * MAX_RUNS + gi]; }
};

namespace {
thread_local char g_xerr[256];
int32_t xfail(const char * msg) {
    snprintf(g_xerr, sizeof g_xerr, "%s", msg);
    return -1;
}
}  // namespace

extern "C" {

const char * llapis_xfer_last_error(void) { return g_xerr; }

int32_t llapis_device_memory_mib(long long * free_mib, long long * total_mib) {
    size_t f = 0, t = 0;
    if (hipMemGetInfo(&f, &t) != hipSuccess) {
        (void)hipGetLastError();
        return xfail("llapis_device_memory_mib: hipMemGetInfo failed");
    }
    if (free_mib) *free_mib = (long long)(f >> 20);
    if (total_mib) *total_mib = (long long)(t >> 20);
    return 0;
}

llapis_xfer * llapis_xfer_create(int32_t n_layers, int32_t n_expert, int32_t k_slots, int32_t copy_wgs) {
    if (n_layers <= 0 || n_expert <= 0 || k_slots <= 0 || copy_wgs < 0) {
        xfail("llapis_xfer_create: bad geometry");
        return nullptr;
    }
    llapis_xfer * x = new llapis_xfer();
    x->n_layers = n_layers;
    x->n_expert = n_expert;
    x->k_slots = k_slots;
    x->wgs = std::min<int32_t>(copy_wgs, 4096);
    x->groups.resize((size_t)n_layers * MAX_RUNS);
    if (hipStreamCreateWithFlags(&x->st, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&x->after, hipEventDisableTiming) != hipSuccess) {
        (void)hipGetLastError();
        xfail("llapis_xfer_create: stream or event creation failed");
        delete x;
        return nullptr;
    }
    return x;
}

void llapis_xfer_free(llapis_xfer * x) {
    if (!x) return;
    (void)hipStreamSynchronize(x->st);
    for (auto & b : x->live) (void)hipEventDestroy(b.ev);
    for (auto e : x->ev_pool) (void)hipEventDestroy(e);
    (void)hipEventDestroy(x->after);
    (void)hipStreamDestroy(x->st);
    delete x;
}

int32_t llapis_xfer_set_group(llapis_xfer * x, int32_t il, int32_t group, void * slab, const void * src,
                              uint64_t src_stride, uint64_t bytes_per_expert) {
    if (!x || il < 0 || il >= x->n_layers || group < 0 || group >= MAX_RUNS)
        return xfail("llapis_xfer_set_group: layer or group out of range");
    if (!slab || !src || !bytes_per_expert || src_stride < bytes_per_expert)
        return xfail("llapis_xfer_set_group: null pointer, empty page or overlapping source stride");
    const SrcKind dk = src_kind(slab), sk = src_kind(src);
    if (dk != SRC_DEVICE) return xfail("llapis_xfer_set_group: the slab must be device memory");
    if (sk == SRC_PAGEABLE) return xfail("llapis_xfer_set_group: the source must be device or pinned host memory");
    std::lock_guard<std::mutex> lk(x->mu);
    llapis_xfer::Group & g = x->g(il, group);
    g.slab = (uint8_t *)slab;
    g.src = (const uint8_t *)src;
    g.stride = src_stride;
    g.bytes = bytes_per_expert;
    g.kind = sk;
    return 0;
}

int32_t llapis_xfer_submit(llapis_xfer * x, int32_t il, int32_t e, int32_t slot) {
    if (!x || il < 0 || il >= x->n_layers || e < 0 || e >= x->n_expert || slot < 0 || slot >= x->k_slots)
        return xfail("llapis_xfer_submit: layer, expert or slot out of range");
    std::lock_guard<std::mutex> lk(x->mu);
    x->pending.push_back({il, e, slot, 0});
    ++x->s.submitted;
    return 0;
}

int32_t llapis_xfer_flush(llapis_xfer * x, void * after_stream) {
    if (!x) return xfail("llapis_xfer_flush: null engine");
    std::lock_guard<std::mutex> lk(x->mu);
    if (x->pending.empty()) return 0;
    // the copies may overwrite slots that kernels already queued on the
    // compute stream still read: start them after that work
    if (hipEventRecord(x->after, (hipStream_t)after_stream) != hipSuccess ||
        hipStreamWaitEvent(x->st, x->after, 0) != hipSuccess) {
        (void)hipGetLastError();
        return xfail("llapis_xfer_flush: could not order the copies after the compute stream");
    }
    // the batch's completion event first: without one the jobs stay pending
    // (nothing issued, nothing lost) and the next flush tries again
    hipEvent_t ev = nullptr;
    if (x->ev_pool.empty()) {
        if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
            (void)hipGetLastError();
            return xfail("llapis_xfer_flush: event creation failed");
        }
    } else {
        ev = x->ev_pool.back();
        x->ev_pool.pop_back();
    }
    x->s.max_queue = std::max<long long>(x->s.max_queue, (long long)x->pending.size());
    // device sources: one copy kernel per BATCH_RUNS page runs; pinned
    // sources (or no copy workgroups): the runtime's asynchronous copies
    Batcher bt(x->wgs, x->st);
    bool ok = true;
    for (const llapis_xfer_done & d : x->pending) {
        for (int gi = 0; gi < MAX_RUNS; ++gi) {
            const llapis_xfer::Group & g = x->g(d.il, gi);
            if (!g.slab) continue;
            const uint8_t * src = g.src + (uint64_t)d.e * g.stride;
            uint8_t * dst = g.slab + (uint64_t)d.slot * g.bytes;
            if (g.kind == SRC_DEVICE && x->wgs > 0) {
                bt.add(src, dst, g.bytes);
            } else if (hipMemcpyAsync(dst, src, g.bytes, hipMemcpyDefault, x->st) != hipSuccess) {
                (void)hipGetLastError();
                ok = false;
            }
            x->s.bytes += (long long)g.bytes;
        }
    }
    if (bt.launch() != hipSuccess) {
        (void)hipGetLastError();
        ok = false;
    }
    llapis_xfer::Batch b = {std::move(x->pending), 0, ev, false};
    x->pending.clear();
    for (auto & d : b.jobs) d.ok = ok ? 1 : 0;
    int32_t rc = 0;
    if (hipEventRecord(b.ev, x->st) != hipSuccess) {
        // the copies are issued but cannot be tracked: wait for the stream,
        // then hand the jobs out as failed, so their slots are released
        (void)hipGetLastError();
        if (hipStreamSynchronize(x->st) != hipSuccess) (void)hipGetLastError();
        for (auto & d : b.jobs) d.ok = 0;
        b.settled = true;
        rc = xfail("llapis_xfer_flush: event record failed; the batch is reported as failed");
    }
    x->n_live += (long long)b.jobs.size();
    x->live.push_back(std::move(b));
    return rc;
}

int32_t llapis_xfer_take_done(llapis_xfer * x, llapis_xfer_done * out, int32_t max_out) {
    if (!x || (!out && max_out > 0)) return xfail("llapis_xfer_take_done: null argument");
    std::lock_guard<std::mutex> lk(x->mu);
    int32_t n = 0;
    while (n < max_out && !x->live.empty()) {
        llapis_xfer::Batch & b = x->live.front();
        if (b.next == 0 && !b.settled) {   // not yet known to be finished
            const hipError_t e = hipEventQuery(b.ev);
            if (e == hipErrorNotReady) {
                (void)hipGetLastError();
                break;
            }
            if (e != hipSuccess) {
                (void)hipGetLastError();
                for (auto & d : b.jobs) d.ok = 0;
            }
        }
        while (n < max_out && b.next < b.jobs.size()) {
            const llapis_xfer_done & d = b.jobs[b.next++];
            out[n++] = d;
            --x->n_live;
            if (d.ok) ++x->s.completed;
            else ++x->s.failed;
        }
        if (b.next < b.jobs.size()) break;
        x->ev_pool.push_back(b.ev);
        x->live.pop_front();
    }
    return n;
}

int64_t llapis_xfer_in_flight(llapis_xfer * x) {
    if (!x) return 0;
    std::lock_guard<std::mutex> lk(x->mu);
    return (int64_t)x->pending.size() + x->n_live;
}

int32_t llapis_xfer_wait_idle(llapis_xfer * x, void * after_stream) {
    if (!x) return xfail("llapis_xfer_wait_idle: null engine");
    if (llapis_xfer_flush(x, after_stream) != 0) return -1;
    const auto t0 = std::chrono::steady_clock::now();
    if (hipStreamSynchronize(x->st) != hipSuccess) {
        (void)hipGetLastError();
        return xfail("llapis_xfer_wait_idle: copy stream failed");
    }
    std::lock_guard<std::mutex> lk(x->mu);
    x->s.wait_idle_calls += 1;
    x->s.wait_idle_ms += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    return 0;
}

void llapis_xfer_get_stats(llapis_xfer * x, llapis_xfer_stats * out) {
    if (!out) return;
    memset(out, 0, sizeof(*out));
    if (!x) return;
    std::lock_guard<std::mutex> lk(x->mu);
    *out = x->s;
}

}  // extern "C"
