// api.hip -- host side of the C ABI: the moert island (moert_hip.h) and the
// llapis entry points (llapis_moe.h).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>

#include "../../include/llapis_moe.h"
#include "device.h"
#include "formats.h"
#include "launch.h"

using namespace llapis;

namespace {

// The island's error contract (ffn_moe.cu:38-46): a device-API failure prints
// and aborts.
#define MOERT_HIP_CHECK(expr)                                                                       \
    do {                                                                                            \
        const hipError_t err_ = (expr);                                                             \
        if (err_ != hipSuccess) {                                                                   \
            fprintf(stderr, "moert/hip: HIP error %s at %s:%d: %s\n", hipGetErrorName(err_), __FILE__, \
                    __LINE__, hipGetErrorString(err_));                                             \
            abort();                                                                                \
        }                                                                                           \
    } while (0)

thread_local std::string g_err;

int32_t fail(const std::string & msg) {
    g_err = msg;
    return -1;
}

#define LL_TRY(expr)                                                                 \
    do {                                                                             \
        const hipError_t e_ = (expr);                                                \
        if (e_ != hipSuccess) return fail(std::string(#expr) + ": " + hipGetErrorString(e_)); \
    } while (0)

std::atomic<int> g_decode_path{1}, g_prefill{1}, g_dn_rows_log2{-1}, g_dn_by_group{-1}, g_fused_fire{1};

// the largest LDS allocation of one workgroup on the current device (cached)
int max_lds_per_wg() {
    static std::mutex mu;
    static std::map<int, int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 65536;
    std::lock_guard<std::mutex> lk(mu);
    auto it = cache.find(dev);
    if (it != cache.end()) return it->second;
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0) v = 65536;
    cache[dev] = v;
    return v;
}

std::atomic<int> g_act_mode{LLAPIS_ACT_CPU};
std::atomic<int> g_gelu_mode{LLAPIS_GELU_TABLE};

moert_cuda_config g_cfg = [] {
    moert_cuda_config c;
    moert_cuda_config_defaults(&c);
    return c;
}();

// device routing counters: [n_layers][n_expert] then [n_layers][2]
struct RouteCounters {
    int32_t * dev = nullptr;
    int32_t nl = 0, ne = 0;
    bool on = false;
    size_t n_ints() const { return (size_t)nl * ne + (size_t)nl * 2; }
} g_rc;
std::mutex g_rc_mu;

std::atomic<long long> g_fires{0}, g_op_ns{0};

struct HotTable {
    const void * const * ptrs = nullptr;
    int32_t n = 0, type = 0;
};
HotTable g_hot_tab[128][2];

long long now_ns() {
    return std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

bool is_gu_type(int t) { return t == T_Q4_K || t == T_IQ2_S; }
bool is_dn_type(int t) { return t == T_Q5_0 || t == T_IQ4_NL; }
bool supported_w(int t) { return is_gu_type(t) || is_dn_type(t); }

uint64_t rbytes(int t, int64_t n) { return (n % blk_elems(t)) ? 0 : row_bytes(t, n); }

}  // namespace

extern "C" {

const char * llapis_last_error(void) { return g_err.c_str(); }

void llapis_set_modes(int32_t act_mode, int32_t gelu_mode) {
    g_act_mode = act_mode == LLAPIS_ACT_Q8_1 ? LLAPIS_ACT_Q8_1 : LLAPIS_ACT_CPU;
    g_gelu_mode = gelu_mode == LLAPIS_GELU_TANH ? LLAPIS_GELU_TANH : LLAPIS_GELU_TABLE;
}

// ------------------------------------------------------------ mm service

int32_t llapis_mul_mat_id(const moert_mm_call * c, int32_t w_type, const void * w_base, int64_t w_n, int32_t d_in,
                          int32_t d_out, void * stream) {
    if (!c) return fail("llapis_mul_mat_id: null call");
    if (!supported_w(w_type)) return fail("llapis_mul_mat_id: unsupported weight type " + std::to_string(w_type));
    const uint64_t rb = rbytes(w_type, d_in);
    if (!rb || d_in > dev::MAX_D_IN) return fail("llapis_mul_mat_id: d_in does not fit the format");
    const uint64_t eb = rb * (uint64_t)d_out;
    if (eb % 16) return fail("llapis_mul_mat_id: expert slab is not a multiple of 16 bytes");
    if (c->n_ids <= 0) return 0;
    if (c->b_ncols != 1 && c->b_ncols != c->n_ids) return fail("llapis_mul_mat_id: b_ncols must be 1 or n_ids");
    // the fire kernels where the format and size allow (one workgroup per
    // (rows, channel), the channel's column quantised in LDS, every load of a
    // round issued together); a per-expert pointer table takes the generic one
    const bool k256 = (w_type == T_Q4_K || w_type == T_IQ2_S) && d_in % 256 == 0 && d_in <= 3072;
    const bool k32 = (w_type == T_Q5_0 || w_type == T_IQ4_NL) && d_in % 64 == 0 && d_in <= 1024;
    if (g_fused_fire.load() && (k256 || k32) && !c->w_ptrs && w_n <= INT32_MAX && c->n_ids <= INT32_MAX) {
        FireParams f = {};
        f.kind = k256 ? 0 : 1;
        f.d_in = d_in; f.d_out = d_out; f.n_used = 1; f.n_tokens = (int)c->n_ids; f.ids_s1 = 1;
        f.n_expert = (int)w_n; f.k_slots = 0;
        f.cur = static_cast<const float *>(c->b);
        f.cur_shared = c->b_ncols == 1;
        f.ids = static_cast<const int32_t *>(c->ids);
        f.hot = f.cold = static_cast<const uint8_t *>(w_base);
        f.hot_stride = f.cold_stride = eb;
        f.dst = static_cast<float *>(c->y);
        f.n_live = c->ne_live;
        f.w_lds = dev::align16(dev::fire_gu_rows(d_in) * (int)rb + 32);
        if (fire_lds(f, w_type, w_type) + 16 * 1024 <= max_lds_per_wg()) {
            LL_TRY(launch_fire(f, w_type, w_type, g_act_mode.load(), (hipStream_t)stream));
            return 0;
        }
    }
    MmvParams p = {};
    p.mode = MMV_COMPACT;
    p.d_in = d_in;
    p.d_out = d_out;
    p.w0 = static_cast<const uint8_t *>(w_base);
    p.stride0 = eb;
    p.ptrs0 = c->w_ptrs;
    p.n0 = w_n;
    p.ids = static_cast<const int32_t *>(c->ids);
    p.ne_live = c->ne_live;
    p.b_ncols = (int)c->b_ncols;
    p.act = static_cast<const float *>(c->b);
    p.act_ld = d_in;
    p.y = static_cast<float *>(c->y);
    mmv_prepare(p, w_type, w_type);
    LL_TRY(launch_mmv(p, w_type, w_type, g_act_mode.load(), dev::SRC_PLAIN, (int)c->n_ids, (hipStream_t)stream));
    return 0;
}

// --------------------------------------------------------------- island

void moert_cuda_configure(const moert_cuda_config * cfg) {
    if (cfg) g_cfg = *cfg;
}

int32_t moert_cuda_route_counts_enable(int32_t n_layers, int32_t n_expert) {
    if (n_layers <= 0 || n_expert <= 0) return 0;
    std::lock_guard<std::mutex> lk(g_rc_mu);
    if (g_rc.on && g_rc.nl == n_layers && g_rc.ne == n_expert) return 1;
    if (g_rc.dev) {
        MOERT_HIP_CHECK(hipFree(g_rc.dev));
        g_rc.dev = nullptr;
        g_rc.on = false;
    }
    g_rc.nl = n_layers;
    g_rc.ne = n_expert;
    const size_t bytes = g_rc.n_ints() * sizeof(int32_t);
    if (hipMalloc(&g_rc.dev, bytes) != hipSuccess) {
        (void)hipGetLastError();
        g_rc.nl = g_rc.ne = 0;
        g_rc.dev = nullptr;
        return 0;
    }
    MOERT_HIP_CHECK(hipMemset(g_rc.dev, 0, bytes));
    g_rc.on = true;
    return 1;
}

int32_t moert_cuda_route_counts_fetch(int32_t * dst, int32_t reset) {
    std::lock_guard<std::mutex> lk(g_rc_mu);
    if (!g_rc.on || !dst) return 0;
    const size_t n = g_rc.n_ints();
    MOERT_HIP_CHECK(hipDeviceSynchronize());
    MOERT_HIP_CHECK(hipMemcpy(dst, g_rc.dev, n * sizeof(int32_t), hipMemcpyDeviceToHost));
    if (reset) MOERT_HIP_CHECK(hipMemset(g_rc.dev, 0, n * sizeof(int32_t)));
    return (int32_t)n;
}

int32_t moert_cuda_host_register_pinned(void *, uint64_t) { return 0; }
void moert_cuda_host_unregister(void *) {}
int32_t moert_cuda_host_register_mapped(void *, uint64_t) { return 0; }
void * moert_cuda_host_map(void *, uint64_t) { return nullptr; }

void moert_cuda_stats_get(moert_cuda_stats * out) {
    if (!out) return;
    memset(out, 0, sizeof(*out));
    out->fires = g_fires.load();
    out->op_host_ns = g_op_ns.load();
}

// the batch transport and the early-decision gate are in transfer.hip

void moert_cuda_set_hot_table(int32_t il, int32_t kind, const void * const * dev_ptrs, int32_t n, int32_t type_tag) {
    if (il < 0 || il >= 128 || kind < 0 || kind > 1) return;
    g_hot_tab[il][kind].ptrs = n > 0 ? dev_ptrs : nullptr;
    g_hot_tab[il][kind].n = n > 0 ? n : 0;
    g_hot_tab[il][kind].type = type_tag;
}

// One (layer, kind) fire (ffn_moe.cu:892-1246 with the cold pool in HBM):
// partition -> [gather] -> hot mm -> cold mm -> scatter, scratch from the
// host's LIFO pool in a fixed order and released in reverse.
void moert_ffn_moe(const moert_ffn_moe_args * a, const moert_ffn_moe_host * h) {
    const long long t0 = now_ns();
    const int kind = a->kind;
    const int n_used = a->n_used, n_tokens = a->n_tokens;
    const int Pmax = n_used * n_tokens;
    const int D_in = a->d_in, D_out = a->d_out;
    hipStream_t stream = (hipStream_t)a->stream;
    if (a->planc_mode != 0 || !a->has_w_cold) {
        fprintf(stderr, "moert/hip: planc_mode %d / has_w_cold %d: only an HBM-resident cold pool is supported\n",
                a->planc_mode, a->has_w_cold);
        abort();
    }
    if (Pmax <= 0 || Pmax > MOERT_COLDCPU_GS_PMAX_MAX) {
        fprintf(stderr, "moert/hip: %d routed pairs per fire (max %d)\n", Pmax, MOERT_COLDCPU_GS_PMAX_MAX);
        abort();
    }
    const bool gather_x = (kind != 0 || n_tokens > 1);

    void * scratch[16];
    int n_scratch = 0;
    auto pool_alloc = [&](uint64_t nbytes) -> void * {
        void * p = h->pool_alloc(h->user, nbytes);
        scratch[n_scratch++] = p;
        return p;
    };
    float * x_hot = (float *)pool_alloc((uint64_t)D_in * Pmax * sizeof(float));
    float * x_cold = (float *)pool_alloc((uint64_t)D_in * Pmax * sizeof(float));
    int32_t * ids_hot = (int32_t *)pool_alloc((uint64_t)Pmax * sizeof(int32_t));
    int32_t * ids_cold = (int32_t *)pool_alloc((uint64_t)Pmax * sizeof(int32_t));
    int32_t * hot_dst = (int32_t *)pool_alloc((uint64_t)Pmax * sizeof(int32_t));
    int32_t * cold_dst = (int32_t *)pool_alloc((uint64_t)Pmax * sizeof(int32_t));
    int32_t * counts = (int32_t *)pool_alloc(2 * sizeof(int32_t));
    float * y_hot = (float *)pool_alloc((uint64_t)D_out * Pmax * sizeof(float));
    float * y_cold = (float *)pool_alloc((uint64_t)D_out * Pmax * sizeof(float));

    int32_t * rc_counts = nullptr, * rc_hits = nullptr;
    if (g_rc.on && kind == 0 && a->il >= 0 && a->il < g_rc.nl) {
        rc_counts = g_rc.dev + (size_t)a->il * g_rc.ne;
        rc_hits = g_rc.dev + (size_t)g_rc.nl * g_rc.ne + (size_t)a->il * 2;
    }
    if (!g_cfg.counted) {          // padded channels read id 0 and, when gathered, x = 0
        MOERT_HIP_CHECK(hipMemsetAsync(ids_hot, 0, (size_t)Pmax * sizeof(int32_t), stream));
        MOERT_HIP_CHECK(hipMemsetAsync(ids_cold, 0, (size_t)Pmax * sizeof(int32_t), stream));
        if (gather_x) {
            MOERT_HIP_CHECK(hipMemsetAsync(x_hot, 0, (size_t)D_in * Pmax * sizeof(float), stream));
            MOERT_HIP_CHECK(hipMemsetAsync(x_cold, 0, (size_t)D_in * Pmax * sizeof(float), stream));
        }
    }
    MOERT_HIP_CHECK(launch_partition((const int32_t *)a->ids, n_used, a->ids_s1, Pmax, (const int32_t *)a->exp_slot,
                                     (const int32_t *)a->slot_exp, (const int32_t *)a->slot_state, a->n_expert, a->k,
                                     ids_hot, ids_cold, hot_dst, cold_dst, counts, rc_counts, rc_hits, stream));
    if (gather_x)
        MOERT_HIP_CHECK(launch_gather((const float *)a->cur, D_in, kind, n_used, counts, hot_dst, cold_dst, x_hot,
                                      x_cold, Pmax, stream));
    const int32_t * ne_hot = g_cfg.counted ? counts : nullptr;
    const int32_t * ne_cold = g_cfg.counted ? counts + 1 : nullptr;
    {
        moert_mm_call c = {};
        c.w_sel = MOERT_MM_W_HOT;
        if (a->il >= 0 && a->il < 128 && (kind == 0 || kind == 1)) {
            const HotTable & ht = g_hot_tab[a->il][kind];
            if (ht.ptrs && ht.n == a->k) {
                c.w_sel = MOERT_MM_W_RAW;
                c.w_type_tag = ht.type;
                c.w_n = a->k;
                c.w_ptrs = ht.ptrs;
                c.w_data = (const void *)ht.ptrs;
            }
        }
        c.b = gather_x ? (const void *)x_hot : a->cur;
        c.b_ncols = gather_x ? Pmax : 1;
        c.ids = ids_hot;
        c.n_ids = Pmax;
        c.y = y_hot;
        c.ne_live = ne_hot;
        h->mm(h->user, &c);
    }
    {
        moert_mm_call c = {};
        c.w_sel = MOERT_MM_W_COLD_SRC;
        c.b = gather_x ? (const void *)x_cold : a->cur;
        c.b_ncols = gather_x ? Pmax : 1;
        c.ids = ids_cold;
        c.n_ids = Pmax;
        c.y = y_cold;
        c.ne_live = ne_cold;
        h->mm(h->user, &c);
    }
    MOERT_HIP_CHECK(launch_scatter(y_hot, y_cold, D_out, kind, counts, ids_hot, hot_dst, ids_cold, cold_dst,
                                   (const float *)a->s_hot, (const float *)a->s_cold, (float *)a->dst, Pmax, stream));
    for (int i = n_scratch - 1; i >= 0; --i) h->pool_free(h->user, scratch[i]);
    dir_gate_after_fire(a->il, kind, stream);
    g_op_ns += now_ns() - t0;
    ++g_fires;
}

}  // extern "C"

// ---------------------------------------------------------- trampoline

namespace {

// LIFO bump allocator over the caller's workspace (the ggml pool contract:
// frees in exact reverse order of allocation within one fire).
struct HostCtx {
    uint8_t * base = nullptr;
    uint64_t cap = 0, top = 0;
    struct Rec { void * p; uint64_t prev_top; } stack[16];
    int n = 0;
    const llapis_tensor * w_hot = nullptr;
    const llapis_tensor * w_cold = nullptr;
    int32_t d_in = 0, d_out = 0;
    bool failed = false;
};

void * host_pool_alloc(void * user, uint64_t nbytes) {
    HostCtx * hc = (HostCtx *)user;
    const uint64_t at = (hc->top + 255) & ~uint64_t(255);
    if (hc->n >= 16 || at + nbytes > hc->cap) {
        fprintf(stderr, "moert/hip: workspace exhausted (%llu + %llu > %llu)\n", (unsigned long long)at,
                (unsigned long long)nbytes, (unsigned long long)hc->cap);
        abort();
    }
    hc->stack[hc->n++] = {hc->base + at, hc->top};
    hc->top = at + nbytes;
    return hc->base + at;
}

void host_pool_free(void * user, void * ptr) {
    HostCtx * hc = (HostCtx *)user;
    if (hc->n <= 0 || hc->stack[hc->n - 1].p != ptr) {
        fprintf(stderr, "moert/hip: pool free must be LIFO\n");
        abort();
    }
    hc->top = hc->stack[--hc->n].prev_top;
}

thread_local hipStream_t g_tramp_stream = nullptr;

void host_mm_stream(void * user, const moert_mm_call * c) {
    HostCtx * hc = (HostCtx *)user;
    int32_t type;
    const void * base;
    int64_t n;
    if (c->w_sel == MOERT_MM_W_HOT) {
        type = hc->w_hot->type; base = hc->w_hot->data; n = hc->w_hot->ne[2];
    } else if (c->w_sel == MOERT_MM_W_COLD_SRC) {
        type = hc->w_cold->type; base = hc->w_cold->data; n = hc->w_cold->ne[2];
    } else {
        type = c->w_type_tag; base = c->w_data; n = c->w_n;
    }
    moert_mm_call cc = *c;
    if (c->w_sel != MOERT_MM_W_RAW) cc.w_ptrs = nullptr;
    if (llapis_mul_mat_id(&cc, type, base, n, hc->d_in, hc->d_out, (void *)g_tramp_stream) != 0) {
        fprintf(stderr, "moert/hip: mul_mat_id refused: %s\n", llapis_last_error());
        abort();
    }
}

uint64_t fire_scratch_bytes(int d_in, int d_out, int pmax) {
    auto al = [](uint64_t x) { return (x + 255) & ~uint64_t(255); };
    return 2 * al((uint64_t)d_in * pmax * 4) + 4 * al((uint64_t)pmax * 4) + al(8) + 2 * al((uint64_t)d_out * pmax * 4) +
           256;
}

}  // namespace

extern "C" {

uint64_t llapis_moe_dual_workspace_size(const llapis_moe_dual_op * op) {
    if (!op || !op->src[0] || !op->src[1] || !op->src[2]) return 0;
    const int d_in = (int)op->src[0]->ne[0];
    const int d_out = (int)op->src[2]->ne[1];
    const int pmax = (int)(op->src[1]->ne[0] * op->src[1]->ne[1]);
    return fire_scratch_bytes(d_in, d_out, pmax);
}

int32_t llapis_moe_dual_compute(const llapis_moe_dual_op * op, void * workspace, uint64_t ws_bytes, void * stream) {
    if (!op || !op->dst) return fail("llapis_moe_dual_compute: null op");
    for (int i : {0, 1, 2, 3, 4, 5, 6})
        if (!op->src[i]) return fail("llapis_moe_dual_compute: missing src " + std::to_string(i));
    const llapis_tensor * cur = op->src[0];
    const llapis_tensor * ids = op->src[1];
    const llapis_tensor * w_hot = op->src[2];
    const llapis_tensor * w_cold = op->src[3];
    const int32_t * prm = op->op_params;
    moert_ffn_moe_args a = {};
    a.kind = prm[0];
    a.top_k = prm[1];
    a.il = prm[2];
    a.planc_mode = prm[9];
    a.n_used = (int32_t)ids->ne[0];
    a.n_tokens = (int32_t)ids->ne[1];
    a.ids_s1 = (int32_t)(ids->nb[1] / sizeof(int32_t));
    a.d_in = (int32_t)cur->ne[0];
    a.d_out = (int32_t)w_hot->ne[1];
    a.n_expert = (int32_t)w_cold->ne[2];
    a.k = (int32_t)op->src[5]->ne[0];
    a.cold_type_tag = w_cold->type;
    a.expert_bytes = rbytes(w_cold->type, a.d_in) * (uint64_t)a.d_out;
    a.cur = cur->data;
    a.ids = ids->data;
    a.exp_slot = op->src[4]->data;
    a.slot_exp = op->src[5]->data;
    a.slot_state = op->src[6]->data;
    a.s_hot = op->src[7] ? op->src[7]->data : nullptr;
    a.s_cold = op->src[8] ? op->src[8]->data : nullptr;
    memcpy(&a.w_cold_dev, &prm[5], sizeof(uint64_t));
    memcpy(&a.s_cold_dev, &prm[7], sizeof(uint64_t));
    a.has_w_cold = 1;
    a.dst = op->dst->data;
    a.stream = stream;
    if (a.n_used * a.n_tokens > MOERT_COLDCPU_GS_PMAX_MAX)
        return fail("llapis_moe_dual_compute: more than 32 routed pairs per fire");
    if (a.planc_mode != 0) return fail("llapis_moe_dual_compute: planc_mode must be 0 (cold pool in HBM)");
    if (ws_bytes < fire_scratch_bytes(a.d_in, a.d_out, a.n_used * a.n_tokens))
        return fail("llapis_moe_dual_compute: workspace too small");
    if (!supported_w(w_hot->type) || w_hot->type == T_F32 || !supported_w(w_cold->type))
        return fail("llapis_moe_dual_compute: unsupported pool type");

    // one kernel per fire when the formats and sizes allow it (and no
    // per-slot pointer table overrides the hot slab); otherwise the island
    const bool k256 = a.kind == 0 && (w_hot->type == T_Q4_K || w_hot->type == T_IQ2_S) &&
                      (w_cold->type == T_Q4_K || w_cold->type == T_IQ2_S) && a.d_in % 256 == 0 && a.d_in <= 3072;
    const bool k32 = a.kind == 1 && (w_hot->type == T_Q5_0 || w_hot->type == T_IQ4_NL) &&
                     (w_cold->type == T_Q5_0 || w_cold->type == T_IQ4_NL) && a.d_in % 64 == 0 && a.d_in <= 1024;
    const bool table = a.il >= 0 && a.il < 128 && g_hot_tab[a.il][a.kind].ptrs && g_hot_tab[a.il][a.kind].n == a.k;
    if (g_fused_fire.load() && (k256 || k32) && !table && a.n_expert <= 256 && a.k <= 256) {
        const long long t0 = now_ns();
        FireParams f = {};
        f.kind = a.kind; f.d_in = a.d_in; f.d_out = a.d_out; f.n_used = a.n_used; f.n_tokens = a.n_tokens;
        f.ids_s1 = a.ids_s1; f.n_expert = a.n_expert; f.k_slots = w_hot->data ? a.k : 0;
        f.cur = static_cast<const float *>(a.cur);
        f.ids = static_cast<const int32_t *>(a.ids);
        f.exp_slot = static_cast<const int32_t *>(a.exp_slot);
        f.slot_exp = static_cast<const int32_t *>(a.slot_exp);
        f.slot_state = static_cast<const int32_t *>(a.slot_state);
        f.hot = static_cast<const uint8_t *>(w_hot->data);
        f.hot_stride = rbytes(w_hot->type, a.d_in) * (uint64_t)a.d_out;
        f.cold = static_cast<const uint8_t *>(w_cold->data);
        f.cold_stride = rbytes(w_cold->type, a.d_in) * (uint64_t)a.d_out;
        f.s_hot = static_cast<const float *>(a.s_hot);
        f.s_cold = static_cast<const float *>(a.s_cold);
        f.dst = static_cast<float *>(a.dst);
        if (g_rc.on && a.kind == 0 && a.il >= 0 && a.il < g_rc.nl) {
            f.rc_counts = g_rc.dev + (size_t)a.il * g_rc.ne;
            f.rc_hits = g_rc.dev + (size_t)g_rc.nl * g_rc.ne + (size_t)a.il * 2;
        }
        const int rb = (int)std::max(rbytes(w_hot->type, a.d_in), rbytes(w_cold->type, a.d_in));
        f.w_lds = dev::align16(dev::fire_gu_rows(a.d_in) * rb + 32);
        if (fire_lds(f, w_hot->type, w_cold->type) + 16 * 1024 <= max_lds_per_wg()) {
            LL_TRY(launch_fire(f, w_hot->type, w_cold->type, g_act_mode.load(), (hipStream_t)stream));
            dir_gate_after_fire(a.il, a.kind, (hipStream_t)stream);
            g_op_ns += now_ns() - t0;
            ++g_fires;
            return 0;
        }
    }

    HostCtx hc;
    hc.base = static_cast<uint8_t *>(workspace);
    hc.cap = ws_bytes;
    hc.w_hot = w_hot;
    hc.w_cold = w_cold;
    hc.d_in = a.d_in;
    hc.d_out = a.d_out;
    g_tramp_stream = (hipStream_t)stream;
    moert_ffn_moe_host h;
    h.user = &hc;
    h.pool_alloc = &host_pool_alloc;
    h.pool_free = &host_pool_free;
    h.mm = &host_mm_stream;
    moert_ffn_moe(&a, &h);
    if (hc.n != 0) return fail("llapis_moe_dual_compute: island did not release its scratch");
    return 0;
}

// -------------------------------------------------------- router / GEGLU

int32_t llapis_router_topk(const float * x, int32_t n_tokens, const float * w_r, const float * bias, int32_t d,
                           int32_t n_expert, int32_t top_k, int32_t * ids, float * weights, float * probs,
                           void * stream) {
    if (n_tokens <= 0) return 0;
    if (!x || !w_r || !ids || !weights || !probs) return fail("llapis_router_topk: null pointer (probs is required)");
    if (n_expert <= 0 || n_expert > 256 || top_k <= 0 || top_k > 16 || top_k > n_expert)
        return fail("llapis_router_topk: need 0 < top_k <= 16, top_k <= n_expert <= 256");
    hipStream_t s = (hipStream_t)stream;
    LL_TRY(launch_router_logits(x, n_tokens, w_r, bias, d, n_expert, probs, s));
    LL_TRY(launch_topk(probs, n_tokens, n_expert, top_k, ids, weights, s));
    return 0;
}

int32_t llapis_geglu(const float * gate_up, int32_t n_ff, int32_t n_cols, float * out, int32_t gelu_mode,
                     void * stream) {
    if (n_cols <= 0 || n_ff <= 0) return 0;
    LL_TRY(launch_geglu(gate_up, n_ff, n_cols, out, gelu_mode, (hipStream_t)stream));
    return 0;
}

int32_t llapis_residual_rmsnorm(float * h, const float * add, int32_t n_tokens, int32_t d, float eps, float * x,
                                void * stream) {
    if (n_tokens <= 0) return 0;
    if (!h || !x) return fail("llapis_residual_rmsnorm: null pointer");
    if (d <= 0 || d > 4096) return fail("llapis_residual_rmsnorm: need 0 < d <= 4096");
    LL_TRY(launch_residual_rmsnorm(h, add, n_tokens, d, eps, x, (hipStream_t)stream));
    return 0;
}

int32_t llapis_moe_combine(const float * y, const float * weights, int32_t n_tokens, int32_t top_k, int32_t d,
                           float * out, void * stream) {
    if (n_tokens <= 0 || d <= 0) return 0;
    if (!y || !weights || !out) return fail("llapis_moe_combine: null pointer");
    if (top_k < 1 || top_k > 64) return fail("llapis_moe_combine: need 1 <= top_k <= 64");
    LL_TRY(launch_combine(y, weights, n_tokens, top_k, d, out, (hipStream_t)stream));
    return 0;
}

// ------------------------------------------------------------ profiling

namespace {
constexpr int PROF_STAGES = 5;      // router, top-k, gate_up, down, combine
constexpr int PROF_RING = 4096;
// Per call and stage a begin/end event pair.  Single-kernel stages (the
// decode path's kernels, the generic path's matvecs) get the dispatch's own
// begin/end timestamps; multi-kernel or small stages are bracketed by event
// records.  A stage a path does not have stays unrecorded and reads as 0.
struct Profiler {
    std::mutex mu;
    bool on = false;
    hipEvent_t ev[PROF_RING][2 * PROF_STAGES] = {};
    bool used[PROF_RING][PROF_STAGES] = {};
    int n = 0;          // calls recorded since the last read
    bool created = false;
};
Profiler g_prof;

// a profiling slot for this call, or -1
int prof_slot() {
    if (!g_prof.on) return -1;
    std::lock_guard<std::mutex> lk(g_prof.mu);
    if (g_prof.n >= PROF_RING) return -1;
    const int c = g_prof.n++;
    for (bool & u : g_prof.used[c]) u = false;
    return c;
}
// the event pair of stage st of slot c (nullptrs when not profiling)
hipEvent_t prof_ev(int c, int st, int end) {
    if (c < 0) return nullptr;
    g_prof.used[c][st] = true;
    return g_prof.ev[c][2 * st + end];
}
hipError_t prof_record(int c, int st, int end, hipStream_t s) {
    if (c < 0) return hipSuccess;
    return hipEventRecord(prof_ev(c, st, end), s);
}
}  // namespace

void llapis_profile_enable(int32_t on) {
    std::lock_guard<std::mutex> lk(g_prof.mu);
    if (on && !g_prof.created) {
        for (auto & row : g_prof.ev)
            for (auto & e : row) MOERT_HIP_CHECK(hipEventCreate(&e));
        g_prof.created = true;
    }
    g_prof.on = on != 0;
    g_prof.n = 0;
}

int32_t llapis_profile_read(float * ms, int32_t n) {
    std::lock_guard<std::mutex> lk(g_prof.mu);
    for (int i = 0; i < n; ++i) ms[i] = 0.0f;
    const int calls = g_prof.n;
    for (int c = 0; c < calls; ++c) {
        for (int st = 0; st < PROF_STAGES && st < n; ++st) {
            if (!g_prof.used[c][st]) continue;
            float t = 0.0f;
            if (hipEventSynchronize(g_prof.ev[c][2 * st + 1]) != hipSuccess) return -1;
            if (hipEventElapsedTime(&t, g_prof.ev[c][2 * st], g_prof.ev[c][2 * st + 1]) != hipSuccess) return -1;
            ms[st] += t;
        }
    }
    g_prof.n = 0;
    return calls;
}

// ------------------------------------------------------------- fused layer

namespace {

uint64_t al256(uint64_t x) { return (x + 255) & ~uint64_t(255); }

uint64_t dec_ctl_bytes(const llapis_moe_layer *) { return al256(sizeof(DecCtl)); }

// generic path (any T): probs, ids, w, y_gu, y_dn -- after the decode path's
// control block, which every layout reserves so the two paths can share a
// workspace
struct FfnWs {
    uint64_t probs, ids, w, ygu, ydn, total;
};
FfnWs ffn_ws(const llapis_moe_layer * L, int32_t T) {
    const uint64_t P = (uint64_t)T * L->top_k;
    FfnWs w;
    w.probs = dec_ctl_bytes(L);
    w.ids = w.probs + al256((uint64_t)T * L->n_expert * 4);
    w.w = w.ids + al256(P * 4);
    w.ygu = w.w + al256(P * 4);
    w.ydn = w.ygu + al256(P * 2 * L->n_ff * 4);
    w.total = w.ydn + al256(P * L->d_model * 4);
    return w;
}

// decode path (T <= DEC_MAXT): control block first
struct DecWs {
    uint64_t ctl, logits, ids, w, xq, yq, ydn, total, ctl_bytes;
    int64_t xq_stride, yq_stride;
};
DecWs dec_ws(const llapis_moe_layer * L, int32_t T) {
    const uint64_t P = (uint64_t)T * L->top_k;
    DecWs w;
    w.xq_stride = dec_act_bytes(L->d_model);
    w.yq_stride = dec_act_bytes(L->n_ff);
    w.ctl = 0;
    w.ctl_bytes = dec_ctl_bytes(L);
    w.logits = w.ctl_bytes;
    w.ids = w.logits + al256((uint64_t)T * L->n_expert * 4);
    w.w = w.ids + al256(P * 4);
    w.xq = w.w + al256(P * 4);
    w.yq = w.xq + al256((uint64_t)T * w.xq_stride);
    w.ydn = w.yq + al256(P * w.yq_stride);
    w.total = w.ydn + (T > 1 ? al256(P * L->d_model * 4) : 0);
    return w;
}

bool decode_eligible(const llapis_moe_layer * L, int32_t T) {
    // n_ff <= 1024 and a multiple of 64: 16 lanes hold a down row as whole
    // block pairs, and gate_up items are whole 32-blocks
    return g_decode_path.load() && T <= DEC_MAXT && L->top_k <= 16 && L->n_expert <= 256 && L->k_slots <= 256 &&
           (L->d_model % 4) == 0 && L->n_ff <= 1024 && L->n_ff % 64 == 0;
}

// prefill path (T > DEC_MAXT, either activation mode): tokens are processed in
// chunks of Tc = PF_MAX_PAIRS / top_k; one chunk's scratch
struct PfWs {
    uint64_t probs, ids, w, ntiles, sorted, tiles, gtiles, xq, xd, xm, xh, ah, al, ydn, parts, total;
    int Tc, max_tiles, max_gtiles;
};
PfWs pf_ws(const llapis_moe_layer * L, int32_t T) {
    PfWs w;
    w.Tc = std::min<int>(T, PF_MAX_PAIRS / std::max(1, L->top_k));
    const uint64_t P = (uint64_t)w.Tc * L->top_k;
    const uint64_t D = L->d_model, F = L->n_ff, NSB = L->d_model / 256;
    w.max_tiles = pf_max_tiles((int)P, L->n_expert);
    w.max_gtiles = pf_max_gtiles((int)P, L->n_expert);
    w.probs = dec_ctl_bytes(L);
    w.ids = w.probs + al256((uint64_t)w.Tc * L->n_expert * 4);
    w.w = w.ids + al256(P * 4);
    w.ntiles = w.w + al256(P * 4);
    w.sorted = w.ntiles + 256;
    w.tiles = w.sorted + al256(P * 4);
    w.gtiles = w.tiles + al256((uint64_t)w.max_tiles * sizeof(PfTile));
    w.xq = w.gtiles + al256((uint64_t)w.max_gtiles * sizeof(PfTile));
    w.xd = w.xq + al256((uint64_t)w.Tc * D);
    w.xm = w.xd + al256((uint64_t)w.Tc * NSB * 4);
    w.xh = w.xm + al256((uint64_t)w.Tc * NSB * 32);
    w.ah = w.xh + al256((uint64_t)w.Tc * D * 4);
    w.al = w.ah + al256(P * F * 2);
    w.ydn = w.al + al256(P * F * 2);
    w.parts = w.ydn + al256(P * D * 4);
    w.total = w.parts + al256((uint64_t)router_parts_floats(w.Tc, L->n_expert) * 4);
    return w;
}

bool prefill_eligible(const llapis_moe_layer * L, int32_t T) {
    return g_prefill.load() && T > DEC_MAXT && L->top_k >= 1 &&
           L->top_k <= PF_MAX_PAIRS && L->n_expert <= 256 && L->k_slots <= 256 && L->n_ff <= PF_MAX_FF &&
           L->d_model % 256 == 0 &&
           L->n_ff % 32 == 0;
}
}  // namespace

void llapis_set_tuning(int32_t key, int32_t value) {
    if (key == 0) g_decode_path = value != 0;
    if (key == 2) g_prefill = value != 0;
    if (key == 3) g_dn_rows_log2 = value >= 0 && value <= 5 ? value : -1;
    if (key == 4) g_dn_by_group = value == 0 || value == 1 ? value : -1;
    if (key == 6) g_fused_fire = value != 0;
}

uint64_t llapis_moe_ffn_workspace_size(const llapis_moe_layer * L, int32_t n_tokens) {
    if (!L || n_tokens <= 0) return 0;
    uint64_t b = ffn_ws(L, n_tokens).total;
    if (n_tokens <= DEC_MAXT) b = std::max(b, dec_ws(L, n_tokens).total);
    if (n_tokens > DEC_MAXT) b = std::max(b, pf_ws(L, n_tokens).total);
    return b;
}

int32_t llapis_moe_ffn_workspace_init(const llapis_moe_layer * L, void * workspace, uint64_t ws_bytes, void * stream) {
    if (!L || !workspace) return fail("llapis_moe_ffn_workspace_init: null argument");
    const DecWs dw = dec_ws(L, 1);
    const uint64_t n = std::min<uint64_t>(ws_bytes, dw.ctl_bytes);
    LL_TRY(launch_zero_i32(static_cast<int *>(workspace), (int)(n / 4), (hipStream_t)stream));
    return 0;
}

int32_t llapis_moe_ffn(const llapis_moe_layer * L, const float * x, const float * x_router, int32_t T, float * out,
                       int32_t * ids_out, float * w_out, void * workspace, uint64_t ws_bytes, void * stream) {
    if (!L) return fail("llapis_moe_ffn: null layer");
    if (T <= 0) return 0;
    const float * xr = x_router ? x_router : x;     // the router's input (gemma4.cpp:400-403)
    if (!is_gu_type(L->hot_gu_type) || !is_gu_type(L->cold_gu_type) || !is_dn_type(L->hot_dn_type) ||
        !is_dn_type(L->cold_dn_type))
        return fail("llapis_moe_ffn: gate_up pools must be Q4_K/IQ2_S and down pools Q5_0/IQ4_NL");
    if (L->d_model % 256 || L->n_ff % 32 || L->d_model > dev::MAX_D_IN || L->n_ff > dev::MAX_D_IN)
        return fail("llapis_moe_ffn: d_model must be a multiple of 256 and n_ff of 32");
    if (L->k_slots > 0 && (!L->hot_gu || !L->hot_dn || !L->exp_slot || !L->slot_exp || !L->slot_state))
        return fail("llapis_moe_ffn: hot pool or residency mirrors missing");
    if (!L->cold_gu || !L->cold_dn || !L->router_w) return fail("llapis_moe_ffn: cold pool or router missing");
    const uint64_t gu_hot = rbytes(L->hot_gu_type, L->d_model) * 2 * L->n_ff;
    const uint64_t gu_cold = rbytes(L->cold_gu_type, L->d_model) * 2 * L->n_ff;
    const uint64_t dn_hot = rbytes(L->hot_dn_type, L->n_ff) * L->d_model;
    const uint64_t dn_cold = rbytes(L->cold_dn_type, L->n_ff) * L->d_model;
    if ((gu_hot | gu_cold | dn_hot | dn_cold) % 16) return fail("llapis_moe_ffn: expert slabs must be multiples of 16 bytes");
    hipStream_t s = (hipStream_t)stream;
    uint8_t * base = static_cast<uint8_t *>(workspace);
    if (decode_eligible(L, T)) {
        const DecWs dw = dec_ws(L, T);
        if (!workspace || ws_bytes < dw.total) return fail("llapis_moe_ffn: workspace too small");
        DecParams p = {};
        p.d_model = L->d_model; p.n_ff = L->n_ff; p.n_expert = L->n_expert; p.top_k = L->top_k;
        p.k_slots = L->k_slots; p.T = T;
        p.x = x; p.xr = xr; p.router_w = L->router_w; p.router_b = L->router_b;
        p.hot_gu = static_cast<const uint8_t *>(L->hot_gu); p.hot_gu_stride = gu_hot;
        p.cold_gu = static_cast<const uint8_t *>(L->cold_gu); p.cold_gu_stride = gu_cold;
        p.hot_dn = static_cast<const uint8_t *>(L->hot_dn); p.hot_dn_stride = dn_hot;
        p.cold_dn = static_cast<const uint8_t *>(L->cold_dn); p.cold_dn_stride = dn_cold;
        p.exp_slot = L->exp_slot; p.slot_exp = L->slot_exp; p.slot_state = L->slot_state;
        p.s_hot = L->s_hot; p.s_cold = L->s_cold;
        p.ctl = reinterpret_cast<DecCtl *>(base + dw.ctl);
        p.rc_counts = L->route_counts;
        p.rc_hits = L->route_counts ? L->route_hits : nullptr;
        p.logits = reinterpret_cast<float *>(base + dw.logits);
        p.ids = ids_out ? ids_out : reinterpret_cast<int32_t *>(base + dw.ids);
        p.w = w_out ? w_out : reinterpret_cast<float *>(base + dw.w);
        p.xq = base + dw.xq; p.xq_stride = dw.xq_stride;
        p.yq = base + dw.yq; p.yq_stride = dw.yq_stride;
        p.ydn = reinterpret_cast<float *>(base + dw.ydn);
        p.dn_by_group = g_dn_by_group.load() >= 0 ? g_dn_by_group.load() : 1;
        p.out = out;
        const int rbg = (int)std::max(rbytes(L->hot_gu_type, L->d_model), rbytes(L->cold_gu_type, L->d_model));
        p.w_lds_gu = dec_gu_half_bytes(T, rbg);
        // the down rows: a power of two giving about three blocks per CU of
        // the part (256 CUs on MI355X: 4 rows, 704 blocks at d_model 2816)
        int lg2r = 0;
        while ((1 << lg2r) < DEC_DN_MAXR && (1 << lg2r) * 768 < L->d_model) ++lg2r;
        if (g_dn_rows_log2.load() >= 0) lg2r = g_dn_rows_log2.load();
        p.dn_rows_log2 = lg2r;
        const int lds_max = max_lds_per_wg();
        // the LDS of the down kernel that will run: every pair's column at one
        // token, the group's members' columns by group
        const int dn_lds = T == 1 || !p.dn_by_group ? dec_lds_down(p) : std::min(T, DEC_MAXT) * dec_act_bytes(L->n_ff);
        if (dn_lds + 16 * 1024 <= lds_max && dec_lds_gate_up(p, L->hot_gu_type, L->cold_gu_type) + 16 * 1024 <= lds_max) {
            const int pc = prof_slot();
            const int src = L->gelu_mode == LLAPIS_GELU_TANH ? dev::SRC_GEGLU_TANH : dev::SRC_GEGLU_TABLE;
            const bool comb = T > 1 && p.dn_by_group;
            hipEvent_t ev[8] = {prof_ev(pc, 0, 0), prof_ev(pc, 0, 1), prof_ev(pc, 2, 0), prof_ev(pc, 2, 1),
                                prof_ev(pc, 3, 0), prof_ev(pc, 3, 1),
                                comb ? prof_ev(pc, 4, 0) : nullptr, comb ? prof_ev(pc, 4, 1) : nullptr};
            LL_TRY(launch_decode(p, L->hot_gu_type, L->cold_gu_type, L->hot_dn_type, L->cold_dn_type, L->act_mode,
                                 src, s, pc >= 0 ? ev : nullptr));
            return 0;
        }
    }
    if (prefill_eligible(L, T)) {
        const PfWs pw = pf_ws(L, T);
        if (!workspace || ws_bytes < pw.total) return fail("llapis_moe_ffn: workspace too small");
        const int K = L->top_k;
        const int src = L->gelu_mode == LLAPIS_GELU_TANH ? dev::SRC_GEGLU_TANH : dev::SRC_GEGLU_TABLE;
        for (int t0 = 0; t0 < T; t0 += pw.Tc) {
            const int Tc = std::min(pw.Tc, T - t0);
            float * probs = (float *)(base + pw.probs);
            int32_t * ids = ids_out ? ids_out + (int64_t)t0 * K : (int32_t *)(base + pw.ids);
            float * w = w_out ? w_out + (int64_t)t0 * K : (float *)(base + pw.w);
            const float * xc = x + (int64_t)t0 * L->d_model;
            const float * xrc = xr + (int64_t)t0 * L->d_model;
            const int pc = prof_slot();
            float * parts = (float *)(base + pw.parts);
            LL_TRY(prof_record(pc, 0, 0, s));
            LL_TRY(launch_router_mfma(xrc, Tc, L->router_w, L->d_model, L->n_expert, parts, s));
            LL_TRY(prof_record(pc, 0, 1, s));
            LL_TRY(prof_record(pc, 1, 0, s));
            LL_TRY(launch_topk_parts(parts, L->router_b, Tc, L->n_expert, K, probs, ids, w, s));
            LL_TRY(prof_record(pc, 1, 1, s));
            PfParams p = {};
            p.d_model = L->d_model; p.n_ff = L->n_ff; p.n_expert = L->n_expert; p.top_k = K;
            p.k_slots = L->k_slots; p.T = Tc;
            p.x = xc; p.ids = ids;
            p.exp_slot = L->exp_slot; p.slot_exp = L->slot_exp; p.slot_state = L->slot_state;
            p.hot_gu = static_cast<const uint8_t *>(L->hot_gu); p.hot_gu_stride = gu_hot;
            p.cold_gu = static_cast<const uint8_t *>(L->cold_gu); p.cold_gu_stride = gu_cold;
            p.hot_dn = static_cast<const uint8_t *>(L->hot_dn); p.hot_dn_stride = dn_hot;
            p.cold_dn = static_cast<const uint8_t *>(L->cold_dn); p.cold_dn_stride = dn_cold;
            p.s_hot = L->s_hot; p.s_cold = L->s_cold;
            p.n_tiles = (int *)(base + pw.ntiles);
            p.sorted = (int32_t *)(base + pw.sorted);
            p.tiles = (PfTile *)(base + pw.tiles);
            p.max_tiles = pw.max_tiles;
            p.gtiles = (PfTile *)(base + pw.gtiles);
            p.max_gtiles = pw.max_gtiles;
            p.n_gtiles = p.n_tiles + 1;
            p.xq = (int8_t *)(base + pw.xq);
            p.xd = (float *)(base + pw.xd);
            p.xm = (_Float16 *)(base + pw.xm);
            p.act_mode = L->act_mode == LLAPIS_ACT_Q8_1 ? dev::AM_Q8_1 : dev::AM_CPU;
            p.xh = (_Float16 *)(base + pw.xh);
            p.ah = (_Float16 *)(base + pw.ah);
            p.al = (_Float16 *)(base + pw.al);
            p.ydn = (float *)(base + pw.ydn);
            p.rc_counts = L->route_counts;
            p.rc_hits = L->route_counts ? L->route_hits : nullptr;
            hipEvent_t ev[4] = {prof_ev(pc, 2, 0), prof_ev(pc, 2, 1), prof_ev(pc, 3, 0), prof_ev(pc, 3, 1)};
            LL_TRY(launch_prefill(p, L->hot_gu_type, L->cold_gu_type, L->hot_dn_type, L->cold_dn_type, src, s,
                                  pc >= 0 ? ev : nullptr));
            LL_TRY(prof_record(pc, 4, 0, s));
            LL_TRY(launch_combine(p.ydn, w, Tc, K, L->d_model, out + (int64_t)t0 * L->d_model, s));
            LL_TRY(prof_record(pc, 4, 1, s));
        }
        return 0;
    }
    const FfnWs ws = ffn_ws(L, T);
    if (!workspace || ws_bytes < ws.total) return fail("llapis_moe_ffn: workspace too small");
    float * probs = (float *)(base + ws.probs);
    int32_t * ids = ids_out ? ids_out : (int32_t *)(base + ws.ids);
    float * w = w_out ? w_out : (float *)(base + ws.w);
    float * ygu = (float *)(base + ws.ygu);
    float * ydn = (float *)(base + ws.ydn);
    const int P = T * L->top_k;

    const int pc = prof_slot();        // profiling slot of this call
    LL_TRY(prof_record(pc, 0, 0, s));
    LL_TRY(launch_router_logits(xr, T, L->router_w, L->router_b, L->d_model, L->n_expert, probs, s));
    LL_TRY(prof_record(pc, 0, 1, s));
    LL_TRY(prof_record(pc, 1, 0, s));
    LL_TRY(launch_topk(probs, T, L->n_expert, L->top_k, ids, w, s));
    LL_TRY(prof_record(pc, 1, 1, s));
    LL_TRY(launch_route_count(ids, L->top_k, L->top_k, P, L->exp_slot, L->slot_exp, L->slot_state, L->n_expert,
                              L->k_slots, L->route_counts, L->route_hits, s));

    MmvParams p = {};
    p.mode = MMV_ROUTED;
    p.top_k = L->top_k;
    p.ids_s1 = L->top_k;
    p.n_expert = L->n_expert;
    p.k_slots = L->k_slots;
    p.exp_slot = L->exp_slot;
    p.slot_exp = L->slot_exp;
    p.slot_state = L->slot_state;
    p.ids = ids;
    // gate_up: activation column = token
    p.d_in = L->d_model;
    p.d_out = 2 * L->n_ff;
    p.w0 = static_cast<const uint8_t *>(L->hot_gu);
    p.stride0 = gu_hot;
    p.n0 = L->k_slots;
    p.w1 = static_cast<const uint8_t *>(L->cold_gu);
    p.stride1 = gu_cold;
    p.n1 = L->n_expert;
    p.act = x;
    p.act_ld = L->d_model;
    p.act_by_token = 1;
    p.y = ygu;
    mmv_prepare(p, L->hot_gu_type, L->cold_gu_type);
    LL_TRY(launch_mmv(p, L->hot_gu_type, L->cold_gu_type, L->act_mode, dev::SRC_PLAIN, P, s, prof_ev(pc, 2, 0),
                      prof_ev(pc, 2, 1)));
    // down: activation column = pair, GEGLU of its gate_up output on the fly
    p.d_in = L->n_ff;
    p.d_out = L->d_model;
    p.w0 = static_cast<const uint8_t *>(L->hot_dn);
    p.stride0 = dn_hot;
    p.w1 = static_cast<const uint8_t *>(L->cold_dn);
    p.stride1 = dn_cold;
    p.s0 = L->s_hot;
    p.s1 = L->s_cold;
    p.act = ygu;
    p.act_ld = 2 * L->n_ff;
    p.act_by_token = 0;
    p.y = ydn;
    mmv_prepare(p, L->hot_dn_type, L->cold_dn_type);
    const int src = L->gelu_mode == LLAPIS_GELU_TANH ? dev::SRC_GEGLU_TANH : dev::SRC_GEGLU_TABLE;
    LL_TRY(launch_mmv(p, L->hot_dn_type, L->cold_dn_type, L->act_mode, src, P, s, prof_ev(pc, 3, 0),
                      prof_ev(pc, 3, 1)));
    LL_TRY(prof_record(pc, 4, 0, s));
    LL_TRY(launch_combine(ydn, w, T, L->top_k, L->d_model, out, s));
    LL_TRY(prof_record(pc, 4, 1, s));
    return 0;
}

// ------------------------------------------------- entry point without allocation

}  // extern "C"

namespace {
// The scratch of llapis_moe_ffn_noalloc: one fixed array per GPU, held until
// the process ends.  Host code never uses this name as an address (on the
// host it is only a stand-in for the symbol); it uses the device address
// hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) uint8_t scratch[LLAPIS_NOALLOC_SCRATCH_BYTES];

std::mutex g_na_mu;
std::map<int, uint8_t *> g_na_ptr;     // device -> address of that device's scratch

// The current device's scratch address, looked up at the first call on each
// device.  Nothing is launched: every path of llapis_moe_ffn writes each
// scratch word before it reads it, so the array needs no clearing (and a
// first call made under stream capture records no extra node).
int32_t noalloc_scratch(uint8_t ** out) {
    int dev = 0;
    LL_TRY(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_na_mu);
    auto it = g_na_ptr.find(dev);
    if (it != g_na_ptr.end()) {
        *out = it->second;
        return 0;
    }
    void * p = nullptr;
    LL_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return fail("llapis_moe_ffn_noalloc: no device address for the scratch array");
    g_na_ptr[dev] = static_cast<uint8_t *>(p);
    *out = static_cast<uint8_t *>(p);
    return 0;
}
}  // namespace

extern "C" {

int32_t llapis_moe_ffn_noalloc(const llapis_moe_layer * L, const float * x, const float * x_router, int32_t T,
                               float * out, int32_t * ids_out, float * w_out, void * stream) {
    if (!L) return fail("llapis_moe_ffn_noalloc: null layer");
    if (T <= 0) return 0;
    const uint64_t need = llapis_moe_ffn_workspace_size(L, T);
    if (need > LLAPIS_NOALLOC_SCRATCH_BYTES)
        return fail("llapis_moe_ffn_noalloc: this call needs " + std::to_string(need) +
                    " bytes of scratch, more than the fixed " + std::to_string(LLAPIS_NOALLOC_SCRATCH_BYTES) +
                    " bytes; use llapis_moe_ffn with a workspace");
    uint8_t * ptr = nullptr;
    if (const int32_t rc = noalloc_scratch(&ptr)) return rc;
    return llapis_moe_ffn(L, x, x_router, T, out, ids_out, w_out, ptr, LLAPIS_NOALLOC_SCRATCH_BYTES, stream);
}

}  // extern "C"
