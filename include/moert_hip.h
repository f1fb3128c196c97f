/*
 * moert_hip.h -- the MoE expert island's C ABI, implemented for MI355X.
 *
 * Drop-in replacement for the reference's moert/cuda library: the same entry
 * points, the same plain-C structs with the same field order, types and sizes
 * (moert/include/moert/cuda.h:41-276), so the reference's GGML_OP_MOE_DUAL
 * trampoline (ggml-cuda/moe-dual.cu:98-157) links against this library
 * unchanged except for its CUDA stream type.  Pointers are device pointers
 * unless a field says otherwise; `stream` is a hipStream_t.
 *
 * What differs from the CUDA island, by design:
 *  - the cold tier is resident in HBM (planc_mode 0): the RAM-cold modes 1
 *    and 2 and the CPU sidecar callbacks are accepted in the config but
 *    moert_ffn_moe refuses a fire with planc_mode != 0 (prints and aborts,
 *    the island's error contract);
 *  - the host-memory registration services refuse (return 0 / NULL): the
 *    cold tier lives in HBM, so nothing host-side is mapped for kernels.  The
 *    batch transport (moert_cuda_dir_*, moert_cuda_publish_h2d and the
 *    early-decision gate) is implemented: see its declarations below.
 */
#ifndef MOERT_HIP_H
#define MOERT_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Routed pairs per fire the partition handles (one wavefront lane per pair).
 * Kept at the reference's value (cuda.h:39) for ABI compatibility even though
 * a 64-lane wavefront could take 64. */
#define MOERT_COLDCPU_GS_PMAX_MAX 32

/* Replaces moert_cuda_config (moert/include/moert/cuda.h:41-69). */
typedef struct moert_cuda_config {
    int32_t  counted;           /* skip padded channels via the device count (default 1) */
    int32_t  copy_stream;       /* RAM-cold copy stream: no effect here (cold is in HBM) */
    int32_t  coldcpu;           /* CPU cold sidecar: no effect here */
    int32_t  coldcpu_max;
    uint64_t coldcpu_fn;
    uint64_t cold_guard_fn;
    int32_t  cold_ffn;
    uint64_t coldffn_submit_fn;
    uint64_t coldffn_wait_fn;
} moert_cuda_config;

/* Host callback types the config carries (cuda.h:70-119).  They are part of
 * the interface the embedding host compiles against; this backend stores the
 * config but never calls them (the cold tier is in HBM, so no fire takes the
 * RAM-cold sidecar path). */
typedef void (*moert_cold_guard_fn)(int32_t il, const int32_t * ids, int32_t n);

/* cuda.h:80-94: one (layer, kind) cold matmul for the host sidecar */
typedef struct moert_coldcpu_call {
    int32_t         il, kind;
    int32_t         n_cold;
    const int32_t * cold_ids;      /* host, compaction order */
    const float   * x;             /* host activations */
    int32_t         x_per_pair;    /* 0: one shared column [d_in]; 1: [d_in, n_cold] */
    const void    * w_host;        /* cold pool host base */
    uint64_t        expert_bytes;
    uint64_t        stride;        /* base + e * stride; 0 means expert_bytes */
    int32_t         w_type_tag;
    int32_t         d_in, d_out;
    float         * y;             /* out [d_out, n_cold], host */
    const int32_t * x_col;         /* optional per-pair column of x, or NULL */
} moert_coldcpu_call;
typedef void (*moert_coldcpu_fn)(const moert_coldcpu_call * call);

/* cuda.h:102-115: one layer's whole cold FFN for the host */
typedef struct moert_coldffn_job {
    int32_t         il;
    int32_t         n_used, n_tokens;
    const int32_t * h_counts;      /* [0] n_hot, [1] n_cold */
    const int32_t * h_ids;         /* cold expert ids, compaction order */
    const int32_t * h_cdst;        /* cold pair index, same order */
    const float   * x;             /* token columns [d_in, n_tokens] */
    const void    * w_gu;          /* gate_up cold pool host base */
    uint64_t        gu_bytes, gu_stride;
    int32_t         gu_type, d_in, d_gu;
    float         * y;             /* out */
    void          (*wait_ready)(void * ev);
    void          * ev;
} moert_coldffn_job;
typedef void    (*moert_coldffn_submit_fn)(const moert_coldffn_job * job);
typedef int32_t (*moert_coldffn_wait_fn)(int32_t il, int64_t * cpu_ns);

/* Replaces the header-inline moert_cuda_config_defaults (cuda.h:121-131). */
static inline void moert_cuda_config_defaults(moert_cuda_config * cfg) {
    cfg->counted = 1;
    cfg->copy_stream = 0;
    cfg->coldcpu = 0;
    cfg->coldcpu_max = 3;
    cfg->coldcpu_fn = 0;
    cfg->cold_guard_fn = 0;
    cfg->cold_ffn = 0;
    cfg->coldffn_submit_fn = 0;
    cfg->coldffn_wait_fn = 0;
}

/* Replaces moert_cuda_configure (cuda.h:135, ffn_moe.cu:772). */
void moert_cuda_configure(const moert_cuda_config * cfg);

/* weight selectors of a quantised mul_mat_id call (cuda.h:140-144) */
enum {
    MOERT_MM_W_HOT      = 0,
    MOERT_MM_W_COLD_SRC = 1,
    MOERT_MM_W_RAW      = 2,
};

/* Replaces moert_mm_call (cuda.h:150-166): y[d_out, i] = W[ids[i]] . b[:, col(i)]
 * for channels i < *ne_live (all n_ids channels when ne_live is NULL). */
typedef struct moert_mm_call {
    int32_t      w_sel;
    int32_t      w_type_tag;       /* MOERT_MM_W_RAW: ggml type of the pool */
    const void * w_data;           /* MOERT_MM_W_RAW: pool base */
    int64_t      w_n;              /* MOERT_MM_W_RAW: experts in the pool */
    const void * b;                /* f32 [d_in, b_ncols] */
    int64_t      b_ncols;          /* 1 (shared column) or n_ids */
    const void * ids;              /* i32 [n_ids] */
    int64_t      n_ids;
    void *       y;                /* f32 [d_out, n_ids] */
    const int32_t * ne_live;       /* device count of live channels, or NULL */
    const void * const * w_ptrs;   /* MOERT_MM_W_RAW: per-expert base table, or NULL */
} moert_mm_call;

/* Replaces moert_ffn_moe_host (cuda.h:170-175): services lent by the embedding
 * backend -- LIFO device scratch and the quantised mul_mat_id.  The MI355X
 * backend binds `mm` to llapis_mul_mat_id (llapis_moe.h). */
typedef struct moert_ffn_moe_host {
    void *  user;
    void * (*pool_alloc)(void * user, uint64_t nbytes);
    void   (*pool_free)(void * user, void * ptr);
    void   (*mm)(void * user, const moert_mm_call * call);
} moert_ffn_moe_host;

/* Replaces moert_ffn_moe_args (cuda.h:177-206). */
typedef struct moert_ffn_moe_args {
    int32_t kind;            /* 0 = merged gate_up, 1 = down */
    int32_t top_k;
    int32_t il;
    int32_t planc_mode;      /* 0 only (cold pool resident in HBM) */
    int32_t n_used;
    int32_t n_tokens;        /* n_used * n_tokens <= MOERT_COLDCPU_GS_PMAX_MAX */
    int32_t ids_s1;          /* row stride of ids in int32 elements */
    int32_t d_in, d_out;
    int32_t n_expert;
    int32_t k;
    int32_t cold_type_tag;
    uint64_t expert_bytes;
    const void * cur;        /* f32 [d_in, 1 | n_used*n_tokens] (kind 0 | 1) */
    const void * ids;        /* i32 [n_used, n_tokens], row stride ids_s1 */
    const void * exp_slot;   /* i32 [n_expert] */
    const void * slot_exp;   /* i32 [k] */
    const void * slot_state; /* i32 [k]: 0 FREE, 1 FILLING, 2 READY */
    const void * s_hot;      /* f32 [k] or NULL */
    const void * s_cold;     /* f32 [n_expert] or NULL */
    uint64_t w_cold_dev;
    uint64_t s_cold_dev;
    int32_t  has_w_cold;
    void *   dst;            /* f32 [d_out, n_used*n_tokens] in routed-pair order */
    void *   stream;         /* hipStream_t */
} moert_ffn_moe_args;

/* Replaces moert_ffn_moe (cuda.h:208, ffn_moe.cu:892-1246): one (layer, kind)
 * fire -- partition by residency, hot and cold quantised matmuls through
 * host->mm, scatter back to routed-pair order with the down .scale applied
 * once.  All scratch comes from host->pool_alloc and is released LIFO. */
void moert_ffn_moe(const moert_ffn_moe_args * args, const moert_ffn_moe_host * host);

/* Replaces the device routing counters (cuda.h:215-219, ffn_moe.cu:778-799).
 * Layout: [n_layers][n_expert] routed-pair counts, then [n_layers][2] hot/cold. */
int32_t moert_cuda_route_counts_enable(int32_t n_layers, int32_t n_expert);
int32_t moert_cuda_route_counts_fetch(int32_t * dst, int32_t reset);

/* Host registration services (cuda.h:224-230): refused on this backend (the
 * cold tier lives in HBM).  register_* return 0, host_map returns NULL. */
int32_t moert_cuda_host_register_pinned(void * base, uint64_t size);
void    moert_cuda_host_unregister(void * base);
int32_t moert_cuda_host_register_mapped(void * base, uint64_t size);
void *  moert_cuda_host_map(void * base, uint64_t size);

/* Replaces moert_cuda_stats (cuda.h:234-244). */
typedef struct moert_cuda_stats {
    long long fires;
    long long op_host_ns;
    long long seam_syncs;
    long long seam_ns;
    long long coldcpu_calls;
    long long coldcpu_pairs;
    long long coldcpu_ns;
    long long coldcpu_over_max;
} moert_cuda_stats;
void moert_cuda_stats_get(moert_cuda_stats * out);

/* Replaces the batch transport (cuda.h:246-262, ffn_moe.cu:521-690).
 * init: a side stream of default priority; sm_blocks > 0 copies device
 * sources with a copy kernel of that many workgroups (else hipMemcpyAsync),
 * sm_ring_mib sizes the pinned ring for small pageable sources (>= 1 MiB),
 * sm_stage_threads is ignored.  async: issue one copy now (device or pinned
 * source in place; a pageable source <= 4 KiB staged; a larger pageable
 * source refused: 0, the caller copies it itself).  mark: an event after the
 * copies issued so far, returns its id (0, 1, ...); poll: the highest id
 * whose copies landed (-1 before any; wait_all synchronises first).  mark and
 * poll return -1 before init.  publish_h2d: n copies from pageable views,
 * staged through pinned memory, landed before it returns.  Thread-safe. */
int32_t moert_cuda_dir_init(int32_t sm_blocks, int32_t sm_ring_mib, int32_t sm_stage_threads);
int32_t moert_cuda_dir_async(void * dst_dev, const void * src, uint64_t nbytes);
int64_t moert_cuda_dir_mark(void);
int64_t moert_cuda_dir_poll(int32_t wait_all);
int32_t moert_cuda_publish_h2d(int32_t n, void * const * dsts, const void * const * srcs, const uint64_t * sizes);

/* Replaces moert_cuda_dir_stats (cuda.h:263-270): sm_copies counts the
 * copy-kernel launches, sm_ring_* the staged pageable sources; the GPU-time
 * fields stay 0. */
typedef struct moert_cuda_dir_stats {
    long long async_copies, async_marks, bytes;
    long long pub_calls, pub_copies;
    long long sm_copies, sm_fallback;
    long long sm_timed, sm_gpu_ns, sm_gpu_ns_max;
    long long sm_ring_copies, sm_ring_waits; double sm_ring_wait_ms, sm_stage_ms;
} moert_cuda_dir_stats;
void    moert_cuda_dir_stats_get(moert_cuda_dir_stats * out);
/* Replaces the early-decision gate (cuda.h:271-274, ffn_moe.cu:693-745):
 * 0 enable (arg = last MoE layer | per_layer << 16), 1 arm -> target,
 * 2 wait((layer << 40) | target) on the host (at most 2 s), then the copy
 * stream waits on the layer's event on the device, 3 open (host),
 * 4 stats (arg 0 waits, 1 timeouts, 2 wait us), 5 engine pacing (accepted,
 * every copy is issued at once), 6 engine stats (0).  moert_ffn_moe's down
 * fire of a gated layer records the event. */
int64_t moert_cuda_dir_gate(int32_t op, int64_t arg);

/* Replaces moert_cuda_set_hot_table (cuda.h:276): per (layer, kind) table of
 * n slot base pointers (device array) the hot matmul reads instead of the
 * contiguous pool; n = 0 clears it. */
void moert_cuda_set_hot_table(int32_t il, int32_t kind, const void * const * dev_ptrs, int32_t n, int32_t type_tag);

#ifdef __cplusplus
}
#endif
#endif
