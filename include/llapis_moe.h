/*
 * llapis_moe.h -- the MI355X dual-precision MoE expert FFN: entry points
 * beside the moert island ABI (moert_hip.h).
 *
 * All device entry points take device pointers and a hipStream_t passed as
 * void*, never allocate (scratch comes from the caller: a workspace pointer
 * and its size, or the island's host->pool_alloc), and launch asynchronously
 * on that stream.  Functions returning int32_t return 0 on success and a
 * negative code on a refused call; llapis_last_error() then says why.
 *
 * Weight pools hold ggml blocks byte-for-byte (ggml-common.h layouts):
 * an expert is a contiguous [d_out rows][row_size(type, d_in)] slab and a
 * pool is slabs back to back.  Type tags are ggml's (ggml.h:390-412).
 */
#ifndef LLAPIS_MOE_H
#define LLAPIS_MOE_H

#include <stdint.h>

#include "moert_hip.h"
#include "moert_policy.h"

#ifdef __cplusplus
extern "C" {
#endif

enum {
    LLAPIS_T_F32 = 0, LLAPIS_T_Q5_0 = 6, LLAPIS_T_Q8_0 = 8, LLAPIS_T_Q8_1 = 9,
    LLAPIS_T_Q4_K = 12, LLAPIS_T_Q8_K = 15, LLAPIS_T_IQ4_NL = 20, LLAPIS_T_IQ2_S = 22,
};

/* Activation format of the integer dot products.
 *  LLAPIS_ACT_CPU:  what the reference CPU path quantises to -- q8_K for
 *                   256-wide blocks, q8_0 for 32-wide blocks (ggml-cpu.c:
 *                   250-373 vec_dot_type; quants.c / arch/x86/quants.c).
 *  LLAPIS_ACT_Q8_1: q8_1 and the per-block arithmetic of ggml-cuda's
 *                   vec_dot_*_q8_1 (quantize.cu:5-50, vecdotq.cuh). */
enum { LLAPIS_ACT_CPU = 0, LLAPIS_ACT_Q8_1 = 1 };
/* GELU of the GEGLU: the CPU's fp16 table (vec.h:1414-1428) or exact tanh
 * (ggml-cuda unary.cuh:101-104). */
enum { LLAPIS_GELU_TABLE = 0, LLAPIS_GELU_TANH = 1 };

const char * llapis_last_error(void);

/* Modes used by moert_ffn_moe's matmuls (the island ABI has no field for
 * them).  Defaults: LLAPIS_ACT_CPU, LLAPIS_GELU_TABLE. */
void llapis_set_modes(int32_t act_mode, int32_t gelu_mode);

/* ------------------------------------------------------------ host side */

/* Bytes of a row of n values of `type`; 0 if unsupported. */
uint64_t llapis_row_size(int32_t type, int64_t n);

/* Replaces ggml_quantize_chunk (ggml.c:7761-7800) for Q4_K, Q5_0 (imatrix
 * NULL), IQ2_S and IQ4_NL (imatrix or NULL), byte-identical output.
 * Multithreaded on the host.  Returns bytes written, 0 if refused. */
uint64_t llapis_quantize(int32_t type, const float * src, void * dst, int64_t nrow, int64_t n_per_row,
                         const float * imatrix);

/* Seeded N(mean, std) synthetic data; element i depends on (seed, offset+i) only. */
void llapis_synth_normal(uint64_t seed, int64_t offset, int64_t n, float mean, float stddev, float * out);

/* ---------------------------------------------------------- device side */

/* The quantised mul_mat_id service for moert_ffn_moe_host.mm: replaces the
 * trampoline's call of ggml_cuda_mul_mat_vec_q (ggml-cuda/moe-dual.cu:74-94,
 * mmvq.cu:470-640).  For channel i < *ne_live (or < n_ids):
 *   y[i*d_out + r] = W_{ids[i]}[r, :] . b[:, b_ncols == 1 ? 0 : i]
 * with W_{j} = w_ptrs ? w_ptrs[j] : w_base + j * row_size(w_type, d_in) * d_out,
 * activations quantised on the fly in the mode set by llapis_set_modes.
 * Every expert slab must be a multiple of 16 bytes. */
int32_t llapis_mul_mat_id(const moert_mm_call * call, int32_t w_type, const void * w_base, int64_t w_n,
                          int32_t d_in, int32_t d_out, void * stream);

/* A ggml tensor as the op sees it (ggml.h ggml_tensor: type, ne, nb, data). */
typedef struct llapis_tensor {
    int32_t  type;
    int64_t  ne[4];
    uint64_t nb[4];
    void *   data;
} llapis_tensor;

/* Replaces ggml_cuda_moe_dual (ggml-cuda/moe-dual.cu:98-157): GGML_OP_MOE_DUAL
 * with srcs {cur, ids, w_hot, w_cold, exp_slot, slot_exp, slot_state, s_hot,
 * s_cold} and op_params {kind, top_k, il, cold_type, n_expert, w_cold_dev(2),
 * s_cold_dev(2), planc_mode} (ggml.c:3322-3370), dst f32 [d_out, n_used, T].
 * The island's LIFO scratch comes from `workspace` (see
 * llapis_moe_dual_workspace_size). */
typedef struct llapis_moe_dual_op {
    const llapis_tensor * src[9];
    int32_t op_params[10];
    llapis_tensor * dst;
} llapis_moe_dual_op;
uint64_t llapis_moe_dual_workspace_size(const llapis_moe_dual_op * op);
int32_t  llapis_moe_dual_compute(const llapis_moe_dual_op * op, void * workspace, uint64_t ws_bytes, void * stream);

/* Router + selection (llama-graph.cpp:1548-1650; ggml-cuda topk-moe.cu:80):
 * logits = W_r x_t (+ bias), p = softmax, ids = top_k of p (descending, ties
 * to the lower index), w = p[ids] / max(sum p[ids], 6.103515625e-5).
 * x [T][d], W_r [n_expert][d] (ggml ne0 = d), bias [n_expert] or NULL,
 * ids/w [T][top_k], probs [T][n_expert] (required: it also holds the logits
 * between the two kernels).  n_expert <= 256, top_k <= 16, d a multiple of
 * 4.  The logits are computed in the same order as llapis_moe_ffn's decode
 * path, so both route a token alike. */
int32_t llapis_router_topk(const float * x, int32_t n_tokens, const float * w_r, const float * bias,
                           int32_t d, int32_t n_expert, int32_t top_k,
                           int32_t * ids, float * weights, float * probs, void * stream);

/* GEGLU over the merged gate_up output (llama-graph.cpp:1687-1761):
 * out[c][i] = gelu(gu[c][i]) * gu[c][n_ff + i] for n_cols columns of 2*n_ff. */
int32_t llapis_geglu(const float * gate_up, int32_t n_ff, int32_t n_cols, float * out, int32_t gelu_mode,
                     void * stream);

/* The weighted sum of each token's expert outputs (llama-graph.cpp:1812-1840:
 * ggml_mul by the routing weights, then the top_k views added in order):
 * out[t][r] = ((w[t][0] y[t K][r] + w[t][1] y[t K + 1][r]) + ...) for
 * y [n_tokens * top_k][d] (the down fire's output), w [n_tokens][top_k]. */
int32_t llapis_moe_combine(const float * y, const float * weights, int32_t n_tokens, int32_t top_k, int32_t d,
                           float * out, void * stream);

/* The glue between two layers of a residual stream, in one kernel: h += add
 * (when add is not NULL; h [n_tokens][d] updated in place), then
 * x = h / sqrt(mean(h^2) + eps) per token (ggml_rms_norm without a weight:
 * the sum of squares in fp32 in a fixed order, an IEEE square root and
 * division).  Not part of the MoE operator: the residual add and the next
 * block's input norm a model runs between its blocks (llama-graph.cpp
 * build_norm, ggml_add), here for a stack of MoE layers that skips
 * attention. */
int32_t llapis_residual_rmsnorm(float * h, const float * add, int32_t n_tokens, int32_t d, float eps, float * x,
                                void * stream);

/* One dual-precision MoE FFN layer: build_moe_ffn's merged gate_up path for
 * gemma4-style MoE (llama-graph.cpp:1507-1850) with each routed pair computed
 * at its tier.  Pools are device slabs (see the note at the top):
 *   hot_gu  [k_slots][2 n_ff][row(hot_gu_type, d_model)]
 *   hot_dn  [k_slots][d_model][row(hot_dn_type, n_ff)]
 *   cold_gu [n_expert][2 n_ff][row(cold_gu_type, d_model)]
 *   cold_dn [n_expert][d_model][row(cold_dn_type, n_ff)]
 * A pair (t, e) is hot iff exp_slot[e] = s, 0 <= s < k_slots,
 * slot_state[s] == 2 (READY) and slot_exp[s] == e (ffn_moe.cu:80-130). */
typedef struct llapis_moe_layer {
    int32_t d_model, n_ff, n_expert, top_k, k_slots;
    int32_t hot_gu_type, hot_dn_type, cold_gu_type, cold_dn_type;
    int32_t act_mode, gelu_mode;
    const float * router_w;        /* [n_expert][d_model] */
    const float * router_b;        /* [n_expert] or NULL */
    const void * hot_gu;  const void * hot_dn;
    const void * cold_gu; const void * cold_dn;
    const int32_t * exp_slot;      /* [n_expert] */
    const int32_t * slot_exp;      /* [k_slots] */
    const int32_t * slot_state;    /* [k_slots] */
    const float * s_hot;           /* [k_slots] down scale, or NULL */
    const float * s_cold;          /* [n_expert] down scale, or NULL */
    /* Routing counters (replaces the island's, ffn_moe.cu:123-128, for this
     * entry point), or NULL: every call adds, with device atomics, its routed
     * pairs per expert to route_counts[n_expert] and its hot pairs and other
     * pairs to route_hits[0] and [1] (route_hits may be NULL).  The caller
     * owns, zeroes and reads them (e.g. a row of the moert_cuda_route_counts
     * layout, fetched at refresh points into moert_policy_add_external_counts). */
    int32_t * route_counts;
    int32_t * route_hits;
} llapis_moe_layer;

/* Device scratch the layer needs for n_tokens (bytes). */
uint64_t llapis_moe_ffn_workspace_size(const llapis_moe_layer * L, int32_t n_tokens);

/* out [T][d_model] = the layer applied to x [T][d_model] (the experts'
 * input), routed on x_router [T][d_model]: logits = W_r x_router (+ b).
 * x_router NULL routes on x.  Gemma4's MoE block routes on a tensor of its
 * own (gemma4.cpp:393-403: the experts read ffn_pre_norm_2(attn_out), the
 * router rms_norm(attn_out) / sqrt(n_embd) * ffn_gate_inp_s, handed to
 * build_moe_ffn as probs_in, llama-graph.cpp:1537-1541); pass that tensor
 * as x_router and ffn_gate_inp as router_w.  ids/weights ([T][top_k],
 * optional) receive the routing.  Batches of up to 4 tokens take the
 * three-kernel decode path.  Each call writes every workspace word before it
 * reads it, so nothing is carried from one call to the next (and calls can
 * be captured in HIP graphs); calls that share a workspace must not run
 * concurrently. */
int32_t llapis_moe_ffn(const llapis_moe_layer * L, const float * x, const float * x_router, int32_t n_tokens,
                       float * out, int32_t * ids, float * weights, void * workspace, uint64_t ws_bytes, void * stream);

/* llapis_moe_ffn without a workspace argument.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * call's scratch is a fixed device array of LLAPIS_NOALLOC_SCRATCH_BYTES in
 * the library, one per GPU, held until the process ends; nothing is
 * allocated.  A call whose llapis_moe_ffn_workspace_size exceeds it is
 * refused (-1, llapis_last_error() says how much it needs): at the
 * benchmark's shapes (d_model 2816, n_ff 704, 128 experts, top-8) that
 * admits batches of up to 61 tokens.  Nothing is launched to prepare the
 * array: every call writes each scratch word before it reads it, so the first
 * call may itself be captured in a HIP graph.  Every call on one GPU shares
 * that GPU's array and leaves its contents behind: calls that overlap on one
 * GPU (other streams, other threads) race, so order them as one stream
 * would. */
#define LLAPIS_NOALLOC_SCRATCH_BYTES (8u << 20)
int32_t llapis_moe_ffn_noalloc(const llapis_moe_layer * L, const float * x, const float * x_router,
                               int32_t n_tokens, float * out, int32_t * ids, float * weights, void * stream);

/* Zero the control block at the start of a workspace (a kernel on
 * `stream`).  Optional: no call reads a workspace word it has not written. */
int32_t llapis_moe_ffn_workspace_init(const llapis_moe_layer * L, void * workspace, uint64_t ws_bytes, void * stream);

/* ------------------------------------------------------ promotion engine
 *
 * Replaces the transfer engine and the memmgr's promotion for a hot slab in
 * HBM (src/moe_xfer.hpp:55-110 start/submit/flush/take_done/
 * promotions_in_flight/wait_idle/stats; moert/memmgr.h:147-158
 * moert_memmgr_promote): a promotion copies every page group of expert e of
 * layer il from its promotion source into hot slot `slot`.  Mechanism only,
 * as the reference's: the policy decides and marks the slot FILLING
 * (moert/policy.h:95-104, stream_expert returning 2), the host submits, and
 * applies each completion with moert_policy_complete_fill (ok) or
 * moert_policy_abort_fill (failed), then publishes the layer's mirrors.
 *
 * Ordering contract (the reference's submit/flush split): submitted jobs stay
 * pending until llapis_xfer_flush(after_stream), which starts their copies on
 * the engine's own stream only after all work already queued on
 * after_stream -- so publish the mirrors that mark the slots FILLING (and
 * queue every fire that may still read the old experts) before flushing.
 * The pages of device sources move in copy kernels of at most copy_wgs
 * workgroups (one launch per 96 pages of a flush), so the copies leave the
 * other CUs to the decode; copy_wgs 0, or a pinned host source:
 * hipMemcpyAsync.  The jobs of one flush complete together. */
#define LLAPIS_XFER_MAX_GROUPS 4
typedef struct llapis_xfer llapis_xfer;
typedef struct llapis_xfer_done {
    int32_t il, e, slot;
    int32_t ok;                    /* 1 copied, 0 a copy failed */
} llapis_xfer_done;
typedef struct llapis_xfer_stats {
    long long submitted, completed, failed;
    long long max_queue;           /* most jobs issued by one flush */
    long long bytes;               /* bytes of the copies issued */
    long long wait_idle_calls;
    double    wait_idle_ms;
} llapis_xfer_stats;
/* NULL on bad geometry (llapis_xfer_last_error says why). */
llapis_xfer * llapis_xfer_create(int32_t n_layers, int32_t n_expert, int32_t k_slots, int32_t copy_wgs);
/* Waits for the copies in flight, then frees the engine. */
void          llapis_xfer_free(llapis_xfer * x);
const char *  llapis_xfer_last_error(void);
/* Page group `group` (< LLAPIS_XFER_MAX_GROUPS) of layer il -- one group per
 * (kind, weight|scale) as the memmgr's page groups (memmgr.h:120-135): expert
 * e's bytes_per_expert bytes at src + e * src_stride go to
 * slab + slot * bytes_per_expert.  slab: device memory; src: device memory or
 * pinned host memory.  0 ok, -1 refused. */
int32_t llapis_xfer_set_group(llapis_xfer * x, int32_t il, int32_t group, void * slab, const void * src,
                              uint64_t src_stride, uint64_t bytes_per_expert);
/* Queue a promotion (pending until flush).  0 ok, -1 out of range. */
int32_t llapis_xfer_submit(llapis_xfer * x, int32_t il, int32_t e, int32_t slot);
/* Issue every pending job, ordered after the work queued on after_stream. */
int32_t llapis_xfer_flush(llapis_xfer * x, void * after_stream);
/* Move up to max_out finished jobs, oldest first, into out; non-blocking.
 * Returns how many were moved (-1 on a null argument). */
int32_t llapis_xfer_take_done(llapis_xfer * x, llapis_xfer_done * out, int32_t max_out);
/* Jobs pending or with copies in flight (not yet taken). */
int64_t llapis_xfer_in_flight(llapis_xfer * x);
/* Flush, then block until every copy issued has landed. */
int32_t llapis_xfer_wait_idle(llapis_xfer * x, void * after_stream);
void    llapis_xfer_get_stats(llapis_xfer * x, llapis_xfer_stats * out);

/* ------------------------------------------------------ residency loop
 *
 * The per-token host loop around the fused op in native code: a policy
 * (moert_policy.h, external observation), a promotion engine and the
 * device routing counters of every layer, as moe_dual.cpp drives them
 * (publish_fence / push_residency moe_dual.cpp:640-705, the batch transport
 * :862-880, the policy callbacks policy.h:82-104).  Give each layer's
 * llapis_moe_layer the counters of llapis_residency_counters, register its
 * mirrors and its engine page groups, seed the policy, publish once; then
 * after each visible token's layers are queued on `stream` call
 * llapis_residency_token_end, which (1) hands finished copies to the policy
 * (READY), (2) runs the per-token decision -- it pulls every layer's counters
 * with one copy on `stream`, the loop's only wait (for the token), and
 * submits promotions as FILLING -- (3) publishes the changed layers' mirrors
 * with copies on `stream` (the next token sees them in stream order) and (4)
 * flushes the engine, whose copies overlap the next token.  Counts reach the
 * policy only there and in llapis_residency_refresh (stats reads and
 * refreshes called on the policy directly do not pull them). */
typedef struct llapis_residency llapis_residency;
typedef struct llapis_residency_stats {
    long long tokens, fetches, submitted, completed, publications;
    long long hot_pairs, cold_pairs;     /* routed pairs the counters saw */
    double wait_ms;                      /* in token_end, waiting for the token's kernels */
    double host_ms;                      /* in token_end, everything else (the loop's own cost) */
} llapis_residency_stats;
/* cfg as moert_policy_create's (callbacks are the runtime's own); copy_wgs
 * as llapis_xfer_create's.  Allocates the counters (device), their pinned
 * read-back and the publication staging, sized for the largest capacity in
 * cfg.  After a K re-fit (moert_policy_resize_k) publish every layer with
 * llapis_residency_publish_all; a capacity above the one at creation needs a
 * new runtime, and publication fails with an error rather than write past
 * the staging.  All
 * calls on one runtime must come from one thread.  NULL on failure (the
 * geometry is checked before any device call). */
llapis_residency * llapis_residency_create(const moert_policy_config * cfg, int32_t copy_wgs);
/* Waits for the engine's copies and the last publication; the calls that
 * count into the runtime's counters must have completed before it is freed
 * (synchronise their stream first). */
void               llapis_residency_free(llapis_residency * r);
const char *       llapis_residency_last_error(void);
/* The policy (seed it, read views and stats) and the engine (set its page
 * groups) the runtime drives. */
moert_policy *     llapis_residency_policy(llapis_residency * r);
llapis_xfer *      llapis_residency_xfer(llapis_residency * r);
/* Layer il's device mirrors: exp_slot [n_expert], slot_exp and slot_state
 * [the policy's capacity]. */
int32_t llapis_residency_set_mirrors(llapis_residency * r, int32_t il, int32_t * exp_slot, int32_t * slot_exp,
                                     int32_t * slot_state);
/* Layer il's counters for llapis_moe_layer.route_counts / route_hits. */
int32_t llapis_residency_counters(llapis_residency * r, int32_t il, int32_t ** counts, int32_t ** hits);
/* Every layer's mirrors, copied on stream (after seeding). */
int32_t llapis_residency_publish_all(llapis_residency * r, void * stream);
int32_t llapis_residency_token_end(llapis_residency * r, void * stream);
/* The same steps around moert_policy_refresh(reason) (a MOERT_REFRESH_*
 * value): the prompt-end and turn-end decisions (moe_dual.cpp calls them at
 * those points).  Prompt tokens are counted with moert_policy_on_prompt_token
 * on llapis_residency_policy(r); their routing stays in the counters until
 * the next token_end or refresh drains them. */
int32_t llapis_residency_refresh(llapis_residency * r, int32_t reason, void * stream);
void    llapis_residency_get_stats(llapis_residency * r, llapis_residency_stats * out);

/* ------------------------------------------------------------ model files
 *
 * The on-disk sources of expert pages, read into device memory.  GGUF model
 * files (versions 2 and 3 of the format ggml's gguf.cpp reads): the tensor
 * table with absolute file offsets, and the stacked expert tensors
 * blk.L.ffn_{gate_up,down}_exps.{weight,scale} as the page groups the
 * memmgr registers from them (moe_dual_init.cpp:230-263: the expert axis is
 * the highest dimension equal to n_expert, bytes per expert its stride).
 * The expert store is in moert_store.h.  Uploads read the file with pread
 * into two pinned staging buffers in turn, each copied to the device with
 * hipMemcpyAsync on `stream` while the next read runs, and return when the
 * copies have landed.  Errors: -1 / NULL with llapis_files_last_error(). */
typedef struct llapis_gguf llapis_gguf;
typedef struct llapis_gguf_tensor_info {
    char     name[64];
    int32_t  type;             /* ggml_type value */
    int32_t  n_dims;
    int64_t  ne[4];
    uint64_t nb[4];            /* 0 for a type this build cannot size */
    uint64_t offset;           /* absolute file offset of the data */
    uint64_t nbytes;
} llapis_gguf_tensor_info;
typedef struct llapis_page_group {
    int32_t  type;
    int32_t  expert_axis;
    int32_t  n_expert;
    int32_t  reserved;
    int64_t  ne[4];
    uint64_t offset;           /* absolute file offset of expert 0 */
    uint64_t bytes_per_expert;
} llapis_page_group;
const char *  llapis_files_last_error(void);
llapis_gguf * llapis_gguf_open(const char * path);
void          llapis_gguf_close(llapis_gguf * g);
int64_t       llapis_gguf_n_tensors(const llapis_gguf * g);
uint64_t      llapis_gguf_data_offset(const llapis_gguf * g);
uint64_t      llapis_gguf_alignment(const llapis_gguf * g);
int32_t       llapis_gguf_tensor(const llapis_gguf * g, int64_t i, llapis_gguf_tensor_info * out);
int64_t       llapis_gguf_find(const llapis_gguf * g, const char * name);
/* kind 0 gate_up, 1 down; is_scale 1 = the .scale tensor.  0 ok. */
int32_t       llapis_gguf_expert_group(const llapis_gguf * g, int32_t layer, int32_t kind, int32_t is_scale,
                                       int32_t n_expert, llapis_page_group * out);
/* experts [e0, e0 + n) of the group into dst (n * bytes_per_expert bytes). */
int32_t       llapis_gguf_upload(const llapis_gguf * g, const llapis_page_group * grp, int32_t e0, int32_t n,
                                 void * dst, void * stream);
/* Pages (layer, kind, is_scale, experts[i]) of an expert store into
 * dst + i * dst_stride (verify: checksums checked as the bytes stream).  0 ok. */
struct moert_store_reader;
int32_t       llapis_store_upload(struct moert_store_reader * r, int32_t layer, int32_t kind, int32_t is_scale,
                                  const int32_t * experts, int32_t n, void * dst, uint64_t dst_stride,
                                  int32_t verify, void * stream);

/* ------------------------------------------------------------ K re-fit
 *
 * Replaces kfit::fit (src/kfit_policy.hpp:38-94), the decision of how many
 * hot slots per layer fit in device memory, with its four rules unchanged:
 * pool = slab_now + free (bounded by slab_now + headroom when headroom >= 0);
 * k = (pool - keep_free) / per_k, lifted to k_min, capped at n_expert, and
 * capped at pool / per_k (floor_capped); no rebuild within one slot of k_cur
 * unless the slab is evicted.  Host code.  On one MI355X there is no WDDM
 * budget (headroom -1) and 288 GB holds every expert, so the usual answer is
 * k = n_expert; the host then re-lays the slab (moert_policy_resize_k, the
 * survivors re-streamed into their new slots with llapis_xfer_*) as
 * slab_rebuild_at_k does (moe_dual_init.cpp:684-790). */
typedef struct llapis_kfit_inputs {
    long long free_mib;        /* device-free memory now */
    long long slab_mib_now;    /* the slab's bytes now; 0 when evicted */
    long long headroom_mib;    /* per-process budget; < 0: none */
    long long per_k_mib;       /* one slot across all layers */
    long long keep_free_mib;   /* margin left unallocated */
    int32_t   k_cur, k_min, n_expert;
    int32_t   evicted;
} llapis_kfit_inputs;
typedef struct llapis_kfit_decision {
    int32_t   k;
    int32_t   rebuild, wddm_bound, floor_capped;
    long long pool_mib;
} llapis_kfit_decision;
void    llapis_kfit(const llapis_kfit_inputs * in, llapis_kfit_decision * out);
/* Free and total memory of the current device in MiB (hipMemGetInfo):
 * free_mib for llapis_kfit_inputs.  0 ok, -1 on a HIP error. */
int32_t llapis_device_memory_mib(long long * free_mib, long long * total_mib);

/* Switches for measurement: key 0 = the decode path for <= 4 tokens
 * (default 1; 0 sends those calls down the generic path), key 2 = the MFMA
 * prefill path for > 4 tokens (default 1), key 3 = log2 of the output rows
 * per workgroup of the decode path's down kernel (0..5; -1, the default,
 * picks it from d_model), key 4 = the decode path's down kernel for 2-4
 * tokens (1, the default: by expert group with a combine kernel after it;
 * 0: over every group with the combine in it), key 6 = the one-kernel fires of
 * llapis_moe_dual_compute and of llapis_mul_mat_id (default 1; 0 runs every
 * fire through the island's generic pipeline and every mul_mat_id through
 * the generic matvec).  Other keys are ignored. */
void llapis_set_tuning(int32_t key, int32_t value);

/* Stage timing of llapis_moe_ffn for measurement (not under stream capture):
 * while enabled, every call times its stages on the call's stream with HIP
 * events -- a stage that is one kernel (gate_up and down on both paths; the
 * decode path's router+top-k kernel, reported as the router stage) takes the
 * dispatch's own begin/end timestamps, the generic path's router, top-k and
 * combine kernels are bracketed by event records.  llapis_profile_read waits
 * for the events, writes the summed milliseconds per stage {router, top-k,
 * gate_up, down, combine} to ms[0..n) (0 for a stage the path does not have)
 * and returns the number of timed calls since the last read (-1 on a HIP
 * error); reading resets the sums.  Disabled by default (no events). */
void    llapis_profile_enable(int32_t on);
int32_t llapis_profile_read(float * ms, int32_t n);

#ifdef __cplusplus
}
#endif
#endif
