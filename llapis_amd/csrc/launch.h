// launch.h -- host-visible launchers of the gfx950 kernels (defined in the
// .hip translation units) and the parameter blocks they take.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llapis {

// How a matvec channel (blockIdx.y) finds its weights, activation and output.
enum { MMV_COMPACT = 0, MMV_ROUTED = 1 };

struct MmvParams {
    int mode;                    // MMV_COMPACT or MMV_ROUTED
    int d_in, d_out;
    int w_lds_bytes;             // LDS bytes reserved for staged weights (host computed)
    // tier 0 (the hot pool, or the only pool) and tier 1 (the cold pool)
    const uint8_t * w0; uint64_t stride0; const void * const * ptrs0; int64_t n0;
    const uint8_t * w1; uint64_t stride1; int64_t n1;
    // MMV_COMPACT: channel i uses expert/slot ids[i], column (b_ncols == 1 ? 0 : i)
    const int32_t * ids; const int32_t * ne_live; int b_ncols;
    // MMV_ROUTED: channel p is routed pair p of token p / top_k (ids row stride ids_s1)
    int top_k, ids_s1, n_expert, k_slots;
    const int32_t * exp_slot; const int32_t * slot_exp; const int32_t * slot_state;
    const float * s0; const float * s1;      // per-slot / per-expert output scale, or NULL
    int act_by_token;                        // activation column: token (1) or pair (0)
    // activations: column c starts at act + c * act_ld
    const float * act; int64_t act_ld;
    float * y;                               // y[ch * d_out + r]
};

// rows of one workgroup for a weight type
int mmv_rows_per_wg(int wtype);
// dynamic LDS bytes of a matvec launch; 0 if the shape is not supported
int mmv_lds_bytes(const MmvParams & p, int ht, int ct);
// fill w_lds_bytes for the format pair
void mmv_prepare(MmvParams & p, int ht, int ct);
// launch over n_channels channels; returns hipSuccess or the launch error
// e0/e1 (optional, profiling): receive the dispatch's begin and end timestamps
hipError_t launch_mmv(const MmvParams & p, int ht, int ct, int act_mode, int src, int n_channels, hipStream_t s,
                      hipEvent_t e0 = nullptr, hipEvent_t e1 = nullptr);

// ------------------------------------------------------------ decode path

constexpr int DEC_MAXT = 4;     // tokens per decode call (a 3-deep MTP verify plus the token)
constexpr int DEC_PMAX = 64;    // routed pairs per call (DEC_MAXT * top_k, top_k <= 16)

// one routed expert of the call and the pairs that use it
struct GroupInfo {
    int tier;                   // 0 hot (idx = slot), 1 cold (idx = expert), 2 invalid id
    int idx;
    int n_mem;
    int ord;                    // the gate_up kernel's item order: group ord is the (this entry's index)-th cheapest
    int mem[DEC_MAXT];          // routed-pair indices, one per member token
};

constexpr int DEC_DN_MAXR = 32;  // output rows of one down workgroup, at most
constexpr int DEC_GU_BLK = 32;   // gate rows of one gate_up item (one q8 block of the down activations)

// control block at the start of the decode workspace: the expert groups the
// gate_up kernel selected, for the down kernel
struct DecCtl {
    int n_groups;
    int pad[3];
    GroupInfo groups[DEC_PMAX];
};

struct DecParams {
    int d_model, n_ff, n_expert, top_k, k_slots, T;
    const float * x;            // [T][d_model] the experts' input
    const float * xr;           // [T][d_model] the router's input
    const float * router_w;
    const float * router_b;
    const uint8_t * hot_gu; uint64_t hot_gu_stride;
    const uint8_t * cold_gu; uint64_t cold_gu_stride;
    const uint8_t * hot_dn; uint64_t hot_dn_stride;
    const uint8_t * cold_dn; uint64_t cold_dn_stride;
    const int32_t * exp_slot; const int32_t * slot_exp; const int32_t * slot_state;
    const float * s_hot; const float * s_cold;
    DecCtl * ctl;
    float * logits;             // [T][n_expert]
    int32_t * ids;              // [T][top_k]
    float * w;                  // [T][top_k]
    uint8_t * xq; int64_t xq_stride;     // quantised tokens
    uint8_t * yq; int64_t yq_stride;     // [P] quantised down activations (GEGLU outputs in q8_0 / q8_1)
    float * ydn;                // [P][d_model] scaled down rows per routed pair (down by group, T > 1)
    int dn_by_group;            // T > 1: 1 the down kernel by group + k_dec_combine, 0 the kernel over every group
    float * out;                // [T][d_model]
    int w_lds_gu;               // LDS bytes of one half of a gate_up pass (dec_gu_half_bytes)
    int dn_rows_log2;           // log2 of the output rows per down workgroup (<= DEC_DN_MAXR)
    int32_t * rc_counts;        // [n_expert] routed pairs per expert, or NULL
    int32_t * rc_hits;          // [2] hot pairs, other pairs (with rc_counts)
};

int dec_act_bytes(int n);
int dec_gu_half_bytes(int T, int row_bytes);
int dec_lds_gate_up(const DecParams & p, int ht, int ct);
int dec_lds_down(const DecParams & p);
// ev (optional, profiling): 8 events that receive the begin and end
// timestamps of the router, gate_up, down and combine kernels (ev[0..1],
// ev[2..3], ev[4..5], ev[6..7]; the last two stay unrecorded at one token,
// which has no combine kernel).
hipError_t launch_decode(const DecParams & p, int hgu, int cgu, int hdn, int cdn, int act_mode, int gelu_src,
                         hipStream_t s, hipEvent_t * ev);
hipError_t launch_zero_i32(int * p, int n, hipStream_t s);

// One fire of the dual op in one kernel (the island's partition, gather,
// mul_mat_id and scatter fused): see k_fire_k256 / k_fire_k32.
struct FireParams {
    int kind, d_in, d_out, n_used, n_tokens, ids_s1, n_expert, k_slots;
    const float * cur;          // kind 0: [n_tokens][d_in] token columns; kind 1: [n_tokens * n_used][d_in]
    const int32_t * ids;        // [n_tokens] rows of stride ids_s1
    const int32_t * exp_slot; const int32_t * slot_exp; const int32_t * slot_state;
    const uint8_t * hot; uint64_t hot_stride;     // slab bytes per slot
    const uint8_t * cold; uint64_t cold_stride;   // slab bytes per expert
    const float * s_hot; const float * s_cold;
    float * dst;                // [n_tokens * n_used][d_out]
    int32_t * rc_counts;        // routing counters of a gate_up fire, or NULL
    int32_t * rc_hits;
    int w_lds;                  // LDS bytes of 16 staged rows (256-value block formats)
    int cur_shared;             // 1: every pair reads cur's first column (mul_mat_id with one shared column)
    const int32_t * n_live;     // device count of the pairs to compute (the rest are left untouched), or NULL
};
int fire_lds(const FireParams & f, int ht, int ct);
hipError_t launch_fire(const FireParams & f, int ht, int ct, int act_mode, hipStream_t s);

// ------------------------------------------------------------ prefill path

constexpr int PF_ROWS = 128;          // weight rows per workgroup (4 waves x 32)
constexpr int PF_TOK = 96;            // routed pairs per down group (six 16-token MFMA tiles)
constexpr int PF_GTOK = 128;          // routed pairs per gate_up group, at most
constexpr int PF_MAX_PAIRS = 4096;    // routed pairs per prefill launch (T * top_k)
constexpr int PF_MAX_FF = 4096;       // longest n_ff the down activation kernel stages

// a group: a run of up to PF_TOK pairs routed to one expert
struct PfTile {
    int tier;                   // 0 hot (idx = slot), 1 cold (idx = expert)
    int idx;
    int begin;                  // first entry in the sorted pair list
    int n;
};

struct PfParams {
    int d_model, n_ff, n_expert, top_k, k_slots, T;
    const float * x;                     // [T][d_model]
    const int32_t * ids;                 // [T][top_k]
    const int32_t * exp_slot; const int32_t * slot_exp; const int32_t * slot_state;
    const uint8_t * hot_gu; uint64_t hot_gu_stride;
    const uint8_t * cold_gu; uint64_t cold_gu_stride;
    const uint8_t * hot_dn; uint64_t hot_dn_stride;
    const uint8_t * cold_dn; uint64_t cold_dn_stride;
    const float * s_hot; const float * s_cold;
    int * n_tiles;                       // [1]
    int32_t * sorted;                    // [P] pair indices grouped by expert, ascending within
    PfTile * tiles;                      // [max_tiles]
    int max_tiles;
    // the gate_up kernel's groups: runs of up to gcap[tier] pairs of one
    // expert, the full groups of every expert first, then the remainders
    PfTile * gtiles;                     // [max_gtiles]
    int * n_gtiles;                      // [1]
    int max_gtiles;
    int gcap[2];                         // hot, cold (a multiple of 16 in [16, PF_GTOK])
    int8_t * xq;                         // [T][d_model] q8_K values
    float * xd;                          // [T][d_model / 256] q8_K scales
    _Float16 * xm;                       // [T][d_model / 256][16] q8_K: per-32 sums as 32 hi + lo;
                                         //   q8_1: per-32 d sum(q) as hi, lo
    int act_mode;                        // AM_CPU (q8_K / q8_0) or AM_Q8_1
    _Float16 * xh;                       // [T][d_model / 256][512] q8_1 values d q as fp16 hi (256), lo (256)
    _Float16 * ah;                       // [P][n_ff] down activations d8 q: fp16 high part
    _Float16 * al;                       // [P][n_ff]                        exact remainder
    float * ydn;                         // [P][d_model]
    int32_t * rc_counts;                 // [n_expert] routed pairs per expert, or NULL
    int32_t * rc_hits;                   // [2] hot pairs, other pairs (with rc_counts)
};

int pf_max_tiles(int P, int n_expert);
int pf_max_gtiles(int P, int n_expert);
// ev (optional, profiling): begin/end timestamps of the gate_up and down GEMMs
hipError_t launch_prefill(const PfParams & p, int hgu, int cgu, int hdn, int cdn, int gelu_src, hipStream_t s,
                          hipEvent_t * ev);

hipError_t launch_router_logits(const float * x, int T, const float * w_r, const float * bias, int d, int E,
                                float * logits, hipStream_t s);
hipError_t launch_topk(float * probs_inout, int T, int E, int K, int32_t * ids, float * w, hipStream_t s);
// Router logits on the matrix cores (d a multiple of 256): the K-split
// partial dot products go to `parts` (router_parts_floats(T, E) floats);
// launch_topk_parts adds them in split order plus the bias, then selects as
// launch_topk (probs, ids, w).
int router_parts_floats(int T, int E);
hipError_t launch_router_mfma(const float * x, int T, const float * w_r, int d, int E, float * parts, hipStream_t s);
hipError_t launch_topk_parts(const float * parts, const float * bias, int T, int E, int K, float * probs, int32_t * ids,
                             float * w, hipStream_t s);
hipError_t launch_combine(const float * y, const float * w, int T, int K, int D, float * out, hipStream_t s);
hipError_t launch_residual_rmsnorm(float * h, const float * add, int T, int d, float eps, float * x, hipStream_t s);
hipError_t launch_geglu(const float * gu, int F, int n_cols, float * out, int mode, hipStream_t s);

hipError_t launch_partition(const int32_t * ids, int n_used, int ids_s1, int n_pairs, const int32_t * exp_slot,
                            const int32_t * slot_exp, const int32_t * slot_state, int n_expert, int K,
                            int32_t * ids_hot, int32_t * ids_cold, int32_t * hot_dst, int32_t * cold_dst,
                            int32_t * counts, int32_t * rc_counts, int32_t * rc_hits, hipStream_t s);
// Routing counters for n_pairs routed ids (row stride ids_s1, n_used per
// token): as the partition kernel counts them.  One workgroup.
hipError_t launch_route_count(const int32_t * ids, int n_used, int ids_s1, int n_pairs, const int32_t * exp_slot,
                              const int32_t * slot_exp, const int32_t * slot_state, int n_expert, int K,
                              int32_t * rc_counts, int32_t * rc_hits, hipStream_t s);
// Transport hook of moert_ffn_moe: the early-decision gate's event after a
// gated layer's last fire.
void dir_gate_after_fire(int il, int kind, hipStream_t stream);
hipError_t launch_gather(const float * cur, int D_in, int kind, int n_used, const int32_t * counts,
                         const int32_t * hot_dst, const int32_t * cold_dst, float * x_hot, float * x_cold,
                         int Pmax, hipStream_t s);
hipError_t launch_scatter(const float * y_hot, const float * y_cold, int D_out, int kind, const int32_t * counts,
                          const int32_t * ids_hot, const int32_t * hot_dst, const int32_t * ids_cold,
                          const int32_t * cold_dst, const float * s_hot, const float * s_cold, float * y_full,
                          int Pmax, hipStream_t s);

}  // namespace llapis
