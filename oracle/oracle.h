/*
 * oracle.h -- CPU restatement of the dual-precision MoE expert FFN path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (llapis_amd/) links,
 * loads or calls this code; only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py use it, and there only as the checker.
 *
 * Every function restates the arithmetic of the reference's CPU path
 * (ggml CPU, vendored by the reference under third_party/llama/ggml) or,
 * for the q8_1 activation mode, of the reference's GPU path (ggml-cuda).
 * The citation on each declaration names the file:line it follows; paths are
 * relative to the reference root.  How each one is pinned (golden vectors
 * from the compiled reference, closed forms, brute force) is listed in the
 * header of tests/test_oracle.py.
 */
#ifndef LLAPIS_ORACLE_H
#define LLAPIS_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type tags (third_party/llama/ggml/include/ggml.h:390-412) */
enum {
    ORC_F32 = 0, ORC_Q5_0 = 6, ORC_Q8_0 = 8, ORC_Q8_1 = 9, ORC_Q4_K = 12,
    ORC_Q8_K = 15, ORC_IQ4_NL = 20, ORC_IQ2_S = 22,
};

/* activation formats: 0 = what the x86 ggml CPU path quantises to (q8_K for
 * 256-wide blocks, q8_0 for 32-wide blocks); 1 = q8_1 as ggml-cuda does. */
/* ORC_ACT_Q8_1_MMA: q8_1 activations with the sums ggml-cuda's matrix-core
 * path (mmq.cuh) forms for IQ2_S and Q5_0 -- the per-16 scale d (2 ls + 1) / 8
 * applied exactly (no integer truncation) and Q5_0 as d d8 sum (q - 16) a
 * (no s8 term); Q4_K and IQ4_NL as in ORC_ACT_Q8_1.  The device's prefill
 * path in its q8_1 mode computes these. */
enum { ORC_ACT_CPU = 0, ORC_ACT_Q8_1 = 1, ORC_ACT_Q8_1_MMA = 2 };
/* GEGLU: 0 = the CPU's fp16 GELU table (ggml-cpu/vec.h:1414-1428),
 *        1 = exact tanh GELU (ggml-cuda/unary.cuh:101-104). */
enum { ORC_GELU_TABLE = 0, ORC_GELU_TANH = 1 };

float    orc_fp16_to_fp32(uint16_t h);
uint16_t orc_fp32_to_fp16(float f);

/* bytes of one row of `n` weights of `type` */
size_t orc_row_size(int type, int64_t n);

/* dequantisation (ggml-quants.c:442 q5_0, :1471-1493 q4_K, :2471-2498 iq2_s,
 * :2653-2668 iq4_nl) */
void orc_dequantize(int type, const void * x, float * y, int64_t k);

/* activation quantisers.
 *   q8_K: ggml-quants.c:2696-2733 (used verbatim by the x86 build,
 *         ggml-cpu/arch/x86/quants.c:505-507)
 *   q8_0: ggml-cpu/arch/x86/quants.c:302-360 (AVX: d = max/127, id = 127/max,
 *         round-to-nearest-even)
 *   q8_1: ggml-cuda/quantize.cu:5-50 (d = amax/127, q = roundf(x/d),
 *         s = sum of x) */
void orc_quantize_act(int act_type, const float * x, void * y, int64_t k);

/* vec_dot of one quantised weight row with a quantised activation.
 *   q4_K.q8_K  ggml-cpu/quants.c:645-718     iq2_s.q8_K  quants.c:947-997
 *   q5_0.q8_0  quants.c:314-352              iq4_nl.q8_0 quants.c:1203-1228
 *   *.q8_1     ggml-cuda/vecdotq.cuh:172-198 (q5_0), :505-528 + :864-907
 *              (q4_K), :1061-1105 (iq2_s), :1270-1289 (iq4_nl)          */
float orc_vec_dot(int wtype, int act_mode, int64_t n, const void * w, const void * a);

/* the activation type the weight type is dotted with in a given mode */
int orc_act_type(int wtype, int act_mode);

/* y[r] = W[r,:] . x for nrows rows of W (quantised) with x quantised once in
 * the mode's activation format (ggml-cpu/ggml-cpu.c:1447-1517: src1 is
 * converted to vec_dot_type once per column, then vec_dot per row). */
void orc_matvec(int wtype, int act_mode, const void * w, int64_t nrows, int64_t ncols,
                const float * x, float * y);

/* GELU/GEGLU: out[i] = gelu(g[i]) * u[i] */
void orc_geglu(const float * g, const float * u, float * out, int64_t n, int gelu_mode);

/* Router: logits = W_r x (+ bias), softmax, top-k by descending probability,
 * weights = p[ids] / max(sum, 6.103515625e-5)
 * (llama-graph.cpp:1548-1650: soft_max, argsort_top_k, get_rows, sum_rows,
 * clamp, div).  W_r is [n_expert][d] row-major (ggml ne0 = d).
 * ids: [T][top_k], w: [T][top_k], probs (optional): [T][n_expert]. */
void orc_router(const float * x, int64_t T, const float * w_r, const float * bias,
                int64_t d, int64_t n_expert, int64_t top_k,
                int32_t * ids, float * w, float * probs);

/* One dual-precision MoE layer.  Pools are expert-major contiguous slabs:
 *   hot gate_up  [k_slots][2*n_ff rows of d_model]   (type hot_gu_type)
 *   hot down     [k_slots][d_model rows of n_ff]     (type hot_dn_type)
 *   cold gate_up [n_expert][2*n_ff rows of d_model]  (type cold_gu_type)
 *   cold down    [n_expert][d_model rows of n_ff]    (type cold_dn_type)
 * A routed pair (t, e) is hot iff exp_slot[e] = s with 0 <= s < k_slots,
 * slot_state[s] == 2 (READY) and slot_exp[s] == e
 * (moert/cuda/ffn_moe.cu:80-130, moert/include/moert/policy.h:46).
 * s_hot[k_slots] / s_cold[n_expert] are optional down scales
 * (ffn_moe.cu:158-176).  Gate rows are [0, n_ff), up rows [n_ff, 2 n_ff)
 * (llama-graph.cpp:1687-1693).  Combine: out_t = ((w0 y0 + w1 y1) + w2 y2)...
 * (llama-graph.cpp:1812-1840). */
typedef struct orc_layer {
    int64_t d_model, n_ff, n_expert, top_k, k_slots;
    int32_t hot_gu_type, hot_dn_type, cold_gu_type, cold_dn_type;
    const void * hot_gu;  const void * hot_dn;
    const void * cold_gu; const void * cold_dn;
    const int32_t * exp_slot; const int32_t * slot_exp; const int32_t * slot_state;
    const float * s_hot; const float * s_cold;
} orc_layer;

/* Expert part of the layer for given routing (ids/w from the router).
 * y_pairs (optional): [T*top_k][d_model] per-pair down outputs after scale,
 * before the router weight. */
void orc_moe_experts(const orc_layer * L, const float * x, int64_t T,
                     const int32_t * ids, const float * w, int act_mode, int gelu_mode,
                     float * out, float * y_pairs);

/* A control for chained-layer tests, not part of the restatement: with a
 * nonzero seed, orc_moe_experts moves every gate_up and down matvec output
 * one ulp up or down (a seeded coin per token, pair and row) before it is
 * used -- the last-bit differences another fp32 summation order makes.
 * 0 (the default) turns it off. */
void orc_set_sum_jitter(uint64_t seed);

#ifdef __cplusplus
}
#endif
#endif
