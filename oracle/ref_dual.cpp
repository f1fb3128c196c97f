/*
 * ref_dual.cpp -- the reference's CPU path for a dual-precision MoE layer,
 * as plain-C entry points over its own code: the ggml CPU graph
 * (third_party/llama/ggml) for the router, the top-k and the hot pairs, and
 * the reference's CPU cold executor (src/moe_sidecar.cpp, moe_sidecar_compute)
 * for the cold pairs.  Compiled into oracle/_ref/libggml_ref*.so by
 * oracle/Makefile from the sources where they lie.
 *
 * TEST INFRASTRUCTURE ONLY: bench.py's CPU baseline times it.  One call:
 *   1. the routing graph (llama-graph.cpp:1541-1650): router mul_mat (+ bias),
 *      soft_max, argsort_top_k, get_rows, sum_rows, clamp, div;
 *   2. on the host, each routed pair is hot when the residency predicate holds
 *      (ffn_moe.cu:80-130 with every slot READY: slot_of[e] >= 0);
 *   3. the cold pairs' gate_up through moe_sidecar_compute (at most 32 pairs a
 *      call, its PMAX), each pair reading its token's column;
 *   4. one graph for the hot pairs -- mul_mat_id(gate_up) on the hot pool,
 *      geglu_split, mul_mat_id(down) -- and geglu_split of the cold pairs'
 *      gate_up outputs;
 *   5. the cold pairs' down through moe_sidecar_compute;
 *   6. out_t = sum_k w_tk y_tk in k order.
 */
#include "ggml.h"
#include "ggml-cpu.h"
#include "moe_sidecar.hpp"

#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

namespace {

ggml_context * make_ctx(size_t bytes) {
    ggml_init_params ip = {bytes + (size_t)64 * 1024 * 1024, nullptr, false};
    return ggml_init(ip);
}

struct DualLayer {
    int64_t d, E, k, F, T, K;
    int n_threads;
    std::vector<int32_t> slot_of;                 // expert -> hot slot, or -1
    ggml_context * wctx = nullptr;                // weights and the routing graph
    ggml_tensor * x = nullptr, * sel = nullptr, * w = nullptr;
    ggml_cgraph * route = nullptr;
    ggml_tensor * hot_gu = nullptr, * hot_dn = nullptr;
    int cold_gu_type, cold_dn_type;
    const uint8_t * cold_gu;                      // host cold pools (caller-owned)
    const uint8_t * cold_dn;
    uint64_t cold_gu_bytes, cold_dn_bytes;
    std::vector<float> xs;                        // the call's tokens
};

void sidecar_fire(const DualLayer & L, int kind, const std::vector<int32_t> & ids, const float * x, bool per_pair,
                  const std::vector<int32_t> & col, float * y) {
    const int n = (int)ids.size();
    const int64_t d_in = kind == 0 ? L.d : L.F, d_out = kind == 0 ? 2 * L.F : L.d;
    for (int i0 = 0; i0 < n; i0 += 32) {
        const int m = std::min(32, n - i0);
        moert_coldcpu_call c = {};
        c.il = 0;
        c.kind = kind;
        c.n_cold = m;
        c.cold_ids = ids.data() + i0;
        c.x = per_pair ? x + (size_t)i0 * d_in : x;
        c.x_per_pair = per_pair ? 1 : 0;
        c.x_col = per_pair ? nullptr : col.data() + i0;
        c.w_host = kind == 0 ? L.cold_gu : L.cold_dn;
        c.expert_bytes = kind == 0 ? L.cold_gu_bytes : L.cold_dn_bytes;
        c.stride = 0;
        c.w_type_tag = kind == 0 ? L.cold_gu_type : L.cold_dn_type;
        c.d_in = (int32_t)d_in;
        c.d_out = (int32_t)d_out;
        c.y = y + (size_t)i0 * d_out;
        moe_sidecar_compute(&c);
    }
}

}  // namespace

extern "C" {

void * ref_dual_create(const float * w_r, const float * bias, int64_t d, int64_t n_expert, int64_t top_k,
                       int64_t n_ff, int64_t T, const int32_t * slot_of, int64_t k_slots, int hot_gu_type,
                       const void * hot_gu, int hot_dn_type, const void * hot_dn, int cold_gu_type,
                       const void * cold_gu, int cold_dn_type, const void * cold_dn, int n_threads) {
    ggml_cpu_init();
    moe_sidecar::init(n_threads);
    DualLayer * L = new DualLayer();
    L->d = d; L->E = n_expert; L->k = top_k; L->F = n_ff; L->T = T; L->K = k_slots;
    L->n_threads = n_threads;
    L->slot_of.assign(slot_of, slot_of + n_expert);
    const size_t gub = ggml_row_size((ggml_type)hot_gu_type, d) * 2 * n_ff * k_slots;
    const size_t dnb = ggml_row_size((ggml_type)hot_dn_type, n_ff) * d * k_slots;
    L->wctx = make_ctx(gub + dnb + (size_t)d * n_expert * 4 + (size_t)T * (d + 8 * n_expert) * 4);
    ggml_context * ctx = L->wctx;
    L->hot_gu = ggml_new_tensor_3d(ctx, (ggml_type)hot_gu_type, d, 2 * n_ff, k_slots);
    memcpy(L->hot_gu->data, hot_gu, gub);
    L->hot_dn = ggml_new_tensor_3d(ctx, (ggml_type)hot_dn_type, n_ff, d, k_slots);
    memcpy(L->hot_dn->data, hot_dn, dnb);
    L->cold_gu_type = cold_gu_type;
    L->cold_dn_type = cold_dn_type;
    L->cold_gu = (const uint8_t *)cold_gu;
    L->cold_dn = (const uint8_t *)cold_dn;
    L->cold_gu_bytes = ggml_row_size((ggml_type)cold_gu_type, d) * 2 * n_ff;
    L->cold_dn_bytes = ggml_row_size((ggml_type)cold_dn_type, n_ff) * d;

    ggml_tensor * wr = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, d, n_expert);
    memcpy(wr->data, w_r, sizeof(float) * d * n_expert);
    L->x = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, d, T);
    ggml_tensor * logits = ggml_mul_mat(ctx, wr, L->x);
    if (bias) {
        ggml_tensor * tb = ggml_new_tensor_1d(ctx, GGML_TYPE_F32, n_expert);
        memcpy(tb->data, bias, sizeof(float) * n_expert);
        logits = ggml_add(ctx, logits, tb);
    }
    ggml_tensor * probs = ggml_soft_max(ctx, logits);
    L->sel = ggml_argsort_top_k(ctx, probs, top_k);
    ggml_tensor * w = ggml_get_rows(ctx, ggml_reshape_3d(ctx, probs, 1, n_expert, T), L->sel);
    w = ggml_reshape_2d(ctx, w, top_k, T);
    ggml_tensor * wsum = ggml_sum_rows(ctx, w);
    wsum = ggml_clamp(ctx, wsum, 6.103515625e-5f, INFINITY);
    L->w = ggml_div(ctx, w, wsum);
    L->route = ggml_new_graph(ctx);
    ggml_build_forward_expand(L->route, L->w);
    return L;
}

void ref_dual_run(void * h, const float * x, float * out, int32_t * ids_out, int32_t * n_hot_out) {
    DualLayer * L = static_cast<DualLayer *>(h);
    const int64_t d = L->d, F = L->F, T = L->T, k = L->k;
    memcpy(L->x->data, x, sizeof(float) * d * T);
    ggml_graph_compute_with_ctx(L->wctx, L->route, L->n_threads);
    // the routing, split by tier
    std::vector<int32_t> hot_pairs, hot_slots, cold_pairs, cold_ids, cold_col;
    for (int64_t t = 0; t < T; ++t) {
        const int32_t * sel = (const int32_t *)((const char *)L->sel->data + t * L->sel->nb[1]);
        for (int64_t j = 0; j < k; ++j) {
            const int32_t e = sel[j];
            const int32_t p = (int32_t)(t * k + j);
            if (ids_out) ids_out[p] = e;
            const int32_t s = (e >= 0 && e < L->E) ? L->slot_of[e] : -1;
            if (s >= 0) {
                hot_pairs.push_back(p);
                hot_slots.push_back(s);
            } else {
                cold_pairs.push_back(p);
                cold_ids.push_back(e);
                cold_col.push_back((int32_t)t);
            }
        }
    }
    if (n_hot_out) *n_hot_out = (int32_t)hot_pairs.size();
    const int64_t Ph = (int64_t)hot_pairs.size(), Pc = (int64_t)cold_pairs.size();
    // 3. the cold pairs' gate_up on the sidecar: each pair reads its token's
    // column (quantised once per token) while the call's tokens fit its
    // 32 columns, else the pairs' columns gathered one per pair
    std::vector<float> gu_c((size_t)Pc * 2 * F);
    if (Pc && T <= 32) sidecar_fire(*L, 0, cold_ids, x, false, cold_col, gu_c.data());
    if (Pc && T > 32) {
        std::vector<float> xg((size_t)Pc * d);
        for (int64_t i = 0; i < Pc; ++i) memcpy(xg.data() + i * d, x + (int64_t)cold_col[i] * d, sizeof(float) * d);
        sidecar_fire(*L, 0, cold_ids, xg.data(), true, cold_col, gu_c.data());
    }
    // 4. the hot pairs and the cold GEGLU in one graph
    const size_t need = (size_t)(Ph * (d + 2 * F + F + d) + Pc * (2 * F + F) + Ph) * 4;
    ggml_context * ctx = make_ctx(need);
    ggml_cgraph * g = ggml_new_graph(ctx);
    ggml_tensor * yh = nullptr, * ac = nullptr;
    if (Ph) {
        ggml_tensor * cur = ggml_new_tensor_3d(ctx, GGML_TYPE_F32, d, 1, Ph);
        ggml_tensor * ids = ggml_new_tensor_2d(ctx, GGML_TYPE_I32, 1, Ph);
        for (int64_t i = 0; i < Ph; ++i) {
            memcpy((float *)cur->data + i * d, x + (hot_pairs[i] / k) * d, sizeof(float) * d);
            ((int32_t *)ids->data)[i] = hot_slots[i];
        }
        ggml_tensor * gu = ggml_mul_mat_id(ctx, L->hot_gu, cur, ids);               /* [2F, 1, Ph] */
        ggml_tensor * gate = ggml_view_3d(ctx, gu, F, gu->ne[1], gu->ne[2], gu->nb[1], gu->nb[2], 0);
        ggml_tensor * up = ggml_view_3d(ctx, gu, F, gu->ne[1], gu->ne[2], gu->nb[1], gu->nb[2], F * gu->nb[0]);
        ggml_tensor * a = ggml_geglu_split(ctx, gate, up);
        yh = ggml_mul_mat_id(ctx, L->hot_dn, a, ids);                              /* [d, 1, Ph] */
        ggml_build_forward_expand(g, yh);
    }
    if (Pc) {
        ggml_tensor * guc = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, 2 * F, Pc);
        memcpy(guc->data, gu_c.data(), sizeof(float) * 2 * F * Pc);
        ggml_tensor * gate = ggml_view_2d(ctx, guc, F, Pc, guc->nb[1], 0);
        ggml_tensor * up = ggml_view_2d(ctx, guc, F, Pc, guc->nb[1], F * guc->nb[0]);
        ac = ggml_cont(ctx, ggml_geglu_split(ctx, gate, up));                      /* [F, Pc] */
        ggml_build_forward_expand(g, ac);
    }
    if (Ph || Pc) ggml_graph_compute_with_ctx(ctx, g, L->n_threads);
    // 5. the cold pairs' down on the sidecar
    std::vector<float> yc((size_t)Pc * d);
    if (Pc) sidecar_fire(*L, 1, cold_ids, (const float *)ac->data, true, cold_col, yc.data());
    // 6. the combine in k order
    std::vector<const float *> yp((size_t)T * k, nullptr);
    for (int64_t i = 0; i < Ph; ++i) yp[hot_pairs[i]] = (const float *)((const char *)yh->data + i * yh->nb[2]);
    for (int64_t i = 0; i < Pc; ++i) yp[cold_pairs[i]] = yc.data() + i * d;
    const float * wv = (const float *)L->w->data;
    for (int64_t t = 0; t < T; ++t) {
        float * o = out + t * d;
        for (int64_t r = 0; r < d; ++r) o[r] = yp[t * k][r] * wv[t * k];
        for (int64_t j = 1; j < k; ++j)
            for (int64_t r = 0; r < d; ++r) o[r] += yp[t * k + j][r] * wv[t * k + j];
    }
    ggml_free(ctx);
}

void ref_dual_free(void * h) {
    DualLayer * L = static_cast<DualLayer *>(h);
    if (!L) return;
    ggml_free(L->wctx);
    delete L;
}

}  // extern "C"
