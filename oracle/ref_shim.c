/*
 * ref_shim.c -- plain-C entry points over the reference's own ggml CPU build
 * (oracle/_ref/libggml_ref.so, compiled by oracle/Makefile from the sources
 * under the reference's third_party/llama/ggml).
 *
 * TEST INFRASTRUCTURE ONLY: this is the checker the CPU restatement
 * (oracle.c) and the GPU path are compared against, and the CPU baseline
 * bench.py times.  It calls ggml's public API and CPU type traits only.
 */
#include "ggml.h"
#include "ggml-cpu.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ggml_quantize_chunk (ggml.c:7761) over nrow rows */
size_t ref_quantize(int type, const float * src, void * dst, int64_t nrow, int64_t n_per_row,
                    const float * imatrix) {
    ggml_cpu_init();
    return ggml_quantize_chunk((enum ggml_type)type, src, dst, 0, nrow, n_per_row, imatrix);
}

/* the format's to_float (ggml-quants.c dequantize_row_*) */
void ref_dequantize(int type, const void * src, float * dst, int64_t n) {
    ggml_get_type_traits((enum ggml_type)type)->to_float(src, dst, n);
}

size_t ref_row_size(int type, int64_t n) { return ggml_row_size((enum ggml_type)type, n); }

/* the CPU build's activation type for a weight type, and its quantiser */
int ref_vec_dot_type(int type) {
    ggml_cpu_init();
    return (int)ggml_get_type_traits_cpu((enum ggml_type)type)->vec_dot_type;
}

void ref_quantize_act(int act_type, const float * x, void * y, int64_t n) {
    ggml_cpu_init();
    ggml_get_type_traits_cpu((enum ggml_type)act_type)->from_float(x, y, n);
}

float ref_vec_dot(int type, int64_t n, const void * w, const void * a) {
    ggml_cpu_init();
    float s = 0;
    ggml_get_type_traits_cpu((enum ggml_type)type)->vec_dot((int)n, &s, 0, w, 0, a, 0, 1);
    return s;
}

static struct ggml_context * mk_ctx(size_t extra) {
    /* weights + activations + graph metadata + ggml's work buffer (also
     * allocated in the context by ggml_graph_compute_with_ctx) */
    struct ggml_init_params p = { .mem_size = extra + extra / 8 + 512u * 1024 * 1024, .mem_buffer = NULL,
                                  .no_alloc = false };
    return ggml_init(p);
}

/* y[D_out, P] = mul_mat_id(W[D_in, D_out, n_pool], x[D_in, n_cols], ids[P])
 * exactly as a model graph computes it (ggml-cpu.c:1447-1700).  n_cols is 1
 * (one activation column shared by every pair) or P (one column per pair). */
void ref_mul_mat_id(int wtype, const void * w, int64_t d_in, int64_t d_out, int64_t n_pool,
                    const float * x, int64_t n_cols, const int32_t * ids, int64_t P,
                    float * y, int n_threads) {
    ggml_cpu_init();
    const size_t wbytes = ggml_row_size((enum ggml_type)wtype, d_in) * d_out * n_pool;
    struct ggml_context * ctx = mk_ctx(wbytes + (size_t)(d_in * P + d_out * P) * 4 * 2);
    struct ggml_tensor * tw = ggml_new_tensor_3d(ctx, (enum ggml_type)wtype, d_in, d_out, n_pool);
    memcpy(tw->data, w, wbytes);
    struct ggml_tensor * tx = ggml_new_tensor_3d(ctx, GGML_TYPE_F32, d_in, n_cols, 1);
    memcpy(tx->data, x, sizeof(float) * d_in * n_cols);
    struct ggml_tensor * ti = ggml_new_tensor_2d(ctx, GGML_TYPE_I32, P, 1);
    memcpy(ti->data, ids, sizeof(int32_t) * P);
    struct ggml_tensor * ty = ggml_mul_mat_id(ctx, tw, tx, ti);
    struct ggml_cgraph * g = ggml_new_graph(ctx);
    ggml_build_forward_expand(g, ty);
    ggml_graph_compute_with_ctx(ctx, g, n_threads);
    memcpy(y, ty->data, sizeof(float) * d_out * P);
    ggml_free(ctx);
}

/* out = geglu_split(gate, up) over n_cols columns of n (ops.cpp:3024-3080) */
void ref_geglu(const float * gate, const float * up, float * out, int64_t n, int64_t n_cols) {
    ggml_cpu_init();
    struct ggml_context * ctx = mk_ctx((size_t)n * n_cols * 4 * 3);
    struct ggml_tensor * tg = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, n, n_cols);
    struct ggml_tensor * tu = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, n, n_cols);
    memcpy(tg->data, gate, sizeof(float) * n * n_cols);
    memcpy(tu->data, up, sizeof(float) * n * n_cols);
    struct ggml_tensor * to = ggml_geglu_split(ctx, tg, tu);
    struct ggml_cgraph * g = ggml_new_graph(ctx);
    ggml_build_forward_expand(g, to);
    ggml_graph_compute_with_ctx(ctx, g, 1);
    memcpy(out, to->data, sizeof(float) * n * n_cols);
    ggml_free(ctx);
}

/*
 * A prepared single-tier MoE layer graph, as build_moe_ffn builds it for a
 * merged gate_up model with softmax gating and normalised weights
 * (llama-graph.cpp:1507-1850): router mul_mat (+ bias), soft_max,
 * argsort_top_k, get_rows, sum_rows, clamp, div, mul_mat_id(gate_up), views,
 * geglu_split, mul_mat_id(down), mul by weights, sum of the top_k views.
 * Built once (weights copied in), then run many times (ref_layer_run) so the
 * CPU baseline times compute only.
 */
typedef struct ref_layer {
    struct ggml_context * ctx;
    struct ggml_cgraph * g;
    struct ggml_tensor * x, * out, * ids, * w;
    int64_t d, T, k;
} ref_layer;

void * ref_layer_create(const float * w_r, const float * bias, int64_t d, int64_t n_expert, int64_t top_k,
                        int gu_type, const void * w_gu, int dn_type, const void * w_dn, int64_t n_ff,
                        int64_t T) {
    ggml_cpu_init();
    const size_t gub = ggml_row_size((enum ggml_type)gu_type, d) * 2 * n_ff * n_expert;
    const size_t dnb = ggml_row_size((enum ggml_type)dn_type, n_ff) * d * n_expert;
    const size_t act = (size_t)T * (d * (4 + 2 * top_k) + 2 * n_ff * top_k * 3 + n_expert * 8) * 4;
    ref_layer * L = calloc(1, sizeof(ref_layer));
    L->ctx = mk_ctx(gub + dnb + (size_t)d * n_expert * 4 + act);
    L->d = d; L->T = T; L->k = top_k;
    struct ggml_context * ctx = L->ctx;
    struct ggml_tensor * wr = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, d, n_expert);
    memcpy(wr->data, w_r, sizeof(float) * d * n_expert);
    struct ggml_tensor * wgu = ggml_new_tensor_3d(ctx, (enum ggml_type)gu_type, d, 2 * n_ff, n_expert);
    memcpy(wgu->data, w_gu, gub);
    struct ggml_tensor * wdn = ggml_new_tensor_3d(ctx, (enum ggml_type)dn_type, n_ff, d, n_expert);
    memcpy(wdn->data, w_dn, dnb);
    L->x = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, d, T);

    struct ggml_tensor * logits = ggml_mul_mat(ctx, wr, L->x);                 /* [E, T] */
    if (bias) {
        struct ggml_tensor * tb = ggml_new_tensor_1d(ctx, GGML_TYPE_F32, n_expert);
        memcpy(tb->data, bias, sizeof(float) * n_expert);
        logits = ggml_add(ctx, logits, tb);
    }
    struct ggml_tensor * probs = ggml_soft_max(ctx, logits);
    struct ggml_tensor * sel = ggml_argsort_top_k(ctx, probs, top_k);           /* [k, T] */
    struct ggml_tensor * w = ggml_get_rows(ctx, ggml_reshape_3d(ctx, probs, 1, n_expert, T), sel);
    w = ggml_reshape_2d(ctx, w, top_k, T);
    struct ggml_tensor * wsum = ggml_sum_rows(ctx, w);
    wsum = ggml_clamp(ctx, wsum, 6.103515625e-5f, INFINITY);
    w = ggml_div(ctx, w, wsum);
    w = ggml_reshape_3d(ctx, w, 1, top_k, T);
    struct ggml_tensor * cur = ggml_reshape_3d(ctx, L->x, d, 1, T);
    struct ggml_tensor * gu = ggml_mul_mat_id(ctx, wgu, cur, sel);              /* [2F, k, T] */
    struct ggml_tensor * gate = ggml_view_3d(ctx, gu, n_ff, gu->ne[1], gu->ne[2], gu->nb[1], gu->nb[2], 0);
    struct ggml_tensor * up = ggml_view_3d(ctx, gu, n_ff, gu->ne[1], gu->ne[2], gu->nb[1], gu->nb[2],
                                           n_ff * gu->nb[0]);
    struct ggml_tensor * a = ggml_geglu_split(ctx, gate, up);                   /* [F, k, T] */
    struct ggml_tensor * ex = ggml_mul_mat_id(ctx, wdn, a, sel);                /* [D, k, T] */
    ex = ggml_mul(ctx, ex, w);
    struct ggml_tensor * out = ggml_view_2d(ctx, ex, d, T, ex->nb[2], 0);
    for (int64_t i = 1; i < top_k; ++i)
        out = ggml_add(ctx, out, ggml_view_2d(ctx, ex, d, T, ex->nb[2], i * ex->nb[1]));
    L->out = out;
    L->ids = sel;
    L->w = w;
    L->g = ggml_new_graph(ctx);
    ggml_build_forward_expand(L->g, out);
    return L;
}

void ref_layer_run(void * h, const float * x, float * out, int32_t * ids, float * w, int n_threads) {
    ref_layer * L = h;
    memcpy(L->x->data, x, sizeof(float) * L->d * L->T);
    ggml_graph_compute_with_ctx(L->ctx, L->g, n_threads);
    if (out) {
        for (int64_t t = 0; t < L->T; ++t)
            memcpy(out + t * L->d, (const char *)L->out->data + t * L->out->nb[1], sizeof(float) * L->d);
    }
    if (ids) {
        for (int64_t t = 0; t < L->T; ++t)
            memcpy(ids + t * L->k, (const char *)L->ids->data + t * L->ids->nb[1], sizeof(int32_t) * L->k);
    }
    if (w) memcpy(w, L->w->data, sizeof(float) * L->k * L->T);
}

void ref_layer_free(void * h) {
    ref_layer * L = h;
    if (!L) return;
    ggml_free(L->ctx);
    free(L);
}

/* ---- GGUF through ggml's own gguf.cpp (the checker of the GGUF reader) ---- */
#include "gguf.h"

/* Writes n tensors (name, type, rank, ne, data) and two keys with ggml's
 * writer; alignment 0 keeps the default.  Returns 1 on success. */
int ref_gguf_write(const char * path, int n, const char * const * names, const int * types, const int * n_dims,
                   const int64_t * ne, const void * const * data, uint32_t alignment) {
    struct ggml_init_params ip = {(size_t)(n + 1) * ggml_tensor_overhead(), NULL, true};
    struct ggml_context * ctx = ggml_init(ip);
    struct gguf_context * g = gguf_init_empty();
    gguf_set_val_str(g, "general.architecture", "gemma4");
    if (alignment) gguf_set_val_u32(g, "general.alignment", alignment);
    for (int i = 0; i < n; ++i) {
        struct ggml_tensor * t = ggml_new_tensor(ctx, (enum ggml_type)types[i], n_dims[i], ne + 4 * i);
        ggml_set_name(t, names[i]);
        gguf_add_tensor(g, t);
        gguf_set_tensor_data(g, names[i], data[i]);
    }
    const int ok = gguf_write_to_file(g, path, false) ? 1 : 0;
    gguf_free(g);
    ggml_free(ctx);
    return ok;
}

/* Reads the tensor table with ggml's reader: per tensor its name (64 bytes
 * each), type, offset relative to the data section and size.  Returns the
 * tensor count (at most max are written), -1 on failure. */
int64_t ref_gguf_read(const char * path, uint64_t * data_offset, uint64_t * alignment, int64_t max, char * names,
                      int * types, uint64_t * offsets, uint64_t * sizes) {
    struct gguf_init_params p = {true, NULL};
    struct gguf_context * g = gguf_init_from_file(path, p);
    if (!g) return -1;
    *data_offset = gguf_get_data_offset(g);
    *alignment = gguf_get_alignment(g);
    const int64_t n = gguf_get_n_tensors(g);
    for (int64_t i = 0; i < n && i < max; ++i) {
        strncpy(names + 64 * i, gguf_get_tensor_name(g, i), 63);
        names[64 * i + 63] = 0;
        types[i] = (int)gguf_get_tensor_type(g, i);
        offsets[i] = gguf_get_tensor_offset(g, i);
        sizes[i] = gguf_get_tensor_size(g, i);
    }
    gguf_free(g);
    return n;
}
