// small_kernels.hip -- the path's small kernels on gfx950: router logits,
// softmax/top-k selection, the island's residency partition / gather /
// scatter, the weighted combine, and a standalone GEGLU.
#include "device.h"
#include "launch.h"

namespace llapis {
namespace dev {

// ------------------------------------------------------------- router

constexpr int ROUTER_TOK = 4;    // tokens per workgroup of k_router_logits

// logits[t][e] = W_r[e] . x[t] (+ bias[e]) (build_lora_mm(gate_inp, cur),
// llama-graph.cpp:1541; ggml mul_mat f32): one workgroup per (expert, 4
// tokens), every load of the row and the tokens issued before the first
// product (one memory round trip for d <= 4096); per-thread partial sums
// over its float4s in order, a wave sum, the four waves' sums in order --
// the decode path's router arithmetic, so both give the same logits.
__global__ __launch_bounds__(WG) void k_router_logits(const float * __restrict__ x, int T,
                                                      const float * __restrict__ w_r, const float * __restrict__ bias,
                                                      int d, int E, float * __restrict__ logits) {
    constexpr int RU = 4;
    __shared__ float s_part[ROUTER_TOK][WG / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int e = blockIdx.x, t0 = blockIdx.y * ROUTER_TOK, nt = min(ROUTER_TOK, T - t0), n4 = d / 4;
    const float4 * wrow = reinterpret_cast<const float4 *>(w_r + (int64_t)e * d);
    const float4 * x4 = reinterpret_cast<const float4 *>(x);
    const float b = bias ? bias[e] : 0.0f;
    float acc[ROUTER_TOK];
#pragma unroll
    for (int j = 0; j < ROUTER_TOK; ++j) acc[j] = 0.0f;
    for (int k0 = threadIdx.x; k0 < n4; k0 += RU * WG) {
        float4 w4[RU], xv[ROUTER_TOK][RU];
#pragma unroll
        for (int u = 0; u < RU; ++u) w4[u] = wrow[min(k0 + u * WG, n4 - 1)];
#pragma unroll
        for (int j = 0; j < ROUTER_TOK; ++j)
#pragma unroll
            for (int u = 0; u < RU; ++u) xv[j][u] = x4[(int64_t)(t0 + min(j, nt - 1)) * n4 + min(k0 + u * WG, n4 - 1)];
#pragma unroll
        for (int j = 0; j < ROUTER_TOK; ++j)
#pragma unroll
            for (int u = 0; u < RU; ++u)
                if (j < nt && k0 + u * WG < n4)
                    acc[j] += w4[u].x * xv[j][u].x + w4[u].y * xv[j][u].y + w4[u].z * xv[j][u].z +
                              w4[u].w * xv[j][u].w;
    }
#pragma unroll
    for (int j = 0; j < ROUTER_TOK; ++j) {
        const float sj = wave_sum_dpp(acc[j]);
        if (lane == 0) s_part[j][wave] = sj;
    }
    __syncthreads();
    if ((int)threadIdx.x < nt) {
        const int j = threadIdx.x;
        float sj = 0.0f;
#pragma unroll
        for (int q = 0; q < WG / 64; ++q) sj += s_part[j][q];
        logits[(int64_t)(t0 + j) * E + e] = sj + b;
    }
}

// The same logits for long token batches on the matrix cores: one 256-thread
// workgroup per (64 tokens, 64 experts, K split), each wave a 32 x 32 tile on
// v_mfma_f32_32x32x2_f32 in fp32.  16-k slices of x and W_r are loaded with
// one coalesced 16-byte load per thread each (4 threads per 64-byte row
// piece), staged in LDS (double-buffered, rows padded to 20 floats so the 16
// rows a half-wave reads fall in different banks), and lane l feeds
// x[row l%32][k + 8(l/32) + i] and W_r[expert l%32][same k] to the i-th of
// eight MFMAs per slice.  The RSPLIT partial dot products per logit go to
// parts[split][t][e]; k_topk adds them in split order (and the bias).
constexpr int RSPLIT = 16;
constexpr int RT = 64, RK = 16, RPAD = 20;

__global__ __launch_bounds__(WG) void k_router_mfma(const float * __restrict__ x, int T,
                                                    const float * __restrict__ w_r, int d, int E, int kc,
                                                    float * __restrict__ parts) {
    typedef float f16v __attribute__((ext_vector_type(16)));
    __shared__ __align__(16) float s_x[2][RT * RPAD], s_w[2][RT * RPAD];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 31, h = lane >> 5;
    const int t0 = blockIdx.x * RT, e0 = blockIdx.y * RT, sp = blockIdx.z;
    const int k0 = sp * kc, k1 = min(d, k0 + kc);
    // loader: thread -> (row tid / 4, 4 floats at 4 (tid % 4))
    const int lr = tid >> 2, lc = 4 * (tid & 3);
    const float * xs = x + (int64_t)min(t0 + lr, T - 1) * d + lc;
    const float * ws = w_r + (int64_t)min(e0 + lr, E - 1) * d + lc;
    // compute: wave -> tokens 32 (wave >> 1), experts 32 (wave & 1)
    const int xo = (32 * (wave >> 1) + r) * RPAD + 8 * h, wo = (32 * (wave & 1) + r) * RPAD + 8 * h;
    f16v acc = {};
    float4 gx = *reinterpret_cast<const float4 *>(xs + k0);
    float4 gw = *reinterpret_cast<const float4 *>(ws + k0);
    int buf = 0;
    for (int k = k0; k < k1; k += RK) {
        *reinterpret_cast<float4 *>(&s_x[buf][lr * RPAD + lc]) = gx;
        *reinterpret_cast<float4 *>(&s_w[buf][lr * RPAD + lc]) = gw;
        __syncthreads();
        if (k + RK < k1) {
            gx = *reinterpret_cast<const float4 *>(xs + k + RK);
            gw = *reinterpret_cast<const float4 *>(ws + k + RK);
        }
        const float4 xa = *reinterpret_cast<const float4 *>(&s_x[buf][xo]);
        const float4 xb = *reinterpret_cast<const float4 *>(&s_x[buf][xo + 4]);
        const float4 wa = *reinterpret_cast<const float4 *>(&s_w[buf][wo]);
        const float4 wb = *reinterpret_cast<const float4 *>(&s_w[buf][wo + 4]);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xa.x, wa.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xa.y, wa.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xa.z, wa.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xa.w, wa.w, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xb.x, wb.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xb.y, wb.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xb.z, wb.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xb.w, wb.w, acc, 0, 0, 0);
        buf ^= 1;
    }
    const int e = e0 + 32 * (wave & 1) + r;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int t = t0 + 32 * (wave >> 1) + 8 * i + 4 * h + j;
            if (t < T && e < E) parts[((int64_t)sp * T + t) * E + e] = acc[4 * i + j];
        }
}

// The same tiles and the same MFMA sequence (so the same partial sums, bit
// for bit) with the whole K split staged at once: every thread issues all of
// its loads of x and W_r (kc / 16 of each) before the first wait, the
// workgroup stores them to LDS and meets at one barrier, instead of one
// load round trip per 16-k slice.  kc <= RKC_MAX (d <= 3072 at RSPLIT 16).
// The row pitch is 4 mod 32 floats, so the 8 rows of a 16-byte read's lane
// group fall in different banks.
constexpr int RKC_MAX = 192, RPITCH = RKC_MAX + 4;

__global__ __launch_bounds__(WG) void k_router_mfma_st(const float * __restrict__ x, int T,
                                                       const float * __restrict__ w_r, int d, int E, int kc,
                                                       float * __restrict__ parts) {
    typedef float f16v __attribute__((ext_vector_type(16)));
    constexpr int NJ = RKC_MAX / RK;
    __shared__ __align__(16) float s_x[RT * RPITCH], s_w[RT * RPITCH];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 31, h = lane >> 5;
    const int t0 = blockIdx.x * RT, e0 = blockIdx.y * RT, sp = blockIdx.z;
    const int nk = kc / RK;
    const int lr = tid >> 2, lc = 4 * (tid & 3);
    const float * xs = x + (int64_t)min(t0 + lr, T - 1) * d + sp * kc + lc;
    const float * ws = w_r + (int64_t)min(e0 + lr, E - 1) * d + sp * kc + lc;
    // slices past the split (j >= nk) reload its last one into LDS room that
    // no MFMA reads: no branch, so the values stay in registers
    float4 gx[NJ], gw[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) gx[j] = *reinterpret_cast<const float4 *>(xs + RK * min(j, nk - 1));
#pragma unroll
    for (int j = 0; j < NJ; ++j) gw[j] = *reinterpret_cast<const float4 *>(ws + RK * min(j, nk - 1));
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        *reinterpret_cast<float4 *>(&s_x[lr * RPITCH + RK * j + lc]) = gx[j];
        *reinterpret_cast<float4 *>(&s_w[lr * RPITCH + RK * j + lc]) = gw[j];
    }
    __syncthreads();
    const int xo = (32 * (wave >> 1) + r) * RPITCH + 8 * h, wo = (32 * (wave & 1) + r) * RPITCH + 8 * h;
    f16v acc = {};
    for (int j = 0; j < nk; ++j) {
        const float4 xa = *reinterpret_cast<const float4 *>(&s_x[xo + RK * j]);
        const float4 xb = *reinterpret_cast<const float4 *>(&s_x[xo + RK * j + 4]);
        const float4 wa = *reinterpret_cast<const float4 *>(&s_w[wo + RK * j]);
        const float4 wb = *reinterpret_cast<const float4 *>(&s_w[wo + RK * j + 4]);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xa.x, wa.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xa.y, wa.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xa.z, wa.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xa.w, wa.w, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xb.x, wb.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xb.y, wb.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xb.z, wb.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xb.w, wb.w, acc, 0, 0, 0);
    }
    const int e = e0 + 32 * (wave & 1) + r;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int t = t0 + 32 * (wave >> 1) + 8 * i + 4 * h + j;
            if (t < T && e < E) parts[((int64_t)sp * T + t) * E + e] = acc[4 * i + j];
        }
}

// In place: logits -> probabilities (ggml soft_max: exp(x - max), sum in
// double, scaled by float(1/sum); ops.cpp:5344-5450), then top-K by
// descending p with ties to the lower index (argsort_top_k), weights
// p[ids] / max(sum, 6.103515625e-5) with the sum in double (sum_rows, clamp,
// div: llama-graph.cpp:1636-1650).  One wave per token, E <= 256, K <= 16.
// With `parts` the logits are first summed from the router's K splits.
__global__ __launch_bounds__(64) void k_topk(float * __restrict__ probs, int E, int K,
                                             int32_t * __restrict__ ids, float * __restrict__ w,
                                             const float * __restrict__ parts, int T, const float * __restrict__ bias) {
    const int lane = threadIdx.x, t = blockIdx.x;
    float * row = probs + (int64_t)t * E;
    float v[4];
    if (parts) {
        // every partial of the token's experts in flight before the first
        // sum (the 64-expert quarters are wave-uniform), then the sums in
        // split order
        float pv[4][RSPLIT];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (64 * j < E) {
                const int e = min(lane + 64 * j, E - 1);
#pragma unroll
                for (int q = 0; q < RSPLIT; ++q) pv[j][q] = parts[((int64_t)q * T + t) * E + e];
            }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = lane + 64 * j;
            if (e >= E) {
                v[j] = -INFINITY;
            } else {
                float a = pv[j][0];
#pragma unroll
                for (int q = 1; q < RSPLIT; ++q) a += pv[j][q];
                v[j] = bias ? a + bias[e] : a;
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = lane + 64 * j;
            v[j] = e < E ? row[e] : -INFINITY;
        }
    }
    const float mx = wave_max_dpp(fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])));
    double ls = 0.0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = lane + 64 * j;
        v[j] = e < E ? expf(v[j] - mx) : 0.0f;
        ls += (double)v[j];
    }
    ls = wave_sum_dpp(ls);
    const float inv = (float)(1.0 / ls);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = lane + 64 * j;
        v[j] = __fmul_rn(v[j], inv);
        if (e < E) row[e] = v[j];
        if (e >= E) v[j] = -1.0f;            // probabilities are >= 0; a taken entry drops to -1
    }
    float sel = 0.0f;        // lane k (< K) keeps the k-th selected probability
    for (int k = 0; k < K; ++k) {
        const float m = wave_max_dpp(fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])));
        int eb = -1;                          // the lowest index holding the maximum
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint64_t b = __ballot(v[j] == m);
            if (eb < 0 && b) eb = 64 * j + __builtin_ctzll(b);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) if (lane + 64 * j == eb) v[j] = -1.0f;
        if (lane == k) sel = m;
        if (lane == 0) ids[(int64_t)t * K + k] = (int32_t)eb;
    }
    double s = lane < K ? (double)sel : 0.0;
    for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
    float sf = (float)s;
    if (sf < 6.103515625e-5f) sf = 6.103515625e-5f;
    if (lane < K) w[(int64_t)t * K + lane] = sel / sf;
}

// h += add (add may be null), then x = h * (1 / sqrt(mean(h^2) + eps)); one
// workgroup per token, every load issued before the first sum; the squares
// summed per thread in element order, then over the wave, then the four
// waves in order
constexpr int RMS_PER_THREAD = 16;               // d <= 4096
__global__ __launch_bounds__(WG) void k_residual_rmsnorm(float * __restrict__ h, const float * __restrict__ add,
                                                          int d, float eps, float * __restrict__ x) {
    __shared__ float s_part[WG / 64];
    const int t = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float * ht = h + (int64_t)t * d;
    const float * at = add ? add + (int64_t)t * d : nullptr;
    float v[RMS_PER_THREAD];
#pragma unroll
    for (int j = 0; j < RMS_PER_THREAD; ++j) {
        const int i = threadIdx.x + j * WG;
        v[j] = i < d ? ht[i] : 0.0f;
    }
    if (at) {
#pragma unroll
        for (int j = 0; j < RMS_PER_THREAD; ++j) {
            const int i = threadIdx.x + j * WG;
            if (i < d) {
                v[j] = v[j] + at[i];
                ht[i] = v[j];
            }
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < RMS_PER_THREAD; ++j) ss = __builtin_fmaf(v[j], v[j], ss);
    ss = wave_sum_dpp(ss);
    if (lane == 0) s_part[wave] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int q = 0; q < WG / 64; ++q) tot += s_part[q];
    const float inv = 1.0f / __fsqrt_rn(tot / (float)d + eps);
#pragma unroll
    for (int j = 0; j < RMS_PER_THREAD; ++j) {
        const int i = threadIdx.x + j * WG;
        if (i < d) x[(int64_t)t * d + i] = v[j] * inv;
    }
}

// out[t][r] = ((w0 y0 + w1 y1) + w2 y2) + ...   (llama-graph.cpp:1812-1840:
// ggml_mul by the weights, then the views added in order)
__global__ __launch_bounds__(WG) void k_combine(const float * __restrict__ y, const float * __restrict__ w, int K, int D,
                                                float * __restrict__ out) {
#pragma clang fp contract(off)
    const int r = blockIdx.x * WG + threadIdx.x, t = blockIdx.y;
    if (r >= D) return;
    // every product and sum rounded on its own (ggml_mul, then ggml_add):
    // plain operators under the pragma (__fmul_rn / __fadd_rn are header
    // functions whose operations the compiler may still fuse)
    const float * yp = y + (int64_t)t * K * D + r;
    const float * wt = w + (int64_t)t * K;
    float o;
    if (K <= 16) {
        // every load issued before the first use
        float yv[16], wv[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            yv[k] = k < K ? yp[(int64_t)k * D] : 0.0f;
            wv[k] = k < K ? wt[k] : 0.0f;
        }
        o = yv[0] * wv[0];
#pragma unroll
        for (int k = 1; k < 16; ++k)
            if (k < K) o = o + yv[k] * wv[k];
    } else {
        o = yp[0] * wt[0];
        for (int k = 1; k < K; ++k) o = o + yp[(int64_t)k * D] * wt[k];
    }
    out[(int64_t)t * D + r] = o;
}

template <int SRC>
__global__ __launch_bounds__(WG) void k_geglu(const float * __restrict__ gu, int F, float * __restrict__ out) {
    const int i = blockIdx.x * WG + threadIdx.x, c = blockIdx.y;
    if (i >= F) return;
    const float * col = gu + (int64_t)c * 2 * F;
    out[(int64_t)c * F + i] = geglu1<SRC>(col[i], col[F + i]);
}

// ----------------------------------------------------------- island

// Residency partition of the routed pairs of one fire, one lane per pair
// (moert/cuda/ffn_moe.cu:80-130): pair p of token t = p / n_used reads
// ids[t*ids_s1 + p - t*n_used]; hot iff the READY mirror predicate holds.
// Compaction keeps ascending p on both sides (64-bit ballot + popcount).
__global__ __launch_bounds__(64) void k_partition(const int32_t * __restrict__ ids, int n_used, int ids_s1, int n_pairs,
                                                  const int32_t * __restrict__ exp_slot, const int32_t * __restrict__ slot_exp,
                                                  const int32_t * __restrict__ slot_state, int n_expert, int K,
                                                  int32_t * __restrict__ ids_hot, int32_t * __restrict__ ids_cold,
                                                  int32_t * __restrict__ hot_dst, int32_t * __restrict__ cold_dst,
                                                  int32_t * __restrict__ counts, int32_t * __restrict__ rc_counts,
                                                  int32_t * __restrict__ rc_hits) {
    const int lane = threadIdx.x;
    const bool valid = lane < n_pairs;
    int e = -1, slot = -1;
    bool hot = false;
    if (valid) {
        const int t = lane / n_used;
        e = ids[t * ids_s1 + (lane - t * n_used)];
        if (e >= 0 && e < n_expert && K > 0) {
            const int s = exp_slot[e];
            if (s >= 0 && s < K && slot_state[s] == 2 && slot_exp[s] == e) { hot = true; slot = s; }
        }
    }
    const uint64_t hm = __ballot(valid && hot), cm = __ballot(valid && !hot);
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    if (valid && hot) {
        const int i = __popcll(hm & below);
        ids_hot[i] = slot;
        hot_dst[i] = lane;
    } else if (valid) {
        const int i = __popcll(cm & below);
        ids_cold[i] = e;
        cold_dst[i] = lane;
    }
    if (lane == 0) {
        counts[0] = __popcll(hm);
        counts[1] = __popcll(cm);
    }
    if (rc_counts && valid && e >= 0 && e < n_expert) atomicAdd(&rc_counts[e], 1);
    if (rc_hits && lane == 0) {
        atomicAdd(&rc_hits[0], (int)__popcll(hm));
        atomicAdd(&rc_hits[1], (int)__popcll(cm));
    }
}

// Routing counters without the partition (the fused layer's generic path):
// the same counts k_partition adds, for any number of pairs.  One workgroup.
__global__ __launch_bounds__(WG) void k_route_count(const int32_t * __restrict__ ids, int n_used, int ids_s1,
                                                    int n_pairs, const int32_t * __restrict__ exp_slot,
                                                    const int32_t * __restrict__ slot_exp,
                                                    const int32_t * __restrict__ slot_state, int n_expert, int K,
                                                    int32_t * __restrict__ rc_counts, int32_t * __restrict__ rc_hits) {
    __shared__ int s_hot;
    if (threadIdx.x == 0) s_hot = 0;
    __syncthreads();
    int hot = 0;
    for (int q = threadIdx.x; q < n_pairs; q += WG) {
        const int t = q / n_used;
        const int e = ids[t * ids_s1 + (q - t * n_used)];
        if (e >= 0 && e < n_expert) {
            atomicAdd(&rc_counts[e], 1);
            if (K > 0) {
                const int sl = exp_slot[e];
                if (sl >= 0 && sl < K && slot_state[sl] == 2 && slot_exp[sl] == e) ++hot;
            }
        }
    }
    if (hot) atomicAdd(&s_hot, hot);
    __syncthreads();
    if (threadIdx.x == 0 && rc_hits) {
        atomicAdd(&rc_hits[0], s_hot);
        atomicAdd(&rc_hits[1], n_pairs - s_hot);
    }
}

// x_side[i] = activation column of compact pair i (ffn_moe.cu:135-153)
__global__ __launch_bounds__(WG) void k_gather(const float * __restrict__ cur, int D_in, int kind, int n_used,
                                               const int32_t * __restrict__ counts, const int32_t * __restrict__ hot_dst,
                                               const int32_t * __restrict__ cold_dst, float * __restrict__ x_hot,
                                               float * __restrict__ x_cold) {
    const int i = blockIdx.x, side = blockIdx.y;
    if (i >= counts[side]) return;
    const int p = side == 0 ? hot_dst[i] : cold_dst[i];
    const int src_col = kind == 0 ? p / n_used : p;
    float * dst = (side == 0 ? x_hot : x_cold) + (int64_t)i * D_in;
    const float * src = cur + (int64_t)src_col * D_in;
    if ((D_in & 3) == 0) {
        for (int k = threadIdx.x; k < (D_in >> 2); k += WG)
            reinterpret_cast<float4 *>(dst)[k] = reinterpret_cast<const float4 *>(src)[k];
    } else {
        for (int k = threadIdx.x; k < D_in; k += WG) dst[k] = src[k];
    }
}

// y_full[p] = y_side[i] * (kind == 1 ? scale : 1) (ffn_moe.cu:158-176)
__global__ __launch_bounds__(WG) void k_scatter(const float * __restrict__ y_hot, const float * __restrict__ y_cold, int D_out,
                                                int kind, const int32_t * __restrict__ counts,
                                                const int32_t * __restrict__ ids_hot, const int32_t * __restrict__ hot_dst,
                                                const int32_t * __restrict__ ids_cold, const int32_t * __restrict__ cold_dst,
                                                const float * __restrict__ s_hot, const float * __restrict__ s_cold,
                                                float * __restrict__ y_full) {
    const int i = blockIdx.x;
    if (i < counts[0]) {
        const int p = hot_dst[i];
        const float sc = (kind == 1 && s_hot) ? s_hot[ids_hot[i]] : 1.0f;
        for (int o = threadIdx.x; o < D_out; o += WG) y_full[(int64_t)p * D_out + o] = y_hot[(int64_t)i * D_out + o] * sc;
    }
    if (i < counts[1]) {
        const int p = cold_dst[i];
        const float sc = (kind == 1 && s_cold) ? s_cold[ids_cold[i]] : 1.0f;
        for (int o = threadIdx.x; o < D_out; o += WG) y_full[(int64_t)p * D_out + o] = y_cold[(int64_t)i * D_out + o] * sc;
    }
}

}  // namespace dev

using namespace dev;

hipError_t launch_router_logits(const float * x, int T, const float * w_r, const float * bias, int d, int E,
                                float * logits, hipStream_t s) {
    if (d % 4) return hipErrorInvalidValue;
    dim3 grid(E, (T + ROUTER_TOK - 1) / ROUTER_TOK);
    hipLaunchKernelGGL(k_router_logits, grid, dim3(WG), 0, s, x, T, w_r, bias, d, E, logits);
    return hipGetLastError();
}

hipError_t launch_topk(float * probs, int T, int E, int K, int32_t * ids, float * w, hipStream_t s) {
    hipLaunchKernelGGL(k_topk, dim3(T), dim3(64), 0, s, probs, E, K, ids, w, (const float *)nullptr, T,
                       (const float *)nullptr);
    return hipGetLastError();
}

int router_parts_floats(int T, int E) { return RSPLIT * T * E; }

hipError_t launch_router_mfma(const float * x, int T, const float * w_r, int d, int E, float * parts, hipStream_t s) {
    if (d % (16 * RSPLIT) != 0 || T <= 0 || E <= 0) return hipErrorInvalidValue;
    dim3 grid((T + RT - 1) / RT, (E + RT - 1) / RT, RSPLIT);
    if (d / RSPLIT <= RKC_MAX)
        hipLaunchKernelGGL(k_router_mfma_st, grid, dim3(WG), 0, s, x, T, w_r, d, E, d / RSPLIT, parts);
    else hipLaunchKernelGGL(k_router_mfma, grid, dim3(WG), 0, s, x, T, w_r, d, E, d / RSPLIT, parts);
    return hipGetLastError();
}

hipError_t launch_topk_parts(const float * parts, const float * bias, int T, int E, int K, float * probs, int32_t * ids,
                             float * w, hipStream_t s) {
    hipLaunchKernelGGL(k_topk, dim3(T), dim3(64), 0, s, probs, E, K, ids, w, parts, T, bias);
    return hipGetLastError();
}

hipError_t launch_residual_rmsnorm(float * h, const float * add, int T, int d, float eps, float * x, hipStream_t s) {
    if (d <= 0 || d > RMS_PER_THREAD * WG) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_residual_rmsnorm, dim3(T), dim3(WG), 0, s, h, add, d, eps, x);
    return hipGetLastError();
}

hipError_t launch_combine(const float * y, const float * w, int T, int K, int D, float * out, hipStream_t s) {
    hipLaunchKernelGGL(k_combine, dim3((D + WG - 1) / WG, T), dim3(WG), 0, s, y, w, K, D, out);
    return hipGetLastError();
}

hipError_t launch_geglu(const float * gu, int F, int n_cols, float * out, int mode, hipStream_t s) {
    dim3 grid((F + WG - 1) / WG, n_cols);
    if (mode == 1) hipLaunchKernelGGL(k_geglu<SRC_GEGLU_TANH>, grid, dim3(WG), 0, s, gu, F, out);
    else hipLaunchKernelGGL(k_geglu<SRC_GEGLU_TABLE>, grid, dim3(WG), 0, s, gu, F, out);
    return hipGetLastError();
}

hipError_t launch_partition(const int32_t * ids, int n_used, int ids_s1, int n_pairs, const int32_t * exp_slot,
                            const int32_t * slot_exp, const int32_t * slot_state, int n_expert, int K,
                            int32_t * ids_hot, int32_t * ids_cold, int32_t * hot_dst, int32_t * cold_dst,
                            int32_t * counts, int32_t * rc_counts, int32_t * rc_hits, hipStream_t s) {
    hipLaunchKernelGGL(k_partition, dim3(1), dim3(64), 0, s, ids, n_used, ids_s1, n_pairs, exp_slot, slot_exp,
                       slot_state, n_expert, K, ids_hot, ids_cold, hot_dst, cold_dst, counts, rc_counts, rc_hits);
    return hipGetLastError();
}

hipError_t launch_route_count(const int32_t * ids, int n_used, int ids_s1, int n_pairs, const int32_t * exp_slot,
                              const int32_t * slot_exp, const int32_t * slot_state, int n_expert, int K,
                              int32_t * rc_counts, int32_t * rc_hits, hipStream_t s) {
    if (!rc_counts || n_pairs <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_route_count, dim3(1), dim3(WG), 0, s, ids, n_used, ids_s1, n_pairs, exp_slot, slot_exp,
                       slot_state, n_expert, K, rc_counts, rc_hits);
    return hipGetLastError();
}

hipError_t launch_gather(const float * cur, int D_in, int kind, int n_used, const int32_t * counts,
                         const int32_t * hot_dst, const int32_t * cold_dst, float * x_hot, float * x_cold,
                         int Pmax, hipStream_t s) {
    hipLaunchKernelGGL(k_gather, dim3(Pmax, 2), dim3(WG), 0, s, cur, D_in, kind, n_used, counts, hot_dst, cold_dst,
                       x_hot, x_cold);
    return hipGetLastError();
}

hipError_t launch_scatter(const float * y_hot, const float * y_cold, int D_out, int kind, const int32_t * counts,
                          const int32_t * ids_hot, const int32_t * hot_dst, const int32_t * ids_cold,
                          const int32_t * cold_dst, const float * s_hot, const float * s_cold, float * y_full,
                          int Pmax, hipStream_t s) {
    hipLaunchKernelGGL(k_scatter, dim3(Pmax), dim3(WG), 0, s, y_hot, y_cold, D_out, kind, counts, ids_hot, hot_dst,
                       ids_cold, cold_dst, s_hot, s_cold, y_full);
    return hipGetLastError();
}

}  // namespace llapis
