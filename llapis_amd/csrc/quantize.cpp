// quantize.cpp -- host-side expert-pool preparation: the weight quantisers of
// the four formats on the path, and the seeded synthetic-data generator.
//
// The quantisers follow ggml's algorithms operation for operation, so a pool
// prepared here is byte-identical to one written by ggml_quantize_chunk
// (third_party/llama/ggml/src/ggml.c:7761-7800):
//   Q4_K   quantize_row_q4_K_ref + make_qkx2_quants   (ggml-quants.c:741-820, 1399-1469)
//   Q5_0   quantize_row_q5_0_ref                      (ggml-quants.c:149-190)
//   IQ4_NL quantize_iq4_nl / quantize_row_iq4_nl_impl (ggml-quants.c:4894-5026)
//   IQ2_S  quantize_iq2_s + iq2xs_init_impl           (ggml-quants.c:2781-3196, 5070-5249)
// This file is built with -ffp-contract=off: every float expression rounds in
// the order written, as ggml-base's own (no -march) build does.
#include "formats.h"

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <thread>
#include <vector>

namespace llapis {
namespace {

// round to nearest, ties to even, for |x| <= 2^22 (ggml-quants.c:563-568)
inline int nearest_int(float fval) {
    float val = fval + 12582912.f;
    int i;
    memcpy(&i, &val, sizeof(int));
    return (i & 0x007fffff) - 0x00400000;
}

// ---------------------------------------------------------------- Q4_K

float make_qkx2_quants(int n, int nmax, const float * x, const float * weights, uint8_t * L, float * the_min,
                       uint8_t * Laux, float rmin, float rdelta, int nstep) {
    float min = x[0], max = x[0];
    float sum_w = weights[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        const float w = weights[i];
        sum_w += w;
        sum_x += w * x[i];
    }
    if (min > 0) min = 0;
    if (max == min) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *the_min = -min;
        return 0.f;
    }
    float iscale = nmax / (max - min);
    float scale = 1 / iscale;
    float best_error = 0;
    for (int i = 0; i < n; ++i) {
        const int l = nearest_int(iscale * (x[i] - min));
        L[i] = (uint8_t)std::max(0, std::min(nmax, l));
        float diff = scale * L[i] + min - x[i];
        diff = diff * diff;
        best_error += weights[i] * diff;
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * (x[i] - min));
            l = std::max(0, std::min(nmax, l));
            Laux[i] = (uint8_t)l;
            const float w = weights[i];
            sum_l += w * l;
            sum_l2 += w * l * l;
            sum_xl += w * l * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float cur_error = 0;
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * Laux[i] + this_min - x[i];
                diff = diff * diff;
                cur_error += weights[i] * diff;
            }
            if (cur_error < best_error) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best_error = cur_error;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    *the_min = -min;
    return scale;
}

inline void q4k_scale_min(int j, const uint8_t * q, uint8_t * d, uint8_t * m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4);
    }
}

void quantize_block_q4_K(const float * x, blk_q4_K * y) {
    uint8_t L[QK_K], Laux[32];
    float weights[32], mins[8], scales[8];
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 8; ++j) {
        float sum_x2 = 0;
        for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
        const float av_x = sqrtf(sum_x2 / 32);
        for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(x[32 * j + l]);
        scales[j] = make_qkx2_quants(32, 15, x + 32 * j, weights, L + 32 * j, &mins[j], Laux, -1.f, 0.1f, 20);
        if (scales[j] > max_scale) max_scale = scales[j];
        if (mins[j] > max_min) max_min = mins[j];
    }
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    memset(y->scales, 0, 12);
    for (int j = 0; j < 8; ++j) {
        uint8_t ls = (uint8_t)nearest_int(inv_scale * scales[j]);
        uint8_t lm = (uint8_t)nearest_int(inv_min * mins[j]);
        ls = std::min<uint8_t>(63, ls);
        lm = std::min<uint8_t>(63, lm);
        if (j < 4) {
            y->scales[j] = ls;
            y->scales[j + 4] = lm;
        } else {
            y->scales[j + 4] = (ls & 0xF) | ((lm & 0xF) << 4);
            y->scales[j - 4] |= ((ls >> 4) << 6);
            y->scales[j - 0] |= ((lm >> 4) << 6);
        }
    }
    y->d = float_to_half(max_scale / 63.f);
    y->dmin = float_to_half(max_min / 63.f);
    for (int j = 0; j < 8; ++j) {
        uint8_t sc, m;
        q4k_scale_min(j, y->scales, &sc, &m);
        const float d = half_to_float(y->d) * sc;
        if (!d) continue;
        const float dm = half_to_float(y->dmin) * m;
        for (int ii = 0; ii < 32; ++ii) {
            int l = nearest_int((x[32 * j + ii] + dm) / d);
            L[32 * j + ii] = (uint8_t)std::max(0, std::min(15, l));
        }
    }
    uint8_t * q = y->qs;
    for (int j = 0; j < QK_K; j += 64) {
        for (int l = 0; l < 32; ++l) q[l] = L[j + l] | (L[j + l + 32] << 4);
        q += 32;
    }
}

// ---------------------------------------------------------------- Q5_0

void quantize_block_q5_0(const float * x, blk_q5_0 * y) {
    float amax = 0.0f, max = 0.0f;
    for (int j = 0; j < 32; j++) {
        const float v = x[j];
        if (amax < fabsf(v)) {
            amax = fabsf(v);
            max = v;
        }
    }
    const float d = max / -16;
    const float id = d ? 1.0f / d : 0.0f;
    y->d = float_to_half(d);
    uint32_t qh = 0;
    for (int j = 0; j < 16; ++j) {
        const float x0 = x[0 + j] * id;
        const float x1 = x[16 + j] * id;
        const uint8_t xi0 = std::min<uint8_t>(31, (uint8_t)(int8_t)(x0 + 16.5f));
        const uint8_t xi1 = std::min<uint8_t>(31, (uint8_t)(int8_t)(x1 + 16.5f));
        y->qs[j] = (xi0 & 0x0F) | ((xi1 & 0x0F) << 4);
        qh |= ((xi0 & 0x10u) >> 4) << (j + 0);
        qh |= ((xi1 & 0x10u) >> 4) << (j + 16);
    }
    memcpy(y->qh, &qh, 4);
}

// ---------------------------------------------------------------- IQ4_NL

const int8_t kIq4nl[16] = LLAPIS_IQ4NL_VALUES;

inline int best_index_int8(int n, const int8_t * val, float x) {
    if (x <= val[0]) return 0;
    if (x >= val[n - 1]) return n - 1;
    int ml = 0, mu = n - 1;
    while (mu - ml > 1) {
        const int mav = (ml + mu) / 2;
        if (x < val[mav]) mu = mav; else ml = mav;
    }
    return x - val[mu - 1] < val[mu] - x ? mu - 1 : mu;
}

// one 32-value block (super-block size == block size == 32, ntry = 7)
void quantize_block_iq4_nl(const float * x, blk_iq4_nl * y, const float * qw) {
    const int ntry = 7;
    uint8_t L[32];
    float weight[32];
    float sigma2 = 0;
    for (int j = 0; j < 32; ++j) sigma2 += x[j] * x[j];
    sigma2 *= 2.f / 32;
    memset(y->qs, 0, 16);
    y->d = float_to_half(0.f);
    float scale0;
    if (qw) {
        for (int j = 0; j < 32; ++j) weight[j] = qw[j] * sqrtf(sigma2 + x[j] * x[j]);
    } else {
        for (int j = 0; j < 32; ++j) weight[j] = x[j] * x[j];
    }
    float amax = 0, max = 0;
    for (int j = 0; j < 32; ++j) {
        const float ax = fabsf(x[j]);
        if (ax > amax) {
            amax = ax;
            max = x[j];
        }
    }
    if (amax < 1e-15f) {
        scale0 = 0;
    } else {
        float d = ntry > 0 ? -max / kIq4nl[0] : max / kIq4nl[0];
        float id = 1 / d;
        float sumqx = 0, sumq2 = 0;
        for (int j = 0; j < 32; ++j) {
            const float al = id * x[j];
            const int l = best_index_int8(16, kIq4nl, al);
            L[j] = (uint8_t)l;
            const float q = kIq4nl[l];
            const float w = weight[j];
            sumqx += w * q * x[j];
            sumq2 += w * q * q;
        }
        d = sumq2 > 0 ? sumqx / sumq2 : 0.f;
        float best = d * sumqx;
        for (int itry = -ntry; itry <= ntry; ++itry) {
            id = (itry + kIq4nl[0]) / max;
            sumqx = sumq2 = 0;
            for (int j = 0; j < 32; ++j) {
                const float al = id * x[j];
                const int l = best_index_int8(16, kIq4nl, al);
                const float q = kIq4nl[l];
                const float w = weight[j];
                sumqx += w * q * x[j];
                sumq2 += w * q * q;
            }
            if (sumq2 > 0 && sumqx * sumqx > best * sumq2) {
                d = sumqx / sumq2;
                best = d * sumqx;
            }
        }
        scale0 = d;
    }
    y->d = float_to_half(scale0);
    const float id = scale0 ? 1 / scale0 : 0;
    for (int j = 0; j < 32; ++j) L[j] = (uint8_t)best_index_int8(16, kIq4nl, id * x[j]);
    for (int j = 0; j < 16; ++j) y->qs[j] = L[j] | (L[16 + j] << 4);
}

// ---------------------------------------------------------------- IQ2_S

const uint16_t kIq2sCodes[1024] = {
#include "iq2s_grid.inc"
};

// The quantiser's view of the codebook: per grid point the 8 levels as bytes
// 2l+1, the map from a 16-bit level code to its grid index (or -1), and for
// every level code off the grid the grid points at minimum squared distance,
// in ascending index order (ggml-quants.c:3036-3186 with nwant = 1).
struct Iq2sTables {
    int8_t grid[1024][8];
    std::vector<int> map;                       // 43692 entries
    std::vector<std::vector<uint16_t>> neigh;   // per off-grid code
    Iq2sTables() : map(43692, -1), neigh(43692) {
        for (int k = 0; k < 1024; ++k) {
            uint16_t index = 0;
            for (int i = 0; i < 8; ++i) {
                const int l = (kIq2sCodes[k] >> (2 * i)) & 3;
                grid[k][i] = (int8_t)(2 * l + 1);
                index |= (uint16_t)(l << (2 * i));
            }
            map[index] = k;
        }
        for (int u = 0; u < 43692; ++u) {
            if (map[u] >= 0) continue;
            bool valid = true;                  // codes the quantiser can form: levels 0..2
            int8_t pos[8];
            for (int i = 0; i < 8; ++i) {
                const int l = (u >> (2 * i)) & 3;
                if (l == 3) valid = false;
                pos[i] = (int8_t)(2 * l + 1);
            }
            if (!valid) continue;
            int best = 1 << 30;
            for (int j = 0; j < 1024; ++j) {
                int d2 = 0;
                for (int i = 0; i < 8; ++i) d2 += (grid[j][i] - pos[i]) * (grid[j][i] - pos[i]);
                if (d2 < best) { best = d2; neigh[u].clear(); }
                if (d2 == best) neigh[u].push_back((uint16_t)j);
            }
        }
    }
};

const Iq2sTables & iq2s_tables() {
    static const Iq2sTables t;
    return t;
}

int iq2_find_best_neighbour(const Iq2sTables & T, const std::vector<uint16_t> & nb, const float * xval,
                            const float * weight, float scale, int8_t * L) {
    float best_d2 = FLT_MAX;
    int grid_index = -1;
    for (const uint16_t j : nb) {
        const int8_t * pg = T.grid[j];
        float d2 = 0;
        for (int i = 0; i < 8; ++i) {
            const float q = pg[i];
            const float diff = scale * q - xval[i];
            d2 += weight[i] * diff * diff;
        }
        if (d2 < best_d2) {
            best_d2 = d2;
            grid_index = j;
        }
    }
    const int8_t * pg = T.grid[grid_index];
    for (int i = 0; i < 8; ++i) L[i] = (int8_t)((pg[i] - 1) / 2);
    return grid_index;
}

void quantize_superblock_iq2_s(const float * xbl, blk_iq2_s * y, const float * qw_row) {
    const Iq2sTables & T = iq2s_tables();
    const int kMaxQ = 3;
    float scales[16], weight[16], xval[16], waux[16];
    int8_t L[16], Laux[16];
    bool is_on_grid[2], is_on_grid_aux[2];
    uint8_t block_signs[2];

    memset(y, 0, sizeof(blk_iq2_s));
    y->d = float_to_half(0.f);
    float max_scale = 0;
    float sumx2 = 0;
    for (int i = 0; i < QK_K; ++i) sumx2 += xbl[i] * xbl[i];
    const float sigma2 = 2 * sumx2 / QK_K;

    for (int ib = 0; ib < 16; ++ib) {
        const float * xb = xbl + 16 * ib;
        if (qw_row) {
            const float * qw = qw_row + 16 * ib;
            for (int i = 0; i < 16; ++i) weight[i] = qw[i] * sqrtf(sigma2 + xb[i] * xb[i]);
        } else {
            for (int i = 0; i < 16; ++i) weight[i] = 0.25f * sigma2 + xb[i] * xb[i];
        }
        for (int i = 0; i < 16; ++i) waux[i] = sqrtf(weight[i]);
        for (int k = 0; k < 2; ++k) {
            uint8_t s = 0;
            for (int i = 0; i < 8; ++i) {
                if (xb[8 * k + i] >= 0) {
                    xval[8 * k + i] = xb[8 * k + i];
                } else {
                    xval[8 * k + i] = -xb[8 * k + i];
                    s |= (uint8_t)(1 << i);
                }
            }
            block_signs[k] = s;
        }
        float max = xval[0];
        for (int i = 1; i < 16; ++i) max = std::max(max, xval[i]);
        memset(L, 0, 16);
        if (max < 1e-8f) {
            scales[ib] = 0;
            continue;
        }
        float best = 0;
        float scale = max / (2 * kMaxQ - 1);
        is_on_grid[0] = is_on_grid[1] = true;
        for (int is = -9; is <= 9; ++is) {
            const float id = (2 * kMaxQ - 1 + is * 0.1f) / max;
            const float this_scale = 1 / id;
            for (int k = 0; k < 2; ++k) {
                for (int i = 0; i < 8; ++i) {
                    const int l = nearest_int(0.5f * (id * xval[8 * k + i] - 1));
                    Laux[8 * k + i] = (int8_t)std::max(0, std::min(kMaxQ - 1, l));
                }
                uint16_t u = 0;
                for (int i = 0; i < 8; ++i) u |= (uint16_t)(Laux[8 * k + i] << (2 * i));
                is_on_grid_aux[k] = true;
                if (T.map[u] < 0) {
                    is_on_grid_aux[k] = false;
                    iq2_find_best_neighbour(T, T.neigh[u], xval + 8 * k, waux + 8 * k, this_scale, Laux + 8 * k);
                }
            }
            float sumqx = 0, sumq2 = 0;
            for (int i = 0; i < 16; ++i) {
                const float w = weight[i];
                const float q = 2 * Laux[i] + 1;
                sumqx += w * xval[i] * q;
                sumq2 += w * q * q;
            }
            if (sumq2 > 0 && sumqx * sumqx > best * sumq2) {
                scale = sumqx / sumq2;
                best = scale * sumqx;
                for (int i = 0; i < 16; ++i) L[i] = Laux[i];
                for (int k = 0; k < 2; ++k) is_on_grid[k] = is_on_grid_aux[k];
            }
        }
        int n_not_ongrid = 0;
        for (int k = 0; k < 2; ++k) if (!is_on_grid[k]) ++n_not_ongrid;
        if (n_not_ongrid > 0 && scale > 0) {
            const float id = 1 / scale;
            for (int k = 0; k < 2; ++k) {
                if (is_on_grid[k]) continue;
                uint16_t u = 0;
                for (int i = 0; i < 8; ++i) {
                    int l = nearest_int(0.5f * (id * xval[8 * k + i] - 1));
                    l = std::max(0, std::min(kMaxQ - 1, l));
                    u |= (uint16_t)(l << (2 * i));
                    L[8 * k + i] = (int8_t)l;
                }
                if (T.map[u] < 0)
                    iq2_find_best_neighbour(T, T.neigh[u], xval + 8 * k, waux + 8 * k, scale, L + 8 * k);
            }
            float sumqx = 0, sumq2 = 0;
            for (int i = 0; i < 16; ++i) {
                const float w = weight[i];
                const float q = 2 * L[i] + 1;
                sumqx += w * xval[i] * q;
                sumq2 += w * q * q;
            }
            if (sumq2 > 0) scale = sumqx / sumq2;
        }
        if (scale < 0) {
            scale = -scale;
            for (int k = 0; k < 2; ++k) block_signs[k] = (uint8_t)~block_signs[k];
        }
        for (int k = 0; k < 2; ++k) {
            uint16_t u = 0;
            for (int i = 0; i < 8; ++i) u |= (uint16_t)(L[8 * k + i] << (2 * i));
            const int grid_index = T.map[u];
            if (grid_index < 0) {
                fprintf(stderr, "llapis: IQ2_S level code %u is not on the grid\n", u);
                abort();
            }
            const int i8 = 2 * ib + k;
            y->qs[i8] = (uint8_t)(grid_index & 255);
            y->qh[i8 / 4] |= (uint8_t)((grid_index >> 8) << (2 * (i8 % 4)));
            y->qs[32 + i8] = block_signs[k];
        }
        scales[ib] = scale;
        max_scale = std::max(max_scale, scale);
    }
    if (!max_scale) return;
    const float d = max_scale / 31;
    y->d = float_to_half(d * 0.9875f);
    const float id = 1 / d;
    for (int ib = 0; ib < 16; ++ib) {
        int l = nearest_int(0.5f * (id * scales[ib] - 1));
        l = std::max(0, std::min(15, l));
        if (ib % 2 == 0) y->scales[ib / 2] = (uint8_t)l;
        else y->scales[ib / 2] |= (uint8_t)(l << 4);
    }
}

// ------------------------------------------------------------- driver

void quantize_row(int type, const float * x, uint8_t * dst, int64_t n, const float * imatrix) {
    switch (type) {
        case T_Q4_K:
            for (int64_t b = 0; b < n / QK_K; ++b) quantize_block_q4_K(x + b * QK_K, (blk_q4_K *)dst + b);
            break;
        case T_Q5_0:
            for (int64_t b = 0; b < n / 32; ++b) quantize_block_q5_0(x + b * 32, (blk_q5_0 *)dst + b);
            break;
        case T_IQ4_NL:
            for (int64_t b = 0; b < n / 32; ++b)
                quantize_block_iq4_nl(x + b * 32, (blk_iq4_nl *)dst + b, imatrix ? imatrix + b * 32 : nullptr);
            break;
        case T_IQ2_S:
            for (int64_t b = 0; b < n / QK_K; ++b)
                quantize_superblock_iq2_s(x + b * QK_K, (blk_iq2_s *)dst + b, imatrix ? imatrix + b * QK_K : nullptr);
            break;
        default:
            abort();
    }
}

int n_workers(int64_t nrow) {
    const unsigned hc = std::thread::hardware_concurrency();
    int n = (int)std::min<unsigned>(hc ? hc : 1, 16);
    if (nrow < n) n = (int)std::max<int64_t>(1, nrow);
    return n;
}

template <class F>
void parallel_rows(int64_t nrow, F f) {
    const int nw = n_workers(nrow);
    if (nw <= 1) { f(0, nrow); return; }
    std::vector<std::thread> th;
    const int64_t chunk = (nrow + nw - 1) / nw;
    for (int w = 0; w < nw; ++w) {
        const int64_t r0 = w * chunk, r1 = std::min(nrow, r0 + chunk);
        if (r0 >= r1) break;
        th.emplace_back([=] { f(r0, r1); });
    }
    for (auto & t : th) t.join();
}

inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

}  // namespace
}  // namespace llapis

using namespace llapis;

extern "C" {

uint64_t llapis_row_size(int32_t type, int64_t n) {
    if (blk_bytes(type) == 0 || n % blk_elems(type) != 0) return 0;
    return row_bytes(type, n);
}

// Same contract as ggml_quantize_chunk for a whole tensor (ggml.c:7761):
// nrow rows of n_per_row floats into dst; imatrix (n_per_row floats) or NULL
// (IQ2_S and IQ4_NL only).  Returns bytes written, 0 for an unsupported
// type, shape or imatrix use.
uint64_t llapis_quantize(int32_t type, const float * src, void * dst, int64_t nrow, int64_t n_per_row,
                         const float * imatrix) {
    if (type != T_Q4_K && type != T_Q5_0 && type != T_IQ4_NL && type != T_IQ2_S) return 0;
    if (n_per_row % blk_elems(type) != 0) return 0;
    // Q4_K and Q5_0 with an importance matrix take ggml's *_impl variants,
    // which this library does not restate: refuse rather than differ.
    if (imatrix && (type == T_Q4_K || type == T_Q5_0)) return 0;
    const uint64_t rb = row_bytes(type, n_per_row);
    if (type == T_IQ2_S) (void)iq2s_tables();   // build once, before the workers start
    parallel_rows(nrow, [&](int64_t r0, int64_t r1) {
        for (int64_t r = r0; r < r1; ++r)
            quantize_row(type, src + r * n_per_row, (uint8_t *)dst + r * rb, n_per_row, imatrix);
    });
    return rb * (uint64_t)nrow;
}

// Seeded N(mean, std) floats: element i depends only on (seed, i), so any
// slice can be generated independently (Box-Muller over a counter hash).
void llapis_synth_normal(uint64_t seed, int64_t offset, int64_t n, float mean, float stddev, float * out) {
    const int64_t pairs_lo = offset / 2, pairs_hi = (offset + n + 1) / 2;
    parallel_rows(pairs_hi - pairs_lo, [&](int64_t p0, int64_t p1) {
        for (int64_t p = pairs_lo + p0; p < pairs_lo + p1; ++p) {
            const uint64_t a = mix64(seed * 0x9e3779b97f4a7c15ULL + 2 * (uint64_t)p + 1);
            const uint64_t b = mix64(seed * 0x9e3779b97f4a7c15ULL + 2 * (uint64_t)p + 2);
            const double u1 = ((double)(a >> 11) + 0.5) * (1.0 / 9007199254740992.0);
            const double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);
            const double r = sqrt(-2.0 * log(u1));
            const double z0 = r * cos(6.283185307179586 * u2), z1 = r * sin(6.283185307179586 * u2);
            const int64_t i0 = 2 * p - offset, i1 = i0 + 1;
            if (i0 >= 0 && i0 < n) out[i0] = (float)(mean + stddev * z0);
            if (i1 >= 0 && i1 < n) out[i1] = (float)(mean + stddev * z1);
        }
    });
}

}  // extern "C"
