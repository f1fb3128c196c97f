// quantize.cpp -- host-side expert-pool preparation: the weight quantisers of
// the four formats on the path, and the seeded synthetic-data generator.
//
// A pool prepared here is byte-identical to one written by the reference's
// ggml_quantize_chunk (third_party/llama/ggml/src/ggml.c:7761-7800), whose
// quantisers are (ggml-quants.c):
//   Q4_K   quantize_row_q4_K_ref, make_qkx2_quants          (:741-820, :1399-1469)
//   Q5_0   quantize_row_q5_0_ref                            (:149-190)
//   IQ4_NL quantize_iq4_nl, quantize_row_iq4_nl_impl        (:4894-5026)
//   IQ2_S  quantize_iq2_s, quantize_row_iq2_s_impl          (:5070-5249)
// Byte equality fixes each algorithm's float operations and their order:
// every weight, sum, candidate scale and comparison below is formed with the
// same operands in the same association as there (this file is built with
// -ffp-contract=off, like ggml-base's own build).  Rounding to the nearest
// integer, halves to even, is lrintf (exact for the magnitudes that occur,
// all far below 2^22).
#include "formats.h"

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <thread>
#include <vector>

namespace llapis {
namespace {

inline int rne(float v) { return (int)lrintf(v); }
inline int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

// ----------------------------------------------------------------- Q4_K
//
// A super-block is 8 sub-blocks of 32.  Each sub-block gets an affine fit
// x ~ s q + m (q in 0..15, m <= 0) by weighted least squares over candidate
// level assignments; the 8 scales and 8 offsets are then stored as 6-bit
// multiples of two fp16 super-block steps, and the levels re-derived from the
// stored (rounded) scales.

constexpr int kQ4Top = 15;

struct SubBlockFit {
    float scale = 0.0f;      // s
    float neg_min = 0.0f;    // -m
};

// The weighted squared error of (s, m) with levels q.
inline float affine_error(const float * x, const float * w, const uint8_t * q, float s, float m) {
    float e = 0;
    for (int i = 0; i < 32; ++i) {
        float r = s * q[i] + m - x[i];
        r = r * r;
        e += w[i] * r;
    }
    return e;
}

// levels of x at inverse step inv from origin lo
inline void affine_levels(const float * x, float inv, float lo, uint8_t * q) {
    for (int i = 0; i < 32; ++i) q[i] = (uint8_t)clampi(rne(inv * (x[i] - lo)), 0, kQ4Top);
}

// The fit of one sub-block: the range's own step first, then 21 steps around
// it (inverse steps (15 - 1 + 0.1 t) / range, t = 0..20), each with the least-
// squares (s, m) of its levels; the lowest error wins.  The range of a trial
// runs from the offset of the best fit so far (the block's minimum until a
// trial wins), and its levels are counted from that offset.
SubBlockFit fit_sub_block(const float * x, const float * w, uint8_t * q) {
    float lo = x[0], hi = x[0], sw = 0, swx = 0;
    for (int i = 0; i < 32; ++i) {
        lo = std::min(lo, x[i]);
        hi = std::max(hi, x[i]);
        sw += w[i];
        swx += w[i] * x[i];
    }
    lo = std::min(lo, 0.0f);
    SubBlockFit fit;
    if (hi == lo) {
        std::fill(q, q + 32, 0);
        fit.neg_min = -lo;
        return fit;
    }
    float inv = kQ4Top / (hi - lo);
    float s = 1 / inv, m = lo;
    affine_levels(x, inv, lo, q);
    float err = affine_error(x, w, q, s, m);
    uint8_t trial[32];
    for (int t = 0; t <= 20; ++t) {
        inv = (-1.f + 0.1f * t + kQ4Top) / (hi - m);
        affine_levels(x, inv, m, trial);
        float sl = 0, sll = 0, sxl = 0;
        for (int i = 0; i < 32; ++i) {
            const int l = trial[i];
            sl += w[i] * l;
            sll += w[i] * l * l;
            sxl += w[i] * l * x[i];
        }
        const float det = sw * sll - sl * sl;
        if (!(det > 0)) continue;
        float ts = (sw * sxl - swx * sl) / det;
        float tm = (sll * swx - sl * sxl) / det;
        if (tm > 0) {
            tm = 0;
            ts = sxl / sll;
        }
        const float te = affine_error(x, w, trial, ts, tm);
        if (te < err) {
            std::copy(trial, trial + 32, q);
            err = te;
            s = ts;
            m = tm;
        }
    }
    fit.scale = s;
    fit.neg_min = -m;
    return fit;
}

// 6-bit code of v on a step of 1 / inv: the integer cast to a byte, then at most 63
inline uint8_t six_bit(float inv, float v) { return std::min<uint8_t>(63, (uint8_t)rne(inv * v)); }

void q4k_super_block(const float * x, blk_q4_K * out) {
    uint8_t lv[QK_K];
    SubBlockFit fits[8];
    float top_scale = 0, top_min = 0;
    for (int j = 0; j < 8; ++j) {
        const float * xs = x + 32 * j;
        float energy = 0;
        for (int i = 0; i < 32; ++i) energy += xs[i] * xs[i];
        const float rms = sqrtf(energy / 32);
        float w[32];
        for (int i = 0; i < 32; ++i) w[i] = rms + fabsf(xs[i]);
        fits[j] = fit_sub_block(xs, w, lv + 32 * j);
        if (fits[j].scale > top_scale) top_scale = fits[j].scale;
        if (fits[j].neg_min > top_min) top_min = fits[j].neg_min;
    }
    const float inv_s = top_scale > 0 ? 63.f / top_scale : 0.f;
    const float inv_m = top_min > 0 ? 63.f / top_min : 0.f;
    uint8_t sc[8], mn[8];
    for (int j = 0; j < 8; ++j) {
        sc[j] = six_bit(inv_s, fits[j].scale);
        mn[j] = six_bit(inv_m, fits[j].neg_min);
    }
    // the 12-byte scale field: sub-blocks 0..3 in the low 6 bits of bytes
    // 0..3 (scales) and 4..7 (mins); sub-blocks 4..7 as nibbles of bytes 8..11
    // with their top two bits in the high bits of bytes 0..7
    for (int j = 0; j < 4; ++j) {
        out->scales[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
        out->scales[j + 4] = (uint8_t)(mn[j] | ((mn[j + 4] >> 4) << 6));
        out->scales[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4));
    }
    out->d = float_to_half(top_scale / 63.f);
    out->dmin = float_to_half(top_min / 63.f);
    // levels against the stored steps (a sub-block whose step rounds to zero
    // keeps its fitted levels)
    const float dd = half_to_float(out->d), dm = half_to_float(out->dmin);
    for (int j = 0; j < 8; ++j) {
        const float step = dd * sc[j];
        if (!step) continue;
        const float off = dm * mn[j];
        for (int i = 0; i < 32; ++i) lv[32 * j + i] = (uint8_t)clampi(rne((x[32 * j + i] + off) / step), 0, kQ4Top);
    }
    // 64 values per 32 bytes: value i in the low nibble, value i + 32 in the high
    for (int c = 0; c < 4; ++c)
        for (int i = 0; i < 32; ++i) out->qs[32 * c + i] = (uint8_t)(lv[64 * c + i] | (lv[64 * c + 32 + i] << 4));
}

// ----------------------------------------------------------------- Q5_0
//
// Symmetric 5-bit levels around 16 on the step of the signed extreme / -16.

void q50_block(const float * x, blk_q5_0 * out) {
    float peak = 0.0f, extreme = 0.0f;          // the first value of largest magnitude
    for (int i = 0; i < 32; ++i)
        if (fabsf(x[i]) > peak) {
            peak = fabsf(x[i]);
            extreme = x[i];
        }
    const float step = extreme / -16;
    const float inv = step ? 1.0f / step : 0.0f;
    out->d = float_to_half(step);
    uint32_t high = 0;
    for (int i = 0; i < 16; ++i) {
        // truncation of a value in [0.5, 32.5], at most 31
        const int a = std::min(31, (int)(x[i] * inv + 16.5f));
        const int b = std::min(31, (int)(x[16 + i] * inv + 16.5f));
        out->qs[i] = (uint8_t)((a & 0xF) | ((b & 0xF) << 4));
        high |= (uint32_t)(a >> 4) << i;
        high |= (uint32_t)(b >> 4) << (16 + i);
    }
    memcpy(out->qh, &high, 4);
}

// ----------------------------------------------------------------- IQ4_NL
//
// Each 32-value block: 16 fixed non-linear levels times one fp16 step, the
// step chosen among the least-squares steps of 16 level assignments.

const int8_t kNlLevels[16] = LLAPIS_IQ4NL_VALUES;

// the level nearest to v (ties to the upper one)
inline int nl_nearest(float v) {
    if (v <= kNlLevels[0]) return 0;
    if (v >= kNlLevels[15]) return 15;
    int up = 1;
    while (kNlLevels[up] <= v) ++up;
    return v - kNlLevels[up - 1] < kNlLevels[up] - v ? up - 1 : up;
}

struct SymSums {
    float qx = 0, qq = 0;   // sum w q x, sum w q q
};

// levels of x at inverse step inv (into lv when given) and their sums
inline SymSums nl_assign(const float * x, const float * w, float inv, uint8_t * lv) {
    SymSums s;
    for (int i = 0; i < 32; ++i) {
        const int l = nl_nearest(inv * x[i]);
        if (lv) lv[i] = (uint8_t)l;
        const float q = kNlLevels[l];
        s.qx += w[i] * q * x[i];
        s.qq += w[i] * q * q;
    }
    return s;
}

void iq4nl_block(const float * x, blk_iq4_nl * out, const float * imat) {
    float w[32];
    if (imat) {
        float energy = 0;
        for (int i = 0; i < 32; ++i) energy += x[i] * x[i];
        energy *= 2.f / 32;
        for (int i = 0; i < 32; ++i) w[i] = imat[i] * sqrtf(energy + x[i] * x[i]);
    } else {
        for (int i = 0; i < 32; ++i) w[i] = x[i] * x[i];
    }
    float peak = 0, extreme = 0;
    for (int i = 0; i < 32; ++i)
        if (fabsf(x[i]) > peak) {
            peak = fabsf(x[i]);
            extreme = x[i];
        }
    float step = 0;
    if (peak >= 1e-15f) {
        // the extreme on the lowest level, then 15 inverse steps around it
        const SymSums s0 = nl_assign(x, w, 1 / (-extreme / kNlLevels[0]), nullptr);
        step = s0.qq > 0 ? s0.qx / s0.qq : 0.f;
        float gain = step * s0.qx;
        for (int t = -7; t <= 7; ++t) {
            const SymSums s = nl_assign(x, w, (t + kNlLevels[0]) / extreme, nullptr);
            if (s.qq > 0 && s.qx * s.qx > gain * s.qq) {
                step = s.qx / s.qq;
                gain = step * s.qx;
            }
        }
    }
    out->d = float_to_half(step);
    const float inv = step ? 1 / step : 0;
    uint8_t lv[32];
    for (int i = 0; i < 32; ++i) lv[i] = (uint8_t)nl_nearest(inv * x[i]);
    for (int i = 0; i < 16; ++i) out->qs[i] = (uint8_t)(lv[i] | (lv[16 + i] << 4));
}

// ----------------------------------------------------------------- IQ2_S
//
// A super-block is 16 blocks of 16 values; each block is two groups of 8,
// each group one of 1024 codebook points of {1, 3, 5}^8 (magnitudes) with a
// sign byte, and the block a 4-bit step multiple.

const uint16_t kIq2sCodes[1024] = {
#include "iq2s_grid.inc"
};

// The codebook as the quantiser uses it: per point the 8 magnitudes 2l + 1;
// the index of each base-4 level code (2 bits per value, levels 0..2) that is
// a point, -1 otherwise; and for each level code off the book the points at
// minimum squared distance, in ascending index order.
struct Codebook {
    int8_t mag[1024][8];
    std::vector<int> index_of;                 // 4^8 codes (the largest formable one is < 43692)
    std::vector<std::vector<uint16_t>> near;   // per off-book code
    Codebook() : index_of(43692, -1), near(43692) {
        for (int k = 0; k < 1024; ++k) {
            uint16_t code = 0;
            for (int i = 0; i < 8; ++i) {
                const int l = (kIq2sCodes[k] >> (2 * i)) & 3;
                mag[k][i] = (int8_t)(2 * l + 1);
                code |= (uint16_t)(l << (2 * i));
            }
            index_of[code] = k;
        }
        for (int code = 0; code < 43692; ++code) {
            if (index_of[code] >= 0) continue;
            int8_t v[8];
            bool formable = true;              // levels 0..2 only
            for (int i = 0; i < 8; ++i) {
                const int l = (code >> (2 * i)) & 3;
                formable = formable && l < 3;
                v[i] = (int8_t)(2 * l + 1);
            }
            if (!formable) continue;
            int best = 1 << 30;
            for (int k = 0; k < 1024; ++k) {
                int d2 = 0;
                for (int i = 0; i < 8; ++i) d2 += (mag[k][i] - v[i]) * (mag[k][i] - v[i]);
                if (d2 < best) {
                    best = d2;
                    near[code].clear();
                }
                if (d2 == best) near[code].push_back((uint16_t)k);
            }
        }
    }
};

const Codebook & codebook() {
    static const Codebook cb;
    return cb;
}

// One group of 8 magnitudes set to levels.  Off the book, the levels become
// those of the nearest point (weighted distance at `step`, the first of equals).
// Returns whether the plain levels were on the book.
bool snap_group(const Codebook & cb, const float * v, const float * sw, float inv, float step, int8_t * lv) {
    uint16_t code = 0;
    for (int i = 0; i < 8; ++i) {
        lv[i] = (int8_t)clampi(rne(0.5f * (inv * v[i] - 1)), 0, 2);
        code |= (uint16_t)(lv[i] << (2 * i));
    }
    if (cb.index_of[code] >= 0) return true;
    float best = FLT_MAX;
    int pick = -1;
    for (const uint16_t k : cb.near[code]) {
        float d2 = 0;
        for (int i = 0; i < 8; ++i) {
            const float q = cb.mag[k][i];
            const float r = step * q - v[i];
            d2 += sw[i] * r * r;
        }
        if (d2 < best) {
            best = d2;
            pick = k;
        }
    }
    for (int i = 0; i < 8; ++i) lv[i] = (int8_t)((cb.mag[pick][i] - 1) / 2);
    return false;
}

// sum w v q and sum w q q of a block's 16 levels (q = 2 l + 1)
inline SymSums iq2_sums(const float * v, const float * w, const int8_t * lv) {
    SymSums s;
    for (int i = 0; i < 16; ++i) {
        const float q = 2 * lv[i] + 1;
        s.qx += w[i] * v[i] * q;
        s.qq += w[i] * q * q;
    }
    return s;
}

void iq2s_super_block(const float * x, blk_iq2_s * out, const float * imat) {
    const Codebook & cb = codebook();
    memset(out, 0, sizeof(*out));
    float energy = 0;
    for (int i = 0; i < QK_K; ++i) energy += x[i] * x[i];
    const float sigma2 = 2 * energy / QK_K;
    float steps[16];
    float top = 0;
    for (int b = 0; b < 16; ++b) {
        const float * xb = x + 16 * b;
        float w[16], sw[16], v[16];
        for (int i = 0; i < 16; ++i) {
            w[i] = imat ? imat[16 * b + i] * sqrtf(sigma2 + xb[i] * xb[i]) : 0.25f * sigma2 + xb[i] * xb[i];
            sw[i] = sqrtf(w[i]);
        }
        uint8_t signs[2] = {0, 0};
        for (int i = 0; i < 16; ++i) {
            v[i] = xb[i] >= 0 ? xb[i] : -xb[i];
            if (!(xb[i] >= 0)) signs[i >> 3] |= (uint8_t)(1 << (i & 7));
        }
        float peak = v[0];
        for (int i = 1; i < 16; ++i) peak = std::max(peak, v[i]);
        steps[b] = 0;
        if (peak < 1e-8f) continue;                        // an empty block: all zero bytes

        // 19 inverse steps (5 + 0.1 t) / peak, t = -9..9; the least-squares
        // step of each assignment, the best gain kept
        int8_t lv[16] = {}, trial[16];
        bool on_book[2] = {true, true};
        float step = peak / 5, gain = 0;
        for (int t = -9; t <= 9; ++t) {
            const float inv = (5 + t * 0.1f) / peak;
            const float at = 1 / inv;
            bool trial_on[2];
            for (int g = 0; g < 2; ++g) trial_on[g] = snap_group(cb, v + 8 * g, sw + 8 * g, inv, at, trial + 8 * g);
            const SymSums s = iq2_sums(v, w, trial);
            if (s.qq > 0 && s.qx * s.qx > gain * s.qq) {
                step = s.qx / s.qq;
                gain = step * s.qx;
                std::copy(trial, trial + 16, lv);
                on_book[0] = trial_on[0];
                on_book[1] = trial_on[1];
            }
        }
        // a group the best assignment had to move onto the book is re-snapped
        // at the final step, and the step refitted
        if ((!on_book[0] || !on_book[1]) && step > 0) {
            const float inv = 1 / step;
            for (int g = 0; g < 2; ++g)
                if (!on_book[g]) snap_group(cb, v + 8 * g, sw + 8 * g, inv, step, lv + 8 * g);
            const SymSums s = iq2_sums(v, w, lv);
            if (s.qq > 0) step = s.qx / s.qq;
        }
        if (step < 0) {
            step = -step;
            signs[0] = (uint8_t)~signs[0];
            signs[1] = (uint8_t)~signs[1];
        }
        for (int g = 0; g < 2; ++g) {
            uint16_t code = 0;
            for (int i = 0; i < 8; ++i) code |= (uint16_t)(lv[8 * g + i] << (2 * i));
            const int k = cb.index_of[code];
            if (k < 0) {
                fprintf(stderr, "llapis: IQ2_S level code %u is not in the codebook\n", code);
                abort();
            }
            const int slot = 2 * b + g;                // 10-bit index: 8 bits in qs, 2 in qh
            out->qs[slot] = (uint8_t)(k & 255);
            out->qh[slot / 4] |= (uint8_t)((k >> 8) << (2 * (slot % 4)));
            out->qs[32 + slot] = signs[g];
        }
        steps[b] = step;
        top = std::max(top, step);
    }
    if (!top) return;
    // block steps as 4-bit odd multiples (2 l + 1) of half the super-block step
    const float unit = top / 31;
    out->d = float_to_half(unit * 0.9875f);
    const float inv = 1 / unit;
    for (int b = 0; b < 16; ++b) {
        const int l = clampi(rne(0.5f * (inv * steps[b] - 1)), 0, 15);
        out->scales[b / 2] |= (uint8_t)(l << (4 * (b % 2)));
    }
}

// ------------------------------------------------------------- driver

void quantize_row(int type, const float * x, uint8_t * dst, int64_t n, const float * imatrix) {
    const int per = blk_elems(type), bytes = blk_bytes(type);
    for (int64_t b = 0; b < n / per; ++b) {
        const float * xb = x + b * per;
        uint8_t * yb = dst + b * bytes;
        const float * im = imatrix ? imatrix + b * per : nullptr;
        switch (type) {
            case T_Q4_K: q4k_super_block(xb, (blk_q4_K *)yb); break;
            case T_Q5_0: q50_block(xb, (blk_q5_0 *)yb); break;
            case T_IQ4_NL: iq4nl_block(xb, (blk_iq4_nl *)yb, im); break;
            case T_IQ2_S: iq2s_super_block(xb, (blk_iq2_s *)yb, im); break;
            default: abort();
        }
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
    if (type == T_IQ2_S) (void)codebook();   // build once, before the workers start
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
