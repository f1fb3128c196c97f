// device.h -- device-side building blocks shared by the gfx950 kernels:
// LDS addressing, activation quantisation into LDS, and the per-unit integer
// dot products of the four weight formats against q8 activations.
#pragma once

#include <hip/hip_runtime.h>

#include "formats.h"

namespace llapis {
namespace dev {

constexpr int WG = 256;         // threads per workgroup (4 wave64)

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));   // one 128-bit load/store
constexpr int MAX_D_IN = 8192;  // longest activation column a workgroup quantises

// Activation modes (llapis_moe.h LLAPIS_ACT_*) and activation sources.  The
// _COH sources read their input with device-coherent loads (data written by
// other workgroups of the same kernel).
enum { AM_CPU = 0, AM_Q8_1 = 1 };
enum { SRC_PLAIN = 0, SRC_GEGLU_TABLE = 1, SRC_GEGLU_TANH = 2, SRC_GEGLU_TABLE_COH = 3, SRC_GEGLU_TANH_COH = 4 };

// --------------------------------------------------------------- LDS views

// Byte offsets of one quantised activation column (relative to some base):
// int8 values, per-32 scale and sum, per-256 scale, per-16 block sums.  The
// same layout is used in LDS and for columns stored in global memory.
struct ActView {
    int q, d32, s32, dK, bsum;
};

LL_HD inline int align16i(int x) { return (x + 15) & ~15; }

// layout of an n-value column placed at byte offset `at`; returns its size
// Byte position of activation value x in the int8 region: 16 bytes of
// padding after every 256 values.  A lane reading the 64-value unit u of a
// 256-block starts at 64u + 16(u/4), so the 16 lanes of a row that read units
// 0..15 hit 16 different bank groups (without the padding lanes 0, 4, 8, 12
// would all start in bank 0).
LL_HD constexpr int qpos(int x) { return x + ((x >> 8) << 4); }

LL_HD inline int act_layout(int n, int at, ActView * v) {
    v->q = at;
    v->d32 = align16i(at + qpos(n));
    v->s32 = v->d32 + (n / 32) * 4;
    v->dK = align16i(v->s32 + (n / 32) * 4);
    v->bsum = align16i(v->dK + (n / 256 + 1) * 4);
    return align16i(v->bsum + (n / 16) * 4 + 16) - at;
}

// Byte offsets inside the dynamic LDS block of one workgroup.
struct LdsLayout {
    int w;        // staged weight bytes (16-aligned)
    int q;        // int8 activation values, d_in bytes
    int d32;      // float per 32 values (q8_0 / q8_1 scale)
    int s32;      // float per 32 values (q8_1 sum)
    int dK;       // float per 256 values (q8_K scale)
    int bsum;     // int per 16 values (q8_K block sums)
    int grid;     // IQ2_S codebook, 1024 x uint2
    int total;
};

LL_HD inline int align16(int x) { return (x + 15) & ~15; }

// The gate_up fire's lanes per row: the largest divisor of the row's
// 64-value units (d_in / 64) up to 16, so that every lane takes as many
// units (11 lanes of 4 units at d_in 2816); its rows per workgroup: as many
// as fit WG lanes (23).
LL_HD inline int fire_gu_lanes(int d_in) {
    const int u = d_in / 64;
    int l = 16;
    while (l > 1 && u % l) --l;
    return l;
}
LL_HD inline int fire_gu_rows(int d_in) { return WG / fire_gu_lanes(d_in); }

LL_HD inline LdsLayout lds_layout(int w_bytes, int d_in, bool iq2_tables) {
    LdsLayout L;
    L.w = 0;
    L.q = align16(w_bytes + 16);            // +16: funnel reads may touch one dword past the end
    L.d32 = align16(L.q + qpos(d_in) + 16);
    L.s32 = align16(L.d32 + (d_in / 32) * 4);
    L.dK = align16(L.s32 + (d_in / 32) * 4);
    L.bsum = align16(L.dK + (d_in / 256 + 1) * 4);
    L.grid = align16(L.bsum + (d_in / 16) * 4);
    L.total = L.grid + (iq2_tables ? 1024 * 8 : 0);   // the IQ2_S codebook
    return L;
}

#if defined(__HIPCC__)

// a dword at an even (2-aligned) byte offset
__device__ __forceinline__ uint32_t lds32u(const uint8_t * smem, int off) {
    const int a = off & ~3;
    const uint32_t lo = *reinterpret_cast<const uint32_t *>(smem + a);
    const uint32_t hi = *reinterpret_cast<const uint32_t *>(smem + a + 4);
    return __builtin_amdgcn_alignbit(hi, lo, (off & 3) * 8);
}

__device__ __forceinline__ float h2f(uint32_t h16) {
    const uint16_t h = (uint16_t)h16;
    _Float16 f;
    __builtin_memcpy(&f, &h, 2);
    return (float)f;
}
__device__ __forceinline__ float round_to_half(float x) { return (float)(_Float16)x; }

__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

__device__ __forceinline__ uint32_t byte_of(uint32_t w0, uint32_t w1, int i) {   // byte i (0..7) of w1:w0
    const uint32_t w = i < 4 ? w0 : w1;
    return (w >> ((i & 3) * 8)) & 0xFF;
}

// ----------------------------------------------------- GELU (exact tanh)

__device__ __forceinline__ float gelu_tanh(float x) {
    const float GELU_COEF_A = 0.044715f;
    const float SQRT_2_OVER_PI = 0.79788456080286535587989211986876f;
    return 0.5f * x * (1.0f + tanhf(SQRT_2_OVER_PI * x * (1.0f + GELU_COEF_A * x * x)));
}

// The CPU path's fp16 GELU table, generated at build time by
// gen_gelu_table.c with the host's float arithmetic and tanhf.
#include "gelu_table.inc"

// GEGLU of one element in a given mode.  Table mode is the CPU's fp16
// lookup (vec.h:1414-1428): the table entry at fp16(g) (round to nearest
// even), clamped to 0 below -10 and to the identity above 10.
template <int SRC>
__device__ __forceinline__ float geglu1(float g, float u) {
    if (SRC == SRC_GEGLU_TANH || SRC == SRC_GEGLU_TANH_COH) return __fmul_rn(gelu_tanh(g), u);
    if (g <= -10.0f) return 0.0f;
    if (g >= 10.0f) return __fmul_rn(g, u);
    const uint32_t h = __builtin_bit_cast(uint16_t, (_Float16)g);
    const uint32_t mag = min(h & 0x7FFFu, (uint32_t)LLAPIS_GELU_TAB_SPAN - 1u);    // |g| < 10: mag <= 0x4900
    const uint16_t y = gelu_f16_table[mag + (h >> 15) * LLAPIS_GELU_TAB_SPAN];
    return __fmul_rn((float)__builtin_bit_cast(_Float16, y), u);
}

// GEGLU in two parts, for a gate value known before its up value: the
// factor f of g (the table entry, g itself at or above 10, NaN for the zero
// below -10) and then the product; geglu_apply(geglu_factor(g), u) ==
// geglu1(g, u) bit for bit
template <int SRC>
__device__ __forceinline__ float geglu_factor(float g) {
    if (SRC == SRC_GEGLU_TANH || SRC == SRC_GEGLU_TANH_COH) return gelu_tanh(g);
    if (g <= -10.0f) return __builtin_nanf("");
    if (g >= 10.0f) return g;
    const uint32_t h = __builtin_bit_cast(uint16_t, (_Float16)g);
    const uint32_t mag = min(h & 0x7FFFu, (uint32_t)LLAPIS_GELU_TAB_SPAN - 1u);
    return (float)__builtin_bit_cast(_Float16, gelu_f16_table[mag + (h >> 15) * LLAPIS_GELU_TAB_SPAN]);
}
template <int SRC>
__device__ __forceinline__ float geglu_apply(float f, float u) {
    if (SRC == SRC_GEGLU_TANH || SRC == SRC_GEGLU_TANH_COH) return __fmul_rn(f, u);
    return f != f ? 0.0f : __fmul_rn(f, u);
}

// ----------------------------------------------- wave reductions (wave64)

// DPP lane moves (quad perms, row mirrors, row broadcasts): cross-lane data
// without LDS round trips.  CTRL: 0xB1 quad_perm [1,0,3,2], 0x4E quad_perm
// [2,3,0,1], 0x141 row_half_mirror, 0x140 row_mirror, 0x142 row_bcast15
// (row mask 0xA), 0x143 row_bcast31 (row mask 0xC).
template <int CTRL, int ROWMASK = 0xF>
__device__ __forceinline__ int dpp_i(int old, int v) {
    return __builtin_amdgcn_update_dpp(old, v, CTRL, ROWMASK, 0xF, false);
}
template <int CTRL, int ROWMASK = 0xF>
__device__ __forceinline__ float dpp_f(float old, float v) {
    return __int_as_float(dpp_i<CTRL, ROWMASK>(__float_as_int(old), __float_as_int(v)));
}
template <int CTRL, int ROWMASK = 0xF>
__device__ __forceinline__ double dpp_d(double old, double v) {
    const long long o = __double_as_longlong(old), x = __double_as_longlong(v);
    const int lo = dpp_i<CTRL, ROWMASK>((int)o, (int)x);
    const int hi = dpp_i<CTRL, ROWMASK>((int)(o >> 32), (int)(x >> 32));
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}
// wave64 reductions; the result is read from lane 63 and is wave-uniform
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v, v));
    v = fmaxf(v, dpp_f<0x4E>(v, v));
    v = fmaxf(v, dpp_f<0x141>(v, v));
    v = fmaxf(v, dpp_f<0x140>(v, v));
    v = fmaxf(v, dpp_f<0x142, 0xA>(v, v));
    v = fmaxf(v, dpp_f<0x143, 0xC>(v, v));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// max over each half-wave (lanes 0-31, 32-63), in every lane of the half
__device__ __forceinline__ float half_max_dpp(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v, v));
    v = fmaxf(v, dpp_f<0x4E>(v, v));
    v = fmaxf(v, dpp_f<0x141>(v, v));
    v = fmaxf(v, dpp_f<0x140>(v, v));           // row (16-lane) max in every lane
    const int b = __float_as_int(v);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(b, 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(b, 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(b, 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(b, 48));
    return (threadIdx.x & 32) ? fmaxf(r2, r3) : fmaxf(r0, r1);
}
// integer sum over each 32-lane half of the wave, in every lane of it
__device__ __forceinline__ int half_sum_dpp_i(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false);   // row (16-lane) sum in every lane
    const int r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
    const int r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
    return (threadIdx.x & 32) ? r2 + r3 : r0 + r1;
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += dpp_f<0xB1>(0.0f, v);
    v += dpp_f<0x4E>(0.0f, v);
    v += dpp_f<0x141>(0.0f, v);
    v += dpp_f<0x140>(0.0f, v);
    v += dpp_f<0x142, 0xA>(0.0f, v);
    v += dpp_f<0x143, 0xC>(0.0f, v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ double wave_sum_dpp(double v) {
    v += dpp_d<0xB1>(0.0, v);
    v += dpp_d<0x4E>(0.0, v);
    v += dpp_d<0x141>(0.0, v);
    v += dpp_d<0x140>(0.0, v);
    v += dpp_d<0x142, 0xA>(0.0, v);
    v += dpp_d<0x143, 0xC>(0.0, v);
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)b, 63), hi = __builtin_amdgcn_readlane((int)(b >> 32), 63);
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}
// sum over each row of 16 lanes, in every lane of the row
__device__ __forceinline__ int row16_sum(int v) {
    v += dpp_i<0xB1>(0, v);
    v += dpp_i<0x4E>(0, v);
    v += dpp_i<0x141>(0, v);
    v += dpp_i<0x140>(0, v);
    return v;
}

// ---------------------------------------- activation quantisation into LDS

// Source element k of activation column `col`.
struct ActSrc {
    const float * p;   // SRC_PLAIN: column base; GEGLU: merged gate_up column base
    int n;             // d_in (GEGLU: n_ff; up half starts at p + n)
};

__device__ __forceinline__ float ld_coh_f(const float * p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int SRC>
__device__ __forceinline__ float act_at(const ActSrc & s, int k) {
    if (SRC == SRC_PLAIN) return s.p[k];
    if (SRC == SRC_GEGLU_TABLE_COH || SRC == SRC_GEGLU_TANH_COH)
        return geglu1<SRC>(ld_coh_f(s.p + k), ld_coh_f(s.p + s.n + k));
    return geglu1<SRC>(s.p[k], s.p[s.n + k]);
}

// q8_K of one 256-block b of a column (ggml-quants.c:2696-2733), one wave:
// max is the first element of largest magnitude; iscale = -127/max;
// q = min(127, nearest_int(iscale x)); d = 1/iscale; bsums over 16.
template <int SRC>
__device__ __forceinline__ void q8K_block(uint8_t * base, const ActView & L, const ActSrc & src, int b) {
    const int lane = threadIdx.x & 63;
    int8_t * q = reinterpret_cast<int8_t *>(base + L.q);
    float * dK = reinterpret_cast<float *>(base + L.dK);
    int * bsum = reinterpret_cast<int *>(base + L.bsum);
    float v[4];
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        v[j] = act_at<SRC>(src, b * 256 + lane + 64 * j);
        amax = fmaxf(amax, fabsf(v[j]));
    }
    amax = wave_max_dpp(amax);
    // first position holding |x| == amax: positions are lane + 64 j
    float max = 0.0f;
#pragma unroll
    for (int j = 3; j >= 0; --j) {
        const uint64_t m = __ballot(fabsf(v[j]) == amax);
        if (m) max = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[j]), (int)__builtin_ctzll(m)));
    }
    int qi[4];
    if (amax == 0.0f) {
#pragma unroll
        for (int j = 0; j < 4; ++j) qi[j] = 0;
        if (lane == 0) dK[b] = 0.0f;
    } else {
        const float iscale = -127.f / max;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int r = (int)rintf(__fmul_rn(iscale, v[j]));
            qi[j] = r < 127 ? r : 127;
        }
        if (lane == 0) dK[b] = 1.0f / iscale;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        q[b * 272 + lane + 64 * j] = (int8_t)qi[j];        // qpos(b * 256 + lane + 64 j)
        const int s = row16_sum(qi[j]);
        if ((lane & 15) == 0) bsum[b * 16 + (lane >> 4) + 4 * j] = s;
    }
}

template <int SRC>
__device__ __forceinline__ void quantize_q8_K(uint8_t * base, const ActView & L, const ActSrc & src, int d_in) {
    for (int b = threadIdx.x >> 6; b < d_in / 256; b += WG / 64) q8K_block<SRC>(base, L, src, b);
}

// q8_0 as the x86 CPU build computes it (arch/x86/quants.c:302-360):
// d = amax/127 stored as fp16, id = 127/amax, q = round-to-nearest-even(x id).
// q8_1 as ggml-cuda computes it (quantize.cu:5-50): d = amax/127,
// q = roundf(x/d), s = butterfly sum of x; both stored as fp16.
// One wave quantises the two 32-blocks starting at `at`.
template <int AM>
__device__ __forceinline__ void q8_32_put(uint8_t * base, const ActView & L, float v, int pos, bool live) {
    const int lane = threadIdx.x & 63;
    int8_t * q = reinterpret_cast<int8_t *>(base + L.q);
    float * d32 = reinterpret_cast<float *>(base + L.d32);
    float * s32 = reinterpret_cast<float *>(base + L.s32);
    const float amax = half_max_dpp(fabsf(v));
    int qi;
    float dstore;
    if (AM == AM_CPU) {
        const float d = amax / 127.f;
        const float id = amax != 0.0f ? 127.f / amax : 0.0f;
        qi = (int)rintf(__fmul_rn(v, id));
        qi = qi > 127 ? 127 : (qi < -128 ? -128 : qi);
        dstore = round_to_half(d);
        // the block's sum of q (exact), for the q8_0 dots' - 16 sum a term
        const int qs = half_sum_dpp_i(live ? qi : 0);
        if (live && (lane & 31) == 0) s32[pos >> 5] = (float)qs;
    } else {
        float s = v;
        for (int o = 16; o >= 1; o >>= 1) s = __fadd_rn(s, __shfl_xor(s, o, 32));
        const float d = amax / 127.0f;
        qi = amax == 0.0f ? 0 : (int)roundf(v / d);
        dstore = round_to_half(d);
        if (live && (lane & 31) == 0) s32[pos >> 5] = round_to_half(s);
    }
    if (live) {
        q[qpos(pos)] = (int8_t)qi;
        if ((lane & 31) == 0) d32[pos >> 5] = dstore;
    }
}

// One wave quantises the 64 values at at, at + WG, ... (up to Q8_BATCH
// steps); every source load of the batch is issued before the first value is
// used, so the batch costs one memory round trip.
constexpr int Q8_BATCH = 4;

template <int SRC>
__device__ __forceinline__ float ld_src(const float * p) {
    if (SRC == SRC_GEGLU_TABLE_COH || SRC == SRC_GEGLU_TANH_COH) return ld_coh_f(p);
    return *p;
}

// One batch: the Q8_BATCH steps at0, at0 + WG, ... of one wave.  Loading is
// separate from quantising so a caller can issue the loads early.
struct ActBatch {
    float g[Q8_BATCH], u[Q8_BATCH];
};

template <int SRC>
__device__ __forceinline__ void act_batch_load(ActBatch & b, const ActSrc & src, int d_in, int at0) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < Q8_BATCH; ++j) {
        const int pos = at0 + j * WG + lane;
        const bool live = pos < d_in;             // d_in is a multiple of 32, not always of 64
        b.g[j] = live ? ld_src<SRC>(src.p + pos) : 0.0f;
        b.u[j] = (SRC != SRC_PLAIN && live) ? ld_src<SRC>(src.p + src.n + pos) : 0.0f;
    }
}

template <int SRC, int AM>
__device__ __forceinline__ void act_batch_quant(uint8_t * base, const ActView & L, const ActBatch & b, int d_in,
                                                int at0) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < Q8_BATCH; ++j) {
        const int at = at0 + j * WG;
        if (at >= d_in) break;                    // wave-uniform
        const int pos = at + lane;
        const bool live = pos < d_in;
        const float v = SRC == SRC_PLAIN ? b.g[j] : (live ? geglu1<SRC>(b.g[j], b.u[j]) : 0.0f);
        q8_32_put<AM>(base, L, v, pos, live);
    }
}

template <int SRC, int AM>
__device__ __forceinline__ void quantize_q8_32(uint8_t * base, const ActView & L, const ActSrc & src, int d_in) {
    for (int at0 = (threadIdx.x >> 6) * 64; at0 < d_in; at0 += Q8_BATCH * WG) {
        ActBatch b;
        act_batch_load<SRC>(b, src, d_in, at0);
        act_batch_quant<SRC, AM>(base, L, b, d_in, at0);
    }
}

// Quantise an activation column into the format weight type T is dotted with.
template <int T, int AM, int SRC>
__device__ __forceinline__ void quantize_act(uint8_t * base, const ActView & v, const ActSrc & src, int n) {
    if constexpr (AM == AM_CPU && (T == T_Q4_K || T == T_IQ2_S)) quantize_q8_K<SRC>(base, v, src, n);
    else quantize_q8_32<SRC, AM>(base, v, src, n);
}

// IQ2_S codebook in LDS: for each of the 1024 grid points its eight level
// codes, one byte each (0, 1, 2 stand for the magnitudes 0x08, 0x19, 0x2b of
// iq2s_grid, ggml-common.h:748).  Signs are applied in registers: a byte
// selector code | 4*sign picks the signed magnitude out of the eight bytes
// {8, 25, 43, 0, -8, -25, -43, 0} with one v_perm, so no sign table is read.
// Expanded at compile time; a workgroup copies it into LDS.
struct Iq2sTables {
    uint32_t grid[1024][2];
};
constexpr uint16_t k_iq2s_codes[1024] = {
#include "iq2s_grid.inc"
};
constexpr Iq2sTables make_iq2s_tables() {
    Iq2sTables t{};
    for (int k = 0; k < 1024; ++k) {
        const uint32_t c = k_iq2s_codes[k];
        uint32_t lo = 0, hi = 0;
        for (int i = 0; i < 8; ++i) {
            const uint32_t l = (c >> (2 * i)) & 3;
            if (i < 4) lo |= l << (8 * i); else hi |= l << (8 * (i - 4));
        }
        t.grid[k][0] = lo;
        t.grid[k][1] = hi;
    }
    return t;
}
static_assert(sizeof(Iq2sTables) == 1024 * 8, "table layout");

constexpr uint32_t IQ2S_POS = 0x002B1908u, IQ2S_NEG = 0x00D5E7F8u;   // {8,25,43,0}, {-8,-25,-43,0}

// four signed codebook bytes from four level codes (one per byte) and the
// four matching sign bits (bit i of `nib` for byte i).  nib * 0x810204 (an
// unsigned 24-bit multiply: bit 23 of the constant is set) puts
// bit i at bits 8i+2 (and at 12 other bits, all distinct, so no carries);
// the mask keeps bit 2 of every byte.
__device__ __forceinline__ uint32_t iq2s_signed4(uint32_t codes, uint32_t nib) {
    const uint32_t sel = (__umul24(nib, 0x810204u) & 0x04040404u) | codes;
    return __builtin_amdgcn_perm(IQ2S_NEG, IQ2S_POS, sel);
}

// copy the codebook to smem + grid_off
__device__ __forceinline__ void copy_iq2s_tables(uint8_t * smem, int grid_off, const Iq2sTables * tab) {
    const u32x4 * src = reinterpret_cast<const u32x4 *>(tab);
    u32x4 * dst = reinterpret_cast<u32x4 *>(smem + grid_off);
    for (int i = threadIdx.x; i < (int)(sizeof(Iq2sTables) / 16); i += WG) dst[i] = src[i];
}

// ------------------------------------------------------------ unit dots
//
// A unit is the slice of a weight row one lane handles at a time:
//   Q4_K, IQ2_S: a quarter super-block (64 values, two 32-sub-blocks)
//   Q5_0, IQ4_NL: one 32-block
// Each unit is decoded from LDS once and dotted against up to NC activation
// columns (decode once, dot N: the columns of the tokens that routed to the
// same expert).  `wb` is the LDS byte offset of the row, `u` the unit index,
// av[c] the LDS offsets of column c's quantised activation.

template <int T> struct Fmt;
template <> struct Fmt<T_Q4_K>   { static constexpr int UNIT = 64; static constexpr int LPR = 16; };
template <> struct Fmt<T_IQ2_S>  { static constexpr int UNIT = 64; static constexpr int LPR = 16; };
template <> struct Fmt<T_Q5_0>   { static constexpr int UNIT = 32; static constexpr int LPR = 8; };
template <> struct Fmt<T_IQ4_NL> { static constexpr int UNIT = 32; static constexpr int LPR = 8; };

typedef const void __attribute__((address_space(1))) * gptr_t;
typedef void __attribute__((address_space(3))) * lptr_t;

// 16 (or 4) bytes per lane from global memory into LDS at dst + 16 lane
// (4 lane): the load unit writes LDS itself, tracked by the vector memory
// counter (dst is the wave's base: the same in every lane)
__device__ __forceinline__ void lds_dma16(const void * src, void * dst) {
    __builtin_amdgcn_global_load_lds((gptr_t)src, (lptr_t)dst, 16, 0, 0);
}
__device__ __forceinline__ void lds_dma4(const void * src, void * dst) {
    __builtin_amdgcn_global_load_lds((gptr_t)src, (lptr_t)dst, 4, 0, 0);
}

__device__ __forceinline__ u32x4 lds128(const uint8_t * smem, int off) {   // off % 16 == 0
    return *reinterpret_cast<const u32x4 *>(smem + off);
}

// Q4_K . q8_K   (ggml-cpu/quants.c:645-718): per super-block
//   d_w dK sum_j sc_j dot_j  -  dmin_w dK sum_j m_j (bsum_2j + bsum_2j+1)
// Q4_K . q8_1   (ggml-cuda/vecdotq.cuh:505-528): per 32-block b
//   d_w d8_b sc_b dot_b  -  dmin_w d8_b m_b sum(q8_b)
template <int AM, int NC>
__device__ __forceinline__ void q4k_unit(const uint8_t * smem, int wb, int u, const ActView * av, int nc,
                                         float * acc) {
    const int sb = u >> 2, qq = u & 3;
    const int blk = wb + sb * 144;                        // 16-aligned
    const u32x4 hdr = lds128(smem, blk);
    const u32x4 qa = lds128(smem, blk + 16 + 32 * qq);
    const u32x4 qb = lds128(smem, blk + 32 + 32 * qq);
    // 6-bit scales/mins of sub-blocks j0 = 2qq, j1 = 2qq + 1 (get_scale_min_k4)
    const uint32_t s03 = hdr.y, s47 = hdr.z, s8b = hdr.w;
    int sc0, m0, sc1, m1;
    if (qq < 2) {
        const int sh0 = 16 * qq, sh1 = 16 * qq + 8;
        sc0 = (s03 >> sh0) & 63; m0 = (s47 >> sh0) & 63;
        sc1 = (s03 >> sh1) & 63; m1 = (s47 >> sh1) & 63;
    } else {
        const int sh0 = 16 * (qq - 2), sh1 = sh0 + 8;     // j-4 in 0..3
        sc0 = ((s8b >> sh0) & 0xF) | (((s03 >> sh0) >> 6 & 3) << 4);
        m0  = ((s8b >> sh0) >> 4 & 0xF) | (((s47 >> sh0) >> 6 & 3) << 4);
        sc1 = ((s8b >> sh1) & 0xF) | (((s03 >> sh1) >> 6 & 3) << 4);
        m1  = ((s8b >> sh1) >> 4 & 0xF) | (((s47 >> sh1) >> 6 & 3) << 4);
    }
    const float d = h2f(hdr.x & 0xFFFF), dmin = h2f(hdr.x >> 16);
    // the integer sums below are formed in fp32: every product and partial
    // sum is an integer below 2^24, so exact (and fp32 multiplies are full
    // rate, where 32-bit integer ones are not)
    const float fsc0 = (float)sc0, fsc1 = (float)sc1, fm0 = (float)m0, fm1 = (float)m1;
    const uint32_t w[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        lo[i] = w[i] & 0x0F0F0F0Fu;
        hi[i] = (w[i] >> 4) & 0x0F0F0F0Fu;
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        if (c >= nc) break;
        const int ao = av[c].q + sb * 272 + 64 * qq;         // qpos(64 u)
        const u32x4 a0 = lds128(smem, ao), a1 = lds128(smem, ao + 16);
        const u32x4 a2 = lds128(smem, ao + 32), a3 = lds128(smem, ao + 48);
        const uint32_t alo[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        const uint32_t ahi[8] = {a2.x, a2.y, a2.z, a2.w, a3.x, a3.y, a3.z, a3.w};
        int dot1 = 0, dot2 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            dot1 = dot4((int)lo[i], (int)alo[i], dot1);
            dot2 = dot4((int)hi[i], (int)ahi[i], dot2);
        }
        if (AM == AM_CPU) {
            const float dK = reinterpret_cast<const float *>(smem + av[c].dK)[sb];
            const int * bs = reinterpret_cast<const int *>(smem + av[c].bsum) + sb * 16 + 4 * qq;
            // |dot| <= 32 * 15 * 128, sc and m <= 63, |bs| <= 16 * 128
            const float sumi = __fmaf_rn(fsc0, (float)dot1, __fmul_rn(fsc1, (float)dot2));
            const float summ = __fmaf_rn(fm0, (float)(bs[0] + bs[1]), __fmul_rn(fm1, (float)(bs[2] + bs[3])));
            acc[c] += __fmul_rn(d * dK, sumi) - __fmul_rn(dmin * dK, summ);
        } else {
            int sq0 = 0, sq1 = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                sq0 = dot4(0x01010101, (int)alo[i], sq0);
                sq1 = dot4(0x01010101, (int)ahi[i], sq1);
            }
            const float * d32 = reinterpret_cast<const float *>(smem + av[c].d32) + (sb * 256 + 64 * qq) / 32;
            const float sd = d32[0] * __fmul_rn((float)dot1, fsc0) + d32[1] * __fmul_rn((float)dot2, fsc1);
            const float sm = d32[0] * __fmul_rn((float)sq0, fm0) + d32[1] * __fmul_rn((float)sq1, fm1);
            acc[c] += d * sd - dmin * sm;
        }
    }
}

// IQ2_S . q8_K  (ggml-cpu/quants.c:947-997): per super-block
//   0.125 d_w dK sum_ib [(2 sc_lo + 1) s_1 + (2 sc_hi + 1) s_2]
// IQ2_S . q8_1  (ggml-cuda/vecdotq.cuh:1061-1105): per 32-block
//   d_w d8 ((s_1 sc_lo + s_2 sc_hi + (s_1 + s_2)/2) / 4)   (C integer division)
// The codebook is in LDS at `grid_off`; signs are applied with iq2s_signed4.
template <int AM, int NC>
__device__ __forceinline__ void iq2s_unit(const uint8_t * smem, int wb, int u, const ActView * av, int nc,
                                          float * acc, int grid_off) {
    const int sb = u >> 2, qq = u & 3;
    const int blk = wb + sb * 82;                         // 2-aligned
    const float d = h2f(lds32u(smem, blk));
    const uint32_t qs0 = lds32u(smem, blk + 2 + 8 * qq), qs1 = lds32u(smem, blk + 6 + 8 * qq);
    const uint32_t sg0 = lds32u(smem, blk + 34 + 8 * qq), sg1 = lds32u(smem, blk + 38 + 8 * qq);
    const uint32_t qh2 = lds32u(smem, blk + 66 + 2 * qq);
    const uint32_t sc2 = lds32u(smem, blk + 74 + 2 * qq);
    const uint2 * grid = reinterpret_cast<const uint2 *>(smem + grid_off);
    // signed codebook bytes of the unit's 8 groups of 8
    uint32_t g0[8], g1[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        const uint32_t qhb = (qh2 >> (8 * (g >> 2))) & 0xFF;
        const uint32_t idx = byte_of(qs0, qs1, g) | (((qhb >> (2 * (g & 3))) & 3) << 8);
        const uint2 gv = grid[idx];
        const uint32_t sw = (g < 4 ? sg0 : sg1) >> (8 * (g & 3));
        g0[g] = iq2s_signed4(gv.x, sw & 15);
        g1[g] = iq2s_signed4(gv.y, (sw >> 4) & 15);
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        if (c >= nc) break;
        const int ao = av[c].q + sb * 272 + 64 * qq;         // qpos(64 u)
        float bsum = 0.0f;          // an integer below 2^24 (|s| <= 16 * 43 * 128, scales <= 31): exact in fp32
        float accf = 0.0f;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t scb = (sc2 >> (8 * h)) & 0xFF;
            int s[2] = {0, 0};
#pragma unroll
            for (int l = 0; l < 4; ++l) {
                const int g = 4 * h + l;
                const uint2 a = *reinterpret_cast<const uint2 *>(smem + ao + 32 * h + 8 * l);
                s[l >> 1] = dot4((int)g0[g], (int)a.x, s[l >> 1]);
                s[l >> 1] = dot4((int)g1[g], (int)a.y, s[l >> 1]);
            }
            if (AM == AM_CPU) {
                bsum = __fadd_rn(bsum, __fmaf_rn((float)(2 * (int)(scb & 15) + 1), (float)s[0],
                                                 __fmul_rn((float)(2 * (int)(scb >> 4) + 1), (float)s[1])));
            } else {
                const int sumi = (__mul24(s[0], (int)(scb & 15)) + __mul24(s[1], (int)(scb >> 4)) + (s[0] + s[1]) / 2) / 4;
                const float d8 = reinterpret_cast<const float *>(smem + av[c].d32)[(sb * 256 + 64 * qq + 32 * h) / 32];
                accf += (d * d8) * (float)sumi;
            }
        }
        if (AM == AM_CPU) {
            const float dK = reinterpret_cast<const float *>(smem + av[c].dK)[sb];
            acc[c] += 0.125f * __fmul_rn(d * dK, bsum);
        } else {
            acc[c] += accf;
        }
    }
}

// Q5_0 . q8_0  (ggml-cpu/quants.c:314-352):  d_w d8 sum (q - 16) a
// Q5_0 . q8_1  (ggml-cuda/vecdotq.cuh:172-198): d_w (d8 sum q a - 16 s8)
template <int AM, int NC>
__device__ __forceinline__ void q5_0_unit(const uint8_t * smem, int wb, int u, const ActView * av, int nc,
                                          float * acc) {
    const int blk = wb + u * 22;                          // 2-aligned
    const float d = h2f(lds32u(smem, blk));
    const uint32_t qh = lds32u(smem, blk + 2);
    uint32_t v0[4], v1[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t qsw = lds32u(smem, blk + 6 + 4 * i);
        const uint32_t vh0 = qh >> (4 * i), vh1 = qh >> (16 + 4 * i);
        uint32_t a = qsw & 0x0F0F0F0Fu;
        a |= (vh0 << 4) & 0x10u; a |= (vh0 << 11) & 0x1000u; a |= (vh0 << 18) & 0x100000u; a |= (vh0 << 25) & 0x10000000u;
        uint32_t b = (qsw >> 4) & 0x0F0F0F0Fu;
        b |= (vh1 << 4) & 0x10u; b |= (vh1 << 11) & 0x1000u; b |= (vh1 << 18) & 0x100000u; b |= (vh1 << 25) & 0x10000000u;
        v0[i] = a;
        v1[i] = b;
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        if (c >= nc) break;
        const int ao = av[c].q + qpos(u * 32);
        const u32x4 a0 = lds128(smem, ao), a1 = lds128(smem, ao + 16);
        const uint32_t alo[4] = {a0.x, a0.y, a0.z, a0.w}, ahi[4] = {a1.x, a1.y, a1.z, a1.w};
        int sumi = 0, suma = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sumi = dot4((int)v0[i], (int)alo[i], sumi);
            sumi = dot4((int)v1[i], (int)ahi[i], sumi);
            if (AM == AM_CPU) {
                suma = dot4(0x01010101, (int)alo[i], suma);
                suma = dot4(0x01010101, (int)ahi[i], suma);
            }
        }
        const float d8 = reinterpret_cast<const float *>(smem + av[c].d32)[u];
        if (AM == AM_CPU) {
            acc[c] += __fmul_rn(d * d8, (float)(sumi - 16 * suma));
        } else {
            const float s8 = reinterpret_cast<const float *>(smem + av[c].s32)[u];
            acc[c] += d * ((float)sumi * d8 - 16.0f * s8);
        }
    }
}

// 16-entry signed-byte table lookup of four nibble indices (one per byte).
__device__ __forceinline__ uint32_t iq4nl_lookup(uint32_t idx) {
    // kvalues_iq4nl (ggml-common.h:1110) as little-endian bytes
    const uint32_t t0 = 0xBFAD9881u, t1 = 0xF6EADDCFu, t2 = 0x26190D01u, t3 = 0x71594535u;
    const uint32_t sel = idx & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(t1, t0, sel);
    const uint32_t hi = __builtin_amdgcn_perm(t3, t2, sel);
    // byte mask 0xFF where bit 3 is set: perm selector 12 gives 0x00, 13 gives 0xFF
    const uint32_t m = __builtin_amdgcn_perm(0u, 0u, ((idx >> 3) & 0x01010101u) | 0x0C0C0C0Cu);
    return (hi & m) | (lo & ~m);
}

// IQ4_NL . q8_0 (ggml-cpu/quants.c:1203-1228) and . q8_1 (vecdotq.cuh:1270-1289):
//   d_w d8 sum kvalues[q] a
template <int AM, int NC>
__device__ __forceinline__ void iq4nl_unit(const uint8_t * smem, int wb, int u, const ActView * av, int nc,
                                           float * acc) {
    const int blk = wb + u * 18;                          // 2-aligned
    const float d = h2f(lds32u(smem, blk));
    uint32_t v0[4], v1[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t qsw = lds32u(smem, blk + 2 + 4 * i);
        v0[i] = iq4nl_lookup(qsw & 0x0F0F0F0Fu);
        v1[i] = iq4nl_lookup((qsw >> 4) & 0x0F0F0F0Fu);
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        if (c >= nc) break;
        const int ao = av[c].q + qpos(u * 32);
        const u32x4 a0 = lds128(smem, ao), a1 = lds128(smem, ao + 16);
        const uint32_t alo[4] = {a0.x, a0.y, a0.z, a0.w}, ahi[4] = {a1.x, a1.y, a1.z, a1.w};
        int sumi = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sumi = dot4((int)v0[i], (int)alo[i], sumi);
            sumi = dot4((int)v1[i], (int)ahi[i], sumi);
        }
        const float d8 = reinterpret_cast<const float *>(smem + av[c].d32)[u];
        if (AM == AM_CPU) acc[c] += __fmul_rn(d8 * d, (float)sumi);
        else acc[c] += (d * d8) * (float)sumi;
    }
}

template <int T, int AM, int NC>
__device__ __forceinline__ void unit_dot_n(const uint8_t * smem, int wb, int u, const ActView * av, int nc,
                                           float * acc, int grid_off) {
    if constexpr (T == T_Q4_K) q4k_unit<AM, NC>(smem, wb, u, av, nc, acc);
    else if constexpr (T == T_IQ2_S) iq2s_unit<AM, NC>(smem, wb, u, av, nc, acc, grid_off);
    else if constexpr (T == T_Q5_0) q5_0_unit<AM, NC>(smem, wb, u, av, nc, acc);
    else iq4nl_unit<AM, NC>(smem, wb, u, av, nc, acc);
}

#endif  // __HIPCC__

}  // namespace dev
}  // namespace llapis
