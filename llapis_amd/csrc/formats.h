// formats.h -- ggml block formats used on the MoE expert path, shared by the
// host quantisers and the gfx950 kernels.
//
// Layouts are ggml's (third_party/llama/ggml/src/ggml-common.h): the expert
// pools hold bytes exactly as a GGUF file or ggml_quantize_chunk produces
// them, so a pool written by the reference is read here unchanged.
#pragma once

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define LL_HD __host__ __device__
#else
#define LL_HD
#endif

namespace llapis {

// ggml type tags (ggml/include/ggml.h:390-412)
enum : int32_t {
    T_F32 = 0, T_Q5_0 = 6, T_Q8_0 = 8, T_Q8_1 = 9, T_Q4_K = 12, T_Q8_K = 15,
    T_IQ4_NL = 20, T_IQ2_S = 22,
};

constexpr int QK_K = 256;

struct blk_q4_K  { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; };          // ggml-common.h:317-327
struct blk_iq2_s { uint16_t d; uint8_t qs[64]; uint8_t qh[8]; uint8_t scales[8]; };    // :386-391
struct blk_q5_0  { uint16_t d; uint8_t qh[4]; uint8_t qs[16]; };                       // :219-224
struct blk_iq4_nl{ uint16_t d; uint8_t qs[16]; };                                      // :437-441
struct blk_q8_K  { float d; int8_t qs[QK_K]; int16_t bsums[16]; };                     // :361-365
struct blk_q8_0  { uint16_t d; int8_t qs[32]; };                                       // :241-245
struct blk_q8_1  { uint16_t d, s; int8_t qs[32]; };                                    // :248-258

static_assert(sizeof(blk_q4_K) == 144, "q4_K");
static_assert(sizeof(blk_iq2_s) == 82, "iq2_s");
static_assert(sizeof(blk_q5_0) == 22, "q5_0");
static_assert(sizeof(blk_iq4_nl) == 18, "iq4_nl");
static_assert(sizeof(blk_q8_K) == 292, "q8_K");

// values per block and bytes per block
LL_HD constexpr int blk_elems(int t) {
    return (t == T_Q4_K || t == T_IQ2_S || t == T_Q8_K) ? QK_K : (t == T_F32 ? 1 : 32);
}
LL_HD constexpr int blk_bytes(int t) {
    return t == T_Q4_K ? 144 : t == T_IQ2_S ? 82 : t == T_Q5_0 ? 22 : t == T_IQ4_NL ? 18 :
           t == T_Q8_K ? 292 : t == T_Q8_0 ? 34 : t == T_Q8_1 ? 36 : t == T_F32 ? 4 : 0;
}
inline uint64_t row_bytes(int t, int64_t n) { return (uint64_t)(n / blk_elems(t)) * blk_bytes(t); }

// IQ4_NL non-linear levels (ggml-common.h:1110)
#define LLAPIS_IQ4NL_VALUES {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113}

// IEEE half <-> float, round to nearest even.
LL_HD inline float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1f, man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) { bits = sign; }
        else {
            float f = (float)man * 5.9604644775390625e-8f;
            memcpy(&bits, &f, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112) << 23) | (man << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

LL_HD inline uint16_t float_to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) {
        float a;
        memcpy(&a, &ax, 4);
        const float q = a * 16777216.0f;
        // round half to even on a value < 2^10
        float r = (float)(int)q;
        const float diff = q - r;
        if (diff > 0.5f || (diff == 0.5f && ((int)r & 1))) r += 1.0f;
        return (uint16_t)(sign | (uint32_t)r);
    }
    const uint32_t e = ((ax >> 23) - 112) << 10, m = (ax >> 13) & 0x3ff, rest = ax & 0x1fff;
    uint32_t h = e | m;
    if (rest > 0x1000u || (rest == 0x1000u && (m & 1))) h += 1;
    return (uint16_t)(sign | h);
}

}  // namespace llapis
