// prefill.hip -- the MoE layer for long token batches (prefill chunks) on
// gfx950 matrix cores.
//
//   k_pf_bucket    routed pairs grouped by expert (a counting sort with LDS
//                  atomics) and cut into tiles of <= PF_TOK pairs,
//                  each tile tagged with its tier by the residency predicate
//                  (ggml-cuda/mmid.cu:28-116 groups the same way; moert/cuda/
//                  ffn_moe.cu:80-130 is the predicate).
//   k_pf_quant_x   each token quantised once to q8_K (the CPU path's
//                  activation format for 256-blocks) and stored as exact fp16
//                  integers (converted once, not per GEMM workgroup), with the
//                  per-256 scale and the per-32 sums split into fp16-exact
//                  high and low parts.
//   k_pf_gate_up   grouped GEMM per (tile, 128-row block): weights staged raw
//                  in LDS one super-block at a time and expanded in registers
//                  to fp16 integers (Q4_K: q*sc <= 945; IQ2_S: grid*(2ls+1)
//                  <= 1333, both exact in fp16), activations exact, so one
//                  v_mfma_f32_32x32x16_f16 chain per super-block gives the
//                  integer dot exactly; the Q4_K mins term is one more exact
//                  MFMA.  Scales are applied once per super-block in fp32.
//   k_pf_act       GEGLU and q8_0 quantisation of each pair's gate_up output
//                  (bit-identical to the CPU path); d8*q (19 significant bits)
//                  with a per-pair power-of-two range scale is stored as the
//                  exact sum of two fp16 parts, ready for the MFMA operands.
//   k_pf_down      grouped GEMM of the down projection.  Its scales are per
//                  32-value block, so they are folded into the operands
//                  instead of rescaling every output per block: d*q of the
//                  weights also splits exactly into fp16 hi + lo, and three
//                  MFMAs per step (hi*hi, hi*lo, lo*hi) give the dot to about
//                  2^-21 relative.
// The combine is the generic k_combine.
#include <hip/hip_ext.h>

#include <type_traits>

#include "device.h"
#include "launch.h"

namespace llapis {
namespace dev {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));

__constant__ uint16_t c_iq2s_codes_pf[1024] = {
#include "iq2s_grid.inc"
};

constexpr int PF_XS = 256 + 8;            // halfs per staged activation row of gate_up (padded)
constexpr int PF_DCB = 4;                 // 32-blocks per down K chunk
constexpr int PF_DXS = PF_DCB * 32 + 8;   // halfs per staged activation row of down (padded)
constexpr int PF_WROW_GU = 144;           // LDS bytes per weight row and super-block (Q4_K 144, IQ2_S <= 96)
constexpr int PF_WROW_DN = 112;           // staged bytes per weight row and down chunk (<= 4 * 22 + 14)
constexpr int PF_WPITCH_DN = 120;         // LDS pitch of those rows: 30 dwords, so the 32 rows a half-wave
                                          // reads at one offset fall in 32 different bank pairs

__device__ __forceinline__ uint32_t hbits(h2 v) {
    uint32_t u;
    __builtin_memcpy(&u, &v, 4);
    return u;
}
__device__ __forceinline__ h2 as_h2(uint32_t u) {
    h2 v;
    __builtin_memcpy(&v, &u, 4);
    return v;
}
__device__ __forceinline__ h8 as_h8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const u32x4 u = {a, b, c, d};
    h8 v;
    __builtin_memcpy(&v, &u, 16);
    return v;
}
__device__ __forceinline__ h2 splat(_Float16 x) { return h2{x, x}; }

// four unsigned bytes -> two packed fp16 pairs of (1024 + byte)
__device__ __forceinline__ void bytes_to_magic(uint32_t x, uint32_t & lo, uint32_t & hi) {
    lo = __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u);
    hi = __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u);
}

// 16 signed bytes -> 16 exact fp16 values (8 packed dwords)
__device__ __forceinline__ void i8x16_to_h(const u32x4 & v, uint32_t (&o)[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    const h2 off = splat((_Float16)(-1152.0f));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t a, b;
        bytes_to_magic(w[i] ^ 0x80808080u, a, b);      // 1024 + (v + 128)
        o[2 * i] = hbits(as_h2(a) + off);
        o[2 * i + 1] = hbits(as_h2(b) + off);
    }
}

__device__ __forceinline__ bool tile_valid(const PfParams & p, const PfTile & t) {
    return (t.tier == 0 && t.idx >= 0 && t.idx < p.k_slots) || (t.tier == 1 && t.idx >= 0 && t.idx < p.n_expert);
}

// ----------------------------------------------------------------- bucket

// One workgroup.  P = T * top_k <= PF_MAX_PAIRS, n_expert <= 256.  A
// counting sort by expert with LDS atomics: counts, an exclusive scan over
// the experts (pair offsets and tile offsets), then each pair takes the next
// slot of its expert.  The order of pairs inside an expert's range is not
// fixed, and need not be: each pair's output column is computed on its own.
__global__ __launch_bounds__(WG) void k_pf_bucket(const PfParams p) {
    constexpr int PER = PF_MAX_PAIRS / WG;
    __shared__ int s_cnt[257], s_fill[257], s_off[257], s_nt[257], s_hot;
    const int P = p.T * p.top_k, E = p.n_expert;
    // the ids, read once with every load in flight together
    int ev[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int q = threadIdx.x + WG * k;
        const int v = q < P ? p.ids[q] : -1;
        ev[k] = (v >= 0 && v < E) ? v : 256;     // 256: invalid id
    }
    for (int i = threadIdx.x; i < 257; i += WG) {
        s_cnt[i] = 0;
        s_fill[i] = 0;
    }
    if (threadIdx.x == 0) s_hot = 0;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < PER; ++k)
        if (threadIdx.x + WG * k < P) atomicAdd(&s_cnt[ev[k]], 1);
    __syncthreads();
    // per expert (one thread each): tier, pair offset and tile offset by
    // exclusive scans over the experts
    const int e0 = threadIdx.x;
    int n_e = 0, tier = 1, idx = e0;
    if (e0 < E) {
        n_e = s_cnt[e0];
        if (p.k_slots > 0) {
            const int sl = p.exp_slot[e0];
            if (sl >= 0 && sl < p.k_slots && p.slot_state[sl] == 2 && p.slot_exp[sl] == e0) {
                tier = 0;
                idx = sl;
            }
        }
    }
    const int nt_e = (n_e + PF_TOK - 1) / PF_TOK;
    if (p.rc_counts) {
        // routing counters (ffn_moe.cu:123-128): pairs per expert, hot pairs,
        // the other pairs (invalid ids included)
        if (n_e) atomicAdd(p.rc_counts + e0, n_e);
        const int hot = tier == 0 ? n_e : 0;
        if (hot) atomicAdd(&s_hot, hot);
    }
    s_off[threadIdx.x] = n_e;
    s_nt[threadIdx.x] = nt_e;
    __syncthreads();
    // inclusive scans (Hillis-Steele over 256 entries)
    for (int o = 1; o < 256; o <<= 1) {
        const int a = threadIdx.x >= o ? s_off[threadIdx.x - o] : 0;
        const int b = threadIdx.x >= o ? s_nt[threadIdx.x - o] : 0;
        __syncthreads();
        s_off[threadIdx.x] += a;
        s_nt[threadIdx.x] += b;
        __syncthreads();
    }
    const int pair0 = s_off[threadIdx.x] - n_e, tile0 = s_nt[threadIdx.x] - nt_e;
    const int total = s_off[255], tiles = min(s_nt[255], p.max_tiles);
    if (p.rc_hits && threadIdx.x == 0) {
        atomicAdd(p.rc_hits, s_hot);
        atomicAdd(p.rc_hits + 1, P - s_hot);
    }
    __syncthreads();
    s_off[threadIdx.x] = pair0;                 // exclusive offsets
    if (threadIdx.x == 0) {
        s_off[256] = total;                     // invalid ids are placed after every expert's pairs
        *p.n_tiles = tiles;
    }
    for (int b = 0; b < nt_e; ++b) {
        if (tile0 + b >= p.max_tiles) break;
        PfTile t;
        t.tier = tier;
        t.idx = idx;
        t.begin = pair0 + b * PF_TOK;
        t.n = min(PF_TOK, n_e - b * PF_TOK);
        p.tiles[tile0 + b] = t;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int q = threadIdx.x + WG * k;
        if (q < P) p.sorted[s_off[ev[k]] + atomicAdd(&s_fill[ev[k]], 1)] = q;
    }
}

// ------------------------------------------------------------ token quant

// One wave per (token, 256-block): q8_K exactly as the CPU path; the int8
// values, the scale, and the 8 per-32 sums as {hi_0..hi_7, lo_0..lo_7} with
// sum = 32 hi + lo, 0 <= lo < 32 (each part exact in fp16).
__global__ __launch_bounds__(WG) void k_pf_quant_x(const PfParams p) {
    __shared__ __align__(16) uint8_t scratch[WG / 64][512];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int NSB = p.d_model / 256;
    const int job = blockIdx.x * (WG / 64) + wave;
    const bool live = job < p.T * NSB;
    const int t = live ? job / NSB : 0, s = live ? job % NSB : 0;
    ActView L;
    act_layout(256, 0, &L);                     // 416 bytes
    uint8_t * base = scratch[wave];
    if (live) {
        ActSrc src;
        src.p = p.x + (int64_t)t * p.d_model + 256 * s;
        src.n = 256;
        q8K_block<SRC_PLAIN>(base, L, src, 0);
    }
    __syncthreads();
    if (!live) return;
    if (lane < 16) {
        uint32_t h[8];
        i8x16_to_h(reinterpret_cast<const u32x4 *>(base + L.q)[lane], h);
        u32x4 * d = reinterpret_cast<u32x4 *>(p.xq + (int64_t)t * p.d_model + 256 * s + 16 * lane);
        d[0] = u32x4{h[0], h[1], h[2], h[3]};
        d[1] = u32x4{h[4], h[5], h[6], h[7]};
    }
    if (lane == 0) p.xd[(int64_t)t * NSB + s] = reinterpret_cast<const float *>(base + L.dK)[0];
    if (lane < 8) {
        const int * bs = reinterpret_cast<const int *>(base + L.bsum);
        const int sum = bs[2 * lane] + bs[2 * lane + 1];
        const int lo = sum & 31, hi = (sum - lo) / 32;
        _Float16 * xm = p.xm + ((int64_t)t * NSB + s) * 16;
        xm[lane] = (_Float16)(float)hi;
        xm[8 + lane] = (_Float16)(float)lo;
    }
}

// -------------------------------------------------------------- gate_up

// The (multiplier, offset) pair of Q4_K sub-block j with 6-bit scale sc, as
// packed fp16 splats: sub-blocks come as the low nibbles (j even: (1024 + q)
// sc - 1024 sc) or the high nibbles (j odd: (1024 + 16 q) sc/16 - 64 sc) of a
// 32-byte run, both exact.  Computed once per super-block and row.
__device__ __forceinline__ void q4k_scale(int sc, int j, h2 & m, h2 & o) {
    const _Float16 scf = (_Float16)(float)sc;
    const bool hi = (j & 1) != 0;
    m = splat(hi ? scf * (_Float16)0.0625f : scf);
    o = splat(hi ? scf * (_Float16)(-64.0f) : scf * (_Float16)(-1024.0f));
}

// A fragment of lane (row, half) for k-step `step` (16 values) of a Q4_K
// super-block piece at `w`: 8 values q*sc as exact fp16, (m, o) from
// q4k_scale for sub-block step / 2.
__device__ __forceinline__ h8 q4k_frag(const uint8_t * w, int step, int half, h2 m, h2 o) {
    const int off = 16 + 32 * (step >> 2) + 16 * (step & 1) + 8 * half;
    const uint2 v = *reinterpret_cast<const uint2 *>(w + off);
    const bool hi = (step & 2) != 0;
    const uint32_t x0 = hi ? (v.x & 0xF0F0F0F0u) : (v.x & 0x0F0F0F0Fu);
    const uint32_t x1 = hi ? (v.y & 0xF0F0F0F0u) : (v.y & 0x0F0F0F0Fu);
    uint32_t a, b, c, d;
    bytes_to_magic(x0, a, b);
    bytes_to_magic(x1, c, d);
    return as_h8(hbits(__builtin_elementwise_fma(as_h2(a), m, o)), hbits(__builtin_elementwise_fma(as_h2(b), m, o)),
                 hbits(__builtin_elementwise_fma(as_h2(c), m, o)), hbits(__builtin_elementwise_fma(as_h2(d), m, o)));
}

// A fragment for IQ2_S: 8-group g8 = 2 step + half of the piece at `w`
// (2-aligned): grid * sign * (2 ls + 1) as exact fp16.
__device__ __forceinline__ h8 iq2s_frag(const uint8_t * w, int step, int half, const uint8_t * grid16,
                                        const uint8_t * sign16) {
    const int g8 = 2 * step + half;
    const uint32_t qs = w[2 + g8], sg = w[34 + g8], qh = w[66 + (g8 >> 2)], scb = w[74 + (g8 >> 2)];
    const uint32_t idx = qs | (((qh >> (2 * (g8 & 3))) & 3u) << 8);
    const uint32_t ls = (g8 & 2) ? (scb >> 4) : (scb & 15u);
    const u32x4 g = *reinterpret_cast<const u32x4 *>(grid16 + 16 * idx);
    const u32x4 s = *reinterpret_cast<const u32x4 *>(sign16 + 16 * sg);
    const h2 m = splat((_Float16)(float)(2 * ls + 1));
    return as_h8(hbits(as_h2(g.x ^ s.x) * m), hbits(as_h2(g.y ^ s.y) * m), hbits(as_h2(g.z ^ s.z) * m),
                 hbits(as_h2(g.w ^ s.w) * m));
}

// fp16 IQ2_S codebook [1024][8] and sign masks [256][8] (0x8000 per set bit)
__device__ __forceinline__ void build_iq2s_f16_tables(uint8_t * grid16, uint8_t * sign16) {
    const uint16_t lv[3] = {0x4800, 0x4E40, 0x5160};    // 8.0, 25.0, 43.0
    for (int k = threadIdx.x; k < 1024; k += WG) {
        const uint32_t c = c_iq2s_codes_pf[k];
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t l0 = (c >> (4 * i)) & 3, l1 = (c >> (4 * i + 2)) & 3;
            const uint32_t v0 = l0 == 0 ? lv[0] : l0 == 1 ? lv[1] : lv[2];
            const uint32_t v1 = l1 == 0 ? lv[0] : l1 == 1 ? lv[1] : lv[2];
            w[i] = v0 | (v1 << 16);
        }
        *reinterpret_cast<u32x4 *>(grid16 + 16 * k) = u32x4{w[0], w[1], w[2], w[3]};
    }
    {
        const uint32_t s = threadIdx.x;                  // WG == 256 sign bytes
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            w[i] = (((s >> (2 * i)) & 1) ? 0x8000u : 0u) | (((s >> (2 * i + 1)) & 1) ? 0x80000000u : 0u);
        *reinterpret_cast<u32x4 *>(sign16 + 16 * s) = u32x4{w[0], w[1], w[2], w[3]};
    }
}

// 16-byte chunks covering [ps, ps + len) of a slab; they stay inside the
// slab because slabs are whole 16-byte chunks
__device__ __forceinline__ int chunk_count(uint64_t ps, int len) {
    return (int)(((ps + len + 15) >> 4) - (ps >> 4));
}

constexpr int GU_WREG = 5;     // weight chunks per thread per super-block (Q4_K: 128 rows x 9)
constexpr int GU_XREG = 8;     // fp16 activation chunks per thread per super-block (64 tokens x 32)

// Registers of the next super-block in flight while the current one computes.
struct GuStage {
    u32x4 w[GU_WREG];
    u32x4 x[GU_XREG];
    u32x4 mb;
    uint32_t dw;
    float d8;
};

struct GuSmem {
    uint8_t w[PF_ROWS * PF_WROW_GU];
    _Float16 x[PF_TOK * PF_XS];
    _Float16 mb[PF_TOK * 16];
    uint8_t grid[1024 * 16];
    uint8_t sign[256 * 16];
    float d8[PF_TOK];
    float2 dw[PF_ROWS];
    int tok[PF_TOK], pair[PF_TOK], poff[PF_ROWS];
};

// One (tile, 128-row block) of the gate_up GEMM with NTT 32-token column
// tiles (a tile of at most 32 pairs computes, stages and stores one).
template <int HT, int CT, int NTT>
__device__ __forceinline__ void pf_gate_up_tile(const PfParams & p, const PfTile & tile, GuSmem & sm) {
    uint8_t * s_w = sm.w;
    _Float16 * s_x = sm.x;
    _Float16 * s_mb = sm.mb;
    uint8_t * s_grid = sm.grid;
    uint8_t * s_sign = sm.sign;
    float * s_d8 = sm.d8;
    float2 * s_dw = sm.dw;
    int * s_tok = sm.tok;
    int * s_pair = sm.pair;
    int * s_poff = sm.poff;
    constexpr int NTOK = 32 * NTT;
    static_assert(HT == T_Q4_K || HT == T_IQ2_S, "gate_up formats");
    static_assert(CT == T_Q4_K || CT == T_IQ2_S, "gate_up formats");
    static_assert(PF_ROWS * 9 <= GU_WREG * WG && PF_TOK * 32 == GU_XREG * WG, "staging shape");

    const int wtype = tile.tier == 0 ? HT : CT;
    const bool q4 = wtype == T_Q4_K;
    const int F2 = 2 * p.n_ff, NSB = p.d_model / 256, K = p.top_k;
    const int r0 = blockIdx.x * PF_ROWS;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, half = lane >> 5, col = lane & 31;
    const int bb = q4 ? 144 : 82;                              // bytes per super-block
    const int nwc = q4 ? 9 : 6;                                // staged 16-byte chunks per row
    const uint64_t rb = (uint64_t)NSB * bb;                    // bytes per row
    const uint8_t * W = tile.tier == 0 ? p.hot_gu + (uint64_t)tile.idx * p.hot_gu_stride
                                       : p.cold_gu + (uint64_t)tile.idx * p.cold_gu_stride;
    if (tid < PF_TOK) {
        const int q = p.sorted[tile.begin + min(tid, tile.n - 1)];
        s_pair[tid] = q;
        s_tok[tid] = q / K;
    }
    if (!q4) build_iq2s_f16_tables(s_grid, s_sign);
    __syncthreads();

    // per-thread staging geometry, fixed for the whole K loop (no divisions
    // or token lookups per super-block)
    uint32_t wrow[GU_WREG];      // byte offset of the chunk's row in the slab (row * rb); ~0u: no row
    uint32_t wdst[GU_WREG];      // LDS offset of the chunk | chunk index << 16
#pragma unroll
    for (int k = 0; k < GU_WREG; ++k) {
        const int i = tid + WG * k;
        const int r = i / nwc, c = i - nwc * r;
        wrow[k] = r < PF_ROWS ? (uint32_t)((uint64_t)min(r0 + r, F2 - 1) * rb) : ~0u;
        wdst[k] = (uint32_t)(r * (q4 ? 144 : 96) + 16 * c) | ((uint32_t)c << 16);
    }
    uint32_t xsrc[GU_XREG];      // element offset of the chunk's token row and column
#pragma unroll
    for (int k = 0; k < GU_XREG; ++k) {
        const int i = tid + WG * k, j = i >> 5, c = i & 31;
        xsrc[k] = (uint32_t)(s_tok[j] * p.d_model + 8 * c);
    }
    const int tok_s = tid < NTOK ? s_tok[tid] * NSB : 0;
    const int tok_m = (tid >= 64 && tid < 64 + 2 * NTOK) ? (s_tok[(tid - 64) >> 1] * NSB) * 16 + 8 * ((tid - 64) & 1) : 0;
    const uint32_t drow = tid >= WG - PF_ROWS ? (uint32_t)((uint64_t)min(r0 + tid - (WG - PF_ROWS), F2 - 1) * rb) : 0u;

    GuStage g;
    auto fetch = [&](int s) {
#pragma unroll
        for (int k = 0; k < GU_WREG; ++k) {
            g.w[k] = u32x4{0, 0, 0, 0};
            if (wrow[k] != ~0u) {
                const uint32_t ps = wrow[k] + (uint32_t)(bb * s);
                const int c = (int)(wdst[k] >> 16);
                if (q4 || c < chunk_count(ps, 82))
                    g.w[k] = *reinterpret_cast<const u32x4 *>(W + (ps & ~15u) + 16 * c);
            }
        }
#pragma unroll
        for (int k = 0; k < GU_XREG * NTT / 2; ++k)
            g.x[k] = *reinterpret_cast<const u32x4 *>(p.xq + xsrc[k] + 256 * s);
        if (tid < NTOK) g.d8 = p.xd[tok_s + s];
        if (tid >= 64 && tid < 64 + 2 * NTOK) g.mb = *reinterpret_cast<const u32x4 *>(p.xm + tok_m + 16 * s);
        if (tid >= WG - PF_ROWS) {
            const uint32_t ps = drow + (uint32_t)(bb * s);
            g.dw = q4 ? *reinterpret_cast<const uint32_t *>(W + ps) : *reinterpret_cast<const uint16_t *>(W + ps);
        }
    };
    auto store = [&](int s) {
#pragma unroll
        for (int k = 0; k < GU_WREG; ++k)
            if (wrow[k] != ~0u) *reinterpret_cast<u32x4 *>(s_w + (wdst[k] & 0xFFFF)) = g.w[k];
#pragma unroll
        for (int k = 0; k < GU_XREG * NTT / 2; ++k) {
            const int i = tid + WG * k, j = i >> 5, c = i & 31;
            *reinterpret_cast<u32x4 *>(s_x + j * PF_XS + 8 * c) = g.x[k];
        }
        if (tid < NTOK) s_d8[tid] = g.d8;
        if (tid >= 64 && tid < 64 + 2 * NTOK) {
            const int i = tid - 64;
            *reinterpret_cast<u32x4 *>(s_mb + 16 * (i >> 1) + 8 * (i & 1)) = g.mb;
        }
        if (tid >= WG - PF_ROWS) {
            const int r = tid - (WG - PF_ROWS);
            const uint32_t ps = drow + (uint32_t)(bb * s);
            s_dw[r] = make_float2(h2f(g.dw & 0xFFFF), q4 ? h2f(g.dw >> 16) : 0.0f);
            s_poff[r] = q4 ? r * 144 : r * 96 + (int)(ps & 15);
        }
    };

    f16v y0 = {}, y1 = {};
    const int row_l = 32 * wave + col;                          // this lane's A row in the block
    fetch(0);
    for (int s = 0; s < NSB; ++s) {
        if (s) __syncthreads();                                 // the previous super-block is consumed
        store(s);
        __syncthreads();
        if (s + 1 < NSB) fetch(s + 1);

        f16v a0 = {}, a1 = {};
        const uint8_t * wp = s_w + s_poff[row_l];
        const _Float16 * xb0 = s_x + col * PF_XS + 8 * half;
        const _Float16 * xb1 = xb0 + 32 * PF_XS;
        const float d80 = s_d8[col], d81 = NTT == 2 ? s_d8[32 + col] : 0.0f;
        if (q4) {
            // 6-bit scales and mins of this row (get_scale_min_k4, ggml-quants.c:822)
            const uint32_t q0 = *reinterpret_cast<const uint32_t *>(wp + 4);
            const uint32_t q1 = *reinterpret_cast<const uint32_t *>(wp + 8);
            const uint32_t q2 = *reinterpret_cast<const uint32_t *>(wp + 12);
            int sc[8], mn[8];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                sc[j] = (q0 >> (8 * j)) & 63;
                mn[j] = (q1 >> (8 * j)) & 63;
                sc[j + 4] = ((q2 >> (8 * j)) & 15) | (((q0 >> (8 * j + 6)) & 3) << 4);
                mn[j + 4] = ((q2 >> (8 * j + 4)) & 15) | (((q1 >> (8 * j + 6)) & 3) << 4);
            }
            h2 qm[8], qo[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) q4k_scale(sc[j], j, qm[j], qo[j]);
#pragma unroll
            for (int step = 0; step < 16; ++step) {
                const h8 a = q4k_frag(wp, step, half, qm[step >> 1], qo[step >> 1]);
                a0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, *reinterpret_cast<const h8 *>(xb0 + 16 * step), a0, 0, 0, 0);
                if (NTT == 2) a1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, *reinterpret_cast<const h8 *>(xb1 + 16 * step), a1, 0, 0, 0);
            }
            // mins: sum_j m_j * (32 hi_j + lo_j), exact
            const _Float16 f = half ? (_Float16)1.0f : (_Float16)32.0f;
            h8 am;
#pragma unroll
            for (int j = 0; j < 8; ++j) am[j] = (_Float16)(float)mn[j] * f;
            f16v m0 = {}, m1 = {};
            m0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(am, *reinterpret_cast<const h8 *>(s_mb + 16 * col + 8 * half), m0, 0, 0, 0);
            if (NTT == 2) m1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(am, *reinterpret_cast<const h8 *>(s_mb + 16 * (32 + col) + 8 * half), m1, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const float2 dm = s_dw[32 * wave + 8 * i + 4 * half + jj];
                    const int v = 4 * i + jj;
                    y0[v] += __fmul_rn(d80, dm.x) * a0[v] - __fmul_rn(d80, dm.y) * m0[v];
                    if (NTT == 2) y1[v] += __fmul_rn(d81, dm.x) * a1[v] - __fmul_rn(d81, dm.y) * m1[v];
                }
        } else {
#pragma unroll
            for (int step = 0; step < 16; ++step) {
                const h8 a = iq2s_frag(wp, step, half, s_grid, s_sign);
                a0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, *reinterpret_cast<const h8 *>(xb0 + 16 * step), a0, 0, 0, 0);
                if (NTT == 2) a1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, *reinterpret_cast<const h8 *>(xb1 + 16 * step), a1, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const float dw = s_dw[32 * wave + 8 * i + 4 * half + jj].x;
                    const int v = 4 * i + jj;
                    y0[v] += __fmul_rn(dw, d80) * a0[v];
                    if (NTT == 2) y1[v] += __fmul_rn(dw, d81) * a1[v];
                }
        }
    }
    // ---- store: rows 8i + 4 half + 0..3 of this wave's 32, tokens col and 32 + col
    const float f = q4 ? 1.0f : 0.125f;
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt) {
        const int j = col + 32 * tt;
        if (j < tile.n) {
            const f16v & y = tt ? y1 : y0;
            float * out = p.ygu + (int64_t)s_pair[j] * F2;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = r0 + 32 * wave + 8 * i + 4 * half;
                if (r + 3 < F2)
                    *reinterpret_cast<float4 *>(out + r) =
                        make_float4(f * y[4 * i], f * y[4 * i + 1], f * y[4 * i + 2], f * y[4 * i + 3]);
            }
        }
    }
}

template <int HT, int CT>
__global__ __launch_bounds__(WG) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_pf_gate_up(const PfParams p) {
    __shared__ __align__(16) GuSmem sm;
    if ((int)blockIdx.y >= *p.n_tiles) return;
    const PfTile tile = p.tiles[blockIdx.y];
    if (!tile_valid(p, tile) || tile.n <= 0 || tile.n > PF_TOK) return;
    if (tile.n > 32) pf_gate_up_tile<HT, CT, 2>(p, tile, sm);
    else pf_gate_up_tile<HT, CT, 1>(p, tile, sm);
}

// exact ints (as fp16 pairs) times the block scale d: hi = fp16(d * v),
// lo = fp16(d * v - hi) (exact: d * v has at most 11 + 8 significant bits)
__device__ __forceinline__ void scale_split(const uint32_t (&v)[4], _Float16 d, h8 & hi, h8 & lo) {
    const h2 m = splat(d);
    uint32_t h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const h2 x = as_h2(v[i]);
        const h2 a = x * m;
        h[i] = hbits(a);
        l[i] = hbits(__builtin_elementwise_fma(x, m, -a));
    }
    hi = as_h8(h[0], h[1], h[2], h[3]);
    lo = as_h8(l[0], l[1], l[2], l[3]);
}

// ----------------------------------------------------- down activations

// One workgroup per routed pair: GEGLU + q8_0 (the CPU path's activation
// format for 32-blocks, bit-identical).  Stored: d8 q times a per-pair power
// of two 2^e (2^e puts the largest |d8 q| in [2^14, 2^15)) as the exact sum
// of an fp16 high part and an fp16 remainder, and 2^-e.
template <int GSRC>
__global__ __launch_bounds__(WG) void k_pf_act(const PfParams p) {
    __shared__ __align__(16) uint8_t scratch[6400];     // act_layout(PF_MAX_FF) = 6240 bytes
    __shared__ float s_red[WG / 64];
    const int q = blockIdx.x;
    const int F = p.n_ff;
    const int e = p.ids[q];
    if (e < 0 || e >= p.n_expert) {
        // an invalid id contributes zeros (its pair is in no tile)
        for (int r = threadIdx.x; r < p.d_model; r += WG) p.ydn[(int64_t)q * p.d_model + r] = 0.0f;
        if (threadIdx.x == 0) p.ae[q] = 0.0f;
        return;
    }
    ActView L;
    act_layout(F, 0, &L);
    ActSrc src;
    src.p = p.ygu + (int64_t)q * 2 * F;
    src.n = F;
    quantize_q8_32<GSRC, AM_CPU>(scratch, L, src, F);
    __syncthreads();
    const int8_t * qv = reinterpret_cast<const int8_t *>(scratch + L.q);
    const float * d32 = reinterpret_cast<const float *>(scratch + L.d32);
    float amax = 0.0f;
    for (int b = threadIdx.x; b < F / 32; b += WG) amax = fmaxf(amax, d32[b] * 127.0f);
    amax = wave_max(amax);
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    int ex = 0;
    if (amax > 0.0f) ex = 14 - ilogbf(amax);
    ex = max(-100, min(100, ex));
    const float sc = ldexpf(1.0f, ex);
    // 16 values per thread step (within one 32-block: one scale)
    for (int i = threadIdx.x; i < F / 16; i += WG) {
        uint32_t h[8];
        i8x16_to_h(*reinterpret_cast<const u32x4 *>(qv + qpos(16 * i)), h);
        const _Float16 sv = (_Float16)(d32[i >> 1] * sc);
        h8 hi0, lo0, hi1, lo1;
        scale_split(*reinterpret_cast<const uint32_t (*)[4]>(h), sv, hi0, lo0);
        scale_split(*reinterpret_cast<const uint32_t (*)[4]>(h + 4), sv, hi1, lo1);
        h8 * dh = reinterpret_cast<h8 *>(p.ah + (int64_t)q * F + 16 * i);
        h8 * dl = reinterpret_cast<h8 *>(p.al + (int64_t)q * F + 16 * i);
        dh[0] = hi0;
        dh[1] = hi1;
        dl[0] = lo0;
        dl[1] = lo1;
    }
    if (threadIdx.x == 0) p.ae[q] = ldexpf(1.0f, -ex);
}

// ------------------------------------------------------------------ down


// 8 values at offset o (0, 8, 16, 24) of a Q5_0 block at `b` (2-aligned):
// q - 16 as exact fp16, then split-scaled by d
// (the block starts at byte `b` of the 16-aligned staging buffer `sw`; dwords
// are read at 4-aligned addresses and funnel-shifted)
__device__ __forceinline__ void q5_0_frag(const uint8_t * sw, int b, int o, h8 & hi, h8 & lo) {
    const _Float16 d = __builtin_bit_cast(_Float16, *reinterpret_cast<const uint16_t *>(sw + b));
    const uint32_t qh = lds32u(sw, b + 2);
    const int lw = o & 15;
    const uint32_t w0 = lds32u(sw, b + 6 + lw), w1 = lds32u(sw, b + 10 + lw);
    const bool hn = o >= 16;
    uint32_t x0 = (hn ? (w0 >> 4) : w0) & 0x0F0F0F0Fu;
    uint32_t x1 = (hn ? (w1 >> 4) : w1) & 0x0F0F0F0Fu;
    const uint32_t hb = (qh >> o) & 0xFFu;
    x0 |= (((hb & 15u) * 0x00204081u) & 0x01010101u) << 4;
    x1 |= (((hb >> 4) * 0x00204081u) & 0x01010101u) << 4;
    uint32_t m[4];
    bytes_to_magic(x0, m[0], m[1]);
    bytes_to_magic(x1, m[2], m[3]);
    const h2 off = splat((_Float16)(-1040.0f));
    uint32_t v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = hbits(as_h2(m[i]) + off);
    scale_split(v, d, hi, lo);
}

// IQ4_NL: kvalues[q] as exact fp16, split-scaled by d
__device__ __forceinline__ void iq4nl_frag(const uint8_t * sw, int b, int o, h8 & hi, h8 & lo) {
    const _Float16 d = __builtin_bit_cast(_Float16, *reinterpret_cast<const uint16_t *>(sw + b));
    const int lw = o & 15;
    const uint32_t w0 = lds32u(sw, b + 2 + lw), w1 = lds32u(sw, b + 6 + lw);
    const bool hn = o >= 16;
    // signed bytes + 128 -> unsigned, then (1024 + 128 + v) - 1152
    const uint32_t x0 = iq4nl_lookup((hn ? (w0 >> 4) : w0) & 0x0F0F0F0Fu) ^ 0x80808080u;
    const uint32_t x1 = iq4nl_lookup((hn ? (w1 >> 4) : w1) & 0x0F0F0F0Fu) ^ 0x80808080u;
    uint32_t m[4];
    bytes_to_magic(x0, m[0], m[1]);
    bytes_to_magic(x1, m[2], m[3]);
    const h2 off = splat((_Float16)(-1152.0f));
    uint32_t v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = hbits(as_h2(m[i]) + off);
    scale_split(v, d, hi, lo);
}

constexpr int DN_WREG = 4;     // weight chunks per thread per down chunk (128 rows x 7)
constexpr int DN_XREG = 4;     // fp16 activation chunks per thread per down chunk and part (64 tokens x 16)

struct DnStage {
    u32x4 w[DN_WREG];
    u32x4 xh[DN_XREG], xl[DN_XREG];
};

struct DnSmem {
    uint8_t w[PF_ROWS * PF_WPITCH_DN + 16];    // +16: funnel reads past a row's end
    _Float16 x[PF_TOK * PF_DXS];
    _Float16 xl[PF_TOK * PF_DXS];
    int pair[PF_TOK], poff[PF_ROWS];
};

// One (tile, 128-row block) of the down GEMM with NTT 32-token column tiles.
template <int HT, int CT, int NTT>
__device__ __forceinline__ void pf_down_tile(const PfParams & p, const PfTile & tile, DnSmem & sm) {
    uint8_t * s_w = sm.w;
    _Float16 * s_x = sm.x;
    _Float16 * s_xl = sm.xl;
    int * s_pair = sm.pair;
    int * s_poff = sm.poff;
    static_assert(HT == T_Q5_0 || HT == T_IQ4_NL, "down formats");
    static_assert(CT == T_Q5_0 || CT == T_IQ4_NL, "down formats");
    static_assert(PF_ROWS * (PF_WROW_DN / 16) <= DN_WREG * WG && PF_TOK * PF_DCB * 4 == DN_XREG * WG, "staging shape");

    const int wtype = tile.tier == 0 ? HT : CT;
    const int D = p.d_model, F = p.n_ff, NB = F / 32;
    const int r0 = blockIdx.x * PF_ROWS;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, half = lane >> 5, col = lane & 31;
    const int bs = wtype == T_Q5_0 ? 22 : 18;
    const uint64_t rb = (uint64_t)NB * bs;
    constexpr int WCH = PF_WROW_DN / 16;
    const uint8_t * W = tile.tier == 0 ? p.hot_dn + (uint64_t)tile.idx * p.hot_dn_stride
                                       : p.cold_dn + (uint64_t)tile.idx * p.cold_dn_stride;
    if (tid < PF_TOK) s_pair[tid] = p.sorted[tile.begin + min(tid, tile.n - 1)];
    __syncthreads();

    DnStage g;
    auto fetch = [&](int c0) {
        const int cb = min(PF_DCB, NB - c0);
#pragma unroll
        for (int k = 0; k < DN_WREG; ++k) {
            const int i = tid + WG * k, r = i / WCH, c = i - WCH * (i / WCH);
            g.w[k] = u32x4{0, 0, 0, 0};
            if (r < PF_ROWS) {
                const uint64_t ps = (uint64_t)min(r0 + r, D - 1) * rb + (uint64_t)c0 * bs;
                if (c < chunk_count(ps, cb * bs))
                    g.w[k] = *reinterpret_cast<const u32x4 *>(W + (ps & ~(uint64_t)15) + 16 * c);
            }
        }
#pragma unroll
        for (int k = 0; k < DN_XREG * NTT / 2; ++k) {
            const int i = tid + WG * k, j = i / (4 * PF_DCB), c = i - (4 * PF_DCB) * j;   // 8-value chunk c
            g.xh[k] = u32x4{0, 0, 0, 0};
            g.xl[k] = u32x4{0, 0, 0, 0};
            if (c < 4 * cb) {
                const int64_t q = s_pair[j];
                g.xh[k] = *reinterpret_cast<const u32x4 *>(p.ah + q * F + 32 * c0 + 8 * c);
                g.xl[k] = *reinterpret_cast<const u32x4 *>(p.al + q * F + 32 * c0 + 8 * c);
            }
        }
    };
    auto store = [&](int c0) {
#pragma unroll
        for (int k = 0; k < DN_WREG; ++k) {
            const int i = tid + WG * k, r = i / WCH, c = i - WCH * (i / WCH);
            if (r < PF_ROWS) {
                uint2 * d = reinterpret_cast<uint2 *>(s_w + r * PF_WPITCH_DN + 16 * c);   // 8-aligned
                d[0] = make_uint2(g.w[k].x, g.w[k].y);
                d[1] = make_uint2(g.w[k].z, g.w[k].w);
                if (c == 0) {
                    const uint64_t ps = (uint64_t)min(r0 + r, D - 1) * rb + (uint64_t)c0 * bs;
                    s_poff[r] = r * PF_WPITCH_DN + (int)(ps & 15);
                }
            }
        }
#pragma unroll
        for (int k = 0; k < DN_XREG * NTT / 2; ++k) {
            const int i = tid + WG * k, j = i / (4 * PF_DCB), c = i - (4 * PF_DCB) * j;
            *reinterpret_cast<u32x4 *>(s_x + j * PF_DXS + 8 * c) = g.xh[k];
            *reinterpret_cast<u32x4 *>(s_xl + j * PF_DXS + 8 * c) = g.xl[k];
        }
    };

    f16v y0 = {}, y1 = {};
    const int row_l = 32 * wave + col;
    fetch(0);
    for (int c0 = 0; c0 < NB; c0 += PF_DCB) {
        const int cb = min(PF_DCB, NB - c0);           // blocks in this chunk
        if (c0) __syncthreads();
        store(c0);
        __syncthreads();
        if (c0 + PF_DCB < NB) fetch(c0 + PF_DCB);
        const int wp = s_poff[row_l];
        const int xo0 = col * PF_DXS + 8 * half, xo1 = xo0 + 32 * PF_DXS;
        // one 16-value step: weight fragment hi/lo, three MFMAs per token tile
        auto step_fn = [&](auto wt, int step) {
            h8 ah, al;
            if constexpr (decltype(wt)::value == T_Q5_0) q5_0_frag(s_w, wp + 22 * (step >> 1), 16 * (step & 1) + 8 * half, ah, al);
            else iq4nl_frag(s_w, wp + 18 * (step >> 1), 16 * (step & 1) + 8 * half, ah, al);
            const h8 b0h = *reinterpret_cast<const h8 *>(s_x + xo0 + 16 * step);
            const h8 b0l = *reinterpret_cast<const h8 *>(s_xl + xo0 + 16 * step);
            y0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, b0h, y0, 0, 0, 0);
            y0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, b0l, y0, 0, 0, 0);
            y0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, b0h, y0, 0, 0, 0);
            if (NTT == 2) {
                const h8 b1h = *reinterpret_cast<const h8 *>(s_x + xo1 + 16 * step);
                const h8 b1l = *reinterpret_cast<const h8 *>(s_xl + xo1 + 16 * step);
                y1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, b1h, y1, 0, 0, 0);
                y1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, b1l, y1, 0, 0, 0);
                y1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, b1h, y1, 0, 0, 0);
            }
        };
        // the weight format is uniform per tile: one branch per chunk, and
        // whole chunks run fully unrolled
        auto chunk = [&](auto wt) {
            if (cb == PF_DCB) {
#pragma unroll
                for (int step = 0; step < 2 * PF_DCB; ++step) step_fn(wt, step);
            } else {
                for (int step = 0; step < 2 * cb; ++step) step_fn(wt, step);
            }
        };
        if (wtype == T_Q5_0) chunk(std::integral_constant<int, T_Q5_0>{});
        else chunk(std::integral_constant<int, T_IQ4_NL>{});
    }
    const float sc = tile.tier == 0 ? (p.s_hot ? p.s_hot[tile.idx] : 1.0f) : (p.s_cold ? p.s_cold[tile.idx] : 1.0f);
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt) {
        const int j = col + 32 * tt;
        if (j < tile.n) {
            const int q = s_pair[j];
            const float f = p.ae[q] * sc;
            const f16v & y = tt ? y1 : y0;
            float * out = p.ydn + (int64_t)q * D;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = r0 + 32 * wave + 8 * i + 4 * half;
                if (r + 3 < D)
                    *reinterpret_cast<float4 *>(out + r) =
                        make_float4(f * y[4 * i], f * y[4 * i + 1], f * y[4 * i + 2], f * y[4 * i + 3]);
            }
        }
    }
}

template <int HT, int CT>
__global__ __launch_bounds__(WG) void k_pf_down(const PfParams p) {
    __shared__ __align__(16) DnSmem sm;
    if ((int)blockIdx.y >= *p.n_tiles) return;
    const PfTile tile = p.tiles[blockIdx.y];
    if (!tile_valid(p, tile) || tile.n <= 0 || tile.n > PF_TOK) return;
    if (tile.n > 32) pf_down_tile<HT, CT, 2>(p, tile, sm);
    else pf_down_tile<HT, CT, 1>(p, tile, sm);
}

}  // namespace dev

using namespace dev;

int pf_max_tiles(int P, int n_expert) { return (P + PF_TOK - 1) / PF_TOK + std::min(n_expert, P); }

namespace {
template <typename F>
void launch_pf(F k, dim3 grid, hipStream_t s, hipEvent_t e0, hipEvent_t e1, const PfParams & p) {
    if (e0) hipExtLaunchKernelGGL(k, grid, dim3(WG), 0u, s, e0, e1, 0u, p);
    else hipLaunchKernelGGL(k, grid, dim3(WG), 0, s, p);
}
}  // namespace

hipError_t launch_prefill(const PfParams & p, int hgu, int cgu, int hdn, int cdn, int gelu, hipStream_t s,
                          hipEvent_t * ev) {
    hipEvent_t e[4] = {};
    if (ev)
        for (int i = 0; i < 4; ++i) e[i] = ev[i];
    const int P = p.T * p.top_k;
    const int NSB = p.d_model / 256;
    hipLaunchKernelGGL(k_pf_bucket, dim3(1), dim3(WG), 0, s, p);
    hipLaunchKernelGGL(k_pf_quant_x, dim3((p.T * NSB + 3) / 4), dim3(WG), 0, s, p);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    {
        dim3 grid((2 * p.n_ff + PF_ROWS - 1) / PF_ROWS, p.max_tiles);
        if (hgu == T_Q4_K && cgu == T_IQ2_S) launch_pf(k_pf_gate_up<T_Q4_K, T_IQ2_S>, grid, s, e[0], e[1], p);
        else if (hgu == T_Q4_K && cgu == T_Q4_K) launch_pf(k_pf_gate_up<T_Q4_K, T_Q4_K>, grid, s, e[0], e[1], p);
        else if (hgu == T_IQ2_S && cgu == T_IQ2_S) launch_pf(k_pf_gate_up<T_IQ2_S, T_IQ2_S>, grid, s, e[0], e[1], p);
        else if (hgu == T_IQ2_S && cgu == T_Q4_K) launch_pf(k_pf_gate_up<T_IQ2_S, T_Q4_K>, grid, s, e[0], e[1], p);
        else return hipErrorInvalidValue;
        err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    if (gelu == SRC_GEGLU_TANH) hipLaunchKernelGGL(k_pf_act<SRC_GEGLU_TANH>, dim3(P), dim3(WG), 0, s, p);
    else hipLaunchKernelGGL(k_pf_act<SRC_GEGLU_TABLE>, dim3(P), dim3(WG), 0, s, p);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    {
        dim3 grid((p.d_model + PF_ROWS - 1) / PF_ROWS, p.max_tiles);
        if (hdn == T_Q5_0 && cdn == T_IQ4_NL) launch_pf(k_pf_down<T_Q5_0, T_IQ4_NL>, grid, s, e[2], e[3], p);
        else if (hdn == T_Q5_0 && cdn == T_Q5_0) launch_pf(k_pf_down<T_Q5_0, T_Q5_0>, grid, s, e[2], e[3], p);
        else if (hdn == T_IQ4_NL && cdn == T_IQ4_NL) launch_pf(k_pf_down<T_IQ4_NL, T_IQ4_NL>, grid, s, e[2], e[3], p);
        else if (hdn == T_IQ4_NL && cdn == T_Q5_0) launch_pf(k_pf_down<T_IQ4_NL, T_Q5_0>, grid, s, e[2], e[3], p);
        else return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace llapis
