// prefill.hip -- the MoE layer for long token batches (prefill chunks) on
// gfx950 matrix cores.
//
//   k_pf_bucket    routed pairs grouped by expert (a stable counting sort:
//                  per-64-pair chunk ranks from wave ballots, chunk prefix
//                  sums per expert) and cut into tiles of <= PF_TOK pairs,
//                  each tile tagged with its tier by the residency predicate
//                  (ggml-cuda/mmid.cu:28-116 groups the same way; moert/cuda/
//                  ffn_moe.cu:80-130 is the predicate).
//   k_pf_quant_x   each token quantised once to q8_K (the CPU path's
//                  activation format for 256-blocks) and stored as exact fp16
//                  integers, with the per-256 scale and the per-32 sums split
//                  into fp16-exact high and low parts.
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
//                  exact sum of two fp16 parts.
//   k_pf_down      grouped GEMM of the down projection.  Its scales are per
//                  32-value block, so they are folded into the operands
//                  instead of rescaling every output per block: d*q of the
//                  weights also splits exactly into fp16 hi + lo, and three
//                  MFMAs per step (hi*hi, hi*lo, lo*hi) give the dot to about
//                  2^-21 relative.
// The combine is the generic k_combine.
#include <hip/hip_ext.h>

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
constexpr int PF_DCB = 8;                 // 32-blocks per down K chunk
constexpr int PF_DXS = PF_DCB * 32 + 8;   // halfs per staged activation row of down (padded)
constexpr int PF_WROW_GU = 144;           // LDS bytes per weight row and super-block (Q4_K 144, IQ2_S <= 96)
constexpr int PF_WROW_DN = 192;           // LDS bytes per weight row and down chunk (<= 8 * 22 + 14)

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

__device__ __forceinline__ bool tile_valid(const PfParams & p, const PfTile & t) {
    return (t.tier == 0 && t.idx >= 0 && t.idx < p.k_slots) || (t.tier == 1 && t.idx >= 0 && t.idx < p.n_expert);
}

// ----------------------------------------------------------------- bucket

// One workgroup.  P = T * top_k <= PF_MAX_PAIRS, n_expert <= 256.
__global__ __launch_bounds__(WG) void k_pf_bucket(const PfParams p) {
    constexpr int MAXCH = PF_MAX_PAIRS / 64;
    __shared__ uint16_t s_cc[MAXCH][257];      // per chunk, per expert (+1 column: invalid ids)
    __shared__ int s_off[257];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int P = p.T * p.top_k, E = p.n_expert;
    const int nch = (P + 63) / 64;
    for (int i = threadIdx.x; i < nch * 257; i += WG) s_cc[i / 257][i % 257] = 0;
    __syncthreads();
    // pass 1: per chunk, per expert counts (leaders of equal-expert lane groups)
    for (int c = wave; c < nch; c += WG / 64) {
        const int q = 64 * c + lane;
        int e = 256;                            // past-the-end lanes and invalid ids
        if (q < P) {
            const int v = p.ids[q];
            e = (v >= 0 && v < E) ? v : 256;
        }
        uint64_t eq = ~0ull;
#pragma unroll
        for (int b = 0; b < 9; ++b) {
            const uint64_t m = __ballot((e >> b) & 1);
            eq &= ((e >> b) & 1) ? m : ~m;
        }
        const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
        const uint64_t live = __ballot(q < P);          // every lane votes (outside the branch)
        if ((eq & below) == 0 && q < P) s_cc[c][e] = (uint16_t)__popcll(eq & live);
    }
    __syncthreads();
    // chunk prefix per expert; totals
    for (int e = threadIdx.x; e < 257; e += WG) {
        int run = 0;
        for (int c = 0; c < nch; ++c) {
            const int t = s_cc[c][e];
            s_cc[c][e] = (uint16_t)run;
            run += t;
        }
        s_off[e] = run;                         // count for now
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int acc = 0, nt = 0;
        for (int e = 0; e < E; ++e) {
            const int n = s_off[e];
            s_off[e] = acc;
            int tier = 1, idx = e;
            if (p.k_slots > 0) {
                const int s = p.exp_slot[e];
                if (s >= 0 && s < p.k_slots && p.slot_state[s] == 2 && p.slot_exp[s] == e) {
                    tier = 0;
                    idx = s;
                }
            }
            for (int b = 0; b < n && nt < p.max_tiles; b += PF_TOK) {
                PfTile t;
                t.tier = tier;
                t.idx = idx;
                t.begin = acc + b;
                t.n = min(PF_TOK, n - b);
                p.tiles[nt++] = t;
            }
            acc += n;
        }
        s_off[256] = acc;                       // invalid ids are placed after every expert's pairs
        *p.n_tiles = nt;
    }
    __syncthreads();
    // pass 2: positions
    for (int c = wave; c < nch; c += WG / 64) {
        const int q = 64 * c + lane;
        int e = 256;
        if (q < P) {
            const int v = p.ids[q];
            e = (v >= 0 && v < E) ? v : 256;
        }
        uint64_t eq = ~0ull;
#pragma unroll
        for (int b = 0; b < 9; ++b) {
            const uint64_t m = __ballot((e >> b) & 1);
            eq &= ((e >> b) & 1) ? m : ~m;
        }
        const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
        const int rank = __popcll(eq & below);
        if (q < P) p.sorted[s_off[e] + s_cc[c][e] + rank] = q;
    }
}

// ------------------------------------------------------------ token quant

// One wave per (token, 256-block): q8_K exactly as the CPU path, then the
// values as fp16 (exact), the scale, and the 8 per-32 sums as
// {hi_0..hi_7, lo_0..lo_7} with sum = 32 hi + lo, 0 <= lo < 32.
__global__ __launch_bounds__(WG) void k_pf_quant_x(const PfParams p) {
    __shared__ __align__(16) uint8_t scratch[WG / 64][512];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int NSB = p.d_model / 256;
    const int job = blockIdx.x * (WG / 64) + wave;
    const bool live = job < p.T * NSB;
    const int t = live ? job / NSB : 0, s = live ? job % NSB : 0;
    ActView L;
    act_layout(256, 0, &L);                     // 256 + 16 + 16 + ... < 512 bytes
    uint8_t * base = scratch[wave];
    if (live) {
        ActSrc src;
        src.p = p.x + (int64_t)t * p.d_model + 256 * s;
        src.n = 256;
        q8K_block<SRC_PLAIN>(base, L, src, 0);
    }
    __syncthreads();
    if (!live) return;
    const int8_t * q = reinterpret_cast<const int8_t *>(base + L.q);
    _Float16 * xh = p.xh + (int64_t)t * p.d_model + 256 * s;
#pragma unroll
    for (int j = 0; j < 4; ++j) xh[lane + 64 * j] = (_Float16)(float)q[lane + 64 * j];
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

// A fragment of lane (row, half) for k-step `step` (16 values) of a Q4_K
// super-block piece at `w`: 8 values q*sc as exact fp16.
__device__ __forceinline__ h8 q4k_frag(const uint8_t * w, int step, int half, int sc) {
    const int off = 16 + 32 * (step >> 2) + 16 * (step & 1) + 8 * half;
    const uint2 v = *reinterpret_cast<const uint2 *>(w + off);
    const bool hi = (step & 2) != 0;
    const uint32_t x0 = hi ? (v.x & 0xF0F0F0F0u) : (v.x & 0x0F0F0F0Fu);
    const uint32_t x1 = hi ? (v.y & 0xF0F0F0F0u) : (v.y & 0x0F0F0F0Fu);
    // lo: (1024 + q) sc - 1024 sc;  hi: (1024 + 16 q) sc/16 - 64 sc  (exact)
    const _Float16 scf = (_Float16)(float)sc;
    const h2 m = splat(hi ? scf * (_Float16)0.0625f : scf);
    const h2 o = splat(hi ? scf * (_Float16)(-64.0f) : scf * (_Float16)(-1024.0f));
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

// copy the 16-byte chunks covering [ps, ps + len) of a slab into LDS at dst;
// returns nothing -- the piece starts at dst + (ps & 15).  Chunks stay inside
// the slab because slabs are whole 16-byte chunks.
__device__ __forceinline__ int chunk_count(uint64_t ps, int len) {
    return (int)(((ps + len + 15) >> 4) - (ps >> 4));
}

template <int HT, int CT>
__global__ __launch_bounds__(WG) void k_pf_gate_up(const PfParams p) {
    __shared__ __align__(16) uint8_t s_w[PF_ROWS * PF_WROW_GU];
    __shared__ __align__(16) _Float16 s_x[PF_TOK * PF_XS];
    __shared__ __align__(16) _Float16 s_mb[PF_TOK * 16];
    __shared__ __align__(16) uint8_t s_grid[1024 * 16];
    __shared__ __align__(16) uint8_t s_sign[256 * 16];
    __shared__ float s_d8[PF_TOK];
    __shared__ float2 s_dw[PF_ROWS];
    __shared__ int s_tok[PF_TOK], s_pair[PF_TOK], s_poff[PF_ROWS];
    static_assert(HT == T_Q4_K || HT == T_IQ2_S, "gate_up formats");
    static_assert(CT == T_Q4_K || CT == T_IQ2_S, "gate_up formats");

    if ((int)blockIdx.y >= *p.n_tiles) return;
    const PfTile tile = p.tiles[blockIdx.y];
    if (!tile_valid(p, tile) || tile.n <= 0 || tile.n > PF_TOK) return;
    const int wtype = tile.tier == 0 ? HT : CT;
    const int F2 = 2 * p.n_ff, NSB = p.d_model / 256, K = p.top_k;
    const int r0 = blockIdx.x * PF_ROWS;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, half = lane >> 5, col = lane & 31;
    const int bb = wtype == T_Q4_K ? 144 : 82;                 // bytes per super-block
    const uint64_t rb = (uint64_t)NSB * bb;                     // bytes per row
    const uint8_t * W = tile.tier == 0 ? p.hot_gu + (uint64_t)tile.idx * p.hot_gu_stride
                                       : p.cold_gu + (uint64_t)tile.idx * p.cold_gu_stride;
    if (threadIdx.x < PF_TOK) {
        const int j = threadIdx.x;
        const int q = p.sorted[tile.begin + min(j, tile.n - 1)];
        s_pair[j] = q;
        s_tok[j] = q / K;
    }
    if (wtype == T_IQ2_S) build_iq2s_f16_tables(s_grid, s_sign);
    __syncthreads();

    f16v y = {};
    const int row_l = 32 * wave + col;                          // this lane's A row in the block
    for (int s = 0; s < NSB; ++s) {
        if (s) __syncthreads();
        // ---- stage
        if (wtype == T_Q4_K) {
            for (int i = threadIdx.x; i < PF_ROWS * 9; i += WG) {
                const int r = i / 9, c = i - 9 * (i / 9);
                const uint64_t rr = (uint64_t)min(r0 + r, F2 - 1);
                *reinterpret_cast<u32x4 *>(s_w + r * 144 + 16 * c) =
                    *reinterpret_cast<const u32x4 *>(W + rr * rb + 144 * s + 16 * c);
            }
        } else {
            for (int i = threadIdx.x; i < PF_ROWS * 6; i += WG) {
                const int r = i / 6, c = i - 6 * (i / 6);
                const uint64_t rr = (uint64_t)min(r0 + r, F2 - 1);
                const uint64_t ps = rr * rb + 82 * s;
                if (c < chunk_count(ps, 82))
                    *reinterpret_cast<u32x4 *>(s_w + r * 96 + 16 * c) =
                        *reinterpret_cast<const u32x4 *>(W + (ps & ~(uint64_t)15) + 16 * c);
            }
        }
        for (int i = threadIdx.x; i < PF_TOK * 32; i += WG) {
            const int j = i >> 5, c = i & 31;
            *reinterpret_cast<u32x4 *>(s_x + j * PF_XS + 8 * c) =
                *reinterpret_cast<const u32x4 *>(p.xh + (int64_t)s_tok[j] * p.d_model + 256 * s + 8 * c);
        }
        if (threadIdx.x < PF_TOK) s_d8[threadIdx.x] = p.xd[(int64_t)s_tok[threadIdx.x] * NSB + s];
        if (threadIdx.x >= 64 && threadIdx.x < 64 + 2 * PF_TOK) {
            const int i = threadIdx.x - 64, j = i >> 1, hh = i & 1;
            *reinterpret_cast<u32x4 *>(s_mb + 16 * j + 8 * hh) =
                *reinterpret_cast<const u32x4 *>(p.xm + ((int64_t)s_tok[j] * NSB + s) * 16 + 8 * hh);
        }
        if (threadIdx.x >= 128) {
            const int r = threadIdx.x - 128;
            const uint64_t rr = (uint64_t)min(r0 + r, F2 - 1);
            const uint64_t ps = rr * rb + (uint64_t)bb * s;
            if (wtype == T_Q4_K) {
                const uint32_t dd = *reinterpret_cast<const uint32_t *>(W + ps);
                s_dw[r] = make_float2(h2f(dd & 0xFFFF), h2f(dd >> 16));
                s_poff[r] = r * 144;
            } else {
                s_dw[r] = make_float2(h2f(*reinterpret_cast<const uint16_t *>(W + ps)), 0.0f);
                s_poff[r] = r * 96 + (int)(ps & 15);
            }
        }
        __syncthreads();

        // ---- MFMA over the super-block
        f16v acc = {};
        const uint8_t * wp = s_w + s_poff[row_l];
        const _Float16 * xb = s_x + col * PF_XS + 8 * half;
        if (wtype == T_Q4_K) {
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
#pragma unroll
            for (int step = 0; step < 16; ++step) {
                const int j = step >> 1;
                const int scj = j == 0 ? sc[0] : j == 1 ? sc[1] : j == 2 ? sc[2] : j == 3 ? sc[3]
                              : j == 4 ? sc[4] : j == 5 ? sc[5] : j == 6 ? sc[6] : sc[7];
                const h8 a = q4k_frag(wp, step, half, scj);
                const h8 b = *reinterpret_cast<const h8 *>(xb + 16 * step);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
            }
            // mins: sum_j m_j * (32 hi_j + lo_j), exact
            const _Float16 f = half ? (_Float16)1.0f : (_Float16)32.0f;
            const h8 am = {(_Float16)(float)mn[0] * f, (_Float16)(float)mn[1] * f, (_Float16)(float)mn[2] * f,
                           (_Float16)(float)mn[3] * f, (_Float16)(float)mn[4] * f, (_Float16)(float)mn[5] * f,
                           (_Float16)(float)mn[6] * f, (_Float16)(float)mn[7] * f};
            const h8 bm = *reinterpret_cast<const h8 *>(s_mb + 16 * col + 8 * half);
            f16v mins = {};
            mins = __builtin_amdgcn_mfma_f32_32x32x16_f16(am, bm, mins, 0, 0, 0);
            const float d8 = s_d8[col];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const float2 dm = s_dw[32 * wave + 8 * i + 4 * half + jj];
                    const int v = 4 * i + jj;
                    y[v] += __fmul_rn(d8, dm.x) * acc[v] - __fmul_rn(d8, dm.y) * mins[v];
                }
        } else {
#pragma unroll
            for (int step = 0; step < 16; ++step) {
                const h8 a = iq2s_frag(wp, step, half, s_grid, s_sign);
                const h8 b = *reinterpret_cast<const h8 *>(xb + 16 * step);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
            }
            const float d8 = s_d8[col];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const int v = 4 * i + jj;
                    y[v] += __fmul_rn(s_dw[32 * wave + 8 * i + 4 * half + jj].x, d8) * acc[v];
                }
        }
    }
    // ---- store: rows 8i + 4 half + 0..3 of this wave's 32, token `col`
    if (col < tile.n) {
        float * out = p.ygu + (int64_t)s_pair[col] * F2;
        const float f = wtype == T_IQ2_S ? 0.125f : 1.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = r0 + 32 * wave + 8 * i + 4 * half;
            if (r + 3 < F2)
                *reinterpret_cast<float4 *>(out + r) = make_float4(f * y[4 * i], f * y[4 * i + 1], f * y[4 * i + 2],
                                                                   f * y[4 * i + 3]);
        }
    }
}

// ----------------------------------------------------- down activations

// One workgroup per routed pair: GEGLU + q8_0 (the CPU path's activation
// format for 32-blocks, bit-identical), then v = d8 * q * 2^e (exact in fp32)
// with 2^e chosen per pair so the largest magnitude lands in [2^14, 2^15),
// stored as hi = fp16(v) and lo = fp16(v - hi) (exact: v has <= 19 bits).
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
    for (int k = threadIdx.x; k < F; k += WG) amax = fmaxf(amax, fabsf(d32[k >> 5] * (float)qv[k]));
    amax = wave_max(amax);
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    int ex = 0;
    if (amax > 0.0f) ex = 14 - ilogbf(amax);
    ex = max(-100, min(100, ex));
    const float sc = ldexpf(1.0f, ex);
    _Float16 * hi = p.ah + (int64_t)q * F;
    _Float16 * lo = p.al + (int64_t)q * F;
    for (int k = threadIdx.x; k < F; k += WG) {
        const float v = d32[k >> 5] * (float)qv[k] * sc;
        const _Float16 h = (_Float16)v;
        hi[k] = h;
        lo[k] = (_Float16)(v - (float)h);
    }
    if (threadIdx.x == 0) p.ae[q] = ldexpf(1.0f, -ex);
}

// ------------------------------------------------------------------ down

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

// 8 values at offset o (0, 8, 16, 24) of a Q5_0 block at `b` (2-aligned):
// q - 16 as exact fp16, then split-scaled by d
__device__ __forceinline__ void q5_0_frag(const uint8_t * b, int o, h8 & hi, h8 & lo) {
    const _Float16 d = __builtin_bit_cast(_Float16, *reinterpret_cast<const uint16_t *>(b));
    const uint32_t qh = lds32u(b, 2);
    const int lw = o & 15;
    const uint32_t w0 = lds32u(b, 6 + lw), w1 = lds32u(b, 10 + lw);
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
__device__ __forceinline__ void iq4nl_frag(const uint8_t * b, int o, h8 & hi, h8 & lo) {
    const _Float16 d = __builtin_bit_cast(_Float16, *reinterpret_cast<const uint16_t *>(b));
    const int lw = o & 15;
    const uint32_t w0 = lds32u(b, 2 + lw), w1 = lds32u(b, 6 + lw);
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

template <int HT, int CT>
__global__ __launch_bounds__(WG) void k_pf_down(const PfParams p) {
    __shared__ __align__(16) uint8_t s_w[PF_ROWS * PF_WROW_DN + 16];   // +16: funnel reads past a row's end
    __shared__ __align__(16) _Float16 s_x[PF_TOK * PF_DXS];
    __shared__ __align__(16) _Float16 s_xl[PF_TOK * PF_DXS];
    __shared__ int s_pair[PF_TOK], s_poff[PF_ROWS];
    static_assert(HT == T_Q5_0 || HT == T_IQ4_NL, "down formats");
    static_assert(CT == T_Q5_0 || CT == T_IQ4_NL, "down formats");

    if ((int)blockIdx.y >= *p.n_tiles) return;
    const PfTile tile = p.tiles[blockIdx.y];
    if (!tile_valid(p, tile) || tile.n <= 0 || tile.n > PF_TOK) return;
    const int wtype = tile.tier == 0 ? HT : CT;
    const int D = p.d_model, F = p.n_ff, NB = F / 32;
    const int r0 = blockIdx.x * PF_ROWS;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, half = lane >> 5, col = lane & 31;
    const int bs = wtype == T_Q5_0 ? 22 : 18;
    const uint64_t rb = (uint64_t)NB * bs;
    const uint8_t * W = tile.tier == 0 ? p.hot_dn + (uint64_t)tile.idx * p.hot_dn_stride
                                       : p.cold_dn + (uint64_t)tile.idx * p.cold_dn_stride;
    if (threadIdx.x < PF_TOK) s_pair[threadIdx.x] = p.sorted[tile.begin + min((int)threadIdx.x, tile.n - 1)];
    __syncthreads();

    f16v y = {};
    const int row_l = 32 * wave + col;
    for (int c0 = 0; c0 < NB; c0 += PF_DCB) {
        const int cb = min(PF_DCB, NB - c0);           // blocks in this chunk
        if (c0) __syncthreads();
        constexpr int WCH = PF_WROW_DN / 16;
        for (int i = threadIdx.x; i < PF_ROWS * WCH; i += WG) {
            const int r = i / WCH, c = i - WCH * (i / WCH);
            const uint64_t rr = (uint64_t)min(r0 + r, D - 1);
            const uint64_t ps = rr * rb + (uint64_t)c0 * bs;
            if (c < chunk_count(ps, cb * bs))
                *reinterpret_cast<u32x4 *>(s_w + r * PF_WROW_DN + 16 * c) =
                    *reinterpret_cast<const u32x4 *>(W + (ps & ~(uint64_t)15) + 16 * c);
            if (c == 0) s_poff[r] = r * PF_WROW_DN + (int)(ps & 15);
        }
        const int xc = cb * 4;                          // 16-byte chunks per staged token row
        for (int i = threadIdx.x; i < PF_TOK * xc; i += WG) {
            const int j = i / xc, c = i - xc * (i / xc);
            const int64_t g = (int64_t)s_pair[j] * F + 32 * c0 + 8 * c;
            *reinterpret_cast<u32x4 *>(s_x + j * PF_DXS + 8 * c) = *reinterpret_cast<const u32x4 *>(p.ah + g);
            *reinterpret_cast<u32x4 *>(s_xl + j * PF_DXS + 8 * c) = *reinterpret_cast<const u32x4 *>(p.al + g);
        }
        __syncthreads();
        const uint8_t * wp = s_w + s_poff[row_l];
        const int xo = col * PF_DXS + 8 * half;
        const int nsteps = 2 * cb;
        for (int step = 0; step < nsteps; ++step) {
            h8 ah, al;
            if (wtype == T_Q5_0) q5_0_frag(wp + 22 * (step >> 1), 16 * (step & 1) + 8 * half, ah, al);
            else iq4nl_frag(wp + 18 * (step >> 1), 16 * (step & 1) + 8 * half, ah, al);
            const h8 bh = *reinterpret_cast<const h8 *>(s_x + xo + 16 * step);
            const h8 bl = *reinterpret_cast<const h8 *>(s_xl + xo + 16 * step);
            y = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bh, y, 0, 0, 0);
            y = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bl, y, 0, 0, 0);
            y = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, bh, y, 0, 0, 0);
        }
    }
    if (col < tile.n) {
        const int q = s_pair[col];
        const float sc = tile.tier == 0 ? (p.s_hot ? p.s_hot[tile.idx] : 1.0f) : (p.s_cold ? p.s_cold[tile.idx] : 1.0f);
        const float f = p.ae[q] * sc;
        float * out = p.ydn + (int64_t)q * D;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = r0 + 32 * wave + 8 * i + 4 * half;
            if (r + 3 < D)
                *reinterpret_cast<float4 *>(out + r) = make_float4(f * y[4 * i], f * y[4 * i + 1], f * y[4 * i + 2],
                                                                   f * y[4 * i + 3]);
        }
    }
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
