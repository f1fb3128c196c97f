// prefill.hip -- the MoE layer for long token batches (prefill chunks) on
// gfx950 int8 matrix cores (v_mfma_i32_16x16x64_i8).
//
//   k_pf_prep      one kernel for two independent jobs: its workgroup 0
//                  buckets, the others quantise the tokens.
//     pf_bucket    routed pairs grouped by expert (a counting sort with LDS
//                  atomics) and cut into groups two ways over the same sorted
//                  list: down groups of <= PF_TOK pairs and gate_up groups
//                  (their sizes set per tier by the host), each tagged with
//                  its tier by the residency predicate (ggml-cuda/mmid.cu:
//                  28-116 groups the same way; moert/cuda/ffn_moe.cu:80-130 is
//                  the predicate).
//     pf_quant_x   each token quantised once to q8_K (the CPU path's
//                  activation format for 256-blocks): int8 values, the
//                  per-256 scale, and the per-32 sums split as 32 hi + lo
//                  (both exact in fp16) for the Q4_K mins term
//                  (pf_quant_x1: q8_1, as exact fp16 parts).
//   k_pf_gate_up   grouped GEMM per (group, 64 gate rows + the 64 matching up
//                  rows), on groups of its own (<= 48 pairs of a Q4_K expert,
//                  <= 64 of an IQ2_S one), the full groups first, every row
//                  block of a group on one XCD.  Each super-block of weights
//                  is expanded once into int8 MFMA operands and used for
//                  every token of the group.  The sub-block scales are folded
//                  into the weights: Q4_K's 6-bit scale splits as 8 sh + sl,
//                  so q sh and q sl (<= 105) are int8 and two accumulators
//                  give sum_j sc_j dot_j exactly; IQ2_S's grid * (2 ls + 1)
//                  (<= 1333) splits as 64 h + l.  The Q4_K mins term is one
//                  exact fp16 MFMA against the split per-32 sums.  Scales
//                  d_w * d8 are applied once per super-block in fp32.  The
//                  load unit copies the next super-block's activations (and
//                  Q4_K rows) into LDS while the current one is used; IQ2_S
//                  rows go straight to registers.  The epilogue pairs gate
//                  row i with up row n_ff + i: GEGLU and the q8_0
//                  quantisation of the down activations happen here, so the
//                  gate_up outputs never go to memory; each down activation
//                  d8 q is stored exactly as two fp16 parts.
//   k_pf_gate_up_q1  the same GEMM in the q8_1 activation mode (fp16 MFMA).
//   k_pf_down      grouped GEMM of the down projection on fp16 MFMA
//                  (v_mfma_f32_16x16x32_f16, K = one 32-block): the weights as
//                  exact small integers (Q5_0 q - 16, IQ4_NL kvalues), the
//                  activations as the exact hi + lo parts of d8 q (two MFMAs
//                  into one fp32 accumulator), so the block's integer dot
//                  times d8 comes out of the matrix core and one fma per
//                  output applies the weight scale d_w.  Both operands carry a
//                  scale per 32-block here; on int8 MFMA every output would
//                  need a per-block fp32 rescale by d_w d8 (three VALU
//                  operations per output and block), which made that variant
//                  VALU-bound at several times this one's time.  K runs in
//                  chunks of two blocks, copied into LDS by the load unit one
//                  chunk ahead; every row block of a group on one XCD.
// The combine is the generic k_combine.
#include <hip/hip_ext.h>

#include <type_traits>

#include "device.h"
#include "launch.h"

namespace llapis {
namespace dev {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));

__constant__ Iq2sTables c_iq2s_tab_pf = make_iq2s_tables();

constexpr int PF_WROW_GU = 144;           // LDS pitch of a staged Q4_K super-block row

__device__ __forceinline__ v4i mfma_i8(v4i a, v4i b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f4 mfma_f16(h8 a, h8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v4i as_v4i(const u32x4 & u) {
    v4i v;
    __builtin_memcpy(&v, &u, 16);
    return v;
}
// four bytes (each < 16) times s (< 8) in one packed 16-bit multiply: every
// product stays below 256, so no byte carries into its neighbour
__device__ __forceinline__ uint32_t bytes_mul(uint32_t x, uint32_t s2) {
    u16x2 a, b;
    __builtin_memcpy(&a, &x, 4);
    __builtin_memcpy(&b, &s2, 4);
    const u16x2 c = a * b;
    uint32_t r;
    __builtin_memcpy(&r, &c, 4);
    return r;
}
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ h2 as_h2(uint32_t u) {
    h2 v;
    __builtin_memcpy(&v, &u, 4);
    return v;
}
__device__ __forceinline__ uint32_t h2bits(h2 v) {
    uint32_t u;
    __builtin_memcpy(&u, &v, 4);
    return u;
}
// four small unsigned bytes -> two packed fp16 pairs of (1024 + byte):
// bytes {0, 1} and {2, 3}
__device__ __forceinline__ uint32_t magic_lo(uint32_t x) { return __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u); }
__device__ __forceinline__ uint32_t magic_hi(uint32_t x) { return __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u); }

__device__ __forceinline__ bool tile_valid(const PfParams & p, const PfTile & t) {
    return (t.tier == 0 && t.idx >= 0 && t.idx < p.k_slots) || (t.tier == 1 && t.idx >= 0 && t.idx < p.n_expert);
}

// ------------------------------------------------------------ IQ2_S tables

// For a 4-bit IQ2_S scale ls: the three grid magnitudes {8, 25, 43} times
// (2 ls + 1), each split as 64 h + l (h <= 20, l < 64), as the byte tables a
// v_perm selector code | 4 sign picks from: {h+, h-, l+, l-}, bytes 0..2 for
// codes 0..2 and byte 3 zero.
struct Iq2sSplit {
    uint32_t t[16][4];
};
constexpr Iq2sSplit make_iq2s_split() {
    Iq2sSplit s{};
    const int lev[3] = {8, 25, 43};
    for (int ls = 0; ls < 16; ++ls) {
        uint32_t hp = 0, hn = 0, lp = 0, ln = 0;
        for (int c = 0; c < 3; ++c) {
            const int w = lev[c] * (2 * ls + 1);
            const int h = w >> 6, l = w & 63;
            hp |= (uint32_t)(h & 0xFF) << (8 * c);
            hn |= (uint32_t)((-h) & 0xFF) << (8 * c);
            lp |= (uint32_t)(l & 0xFF) << (8 * c);
            ln |= (uint32_t)((-l) & 0xFF) << (8 * c);
        }
        s.t[ls][0] = hp;
        s.t[ls][1] = hn;
        s.t[ls][2] = lp;
        s.t[ls][3] = ln;
    }
    return s;
}
__constant__ Iq2sSplit c_iq2s_split = make_iq2s_split();

// ----------------------------------------------------------------- bucket

// One workgroup.  P = T * top_k <= PF_MAX_PAIRS, n_expert <= 256.  A
// counting sort by expert with LDS atomics: counts, an exclusive scan over
// the experts (pair offsets and group offsets), then each pair takes the
// next slot of its expert.  The order of pairs inside an expert's range is
// not fixed, and need not be: each pair's output column is computed on its
// own.
__device__ __forceinline__ void pf_bucket(const PfParams & p) {
    constexpr int PER = PF_MAX_PAIRS / WG;
    __shared__ int s_cnt[257], s_fill[257], s_off[257], s_nt[257], s_gf[256], s_gr[256], s_hot;
    const int P = p.T * p.top_k, E = p.n_expert;
    __shared__ int s_se[256], s_ss[256];
    int ev[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int q = threadIdx.x + WG * k;
        const int v = q < P ? p.ids[q] : -1;
        ev[k] = (v >= 0 && v < E) ? v : 256;     // 256: invalid id
    }
    // the residency mirrors in the same round of loads (a thread per expert
    // and per slot), looked up in LDS
    const int e0 = threadIdx.x, ks = p.k_slots;
    const int sl = ks > 0 && e0 < E ? p.exp_slot[e0] : -1;
    if (ks > 0 && e0 < ks) {
        s_se[e0] = p.slot_exp[e0];
        s_ss[e0] = p.slot_state[e0];
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
    int n_e = 0, tier = 1, idx = e0;
    if (e0 < E) {
        n_e = s_cnt[e0];
        if (sl >= 0 && sl < ks && s_ss[sl] == 2 && s_se[sl] == e0) {
            tier = 0;
            idx = sl;
        }
    }
    const int nt_e = (n_e + PF_TOK - 1) / PF_TOK;
    // gate_up groups: full groups of gcap pairs, then one remainder group
    const int gcap = max(16, min(PF_GTOK, p.gcap[tier]));
    const int gf_e = n_e / gcap, gr_e = n_e - gf_e * gcap > 0 ? 1 : 0;
    if (p.rc_counts) {
        // routing counters (ffn_moe.cu:123-128): pairs per expert, hot pairs,
        // the other pairs (invalid ids included)
        if (n_e) atomicAdd(p.rc_counts + e0, n_e);
        const int hot = tier == 0 ? n_e : 0;
        if (hot) atomicAdd(&s_hot, hot);
    }
    s_off[threadIdx.x] = n_e;
    s_nt[threadIdx.x] = nt_e;
    s_gf[threadIdx.x] = gf_e;
    s_gr[threadIdx.x] = gr_e;
    __syncthreads();
    for (int o = 1; o < 256; o <<= 1) {          // inclusive scans over the experts
        const int a = threadIdx.x >= o ? s_off[threadIdx.x - o] : 0;
        const int b = threadIdx.x >= o ? s_nt[threadIdx.x - o] : 0;
        const int c = threadIdx.x >= o ? s_gf[threadIdx.x - o] : 0;
        const int d = threadIdx.x >= o ? s_gr[threadIdx.x - o] : 0;
        __syncthreads();
        s_off[threadIdx.x] += a;
        s_nt[threadIdx.x] += b;
        s_gf[threadIdx.x] += c;
        s_gr[threadIdx.x] += d;
        __syncthreads();
    }
    const int pair0 = s_off[threadIdx.x] - n_e, tile0 = s_nt[threadIdx.x] - nt_e;
    const int total = s_off[255], tiles = min(s_nt[255], p.max_tiles);
    const int nfull = s_gf[255], gf0 = s_gf[threadIdx.x] - gf_e, gr0 = nfull + s_gr[threadIdx.x] - gr_e;
    for (int b = 0; b <= gf_e; ++b) {
        const int gi = b < gf_e ? gf0 + b : gr0;
        if ((b == gf_e && !gr_e) || gi >= p.max_gtiles) continue;
        PfTile t;
        t.tier = tier;
        t.idx = idx;
        t.begin = pair0 + b * gcap;
        t.n = min(gcap, n_e - b * gcap);
        p.gtiles[gi] = t;
    }
    if (p.rc_hits && threadIdx.x == 0) {
        atomicAdd(p.rc_hits, s_hot);
        atomicAdd(p.rc_hits + 1, P - s_hot);
    }
    __syncthreads();
    s_off[threadIdx.x] = pair0;
    if (threadIdx.x == 0) {
        s_off[256] = total;                     // invalid ids are placed after every expert's pairs
        *p.n_tiles = tiles;
        *p.n_gtiles = min(nfull + s_gr[255], p.max_gtiles);
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
    // a pair with an invalid id is in no group: it contributes zeros to the combine
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int q = threadIdx.x + WG * k;
        if (q < P && ev[k] == 256)
            for (int r = 0; r < p.d_model; ++r) p.ydn[(int64_t)q * p.d_model + r] = 0.0f;
    }
}

// ------------------------------------------------------------ token quant

// One wave per (token, 256-block): q8_K exactly as the CPU path; the int8
// values, the scale, and the 8 per-32 sums as {hi_0..hi_7, lo_0..lo_7} with
// sum = 32 hi + lo, 0 <= lo < 32 (each part exact in fp16).
__device__ __forceinline__ void pf_quant_x(const PfParams & p, int blk) {
    __shared__ __align__(16) uint8_t scratch[WG / 64][512];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int NSB = p.d_model / 256;
    const int job = blk * (WG / 64) + wave;
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
    if (lane < 16)
        *reinterpret_cast<u32x4 *>(p.xq + (int64_t)t * p.d_model + 256 * s + 16 * lane) =
            reinterpret_cast<const u32x4 *>(base + L.q)[lane];
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

// One wave per (token, 64 values): q8_1 of two 32-blocks as ggml-cuda's
// quantize_q8_1 computes it (quantize.cu:5-50: d = amax / 127, q =
// roundf(x / d), d kept as fp16), stored for the fp16 matrix cores: each
// value d q (at most 19 significant bits) as its exact fp16 hi + lo parts,
// [token][256-block] {256 hi, 256 lo}; and per 32-block u = d sum(q) (the
// Q4_K mins term of vecdotq.cuh's q4_K . q8_1) as exact hi + lo,
// [token][256-block] {hi_0..hi_7, lo_0..lo_7}.
__device__ __forceinline__ void pf_quant_x1(const PfParams & p, int blk) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int D = p.d_model, per = D / 64;
    const int job = blk * (WG / 64) + wave;
    if (job >= p.T * per) return;                        // whole waves leave
    const int t = job / per, pos = 64 * (job - t * per) + lane;
    const float v = p.x[(int64_t)t * D + pos];
    const float amax = half_max_dpp(fabsf(v));
    const float d = amax / 127.0f;
    const int qi = amax == 0.0f ? 0 : (int)roundf(v / d);
    const float dstore = (float)(_Float16)d;
    const float xv = dstore * (float)qi;                // exact
    const _Float16 xh = (_Float16)xv;
    const _Float16 xl = (_Float16)(xv - (float)xh);     // exact
    int sq = qi;
    for (int o = 16; o >= 1; o >>= 1) sq += __shfl_xor(sq, o, 32);
    const int sb = pos >> 8, k = pos & 255;
    _Float16 * row = p.xh + ((int64_t)t * (D / 256) + sb) * 512;
    row[k] = xh;
    row[256 + k] = xl;
    if ((lane & 31) == 0) {
        const int j = k >> 5;
        const float u = dstore * (float)sq;             // exact: 11 x 13 bits
        const _Float16 h = (_Float16)u;
        const _Float16 l = (_Float16)(u - (float)h);
        _Float16 * xm = p.xm + ((int64_t)t * (D / 256) + sb) * 16;
        xm[j] = h;
        xm[8 + j] = l;
    }
}

// Workgroup 0 buckets the pairs; the others quantise the tokens (neither
// depends on the other), so the quantisation runs while the one bucketing
// workgroup does and the chunk has one kernel boundary fewer.
template <int AM>
__global__ __launch_bounds__(WG) void k_pf_prep(const PfParams p) {
    if (blockIdx.x == 0) pf_bucket(p);
    else if (AM == AM_Q8_1) pf_quant_x1(p, blockIdx.x - 1);
    else pf_quant_x(p, blockIdx.x - 1);
}

// -------------------------------------------------------------- gate_up

// the epilogue's staging of one 16-token tile: [128 rows][17]
constexpr int GU_STP = 17;
constexpr int GU_WREG = 5;     // weight chunks per thread per super-block (q8_1 kernel; 128 rows x 9)

// q8_0 (x86 CPU build, arch/x86/quants.c:302-360) or q8_1 (ggml-cuda
// quantize.cu:5-50) of one 32-block held one value per lane of a half-wave,
// stored as the value d8 q, exactly, in two fp16 parts: d8 (fp16) times q
// (8 bits) has at most 19 significant bits and is a multiple of 2^-24, so
// hi = fp16(d8 q) and lo = fp16(d8 q - hi) are exact and hi + lo = d8 q.
// (q8_1 also stores its per-block sum s.)
template <int AM>
__device__ __forceinline__ void q8_store32(float v, _Float16 * hi, _Float16 * lo, float * s, bool live) {
    const float amax = half_max_dpp(fabsf(v));
    int qi;
    float dstore, sstore = 0.0f;
    if (AM == AM_CPU) {
        const float dd = amax / 127.f;
        const float id = amax != 0.0f ? 127.f / amax : 0.0f;
        qi = (int)rintf(__fmul_rn(v, id));
        qi = qi > 127 ? 127 : (qi < -128 ? -128 : qi);
        dstore = round_to_half(dd);
    } else {
        float sm = v;
        for (int o = 16; o >= 1; o >>= 1) sm = __fadd_rn(sm, __shfl_xor(sm, o, 32));
        const float dd = amax / 127.0f;
        qi = amax == 0.0f ? 0 : (int)roundf(v / dd);
        dstore = round_to_half(dd);
        sstore = round_to_half(sm);
    }
    const float x = dstore * (float)qi;                 // exact
    const _Float16 h = (_Float16)x;
    const _Float16 l = (_Float16)(x - (float)h);       // exact
    if (live) {
        *hi = h;
        *lo = l;
        if (AM != AM_CPU && s && (threadIdx.x & 31) == 0) *s = sstore;
    }
}

// ------------------------------------------------------ gate_up, q8_K
//
// One workgroup per (gate_up group, 64 gate rows + the 64 matching up rows).
// Wave w owns local rows 32 w .. 32 w + 31 (waves 0, 1: gate rows; 2, 3: the
// up rows of the same indices) as two 16-row MFMA tiles.  The load unit
// copies the group's activations of the next super-block (and the Q4_K rows)
// into LDS (global_load_lds) while the current one is expanded and used;
// IQ2_S rows go straight to registers with buffer loads, as their 82-byte
// super-blocks are not 16-byte aligned.  Two buffers of each kind, so one
// barrier per super-block both publishes super-block s and retires s - 1.
// A token's 16-byte chunk c of a super-block sits in slot c ^ (token & 15)
// of its 256-byte LDS row: the 16 tokens of an MFMA fragment read 16
// distinct slots, so the fragment loads meet no bank conflict.

constexpr int G2_TOKQ4 = 48;            // pairs per group of a Q4_K expert (at 64 the kernel spills registers)
constexpr int G2_TOKIQ2 = 64;           // of an IQ2_S expert (its tables share the LDS)
static_assert(G2_TOKQ4 <= PF_GTOK && G2_TOKIQ2 <= PF_GTOK, "group caps");
constexpr int G2_TOKMAX = G2_TOKQ4 > G2_TOKIQ2 ? G2_TOKQ4 : G2_TOKIQ2;
constexpr int G2_MBT = (G2_TOKQ4 + 31) / 32 * 32;     // tokens of a mins buffer: 32 per moving wave

// LDS of one workgroup.  Each of the two buffers of a kind is a separate
// object: the compiler then knows that a copy into one does not write the
// other, and it does not make reads of the current buffer wait for the copy
// of the next.  The epilogue stages gate rows in x0 and up rows in x1
// ([64 rows][NTOK + 1] floats each); the IQ2_S tables live in w0 / w1 (that
// format's rows go straight to registers).
constexpr int G2_XB = 64 * (G2_TOKMAX + 1) * 4;
constexpr int G2_WB = PF_ROWS * 144;                      // one super-block of 128 Q4_K rows
static_assert(G2_XB >= G2_TOKQ4 * 256 && G2_XB >= G2_TOKIQ2 * 256, "activation buffers");
static_assert(G2_WB >= 1024 * 8 && G2_WB >= 16 * 16, "IQ2_S tables fit the weight buffers");
struct Gu2Lds {
    uint8_t * x0; uint8_t * x1;                   // the group's q8_K values of one super-block
    uint8_t * w0; uint8_t * w1;                   // Q4_K: the 128 rows of one super-block, [row][144]
    _Float16 * mb0; _Float16 * mb1;               // their per-32 sums (32 hi + lo), Q4_K
    float * d80; float * d81;                     // their q8_K scales
    uint2 * codes;                                // IQ2_S grid: a level code per value (in w0)
    u32x4 * split;                                // Iq2sSplit (in w1)
    int * tok; int * pair;
};

// one lane's bytes of one IQ2_S super-block of a 16-row tile
struct Iq2Raw {
    uint32_t d;                 // dword holding d
    u32x3 qs;                   // three dwords holding qs[8 q .. 8 q + 7]
    u32x3 sg;                   //          ... and the signs
    uint32_t qh, sc;            // dwords holding qh[2 q, 2 q + 1], scales[2 q, 2 q + 1]
    int sh_d, sh_q, sh_h;       // byte shifts of those fields in their dwords
};

// IQ2_S super-blocks are 82 bytes, so a field is 2-aligned: each is read
// from the dword-aligned address at or below it and shifted into place.
// Super-block s of a row starts at row_start + 82 s, which is
// 2 (rowpar + s) mod 4 (rowpar: row_start mod 4, halved).
__device__ __forceinline__ void iq2_raw_load(Iq2Raw & w, __amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t rowpar,
                                             int s, int q) {
    const uint32_t a = ((rowpar + (uint32_t)s) & 1u) * 2u;      // super-block start mod 4
    const uint32_t aq = a ^ 2u;                                  // qs, signs: start + 2 + 8 q
    const uint32_t ah = (a + 2u + 2u * (uint32_t)q) & 2u;       // qh, scales: start + 66 / 74 + 2 q
    // every offset is taken in the lane's register (>= 0), none in soffset
    const uint32_t v0 = voff + 82u * (uint32_t)s;
    w.d = __builtin_amdgcn_raw_buffer_load_b32(r, v0 - a, 0, 0);
    const uint32_t vq = v0 + 2 + 8 * (uint32_t)q - aq;
    w.qs = __builtin_amdgcn_raw_buffer_load_b96(r, vq, 0, 0);
    w.sg = __builtin_amdgcn_raw_buffer_load_b96(r, vq + 32, 0, 0);
    const uint32_t vh = v0 + 66 + 2 * (uint32_t)q - ah;
    w.qh = __builtin_amdgcn_raw_buffer_load_b32(r, vh, 0, 0);
    w.sc = __builtin_amdgcn_raw_buffer_load_b32(r, vh + 8, 0, 0);
    w.sh_d = 8 * (int)a;
    w.sh_q = 8 * (int)aq;
    w.sh_h = 8 * (int)ah;
}

// The v_perm sign picks of 8 IQ2_S values from their sign byte (bits b ..
// b + 7 of w): bit 2 of byte k set when value k is negative.  A 4-bit
// nibble times 0x810204 = 2^2 + 2^9 + 2^16 + 2^23 puts its bit k at bit
// 8 k + 2 (the four shifted copies do not overlap, so nothing carries).
__device__ __forceinline__ uint2 sign_sel(uint32_t w, int b) {
    const uint32_t lo = __builtin_amdgcn_ubfe(w, b, 4), hi = __builtin_amdgcn_ubfe(w, b + 4, 4);
    return make_uint2((lo * 0x810204u) & 0x04040404u, (hi * 0x810204u) & 0x04040404u);
}

// Table-mode GEGLU (geglu1) in two steps, so that a lane's table reads can
// all be in flight at once: the entry at fp16(g) (index clamped, read
// unconditionally), then the clamps at -10 and 10 and the product.
__device__ __forceinline__ uint32_t gelu_entry(float g) {
    const uint32_t h = __builtin_bit_cast(uint16_t, (_Float16)g);
    const uint32_t mag = min(h & 0x7FFFu, (uint32_t)LLAPIS_GELU_TAB_SPAN - 1u);
    return gelu_f16_table[mag + (h >> 15) * LLAPIS_GELU_TAB_SPAN];
}
__device__ __forceinline__ float geglu_from_entry(float g, float u, uint32_t e) {
    const float t = __fmul_rn((float)__builtin_bit_cast(_Float16, (uint16_t)e), u);
    return g <= -10.0f ? 0.0f : (g >= 10.0f ? __fmul_rn(g, u) : t);
}

template <int WT, int GSRC, int NT>
__device__ __forceinline__ void pf_gu2_group(const PfParams & p, const PfTile & tile, const Gu2Lds & L, const int rb) {
    constexpr bool Q4 = WT == T_Q4_K;
    static_assert(Q4 || WT == T_IQ2_S, "gate_up formats");
    constexpr int NTOK = 16 * NT;
    static_assert(NTOK <= (Q4 ? G2_TOKQ4 : G2_TOKIQ2), "group fits the LDS");
    constexpr int BB = Q4 ? 144 : 82;                           // bytes per super-block
    const int F = p.n_ff, NSB = p.d_model / 256, K = p.top_k, D = p.d_model;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, q = lane >> 4, l16 = lane & 15;
    const uint32_t rbytes = (uint32_t)(NSB * BB);
    const uint8_t * W = tile.tier == 0 ? p.hot_gu + (uint64_t)tile.idx * p.hot_gu_stride
                                       : p.cold_gu + (uint64_t)tile.idx * p.cold_gu_stride;
    const uint32_t slab = (uint32_t)(2u * (uint32_t)F * rbytes);
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(W), 0, (int)slab,
                                                                         0x00020000);
    if (tid < NTOK) {
        const int qp = p.sorted[tile.begin + min(tid, tile.n - 1)];
        L.pair[tid] = qp;
        L.tok[tid] = qp / K;
    }
    if (!Q4) {
        const u32x4 * src = reinterpret_cast<const u32x4 *>(&c_iq2s_tab_pf);
        u32x4 * dst = reinterpret_cast<u32x4 *>(L.codes);
        for (int i = tid; i < 1024 * 8 / 16; i += WG) dst[i] = src[i];
        if (tid < 16) {
            const uint32_t * t = c_iq2s_split.t[tid];
            L.split[tid] = u32x4{t[0], t[1], t[2], t[3]};
        }
    }
    __syncthreads();

    // ---- copies into LDS: wave w moves token blocks 4 (w NT + i) .. + 3 (16
    // lanes a token, lane slot i ^ token), the mins sums of 32 tokens (wave <
    // ceil(NT / 2), Q4_K) and the scales of 64 tokens (wave < ceil(NT / 4))
    const bool mb_mover = Q4 && 32 * wave < NTOK, d8_mover = 64 * wave < NTOK;
    // Q4_K rows: 128 rows x 9 chunks of one super-block, [row][144] in LDS;
    // copy j (0..17, wave w takes j = w, w + 4, ...) moves chunks 64 j .. + 63
    auto wrow_off = [&](int j) {
        const int i = 64 * j + lane, r = i / 9, c = i - 9 * r;
        const int gi = min(64 * rb + (r & 63), F - 1);
        return (uint32_t)(r < 64 ? gi : F + gi) * rbytes + 16u * (uint32_t)c;
    };
    auto copy_in = [&](int s, uint8_t * xb, _Float16 * mbb, float * d8b, uint8_t * wb) {
        if constexpr (Q4) {
            const uint8_t * wsb = W + 144 * s;
            asm volatile("" : "+s"(wsb));
#pragma unroll
            for (int k = 0; k < 5; ++k) {
                const int j = wave + 4 * k;
                if (j < 18) lds_dma16(wsb + wrow_off(j), wb + 1024 * j);
            }
        }
        // the super-block's offsets are made opaque, so that the compiler
        // keeps one uniform base per copy (an SGPR pair) and the lanes' 32-bit
        // offsets (recomputed from the token list: no registers held)
        const uint8_t * xs = reinterpret_cast<const uint8_t *>(p.xq) + 256 * s;
        const uint8_t * ms = reinterpret_cast<const uint8_t *>(p.xm) + 32 * s;
        const uint8_t * ds = reinterpret_cast<const uint8_t *>(p.xd) + 4 * s;
        asm volatile("" : "+s"(xs), "+s"(ms), "+s"(ds));
#pragma unroll
        for (int i = 0; i < NT; ++i) {
            const int t = 4 * (wave * NT + i) + (lane >> 4);
            const int c = (lane & 15) ^ (t & 15);
            lds_dma16(xs + (uint32_t)(L.tok[t] * D + 16 * c), xb + 1024 * (wave * NT + i));
        }
        if (mb_mover) {
            const int t = min(32 * wave + (lane >> 1), NTOK - 1);
            lds_dma16(ms + (uint32_t)(L.tok[t] * NSB * 32 + 16 * (lane & 1)), mbb + 16 * 32 * wave);
        }
        if (d8_mover) lds_dma4(ds + (uint32_t)(L.tok[min(64 * wave + lane, NTOK - 1)] * NSB * 4), d8b + 64 * wave);
    };

    // ---- this lane's rows: local row 32 wave + 16 rs + l16 is gate row
    // 64 rb + r (r < 64) or up row F + 64 rb + r - 64, clamped into the slab
    // (rows past n_ff are computed and discarded)
    uint32_t voff[2], rowpar[2];
#pragma unroll
    for (int rs = 0; rs < 2; ++rs) {
        const int r = 32 * wave + 16 * rs + l16;
        const int gi = min(64 * rb + (r & 63), F - 1);
        const int row = r < 64 ? gi : F + gi;
        voff[rs] = (uint32_t)row * rbytes;
        rowpar[rs] = (voff[rs] >> 1) & 1u;                      // row start mod 4, halved (slabs are 16-aligned)
    }
    Iq2Raw wi[Q4 ? 1 : 2];
    auto load_rows = [&](int s) {
        if constexpr (!Q4) {
#pragma unroll
            for (int rs = 0; rs < 2; ++rs) iq2_raw_load(wi[rs], wr, voff[rs], rowpar[rs], s, q);
        }
    };

    f4 y[2][NT];
#pragma unroll
    for (int rs = 0; rs < 2; ++rs)
#pragma unroll
        for (int ts = 0; ts < NT; ++ts) y[rs][ts] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    // per-lane constants of the Q4_K expansion: the byte of this lane's
    // sub-block scale in both 16-bit halves (sub-block 2 st + q / 2: byte
    // q / 2 for even st, 2 + q / 2 for odd), the nibble, and the mins
    // operand's (1024 + m) * mult + off (32 m, m or 0 by quarter)
    const uint32_t jb_e = (uint32_t)(q >> 1), jb_o = 2u + (uint32_t)(q >> 1);
    const uint32_t sel_even = jb_e | 0x0C00u | (jb_e << 16) | 0x0C000000u;
    const uint32_t sel_odd = jb_o | 0x0C00u | (jb_o << 16) | 0x0C000000u;
    const uint32_t nib_shift = 4u * (uint32_t)(q >> 1);
    const _Float16 mm = q == 0 ? (_Float16)32.0f : q == 1 ? (_Float16)1.0f : (_Float16)0.0f;
    const _Float16 mo = q == 0 ? (_Float16)(-32768.0f) : q == 1 ? (_Float16)(-1024.0f) : (_Float16)0.0f;
    const h2 mn_mul = h2{mm, mm}, mn_off = h2{mo, mo};

    // One super-block, K-slice major: the rows' per-super-block words (scales,
    // mins, IQ2_S index and sign words) first, then the next super-block's
    // copies and rows, then for each K-slice st (64 values) the expansion of
    // both row tiles' slice and the MFMAs of every 16-token tile against it,
    // into int32 accumulators that live across the slices -- so one slice's
    // expansion (VALU) overlaps the previous slice's MFMAs -- and last the
    // per-output scaling of every tile.
    auto step = [&](int s, const uint8_t * xb, const _Float16 * mbb, const float * d8b, const uint8_t * wb,
                    uint8_t * xn, _Float16 * mbn, float * d8n, uint8_t * wn) {
        // this wave's copies and rows of super-block s have landed; after the
        // barrier every wave's have, and every wave is done with s - 1
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();

        // ---- per row tile: Q4_K lane (row l16, quarter q) takes values 64 st
        // + 16 q of slice st (sub-block 2 st + q / 2); IQ2_S the 16-value group
        // 4 q + st.  The activations are read in the same order.  The
        // sub-block scales are folded in: Q4_K's 6-bit scale as 8 sh + sl
        // (q sh, q sl <= 105), IQ2_S's grid (2 ls + 1) as 64 h + l.
        float dr[2], mr[2];
        uint32_t sh03[2], sl03[2], sh47[2], sl47[2];         // Q4_K
        uint2 qs8[2], sg8[2];                                // IQ2_S
        uint32_t qh2[2], sc2[2];
        h8 bm[2];
#pragma unroll
        for (int rs = 0; rs < 2; ++rs) {
            if constexpr (Q4) {
                const uint8_t * wrw = wb + (32 * wave + 16 * rs + l16) * 144;
                const u32x4 hdr = *reinterpret_cast<const u32x4 *>(wrw);
                dr[rs] = h2f(hdr.x & 0xFFFF);
                mr[rs] = h2f(hdr.x >> 16);
                // 6-bit scales and mins, four per dword (get_scale_min_k4,
                // ggml-quants.c:822): bytes j of sc03 / mn03 for j < 4, of
                // sc47 / mn47 for j - 4
                const uint32_t sc03 = hdr.y & 0x3F3F3F3Fu;
                const uint32_t mn03 = hdr.z & 0x3F3F3F3Fu;
                const uint32_t sc47 = (hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u);
                const uint32_t mn47 = ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u);
                sh03[rs] = (sc03 >> 3) & 0x07070707u; sl03[rs] = sc03 & 0x07070707u;
                sh47[rs] = (sc47 >> 3) & 0x07070707u; sl47[rs] = sc47 & 0x07070707u;
                // mins B operand (16x16x32 f16): k 0..7 = 32 m_j, 8..15 = m_j,
                // 16..31 = 0; (1024 + m) * mult + off per lane quarter
                const uint32_t mb4[4] = {magic_lo(mn03), magic_hi(mn03), magic_lo(mn47), magic_hi(mn47)};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const h2 mv = __builtin_elementwise_fma(as_h2(mb4[i]), mn_mul, mn_off);
                    bm[rs][2 * i] = mv.x;
                    bm[rs][2 * i + 1] = mv.y;
                }
            } else {
                const Iq2Raw & w = wi[rs];
                dr[rs] = h2f((w.d >> w.sh_d) & 0xFFFFu);
                mr[rs] = 0.0f;
                // this lane's groups 4q .. 4q + 3: grid entries 8q .. 8q + 7
                qs8[rs] = make_uint2(__builtin_amdgcn_alignbit(w.qs.y, w.qs.x, w.sh_q),
                                     __builtin_amdgcn_alignbit(w.qs.z, w.qs.y, w.sh_q));
                sg8[rs] = make_uint2(__builtin_amdgcn_alignbit(w.sg.y, w.sg.x, w.sh_q),
                                     __builtin_amdgcn_alignbit(w.sg.z, w.sg.y, w.sh_q));
                qh2[rs] = (w.qh >> w.sh_h) & 0xFFFFu;               // 2 bits per entry
                sc2[rs] = (w.sc >> w.sh_h) & 0xFFFFu;               // 4 bits per group
#pragma unroll
                for (int j = 0; j < 8; ++j) bm[rs][j] = (_Float16)0.0f;
            }
        }

        // ---- the next super-block in flight during this one's MFMAs
        if (s + 1 < NSB) {
            copy_in(s + 1, xn, mbn, d8n, wn);
            load_rows(s + 1);
        }

        // ---- slice by slice: expand, then every tile's MFMAs
        v4i ah[2][NT], al[2][NT];
#pragma unroll
        for (int rs = 0; rs < 2; ++rs)
#pragma unroll
            for (int ts = 0; ts < NT; ++ts) {
                ah[rs][ts] = v4i{0, 0, 0, 0};
                al[rs][ts] = v4i{0, 0, 0, 0};
            }
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            v4i bh[2], bl[2];
#pragma unroll
            for (int rs = 0; rs < 2; ++rs) {
                if constexpr (Q4) {
                    const uint8_t * wrw = wb + (32 * wave + 16 * rs + l16) * 144;
                    const u32x4 v = *reinterpret_cast<const u32x4 *>(wrw + 16 + 32 * st + 16 * (q & 1));
                    const uint32_t sel = (st & 1) ? sel_odd : sel_even;
                    const uint32_t sh2 = __builtin_amdgcn_perm(0u, st < 2 ? sh03[rs] : sh47[rs], sel);
                    const uint32_t sl2 = __builtin_amdgcn_perm(0u, st < 2 ? sl03[rs] : sl47[rs], sel);
                    const uint32_t w4v[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t nb = (w4v[i] >> nib_shift) & 0x0F0F0F0Fu;
                        bh[rs][i] = (int)bytes_mul(nb, sh2);
                        bl[rs][i] = (int)bytes_mul(nb, sl2);
                    }
                } else {
                    const uint32_t qsw = st < 2 ? qs8[rs].x : qs8[rs].y, sgw = st < 2 ? sg8[rs].x : sg8[rs].y;
                    const int b0 = 16 * (st & 1);                       // bit of entry 2 st in its dword
                    const uint32_t i0 = __builtin_amdgcn_ubfe(qsw, b0, 8) | (__builtin_amdgcn_ubfe(qh2[rs], 4 * st, 2) << 8);
                    const uint32_t i1 = __builtin_amdgcn_ubfe(qsw, b0 + 8, 8) | (__builtin_amdgcn_ubfe(qh2[rs], 4 * st + 2, 2) << 8);
                    const uint2 c0 = L.codes[i0], c1 = L.codes[i1];
                    const uint2 s0 = sign_sel(sgw, b0), s1 = sign_sel(sgw, b0 + 8);
                    const u32x4 t = L.split[__builtin_amdgcn_ubfe(sc2[rs], 4 * st, 4)];
                    const uint32_t sel[4] = {c0.x | s0.x, c0.y | s0.y, c1.x | s1.x, c1.y | s1.y};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        bh[rs][i] = (int)__builtin_amdgcn_perm(t.y, t.x, sel[i]);
                        bl[rs][i] = (int)__builtin_amdgcn_perm(t.w, t.z, sel[i]);
                    }
                }
            }
#pragma unroll
            for (int ts = 0; ts < NT; ++ts) {
                const uint8_t * xr = xb + (16 * ts + l16) * 256;
                const int c = Q4 ? q + 4 * st : 4 * q + st;
                const v4i a = as_v4i(*reinterpret_cast<const u32x4 *>(xr + 16 * (c ^ l16)));
#pragma unroll
                for (int rs = 0; rs < 2; ++rs) {
                    ah[rs][ts] = mfma_i8(a, bh[rs], ah[rs][ts]);
                    al[rs][ts] = mfma_i8(a, bl[rs], al[rs][ts]);
                }
            }
        }

        // ---- every tile's per-output scaling.  Explicit fmas: every token
        // column rounds alike.  A pair's column in its group depends on the
        // bucketing order, and left to itself the compiler contracts some
        // unrolled columns into an fma and not others.
#pragma unroll
        for (int ts = 0; ts < NT; ++ts) {
            const f4 d8 = *reinterpret_cast<const f4 *>(d8b + 16 * ts + 4 * q);
            h8 am;
            if constexpr (Q4) {
                // every lane loads (no branch); quarters 2, 3 are zeroed
                u32x4 mv = *reinterpret_cast<const u32x4 *>(mbb + 16 * (16 * ts + l16) + 8 * (q & 1));
                const uint32_t keep = q < 2 ? ~0u : 0u;
                mv.x &= keep; mv.y &= keep; mv.z &= keep; mv.w &= keep;
                __builtin_memcpy(&am, &mv, 16);
            }
#pragma unroll
            for (int rs = 0; rs < 2; ++rs) {
                if constexpr (Q4) {
                    const f4 m = mfma_f16(am, bm[rs], f4{0.0f, 0.0f, 0.0f, 0.0f});
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float sf = (float)(8 * ah[rs][ts][r] + al[rs][ts][r]);
                        const float t = __builtin_fmaf(dr[rs], sf, -(mr[rs] * m[r]));
                        y[rs][ts][r] = __builtin_fmaf(d8[r], t, y[rs][ts][r]);
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float sf = (float)(64 * ah[rs][ts][r] + al[rs][ts][r]);
                        y[rs][ts][r] = __builtin_fmaf(d8[r], dr[rs] * sf, y[rs][ts][r]);
                    }
                }
            }
        }
    };

    copy_in(0, L.x0, L.mb0, L.d80, L.w0);
    load_rows(0);
    for (int s = 0; s < NSB; s += 2) {
        step(s, L.x0, L.mb0, L.d80, L.w0, L.x1, L.mb1, L.d81, L.w1);
        if (s + 1 < NSB) step(s + 1, L.x1, L.mb1, L.d81, L.w1, L.x0, L.mb0, L.d80, L.w0);
    }

    // ---- epilogue: every tile's outputs into LDS at once (gate rows in x0,
    // up rows in x1: [64 rows][NTOK + 1]), then per (token, 32-block) unit --
    // one per half-wave and pass -- GEGLU of gate row i and up row i and q8_0
    // of the 32 results into the pair's down activations.  A lane reads all
    // its units' values and GEGLU table entries before it uses the first.
    constexpr int SP = NTOK + 1;
    constexpr int NU = NTOK / 4;                                // units per half-wave
    const float f = Q4 ? 1.0f : 0.125f;
    float * sg = reinterpret_cast<float *>(L.x0);
    float * su = reinterpret_cast<float *>(L.x1);
    __syncthreads();                                            // the K loop's readers are done
    {
        float * dst = wave < 2 ? sg : su;
#pragma unroll
        for (int ts = 0; ts < NT; ++ts)
#pragma unroll
            for (int rs = 0; rs < 2; ++rs)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    dst[(32 * (wave & 1) + 16 * rs + l16) * SP + 16 * ts + 4 * q + r] = f * y[rs][ts][r];
    }
    __syncthreads();
    const int hw = 2 * wave + (lane >> 5), i = lane & 31;
    float gv[NU], uv[NU];
    uint32_t te[NU];
#pragma unroll
    for (int k = 0; k < NU; ++k) {
        const int u = 8 * k + hw, j = u >> 1, blk = u & 1;
        gv[k] = sg[(32 * blk + i) * SP + j];
        uv[k] = su[(32 * blk + i) * SP + j];
    }
    if constexpr (GSRC == SRC_GEGLU_TABLE) {
#pragma unroll
        for (int k = 0; k < NU; ++k) te[k] = gelu_entry(gv[k]);
    }
#pragma unroll
    for (int k = 0; k < NU; ++k) {
        const int u = 8 * k + hw, j = u >> 1, blk = u & 1;
        const int fi = 64 * rb + 32 * blk;                      // first gate index of the block
        const bool live = j < tile.n && fi < F;
        const int64_t qp = L.pair[j];
        const float v = GSRC == SRC_GEGLU_TABLE ? geglu_from_entry(gv[k], uv[k], te[k]) : geglu1<GSRC>(gv[k], uv[k]);
        q8_store32<AM_CPU>(v, p.ah + qp * F + fi + i, p.al + qp * F + fi + i, nullptr, live);
    }
}

// Grid: 8 x ceil(max_tiles / 8) x RB workgroups in one dimension.  The
// hardware deals workgroups to the 8 XCDs in turn (workgroup i to XCD
// i mod 8), so workgroup i serves group 8 (k / RB) + i mod 8, row block
// k mod RB (k = i / 8): all row blocks of a group run on one XCD and read
// its activations through one L2, and every XCD takes the full groups first.
template <int HT, int CT, int GSRC>
__global__ __launch_bounds__(WG) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_pf_gate_up(const PfParams p) {
    __shared__ __align__(16) uint8_t x0[G2_XB];
    __shared__ __align__(16) uint8_t x1[G2_XB];
    __shared__ __align__(16) _Float16 mb0[G2_MBT * 16];
    __shared__ __align__(16) _Float16 mb1[G2_MBT * 16];
    __shared__ __align__(16) float d80[128];
    __shared__ __align__(16) float d81[128];
    __shared__ __align__(16) uint8_t w0[G2_WB];
    __shared__ __align__(16) uint8_t w1[G2_WB];
    __shared__ int tok[G2_TOKMAX], pair[G2_TOKMAX];
    const Gu2Lds sm = {x0, x1, w0, w1, mb0, mb1, d80, d81, reinterpret_cast<uint2 *>(w0),
                       reinterpret_cast<u32x4 *>(w1), tok, pair};
    const int RB = (p.n_ff + 63) / 64;
    const int i = blockIdx.x, k = i >> 3;
    const int g = 8 * (k / RB) + (i & 7), rb = k - (k / RB) * RB;
    if (g >= *p.n_gtiles) return;
    const PfTile tile = p.gtiles[g];
    if (!tile_valid(p, tile) || tile.n <= 0) return;
    const int wt = tile.tier == 0 ? HT : CT;
    const int nt = (tile.n + 15) >> 4;
    if (wt == T_Q4_K) {
        if (tile.n > G2_TOKQ4) return;
        switch (nt) {
        case 1: pf_gu2_group<T_Q4_K, GSRC, 1>(p, tile, sm, rb); break;
        case 2: pf_gu2_group<T_Q4_K, GSRC, 2>(p, tile, sm, rb); break;
        case 3: pf_gu2_group<T_Q4_K, GSRC, 3>(p, tile, sm, rb); break;
        default: pf_gu2_group<T_Q4_K, GSRC, 3>(p, tile, sm, rb); break;
        }
    } else {
        if (tile.n > G2_TOKIQ2) return;
        switch (nt) {
        case 1: pf_gu2_group<T_IQ2_S, GSRC, 1>(p, tile, sm, rb); break;
        case 2: pf_gu2_group<T_IQ2_S, GSRC, 2>(p, tile, sm, rb); break;
        case 3: pf_gu2_group<T_IQ2_S, GSRC, 3>(p, tile, sm, rb); break;
        default: pf_gu2_group<T_IQ2_S, GSRC, 4>(p, tile, sm, rb); break;
        }
    }
}

// ---------------------------------------------------- gate_up, q8_1 mode

// IQ2_S on fp16 operands: for each 4-bit scale ls, the fp16 bit patterns of
// the three grid magnitudes {8, 25, 43} times (2 ls + 1) (<= 1333, exact),
// low bytes in .x and high bytes in .y (byte 3 zero), for v_perm.
struct Iq2sHalf {
    uint32_t t[16][2];
};
constexpr uint32_t half_bits_of_int(int v) {      // v < 2048, v > 0: exact
    int e = 0;
    while ((v >> e) >= 2) ++e;                      // 2^e <= v < 2^(e + 1)
    const uint32_t mant = (uint32_t)((v << (10 - e)) & 0x3FF);
    return ((uint32_t)(e + 15) << 10) | mant;
}
constexpr Iq2sHalf make_iq2s_half() {
    Iq2sHalf h{};
    const int lev[3] = {8, 25, 43};
    for (int ls = 0; ls < 16; ++ls) {
        uint32_t lo = 0, hi = 0;
        for (int c = 0; c < 3; ++c) {
            const uint32_t b = half_bits_of_int(lev[c] * (2 * ls + 1));
            lo |= (b & 0xFF) << (8 * c);
            hi |= (b >> 8) << (8 * c);
        }
        h.t[ls][0] = lo;
        h.t[ls][1] = hi;
    }
    return h;
}
__constant__ Iq2sHalf c_iq2s_half = make_iq2s_half();

constexpr int PF_XH = 512 + 8;            // halfs per staged token row of one super-block: 256 hi, 256 lo, pad
constexpr int PF_TOK1Q4 = 48;             // pairs per gate_up group in the q8_1 mode, Q4_K expert
constexpr int PF_TOK1IQ2 = 32;            // IQ2_S expert (its tables take the room of 16 tokens)
constexpr int GU1_XREG = 4;               // activation chunks per thread per super-block and 16-token tile (16 x 64)

// The LDS of one workgroup.  An IQ2_S group (its rows go straight to
// registers) keeps its tables in the room it leaves: the grid selectors and
// Iq2sHalf past 32 tokens' activations, the sign masks in the row buffer.
struct GuSmemQ1 {
    uint8_t w[PF_ROWS * PF_WROW_GU];      // Q4_K: the 128 rows of one super-block, [row][144]
    _Float16 x[PF_TOK1Q4 * PF_XH];        // the tokens' d q of this super-block, exact hi and lo parts
    _Float16 mb[PF_TOK1Q4 * 16];          // their per-32 mins terms u = d sum(q), {hi_0..7, lo_0..7}, Q4_K
    int tok[PF_TOK1Q4], pair[PF_TOK1Q4];
    // IQ2_S grid: v_perm selectors (lo byte c, hi byte 4 + c) per value pair
    __device__ u32x4 * csel() { return reinterpret_cast<u32x4 *>(x + PF_TOK1IQ2 * PF_XH); }
    __device__ uint2 * lsT() { return reinterpret_cast<uint2 *>(csel() + 1024); }       // Iq2sHalf
    // IQ2_S sign byte: 0x8000 per negative value, per value pair
    __device__ u32x4 * sgnh() { return reinterpret_cast<u32x4 *>(w); }
};
static_assert(sizeof(GuSmemQ1) <= 80 * 1024, "two workgroups per CU");
static_assert(PF_ROWS * GU_STP * 4 <= PF_TOK1IQ2 * PF_XH * 2, "epilogue staging stays below the IQ2_S tables");
static_assert((PF_TOK1Q4 - PF_TOK1IQ2) * PF_XH * 2 >= 1024 * 16 + 16 * 8 && (PF_TOK1IQ2 * PF_XH * 2) % 16 == 0,
              "IQ2_S grid selectors and Iq2sHalf past 32 tokens");
static_assert(PF_ROWS * PF_WROW_GU >= 256 * 16, "IQ2_S sign masks in the row buffer");

template <int NT>
struct GuStageQ1 {
    u32x4 w[GU_WREG];
    u32x4 x[NT * GU1_XREG];
    u32x4 mb;
};

// One (group of <= 48 pairs, row block) of the gate_up GEMM in the q8_1 activation mode
// (ggml-cuda's arithmetic, vecdotq.cuh:504-522 / 864-907): the activation
// scale is per 32 values, so it is carried by the activation operand -- each
// value d q as exact fp16 hi + lo parts, two v_mfma_f32_16x16x32_f16 per
// 32-block -- and the weights are exact fp16 integers with the sub-block
// scale folded in (Q4_K q sc <= 945, IQ2_S grid (2 ls + 1) <= 1333, both
// exact).  Every product is exact and one fp32 accumulator chains through the
// super-block; then d_w per super-block (Q4_K minus dmin times the mins MFMA,
// IQ2_S d / 8 in the epilogue).  The epilogue quantises the down activations
// to q8_1.
template <int WT, int GSRC, int NT>
__device__ __forceinline__ void pf_gate_up_group_q1(const PfParams & p, const PfTile & tile, GuSmemQ1 & sm,
                                                    const int rb, const int n) {
    static_assert(PF_ROWS * 9 <= GU_WREG * WG && 16 * 64 == GU1_XREG * WG, "staging shape");
    constexpr int NTOK = 16 * NT;
    constexpr bool q4 = WT == T_Q4_K;
    static_assert(q4 || WT == T_IQ2_S, "gate_up formats");
    constexpr int CAP = q4 ? PF_TOK1Q4 : PF_TOK1IQ2;
    static_assert(NTOK <= CAP, "group fits the LDS");
    const int F = p.n_ff, D = p.d_model, NSB = D / 256, K = p.top_k;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, q = lane >> 4, l16 = lane & 15;
    constexpr int bb = q4 ? 144 : 82;
    const uint64_t rbytes = (uint64_t)NSB * bb;
    const uint8_t * W = tile.tier == 0 ? p.hot_gu + (uint64_t)tile.idx * p.hot_gu_stride
                                       : p.cold_gu + (uint64_t)tile.idx * p.cold_gu_stride;
    if (tid < NTOK) {
        const int qp = p.sorted[tile.begin + min(tid, n - 1)];
        sm.pair[tid] = qp;
        sm.tok[tid] = qp / K;
    }
    if constexpr (!q4) {
        // selectors from the level codes (one byte 0..2 per value)
        const uint2 * codes = reinterpret_cast<const uint2 *>(&c_iq2s_tab_pf);
        for (int i = tid; i < 1024; i += WG) {
            const uint2 c = codes[i];
            u32x4 v;
            v.x = __builtin_amdgcn_perm(0u, c.x, 0x01010000u) + 0x04000400u;
            v.y = __builtin_amdgcn_perm(0u, c.x, 0x03030202u) + 0x04000400u;
            v.z = __builtin_amdgcn_perm(0u, c.y, 0x01010000u) + 0x04000400u;
            v.w = __builtin_amdgcn_perm(0u, c.y, 0x03030202u) + 0x04000400u;
            sm.csel()[i] = v;
        }
        u32x4 sg;
        sg.x = ((tid & 1) ? 0x8000u : 0u) | ((tid & 2) ? 0x80000000u : 0u);
        sg.y = ((tid & 4) ? 0x8000u : 0u) | ((tid & 8) ? 0x80000000u : 0u);
        sg.z = ((tid & 16) ? 0x8000u : 0u) | ((tid & 32) ? 0x80000000u : 0u);
        sg.w = ((tid & 64) ? 0x8000u : 0u) | ((tid & 128) ? 0x80000000u : 0u);
        sm.sgnh()[tid] = sg;                                    // WG == 256 sign bytes
        if (tid < 16) sm.lsT()[tid] = make_uint2(c_iq2s_half.t[tid][0], c_iq2s_half.t[tid][1]);
    }
    __syncthreads();

    // Q4_K rows: 128 rows x 9 chunks of one super-block, [row][144] in LDS
    uint32_t wrow[GU_WREG], wdst[GU_WREG];
#pragma unroll
    for (int k = 0; k < GU_WREG; ++k) {
        const int i = tid + WG * k;
        const int r = i / 9, c = i - 9 * r;
        const int gi = min(64 * rb + (r & 63), F - 1);
        const int row = r < 64 ? gi : F + gi;
        wrow[k] = r < PF_ROWS ? (uint32_t)((uint64_t)row * rbytes) : ~0u;
        wdst[k] = (uint32_t)(r * 144 + 16 * c) | ((uint32_t)c << 16);
    }
    const int tok_m = tid < 2 * NTOK ? sm.tok[tid >> 1] * NSB * 16 + 8 * (tid & 1) : 0;
    // IQ2_S rows go straight to registers (as k_pf_gate_up's): local row
    // 32 wave + 16 rs + l16 is gate row 64 rb + r (r < 64) or up row
    // F + 64 rb + r - 64, clamped into the slab
    uint32_t voff[2], rowpar[2];
#pragma unroll
    for (int rs = 0; rs < 2; ++rs) {
        const int r = 32 * wave + 16 * rs + l16;
        const int gi = min(64 * rb + (r & 63), F - 1);
        voff[rs] = (uint32_t)((uint64_t)(r < 64 ? gi : F + gi) * rbytes);
        rowpar[rs] = (voff[rs] >> 1) & 1u;                      // row start mod 4, halved (slabs are 16-aligned)
    }
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(W), 0, (int)(2u * (uint32_t)F * (uint32_t)rbytes), 0x00020000);
    Iq2Raw wi[q4 ? 1 : 2];

    GuStageQ1<NT> g;
    // buffer loads: a lane's offset in its register (fixed over the
    // super-blocks), the super-block's in the scalar offset
    const __amdgpu_buffer_rsrc_t xr4 = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<_Float16 *>(p.xh), 0, (int)((uint32_t)p.T * (uint32_t)NSB * 1024u), 0x00020000);
    const __amdgpu_buffer_rsrc_t mr4 = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<_Float16 *>(p.xm), 0, (int)((uint32_t)p.T * (uint32_t)NSB * 32u), 0x00020000);
    auto fetch = [&](int s) {
        if constexpr (q4) {
#pragma unroll
            for (int k = 0; k < GU_WREG; ++k) {
                g.w[k] = u32x4{0, 0, 0, 0};
                if (wrow[k] != ~0u)
                    g.w[k] = __builtin_amdgcn_raw_buffer_load_b128(wr, wrow[k] + 16 * (wdst[k] >> 16), bb * s, 0);
            }
        }
#pragma unroll
        for (int k = 0; k < NT * GU1_XREG; ++k) {
            const int i = tid + WG * k, j = i >> 6, c = i & 63;
            g.x[k] = __builtin_amdgcn_raw_buffer_load_b128(xr4, (uint32_t)sm.tok[j] * (uint32_t)(NSB * 1024) + 16u * (uint32_t)c,
                                                           1024 * s, 0);
        }
        if (q4 && tid < 2 * NTOK) g.mb = __builtin_amdgcn_raw_buffer_load_b128(mr4, 2u * (uint32_t)tok_m, 32 * s, 0);
    };
    auto store = [&](int s) {
        if constexpr (q4) {
#pragma unroll
            for (int k = 0; k < GU_WREG; ++k)
                if (wrow[k] != ~0u) *reinterpret_cast<u32x4 *>(sm.w + (wdst[k] & 0xFFFF)) = g.w[k];
        }
#pragma unroll
        for (int k = 0; k < NT * GU1_XREG; ++k) {
            const int i = tid + WG * k, j = i >> 6, c = i & 63;
            *reinterpret_cast<u32x4 *>(sm.x + j * PF_XH + 8 * c) = g.x[k];
        }
        if (q4 && tid < 2 * NTOK) *reinterpret_cast<u32x4 *>(sm.mb + 16 * (tid >> 1) + 8 * (tid & 1)) = g.mb;
    };

    f4 y[2][NT];
#pragma unroll
    for (int rs = 0; rs < 2; ++rs)
#pragma unroll
        for (int ts = 0; ts < NT; ++ts) y[rs][ts] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    const _Float16 mm = q < 2 ? (_Float16)1.0f : (_Float16)0.0f;
    const _Float16 mo = q < 2 ? (_Float16)(-1024.0f) : (_Float16)0.0f;
    const h2 mn_mul = h2{mm, mm}, mn_off = h2{mo, mo};
    const h2 m1024 = h2{(_Float16)(-1024.0f), (_Float16)(-1024.0f)};

    fetch(0);
    if constexpr (!q4) {
#pragma unroll
        for (int rs = 0; rs < 2; ++rs) iq2_raw_load(wi[rs], wr, voff[rs], rowpar[rs], 0, q);
    }
#pragma unroll 1
    for (int s = 0; s < NSB; ++s) {
        if (s) __syncthreads();
        store(s);
        __syncthreads();
        if (s + 1 < NSB) fetch(s + 1);

        // ---- per row tile: the super-block's header (Q4_K from LDS, IQ2_S
        // from the registers its loads landed in; then the next super-block's
        // IQ2_S loads are issued)
        int wo[2];
        float dr[2], mr[2];
        h2 scp[2][4];
        uint2 qs8[2], sg8[2];
        uint32_t qh2[2], sc2[2];
        h8 bm[2];
#pragma unroll
        for (int rs = 0; rs < 2; ++rs) {
            wo[rs] = (32 * wave + 16 * rs + l16) * 144;
            if constexpr (q4) {
                const u32x4 hdr = *reinterpret_cast<const u32x4 *>(sm.w + wo[rs]);
                dr[rs] = h2f(hdr.x & 0xFFFF);
                mr[rs] = h2f(hdr.x >> 16);
                const uint32_t sc03 = hdr.y & 0x3F3F3F3Fu;
                const uint32_t mn03 = hdr.z & 0x3F3F3F3Fu;
                const uint32_t sc47 = (hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u);
                const uint32_t mn47 = ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u);
                // the 8 scales as fp16 (1024 + sc) - 1024, pairs {sc_2i, sc_2i+1}
                scp[rs][0] = as_h2(magic_lo(sc03)) + m1024;
                scp[rs][1] = as_h2(magic_hi(sc03)) + m1024;
                scp[rs][2] = as_h2(magic_lo(sc47)) + m1024;
                scp[rs][3] = as_h2(magic_hi(sc47)) + m1024;
                // mins B operand: k 0..7 and 8..15 = m_j, 16..31 = 0
                const uint32_t mb4[4] = {magic_lo(mn03), magic_hi(mn03), magic_lo(mn47), magic_hi(mn47)};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const h2 mv = __builtin_elementwise_fma(as_h2(mb4[i]), mn_mul, mn_off);
                    bm[rs][2 * i] = mv.x;
                    bm[rs][2 * i + 1] = mv.y;
                }
            } else {
                // this lane's grid entries 8 q .. 8 q + 7 (values 64 q .. 64 q + 63)
                const Iq2Raw & w = wi[rs];
                dr[rs] = h2f((w.d >> w.sh_d) & 0xFFFFu);
                mr[rs] = 0.0f;
                qs8[rs] = make_uint2(__builtin_amdgcn_alignbit(w.qs.y, w.qs.x, w.sh_q),
                                     __builtin_amdgcn_alignbit(w.qs.z, w.qs.y, w.sh_q));
                sg8[rs] = make_uint2(__builtin_amdgcn_alignbit(w.sg.y, w.sg.x, w.sh_q),
                                     __builtin_amdgcn_alignbit(w.sg.z, w.sg.y, w.sh_q));
                qh2[rs] = (w.qh >> w.sh_h) & 0xFFFFu;               // 2 bits per entry
                sc2[rs] = (w.sc >> w.sh_h) & 0xFFFFu;               // 4 bits per two entries
            }
        }
        if constexpr (!q4) {
            if (s + 1 < NSB) {
#pragma unroll
                for (int rs = 0; rs < 2; ++rs) iq2_raw_load(wi[rs], wr, voff[rs], rowpar[rs], s + 1, q);
            }
        }

        // ---- per step j: B (lane (row l16, quarter q): Q4_K values 8 q ..
        // 8 q + 7 of block j, IQ2_S grid entry 8 q + j; exact fp16 integers,
        // scale folded in), then hi and lo of the same values of every token
        // tile into the chained accumulators (the super-block's K order is
        // free: the activation scales are in the parts)
        f4 acc[2][NT];
#pragma unroll
        for (int rs = 0; rs < 2; ++rs)
#pragma unroll
            for (int ts = 0; ts < NT; ++ts) acc[rs][ts] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            h8 bw[2];
#pragma unroll
            for (int rs = 0; rs < 2; ++rs) {
                uint32_t hv[4];
                if constexpr (q4) {
                    const h2 spair = scp[rs][j >> 1];
                    const _Float16 scj = (j & 1) ? spair.y : spair.x;
                    const h2 sc2 = h2{scj, scj};
                    const h2 off = sc2 * m1024;                 // -1024 sc, exact
                    // nibbles of qs bytes 32 (j / 2) + 8 q ..: low for even j, high for odd
                    const uint2 wq = *reinterpret_cast<const uint2 *>(sm.w + wo[rs] + 16 + 32 * (j >> 1) + 8 * q);
                    const uint32_t sh = 4u * (uint32_t)(j & 1);
                    const uint32_t n0 = (wq.x >> sh) & 0x0F0F0F0Fu, n1 = (wq.y >> sh) & 0x0F0F0F0Fu;
                    hv[0] = h2bits(__builtin_elementwise_fma(as_h2(magic_lo(n0)), sc2, off));
                    hv[1] = h2bits(__builtin_elementwise_fma(as_h2(magic_hi(n0)), sc2, off));
                    hv[2] = h2bits(__builtin_elementwise_fma(as_h2(magic_lo(n1)), sc2, off));
                    hv[3] = h2bits(__builtin_elementwise_fma(as_h2(magic_hi(n1)), sc2, off));
                } else {
                    // grid entry 8 q + j: its index, signs, the 4-bit scale of its 16 values
                    const uint32_t qsw = j < 4 ? qs8[rs].x : qs8[rs].y, sgw = j < 4 ? sg8[rs].x : sg8[rs].y;
                    const uint32_t idx = __builtin_amdgcn_ubfe(qsw, 8 * (j & 3), 8) |
                                         (__builtin_amdgcn_ubfe(qh2[rs], 2 * j, 2) << 8);
                    const uint32_t ls = __builtin_amdgcn_ubfe(sc2[rs], 4 * (j >> 1), 4);
                    const u32x4 sel = sm.csel()[idx];
                    const u32x4 sg = sm.sgnh()[__builtin_amdgcn_ubfe(sgw, 8 * (j & 3), 8)];
                    const uint2 t = sm.lsT()[ls];
                    hv[0] = __builtin_amdgcn_perm(t.y, t.x, sel.x) | sg.x;
                    hv[1] = __builtin_amdgcn_perm(t.y, t.x, sel.y) | sg.y;
                    hv[2] = __builtin_amdgcn_perm(t.y, t.x, sel.z) | sg.z;
                    hv[3] = __builtin_amdgcn_perm(t.y, t.x, sel.w) | sg.w;
                }
                __builtin_memcpy(&bw[rs], hv, 16);
            }
#pragma unroll
            for (int ts = 0; ts < NT; ++ts) {
                const _Float16 * xr = sm.x + (16 * ts + l16) * PF_XH + (q4 ? 32 * j + 8 * q : 64 * q + 8 * j);
                h8 ah, al;
                __builtin_memcpy(&ah, xr, 16);
                __builtin_memcpy(&al, xr + 256, 16);
#pragma unroll
                for (int rs = 0; rs < 2; ++rs) acc[rs][ts] = mfma_f16(al, bw[rs], mfma_f16(ah, bw[rs], acc[rs][ts]));
            }
        }
        // ---- the super-block into y: d_w (Q4_K: minus dmin times the mins MFMA)
#pragma unroll
        for (int ts = 0; ts < NT; ++ts) {
            if constexpr (q4) {
                h8 am;
                const u32x4 mv = q < 2 ? *reinterpret_cast<const u32x4 *>(sm.mb + 16 * (16 * ts + l16) + 8 * q)
                                       : u32x4{0, 0, 0, 0};
                __builtin_memcpy(&am, &mv, 16);
#pragma unroll
                for (int rs = 0; rs < 2; ++rs) {
                    const f4 m = mfma_f16(am, bm[rs], f4{0.0f, 0.0f, 0.0f, 0.0f});
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        y[rs][ts][r] = __builtin_fmaf(-mr[rs], m[r], __builtin_fmaf(dr[rs], acc[rs][ts][r], y[rs][ts][r]));
                }
            } else {
#pragma unroll
                for (int rs = 0; rs < 2; ++rs)
#pragma unroll
                    for (int r = 0; r < 4; ++r) y[rs][ts][r] = __builtin_fmaf(dr[rs], acc[rs][ts][r], y[rs][ts][r]);
            }
        }
    }

    // ---- epilogue: GEGLU of gate row i and up row i, q8_1 of each 32-block
    const float f = q4 ? 1.0f : 0.125f;
    float * stg = reinterpret_cast<float *>(sm.x);
#pragma unroll
    for (int ts = 0; ts < NT; ++ts) {
        __syncthreads();
#pragma unroll
        for (int rs = 0; rs < 2; ++rs)
#pragma unroll
            for (int r = 0; r < 4; ++r) stg[(32 * wave + 16 * rs + l16) * GU_STP + 4 * q + r] = f * y[rs][ts][r];
        __syncthreads();
#pragma unroll
        for (int pass = 0; pass < 4; ++pass) {
            const int u = 8 * pass + 2 * wave + (lane >> 5);
            const int tk = u >> 1, blk = u & 1, i = lane & 31;
            const int j = 16 * ts + tk;
            const int fi = 64 * rb + 32 * blk;
            const bool live = j < n && fi < F;
            const float gv = stg[(32 * blk + i) * GU_STP + tk];
            const float uv = stg[(64 + 32 * blk + i) * GU_STP + tk];
            const float v = geglu1<GSRC>(gv, uv);
            const int64_t qp = sm.pair[min(j, NTOK - 1)];
            q8_store32<AM_Q8_1>(v, p.ah + qp * F + fi + i, p.al + qp * F + fi + i, nullptr, live);
        }
    }
}

template <int HT, int CT, int GSRC>
__global__ __launch_bounds__(WG) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_pf_gate_up_q1(const PfParams p) {
    __shared__ __align__(16) GuSmemQ1 sm;
    // the gate_up groups of this mode hold <= PF_TOK1Q4 pairs of a Q4_K
    // expert, <= PF_TOK1IQ2 of an IQ2_S one; workgroups are dealt to the XCDs
    // as k_pf_gate_up's (all row blocks of a group on one)
    const int RB = (p.n_ff + 63) / 64;
    const int i = blockIdx.x, k = i >> 3;
    const int g = 8 * (k / RB) + (i & 7), rb = k - (k / RB) * RB;
    if (g >= *p.n_gtiles) return;
    const PfTile tile = p.gtiles[g];
    const bool q4 = (tile.tier == 0 ? HT : CT) == T_Q4_K;
    if (!tile_valid(p, tile) || tile.n <= 0 || tile.n > (q4 ? PF_TOK1Q4 : PF_TOK1IQ2)) return;
    const int n = tile.n;
    if (q4) {
        if (n > 32) pf_gate_up_group_q1<T_Q4_K, GSRC, 3>(p, tile, sm, rb, n);
        else if (n > 16) pf_gate_up_group_q1<T_Q4_K, GSRC, 2>(p, tile, sm, rb, n);
        else pf_gate_up_group_q1<T_Q4_K, GSRC, 1>(p, tile, sm, rb, n);
    } else {
        if (n > 16) pf_gate_up_group_q1<T_IQ2_S, GSRC, 2>(p, tile, sm, rb, n);
        else pf_gate_up_group_q1<T_IQ2_S, GSRC, 1>(p, tile, sm, rb, n);
    }
}

// ------------------------------------------------------------------ down

// One (group, 128-row block) of the down GEMM with NT 16-token tiles.  Wave
// w owns rows 32 w .. 32 w + 31 as two 16-row MFMA tiles.  K (n_ff) runs in
// chunks of two 32-blocks, CPS chunks a step (groups of up to 32 pairs take
// two: a small group's step is short, and each step waits for its loads).
// The load unit copies the next step's activation parts into LDS while the
// current one's are used (two buffers, separately declared, one barrier per
// step): a pair's chunk is 16 slots of 16 bytes (slots 0..7 the high parts
// of its 64 values, 8..15 the low parts), slot s at s ^ (pair & 15), so the
// 16 pairs of an MFMA fragment read 16 distinct slots.  Each lane loads its
// rows' window of the step (44 bytes of Q5_0, 36 of IQ4_NL a chunk) straight
// into registers, the next step's in flight during the current one's MFMAs.
constexpr int D2_XB = PF_TOK * 256;                // activations of one step: [chunk][pair slot][16][16 bytes]

struct Dn2Lds {
    uint8_t * x0; uint8_t * x1;
    int * pair;
};

// One lane's row window of a two-block chunk: 44 bytes (Q5_0) or 36
// (IQ4_NL), from the chunk's first byte.
struct DnWin {
    u32x4 a, b;
    u32x3 e;
};
template <int I>
__device__ __forceinline__ uint32_t win_dword(const DnWin & w) {
    if constexpr (I < 4) return w.a[I];
    else if constexpr (I < 8) return w.b[I - 4];
    else return w.e[I - 8];
}
// the dword holding bytes BYTE .. BYTE + 3 of the window (BYTE even)
template <int BYTE>
__device__ __forceinline__ uint32_t win_at(const DnWin & w) {
    if constexpr (BYTE & 3) return __builtin_amdgcn_alignbit(win_dword<(BYTE >> 2) + 1>(w), win_dword<(BYTE >> 2)>(w), 16);
    else return win_dword<(BYTE >> 2)>(w);
}

// 8 values (8 u .. 8 u + 7 of block B of the chunk) as exact fp16 integers:
// Q5_0 q - 16 (ggml-quants.c:442), IQ4_NL kvalues[q] (:2653); the block
// scale d_w out.  Block 1 starts 2 bytes into a dword of the window.
template <int T, int B>
__device__ __forceinline__ h8 down_frag_r(const DnWin & w, int u, float & d) {
    constexpr int BS = T == T_Q5_0 ? 22 : 18;
    constexpr int o0 = BS * B;                          // the block's first byte
    d = h2f((o0 & 3) ? (win_dword<(o0 >> 2)>(w) >> 16) : (win_dword<(o0 >> 2)>(w) & 0xFFFFu));
    const bool hiq = (u & 1) != 0;                      // bytes 8..15 of the qs
    uint32_t h[4];
    if constexpr (T == T_Q5_0) {
        // values 0..15: low nibbles of qs[0..15]; 16..31: high nibbles
        const uint32_t qs0 = hiq ? win_at<o0 + 14>(w) : win_at<o0 + 6>(w);
        const uint32_t qs1 = hiq ? win_at<o0 + 18>(w) : win_at<o0 + 10>(w);
        const uint32_t qh = __builtin_amdgcn_ubfe(win_at<o0 + 2>(w), 8 * u, 8);
        const int sh = 4 * (u >> 1);
        uint32_t x[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t nib = ((i ? qs1 : qs0) >> sh) & 0x0F0F0F0Fu;
            const uint32_t hb = (qh >> (4 * i)) & 15u;
            x[i] = nib | (((hb * 0x00204081u) & 0x01010101u) << 4);   // bit k -> bit 4 of byte k
        }
        const h2 off = h2{(_Float16)(-1040.0f), (_Float16)(-1040.0f)};
        h[0] = h2bits(as_h2(magic_lo(x[0])) + off);
        h[1] = h2bits(as_h2(magic_hi(x[0])) + off);
        h[2] = h2bits(as_h2(magic_lo(x[1])) + off);
        h[3] = h2bits(as_h2(magic_hi(x[1])) + off);
    } else {
        const uint32_t qs0 = hiq ? win_at<o0 + 10>(w) : win_at<o0 + 2>(w);
        const uint32_t qs1 = hiq ? win_at<o0 + 14>(w) : win_at<o0 + 6>(w);
        const int sh = 4 * (u >> 1);
        const h2 off = h2{(_Float16)(-1152.0f), (_Float16)(-1152.0f)};
        uint32_t x[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) x[i] = iq4nl_lookup(((i ? qs1 : qs0) >> sh) & 0x0F0F0F0Fu) ^ 0x80808080u;
        h[0] = h2bits(as_h2(magic_lo(x[0])) + off);
        h[1] = h2bits(as_h2(magic_hi(x[0])) + off);
        h[2] = h2bits(as_h2(magic_lo(x[1])) + off);
        h[3] = h2bits(as_h2(magic_hi(x[1])) + off);
    }
    h8 o;
    __builtin_memcpy(&o, h, 16);
    return o;
}

template <int WT, int NT, int CPS>
__device__ __forceinline__ void pf_down2_group(const PfParams & p, const PfTile & tile, const Dn2Lds & L,
                                               const int rb) {
    static_assert(WT == T_Q5_0 || WT == T_IQ4_NL, "down formats");
    constexpr int NTOK = 16 * NT;
    static_assert(NTOK * 256 * CPS <= D2_XB, "a step's chunks fit an activation buffer");
    constexpr int BS = WT == T_Q5_0 ? 22 : 18;
    constexpr int CW = BS / 2;                                  // dwords of a chunk (two blocks)
    constexpr int NW = (4 * CW * CPS + 3 + 15) / 16;            // 16-byte loads of a step's row window
    const int D = p.d_model, F = p.n_ff, NB = F / 32, NC = (NB + 1) / 2, NS = (NC + CPS - 1) / CPS;
    const int r0 = rb * PF_ROWS;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, q = lane >> 4, l16 = lane & 15;
    const uint32_t rbytes = (uint32_t)(NB * BS);
    const uint8_t * W = tile.tier == 0 ? p.hot_dn + (uint64_t)tile.idx * p.hot_dn_stride
                                       : p.cold_dn + (uint64_t)tile.idx * p.cold_dn_stride;
    // the slab as a buffer: a last chunk of one block (and a step's window)
    // reads past its row (unused bytes; past the slab they read as zero)
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(W), 0,
                                                                         (int)((uint32_t)D * rbytes), 0x00020000);
    if (tid < NTOK) L.pair[tid] = p.sorted[tile.begin + min(tid, tile.n - 1)];
    __syncthreads();

    // step s: chunks CPS s .. CPS s + CPS - 1, chunk c of the step at xb + c NTOK 256
    auto copy_in = [&](int s, uint8_t * xb) {
        const _Float16 * ah = p.ah;
        const _Float16 * al = p.al;
        asm volatile("" : "+s"(ah), "+s"(al));
        // wave w moves pair blocks w NT + k (four pair slots each); a last
        // chunk of one block reads its second block's slots from inside the row
#pragma unroll
        for (int cc = 0; cc < CPS; ++cc) {
            const int c = min(CPS * s + cc, NC - 1);
#pragma unroll
            for (int k = 0; k < NT; ++k) {
                const int j = 4 * (wave * NT + k) + (lane >> 4);
                const int sg = (lane & 15) ^ (j & 15);
                const uint32_t off = (uint32_t)(L.pair[j] * F + min(64 * c + 8 * (sg & 7), F - 8));
                lds_dma16((sg < 8 ? ah : al) + off, xb + NTOK * 256 * cc + 1024 * (wave * NT + k));
            }
        }
    };
    uint32_t voff[2];
#pragma unroll
    for (int rs = 0; rs < 2; ++rs) voff[rs] = (uint32_t)min(r0 + 32 * wave + 16 * rs + l16, D - 1) * rbytes;
    // raw windows: from the dword at or below the step's start (a row of an
    // odd block count starts 2 bytes into a dword), NW x 16 bytes
    u32x4 wraw[2][NW];
    uint32_t wsh[2];
    auto load_rows = [&](int s) {
#pragma unroll
        for (int rs = 0; rs < 2; ++rs) {
            const uint32_t st = voff[rs] + (uint32_t)(2 * BS * CPS * s);
            const uint32_t v0 = st & ~3u;
            wsh[rs] = 8u * (st & 3u);
#pragma unroll
            for (int k = 0; k < NW; ++k) wraw[rs][k] = __builtin_amdgcn_raw_buffer_load_b128(wr, v0 + 16 * k, 0, 0);
        }
    };

    f4 y[2][NT];
#pragma unroll
    for (int rs = 0; rs < 2; ++rs)
#pragma unroll
        for (int ts = 0; ts < NT; ++ts) y[rs][ts] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    auto step = [&](int s, const uint8_t * xb, uint8_t * xn) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        // this step's rows out of the registers the loads land in, the next
        // step's copies and loads in flight during the MFMAs
        DnWin wc[CPS][2];
#pragma unroll
        for (int rs = 0; rs < 2; ++rs) {
            uint32_t r[4 * NW];
#pragma unroll
            for (int k = 0; k < NW; ++k) {
                r[4 * k] = wraw[rs][k].x;
                r[4 * k + 1] = wraw[rs][k].y;
                r[4 * k + 2] = wraw[rs][k].z;
                r[4 * k + 3] = wraw[rs][k].w;
            }
#pragma unroll
            for (int cc = 0; cc < CPS; ++cc) {
                uint32_t t[11];
#pragma unroll
                for (int i = 0; i < 11; ++i) {
                    const int a = min(CW * cc + i, 4 * NW - 2);
                    t[i] = __builtin_amdgcn_alignbit(r[a + 1], r[a], wsh[rs]);
                }
                wc[cc][rs].a = u32x4{t[0], t[1], t[2], t[3]};
                wc[cc][rs].b = u32x4{t[4], t[5], t[6], t[7]};
                wc[cc][rs].e = u32x3{t[8], t[9], t[10]};
            }
        }
        if (s + 1 < NS) {
            copy_in(s + 1, xn);
            load_rows(s + 1);
        }
#pragma unroll
        for (int cc = 0; cc < CPS; ++cc) {
            const int c = CPS * s + cc;
            if (c < NC) {                                       // workgroup-uniform
                const int cb = min(2, NB - 2 * c);
                const uint8_t * xc = xb + NTOK * 256 * cc;
                auto block = [&](auto bc) {
                    constexpr int B = decltype(bc)::value;
                    // B operand: lane (row l16, quarter q) holds values 8 q .. 8 q + 7 of block B
                    h8 bw[2];
                    float dw[2];
#pragma unroll
                    for (int rs = 0; rs < 2; ++rs) bw[rs] = down_frag_r<WT, B>(wc[cc][rs], q, dw[rs]);
#pragma unroll
                    for (int ts = 0; ts < NT; ++ts) {
                        const uint8_t * xr = xc + (16 * ts + l16) * 256;
                        h8 ah, al;
                        __builtin_memcpy(&ah, xr + 16 * ((4 * B + q) ^ l16), 16);
                        __builtin_memcpy(&al, xr + 16 * ((8 + 4 * B + q) ^ l16), 16);
#pragma unroll
                        for (int rs = 0; rs < 2; ++rs) {
                            const f4 sb = mfma_f16(al, bw[rs], mfma_f16(ah, bw[rs], f4{0.0f, 0.0f, 0.0f, 0.0f}));
#pragma unroll
                            for (int r = 0; r < 4; ++r) y[rs][ts][r] = __builtin_fmaf(dw[rs], sb[r], y[rs][ts][r]);
                        }
                    }
                };
                block(std::integral_constant<int, 0>{});
                if (cb > 1) block(std::integral_constant<int, 1>{});
            }
        }
    };

    copy_in(0, L.x0);
    load_rows(0);
    for (int s = 0; s < NS; s += 2) {
        step(s, L.x0, L.x1);
        if (s + 1 < NS) step(s + 1, L.x1, L.x0);
    }
    const float sc = tile.tier == 0 ? (p.s_hot ? p.s_hot[tile.idx] : 1.0f) : (p.s_cold ? p.s_cold[tile.idx] : 1.0f);
#pragma unroll
    for (int ts = 0; ts < NT; ++ts) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int j = 16 * ts + 4 * q + r;
            if (j >= tile.n) continue;
            float * out = p.ydn + (int64_t)L.pair[j] * D;
#pragma unroll
            for (int rs = 0; rs < 2; ++rs) {
                const int row = r0 + 32 * wave + 16 * rs + l16;
                if (row < D) out[row] = sc * y[rs][ts][r];
            }
        }
    }
}

// Grid: 8 x ceil(max_tiles / 8) x RB workgroups in one dimension, dealt to
// the XCDs as the gate_up kernel's: all row blocks of a group on one XCD.
template <int HT, int CT>
__global__ __launch_bounds__(WG) __attribute__((amdgpu_waves_per_eu(3, 3))) void k_pf_down(const PfParams p) {
    __shared__ __align__(16) uint8_t x0[D2_XB];
    __shared__ __align__(16) uint8_t x1[D2_XB];
    __shared__ int pair[PF_TOK];
    const Dn2Lds sm = {x0, x1, pair};
    const int RB = (p.d_model + PF_ROWS - 1) / PF_ROWS;
    const int i = blockIdx.x, k = i >> 3;
    const int g = 8 * (k / RB) + (i & 7), rb = k - (k / RB) * RB;
    if (g >= *p.n_tiles) return;
    const PfTile tile = p.tiles[g];
    if (!tile_valid(p, tile) || tile.n <= 0 || tile.n > PF_TOK) return;
    const int nt = (tile.n + 15) >> 4;
    static_assert(PF_TOK == 96, "six tile counts");
    if ((tile.tier == 0 ? HT : CT) == T_Q5_0) {
        switch (nt) {
        case 1: pf_down2_group<T_Q5_0, 1, 2>(p, tile, sm, rb); break;
        case 2: pf_down2_group<T_Q5_0, 2, 2>(p, tile, sm, rb); break;
        case 3: pf_down2_group<T_Q5_0, 3, 1>(p, tile, sm, rb); break;
        case 4: pf_down2_group<T_Q5_0, 4, 1>(p, tile, sm, rb); break;
        case 5: pf_down2_group<T_Q5_0, 5, 1>(p, tile, sm, rb); break;
        default: pf_down2_group<T_Q5_0, 6, 1>(p, tile, sm, rb); break;
        }
    } else {
        switch (nt) {
        case 1: pf_down2_group<T_IQ4_NL, 1, 2>(p, tile, sm, rb); break;
        case 2: pf_down2_group<T_IQ4_NL, 2, 2>(p, tile, sm, rb); break;
        case 3: pf_down2_group<T_IQ4_NL, 3, 1>(p, tile, sm, rb); break;
        case 4: pf_down2_group<T_IQ4_NL, 4, 1>(p, tile, sm, rb); break;
        case 5: pf_down2_group<T_IQ4_NL, 5, 1>(p, tile, sm, rb); break;
        default: pf_down2_group<T_IQ4_NL, 6, 1>(p, tile, sm, rb); break;
        }
    }
}

}  // namespace dev

using namespace dev;

int pf_max_tiles(int P, int n_expert) { return (P + PF_TOK - 1) / PF_TOK + std::min(n_expert, P); }
int pf_max_gtiles(int P, int n_expert) { return (P + 15) / 16 + std::min(n_expert, P); }

namespace {
template <typename F>
void launch_pf(F k, dim3 grid, hipStream_t s, hipEvent_t e0, hipEvent_t e1, const PfParams & p) {
    if (e0) hipExtLaunchKernelGGL(k, grid, dim3(WG), 0u, s, e0, e1, 0u, p);
    else hipLaunchKernelGGL(k, grid, dim3(WG), 0, s, p);
}
template <int HT, int CT>
void launch_gu(int gelu, hipStream_t s, hipEvent_t e0, hipEvent_t e1, const PfParams & p) {
    const dim3 g2(8 * ((p.max_gtiles + 7) / 8) * ((p.n_ff + 63) / 64));
    if (p.act_mode == AM_Q8_1) {
        if (gelu == SRC_GEGLU_TANH) launch_pf(k_pf_gate_up_q1<HT, CT, SRC_GEGLU_TANH>, g2, s, e0, e1, p);
        else launch_pf(k_pf_gate_up_q1<HT, CT, SRC_GEGLU_TABLE>, g2, s, e0, e1, p);
    } else {
        if (gelu == SRC_GEGLU_TANH) launch_pf(k_pf_gate_up<HT, CT, SRC_GEGLU_TANH>, g2, s, e0, e1, p);
        else launch_pf(k_pf_gate_up<HT, CT, SRC_GEGLU_TABLE>, g2, s, e0, e1, p);
    }
}
// pairs per gate_up group of an expert in format t (the Q4_K kernel holds
// 128 tokens' activations in LDS; IQ2_S's tables take the room of half)
int gate_up_cap(int t) { return t == T_Q4_K ? G2_TOKQ4 : G2_TOKIQ2; }
// in the q8_1 mode (1 KB of activation parts per token and super-block)
int gate_up_cap_q1(int t) { return t == T_Q4_K ? PF_TOK1Q4 : PF_TOK1IQ2; }
}  // namespace

hipError_t launch_prefill(const PfParams & p0, int hgu, int cgu, int hdn, int cdn, int gelu, hipStream_t s,
                          hipEvent_t * ev) {
    PfParams p = p0;
    p.gcap[0] = p.act_mode == AM_Q8_1 ? gate_up_cap_q1(hgu) : gate_up_cap(hgu);
    p.gcap[1] = p.act_mode == AM_Q8_1 ? gate_up_cap_q1(cgu) : gate_up_cap(cgu);
    hipEvent_t e[4] = {};
    if (ev)
        for (int i = 0; i < 4; ++i) e[i] = ev[i];
    const int NSB = p.d_model / 256;
    if (p.act_mode == AM_Q8_1)
        hipLaunchKernelGGL(k_pf_prep<AM_Q8_1>, dim3(1 + (p.T * (p.d_model / 64) + 3) / 4), dim3(WG), 0, s, p);
    else hipLaunchKernelGGL(k_pf_prep<AM_CPU>, dim3(1 + (p.T * NSB + 3) / 4), dim3(WG), 0, s, p);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    {
        if (hgu == T_Q4_K && cgu == T_IQ2_S) launch_gu<T_Q4_K, T_IQ2_S>(gelu, s, e[0], e[1], p);
        else if (hgu == T_Q4_K && cgu == T_Q4_K) launch_gu<T_Q4_K, T_Q4_K>(gelu, s, e[0], e[1], p);
        else if (hgu == T_IQ2_S && cgu == T_IQ2_S) launch_gu<T_IQ2_S, T_IQ2_S>(gelu, s, e[0], e[1], p);
        else if (hgu == T_IQ2_S && cgu == T_Q4_K) launch_gu<T_IQ2_S, T_Q4_K>(gelu, s, e[0], e[1], p);
        else return hipErrorInvalidValue;
        err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    {
        dim3 grid(8 * ((p.max_tiles + 7) / 8) * ((p.d_model + PF_ROWS - 1) / PF_ROWS));
        if (hdn == T_Q5_0 && cdn == T_IQ4_NL) launch_pf(k_pf_down<T_Q5_0, T_IQ4_NL>, grid, s, e[2], e[3], p);
        else if (hdn == T_Q5_0 && cdn == T_Q5_0) launch_pf(k_pf_down<T_Q5_0, T_Q5_0>, grid, s, e[2], e[3], p);
        else if (hdn == T_IQ4_NL && cdn == T_IQ4_NL) launch_pf(k_pf_down<T_IQ4_NL, T_IQ4_NL>, grid, s, e[2], e[3], p);
        else if (hdn == T_IQ4_NL && cdn == T_Q5_0) launch_pf(k_pf_down<T_IQ4_NL, T_Q5_0>, grid, s, e[2], e[3], p);
        else return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace llapis
