// decode.hip -- the MoE layer for decode batches (1..4 tokens) in three
// kernels on gfx950:
//
//   A  k_dec_route   router logits (one workgroup per expert, all tokens) and
//                    the tokens' activation quantisation spread over the
//                    workgroups; for several tokens the last workgroup to
//                    finish also selects the routing (below) and writes the
//                    groups.
//   B  k_dec_gate_up per (expert group, 16-row block): for one token every
//                    workgroup selects the routing from the logits itself
//                    (softmax, top-k with DPP wave reductions, ties to the
//                    lower index), groups the routed pairs by expert (decode
//                    once, dot N: the tokens that share an expert read its
//                    slab once) and resolves each group's tier (the residency
//                    predicate of moert/cuda/ffn_moe.cu:80-130); the first
//                    workgroup publishes ids, weights and groups for C.  Then the
//                    expert's gate_up rows stream through LDS with 128-bit
//                    loads, dotted against every member token; a slice of the
//                    same expert's down slab can be prefetched into L2/MALL.
//   C  k_dec_down    per (expert group, 32-row block): GEGLU and down
//                    activation quantisation of the group's pairs in the
//                    prologue (while the weight loads are in flight), the down
//                    projection with the expert's .scale, and the combine:
//                    the last arrival of a (token, row block) writes the
//                    weighted sum of the token's top_k outputs for those rows.
//
// Hand-offs inside a kernel (A's logits, C's partial outputs) write with
// device-scope coherent stores, wait for their completion, then count
// arrivals with an atomic; the last arriver reads with device-scope coherent
// loads -- no L2 writeback or invalidate.  Whoever selects the routing (A's
// last workgroup, or B's first) clears C's counters for the call.
#include <hip/hip_ext.h>

#include <map>
#include <mutex>
#include <tuple>

#include "device.h"
#include "launch.h"

namespace llapis {
namespace dev {

__constant__ Iq2sTables c_iq2s_tab_dec = make_iq2s_tables();

template <int T> constexpr bool k256() { return T == T_Q4_K || T == T_IQ2_S; }
static_assert(DEC_MAXT == 4, "accumulator initialisers below assume four columns");

__device__ __forceinline__ void st_coh(float * p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coh(const float * p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// this thread's outstanding vector memory operations have completed
__device__ __forceinline__ void wait_vm() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// all threads' coherent stores are complete; thread 0 arrives on `counter`;
// returns (to every thread) whether this workgroup arrived last of `n`
__device__ __forceinline__ bool arrive_last(int * counter, int n, int * s_flag) {
    wait_vm();
    __syncthreads();
    if (threadIdx.x == 0) *s_flag = atomicAdd(counter, 1) == n - 1;
    __syncthreads();
    return *s_flag != 0;
}

__device__ __forceinline__ int member(const GroupInfo & g, int i) {
    return i == 0 ? g.mem[0] : i == 1 ? g.mem[1] : i == 2 ? g.mem[2] : g.mem[3];
}

__device__ __forceinline__ const uint8_t * group_slab(int tier, int idx, const uint8_t * hot, uint64_t hs,
                                                      const uint8_t * cold, uint64_t cs) {
    return tier == 0 ? hot + (uint64_t)idx * hs : cold + (uint64_t)idx * cs;
}

// ---------------------------------------------------------------- A

// Softmax + top-K of one token in one wave (ggml soft_max: exp(x - max), sum
// in double, scaled by float(1/sum); argsort_top_k: descending, equal
// probabilities in index order; weights p[ids] / max(sum, 6.103515625e-5)
// with the sum accumulated in double in id order).  E <= 256.
template <int NJ>
__device__ __forceinline__ float vmax(const float (&v)[4]) {
    float m = v[0];
#pragma unroll
    for (int j = 1; j < NJ; ++j) m = fmaxf(m, v[j]);
    return m;
}

template <int NJ>
__device__ void select_token_n(const float * logits, int E, int K, int32_t * ids, float * w, int * s_ids,
                               float * s_w) {
    const int lane = threadIdx.x & 63;
    float v[4];                 // entries lane + 64 j, j < NJ (the rest are never read)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int e = lane + 64 * j;
        v[j] = e < E ? ld_coh(logits + e) : -INFINITY;
    }
    const float mx = wave_max_dpp(vmax<NJ>(v));
    double ls = 0.0;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int e = lane + 64 * j;
        v[j] = e < E ? expf(v[j] - mx) : 0.0f;
        ls += (double)v[j];
    }
    ls = wave_sum_dpp(ls);
    const float inv = (float)(1.0 / ls);
#pragma unroll
    for (int j = 0; j < NJ; ++j) v[j] = lane + 64 * j < E ? __fmul_rn(v[j], inv) : -1.0f;
    // probabilities are >= 0; a taken entry drops to -1
    float sel = 0.0f;
    double sum = 0.0;
    for (int k = 0; k < K; ++k) {
        const float m = wave_max_dpp(vmax<NJ>(v));
        int e = -1;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const uint64_t b = __ballot(v[j] == m);
            if (e < 0 && b) e = 64 * j + __builtin_ctzll(b);
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j) if (lane + 64 * j == e) v[j] = -1.0f;
        sum += (double)m;
        if (lane == k) sel = m;
        if (lane == 0) {
            if (ids) ids[k] = e;
            s_ids[k] = e;
        }
    }
    float sf = (float)sum;
    if (sf < 6.103515625e-5f) sf = 6.103515625e-5f;
    if (lane < K) {
        if (w) w[lane] = sel / sf;
        if (s_w) s_w[lane] = sel / sf;
    }
}

// NJ = ceil(E / 64) entries per lane
__device__ void select_token(const float * logits, int E, int K, int32_t * ids, float * w, int * s_ids,
                             float * s_w = nullptr) {
    if (E <= 64) select_token_n<1>(logits, E, K, ids, w, s_ids, s_w);
    else if (E <= 128) select_token_n<2>(logits, E, K, ids, w, s_ids, s_w);
    else if (E <= 192) select_token_n<3>(logits, E, K, ids, w, s_ids, s_w);
    else select_token_n<4>(logits, E, K, ids, w, s_ids, s_w);
}

// Expert groups of the call from the routed ids in LDS (one wave): pairs that
// share an expert form one group (at most one member per token), in the order
// of their first pair; each group's tier by the residency predicate.
__device__ void build_groups(const DecParams & p, const int * s_ids, GroupInfo * groups, int * n_groups) {
    const int lane = threadIdx.x & 63;
    const int T = p.T, E = p.n_expert, P = T * p.top_k;
    const bool live = lane < P;
    const int ex = live ? s_ids[lane] : -1;
    int leader = lane, slot = 0, nmem = 0;
    for (int q = 0; q < P; ++q) {
        if (s_ids[q] == ex) {
            if (q < lane) ++slot;
            if (q < leader) leader = q;
            ++nmem;
        }
    }
    const bool is_leader = live && leader == lane;
    const uint64_t lm = __ballot(is_leader);
    const int gid = __popcll(lm & (leader == 0 ? 0ull : (~0ull >> (64 - leader))));
    if (is_leader) {
        int tier = 2, idx = 0;
        if (ex >= 0 && ex < E) {
            tier = 1;
            idx = ex;
            if (p.k_slots > 0) {
                const int s = p.exp_slot[ex];
                if (s >= 0 && s < p.k_slots && p.slot_state[s] == 2 && p.slot_exp[s] == ex) {
                    tier = 0;
                    idx = s;
                }
            }
        }
        groups[gid].tier = tier;
        groups[gid].idx = idx;
        groups[gid].n_mem = min(nmem, min(T, DEC_MAXT));     // one member per token at most
    }
    if (live && slot < DEC_MAXT) groups[gid].mem[slot] = lane;
    if (lane == 0) *n_groups = __popcll(lm);
}

// Router logits of expert e for every token (one workgroup), written with
// device-coherent stores.  Each lane issues all of its row loads (RU float4
// per pass) before any arithmetic.
__device__ void router_expert(const DecParams & p, int e, float (*s_part)[WG / 64]) {
    constexpr int RU = 4;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int d = p.d_model, E = p.n_expert, T = p.T, n4 = d / 4;
    const float4 * wrow = reinterpret_cast<const float4 *>(p.router_w + (int64_t)e * d);
    const float4 * x4 = reinterpret_cast<const float4 *>(p.x);
    float acc[DEC_MAXT];
#pragma unroll
    for (int t = 0; t < DEC_MAXT; ++t) acc[t] = 0.0f;
    for (int k0 = threadIdx.x; k0 < n4; k0 += RU * WG) {
        // clamped indices (row end, last token): every load is unconditional
        float4 w4[RU], xv[DEC_MAXT][RU];
#pragma unroll
        for (int u = 0; u < RU; ++u) w4[u] = wrow[min(k0 + u * WG, n4 - 1)];
#pragma unroll
        for (int t = 0; t < DEC_MAXT; ++t)
#pragma unroll
            for (int u = 0; u < RU; ++u) xv[t][u] = x4[(int64_t)min(t, T - 1) * n4 + min(k0 + u * WG, n4 - 1)];
#pragma unroll
        for (int t = 0; t < DEC_MAXT; ++t)
#pragma unroll
            for (int u = 0; u < RU; ++u)
                if (t < T && k0 + u * WG < n4)
                    acc[t] += w4[u].x * xv[t][u].x + w4[u].y * xv[t][u].y + w4[u].z * xv[t][u].z +
                              w4[u].w * xv[t][u].w;
    }
#pragma unroll
    for (int t = 0; t < DEC_MAXT; ++t) {
        const float s = wave_sum_dpp(acc[t]);
        if (lane == 0) s_part[t][wave] = s;
    }
    __syncthreads();
    if ((int)threadIdx.x < T) {
        const int t = threadIdx.x;
        float s = 0.0f;
#pragma unroll
        for (int q = 0; q < WG / 64; ++q) s += s_part[t][q];
        st_coh(p.logits + (int64_t)t * E + e, s + (p.router_b ? p.router_b[e] : 0.0f));
    }
}

// SEL: the last workgroup to finish also selects the routing and writes the
// groups (used for several tokens; for one token every gate_up workgroup
// selects it itself, which takes the selection off the critical path).
template <int AM, bool SEL>
__global__ __launch_bounds__(WG) void k_dec_route(const DecParams p) {
    __shared__ float s_part[DEC_MAXT][WG / 64];
    __shared__ int s_last;
    __shared__ int s_ids[DEC_PMAX];
    const int wave = threadIdx.x >> 6;
    const int gw = blockIdx.x * (WG / 64) + wave;          // wave id in the grid
    const int nw = gridDim.x * (WG / 64);
    const int d = p.d_model, E = p.n_expert, T = p.T, K = p.top_k;
    if ((int)blockIdx.x < E) router_expert(p, blockIdx.x, s_part);
    // the tokens' gate_up activations: one wave per 256-block (q8_K) or per
    // 64 values (q8_1)
    {
        ActView v;
        act_layout(d, 0, &v);
        const int per_tok = AM == AM_CPU ? d / 256 : (d + 63) / 64;
        for (int j = gw; j < T * per_tok; j += nw) {
            const int t = j / per_tok, b = j - t * per_tok;
            ActSrc src;
            src.p = p.x + (int64_t)t * d;
            src.n = d;
            uint8_t * col = p.xq + (int64_t)t * p.xq_stride;
            if (AM == AM_CPU) q8K_block<SRC_PLAIN>(col, v, src, b);
            else {
                const int pos = 64 * b + (threadIdx.x & 63);
                const bool live = pos < d;
                q8_32_put<AM_Q8_1>(col, v, live ? src.p[pos] : 0.0f, pos, live);
            }
        }
    }
    if (!SEL) return;
    if (!arrive_last(&p.ctl->route_count, gridDim.x, &s_last)) return;
    // ---- last workgroup: selection and groups
    if (wave < T) select_token(p.logits + (int64_t)wave * E, E, K, p.ids + wave * K, p.w + wave * K, s_ids + wave * K);
    for (int i = threadIdx.x; i < DEC_MAXT * p.n_rb_down; i += WG) p.comb_count[i] = 0;
    if (threadIdx.x == 0) p.ctl->route_count = 0;        // every workgroup has arrived
    __syncthreads();
    if (wave == 0) build_groups(p, s_ids, p.ctl->groups, &p.ctl->n_groups);
}

// The group record g written by A, or an empty group when g is past the
// call's groups.  Validated so that no field can send a load or store out of
// bounds: member count <= min(T, DEC_MAXT) and members < P, else the group is
// emptied; a tier other than 0/1 or an index outside its pool makes the group
// invalid (tier 2: its members contribute zeros, their combine still counts).
// The record and the count are read together (one round trip).
__device__ __forceinline__ GroupInfo validate_group(const DecParams & p, GroupInfo gi, int ng, int g) {
    const int P = p.T * p.top_k;
    bool ok = g < ng;
    gi.n_mem = max(0, min(gi.n_mem, min(p.T, DEC_MAXT)));
#pragma unroll
    for (int c = 0; c < DEC_MAXT; ++c)
        if (c < gi.n_mem && (gi.mem[c] < 0 || gi.mem[c] >= P)) ok = false;
    if (!ok) gi.n_mem = 0;
    const bool idx_ok = (gi.tier == 0 && gi.idx >= 0 && gi.idx < p.k_slots) ||
                        (gi.tier == 1 && gi.idx >= 0 && gi.idx < p.n_expert);
    if (!idx_ok) {
        gi.tier = 2;
        gi.idx = 0;
    }
    return gi;
}
__device__ __forceinline__ GroupInfo load_group(const DecParams & p, int g) {
    return validate_group(p, p.ctl->groups[g], p.ctl->n_groups, g);
}

// ---------------------------------------------------------------- B / C

constexpr int MAXPER_DEC = 8;

struct Staged {
    u32x4 r[MAXPER_DEC];
};

// loads of `nch` 16-byte chunks (issued now, stored to LDS later); lanes
// past the end re-read the last chunk so the loads carry no condition
__device__ __forceinline__ void stage_load(Staged & s, const u32x4 * g, int nch) {
    if (nch > 0) {
#pragma unroll
        for (int k = 0; k < MAXPER_DEC; ++k) s.r[k] = g[min((int)threadIdx.x + k * WG, nch - 1)];
    }
}
__device__ __forceinline__ void stage_store(const Staged & s, const u32x4 * g, int nch, uint8_t * smem, int at) {
    if (nch > 0) {
#pragma unroll
        for (int k = 0; k < MAXPER_DEC; ++k) {
            const int i = threadIdx.x + k * WG;
            if (i < nch) *reinterpret_cast<u32x4 *>(smem + at + 16 * i) = s.r[k];
        }
    }
    for (int i = threadIdx.x + MAXPER_DEC * WG; i < nch; i += WG) *reinterpret_cast<u32x4 *>(smem + at + 16 * i) = g[i];
}

__device__ __forceinline__ void copy16(uint8_t * smem, int at, const uint8_t * src, int n) {
    for (int i = threadIdx.x; i < n / 16; i += WG)
        *reinterpret_cast<u32x4 *>(smem + at + 16 * i) = reinterpret_cast<const u32x4 *>(src)[i];
}

// A small copy into LDS split in two: the first N chunks per thread are
// loaded into registers (issue), stored later (land), and any rest is copied
// in land.  Issued before the weight slab's loads, the copy's wait does not
// wait for the slab (loads complete in issue order).
template <int N>
struct Early {
    u32x4 r[N];
    __device__ __forceinline__ void issue(const void * src, int n16) {
        const u32x4 * g = reinterpret_cast<const u32x4 *>(src);
#pragma unroll
        for (int k = 0; k < N; ++k) {
            const int i = threadIdx.x + k * WG;
            if (i < n16) r[k] = g[i];
        }
    }
    __device__ __forceinline__ void land(uint8_t * dst, const void * src, int n16) const {
#pragma unroll
        for (int k = 0; k < N; ++k) {
            const int i = threadIdx.x + k * WG;
            if (i < n16) reinterpret_cast<u32x4 *>(dst)[i] = r[k];
        }
        const u32x4 * g = reinterpret_cast<const u32x4 *>(src);
        for (int i = threadIdx.x + N * WG; i < n16; i += WG) reinterpret_cast<u32x4 *>(dst)[i] = g[i];
    }
};
constexpr int TAB_CHUNKS = (int)(sizeof(Iq2sTables) / 16);

template <int HT, int CT, int AM, bool SEL>
__global__ __launch_bounds__(WG) __attribute__((amdgpu_waves_per_eu(1, 4))) void k_dec_gate_up(const DecParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int LPR = Fmt<HT>::LPR, ROWS = WG / LPR;
    static_assert(Fmt<HT>::LPR == Fmt<CT>::LPR && k256<HT>() && k256<CT>(), "gate_up formats");
    __shared__ int s_ids[DEC_PMAX];
    __shared__ GroupInfo s_grp[DEC_PMAX];
    __shared__ int s_ng;
    const int g = blockIdx.y;
    const int wave = threadIdx.x >> 6, T = p.T, K = p.top_k, E = p.n_expert;
    // IQ2_S codebook loads first: they depend on nothing; with the routing
    // selected here (one token) the member column is token 0's, so its loads
    // go out before the selection too
    Early<TAB_CHUNKS / WG> tab;
    if (HT == T_IQ2_S || CT == T_IQ2_S) tab.issue(&c_iq2s_tab_dec, TAB_CHUNKS);
    ActView tmp;
    const int abytes = act_layout(p.d_model, 0, &tmp);
    Early<2> col[DEC_MAXT];
    if (SEL) col[0].issue(p.xq, abytes / 16);
    GroupInfo gi;
    if (SEL) {
        // the routing: every workgroup selects it from the logits (identical
        // results); the first one publishes ids, weights and groups for the
        // down kernel and clears the combine counters
        const bool first = blockIdx.x == 0 && g == 0;
        if (wave < T)
            select_token(p.logits + (int64_t)wave * E, E, K, first ? p.ids + wave * K : nullptr,
                         first ? p.w + wave * K : nullptr, s_ids + wave * K);
        __syncthreads();
        if (wave == 0) build_groups(p, s_ids, s_grp, &s_ng);
        __syncthreads();
        const int ng = s_ng;
        if (first) {
            for (int i = threadIdx.x; i < DEC_MAXT * p.n_rb_down; i += WG) p.comb_count[i] = 0;
            for (int i = threadIdx.x; i < ng; i += WG) p.ctl->groups[i] = s_grp[i];
            if (threadIdx.x == 0) p.ctl->n_groups = ng;
        }
        gi = validate_group(p, s_grp[min(g, DEC_PMAX - 1)], ng, g);
    } else {
        gi = load_group(p, g);              // written by A's last workgroup
    }
    if (gi.n_mem == 0) return;
    const int F2 = 2 * p.n_ff, d_in = p.d_model;
    const bool valid = gi.tier < 2;
    const int wtype = gi.tier == 0 ? HT : CT;
    const int r0 = blockIdx.x * ROWS;
    const int rows = min(ROWS, F2 - r0);
    const int rb = (d_in / blk_elems(wtype)) * blk_bytes(wtype);
    const uint64_t start = (uint64_t)r0 * rb;
    const uint64_t c0 = start >> 4;
    const int nch = valid ? (int)(((start + (uint64_t)rows * rb + 15) >> 4) - c0) : 0;
    const uint8_t * W = valid ? group_slab(gi.tier, gi.idx, p.hot_gu, p.hot_gu_stride, p.cold_gu, p.cold_gu_stride)
                              : nullptr;
    const u32x4 * gW = reinterpret_cast<const u32x4 *>(W) + c0;

    // member columns first, then the slab
    const int n_mem = gi.n_mem;
    const bool iq2 = valid && wtype == T_IQ2_S;
    const uint8_t * csrc[DEC_MAXT];
#pragma unroll
    for (int c = 0; c < DEC_MAXT; ++c) {
        csrc[c] = p.xq + (int64_t)(member(gi, c) / p.top_k) * p.xq_stride;
        if (c < n_mem && !(SEL && c == 0)) col[c].issue(csrc[c], abytes / 16);
    }
    Staged st;
    stage_load(st, gW, nch);

    // prefetch this workgroup's slice of the expert's down slab (into L2/MALL)
    uint32_t sink = 0;
    if (p.prefetch && valid) {
        const u32x4 * D = reinterpret_cast<const u32x4 *>(
            group_slab(gi.tier, gi.idx, p.hot_dn, p.hot_dn_stride, p.cold_dn, p.cold_dn_stride));
        const uint64_t dstride = gi.tier == 0 ? p.hot_dn_stride : p.cold_dn_stride;
        const int dch = (int)(dstride >> 4);
        const int per = (dch + gridDim.x - 1) / gridDim.x;
        const int b0 = blockIdx.x * per, b1 = min(dch, b0 + per);
        for (int i = b0 + threadIdx.x; i < b1; i += WG) sink ^= D[i].x;
    }

    const int a0 = p.w_lds_gu;
    ActView av[DEC_MAXT];
#pragma unroll
    for (int c = 0; c < DEC_MAXT; ++c) act_layout(d_in, a0 + c * abytes, &av[c]);
#pragma unroll
    for (int c = 0; c < DEC_MAXT; ++c)
        if (c < n_mem) col[c].land(smem + a0 + c * abytes, csrc[c], abytes / 16);
    const int grid_off = align16i(a0 + min(p.T, DEC_MAXT) * abytes);
    if (iq2) tab.land(smem + grid_off, &c_iq2s_tab_dec, TAB_CHUNKS);
    stage_store(st, gW, nch, smem, 0);
    __syncthreads();

    const int rw = threadIdx.x / LPR, lr = threadIdx.x % LPR;
    float acc[DEC_MAXT] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (valid && rw < rows) {
        const int wb = (int)(start & 15) + rw * rb;
        const int U = d_in / Fmt<HT>::UNIT;
        if (gi.tier == 0) {
            if (n_mem == 1) {           // one member: the single-column unit
                for (int u = lr; u < U; u += LPR) unit_dot_n<HT, AM, 1>(smem, wb, u, av, n_mem, acc, grid_off);
            } else {
                for (int u = lr; u < U; u += LPR) unit_dot_n<HT, AM, DEC_MAXT>(smem, wb, u, av, n_mem, acc, grid_off);
            }
        } else {
            if (n_mem == 1) {           // one member: the single-column unit
                for (int u = lr; u < U; u += LPR) unit_dot_n<CT, AM, 1>(smem, wb, u, av, n_mem, acc, grid_off);
            } else {
                for (int u = lr; u < U; u += LPR) unit_dot_n<CT, AM, DEC_MAXT>(smem, wb, u, av, n_mem, acc, grid_off);
            }
        }
    }
#pragma unroll
    for (int c = 0; c < DEC_MAXT; ++c)
#pragma unroll
        for (int o = LPR / 2; o >= 1; o >>= 1) acc[c] += __shfl_xor(acc[c], o, LPR);
    if (lr == 0 && rw < rows) {
#pragma unroll
        for (int c = 0; c < DEC_MAXT; ++c)
            if (c < n_mem) p.ygu[(int64_t)member(gi, c) * F2 + r0 + rw] = acc[c];
    }
    if (p.never) p.ygu[threadIdx.x] = (float)sink;        // keeps the prefetch loads alive
}

// out = sum_k w_k y_k in k order (llama-graph.cpp:1812-1840), the K outputs
// loaded together (one round trip) before the ordered sum
constexpr int DEC_KMAX = 16;
__device__ __forceinline__ float combine_row(const float * y, const float * w, int K, int D) {
    float yv[DEC_KMAX];
#pragma unroll
    for (int k = 0; k < DEC_KMAX; ++k) yv[k] = k < K ? ld_coh(y + (int64_t)k * D) : 0.0f;
    float o = __fmul_rn(yv[0], w[0]);
#pragma unroll
    for (int k = 1; k < DEC_KMAX; ++k)
        if (k < K) o = __fadd_rn(o, __fmul_rn(yv[k], w[k]));
    return o;
}

template <int HT, int CT, int AM, int GSRC>
__global__ __launch_bounds__(WG) __attribute__((amdgpu_waves_per_eu(1, 4))) void k_dec_down(const DecParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int s_lastc[DEC_MAXT];
    constexpr int LPR = Fmt<HT>::LPR, ROWS = WG / LPR;
    static_assert(Fmt<HT>::LPR == Fmt<CT>::LPR && !k256<HT>() && !k256<CT>(), "down formats");
    const int g = blockIdx.y;
    const int D = p.d_model, d_in = p.n_ff, K = p.top_k;
    const GroupInfo gi = load_group(p, g);
    if (gi.n_mem == 0) return;
    const bool valid = gi.tier < 2;
    const int wtype = gi.tier == 0 ? HT : CT;
    const int r0 = blockIdx.x * ROWS;
    const int rows = min(ROWS, D - r0);
    const int rb = (d_in / blk_elems(wtype)) * blk_bytes(wtype);
    const uint64_t start = (uint64_t)r0 * rb;
    const uint64_t c0 = start >> 4;
    const int nch = valid ? (int)(((start + (uint64_t)rows * rb + 15) >> 4) - c0) : 0;
    const uint8_t * W = valid ? group_slab(gi.tier, gi.idx, p.hot_dn, p.hot_dn_stride, p.cold_dn, p.cold_dn_stride)
                              : nullptr;
    const u32x4 * gW = reinterpret_cast<const u32x4 *>(W) + c0;

    // the members' gate_up rows (first batch) are loaded before the slab, so
    // their GEGLU and quantisation overlap the slab's loads
    const int n_mem = gi.n_mem;
    const int at0 = (threadIdx.x >> 6) * 64;
    ActSrc src[DEC_MAXT];
    ActBatch ab[DEC_MAXT];
#pragma unroll
    for (int c = 0; c < DEC_MAXT; ++c) {
        src[c].p = p.ygu + (int64_t)member(gi, c) * 2 * d_in;
        src[c].n = d_in;
        if (c < n_mem) act_batch_load<GSRC>(ab[c], src[c], d_in, at0);
    }
    Staged st;
    stage_load(st, gW, nch);

    // GEGLU of the members' gate_up rows, quantised into LDS
    ActView tmp;
    const int abytes = act_layout(d_in, 0, &tmp);
    const int a0 = p.w_lds_dn;
    ActView av[DEC_MAXT];
#pragma unroll
    for (int c = 0; c < DEC_MAXT; ++c) act_layout(d_in, a0 + c * abytes, &av[c]);
#pragma unroll
    for (int c = 0; c < DEC_MAXT; ++c) {
        if (c >= n_mem) break;
        if (at0 < d_in) act_batch_quant<GSRC, AM>(smem, av[c], ab[c], d_in, at0);
        quantize_q8_32_rest<GSRC, AM>(smem, av[c], src[c], d_in);
    }
    stage_store(st, gW, nch, smem, 0);
    __syncthreads();

    const int rw = threadIdx.x / LPR, lr = threadIdx.x % LPR;
    float acc[DEC_MAXT] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (valid && rw < rows) {
        const int wb = (int)(start & 15) + rw * rb;
        const int U = d_in / Fmt<HT>::UNIT;
        if (gi.tier == 0) {
            if (n_mem == 1) {           // one member: the single-column unit
                for (int u = lr; u < U; u += LPR) unit_dot_n<HT, AM, 1>(smem, wb, u, av, n_mem, acc, 0);
            } else {
                for (int u = lr; u < U; u += LPR) unit_dot_n<HT, AM, DEC_MAXT>(smem, wb, u, av, n_mem, acc, 0);
            }
        } else {
            if (n_mem == 1) {           // one member: the single-column unit
                for (int u = lr; u < U; u += LPR) unit_dot_n<CT, AM, 1>(smem, wb, u, av, n_mem, acc, 0);
            } else {
                for (int u = lr; u < U; u += LPR) unit_dot_n<CT, AM, DEC_MAXT>(smem, wb, u, av, n_mem, acc, 0);
            }
        }
    }
#pragma unroll
    for (int c = 0; c < DEC_MAXT; ++c)
#pragma unroll
        for (int o = LPR / 2; o >= 1; o >>= 1) acc[c] += __shfl_xor(acc[c], o, LPR);
    const float sc = !valid ? 0.0f
                   : gi.tier == 0 ? (p.s_hot ? p.s_hot[gi.idx] : 1.0f) : (p.s_cold ? p.s_cold[gi.idx] : 1.0f);
    if (lr == 0 && rw < rows) {
#pragma unroll
        for (int c = 0; c < DEC_MAXT; ++c)
            if (c < n_mem) st_coh(p.ydn + (int64_t)member(gi, c) * D + r0 + rw, valid ? acc[c] * sc : 0.0f);
    }

    // ---- combine: the last pair of a token to finish these rows sums them
    wait_vm();
    __syncthreads();
    if ((int)threadIdx.x < n_mem) {
        const int t = member(gi, threadIdx.x) / K;
        s_lastc[threadIdx.x] = atomicAdd(&p.comb_count[t * p.n_rb_down + blockIdx.x], 1) == K - 1;
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < DEC_MAXT; ++c) {
        if (c >= n_mem) break;
        if (!s_lastc[c]) continue;
        const int t = member(gi, c) / K;
        const float * yt = p.ydn + (int64_t)t * K * D + r0;
        const float * wt = p.w + t * K;
        for (int r = threadIdx.x; r < rows; r += WG) p.out[(int64_t)t * D + r0 + r] = combine_row(yt + r, wt, K, D);
    }
}

// ------------------------------------------------------------ single kernel
//
// The layer in one launch.  Phases hand off through arrival counters in the
// control block; a consumer waits (thread 0, bounded by p.spin_limit ticks of
// the wall clock) until a counter reaches its target.  The grid is sized so
// every workgroup is resident (occupancy x CUs); a wait that times out sets
// ctl->error and the workgroup skips the rest of its work, so every wave
// still exits.
//   1  workgroup e < E: router logits of expert e (coherent stores, then one
//      arrival); every workgroup: the tokens quantised into its own LDS and
//      the IQ2_S tables
//   2  wait for the router (its last arrival sets a flag); every workgroup
//      selects the routing itself (DPP top-k per token) and builds the
//      expert groups in LDS
//   3  gate_up items (group, 16-row block) round-robin over the workgroups;
//      outputs with coherent stores, then one arrival on the group's counter
//      (the last one sets the group's flag)
//   4  down items (group, 32-row block): wait for the group's flag, GEGLU +
//      quantise its members (coherent loads), down, combine
//   5  the last workgroup out resets every counter for the next call

__device__ __forceinline__ int ld_coh_i(const int * q) {
    return __hip_atomic_load(const_cast<int *>(q), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Thread 0 waits until the write-once flag is set (polling with a short
// sleep; the counters themselves are only touched by their arrivals), or
// until the wall-clock bound passes; the result is broadcast.
__device__ bool wait_flag(const DecParams & p, const int * flag, int * s_flag) {
    if (threadIdx.x == 0) {
        int ok = 1;
        const long long t0 = wall_clock64();
        while (ld_coh_i(flag) == 0) {
            if (wall_clock64() - t0 > p.spin_limit) {
                ok = 0;
                __hip_atomic_store(&p.ctl->error, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(4);
        }
        *s_flag = ok;
    }
    __syncthreads();
    return *s_flag != 0;
}

// thread 0: one arrival on `ctr`; the arrival that completes `target` sets
// the flag (after this workgroup's coherent stores have completed)
__device__ __forceinline__ void arrive_flag(int * ctr, int target, int * flag) {
    if (threadIdx.x == 0 && atomicAdd(ctr, 1) == target - 1)
        __hip_atomic_store(flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int HT, int CT, int HD, int CD, int AM, int GSRC>
__global__ __launch_bounds__(WG) __attribute__((amdgpu_waves_per_eu(1, 4))) void k_dec_fused(const DecParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float s_part[DEC_MAXT][WG / 64];
    __shared__ int s_ids[DEC_PMAX];
    __shared__ float s_wt[DEC_PMAX];
    __shared__ GroupInfo s_grp[DEC_PMAX];
    __shared__ int s_ng, s_flag, s_lastc[DEC_MAXT];
    constexpr int LPR_G = Fmt<HT>::LPR, ROWS_G = WG / LPR_G;
    constexpr int LPR_D = Fmt<HD>::LPR, ROWS_D = WG / LPR_D;
    static_assert(Fmt<HT>::LPR == Fmt<CT>::LPR && k256<HT>() && k256<CT>(), "gate_up formats");
    static_assert(Fmt<HD>::LPR == Fmt<CD>::LPR && !k256<HD>() && !k256<CD>(), "down formats");
    const int wave = threadIdx.x >> 6;
    const int d = p.d_model, F = p.n_ff, E = p.n_expert, T = p.T, K = p.top_k;
    const int F2 = 2 * F;
    const int NRB_G = (F2 + ROWS_G - 1) / ROWS_G, NRB_D = (d + ROWS_D - 1) / ROWS_D;

    // ---- phase 1
    if ((int)blockIdx.x < E) {
        router_expert(p, blockIdx.x, s_part);
        wait_vm();
        __syncthreads();
        arrive_flag(&p.ctl->route_count, E, &p.ctl->route_ready);
    }
    ActView tmp;
    const int abg = act_layout(d, 0, &tmp);
    const int ag0 = p.w_lds_gu;
    // token t's column: the layout at ag0 shifted by t * abg
    ActView av0;
    act_layout(d, ag0, &av0);
    // each token is staged in LDS (the weight region, free until phase 3)
    // with one round of 16-byte loads, then quantised from there
    for (int t = 0; t < T; ++t) {
        const u32x4 * xs = reinterpret_cast<const u32x4 *>(p.x + (int64_t)t * d);
        for (int i = threadIdx.x; i < d / 4; i += WG) reinterpret_cast<u32x4 *>(smem)[i] = xs[i];
        __syncthreads();
        ActView v;
        act_layout(d, ag0 + t * abg, &v);
        ActSrc src;
        src.p = reinterpret_cast<const float *>(smem);
        src.n = d;
        quantize_act<HT, AM, SRC_PLAIN>(smem, v, src, d);
        __syncthreads();
    }
    const int grid_off = align16i(ag0 + min(T, DEC_MAXT) * abg);
    if (HT == T_IQ2_S || CT == T_IQ2_S) copy_iq2s_tables(smem, grid_off, &c_iq2s_tab_dec);

    // ---- phase 2
    bool ok = wait_flag(p, &p.ctl->route_ready, &s_flag);
    if (ok && wave < T) select_token(p.logits + (int64_t)wave * E, E, K, nullptr, nullptr, s_ids + wave * K, s_wt + wave * K);
    __syncthreads();
    if (ok && wave == 0) build_groups(p, s_ids, s_grp, &s_ng);
    __syncthreads();
    if (ok && blockIdx.x == 0 && (int)threadIdx.x < T * K) {
        p.ids[threadIdx.x] = s_ids[threadIdx.x];
        p.w[threadIdx.x] = s_wt[threadIdx.x];
    }
    const int ng = ok ? min(s_ng, DEC_PMAX) : 0;

    // ---- phase 3: gate_up
    for (int it = blockIdx.x; it < ng * NRB_G; it += gridDim.x) {
        const int g = it / NRB_G, rbi = it - g * NRB_G;
        const GroupInfo gi = s_grp[g];
        const bool valid = gi.tier < 2;
        const int wtype = gi.tier == 0 ? HT : CT;
        const int r0 = rbi * ROWS_G;
        const int rows = min(ROWS_G, F2 - r0);
        const int rb = (d / blk_elems(wtype)) * blk_bytes(wtype);
        const uint64_t start = (uint64_t)r0 * rb;
        const uint64_t c0 = start >> 4;
        const int nch = valid ? (int)(((start + (uint64_t)rows * rb + 15) >> 4) - c0) : 0;
        const uint8_t * W = valid ? group_slab(gi.tier, gi.idx, p.hot_gu, p.hot_gu_stride, p.cold_gu, p.cold_gu_stride)
                                  : nullptr;
        const u32x4 * gW = reinterpret_cast<const u32x4 *>(W) + c0;
        Staged st;
        stage_load(st, gW, nch);
        stage_store(st, gW, nch, smem, 0);
        __syncthreads();
        const int rw = threadIdx.x / LPR_G, lr = threadIdx.x % LPR_G;
        float acc[DEC_MAXT] = {0.0f, 0.0f, 0.0f, 0.0f};
        const int n_mem = gi.n_mem;
        if (valid && rw < rows) {
            const int wb = (int)(start & 15) + rw * rb;
            const int U = d / Fmt<HT>::UNIT;
            // member c's activation column is its token's
            ActView avm[DEC_MAXT];
#pragma unroll
            for (int c = 0; c < DEC_MAXT; ++c) {
                const int sh = max(0, min(member(gi, c) / K, T - 1)) * abg;   // slots past n_mem are unused
                avm[c] = ActView{av0.q + sh, av0.d32 + sh, av0.s32 + sh, av0.dK + sh, av0.bsum + sh};
            }
            if (gi.tier == 0) {
                if (n_mem == 1) {           // one member: the single-column unit
                    for (int u = lr; u < U; u += LPR_G) unit_dot_n<HT, AM, 1>(smem, wb, u, avm, n_mem, acc, grid_off);
                } else {
                    for (int u = lr; u < U; u += LPR_G) unit_dot_n<HT, AM, DEC_MAXT>(smem, wb, u, avm, n_mem, acc, grid_off);
                }
            } else {
                if (n_mem == 1) {           // one member: the single-column unit
                    for (int u = lr; u < U; u += LPR_G) unit_dot_n<CT, AM, 1>(smem, wb, u, avm, n_mem, acc, grid_off);
                } else {
                    for (int u = lr; u < U; u += LPR_G) unit_dot_n<CT, AM, DEC_MAXT>(smem, wb, u, avm, n_mem, acc, grid_off);
                }
            }
        }
#pragma unroll
        for (int c = 0; c < DEC_MAXT; ++c)
#pragma unroll
            for (int o = LPR_G / 2; o >= 1; o >>= 1) acc[c] += __shfl_xor(acc[c], o, LPR_G);
        if (lr == 0 && rw < rows) {
#pragma unroll
            for (int c = 0; c < DEC_MAXT; ++c)
                if (c < n_mem) st_coh(p.ygu + (int64_t)member(gi, c) * F2 + r0 + rw, acc[c]);
        }
        wait_vm();
        __syncthreads();
        arrive_flag(&p.ctl->group_count[g], NRB_G, &p.ctl->group_ready[g]);
    }

    // ---- phase 4: down (its LDS reuses the gate_up region)
    ActView tmpd;
    const int abd = act_layout(F, 0, &tmpd);
    const int ad0 = p.w_lds_dn;
    ActView avd[DEC_MAXT];
#pragma unroll
    for (int c = 0; c < DEC_MAXT; ++c) act_layout(F, ad0 + c * abd, &avd[c]);
    constexpr int GCOH = GSRC == SRC_GEGLU_TANH ? SRC_GEGLU_TANH_COH : SRC_GEGLU_TABLE_COH;
    for (int it = blockIdx.x; ok && it < ng * NRB_D; it += gridDim.x) {
        const int g = it / NRB_D, rbi = it - g * NRB_D;
        __syncthreads();                        // the previous item (or phase 3) is done with LDS
        if (!wait_flag(p, &p.ctl->group_ready[g], &s_flag)) {
            ok = false;
            break;
        }
        const GroupInfo gi = s_grp[g];
        const bool valid = gi.tier < 2;
        const int wtype = gi.tier == 0 ? HD : CD;
        const int r0 = rbi * ROWS_D;
        const int rows = min(ROWS_D, d - r0);
        const int rb = (F / blk_elems(wtype)) * blk_bytes(wtype);
        const uint64_t start = (uint64_t)r0 * rb;
        const uint64_t c0 = start >> 4;
        const int nch = valid ? (int)(((start + (uint64_t)rows * rb + 15) >> 4) - c0) : 0;
        const uint8_t * W = valid ? group_slab(gi.tier, gi.idx, p.hot_dn, p.hot_dn_stride, p.cold_dn, p.cold_dn_stride)
                                  : nullptr;
        const u32x4 * gW = reinterpret_cast<const u32x4 *>(W) + c0;
        Staged st;
        stage_load(st, gW, nch);
        const int n_mem = gi.n_mem;
#pragma unroll
        for (int c = 0; c < DEC_MAXT; ++c) {
            if (c >= n_mem) break;
            ActSrc src;
            src.p = p.ygu + (int64_t)member(gi, c) * F2;
            src.n = F;
            quantize_act<T_Q5_0, AM, GCOH>(smem, avd[c], src, F);
        }
        stage_store(st, gW, nch, smem, 0);
        __syncthreads();
        const int rw = threadIdx.x / LPR_D, lr = threadIdx.x % LPR_D;
        float acc[DEC_MAXT] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (valid && rw < rows) {
            const int wb = (int)(start & 15) + rw * rb;
            const int U = F / Fmt<HD>::UNIT;
            if (gi.tier == 0) {
                if (n_mem == 1) {           // one member: the single-column unit
                    for (int u = lr; u < U; u += LPR_D) unit_dot_n<HD, AM, 1>(smem, wb, u, avd, n_mem, acc, 0);
                } else {
                    for (int u = lr; u < U; u += LPR_D) unit_dot_n<HD, AM, DEC_MAXT>(smem, wb, u, avd, n_mem, acc, 0);
                }
            } else {
                if (n_mem == 1) {           // one member: the single-column unit
                    for (int u = lr; u < U; u += LPR_D) unit_dot_n<CD, AM, 1>(smem, wb, u, avd, n_mem, acc, 0);
                } else {
                    for (int u = lr; u < U; u += LPR_D) unit_dot_n<CD, AM, DEC_MAXT>(smem, wb, u, avd, n_mem, acc, 0);
                }
            }
        }
#pragma unroll
        for (int c = 0; c < DEC_MAXT; ++c)
#pragma unroll
            for (int o = LPR_D / 2; o >= 1; o >>= 1) acc[c] += __shfl_xor(acc[c], o, LPR_D);
        const float sc = !valid ? 0.0f
                       : gi.tier == 0 ? (p.s_hot ? p.s_hot[gi.idx] : 1.0f) : (p.s_cold ? p.s_cold[gi.idx] : 1.0f);
        if (lr == 0 && rw < rows) {
#pragma unroll
            for (int c = 0; c < DEC_MAXT; ++c)
                if (c < n_mem) st_coh(p.ydn + (int64_t)member(gi, c) * d + r0 + rw, valid ? acc[c] * sc : 0.0f);
        }
        // combine: the last pair of a token to finish these rows sums them
        wait_vm();
        __syncthreads();
        if ((int)threadIdx.x < n_mem) {
            const int t = member(gi, threadIdx.x) / K;
            s_lastc[threadIdx.x] = atomicAdd(&p.comb_count[t * p.n_rb_down + rbi], 1) == K - 1;
        }
        __syncthreads();
#pragma unroll
        for (int c = 0; c < DEC_MAXT; ++c) {
            if (c >= n_mem) break;
            if (!s_lastc[c]) continue;
            const int t = member(gi, c) / K;
            const float * yt = p.ydn + (int64_t)t * K * d + r0;
            const float * wt = s_wt + t * K;
            for (int r = threadIdx.x; r < rows; r += WG) p.out[(int64_t)t * d + r0 + r] = combine_row(yt + r, wt, K, d);
        }
    }

    // ---- phase 5
    wait_vm();
    __syncthreads();
    if (threadIdx.x == 0) s_flag = atomicAdd(&p.ctl->done_count, 1) == (int)gridDim.x - 1;
    __syncthreads();
    if (s_flag) {
        for (int i = threadIdx.x; i < DEC_MAXT * p.n_rb_down; i += WG) p.comb_count[i] = 0;
        for (int i = threadIdx.x; i < DEC_PMAX; i += WG) {
            p.ctl->group_count[i] = 0;
            p.ctl->group_ready[i] = 0;
        }
        if (threadIdx.x == 0) {
            p.ctl->route_count = 0;
            p.ctl->route_ready = 0;
            p.ctl->done_count = 0;
        }
    }
}

__global__ void k_zero(int * p, int n) {
    for (int i = blockIdx.x * WG + threadIdx.x; i < n; i += gridDim.x * WG) p[i] = 0;
}

}  // namespace dev

using namespace dev;

int dec_act_bytes(int n) {
    ActView v;
    return act_layout(n, 0, &v);
}

// dynamic LDS: staged weights, one activation column per token of the call
// (a group has at most one member per token), IQ2_S tables when used
int dec_lds_gate_up(const DecParams & p, int ht, int ct) {
    ActView v;
    const int ab = act_layout(p.d_model, 0, &v);
    const bool iq2 = ht == T_IQ2_S || ct == T_IQ2_S;
    return align16i(p.w_lds_gu + std::min(p.T, DEC_MAXT) * ab) + (iq2 ? (int)sizeof(Iq2sTables) : 0);
}

int dec_lds_down(const DecParams & p) {
    ActView v;
    const int ab = act_layout(p.n_ff, 0, &v);
    return p.w_lds_dn + std::min(p.T, DEC_MAXT) * ab;
}

namespace {
// launch with the dispatch's own begin/end timestamps recorded into e0/e1
// when profiling (e0 != nullptr)
template <typename F>
void launch_timed(F k, dim3 grid, int lds, hipStream_t s, hipEvent_t e0, hipEvent_t e1, const DecParams & p) {
    if (e0) hipExtLaunchKernelGGL(k, grid, dim3(WG), (uint32_t)lds, s, e0, e1, 0u, p);
    else hipLaunchKernelGGL(k, grid, dim3(WG), lds, s, p);
}
}  // namespace

hipError_t launch_decode(const DecParams & p, int hgu, int cgu, int hdn, int cdn, int am, int gelu, hipStream_t s,
                         hipEvent_t * ev) {
    hipEvent_t e[6] = {};
    if (ev)
        for (int i = 0; i < 6; ++i) e[i] = ev[i];
    const int P = p.T * p.top_k;
    {
        const int per_tok = am == AM_CPU ? p.d_model / 256 : (p.d_model + 63) / 64;
        dim3 grid(std::max(p.n_expert, (p.T * per_tok + 3) / 4));
        // one token: selection in every gate_up workgroup; more: in A
        const bool sel_a = p.T > 1;
        if (am == AM_CPU) {
            if (sel_a) launch_timed(k_dec_route<AM_CPU, true>, grid, 0, s, e[0], e[1], p);
            else launch_timed(k_dec_route<AM_CPU, false>, grid, 0, s, e[0], e[1], p);
        } else {
            if (sel_a) launch_timed(k_dec_route<AM_Q8_1, true>, grid, 0, s, e[0], e[1], p);
            else launch_timed(k_dec_route<AM_Q8_1, false>, grid, 0, s, e[0], e[1], p);
        }
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    {
        dim3 grid((2 * p.n_ff + 15) / 16, P);
        const int lds = dec_lds_gate_up(p, hgu, cgu);
#define LL_GU(A, B, M) \
        if (hgu == A && cgu == B && am == M) { \
            if (p.T > 1) launch_timed(k_dec_gate_up<A, B, M, false>, grid, lds, s, e[2], e[3], p); \
            else launch_timed(k_dec_gate_up<A, B, M, true>, grid, lds, s, e[2], e[3], p); \
        } else
#define LL_GU2(A, B) LL_GU(A, B, AM_CPU) LL_GU(A, B, AM_Q8_1)
        LL_GU2(T_Q4_K, T_IQ2_S) LL_GU2(T_Q4_K, T_Q4_K) LL_GU2(T_IQ2_S, T_IQ2_S) LL_GU2(T_IQ2_S, T_Q4_K)
        return hipErrorInvalidValue;
#undef LL_GU2
#undef LL_GU
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    {
        dim3 grid(p.n_rb_down, P);
        const int lds = dec_lds_down(p);
#define LL_DN(A, B, M, G) \
        if (hdn == A && cdn == B && am == M && gelu == G) launch_timed(k_dec_down<A, B, M, G>, grid, lds, s, e[4], e[5], p); else
#define LL_DN2(A, B) LL_DN(A, B, AM_CPU, SRC_GEGLU_TABLE) LL_DN(A, B, AM_CPU, SRC_GEGLU_TANH) \
                     LL_DN(A, B, AM_Q8_1, SRC_GEGLU_TABLE) LL_DN(A, B, AM_Q8_1, SRC_GEGLU_TANH)
        LL_DN2(T_Q5_0, T_IQ4_NL) LL_DN2(T_Q5_0, T_Q5_0) LL_DN2(T_IQ4_NL, T_IQ4_NL) LL_DN2(T_IQ4_NL, T_Q5_0)
        return hipErrorInvalidValue;
#undef LL_DN2
#undef LL_DN
    }
    return hipGetLastError();
}

namespace {
// resident workgroups of a kernel on the current device (cached per device
// and instantiation; LDS bytes are part of the key)
template <typename F>
int resident_wgs(F k, int lds) {
    static std::mutex mu;
    static std::map<std::tuple<int, const void *, int>, int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    const auto key = std::make_tuple(dev, reinterpret_cast<const void *>(k), lds);
    std::lock_guard<std::mutex> lk(mu);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, WG, lds) != hipSuccess) per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) cus = 0;
    const int n = per_cu * cus;
    cache[key] = n;
    return n;
}
}  // namespace

hipError_t launch_decode_fused(const DecParams & p, int hgu, int cgu, int hdn, int cdn, int am, int gelu, hipStream_t s,
                               hipEvent_t * ev) {
    if (!(hgu == T_Q4_K && cgu == T_IQ2_S && hdn == T_Q5_0 && cdn == T_IQ4_NL)) return hipErrorNotSupported;
    const int lds = std::max(dec_lds_gate_up(p, hgu, cgu), dec_lds_down(p));
    const int P = p.T * p.top_k;
    const int items = P * std::max((2 * p.n_ff + 15) / 16, p.n_rb_down);
    auto go = [&](auto k) -> hipError_t {
        const int cap = resident_wgs(k, lds);
        const int want = std::max(p.n_expert, items);
        const int grid = std::min(cap, want);
        if (cap < p.n_expert || grid < 1) return hipErrorNotSupported;   // the router needs E resident workgroups
        launch_timed(k, dim3(grid), lds, s, ev ? ev[0] : nullptr, ev ? ev[1] : nullptr, p);
        return hipGetLastError();
    };
    if (am == AM_CPU && gelu == SRC_GEGLU_TANH) return go(k_dec_fused<T_Q4_K, T_IQ2_S, T_Q5_0, T_IQ4_NL, AM_CPU, SRC_GEGLU_TANH>);
    if (am == AM_CPU) return go(k_dec_fused<T_Q4_K, T_IQ2_S, T_Q5_0, T_IQ4_NL, AM_CPU, SRC_GEGLU_TABLE>);
    if (gelu == SRC_GEGLU_TANH) return go(k_dec_fused<T_Q4_K, T_IQ2_S, T_Q5_0, T_IQ4_NL, AM_Q8_1, SRC_GEGLU_TANH>);
    return go(k_dec_fused<T_Q4_K, T_IQ2_S, T_Q5_0, T_IQ4_NL, AM_Q8_1, SRC_GEGLU_TABLE>);
}

hipError_t launch_zero_i32(int * p, int n, hipStream_t s) {
    hipLaunchKernelGGL(k_zero, dim3(std::min(1024, (n + WG - 1) / WG)), dim3(WG), 0, s, p, n);
    return hipGetLastError();
}

}  // namespace llapis
