// decode.hip -- the MoE layer for decode batches (1..4 tokens) on gfx950,
// and the one-kernel fires of the dual op.
//
//   A  k_dec_route     router logits (one workgroup per expert, all tokens)
//                      and, in the workgroups after those, the tokens'
//                      activation quantisation.
//   B  k_dec_gate_up   every workgroup selects the routing from the logits
//                      (softmax, then the top-k largest probabilities taken
//                      one by one, ties to the lower index), groups the
//                      routed pairs by expert (the tokens that share an expert
//                      read its slab once) and resolves each group's tier (the
//                      residency predicate of moert/cuda/ffn_moe.cu:80-130);
//                      the first workgroup publishes ids, weights and groups.
//                      Then its item: one group's 32 gate rows and the 32 up
//                      rows paired with them (rows i and n_ff + i), in four
//                      passes of 8 + 8 rows, one row per 16 lanes, the next
//                      passes' loads in flight; the rows are dotted against
//                      every member token, GEGLU pairs them, and the item ends
//                      with each member's 32 values quantised (q8_0 / q8_1):
//                      one block of the pair's down activation, quantised once.
//   C  k_dec_down      one workgroup per block of output rows over every
//                      group; each row's lanes load its block pairs straight
//                      into registers and dot them against the members'
//                      quantised down columns (copied into LDS), scale by the
//                      expert's .scale and sum each token's top_k outputs in k
//                      order (llama-graph.cpp:1812-1840).
//
//   k_fire_k256 / k_fire_k32: one GGML_OP_MOE_DUAL fire (gate_up over the
//   256-value block formats, down over the 32-value ones) as one kernel.
//
// No workgroup waits on another: every hand-over is a kernel boundary, so any
// grid is safe.  Every load a kernel issues before its first wait is
// unconditional (clamped addresses instead of branches) and issued in the
// order its data are needed: loads complete in issue order, so a wait covers
// only the loads before it.
#include <hip/hip_ext.h>

#include <climits>
#include <map>
#include <mutex>
#include <tuple>

#include "device.h"
#include "launch.h"

namespace llapis {
namespace dev {

__constant__ Iq2sTables c_iq2s_tab_dec = make_iq2s_tables();

template <int T> constexpr bool k256() { return T == T_Q4_K || T == T_IQ2_S; }
inline bool k256_type(int t) { return t == T_Q4_K || t == T_IQ2_S; }
static_assert(DEC_MAXT == 4, "one member column per wave in the gate_up epilogue");

__device__ __forceinline__ int member(const GroupInfo & g, int i) {
    return i == 0 ? g.mem[0] : i == 1 ? g.mem[1] : i == 2 ? g.mem[2] : g.mem[3];
}

__device__ __forceinline__ const uint8_t * group_slab(int tier, int idx, const uint8_t * hot, uint64_t hs,
                                                      const uint8_t * cold, uint64_t cs) {
    return tier == 0 ? hot + (uint64_t)idx * hs : cold + (uint64_t)idx * cs;
}

__device__ __forceinline__ uint64_t lanes_below() {
    const int lane = threadIdx.x & 63;
    return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// ---------------------------------------------------------------- A

// Router logits of expert e for every token (one workgroup), from the
// router's input p.xr.  Each lane issues all of its row loads (RU float4 per
// pass) before any arithmetic.
__device__ void router_expert(const DecParams & p, int e, float (*s_part)[WG / 64]) {
    constexpr int RU = 4;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int d = p.d_model, E = p.n_expert, T = p.T, n4 = d / 4;
    const float4 * wrow = reinterpret_cast<const float4 *>(p.router_w + (int64_t)e * d);
    const float4 * x4 = reinterpret_cast<const float4 *>(p.xr);
    const float bias = p.router_b ? p.router_b[e] : 0.0f;     // issued with the row's loads
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
        p.logits[(int64_t)t * E + e] = s + bias;
    }
}

// Router logits of every token (workgroups e < E, one expert each, from the
// router's input) and the quantisation of the experts' input for gate_up
// (the workgroups after them: one wave per q8_K 256-block, or per 64 values
// of q8_1).
template <int AM>
__global__ __launch_bounds__(WG) void k_dec_route(const DecParams p) {
    __shared__ float s_part[DEC_MAXT][WG / 64];
    const int E = p.n_expert;
    if ((int)blockIdx.x < E) {
        router_expert(p, blockIdx.x, s_part);
        return;
    }
    const int d = p.d_model, T = p.T;
    const int gw = ((int)blockIdx.x - E) * (WG / 64) + (int)(threadIdx.x >> 6);
    const int nw = ((int)gridDim.x - E) * (WG / 64);
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

// ------------------------------------------------------------ routing

// order-preserving map of floats to ints (larger float <=> larger signed int)
__device__ __forceinline__ int f2o(float f) {
    const int b = __float_as_int(f);
    return b ^ ((b >> 31) & 0x7FFFFFFF);
}
__device__ __forceinline__ float o2f(int o) { return __int_as_float(o ^ ((o >> 31) & 0x7FFFFFFF)); }
// wave64 integer maximum (one DPP step each), wave-uniform
__device__ __forceinline__ int wave_max_i(int v) {
    v = max(v, dpp_i<0xB1>(v, v));
    v = max(v, dpp_i<0x4E>(v, v));
    v = max(v, dpp_i<0x141>(v, v));
    v = max(v, dpp_i<0x140>(v, v));
    v = max(v, dpp_i<0x142, 0xA>(v, v));
    v = max(v, dpp_i<0x143, 0xC>(v, v));
    return __builtin_amdgcn_readlane(v, 63);
}

constexpr int DEC_KMAX = 16;    // top_k of a decode call, at most

// one wave's scratch for ordering its selected entries
struct SelScratch {
    int key[DEC_KMAX], idx[DEC_KMAX];
};

// Softmax + top-K of one token in one wave, from its logits in registers
// (v[j] = entry lane + 64 j; entries at or past E are ignored), as ggml's CPU
// graph computes them (soft_max: exp(x - max), the sum in double,
// probabilities scaled by float(1/sum); argsort_top_k: descending, equal
// probabilities in index order; weights p / max(sum of the K in double, in
// order, 6.103515625e-5)).  Probabilities are >= 0, so they compare as ints.
// The K-th largest probability is found by bisection over its bits (the
// largest t with at least K probabilities >= t: one ballot count per step),
// stopping early once exactly K entries are >= t; the entries above it and
// the lowest-indexed ones equal to it are taken, and each taken entry's rank
// (larger first, then the lower index) counts the taken entries before it,
// read from the lanes.  No cross-lane shuffles in the loops; one LDS round
// trip orders the K entries.  ids and weights go to LDS when `wr`; entries
// past the valid ones (K > E) get id -1 and weight 0.
template <int NJ>
__device__ __forceinline__ void select_topk(const float (&v)[4], int E, int K, int * s_ids, float * s_w, bool wr,
                                            SelScratch & sc) {
    const int lane = threadIdx.x & 63;
    int mo = INT_MIN;
#pragma unroll
    for (int j = 0; j < NJ; ++j) mo = max(mo, lane + 64 * j < E ? f2o(v[j]) : INT_MIN);
    const float mx = o2f(wave_max_i(mo));
    float ev[NJ];
    double ls = 0.0;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        ev[j] = lane + 64 * j < E ? expf(v[j] - mx) : 0.0f;
        ls += (double)ev[j];
    }
    ls = wave_sum_dpp(ls);
    const float inv = (float)(1.0 / ls);
    int q[NJ];                  // probabilities as ints; -1: absent
#pragma unroll
    for (int j = 0; j < NJ; ++j) q[j] = lane + 64 * j < E ? __float_as_int(__fmul_rn(ev[j], inv)) : -1;
    // the threshold (probabilities are at most 1.0f: below 0x40000000)
    int nv = 0;
#pragma unroll
    for (int j = 0; j < NJ; ++j) nv += __popcll(__ballot(q[j] >= 0));
    const int kk = min(K, nv);
    int lo = 0, hi = 0x40000000;
    bool exact = nv == kk;              // every valid entry is taken
    while (!exact && hi - lo > 1) {
        const int c = lo + ((hi - lo) >> 1);
        int n = 0;
#pragma unroll
        for (int j = 0; j < NJ; ++j) n += __popcll(__ballot(q[j] >= c));
        if (n >= kk) {
            lo = c;
            exact = n == kk;
        } else {
            hi = c;
        }
    }
    // the taken entries: those >= lo when exactly kk are; otherwise lo is the
    // kk-th largest value: those above it, then the lowest-indexed equal ones
    uint64_t sel[NJ];
    if (exact) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) sel[j] = __ballot(q[j] >= lo);
    } else {
        int need = kk;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            sel[j] = __ballot(q[j] > lo);
            need -= __popcll(sel[j]);
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            uint64_t eq = __ballot(q[j] == lo);
            while (need > 0 && eq) {
                const uint64_t b = eq & (~eq + 1);
                sel[j] |= b;
                eq ^= b;
                --need;
            }
        }
    }
    // ranks of this lane's taken entries
    int rank[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) rank[j] = 0;
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) {
        uint64_t m = sel[jj];
        while (m) {
            const int l = (int)__builtin_ctzll(m);
            m &= m - 1;
            const int kq = __builtin_amdgcn_readlane(q[jj], l), ki = l + 64 * jj;
#pragma unroll
            for (int j = 0; j < NJ; ++j)
                rank[j] += (kq > q[j] || (kq == q[j] && ki < lane + 64 * j)) ? 1 : 0;
        }
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j)
        if ((sel[j] >> lane) & 1) {
            sc.key[rank[j]] = q[j];
            sc.idx[rank[j]] = lane + 64 * j;
        }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int mine = min(lane, DEC_KMAX - 1);
    const int myid = lane < kk ? sc.idx[mine] : -1;
    const int mykey = lane < kk ? sc.key[mine] : 0;
    double sum = 0.0;
    for (int k = 0; k < kk; ++k) sum += (double)__int_as_float(__builtin_amdgcn_readlane(mykey, k));
    float sf = (float)sum;
    if (sf < 6.103515625e-5f) sf = 6.103515625e-5f;
    if (wr && lane < K) {
        s_ids[lane] = myid;
        s_w[lane] = __int_as_float(mykey) / sf;
    }
}

// Expert groups of the call from the routed ids in LDS (one wave): pairs that
// share an expert form one group (at most one member per token: a token's
// top-k experts are distinct), in the order of their first pair; each
// group's tier by the residency predicate, read from es/se/ss (the
// exp_slot/slot_exp/slot_state mirrors or copies of them).  s_first[e] must
// hold 64 and s_tm[e] 0 for every e < E on entry (s_gid is scratch): the
// pairs of expert e meet there by LDS atomics (its first pair, the tokens
// that chose it), so no step loops over the pairs.  A pair with an invalid
// id forms a group of its own (tier 2).
__device__ void build_groups(const DecParams & p, const int * s_ids, GroupInfo * groups, int * n_groups,
                             const int32_t * es, const int32_t * se, const int32_t * ss, int * s_first, int * s_tm,
                             int * s_gid) {
    const int lane = threadIdx.x & 63;
    const int T = p.T, E = p.n_expert, K = p.top_k, P = T * K;
    const bool live = lane < P;
    const int ex = live ? s_ids[lane] : -1;
    auto tier_of = [&](int e, int * idx) {
        int tier = 2;
        *idx = 0;
        if (e >= 0 && e < E) {
            tier = 1;
            *idx = e;
            if (p.k_slots > 0) {
                const int s = es[e];
                if (s >= 0 && s < p.k_slots && ss[s] == 2 && se[s] == e) {
                    tier = 0;
                    *idx = s;
                }
            }
        }
        return tier;
    };
    if (T == 1 && p.top_k <= E) {
        // one token: its top_k experts are distinct, so pair k is group k
        if (live) {
            int idx;
            groups[lane].tier = tier_of(ex, &idx);
            groups[lane].idx = idx;
            groups[lane].n_mem = 1;
            groups[lane].ord = lane;
            groups[lane].mem[0] = lane;
        }
        if (lane == 0) *n_groups = P;
        return;
    }
    const bool valid = live && ex >= 0 && ex < E;
    const int t = live ? lane / K : 0;
    if (valid) {
        atomicMin(s_first + ex, lane);
        atomicOr(s_tm + ex, 1 << t);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int leader = valid ? s_first[ex] : lane;
    const int tm = valid ? s_tm[ex] : (1 << t);
    const bool is_leader = live && leader == lane;
    const uint64_t lm = __ballot(is_leader);
    const int gid_lead = __popcll(lm & lanes_below());
    // the groups in order of first appearance; .ord lists them in order of
    // their dot passes, cheapest first (invalid ids: none; a hot expert's
    // Q4_K dots take about half an IQ2_S expert's; a pass per two members),
    // ties in order of first appearance
    int idx = 0, tier = 2, key = 0;
    const int nm = min(__popc(tm), min(T, DEC_MAXT));
    if (is_leader) {
        tier = tier_of(ex, &idx);
        key = tier == 2 ? 0 : (tier == 1 ? 2 : 1) * ((nm + 1) / 2);
    }
    int rank = 0;
    for (int k = 0; k <= 2 * ((DEC_MAXT + 1) / 2); ++k) {
        const uint64_t b = __ballot(is_leader && key == k);
        rank += k < key ? __popcll(b) : (k == key ? __popcll(b & lanes_below()) : 0);
    }
    if (is_leader) {
        groups[gid_lead].tier = tier;
        groups[gid_lead].idx = idx;
        groups[gid_lead].n_mem = nm;
        groups[rank].ord = gid_lead;
        if (valid) s_gid[ex] = gid_lead;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int gid = valid ? s_gid[ex] : gid_lead;
    const int slot = __popc(tm & ((1 << t) - 1));          // tokens before t that chose the expert
    if (live && slot < DEC_MAXT) groups[gid].mem[slot] = lane;
    if (lane == 0) *n_groups = __popcll(lm);
}

// Routing counters of the call (one workgroup, as the island's partition
// kernel counts them, ffn_moe.cu:123-128): routed pairs per valid expert id,
// then the hot pairs and the other pairs.
__device__ void count_routes(const DecParams & p, const int * s_ids, const GroupInfo * groups, int ng) {
    if (!p.rc_counts) return;
    const int P = p.T * p.top_k;
    if ((int)threadIdx.x < P) {
        const int e = s_ids[threadIdx.x];
        if (e >= 0 && e < p.n_expert) atomicAdd(p.rc_counts + e, 1);
    }
    if (threadIdx.x == 0 && p.rc_hits) {
        int hot = 0;
        for (int i = 0; i < ng; ++i)
            if (groups[i].tier == 0) hot += groups[i].n_mem;
        atomicAdd(p.rc_hits, hot);
        atomicAdd(p.rc_hits + 1, P - hot);
    }
}

// The group record g, or an empty group when g is past the call's groups.
// Validated so that no field can send a load or store out of bounds: member
// count <= min(T, DEC_MAXT) and members < P, else the group is emptied; a
// tier other than 0/1 or an index outside its pool makes the group invalid
// (tier 2: its members contribute zeros).
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

// ------------------------------------------------------------- staging

template <int N>
struct Regs {
    u32x4 r[N];
};

// `rows` rows of one expert's slab from row r0: `nch` 16-byte chunks from
// `src` (row r0 at byte `off` of the first chunk).  Without weights to read
// (an invalid group, or past the workgroup's items) one chunk of a valid
// dummy address, so that its loads, like every other, are unconditional.
struct Span {
    const u32x4 * src;
    int nch, off, rb;
    int valid;                  // tier 0/1 with members
};

__device__ __forceinline__ Span make_span(const GroupInfo & gi, int r0, int rows, int d_in, int ht, int ct,
                                          const uint8_t * hot, uint64_t hs, const uint8_t * cold, uint64_t cs,
                                          const void * dummy) {
    Span s;
    s.valid = gi.tier < 2 && gi.n_mem > 0;
    const int wt = gi.tier == 0 ? ht : ct;
    s.rb = (d_in / blk_elems(wt)) * blk_bytes(wt);
    const uint64_t start = (uint64_t)r0 * s.rb;
    s.off = (int)(start & 15);
    if (s.valid) {
        s.src = reinterpret_cast<const u32x4 *>(group_slab(gi.tier, gi.idx, hot, hs, cold, cs)) + (start >> 4);
        s.nch = (int)(((start + (uint64_t)rows * s.rb + 15) >> 4) - (start >> 4));
    } else {
        s.src = reinterpret_cast<const u32x4 *>(dummy);
        s.nch = 1;
    }
    return s;
}

template <int N>
__device__ __forceinline__ void span_load(Regs<N> & s, const Span & sp) {
#pragma unroll
    for (int k = 0; k < N; ++k) s.r[k] = sp.src[min((int)threadIdx.x + k * WG, sp.nch - 1)];
}
// the span's chunks into LDS at `dst` (chunks past N per thread: loaded here)
template <int N>
__device__ __forceinline__ void span_store(const Regs<N> & s, const Span & sp, uint8_t * dst) {
#pragma unroll
    for (int k = 0; k < N; ++k) {
        const int i = threadIdx.x + k * WG;
        if (i < sp.nch) *reinterpret_cast<u32x4 *>(dst + 16 * i) = s.r[k];
    }
    for (int i = threadIdx.x + N * WG; i < sp.nch; i += WG) *reinterpret_cast<u32x4 *>(dst + 16 * i) = sp.src[i];
}

// ---------------------------------------------------------------- B

constexpr int TAB_CHUNKS = (int)(sizeof(Iq2sTables) / 16);

// A one-token gate_up workgroup: 16 waves take the 64 rows of an item (32
// gate, 32 up) at once, one row per 16 lanes, and the device holds one per
// CU.  With 2-4 tokens a workgroup is 8 waves and takes an item in two
// steps, its 32 gate rows and then its 32 up rows (one row per 16 lanes), so
// its LDS holds half an item and a CU holds two workgroups.  Either way wave
// w stages four rows in an LDS region of its own.
template <int MT> constexpr int gu_nw() { return MT == 1 ? 16 : 8; }
template <int MT> constexpr int gu_nt() { return 64 * gu_nw<MT>(); }
template <int MT> constexpr int gu_halves() { return MT == 1 ? 2 : 1; }   // halves staged at once
constexpr int GU_HR = DEC_GU_BLK;             // rows of each half (gate, up) of an item

// The dots of the staged row at `wb` (one row per 16 lanes) against the
// members' columns av[c], c < n_mem <= MT; the row sums are complete in lane
// 0 of the row.  A unit is decoded once for at most two members (3-4 member
// groups decode it twice: the registers of four columns would halve the
// waves a CU holds).
template <int WT, int AM, int MT>
__device__ __forceinline__ void item_dot(const uint8_t * sm, int wb, int n_mem, int d_in, bool live,
                                         const ActView * av, float * acc, int grid_off) {
    constexpr int LPR = Fmt<WT>::LPR;
    const int lr = threadIdx.x % LPR;
#pragma unroll
    for (int c = 0; c < MT; ++c) acc[c] = 0.0f;
    if (live) {
        const int U = d_in / Fmt<WT>::UNIT;
        if (MT == 1 || n_mem == 1) {
#pragma unroll 1
            for (int u = lr; u < U; u += LPR) unit_dot_n<WT, AM, 1>(sm, wb, u, av, 1, acc, grid_off);
        } else {
#pragma unroll 1
            for (int u = lr; u < U; u += LPR) unit_dot_n<WT, AM, 2>(sm, wb, u, av, 2, acc, grid_off);
            if (MT > 2 && n_mem > 2) {
#pragma unroll 1
                for (int u = lr; u < U; u += LPR)
                    unit_dot_n<WT, AM, 2>(sm, wb, u, av + 2, n_mem - 2, acc + 2, grid_off);
            }
        }
    }
#pragma unroll
    for (int c = 0; c < MT; ++c)
#pragma unroll
        for (int o = LPR / 2; o >= 1; o >>= 1) acc[c] += __shfl_xor(acc[c], o, LPR);
}

// Wave w stages and dots four rows of an item: rows 4 (w mod 8) .. + 3 of the
// gate half (0) or the up half (1) -- one token: half w / 8, the 16 waves
// cover both; more: the step's half h -- in an LDS region of its own,
// w_lds_gu / 8 bytes at w w_lds_gu / 8.  The load unit copies the rows'
// chunks into it (global_load_lds, no registers), so a wave waits only for
// its own rows and needs no barrier before its dots, and it starts its rows
// of the next step as soon as its dots are done.
template <int MT>
__device__ __forceinline__ int gu_wave_half(int h) {
    return gu_halves<MT>() == 2 ? (int)(threadIdx.x >> 9) : h;
}
template <int HT, int CT, int MT>
__device__ __forceinline__ Span gu_wave_span(const DecParams & p, const GroupInfo & gi, int j, int h) {
    const int wave = threadIdx.x >> 6;
    return make_span(gi, gu_wave_half<MT>(h) * p.n_ff + DEC_GU_BLK * j + 4 * (wave & 7), 4, p.d_model, HT, CT,
                     p.hot_gu, p.hot_gu_stride, p.cold_gu, p.cold_gu_stride, p.logits);
}
template <int HT, int CT, int MT>
__device__ __forceinline__ void gu_wave_load(const DecParams & p, const GroupInfo & gi, int j, int h, uint8_t * smem) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const Span sp = gu_wave_span<HT, CT, MT>(p, gi, j, h);
    uint8_t * dst = smem + wave * (p.w_lds_gu / 8);
    for (int k = 0; 64 * k < sp.nch; ++k) {                // wave-uniform bound
        const int c = 64 * k + lane;
        if (c < sp.nch) lds_dma16(sp.src + c, dst + 1024 * k);
    }
}
// the four rows' dots against the members' columns: acc[c], complete in
// every lane of the row
template <int WT, int HT, int CT, int AM, int MT>
__device__ __forceinline__ void gu_wave_dots(const DecParams & p, const GroupInfo & gi, int j, int h,
                                             const uint8_t * smem, const ActView * av, int grid_off, float * acc) {
    const int wave = threadIdx.x >> 6, r = (threadIdx.x >> 4) & 3;
    const bool live = gi.tier < 2 && gi.n_mem > 0;
    const Span sp = gu_wave_span<HT, CT, MT>(p, gi, j, h);
    const int wb = wave * (p.w_lds_gu / 8) + sp.off + r * sp.rb;
    item_dot<WT, AM, MT>(smem, wb, gi.n_mem, p.d_model, live, av, acc, grid_off);
}

// the row of s_y the lane's row sums go to: 32 half + 4 (w mod 8) + row
template <int MT>
__device__ __forceinline__ int gu_y_row(int h) {
    return GU_HR * gu_wave_half<MT>(h) + 4 * ((threadIdx.x >> 6) & 7) + ((threadIdx.x >> 4) & 3);
}

// Each member's 32 GEGLU values (s_y: the gate rows at i -- one token: their
// GELU factors, geglu_factor --, the up rows at 32 + i) quantised (q8_0 / q8_1, block j of the
// pair's down activation) into the pair's down column: wave c takes member c
// (32 lanes).  One barrier: s_y is kept per item parity, so the next item's
// rows cannot overwrite what a slower wave still reads.
template <int AM, int MT, int GSRC>
__device__ __forceinline__ void gu_epilogue(const DecParams & p, const GroupInfo & gi, int j,
                                            const float (*s_y)[MT]) {
    const int T = p.T, K = p.top_k, F = p.n_ff;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (gi.tier < 2 && wave < gi.n_mem) {
        ActView L;
        act_layout(F, 0, &L);
        const int pair = max(0, min(member(gi, wave), T * K - 1));
        const int i = lane & 31;
        const float f = MT == 1 ? s_y[i][wave] : geglu_factor<GSRC>(s_y[i][wave]);
        const float v = lane < DEC_GU_BLK ? geglu_apply<GSRC>(f, s_y[GU_HR + i][wave]) : 0.0f;
        q8_32_put<AM>(p.yq + (int64_t)pair * p.yq_stride, L, v, DEC_GU_BLK * j + i, lane < DEC_GU_BLK);
    }
}

// the routing's LDS scratch in a gate_up workgroup (at the start of the
// weight staging area, which the host sizes to hold it: dec_gu_half_bytes)
struct GuScratch {
    int32_t res[3][256];
    int first[256], tm[256];
    SelScratch sel[DEC_MAXT];
};

// B: the routing, selected by every workgroup from the logits (wave t
// selects token t), grouped by expert, each group's tier by the residency
// predicate; the first workgroup publishes ids, weights and groups.  Then the
// workgroup's items: item i is group i / (n_ff / 32) and block j = i mod
// (n_ff / 32) of its down activation (32 gate rows and the 32 up rows paired
// with them); workgroup b takes items b, b + gridDim.x, ... (the grid is at
// most what the device holds resident, so every workgroup runs at once).
// MT: members a group can have (1 or DEC_MAXT).
template <int HT, int CT, int AM, int MT, int GSRC>
__global__ __launch_bounds__(gu_nt<MT>()) __attribute__((amdgpu_waves_per_eu(4)))
void k_dec_gate_up(const DecParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int GU_NT = gu_nt<MT>();
    static_assert(Fmt<HT>::LPR == 16 && Fmt<CT>::LPR == 16 && k256<HT>() && k256<CT>(), "gate_up formats");
    static_assert(gu_nw<MT>() >= DEC_MAXT && GU_NT >= 256, "a wave per token and a thread per expert");
    static_assert(GU_NT / 16 == gu_halves<MT>() * GU_HR, "one row per 16 lanes of the staged halves");
    constexpr bool IQ2 = HT == T_IQ2_S || CT == T_IQ2_S;
    constexpr int COLL = MT == 1 ? 1 : 2;                 // quantised column chunks per thread issued at once
    constexpr int TABL = (TAB_CHUNKS + GU_NT - 1) / GU_NT;   // codebook chunks per thread
    // the routing's scratch lives where the weights are staged later (the
    // first item starts with a barrier, after every read of it)
    GuScratch & sr = *reinterpret_cast<GuScratch *>(smem);
    __shared__ int s_ids[DEC_PMAX];           // the routing, kept past the scratch's reuse
    __shared__ float s_w[DEC_PMAX];
    int32_t (*s_res)[256] = sr.res;           // exp_slot, slot_exp, slot_state
    int * s_first = sr.first;                 // also each expert's group id, once its first pair is known
    int * s_tm = sr.tm;
    SelScratch * s_sel = sr.sel;
    __shared__ GroupInfo s_grp[DEC_PMAX];     // kept for every item of the workgroup
    __shared__ int s_ng;
    __shared__ float s_y[2][2 * GU_HR][MT];   // by item parity (the epilogue has one barrier)
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int T = p.T, K = p.top_k, E = p.n_expert, d_in = p.d_model, F = p.n_ff;

    // 1. the routing's loads, none under a lane condition: the logits of this
    //    wave's token (waves below T), the residency mirrors
    float lg[4];
    if (wave < T) {
        const float * lt = p.logits + (int64_t)wave * E;
#pragma unroll
        for (int j = 0; j < 4; ++j) lg[j] = lt[min(lane + 64 * j, E - 1)];
    }
    int32_t res[3] = {0, 0, 0};
    if (threadIdx.x < 256) {
        // without hot slots the mirrors may be absent: read a valid dummy
        const int ks = p.k_slots;
        const int32_t * dummy = reinterpret_cast<const int32_t *>(p.logits);
        const int32_t * es = ks > 0 ? p.exp_slot : dummy;
        const int32_t * se = ks > 0 ? p.slot_exp : dummy;
        const int32_t * ss = ks > 0 ? p.slot_state : dummy;
        const int is = ks > 0 ? min((int)threadIdx.x, ks - 1) : 0;
        res[0] = es[min((int)threadIdx.x, E - 1)];
        res[1] = se[is];
        res[2] = ss[is];
        s_first[threadIdx.x] = 64;
        s_tm[threadIdx.x] = 0;
    }

    // 2. the routing: wave t < T selects token t; then the expert groups
    if (wave < T) {
        asm volatile("" ::"v"(lg[2]), "v"(lg[3]));
        if (E <= 128) select_topk<2>(lg, E, K, s_ids + wave * K, s_w + wave * K, true, s_sel[wave]);
        else select_topk<4>(lg, E, K, s_ids + wave * K, s_w + wave * K, true, s_sel[wave]);
    }
    if (threadIdx.x < 256) {
#pragma unroll
        for (int i = 0; i < 3; ++i) s_res[i][threadIdx.x] = res[i];
    }
    __syncthreads();
    if (wave == 0) build_groups(p, s_ids, s_grp, &s_ng, s_res[0], s_res[1], s_res[2], s_first, s_tm, s_first);
    __syncthreads();
    const int ng = max(0, min(s_ng, DEC_PMAX));
    const int NBLK = F / DEC_GU_BLK, n_items = ng * NBLK;
    if ((int)blockIdx.x >= n_items) return;   // workgroup-uniform (workgroup 0 always has item 0)
    // workgroup b takes the items at positions b, b + grid, ...; with more
    // items than workgroups, positions past the grid (second items) take the
    // cheapest items and the first workgroups (the ones with a second item)
    // the next cheapest (the groups taken in .ord order, cheapest first)
    const int G = (int)gridDim.x, shift = max(0, n_items - G);
    auto item = [&](int pos, int * jo) {
        const int it = pos >= G ? pos - G : pos + shift;
        const int k = it / NBLK;
        const int g = max(0, min(s_grp[k].ord, ng - 1));
        *jo = it - k * NBLK;
        return validate_group(p, s_grp[g], ng, g);
    };

    // 3. every token's quantised column (contiguous: xq_stride == their
    //    size), the IQ2_S codebook and the first item's weights, in that
    //    order; the columns and the codebook then land in LDS (after the two
    //    halves: at a0), waiting for their own loads only
    ActView tmp;
    const int abytes = act_layout(d_in, 0, &tmp), a16 = abytes / 16;
    const int ncol = min(T, MT) * a16;
    const u32x4 * xq4 = reinterpret_cast<const u32x4 *>(p.xq);
    u32x4 col[COLL];
#pragma unroll
    for (int k = 0; k < COLL; ++k) col[k] = xq4[min((int)threadIdx.x + k * GU_NT, ncol - 1)];
    u32x4 tab[TABL];
    if (IQ2) {
#pragma unroll
        for (int k = 0; k < TABL; ++k)
            tab[k] = reinterpret_cast<const u32x4 *>(&c_iq2s_tab_dec)[min((int)threadIdx.x + k * GU_NT, TAB_CHUNKS - 1)];
    }
    int it = blockIdx.x, j, h = 0;
    GroupInfo gi = item(it, &j);
    // the first step's rows (the routing's scratch is dead: the barrier above)
    gu_wave_load<HT, CT, MT>(p, gi, j, 0, smem);
    const int a0 = gu_halves<MT>() * p.w_lds_gu;
#pragma unroll
    for (int k = 0; k < COLL; ++k) {
        const int i = threadIdx.x + k * GU_NT;
        if (i < ncol) reinterpret_cast<u32x4 *>(smem + a0)[i] = col[k];
    }
    for (int i = threadIdx.x + COLL * GU_NT; i < ncol; i += GU_NT) reinterpret_cast<u32x4 *>(smem + a0)[i] = xq4[i];
    const int grid_off = align16i(a0 + min(T, DEC_MAXT) * abytes);
    if (IQ2) {
#pragma unroll
        for (int k = 0; k < TABL; ++k) {
            const int i = threadIdx.x + k * GU_NT;
            if (i < TAB_CHUNKS) reinterpret_cast<u32x4 *>(smem + grid_off)[i] = tab[k];
        }
    }

    // 4. the first workgroup publishes the routing
    if (blockIdx.x == 0) {
        if ((int)threadIdx.x < T * K) {
            p.ids[threadIdx.x] = s_ids[threadIdx.x];
            p.w[threadIdx.x] = s_w[threadIdx.x];
        }
        for (int i = threadIdx.x; i < ng; i += GU_NT) p.ctl->groups[i] = s_grp[i];
        if (threadIdx.x == 0) p.ctl->n_groups = ng;
        count_routes(p, s_ids, s_grp, ng);
    }

    // 5. the steps: (item, half) -- one token: both halves in one step.  A
    //    wave dots its rows once they have landed, starts its rows of the
    //    next step, and after an item's up rows the workgroup's epilogue runs
    //    (its barrier orders s_y between the waves)
    __syncthreads();                                      // the columns and the codebook
    int par = 0;
    while (true) {
        ActView av[MT];
#pragma unroll
        for (int c = 0; c < MT; ++c) act_layout(d_in, a0 + max(0, min(member(gi, c) / K, T - 1)) * abytes, &av[c]);
        __builtin_amdgcn_s_waitcnt(0);                    // this wave's rows have landed
        float acc[MT];
        if (gi.tier == 0) gu_wave_dots<HT, HT, CT, AM, MT>(p, gi, j, h, smem, av, grid_off, acc);
        else gu_wave_dots<CT, HT, CT, AM, MT>(p, gi, j, h, smem, av, grid_off, acc);
        // one token: a gate row's sum becomes its GELU factor at once (the
        // table read is in flight while the up waves finish); 2-4 tokens:
        // the sums, the epilogue takes the factors
        if ((threadIdx.x & 15) == 0) {
            if (MT == 1 && gu_wave_half<MT>(h) == 0) {
                s_y[par][gu_y_row<MT>(h)][0] = geglu_factor<GSRC>(acc[0]);
            } else {
#pragma unroll
                for (int c = 0; c < MT; ++c) s_y[par][gu_y_row<MT>(h)][c] = acc[c];
            }
        }
        const bool last = h + gu_halves<MT>() >= 2;       // the item's up rows are done
        int nit = it, nj = j, nh = h + gu_halves<MT>();
        GroupInfo nx = gi;
        if (last) {
            nit = it + (int)gridDim.x;
            nh = 0;
            if (nit < n_items) nx = item(nit, &nj);
        }
        if (nit < n_items) gu_wave_load<HT, CT, MT>(p, nx, nj, nh, smem);   // in flight meanwhile
        if (last) {
            gu_epilogue<AM, MT, GSRC>(p, gi, j, s_y[par]);
            par ^= 1;
        }
        if (nit >= n_items) break;
        it = nit;
        j = nj;
        h = nh;
        gi = nx;
    }
}

// ---------------------------------------------------------------- C

constexpr int DN_LPR = 16;      // lanes per row: lane l holds the row's block pair l (blocks 2 l, 2 l + 1)
constexpr int DN_RPP = WG / DN_LPR;   // rows per pass
constexpr int DN_CL = 8;        // 16-byte chunks of the pairs' down columns per thread loaded first
constexpr int DN_GRP_NPS = 2;   // passes of a down-by-group workgroup (dn_grp_rpp rows each), all in flight
// down by group: a row's NP = n_ff / 64 block pairs take NP consecutive
// lanes, so a pass covers WG / NP rows (23 at n_ff 704, where 16 lanes a row
// would leave 5 of them idle)
__host__ __device__ inline int dn_grp_rpp(int n_ff) { return WG / (n_ff / 64); }
typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(4)));

// per-group state of the down kernel, in LDS.  The slab is kept as a byte
// offset into its pool, not as a pointer: a pointer read back from LDS is
// generic, and loads through it would be flat loads, which also count on the
// LDS counter (every LDS wait would then wait for them).
struct DnGroup {
    int tier, n_mem, pad0, pad1;
    int mem[DEC_MAXT];
    float scale;
    int rb;                     // bytes per row
    uint64_t row0;              // byte offset of this block's first row in the pool (tier 0 hot, else cold)
};

// one block pair of a down row (Q5_0: 44 bytes, IQ4_NL: 36), loaded as dwords
// from a 4-aligned address
struct DnPair {
    uint32_t w[11];
};

template <int T>
__device__ __forceinline__ void dn_pair_load(DnPair & q, const uint8_t * src) {
    const u32x4a * s4 = reinterpret_cast<const u32x4a *>(src);
    const u32x4a a = s4[0], b = s4[1];
    q.w[0] = a.x; q.w[1] = a.y; q.w[2] = a.z; q.w[3] = a.w;
    q.w[4] = b.x; q.w[5] = b.y; q.w[6] = b.z; q.w[7] = b.w;
    const uint32_t * s1 = reinterpret_cast<const uint32_t *>(src + 32);
    if constexpr (T == T_Q5_0) {
        q.w[8] = s1[0]; q.w[9] = s1[1]; q.w[10] = s1[2];
    } else {
        q.w[8] = s1[0]; q.w[9] = 0u; q.w[10] = 0u;
    }
}

// the member activation's 32-block b from LDS: 32 int8 values, its scale
// and its sum (q8_1: of the values, stored as fp16; q8_0: of the int8
// values, exact)
struct Act32 {
    u32x4 lo, hi;
    float d, s;
};
template <int AM>
__device__ __forceinline__ Act32 act32(const uint8_t * smem, const ActView & av, int b) {
    Act32 a;
    const int ao = av.q + qpos(32 * b);
    a.lo = lds128(smem, ao);
    a.hi = lds128(smem, ao + 16);
    a.d = reinterpret_cast<const float *>(smem + av.d32)[b];
    a.s = reinterpret_cast<const float *>(smem + av.s32)[b];
    return a;
}

// A block of a down row's pair, decoded once for every member's column: its
// 32 weights as int8 (v[2 i]: values 4 i .. 4 i + 3, v[2 i + 1]: 16 + 4 i ..;
// Q5_0: q in 0 .. 31, IQ4_NL: the table values) and its scale
struct DnBlk {
    uint32_t v[8];
    float d;
};
// bit j of the nibble n4 / 16 (n4 = nibble << 4) at bit 4 of byte j
__device__ __forceinline__ uint32_t q5_hi4(uint32_t n4) { return __umul24(n4, 0x204081u) & 0x10101010u; }
template <int T>
__device__ __forceinline__ DnBlk dn_block(const DnPair & q, int h) {
    DnBlk b;
    uint32_t d16, qs[4];
    if (T == T_Q5_0) {
        uint32_t qh;
        if (h == 0) {
            d16 = q.w[0] & 0xFFFF;
            qh = __builtin_amdgcn_alignbit(q.w[1], q.w[0], 16);
#pragma unroll
            for (int i = 0; i < 4; ++i) qs[i] = __builtin_amdgcn_alignbit(q.w[2 + i], q.w[1 + i], 16);
        } else {
            d16 = q.w[5] >> 16;
            qh = q.w[6];
#pragma unroll
            for (int i = 0; i < 4; ++i) qs[i] = q.w[7 + i];
        }
        // the fifth bits: value 4 i + j from qh bit 4 i + j, value 16 + 4 i + j from bit 16 + 4 i + j
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo4 = (i == 0 ? qh << 4 : qh >> (4 * i - 4)) & 0xF0u;
            const uint32_t hi4 = (qh >> (12 + 4 * i)) & 0xF0u;
            b.v[2 * i] = (qs[i] & 0x0F0F0F0Fu) | q5_hi4(lo4);
            b.v[2 * i + 1] = ((qs[i] >> 4) & 0x0F0F0F0Fu) | q5_hi4(hi4);
        }
    } else {
        if (h == 0) {
            d16 = q.w[0] & 0xFFFF;
#pragma unroll
            for (int i = 0; i < 4; ++i) qs[i] = __builtin_amdgcn_alignbit(q.w[1 + i], q.w[i], 16);
        } else {
            d16 = q.w[4] >> 16;
#pragma unroll
            for (int i = 0; i < 4; ++i) qs[i] = q.w[5 + i];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            b.v[2 * i] = iq4nl_lookup(qs[i] & 0x0F0F0F0Fu);
            b.v[2 * i + 1] = iq4nl_lookup((qs[i] >> 4) & 0x0F0F0F0Fu);
        }
    }
    b.d = h2f(d16);
    return b;
}

// Q5_0 . q8_0 (ggml-cpu/quants.c:314-352):  d_w d8 sum (q - 16) a
// Q5_0 . q8_1 (ggml-cuda/vecdotq.cuh:172-198): d_w (d8 sum q a - 16 s8)
// IQ4_NL . q8_0 (ggml-cpu/quants.c:1203-1228) and . q8_1 (vecdotq.cuh:1270-1289):
//   d_w d8 sum kvalues[q] a
template <int AM, int T>
__device__ __forceinline__ float dn_dot(const DnBlk & b, const Act32 & a) {
    const uint32_t al[4] = {a.lo.x, a.lo.y, a.lo.z, a.lo.w}, ah[4] = {a.hi.x, a.hi.y, a.hi.z, a.hi.w};
    int sumi = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        sumi = dot4((int)b.v[2 * i], (int)al[i], sumi);
        sumi = dot4((int)b.v[2 * i + 1], (int)ah[i], sumi);
    }
    if (T == T_Q5_0) {
        if (AM == AM_CPU) return __fmul_rn(b.d * a.d, (float)(sumi - 16 * (int)a.s));
        return b.d * ((float)sumi * a.d - 16.0f * a.s);
    }
    if (AM == AM_CPU) return __fmul_rn(a.d * b.d, (float)sumi);
    return (b.d * a.d) * (float)sumi;
}

// max over each group of 8 lanes (lanes 8 m .. 8 m + 7), in every lane of it
__device__ __forceinline__ float oct_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v, v));        // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_f<0x4E>(v, v));        // quad_perm [2,3,0,1]
    v = fmaxf(v, __shfl_xor(v, 4, 8));
    return v;
}

// q8 of one 32-block held as 4 values per lane by 8 consecutive lanes, into
// a column at `col` (layout L): q8_0 as the x86 CPU build computes it
// (arch/x86/quants.c:302-360: d = amax / 127 stored as fp16, q =
// round-to-nearest-even(x 127 / amax)) or q8_1 (ggml-cuda quantize.cu:5-50:
// q = roundf(x / d), and the block sum, stored as fp16).  `c4` is the index
// of the lane's 4 values in the column.
template <int AM>
__device__ __forceinline__ void q8_quad(uint8_t * col, const ActView & L, const float (&v)[4], int c4, bool live) {
    float m = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    const float amax = oct_max(m);
    int q[4];
    float dstore, sstore = 0.0f;
    if (AM == AM_CPU) {
        const float id = amax != 0.0f ? 127.f / amax : 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int r = (int)rintf(__fmul_rn(v[j], id));
            q[j] = r > 127 ? 127 : (r < -128 ? -128 : r);
        }
        dstore = round_to_half(amax / 127.f);
        int qs = q[0] + q[1] + q[2] + q[3];                 // the block's sum of q (exact)
        qs += __builtin_amdgcn_update_dpp(0, qs, 0xB1, 0xF, 0xF, false);
        qs += __builtin_amdgcn_update_dpp(0, qs, 0x4E, 0xF, 0xF, false);
        qs += __shfl_xor(qs, 4, 8);
        sstore = (float)qs;
    } else {
        const float d = amax / 127.0f;
        float s = __fadd_rn(__fadd_rn(v[0], v[1]), __fadd_rn(v[2], v[3]));
        s = __fadd_rn(s, dpp_f<0xB1>(0.0f, s));
        s = __fadd_rn(s, dpp_f<0x4E>(0.0f, s));
        s = __fadd_rn(s, __shfl_xor(s, 4, 8));
#pragma unroll
        for (int j = 0; j < 4; ++j) q[j] = amax == 0.0f ? 0 : (int)roundf(v[j] / d);
        dstore = round_to_half(d);
        sstore = round_to_half(s);
    }
    if (live) {
        const uint32_t w = (uint32_t)(q[0] & 0xFF) | ((uint32_t)(q[1] & 0xFF) << 8) | ((uint32_t)(q[2] & 0xFF) << 16) |
                           ((uint32_t)(q[3] & 0xFF) << 24);
        *reinterpret_cast<uint32_t *>(col + L.q + qpos(4 * c4)) = w;
        if ((c4 & 7) == 0) {
            reinterpret_cast<float *>(col + L.d32)[c4 >> 3] = dstore;
            reinterpret_cast<float *>(col + L.s32)[c4 >> 3] = sstore;
        }
    }
}

// C: output rows [r0, r0 + R) of every token, r0 = blockIdx.x R, R =
// 2^dn_rows_log2.  First, with no dependence on anything, the loads of the
// pairs' quantised down columns (written by B; the pairs are 0 .. T top_k - 1
// whatever the grouping) and of the groups' records and routing weights
// (from B's first workgroup); then a table of the groups (tier, members,
// .scale, where this block's rows start in the pool).  The weights never
// pass through LDS: each row's lanes load its block pairs straight into
// registers (lane l: blocks 2 l, 2 l + 1, dword-aligned), the next pass's
// rows in flight while the current ones are dotted against the members'
// columns in LDS.  Each row is scaled by the expert's .scale into
// s_y[pair][row]; then each (token, row) output is the sum of w_k y_k in k
// order.  Invalid groups leave their pairs at zero.
template <int HD, int CD, int AM, int MT>
__global__ __launch_bounds__(WG) __attribute__((amdgpu_waves_per_eu(1, 4))) void k_dec_down(const DecParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    static_assert(!k256<HD>() && !k256<CD>(), "down formats");
    __shared__ DnGroup s_gi[DEC_PMAX];
    __shared__ float s_wt[DEC_PMAX];
    __shared__ float s_y[DEC_PMAX][DEC_DN_MAXR];
    __shared__ int s_ng;
    const int D = p.d_model, F = p.n_ff, K = p.top_k, T = p.T, P = T * K;
    const int lg2r = p.dn_rows_log2, R = 1 << lg2r, r0 = blockIdx.x << lg2r, nr = max(0, min(R, D - r0));
    const int abytes = (int)p.yq_stride;                      // one quantised column, a multiple of 16
    const int NP = F / 64;                                    // block pairs per row

    // 1. the columns' first loads, then the records
    const u32x4 * yq4 = reinterpret_cast<const u32x4 *>(p.yq);
    const int nch = P * (abytes / 16);
    u32x4 col[DN_CL];
#pragma unroll
    for (int k = 0; k < DN_CL; ++k) col[k] = yq4[min((int)threadIdx.x + k * WG, nch - 1)];
    {
        const GroupInfo gi_in = p.ctl->groups[min((int)threadIdx.x, DEC_PMAX - 1)];
        const int ngv = p.ctl->n_groups;
        const float wv = p.w[min((int)threadIdx.x, P - 1)];
        if (threadIdx.x == 0) s_ng = ngv;
        if ((int)threadIdx.x < DEC_PMAX) s_wt[threadIdx.x] = (int)threadIdx.x < P ? wv : 0.0f;
        for (int i = threadIdx.x; i < P * DEC_DN_MAXR; i += WG) (&s_y[0][0])[i] = 0.0f;
        __syncthreads();
        const int ng = max(0, min(s_ng, DEC_PMAX));
        if ((int)threadIdx.x < ng) {
            const GroupInfo gi = validate_group(p, gi_in, ng, threadIdx.x);
            DnGroup d;
            d.tier = gi.tier;
            d.n_mem = gi.tier < 2 ? gi.n_mem : 0;
            d.pad0 = d.pad1 = 0;
#pragma unroll
            for (int c = 0; c < DEC_MAXT; ++c) d.mem[c] = gi.mem[c];
            d.scale = gi.tier == 0 ? (p.s_hot ? p.s_hot[gi.idx] : 1.0f)
                                   : (gi.tier == 1 ? (p.s_cold ? p.s_cold[gi.idx] : 1.0f) : 0.0f);
            const int wt = gi.tier == 0 ? HD : CD;
            d.rb = (F / 32) * blk_bytes(wt);
            d.row0 = d.n_mem > 0 ? (gi.tier == 0 ? (uint64_t)gi.idx * p.hot_dn_stride : (uint64_t)gi.idx * p.cold_dn_stride) +
                                       (uint64_t)r0 * d.rb
                                 : 0;
            s_gi[threadIdx.x] = d;
        }
    }
    __syncthreads();
    const int ng = max(0, min(s_ng, DEC_PMAX));
    const int rows = ng << lg2r, passes = (rows + DN_RPP - 1) / DN_RPP;
    const int lrow = threadIdx.x / DN_LPR, lane16 = threadIdx.x % DN_LPR;
    const int pl = min(lane16, NP - 1);

    // the block pair of this lane in pass `ps` (a clamped, valid address when
    // the lane has none)
    auto pair_src = [&](int ps, int * kind) {
        const int k = ps * DN_RPP + lrow, s = min(k >> lg2r, max(ng - 1, 0)), r = min(k & (R - 1), max(nr - 1, 0));
        const DnGroup & d = s_gi[s];
        *kind = d.tier == 0 ? 0 : 1;
        const uint8_t * base = d.tier == 0 ? p.hot_dn : p.cold_dn;
        return base + d.row0 + (uint64_t)r * d.rb + (uint64_t)pl * (blk_bytes(d.tier == 0 ? HD : CD) * 2);
    };
    auto load = [&](DnPair & q, int ps, int * kind) {
        const uint8_t * src = pair_src(ps, kind);
        if (*kind == 0) dn_pair_load<HD>(q, src);
        else dn_pair_load<CD>(q, src);
    };
    // every pass's block pairs in flight at once (up to DA passes; later ones
    // are loaded when they come)
    constexpr int DA = MT == 1 ? 2 : 8;
    DnPair w[DA];
    int kw[DA];
#pragma unroll
    for (int q = 0; q < DA; ++q) {
        kw[q] = 0;
        if (q < passes) load(w[q], q, &kw[q]);
    }

    // 2. the columns into LDS
#pragma unroll
    for (int k = 0; k < DN_CL; ++k) {
        const int i = threadIdx.x + k * WG;
        if (i < nch) reinterpret_cast<u32x4 *>(smem)[i] = col[k];
    }
    for (int i = threadIdx.x + DN_CL * WG; i < nch; i += WG) reinterpret_cast<u32x4 *>(smem)[i] = yq4[i];
    __syncthreads();

    // 3. the passes: DN_RPP rows each, one row per DN_LPR lanes
    auto pass = [&](const DnPair & cur, int kc, int ps) {
        const int k = ps * DN_RPP + lrow, s = min(k >> lg2r, ng - 1), r = k & (R - 1);
        const DnGroup & d = s_gi[s];
        const bool live = k < rows && r < nr && d.n_mem > 0 && lane16 < NP;
        float acc[MT];
#pragma unroll
        for (int c = 0; c < MT; ++c) acc[c] = 0.0f;
        if (live) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const DnBlk bk = kc == 0 ? dn_block<HD>(cur, h) : dn_block<CD>(cur, h);
#pragma unroll
                for (int c = 0; c < MT; ++c) {
                    if (c >= d.n_mem) break;
                    ActView av;
                    act_layout(F, max(0, min(d.mem[c], P - 1)) * abytes, &av);
                    const Act32 a = act32<AM>(smem, av, 2 * lane16 + h);
                    acc[c] += kc == 0 ? dn_dot<AM, HD>(bk, a) : dn_dot<AM, CD>(bk, a);
                }
            }
        }
#pragma unroll
        for (int c = 0; c < MT; ++c)
#pragma unroll
            for (int o = DN_LPR / 2; o >= 1; o >>= 1) acc[c] += __shfl_xor(acc[c], o, DN_LPR);
        if (live && lane16 == 0) {
#pragma unroll
            for (int c = 0; c < MT; ++c)
                if (c < d.n_mem) s_y[d.mem[c]][r] = acc[c] * d.scale;
        }
    };
#pragma unroll
    for (int q = 0; q < DA; ++q)
        if (q < passes) pass(w[q], kw[q], q);
    for (int ps = DA; ps < passes; ++ps) {
        DnPair t;
        int kt = 0;
        load(t, ps, &kt);
        pass(t, kt, ps);
    }
    __syncthreads();

    // 4. the combine (llama-graph.cpp:1812-1840): out = sum_k w_k y_k in k order,
    // every product and sum rounded on its own (ggml_mul, then ggml_add)
    for (int i = threadIdx.x; i < (T << lg2r); i += WG) {
#pragma clang fp contract(off)
        const int t = i >> lg2r, r = i & (R - 1);
        if (r >= nr) continue;
        float o = s_y[t * K][r] * s_wt[t * K];
        for (int k = 1; k < K; ++k) o = o + s_y[t * K + k][r] * s_wt[t * K + k];
        p.out[(int64_t)t * D + r0 + r] = o;
    }
}

// C by group (more than one token): workgroup (b, g) computes output rows
// [b R, b R + R) of group g's expert for the group's members only (R = NPS
// passes of dn_grp_rpp rows, all of them in flight at once: lane l of a
// row's NP holds its block pair l), writing the scaled rows y_pair = .scale
// W a_pair to ydn;
// workgroups of groups past the call's count return at once.  Only the
// members' quantised columns are read (one to four, where the kernel over
// every group copies all T top_k of them into every workgroup).
// k_dec_combine then sums each token's top_k rows.
template <int HD, int CD, int AM, int MT, int NPS>
__global__ __launch_bounds__(WG) void k_dec_down_grp(const DecParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    static_assert(!k256<HD>() && !k256<CD>(), "down formats");
    __shared__ float s_red[NPS][WG][MT];      // the lanes' partial row sums
    const int D = p.d_model, F = p.n_ff, K = p.top_k, T = p.T, P = T * K;
    const int RPP = dn_grp_rpp(F), R = NPS * RPP;
    const int b = blockIdx.x, r0 = b * R, nr = max(0, min(R, D - r0));
    const int g = blockIdx.y;
    const int ng = max(0, min(p.ctl->n_groups, P));
    if (g >= ng) return;
    const GroupInfo gi = validate_group(p, p.ctl->groups[g], ng, g);
    const int nm = gi.tier < 2 ? gi.n_mem : 0;
    const int NP = F / 64;
    const int abytes = (int)p.yq_stride, a16 = abytes / 16;

    // 1. the members' columns, then every row's block pairs
    const u32x4 * yq4 = reinterpret_cast<const u32x4 *>(p.yq);
    u32x4 col[MT];                                          // one chunk of each column per thread (n_ff <= 1024)
#pragma unroll
    for (int c = 0; c < MT; ++c) {
        const int pr = max(0, min(c < nm ? gi.mem[c] : gi.mem[0], P - 1));
        col[c] = yq4[(int64_t)pr * a16 + min((int)threadIdx.x, a16 - 1)];
    }
    // lane: row lrow of each pass, block pair pl (lanes past RPP rows idle)
    const int lrow = threadIdx.x / NP, pl = threadIdx.x - lrow * NP;
    const bool lane_live = lrow < RPP;
    const int wt = gi.tier == 0 ? HD : CD;
    const int rbytes = (F / 32) * blk_bytes(wt);
    const uint8_t * slab = gi.tier == 0 ? p.hot_dn + (uint64_t)gi.idx * p.hot_dn_stride
                                        : p.cold_dn + (uint64_t)gi.idx * p.cold_dn_stride;
    DnPair w[NPS];
#pragma unroll
    for (int ps = 0; ps < NPS; ++ps) {
        const int r = min(ps * RPP + min(lrow, RPP - 1), max(nr - 1, 0));
        const uint8_t * src = slab + (uint64_t)(r0 + r) * rbytes + (uint64_t)pl * (2 * blk_bytes(wt));
        if (gi.tier == 0) dn_pair_load<HD>(w[ps], src);
        else dn_pair_load<CD>(w[ps], src);
    }

    // 2. the members' columns into LDS
#pragma unroll
    for (int c = 0; c < MT; ++c) {
        if (c >= max(nm, 1)) break;
        if ((int)threadIdx.x < a16) reinterpret_cast<u32x4 *>(smem + c * abytes)[threadIdx.x] = col[c];
    }
    __syncthreads();

    // 3. the rows: each lane dots its block pair, the row's NP partial sums
    //    meet in LDS and one thread a row adds them in pair order, scales
    //    and stores
#pragma unroll
    for (int ps = 0; ps < NPS; ++ps) {
        float acc[MT];
#pragma unroll
        for (int c = 0; c < MT; ++c) acc[c] = 0.0f;
        if (lane_live) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const DnBlk bk = gi.tier == 0 ? dn_block<HD>(w[ps], h) : dn_block<CD>(w[ps], h);
#pragma unroll
                for (int c = 0; c < MT; ++c) {
                    if (c >= nm) break;
                    ActView av;
                    act_layout(F, c * abytes, &av);
                    const Act32 a = act32<AM>(smem, av, 2 * pl + h);
                    acc[c] += gi.tier == 0 ? dn_dot<AM, HD>(bk, a) : dn_dot<AM, CD>(bk, a);
                }
            }
        }
#pragma unroll
        for (int c = 0; c < MT; ++c) s_red[ps][threadIdx.x][c] = acc[c];
    }
    __syncthreads();
    const float scale = gi.tier == 0 ? (p.s_hot ? p.s_hot[gi.idx] : 1.0f)
                                     : (gi.tier == 1 ? (p.s_cold ? p.s_cold[gi.idx] : 1.0f) : 0.0f);
    // an invalid id's members get zero rows
    const int nw = gi.tier < 2 ? nm : max(0, min(gi.n_mem, MT));
    for (int i = threadIdx.x; i < NPS * RPP; i += WG) {
        const int ps = i / RPP, lr = i - ps * RPP, r = ps * RPP + lr;
        if (r >= nr) continue;
        float sum[MT];
#pragma unroll
        for (int c = 0; c < MT; ++c) sum[c] = 0.0f;
        for (int j = 0; j < NP; ++j)
#pragma unroll
            for (int c = 0; c < MT; ++c) sum[c] += s_red[ps][lr * NP + j][c];
#pragma unroll
        for (int c = 0; c < MT; ++c)
            if (c < nw) p.ydn[(int64_t)max(0, min(gi.mem[c], P - 1)) * D + r0 + r] = sum[c] * scale;
    }
}

// the combine after the down kernel by group (llama-graph.cpp:1812-1840):
// out[t][r] = sum_k w_k ydn[t K + k][r] in k order
__global__ __launch_bounds__(WG) void k_dec_combine(const DecParams p) {
    const int D = p.d_model, K = p.top_k;
    const int i = blockIdx.x * WG + threadIdx.x;
    if (i >= p.T * D) return;
    const int t = i / D, r = i - t * D;
    const float * y = p.ydn + (int64_t)t * K * D + r;
    const float * wk = p.w + t * K;
    // every load issued before the first use (K <= DEC_KMAX)
    float yv[DEC_KMAX], wv[DEC_KMAX];
#pragma unroll
    for (int k = 0; k < DEC_KMAX; ++k) {
        yv[k] = k < K ? y[(int64_t)k * D] : 0.0f;
        wv[k] = k < K ? wk[k] : 0.0f;
    }
    // every product and sum rounded on its own (ggml_mul, then ggml_add)
    float o;
    {
#pragma clang fp contract(off)
        o = yv[0] * wv[0];
#pragma unroll
        for (int k = 1; k < DEC_KMAX; ++k)
            if (k < K) o = o + yv[k] * wv[k];
    }
    p.out[i] = o;
}

// ------------------------------------------------------------ fires

// One fire of the dual op (the reference's moert_ffn_moe: partition, gather,
// hot and cold mul_mat_id, scatter; ffn_moe.cu:892-1246) as one kernel:
// workgroup (b, p) computes output rows of routed pair p (p = t n_used + j,
// expert ids[t ids_s1 + j]) from the hot slab when the residency predicate
// holds (ffn_moe.cu:80-130: exp_slot[e] = s, slot_state[s] READY,
// slot_exp[s] = e) and from the cold pool otherwise, into dst[p]; the down
// fire (kind 1) scales by the expert's .scale, as the island's scatter does.
// A pair with an invalid id gets zeros.  Every workgroup reads its pair's id
// and the whole residency mirrors in one round of loads (no chain of
// dependent loads), then its rows' weights.

struct FireRes {
    int tier, idx;              // 0 hot (slot), 1 cold (expert), 2 invalid id
};

// the pair's id and tier from the mirrors, staged through LDS (s_m: 3 x 256)
__device__ __forceinline__ FireRes fire_resolve(const FireParams & f, int p, int32_t (*s_m)[256], int * e_out) {
    const int t = p / f.n_used, j = p - t * f.n_used;
    const int e = f.ids[(int64_t)t * f.ids_s1 + j];
    const int ks = f.k_slots, E = f.n_expert;
    {
        const int32_t * dummy = f.ids;
        const int is = ks > 0 ? min((int)threadIdx.x, ks - 1) : 0;
        const int32_t a = ks > 0 ? f.exp_slot[min((int)threadIdx.x, E - 1)] : dummy[0];
        const int32_t b = ks > 0 ? f.slot_exp[is] : dummy[0];
        const int32_t c = ks > 0 ? f.slot_state[is] : dummy[0];
        s_m[0][threadIdx.x] = a;
        s_m[1][threadIdx.x] = b;
        s_m[2][threadIdx.x] = c;
    }
    __syncthreads();
    FireRes r = {2, 0};
    if (e >= 0 && e < E) {
        r.tier = 1;
        r.idx = e;
        if (ks > 0) {
            const int sl = s_m[0][e];
            if (sl >= 0 && sl < ks && s_m[2][sl] == 2 && s_m[1][sl] == e) {
                r.tier = 0;
                r.idx = sl;
            }
        }
    }
    *e_out = e;
    return r;
}

// the routing counters of a gate_up fire (k_partition's counts), once per pair
__device__ __forceinline__ void fire_count(const FireParams & f, int e, const FireRes & r) {
    if (f.rc_counts && blockIdx.x == 0 && threadIdx.x == 0) {
        if (e >= 0 && e < f.n_expert) atomicAdd(f.rc_counts + e, 1);
        if (f.rc_hits) atomicAdd(f.rc_hits + (r.tier == 0 ? 0 : 1), 1);
    }
}

constexpr int FIRE_GU_LOADS = 9;        // 16-byte weight chunks per thread in flight (23 Q4_K rows of 2816)
constexpr int FIRE_XV = 12;             // fp32 input values per lane (d_in <= 3072)

// q8_K of 256-block b held as v[j] = x[256 b + lane + 64 j] by one wave
// (ggml-quants.c:2696-2733, as q8K_block computes it from memory)
__device__ __forceinline__ void q8K_block_v(uint8_t * base, const ActView & L, const float (&v)[4], int b) {
    const int lane = threadIdx.x & 63;
    int8_t * q = reinterpret_cast<int8_t *>(base + L.q);
    float * dK = reinterpret_cast<float *>(base + L.dK);
    int * bsum = reinterpret_cast<int *>(base + L.bsum);
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) amax = fmaxf(amax, fabsf(v[j]));
    amax = wave_max_dpp(amax);
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
        q[b * 272 + lane + 64 * j] = (int8_t)qi[j];
        const int s = row16_sum(qi[j]);
        if ((lane & 15) == 0) bsum[b * 16 + (lane >> 4) + 4 * j] = s;
    }
}

// gate_up fire (Q4_K / IQ2_S weights, d_in a multiple of 256, <= 3072):
// 16 rows of one pair per workgroup, staged through LDS like the decode
// path's gate_up items; the token's column quantised here (q8_K, or q8_1 in
// the GPU activation mode).
template <int HT, int CT, int AM>
__global__ __launch_bounds__(WG) void k_fire_k256(const FireParams f) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr bool IQ2 = HT == T_IQ2_S || CT == T_IQ2_S;
    __shared__ int32_t s_m[3][256];
    const int p = blockIdx.y, d_in = f.d_in, NPL = fire_gu_lanes(d_in), RW = WG / NPL, r0 = blockIdx.x * RW;
    if (f.n_live && p >= *f.n_live) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = p / f.n_used;
    // 1. the column's values and the codebook (no dependence on the routing)
    const float * x = f.cur + (f.cur_shared ? 0 : (int64_t)t * d_in);
    float xv[FIRE_XV];
#pragma unroll
    for (int i = 0; i < FIRE_XV; ++i) {
        const int pos = AM == AM_CPU ? 256 * (wave + 4 * (i / 4)) + lane + 64 * (i % 4) : 64 * (wave + 4 * i) + lane;
        xv[i] = x[min(pos, d_in - 1)];
    }
    u32x4 tab[TAB_CHUNKS / WG];
    if (IQ2) {
#pragma unroll
        for (int k = 0; k < TAB_CHUNKS / WG; ++k)
            tab[k] = reinterpret_cast<const u32x4 *>(&c_iq2s_tab_dec)[threadIdx.x + k * WG];
    }
    // 2. the pair's tier, then its rows
    int e;
    const FireRes rs = fire_resolve(f, p, s_m, &e);
    if (f.kind == 0) fire_count(f, e, rs);
    GroupInfo gi = {};
    gi.tier = rs.tier;
    gi.idx = rs.idx;
    gi.n_mem = 1;
    const int nr = min(RW, f.d_out - r0);
    const Span sp = make_span(gi, r0, nr, d_in, HT, CT, f.hot, f.hot_stride, f.cold, f.cold_stride, f.ids);
    Regs<FIRE_GU_LOADS> st;
    span_load(st, sp);
    // 3. the column's q8 into LDS (after the rows), the codebook after it
    const int a0 = f.w_lds;
    ActView av[1], L0;                      // av: offsets from smem (the dots), L0: from the column
    const int abytes = act_layout(d_in, a0, &av[0]);
    act_layout(d_in, 0, &L0);
    if (AM == AM_CPU) {
#pragma unroll
        for (int k = 0; k < FIRE_XV / 4; ++k) {
            const int b = wave + 4 * k;
            if (b < d_in / 256) {
                const float v[4] = {xv[4 * k], xv[4 * k + 1], xv[4 * k + 2], xv[4 * k + 3]};
                q8K_block_v(smem + a0, L0, v, b);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < FIRE_XV; ++i) {
            const int pos = 64 * (wave + 4 * i) + lane;
            if (64 * (wave + 4 * i) < d_in) q8_32_put<AM_Q8_1>(smem + a0, L0, xv[i], pos, pos < d_in);
        }
    }
    const int grid_off = align16i(a0 + abytes);
    if (IQ2) {
#pragma unroll
        for (int k = 0; k < TAB_CHUNKS / WG; ++k)
            reinterpret_cast<u32x4 *>(smem + grid_off)[threadIdx.x + k * WG] = tab[k];
    }
    span_store(st, sp, smem);
    __syncthreads();
    // 4. NPL lanes a row, units lr, lr + NPL, ...; the row's partial sums
    //    meet in LDS and one thread a row adds them in lane order
    __shared__ float s_red[WG];
    const int row = threadIdx.x / NPL, lr = threadIdx.x - row * NPL;
    const bool live = sp.valid != 0 && row < nr;
    float acc = 0.0f;
    if (live) {
        const int U = d_in / 64, wb = sp.off + row * sp.rb;
        if (gi.tier == 0) {
            for (int u = lr; u < U; u += NPL) unit_dot_n<HT, AM, 1>(smem, wb, u, av, 1, &acc, grid_off);
        } else {
            for (int u = lr; u < U; u += NPL) unit_dot_n<CT, AM, 1>(smem, wb, u, av, 1, &acc, grid_off);
        }
    }
    s_red[threadIdx.x] = acc;
    __syncthreads();
    if ((int)threadIdx.x < nr) {
        float sum = 0.0f;
        for (int j = 0; j < NPL; ++j) sum += s_red[threadIdx.x * NPL + j];
        f.dst[(int64_t)p * f.d_out + r0 + threadIdx.x] = sp.valid != 0 ? sum : 0.0f;
    }
}

// down fire (Q5_0 / IQ4_NL weights, d_in a multiple of 64, <= 1024): two
// passes of WG / (d_in / 64) rows of one pair per workgroup (23 rows a pass
// at n_ff 704), a row's block pairs on consecutive lanes and loaded straight
// into registers (as the decode path's down kernels do), the row's partial
// sums added in LDS in pair order; the pair's column quantised here (q8_0,
// or q8_1), y = .scale W a.
template <int HD, int CD, int AM>
__global__ __launch_bounds__(WG) void k_fire_k32(const FireParams f) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int32_t s_m[3][256];
    constexpr int NPS = 2;
    __shared__ float s_red[NPS][WG];          // the lanes' partial row sums
    const int p = blockIdx.y, F = f.d_in, D = f.d_out;
    const int NP = F / 64, RPP = dn_grp_rpp(F), R = NPS * RPP;
    const int r0 = blockIdx.x * R, nr = max(0, min(R, D - r0));
    if (f.n_live && p >= *f.n_live) return;
    const int F4 = F / 4;
    // 1. the pair's column (fp32), then its tier
    const u32x4 a4 = reinterpret_cast<const u32x4 *>(f.cur + (f.cur_shared ? 0 : (int64_t)p * F))[min((int)threadIdx.x, F4 - 1)];
    int e;
    const FireRes rs = fire_resolve(f, p, s_m, &e);
    if (f.kind == 0) fire_count(f, e, rs);
    // 2. the rows' block pairs: lane -> row lrow of each pass, block pair pl
    //    (lanes past RPP rows idle)
    const int lrow = threadIdx.x / NP, pl = threadIdx.x - lrow * NP;
    const bool lane_live = lrow < RPP;
    const int tier = rs.tier < 2 ? rs.tier : 1, idx = rs.tier < 2 ? rs.idx : 0;
    const int wt = tier == 0 ? HD : CD;
    const int rbytes = (F / 32) * blk_bytes(wt);
    const uint8_t * slab = tier == 0 ? f.hot + (uint64_t)idx * f.hot_stride : f.cold + (uint64_t)idx * f.cold_stride;
    DnPair w[NPS];
#pragma unroll
    for (int ps = 0; ps < NPS; ++ps) {
        const int r = min(ps * RPP + min(lrow, RPP - 1), max(nr - 1, 0));
        const uint8_t * src = slab + (uint64_t)(r0 + r) * rbytes + (uint64_t)pl * (2 * blk_bytes(wt));
        if (tier == 0) dn_pair_load<HD>(w[ps], src);
        else dn_pair_load<CD>(w[ps], src);
    }
    // 3. the column's q8 in LDS
    ActView L;
    act_layout(F, 0, &L);
    {
        const float v[4] = {__uint_as_float(a4.x), __uint_as_float(a4.y), __uint_as_float(a4.z), __uint_as_float(a4.w)};
        q8_quad<AM>(smem, L, v, threadIdx.x, (int)threadIdx.x < F4);
    }
    __syncthreads();
    const float scale = f.kind == 1 ? (rs.tier == 0 ? (f.s_hot ? f.s_hot[rs.idx] : 1.0f)
                                                    : (rs.tier == 1 ? (f.s_cold ? f.s_cold[rs.idx] : 1.0f) : 0.0f))
                                    : (rs.tier < 2 ? 1.0f : 0.0f);
    // 4. each lane dots its block pair; the row's NP partial sums meet in LDS
    //    and one thread a row adds them in pair order, scales and stores
#pragma unroll
    for (int ps = 0; ps < NPS; ++ps) {
        float acc = 0.0f;
        if (lane_live && rs.tier < 2) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const Act32 a = act32<AM>(smem, L, 2 * pl + h);
                acc += tier == 0 ? dn_dot<AM, HD>(dn_block<HD>(w[ps], h), a) : dn_dot<AM, CD>(dn_block<CD>(w[ps], h), a);
            }
        }
        s_red[ps][threadIdx.x] = acc;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < NPS * RPP; i += WG) {
        const int ps = i / RPP, lr = i - ps * RPP, r = ps * RPP + lr;
        if (r >= nr) continue;
        float sum = 0.0f;
        for (int j = 0; j < NP; ++j) sum += s_red[ps][lr * NP + j];
        f.dst[(int64_t)p * D + r0 + r] = sum * scale;
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

// LDS bytes of one half of a gate_up item (32 rows of the longer gate_up
// row, plus one dword a funnel read may touch past the end), at least half
// the routing's scratch, which the two halves hold before the first item
int dec_gu_half_bytes(int T, int row_bytes) {
    const int halves = T == 1 ? gu_halves<1>() : gu_halves<DEC_MAXT>();
    // eight waves' regions of 4 rows each (plus a dword a funnel read may
    // touch past a span's end), at least the routing's scratch over the halves
    const int rows = 8 * align16i(4 * row_bytes + 32);
    const int b = std::max(rows, align16i((int)sizeof(GuScratch) / halves + 16));
    return (b + 127) / 128 * 128;                     // eight 16-aligned regions
}

// dynamic LDS of B: the halves of an item staged at once (both with one
// token, one with more), one activation column per token of the call (a
// group has at most one member per token), the IQ2_S codebook when used
int dec_lds_gate_up(const DecParams & p, int ht, int ct) {
    const bool iq2 = ht == T_IQ2_S || ct == T_IQ2_S;
    const int halves = p.T == 1 ? gu_halves<1>() : gu_halves<DEC_MAXT>();
    return align16i(halves * p.w_lds_gu + std::min(p.T, DEC_MAXT) * dec_act_bytes(p.d_model)) +
           (iq2 ? (int)sizeof(Iq2sTables) : 0);
}

// dynamic LDS of C: every pair's quantised down column
int dec_lds_down(const DecParams & p) {
    return p.T * p.top_k * dec_act_bytes(p.n_ff);
}

namespace {
// resident workgroups of a kernel on the current device (cached per device,
// kernel and LDS bytes; a kernel's block size is fixed)
template <typename F>
int resident_wgs(F k, int lds, int block) {
    static std::mutex mu;
    static std::map<std::tuple<int, const void *, int>, int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    const auto key = std::make_tuple(dev, reinterpret_cast<const void *>(k), lds);
    std::lock_guard<std::mutex> lk(mu);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, block, lds) != hipSuccess) per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) cus = 0;
    const int n = per_cu * cus;
    cache[key] = n;
    return n;
}

// launch with the dispatch's own begin/end timestamps recorded into e0/e1
// when profiling (e0 != nullptr)
template <typename F>
void launch_timed(F k, dim3 grid, int lds, hipStream_t s, hipEvent_t e0, hipEvent_t e1, const DecParams & p,
                  int block = WG) {
    if (e0) hipExtLaunchKernelGGL(k, grid, dim3(block), (uint32_t)lds, s, e0, e1, 0u, p);
    else hipLaunchKernelGGL(k, grid, dim3(block), lds, s, p);
}

}  // namespace

hipError_t launch_decode(const DecParams & p, int hgu, int cgu, int hdn, int cdn, int am, int gelu, hipStream_t s,
                         hipEvent_t * ev) {
    hipEvent_t e[8] = {};
    if (ev)
        for (int i = 0; i < 8; ++i) e[i] = ev[i];
    {
        // E router workgroups, then the quantisation workgroups (4 waves each)
        const int per_tok = am == AM_CPU ? p.d_model / 256 : (p.d_model + 63) / 64;
        const dim3 grid(p.n_expert + (p.T * per_tok + 3) / 4);
        if (am == AM_CPU) launch_timed(k_dec_route<AM_CPU>, grid, 0, s, e[0], e[1], p);
        else launch_timed(k_dec_route<AM_Q8_1>, grid, 0, s, e[0], e[1], p);
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    {
        // one workgroup per possible item: every routed pair could be a group
        // of its own; the workgroups past the call's groups stop after the
        // routing.  No workgroup waits on another, so any grid is safe.
        const int groups_max = std::min(p.T * p.top_k, DEC_PMAX);
        const int items = groups_max * (p.n_ff / DEC_GU_BLK);     // at most; the groups decide
        const int lds = dec_lds_gate_up(p, hgu, cgu);
        auto go = [&](auto k, int block) {
            const int cap = resident_wgs(k, lds, block);
            const int grid = std::max(1, cap > 0 ? std::min(items, cap) : items);
            launch_timed(k, dim3(grid), lds, s, e[2], e[3], p, block);
        };
#define LL_GU(A, B, M, G) \
        if (hgu == A && cgu == B && am == M && gelu == G) { \
            if (p.T == 1) go(k_dec_gate_up<A, B, M, 1, G>, gu_nt<1>()); \
            else go(k_dec_gate_up<A, B, M, DEC_MAXT, G>, gu_nt<DEC_MAXT>()); \
        } else
#define LL_GU2(A, B) LL_GU(A, B, AM_CPU, SRC_GEGLU_TABLE) LL_GU(A, B, AM_CPU, SRC_GEGLU_TANH) \
                     LL_GU(A, B, AM_Q8_1, SRC_GEGLU_TABLE) LL_GU(A, B, AM_Q8_1, SRC_GEGLU_TANH)
        LL_GU2(T_Q4_K, T_IQ2_S) LL_GU2(T_Q4_K, T_Q4_K) LL_GU2(T_IQ2_S, T_IQ2_S) LL_GU2(T_IQ2_S, T_Q4_K)
        return hipErrorInvalidValue;
#undef LL_GU2
#undef LL_GU
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    {
        // one token: the kernel over every group (its 8 columns are 9 KB); more:
        // by group (each workgroup reads its members' columns only) + combine,
        // or over every group (every pair's column in each workgroup)
        const int lds = dec_lds_down(p);
        const int rows = 1 << p.dn_rows_log2;
        const dim3 grid((p.d_model + rows - 1) / rows);
        const int grows = DN_GRP_NPS * dn_grp_rpp(p.n_ff);
        const dim3 ggrid((p.d_model + grows - 1) / grows, std::min(p.T * p.top_k, DEC_PMAX));
        const int glds = std::min(p.T, DEC_MAXT) * dec_act_bytes(p.n_ff);
#define LL_DN(A, B, M) \
        if (hdn == A && cdn == B && am == M) { \
            if (p.T == 1) launch_timed(k_dec_down<A, B, M, 1>, grid, lds, s, e[4], e[5], p); \
            else if (!p.dn_by_group) launch_timed(k_dec_down<A, B, M, DEC_MAXT>, grid, lds, s, e[4], e[5], p); \
            else launch_timed(k_dec_down_grp<A, B, M, DEC_MAXT, DN_GRP_NPS>, ggrid, glds, s, e[4], e[5], p); \
        } else
#define LL_DN2(A, B) LL_DN(A, B, AM_CPU) LL_DN(A, B, AM_Q8_1)
        LL_DN2(T_Q5_0, T_IQ4_NL) LL_DN2(T_Q5_0, T_Q5_0) LL_DN2(T_IQ4_NL, T_IQ4_NL) LL_DN2(T_IQ4_NL, T_Q5_0)
        return hipErrorInvalidValue;
#undef LL_DN2
#undef LL_DN
        if (p.T > 1 && p.dn_by_group)
            launch_timed(k_dec_combine, dim3((p.T * p.d_model + WG - 1) / WG), 0, s, e[6], e[7], p);
    }
    return hipGetLastError();
}

int fire_lds(const FireParams & f, int ht, int ct) {
    if (k256_type(ht)) {
        const bool iq2 = ht == T_IQ2_S || ct == T_IQ2_S;
        return align16i(f.w_lds + dec_act_bytes(f.d_in)) + (iq2 ? (int)sizeof(Iq2sTables) : 0);
    }
    return dec_act_bytes(f.d_in);
}

hipError_t launch_fire(const FireParams & f, int ht, int ct, int am, hipStream_t s) {
    const int P = f.n_used * f.n_tokens;
    const int lds = fire_lds(f, ht, ct);
    if (k256_type(ht)) {
        const int rows = fire_gu_rows(f.d_in);
        const dim3 grid((f.d_out + rows - 1) / rows, P);
#define LL_F(A, B, M) if (ht == A && ct == B && am == M) hipLaunchKernelGGL((k_fire_k256<A, B, M>), grid, dim3(WG), lds, s, f); else
#define LL_F2(A, B) LL_F(A, B, AM_CPU) LL_F(A, B, AM_Q8_1)
        LL_F2(T_Q4_K, T_IQ2_S) LL_F2(T_Q4_K, T_Q4_K) LL_F2(T_IQ2_S, T_IQ2_S) LL_F2(T_IQ2_S, T_Q4_K)
        return hipErrorInvalidValue;
#undef LL_F2
#undef LL_F
    } else {
        const int rows = 2 * dn_grp_rpp(f.d_in);              // k_fire_k32's two passes
        const dim3 grid((f.d_out + rows - 1) / rows, P);
#define LL_F(A, B, M) if (ht == A && ct == B && am == M) hipLaunchKernelGGL((k_fire_k32<A, B, M>), grid, dim3(WG), lds, s, f); else
#define LL_F2(A, B) LL_F(A, B, AM_CPU) LL_F(A, B, AM_Q8_1)
        LL_F2(T_Q5_0, T_IQ4_NL) LL_F2(T_Q5_0, T_Q5_0) LL_F2(T_IQ4_NL, T_IQ4_NL) LL_F2(T_IQ4_NL, T_Q5_0)
        return hipErrorInvalidValue;
#undef LL_F2
#undef LL_F
    }
    return hipGetLastError();
}

hipError_t launch_zero_i32(int * p, int n, hipStream_t s) {
    hipLaunchKernelGGL(k_zero, dim3(std::min(1024, (n + WG - 1) / WG)), dim3(WG), 0, s, p, n);
    return hipGetLastError();
}

}  // namespace llapis
