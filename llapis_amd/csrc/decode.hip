// decode.hip -- the MoE layer for decode batches (1..4 tokens) in three
// kernels on gfx950:
//
//   A  k_dec_route   router logits (one workgroup per expert, all tokens) and,
//                    in the workgroups after those, the tokens' activation
//                    quantisation.
//   B  k_dec_gate_up every workgroup selects the routing from the logits
//                    (softmax, top-k with DPP wave reductions, ties to the
//                    lower index), groups the routed pairs by expert (decode
//                    once, dot N: the tokens that share an expert read its
//                    slab once) and resolves each group's tier (the residency
//                    predicate of moert/cuda/ffn_moe.cu:80-130); the first
//                    workgroup publishes ids, weights and groups for C.  Then a
//                    loop over the workgroup's (expert group, 16-row block)
//                    items: the expert's rows stream through LDS with 128-bit
//                    loads and are dotted against every member token, the next
//                    item's loads in flight meanwhile.
//   C  k_dec_down    a loop over (expert group, 32-row block) items: GEGLU and
//                    down activation quantisation of each group's pairs (while
//                    the first slab is in flight), the down projection with
//                    the expert's .scale, and the combine: the last arrival of
//                    a (token, row block) writes the weighted sum of the
//                    token's top_k outputs for those rows.
//
// Every load a kernel issues before its first wait is unconditional (clamped
// addresses instead of branches) and issued in the order its data are needed:
// loads complete in issue order, so a wait then covers only the loads before
// it -- the routing does not wait for the codebook, nor the GEGLU for the
// weight slab.  B and C grids are sized to the resident workgroups; no
// workgroup ever waits on another.  C's per-pair outputs are handed to the
// combine with device-scope coherent stores and one arrival atomic each; the
// last arriver reads them with device-scope coherent loads.
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
// of their first pair; each group's tier by the residency predicate, read
// from es/se/ss (the exp_slot/slot_exp/slot_state mirrors or copies of them).
__device__ void build_groups(const DecParams & p, const int * s_ids, GroupInfo * groups, int * n_groups,
                             const int32_t * es, const int32_t * se, const int32_t * ss) {
    const int lane = threadIdx.x & 63;
    const int T = p.T, E = p.n_expert, P = T * p.top_k;
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
            groups[lane].mem[0] = lane;
        }
        if (lane == 0) *n_groups = P;
        return;
    }
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
        int idx;
        const int tier = tier_of(ex, &idx);
        groups[gid].tier = tier;
        groups[gid].idx = idx;
        groups[gid].n_mem = min(nmem, min(T, DEC_MAXT));     // one member per token at most
    }
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

// Router logits of every token (workgroups e < E, one expert each) and the
// tokens' gate_up activation quantisation (the workgroups after them: one
// wave per q8_K 256-block, or per 64 values of q8_1); the first of those also
// zeroes the call's hand-off counters and flags.  Nothing waits on anything:
// the kernel ends when the router rows have been read.
template <int AM>
__global__ __launch_bounds__(WG) void k_dec_route(const DecParams p) {
    __shared__ float s_part[DEC_MAXT][WG / 64];
    const int E = p.n_expert;
    if ((int)blockIdx.x < E) {
        router_expert(p, blockIdx.x, s_part);
        return;
    }
    const int d = p.d_model, T = p.T;
    if ((int)blockIdx.x == E) {
        // the call's hand-off counters start at zero (the down kernel's
        // combine arrivals; the fused gate_up+down kernel's item done flags)
        for (int i = threadIdx.x; i < DEC_MAXT * p.n_rb_down; i += WG) p.comb_count[i] = 0;
        const int n_done = p.T * p.top_k * ((2 * p.n_ff + 15) / 16);
        for (int i = threadIdx.x; i < n_done; i += WG) p.gu_done[i] = 0;
    }
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

// Softmax + top-K of one token in one wave, from its logits already in
// registers (v[j] = entry lane + 64 j; entries at or past E are ignored): the
// arithmetic of select_token_n (exp(x - max), the sum in double, probabilities
// scaled by float(1/sum); the K largest in descending order, equal
// probabilities to the lower index; weights p / max(sum of the K in double,
// 6.103515625e-5)).  Probabilities are >= 0, so they are compared as ints (one
// DPP max per step, no NaN canonicalisation); nothing branches per lane; ids
// and weights stay in lane k until the end, written to LDS when `wr`.
template <int NJ>
__device__ __forceinline__ void select_fast(const float (&v)[4], int E, int K, int * s_ids, float * s_w, bool wr) {
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
    int q[NJ];                  // probabilities as ints; -1: absent or taken
#pragma unroll
    for (int j = 0; j < NJ; ++j) q[j] = lane + 64 * j < E ? __float_as_int(__fmul_rn(ev[j], inv)) : -1;
    int myid = 0, mysel = 0;
    for (int k = 0; k < K; ++k) {
        int m = q[0];
#pragma unroll
        for (int j = 1; j < NJ; ++j) m = max(m, q[j]);
        m = wave_max_i(m);
        int e = -1;             // the lowest index holding m
#pragma unroll
        for (int j = NJ - 1; j >= 0; --j) {
            const uint64_t b = __ballot(q[j] == m);
            e = b ? 64 * j + (int)__builtin_ctzll(b) : e;
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j) q[j] = lane + 64 * j == e ? -1 : q[j];
        myid = lane == k ? e : myid;
        mysel = lane == k ? m : mysel;
    }
    double sum = 0.0;
    for (int k = 0; k < K; ++k) sum += (double)__int_as_float(__builtin_amdgcn_readlane(mysel, k));
    float sf = (float)sum;
    if (sf < 6.103515625e-5f) sf = 6.103515625e-5f;
    if (wr && lane < K) {
        s_ids[lane] = myid;
        s_w[lane] = __int_as_float(mysel) / sf;
    }
}

// The group record g, or an empty group when g is past the call's groups.
// Validated so that no field can send a load or store out of bounds: member
// count <= min(T, DEC_MAXT) and members < P, else the group is emptied; a
// tier other than 0/1 or an index outside its pool makes the group invalid
// (tier 2: its members contribute zeros, their combine still counts).
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

// ---------------------------------------------------------------- B / C

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

// Wave 0 waits until all n write-once flags are set (each lane polls its
// share with coherent loads; a wave vote decides), or until the wall-clock
// bound passes (the error word is set); the result is broadcast.  The flags
// are distinct words written by distinct workgroups: no atomic, so no
// contention on one address.
__device__ bool wait_all(const DecParams & p, const int * flags, int n, int * s_flag) {
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        int ok = 1;
        const long long t0 = wall_clock64();
        while (true) {
            bool mine = true;
            for (int i = lane; i < n; i += 64) mine = mine && ld_coh_i(flags + i) != 0;
            if (__all(mine)) break;
            if (wall_clock64() - t0 > p.spin_limit) {
                ok = 0;
                if (lane == 0) __hip_atomic_store(&p.ctl->error, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        if (lane == 0) *s_flag = ok;
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

constexpr int TAB_CHUNKS = (int)(sizeof(Iq2sTables) / 16);
static_assert(TAB_CHUNKS % WG == 0, "codebook chunks per thread");
constexpr int GU_LOADS = 7;     // 16-byte loads per thread issued for one gate_up item (16 rows <= 1792 B)
constexpr int DN_LOADS = 4;     // ... for one down item (32 rows <= 512 B)
constexpr int COL_LOADS = 2;    // ... for one quantised token column, issued early (the rest later)
constexpr int DEC_MAXI = 16;    // items one workgroup may take (the grid is sized for it)

// One work item of the gate_up or down kernel: `rows` weight rows from r0 of
// one expert group's slab.  Its bytes are `nch` 16-byte chunks from src (row
// r0 at byte `off` of the first chunk).  An item without weights to read
// (past the call's items, or an invalid group) reads one chunk of a valid
// dummy address so that its loads, like every other, are unconditional.
struct DecItem {
    GroupInfo gi;
    const u32x4 * src;
    int nch, off, r0, rows, rb;
    int valid;                  // tier 0/1 with members: weights to dot (an int: a struct copy then
                                // moves no sub-dword padding through scratch)
};

__device__ __forceinline__ DecItem dec_item(const DecParams & p, const GroupInfo * grp, int ng, int it, int nrb,
                                            int rows_per, int n_rows, int d_in, int ht, int ct, const uint8_t * hot,
                                            uint64_t hs, const uint8_t * cold, uint64_t cs) {
    DecItem r;
    const int g = it / nrb, rbi = it - g * nrb;
    r.gi = validate_group(p, grp[max(0, min(g, DEC_PMAX - 1))], ng, g);
    r.valid = r.gi.tier < 2 && r.gi.n_mem > 0;
    const int wtype = r.gi.tier == 0 ? ht : ct;
    r.r0 = rbi * rows_per;
    r.rows = min(rows_per, n_rows - r.r0);
    r.rb = (d_in / blk_elems(wtype)) * blk_bytes(wtype);
    const uint64_t start = (uint64_t)r.r0 * r.rb;
    r.off = (int)(start & 15);
    if (r.valid) {
        const uint8_t * W = group_slab(r.gi.tier, r.gi.idx, hot, hs, cold, cs);
        r.src = reinterpret_cast<const u32x4 *>(W) + (start >> 4);
        r.nch = (int)(((start + (uint64_t)r.rows * r.rb + 15) >> 4) - (start >> 4));
    } else {
        r.src = reinterpret_cast<const u32x4 *>(p.logits);
        r.nch = 1;
    }
    return r;
}

template <int N>
struct Regs {
    u32x4 r[N];
};
template <int N>
__device__ __forceinline__ void item_load(Regs<N> & s, const DecItem & it) {
#pragma unroll
    for (int k = 0; k < N; ++k) s.r[k] = it.src[min((int)threadIdx.x + k * WG, it.nch - 1)];
}
// the item's chunks into LDS from 0 (chunks past N per thread: loaded here)
template <int N>
__device__ __forceinline__ void item_store(const Regs<N> & s, const DecItem & it, uint8_t * smem) {
#pragma unroll
    for (int k = 0; k < N; ++k) {
        const int i = threadIdx.x + k * WG;
        if (i < it.nch) *reinterpret_cast<u32x4 *>(smem + 16 * i) = s.r[k];
    }
    for (int i = threadIdx.x + N * WG; i < it.nch; i += WG) *reinterpret_cast<u32x4 *>(smem + 16 * i) = it.src[i];
}

// the workgroup's items: a contiguous range, so that consecutive items of a
// workgroup are neighbouring row blocks of one expert
__device__ __forceinline__ void item_range(int n_items, int * i0, int * i1) {
    *i0 = (int)((int64_t)blockIdx.x * n_items / gridDim.x);
    *i1 = (int)((int64_t)(blockIdx.x + 1) * n_items / gridDim.x);
}

// Dots of one item's rows (staged in LDS at 0) against its members' columns
// av[c], c < n_mem <= MT; the per-row sums are complete in lane lr == 0 of
// the row.
template <int HT, int CT, int AM, int MT>
__device__ __forceinline__ void item_dot(const uint8_t * smem, const DecItem & it, int d_in, const ActView * av,
                                         float * acc, int grid_off) {
    constexpr int LPR = Fmt<HT>::LPR;
    const int rw = threadIdx.x / LPR, lr = threadIdx.x % LPR;
#pragma unroll
    for (int c = 0; c < MT; ++c) acc[c] = 0.0f;
    const int n_mem = it.gi.n_mem;
    if (it.valid && rw < it.rows) {
        const int wb = it.off + rw * it.rb;
        const int U = d_in / Fmt<HT>::UNIT;
        if (it.gi.tier == 0) {
            if (MT == 1 || n_mem == 1) {    // one member: the single-column unit
                for (int u = lr; u < U; u += LPR) unit_dot_n<HT, AM, 1>(smem, wb, u, av, n_mem, acc, grid_off);
            } else {
                for (int u = lr; u < U; u += LPR) unit_dot_n<HT, AM, MT>(smem, wb, u, av, n_mem, acc, grid_off);
            }
        } else {
            if (MT == 1 || n_mem == 1) {
                for (int u = lr; u < U; u += LPR) unit_dot_n<CT, AM, 1>(smem, wb, u, av, n_mem, acc, grid_off);
            } else {
                for (int u = lr; u < U; u += LPR) unit_dot_n<CT, AM, MT>(smem, wb, u, av, n_mem, acc, grid_off);
            }
        }
    }
#pragma unroll
    for (int c = 0; c < MT; ++c)
#pragma unroll
        for (int o = LPR / 2; o >= 1; o >>= 1) acc[c] += __shfl_xor(acc[c], o, LPR);
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

// The members' gate_up rows of group gi (loads only, unconditional: members
// past n_mem and positions past d_in re-read valid entries).  SRC _COH: the
// rows were written by other workgroups of the same kernel.
template <int SRC, int MT>
__device__ __forceinline__ void members_load(ActBatch (&ab)[MT], const DecParams & p, const GroupInfo & gi, int d_in) {
    const int P = p.T * p.top_k, lane = threadIdx.x & 63, at0 = (threadIdx.x >> 6) * 64;
#pragma unroll
    for (int c = 0; c < MT; ++c) {
        const int m = max(0, min(member(gi, min(c, max(gi.n_mem - 1, 0))), P - 1));
        const float * g = p.ygu + (int64_t)m * 2 * d_in;
#pragma unroll
        for (int j = 0; j < Q8_BATCH; ++j) {
            const int pos = min(at0 + j * WG + lane, d_in - 1);
            ab[c].g[j] = ld_src<SRC>(g + pos);
            ab[c].u[j] = ld_src<SRC>(g + d_in + pos);
        }
    }
}
// GEGLU + q8 quantisation of the members' down activations into LDS (the
// batch loaded by members_load; values past Q8_BATCH * WG are loaded here)
template <int SRC, int AM, int MT>
__device__ __forceinline__ void members_quant(uint8_t * smem, const ActView * av, const ActBatch (&ab)[MT],
                                              const DecParams & p, const GroupInfo & gi, int d_in) {
    const int at0 = (threadIdx.x >> 6) * 64;
#pragma unroll
    for (int c = 0; c < MT; ++c) {
        if (c < gi.n_mem) {
            if (at0 < d_in) act_batch_quant<SRC, AM>(smem, av[c], ab[c], d_in, at0);
            ActSrc src;
            src.p = p.ygu + (int64_t)member(gi, c) * 2 * d_in;
            src.n = d_in;
            quantize_q8_32_rest<SRC, AM>(smem, av[c], src, d_in);
        }
    }
}

constexpr int DEC_NARR = DEC_MAXI * DEC_MAXT;     // down-item arrivals one workgroup can make
static_assert(DEC_NARR <= 64, "one wave compacts the arrivals");

// The down items [i0, i1) of the call (32-row blocks of the groups' experts):
// per group its members' GEGLU and down activation quantisation; per item the
// down projection with the expert's .scale, the next item's slab loaded into
// registers meanwhile; outputs per pair with coherent stores.  Then the
// combine: one arrival per (member, item); the last arrival of a (token, row
// block) writes the weighted sum of that token's top_k outputs for those
// rows.  The first item's slab loads were issued by the caller (st, cur).
// WAIT: the gate_up outputs come from the same kernel -- the done flags of
// all of a group's gate_up items are awaited (bounded) before its members are
// read; a wait that times out ends the loop (the error word is set).  Without
// WAIT the caller has loaded the first group's members (ab) before the slab.
// w: the routing weights [T][top_k] (LDS or global, as the caller has them).
template <int HD, int CD, int AM, int SRC, int MT, bool WAIT>
__device__ __forceinline__ void down_items(const DecParams & p, uint8_t * smem, const GroupInfo * grp, int ng, int i0, int i1,
                           Regs<DN_LOADS> & st, DecItem cur, ActBatch (&ab)[MT], const float * w, int * s_arr,
                           int * s_done, int * s_nd, int * s_flag) {
    constexpr int LPR = Fmt<HD>::LPR, ROWS = WG / LPR;
    static_assert(Fmt<HD>::LPR == Fmt<CD>::LPR && !k256<HD>() && !k256<CD>(), "down formats");
    const int D = p.d_model, d_in = p.n_ff, K = p.top_k, nrb = p.n_rb_down;
    const int nrb_gu = (2 * d_in + 15) / 16;
    bool ok = true;
    if (WAIT) {
        ok = wait_all(p, p.gu_done + (i0 / nrb) * nrb_gu, nrb_gu, s_flag);
        members_load<SRC, MT>(ab, p, cur.gi, d_in);
    }
    ActView tmp;
    const int abytes = act_layout(d_in, 0, &tmp);
    const int a0 = p.w_lds_dn;
    ActView av[MT];
#pragma unroll
    for (int c = 0; c < MT; ++c) act_layout(d_in, a0 + c * abytes, &av[c]);
    members_quant<SRC, AM, MT>(smem, av, ab, p, cur.gi, d_in);

    int n_arr = 0;
    for (int it = i0; it < i1 && ok; ++it) {
        __syncthreads();
        item_store(st, cur, smem);
        __syncthreads();
        DecItem nxt = cur;
        if (it + 1 < i1) {
            nxt = dec_item(p, grp, ng, it + 1, nrb, ROWS, D, d_in, HD, CD, p.hot_dn, p.hot_dn_stride, p.cold_dn,
                           p.cold_dn_stride);
            item_load(st, nxt);
        }
        float acc[MT];
        item_dot<HD, CD, AM, MT>(smem, cur, d_in, av, acc, 0);
        const float sc = !cur.valid ? 0.0f
                       : cur.gi.tier == 0 ? (p.s_hot ? p.s_hot[cur.gi.idx] : 1.0f)
                                          : (p.s_cold ? p.s_cold[cur.gi.idx] : 1.0f);
        const int rw = threadIdx.x / LPR, lr = threadIdx.x % LPR;
        const int n_mem = cur.gi.n_mem;
        if (lr == 0 && rw < cur.rows) {
#pragma unroll
            for (int c = 0; c < MT; ++c)
                if (c < n_mem) st_coh(p.ydn + (int64_t)member(cur.gi, c) * D + cur.r0 + rw, cur.valid ? acc[c] * sc : 0.0f);
        }
        if ((int)threadIdx.x < n_mem && n_arr + n_mem <= DEC_NARR)
            s_arr[n_arr + threadIdx.x] = (member(cur.gi, threadIdx.x) / K) * nrb + cur.r0 / ROWS;
        n_arr = min(n_arr + n_mem, DEC_NARR);
        if (it + 1 < i1 && (it + 1) / nrb != it / nrb) {
            // the next item is another group's: its members' activations
            __syncthreads();                  // every wave is done with these
            if (WAIT) ok = wait_all(p, p.gu_done + ((it + 1) / nrb) * nrb_gu, nrb_gu, s_flag);
            if (ok) {
                members_load<SRC, MT>(ab, p, nxt.gi, d_in);
                members_quant<SRC, AM, MT>(smem, av, ab, p, nxt.gi, d_in);
            }
        }
        cur = nxt;
    }

    // combine: the arrivals (one atomic each, all in flight together), the
    // completed ones compacted by one wave, then every row of every completed
    // (token, row block) spread over the workgroup's threads
    wait_vm();
    __syncthreads();
    if (threadIdx.x < 64) {
        const int a = threadIdx.x;
        const bool last = a < n_arr && atomicAdd(&p.comb_count[s_arr[a]], 1) == K - 1;
        const uint64_t m = __ballot(last);
        if (last) s_done[__popcll(m & ((1ull << a) - 1))] = s_arr[a];
        if (a == 0) *s_nd = __popcll(m);
    }
    __syncthreads();
    const int nd = *s_nd;
    for (int i = threadIdx.x; i < nd * ROWS; i += WG) {
        const int a = i / ROWS, r = i - a * ROWS;
        const int t = s_done[a] / nrb, r0 = (s_done[a] - t * nrb) * ROWS;
        if (r0 + r < D)
            p.out[(int64_t)t * D + r0 + r] = combine_row(p.ydn + (int64_t)t * K * D + r0 + r, w + t * K, K, D);
    }
}

template <int SRC> struct CohSrc;
template <> struct CohSrc<SRC_GEGLU_TABLE> { static constexpr int v = SRC_GEGLU_TABLE_COH; };
template <> struct CohSrc<SRC_GEGLU_TANH> { static constexpr int v = SRC_GEGLU_TANH_COH; };

// B: the routing, selected by every workgroup from the logits (softmax, top-k
// with DPP wave reductions, ties to the lower index), grouped by expert
// (decode once, dot N: the tokens that share an expert read its slab once),
// each group's tier by the residency predicate (moert/cuda/ffn_moe.cu:80-130);
// the first workgroup publishes ids, weights and groups.  Then a loop over the
// workgroup's (group, 16-row block) items: the next item's slab is loaded into
// registers while the current one is dotted from LDS against every member
// token.  MT: members a group can have (min(T, DEC_MAXT); 1 or DEC_MAXT),
// which bounds the columns loaded and dotted.
//
// FUSE: the down projection follows in the same kernel (HD, CD its formats,
// GSRC its GEGLU source).  Each workgroup issues its first down item's slab
// loads right after its first gate_up slab's, so they land while gate_up is
// computed; gate_up outputs are stored with coherent stores and counted per
// group (the arrival that completes a group sets its write-once ready flag);
// then the workgroup's down items (down_items, waiting on those flags).  The
// grid must not exceed the resident workgroups: every workgroup finishes all
// of its gate_up items before it waits on anything, so every wait ends.
template <int HT, int CT, int AM, int MT, bool FUSE, int HD, int CD, int GSRC>
__global__ __launch_bounds__(WG) __attribute__((amdgpu_waves_per_eu(1, 4))) void k_dec_gate_up(const DecParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int LPR = Fmt<HT>::LPR, ROWS = WG / LPR;
    static_assert(Fmt<HT>::LPR == Fmt<CT>::LPR && k256<HT>() && k256<CT>(), "gate_up formats");
    constexpr bool IQ2 = HT == T_IQ2_S || CT == T_IQ2_S;
    constexpr int ROWS_D = WG / Fmt<HD>::LPR;
    __shared__ int s_ids[DEC_PMAX];
    __shared__ float s_w[DEC_PMAX];
    __shared__ GroupInfo s_grp[DEC_PMAX];
    __shared__ int32_t s_res[3][256];       // exp_slot, slot_exp, slot_state
    __shared__ int s_ng;
    __shared__ int s_arr[FUSE ? DEC_NARR : 1], s_done[FUSE ? DEC_NARR : 1], s_nd, s_flag;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int T = p.T, K = p.top_k, E = p.n_expert, d_in = p.d_model, F2 = 2 * p.n_ff;

    // 1. every load of the prologue, in the order the data are needed and none
    //    under a condition, so each wait below waits for its own loads only:
    //    this wave's token's logits, the residency mirrors, the IQ2_S codebook,
    //    every token's quantised column
    float lg[4];
    {
        const float * lt = p.logits + (int64_t)min(wave, T - 1) * E;
#pragma unroll
        for (int j = 0; j < 4; ++j) lg[j] = lt[min(lane + 64 * j, E - 1)];
    }
    int32_t res[3];
    {
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
    }
    u32x4 tab[TAB_CHUNKS / WG];
    if (IQ2) {
#pragma unroll
        for (int k = 0; k < TAB_CHUNKS / WG; ++k)
            tab[k] = reinterpret_cast<const u32x4 *>(&c_iq2s_tab_dec)[threadIdx.x + k * WG];
    }
    ActView tmp;
    const int abytes = act_layout(d_in, 0, &tmp), a16 = abytes / 16;
    u32x4 col[MT][COL_LOADS];
#pragma unroll
    for (int c = 0; c < MT; ++c) {
        const u32x4 * src = reinterpret_cast<const u32x4 *>(p.xq + (int64_t)min(c, T - 1) * p.xq_stride);
#pragma unroll
        for (int k = 0; k < COL_LOADS; ++k) col[c][k] = src[min((int)threadIdx.x + k * WG, a16 - 1)];
    }

    // 2. the routing: wave t < T selects token t (a wave past T repeats the
    //    last token and writes nothing); then the expert groups.  The asm
    //    statement uses every logits load on every path, so the compiler
    //    cannot sink the loads an E <= 128 call leaves unused behind the later
    //    loads.
    {
        asm volatile("" ::"v"(lg[2]), "v"(lg[3]));
        const int o = min(wave, T - 1) * K;
        if (E <= 128) select_fast<2>(lg, E, K, s_ids + o, s_w + o, wave < T);
        else select_fast<4>(lg, E, K, s_ids + o, s_w + o, wave < T);
    }
#pragma unroll
    for (int i = 0; i < 3; ++i) s_res[i][threadIdx.x] = res[i];
    __syncthreads();
    if (wave == 0) build_groups(p, s_ids, s_grp, &s_ng, s_res[0], s_res[1], s_res[2]);
    __syncthreads();
    const int ng = max(0, min(s_ng, DEC_PMAX));
    const int NRB = (F2 + ROWS - 1) / ROWS;
    int i0, i1;
    item_range(ng * NRB, &i0, &i1);

    // 3. the first item's slab loads (a dummy one when there is none); fused:
    //    the first down item (its loads go out once this slab has landed, so
    //    they overlap the gate_up dots instead of sharing HBM with this slab)
    DecItem cur = dec_item(p, s_grp, ng, i0, NRB, ROWS, F2, d_in, HT, CT, p.hot_gu, p.hot_gu_stride, p.cold_gu,
                           p.cold_gu_stride);
    Regs<GU_LOADS> st;
    item_load(st, cur);
    int d0 = 0, d1 = 0;
    DecItem dcur;
    Regs<DN_LOADS> dst;
    if (FUSE) {
        item_range(ng * p.n_rb_down, &d0, &d1);
        dcur = dec_item(p, s_grp, ng, d0, p.n_rb_down, ROWS_D, p.d_model, p.n_ff, HD, CD, p.hot_dn,
                        p.hot_dn_stride, p.cold_dn, p.cold_dn_stride);
    }

    // 4. the first workgroup publishes the routing; the codebook and the
    //    columns land in LDS
    if (blockIdx.x == 0) {
        if ((int)threadIdx.x < T * K) {
            p.ids[threadIdx.x] = s_ids[threadIdx.x];
            p.w[threadIdx.x] = s_w[threadIdx.x];
        }
        for (int i = threadIdx.x; i < ng; i += WG) p.ctl->groups[i] = s_grp[i];
        if (threadIdx.x == 0) p.ctl->n_groups = ng;
        count_routes(p, s_ids, s_grp, ng);
    }
    const int a0 = p.w_lds_gu;
#pragma unroll
    for (int c = 0; c < MT; ++c) {
        if (c >= T) break;
        uint8_t * dst8 = smem + a0 + c * abytes;
#pragma unroll
        for (int k = 0; k < COL_LOADS; ++k) {
            const int i = threadIdx.x + k * WG;
            if (i < a16) reinterpret_cast<u32x4 *>(dst8)[i] = col[c][k];
        }
        const u32x4 * src = reinterpret_cast<const u32x4 *>(p.xq + (int64_t)c * p.xq_stride);
        for (int i = threadIdx.x + COL_LOADS * WG; i < a16; i += WG) reinterpret_cast<u32x4 *>(dst8)[i] = src[i];
    }
    const int grid_off = align16i(a0 + min(T, DEC_MAXT) * abytes);
    if (IQ2) {
#pragma unroll
        for (int k = 0; k < TAB_CHUNKS / WG; ++k)
            reinterpret_cast<u32x4 *>(smem + grid_off)[threadIdx.x + k * WG] = tab[k];
    }

    // 5. the items
    ActView av[MT];
    uint32_t sink = 0;
    for (int it = i0; it < i1; ++it) {
        __syncthreads();                      // the previous item's dots are done with LDS
        item_store(st, cur, smem);
        __syncthreads();
        if (FUSE && it == i0) item_load(dst, dcur);
        DecItem nxt = cur;
        if (it + 1 < i1) {
            nxt = dec_item(p, s_grp, ng, it + 1, NRB, ROWS, F2, d_in, HT, CT, p.hot_gu, p.hot_gu_stride, p.cold_gu,
                           p.cold_gu_stride);
            item_load(st, nxt);               // in flight during this item's dots
        }
        // down kernel only: touch this item's share of its expert's down slab
        // (one 16-byte load per 128-byte line; unconditional, the index
        // clamped) so the down kernel's loads find it in L2/MALL; issued
        // after this item's slab has landed, it overlaps the dots below
        if (!FUSE && p.prefetch_dn) {
            const DecItem pf = dec_item(p, s_grp, ng, (int)((int64_t)it * p.n_rb_down / NRB), p.n_rb_down,
                                        WG / Fmt<HD>::LPR, p.d_model, p.n_ff, p.hot_dn_type, p.cold_dn_type, p.hot_dn,
                                        p.hot_dn_stride, p.cold_dn, p.cold_dn_stride);
            sink ^= pf.src[min(8 * (int)threadIdx.x, pf.nch - 1)].x;
        }
        // member c's column is its token's
#pragma unroll
        for (int c = 0; c < MT; ++c)
            act_layout(d_in, a0 + max(0, min(member(cur.gi, c) / K, T - 1)) * abytes, &av[c]);
        float acc[MT];
        item_dot<HT, CT, AM, MT>(smem, cur, d_in, av, acc, grid_off);
        const int rw = threadIdx.x / LPR, lr = threadIdx.x % LPR;
        if (lr == 0 && rw < cur.rows && cur.valid) {
#pragma unroll
            for (int c = 0; c < MT; ++c)
                if (c < cur.gi.n_mem) {
                    float * y = p.ygu + (int64_t)member(cur.gi, c) * F2 + cur.r0 + rw;
                    if (FUSE) st_coh(y, acc[c]);
                    else *y = acc[c];
                }
        }
        cur = nxt;
    }
    if (!FUSE) {
        if (p.never) p.ygu[threadIdx.x] = (float)sink;      // keeps the touch loads alive
        return;
    }

    // 6. fused: each gate_up item's done flag (item index = group * NRB +
    //    row block), once this workgroup's coherent stores have completed
    wait_vm();
    __syncthreads();
    if ((int)threadIdx.x < i1 - i0)
        __hip_atomic_store(p.gu_done + i0 + threadIdx.x, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (i0 >= i1) item_load(dst, dcur);       // no gate_up item: the first down slab was not loaded yet
    // 7. the down items (the LDS of the gate_up items is free again)
    if (d0 < d1) {
        ActBatch ab[MT];
        down_items<HD, CD, AM, CohSrc<GSRC>::v, MT, true>(p, smem, s_grp, ng, d0, d1, dst, dcur, ab, s_w, s_arr,
                                                          s_done, &s_nd, &s_flag);
    }
}

// C: the down items of the gate_up kernel's groups, as a kernel of its own.
template <int HT, int CT, int AM, int GSRC, int MT>
__global__ __launch_bounds__(WG) __attribute__((amdgpu_waves_per_eu(1, 4))) void k_dec_down(const DecParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int ROWS = WG / Fmt<HT>::LPR;
    __shared__ GroupInfo s_grp[DEC_PMAX];
    __shared__ int s_arr[DEC_NARR], s_done[DEC_NARR];
    __shared__ int s_ng, s_nd, s_flag;
    const int nrb = p.n_rb_down;
    // the call's groups, written by B's first workgroup
    {
        constexpr int GW = (int)(sizeof(GroupInfo) / 4) * DEC_PMAX;
        static_assert(GW % WG == 0, "group words per thread");
        const int * gsrc = reinterpret_cast<const int *>(p.ctl->groups);
        int v[GW / WG];
#pragma unroll
        for (int k = 0; k < GW / WG; ++k) v[k] = gsrc[threadIdx.x + k * WG];
        const int ngv = p.ctl->n_groups;
#pragma unroll
        for (int k = 0; k < GW / WG; ++k) reinterpret_cast<int *>(s_grp)[threadIdx.x + k * WG] = v[k];
        if (threadIdx.x == 0) s_ng = ngv;
    }
    __syncthreads();
    const int ng = max(0, min(s_ng, DEC_PMAX));
    int i0, i1;
    item_range(ng * nrb, &i0, &i1);
    if (i0 >= i1) return;
    // the first group's members, then the first item's slab: the members'
    // GEGLU and quantisation run while the slab is in flight
    DecItem cur = dec_item(p, s_grp, ng, i0, nrb, ROWS, p.d_model, p.n_ff, HT, CT, p.hot_dn, p.hot_dn_stride, p.cold_dn,
                           p.cold_dn_stride);
    ActBatch ab[MT];
    members_load<GSRC, MT>(ab, p, cur.gi, p.n_ff);
    Regs<DN_LOADS> st;
    item_load(st, cur);
    down_items<HT, CT, AM, GSRC, MT, false>(p, smem, s_grp, ng, i0, i1, st, cur, ab, p.w, s_arr, s_done, &s_nd,
                                            &s_flag);
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
    if (ok && wave == 0) build_groups(p, s_ids, s_grp, &s_ng, p.exp_slot, p.slot_exp, p.slot_state);
    __syncthreads();
    if (ok && blockIdx.x == 0 && (int)threadIdx.x < T * K) {
        p.ids[threadIdx.x] = s_ids[threadIdx.x];
        p.w[threadIdx.x] = s_wt[threadIdx.x];
    }
    const int ng = ok ? min(s_ng, DEC_PMAX) : 0;
    if (ok && blockIdx.x == 0) count_routes(p, s_ids, s_grp, ng);

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

// grid of a persistent item loop: as many workgroups as can be resident (the
// next item's loads then overlap the current item's dots), at most one per
// item, and enough that no workgroup takes more than DEC_MAXI items.  No
// workgroup waits on another, so any grid is safe.
template <typename F>
int item_grid(F k, int lds, int max_items) {
    const int cap = resident_wgs(k, lds);
    const int g = cap > 0 ? std::min(max_items, cap) : max_items;
    return std::max(std::max(g, 1), (max_items + DEC_MAXI - 1) / DEC_MAXI);
}
}  // namespace

hipError_t launch_decode(const DecParams & p, int hgu, int cgu, int hdn, int cdn, int am, int gelu, bool fuse_bc,
                         hipStream_t s, hipEvent_t * ev) {
    hipEvent_t e[6] = {};
    if (ev)
        for (int i = 0; i < 6; ++i) e[i] = ev[i];
    const int P = p.T * p.top_k;
    {
        // E router workgroups, then the quantisation workgroups (4 waves each)
        const int per_tok = am == AM_CPU ? p.d_model / 256 : (p.d_model + 63) / 64;
        const dim3 grid(p.n_expert + (p.T * per_tok + 3) / 4);
        if (am == AM_CPU) launch_timed(k_dec_route<AM_CPU>, grid, 0, s, e[0], e[1], p);
        else launch_timed(k_dec_route<AM_Q8_1>, grid, 0, s, e[0], e[1], p);
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    const int gu_items = P * ((2 * p.n_ff + 15) / 16), dn_items = P * p.n_rb_down;
    if (fuse_bc && p.T == 1 && hgu == T_Q4_K && cgu == T_IQ2_S && hdn == T_Q5_0 && cdn == T_IQ4_NL) {
        // gate_up and down in one kernel for one token (with more, the four
        // member columns leave too few registers for the fused loop): only
        // with every workgroup resident (its down items wait on gate_up items
        // of other workgroups)
        const int lds = std::max(dec_lds_gate_up(p, hgu, cgu), dec_lds_down(p));
        auto go = [&](auto k) -> bool {
            const int cap = resident_wgs(k, lds);
            const int grid = std::min(std::max(gu_items, dn_items), cap);
            if (grid < 1 || (gu_items + grid - 1) / grid > DEC_MAXI || (dn_items + grid - 1) / grid > DEC_MAXI)
                return false;
            launch_timed(k, dim3(grid), lds, s, e[2], e[3], p);
            return true;
        };
        bool launched = false;
#define LL_F(M, G) \
        if (am == M && gelu == G) launched = go(k_dec_gate_up<T_Q4_K, T_IQ2_S, M, 1, true, T_Q5_0, T_IQ4_NL, G>);
        LL_F(AM_CPU, SRC_GEGLU_TABLE) LL_F(AM_CPU, SRC_GEGLU_TANH) LL_F(AM_Q8_1, SRC_GEGLU_TABLE)
        LL_F(AM_Q8_1, SRC_GEGLU_TANH)
#undef LL_F
        if (launched) {
            const hipError_t err = hipGetLastError();
            if (err != hipSuccess) return err;
            // profiling: the fused kernel is timed as the gate_up stage; the
            // down stage's events are recorded back to back (0 ms)
            if (e[4]) {
                const hipError_t e4 = hipEventRecord(e[4], s);
                if (e4 != hipSuccess) return e4;
                return hipEventRecord(e[5], s);
            }
            return hipSuccess;
        }
    }
    {
        const int lds = dec_lds_gate_up(p, hgu, cgu);
        auto go = [&](auto k) { launch_timed(k, dim3(item_grid(k, lds, gu_items)), lds, s, e[2], e[3], p); };
#define LL_GU(A, B, M) \
        if (hgu == A && cgu == B && am == M) { \
            if (p.T == 1) go(k_dec_gate_up<A, B, M, 1, false, T_Q5_0, T_IQ4_NL, SRC_GEGLU_TABLE>); \
            else go(k_dec_gate_up<A, B, M, DEC_MAXT, false, T_Q5_0, T_IQ4_NL, SRC_GEGLU_TABLE>); \
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
        const int lds = dec_lds_down(p);
        auto go = [&](auto k) { launch_timed(k, dim3(item_grid(k, lds, dn_items)), lds, s, e[4], e[5], p); };
#define LL_DN(A, B, M, G) \
        if (hdn == A && cdn == B && am == M && gelu == G) { \
            if (p.T == 1) go(k_dec_down<A, B, M, G, 1>); else go(k_dec_down<A, B, M, G, DEC_MAXT>); \
        } else
#define LL_DN2(A, B) LL_DN(A, B, AM_CPU, SRC_GEGLU_TABLE) LL_DN(A, B, AM_CPU, SRC_GEGLU_TANH) \
                     LL_DN(A, B, AM_Q8_1, SRC_GEGLU_TABLE) LL_DN(A, B, AM_Q8_1, SRC_GEGLU_TANH)
        LL_DN2(T_Q5_0, T_IQ4_NL) LL_DN2(T_Q5_0, T_Q5_0) LL_DN2(T_IQ4_NL, T_IQ4_NL) LL_DN2(T_IQ4_NL, T_Q5_0)
        return hipErrorInvalidValue;
#undef LL_DN2
#undef LL_DN
    }
    return hipGetLastError();
}

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
