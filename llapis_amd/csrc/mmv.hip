// mmv.hip -- grouped quantised matvec for MoE decode on gfx950.
//
// One workgroup (4 wave64) computes ROWS consecutive output rows of one
// channel (a routed pair, or one compact channel of the island's mul_mat_id):
//   1. resolve the channel: which expert slab, which tier/format, which
//      activation column, which output scale (partition predicate of
//      moert/cuda/ffn_moe.cu:80-130 evaluated per channel);
//   2. issue 128-bit loads of the rows' contiguous byte range (the slab is
//      row-major ggml blocks, so ROWS rows are one contiguous stream);
//   3. while they are in flight, quantise the activation column into LDS in
//      the format the reference's dot product uses (q8_K / q8_0 / q8_1),
//      evaluating the GEGLU on the fly for the down projection, and build the
//      IQ2_S codebook in LDS when the tier is IQ2_S;
//   4. store the weight bytes to LDS, then lanes in groups of LPR dot whole
//      units (quarter super-blocks or 32-blocks) with v_dot4_i32_i8 and
//      reduce with cross-lane shuffles.
#include <hip/hip_ext.h>

#include "device.h"
#include "launch.h"

namespace llapis {
namespace dev {

__constant__ Iq2sTables c_iq2s_tab = make_iq2s_tables();

constexpr int MAXPER = 8;   // 128-bit weight loads in flight per thread before the activation work

template <int T> constexpr bool is_k256() { return T == T_Q4_K || T == T_IQ2_S; }

template <int HT, int CT, int AM, int SRC>
__global__ __launch_bounds__(WG) __attribute__((amdgpu_waves_per_eu(1, 4))) void k_mmv(const MmvParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    static_assert(Fmt<HT>::LPR == Fmt<CT>::LPR, "one lane layout per launch");
    static_assert(is_k256<HT>() == is_k256<CT>(), "one activation format per launch");
    constexpr int LPR = Fmt<HT>::LPR;
    constexpr int ROWS = WG / LPR;

    const int ch = blockIdx.y;
    const int r0 = blockIdx.x * ROWS;

    // ---- 1. resolve the channel (uniform per workgroup)
    bool valid = true;
    int tier = 0, col = 0;
    const uint8_t * W = nullptr;
    float osc = 1.0f;
    if (p.mode == MMV_COMPACT) {
        if (p.ne_live && ch >= *p.ne_live) return;       // padded channel: nothing to compute or write
        const int id = p.ids[ch];
        if (id < 0 || id >= p.n0) {
            valid = false;
        } else {
            W = p.ptrs0 ? static_cast<const uint8_t *>(p.ptrs0[id]) : p.w0 + (uint64_t)id * p.stride0;
        }
        col = p.b_ncols == 1 ? 0 : ch;
    } else {
        const int t = ch / p.top_k;
        const int e = p.ids[t * p.ids_s1 + (ch - t * p.top_k)];
        int s = -1;
        if (e >= 0 && e < p.n_expert && p.k_slots > 0) {
            const int ss = p.exp_slot[e];
            if (ss >= 0 && ss < p.k_slots && p.slot_state[ss] == 2 && p.slot_exp[ss] == e) s = ss;
        }
        if (s >= 0) {
            W = p.ptrs0 ? static_cast<const uint8_t *>(p.ptrs0[s]) : p.w0 + (uint64_t)s * p.stride0;
            osc = p.s0 ? p.s0[s] : 1.0f;
        } else if (e >= 0 && e < p.n_expert) {
            tier = 1;
            W = p.w1 + (uint64_t)e * p.stride1;
            osc = p.s1 ? p.s1[e] : 1.0f;
        } else {
            valid = false;
        }
        col = p.act_by_token ? t : ch;
    }
    const int wtype = tier ? CT : HT;
    const bool iq2 = (HT == T_IQ2_S || CT == T_IQ2_S);
    const LdsLayout L = lds_layout(p.w_lds_bytes, p.d_in, iq2);
    const int rows = min(ROWS, p.d_out - r0);
    const int rb = (p.d_in / blk_elems(wtype)) * blk_bytes(wtype);
    const uint64_t start = (uint64_t)r0 * rb;
    const uint64_t c0 = start >> 4;
    const int nch = valid ? (int)(((start + (uint64_t)rows * rb + 15) >> 4) - c0) : 0;
    const u32x4 * g = reinterpret_cast<const u32x4 *>(W) + c0;

    // ---- 2. weight loads in flight
    // Lanes past the end re-read the last chunk (in bounds, a cache hit) so
    // the loads carry no per-lane condition and stay in registers.
    u32x4 wr[MAXPER];
    if (nch > 0) {
#pragma unroll
        for (int k = 0; k < MAXPER; ++k) wr[k] = g[min((int)threadIdx.x + k * WG, nch - 1)];
    }

    // ---- 3. activation into LDS (+ IQ2_S tables)
    const ActView av = {L.q, L.d32, L.s32, L.dK, L.bsum};
    if (wtype == T_IQ2_S) copy_iq2s_tables(smem, L.grid, &c_iq2s_tab);
    if (valid) {
        ActSrc src;
        src.p = p.act + (int64_t)col * p.act_ld;
        src.n = p.d_in;
        quantize_act<HT, AM, SRC>(smem, av, src, p.d_in);
    }

    // ---- 4. weights into LDS, then dot
    if (nch > 0) {
#pragma unroll
        for (int k = 0; k < MAXPER; ++k) {
            const int i = threadIdx.x + k * WG;
            if (i < nch) *reinterpret_cast<u32x4 *>(smem + L.w + 16 * i) = wr[k];
        }
    }
    for (int i = threadIdx.x + MAXPER * WG; i < nch; i += WG)
        *reinterpret_cast<u32x4 *>(smem + L.w + 16 * i) = g[i];
    __syncthreads();

    const int rw = threadIdx.x / LPR, lr = threadIdx.x % LPR;
    float acc = 0.0f;
    if (valid && rw < rows) {
        const int wb = L.w + (int)(start & 15) + rw * rb;
        constexpr int UNIT = Fmt<HT>::UNIT;
        const int U = p.d_in / UNIT;
        if (tier == 0) {
            for (int u = lr; u < U; u += LPR) unit_dot_n<HT, AM, 1>(smem, wb, u, &av, 1, &acc, L.grid);
        } else {
            for (int u = lr; u < U; u += LPR) unit_dot_n<CT, AM, 1>(smem, wb, u, &av, 1, &acc, L.grid);
        }
    }
#pragma unroll
    for (int o = LPR / 2; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, LPR);
    if (rw < rows && lr == 0) p.y[(int64_t)ch * p.d_out + r0 + rw] = valid ? acc * osc : 0.0f;
}

}  // namespace dev

using namespace dev;

int mmv_rows_per_wg(int wtype) {
    return (wtype == T_Q4_K || wtype == T_IQ2_S) ? WG / 16 : WG / 8;
}

static int rb_of(int t, int d_in) { return (d_in / blk_elems(t)) * blk_bytes(t); }

void mmv_prepare(MmvParams & p, int ht, int ct) {
    const int rows = mmv_rows_per_wg(ht);
    const int wb = std::max(rb_of(ht, p.d_in), rb_of(ct, p.d_in)) * rows;
    p.w_lds_bytes = align16(wb + 32);
}

int mmv_lds_bytes(const MmvParams & p, int ht, int ct) {
    return lds_layout(p.w_lds_bytes, p.d_in, ht == T_IQ2_S || ct == T_IQ2_S).total;
}

using Ev = hipEvent_t;

template <int HT, int CT, int AM, int SRC>
static hipError_t go(const MmvParams & p, int n_channels, hipStream_t s, Ev e0, Ev e1) {
    const int rows = WG / Fmt<HT>::LPR;
    dim3 grid((p.d_out + rows - 1) / rows, n_channels);
    const int lds = mmv_lds_bytes(p, HT, CT);
    if (e0) hipExtLaunchKernelGGL((k_mmv<HT, CT, AM, SRC>), grid, dim3(WG), (uint32_t)lds, s, e0, e1, 0u, p);
    else hipLaunchKernelGGL((k_mmv<HT, CT, AM, SRC>), grid, dim3(WG), lds, s, p);
    return hipGetLastError();
}

template <int HT, int CT, int SRC>
static hipError_t go_am(const MmvParams & p, int am, int n, hipStream_t s, Ev e0, Ev e1) {
    return am == AM_CPU ? go<HT, CT, AM_CPU, SRC>(p, n, s, e0, e1) : go<HT, CT, AM_Q8_1, SRC>(p, n, s, e0, e1);
}

template <int HT, int CT>
static hipError_t go_src(const MmvParams & p, int am, int src, int n, hipStream_t s, Ev e0, Ev e1) {
    if constexpr (is_k256<HT>()) {
        if (src != SRC_PLAIN) return hipErrorInvalidValue;      // GEGLU feeds the 32-block down formats only
        return go_am<HT, CT, SRC_PLAIN>(p, am, n, s, e0, e1);
    } else {
        switch (src) {
            case SRC_PLAIN: return go_am<HT, CT, SRC_PLAIN>(p, am, n, s, e0, e1);
            case SRC_GEGLU_TABLE: return go_am<HT, CT, SRC_GEGLU_TABLE>(p, am, n, s, e0, e1);
            case SRC_GEGLU_TANH: return go_am<HT, CT, SRC_GEGLU_TANH>(p, am, n, s, e0, e1);
        }
        return hipErrorInvalidValue;
    }
}

hipError_t launch_mmv(const MmvParams & p, int ht, int ct, int am, int src, int n_channels, hipStream_t s, Ev e0,
                      Ev e1) {
    if (n_channels <= 0 || p.d_out <= 0) return hipSuccess;
#define LL_PAIR(A, B) if (ht == A && ct == B) return go_src<A, B>(p, am, src, n_channels, s, e0, e1);
    LL_PAIR(T_Q4_K, T_IQ2_S) LL_PAIR(T_Q4_K, T_Q4_K) LL_PAIR(T_IQ2_S, T_IQ2_S) LL_PAIR(T_IQ2_S, T_Q4_K)
    LL_PAIR(T_Q5_0, T_IQ4_NL) LL_PAIR(T_Q5_0, T_Q5_0) LL_PAIR(T_IQ4_NL, T_IQ4_NL) LL_PAIR(T_IQ4_NL, T_Q5_0)
#undef LL_PAIR
    return hipErrorInvalidValue;
}

}  // namespace llapis
