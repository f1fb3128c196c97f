// Plain-C entry point over the reference's K re-fit decision
// (src/kfit_policy.hpp, header-only, compiled from where it lies in the
// reference tree).  Test infrastructure only: the checker of llapis_kfit.
#include "kfit_policy.hpp"

extern "C" void ref_kfit(long long free_mib, long long slab_mib_now, long long headroom_mib, long long per_k_mib,
                         long long keep_free_mib, int k_cur, int k_min, int n_expert, int evicted, int * k,
                         int * rebuild, int * wddm_bound, int * floor_capped, long long * pool_mib) {
    kfit::inputs in;
    in.free_mib = free_mib;
    in.slab_mib_now = slab_mib_now;
    in.headroom_mib = headroom_mib;
    in.per_k_mib = per_k_mib;
    in.keep_free_mib = keep_free_mib;
    in.k_cur = k_cur;
    in.k_min = k_min;
    in.n_expert = n_expert;
    in.evicted = evicted != 0;
    const kfit::decision d = kfit::fit(in);
    *k = d.k;
    *rebuild = d.rebuild;
    *wddm_bound = d.wddm_bound;
    *floor_capped = d.floor_capped;
    *pool_mib = d.pool_mib;
}
