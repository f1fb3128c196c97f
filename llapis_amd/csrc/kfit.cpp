// kfit.cpp -- the slot count the device can hold now (llapis_kfit), the four
// rules of the reference's K re-fit (src/kfit_policy.hpp:61-94): one pool
// formula for a resident and an evicted slab, bounded by a per-process budget
// when there is one; the slots that fit after the margin, raised to the
// preferred floor and lowered to the expert count; what the pool can hold
// before the floor caps it afterwards; and no rebuild for a change of one
// slot unless the slab was evicted.
#include "../../include/llapis_moe.h"

#include <algorithm>

extern "C" void llapis_kfit(const llapis_kfit_inputs * in, llapis_kfit_decision * out) {
    if (!in || !out) return;
    llapis_kfit_decision d = {};
    d.pool_mib = in->slab_mib_now + in->free_mib;
    if (in->headroom_mib >= 0 && in->slab_mib_now + in->headroom_mib < d.pool_mib) {
        d.pool_mib = in->slab_mib_now + in->headroom_mib;
        d.wddm_bound = 1;
    }
    const long long per_slot = std::max<long long>(in->per_k_mib, 1);
    const long long holdable = d.pool_mib / per_slot;
    long long k = std::min<long long>(std::max<long long>((d.pool_mib - in->keep_free_mib) / per_slot, in->k_min),
                                      in->n_expert);
    if (k > holdable) {
        k = std::max<long long>(holdable, 1);
        d.floor_capped = 1;
    }
    d.k = (int32_t)k;
    d.rebuild = in->evicted || d.k <= in->k_cur - 2 || d.k >= in->k_cur + 2;
    if (!d.rebuild) d.k = in->k_cur;
    *out = d;
}
