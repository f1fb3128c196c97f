"""The K re-fit decision (llapis_kfit, include/llapis_moe.h), CPU only.

The reference's own test cases (tests/test_kfit_policy.cpp, with its numbers
from the reference box: 107 MiB per slot, 500 MiB kept free, floor 4) with
their expected answers, and a differential test against the reference's
header-only kfit::fit (src/kfit_policy.hpp) compiled into oracle/_ref over
random inputs that cross every rule's boundary."""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest

import llapis_amd as la
from llapis_amd import _lib as L

ROOT = Path(__file__).resolve().parents[1]
REF_KFIT = ROOT / "oracle" / "_ref" / "libkfit_ref.so"


def fit(**kw):
    base = dict(free_mib=0, slab_mib_now=0, headroom_mib=-1, per_k_mib=107, keep_free_mib=500, k_cur=0, k_min=4,
                n_expert=128, evicted=0)
    base.update(kw)
    i = L.LlapisKfitInputs(**{k: int(v) for k, v in base.items()})
    d = L.LlapisKfitDecision()
    la.lib().llapis_kfit(C.byref(i), C.byref(d))
    return d


def test_rule1_one_formula_for_both_regimes():
    a = fit(slab_mib_now=3103, free_mib=725, k_cur=29, evicted=0)
    b = fit(slab_mib_now=0, free_mib=3828, k_cur=29, evicted=1)
    assert a.pool_mib == b.pool_mib == 3828
    assert a.k == b.k == 31


def test_rule2_budget_binds_when_tighter():
    d = fit(free_mib=3828, k_cur=4, evicted=1, headroom_mib=2821)
    assert d.wddm_bound and d.pool_mib == 2821 and d.k == (2821 - 500) // 107
    d = fit(free_mib=2000, k_cur=4, evicted=1, headroom_mib=3500)
    assert not d.wddm_bound and d.pool_mib == 2000
    d = fit(free_mib=2000, k_cur=4, evicted=1, headroom_mib=-1)
    assert not d.wddm_bound and d.pool_mib == 2000


def test_rule3_floor_is_a_preference():
    d = fit(free_mib=376, k_cur=8, evicted=1)
    assert d.floor_capped and d.k == 376 // 107 and d.k < 4
    d = fit(free_mib=900, k_cur=8, evicted=1)
    assert not d.floor_capped and d.k == 4
    assert fit(free_mib=999999, k_cur=4, evicted=1).k == 128


def test_rule4_hysteresis():
    for delta in (-1, 0, 1):
        kc = (2247 + 500 - 500) // 107 - delta
        d = fit(slab_mib_now=2247, free_mib=500, k_cur=kc)
        assert not d.rebuild and d.k == kc
    assert fit(slab_mib_now=2247, free_mib=500, k_cur=10).rebuild
    d = fit(free_mib=3828, evicted=1, k_cur=(3828 - 500) // 107)
    assert d.rebuild


def test_the_measured_collapse():
    assert fit(free_mib=2850, k_cur=22, evicted=1).k >= 20
    d = fit(free_mib=950, k_cur=22, evicted=1)
    assert d.k <= 5 and d.rebuild


def test_matches_reference_kfit():
    if not REF_KFIT.exists():
        pytest.skip("oracle/_ref/libkfit_ref.so not built (needs the reference tree)")
    ref = C.CDLL(str(REF_KFIT))
    ll = C.c_longlong
    ref.ref_kfit.argtypes = [ll, ll, ll, ll, ll, C.c_int, C.c_int, C.c_int, C.c_int] + [C.POINTER(C.c_int)] * 4 + \
                            [C.POINTER(ll)]
    rng = np.random.default_rng(7)
    out = [C.c_int() for _ in range(4)] + [ll()]
    for n in range(20000):
        per_k = int(rng.choice([0, 1, 3, 107, 1000, int(rng.integers(-5, 3000))]))
        kw = dict(free_mib=int(rng.integers(-100, 300000)), slab_mib_now=int(rng.choice([0, rng.integers(0, 20000)])),
                  headroom_mib=int(rng.choice([-1, rng.integers(-5, 20000)])), per_k_mib=per_k,
                  keep_free_mib=int(rng.integers(0, 2000)), k_cur=int(rng.integers(0, 140)),
                  k_min=int(rng.integers(0, 10)), n_expert=int(rng.choice([8, 64, 128, 256])),
                  evicted=int(rng.integers(0, 2)))
        d = fit(**kw)
        ref.ref_kfit(*[kw[k] for k in ("free_mib", "slab_mib_now", "headroom_mib", "per_k_mib", "keep_free_mib",
                                       "k_cur", "k_min", "n_expert", "evicted")], *[C.byref(o) for o in out])
        got = (d.k, d.rebuild, d.wddm_bound, d.floor_capped, d.pool_mib)
        want = tuple(o.value for o in out)
        assert got == want, (kw, got, want)
