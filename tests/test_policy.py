"""The residency policy (llapis_amd/csrc/policy.cpp, include/moert_policy.h),
CPU only.

The scenarios of the reference's own policy tests (tests/test_moert_policy_
async.cpp, test_moert_policy_cost.cpp, test_moert_policy_resize.cpp) with
their expected outcomes, and a differential test: the reference's policy.cpp,
compiled from its source into oracle/_ref, and this library's policy are
driven through the same seeded call sequences (routing, prompt chunks,
external counts, refreshes, asynchronous fills completed, aborted or stale,
resizes, boundary passes, external forecasts) and must leave identical page
tables, mirrors and counters after every call."""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest

from llapis_amd import _lib as L
from llapis_amd.policy import Policy, TIMING_FIELDS, bind

ROOT = Path(__file__).resolve().parents[1]
REF_POLICY = ROOT / "oracle" / "_ref" / "libmoert_policy_ref.so"
FREE, FILLING, READY = L.SLOT_FREE, L.SLOT_FILLING, L.SLOT_READY


class Host:
    """Stands in for the host's callbacks: records streams and publications;
    `ret` is what stream_expert answers (a list is cycled through)."""

    def __init__(self, ret=1):
        self.ret = ret
        self.calls = 0
        self.jobs = []
        self.published = []

    def stream(self, il, e, slot):
        r = self.ret[self.calls % len(self.ret)] if isinstance(self.ret, list) else self.ret
        self.calls += 1
        if r == 2:
            self.jobs.append((il, e, slot))
        return r

    def publish(self, il):
        self.published.append(il)


def make(host, n_layers=1, n_expert=16, k=4, lib=None, seeds=True, **cfg):
    p = Policy(n_layers, n_expert, k, lib=lib, stream_expert=host.stream, publish_layer=host.publish, **cfg)
    if seeds:
        for il in range(n_layers):
            for e in range(k):
                assert p.seed(il, e, e) == 1
    return p


def tok(p, ids, il=0):
    p.observe(il, np.array(ids, np.int32), len(ids), 1)
    p.token_end()


# ------------------------------------------------ the reference's scenarios

def test_async_fill_becomes_ready_on_completion():
    """test_moert_policy_async.cpp:49-68"""
    h = Host(ret=2)
    p = make(h, cost_horizon=128, cost_reuse=51.0, cost_per_token=4)
    for _ in range(64):
        tok(p, [10, 11, 12, 13])
    assert len(h.jobs) == 4
    for il, e, s in h.jobs:
        v = p.views(il)
        assert v["exp_slot"][e] == s and v["slot_state"][s] == FILLING and v["resid"][e] == 0.0
    st = p.stats()
    assert st["fills_async"] == 4 and st["fills_completed"] == 0 and st["occupancy"] == 0.0
    for il, e, s in h.jobs:
        assert p.complete(il, s, e) == 1
    v = p.views(0)
    for il, e, s in h.jobs:
        assert v["slot_state"][s] == READY and v["hotmap"][e] == s and v["resid"][e] == 1.0
    st = p.stats()
    assert st["fills_completed"] == 4 and st["occupancy"] == 1.0
    il, e, s = h.jobs[0]
    assert p.complete(il, s, e) == 0           # twice: stale


def test_async_stale_completion_and_abort():
    """test_moert_policy_async.cpp:70-101"""
    h = Host(ret=2)
    p = make(h, cost_horizon=128, cost_reuse=51.0, cost_per_token=4)
    for _ in range(64):
        tok(p, [10, 11, 12, 13])
    il, e, s = h.jobs[0]
    assert p.complete(0, s, 9) == 0            # wrong expert
    assert p.views(0)["slot_state"][s] == FILLING
    assert p.complete(0, s, e) == 1
    il, e, s = h.jobs[1]
    assert p.abort(0, s, e) == 1
    v = p.views(0)
    assert v["slot_state"][s] == FREE and v["exp_slot"][e] < 0
    assert p.abort(0, s, e) == 0 and p.complete(0, s, e) == 0
    st = p.stats()
    assert st["fills_aborted"] == 1 and st["fills_stale"] == 3


def test_sync_streaming_is_ready_at_once():
    """test_moert_policy_async.cpp:103-114"""
    h = Host(ret=1)
    p = make(h, cost_horizon=128, cost_reuse=51.0, cost_per_token=4)
    for _ in range(64):
        tok(p, [10, 11, 12, 13])
    v = p.views(0)
    for e in range(10, 14):
        assert v["exp_slot"][e] >= 0 and v["slot_state"][v["exp_slot"][e]] == READY
    st = p.stats()
    assert st["fills_async"] == 0 and st["occupancy"] == 1.0


@pytest.mark.parametrize("reuse,moves", [(51.0, True), (500.0, False)])
def test_cost_price_binds(reuse, moves):
    """test_moert_policy_cost.cpp:47-64"""
    h = Host()
    p = make(h, cost_horizon=128, cost_reuse=reuse, cost_per_token=4)
    for _ in range(64):
        tok(p, [10, 11, 12, 13])
    es = p.views(0)["exp_slot"]
    if moves:
        assert all(es[e] >= 0 for e in (10, 11, 12, 13)) and h.calls == 4
    else:
        assert es[10] < 0 and es[0] >= 0 and h.calls == 0


def test_prompt_routing_never_promotes():
    """test_moert_policy_cost.cpp:66-79"""
    h = Host()
    p = make(h, cost_horizon=128, cost_reuse=51.0, cost_per_token=4)
    p.observe(0, np.full(200, 9, np.int32), 1, 200)
    p.prompt_tokens(200)
    p.refresh(L.REFRESH_PROMPT_END)
    assert p.views(0)["exp_slot"][9] < 0 and h.calls == 0


def test_per_token_cap():
    """test_moert_policy_cost.cpp:81-101"""
    h = Host()
    p = make(h, cost_horizon=16, cost_reuse=2.0, cost_per_token=1)
    prev, max_step, first = 0, 0, -1
    for t in range(1, 33):
        tok(p, [10, 11, 12, 13])
        max_step = max(max_step, h.calls - prev)
        if first < 0 and h.calls > 0:
            first = t
        prev = h.calls
    assert 0 < first < 16 and max_step == 1 and h.calls == 4
    assert all(p.views(0)["exp_slot"][e] >= 0 for e in (10, 11, 12, 13))


def test_prompt_end_is_uncapped_and_boundary_pass():
    """test_moert_policy_cost.cpp:103-140"""
    h = Host()
    p = make(h, cost_horizon=16, cost_reuse=2.0, cost_per_token=1)
    cnt = np.zeros(16, np.int32)
    cnt[10:14] = 100
    assert p.boundary(0, cnt, 100, 1.0, 1000.0) == 0
    p.refresh(L.REFRESH_PROMPT_END)
    assert h.calls == 4
    h = Host()
    p = make(h, cost_horizon=16, cost_reuse=51.0, cost_per_token=4)
    cnt = np.zeros(16, np.int32)
    cnt[9], cnt[7] = 100, 50
    assert p.boundary(0, cnt, 100, 1.0, 0.5) == 2 and h.calls == 2
    es = p.views(0)["exp_slot"]
    assert es[9] >= 0 and es[7] >= 0 and sum(es[e] >= 0 for e in range(4)) == 2
    assert p.boundary(0, cnt, 100, 1.0, 0.5) == 0
    c2 = np.zeros(16, np.int32)
    c2[12] = 100
    assert p.boundary(0, c2, 100, 0.0, 0.5) == 0 and p.views(0)["exp_slot"][12] < 0
    assert p.boundary(5, cnt, 100, 1.0, 0.5) == -1 and p.boundary(0, cnt, 0, 1.0, 0.5) == -1


def test_resize_ranks_compacts_and_grows():
    """test_moert_policy_resize.cpp:29-106"""
    h = Host()
    p = make(h, n_layers=2, n_expert=8, k=4, cost_reuse=1000.0)
    ids = [1] * 4 + [0] * 3 + [3] + [7] * 6
    for il in range(2):
        p.observe(il, np.array(ids, np.int32), len(ids), 1)
    p.token_end()
    d0 = p.stats()["demotions"]
    assert p.resize(2) == 1 and h.calls == 0
    for il in range(2):
        v = p.views(il)
        assert p.layer_k(il) == 2
        assert list(v["slot_exp"]) == [1, 0] and list(v["slot_state"]) == [READY, READY]
        assert v["exp_slot"][1] == 0 and v["exp_slot"][0] == 1
        assert v["exp_slot"][2] == v["exp_slot"][3] == v["exp_slot"][7] == -1
        assert v["resid"][1] == v["resid"][0] == 1.0 and v["resid"][3] == 0.0
    assert p.stats()["demotions"] == d0 + 4
    assert p.resize(5) == 1
    for il in range(2):
        v = p.views(il)
        assert list(v["slot_exp"]) == [1, 0, -1, -1, -1] and v["slot_state"][4] == FREE
    assert p.can_seed(0, 7) == 1 and p.can_seed(0, 1) == 0
    assert p.resize(0) == 0 and p.resize(9) == 0
    assert p.resize(5) == 1 and list(p.views(0)["slot_exp"][:3]) == [1, 0, -1]


def test_create_refuses_bad_geometry():
    with pytest.raises(ValueError):
        Policy(1, 8, 9)
    with pytest.raises(ValueError):
        Policy(2, 8, 4, k_per_layer=[4, 0])


# ------------------------------------------- differential against the reference

def ref_lib():
    if not REF_POLICY.exists():
        pytest.skip("oracle/_ref/libmoert_policy_ref.so not built (needs the reference tree)")
    return bind(C.CDLL(str(REF_POLICY)))


def snapshot(p, host):
    out = {"k": [p.layer_k(il) for il in range(p.n_layers)], "hit": p.hit_rate(),
           "published": list(host.published), "jobs": list(host.jobs), "calls": host.calls}
    st = p.stats()
    for f in TIMING_FIELDS:
        st.pop(f)
    out["stats"] = st
    for il in range(p.n_layers):
        for name, a in p.views(il).items():
            out[f"{name}{il}"] = a.tolist()
    w = p.window(16)
    out["window"] = (w["tokens"], w["hot_routes"], w["cold_routes"], w["hit_rate"])
    return out


def routing(rng, n_tok, E, top_k, skew):
    pr = 1.0 / np.arange(1, E + 1) ** skew
    pr = pr[rng.permutation(E)]
    pr /= pr.sum()
    return np.concatenate([rng.choice(E, top_k, replace=False, p=pr) for _ in range(n_tok)]).astype(np.int32)


@pytest.mark.parametrize("seed", range(12))
def test_matches_reference_policy(seed):
    ref = ref_lib()
    rng = np.random.default_rng(1000 + seed)
    NL, E, top_k = int(rng.integers(1, 4)), int(rng.choice([8, 16, 32])), 4
    K = int(rng.integers(2, E // 2 + 1))
    kpl = [int(v) for v in rng.integers(1, E + 1, NL)] if rng.random() < 0.3 else None
    cfg = dict(cost_horizon=int(rng.choice([4, 16, 64])), cost_reuse=float(rng.choice([0.25, 2.0, 6.0])),
               cost_per_token=int(rng.integers(1, 5)), blend_c=float(rng.choice([0.0, 0.5])))
    schedule = [int(v) for v in rng.choice([1, 2, 2, 0], 64)]
    external = bool(rng.random() < 0.5)
    sides = []
    for lib in (None, ref):
        h = Host(ret=schedule)
        p = Policy(NL, E, K, lib=lib, k_per_layer=kpl, stream_expert=h.stream, publish_layer=h.publish, **cfg)
        p.set_external(external)
        sides.append((p, h))
    for il in range(NL):
        k_il = sides[0][0].layer_k(il)
        for e in rng.choice(E, min(k_il, E) // 2, replace=False):
            slot = int(rng.integers(0, k_il))
            assert sides[0][0].seed(il, int(e), slot) == sides[1][0].seed(il, int(e), slot)
    skew = float(rng.choice([0.6, 1.1, 2.0]))
    ops = ["tok"] * 14 + ["prompt", "refresh", "complete", "complete", "complete", "abort", "stale", "boundary",
                          "forecast", "resize", "active", "seed"]
    for step in range(300):
        op = "reset" if rng.random() < 0.01 else ops[int(rng.integers(0, len(ops)))]
        args = {}
        if op in ("tok", "prompt"):
            n = 1 if op == "tok" else int(rng.integers(2, 40))
            args["ids"] = [routing(rng, n, E, top_k, skew) for _ in range(NL)]
            args["hc"] = [(int(rng.integers(0, 5)), int(rng.integers(0, 5))) for _ in range(NL)]
            args["n"] = n
        elif op == "refresh":
            args["reason"] = int(rng.choice([L.REFRESH_PROMPT_END, L.REFRESH_VISIBLE_INTERVAL, L.REFRESH_TURN_END]))
        elif op in ("complete", "abort", "stale"):
            args["pick"] = int(rng.integers(0, 1 << 30))
        elif op == "boundary":
            args["il"] = int(rng.integers(0, NL + 1)) if rng.random() < 0.1 else int(rng.integers(0, NL))
            args["counts"] = rng.integers(0, 60, E).astype(np.int32)
            args["n_tok"] = int(rng.integers(0, 50))
            args["w"], args["r"] = float(rng.choice([0.0, 0.3, 1.0])), float(rng.choice([0.1, 0.5, 3.0]))
        elif op == "forecast":
            args["f"] = None if rng.random() < 0.4 else (rng.random((NL, E)) * cfg["cost_horizon"]).astype(np.float32)
            args["r"], args["cap"] = float(rng.choice([0.5, 2.0])), int(rng.integers(0, 3))
        elif op == "resize":
            args["k"] = int(rng.integers(0, E + 2))
        elif op == "active":
            args["k"] = int(rng.integers(0, E + 1))
        elif op == "seed":
            args["il"], args["e"] = int(rng.integers(0, NL)), int(rng.integers(0, E))
            args["slot"] = int(rng.integers(0, E))
        results = []
        for p, h in sides:
            r = None
            if op in ("tok", "prompt"):
                for il in range(NL):
                    ids = args["ids"][il]
                    if external:
                        cnt = np.bincount(ids, minlength=E).astype(np.int32)
                        p.add_counts(il, cnt, *args["hc"][il])
                    else:
                        p.observe(il, ids, top_k, args["n"])
                if op == "tok":
                    p.token_end()
                else:
                    p.prompt_tokens(args["n"])
            elif op == "refresh":
                p.refresh(args["reason"])
            elif op in ("complete", "abort", "stale"):
                if h.jobs:
                    il, e, s = h.jobs.pop(args["pick"] % len(h.jobs))
                    if op == "stale":
                        e = (e + 1) % E
                    r = p.abort(il, s, e) if op == "abort" else p.complete(il, s, e)
            elif op == "boundary":
                r = p.boundary(args["il"], args["counts"], args["n_tok"], args["w"], args["r"])
            elif op == "forecast":
                p.set_forecast(args["f"], args["r"], args["cap"])
            elif op == "resize":
                r = p.resize(args["k"])
            elif op == "active":
                r = p.active_k(args["k"])
            elif op == "reset":
                p.reset_stats()
            elif op == "seed":
                r = p.seed(args["il"], args["e"], args["slot"])
            results.append((r, snapshot(p, h)))
        assert results[0] == results[1], (seed, step, op)
    # the sequence exercised the decision, not only the bookkeeping
    assert sides[0][1].calls >= 3, sides[0][1].calls
    for p, _ in sides:
        p.close()


def test_residency_runtime_refuses_bad_geometry():
    """llapis_residency_create checks the geometry before any device call,
    so the refusal is testable without a GPU."""
    lib = L.lib()
    for n_layers, n_expert, k in ((0, 16, 4), (2, 0, 4), (2, 16, 0)):
        c = L.MoertPolicyConfig()
        lib.moert_policy_config_defaults(C.byref(c))
        c.n_layers, c.n_expert, c.k = n_layers, n_expert, k
        assert not lib.llapis_residency_create(C.byref(c), 0)
        assert b"bad geometry" in lib.llapis_residency_last_error()
    assert not lib.llapis_residency_create(None, 0)
    # the handle-taking calls refuse a null runtime
    assert lib.llapis_residency_token_end(None, None) == -1
    assert lib.llapis_residency_publish_all(None, None) == -1
    assert lib.llapis_residency_refresh(None, 0, None) == -1
    assert lib.llapis_residency_set_mirrors(None, 0, None, None, None) == -1
    assert not lib.llapis_residency_policy(None)
    s = L.LlapisResidencyStats()
    lib.llapis_residency_get_stats(None, C.byref(s))
    assert s.tokens == 0
