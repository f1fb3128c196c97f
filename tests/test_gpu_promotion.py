"""GPU: the promotion path and the routing-counter loop.

* The island's batch transport (moert_cuda_dir_*): device, pinned and small
  pageable sources land byte for byte, large pageable ones are refused, marks
  complete in order, the pinned ring is reused behind its events, the gate
  orders a copy after the last MoE fire of a layer, publish_h2d lands.
* The promotion engine (llapis_xfer_*): jobs stay pending until flush,
  then every page group of the expert lands in its slot bit for bit (copy
  kernel, and hipMemcpyAsync from pinned memory).
* The loop a server runs: decode and prefill calls count their routing on the
  device; the policy pulls the counts at each decision (they must equal the
  counts of the ids the GPU returned), promotes asynchronously (FILLING), the
  engine copies the expert from the promotion source in HBM, the completion
  makes the slot READY and the mirrors are published.  Every call's output
  is checked against the oracle under the page table it ran with: a FILLING
  expert is served cold, a READY one hot from its new slot.
"""
import copy
import ctypes as C
import sys

import numpy as np
import pytest

import llapis_amd as la
from llapis_amd import _lib as L
from llapis_amd.policy import Policy
from helpers import FULL16, layer, rel_l2, tokens

pytestmark = pytest.mark.gpu


# Per call, the required relative L2 bar of a whole layer.  A one-token call
# sits near 1e-7 unless a last-bit difference in a gate_up output flips a
# q8_0 rounding of the down activation (then up to a few 1e-4 on that token,
# deterministic); an expert served in the wrong tier or with stale bytes costs
# 1e-2 or more.  The loops also bound the median call at 1e-6.
FLIP_BAR = 1e-3


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def torch_mod():
    import torch
    return torch


def u8(torch, a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def test_batch_transport(gpu):
    torch = torch_mod()
    lib = la.lib()
    say("transport: init, device / pinned / pageable sources")
    assert lib.moert_cuda_dir_init(0, 1, 0) == 1
    assert lib.moert_cuda_dir_init(0, 1, 0) == 1             # idempotent
    st0 = L.MoertCudaDirStats()
    lib.moert_cuda_dir_stats_get(C.byref(st0))
    rng = np.random.default_rng(5)
    n = 3_593_216
    src_h = rng.integers(0, 256, n, dtype=np.uint8)
    src_d = u8(torch, src_h, gpu)
    dst = torch.zeros(3 * n + 8192, dtype=torch.uint8, device=gpu)
    pin = torch.empty(n, dtype=torch.uint8, pin_memory=True)
    pin.copy_(torch.from_numpy(src_h[::-1].copy()))
    small = rng.integers(0, 256, 4096, dtype=np.uint8)
    small_orig = small.copy()
    big = rng.integers(0, 256, 8192, dtype=np.uint8)
    base = dst.data_ptr()
    assert lib.moert_cuda_dir_async(base, src_d.data_ptr(), n) == 1
    assert lib.moert_cuda_dir_async(base + n, pin.data_ptr(), n) == 1
    assert lib.moert_cuda_dir_async(base + 2 * n, small.ctypes.data, 4096) == 1
    assert lib.moert_cuda_dir_async(base + 2 * n + 4096, big.ctypes.data, 8192) == 0    # pageable > 4 KiB
    small[:] = 0                                              # staged: the caller may reuse it at once
    m0 = lib.moert_cuda_dir_mark()
    assert m0 >= 0
    assert lib.moert_cuda_dir_poll(1) == m0
    h = dst.cpu().numpy()
    assert np.array_equal(h[:n], src_h)
    assert np.array_equal(h[n:2 * n], src_h[::-1])
    assert np.array_equal(h[2 * n:2 * n + 4096], small_orig)
    assert not h[2 * n + 4096:].any()                         # the refused copy wrote nothing
    say("transport: 600 small pageable copies through the pinned ring")
    pages = rng.integers(0, 256, (600, 256), dtype=np.uint8)
    out = torch.zeros(600 * 256, dtype=torch.uint8, device=gpu)
    for i in range(600):
        assert lib.moert_cuda_dir_async(out.data_ptr() + 256 * i, pages[i].ctypes.data, 256) == 1
    m1 = lib.moert_cuda_dir_mark()
    assert m1 == m0 + 1
    while lib.moert_cuda_dir_poll(0) < m1:
        pass
    assert np.array_equal(out.cpu().numpy().reshape(600, 256), pages)
    st = L.MoertCudaDirStats()
    lib.moert_cuda_dir_stats_get(C.byref(st))
    assert st.async_copies - st0.async_copies == 603
    assert st.async_marks - st0.async_marks == 2
    assert st.bytes - st0.bytes == 2 * n + 4096 + 600 * 256
    assert st.sm_ring_copies - st0.sm_ring_copies == 601
    say("transport: publish_h2d")
    views = [np.arange(16, dtype=np.int32), np.full(4, 7, np.int32), np.array([2, 1, 0, 2], np.int32)]
    dev = [torch.zeros(v.size, dtype=torch.int32, device=gpu) for v in views]
    dsts = (C.c_void_p * 3)(*[d.data_ptr() for d in dev])
    srcs = (C.c_void_p * 3)(*[v.ctypes.data for v in views])
    sizes = (C.c_uint64 * 3)(*[v.nbytes for v in views])
    assert lib.moert_cuda_publish_h2d(3, dsts, srcs, sizes) == 1
    for d, v in zip(dev, views):
        assert np.array_equal(d.cpu().numpy(), v)


def test_transport_gate_orders_copy_after_last_fire(gpu):
    """Gate ops of moert_cuda_dir_gate: a wait for a target no fire reached
    times out on the host (2 s); after the layer's down fire the wait returns
    at once and the copy stream waits for that fire on the device."""
    torch = torch_mod()
    lib = la.lib()
    assert lib.moert_cuda_dir_init(0, 1, 0) == 1
    spec = FULL16
    lay = layer(spec, 61, [0, 3, 5], scales=True)
    dl = la.DeviceLayer(lay, gpu)
    assert lib.moert_cuda_dir_gate(0, 0) == 1                 # last MoE layer 0, one gate for the forward
    w0, t0 = lib.moert_cuda_dir_gate(4, 0), lib.moert_cuda_dir_gate(4, 1)
    target = lib.moert_cuda_dir_gate(1, 0)
    assert target >= 1
    say("gate: wait with no fire (times out)")
    assert lib.moert_cuda_dir_gate(2, target) == 1
    assert lib.moert_cuda_dir_gate(4, 1) == t0 + 1
    say("gate: fires of layer 0, then the wait returns and orders the copy")
    T = 2
    x = torch.from_numpy(tokens(3, T, spec.d_model)).to(gpu)
    ids, w, _ = dl.router(x)
    gu = dl.moe_dual(0, x, ids, il=0)
    act = la.geglu(gu.reshape(-1, 2 * spec.n_ff).contiguous(), spec.n_ff)
    dn = dl.moe_dual(1, act, ids, il=0)
    target = lib.moert_cuda_dir_gate(1, 0)
    assert lib.moert_cuda_dir_gate(2, target - 1) == 1       # the fire above reached it
    assert lib.moert_cuda_dir_gate(4, 1) == t0 + 1            # no new timeout
    src = torch.arange(1 << 20, dtype=torch.int32, device=gpu)
    dst = torch.zeros_like(src)
    assert lib.moert_cuda_dir_async(dst.data_ptr(), src.data_ptr(), src.numel() * 4) == 1
    m = lib.moert_cuda_dir_mark()
    assert lib.moert_cuda_dir_poll(1) == m
    assert torch.equal(dst, src)
    assert lib.moert_cuda_dir_gate(3, 0) == 1                 # open: every layer reaches the armed target
    assert lib.moert_cuda_dir_gate(4, 0) == w0 + 2
    torch.cuda.synchronize()
    assert dn.shape[-1] == spec.d_model


@pytest.mark.parametrize("copy_wgs,pinned", [(8, False), (0, False), (0, True)])
def test_xfer_copies_expert_pages(gpu, copy_wgs, pinned):
    torch = torch_mod()
    lib = la.lib()
    say(f"xfer copy_wgs={copy_wgs} pinned={pinned}")
    rng = np.random.default_rng(copy_wgs + 3 * pinned)
    NL, E, K = 2, 6, 3
    sizes = [2_230_272, 1_362_944, 4]          # Q4_K gate_up, Q5_0 down, a scale page
    src_h = [[rng.integers(0, 256, E * b, dtype=np.uint8) for b in sizes] for _ in range(NL)]
    if pinned:
        src = [[torch.from_numpy(a).pin_memory() for a in row] for row in src_h]
    else:
        src = [[u8(torch, a, gpu) for a in row] for row in src_h]
    slab = [[torch.zeros(K * b, dtype=torch.uint8, device=gpu) for b in sizes] for _ in range(NL)]
    x = lib.llapis_xfer_create(NL, E, K, copy_wgs)
    assert x
    try:
        for il in range(NL):
            for g, b in enumerate(sizes):
                assert lib.llapis_xfer_set_group(x, il, g, slab[il][g].data_ptr(), src[il][g].data_ptr(), b, b) == 0
        assert lib.llapis_xfer_set_group(x, 0, 0, slab[0][0].data_ptr(), src_h[0][0].ctypes.data, sizes[0],
                                         sizes[0]) == -1               # pageable source refused
        assert lib.llapis_xfer_submit(x, 0, E, 0) == -1
        jobs = [(0, 4, 1), (1, 2, 0), (0, 5, 2), (1, 0, 2), (0, 1, 0)]
        for il, e, s in jobs:
            assert lib.llapis_xfer_submit(x, il, e, s) == 0
        assert lib.llapis_xfer_in_flight(x) == len(jobs)
        torch.cuda.synchronize()
        assert not any(t.any().item() for row in slab for t in row)    # pending: nothing issued
        stream = torch.cuda.current_stream().cuda_stream
        assert lib.llapis_xfer_flush(x, stream) == 0
        assert lib.llapis_xfer_wait_idle(x, stream) == 0
        done = (L.LlapisXferDone * 8)()
        n = lib.llapis_xfer_take_done(x, done, 8)
        assert n == len(jobs)
        assert [(d.il, d.e, d.slot, d.ok) for d in done[:n]] == [j + (1,) for j in jobs]
        assert lib.llapis_xfer_in_flight(x) == 0
        expect = [[np.zeros(K * b, np.uint8) for b in sizes] for _ in range(NL)]
        for il, e, s in jobs:
            for g, b in enumerate(sizes):
                expect[il][g][s * b:(s + 1) * b] = src_h[il][g][e * b:(e + 1) * b]
        for il in range(NL):
            for g in range(len(sizes)):
                assert np.array_equal(slab[il][g].cpu().numpy(), expect[il][g]), (il, g)
        st = L.LlapisXferStats()
        lib.llapis_xfer_get_stats(x, C.byref(st))
        assert (st.submitted, st.completed, st.failed) == (5, 5, 0)
        assert st.bytes == 5 * sum(sizes)
    finally:
        lib.llapis_xfer_free(x)


def _view_layer(lay_all, src_s, es, se, ss):
    """The layer as the kernels see it under a page table: READY slots hold
    their expert's promotion-source bytes, other slots are never read."""
    sp = lay_all.spec
    K = len(se)
    gb, db = sp.gu_bytes(sp.hot_gu_type), sp.dn_bytes(sp.hot_dn_type)
    v = copy.copy(lay_all)
    v.residency = la.Residency(sp.n_expert, K, es.copy(), se.copy(), ss.copy())
    v.hot_gu = np.zeros(K * gb, np.uint8)
    v.hot_dn = np.zeros(K * db, np.uint8)
    v.s_hot = np.ones(K, np.float32)
    for s in range(K):
        e = int(se[s])
        if e >= 0 and ss[s] == la.SLOT_READY:
            v.hot_gu[s * gb:(s + 1) * gb] = lay_all.hot_gu[e * gb:(e + 1) * gb]
            v.hot_dn[s * db:(s + 1) * db] = lay_all.hot_dn[e * db:(e + 1) * db]
            v.s_hot[s] = src_s[e]
    return v


def test_promotion_loop_with_device_counts(gpu, oracle):
    torch = torch_mod()
    lib = la.lib()
    spec = FULL16
    E, K, top_k = spec.n_expert, 4, spec.top_k
    # the promotion source: every expert in the hot formats (slot e = expert e)
    lay_all = layer(spec, 71, list(range(E)), scales=True)
    src_s = lay_all.s_hot.copy()
    gb, db = spec.gu_bytes(spec.hot_gu_type), spec.dn_bytes(spec.hot_dn_type)
    src_gu, src_dn, src_sc = u8(torch, lay_all.hot_gu, gpu), u8(torch, lay_all.hot_dn, gpu), u8(torch, src_s, gpu)
    # the live layer: K slots seeded with experts 0..3
    live = copy.copy(lay_all)
    live.residency = la.Residency.from_hot(E, list(range(K)))
    live.hot_gu = lay_all.hot_gu[:K * gb].copy()
    live.hot_dn = lay_all.hot_dn[:K * db].copy()
    live.s_hot = src_s[:K].copy()
    live.router_b = np.zeros(E, np.float32)
    dl = la.DeviceLayer(live, gpu)
    dl.route_counts = torch.zeros(E, dtype=torch.int32, device=gpu)
    dl.route_hits = torch.zeros(2, dtype=torch.int32, device=gpu)
    x_eng = lib.llapis_xfer_create(1, E, K, 8)
    assert x_eng
    for g, (slab, src, b) in enumerate(((dl.hot_gu, src_gu, gb), (dl.hot_dn, src_dn, db), (dl.s_hot, src_sc, 4))):
        assert lib.llapis_xfer_set_group(x_eng, 0, g, slab.data_ptr(), src.data_ptr(), b, b) == 0

    expect = {"counts": np.zeros(E, np.int64), "hot": 0, "cold": 0}
    errs = []
    log = {"fetches": 0, "submitted": 0, "completed": 0, "filling_served_cold": 0, "promoted_used_hot": 0}
    pol = None

    def fetch():
        c = dl.route_counts.cpu().numpy()
        hc = dl.route_hits.cpu().numpy()
        assert np.array_equal(c, expect["counts"]), (c, expect["counts"])
        assert (int(hc[0]), int(hc[1])) == (expect["hot"], expect["cold"])
        pol.add_counts(0, c, int(hc[0]), int(hc[1]))
        dl.route_counts.zero_()
        dl.route_hits.zero_()
        expect["counts"][:] = 0
        expect["hot"] = expect["cold"] = 0
        log["fetches"] += 1

    def stream_expert(il, e, slot):
        assert lib.llapis_xfer_submit(x_eng, il, e, slot) == 0
        log["submitted"] += 1
        return 2

    def publish(il):
        v = pol.views(il)
        dev = [dl.exp_slot, dl.slot_exp, dl.slot_state]
        host = [v["exp_slot"], v["slot_exp"], v["slot_state"]]
        dsts = (C.c_void_p * 3)(*[d.data_ptr() for d in dev])
        srcs = (C.c_void_p * 3)(*[h.ctypes.data for h in host])
        sizes = (C.c_uint64 * 3)(*[h.nbytes for h in host])
        assert lib.moert_cuda_publish_h2d(3, dsts, srcs, sizes) == 1

    pol = Policy(1, E, K, stream_expert=stream_expert, publish_layer=publish, fetch_external=fetch,
                 cost_horizon=64, cost_reuse=2.0, cost_per_token=2)
    pol.set_external(True)
    for e in range(K):
        assert pol.seed(0, e, e) == 1
    publish(0)
    stream = torch.cuda.current_stream().cuda_stream
    done = (L.LlapisXferDone * 64)()
    try:
        # phase A favours experts 8..15, phase B experts 0..7; T = 1 decode
        # mostly, 4-token steps, a generic-path step and a prompt chunk on the
        # prefill path (no decision: its counts are pulled at the turn end)
        plan = [(1, "A")] * 8 + [(4, "A")] + [(1, "B"), (4, "B")] + [(1, "B")] * 14 + [(2, "Bg"), (40, "Bp")]
        for step, (T, phase) in enumerate(plan):
            if step % 2 == 0:
                n = lib.llapis_xfer_take_done(x_eng, done, 64)
                touched = False
                for d in done[:n]:
                    assert d.ok == 1
                    if pol.complete(d.il, d.slot, d.e) == 1:
                        touched = True
                        log["completed"] += 1
                if touched:
                    publish(0)
            bias = np.zeros(E, np.float32)
            bias[8:] = 3.0 if phase == "A" else -3.0
            dl.router_b.copy_(torch.from_numpy(bias))
            live.router_b = bias
            v = pol.views(0)
            res = la.Residency(E, K, v["exp_slot"], v["slot_exp"], v["slot_state"])
            say(f"step {step} T={T} phase {phase} slots {list(v['slot_exp'])} states {list(v['slot_state'])}")
            x = tokens(500 + step, T, spec.d_model)
            if phase == "Bg":
                lib.llapis_set_tuning(0, 0)
            try:
                out, ids, w = dl.forward(torch.from_numpy(x).to(gpu))
                torch.cuda.synchronize()
            finally:
                lib.llapis_set_tuning(0, 1)
            ids_h, w_h = ids.cpu().numpy(), w.cpu().numpy()
            vl = _view_layer(lay_all, src_s, v["exp_slot"], v["slot_exp"], v["slot_state"])
            vl.router_b = bias
            ids_o, _, _ = oracle.router(x, vl.router_w, bias, top_k)
            assert np.array_equal(ids_h, ids_o)
            out_o, _ = oracle.moe_experts(vl, x, ids_h, w_h, la.ACT_CPU, la.GELU_TABLE)
            err = rel_l2(out.cpu().numpy(), out_o)
            errs.append(float(err))
            assert err <= FLIP_BAR, (step, err)
            for e in ids_h.ravel():
                s = int(v["exp_slot"][e])
                if s >= 0 and v["slot_state"][s] == la.SLOT_FILLING:
                    log["filling_served_cold"] += 1
                if res.is_hot(int(e)) and s >= 0 and int(e) >= K:
                    log["promoted_used_hot"] += 1
            expect["counts"] += np.bincount(ids_h.ravel(), minlength=E)
            hot = sum(res.is_hot(int(e)) for e in ids_h.ravel())
            expect["hot"] += hot
            expect["cold"] += ids_h.size - hot
            if phase == "Bp":
                pol.prompt_tokens(T)
            else:
                pol.token_end()                   # fetch -> decide -> submit / publish FILLING
            assert lib.llapis_xfer_flush(x_eng, stream) == 0
        assert np.median(errs) <= 1e-6, errs
        pol.refresh(L.REFRESH_TURN_END)
        # one pull per decision: each visible token and the turn end (the
        # prompt chunk's counts wait for the turn end)
        assert log["fetches"] == len(plan)
        assert lib.llapis_xfer_wait_idle(x_eng, stream) == 0
        n = lib.llapis_xfer_take_done(x_eng, done, 64)
        for d in done[:n]:
            if pol.complete(d.il, d.slot, d.e) == 1:
                log["completed"] += 1
        publish(0)
        torch.cuda.synchronize()
        # every READY slot holds its expert's bytes, bit for bit
        v = pol.views(0)
        hg, hd, hs = dl.hot_gu.cpu().numpy(), dl.hot_dn.cpu().numpy(), dl.s_hot.cpu().numpy()
        for s in range(K):
            e = int(v["slot_exp"][s])
            assert v["slot_state"][s] == la.SLOT_READY and e >= 0
            assert np.array_equal(hg[s * gb:(s + 1) * gb], lay_all.hot_gu[e * gb:(e + 1) * gb])
            assert np.array_equal(hd[s * db:(s + 1) * db], lay_all.hot_dn[e * db:(e + 1) * db])
            assert hs[s] == src_s[e]
        st = pol.stats()
        say(f"loop: {log}; policy promotions {st['promotions']} demotions {st['demotions']} "
            f"hit rate {pol.hit_rate():.3f}")
        assert log["submitted"] >= 6 and log["completed"] == log["submitted"] == st["fills_completed"]
        assert st["demotions"] >= 4
        assert log["filling_served_cold"] > 0 and log["promoted_used_hot"] > 0
        assert set(int(e) for e in v["slot_exp"]) <= set(range(8))      # phase B's experts hold the slots
    finally:
        lib.llapis_xfer_free(x_eng)
        pol.close()


@pytest.mark.parametrize("kpl", [None, (4, 2)])
def test_native_residency_loop_two_layers(gpu, oracle, kpl):
    """The same loop run by the native runtime (llapis_residency_*) over two
    layers whose routing drifts in opposite directions: every call's output
    matches the oracle under the page table published at the previous token
    end, the device mirrors equal the policy's after each token end, the
    counters the runtime pulled add up to the pairs the GPU routed, and each
    layer ends holding its own phase's experts, byte for byte.  With
    per-layer capacities each layer's mirrors are published at its own K
    from the runtime's staging (sized for the largest)."""
    from llapis_amd.policy import ResidencyLoop
    torch = torch_mod()
    lib = la.lib()
    spec = FULL16
    E, K, top_k, NL = spec.n_expert, 4, spec.top_k, 2
    gb, db = spec.gu_bytes(spec.hot_gu_type), spec.dn_bytes(spec.hot_dn_type)
    rl = ResidencyLoop(NL, E, K, copy_wgs=8, k_per_layer=kpl, cost_horizon=64, cost_reuse=2.0, cost_per_token=2)
    pol = rl.policy
    layers = []
    try:
        for il in range(NL):
            K = kpl[il] if kpl else 4
            assert pol.layer_k(il) == K
            lay_all = layer(spec, 81 + il, list(range(E)), scales=True)
            src_s = lay_all.s_hot.copy()
            srcs = [u8(torch, lay_all.hot_gu, gpu), u8(torch, lay_all.hot_dn, gpu), u8(torch, src_s, gpu)]
            live = copy.copy(lay_all)
            live.residency = la.Residency.from_hot(E, list(range(K)))
            live.hot_gu = lay_all.hot_gu[:K * gb].copy()
            live.hot_dn = lay_all.hot_dn[:K * db].copy()
            live.s_hot = src_s[:K].copy()
            live.router_b = np.zeros(E, np.float32)
            dl = la.DeviceLayer(live, gpu)
            dl.route_counts, dl.route_hits = rl.counters(il)
            for g, (slab, src, b) in enumerate(((dl.hot_gu, srcs[0], gb), (dl.hot_dn, srcs[1], db),
                                                (dl.s_hot, srcs[2], 4))):
                assert lib.llapis_xfer_set_group(rl.xfer, il, g, slab.data_ptr(), src.data_ptr(), b, b) == 0
            rl.set_mirrors(il, dl.exp_slot.data_ptr(), dl.slot_exp.data_ptr(), dl.slot_state.data_ptr())
            for e in range(K):
                assert pol.seed(il, e, e) == 1
            layers.append((lay_all, src_s, srcs, dl))
        stream = torch.cuda.current_stream().cuda_stream
        rl.publish_all(stream)
        routed = {"hot": 0, "cold": 0}
        errs = []
        # a 40-token prompt chunk (prefill path) near the end: no decision, its
        # routing waits in the counters for the next token end
        plan = [(1, "A")] * 10 + [(4, "A")] + [(1, "B")] * 16 + [(4, "B")] + [(40, "Bp")] + [(1, "B")] * 4
        for step, (T, phase) in enumerate(plan):
            for il, (lay_all, src_s, _, dl) in enumerate(layers):
                v = pol.views(il)
                assert np.array_equal(dl.exp_slot.cpu().numpy(), v["exp_slot"])
                assert np.array_equal(dl.slot_exp.cpu().numpy(), v["slot_exp"])
                assert np.array_equal(dl.slot_state.cpu().numpy(), v["slot_state"])
                bias = np.zeros(E, np.float32)
                up = (phase == "A") == (il == 0)
                bias[8:] = 3.0 if up else -3.0
                dl.router_b.copy_(torch.from_numpy(bias))
                x = tokens(900 + 10 * step + il, T, spec.d_model)
                out, ids, w = dl.forward(torch.from_numpy(x).to(gpu))
                ids_h, w_h = ids.cpu().numpy(), w.cpu().numpy()
                vl = _view_layer(lay_all, src_s, v["exp_slot"], v["slot_exp"], v["slot_state"])
                vl.router_b = bias
                ids_o, _, _ = oracle.router(x, vl.router_w, bias, top_k)
                assert np.array_equal(ids_h, ids_o)
                out_o, _ = oracle.moe_experts(vl, x, ids_h, w_h, la.ACT_CPU, la.GELU_TABLE)
                err = rel_l2(out.cpu().numpy(), out_o)
                errs.append(float(err))
                assert err <= FLIP_BAR, (step, il, err)
                hot = sum(vl.residency.is_hot(int(e)) for e in ids_h.ravel())
                routed["hot"] += hot
                routed["cold"] += ids_h.size - hot
            if phase == "Bp":
                pol.prompt_tokens(T)
            else:
                rl.token_end(stream)
            say(f"step {step} T={T} {phase}: " + "; ".join(
                f"L{il} slots {list(pol.views(il)['slot_exp'])} states {list(pol.views(il)['slot_state'])}"
                for il in range(NL)))
        rl.refresh(L.REFRESH_TURN_END, stream)             # drains the counters too
        torch.cuda.synchronize()
        assert np.median(errs) <= 1e-6, errs
        st = rl.stats()
        say(f"runtime {st}; policy {pol.stats()}")
        n_visible = sum(ph != "Bp" for _, ph in plan)
        assert st["tokens"] == n_visible and st["fetches"] == n_visible + 1
        assert (st["hot_pairs"], st["cold_pairs"]) == (routed["hot"], routed["cold"])
        assert st["submitted"] >= 8 and st["completed"] >= 4
        # drain: the last copies land, one more token end makes them READY
        assert lib.llapis_xfer_wait_idle(rl.xfer, stream) == 0
        rl.token_end(stream)
        assert lib.llapis_xfer_wait_idle(rl.xfer, stream) == 0
        torch.cuda.synchronize()
        for il, (lay_all, src_s, _, dl) in enumerate(layers):
            v = pol.views(il)
            assert np.array_equal(dl.slot_state.cpu().numpy(), v["slot_state"])
            hg, hd, hs = dl.hot_gu.cpu().numpy(), dl.hot_dn.cpu().numpy(), dl.s_hot.cpu().numpy()
            ready = [s for s in range(pol.layer_k(il)) if v["slot_state"][s] == la.SLOT_READY]
            assert len(ready) >= 2
            for s in ready:
                e = int(v["slot_exp"][s])
                assert np.array_equal(hg[s * gb:(s + 1) * gb], lay_all.hot_gu[e * gb:(e + 1) * gb])
                assert np.array_equal(hd[s * db:(s + 1) * db], lay_all.hot_dn[e * db:(e + 1) * db])
                assert hs[s] == src_s[e]
            held = {int(v["slot_exp"][s]) for s in ready}
            assert held <= (set(range(8)) if il == 0 else set(range(8, 16))), (il, held)
    finally:
        rl.close()


def test_native_residency_refuses_growth_past_its_staging(gpu):
    """A re-fit that grows a layer above the capacity the runtime was created
    for: the publication that follows a resize fails with an error (nothing
    is written past the staging), and shrinking back makes it work again."""
    from llapis_amd.policy import ResidencyLoop
    torch = torch_mod()
    E, K = 16, 2
    rl = ResidencyLoop(1, E, K)
    try:
        mir = [torch.full((n,), -1, dtype=torch.int32, device=gpu) for n in (E, 2 * K, 2 * K)]
        rl.set_mirrors(0, *[m.data_ptr() for m in mir])
        stream = torch.cuda.current_stream().cuda_stream
        rl.token_end(stream)
        assert rl.policy.resize(K + 1) == 1 and rl.policy.layer_k(0) == K + 1
        with pytest.raises(RuntimeError, match="capacity above"):
            rl.publish_all(stream)
        assert rl.policy.resize(K) == 1
        rl.publish_all(stream)
        rl.token_end(stream)
        torch.cuda.synchronize()
        assert rl.stats()["fetches"] == 2
        assert torch.equal(mir[0].cpu(), torch.full((E,), -1, dtype=torch.int32))   # nothing resident
    finally:
        rl.close()


def test_q4stream_prefill_reads_the_promotion_source(gpu, oracle):
    """q4stream (every expert of a prefill chunk at the hot precision) on a
    view of a dual layer whose hot pool is the promotion source: the outputs
    equal the oracle's all-hot layer, the view reads the source in place, and
    the dual layer itself still serves its non-resident experts cold."""
    torch = torch_mod()
    spec = FULL16
    E, K = spec.n_expert, 4
    gb, db = spec.gu_bytes(spec.hot_gu_type), spec.dn_bytes(spec.hot_dn_type)
    lay_all = layer(spec, 91, list(range(E)), scales=True)       # every expert in the hot formats
    src_s = lay_all.s_hot.copy()
    src_gu, src_dn = u8(torch, lay_all.hot_gu, gpu), u8(torch, lay_all.hot_dn, gpu)
    src_sc = torch.from_numpy(src_s).to(gpu)
    live = copy.copy(lay_all)
    live.residency = la.Residency.from_hot(E, list(range(K)))
    live.hot_gu, live.hot_dn, live.s_hot = lay_all.hot_gu[:K * gb].copy(), lay_all.hot_dn[:K * db].copy(), src_s[:K].copy()
    dl = la.DeviceLayer(live, gpu)
    q = dl.q4stream(src_gu, src_dn, src_sc)
    assert q.hot_gu.data_ptr() == src_gu.data_ptr() and q.router_w.data_ptr() == dl.router_w.data_ptr()
    with pytest.raises(ValueError):
        dl.q4stream(src_gu[:gb], src_dn, src_sc)
    for T in (40, 130):
        say(f"q4stream prefill T={T}")
        x = tokens(1200 + T, T, spec.d_model)
        out, ids, w = q.forward(torch.from_numpy(x).to(gpu))
        ids_h, w_h = ids.cpu().numpy(), w.cpu().numpy()
        ids_o, _, _ = oracle.router(x, lay_all.router_w, lay_all.router_b, spec.top_k)
        assert np.array_equal(ids_h, ids_o)
        out_o, _ = oracle.moe_experts(lay_all, x, ids_h, w_h, la.ACT_CPU, la.GELU_TABLE)
        err = rel_l2(out.cpu().numpy(), out_o)
        assert err <= 5e-4, (T, err)
        out_d = dl.forward(torch.from_numpy(x).to(gpu))[0].cpu().numpy()
        assert rel_l2(out_d, out_o) > 1e-2          # the dual layer serves experts >= K cold


def test_xfer_large_flush_split_into_launches(gpu):
    """A flush of 40 jobs x 3 pages (two copy launches), pages that are not
    a multiple of the copy chunk or of 16 bytes, and completions handed out a
    few at a time."""
    torch = torch_mod()
    lib = la.lib()
    rng = np.random.default_rng(11)
    E, K = 50, 40
    sizes = [200_000, 1000, 4]
    src_h = [rng.integers(0, 256, E * b, dtype=np.uint8) for b in sizes]
    src = [u8(torch, a, gpu) for a in src_h]
    slab = [torch.zeros(K * b, dtype=torch.uint8, device=gpu) for b in sizes]
    x = lib.llapis_xfer_create(1, E, K, 16)
    assert x
    try:
        for g, b in enumerate(sizes):
            assert lib.llapis_xfer_set_group(x, 0, g, slab[g].data_ptr(), src[g].data_ptr(), b, b) == 0
        jobs = [(0, int(e), s) for s, e in enumerate(rng.permutation(E)[:K])]
        for j in jobs:
            assert lib.llapis_xfer_submit(x, *j) == 0
        stream = torch.cuda.current_stream().cuda_stream
        assert lib.llapis_xfer_wait_idle(x, stream) == 0
        got = []
        done = (L.LlapisXferDone * 3)()
        while True:
            n = lib.llapis_xfer_take_done(x, done, 3)
            if n == 0:
                break
            got += [(d.il, d.e, d.slot, d.ok) for d in done[:n]]
        assert got == [j + (1,) for j in jobs]
        assert lib.llapis_xfer_in_flight(x) == 0
        for g, b in enumerate(sizes):
            h = slab[g].cpu().numpy()
            for il, e, s in jobs:
                assert np.array_equal(h[s * b:(s + 1) * b], src_h[g][e * b:(e + 1) * b]), (g, e, s)
    finally:
        lib.llapis_xfer_free(x)


def _rebuild_at_k(torch, lib, gpu, pol, lay_all, src, K_new):
    """slab_rebuild_at_k for one layer: resize the page table, a slab of the
    new size, every survivor re-streamed into its new slot by the engine,
    the mirrors published with the new layer."""
    spec = lay_all.spec
    E = spec.n_expert
    gb, db = spec.gu_bytes(spec.hot_gu_type), spec.dn_bytes(spec.hot_dn_type)
    assert pol.resize(K_new) == 1
    v = pol.views(0)
    live = copy.copy(lay_all)
    live.residency = la.Residency(E, K_new, v["exp_slot"].copy(), v["slot_exp"].copy(), v["slot_state"].copy())
    live.hot_gu = np.zeros(K_new * gb, np.uint8)          # the new slab: nothing in it yet
    live.hot_dn = np.zeros(K_new * db, np.uint8)
    live.s_hot = np.zeros(K_new, np.float32)
    dl = la.DeviceLayer(live, gpu)
    x = lib.llapis_xfer_create(1, E, K_new, 32)
    assert x
    try:
        for g, (slab, s, b) in enumerate(((dl.hot_gu, src[0], gb), (dl.hot_dn, src[1], db), (dl.s_hot, src[2], 4))):
            assert lib.llapis_xfer_set_group(x, 0, g, slab.data_ptr(), s.data_ptr(), b, b) == 0
        n = 0
        for s_, e in enumerate(v["slot_exp"]):
            if e >= 0:
                assert lib.llapis_xfer_submit(x, 0, int(e), s_) == 0
                n += 1
        assert lib.llapis_xfer_wait_idle(x, torch.cuda.current_stream().cuda_stream) == 0
        done = (L.LlapisXferDone * 256)()
        assert lib.llapis_xfer_take_done(x, done, 256) == n
        assert all(d.ok for d in done[:n])
    finally:
        lib.llapis_xfer_free(x)
    return dl, v


def test_refit_k_restreams_survivors(gpu, oracle):
    """The K re-fit (moe_dual_init.cpp:565-630, 684-790) on one layer: the
    measured device memory decides K (on 288 GB: every expert); under set
    budgets the layer shrinks and grows again.  The policy keeps its best
    residents compacted into slots 0..K-1, the engine re-streams them into a
    slab of the new size, and the layer's output equals the oracle's under
    the new page table."""
    torch = torch_mod()
    lib = la.lib()
    spec = FULL16
    E, K0, top_k = spec.n_expert, 8, spec.top_k
    lay_all = layer(spec, 81, list(range(E)), scales=True)
    src_s = lay_all.s_hot.copy()
    src = (u8(torch, lay_all.hot_gu, gpu), u8(torch, lay_all.hot_dn, gpu), u8(torch, src_s, gpu))
    gb, db = spec.gu_bytes(spec.hot_gu_type), spec.dn_bytes(spec.hot_dn_type)
    pol = Policy(1, E, K0, stream_expert=lambda il, e, s: 1, publish_layer=lambda il: None, cost_reuse=1000.0)
    for e in range(K0):
        assert pol.seed(0, e, e) == 1
    # a routing history that ranks the residents 5 > 2 > 7 > 0 > the rest
    ids = [5] * 6 + [2] * 5 + [7] * 4 + [0] * 3 + [11] * 9
    pol.observe(0, np.array(ids, np.int32), len(ids), 1)
    pol.token_end()
    free, total = C.c_longlong(), C.c_longlong()
    assert lib.llapis_device_memory_mib(C.byref(free), C.byref(total)) == 0
    say(f"refit: device memory free {free.value} MiB of {total.value} MiB")
    per_k = max(1, (gb + db + 4) >> 20)
    plan = [("measured", dict(free_mib=free.value, slab_mib_now=K0 * per_k)),
            ("shrink", dict(free_mib=per_k, slab_mib_now=2 * per_k)),     # pool 3 slots, 0 kept free
            ("grow", dict(free_mib=6 * per_k, slab_mib_now=3 * per_k))]
    k_cur = K0
    rank = [5, 2, 7, 0]
    for name, kw in plan:
        inp = L.LlapisKfitInputs(kw["free_mib"], kw["slab_mib_now"], -1, per_k, 0 if name != "measured" else 1024,
                                 k_cur, 1, E, 0)
        d = L.LlapisKfitDecision()
        lib.llapis_kfit(C.byref(inp), C.byref(d))
        say(f"refit {name}: K {k_cur} -> {d.k} (rebuild {d.rebuild}, pool {d.pool_mib} MiB)")
        if name == "measured":
            assert d.k == E and d.rebuild                 # 288 GB: every expert fits
        elif name == "shrink":
            assert d.k == 3 and d.rebuild and not d.floor_capped
        else:
            assert d.k == 9 and d.rebuild
        dl, v = _rebuild_at_k(torch, lib, gpu, pol, lay_all, src, d.k)
        resid = [int(e) for e in v["slot_exp"] if e >= 0]
        if name == "shrink":
            assert resid == rank[:3]                       # the best three, compacted in rank order
        if name == "grow":
            assert resid == rank[:3] and list(v["slot_state"][:3]) == [la.SLOT_READY] * 3
        x = tokens(900 + d.k, 4, spec.d_model)
        out, ids_d, w = dl.forward(torch.from_numpy(x).to(gpu))
        torch.cuda.synchronize()
        ids_h, w_h = ids_d.cpu().numpy(), w.cpu().numpy()
        vl = _view_layer(lay_all, src_s, v["exp_slot"], v["slot_exp"], v["slot_state"])
        out_o, _ = oracle.moe_experts(vl, x, ids_h, w_h, la.ACT_CPU, la.GELU_TABLE)
        err = rel_l2(out.cpu().numpy(), out_o)
        say(f"  K={d.k} residents {resid}: rel_l2 vs oracle {err:.2e}")
        assert err <= 1e-4
        # the slab holds each survivor's bytes in its new slot
        hg = dl.hot_gu.cpu().numpy()
        for s_, e in enumerate(v["slot_exp"]):
            if e >= 0:
                assert np.array_equal(hg[s_ * gb:(s_ + 1) * gb], lay_all.hot_gu[e * gb:(e + 1) * gb])
        k_cur = d.k
    pol.close()
