#!/usr/bin/env python3
"""MoE-layer decode benchmark of the MI355X dual-precision expert FFN.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Workload (the headline: decode on the mixed-precision weights): one MoE FFN
layer, d_model 2816, 128 experts, top-8, n_ff 704, GeGLU; K=57 experts hot
(Q4_K gate_up, Q5_0 down), chosen from a Zipf(1.1) routing prior, the other 71
cold (IQ2_S gate_up, IQ4_NL down); the router bias puts ~85 % of the top-8
picks on the hot set; 4 tokens per step (a depth-3 speculative verify).  A
step is router -> top-8 -> gate_up -> GEGLU -> down -> combine for those
tokens, launched as a captured HIP graph.  Inputs are resident in HBM before
timing starts.  Each step reads a different layer replica (and tokens) so the
bytes touched per cycle exceed the 256 MB MALL: the HBM rate is HBM, not cache.

Also reported (extra): all-IQ2_S and all-Q4_K decode of one token, the
promotion path (expert copies into hot slots, alone and beside the decode),
and the dual-precision 512-token prefill (grouped MFMA GEMMs; int8
TOP/s = 2 x 11 894 784 ops per routed pair, against the int8 peak and against
the attainable min(peak, arithmetic intensity x HBM)), each with its own
roofline; the dominant kernel's duration is timed live with HIP events on the
stream it runs on; the reference's ggml CPU path (oracle/_ref, built from the
reference's sources) is timed on a bounded sample of the same workload on the
host cores.
"""
import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0                  # MI355X HBM3E, GB/s
OPS_PER_PAIR = 2 * (2816 * 1408 + 704 * 2816)   # int8 multiply-adds x 2 per routed pair (gate_up + down)
INT8_PEAK_TOPS = 5000.0                # MI355X dense int8 MFMA, TOP/s
HEAD_TOKENS = {"dual": 4, "iq2s": 1, "q4k": 1, "prefill": 512, "prefill_q81": 512, "q4stream": 512}
HEAD_FORMATS = {
    "dual": "K=57 hot: Q4_K gate_up / Q5_0 down; 71 cold: IQ2_S gate_up / IQ4_NL down; ~85 % of picks hot",
    "iq2s": "IQ2_S gate_up / IQ4_NL down", "q4k": "Q4_K gate_up / Q5_0 down",
    "prefill": "dual K=57, q8_K/q8_0 activations", "prefill_q81": "dual K=57, q8_1 activations",
    "q4stream": "every expert Q4_K gate_up / Q5_0 down"}
DOWN_BY_GROUP = True                   # 2-4 token decode: down per expert group + combine (tuning key 4)
METRIC = "MoE-layer decode tok/s + HBM TB/s (% peak); 512-tok prefill int8 TOPS (% peak)"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def layer_bytes(spec, n_hot, n_cold, T):
    """Algorithmic HBM bytes of one layer step: each distinct routed expert's
    gate_up + down slabs once (n_hot / n_cold distinct experts per tier), the
    fp32 router once, the activations in and out."""
    hot = spec.gu_bytes(spec.hot_gu_type) + spec.dn_bytes(spec.hot_dn_type)
    cold = spec.gu_bytes(spec.cold_gu_type) + spec.dn_bytes(spec.cold_dn_type)
    return n_hot * hot + n_cold * cold + spec.n_expert * spec.d_model * 4 + 2 * T * spec.d_model * 4


class Workload:
    """R device replicas of one layer, prebuilt descriptors and buffers."""

    def __init__(self, la, torch, host_layer, R, T, n_tok, seed, dev, act_mode, gelu_mode, counts=False):
        self.la, self.torch, self.T, self.R = la, torch, T, R
        self.spec = host_layer.spec
        base = la.DeviceLayer(host_layer, dev, act_mode, gelu_mode)
        if counts:   # device routing counters on every call (the policy's observation)
            base.route_counts = torch.zeros(host_layer.spec.n_expert, dtype=torch.int32, device=dev)
            base.route_hits = torch.zeros(2, dtype=torch.int32, device=dev)
        self.layers = [base]
        for _ in range(R - 1):
            d = la.DeviceLayer.__new__(la.DeviceLayer)
            d.__dict__.update(base.__dict__)
            # every tensor a step reads is the replica's own (the router too:
            # its 1.44 MB is counted in the step's bytes)
            for k in ("hot_gu", "hot_dn", "cold_gu", "cold_dn", "router_w", "router_b"):
                if getattr(base, k) is not None:
                    setattr(d, k, getattr(base, k).clone())
            d._ws = None
            self.layers.append(d)
        sp = self.spec
        xs = la.synth_normal(seed, n_tok * T * sp.d_model).reshape(n_tok, T, sp.d_model)
        self.x = torch.from_numpy(xs).to(dev)
        self.out = torch.empty(T, sp.d_model, device=dev)
        self.ids = torch.empty(T, sp.top_k, dtype=torch.int32, device=dev)
        self.w = torch.empty(T, sp.top_k, device=dev)
        self.descs = [l.desc() for l in self.layers]
        need = int(la.lib().llapis_moe_ffn_workspace_size(C.byref(self.descs[0]), T))
        self.ws = torch.zeros(need, dtype=torch.uint8, device=dev)
        self.n_tok = n_tok
        self.fn = la.lib().llapis_moe_ffn

    def step(self, i, stream):
        d = self.descs[i % self.R]
        rc = self.fn(C.byref(d), self.x[i % self.n_tok].data_ptr(), None, self.T, self.out.data_ptr(), self.ids.data_ptr(),
                     self.w.data_ptr(), self.ws.data_ptr(), self.ws.numel(), stream)
        if rc != 0:
            raise RuntimeError(self.la.lib().llapis_last_error().decode())

    def routing(self):
        """Mean over the token sets of (distinct hot experts, distinct cold
        experts, routed pairs) per step."""
        torch = self.torch
        s = torch.cuda.current_stream().cuda_stream
        res = self.layers[0].layer.residency
        acc = np.zeros(3)
        for i in range(self.n_tok):
            self.step(i, s)
            torch.cuda.synchronize()
            ids = set(self.ids.cpu().numpy().ravel().tolist())
            hot = sum(1 for e in ids if res.is_hot(int(e)))
            acc += (hot, len(ids) - hot, self.T * self.spec.top_k)
        return acc / self.n_tok


class IslandWorkload(Workload):
    """The same replicas driven through the reference's operator boundary:
    llapis_router_topk, the gate_up fire of the dual op (one kernel, or
    moert_ffn_moe's partition, gather, hot and cold mul_mat_id, scatter),
    GEGLU, the down fire, and the weighted sum over top_k (ggml's mul + adds:
    llapis_moe_combine) -- the per-fire island a relinked ggml graph runs."""

    def step(self, i, stream):
        torch = self.torch
        dl = self.layers[i % self.R]
        sp = self.spec
        x = self.x[i % self.n_tok]
        ids, w, _ = dl.router(x)
        gu = dl.moe_dual(0, x, ids)
        act = self.la.geglu(gu.reshape(-1, 2 * sp.n_ff), sp.n_ff, dl.gelu_mode)
        dn = dl.moe_dual(1, act, ids)
        if self.la.lib().llapis_moe_combine(dn.data_ptr(), w.data_ptr(), self.T, sp.top_k, sp.d_model,
                                            self.out.data_ptr(), stream) != 0:
            raise RuntimeError(self.la.lib().llapis_last_error())


def run_island(la, torch, name, host_layer, T, steps, warmup, dev, layer_res):
    """Tokens per second of the island path beside llapis_moe_ffn's on the
    same workload (layer_res: run_config's result for it)."""
    sp = host_layer.spec
    R = layer_res["replicas"]
    wl = IslandWorkload(la, torch, host_layer, R, T, 16, 1234, dev, 0, 0)
    ms_graph, timed = time_graph(wl, steps, warmup)
    ms_eager = time_eager(wl, min(steps, 200), min(warmup, 20))
    res = {"tok_per_s": T * 1e3 / ms_graph, "ms_per_step": ms_graph, "ms_per_step_eager": ms_eager,
           "steps_timed": timed, "replicas": R,
           "hbm_gbs_step": layer_res["algo_bytes_step"] / (ms_graph * 1e-3) / 1e9,
           "vs_moe_ffn": layer_res["ms_per_step"] / ms_graph}
    log(f"[island {name}] {res['tok_per_s']:.0f} tok/s, {ms_graph * 1e3:.1f} us/step (eager {ms_eager * 1e3:.1f} us); "
        f"llapis_moe_ffn {layer_res['ms_per_step'] * 1e3:.1f} us/step: island at {res['vs_moe_ffn']:.2f}x its rate")
    del wl
    torch.cuda.empty_cache()
    return res


def time_graph(wl, steps, warmup):
    """Capture R consecutive steps (one pass over the replicas) in a HIP graph
    and K mod R steps in a second one; time exactly K steps of replays."""
    torch = wl.torch
    R = wl.R
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for i in range(max(warmup, 1)):
            wl.step(i, stream.cuda_stream)
    torch.cuda.synchronize()
    reps, tail = divmod(steps, R)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for i in range(R):
            wl.step(i, stream.cuda_stream)
    gt = None
    if tail:
        gt = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gt, stream=stream):
            for i in range(tail):
                wl.step(i, stream.cuda_stream)
    torch.cuda.synchronize()
    for _ in range(max(1, warmup // R)):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(torch.cuda.current_stream())
    for _ in range(reps):
        g.replay()
    if gt is not None:
        gt.replay()
    e1.record(torch.cuda.current_stream())
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    return ms / steps, steps


def time_eager(wl, steps, warmup):
    torch = wl.torch
    s = torch.cuda.current_stream().cuda_stream
    for i in range(warmup):
        wl.step(i, s)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        wl.step(i, s)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def stage_times(wl, n):
    """Average per-stage kernel durations (ms) from HIP events recorded on the
    stream each kernel runs on."""
    torch, la = wl.torch, wl.la
    lib = la.lib()
    s = torch.cuda.current_stream().cuda_stream
    for i in range(8):
        wl.step(i, s)
    torch.cuda.synchronize()
    lib.llapis_profile_enable(1)
    for i in range(n):
        wl.step(i, s)
    ms = (C.c_float * 5)()
    calls = lib.llapis_profile_read(ms, 5)
    lib.llapis_profile_enable(0)
    if calls <= 0:
        raise RuntimeError("profile read failed")
    return {k: ms[j] / calls for j, k in enumerate(la._lib.STAGES)}


def stage_bytes(spec, n_hot, n_cold, T, pairs):
    """Algorithmic bytes per launch of the gate_up and down matvecs: the
    distinct experts' slabs once, activations in, outputs out (the down
    kernel also writes the combined layer output)."""
    gu_w = n_hot * spec.gu_bytes(spec.hot_gu_type) + n_cold * spec.gu_bytes(spec.cold_gu_type)
    dn_w = n_hot * spec.dn_bytes(spec.hot_dn_type) + n_cold * spec.dn_bytes(spec.cold_dn_type)
    gu = gu_w + T * spec.d_model * 4 + pairs * 2 * spec.n_ff * 4
    dn = dn_w + pairs * 2 * spec.n_ff * 4 + pairs * spec.d_model * 4 + T * spec.d_model * 4
    return {"gate_up": gu, "down": dn}


def replicas_for(spec, per_step_bytes, mall=256 << 20, floor=512 << 20):
    """Enough distinct replicas that one rotation touches >= 512 MB (2x MALL)."""
    return max(2, int(np.ceil(max(floor, 2 * mall) / max(per_step_bytes, 1))))


def run_config(la, torch, name, host_layer, T, steps, warmup, dev, seed=1234, act=0, gelu=0):
    sp = host_layer.spec
    probe = Workload(la, torch, host_layer, 1, T, 16, seed, dev, act, gelu)
    n_hot, n_cold, pairs = probe.routing()
    bytes_step = layer_bytes(sp, n_hot, n_cold, T)
    R = replicas_for(sp, bytes_step)
    del probe
    wl = Workload(la, torch, host_layer, R, T, 16, seed, dev, act, gelu)
    log(f"[{name}] T={T} distinct experts/step hot {n_hot:.2f} cold {n_cold:.2f}; "
        f"{R} replicas x {bytes_step / 1e6:.1f} MB/step")
    ms_graph, timed = time_graph(wl, steps, warmup)
    ms_eager = time_eager(wl, min(steps, 200), min(warmup, 20))
    st = stage_times(wl, max(2 * R, 64))
    ms_counts = None
    if T <= 4:
        # the same decode with the device routing counters on
        wlc = Workload(la, torch, host_layer, R, T, 16, seed, dev, act, gelu, counts=True)
        ms_counts, _ = time_graph(wlc, steps, warmup)
        del wlc
    sb = stage_bytes(sp, n_hot, n_cold, T, pairs)
    dom = max(("gate_up", "down"), key=lambda k: st[k])
    dec_down = "k_dec_down" if T == 1 or not DOWN_BY_GROUP else "k_dec_down_grp"
    kernel = ({"gate_up": "k_dec_gate_up", "down": dec_down} if T <= 4 else
              {"gate_up": "k_pf_gate_up" if act == 0 else "k_pf_gate_up_q1", "down": "k_pf_down"})[dom]
    res = {
        "tok_per_s": T * 1e3 / ms_graph,
        "ms_per_step": ms_graph,
        "ms_per_step_route_counts": ms_counts,
        "ms_per_step_eager": ms_eager,
        "steps_timed": timed,
        "hbm_gbs_step": bytes_step / (ms_graph * 1e-3) / 1e9,
        "hbm_frac_step": bytes_step / (ms_graph * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "algo_bytes_step": bytes_step,
        "replicas": R,
        "stage_ms": st,
        "dominant": dom,
        "dominant_kernel": kernel,
        "dominant_bytes": sb[dom],
        "dominant_gbs": sb[dom] / (st[dom] * 1e-3) / 1e9,
        "distinct_hot": n_hot,
        "distinct_cold": n_cold,
        "pairs": pairs,
    }
    if T > 4:
        ops = pairs * OPS_PER_PAIR
        ai = ops / max(bytes_step, 1)
        tops = ops / (ms_graph * 1e-3) / 1e12
        attain = min(INT8_PEAK_TOPS, ai * HBM_PEAK_GBS / 1e3)
        gemm_ms = st["gate_up"] + st["down"]
        res.update({"int8_tops": tops, "frac_int8_peak": tops / INT8_PEAK_TOPS, "ops_per_byte": ai,
                    "attainable_tops": attain, "frac_attainable": tops / attain,
                    "gemm_int8_tops": ops / (gemm_ms * 1e-3) / 1e12,
                    "gemm_frac_int8_peak": ops / (gemm_ms * 1e-3) / 1e12 / INT8_PEAK_TOPS})
        log(f"[{name}] {tops:.1f} int8 TOP/s = {100 * tops / INT8_PEAK_TOPS:.2f}% of peak, "
            f"{100 * tops / attain:.1f}% of attainable {attain:.0f} (AI {ai:.0f} op/B); GEMMs alone "
            f"{res['gemm_int8_tops']:.1f} TOP/s")
    log(f"[{name}] {res['tok_per_s']:.0f} tok/s, {ms_graph * 1e3:.1f} us/step (eager {ms_eager * 1e3:.1f} us), "
        f"step {res['hbm_gbs_step']:.0f} GB/s, {dom} {res['dominant_gbs']:.0f} GB/s, stages "
        + ", ".join(f"{k} {v * 1e3:.1f}us" for k, v in st.items()))
    if ms_counts is not None:
        log(f"[{name}] with device routing counters: {ms_counts * 1e3:.1f} us/step")
    del wl
    torch.cuda.empty_cache()
    return res


def run_promote(la, torch, full, dual, spec, dev, jobs=256, steps=256):
    """The promotion path: one promotion copies an expert's Q4_K gate_up and
    Q5_0 down pages (3 593 216 B) from the promotion source in HBM (all 128
    experts, 460 MB, rotated so the MALL does not hold them) into a slot of a
    spare slab, through the promotion engine (llapis_xfer_*).  Measured alone
    (back-to-back jobs per copy mode: hipMemcpyAsync, or the copy kernel with
    8 / 32 / 128 workgroups) and overlapped with the K=57 4-token decode
    (graph replays on the compute stream while 4 promotions per decode step
    run on the engine's stream): the decode slowdown and the promotion rate."""
    lib = la.lib()
    E = spec.n_expert
    gb, db = spec.gu_bytes(spec.hot_gu_type), spec.dn_bytes(spec.hot_dn_type)
    per = gb + db
    NS = 16
    src_gu = torch.from_numpy(full.hot_gu).to(dev)
    src_dn = torch.from_numpy(full.hot_dn).to(dev)
    dst_gu = torch.zeros(NS * gb, dtype=torch.uint8, device=dev)
    dst_dn = torch.zeros(NS * db, dtype=torch.uint8, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    done = (la._lib.LlapisXferDone * 1024)()

    def engine(wgs):
        x = lib.llapis_xfer_create(1, E, NS, wgs)
        if not x:
            raise RuntimeError(lib.llapis_xfer_last_error().decode())
        for g, (d, src, b) in enumerate(((dst_gu, src_gu, gb), (dst_dn, src_dn, db))):
            if lib.llapis_xfer_set_group(x, 0, g, d.data_ptr(), src.data_ptr(), b, b) != 0:
                raise RuntimeError(lib.llapis_xfer_last_error().decode())
        return x

    def issue(x, n, k0):
        for i in range(n):
            lib.llapis_xfer_submit(x, 0, ((k0 + i) * 37) % E, (k0 + i) % NS)
        lib.llapis_xfer_flush(x, s)

    def drain(x):
        lib.llapis_xfer_wait_idle(x, s)
        while lib.llapis_xfer_take_done(x, done, 1024) > 0:
            pass

    alone = {}
    for wgs in (0, 8, 32, 128):
        x = engine(wgs)
        issue(x, 16, 0)
        drain(x)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        issue(x, jobs, 16)
        drain(x)
        us = (time.perf_counter() - t0) * 1e6 / jobs
        alone[str(wgs)] = {"us_per_promotion": us, "gbs": 2 * per / (us * 1e-6) / 1e9}
        lib.llapis_xfer_free(x)
        log(f"[promote] copy mode {'hipMemcpyAsync' if wgs == 0 else f'kernel x{wgs} WGs'}: {us:.2f} us per "
            f"promotion, {alone[str(wgs)]['gbs']:.0f} GB/s (read + write)")
    # overlap with the dual 4-token decode, replayed as a graph
    wl = Workload(la, torch, dual, 1, 4, 16, 1234, dev, 0, 0)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for i in range(8):
            wl.step(i, stream.cuda_stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for i in range(16):
            wl.step(i, stream.cuda_stream)
    reps = steps // 16
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def decode_ms():
        e0.record(torch.cuda.current_stream())
        for _ in range(reps):
            g.replay()
        e1.record(torch.cuda.current_stream())
        return e0, e1

    for _ in range(2):
        g.replay()
    torch.cuda.synchronize()
    a, b = decode_ms()
    torch.cuda.synchronize()
    base_us = a.elapsed_time(b) * 1e3 / (reps * 16)
    over = {}
    for wgs in (0, 32, 128):
        x = engine(wgs)
        issue(x, 8, 0)
        drain(x)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        issue(x, 4 * reps * 16, 0)          # queued first: the copies run beside the replays
        a, b = decode_ms()
        b.synchronize()
        t_dec = time.perf_counter() - t0
        drain(x)
        t_all = time.perf_counter() - t0
        us = a.elapsed_time(b) * 1e3 / (reps * 16)
        over[str(wgs)] = {"decode_us_per_step": us, "slowdown": us / base_us,
                          "promotions_per_s": 4 * reps * 16 / t_all,
                          "copies_done_with_decode": t_all <= 1.05 * t_dec}
        lib.llapis_xfer_free(x)
        log(f"[promote] decode T=4 with 4 promotions per step ({'hipMemcpyAsync' if wgs == 0 else f'kernel x{wgs}'}): "
            f"{us:.1f} us/step vs {base_us:.1f} alone (x{us / base_us:.2f}); {over[str(wgs)]['promotions_per_s']:.0f} "
            "promotions/s")
    del wl, src_gu, src_dn, dst_gu, dst_dn
    torch.cuda.empty_cache()
    return {"bytes_per_promotion": per, "alone": alone, "decode_alone_us_per_step": base_us,
            "with_decode": over}


def copy_ceiling(torch, dev, nbytes, reps=400):
    """GB/s that a plain device-to-device copy moving `nbytes` per launch (half
    read, half written) reaches, rotated over >= 512 MB of buffers so the MALL
    does not hold them: what any kernel of this size can expect, launch and
    ramp included."""
    half = max(1 << 20, int(nbytes) // 2)
    n = max(2, (512 << 20) // half + 1)
    src = [torch.empty(half, dtype=torch.uint8, device=dev).fill_(1) for _ in range(n)]
    dst = [torch.empty(half, dtype=torch.uint8, device=dev) for _ in range(n)]
    s = torch.cuda.current_stream()
    for i in range(n):
        dst[i].copy_(src[i])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for i in range(reps):
        dst[i % n].copy_(src[i % n])
    e1.record(s)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del src, dst
    torch.cuda.empty_cache()
    return 2 * half / (ms * 1e-3) / 1e9


def measured_traffic(workload, kernel):
    """HBM bytes per launch of `kernel` from the rocprofv3 FETCH_SIZE and
    WRITE_SIZE passes committed under profiles/ (scaled by a plain copy's
    counts), or None when that kernel was not measured for this workload."""
    try:
        d = json.loads((ROOT / "profiles" / "pmc_traffic.json").read_text())
        return d[workload][kernel]["traffic_bytes"]
    except (OSError, KeyError, TypeError, ValueError):
        return None


class Stack:
    """The 30-layer stack: per layer its own fp32 router (seeded per layer),
    its own Zipf(1.1) hot set of 57 experts (a per-layer permutation) and a
    router bias that puts ~85 % of the picks on them; the expert slabs are
    per-layer device copies of the one quantised layer (distinct memory, the
    same bytes).  Attention is omitted: each layer is h += moe(rms_norm(h)),
    the MoE input normalised as the model's is (without the norm the
    residual stream grows until q8 scales overflow fp16); the residual add
    and the next layer's norm run as one kernel."""

    def __init__(self, la, torch, full, spec, n_layers, dev):
        self.la, self.torch, self.spec = la, torch, spec
        gb, db = spec.gu_bytes(spec.hot_gu_type), spec.dn_bytes(spec.hot_dn_type)
        cold_gu = torch.from_numpy(full.cold_gu).to(dev)
        cold_dn = torch.from_numpy(full.cold_dn).to(dev)
        self.layers, self.descs, self.bytes_tok, self.hot_frac = [], [], 0.0, []
        import copy
        from llapis_amd.moe import seed_for
        for il in range(n_layers):
            prior, hot = la.zipf_hot_set(spec.n_expert, 57, 1000 + il)
            lay = copy.copy(full)
            lay.router_w = la.synth_normal(seed_for(2000 + il, 0, 0), spec.n_expert * spec.d_model,
                                           0.0, 0.02).reshape(spec.n_expert, spec.d_model)
            lay.hot_gu = np.concatenate([full.hot_gu[e * gb:(e + 1) * gb] for e in hot])
            lay.hot_dn = np.concatenate([full.hot_dn[e * db:(e + 1) * db] for e in hot])
            lay.residency = la.Residency.from_hot(spec.n_expert, hot)
            bias, frac = la.tune_router_bias(lay.router_w, prior, hot, 0.85, 3000 + il)
            lay.router_b = bias
            self.hot_frac.append(frac)
            lay.cold_gu = lay.cold_dn = None          # the shared cold pools are cloned on the device
            d = la.DeviceLayer(lay, dev)
            d.cold_gu, d.cold_dn = cold_gu.clone(), cold_dn.clone()
            lay.hot_gu = lay.hot_dn = None            # host copies no longer needed
            self.layers.append(d)
            self.descs.append(d.desc())
        self.fn = la.lib().llapis_moe_ffn

    def routed_tiers(self, h0, ws, stream):
        """Distinct hot and cold experts one pass of h0 routes to, over every
        layer (each layer's ids read back after its call)."""
        torch, sp = self.torch, self.spec
        T = h0.shape[0]
        h = h0.clone()
        out = torch.zeros_like(h0)
        ids = torch.empty(T, sp.top_k, dtype=torch.int32, device=h.device)
        w = torch.empty(T, sp.top_k, device=h.device)
        n_hot = n_cold = 0
        for d, dl in zip(self.descs, self.layers):
            xl = torch.nn.functional.rms_norm(h, (sp.d_model,), eps=1e-6)
            rc = self.fn(C.byref(d), xl.data_ptr(), None, T, out.data_ptr(), ids.data_ptr(), w.data_ptr(),
                         ws.data_ptr(), ws.numel(), stream)
            if rc != 0:
                raise RuntimeError(self.la.lib().llapis_last_error().decode())
            torch.cuda.synchronize()
            res = dl.layer.residency
            ex = set(ids.cpu().numpy().ravel().tolist())
            hot = sum(1 for e in ex if res.is_hot(int(e)))
            n_hot += hot
            n_cold += len(ex) - hot
            h.add_(out)
        return n_hot, n_cold

    def run(self, h, xn, out, ws, stream, T, moe=True):
        """h [T, d_model] (the residual stream) is updated in place through
        every layer; xn holds each layer's input rms_norm(h), out its MoE
        output.  The glue between layers is one kernel (h += out, then the
        next input's norm: llapis_residual_rmsnorm).  moe=False runs only the
        glue, to time it on its own."""
        torch = self.torch
        sp = self.spec
        ids = torch.empty(T, sp.top_k, dtype=torch.int32, device=h.device)
        w = torch.empty(T, sp.top_k, device=h.device)
        self.la.residual_rmsnorm(h, None, xn, eps=1e-6, stream=stream)
        for d in self.descs:
            if moe:
                rc = self.fn(C.byref(d), xn.data_ptr(), None, T, out.data_ptr(), ids.data_ptr(), w.data_ptr(),
                             ws.data_ptr(), ws.numel(), stream)
                if rc != 0:
                    raise RuntimeError(self.la.lib().llapis_last_error().decode())
            self.la.residual_rmsnorm(h, out, xn, eps=1e-6, stream=stream)


def run_stack(la, torch, full, spec, dev, n_layers=30, decode_steps=50, prefill_tokens=11200):
    t0 = time.time()
    st = Stack(la, torch, full, spec, n_layers, dev)
    log(f"[stack] {n_layers} layers ready in {time.time() - t0:.1f} s (hot share of picks "
        f"{np.mean(st.hot_frac):.2f})")
    s = torch.cuda.current_stream()
    res = {"layers": n_layers}
    for T, steps, name in ((1, decode_steps, "decode"), (prefill_tokens, 2, "prefill")):
        need = int(la.lib().llapis_moe_ffn_workspace_size(C.byref(st.descs[0]), T))
        ws = torch.zeros(need, dtype=torch.uint8, device=dev)
        h0 = torch.from_numpy(la.synth_normal(4000 + T, T * spec.d_model).reshape(T, spec.d_model)).to(dev)
        h, xn, out = h0.clone(), torch.empty_like(h0), torch.zeros_like(h0)

        def timed(moe):
            # one pass (the reset of h included) captured as a HIP graph for
            # the decode token; the long prefill pass is launched eagerly
            cs = torch.cuda.Stream()
            with torch.cuda.stream(cs):
                h.copy_(h0)
                st.run(h, xn, out, ws, cs.cuda_stream, T, moe)     # warm-up pass
            torch.cuda.synchronize()
            g = None
            if T == 1:
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=cs):
                    h.copy_(h0)
                    st.run(h, xn, out, ws, cs.cuda_stream, T, moe)
                torch.cuda.synchronize()
                g.replay()
                torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            for _ in range(steps):
                if g is not None:
                    g.replay()
                else:
                    h.copy_(h0)
                    st.run(h, xn, out, ws, s.cuda_stream, T, moe)
            e1.record(s)
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) / steps

        ms = timed(True)
        assert torch.isfinite(h).all().item(), "non-finite residual stream"
        out.zero_()
        glue = timed(False)
        moe_ms = max(ms - glue, 1e-9)
        ops = T * spec.top_k * OPS_PER_PAIR * n_layers
        r = {"tokens": T, "ms_per_pass": ms, "glue_ms_per_pass": glue, "moe_ms_per_pass": moe_ms,
             "tok_per_s": T * 1e3 / ms, "moe_tok_per_s": T * 1e3 / moe_ms,
             "moe_us_per_layer": moe_ms * 1e3 / n_layers, "moe_int8_tops": ops / (moe_ms * 1e-3) / 1e12}
        if T == 1:
            # bytes: each layer's routed experts of this token (hot and cold
            # counted from the pass's own routing) once + its router
            per = spec.gu_bytes(spec.hot_gu_type) + spec.dn_bytes(spec.hot_dn_type)
            per_c = spec.gu_bytes(spec.cold_gu_type) + spec.dn_bytes(spec.cold_dn_type)
            n_hot, n_cold = st.routed_tiers(h0, ws, s.cuda_stream)
            b = n_hot * per + n_cold * per_c + n_layers * spec.n_expert * spec.d_model * 4
            r["distinct_hot_per_pass"], r["distinct_cold_per_pass"] = n_hot, n_cold
            r["moe_hbm_gbs"] = b / (moe_ms * 1e-3) / 1e9
            r["moe_hbm_frac"] = r["moe_hbm_gbs"] / HBM_PEAK_GBS
        res[name] = r
        log(f"[stack {name}] {T} token(s) x {n_layers} layers: {ms:.3f} ms per pass ({glue:.3f} ms of it the "
            f"norm/add glue); MoE {r['moe_us_per_layer']:.1f} us per layer, {r['moe_tok_per_s']:.0f} tok/s"
            + (f", {r['moe_hbm_gbs']:.0f} GB/s ({r['distinct_hot_per_pass']} hot + {r['distinct_cold_per_pass']} "
               f"cold experts per pass)" if T == 1 else f", {r['moe_int8_tops']:.1f} int8 TOP/s"))
        del ws, h, h0, xn, out
    del st
    torch.cuda.empty_cache()
    return res


def run_stack_dynamic(la, torch, full, spec, dev, n_layers=30, tokens=192, drift_every=64, copy_wgs=0):
    """The 30-layer decode with the residency loop a server runs, in native
    code (llapis_residency_*): every call counts its routing on the device;
    after each token the runtime pulls the counts (one D2H copy for all
    layers), the policy decides (cost rule, at most 4 promotions per token),
    the FILLING mirrors are published with copies on the stream and the
    promotion engine copies the experts from the promotion source in HBM
    (every expert in the hot formats) on its own stream while the next token
    runs; finished copies become READY at the next token end.  Every
    `drift_every` tokens each layer's router bias is permuted, so the routing
    moves away from the resident experts and the policy has to follow.  Token
    passes are graph replays; the host work between them is part of the
    time."""
    from llapis_amd.policy import ResidencyLoop
    lib = la.lib()
    t0 = time.time()
    st = Stack(la, torch, full, spec, n_layers, dev)
    E, K = spec.n_expert, 57
    gb, db = spec.gu_bytes(spec.hot_gu_type), spec.dn_bytes(spec.hot_dn_type)
    rl = ResidencyLoop(n_layers, E, K, copy_wgs=copy_wgs)
    pol = rl.policy
    src_gu = torch.from_numpy(full.hot_gu).to(dev)       # the promotion source: all experts, hot formats
    src_dn = torch.from_numpy(full.hot_dn).to(dev)
    for il, d in enumerate(st.layers):
        d.route_counts, d.route_hits = rl.counters(il)
        st.descs[il] = d.desc()
        for g, (slab, src, b) in enumerate(((d.hot_gu, src_gu, gb), (d.hot_dn, src_dn, db))):
            if lib.llapis_xfer_set_group(rl.xfer, il, g, slab.data_ptr(), src.data_ptr(), b, b) != 0:
                raise RuntimeError(lib.llapis_xfer_last_error().decode())
        rl.set_mirrors(il, d.exp_slot.data_ptr(), d.slot_exp.data_ptr(), d.slot_state.data_ptr())
        for s_, e in enumerate(d.slot_exp.cpu().numpy()):
            pol.seed(il, int(e), s_)
    stream = torch.cuda.Stream()
    rl.publish_all(stream.cuda_stream)
    rng = np.random.default_rng(5)
    # the drift phases' router biases, permuted ahead (device tensors)
    n_drift = (tokens - 1) // drift_every
    drifted = []
    for il, d in enumerate(st.layers):
        b = d.router_b.clone()
        row = []
        for _ in range(n_drift):
            b = b[torch.from_numpy(rng.permutation(E)).to(dev)]
            row.append(b.clone())
        drifted.append(row)
    T = 1
    need = int(lib.llapis_moe_ffn_workspace_size(C.byref(st.descs[0]), T))
    ws = torch.zeros(need, dtype=torch.uint8, device=dev)
    h0 = torch.from_numpy(la.synth_normal(4001, spec.d_model).reshape(1, spec.d_model)).to(dev)
    h, xn, out = h0.clone(), torch.empty_like(h0), torch.zeros_like(h0)
    with torch.cuda.stream(stream):
        h.copy_(h0)
        st.run(h, xn, out, ws, stream.cuda_stream, T)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        h.copy_(h0)
        st.run(h, xn, out, ws, stream.cuda_stream, T)
    torch.cuda.synchronize()
    rl.token_end(stream.cuda_stream)                     # drains the warm-up passes' counts
    r0 = rl.stats()
    hits = []                                            # per token: (hot pairs, other pairs) over all layers
    host_s = 0.0
    log(f"[stack dynamic] {n_layers} layers, native residency loop ready in {time.time() - t0:.1f} s")
    t_start = time.perf_counter()
    prev = r0
    with torch.cuda.stream(stream):
        for tok in range(tokens):
            if tok and tok % drift_every == 0:
                for il, d in enumerate(st.layers):
                    d.router_b.copy_(drifted[il][tok // drift_every - 1])
            g.replay()
            a = time.perf_counter()
            rl.token_end(stream.cuda_stream)            # waits for the token, decides, publishes, flushes
            host_s += time.perf_counter() - a
            cur = rl.stats()
            hits.append((cur["hot_pairs"] - prev["hot_pairs"], cur["cold_pairs"] - prev["cold_pairs"]))
            prev = cur
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    lib.llapis_xfer_wait_idle(rl.xfer, stream.cuda_stream)
    # the same token passes with a wait after each and no residency loop:
    # what a server's synchronous decode costs without the loop
    t_sync = time.perf_counter()
    with torch.cuda.stream(stream):
        for tok in range(tokens):
            g.replay()
            stream.synchronize()
    sync_ms = (time.perf_counter() - t_sync) * 1e3 / tokens
    xs = la._lib.LlapisXferStats()
    lib.llapis_xfer_get_stats(rl.xfer, C.byref(xs))
    pst = pol.stats()
    rst = rl.stats()
    rl.close()
    hw = np.array([hh / max(1, hh + cc) for hh, cc in hits])
    segs = [float(hw[i:i + drift_every].mean()) for i in range(0, tokens, drift_every)]
    first = [float(hw[i:i + 8].mean()) for i in range(0, tokens, drift_every)]
    res = {"layers": n_layers, "tokens": tokens, "ms_per_token": wall * 1e3 / tokens, "tok_per_s": tokens / wall,
           "loop": "native", "engine_copy_wgs": copy_wgs, "promotions": int(pst["promotions"]), "fills_completed": int(pst["fills_completed"]),
           "publications": int(rst["publications"] - r0["publications"]), "copies_bytes": int(xs.bytes),
           "hit_rate_per_phase": segs, "hit_rate_first_8_tokens_per_phase": first,
           "token_end_ms_per_token": host_s * 1e3 / tokens, "sync_no_loop_ms_per_token": sync_ms,
           "loop_host_ms_per_token": (rst["host_ms"] - r0["host_ms"]) / tokens,
           "decision_ms_per_token": float(pst["refresh_pause_ms_total"]) / max(1, int(pst["refresh_count"]))}
    log(f"[stack dynamic] {tokens} tokens x {n_layers} layers: {res['ms_per_token']:.3f} ms per token "
        f"({res['tok_per_s']:.0f} tok/s) with the native residency loop; {res['promotions']} promotions "
        f"({xs.bytes / 1e9:.2f} GB copied), hit rate per {drift_every}-token phase "
        + ", ".join(f"{v:.2f}" for v in segs) + " (first 8 tokens of each: " + ", ".join(f"{v:.2f}" for v in first)
        + f"); token end (waits for the token's pass) {res['token_end_ms_per_token']:.3f} ms per token; the same "
        f"passes with a wait after each and no loop: {sync_ms:.3f} ms per token; the loop's own host time "
        f"{res['loop_host_ms_per_token']:.3f} ms per token (decision {res['decision_ms_per_token']:.3f})")
    del st, src_gu, src_dn, ws
    torch.cuda.empty_cache()
    return res


AVX512_FLAGS = ("avx512f", "avx512bw", "avx512vl", "avx512dq", "avx512cd", "avx512_vnni", "avx512vbmi")


def host_cpu():
    """(model name, logical CPUs, ISA of the reference build to load, path)."""
    model, flags, n = "unknown", set(), 0
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name") and model == "unknown":
                model = line.split(":", 1)[1].strip()
            elif line.startswith("flags") and not flags:
                flags = set(line.split(":", 1)[1].split())
            elif line.startswith("processor"):
                n += 1
    except OSError:
        pass
    lib512 = ROOT / "oracle" / "_ref" / "libggml_ref_avx512.so"
    if all(f in flags for f in AVX512_FLAGS) and lib512.exists():
        return model, n, "avx512", lib512
    return model, n, "avx2", ROOT / "oracle" / "_ref" / "libggml_ref.so"


def cpu_threads():
    """The threads the CPU baseline runs on: every core this process may use,
    up to the host CPU share a one-GPU job gets (OMP_NUM_THREADS, 16 when
    unset) -- the reference's own sidecar pool also stops at 16 workers."""
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    share = int(os.environ.get("OMP_NUM_THREADS", "16") or 16)
    return max(1, min(cores, share, 16))


def cpu_baseline(layers, budget_s=8.0):
    """The reference's CPU path, built from its sources (oracle/_ref), timed on
    the host cores on a bounded sample of each workload, with the same
    quantised bytes as the GPU run and weights rotating over >= 512 MB of
    layer replicas (DRAM, not the LLC):
      iq2s, q4k   the ggml CPU graph of one layer (router, soft_max, top-k,
                  mul_mat_id gate_up, geglu, mul_mat_id down, combine);
      dual, prefill  that graph for the routing and the hot pairs, the
                  reference's CPU cold executor (src/moe_sidecar.cpp) for the
                  cold pairs.
    layers: {name: (host layer, tokens per step, single tier: 'cold'/'hot'/None)}."""
    sys.path.insert(0, str(ROOT / "oracle"))
    from oracle import Ref
    import llapis_amd as la
    model, n_cpu, isa, lib = host_cpu()
    threads = cpu_threads()
    ref = Ref(str(lib))
    res = {"cpu_model": model, "logical_cpus": n_cpu, "isa": isa, "threads": threads, "configs": {}}
    for name, (lay, T, tier) in layers.items():
        sp = lay.spec
        if tier is not None:
            gt, dt = (sp.cold_gu_type, sp.cold_dn_type) if tier == "cold" else (sp.hot_gu_type, sp.hot_dn_type)
            gu, dn = (lay.cold_gu, lay.cold_dn) if tier == "cold" else (lay.hot_gu, lay.hot_dn)
            per = len(gu) + len(dn) + lay.router_w.nbytes
            R = max(2, int(np.ceil((512 << 20) / per)))
            reps = [ref.layer(lay.router_w, lay.router_b, sp.top_k, gt, gu, dt, dn, sp.n_ff, T) for _ in range(R)]

            def step(i, x, reps=reps):
                reps[i % len(reps)].run(x, threads, False)
        else:
            import copy
            per = len(lay.hot_gu) + len(lay.hot_dn) + len(lay.cold_gu) + len(lay.cold_dn) + lay.router_w.nbytes
            R = max(2, int(np.ceil((512 << 20) / per)))
            reps = []
            for _ in range(R):
                c = copy.copy(lay)
                c.cold_gu, c.cold_dn = lay.cold_gu.copy(), lay.cold_dn.copy()
                reps.append(ref.dual(c, T, threads))

            def step(i, x, reps=reps):
                reps[i % len(reps)].run(x)
        xs = la.synth_normal(99, 8 * T * sp.d_model).reshape(8, T, sp.d_model)
        for i in range(2):
            step(i, xs[i])
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < budget_s and n < 100000:
            step(n, xs[n % 8])
            n += 1
        dt_s = time.perf_counter() - t0
        res["configs"][name] = {"tok_per_s": n * T / dt_s, "ms_per_step": dt_s * 1e3 / n, "steps": n,
                                "seconds": dt_s, "replicas": R, "replica_mb": per / 1e6,
                                "tokens_per_step": T}
        log(f"[cpu {name}] {n * T / dt_s:.1f} tok/s ({dt_s * 1e3 / n:.2f} ms per step of {T} token(s), {n} steps, "
            f"{R} replicas x {per / 1e6:.0f} MB) on {threads} threads ({isa}, {model})")
        del reps
    return res


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--configs", default="iq2s,q4k,dual,island,prefill,prefill_q81,q4stream,stack,promote,stackdyn",
                    help="comma list of iq2s,q4k,dual,island,prefill,prefill_q81,q4stream,stack,promote,stackdyn (island: "
                         "the operator-boundary path beside each decode config run)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--engine-wgs", type=int, default=0,
                    help="stackdyn: the promotion engine's copy mode (0 hipMemcpyAsync, else copy-kernel workgroups)")
    ap.add_argument("--cpu-seconds", type=float, default=8.0, help="CPU baseline seconds per workload")
    ap.add_argument("--tune", default="", help="key=value,... passed to llapis_set_tuning (measurement switches)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run 20 device-to-device copies of MIB MiB (scales the HBM byte counters) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for {args.gpus}); the path's multi-GPU "
              "sharding is a design note, not a measured mode.", file=sys.stderr)
        sys.exit(2)

    import torch
    import llapis_amd as la
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    if args.copy_probe:
        n = args.copy_probe << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": n, "copies": 20}))
        return
    global DOWN_BY_GROUP
    for kv in filter(None, args.tune.split(",")):
        k, v = kv.split("=")
        la.lib().llapis_set_tuning(int(k), int(v))
        if int(k) == 4:
            DOWN_BY_GROUP = int(v) != 0
    cfgs = [c.strip() for c in args.configs.split(",") if c.strip()]
    spec = la.LayerSpec()
    t0 = time.time()
    # all fp32 expert weights are generated once per expert; each tier is
    # quantised from the same floats (seed 1)
    need_hot = any(c in cfgs for c in ("q4k", "dual", "prefill", "prefill_q81", "q4stream", "stack", "promote",
                                       "stackdyn"))
    prior, hot57 = la.zipf_hot_set(spec.n_expert, 57, 7)
    full = la.make_layer(spec, 1, list(range(spec.n_expert)) if need_hot else [], cold=True)
    log(f"quantised {spec.n_expert} experts x {'4' if need_hot else '2'} formats in {time.time() - t0:.1f} s")

    import copy
    results = {}
    island = {}
    if "iq2s" in cfgs:
        cold_only = copy.copy(full)
        cold_only.residency = la.Residency.from_hot(spec.n_expert, [])
        results["iq2s"] = run_config(la, torch, "decode all-IQ2_S T=1", cold_only, 1, args.steps, args.warmup, dev)
        if "island" in cfgs:
            island["iq2s"] = run_island(la, torch, "decode all-IQ2_S T=1", cold_only, 1, args.steps, args.warmup,
                                        dev, results["iq2s"])
    if "q4k" in cfgs:
        results["q4k"] = run_config(la, torch, "decode all-Q4_K T=1", full, 1, args.steps, args.warmup, dev)
        if "island" in cfgs:
            island["q4k"] = run_island(la, torch, "decode all-Q4_K T=1", full, 1, args.steps, args.warmup, dev,
                                       results["q4k"])
    if any(c in cfgs for c in ("dual", "prefill", "prefill_q81", "q4stream", "promote")):
        dual = copy.copy(full)
        gb, db = spec.gu_bytes(spec.hot_gu_type), spec.dn_bytes(spec.hot_dn_type)
        dual.hot_gu = np.concatenate([full.hot_gu[e * gb:(e + 1) * gb] for e in hot57])
        dual.hot_dn = np.concatenate([full.hot_dn[e * db:(e + 1) * db] for e in hot57])
        dual.residency = la.Residency.from_hot(spec.n_expert, hot57)
        bias, frac = la.tune_router_bias(full.router_w, prior, hot57, 0.85, 11)
        dual.router_b = bias
        log(f"dual: router bias puts {frac:.2f} of picks on the 57 hot experts")
        if "dual" in cfgs:
            results["dual"] = run_config(la, torch, "decode dual K=57 T=4", dual, 4, args.steps, args.warmup, dev)
            if "island" in cfgs:
                island["dual"] = run_island(la, torch, "decode dual K=57 T=4", dual, 4, args.steps, args.warmup, dev,
                                            results["dual"])
        if "prefill" in cfgs:
            results["prefill"] = run_config(la, torch, "prefill dual K=57 T=512", dual, 512,
                                            max(10, args.steps // 40), max(2, args.warmup // 20), dev)
        if "prefill_q81" in cfgs:
            # the same chunk in the reference GPU path's activation mode (q8_1, GELU tanh)
            results["prefill_q81"] = run_config(la, torch, "prefill dual K=57 T=512 q8_1", dual, 512,
                                                max(10, args.steps // 40), max(2, args.warmup // 20), dev,
                                                act=1, gelu=1)
        if "q4stream" in cfgs:
            # q4stream: the same chunk with every expert at the hot precision,
            # read from the all-expert hot source (identity page table)
            q4s = copy.copy(full)
            q4s.router_b = dual.router_b
            results["q4stream"] = run_config(la, torch, "prefill q4stream (every expert Q4_K) T=512", q4s, 512,
                                             max(10, args.steps // 40), max(2, args.warmup // 20), dev)
        if "promote" in cfgs:
            results["promote"] = run_promote(la, torch, full, dual, spec, dev)

    if island:
        results["island"] = island
    if "stack" in cfgs:
        results["stack"] = run_stack(la, torch, full, spec, dev)
    if "stackdyn" in cfgs:
        results["stack_dynamic"] = run_stack_dynamic(la, torch, full, spec, dev, copy_wgs=args.engine_wgs)

    # the headline: the mixed-precision 4-token decode; the single-format
    # decodes and the prefill stay in extra
    head_name = next((n for n in ("dual", "iq2s", "q4k") if n in results), None)
    if head_name is None:
        head_name = next((n for n, v in results.items() if isinstance(v, dict) and "dominant_gbs" in v), None)
    if head_name is None:
        print(json.dumps({"extra": results}))
        return
    head = results[head_name]
    workload = {"dual": "decode_dual_k57_4tok", "iq2s": "decode_all_iq2s_1tok", "q4k": "decode_all_q4k_1tok",
                "prefill": "prefill_dual_k57_512tok", "prefill_q81": "prefill_dual_k57_512tok_q8_1",
                "q4stream": "prefill_q4stream_512tok"}.get(head_name)
    roof = {"bound": "hbm", "achieved": head["dominant_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": head["dominant_gbs"] / HBM_PEAK_GBS,
            "traffic": measured_traffic(workload, head["dominant_kernel"]),
            "kernel": head["dominant_kernel"], "algo_bytes_per_launch": head["dominant_bytes"],
            "avg_launch_ms": head["stage_ms"][head["dominant"]]}
    ceil = copy_ceiling(torch, dev, head["dominant_bytes"])
    roof["copy_ceiling_gbs_at_size"] = ceil
    roof["frac_of_copy_ceiling"] = head["dominant_gbs"] / ceil
    log(f"copy of the same {head['dominant_bytes'] / 1e6:.1f} MB per launch: {ceil:.0f} GB/s "
        f"({100 * ceil / HBM_PEAK_GBS:.0f} % of peak); dominant kernel at {100 * head['dominant_gbs'] / ceil:.0f} % of it")
    cpu = None
    if not args.no_cpu_baseline and head_name in ("dual", "iq2s", "q4k"):
        try:
            layers = {}
            if "iq2s" in results:
                cold_only = copy.copy(full)
                cold_only.residency = la.Residency.from_hot(spec.n_expert, [])
                layers["iq2s"] = (cold_only, 1, "cold")
            if "q4k" in results:
                layers["q4k"] = (full, 1, "hot")
            if "dual" in results:
                layers["dual"] = (dual, 4, None)
            if "prefill" in results:
                layers["prefill"] = (dual, 512, None)
            cb = cpu_baseline(layers, args.cpu_seconds)
            for name, c in cb["configs"].items():
                g = results.get(name)
                if g:
                    c["gpu_over_cpu"] = g["tok_per_s"] / c["tok_per_s"]
                    c["effective_gbs"] = g["algo_bytes_step"] / (c["ms_per_step"] * 1e-3) / 1e9
            h = cb["configs"][head_name]
            what = {"dual": "4 tokens on the dual K=57 layer; the reference's ggml CPU graph for the routing "
                            "and the hot pairs and its CPU cold executor for the cold pairs",
                    "iq2s": "1 token on the all-IQ2_S layer; the reference's ggml CPU graph",
                    "q4k": "1 token on the all-Q4_K layer; the reference's ggml CPU graph"}[head_name]
            cpu = {"value": h["tok_per_s"], "unit": "tok/s", "cores": cb["threads"], "kind": "reference",
                   "sample": f"{h['steps']} decode steps of {what}, {h['seconds']:.1f} s, weights rotated over "
                             f"{h['replicas']} replicas of {h['replica_mb']:.0f} MB; built from the reference's "
                             f"sources for {cb['isa']} ({cb['cpu_model']}, {cb['logical_cpus']} logical CPUs, "
                             f"{cb['threads']} threads)",
                   "cpu_model": cb["cpu_model"], "isa": cb["isa"], "configs": cb["configs"]}
            log(f"cpu baseline: {cpu['value']:.1f} tok/s on {cpu['cores']} threads")
        except Exception as e:  # the checker library may be absent; say so
            cpu = {"value": None, "unit": "tok/s", "cores": 0, "kind": "reference", "sample": f"unavailable: {e}"}
    line = {
        "metric": METRIC,
        "value": head["tok_per_s"],
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "moe_layer_" + (workload or head_name), "d_model": spec.d_model,
                   "n_ff": spec.n_ff, "n_expert": spec.n_expert, "top_k": spec.top_k,
                   "tokens_per_step": HEAD_TOKENS.get(head_name), "formats": HEAD_FORMATS.get(head_name),
                   "replicas": head["replicas"], "distinct_hot": head["distinct_hot"],
                   "distinct_cold": head["distinct_cold"],
                   "hbm_gbs_step": head["hbm_gbs_step"], "hbm_frac_step": head["hbm_frac_step"]},
        "roofline": roof,
        "cpu_baseline": cpu,
        "extra": results,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
