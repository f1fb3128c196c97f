"""Config 5 at full depth: the 30-layer stack, h += moe(rms_norm(h)) per
layer, in both activation modes -- decode (16 sequences of 1 token and 4 of
4 tokens, one llapis call per sequence and layer) and a 530-token prefill (two
chunks of at most 4096 routed pairs) -- against the oracle's own 30-layer
chain.

Every layer has its own router (seeded per layer), its own Zipf(1.1) hot set
of K = 57 experts with a router bias that puts ~85 % of the picks on it, and
its own expert weights: the 128 quantised experts of one seeded layer,
relabelled by a per-layer seeded permutation and each scaled by a per-layer
seeded factor in [0.75, 1.25] (every block scale, and Q4_K's dmin, times the
factor and re-rounded to fp16; both tiers of an expert get the same factor, so
they stay two precisions of one set of weights).  Quantising 30 x 128 experts
in four formats afresh takes about half an hour of CPU; the relabelled,
rescaled layers compute 30 different functions, which is what a chain of
layers tests.

Two kinds of check:

1. Each checked layer against the oracle on the GPU's own input to it:
   routing identical, and the layer bars of helpers.check_layer_bars
   counted over all checked layers together where a decode layer's 32
   tokens are too few for them (the whole output within relative L2 5e-4,
   at most 1 % of the token outputs above 1e-3), with each layer's whole
   output within the requirement's 1e-3 and each token within 3e-3.  This is
   the parity check proper, at every depth.
2. The GPU's 30-layer chain against the oracle's own chain from the same
   input.  Past a few layers this chain is chaotic, in the oracle alone: each
   layer quantises its input to q8, so a difference of 1e-6 in the residual
   stream re-rounds some q8 values, the layer's output then moves by ~1e-4,
   which re-rounds more values in the next layer, and a top-8 choice whose
   two candidates are close flips, after which that token's stream differs by
   ~1 %.  The control is the oracle's chain with the last-bit differences of
   another fp32 summation order put in (oracle.set_sum_jitter: every gate_up
   and down sum moved one ulp): it routes 23 (q8_1 mode) and 29 (CPU mode) of
   32 tokens differently by layer 30, and its tokens end 1e-2 - 5e-2 apart
   at the median and up to ~0.2 (the GPU's chain measures the same).  So the
   chains are held to the 3-layer slice's bars after three layers (at most
   1 % + 1 of the tokens routed differently; the ones routed alike within
   relative L2 1e-3 together, 3e-3 in q8_1 mode, 1e-2 each, median 1e-5 --
   1e-4 for decode in q8_1 mode, whose per-token re-roundings are more
   frequent),
   and at layer 30 to the control's spread: the median token within 5x the
   control's median plus 1e-3 and the worst within 2x the control's worst
   plus 0.05 -- a check against an error in every token, which the per-layer
   checks bound far more tightly.
   The oracle and the GPU path treat tokens independently (each token's
   routing, quantisation and sums use only its own row), so the chains are
   compared on a subset of the tokens spread over both prefill chunks."""
import copy
import sys

import numpy as np
import pytest

import llapis_amd as la
from helpers import FULL, full_layer, oracle_mode, per_token_rel_l2, rel_l2, tokens

pytestmark = pytest.mark.gpu

MODES = [(la.ACT_CPU, la.GELU_TABLE), (la.ACT_Q8_1, la.GELU_TANH)]
N_LAYERS = 30
SEED = 1

# (block bytes, offsets of the fp16 scales) per format
_SCALES = {la.Q4_K: (144, (0, 2)), la.IQ2_S: (82, (0,)), la.Q5_0: (22, (0,)), la.IQ4_NL: (18, (0,))}


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _relabel(buf, n_exp, t, perm, f):
    """Slab i of the result = expert slab perm[i] of buf (n_exp slabs) with its
    block scales times f[i], re-rounded to fp16."""
    bb, offs = _SCALES[t]
    a = buf.reshape(n_exp, -1, bb)[perm].copy()
    for o in offs:
        d = a[:, :, o:o + 2].copy().view(np.float16)[..., 0].astype(np.float32)
        d = (d * np.asarray(f, np.float32)[:, None]).astype(np.float16)
        a[:, :, o:o + 2] = d.view(np.uint8).reshape(a.shape[0], a.shape[1], 2)
    return a.reshape(-1)


def _depth_layer(full, il):
    """Layer il: expert e is `full`'s expert perm[e] scaled by f[e]; its hot
    slots hold the 57 experts a Zipf(1.1) prior ranks first (seed 1000 + il),
    its router is seeded 2000 + il and biased so ~85 % of picks are hot."""
    sp = full.spec
    n = sp.n_expert
    rng = np.random.default_rng(3000 + il)
    perm = rng.permutation(n)
    f = rng.uniform(0.75, 1.25, n).astype(np.float32)
    prior, hot = la.zipf_hot_set(n, 57, 1000 + il)
    rw = la.synth_normal(la.seed_for(2000 + il, 0, 0), n * sp.d_model, 0.0, 0.02).reshape(n, sp.d_model)
    bias, frac = la.tune_router_bias(rw, prior, hot, 0.85, 1001 + il)
    hot = list(hot)
    lay = copy.copy(full)
    lay.meta = dict(full.meta)
    lay.residency = la.Residency.from_hot(n, hot)
    lay.hot_gu = _relabel(full.hot_gu, n, sp.hot_gu_type, perm[hot], f[hot])
    lay.hot_dn = _relabel(full.hot_dn, n, sp.hot_dn_type, perm[hot], f[hot])
    lay.cold_gu = _relabel(full.cold_gu, n, sp.cold_gu_type, perm, f)
    lay.cold_dn = _relabel(full.cold_dn, n, sp.cold_dn_type, perm, f)
    lay.router_w, lay.router_b = rw, bias
    lay.meta["hot_frac"] = frac
    return lay


_layers = []


def _stack():
    if not _layers:
        full = full_layer(SEED)
        for il in range(N_LAYERS):
            _layers.append(_depth_layer(full, il))
    return _layers


def _rms_norm_np(h, eps=1e-6):
    h = h.astype(np.float32)
    return (h / np.sqrt(np.mean(h * h, axis=1, keepdims=True, dtype=np.float32) + np.float32(eps))).astype(np.float32)


SLICE = 3                   # the depth at which the 3-layer slice's bars apply


def _oracle_chain(oracle, layers, h, act_mode, gelu_mode, T_call):
    """The oracle's chain from h: per layer the routing ids, the residual
    stream after SLICE layers and at the end."""
    ids_all = []
    h_slice = None
    for il, lay in enumerate(layers):
        x = _rms_norm_np(h)
        ids, w, _ = oracle.router(x, lay.router_w, lay.router_b, FULL.top_k)
        out, _ = oracle.moe_experts(lay, x, ids, w, oracle_mode(act_mode, T_call), gelu_mode)
        h = h + out
        ids_all.append(ids)
        if il == SLICE - 1:
            h_slice = h.copy()
    return ids_all, h_slice, h


def _flips(ids_a, ids_b):
    """Per layer, the number of tokens whose routing differs at that layer or
    before."""
    gone = np.zeros(ids_a[0].shape[0], bool)
    out = []
    for a, b in zip(ids_a, ids_b):
        gone |= ~(a == b).all(axis=1)
        out.append(int(gone.sum()))
    return np.array(out), gone


def _run(gpu, oracle, calls, act_mode, gelu_mode, check_every, subset):
    """calls: (first token, token count) of each llapis call per layer over
    the input rows; subset: the rows the chains are compared on."""
    import torch
    layers = _stack()
    n_rows = sum(c for _, c in calls)
    T_call = max(c for _, c in calls)
    h0 = tokens(4100 + n_rows, n_rows, FULL.d_model)
    h = torch.from_numpy(h0).to(gpu)
    ids_gpu, pooled, sq = [], [], [0.0, 0.0]
    for il, lay in enumerate(layers):
        xl = torch.nn.functional.rms_norm(h, (FULL.d_model,), eps=1e-6).contiguous()
        dl = la.DeviceLayer(lay, gpu, act_mode, gelu_mode)
        outs, idss, ws = [], [], []
        for b, c in calls:
            o, i, w = dl.forward(xl[b:b + c])
            outs.append(o.clone()); idss.append(i.clone()); ws.append(w.clone())
        torch.cuda.synchronize()
        out, ids, w = torch.cat(outs), torch.cat(idss), torch.cat(ws)
        ids_g = ids.cpu().numpy()
        if il % check_every == 0 or il == len(layers) - 1:
            x = xl.cpu().numpy()
            ids_o, _, _ = oracle.router(x, lay.router_w, lay.router_b, FULL.top_k)
            assert np.array_equal(ids_g, ids_o), f"layer {il}: routing differs"
            out_o, _ = oracle.moe_experts(lay, x, ids_g, w.cpu().numpy(), oracle_mode(act_mode, T_call), gelu_mode)
            out_g = out.cpu().numpy()
            err, per = rel_l2(out_g, out_o), per_token_rel_l2(out_g, out_o)
            say(f" layer {il}: rel_l2 {err:.1e}; tokens median {np.median(per):.1e} max {per.max():.1e} "
                f"({int((per > 1e-3).sum())} of {per.size} above 1e-3)")
            assert err <= 1e-3 and per.max() <= 3e-3, (il, err, per.max())
            assert np.median(per) <= 1e-5, il
            pooled.append(per)
            sq[0] += float(np.sum((out_g.astype(np.float64) - out_o) ** 2))
            sq[1] += float(np.sum(out_o.astype(np.float64) ** 2))
        ids_gpu.append(ids_g[subset])
        h = h + out
        if il == SLICE - 1:
            h_slice_gpu = h.cpu().numpy()[subset]
        del dl
    pooled = np.concatenate(pooled)
    say(f"  checked layers together: rel_l2 {np.sqrt(sq[0] / sq[1]):.1e}, {int((pooled > 1e-3).sum())} of "
        f"{pooled.size} token outputs above 1e-3")
    assert np.sqrt(sq[0] / sq[1]) <= 5e-4
    frac = 0.02 if act_mode == la.ACT_Q8_1 else 0.01
    assert (pooled > 1e-3).sum() <= int(frac * pooled.size), (int((pooled > 1e-3).sum()), pooled.size)
    h_gpu = h.cpu().numpy()[subset]
    n = len(subset)
    # the oracle's chain from the same rows, and the control: the same chain
    # with every fp32 sum moved by one ulp
    ids_o, hs_o, h_o = _oracle_chain(oracle, layers, h0[subset], act_mode, gelu_mode, T_call)
    oracle.set_sum_jitter(12345)
    try:
        ids_c, hs_c, h_c = _oracle_chain(oracle, layers, h0[subset], act_mode, gelu_mode, T_call)
    finally:
        oracle.set_sum_jitter(0)
    g, g_gone = _flips(ids_gpu, ids_o)
    c, _ = _flips(ids_c, ids_o)
    say(f"  tokens routed differently by layer (of {n}): gpu vs oracle {g.tolist()}")
    say(f"                                        control {c.tolist()}")
    # the slice's bars after SLICE layers
    _, gone3 = _flips(ids_gpu[:SLICE], ids_o[:SLICE])
    same = ~gone3
    per3 = per_token_rel_l2(h_slice_gpu, hs_o)
    med3_c = float(np.median(per_token_rel_l2(hs_c, hs_o)))
    say(f"  after {SLICE} layers: {int(gone3.sum())} routed differently; routed alike: rel_l2 "
        f"{rel_l2(h_slice_gpu[same], hs_o[same]):.1e}, max {per3[same].max():.1e}, median {np.median(per3[same]):.1e} "
        f"(control median {med3_c:.1e})")
    assert gone3.sum() <= n // 100 + 1
    assert rel_l2(h_slice_gpu[same], hs_o[same]) <= (3e-3 if act_mode == la.ACT_Q8_1 else 1e-3)
    # the median bar: 1e-5; 1e-4 for decode in q8_1 mode, whose per-32-block
    # fp32 scaling on both matvecs differs from the oracle's order in more
    # places: after three layers about half its tokens carry a re-rounded q8
    # value (measured 1.4e-5 at the median of 32)
    med_bar = 1e-4 if act_mode == la.ACT_Q8_1 and T_call <= 4 else 1e-5
    assert per3[same].max() <= 1e-2 and np.median(per3[same]) <= med_bar
    # layer 30 against the control's spread
    per_g = per_token_rel_l2(h_gpu, h_o)
    per_c = per_token_rel_l2(h_c, h_o)
    say(f"  after {len(layers)} layers per-token rel_l2: gpu median {np.median(per_g):.1e} max {per_g.max():.1e}; "
        f"control median {np.median(per_c):.1e} max {per_c.max():.1e}")
    assert np.median(per_g) <= 5 * np.median(per_c) + 1e-3
    assert per_g.max() <= 2 * per_c.max() + 0.05


@pytest.mark.timeout(600)
@pytest.mark.parametrize("act_mode,gelu_mode", MODES)
def test_stack_full_depth_decode(gpu, oracle, act_mode, gelu_mode):
    """16 sequences of 1 token (the one-token decode kernels) and 4 of 4
    tokens (the 2-4 token kernels) through the 30 layers."""
    say(f"workload stack 30 layers decode 16 x 1 + 4 x 4 tokens act={act_mode}")
    calls = [(i, 1) for i in range(16)] + [(16 + 4 * i, 4) for i in range(4)]
    _run(gpu, oracle, calls, act_mode, gelu_mode, 2, np.arange(32))


@pytest.mark.timeout(600)
@pytest.mark.parametrize("act_mode,gelu_mode", MODES)
def test_stack_full_depth_prefill_two_chunks(gpu, oracle, act_mode, gelu_mode):
    """One 530-token call per layer (4240 routed pairs: two chunks); the
    chains compared on 64 rows spread over both chunks."""
    say(f"workload stack 30 layers prefill T=530 act={act_mode}")
    subset = np.unique(np.linspace(0, 529, 64).astype(int))
    _run(gpu, oracle, [(0, 530)], act_mode, gelu_mode, 5, subset)
