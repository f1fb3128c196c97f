"""GPU parity at the benchmark's own workloads: d_model 2816, n_ff 704,
128 experts, top-8, GeGLU (tanh), expert weights N(0, 0.02) quantised per
tier, tokens N(0, 1), router N(0, 0.02) in fp32.

1. decode of 1 token, every expert hot (Q4_K gate_up, Q5_0 down);
2. decode of 1 token, every expert cold (IQ2_S gate_up, IQ4_NL down);
3. dual precision, K = 57 hot slots chosen by a Zipf(1.1) prior and a router
   biased so ~85 % of picks are hot, 4 tokens (a depth-3 MTP verify batch),
   checked token by token;
4. the same dual layer on a 512-token prefill chunk (uneven expert groups);
5. a 3-layer slice of the 30-layer stack (per-layer routers and hot sets,
   h += moe(rms_norm(h))), decode of 1 token and a prefill of 530 tokens
   (one full chunk and a partial one).

Each runs in both activation modes: the CPU path's (q8_K / q8_0 + the fp16
GELU table) and the reference GPU path's (q8_1 + tanh).  The oracle gets the
same inputs; routing ids must be identical and every token within relative L2
1e-3 -- or, on the longer batches, within the bars of
helpers.check_layer_bars, which allow for q8 re-roundings after last-bit
fp32 differences.
"""
import sys

import numpy as np
import pytest

import llapis_amd as la
from helpers import (FULL, check_layer_bars, dual_k57, full_layer, oracle_mode, per_token_rel_l2, rel_l2, tokens,
                     with_hot_set)

pytestmark = pytest.mark.gpu

MODES = [(la.ACT_CPU, la.GELU_TABLE), (la.ACT_Q8_1, la.GELU_TANH)]
SEED = 1


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def run_layer(gpu, oracle, lay, x, act_mode, gelu_mode):
    import torch
    dl = la.DeviceLayer(lay, gpu, act_mode, gelu_mode)
    out, ids, w = dl.forward(torch.from_numpy(x).to(gpu))
    torch.cuda.synchronize()
    ids_g, w_g, out_g = ids.cpu().numpy(), w.cpu().numpy(), out.cpu().numpy()
    ids_o, w_o, _ = oracle.router(x, lay.router_w, lay.router_b, lay.spec.top_k)
    assert np.array_equal(ids_g, ids_o), "routing differs from the oracle"
    assert np.allclose(w_g, w_o, rtol=1e-5, atol=1e-7)
    out_o, _ = oracle.moe_experts(lay, x, ids_g, w_g, oracle_mode(act_mode, x.shape[0]), gelu_mode)
    return out_g, out_o, ids_g


@pytest.mark.parametrize("act_mode,gelu_mode", MODES)
@pytest.mark.parametrize("tier", ["q4k", "iq2s"])
def test_decode_one_token_all_one_tier(gpu, oracle, tier, act_mode, gelu_mode):
    """Configs 1 and 2: eight single-token calls on one layer, every expert
    hot (K = 128, slot e = expert e) or every expert cold (K = 0)."""
    say(f"workload decode all-{tier} T=1 act={act_mode}")
    full = full_layer(SEED)
    lay = with_hot_set(full, list(range(FULL.n_expert)) if tier == "q4k" else [])
    for i in range(8):
        x = tokens(900 + i, 1, FULL.d_model)
        got, want, ids = run_layer(gpu, oracle, lay, x, act_mode, gelu_mode)
        err = rel_l2(got, want)
        assert err <= 1e-3, (i, err)
    say(f"  8 tokens ok; last rel_l2 {err:.2e}")


@pytest.mark.parametrize("act_mode,gelu_mode", MODES)
def test_decode_dual_k57_four_tokens_per_token(gpu, oracle, act_mode, gelu_mode):
    """Config 3: dual K = 57, batches of 4 tokens, checked token by token;
    the router bias puts about 85 % of the picks on hot experts."""
    say(f"workload dual K=57 T=4 act={act_mode}")
    lay = dual_k57(full_layer(SEED), 7)
    assert 0.75 <= lay.meta["hot_frac"] <= 0.95
    res = lay.residency
    hot_picks = picks = 0
    for b in range(6):
        x = tokens(950 + b, 4, FULL.d_model)
        got, want, ids = run_layer(gpu, oracle, lay, x, act_mode, gelu_mode)
        per = per_token_rel_l2(got, want)
        say(f"  batch {b}: tokens " + " ".join(f"{v:.1e}" for v in per))
        assert per.max() <= 1e-3, (b, per)
        hot_picks += sum(res.is_hot(int(e)) for e in ids.ravel())
        picks += ids.size
    say(f"  6 batches ok; {hot_picks} of {picks} picks hot")
    assert hot_picks >= 0.6 * picks


@pytest.mark.parametrize("act_mode,gelu_mode", MODES)
def test_prefill_dual_k57_512_tokens(gpu, oracle, act_mode, gelu_mode):
    """Config 4: a 512-token prefill chunk of the dual layer (4096 routed
    pairs: the largest chunk the prefill path takes at top-8), bucketed by
    expert into uneven groups."""
    say(f"workload prefill dual K=57 T=512 act={act_mode}")
    lay = dual_k57(full_layer(SEED), 7)
    x = tokens(990, 512, FULL.d_model)
    got, want, ids = run_layer(gpu, oracle, lay, x, act_mode, gelu_mode)
    sizes = np.bincount(ids.ravel(), minlength=FULL.n_expert)
    say(f"  expert groups: {int((sizes == 0).sum())} empty, largest {sizes.max()}, "
        f"hot share {np.mean([lay.residency.is_hot(int(e)) for e in ids.ravel()]):.2f}")
    assert sizes.max() > 64 and (sizes > 0).sum() > 64          # uneven groups over most experts
    check_layer_bars(got, want, say, 0.02 if act_mode == la.ACT_Q8_1 else 0.01)


def _stack(full, n_layers):
    return [dual_k57(full, 1000 + il, router_seed=2000 + il) for il in range(n_layers)]


def _rms_norm_np(h, eps=1e-6):
    h = h.astype(np.float32)
    return (h / np.sqrt(np.mean(h * h, axis=1, keepdims=True, dtype=np.float32) + np.float32(eps))).astype(np.float32)


@pytest.mark.parametrize("act_mode,gelu_mode", MODES)
@pytest.mark.parametrize("T", [1, 530])
def test_stack_slice_three_layers(gpu, oracle, T, act_mode, gelu_mode):
    """Config 5, three layers of the stack: h += moe(rms_norm(h)).  Each
    layer against the oracle on the GPU's own input to it (ids identical,
    within the layer bars), then the oracle's own chain (numpy RMSNorm and
    add) against the GPU's final residual stream: tokens routed alike in every
    layer within relative L2 1e-3 together (3e-3 in q8_1 mode), 1e-2 each
    (median 1e-5), and at most 1 % of the tokens routed differently (a
    top-8 boundary moved by the two chains' last-bit differences).  A token
    that re-rounded one q8 value in layer l enters layer l + 1 with a different
    input, whose own quantisation then differs in more places: the chain's
    worst token is bounded loosely, the per-layer checks above are the tight
    ones."""
    import torch
    say(f"workload stack slice 3 layers T={T} act={act_mode}")
    layers = _stack(full_layer(SEED), 3)
    h0 = tokens(4000 + T, T, FULL.d_model)
    h = torch.from_numpy(h0).to(gpu)
    ids_gpu = []
    for il, lay in enumerate(layers):
        xl = torch.nn.functional.rms_norm(h, (FULL.d_model,), eps=1e-6)
        x = xl.cpu().numpy()
        dl = la.DeviceLayer(lay, gpu, act_mode, gelu_mode)
        out, ids, w = dl.forward(xl.contiguous())
        torch.cuda.synchronize()
        ids_g, w_g, out_g = ids.cpu().numpy(), w.cpu().numpy(), out.cpu().numpy()
        ids_o, _, _ = oracle.router(x, lay.router_w, lay.router_b, FULL.top_k)
        assert np.array_equal(ids_g, ids_o), f"layer {il}: routing differs"
        out_o, _ = oracle.moe_experts(lay, x, ids_g, w_g, oracle_mode(act_mode, T), gelu_mode)
        say(f" layer {il}:")
        check_layer_bars(out_g, out_o, say, 0.02 if act_mode == la.ACT_Q8_1 else 0.01)
        ids_gpu.append(ids_g)
        h = h + out
    h_gpu = h.cpu().numpy()
    # the oracle's own chain
    ho = h0.copy()
    same = np.ones(T, bool)
    for il, lay in enumerate(layers):
        x = _rms_norm_np(ho)
        ids_o, w_o, _ = oracle.router(x, lay.router_w, lay.router_b, FULL.top_k)
        same &= (ids_o == ids_gpu[il]).all(axis=1)
        out_o, _ = oracle.moe_experts(lay, x, ids_o, w_o, oracle_mode(act_mode, T), gelu_mode)
        ho = ho + out_o
    per = per_token_rel_l2(h_gpu, ho)
    say(f"  chain: {int((~same).sum())} of {T} tokens routed differently; routed alike: max rel_l2 "
        f"{per[same].max():.1e}")
    assert (~same).sum() <= max(0, T // 100)
    # q8_1 re-quantises each input in 32-blocks, so a perturbed input flips
    # more of its own activations: its chain drifts about twice as far
    assert rel_l2(h_gpu[same], ho[same]) <= (3e-3 if act_mode == la.ACT_Q8_1 else 1e-3)
    assert per[same].max() <= 1e-2 and np.median(per[same]) <= 1e-5


def _gemma4_inputs(seed, T):
    """Gemma4's two MoE inputs from one residual stream h (gemma4.cpp:393-403):
    the experts read ffn_pre_norm_2(h) = rms_norm(h) * s2, the router reads
    rms_norm(h) / sqrt(n_embd) * ffn_gate_inp_s.  s2 and ffn_gate_inp_s are
    seeded per-channel scales; ffn_gate_inp_s carries sqrt(n_embd) so the
    logits keep the scale the router's bias was tuned for."""
    d = FULL.d_model
    h = tokens(seed, T, d)
    r = _rms_norm_np(h)
    rng = np.random.default_rng(seed)
    s2 = rng.uniform(0.5, 1.5, d).astype(np.float32)
    s_inp = (np.float32(np.sqrt(d)) * rng.uniform(0.5, 1.5, d)).astype(np.float32)
    x = (r * s2).astype(np.float32)
    xr = ((r * np.float32(1.0 / np.sqrt(d))).astype(np.float32) * s_inp).astype(np.float32)
    return x, xr


@pytest.mark.parametrize("act_mode,gelu_mode", MODES)
@pytest.mark.parametrize("T", [4, 512])
def test_router_input_differs_from_expert_input(gpu, oracle, T, act_mode, gelu_mode):
    """The fused layer routes on its own router input (x_router) and runs the
    experts on x, as gemma4's MoE block does (gemma4.cpp:393-403, logits
    handed to build_moe_ffn as probs_in, llama-graph.cpp:1537-1541): dual
    K = 57 at 4 tokens (the decode path, token by token) and a 512-token
    chunk (the prefill path).  The ids equal the oracle's router on x_router
    (and differ from routing on x, so the second input is really used); the
    outputs equal the oracle's experts on x with those ids, to the same bars
    as the single-input workloads."""
    import torch
    say(f"workload router input != expert input T={T} act={act_mode}")
    lay = dual_k57(full_layer(SEED), 7)
    batches = 3 if T == 4 else 1
    differ = 0
    for b in range(batches):
        x, xr = _gemma4_inputs(5100 + 10 * T + b, T)
        dl = la.DeviceLayer(lay, gpu, act_mode, gelu_mode)
        out, ids, w = dl.forward(torch.from_numpy(x).to(gpu), x_router=torch.from_numpy(xr).to(gpu))
        torch.cuda.synchronize()
        ids_g, w_g, out_g = ids.cpu().numpy(), w.cpu().numpy(), out.cpu().numpy()
        ids_o, w_o, _ = oracle.router(xr, lay.router_w, lay.router_b, FULL.top_k)
        assert np.array_equal(ids_g, ids_o), "routing differs from the oracle's router on x_router"
        assert np.allclose(w_g, w_o, rtol=1e-5, atol=1e-7)
        ids_x, _, _ = oracle.router(x, lay.router_w, lay.router_b, FULL.top_k)
        differ += int((ids_x != ids_o).any(axis=1).sum())
        out_o, _ = oracle.moe_experts(lay, x, ids_g, w_g, oracle_mode(act_mode, T), gelu_mode)
        if T == 4:
            per = per_token_rel_l2(out_g, out_o)
            say(f"  batch {b}: tokens " + " ".join(f"{v:.1e}" for v in per))
            assert per.max() <= 1e-3, (b, per)
        else:
            check_layer_bars(out_g, out_o, say, 0.02 if act_mode == la.ACT_Q8_1 else 0.01)
    say(f"  {differ} of {batches * T} tokens would route differently on x")
    assert differ >= max(1, batches * T // 4)
