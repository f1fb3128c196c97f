"""GPU parity at the edges of the path's domain, against the CPU oracle:
expert counts that are not a multiple of the wave width, top_k at its limits
(1 and 16), and placement masks whose slots are FILLING or FREE or whose
mapping is stale or out of range (ffn_moe.cu:80-130 with policy.h:46: only a
READY slot whose slot_exp points back at the expert is hot).  Each case runs
the decode path (1 and 3 tokens) and the prefill path (40 tokens), in the
CPU-parity activation mode and in the q8_1 mode."""
import copy

import numpy as np
import pytest

import llapis_amd as la
from llapis_amd import LayerSpec
from helpers import check_layer_bars, layer, oracle_mode, rel_l2, tokens
from test_gpu_parity import check_flip_tolerant, say, torch_mod

pytestmark = pytest.mark.gpu

EDGE_SPECS = {
    "E100_k6": LayerSpec(d_model=512, n_ff=96, n_expert=100, top_k=6),
    "E32_k16": LayerSpec(d_model=256, n_ff=64, n_expert=32, top_k=16),
    "E20_k1": LayerSpec(d_model=256, n_ff=32, n_expert=20, top_k=1),
}


def mixed_mask_layer(spec, seed):
    """Hot slots for about 40% of the experts, then: slot 1 FILLING, slot 3
    FREE, expert hot[4] pointing at slot 5 (which holds hot[5]: stale), and
    expert hot[6] pointing past the slots.  The pools are untouched, so a
    kernel that ignored the mask would read a valid but wrong slab."""
    rng = np.random.default_rng(seed)
    n_hot = max(7, (2 * spec.n_expert) // 5)
    hot = sorted(rng.choice(spec.n_expert, n_hot, replace=False).tolist())
    base = layer(spec, seed, hot, scales=True)
    lay = copy.copy(base)
    r = copy.deepcopy(base.residency)
    r.slot_state[1] = la.SLOT_FILLING
    r.slot_state[3] = la.SLOT_FREE
    r.exp_slot[hot[4]] = 5
    r.exp_slot[hot[6]] = r.k_slots + 3
    lay.residency = r
    cold_now = {hot[1], hot[3], hot[4], hot[6]}
    assert all(not r.is_hot(e) for e in cold_now)
    assert sum(r.is_hot(e) for e in range(spec.n_expert)) == n_hot - 4
    return lay


@pytest.mark.parametrize("act_mode,gelu_mode", [(la.ACT_CPU, la.GELU_TABLE), (la.ACT_Q8_1, la.GELU_TANH)])
@pytest.mark.parametrize("T", [1, 3, 40])
@pytest.mark.parametrize("spec_name", list(EDGE_SPECS))
def test_shapes_and_placement_states(gpu, oracle, spec_name, T, act_mode, gelu_mode):
    torch = torch_mod()
    spec = EDGE_SPECS[spec_name]
    say(f"edges {spec_name} T={T} act={act_mode}")
    lay = mixed_mask_layer(spec, 700 + spec.n_expert)
    dl = la.DeviceLayer(lay, gpu, act_mode, gelu_mode)
    x = tokens(710 + T, T, spec.d_model)
    out, ids, w = dl.forward(torch.from_numpy(x).to(gpu))
    torch.cuda.synchronize()
    ids_g, w_g = ids.cpu().numpy(), w.cpu().numpy()
    ids_o, w_o, _ = oracle.router(x, lay.router_w, lay.router_b, spec.top_k)
    assert np.array_equal(ids_g, ids_o)
    assert np.allclose(w_g, w_o, rtol=1e-5, atol=1e-7)
    out_o, _ = oracle.moe_experts(lay, x, ids_g, w_g, oracle_mode(act_mode, T), gelu_mode)
    if T <= 4:
        err = rel_l2(out.cpu().numpy(), out_o)
        say(f"  rel_l2 vs oracle = {err:.3e}")
        assert err <= 1e-4
    elif act_mode == la.ACT_CPU:
        check_flip_tolerant(out.cpu().numpy(), out_o)
    else:
        check_layer_bars(out.cpu().numpy(), out_o, say, 0.02)


@pytest.mark.parametrize("act_mode,gelu_mode", [(la.ACT_CPU, la.GELU_TABLE), (la.ACT_Q8_1, la.GELU_TANH)])
def test_prefill_wide_model(gpu, oracle, act_mode, gelu_mode):
    """d_model 4096 at 40 tokens: the router's 16 K splits are 256 values
    each, past what the staged router kernel holds (192), so the chunk's
    logits come from the slice-by-slice kernel; 16 super-blocks a row in
    the grouped GEMMs."""
    torch = torch_mod()
    spec = LayerSpec(d_model=4096, n_ff=64, n_expert=16, top_k=2)
    T = 40
    say(f"wide d_model=4096 T={T} act={act_mode}")
    lay = mixed_mask_layer(spec, 730)
    dl = la.DeviceLayer(lay, gpu, act_mode, gelu_mode)
    x = tokens(731, T, spec.d_model)
    out, ids, w = dl.forward(torch.from_numpy(x).to(gpu))
    torch.cuda.synchronize()
    ids_g, w_g = ids.cpu().numpy(), w.cpu().numpy()
    ids_o, w_o, _ = oracle.router(x, lay.router_w, lay.router_b, spec.top_k)
    assert np.array_equal(ids_g, ids_o)
    assert np.allclose(w_g, w_o, rtol=1e-5, atol=1e-7)
    out_o, _ = oracle.moe_experts(lay, x, ids_g, w_g, oracle_mode(act_mode, T), gelu_mode)
    if act_mode == la.ACT_CPU:
        check_flip_tolerant(out.cpu().numpy(), out_o)
    else:
        check_layer_bars(out.cpu().numpy(), out_o, say, 0.02)


def test_zero_tokens_is_a_no_op(gpu):
    """n_tokens = 0: nothing is launched, nothing is written, status 0."""
    torch = torch_mod()
    spec = EDGE_SPECS["E20_k1"]
    lay = mixed_mask_layer(spec, 720)
    dl = la.DeviceLayer(lay, gpu)
    x = torch.zeros((0, spec.d_model), dtype=torch.float32, device=gpu)
    out, ids, w = dl.forward(x)
    torch.cuda.synchronize()
    assert out.shape[0] == 0 and ids.numel() == 0 and w.numel() == 0
