"""Host-side code of the product, CPU only: the quantisers (byte-exact against
the reference's ggml_quantize_chunk goldens), the synthetic generators, the
residency mask, the format sizes and the workspace arithmetic of the C ABI."""
from pathlib import Path

import numpy as np
import pytest

import llapis_amd as la
from llapis_amd import IQ2_S, IQ4_NL, Q4_K, Q5_0, LayerSpec, Residency

GOLD = Path(__file__).resolve().parent / "golden"
WTYPES = {"q4_K": Q4_K, "iq2_s": IQ2_S, "q5_0": Q5_0, "iq4_nl": IQ4_NL}


def test_quantisers_byte_exact_against_reference():
    g = np.load(GOLD / "quant.npz", allow_pickle=False)
    keys = sorted(k[:-2] for k in g.files if k.endswith("_q"))
    seen = set()
    for key in keys:
        name, variant = key.rsplit("_", 1)
        t = WTYPES[name]
        im = g[key + "_imatrix"]
        got = la.quantize(t, g[key + "_x"], im if im.size else None)
        assert np.array_equal(got, g[key + "_q"]), key
        seen.add((name, variant))
    assert {("iq2_s", "ones"), ("iq2_s", "none"), ("iq2_s", "ramp"), ("q4_K", "none"), ("q5_0", "none"),
            ("iq4_nl", "ones"), ("iq4_nl", "ramp")} <= seen


REF_GGML = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "libggml_ref.so"


@pytest.mark.parametrize("name", sorted(WTYPES))
def test_quantisers_match_reference_on_random_rows(name):
    """The reference's ggml_quantize_chunk, compiled from its sources into
    oracle/_ref, and this library's quantisers on the same rows, byte for
    byte: 48 rows of 2816 values per format drawn from eight distributions
    (the expert weights' N(0, 0.02), unit normal, heavy tails, one-signed,
    sparse, a wide dynamic range, tiny magnitudes, repeated values), with and
    without an importance matrix where the format takes one."""
    if not REF_GGML.exists():
        pytest.skip("oracle/_ref/libggml_ref.so not built (needs the reference tree)")
    import sys
    sys.path.insert(0, str(REF_GGML.parents[1]))
    from oracle import Ref
    ref = Ref(str(REF_GGML))
    t = WTYPES[name]
    n = 2816                                    # 11 super-blocks, 88 blocks of 32
    rng = np.random.default_rng(sum(name.encode()))
    rows = []
    for kind in range(8):
        for _ in range(6):
            if kind == 0:
                r = rng.normal(0, 0.02, n)
            elif kind == 1:
                r = rng.normal(0, 1, n)
            elif kind == 2:
                r = rng.standard_t(2, n) * 0.05
            elif kind == 3:
                r = np.abs(rng.normal(0, 1, n)) * (1 if rng.random() < 0.5 else -1)
            elif kind == 4:
                r = rng.normal(0, 1, n) * (rng.random(n) < 0.1)
            elif kind == 5:
                r = rng.normal(0, 1, n) * np.logspace(-5, 2, n)[rng.permutation(n)]
            elif kind == 6:
                r = rng.normal(0, 1e-6, n)
            else:
                r = rng.choice([-0.5, 0.25, 0.0, 1.0], n)
            rows.append(r)
    x = np.stack(rows).astype(np.float32)
    imats = [None]
    if t in (IQ2_S, IQ4_NL):
        imats += [np.ones(n, np.float32), rng.uniform(0.1, 4.0, n).astype(np.float32)]
    for im in imats:
        want = ref.quantize(t, x, im)
        got = la.quantize(t, x, im)
        assert np.array_equal(got.ravel(), want.ravel()), (name, None if im is None else float(im[0]))


@pytest.mark.parametrize("t", [Q4_K, Q5_0])
def test_quantiser_refuses_imatrix_for_hot_formats(t):
    n = 256
    with pytest.raises(la.LlapisError):
        la.quantize(t, np.zeros((1, n), np.float32), np.ones(n, np.float32))


def test_quantiser_refuses_ragged_rows():
    with pytest.raises(ValueError):
        la.quantize(Q4_K, np.zeros((1, 300), np.float32))


def test_format_sizes():
    # bytes per row at the benchmark shapes and per expert slab
    assert la.row_size(Q4_K, 2816) == 1584
    assert la.row_size(IQ2_S, 2816) == 902
    assert la.row_size(Q5_0, 704) == 484
    assert la.row_size(IQ4_NL, 704) == 396
    sp = LayerSpec()
    assert sp.gu_bytes(Q4_K) == 2_230_272 and sp.dn_bytes(Q5_0) == 1_362_944
    assert sp.gu_bytes(IQ2_S) == 1_270_016 and sp.dn_bytes(IQ4_NL) == 1_115_136
    assert sp.gu_bytes(Q4_K) + sp.dn_bytes(Q5_0) == 3_593_216
    assert sp.gu_bytes(IQ2_S) + sp.dn_bytes(IQ4_NL) == 2_385_152


def test_synth_normal_deterministic_and_normal():
    a = la.synth_normal(42, 1 << 20)
    b = la.synth_normal(42, 1 << 20)
    assert np.array_equal(a, b)
    assert not np.array_equal(a, la.synth_normal(43, 1 << 20))
    # counter-based: any window of the stream is reproducible on its own
    assert np.array_equal(la.synth_normal(42, 1000, offset=12345), a[12345:13345])
    assert abs(float(a.mean())) < 5e-3 and abs(float(a.std()) - 1.0) < 5e-3
    s = la.synth_normal(7, 100000, mean=0.0, std=0.02)
    assert abs(float(s.std()) - 0.02) < 5e-4
    # tails: the fraction beyond 3 sigma is close to 0.27 %
    assert 0.0020 < float(np.mean(np.abs(a) > 3)) < 0.0034


def _hot_by_definition(r, e):
    s = int(r.exp_slot[e])
    return 0 <= s < r.k_slots and int(r.slot_state[s]) == 2 and int(r.slot_exp[s]) == e


def test_residency_predicate_brute_force():
    rng = np.random.default_rng(11)
    E, K = 32, 9
    for _ in range(50):
        r = Residency(E, K, rng.integers(-2, K + 3, E).astype(np.int32), rng.integers(-1, E + 2, K).astype(np.int32),
                      rng.integers(0, 3, K).astype(np.int32))
        for e in range(E):
            assert r.is_hot(e) == _hot_by_definition(r, e)
    hot = [5, 1, 30]
    r = Residency.from_hot(E, hot)
    assert [e for e in range(E) if r.is_hot(e)] == sorted(hot)
    assert list(r.slot_exp) == hot and all(r.exp_slot[e] == s for s, e in enumerate(hot))
    filling = Residency.from_hot(E, hot, state=1)
    assert not any(filling.is_hot(e) for e in range(E))


def test_zipf_hot_set():
    prior, hot = la.zipf_hot_set(128, 57, 7)
    prior2, hot2 = la.zipf_hot_set(128, 57, 7)
    assert hot == hot2 and np.array_equal(prior, prior2)
    assert abs(prior.sum() - 1.0) < 1e-12
    assert set(hot) == set(np.argsort(-prior)[:57].tolist())
    # Zipf(1.1): the ratio of the first two frequencies is 2^1.1
    p = np.sort(prior)[::-1]
    assert abs(p[0] / p[1] - 2 ** 1.1) < 1e-9


def test_router_bias_tuning_hits_target():
    sp = LayerSpec(d_model=256, n_expert=32, top_k=4)
    rng = np.random.default_rng(12)
    w_r = (rng.standard_normal((sp.n_expert, sp.d_model)) * 0.02).astype(np.float32)
    prior, hot = la.zipf_hot_set(sp.n_expert, 10, 3)
    bias, frac = la.tune_router_bias(w_r, prior, hot, 0.85, 5, top_k=sp.top_k)
    assert abs(frac - 0.85) < 0.05 and bias.shape == (sp.n_expert,)


def test_make_layer_pools_match_quantised_experts():
    sp = LayerSpec(d_model=256, n_ff=32, n_expert=6, top_k=2)
    lay = la.make_layer(sp, 3, [4, 1])
    gu, dn = lay.expert_weights_f32(4, 3)
    gb, db = sp.gu_bytes(Q4_K), sp.dn_bytes(Q5_0)
    assert np.array_equal(lay.hot_gu[0:gb], la.quantize(Q4_K, gu))
    assert np.array_equal(lay.hot_dn[0:db], la.quantize(Q5_0, dn))
    cb = sp.gu_bytes(IQ2_S)
    assert np.array_equal(lay.cold_gu[4 * cb:5 * cb], la.quantize(IQ2_S, gu, np.ones(256, np.float32)))
    assert lay.residency.is_hot(1) and not lay.residency.is_hot(0)


def test_workspace_sizes():
    import ctypes as C
    lib = la.lib()
    sp = LayerSpec()
    desc = la._lib.LlapisMoeLayer()
    desc.d_model, desc.n_ff, desc.n_expert, desc.top_k, desc.k_slots = sp.d_model, sp.n_ff, sp.n_expert, sp.top_k, 57
    desc.hot_gu_type, desc.hot_dn_type, desc.cold_gu_type, desc.cold_dn_type = Q4_K, Q5_0, IQ2_S, IQ4_NL
    sizes = [int(lib.llapis_moe_ffn_workspace_size(C.byref(desc), T)) for T in (1, 2, 4, 5, 64, 512)]
    assert all(b > a for a, b in zip(sizes, sizes[1:]))
    # at least the per-pair gate_up and down outputs in fp32
    for T, b in zip((1, 2, 4, 5, 64, 512), sizes):
        assert b >= T * sp.top_k * (2 * sp.n_ff + sp.d_model) * 4
        assert b % 256 == 0
    assert int(lib.llapis_moe_ffn_workspace_size(C.byref(desc), 0)) == 0
