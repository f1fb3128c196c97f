"""The oracle (oracle/oracle.c, the CPU restatement used as the checker) pinned
before it is trusted.  CPU only.

How each oracle function is pinned:

  orc_dequantize (q4_K, iq2_s, q5_0, iq4_nl)
      bit-exact against the reference ggml's dequantize_row_* on the golden
      rows (quant.npz), and on blocks that enumerate all 1024 IQ2_S grid
      indices with and without signs (iq2s_grid.npz); closed-form special
      cases: a Q4_K block with unit scales and zero mins dequantises to its
      nibbles in ggml's order; per-sub-block scales multiply the right 32.
  orc_quantize_act (q8_K, q8_0)
      byte-exact against the reference x86 build (act.npz), including
      equal-magnitude maxima of opposite sign; invariants of q8_K: the first
      largest-magnitude value maps to -127, d = -max/127, bsums are the
      16-wide sums.
  orc_quantize_act (q8_1)
      parity unpinned against the reference (its quantiser is CUDA code that
      cannot be compiled here); pinned by its definition's invariants: the
      largest magnitude maps to +-127, d = amax/127, s = sum of x.
  orc_vec_dot CPU mode
      against the reference's vec_dot on the golden rows (dot.npz), and
      against the float64 dot of the dequantised operands.
  orc_vec_dot q8_1 mode
      q4_K, q5_0, iq4_nl: equal to the float64 dot of the dequantised operands
      (their q8_1 formulas are exact integer sums times scales); iq2_s: within
      the truncation bound of its integer formula (at most one unit of
      d*d8 per 32 values).  Known answers worked out by hand from the
      reference's integer formulas on blocks built field by field pin the
      two forms that differ from the dequantised dot: iq2_s's divisions
      truncate toward zero (where floor, rounding or exact arithmetic give
      other values), q5_0 uses the block's stored sum s.  The reference's
      CUDA code itself is not run (no CUDA compiler here).
  orc_vec_dot q8_1 matrix-core mode (ACT_Q8_1_MMA: the prefill's sums)
      every format equal to the float64 dot of the dequantised operands: its
      IQ2_S keeps the per-16 scale exact and its Q5_0 uses (q - 16) against
      d8 q, so every sum is an exact integer times scales.
  orc_geglu
      table mode bit-exact against the reference's geglu_split (geglu.npz),
      including the +-10 clamps; tanh mode against the closed form in float64.
  orc_router
      the golden layers' ids and weights (layer.npz); closed forms: equal
      logits give ids 0..k-1 and weights 1/k, Σw = 1, probabilities sum to 1,
      ids ordered by descending probability.
  orc_matvec, orc_moe_experts
      the reference's mul_mat_id (mmid.npz) and whole single-tier layers
      (layer.npz); the dual-precision mask by brute force: each routed pair
      takes the hot pool exactly when the READY predicate holds, the down
      .scale is applied once, and the combine is the weighted sum.
  Live reference (oracle/_ref, where it is built): randomised cases of all
      of the above.
"""
import math
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import pytest

from oracle import (ACT_CPU, ACT_Q8_1, ACT_Q8_1_MMA, GELU_TABLE, GELU_TANH, IQ2_S, IQ4_NL, Q4_K, Q5_0, Q8_0, Q8_1, Q8_K,
                    row_size)

GOLD = Path(__file__).resolve().parent / "golden"
WTYPES = {"q4_K": Q4_K, "iq2_s": IQ2_S, "q5_0": Q5_0, "iq4_nl": IQ4_NL}


def load(name):
    return np.load(GOLD / name, allow_pickle=False)


def rows_of(q, t, n):
    rs = row_size(t, n)
    return [q[i * rs:(i + 1) * rs] for i in range(q.size // rs)]


# ------------------------------------------------------------ dequantisation

def test_dequant_matches_reference_goldens(oracle):
    g = load("quant.npz")
    keys = sorted(k[:-2] for k in g.files if k.endswith("_q"))
    assert len(keys) >= 8
    for key in keys:
        t = WTYPES[key.rsplit("_", 1)[0]]
        x, q, deq = g[key + "_x"], g[key + "_q"], g[key + "_deq"]
        n = x.shape[1]
        for r, blk in enumerate(rows_of(q, t, n)):
            got = oracle.dequantize(t, blk, n)
            assert np.array_equal(got.view(np.uint32), deq[r].view(np.uint32)), (key, r)


def test_iq2s_every_grid_index(oracle):
    g = load("iq2s_grid.npz")
    plain = oracle.dequantize(IQ2_S, g["plain_q"], 32 * 256)
    assert np.array_equal(plain, g["plain_deq"])
    signed = oracle.dequantize(IQ2_S, g["signed_q"], 32 * 256)
    assert np.array_equal(signed, g["signed_deq"])
    table = g["plain_deq"].reshape(1024, 8)
    # the codebook: bytes 0x08, 0x19, 0x2b; 1024 distinct entries
    assert set(np.unique(table).tolist()) <= {8.0, 25.0, 43.0}
    assert len({tuple(r) for r in table}) == 1024


def test_iq2s_product_table_is_the_codebook():
    """The product's 2-bit code table (llapis_amd/csrc/iq2s_grid.inc) expands
    to the reference's codebook."""
    src = (Path(__file__).resolve().parents[1] / "llapis_amd/csrc/iq2s_grid.inc").read_text()
    body = " ".join(l.split("//")[0] for l in src.splitlines())
    codes = [int(v, 0) for v in body.split(",") if v.strip()]
    assert len(codes) == 1024
    vals = np.array([8.0, 25.0, 43.0, np.nan])
    table = np.array([[vals[(c >> (2 * k)) & 3] for k in range(8)] for c in codes])
    assert np.array_equal(table, load("iq2s_grid.npz")["plain_deq"].reshape(1024, 8))


def _q4k_block(d, dmin, sc, mn, qs):
    """Q4_K block from 8 6-bit scales and mins (packing of ggml-common.h:
    the inverse of get_scale_min_k4)."""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.float16(dmin).tobytes(), np.uint8)
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    b[4:16] = s
    b[16:144] = qs
    return b


def test_q4k_closed_form_nibble_order(oracle):
    rng = np.random.default_rng(3)
    qs = rng.integers(0, 256, 128, dtype=np.uint8)
    blk = _q4k_block(1.0, 0.0, [1] * 8, [0] * 8, qs)
    y = oracle.dequantize(Q4_K, blk, 256)
    want = np.zeros(256)
    for j in range(4):                         # 64 values per 32 bytes: low nibbles, then high
        want[64 * j:64 * j + 32] = qs[32 * j:32 * j + 32] & 15
        want[64 * j + 32:64 * j + 64] = qs[32 * j:32 * j + 32] >> 4
    assert np.array_equal(y, want)


def test_q4k_closed_form_scales_and_mins(oracle):
    rng = np.random.default_rng(4)
    qs = rng.integers(0, 256, 128, dtype=np.uint8)
    sc = [3, 17, 63, 1, 40, 9, 62, 33]         # exercises both halves of the 6-bit packing
    mn = [0, 5, 63, 12, 50, 7, 1, 31]
    blk = _q4k_block(0.5, 0.25, sc, mn, qs)
    y = oracle.dequantize(Q4_K, blk, 256)
    nib = np.zeros(256)
    for j in range(4):
        nib[64 * j:64 * j + 32] = qs[32 * j:32 * j + 32] & 15
        nib[64 * j + 32:64 * j + 64] = qs[32 * j:32 * j + 32] >> 4
    want = np.array([0.5 * sc[i // 32] * nib[i] - 0.25 * mn[i // 32] for i in range(256)])
    assert np.allclose(y, want, rtol=1e-6, atol=1e-6)


# ------------------------------------------------------------ activations

def test_act_quant_matches_reference(oracle):
    g = load("act.npz")
    for r, x in enumerate(g["x"]):
        assert np.array_equal(oracle.quantize_act(Q8_K, x), g["q8_K"][r]), ("q8_K", r)
        assert np.array_equal(oracle.quantize_act(Q8_0, x), g["q8_0"][r]), ("q8_0", r)


def _q8k_fields(b, n):
    nb = n // 256
    blk = b.reshape(nb, 292)
    d = blk[:, 0:4].copy().view(np.float32).ravel()
    q = blk[:, 4:260].view(np.int8).astype(np.int64)
    bs = blk[:, 260:292].copy().view(np.int16).astype(np.int64)
    return d, q, bs


def test_q8k_invariants(oracle):
    rng = np.random.default_rng(5)
    for trial in range(20):
        x = (rng.standard_normal(512) * rng.uniform(0.01, 10)).astype(np.float32)
        d, q, bs = _q8k_fields(oracle.quantize_act(Q8_K, x), 512)
        for b in range(2):
            xb = x[256 * b:256 * (b + 1)]
            i = int(np.argmax(np.abs(xb)))          # first largest magnitude
            assert q[b, i] == -127
            assert np.float32(d[b]) == np.float32(1.0 / np.float32(-127.0 / xb[i]))
            assert np.all(np.abs(q[b]) <= 127)
            assert np.array_equal(bs[b], q[b].reshape(16, 16).sum(1))
            assert np.max(np.abs(d[b] * q[b] - xb)) <= abs(d[b]) * 0.5 + 1e-6


def test_q8_1_invariants(oracle):
    """q8_1 (the GPU activation format): d = amax/127, q = round(x/d), s = Σx."""
    rng = np.random.default_rng(6)
    x = (rng.standard_normal(256) * 2).astype(np.float32)
    b = oracle.quantize_act(Q8_1, x).reshape(8, 36)
    for k in range(8):
        xb = x[32 * k:32 * (k + 1)]
        d = float(b[k, 0:2].copy().view(np.float16)[0])
        s = float(b[k, 2:4].copy().view(np.float16)[0])
        q = b[k, 4:36].view(np.int8).astype(np.int64)
        amax = np.abs(xb).max()
        assert abs(d - amax / 127) <= 1e-3 * amax / 127
        assert abs(abs(q[np.argmax(np.abs(xb))]) - 127) == 0
        assert abs(s - xb.sum(dtype=np.float64)) <= 2e-3 * max(1.0, abs(xb.sum()))
        assert np.max(np.abs(q * (amax / 127) - xb)) <= amax / 127 * 0.5 + 1e-6


# ------------------------------------------------------------ dots

def test_vec_dot_matches_reference(oracle):
    g = load("dot.npz")
    for name, t in WTYPES.items():
        n = int(g[f"{name}_n"])
        at = int(g[f"{name}_act_type"])
        assert oracle.act_type(t, ACT_CPU) == at
        for r, w in enumerate(rows_of(g[f"{name}_w_q"], t, n)):
            wf = np.abs(oracle.dequantize(t, w, n).astype(np.float64))
            for j, a in enumerate(g[f"{name}_act_q"]):
                want = float(g[f"{name}_dot"][r, j])
                got = oracle.vec_dot(t, ACT_CPU, n, w, a)
                # the reference's x86 dots accumulate in FMA lanes, the oracle
                # in the generic order: equal up to rounding of the magnitude sum
                scale = float(wf @ np.abs(_deq_act(oracle, at, a, n))) + 1e-30
                assert abs(got - want) <= 2e-6 * scale, (name, r, j, got, want)


def _deq_act(oracle, at, a, n):
    if at == Q8_K:
        d, q, _ = _q8k_fields(a, n)
        return (d[:, None].astype(np.float64) * q).ravel()
    blk = a.reshape(n // 32, -1)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float64).ravel()
    off = 2 if at == Q8_0 else 4
    q = blk[:, off:off + 32].view(np.int8).astype(np.float64)
    return (d[:, None] * q).ravel()


@pytest.mark.parametrize("name", list(WTYPES))
@pytest.mark.parametrize("mode", [ACT_CPU, ACT_Q8_1, ACT_Q8_1_MMA])
def test_vec_dot_equals_dequantised_dot(oracle, name, mode):
    t = WTYPES[name]
    g = load("quant.npz")
    key = f"{name}_{'ones' if t == IQ2_S else 'none'}"
    n = g[key + "_x"].shape[1]
    rng = np.random.default_rng(7)
    at = oracle.act_type(t, mode)
    for r, w in enumerate(rows_of(g[key + "_q"], t, n)):
        wf = oracle.dequantize(t, w, n).astype(np.float64)
        x = rng.standard_normal(n).astype(np.float32)
        a = oracle.quantize_act(at, x)
        af = _deq_act(oracle, at, a, n)
        exact = float(wf @ af)
        got = oracle.vec_dot(t, mode, n, w, a)
        scale = float(np.abs(wf) @ np.abs(af)) + 1e-30
        if t == Q5_0 and mode == ACT_Q8_1:
            # the q8_1 formula d_w (d8 Σ q a - 16 s) uses the block's stored sum s
            # of the unquantised x in place of d8 Σ q_a: the difference is bounded
            # by 16 |d_w| |s - d8 Σ q_a| per block
            dw = np.abs(np.frombuffer(w.tobytes(), np.uint8).reshape(-1, 22)[:, 0:2].copy().view(np.float16)
                        .astype(np.float64).ravel())
            ab = a.reshape(n // 32, 36)
            d8 = ab[:, 0:2].copy().view(np.float16).astype(np.float64).ravel()
            s8 = ab[:, 2:4].copy().view(np.float16).astype(np.float64).ravel()
            sq = ab[:, 4:36].view(np.int8).astype(np.float64).sum(1)
            bound = float(np.sum(16 * dw * np.abs(s8 - d8 * sq))) + 3e-6 * scale
            assert abs(got - exact) <= bound, (r, got, exact, bound)
        elif t == IQ2_S and mode == ACT_Q8_1:
            # integer formula (s0*ls0 + s1*ls1 + (s0+s1)/2)/4 truncates: at most
            # one unit of d*d8 per 32 values
            dw = np.frombuffer(w.tobytes(), np.uint8).reshape(-1, 82)[:, 0:2].copy().view(np.float16).astype(np.float64)
            d8 = np.abs(a.reshape(n // 32, 36)[:, 0:2].copy().view(np.float16).astype(np.float64).ravel())
            bound = float(np.sum(np.repeat(np.abs(dw.ravel()), 8) * d8)) + 1e-6 * scale
            assert abs(got - exact) <= bound, (r, got, exact, bound)
        else:
            assert abs(got - exact) <= 3e-6 * scale, (r, got, exact)


# Known answers for the two q8_1-mode formulas that are not the dot of the
# dequantised operands, worked out by hand from the reference's integer
# arithmetic on blocks built field by field (every scale a power of two, so
# the float steps are exact):
#   vec_dot_iq2_s_q8_1 (vecdotq.cuh:1061-1102): per 32-block
#       sumi = (s0 ls0 + s1 ls1 + (s0 + s1) / 2) / 4 in C integer division
#       (truncation toward zero), times d d8;
#   vec_dot_q5_0_q8_1_impl (vecdotq.cuh:172-198): d5 (d8 sum(q5 q8) - 16 s8)
#       with q5 in 0..31 and s8 the q8_1 block's stored sum, not d8 sum(q8).

def _q8_1_row(d8, s8, q):
    """q8_1 blocks [d fp16][s fp16][32 x int8] from per-block d8, s8 and the
    int8 values q (n values)."""
    nb = len(q) // 32
    a = np.zeros((nb, 36), np.uint8)
    a[:, 0:2] = np.asarray(d8, np.float16).reshape(nb, 1).view(np.uint8)
    a[:, 2:4] = np.asarray(s8, np.float16).reshape(nb, 1).view(np.uint8)
    a[:, 4:36] = np.asarray(q, np.int8).reshape(nb, 32).view(np.uint8)
    return a.ravel()


def _iq2s_super_block(d, groups, scales):
    """One block_iq2_s {d fp16, qs[64], qh[8], scales[8]}: groups maps the
    8-value group l (0..31) to (grid index, sign byte); scales[ib] =
    (ls0, ls1) of 32-block ib."""
    b = np.zeros(82, np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    for l, (idx, sg) in groups.items():
        b[2 + l] = idx & 0xFF
        b[2 + 32 + l] = sg
        b[2 + 64 + l // 4] |= ((idx >> 8) & 3) << (2 * (l % 4))
    for ib, (ls0, ls1) in scales.items():
        b[2 + 64 + 8 + ib] = ls0 | (ls1 << 4)
    return b


def _grid_index_with_first(oracle, v):
    """The first IQ2_S grid index whose value 0 is v (d = 1, ls = 0: the
    dequantised value is v / 8)."""
    for idx in range(1024):
        w = _iq2s_super_block(1.0, {0: (idx, 0)}, {})
        if oracle.dequantize(IQ2_S, w, 256)[0] == v / 8.0:
            return idx
    raise AssertionError(f"no grid entry starts with {v}")


def test_iq2s_q8_1_truncates_toward_zero(oracle):
    i25, i43 = _grid_index_with_first(oracle, 25), _grid_index_with_first(oracle, 43)
    d8 = np.ones(8, np.float32)

    def dot(groups, scales, q, d8=d8):
        return oracle.vec_dot(IQ2_S, ACT_Q8_1, 256, _iq2s_super_block(1.0, groups, scales),
                              _q8_1_row(d8, np.zeros(8), q))

    q = np.zeros(256, np.int64)
    q[0] = -1
    # s0 = -25, ls0 = 3: (-75 + (-25)/2) / 4 = (-75 - 12) / 4 = -87 / 4 = -21
    # (floor division would give -22, rounding -22, exact arithmetic -21.875)
    assert dot({0: (i25, 0)}, {0: (3, 0)}, q) == -21.0
    q[0] = 1
    assert dot({0: (i25, 0)}, {0: (3, 0)}, q) == 21.0            # 87 / 4
    assert dot({0: (i25, 0x01)}, {0: (3, 0)}, q) == -21.0         # sign bit 0: value -25
    # s0 = -25 (ls0 3), s1 = 43 (ls1 5, group 2 = values 16..23):
    # (-75 + 215 + 18/2) / 4 = 149 / 4 = 37
    q[0], q[16] = -1, 1
    groups = {0: (i25, 0), 2: (i43, 0)}
    assert dot(groups, {0: (3, 5)}, q) == 37.0
    # plus 32-block 1 at d8 = 1/2: s0 = 75 (q = 3), ls = 0: (75 / 2) / 4 = 37 / 4 = 9
    q[32] = 3
    groups[4] = (i25, 0)
    d8b = d8.copy()
    d8b[1] = 0.5
    assert dot(groups, {0: (3, 5)}, q, d8b) == 37.0 + 4.5


def test_q5_0_q8_1_uses_the_stored_sum(oracle):
    # q5 values: 16 everywhere (weight 0) but value 0 = 31 and value 17 = 5
    b = np.zeros(22, np.uint8)
    b[0:2] = np.array([1.0], np.float16).view(np.uint8)
    qh = 1 << 0                                   # value 0's fifth bit
    for j in range(16):
        if j != 0:
            qh |= 1 << j                          # 16 = 0b10000
        if j != 1:
            qh |= 1 << (j + 16)
    b[2:6] = np.array([qh], np.uint32).view(np.uint8)
    lo = np.zeros(16, np.int64)
    hi = np.zeros(16, np.int64)
    lo[0] = 15                                    # 15 + 16 = 31
    hi[1] = 5                                     # value 17: fifth bit clear
    b[6:22] = (lo | (hi << 4)).astype(np.uint8)
    assert np.array_equal(oracle.dequantize(Q5_0, b, 32)[[0, 17, 5]], [15.0, -11.0, 0.0])
    q = np.zeros(32, np.int64)
    q[0], q[17] = 2, -3
    # sum(q5 q8) = 31*2 + 5*(-3) = 47; stored s8 = 7 (not d8 sum q8 = -1):
    # 1 * (47 - 16 * 7) = -65 (the (q5 - 16) form would give 63)
    assert oracle.vec_dot(Q5_0, ACT_Q8_1, 32, b, _q8_1_row([1.0], [7.0], q)) == -65.0
    # and with s8 = d8 sum(q8) the two forms agree
    assert oracle.vec_dot(Q5_0, ACT_Q8_1, 32, b, _q8_1_row([1.0], [-1.0], q)) == 63.0


# ------------------------------------------------------------ geglu

def test_geglu_table_matches_reference(oracle):
    g = load("geglu.npz")
    got = oracle.geglu(g["g"], g["u"], GELU_TABLE)
    assert np.array_equal(got.view(np.uint32), g["out"].view(np.uint32))


def test_geglu_tanh_closed_form(oracle):
    x = np.linspace(-8, 8, 4001).astype(np.float32)
    u = np.ones_like(x)
    got = oracle.geglu(x, u, GELU_TANH).astype(np.float64)
    xd = x.astype(np.float64)
    want = 0.5 * xd * (1 + np.tanh(math.sqrt(2 / math.pi) * (xd + 0.044715 * xd ** 3)))
    assert np.allclose(got, want, rtol=2e-6, atol=2e-7)
    tab = oracle.geglu(x, u, GELU_TABLE).astype(np.float64)
    assert np.allclose(tab, want, rtol=2e-3, atol=2e-3)      # fp16 table


# ------------------------------------------------------------ router

def test_router_closed_forms(oracle):
    T, d, E, k = 2, 64, 16, 4
    x = np.ones((T, d), np.float32)
    ids, w, p = oracle.router(x, np.zeros((E, d), np.float32), None, k)
    assert np.array_equal(ids, np.tile(np.arange(k), (T, 1)))      # ties go to the lower index
    assert np.allclose(w, 1.0 / k, rtol=0, atol=1e-7)
    bias = np.arange(E, dtype=np.float32) * 0.1
    ids, w, p = oracle.router(x, np.zeros((E, d), np.float32), bias, k)
    assert np.array_equal(ids[0], np.arange(E - 1, E - 1 - k, -1))
    rng = np.random.default_rng(8)
    x = rng.standard_normal((T, d)).astype(np.float32)
    wr = (rng.standard_normal((E, d)) * 0.3).astype(np.float32)
    ids, w, p = oracle.router(x, wr, None, k)
    assert np.allclose(p.sum(1), 1.0, atol=1e-6)
    for t in range(T):
        assert len(set(ids[t])) == k
        assert np.all(np.diff(p[t, ids[t]]) <= 0)
        assert np.array_equal(np.sort(ids[t]), np.sort(np.argsort(-p[t], kind="stable")[:k]))
        assert abs(w[t].sum() - 1.0) <= 1e-6
        logits = x[t].astype(np.float64) @ wr.T.astype(np.float64)
        ref_p = np.exp(logits - logits.max())
        ref_p /= ref_p.sum()
        assert np.allclose(p[t], ref_p, rtol=1e-5, atol=1e-7)


# ------------------------------------------------------------ matvec / layer

def test_mul_mat_id_matches_reference(oracle):
    g = load("mmid.npz")
    for name, t in WTYPES.items():
        d_in, d_out, n_pool = (int(v) for v in g[f"{name}_shape"])
        w = g[f"{name}_w"]
        eb = row_size(t, d_in) * d_out
        for i, e in enumerate(g[f"{name}_ids"]):
            got = oracle.matvec(t, ACT_CPU, w[e * eb:(e + 1) * eb], d_out, d_in, g[f"{name}_x"][i])
            want = g[f"{name}_y"][i]
            assert np.max(np.abs(got - want)) <= 2e-6 * max(1.0, np.abs(want).max()), (name, i)


def single_tier_layer(g, tag, sfx=""):
    d, F, E, K, T = (int(v) for v in g[f"{tag}{sfx}_shape"])
    gt, dt = (int(v) for v in g[f"{tag}_types"])
    hot = tag == "hot"
    L = SimpleNamespace(d_model=d, n_ff=F, n_expert=E, top_k=K, k_slots=E if hot else 0,
                        hot_gu_type=gt, hot_dn_type=dt, cold_gu_type=gt, cold_dn_type=dt,
                        hot_gu=g[f"{tag}_gu"] if hot else None, hot_dn=g[f"{tag}_dn"] if hot else None,
                        cold_gu=None if hot else g[f"{tag}_gu"], cold_dn=None if hot else g[f"{tag}_dn"],
                        exp_slot=np.arange(E, dtype=np.int32) if hot else np.full(E, -1, np.int32),
                        slot_exp=np.arange(E, dtype=np.int32) if hot else np.full(1, -1, np.int32),
                        slot_state=np.full(E, 2, np.int32) if hot else np.zeros(1, np.int32),
                        s_hot=None, s_cold=None)
    return L


@pytest.mark.parametrize("tag", ["cold", "hot"])
@pytest.mark.parametrize("sfx", ["", "_long"])
def test_layer_matches_reference(oracle, tag, sfx):
    g = load("layer.npz")
    L = single_tier_layer(g, tag, sfx)
    x = g[f"{tag}{sfx}_x"]
    ids, w, _ = oracle.router(x, g[f"{tag}_router_w"], g[f"{tag}_bias"], L.top_k)
    assert np.array_equal(ids, g[f"{tag}{sfx}_ids"])
    assert np.allclose(w, g[f"{tag}{sfx}_w"], rtol=1e-6, atol=1e-7)
    out, _ = oracle.moe_experts(L, x, g[f"{tag}{sfx}_ids"], g[f"{tag}{sfx}_w"])
    want = g[f"{tag}{sfx}_out"]
    err = np.linalg.norm(out - want) / np.linalg.norm(want)
    assert err <= 1e-6, err


def test_dual_mask_brute_force(oracle):
    """Pairs read the hot pool exactly when the READY predicate holds."""
    g = load("layer.npz")
    hot = single_tier_layer(g, "hot")
    cold = single_tier_layer(g, "cold")
    E, K = hot.n_expert, hot.top_k
    rng = np.random.default_rng(9)
    # a dual layer: hot pool = the "hot" pools for slots, cold pool = the "cold" pools;
    # slot s holds expert perm[s]; some slots not READY, one slot_exp mismatched
    ks = 5
    perm = rng.permutation(E)[:ks]
    gb, db = row_size(hot.hot_gu_type, hot.d_model) * 2 * hot.n_ff, row_size(hot.hot_dn_type, hot.n_ff) * hot.d_model
    hot_gu = np.concatenate([hot.hot_gu[e * gb:(e + 1) * gb] for e in perm])
    hot_dn = np.concatenate([hot.hot_dn[e * db:(e + 1) * db] for e in perm])
    exp_slot = np.full(E, -1, np.int32)
    slot_exp = perm.astype(np.int32).copy()
    state = np.array([2, 1, 2, 0, 2], np.int32)             # FILLING and FREE slots are cold
    exp_slot[perm] = np.arange(ks)
    slot_exp[4] = (perm[4] + 1) % E                          # mirror disagreement: cold
    s_hot = (1 + rng.random(ks)).astype(np.float32)
    s_cold = (1 + rng.random(E)).astype(np.float32)
    dual = SimpleNamespace(**{**cold.__dict__, "k_slots": ks, "hot_gu_type": hot.hot_gu_type,
                              "hot_dn_type": hot.hot_dn_type, "hot_gu": hot_gu, "hot_dn": hot_dn,
                              "exp_slot": exp_slot, "slot_exp": slot_exp, "slot_state": state,
                              "s_hot": s_hot, "s_cold": s_cold})
    x = g["cold_x"]
    T = x.shape[0]
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    ids[0, 0] = perm[0]; ids[1, 0] = perm[1]; ids[2, 0] = perm[4]    # READY, FILLING, mismatched
    w = rng.random((T, K)).astype(np.float32)
    out, yp = oracle.moe_experts(dual, x, ids, w)
    _, y_hot = oracle.moe_experts(hot, x, ids, w)
    _, y_cold = oracle.moe_experts(cold, x, ids, w)
    want = np.zeros_like(out, dtype=np.float64)
    for t in range(T):
        for k in range(K):
            e = int(ids[t, k])
            s = int(exp_slot[e])
            is_hot = 0 <= s < ks and state[s] == 2 and slot_exp[s] == e
            y = y_hot[t * K + k] * s_hot[s] if is_hot else y_cold[t * K + k] * s_cold[e]
            assert np.allclose(yp[t * K + k], y, rtol=1e-6, atol=1e-7), (t, k, is_hot)
            want[t] += float(w[t, k]) * y.astype(np.float64)
    assert np.allclose(out, want, rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------ live reference

@pytest.fixture(scope="module")
def live_ref():
    try:
        from oracle import Ref
        return Ref()
    except (FileNotFoundError, OSError):
        pytest.skip("oracle/_ref not built (needs the reference sources)")


@pytest.mark.parametrize("name", list(WTYPES))
def test_live_reference_random_rows(oracle, live_ref, name):
    t = WTYPES[name]
    n = 1024 if t in (Q4_K, IQ2_S) else 512
    rng = np.random.default_rng(10 + t)
    x = (rng.standard_normal((6, n)) * 0.02).astype(np.float32)
    im = np.ones(n, np.float32) if t == IQ2_S else None
    q = live_ref.quantize(t, x, im)
    at = live_ref.vec_dot_type(t)
    for r, w in enumerate(rows_of(q, t, n)):
        assert np.array_equal(oracle.dequantize(t, w, n), live_ref.dequantize(t, w, n))
        a = rng.standard_normal(n).astype(np.float32)
        aq = live_ref.quantize_act(at, a)
        assert np.array_equal(oracle.quantize_act(at, a), aq)
        want = live_ref.vec_dot(t, n, w, aq)
        assert abs(oracle.vec_dot(t, ACT_CPU, n, w, aq) - want) <= 2e-6 * max(1.0, abs(want))


@pytest.mark.parametrize("T,n_hot", [(3, 6), (40, 10), (4, 0)])
def test_reference_dual_layer_matches_oracle(oracle, live_ref, T, n_hot):
    """The CPU baseline's dual-precision layer (the reference's ggml graph for
    the routing and the hot pairs, its CPU cold executor for the cold pairs)
    against the oracle's layer in the CPU activation mode: the same routing,
    the same hot/cold split, the same outputs."""
    import llapis_amd as la
    from helpers import SMALL, layer, rel_l2, tokens
    rng = np.random.default_rng(n_hot)
    hot = sorted(rng.choice(SMALL.n_expert, n_hot, replace=False).tolist()) if n_hot else []
    lay = layer(SMALL, 120 + n_hot, hot)
    x = tokens(130 + T, T, SMALL.d_model)
    rd = live_ref.dual(lay, T, n_threads=2)
    out, ids, n_hot_pairs = rd.run(x)
    ids_o, w_o, _ = oracle.router(x, lay.router_w, lay.router_b, SMALL.top_k)
    assert np.array_equal(ids, ids_o)
    assert n_hot_pairs == sum(lay.residency.is_hot(int(e)) for e in ids.ravel())
    out_o, _ = oracle.moe_experts(lay, x, ids_o, w_o)
    assert rel_l2(out, out_o) <= 1e-6, rel_l2(out, out_o)


def test_reference_avx512_build_matches_oracle(oracle):
    """The AVX-512 build of the reference's ggml (the CPU baseline on hosts
    that have it) computes the same layer as the oracle."""
    import bench
    from helpers import SMALL, layer, rel_l2, tokens
    from oracle import Ref
    _, _, isa, lib = bench.host_cpu()
    if isa != "avx512":
        pytest.skip("no AVX-512 build or host support")
    ref = Ref(str(lib))
    lay = layer(SMALL, 140, [])
    x = tokens(141, 3, SMALL.d_model)
    rl = ref.layer(lay.router_w, lay.router_b, SMALL.top_k, SMALL.cold_gu_type, lay.cold_gu, SMALL.cold_dn_type,
                   lay.cold_dn, SMALL.n_ff, 3)
    out, ids, w = rl.run(x, 2)
    ids_o, w_o, _ = oracle.router(x, lay.router_w, lay.router_b, SMALL.top_k)
    assert np.array_equal(ids, ids_o)
    out_o, _ = oracle.moe_experts(lay, x, ids_o, w_o)
    assert rel_l2(out, out_o) <= 1e-5, rel_l2(out, out_o)
