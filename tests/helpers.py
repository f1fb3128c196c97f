"""Shared test helpers: synthetic layers at test sizes and error metrics."""
import numpy as np

import llapis_amd as la
from llapis_amd import IQ2_S, IQ4_NL, Q4_K, Q5_0, LayerSpec

SMALL = LayerSpec(d_model=512, n_ff=96, n_expert=16, top_k=4)
# the benchmark's per-expert shapes with fewer experts (fast to quantise)
FULL16 = LayerSpec(d_model=2816, n_ff=704, n_expert=16, top_k=8)


def rel_l2(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))


def all_hot(spec):
    return list(range(spec.n_expert))


_cache = {}


def layer(spec, seed, hot, scales=False, router_bias=None):
    key = (spec.d_model, spec.n_ff, spec.n_expert, spec.top_k, spec.hot_gu_type, spec.hot_dn_type,
           spec.cold_gu_type, spec.cold_dn_type, seed, tuple(hot), scales,
           None if router_bias is None else router_bias.tobytes())
    if key not in _cache:
        _cache[key] = la.make_layer(spec, seed, hot, router_bias=router_bias, scales=scales)
    return _cache[key]


def tokens(seed, T, d):
    return la.synth_normal(seed, T * d).reshape(T, d)
