#!/usr/bin/env python3
"""Write the golden vectors under tests/golden/ from the reference's own ggml
CPU code: oracle/_ref/libggml_ref.so, compiled by oracle/Makefile from the
reference's sources (third_party/llama/ggml).  Every input is stored next to
the outputs, so the fixtures are self-contained data.

    make -C oracle ref REF=/path/to/reference && python tests/golden/make_golden.py

Files (numpy .npz, no pickled objects):
  quant.npz    quantiser bytes + dequantised floats per weight type, including
               edge rows (zeros, a spike, a constant, a wide range, denormal-
               size values) and importance-matrix variants
               (ggml_quantize_chunk, ggml.c:7721-7800; dequantize_row_*).
  iq2s_grid.npz  dequantised IQ2_S blocks that enumerate all 1024 grid
               indices with unit scale, without and with sign bytes
               (ggml-quants.c:2471-2498, ggml-common.h:748).
  act.npz      q8_K and q8_0 activation bytes of the x86 build
               (ggml-quants.c:2696-2733; ggml-cpu/arch/x86/quants.c:302).
  dot.npz      vec_dot of every quantised row with every activation
               (ggml-cpu/arch/x86/quants.c: q4_K, iq2_s, q5_0, iq4_nl).
  geglu.npz    ggml_geglu_split outputs of the CPU path (fp16 GELU table).
  mmid.npz     ggml mul_mat_id over small pools with repeated ids.
  layer.npz    whole single-tier MoE layers of the CPU graph (router mul_mat,
               soft_max, argsort_top_k, get_rows, sum_rows, clamp, div,
               mul_mat_id gate_up, geglu_split, mul_mat_id down, mul, adds;
               llama-graph.cpp:1507-1850) for two tiers of formats, at 3 and
               at 40 tokens.
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT / "oracle"))

from oracle import F32, IQ2_S, IQ4_NL, Q4_K, Q5_0, Q8_0, Q8_K, Ref, row_size  # noqa: E402

WTYPES = {"q4_K": Q4_K, "iq2_s": IQ2_S, "q5_0": Q5_0, "iq4_nl": IQ4_NL}
BLOCK = {Q4_K: 256, IQ2_S: 256, Q5_0: 32, IQ4_NL: 32}


def edge_rows(rng, n):
    rows = [
        np.zeros(n),                                        # all zero
        np.where(np.arange(n) == n // 3, 1.5, 0.0),         # a single spike
        np.full(n, -0.75),                                  # constant negative
        rng.standard_normal(n) * np.logspace(-4, 1, n),     # wide dynamic range
        rng.standard_normal(n) * 1e-30,                     # tiny magnitudes
        rng.standard_normal(n) * 0.02,                      # the expert-weight distribution
        rng.standard_normal(n),                             # unit normal
        np.abs(rng.standard_normal(n)),                     # one-signed
    ]
    return np.stack(rows).astype(np.float32)


def make_quant(ref, rng):
    out = {}
    for name, t in WTYPES.items():
        n = 512 if BLOCK[t] == 256 else 256
        x = edge_rows(rng, n)
        variants = [("none", None)]
        if t in (IQ2_S, IQ4_NL):
            variants.append(("ones", np.ones(n, np.float32)))
            variants.append(("ramp", (0.25 + rng.random(n)).astype(np.float32)))
        for vname, im in variants:
            q = ref.quantize(t, x, im)
            rs = row_size(t, n)
            deq = np.stack([ref.dequantize(t, q[r * rs:(r + 1) * rs], n) for r in range(x.shape[0])])
            key = f"{name}_{vname}"
            out[f"{key}_x"] = x
            out[f"{key}_imatrix"] = im if im is not None else np.zeros(0, np.float32)
            out[f"{key}_q"] = q
            out[f"{key}_deq"] = deq
    return out


def make_iq2s_grid(ref, rng):
    """32 blocks x 32 groups = every grid index once; d = 8 (fp16) and scale
    nibble 0 give a per-value factor 8 * 0.5 * 0.25 = 1, so the dequantised
    bytes are the codebook values themselves."""
    blocks_plain, blocks_signed = [], []
    for b in range(32):
        blk = np.zeros(82, np.uint8)
        blk[0:2] = np.frombuffer(np.float16(8.0).tobytes(), np.uint8)
        for g in range(32):
            idx = 32 * b + g
            blk[2 + g] = idx & 0xFF
            blk[66 + g // 4] |= ((idx >> 8) & 3) << (2 * (g % 4))
        blocks_plain.append(blk.copy())
        blk[34:66] = rng.integers(0, 256, 32, dtype=np.uint8)      # sign bytes
        blk[74:82] = rng.integers(0, 256, 8, dtype=np.uint8)       # both scale nibbles
        blocks_signed.append(blk)
    plain = np.concatenate(blocks_plain)
    signed = np.concatenate(blocks_signed)
    return {
        "plain_q": plain, "plain_deq": ref.dequantize(IQ2_S, plain, 32 * 256),
        "signed_q": signed, "signed_deq": ref.dequantize(IQ2_S, signed, 32 * 256),
    }


def make_act(ref, rng):
    n = 512
    x = edge_rows(rng, n)
    ties = np.zeros(n, np.float32)
    ties[[7, 300]] = [-2.0, 2.0]               # equal |max| with opposite signs: the first one wins
    ties[[8, 301]] = [1.0, -1.0]
    x = np.vstack([x, ties[None]])
    out = {"x": x}
    out["q8_K"] = np.stack([ref.quantize_act(Q8_K, r) for r in x])
    out["q8_0"] = np.stack([ref.quantize_act(Q8_0, r) for r in x])
    return out


def make_dot(ref, quant, act):
    out = {}
    for name, t in WTYPES.items():
        vname = "ones" if t == IQ2_S else "none"
        x = quant[f"{name}_{vname}_x"]
        q = quant[f"{name}_{vname}_q"]
        n = x.shape[1]
        at = ref.vec_dot_type(t)
        rs = row_size(t, n)
        acts = act["x"][:, :n]
        aq = np.stack([ref.quantize_act(at, a) for a in acts])
        vals = np.array([[ref.vec_dot(t, n, q[r * rs:(r + 1) * rs], aq[j]) for j in range(len(acts))]
                         for r in range(x.shape[0])], np.float32)
        out[f"{name}_act_type"] = np.int32(at)
        out[f"{name}_act_q"] = aq
        out[f"{name}_w_q"] = q
        out[f"{name}_n"] = np.int32(n)
        out[f"{name}_dot"] = vals
    return out


def make_geglu(ref, rng):
    g = np.concatenate([np.linspace(-12, 12, 2401), [-10.0, 10.0, -10.000001, 10.000001, 0.0, -0.0, 1e-8, -1e-8],
                        rng.standard_normal(1000) * 3]).astype(np.float32)
    g = g[: (g.size // 8) * 8]
    u = rng.standard_normal(g.size).astype(np.float32)
    return {"g": g, "u": u, "out": ref.geglu(g[None], u[None])[0]}


def make_mmid(ref, rng):
    out = {}
    for name, t in WTYPES.items():
        d_in = 512 if BLOCK[t] == 256 else 256
        d_out, n_pool = 32, 5
        w = rng.standard_normal((n_pool * d_out, d_in)).astype(np.float32) * 0.02
        im = np.ones(d_in, np.float32) if t == IQ2_S else None
        wq = ref.quantize(t, w, im)
        x = rng.standard_normal((3, d_in)).astype(np.float32)
        ids = np.array([4, 0, 4, 2, 1, 2], np.int32)      # repeats; 2 columns per token
        # column i of x for channel i // 2
        xs = np.repeat(x, 2, axis=0)
        y = ref.mul_mat_id(t, wq, d_in, d_out, n_pool, xs, ids)
        out.update({f"{name}_w": wq, f"{name}_x": xs, f"{name}_ids": ids, f"{name}_y": y,
                    f"{name}_shape": np.array([d_in, d_out, n_pool], np.int32)})
    return out


def make_layer(ref, rng):
    out = {}
    d, F, E, K, T = 256, 32, 8, 2, 3
    for tag, (gt, dt) in {"cold": (IQ2_S, IQ4_NL), "hot": (Q4_K, Q5_0)}.items():
        w_r = (rng.standard_normal((E, d)) * 0.02).astype(np.float32)
        bias = (rng.standard_normal(E) * 0.05).astype(np.float32)
        gu = (rng.standard_normal((E * 2 * F, d)) * 0.02).astype(np.float32)
        dn = (rng.standard_normal((E * d, F)) * 0.02).astype(np.float32)
        cold = tag == "cold"
        gq = ref.quantize(gt, gu, np.ones(d, np.float32) if cold else None)
        dq = ref.quantize(dt, dn, np.ones(F, np.float32) if cold else None)
        out.update({f"{tag}_router_w": w_r, f"{tag}_bias": bias, f"{tag}_gu": gq, f"{tag}_dn": dq,
                    f"{tag}_types": np.array([gt, dt], np.int32)})
        # a decode batch and a prefill-sized batch through the same layer
        for sfx, TT in (("", T), ("_long", 40)):
            x = rng.standard_normal((TT, d)).astype(np.float32)
            rl = ref.layer(w_r, bias, K, gt, gq, dt, dq, F, TT)
            o, ids, w = rl.run(x, 1, True)
            del rl
            out.update({f"{tag}{sfx}_x": x, f"{tag}{sfx}_out": o, f"{tag}{sfx}_ids": ids, f"{tag}{sfx}_w": w,
                        f"{tag}{sfx}_shape": np.array([d, F, E, K, TT], np.int32)})
    return out


def main():
    ref = Ref()
    rng = np.random.default_rng(20260512)
    quant = make_quant(ref, rng)
    np.savez_compressed(HERE / "quant.npz", **quant)
    np.savez_compressed(HERE / "iq2s_grid.npz", **make_iq2s_grid(ref, rng))
    act = make_act(ref, rng)
    np.savez_compressed(HERE / "act.npz", **act)
    np.savez_compressed(HERE / "dot.npz", **make_dot(ref, quant, act))
    np.savez_compressed(HERE / "geglu.npz", **make_geglu(ref, rng))
    np.savez_compressed(HERE / "mmid.npz", **make_mmid(ref, rng))
    np.savez_compressed(HERE / "layer.npz", **make_layer(ref, rng))
    for p in sorted(HERE.glob("*.npz")):
        print(f"{p.name}: {p.stat().st_size} bytes")


if __name__ == "__main__":
    main()
