"""llapis_moe_ffn_noalloc (the entry point that allocates nothing: its
scratch is a fixed device array in the library) against llapis_moe_ffn with a
workspace, through the C ABI: identical routing and outputs, bit for bit, on
consecutive calls that share the array -- a larger call, then smaller ones
(fewer tokens, a smaller layer) -- and a call too large for the array is
refused without touching the outputs."""
import ctypes as C
import sys

import numpy as np
import pytest

import llapis_amd as la
from helpers import FULL16, SMALL, layer, tokens

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _layer(spec, seed, n_hot):
    rng = np.random.default_rng(seed)
    hot = sorted(rng.choice(spec.n_expert, n_hot, replace=False).tolist())
    return layer(spec, seed, hot, scales=True)


def _both(gpu, dl, x):
    """(out, ids, w) of llapis_moe_ffn (workspace) and of llapis_moe_ffn_noalloc."""
    import torch
    T = x.shape[0]
    sp = dl.layer.spec
    xd = torch.from_numpy(x).to(gpu)
    ref = tuple(t.clone() for t in dl.forward(xd))
    out = torch.full((T, sp.d_model), float("nan"), device=gpu)
    ids = torch.full((T, sp.top_k), -1, dtype=torch.int32, device=gpu)
    w = torch.full((T, sp.top_k), float("nan"), device=gpu)
    d = dl.desc()
    s = torch.cuda.current_stream().cuda_stream
    rc = la.lib().llapis_moe_ffn_noalloc(C.byref(d), xd.data_ptr(), None, T, out.data_ptr(), ids.data_ptr(),
                                          w.data_ptr(), s)
    assert rc == 0, la.lib().llapis_last_error()
    torch.cuda.synchronize()
    return ref, (out, ids, w)


@pytest.mark.parametrize("act_mode,gelu_mode", [(la.ACT_CPU, la.GELU_TABLE), (la.ACT_Q8_1, la.GELU_TANH)])
def test_noalloc_matches_workspace_entry(gpu, act_mode, gelu_mode):
    import torch
    cases = [(FULL16, 61, 7, 4), (FULL16, 61, 7, 1), (SMALL, 62, 5, 3), (FULL16, 63, 9, 24), (SMALL, 62, 5, 2)]
    for spec, seed, n_hot, T in cases:
        name = "FULL16" if spec is FULL16 else "SMALL"
        say(f"noalloc {name} hot={n_hot} T={T} act={act_mode}")
        dl = la.DeviceLayer(_layer(spec, seed, n_hot), gpu, act_mode, gelu_mode)
        ref, got = _both(gpu, dl, tokens(800 + T, T, spec.d_model))
        for a, b, what in zip(ref, got, ("out", "ids", "weights")):
            assert torch.equal(a, b), (name, T, what)


def test_noalloc_refuses_a_call_beyond_its_array(gpu):
    import torch
    say("noalloc refuses T=512")
    spec = FULL16
    dl = la.DeviceLayer(_layer(spec, 61, 7), gpu)
    T = 512
    need = int(la.lib().llapis_moe_ffn_workspace_size(C.byref(dl.desc()), T))
    assert need > la._lib.NOALLOC_SCRATCH_BYTES
    x = torch.from_numpy(tokens(5, T, spec.d_model)).to(gpu)
    out = torch.full((T, spec.d_model), 7.0, device=gpu)
    d = dl.desc()
    rc = la.lib().llapis_moe_ffn_noalloc(C.byref(d), x.data_ptr(), None, T, out.data_ptr(), None, None,
                                          torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc != 0 and b"bytes of scratch" in la.lib().llapis_last_error()
    assert bool((out == 7.0).all())
    # the next call that fits still works
    ref, got = _both(gpu, dl, tokens(6, 2, spec.d_model))
    assert all(torch.equal(a, b) for a, b in zip(ref, got))


@pytest.mark.parametrize("T", [1, 4, 40])
def test_noalloc_captured_in_a_graph(gpu, T):
    """Three llapis_moe_ffn_noalloc calls captured in one HIP graph (one
    eager call first, as any capture is warmed up): every replay, with eager
    no-alloc calls on the same fixed array between replays, reproduces the
    eager llapis_moe_ffn results bit for bit, and the capture records no
    clearing of the array (each call writes its scratch before reading it)."""
    import torch
    say(f"noalloc graph replays T={T}")
    spec = FULL16
    dl = la.DeviceLayer(_layer(spec, 64 + T, 6), gpu)
    xs = [torch.from_numpy(tokens(700 + 10 * T + i, T, spec.d_model)).to(gpu) for i in range(3)]
    eager = [tuple(t.clone() for t in dl.forward(x)) for x in xs]
    torch.cuda.synchronize()
    outs = [(torch.empty(T, spec.d_model, device=gpu), torch.empty(T, spec.top_k, dtype=torch.int32, device=gpu),
             torch.empty(T, spec.top_k, device=gpu)) for _ in range(3)]
    d = dl.desc()
    s = torch.cuda.Stream()

    def calls(stream):
        for x, (o, i, w) in zip(xs, outs):
            rc = la.lib().llapis_moe_ffn_noalloc(C.byref(d), x.data_ptr(), None, T, o.data_ptr(), i.data_ptr(),
                                                  w.data_ptr(), stream)
            assert rc == 0, la.lib().llapis_last_error()

    with torch.cuda.stream(s):
        calls(s.cuda_stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        calls(s.cuda_stream)
    torch.cuda.synchronize()
    scratch_o = torch.empty(T, spec.d_model, device=gpu)
    for rep in range(4):
        for o, i, w in outs:
            o.fill_(float("nan"))
            i.fill_(-1)
        x = xs[(rep + 1) % 3]
        rc = la.lib().llapis_moe_ffn_noalloc(C.byref(d), x.data_ptr(), None, T, scratch_o.data_ptr(), None, None,
                                              torch.cuda.current_stream().cuda_stream)
        assert rc == 0
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for (o, i, w), (oe, ie, we) in zip(outs, eager):
            assert torch.equal(i, ie), rep
            assert torch.equal(w, we), rep
            assert torch.equal(o, oe), rep
