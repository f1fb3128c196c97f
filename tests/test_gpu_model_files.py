"""GPU: a dual layer loaded from model files into HBM.  The cold pools and
their scales come from a GGUF (the stacked blk.0.ffn_*_exps tensors, read by
llapis_gguf_upload), the hot experts' Q4_K / Q5_0 pages and scales from an
expert store (llapis_store_upload, checksums checked as the bytes stream).
The device pools equal the in-memory ones bit for bit and the layer's output
is identical to the layer uploaded from memory; a corrupted page is refused."""
import ctypes as C
import sys

import numpy as np
import pytest

import llapis_amd as la
from llapis_amd import _lib as L
from gguf_file import layer_tensors, write_gguf
from helpers import FULL16, layer, rel_l2, tokens

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def test_layer_from_gguf_and_store(gpu, oracle, tmp_path):
    import torch
    lib = la.lib()
    spec = FULL16
    E = spec.n_expert
    hot = [1, 4, 6, 9, 12]
    lay = layer(spec, 93, hot, scales=True)
    say("model files: writing the GGUF and the expert store")
    gguf = tmp_path / "layer.gguf"
    write_gguf(gguf, layer_tensors(lay, il=0), alignment=64)
    gb, db = spec.gu_bytes(spec.hot_gu_type), spec.dn_bytes(spec.hot_dn_type)
    idx, pack = tmp_path / "layer.experts.index", tmp_path / "layer.experts.pack"
    info = L.MoertStoreInfo()
    info.source_uuid, info.arch, info.n_layers, info.n_expert = 1, b"gemma4", 1, E
    w = lib.moert_store_writer_open(str(idx).encode(), str(pack).encode(), C.byref(info))
    assert w
    for s, e in enumerate(hot):
        for kind, is_scale, qt, data in ((0, 0, spec.hot_gu_type, lay.hot_gu[s * gb:(s + 1) * gb]),
                                         (1, 0, spec.hot_dn_type, lay.hot_dn[s * db:(s + 1) * db]),
                                         (1, 1, 0, lay.s_hot[s:s + 1].view(np.uint8))):
            d = np.ascontiguousarray(data)
            sh = (C.c_int64 * 4)(1, 1, 1, 1)
            assert lib.moert_store_writer_add_page(w, 0, e, kind, is_scale, qt, qt, 0, sh, 1, d.ctypes.data,
                                                   d.nbytes) == 1
    assert lib.moert_store_writer_close(w) == 1
    assert lib.moert_store_verify(str(idx).encode()) == 0

    dl_mem = la.DeviceLayer(lay, gpu)
    dl = la.DeviceLayer(lay, gpu)
    for t in (dl.hot_gu, dl.hot_dn, dl.cold_gu, dl.cold_dn, dl.s_hot, dl.s_cold):
        t.zero_()
    stream = torch.cuda.current_stream().cuda_stream
    say("model files: GGUF -> cold pools")
    g = lib.llapis_gguf_open(str(gguf).encode())
    assert g, lib.llapis_files_last_error()
    try:
        for kind, is_scale, dst in ((0, 0, dl.cold_gu), (1, 0, dl.cold_dn), (1, 1, dl.s_cold)):
            grp = L.LlapisPageGroup()
            assert lib.llapis_gguf_expert_group(g, 0, kind, is_scale, E, C.byref(grp)) == 0
            assert grp.bytes_per_expert * E == dst.numel() * dst.element_size()
            assert lib.llapis_gguf_upload(g, C.byref(grp), 0, E, dst.data_ptr(), stream) == 0, \
                lib.llapis_files_last_error()
    finally:
        lib.llapis_gguf_close(g)
    say("model files: store -> hot slots")
    r = lib.moert_store_reader_open(str(idx).encode(), 1)
    assert r
    ids = (C.c_int32 * len(hot))(*hot)
    try:
        for kind, is_scale, dst, stride in ((0, 0, dl.hot_gu, gb), (1, 0, dl.hot_dn, db), (1, 1, dl.s_hot, 4)):
            assert lib.llapis_store_upload(r, 0, kind, is_scale, ids, len(hot), dst.data_ptr(), stride, 1,
                                           stream) == 0, lib.llapis_files_last_error()
    finally:
        lib.moert_store_reader_free(r)
    torch.cuda.synchronize()
    for name in ("hot_gu", "hot_dn", "cold_gu", "cold_dn", "s_hot", "s_cold"):
        assert torch.equal(getattr(dl, name), getattr(dl_mem, name)), name
    for T in (1, 4, 40):
        x = torch.from_numpy(tokens(40 + T, T, spec.d_model)).to(gpu)
        a, ia, wa = dl.forward(x)
        b, ib, wb = dl_mem.forward(x)
        torch.cuda.synchronize()
        assert torch.equal(ia, ib) and torch.equal(a, b), T
        out_o, _ = oracle.moe_experts(lay, x.cpu().numpy(), ia.cpu().numpy(), wa.cpu().numpy(), la.ACT_CPU,
                                      la.GELU_TABLE)
        err = rel_l2(a.cpu().numpy(), out_o)
        say(f"  T={T}: identical to the layer from memory; rel_l2 vs oracle {err:.2e}")
        assert err <= (1e-4 if T <= 4 else 5e-4)
    # a corrupted page: the upload with verification is refused
    raw = bytearray(pack.read_bytes())
    raw[4096] ^= 1
    pack.write_bytes(bytes(raw))
    r = lib.moert_store_reader_open(str(idx).encode(), 1)
    try:
        scratch = torch.zeros(len(hot) * gb, dtype=torch.uint8, device=gpu)
        assert lib.llapis_store_upload(r, 0, 0, 0, ids, len(hot), scratch.data_ptr(), gb, 1, stream) == -1
        assert b"checksum" in lib.llapis_files_last_error()
    finally:
        lib.moert_store_reader_free(r)
