"""Model files, CPU only: the GGUF reader against ggml's own gguf.cpp (built
from the reference's sources into oracle/_ref/libggml_ref.so), and the expert
store against the reference's moert/memmgr/store.cpp (oracle/_ref/
libmoert_store_ref.so), in both directions: stores either side writes, the
other reads byte for byte, and both catch a corrupted page."""
import ctypes as C
import os
from pathlib import Path

import numpy as np
import pytest

import llapis_amd as la
from llapis_amd import _lib as L
from gguf_file import layer_tensors, nbytes, write_gguf

ROOT = Path(__file__).resolve().parents[1]
REF_GGML = ROOT / "oracle" / "_ref" / "libggml_ref.so"
REF_STORE = ROOT / "oracle" / "_ref" / "libmoert_store_ref.so"


def ref_ggml():
    if not REF_GGML.exists():
        pytest.skip("oracle/_ref not built (needs the reference tree)")
    r = C.CDLL(str(REF_GGML))
    r.ref_gguf_write.argtypes = [C.c_char_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                 C.c_uint32]
    r.ref_gguf_read.argtypes = [C.c_char_p, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64), C.c_int64, C.c_void_p,
                                C.c_void_p, C.c_void_p, C.c_void_p]
    r.ref_gguf_read.restype = C.c_int64
    return r


def ref_store():
    if not REF_STORE.exists():
        pytest.skip("oracle/_ref not built (needs the reference tree)")
    return L.bind(C.CDLL(str(REF_STORE)), L.STORE_SIGNATURES)


def ggml_table(r, path):
    do, al = C.c_uint64(), C.c_uint64()
    names = C.create_string_buffer(64 * 64)
    types, offs, sizes = (C.c_int * 64)(), (C.c_uint64 * 64)(), (C.c_uint64 * 64)()
    n = r.ref_gguf_read(str(path).encode(), C.byref(do), C.byref(al), 64, names, types, offs, sizes)
    assert n >= 0
    rows = [(names.raw[64 * i:64 * i + 64].split(b"\0")[0].decode(), types[i], do.value + offs[i], sizes[i])
            for i in range(n)]
    return do.value, al.value, rows


def our_table(path):
    lib = la.lib()
    g = lib.llapis_gguf_open(str(path).encode())
    assert g, lib.llapis_files_last_error()
    try:
        rows = []
        for i in range(lib.llapis_gguf_n_tensors(g)):
            t = L.LlapisGgufTensorInfo()
            assert lib.llapis_gguf_tensor(g, i, C.byref(t)) == 0
            rows.append((t.name.decode(), t.type, t.offset, t.nbytes))
        return lib.llapis_gguf_data_offset(g), lib.llapis_gguf_alignment(g), rows
    finally:
        lib.llapis_gguf_close(g)


def random_tensors(rng, n):
    shapes = {12: [256, 3, 2], 22: [512, 2, 3], 6: [64, 5, 2], 20: [96, 4, 3], 0: [7, 3], 1: [5, 9]}
    out = []
    for i in range(n):
        t = int(rng.choice(list(shapes)))
        ne = shapes[t]
        out.append((f"blk.{i}.t{t}", t, ne, rng.integers(0, 256, nbytes(t, ne), dtype=np.uint8).tobytes()))
    return out


def test_gguf_table_matches_ggml(tmp_path):
    """A file written by ggml's writer (its default alignment: its writer
    places tensors by the context's alignment, not by a general.alignment
    key set on it) is read by ours as by ggml's reader."""
    alignment = 0
    r = ref_ggml()
    rng = np.random.default_rng(alignment)
    ts = random_tensors(rng, 7)
    path = tmp_path / "ggml.gguf"
    n = len(ts)
    names = (C.c_char_p * n)(*[t[0].encode() for t in ts])
    types = (C.c_int * n)(*[t[1] for t in ts])
    dims = (C.c_int * n)(*[len(t[2]) for t in ts])
    ne = (C.c_int64 * (4 * n))(*[v for t in ts for v in (t[2] + [1] * (4 - len(t[2])))])
    bufs = [C.create_string_buffer(t[3], len(t[3])) for t in ts]
    data = (C.c_void_p * n)(*[C.addressof(b) for b in bufs])
    assert r.ref_gguf_write(str(path).encode(), n, names, types, dims, ne, data, alignment) == 1
    assert our_table(path) == ggml_table(r, path)
    # the bytes at our offsets are the tensors' bytes
    raw = path.read_bytes()
    for (name, t, off, nb), (_, _, _, b) in zip(our_table(path)[2], ts):
        assert raw[off:off + nb] == b


@pytest.mark.parametrize("alignment", [32, 64, 256])
def test_gguf_test_writer_matches_ggml(tmp_path, alignment):
    """Files with a general.alignment key, from the fixture writer the GPU
    test uses, are read by ggml's reader as by ours."""
    r = ref_ggml()
    path = tmp_path / "ours.gguf"
    ts = random_tensors(np.random.default_rng(alignment), 6)
    write_gguf(path, ts, alignment=alignment)
    table = our_table(path)
    assert table == ggml_table(r, path) and table[1] == alignment
    raw = path.read_bytes()
    for (name, t, off, nb), (_, _, _, b) in zip(table[2], ts):
        assert off % alignment == 0 and raw[off:off + nb] == b


def test_gguf_expert_groups(tmp_path):
    from helpers import SMALL, layer
    lay = layer(SMALL, 5, [1, 2], scales=True)
    path = tmp_path / "layer.gguf"
    write_gguf(path, layer_tensors(lay, il=3))
    lib = la.lib()
    g = lib.llapis_gguf_open(str(path).encode())
    assert g
    raw = path.read_bytes()
    E = SMALL.n_expert
    try:
        for kind, is_scale, host, per in ((0, 0, lay.cold_gu, SMALL.gu_bytes(SMALL.cold_gu_type)),
                                          (1, 0, lay.cold_dn, SMALL.dn_bytes(SMALL.cold_dn_type)),
                                          (1, 1, lay.s_cold.view(np.uint8), 4)):
            grp = L.LlapisPageGroup()
            assert lib.llapis_gguf_expert_group(g, 3, kind, is_scale, E, C.byref(grp)) == 0
            assert grp.bytes_per_expert == per and grp.expert_axis == (0 if is_scale else 2)
            for e in (0, 5, E - 1):
                o = grp.offset + e * per
                assert raw[o:o + per] == host[e * per:(e + 1) * per].tobytes()
        grp = L.LlapisPageGroup()
        assert lib.llapis_gguf_expert_group(g, 0, 0, 0, E, C.byref(grp)) == -1      # no layer 0
        assert lib.llapis_gguf_expert_group(g, 3, 0, 0, E + 1, C.byref(grp)) == -1  # no such expert axis
    finally:
        lib.llapis_gguf_close(g)


def test_gguf_refuses_bad_files(tmp_path):
    lib = la.lib()
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"GGUX" + b"\0" * 64)
    assert not lib.llapis_gguf_open(str(p).encode())
    assert b"not a GGUF" in lib.llapis_files_last_error()
    write_gguf(p, random_tensors(np.random.default_rng(1), 3))
    p.write_bytes(p.read_bytes()[:60])
    assert not lib.llapis_gguf_open(str(p).encode())
    assert not lib.llapis_gguf_open(str(tmp_path / "missing.gguf").encode())


def write_store(lib, idx, pack, pages, n_layers=2, n_expert=6, pack_uuid=77):
    info = L.MoertStoreInfo()
    info.source_uuid, info.arch, info.n_layers, info.n_expert = 0xABC, b"gemma4", n_layers, n_expert
    info.n_embd, info.n_ff_exp, info.pack_uuid = 2816, 704, pack_uuid
    w = lib.moert_store_writer_open(str(idx).encode(), str(pack).encode(), C.byref(info))
    assert w
    for (layer, e, kind, sc, qt, shape, data) in pages:
        sh = (C.c_int64 * 4)(*shape)
        assert lib.moert_store_writer_add_page(w, layer, e, kind, sc, qt, qt, 0, sh, len(shape), data, len(data)) == 1
    assert lib.moert_store_writer_close(w) == 1


def store_pages(rng):
    pages = []
    for layer in range(2):
        for e in range(6):
            pages.append((layer, e, 0, 0, 12, [256, 7], rng.integers(0, 256, 144 * 7, dtype=np.uint8).tobytes()))
            pages.append((layer, e, 1, 0, 6, [64, 9], rng.integers(0, 256, 44 * 9, dtype=np.uint8).tobytes()))
            pages.append((layer, e, 1, 1, 0, [1], np.float32(1 + e).tobytes()))
    return pages


def read_all(lib, idx, pages):
    r = lib.moert_store_reader_open(str(idx).encode(), 0)
    assert r
    try:
        nl, ne = C.c_int32(), C.c_int32()
        assert lib.moert_store_reader_geometry(r, C.byref(nl), C.byref(ne)) == 1
        out = [(nl.value, ne.value)]
        for (layer, e, kind, sc, qt, shape, data) in pages:
            q, nb, sh = C.c_int32(), C.c_uint64(), (C.c_int64 * 4)()
            assert lib.moert_store_reader_page_info(r, layer, kind, sc, e, C.byref(q), C.byref(nb), sh) == 1
            buf = C.create_string_buffer(nb.value)
            assert lib.moert_store_reader_read(r, layer, kind, sc, e, buf, nb.value, 1) == nb.value
            out.append((q.value, nb.value, list(sh), buf.raw))
            assert buf.raw == data
        assert lib.moert_store_reader_page_nbytes(r, 0, 2, 0, 0) == 0            # absent page
        assert lib.moert_store_reader_page_nbytes(r, 9, 0, 0, 0) == 0            # out of range
        return out
    finally:
        lib.moert_store_reader_free(r)


@pytest.mark.parametrize("writer", ["ours", "reference"])
def test_store_round_trip_with_reference(tmp_path, writer):
    ref = ref_store()
    ours = la.lib()
    w, rd = (ours, ref) if writer == "ours" else (ref, ours)
    pages = store_pages(np.random.default_rng(11))
    idx, pack = tmp_path / "m.experts.index", tmp_path / "m.experts.pack"
    write_store(w, idx, pack, pages)
    assert read_all(ours, idx, pages) == read_all(ref, idx, pages)
    for lib in (ours, ref):
        info = L.MoertStoreInfo()
        assert lib.moert_store_probe(str(idx).encode(), C.byref(info)) == 1
        assert (info.format_version, info.source_uuid, info.arch, info.n_layers, info.n_expert, info.pack_uuid,
                info.record_count) == (1, 0xABC, b"gemma4", 2, 6, 77, len(pages))
        assert lib.moert_store_verify(str(idx).encode()) == 0
    # identical files from both writers (same uuid, same pages)
    if writer == "ours":
        idx2, pack2 = tmp_path / "r.experts.index", tmp_path / "r.experts.pack"
        write_store(ref, idx2, pack2, pages)
        assert idx.read_bytes() == idx2.read_bytes() and pack.read_bytes() == pack2.read_bytes()
    # one flipped byte in a page: both verifiers count it, both readers refuse it
    raw = bytearray(pack.read_bytes())
    raw[300] ^= 0x40
    pack.write_bytes(bytes(raw))
    for lib in (ours, ref):
        assert lib.moert_store_verify(str(idx).encode()) == 1
        r = lib.moert_store_reader_open(str(idx).encode(), 0)
        buf = C.create_string_buffer(4096)
        assert lib.moert_store_reader_read(r, 0, 0, 0, 0, buf, 4096, 1) == 0
        assert lib.moert_store_reader_read(r, 0, 0, 0, 0, buf, 4096, 0) == 144 * 7
        lib.moert_store_reader_free(r)
    # a source uuid the caller did not expect is refused
    assert not ours.moert_store_reader_open(str(idx).encode(), 0x123)


def test_store_refuses_corrupt_index(tmp_path):
    """A damaged index is refused with an error return (no allocation sized
    from it): a record count beyond the index's own size, a truncated index,
    a geometry whose page table would be huge, a record reaching past the
    end of the pack."""
    import struct
    lib = la.lib()
    pages = store_pages(np.random.default_rng(12))
    idx, pack = tmp_path / "c.experts.index", tmp_path / "c.experts.pack"
    write_store(lib, idx, pack, pages)
    good = idx.read_bytes()

    def patched(off, fmt, val):
        raw = bytearray(good)
        struct.pack_into(fmt, raw, off, val)
        return bytes(raw)

    header = 96                                   # records follow the 96-byte header, 72 bytes each
    bad = [patched(72, "<Q", 1 << 31),            # record_count
           good[:header + 72 * 3 + 10],           # truncated
           patched(40, "<I", 1 << 20),            # n_layers (x 6 experts)
           patched(header + 16, "<Q", 1 << 40),   # first record's nbytes
           patched(header + 8, "<Q", 1 << 62)]    # first record's offset
    for i, raw in enumerate(bad):
        idx.write_bytes(raw)
        assert not lib.moert_store_reader_open(str(idx).encode(), 0), i
        assert lib.moert_store_verify(str(idx).encode()) == -1, i
    idx.write_bytes(good)
    assert lib.moert_store_verify(str(idx).encode()) == 0
    r = lib.moert_store_reader_open(str(idx).encode(), 0)
    assert r
    lib.moert_store_reader_free(r)


def test_store_fnv_matches(tmp_path):
    ref = ref_store()
    data = np.random.default_rng(2).integers(0, 256, 1000, dtype=np.uint8)
    for seed in (L.FNV_SEED, 0, 12345):
        assert la.lib().moert_store_fnv1a64(data.ctypes.data, 1000, seed) == ref.moert_store_fnv1a64(
            data.ctypes.data, 1000, seed)
