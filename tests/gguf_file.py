"""A minimal GGUF v3 writer for test fixtures (test infrastructure): the
header, two keys (general.architecture, general.alignment), the tensor table
and the data section with every tensor at an aligned offset.  Files it
writes are checked against ggml's own reader in tests/test_model_files.py."""
import struct

import numpy as np

from llapis_amd import row_size

TYPE_BLCK = {0: (4, 1), 1: (2, 1), 6: (22, 32), 12: (144, 256), 20: (18, 32), 22: (82, 256)}


def nbytes(t, ne):
    b, k = TYPE_BLCK[t]
    n = b * (ne[0] // k)
    for d in ne[1:]:
        n *= d
    return n


def _str(s):
    s = s.encode()
    return struct.pack("<Q", len(s)) + s


def write_gguf(path, tensors, alignment=32, arch="gemma4"):
    """tensors: list of (name, ggml type, ne (list, ne0 first), bytes)."""
    kv = [_str("general.architecture") + struct.pack("<i", 8) + _str(arch),
          _str("general.alignment") + struct.pack("<iI", 4, alignment)]
    head = b"GGUF" + struct.pack("<Iqq", 3, len(tensors), len(kv)) + b"".join(kv)
    infos, off = [], 0
    for name, t, ne, data in tensors:
        assert len(data) == nbytes(t, ne), name
        infos.append(_str(name) + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}q", *ne) +
                     struct.pack("<iQ", t, off))
        off += (len(data) + alignment - 1) // alignment * alignment
    meta = head + b"".join(infos)
    pad = (-len(meta)) % alignment
    with open(path, "wb") as f:
        f.write(meta + b"\0" * pad)
        for name, t, ne, data in tensors:
            f.write(bytes(data))
            f.write(b"\0" * ((-len(data)) % alignment))


def layer_tensors(lay, il=0):
    """One layer's stacked expert tensors as a GGUF holds them: the cold
    pools (IQ2_S gate_up [d_model, 2 n_ff, E], IQ4_NL down [n_ff, d_model, E])
    with the down .scale [E], and the fp32 router."""
    sp = lay.spec
    E = sp.n_expert
    out = [(f"blk.{il}.ffn_gate_inp.weight", 0, [sp.d_model, E], np.ascontiguousarray(lay.router_w).tobytes()),
           (f"blk.{il}.ffn_gate_up_exps.weight", sp.cold_gu_type, [sp.d_model, 2 * sp.n_ff, E], lay.cold_gu.tobytes()),
           (f"blk.{il}.ffn_down_exps.weight", sp.cold_dn_type, [sp.n_ff, sp.d_model, E], lay.cold_dn.tobytes())]
    if lay.s_cold is not None:
        out.append((f"blk.{il}.ffn_down_exps.scale", 0, [E], np.ascontiguousarray(lay.s_cold, np.float32).tobytes()))
    return out
