"""The fp16 GELU table compiled into the device code (generated at build
time by llapis_amd/csrc/gen_gelu_table.c) against the CPU checkers: every
entry the device can read -- fp16 inputs of magnitude below 10, and 10.0
itself, which an input just below 10 rounds to -- equals the table-mode GEGLU
of the oracle (pinned to the reference's outputs in test_oracle.py) and, where
oracle/_ref is built, of the reference's own ggml CPU path, bit for bit."""
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
INC = ROOT / "llapis_amd" / "_build" / "gelu_table.inc"
GELU_TABLE = 0


def table():
    if not INC.exists():
        pytest.fail("llapis_amd/_build/gelu_table.inc missing: run the build first")
    txt = INC.read_text()
    span = int(re.search(r"LLAPIS_GELU_TAB_SPAN (0x[0-9A-Fa-f]+)", txt).group(1), 16)
    body = txt[txt.index("{") + 1:txt.rindex("}")]
    vals = np.array([int(v, 16) for v in re.findall(r"0x[0-9a-fA-F]{4}", body)], np.uint16)
    assert vals.size == 2 * span
    return span, vals


def inputs():
    """(fp32 input, table index) for every entry the device reads."""
    xs, idx = [], []
    for sign in (0, 1):
        mags = np.arange(0, 0x4900, dtype=np.uint16)
        h = (mags | (sign << 15)).astype(np.uint16)
        xs.append(h.view(np.float16).astype(np.float32))
        idx.append(mags.astype(np.int64) + sign * SPAN)
        # just inside +-10: fp16(x) = +-10.0 (0x4900), the table's last used entry
        xs.append(np.array([np.nextafter(np.float32(10), np.float32(0)) * (-1 if sign else 1)], np.float32))
        idx.append(np.array([0x4900 + sign * SPAN]))
    return np.concatenate(xs), np.concatenate(idx)


SPAN = 0x4A00


def test_table_matches_oracle(oracle):
    span, tab = table()
    assert span == SPAN
    x, idx = inputs()
    got = tab[idx]
    want = oracle.geglu(x, np.ones_like(x), GELU_TABLE).astype(np.float16).view(np.uint16)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(float(x[i]), hex(got[i]), hex(want[i])) for i in bad[:5]]


def test_table_matches_reference_ggml():
    try:
        from oracle import Ref
        ref = Ref()
    except (FileNotFoundError, OSError):
        pytest.skip("oracle/_ref not built (the reference tree is absent)")
    _, tab = table()
    x, idx = inputs()
    n = (x.size // 8) * 8
    want = ref.geglu(x[None, :n], np.ones((1, n), np.float32))[0].astype(np.float16).view(np.uint16)
    assert np.array_equal(tab[idx[:n]], want)
