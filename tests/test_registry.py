"""The expert registry (include/moert_registry.h) against the reference's
header-only registry (moert/include/moert/registry.h), both compiled here:
every combination of the five where-flags (slot set or not, arena valid,
same bytes, hot file, cold file), with flag values 0 / 1 / 7 and slots -1,
-5, 0 and 9, both representations and a NULL where, gives the same source;
the names of every source value (and out-of-range values) agree.  The
reference's own scenarios (tests/test_moert_registry.cpp) hold with our
header alone."""
import ctypes as C
import itertools
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
REF_INC = Path("/root/reference/moert/include")

WRAP = r"""
#include <stdint.h>
#include "%s"
int32_t %s_for(int32_t slot, int32_t arena, int32_t same, int32_t fh, int32_t fc, int32_t rep, int32_t null_w) {
    moert_expert_where w = {slot, arena, same, fh, fc};
    return moert_source_for(null_w ? 0 : &w, rep);
}
const char * %s_name(int32_t s) { return moert_source_name(s); }
"""


class Where(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("slot", "arena_valid", "same_bytes", "file_hot", "file_cold")]


def build(tmp_path, with_ref):
    srcs = []
    (tmp_path / "ours.c").write_text(WRAP % (str(ROOT / "include" / "moert_registry.h"), "ours", "ours"))
    srcs.append(str(tmp_path / "ours.c"))
    if with_ref:
        (tmp_path / "ref.c").write_text(WRAP % ("moert/registry.h", "ref", "ref"))
        srcs.append(str(tmp_path / "ref.c"))
    so = tmp_path / "libreg.so"
    subprocess.run(["gcc", "-O1", "-shared", "-fPIC", "-std=c11", "-Wall", "-Werror", f"-I{REF_INC}", *srcs,
                    "-o", str(so)], check=True)
    lib = C.CDLL(str(so))
    for n in ("ours", "ref") if with_ref else ("ours",):
        getattr(lib, f"{n}_name").restype = C.c_char_p
    return lib


@pytest.mark.skipif(not (REF_INC / "moert" / "registry.h").exists(), reason="reference tree not present")
def test_registry_matches_reference_exhaustively(tmp_path):
    lib = build(tmp_path, True)
    n = 0
    for slot in (-5, -1, 0, 9):
        for arena, same, fh, fc in itertools.product((0, 1, 7), repeat=4):
            for rep in (0, 1):
                args = (slot, arena, same, fh, fc, rep, 0)
                assert lib.ours_for(*args) == lib.ref_for(*args), args
                n += 1
    assert lib.ours_for(0, 1, 1, 1, 1, 0, 1) == lib.ref_for(0, 1, 1, 1, 1, 0, 1) == 0
    for s in range(-3, 8):
        assert lib.ours_name(s) == lib.ref_name(s), s
    assert n == 4 * 81 * 2


def test_registry_reference_scenarios(tmp_path):
    """The reference test's cases, with our header alone (expected values
    from moert registry semantics: slot < arena < file)."""
    lib = build(tmp_path, False)
    SLOT, ARENA, FILE, NONE = 1, 2, 3, 0
    f = lambda slot, arena, same, fh, fc, rep: lib.ours_for(slot, arena, same, fh, fc, rep, 0)
    # the same bytes in both representations (a full-IQ2 regime)
    assert f(-1, 1, 1, 1, 1, 0) == ARENA and f(-1, 1, 1, 1, 1, 1) == ARENA
    assert f(3, 1, 1, 1, 1, 0) == SLOT and f(3, 1, 1, 1, 1, 1) == SLOT
    assert f(3, 0, 1, 1, 1, 1) == SLOT
    assert f(-1, 0, 1, 1, 1, 0) == FILE
    assert f(-1, 0, 1, 0, 0, 0) == NONE
    # distinct representations (hot Q4, cold IQ2)
    assert f(-1, 1, 0, 1, 1, 0) == FILE and f(-1, 1, 0, 1, 1, 1) == ARENA
    assert f(3, 1, 0, 1, 1, 0) == SLOT and f(3, 1, 0, 1, 1, 1) == ARENA
    assert f(3, 0, 0, 1, 1, 1) == FILE
    assert lib.ours_for(3, 1, 1, 1, 1, 0, 1) == NONE
    assert [lib.ours_name(s) for s in (0, 1, 2, 3, 4, -1)] == [b"none", b"slot", b"arena", b"file", b"none", b"none"]
