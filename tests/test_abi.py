"""The C ABI, CPU only: libllapis_moe.so loads, exports every function the
public headers declare, and the plain-C structs have the byte layout of the
reference's moert/include/moert/cuda.h (compiled and compared here when the
reference tree is present) and of the ctypes mirror in llapis_amd/_lib.py."""
import ctypes as C
import re
import shutil
import subprocess
from pathlib import Path

import pytest

import llapis_amd as la
from llapis_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
INCLUDE = ROOT / "include"
REF_HEADER = Path("/root/reference/moert/include/moert/cuda.h")

DECL = re.compile(r"^\s*(?!typedef|static|#|/\*|\*)[A-Za-z_][\w\s\*]*?\b((?:moert|llapis)_\w+)\s*\(", re.M)


def declared_functions():
    names = set()
    for h in INCLUDE.glob("*.h"):
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"static inline[^{]*\{.*?\n\}", "", text, flags=re.S)
        names.update(DECL.findall(text))
    return names


def test_library_exports_every_declared_function():
    names = declared_functions()
    assert len(names) >= 30, sorted(names)
    lib = C.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    # the ctypes binding covers the same set
    assert names == set(_lib.SIGNATURES), sorted(names ^ set(_lib.SIGNATURES))


MIRRORS = {
    "moert_cuda_config": _lib.MoertCudaConfig,
    "moert_mm_call": _lib.MoertMmCall,
    "moert_ffn_moe_host": _lib.MoertFfnMoeHost,
    "moert_ffn_moe_args": _lib.MoertFfnMoeArgs,
    "moert_cuda_stats": _lib.MoertCudaStats,
    "moert_cuda_dir_stats": _lib.MoertCudaDirStats,
    "llapis_tensor": _lib.LlapisTensor,
    "llapis_moe_dual_op": _lib.LlapisMoeDualOp,
    "llapis_moe_layer": _lib.LlapisMoeLayer,
    "llapis_xfer_done": _lib.LlapisXferDone,
    "llapis_xfer_stats": _lib.LlapisXferStats,
    "llapis_kfit_inputs": _lib.LlapisKfitInputs,
    "llapis_gguf_tensor_info": _lib.LlapisGgufTensorInfo,
    "llapis_page_group": _lib.LlapisPageGroup,
    "llapis_residency_stats": _lib.LlapisResidencyStats,
    "moert_store_info": _lib.MoertStoreInfo,
    "llapis_kfit_decision": _lib.LlapisKfitDecision,
    "moert_policy_config": _lib.MoertPolicyConfig,
    "moert_policy_callbacks": _lib.MoertPolicyCallbacks,
    "moert_policy_stats": _lib.MoertPolicyStats,
    "moert_policy_window": _lib.MoertPolicyWindow,
}
POLICY_STRUCTS = ("moert_policy_config", "moert_policy_callbacks", "moert_policy_stats", "moert_policy_window")
REF_STORE_HEADER = Path("/root/reference/moert/include/moert/store.h")
REF_POLICY_HEADER = Path("/root/reference/moert/include/moert/policy.h")
# structs of the reference header with no ctypes mirror (host callback payloads)
CALLBACK_STRUCTS = {
    "moert_coldcpu_call": ["il", "kind", "n_cold", "cold_ids", "x", "x_per_pair", "w_host", "expert_bytes",
                           "stride", "w_type_tag", "d_in", "d_out", "y", "x_col"],
    "moert_coldffn_job": ["il", "n_used", "n_tokens", "h_counts", "h_ids", "h_cdst", "x", "w_gu", "gu_bytes",
                          "gu_stride", "gu_type", "d_in", "d_gu", "y", "wait_ready", "ev"],
}


def layout_program(header, structs):
    lines = ["#include <cstddef>", "#include <cstdio>", f'#include "{header}"', "int main() {"]
    for s, fields in structs.items():
        lines.append(f'  std::printf("{s} sizeof %zu\\n", sizeof({s}));')
        for f in fields:
            lines.append(f'  std::printf("{s} {f} %zu\\n", offsetof({s}, {f}));')
    lines += ["  return 0;", "}"]
    return "\n".join(lines)


def compile_layouts(tmp_path, header, structs):
    if not shutil.which("g++"):
        pytest.skip("no host C++ compiler")
    src = tmp_path / "layout.cpp"
    src.write_text(layout_program(header, structs))
    exe = tmp_path / "layout"
    subprocess.run(["g++", "-std=c++17", "-I", str(INCLUDE), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, stdout=subprocess.PIPE, text=True).stdout
    return {tuple(l.split()[:2]): int(l.split()[2]) for l in out.splitlines()}


def moert_structs():
    out = {k: [f[0] for f in v._fields_] for k, v in MIRRORS.items()
           if k.startswith("moert_") and k not in POLICY_STRUCTS and k != "moert_store_info"}
    out.update(CALLBACK_STRUCTS)
    return out


def test_ctypes_mirror_matches_headers(tmp_path):
    structs = {k: [f[0] for f in v._fields_] for k, v in MIRRORS.items()}
    prog_header = tmp_path / "both.h"
    prog_header.write_text('#include "moert_hip.h"\n#include "llapis_moe.h"\n#include "moert_policy.h"\n'
                           '#include "moert_store.h"\n')
    got = compile_layouts(tmp_path, str(prog_header), structs)
    for s, cls in MIRRORS.items():
        assert got[(s, "sizeof")] == C.sizeof(cls), s
        for f in structs[s]:
            assert got[(s, f)] == getattr(cls, f).offset, (s, f)


@pytest.mark.skipif(not REF_HEADER.exists(), reason="reference tree not present")
def test_moert_structs_match_reference_header(tmp_path):
    ours = compile_layouts(tmp_path, str(INCLUDE / "moert_hip.h"), moert_structs())
    (tmp_path / "r").mkdir()
    theirs = compile_layouts(tmp_path / "r", str(REF_HEADER), moert_structs())
    assert ours == theirs
    assert ours[("moert_ffn_moe_args", "sizeof")] > 0


@pytest.mark.skipif(not REF_POLICY_HEADER.exists(), reason="reference tree not present")
def test_policy_structs_match_reference_header(tmp_path):
    structs = {k: [f[0] for f in MIRRORS[k]._fields_] for k in POLICY_STRUCTS}
    ours = compile_layouts(tmp_path, str(INCLUDE / "moert_policy.h"), structs)
    (tmp_path / "r").mkdir()
    theirs = compile_layouts(tmp_path / "r", str(REF_POLICY_HEADER), structs)
    assert ours == theirs


@pytest.mark.skipif(not REF_STORE_HEADER.exists(), reason="reference tree not present")
def test_store_info_matches_reference_header(tmp_path):
    structs = {"moert_store_info": [f[0] for f in _lib.MoertStoreInfo._fields_]}
    ours = compile_layouts(tmp_path, str(INCLUDE / "moert_store.h"), structs)
    (tmp_path / "r").mkdir()
    theirs = compile_layouts(tmp_path / "r", str(REF_STORE_HEADER), structs)
    assert ours == theirs


def test_config_defaults_match():
    """moert_cuda_config_defaults is header-inline in both; compare the values
    ours sets with the reference's documented defaults."""
    cfg = _lib.MoertCudaConfig()
    la.lib().moert_cuda_configure(C.byref(cfg))      # accepted without a device
    text = (INCLUDE / "moert_hip.h").read_text()
    body = text[text.index("moert_cuda_config_defaults"):]
    body = body[:body.index("}")]
    vals = dict(re.findall(r"cfg->(\w+)\s*=\s*(\d+)", body))
    assert vals == {"counted": "1", "copy_stream": "0", "coldcpu": "0", "coldcpu_max": "3", "coldcpu_fn": "0",
                    "cold_guard_fn": "0", "cold_ffn": "0", "coldffn_submit_fn": "0", "coldffn_wait_fn": "0"}


def test_host_services_and_transport_before_init():
    """Registration is refused (the cold tier is in HBM); the transport
    answers as the reference's does before moert_cuda_dir_init (no device
    call is made)."""
    lib = la.lib()
    assert lib.moert_cuda_host_register_pinned(None, 0) == 0
    assert lib.moert_cuda_host_register_mapped(None, 0) == 0
    assert lib.moert_cuda_host_map(None, 0) is None
    assert lib.moert_cuda_dir_async(None, None, 0) == 0
    assert lib.moert_cuda_dir_mark() == -1
    assert lib.moert_cuda_dir_poll(0) == -1
    assert lib.moert_cuda_dir_gate(4, 0) == 0            # no waits yet
    assert lib.moert_cuda_dir_gate(2, 5) == 0            # gate not enabled: nothing to wait for
    assert lib.moert_cuda_dir_gate(1, 0) == 1            # arm: target 1
    assert lib.moert_cuda_dir_gate(3, 0) == 1
    assert lib.moert_cuda_publish_h2d(0, None, None, None) == 1
    st = _lib.MoertCudaDirStats()
    lib.moert_cuda_dir_stats_get(C.byref(st))
    assert st.async_copies == 0 and st.pub_calls == 0


def test_xfer_refuses_bad_arguments_without_a_device():
    lib = la.lib()
    assert lib.llapis_xfer_create(0, 128, 57, 8) is None
    assert b"geometry" in lib.llapis_xfer_last_error()
    assert lib.llapis_xfer_submit(None, 0, 0, 0) == -1
    assert lib.llapis_xfer_take_done(None, None, 0) == -1
    assert lib.llapis_xfer_in_flight(None) == 0


RESIDENCY_BINDING_C = r"""
#include "llapis_moe.h"
void bind(llapis_moe_layer * layer, int32_t n_layers, int32_t n_expert, int32_t k, void * compute_stream,
          int32_t ** es, int32_t ** se, int32_t ** ss, int64_t n_prompt) {
    moert_policy_config cfg;
    moert_policy_config_defaults(&cfg);
    cfg.n_layers = n_layers; cfg.n_expert = n_expert; cfg.k = k;
    llapis_residency * R = llapis_residency_create(&cfg, 0);
    moert_policy * P = llapis_residency_policy(R);
    llapis_xfer * X = llapis_residency_xfer(R);
    (void)X;
    for (int il = 0; il < n_layers; ++il) {
        llapis_residency_counters(R, il, &layer[il].route_counts, &layer[il].route_hits);
        llapis_residency_set_mirrors(R, il, es[il], se[il], ss[il]);
        moert_policy_commit_seed(P, il, 0, 0);
    }
    llapis_residency_publish_all(R, compute_stream);
    moert_policy_on_prompt_token(P, n_prompt);
    llapis_residency_refresh(R, MOERT_REFRESH_PROMPT_END, compute_stream);
    llapis_residency_token_end(R, compute_stream);
    llapis_residency_refresh(R, MOERT_REFRESH_TURN_END, compute_stream);
    llapis_residency_stats st;
    llapis_residency_get_stats(R, &st);
    llapis_residency_free(R);
}
"""


def test_residency_binding_compiles_as_c(tmp_path):
    """The residency loop's binding, as an integrator writes it in C against
    the shipped headers, compiles (C11, warnings as errors)."""
    src = tmp_path / "bind.c"
    src.write_text(RESIDENCY_BINDING_C)
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-fsyntax-only", "-I", str(INCLUDE), str(src)], check=True)


def test_noalloc_scratch_size_matches_header():
    text = (INCLUDE / "llapis_moe.h").read_text()
    m = re.search(r"#define LLAPIS_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)", text)
    assert m and int(m.group(1)) << int(m.group(2)) == _lib.NOALLOC_SCRATCH_BYTES


def test_noalloc_refuses_before_any_device_call():
    """A null layer and a call larger than the fixed array are refused on the
    host, with no GPU in the process."""
    lib = _lib.lib()
    assert lib.llapis_moe_ffn_noalloc(None, None, None, 1, None, None, None, None) != 0
    d = _lib.LlapisMoeLayer(2816, 704, 128, 8, 57, 12, 6, 22, 20, 0, 0, *([None] * 12))
    assert lib.llapis_moe_ffn_noalloc(C.byref(d), None, None, 512, None, None, None, None) != 0
    assert b"bytes of scratch" in lib.llapis_last_error()
