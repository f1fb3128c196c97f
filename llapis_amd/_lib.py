"""ctypes binding of libllapis_moe.so (include/moert_hip.h + include/llapis_moe.h).

The library is the product: loading fails loudly if it has not been built
(python -m llapis_amd.build); there is no fallback implementation.
"""
import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libllapis_moe.so"

# ggml type tags (ggml.h:390-412)
F32, Q5_0, Q8_0, Q8_1, Q4_K, Q8_K, IQ4_NL, IQ2_S = 0, 6, 8, 9, 12, 15, 20, 22
ACT_CPU, ACT_Q8_1 = 0, 1
GELU_TABLE, GELU_TANH = 0, 1
MM_W_HOT, MM_W_COLD_SRC, MM_W_RAW = 0, 1, 2
SLOT_FREE, SLOT_FILLING, SLOT_READY = 0, 1, 2
PMAX_MAX = 32

vp, i32, i64, u64 = C.c_void_p, C.c_int32, C.c_int64, C.c_uint64


class MoertCudaConfig(C.Structure):
    _fields_ = [("counted", i32), ("copy_stream", i32), ("coldcpu", i32), ("coldcpu_max", i32),
                ("coldcpu_fn", u64), ("cold_guard_fn", u64), ("cold_ffn", i32),
                ("coldffn_submit_fn", u64), ("coldffn_wait_fn", u64)]


class MoertMmCall(C.Structure):
    _fields_ = [("w_sel", i32), ("w_type_tag", i32), ("w_data", vp), ("w_n", i64), ("b", vp),
                ("b_ncols", i64), ("ids", vp), ("n_ids", i64), ("y", vp), ("ne_live", vp), ("w_ptrs", vp)]


POOL_ALLOC = C.CFUNCTYPE(vp, vp, u64)
POOL_FREE = C.CFUNCTYPE(None, vp, vp)
MM_FN = C.CFUNCTYPE(None, vp, C.POINTER(MoertMmCall))


class MoertFfnMoeHost(C.Structure):
    _fields_ = [("user", vp), ("pool_alloc", POOL_ALLOC), ("pool_free", POOL_FREE), ("mm", MM_FN)]


class MoertFfnMoeArgs(C.Structure):
    _fields_ = [("kind", i32), ("top_k", i32), ("il", i32), ("planc_mode", i32), ("n_used", i32),
                ("n_tokens", i32), ("ids_s1", i32), ("d_in", i32), ("d_out", i32), ("n_expert", i32),
                ("k", i32), ("cold_type_tag", i32), ("expert_bytes", u64), ("cur", vp), ("ids", vp),
                ("exp_slot", vp), ("slot_exp", vp), ("slot_state", vp), ("s_hot", vp), ("s_cold", vp),
                ("w_cold_dev", u64), ("s_cold_dev", u64), ("has_w_cold", i32), ("dst", vp), ("stream", vp)]


class MoertCudaStats(C.Structure):
    _fields_ = [(n, C.c_longlong) for n in ("fires", "op_host_ns", "seam_syncs", "seam_ns", "coldcpu_calls",
                                            "coldcpu_pairs", "coldcpu_ns", "coldcpu_over_max")]


class MoertCudaDirStats(C.Structure):
    _fields_ = [(n, C.c_longlong) for n in ("async_copies", "async_marks", "bytes", "pub_calls", "pub_copies",
                                            "sm_copies", "sm_fallback", "sm_timed", "sm_gpu_ns", "sm_gpu_ns_max",
                                            "sm_ring_copies", "sm_ring_waits")] + \
               [("sm_ring_wait_ms", C.c_double), ("sm_stage_ms", C.c_double)]


class LlapisTensor(C.Structure):
    _fields_ = [("type", i32), ("ne", i64 * 4), ("nb", u64 * 4), ("data", vp)]


class LlapisMoeDualOp(C.Structure):
    _fields_ = [("src", C.POINTER(LlapisTensor) * 9), ("op_params", i32 * 10), ("dst", C.POINTER(LlapisTensor))]


class LlapisMoeLayer(C.Structure):
    _fields_ = [("d_model", i32), ("n_ff", i32), ("n_expert", i32), ("top_k", i32), ("k_slots", i32),
                ("hot_gu_type", i32), ("hot_dn_type", i32), ("cold_gu_type", i32), ("cold_dn_type", i32),
                ("act_mode", i32), ("gelu_mode", i32),
                ("router_w", vp), ("router_b", vp), ("hot_gu", vp), ("hot_dn", vp), ("cold_gu", vp),
                ("cold_dn", vp), ("exp_slot", vp), ("slot_exp", vp), ("slot_state", vp), ("s_hot", vp),
                ("s_cold", vp), ("route_counts", vp), ("route_hits", vp)]


XFER_MAX_GROUPS = 4
NOALLOC_SCRATCH_BYTES = 8 << 20          # LLAPIS_NOALLOC_SCRATCH_BYTES


class LlapisKfitInputs(C.Structure):
    _fields_ = [("free_mib", C.c_longlong), ("slab_mib_now", C.c_longlong), ("headroom_mib", C.c_longlong),
                ("per_k_mib", C.c_longlong), ("keep_free_mib", C.c_longlong), ("k_cur", i32), ("k_min", i32),
                ("n_expert", i32), ("evicted", i32)]


class LlapisKfitDecision(C.Structure):
    _fields_ = [("k", i32), ("rebuild", i32), ("wddm_bound", i32), ("floor_capped", i32), ("pool_mib", C.c_longlong)]


class LlapisXferDone(C.Structure):
    _fields_ = [("il", i32), ("e", i32), ("slot", i32), ("ok", i32)]


class LlapisXferStats(C.Structure):
    _fields_ = [(n, C.c_longlong) for n in ("submitted", "completed", "failed", "max_queue", "bytes",
                                            "wait_idle_calls")] + [("wait_idle_ms", C.c_double)]


class LlapisGgufTensorInfo(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("type", i32), ("n_dims", i32), ("ne", i64 * 4), ("nb", u64 * 4),
                ("offset", u64), ("nbytes", u64)]


class LlapisPageGroup(C.Structure):
    _fields_ = [("type", i32), ("expert_axis", i32), ("n_expert", i32), ("reserved", i32), ("ne", i64 * 4),
                ("offset", u64), ("bytes_per_expert", u64)]


class LlapisResidencyStats(C.Structure):
    _fields_ = [(n, C.c_longlong) for n in ("tokens", "fetches", "submitted", "completed", "publications",
                                            "hot_pairs", "cold_pairs")] + [("wait_ms", C.c_double),
                                                                           ("host_ms", C.c_double)]


# moert_store.h
class MoertStoreInfo(C.Structure):
    _fields_ = [("format_version", C.c_uint32), ("source_uuid", u64), ("arch", C.c_char * 16), ("n_layers", i32),
                ("n_expert", i32), ("n_embd", u64), ("n_ff_exp", u64), ("pack_uuid", u64), ("record_count", u64)]


PAGE_SCALE = 1 << 3
FNV_SEED = 14695981039346656037
STORE_SIGNATURES = {
    "moert_store_probe": (i32, [C.c_char_p, C.POINTER(MoertStoreInfo)]),
    "moert_store_verify": (i64, [C.c_char_p]),
    "moert_store_writer_open": (vp, [C.c_char_p, C.c_char_p, C.POINTER(MoertStoreInfo)]),
    "moert_store_writer_add_page": (i32, [vp, i32, i32, i32, i32, i32, i32, C.c_uint32, vp, i32, vp, u64]),
    "moert_store_writer_close": (i32, [vp]),
    "moert_store_fnv1a64": (u64, [vp, u64, u64]),
    "moert_store_reader_open": (vp, [C.c_char_p, u64]),
    "moert_store_reader_free": (None, [vp]),
    "moert_store_reader_geometry": (i32, [vp, vp, vp]),
    "moert_store_reader_page_nbytes": (u64, [vp, i32, i32, i32, i32]),
    "moert_store_reader_page_info": (i32, [vp, i32, i32, i32, i32, vp, vp, vp]),
    "moert_store_reader_read": (u64, [vp, i32, i32, i32, i32, vp, u64, i32]),
}


def bind(cdll, table):
    """Set a signature table on a loaded library (this one, or a checker
    exporting the same ABI); returns it."""
    for name, (res, args) in table.items():
        fn = getattr(cdll, name)
        fn.restype = res
        fn.argtypes = args
    return cdll


# moert_policy.h
REFRESH_PROMPT_END, REFRESH_VISIBLE_INTERVAL, REFRESH_TURN_END, REFRESH_BOUNDARY = 0, 1, 2, 4
f32 = C.c_float


class MoertPolicyConfig(C.Structure):
    _fields_ = [("n_layers", i32), ("n_expert", i32), ("k", i32), ("seed_prior", f32), ("session_decay", f32),
                ("recent_decay", f32), ("blend_a", f32), ("blend_b", f32), ("blend_c", f32),
                ("k_per_layer", vp), ("cost_horizon", i32), ("cost_reuse", f32), ("cost_rate_decay", f32),
                ("cost_per_token", i32)]


STREAM_EXPERT = C.CFUNCTYPE(i32, vp, i32, i32, i32)
PUBLISH_LAYER = C.CFUNCTYPE(None, vp, i32)
FETCH_EXTERNAL = C.CFUNCTYPE(None, vp)


class MoertPolicyCallbacks(C.Structure):
    _fields_ = [("stream_expert", STREAM_EXPERT), ("publish_layer", PUBLISH_LAYER),
                ("fetch_external", FETCH_EXTERNAL), ("user", vp)]


class MoertPolicyStats(C.Structure):
    _fields_ = [(n, i64) for n in ("promotions", "demotions", "tokens", "visible_tokens", "hot_routes",
                                   "cold_routes", "refresh_count", "refresh_promotions", "refresh_demotions")] + \
               [("refresh_pause_ms_total", C.c_double), ("refresh_pause_ms_max", C.c_double),
                ("last_refresh_tok", i64), ("last_refresh_promos", i64), ("last_refresh_pause_ms", C.c_double),
                ("occupancy", C.c_double)] + \
               [(n, i64) for n in ("fills_async", "fills_completed", "fills_stale", "fills_aborted")]


class MoertPolicyWindow(C.Structure):
    _fields_ = [("tokens", i32), ("span_ms", C.c_double), ("tok_per_s", C.c_double), ("ms_per_tok", C.c_double),
                ("hit_rate", C.c_double), ("hot_routes", i64), ("cold_routes", i64)]


_P = vp   # moert_policy *
POLICY_SIGNATURES = {
    "moert_policy_config_defaults": (None, [C.POINTER(MoertPolicyConfig)]),
    "moert_policy_create": (_P, [C.POINTER(MoertPolicyConfig), C.POINTER(MoertPolicyCallbacks)]),
    "moert_policy_free": (None, [_P]),
    "moert_policy_set_external_observation": (None, [_P, i32]),
    "moert_policy_observe": (None, [_P, i32, vp, i32, i64]),
    "moert_policy_on_prompt_token": (None, [_P, i64]),
    "moert_policy_on_token_end": (None, [_P]),
    "moert_policy_refresh": (None, [_P, i32]),
    "moert_policy_resize_k": (i32, [_P, i32]),
    "moert_policy_set_active_k": (i32, [_P, i32]),
    "moert_policy_can_seed": (i32, [_P, i32, i32]),
    "moert_policy_commit_seed": (i32, [_P, i32, i32, i32]),
    "moert_policy_complete_fill": (i32, [_P, i32, i32, i32]),
    "moert_policy_abort_fill": (i32, [_P, i32, i32, i32]),
    "moert_policy_boundary_layer": (i32, [_P, i32, vp, i64, f32, f32]),
    "moert_policy_add_external_counts": (None, [_P, i32, vp, i64, i64]),
    "moert_policy_reset_stats": (None, [_P]),
    "moert_policy_layer_k": (i32, [_P, i32]),
    "moert_policy_set_external_forecast": (None, [_P, vp, f32, i32]),
    "moert_policy_hit_rate": (C.c_double, [_P]),
    "moert_policy_get_stats": (None, [_P, C.POINTER(MoertPolicyStats)]),
    "moert_policy_get_window": (None, [_P, i32, C.POINTER(MoertPolicyWindow)]),
    "moert_policy_exp_slot_view": (C.POINTER(i32), [_P, i32]),
    "moert_policy_slot_exp_view": (C.POINTER(i32), [_P, i32]),
    "moert_policy_slot_state_view": (C.POINTER(i32), [_P, i32]),
    "moert_policy_hotmap_view": (C.POINTER(i32), [_P, i32]),
    "moert_policy_resid_view": (C.POINTER(f32), [_P, i32]),
}


# every symbol the two public headers declare, with its signature
SIGNATURES = {
    # moert_hip.h
    "moert_cuda_configure": (None, [C.POINTER(MoertCudaConfig)]),
    "moert_ffn_moe": (None, [C.POINTER(MoertFfnMoeArgs), C.POINTER(MoertFfnMoeHost)]),
    "moert_cuda_route_counts_enable": (i32, [i32, i32]),
    "moert_cuda_route_counts_fetch": (i32, [vp, i32]),
    "moert_cuda_host_register_pinned": (i32, [vp, u64]),
    "moert_cuda_host_unregister": (None, [vp]),
    "moert_cuda_host_register_mapped": (i32, [vp, u64]),
    "moert_cuda_host_map": (vp, [vp, u64]),
    "moert_cuda_stats_get": (None, [C.POINTER(MoertCudaStats)]),
    "moert_cuda_dir_init": (i32, [i32, i32, i32]),
    "moert_cuda_dir_async": (i32, [vp, vp, u64]),
    "moert_cuda_dir_mark": (i64, []),
    "moert_cuda_dir_poll": (i64, [i32]),
    "moert_cuda_publish_h2d": (i32, [i32, vp, vp, vp]),
    "moert_cuda_dir_stats_get": (None, [C.POINTER(MoertCudaDirStats)]),
    "moert_cuda_dir_gate": (i64, [i32, i64]),
    "moert_cuda_set_hot_table": (None, [i32, i32, vp, i32, i32]),
    # llapis_moe.h
    "llapis_last_error": (C.c_char_p, []),
    "llapis_set_modes": (None, [i32, i32]),
    "llapis_row_size": (u64, [i32, i64]),
    "llapis_quantize": (u64, [i32, vp, vp, i64, i64, vp]),
    "llapis_synth_normal": (None, [u64, i64, i64, C.c_float, C.c_float, vp]),
    "llapis_mul_mat_id": (i32, [C.POINTER(MoertMmCall), i32, vp, i64, i32, i32, vp]),
    "llapis_moe_dual_workspace_size": (u64, [C.POINTER(LlapisMoeDualOp)]),
    "llapis_moe_dual_compute": (i32, [C.POINTER(LlapisMoeDualOp), vp, u64, vp]),
    "llapis_router_topk": (i32, [vp, i32, vp, vp, i32, i32, i32, vp, vp, vp, vp]),
    "llapis_geglu": (i32, [vp, i32, i32, vp, i32, vp]),
    "llapis_moe_combine": (i32, [vp, vp, i32, i32, i32, vp, vp]),
    "llapis_residual_rmsnorm": (i32, [vp, vp, i32, i32, C.c_float, vp, vp]),
    "llapis_moe_ffn_workspace_size": (u64, [C.POINTER(LlapisMoeLayer), i32]),
    "llapis_moe_ffn": (i32, [C.POINTER(LlapisMoeLayer), vp, vp, i32, vp, vp, vp, vp, u64, vp]),
    "llapis_moe_ffn_workspace_init": (i32, [C.POINTER(LlapisMoeLayer), vp, u64, vp]),
    "llapis_moe_ffn_noalloc": (i32, [C.POINTER(LlapisMoeLayer), vp, vp, i32, vp, vp, vp, vp]),
    "llapis_set_tuning": (None, [i32, i32]),
    "llapis_profile_enable": (None, [i32]),
    "llapis_profile_read": (i32, [vp, i32]),
    "llapis_xfer_create": (vp, [i32, i32, i32, i32]),
    "llapis_xfer_free": (None, [vp]),
    "llapis_xfer_last_error": (C.c_char_p, []),
    "llapis_xfer_set_group": (i32, [vp, i32, i32, vp, vp, u64, u64]),
    "llapis_xfer_submit": (i32, [vp, i32, i32, i32]),
    "llapis_xfer_flush": (i32, [vp, vp]),
    "llapis_xfer_take_done": (i32, [vp, C.POINTER(LlapisXferDone), i32]),
    "llapis_xfer_in_flight": (i64, [vp]),
    "llapis_xfer_wait_idle": (i32, [vp, vp]),
    "llapis_xfer_get_stats": (None, [vp, C.POINTER(LlapisXferStats)]),
    "llapis_kfit": (None, [C.POINTER(LlapisKfitInputs), C.POINTER(LlapisKfitDecision)]),
    "llapis_device_memory_mib": (i32, [C.POINTER(C.c_longlong), C.POINTER(C.c_longlong)]),
    "llapis_files_last_error": (C.c_char_p, []),
    "llapis_gguf_open": (vp, [C.c_char_p]),
    "llapis_gguf_close": (None, [vp]),
    "llapis_gguf_n_tensors": (i64, [vp]),
    "llapis_gguf_data_offset": (u64, [vp]),
    "llapis_gguf_alignment": (u64, [vp]),
    "llapis_gguf_tensor": (i32, [vp, i64, C.POINTER(LlapisGgufTensorInfo)]),
    "llapis_gguf_find": (i64, [vp, C.c_char_p]),
    "llapis_gguf_expert_group": (i32, [vp, i32, i32, i32, i32, C.POINTER(LlapisPageGroup)]),
    "llapis_gguf_upload": (i32, [vp, C.POINTER(LlapisPageGroup), i32, i32, vp, vp]),
    "llapis_store_upload": (i32, [vp, i32, i32, i32, vp, i32, vp, u64, i32, vp]),
    "llapis_residency_create": (vp, [vp, i32]),
    "llapis_residency_free": (None, [vp]),
    "llapis_residency_last_error": (C.c_char_p, []),
    "llapis_residency_policy": (vp, [vp]),
    "llapis_residency_xfer": (vp, [vp]),
    "llapis_residency_set_mirrors": (i32, [vp, i32, vp, vp, vp]),
    "llapis_residency_counters": (i32, [vp, i32, C.POINTER(vp), C.POINTER(vp)]),
    "llapis_residency_publish_all": (i32, [vp, vp]),
    "llapis_residency_token_end": (i32, [vp, vp]),
    "llapis_residency_refresh": (i32, [vp, i32, vp]),
    "llapis_residency_get_stats": (None, [vp, C.POINTER(LlapisResidencyStats)]),
    **POLICY_SIGNATURES,
    **STORE_SIGNATURES,
}

STAGES = ("router", "topk", "gate_up", "down", "combine")

_lib = None


def lib():
    """The loaded library (loaded once).  Raises if it is not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built: run `python -m llapis_amd.build` first")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


class LlapisError(RuntimeError):
    pass


def check(rc, what):
    if rc != 0:
        raise LlapisError(f"{what}: {lib().llapis_last_error().decode()}")
