"""ctypes access to the two CPU checkers.  TEST INFRASTRUCTURE ONLY.

``Oracle`` wraps liboracle.so (the C restatement in oracle.c); ``Ref`` wraps
_ref/libggml_ref.so (the reference's own ggml CPU path built from its sources
by oracle/Makefile).  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this module.
"""
import ctypes as C
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent

F32, Q5_0, Q8_0, Q8_1, Q4_K, Q8_K, IQ4_NL, IQ2_S = 0, 6, 8, 9, 12, 15, 20, 22
ACT_CPU, ACT_Q8_1, ACT_Q8_1_MMA = 0, 1, 2
GELU_TABLE, GELU_TANH = 0, 1

_BLOCK = {Q4_K: (256, 144), IQ2_S: (256, 82), Q5_0: (32, 22), IQ4_NL: (32, 18),
          Q8_K: (256, 292), Q8_0: (32, 34), Q8_1: (32, 36), F32: (1, 4)}


def row_size(t, n):
    qk, b = _BLOCK[t]
    assert n % qk == 0, (t, n)
    return n // qk * b


def _p(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class Oracle:
    def __init__(self, path=None):
        lib = C.CDLL(str(path or HERE / "liboracle.so"))
        vp, i64, i32 = C.c_void_p, C.c_int64, C.c_int
        lib.orc_dequantize.argtypes = [i32, vp, vp, i64]
        lib.orc_quantize_act.argtypes = [i32, vp, vp, i64]
        lib.orc_vec_dot.argtypes = [i32, i32, i64, vp, vp]
        lib.orc_vec_dot.restype = C.c_float
        lib.orc_act_type.argtypes = [i32, i32]
        lib.orc_matvec.argtypes = [i32, i32, vp, i64, i64, vp, vp]
        lib.orc_geglu.argtypes = [vp, vp, vp, i64, i32]
        lib.orc_router.argtypes = [vp, i64, vp, vp, i64, i64, i64, vp, vp, vp]
        lib.orc_moe_experts.argtypes = [vp, vp, i64, vp, vp, i32, i32, vp, vp]
        lib.orc_set_sum_jitter.argtypes = [C.c_uint64]
        lib.orc_set_sum_jitter.restype = None
        lib.orc_fp32_to_fp16.argtypes = [C.c_float]
        lib.orc_fp32_to_fp16.restype = C.c_uint16
        lib.orc_fp16_to_fp32.argtypes = [C.c_uint16]
        lib.orc_fp16_to_fp32.restype = C.c_float
        self.lib = lib

    def dequantize(self, t, q, n):
        y = np.empty(n, np.float32)
        self.lib.orc_dequantize(t, _p(np.ascontiguousarray(q)), _p(y), n)
        return y

    def act_type(self, wtype, mode):
        return self.lib.orc_act_type(wtype, mode)

    def quantize_act(self, at, x):
        x = _f32(x)
        y = np.zeros(row_size(at, x.size), np.uint8)
        self.lib.orc_quantize_act(at, _p(x), _p(y), x.size)
        return y

    def vec_dot(self, wtype, mode, n, w, a):
        return self.lib.orc_vec_dot(wtype, mode, n, _p(np.ascontiguousarray(w)), _p(np.ascontiguousarray(a)))

    def matvec(self, wtype, mode, w, nrows, ncols, x):
        y = np.empty(nrows, np.float32)
        self.lib.orc_matvec(wtype, mode, _p(np.ascontiguousarray(w)), nrows, ncols, _p(_f32(x)), _p(y))
        return y

    def geglu(self, g, u, mode):
        g, u = _f32(g), _f32(u)
        out = np.empty_like(g)
        self.lib.orc_geglu(_p(g), _p(u), _p(out), g.size, mode)
        return out

    def router(self, x, w_r, bias, top_k):
        x, w_r = _f32(x), _f32(w_r)
        T, d = x.shape
        E = w_r.shape[0]
        ids = np.empty((T, top_k), np.int32)
        w = np.empty((T, top_k), np.float32)
        probs = np.empty((T, E), np.float32)
        b = _f32(bias) if bias is not None else None
        self.lib.orc_router(_p(x), T, _p(w_r), _p(b), d, E, top_k, _p(ids), _p(w), _p(probs))
        return ids, w, probs

    def set_sum_jitter(self, seed):
        """A control for chained-layer tests (0: off): every gate_up and down
        matvec output moved one ulp up or down by a seeded coin."""
        self.lib.orc_set_sum_jitter(int(seed))

    def moe_experts(self, L, x, ids, w, act_mode=ACT_CPU, gelu_mode=GELU_TABLE):
        """L: a LayerData-like object (see tests/helpers.py) with numpy fields."""
        x = _f32(x)
        T = x.shape[0]

        class S(C.Structure):
            _fields_ = [("d_model", C.c_int64), ("n_ff", C.c_int64), ("n_expert", C.c_int64),
                        ("top_k", C.c_int64), ("k_slots", C.c_int64),
                        ("hot_gu_type", C.c_int32), ("hot_dn_type", C.c_int32),
                        ("cold_gu_type", C.c_int32), ("cold_dn_type", C.c_int32),
                        ("hot_gu", C.c_void_p), ("hot_dn", C.c_void_p),
                        ("cold_gu", C.c_void_p), ("cold_dn", C.c_void_p),
                        ("exp_slot", C.c_void_p), ("slot_exp", C.c_void_p), ("slot_state", C.c_void_p),
                        ("s_hot", C.c_void_p), ("s_cold", C.c_void_p)]

        keep = []

        def ptr(a, dt=None):
            if a is None:
                return None
            a = np.ascontiguousarray(a, dtype=dt) if dt else np.ascontiguousarray(a)
            keep.append(a)
            return a.ctypes.data

        s = S(L.d_model, L.n_ff, L.n_expert, L.top_k, L.k_slots,
              L.hot_gu_type, L.hot_dn_type, L.cold_gu_type, L.cold_dn_type,
              ptr(L.hot_gu), ptr(L.hot_dn), ptr(L.cold_gu), ptr(L.cold_dn),
              ptr(L.exp_slot, np.int32), ptr(L.slot_exp, np.int32), ptr(L.slot_state, np.int32),
              ptr(L.s_hot, np.float32), ptr(L.s_cold, np.float32))
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        w = _f32(w)
        out = np.empty((T, L.d_model), np.float32)
        yp = np.empty((T * L.top_k, L.d_model), np.float32)
        self.lib.orc_moe_experts(C.byref(s), _p(x), T, _p(ids), _p(w), act_mode, gelu_mode, _p(out), _p(yp))
        return out, yp


class Ref:
    def __init__(self, path=None):
        p = Path(path) if path else HERE / "_ref" / "libggml_ref.so"
        if not p.exists():
            raise FileNotFoundError(f"{p} not built (run make -C oracle)")
        lib = C.CDLL(str(p))
        vp, i64, i32 = C.c_void_p, C.c_int64, C.c_int
        lib.ref_quantize.argtypes = [i32, vp, vp, i64, i64, vp]
        lib.ref_quantize.restype = C.c_size_t
        lib.ref_dequantize.argtypes = [i32, vp, vp, i64]
        lib.ref_row_size.argtypes = [i32, i64]
        lib.ref_row_size.restype = C.c_size_t
        lib.ref_vec_dot_type.argtypes = [i32]
        lib.ref_quantize_act.argtypes = [i32, vp, vp, i64]
        lib.ref_vec_dot.argtypes = [i32, i64, vp, vp]
        lib.ref_vec_dot.restype = C.c_float
        lib.ref_mul_mat_id.argtypes = [i32, vp, i64, i64, i64, vp, i64, vp, i64, vp, i32]
        lib.ref_geglu.argtypes = [vp, vp, vp, i64, i64]
        lib.ref_layer_create.argtypes = [vp, vp, i64, i64, i64, i32, vp, i32, vp, i64, i64]
        lib.ref_layer_create.restype = vp
        lib.ref_layer_run.argtypes = [vp, vp, vp, vp, vp, i32]
        lib.ref_layer_free.argtypes = [vp]
        lib.ref_dual_create.argtypes = [vp, vp, i64, i64, i64, i64, i64, vp, i64, i32, vp, i32, vp, i32, vp, i32, vp,
                                        i32]
        lib.ref_dual_create.restype = vp
        lib.ref_dual_run.argtypes = [vp, vp, vp, vp, vp]
        lib.ref_dual_free.argtypes = [vp]
        self.lib = lib

    def quantize(self, t, x, imatrix=None):
        x = _f32(x)
        nrow, n = x.shape
        out = np.zeros(nrow * row_size(t, n), np.uint8)
        im = _f32(imatrix) if imatrix is not None else None
        self.lib.ref_quantize(t, _p(x), _p(out), nrow, n, _p(im))
        return out

    def dequantize(self, t, q, n):
        y = np.empty(n, np.float32)
        self.lib.ref_dequantize(t, _p(np.ascontiguousarray(q)), _p(y), n)
        return y

    def vec_dot_type(self, t):
        return self.lib.ref_vec_dot_type(t)

    def quantize_act(self, at, x):
        x = _f32(x)
        y = np.zeros(row_size(at, x.size), np.uint8)
        self.lib.ref_quantize_act(at, _p(x), _p(y), x.size)
        return y

    def vec_dot(self, t, n, w, a):
        return self.lib.ref_vec_dot(t, n, _p(np.ascontiguousarray(w)), _p(np.ascontiguousarray(a)))

    def mul_mat_id(self, t, w, d_in, d_out, n_pool, x, ids, n_threads=1):
        x = _f32(x)
        n_cols = x.shape[0] if x.ndim == 2 else 1
        ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
        y = np.empty((ids.size, d_out), np.float32)
        self.lib.ref_mul_mat_id(t, _p(np.ascontiguousarray(w)), d_in, d_out, n_pool, _p(x), n_cols,
                                _p(ids), ids.size, _p(y), n_threads)
        return y

    def geglu(self, g, u):
        g, u = _f32(g), _f32(u)
        n = g.shape[-1]
        cols = g.size // n
        out = np.empty_like(g)
        self.lib.ref_geglu(_p(g), _p(u), _p(out), n, cols)
        return out

    def layer(self, w_r, bias, top_k, gu_type, w_gu, dn_type, w_dn, n_ff, T):
        return RefLayer(self, w_r, bias, top_k, gu_type, w_gu, dn_type, w_dn, n_ff, T)

    def dual(self, L, T, n_threads=1):
        """The reference's CPU path for a dual-precision layer: ggml graph for
        the routing and the hot pairs, its CPU cold executor for the cold
        pairs (ref_dual.cpp).  L: a LayerData-like object with numpy fields
        and a residency (slot_of via exp_slot with every slot READY)."""
        return RefDual(self, L, T, n_threads)


class RefLayer:
    """A built single-tier ggml MoE layer graph (reference CPU path)."""

    def __init__(self, ref, w_r, bias, top_k, gu_type, w_gu, dn_type, w_dn, n_ff, T):
        self.ref, self.T, self.k = ref, T, top_k
        w_r = _f32(w_r)
        self.E, self.d = w_r.shape
        b = _f32(bias) if bias is not None else None
        self.h = ref.lib.ref_layer_create(_p(w_r), _p(b), self.d, self.E, top_k, gu_type,
                                          _p(np.ascontiguousarray(w_gu)), dn_type,
                                          _p(np.ascontiguousarray(w_dn)), n_ff, T)

    def run(self, x, n_threads=1, want_routing=True):
        x = _f32(x)
        out = np.empty((self.T, self.d), np.float32)
        ids = np.empty((self.T, self.k), np.int32) if want_routing else None
        w = np.empty((self.T, self.k), np.float32) if want_routing else None
        self.ref.lib.ref_layer_run(self.h, _p(x), _p(out), _p(ids), _p(w), n_threads)
        return out, ids, w

    def __del__(self):
        if getattr(self, "h", None):
            self.ref.lib.ref_layer_free(self.h)
            self.h = None


class RefDual:
    """A built dual-precision layer over the reference's ggml graph and CPU
    cold executor.  The cold pools stay the caller's arrays (kept alive here)."""

    def __init__(self, ref, L, T, n_threads=1):
        self.ref, self.T, self.k, self.d = ref, T, L.top_k, L.d_model
        r = L.residency
        slot_of = np.full(L.n_expert, -1, np.int32)
        for e in range(L.n_expert):
            if r.is_hot(e):
                slot_of[e] = int(r.exp_slot[e])
        self._keep = [np.ascontiguousarray(a) for a in (L.router_w, L.hot_gu, L.hot_dn, L.cold_gu, L.cold_dn)]
        self._keep[0] = _f32(self._keep[0])
        b = _f32(L.router_b) if L.router_b is not None else None
        self._keep.append(b)
        self._keep.append(slot_of)
        k_slots = max(int(L.k_slots), 1)
        self.h = ref.lib.ref_dual_create(_p(self._keep[0]), _p(b), L.d_model, L.n_expert, L.top_k, L.n_ff, T,
                                         _p(slot_of), k_slots, L.hot_gu_type, _p(self._keep[1]), L.hot_dn_type,
                                         _p(self._keep[2]), L.cold_gu_type, _p(self._keep[3]), L.cold_dn_type,
                                         _p(self._keep[4]), n_threads)

    def run(self, x):
        x = _f32(x)
        out = np.empty((self.T, self.d), np.float32)
        ids = np.empty((self.T, self.k), np.int32)
        n_hot = np.zeros(1, np.int32)
        self.ref.lib.ref_dual_run(self.h, _p(x), _p(out), _p(ids), _p(n_hot))
        return out, ids, int(n_hot[0])

    def __del__(self):
        if getattr(self, "h", None):
            self.ref.lib.ref_dual_free(self.h)
            self.h = None
