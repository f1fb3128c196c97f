"""Python handle of the residency policy (include/moert_policy.h).

The policy is the library's C++ (llapis_amd/csrc/policy.cpp); this class only
holds the handle, keeps the ctypes callbacks alive and copies views out.  Any
library exporting the same C ABI can be passed as `lib`.
"""
import ctypes as C

import numpy as np

from . import _lib as L


def bind(cdll):
    """Set the moert_policy_* signatures on a loaded library; returns it."""
    for name, (res, args) in L.POLICY_SIGNATURES.items():
        fn = getattr(cdll, name)
        fn.restype = res
        fn.argtypes = args
    return cdll


# fields of moert_policy_stats that are wall-clock timings
TIMING_FIELDS = ("refresh_pause_ms_total", "refresh_pause_ms_max", "last_refresh_pause_ms")


def _config(lib, n_layers, n_expert, k, k_per_layer, cfg):
    c = L.MoertPolicyConfig()
    lib.moert_policy_config_defaults(C.byref(c))
    c.n_layers, c.n_expert, c.k = n_layers, n_expert, k
    for name, v in cfg.items():
        if not hasattr(c, name):
            raise TypeError(f"no config field {name}")
        setattr(c, name, v)
    kpl = None
    if k_per_layer is not None:
        kpl = (L.i32 * n_layers)(*k_per_layer)
        c.k_per_layer = C.cast(kpl, C.c_void_p)
    return c, kpl


class Policy:
    """moert_policy with Python callbacks.

    stream_expert(il, e, slot) -> 0 | 1 | 2, publish_layer(il) and
    fetch_external() are optional callables; config fields of
    moert_policy_config may be overridden by keyword (cost_reuse=51.0, ...).
    """

    def __init__(self, n_layers, n_expert, k, lib=None, k_per_layer=None, stream_expert=None, publish_layer=None,
                 fetch_external=None, **cfg):
        self.lib = lib if lib is not None else L.lib()
        c, self._kpl = _config(self.lib, n_layers, n_expert, k, k_per_layer, cfg)
        self._owned = True
        cb = L.MoertPolicyCallbacks()
        self._cbs = []
        if stream_expert is not None:
            f = L.STREAM_EXPERT(lambda u, il, e, s: int(stream_expert(il, e, s)))
            self._cbs.append(f)
            cb.stream_expert = f
        if publish_layer is not None:
            f = L.PUBLISH_LAYER(lambda u, il: publish_layer(il))
            self._cbs.append(f)
            cb.publish_layer = f
        if fetch_external is not None:
            f = L.FETCH_EXTERNAL(lambda u: fetch_external())
            self._cbs.append(f)
            cb.fetch_external = f
        self.n_layers, self.n_expert = n_layers, n_expert
        self.p = self.lib.moert_policy_create(C.byref(c), C.byref(cb))
        if not self.p:
            raise ValueError("moert_policy_create refused the configuration")
        self._forecast = None

    @classmethod
    def wrap(cls, p, n_layers, n_expert, lib=None):
        """A view of a policy that something else owns and frees (the
        residency runtime's)."""
        self = cls.__new__(cls)
        self.lib = lib if lib is not None else L.lib()
        self.p, self.n_layers, self.n_expert = p, n_layers, n_expert
        self._kpl, self._cbs, self._forecast, self._owned = None, [], None, False
        return self

    def close(self):
        if self.p and self._owned:
            self.lib.moert_policy_free(self.p)
        self.p = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- observation and decisions
    def observe(self, il, ids, n_used, n_tok):
        a = np.ascontiguousarray(ids, dtype=np.int32)
        self.lib.moert_policy_observe(self.p, il, a.ctypes.data, n_used, n_tok)

    def token_end(self):
        self.lib.moert_policy_on_token_end(self.p)

    def prompt_tokens(self, n):
        self.lib.moert_policy_on_prompt_token(self.p, n)

    def refresh(self, reason):
        self.lib.moert_policy_refresh(self.p, reason)

    def set_external(self, on):
        self.lib.moert_policy_set_external_observation(self.p, int(on))

    def add_counts(self, il, counts, hot, cold):
        a = np.ascontiguousarray(counts, dtype=np.int32)
        self.lib.moert_policy_add_external_counts(self.p, il, a.ctypes.data, int(hot), int(cold))

    def set_forecast(self, f, r, cap):
        """f: [n_layers, n_expert] float32 (kept alive here) or None."""
        self._forecast = None if f is None else np.ascontiguousarray(f, dtype=np.float32)
        ptr = None if self._forecast is None else self._forecast.ctypes.data
        self.lib.moert_policy_set_external_forecast(self.p, ptr, r, cap)

    def boundary(self, il, counts, n_tok, weight, r):
        a = np.ascontiguousarray(counts, dtype=np.int32)
        return self.lib.moert_policy_boundary_layer(self.p, il, a.ctypes.data, n_tok, weight, r)

    # ---- slots
    def seed(self, il, e, slot):
        return self.lib.moert_policy_commit_seed(self.p, il, e, slot)

    def can_seed(self, il, e):
        return self.lib.moert_policy_can_seed(self.p, il, e)

    def complete(self, il, slot, e):
        return self.lib.moert_policy_complete_fill(self.p, il, slot, e)

    def abort(self, il, slot, e):
        return self.lib.moert_policy_abort_fill(self.p, il, slot, e)

    def resize(self, k):
        return self.lib.moert_policy_resize_k(self.p, k)

    def active_k(self, k):
        return self.lib.moert_policy_set_active_k(self.p, k)

    def layer_k(self, il):
        return self.lib.moert_policy_layer_k(self.p, il)

    def reset_stats(self):
        self.lib.moert_policy_reset_stats(self.p)

    # ---- reads
    def views(self, il):
        """Copies of layer il's page table and mirrors."""
        k = self.layer_k(il)
        E = self.n_expert
        grab = lambda ptr, n, dt: np.ctypeslib.as_array(ptr, shape=(n,)).astype(dt, copy=True)
        return {"exp_slot": grab(self.lib.moert_policy_exp_slot_view(self.p, il), E, np.int32),
                "slot_exp": grab(self.lib.moert_policy_slot_exp_view(self.p, il), k, np.int32),
                "slot_state": grab(self.lib.moert_policy_slot_state_view(self.p, il), k, np.int32),
                "hotmap": grab(self.lib.moert_policy_hotmap_view(self.p, il), E, np.int32),
                "resid": grab(self.lib.moert_policy_resid_view(self.p, il), E, np.float32)}

    def stats(self):
        s = L.MoertPolicyStats()
        self.lib.moert_policy_get_stats(self.p, C.byref(s))
        return {f: getattr(s, f) for f, _ in s._fields_}

    def hit_rate(self):
        return self.lib.moert_policy_hit_rate(self.p)

    def window(self, n):
        w = L.MoertPolicyWindow()
        self.lib.moert_policy_get_window(self.p, n, C.byref(w))
        return {f: getattr(w, f) for f, _ in w._fields_}


class ResidencyLoop:
    """The native per-token residency loop (llapis_residency_*): a policy on
    external observation, a promotion engine and every layer's device routing
    counters.  `policy` views the runtime's policy (seed, views, stats);
    `xfer` is its engine handle (set its page groups with
    llapis_xfer_set_group).  Config keywords as Policy's."""

    def __init__(self, n_layers, n_expert, k, copy_wgs=0, lib=None, k_per_layer=None, **cfg):
        self.lib = lib if lib is not None else L.lib()
        c, self._kpl = _config(self.lib, n_layers, n_expert, k, k_per_layer, cfg)
        self.r = self.lib.llapis_residency_create(C.byref(c), copy_wgs)
        if not self.r:
            raise RuntimeError(self.lib.llapis_residency_last_error().decode())
        self.policy = Policy.wrap(self.lib.llapis_residency_policy(self.r), n_layers, n_expert, self.lib)
        self.xfer = self.lib.llapis_residency_xfer(self.r)

    def _check(self, rc):
        if rc != 0:
            raise RuntimeError(self.lib.llapis_residency_last_error().decode())

    def counters(self, il):
        """Device addresses of layer il's counters: (counts [n_expert], hits [2])."""
        cp, hp = C.c_void_p(), C.c_void_p()
        self._check(self.lib.llapis_residency_counters(self.r, il, C.byref(cp), C.byref(hp)))
        return cp.value, hp.value

    def set_mirrors(self, il, exp_slot, slot_exp, slot_state):
        self._check(self.lib.llapis_residency_set_mirrors(self.r, il, exp_slot, slot_exp, slot_state))

    def publish_all(self, stream):
        self._check(self.lib.llapis_residency_publish_all(self.r, stream))

    def token_end(self, stream):
        self._check(self.lib.llapis_residency_token_end(self.r, stream))

    def refresh(self, reason, stream):
        """A prompt-end / turn-end decision (L.REFRESH_*) with the counters drained."""
        self._check(self.lib.llapis_residency_refresh(self.r, reason, stream))

    def stats(self):
        s = L.LlapisResidencyStats()
        self.lib.llapis_residency_get_stats(self.r, C.byref(s))
        return {f: getattr(s, f) for f, _ in s._fields_}

    def close(self):
        if self.r:
            self.policy.p = None
            self.lib.llapis_residency_free(self.r)
            self.r = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
