"""Host-side interface of the dual-precision MoE expert FFN.

Mirrors the reference's host objects for this path with the MI355X library
underneath (torch is used only for device memory and the current stream):

* ``Residency`` -- the hot/cold placement mask exactly as the reference
  publishes it to the device: exp_slot[E], slot_exp[K], slot_state[K] with
  FREE 0 / FILLING 1 / READY 2 (moert/include/moert/policy.h:46,
  src/moe_dual.cpp:691-705 push_residency, src/moe_dual_init.cpp:141-164).
* ``DualLayer`` -- one MoE layer's pools: the K-slot hot pool (Q4_K gate_up,
  Q5_0 down) and the all-expert cold pool (IQ2_S gate_up, IQ4_NL down), laid
  out as the reference's pool tensors [D_in, D_out, K] / [D_in, D_out, E]
  (src/moe_dual_init.cpp:73-110), plus the fp32 router.
* ``DeviceLayer.forward`` -- build_moe_ffn for the gemma4 merged gate_up MoE
  (third_party/llama/src/llama-graph.cpp:1507-1850) in one call.
* ``DeviceLayer.moe_dual`` -- one GGML_OP_MOE_DUAL fire (ggml.c:3322-3370,
  ggml-cuda/moe-dual.cu:98-157) through the island ABI.
"""
from dataclasses import dataclass, field

import copy
import ctypes as C
import numpy as np

from . import _lib as L
from ._lib import F32, IQ2_S, IQ4_NL, Q4_K, Q5_0, SLOT_READY, check, lib

_BLK = {Q4_K: (256, 144), IQ2_S: (256, 82), Q5_0: (32, 22), IQ4_NL: (32, 18)}


def row_size(t, n):
    r = int(lib().llapis_row_size(t, n))
    if r == 0:
        raise ValueError(f"type {t} cannot hold rows of {n}")
    return r


def quantize(t, x, imatrix=None):
    """ggml_quantize_chunk for a [nrow, n_per_row] float32 array -> uint8 bytes."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    nrow, n = x.shape
    out = np.empty(nrow * row_size(t, n), np.uint8)
    im = None if imatrix is None else np.ascontiguousarray(imatrix, dtype=np.float32)
    got = lib().llapis_quantize(t, x.ctypes.data, out.ctypes.data, nrow, n,
                                None if im is None else im.ctypes.data)
    if got != out.size:
        raise L.LlapisError(f"quantize(type={t}) refused")
    return out


def synth_normal(seed, n, mean=0.0, std=1.0, offset=0):
    out = np.empty(n, np.float32)
    lib().llapis_synth_normal(seed, offset, n, mean, std, out.ctypes.data)
    return out


def seed_for(layer_seed, expert, what):
    """Independent stream per (layer, expert, tensor kind)."""
    return (layer_seed * 1_000_003 + expert * 7 + what) & 0xFFFFFFFFFFFFFFFF


@dataclass
class Residency:
    """The placement mask mirrors.  hot_experts[s] is the expert in slot s."""
    n_expert: int
    k_slots: int
    exp_slot: np.ndarray = None
    slot_exp: np.ndarray = None
    slot_state: np.ndarray = None

    @classmethod
    def from_hot(cls, n_expert, hot_experts, state=SLOT_READY):
        k = len(hot_experts)
        r = cls(n_expert, k)
        r.exp_slot = np.full(n_expert, -1, np.int32)
        r.slot_exp = np.full(max(k, 1), -1, np.int32)
        r.slot_state = np.zeros(max(k, 1), np.int32)
        for s, e in enumerate(hot_experts):
            r.exp_slot[e] = s
            r.slot_exp[s] = e
            r.slot_state[s] = state
        return r

    def is_hot(self, e):
        s = int(self.exp_slot[e])
        return 0 <= s < self.k_slots and self.slot_state[s] == SLOT_READY and self.slot_exp[s] == e


@dataclass
class LayerSpec:
    d_model: int = 2816
    n_ff: int = 704
    n_expert: int = 128
    top_k: int = 8
    hot_gu_type: int = Q4_K
    hot_dn_type: int = Q5_0
    cold_gu_type: int = IQ2_S
    cold_dn_type: int = IQ4_NL

    def gu_bytes(self, t):
        return row_size(t, self.d_model) * 2 * self.n_ff

    def dn_bytes(self, t):
        return row_size(t, self.n_ff) * self.d_model


@dataclass
class DualLayer:
    spec: LayerSpec
    residency: Residency
    router_w: np.ndarray                 # [E][d_model] f32
    router_b: np.ndarray = None          # [E] f32 or None
    hot_gu: np.ndarray = None            # uint8 [K * gu_bytes(hot)]
    hot_dn: np.ndarray = None
    cold_gu: np.ndarray = None           # uint8 [E * gu_bytes(cold)]
    cold_dn: np.ndarray = None
    s_hot: np.ndarray = None             # [K] f32 or None
    s_cold: np.ndarray = None            # [E] f32 or None
    meta: dict = field(default_factory=dict)

    # field names the oracle's layer descriptor reads
    @property
    def d_model(self): return self.spec.d_model
    @property
    def n_ff(self): return self.spec.n_ff
    @property
    def n_expert(self): return self.spec.n_expert
    @property
    def top_k(self): return self.spec.top_k
    @property
    def k_slots(self): return self.residency.k_slots
    @property
    def hot_gu_type(self): return self.spec.hot_gu_type
    @property
    def hot_dn_type(self): return self.spec.hot_dn_type
    @property
    def cold_gu_type(self): return self.spec.cold_gu_type
    @property
    def cold_dn_type(self): return self.spec.cold_dn_type
    @property
    def exp_slot(self): return self.residency.exp_slot
    @property
    def slot_exp(self): return self.residency.slot_exp
    @property
    def slot_state(self): return self.residency.slot_state

    def expert_weights_f32(self, e, layer_seed):
        """Regenerate expert e's fp32 gate_up [2F, D] and down [D, F]."""
        sp = self.spec
        gu = synth_normal(seed_for(layer_seed, e, 1), 2 * sp.n_ff * sp.d_model, 0.0, 0.02)
        dn = synth_normal(seed_for(layer_seed, e, 2), sp.d_model * sp.n_ff, 0.0, 0.02)
        return gu.reshape(2 * sp.n_ff, sp.d_model), dn.reshape(sp.d_model, sp.n_ff)


def zipf_hot_set(n_expert, k, seed, s=1.1):
    """Routing-frequency prior Zipf(s) over a seeded permutation of the experts;
    the hot set is the k most frequent (prior, hot_experts)."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(n_expert)
    prior = np.empty(n_expert, np.float64)
    prior[perm] = 1.0 / np.arange(1, n_expert + 1) ** s
    prior /= prior.sum()
    hot = [int(e) for e in perm[:k]]
    return prior, hot


def make_layer(spec, layer_seed, hot_experts=(), router_bias=None, cold_imatrix_ones=True,
               scales=False, cold=True):
    """Synthetic layer per the benchmark spec: expert weights N(0, 0.02),
    quantised per tier (hot: Q4_K/Q5_0 without imatrix; cold: IQ2_S/IQ4_NL with
    an importance matrix of ones); router N(0, 0.02) fp32."""
    sp = spec
    res = Residency.from_hot(sp.n_expert, list(hot_experts))
    router_w = synth_normal(seed_for(layer_seed, 0, 0), sp.n_expert * sp.d_model, 0.0, 0.02)
    lay = DualLayer(sp, res, router_w.reshape(sp.n_expert, sp.d_model),
                    None if router_bias is None else np.asarray(router_bias, np.float32))
    gu_hot, dn_hot = sp.gu_bytes(sp.hot_gu_type), sp.dn_bytes(sp.hot_dn_type)
    gu_cold, dn_cold = sp.gu_bytes(sp.cold_gu_type), sp.dn_bytes(sp.cold_dn_type)
    K = res.k_slots
    lay.hot_gu = np.zeros(max(K, 1) * gu_hot, np.uint8)
    lay.hot_dn = np.zeros(max(K, 1) * dn_hot, np.uint8)
    if cold:
        lay.cold_gu = np.zeros(sp.n_expert * gu_cold, np.uint8)
        lay.cold_dn = np.zeros(sp.n_expert * dn_cold, np.uint8)
    im_gu = np.ones(sp.d_model, np.float32) if cold_imatrix_ones else None
    im_dn = np.ones(sp.n_ff, np.float32) if cold_imatrix_ones else None
    slot_of = {e: s for s, e in enumerate(hot_experts)}
    for e in range(sp.n_expert):
        if not cold and e not in slot_of:
            continue
        gu, dn = lay.expert_weights_f32(e, layer_seed)
        if e in slot_of:
            s = slot_of[e]
            lay.hot_gu[s * gu_hot:(s + 1) * gu_hot] = quantize(sp.hot_gu_type, gu)
            lay.hot_dn[s * dn_hot:(s + 1) * dn_hot] = quantize(sp.hot_dn_type, dn)
        if cold:
            lay.cold_gu[e * gu_cold:(e + 1) * gu_cold] = quantize(sp.cold_gu_type, gu, im_gu)
            lay.cold_dn[e * dn_cold:(e + 1) * dn_cold] = quantize(sp.cold_dn_type, dn, im_dn)
    if scales:
        lay.s_hot = (1.0 + 0.25 * synth_normal(seed_for(layer_seed, 0, 3), max(K, 1))).astype(np.float32)
        lay.s_cold = (1.0 + 0.25 * synth_normal(seed_for(layer_seed, 0, 4), sp.n_expert)).astype(np.float32)
    lay.meta["layer_seed"] = layer_seed
    return lay


def tune_router_bias(router_w, prior, hot, target, seed, n_tok=256, top_k=8):
    """Bias b = alpha * log(prior) so that about `target` of the top_k picks of
    N(0,1) tokens land on hot experts (bisection on alpha; host-side setup)."""
    x = np.random.default_rng(seed).standard_normal((n_tok, router_w.shape[1])).astype(np.float32)
    logits = x @ router_w.T.astype(np.float32)
    hot_mask = np.zeros(router_w.shape[0], bool)
    hot_mask[list(hot)] = True
    logp = np.log(prior)

    def frac(alpha):
        z = logits + alpha * logp
        sel = np.argpartition(-z, top_k - 1, axis=1)[:, :top_k]
        return hot_mask[sel].mean()

    lo, hi = 0.0, 10.0
    for _ in range(40):
        mid = 0.5 * (lo + hi)
        if frac(mid) < target:
            lo = mid
        else:
            hi = mid
    alpha = 0.5 * (lo + hi)
    return (alpha * logp).astype(np.float32), frac(alpha)


# ------------------------------------------------------------ device side

def _torch():
    import torch
    return torch


def _ptr(t):
    """A device address: None, a raw address (int) or a tensor's."""
    return None if t is None else t if isinstance(t, int) else t.data_ptr()


class DeviceLayer:
    """A DualLayer resident in HBM (one torch uint8 tensor per pool)."""

    def __init__(self, layer, device="cuda", act_mode=L.ACT_CPU, gelu_mode=L.GELU_TABLE):
        torch = _torch()
        self.layer, self.device = layer, device
        self.act_mode, self.gelu_mode = act_mode, gelu_mode
        up = lambda a, dt=None: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(device)
        self.router_w = up(layer.router_w)
        self.router_b = up(layer.router_b)
        self.hot_gu, self.hot_dn = up(layer.hot_gu), up(layer.hot_dn)
        self.cold_gu, self.cold_dn = up(layer.cold_gu), up(layer.cold_dn)
        self.exp_slot, self.slot_exp = up(layer.exp_slot), up(layer.slot_exp)
        self.slot_state = up(layer.slot_state)
        self.s_hot, self.s_cold = up(layer.s_hot), up(layer.s_cold)
        self.route_counts = self.route_hits = None   # optional int32 [n_expert], [2]: tensors or addresses
        self._ws = None

    def desc(self):
        sp, r = self.layer.spec, self.layer.residency
        return L.LlapisMoeLayer(sp.d_model, sp.n_ff, sp.n_expert, sp.top_k, r.k_slots,
                                sp.hot_gu_type, sp.hot_dn_type, sp.cold_gu_type, sp.cold_dn_type,
                                self.act_mode, self.gelu_mode,
                                _ptr(self.router_w), _ptr(self.router_b), _ptr(self.hot_gu), _ptr(self.hot_dn),
                                _ptr(self.cold_gu), _ptr(self.cold_dn), _ptr(self.exp_slot), _ptr(self.slot_exp),
                                _ptr(self.slot_state), _ptr(self.s_hot), _ptr(self.s_cold),
                                _ptr(self.route_counts), _ptr(self.route_hits))

    def q4stream(self, src_gu, src_dn, src_scales=None):
        """The reference's q4stream prefill (moe_dual_q4stream.cpp:723, 1123;
        the hook's n_tokens > 1 branch, moe_dual.cpp:205-227): every expert of
        a chunk at the hot tier's precision.  The reference stages each
        layer's experts into a full-layer tensor at its top-k callback; here
        the promotion source (every expert in the hot formats, resident in
        HBM: src_gu / src_dn uint8 [n_expert * bytes per expert], src_scales
        f32 [n_expert] when the layer has .scale factors) is that tensor
        already, so nothing is copied.  The returned view shares this layer's
        router, cold pools and counters and reads its hot pool from the source
        with n_expert slots and the identity page table."""
        torch = _torch()
        sp = self.layer.spec
        E = sp.n_expert
        nbytes = lambda t: t.numel() * t.element_size()
        if nbytes(src_gu) < E * sp.gu_bytes(sp.hot_gu_type) or nbytes(src_dn) < E * sp.dn_bytes(sp.hot_dn_type):
            raise ValueError("q4stream: the source must hold every expert in the hot formats")
        if (self.s_hot is None) != (src_scales is None) or (src_scales is not None and src_scales.numel() < E):
            raise ValueError("q4stream: scales for every expert exactly when the layer has scales")
        v = copy.copy(self)
        v.layer = copy.copy(self.layer)
        v.layer.residency = Residency.from_hot(E, list(range(E)))
        v.hot_gu, v.hot_dn, v.s_hot = src_gu, src_dn, src_scales
        v.exp_slot = torch.arange(E, dtype=torch.int32, device=self.device)
        v.slot_exp = v.exp_slot.clone()
        v.slot_state = torch.full((E,), SLOT_READY, dtype=torch.int32, device=self.device)
        v._ws = None
        return v

    def workspace(self, n_tokens):
        torch = _torch()
        d = self.desc()
        need = int(lib().llapis_moe_ffn_workspace_size(C.byref(d), n_tokens))
        if self._ws is None or self._ws.numel() < need:
            # zero-filled: the decode path keeps its control block here
            self._ws = torch.zeros(need, dtype=torch.uint8, device=self.device)
        return self._ws

    def forward(self, x, out=None, ids=None, weights=None, stream=None, x_router=None):
        """x: [T, d_model] f32 device tensor (the experts' input) -> out [T, d_model]
        (+ ids, weights).  x_router: the router's input, same shape (None: x)."""
        torch = _torch()
        T = x.shape[0]
        if x_router is not None and (tuple(x_router.shape) != tuple(x.shape) or not x_router.is_contiguous()):
            raise ValueError("x_router must be a contiguous tensor shaped like x")
        sp = self.layer.spec
        out = out if out is not None else torch.empty(T, sp.d_model, dtype=torch.float32, device=self.device)
        ids = ids if ids is not None else torch.empty(T, sp.top_k, dtype=torch.int32, device=self.device)
        weights = weights if weights is not None else torch.empty(T, sp.top_k, dtype=torch.float32,
                                                                  device=self.device)
        ws = self.workspace(T)
        d = self.desc()
        s = stream if stream is not None else torch.cuda.current_stream().cuda_stream
        xr = x_router.data_ptr() if x_router is not None else None
        check(lib().llapis_moe_ffn(C.byref(d), x.data_ptr(), xr, T, out.data_ptr(), ids.data_ptr(),
                                   weights.data_ptr(), ws.data_ptr(), ws.numel(), s), "llapis_moe_ffn")
        return out, ids, weights

    # ---- the GGML_OP_MOE_DUAL fire through the island ABI
    def moe_dual(self, kind, cur, ids, il=0, ids_row_stride=None):
        """kind 0: cur [T, d_model] -> dst [T, top_k, 2 n_ff];  kind 1: cur [T*top_k, n_ff] -> [T, top_k, d_model].
        ids: [T, >= top_k] int32 device tensor (row stride ids_row_stride)."""
        torch = _torch()
        sp, r = self.layer.spec, self.layer.residency
        T = ids.shape[0]
        n_used = sp.top_k
        if kind == 0:
            d_in, d_out = sp.d_model, 2 * sp.n_ff
            hot, cold, ht, ct = self.hot_gu, self.cold_gu, sp.hot_gu_type, sp.cold_gu_type
            cur_ne1 = 1
        else:
            d_in, d_out = sp.n_ff, sp.d_model
            hot, cold, ht, ct = self.hot_dn, self.cold_dn, sp.hot_dn_type, sp.cold_dn_type
            cur_ne1 = n_used
        dst = torch.empty(T, n_used, d_out, dtype=torch.float32, device=self.device)
        keep = []

        def tensor(ttype, ne, data, elsize=None):
            t = L.LlapisTensor()
            t.type = ttype
            for i in range(4):
                t.ne[i] = ne[i] if i < len(ne) else 1
            if elsize is None:          # quantised rows
                t.nb[0] = 0
                t.nb[1] = row_size(ttype, ne[0])
            else:
                t.nb[0] = elsize
                t.nb[1] = elsize * ne[0]
            t.nb[2] = t.nb[1] * t.ne[1]
            t.nb[3] = t.nb[2] * t.ne[2]
            t.data = data
            keep.append(t)
            return C.pointer(t)

        stride = ids_row_stride if ids_row_stride is not None else ids.stride(0)
        t_ids = tensor(L.F32, [n_used, T], ids.data_ptr(), 4)
        t_ids.contents.type = 26        # GGML_TYPE_I32
        t_ids.contents.nb[1] = 4 * stride
        op = L.LlapisMoeDualOp()
        op.src[0] = tensor(F32, [d_in, cur_ne1, T], cur.data_ptr(), 4)
        op.src[1] = t_ids
        op.src[2] = tensor(ht, [d_in, d_out, max(r.k_slots, 1)], _ptr(hot))
        op.src[3] = tensor(ct, [d_in, d_out, sp.n_expert], _ptr(cold))
        op.src[4] = tensor(26, [sp.n_expert], _ptr(self.exp_slot), 4)
        op.src[5] = tensor(26, [max(r.k_slots, 1)], _ptr(self.slot_exp), 4)
        op.src[6] = tensor(26, [max(r.k_slots, 1)], _ptr(self.slot_state), 4)
        if kind == 1 and self.s_hot is not None:
            op.src[7] = tensor(F32, [max(r.k_slots, 1)], _ptr(self.s_hot), 4)
        if kind == 1 and self.s_cold is not None:
            op.src[8] = tensor(F32, [sp.n_expert], _ptr(self.s_cold), 4)
        prm = [kind, sp.top_k, il, ct, sp.n_expert, 0, 0, 0, 0, 0]
        for i, v in enumerate(prm):
            op.op_params[i] = v
        op.dst = tensor(F32, [d_out, n_used, T], dst.data_ptr(), 4)
        need = int(lib().llapis_moe_dual_workspace_size(C.byref(op)))
        ws = torch.empty(need, dtype=torch.uint8, device=self.device)
        lib().llapis_set_modes(self.act_mode, self.gelu_mode)
        s = torch.cuda.current_stream().cuda_stream
        check(lib().llapis_moe_dual_compute(C.byref(op), ws.data_ptr(), need, s), "llapis_moe_dual_compute")
        keep.append(ws)
        return dst

    def router(self, x):
        torch = _torch()
        sp = self.layer.spec
        T = x.shape[0]
        ids = torch.empty(T, sp.top_k, dtype=torch.int32, device=self.device)
        w = torch.empty(T, sp.top_k, dtype=torch.float32, device=self.device)
        probs = torch.empty(T, sp.n_expert, dtype=torch.float32, device=self.device)
        s = torch.cuda.current_stream().cuda_stream
        check(lib().llapis_router_topk(x.data_ptr(), T, self.router_w.data_ptr(), _ptr(self.router_b), sp.d_model,
                                       sp.n_expert, sp.top_k, ids.data_ptr(), w.data_ptr(), probs.data_ptr(), s),
              "llapis_router_topk")
        return ids, w, probs


def combine(y, weights):
    """out[t] = sum_k weights[t][k] y[t top_k + k] in k order (the graph's
    weighted sum of the down fire's outputs), y [T * top_k][d]."""
    torch = _torch()
    T, K = weights.shape
    d = y.shape[-1]
    out = torch.empty(T, d, dtype=torch.float32, device=y.device)
    s = torch.cuda.current_stream().cuda_stream
    check(lib().llapis_moe_combine(y.data_ptr(), weights.data_ptr(), T, K, d, out.data_ptr(), s), "llapis_moe_combine")
    return out


def residual_rmsnorm(h, add=None, x=None, eps=1e-6, stream=None):
    """h += add (in place, when add is given), then x = rms_norm(h) per row
    (no weight); returns x.  The glue between two layers of a residual
    stream, one kernel."""
    torch = _torch()
    T, d = h.shape
    if not h.is_contiguous() or (add is not None and (not add.is_contiguous() or add.shape != h.shape)):
        raise ValueError("residual_rmsnorm: h and add must be contiguous [T, d]")
    if x is None:
        x = torch.empty_like(h)
    s = stream if stream is not None else torch.cuda.current_stream().cuda_stream
    check(lib().llapis_residual_rmsnorm(h.data_ptr(), None if add is None else add.data_ptr(), T, d, eps,
                                        x.data_ptr(), s), "llapis_residual_rmsnorm")
    return x


def geglu(gate_up, n_ff, gelu_mode=L.GELU_TABLE):
    torch = _torch()
    n_cols = gate_up.numel() // (2 * n_ff)
    out = torch.empty(n_cols, n_ff, dtype=torch.float32, device=gate_up.device)
    s = torch.cuda.current_stream().cuda_stream
    check(lib().llapis_geglu(gate_up.data_ptr(), n_ff, n_cols, out.data_ptr(), gelu_mode, s), "llapis_geglu")
    return out
