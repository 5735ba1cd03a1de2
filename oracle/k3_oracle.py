# SPDX-License-Identifier: Apache-2.0
"""ctypes binding of the CPU oracle. TEST INFRASTRUCTURE ONLY.

Loads ``oracle/libk3oracle.so`` (the C restatement of the reference KDA path) and, when it
has been built, ``oracle/_ref/libk3ref.so`` (the reference's own src/core/k3_ops.c
compiled from source by oracle/Makefile). Imported by tests/, __graft_entry__.smoke() and
bench.py's CPU baseline only; the shipped library never uses it.
"""
from __future__ import annotations

import ctypes as C
import subprocess
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
ORACLE_SO = HERE / "libk3oracle.so"
REF_SO = HERE / "_ref" / "libk3ref.so"
REF_SRC = Path("/root/reference/src/core/k3_ops.c")

sys.path.insert(0, str(REPO / "kimi-k3-in-c_amd"))
from k3kda import K3Cfg, K3KdaW, K3MlaW, make_cfg  # noqa: E402  (ABI struct mirrors)

_P = C.c_void_p


def build(ref: bool = True) -> None:
    """make -C oracle (and the reference build when its sources are present)."""
    subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)
    if ref and REF_SRC.exists():
        subprocess.run(["make", "-s", "-C", str(HERE), "ref"], check=True)


def _bind(L: C.CDLL, prefix: str) -> C.CDLL:
    i, f = C.c_int, C.c_float
    sig = {
        "rmsnorm": (None, [_P, _P, _P, i, f]),
        "shortconv": (None, [_P, _P, _P, _P, i, i, i]),
        "kda_decay": (None, [_P, _P, _P, _P, _P, i, i, f]),
        "kda_step": (None, [_P, _P, _P, _P, _P, _P, f, i, i]),
        "matmul": (None, [_P, _P, _P, i, i]),
        "matmul_bf16": (None, [_P, _P, _P, i, i]),
        "matmul_q8": (None, [_P, _P, _P, i, i]),
        "kda_scratch": (C.c_size_t, [C.POINTER(K3Cfg), i]),
        "kda_layer": (None, [_P, _P, C.POINTER(K3KdaW), C.POINTER(K3Cfg), i, _P, _P]),
    }
    if prefix == "orc_":
        sig.update({
            "kda_decay_softplus": (None, [_P, _P, _P, _P, _P, i, i]),
            "kda_decode_batch": (None, [i, i, i, _P, _P, _P, _P, _P, _P, _P, f, i]),
            "kda_core": (None, [_P, _P, _P, _P, _P, _P, _P, _P, C.POINTER(K3KdaW),
                                C.POINTER(K3Cfg), i, _P, i]),
            "kda_recurrence": (None, [i, i, i, _P, _P, _P, _P, _P, _P, _P, f, i]),
            "l2norm": (None, [_P, i, f]),
            "sigmoid": (f, [f]),
            "mla_cached": (None, [_P, _P, C.POINTER(K3MlaW), C.POINTER(K3Cfg), i, _P, _P, i, i]),
        })
    else:   # the reference's own MLA (src/core/k3_ops.c:321-424) takes a scratch buffer
        sig.update({
            "mla_cached": (None, [_P, _P, C.POINTER(K3MlaW), C.POINTER(K3Cfg), i, _P, _P, _P, i, i]),
            "mla_scratch_cached": (C.c_size_t, [C.POINTER(K3Cfg), i, i, i]),
        })
    for name, (res, args) in sig.items():
        fn = getattr(L, prefix + name)
        fn.restype, fn.argtypes = res, args
    return L


_orc = None
_ref = None


def orc() -> C.CDLL:
    global _orc
    if _orc is None:
        if not ORACLE_SO.exists():
            build(ref=False)
        _orc = _bind(C.CDLL(str(ORACLE_SO)), "orc_")
    return _orc


def ref():
    """The reference C compiled from source, or None when it has not been built here."""
    global _ref
    if _ref is None:
        if not REF_SO.exists() and REF_SRC.exists():
            build(ref=True)
        if not REF_SO.exists():
            return None
        _ref = _bind(C.CDLL(str(REF_SO)), "k3_")
    return _ref


def ptr(a: np.ndarray | None):
    """Pointer to a C-contiguous array. data_as keeps a reference to the array, so a
    temporary passed as ptr(f32(x)) stays alive for the duration of the call."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle buffers must be C-contiguous"
    return a.ctypes.data_as(C.c_void_p)


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


# ------------------------------------------------------------ typed helpers ----
def call(L, name: str, *args):
    prefix = "orc_" if L is orc() else "k3_"
    return getattr(L, prefix + name)(*args)


class Weights:
    """Holds numpy weight arrays and the K3KdaW of pointers into them."""

    NAMES = ("q", "k", "v", "q_conv", "k_conv", "v_conv", "f_a", "f_b", "A_log", "dt_bias",
             "b", "g", "o_norm", "o")

    def __init__(self, arrays: dict, wdt: int = 0):
        self.arrays = {}
        for n in self.NAMES:
            a = arrays[n]
            if a.dtype in (np.uint16, np.uint8):   # bf16 bit patterns / int8 rows (q8_rows)
                self.arrays[n] = np.ascontiguousarray(a)
            else:
                self.arrays[n] = f32(a)
        self.w = K3KdaW()
        C.memset(C.byref(self.w), 0, C.sizeof(self.w))
        for n in self.NAMES:
            setattr(self.w, n, self.arrays[n].ctypes.data)
        self.w.wdt = wdt
        self.w._arrays = self.arrays   # the struct holds raw addresses: keep their owners alive


def q8_rows(W) -> np.ndarray:
    """A float matrix [out][in] in the reference's per-row int8 draft format (K3_WI8,
    include/k3/k3.h:266-283): each row [f32 scale][int8 * in] with scale = max|row| / 127 and
    the weights rounded to nearest; returned as raw bytes [out][4 + in]."""
    W = np.asarray(W, np.float32)
    out, n = W.shape
    amax = np.abs(W).max(axis=1)
    scale = np.where(amax > 0, amax / np.float32(127), np.float32(1)).astype(np.float32)
    q = np.clip(np.rint(W / scale[:, None]), -127, 127).astype(np.int8)
    rows = np.empty((out, 4 + n), np.uint8)
    rows[:, :4] = scale.view(np.uint8).reshape(out, 4)
    rows[:, 4:] = q.view(np.uint8)
    return rows


def q8_dequant(rows: np.ndarray, n: int) -> np.ndarray:
    """The float matrix a K3_WI8 row block stands for: scale * int8, exact in fp32."""
    scale = np.ascontiguousarray(rows[:, :4]).view(np.float32)[:, 0]
    return rows[:, 4:4 + n].view(np.int8).astype(np.float32) * scale[:, None]


def kda_layer(L, x: np.ndarray, W: Weights, cfg: K3Cfg, T: int, state: np.ndarray | None):
    """Run <prefix>kda_layer; returns out [T][hidden] (state updated in place)."""
    out = np.zeros((T, cfg.hidden), np.float32)
    scratch = np.zeros(max(1, call(L, "kda_scratch", C.byref(cfg), T)), np.float32)
    call(L, "kda_layer", ptr(out), ptr(f32(x)), C.byref(W.w), C.byref(cfg), T, ptr(state),
         ptr(scratch))
    return out


def decode_batch(S, q, k, v, alpha, beta, q_scale: float, nthreads: int = 1):
    """orc_kda_decode_batch: S [B,H,D,D] updated in place; returns o [B,H,D]."""
    B, H, D = q.shape
    o = np.zeros((B, H, D), np.float32)
    orc().orc_kda_decode_batch(B, H, D, ptr(S), ptr(o), ptr(q), ptr(k), ptr(v), ptr(alpha),
                               ptr(beta), q_scale, nthreads)
    return o


def recurrence(S, q, k, v, alpha, beta, H: int, D: int, q_scale: float, nthreads: int = 1):
    """orc_kda_recurrence over [T][P] inputs; S [H,D,D] in place; returns o [T][P]."""
    T = q.shape[0]
    o = np.zeros((T, H * D), np.float32)
    orc().orc_kda_recurrence(T, H, D, ptr(S), ptr(o), ptr(q), ptr(k), ptr(v), ptr(alpha),
                             ptr(beta), q_scale, nthreads)
    return o


def core(q_in, k_in, v_in, z, b_logit, gate_logit, W: Weights, cfg: K3Cfg, T: int,
         state: np.ndarray | None, nthreads: int = 1, want_rec: bool = False):
    """orc_kda_core: conv..gate on projected inputs; returns y [T][P] (and o_rec)."""
    P = cfg.kda_heads * cfg.kda_head_dim
    y = np.zeros((T, P), np.float32)
    rec = np.zeros((T, P), np.float32) if want_rec else None
    orc().orc_kda_core(ptr(y), ptr(rec), ptr(f32(q_in)), ptr(f32(k_in)), ptr(f32(v_in)),
                       ptr(f32(z)), ptr(f32(b_logit)), ptr(f32(gate_logit)), C.byref(W.w),
                       C.byref(cfg), T, ptr(state), nthreads)
    return (y, rec) if want_rec else y


def prep(q_in, k_in, v_in, z, b_logit, W: Weights, cfg: K3Cfg, T: int, conv_state=None):
    """K1 on the CPU: conv+SiLU (carried state), L2 on q,k, beta, decay.
    Returns q, k, v, g, alpha [T][P] and beta [T][H]."""
    L = orc()
    H, D, K = cfg.kda_heads, cfg.kda_head_dim, cfg.conv_k
    P = H * D
    nh = K - 1
    outs = [np.zeros((T, P), np.float32) for _ in range(3)]
    ins = [f32(q_in), f32(k_in), f32(v_in)]
    convs = [W.arrays["q_conv"], W.arrays["k_conv"], W.arrays["v_conv"]]
    for b in range(3):
        st = None if conv_state is None else conv_state[b * P * nh:(b + 1) * P * nh]
        L.orc_shortconv(ptr(outs[b]), ptr(ins[b]), ptr(convs[b]), ptr(st), P, K, T)
    q, k, v = outs
    for t in range(T):
        for h in range(H):
            L.orc_l2norm(C.c_void_p(q.ctypes.data + 4 * (t * P + h * D)), D, 1e-6)
            L.orc_l2norm(C.c_void_p(k.ctypes.data + 4 * (t * P + h * D)), D, 1e-6)
    bl = f32(b_logit)
    beta = np.array([[L.orc_sigmoid(float(x)) for x in row] for row in bl], np.float32)
    zz = f32(z)
    g = np.zeros((T, P), np.float32)
    al = np.zeros((T, P), np.float32)
    for t in range(T):
        gp, ap, zp = (C.c_void_p(a.ctypes.data + 4 * t * P) for a in (g, al, zz))
        if cfg.gate_lb != 0.0:
            L.orc_kda_decay(gp, ap, zp, ptr(W.arrays["A_log"]), ptr(W.arrays["dt_bias"]), H, D,
                            cfg.gate_lb)
        else:   # no lower bound: the softplus gate
            L.orc_kda_decay_softplus(gp, ap, zp, ptr(W.arrays["A_log"]), ptr(W.arrays["dt_bias"]), H, D)
    return q, k, v, g, al, beta.reshape(T, H)


class MlaWeights:
    """Numpy arrays for a gated MLA layer and the K3MlaW of pointers into them. Matrices are
    float32 (wdt 0) or uint16 bf16 bit patterns (wdt 1); the layernorm weights are fp32."""

    MATS = ("q_a", "q_b", "kv_a", "kv_b", "o", "g")

    def __init__(self, arrays: dict, wdt: int = 0):
        self.arrays = {}
        for n in self.MATS + ("q_a_norm", "kv_a_norm"):
            a = arrays.get(n)
            if a is None:
                continue
            self.arrays[n] = np.ascontiguousarray(a) if a.dtype == np.uint16 else f32(a)
        self.w = K3MlaW()
        C.memset(C.byref(self.w), 0, C.sizeof(self.w))
        for n, a in self.arrays.items():
            setattr(self.w, n, a.ctypes.data)
        self.w.wdt = wdt
        self.w._arrays = self.arrays   # the struct holds raw addresses: keep their owners alive


def mla_cfg(hidden: int, n_heads: int, q_lora: int, kv_lora: int, qk_nope: int, qk_rope: int,
            v_head: int, rms_eps: float = 1e-5, gate: int = 1) -> K3Cfg:
    c = make_cfg(hidden, 1, 16, 1, -5.0, rms_eps)
    c.n_heads, c.q_lora, c.kv_lora = n_heads, q_lora, kv_lora
    c.qk_nope, c.qk_rope, c.v_head, c.mla_out_gate = qk_nope, qk_rope, v_head, gate
    return c


def mla(x: np.ndarray, W: MlaWeights, cfg: K3Cfg, T: int, kvc=None, ropec=None, cached: int = 0,
        cap: int = 0, lib: str = "orc"):
    """Gated MLA over T tokens (k3_mla_cached); kvc [cap][H*(nope+v)] and ropec [cap][rope]
    are updated in place when given. lib = "orc" (this restatement) or "ref" (the
    reference compiled from its own sources)."""
    out = np.zeros((T, cfg.hidden), np.float32)
    if lib == "orc":
        orc().orc_mla_cached(ptr(out), ptr(f32(x)), C.byref(W.w), C.byref(cfg), T, ptr(kvc),
                             ptr(ropec), cached, cap)
    else:
        L = ref()
        n = L.k3_mla_scratch_cached(C.byref(cfg), T, cap, 1 if kvc is not None else 0)
        scratch = np.zeros(max(1, n), np.float32)
        L.k3_mla_cached(ptr(out), ptr(f32(x)), C.byref(W.w), C.byref(cfg), T, ptr(scratch),
                        ptr(kvc), ptr(ropec), cached, cap)
    return out
