# SPDX-License-Identifier: Apache-2.0
"""ctypes binding of ``libk3kda_hip.so``, the gfx950 Kimi Delta Attention path.

The product is the C-ABI library declared in ``include/k3kda.h``; this module only loads
it and forwards device pointers (torch tensors are used as device memory and streams).
Every call goes to the HIP library: there is no CPU fallback, and a missing library or a
missing GPU raises.

Reference interface mirrored: ``k3_kda_layer`` / ``k3_kda_scratch``
(kimi-k3-in-c include/k3/k3.h:464-469) with the ``K3Cfg`` / ``K3KdaW`` structs
(include/k3/k3.h:73-120, :448-462).
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libk3kda_hip.so"

K3_WF32, K3_WBF16, K3_WI8 = 0, 1, 2
F32, BF16, F16 = 0, 1, 3
UPLOAD_DEV, UPLOAD_PREFILL, UPLOAD_DECODE, UPLOAD_ALL = 1, 2, 4, 7
OK, EINVAL, EHIP, EUNSUPPORTED, ENOMEM = 0, 1, 2, 3, 4

EXPORTS = (
    "k3_kda_scratch", "k3_kda_layer", "k3hip_last_error", "k3hip_version",
    "k3hip_device_count", "k3hip_kda_decode", "k3hip_kda_prep", "k3hip_kda_chunk_workspace",
    "k3hip_kda_chunk", "k3hip_kda_prefill", "k3hip_kda_recurrent", "k3hip_kda_epilogue",
    "k3hip_kda_upload", "k3hip_kda_release", "k3hip_kda_layer_dev", "k3hip_kda_layer_prefill",
    "k3hip_kda_state_floats", "k3hip_kda_states_create", "k3hip_kda_states_release",
    "k3hip_kda_states_layer", "k3hip_kda_states_zero", "k3hip_kda_states_copy",
    "k3hip_kda_states_download", "k3hip_kda_states_upload",
    "k3hip_mla_upload", "k3hip_mla_release", "k3hip_mla_cache_floats", "k3hip_mla_decode",
    "k3hip_kda_layer_decode", "k3hip_kda_upload_ex", "k3hip_kda_weights_bytes",
    "k3hip_kda_dropin_bytes", "k3hip_proj_gemm", "k3hip_kda_layer_decode_noalloc",
    "k3hip_set_projection_gemm", "k3hip_kda_decode_step",
)


class K3Cfg(C.Structure):
    """Layout mirror of the reference K3Cfg (include/k3/k3.h:73-120)."""
    _fields_ = [
        ("hidden", C.c_int), ("n_layers", C.c_int), ("vocab", C.c_int), ("rms_eps", C.c_float),
        ("kda_heads", C.c_int), ("kda_head_dim", C.c_int), ("conv_k", C.c_int),
        ("gate_lb", C.c_float), ("n_heads", C.c_int), ("q_lora", C.c_int), ("kv_lora", C.c_int),
        ("qk_nope", C.c_int), ("qk_rope", C.c_int), ("v_head", C.c_int),
        ("mla_out_gate", C.c_int), ("n_experts", C.c_int), ("topk", C.c_int),
        ("n_shared", C.c_int), ("latent", C.c_int), ("moe_inter", C.c_int),
        ("routed_scale", C.c_float), ("moe_renorm", C.c_int), ("latent_norm", C.c_int),
        ("first_dense", C.c_int), ("dense_inter", C.c_int), ("attn_res_block", C.c_int),
        ("situ_b1", C.c_float), ("situ_b2", C.c_float), ("n_full_attn", C.c_int),
        ("full_attn", C.POINTER(C.c_int)),
    ]


class K3KdaW(C.Structure):
    """Layout mirror of the reference K3KdaW (include/k3/k3.h:448-462)."""
    _fields_ = [
        ("q", C.c_void_p), ("k", C.c_void_p), ("v", C.c_void_p),
        ("q_conv", C.c_void_p), ("k_conv", C.c_void_p), ("v_conv", C.c_void_p),
        ("f_a", C.c_void_p), ("f_b", C.c_void_p), ("A_log", C.c_void_p),
        ("dt_bias", C.c_void_p), ("b", C.c_void_p), ("g", C.c_void_p),
        ("o_norm", C.c_void_p), ("o", C.c_void_p), ("wdt", C.c_int),
    ]


class K3MlaW(C.Structure):
    """Mirror of the reference K3MlaW (include/k3/k3.h:203-210)."""
    _fields_ = [("q_a", C.c_void_p), ("q_b", C.c_void_p), ("kv_a", C.c_void_p),
                ("kv_b", C.c_void_p), ("o", C.c_void_p), ("g", C.c_void_p),
                ("q_a_norm", C.c_void_p), ("kv_a_norm", C.c_void_p), ("wdt", C.c_int)]


def make_cfg(hidden: int, heads: int, head_dim: int, conv_k: int = 4, gate_lb: float = -5.0,
             rms_eps: float = 1e-5) -> K3Cfg:
    c = K3Cfg()
    C.memset(C.byref(c), 0, C.sizeof(c))
    c.hidden, c.kda_heads, c.kda_head_dim, c.conv_k = hidden, heads, head_dim, conv_k
    c.gate_lb, c.rms_eps = gate_lb, rms_eps
    return c


class K3HipError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"k3kda error {code}: {msg}")
        self.code = code


_lib = None
_P = C.c_void_p


def lib() -> C.CDLL:
    """Load the HIP library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
    L = C.CDLL(str(LIB_PATH))
    i, f, sz = C.c_int, C.c_float, C.c_size_t
    sig = {
        "k3_kda_scratch": (sz, [C.POINTER(K3Cfg), i]),
        "k3_kda_layer": (None, [_P, _P, C.POINTER(K3KdaW), C.POINTER(K3Cfg), i, _P, _P]),
        "k3hip_last_error": (C.c_char_p, []),
        "k3hip_version": (C.c_char_p, []),
        "k3hip_device_count": (i, []),
        "k3hip_kda_decode": (i, [i, i, i, _P, _P, _P, _P, _P, _P, _P, f, _P]),
        "k3hip_kda_prep": (i, [i, i, i, i, f, i, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                               _P, _P, _P, _P, _P, _P, _P]),
        "k3hip_kda_chunk_workspace": (sz, [i, i, i, i]),
        "k3hip_kda_chunk": (i, [i, i, i, i, _P, _P, _P, _P, _P, f, _P, _P, _P, sz, _P]),
        "k3hip_kda_prefill": (i, [i, i, i, i, f, i, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                  f, _P, _P, _P, sz, _P]),
        "k3hip_kda_recurrent": (i, [i, i, i, _P, _P, _P, _P, _P, f, _P, _P, _P]),
        "k3hip_kda_epilogue": (i, [i, i, i, f, _P, _P, i, _P, _P, i, _P]),
        "k3hip_kda_upload": (i, [C.POINTER(K3KdaW), C.POINTER(K3Cfg), C.POINTER(_P)]),
        "k3hip_kda_release": (i, [_P]),
        "k3hip_kda_layer_dev": (i, [_P, i, _P, _P, _P, _P]),
        "k3hip_kda_layer_prefill": (i, [_P, i, _P, i, _P, i, _P, _P]),
        "k3hip_kda_state_floats": (sz, [C.POINTER(K3Cfg)]),
        "k3hip_kda_states_create": (i, [C.POINTER(K3Cfg), i, C.POINTER(_P)]),
        "k3hip_kda_states_release": (i, [_P]),
        "k3hip_kda_states_layer": (_P, [_P, i]),
        "k3hip_kda_states_zero": (i, [_P, _P]),
        "k3hip_kda_states_copy": (i, [_P, _P, _P]),
        "k3hip_kda_states_download": (i, [_P, _P, _P]),
        "k3hip_kda_states_upload": (i, [_P, _P, _P]),
        "k3hip_mla_upload": (i, [C.POINTER(K3MlaW), C.POINTER(K3Cfg), C.POINTER(_P)]),
        "k3hip_mla_release": (i, [_P]),
        "k3hip_mla_cache_floats": (sz, [C.POINTER(K3Cfg), i]),
        "k3hip_mla_decode": (i, [_P, i, i, i, _P, _P, _P, _P]),
        "k3hip_kda_layer_decode": (i, [_P, i, _P, _P, _P, C.c_long, _P]),
        "k3hip_kda_upload_ex": (i, [C.POINTER(K3KdaW), C.POINTER(K3Cfg), i, C.POINTER(_P)]),
        "k3hip_kda_weights_bytes": (sz, [_P]),
        "k3hip_kda_dropin_bytes": (sz, []),
        "k3hip_proj_gemm": (i, [i, i, i, i, _P, C.c_long, _P, C.c_long, _P, i, C.c_long, _P]),
        "k3hip_kda_layer_decode_noalloc": (i, [_P, i, _P, _P, _P, C.c_long, _P]),
        "k3hip_set_projection_gemm": (i, [i]),
        "k3hip_kda_decode_step": (i, [i, i, i, i, f, f, i, _P, _P, _P, _P, _P, _P, i, _P, _P, _P, _P, _P, _P,
                                      _P, f, _P, _P, i, _P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype, fn.argtypes = res, args
    _lib = L
    return L


def last_error() -> str:
    return lib().k3hip_last_error().decode()


def _check(rc: int) -> None:
    if rc != OK:
        raise K3HipError(rc, last_error())


# ------------------------------------------------------------- torch plumbing ----
def _ptr(t):
    """Device pointer of a torch tensor (None -> NULL). Refuses host tensors and
    non-contiguous views: the kernels index dense row-major memory."""
    if t is None:
        return None
    if isinstance(t, _DevPtr):
        return C.c_void_p(t.addr)
    if not t.is_cuda:
        raise ValueError("k3kda: device tensor required")
    if not t.is_contiguous():
        raise ValueError("k3kda: contiguous tensor required")
    return C.c_void_p(t.data_ptr())


def _stream(stream):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


def _dt(t) -> int:
    import torch
    if t.dtype == torch.float32:
        return F32
    if t.dtype == torch.bfloat16:
        return BF16
    if t.dtype == torch.float16:
        return F16
    raise ValueError(f"k3kda: dtype {t.dtype} not supported (float32, bfloat16 or float16)")


def proj_gemm(a, b, c, stream=None) -> None:
    """c[M,N] = a[M,K] . b[N,K]^T on the hand-written MFMA GEMM (a, b bf16 or fp16 alike;
    c float32, bfloat16 or float16). Row strides are taken from the tensors."""
    M, K = a.shape
    N = b.shape[0]
    for t in (a, b, c):
        if not t.is_cuda or t.stride(-1) != 1:
            raise ValueError("k3kda.proj_gemm: device tensors with unit column stride required")
    _check(lib().k3hip_proj_gemm(M, N, K, _dt(a), C.c_void_p(a.data_ptr()), a.stride(0),
                                 C.c_void_p(b.data_ptr()), b.stride(0), C.c_void_p(c.data_ptr()),
                                 _dt(c), c.stride(0), _stream(stream)))


GEMM_HIPBLASLT, GEMM_HANDWRITTEN = 0, 1


def set_projection_gemm(impl: int) -> None:
    """Select the projection GEMMs of layer_prefill (process-wide): GEMM_HIPBLASLT (default)
    or GEMM_HANDWRITTEN (the hand-written MFMA kernel of proj_gemm for every projection)."""
    _check(lib().k3hip_set_projection_gemm(impl))


def kda_decode(S, o, q, k, v, alpha, beta, q_scale: float, stream=None) -> None:
    """K3: S[B,H,D,D] in/out, o/q/k/v/alpha [B,H,D], beta [B,H] (fp32, device)."""
    B, H, D = q.shape
    _check(lib().k3hip_kda_decode(B, H, D, _ptr(S), _ptr(o), _ptr(q), _ptr(k), _ptr(v),
                                  _ptr(alpha), _ptr(beta), q_scale, _stream(stream)))


def kda_prep(q_in, k_in, v_in, z, b_logit, q_conv, k_conv, v_conv, A_log, dt_bias, conv_state,
             q_out, k_out, v_out, g_out, alpha_out, beta_out, H: int, D: int, K: int,
             gate_lb: float, stream=None) -> None:
    """K1 over one sequence: inputs [T,P] (fp32 or bf16), outputs [T,P] fp32, beta [T,H]."""
    T = q_in.shape[0]
    _check(lib().k3hip_kda_prep(T, H, D, K, gate_lb, _dt(q_in), _ptr(q_in), _ptr(k_in),
                                _ptr(v_in), _ptr(z), _ptr(b_logit), _ptr(q_conv), _ptr(k_conv),
                                _ptr(v_conv), _ptr(A_log), _ptr(dt_bias), _ptr(conv_state),
                                _ptr(q_out), _ptr(k_out), _ptr(v_out), _ptr(g_out),
                                _ptr(alpha_out), _ptr(beta_out), _stream(stream)))


def kda_chunk(q, k, v, g, beta, S, o, H: int, D: int, q_scale: float, chunk: int = 64,
              workspace=None, stream=None) -> None:
    """K2 chunked prefill: q,k,v,g,o [T,P] fp32; beta [T,H]; S [H,D,D] in/out."""
    T = q.shape[0]
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    _check(lib().k3hip_kda_chunk(T, H, D, chunk, _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta),
                                 q_scale, _ptr(S), _ptr(o), _ptr(workspace), ws_bytes,
                                 _stream(stream)))


def kda_prefill(q_in, k_in, v_in, z, b_logit, q_conv, k_conv, v_conv, A_log, dt_bias,
                conv_state, S, o, H: int, D: int, K: int, gate_lb: float, q_scale: float,
                workspace=None, stream=None) -> None:
    """K1 + K2 fused: bf16 or fp32 inputs [T,P], z [T,P] fp32, b_logit [T,H]; S [H,D,D] in/out."""
    T = q_in.shape[0]
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    _check(lib().k3hip_kda_prefill(T, H, D, K, gate_lb, _dt(q_in), _ptr(q_in), _ptr(k_in),
                                   _ptr(v_in), _ptr(z), _ptr(b_logit), _ptr(q_conv),
                                   _ptr(k_conv), _ptr(v_conv), _ptr(A_log), _ptr(dt_bias),
                                   _ptr(conv_state), q_scale, _ptr(S), _ptr(o), _ptr(workspace),
                                   ws_bytes, _stream(stream)))


def kda_chunk_workspace(T: int, H: int, D: int, chunk: int = 64) -> int:
    return int(lib().k3hip_kda_chunk_workspace(T, H, D, chunk))


def kda_recurrent(q, k, v, alpha, beta, S, o, H: int, D: int, q_scale: float,
                  stream=None) -> None:
    """Sequential GPU recurrence: same layouts as kda_chunk, with alpha instead of g."""
    T = q.shape[0]
    _check(lib().k3hip_kda_recurrent(T, H, D, _ptr(q), _ptr(k), _ptr(v), _ptr(alpha),
                                     _ptr(beta), q_scale, _ptr(S), _ptr(o), _stream(stream)))


def kda_decode_step(q_in, k_in, v_in, z, b_logit, gate, q_conv, k_conv, v_conv, A_log, dt_bias, o_norm,
                    conv_state, S, y, H: int, D: int, K: int, gate_lb: float, rms_eps: float,
                    q_scale: float, stream=None) -> None:
    """K1 (T=1) + K3 + K4 in one launch for B = q_in.shape[0] sequences: q_in/k_in/v_in [B,P]
    (fp32 or bf16), z [B,P], b_logit [B,H], gate [B,P] (fp32 or bf16), conv_state
    [B,3,P,K-1] and S [B,H,D,D] in/out, y [B,P] (fp32 or bf16)."""
    B = q_in.shape[0]
    _check(lib().k3hip_kda_decode_step(B, H, D, K, gate_lb, rms_eps, _dt(q_in), _ptr(q_in), _ptr(k_in),
                                       _ptr(v_in), _ptr(z), _ptr(b_logit), _ptr(gate), _dt(gate), _ptr(q_conv),
                                       _ptr(k_conv), _ptr(v_conv), _ptr(A_log), _ptr(dt_bias), _ptr(o_norm),
                                       _ptr(conv_state), q_scale, _ptr(S), _ptr(y), _dt(y), _stream(stream)))


def kda_epilogue(o, gate, o_norm, y, H: int, D: int, rms_eps: float, stream=None) -> None:
    """K4: o [T,P] fp32, gate [T,P] fp32|bf16, o_norm [D], y [T,P] fp32|bf16."""
    T = o.shape[0]
    _check(lib().k3hip_kda_epilogue(T, H, D, rms_eps, _ptr(o), _ptr(gate), _dt(gate),
                                    _ptr(o_norm), _ptr(y), _dt(y), _stream(stream)))


class DeviceWeights:
    """k3hip_kda_upload / k3hip_kda_release around a K3KdaW of host pointers."""

    def __init__(self, w: K3KdaW, cfg: K3Cfg, parts: int = UPLOAD_ALL):
        self.handle = C.c_void_p()
        _check(lib().k3hip_kda_upload_ex(C.byref(w), C.byref(cfg), parts, C.byref(self.handle)))

    def nbytes(self) -> int:
        """Device bytes the uploaded weight set holds."""
        return int(lib().k3hip_kda_weights_bytes(self.handle))

    def layer(self, out, x, state, T: int, stream=None) -> None:
        _check(lib().k3hip_kda_layer_dev(self.handle, T, _ptr(out), _ptr(x), _ptr(state),
                                         _stream(stream)))

    def layer_decode(self, out, x, states, stride: int, stream=None) -> None:
        """One token for each of B = x.shape[0] sequences; states: B slots `stride` floats apart."""
        _check(lib().k3hip_kda_layer_decode(self.handle, x.shape[0], _ptr(out), _ptr(x),
                                            _ptr(states), stride, _stream(stream)))

    def layer_decode_noalloc(self, out, x, states, stride: int, stream=None) -> None:
        """k3hip_kda_layer_decode_noalloc: the same step on the library's fixed scratch."""
        _check(lib().k3hip_kda_layer_decode_noalloc(self.handle, x.shape[0], _ptr(out), _ptr(x),
                                                    _ptr(states), stride, _stream(stream)))

    def layer_prefill(self, out, x, state, T: int, stream=None) -> None:
        """bf16 full-layer prefill: x, out [T, hidden] float32 or bfloat16 tensors."""
        _check(lib().k3hip_kda_layer_prefill(self.handle, T, _ptr(out), _dt(out), _ptr(x), _dt(x),
                                             _ptr(state), _stream(stream)))

    def close(self) -> None:
        if self.handle:
            lib().k3hip_kda_release(self.handle)
            self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class _DevPtr:
    """A raw device address usable wherever a tensor pointer is expected."""

    def __init__(self, addr: int):
        self.addr = addr


class States:
    """k3hip_kda_states: per-layer device state slots in the reference kstate layout."""

    def __init__(self, cfg: K3Cfg, n_layers: int):
        self.handle = C.c_void_p()
        self.n_layers = n_layers
        self.kper = int(lib().k3hip_kda_state_floats(C.byref(cfg)))
        _check(lib().k3hip_kda_states_create(C.byref(cfg), n_layers, C.byref(self.handle)))

    def layer(self, L: int) -> "_DevPtr":
        p = lib().k3hip_kda_states_layer(self.handle, L)
        if not p:
            raise K3HipError(EINVAL, f"layer {L} out of range")
        return _DevPtr(p)

    def zero(self, stream=None) -> None:
        _check(lib().k3hip_kda_states_zero(self.handle, _stream(stream)))

    def copy_from(self, other: "States", stream=None) -> None:
        _check(lib().k3hip_kda_states_copy(self.handle, other.handle, _stream(stream)))

    def download(self):
        import numpy as np
        out = np.empty(self.n_layers * self.kper, np.float32)
        _check(lib().k3hip_kda_states_download(self.handle, out.ctypes.data_as(C.c_void_p), None))
        return out

    def upload(self, host) -> None:
        import numpy as np
        a = np.ascontiguousarray(host, np.float32)
        assert a.size == self.n_layers * self.kper
        _check(lib().k3hip_kda_states_upload(self.handle, a.ctypes.data_as(C.c_void_p), None))

    def close(self) -> None:
        if self.handle:
            lib().k3hip_kda_states_release(self.handle)
            self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class MlaWeights:
    """k3hip_mla_upload / k3hip_mla_release around a K3MlaW of host pointers."""

    def __init__(self, w: "K3MlaW", cfg: K3Cfg):
        self.handle = C.c_void_p()
        _check(lib().k3hip_mla_upload(C.byref(w), C.byref(cfg), C.byref(self.handle)))

    def decode(self, out, x, cache, pos: int, cap: int, stream=None) -> None:
        """One step for B = x.shape[0] sequences: x, out [B, hidden] fp32, cache
        [B, cap, kv_lora + rope] fp32 holding `pos` positions per sequence."""
        _check(lib().k3hip_mla_decode(self.handle, x.shape[0], pos, cap, _ptr(cache), _ptr(x),
                                      _ptr(out), _stream(stream)))

    def close(self) -> None:
        if self.handle:
            lib().k3hip_mla_release(self.handle)
            self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def dropin_bytes() -> int:
    """Host<->device bytes of the calling thread's last k3_kda_layer call."""
    return int(lib().k3hip_kda_dropin_bytes())


def kda_layer_host(out, x, w: K3KdaW, cfg: K3Cfg, T: int, state=None) -> None:
    """The drop-in k3_kda_layer on host (numpy float32) buffers."""
    def hp(a):
        return None if a is None else C.c_void_p(a.ctypes.data)
    lib().k3_kda_layer(hp(out), hp(x), C.byref(w), C.byref(cfg), T, hp(state), None)
