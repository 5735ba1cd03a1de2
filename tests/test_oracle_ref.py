# SPDX-License-Identifier: Apache-2.0
"""The oracle against the reference C (kimi-k3-in-c src/core/k3_ops.c compiled from source
by oracle/Makefile) on seeded random inputs beyond the fixtures' shapes: wider heads,
bf16 weights, odd lengths, carried state, conv_k edge cases. Bit-for-bit equality is
required: the restatement keeps the reference's accumulation widths and orders."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import k3_oracle as ko
from k3_oracle import ptr, f32

R = ko.ref()
pytestmark = pytest.mark.skipif(R is None, reason="reference C not built (sources absent)")


def bits_equal(a, b) -> bool:
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


def rand_layer(rng, hidden, H, D, K, wdt):
    P = H * D

    def mat(o, i, s=0.02):
        m = (rng.standard_normal((o, i)) * s).astype(np.float32)
        return bf16(m) if wdt == 1 else (ko.q8_rows(m) if wdt == 2 else m)

    arrays = {
        "q": mat(P, hidden), "k": mat(P, hidden), "v": mat(P, hidden), "g": mat(P, hidden),
        "o": mat(hidden, P), "f_a": mat(D, hidden), "f_b": mat(P, D, 0.1), "b": mat(H, hidden),
        "q_conv": f32(rng.standard_normal((P, K)) * 0.5),
        "k_conv": f32(rng.standard_normal((P, K)) * 0.5),
        "v_conv": f32(rng.standard_normal((P, K)) * 0.5),
        "A_log": f32(rng.uniform(0, 1.5, H)), "dt_bias": f32(rng.standard_normal(P)),
        "o_norm": f32(1 + 0.1 * rng.standard_normal(D)),
    }
    return ko.Weights(arrays, wdt)


def bf16(m: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (finite inputs)."""
    u = np.ascontiguousarray(m, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


@pytest.mark.parametrize("hidden,H,D,K,T,wdt", [
    (256, 4, 64, 4, 33, 0),
    (256, 2, 128, 4, 17, 1),
    (96, 3, 32, 1, 5, 0),      # conv_k = 1: no history at all
    (64, 2, 16, 2, 3, 1),
    (256, 4, 64, 4, 9, 2),     # the int8 draft format (K3_WI8), hidden a multiple of 16
    (200, 3, 32, 3, 5, 2),     # and with ragged int8 row tails
])
def test_layer_bitwise_vs_reference(hidden, H, D, K, T, wdt):
    rng = np.random.default_rng(1000 + hidden + D + T)
    W = rand_layer(rng, hidden, H, D, K, wdt)
    cfg = ko.make_cfg(hidden, H, D, K, -5.0, 1e-5)
    P = H * D
    n = P * D + 3 * P * (K - 1)
    s0 = f32(rng.standard_normal(n) * 0.1)
    s1, s2 = s0.copy(), s0.copy()
    x = f32(rng.standard_normal((T, hidden)))
    o1 = ko.kda_layer(ko.orc(), x, W, cfg, T, s1)
    o2 = ko.kda_layer(R, x, W, cfg, T, s2)
    assert bits_equal(o1, o2)
    assert bits_equal(s1, s2)
    # and once more from the carried state (decode step, T = 1)
    x1 = f32(rng.standard_normal((1, hidden)))
    assert bits_equal(ko.kda_layer(ko.orc(), x1, W, cfg, 1, s1), ko.kda_layer(R, x1, W, cfg, 1, s2))
    assert bits_equal(s1, s2)


def test_layer_null_state_bitwise():
    rng = np.random.default_rng(7)
    W = rand_layer(rng, 128, 2, 32, 4, 0)
    cfg = ko.make_cfg(128, 2, 32, 4, -5.0, 1e-5)
    x = f32(rng.standard_normal((6, 128)))
    assert bits_equal(ko.kda_layer(ko.orc(), x, W, cfg, 6, None), ko.kda_layer(R, x, W, cfg, 6, None))


@pytest.mark.parametrize("D", [16, 64, 128])
def test_step_bitwise_with_zero_rows(D):
    """k3_kda_step, including rows where k[i] == 0 or q[i] == 0 (skipped rows)."""
    rng = np.random.default_rng(D)
    S1 = f32(rng.standard_normal((D, D)))
    S2 = S1.copy()
    q, k, v = (f32(rng.standard_normal(D)) for _ in range(3))
    k[::5] = 0.0
    q[::7] = 0.0
    al = f32(rng.uniform(0.005, 1.0, D))
    al[3] = 1.0
    o1, o2 = np.zeros(D, np.float32), np.zeros(D, np.float32)
    ko.orc().orc_kda_step(ptr(S1), ptr(o1), ptr(q), ptr(k), ptr(v), ptr(al), 0.37, D, D)
    R.k3_kda_step(ptr(S2), ptr(o2), ptr(q), ptr(k), ptr(v), ptr(al), 0.37, D, D)
    assert bits_equal(S1, S2) and bits_equal(o1, o2)


@pytest.mark.parametrize("i_n,o_n", [(257, 129), (16, 3), (7168 // 8, 40)])
def test_matmul_bitwise(i_n, o_n):
    rng = np.random.default_rng(i_n)
    W = f32(rng.standard_normal((o_n, i_n)))
    x = f32(rng.standard_normal(i_n))
    y1, y2 = np.zeros(o_n, np.float32), np.zeros(o_n, np.float32)
    ko.orc().orc_matmul(ptr(y1), ptr(x), ptr(W), i_n, o_n)
    R.k3_matmul(ptr(y2), ptr(x), ptr(W), i_n, o_n)
    assert bits_equal(y1, y2)
    Wb = bf16(W)
    ko.orc().orc_matmul_bf16(ptr(y1), ptr(x), ptr(Wb), i_n, o_n)
    R.k3_matmul_bf16(ptr(y2), ptr(x), ptr(Wb), i_n, o_n)
    assert bits_equal(y1, y2)


@pytest.mark.parametrize("i_n,o_n", [(257, 129), (16, 3), (15, 5), (7168 // 8, 40)])
def test_matmul_q8_bitwise(i_n, o_n):
    """The per-row int8 draft matmul (K3_WI8, src/core/k3_ops.c:1228-1301): the oracle's
    restatement of the reference's AVX2 summation order equals the reference bit for bit,
    and both lie within float rounding of the double-precision dot of the dequantised row."""
    rng = np.random.default_rng(5000 + i_n)
    Wf = f32(rng.standard_normal((o_n, i_n)))
    Wq = ko.q8_rows(Wf)
    x = f32(rng.standard_normal(i_n))
    y1, y2 = np.zeros(o_n, np.float32), np.zeros(o_n, np.float32)
    ko.orc().orc_matmul_q8(ptr(y1), ptr(x), ptr(Wq), i_n, o_n)
    R.k3_matmul_q8(ptr(y2), ptr(x), ptr(Wq), i_n, o_n)
    assert bits_equal(y1, y2)
    deq = ko.q8_dequant(Wq, i_n).astype(np.float64)
    exact = deq @ x.astype(np.float64)
    mag = np.abs(deq) @ np.abs(x.astype(np.float64))
    assert np.all(np.abs(y1 - exact) <= 2.0 ** -20 * mag + 1e-30)


def test_shortconv_short_sequence_carries_history():
    """T < conv_k - 1: the carried history shifts inside itself."""
    rng = np.random.default_rng(3)
    Cn, K = 40, 4
    w = f32(rng.standard_normal((Cn, K)))
    st1 = f32(rng.standard_normal(Cn * (K - 1)))
    st2 = st1.copy()
    for T in (1, 2, 5):
        x = f32(rng.standard_normal((T, Cn)))
        y1, y2 = np.zeros_like(x), np.zeros_like(x)
        ko.orc().orc_shortconv(ptr(y1), ptr(x), ptr(w), ptr(st1), Cn, K, T)
        R.k3_shortconv(ptr(y2), ptr(x), ptr(w), ptr(st2), Cn, K, T)
        assert bits_equal(y1, y2) and bits_equal(st1, st2)


@pytest.mark.parametrize("wdt", [0, 1])
def test_mla_bitwise_vs_reference(wdt):
    """orc_mla_cached against the reference's k3_mla_cached, built from its own sources:
    uncached over T tokens, then cached decode steps, fp32 and bf16 weights."""
    L = ko.ref()
    if L is None:
        pytest.skip("reference C not built in this container (no /root/reference)")
    rng = np.random.default_rng(77 + wdt)
    hidden, H, ql, kvl, qn, qr, vh = 96, 3, 48, 40, 24, 8, 16
    cfg = ko.mla_cfg(hidden, H, ql, kvl, qn, qr, vh)
    mats = {"q_a": (ql, hidden), "q_b": (H * (qn + qr), ql), "kv_a": (kvl + qr, hidden),
            "kv_b": (H * (qn + vh), kvl), "o": (hidden, H * vh), "g": (H * vh, hidden)}
    arrays = {n: rng.standard_normal(s).astype(np.float32) * 0.1 for n, s in mats.items()}
    if wdt:
        arrays = {n: bf16(a) for n, a in arrays.items()}
    arrays["q_a_norm"] = (1 + 0.1 * rng.standard_normal(ql)).astype(np.float32)
    arrays["kv_a_norm"] = (1 + 0.1 * rng.standard_normal(kvl)).astype(np.float32)
    W = ko.MlaWeights(arrays, wdt)
    T = 7
    x = rng.standard_normal((T, hidden)).astype(np.float32)
    assert np.array_equal(ko.mla(x, W, cfg, T, lib="orc"), ko.mla(x, W, cfg, T, lib="ref"))
    cap = 12
    caches = {lib: (np.zeros((cap, H * (qn + vh)), np.float32), np.zeros((cap, qr), np.float32))
              for lib in ("orc", "ref")}
    for t in range(5):
        xt = rng.standard_normal((1, hidden)).astype(np.float32)
        a = ko.mla(xt, W, cfg, 1, *caches["orc"], t, cap, lib="orc")
        b = ko.mla(xt, W, cfg, 1, *caches["ref"], t, cap, lib="ref")
        assert np.array_equal(a, b), t
    assert np.array_equal(caches["orc"][0], caches["ref"][0])
