# SPDX-License-Identifier: Apache-2.0
"""Closed forms and invariants that pin the oracle where fixtures leave room, chosen so that
a plausible mistake (a dropped term, a wrong sign, index or order) fails one of them."""
from __future__ import annotations

import numpy as np
import pytest

import k3_oracle as ko
from k3_oracle import f32, ptr

L = ko.orc()


def test_l2norm_is_sum_not_mean():
    """l2norm_ divides by sqrt(sum + eps), not sqrt(mean + eps) (src/core/k3_ops.c:845-851):
    the result has unit norm up to eps; the mean form would scale it by sqrt(n)."""
    rng = np.random.default_rng(1)
    for n in (16, 64, 128):
        v = f32(rng.standard_normal(n) * 3)
        w = v.copy()
        L.orc_l2norm(ptr(w), n, 1e-6)
        ss = float(np.sum(v.astype(np.float64) ** 2))
        np.testing.assert_allclose(w, v / np.sqrt(ss + 1e-6), rtol=2e-7)
        assert abs(np.linalg.norm(w.astype(np.float64)) - 1.0) < 1e-6


def test_rmsnorm_closed_form():
    rng = np.random.default_rng(2)
    x, wt = f32(rng.standard_normal(128)), f32(1 + rng.standard_normal(128) * 0.1)
    y = np.zeros(128, np.float32)
    L.orc_rmsnorm(ptr(y), ptr(x), ptr(wt), 128, 1e-5)
    ref = wt.astype(np.float64) * x / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-5)
    np.testing.assert_allclose(y, ref, rtol=3e-7, atol=1e-7)


def test_shortconv_is_left_padded_conv1d_plus_silu():
    """y_t = SiLU(sum_j w[j] x_{t-K+1+j}) with zero history (tools/k3_ref.py:201-209 form)."""
    rng = np.random.default_rng(3)
    C, K, T = 6, 4, 9
    w = f32(rng.standard_normal((C, K)))
    x = f32(rng.standard_normal((T, C)))
    y = np.zeros_like(x)
    L.orc_shortconv(ptr(y), ptr(x), ptr(w), None, C, K, T)
    xp = np.vstack([np.zeros((K - 1, C)), x.astype(np.float64)])
    acc = np.stack([sum(w[:, j] * xp[t + j] for j in range(K)) for t in range(T)])
    np.testing.assert_allclose(y, acc / (1 + np.exp(-acc)), rtol=1e-5, atol=1e-6)


def test_decay_per_head_and_range():
    """A_log indexed per head (a per-channel misindex changes every element), g in (lb, 0]."""
    rng = np.random.default_rng(4)
    H, D, lb = 3, 8, -5.0
    z, A, dt = f32(rng.standard_normal(H * D) * 3), f32(np.linspace(-0.4, 1.2, H)), f32(rng.standard_normal(H * D))
    g, al = np.zeros(H * D, np.float32), np.zeros(H * D, np.float32)
    L.orc_kda_decay(ptr(g), ptr(al), ptr(z), ptr(A), ptr(dt), H, D, lb)
    a = np.repeat(np.exp(A.astype(np.float64)), D)
    ref = lb / (1 + np.exp(-a * (z + dt)))
    np.testing.assert_allclose(g, ref, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(al, np.exp(ref), rtol=1e-6)
    assert np.all(g <= 0) and np.all(g > lb)


def test_softplus_gate_closed_form():
    """The unbounded gate g = -exp(A_log[h]) softplus(z + dt) (parity unpinned: this closed
    form is its only check)."""
    rng = np.random.default_rng(5)
    H, D = 2, 16
    z, A, dt = f32(rng.standard_normal(H * D) * 10), f32(rng.uniform(0, 1.5, H)), f32(rng.standard_normal(H * D))
    g, al = np.zeros(H * D, np.float32), np.zeros(H * D, np.float32)
    L.orc_kda_decay_softplus(ptr(g), ptr(al), ptr(z), ptr(A), ptr(dt), H, D)
    x = (z + dt).astype(np.float64)
    ref = -np.repeat(np.exp(A.astype(np.float64)), D) * np.logaddexp(0.0, x)
    np.testing.assert_allclose(g, ref, rtol=2e-6, atol=1e-6)
    np.testing.assert_allclose(al, np.exp(ref), rtol=2e-5, atol=1e-30)


def _step(S, q, k, v, al, beta):
    D = q.size
    o = np.zeros(D, np.float32)
    L.orc_kda_step(ptr(S), ptr(o), ptr(f32(q)), ptr(f32(k)), ptr(f32(v)), ptr(f32(al)), float(beta), D, D)
    return o


def test_step_frozen_state():
    """alpha = 1, beta = 0: the state is untouched and o = S^T q."""
    rng = np.random.default_rng(6)
    D = 32
    S = f32(rng.standard_normal((D, D)))
    S0 = S.copy()
    q, k, v = (rng.standard_normal(D) for _ in range(3))
    o = _step(S, q, k, v, np.ones(D), 0.0)
    assert np.array_equal(S, S0)
    np.testing.assert_allclose(o, S0.astype(np.float64).T @ f32(q), rtol=1e-5, atol=1e-5)


def test_step_exact_write_then_read():
    """beta = 1, alpha = 1, |k| = 1: after the delta write S^T k = v exactly (up to rounding),
    and reading with q = k returns v. Reading the state BEFORE the write (a wrong order)
    would return the old S^T k instead."""
    rng = np.random.default_rng(7)
    D = 64
    S = f32(rng.standard_normal((D, D)) * 0.3)
    k = rng.standard_normal(D)
    k /= np.linalg.norm(k)
    v = rng.standard_normal(D)
    o = _step(S, k, k, v, np.ones(D), 1.0)
    np.testing.assert_allclose(o, v, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(S.astype(np.float64).T @ f32(k), v, rtol=1e-4, atol=1e-4)


def test_step_matches_brute_force_float64():
    """The step against a float64 transcription of decay -> read -> delta write -> read."""
    rng = np.random.default_rng(8)
    D = 16
    S = f32(rng.standard_normal((D, D)))
    Sd = S.astype(np.float64)
    for _ in range(5):
        q, k, v = (f32(rng.standard_normal(D)) for _ in range(3))
        al = f32(rng.uniform(0.01, 1.0, D))
        b = float(rng.uniform())
        o = _step(S, q, k, v, al, b)
        Sd = Sd * al[:, None]
        u = Sd.T @ k
        Sd = Sd + np.outer(k, b * (v - u))
        np.testing.assert_allclose(o, Sd.T @ q, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(S, Sd, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("lb", [-5.0, 0.0])
def test_core_equals_layer_minus_projections(lb):
    """orc_kda_core on projected inputs reproduces orc_kda_layer before its o_proj."""
    from test_oracle_ref import rand_layer
    rng = np.random.default_rng(9)
    hidden, H, D, K, T = 64, 2, 16, 4, 7
    W = rand_layer(rng, hidden, H, D, K, 0)
    cfg = ko.make_cfg(hidden, H, D, K, lb, 1e-5)
    x = f32(rng.standard_normal((T, hidden)))
    a = W.arrays
    proj = lambda M: f32(x.astype(np.float64) @ M.T.astype(np.float64))
    fa = proj(a["f_a"])
    z = f32(fa.astype(np.float64) @ a["f_b"].T.astype(np.float64))
    y = ko.core(proj(a["q"]), proj(a["k"]), proj(a["v"]), z, proj(a["b"]), proj(a["g"]), W, cfg, T, None)
    out = ko.kda_layer(ko.orc(), x, W, cfg, T, None)
    np.testing.assert_allclose(f32(y.astype(np.float64) @ a["o"].T.astype(np.float64)), out, rtol=2e-4, atol=2e-5)
