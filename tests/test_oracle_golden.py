# SPDX-License-Identifier: Apache-2.0
"""The CPU oracle against the reference's own golden fixtures (tests/golden/ref_ops, copied
from kimi-k3-in-c tests/fixtures/ops). Mirrors the KDA checks of the reference's
tests/unit/test_ops.c (t_rmsnorm :133-147, t_shortconv :193-232, t_decay :234-278,
t_recur :310-351, t_kda_layer :576-634) at the manifest tolerance, and runs the same
checks on the reference C compiled from source when it is present, so a fixture-loading
mistake here cannot pass silently."""
from __future__ import annotations

import ctypes as C
import hashlib

import numpy as np
import pytest

from conftest import REF_OPS, load_fixture, manifest_tol, worst_ratio
import k3_oracle as ko

ATOL, RTOL = manifest_tol()


def impls():
    out = [("oracle", ko.orc())]
    r = ko.ref()
    if r is not None:
        out.append(("reference", r))
    return out


def test_fixture_hashes():
    """The copied fixtures are byte-identical to the ones the reference ships."""
    for line in (REF_OPS / "SHA256SUMS").read_text().splitlines():
        digest, name = line.split()
        assert hashlib.sha256((REF_OPS / name).read_bytes()).hexdigest() == digest, name


def test_manifest_tolerance():
    assert (ATOL, RTOL) == (1e-5, 1e-4)


@pytest.mark.parametrize("name,L", impls())
def test_rmsnorm(name, L):
    f = load_fixture("rmsnorm")
    w, x, e = f["weight"], f["in"], f["out"]
    n = w.size
    y = np.zeros_like(x)
    for r in range(x.shape[0]):
        row_in = np.ascontiguousarray(x[r])
        row_out = np.zeros(n, np.float32)
        ko.call(L, "rmsnorm", ko.ptr(row_out), ko.ptr(row_in), ko.ptr(w), n, f["eps"])
        y[r] = row_out
    assert worst_ratio(y, e, ATOL, RTOL) <= 1.0


@pytest.mark.parametrize("name,L", impls())
def test_shortconv_with_continuation(name, L):
    f = load_fixture("shortconv")
    K, Cn = int(f["kernel"]), int(f["channels"])
    w = ko.f32(f["weight"].reshape(Cn, K))
    x = ko.f32(f["in"].reshape(-1, Cn))
    T = x.shape[0]
    y = np.zeros_like(x)
    st = np.zeros(Cn * (K - 1), np.float32)
    ko.call(L, "shortconv", ko.ptr(y), ko.ptr(x), ko.ptr(w), ko.ptr(st), Cn, K, T)
    assert worst_ratio(y, f["out"], ATOL, RTOL) <= 1.0
    assert worst_ratio(st, f["state_after"], ATOL, RTOL) <= 1.0
    # the only check that sees the READ side of the carried history (test_ops.c:212-229)
    xn = ko.f32(f["in_next"].reshape(-1, Cn))
    yn = np.zeros_like(xn)
    ko.call(L, "shortconv", ko.ptr(yn), ko.ptr(xn), ko.ptr(w), ko.ptr(st), Cn, K, xn.shape[0])
    assert worst_ratio(yn, f["out_next"], ATOL, RTOL) <= 1.0


@pytest.mark.parametrize("name,L", impls())
def test_kda_decay(name, L):
    f = load_fixture("kda_decay")
    A, dt, z = f["A_log"], f["dt_bias"], f["z"].reshape(-1)
    H = A.size
    D = dt.size // H
    tok = z.size // dt.size
    g = np.zeros(z.size, np.float32)
    al = np.zeros(z.size, np.float32)
    for t in range(tok):
        o = t * H * D
        zz = np.ascontiguousarray(z[o:o + H * D])
        gg = np.zeros(H * D, np.float32)
        aa = np.zeros(H * D, np.float32)
        ko.call(L, "kda_decay", ko.ptr(gg), ko.ptr(aa), ko.ptr(zz), ko.ptr(A), ko.ptr(dt), H, D,
                f["lower_bound"])
        g[o:o + H * D], al[o:o + H * D] = gg, aa
    # the reference gate: absolute error <= 1e-5 on g and alpha (test_ops.c:262)
    assert np.max(np.abs(g - f["g"].reshape(-1))) <= 1e-5
    assert np.max(np.abs(al - f["alpha"].reshape(-1))) <= 1e-5


@pytest.mark.parametrize("fname", ["kda_recur1", "kda_recur8"])
@pytest.mark.parametrize("name,L", impls())
def test_kda_recur(fname, name, L):
    f = load_fixture(fname)
    T, H, dk, dv = int(f["T"]), int(f["H"]), int(f["d_k"]), int(f["d_v"])
    qs = np.float32(f["q_scale"])
    q, k, v = f["q"], f["k"], f["v"]
    al, bt = f["alpha"], f["beta"]
    S = np.zeros((H, dk, dv), np.float32)
    out = np.zeros((T, H, dv), np.float32)
    for t in range(T):
        for h in range(H):
            qsc = ko.f32(q[t, h] * qs)
            Sh = S[h]
            o = np.zeros(dv, np.float32)
            ko.call(L, "kda_step", ko.ptr(Sh), ko.ptr(o), ko.ptr(qsc), ko.ptr(ko.f32(k[t, h])),
                    ko.ptr(ko.f32(v[t, h])), ko.ptr(ko.f32(al[t, h])), float(bt[t, h]), dk, dv)
            out[t, h] = o
    assert worst_ratio(out, f["out"], ATOL, RTOL) <= 1.0
    assert worst_ratio(S, f["state_out"], ATOL, RTOL) <= 1.0


def layer_weights(f) -> ko.Weights:
    P = int(f["H"]) * int(f["d_k"])
    K = int(f["conv_k"])
    arrays = {
        "q": f["q_proj"], "k": f["k_proj"], "v": f["v_proj"], "g": f["g_proj"],
        "o": f["o_proj"], "f_a": f["f_a"], "f_b": f["f_b"], "b": f["b_proj"],
        "q_conv": f["q_conv"].reshape(P, K), "k_conv": f["k_conv"].reshape(P, K),
        "v_conv": f["v_conv"].reshape(P, K), "A_log": f["A_log"], "dt_bias": f["dt_bias"],
        "o_norm": f["o_norm"],
    }
    return ko.Weights(arrays, 0)


def layer_cfg(f):
    x = f["in"]
    return ko.make_cfg(hidden=x.shape[2], heads=int(f["H"]), head_dim=int(f["d_k"]),
                       conv_k=int(f["conv_k"]), gate_lb=float(f["lower_bound"]),
                       rms_eps=float(f["rms_eps"]))


@pytest.mark.parametrize("fname", ["kda_layer1", "kda_layer8"])
@pytest.mark.parametrize("name,L", impls())
def test_kda_layer(fname, name, L):
    f = load_fixture(fname)
    cfg = layer_cfg(f)
    W = layer_weights(f)
    H, D, K = cfg.kda_heads, cfg.kda_head_dim, cfg.conv_k
    P = H * D
    T = f["in"].shape[1]
    state = np.zeros(P * D + 3 * P * (K - 1), np.float32)
    out = ko.kda_layer(L, f["in"].reshape(T, -1), W, cfg, T, state)
    assert worst_ratio(out, f["out"].reshape(T, -1), ATOL, RTOL) <= 1.0
    assert worst_ratio(state[:H * D * D], f["state_out"], ATOL, RTOL) <= 1.0


def test_oracle_equals_reference_on_fixtures():
    """Where the reference C is built, the restatement reproduces it bit for bit on the
    fixture layers (same arithmetic, same summation trees)."""
    R = ko.ref()
    if R is None:
        pytest.skip("reference C not built on this machine (its sources are absent)")
    for fname in ("kda_layer1", "kda_layer8"):
        f = load_fixture(fname)
        cfg, W = layer_cfg(f), layer_weights(f)
        P = cfg.kda_heads * cfg.kda_head_dim
        T = f["in"].shape[1]
        n = P * cfg.kda_head_dim + 3 * P * (cfg.conv_k - 1)
        s1, s2 = np.zeros(n, np.float32), np.zeros(n, np.float32)
        o1 = ko.kda_layer(ko.orc(), f["in"].reshape(T, -1), W, cfg, T, s1)
        o2 = ko.kda_layer(R, f["in"].reshape(T, -1), W, cfg, T, s2)
        assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32)), fname
        assert np.array_equal(s1.view(np.uint32), s2.view(np.uint32)), fname


def mla_from_fixture():
    r = load_fixture("mla")
    T, hidden = r["in"].shape[1], r["in"].shape[2]
    cfg = ko.mla_cfg(hidden, int(r["n_heads"]), int(r["q_lora"]), int(r["kv_lora"]),
                     int(r["qk_nope"]), int(r["qk_rope"]), int(r["v_head"]), float(r["rms_eps"]))
    names = {"q_a": "q_a_proj_weight", "q_a_norm": "q_a_layernorm_weight", "q_b": "q_b_proj_weight",
             "kv_a": "kv_a_proj_with_mqa_weight", "kv_a_norm": "kv_a_layernorm_weight",
             "kv_b": "kv_b_proj_weight", "o": "o_proj_weight", "g": "g_proj_weight"}
    W = ko.MlaWeights({k: r[v] for k, v in names.items()}, 0)
    return r, cfg, W, T


def test_mla_fixture():
    """t_mla (tests/unit/test_ops.c:410-470): the uncached gated MLA over the fixture's T
    tokens, the softmax scale over the full head width (nope + rope)."""
    r, cfg, W, T = mla_from_fixture()
    assert abs(float(r["scale"]) - 1.0 / np.sqrt(cfg.qk_nope + cfg.qk_rope)) < 1e-7
    x = r["in"].reshape(T, cfg.hidden)
    libs = ["orc"] + (["ref"] if ko.ref() is not None else [])
    for lib in libs:
        y = ko.mla(x, W, cfg, T, lib=lib)
        assert worst_ratio(y, r["out"].reshape(T, cfg.hidden), ATOL, RTOL) <= 1.0, lib


def test_mla_cached_equals_uncached():
    """The expanded-KV cache path token by token gives the uncached sequence's outputs
    (the property tests/unit/k3_model.c gates between the two reference paths)."""
    r, cfg, W, T = mla_from_fixture()
    x = r["in"].reshape(T, cfg.hidden)
    want = ko.mla(x, W, cfg, T)
    H, kvd = cfg.n_heads, cfg.qk_nope + cfg.v_head
    cap = T + 2
    kvc = np.zeros((cap, H * kvd), np.float32)
    ropec = np.zeros((cap, cfg.qk_rope), np.float32)
    rows = [ko.mla(x[t:t + 1], W, cfg, 1, kvc, ropec, t, cap) for t in range(T)]
    assert np.array_equal(np.concatenate(rows), want)
