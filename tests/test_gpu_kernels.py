# SPDX-License-Identifier: Apache-2.0
"""GPU parity: each HIP kernel, through the C ABI, against the CPU oracle on the same
seeded inputs.

Tolerances, in the reference comparator form |got - want| <= atol + rtol |want|:
  decode (K3), recurrence: rtol 1e-4, atol 1e-4 * rms(want)   (fp32 state)
  prep (K1), epilogue (K4): rtol 1e-5, atol 1e-6              (elementwise fp32)
  drop-in layer vs fixtures: the manifest's atol 1e-5, rtol 1e-4
The sequential GPU recurrence keeps the reference's operation order, so it must equal the
oracle bit for bit."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_close, load_fixture, manifest_tol
import k3_oracle as ko
from k3_oracle import f32

pytestmark = pytest.mark.gpu


def dev(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


def host(t):
    return t.float().cpu().numpy() if t.dtype != __import__("torch").float32 else t.cpu().numpy()


def rms(a):
    return float(np.sqrt(np.mean(np.asarray(a, np.float64) ** 2)))


def decode_inputs(rng, B, H, D):
    S = f32(rng.standard_normal((B, H, D, D)) * 0.1)
    q = rng.standard_normal((B, H, D))
    k = rng.standard_normal((B, H, D))
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((B, H, D))
    g = rng.uniform(-5.0, 0.0, (B, H, D))
    return S, f32(q), f32(k), f32(v), f32(np.exp(g)), f32(rng.uniform(0, 1, (B, H)))


@pytest.mark.parametrize("B,H,D", [(2, 3, 16), (3, 2, 32), (4, 8, 64), (4, 8, 128), (37, 32, 128), (64, 32, 128)])
def test_decode_vs_oracle(gpu, B, H, D):
    import torch
    rng = np.random.default_rng(0x4B334441 + 1 + B + D)
    S, q, k, v, al, bt = decode_inputs(rng, B, H, D)
    k[0, 0, ::9] = 0.0          # skipped rows
    q[-1, -1, ::5] = 0.0
    al[0, -1, :7] = 1.0         # saturated retention is legal
    qs = np.float32(1.0) / np.sqrt(np.float32(D))
    Sref = S.copy()
    oref = ko.decode_batch(Sref, q, k, v, al, bt, float(qs), nthreads=8)
    dS, do = dev(S), torch.zeros((B, H, D), device="cuda")
    gpu.kda_decode(dS, do, dev(q), dev(k), dev(v), dev(al), dev(bt), float(qs))
    torch.cuda.synchronize()
    assert_close(host(do), oref, 1e-4 * rms(oref), 1e-4, "decode o")
    assert_close(host(dS), Sref, 1e-4 * rms(Sref), 1e-4, "decode S")


def test_decode_deterministic_and_isolated(gpu):
    """Same inputs, same bits; a sequence's result does not depend on its neighbours."""
    import torch
    rng = np.random.default_rng(11)
    B, H, D = 8, 4, 128
    S, q, k, v, al, bt = decode_inputs(rng, B, H, D)
    outs = []
    for _ in range(2):
        dS, do = dev(S), torch.zeros((B, H, D), device="cuda")
        gpu.kda_decode(dS, do, dev(q), dev(k), dev(v), dev(al), dev(bt), 0.125)
        torch.cuda.synchronize()
        outs.append((host(dS), host(do)))
    assert np.array_equal(outs[0][0].view(np.uint32), outs[1][0].view(np.uint32))
    assert np.array_equal(outs[0][1].view(np.uint32), outs[1][1].view(np.uint32))
    # sequence 3 alone gives the same bits as inside the batch
    dS1, do1 = dev(S[3:4]), torch.zeros((1, H, D), device="cuda")
    gpu.kda_decode(dS1, do1, dev(q[3:4]), dev(k[3:4]), dev(v[3:4]), dev(al[3:4]), dev(bt[3:4]), 0.125)
    torch.cuda.synchronize()
    assert np.array_equal(host(do1)[0].view(np.uint32), outs[0][1][3].view(np.uint32))


def test_decode_empty_and_errors(gpu):
    """B = 0 is a no-op; an unsupported head size is refused before any launch."""
    import torch
    e0 = torch.zeros((0, 1, 16), device="cuda")
    gpu.kda_decode(torch.zeros((0, 1, 16, 16), device="cuda"), e0, e0, e0, e0, e0,
                   torch.zeros((0, 1), device="cuda"), 0.25)
    t = torch.zeros((1, 1, 48), device="cuda")
    with pytest.raises(gpu.K3HipError) as e:
        gpu.kda_decode(torch.zeros((1, 1, 48, 48), device="cuda"), t, t, t, t, t,
                       torch.zeros((1, 1), device="cuda"), 0.1)
    assert e.value.code == gpu.EUNSUPPORTED


def prep_case(rng, T, H, D, K):
    P = H * D
    arrays = {
        "q_conv": f32(rng.standard_normal((P, K)) * 0.5),
        "k_conv": f32(rng.standard_normal((P, K)) * 0.5),
        "v_conv": f32(rng.standard_normal((P, K)) * 0.5),
        "A_log": f32(rng.uniform(0, 1.5, H)), "dt_bias": f32(rng.standard_normal(P)),
        "o_norm": f32(1 + 0.1 * rng.standard_normal(D)),
    }
    for n in ("q", "k", "v", "g", "f_a", "f_b", "b", "o"):
        arrays[n] = np.zeros((1, 1), np.float32)
    W = ko.Weights(arrays, 0)
    ins = [f32(rng.standard_normal((T, P))) for _ in range(3)]
    z = f32(rng.standard_normal((T, P)) * 2.0)
    bl = f32(rng.standard_normal((T, H)))
    return W, ins, z, bl


def run_prep_gpu(gpu, W, ins, z, bl, H, D, K, lb, cs_dev, dtype=None):
    import torch
    T, P = ins[0].shape
    outs = [torch.zeros((T, P), device="cuda") for _ in range(5)]
    beta = torch.zeros((T, H), device="cuda")
    a = W.arrays
    gpu.kda_prep(dev(ins[0], dtype), dev(ins[1], dtype), dev(ins[2], dtype), dev(z), dev(bl),
                 dev(a["q_conv"]), dev(a["k_conv"]), dev(a["v_conv"]), dev(a["A_log"]),
                 dev(a["dt_bias"]), cs_dev, *outs, beta, H, D, K, lb)
    torch.cuda.synchronize()
    return [host(o) for o in outs] + [host(beta)]


@pytest.mark.parametrize("T,H,D,K", [(1, 2, 16, 4), (2, 3, 32, 4), (5, 2, 64, 2), (33, 4, 128, 4),
                                     (100, 2, 128, 1), (70, 3, 64, 3)])
def test_prep_vs_oracle_with_carried_state(gpu, T, H, D, K):
    rng = np.random.default_rng(T * 131 + D + K)
    cfg = ko.make_cfg(8, H, D, K, -5.0, 1e-5)
    P = H * D
    W, ins, z, bl = prep_case(rng, T, H, D, K)
    cs = f32(rng.standard_normal(3 * P * (K - 1)))
    cs_ref = cs.copy()
    want = ko.prep(*ins, z, bl, W, cfg, T, cs_ref)
    dcs = dev(cs) if K > 1 else None
    got = run_prep_gpu(gpu, W, ins, z, bl, H, D, K, -5.0, dcs)
    names = ["q", "k", "v", "g", "alpha", "beta"]
    for n, g_, w_ in zip(names, got, want):
        assert_close(g_, w_, 1e-6, 1e-5, f"prep {n}")
    if K > 1:
        assert np.array_equal(host(dcs), cs_ref), "outgoing conv history"
        # continuation: a second call reads the history the first one left
        W2 = W
        _, ins2, z2, bl2 = prep_case(rng, 3, H, D, K)
        want2 = ko.prep(*ins2, z2, bl2, W2, cfg, 3, cs_ref)
        got2 = run_prep_gpu(gpu, W2, ins2, z2, bl2, H, D, K, -5.0, dcs)
        for n, g_, w_ in zip(names, got2, want2):
            assert_close(g_, w_, 1e-6, 1e-5, f"prep continuation {n}")
        assert np.array_equal(host(dcs), cs_ref)


def test_prep_null_state_and_bf16_inputs(gpu):
    import torch
    rng = np.random.default_rng(5)
    T, H, D, K = 40, 2, 128, 4
    cfg = ko.make_cfg(8, H, D, K, -5.0, 1e-5)
    W, ins, z, bl = prep_case(rng, T, H, D, K)
    ins_bf = [host(dev(x, torch.bfloat16)) for x in ins]   # the values the GPU will see
    want = ko.prep(*ins_bf, z, bl, W, cfg, T, None)
    got = run_prep_gpu(gpu, W, ins, z, bl, H, D, K, -5.0, None, torch.bfloat16)
    for g_, w_ in zip(got, want):
        assert_close(g_, w_, 1e-6, 1e-5, "prep bf16")


def rec_inputs(rng, T, H, D):
    P = H * D
    q = rng.standard_normal((T, H, D))
    k = rng.standard_normal((T, H, D))
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((T, P))
    g = rng.uniform(-5.0, 0.0, (T, P))
    return (f32(q.reshape(T, P)), f32(k.reshape(T, P)), f32(v), f32(g), f32(np.exp(g)),
            f32(rng.uniform(0, 1, (T, H))))


@pytest.mark.parametrize("T,H,D", [(1, 2, 16), (37, 3, 32), (64, 2, 64), (130, 4, 128)])
def test_recurrent_bitwise_vs_oracle(gpu, T, H, D):
    import torch
    rng = np.random.default_rng(T + H + D)
    q, k, v, g, al, bt = rec_inputs(rng, T, H, D)
    k[3 % T, :5] = 0.0
    S0 = f32(rng.standard_normal((H, D, D)) * 0.1)
    qs = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    Sref = S0.copy()
    oref = ko.recurrence(Sref, q, k, v, al, bt, H, D, qs, nthreads=4)
    dS, do = dev(S0), torch.zeros((T, H * D), device="cuda")
    gpu.kda_recurrent(dev(q), dev(k), dev(v), dev(al), dev(bt), dS, do, H, D, qs)
    torch.cuda.synchronize()
    assert np.array_equal(host(do).view(np.uint32), oref.view(np.uint32)), \
        f"max |d| {np.max(np.abs(host(do) - oref))}"
    assert np.array_equal(host(dS).view(np.uint32), Sref.view(np.uint32))


@pytest.mark.parametrize("T,H,D", [(1, 1, 16), (5, 3, 64), (77, 4, 128), (3, 5, 64), (1037, 2, 128)])
def test_epilogue_vs_oracle(gpu, T, H, D):
    import torch
    rng = np.random.default_rng(T * 7 + D)
    P = H * D
    o = f32(rng.standard_normal((T, P)))
    gate = f32(rng.standard_normal((T, P)) * 2)
    wn = f32(1 + 0.1 * rng.standard_normal(D))
    L = ko.orc()
    want = np.zeros((T, P), np.float32)
    for t in range(T):
        for h in range(H):
            row = np.ascontiguousarray(o[t, h * D:(h + 1) * D])
            y = np.zeros(D, np.float32)
            L.orc_rmsnorm(ko.ptr(y), ko.ptr(row), ko.ptr(wn), D, 1e-5)
            want[t, h * D:(h + 1) * D] = y * np.array([L.orc_sigmoid(float(x)) for x in gate[t, h * D:(h + 1) * D]], np.float32)
    y = torch.zeros((T, P), device="cuda")
    gpu.kda_epilogue(dev(o), dev(gate), dev(wn), y, H, D, 1e-5)
    torch.cuda.synchronize()
    assert_close(host(y), want, 1e-6, 1e-5, "epilogue")
    yb = torch.zeros((T, P), device="cuda", dtype=torch.bfloat16)
    gpu.kda_epilogue(dev(o), dev(gate), dev(wn), yb, H, D, 1e-5)
    torch.cuda.synchronize()
    assert_close(host(yb), want, 1e-6, 2 ** -8, "epilogue bf16 out")
    # bf16 gate -> bf16 y (the prefill core's form, its own kernel for D >= 64): the oracle on
    # the bf16-rounded gate
    gb = torch.from_numpy(gate).to(torch.bfloat16)
    gr = gb.float().numpy()
    want_b = np.zeros((T, P), np.float32)
    for t in range(T):
        for h in range(H):
            row = np.ascontiguousarray(o[t, h * D:(h + 1) * D])
            yy = np.zeros(D, np.float32)
            L.orc_rmsnorm(ko.ptr(yy), ko.ptr(row), ko.ptr(wn), D, 1e-5)
            want_b[t, h * D:(h + 1) * D] = yy * np.array([L.orc_sigmoid(float(x)) for x in gr[t, h * D:(h + 1) * D]], np.float32)
    ybb = torch.zeros((T, P), device="cuda", dtype=torch.bfloat16)
    gpu.kda_epilogue(dev(o), gb.cuda(), dev(wn), ybb, H, D, 1e-5)
    torch.cuda.synchronize()
    assert_close(host(ybb), want_b, 1e-6, 2 ** -8, "epilogue bf16 gate, bf16 out")


@pytest.mark.parametrize("fname", ["kda_layer1", "kda_layer8"])
def test_dropin_layer_vs_reference_fixtures(gpu, fname):
    """k3_kda_layer (host pointers, the reference signature) against the reference's own
    fixture at the manifest tolerance, then a decode step from the returned state
    against the oracle."""
    from test_oracle_golden import layer_cfg, layer_weights
    f = load_fixture(fname)
    cfg, W = layer_cfg(f), layer_weights(f)
    atol, rtol = manifest_tol()
    H, D, K = cfg.kda_heads, cfg.kda_head_dim, cfg.conv_k
    P = H * D
    T = f["in"].shape[1]
    x = f32(f["in"].reshape(T, -1))
    state = np.zeros(P * D + 3 * P * (K - 1), np.float32)
    out = np.zeros((T, cfg.hidden), np.float32)
    gpu.kda_layer_host(out, x, W.w, cfg, T, state)
    assert_close(out, f["out"].reshape(T, -1), atol, rtol, f"{fname} out")
    assert_close(state[:H * D * D], f["state_out"], atol, rtol, f"{fname} state")
    st_ref = np.zeros_like(state)
    ko.kda_layer(ko.orc(), x, W, cfg, T, st_ref)
    assert_close(state, st_ref, 1e-6, 1e-5, "full state incl. conv history")
    x1 = f32(np.random.default_rng(1).standard_normal((1, cfg.hidden)))
    out1 = np.zeros((1, cfg.hidden), np.float32)
    gpu.kda_layer_host(out1, x1, W.w, cfg, 1, state)
    want1 = ko.kda_layer(ko.orc(), x1, W, cfg, 1, st_ref)
    assert_close(out1, want1, atol, rtol, "decode after prefill")
    assert_close(state, st_ref, 1e-6, 1e-5, "state after decode")


@pytest.mark.parametrize("hidden,H,D,T,wdt", [(256, 4, 64, 32, 0), (256, 2, 128, 9, 1)])
def test_device_layer_vs_oracle(gpu, hidden, H, D, T, wdt):
    import torch
    from test_oracle_ref import rand_layer
    rng = np.random.default_rng(hidden + T)
    W = rand_layer(rng, hidden, H, D, 4, wdt)
    cfg = ko.make_cfg(hidden, H, D, 4, -5.0, 1e-5)
    P = H * D
    n = P * D + 3 * P * 3
    s0 = f32(rng.standard_normal(n) * 0.1)
    x = f32(rng.standard_normal((T, hidden)))
    st_ref = s0.copy()
    want = ko.kda_layer(ko.orc(), x, W, cfg, T, st_ref)
    dw = gpu.DeviceWeights(W.w, cfg)
    dst = dev(s0)
    out = torch.zeros((T, hidden), device="cuda")
    dw.layer(out, dev(x), dst, T)
    torch.cuda.synchronize()
    assert_close(host(out), want, 1e-4 * rms(want), 1e-4, "device layer out")
    assert_close(host(dst), st_ref, 1e-4 * rms(st_ref), 1e-4, "device layer state")
    # NULL state: a fresh sequence
    out0 = torch.zeros((T, hidden), device="cuda")
    dw.layer(out0, dev(x), None, T)
    torch.cuda.synchronize()
    want0 = ko.kda_layer(ko.orc(), x, W, cfg, T, None)
    assert_close(host(out0), want0, 1e-4 * rms(want0), 1e-4, "device layer, NULL state")
    dw.close()
