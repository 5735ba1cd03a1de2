# SPDX-License-Identifier: Apache-2.0
"""Device-resident state for a decode loop (k3hip_kda_states_*), and weight binding.

- A 3-layer KDA stack run as the reference's forward() runs it (src/cli/k3_run.c:514-567):
  one state slot per layer in kstate[L * kper], a T=24 prefill then 5 single-token decode
  steps, each layer's output feeding the next. Compared step by step with the CPU oracle's
  k3_kda_layer on host slots, and the downloaded device array against the oracle's kstate.
  Prefill runs the chunked kernel, so the bar is the chunked one (rtol 2e-3,
  atol 2e-3 * rms); the 1e-4 ratio is printed.
- Speculative-decode snapshot / restore (src/cli/k3_run.c:1969-1984) as device copies:
  the replay after a restore is bit-identical to the first pass.
- Upload of a host kstate (as k3_state_load fills it) continues exactly like the oracle
  continuing from the same array (decode bar, rtol 1e-4).
- Decode after a prefill of T equals a prefill of T+1 (last row).
- A_log shipped as [128] with a non-zero tail: only the first H values are per-head
  (src/model/k3_bind.c:212-216, k3_bind.h:29-31); the tail must not change anything.
- The batched decode layer (k3hip_kda_layer_decode): B sequences, one token each, states in
  strided slots, against the oracle's k3_kda_layer per sequence at the decode bar.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_close, worst_ratio
import k3_oracle as ko
from k3_oracle import f32

pytestmark = pytest.mark.gpu

HID, H, D, K, LAYERS = 256, 4, 64, 4, 3


def rms(a):
    return float(np.sqrt(np.mean(np.asarray(a, np.float64) ** 2)))


def weights(rng, a_log_len=H):
    P = H * D
    nrm = lambda *s: f32(rng.standard_normal(s) * 0.02)
    A_log = f32(rng.uniform(0, 1.5, a_log_len))
    arrays = {"q": nrm(P, HID), "k": nrm(P, HID), "v": nrm(P, HID), "g": nrm(P, HID),
              "o": nrm(HID, P), "f_a": nrm(D, HID), "f_b": nrm(P, D), "b": nrm(H, HID),
              "q_conv": nrm(P, K), "k_conv": nrm(P, K), "v_conv": nrm(P, K), "A_log": A_log,
              "dt_bias": f32(rng.standard_normal(P)), "o_norm": f32(1 + 0.02 * rng.standard_normal(D))}
    return ko.Weights(arrays, 0)


def stack(gpu, rng):
    cfg = ko.make_cfg(HID, H, D, K, -5.0, 1e-5)
    Ws = [weights(rng) for _ in range(LAYERS)]
    dws = [gpu.DeviceWeights(W.w, cfg) for W in Ws]
    return cfg, Ws, dws


def gpu_forward(dws, pool, x, T):
    import torch
    h = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    for L, dw in enumerate(dws):
        out = torch.empty((T, HID), device="cuda")
        dw.layer(out, h, pool.layer(L), T)
        h = out
    torch.cuda.synchronize()
    return h


def cpu_forward(Ws, cfg, kstate, x, T):
    kper = kstate.size // LAYERS
    h = x
    for L, W in enumerate(Ws):
        st = kstate[L * kper:(L + 1) * kper]          # a view: updated in place
        h = ko.kda_layer(ko.orc(), h, W, cfg, T, st)
    return h


def test_decode_loop_stack_and_state_array(gpu):
    rng = np.random.default_rng(0x4B334441 + 20)
    cfg, Ws, dws = stack(gpu, rng)
    pool = gpu.States(cfg, LAYERS)
    kstate = np.zeros(LAYERS * pool.kper, np.float32)
    assert pool.kper == H * D * D + 3 * H * D * (K - 1)
    for step, T in enumerate([24] + [1] * 5):
        x = f32(rng.standard_normal((T, HID)))
        want = cpu_forward(Ws, cfg, kstate, x, T)
        got = gpu_forward(dws, pool, x, T).cpu().numpy()
        r = assert_close(got, want, 2e-3 * rms(want), 2e-3, f"stack step {step}")
        print(f"step {step} T={T}: worst {r:.4f}x of 2e-3, {worst_ratio(got, want, 1e-4 * rms(want), 1e-4):.3f}x of 1e-4")
    dev = pool.download()
    assert_close(dev, kstate, 2e-3 * rms(kstate), 2e-3, "downloaded kstate vs oracle")
    pool.close()
    for dw in dws:
        dw.close()


def test_snapshot_restore_replays_bitwise(gpu):
    import torch
    rng = np.random.default_rng(0x4B334441 + 21)
    cfg, Ws, dws = stack(gpu, rng)
    pool, snap = gpu.States(cfg, LAYERS), gpu.States(cfg, LAYERS)
    gpu_forward(dws, pool, f32(rng.standard_normal((40, HID))), 40)
    xs = [f32(rng.standard_normal((1, HID))) for _ in range(3)]
    snap.copy_from(pool)
    before = snap.download()
    first = [gpu_forward(dws, pool, x, 1).clone() for x in xs]        # a rejected draft
    assert not np.array_equal(pool.download(), before)
    pool.copy_from(snap)                                               # restore
    assert np.array_equal(pool.download(), before)
    again = [gpu_forward(dws, pool, x, 1) for x in xs]
    for a, b in zip(first, again):
        assert torch.equal(a, b), "replay after restore differs"
    for o in (pool, snap):
        o.close()
    for dw in dws:
        dw.close()


def test_upload_host_state_continues_like_oracle(gpu):
    rng = np.random.default_rng(0x4B334441 + 22)
    cfg, Ws, dws = stack(gpu, rng)
    kper = ko_kper = H * D * D + 3 * H * D * (K - 1)
    kstate = f32(rng.standard_normal(LAYERS * ko_kper) * 0.1)   # as k3_state_load would fill it
    pool = gpu.States(cfg, LAYERS)
    pool.upload(kstate)
    assert np.array_equal(pool.download(), kstate)
    for step in range(3):
        x = f32(rng.standard_normal((1, HID)))
        want = cpu_forward(Ws, cfg, kstate, x, 1)
        got = gpu_forward(dws, pool, x, 1).cpu().numpy()
        assert_close(got, want, 1e-4 * rms(want), 1e-4, f"decode after upload, step {step}")
    assert_close(pool.download(), kstate, 1e-4 * rms(kstate), 1e-4, "state after 3 decodes")
    assert kper == pool.kper
    pool.close()
    for dw in dws:
        dw.close()


def test_decode_after_prefill_equals_longer_prefill(gpu):
    import torch
    rng = np.random.default_rng(0x4B334441 + 23)
    cfg = ko.make_cfg(HID, H, D, K, -5.0, 1e-5)
    W = weights(rng)
    dw = gpu.DeviceWeights(W.w, cfg)
    T = 37
    x = torch.from_numpy(f32(rng.standard_normal((T + 1, HID)))).cuda()
    a, b = gpu.States(cfg, 1), gpu.States(cfg, 1)
    out_a = torch.empty((T, HID), device="cuda")
    dw.layer(out_a, x[:T].contiguous(), a.layer(0), T)
    last = torch.empty((1, HID), device="cuda")
    dw.layer(last, x[T:].contiguous(), a.layer(0), 1)
    out_b = torch.empty((T + 1, HID), device="cuda")
    dw.layer(out_b, x, b.layer(0), T + 1)
    torch.cuda.synchronize()
    want, got = out_b[T:].cpu().numpy(), last.cpu().numpy()
    assert_close(got, want, 2e-3 * rms(want), 2e-3, "decode after prefill vs prefill T+1")
    sa, sb = a.download(), b.download()
    assert_close(sa, sb, 2e-3 * rms(sb), 2e-3, "state")
    for o in (a, b, dw):
        o.close()


def test_a_log_per_head_binding(gpu):
    import torch
    rng = np.random.default_rng(0x4B334441 + 24)
    cfg = ko.make_cfg(HID, H, D, K, -5.0, 1e-5)
    W = weights(rng, a_log_len=H)
    arrays = dict(W.arrays)
    shipped = np.concatenate([arrays["A_log"], f32(rng.uniform(-3, 3, 128 - H))])   # [128], live tail
    arrays["A_log"] = shipped
    W128 = ko.Weights(arrays, 0)
    x = torch.from_numpy(f32(rng.standard_normal((20, HID)))).cuda()
    outs = []
    for w_ in (W, W128):
        dw = gpu.DeviceWeights(w_.w, cfg)
        o = torch.empty((20, HID), device="cuda")
        dw.layer(o, x, None, 20)
        torch.cuda.synchronize()
        outs.append(o.clone())
        dw.close()
    assert torch.equal(outs[0], outs[1]), "A_log beyond the first H heads changed the output"
    want = ko.kda_layer(ko.orc(), x.cpu().numpy(), W128, cfg, 20, None)   # oracle reads A_log[h] too
    assert_close(outs[1].cpu().numpy(), want, 2e-3 * rms(want), 2e-3, "128-entry A_log vs oracle")


@pytest.mark.parametrize("D,K,B,lb", [(64, 4, 5, -5.0), (128, 3, 3, -5.0), (32, 4, 2, 0.0),
                                      (128, 4, 17, -5.0), (16, 2, 70, -5.0)])
def test_batched_layer_decode_vs_oracle(gpu, D, K, B, lb):
    """k3hip_kda_layer_decode: B sequences, one token each per step, states in B slots of a
    strided array (stride > kper), bf16 weights; each sequence against the oracle's
    k3_kda_layer with T = 1 on its own state, at the decode bar (rtol 1e-4, atol 1e-4*rms).
    B = 17 and 70 take two 16-row tiles and two 64-row passes of the projection kernel; D = 16
    gives K = 16 for f_b. The lb = 0 case runs the unbounded softplus gate (parity unpinned)."""
    _batched_layer_decode(gpu, D, K, B, lb, 3, 192, 0x4B334441 + 25 + D + B)


@pytest.mark.parametrize("case", range(10))
def test_batched_layer_decode_random_vs_oracle(gpu, case):
    """Seeded random batched decodes at the decode bar: D 16-128, conv_k 1-4, B 1-40, 1-4 heads,
    hidden a multiple of 64 in [64, 512], a gate bound in [-5.3, -0.1] (every fourth case the
    unbounded softplus gate)."""
    rng = np.random.default_rng(0x4B334441 + 0xDEC + case)
    D, K = int(rng.choice([16, 32, 64, 128])), int(rng.integers(1, 5))
    B, Hh, hid = int(rng.integers(1, 41)), int(rng.integers(1, 5)), 64 * int(rng.integers(1, 9))
    lb = 0.0 if case % 4 == 3 else float(np.float32(-rng.uniform(0.1, 5.3)))
    _batched_layer_decode(gpu, D, K, B, lb, Hh, hid, 0x4B334441 + 0xDEC + case)


def _batched_layer_decode(gpu, D, K, B, lb, Hh, hid, seed):
    import torch
    from test_oracle_ref import bf16
    rng = np.random.default_rng(seed)
    print(f"D={D} K={K} B={B} heads={Hh} hidden={hid} gate_lb={lb:.3f}", flush=True)
    P = Hh * D
    cfg = ko.make_cfg(hid, Hh, D, K, lb, 1e-5)
    nrm = lambda *s: rng.standard_normal(s) * 0.05
    arrays = {n: bf16(nrm(*s)) for n, s in {"q": (P, hid), "k": (P, hid), "v": (P, hid), "g": (P, hid),
                                             "o": (hid, P), "f_a": (D, hid), "f_b": (P, D), "b": (Hh, hid)}.items()}
    arrays.update({"q_conv": f32(rng.standard_normal((P, K)) * 0.5), "k_conv": f32(rng.standard_normal((P, K)) * 0.5),
                   "v_conv": f32(rng.standard_normal((P, K)) * 0.5), "A_log": f32(rng.uniform(0, 1.5, Hh)),
                   "dt_bias": f32(rng.standard_normal(P)), "o_norm": f32(1 + 0.1 * rng.standard_normal(D))})
    W = ko.Weights(arrays, 1)
    kper = P * D + 3 * P * (K - 1)
    stride = kper + 8
    host = [f32(rng.standard_normal(kper) * 0.05) for _ in range(B)]
    dev = torch.zeros((B, stride), device="cuda")
    for b in range(B):
        dev[b, :kper] = torch.from_numpy(host[b])
    dw = gpu.DeviceWeights(W.w, cfg)
    worst = 0.0
    for step in range(4):
        x = f32(rng.standard_normal((B, hid)))
        want = np.concatenate([ko.kda_layer(ko.orc(), x[b:b + 1], W, cfg, 1, host[b]) for b in range(B)])
        out = torch.full((B, hid), float("nan"), device="cuda")
        dw.layer_decode(out, torch.from_numpy(x).cuda(), dev, stride)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert_close(got, want, 1e-4 * rms(want), 1e-4, f"batched decode step {step}")
        worst = max(worst, worst_ratio(got, want, 1e-4 * rms(want), 1e-4))
    st = dev.cpu().numpy()
    for b in range(B):
        assert_close(st[b, :kper], host[b], 1e-4 * rms(host[b]), 1e-4, f"state of sequence {b}")
        assert np.all(st[b, kper:] == 0.0), "padding between slots untouched"
    print(f"  worst {worst:.3f}x of the 1e-4 bar")
    dw.close()
