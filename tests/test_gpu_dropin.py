# SPDX-License-Identifier: Apache-2.0
"""The drop-in k3_kda_layer as the engine would use it.

1. From C: oracle/_ref/dropin_harness is compiled against the reference's own header
   (include/k3/k3.h) and linked to libk3kda_hip.so in place of the reference's k3_ops.c, the
   link-time substitution of the integration notes. It runs the reference's t_kda_layer
   (tests/unit/test_ops.c:576-634) on the reference's fixtures kda_layer1 / kda_layer8 and is
   compared at the manifest tolerance (atol 1e-5 + rtol 1e-4), and a two-call sequence with
   int8 weights against the oracle at the decode bar.
2. The per-row int8 draft format (K3_WI8, include/k3/k3.h:266-283), which the engine binds
   for its --draft-trunk hybrid decode (src/model/k3_bind.c:441): k3_kda_layer and
   k3hip_kda_layer_dev against the oracle's k3_kda_layer on the same int8 rows (the oracle
   is bit-identical to the reference's k3_matmul_q8 and k3_kda_layer, tests/test_oracle_ref.py).
   Tolerance: the decode bar, rtol 1e-4 and atol 1e-4 * rms (the GPU sums the int8 dot in
   double, the reference in float; the format has no exactness contract).
"""
from __future__ import annotations

import subprocess
from pathlib import Path

import numpy as np
import pytest

from conftest import REPO, assert_close, load_fixture, manifest_tol
import k3_oracle as ko
from k3_oracle import f32

pytestmark = pytest.mark.gpu

HARNESS = REPO / "oracle" / "_ref" / "dropin_harness"
NAMES = ("q", "k", "v", "q_conv", "k_conv", "v_conv", "f_a", "f_b", "A_log", "dt_bias", "b", "g", "o_norm", "o")


def rms(a):
    return float(np.sqrt(np.mean(np.asarray(a, np.float64) ** 2)))


def q8_layer(rng, hidden, H, D, K):
    P = H * D
    nrm = lambda *s: f32(rng.standard_normal(s) * 0.02)
    arrays = {"q": ko.q8_rows(nrm(P, hidden)), "k": ko.q8_rows(nrm(P, hidden)), "v": ko.q8_rows(nrm(P, hidden)),
              "g": ko.q8_rows(nrm(P, hidden)), "o": ko.q8_rows(nrm(hidden, P)), "f_a": ko.q8_rows(nrm(D, hidden)),
              "f_b": ko.q8_rows(f32(rng.standard_normal((P, D)) * 0.1)), "b": ko.q8_rows(nrm(H, hidden)),
              "q_conv": f32(rng.standard_normal((P, K)) * 0.5), "k_conv": f32(rng.standard_normal((P, K)) * 0.5),
              "v_conv": f32(rng.standard_normal((P, K)) * 0.5), "A_log": f32(rng.uniform(0, 1.5, H)),
              "dt_bias": f32(rng.standard_normal(P)), "o_norm": f32(1 + 0.1 * rng.standard_normal(D))}
    return ko.Weights(arrays, 2)


def run_harness(tmp: Path, W, cfg, xs, state0=None):
    """Write the case, run the C harness as a child process, read its outputs and states."""
    if not HARNESS.exists():
        pytest.fail(f"{HARNESS} is not built (oracle/Makefile 'ref', run by __graft_entry__.build())")
    for n in NAMES:
        np.ascontiguousarray(W.arrays[n]).tofile(tmp / f"{n}.bin")
    for i, x in enumerate(xs):
        f32(x).tofile(tmp / f"x{i}.bin")
    if state0 is not None:
        f32(state0).tofile(tmp / "state_in.bin")
    Ts = " ".join(str(x.shape[0]) for x in xs)
    (tmp / "case.txt").write_text(f"{cfg.hidden} {cfg.kda_heads} {cfg.kda_head_dim} {cfg.conv_k} {W.w.wdt} "
                                  f"{cfg.gate_lb!r} {cfg.rms_eps!r} {len(xs)} {Ts} {int(state0 is not None)}\n")
    print(f"dropin_harness on {tmp} (T = {Ts})", flush=True)
    r = subprocess.run([str(HARNESS), str(tmp)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, f"harness exit {r.returncode}: {r.stdout[-1000:]} {r.stderr[-2000:]}"
    outs = [np.fromfile(tmp / f"out{i}.bin", np.float32).reshape(x.shape[0], cfg.hidden) for i, x in enumerate(xs)]
    states = [np.fromfile(tmp / f"state{i}.bin", np.float32) for i in range(len(xs))]
    return outs, states


@pytest.mark.parametrize("fname", ["kda_layer1", "kda_layer8"])
def test_c_harness_on_reference_fixtures(gpu, tmp_path, fname):
    from test_oracle_golden import layer_cfg, layer_weights
    f = load_fixture(fname)
    cfg, W = layer_cfg(f), layer_weights(f)
    atol, rtol = manifest_tol()
    H, D = cfg.kda_heads, cfg.kda_head_dim
    T = f["in"].shape[1]
    (out,), (st,) = run_harness(tmp_path, W, cfg, [f["in"].reshape(T, -1)])
    assert_close(out, f["out"].reshape(T, -1), atol, rtol, f"C harness {fname} out")
    assert_close(st[:H * D * D], f["state_out"].ravel(), atol, rtol, f"C harness {fname} state")


def test_c_harness_int8_weights(gpu, tmp_path):
    rng = np.random.default_rng(0x4B334441 + 8)
    hidden, H, D, K = 256, 4, 64, 4
    W = q8_layer(rng, hidden, H, D, K)
    cfg = ko.make_cfg(hidden, H, D, K, -5.0, 1e-5)
    P = H * D
    s0 = f32(rng.standard_normal(P * D + 3 * P * (K - 1)) * 0.1)
    xs = [f32(rng.standard_normal((T, hidden))) for T in (12, 1)]
    outs, states = run_harness(tmp_path, W, cfg, xs, s0)
    st = s0.copy()
    for i, x in enumerate(xs):
        want = ko.kda_layer(ko.orc(), x, W, cfg, x.shape[0], st)
        assert_close(outs[i], want, 1e-4 * rms(want), 1e-4, f"C harness int8 call {i} out")
        assert_close(states[i], st, 1e-4 * rms(st), 1e-4, f"C harness int8 call {i} state")


@pytest.mark.parametrize("hidden,H,D,K,Ts", [(256, 4, 64, 4, (8, 1, 1)), (200, 2, 128, 3, (70, 1)),
                                             (128, 2, 16, 2, (3, 1))])
def test_dropin_int8_weights_vs_oracle(gpu, hidden, H, D, K, Ts):
    """k3_kda_layer on host pointers and k3hip_kda_layer_dev on device pointers, int8 rows
    (ragged when hidden is not a multiple of 4, so every row's scale sits unaligned), a
    prefill then decode steps with the state carried, against the oracle."""
    import torch
    rng = np.random.default_rng(0x4B334441 + hidden + D)
    W = q8_layer(rng, hidden, H, D, K)
    cfg = ko.make_cfg(hidden, H, D, K, -5.0, 1e-5)
    P = H * D
    nst = P * D + 3 * P * (K - 1)
    st_ref = np.zeros(nst, np.float32)
    st_host = np.zeros(nst, np.float32)
    dw = gpu.DeviceWeights(W.w, cfg)
    dst = torch.zeros(nst, device="cuda")
    for i, T in enumerate(Ts):
        x = f32(rng.standard_normal((T, hidden)))
        want = ko.kda_layer(ko.orc(), x, W, cfg, T, st_ref)
        out_h = np.zeros((T, hidden), np.float32)
        gpu.kda_layer_host(out_h, x, W.w, cfg, T, st_host)
        r = assert_close(out_h, want, 1e-4 * rms(want), 1e-4, f"int8 drop-in call {i} out")
        assert_close(st_host, st_ref, 1e-4 * rms(st_ref), 1e-4, f"int8 drop-in call {i} state")
        out_d = torch.zeros((T, hidden), device="cuda")
        dw.layer(out_d, torch.from_numpy(x).cuda(), dst, T)
        torch.cuda.synchronize()
        assert_close(out_d.cpu().numpy(), want, 1e-4 * rms(want), 1e-4, f"int8 device layer call {i} out")
        assert_close(dst.cpu().numpy(), st_ref, 1e-4 * rms(st_ref), 1e-4, f"int8 device layer call {i} state")
        print(f"int8 hidden={hidden} H={H} D={D} T={T}: worst {r:.3f}x of the 1e-4 bar", flush=True)
    # the bf16-only entry points refuse int8 weights
    with pytest.raises(gpu.K3HipError) as e:
        dw.layer_prefill(torch.zeros((4, hidden), device="cuda"), torch.zeros((4, hidden), device="cuda"), None, 4)
    assert e.value.code == gpu.EUNSUPPORTED
    dw.close()


@pytest.mark.parametrize("hidden,H,D,K,Ts", [(256, 2, 128, 4, (40, 1, 300)), (512, 4, 64, 3, (17, 64))])
def test_dropin_bf16_prefill_mfma_vs_oracle(gpu, hidden, H, D, K, Ts):
    """bf16 weights on prefills of T >= 16 take the MFMA projections (x split into bf16 hi + lo,
    the two fp32 products added); the layer stays at the reference's decode bar (rtol 1e-4,
    atol 1e-4 * rms) against the oracle's k3_kda_layer, on the host drop-in and on
    k3hip_kda_layer_dev, with the state carried through a T = 1 call in between."""
    import torch
    from test_gpu_layer_prefill import layer_weights
    rng = np.random.default_rng(0x4B334441 + 16 + hidden + D)
    W = layer_weights(rng, hidden, H, D, K)
    cfg = ko.make_cfg(hidden, H, D, K, -5.0, 1e-5)
    P = H * D
    nst = P * D + 3 * P * (K - 1)
    st_ref, st_host = np.zeros(nst, np.float32), np.zeros(nst, np.float32)
    dw = gpu.DeviceWeights(W.w, cfg, gpu.UPLOAD_DEV)
    dst = torch.zeros(nst, device="cuda")
    for i, T in enumerate(Ts):
        x = f32(rng.standard_normal((T, hidden)))
        want = ko.kda_layer(ko.orc(), x, W, cfg, T, st_ref)
        out_h = np.zeros((T, hidden), np.float32)
        gpu.kda_layer_host(out_h, x, W.w, cfg, T, st_host)
        r = assert_close(out_h, want, 1e-4 * rms(want), 1e-4, f"bf16 drop-in call {i} (T={T}) out")
        assert_close(st_host, st_ref, 1e-4 * rms(st_ref), 1e-4, f"bf16 drop-in call {i} state")
        out_d = torch.zeros((T, hidden), device="cuda")
        dw.layer(out_d, torch.from_numpy(x).cuda(), dst, T)
        torch.cuda.synchronize()
        assert_close(out_d.cpu().numpy(), want, 1e-4 * rms(want), 1e-4, f"bf16 device layer call {i} out")
        assert_close(dst.cpu().numpy(), st_ref, 1e-4 * rms(st_ref), 1e-4, f"bf16 device layer call {i} state")
        print(f"bf16 drop-in hidden={hidden} H={H} D={D} T={T}: worst {r:.3f}x of the 1e-4 bar", flush=True)
    dw.close()


@pytest.mark.parametrize("case", range(5))
def test_dropin_int8_random_vs_oracle(gpu, case):
    """Seeded random int8-weight layers through the host drop-in: hidden 64-520 (any width,
    so row scales sit at every byte alignment), H 1-4, D in {16, 32, 64, 128}, conv_k 1-4, a
    prefill of 1-90 tokens then one decode step, against the oracle at the 1e-4 bar."""
    rng = np.random.default_rng(0x4B334441 + 0x18 + case)
    hidden, H = int(rng.integers(64, 521)), int(rng.integers(1, 5))
    D, K, T = int(rng.choice([16, 32, 64, 128])), int(rng.integers(1, 5)), int(rng.integers(1, 91))
    print(f"hidden={hidden} H={H} D={D} K={K} T={T}", flush=True)
    W = q8_layer(rng, hidden, H, D, K)
    cfg = ko.make_cfg(hidden, H, D, K, -5.0, 1e-5)
    P = H * D
    st_ref = f32(rng.standard_normal(P * D + 3 * P * (K - 1)) * 0.1)
    st = st_ref.copy()
    for Tc in (T, 1):
        x = f32(rng.standard_normal((Tc, hidden)))
        want = ko.kda_layer(ko.orc(), x, W, cfg, Tc, st_ref)
        out = np.zeros((Tc, hidden), np.float32)
        gpu.kda_layer_host(out, x, W.w, cfg, Tc, st)
        assert_close(out, want, 1e-4 * rms(want), 1e-4, f"int8 random case {case} T={Tc} out")
        assert_close(st, st_ref, 1e-4 * rms(st_ref), 1e-4, f"int8 random case {case} T={Tc} state")
