# SPDX-License-Identifier: Apache-2.0
"""k3hip_kda_decode_step, one launch per decode token for K1 (T = 1) + K3 + K4, against the
oracle's orc_kda_core run one token at a time per sequence (conv + SiLU, L2, beta, decay,
the k3_kda_step recurrence, RMSNorm then gate: src/core/k3_ops.c:888-947 at T = 1), three
steps with the state and conv history carried in place. Shapes from the batch-64 decode
configuration (H=32, D=128) down to D=16 with conv_k 1-4, both input and output dtypes, the
bounded and the softplus gate.

Tolerance: the decode bar, rtol 1e-4 and atol 1e-4 * rms(ref) on fp32 outputs and on the
state; a bf16 y adds one bf16 ulp (rtol 2^-7: a value within the kernel's fp32 error of a
rounding midpoint may round either way). The same step through the three launches
(k3hip_kda_prep, k3hip_kda_decode, k3hip_kda_epilogue) is held to the same bar."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_close
import k3_oracle as ko
from k3_oracle import f32

pytestmark = pytest.mark.gpu


def rms(a):
    return float(np.sqrt(np.mean(np.asarray(a, np.float64) ** 2)))


@pytest.mark.parametrize("B,H,D,K,in_bf16,g_bf16,y_bf16,lb", [
    (64, 32, 128, 4, True, True, True, -5.0),
    (3, 2, 64, 3, False, False, False, -5.0),
    (5, 4, 32, 1, False, True, False, 0.0),     # conv_k 1 (no history), softplus gate
    (2, 3, 16, 2, True, False, True, -5.0),
    (9, 1, 128, 4, False, False, False, -2.0),
])
def test_decode_step_vs_oracle(gpu, B, H, D, K, in_bf16, g_bf16, y_bf16, lb):
    import torch
    rng = np.random.default_rng(0x4B334441 + 1 + B * 7 + H * 3 + D + K)
    P = H * D
    nh = K - 1
    W_arrays = {"q_conv": f32(rng.standard_normal((P, K)) * 0.5), "k_conv": f32(rng.standard_normal((P, K)) * 0.5),
                "v_conv": f32(rng.standard_normal((P, K)) * 0.5), "A_log": f32(rng.uniform(0, 1.5, H)),
                "dt_bias": f32(rng.standard_normal(P)), "o_norm": f32(1 + 0.1 * rng.standard_normal(D))}
    for n in ("q", "k", "v", "g", "f_a", "f_b", "b", "o"):
        W_arrays[n] = np.zeros((1, 1), np.float32)
    W = ko.Weights(W_arrays, 0)
    cfg = ko.make_cfg(8, H, D, K, lb, 1e-5)
    S0 = f32(rng.standard_normal((B, H, D, D)) * 0.1)
    C0 = f32(rng.standard_normal((B, 3 * P * nh)))
    ref_st = [np.concatenate([S0[b].ravel(), C0[b]]) for b in range(B)]
    cu = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    dev = {n: cu(W_arrays[n]) for n in ("q_conv", "k_conv", "v_conv", "A_log", "dt_bias", "o_norm")}
    S, cs = cu(S0), cu(C0) if nh else None
    S3, cs3 = cu(S0), cu(C0) if nh else None   # the three-launch path, per sequence
    bf = torch.bfloat16
    qs = float(np.float32(1) / np.sqrt(np.float32(D)))
    for step in range(3):
        raw = [f32(rng.standard_normal((B, P))) for _ in range(3)]
        if in_bf16:   # what the kernel sees: the bf16-rounded values
            raw = [torch.from_numpy(r).to(bf).float().numpy() for r in raw]
        z = f32(rng.standard_normal((B, P)) * 0.5)
        bl = f32(rng.standard_normal((B, H)))
        gate = f32(rng.standard_normal((B, P)))
        if g_bf16:
            gate = torch.from_numpy(gate).to(bf).float().numpy()
        want = np.concatenate([ko.core(raw[0][b:b + 1], raw[1][b:b + 1], raw[2][b:b + 1], z[b:b + 1], bl[b:b + 1],
                                       gate[b:b + 1], W, cfg, 1, ref_st[b]) for b in range(B)])
        dq, dk, dv = (cu(r).to(bf) if in_bf16 else cu(r) for r in raw)
        dg = cu(gate).to(bf) if g_bf16 else cu(gate)
        y = torch.full((B, P), float("nan"), device="cuda", dtype=bf if y_bf16 else torch.float32)
        gpu.kda_decode_step(dq, dk, dv, cu(z), cu(bl), dg, dev["q_conv"], dev["k_conv"], dev["v_conv"],
                            dev["A_log"], dev["dt_bias"], dev["o_norm"], cs, S, y, H, D, K, lb, 1e-5, qs)
        # the same token through k3hip_kda_prep + k3hip_kda_decode + k3hip_kda_epilogue
        q1, k1, v1, g1, a1 = (torch.zeros((B, P), device="cuda") for _ in range(5))
        b1 = torch.zeros((B, H), device="cuda")
        for b in range(B):
            csb = cs3[b] if nh else None
            gpu.kda_prep(dq[b:b + 1], dk[b:b + 1], dv[b:b + 1], cu(z[b:b + 1]), cu(bl[b:b + 1]), dev["q_conv"],
                         dev["k_conv"], dev["v_conv"], dev["A_log"], dev["dt_bias"], csb, q1[b:b + 1], k1[b:b + 1],
                         v1[b:b + 1], g1[b:b + 1], a1[b:b + 1], b1[b:b + 1], H, D, K, lb)
        o3 = torch.zeros((B, H, D), device="cuda")
        gpu.kda_decode(S3, o3, q1.view(B, H, D), k1.view(B, H, D), v1.view(B, H, D), a1.view(B, H, D), b1, qs)
        y3 = torch.zeros((B, P), device="cuda")
        gpu.kda_epilogue(o3.view(B, P), dg, dev["o_norm"], y3, H, D, 1e-5)
        torch.cuda.synchronize()
        got = y.float().cpu().numpy()
        yr = 2.0 ** -7 + 1e-4 if y_bf16 else 1e-4
        r = assert_close(got, want, 1e-4 * rms(want), yr, f"decode step {step} y")
        r3 = assert_close(y3.cpu().numpy(), want, 1e-4 * rms(want), 1e-4, f"three-launch step {step} y")
        gS = S.cpu().numpy()
        for b in range(B):
            assert_close(gS[b].ravel(), ref_st[b][:H * D * D], 1e-4 * rms(ref_st[b][:H * D * D]), 1e-4,
                         f"decode step {step} seq {b} S")
            if nh:   # the history holds the inputs themselves: bitwise
                assert np.array_equal(cs[b].cpu().numpy(), ref_st[b][H * D * D:]), f"step {step} seq {b} conv history"
        print(f"B={B} H={H} D={D} K={K} step {step}: worst {r:.3f}x (one launch) / {r3:.3f}x (three) of the bar",
              flush=True)


def test_decode_step_refusals(gpu):
    import torch
    z = torch.zeros(64, device="cuda")
    with pytest.raises(gpu.K3HipError) as e:   # conv_k > 1 needs the conv history
        gpu.kda_decode_step(z[None], z[None], z[None], z[None], z[None, :1], z[None], z, z, z, z[:1], z, z, None,
                            torch.zeros((1, 1, 64, 64), device="cuda"), torch.zeros((1, 64), device="cuda"),
                            1, 64, 4, -5.0, 1e-5, 0.125)
    assert e.value.code == gpu.EINVAL
    with pytest.raises(gpu.K3HipError) as e:   # D outside the kernel set
        gpu.kda_decode_step(z[None], z[None], z[None], z[None], z[None, :1], z[None], z, z, z, z[:1], z, z, None,
                            torch.zeros((1, 1, 48, 48), device="cuda"), torch.zeros((1, 48), device="cuda"),
                            1, 48, 1, -5.0, 1e-5, 0.125)
    assert e.value.code == gpu.EUNSUPPORTED


@pytest.mark.parametrize("case", range(8))
def test_decode_step_random_vs_oracle(gpu, case):
    """Seeded random decode steps: B 1-70, H 1-6, D in {16, 32, 64, 128}, conv_k 1-4, gate bound
    -0.1 to -5.3 or the softplus gate, either input, gate and output dtype, two steps."""
    rng = np.random.default_rng(0x4B334441 + 0x5E9 + case)
    B, H = int(rng.integers(1, 71)), int(rng.integers(1, 7))
    D, K = int(rng.choice([16, 32, 64, 128])), int(rng.integers(1, 5))
    lb = 0.0 if rng.random() < 0.25 else -float(rng.uniform(0.1, 5.3))
    flags = [bool(b) for b in rng.integers(0, 2, 3)]
    print(f"B={B} H={H} D={D} K={K} lb={lb:.3f} bf16 in/gate/y={flags}", flush=True)
    test_decode_step_vs_oracle(gpu, B, H, D, K, *flags, lb)
