# SPDX-License-Identifier: Apache-2.0
"""The bf16 full-layer prefill (k3hip_kda_layer_prefill): projections on bf16 MFMA through
hipBLASLt, the fused conv..recurrence, the epilogue and o_proj, against the CPU oracle's
k3_kda_layer on the same bf16 weights and the same bf16-rounded inputs.

The GPU projections accumulate in fp32 (the oracle in double) and the core runs on
split-bf16 MFMA; f_a reaches its GEMM as a bf16 hi/lo pair and the RMS-normalised epilogue
output as fp16 (against an exact fp16 copy of W_o), so no intermediate is rounded to bf16. Held to the chunked bf16-MFMA bar:
|got - want| <= 2e-3 * rms(want) + 2e-3 |want|, for the layer output and the carried state
(recurrent part and conv history), over two prefills in a row with the state carried.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_close
from test_oracle_ref import bf16
import k3_oracle as ko
from k3_oracle import f32

pytestmark = pytest.mark.gpu

TOL = 2e-3


def rms(a):
    return float(np.sqrt(np.mean(np.asarray(a, np.float64) ** 2)))


def bf16_to_f32(u):
    return (np.asarray(u, np.uint16).astype(np.uint32) << 16).view(np.float32)


def layer_weights(rng, hidden, H, D, K):
    P = H * D
    nrm = lambda *s: rng.standard_normal(s) * 0.02
    arrays = {"q": bf16(nrm(P, hidden)), "k": bf16(nrm(P, hidden)), "v": bf16(nrm(P, hidden)),
              "g": bf16(nrm(P, hidden)), "o": bf16(nrm(hidden, P)), "f_a": bf16(nrm(D, hidden)),
              "f_b": bf16(nrm(P, D)), "b": bf16(nrm(H, hidden)),
              "q_conv": f32(rng.standard_normal((P, K)) * 0.5),
              "k_conv": f32(rng.standard_normal((P, K)) * 0.5),
              "v_conv": f32(rng.standard_normal((P, K)) * 0.5),
              "A_log": f32(rng.uniform(0, 1.5, H)), "dt_bias": f32(rng.standard_normal(P)),
              "o_norm": f32(1 + 0.1 * rng.standard_normal(D))}
    return ko.Weights(arrays, 1)


@pytest.mark.parametrize("gemm", ["hipblaslt", "hand_written"])
@pytest.mark.parametrize("hidden,H,D,K,Ts", [(512, 4, 128, 4, (200, 77)), (256, 4, 64, 4, (1, 130)),
                                             (384, 3, 128, 2, (64, 1000))])
def test_layer_prefill_vs_oracle(gpu, hidden, H, D, K, Ts, gemm):
    """Both projection GEMM implementations (k3hip_set_projection_gemm) hold the bar."""
    gpu.set_projection_gemm(gpu.GEMM_HANDWRITTEN if gemm == "hand_written" else gpu.GEMM_HIPBLASLT)
    try:
        _layer_prefill_vs_oracle(gpu, hidden, H, D, K, Ts)
    finally:
        gpu.set_projection_gemm(gpu.GEMM_HIPBLASLT)


@pytest.mark.parametrize("case", range(12))
def test_layer_prefill_random_shapes_vs_oracle(gpu, case):
    """Seeded random layers: hidden a multiple of 64 in [128, 768], H 1-5, D 64 or 128,
    conv_k 1-4, a gate bound the chunked form takes, two calls carrying the state; even cases
    on hipBLASLt, odd ones on the hand-written GEMM."""
    rng = np.random.default_rng(0x4B334441 + 0x1A7E + case)
    hidden, H = 64 * int(rng.integers(2, 13)), int(rng.integers(1, 6))
    D, K = int(rng.choice([64, 128])), int(rng.integers(1, 5))
    Ts = (int(rng.integers(1, 401)), int(rng.integers(1, 401)))
    lb = float(np.float32(-rng.uniform(0.1, 5.3)))
    gpu.set_projection_gemm(gpu.GEMM_HANDWRITTEN if case % 2 else gpu.GEMM_HIPBLASLT)
    try:
        _layer_prefill_vs_oracle(gpu, hidden, H, D, K, Ts, lb, 0x4B334441 + 0x1A7E + case)
    finally:
        gpu.set_projection_gemm(gpu.GEMM_HIPBLASLT)


def _layer_prefill_vs_oracle(gpu, hidden, H, D, K, Ts, lb=-5.0, seed=None):
    import torch
    rng = np.random.default_rng(0x4B334441 + 2 + hidden + sum(Ts) if seed is None else seed)
    print(f"hidden={hidden} H={H} D={D} K={K} T={Ts} gate_lb={lb:.3f}", flush=True)
    W = layer_weights(rng, hidden, H, D, K)
    cfg = ko.make_cfg(hidden, H, D, K, lb, 1e-5)
    P = H * D
    nst = P * D + 3 * P * (K - 1)
    st_ref = np.zeros(nst, np.float32)
    dw = gpu.DeviceWeights(W.w, cfg)
    dst = torch.zeros(nst, device="cuda")
    for i, T in enumerate(Ts):
        xb = bf16(rng.standard_normal((T, hidden)))
        x = bf16_to_f32(xb)                     # the bf16-rounded inputs both sides see
        want = ko.kda_layer(ko.orc(), x, W, cfg, T, st_ref)
        dx = torch.from_numpy(x).cuda().to(torch.bfloat16)
        out = torch.full((T, hidden), float("nan"), device="cuda")
        dw.layer_prefill(out, dx, dst, T)
        torch.cuda.synchronize()
        got, gst = out.cpu().numpy(), dst.cpu().numpy()
        ro = assert_close(got, want, TOL * rms(want), TOL, f"layer T={T} out")
        rs = assert_close(gst[:P * D], st_ref[:P * D], TOL * rms(st_ref[:P * D]), TOL, f"layer T={T} S")
        # the conv history holds the last projected inputs: fp32 vs double accumulation
        if K > 1:
            assert_close(gst[P * D:], st_ref[P * D:], 1e-5 * rms(st_ref[P * D:]), 1e-5,
                         f"layer T={T} conv history")
        print(f"hidden={hidden} H={H} D={D} K={K} call {i} T={T}: worst {ro:.3f}x (out) / "
              f"{rs:.3f}x (S) of the 2e-3 bar")
    dw.close()


def test_layer_prefill_fp32_io_and_refusals(gpu):
    import torch
    rng = np.random.default_rng(11)
    hidden, H, D, K, T = 256, 2, 64, 4, 70
    W = layer_weights(rng, hidden, H, D, K)
    cfg = ko.make_cfg(hidden, H, D, K, -5.0, 1e-5)
    x = bf16_to_f32(bf16(rng.standard_normal((T, hidden))))
    want = ko.kda_layer(ko.orc(), x, W, cfg, T, None)
    dw = gpu.DeviceWeights(W.w, cfg)
    out = torch.zeros((T, hidden), device="cuda", dtype=torch.bfloat16)
    dw.layer_prefill(out, torch.from_numpy(x).cuda(), None, T)     # fp32 in, bf16 out, no state
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert_close(got, want, 2 * TOL * rms(want), 2 * TOL, "fp32 in / bf16 out")   # + bf16 output rounding
    dw.close()
    # fp32 weights and the softplus gate stay on k3hip_kda_layer_dev
    W32 = ko.Weights({n: (bf16_to_f32(a) if a.dtype == np.uint16 else a) for n, a in W.arrays.items()}, 0)
    for w_, c_ in ((W32, cfg), (W, ko.make_cfg(hidden, H, D, K, 0.0, 1e-5))):
        d2 = gpu.DeviceWeights(w_.w, c_)
        with pytest.raises(gpu.K3HipError) as e:
            d2.layer_prefill(torch.zeros((T, hidden), device="cuda"), torch.from_numpy(x).cuda(), None, T)
        assert e.value.code == 3
        d2.close()
