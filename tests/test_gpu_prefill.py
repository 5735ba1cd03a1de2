# SPDX-License-Identifier: Apache-2.0
"""K1 + K2 fused (k3hip_kda_prefill) for bf16 and fp32 conv inputs, through the C ABI.

1. Bit-identical to k3hip_kda_prep followed by k3hip_kda_chunk on the same device inputs:
   the output, the final state and the outgoing conv history, over ragged T, every conv
   size, with and without incoming history, and with workgroups whose item ranges cross
   heads (H * chunks not a multiple of the workgroup count); both input dtypes.
2. Against the CPU oracle (prep, then the sequential recurrence, on the inputs the GPU
   sees) at the chunked bar: |got - want| <= 2e-3 * rms(want) + 2e-3 |want|; also over 24
   seeded random shapes, gate bounds, dtypes and pass sizes.
3. Shapes outside the fused kernel are refused with K3HIP_EUNSUPPORTED / K3HIP_EINVAL.
4. A workspace for fewer chunks than the sequence runs it in passes with the same bits (the
   conv history carried in conv_state, or in the workspace when conv_state is NULL).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_close, worst_ratio
from test_gpu_kernels import dev, host, prep_case
import k3_oracle as ko
from k3_oracle import f32

pytestmark = pytest.mark.gpu

LB = -5.0
TOL = 2e-3


def rms(a):
    return float(np.sqrt(np.mean(np.asarray(a, np.float64) ** 2)))


def setup(rng, T, H, D, K, with_history, fp32=False):
    import torch
    P = H * D
    W, ins, z, bl = prep_case(rng, T, H, D, K)
    a = W.arrays
    d = {
        "ins": [dev(x, torch.float32 if fp32 else torch.bfloat16) for x in ins], "z": dev(z), "bl": dev(bl),
        "conv": [dev(a["q_conv"]), dev(a["k_conv"]), dev(a["v_conv"])],
        "A_log": dev(a["A_log"]), "dt": dev(a["dt_bias"]),
    }
    cs = f32(rng.standard_normal(3 * P * (K - 1))) if (with_history and K > 1) else None
    S0 = f32(rng.standard_normal((H, D, D)) * 0.1)
    return W, ins, z, bl, d, cs, S0


def run_two_step(gpu, d, cs, S0, T, H, D, K, qs):
    import torch
    P = H * D
    outs = [torch.zeros((T, P), device="cuda") for _ in range(5)]
    beta = torch.zeros((T, H), device="cuda")
    dcs = dev(cs) if cs is not None else None
    gpu.kda_prep(*d["ins"], d["z"], d["bl"], *d["conv"], d["A_log"], d["dt"], dcs, *outs, beta,
                 H, D, K, LB)
    S = dev(S0)
    o = torch.full((T, P), float("nan"), device="cuda")
    gpu.kda_chunk(outs[0], outs[1], outs[2], outs[3], beta, S, o, H, D, qs)
    torch.cuda.synchronize()
    return o, S, dcs


def run_fused(gpu, d, cs, S0, T, H, D, K, qs, workspace=True):
    import torch
    P = H * D
    dcs = dev(cs) if cs is not None else None
    S = dev(S0)
    o = torch.full((T, P), float("nan"), device="cuda")
    ws = None
    if workspace:
        ws = torch.empty(max(1, gpu.kda_chunk_workspace(T, H, D)), dtype=torch.uint8, device="cuda")
    gpu.kda_prefill(*d["ins"], d["z"], d["bl"], *d["conv"], d["A_log"], d["dt"], dcs, S, o, H, D,
                    K, LB, qs, ws)
    torch.cuda.synchronize()
    return o, S, dcs


@pytest.mark.parametrize("T,H,D,K,hist,fp32", [
    (1, 2, 128, 4, True, False), (2, 1, 64, 4, True, False), (3, 2, 128, 3, True, False),
    (64, 2, 128, 4, False, False), (65, 3, 128, 2, True, False), (130, 2, 64, 1, False, False),
    (200, 2, 64, 3, True, False), (1000, 3, 128, 4, True, False), (1000, 20, 64, 4, True, False),
    (4096 + 17, 5, 128, 4, True, False), (16384, 4, 128, 4, False, False),
    (1, 2, 128, 4, True, True), (3, 2, 64, 3, True, True), (200, 2, 64, 4, True, True),
    (1000, 3, 128, 4, True, True), (4096 + 17, 5, 128, 2, False, True)])
def test_prefill_bitwise_vs_prep_then_chunk(gpu, T, H, D, K, hist, fp32):
    import torch
    rng = np.random.default_rng(0x4B334441 + 7 + T + H + D + K)
    qs = float(np.float32(1) / np.sqrt(np.float32(D)))
    _, _, _, _, d, cs, S0 = setup(rng, T, H, D, K, hist, fp32)
    oa, Sa, csa = run_two_step(gpu, d, cs, S0, T, H, D, K, qs)
    ob, Sb, csb = run_fused(gpu, d, cs, S0, T, H, D, K, qs)
    print(f"T={T} H={H} D={D} K={K} history={hist} fp32={fp32}: max |do| "
          f"{(oa - ob).abs().max().item():.3g}, max |dS| {(Sa - Sb).abs().max().item():.3g}")
    assert torch.equal(oa, ob), "fused output differs from prep + chunk"
    assert torch.equal(Sa, Sb), "fused final state differs from prep + chunk"
    if csa is not None:
        assert torch.equal(csa, csb), "fused outgoing conv history differs"


@pytest.mark.parametrize("T,H,D,K,hist,fp32,chunks", [
    (1000, 3, 128, 4, True, False, 3),    # 16 chunks in passes of 3, a last pass of 40 tokens
    (193, 2, 128, 4, True, False, 3),     # a last pass of 1 token: older history slots shift
    (300, 2, 64, 3, False, True, 2),      # no caller history: it lives in the workspace
    (130, 2, 128, 1, False, False, 1)])   # conv_k 1: no history at all
def test_prefill_in_passes_bitwise(gpu, T, H, D, K, hist, fp32, chunks):
    """A workspace for fewer chunks than the sequence: passes of whole chunks, the same bits."""
    import torch
    rng = np.random.default_rng(0x4B334441 + 11 + T + D + K)
    qs = float(np.float32(1) / np.sqrt(np.float32(D)))
    P = H * D
    _, _, _, _, d, cs, S0 = setup(rng, T, H, D, K, hist, fp32)
    oa, Sa, csa = run_fused(gpu, d, cs, S0, T, H, D, K, qs)
    nbytes = gpu.kda_chunk_workspace(64 * chunks, H, D)
    hist_bytes = (3 * P * (K - 1) * 4 + 255) // 256 * 256 if (cs is None and K > 1) else 0
    ws = torch.empty(nbytes + hist_bytes, dtype=torch.uint8, device="cuda")
    dcs = dev(cs) if cs is not None else None
    S = dev(S0)
    ob = torch.full((T, P), float("nan"), device="cuda")
    args = lambda w: (*d["ins"], d["z"], d["bl"], *d["conv"], d["A_log"], d["dt"], dcs, S, ob, H, D, K,
                      LB, qs, w)
    gpu.kda_prefill(*args(ws))
    torch.cuda.synchronize()
    assert torch.equal(oa, ob), "output in passes differs from one pass"
    assert torch.equal(Sa, S), "final state in passes differs from one pass"
    if csa is not None:
        assert torch.equal(csa, dcs), "outgoing conv history in passes differs from one pass"
    # less than one chunk (and the history it needs) is refused
    small = torch.empty(gpu.kda_chunk_workspace(64, H, D) + hist_bytes - 16, dtype=torch.uint8, device="cuda")
    with pytest.raises(gpu.K3HipError) as e:
        gpu.kda_prefill(*args(small))
    assert e.value.code == 1


@pytest.mark.parametrize("T,H,D,K,fp32", [(1, 2, 128, 4, False), (70, 2, 64, 2, False),
                                         (300, 3, 128, 4, False), (1000, 2, 64, 3, False),
                                         (70, 2, 128, 4, True), (1000, 2, 64, 3, True)])
def test_prefill_vs_oracle(gpu, T, H, D, K, fp32):
    rng = np.random.default_rng(0x4B334441 + 8 + T + D + K)
    qs = float(np.float32(1) / np.sqrt(np.float32(D)))
    cfg = ko.make_cfg(8, H, D, K, LB, 1e-5)
    W, ins, z, bl, d, cs, S0 = setup(rng, T, H, D, K, True, fp32)
    ins_bf = [host(x) for x in d["ins"]]              # the values the GPU sees
    cs_ref = cs.copy() if cs is not None else None
    q, k, v, g, al, beta = ko.prep(*ins_bf, z, bl, W, cfg, T, cs_ref)
    S_ref = S0.copy()
    o_ref = ko.recurrence(S_ref, q, k, v, al, beta, H, D, qs, nthreads=4)
    o, S, dcs = run_fused(gpu, d, cs, S0, T, H, D, K, qs, workspace=False)
    o, S = host(o), host(S)
    ro = assert_close(o, o_ref, TOL * rms(o_ref), TOL, f"prefill T={T} o")
    rs = assert_close(S, S_ref, TOL * rms(S_ref), TOL, f"prefill T={T} S")
    to = worst_ratio(o, o_ref, 1e-4 * rms(o_ref), 1e-4)
    print(f"T={T} H={H} D={D} K={K}: worst {ro:.4f}x / {rs:.4f}x of the 2e-3 bar; {to:.3f}x of 1e-4 (o)")
    # regression guard 20x tighter than the bar: the split-bf16 products have stayed within
    # the decode-grade 1e-4 bar at these sizes (worst seen 0.54x at T = 1000)
    assert to <= 1.0, f"prefill T={T}: {to:.3f}x of the 1e-4 regression guard"
    if cs is not None:
        assert np.array_equal(host(dcs), cs_ref), "outgoing conv history"


@pytest.mark.parametrize("case", range(24))
def test_prefill_random_shapes_vs_oracle(gpu, case):
    """Seeded random shapes against the oracle at the chunked bar: T in [1, 700], H in [1, 6],
    D 64 or 128, conv_k 1-4, any gate bound the chunked form takes, either input dtype, with
    or without incoming history, and every third case in passes over a random workspace."""
    import torch
    rng = np.random.default_rng(0x4B334441 + 0x5EED + case)
    T, H = int(rng.integers(1, 701)), int(rng.integers(1, 7))
    D, K = int(rng.choice([64, 128])), int(rng.integers(1, 5))
    hist, fp32 = bool(rng.integers(0, 2)), bool(rng.integers(0, 2))
    lb = float(np.float32(-rng.uniform(0.1, 5.3)))
    qs = float(np.float32(1) / np.sqrt(np.float32(D)))
    P = H * D
    W, ins, z, bl, d, cs, S0 = setup(rng, T, H, D, K, hist, fp32)
    cfg = ko.make_cfg(8, H, D, K, lb, 1e-5)
    ins_bf = [host(x) for x in d["ins"]]
    cs_ref = cs.copy() if cs is not None else None
    q, k, v, g, al, beta = ko.prep(*ins_bf, z, bl, W, cfg, T, cs_ref)
    S_ref = S0.copy()
    o_ref = ko.recurrence(S_ref, q, k, v, al, beta, H, D, qs, nthreads=4)
    nch = (T + 63) // 64
    chunks = int(rng.integers(1, nch + 1)) if case % 3 == 2 else nch
    hist_bytes = (3 * P * (K - 1) * 4 + 255) // 256 * 256 if (cs is None and K > 1 and chunks < nch) else 0
    ws = torch.empty(gpu.kda_chunk_workspace(64 * chunks, H, D) + hist_bytes, dtype=torch.uint8, device="cuda")
    dcs = dev(cs) if cs is not None else None
    S = dev(S0)
    o = torch.full((T, P), float("nan"), device="cuda")
    print(f"case {case}: T={T} H={H} D={D} K={K} history={hist} fp32={fp32} gate_lb={lb:.3f} "
          f"chunks per pass {chunks} of {nch}", flush=True)
    gpu.kda_prefill(*d["ins"], d["z"], d["bl"], *d["conv"], d["A_log"], d["dt"], dcs, S, o, H, D, K,
                    lb, qs, ws)
    torch.cuda.synchronize()
    o, S = host(o), host(S)
    ro = assert_close(o, o_ref, TOL * rms(o_ref), TOL, f"case {case} o")
    rs = assert_close(S, S_ref, TOL * rms(S_ref), TOL, f"case {case} S")
    print(f"  worst {ro:.4f}x (o) / {rs:.4f}x (S) of the 2e-3 bar")
    if cs is not None:
        assert np.array_equal(host(dcs), cs_ref), "outgoing conv history"


def test_prefill_refuses_other_shapes(gpu):
    import torch
    rng = np.random.default_rng(9)
    T, H, D, K = 10, 1, 64, 4
    _, _, _, _, d, _, S0 = setup(rng, T, H, D, K, False)
    S, o = dev(S0), torch.zeros((T, H * D), device="cuda")
    args = lambda ins, lb=LB, Dx=D: (*ins, d["z"], d["bl"], *d["conv"], d["A_log"], d["dt"], None,
                                     S, o, H, Dx, K, lb, 0.125)
    with pytest.raises(gpu.K3HipError) as e:          # unbounded (softplus) gate
        gpu.kda_prefill(*args(d["ins"], lb=0.0))
    assert e.value.code == 3
    with pytest.raises(gpu.K3HipError) as e:          # gate bound past the exponent range
        gpu.kda_prefill(*args(d["ins"], lb=-6.0))
    assert e.value.code == 3
    with pytest.raises(gpu.K3HipError) as e:          # head size
        gpu.kda_prefill(*args(d["ins"], Dx=32))
    assert e.value.code == 3
    odd = [torch.zeros(T * H * D + 8, dtype=torch.bfloat16, device="cuda")[1:1 + T * H * D].view(T, H * D)
           for _ in range(3)]
    with pytest.raises(gpu.K3HipError) as e:          # misaligned rows
        gpu.kda_prefill(*args(odd))
    assert e.value.code == 1
