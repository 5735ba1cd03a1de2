# SPDX-License-Identifier: Apache-2.0
"""The hand-written MFMA projection GEMM (k3hip_proj_gemm, kimi-k3-in-c_amd/csrc/kda_mm.hip)
against a float64 product of the same bf16 / fp16 operands.

It stands for the reference's per-token k3_mmw -> k3_matmul_bf16 (src/core/k3_ops.c:1122-1227)
over T tokens. fp32 accumulation in another order than the reference's double sum: each
output is held to |got - ref| <= 2^-16 * sum_k |a_k b_k| (plus the output format's own
rounding for bf16 / fp16 outputs), far inside what the 2e-3 layer bar needs. Ragged M and N
(tile edges), fp16 operands, every output format, run-twice bit identity, and refusals.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def check(got, a, b, out_rel):
    import torch
    ad, bd = a.double(), b.double()
    ref = ad @ bd.t()
    mag = ad.abs() @ bd.abs().t()
    err = (got.double() - ref).abs()
    bound = 2.0 ** -16 * mag + out_rel * ref.abs() + 1e-30
    worst = (err / bound).max().item()
    assert torch.isfinite(got).all(), "non-finite output"
    return worst


@pytest.mark.parametrize("M,N,K,ab,out", [
    (1, 1, 64, "bf16", "f32"), (255, 257, 64, "bf16", "f32"), (1000, 520, 256, "bf16", "f32"),
    (300, 160, 4096, "bf16", "f32"), (513, 384, 128, "f16", "f32"), (777, 1000, 192, "bf16", "bf16"),
    (256, 768, 512, "bf16", "f16"), (1024, 4096, 4096, "bf16", "f32"), (640, 2048, 4096, "f16", "bf16"),
    # more tiles than CUs: the persistent grid, its load stream running across tiles
    (4352, 4352, 256, "bf16", "f32"), (4608, 4352, 128, "f16", "f16")])
def test_proj_gemm_vs_float64(gpu, M, N, K, ab, out):
    import torch
    g = torch.Generator(device="cuda").manual_seed(M * 7 + N * 3 + K)
    dt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}
    a = torch.randn((M, K), device="cuda", generator=g).to(dt[ab])
    b = (torch.randn((N, K), device="cuda", generator=g) * 0.05).to(dt[ab])
    c = torch.full((M, N), float("nan"), device="cuda", dtype=dt[out])
    gpu.proj_gemm(a, b, c)
    torch.cuda.synchronize()
    rel = {"f32": 0.0, "bf16": 2.0 ** -8, "f16": 2.0 ** -11}[out]
    w = check(c, a, b, rel)
    print(f"{M}x{N}x{K} {ab}->{out}: worst {w:.3f}x of the bound")
    assert w <= 1.0


def test_proj_gemm_strided_and_bitwise(gpu):
    """Leading dimensions wider than the matrices (a column slice of a wider weight, an
    output written into a wider row), and two runs give the same bits."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(5)
    M, N, K = 700, 300, 320
    abig = torch.randn((M, K + 64), device="cuda", generator=g).bfloat16()
    bbig = (torch.randn((N, K + 128), device="cuda", generator=g) * 0.05).bfloat16()
    a, b = abig[:, :K], bbig[:, :K]
    cbig = torch.full((M, N + 40), -7.0, device="cuda")
    c = cbig[:, 8:8 + N]
    gpu.proj_gemm(a, b, c)
    torch.cuda.synchronize()
    assert check(c, a, b, 0.0) <= 1.0
    assert (cbig[:, :8] == -7.0).all() and (cbig[:, 8 + N:] == -7.0).all(), "wrote outside its columns"
    c2 = torch.empty((M, N), device="cuda")
    gpu.proj_gemm(a, b, c2)
    torch.cuda.synchronize()
    assert torch.equal(c.contiguous(), c2), "two runs differ"


def test_proj_gemm_refusals(gpu):
    import torch
    a = torch.zeros((64, 96), device="cuda", dtype=torch.bfloat16)
    b = torch.zeros((64, 96), device="cuda", dtype=torch.bfloat16)
    c = torch.zeros((64, 64), device="cuda")
    with pytest.raises(gpu.K3HipError) as e:          # K not a multiple of 64
        gpu.proj_gemm(a, b, c)
    assert e.value.code == 3
    import ctypes as C
    L = gpu.lib()
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    pa, pb, pc = (C.c_void_p(t.data_ptr()) for t in (a, b, c))
    assert L.k3hip_proj_gemm(64, 64, 64, gpu.F32, pa, 96, pb, 96, pc, gpu.F32, 64, st) == gpu.EINVAL
    assert L.k3hip_proj_gemm(64, 64, 64, gpu.BF16, pa, 93, pb, 96, pc, gpu.F32, 64, st) == gpu.EUNSUPPORTED
    assert L.k3hip_proj_gemm(64, 64, 64, gpu.BF16, pa, 96, pb, 96, pc, gpu.F32, 32, st) == gpu.EINVAL
