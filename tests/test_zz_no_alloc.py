# SPDX-License-Identifier: Apache-2.0
"""k3hip_kda_layer_decode_noalloc, the decode step that allocates nothing (its scratch is a
fixed device array inside the library), against k3hip_kda_layer_decode through the C ABI:
outputs and updated states bit-identical on two calls in a row, the second with fewer
sequences (the array keeps the first call's contents); a batch beyond the array's size is
refused with K3HIP_EINVAL and leaves out and the states untouched.

Three widths cover every scratch path of the step: hidden 512 with 4 heads (every decode
GEMV one K-range), hidden 512 with 32 heads (o_proj in 16 K-ranges: the partial planes in
the scratch and a reduction launch) and hidden 7168 with 2 heads (q/k/v/f_a/b and the gate
in 16 K-ranges, so the first GEMV needs its reduction and runs as two launches; o_proj in
two K-ranges added into the output by atomics). The no-allocation call refuses any step that
would allocate, so a scratch sized too small fails here instead of allocating."""
from __future__ import annotations

import numpy as np
import pytest

from test_gpu_layer_prefill import layer_weights
import k3_oracle as ko
from k3_oracle import f32

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("hidden,H", [(512, 4), (512, 32), (7168, 2)])
def test_noalloc_decode_matches_allocating_decode(gpu, hidden, H):
    import torch
    D, K = 128, 4
    rng = np.random.default_rng(0x4B334441 + 123 + hidden + H)
    W = layer_weights(rng, hidden, H, D, K)
    cfg = ko.make_cfg(hidden, H, D, K, -5.0, 1e-5)
    P = H * D
    kper = P * D + 3 * P * (K - 1)
    stride = kper + 8
    dw = gpu.DeviceWeights(W.w, cfg, gpu.UPLOAD_DEV | gpu.UPLOAD_DECODE)
    for call, B in enumerate((19, 6)):
        init = torch.from_numpy(f32(rng.standard_normal((B, stride)) * 0.05)).cuda()
        sa, sb = init.clone(), init.clone()
        x = torch.from_numpy(f32(rng.standard_normal((B, hidden)))).cuda()
        oa = torch.full((B, hidden), float("nan"), device="cuda")
        ob = torch.full((B, hidden), float("nan"), device="cuda")
        dw.layer_decode(oa, x, sa, stride)
        dw.layer_decode_noalloc(ob, x, sb, stride)
        torch.cuda.synchronize()
        print(f"call {call} B={B}: max |dout| {(oa - ob).abs().max().item():.3g}", flush=True)
        assert torch.isfinite(oa).all()
        assert torch.equal(oa, ob), f"call {call}: outputs differ"
        assert torch.equal(sa, sb), f"call {call}: states differ"
    # too many sequences for the fixed 16 MiB scratch (the projections alone take more than
    # 12 P bytes per sequence): refused before any launch
    B = (16 << 20) // (12 * P) + 1
    x = torch.zeros((B, hidden), device="cuda")
    out = torch.full((B, hidden), 3.0, device="cuda")
    st = torch.full((B, stride), 5.0, device="cuda")
    with pytest.raises(gpu.K3HipError) as e:
        dw.layer_decode_noalloc(out, x, st, stride)
    assert e.value.code == gpu.EINVAL and "no-allocation" in str(e.value)
    torch.cuda.synchronize()
    assert (out == 3.0).all() and (st == 5.0).all()
    dw.close()
