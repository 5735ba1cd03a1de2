# SPDX-License-Identifier: Apache-2.0
"""k3hip_kda_layer_decode_noalloc, the decode step that allocates nothing (its scratch is a
fixed device array inside the library), against k3hip_kda_layer_decode through the C ABI:
outputs and updated states bit-identical on two calls in a row, the second with fewer
sequences (the array keeps the first call's contents); a batch beyond the array's size is
refused with K3HIP_EINVAL and leaves out and the states untouched."""
from __future__ import annotations

import numpy as np
import pytest

from test_gpu_layer_prefill import layer_weights
import k3_oracle as ko
from k3_oracle import f32

pytestmark = pytest.mark.gpu


def test_noalloc_decode_matches_allocating_decode(gpu):
    import torch
    hidden, H, D, K = 512, 4, 128, 4
    rng = np.random.default_rng(0x4B334441 + 123)
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
    # too many sequences for the fixed scratch (about 12.8 KB per sequence at this width
    # against 64 MiB): refused before any launch
    B = 20000
    x = torch.zeros((B, hidden), device="cuda")
    out = torch.full((B, hidden), 3.0, device="cuda")
    st = torch.full((B, stride), 5.0, device="cuda")
    with pytest.raises(gpu.K3HipError) as e:
        dw.layer_decode_noalloc(out, x, st, stride)
    assert e.value.code == gpu.EINVAL and "no-allocation" in str(e.value)
    torch.cuda.synchronize()
    assert (out == 3.0).all() and (st == 5.0).all()
    dw.close()
