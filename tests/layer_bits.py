# SPDX-License-Identifier: Apache-2.0
"""Helper for tests/test_gpu_determinism.py (not a test module): runs seeded layer work on
cuda:0 and prints one sha256 line of every output and state byte, so two fresh processes
can be compared. The work covers every summation path of the layer entry points:

- the bf16 layer prefill with hipBLASLt's GEMMs and again with the hand-written GEMMs
  (split-K f_a / b planes summed by an ordered reduction);
- the batched decode layer at hidden 512, H=4 (every decode GEMV one K-range), at hidden 512,
  H=32 (o_proj in 16 K-ranges summed by the reduction kernel) and at hidden 7168, H=2
  (o_proj in two K-ranges added into the output by float atomics; the gate and q/k/v GEMVs
  in 16 K-ranges);
- the gated MLA decode at the hybrid slice's width (hidden 7168, 64 heads, kv_lora 512), whose
  o_proj also adds two K-ranges by atomics.
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

REPO = Path(__file__).resolve().parent.parent
for p in (REPO / "tests", REPO / "kimi-k3-in-c_amd", REPO / "oracle"):
    sys.path.insert(0, str(p))


def _decode(k3kda, ko, layer_weights, h, hidden, H, D, K, B, seed):
    import numpy as np
    import torch
    rng = np.random.default_rng(seed)
    W = layer_weights(rng, hidden, H, D, K)
    cfg = ko.make_cfg(hidden, H, D, K, -5.0, 1e-5)
    P = H * D
    kper = P * D + 3 * P * (K - 1)
    dw = k3kda.DeviceWeights(W.w, cfg, k3kda.UPLOAD_DEV | k3kda.UPLOAD_DECODE)
    states = torch.from_numpy((rng.standard_normal((B, kper)) * 0.05).astype(np.float32)).cuda()
    for _ in range(2):
        xd = torch.from_numpy(rng.standard_normal((B, hidden)).astype(np.float32)).cuda()
        od = torch.empty((B, hidden), device="cuda")
        dw.layer_decode(od, xd, states, kper)
        torch.cuda.synchronize()
        h.update(od.cpu().numpy().tobytes())
    h.update(states.cpu().numpy().tobytes())
    dw.close()


def run() -> str:
    import numpy as np
    import torch
    import k3kda
    import k3_oracle as ko
    from test_gpu_layer_prefill import layer_weights, bf16_to_f32
    from test_gpu_mla import mla_case
    from test_oracle_ref import bf16
    hidden, H, D, K, T, B = 512, 4, 128, 4, 300, 5
    rng = np.random.default_rng(0x4B334441 + 99)
    W = layer_weights(rng, hidden, H, D, K)
    cfg = ko.make_cfg(hidden, H, D, K, -5.0, 1e-5)
    P = H * D
    kper = P * D + 3 * P * (K - 1)
    dw = k3kda.DeviceWeights(W.w, cfg)
    h = hashlib.sha256()
    x = torch.from_numpy(bf16_to_f32(bf16(rng.standard_normal((T, hidden))))).cuda().to(torch.bfloat16)
    for impl in (k3kda.GEMM_HIPBLASLT, k3kda.GEMM_HANDWRITTEN):
        k3kda.set_projection_gemm(impl)
        try:
            state = torch.zeros(kper, device="cuda")
            out = torch.empty((T, hidden), device="cuda")
            dw.layer_prefill(out, x, state, T)
            torch.cuda.synchronize()
        finally:
            k3kda.set_projection_gemm(k3kda.GEMM_HIPBLASLT)
        h.update(out.cpu().numpy().tobytes())
        h.update(state.cpu().numpy().tobytes())
    states = state.repeat(B, 1).contiguous()
    for _ in range(2):
        xd = torch.from_numpy(rng.standard_normal((B, hidden)).astype(np.float32)).cuda()
        od = torch.empty((B, hidden), device="cuda")
        dw.layer_decode(od, xd, states, kper)
        torch.cuda.synchronize()
        h.update(od.cpu().numpy().tobytes())
    h.update(states.cpu().numpy().tobytes())
    dw.close()
    _decode(k3kda, ko, layer_weights, h, 512, 32, 128, 4, 9, 0x4B334441 + 98)
    _decode(k3kda, ko, layer_weights, h, 7168, 2, 128, 4, 17, 0x4B334441 + 97)
    # MLA at the hybrid width, one step over 300 seeded cache positions
    rng = np.random.default_rng(0x4B334441 + 96)
    mhidden, MH, ql, kvl, qn, qr, vh, MB, pos, cap = 7168, 64, 1536, 512, 128, 64, 128, 16, 300, 320
    mcfg, MW = mla_case(rng, mhidden, MH, ql, kvl, qn, qr, vh, 1)
    mw = k3kda.MlaWeights(MW.w, mcfg)
    cache = torch.from_numpy((rng.standard_normal((MB, cap, kvl + qr)) * 0.5).astype(np.float32)).cuda()
    xm = torch.from_numpy(rng.standard_normal((MB, mhidden)).astype(np.float32)).cuda()
    om = torch.empty((MB, mhidden), device="cuda")
    mw.decode(om, xm, cache, pos, cap)
    torch.cuda.synchronize()
    h.update(om.cpu().numpy().tobytes())
    h.update(cache.cpu().numpy().tobytes())
    mw.close()
    return h.hexdigest()


if __name__ == "__main__":
    print("bits", run(), flush=True)
