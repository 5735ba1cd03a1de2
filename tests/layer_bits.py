# SPDX-License-Identifier: Apache-2.0
"""Helper for tests/test_gpu_determinism.py (not a test module): runs a seeded bf16 layer
prefill and two batched decode steps on cuda:0 and prints one sha256 line of every output
and state byte, so two fresh processes can be compared."""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

REPO = Path(__file__).resolve().parent.parent
for p in (REPO / "tests", REPO / "kimi-k3-in-c_amd", REPO / "oracle"):
    sys.path.insert(0, str(p))


def run() -> str:
    import numpy as np
    import torch
    import k3kda
    import k3_oracle as ko
    from test_gpu_layer_prefill import layer_weights, bf16_to_f32
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
    state = torch.zeros(kper, device="cuda")
    out = torch.empty((T, hidden), device="cuda")
    dw.layer_prefill(out, x, state, T)
    torch.cuda.synchronize()
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
    return h.hexdigest()


if __name__ == "__main__":
    print("bits", run(), flush=True)
