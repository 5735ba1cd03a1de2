# SPDX-License-Identifier: Apache-2.0
"""Writes the chunked-prefill golden fixtures (tests/golden/chunk/*.npz).

The reference has no chunked KDA path and so no fixture for one (kimi-k3-in-c
include/k3/k3.h:51-60 asks that a chunked path ship its own). These fixtures hold seeded
inputs (numpy default_rng) and the outputs of T sequential k3_kda_step calls per head
computed by the C oracle (oracle/k3_oracle.c, itself pinned to the reference fixtures
and to the reference C), with the recurrent state snapshotted at the lengths where a
chunked kernel changes behaviour: 1, chunk edges 63/64/65, 127/128, sub-block edges
15/16/17, and the full length. Run from the repository root:
    python tests/golden/make_chunk_fixtures.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
sys.path.insert(0, str(HERE.parent.parent / "oracle"))
from test_chunk_form import inputs, sequential  # noqa: E402

CASES = [
    ("chunk_h2_d64_t130", 0x4B334441 + 20, 130, 2, 64, [1, 15, 16, 17, 63, 64, 65, 127, 128, 130]),
    ("chunk_h1_d128_t70", 0x4B334441 + 21, 70, 1, 128, [64, 70]),
]


def main() -> None:
    out = HERE / "chunk"
    out.mkdir(exist_ok=True)
    for name, seed, T, H, D, snaps in CASES:
        rng = np.random.default_rng(seed)
        q, k, v, g, beta, S0 = inputs(rng, T, H, D)
        qs = np.float32(1) / np.sqrt(np.float32(D))
        o, _ = sequential(q, k, v, g, beta, S0, float(qs))
        snap_S = np.stack([sequential(q[:t], k[:t], v[:t], g[:t], beta[:t], S0, float(qs))[1]
                           for t in snaps])
        np.savez(out / f"{name}.npz", q=q, k=k, v=v, g=g, beta=beta, S0=S0,
                 q_scale=np.float32(qs), o=o, snap_T=np.array(snaps, np.int32), snap_S=snap_S)
        print(name, T, H, D, "->", (out / f"{name}.npz").stat().st_size, "bytes")


if __name__ == "__main__":
    main()
