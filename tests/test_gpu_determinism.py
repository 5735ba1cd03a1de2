# SPDX-License-Identifier: Apache-2.0
"""Bit identity as the race detector (the reference's own gate, tests/unit/test_ops.c:457-472):
the work of tests/layer_bits.py gives the same bits twice in one process and in two fresh
processes. It covers the bf16 layer prefill on both projection GEMMs (hipBLASLt's heuristic
first choice, never a timing; the hand-written GEMM with split-K f_a / b planes summed in
order), the batched decode layer with its decode GEMVs in one K-range, in 16 K-ranges (an
ordered reduction) and in two K-ranges added into the output by float atomics (a two-term
sum, the same in either order), and the gated MLA decode at the hybrid width."""
from __future__ import annotations

import subprocess
import sys

import pytest

from conftest import REPO

pytestmark = pytest.mark.gpu


def test_layer_paths_bitwise_in_process(gpu):
    import layer_bits
    assert layer_bits.run() == layer_bits.run()


def test_layer_paths_bitwise_across_processes(gpu):
    digests = []
    for i in range(2):
        r = subprocess.run([sys.executable, str(REPO / "tests" / "layer_bits.py")], capture_output=True,
                           text=True, timeout=300)
        assert r.returncode == 0, r.stderr[-2000:]
        line = [l for l in r.stdout.splitlines() if l.startswith("bits ")]
        assert line, r.stdout[-2000:]
        digests.append(line[-1].split()[1])
        print(f"process {i}: {digests[-1]}", flush=True)
    assert digests[0] == digests[1], "two processes produced different bits"
