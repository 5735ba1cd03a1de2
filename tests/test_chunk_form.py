# SPDX-License-Identifier: Apache-2.0
"""The chunked form (tests/chunk_form.py) against the sequential oracle (the restatement of
k3_kda_step, kimi-k3-in-c src/core/k3_ops.c:186-243) and the committed chunked fixtures.

This is where the two invariants a chunked KDA path must keep are gated (the reference
header asks for exactly these, include/k3/k3.h:51-60): Tm = (I + A_kk)^-1 with A_kk
STRICTLY lower, and A_qk INCLUDING its diagonal. Each planted mistake must fail."""
from __future__ import annotations

import numpy as np
import pytest

from chunk_form import chunked
from conftest import GOLDEN, worst_ratio
import k3_oracle as ko
from k3_oracle import f32


def inputs(rng, T, H, D, S_scale=0.1, lb=-5.0):
    q = rng.standard_normal((T, H, D))
    k = rng.standard_normal((T, H, D))
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((T, H, D))
    g = rng.uniform(lb, 0.0, (T, H, D))
    beta = rng.uniform(0, 1, (T, H))
    S0 = rng.standard_normal((H, D, D)) * S_scale
    return tuple(f32(a) for a in (q, k, v, g, beta, S0))


def sequential(q, k, v, g, beta, S0, qs):
    T, H, D = q.shape
    S = S0.copy()
    o = ko.recurrence(S, q.reshape(T, -1), k.reshape(T, -1), v.reshape(T, -1),
                      f32(np.exp(g.astype(np.float64))).reshape(T, -1), beta, H, D, qs, 4)
    return o.reshape(T, H, D), S


@pytest.mark.parametrize("T", [1, 15, 16, 17, 63, 64, 65, 127, 128, 200])
def test_chunked_form_equals_sequential(T):
    rng = np.random.default_rng(T)
    H, D = 2, 16
    q, k, v, g, beta, S0 = inputs(rng, T, H, D)
    qs = float(np.float32(1) / np.sqrt(np.float32(D)))
    o1, S1 = sequential(q, k, v, g, beta, S0, qs)
    o2, S2 = chunked(q, k, v, g, beta, S0, qs)
    assert worst_ratio(o2, o1, 1e-6, 1e-5) <= 1.0
    assert worst_ratio(S2, S1, 1e-6, 1e-5) <= 1.0


@pytest.mark.parametrize("akk_diag,aqk_diag", [(True, True), (False, False)])
def test_planted_diagonal_mistakes_fail(akk_diag, aqk_diag):
    """Keeping A_kk's diagonal, or dropping A_qk's, must move the output far past the
    chunked-prefill tolerance (2e-3)."""
    rng = np.random.default_rng(99)
    T, H, D = 70, 2, 16
    q, k, v, g, beta, S0 = inputs(rng, T, H, D)
    qs = float(np.float32(1) / np.sqrt(np.float32(D)))
    o1, _ = sequential(q, k, v, g, beta, S0, qs)
    o2, _ = chunked(q, k, v, g, beta, S0, qs, akk_diag=akk_diag, aqk_diag=aqk_diag)
    rms = float(np.sqrt(np.mean(o1.astype(np.float64) ** 2)))
    assert worst_ratio(o2, o1, 2e-3 * rms, 2e-3) > 10.0


def test_chunk_fixtures_pin_the_oracle():
    """The committed chunked fixtures (tests/golden/chunk, written by
    make_chunk_fixtures.py from the oracle) still match the oracle and the chunked form,
    and a planted diagonal mistake fails them."""
    for f in sorted((GOLDEN / "chunk").glob("*.npz")):
        z = np.load(f)
        q, k, v, g, beta, S0 = (z[n] for n in ("q", "k", "v", "g", "beta", "S0"))
        qs = float(z["q_scale"])
        T = q.shape[0]
        o_seq, _ = sequential(q, k, v, g, beta, S0, qs)
        assert np.array_equal(o_seq.view(np.uint32), z["o"].view(np.uint32)), f.name
        for Tp, Sp in zip(z["snap_T"], z["snap_S"]):
            _, S_t = sequential(q[:Tp], k[:Tp], v[:Tp], g[:Tp], beta[:Tp], S0, qs)
            assert np.array_equal(S_t.view(np.uint32), Sp.view(np.uint32)), (f.name, Tp)
        o_ch, S_ch = chunked(q, k, v, g, beta, S0, qs)
        assert worst_ratio(o_ch, z["o"], 1e-6, 1e-5) <= 1.0
        assert worst_ratio(S_ch, z["snap_S"][-1], 1e-6, 1e-5) <= 1.0
        o_bad, _ = chunked(q, k, v, g, beta, S0, qs, akk_diag=True)
        rms = float(np.sqrt(np.mean(z["o"].astype(np.float64) ** 2)))
        assert worst_ratio(o_bad, z["o"], 2e-3 * rms, 2e-3) > 10.0
