# SPDX-License-Identifier: Apache-2.0
"""K2 (chunked prefill, split-bf16 MFMA) through the C ABI against the sequential oracle.

Tolerance (the benchmark's stated bar for bf16-MFMA prefill): |got - want| <=
2e-3 * rms(want) + 2e-3 |want|. The split-bf16 products keep about 2^-17 relative error
per product (measured worst case about 5e-5 of rms at T = 1000), so the same runs are
also held to a 20x tighter bar (1e-4) to catch a precision regression long before the
stated bar would."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import GOLDEN, assert_close, worst_ratio
from test_chunk_form import inputs, sequential
import k3_oracle as ko
from k3_oracle import f32

pytestmark = pytest.mark.gpu

TOL = 2e-3
TIGHT = 1e-4


def rms(a):
    return float(np.sqrt(np.mean(np.asarray(a, np.float64) ** 2)))


def run_chunk(gpu, q, k, v, g, beta, S0, qs, workspace=True):
    import torch
    T, H, D = q.shape
    dq, dk, dv, dg = (torch.from_numpy(np.ascontiguousarray(a.reshape(T, -1))).cuda() for a in (q, k, v, g))
    db = torch.from_numpy(np.ascontiguousarray(beta)).cuda()
    dS = torch.from_numpy(S0.copy()).cuda()
    do = torch.full((T, H * D), float("nan"), device="cuda")
    ws = None
    if workspace:
        ws = torch.empty(max(1, gpu.kda_chunk_workspace(T, H, D)), dtype=torch.uint8, device="cuda")
    gpu.kda_chunk(dq, dk, dv, dg, db, dS, do, H, D, qs, 64, ws)
    torch.cuda.synchronize()
    return do.cpu().numpy().reshape(T, H, D), dS.cpu().numpy()


def check(got_o, got_S, want_o, want_S, what):
    ro = assert_close(got_o, want_o, TOL * rms(want_o), TOL, f"{what} o")
    rs = assert_close(got_S, want_S, TOL * rms(want_S), TOL, f"{what} S")
    to = worst_ratio(got_o, want_o, TIGHT * rms(want_o), TIGHT)
    ts = worst_ratio(got_S, want_S, TIGHT * rms(want_S), TIGHT)
    print(f"{what}: worst {ro:.4f}x / {rs:.4f}x of the 2e-3 bar; {to:.3f}x / {ts:.3f}x of 1e-4")
    assert to <= 1.0 and ts <= 1.0, f"{what}: precision regression ({to:.3f}x, {ts:.3f}x of 1e-4)"


@pytest.mark.parametrize("T", [1, 15, 16, 17, 63, 64, 65, 127, 128, 1000])
@pytest.mark.parametrize("D", [64, 128])
def test_chunk_vs_sequential_oracle(gpu, T, D):
    H = 3
    rng = np.random.default_rng(0x4B334441 + 2 + T + D)
    q, k, v, g, beta, S0 = inputs(rng, T, H, D)
    qs = float(np.float32(1) / np.sqrt(np.float32(D)))
    want_o, want_S = sequential(q, k, v, g, beta, S0, qs)
    got_o, got_S = run_chunk(gpu, q, k, v, g, beta, S0, qs)
    check(got_o, got_S, want_o, want_S, f"T={T} D={D}")


@pytest.mark.parametrize("D", [64, 128])
def test_chunk_tiny_unnormalised_inputs(gpu, D):
    """q, k of ~1e-6 (what the L2 norm leaves when eps dominates), v ~1e-9, zero S0, decays
    at the bound: every factored operand of the intra-chunk products must stay a normal
    bf16 number. With the pivot at a block's first row this case lost ~4% of the output."""
    T, H = 200, 2
    rng = np.random.default_rng(0x4B334441 + 30 + D)
    q, k, v, g, beta, S0 = inputs(rng, T, H, D)
    q, k, v = f32(q * 1e-6), f32(k * 1e-6), f32(v * 1e-9)
    g = f32(np.full_like(g, -5.0) * rng.uniform(0.9, 1.0, g.shape))
    S0[:] = 0.0
    qs = float(np.float32(1) / np.sqrt(np.float32(D)))
    want_o, want_S = sequential(q, k, v, g, beta, S0, qs)
    got_o, got_S = run_chunk(gpu, q, k, v, g, beta, S0, qs)
    check(got_o, got_S, want_o, want_S, f"tiny inputs D={D}")


def test_chunk_library_workspace_and_zero_state(gpu):
    rng = np.random.default_rng(3)
    T, H, D = 300, 4, 128
    q, k, v, g, beta, S0 = inputs(rng, T, H, D)
    S0[:] = 0.0
    qs = float(np.float32(1) / np.sqrt(np.float32(D)))
    want_o, want_S = sequential(q, k, v, g, beta, S0, qs)
    got_o, got_S = run_chunk(gpu, q, k, v, g, beta, S0, qs, workspace=False)
    check(got_o, got_S, want_o, want_S, "library workspace")


def test_chunk_fixtures(gpu):
    """The committed chunked fixtures: outputs over the whole sequence, and the state at
    every snapshot length (each length is its own prefill from S0)."""
    for f in sorted((GOLDEN / "chunk").glob("*.npz")):
        z = np.load(f)
        q, k, v, g, beta, S0 = (z[n] for n in ("q", "k", "v", "g", "beta", "S0"))
        qs = float(z["q_scale"])
        got_o, _ = run_chunk(gpu, q, k, v, g, beta, S0, qs)
        assert_close(got_o, z["o"], TOL * rms(z["o"]), TOL, f"{f.name} o")
        for Tp, Sp in zip(z["snap_T"], z["snap_S"]):
            _, got_S = run_chunk(gpu, q[:Tp], k[:Tp], v[:Tp], g[:Tp], beta[:Tp], S0, qs)
            assert_close(got_S, Sp, TOL * rms(Sp), TOL, f"{f.name} S after {Tp}")


def test_chunk_split_invariance_and_decode_continuation(gpu):
    """prefill(T1) then prefill(T2) from the carried state == prefill(T1 + T2), and a
    decode step (K3) after the prefill == the (T+1)-th step of the sequential oracle."""
    import torch
    rng = np.random.default_rng(17)
    T1, T2, H, D = 100, 77, 2, 128
    q, k, v, g, beta, S0 = inputs(rng, T1 + T2 + 1, H, D)
    qs = float(np.float32(1) / np.sqrt(np.float32(D)))
    T = T1 + T2
    want_o, want_S = sequential(q[:T], k[:T], v[:T], g[:T], beta[:T], S0, qs)
    o1, S1 = run_chunk(gpu, q[:T1], k[:T1], v[:T1], g[:T1], beta[:T1], S0, qs)
    o2, S2 = run_chunk(gpu, q[T1:T], k[T1:T], v[T1:T], g[T1:T], beta[T1:T], S1, qs)
    check(np.concatenate([o1, o2]), S2, want_o, want_S, "split 100+77")
    # one decode step on top
    dS = torch.from_numpy(S2[None].copy()).cuda()
    do = torch.zeros((1, H, D), device="cuda")
    al = f32(np.exp(g[T:T + 1].astype(np.float64)))
    to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    gpu.kda_decode(dS, do, to(q[T:T + 1]), to(k[T:T + 1]), to(v[T:T + 1]), to(al), to(beta[T:T + 1]), qs)
    torch.cuda.synchronize()
    w_o, w_S = sequential(q, k, v, g, beta, S0, qs)
    check(do.cpu().numpy(), dS.cpu().numpy()[0], w_o[T:T + 1], w_S, "decode after prefill")


def test_chunk_frozen_state_invariant(gpu):
    """alpha = 1 (g = 0) and beta = 0: the state never changes and o_t = S0^T q_t."""
    rng = np.random.default_rng(23)
    T, H, D = 150, 2, 128
    q, k, v, g, beta, S0 = inputs(rng, T, H, D)
    g[:] = 0.0
    beta[:] = 0.0
    qs = float(np.float32(1) / np.sqrt(np.float32(D)))
    got_o, got_S = run_chunk(gpu, q, k, v, g, beta, S0, qs)
    want_o = np.einsum("thi,hij->thj", q.astype(np.float64) * qs, S0.astype(np.float64))
    assert_close(got_o, want_o, TIGHT * rms(want_o), TIGHT, "frozen o")
    assert_close(got_S, S0, 1e-7, 1e-6, "frozen S")


def test_chunk_in_passes_bitwise(gpu):
    """A workspace for 4 chunks runs a 1000-token sequence in passes of 256 tokens with S
    carried between them: the same bits as one pass."""
    import torch
    rng = np.random.default_rng(31)
    T, H, D = 1000, 2, 128
    q, k, v, g, beta, S0 = inputs(rng, T, H, D)
    qs = float(np.float32(1) / np.sqrt(np.float32(D)))
    a_o, a_S = run_chunk(gpu, q, k, v, g, beta, S0, qs)
    dq, dk, dv, dg = (torch.from_numpy(np.ascontiguousarray(x.reshape(T, -1))).cuda() for x in (q, k, v, g))
    db = torch.from_numpy(np.ascontiguousarray(beta)).cuda()
    dS = torch.from_numpy(S0.copy()).cuda()
    do = torch.full((T, H * D), float("nan"), device="cuda")
    ws = torch.empty(gpu.kda_chunk_workspace(4 * 64, H, D), dtype=torch.uint8, device="cuda")
    gpu.kda_chunk(dq, dk, dv, dg, db, dS, do, H, D, qs, 64, ws)
    torch.cuda.synchronize()
    assert np.array_equal(do.cpu().numpy().reshape(T, H, D).view(np.uint32), a_o.view(np.uint32))
    assert np.array_equal(dS.cpu().numpy().view(np.uint32), a_S.view(np.uint32))


def test_chunk_deterministic(gpu):
    rng = np.random.default_rng(29)
    q, k, v, g, beta, S0 = inputs(rng, 200, 2, 128)
    a = run_chunk(gpu, q, k, v, g, beta, S0, 0.0883883)
    b = run_chunk(gpu, q, k, v, g, beta, S0, 0.0883883)
    assert np.array_equal(a[0].view(np.uint32), b[0].view(np.uint32))
    assert np.array_equal(a[1].view(np.uint32), b[1].view(np.uint32))


def test_chunk_refuses_bad_arguments(gpu):
    import torch
    t = torch.zeros((64, 48), device="cuda")
    with pytest.raises(gpu.K3HipError):
        gpu.kda_chunk(t, t, t, t, torch.zeros((64, 1), device="cuda"),
                      torch.zeros((1, 48, 48), device="cuda"), t, 1, 48, 0.1)
    t = torch.zeros((64, 128), device="cuda")
    small = torch.empty(16, dtype=torch.uint8, device="cuda")
    with pytest.raises(gpu.K3HipError):
        gpu.kda_chunk(t, t, t, t, torch.zeros((64, 1), device="cuda"),
                      torch.zeros((1, 128, 128), device="cuda"), t, 1, 128, 0.1, 64, small)
