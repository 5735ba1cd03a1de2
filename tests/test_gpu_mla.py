# SPDX-License-Identifier: Apache-2.0
"""Gated MLA decode with absorbed weights (k3hip_mla_decode) against the oracle's
expanded-KV restatement of k3_mla_cached (src/core/k3_ops.c:321-424), which is itself
pinned to the reference's mla.json fixture and to the reference C bit for bit.

B sequences decode token by token from an empty cache: the GPU keeps the compressed latent
per position, the oracle the expanded per-head keys and values, one cache per sequence.
Every output of every step is compared at the decode bar (rtol 1e-4, atol 1e-4 * rms):
the two orders of the same maths differ by fp32 rounding only."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_close, worst_ratio
from test_oracle_ref import bf16
import k3_oracle as ko

pytestmark = pytest.mark.gpu


def rms(a):
    return float(np.sqrt(np.mean(np.asarray(a, np.float64) ** 2)))


def mla_case(rng, hidden, H, ql, kvl, qn, qr, vh, gate=1):
    cfg = ko.mla_cfg(hidden, H, ql, kvl, qn, qr, vh, 1e-5, gate)
    mats = {"q_a": (ql, hidden), "q_b": (H * (qn + qr), ql), "kv_a": (kvl + qr, hidden),
            "kv_b": (H * (qn + vh), kvl), "o": (hidden, H * vh), "g": (H * vh, hidden)}
    arrays = {n: bf16(rng.standard_normal(s) * (0.5 / np.sqrt(s[1]))) for n, s in mats.items()}
    if not gate:
        del arrays["g"]
    arrays["q_a_norm"] = (1 + 0.1 * rng.standard_normal(ql)).astype(np.float32)
    arrays["kv_a_norm"] = (1 + 0.1 * rng.standard_normal(kvl)).astype(np.float32)
    return cfg, ko.MlaWeights(arrays, 1)


@pytest.mark.parametrize("hidden,H,ql,kvl,qn,qr,vh,B,T,gate", [
    (256, 4, 64, 64, 32, 16, 32, 3, 9, 1),
    (384, 8, 96, 128, 64, 32, 64, 17, 6, 1),     # B above one absorb pass of 16
    (128, 2, 32, 32, 16, 8, 16, 2, 40, 0),       # ungated, longer context
    (256, 64, 64, 512, 32, 64, 32, 2, 150, 1),   # the 576-channel latent + rope rows of Kimi K3
    (256, 4, 64, 64, 20, 12, 32, 3, 5, 1),       # nope not a multiple of 8: the absorb's element loads
    (128, 2, 32, 32, 264, 8, 16, 2, 3, 1),       # nope above 256: the absorb on the batched library GEMM
])
def test_mla_decode_vs_expanded_oracle(gpu, hidden, H, ql, kvl, qn, qr, vh, B, T, gate):
    _mla_decode_vs_oracle(gpu, hidden, H, ql, kvl, qn, qr, vh, B, T, gate, 0x4B334441 + 4 + hidden + B + T)


@pytest.mark.parametrize("case", range(10))
def test_mla_decode_random_vs_expanded_oracle(gpu, case):
    """Seeded random MLA layers inside the one-pass attention kernel's geometry: 1-64 heads,
    kv_lora a multiple of 16 up to 512, rope 8-64 channels, nope and v heads 16-64, gated or
    not, B 1-12 sequences over 1-40 steps."""
    rng = np.random.default_rng(0x4B334441 + 0x31A + case)
    hidden, H, ql = 64 * int(rng.integers(1, 7)), int(rng.integers(1, 65)), 32 * int(rng.integers(1, 5))
    kvl, qr = 16 * int(rng.integers(1, 33)), int(rng.choice([8, 16, 32, 64]))
    qn, vh = int(rng.choice([16, 32, 64])), int(rng.choice([16, 32, 64]))
    B, T, gate = int(rng.integers(1, 13)), int(rng.integers(1, 41)), int(rng.integers(0, 2))
    _mla_decode_vs_oracle(gpu, hidden, H, ql, kvl, qn, qr, vh, B, T, gate, 0x4B334441 + 0x31A + case)


def _mla_decode_vs_oracle(gpu, hidden, H, ql, kvl, qn, qr, vh, B, T, gate, seed):
    import torch
    rng = np.random.default_rng(seed)
    print(f"hidden={hidden} H={H} q_lora={ql} kv_lora={kvl} nope={qn} rope={qr} v_head={vh} B={B} T={T} "
          f"gate={gate}", flush=True)
    cfg, W = mla_case(rng, hidden, H, ql, kvl, qn, qr, vh, gate)
    cap = T + 3
    kvcs = [np.zeros((cap, H * (qn + vh)), np.float32) for _ in range(B)]
    ropecs = [np.zeros((cap, qr), np.float32) for _ in range(B)]
    mw = gpu.MlaWeights(W.w, cfg)
    cache = torch.zeros((B, cap, kvl + qr), device="cuda")
    worst = 0.0
    for t in range(T):
        x = rng.standard_normal((B, hidden)).astype(np.float32)
        want = np.concatenate([ko.mla(x[b:b + 1], W, cfg, 1, kvcs[b], ropecs[b], t, cap) for b in range(B)])
        out = torch.full((B, hidden), float("nan"), device="cuda")
        mw.decode(out, torch.from_numpy(x).cuda(), cache, t, cap)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert_close(got, want, 1e-4 * rms(want), 1e-4, f"MLA step {t}")
        worst = max(worst, worst_ratio(got, want, 1e-4 * rms(want), 1e-4))
    print(f"  worst {worst:.3f}x of the 1e-4 bar")
    mw.close()


def test_mla_refusals(gpu):
    import torch
    rng = np.random.default_rng(5)
    cfg, W = mla_case(rng, 128, 2, 32, 32, 16, 8, 16)
    mw = gpu.MlaWeights(W.w, cfg)
    cache = torch.zeros((1, 4, 40), device="cuda")
    x, out = torch.zeros((1, 128), device="cuda"), torch.zeros((1, 128), device="cuda")
    with pytest.raises(gpu.K3HipError) as e:
        mw.decode(out, x, cache, 4, 4)          # position past the cache
    assert e.value.code == 1
    mw.close()
    W32 = ko.MlaWeights({n: a for n, a in W.arrays.items()}, 0)   # fp32 tag: not supported
    with pytest.raises(gpu.K3HipError) as e:
        gpu.MlaWeights(W32.w, cfg)
    assert e.value.code == 3


def seeded_caches(rng, W, H, kvl, qn, qr, vh, B, pos, cap, ncache=4):
    """Positions 0..pos-1 filled with random (rmsnorm-scale) latents and rope slots: the GPU's
    compressed rows [latent | rope] and the oracle's expanded rows kv_b . latent (float64
    product rounded to fp32) for the same values; sequence b uses cache b % ncache."""
    kvb = np.asarray(W.arrays["kv_b"]).astype(np.uint32) << 16
    kvb = kvb.view(np.float32).astype(np.float64)                 # [H*(qn+vh)][kvl]
    gcache = np.zeros((B, cap, kvl + qr), np.float32)
    kvcs, ropecs = [], []
    base = []
    for c in range(ncache):
        L = rng.standard_normal((pos, kvl)).astype(np.float32)
        R = rng.standard_normal((pos, qr)).astype(np.float32)
        kv = np.zeros((cap, H * (qn + vh)), np.float32)
        kv[:pos] = (L.astype(np.float64) @ kvb.T).astype(np.float32)
        rp = np.zeros((cap, qr), np.float32)
        rp[:pos] = R
        base.append((L, R, kv, rp))
    for b in range(B):
        L, R, kv, rp = base[b % ncache]
        gcache[b, :pos, :kvl], gcache[b, :pos, kvl:] = L, R
        kvcs.append(kv.copy())
        ropecs.append(rp.copy())
    return gcache, kvcs, ropecs


def run_steps(gpu, rng, W, cfg, hidden, B, gcache, kvcs, ropecs, positions, cap):
    import torch
    mw = gpu.MlaWeights(W.w, cfg)
    cache = torch.from_numpy(gcache).cuda()
    worst = 0.0
    for pos in positions:
        x = rng.standard_normal((B, hidden)).astype(np.float32)
        want = np.concatenate([ko.mla(x[b:b + 1], W, cfg, 1, kvcs[b], ropecs[b], pos, cap) for b in range(B)])
        out = torch.full((B, hidden), float("nan"), device="cuda")
        mw.decode(out, torch.from_numpy(x).cuda(), cache, pos, cap)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        worst = max(worst, assert_close(got, want, 1e-4 * rms(want), 1e-4, f"MLA pos {pos}"))
    mw.close()
    return worst


def test_mla_fallback_heads_above_64(gpu):
    """H = 96 (the reference's real MLA head count, src/cli/k3_run.c:105) is outside the fused
    attention kernel: scores and P . cache as strided-batched fp32 GEMMs around the softmax.
    Contexts 40, 2100 and 8300 cross its three softmax variants (<= 2048, <= 8192, longer)."""
    rng = np.random.default_rng(0x4B334441 + 96)
    hidden, H, ql, kvl, qn, qr, vh, B = 128, 96, 32, 32, 16, 8, 16, 2
    cfg, W = mla_case(rng, hidden, H, ql, kvl, qn, qr, vh, 1)
    positions, cap = (40, 2100, 8300), 8304
    gcache, kvcs, ropecs = seeded_caches(rng, W, H, kvl, qn, qr, vh, B, positions[-1], cap, ncache=2)
    # positions after the first seeded one are overwritten step by step on both sides
    w = run_steps(gpu, rng, W, cfg, hidden, B, gcache, kvcs, ropecs, positions, cap)
    print(f"H=96 fallback: worst {w:.3f}x of the 1e-4 bar")


def test_mla_at_hybrid_width(gpu):
    """The hybrid slice's MLA layer: hidden 7168, 64 heads, q_lora 1536, kv_lora 512, rope 64,
    nope 128, v 128, B = 16 over ~600 cached positions, so the fused attention splits every
    sequence into 16 position ranges (ragged, not multiples of its 16-position tile) and the
    merge combines them."""
    rng = np.random.default_rng(0x4B334441 + 77)
    hidden, H, ql, kvl, qn, qr, vh, B = 7168, 64, 1536, 512, 128, 64, 128, 16
    cfg, W = mla_case(rng, hidden, H, ql, kvl, qn, qr, vh, 1)
    cap = 640
    gcache, kvcs, ropecs = seeded_caches(rng, W, H, kvl, qn, qr, vh, B, 597, cap)
    w = run_steps(gpu, rng, W, cfg, hidden, B, gcache, kvcs, ropecs, (597, 598), cap)
    print(f"hybrid-width MLA B={B}: worst {w:.3f}x of the 1e-4 bar")


def test_mla_at_hybrid_width_timed_context(gpu):
    """The hybrid slice's MLA layer at the context the benchmark times: hidden 7168, 64 heads,
    q_lora 1536, kv_lora 512, rope 64, B = 16 sequences attending over 8,192 then 8,193 cached
    positions (the fused attention's position ranges at their timed lengths). The nope and v
    heads are 16 wide so that the oracle's expanded per-head cache stays small (two seeded
    caches shared by the 16 sequences); the attention kernel reads only the latent rows,
    whose width does not depend on them."""
    rng = np.random.default_rng(0x4B334441 + 78)
    hidden, H, ql, kvl, qn, qr, vh, B = 7168, 64, 1536, 512, 16, 64, 16, 16
    cfg, W = mla_case(rng, hidden, H, ql, kvl, qn, qr, vh, 1)
    cap = 8200
    gcache, kvcs, ropecs = seeded_caches(rng, W, H, kvl, qn, qr, vh, B, 8192, cap, ncache=2)
    w = run_steps(gpu, rng, W, cfg, hidden, B, gcache, kvcs, ropecs, (8192, 8193), cap)
    print(f"hybrid-width MLA B={B} over 8,192 positions: worst {w:.3f}x of the 1e-4 bar")
