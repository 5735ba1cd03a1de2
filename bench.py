# SPDX-License-Identifier: Apache-2.0
"""KDA path benchmark on one MI355X.

Workloads (synthetic inputs resident in HBM before the timed region):
  prefill  hidden 4096, H=32, D=128, chunk 64, T=8192, batch 1: one step = K1 (conv +
           SiLU + L2 + decay + beta, bf16 activations in) fused with K2 (chunked delta-rule
           prefill, fp32 state) -> K4 (head RMSNorm + sigmoid gate, bf16 out). The
           projections are not part of the step (they are plain GEMMs).
  decode   H=32, D=128, B=64 sequences, one token each: one step = K3 over all 2048
           (sequence, head) states. The state sets rotate over 4 independent buffers
           (512 MiB) so that the 256 MB last-level cache cannot hold the working set.
  long     the prefill step above at T=65,536, then 256 single-token decode steps of the
           same sequence (K1 at T=1 -> K3 at B=1 -> K4).
  small    one KDA layer on fp32 weights, hidden 256, H=4, D=64: a 32-token prefill then 8
           single-token decode steps.

Prints ONE JSON line. `value` is prefill tokens/s; the decode result (state-update GB/s)
is the `decode` object of the same line. `roofline` is for the dominant prefill kernel;
`decode.roofline` for K3. Kernel durations come from HIP events recorded on the launch
stream around every launch inside the timed region. `cpu_baseline` is the CPU oracle
timed on this host on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import subprocess
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "kimi-k3-in-c_amd"))

HBM_PEAK = 8.0e12          # bytes/s, MI355X HBM3E
BF16_PEAK = 2.5e15         # flop/s, dense bf16 MFMA
FP32_PEAK = 157.3e12       # flop/s, dense fp32 MFMA

# prefill core / layer at T=8192, hidden 4096; batch-64 decode
PRE = dict(hidden=4096, H=32, D=128, T=8192, chunk=64, K=4, gate_lb=-5.0, rms_eps=1e-5)
DEC = dict(B=64, H=32, D=128)
# long context: the core alone over 65,536 tokens, then 256 single-token decode steps
LONG = dict(T=65536, decode=256)
# the small CPU-runnable layer: hidden 256, H=4, D=64, fp32, 32-token prefill + 8 decode steps
SMALL = dict(hidden=256, H=4, D=64, K=4, T=32, decode=8, gate_lb=-5.0, rms_eps=1e-5)
# hybrid decode slice: 3 KDA layers + 1 gated MLA layer, decode at batch 16 over an 8192 context
HYB = dict(hidden=7168, B=16, ctx=8192, kda_layers=3, H=32, D=128, K=4, gate_lb=-5.0,
           mla_heads=64, q_lora=1536, kv_lora=512, qk_nope=128, qk_rope=64, v_head=128)


def decode_bytes_per_token(H: int, D: int) -> int:
    """Algorithmic HBM bytes of one decode token (all heads of one sequence): state read
    and write 2*H*D*D*4, q k v alpha 4*H*D*4, beta 4*H, o H*D*4."""
    return 2 * H * D * D * 4 + 4 * H * D * 4 + 4 * H + H * D * 4


def prefill_core_flops_per_token(H: int, D: int, C: int) -> float:
    """Algorithmic flops of the chunked core per token: 2*H*(5*C*D + 3*D*D + C*C/6)."""
    return 2.0 * H * (5 * C * D + 3 * D * D + C * C / 6.0)


def layer_flops_per_token(hidden: int, H: int, D: int, C: int) -> float:
    """Algorithmic flops of the full layer per token: projections q k v g (4P x hidden), f_a
    (D x hidden), b (H x hidden), f_b (P x D), o_proj (hidden x P), plus the chunked core."""
    P = H * D
    return (2.0 * hidden * (4 * P + D + H) + 2.0 * D * P + 2.0 * P * hidden
            + prefill_core_flops_per_token(H, D, C))


def prefill_core_bytes_per_token(H: int, D: int) -> int:
    """Algorithmic HBM bytes of the fused K1+K2 core per token: conv inputs q k v (bf16)
    6*P, gate pre-activation z (fp32) 4*P, beta logits 4*H, o out (fp32) 4*P."""
    P = H * D
    return 6 * P + 4 * P + 4 * H + 4 * P


def cpu_info() -> dict:
    """The host CPU: lscpu model, physical cores (all, and those in this process's CPU
    affinity share), and the OpenMP threads the baselines use: one per physical core of the
    share, as the reference sizes its pool (src/cli/k3_run.c:1096-1106), capped by
    OMP_NUM_THREADS when the environment sets it."""
    model = "unknown"
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        allowed = sorted(os.sched_getaffinity(0))
    except AttributeError:
        allowed = list(range(os.cpu_count() or 1))

    def core_of(cpu):
        base = Path(f"/sys/devices/system/cpu/cpu{cpu}/topology")
        try:
            return (base / "physical_package_id").read_text().strip(), (base / "core_id").read_text().strip()
        except OSError:
            return ("cpu", str(cpu))
    every = [c for c in range(os.cpu_count() or 1) if Path(f"/sys/devices/system/cpu/cpu{c}").exists()]
    phys_total = len({core_of(c) for c in every}) or len(every)
    phys_share = len({core_of(c) for c in allowed}) or len(allowed)
    threads = phys_share
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        threads = min(threads, int(omp))
    return {"model": model, "physical_cores": phys_total, "physical_cores_in_share": phys_share,
            "threads": max(1, threads)}


def set_omp_threads(n: int) -> None:
    """OpenMP thread count of the calling thread for the CPU baselines (libgomp is shared by
    the oracle and the reference libraries)."""
    try:
        import ctypes
        ctypes.CDLL("libgomp.so.1").omp_set_num_threads(int(n))
    except OSError:
        pass


def measured_traffic(*kernels: str):
    """HBM bytes per launch of the named kernels from the committed counter profile
    (profiles/traffic.json: FETCH_SIZE and WRITE_SIZE runs, copy-calibrated), or None."""
    try:
        t = json.loads((REPO / "profiles" / "traffic.json").read_text())["kernels"]
        return sum(t[k]["read_bytes"] + t[k]["write_bytes"] for k in kernels)
    except (OSError, KeyError, ValueError):
        return None


def ev_pair(torch):
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


RAMP_S = 0.3


def ramp(torch, step):
    """Untimed: repeat the workload's own step for RAMP_S seconds before its warm-up steps.
    From idle the GPU takes tens of milliseconds of sustained load to reach its working
    clocks (T=8192 prefill core: 0.63 ms per step after 3 warm-up steps, 0.585 after 20, 0.56 after
    ~60), so a few warm-up steps alone measure the ramp, not the kernels."""
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < RAMP_S:
        for _ in range(4):
            step()
        torch.cuda.synchronize()


# -------------------------------------------------------------------- decode ----
def bench_decode(torch, k3, steps: int, warmup: int, cpu: bool) -> dict:
    B, H, D = DEC["B"], DEC["H"], DEC["D"]
    nsets = 4
    g = torch.Generator(device="cuda").manual_seed(0x4B334441 + 1)
    sets = []
    for _ in range(nsets):
        S = torch.randn((B, H, D, D), device="cuda", generator=g) * 0.1
        q = torch.nn.functional.normalize(torch.randn((B, H, D), device="cuda", generator=g), dim=-1)
        k = torch.nn.functional.normalize(torch.randn((B, H, D), device="cuda", generator=g), dim=-1)
        v = torch.randn((B, H, D), device="cuda", generator=g)
        alpha = torch.exp(torch.rand((B, H, D), device="cuda", generator=g) * -5.0)
        beta = torch.rand((B, H), device="cuda", generator=g)
        o = torch.empty((B, H, D), device="cuda")
        sets.append((S, o, q.contiguous(), k.contiguous(), v, alpha, beta))
    qs = 1.0 / math.sqrt(D)
    ramp(torch, lambda: [k3.kda_decode(*sets[j], qs) for j in range(nsets)])
    for i in range(warmup):
        k3.kda_decode(*sets[i % nsets], qs)
    torch.cuda.synchronize()
    # One event pair around the K back-to-back launches (a decode step is one kernel), so
    # the average is the kernel's own duration without per-launch event gaps; three
    # repeats give the spread.
    reps = []
    t0 = time.perf_counter()
    for _ in range(3):
        e0, e1 = ev_pair(torch)
        e0.record()
        for i in range(steps):
            k3.kda_decode(*sets[i % nsets], qs)
        e1.record()
        torch.cuda.synchronize()
        reps.append(e0.elapsed_time(e1) * 1e-3 / steps)
    wall = (time.perf_counter() - t0) / 3
    ks = sorted(reps)
    kavg = sum(ks) / len(ks)
    step_s = wall / steps
    bytes_step = decode_bytes_per_token(H, D) * B
    out = {
        "value": bytes_step / step_s / 1e9, "unit": "GB/s", "tokens_per_s": B / step_s,
        "ms_per_step": step_s * 1e3, "kernel_ms_avg": kavg * 1e3,
        "kernel_ms_min_of_3": ks[0] * 1e3, "kernel_ms_max_of_3": ks[-1] * 1e3,
        "config": {"workload": "kda_decode", "batch": B, "heads": H, "head_dim": D,
                   "state_sets_rotated": nsets, "bytes_per_step": bytes_step},
        "roofline": {"kernel": "kda_decode_kernel<128,512>", "bound": "hbm",
                     "achieved": bytes_step / kavg / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                     "frac": bytes_step / kavg / HBM_PEAK,
                     "traffic": measured_traffic("kda_decode_kernel<128, 512>")},
        "tolerance": "rtol 1e-4, atol 1e-4*rms (tests/test_gpu_kernels.py)",
    }
    if cpu:   # timed after every GPU workload (its OpenMP threads would load the host)
        dset = [t.cpu() for t in sets[0]]
        out["_cpu"] = lambda: cpu_decode(torch, dset)
    return out


def cpu_decode(torch, dset) -> dict:
    import numpy as np
    sys.path.insert(0, str(REPO / "oracle"))
    import k3_oracle as ko
    S, o, q, k, v, alpha, beta = (t.cpu().numpy() for t in dset)
    B, H, D = q.shape
    ci = cpu_info()
    nt = ci["threads"]
    S = np.ascontiguousarray(S)
    ko.decode_batch(S, q, k, v, alpha, beta, 1.0 / math.sqrt(D), nt)   # warm
    n, t0 = 0, time.perf_counter()
    while True:
        ko.decode_batch(S, q, k, v, alpha, beta, 1.0 / math.sqrt(D), nt)
        n += 1
        el = time.perf_counter() - t0
        if el > 8.0 or n >= 5000:
            break
    step = el / n
    bytes_step = decode_bytes_per_token(H, D) * B
    return {"value": bytes_step / step / 1e9, "unit": "GB/s", "tokens_per_s": B / step,
            "cores": nt, "kind": "port", "cpu": ci["model"], "physical_cores": ci["physical_cores"],
            "physical_cores_in_share": ci["physical_cores_in_share"],
            "sample": f"{n} full decode steps (B={B}, H={H}, D={D}) of the C oracle, OpenMP over "
                      f"(sequence, head) pairs, {el:.1f} s"}


# ------------------------------------------------------------------- prefill ----
def bench_prefill(torch, k3, steps: int, warmup: int, cpu: bool) -> dict:
    c = PRE
    H, D, T, K = c["H"], c["D"], c["T"], c["K"]
    P = H * D
    g = torch.Generator(device="cuda").manual_seed(0x4B334441 + 2)
    bf = torch.bfloat16
    q_in = torch.randn((T, P), device="cuda", generator=g).to(bf)
    k_in = torch.randn((T, P), device="cuda", generator=g).to(bf)
    v_in = torch.randn((T, P), device="cuda", generator=g).to(bf)
    z = torch.randn((T, P), device="cuda", generator=g) * 0.02
    b_logit = torch.randn((T, H), device="cuda", generator=g)
    gate = torch.randn((T, P), device="cuda", generator=g).to(bf)
    conv = [torch.randn((P, K), device="cuda", generator=g) * 0.5 for _ in range(3)]
    A_log = torch.rand((H,), device="cuda", generator=g) * 1.5
    dt_bias = torch.randn((P,), device="cuda", generator=g)
    o_norm = 1 + 0.1 * torch.randn((D,), device="cuda", generator=g)
    f32 = dict(device="cuda", dtype=torch.float32)
    q, k, v, gg = (torch.empty((T, P), **f32) for _ in range(4))
    beta = torch.empty((T, H), **f32)
    o = torch.empty((T, P), **f32)
    y = torch.empty((T, P), device="cuda", dtype=bf)
    S = torch.zeros((H, D, D), **f32)
    conv_state = torch.zeros(3 * P * (K - 1), **f32)
    qs = 1.0 / math.sqrt(D)
    # core: "fused" = k3hip_kda_prefill (K1 + K2 in one pass over the activations), else
    # k3hip_kda_prep + k3hip_kda_chunk, else the sequential GPU recurrence
    mode = "fused"
    ws = torch.empty(max(1, k3.kda_chunk_workspace(T, H, D, 64)), dtype=torch.uint8, device="cuda")
    alpha = torch.empty((T, P), **f32)

    def step(evk=None):
        S.zero_()
        conv_state.zero_()
        if evk:
            evk[0].record()
        if mode == "fused":
            k3.kda_prefill(q_in, k_in, v_in, z, b_logit, conv[0], conv[1], conv[2], A_log, dt_bias,
                           conv_state, S, o, H, D, K, c["gate_lb"], qs, ws)
        else:
            k3.kda_prep(q_in, k_in, v_in, z, b_logit, conv[0], conv[1], conv[2], A_log, dt_bias,
                        conv_state, q, k, v, gg, alpha, beta, H, D, K, c["gate_lb"])
            if mode == "chunk":
                k3.kda_chunk(q, k, v, gg, beta, S, o, H, D, qs, 64, ws)
            else:
                k3.kda_recurrent(q, k, v, alpha, beta, S, o, H, D, qs)
        if evk:
            evk[1].record()
        k3.kda_epilogue(o, gate, o_norm, y, H, D, c["rms_eps"])

    for fallback in ("chunk", "recurrent", None):
        try:
            step()
            torch.cuda.synchronize()
            break
        except k3.K3HipError:
            if fallback is None:
                raise
            mode = fallback
    ramp(torch, step)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    evs = [ev_pair(torch) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        step(evs[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ks = sorted(a.elapsed_time(b) * 1e-3 for a, b in evs)
    kavg = sum(ks) / len(ks)
    step_s = wall / steps
    flops_launch = prefill_core_flops_per_token(H, D, 64) * T
    bytes_launch = prefill_core_bytes_per_token(H, D) * T
    kname = {"fused": "kda_prefill (K1+K2: kda_chunk_intra_act<128,4,bf16> + kda_chunk_state<128,1>)",
             "chunk": "kda_prep2 + kda_chunk (K1, K2)",
             "recurrent": "kda_prep2 + kda_recurrent_kernel<128> (sequential)"}[mode]
    traffic = None
    if mode == "fused":
        traffic = measured_traffic("kda_chunk_intra_act<128, 4, 1>", "kda_chunk_state<128, 1>")
    out = {
        "value": T / step_s, "unit": "tokens/s", "ms_per_step": step_s * 1e3,
        "core_ms_avg": kavg * 1e3, "core_ms_median": ks[len(ks) // 2] * 1e3,
        "core_ms_min": ks[0] * 1e3, "core_ms_max": ks[-1] * 1e3,
        "config": {"workload": "kda_prefill_core", "hidden": c["hidden"], "heads": H, "head_dim": D,
                   "T": T, "chunk": 64, "batch": 1, "conv_k": K, "activations": "bf16",
                   "state": "fp32", "core": kname},
        # The core's algorithmic intensity (flops_per_launch / bytes_per_launch, ~101 FLOP/B)
        # is below MI355X's ridge (2.5 PFLOP/s / 8 TB/s = 312 FLOP/B): the HBM roof binds, so
        # frac is the HBM fraction; the MFMA fraction is kept beside it.
        "roofline": {"kernel": kname, "bound": "hbm", "achieved": bytes_launch / kavg / 1e9,
                     "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": bytes_launch / kavg / HBM_PEAK,
                     "traffic": traffic,
                     "intensity_flop_per_byte": flops_launch / bytes_launch,
                     "ridge_flop_per_byte": BF16_PEAK / HBM_PEAK,
                     "mfma_achieved_TFs": flops_launch / kavg / 1e12, "mfma_peak_TFs": BF16_PEAK / 1e12,
                     "mfma_frac": flops_launch / kavg / BF16_PEAK,
                     "flops_per_launch": flops_launch, "bytes_per_launch": bytes_launch},
    }
    if cpu:   # timed after every GPU workload (its OpenMP threads would load the host)
        out["_cpu"] = lambda: cpu_prefill(torch, q_in, k_in, v_in, z, b_logit, gate, conv, A_log,
                                          dt_bias, o_norm)
    return out


def bench_layer(torch, k3, steps: int, warmup: int, cpu: bool) -> dict:
    """The full k3_kda_layer prefill at T=8192, hidden 4096 on bf16 weights: projections (bf16 MFMA GEMMs),
    K1, K2, K4, o_proj -- k3hip_kda_layer_prefill, x bf16 in, fp32 out, zero initial state."""
    import ctypes as C
    c = PRE
    E, H, D, T, K = c["hidden"], c["H"], c["D"], c["T"], c["K"]
    P = H * D
    g = torch.Generator(device="cuda").manual_seed(0x4B334441 + 2)
    bf = torch.bfloat16
    host = {}
    def mat(name, rows, cols):
        t = (torch.randn((rows, cols), device="cuda", generator=g) * 0.02).to(bf)
        host[name] = t.view(torch.int16).cpu().numpy()
    for n, (r_, c_) in {"q": (P, E), "k": (P, E), "v": (P, E), "g": (P, E), "o": (E, P),
                        "f_a": (D, E), "f_b": (P, D), "b": (H, E)}.items():
        mat(n, r_, c_)
    vec = lambda t: t.float().cpu().numpy().copy()
    host["q_conv"], host["k_conv"], host["v_conv"] = (
        vec(torch.randn((P, K), device="cuda", generator=g) * 0.5) for _ in range(3))
    host["A_log"] = vec(torch.rand((H,), device="cuda", generator=g) * 1.5)
    host["dt_bias"] = vec(torch.randn((P,), device="cuda", generator=g))
    host["o_norm"] = vec(1 + 0.1 * torch.randn((D,), device="cuda", generator=g))
    w = k3.K3KdaW()
    C.memset(C.byref(w), 0, C.sizeof(w))
    for n, a in host.items():
        setattr(w, n, a.ctypes.data)
    w.wdt = 1
    cfg = k3.make_cfg(E, H, D, K, c["gate_lb"], c["rms_eps"])
    dw = k3.DeviceWeights(w, cfg)
    x = torch.randn((T, E), device="cuda", generator=g).to(bf)
    out = torch.empty((T, E), device="cuda", dtype=torch.float32)
    state = torch.zeros(P * D + 3 * P * (K - 1), device="cuda")
    x_host = x.float().cpu().numpy()

    def step():
        state.zero_()
        dw.layer_prefill(out, x, state, T)

    # the default projections (hipBLASLt) and the same step with every projection on the
    # hand-written MFMA GEMM, timed step by step in alternating order: the part's clock falls
    # under seconds of dense MFMA work, so paths timed one after the other would not see the
    # same clock
    paths = (k3.GEMM_HIPBLASLT, k3.GEMM_HANDWRITTEN)
    step()
    torch.cuda.synchronize()
    ramp(torch, step)
    try:
        for p in paths:
            k3.set_projection_gemm(p)
            for _ in range(warmup + 1):
                step()
        torch.cuda.synchronize()
        # one event between consecutive steps, read after the last one (no host wait between
        # steps, which would idle the part and let the clock drop)
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(2 * steps + 1)]
        order = []
        t0 = time.perf_counter()
        evs[0].record()
        for i in range(steps):
            for p in (paths if i % 2 == 0 else paths[::-1]):
                k3.set_projection_gemm(p)
                step()
                evs[len(order) + 1].record()
                order.append(p)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        times = {p: [] for p in paths}
        for n, p in enumerate(order):
            times[p].append(evs[n].elapsed_time(evs[n + 1]) * 1e-3)
    finally:
        k3.set_projection_gemm(k3.GEMM_HIPBLASLT)
    step_s = sum(times[paths[0]]) / steps
    hw_s = sum(times[paths[1]]) / steps
    flops = layer_flops_per_token(E, H, D, 64) * T
    dw.close()
    dropin = bench_dropin(torch, k3, w, cfg, x_host)
    out_d = {
        "value": T / step_s, "unit": "tokens/s", "ms_per_step": step_s * 1e3,
        "wall_ms_per_step": wall / (2 * steps) * 1e3,
        "timing": "both projection paths timed step by step in alternating order (HIP events per step); "
                  "wall_ms_per_step is the wall clock over both paths' steps",
        "config": {"workload": "kda_layer_prefill", "hidden": E, "heads": H, "head_dim": D, "T": T,
                   "chunk": 64, "batch": 1, "conv_k": K, "weights": "bf16", "activations": "bf16 in",
                   "intermediates": "fp32; f_a as a bf16 hi/lo pair into f_b; y in fp16 into o_proj (fp16 copy of W_o)"},
        "roofline": {"kernel": "k3hip_kda_layer_prefill (full layer, full-layer accounting)",
                     "bound": "mfma", "achieved": flops / step_s / 1e12, "peak": BF16_PEAK / 1e12,
                     "unit": "TFLOP/s", "frac": flops / step_s / BF16_PEAK, "traffic": None,
                     "flops_per_step": flops},
        "hand_written_gemms": {"ms_per_step": hw_s * 1e3, "tokens_per_s": T / hw_s,
                               "frac_bf16_peak": flops / hw_s / BF16_PEAK,
                               "note": "the same step with every projection on k3hip_proj_gemm's kernel"},
        "dropin": dropin,
    }
    if cpu:   # timed after every GPU workload
        out_d["_cpu"] = lambda: cpu_layer(host, x_host)
    return out_d


def bench_dropin(torch, k3, w, cfg, x_host) -> dict:
    """The drop-in k3_kda_layer itself (host pointers, the reference's signature) on the layer
    workload's bf16 weights: a T=8192 prefill from a zero state and single-token decode calls
    from the state it leaves, timed on the host clock around each call (its weight upload, the
    host-to-device and device-to-host copies and the compute: the call is synchronous)."""
    import numpy as np
    T, E = x_host.shape
    P = cfg.kda_heads * cfg.kda_head_dim
    nst = P * cfg.kda_head_dim + 3 * P * (cfg.conv_k - 1)
    out = np.empty((T, E), np.float32)
    st = np.zeros(nst, np.float32)
    k3.kda_layer_host(out, x_host, w, cfg, T, st)   # first call: page-in and kernel loads
    pre = []
    for _ in range(3):
        st[:] = 0
        t0 = time.perf_counter()
        k3.kda_layer_host(out, x_host, w, cfg, T, st)
        pre.append(time.perf_counter() - t0)
    moved = k3.dropin_bytes()
    dec = []
    o1 = np.empty((1, E), np.float32)
    for i in range(10):
        x1 = np.ascontiguousarray(x_host[i:i + 1])
        t0 = time.perf_counter()
        k3.kda_layer_host(o1, x1, w, cfg, 1, st)
        dec.append(time.perf_counter() - t0)
    moved1 = k3.dropin_bytes()
    p_ms, d_ms = 1e3 * sorted(pre)[1], 1e3 * sorted(dec)[len(dec) // 2]
    return {"prefill_ms": p_ms, "prefill_tokens_per_s": T / (p_ms * 1e-3), "prefill_bytes_moved": moved,
            "decode_ms_per_call": d_ms, "decode_bytes_moved": moved1,
            "config": {"entry_point": "k3_kda_layer (host pointers)", "hidden": E, "heads": cfg.kda_heads,
                       "head_dim": cfg.kda_head_dim, "T": T, "weights": "bf16",
                       "projections": "T >= 16: bf16 MFMA GEMMs of x split into bf16 hi + lo (fp32 accuracy); "
                                      "T = 1: double-accumulating GEMV"},
            "note": "median host time per call; every call uploads the layer's weights (the reference binds "
                    "them per call) and copies x, out and the state between host and device"}


def cpu_layer(host: dict, x) -> dict:
    """The reference's own k3_kda_layer (src/core/k3_ops.c:864-951, compiled from its sources
    into oracle/_ref; the C restatement where that is absent) on the same bf16 weights and
    the first Ts tokens of the same input: a prefill of Ts tokens from a zero state, Ts
    doubled until the call takes a few seconds."""
    import numpy as np
    sys.path.insert(0, str(REPO / "oracle"))
    import k3_oracle as ko
    c = PRE
    ci = cpu_info()
    nt = ci["threads"]
    set_omp_threads(nt)
    L, kind = ko.ref(), "reference"
    if L is None:
        L, kind = ko.orc(), "port"
    arrays = {n: (a.view(np.uint16) if a.dtype == np.int16 else a) for n, a in host.items()}
    W = ko.Weights(arrays, 1)
    cfg = ko.make_cfg(c["hidden"], c["H"], c["D"], c["K"], c["gate_lb"], c["rms_eps"])
    P = c["H"] * c["D"]
    Ts = 8
    while True:
        st = np.zeros(P * c["D"] + 3 * P * (c["K"] - 1), np.float32)
        t0 = time.perf_counter()
        ko.kda_layer(L, np.ascontiguousarray(x[:Ts]), W, cfg, Ts, st)
        el = time.perf_counter() - t0
        if el > 8.0 or Ts >= len(x):
            break
        Ts = min(len(x), Ts * 2)
    return {"value": Ts / el, "unit": "tokens/s", "cores": nt, "kind": kind, "cpu": ci["model"],
            "physical_cores": ci["physical_cores"], "physical_cores_in_share": ci["physical_cores_in_share"],
            "sample": f"k3_kda_layer ({'reference C from its own sources' if kind == 'reference' else 'C oracle'}) "
                      f"prefill of the first {Ts} of {c['T']} tokens, hidden {c['hidden']}, H={c['H']}, "
                      f"D={c['D']}, bf16 weights, zero state, OpenMP {nt} threads, {el:.2f} s"}


def bench_small(torch, k3, steps: int, warmup: int, cpu: bool) -> dict:
    """The small CPU-runnable layer: one KDA layer on fp32 weights N(0, 0.02) (hidden 256, H=4,
    D=64, conv 4), a 32-token prefill then 8 single-token decode steps carrying the state,
    x N(0, 1), A_log U(0, 1.5), dt_bias N(0, 1) -- nine k3hip_kda_layer_dev calls per step."""
    import ctypes as C
    import numpy as np
    c = SMALL
    E, H, D, K, T, ND = c["hidden"], c["H"], c["D"], c["K"], c["T"], c["decode"]
    P = H * D
    rng = np.random.default_rng(0x4B334441 + 0)
    nrm = lambda *s: (rng.standard_normal(s) * 0.02).astype(np.float32)
    host = {"q": nrm(P, E), "k": nrm(P, E), "v": nrm(P, E), "g": nrm(P, E), "o": nrm(E, P), "f_a": nrm(D, E),
            "f_b": nrm(P, D), "b": nrm(H, E), "q_conv": nrm(P, K), "k_conv": nrm(P, K), "v_conv": nrm(P, K),
            "A_log": rng.uniform(0, 1.5, H).astype(np.float32),
            "dt_bias": rng.standard_normal(P).astype(np.float32),
            "o_norm": (1 + 0.02 * rng.standard_normal(D)).astype(np.float32)}
    w = k3.K3KdaW()
    C.memset(C.byref(w), 0, C.sizeof(w))
    for n, a in host.items():
        setattr(w, n, a.ctypes.data)
    w.wdt = 0
    cfg = k3.make_cfg(E, H, D, K, c["gate_lb"], c["rms_eps"])
    dw = k3.DeviceWeights(w, cfg, k3.UPLOAD_DEV)
    xs = rng.standard_normal((T + ND, E)).astype(np.float32)
    x = torch.from_numpy(xs).cuda()
    out = torch.empty((T + ND, E), device="cuda")
    state = torch.zeros(P * D + 3 * P * (K - 1), device="cuda")

    def step():
        state.zero_()
        dw.layer(out[:T], x[:T], state, T)
        for t in range(T, T + ND):
            dw.layer(out[t:t + 1], x[t:t + 1], state, 1)

    step()
    torch.cuda.synchronize()
    ramp(torch, step)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = ev_pair(torch)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    step_s = e0.elapsed_time(e1) * 1e-3 / steps
    dw.close()
    out_d = {"value": (T + ND) / step_s, "unit": "tokens/s", "ms_per_step": step_s * 1e3,
             "config": {"workload": "kda_small_layer", "hidden": E, "heads": H, "head_dim": D, "conv_k": K,
                        "prefill_T": T, "decode_steps": ND, "weights": "fp32", "activations": "fp32",
                        "entry_point": "k3hip_kda_layer_dev (exact-order fp32 projections), nine calls per step",
                        "note": "launch-bound at this size"}}
    if cpu:
        out_d["_cpu"] = lambda: cpu_small(host, xs)
    return out_d


def cpu_small(host: dict, xs) -> dict:
    """The reference's own k3_kda_layer (compiled from its sources into oracle/_ref; the C
    restatement where that is absent) on the same sequence: the 32-token prefill then 8
    single-token steps, repeated for a few seconds."""
    import numpy as np
    sys.path.insert(0, str(REPO / "oracle"))
    import k3_oracle as ko
    c = SMALL
    ci = cpu_info()
    nt = ci["threads"]
    set_omp_threads(nt)
    L, kind = ko.ref(), "reference"
    if L is None:
        L, kind = ko.orc(), "port"
    W = ko.Weights(dict(host), 0)
    cfg = ko.make_cfg(c["hidden"], c["H"], c["D"], c["K"], c["gate_lb"], c["rms_eps"])
    P, T, ND = c["H"] * c["D"], c["T"], c["decode"]
    n, t0 = 0, time.perf_counter()
    while True:
        st = np.zeros(P * c["D"] + 3 * P * (c["K"] - 1), np.float32)
        ko.kda_layer(L, np.ascontiguousarray(xs[:T]), W, cfg, T, st)
        for t in range(T, T + ND):
            ko.kda_layer(L, np.ascontiguousarray(xs[t:t + 1]), W, cfg, 1, st)
        n += 1
        el = time.perf_counter() - t0
        if el > 3.0:
            break
    return {"value": n * (T + ND) / el, "unit": "tokens/s", "cores": nt, "kind": kind, "cpu": ci["model"],
            "physical_cores": ci["physical_cores"], "physical_cores_in_share": ci["physical_cores_in_share"],
            "sample": f"k3_kda_layer ({'reference C from its own sources' if kind == 'reference' else 'C oracle'}), "
                      f"{n} sequences of a {T}-token prefill + {ND} decode steps, hidden {c['hidden']}, "
                      f"H={c['H']}, D={c['D']}, fp32 weights, OpenMP {nt} threads, {el:.2f} s"}


def bench_hybrid(torch, k3, steps: int, warmup: int, cpu: bool = False) -> dict:
    """Hybrid slice: one decode step of batch 16 through 3 KDA layers (k3hip_kda_layer_decode) and one
    gated MLA layer with absorbed weights over an 8192-position latent cache
    (k3hip_mla_decode), hidden 7168, bf16 weights N(0, 0.02). Each part is timed with HIP
    events over `steps` back-to-back steps. Bytes: each layer's weights once + its
    state / cache traffic."""
    import ctypes as C
    c = HYB
    E, B, ctx = c["hidden"], c["B"], c["ctx"]
    H, D, K = c["H"], c["D"], c["K"]
    P = H * D
    g = torch.Generator(device="cuda").manual_seed(0x4B334441 + 4)
    bf = torch.bfloat16

    def host_bf16(rows, cols):
        return (torch.randn((rows, cols), device="cuda", generator=g) * 0.02).to(bf).view(torch.int16).cpu().numpy()

    def host_f32(t):
        return t.float().cpu().numpy().copy()

    keep = []
    kcfg = k3.make_cfg(E, H, D, K, c["gate_lb"], 1e-5)
    kdas = []
    for _ in range(c["kda_layers"]):
        a = {n: host_bf16(r_, c_) for n, (r_, c_) in {"q": (P, E), "k": (P, E), "v": (P, E), "g": (P, E),
                                                      "o": (E, P), "f_a": (D, E), "f_b": (P, D), "b": (H, E)}.items()}
        a["q_conv"], a["k_conv"], a["v_conv"] = (host_f32(torch.randn((P, K), device="cuda", generator=g) * 0.5) for _ in range(3))
        a["A_log"] = host_f32(torch.rand((H,), device="cuda", generator=g) * 1.5)
        a["dt_bias"] = host_f32(torch.randn((P,), device="cuda", generator=g))
        a["o_norm"] = host_f32(1 + 0.1 * torch.randn((D,), device="cuda", generator=g))
        w = k3.K3KdaW()
        C.memset(C.byref(w), 0, C.sizeof(w))
        for n, arr in a.items():
            setattr(w, n, arr.ctypes.data)
        w.wdt = 1
        kdas.append(k3.DeviceWeights(w, kcfg))
        keep.append(a)
    Hm, QL, KL, QN, QR, VH = c["mla_heads"], c["q_lora"], c["kv_lora"], c["qk_nope"], c["qk_rope"], c["v_head"]
    mcfg = k3.make_cfg(E, 1, 16, 1, -5.0, 1e-5)
    mcfg.n_heads, mcfg.q_lora, mcfg.kv_lora, mcfg.qk_nope, mcfg.qk_rope, mcfg.v_head, mcfg.mla_out_gate = \
        Hm, QL, KL, QN, QR, VH, 1
    ma = {n: host_bf16(r_, c_) for n, (r_, c_) in {"q_a": (QL, E), "q_b": (Hm * (QN + QR), QL), "kv_a": (KL + QR, E),
                                                    "kv_b": (Hm * (QN + VH), KL), "o": (E, Hm * VH), "g": (Hm * VH, E)}.items()}
    ma["q_a_norm"] = host_f32(1 + 0.1 * torch.randn((QL,), device="cuda", generator=g))
    ma["kv_a_norm"] = host_f32(1 + 0.1 * torch.randn((KL,), device="cuda", generator=g))
    mw_ = k3.K3MlaW()
    C.memset(C.byref(mw_), 0, C.sizeof(mw_))
    for n, arr in ma.items():
        setattr(mw_, n, arr.ctypes.data)
    mw_.wdt = 1
    mla = k3.MlaWeights(mw_, mcfg)
    keep.append(ma)
    kper = P * D + 3 * P * (K - 1)
    states = [torch.zeros((B, kper), device="cuda") for _ in kdas]
    cache = torch.randn((B, ctx, KL + QR), device="cuda", generator=g)
    x = torch.randn((B, E), device="cuda", generator=g)
    hbuf = [torch.empty((B, E), device="cuda") for _ in range(len(kdas) + 1)]

    def kda_part():
        h = x
        for i, dw in enumerate(kdas):
            dw.layer_decode(hbuf[i], h, states[i], kper)
            h = hbuf[i]
        return h

    def mla_part(h):
        mla.decode(hbuf[-1], h, cache, ctx - 1, ctx)

    h = kda_part()
    mla_part(h)
    torch.cuda.synchronize()
    ramp(torch, lambda: mla_part(kda_part()))
    for _ in range(warmup):
        mla_part(kda_part())
    torch.cuda.synchronize()
    evs = [ev_pair(torch) for _ in range(2)]
    evs[0][0].record()
    for _ in range(steps):
        h = kda_part()
    evs[0][1].record()
    evs[1][0].record()
    for _ in range(steps):
        mla_part(h)
    evs[1][1].record()
    torch.cuda.synchronize()
    kda_s = evs[0][0].elapsed_time(evs[0][1]) * 1e-3 / steps
    mla_s = evs[1][0].elapsed_time(evs[1][1]) * 1e-3 / steps
    kda_w = (4 * P * E + E * P + D * E + P * D + H * E) * 2
    kda_bytes = len(kdas) * (kda_w + 2 * B * kper * 4)
    mla_w = (QL * E + Hm * (QN + QR) * QL + (KL + QR) * E + Hm * (QN + VH) * KL + 2 * E * Hm * VH) * 2
    mla_bytes = mla_w + B * ctx * (KL + QR) * 4
    for dw in kdas:
        dw.close()
    mla.close()
    res = {
        "config": {"workload": "hybrid_decode_slice", "hidden": E, "batch": B, "context": ctx,
                   "kda_layers": len(kdas), "kda_heads": H, "kda_head_dim": D,
                   "mla_heads": Hm, "kv_lora": KL, "qk_rope": QR, "qk_nope": QN, "v_head": VH, "q_lora": QL,
                   "weights": "bf16 N(0,0.02)", "mla_cache": "compressed latent + rope slot, fp32"},
        "kda_ms_per_step": kda_s * 1e3, "kda_ms_per_layer": kda_s * 1e3 / len(kdas),
        "mla_ms_per_step": mla_s * 1e3, "mla_over_kda_layer": mla_s / (kda_s / len(kdas)),
        "tokens_per_s": B / (kda_s + mla_s),
        "kda_hbm_frac": kda_bytes / kda_s / HBM_PEAK, "mla_hbm_frac": mla_bytes / mla_s / HBM_PEAK,
        "kda_bytes_per_step": kda_bytes, "mla_bytes_per_step": mla_bytes,
    }
    if cpu:   # timed after every GPU workload
        res["_cpu"] = lambda: cpu_hybrid(keep[0], keep[-1])
    return res


def cpu_hybrid(kda_host: dict, mla_host: dict) -> dict:
    """The reference's own k3_kda_layer and k3_mla_cached (src/core/k3_ops.c:864-951,
    :321-424, from oracle/_ref; the C restatement where that is absent) on the hybrid
    slice's bf16 weights, one sequence at a time as the reference decodes: KDA decode tokens
    (T = 1, state carried) until ~3 s, then MLA decode tokens over a cache of the slice's
    context in the reference's expanded layout (H (nope + v) floats per position, random
    contents), until ~3 s. Slice tokens/s = 1 / (3 t_kda + t_mla)."""
    import numpy as np
    sys.path.insert(0, str(REPO / "oracle"))
    import k3_oracle as ko
    c = HYB
    ci = cpu_info()
    nt = ci["threads"]
    set_omp_threads(nt)
    lib = "ref" if ko.ref() is not None else "orc"
    L = ko.ref() if lib == "ref" else ko.orc()
    arrays = {n: (a.view(np.uint16) if a.dtype == np.int16 else a) for n, a in kda_host.items()}
    W = ko.Weights(arrays, 1)
    E, H, D, K = c["hidden"], c["H"], c["D"], c["K"]
    cfg = ko.make_cfg(E, H, D, K, c["gate_lb"], 1e-5)
    P = H * D
    st = np.zeros(P * D + 3 * P * (K - 1), np.float32)
    rng = np.random.default_rng(7)
    x = rng.standard_normal((1, E)).astype(np.float32)
    n_kda, t0 = 0, time.perf_counter()
    while True:
        ko.kda_layer(L, x, W, cfg, 1, st)
        n_kda += 1
        if time.perf_counter() - t0 > 3.0:
            break
    t_kda = (time.perf_counter() - t0) / n_kda
    MW = ko.MlaWeights({n: (a.view(np.uint16) if a.dtype == np.int16 else a) for n, a in mla_host.items()}, 1)
    ctx = c["ctx"]
    Hm, QN, QR, VH = c["mla_heads"], c["qk_nope"], c["qk_rope"], c["v_head"]
    mcfg = ko.mla_cfg(E, Hm, c["q_lora"], c["kv_lora"], QN, QR, VH, 1e-5, 1)
    kvc = rng.standard_normal((ctx, Hm * (QN + VH)), dtype=np.float32)
    ropec = rng.standard_normal((ctx, QR), dtype=np.float32)
    n_mla, t0 = 0, time.perf_counter()
    while True:
        ko.mla(x, MW, mcfg, 1, kvc, ropec, ctx - 1, ctx, lib=lib)
        n_mla += 1
        if time.perf_counter() - t0 > 3.0:
            break
    t_mla = (time.perf_counter() - t0) / n_mla
    kind = "reference" if lib == "ref" else "port"
    return {"value": 1.0 / (c["kda_layers"] * t_kda + t_mla), "unit": "tokens/s", "cores": nt, "kind": kind,
            "cpu": ci["model"], "physical_cores": ci["physical_cores"],
            "physical_cores_in_share": ci["physical_cores_in_share"],
            "kda_ms_per_layer_token": t_kda * 1e3, "mla_ms_per_token": t_mla * 1e3,
            "sample": f"{'reference C from its own sources' if kind == 'reference' else 'C oracle'}: "
                      f"{n_kda} k3_kda_layer decode tokens (hidden {E}, H={H}, D={D}) and {n_mla} "
                      f"k3_mla_cached decode tokens over {ctx} cached positions (64 heads, expanded "
                      f"cache), one sequence at a time, OpenMP {nt} threads"}


def cpu_prefill(torch, q_in, k_in, v_in, z, b_logit, gate, conv, A_log, dt_bias, o_norm) -> dict:
    """orc_kda_core (conv .. gate, the same steps as the GPU step) on the first Ts tokens."""
    import numpy as np
    sys.path.insert(0, str(REPO / "oracle"))
    import k3_oracle as ko
    c = PRE
    H, D, K = c["H"], c["D"], c["K"]
    ci = cpu_info()
    nt = ci["threads"]
    cfg = ko.make_cfg(c["hidden"], H, D, K, c["gate_lb"], c["rms_eps"])
    arrays = {"q_conv": conv[0].cpu().numpy(), "k_conv": conv[1].cpu().numpy(),
              "v_conv": conv[2].cpu().numpy(), "A_log": A_log.cpu().numpy(),
              "dt_bias": dt_bias.cpu().numpy(), "o_norm": o_norm.cpu().numpy()}
    for n in ("q", "k", "v", "g", "f_a", "f_b", "b", "o"):
        arrays[n] = np.zeros((1, 1), np.float32)
    W = ko.Weights(arrays, 0)
    Ts, runs = 64, []
    while True:
        sl = lambda t: t[:Ts].float().cpu().numpy()
        ins = [sl(q_in), sl(k_in), sl(v_in), sl(z), sl(b_logit), sl(gate)]
        t0 = time.perf_counter()
        ko.core(*ins, W, cfg, Ts, None, nt)
        el = time.perf_counter() - t0
        runs.append((Ts, el))
        if el > 3.0 or Ts >= c["T"]:
            break
        Ts = min(c["T"], Ts * 4)
    Ts, el = runs[-1]
    return {"value": Ts / el, "unit": "tokens/s", "cores": nt, "kind": "port",
            "cpu": ci["model"], "physical_cores": ci["physical_cores"],
            "physical_cores_in_share": ci["physical_cores_in_share"],
            "sample": f"C oracle orc_kda_core (conv+SiLU, L2, beta, decay, sequential recurrence, "
                      f"RMSNorm, gate) on the first {Ts} of {c['T']} tokens, H={H}, D={D}, "
                      f"OpenMP over heads, {el:.2f} s"}


def bench_long(torch, k3, steps: int, warmup: int, cpu: bool) -> dict:
    """Long context, the core alone: one prefill of T=65,536 tokens (fused K1+K2 -> K4, bf16
    activations, zero state), then 256 single-token decode steps of the same sequence, H=32,
    D=128. A decode step is one k3hip_kda_decode_step launch (K1 at T=1 with the conv history
    carried, K3 at B=1, K4); the 256 launches are captured in one HIP graph and its replay is
    timed with HIP events (device time per token), beside the same launches issued one by one
    from Python (host-bound)."""
    c = PRE
    H, D, K, T, ND = c["H"], c["D"], c["K"], LONG["T"], LONG["decode"]
    P, Ta = H * D, LONG["T"] + LONG["decode"]
    g = torch.Generator(device="cuda").manual_seed(0x4B334441 + 3)
    bf = torch.bfloat16
    q_in, k_in, v_in = (torch.randn((Ta, P), device="cuda", generator=g).to(bf) for _ in range(3))
    z = torch.randn((Ta, P), device="cuda", generator=g) * 0.02
    b_logit = torch.randn((Ta, H), device="cuda", generator=g)
    gate = torch.randn((Ta, P), device="cuda", generator=g).to(bf)
    conv = [torch.randn((P, K), device="cuda", generator=g) * 0.5 for _ in range(3)]
    A_log = torch.rand((H,), device="cuda", generator=g) * 1.5
    dt_bias = torch.randn((P,), device="cuda", generator=g)
    o_norm = 1 + 0.1 * torch.randn((D,), device="cuda", generator=g)
    f32 = dict(device="cuda", dtype=torch.float32)
    S = torch.zeros((H, D, D), **f32)
    cs = torch.zeros(3 * P * (K - 1), **f32)
    o = torch.empty((T, P), **f32)
    y = torch.empty((T, P), device="cuda", dtype=bf)
    ws = torch.empty(k3.kda_chunk_workspace(T, H, D, 64), dtype=torch.uint8, device="cuda")
    qs = 1.0 / math.sqrt(D)
    # decode tail: the state as one B=1 slot, one output row per token
    S1, cs1 = S.view(1, H, D, D), cs.view(1, -1)
    y_dec = torch.empty((ND, P), device="cuda", dtype=bf)

    def prefill():
        S.zero_()
        cs.zero_()
        k3.kda_prefill(q_in[:T], k_in[:T], v_in[:T], z[:T], b_logit[:T], conv[0], conv[1], conv[2], A_log,
                       dt_bias, cs, S, o, H, D, K, c["gate_lb"], qs, ws)
        k3.kda_epilogue(o, gate[:T], o_norm, y, H, D, c["rms_eps"])

    def tail():
        for i in range(ND):
            t = T + i
            k3.kda_decode_step(q_in[t:t + 1], k_in[t:t + 1], v_in[t:t + 1], z[t:t + 1], b_logit[t:t + 1],
                               gate[t:t + 1], conv[0], conv[1], conv[2], A_log, dt_bias, o_norm, cs1, S1,
                               y_dec[i:i + 1], H, D, K, c["gate_lb"], c["rms_eps"], qs)

    prefill()
    tail()
    torch.cuda.synchronize()
    # the 256 decode launches as one graph (no memset nodes: the step kernel only reads and
    # writes its operands), captured after an eager pass on the capture's side stream
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        tail()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        tail()
    torch.cuda.synchronize()
    ramp(torch, prefill)
    for _ in range(warmup):
        prefill()
        graph.replay()
    torch.cuda.synchronize()
    e0, e1 = ev_pair(torch)
    pre_ms, dec_ms, eager_ms = [], [], []
    for _ in range(steps):
        e0.record()
        prefill()
        e1.record()
        torch.cuda.synchronize()
        pre_ms.append(e0.elapsed_time(e1))
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        dec_ms.append(e0.elapsed_time(e1) / ND)
        e0.record()
        tail()
        e1.record()
        torch.cuda.synchronize()
        eager_ms.append(e0.elapsed_time(e1) / ND)
    pre, dec, eager = sum(pre_ms) / steps, sum(dec_ms) / steps, sum(eager_ms) / steps
    floor_us = decode_bytes_per_token(H, D) / HBM_PEAK * 1e6
    out = {
        "prefill_tokens_per_s": T / (pre * 1e-3), "prefill_ms": pre,
        "decode_tail_ms_per_token": dec,
        "decode_tail_hbm_floor_ms_per_token": floor_us * 1e-3,
        "decode_tail_roofline_frac": floor_us * 1e-3 / dec,
        "decode_tail_eager_ms_per_token": eager,
        "decode_tail_note": "one k3hip_kda_decode_step launch per token at B=1 (32 workgroups, one per head); "
                            "the 256 launches replayed as one HIP graph, HIP events around the replay; the eager "
                            "figure issues the same launches one by one from Python (host-bound)",
        "config": {"workload": "kda_long_context", "heads": H, "head_dim": D, "T": T, "decode_steps": ND,
                   "chunk": 64, "conv_k": K, "activations": "bf16", "state": "fp32",
                   "workspace_bytes": k3.kda_chunk_workspace(T, H, D, 64),
                   "step": "prefill = k3hip_kda_prefill + k3hip_kda_epilogue; decode token = "
                           "k3hip_kda_decode_step (K1 at T=1 + K3 at B=1 + K4, one launch)"},
    }
    del ws
    if cpu:
        host = [t.cpu() for t in (q_in, k_in, v_in, z, b_logit, gate)] + [
            t.cpu() for t in (*conv, A_log, dt_bias, o_norm)]
        out["_cpu"] = lambda: cpu_long(host)
    return out


def cpu_long(host) -> dict:
    """orc_kda_core over all 65,792 tokens (the prefill's and the decode tail's steps, one
    sequential recurrence from zero state)."""
    import numpy as np
    sys.path.insert(0, str(REPO / "oracle"))
    import k3_oracle as ko
    c = PRE
    H, D, K = c["H"], c["D"], c["K"]
    Ta = LONG["T"] + LONG["decode"]
    ci = cpu_info()
    nt = ci["threads"]
    cfg = ko.make_cfg(c["hidden"], H, D, K, c["gate_lb"], c["rms_eps"])
    q_in, k_in, v_in, z, bl, gate, qc, kc, vc, A_log, dt_bias, o_norm = host
    arrays = {"q_conv": qc.numpy(), "k_conv": kc.numpy(), "v_conv": vc.numpy(), "A_log": A_log.numpy(),
              "dt_bias": dt_bias.numpy(), "o_norm": o_norm.numpy()}
    for n in ("q", "k", "v", "g", "f_a", "f_b", "b", "o"):
        arrays[n] = np.zeros((1, 1), np.float32)
    W = ko.Weights(arrays, 0)
    ins = [t.float().numpy() for t in (q_in, k_in, v_in, z, bl, gate)]
    t0 = time.perf_counter()
    ko.core(*ins, W, cfg, Ta, None, nt)
    el = time.perf_counter() - t0
    return {"value": Ta / el, "unit": "tokens/s", "cores": nt, "kind": "port", "cpu": ci["model"],
            "physical_cores": ci["physical_cores"], "physical_cores_in_share": ci["physical_cores_in_share"],
            "sample": f"C oracle orc_kda_core over all {Ta} tokens (the prefill's and the decode tail's), "
                      f"H={H}, D={D}, OpenMP over heads, {el:.2f} s"}


def bench_gemm(torch, k3, steps: int) -> dict:
    """The layer's projection shapes at T=8192, hidden 4096 on the hand-written MFMA GEMM
    (k3hip_proj_gemm) and on hipBLASLt (torch.mm, fp32 output), bf16 operands N(0,1), each
    timed with HIP events over `steps` back-to-back calls after a clock ramp."""
    g = torch.Generator(device="cuda").manual_seed(0x4B334441 + 5)
    res = {}
    for name, (M, N, K) in {"qkv": (8192, 12288, 4096), "gate_or_o_proj": (8192, 4096, 4096),
                            "z": (8192, 4096, 256)}.items():
        a = torch.randn((M, K), device="cuda", generator=g).to(torch.bfloat16)
        b = torch.randn((N, K), device="cuda", generator=g).to(torch.bfloat16)
        c = torch.empty((M, N), device="cuda")
        row = {"M": M, "N": N, "K": K}
        for impl, fn in (("hand_written_mfma", lambda: k3.proj_gemm(a, b, c)),
                         ("hipblaslt", lambda: torch.mm(a, b.t(), out_dtype=torch.float32))):
            fn()
            ramp(torch, fn)
            e0, e1 = ev_pair(torch)
            e0.record()
            for _ in range(steps):
                fn()
            e1.record()
            torch.cuda.synchronize()
            s = e0.elapsed_time(e1) * 1e-3 / steps
            row[impl] = {"us": s * 1e6, "TFLOP_s": 2.0 * M * N * K / s / 1e12,
                         "frac_bf16_peak": 2.0 * M * N * K / s / BF16_PEAK}
        res[name] = row
    return res


def bench_copy(torch, steps: int) -> dict:
    """A plain device-to-device copy of 1 GiB: the calibration kernel for the HBM traffic
    counters (FETCH_SIZE / WRITE_SIZE read per byte actually moved)."""
    n = 1 << 28
    src = torch.empty(n, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = ev_pair(torch)
    e0.record()
    for _ in range(steps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    s = e0.elapsed_time(e1) * 1e-3 / steps
    return {"bytes_per_copy": 4 * n, "read_bytes": 4 * n, "write_bytes": 4 * n,
            "ms": s * 1e3, "GBs_rw": 8 * n / s / 1e9}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=["all", "prefill", "decode", "layer", "hybrid", "long", "small", "copy",
                                           "gemm"],
                    default="all", help="copy: the 1 GiB device copy used to calibrate HBM traffic counters; "
                    "gemm: the layer's projection shapes on the hand-written GEMM and on hipBLASLt")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: the benchmark runs on one GPU (the path is measured per GPU); run with --gpus 1", file=sys.stderr)
        return 2
    import torch
    import k3kda as k3
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 2
    k3.lib()
    if a.workload == "copy":
        print(json.dumps({"workload": "copy_calibration", **bench_copy(torch, a.steps)}))
        return 0
    if a.workload == "gemm":
        print(json.dumps({"workload": "projection_gemms", **bench_gemm(torch, k3, a.steps)}))
        return 0
    res = {}
    if a.workload in ("all", "decode"):
        # 1,000 launches (~48 ms) per repeat: the host's synchronize after a repeat then adds
        # well under 0.1 us per launch to the wall figure (50 launches: ~0.6 us)
        res["decode"] = bench_decode(torch, k3, max(a.steps, 1000), a.warmup + 2, not a.no_cpu)
    if a.workload in ("all", "prefill"):
        res["prefill"] = bench_prefill(torch, k3, a.steps, a.warmup, not a.no_cpu)
    # the streaming (HBM-bound) workloads before the layer: its seconds of dense MFMA leave the
    # GPU power-limited for a while, which measured the hybrid slice ~5% slower after it
    if a.workload in ("all", "hybrid"):
        res["hybrid"] = bench_hybrid(torch, k3, a.steps, a.warmup, not a.no_cpu)
    if a.workload in ("all", "long"):
        res["long_context"] = bench_long(torch, k3, 3, 1, not a.no_cpu)
        torch.cuda.empty_cache()
    if a.workload in ("all", "small"):
        res["small_layer"] = bench_small(torch, k3, a.steps, a.warmup, not a.no_cpu)
    if a.workload in ("all", "layer"):
        res["layer"] = bench_layer(torch, k3, max(3, a.steps // 2), a.warmup, not a.no_cpu)
    for r in res.values():   # CPU baselines last, after all GPU timing
        f = r.pop("_cpu", None)
        if f is not None:
            r["cpu_baseline"] = f()
    head = res.get("prefill") or res.get("layer") or res.get("decode")
    if head is None:   # hybrid, long context or the small layer alone
        name = next(iter(res))
        print(json.dumps({"workload": name, **res[name]}))
        return 0
    line = {
        "metric": "KDA prefill tokens/s (H=32,d=128,T=8k) + decode state-update GB/s, 1 GPU",
        "value": head["value"], "unit": head["unit"], "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": head["ms_per_step"], "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 in, split-bf16 MFMA (hi/lo pairs, fp32 accumulation), fp32 state",
        "data": "synthetic (torch Philox on device, distributions of the benchmark configs)",
        "config": head["config"], "roofline": head["roofline"],
        "cpu_baseline": head.get("cpu_baseline"),
        "device": torch.cuda.get_device_name(0),
    }
    if head is res.get("layer"):
        line["hand_written_gemms"] = head["hand_written_gemms"]
        line["dropin"] = head["dropin"]
    if "prefill" in res and "decode" in res:
        line["decode"] = res["decode"]
    if "layer" in res and head is not res["layer"]:
        line["layer"] = res["layer"]
    if "hybrid" in res:
        line["hybrid"] = res["hybrid"]
    if "long_context" in res:
        line["long_context"] = res["long_context"]
    if "small_layer" in res:
        line["small_layer"] = res["small_layer"]
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
