#!/usr/bin/env python3
"""Benchmark of the attention + Gated DeltaNet hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--decode-steps N]

One bench step is one pass over the hot path with every input already resident in HBM:
  * attention forward, B=1 H=32 S=8192 D=128 causal, fp16, N(0, 0.5) with 1% of the
    entries x8 (outlier stress), fp32 softmax statistics;
  * chunked Gated DeltaNet prefill, B=1 T=4096 Hq=16 Hv=32 dk=dv=128 C=64, fp16 q/k/v
    (q, k rows L2-normalised), beta = sigmoid(N(0,1)), g_log = -softplus(N(0,1)), fp32
    state from zero;
  * 16 Gated DeltaNet decode steps for 16 sequences x 32 V-heads (128x128 fp32 state each,
    N(0, 0.02)), one per state replica (16 replicas, 512 MiB > the 256 MiB Infinity
    Cache) so every step streams its state from HBM.
The decode part's figure is the decode workload itself, timed after the step: 512 decode
steps back to back, each with its own pre-generated token (fresh q, k, v, g, beta per step),
cycling the 16 replicas, between one pair of events (a serving loop's step time, not one
launch's latency); the 16 in-step launches are reported beside it.
W untimed warmup steps (default 50, grouped by part with attention last; attention itself
always gets at least ATTN_MIN_WARMUP launches back to back, ~45 ms, whatever W is: after an
idle gap the board's power management needs ~12 ms of continuous attention to settle, and a
timed loop inside that transient measures the power controller, not the kernel), then
exactly K timed steps
between two synchronisations, their work grouped by part (K attention launches back to
back, then K prefills, then the K x 16 decode launches), so each kernel is timed in its own
loop as the reference's lab drivers time theirs: a part's average launch duration is one
pair of HIP events around its K launches, on the stream they run on, divided by K (the
prefill's per-call state reset is timed alone the same way and subtracted).
After the timed steps, outside the step, the gated grouped-query attention layer of the
reference's target model (B=1, 24 query / 4 K/V heads, D=256, S=8192, causal, gate after
softmax) is timed on its own and reported as the part `attn_gqa_gated` (GQA_MIN_WARMUP launches
back to back, then GQA_TIMED timed ones: it follows the light decode loop, so like attention it
needs continuous load before its timed launches); so is the GDN
recurrence with the layer's pre/post ops at the prefill shape (`gdn_layer_ops`): raw q/k
and gate projections -> fused chunked prefill -> gated RMSNorm, against the unfused
pipeline (pre-op pass, chunked prefill, gated RMSNorm); and, for context only, one GPU's
share of the prefill under 8-way head sharding (2 QK / 4 V heads, `gdn_prefill_head_shard`:
the call splits the sequence, timed beside the same call without the split) and the GDN
layer at the reference's own published shape (T=512, 16 QK / 48 V heads, its LCG inputs:
token-serial and chunked, `gdn_reference_shape`) beside its 2080 Ti times.
Last (skip with --no-sustained), the attention kernel runs back to back for ~6 s with the
board's socket power and GFX clocks read meanwhile (`attn_fwd.sustained`), and an fp16
8192^3 GEMM through torch (hipBLASLt) runs back to back the same way
(`attn_fwd.mfma_gemm_reference`): the MI355X holds these MFMA-dense loads at its board power
limit, well below the clock the nominal peak assumes, and the vendor GEMM's rate is the
practical MFMA ceiling beside the nominal one.

Printed: one JSON line.  `value` is the attention forward throughput (TFLOP/s, causal
executed FLOPs 2*B*H*S*(S+1)*D, the convention of src/attn_sm75.cu:534), the kernel that
dominates the step; `parts` carries all three components, each with its absolute
throughput, its roofline fraction and a CPU baseline (the oracle, timed on a bounded
sample on this machine's host cores, all threads and one thread).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "turing-sm75_amd"))

PEAK_MFMA_F16_TFLOPS = 2500.0  # MI355X dense fp16 MFMA (no sparsity)
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E
# continuous attention launches right before the timed region, whatever --warmup is (~45 ms
# at config 3; the power controller's start-up transient lasts ~12 ms)
ATTN_MIN_WARMUP = 80
# the same for the gated GQA layer, timed after the light decode loop (~40 ms at 0.81 ms a launch)
GQA_MIN_WARMUP = 50
GQA_TIMED = 20

# configuration of each part
ATTN = dict(B=1, H=32, S=8192, D=128, causal=True)
# the target model's gated attention layer (24 query / 4 K/V heads, head_dim 256)
GQA = dict(B=1, Hq=24, Hkv=4, S=8192, D=256, causal=True)
PREFILL = dict(B=1, T=4096, Hq=16, Hv=32, d=128, chunk=64)
DECODE = dict(B=16, Hq=16, Hv=32, d=128, replicas=16, steps=512)
# the reference's published GDN shape (docs/kernels.md:31-39): T=512, 16 QK / 48 V heads
REF_GDN = dict(B=1, T=512, Hq=16, Hv=48, d=128)
REF_GDN_MS = {"token_serial_occ8": 0.91, "chunked_wmma_cs16": 5.00}  # RTX 2080 Ti, fp32 I/O


def attn_flops(B, H, S, D, causal, **_):
    return 2.0 * B * H * S * (S + 1) * D if causal else 4.0 * B * H * S * S * D


def prefill_flops(B, T, Hq, Hv, d, chunk, **_):
    # per (head, chunk), full (not triangle-halved) products:
    # K K^T, Q K^T, Tm K, Tm V, (M.QK^T) Vnew, W S, Q S, K^T Vnew
    nch = math.ceil(T / chunk)
    per = 2 * chunk * (chunk * (3 * d + 2 * d) + 3 * d * d)
    return float(B * Hv * nch * per)


def prefill_bytes(B, T, Hq, Hv, d, **_):
    return float(2 * B * T * Hq * d * 2 + 2 * B * T * Hv * d * 2 + 2 * B * T * Hv * 4
                 + 2 * B * Hv * d * d * 4)


def rmsnorm_bytes(B, T, Hv, d, **_):
    """Gated RMSNorm: read x and z, write y (fp16 rows of d), plus the fp32 weight."""
    return 3 * B * T * Hv * d * 2 + d * 4


def decode_bytes(B, Hq, Hv, d, **_):
    return float(2 * B * Hv * d * d * 4 + 2 * B * Hq * d * 2 + B * Hv * d * 2 + 2 * B * Hv * 4
                 + B * Hv * d * 2)


def omp_threads():
    env = os.environ.get("OMP_NUM_THREADS", "")
    return int(env) if env.isdigit() and int(env) > 0 else (os.cpu_count() or 1)


def load_traffic():
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, scaled by a
    copy-kernel calibration), committed in profiles/traffic.json; None when absent."""
    p = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(p):
        return {}
    with open(p) as f:
        return json.load(f)


def make_inputs(torch, dev, seed=2026):
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)

    def attn_tensor():
        s = ATTN
        x = 0.5 * torch.randn(s["B"], s["H"], s["S"], s["D"], device=dev, generator=gen)
        x = torch.where(torch.rand(x.shape, device=dev, generator=gen) < 0.01, 8 * x, x)
        return x.half().contiguous()

    def l2n(x):
        return x / x.norm(dim=-1, keepdim=True)

    a = {n: attn_tensor() for n in ("q", "k", "v")}
    a["o"] = torch.empty_like(a["q"])

    p = PREFILL
    pre = dict(
        q=l2n(torch.randn(p["B"], p["T"], p["Hq"], p["d"], device=dev, generator=gen)).half(),
        k=l2n(torch.randn(p["B"], p["T"], p["Hq"], p["d"], device=dev, generator=gen)).half(),
        v=torch.randn(p["B"], p["T"], p["Hv"], p["d"], device=dev, generator=gen).half(),
        beta=torch.sigmoid(torch.randn(p["B"], p["T"], p["Hv"], device=dev, generator=gen)),
        g=-torch.nn.functional.softplus(torch.randn(p["B"], p["T"], p["Hv"], device=dev, generator=gen)),
    )
    pre["state"] = torch.zeros(p["B"], p["Hv"], p["d"], p["d"], device=dev)
    pre["out"] = torch.empty_like(pre["v"])

    d = DECODE
    n = d["steps"]  # every decode step has its own token: [steps][B][...]
    dec = dict(
        q=l2n(torch.randn(n, d["B"], d["Hq"], d["d"], device=dev, generator=gen)).half(),
        k=l2n(torch.randn(n, d["B"], d["Hq"], d["d"], device=dev, generator=gen)).half(),
        v=torch.randn(n, d["B"], d["Hv"], d["d"], device=dev, generator=gen).half(),
        beta=torch.sigmoid(torch.randn(n, d["B"], d["Hv"], device=dev, generator=gen)),
        g=-torch.nn.functional.softplus(torch.randn(n, d["B"], d["Hv"], device=dev, generator=gen)),
    )
    dec["states"] = [0.02 * torch.randn(d["B"], d["Hv"], d["d"], d["d"], device=dev, generator=gen)
                     for _ in range(d["replicas"])]
    dec["out"] = torch.empty_like(dec["v"][0])

    g = GQA
    gq = dict(
        q=(0.5 * torch.randn(g["B"], g["Hq"], g["S"], g["D"], device=dev, generator=gen)).half(),
        k=(0.5 * torch.randn(g["B"], g["Hkv"], g["S"], g["D"], device=dev, generator=gen)).half(),
        v=(0.5 * torch.randn(g["B"], g["Hkv"], g["S"], g["D"], device=dev, generator=gen)).half(),
        gate=torch.randn(g["B"], g["Hq"], g["S"], g["D"], device=dev, generator=gen).half(),
    )
    gq["o"] = torch.empty_like(gq["q"])
    a["gqa"] = gq
    return a, pre, dec


def layer_inputs(torch, dev, pre):
    """Raw inputs of the GDN layer at the prefill shape: q, k rows before the l2 norm, the
    gate projections a, b, dt_bias, A = -exp(A_log), the output gate z and norm weight w."""
    p = PREFILL
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    B, T, Hq, Hv, d = p["B"], p["T"], p["Hq"], p["Hv"], p["d"]
    r = lambda *shape: torch.randn(*shape, device=dev, generator=gen)
    lay = dict(q=r(B, T, Hq, d).half(), k=r(B, T, Hq, d).half(), a=r(B, T, Hv), b=r(B, T, Hv),
               dt=0.5 * r(Hv), A=-torch.exp(0.5 * r(Hv)), z=r(B, T, Hv, d).half(),
               w=1 + 0.1 * r(d))
    lay["state"] = torch.zeros(B, Hv, d, d, device=dev)
    lay["o"] = torch.empty(B, T, Hv, d, device=dev, dtype=torch.float16)
    lay["y"] = torch.empty_like(lay["o"])
    return lay


def host_info():
    """The host the CPU baseline ran on: its CPU model, the logical CPUs it has, and the CPUs
    this process may run on (its share of the machine)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return {"cpu_model": model, "nproc": os.cpu_count() or 1, "usable_cpus": usable}


def read_board():
    """Socket power (W) and the GFX clocks (MHz) of GPU 0 from amd-smi, or None without it.
    Reading only: called while kernels run, to see the board's operating point."""
    import re
    import shutil
    import subprocess
    exe = shutil.which("amd-smi") or ("/opt/rocm/bin/amd-smi" if os.path.exists("/opt/rocm/bin/amd-smi") else None)
    if exe is None:
        return None
    try:
        txt = subprocess.run([exe, "metric", "-p", "-c", "-g", "0"], capture_output=True, text=True,
                             timeout=20).stdout
    except (OSError, subprocess.SubprocessError):
        return None
    pw = re.search(r"SOCKET_POWER:\s*([0-9.]+)\s*W", txt)
    clks = [int(c) for c in re.findall(r"GFX_\d+:\s*\n\s*CLK:\s*(\d+)\s*MHz", txt)]
    if pw is None and not clks:
        return None
    return {"socket_power_w": float(pw.group(1)) if pw else None, "gfx_clock_mhz": clks}


def run_sustained(torch, dev, stream, attn, attn_ms):
    """The attention kernel back to back for ~6 s (the board settles at its power limit),
    with the board's socket power and GFX clocks read (amd-smi, when present) while the
    launches run; then an fp16 GEMM through torch (hipBLASLt) back to back: the rate the
    vendor's own MFMA kernel sustains on the same board.  Returns (ms per attention launch,
    launches, board, GEMM TFLOP/s, GEMM size, GEMM launches, board during the GEMMs)."""
    n_sus = max(1, int(6.0 / max(attn_ms * 1e-3, 1e-6)))
    s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s0.record(stream)
    for _ in range(n_sus):
        attn()
    s1.record(stream)
    board = read_board()  # the launches above are still running on the device
    torch.cuda.synchronize()
    sus_ms = s0.elapsed_time(s1) / n_sus
    gm = 8192
    ga = torch.randn(gm, gm, device=dev, dtype=torch.float16)
    gb = torch.randn(gm, gm, device=dev, dtype=torch.float16)
    gc = torch.empty(gm, gm, device=dev, dtype=torch.float16)
    torch.matmul(ga, gb, out=gc)
    torch.cuda.synchronize()
    n_gemm = 4000  # ~1 ms each
    g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    g0.record(stream)
    for _ in range(n_gemm):
        torch.matmul(ga, gb, out=gc)
    g1.record(stream)
    gemm_board = read_board()
    torch.cuda.synchronize()
    gemm_ms = g0.elapsed_time(g1) / n_gemm
    gemm_tflops = 2.0 * gm ** 3 / (gemm_ms * 1e-3) / 1e12
    del ga, gb, gc
    return sus_ms, n_sus, board, gemm_tflops, gm, n_gemm, gemm_board


def cpu_baselines(torch, a, pre, dec, threads, lay=None):
    """Time the oracle (the reference's naive paths restated in C++) on bounded samples, with
    all `threads` OpenMP threads over independent (sequence, head) pairs and with one thread
    (the reference's gdn_cpu is single-threaded, src/gdn_sm75.cu:1078-1106)."""
    import numpy as np
    import oracle
    info = host_info()
    res = {}

    def entry(value, unit, sample, one_value, one_sample):
        return dict(value=value, unit=unit, cores=threads, kind="port", sample=sample,
                    single_thread={"value": one_value, "cores": 1, "sample": one_sample}, **info)

    def clock(fn):
        t0 = time.perf_counter()
        fn()
        return time.perf_counter() - t0

    # attention: every causal row of all 32 heads (all threads), of one head (one thread)
    s = ATTN
    nh = s["H"]
    q, k, v = (a[n][:, :nh].cpu().numpy() for n in ("q", "k", "v"))
    rows = np.arange(nh * s["S"], dtype=np.int64)
    dt = clock(lambda: oracle.attn_rows(q, k, v, rows, True, nthreads=threads))
    dt1 = clock(lambda: oracle.attn_rows(q[:, :1].copy(), k[:, :1].copy(), v[:, :1].copy(),
                                         rows[:s["S"]], True, nthreads=1))
    fl = attn_flops(1, nh, s["S"], s["D"], True)
    res["attn_fwd"] = entry(fl / dt / 1e12, "TFLOP/s",
                            f"all {s['S']} causal rows of {nh} of {s['H']} heads ({dt:.1f} s)",
                            fl / nh / dt1 / 1e12, f"all {s['S']} causal rows of 1 head ({dt1:.1f} s)")
    # gated GQA layer: every row of the first query-head group (6 heads sharing K/V head 0)
    c = GQA
    gq = a["gqa"]
    grp = c["Hq"] // c["Hkv"]
    qn, gn = (gq[n][:, :grp].cpu().numpy() for n in ("q", "gate"))
    kn, vn = (gq[n][:, :1].cpu().numpy() for n in ("k", "v"))
    rows = np.arange(grp * c["S"], dtype=np.int64)
    dt = clock(lambda: oracle.attn_gqa_rows(qn, kn, vn, gn, rows, True, nthreads=threads))
    dt1 = clock(lambda: oracle.attn_gqa_rows(qn, kn, vn, gn, rows[:c["S"]], True, nthreads=1))
    fl = attn_flops(1, grp, c["S"], c["D"], True)
    res["attn_gqa_gated"] = entry(fl / dt / 1e12, "TFLOP/s",
                                  f"all {c['S']} causal rows of {grp} of {c['Hq']} query heads ({dt:.1f} s)",
                                  fl / grp / dt1 / 1e12,
                                  f"all {c['S']} causal rows of 1 query head ({dt1:.1f} s)")
    # prefill: serial recurrence, all 4096 tokens of all 32 V-heads; one thread: 2 V-heads
    p = PREFILL
    g = lambda n: pre[n].float().cpu().numpy()
    qn, kn, vn, bn, gn = g("q"), g("k"), g("v"), g("beta"), g("g")
    st = np.zeros((1, p["Hv"], p["d"], p["d"]), np.float32)
    reps = 10
    dt = clock(lambda: [oracle.gdn_serial(qn, kn, vn, gn, bn, st, nthreads=threads) for _ in range(reps)])
    h1 = 2
    dt1 = clock(lambda: oracle.gdn_serial(qn, kn, vn[:, :, :h1].copy(), gn[:, :, :h1].copy(),
                                          bn[:, :, :h1].copy(), st[:, :h1].copy(), nthreads=1))
    res["gdn_prefill"] = entry(reps * p["B"] * p["T"] / dt, "tok/s",
                               f"{reps} x T={p['T']} for all {p['Hv']} V-heads ({dt:.1f} s)",
                               p["B"] * p["T"] / (dt1 * p["Hv"] / h1),
                               f"T={p['T']} for {h1} of {p['Hv']} V-heads, scaled to all ({dt1:.1f} s)")
    # GDN layer ops: the pre-ops, the serial recurrence and the gated RMSNorm on all heads
    if lay is not None:
        ln = lambda n: lay[n].float().cpu().numpy()

        def layer(nt, hv):
            qn, kn, gg, bb = oracle.gdn_preprocess(ln("q"), ln("k"), ln("a")[:, :, :hv],
                                                   ln("b")[:, :, :hv], ln("dt")[:hv], ln("A")[:hv])
            o, _ = oracle.gdn_serial(qn, kn, np.ascontiguousarray(vn[:, :, :hv]), gg, bb,
                                     np.zeros((1, hv, p["d"], p["d"]), np.float32), nthreads=nt)
            oracle.gated_rmsnorm(o, ln("z")[:, :, :hv], ln("w"))

        dt = clock(lambda: layer(threads, p["Hv"]))
        dt1 = clock(lambda: layer(1, h1))
        res["gdn_layer_ops"] = entry(p["B"] * p["T"] / dt, "tok/s",
                                     f"T={p['T']} x {p['Hv']} V-heads, pre-ops + serial recurrence "
                                     f"+ gated RMSNorm ({dt:.1f} s)",
                                     p["B"] * p["T"] / (dt1 * p["Hv"] / h1),
                                     f"the same for {h1} of {p['Hv']} V-heads, scaled to all ({dt1:.1f} s)")
    # decode: 1024 single-token steps over the full 16 x 32-head state, each step its own
    # token (the pre-generated inputs, cycled); one thread: 64 steps
    d = DECODE
    qd, kd, vd = (dec[n].float().cpu().numpy()[:, :, None] for n in ("q", "k", "v"))
    bd, gd = (dec[n].cpu().numpy()[:, :, None] for n in ("beta", "g"))
    st0 = dec["states"][0].cpu().numpy()

    def run_steps(n, nt):
        st = st0
        for i in range(n):
            j = i % d["steps"]
            _, st = oracle.gdn_serial(qd[j], kd[j], vd[j], gd[j], bd[j], st, nthreads=nt)

    steps, steps1 = 1024, 64
    dt = clock(lambda: run_steps(steps, threads))
    dt1 = clock(lambda: run_steps(steps1, 1))
    res["gdn_decode"] = entry(decode_bytes(**d) * steps / dt / 1e9, "GB/s",
                              f"{steps} steps of 16 sequences x 32 heads ({dt:.1f} s)",
                              decode_bytes(**d) * steps1 / dt1 / 1e9,
                              f"{steps1} steps of 16 sequences x 32 heads ({dt1:.1f} s)")
    return res


def dispatch_sweep(torch, tsa, dev, stream, Hq=16, Hv=48, d=128, reps=20):
    """Token-serial (tsa_gdn_recurrent_fwd) vs chunked (tsa_gdn_chunked_fwd) time per call at
    the reference's head counts, for the short sequences where the ggml adapter switches from
    one to the other (T < 32 token-serial, else chunked).  HIP events around `reps` calls of
    each kernel, in order B, T, kernel; fp16 q/k/v, gates as the prefill's."""
    rows = []
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    for B in (1, 4):
        for T in (8, 16, 24, 32, 40, 48, 64, 96):
            l2n = lambda x: x / x.norm(dim=-1, keepdim=True)
            q = l2n(torch.randn(B, T, Hq, d, device=dev, generator=g)).half()
            k = l2n(torch.randn(B, T, Hq, d, device=dev, generator=g)).half()
            v = torch.randn(B, T, Hv, d, device=dev, generator=g).half()
            gl = -torch.nn.functional.softplus(torch.randn(B, T, Hv, device=dev, generator=g))
            beta = torch.sigmoid(torch.randn(B, T, Hv, device=dev, generator=g))
            st = torch.zeros(B, Hv, d, d, device=dev)
            out = torch.empty_like(v)
            ws = torch.empty(tsa.gdn_chunked_workspace_bytes(B, T, Hq, Hv), dtype=torch.uint8, device=dev)
            row = {"B": B, "T": T}
            for name, fn in (("token_serial", lambda: tsa.gdn_recurrent_fwd(q, k, v, gl, beta, st, out, stream=stream)),
                             ("chunked", lambda: tsa.gdn_chunked_fwd(q, k, v, gl, beta, st, out, ws=ws, stream=stream))):
                fn()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for _ in range(reps):
                    fn()
                e1.record(stream)
                torch.cuda.synchronize()
                row["us_" + name] = round(e0.elapsed_time(e1) / reps * 1e3, 2)
            rows.append(row)
    return {"dispatch_sweep": rows, "heads": {"Hq": Hq, "Hv": Hv}, "reps": reps,
            "adapter_rule": "T = 1 decode step, T < 32 token-serial, else chunked"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--decode-steps", type=int, default=512,
                    help="length of the extra decode-only run (the 512-step workload)")
    ap.add_argument("--no-sustained", action="store_true",
                    help="skip the sustained attention run and the GEMM reference (~5 s; under a "
                         "profiler their launches would outnumber the step's)")
    ap.add_argument("--dispatch-sweep", action="store_true",
                    help="only time the token-serial and the chunked GDN kernels at 16 QK / 48 V "
                         "heads for B = 1, 4 and T = 8 .. 96 (the ggml adapter's dispatch "
                         "threshold) and print that table as one JSON line")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="after the measurements, run one plain copy kernel over this many MiB "
                         "(reference kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: sharding this path over GPUs (heads or sequences, "
              "no exchange) is design-only and no multi-GPU figure is produced", file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0:
        print("--steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        return 2

    import torch
    import tsa
    tsa.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream()
    if args.dispatch_sweep:
        print(json.dumps(dispatch_sweep(torch, tsa, dev, stream)))
        return 0
    a, pre, dec = make_inputs(torch, dev)
    ws = torch.empty(tsa.gdn_chunked_workspace_bytes(PREFILL["B"], PREFILL["T"], PREFILL["Hq"],
                                                     PREFILL["Hv"]), dtype=torch.uint8, device=dev)

    def attn():
        tsa.attn_fwd(a["q"], a["k"], a["v"], a["o"], causal=True, stream=stream)

    def prefill():
        pre["state"].zero_()  # each step is the same prefill from a zero state
        tsa.gdn_chunked_fwd(pre["q"], pre["k"], pre["v"], pre["g"], pre["beta"], pre["state"],
                            pre["out"], ws=ws, stream=stream)

    # Decode launches go straight to the C-ABI with their arguments prepared beforehand: a
    # decode step is ~11 us of GPU time, about what the binding's per-call checks cost in
    # Python, so through the wrapper a back-to-back loop measures the host, not the kernel.
    import ctypes
    dec_fn = tsa.load().tsa_gdn_decode_step
    dptr = lambda t: ctypes.c_void_p(t.data_ptr())
    dstream = ctypes.c_void_p(stream.cuda_stream)
    dscale = 1.0 / math.sqrt(DECODE["d"])
    dec_args = [[(dptr(dec["q"][j]), dptr(dec["k"][j]), dptr(dec["v"][j]), dptr(dec["g"][j]),
                  dptr(dec["beta"][j]), dptr(st), dptr(dec["out"]), DECODE["B"], DECODE["Hq"],
                  DECODE["Hv"], DECODE["d"], DECODE["d"], dscale, dstream)
                 for st in dec["states"]] for j in range(DECODE["steps"])]
    dstep = [0]  # decode steps issued so far: step i uses token i % 512 of the inputs

    def decode_step(r):
        j = dstep[0] % DECODE["steps"]
        dstep[0] += 1
        rc = dec_fn(*dec_args[j][r])
        if rc:
            raise tsa.TsaError(rc, tsa.strerror(rc))

    def decode():
        for r in range(DECODE["replicas"]):
            decode_step(r)

    parts = [("attn_fwd", attn), ("gdn_prefill", prefill), ("gdn_decode", decode)]
    # Warm-up grouped by part, attention last, so that the timed region (attention first)
    # starts under the load it measures: after an idle gap or a lighter kernel the board's
    # power management overshoots on the first ~12 ms of attention (launches 4-20 measured at
    # 630-700 us against a steady ~555 us), a transient of the power controller, not of the
    # kernel.  Attention gets at least ATTN_MIN_WARMUP launches (~45 ms of continuous load)
    # whatever --warmup asks for; the other parts get --warmup steps each.
    attn_warm = max(args.warmup, ATTN_MIN_WARMUP)
    for name, fn in parts[1:] + parts[:1]:
        for _ in range(attn_warm if name == "attn_fwd" else args.warmup):
            fn()
    torch.cuda.synchronize()

    K = args.steps
    grp = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in parts]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    # The K steps' work grouped by part: K attention launches back to back, then K prefills,
    # then K x 16 decode steps -- each kernel timed in its own loop, as the reference's lab
    # drivers time theirs (src/attn_sm75.cu:507-519): one pair of events on the kernels'
    # stream around each part's K launches (an event record between launches adds a few
    # microseconds of barrier to each).
    for j, (name, fn) in enumerate(parts):
        grp[j][0].record(stream)
        for i in range(K):
            fn()
        grp[j][1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = {name: grp[j][0].elapsed_time(grp[j][1]) / K for j, (name, _) in enumerate(parts)}
    ms_step = wall * 1e3 / K
    # the prefill part resets the state before each call (every step is the same prefill
    # from a zero state): that reset, timed alone the same way, is not the kernel's
    z0, z1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    z0.record(stream)
    for i in range(K):
        pre["state"].zero_()
    z1.record(stream)
    torch.cuda.synchronize()
    ms["gdn_prefill"] -= z0.elapsed_time(z1) / K
    ms["gdn_decode"] /= DECODE["replicas"]  # per decode step (one launch)

    redo = tsa.gdn_chunked_redo_count(ws, PREFILL["B"], PREFILL["T"], PREFILL["Hq"], PREFILL["Hv"],
                                      stream=stream)

    # decode-only runs: the 512-step workload (each step its own token) cycling replicas,
    # and one resident buffer
    n = args.decode_steps
    dstep[0] = 0
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(n):
        decode_step(i % DECODE["replicas"])
    e1.record(stream)
    e2, e3 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e2.record(stream)
    for i in range(n):
        decode_step(0)
    e3.record(stream)
    torch.cuda.synchronize()
    dec_rot_ms = e0.elapsed_time(e1) / n
    dec_res_ms = e2.elapsed_time(e3) / n

    # gated GQA layer (outside the step): warm-up launch, then timed launches
    gq = a["gqa"]

    def gqa():
        tsa.attn_gqa_fwd(gq["q"], gq["k"], gq["v"], gq["gate"], gq["o"], causal=True, stream=stream)

    # continuous GQA load before its timed launches: it follows the HBM-bound decode loop, and
    # one warm-up launch left its 10 timed launches inside the power controller's start-up
    # transient (0.384-0.395 of peak against 0.409 at steady state on one box)
    for _ in range(GQA_MIN_WARMUP):
        gqa()
    n_gqa = GQA_TIMED
    e4, e5 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e4.record(stream)
    for _ in range(n_gqa):
        gqa()
    e5.record(stream)
    torch.cuda.synchronize()
    gqa_ms = e4.elapsed_time(e5) / n_gqa

    # GDN layer ops at the prefill shape (outside the step): fused vs unfused pipelines
    lay = layer_inputs(torch, dev, pre)

    def fused_layer():
        lay["state"].zero_()
        tsa.gdn_chunked_fused_fwd(lay["q"], lay["k"], pre["v"], lay["a"], lay["b"], lay["dt"],
                                  lay["A"], lay["state"], lay["o"], ws=ws, stream=stream)
        tsa.gdn_gated_rmsnorm(lay["o"], lay["z"], lay["w"], out=lay["y"], stream=stream)

    def unfused_layer():
        lay["state"].zero_()
        qn, kn, gl, be = tsa.gdn_preprocess(lay["q"], lay["k"], lay["a"], lay["b"], lay["dt"],
                                            lay["A"], stream=stream)
        tsa.gdn_chunked_fwd(qn, kn, pre["v"], gl, be, lay["state"], lay["o"], ws=ws, stream=stream)
        tsa.gdn_gated_rmsnorm(lay["o"], lay["z"], lay["w"], out=lay["y"], stream=stream)

    def rms_only():
        tsa.gdn_gated_rmsnorm(lay["o"], lay["z"], lay["w"], out=lay["y"], stream=stream)

    def time_fn(fn, n):
        fn()
        a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a0.record(stream)
        for _ in range(n):
            fn()
        a1.record(stream)
        torch.cuda.synchronize()
        return a0.elapsed_time(a1) / n

    n_lay = max(5, min(K, 20))
    fused_ms = time_fn(fused_layer, n_lay)
    unfused_ms = time_fn(unfused_layer, n_lay)
    rms_ms = time_fn(rms_only, n_lay)

    # context: one GPU's share of the prefill under 8-way head sharding (Hq=2, Hv=4 of the
    # 16 / 32 heads).  With so few heads the chunk carry alone would leave most CUs idle, so
    # the call splits the sequence (segment state maps side by side, a combine, a fix-up);
    # the same call with the split turned off (an explicit plan of one segment) is timed beside it.
    shq, shv = PREFILL["Hq"] // 8, PREFILL["Hv"] // 8
    sq, sk = (x[:, :, :shq].contiguous() for x in (pre["q"], pre["k"]))
    sv = pre["v"][:, :, :shv].contiguous()
    sg, sb = (x[:, :, :shv].contiguous() for x in (pre["g"], pre["beta"]))
    sst = torch.zeros(PREFILL["B"], shv, PREFILL["d"], PREFILL["d"], device=dev)
    so = torch.empty_like(sv)

    def shard_ms(nseg):
        nbytes = tsa.gdn_chunked_workspace_bytes(PREFILL["B"], PREFILL["T"], shq, shv, nseg=nseg)
        sws = torch.empty(nbytes, dtype=torch.uint8, device=dev)

        def f():
            sst.zero_()
            tsa.gdn_chunked_fwd(sq, sk, sv, sg, sb, sst, so, ws=sws, stream=stream, nseg=nseg)
        return time_fn(f, n_lay), nbytes

    def shard_zero():
        sst.zero_()

    shard_zero_ms = time_fn(shard_zero, n_lay)
    shard_split_ms, shard_ws = shard_ms(0)
    shard_plain_ms, shard_ws_plain = shard_ms(1)
    shard_split_ms -= shard_zero_ms
    shard_plain_ms -= shard_zero_ms

    # context: one GDN layer at the reference's published shape (T=512, Hq=16, Hv=48), fp32
    # q / k / v / out as the reference's kernels take them (src/gdn_sm75.cu:57-64), inputs in
    # the ranges of its LCG generator (:1270-1279), state from zero
    r = REF_GDN
    rgen = torch.Generator(device=dev)
    rgen.manual_seed(11)
    uni = lambda lo, hi, *shape: lo + (hi - lo) * torch.rand(*shape, device=dev, generator=rgen)
    rq = uni(-0.1, 0.1, r["B"], r["T"], r["Hq"], r["d"])
    rk = uni(-0.1, 0.1, r["B"], r["T"], r["Hq"], r["d"])
    rv = uni(-0.1, 0.1, r["B"], r["T"], r["Hv"], r["d"])
    rg = uni(-0.225, -0.175, r["B"], r["T"], r["Hv"])
    rb = uni(0.4, 0.8, r["B"], r["T"], r["Hv"])
    rst = torch.zeros(r["B"], r["Hv"], r["d"], r["d"], device=dev)
    ro = torch.empty_like(rv)
    rws = torch.empty(tsa.gdn_chunked_workspace_bytes(r["B"], r["T"], r["Hq"], r["Hv"], f32=True),
                      dtype=torch.uint8, device=dev)

    def ref_serial():
        rst.zero_()
        tsa.gdn_recurrent_fwd(rq, rk, rv, rg, rb, rst, ro, stream=stream)

    def ref_chunked():
        rst.zero_()
        tsa.gdn_chunked_fwd(rq, rk, rv, rg, rb, rst, ro, ws=rws, stream=stream)

    def ref_zero():
        rst.zero_()

    zero_ms = time_fn(ref_zero, 20)
    ref_serial_ms = time_fn(ref_serial, 20) - zero_ms
    ref_chunked_ms = time_fn(ref_chunked, 20) - zero_ms

    # Sustained attention and the GEMM reference (see run_sustained)
    sustained = None
    if not args.no_sustained:
        sustained = run_sustained(torch, dev, stream, attn, ms["attn_fwd"])

    if args.copy_calibration_mib > 0:
        n_el = args.copy_calibration_mib * (1 << 20) // 4
        src = torch.ones(n_el, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        torch.mul(src, 1.0, out=dst)  # one elementwise copy kernel (a device copy may use DMA)
        torch.cuda.synchronize()
        del src, dst

    finite = bool(torch.isfinite(a["o"]).all() and torch.isfinite(pre["out"]).all()
                  and torch.isfinite(pre["state"]).all() and torch.isfinite(dec["out"]).all()
                  and torch.isfinite(gq["o"]).all() and torch.isfinite(lay["y"]).all()
                  and torch.isfinite(so).all() and torch.isfinite(sst).all())

    traffic = load_traffic()
    fa = attn_flops(**ATTN)
    fp = prefill_flops(**PREFILL)
    bp = prefill_bytes(**PREFILL)
    bd = decode_bytes(**DECODE)
    attn_tflops = fa / (ms["attn_fwd"] * 1e-3) / 1e12
    fg = attn_flops(GQA["B"], GQA["Hq"], GQA["S"], GQA["D"], True)
    gqa_tflops = fg / (gqa_ms * 1e-3) / 1e12
    pre_tflops = fp / (ms["gdn_prefill"] * 1e-3) / 1e12
    dec_gbs = bd / (dec_rot_ms * 1e-3) / 1e9

    def roof(bound, achieved, peak, unit, key):
        return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
                "frac": round(achieved / peak, 4), "traffic": traffic.get(key)}

    out_parts = {
        "attn_fwd": {
            "workload": "attention fwd B=1 H=32 S=8192 D=128 causal fp16, N(0,0.5) + 1% x8 outliers",
            "value": round(attn_tflops, 2), "unit": "TFLOP/s", "ms": round(ms["attn_fwd"], 5),
            "flop_per_launch": fa, "warmup_launches": attn_warm,
            "roofline": roof("mfma", attn_tflops, PEAK_MFMA_F16_TFLOPS, "TFLOP/s", "attn_fwd"),
        },
        "gdn_prefill": {
            "workload": "chunked GDN prefill B=1 T=4096 Hq=16 Hv=32 d=128 C=64, fp16 I/O, fp32 state",
            "value": round(PREFILL["B"] * PREFILL["T"] / (ms["gdn_prefill"] * 1e-3), 1),
            "unit": "tok/s", "ms": round(ms["gdn_prefill"], 5), "flop_per_launch": fp,
            "bytes_per_launch": bp,
            "roofline": roof("mfma", pre_tflops, PEAK_MFMA_F16_TFLOPS, "TFLOP/s", "gdn_prefill"),
            "hbm_frac": round(bp / (ms["gdn_prefill"] * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "carry_workgroups_redone_last_call": redo,
        },
        "gdn_prefill_head_shard": {
            "workload": "context only: one GPU's share of the chunked GDN prefill under 8-way "
                        f"head sharding, B=1 T={PREFILL['T']} Hq={shq} Hv={shv} d=128 C=64, fp16 "
                        "I/O, state from zero; timed outside the step",
            "ms_sequence_split": round(shard_split_ms, 5), "ms_no_split": round(shard_plain_ms, 5),
            "tok_s": round(PREFILL["B"] * PREFILL["T"] / (shard_split_ms * 1e-3), 1),
            "mfma_frac": round(prefill_flops(**dict(PREFILL, Hq=shq, Hv=shv)) / (shard_split_ms * 1e-3)
                               / 1e12 / PEAK_MFMA_F16_TFLOPS, 4),
            "workspace_bytes": shard_ws, "workspace_bytes_no_split": shard_ws_plain,
        },
        "gdn_reference_shape": {
            "workload": "context only: one GDN layer at the reference's published shape, B=1 "
                        "T=512 Hq=16 Hv=48 d=128, fp32 q/k/v/out (its own I/O type) in the ranges "
                        "of its LCG inputs, state from zero; its figures are from an RTX 2080 Ti",
            "ms_token_serial": round(ref_serial_ms, 5), "ms_chunked": round(ref_chunked_ms, 5),
            "reference_ms_2080ti": REF_GDN_MS,
            "reference_source": "docs/kernels.md:31-39, docs/tu102.md:265-274",
        },
        "attn_gqa_gated": {
            "workload": "gated GQA attention fwd B=1 Hq=24 Hkv=4 S=8192 D=256 causal fp16, "
                        "N(0,0.5), gate N(0,1); timed outside the step",
            "value": round(gqa_tflops, 2), "unit": "TFLOP/s", "ms": round(gqa_ms, 5),
            "flop_per_launch": fg, "warmup_launches": GQA_MIN_WARMUP, "timed_launches": GQA_TIMED,
            "roofline": roof("mfma", gqa_tflops, PEAK_MFMA_F16_TFLOPS, "TFLOP/s", "attn_gqa_gated"),
        },
        "gdn_layer_ops": {
            "workload": "GDN layer at the prefill shape from raw inputs (q/k rows N(0,1), gate "
                        "projections a, b): fused pre-ops + chunked prefill + gated RMSNorm; "
                        "timed outside the step",
            "value": round(PREFILL["B"] * PREFILL["T"] / (fused_ms * 1e-3), 1), "unit": "tok/s",
            "ms_fused": round(fused_ms, 5), "ms_unfused": round(unfused_ms, 5),
            "ms_gated_rmsnorm": round(rms_ms, 5),
            "gated_rmsnorm_bytes": rmsnorm_bytes(**PREFILL),
            "roofline": roof("hbm", rmsnorm_bytes(**PREFILL) / (rms_ms * 1e-3) / 1e9, PEAK_HBM_GBS,
                             "GB/s", "gdn_gated_rmsnorm"),
        },
        "gdn_decode": {
            "workload": f"GDN decode, {n} steps back to back, each with its own token, 16 sequences "
                        "x 32 V-heads, 128x128 fp32 state, 16 state replicas cycled (512 MiB, "
                        "streamed from HBM)",
            "value": round(dec_gbs, 1), "unit": "GB/s", "ms": round(dec_rot_ms, 5),
            "bytes_per_launch": bd,
            "tok_s": round(DECODE["B"] / (dec_rot_ms * 1e-3), 1),
            "roofline": roof("hbm", dec_gbs, PEAK_HBM_GBS, "GB/s", "gdn_decode"),
            "in_step": {"ms_per_launch": round(ms["gdn_decode"], 5),
                        "gbs": round(bd / (ms["gdn_decode"] * 1e-3) / 1e9, 1),
                        "note": "16 launches inside the mixed step, after the prefill"},
            "resident_in_cache": {"ms_per_step": round(dec_res_ms, 5),
                                  "gbs": round(bd / (dec_res_ms * 1e-3) / 1e9, 1),
                                  "note": "one 32 MiB state buffer, held in the Infinity Cache"},
        },
    }
    if sustained is not None:
        sus_ms, n_sus, board, gemm_tflops, gm, n_gemm, gemm_board = sustained
        sus_tflops = fa / (sus_ms * 1e-3) / 1e12
        out_parts["attn_fwd"]["sustained"] = {
            "launches": n_sus, "ms": round(sus_ms, 5), "value": round(sus_tflops, 2),
            "unit": "TFLOP/s", "frac": round(sus_tflops / PEAK_MFMA_F16_TFLOPS, 4), "board": board,
            "note": "the kernel back to back for ~6 s; board power / clocks read meanwhile"}
        out_parts["attn_fwd"]["mfma_gemm_reference"] = {
            "workload": f"torch.matmul fp16 {gm}x{gm}x{gm} (hipBLASLt) back to back, {n_gemm} launches",
            "value": round(gemm_tflops, 2), "unit": "TFLOP/s",
            "frac": round(gemm_tflops / PEAK_MFMA_F16_TFLOPS, 4), "board": gemm_board,
            "attn_sustained_over_gemm": round(sus_tflops / gemm_tflops, 4),
            "note": "what the vendor's fp16 GEMM sustains on this board: the practical MFMA "
                    "ceiling under its power limit, for context beside the nominal peak"}
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baselines(torch, a, pre, dec, omp_threads(), lay)
        rnd = lambda d: {kk: (round(vv, 4) if isinstance(vv, float) else rnd(vv) if isinstance(vv, dict)
                              else vv) for kk, vv in d.items()}
        for k, v in cpu.items():
            out_parts[k]["cpu_baseline"] = rnd(v)

    line = {
        "metric": "attn fwd TFLOP/s + GDN prefill tok/s + decode GB/s, % of MI355X roofline",
        "value": round(attn_tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded torch generators on the device)",
        "config": {"workload": "attention fwd B=1 H=32 S=8192 D=128 causal + chunked GDN prefill "
                               "B=1 T=4096 Hq=16 Hv=32 C=64 + GDN decode step B=16 Hv=32",
                   "parallelism": "single GPU"},
        "roofline": out_parts["attn_fwd"]["roofline"],
        "cpu_baseline": out_parts["attn_fwd"].get("cpu_baseline"),
        "parts": out_parts,
        "outputs_finite": finite,
    }
    print(json.dumps(line), flush=True)
    return 0 if finite else 1


if __name__ == "__main__":
    sys.exit(main())
