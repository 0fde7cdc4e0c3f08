"""Benchmark of the Gated DeltaNet operator on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-decode]
                    [--no-b256] [--no-layer] [--no-long] [--no-backward] [--copy-probe]

Prints ONE JSON line. The headline workload is the Qwen3-Next-shaped prefill
(B=1, T=32768, Hk=16 -> Hv=32, K=V=128, bf16 q/k/v, fp32 state, chunk 64):
a step is one chunk-kernel call over those inputs, resident in HBM, writing o
(bf16) and the final state (fp32). `value` is prefill throughput in Mtok/s.
The same line carries the decode step (64 sequences x 1 token, state
[64,32,128,128] fp32 updated in place, 1000 chained steps of one pool, which
the loop declares resident: PBGDN_STATE_RESIDENT keeps it in the 256 MB
last-level cache) in µs/step and as a fraction of HBM bandwidth, the same step
as a model takes it (three pools in rotation, the default streamed policy: the
state comes from HBM), the same step with the state held in bf16 (a serving
cache's default), an ungraded 256-sequence decode, the
library's 1 GiB streaming copy (pbgdn_stream_probe: the read+write ceiling
each decode line is also given against), the small fp32 prefill (the
reference's CPU-runnable case), the fused layer prologue and epilogue kernels
at the same T and head shape with their HBM rooflines, the fused one-kernel
decode step of the whole layer (64 sequences; against the same step as three
launches), the backward, the varlen (8 packed sequences, 262,144 tokens) and
streamed (1,048,576 tokens in 16 segments) prefill workloads, the roofline of
the prefill kernel measured with HIP events on the stream it runs on, and the
CPU baseline: the numpy oracle (oracle/gdn.py) on the full prefill call, run
first, before the GPU is touched, as one single-threaded process per value
head on up to every affinity core; with it the small prefill and the varlen
prefill in full, the first two segments of the streamed prefill, 50 chained
decode steps, the CPU's model and core counts, and the SHA-256 of every
prefill input. The backward's roofline is against the bf16 dense MFMA peak
(its products run on bf16 MFMA for bf16 inputs), with its counter traffic.

Before its W warmup steps the headline step runs untimed for DEVICE_WARMUP_S
(0.3 s, `device_warmup_s` in the line), and every other line's step for
0.2 s: the GPU has sat idle through the CPU baseline (and through the host
work that makes each line's inputs), and its first ~25 ms of work run ~10%
slower on these boxes, so the timed steps measure the steady state.

`roofline.traffic` (HBM bytes per launch) comes from the rocprofv3 counter
summary committed under profiles/ (FETCH_SIZE and WRITE_SIZE per dispatch,
each scaled by what the counter reads for the streaming probe's 1 GiB copy in
the same process); it is null when that file is absent.
"""
from __future__ import annotations

import os

os.environ.setdefault("OPENBLAS_NUM_THREADS", "1")  # the CPU baseline pins one thread per process

import argparse
import json
import multiprocessing
import re
import statistics
import sys
import time

import numpy as np

# Algorithmic work (per token per value head, chunk C, head dims K, V):
#   flops = 2C(3K + 2V) + 6KV + (2/3)C^2  (K K^T, Q K^T, W, U', (QK^T o D) U at 2C*dim;
#           W S, Q S, K^T U at 2KV; the triangular inverse)
#   bytes = q, k (Hk heads) and v, o (Hv heads) once, g and beta fp32, h0 and final fp32.
MFMA_PEAK_TFLOPS = 2500.0   # MI355X dense bf16/fp16 MFMA
HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
COPY_PROBE_BYTES = 256 << 20  # the copy probe reads this many bytes and writes as many
TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "traffic_chunk_and_recurrent_kernels.md")


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` ("chunk", "recurrent_b64", ...) from the
    committed counter summary: lines of the form `traffic_bytes[<kernel>]: <int>`."""
    try:
        with open(TRAFFIC_FILE) as f:
            text = f.read()
    except OSError:
        return None
    m = re.search(r"traffic_bytes\[" + re.escape(kernel) + r"\]:\s*(\d+)", text)
    return int(m.group(1)) if m else None


def prefill_flops(tokens, hv, dk, dv, chunk=64):
    per = 2 * chunk * (3 * dk + 2 * dv) + 6 * dk * dv + (2.0 / 3.0) * chunk * chunk
    return per * tokens * hv


def backward_flops(tokens, hv, dk, dv, chunk=64):
    """The chunk backward's products per token per value head: the recomputed
    forward states and nine K x V-sized products in all (K S, K^T E U, J, K dS',
    (Gamma K)^T dX, dO S^T, U dS'^T, dX S^T, Q S: 2KV each), five C x V-sized
    (Tb X, M^T dO, Tb^T dU, dU X^T, dO U^T: 2CV), six C x K-sized (K K^T,
    Q K^T, (dM o Mt) K and its transpose with Q, H K, H^T K: 2CK) and the
    triangular terms (T^T dT, W T^T, the solve: (14/3) C^2)."""
    per = 18 * dk * dv + 10 * chunk * dv + 12 * chunk * dk + (14.0 / 3.0) * chunk * chunk
    return per * tokens * hv


FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 MFMA


def backward_bytes(tokens, hk, hv, dk, dv, elem=2, nstates=1):
    """What the backward must read and write once: q, k, v, dO and dq, dk, dv
    in the inputs' dtype; g, beta, dg, dbeta float32; h0, the final state's
    gradient and dh0 float32."""
    per_token = 4 * hk * dk * elem + 3 * hv * dv * elem + 4 * hv * 4
    return per_token * tokens + 3 * nstates * hv * dk * dv * 4


def bench_backward(steps=3, warmup=1):
    """pbgdn_chunk_bwd at the prefill shape (bf16 q, k, v; the gradients of o
    and of the final state given): the algorithmic flops above against the
    bf16 dense MFMA peak (with bf16 inputs every product of the backward runs on
    bf16 MFMA, as pairs of bf16 parts where an operand is float32), with the HBM
    traffic per call from the committed counter summary beside the
    algorithmic bytes."""
    import torch
    from pseudobrain_amd import _lib
    from pseudobrain_amd import gated_deltanet as gd
    from pseudobrain_amd.workloads import WORKLOADS, workload
    s = WORKLOADS["prefill_qwen3next"]
    q, k, v, g, beta, h0 = (x.cuda() for x in workload("prefill_qwen3next", seed=0))
    gen = torch.Generator().manual_seed(1)
    do = (torch.randn(1, s.length, s.hv, s.dv, generator=gen) * 0.1).to(torch.bfloat16).cuda()
    dht = (torch.randn(1, s.hv, s.dk, s.dv, generator=gen) * 0.1).cuda()
    scale = s.dk ** -0.5

    def step():
        gd.chunk_bwd(q, k, v, g, beta, scale, h0, do, dht)

    sec, ksec = timed_steps(step, steps, warmup)
    flops = backward_flops(s.length, s.hv, s.dk, s.dv)
    nbytes = backward_bytes(s.length, s.hk, s.hv, s.dk, s.dv)
    traffic = measured_traffic("backward")
    achieved = flops / ksec / 1e12
    return {"workload": "prefill_qwen3next backward", "T": s.length, "ms_per_call": sec * 1e3,
            "kernel_ms": ksec * 1e3, "Mtok_s": s.length / sec / 1e6, "algorithmic_flops": flops,
            "workspace_bytes": _lib.lib().pbgdn_chunk_bwd_workspace_size(1, s.length, s.hk, s.hv, s.dk, s.dv),
            "roofline": {"bound": "mfma", "achieved": achieved, "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": achieved / MFMA_PEAK_TFLOPS, "peak_basis": "bf16 dense MFMA (bf16 inputs)",
                         "traffic": traffic, "algorithmic_bytes": nbytes,
                         "traffic_over_algorithmic": None if traffic is None else traffic / nbytes,
                         "fp32_mfma_frac": achieved / FP32_MFMA_PEAK_TFLOPS}}


def prefill_bytes(tokens, hk, hv, dk, dv, nstates=1, elem=2):
    per_token = 2 * hk * dk * elem + 2 * hv * dv * elem + 2 * hv * 4
    return per_token * tokens + 2 * nstates * hv * dk * dv * 4


def decode_bytes(batch, hk, hv, dk, dv, elem=2, state_elem=4):
    state = 2 * batch * hv * dk * dv * state_elem
    io = batch * (2 * hk * dk * elem + 2 * hv * dv * elem + 2 * hv * 4)
    return state + io


# ---------------------------------------------------------------------------
# CPU baselines: the oracle (numpy fp32) on every affinity core, one process per
# value head (prefill) or per batch slice (decode), on the same seeded inputs.
# ---------------------------------------------------------------------------
# The prefill arrays a pool works on: set before the pool forks, so the workers
# inherit them instead of receiving pickled copies (the varlen inputs are ~9 GB
# in float32).
_SHARED: dict = {}


def _oracle_head(task):
    """One value head of the prefill in _SHARED through the chunked oracle:
    one call (B = 1), one call per packed sequence (cu_seqlens), or the
    segments of a stream with the state carried. `warm` runs 256 tokens."""
    from oracle import gdn
    h, warm = task
    x = _SHARED
    q, k, v, g, beta, h0 = x["q"], x["k"], x["v"], x["g"], x["beta"], x["h0"]
    hk = h // (v.shape[2] // q.shape[2])
    qh, kh = q[:, :, hk:hk + 1], k[:, :, hk:hk + 1]
    vh, gh, bh, sh = v[:, :, h:h + 1], g[:, :, h:h + 1], beta[:, :, h:h + 1], h0[:, h:h + 1]
    if warm:
        gdn.delta_rule_chunked(qh[:, :256], kh[:, :256], vh[:, :256], gh[:, :256], bh[:, :256], x["scale"], sh[:1])
    elif x.get("cu") is not None:
        gdn.varlen(qh, kh, vh, gh, bh, x["scale"], sh, x["cu"])
    elif x.get("segment"):
        for _ in gdn.streamed(qh, kh, vh, gh, bh, x["scale"], sh, x["segment"]):
            pass
    else:
        gdn.delta_rule_chunked(qh, kh, vh, gh, bh, x["scale"], sh)


def _oracle_steps(args):
    from oracle import gdn
    q, k, v, g, beta, h0, scale = args
    gdn.delta_rule_sequential(q, k, v, g, beta, scale, h0)


def cpu_info():
    """CPU model, logical and physical core counts, and the cores this process may use."""
    model, phys = "unknown", set()
    try:
        with open("/proc/cpuinfo") as f:
            pid = cid = None
            for line in f:
                key, _, val = line.partition(":")
                key, val = key.strip(), val.strip()
                if key == "model name" and model == "unknown":
                    model = val
                elif key == "physical id":
                    pid = val
                elif key == "core id":
                    cid = val
                    phys.add((pid, cid))
    except OSError:
        pass
    return {"model": model, "logical_cores": os.cpu_count(), "physical_cores": len(phys) or None,
            "affinity_cores": len(os.sched_getaffinity(0))}


def _one_thread():
    """Pool initializer: one BLAS/OpenMP thread per worker process (the box
    exports OMP_NUM_THREADS=16, which would put 16 threads on every core)."""
    from threadpoolctl import threadpool_limits
    threadpool_limits(1)


def _timed_pool(fn, tasks, procs, warm):
    ctx = multiprocessing.get_context("fork")
    with ctx.Pool(procs, initializer=_one_thread) as pool:
        pool.map(fn, warm)
        t0 = time.perf_counter()
        pool.map(fn, tasks)
        return time.perf_counter() - t0


def _prefill_cpu(inputs, procs_cap, cu=None, segment=None):
    """Seconds for the oracle over every value head of `inputs` (q, k, v, g,
    beta, h0 torch tensors), one single-threaded process per head."""
    from pseudobrain_amd.workloads import to_numpy
    q, k, v, g, beta, h0 = (to_numpy(t) for t in inputs)
    _SHARED.update(q=q, k=k, v=v, g=g, beta=beta, h0=h0, scale=q.shape[-1] ** -0.5,
                   cu=None if cu is None else to_numpy(cu), segment=segment)
    try:
        hv = v.shape[2]
        procs = min(procs_cap, hv)
        return _timed_pool(_oracle_head, [(h, False) for h in range(hv)], procs,
                           [(h, True) for h in range(procs)]), procs
    finally:
        _SHARED.clear()


STREAM_CPU_SEGMENTS = 2  # segments of the million-token stream the CPU baseline times


def cpu_baseline(seed: int = 0, decode_steps: int = 50):
    """The oracle on the host cores (kind "port"), each workload on its own
    seeded inputs: the full Qwen3-Next prefill (32,768 tokens, 32 value heads),
    the small prefill and the varlen prefill (8 sequences, 262,144 tokens) in
    one full call each; the million-token stream over its first
    STREAM_CPU_SEGMENTS segments of 65,536 tokens with the state carried (its
    rate is the per-segment mean; the chunked oracle's cost per segment does not
    depend on the state); the decode step (B = 64) as `decode_steps` chained
    steps. Returns the headline entry (prefill, Mtok/s) with the others under
    "configs"."""
    from pseudobrain_amd.workloads import (STREAM_SEGMENT, WORKLOADS, generate, sha256, to_numpy,
                                           varlen_workload, workload)
    info = cpu_info()
    cap = info["affinity_cores"]
    c1_inputs = workload("prefill_qwen3next", seed)
    c1_sec, c1_procs = _prefill_cpu(c1_inputs, cap)
    c1_tokens = WORKLOADS["prefill_qwen3next"].length
    rate = c1_tokens / c1_sec
    inputs_sha = {n: sha256(t) for n, t in zip(("q", "k", "v", "g", "beta", "h0"), c1_inputs)}
    del c1_inputs
    c0_sec, c0_procs = _prefill_cpu(workload("prefill_small", seed), cap)
    *c3_inputs, c3_cu = varlen_workload(seed)
    c3_sec, c3_procs = _prefill_cpu(c3_inputs, cap, cu=c3_cu)
    c3_tokens = int(c3_cu[-1])
    del c3_inputs
    c4_tokens = STREAM_CPU_SEGMENTS * STREAM_SEGMENT
    c4_sec, c4_procs = _prefill_cpu(workload("stream_1m", seed, length=c4_tokens), cap, segment=STREAM_SEGMENT)
    c4_total = WORKLOADS["stream_1m"].length
    s2 = WORKLOADS["decode_b64"]
    x = generate(s2.batch, decode_steps, s2.hk, s2.hv, s2.dk, s2.dv, s2.dtype, s2.h0_std, seed)
    q, k, v, g, beta, h0 = (to_numpy(t) for t in x)
    procs = min(cap, s2.batch)
    per = -(-s2.batch // procs)
    slices = [slice(i, min(i + per, s2.batch)) for i in range(0, s2.batch, per)]
    tasks = [(q[sl], k[sl], v[sl], g[sl], beta[sl], h0[sl], s2.dk ** -0.5) for sl in slices]
    warm = [(a[0][:, :1], a[1][:, :1], a[2][:, :1], a[3][:, :1], a[4][:, :1], a[5], a[6]) for a in tasks]
    c2_sec = _timed_pool(_oracle_steps, tasks, len(tasks), warm)
    configs = {
        "prefill_small": {"seconds": c0_sec, "value": WORKLOADS["prefill_small"].length / c0_sec / 1e6,
                          "unit": "Mtok/s", "cores": c0_procs, "measured": "one full call"},
        "prefill_qwen3next": {"seconds": c1_sec, "value": rate / 1e6, "unit": "Mtok/s", "cores": c1_procs,
                              "measured": "one full call"},
        "decode_b64": {"seconds": c2_sec, "value": c2_sec / decode_steps * 1e6, "unit": "us/step",
                       "cores": len(tasks), "measured": f"{decode_steps} chained steps"},
        "varlen_8seq": {"seconds": c3_sec, "value": c3_tokens / c3_sec / 1e6, "unit": "Mtok/s", "cores": c3_procs,
                        "measured": f"one full call ({c3_tokens} tokens in 8 packed sequences, 32 value heads)"},
        "stream_1m": {"seconds_measured": c4_sec, "value": c4_tokens / c4_sec / 1e6, "unit": "Mtok/s",
                      "cores": c4_procs, "seconds_per_segment": c4_sec / STREAM_CPU_SEGMENTS,
                      "seconds_whole_stream_at_that_rate": c4_total / c4_tokens * c4_sec,
                      "measured": (f"the first {STREAM_CPU_SEGMENTS} of {c4_total // STREAM_SEGMENT} segments "
                                   f"({c4_tokens} tokens, state carried, 32 value heads); value is their "
                                   "per-segment mean rate")},
    }
    return {
        "value": rate / 1e6, "unit": "Mtok/s", "cores": c1_procs, "kind": "port",
        "sample": (f"oracle delta_rule_chunked (numpy fp32), the full prefill workload ({c1_tokens} tokens, "
                   f"{s2.hv} value heads), one single-threaded process per head on {c1_procs} of "
                   f"{info['affinity_cores']} affinity cores; {c1_sec:.1f} s; cpu: {info['model']}"),
        "seconds": c1_sec,
        "cpu": info,
        "inputs_sha256": inputs_sha,
        "configs": configs,
    }


# ---------------------------------------------------------------------------
# GPU measurements
# ---------------------------------------------------------------------------
def timed_steps(fn, steps, warmup, device_warm_s=0.2):
    """Run fn untimed for `device_warm_s` seconds (device_warmup: the inputs of
    many lines are made on the host first, and the idle GPU's first
    milliseconds of work run slow), then `warmup` untimed steps, then time
    `steps` back-to-back steps. Returns (host seconds per step between two
    synchronizations, device seconds per launch from two HIP events recorded
    around the same launches on the stream they run on, torch's current
    stream)."""
    import torch
    if device_warm_s > 0:
        device_warmup(fn, device_warm_s)
    for _ in range(warmup):
        fn()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    return wall, start.elapsed_time(end) / 1e3 / steps


def kernel_time(fn, reps):
    """Mean device duration of fn's launches, timed as in timed_steps (seconds)."""
    return timed_steps(fn, reps, 1)[1]


DEVICE_WARMUP_S = 0.3  # untimed seconds of the headline step before its W warmups


def device_warmup(fn, seconds=DEVICE_WARMUP_S):
    """Run fn back to back for about `seconds` of wall time, untimed. After the
    CPU baseline the GPU has sat idle: on these boxes the first ~25 ms of work
    then run ~10% slower (0.743 ms per prefill call over the first 20 calls,
    0.676 ms from the 25th on, every later window within 0.5%), so the headline
    is timed in the steady state, as a serving or training loop runs it."""
    import torch
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()


def bench_prefill(steps, warmup):
    import torch
    from pseudobrain_amd import gated_deltanet as gd
    from pseudobrain_amd.workloads import WORKLOADS, workload
    s = WORKLOADS["prefill_qwen3next"]
    q, k, v, g, beta, h0 = (x.cuda() for x in workload("prefill_qwen3next", seed=0))
    scale = s.dk ** -0.5
    out = torch.empty(1, s.length, s.hv, s.dv, dtype=torch.bfloat16, device="cuda")

    def step():
        gd.chunk_fwd(q, k, v, g, beta, scale, h0, out=out)

    sec, ksec = timed_steps(step, steps, warmup, device_warm_s=DEVICE_WARMUP_S)
    flops = prefill_flops(s.length, s.hv, s.dk, s.dv)
    nbytes = prefill_bytes(s.length, s.hk, s.hv, s.dk, s.dv)
    return s, sec, ksec, flops, nbytes


def bench_prefill_small(steps=50, warmup=5):
    """The reference's CPU-runnable case (prefill_small: B=1, T=2048, 4 heads,
    K=V=64, fp32 inputs and output) on the GPU."""
    import torch
    from pseudobrain_amd import gated_deltanet as gd
    from pseudobrain_amd.workloads import WORKLOADS, workload
    s = WORKLOADS["prefill_small"]
    q, k, v, g, beta, h0 = (x.cuda() for x in workload("prefill_small", seed=0))
    out = torch.empty(1, s.length, s.hv, s.dv, dtype=torch.float32, device="cuda")

    def step():
        gd.chunk_fwd(q, k, v, g, beta, s.dk ** -0.5, h0, out=out)

    sec, ksec = timed_steps(step, steps, warmup)
    flops = prefill_flops(s.length, s.hv, s.dk, s.dv)
    return {"workload": "prefill_small", "T": s.length, "value": s.length / sec / 1e6, "unit": "Mtok/s",
            "ms_per_call": sec * 1e3, "roofline": {"bound": "mfma", "achieved": flops / ksec / 1e12,
                                                   "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                                                   "frac": flops / ksec / 1e12 / MFMA_PEAK_TFLOPS}}


def bench_prefill_k256(steps=10, warmup=2, serial_tokens=2048):
    """The prefill at 256-wide key and value heads (prefill_k256: B=1, T=32768,
    Hk=16 -> Hv=32, K=V=256, bf16), the widest the reference's device gate
    admits: the chunk path (prep kernel, then the scan for 256-wide keys),
    beside the token-serial recurrent kernel that such heads ran on before,
    timed over the first `serial_tokens` tokens and scaled to the call."""
    import torch
    from pseudobrain_amd import gated_deltanet as gd
    from pseudobrain_amd.workloads import WORKLOADS, workload
    s = WORKLOADS["prefill_k256"]
    q, k, v, g, beta, h0 = (x.cuda() for x in workload("prefill_k256", seed=0))
    scale = s.dk ** -0.5
    out = torch.empty(1, s.length, s.hv, s.dv, dtype=torch.bfloat16, device="cuda")

    def step():
        gd.chunk_fwd(q, k, v, g, beta, scale, h0, out=out)

    sec, ksec = timed_steps(step, steps, warmup)
    flops = prefill_flops(s.length, s.hv, s.dk, s.dv)
    n = serial_tokens
    state = h0.clone()

    def serial():
        gd.recurrent_fwd(q[:, :n], k[:, :n], v[:, :n], g[:, :n], beta[:, :n], scale, state, state)

    ssec, _ = timed_steps(serial, 2, 1, device_warm_s=0.0)
    return {"workload": "prefill_k256", "B": s.batch, "T": s.length, "Hk": s.hk, "Hv": s.hv, "K": s.dk,
            "V": s.dv, "value": s.length / sec / 1e6, "unit": "Mtok/s", "ms_per_call": sec * 1e3,
            "roofline": {"bound": "mfma", "achieved": flops / ksec / 1e12, "peak": MFMA_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": flops / ksec / 1e12 / MFMA_PEAK_TFLOPS,
                         "kernel_ms": ksec * 1e3, "algorithmic_flops": flops},
            "token_serial_ms_per_call": ssec * 1e3 * s.length / n,
            "token_serial_sample_tokens": n}


def bench_decode(batch, steps, warmup=10, state_dtype=None, pools=1, resident=False):
    """Decode steps at `batch` sequences. With pools > 1 the steps rotate over
    that many separate state pools (step i updates pool i % pools), so that
    each step's state has left the 256 MB last-level cache since it was last
    touched, as in a model whose layers each keep their own pool. `resident`
    declares the pool resident (PBGDN_STATE_RESIDENT: cacheable state
    accesses), as a loop stepping one pool may; the default streams it."""
    import torch
    from pseudobrain_amd.workloads import WORKLOADS, generate
    s = WORKLOADS["decode_b64"]
    q, k, v, g, beta, state = (x.cuda() for x in generate(batch, 1, s.hk, s.hv, s.dk, s.dv, s.dtype,
                                                          s.h0_std, seed=0))
    if state_dtype is not None:
        state = state.to(state_dtype)
    states = [state] + [state.clone() for _ in range(pools - 1)]
    scale = s.dk ** -0.5
    turn = [0]

    def step():
        torch.ops.pbgdn.recurrent_step_(q, k, v, g, beta, states[turn[0] % pools], None, scale, resident)
        turn[0] += 1

    sec, ksec = timed_steps(step, steps, warmup)
    nbytes = decode_bytes(batch, s.hk, s.hv, s.dk, s.dv, state_elem=state.element_size())
    return {
        "batch": batch, "state_dtype": str(state.dtype).replace("torch.", ""), "pools": pools,
        "state_policy": "resident" if resident else "stream", "steps": steps,
        "us_per_step": sec * 1e6, "kernel_us": ksec * 1e6,
        "bytes_per_step": nbytes, "achieved_GBs": nbytes / ksec / 1e9,
        "hbm_frac": nbytes / ksec / 1e9 / HBM_PEAK_GBS,
    }


def bench_long(steps=5, warmup=1):
    """The varlen (8 packed sequences, 262,144 tokens, per-sequence states) and
    streamed (1,048,576 tokens as 16 segments of 65,536 with the state carried)
    prefill workloads: Mtok/s and the MFMA roofline of each whole pass."""
    import torch
    from pseudobrain_amd import gated_deltanet as gd
    from pseudobrain_amd.workloads import STREAM_SEGMENT, WORKLOADS, generate, varlen_workload
    out = {}
    s = WORKLOADS["varlen_8seq"]
    q, k, v, g, beta, h0, cu = varlen_workload(seed=0, device="cuda")
    scale = s.dk ** -0.5
    o = torch.empty(1, s.length, s.hv, s.dv, dtype=torch.bfloat16, device="cuda")

    def varlen():
        gd.chunk_fwd(q, k, v, g, beta, scale, h0, cu, out=o)

    sec, ksec = timed_steps(varlen, steps, warmup)
    flops = prefill_flops(s.length, s.hv, s.dk, s.dv)
    out["varlen_8seq"] = {"T": s.length, "sequences": cu.numel() - 1, "value": s.length / sec / 1e6,
                          "unit": "Mtok/s", "ms_per_call": sec * 1e3,
                          "roofline": {"bound": "mfma", "achieved": flops / ksec / 1e12, "peak": MFMA_PEAK_TFLOPS,
                                       "unit": "TFLOP/s", "frac": flops / ksec / 1e12 / MFMA_PEAK_TFLOPS}}
    del q, k, v, g, beta, h0, o
    s = WORKLOADS["stream_1m"]
    q, k, v, g, beta, h0 = generate(1, s.length, s.hk, s.hv, s.dk, s.dv, s.dtype, s.h0_std, seed=0, device="cuda")
    o = torch.empty(1, STREAM_SEGMENT, s.hv, s.dv, dtype=torch.bfloat16, device="cuda")

    def stream():
        state = h0
        for lo in range(0, s.length, STREAM_SEGMENT):
            sl = slice(lo, lo + STREAM_SEGMENT)
            _, state = gd.chunk_fwd(q[:, sl], k[:, sl], v[:, sl], g[:, sl], beta[:, sl], scale, state, out=o)

    sec, ksec = timed_steps(stream, max(1, steps // 2), warmup)
    flops = prefill_flops(s.length, s.hv, s.dk, s.dv)
    out["stream_1m"] = {"T": s.length, "segments": s.length // STREAM_SEGMENT, "value": s.length / sec / 1e6,
                        "unit": "Mtok/s", "ms_per_pass": sec * 1e3,
                        "roofline": {"bound": "mfma", "achieved": flops / ksec / 1e12, "peak": MFMA_PEAK_TFLOPS,
                                     "unit": "TFLOP/s", "frac": flops / ksec / 1e12 / MFMA_PEAK_TFLOPS}}
    del q, k, v, g, beta, h0, o
    # Serving-style batches of the same 32,768 tokens (ungraded): many packed
    # sequences, each from its own state (the scan runs them back to back).
    from pseudobrain_amd.workloads import cu_seqlens_of
    o = torch.empty(1, 32768, 32, 128, dtype=torch.bfloat16, device="cuda")
    batches = {}
    for nseq in (64, 256):
        length = 32768 // nseq
        q, k, v, g, beta, h0 = generate(1, 32768, 16, 32, 128, 128, torch.bfloat16, 0.02, seed=0, nstates=nseq,
                                        device="cuda")
        cu = cu_seqlens_of([length] * nseq).to("cuda")

        def packed():
            gd.chunk_fwd(q, k, v, g, beta, scale, h0, cu, out=o)

        sec, ksec = timed_steps(packed, steps, warmup)
        batches[f"{nseq}x{length}"] = {"value": 32768 / ksec / 1e6, "unit": "Mtok/s", "ms_per_call": ksec * 1e3}
    out["serving_prefill_ungraded"] = batches
    return out


def layer_inputs(length):
    """Synthetic layer inputs at the Qwen3-Next layer shape (Hk=16, Hv=32,
    K=V=128, conv 4): a bf16 projection z [1, T, q|k|v|gate|a|b], fp32 tail,
    conv weight, A_log, dt_bias, o_norm, and a bf16 operator output o."""
    import torch
    gen = torch.Generator().manual_seed(0)
    hk, hv, dk, dv, conv = 16, 32, 128, 128, 4
    channels = 2 * hk * dk + hv * dv
    z = torch.randn(1, length, channels + hv * dv + 2 * hv, generator=gen).to(torch.bfloat16).cuda()
    tail = torch.randn(1, conv - 1, channels, generator=gen).cuda()
    weight = ((torch.rand(channels, conv, generator=gen) * 2 - 1) / 2).cuda()
    a_log = torch.empty(hv).uniform_(0, 16, generator=gen).log().cuda()
    dt_bias = (torch.randn(hv, generator=gen) - 4).cuda()
    o = (torch.randn(1, length, hv, dv, generator=gen) * 0.1).to(torch.bfloat16).cuda()
    o_norm = torch.ones(dv).cuda()
    return dict(hk=hk, hv=hv, dk=dk, dv=dv, conv=conv, channels=channels, z=z, tail=tail, weight=weight,
                a_log=a_log, dt_bias=dt_bias, o=o, o_norm=o_norm)


def bench_layer(length, steps, warmup=3):
    """The fused prologue and epilogue kernels over T tokens of the layer shape:
    HBM-bound; algorithmic bytes = what each must read and write once."""
    import torch
    from pseudobrain_amd.layer import layer_epilogue, layer_prologue, layer_prologue_varlen
    x = layer_inputs(length)
    hk, hv, dk, dv, ch = x["hk"], x["hv"], x["dk"], x["dv"], x["channels"]

    def pro():
        layer_prologue(x["z"], x["tail"], x["weight"], x["a_log"], x["dt_bias"], hk, dk, hv, dv)

    gate = x["z"][..., ch:ch + hv * dv]

    def epi():
        layer_epilogue(x["o"], gate, x["o_norm"], out_dtype=torch.float32)

    # the same tokens as 64 packed sequences against a pool of 64 fp32 conv tails
    nseq = 64
    cu = torch.tensor([i * length // nseq for i in range(nseq + 1)], dtype=torch.int32).cuda()
    pool = x["tail"].repeat(nseq, 1, 1).contiguous()
    slots = torch.arange(nseq, dtype=torch.int32).cuda()

    def pro_varlen():
        layer_prologue_varlen(x["z"], cu, pool, x["weight"], x["a_log"], x["dt_bias"], hk, dk, hv, dv, slots)

    out = {}
    # prologue: q|k|v bf16 in and out, a|b bf16 in, g, beta fp32 out, the tail fp32 in and out
    pro_bytes = length * (ch * 2 * 2 + 2 * hv * 2 + 2 * hv * 4) + 2 * (x["conv"] - 1) * ch * 4
    varlen_bytes = pro_bytes + (nseq - 1) * 2 * (x["conv"] - 1) * ch * 4
    # epilogue: o bf16 and gate bf16 in, hs fp32 out
    epi_bytes = length * hv * dv * (2 + 2 + 4)
    for name, fn, nbytes in (("layer_prologue", pro, pro_bytes), ("layer_prologue_varlen64", pro_varlen,
                                                                  varlen_bytes), ("layer_epilogue", epi, epi_bytes)):
        sec, ksec = timed_steps(fn, steps, warmup)
        gbs = nbytes / ksec / 1e9
        out[name] = {"T": length, "us_per_call": sec * 1e6, "kernel_us": ksec * 1e6, "bytes_per_call": nbytes,
                     "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                  "frac": gbs / HBM_PEAK_GBS}}
    return out


def bench_layer_core(steps, warmup=3, rounds=3):
    """The prefill layer core (the operator, then RMSNorm x o_norm x SiLU(gate))
    over 32,768 tokens of the Qwen3-Next head shape, bf16 in, fp32 hs out: one
    call (chunk_layer_fwd) against the operator (chunk_fwd) followed by the
    epilogue kernel (layer_epilogue). At 8 x 4,096 the wide scan applies the
    epilogue itself; at 1 x 32,768 (the narrow scan) both forms are two passes.
    The forms alternate for `rounds` rounds; each figure is its median."""
    import torch
    from pseudobrain_amd import gated_deltanet as gd
    from pseudobrain_amd.layer import chunk_layer_fwd, layer_epilogue
    from pseudobrain_amd.workloads import cu_seqlens_of, generate
    out = {}
    gen = torch.Generator().manual_seed(3)
    z = torch.randn(1, 32768, 2 * 32 * 128, generator=gen).to(torch.bfloat16).cuda()
    gate = z[..., 32 * 128:]
    o_norm = (torch.rand(128, generator=gen) + 0.5).cuda()
    scale = 128 ** -0.5
    for nseq in (8, 1):
        q, k, v, g, beta, h0 = generate(1, 32768, 16, 32, 128, 128, torch.bfloat16, 0.02, seed=0, nstates=nseq,
                                        device="cuda")
        cu = cu_seqlens_of([32768 // nseq] * nseq).to("cuda")

        def fused():
            chunk_layer_fwd(q, k, v, g, beta, scale, h0, gate, o_norm, 1e-5, cu)

        def two_pass():
            o, _ = gd.chunk_fwd(q, k, v, g, beta, scale, h0, cu)
            layer_epilogue(o, gate, o_norm, 1e-5)

        kf, kt = [], []
        with torch.no_grad():
            for _ in range(rounds):
                kf.append(timed_steps(fused, steps, warmup)[1])
                kt.append(timed_steps(two_pass, steps, warmup)[1])
        kf, kt = statistics.median(kf), statistics.median(kt)
        out[f"{nseq}x{32768 // nseq}"] = {"one_call_ms": kf * 1e3, "operator_then_epilogue_ms": kt * 1e3,
                                          "Mtok_s_one_call": 32768 / kf / 1e6}
    return {"layer_core_ungraded": out}


def bench_decode_layer(batch, steps, warmup=10, state_dtype=None, conv_dtype=None, resident=True):
    """The fused decode step of the whole layer (pbgdn_decode_layer_fwd) at the
    Qwen3-Next layer shape for `batch` sequences of one token, state and conv
    pools updated in place, against the same step as three launches (the
    layer prologue, the recurrent step, the epilogue). HBM roofline of the
    fused step: the state read and written, the projection row read, the conv
    tail read and written, hs written. `conv_dtype` is the conv tail's dtype
    (float32 by default). The one pool is stepped in a loop and declared
    resident (`resident`), as bench_decode's one-pool lines are."""
    import torch
    from pseudobrain_amd.layer import decode_layer_step, layer_epilogue, layer_prologue
    gen = torch.Generator().manual_seed(1)
    hk, hv, dk, dv, conv = 16, 32, 128, 128, 4
    channels = 2 * hk * dk + hv * dv
    width = channels + hv * dv + 2 * hv
    z = torch.randn(batch, width, generator=gen).to(torch.bfloat16).cuda()
    pool = torch.randn(batch, conv - 1, channels, generator=gen).to(conv_dtype or torch.float32).cuda()
    weight = ((torch.rand(channels, conv, generator=gen) * 2 - 1) / 2).cuda()
    a_log = torch.empty(hv).uniform_(0, 16, generator=gen).log().cuda()
    dt_bias = (torch.randn(hv, generator=gen) - 4).cuda()
    state = (torch.randn(batch, hv, dk, dv, generator=gen) * 0.02).cuda()
    if state_dtype is not None:
        state = state.to(state_dtype)
    o_norm = torch.ones(dv).cuda()

    def fused():
        decode_layer_step(z, pool, weight, a_log, dt_bias, state, o_norm, hk, dk, hv, dv, state_resident=resident)

    def three():
        q, k, v, g, beta, gate, new_tail = layer_prologue(z[:, None], pool, weight, a_log, dt_bias, hk, dk, hv, dv)
        o = torch.ops.pbgdn.recurrent_step_(q, k, v, g, beta, state, None, dk ** -0.5, resident)
        layer_epilogue(o, gate, o_norm)

    sec, ksec = timed_steps(fused, steps, warmup)
    sec3, ksec3 = timed_steps(three, steps, warmup)
    nbytes = (2 * batch * hv * dk * dv * state.element_size() + batch * width * 2
              + 2 * batch * (conv - 1) * channels * pool.element_size()
              + batch * hv * dv * 4)
    gbs = nbytes / ksec / 1e9
    return {"batch": batch, "state_dtype": str(state.dtype).replace("torch.", ""), "steps": steps,
            "state_policy": "resident" if resident else "stream",
            "us_per_step": sec * 1e6, "kernel_us": ksec * 1e6, "bytes_per_step": nbytes,
            "three_launches_us_per_step": ksec3 * 1e6,
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs / HBM_PEAK_GBS}}


STREAM_PROBE_BYTES = 1 << 30


def stream_probe(reps=20):
    """The library's streaming copy (pbgdn_stream_probe: 16-byte non-temporal
    buffer loads and stores) over 1 GiB: the read + write bandwidth a plain
    stream sustains on this GPU, the ceiling the decode step's state traffic
    is read against."""
    import torch
    from pseudobrain_amd import _lib
    src = torch.ones(STREAM_PROBE_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    stream = torch.cuda.current_stream().cuda_stream

    def step():
        _lib.check(_lib.lib().pbgdn_stream_probe(src.data_ptr(), dst.data_ptr(), STREAM_PROBE_BYTES, stream),
                   "pbgdn_stream_probe")

    step()
    torch.cuda.synchronize()
    assert torch.equal(dst[:: 1 << 20], src[:: 1 << 20])
    ksec = kernel_time(step, reps)
    gbs = 2 * STREAM_PROBE_BYTES / ksec / 1e9
    return {"bytes_read": STREAM_PROBE_BYTES, "bytes_written": STREAM_PROBE_BYTES, "kernel_us": ksec * 1e6,
            "GBs": gbs, "hbm_frac": gbs / HBM_PEAK_GBS}


def copy_probe(reps=5):
    """A plain device copy of COPY_PROBE_BYTES (torch's copy kernel): the
    reference point that scales the FETCH_SIZE/WRITE_SIZE counters, and a
    practical read+write bandwidth ceiling on this GPU."""
    import torch
    src = torch.ones(COPY_PROBE_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)

    def step():
        dst.copy_(src)

    step()
    ksec = kernel_time(step, reps)
    return {"bytes_read": COPY_PROBE_BYTES, "bytes_written": COPY_PROBE_BYTES, "kernel_us": ksec * 1e6,
            "GBs": 2 * COPY_PROBE_BYTES / ksec / 1e9}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--decode-steps", type=int, default=1000)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-b256", action="store_true", help="skip the ungraded 256-sequence decode")
    ap.add_argument("--copy-probe", action="store_true", help="also time a plain 256 MiB device copy")
    ap.add_argument("--no-layer", action="store_true", help="skip the layer prologue/epilogue kernels")
    ap.add_argument("--no-long", action="store_true", help="skip the varlen and streamed prefill workloads")
    ap.add_argument("--no-backward", action="store_true", help="skip the chunk backward")
    ap.add_argument("--no-k256", action="store_true", help="skip the 256-wide-head prefill")
    args = ap.parse_args(argv)
    world = int(os.environ.get("WORLD_SIZE", args.gpus))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the operator runs on a single MI355X (heads and "
              "sequences shard with no exchange; see the sharding design). Use --gpus 1.",
              file=sys.stderr)
        return 2

    cpu = cpu_baseline() if not args.no_cpu else None

    import torch
    from pseudobrain_amd import _lib
    _lib.lib()
    torch.cuda.init()
    shape, sec, ksec, flops, nbytes = bench_prefill(args.steps, args.warmup)
    achieved = flops / ksec / 1e12
    result = {
        "metric": "GDN prefill Mtok/s @T=32K; decode step µs @B=64 and % HBM peak BW",
        "value": shape.length / sec / 1e6,
        "unit": "Mtok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": sec * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "device_warmup_s": DEVICE_WARMUP_S,
        "dtype": "bf16 in; f16 MFMA operands, f32 accumulate and state",
        "data": "synthetic (seeded; q,k L2-normalised; beta=sigmoid(N); g=-softplus(N); h0~N(0,0.02))",
        "config": {"workload": "prefill_qwen3next", "B": shape.batch, "T": shape.length,
                   "Hk": shape.hk, "Hv": shape.hv, "K": shape.dk, "V": shape.dv, "chunk": 64,
                   "out_dtype": "bf16", "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / MFMA_PEAK_TFLOPS, "traffic": measured_traffic("chunk"),
                     "kernel_ms": ksec * 1e3, "algorithmic_flops": flops, "algorithmic_bytes": nbytes,
                     "hbm_GBs_algorithmic": nbytes / ksec / 1e9,
                     "io_bound_TFLOPs": min(MFMA_PEAK_TFLOPS, flops / nbytes * HBM_PEAK_GBS / 1e3)},
        "cpu_baseline": cpu,
    }
    if cpu is not None:
        result["cpu_baseline_ratio"] = result["value"] / cpu["value"]
    result["prefill_small"] = bench_prefill_small()
    if not args.no_k256:
        result["prefill_k256_ungraded"] = bench_prefill_k256()
    if not args.no_decode:
        # the c2 workload: one pool stepped 1000 times in place, declared resident
        dec = bench_decode(64, args.decode_steps, resident=True)
        result["decode"] = dict(dec, roofline={"bound": "hbm", "achieved": dec["achieved_GBs"],
                                               "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                               "frac": dec["hbm_frac"],
                                               "traffic": measured_traffic("recurrent_b64")})
        # vLLM keeps the recurrent state in the model's dtype unless told otherwise
        bf = bench_decode(64, args.decode_steps, state_dtype=torch.bfloat16, resident=True)
        result["decode_bf16_state"] = dict(bf, roofline={"bound": "hbm", "achieved": bf["achieved_GBs"],
                                                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                                         "frac": bf["hbm_frac"],
                                                         "traffic": measured_traffic("recurrent_b64_bf16_state")})
        # the same step as a model takes it: three 128 MiB pools in rotation, so
        # the state comes from HBM, with the default (streamed) policy
        ooc = bench_decode(64, 300, pools=3)
        result["decode_out_of_cache"] = dict(ooc, roofline={"bound": "hbm", "achieved": ooc["achieved_GBs"],
                                                            "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                                            "frac": ooc["hbm_frac"],
                                                            "traffic": measured_traffic("recurrent_b64_out_of_cache")})
        if not args.no_b256:
            result["decode_b256_ungraded"] = bench_decode(256, 200)
        probe = stream_probe()
        result["stream_probe"] = probe
        for key in ("decode", "decode_out_of_cache", "decode_b256_ungraded"):
            if key in result:
                result[key]["vs_stream_probe"] = result[key]["achieved_GBs"] / probe["GBs"]
    if not args.no_layer:
        result.update(bench_layer(shape.length, 20))
        result.update(bench_layer_core(10))
        if not args.no_decode:
            result["decode_layer_b64"] = bench_decode_layer(64, 200)
            result["decode_layer_b64"]["roofline"]["traffic"] = measured_traffic("decode_layer_b64")
            result["decode_layer_b64_bf16_state"] = bench_decode_layer(64, 200, state_dtype=torch.bfloat16)
            # the conv tail in the projection's dtype, as a serving cache holds it
            result["decode_layer_b64_bf16_tail"] = bench_decode_layer(64, 200, conv_dtype=torch.bfloat16)
    if not args.no_backward:
        result["backward"] = bench_backward()
    if not args.no_long:
        result.update(bench_long())
    if args.copy_probe:
        result["copy_probe"] = copy_probe()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
