#!/usr/bin/env python3
"""Gated delta-rule benchmark on one MI355X (gfx950).

Headline (the JSON line's `value`): chunked prefill throughput in tokens/s on
B=4, H=16, T=4096, d_k=d_v=128, bf16 q/k/v, fp32 gates/state, chunk 64 --
one step = one rhz_gdr_prefill over the whole batch (all heads), inputs
resident in HBM.  Alongside (`decode`): the decode state update on B=256,
H=16, d=128, fp32 state, one rhz_gdr_decode_step launch per step over 64
steps, as HBM GB/s, and (`decode_large_state`) the same step with a 1.07 GB
state (B=1024), four times the last-level cache; (`multistep`)
rhz_gdr_multistep over 8 positions on the same shape, as HBM GB/s;
(`prologue_epilogue`) the conv1d, prepare and per-head RMSNorm ops on the
prefill workload's tokens, as HBM GB/s; (`local_block`)
rhz_gdr_local_prefill, the prefill with prepare fused in, from raw
projections on the prefill shape, beside rhz_gdr_prepare + rhz_gdr_prefill;
(`prefill_long_context`, `prefill_varlen`) the chunked prefill on B=1, H=32,
T=32768, d_v=256 with slow decay, and on 64 packed sequences of 128..8192
tokens with initial states; (`prefill_fp32`) the fp32-input path (the
token-sequential recurrent kernel) on the headline prefill shape;
(`local_chain`) the whole Local-block mixer, from the q, k, v projections
through conv1d, prepare, the prefill and the per-head RMSNorm, in three
arrangements of the library's calls.  Every leg first runs a settle phase of untimed
launches (`--settle-ms`, recorded per leg), then its warmup, then the timed
launches.

Inputs are synthetic and seeded: the reference's Philox-4x32-10 streams
(q=1, k=2, v=3, beta=4, g=5, state=6), generated on the device by
rhz_philox_fill.  Timing uses HIP events on the stream the library launches
on.  `roofline.achieved` counts algorithmic work only:
  prefill bytes per token-head: (2 d_k + d_v) 2 + 2 d_v + 8, plus the fp32
    final state (4 d_k d_v per sequence-head); flops per (chunk of c tokens,
    head): 6 c^2 d_k + 4 c^2 d_v + 6 c d_k d_v (roofline.mfma)
  decode bytes per (b, h): 8 d_k d_v + 4 (2 d_k + 2 d_v) + 8
`cpu_baseline` times the f64 CPU oracle (a restatement of
crates/ops/src/delta.rs) on this host in the same run.

`--calibration-copy` adds one elementwise copy kernel over 256 MiB after
the timed regions: HBM byte counters (rocprofv3 FETCH_SIZE / WRITE_SIZE) read
on that copy give the scale from counter units to bytes.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--settle-ms MS]
                    [--no-cpu-baseline] [--calibration-copy]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "GDR prefill tokens/s + decode state-update HBM GB/s on 1 MI355X"
PEAK_MFMA_TFLOPS = 2500.0   # MI355X dense bf16/fp16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
PEAK_FP32_TFLOPS = 157.3    # MI355X fp32 vector (packed)

PREFILL = dict(batch=4, heads=16, seq_len=4096, d_k=128, d_v=128, chunk=64)
# long context, slow decay: g = -softplus(N(-2, 1))
PREFILL_LONG = dict(batch=1, heads=32, seq_len=32768, d_k=128, d_v=256, chunk=64, g_mean=-2.0)
# 64 packed sequences, lengths 128 + floor(u * 8065) from Philox stream 7,
# initial states N(0, 0.02)
PREFILL_VARLEN = dict(n_seqs=64, heads=16, d_k=128, d_v=128, chunk=64, len_lo=128, len_hi=8192,
                      state_std=0.02)
DECODE = dict(batch=256, heads=16, d_k=128, d_v=128, steps=64)
# the same step with a 1.07 GB state, over 4x the 256 MB last-level cache
DECODE_LARGE = dict(batch=1024, heads=16, d_k=128, d_v=128, steps=16)
MULTISTEP = dict(batch=256, heads=16, d_k=128, d_v=128, positions=8)


def device_info(torch) -> dict:
    """Name, compute units and peak shader clock of GPU 0, and the dense
    fp16/bf16 MFMA peak those give (4096 flop per CU per clock on gfx950),
    beside the published figure the roofline uses."""
    props = torch.cuda.get_device_properties(0)
    info = {"name": torch.cuda.get_device_name(0), "compute_units": props.multi_processor_count}
    try:
        hip = ctypes.CDLL("libamdhip64.so")
        khz = ctypes.c_int(0)
        # hipDeviceGetAttribute(&v, hipDeviceAttributeClockRate (= 5), device 0): kHz
        if hip.hipDeviceGetAttribute(ctypes.byref(khz), 5, 0) == 0 and khz.value > 0:
            info["peak_clock_mhz"] = khz.value / 1000.0
            info["mfma_peak_at_clock_tflops"] = props.multi_processor_count * khz.value * 1e3 * 4096 / 1e12
    except OSError:
        pass
    info["mfma_peak_used_tflops"] = PEAK_MFMA_TFLOPS
    info["hbm_peak_used_gbs"] = PEAK_HBM_GBS
    return info


def prefill_flops(lengths, heads, dk, dv, chunk=64) -> float:
    total = 0
    for n in lengths:
        full, rem = divmod(int(n), chunk)
        for c in [chunk] * full + ([rem] if rem else []):
            total += 6 * c * c * dk + 4 * c * c * dv + 6 * c * dk * dv
    return float(total * heads)


def prefill_bytes(tokens, heads, dk, dv, n_seqs, e_in=2, e_out=2, init_state=False) -> float:
    per_tok = (2 * dk + dv) * e_in + dv * e_out + 2 * 4
    states = n_seqs * heads * dk * dv * 4 * (2 if init_state else 1)
    return float(tokens * heads * per_tok + states)


def decode_bytes(batch, heads, dk, dv) -> float:
    return float(batch * heads * (2 * 4 * dk * dv + 4 * (2 * dk + 2 * dv) + 8))


PROFILES = {
    "prefill": "gdr_chunk_kernel_128_prefill_b4_h16_t4096_d128.md",
    "prefill_long": "gdr_chunk_kernel_128_prefill_b1_h32_t32768_dk128_dv256.md",
    "prefill_varlen": "gdr_chunk_kernel_128_prefill_varlen64_h16_d128.md",
    "decode": "gdr_decode_kernel_decode_b256_h16_d128.md",
    "decode_large": "gdr_decode_kernel_decode_b1024_h16_d128.md",
    "multistep": "gdr_multistep_kernel_b256_h16_d128_n8.md",
    "conv1d": "conv1d_kernel_bf16_t16384_c6144.md",
    "prepare": "prepare_kernel_bf16_t16384_h16_d128.md",
    "rmsnorm": "rmsnorm_kernel_bf16_rows262144_d128.md",
    "local": "gdr_chunk_kernel_128_pro_local_b4_h16_t4096_d128.md",
    "prefill_fp32": "gdr_staged_recurrent_kernel_prefill_fp32_b4_h16_t4096_d128.md",
    "conv_prepare": "conv_prepare_kernel_bf16_t16384_h16_d128.md",
}


def traffic_from_profiles(kind: str):
    """HBM bytes per launch measured with rocprofv3 PMC counters (FETCH_SIZE,
    WRITE_SIZE, scaled by a copy kernel of known size), from the committed
    kernel summary under profiles/ (line `traffic: <bytes>`)."""
    path = os.path.join(ROOT, "profiles", PROFILES[kind])
    if not os.path.exists(path):
        return None
    for line in open(path):
        m = re.match(r"\s*traffic:\s*([0-9.eE+]+)", line)
        if m:
            return float(m.group(1))
    return None


def multistep_bytes(batch, heads, dk, dv, n) -> float:
    """fp32 state read once, n snapshots written, n positions of fp32 q, k, v, o and gates."""
    return float(batch * heads * (4 * dk * dv * (1 + n) + n * (4 * (2 * dk + 2 * dv) + 8)))


SETTLE_MS = 150.0  # wall time of untimed launches before each leg's counted warmup


def set_settle_ms(ms: float) -> None:
    global SETTLE_MS
    SETTLE_MS = float(ms)


def settle(torch, fn, frac: float = 1.0) -> dict:
    """Runs fn back to back for at least frac * SETTLE_MS of wall time before
    anything is counted.  The GPU's clocks ramp up over the first tens of
    milliseconds of sustained work; without this, a short counted warmup
    leaves the timed launches on a rising clock.  Nothing here is timed or
    reported as a result: the JSON line records how long the settle phase ran
    and how many launches it made (so that a kernel trace of the run can be
    split into each leg's settle, warmup and timed launches)."""
    ms = SETTLE_MS * frac
    t0 = time.perf_counter()
    n = 0
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(10):
            fn()
        n += 10
        torch.cuda.synchronize()
    return {"settle_ms": (time.perf_counter() - t0) * 1e3, "settle_launches": n}


def time_region(torch, stream, fn, reps: int) -> float:
    """Milliseconds per call of fn over reps calls, HIP events on `stream`."""
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(reps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / reps


def varlen_lengths_dev(torch, n, lo, hi, seed=0):
    """Seeded lengths lo + floor(u (hi - lo + 1)), u = next_f64 #i of Philox
    stream 7 (rng.rs:78-82), drawn on the device."""
    u = __import__("rhizome_amd").philox_fill("uniform", seed, 7, (n,), torch.float64)
    return [int(x) for x in (lo + torch.floor(u * (hi - lo + 1))).cpu().tolist()]


def bench_prefill(torch, steps, warmup, c=None):
    """One prefill leg: a dense batch (batch, seq_len) or a packed one
    (lengths, with per-sequence initial states).  Returns the timing, the
    algorithmic work and the device inputs."""
    import rhizome_amd
    from rhizome_amd import _abi, gdr

    c = c or PREFILL
    H, dk, dv = c["heads"], c["d_k"], c["d_v"]
    dev = torch.device("cuda:0")
    bf16, f32 = torch.bfloat16, torch.float32
    if "lengths" in c:
        lengths = c["lengths"]
        n_tok, lead = sum(lengths), (sum(lengths),)
        cu = torch.tensor([0] + list(__import__("itertools").accumulate(lengths)), dtype=torch.int32,
                          device=dev)
        n_seq = len(lengths)
    else:
        B, T = c["batch"], c["seq_len"]
        lengths, n_tok, lead, cu, n_seq = [T] * B, B * T, (B, T), None, B
    q = rhizome_amd.philox_fill("unit_rows", 0, 1, lead + (H, dk), bf16)
    k = rhizome_amd.philox_fill("unit_rows", 0, 2, lead + (H, dk), bf16)
    v = rhizome_amd.philox_fill("normal", 0, 3, lead + (H, dv), bf16)
    beta = rhizome_amd.philox_fill("sigmoid", 0, 4, lead + (H,), f32)
    g = rhizome_amd.philox_fill("neg_softplus", 0, 5, lead + (H,), f32, mean=c.get("g_mean", 0.0))
    init = None
    if c.get("state_std"):
        init = rhizome_amd.philox_fill("normal", 0, 6, (n_seq, H, dv, dk), f32, std=c["state_std"])
    o = torch.empty(lead + (H, dv), dtype=bf16, device=dev)
    fin = torch.empty((n_seq, H, dv, dk), dtype=f32, device=dev)
    args = gdr.prefill_args(q, k, v, g, beta, _abi.GATE_LOG_ALPHA, cu, init, fin, o, "chunked")
    ws = torch.empty(max(gdr.workspace_bytes(args), 256), dtype=torch.uint8, device=dev)
    args.workspace, args.workspace_bytes = ws.data_ptr(), ws.numel()
    stream = torch.cuda.current_stream()
    lib, argp, sp = _abi.lib(), ctypes.byref(args), ctypes.c_void_p(stream.cuda_stream or None)

    def step():
        st = lib.rhz_gdr_prefill(argp, sp)
        if st:
            _abi.check(st)

    info = settle(torch, step)
    for _ in range(warmup):
        step()
    ms = time_region(torch, stream, step, steps)
    if rhizome_amd.sync_timeouts() != 0:
        raise RuntimeError("a chunked-kernel LDS wait gave up during the benchmark")
    if rhizome_amd.fp16_range_errors() != 0:
        raise RuntimeError("a chunked-kernel fp16 operand was out of range during the benchmark")
    if rhizome_amd.exact_reruns() != 0:
        raise RuntimeError("chunked-kernel workgroups took the exact rerun during the benchmark")
    flops = prefill_flops(lengths, H, dk, dv)
    algo_bytes = prefill_bytes(n_tok, H, dk, dv, n_seq, init_state=init is not None)
    host = {"q": q, "k": k, "v": v, "g": g, "beta": beta, "tokens": n_tok, **info}
    return ms, flops, algo_bytes, host


def prefill_leg(torch, steps, warmup, c, workload, profile_key) -> dict:
    """A secondary prefill workload as its own JSON object."""
    ms, flops, nbytes, host = bench_prefill(torch, steps, warmup, c)
    gbs = nbytes / (ms * 1e-3) / 1e9
    tflops = flops / (ms * 1e-3) / 1e12
    cfg = {k: v for k, v in c.items() if k != "lengths"}
    if "lengths" in c:
        cfg.update(n_seqs=len(c["lengths"]), tokens=host["tokens"], min_len=min(c["lengths"]),
                   max_len=max(c["lengths"]))
    return {"metric": "GDR prefill tokens/s", "value": host["tokens"] / (ms * 1e-3), "unit": "tokens/s",
            "ms_per_step": ms, "steps": steps, "warmup": warmup, "settle_ms": host["settle_ms"],
            "settle_launches": host["settle_launches"],
            "config": {"workload": workload, **cfg},
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": gbs / PEAK_HBM_GBS, "traffic": traffic_from_profiles(profile_key),
                         "kernel": "gdr_chunk_kernel<128, false>", "algorithmic_bytes": nbytes,
                         "launch_us": ms * 1e3,
                         "mfma": {"achieved": tflops, "peak": PEAK_MFMA_TFLOPS, "unit": "TFLOP/s",
                                  "frac": tflops / PEAK_MFMA_TFLOPS, "flops_per_launch": flops}}}


def bench_prefill_fp32(torch, steps, warmup) -> dict:
    """The fp32-input path on the headline prefill shape: rhz_gdr_prefill with
    fp32 q/k/v/o and RHZ_ALGO_RECURRENT (gdr_staged_recurrent_kernel, token by
    token, one wave per 4 state rows of a head (16 lanes of 8 key columns per
    row), eight waves sharing each 32-position block of k, q, gates and k.q
    staged through LDS, two waves per SIMD)."""
    import rhizome_amd
    from rhizome_amd import _abi, gdr

    c = PREFILL
    B, T, H, dk, dv = c["batch"], c["seq_len"], c["heads"], c["d_k"], c["d_v"]
    dev = torch.device("cuda:0")
    f32 = torch.float32
    lead = (B, T)
    q = rhizome_amd.philox_fill("unit_rows", 0, 1, lead + (H, dk), f32)
    k = rhizome_amd.philox_fill("unit_rows", 0, 2, lead + (H, dk), f32)
    v = rhizome_amd.philox_fill("normal", 0, 3, lead + (H, dv), f32)
    beta = rhizome_amd.philox_fill("sigmoid", 0, 4, lead + (H,), f32)
    g = rhizome_amd.philox_fill("neg_softplus", 0, 5, lead + (H,), f32)
    o = torch.empty(lead + (H, dv), dtype=f32, device=dev)
    fin = torch.empty((B, H, dv, dk), dtype=f32, device=dev)
    args = gdr.prefill_args(q, k, v, g, beta, _abi.GATE_LOG_ALPHA, None, None, fin, o, "recurrent")
    stream = torch.cuda.current_stream()
    lib, argp, sp = _abi.lib(), ctypes.byref(args), ctypes.c_void_p(stream.cuda_stream or None)

    def step():
        st = lib.rhz_gdr_prefill(argp, sp)
        if st:
            _abi.check(st)

    info = settle(torch, step, 1 / 2)
    for _ in range(warmup):
        step()
    ms = time_region(torch, stream, step, steps)
    tokens = B * T
    nbytes = prefill_bytes(tokens, H, dk, dv, B, e_in=4, e_out=4)
    gbs = nbytes / (ms * 1e-3) / 1e9
    # the recurrence's own arithmetic, per token-head: S k, S q and k q, the
    # rank-1 update and o (about 8 d_k d_v multiply-adds' worth; fp32 VALU)
    flops = float(tokens * H * 8 * dk * dv)
    return {"metric": "GDR prefill tokens/s, fp32 inputs", "value": tokens / (ms * 1e-3), "unit": "tokens/s",
            "ms_per_step": ms, "steps": steps, "warmup": warmup, **info,
            "config": {"workload": "recurrent GDR prefill, fp32 q/k/v/o", "batch": B, "heads": H,
                       "seq_len": T, "d_k": dk, "d_v": dv, "inputs": "fp32 q/k/v, fp32 log-decay and beta",
                       "state": "fp32"},
            # token-sequential: every wave walks the T positions of its head
            # one after the other, so the launch is bound by the per-position
            # latency of that chain, not by HBM
            "latency": {"ns_per_position": ms * 1e6 / T, "positions_per_wave": T,
                        "waves": B * H * ((dv + 3) // 4)},
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": gbs / PEAK_HBM_GBS, "traffic": traffic_from_profiles("prefill_fp32"),
                         "kernel": "gdr_staged_recurrent_kernel<16,float,8,8>", "algorithmic_bytes": nbytes,
                         "launch_us": ms * 1e3,
                         "fp32_valu": {"achieved": flops / (ms * 1e-3) / 1e12, "peak": PEAK_FP32_TFLOPS,
                                       "unit": "TFLOP/s",
                                       "frac": flops / (ms * 1e-3) / 1e12 / PEAK_FP32_TFLOPS}}}


def bench_decode(torch, warmup, c=None):
    import rhizome_amd
    from rhizome_amd import _abi, gdr

    c = c or DECODE
    B, H, dk, dv, n = c["batch"], c["heads"], c["d_k"], c["d_v"], c["steps"]
    f32 = torch.float32
    q = rhizome_amd.philox_fill("unit_rows", 0, 1, (n, B, H, dk), f32)
    k = rhizome_amd.philox_fill("unit_rows", 0, 2, (n, B, H, dk), f32)
    v = rhizome_amd.philox_fill("normal", 0, 3, (n, B, H, dv), f32)
    beta = rhizome_amd.philox_fill("sigmoid", 0, 4, (n, B, H), f32)
    g = rhizome_amd.philox_fill("neg_softplus", 0, 5, (n, B, H), f32)
    state = rhizome_amd.philox_fill("normal", 0, 6, (B, H, dv, dk), f32, std=0.02)
    o = torch.empty((n, B, H, dv), dtype=f32, device=q.device)
    lib = _abi.lib()
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream or None)
    argv = [gdr.decode_args(q[t], k[t], v[t], g[t], beta[t], _abi.GATE_LOG_ALPHA, state, o[t])
            for t in range(n)]
    ptrs = [ctypes.byref(a) for a in argv]
    count = [0]

    def step():
        st = lib.rhz_gdr_decode_step(ptrs[count[0] % n], sp)
        count[0] += 1
        if st:
            _abi.check(st)

    info = settle(torch, step)
    for _ in range(warmup):
        step()
    ms = time_region(torch, stream, step, n)
    return ms, decode_bytes(B, H, dk, dv), {"q": q, "k": k, "v": v, "g": g, "beta": beta, **info}


def bench_multistep(torch, steps, warmup):
    import rhizome_amd
    from rhizome_amd import _abi, gdr

    c = MULTISTEP
    B, H, dk, dv, n = c["batch"], c["heads"], c["d_k"], c["d_v"], c["positions"]
    f32 = torch.float32
    q = rhizome_amd.philox_fill("unit_rows", 0, 1, (B, n, H, dk), f32)
    k = rhizome_amd.philox_fill("unit_rows", 0, 2, (B, n, H, dk), f32)
    v = rhizome_amd.philox_fill("normal", 0, 3, (B, n, H, dv), f32)
    beta = rhizome_amd.philox_fill("sigmoid", 0, 4, (B, n, H), f32)
    g = rhizome_amd.philox_fill("neg_softplus", 0, 5, (B, n, H), f32)
    state = rhizome_amd.philox_fill("normal", 0, 6, (B, H, dv, dk), f32, std=0.02)
    o = torch.empty((B, n, H, dv), dtype=f32, device=q.device)
    states = torch.empty((B, n, H, dv, dk), dtype=f32, device=q.device)
    args = gdr.multistep_args(q, k, v, g, beta, _abi.GATE_LOG_ALPHA, state, states, o)
    stream = torch.cuda.current_stream()
    lib, argp, sp = _abi.lib(), ctypes.byref(args), ctypes.c_void_p(stream.cuda_stream or None)

    def step():
        st = lib.rhz_gdr_multistep(argp, sp)
        if st:
            _abi.check(st)

    info = settle(torch, step, 1 / 3)
    for _ in range(warmup):
        step()
    ms = time_region(torch, stream, step, steps)
    return ms, multistep_bytes(B, H, dk, dv, n), info


def bench_aux(torch, steps, warmup):
    """The prologue / epilogue ops on config 1's 16384 tokens (H=16, d=128,
    bf16): conv1d over q, k, v's 6144 channels, prepare, per-head RMSNorm.
    Each is launched through the C ABI with a prebuilt argument struct, so
    that host overhead stays below the kernel time (RMSNorm runs ~21 us).
    GB/s counts each tensor read or written once."""
    import rhizome_amd
    from rhizome_amd import _abi

    T, H, d = PREFILL["batch"] * PREFILL["seq_len"], PREFILL["heads"], PREFILL["d_k"]
    C = 3 * H * d
    bf16, f32 = torch.bfloat16, torch.float32
    x = rhizome_amd.philox_fill("normal", 0, 11, (T, C), bf16)
    w = rhizome_amd.philox_fill("normal", 0, 12, (C, 4), f32, std=0.5)
    cb = rhizome_amd.philox_fill("normal", 0, 13, (C,), f32)
    y = torch.empty_like(x)
    q = rhizome_amd.philox_fill("normal", 0, 14, (T, H, d), bf16)
    k = rhizome_amd.philox_fill("normal", 0, 15, (T, H, d), bf16)
    lg = rhizome_amd.philox_fill("normal", 0, 16, (T, H), f32)
    a = rhizome_amd.philox_fill("normal", 0, 17, (H,), f32)
    qo, ko = torch.empty_like(q), torch.empty_like(k)
    beta, g = torch.empty_like(lg), torch.empty_like(lg)
    o = rhizome_amd.philox_fill("normal", 0, 18, (T, H, d), bf16)
    sc = rhizome_amd.philox_fill("normal", 0, 19, (d,), f32)
    on = torch.empty_like(o)
    stream = torch.cuda.current_stream()
    lib, sp = _abi.lib(), ctypes.c_void_p(stream.cuda_stream or None)

    ca = _abi.Conv1dArgs()
    ca.batch, ca.seq_len, ca.channels, ca.dtype = 1, T, C, _abi.BF16
    ca.x, ca.weight, ca.bias, ca.y = x.data_ptr(), w.data_ptr(), cb.data_ptr(), y.data_ptr()
    pa = _abi.PrepareArgs()
    pa.tokens, pa.heads, pa.d_k, pa.dtype, pa.q_scale = T, H, d, _abi.BF16, float(d) ** 0.5
    pa.q_in, pa.k_in, pa.q_out, pa.k_out = q.data_ptr(), k.data_ptr(), qo.data_ptr(), ko.data_ptr()
    pa.beta_logit, pa.alpha_logit, pa.a_log = lg.data_ptr(), lg.data_ptr(), a.data_ptr()
    pa.beta, pa.g = beta.data_ptr(), g.data_ptr()
    ra = _abi.RmsnormArgs()
    ra.rows, ra.dim, ra.dtype, ra.eps = T * H, d, _abi.BF16, 1e-6
    ra.x, ra.scale, ra.y = o.data_ptr(), sc.data_ptr(), on.data_ptr()
    cap, pap, rap = ctypes.byref(ca), ctypes.byref(pa), ctypes.byref(ra)

    def conv():
        _abi.check(lib.rhz_causal_conv1d(cap, sp))

    def prep():
        _abi.check(lib.rhz_gdr_prepare(pap, sp))

    def norm():
        _abi.check(lib.rhz_rmsnorm_heads(rap, sp))

    # conv1d and prepare in one pass over the same 6144 channels
    vq, vk, vv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(q)
    xa = _abi.ConvPrepareArgs()
    xa.batch, xa.seq_len, xa.heads, xa.d_k, xa.d_v, xa.dtype = 1, T, H, d, d, _abi.BF16
    xa.q_scale = float(d) ** 0.5
    xa.x, xa.weight, xa.bias = x.data_ptr(), w.data_ptr(), cb.data_ptr()
    xa.beta_logit, xa.alpha_logit, xa.a_log = lg.data_ptr(), lg.data_ptr(), a.data_ptr()
    xa.q, xa.k, xa.v, xa.beta, xa.g = vq.data_ptr(), vk.data_ptr(), vv.data_ptr(), beta.data_ptr(), g.data_ptr()
    xap = ctypes.byref(xa)

    def convprep():
        _abi.check(lib.rhz_gdr_conv_prepare(xap, sp))

    jobs = {
        "conv1d": (conv, 2 * T * C * 2 + C * 20, "conv1d_kernel<bf16>", "B=1 T=16384, 6144 channels"),
        "prepare": (prep, 4 * T * H * d * 2 + 4 * T * H * 4 + H * 4, "prepare_kernel<8,2,bf16,vec>",
                    "16384 tokens, H=16, d_k=128"),
        "rmsnorm": (norm, 2 * T * H * d * 2 + d * 4, "rmsnorm_kernel<16,1,bf16,vec>",
                    "16384 x 16 rows of 128"),
        # x read and q, k, v written once (bf16), two fp32 logits read and
        # beta, g written per (token, head), the conv weights and bias
        "conv_prepare": (convprep, 2 * T * C * 2 + 4 * T * H * 4 + C * 20 + H * 4,
                         "conv_prepare_kernel<bf16,16>", "B=1 T=16384, H=16, d_k=d_v=128 (6144 channels)"),
    }
    out = {}
    for name, (fn, nbytes, kernel, shape) in jobs.items():
        info = settle(torch, fn, 1 / 3)
        for _ in range(warmup):
            fn()
        ms = time_region(torch, stream, fn, steps)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"value": gbs, "unit": "GB/s", "ms_per_step": ms, "workload": shape,
                     "steps": steps, "warmup": warmup, **info,
                     "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS,
                                  "frac": gbs / PEAK_HBM_GBS, "traffic": traffic_from_profiles(name),
                                  "kernel": kernel, "bytes_per_launch": float(nbytes),
                                  "launch_us": ms * 1e3}}
    return out


def bench_local(torch, steps, warmup):
    """The Local block's mixer from its projections on config 1's shape:
    rhz_gdr_local_prefill (prepare fused into the chunked prefill) against
    rhz_gdr_prepare followed by rhz_gdr_prefill on the same inputs.  Both
    are driven through the C ABI with prebuilt argument structs."""
    import rhizome_amd
    from rhizome_amd import _abi, gdr

    c = PREFILL
    B, T, H, dk, dv = c["batch"], c["seq_len"], c["heads"], c["d_k"], c["d_v"]
    dev = torch.device("cuda:0")
    bf16, f32 = torch.bfloat16, torch.float32
    lead = (B, T)
    q = rhizome_amd.philox_fill("normal", 0, 21, lead + (H, dk), bf16)
    k = rhizome_amd.philox_fill("normal", 0, 22, lead + (H, dk), bf16)
    v = rhizome_amd.philox_fill("normal", 0, 23, lead + (H, dv), bf16)
    bl = rhizome_amd.philox_fill("normal", 0, 24, lead + (H,), f32)
    al = rhizome_amd.philox_fill("normal", 0, 25, lead + (H,), f32)
    a_log = rhizome_amd.philox_fill("normal", 0, 26, (H,), f32)
    o = torch.empty(lead + (H, dv), dtype=bf16, device=dev)
    fin = torch.empty((B, H, dv, dk), dtype=f32, device=dev)
    qp, kp = torch.empty_like(q), torch.empty_like(k)
    beta, g = torch.empty_like(bl), torch.empty_like(al)
    stream = torch.cuda.current_stream()
    lib, sp = _abi.lib(), ctypes.c_void_p(stream.cuda_stream or None)
    scale = float(dk) ** 0.5

    la = _abi.LocalArgs()
    la.prefill = gdr.prefill_args(q, k, v, None, None, _abi.GATE_LOG_ALPHA, None, None, fin, o, "chunked")
    la.q_scale = scale
    la.beta_logit, la.alpha_logit, la.a_log = bl.data_ptr(), al.data_ptr(), a_log.data_ptr()
    pa = _abi.PrepareArgs()
    pa.tokens, pa.heads, pa.d_k, pa.dtype, pa.q_scale = B * T, H, dk, _abi.BF16, scale
    pa.q_in, pa.k_in, pa.q_out, pa.k_out = q.data_ptr(), k.data_ptr(), qp.data_ptr(), kp.data_ptr()
    pa.beta_logit, pa.alpha_logit, pa.a_log = bl.data_ptr(), al.data_ptr(), a_log.data_ptr()
    pa.beta, pa.g = beta.data_ptr(), g.data_ptr()
    fa = gdr.prefill_args(qp, kp, v, g, beta, _abi.GATE_LOG_ALPHA, None, None, fin, o, "chunked")
    lap, pap, fap = ctypes.byref(la), ctypes.byref(pa), ctypes.byref(fa)

    def fused():
        _abi.check(lib.rhz_gdr_local_prefill(lap, sp))

    def separate():
        _abi.check(lib.rhz_gdr_prepare(pap, sp))
        _abi.check(lib.rhz_gdr_prefill(fap, sp))

    out = {}
    for name, fn in (("fused", fused), ("separate", separate)):
        info = settle(torch, fn, 1 / 2)
        for _ in range(warmup):
            fn()
        out[name] = {"ms_per_step": time_region(torch, stream, fn, steps), **info}
    if rhizome_amd.sync_timeouts() != 0 or rhizome_amd.fp16_range_errors() != 0 or rhizome_amd.exact_reruns() != 0:
        raise RuntimeError("a chunked-kernel diagnostic counter is nonzero after the Local-block leg")
    tokens = B * T
    # raw q, k, v read and o written once (bf16), two fp32 logits per
    # (token, head), fp32 final states, a_log
    nbytes = float(tokens * H * (3 * dk * 2 + dv * 2 + 2 * 4) + B * H * dv * dk * 4 + H * 4)
    gbs = nbytes / (out["fused"]["ms_per_step"] * 1e-3) / 1e9
    return {"metric": "Local-block mixer tokens/s (prepare + chunked prefill)",
            "value": tokens / (out["fused"]["ms_per_step"] * 1e-3), "unit": "tokens/s",
            "ms_per_step": out["fused"]["ms_per_step"],
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": gbs / PEAK_HBM_GBS, "traffic": traffic_from_profiles("local"),
                         "kernel": "gdr_chunk_kernel<128, true>", "bytes_per_launch": nbytes,
                         "launch_us": out["fused"]["ms_per_step"] * 1e3},
            "separate_ms_per_step": out["separate"]["ms_per_step"],
            "separate_tokens_per_s": tokens / (out["separate"]["ms_per_step"] * 1e-3),
            "config": {"workload": "rhz_gdr_local_prefill vs rhz_gdr_prepare + rhz_gdr_prefill",
                       "batch": B, "heads": H, "seq_len": T, "d_k": dk, "d_v": dv,
                       "inputs": "bf16 raw q/k projections and v, fp32 logits"},
            "steps": steps, "warmup": warmup, "settle": out}


def bench_local_chain(torch, steps, warmup):
    """The whole Local-block mixer on config 1's shape (B=4, T=4096, H=16,
    d=128, bf16), from the q, k, v projections and logits to the normed
    output, in three arrangements of the library's calls:
      separate:        conv1d (q, k, v) -> prepare -> prefill -> RMSNorm
      fused_prologue:  conv1d (q, k, v) -> local_prefill -> RMSNorm
      conv_prepare:    conv_prepare -> prefill -> RMSNorm
    Each arrangement is one timed step of all its launches."""
    import rhizome_amd
    from rhizome_amd import _abi, gdr

    c = PREFILL
    B, T, H, d = c["batch"], c["seq_len"], c["heads"], c["d_k"]
    N = B * T
    C = 3 * H * d
    dev = torch.device("cuda:0")
    bf16, f32 = torch.bfloat16, torch.float32
    x = rhizome_amd.philox_fill("normal", 0, 31, (N, C), bf16)
    xq, xk, xv = (x[:, i * H * d:(i + 1) * H * d].contiguous() for i in range(3))
    w = rhizome_amd.philox_fill("normal", 0, 32, (C, 4), f32, std=0.5)
    wq, wk, wv = (w[i * H * d:(i + 1) * H * d].contiguous() for i in range(3))
    bl = rhizome_amd.philox_fill("normal", 0, 33, (N, H), f32)
    al = rhizome_amd.philox_fill("normal", 0, 34, (N, H), f32)
    a_log = rhizome_amd.philox_fill("normal", 0, 35, (H,), f32)
    sc = rhizome_amd.philox_fill("normal", 0, 36, (d,), f32)
    yq, yk, yv = (torch.empty((N, H, d), dtype=bf16, device=dev) for _ in range(3))
    q, k = torch.empty_like(yq), torch.empty_like(yk)
    beta, g = torch.empty_like(bl), torch.empty_like(al)
    o = torch.empty((N, H, d), dtype=bf16, device=dev)
    y = torch.empty_like(o)
    fin = torch.empty((B, H, d, d), dtype=f32, device=dev)
    stream = torch.cuda.current_stream()
    lib, sp = _abi.lib(), ctypes.c_void_p(stream.cuda_stream or None)
    scale = float(d) ** 0.5

    convs = []
    for xi, wi, yi in ((xq, wq, yq), (xk, wk, yk), (xv, wv, yv)):
        ca = _abi.Conv1dArgs()
        ca.batch, ca.seq_len, ca.channels, ca.dtype = B, T, H * d, _abi.BF16
        ca.x, ca.weight, ca.y = xi.data_ptr(), wi.data_ptr(), yi.data_ptr()
        convs.append(ca)
    pa = _abi.PrepareArgs()
    pa.tokens, pa.heads, pa.d_k, pa.dtype, pa.q_scale = N, H, d, _abi.BF16, scale
    pa.q_in, pa.k_in, pa.q_out, pa.k_out = yq.data_ptr(), yk.data_ptr(), q.data_ptr(), k.data_ptr()
    pa.beta_logit, pa.alpha_logit, pa.a_log = bl.data_ptr(), al.data_ptr(), a_log.data_ptr()
    pa.beta, pa.g = beta.data_ptr(), g.data_ptr()
    sh = lambda t: t.view(B, T, *t.shape[1:])  # noqa: E731
    fa = gdr.prefill_args(sh(q), sh(k), sh(yv), sh(g), sh(beta), _abi.GATE_LOG_ALPHA, None, None, fin, sh(o),
                          "chunked")
    la = _abi.LocalArgs()
    la.prefill = gdr.prefill_args(sh(yq), sh(yk), sh(yv), None, None, _abi.GATE_LOG_ALPHA, None, None, fin,
                                  sh(o), "chunked")
    la.q_scale = scale
    la.beta_logit, la.alpha_logit, la.a_log = bl.data_ptr(), al.data_ptr(), a_log.data_ptr()
    xa = _abi.ConvPrepareArgs()
    xa.batch, xa.seq_len, xa.heads, xa.d_k, xa.d_v, xa.dtype, xa.q_scale = B, T, H, d, d, _abi.BF16, scale
    xa.x, xa.weight = x.data_ptr(), w.data_ptr()
    xa.beta_logit, xa.alpha_logit, xa.a_log = bl.data_ptr(), al.data_ptr(), a_log.data_ptr()
    xa.q, xa.k, xa.v, xa.beta, xa.g = q.data_ptr(), k.data_ptr(), yv.data_ptr(), beta.data_ptr(), g.data_ptr()
    ra = _abi.RmsnormArgs()
    ra.rows, ra.dim, ra.dtype, ra.eps = N * H, d, _abi.BF16, 1e-6
    ra.x, ra.scale, ra.y = o.data_ptr(), sc.data_ptr(), y.data_ptr()
    cps = [ctypes.byref(ca) for ca in convs]
    pap, fap, lap, xap, rap = (ctypes.byref(t) for t in (pa, fa, la, xa, ra))

    def conv3():
        for cp in cps:
            _abi.check(lib.rhz_causal_conv1d(cp, sp))

    def separate():
        conv3()
        _abi.check(lib.rhz_gdr_prepare(pap, sp))
        _abi.check(lib.rhz_gdr_prefill(fap, sp))
        _abi.check(lib.rhz_rmsnorm_heads(rap, sp))

    def fused_prologue():
        conv3()
        _abi.check(lib.rhz_gdr_local_prefill(lap, sp))
        _abi.check(lib.rhz_rmsnorm_heads(rap, sp))

    def conv_prepare():
        _abi.check(lib.rhz_gdr_conv_prepare(xap, sp))
        _abi.check(lib.rhz_gdr_prefill(fap, sp))
        _abi.check(lib.rhz_rmsnorm_heads(rap, sp))

    out = {}
    for name, fn in (("separate", separate), ("fused_prologue", fused_prologue), ("conv_prepare", conv_prepare)):
        info = settle(torch, fn, 1 / 3)
        for _ in range(warmup):
            fn()
        ms = time_region(torch, stream, fn, steps)
        out[name] = {"ms_per_step": ms, "tokens_per_s": N / (ms * 1e-3), **info}
    if rhizome_amd.sync_timeouts() != 0 or rhizome_amd.fp16_range_errors() != 0 or rhizome_amd.exact_reruns() != 0:
        raise RuntimeError("a chunked-kernel diagnostic counter is nonzero after the Local-block chain leg")
    best = min(out, key=lambda n: out[n]["ms_per_step"])
    return {"metric": "Local-block mixer tokens/s (conv1d + prepare + GDR prefill + per-head RMSNorm)",
            "value": out[best]["tokens_per_s"], "unit": "tokens/s", "ms_per_step": out[best]["ms_per_step"],
            "fastest": best, "arrangements": out,
            "config": {"workload": "Local block from the q, k, v projections and logits to the normed output",
                       "batch": B, "heads": H, "seq_len": T, "d_k": d, "d_v": d,
                       "inputs": "bf16 projections, fp32 logits, fp32 conv weights"},
            "steps": steps, "warmup": warmup}


def cpu_baseline(pre_host, dec_host):
    """f64 oracle on this host: reference three-pass step with per-call allocations."""
    import numpy as np
    from oracle import oracle as O

    cores = O.default_threads()
    c = PREFILL
    B, T, H, dk = c["batch"], c["seq_len"], c["heads"], c["d_k"]
    # prefill: every (b, h) head of the workload, unit-major f64
    q = pre_host["q"].double().cpu().numpy().transpose(0, 2, 1, 3).reshape(B * H, T, dk)
    k = pre_host["k"].double().cpu().numpy().transpose(0, 2, 1, 3).reshape(B * H, T, dk)
    v = pre_host["v"].double().cpu().numpy().transpose(0, 2, 1, 3).reshape(B * H, T, c["d_v"])
    a = np.exp(pre_host["g"].double().cpu().numpy()).transpose(0, 2, 1).reshape(B * H, T)
    b = pre_host["beta"].double().cpu().numpy().transpose(0, 2, 1).reshape(B * H, T)
    t0 = time.perf_counter()
    O.bench_sequential(q, k, v, a, b, threads=cores)
    t_all = time.perf_counter() - t0
    # single thread: two heads, scaled to the workload
    t0 = time.perf_counter()
    O.bench_sequential(q[:2], k[:2], v[:2], a[:2], b[:2], threads=1)
    t_one = (time.perf_counter() - t0) / 2 * (B * H)
    # decode: 8 steps of every (b, h) of the decode workload
    d = DECODE
    U = d["batch"] * d["heads"]
    nst = 8
    qd = dec_host["q"][:nst].double().cpu().numpy().reshape(nst, U, d["d_k"])
    kd = dec_host["k"][:nst].double().cpu().numpy().reshape(nst, U, d["d_k"])
    vd = dec_host["v"][:nst].double().cpu().numpy().reshape(nst, U, d["d_v"])
    ad = np.exp(dec_host["g"][:nst].double().cpu().numpy()).reshape(nst, U)
    bd = dec_host["beta"][:nst].double().cpu().numpy().reshape(nst, U)
    S = np.zeros((U, d["d_v"], d["d_k"]))
    t0 = time.perf_counter()
    for s in range(nst):
        O.bench_step(qd[s], kd[s], vd[s], ad[s], bd[s], S, threads=cores)
    t_dec = (time.perf_counter() - t0) / nst
    return {
        "value": B * T / t_all,
        "unit": "tokens/s",
        "cores": cores,
        # the thread count is capped at 16, the host CPU share that one GPU
        # of the box is given, whatever the affinity mask shows
        "cores_available": len(os.sched_getaffinity(0)),
        "cores_cap": O.MAX_THREADS,
        "kind": "port",
        "sample": (f"full prefill workload (B={B} H={H} T={T} d={dk}, {B * H} heads) through "
                   "the f64 oracle's gated_delta_sequential, heads spread over all cores"),
        "single_thread_value": B * T / t_one,
        "cpu": _cpu_model(),
        "decode": {"value": decode_bytes(d["batch"], d["heads"], d["d_k"], d["d_v"]) / t_dec / 1e9,
                   "unit": "GB/s", "cores": cores,
                   "sample": f"{nst} steps of gated_delta_step on all {U} (b,h) heads"},
    }


COPY_BYTES = 256 << 20


def calibration_copy(torch):
    """One elementwise kernel that reads COPY_BYTES and writes COPY_BYTES
    (dst = 2 src in fp32; a kernel, where a plain copy_ would be a DMA)."""
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    torch.mul(src, 2.0, out=dst)
    torch.cuda.synchronize()


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    # each leg first runs SETTLE_MS of untimed launches (the GPU clock ramps
    # up over the first tens of ms of back-to-back launches), then the
    # counted warmup, then the timed steps
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--settle-ms", type=float, default=SETTLE_MS,
                    help="untimed launches before each leg's warmup, in ms of wall time")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibration-copy", action="store_true")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: the gated delta-rule needs no collective and this "
              "build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    set_settle_ms(args.settle_ms)
    ms, flops, algo_bytes, pre_host = bench_prefill(torch, args.steps, args.warmup)
    dms, dbytes, dec_host = bench_decode(torch, args.warmup)
    dlms, dlbytes, dl_host = bench_decode(torch, min(args.warmup, 16), DECODE_LARGE)
    mms, mbytes, ms_info = bench_multistep(torch, min(args.steps, 50), min(args.warmup, 20))
    aux = bench_aux(torch, min(args.steps, 50), min(args.warmup, 20))
    local = bench_local(torch, min(args.steps, 50), min(args.warmup, 10))
    fp32_leg = bench_prefill_fp32(torch, min(args.steps, 20), min(args.warmup, 5))
    chain = bench_local_chain(torch, min(args.steps, 30), min(args.warmup, 5))
    long_leg = prefill_leg(torch, min(args.steps, 50), min(args.warmup, 10), PREFILL_LONG,
                           "chunked GDR prefill, long context, slow decay", "prefill_long")
    vc = dict(PREFILL_VARLEN)
    vc["lengths"] = varlen_lengths_dev(torch, vc["n_seqs"], vc["len_lo"], vc["len_hi"])
    varlen_leg = prefill_leg(torch, min(args.steps, 50), min(args.warmup, 10), vc,
                             "chunked GDR prefill, packed variable-length batch with initial states",
                             "prefill_varlen")
    if args.calibration_copy:
        calibration_copy(torch)
    c = PREFILL
    tokens = c["batch"] * c["seq_len"]
    achieved = flops / (ms * 1e-3) / 1e12
    gbs = algo_bytes / (ms * 1e-3) / 1e9
    traffic = traffic_from_profiles("prefill")
    dgbs = dbytes / (dms * 1e-3) / 1e9
    out = {
        "metric": METRIC,
        "value": tokens / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_ms": pre_host["settle_ms"],
        "settle_launches": pre_host["settle_launches"],
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded Philox-4x32-10 on the device)",
        "config": {"workload": "chunked GDR prefill", "batch": c["batch"], "heads": c["heads"],
                   "seq_len": c["seq_len"], "d_k": c["d_k"], "d_v": c["d_v"], "chunk": c["chunk"],
                   "inputs": "bf16 q/k/v, fp32 log-decay and beta", "state": "fp32",
                   "parallelism": "none (1 GPU)"},
        # 47.2 GFLOP over 274.7 MB per launch is ~172 flop/B, below MI355X's
        # ridge (2500 TFLOP/s / 8 TB/s = 312 flop/B): HBM bounds the kernel
        # (34.3 us at 8 TB/s vs 18.9 us at the MFMA peak).  The MFMA figure
        # is reported beside it.
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": gbs / PEAK_HBM_GBS, "traffic": traffic,
                     "kernel": "gdr_chunk_kernel<128, false>", "algorithmic_bytes": algo_bytes,
                     "launch_us": ms * 1e3,
                     "mfma": {"achieved": achieved, "peak": PEAK_MFMA_TFLOPS, "unit": "TFLOP/s",
                              "frac": achieved / PEAK_MFMA_TFLOPS, "flops_per_launch": flops}},
        "decode": {"metric": "decode state-update HBM GB/s", "value": dgbs, "unit": "GB/s",
                   "ms_per_step": dms, "steps": DECODE["steps"],
                   "config": {"workload": "GDR decode step, state in place", **DECODE,
                              "dtype": "fp32"},
                   "roofline": {"bound": "hbm", "achieved": dgbs, "peak": PEAK_HBM_GBS,
                                "unit": "GB/s", "frac": dgbs / PEAK_HBM_GBS,
                                "traffic": traffic_from_profiles("decode"),
                                "kernel": "gdr_decode_kernel<8,4,true,float>",
                                "bytes_per_launch": dbytes, "launch_us": dms * 1e3},
                   "warmup": args.warmup, "settle_ms": dec_host["settle_ms"],
                   "settle_launches": dec_host["settle_launches"]},
        # control: the same step with the state 4x the 256 MB last-level
        # cache, so that the decode rate above is not a cache effect
        "decode_large_state": {
            "metric": "decode state-update HBM GB/s", "value": dlbytes / (dlms * 1e-3) / 1e9,
            "unit": "GB/s", "ms_per_step": dlms, "steps": DECODE_LARGE["steps"],
            "config": {"workload": "GDR decode step, state in place, 1.07 GB state", **DECODE_LARGE,
                       "dtype": "fp32"},
            "roofline": {"bound": "hbm", "achieved": dlbytes / (dlms * 1e-3) / 1e9, "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": dlbytes / (dlms * 1e-3) / 1e9 / PEAK_HBM_GBS,
                         "traffic": traffic_from_profiles("decode_large"),
                         "kernel": "gdr_decode_kernel<8,1,true,float,true>", "bytes_per_launch": dlbytes,
                         "launch_us": dlms * 1e3},
            "warmup": min(args.warmup, 16), "settle_launches": dl_host["settle_launches"]},
        "prefill_long_context": long_leg,
        "prefill_varlen": varlen_leg,
        "multistep": {"metric": "multistep HBM GB/s (state read, per-position snapshots written)",
                      "value": mbytes / (mms * 1e-3) / 1e9, "unit": "GB/s", "ms_per_step": mms,
                      "config": {"workload": "GDR multistep, 8 positions from a given state",
                                 **MULTISTEP, "dtype": "fp32"},
                      "roofline": {"bound": "hbm", "achieved": mbytes / (mms * 1e-3) / 1e9,
                                   "peak": PEAK_HBM_GBS,
                                   "frac": mbytes / (mms * 1e-3) / 1e9 / PEAK_HBM_GBS,
                                   "traffic": traffic_from_profiles("multistep"),
                                   "kernel": "gdr_multistep_kernel<8,2,true,float>",
                                   "bytes_per_launch": mbytes, "launch_us": mms * 1e3},
                      "steps": min(args.steps, 50), "warmup": min(args.warmup, 20), **ms_info},
        "prologue_epilogue": aux,
        "local_block": local,
        "prefill_fp32": fp32_leg,
        "local_chain": chain,
        "device": device_info(torch),
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(pre_host, dec_host)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
