"""Seeded gated delta-rule workloads and the parity check shared by the tests.

Inputs come from the oracle's Philox builders (f64), are rounded once to
what the device receives (bf16 / fp32 q, k, v; fp32 gates, beta, states),
and the SAME rounded values, widened back to f64, feed the oracle -- so
input rounding never counts as kernel error.

Tolerance, elementwise: |out - ref| <= atol + rtol * |ref| with
atol = atol_rms * RMS(ref) (the form of docs/kernels.md:3).
  bf16 path:        rtol 2e-2, atol_rms 1e-2   (docs/kernels.md:25)
  fp32-input path:  rtol 1e-4, atol_rms 1e-4
"""
from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as O

BF16_TOL = (2e-2, 1e-2)
F32_TOL = (1e-4, 1e-4)

# The five workloads (seed 0).
C0 = dict(batch=1, heads=2, seq_len=64, d_k=32, d_v=32)
C1 = dict(batch=4, heads=16, seq_len=4096, d_k=128, d_v=128)
C2 = dict(batch=1, heads=32, seq_len=32768, d_k=128, d_v=256, g_mean=-2.0)
C3 = dict(batch=256, heads=16, d_k=128, d_v=128, steps=64, state_std=0.02)
C4 = dict(n_seqs=64, heads=16, d_k=128, d_v=128, len_lo=128, len_hi=8192, state_std=0.02)


def to_device(x: np.ndarray, dtype: torch.dtype, device) -> tuple[torch.Tensor, np.ndarray]:
    """Round f64 values to `dtype` on the way to the device (f64 -> f32 -> bf16, RNE);
    return the device tensor and the rounded values widened to f64."""
    t32 = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    t = t32.to(dtype)
    widened = t.to(torch.float64).numpy()
    return t.to(device), widened


def check_close(out, ref, tol, what: str) -> dict:
    """Assert the elementwise tolerance; return error metrics."""
    rtol, atol_rms = tol
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert out.shape == ref.shape, f"{what}: shape {out.shape} vs {ref.shape}"
    assert np.all(np.isfinite(out)), f"{what}: non-finite output"
    rms = float(np.sqrt(np.mean(ref * ref))) if ref.size else 0.0
    atol = atol_rms * rms
    err = np.abs(out - ref)
    bound = atol + rtol * np.abs(ref)
    ratio = err / np.maximum(bound, 1e-300)
    worst = int(np.argmax(ratio)) if ref.size else 0
    m = {
        "max_ratio": float(ratio.flat[worst]) if ref.size else 0.0,
        "max_rel": float(np.max(err / np.maximum(np.abs(ref), rms))) if ref.size else 0.0,
        "normwise": float(np.linalg.norm(out - ref) / max(np.linalg.norm(ref), 1e-300)),
        "rms_ref": rms,
    }
    if ref.size and m["max_ratio"] > 1.0:
        idx = np.unravel_index(worst, ref.shape)
        raise AssertionError(
            f"{what}: |out-ref| > atol + rtol|ref| at {idx}: out={out[idx]:.6g} ref={ref[idx]:.6g} "
            f"(atol={atol:.3g}, rtol={rtol}); {int(np.sum(ratio > 1))} of {ref.size} elements; {m}")
    return m


def check_close_dev(out: torch.Tensor, ref: torch.Tensor, tol, what: str, units: int = 1) -> dict:
    """check_close on device tensors (f64 arithmetic on the GPU), for outputs
    too large to copy to the host.  `units`: the leading dimension is split
    into that many equal groups (e.g. heads) whose worst ratios are reported."""
    rtol, atol_rms = tol
    out = out.to(torch.float64)
    ref = ref.to(torch.float64)
    assert out.shape == ref.shape, f"{what}: shape {tuple(out.shape)} vs {tuple(ref.shape)}"
    assert bool(torch.isfinite(out).all()), f"{what}: non-finite output"
    rms = float(torch.sqrt(torch.mean(ref * ref)))
    err = torch.abs(out - ref)
    ratio = err / torch.clamp(atol_rms * rms + rtol * torch.abs(ref), min=1e-300)
    worst = int(torch.argmax(ratio))
    m = {
        "max_ratio": float(ratio.reshape(-1)[worst]),
        "normwise": float(torch.linalg.vector_norm(out - ref) / max(float(torch.linalg.vector_norm(ref)), 1e-300)),
        "rms_ref": rms,
        "elements": ref.numel(),
    }
    if units > 1:
        m["unit_max_ratio_min"] = float(ratio.reshape(units, -1).amax(dim=1).min())
    if m["max_ratio"] > 1.0:
        idx = np.unravel_index(worst, tuple(ref.shape))
        raise AssertionError(f"{what}: |out-ref| > atol + rtol|ref| at {idx}: out={float(out[idx]):.6g} "
                             f"ref={float(ref[idx]):.6g}; {int((ratio > 1).sum())} of {ref.numel()} elements; {m}")
    return m


def nonexpansive_bound(w: "Prefill", fin: torch.Tensor) -> None:
    """Every final state within the closed-form bound of the recurrence:
    with beta in [0, 1] and alpha <= 1, ||alpha S (I - beta k k^T)||_2 <=
    ||S||_2 whenever beta ||k||^2 <= 2, and ||beta v k^T||_2 = beta ||v|| ||k||,
    so ||S_T||_2 <= ||S_0||_2 + sum_t beta_t ||v_t|| ||k_t||."""
    dev = fin.device
    k = w.k.to(torch.float64)
    v = w.v.to(torch.float64)
    beta = w.beta.to(torch.float64)
    assert bool((beta * (k * k).sum(-1) <= 2.0).all())
    step = beta * torch.linalg.vector_norm(v, dim=-1) * torch.linalg.vector_norm(k, dim=-1)  # [tok, H]
    cs = torch.cat([torch.zeros(1, w.heads, dtype=torch.float64, device=dev), torch.cumsum(step, 0)])
    cu = torch.from_numpy(w.cu).to(dev)
    growth = cs[cu[1:]] - cs[cu[:-1]]  # [N, H]
    growth = growth.cpu()
    s0 = 0.0
    if w.init is not None:  # spectral norms on the host (LAPACK)
        s0 = torch.linalg.matrix_norm(w.init.cpu().to(torch.float64), ord=2)
    bound = s0 + growth
    norm = torch.linalg.matrix_norm(fin.cpu().to(torch.float64), ord=2)
    assert bool(torch.isfinite(norm).all()), "non-finite final state"
    assert bool((norm <= bound * (1 + 1e-6) + 1e-30).all()), \
        f"final-state norm above the closed-form bound: max ratio {float((norm / bound).max()):.4g}"


class Prefill:
    """One prefill workload: host f64 inputs, their device copies, and the oracle."""

    def __init__(self, heads, d_k, d_v, *, batch=None, seq_len=None, lengths=None, seed=0,
                 g_mean=0.0, state_std=None, dtype=torch.bfloat16, device="cuda", threads=None):
        self.dense = lengths is None
        if self.dense:
            self.batch, self.seq_len = batch, seq_len
            lengths = [seq_len] * batch
        self.lengths = np.asarray(lengths, dtype=np.int64)
        self.cu = np.concatenate([[0], np.cumsum(self.lengths)]).astype(np.int64)
        self.n_seqs = len(self.lengths)
        self.n_tok = int(self.cu[-1])
        self.heads, self.d_k, self.d_v = heads, d_k, d_v
        self.dtype = dtype
        self.threads = threads
        raw = O.gdr_inputs(self.n_tok, heads, d_k, d_v, seed=seed, g_mean=g_mean,
                           n_state=self.n_seqs if state_std else 0, state_std=state_std or 0.02)
        self.q, self.q64 = to_device(raw["q"], dtype, device)
        self.k, self.k64 = to_device(raw["k"], dtype, device)
        self.v, self.v64 = to_device(raw["v"], dtype, device)
        self.g, self.g64 = to_device(raw["g"], torch.float32, device)
        self.beta, self.beta64 = to_device(raw["beta"], torch.float32, device)
        self.alpha64 = np.exp(self.g64)
        if state_std:
            self.init, self.init64 = to_device(raw["state"], torch.float32, device)
        else:
            self.init, self.init64 = None, None
        self.cu_dev = None if self.dense else torch.from_numpy(self.cu.astype(np.int32)).to(device)

    def shaped(self, t: torch.Tensor) -> torch.Tensor:
        """Packed [tokens, ...] -> dense [B, T, ...] when the workload is dense."""
        if self.dense:
            return t.reshape(self.batch, self.seq_len, *t.shape[1:])
        return t

    def run(self, reruns: int = 0, **kw):
        """Prefill through the C ABI; asserts that no LDS wait of the chunked
        kernel gave up and that exactly `reruns` of its workgroups recomputed
        their rows with the fp32 recurrence (0: every input in the fp16
        path's domain).  The counters are reset by the reads."""
        import rhizome_amd

        o, fin = rhizome_amd.prefill(self.shaped(self.q), self.shaped(self.k), self.shaped(self.v),
                                     self.shaped(self.g), self.shaped(self.beta),
                                     cu_seqlens=self.cu_dev, initial_state=self.init, **kw)
        torch.cuda.synchronize()
        assert rhizome_amd.sync_timeouts() == 0, "a chunked-kernel LDS wait gave up"
        assert rhizome_amd.fp16_range_errors() == 0, "a chunked-kernel fp16 operand out of range"
        n = rhizome_amd.exact_reruns()
        assert n == reruns, f"{n} chunked workgroups reran their rows exactly, expected {reruns}"
        return o.reshape(self.n_tok, self.heads, self.d_v), fin

    def oracle(self, seqs=None, heads=None):
        """f64 reference for all (or the given) sequences and heads:
        (o [tokens, H, d_v] with untouched entries NaN, final [N, H, d_v, d_k])."""
        seqs = range(self.n_seqs) if seqs is None else seqs
        heads = range(self.heads) if heads is None else heads
        if list(seqs) == list(range(self.n_seqs)) and list(heads) == list(range(self.heads)):
            return O.prefill_batched(self.cu, self.q64, self.k64, self.v64, self.alpha64,
                                     self.beta64, self.init64, threads=self.threads)
        o = np.full((self.n_tok, self.heads, self.d_v), np.nan)
        fin = np.full((self.n_seqs, self.heads, self.d_v, self.d_k), np.nan)
        for n in seqs:
            a, b = int(self.cu[n]), int(self.cu[n + 1])
            sl = slice(a, b)
            for h in heads:
                st = (np.zeros((self.d_v, self.d_k)) if self.init64 is None
                      else self.init64[n, h].copy())
                o[sl, h] = O.steps_rect(self.q64[sl, h], self.k64[sl, h], self.v64[sl, h],
                                        self.alpha64[sl, h], self.beta64[sl, h], st)
                fin[n, h] = st
        return o, fin


def varlen_lengths(n: int, lo: int, hi: int, seed: int = 0) -> np.ndarray:
    return O.varlen_lengths(seed, n, lo, hi)
