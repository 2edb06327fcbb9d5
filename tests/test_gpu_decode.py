"""GPU parity of rhz_gdr_decode_step against the f64 oracle, through the C ABI.

Reference behaviour followed: gated_delta_step (crates/ops/src/delta.rs:94-127),
batched over (b, h) with the state updated in place.
"""
import numpy as np
import pytest
import torch

import rhizome_amd
from gdr_cases import BF16_TOL, C3, F32_TOL, check_close, to_device
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _inputs(B, H, dk, dv, steps, dtype, device, seed=0, state_std=0.02):
    raw = O.gdr_inputs(steps * B, H, dk, dv, seed=seed, n_state=B, state_std=state_std)
    q, q64 = to_device(raw["q"].reshape(steps, B, H, dk), dtype, device)
    k, k64 = to_device(raw["k"].reshape(steps, B, H, dk), dtype, device)
    v, v64 = to_device(raw["v"].reshape(steps, B, H, dv), dtype, device)
    g, g64 = to_device(raw["g"].reshape(steps, B, H), torch.float32, device)
    b, b64 = to_device(raw["beta"].reshape(steps, B, H), torch.float32, device)
    s, s64 = to_device(raw["state"], torch.float32, device)
    return (q, k, v, g, b, s), (q64, k64, v64, np.exp(g64), b64, s64)


def _run(dev, host, steps, tol, tag):
    q, k, v, g, b, s = dev
    q64, k64, v64, a64, b64, s64 = host
    s64 = s64.copy()
    outs = []
    for t in range(steps):
        outs.append(rhizome_amd.decode_step(q[t], k[t], v[t], g[t], b[t], state=s))
    torch.cuda.synchronize()
    ref = [O.decode_batched(q64[t], k64[t], v64[t], a64[t], b64[t], s64) for t in range(steps)]
    mo = check_close(torch.stack(outs).float().cpu().numpy(), np.stack(ref), tol, f"{tag} o")
    ms = check_close(s.cpu().numpy(), s64, tol, f"{tag} state")
    print(f"{tag}: o {mo} state {ms}", flush=True)


def test_config3_full(device):
    """B=256 H=16 d=128, fp32 state N(0, 0.02), 64 in-place steps, all heads checked."""
    B, H, dk, dv, steps = C3["batch"], C3["heads"], C3["d_k"], C3["d_v"], C3["steps"]
    dev, host = _inputs(B, H, dk, dv, steps, torch.float32, device)
    _run(dev, host, steps, F32_TOL, "c3")


@pytest.mark.parametrize("dk,dv,dtype,tol", [
    (32, 32, torch.float32, F32_TOL), (64, 64, torch.float32, F32_TOL),
    (128, 256, torch.float32, F32_TOL), (256, 64, torch.float32, F32_TOL),
    (6, 6, torch.float32, F32_TOL), (5, 9, torch.float32, F32_TOL),
    (128, 128, torch.bfloat16, BF16_TOL), (30, 40, torch.bfloat16, BF16_TOL),
])
def test_shapes(device, dk, dv, dtype, tol):
    dev, host = _inputs(3, 5, dk, dv, 4, dtype, device, seed=3)
    _run(dev, host, 4, tol, f"decode {dk}x{dv} {dtype}")


def test_alpha_zero_forgets_the_past(device):
    """delta.rs:348-358: S = 1, k = e0, v = 0, q = 1, alpha = 0, beta = 0.5 -> o = 0."""
    s = torch.ones((1, 1, 3, 3), dtype=torch.float32, device=device)
    k = torch.tensor([[[1.0, 0.0, 0.0]]], device=device)
    v = torch.zeros((1, 1, 3), device=device)
    q = torch.ones((1, 1, 3), device=device)
    a = torch.zeros((1, 1), device=device)
    b = torch.full((1, 1), 0.5, device=device)
    o = rhizome_amd.decode_step(q, k, v, None, b, alpha=a, state=s)
    torch.cuda.synchronize()
    assert torch.all(o.abs() < 1e-12)
    assert torch.all(s == 0)


def test_deterministic(device):
    dev, _ = _inputs(16, 4, 128, 128, 1, torch.float32, device, seed=9)
    q, k, v, g, b, s = dev
    s2 = s.clone()
    o1 = rhizome_amd.decode_step(q[0], k[0], v[0], g[0], b[0], state=s)
    o2 = rhizome_amd.decode_step(q[0], k[0], v[0], g[0], b[0], state=s2)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s, s2)


def test_streamed_state_matches_plain_path(device):
    """A state past the streaming threshold (B=1024 H=16 d=128, 1.07 GB) is
    read by non-temporal loads with one row per thread; the arithmetic per
    row is the same, so the result equals the plain path's (the same batch
    in four quarters of 268 MB each) bit for bit, and a sample of heads
    matches the oracle."""
    B, H, d = 1024, 16, 128
    f32 = torch.float32
    q = rhizome_amd.philox_fill("unit_rows", 3, 1, (B, H, d), f32)
    k = rhizome_amd.philox_fill("unit_rows", 3, 2, (B, H, d), f32)
    v = rhizome_amd.philox_fill("normal", 3, 3, (B, H, d), f32)
    b = rhizome_amd.philox_fill("sigmoid", 3, 4, (B, H), f32)
    g = rhizome_amd.philox_fill("neg_softplus", 3, 5, (B, H), f32)
    s0 = rhizome_amd.philox_fill("normal", 3, 6, (B, H, d, d), f32, std=0.02)
    s1 = s0.clone()
    o1 = rhizome_amd.decode_step(q, k, v, g, b, state=s1)
    s2 = s0.clone()
    o2 = torch.empty_like(o1)
    for i in range(4):
        sl = slice(256 * i, 256 * (i + 1))
        o2[sl] = rhizome_amd.decode_step(q[sl], k[sl], v[sl], g[sl], b[sl], state=s2[sl])
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
    sample = slice(0, B, 97)
    ref_s = s0[sample].double().cpu().numpy().copy()
    ref_o = O.decode_batched(q[sample].double().cpu().numpy(), k[sample].double().cpu().numpy(),
                             v[sample].double().cpu().numpy(), np.exp(g[sample].double().cpu().numpy()),
                             b[sample].double().cpu().numpy(), ref_s)
    check_close(o1[sample].cpu().numpy(), ref_o, F32_TOL, "streamed decode o")
    check_close(s1[sample].cpu().numpy(), ref_s, F32_TOL, "streamed decode state")
    del s0, s1, s2
