"""GPU parity of rhz_gdr_multistep against the f64 oracle, through the C ABI.

Reference behaviour followed: gated_delta_multistep (crates/ops/src/delta.rs:202-230),
batched over (b, h), from a given state (the reference's t = 0 reset is the
caller passing zeros), returning o and the state after every position.  A
segment change inside the window is alpha = 0 at that position, which
forgets the past exactly as the reference's reset does (delta.rs:348-358).
"""
import numpy as np
import pytest
import torch

import rhizome_amd
from gdr_cases import BF16_TOL, F32_TOL, check_close, to_device
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _inputs(B, n, H, dk, dv, dtype, device, seed=0, state_std=0.02):
    raw = O.gdr_inputs(B * n, H, dk, dv, seed=seed, n_state=B, state_std=state_std)
    q, q64 = to_device(raw["q"].reshape(B, n, H, dk), dtype, device)
    k, k64 = to_device(raw["k"].reshape(B, n, H, dk), dtype, device)
    v, v64 = to_device(raw["v"].reshape(B, n, H, dv), dtype, device)
    a, a64 = to_device(np.exp(raw["g"]).reshape(B, n, H), torch.float32, device)
    b, b64 = to_device(raw["beta"].reshape(B, n, H), torch.float32, device)
    s, s64 = to_device(raw["state"], torch.float32, device)
    return (q, k, v, a, b, s), (q64, k64, v64, a64, b64, s64)


def _oracle(host):
    """Repeated gated_delta_step (delta.rs:94-127) from the given state, with a
    snapshot after every position (delta.rs:319-331: multistep == repeated step)."""
    q64, k64, v64, a64, b64, s64 = host
    st = s64.copy()
    n = q64.shape[1]
    outs, snaps = [], []
    for t in range(n):
        outs.append(O.decode_batched(q64[:, t], k64[:, t], v64[:, t], a64[:, t], b64[:, t], st))
        snaps.append(st.copy())
    return np.stack(outs, axis=1), np.stack(snaps, axis=1)


def _check(dev, host, tol, tag):
    q, k, v, a, b, s = dev
    s_before = s.clone()
    o, states = rhizome_amd.multistep(q, k, v, None, b, alpha=a, state=s)
    torch.cuda.synchronize()
    assert torch.equal(s, s_before), "multistep modified its input state"
    ref_o, ref_s = _oracle(host)
    mo = check_close(o.float().cpu().numpy(), ref_o, tol, f"{tag} o")
    ms = check_close(states.cpu().numpy(), ref_s, tol, f"{tag} states")
    print(f"{tag}: o {mo} states {ms}", flush=True)
    return o, states


@pytest.mark.parametrize("B,n,H,dk,dv,dtype,tol", [
    (64, 8, 16, 128, 128, torch.float32, F32_TOL),    # speculative decode window
    (4, 1, 3, 64, 64, torch.float32, F32_TOL),
    (3, 5, 2, 32, 96, torch.float32, F32_TOL),
    (2, 8, 2, 256, 64, torch.float32, F32_TOL),
    (2, 3, 3, 5, 9, torch.float32, F32_TOL),
    (8, 8, 4, 128, 128, torch.bfloat16, BF16_TOL),
    (2, 4, 2, 30, 40, torch.bfloat16, BF16_TOL),
    (1, 64, 2, 128, 128, torch.float32, F32_TOL),     # the largest window
])
def test_shapes(device, B, n, H, dk, dv, dtype, tol):
    dev, host = _inputs(B, n, H, dk, dv, dtype, device, seed=5)
    _check(dev, host, tol, f"multistep B{B} n{n} H{H} {dk}x{dv} {dtype}")


def test_segment_change_is_alpha_zero(device):
    """A segment change at position 3 (alpha = 0 there): positions 3.. do not depend
    on the state or the inputs before position 3."""
    dev, host = _inputs(4, 8, 4, 64, 64, torch.float32, device, seed=7)
    q, k, v, a, b, s = dev
    a[:, 3] = 0.0
    host[3][:, 3] = 0.0
    o1, st1 = _check((q, k, v, a, b, s), host, F32_TOL, "segment change")
    # other history before position 3: a different initial state and inputs
    s2 = torch.randn_like(s)
    q2, k2, v2 = q.clone(), k.clone(), v.clone()
    q2[:, :3] = torch.flip(q[:, :3], dims=[0])
    k2[:, :3] = torch.flip(k[:, :3], dims=[0])
    v2[:, :3] = -v[:, :3]
    o2, st2 = rhizome_amd.multistep(q2, k2, v2, None, b, alpha=a, state=s2)
    torch.cuda.synchronize()
    assert torch.equal(o1[:, 3:], o2[:, 3:]) and torch.equal(st1[:, 3:], st2[:, 3:])


def test_matches_repeated_decode_steps(device):
    """The same per-position arithmetic as rhz_gdr_decode_step: n decode steps
    give the same outputs and states (up to the compiler's choice of fused
    multiply-adds, so to fp32 rounding)."""
    dev, _ = _inputs(16, 6, 4, 128, 128, torch.float32, device, seed=11)
    q, k, v, a, b, s = dev
    o, states = rhizome_amd.multistep(q, k, v, None, b, alpha=a, state=s)
    sd = s.clone()
    for t in range(q.shape[1]):
        ot = rhizome_amd.decode_step(q[:, t].contiguous(), k[:, t].contiguous(), v[:, t].contiguous(),
                                     None, b[:, t].contiguous(), alpha=a[:, t].contiguous(), state=sd)
        torch.cuda.synchronize()
        assert torch.allclose(ot, o[:, t], rtol=1e-6, atol=1e-7), f"o differs at position {t}"
        assert torch.allclose(sd, states[:, t], rtol=1e-6, atol=1e-7), f"state differs at position {t}"


def test_deterministic(device):
    dev, _ = _inputs(8, 8, 4, 128, 128, torch.bfloat16, device, seed=9)
    q, k, v, a, b, s = dev
    o1, s1 = rhizome_amd.multistep(q, k, v, None, b, alpha=a, state=s)
    o2, s2 = rhizome_amd.multistep(q, k, v, None, b, alpha=a, state=s)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
