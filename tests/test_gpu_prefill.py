"""GPU parity of rhz_gdr_prefill (chunked bf16 MFMA path and recurrent fp32 path)
against the f64 oracle on identical seeded inputs, through the C ABI.

Reference behaviour followed: gated_delta_sequential / gated_delta_scan_chunked
(crates/ops/src/delta.rs:133-197), batched and with the initial state honoured.
"""
import os

import numpy as np
import pytest
import torch

from gdr_cases import (BF16_TOL, C0, C1, C2, C4, F32_TOL, Prefill, check_close, check_close_dev,
                        nonexpansive_bound, to_device, varlen_lengths)

pytestmark = pytest.mark.gpu

PATHS = [("chunked", torch.bfloat16, BF16_TOL), ("recurrent", torch.float32, F32_TOL),
         ("recurrent", torch.bfloat16, BF16_TOL)]


def _check(w, o, fin, tol, seqs=None, heads=None, tag=""):
    ref_o, ref_f = w.oracle(seqs, heads)
    o = o.float().cpu().numpy()
    fin = fin.cpu().numpy()
    if seqs is not None or heads is not None:
        mask = ~np.isnan(ref_o)
        mo = check_close(o[mask], ref_o[mask], tol, f"{tag} o")
        fm = ~np.isnan(ref_f)
        mf = check_close(fin[fm], ref_f[fm], tol, f"{tag} final state")
    else:
        mo = check_close(o, ref_o, tol, f"{tag} o")
        mf = check_close(fin, ref_f, tol, f"{tag} final state")
    print(f"{tag}: o {mo}  final {mf}", flush=True)
    return mo, mf


@pytest.mark.parametrize("algo,dtype,tol", PATHS)
def test_config0(device, algo, dtype, tol):
    w = Prefill(**C0, dtype=dtype, device=device)
    o, fin = w.run(algo=algo)
    _check(w, o, fin, tol, tag=f"c0 {algo} {dtype}")


@pytest.mark.parametrize("algo,dtype,tol", PATHS)
@pytest.mark.parametrize("shape", [
    dict(batch=2, heads=3, seq_len=100, d_k=64, d_v=64),
    dict(batch=1, heads=2, seq_len=1, d_k=128, d_v=128),
    dict(batch=3, heads=1, seq_len=63, d_k=32, d_v=96),
    dict(batch=1, heads=2, seq_len=200, d_k=128, d_v=256),
    dict(batch=2, heads=2, seq_len=129, d_k=16, d_v=8),
    # key widths padded inside the chunked kernel (to 64 and 128) and value
    # widths that end inside a 32-row tile
    dict(batch=2, heads=1, seq_len=70, d_k=40, d_v=24),
    dict(batch=1, heads=2, seq_len=130, d_k=96, d_v=40),
    dict(batch=1, heads=1, seq_len=300, d_k=120, d_v=136),
    # the widest value rows the ABI takes, and many heads
    dict(batch=1, heads=1, seq_len=100, d_k=128, d_v=1024),
    dict(batch=1, heads=64, seq_len=66, d_k=32, d_v=32),
])
def test_shapes(device, algo, dtype, tol, shape):
    w = Prefill(**shape, dtype=dtype, device=device, state_std=0.02)
    o, fin = w.run(algo=algo)
    _check(w, o, fin, tol, tag=f"{shape} {algo} {dtype}")


@pytest.mark.parametrize("dtype,tol", [(torch.float32, F32_TOL), (torch.bfloat16, BF16_TOL)])
@pytest.mark.parametrize("shape", [
    # the recurrent path's two kernels: positions staged through LDS (d_k <=
    # 128, d_v a multiple of 4) and loaded one position ahead (the rest)
    dict(lengths=[0, 70, 1, 33], d_k=256, d_v=64),    # d_k past 128: 16 lanes per row
    dict(lengths=[65, 0, 40], d_k=200, d_v=24),
    dict(lengths=[100, 3], d_k=64, d_v=6),            # d_v not a multiple of 4
    dict(lengths=[31, 32, 33, 97], d_k=128, d_v=36),  # blocks of 32 positions, partial last block
])
def test_recurrent_kernels(device, dtype, tol, shape):
    w = Prefill(heads=2, d_k=shape["d_k"], d_v=shape["d_v"], lengths=shape["lengths"], dtype=dtype,
                device=device, state_std=0.02)
    o, fin = w.run(algo="recurrent")
    _check(w, o, fin, tol, tag=f"recurrent {shape} {dtype}")


@pytest.mark.parametrize("algo,dtype,tol", PATHS)
def test_varlen_with_edges(device, algo, dtype, tol):
    # empty, single-token, chunk-boundary and ragged sequences in one pack
    lengths = [0, 1, 63, 64, 65, 200, 0, 130]
    w = Prefill(heads=4, d_k=128, d_v=128, lengths=lengths, dtype=dtype, device=device,
                state_std=0.02)
    o, fin = w.run(algo=algo)
    _check(w, o, fin, tol, tag=f"varlen edges {algo} {dtype}")


@pytest.mark.parametrize("algo,dtype,tol", PATHS)
def test_alpha_gate_with_resets(device, algo, dtype, tol):
    """gate given as alpha, with alpha = 0 at some positions (a reset, delta.rs:348-358)."""
    w = Prefill(batch=2, heads=2, seq_len=150, d_k=64, d_v=64, dtype=dtype, device=device,
                state_std=0.02)
    alpha64 = np.exp(w.g64)
    alpha64[0, :] = 0.0     # sequence start
    alpha64[70, 1] = 0.0    # mid-chunk reset
    alpha64[128, 0] = 0.0   # chunk-start reset
    alpha64[155, :] = 0.0   # inside the second sequence
    alpha_dev = torch.from_numpy(alpha64.astype(np.float32)).to(device)
    w.alpha64 = alpha_dev.double().cpu().numpy()
    import rhizome_amd
    o, fin = rhizome_amd.prefill(w.shaped(w.q), w.shaped(w.k), w.shaped(w.v), None,
                                 w.shaped(w.beta), alpha=w.shaped(alpha_dev),
                                 initial_state=w.init, algo=algo)
    torch.cuda.synchronize()
    _check(w, o.reshape(w.n_tok, w.heads, w.d_v), fin, tol, tag=f"alpha gate {algo}")


@pytest.mark.parametrize("algo,dtype,tol", PATHS)
def test_many_resets_per_chunk(device, algo, dtype, tol):
    """alpha = 0 at random positions (about one token in twelve, so most
    chunks hold several resets, some adjacent), at a chunk's first and last
    token and on two consecutive tokens: every segment boundary inside a
    chunk, in the diagonal and the off-diagonal 16-token blocks."""
    w = Prefill(heads=3, d_k=64, d_v=96, lengths=[300, 64, 129, 1], dtype=dtype, device=device,
                state_std=0.05, seed=4)
    rng = np.random.default_rng(12)
    alpha64 = np.exp(w.g64)
    alpha64[rng.random(alpha64.shape) < 1 / 12] = 0.0
    alpha64[[63, 64, 100, 101, 300 + 63], :] = 0.0
    alpha = torch.from_numpy(alpha64.astype(np.float32)).to(device)
    w.alpha64 = alpha.double().cpu().numpy()
    import rhizome_amd
    o, fin = rhizome_amd.prefill(w.q, w.k, w.v, None, w.beta, alpha=alpha, cu_seqlens=w.cu_dev,
                                 initial_state=w.init, algo=algo)
    torch.cuda.synchronize()
    assert rhizome_amd.sync_timeouts() == 0 and rhizome_amd.fp16_range_errors() == 0
    _check(w, o, fin, tol, tag=f"many resets {algo} {dtype}")


def _random_workload(rng, dtype, device):
    """One seeded draw: shape, packed lengths (empty, 1-token and chunk-edge
    sequences included), decay regime, resets and initial state."""
    d_k = int(rng.choice([8, 16, 24, 32, 40, 48, 64, 72, 96, 112, 120, 128]))
    d_v = int(rng.choice([8, 16, 24, 32, 40, 64, 96, 128, 136, 192, 256]))
    heads = int(rng.integers(1, 6))
    n = int(rng.integers(1, 8))
    if rng.random() < 0.3:
        lengths = [int(rng.choice([0, 1, 2, 63, 64, 65, 127, 128, 129, 191, 192, 193])) for _ in range(n)]
    else:
        lengths = [int(x) for x in rng.integers(0, 260, size=n)]
    if sum(lengths) == 0:
        lengths[0] = 5
    w = Prefill(heads=heads, d_k=d_k, d_v=d_v, lengths=lengths, dtype=dtype, device=device,
                seed=int(rng.integers(0, 1 << 30)), g_mean=float(rng.choice([-6.0, -2.0, 0.0, 2.0, 6.0])),
                state_std=float(rng.choice([0.0, 0.02, 0.5])) or None)
    alpha64 = np.exp(w.g64)
    alpha64[rng.random(alpha64.shape) < float(rng.choice([0.0, 0.0, 0.01, 0.1, 0.5]))] = 0.0
    return w, alpha64


@pytest.mark.parametrize("algo,dtype,tol", PATHS)
def test_random_workloads(device, algo, dtype, tol):
    """Forty seeded random workloads per path against the f64 oracle: d_k
    8..128 (padded widths included), d_v 8..256, 1-5 heads, 1-7 packed
    sequences of 0..259 tokens or of chunk-edge lengths, strong to weak
    decay (g = -softplus(N(mean, 1)), mean -6..6), no, rare, frequent or
    every-other-token resets (alpha = 0), initial states of scale 0, 0.02
    or 0.5.  Each draw runs twice and must give the same bits.
    RHZ_RANDOM_DRAWS and RHZ_RANDOM_SEED widen the sweep (defaults 40 and
    2026)."""
    import rhizome_amd

    draws = int(os.environ.get("RHZ_RANDOM_DRAWS", "40"))
    rng = np.random.default_rng(int(os.environ.get("RHZ_RANDOM_SEED", "2026")))
    worst = 0.0
    for i in range(draws):
        w, alpha64 = _random_workload(rng, dtype, device)
        tag = (f"random {i} {algo} {dtype}: H={w.heads} d_k={w.d_k} d_v={w.d_v} "
               f"lengths={[int(x) for x in w.lengths]} state={w.init is not None}")
        alpha = torch.from_numpy(alpha64.astype(np.float32)).to(device)
        w.alpha64 = alpha.double().cpu().numpy()
        o, fin = rhizome_amd.prefill(w.q, w.k, w.v, None, w.beta, alpha=alpha, cu_seqlens=w.cu_dev,
                                     initial_state=w.init, algo=algo)
        o2, fin2 = rhizome_amd.prefill(w.q, w.k, w.v, None, w.beta, alpha=alpha, cu_seqlens=w.cu_dev,
                                       initial_state=w.init, algo=algo)
        torch.cuda.synchronize()
        assert torch.equal(o, o2) and torch.equal(fin, fin2), f"{tag}: two runs differ"
        assert rhizome_amd.sync_timeouts() == 0 and rhizome_amd.fp16_range_errors() == 0, tag
        ro, rf = w.oracle()
        mo = check_close(o.reshape(w.n_tok, w.heads, w.d_v).float().cpu().numpy(), ro, tol, f"{tag} o")
        mf = check_close(fin.cpu().numpy(), rf, tol, f"{tag} final state")
        worst = max(worst, mo["max_ratio"], mf["max_ratio"])
    print(f"random workloads {algo} {dtype}: {draws} cases, worst ratio {worst:.3f}", flush=True)


@pytest.mark.parametrize("algo,dtype,tol", PATHS)
@pytest.mark.parametrize("m", [37, 64, 70, 128])
def test_reset_forgets_history(device, algo, dtype, tol, m):
    """alpha = 0 at position m of every packed sequence (mid-chunk, at a chunk
    start): the outputs from m on and the final states do not depend on the
    initial state or on any input before m, bit for bit (a reset forgets S,
    delta.rs:137-142).  Both histories keep the chunked path's power-of-two
    state scale at 1, so its fp16 operands after the reset are the same
    numbers."""
    import rhizome_amd

    lengths = [150, 200, 131]
    w = Prefill(heads=2, d_k=64, d_v=64, lengths=lengths, dtype=dtype, device=device, state_std=0.02)
    h = Prefill(heads=2, d_k=64, d_v=64, lengths=lengths, seed=1, dtype=dtype, device=device,
                state_std=0.5)
    starts = w.cu[:-1]
    alpha64 = np.exp(w.g64)
    alpha64[starts + m, :] = 0.0
    alpha = torch.from_numpy(alpha64.astype(np.float32)).to(device)
    w.alpha64 = alpha.double().cpu().numpy()
    before = np.concatenate([np.arange(a, a + m) for a in starts])
    after = np.setdiff1d(np.arange(w.n_tok), before)
    bi = torch.from_numpy(before).to(device)
    ai = torch.from_numpy(after).to(device)

    def run(q, k, v, beta, a, init):
        o, fin = rhizome_amd.prefill(q, k, v, None, beta, alpha=a, cu_seqlens=w.cu_dev,
                                     initial_state=init, algo=algo)
        torch.cuda.synchronize()
        assert rhizome_amd.sync_timeouts() == 0 and rhizome_amd.fp16_range_errors() == 0
        return o, fin

    o1, f1 = run(w.q, w.k, w.v, w.beta, alpha, w.init)
    _check(w, o1, f1, tol, tag=f"reset at {m} {algo} {dtype}")
    other = []
    for x, y in ((w.q, h.q), (w.k, h.k), (w.v, h.v), (w.beta, h.beta), (alpha, torch.exp(h.g))):
        z = x.clone()
        z[bi] = y[bi]
        other.append(z)
    o2, f2 = run(*other, h.init)
    assert not torch.equal(o1[bi], o2[bi])
    assert torch.equal(o1[ai], o2[ai]), "outputs after the reset depend on the history"
    assert torch.equal(f1, f2), "final states depend on the history before the reset"


@pytest.mark.parametrize("algo,dtype,tol", PATHS)
@pytest.mark.parametrize("scale", [1e-4, 1e4])
def test_value_magnitudes(device, algo, dtype, tol, scale):
    """v and S0 scaled by 1e-4 / 1e4: the op is linear in (v, S0) jointly; the
    chunked path's fp16 operands are rescaled by powers of two per chunk."""
    w = Prefill(batch=2, heads=2, seq_len=200, d_k=128, d_v=64, dtype=dtype, device=device,
                state_std=0.02)
    w.v = (w.v.double() * scale).to(dtype)
    w.v64 = w.v.double().cpu().numpy()
    w.init = w.init * scale
    w.init64 = w.init.double().cpu().numpy()
    o, fin = w.run(algo=algo)
    _check(w, o, fin, tol, tag=f"scale {scale} {algo} {dtype}")


@pytest.mark.parametrize("algo,dtype,tol", PATHS)
def test_query_scaled_by_sqrt_dk(device, algo, dtype, tol):
    """q as the prologue hands it over, l2norm(q) * sqrt(d_k) (rhz_gdr_prepare,
    SPEC.md:53): rows of norm 11.3 at d_k = 128."""
    w = Prefill(batch=2, heads=2, seq_len=200, d_k=128, d_v=64, dtype=dtype, device=device,
                state_std=0.02)
    w.q = (w.q.double() * np.sqrt(128.0)).to(dtype)
    w.q64 = w.q.double().cpu().numpy()
    o, fin = w.run(algo=algo)
    _check(w, o, fin, tol, tag=f"q * sqrt(d_k) {algo} {dtype}")


def test_tiny_qk_entries(device):
    """q and k entries below fp16's normal range (|x| < 2^-14): the chunked
    path's bf16 -> fp16 conversion keeps them as fp16 subnormals, exact to
    2^-25 absolute (a bf16 value there can carry more significant bits than
    the subnormal keeps), so a dot product of unit rows moves by less than
    d_k 2^-25.  Half of every row's entries drawn at 1e-7..1e-5, the rest
    rescaled so that each row keeps unit norm; the chunked path stays within
    its tolerance of the oracle on the same bf16 values."""
    w = Prefill(batch=1, heads=2, seq_len=200, d_k=64, d_v=64, dtype=torch.bfloat16, device=device,
                state_std=0.02, seed=9)
    rng = np.random.default_rng(3)
    for name in ("q", "k"):
        x = getattr(w, name + "64").copy()
        tiny = rng.random(x.shape) < 0.5
        x[tiny] = np.sign(x[tiny]) * 10.0 ** rng.uniform(-7, -5, size=int(tiny.sum()))
        x /= np.linalg.norm(x, axis=-1, keepdims=True)
        t, x64 = to_device(x, torch.bfloat16, device)
        assert float(np.mean(np.abs(x64) < 2.0 ** -14)) > 0.4
        setattr(w, name, t)
        setattr(w, name + "64", x64)
    o, fin = w.run(algo="chunked")
    _check(w, o, fin, BF16_TOL, tag="tiny q, k entries, chunked")


def test_q_rows_near_fp16_range(device):
    """q rows of norm 6e4 keep every fp16 operand of the chunked path in range
    (|q_r . k_s| <= 6e4 < 65520): parity with the oracle, and no workgroup
    reruns."""
    w = Prefill(batch=1, heads=2, seq_len=130, d_k=64, d_v=64, dtype=torch.bfloat16, device=device,
                state_std=0.02)
    w.q = (w.q.double() * 6e4).to(torch.bfloat16)
    w.q64 = w.q.double().cpu().numpy()
    assert float(np.abs(w.q64).max()) < 65520.0
    o, fin = w.run(algo="chunked")  # asserts no rerun and no range error
    _check(w, o, fin, BF16_TOL, tag="q rows of norm 6e4, chunked")


def _leave_domain(w, case, seq, head):
    """Edits workload w (device tensors and their f64 copies) so that
    sequence `seq`, head `head` leaves the chunked path's fp16 domain."""
    t0, t1 = int(w.cu[seq]), int(w.cu[seq + 1])
    n = t1 - t0
    if case == "q element 7e4":  # beyond fp16's range on chip
        w.q[t0 + n // 2, head, 5] = 7e4
    elif case == "k element 1e5, its beta 1e-12":  # beyond fp16's range; beta keeps the recurrence tame
        w.k[t0 + 3, head, 0] = 1e5
        w.beta[t0 + 3, head] = 1e-12
    elif case == "k rows of norm^2 1.2":
        w.k[t0:t1, head] = (w.k[t0:t1, head].double() * 1.2 ** 0.5).to(w.k.dtype)
    elif case == "beta 1.2":
        w.beta[t0 + n // 3:t0 + n // 3 + 10, head] = 1.2
    elif case == "beta -0.1":
        w.beta[t0 + 5, head] = -0.1
    elif case == "alpha 1.05":
        w.g[t1 - 30:t1 - 26, head] = float(np.log(1.05))
    else:
        raise ValueError(case)
    w.q64, w.k64 = w.q.double().cpu().numpy(), w.k.double().cpu().numpy()
    w.beta64, w.g64 = w.beta.double().cpu().numpy(), w.g.double().cpu().numpy()
    w.alpha64 = np.exp(w.g64)


OUT_OF_DOMAIN = ["q element 7e4", "k element 1e5, its beta 1e-12", "k rows of norm^2 1.2", "beta 1.2",
                 "beta -0.1", "alpha 1.05"]


@pytest.mark.parametrize("case", OUT_OF_DOMAIN)
def test_out_of_domain_inputs_rerun_exactly(device, case):
    """Inputs outside the domain in which the chunked path's fp16 operands
    are accurate -- a q or k element beyond fp16's range, key rows of norm
    above 1, a beta or alpha outside [0, 1] -- in one (sequence, head) of a
    packed batch with initial states: exactly that unit's workgroups (3 row
    tiles of d_v = 96) recompute their rows with the fp32 recurrence inside
    the same launch, and every unit matches the oracle."""
    w = Prefill(heads=2, d_k=128, d_v=96, lengths=[70, 0, 130, 1, 33], dtype=torch.bfloat16, device=device,
                state_std=0.02)
    _leave_domain(w, case, seq=2, head=1)
    o, fin = w.run(algo="chunked", reruns=3)
    _check(w, o, fin, BF16_TOL, tag=f"{case}, chunked with exact rerun")


def test_out_of_domain_dense_every_unit(device):
    """A dense batch in which every unit leaves the domain (q element 7e4 in
    every (batch, head)): every workgroup reruns, and all match the oracle;
    the same inputs in the domain rerun nothing."""
    w = Prefill(batch=2, heads=3, seq_len=100, d_k=64, d_v=64, dtype=torch.bfloat16, device=device)
    o, fin = w.run(algo="chunked")
    _check(w, o, fin, BF16_TOL, tag="in domain")
    for b in range(2):
        for h in range(3):
            w.q[b * 100 + 7 * h + 10, h, 3] = -7e4
    w.q64 = w.q.double().cpu().numpy()
    o, fin = w.run(algo="chunked", reruns=2 * 3 * 2)
    _check(w, o, fin, BF16_TOL, tag="q elements -7e4 everywhere, chunked with exact rerun")


def test_out_of_domain_alpha_given(device):
    """Gates given as alpha (RHZ_GATE_ALPHA): a negative alpha and one above 1
    take the exact rerun (their logarithm is NaN or positive) and match the
    oracle."""
    import rhizome_amd

    w = Prefill(batch=1, heads=2, seq_len=150, d_k=64, d_v=32, dtype=torch.bfloat16, device=device,
                state_std=0.02)
    alpha = torch.exp(w.g)
    alpha[20, 0] = -0.5
    alpha[90, 1] = 1.02
    w.alpha64 = alpha.double().cpu().numpy()
    o, fin = rhizome_amd.prefill(w.shaped(w.q), w.shaped(w.k), w.shaped(w.v), alpha=w.shaped(alpha),
                                 beta=w.shaped(w.beta), initial_state=w.init, algo="chunked")
    torch.cuda.synchronize()
    assert rhizome_amd.sync_timeouts() == 0 and rhizome_amd.fp16_range_errors() == 0
    assert rhizome_amd.exact_reruns() == 2  # one row tile (d_v = 32) per head
    _check(w, o.reshape(w.n_tok, w.heads, w.d_v), fin, BF16_TOL, tag="alpha -0.5 and 1.02, chunked")


@pytest.mark.parametrize("algo,dtype,tol", PATHS)
@pytest.mark.parametrize("z_mean", [6.0, -6.0])
def test_gate_extremes(device, algo, dtype, tol, z_mean):
    """g = -softplus(z), z ~ N(z_mean, 1): z_mean 6 gives alpha ~ 0.003 (the
    state is forgotten within a few tokens), z_mean -6 gives alpha ~ 0.998
    (the state builds up over the whole sequence).  The chunk decays then
    span many orders of magnitude, and the chunked path's fp16 operands are
    rescaled as the state shrinks or grows."""
    w = Prefill(batch=1, heads=2, seq_len=520, d_k=128, d_v=64, dtype=dtype, device=device,
                state_std=0.02, g_mean=z_mean)
    o, fin = w.run(algo=algo)
    _check(w, o, fin, tol, tag=f"z_mean {z_mean} {algo} {dtype}")


@pytest.mark.parametrize("algo,dtype", [("chunked", torch.bfloat16), ("recurrent", torch.float32)])
def test_deterministic_and_batch_invariant(device, algo, dtype):
    lengths = [300, 77, 640, 1, 129]
    w = Prefill(heads=3, d_k=128, d_v=128, lengths=lengths, dtype=dtype, device=device,
                state_std=0.02)
    o1, f1 = w.run(algo=algo)
    o2, f2 = w.run(algo=algo)
    assert torch.equal(o1, o2) and torch.equal(f1, f2), "run-to-run results differ"
    # sequence 2 alone must give bit-identical results to its slot in the pack
    import rhizome_amd
    a, b = int(w.cu[2]), int(w.cu[3])
    cu = torch.tensor([0, b - a], dtype=torch.int32, device=device)
    o3, f3 = rhizome_amd.prefill(w.q[a:b], w.k[a:b], w.v[a:b], w.g[a:b], w.beta[a:b],
                                 cu_seqlens=cu, initial_state=w.init[2:3].contiguous(), algo=algo)
    torch.cuda.synchronize()
    assert torch.equal(o3, o1[a:b]) and torch.equal(f3[0], f1[2]), "batch invariance broken"


@pytest.mark.parametrize("algo,dtype,tol", [("chunked", torch.bfloat16, BF16_TOL),
                                            ("recurrent", torch.float32, F32_TOL)])
def test_config1_full(device, algo, dtype, tol):
    """B=4 H=16 T=4096 d=128, every head against the oracle."""
    w = Prefill(**C1, dtype=dtype, device=device)
    o, fin = w.run(algo=algo)
    _check(w, o, fin, tol, tag=f"c1 {algo}")


def _recurrent_fp32(w):
    """The fp32 recurrent kernel (held to the oracle at 1e-4 on configs 0 and
    1) on the chunked run's bf16 inputs widened exactly to fp32."""
    import rhizome_amd
    o, fin = rhizome_amd.prefill(w.shaped(w.q).float(), w.shaped(w.k).float(), w.shaped(w.v).float(),
                                 w.shaped(w.g), w.shaped(w.beta), cu_seqlens=w.cu_dev,
                                 initial_state=w.init, algo="recurrent")
    torch.cuda.synchronize()
    return o.reshape(w.n_tok, w.heads, w.d_v), fin


def _check_all_units(w, o, fin, tag):
    """Every (sequence, head) of a large workload: finite, within the bf16
    tolerance of the fp32 recurrent kernel, and within the closed-form norm
    bound; a subset is then checked against the f64 oracle directly."""
    assert bool(torch.isfinite(o.float()).all()) and bool(torch.isfinite(fin).all()), f"{tag}: non-finite"
    ro, rf = _recurrent_fp32(w)
    # o by head: [H, tokens, d_v]
    mo = check_close_dev(o.transpose(0, 1).contiguous(), ro.transpose(0, 1).contiguous(), BF16_TOL,
                         f"{tag} o vs recurrent fp32", units=w.heads)
    mf = check_close_dev(fin, rf, BF16_TOL, f"{tag} final state vs recurrent fp32",
                         units=w.n_seqs * w.heads)
    nonexpansive_bound(w, fin)
    print(f"{tag} all {w.n_seqs * w.heads} units vs recurrent fp32: o {mo}  final {mf}", flush=True)
    return ro, rf


def _check_oracle_dev(w, ref, o, fin, tol, tag):
    """Every (sequence, head) unit against the f64 oracle, compared on the
    device (f64): o by head, the final states by unit."""
    ref_o, ref_f = ref
    dev = o.device
    ro = torch.from_numpy(ref_o).to(dev)
    mo = check_close_dev(o.transpose(0, 1).contiguous(), ro.transpose(0, 1).contiguous(), tol,
                         f"{tag} o vs oracle", units=w.heads)
    del ro
    mf = check_close_dev(fin, torch.from_numpy(ref_f).to(dev), tol, f"{tag} final state vs oracle",
                         units=w.n_seqs * w.heads)
    print(f"{tag} all {w.n_seqs * w.heads} units vs the f64 oracle: o {mo}  final {mf}", flush=True)


def test_config2_long_context(device):
    """B=1 H=32 T=32768 d_k=128 d_v=256, slow decay.  All 32 heads of the
    chunked and the fp32 recurrent kernel against the f64 oracle; the chunked
    kernel also against the recurrent one and the closed-form norm bound."""
    w = Prefill(**C2, dtype=torch.bfloat16, device=device)
    o, fin = w.run(algo="chunked")
    ro, rf = _check_all_units(w, o, fin, "c2 chunked")
    ref = w.oracle()
    _check_oracle_dev(w, ref, o, fin, BF16_TOL, "c2 chunked")
    _check_oracle_dev(w, ref, ro, rf, F32_TOL, "c2 recurrent fp32")


def test_config4_varlen(device):
    """64 packed sequences, lengths U[128, 8192], init states.  All 1024
    (sequence, head) units of the chunked and the fp32 recurrent kernel
    against the f64 oracle; the chunked kernel also against the recurrent one
    and the closed-form norm bound."""
    lengths = varlen_lengths(C4["n_seqs"], C4["len_lo"], C4["len_hi"])
    w = Prefill(heads=C4["heads"], d_k=C4["d_k"], d_v=C4["d_v"], lengths=lengths,
                dtype=torch.bfloat16, device=device, state_std=C4["state_std"])
    o, fin = w.run(algo="chunked")
    ro, rf = _check_all_units(w, o, fin, "c4 chunked")
    ref = w.oracle()
    _check_oracle_dev(w, ref, o, fin, BF16_TOL, "c4 chunked")
    _check_oracle_dev(w, ref, ro, rf, F32_TOL, "c4 recurrent fp32")


@pytest.mark.parametrize("algo,dtype", [("chunked", torch.bfloat16), ("recurrent", torch.float32)])
def test_state_in_place(device, algo, dtype):
    """final_state may be the initial_state buffer: the result is the same as
    with separate buffers, bit for bit, for dense and packed batches (each
    thread reads its slice of the state before it writes the same slice)."""
    for kw in (dict(batch=2, seq_len=150), dict(lengths=[70, 0, 130])):
        w = Prefill(heads=3, d_k=128, d_v=128 if algo == "chunked" else 96, dtype=dtype, device=device,
                    state_std=0.02, **kw)
        o_sep, fin_sep = w.run(algo=algo)  # separate initial and final buffers
        state = w.init.clone()
        saved, w.init = w.init, state
        try:
            o_in, fin_in = w.run(algo=algo, final_state=state)  # initial_state is final_state
        finally:
            w.init = saved
        assert fin_in.data_ptr() == state.data_ptr()
        assert torch.equal(o_in, o_sep) and torch.equal(state, fin_sep), f"{algo} {kw}"
