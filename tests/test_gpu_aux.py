"""GPU parity of the Local-block prologue and epilogue around the op against
the f64 oracle, through the C ABI:
  rhz_causal_conv1d   causal_conv1d_step (crates/ops/src/delta.rs:232-243) along
                      packed sequences, carried state, reset at sequence starts
  rhz_gdr_prepare     l2norm / sigmoid / softplus (elementwise.rs:5-12, 36-42, 125-128)
                      composed as SPEC.md:53-56 describes
  rhz_rmsnorm_heads   rmsnorm / groupnorm_heads (norm.rs:8-13, 48-59)
"""
import numpy as np
import pytest
import torch

import rhizome_amd
from gdr_cases import BF16_TOL, F32_TOL, check_close, to_device
from oracle import oracle as O

pytestmark = pytest.mark.gpu
PATHS = [(torch.float32, F32_TOL), (torch.bfloat16, BF16_TOL)]


def _rng(seed):
    return np.random.default_rng(seed)


@pytest.mark.parametrize("dtype,tol", PATHS)
@pytest.mark.parametrize("lengths,C,with_state", [
    ([100, 100], 300, False),             # dense-shaped pack
    ([0, 1, 2, 3, 31, 32, 33, 0, 200], 257, True),   # empty and short sequences, span edges
    ([4096], 2048, True),
    # empty and short sequences at a vectorized width (16-byte rows): every
    # channel of an empty sequence must get its final state
    ([0, 5, 0, 17, 1, 0], 2048, True),
    ([0, 5, 0, 17, 1, 0], 2048, False),
    ([0, 0, 0], 6144, True),              # zero tokens, final states only
])
def test_conv1d(device, dtype, tol, lengths, C, with_state):
    rng = _rng(len(lengths) + C)
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    x, x64 = to_device(rng.normal(size=(cu[-1], C)), dtype, device)
    w, w64 = to_device(rng.normal(scale=0.5, size=(C, 4)), torch.float32, device)
    b, b64 = to_device(rng.normal(size=C), torch.float32, device)
    init = init64 = None
    if with_state:
        init, init64 = to_device(rng.normal(size=(len(lengths), C, 3)), torch.float32, device)
    cu_dev = torch.from_numpy(cu.astype(np.int32)).to(device)
    y, fin = rhizome_amd.causal_conv1d(x, w, b, cu_seqlens=cu_dev, initial_state=init,
                                       output_final_state=True)
    torch.cuda.synchronize()
    ry, rf = O.conv1d_batched(cu, x64, w64, b64, init64)
    my = check_close(y.float().cpu().numpy(), ry, tol, f"conv1d y {dtype}")
    mf = check_close(fin.cpu().numpy(), rf, tol, f"conv1d final state {dtype}")
    print(f"conv1d {lengths[:4]}.. C={C} {dtype}: y {my} final {mf}", flush=True)


def test_conv1d_dense_equals_packed(device):
    rng = _rng(9)
    B, T, C = 3, 77, 64
    x = torch.from_numpy(rng.normal(size=(B, T, C)).astype(np.float32)).to(device)
    w = torch.from_numpy(rng.normal(size=(C, 4)).astype(np.float32)).to(device)
    y1, f1 = rhizome_amd.causal_conv1d(x, w, output_final_state=True)
    cu = torch.arange(0, B * T + 1, T, dtype=torch.int32, device=device)
    y2, f2 = rhizome_amd.causal_conv1d(x.reshape(B * T, C), w, cu_seqlens=cu, output_final_state=True)
    torch.cuda.synchronize()
    assert torch.equal(y1.reshape(B * T, C), y2) and torch.equal(f1, f2)


@pytest.mark.parametrize("dtype,tol", PATHS)
@pytest.mark.parametrize("tokens,H,dk", [(1000, 4, 128), (5, 3, 64), (37, 2, 256), (64, 3, 37)])
def test_prepare(device, dtype, tol, tokens, H, dk):
    rng = _rng(tokens + dk)
    q, q64 = to_device(rng.normal(size=(tokens, H, dk)), dtype, device)
    k, k64 = to_device(rng.normal(size=(tokens, H, dk)), dtype, device)
    bl, bl64 = to_device(rng.normal(scale=3, size=(tokens, H)), torch.float32, device)
    al, al64 = to_device(rng.normal(scale=3, size=(tokens, H)), torch.float32, device)
    a, a64 = to_device(rng.normal(size=H), torch.float32, device)
    qo, ko, beta, g = rhizome_amd.prepare(q, k, bl, al, a)
    torch.cuda.synchronize()
    rq, rk, rb, rg = O.prepare(q64, k64, bl64, al64, a64, float(dk) ** 0.5)
    m = [check_close(qo.float().cpu().numpy(), rq, tol, "q"), check_close(ko.float().cpu().numpy(), rk, tol, "k"),
         check_close(beta.cpu().numpy(), rb, F32_TOL, "beta"), check_close(g.cpu().numpy(), rg, F32_TOL, "g")]
    print(f"prepare {tokens}x{H}x{dk} {dtype}: {m}", flush=True)


def test_prepare_in_place(device):
    rng = _rng(2)
    q = torch.from_numpy(rng.normal(size=(50, 4, 128)).astype(np.float32)).to(device)
    k = torch.from_numpy(rng.normal(size=(50, 4, 128)).astype(np.float32)).to(device)
    z = torch.zeros((50, 4), device=device)
    a = torch.zeros(4, device=device)
    q1, k1, _, _ = rhizome_amd.prepare(q, k, z, z, a)
    q2, k2, _, _ = rhizome_amd.prepare(q, k, z, z, a, q_out=q, k_out=k)
    torch.cuda.synchronize()
    assert torch.equal(q1, q2) and torch.equal(k1, k2)
    assert torch.allclose(k2.norm(dim=-1), torch.ones(50, 4, device=device), rtol=1e-6)


@pytest.mark.parametrize("dtype,tol", PATHS)
@pytest.mark.parametrize("rows,dim", [(2000, 128), (33, 100), (7, 1024), (300, 64), (9, 1)])
def test_rmsnorm(device, dtype, tol, rows, dim):
    rng = _rng(rows + dim)
    x, x64 = to_device(rng.normal(scale=3, size=(rows, dim)), dtype, device)
    s, s64 = to_device(rng.normal(size=dim), torch.float32, device)
    y = rhizome_amd.rmsnorm_heads(x, s, 1e-6)
    torch.cuda.synchronize()
    m = check_close(y.float().cpu().numpy(), O.rmsnorm_rows(x64, s64, 1e-6), tol, "rmsnorm")
    print(f"rmsnorm {rows}x{dim} {dtype}: {m}", flush=True)


def test_rmsnorm_in_place_and_heads_independent(device):
    x = torch.tensor([[1.0, 1.0], [100.0, 100.0]], device=device)  # norm.rs:117-123
    y = rhizome_amd.rmsnorm_heads(x, torch.ones(2, device=device), 1e-12, out=x)
    torch.cuda.synchronize()
    assert abs(float(y[0, 0]) - float(y[1, 0])) < 1e-6 and y.data_ptr() == x.data_ptr()


@pytest.mark.parametrize("dtype,algo,tol", [(torch.bfloat16, "chunked", BF16_TOL),
                                            (torch.float32, "recurrent", F32_TOL)])
def test_local_block_chain(device, dtype, algo, tol):
    """conv1d over each of the q, k, v projections -> prepare -> prefill ->
    per-head RMSNorm, each stage reading the previous stage's device output
    as it lies (views only, no copies between the library calls), packed
    sequences throughout.  Every stage is checked against the oracle applied
    to the device's own input of that stage, so each stage's tolerance is its
    own."""
    rng = _rng(21)
    H, dk, dv = 4, 64, 64
    lengths = [70, 0, 130, 5]
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    n_tok = int(cu[-1])
    cu_dev = torch.from_numpy(cu.astype(np.int32)).to(device)
    conv = {}
    for name, d in (("q", dk), ("k", dk), ("v", dv)):
        x, x64 = to_device(rng.normal(size=(n_tok, H * d)), dtype, device)
        w, w64 = to_device(rng.normal(scale=0.5, size=(H * d, 4)), torch.float32, device)
        y, _ = rhizome_amd.causal_conv1d(x, w, cu_seqlens=cu_dev)
        ry, _ = O.conv1d_batched(cu, x64, w64, None, None)
        y64 = y.double().cpu().numpy()
        check_close(y64, ry, tol, f"chain conv1d {name}")
        conv[name] = (y.view(n_tok, H, d), y64.reshape(n_tok, H, d))
    bl, bl64 = to_device(rng.normal(size=(n_tok, H)), torch.float32, device)
    al, al64 = to_device(rng.normal(size=(n_tok, H)), torch.float32, device)
    a, a64 = to_device(rng.normal(size=H), torch.float32, device)
    q, k, beta, g = rhizome_amd.prepare(conv["q"][0], conv["k"][0], bl, al, a)
    rq, rk, rb, rg = O.prepare(conv["q"][1], conv["k"][1], bl64, al64, a64, float(dk) ** 0.5)
    q64, k64 = q.double().cpu().numpy(), k.double().cpu().numpy()
    b64, g64 = beta.double().cpu().numpy(), g.double().cpu().numpy()
    check_close(q64, rq, tol, "chain prepare q")
    check_close(k64, rk, tol, "chain prepare k")
    check_close(b64, rb, F32_TOL, "chain prepare beta")
    check_close(g64, rg, F32_TOL, "chain prepare g")
    o, fin = rhizome_amd.prefill(q, k, conv["v"][0], g, beta, cu_seqlens=cu_dev, algo=algo)
    ro, rf = O.prefill_batched(cu, q64, k64, conv["v"][1], np.exp(g64), b64, None)
    check_close(o.double().cpu().numpy(), ro, tol, "chain prefill o")
    check_close(fin.cpu().numpy(), rf, tol, "chain prefill final state")
    s, s64 = to_device(rng.normal(size=dv), torch.float32, device)
    out = rhizome_amd.rmsnorm_heads(o.view(n_tok * H, dv), s, 1e-6)
    torch.cuda.synchronize()
    rr = O.rmsnorm_rows(o.double().cpu().numpy().reshape(n_tok * H, dv), s64, 1e-6)
    m = check_close(out.double().cpu().numpy(), rr, tol, "chain rmsnorm")
    print(f"local block chain {dtype} {algo}: rmsnorm {m}", flush=True)


@pytest.mark.parametrize("shape", [
    dict(lengths=None, batch=2, seq_len=150, H=2, dk=128, dv=128),
    dict(lengths=[0, 1, 63, 64, 65, 200, 0, 130], H=3, dk=64, dv=96),
    dict(lengths=[37, 300], H=2, dk=40, dv=24),
    dict(lengths=None, batch=1, seq_len=70, H=2, dk=32, dv=256),
])
@pytest.mark.parametrize("with_state", [False, True])
def test_local_prefill_matches_prepare_then_prefill(device, shape, with_state):
    """rhz_gdr_local_prefill (prepare fused into the chunked prefill) against
    the oracle's prepare -> prefill on the same raw projections and logits
    (SPEC.md:53-56; elementwise.rs:5-12, 36-42, 125-128; delta.rs:156-197),
    and against the device's own prepare -> prefill, which rounds the
    prepared q and k to bf16 on the way through HBM."""
    rng = _rng(31 + with_state)
    H, dk, dv = shape["H"], shape["dk"], shape["dv"]
    if shape["lengths"] is None:
        B, T = shape["batch"], shape["seq_len"]
        lengths = [T] * B
    else:
        lengths = shape["lengths"]
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    n_tok, n = int(cu[-1]), len(lengths)
    cu_dev = None if shape["lengths"] is None else torch.from_numpy(cu.astype(np.int32)).to(device)

    def shaped(t):
        return t if cu_dev is not None else t.reshape(B, T, *t.shape[1:])

    q, q64 = to_device(rng.normal(scale=2.0, size=(n_tok, H, dk)), torch.bfloat16, device)
    k, k64 = to_device(rng.normal(scale=0.5, size=(n_tok, H, dk)), torch.bfloat16, device)
    v, v64 = to_device(rng.normal(size=(n_tok, H, dv)), torch.bfloat16, device)
    bl, bl64 = to_device(rng.normal(size=(n_tok, H)), torch.float32, device)
    al, al64 = to_device(rng.normal(loc=-1.0, size=(n_tok, H)), torch.float32, device)
    a, a64 = to_device(rng.normal(size=H), torch.float32, device)
    init, init64 = (to_device(rng.normal(scale=0.05, size=(n, H, dv, dk)), torch.float32, device)
                    if with_state else (None, None))
    scale = float(dk) ** 0.5

    o, fin = rhizome_amd.local_prefill(shaped(q), shaped(k), shaped(v), shaped(bl), shaped(al), a,
                                       cu_seqlens=cu_dev, initial_state=init)
    torch.cuda.synchronize()
    assert rhizome_amd.sync_timeouts() == 0 and rhizome_amd.fp16_range_errors() == 0
    o = o.reshape(n_tok, H, dv)
    rq, rk, rb, rg = O.prepare(q64, k64, bl64, al64, a64, scale)
    ro, rf = O.prefill_batched(cu, rq, rk, v64, np.exp(rg), rb, init64)
    mo = check_close(o.double().cpu().numpy(), ro, BF16_TOL, "fused o")
    mf = check_close(fin.cpu().numpy(), rf, BF16_TOL, "fused final state")

    # The separate device kernels for comparison (reported, not asserted:
    # prepare rounds q * q_scale, of norm sqrt(d_k), to bf16 on the way
    # through HBM, so that path lies further from the oracle than the fused
    # one, which rounds to fp16 on chip; the chain test checks it stage by
    # stage).
    qp, kp, beta, g = rhizome_amd.prepare(q, k, bl, al, a, q_scale=scale)
    o2, _ = rhizome_amd.prefill(shaped(qp), shaped(kp), shaped(v), shaped(g), shaped(beta),
                                cu_seqlens=cu_dev, initial_state=init, algo="chunked")
    torch.cuda.synchronize()
    e2 = o2.reshape(n_tok, H, dv).double().cpu().numpy() - ro
    sep = float(np.linalg.norm(e2) / max(np.linalg.norm(ro), 1e-300))
    print(f"local prefill {shape} state={with_state}: o {mo} final {mf}; "
          f"prepare -> prefill normwise {sep:.3g}", flush=True)


def _conv_prepare_case(device, rng, lengths, H, dk, dv, dtype, with_state):
    """Inputs of one rhz_gdr_conv_prepare case and the oracle's conv1d -> prepare."""
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    n_tok, n = int(cu[-1]), len(lengths)
    C = H * (2 * dk + dv)
    x, x64 = to_device(rng.normal(size=(n_tok, C)), dtype, device)
    w, w64 = to_device(rng.normal(scale=0.5, size=(C, 4)), torch.float32, device)
    b, b64 = to_device(rng.normal(scale=0.1, size=C), torch.float32, device)
    bl, bl64 = to_device(rng.normal(size=(n_tok, H)), torch.float32, device)
    al, al64 = to_device(rng.normal(size=(n_tok, H)), torch.float32, device)
    a, a64 = to_device(rng.normal(size=H), torch.float32, device)
    init = init64 = None
    if with_state:
        init, init64 = to_device(rng.normal(size=(n, C, 3)), torch.float32, device)
    ry, rf = O.conv1d_batched(cu, x64, w64, b64, init64)
    qk = H * dk
    rq, rk, rb, rg = O.prepare(ry[:, :qk].reshape(n_tok, H, dk), ry[:, qk:2 * qk].reshape(n_tok, H, dk),
                               bl64, al64, a64, float(dk) ** 0.5)
    rv = ry[:, 2 * qk:].reshape(n_tok, H, dv)
    dev = dict(x=x, w=w, b=b, bl=bl, al=al, a=a, init=init,
               cu=torch.from_numpy(cu.astype(np.int32)).to(device))
    return dev, (rq, rk, rv, rb, rg, rf)


@pytest.mark.parametrize("dtype,tol", PATHS)
@pytest.mark.parametrize("lengths,H,dk,dv,with_state", [
    ([100, 100], 2, 128, 128, False),
    ([0, 1, 2, 3, 31, 32, 33, 0, 200], 3, 64, 96, True),     # empty and short sequences, span edges
    ([300, 17], 4, 32, 256, True),
    ([0, 5, 0, 17, 1, 0], 16, 128, 128, True),
    ([0, 0, 0], 2, 128, 64, True),                          # zero tokens, final states only
    ([513], 1, 8 * 64, 8, False),                            # the widest q/k rows (bf16: 64 lanes)
])
def test_conv_prepare(device, dtype, tol, lengths, H, dk, dv, with_state):
    """rhz_gdr_conv_prepare against the oracle's causal_conv1d_step
    (delta.rs:232-243) along packed sequences followed by prepare
    (elementwise.rs:5-12, 36-42, 125-128; SPEC.md:53-56)."""
    if dtype == torch.float32 and dk == 512:
        pytest.skip("fp32 rows of 512 need 128 lanes; the ABI takes up to 64")
    rng = _rng(77 + len(lengths) + dk)
    d, ref = _conv_prepare_case(device, rng, lengths, H, dk, dv, dtype, with_state)
    rq, rk, rv, rb, rg, rf = ref
    q, k, v, beta, g, fin = rhizome_amd.conv_prepare(d["x"], d["w"], d["b"], d["bl"], d["al"], d["a"], heads=H,
                                                     d_k=dk, d_v=dv, cu_seqlens=d["cu"], initial_state=d["init"],
                                                     output_final_state=True)
    torch.cuda.synchronize()
    n_tok = sum(lengths)
    if n_tok:
        mq = check_close(q.double().cpu().numpy(), rq, tol, "conv prepare q")
        check_close(k.double().cpu().numpy(), rk, tol, "conv prepare k")
        check_close(v.double().cpu().numpy(), rv, tol, "conv prepare v")
        check_close(beta.double().cpu().numpy(), rb, F32_TOL, "conv prepare beta")
        check_close(g.double().cpu().numpy(), rg, F32_TOL, "conv prepare g")
    else:
        mq = None
    mf = check_close(fin.cpu().numpy(), rf, F32_TOL, "conv prepare final conv state")
    print(f"conv prepare {lengths[:4]}.. H={H} d_k={dk} d_v={dv} {dtype}: q {mq} final {mf}", flush=True)


def test_conv_prepare_dense_equals_packed_and_chain(device):
    """Dense and packed calls agree bit for bit, and the pass equals the device's
    own conv1d -> prepare where that chain does not round in between (fp32)."""
    rng = _rng(91)
    B, T, H, dk, dv = 2, 150, 2, 64, 64
    C = H * (2 * dk + dv)
    x = torch.from_numpy(rng.normal(size=(B, T, C)).astype(np.float32)).to(device)
    w = torch.from_numpy(rng.normal(scale=0.5, size=(C, 4)).astype(np.float32)).to(device)
    bl = torch.from_numpy(rng.normal(size=(B, T, H)).astype(np.float32)).to(device)
    al = torch.from_numpy(rng.normal(size=(B, T, H)).astype(np.float32)).to(device)
    a = torch.from_numpy(rng.normal(size=H).astype(np.float32)).to(device)
    d1 = rhizome_amd.conv_prepare(x, w, None, bl, al, a, heads=H, d_k=dk, d_v=dv, output_final_state=True)
    cu = torch.tensor([0, T, 2 * T], dtype=torch.int32, device=device)
    d2 = rhizome_amd.conv_prepare(x.view(B * T, C), w, None, bl.view(B * T, H), al.view(B * T, H), a, heads=H,
                                  d_k=dk, d_v=dv, cu_seqlens=cu, output_final_state=True)
    torch.cuda.synchronize()
    for u, z in zip(d1, d2):
        assert torch.equal(u.reshape(-1), z.reshape(-1))
    y, fin = rhizome_amd.causal_conv1d(x, w, output_final_state=True)
    qk = H * dk
    q2, k2, beta2, g2 = rhizome_amd.prepare(y[..., :qk].contiguous().view(B, T, H, dk),
                                            y[..., qk:2 * qk].contiguous().view(B, T, H, dk), bl, al, a)
    torch.cuda.synchronize()
    assert torch.equal(fin, d1[5])
    assert torch.equal(y[..., 2 * qk:].reshape(B, T, H, dv), d1[2])
    assert torch.allclose(q2, d1[0], rtol=1e-5, atol=1e-6) and torch.allclose(k2, d1[1], rtol=1e-5, atol=1e-6)
    assert torch.equal(beta2, d1[3]) and torch.equal(g2, d1[4])


def test_local_chain_through_conv_prepare(device):
    """The Local block with its prologue in one pass: rhz_gdr_conv_prepare ->
    rhz_gdr_prefill (chunked) -> rhz_rmsnorm_heads, each stage reading the
    previous one's device output, against the oracle's conv1d -> prepare ->
    prefill -> rmsnorm on the same raw inputs."""
    rng = _rng(97)
    lengths, H, dk, dv = [0, 130, 64, 300, 1], 4, 128, 128
    d, ref = _conv_prepare_case(device, rng, lengths, H, dk, dv, torch.bfloat16, True)
    rq, rk, rv, rb, rg, _ = ref
    q, k, v, beta, g, _ = rhizome_amd.conv_prepare(d["x"], d["w"], d["b"], d["bl"], d["al"], d["a"], heads=H,
                                                   d_k=dk, d_v=dv, cu_seqlens=d["cu"], initial_state=d["init"])
    o, fin = rhizome_amd.prefill(q, k, v, g, beta, cu_seqlens=d["cu"], algo="chunked")
    s, s64 = to_device(rng.normal(size=dv), torch.float32, device)
    n_tok = sum(lengths)
    y = rhizome_amd.rmsnorm_heads(o.view(n_tok * H, dv), s, 1e-6)
    torch.cuda.synchronize()
    assert rhizome_amd.sync_timeouts() == 0 and rhizome_amd.fp16_range_errors() == 0 and rhizome_amd.exact_reruns() == 0
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    # each stage against the oracle on that stage's device input
    check_close(q.double().cpu().numpy(), rq, BF16_TOL, "chain conv prepare q")
    check_close(k.double().cpu().numpy(), rk, BF16_TOL, "chain conv prepare k")
    dq, dk_, dv_ = (t.double().cpu().numpy() for t in (q, k, v))
    db, dg = beta.double().cpu().numpy(), g.double().cpu().numpy()
    ro, rf = O.prefill_batched(cu, dq, dk_, dv_, np.exp(dg), db, None)
    mo = check_close(o.double().cpu().numpy(), ro, BF16_TOL, "chain prefill o")
    check_close(fin.cpu().numpy(), rf, BF16_TOL, "chain prefill final state")
    ry = O.rmsnorm_rows(o.double().cpu().numpy().reshape(n_tok * H, dv), s64, 1e-6)
    my = check_close(y.double().cpu().numpy(), ry, BF16_TOL, "chain rmsnorm")
    # end to end against the oracle's chain on the raw inputs (reported: the
    # prepared q and k are rounded to bf16 on the way through HBM, as after
    # rhz_gdr_prepare)
    ro2, _ = O.prefill_batched(cu, rq, rk, rv, np.exp(rg), rb, None)
    e2e = float(np.linalg.norm(o.double().cpu().numpy() - ro2) / max(np.linalg.norm(ro2), 1e-300))
    print(f"local chain through conv_prepare: o {mo} rmsnorm {my}; end-to-end o normwise {e2e:.3g}", flush=True)


def test_local_prefill_config1_shape(device):
    """rhz_gdr_local_prefill at the size it is benchmarked on (B=4, H=16,
    T=4096, d=128, raw projections and logits as the bench draws them)
    against the oracle's prepare -> prefill, every head."""
    from gdr_cases import C1, check_close_dev

    rng = _rng(57)
    B, T, H, dk, dv = C1["batch"], C1["seq_len"], C1["heads"], C1["d_k"], C1["d_v"]
    n_tok = B * T
    q, q64 = to_device(rng.normal(size=(n_tok, H, dk)), torch.bfloat16, device)
    k, k64 = to_device(rng.normal(size=(n_tok, H, dk)), torch.bfloat16, device)
    v, v64 = to_device(rng.normal(size=(n_tok, H, dv)), torch.bfloat16, device)
    bl, bl64 = to_device(rng.normal(size=(n_tok, H)), torch.float32, device)
    al, al64 = to_device(rng.normal(size=(n_tok, H)), torch.float32, device)
    a, a64 = to_device(rng.normal(size=H), torch.float32, device)
    scale = float(dk) ** 0.5
    lead = (B, T)
    o, fin = rhizome_amd.local_prefill(q.view(lead + (H, dk)), k.view(lead + (H, dk)), v.view(lead + (H, dv)),
                                       bl.view(lead + (H,)), al.view(lead + (H,)), a, q_scale=scale)
    torch.cuda.synchronize()
    assert rhizome_amd.sync_timeouts() == 0 and rhizome_amd.fp16_range_errors() == 0
    cu = np.arange(B + 1, dtype=np.int64) * T
    rq, rk, rb, rg = O.prepare(q64, k64, bl64, al64, a64, scale)
    ro, rf = O.prefill_batched(cu, rq, rk, v64, np.exp(rg), rb, None)
    ro_d = torch.from_numpy(ro).to(device).transpose(0, 1).contiguous()
    mo = check_close_dev(o.reshape(n_tok, H, dv).transpose(0, 1).contiguous(), ro_d, BF16_TOL,
                         "fused c1 o", units=H)
    del ro_d
    mf = check_close_dev(fin, torch.from_numpy(rf).to(device), BF16_TOL, "fused c1 final state", units=B * H)
    print(f"local prefill at B=4 H=16 T=4096 d=128: o {mo} final {mf}", flush=True)


@pytest.mark.parametrize("big", [7e4, 1e15])
def test_fused_prologues_take_large_projections(device, big):
    """Projections far beyond fp16's range (the plain chunked path's limit):
    both fused entry points normalise q and k before any fp16 operand is
    formed, so they match the oracle with no range error."""
    rng = _rng(61)
    lengths, H, dk, dv = [70, 130], 2, 64, 64
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    n_tok = int(cu[-1])
    qr = rng.normal(size=(n_tok, H, dk))
    kr = rng.normal(size=(n_tok, H, dk))
    qr[5, 0, 3] = big
    qr[100, 1, :] *= big
    kr[7, 1, 10] = -big
    q, q64 = to_device(qr, torch.bfloat16, device)
    k, k64 = to_device(kr, torch.bfloat16, device)
    v, v64 = to_device(rng.normal(size=(n_tok, H, dv)), torch.bfloat16, device)
    bl, bl64 = to_device(rng.normal(size=(n_tok, H)), torch.float32, device)
    al, al64 = to_device(rng.normal(size=(n_tok, H)), torch.float32, device)
    a, a64 = to_device(rng.normal(size=H), torch.float32, device)
    cu_dev = torch.from_numpy(cu.astype(np.int32)).to(device)
    scale = float(dk) ** 0.5
    rq, rk, rb, rg = O.prepare(q64, k64, bl64, al64, a64, scale)
    ro, rf = O.prefill_batched(cu, rq, rk, v64, np.exp(rg), rb, None)
    rhizome_amd.fp16_range_errors()  # reset
    o, fin = rhizome_amd.local_prefill(q, k, v, bl, al, a, q_scale=scale, cu_seqlens=cu_dev)
    torch.cuda.synchronize()
    assert rhizome_amd.fp16_range_errors() == 0 and rhizome_amd.sync_timeouts() == 0
    check_close(o.double().cpu().numpy(), ro, BF16_TOL, f"fused prologue o, element {big:g}")
    check_close(fin.cpu().numpy(), rf, BF16_TOL, f"fused prologue final state, element {big:g}")
    # the one-pass conv1d + prepare, with an identity conv (weight [0, 0, 0, 1])
    x = torch.cat([q.view(n_tok, H * dk), k.view(n_tok, H * dk), v.view(n_tok, H * dv)], dim=1).contiguous()
    C = x.shape[1]
    w = torch.zeros((C, 4), dtype=torch.float32, device=device)
    w[:, 3] = 1.0
    qp, kp, vp, beta, g, _ = rhizome_amd.conv_prepare(x, w, None, bl, al, a, heads=H, d_k=dk, d_v=dv,
                                                      cu_seqlens=cu_dev)
    o2, fin2 = rhizome_amd.prefill(qp, kp, vp, g, beta, cu_seqlens=cu_dev, algo="chunked")
    torch.cuda.synchronize()
    assert rhizome_amd.fp16_range_errors() == 0 and rhizome_amd.sync_timeouts() == 0 and rhizome_amd.exact_reruns() == 0
    # stage by stage: the prepared q, k against the oracle's prepare, the
    # prefill against the oracle on those (bf16) values
    check_close(qp.double().cpu().numpy(), rq, BF16_TOL, f"conv prepare q, element {big:g}")
    check_close(kp.double().cpu().numpy(), rk, BF16_TOL, f"conv prepare k, element {big:g}")
    ro2, rf2 = O.prefill_batched(cu, qp.double().cpu().numpy(), kp.double().cpu().numpy(), v64,
                                 np.exp(g.double().cpu().numpy()), beta.double().cpu().numpy(), None)
    check_close(o2.double().cpu().numpy(), ro2, BF16_TOL, f"conv prepare -> prefill o, element {big:g}")
    check_close(fin2.cpu().numpy(), rf2, BF16_TOL, f"conv prepare -> prefill final state, element {big:g}")


def test_local_prefill_is_deterministic_and_rejects_fp32(device):
    rng = _rng(41)
    H, dk, dv, T = 2, 64, 64, 200
    q, _ = to_device(rng.normal(size=(1, T, H, dk)), torch.bfloat16, device)
    k, _ = to_device(rng.normal(size=(1, T, H, dk)), torch.bfloat16, device)
    v, _ = to_device(rng.normal(size=(1, T, H, dv)), torch.bfloat16, device)
    bl, _ = to_device(rng.normal(size=(1, T, H)), torch.float32, device)
    al, _ = to_device(rng.normal(size=(1, T, H)), torch.float32, device)
    a, _ = to_device(rng.normal(size=H), torch.float32, device)
    o1, f1 = rhizome_amd.local_prefill(q, k, v, bl, al, a)
    o2, f2 = rhizome_amd.local_prefill(q, k, v, bl, al, a)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(f1, f2)
    with pytest.raises(rhizome_amd.gdr.GdrError, match="CHUNKED"):
        rhizome_amd.local_prefill(q.float(), k.float(), v.float(), bl, al, a)


def test_local_prefill_empty_sequences_copy_the_state(device):
    """No tokens, final states requested: the final state is the initial one,
    and the logits and a_log (NULL here) are never read."""
    from ctypes import byref

    from rhizome_amd import _abi, gdr

    H, dk, dv = 2, 64, 32
    cu = torch.zeros(3, dtype=torch.int32, device=device)
    init = torch.randn(2, H, dv, dk, device=device)
    fin = torch.full_like(init, float("nan"))
    q = torch.empty(0, H, dk, dtype=torch.bfloat16, device=device)
    v = torch.empty(0, H, dv, dtype=torch.bfloat16, device=device)
    o = torch.empty_like(v)
    la = _abi.LocalArgs()
    la.prefill = gdr.prefill_args(q, q, v, None, None, _abi.GATE_LOG_ALPHA, cu, init, fin, o, "chunked")
    ws = torch.empty(256, dtype=torch.uint8, device=device)
    la.prefill.workspace, la.prefill.workspace_bytes = ws.data_ptr(), ws.numel()
    la.q_scale = 8.0
    _abi.check(_abi.lib().rhz_gdr_local_prefill(byref(la), None))
    torch.cuda.synchronize()
    assert torch.equal(fin, init)
