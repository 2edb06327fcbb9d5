"""The C ABI of librhizome_gdr.so without a GPU: the library loads, exports
every function include/rhizome_gdr.h declares, and every validation error is
returned (with its detail message) before any HIP call is made."""
import ctypes
import subprocess
from ctypes import byref, c_size_t

import pytest

from rhizome_amd import _abi

A = 0x10000  # a 256-byte-aligned fake device address; never dereferenced


@pytest.fixture(scope="module")
def lib():
    return _abi.lib()


def test_exports_every_declared_function(lib):
    declared = _abi.declared_functions()
    assert len(declared) >= 8
    out = subprocess.run(["nm", "-D", "--defined-only", _abi.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = [f for f in declared if f not in exported]
    assert not missing, f"declared but not exported: {missing}"
    for f in declared:
        assert hasattr(lib, f)


def test_identity_and_status_strings(lib):
    assert lib.rhz_gdr_abi_version() == 1
    names = {0: "RHZ_OK", 1: "RHZ_ERR_INVALID_ARG", 2: "RHZ_ERR_UNSUPPORTED",
             3: "RHZ_ERR_WORKSPACE", 4: "RHZ_ERR_HIP", 99: "RHZ_ERR_UNKNOWN"}
    for code, name in names.items():
        assert _abi.status_string(code) == name


@pytest.mark.parametrize("op,dtype,dk,dv,algo,want", [
    (_abi.OP_DELTA_SCAN, _abi.BF16, 128, 128, _abi.ALGO_CHUNKED, _abi.OK),
    (_abi.OP_DELTA_SCAN, _abi.BF16, 128, 256, _abi.ALGO_AUTO, _abi.OK),
    (_abi.OP_DELTA_SCAN, _abi.BF16, 64, 64, _abi.ALGO_CHUNKED, _abi.OK),
    (_abi.OP_DELTA_SCAN, _abi.F32, 128, 128, _abi.ALGO_CHUNKED, _abi.ERR_UNSUPPORTED),
    (_abi.OP_DELTA_SCAN, _abi.BF16, 100, 128, _abi.ALGO_CHUNKED, _abi.ERR_UNSUPPORTED),
    (_abi.OP_DELTA_SCAN, _abi.BF16, 256, 128, _abi.ALGO_CHUNKED, _abi.ERR_UNSUPPORTED),
    (_abi.OP_DELTA_SCAN, _abi.BF16, 6, 6, _abi.ALGO_AUTO, _abi.OK),
    (_abi.OP_DELTA_SCAN, _abi.F32, 256, 1024, _abi.ALGO_RECURRENT, _abi.OK),
    (_abi.OP_DELTA_SCAN, _abi.F32, 257, 64, _abi.ALGO_RECURRENT, _abi.ERR_UNSUPPORTED),
    (_abi.OP_DELTA_STEP, _abi.F32, 128, 128, _abi.ALGO_AUTO, _abi.OK),
    (_abi.OP_DELTA_STEP, _abi.F32, 128, 128, _abi.ALGO_CHUNKED, _abi.ERR_UNSUPPORTED),
    (_abi.OP_DELTA_STEP, _abi.F32, 128, 2048, _abi.ALGO_AUTO, _abi.ERR_UNSUPPORTED),
    (_abi.OP_DELTA_MULTISTEP, _abi.BF16, 128, 128, _abi.ALGO_AUTO, _abi.OK),
    (_abi.OP_DELTA_MULTISTEP, _abi.F32, 64, 64, _abi.ALGO_CHUNKED, _abi.ERR_UNSUPPORTED),
    (7, _abi.F32, 128, 128, _abi.ALGO_AUTO, _abi.ERR_INVALID_ARG),
    (3, _abi.F32, 128, 128, _abi.ALGO_AUTO, _abi.ERR_INVALID_ARG),
    (_abi.OP_DELTA_STEP, _abi.F64, 128, 128, _abi.ALGO_AUTO, _abi.ERR_INVALID_ARG),
    (_abi.OP_DELTA_STEP, _abi.F32, 0, 128, _abi.ALGO_AUTO, _abi.ERR_INVALID_ARG),
    (_abi.OP_DELTA_SCAN, _abi.F32, 128, 128, 9, _abi.ERR_INVALID_ARG),
])
def test_query_support(lib, op, dtype, dk, dv, algo, want):
    assert lib.rhz_gdr_query_support(op, dtype, dk, dv, algo) == want


def _prefill(**over):
    a = _abi.PrefillArgs()
    a.batch, a.seq_len, a.heads, a.d_k, a.d_v, a.chunk = 4, 4096, 16, 128, 128, 64
    a.dtype, a.gate_kind, a.algo = _abi.BF16, _abi.GATE_LOG_ALPHA, _abi.ALGO_AUTO
    for name in ("q", "k", "v", "gate", "beta", "o", "final_state"):
        setattr(a, name, A)
    for key, val in over.items():
        setattr(a, key, val)
    return a


def _ws(a):
    n = c_size_t(0)
    st = _abi.lib().rhz_gdr_prefill_workspace_size(byref(a), byref(n))
    return st, n.value


def test_workspace_sizes():
    # dense batches need none; packed batches hold the longest-first order of the sequences
    assert _ws(_prefill()) == (_abi.OK, 0)
    assert _ws(_prefill(dtype=_abi.F32)) == (_abi.OK, 0)
    assert _ws(_prefill(algo=_abi.ALGO_RECURRENT, cu_seqlens=A)) == (_abi.OK, 0)
    assert _ws(_prefill(cu_seqlens=A, batch=64, seq_len=266000)) == (_abi.OK, 256)
    assert _ws(_prefill(cu_seqlens=A, batch=65, seq_len=266000)) == (_abi.OK, 512)
    assert _ws(_prefill(d_k=100, cu_seqlens=A)) == (_abi.OK, 0)  # AUTO falls back to recurrent
    assert _abi.lib().rhz_gdr_prefill_workspace_size(byref(_prefill()), None) == _abi.ERR_INVALID_ARG


@pytest.mark.parametrize("over,status,msg", [
    (dict(batch=0), _abi.ERR_INVALID_ARG, "batch"),
    (dict(seq_len=-1), _abi.ERR_INVALID_ARG, "seq_len"),
    (dict(heads=0), _abi.ERR_INVALID_ARG, "heads"),
    (dict(d_k=0), _abi.ERR_INVALID_ARG, "d_k"),
    (dict(d_v=0), _abi.ERR_INVALID_ARG, "d_v"),
    (dict(chunk=0), _abi.ERR_INVALID_ARG, "chunk"),
    (dict(dtype=_abi.F64), _abi.ERR_INVALID_ARG, "dtype"),
    (dict(gate_kind=5), _abi.ERR_INVALID_ARG, "gate_kind"),
    (dict(algo=-1), _abi.ERR_INVALID_ARG, "algo"),
    (dict(d_k=300), _abi.ERR_UNSUPPORTED, "d_k"),
    (dict(d_v=2000), _abi.ERR_UNSUPPORTED, "d_v"),
    (dict(dtype=_abi.F32, algo=_abi.ALGO_CHUNKED), _abi.ERR_UNSUPPORTED, "bf16"),
    (dict(d_k=100, algo=_abi.ALGO_CHUNKED), _abi.ERR_UNSUPPORTED, "multiples of 8"),
    (dict(batch=70000, seq_len=70000), _abi.ERR_INVALID_ARG, "2^31"),
    (dict(q=None), _abi.ERR_INVALID_ARG, "q is NULL"),
    (dict(k=None), _abi.ERR_INVALID_ARG, "k is NULL"),
    (dict(v=None), _abi.ERR_INVALID_ARG, "v is NULL"),
    (dict(gate=None), _abi.ERR_INVALID_ARG, "gate is NULL"),
    (dict(beta=None), _abi.ERR_INVALID_ARG, "beta is NULL"),
    (dict(o=None), _abi.ERR_INVALID_ARG, "o is NULL"),
    (dict(q=A + 8), _abi.ERR_INVALID_ARG, "16-byte aligned"),
    (dict(final_state=A + 4), _abi.ERR_INVALID_ARG, "final_state"),
    (dict(dtype=_abi.F32, algo=_abi.ALGO_RECURRENT, v=A + 2), _abi.ERR_INVALID_ARG, "v is not aligned"),
    (dict(beta=A + 1), _abi.ERR_INVALID_ARG, "4-byte aligned"),
    (dict(cu_seqlens=A), _abi.ERR_WORKSPACE, "workspace is NULL"),
    (dict(cu_seqlens=A, workspace=A, workspace_bytes=16), _abi.ERR_WORKSPACE, "needed"),
])
def test_prefill_validation(over, status, msg):
    args = _prefill(**over)
    st = _abi.lib().rhz_gdr_prefill(byref(args), None)
    assert st == status, _abi.last_error()
    assert msg in _abi.last_error()


def _local(**over):
    la = _abi.LocalArgs()
    pre = {k: v for k, v in over.items() if k not in ("q_scale", "beta_logit", "alpha_logit", "a_log")}
    la.prefill = _prefill(gate=None, beta=None, **pre)
    la.q_scale = over.get("q_scale", 11.3)
    la.beta_logit = over.get("beta_logit", A)
    la.alpha_logit = over.get("alpha_logit", A)
    la.a_log = over.get("a_log", A)
    return la


@pytest.mark.parametrize("over,status,msg", [
    (dict(batch=0), _abi.ERR_INVALID_ARG, "batch"),
    (dict(dtype=_abi.F32), _abi.ERR_UNSUPPORTED, "CHUNKED path only"),
    (dict(algo=_abi.ALGO_RECURRENT), _abi.ERR_UNSUPPORTED, "CHUNKED path only"),
    (dict(d_k=100), _abi.ERR_UNSUPPORTED, "CHUNKED path only"),
    (dict(dtype=_abi.F32, algo=_abi.ALGO_CHUNKED), _abi.ERR_UNSUPPORTED, "bf16"),
    (dict(beta_logit=None), _abi.ERR_INVALID_ARG, "beta_logit is NULL"),
    (dict(alpha_logit=None), _abi.ERR_INVALID_ARG, "alpha_logit is NULL"),
    (dict(a_log=None), _abi.ERR_INVALID_ARG, "a_log is NULL"),
    (dict(a_log=A + 2), _abi.ERR_INVALID_ARG, "a_log must be 4-byte aligned"),
    (dict(q_scale=float("nan")), _abi.ERR_INVALID_ARG, "q_scale must be finite"),
    (dict(q_scale=float("inf")), _abi.ERR_INVALID_ARG, "q_scale must be finite"),
    # beyond 2^15 the prepared q could leave the kernel's fp16 range
    (dict(q_scale=40000.0), _abi.ERR_UNSUPPORTED, "2^15"),
    (dict(q_scale=-32768.5), _abi.ERR_UNSUPPORTED, "2^15"),
    (dict(q=None), _abi.ERR_INVALID_ARG, "q is NULL"),
    (dict(k=A + 8), _abi.ERR_INVALID_ARG, "16-byte aligned"),
    (dict(beta_logit=A + 1), _abi.ERR_INVALID_ARG, "4-byte aligned"),
    (dict(cu_seqlens=A), _abi.ERR_WORKSPACE, "workspace is NULL"),
])
def test_local_prefill_validation(over, status, msg):
    """rhz_gdr_local_prefill checks its prefill part as rhz_gdr_prefill does,
    with the logits in place of gate and beta, and takes only the CHUNKED path."""
    st = _abi.lib().rhz_gdr_local_prefill(byref(_local(**over)), None)
    assert st == status, _abi.last_error()
    assert msg in _abi.last_error()
    assert _abi.lib().rhz_gdr_local_prefill(None, None) == _abi.ERR_INVALID_ARG


def test_local_prefill_nothing_to_do_is_ok():
    # no tokens and no final state: no pointer is needed or touched
    la = _local(seq_len=0, q=None, k=None, v=None, o=None, final_state=None, beta_logit=None,
                alpha_logit=None, a_log=None)
    assert _abi.lib().rhz_gdr_local_prefill(byref(la), None) == _abi.OK, _abi.last_error()


def test_prefill_workspace_alignment():
    st, need = _ws(_prefill(cu_seqlens=A))
    args = _prefill(cu_seqlens=A, workspace=A + 16, workspace_bytes=need)
    assert _abi.lib().rhz_gdr_prefill(byref(args), None) == _abi.ERR_WORKSPACE
    assert "256-byte" in _abi.last_error()
    assert _abi.lib().rhz_gdr_prefill(None, None) == _abi.ERR_INVALID_ARG


def _decode(**over):
    a = _abi.DecodeArgs()
    a.batch, a.heads, a.d_k, a.d_v = 256, 16, 128, 128
    a.dtype, a.gate_kind = _abi.F32, _abi.GATE_LOG_ALPHA
    for name in ("q", "k", "v", "gate", "beta", "state", "o"):
        setattr(a, name, A)
    for key, val in over.items():
        setattr(a, key, val)
    return a


@pytest.mark.parametrize("over,status,msg", [
    (dict(batch=0), _abi.ERR_INVALID_ARG, "batch"),
    (dict(heads=-3), _abi.ERR_INVALID_ARG, "heads"),
    (dict(d_k=0), _abi.ERR_INVALID_ARG, "d_k"),
    (dict(d_v=0), _abi.ERR_INVALID_ARG, "d_v"),
    (dict(dtype=7), _abi.ERR_INVALID_ARG, "dtype"),
    (dict(gate_kind=2), _abi.ERR_INVALID_ARG, "gate_kind"),
    (dict(d_k=512), _abi.ERR_UNSUPPORTED, "256"),
    (dict(d_v=4096), _abi.ERR_UNSUPPORTED, "1024"),
    (dict(state=None), _abi.ERR_INVALID_ARG, "state is NULL"),
    (dict(q=None), _abi.ERR_INVALID_ARG, "q is NULL"),
    (dict(o=None), _abi.ERR_INVALID_ARG, "o is NULL"),
    (dict(k=A + 2), _abi.ERR_INVALID_ARG, "k is not aligned"),
    (dict(state=A + 2), _abi.ERR_INVALID_ARG, "4-byte aligned"),
])
def test_decode_validation(over, status, msg):
    args = _decode(**over)
    assert _abi.lib().rhz_gdr_decode_step(byref(args), None) == status
    assert msg in _abi.last_error()
    assert _abi.lib().rhz_gdr_decode_step(None, None) == _abi.ERR_INVALID_ARG


def _multistep(**over):
    a = _abi.MultistepArgs()
    a.batch, a.steps, a.heads, a.d_k, a.d_v = 64, 8, 16, 128, 128
    a.dtype, a.gate_kind = _abi.F32, _abi.GATE_ALPHA
    for name in ("q", "k", "v", "gate", "beta", "state", "states", "o"):
        setattr(a, name, A)
    for key, val in over.items():
        setattr(a, key, val)
    return a


@pytest.mark.parametrize("over,status,msg", [
    (dict(batch=0), _abi.ERR_INVALID_ARG, "batch"),
    (dict(steps=0), _abi.ERR_INVALID_ARG, "steps"),
    (dict(heads=0), _abi.ERR_INVALID_ARG, "heads"),
    (dict(d_k=0), _abi.ERR_INVALID_ARG, "d_k"),
    (dict(d_v=-1), _abi.ERR_INVALID_ARG, "d_v"),
    (dict(dtype=_abi.F64), _abi.ERR_INVALID_ARG, "dtype"),
    (dict(gate_kind=3), _abi.ERR_INVALID_ARG, "gate_kind"),
    (dict(steps=_abi.MULTISTEP_MAX + 1), _abi.ERR_UNSUPPORTED, "steps"),
    (dict(d_k=257), _abi.ERR_UNSUPPORTED, "256"),
    (dict(d_v=1025), _abi.ERR_UNSUPPORTED, "1024"),
    (dict(batch=1 << 20, steps=64, heads=64), _abi.ERR_INVALID_ARG, "2^31"),
    (dict(q=None), _abi.ERR_INVALID_ARG, "q is NULL"),
    (dict(state=None), _abi.ERR_INVALID_ARG, "state is NULL"),
    (dict(states=None), _abi.ERR_INVALID_ARG, "states is NULL"),
    (dict(o=None), _abi.ERR_INVALID_ARG, "o is NULL"),
    (dict(v=A + 2), _abi.ERR_INVALID_ARG, "v is not aligned"),
    (dict(states=A + 2), _abi.ERR_INVALID_ARG, "4-byte aligned"),
])
def test_multistep_validation(over, status, msg):
    args = _multistep(**over)
    assert _abi.lib().rhz_gdr_multistep(byref(args), None) == status
    assert msg in _abi.last_error()
    assert _abi.lib().rhz_gdr_multistep(None, None) == _abi.ERR_INVALID_ARG


@pytest.mark.parametrize("args,msg", [
    ((9, 0, 1, 10, 1, 0.0, 1.0, _abi.F32, A), "kind"),
    ((0, 0, 1, -1, 1, 0.0, 1.0, _abi.F32, A), "count"),
    ((0, 0, 1, 10, 1, 0.0, 1.0, 5, A), "out_dtype"),
    ((1, 0, 1, 10, 3, 0.0, 1.0, _abi.F32, A), "row_len"),
    ((1, 0, 1, 10, 0, 0.0, 1.0, _abi.F32, A), "row_len"),
    ((0, 0, 1, 10, 1, 0.0, 1.0, _abi.F32, None), "out is NULL"),
])
def test_philox_fill_validation(args, msg):
    assert _abi.lib().rhz_philox_fill(*args, None) == _abi.ERR_INVALID_ARG
    assert msg in _abi.last_error()


def test_python_front_end_rejects_host_tensors():
    import torch

    import rhizome_amd

    q = torch.zeros((1, 4, 2, 8), dtype=torch.bfloat16)
    g = torch.zeros((1, 4, 2))
    with pytest.raises(ValueError):
        rhizome_amd.prefill(q, q, q, g, g)
    with pytest.raises(ValueError):
        rhizome_amd.prefill(q, q, q[..., :4, :], g, g)
    with pytest.raises(ValueError):
        rhizome_amd.prefill(q, q, q, g, g, alpha=g)


def _conv(**over):
    a = _abi.Conv1dArgs()
    a.batch, a.seq_len, a.channels, a.dtype = 4, 4096, 2048, _abi.BF16
    for name in ("x", "weight", "y"):
        setattr(a, name, A)
    for key, val in over.items():
        setattr(a, key, val)
    return a


@pytest.mark.parametrize("over,msg", [
    (dict(batch=0), "batch"), (dict(seq_len=-1), "seq_len"), (dict(channels=0), "channels"),
    (dict(dtype=_abi.F64), "dtype"), (dict(x=None), "x or y is NULL"), (dict(weight=None), "weight"),
    (dict(x=A + 1), "aligned"), (dict(bias=A + 2), "4-byte"), (dict(seq_len=1 << 20), "2^31"),
])
def test_conv1d_validation(over, msg):
    assert _abi.lib().rhz_causal_conv1d(byref(_conv(**over)), None) == _abi.ERR_INVALID_ARG
    assert msg in _abi.last_error()


def _convprep(**over):
    a = _abi.ConvPrepareArgs()
    a.batch, a.seq_len, a.heads, a.d_k, a.d_v = 4, 4096, 16, 128, 128
    a.dtype, a.q_scale = _abi.BF16, 11.3
    a.x = A
    # outputs at distinct fake addresses, far from x (validation only: every
    # case below fails before any HIP call)
    a.q, a.k, a.v = 1 << 36, 2 << 36, 3 << 36
    for name in ("weight", "beta_logit", "alpha_logit", "a_log", "beta", "g"):
        setattr(a, name, A)
    for key, val in over.items():
        setattr(a, key, val)
    return a


@pytest.mark.parametrize("over,status,msg", [
    (dict(batch=0), _abi.ERR_INVALID_ARG, "batch"), (dict(seq_len=-1), _abi.ERR_INVALID_ARG, "seq_len"),
    (dict(heads=0), _abi.ERR_INVALID_ARG, "heads"), (dict(d_k=0), _abi.ERR_INVALID_ARG, "d_k and d_v"),
    (dict(dtype=_abi.F64), _abi.ERR_INVALID_ARG, "dtype"),
    (dict(q_scale=float("inf")), _abi.ERR_INVALID_ARG, "q_scale must be finite"),
    (dict(d_k=96), _abi.ERR_UNSUPPORTED, "power of two"), (dict(d_v=12), _abi.ERR_UNSUPPORTED, "multiples of 8"),
    (dict(dtype=_abi.F32, d_k=48), _abi.ERR_UNSUPPORTED, "multiples of 4"),
    (dict(d_k=1024), _abi.ERR_UNSUPPORTED, "512"),
    (dict(weight=None), _abi.ERR_INVALID_ARG, "weight is NULL"), (dict(x=None), _abi.ERR_INVALID_ARG, "x is NULL"),
    (dict(g=None), _abi.ERR_INVALID_ARG, "g is NULL"),
    (dict(q=(1 << 36) + 8), _abi.ERR_INVALID_ARG, "q is not 16-byte aligned"),
    (dict(v=A), _abi.ERR_INVALID_ARG, "v overlaps x"),
    (dict(k=A + 4 * 4096 * 16 * 384 * 2 - 16), _abi.ERR_INVALID_ARG, "k overlaps x"),
    (dict(bias=A + 2), _abi.ERR_INVALID_ARG, "4-byte"),
    (dict(seq_len=1 << 20), _abi.ERR_INVALID_ARG, "2^31"),
])
def test_conv_prepare_validation(over, status, msg):
    assert _abi.lib().rhz_gdr_conv_prepare(byref(_convprep(**over)), None) == status
    assert msg in _abi.last_error()


def _prep(**over):
    a = _abi.PrepareArgs()
    a.tokens, a.heads, a.d_k, a.dtype, a.q_scale = 16384, 16, 128, _abi.BF16, 11.3
    for name in ("q_in", "k_in", "q_out", "k_out", "beta_logit", "alpha_logit", "a_log", "beta", "g"):
        setattr(a, name, A)
    for key, val in over.items():
        setattr(a, key, val)
    return a


@pytest.mark.parametrize("over,status,msg", [
    (dict(tokens=-1), _abi.ERR_INVALID_ARG, "tokens"), (dict(heads=0), _abi.ERR_INVALID_ARG, "heads"),
    (dict(d_k=0), _abi.ERR_INVALID_ARG, "d_k"), (dict(dtype=3), _abi.ERR_INVALID_ARG, "dtype"),
    (dict(d_k=257), _abi.ERR_UNSUPPORTED, "256"), (dict(a_log=None), _abi.ERR_INVALID_ARG, "a_log is NULL"),
    (dict(g=A + 2), _abi.ERR_INVALID_ARG, "g is not aligned"),
    (dict(tokens=1 << 20, heads=64), _abi.ERR_INVALID_ARG, "2^31"),
    (dict(q_scale=float("-inf")), _abi.ERR_INVALID_ARG, "q_scale must be finite"),
])
def test_prepare_validation(over, status, msg):
    assert _abi.lib().rhz_gdr_prepare(byref(_prep(**over)), None) == status
    assert msg in _abi.last_error()


def test_prepare_and_rmsnorm_no_rows_is_ok():
    assert _abi.lib().rhz_gdr_prepare(byref(_prep(tokens=0, q_in=None)), None) == _abi.OK
    a = _abi.RmsnormArgs()
    a.rows, a.dim, a.dtype, a.eps = 0, 128, _abi.F32, 1e-6
    assert _abi.lib().rhz_rmsnorm_heads(byref(a), None) == _abi.OK


@pytest.mark.parametrize("over,status,msg", [
    (dict(rows=-1), _abi.ERR_INVALID_ARG, "rows"), (dict(dim=0), _abi.ERR_INVALID_ARG, "dim"),
    (dict(dim=1025), _abi.ERR_UNSUPPORTED, "1024"), (dict(eps=-1.0), _abi.ERR_INVALID_ARG, "eps"),
    (dict(scale=None), _abi.ERR_INVALID_ARG, "NULL"), (dict(dtype=_abi.F64), _abi.ERR_INVALID_ARG, "dtype"),
])
def test_rmsnorm_validation(over, status, msg):
    a = _abi.RmsnormArgs()
    a.rows, a.dim, a.dtype, a.eps = 16384 * 16, 128, _abi.BF16, 1e-6
    a.x, a.scale, a.y = A, A, A
    for key, val in over.items():
        setattr(a, key, val)
    assert _abi.lib().rhz_rmsnorm_heads(byref(a), None) == status
    assert msg in _abi.last_error()
