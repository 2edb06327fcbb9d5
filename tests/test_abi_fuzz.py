"""Property tests of the C ABI's validation, without a GPU.

The header promises that every entry point validates everything it can
before touching the GPU, never aborts, and returns a status.  Here every
integer field takes values from the whole int32 range (negative, zero, huge,
overflowing products) and every pointer field is NULL, aligned or
misaligned.  The pointers are fake addresses, so no call may reach a launch:

* a call with rows to process has a NULL output, so validation must stop it
  with one of the validation errors (never OK, never a HIP error) and set a
  detail message;
* a call with nothing to process (zero tokens or rows) is legal and may
  still launch a kernel that writes final states; such draws get every
  pointer set to NULL, so that the call either returns OK without touching
  the GPU or fails validation.

The module is skipped where a GPU is visible, so that a draw that slips
past these rules can never dereference a fake address on a real device.
"""
from ctypes import byref, c_size_t

import pytest
from hypothesis import given, settings, strategies as st

from rhizome_amd import _abi


def _gpu_visible() -> bool:
    try:
        import torch

        return torch.cuda.device_count() > 0
    except Exception:
        return False


pytestmark = pytest.mark.skipif(_gpu_visible(), reason="fake device addresses: CPU-only property tests")

A = 0x10000  # a 256-byte-aligned fake device address; never dereferenced
VALIDATION = {_abi.ERR_INVALID_ARG, _abi.ERR_UNSUPPORTED, _abi.ERR_WORKSPACE}

ints = st.one_of(st.integers(-3, 300), st.sampled_from([0, 1, 64, 128, 256, 1024, 4096, 65536]),
                 st.integers(-2**31, 2**31 - 1))
enums = st.integers(-2, 5)
ptrs = st.sampled_from([None, A, A + 1, A + 2, A + 4, A + 8, A + 16])
FUZZ = settings(max_examples=300, deadline=None)


def fill(struct, data, ints_fields, enum_fields, ptr_fields, null_field):
    a = struct()
    for f in ints_fields:
        setattr(a, f, data.draw(ints, label=f))
    for f in enum_fields:
        setattr(a, f, data.draw(enums, label=f))
    for f in ptr_fields:
        setattr(a, f, data.draw(ptrs, label=f))
    setattr(a, null_field, None)
    return a


def null_all(a, ptr_fields):
    """A call with nothing to process: every pointer NULL, so that nothing a
    kernel could write through is a fake address."""
    for f in ptr_fields:
        setattr(a, f, None)


def check(status, nothing_to_do=False):
    """A validation error with its message; OK only where the call has no
    rows to process (such a call returns before looking at its pointers)."""
    if nothing_to_do and status == _abi.OK:
        return
    assert status in VALIDATION, (status, _abi.last_error())
    assert _abi.last_error()


PREFILL_PTRS = ["q", "k", "v", "gate", "beta", "cu_seqlens", "initial_state", "final_state", "workspace"]


@FUZZ
@given(st.data())
def test_prefill(data):
    a = fill(_abi.PrefillArgs, data, ["batch", "seq_len", "heads", "d_k", "d_v", "chunk"],
             ["dtype", "gate_kind", "algo"], PREFILL_PTRS, "o")
    a.workspace_bytes = data.draw(st.sampled_from([0, 16, 256, 1 << 20]))
    empty = a.seq_len == 0
    if empty:
        null_all(a, PREFILL_PTRS)
    check(_abi.lib().rhz_gdr_prefill(byref(a), None), nothing_to_do=empty)


@FUZZ
@given(st.data())
def test_prefill_workspace_query(data):
    # a pure query: any outcome but a HIP error, and a size that fits the arena rules
    a = fill(_abi.PrefillArgs, data, ["batch", "seq_len", "heads", "d_k", "d_v", "chunk"],
             ["dtype", "gate_kind", "algo"], ["q", "cu_seqlens"], "o")
    n = c_size_t(12345)
    status = _abi.lib().rhz_gdr_prefill_workspace_size(byref(a), byref(n))
    assert status in VALIDATION | {_abi.OK}, status
    if status == _abi.OK:
        assert n.value % 256 == 0 and n.value < 1 << 40
        if n.value:
            assert a.cu_seqlens  # only packed batches need scratch


@FUZZ
@given(st.data())
def test_decode(data):
    a = fill(_abi.DecodeArgs, data, ["batch", "heads", "d_k", "d_v"], ["dtype", "gate_kind"],
             ["q", "k", "v", "gate", "beta", "state"], "o")
    check(_abi.lib().rhz_gdr_decode_step(byref(a), None))


@FUZZ
@given(st.data())
def test_multistep(data):
    a = fill(_abi.MultistepArgs, data, ["batch", "steps", "heads", "d_k", "d_v"], ["dtype", "gate_kind"],
             ["q", "k", "v", "gate", "beta", "state", "o"], "states")
    check(_abi.lib().rhz_gdr_multistep(byref(a), None))


CONV_PTRS = ["x", "weight", "bias", "cu_seqlens", "initial_state", "final_state"]


@FUZZ
@given(st.data())
def test_conv1d(data):
    a = fill(_abi.Conv1dArgs, data, ["batch", "seq_len", "channels"], ["dtype"], CONV_PTRS, "y")
    empty = a.seq_len == 0
    if empty:
        null_all(a, CONV_PTRS)
    check(_abi.lib().rhz_causal_conv1d(byref(a), None), nothing_to_do=empty)


@FUZZ
@given(st.data())
def test_prepare(data):
    a = fill(_abi.PrepareArgs, data, ["tokens", "heads", "d_k"], ["dtype"],
             ["q_in", "k_in", "q_out", "k_out", "beta_logit", "alpha_logit", "a_log", "beta"], "g")
    a.q_scale = data.draw(st.floats(allow_nan=True, allow_infinity=True, width=32))
    check(_abi.lib().rhz_gdr_prepare(byref(a), None), nothing_to_do=a.tokens == 0)


@FUZZ
@given(st.data())
def test_rmsnorm(data):
    a = fill(_abi.RmsnormArgs, data, ["rows", "dim"], ["dtype"], ["x", "scale"], "y")
    a.eps = data.draw(st.floats(allow_nan=True, allow_infinity=True, width=32))
    check(_abi.lib().rhz_rmsnorm_heads(byref(a), None), nothing_to_do=a.rows == 0)


@FUZZ
@given(kind=enums, count=st.one_of(st.integers(-2**63, -1), st.integers(1, 2**63 - 1)), row_len=ints,
       dtype=enums, mean=st.floats(allow_nan=True), std=st.floats(allow_nan=True))
def test_philox_fill(kind, count, row_len, dtype, mean, std):
    # count != 0 with a NULL output: there is always something wrong
    status = _abi.lib().rhz_philox_fill(kind, 0, 0, count, row_len, mean, std, dtype, None, None)
    check(status)


@FUZZ
@given(op=enums, dtype=enums, dk=ints, dv=ints, algo=enums)
def test_query_support(op, dtype, dk, dv, algo):
    status = _abi.lib().rhz_gdr_query_support(op, dtype, dk, dv, algo)
    assert status in {_abi.OK, _abi.ERR_INVALID_ARG, _abi.ERR_UNSUPPORTED}, status
