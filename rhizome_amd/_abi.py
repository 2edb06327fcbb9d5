"""ctypes mirror of include/rhizome_gdr.h and the loader of librhizome_gdr.so.

The library is loaded from this package directory only (built in-tree by
rhizome_amd.build); if it is missing, loading raises -- there is no
fallback implementation of any entry point.
"""
from __future__ import annotations

import ctypes
import os
import re
from ctypes import (POINTER, Structure, c_char_p, c_double, c_float, c_int32, c_int64, c_size_t,
                    c_uint32, c_uint64, c_void_p)

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
# RHIZOME_GDR_LIB names another build of the same library (the host
# sanitizer build under _build/asan, for example); there is no other backend.
LIB_PATH = os.environ.get("RHIZOME_GDR_LIB") or os.path.join(HERE, "librhizome_gdr.so")
HEADER = os.path.join(ROOT, "include", "rhizome_gdr.h")

# rhz_status
OK, ERR_INVALID_ARG, ERR_UNSUPPORTED, ERR_WORKSPACE, ERR_HIP = 0, 1, 2, 3, 4
# rhz_dtype
F32, BF16, F64 = 0, 1, 2
# rhz_gate
GATE_LOG_ALPHA, GATE_ALPHA = 0, 1
# rhz_algo
ALGO_AUTO, ALGO_RECURRENT, ALGO_CHUNKED = 0, 1, 2
# rhz_op
OP_DELTA_SCAN, OP_DELTA_STEP, OP_DELTA_MULTISTEP = 0, 1, 2
MULTISTEP_MAX = 64
NOALLOC_MAX_SEQS = 65536
# rhz_fill_kind
FILL_NORMAL, FILL_UNIT_ROWS, FILL_SIGMOID, FILL_NEG_SOFTPLUS, FILL_UNIFORM = 0, 1, 2, 3, 4


class PrefillArgs(Structure):
    _fields_ = [
        ("batch", c_int32), ("seq_len", c_int32), ("heads", c_int32), ("d_k", c_int32),
        ("d_v", c_int32), ("chunk", c_int32), ("dtype", c_int32), ("gate_kind", c_int32),
        ("algo", c_int32),
        ("q", c_void_p), ("k", c_void_p), ("v", c_void_p), ("gate", c_void_p), ("beta", c_void_p),
        ("cu_seqlens", c_void_p), ("initial_state", c_void_p), ("final_state", c_void_p),
        ("o", c_void_p), ("workspace", c_void_p), ("workspace_bytes", c_size_t),
    ]


class LocalArgs(Structure):
    _fields_ = [
        ("prefill", PrefillArgs), ("q_scale", c_float),
        ("beta_logit", c_void_p), ("alpha_logit", c_void_p), ("a_log", c_void_p),
    ]


class DecodeArgs(Structure):
    _fields_ = [
        ("batch", c_int32), ("heads", c_int32), ("d_k", c_int32), ("d_v", c_int32),
        ("dtype", c_int32), ("gate_kind", c_int32),
        ("q", c_void_p), ("k", c_void_p), ("v", c_void_p), ("gate", c_void_p), ("beta", c_void_p),
        ("state", c_void_p), ("o", c_void_p),
    ]


class MultistepArgs(Structure):
    _fields_ = [
        ("batch", c_int32), ("steps", c_int32), ("heads", c_int32), ("d_k", c_int32),
        ("d_v", c_int32), ("dtype", c_int32), ("gate_kind", c_int32),
        ("q", c_void_p), ("k", c_void_p), ("v", c_void_p), ("gate", c_void_p), ("beta", c_void_p),
        ("state", c_void_p), ("states", c_void_p), ("o", c_void_p),
    ]


class Conv1dArgs(Structure):
    _fields_ = [
        ("batch", c_int32), ("seq_len", c_int32), ("channels", c_int32), ("dtype", c_int32),
        ("x", c_void_p), ("weight", c_void_p), ("bias", c_void_p), ("cu_seqlens", c_void_p),
        ("initial_state", c_void_p), ("final_state", c_void_p), ("y", c_void_p),
    ]


class PrepareArgs(Structure):
    _fields_ = [
        ("tokens", c_int32), ("heads", c_int32), ("d_k", c_int32), ("dtype", c_int32),
        ("q_scale", c_float),
        ("q_in", c_void_p), ("k_in", c_void_p), ("q_out", c_void_p), ("k_out", c_void_p),
        ("beta_logit", c_void_p), ("alpha_logit", c_void_p), ("a_log", c_void_p),
        ("beta", c_void_p), ("g", c_void_p),
    ]


class ConvPrepareArgs(Structure):
    _fields_ = [
        ("batch", c_int32), ("seq_len", c_int32), ("heads", c_int32), ("d_k", c_int32),
        ("d_v", c_int32), ("dtype", c_int32), ("q_scale", c_float),
        ("x", c_void_p), ("weight", c_void_p), ("bias", c_void_p), ("cu_seqlens", c_void_p),
        ("initial_state", c_void_p), ("final_state", c_void_p),
        ("beta_logit", c_void_p), ("alpha_logit", c_void_p), ("a_log", c_void_p),
        ("q", c_void_p), ("k", c_void_p), ("v", c_void_p), ("beta", c_void_p), ("g", c_void_p),
    ]


class RmsnormArgs(Structure):
    _fields_ = [
        ("rows", c_int32), ("dim", c_int32), ("dtype", c_int32), ("eps", c_float),
        ("x", c_void_p), ("scale", c_void_p), ("y", c_void_p),
    ]


class GdrError(RuntimeError):
    """A non-OK rhz_status, with the library's detail message."""

    def __init__(self, status: int, message: str):
        self.status = status
        super().__init__(f"{status_string(status)}: {message}")


_lib = None


def declared_functions() -> list[str]:
    """Names of the functions declared in include/rhizome_gdr.h."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rhz_\w+)\s*\(", text)))


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m rhizome_amd.build` "
                "(the gated delta-rule ops have no non-HIP implementation)")
        L = ctypes.CDLL(LIB_PATH)
        L.rhz_gdr_abi_version.restype = c_int32
        L.rhz_status_string.argtypes = [c_int32]
        L.rhz_status_string.restype = c_char_p
        L.rhz_last_error.restype = c_char_p
        L.rhz_gdr_query_support.argtypes = [c_int32] * 5
        L.rhz_gdr_query_support.restype = c_int32
        L.rhz_gdr_prefill_workspace_size.argtypes = [POINTER(PrefillArgs), POINTER(c_size_t)]
        L.rhz_gdr_prefill_workspace_size.restype = c_int32
        L.rhz_gdr_prefill.argtypes = [POINTER(PrefillArgs), c_void_p]
        L.rhz_gdr_prefill.restype = c_int32
        L.rhz_gdr_prefill_noalloc.argtypes = [POINTER(PrefillArgs), c_void_p]
        L.rhz_gdr_prefill_noalloc.restype = c_int32
        L.rhz_gdr_local_prefill.argtypes = [POINTER(LocalArgs), c_void_p]
        L.rhz_gdr_local_prefill.restype = c_int32
        L.rhz_gdr_sync_timeouts.argtypes = [POINTER(c_uint32), c_int32]
        L.rhz_gdr_sync_timeouts.restype = c_int32
        L.rhz_gdr_fp16_range_errors.argtypes = [POINTER(c_uint32), c_int32]
        L.rhz_gdr_fp16_range_errors.restype = c_int32
        L.rhz_gdr_exact_reruns.argtypes = [POINTER(c_uint32), c_int32]
        L.rhz_gdr_exact_reruns.restype = c_int32
        L.rhz_gdr_prefill_spin_limit.argtypes = [POINTER(PrefillArgs), c_int32, c_void_p]
        L.rhz_gdr_prefill_spin_limit.restype = c_int32
        L.rhz_gdr_decode_step.argtypes = [POINTER(DecodeArgs), c_void_p]
        L.rhz_gdr_decode_step.restype = c_int32
        L.rhz_gdr_multistep.argtypes = [POINTER(MultistepArgs), c_void_p]
        L.rhz_gdr_multistep.restype = c_int32
        L.rhz_causal_conv1d.argtypes = [POINTER(Conv1dArgs), c_void_p]
        L.rhz_causal_conv1d.restype = c_int32
        L.rhz_gdr_prepare.argtypes = [POINTER(PrepareArgs), c_void_p]
        L.rhz_gdr_prepare.restype = c_int32
        L.rhz_gdr_conv_prepare.argtypes = [POINTER(ConvPrepareArgs), c_void_p]
        L.rhz_gdr_conv_prepare.restype = c_int32
        L.rhz_rmsnorm_heads.argtypes = [POINTER(RmsnormArgs), c_void_p]
        L.rhz_rmsnorm_heads.restype = c_int32
        L.rhz_philox_fill.argtypes = [c_int32, c_uint64, c_uint64, c_int64, c_int32, c_double,
                                      c_double, c_int32, c_void_p, c_void_p]
        L.rhz_philox_fill.restype = c_int32
        if L.rhz_gdr_abi_version() != 1:
            raise RuntimeError("librhizome_gdr.so ABI version mismatch")
        _lib = L
    return _lib


def status_string(status: int) -> str:
    return lib().rhz_status_string(status).decode()


def last_error() -> str:
    return lib().rhz_last_error().decode()


def check(status: int) -> None:
    if status != OK:
        raise GdrError(status, last_error())
