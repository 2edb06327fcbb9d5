"""ctypes front end of the CPU f64 oracle (oracle/gdr_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` -- as the reference that
results are compared against, never as the measured or shipped path.  The
product library never calls into it.

Every function here forwards to a C function that restates the f64
reference (``crates/ops/src/delta.rs``, ``rng.rs``, ``elementwise.rs``);
the C file header lists the file:line each one follows.  The config input
builders at the bottom implement the seeded distributions of the five
workloads (one Philox stream per tensor: q=1, k=2, v=3, beta=4, g=5,
initial state=6, varlen lengths=7; element order row-major).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import POINTER, c_double, c_int, c_int64, c_uint32, c_uint64, c_void_p

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# RHIZOME_ORACLE_LIB names another build of the oracle (the sanitizer build)
_LIB_PATH = os.environ.get("RHIZOME_ORACLE_LIB") or os.path.join(_HERE, "liboracle.so")
_lib = None

_dp = POINTER(c_double)


def build() -> str:
    """Compile liboracle.so with the committed Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.orc_philox_block.argtypes = [c_uint64, c_uint64, c_uint64, POINTER(c_uint32)]
        L.orc_philox_u32.argtypes = [c_uint64, c_uint64, c_int64, POINTER(c_uint32)]
        L.orc_philox_f64.argtypes = [c_uint64, c_uint64, c_int64, _dp]
        L.orc_philox_normal.argtypes = [c_uint64, c_uint64, c_int64, c_double, c_double, _dp, c_int]
        L.orc_sigmoid.argtypes = [c_double]
        L.orc_sigmoid.restype = c_double
        L.orc_softplus.argtypes = [c_double]
        L.orc_softplus.restype = c_double
        L.orc_l2norm.argtypes = [_dp, c_int64, c_double, _dp]
        L.orc_l2norm_rows.argtypes = [_dp, c_int64, c_int64, c_double, c_int]
        L.orc_sigmoid_vec.argtypes = [_dp, c_int64, _dp]
        L.orc_neg_softplus_vec.argtypes = [_dp, c_int64, _dp]
        L.orc_exp_vec.argtypes = [_dp, c_int64, _dp]
        L.orc_gated_delta_step.argtypes = [_dp, c_int64, _dp, _dp, _dp, c_double, c_double]
        L.orc_gated_delta_step.restype = c_void_p
        L.orc_free.argtypes = [c_void_p]
        seq_args = [c_int64, c_int64, _dp, _dp, _dp, _dp, _dp, POINTER(c_uint64), _dp]
        L.orc_gated_delta_sequential.argtypes = seq_args + [_dp, _dp]
        L.orc_gated_delta_scan_chunked.argtypes = seq_args + [c_int64, _dp, _dp]
        L.orc_gated_delta_multistep.argtypes = seq_args + [c_int64, _dp, _dp]
        L.orc_gated_delta_multistep.restype = c_int64
        L.orc_causal_conv1d_step.argtypes = [_dp, _dp, c_double, c_double]
        L.orc_causal_conv1d_step.restype = c_double
        L.orc_conv1d_batched.argtypes = [c_int64, POINTER(c_int64), c_int64, _dp, _dp, c_void_p,
                                         c_void_p, _dp, c_void_p]
        L.orc_rmsnorm_rows.argtypes = [c_int64, c_int64, _dp, _dp, c_double, _dp]
        L.orc_make_inputs.argtypes = [c_int64, c_int64, c_uint64, _dp, _dp, _dp, _dp, _dp]
        L.orc_gdr_steps_rect.argtypes = [
            c_int64, c_int64, c_int64, _dp, c_int64, _dp, c_int64, _dp, c_int64,
            _dp, _dp, c_int64, _dp, _dp, c_int64]
        L.orc_gdr_prefill_batched.argtypes = [
            c_int64, POINTER(c_int64), c_int64, c_int64, c_int64, _dp, _dp, _dp, _dp, _dp,
            _dp, _dp, _dp, c_int]
        L.orc_gdr_decode_batched.argtypes = [
            c_int64, c_int64, c_int64, c_int64, _dp, _dp, _dp, _dp, _dp, _dp, _dp, c_int]
        L.orc_max_threads.restype = c_int
        L.orc_bench_sequential.argtypes = [c_int64, c_int64, c_int64, _dp, _dp, _dp, _dp, _dp,
                                           _dp, _dp, c_int]
        L.orc_bench_step.argtypes = [c_int64, c_int64, _dp, _dp, _dp, _dp, _dp, _dp, _dp, c_int]
        _lib = L
    return _lib


def _f64(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float64)


def _p(a: np.ndarray):
    return a.ctypes.data_as(_dp)


def _pn(a):
    return None if a is None else _p(a)


MAX_THREADS = 16  # the host CPU share one GPU is given


def default_threads() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        n = os.cpu_count() or 1
    return max(1, min(n, MAX_THREADS))


# ----------------------------------------------------------------- Philox
def philox_block(seed: int, stream: int, counter: int) -> list[int]:
    out = (c_uint32 * 4)()
    lib().orc_philox_block(seed, stream, counter, out)
    return [int(x) for x in out]


def philox_u32(seed: int, stream: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint32)
    lib().orc_philox_u32(seed, stream, n, out.ctypes.data_as(POINTER(c_uint32)))
    return out


def philox_f64(seed: int, stream: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float64)
    lib().orc_philox_f64(seed, stream, n, _p(out))
    return out


def philox_normal(seed: int, stream: int, n: int, mean: float = 0.0, std: float = 1.0,
                  threads: int | None = None) -> np.ndarray:
    out = np.empty(n, dtype=np.float64)
    lib().orc_philox_normal(seed, stream, n, mean, std, _p(out), threads or default_threads())
    return out


# ------------------------------------------------------------ elementwise
def sigmoid(x: float) -> float:
    return lib().orc_sigmoid(x)


def softplus(x: float) -> float:
    return lib().orc_softplus(x)


def l2norm(x, scale: float = 1.0) -> np.ndarray:
    x = _f64(x)
    out = np.empty_like(x)
    lib().orc_l2norm(_p(x), x.size, scale, _p(out))
    return out


def l2norm_rows(x: np.ndarray, d: int, scale: float = 1.0, threads: int | None = None) -> None:
    """In place: every consecutive d-vector of the contiguous f64 array x."""
    assert x.dtype == np.float64 and x.flags.c_contiguous and x.size % d == 0
    lib().orc_l2norm_rows(_p(x), x.size // d, d, scale, threads or default_threads())


def sigmoid_vec(z) -> np.ndarray:
    z = _f64(z)
    out = np.empty_like(z)
    lib().orc_sigmoid_vec(_p(z), z.size, _p(out))
    return out


def neg_softplus_vec(z) -> np.ndarray:
    z = _f64(z)
    out = np.empty_like(z)
    lib().orc_neg_softplus_vec(_p(z), z.size, _p(out))
    return out


def exp_vec(z) -> np.ndarray:
    z = _f64(z)
    out = np.empty_like(z)
    lib().orc_exp_vec(_p(z), z.size, _p(out))
    return out


# --------------------------------------------------- reference API (one head)
def gated_delta_step(state: np.ndarray, q, k, v, alpha: float, beta: float) -> np.ndarray:
    """delta.rs:94-127; ``state`` (d*d f64, row-major S[i][j]) is updated in place."""
    assert state.dtype == np.float64 and state.flags.c_contiguous
    d = int(round(np.sqrt(state.size)))
    q, k, v = _f64(q), _f64(k), _f64(v)
    ptr = lib().orc_gated_delta_step(_p(state), d, _p(q), _p(k), _p(v), alpha, beta)
    o = np.ctypeslib.as_array(ctypes.cast(ptr, _dp), shape=(d,)).copy()
    lib().orc_free(ptr)
    return o


def _seq_common(q, k, v, alpha, beta, segment, init):
    q, k, v = _f64(q), _f64(k), _f64(v)
    alpha, beta = _f64(alpha), _f64(beta)
    t = alpha.size
    d = q.size // t if t else int(round(np.sqrt(np.asarray(init).size)))
    seg = np.ascontiguousarray(segment, dtype=np.uint64)
    init = _f64(init)
    return q, k, v, alpha, beta, seg, init, t, d


def gated_delta_sequential(q, k, v, alpha, beta, segment, init):
    """delta.rs:133-154 -> (out [T*d], final state [d*d])."""
    q, k, v, alpha, beta, seg, init, t, d = _seq_common(q, k, v, alpha, beta, segment, init)
    out = np.zeros(t * d)
    fin = np.zeros(d * d)
    lib().orc_gated_delta_sequential(t, d, _p(q), _p(k), _p(v), _p(alpha), _p(beta),
                                     seg.ctypes.data_as(POINTER(c_uint64)), _p(init), _p(out),
                                     _p(fin))
    return out, fin


def gated_delta_scan_chunked(q, k, v, alpha, beta, segment, init, chunk: int):
    """delta.rs:159-197 -> (out [T*d], final state [d*d])."""
    q, k, v, alpha, beta, seg, init, t, d = _seq_common(q, k, v, alpha, beta, segment, init)
    out = np.zeros(t * d)
    fin = np.zeros(d * d)
    lib().orc_gated_delta_scan_chunked(t, d, _p(q), _p(k), _p(v), _p(alpha), _p(beta),
                                       seg.ctypes.data_as(POINTER(c_uint64)), _p(init), chunk,
                                       _p(out), _p(fin))
    return out, fin


def gated_delta_multistep(q, k, v, alpha, beta, segment, init, max_positions: int):
    """delta.rs:202-230 -> (outs [n*d], states [n, d*d])."""
    q, k, v, alpha, beta, seg, init, t, d = _seq_common(q, k, v, alpha, beta, segment, init)
    n = min(t, max_positions)
    outs = np.zeros(max(n, 0) * d)
    states = np.zeros((max(n, 0), d * d))
    lib().orc_gated_delta_multistep(t, d, _p(q), _p(k), _p(v), _p(alpha), _p(beta),
                                    seg.ctypes.data_as(POINTER(c_uint64)), _p(init),
                                    max_positions, _p(outs), _p(states))
    return outs, states


def causal_conv1d_step(state: np.ndarray, weight, x: float, bias: float) -> float:
    """delta.rs:236-243; ``state`` (3 f64) is updated in place."""
    assert state.dtype == np.float64 and state.size == 3
    w = _f64(weight)
    return lib().orc_causal_conv1d_step(_p(state), _p(w), x, bias)


def conv1d_batched(cu_seqlens, x, weight, bias=None, init=None):
    """causal_conv1d_step (delta.rs:236-243) along packed sequences and channels.

    x [tokens, C]; weight [C, 4]; bias [C] or None; init [n, C, 3] or None.
    Returns (y [tokens, C], final state [n, C, 3]); tokens outside every
    sequence stay NaN."""
    x, weight = _f64(x), _f64(weight)
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int64)
    n = cu.size - 1
    tokens, C = x.shape
    y = np.full((tokens, C), np.nan)
    fin = np.zeros((n, C, 3))
    b = _f64(bias) if bias is not None else None
    st = _f64(init) if init is not None else None
    lib().orc_conv1d_batched(n, cu.ctypes.data_as(POINTER(c_int64)), C, _p(x), _p(weight),
                             _pn(b), _pn(st), _p(y), _p(fin))
    return y, fin


def rmsnorm_rows(x, scale, eps: float = 1e-6) -> np.ndarray:
    """rmsnorm (norm.rs:8-13) of every row of x [rows, dim]."""
    x, scale = _f64(x), _f64(scale)
    rows, dim = x.shape
    y = np.zeros_like(x)
    lib().orc_rmsnorm_rows(rows, dim, _p(x), _p(scale), eps, _p(y))
    return y


def prepare(q, k, beta_logit, alpha_logit, a_log, q_scale: float):
    """The op's inputs from the projections (SPEC.md:53-56) per (token, head):
    l2norm(q) * q_scale, l2norm(k), sigmoid(beta_logit),
    g = -softplus(a_log[h]) * softplus(alpha_logit).  q, k [tokens, H, d];
    logits [tokens, H]; a_log [H]."""
    q, k = _f64(q).copy(), _f64(k).copy()
    T, H, d = q.shape
    l2norm_rows(q.reshape(T * H, d), d, q_scale)
    l2norm_rows(k.reshape(T * H, d), d, 1.0)
    beta = sigmoid_vec(_f64(beta_logit).ravel()).reshape(T, H)
    sp_a = -neg_softplus_vec(_f64(a_log))
    sp_l = -neg_softplus_vec(_f64(alpha_logit).ravel()).reshape(T, H)
    return q, k, beta, -sp_a[None, :] * sp_l


def make_inputs(t: int, d: int, seed: int) -> dict:
    """delta.rs:254-280, the reference's own test-fixture builder."""
    q, k, v = np.zeros(t * d), np.zeros(t * d), np.zeros(t * d)
    a, b = np.zeros(t), np.zeros(t)
    lib().orc_make_inputs(t, d, seed, _p(q), _p(k), _p(v), _p(a), _p(b))
    return {"d": d, "q": q, "k": k, "v": v, "alpha": a, "beta": b}


# ------------------------------------------------ extensions (packed layouts)
def steps_rect(q, k, v, alpha, beta, state: np.ndarray) -> np.ndarray:
    """Init-honouring step loop on one head: q,k [T,dk], v [T,dv], state [dv,dk] in place."""
    q, k, v = _f64(q), _f64(k), _f64(v)
    alpha, beta = _f64(alpha), _f64(beta)
    t, dk = q.shape
    dv = v.shape[1]
    assert state.shape == (dv, dk) and state.dtype == np.float64 and state.flags.c_contiguous
    o = np.zeros((t, dv))
    lib().orc_gdr_steps_rect(t, dk, dv, _p(q), dk, _p(k), dk, _p(v), dv, _p(alpha), _p(beta), 1,
                             _p(state), _p(o), dv)
    return o


def prefill_batched(cu_seqlens, q, k, v, alpha, beta, init=None, want_final=True,
                    threads: int | None = None):
    """Packed prefill: q,k [N_tok,H,dk], v [N_tok,H,dv], alpha/beta [N_tok,H],
    init [N,H,dv,dk] or None.  Returns (o [N_tok,H,dv], final [N,H,dv,dk] or None)."""
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int64)
    q, k, v = _f64(q), _f64(k), _f64(v)
    alpha, beta = _f64(alpha), _f64(beta)
    n_tok, heads, dk = q.shape
    dv = v.shape[2]
    n = cu.size - 1
    init_a = None if init is None else _f64(init)
    o = np.zeros((n_tok, heads, dv))
    fin = np.zeros((n, heads, dv, dk)) if want_final else None
    lib().orc_gdr_prefill_batched(n, cu.ctypes.data_as(POINTER(c_int64)), heads, dk, dv, _p(q),
                                  _p(k), _p(v), _p(alpha), _p(beta), _pn(init_a), _p(o), _pn(fin),
                                  threads or default_threads())
    return o, fin


def decode_batched(q, k, v, alpha, beta, state: np.ndarray, threads: int | None = None):
    """One step for all (b,h): q,k [B,H,dk], v [B,H,dv], state [B,H,dv,dk] in place -> o."""
    q, k, v = _f64(q), _f64(k), _f64(v)
    alpha, beta = _f64(alpha), _f64(beta)
    b, h, dk = q.shape
    dv = v.shape[2]
    assert state.dtype == np.float64 and state.flags.c_contiguous and state.shape == (b, h, dv, dk)
    o = np.zeros((b, h, dv))
    lib().orc_gdr_decode_batched(b, h, dk, dv, _p(q), _p(k), _p(v), _p(alpha), _p(beta),
                                 _p(state), _p(o), threads or default_threads())
    return o


# ------------------------------------------------- config input builders
STREAM = {"q": 1, "k": 2, "v": 3, "beta": 4, "g": 5, "state": 6, "lengths": 7}


def unit_rows(seed: int, stream: int, rows: int, d: int) -> np.ndarray:
    """N(0,1) rows L2-normalised per d-vector (elementwise.rs:125-128, scale 1)."""
    x = philox_normal(seed, stream, rows * d)
    l2norm_rows(x, d)
    return x.reshape(rows, d)


def varlen_lengths(seed: int, n: int, lo: int = 128, hi: int = 8192) -> np.ndarray:
    """Seeded lengths lo + floor(u * (hi - lo + 1)), u = next_f64 of stream 7."""
    u = philox_f64(seed, STREAM["lengths"], n)
    return (lo + np.floor(u * (hi - lo + 1))).astype(np.int64)


def gdr_inputs(n_tok: int, heads: int, dk: int, dv: int, seed: int = 0, g_mean: float = 0.0,
               n_state: int = 0, state_std: float = 0.02) -> dict:
    """f64 inputs of one workload before quantisation.

    q,k: N(0,1) L2-normalised per (token, head); v: N(0,1); beta = sigmoid(N(0,1));
    g = -softplus(N(g_mean, 1)); optional initial states N(0, state_std) [n_state,H,dv,dk].
    """
    out = {
        "q": unit_rows(seed, STREAM["q"], n_tok * heads, dk).reshape(n_tok, heads, dk),
        "k": unit_rows(seed, STREAM["k"], n_tok * heads, dk).reshape(n_tok, heads, dk),
        "v": philox_normal(seed, STREAM["v"], n_tok * heads * dv).reshape(n_tok, heads, dv),
        "beta": sigmoid_vec(philox_normal(seed, STREAM["beta"], n_tok * heads)).reshape(
            n_tok, heads),
        "g": neg_softplus_vec(philox_normal(seed, STREAM["g"], n_tok * heads, g_mean)).reshape(
            n_tok, heads),
    }
    if n_state:
        out["state"] = philox_normal(seed, STREAM["state"], n_state * heads * dv * dk, 0.0,
                                     state_std).reshape(n_state, heads, dv, dk)
    return out


# ------------------------------------------------------- CPU baseline timing
def bench_sequential(q, k, v, alpha, beta, threads: int):
    """gated_delta_sequential over independent heads: q,k,v [U,T,d], alpha,beta [U,T]."""
    q, k, v = _f64(q), _f64(k), _f64(v)
    alpha, beta = _f64(alpha), _f64(beta)
    u, t, d = q.shape
    out = np.zeros((u, t, d))
    fin = np.zeros((u, d, d))
    lib().orc_bench_sequential(u, t, d, _p(q), _p(k), _p(v), _p(alpha), _p(beta), _p(out),
                               _p(fin), threads)
    return out, fin


def bench_step(q, k, v, alpha, beta, state: np.ndarray, threads: int):
    """gated_delta_step once per head: q,k,v [U,d], alpha,beta [U], state [U,d,d] in place."""
    q, k, v = _f64(q), _f64(k), _f64(v)
    alpha, beta = _f64(alpha), _f64(beta)
    u, d = q.shape
    o = np.zeros((u, d))
    lib().orc_bench_step(u, d, _p(q), _p(k), _p(v), _p(alpha), _p(beta), _p(state), _p(o), threads)
    return o
