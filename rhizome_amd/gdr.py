"""Torch-tensor front end of the gated delta-rule C ABI (librhizome_gdr.so).

PyTorch is used only for device memory and streams: every function checks
shapes, fills the C argument struct with raw device pointers and calls the
library on the current HIP stream.  Nothing here computes the op.

Layouts follow include/rhizome_gdr.h: q, k [B, T, H, d_k] (dense) or
[tokens, H, d_k] with ``cu_seqlens``; v, o likewise with d_v; gates and
beta [B, T, H] / [tokens, H] fp32; states [N, H, d_v, d_k] fp32 with
S[i][j] = state[..., i, j] (i = value row, j = key column, the layout of
crates/ops/src/delta.rs:63).
"""
from __future__ import annotations

from ctypes import byref, c_size_t, c_uint32

import torch

from . import _abi
from ._abi import GdrError  # noqa: F401  (re-exported)

_ALGOS = {"auto": _abi.ALGO_AUTO, "recurrent": _abi.ALGO_RECURRENT, "chunked": _abi.ALGO_CHUNKED}
_DTYPES = {torch.float32: _abi.F32, torch.bfloat16: _abi.BF16}


def _ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("all tensors must be on the GPU")
    if not t.is_contiguous():
        raise ValueError("all tensors must be contiguous")
    return t.data_ptr() or None


def _stream(stream) -> int | None:
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream or None


def _gate(g, alpha):
    if (g is None) == (alpha is None):
        raise ValueError("pass exactly one of g (log-decay) and alpha")
    return (g, _abi.GATE_LOG_ALPHA) if g is not None else (alpha, _abi.GATE_ALPHA)


def prefill_args(q, k, v, gate, beta, gate_kind, cu_seqlens=None, initial_state=None,
                 final_state=None, o=None, algo="auto", chunk=64, workspace=None) -> _abi.PrefillArgs:
    """Fill the C argument struct (shapes are read from the tensors)."""
    if cu_seqlens is None:
        B, T, H, dk = q.shape
        batch, seq_len = B, T
    else:
        _, H, dk = q.shape
        batch, seq_len = cu_seqlens.numel() - 1, q.shape[0]
    dv = v.shape[-1]
    a = _abi.PrefillArgs()
    a.batch, a.seq_len, a.heads, a.d_k, a.d_v = batch, seq_len, H, dk, dv
    a.chunk = chunk
    a.dtype = _DTYPES[q.dtype]
    a.gate_kind = gate_kind
    a.algo = _ALGOS[algo]
    a.q, a.k, a.v, a.gate, a.beta = _ptr(q), _ptr(k), _ptr(v), _ptr(gate), _ptr(beta)
    a.cu_seqlens = _ptr(cu_seqlens)
    a.initial_state, a.final_state, a.o = _ptr(initial_state), _ptr(final_state), _ptr(o)
    if workspace is not None:
        a.workspace, a.workspace_bytes = _ptr(workspace), workspace.numel()
    return a


def workspace_bytes(args: _abi.PrefillArgs) -> int:
    n = c_size_t(0)
    _abi.check(_abi.lib().rhz_gdr_prefill_workspace_size(byref(args), byref(n)))
    return n.value


def _check_prefill_shapes(q, k, v, gate, beta, cu_seqlens, initial_state):
    dense = cu_seqlens is None
    nd = 4 if dense else 3
    if q.dim() != nd or k.shape != q.shape or v.dim() != nd or v.shape[:-1] != q.shape[:-1]:
        raise ValueError(f"q/k/v shapes {tuple(q.shape)} {tuple(k.shape)} {tuple(v.shape)} "
                         f"do not match the {'dense' if dense else 'packed'} layout")
    if gate.shape != q.shape[:-1] or beta.shape != q.shape[:-1]:
        raise ValueError("gate and beta must have shape q.shape[:-1]")
    if gate.dtype != torch.float32 or beta.dtype != torch.float32:
        raise ValueError("gate and beta must be fp32")
    if k.dtype != q.dtype or v.dtype != q.dtype or q.dtype not in _DTYPES:
        raise ValueError("q, k, v must share one dtype, fp32 or bf16")
    if not dense and cu_seqlens.dtype != torch.int32:
        raise ValueError("cu_seqlens must be int32")
    n = q.shape[0] if dense else cu_seqlens.numel() - 1
    if initial_state is not None:
        want = (n, q.shape[-2], v.shape[-1], q.shape[-1])
        if tuple(initial_state.shape) != want or initial_state.dtype != torch.float32:
            raise ValueError(f"initial_state must be fp32 {want}")
    return n


def prefill(q, k, v, g=None, beta=None, *, alpha=None, cu_seqlens=None, initial_state=None,
            output_final_state=True, algo="auto", chunk=64, workspace=None, out=None,
            final_state=None, stream=None):
    """Gated delta-rule prefill.  Returns (o, final_state or None).

    g is the per-token log-decay (alpha = exp(g)); pass alpha= instead to give
    alpha itself.  ``initial_state=None`` starts from zeros.
    """
    gate, gate_kind = _gate(g, alpha)
    n = _check_prefill_shapes(q, k, v, gate, beta, cu_seqlens, initial_state)
    o = out if out is not None else torch.empty(v.shape, dtype=q.dtype, device=q.device)
    fin = final_state
    if fin is None and output_final_state:
        fin = torch.empty((n, q.shape[-2], v.shape[-1], q.shape[-1]), dtype=torch.float32,
                          device=q.device)
    args = prefill_args(q, k, v, gate, beta, gate_kind, cu_seqlens, initial_state, fin, o, algo,
                        chunk)
    need = workspace_bytes(args)
    if need and workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    if workspace is not None:
        args.workspace, args.workspace_bytes = _ptr(workspace), workspace.numel()
    _abi.check(_abi.lib().rhz_gdr_prefill(byref(args), _stream(stream)))
    return o, fin


def local_prefill(q, k, v, beta_logit, alpha_logit, a_log, *, q_scale=None, cu_seqlens=None,
                  initial_state=None, output_final_state=True, workspace=None, out=None,
                  final_state=None, stream=None):
    """rhz_gdr_prepare fused into the chunked prefill (rhz_gdr_local_prefill).

    q, k are the raw projections (bf16), beta_logit / alpha_logit the gate
    logits [.., H] fp32 and a_log [H] fp32; q_scale defaults to sqrt(d_k).
    Returns (o, final_state or None), as :func:`prefill` does on the
    prepared inputs.
    """
    n = _check_prefill_shapes(q, k, v, alpha_logit, beta_logit, cu_seqlens, initial_state)
    H = q.shape[-2]
    if a_log.shape != (H,) or a_log.dtype != torch.float32:
        raise ValueError(f"a_log must be fp32 ({H},)")
    o = out if out is not None else torch.empty(v.shape, dtype=q.dtype, device=q.device)
    fin = final_state
    if fin is None and output_final_state:
        fin = torch.empty((n, H, v.shape[-1], q.shape[-1]), dtype=torch.float32, device=q.device)
    la = _abi.LocalArgs()
    la.prefill = prefill_args(q, k, v, None, None, _abi.GATE_LOG_ALPHA, cu_seqlens, initial_state,
                              fin, o, "chunked")
    la.q_scale = float(q.shape[-1]) ** 0.5 if q_scale is None else float(q_scale)
    la.beta_logit, la.alpha_logit, la.a_log = _ptr(beta_logit), _ptr(alpha_logit), _ptr(a_log)
    need = workspace_bytes(la.prefill)
    if need and workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    if workspace is not None:
        la.prefill.workspace, la.prefill.workspace_bytes = _ptr(workspace), workspace.numel()
    _abi.check(_abi.lib().rhz_gdr_local_prefill(byref(la), _stream(stream)))
    return o, fin


def sync_timeouts(reset: bool = True) -> int:
    """Number of the chunked kernel's LDS waits that gave up on the current
    device since the last reset (0 unless a launch may have gone wrong).
    Waits for all of the device's outstanding work on every stream first;
    the read and the reset are one atomic exchange on the device."""
    n = c_uint32(0)
    _abi.check(_abi.lib().rhz_gdr_sync_timeouts(byref(n), 1 if reset else 0))
    return n.value


def fp16_range_errors(reset: bool = True) -> int:
    """Number of (workgroup, wave) pairs of fused-prologue launches
    (local_prefill), counted once per launch, on the current device since
    the last reset whose fp16 operands formed from q and k were NaN,
    infinite or beyond fp16's range in any chunk (non-finite projections);
    0 unless such a launch may have gone wrong.  The plain chunked path
    reruns those workgroups exactly instead (exact_reruns).  Waits for all
    of the device's outstanding work on every stream first; the read and the
    reset are one atomic exchange on the device."""
    n = c_uint32(0)
    _abi.check(_abi.lib().rhz_gdr_fp16_range_errors(byref(n), 1 if reset else 0))
    return n.value


def exact_reruns(reset: bool = True) -> int:
    """Number of chunked-kernel workgroups (32 state rows of a (sequence,
    head) each) on the current device since the last reset that recomputed
    their rows with the fp32 recurrence because an input left the fp16
    path's domain (a key row with |k|^2 > 1.03125, beta or alpha outside
    [0, 1], an fp16 operand out of range).  Their results are correct; the
    count says how often the slower path ran.  Same synchronisation as
    fp16_range_errors."""
    n = c_uint32(0)
    _abi.check(_abi.lib().rhz_gdr_exact_reruns(byref(n), 1 if reset else 0))
    return n.value


def decode_args(q, k, v, gate, beta, gate_kind, state, o) -> _abi.DecodeArgs:
    B, H, dk = q.shape
    a = _abi.DecodeArgs()
    a.batch, a.heads, a.d_k, a.d_v = B, H, dk, v.shape[-1]
    a.dtype = _DTYPES[q.dtype]
    a.gate_kind = gate_kind
    a.q, a.k, a.v, a.gate, a.beta = _ptr(q), _ptr(k), _ptr(v), _ptr(gate), _ptr(beta)
    a.state, a.o = _ptr(state), _ptr(o)
    return a


def decode_step(q, k, v, g=None, beta=None, *, alpha=None, state, out=None, stream=None):
    """One decode position for every (b, h); ``state`` [B,H,d_v,d_k] fp32 is updated in place."""
    gate, gate_kind = _gate(g, alpha)
    B, H, dk = q.shape
    dv = v.shape[-1]
    if k.shape != q.shape or v.shape[:2] != (B, H) or gate.shape != (B, H) or beta.shape != (B, H):
        raise ValueError("decode shapes: q,k [B,H,dk], v [B,H,dv], gate/beta [B,H]")
    if tuple(state.shape) != (B, H, dv, dk) or state.dtype != torch.float32:
        raise ValueError("state must be fp32 [B,H,d_v,d_k]")
    o = out if out is not None else torch.empty((B, H, dv), dtype=q.dtype, device=q.device)
    args = decode_args(q, k, v, gate, beta, gate_kind, state, o)
    _abi.check(_abi.lib().rhz_gdr_decode_step(byref(args), _stream(stream)))
    return o


def multistep_args(q, k, v, gate, beta, gate_kind, state, states, o) -> _abi.MultistepArgs:
    B, n, H, dk = q.shape
    a = _abi.MultistepArgs()
    a.batch, a.steps, a.heads, a.d_k, a.d_v = B, n, H, dk, v.shape[-1]
    a.dtype = _DTYPES[q.dtype]
    a.gate_kind = gate_kind
    a.q, a.k, a.v, a.gate, a.beta = _ptr(q), _ptr(k), _ptr(v), _ptr(gate), _ptr(beta)
    a.state, a.states, a.o = _ptr(state), _ptr(states), _ptr(o)
    return a


def multistep(q, k, v, g=None, beta=None, *, alpha=None, state, out=None, states=None,
              stream=None):
    """n consecutive positions for every (b, h) from ``state`` (read only).

    q, k [B, n, H, d_k]; v [B, n, H, d_v]; gates [B, n, H].  Returns
    (o [B, n, H, d_v], states [B, n, H, d_v, d_k]) with the state after each
    position.  A segment change at position t is ``alpha[:, t] = 0``.
    """
    gate, gate_kind = _gate(g, alpha)
    B, n, H, dk = q.shape
    dv = v.shape[-1]
    if (k.shape != q.shape or v.shape[:3] != (B, n, H) or gate.shape != (B, n, H)
            or beta.shape != (B, n, H)):
        raise ValueError("multistep shapes: q,k [B,n,H,dk], v [B,n,H,dv], gate/beta [B,n,H]")
    if tuple(state.shape) != (B, H, dv, dk) or state.dtype != torch.float32:
        raise ValueError("state must be fp32 [B,H,d_v,d_k]")
    o = out if out is not None else torch.empty((B, n, H, dv), dtype=q.dtype, device=q.device)
    if states is None:
        states = torch.empty((B, n, H, dv, dk), dtype=torch.float32, device=q.device)
    args = multistep_args(q, k, v, gate, beta, gate_kind, state, states, o)
    _abi.check(_abi.lib().rhz_gdr_multistep(byref(args), _stream(stream)))
    return o, states


def causal_conv1d(x, weight, bias=None, *, cu_seqlens=None, initial_state=None,
                  output_final_state=False, out=None, stream=None):
    """Causal depthwise conv1d of width 4 (delta.rs:232-243 per channel).

    x [B, T, C] (dense) or [tokens, C] with ``cu_seqlens``; weight [C, 4]
    fp32; bias [C]; initial_state [N, C, 3].  Returns (y, final_state or None).
    """
    if cu_seqlens is None:
        B, T, C = x.shape
        batch, seq_len = B, T
    else:
        seq_len, C = x.shape
        batch = cu_seqlens.numel() - 1
    if tuple(weight.shape) != (C, 4) or weight.dtype != torch.float32:
        raise ValueError("weight must be fp32 [C, 4]")
    y = out if out is not None else torch.empty_like(x)
    fin = None
    if output_final_state:
        fin = torch.empty((batch, C, 3), dtype=torch.float32, device=x.device)
    a = _abi.Conv1dArgs()
    a.batch, a.seq_len, a.channels, a.dtype = batch, seq_len, C, _DTYPES[x.dtype]
    a.x, a.weight, a.bias, a.y = _ptr(x), _ptr(weight), _ptr(bias), _ptr(y)
    a.cu_seqlens, a.initial_state, a.final_state = _ptr(cu_seqlens), _ptr(initial_state), _ptr(fin)
    _abi.check(_abi.lib().rhz_causal_conv1d(byref(a), _stream(stream)))
    return y, fin


def prepare(q, k, beta_logit, alpha_logit, a_log, *, q_scale=None, q_out=None, k_out=None,
            stream=None):
    """q := l2norm(q) * q_scale (default sqrt(d_k)), k := l2norm(k),
    beta := sigmoid(beta_logit), g := -softplus(a_log[h]) * softplus(alpha_logit).

    q, k [..., H, d_k]; logits [..., H]; a_log [H].  Returns (q, k, beta, g).
    """
    *lead, H, dk = q.shape
    tokens = 1
    for n in lead:
        tokens *= n
    qo = q_out if q_out is not None else torch.empty_like(q)
    ko = k_out if k_out is not None else torch.empty_like(k)
    beta = torch.empty(beta_logit.shape, dtype=torch.float32, device=q.device)
    g = torch.empty_like(beta)
    a = _abi.PrepareArgs()
    a.tokens, a.heads, a.d_k, a.dtype = tokens, H, dk, _DTYPES[q.dtype]
    a.q_scale = float(dk) ** 0.5 if q_scale is None else float(q_scale)
    a.q_in, a.k_in, a.q_out, a.k_out = _ptr(q), _ptr(k), _ptr(qo), _ptr(ko)
    a.beta_logit, a.alpha_logit, a.a_log = _ptr(beta_logit), _ptr(alpha_logit), _ptr(a_log)
    a.beta, a.g = _ptr(beta), _ptr(g)
    _abi.check(_abi.lib().rhz_gdr_prepare(byref(a), _stream(stream)))
    return qo, ko, beta, g


def conv_prepare(x, weight, bias, beta_logit, alpha_logit, a_log, *, heads, d_k, d_v, q_scale=None,
                 cu_seqlens=None, initial_state=None, output_final_state=False, q_out=None, k_out=None,
                 v_out=None, stream=None):
    """The Local block's prologue in one pass (rhz_gdr_conv_prepare): causal
    conv1d over x = [q | k | v] projections, then q := l2norm(q) * q_scale
    (default sqrt(d_k)), k := l2norm(k), beta := sigmoid(beta_logit),
    g := -softplus(a_log[h]) * softplus(alpha_logit).

    x [B, T, C] (dense) or [tokens, C] with ``cu_seqlens``, C = heads *
    (2 d_k + d_v); weight [C, 4] fp32; bias [C]; logits [..., heads]; a_log
    [heads]; initial_state [N, C, 3].  Returns (q, k, v, beta, g,
    final_state or None) with q, k [..., heads, d_k] and v [..., heads, d_v].
    """
    if cu_seqlens is None:
        B, T, C = x.shape
        batch, seq_len, lead = B, T, (B, T)
    else:
        seq_len, C = x.shape
        batch, lead = cu_seqlens.numel() - 1, (seq_len,)
    if C != heads * (2 * d_k + d_v):
        raise ValueError(f"x has {C} channels, not heads * (2 d_k + d_v) = {heads * (2 * d_k + d_v)}")
    if tuple(weight.shape) != (C, 4) or weight.dtype != torch.float32:
        raise ValueError("weight must be fp32 [C, 4]")
    q = q_out if q_out is not None else torch.empty(lead + (heads, d_k), dtype=x.dtype, device=x.device)
    k = k_out if k_out is not None else torch.empty(lead + (heads, d_k), dtype=x.dtype, device=x.device)
    v = v_out if v_out is not None else torch.empty(lead + (heads, d_v), dtype=x.dtype, device=x.device)
    beta = torch.empty(lead + (heads,), dtype=torch.float32, device=x.device)
    g = torch.empty_like(beta)
    fin = torch.empty((batch, C, 3), dtype=torch.float32, device=x.device) if output_final_state else None
    a = _abi.ConvPrepareArgs()
    a.batch, a.seq_len, a.heads, a.d_k, a.d_v = batch, seq_len, heads, d_k, d_v
    a.dtype = _DTYPES[x.dtype]
    a.q_scale = float(d_k) ** 0.5 if q_scale is None else float(q_scale)
    a.x, a.weight, a.bias = _ptr(x), _ptr(weight), _ptr(bias)
    a.cu_seqlens, a.initial_state, a.final_state = _ptr(cu_seqlens), _ptr(initial_state), _ptr(fin)
    a.beta_logit, a.alpha_logit, a.a_log = _ptr(beta_logit), _ptr(alpha_logit), _ptr(a_log)
    a.q, a.k, a.v, a.beta, a.g = _ptr(q), _ptr(k), _ptr(v), _ptr(beta), _ptr(g)
    _abi.check(_abi.lib().rhz_gdr_conv_prepare(byref(a), _stream(stream)))
    return q, k, v, beta, g, fin


def rmsnorm_heads(x, scale, eps: float = 1e-6, *, out=None, stream=None):
    """RMSNorm over the last dimension with a learned scale (norm.rs:8-13, 48-59)."""
    dim = x.shape[-1]
    y = out if out is not None else torch.empty_like(x)
    a = _abi.RmsnormArgs()
    a.rows, a.dim, a.dtype, a.eps = x.numel() // dim, dim, _DTYPES[x.dtype], eps
    a.x, a.scale, a.y = _ptr(x), _ptr(scale), _ptr(y)
    _abi.check(_abi.lib().rhz_rmsnorm_heads(byref(a), _stream(stream)))
    return y


_FILL = {"normal": _abi.FILL_NORMAL, "unit_rows": _abi.FILL_UNIT_ROWS,
         "sigmoid": _abi.FILL_SIGMOID, "neg_softplus": _abi.FILL_NEG_SOFTPLUS,
         "uniform": _abi.FILL_UNIFORM}
_FILL_DTYPES = {torch.float64: _abi.F64, torch.float32: _abi.F32, torch.bfloat16: _abi.BF16}


def philox_fill(kind: str, seed: int, stream_id: int, shape, dtype=torch.float32, *,
                mean: float = 0.0, std: float = 1.0, device="cuda", out=None, stream=None):
    """Seeded Philox-4x32-10 synthetic tensor generated on the device (see rhz_philox_fill)."""
    t = out if out is not None else torch.empty(shape, dtype=dtype, device=device)
    row_len = t.shape[-1] if t.dim() else 1
    _abi.check(_abi.lib().rhz_philox_fill(_FILL[kind], seed, stream_id, t.numel(), row_len, mean,
                                          std, _FILL_DTYPES[t.dtype], _ptr(t), _stream(stream)))
    return t


def query_support(op: str, dtype, d_k: int, d_v: int, algo: str = "auto") -> int:
    """rhz_gdr_query_support status for op 'scan', 'step' or 'multistep'."""
    ops = {"scan": _abi.OP_DELTA_SCAN, "step": _abi.OP_DELTA_STEP,
           "multistep": _abi.OP_DELTA_MULTISTEP}
    return _abi.lib().rhz_gdr_query_support(ops[op], _DTYPES[dtype], d_k, d_v, _ALGOS[algo])
