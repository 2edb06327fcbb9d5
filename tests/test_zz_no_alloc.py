"""rhz_gdr_prefill_noalloc: the prefill entry point that allocates nothing.

Its only scratch (a packed batch's longest-first sequence order) is a static
device array shared by every call on a GPU, so two calls in a row -- the
second with fewer sequences -- must each match rhz_gdr_prefill (same kernels,
caller-provided workspace) bit for bit.  A dense batch and the fp32
recurrent path, which use no scratch, must match too.  A call captured in a
HIP graph must match on every replay, with eager noalloc calls that
overwrite the scratch in between; a batch of more than 4096 sequences takes
the identity-order path, and a unit outside the fp16 path's domain takes the
exact rerun through either entry point.  The size limit is checked before any HIP call.
"""
from ctypes import byref

import pytest
import torch

import rhizome_amd
from gdr_cases import Prefill
from rhizome_amd import _abi, gdr


def _noalloc(w, algo):
    """rhz_gdr_prefill_noalloc through the C ABI on workload w."""
    o = torch.empty_like(w.shaped(w.v))
    fin = torch.empty((w.n_seqs, w.heads, w.d_v, w.d_k), dtype=torch.float32, device=w.q.device)
    args = gdr.prefill_args(w.shaped(w.q), w.shaped(w.k), w.shaped(w.v), w.shaped(w.g), w.shaped(w.beta),
                            _abi.GATE_LOG_ALPHA, w.cu_dev, w.init, fin, o, algo)
    stream = torch.cuda.current_stream().cuda_stream or None
    _abi.check(_abi.lib().rhz_gdr_prefill_noalloc(byref(args), stream))
    torch.cuda.synchronize()
    assert rhizome_amd.sync_timeouts() == 0
    return o.reshape(w.n_tok, w.heads, w.d_v), fin


def _noalloc_into(w, o, fin, stream):
    """rhz_gdr_prefill_noalloc on workload w into preallocated o and fin."""
    args = gdr.prefill_args(w.shaped(w.q), w.shaped(w.k), w.shaped(w.v), w.shaped(w.g), w.shaped(w.beta),
                            _abi.GATE_LOG_ALPHA, w.cu_dev, w.init, fin, o, "chunked")
    _abi.check(_abi.lib().rhz_gdr_prefill_noalloc(byref(args), stream))


@pytest.mark.gpu
def test_noalloc_under_graph_capture(device):
    # Defined first in this file, so that (run alone or last) the captured
    # call is normally the process's first noalloc call: the per-device
    # scratch address is then looked up while the stream captures.
    lengths = [int(x) for x in torch.randint(0, 300, (24,), generator=torch.Generator().manual_seed(7))]
    lengths[3] = 0
    w = Prefill(heads=2, d_k=128, d_v=64, lengths=lengths, seed=7, dtype=torch.bfloat16, device=device,
                state_std=0.02)
    o_ref, f_ref = w.run(algo="chunked")  # rhz_gdr_prefill, its own workspace
    o_ref = o_ref.clone()
    f_ref = f_ref.clone()
    o = torch.empty_like(w.shaped(w.v))
    fin = torch.empty((w.n_seqs, w.heads, w.d_v, w.d_k), dtype=torch.float32, device=device)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _noalloc_into(w, o, fin, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for rep in range(3):
        o.fill_(float("nan"))
        fin.fill_(float("nan"))
        # eager work of the program between replays, including a noalloc
        # call on a smaller batch that overwrites the shared scratch
        small = Prefill(heads=1, d_k=32, d_v=32, lengths=[5, 70, 0, 33], seed=rep, dtype=torch.bfloat16,
                        device=device)
        o_s, f_s = _noalloc(small, "chunked")
        o_s2, f_s2 = small.run(algo="chunked")
        assert torch.equal(o_s, o_s2) and torch.equal(f_s, f_s2), f"eager noalloc, replay {rep}"
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert rhizome_amd.sync_timeouts() == 0
        assert torch.equal(o.reshape(w.n_tok, w.heads, w.d_v), o_ref), f"o, replay {rep}"
        assert torch.equal(fin, f_ref), f"final state, replay {rep}"
        print(f"graph replay {rep}: noalloc == prefill, {w.n_seqs} sequences", flush=True)


@pytest.mark.gpu
def test_noalloc_more_sequences_than_the_sort(device):
    # above 4096 packed sequences the order kernel writes the identity order,
    # filling more of the shared scratch than the sorted path does
    lengths = [int(x) for x in torch.randint(0, 6, (5000,), generator=torch.Generator().manual_seed(11))]
    w = Prefill(heads=1, d_k=32, d_v=32, lengths=lengths, seed=11, dtype=torch.bfloat16, device=device,
                state_std=0.02)
    o1, f1 = _noalloc(w, "chunked")
    o2, f2 = w.run(algo="chunked")
    assert torch.equal(o1, o2) and torch.equal(f1, f2)
    print(f"noalloc == prefill, {w.n_seqs} packed sequences, {w.n_tok} tokens", flush=True)


@pytest.mark.gpu
def test_noalloc_matches_prefill_two_calls(device):
    # first call: 40 packed sequences; second: 5 (the shared scratch keeps the
    # first call's order beyond entry 5)
    for n_seqs, seed in ((40, 0), (5, 1)):
        lengths = [int(x) for x in torch.randint(0, 300, (n_seqs,), generator=torch.Generator().manual_seed(seed))]
        lengths[0] = 0
        w = Prefill(heads=3, d_k=128, d_v=128, lengths=lengths, seed=seed, dtype=torch.bfloat16,
                    device=device, state_std=0.02)
        o1, f1 = _noalloc(w, "chunked")
        o2, f2 = w.run(algo="chunked")  # rhz_gdr_prefill with its own workspace
        assert torch.equal(o1, o2) and torch.equal(f1, f2), f"{n_seqs} sequences"
        print(f"noalloc == prefill, {n_seqs} packed sequences, {w.n_tok} tokens", flush=True)


@pytest.mark.gpu
@pytest.mark.parametrize("algo,dtype", [("chunked", torch.bfloat16), ("recurrent", torch.float32)])
def test_noalloc_dense_and_recurrent(device, algo, dtype):
    w = Prefill(batch=2, heads=2, seq_len=150, d_k=64, d_v=64, dtype=dtype, device=device, state_std=0.02)
    o1, f1 = _noalloc(w, algo)
    o2, f2 = w.run(algo=algo)
    assert torch.equal(o1, o2) and torch.equal(f1, f2)


@pytest.mark.gpu
def test_noalloc_exact_rerun(device):
    # a packed batch in which one (sequence, head) leaves the fp16 path's
    # domain (key rows of norm^2 1.2): that unit's two row tiles rerun
    # exactly through either entry point, with identical results
    w = Prefill(heads=2, d_k=64, d_v=64, lengths=[40, 0, 150, 9], seed=3, dtype=torch.bfloat16,
                device=device, state_std=0.02)
    t0, t1 = int(w.cu[2]), int(w.cu[3])
    w.k[t0:t1, 0] = (w.k[t0:t1, 0].double() * 1.2 ** 0.5).to(torch.bfloat16)
    rhizome_amd.exact_reruns(reset=True)
    o1, f1 = _noalloc(w, "chunked")
    assert rhizome_amd.exact_reruns() == 2
    o2, f2 = w.run(algo="chunked", reruns=2)
    assert torch.equal(o1, o2) and torch.equal(f1, f2)


def _gpu_visible() -> bool:
    return torch.cuda.device_count() > 0


@pytest.mark.skipif(_gpu_visible(), reason="fake device addresses: CPU-only validation test")
def test_noalloc_rejects_more_sequences_than_its_scratch():
    A = 0x10000  # aligned fake address: the call must stop before any HIP call
    a = _abi.PrefillArgs()
    a.batch, a.seq_len, a.heads, a.d_k, a.d_v, a.chunk = _abi.NOALLOC_MAX_SEQS + 1, 100, 1, 128, 128, 64
    a.dtype, a.gate_kind, a.algo = _abi.BF16, _abi.GATE_LOG_ALPHA, _abi.ALGO_CHUNKED
    a.q = a.k = a.v = a.gate = a.beta = a.o = a.cu_seqlens = A
    assert _abi.lib().rhz_gdr_prefill_noalloc(byref(a), None) == _abi.ERR_UNSUPPORTED
    assert "at most" in _abi.last_error()
