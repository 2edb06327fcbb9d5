"""The chunked prefill kernel's bounded LDS waits report when they give up.

Its waves synchronise through LDS counters; every wait is bounded so that the
kernel always ends, and a wait that gives up is counted on the device
(rhz_gdr_sync_timeouts).  This test forces give-ups from the host with the
test hook rhz_gdr_prefill_spin_limit (one poll per wait: the scan waves'
first wait for chunk 0's staging cannot be met by then), so every kernel
still exits normally, and checks that they are counted; then that a normal
launch right after counts none and matches the oracle.
"""
from ctypes import byref

import pytest
import torch

import rhizome_amd
from gdr_cases import BF16_TOL, Prefill, check_close
from rhizome_amd import _abi, gdr

@pytest.mark.gpu
def test_forced_giveups_are_counted(device):
    rhizome_amd.sync_timeouts(reset=True)
    w = Prefill(batch=1, heads=4, seq_len=512, d_k=128, d_v=128, dtype=torch.bfloat16, device=device)
    o = torch.empty_like(w.v).reshape(1, w.n_tok, w.heads, w.d_v)
    fin = torch.empty((1, w.heads, w.d_v, w.d_k), dtype=torch.float32, device=device)
    args = gdr.prefill_args(w.shaped(w.q), w.shaped(w.k), w.shaped(w.v), w.shaped(w.g), w.shaped(w.beta),
                            _abi.GATE_LOG_ALPHA, None, None, fin, o, "chunked")
    stream = torch.cuda.current_stream().cuda_stream or None
    _abi.check(_abi.lib().rhz_gdr_prefill_spin_limit(byref(args), 1, stream))
    torch.cuda.synchronize()
    n = rhizome_amd.sync_timeouts(reset=True)
    print(f"forced give-ups counted: {n}", flush=True)
    assert n > 0
    # waves that went on without their inputs may have met any values (and
    # so flagged their workgroups for the exact rerun)
    rhizome_amd.fp16_range_errors(reset=True)
    rhizome_amd.exact_reruns(reset=True)
    # the count was reset; a normal launch counts none (checked inside run) and is right
    o2, fin2 = w.run(algo="chunked")
    ref_o, ref_f = w.oracle()
    check_close(o2.float().cpu().numpy(), ref_o, BF16_TOL, "o after forced give-ups")
    check_close(fin2.cpu().numpy(), ref_f, BF16_TOL, "final state after forced give-ups")


def test_spin_limit_hook_validates():
    # runs without a GPU: the bound is checked before anything else
    a = _abi.PrefillArgs()
    assert _abi.lib().rhz_gdr_prefill_spin_limit(byref(a), 0, None) == _abi.ERR_INVALID_ARG
