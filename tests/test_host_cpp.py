"""The C++ restatement of crates/ops/src/delta.rs's API (rhizome_amd/host,
librhizome_ops.so) through its C++ test program tests/cpp/test_delta_host,
built by __graft_entry__.build().  Without a GPU: shapes, state helpers and
the errors thrown before any GPU work; with one: the reference's own unit
tests (delta.rs:282-358) and agreement with the f64 oracle."""
import os
import subprocess

import pytest

BIN = os.path.join(os.environ.get("RHIZOME_TEST_BIN_DIR") or os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                                        "cpp"), "test_delta_host")


def _run(*args):
    assert os.path.exists(BIN), f"{BIN} is missing: run __graft_entry__.build() (make -C tests/cpp)"
    res = subprocess.run([BIN, *args], capture_output=True, text=True, timeout=300)
    print(res.stdout, flush=True)
    assert res.returncode == 0, res.stdout + res.stderr
    return res.stdout


def test_host_api_without_gpu():
    out = _run("--cpu")
    assert "PASS inconsistent_lengths_throw" in out and "OK: 0 failed" in out


@pytest.mark.gpu
def test_host_api_on_gpu():
    out = _run()
    for name in ("chunked_matches_sequential_single_segment", "multistep_matches_repeated_step",
                 "sequential_matches_oracle", "multistep_matches_oracle", "step_matches_oracle"):
        assert f"PASS {name}" in out
