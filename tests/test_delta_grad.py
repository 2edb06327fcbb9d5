"""The f64 adjoint of the gated delta rule (rhizome_amd/host/rhizome_delta_grad.hpp),
through its C++ test program tests/cpp/test_delta_grad built by
__graft_entry__.build().  CPU only: backward passes stay on the CPU.

Held to central differences of the f64 oracle's forward under the
reference's gradient-check rule (crates/ops/src/gradcheck.rs:33-53, h = 1e-5,
relative error <= 1e-6), and to exact identities: o is linear in v and in q,
a reset cuts every earlier gradient to zero, d g = d alpha * alpha.
"""
import os
import subprocess

BIN = os.path.join(os.environ.get("RHIZOME_TEST_BIN_DIR") or os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                                        "cpp"), "test_delta_grad")


def test_adjoint_gradcheck():
    assert os.path.exists(BIN), f"{BIN} is missing: run __graft_entry__.build() (make -C tests/cpp)"
    res = subprocess.run([BIN], capture_output=True, text=True, timeout=300)
    print(res.stdout, flush=True)
    assert res.returncode == 0, res.stdout + res.stderr
    for name in ("sequential_single_segment", "sequential_with_segments", "sequential_across_windows",
                 "linear_in_v_and_q", "reset_cuts_gradients", "batched_packed_alpha_gate",
                 "batched_log_gate_is_chain_rule", "batched_threads_agree", "batched_equals_one_head"):
        assert f"PASS {name}" in res.stdout
    assert "OK: 0 failed" in res.stdout
