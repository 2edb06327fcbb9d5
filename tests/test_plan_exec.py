"""The plan layer (rhizome_amd/host/rhizome_plan.hpp: crates/plan's graph IR
and arena planner in C++) and the executor over it (rhizome_exec.hpp),
through the C++ test program tests/cpp/test_plan_exec built by
__graft_entry__.build().

Without a GPU: the reference's own graph/arena unit tests, the executor's
plan-time errors, the pure-Python planner oracle (oracle/plan_oracle.py)
pinned by the same reference tests and a hand-computed plan, and the C++
planner equal to that oracle -- every interval and the total -- on 400
seeded random graphs, with the reference's liveness and the executor's.
With a GPU: graphs of DeltaScan / DeltaStep / RmsNorm nodes run through one
device arena, each output against the f64 oracle, and a captured HIP graph
replayed bit-identically.
"""
import os
import subprocess

import pytest

from oracle import plan_oracle as P

BIN = os.path.join(os.environ.get("RHIZOME_TEST_BIN_DIR") or os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                                        "cpp"), "test_plan_exec")


def _run(*args):
    assert os.path.exists(BIN), f"{BIN} is missing: run __graft_entry__.build() (make -C tests/cpp)"
    res = subprocess.run([BIN, *args], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    return res.stdout


# ------------------------------------------------------------ oracle pins
def _chain(n, elems=1024):
    tensors = [(elems, "f32", False)]
    nodes = []
    for i in range(n):
        tensors.append((elems, "f32", False))
        nodes.append(("silu", [i], i + 1))
    return tensors, nodes


def test_oracle_bytes_for():  # dtype.rs:158-162
    assert P.BLOCK["mxfp4"] == 32 and P.bytes_for("bf16", 10) == 20
    assert P.bytes_for("mxfp4", 64) == 34 and P.bytes_for("mxint4", 33) == 19 and P.bytes_for("f64", 3) == 24


def test_oracle_reference_arena_tests():  # arena.rs:162-227
    ivs, total = P.plan(*_chain(8))
    assert total < sum(i[4] for i in ivs)                      # chain_reuses_memory
    assert all(i[3] % 256 == 0 for i in P.plan(*_chain(5))[0])  # offsets_are_aligned
    ivs, _ = P.plan([(16, "f32", False), (4096, "bf16", True), (16, "f32", False)], [("linear", [0, 1], 2)])
    assert all(i[0] != 1 for i in ivs)                         # parameters_are_not_placed_in_the_arena
    t = [(256, "f32", False)] * 4
    ivs, _ = P.plan(t, [("silu", [0], 1), ("silu", [1], 2), ("add", [0, 2], 3)])
    x, b = ivs[0], ivs[2]
    assert not (x[3] < b[3] + b[4] and b[3] < x[3] + x[4])      # long_lived_tensor_does_not_alias
    ivs, _ = P.plan(*_chain(3))
    bad = [(i[0], 0, 10, ivs[0][3], i[4]) for i in ivs]
    with pytest.raises(ValueError):                            # detects_injected_conflicts
        P.verify(bad)


def test_oracle_hand_computed_chain():
    ivs, total = P.plan(*_chain(3))
    assert ivs == [(0, 0, 0, 0, 4096), (1, 0, 1, 4096, 4096), (2, 1, 2, 0, 4096), (3, 2, 2, 4096, 4096)]
    assert total == 8192


def test_oracle_validate():  # graph.rs:252-293
    P.validate([(16, "f32", False), (512, "bf16", True), (32, "f32", False)], [("linear", [0, 1], 2)])
    with pytest.raises(ValueError):
        P.validate([(4, "f32", False)] * 3, [("silu", [2], 1), ("silu", [0], 2)])  # use before define
    with pytest.raises(ValueError):
        P.validate([(4, "f32", False), (4, "f32", True)], [("silu", [0], 1)])      # writes a parameter


# ------------------------------------------------------------ the C++ layer
def test_plan_layer_without_gpu():
    out = _run("--cpu")
    print(out, flush=True)
    for name in ("chain_reuses_memory", "detects_injected_conflicts", "chain3_hand_computed",
                 "boundary_tensors_are_pinned", "compile_layout", "compile_errors"):
        assert f"PASS {name}" in out
    assert "OK: 0 failed" in out


def _parse(text):
    graphs = []
    cur = None
    for line in text.splitlines():
        f = line.split()
        if f[0] == "graph":
            cur = {"tensors": [], "nodes": [], "plans": {}}
            graphs.append(cur)
        elif f[0] == "t":
            cur["tensors"].append((int(f[1]), f[2], f[3] == "1"))
        elif f[0] == "n":
            cur["nodes"].append((int(f[1]), [int(x) for x in f[3:]], int(f[2])))
        elif f[0] == "plan":
            pin = f[1] == "1"
            cur["plans"][pin] = ([], int(f[2]))
        elif f[0] == "i":
            cur["plans"][pin][0].append(tuple(int(x) for x in f[1:]))
    return graphs


def test_planner_matches_oracle():
    graphs = _parse(_run("--dump", "400"))
    assert len(graphs) == 400
    differ_by_pin = 0
    for gi, g in enumerate(graphs):
        for pin in (False, True):
            ivs, total = P.plan(g["tensors"], g["nodes"], pin_boundary=pin)
            assert g["plans"][pin] == (ivs, total), f"graph {gi} pin={pin}"
        differ_by_pin += g["plans"][False] != g["plans"][True]
    assert differ_by_pin > 50  # the two liveness rules are both exercised


@pytest.mark.gpu
def test_executor_on_gpu():
    out = _run()
    print(out, flush=True)
    for name in ("exec_scan_packed_state", "exec_chain_f32", "exec_capture_replay",
                 "exec_unbound_parameter_launches_nothing"):
        assert f"PASS {name}" in out
