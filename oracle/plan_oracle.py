"""Pure-Python restatement of the reference's plan-level IR and arena planner.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the reference for the C++
planner (rhizome_amd/host/rhizome_plan.cpp), never by the product.

  bytes_for   crates/core/src/dtype.rs:32-55   (DType::bits, block_size, bytes_for)
  validate    crates/plan/src/graph.rs:252-293 (Graph::validate)
  plan        crates/plan/src/arena.rs:83-144  (arena::plan)
  verify      crates/plan/src/arena.rs:49-61   (ArenaPlan::verify)

Pins (tests/test_plan_exec.py:43-76): the reference's own arena and graph unit
tests (arena.rs:146-227, graph.rs tests), a hand-computed plan of a
three-node chain, and invariants that fix a wrong placement rule: every pair
of tensors live together is disjoint, offsets are 256-aligned, a chain
reuses memory, parameters are absent, and the total is the end of the
highest interval.

A graph is ``(tensors, nodes)``: tensors a list of ``(elems, dtype,
is_param)`` with dtype a name below, nodes a list of ``(op, inputs,
output)``.  ``plan`` returns ``(intervals, total_bytes)`` with intervals
``(tensor, start, end, offset, size)`` ordered by tensor id.
"""
from __future__ import annotations

ALIGN = 256  # arena.rs:71

# dtype.rs:32-40 bits, 24-29 block size
BITS = {"f64": 64, "f32": 32, "bf16": 16, "f8e4m3": 8, "mxfp4": 4, "mxint4": 4, "i8": 8}
BLOCK = {"mxfp4": 32, "mxint4": 32}
DTYPES = ["f64", "f32", "bf16", "f8e4m3", "mxfp4", "mxint4", "i8"]  # declaration order, dtype.rs:5-20


def bytes_for(dtype: str, n: int) -> int:
    """dtype.rs:44-55: payload bits rounded up to bytes, plus one e8m0 scale
    byte per block for the MX formats."""
    payload = -(-(n * BITS[dtype]) // 8)
    block = BLOCK.get(dtype, 1)
    return payload + -(-n // block) if block > 1 else payload


def validate(tensors, nodes) -> None:
    """graph.rs:252-293; raises ValueError at the first violation."""
    written = {o for _, _, o in nodes}
    live = {i for i, (_, _, p) in enumerate(tensors) if p or i not in written}
    seen = set()
    for idx, (op, ins, out) in enumerate(nodes):
        for i in ins:
            if i not in live:
                raise ValueError(f"node {idx} uses tensor {i} before it is defined")
        if out in seen:
            raise ValueError(f"tensor {out} is written more than once")
        seen.add(out)
        if tensors[out][2]:
            raise ValueError(f"node {idx} writes parameter tensor {out}")
        live.add(out)


def _overlap_time(a, b) -> bool:
    return a[1] <= b[2] and b[1] <= a[2]


def _overlap_mem(a, b) -> bool:
    return a[3] < b[3] + b[4] and b[3] < a[3] + a[4]


def verify(intervals) -> None:
    """arena.rs:49-61."""
    for i, a in enumerate(intervals):
        for b in intervals[i + 1:]:
            if _overlap_time(a, b) and _overlap_mem(a, b):
                raise ValueError(f"tensors {a[0]} and {b[0]} are live together but share arena bytes")


def plan(tensors, nodes, pin_boundary: bool = False):
    """arena.rs:83-144.  pin_boundary: the C++ executor's liveness, in which
    tensors no node writes or no node reads span every node."""
    n = len(tensors)
    start = [None] * n
    end = [0] * n
    used = [False] * n
    read = [False] * n
    written = [False] * n

    def touch(i, idx):
        used[i] = True
        start[i] = idx if start[i] is None else min(start[i], idx)
        end[i] = max(end[i], idx)

    for idx, (_, ins, out) in enumerate(nodes):
        for i in ins:
            if tensors[i][2]:
                continue
            read[i] = True
            touch(i, idx)
        written[out] = True
        touch(out, idx)
    if pin_boundary and nodes:
        for i in range(n):
            if used[i] and (not written[i] or not read[i]):
                start[i], end[i] = 0, len(nodes) - 1

    size_of = [bytes_for(t[1], t[0]) for t in tensors]
    order = sorted((i for i in range(n) if used[i] and not tensors[i][2]), key=lambda i: (-size_of[i], i))
    placed = []
    for i in order:
        size = -(-max(size_of[i], 1) // ALIGN) * ALIGN
        cand = (i, start[i], end[i], 0, size)
        blocks = sorted((p[3], p[3] + p[4]) for p in placed if _overlap_time(p, cand))
        offset = 0
        for lo, hi in blocks:
            if offset + size <= lo:
                break
            offset = max(offset, hi)
        placed.append((i, start[i], end[i], offset, size))
    placed.sort(key=lambda p: p[0])
    total = max((p[3] + p[4] for p in placed), default=0)
    verify(placed)
    return placed, total
