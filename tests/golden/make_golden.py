"""Writes tests/golden/config0.json: a regression fixture of the f64 oracle on
the B=1, H=2, T=64, d_k=d_v=32 workload (seed 0, zero initial state).

The reference (Rust) cannot be built or run in this environment and ships no
golden data, so the fixture records the oracle's own output -- SHA-256 of the
f64 bytes of o [64, 2, 32] and the final state [1, 2, 32, 32], plus a few
values in full precision.  Its trust comes from the oracle tests in
tests/test_oracle.py, not from the reference.

    python tests/golden/make_golden.py
"""
import hashlib
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402


def config0_digest() -> dict:
    raw = O.gdr_inputs(64, 2, 32, 32, seed=0)
    o, fin = O.prefill_batched([0, 64], raw["q"], raw["k"], raw["v"], O.exp_vec(raw["g"]),
                               raw["beta"], None, threads=1)
    return {
        "workload": "B=1 H=2 T=64 d_k=d_v=32 seed 0, f64 inputs, zero initial state",
        "o_sha256": hashlib.sha256(o.tobytes()).hexdigest(),
        "final_sha256": hashlib.sha256(fin.tobytes()).hexdigest(),
        "o[0,0,:4]": [repr(float(x)) for x in o[0, 0, :4]],
        "o[63,1,-4:]": [repr(float(x)) for x in o[63, 1, -4:]],
        "final[0,1,31,-4:]": [repr(float(x)) for x in fin[0, 1, 31, -4:]],
    }


if __name__ == "__main__":
    with open(os.path.join(HERE, "config0.json"), "w") as f:
        json.dump(config0_digest(), f, indent=1)
        f.write("\n")
    print(open(os.path.join(HERE, "config0.json")).read())
