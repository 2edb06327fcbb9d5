"""Pins the CPU f64 oracle (oracle/gdr_oracle.c) before the GPU tests compare against it.

* Philox-4x32-10 against Random123's published known-answer vectors
  (crates/ops/src/rng.rs:43-60 is Random123's philox4x32 with key
  (seed_hi, seed_lo) and counter words [ctr_lo, ctr_hi, stream_lo, stream_hi]).
* The reference's own unit tests: delta.rs:282-369 and rng.rs:113-181.
* Closed forms and invariants of the recurrence, each chosen so that a
  plausible slip (dropped term, wrong sign, transposed state, wrong index)
  fails: pure decay (beta = 0), one-hot overwrite, the d = 1 scalar
  recurrence, linearity, row independence of the rectangular variant,
  chunk-size invariance, segment reset, alpha = 0 reset, non-expansiveness,
  and a dense-matrix brute force of S_t = a S (I - b k k^T) + b v k^T.
"""
import json
import os

import numpy as np
import pytest

from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))


# ------------------------------------------------------------------ Philox
@pytest.mark.parametrize("ctr,key,expect", [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
])
def test_philox_random123_kat(ctr, key, expect):
    counter = ctr[0] | (ctr[1] << 32)
    stream = ctr[2] | (ctr[3] << 32)
    seed = (key[0] << 32) | key[1]
    assert tuple(O.philox_block(seed, stream, counter)) == expect


def test_rng_is_reproducible_and_streams_independent():  # rng.rs:113-133
    assert np.array_equal(O.philox_u32(7, 1, 16), O.philox_u32(7, 1, 16))
    assert not np.array_equal(O.philox_u32(7, 1, 8), O.philox_u32(7, 2, 8))


def test_rng_seek_and_word_order():  # rng.rs:135-145: word 40 = block(10)[0]
    words = O.philox_u32(11, 3, 44)
    assert words[40] == O.philox_block(11, 3, 10)[0]
    assert list(words[4:8]) == O.philox_block(11, 3, 1)


def test_rng_uniform_and_normal():  # rng.rs:78-90, 147-166
    u = O.philox_f64(1, 1, 10000)
    assert np.all((u >= 0) & (u < 1))
    b = O.philox_block(1, 1, 0)
    assert u[0] == ((b[0] >> 5) * 2.0 ** 26 + (b[1] >> 6)) / 2.0 ** 53
    z = O.philox_normal(5, 9, 20000)
    assert abs(z.mean()) < 0.05 and abs(z.var() - 1) < 0.1
    # normal #i is Box-Muller (cosine branch) of block i
    b = O.philox_block(5, 9, 3)
    u1 = ((b[0] >> 5) * 2.0 ** 26 + (b[1] >> 6)) / 2.0 ** 53
    u2 = ((b[2] >> 5) * 2.0 ** 26 + (b[3] >> 6)) / 2.0 ** 53
    assert z[3] == pytest.approx(np.sqrt(-2 * np.log(u1)) * np.cos(2 * np.pi * u2), rel=1e-14)


def test_elementwise():  # elementwise.rs:5-12, 36-42, 125-128
    for x in (-40.0, -3.0, -1e-3, 0.0, 0.5, 7.0, 40.0):
        assert O.sigmoid(x) == pytest.approx(1 / (1 + np.exp(-x)), rel=1e-15)
    assert O.softplus(31.0) == 31.0
    assert O.softplus(2.0) == pytest.approx(np.log1p(np.exp(2.0)), rel=1e-15)
    x = np.array([3.0, 4.0])
    assert np.array_equal(O.l2norm(x, 2.0), np.array([1.2, 1.6]))
    assert np.array_equal(O.l2norm(np.zeros(3)), np.zeros(3))


# ---------------------------------------------- delta.rs unit tests (ported)
def _segs(n):
    return np.zeros(n, dtype=np.uint64)


def test_make_inputs_shapes():  # delta.rs:282-287
    inp = O.make_inputs(4, 3, 1)
    assert inp["q"].size == 12 and inp["alpha"].size == 4 and inp["beta"].size == 4
    q = inp["q"].reshape(4, 3)
    assert np.allclose(np.linalg.norm(q, axis=1), np.sqrt(3))
    assert np.all((inp["alpha"] >= 0.5) & (inp["alpha"] < 1.0))
    assert np.all((inp["beta"] >= 0.1) & (inp["beta"] < 0.9))


def test_chunked_matches_sequential_single_segment():  # delta.rs:289-303
    t, d = 40, 6
    inp = O.make_inputs(t, d, 2)
    args = (inp["q"], inp["k"], inp["v"], inp["alpha"], inp["beta"], _segs(t), np.zeros(d * d))
    a, sa = O.gated_delta_sequential(*args)
    for chunk in (1, 3, 8, 64):
        b, sb = O.gated_delta_scan_chunked(*args, chunk)
        assert np.max(np.abs(a - b)) < 1e-10 and np.max(np.abs(sa - sb)) < 1e-10
        assert np.array_equal(a, b) and np.array_equal(sa, sb)  # same arithmetic, bit for bit


def test_chunked_matches_sequential_with_segments():  # delta.rs:305-317
    d = 4
    segs = np.array([0, 0, 0, 1, 1, 2, 2, 2, 2, 3], dtype=np.uint64)
    inp = O.make_inputs(len(segs), d, 3)
    args = (inp["q"], inp["k"], inp["v"], inp["alpha"], inp["beta"], segs, np.zeros(d * d))
    a, sa = O.gated_delta_sequential(*args)
    b, sb = O.gated_delta_scan_chunked(*args, 4)
    assert np.max(np.abs(a - b)) < 1e-10 and np.max(np.abs(sa - sb)) < 1e-10


def test_multistep_matches_repeated_step():  # delta.rs:319-331
    d, t = 5, 8
    inp = O.make_inputs(t, d, 4)
    args = (inp["q"], inp["k"], inp["v"], inp["alpha"], inp["beta"], _segs(t), np.zeros(d * d))
    outs, states = O.gated_delta_multistep(*args, 8)
    seq, fin = O.gated_delta_sequential(*args)
    assert np.max(np.abs(outs - seq)) < 1e-12
    assert np.max(np.abs(states[t - 1] - fin)) < 1e-12
    # o_t = S_t q_t for every returned state
    q = inp["q"].reshape(t, d)
    for i in range(t):
        assert np.allclose(states[i].reshape(d, d) @ q[i], outs.reshape(t, d)[i], atol=1e-13)
    o3, s3 = O.gated_delta_multistep(*args, 3)
    assert s3.shape == (3, d * d) and np.array_equal(o3, outs[:3 * d])


def test_segment_reset_makes_history_irrelevant():  # delta.rs:333-346
    d = 3
    segs = np.array([0, 0, 1, 1], dtype=np.uint64)
    inp = O.make_inputs(4, d, 5)
    base = (inp["q"], inp["k"], inp["v"], inp["alpha"], inp["beta"], segs)
    a, _ = O.gated_delta_sequential(*base, np.zeros(d * d))
    b, _ = O.gated_delta_sequential(*base, np.full(d * d, 3.0))
    assert np.max(np.abs(a[2 * d:] - b[2 * d:])) < 1e-12
    # the reference also resets at t = 0 (delta.rs:137-141): init never matters
    assert np.array_equal(a, b)


def test_alpha_zero_forgets_the_past():  # delta.rs:348-358
    s = np.ones(9)
    o = O.gated_delta_step(s, [1.0, 1.0, 1.0], [1.0, 0.0, 0.0], [0.0, 0.0, 0.0], 0.0, 0.5)
    assert np.all(np.abs(o) < 1e-12)


def test_conv_state_shifts():  # delta.rs:360-369
    st = np.zeros(3)
    w = [0.1, 0.2, 0.3, 0.4]
    assert abs(O.causal_conv1d_step(st, w, 1.0, 0.0) - 0.4) < 1e-12
    assert abs(O.causal_conv1d_step(st, w, 1.0, 0.0) - 0.7) < 1e-12
    assert list(st) == [0.0, 1.0, 1.0]


# ------------------------------------------------- closed forms / invariants
def _rand_unit(rng, t, d):
    x = rng.standard_normal((t, d))
    return x / np.linalg.norm(x, axis=1, keepdims=True)


def _brute(q, k, v, a, b, s0):
    """S_t = a S (I - b k k^T) + b v k^T, o_t = S_t q_t with dense matrices."""
    s = s0.copy()
    out = []
    dk = k.shape[1]
    for t in range(len(a)):
        s = a[t] * s @ (np.eye(dk) - b[t] * np.outer(k[t], k[t])) + b[t] * np.outer(v[t], k[t])
        out.append(s @ q[t])
    return np.array(out), s


@pytest.mark.parametrize("dk,dv", [(4, 4), (3, 7), (8, 2)])
def test_brute_force_dense(dk, dv):
    rng = np.random.default_rng(1)
    t = 12
    q, k = _rand_unit(rng, t, dk), _rand_unit(rng, t, dk)
    v = rng.standard_normal((t, dv))
    a, b = rng.uniform(0.3, 1.0, t), rng.uniform(0.0, 1.0, t)
    s0 = rng.standard_normal((dv, dk))
    ref_o, ref_s = _brute(q, k, v, a, b, s0)
    s = s0.copy()
    o = O.steps_rect(q, k, v, a, b, s)
    assert np.allclose(o, ref_o, rtol=1e-12, atol=1e-12)
    assert np.allclose(s, ref_s, rtol=1e-12, atol=1e-12)
    # the batched packed entry point runs the same loop
    o2, f2 = O.prefill_batched([0, t], q[:, None], k[:, None], v[:, None], a[:, None],
                               b[:, None], s0[None, None])
    assert np.array_equal(o2[:, 0], o) and np.array_equal(f2[0, 0], s)


def test_beta_zero_is_pure_decay():
    rng = np.random.default_rng(2)
    t, d = 10, 5
    q, k, v = _rand_unit(rng, t, d), _rand_unit(rng, t, d), rng.standard_normal((t, d))
    a = rng.uniform(0.5, 1.0, t)
    s0 = rng.standard_normal((d, d))
    s = s0.copy()
    o = O.steps_rect(q, k, v, a, np.zeros(t), s)
    gam = np.cumprod(a)
    assert np.allclose(s, gam[-1] * s0, rtol=1e-13)
    assert np.allclose(o, gam[:, None] * (q @ s0.T), rtol=1e-12, atol=1e-14)


def test_one_hot_key_overwrites_a_column():
    rng = np.random.default_rng(3)
    d = 6
    s0 = rng.standard_normal((d, d))
    s = s0.copy().reshape(-1)
    v = rng.standard_normal(d)
    e2 = np.eye(d)[2]
    O.gated_delta_step(s, np.ones(d), e2, v, 1.0, 1.0)
    s = s.reshape(d, d)
    assert np.array_equal(s[:, 2], v)
    keep = [j for j in range(d) if j != 2]
    assert np.array_equal(s[:, keep], s0[:, keep])


def test_scalar_recurrence_d1():
    rng = np.random.default_rng(4)
    t = 30
    k = rng.choice([-1.0, 1.0], t)
    q, v = rng.standard_normal(t), rng.standard_normal(t)
    a, b = rng.uniform(0.2, 1.0, t), rng.uniform(0.0, 1.0, t)
    s, ref = np.zeros((1, 1)), []
    x = 0.0
    for i in range(t):
        x = a[i] * (1 - b[i]) * x + b[i] * v[i] * k[i]
        ref.append(x * q[i])
    o = O.steps_rect(q[:, None], k[:, None], v[:, None], a, b, s)
    assert np.allclose(o[:, 0], ref, rtol=1e-13, atol=1e-15)


def test_linearity_in_v_and_q():
    rng = np.random.default_rng(5)
    t, d = 16, 6
    q1, q2, k = _rand_unit(rng, t, d), _rand_unit(rng, t, d), _rand_unit(rng, t, d)
    v1, v2 = rng.standard_normal((t, d)), rng.standard_normal((t, d))
    a, b = rng.uniform(0.5, 1.0, t), rng.uniform(0.1, 0.9, t)
    run = lambda q, v: O.steps_rect(q, k, v, a, b, np.zeros((d, d)))  # noqa: E731
    assert np.allclose(run(q1, v1 + 2 * v2), run(q1, v1) + 2 * run(q1, v2), atol=1e-12)
    assert np.allclose(run(q1 + q2, v1), run(q1, v1) + run(q2, v1), atol=1e-12)


def test_rows_are_independent():
    """A d_v = 2d state equals two d x d runs on the halves of v, bit for bit
    (this pins the rectangular oracle to the square reference step)."""
    inp = O.make_inputs(20, 4, 7)
    q, k = inp["q"].reshape(20, 4), inp["k"].reshape(20, 4)
    rng = np.random.default_rng(6)
    v = rng.standard_normal((20, 8))
    s = np.zeros((8, 4))
    o = O.steps_rect(q, k, v, inp["alpha"], inp["beta"], s)
    for half in range(2):
        vh = v[:, 4 * half:4 * half + 4]
        ref, fin = O.gated_delta_sequential(inp["q"], inp["k"], vh, inp["alpha"], inp["beta"],
                                            _segs(20), np.zeros(16))
        assert np.array_equal(o[:, 4 * half:4 * half + 4].reshape(-1), ref)
        assert np.array_equal(s[4 * half:4 * half + 4].reshape(-1), fin)


def test_alpha_zero_is_a_reset():
    inp = O.make_inputs(12, 5, 8)
    a = inp["alpha"].copy()
    a[6] = 0.0
    q, k, v = (inp[x].reshape(12, 5) for x in ("q", "k", "v"))
    s = np.full((5, 5), 2.0)
    o = O.steps_rect(q, k, v, a, inp["beta"], s)
    s2 = np.zeros((5, 5))
    o2 = O.steps_rect(q[6:], k[6:], v[6:], a[6:], inp["beta"][6:], s2)
    assert np.array_equal(o[6:], o2) and np.array_equal(s, s2)


def test_state_is_non_expansive():
    rng = np.random.default_rng(9)
    d = 8
    s = rng.standard_normal((d, d))
    k = _rand_unit(rng, 50, d)
    prev = np.linalg.norm(s, 2)
    for t in range(50):
        O.steps_rect(k[t:t + 1], k[t:t + 1], np.zeros((1, d)), [rng.uniform(0.5, 1.0)],
                     [rng.uniform(0, 1)], s)
        cur = np.linalg.norm(s, 2)
        assert cur <= prev * (1 + 1e-12)
        prev = cur


def test_init_honouring_loop_matches_reference_without_reset():
    """steps_rect == gated_delta_step looped (delta.rs:94-127), init kept."""
    inp = O.make_inputs(9, 4, 10)
    s_ref = np.linspace(-1, 1, 16)
    outs = []
    for t in range(9):
        outs.append(O.gated_delta_step(s_ref, inp["q"][4 * t:4 * t + 4], inp["k"][4 * t:4 * t + 4],
                                       inp["v"][4 * t:4 * t + 4], inp["alpha"][t], inp["beta"][t]))
    s = np.linspace(-1, 1, 16).reshape(4, 4)
    o = O.steps_rect(inp["q"].reshape(9, 4), inp["k"].reshape(9, 4), inp["v"].reshape(9, 4),
                     inp["alpha"], inp["beta"], s)
    assert np.array_equal(o, np.array(outs)) and np.array_equal(s.reshape(-1), s_ref)


# --------------------------------------------------- workload input builders
def test_config_inputs():
    raw = O.gdr_inputs(50, 3, 16, 8, seed=0, g_mean=-2.0, n_state=2)
    assert np.allclose(np.linalg.norm(raw["q"], axis=-1), 1.0)
    assert np.allclose(np.linalg.norm(raw["k"], axis=-1), 1.0)
    assert np.all((raw["beta"] > 0) & (raw["beta"] < 1)) and np.all(raw["g"] < 0)
    z = O.philox_normal(0, O.STREAM["g"], 150, -2.0)
    assert np.array_equal(raw["g"].reshape(-1), O.neg_softplus_vec(z))
    assert raw["state"].shape == (2, 3, 8, 16) and abs(raw["state"].std() - 0.02) < 0.005
    lens = O.varlen_lengths(0, 64)
    assert lens.min() >= 128 and lens.max() <= 8192


def test_golden_config0():
    """Regression fixture: the oracle's config-0 outputs (tests/golden/make_golden.py)."""
    from golden.make_golden import config0_digest

    with open(os.path.join(HERE, "golden", "config0.json")) as f:
        gold = json.load(f)
    assert config0_digest() == gold


# ------------------------------------------------- prologue / epilogue pins
def test_conv1d_batched_matches_reference_kat_and_step():
    # delta.rs:360-369: w = [0.1, 0.2, 0.3, 0.4], x = 1 -> 0.4, 0.7; state [0, 1, 1]
    y, fin = O.conv1d_batched([0, 2], np.ones((2, 1)), np.array([[0.1, 0.2, 0.3, 0.4]]))
    assert abs(y[0, 0] - 0.4) < 1e-12 and abs(y[1, 0] - 0.7) < 1e-12
    assert np.array_equal(fin[0, 0], [0.0, 1.0, 1.0])


def test_conv1d_batched_against_dense_convolution():
    """Brute force: each sequence and channel is a full convolution of
    (initial state ++ x) with the reversed weights."""
    rng = np.random.default_rng(3)
    C = 5
    cu = np.array([0, 7, 7, 8, 20])
    x = rng.normal(size=(cu[-1], C))
    w = rng.normal(size=(C, 4))
    b = rng.normal(size=C)
    init = rng.normal(size=(4, C, 3))
    y, fin = O.conv1d_batched(cu, x, w, b, init)
    for s in range(4):
        for c in range(C):
            seq = np.concatenate([init[s, c], x[cu[s]:cu[s + 1], c]])
            for t in range(cu[s], cu[s + 1]):
                i = t - cu[s] + 3
                ref = seq[i - 3] * w[c, 0] + seq[i - 2] * w[c, 1] + seq[i - 1] * w[c, 2] + seq[i] * w[c, 3] + b[c]
                assert abs(y[t, c] - ref) < 1e-12
            assert np.allclose(fin[s, c], seq[-3:], rtol=0, atol=0)


def test_conv1d_shift_and_identity_weights():
    x = np.arange(1.0, 11.0).reshape(10, 1)
    y, _ = O.conv1d_batched([0, 4, 10], x, np.array([[0.0, 0.0, 1.0, 0.0]]))  # y_t = x_{t-1}
    assert np.array_equal(y[:, 0], [0, 1, 2, 3, 0, 5, 6, 7, 8, 9])  # reset at the second start
    y, _ = O.conv1d_batched([0, 10], x, np.array([[0.0, 0.0, 0.0, 1.0]]), np.array([0.5]))
    assert np.array_equal(y[:, 0], x[:, 0] + 0.5)


def test_rmsnorm_rows():
    # norm.rs:117-123: heads are normalised independently
    y = O.rmsnorm_rows(np.array([[1.0, 1.0], [100.0, 100.0]]), np.ones(2), 1e-12)
    assert abs(y[0, 0] - y[1, 0]) < 1e-6
    rng = np.random.default_rng(4)
    x = rng.normal(size=(6, 9))
    s = rng.normal(size=9)
    y = O.rmsnorm_rows(x, s, 0.0)
    assert np.allclose(O.rmsnorm_rows(3.7 * x, s, 0.0), y, rtol=1e-13, atol=0)  # scale invariant
    assert np.allclose(np.sqrt(np.mean((y / s) ** 2, axis=1)), 1.0, rtol=1e-13)  # unit RMS
    assert np.allclose(O.rmsnorm_rows(np.full((1, 4), -2.0), np.arange(1.0, 5.0), 0.0), -np.arange(1.0, 5.0))


def test_prepare():
    q, k, beta, g = O.prepare(np.array([[[3.0, 4.0]]]), np.array([[[0.0, -5.0]]]),
                              np.array([[0.0]]), np.array([[0.0]]), np.array([0.0]), 2.0)
    assert np.allclose(q, [[[1.2, 1.6]]], rtol=0, atol=1e-15)  # elementwise.rs:224-227
    assert np.allclose(k, [[[0.0, -1.0]]], rtol=0, atol=1e-15)
    assert beta[0, 0] == 0.5
    assert abs(g[0, 0] + np.log(2.0) ** 2) < 1e-15
    rng = np.random.default_rng(5)
    z = rng.normal(scale=4, size=(7, 3))
    a = rng.normal(size=3)
    _, _, beta, g = O.prepare(np.ones((7, 3, 2)), np.ones((7, 3, 2)), z, z, a, 1.0)
    assert np.allclose(beta, 1 / (1 + np.exp(-z)), rtol=1e-14)
    assert np.allclose(g, -np.log1p(np.exp(a))[None, :] * np.log1p(np.exp(z)), rtol=1e-12)
    _, _, b2, g2 = O.prepare(np.ones((1, 1, 2)), np.ones((1, 1, 2)), np.array([[-1000.0]]),
                             np.array([[40.0]]), np.array([35.0]), 1.0)
    assert 0.0 <= b2[0, 0] < 1e-300  # elementwise.rs:151-153
    assert g2[0, 0] == -35.0 * 40.0  # softplus is linear above 30
