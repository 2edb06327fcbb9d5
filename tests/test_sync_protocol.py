"""Randomized-interleaving check of the chunked prefill kernel's LDS-counter
protocol (rhizome_amd/csrc/gdr_chunked.hip), on the CPU.

The kernel has no workgroup barrier inside its chunk loop: each role waits
for LDS completion counters and signals its own.  This test models every role
as a sequence of steps (wait condition, then the LDS buffers the step reads
and writes) with the kernel's exact wait targets, and runs the roles in
random interleavings.  A step's reads are checked when it starts and when it
ends, so that a buffer overwritten while a reader is still in it is caught,
and writes land when the step ends.  It asserts:

* no deadlock: whenever no step can start or end, every role has finished;
* no stale or overwritten read: every read of a double-buffered (or single)
  LDS buffer sees the chunk the reader expects.

Roles and their kernel functions:
  loader L (4 waves)  prep_loader: wait {scanned[0..1] >= x-1, pdone >= 3(x-1),
                      pdone3 >= x-1, tdiag >= x-1, aoff >= x-1}, stage
                      K/Q/beta V/gates of x into buffer x&1, signal staged;
                      wait staged >= 4(x+1); loaders 0-2 then form Q K^T's
                      block rows -> P[x&1], signal pdone (the gate loader, 3,
                      has no Q K^T share, but waits all the same: without
                      that wait it could stage x+1 before the others staged
                      x, and staged >= 4(x+1) would then not mean that all
                      four staged x, the planted mistake
                      "gate_loader_runs_ahead")
  wave 2              prep_wave2: wait {staged >= 4(x+1), scanned >= x-1,
                      tfull >= 2(x-1)}, K K^T diagonal -> A diag, T diagonal
                      blocks, signal tdiag; wait aoff >= x+1, T blocks, signal tfull
  wave 3              prep_wave3: wait {staged >= 4(x+1), tfull >= 2x}, A below
                      the diagonal, signal aoff; Q K^T's last block row ->
                      P[x&1], signal pdone3; wait tdiag >= x+1, T blocks,
                      signal tfull
  scan s (2 waves)    scan_chunk: wait staged >= 4(c+1), read K, Q, beta V,
                      gates; wait {tfull >= 2(c+1), pdone >= 3(c+1),
                      pdone3 >= c+1}, read T, P, K^T, gates, signal scanned[s]

P's last block row, formed by wave 3, has a counter of its own (pdone3), so
that each counter counts one kind of step.

The planted mistakes at the end (each a wait target the kernel does NOT
have) must be caught, which shows that the model can see a broken protocol.
"""
import random

import pytest


def _roles(nch, cnt, rd, wr, mistake=None):
    def loader(L):
        steps = []
        for x in range(nch):
            b = x & 1

            def w_stage(x=x):
                pd = cnt["pdone"] >= 3 * (x - 1) and cnt["pdone3"] >= x - 1
                if mistake == "loader_ignores_scan":
                    return x < 2 or (pd and cnt["tdiag"] >= x - 1 and cnt["aoff"] >= x - 1)
                return x < 2 or (min(cnt["scanned0"], cnt["scanned1"]) >= x - 1
                                 and pd and cnt["tdiag"] >= x - 1 and cnt["aoff"] >= x - 1)

            def e_stage(x=x, b=b):
                for nm in ("k", "q", "vb", "g"):
                    wr(nm + str(L), b, x)  # each loader writes its quarter
                cnt["staged"] += 1

            steps.append((w_stage, lambda: None, e_stage))

            def w_qk(x=x):
                if mistake == "gate_loader_runs_ahead" and L == 3:
                    return True
                return cnt["staged"] >= 4 * (x + 1)

            if L == 3:  # the gate loader has no Q K^T share; it only waits
                steps.append((w_qk, lambda: None, lambda: None))
                continue

            def s_qk(x=x, b=b):
                for LL in range(4):
                    for nm in ("k", "q", "g"):
                        rd(nm + str(LL), b, x)

            def e_qk(x=x, b=b):
                s_qk(x, b)
                wr("p" + str(L), b, x)
                cnt["pdone"] += 1

            steps.append((w_qk, s_qk, e_qk))
        return steps

    def all_k(b, x):
        for LL in range(4):
            for nm in ("k", "g"):
                rd(nm + str(LL), b, x)

    def wave2():
        steps = []
        for x in range(nch):
            b = x & 1

            def w1(x=x):
                return cnt["staged"] >= 4 * (x + 1) and (
                    x < 2 or (min(cnt["scanned0"], cnt["scanned1"]) >= x - 1 and cnt["tfull"] >= 2 * (x - 1)))

            def e1(x=x, b=b):
                all_k(b, x)
                wr("ad", 0, x)
                wr("tdiag", b, x)
                cnt["tdiag"] += 1

            steps.append((w1, lambda x=x, b=b: all_k(b, x), e1))

            def w2(x=x):
                return cnt["aoff"] >= (x + 1 if mistake != "wave2_ignores_aoff" else 0)

            def s2(x=x, b=b):
                rd("a", 0, x)
                rd("tdiag", b, x)
                rd("ad", 0, x)

            def e2(x=x, b=b):
                s2(x, b)
                wr("toff2", b, x)
                cnt["tfull"] += 1

            steps.append((w2, s2, e2))
        return steps

    def wave3():
        steps = []
        for x in range(nch):
            b = x & 1

            def w1(x=x):
                tf = 2 * x if mistake != "wave3_early" else 2 * x - 1
                return cnt["staged"] >= 4 * (x + 1) and cnt["tfull"] >= tf

            def e1(x=x, b=b):
                all_k(b, x)
                wr("a", 0, x)
                cnt["aoff"] += 1

            steps.append((w1, lambda x=x, b=b: all_k(b, x), e1))

            def s_qk(x=x, b=b):
                for LL in range(4):
                    for nm in ("k", "q", "g"):
                        rd(nm + str(LL), b, x)

            def e_qk(x=x, b=b):
                s_qk(x, b)
                wr("p3", b, x)
                cnt["pdone3"] += 1

            steps.append((lambda: True, s_qk, e_qk))

            def w2(x=x):
                return cnt["tdiag"] >= x + 1

            def s2(x=x, b=b):
                rd("a", 0, x)
                rd("tdiag", b, x)

            def e2(x=x, b=b):
                s2(x, b)
                wr("toff3", b, x)
                cnt["tfull"] += 1

            steps.append((w2, s2, e2))
        return steps

    def scan(sid):
        steps = []
        for c in range(nch):
            b = c & 1

            def wA(c=c):
                return cnt["staged"] >= 4 * (c + 1)

            def sA(c=c, b=b):
                for LL in range(4):
                    for nm in ("k", "q", "vb", "g"):
                        rd(nm + str(LL), b, c)

            steps.append((wA, sA, sA))

            def wB(c=c):
                if mistake == "scan_ignores_pdone":
                    return cnt["tfull"] >= 2 * (c + 1)
                return (cnt["tfull"] >= 2 * (c + 1) and cnt["pdone"] >= 3 * (c + 1)
                        and cnt["pdone3"] >= c + 1)

            def sB(c=c, b=b):
                for nm in ("tdiag", "toff2", "toff3"):
                    rd(nm, b, c)
                for LL in range(4):
                    rd("p" + str(LL), b, c)
                    rd("k" + str(LL), b, c)
                    rd("g" + str(LL), b, c)

            def eB(c=c, b=b, sid=sid):
                sB(c, b)
                cnt["scanned%d" % sid] += 1

            steps.append((wB, sB, eB))
        return steps

    roles = {"L%d" % L: loader(L) for L in range(4)}
    roles.update(w2=wave2(), w3=wave3(), s0=scan(0), s1=scan(1))
    return roles


class ProtocolError(AssertionError):
    pass


def simulate(nch, seed, mistake=None):
    rng = random.Random(seed)
    cnt = dict(staged=0, tdiag=0, aoff=0, tfull=0, pdone=0, pdone3=0, scanned0=0, scanned1=0)
    buf = {}  # (buffer, index) -> chunk whose data it holds

    def rd(name, idx, x):
        if buf.get((name, idx)) != x:
            raise ProtocolError(f"nch={nch} seed={seed}: read {name}[{idx}] expected chunk {x}, "
                                f"found {buf.get((name, idx))}")

    def wr(name, idx, x):
        buf[(name, idx)] = x

    roles = _roles(nch, cnt, rd, wr, mistake)
    pc = {r: 0 for r in roles}  # next step of each role
    inflight = {}               # role -> step started and not ended
    while True:
        choices = []
        for r, steps in roles.items():
            if r in inflight:
                choices.append(("end", r))
            elif pc[r] < len(steps) and steps[pc[r]][0]():
                choices.append(("start", r))
        if not choices:
            if not (all(pc[r] == len(roles[r]) for r in roles) and not inflight):
                raise ProtocolError(f"deadlock nch={nch} seed={seed} pc={pc} cnt={cnt}")
            return
        kind, r = rng.choice(choices)
        if kind == "start":
            roles[r][pc[r]][1]()
            inflight[r] = pc[r]
        else:
            roles[r][inflight.pop(r)][2]()
            pc[r] += 1


@pytest.mark.parametrize("nch", range(0, 8))
def test_protocol_no_deadlock_no_stale_read(nch):
    for seed in range(300):
        simulate(nch, seed)


# Wave 2's first wait has targets that the model shows to be implied: its
# staged >= 4(x+1) target already implies scanned >= x-1 (the loaders waited
# for it before staging x), which implies tfull >= 2(x-1) (a scan counts chunk
# x-2 only after T of x-2 is complete).  Dropping them is therefore no mistake
# and none is planted there.
@pytest.mark.parametrize("mistake", ["loader_ignores_scan", "wave2_ignores_aoff", "wave3_early",
                                     "scan_ignores_pdone", "gate_loader_runs_ahead"])
def test_planted_mistakes_are_caught(mistake):
    caught = 0
    for seed in range(300):
        try:
            simulate(6, seed, mistake)
        except ProtocolError:
            caught += 1
    assert caught > 0, f"the model did not catch the planted mistake {mistake}"
