"""A model of the split-wave prefill schedule (varlen_prefill_ws_kernel), checked on the CPU.

In varlen_prefill_ws_kernel the S waves (QK^T + softmax) and the O waves (PV) of a workgroup
run separate loops over the same barrier sequence.  Each iteration i (after barrier B(i)):
the S waves read K of step i and write P(i) into buffer i % 2; the O waves read P(i - 1) and
V of step i - 1; then every wave runs the ring upkeep: the loaders issue step i + NS - 2 into
its slot, clear the V rows of step i + 1 where needed, and wait (an exact vmcnt count) for
step i + 2.  This model replays that schedule as barrier intervals and checks what the
hardware does not: every K/V read comes after its step's loads landed and were published by
a barrier, from the slot that holds that step; no load or clear shares an interval with a read
of its slot; V rows are cleared before they are read; P is read one interval after it was
written, from the buffer written last, and no write of a buffer shares an interval with a
read of it; each wait count is exact; the O waves' output planes are neither read in the last
interval nor loaded.  A plausible slip fails one of the checks (test_model_catches_slips).
"""
import random

import pytest


class SplitRing:
    def __init__(self, nsteps, ns, vzero, wait_slip=0, stage_slip=0, p_lag=1, clear_lead=1):
        self.n, self.ns, self.vzero = nsteps, ns, vzero
        self.wait_slip, self.stage_slip = wait_slip, stage_slip
        self.p_lag, self.clear_lead = p_lag, clear_lead
        self.interval = 0
        self.issued = []          # steps in load-issue order (each loader's own queue)
        self.published = {}       # step -> first interval in which its loads are visible
        self.cleared = {}
        self.writes = []          # (interval, slot, step, what)
        self.reads = []           # (interval, slot, step, plane)
        self.p_writes = []        # (interval, buffer, step)
        self.p_reads = []         # (interval, buffer, step)

    def stage(self, x):
        self.writes.append((self.interval, x % self.ns, x, "load"))
        self.issued.append(x)

    def wait(self, later):
        later += self.wait_slip
        done = self.issued[:len(self.issued) - later] if later > 0 else list(self.issued)
        for x in done:
            self.published.setdefault(x, self.interval + 1)

    def expect_later(self, need, later):
        assert need in self.issued, f"wait for step {need}, which was never issued"
        assert self.issued.index(need) == len(self.issued) - 1 - later, \
            f"wait for step {need} leaves {later} steps out, issued {self.issued}"

    def barrier(self):
        self.interval += 1

    def clear(self, x):
        assert self.published.get(x, 1 << 30) <= self.interval, f"clear of step {x} before its loads"
        self.cleared[x] = self.interval
        self.writes.append((self.interval, x % self.ns, x, "clear"))

    def read(self, x, plane):
        self.reads.append((self.interval, x % self.ns, x, plane))

    def upkeep(self, i):
        n, ns = self.n, self.ns
        x = i + ns - 2 - self.stage_slip
        if 0 <= x < n:
            self.stage(x)
        c = i + self.clear_lead
        if 0 < c < n and self.vzero[c]:
            self.clear(c)
        if i + 2 < n:
            last = min(i + ns - 2, n - 1)
            self.expect_later(i + 2, last - (i + 2))
            self.wait(last - (i + 2))

    def run(self):
        n, ns = self.n, self.ns
        self.barrier()                              # B_start: previous tile retired
        first = min(n - 1, ns - 3)
        for x in range(first + 1):
            self.stage(x)
        self.expect_later(0, first)
        self.wait(first)
        self.barrier()                              # B(-1): step 0 published
        if self.vzero[0]:
            self.clear(0)
        if n > 1:
            self.expect_later(1, first - 1)
            self.wait(first - 1)
        for i in range(n + 1):
            self.barrier()                          # B(i)
            if i < n:                               # S waves
                self.read(i, "K")
                self.p_writes.append((self.interval, i % 2, i))
            j = i - self.p_lag
            if 0 <= j < n and i >= 1:               # O waves
                self.p_reads.append((self.interval, j % 2, j))
                self.read(j, "V")
            self.upkeep(i)
        return self

    def check(self):
        n = self.n
        assert sorted(self.issued) == list(range(n)), f"issued {self.issued}"
        assert sorted(s for _, _, s in self.p_reads) == list(range(n)), "a step's PV is missing"
        for (iv, slot, x, plane) in self.reads:
            earlier = [w for w in self.writes if w[1] == slot and w[3] == "load" and w[0] < iv]
            assert earlier and earlier[-1][2] == x, f"{plane} of step {x} read from a stale slot"
            assert self.published.get(x, 1 << 30) <= iv, f"{plane} of step {x} read before publish"
            if plane == "V" and self.vzero[x]:
                assert self.cleared.get(x, 1 << 30) < iv, f"V of step {x} read before its clear"
        for (iv, slot, x, what) in self.writes:
            for (riv, rslot, y, plane) in self.reads:
                if riv == iv and rslot == slot and (what == "load" or plane == "V"):
                    raise AssertionError(f"{what} of step {x} races a {plane} read of step {y}")
        for (iv, buf, x) in self.p_reads:
            before = [w for w in self.p_writes if w[1] == buf and w[0] < iv]
            assert before and before[-1][2] == x, f"P of step {x} read from a stale buffer"
            for (wiv, wbuf, y) in self.p_writes:
                assert not (wiv == iv and wbuf == buf), f"P({y}) written while P({x}) is read"
        return self


def output_plane(pair, nsteps, ns):
    """The epilogue's choice: the K plane of slot `pair`, else a V plane after step n - 1's."""
    return (pair, "K") if pair < ns else ((nsteps + pair - ns) % ns, "V")


def cases(seed=1):
    rnd = random.Random(seed)
    for ns in (6, 7, 8):
        for n in range(1, 41):
            pats = [[False] * (n - 1) + [last] for last in (False, True)]
            pats += [[rnd.random() < 0.2 for _ in range(n)] for _ in range(10)]
            for vz in pats:
                yield ns, n, vz


@pytest.mark.parametrize("ns", [6, 7, 8])
def test_split_schedule_orders_every_access(ns):
    count = 0
    for r_ns, n, vz in cases():
        if r_ns != ns:
            continue
        ring = SplitRing(n, ns, vz).run().check()
        last = {(slot, plane) for (iv, slot, x, plane) in ring.reads if iv == ring.interval}
        loads_late = {(slot, "K") for (iv, slot, x, w) in ring.writes if w == "load"
                      and ring.published.get(x, 1 << 30) > ring.interval}
        planes = [output_plane(p, n, ns) for p in range(8)]
        assert len(set(planes)) == 8
        assert not set(planes) & last, (n, planes, last)
        assert not loads_late
        count += 1
    assert count > 300


def test_model_catches_slips():
    def fails(**kw):
        for ns, n, vz in cases(seed=2):
            try:
                SplitRing(n, ns, vz, **kw).run().check()
            except AssertionError:
                return True
        return False
    assert fails(wait_slip=1), "a wait that leaves one step too many out"
    assert fails(stage_slip=-1), "a slot refilled one step early"
    assert fails(p_lag=0), "PV of a step in the interval its P is written"
    assert fails(clear_lead=-1), "V rows cleared in the interval they are read"
