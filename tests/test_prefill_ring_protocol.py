"""A model of the LDS ring schedule of needle_amd/csrc/varlen_prefill.hip, checked on the CPU.

The kernel stages 32-key steps into an NS-slot LDS ring with direct loads, publishes them with
workgroup barriers (one per two steps where it can) and waits for its own loads with vmcnt
counts that must equal the number of steps issued after the one it needs.  This model replays
the kernel's schedule -- the prologue, the steady-state trips, the general trips (paired, or
split when the second step has V rows to clear) and the odd last step -- as a sequence of
barrier intervals, and checks what the hardware does not: every read of a slot happens after
the loads of that step landed and were published by a barrier, no write (load or clear) to a
slot shares a barrier interval with a read of it, every V read of a step that needs clearing
comes after the clear, each wait count is exact, and each wave's output plane is one that no
wave reads after the tile's last barrier.  Changing the schedule in the kernel means changing
it here too; a plausible slip (a wait one step short, a slot refilled one step early, the odd
last step without its barrier) fails one of the checks (see test_model_catches_slips).

The tile prologue is the kernel's: after the barrier that retires the previous tile's reads,
steps 0 and 1 are staged, each wave stages its 32 Q rows into one plane of slots 2 .. 5 (wave
w: slot 2 + w // 2, the K plane for even w, else the V plane), waits for all its loads, reads
its Q plane back (with RoPE, rotates it in place first), and the next barrier publishes steps
0 and 1 and retires the Q reads; only then are steps 2 .. NS - 3 staged.  The fast trips are
steady trips whose load wait is the constant (NS - 5) steps (the ring in full flow: both steps
they stage exist, and step t + 2, which they publish, needs no clearing).  A wave that skips
the reads of steps past its last query row only removes reads, which no check depends on.
"""
import random

import pytest

PAIR, FIRST, SECOND, NONE = "pair", "first", "second", "none"


WAVES = 8
Q = -1    # the "step" of a Q staging write / read


def q_plane(w):
    """The prologue's Q staging plane of wave w: (slot, plane)."""
    return 2 + w // 2, "K" if w % 2 == 0 else "V"


class Ring:
    def __init__(self, nsteps, ns, vzero, wait_slip=0, stage_slip=0, q_slot_slip=0,
                 early_stage=False, fast_wait_slip=0):
        self.n, self.ns, self.vzero = nsteps, ns, vzero
        self.wait_slip, self.stage_slip = wait_slip, stage_slip
        self.q_slot_slip, self.early_stage = q_slot_slip, early_stage
        self.fast_wait_slip = fast_wait_slip
        self.interval = 0
        self.issued = []          # steps in load-issue order (one loader queue)
        self.published = {}       # step -> first interval in which its loads are visible
        self.cleared = {}         # step -> interval of its V clear
        self.writes = []          # (interval, slot, step, what); Q writes: what = ("q", w, plane)
        self.reads = []           # (interval, slot, step, plane); Q reads: step = Q, plane (Q, w, plane)

    # -- kernel primitives -------------------------------------------------------------
    def stage(self, x):
        self.writes.append((self.interval, x % self.ns, x, "load"))
        self.issued.append(x)

    def wait(self, later):
        later += self.wait_slip
        done = self.issued[:len(self.issued) - later] if later > 0 else list(self.issued)
        for x in done:
            self.published.setdefault(x, self.interval + 1)

    def barrier(self):
        self.interval += 1

    def clear(self, x):
        assert self.published.get(x, 1 << 30) <= self.interval, f"clear of step {x} before its loads"
        self.cleared[x] = self.interval
        self.writes.append((self.interval, x % self.ns, x, "clear"))

    def read(self, x, plane):
        self.reads.append((self.interval, x % self.ns, x, plane))

    def expect_later(self, need, later):
        assert need in self.issued, f"wait for step {need}, which was never issued"
        assert self.issued.index(need) == len(self.issued) - 1 - later, \
            f"wait for step {need} leaves {later} steps out, issued {self.issued}"

    # -- the kernel's schedule -----------------------------------------------------------
    def step_reads(self, t):
        self.read(t + 1, "K")     # QK of the next step
        self.read(t, "V")         # PV of this step

    def general(self, t, mode):
        """iteration(step, stage, ..., mode): sync, reads, upkeep."""
        n, ns = self.n, self.ns
        need = t
        if mode != NONE:
            need = min(t + (2 if mode == PAIR else 1), n - 1)
            if need > t:
                ahead = t + (ns - 2 if mode == SECOND else ns - 3)
                later = min(ahead, n - 1) - need
                self.expect_later(need, later)
                self.wait(later)
            self.barrier()
        self.step_reads(t)
        if mode != NONE:
            if mode != SECOND:
                for k in (ns - 2, ns - 1):
                    if t + k - self.stage_slip < n and t + k - self.stage_slip >= 0:
                        self.stage(t + k - self.stage_slip)
            if need > t and self.vzero[need]:
                self.clear(need)

    def steady(self, t, fast=False):
        """The steady-state trip: steps t and t + 1 under one barrier.  fast: the kernel's
        fast trip, which waits for the constant NS - 5 later steps without computing it."""
        n, ns = self.n, self.ns
        need = min(t + 2, n - 1)
        if fast:
            assert t + ns - 1 < n and not self.vzero[t + 2], "fast trip outside its range"
            later = ns - 5 + self.fast_wait_slip
        else:
            later = ns - 5 if t + ns - 3 <= n - 1 else n - 1 - need
        self.expect_later(need, later)
        self.wait(later)
        self.barrier()
        for k in (ns - 2, ns - 1):
            if t + k < n:
                self.stage(t + k)
        if t + 2 < n and self.vzero[t + 2]:
            self.clear(t + 2)
        self.step_reads(t)
        self.step_reads(t + 1)

    def prologue(self):
        n, ns = self.n, self.ns
        self.barrier()                            # retire the previous tile's reads
        self.stage(0)
        if n > 1:
            self.stage(1)
        if self.early_stage:                      # slip: steps 2 .. NS-3 before the Q reads retire
            for t in range(2, min(ns - 2, n)):
                self.stage(t)
        for w in range(WAVES):
            slot, plane = q_plane(w)
            slot = (slot + self.q_slot_slip) % ns
            self.writes.append((self.interval, slot, Q, ("q", w, plane)))
        self.wait(0)                              # each wave: all its loads landed
        for w in range(WAVES):
            slot, plane = q_plane(w)
            slot = (slot + self.q_slot_slip) % ns
            self.writes.append((self.interval, slot, Q, ("rope", w, plane)))   # in place
            self.reads.append((self.interval, slot, Q, ("Q", w, plane)))
        self.barrier()                            # publishes steps 0, 1; retires the Q reads
        if not self.early_stage:
            for t in range(2, min(ns - 2, n)):
                self.stage(t)
        if self.vzero[0]:
            self.clear(0)
        self.read(0, "K")

    def run(self, steady_lim=0, odd_tail_barrier=True, fast_trips=False):
        n, ns = self.n, self.ns
        self.prologue()
        t = 0
        while t < steady_lim:
            assert not self.vzero[t] and not self.vzero[t + 1]
            fast = fast_trips and t + ns - 1 < n and not self.vzero[t + 2]
            self.steady(t, fast=fast)
            t += 2
        while t + 2 <= n:
            if not self.vzero[t + 1]:
                self.general(t, PAIR)
                self.general(t + 1, NONE)
            else:
                self.general(t, FIRST)
                self.general(t + 1, SECOND)
            t += 2
        if t < n:
            self.general(t, SECOND if odd_tail_barrier else NONE)
        return self

    # -- checks ------------------------------------------------------------------------
    @staticmethod
    def _planes(what):
        """Planes a write touches: a step's load both, a clear V, a Q write its own."""
        if what == "load":
            return {"K", "V"}
        if what == "clear":
            return {"V"}
        return {what[2]}

    def check(self):
        n = self.n
        assert sorted(self.issued) == list(range(n)), f"issued {self.issued}"
        for (iv, slot, x, plane) in self.reads:
            if x == Q:
                # a wave's own Q plane, read after its own wait in the interval it was written
                mine = [w for w in self.writes if w[1] == slot and w[0] == iv and w[2] == Q
                        and w[3][1] == plane[1] and w[3][2] == plane[2]]
                assert mine, f"wave {plane[1]} reads a Q plane it did not stage"
                continue
            if x >= n:
                continue                          # QK past the last step: never used
            earlier = [w for w in self.writes if w[1] == slot and w[0] < iv and
                       plane in self._planes(w[3]) and w[3] != "clear"]
            assert earlier and earlier[-1][2] == x, f"{plane} of step {x} read from a stale slot"
            assert self.published.get(x, 1 << 30) <= iv, f"{plane} of step {x} read before publish"
            if plane == "V" and self.vzero[x]:
                assert self.cleared.get(x, 1 << 30) < iv, f"V of step {x} read before its clear"
        for (iv, slot, x, what) in self.writes:
            for (riv, rslot, y, plane) in self.reads:
                if riv != iv or rslot != slot:
                    continue
                if y == Q:
                    rp = plane[2]
                    if rp not in self._planes(what):
                        continue
                    if x == Q and what[1] == plane[1]:
                        continue                  # the wave's own staging / rotation
                    raise AssertionError(f"{what} of step {x} races wave {plane[1]}'s Q read")
                if y < n and (what == "load" or plane == "V") and plane in self._planes(what):
                    raise AssertionError(f"{what} of step {x} races a {plane} read of step {y}")
        return self

    def reads_after_last_barrier(self):
        return {(slot, plane) for (iv, slot, x, plane) in self.reads
                if iv == self.interval and x < self.n}


def output_plane(wave, nsteps, ns):
    """The epilogue's choice: K plane of slot nsteps + w for w < NS - 1, else a V plane."""
    k = wave if wave < ns - 1 else wave - (ns - 1)
    return ((nsteps + k) % ns, "K" if wave < ns - 1 else "V")


def cases(seed=1):
    rnd = random.Random(seed)
    for ns in (5, 6, 7, 8):
        for n in range(1, 41):
            pats = [[False] * (n - 1) + [last] for last in (False, True)]
            pats += [[rnd.random() < 0.2 for _ in range(n)] for _ in range(12)]
            for vz in pats:
                yield ns, n, vz, 0
            for _ in range(12):
                lim = rnd.randrange(0, n) // 2 * 2   # even: trips of two steps
                vz = [rnd.random() < 0.2 for _ in range(n)]
                for x in range(lim):                 # steady steps are full, valid blocks
                    vz[x] = False
                yield ns, n, vz, lim


@pytest.mark.parametrize("ns", [6, 7, 8])
@pytest.mark.parametrize("fast", [False, True])
def test_ring_schedule_orders_every_access(ns, fast):
    # NS >= 6: the Q staging needs slots 2 .. 5 (the kernel asserts NS >= 2 + 8 / 2)
    count = 0
    for r_ns, n, vz, lim in cases():
        if r_ns != ns:
            continue
        ring = Ring(n, ns, vz).run(steady_lim=lim, fast_trips=fast).check()
        if 2 * ns - 3 >= 8:                        # the kernel asserts this for its output planes
            busy = ring.reads_after_last_barrier()
            planes = [output_plane(w, n, ns) for w in range(8)]
            assert len(set(planes)) == 8
            assert not set(planes) & busy, (n, planes, busy)
        count += 1
    assert count > 1000


def test_model_catches_slips():
    """Each plausible schedule mistake fails some check on some case."""
    def fails(**kw):
        run_kw = {"odd_tail_barrier": kw.pop("odd_tail_barrier", True),
                  "fast_trips": kw.pop("fast_trips", False)}
        for ns, n, vz, lim in cases(seed=2):
            if ns < 6:
                continue
            try:
                Ring(n, ns, vz, **kw).run(steady_lim=lim, **run_kw).check()
            except AssertionError:
                return True
        return False
    assert not fails(), "the kernel's schedule itself passes"
    assert not fails(fast_trips=True)
    assert fails(wait_slip=1), "a wait that leaves one step too many out"
    assert fails(stage_slip=-1), "a slot refilled one step early"
    assert fails(odd_tail_barrier=False), "the odd last step without its barrier"
    assert fails(q_slot_slip=-1), "Q staged over step 1's slot"
    assert fails(early_stage=True), "steps 2 .. NS-3 staged before the Q reads retire"
    assert fails(fast_wait_slip=1, fast_trips=True), "a fast trip waiting one step short"
