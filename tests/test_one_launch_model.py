"""CPU model of two cross-workgroup protocols, run as a discrete-event
simulation on the host: workgroups are coroutines, at most R of a grid of G
are resident at once (the others start as resident ones exit), and every
store sits in its workgroup's store buffer until the scheduler drains it --
buffers drain out of order, so a store issued earlier can become visible
later than a store or atomic issued after it, unless the workgroup waits for
its stores first (``s_waitcnt vmcnt(0)``, which an agent-scope release fence
includes). Atomics act on memory at once. Memory starts with the stale
contents an earlier call on the same workspace left (queue entries of a
larger input). Every queue and table index a workgroup reads is checked
against the current call's bounds.

* ``one_launch``: the classified worker that was removed from this build
  (classification and work in one launch): workgroups claim ranges of
  segments from a counter, classify them (a class-count atomic and a queue
  store per segment), count each finished range, and the range that
  completes the count raises a ready flag; every workgroup waits for the
  flag (bounded) and then takes work tickets over the queues; every
  workgroup counts out and the last one resets the counters.
* ``shipped``: the register-resident softmax's protocol: the items were
  written by an earlier launch (visible when the kernel starts); workgroups
  take tickets, publish, may list an item for the drain (its list slot
  reserved with an atomic, then the entry stored: zero means not yet
  written), drain entries they claim with a compare-and-swap (waiting,
  bounded, for an entry to be written), and count out through ``last_out``
  (stores complete, then the count; the last one finishes every listed entry
  and resets).

The model shows two conditions that make the one-launch protocol read a
queue entry nobody wrote in this call: counting a range done before its
queue stores are visible, and a wait for the ready flag that times out
while ranges are left to workgroups that have not started (each workgroup
claiming one range, fewer resident than ranges); the latter also leaves
segments unprocessed. With stale entries from a larger earlier input those
reads index past the current call's segments. With the stores waited for
before the count and ranges claimed in a loop by whichever workgroups run,
it is exact on every schedule tried. The shipped protocol reads no unwritten
entry, finishes every item and resets only after every workgroup's last
read, on every schedule tried (fewer resident workgroups than the grid, slow
store visibility, drain waits that give up), and the model catches a planted
mistake in it (counting out before the workgroup's stores are complete).
Test infrastructure only: no GPU.
"""
from __future__ import annotations

import random

import pytest


class Machine:
    """Memory, per-workgroup store buffers and a random scheduler."""

    def __init__(self, seed: int, grid: int, resident: int, drain_p: float = 0.45):
        self.rng = random.Random(seed)
        self.drain_p = drain_p          # chance per step that a pending store lands
        self.mem: dict[str, int] = {}
        self.grid, self.resident = grid, resident
        self.buffers: dict[int, list[tuple[str, int]]] = {}
        self.finished_reads: set[int] = set()
        self.processed: list[int] = []
        self.drained = self.last_finished = 0

    def load(self, wg: int, addr: str) -> int:
        for a, v in reversed(self.buffers[wg]):
            if a == addr:            # a workgroup sees its own pending stores
                return v
        return self.mem.get(addr, 0)

    def store(self, wg: int, addr: str, value: int) -> None:
        self.buffers[wg].append((addr, value))

    def atomic_add(self, addr: str, value: int) -> int:
        old = self.mem.get(addr, 0)
        self.mem[addr] = old + value
        return old

    def cas(self, addr: str, expected: int, new: int) -> int:
        old = self.mem.get(addr, 0)
        if old == expected:
            self.mem[addr] = new
        return old

    def drain_one(self) -> bool:
        pending = [w for w, b in self.buffers.items() if b]
        if not pending:
            return False
        w = self.rng.choice(pending)
        i = self.rng.randrange(len(self.buffers[w]))      # out of order
        addr, value = self.buffers[w].pop(i)
        self.mem[addr] = value
        return True

    def run(self, program) -> None:
        """program(machine, wg) is a generator; it yields "wait_stores" to
        block until its buffer is empty, anything else to give up the CU."""
        waiting = list(range(self.grid))
        active: dict[int, object] = {}
        blocked: set[int] = set()
        steps = 0
        while waiting or active or any(self.buffers.values()):
            while waiting and len(active) < self.resident:
                wg = waiting.pop(0)
                self.buffers[wg] = []
                active[wg] = program(self, wg)
            steps += 1
            if steps > 2_000_000:
                raise RuntimeError("model did not finish")
            for wg in list(blocked):
                if not self.buffers[wg]:
                    blocked.discard(wg)
            runnable = [w for w in active if w not in blocked]
            if self.rng.random() < self.drain_p and self.drain_one():
                continue
            if not runnable:
                self.drain_one()
                continue
            wg = self.rng.choice(runnable)
            try:
                request = next(active[wg])
            except StopIteration:
                del active[wg]              # its stores still in flight land later
                continue
            if request == "wait_stores" and self.buffers[wg]:
                blocked.add(wg)
        while self.drain_one():
            pass


def one_launch(b: int, range_size: int, stale_b: int, fence_before_count: bool, claim_loop: bool,
               wait_budget: int, violations: list):
    """The removed one-launch classified worker. Segment s has class s % 2;
    class c's queue holds its segments at q{c}_{pos}."""
    n_ranges = (b + range_size - 1) // range_size

    def program(m: Machine, wg: int):
        # 1. Classify ranges.
        while True:
            r = m.atomic_add("claim", 1)
            yield
            if r >= n_ranges:
                break
            for s in range(r * range_size, min(b, (r + 1) * range_size)):
                c = s % 2
                pos = m.atomic_add(f"count{c}", 1)
                yield
                m.store(wg, f"q{c}_{pos}", s)
                yield
            if fence_before_count:
                yield "wait_stores"
            done = m.atomic_add("done", 1)
            yield
            if done == n_ranges - 1:
                m.store(wg, "ready", 1)
            if not claim_loop:
                break
        # 2. Wait (bounded) for every range to be classified.
        for _ in range(wait_budget):
            if m.load(wg, "ready"):
                break
            yield
        # 3. Work over the queues.
        while True:
            t = m.atomic_add("ticket", 1)
            yield
            n0, n1 = m.load(wg, "count0"), m.load(wg, "count1")
            if t >= n0 + n1:
                break
            c, pos = (0, t) if t < n0 else (1, t - n0)
            s = m.load(wg, f"q{c}_{pos}")
            yield
            if not (0 <= s < b) or s % 2 != c:
                violations.append(("unwritten queue entry", wg, c, pos, s))
            else:
                m.processed.append(s)
        m.finished_reads.add(wg)
        # 4. Count out; the last resets.
        yield "wait_stores"
        if m.atomic_add("out", 1) == m.grid - 1:
            if len(m.finished_reads) != m.grid:
                violations.append(("reset before every read", wg))
            for name in ("claim", "done", "ready", "out", "count0", "count1", "ticket"):
                m.store(wg, name, 0)
            yield "wait_stores"

    return program


def shipped(items: int, defer_every: int, drain_budget: int, violations: list, release: bool = True):
    """The register-resident softmax's ticket / deferral / drain / count-out
    protocol. Item i is valid in every call; the deferred list holds item
    index + 1 (0 = not yet written)."""

    def program(m: Machine, wg: int):
        seen = False
        while True:
            t = m.atomic_add("ticket", 1)
            yield
            word = t
            t &= 0xFFFFFFFF
            if t >= items:
                seen = seen or (word >> 32) != 0
                break
            if t % defer_every == 0:
                slot = m.atomic_add("ticket", 1 << 32) >> 32      # reserve a list slot, then write it
                yield
                m.store(wg, f"deferred_{slot}", t + 1)
                yield
            else:
                m.store(wg, f"out_{t}", 1)
                yield
        # Drain: claim listed entries while this workgroup saw deferrals.
        while seen:
            listed = m.load(wg, "ticket") >> 32
            c = m.load(wg, "claimed")
            if c >= listed:
                break
            if m.cas("claimed", c, c + 1) != c:
                yield
                continue
            entry = 0
            for _ in range(drain_budget):
                entry = m.load(wg, f"deferred_{c}")
                if entry:
                    break
                yield
            if entry:
                m.drained += 1
                if not (1 <= entry <= items):
                    violations.append(("bad list entry", wg, c, entry))
                m.store(wg, f"out_{entry - 1}", 1)
                m.store(wg, f"deferred_{c}", -1)            # finished: the last workgroup skips it
            yield
        m.finished_reads.add(wg)
        # last_out: stores complete (release), count; the last one (acquire)
        # finishes what is still listed and resets.
        if release:
            yield "wait_stores"
        if m.atomic_add("out", 1) == m.grid - 1:
            if len(m.finished_reads) != m.grid:
                violations.append(("reset before every read", wg))
            listed = m.load(wg, "ticket") >> 32
            for j in range(listed):
                entry = m.load(wg, f"deferred_{j}")
                if entry == 0:
                    violations.append(("listed entry never written", j))
                elif entry > 0:
                    m.last_finished += 1
                    m.store(wg, f"out_{entry - 1}", 1)
                m.store(wg, f"deferred_{j}", 0)
            for name in ("ticket", "claimed", "out"):
                m.store(wg, name, 0)
            yield "wait_stores"

    return program


def stale_queues(m: Machine, stale_b: int) -> None:
    """What an earlier, larger call left in the queues."""
    for c in (0, 1):
        for pos in range(stale_b):
            m.mem[f"q{c}_{pos}"] = stale_b - 1 - pos


SCHEDULES = [(seed, grid, resident, drain_p) for seed in range(12) for grid, resident in ((8, 8), (8, 3), (6, 1))
             for drain_p in (0.45, 0.02)]


@pytest.mark.parametrize("seed,grid,resident,drain_p", SCHEDULES)
def test_one_launch_safe_with_fence_and_claim_loop(seed, grid, resident, drain_p):
    """Ranges counted only once their queue stores are visible, and claimed
    in a loop by whichever workgroups run: every queue entry read was written
    by this call, whatever the residency, and the reset follows every read."""
    violations = []
    m = Machine(seed, grid, resident, drain_p)
    stale_queues(m, 64)
    m.run(one_launch(b=24, range_size=4, stale_b=64, fence_before_count=True, claim_loop=True,
                     wait_budget=10_000, violations=violations))
    assert violations == []
    assert sorted(m.processed) == list(range(24))
    assert all(m.mem.get(k, 0) == 0 for k in ("claim", "done", "ready", "out", "count0", "count1", "ticket"))


def test_one_launch_count_before_stores_reads_unwritten_entries():
    """Counting a range done before its queue stores are visible lets a
    workgroup pass the ready flag and read an entry this call has not yet
    written: a stale segment id of the earlier, larger input, past this
    call's segments."""
    hits = []
    for seed in range(40):
        violations = []
        m = Machine(seed, grid=8, resident=8, drain_p=0.02)
        stale_queues(m, 64)
        m.run(one_launch(b=24, range_size=4, stale_b=64, fence_before_count=False, claim_loop=True,
                         wait_budget=10_000, violations=violations))
        hits += [v for v in violations if v[0] == "unwritten queue entry"]
    assert hits, "the model found no schedule that exposes the race"
    assert any(v[4] >= 24 for v in hits), "no stale id past the current segments"


def test_one_launch_timeout_with_a_non_resident_claim():
    """Each workgroup claiming one range only (no claim loop) and fewer
    resident workgroups than ranges: the ranges of workgroups that have not
    started stay unclassified, the resident ones' waits time out and they
    work over queues still being filled -- reading entries reserved (counted)
    but not yet stored, stale, and leaving segments unprocessed."""
    hits, lost = [], 0
    for seed in range(20):
        violations = []
        m = Machine(seed, grid=6, resident=2)
        stale_queues(m, 64)
        m.run(one_launch(b=24, range_size=4, stale_b=64, fence_before_count=True, claim_loop=False,
                         wait_budget=20, violations=violations))
        hits += [v for v in violations if v[0] == "unwritten queue entry"]
        lost += sorted(m.processed) != list(range(24))
    assert hits and lost


@pytest.mark.parametrize("seed,grid,resident,drain_p", SCHEDULES)
@pytest.mark.parametrize("drain_budget", [1, 1000])
def test_shipped_protocol_reads_only_written_entries(seed, grid, resident, drain_p, drain_budget):
    """The shipped ticket / deferral / drain / count-out protocol: every item
    is finished exactly once or more (never lost), no list entry is read
    unwritten by the last workgroup, the reset follows every read, and the
    counters and list return to zero -- with out-of-order store visibility,
    fewer resident workgroups than the grid, and drain waits that give up
    (budget 1)."""
    violations = []
    m = Machine(seed, grid, resident, drain_p)
    items = 40
    m.run(shipped(items=items, defer_every=3, drain_budget=drain_budget, violations=violations))
    assert violations == []
    assert all(m.mem.get(f"out_{i}", 0) == 1 for i in range(items))
    assert all(m.mem.get(k, 0) == 0 for k in ("ticket", "claimed", "out"))
    assert all(v == 0 for k, v in m.mem.items() if k.startswith("deferred_"))


def test_shipped_protocol_paths_are_exercised_and_a_missing_release_is_caught():
    """The schedules above reach both ways a deferred item is finished (a
    draining workgroup's claim, the last workgroup's sweep), and the model
    catches a planted mistake: counting out without waiting for the
    workgroup's stores lets the last workgroup find a listed entry that has
    not landed."""
    drained = swept = 0
    for seed in range(12):
        for budget in (1, 1000):
            m = Machine(seed, 8, 3, 0.02)
            m.run(shipped(items=40, defer_every=3, drain_budget=budget, violations=[]))
            drained += m.drained
            swept += m.last_finished
    assert drained > 0 and swept > 0
    caught = []
    for seed in range(40):
        violations = []
        m = Machine(seed, 8, 8, 0.02)
        m.run(shipped(items=40, defer_every=3, drain_budget=1, violations=violations, release=False))
        caught += violations
    assert any(v[0] == "listed entry never written" for v in caught)
