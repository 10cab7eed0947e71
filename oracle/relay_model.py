"""CPU thread model of the relay flag protocol — TEST INFRASTRUCTURE ONLY.

Two models over int32 control blocks of 8 words, run by Python threads so
that tests can drive arbitrary interleavings:

``RefEdge`` restates the reference's per-edge protocol exactly:
  * publish (kernels/kr_publish_aic.cpp:6-22, kr_publish_aiv.cpp:6-23):
    published <- published + 1;
  * wait (kernels/kr_wait_aic.cpp:7-37, kr_wait_aiv.cpp:7-36):
    target = consumed + 1; poll published until >= target or maxSpins
    polls; consumed <- target; status <- 1 if published >= target else 2.
  Word layout [published, consumed, status, pad x5]
  (kernels/kr_sync_common.h:10-15).

``TileRelay`` models the device protocol of kernrelay_amd/csrc/kr_relay.h,
which folds the publish into the producer's epilogue and the wait into the
consumer's prologue:
  * a producer tile has a flag block; each of its ``arrivals`` workgroups
    writes its rows, then takes an arrival ticket; the last one resets the
    ticket and bumps ``published``;
  * each consumer of a tile has a state block; a consumer workgroup reading
    rows [lo, hi) spins, for every producer tile those rows touch, until
    ``published >= consumed + 1`` (or sets ``timed_out`` after max_spins);
  * the last consumer workgroup to finish (done ticket) advances
    ``consumed`` and writes ``status`` (2 if any workgroup timed out) for the
    state blocks [adv_lo, adv_hi) its launch owns.
  Tile data carries a replay stamp so a test can check that every row a
  consumer read came from the current replay (no stale read, no early read).

Pinned by the invariants the reference's design states (control blocks
zeroed once, counters monotone across replays, each wait consumes exactly
one publish, status in {1, 2}, a never-published edge reports 2) and by
planted mistakes that the checks must catch (tests/test_relay_model.py).
"""

import random
import threading
import time

K_WORDS = 8
OFF_PUBLISHED, OFF_CONSUMED, OFF_STATUS = 0, 1, 2
OFF_ARRIVE, OFF_DONE, OFF_TIMED_OUT = 3, 4, 5


class Ctrl:
    """int32 control blocks; ``fetch_add`` / ``exchange`` are atomic, loads
    and stores are single-word (as agent-scope relaxed atomics are)."""

    def __init__(self, blocks):
        self.w = [0] * (blocks * K_WORDS)
        self._lock = threading.Lock()
        self.history = {}  # (block, word) -> values stored, in order

    def load(self, b, off):
        return self.w[b * K_WORDS + off]

    def store(self, b, off, v):
        self.w[b * K_WORDS + off] = v
        self.history.setdefault((b, off), []).append(v)

    def fetch_add(self, b, off, v):
        with self._lock:
            old = self.w[b * K_WORDS + off]
            self.store(b, off, old + v)
            return old

    def exchange(self, b, off, v):
        with self._lock:
            old = self.w[b * K_WORDS + off]
            self.store(b, off, v)
            return old


def _yield(jitter):
    if jitter and random.random() < jitter:
        time.sleep(random.random() * 1e-4)
    else:
        time.sleep(0)


# ------------------------------------------------- the reference's edge ----

class RefEdge:
    """One reference edge: block ``index`` of ``ctrl``."""

    def __init__(self, ctrl, index):
        self.c, self.i = ctrl, index

    def publish(self):
        """kr_publish_aic.cpp:15-19: next = published + 1 (one writer)."""
        self.c.store(self.i, OFF_PUBLISHED, self.c.load(self.i, OFF_PUBLISHED) + 1)

    def wait(self, max_spins, jitter=0.0):
        """kr_wait_aic.cpp:20-35. Returns the status written."""
        target = self.c.load(self.i, OFF_CONSUMED) + 1
        value = self.c.load(self.i, OFF_PUBLISHED)
        spins = 0
        while value < target and spins < max_spins:
            spins += 1
            _yield(jitter)
            value = self.c.load(self.i, OFF_PUBLISHED)
        self.c.store(self.i, OFF_CONSUMED, target)
        status = 1 if value >= target else 2
        self.c.store(self.i, OFF_STATUS, status)
        return status


# ------------------------------------------------- the device protocol ----

class TileRelay:
    """Producer with ``tiles`` row tiles of ``prod_rows`` rows, each written
    by ``arrivals`` workgroups, and consumer launches.

    A launch is ``{"group": g, "ranges": [(lo, hi) per workgroup],
    "row_off": r, "adv": (adv_lo, adv_hi)}``: its workgroups read local rows
    [lo, hi) = producer rows [lo + r, hi + r); launches of one group share
    the group's state blocks (one per producer tile) and run in list order,
    as launches of one consumer do on its stream.
    """

    def __init__(self, tiles, prod_rows, arrivals, launches, max_spins=200000,
                 mistake=None):
        self.tiles, self.prod_rows, self.arrivals = tiles, prod_rows, arrivals
        self.launches = launches
        self.groups = sorted({l["group"] for l in launches})
        self.max_spins = max_spins
        self.mistake = mistake  # a planted bug, for the tests that must catch it
        self.ctrl = Ctrl(tiles * (1 + len(self.groups)))
        self.rows = [-1] * (tiles * prod_rows)  # replay stamp per row
        self.flag0 = 0

    def state0(self, group):
        return self.tiles * (1 + self.groups.index(group))

    def _arrive(self, t):
        """RelayArrive (kr_relay.h): ticket; the last arriver releases."""
        ticket = self.ctrl.fetch_add(self.flag0 + t, OFF_ARRIVE, 1)
        last = self.arrivals if self.mistake == "ticket_off_by_one" else self.arrivals - 1
        if ticket == last:
            self.ctrl.store(self.flag0 + t, OFF_ARRIVE, 0)
            self.ctrl.fetch_add(self.flag0 + t, OFF_PUBLISHED, 1)

    def produce(self, replay, t, w, jitter, delay):
        per = self.prod_rows // self.arrivals
        lo = t * self.prod_rows + w * per
        hi = t * self.prod_rows + (self.prod_rows if w == self.arrivals - 1 else (w + 1) * per)
        if delay:
            time.sleep(delay)
        if self.mistake == "publish_before_store":
            self._arrive(t)
        for r in range(lo, hi):
            if delay:
                time.sleep(delay / 16)
            self.rows[r] = replay
            _yield(jitter)
        if self.mistake != "publish_before_store":
            self._arrive(t)

    def _spin(self, t, state):
        """SpinOnTile (kr_relay.h)."""
        c = self.ctrl
        step = 0 if self.mistake == "target_no_plus_one" else 1
        target = c.load(state, OFF_CONSUMED) + step
        spins = 0
        while c.load(self.flag0 + t, OFF_PUBLISHED) < target:
            spins += 1
            if spins > self.max_spins:
                c.store(state, OFF_TIMED_OUT, 1)
                return
            time.sleep(0)

    def consume(self, replay, launch, g, jitter, seen):
        """RelayWaitRows, the row reads, then RelayFinish (kr_relay.h)."""
        lo, hi = launch["ranges"][g]
        s0, off = self.state0(launch["group"]), launch.get("row_off", 0)
        if hi > lo:
            k0, k1 = (lo + off) // self.prod_rows, (hi - 1 + off) // self.prod_rows
            for k in range(k0, k1 + 1):
                self._spin(k, s0 + k)
            for r in range(lo + off, hi + off):
                seen.append((launch["group"], r, self.rows[r], replay))
                _yield(jitter)
        adv_lo, adv_hi = launch["adv"]
        if adv_hi <= adv_lo:
            return
        c = self.ctrl
        ticket = c.fetch_add(s0 + adv_lo, OFF_DONE, 1)
        if ticket == len(launch["ranges"]) - 1:
            c.store(s0 + adv_lo, OFF_DONE, 0)
            for k in range(adv_lo, adv_hi):
                cons = c.load(s0 + k, OFF_CONSUMED)
                to = c.exchange(s0 + k, OFF_TIMED_OUT, 0)
                c.store(s0 + k, OFF_CONSUMED, cons + 1)
                c.store(s0 + k, OFF_STATUS, 2 if to else 1)

    def _run_launch(self, replay, launch, jitter, seen):
        ths = [threading.Thread(target=self.consume, args=(replay, launch, g, jitter, seen))
               for g in range(len(launch["ranges"]))]
        random.shuffle(ths)
        for th in ths:
            th.start()
        for th in ths:
            th.join()

    def _run_group(self, replay, group, jitter, seen):
        for launch in self.launches:
            if launch["group"] == group:
                self._run_launch(replay, launch, jitter, seen)

    def replay(self, replay, jitter=0.2, producer_delay=0.0, skip_tiles=()):
        """One graph replay: every producer workgroup and every consumer
        group as threads, started in random order. Returns (group, row,
        stamp read, replay) for every row a consumer read."""
        seen = []
        jobs = [threading.Thread(target=self.produce, args=(replay, t, w, jitter, producer_delay))
                for t in range(self.tiles) if t not in skip_tiles for w in range(self.arrivals)]
        jobs += [threading.Thread(target=self._run_group, args=(replay, g, jitter, seen))
                 for g in self.groups]
        random.shuffle(jobs)
        for th in jobs:
            th.start()
        for th in jobs:
            th.join()
        return seen


def even_ranges(rows, groups):
    """Consumer workgroup row ranges: ``groups`` near-equal slices."""
    b = [rows * i // groups for i in range(groups + 1)]
    return [(b[i], b[i + 1]) for i in range(groups)]


# ------------------------------- consumer in the producer's workgroups ----

class InProducerRelay:
    """The relay consumer run by the producer's own workgroups (kr_gemm.hip
    NormTail): each of a tile's ``arrivals`` workgroups writes its share of
    the tile's rows, arrives with an indexed ticket (RelayArriveIndexed) —
    the last one releases — then spins until ``published >= consumed + 1``,
    reads the rows worker, worker + arrivals, ... of the whole tile (its
    ticket is its worker index), and takes a done ticket; the last one
    advances ``consumed`` and writes ``status``. One control block per tile
    serves both roles, as a 1:1 edge does."""

    def __init__(self, tiles, rows, arrivals, max_spins=200000, mistake=None):
        self.tiles, self.rows_per_tile, self.arrivals = tiles, rows, arrivals
        self.max_spins, self.mistake = max_spins, mistake
        self.ctrl = Ctrl(tiles)
        self.rows = [-1] * (tiles * rows)

    def workgroup(self, replay, t, w, jitter, seen, write_delay=0.0):
        c, base = self.ctrl, t * self.rows_per_tile
        per = self.rows_per_tile // self.arrivals
        lo = base + w * per
        hi = base + (self.rows_per_tile if w == self.arrivals - 1 else (w + 1) * per)
        if write_delay:
            time.sleep(write_delay * w)
        for r in range(lo, hi):
            self.rows[r] = replay
            _yield(jitter)
        worker = c.fetch_add(t, OFF_ARRIVE, 1)
        if worker == self.arrivals - 1:
            c.store(t, OFF_ARRIVE, 0)
            c.fetch_add(t, OFF_PUBLISHED, 1)
        if self.mistake != "no_wait":
            target = c.load(t, OFF_CONSUMED) + 1
            spins = 0
            while c.load(t, OFF_PUBLISHED) < target:
                spins += 1
                if spins > self.max_spins:
                    c.store(t, OFF_TIMED_OUT, 1)
                    break
                time.sleep(0)
        for r in range(base + worker, base + self.rows_per_tile, self.arrivals):
            seen.append((r, self.rows[r], replay))
            _yield(jitter)
        if c.fetch_add(t, OFF_DONE, 1) == self.arrivals - 1:
            c.store(t, OFF_DONE, 0)
            to = c.exchange(t, OFF_TIMED_OUT, 0)
            c.store(t, OFF_CONSUMED, c.load(t, OFF_CONSUMED) + 1)
            c.store(t, OFF_STATUS, 2 if to else 1)

    def replay(self, replay, jitter=0.2, write_delay=0.0):
        """All workgroups as threads, started in random order; with
        write_delay, workgroup w starts writing w * write_delay seconds late."""
        seen = []
        ids = [(t, w) for t in range(self.tiles) for w in range(self.arrivals)]
        random.shuffle(ids)
        jobs = [threading.Thread(target=self.workgroup, args=(replay, t, w, jitter, seen, write_delay))
                for t, w in ids]
        for th in jobs:
            th.start()
        for th in jobs:
            th.join()
        return seen


# ------------------------------------------ last-arrival fix-up of pieces ----

class PieceFixup:
    """Split work summed by its last piece (the stream-K GEMM's fix-up in
    kr_gemm_pipe.inc, the split attention's in kr_attn.hip): each of ``n``
    pieces writes its partial, waits for its own stores, then takes a ticket
    on the tile's counter; the piece that draws n - 1 resets the counter and
    sums every partial in piece order. The sum must use each piece's value of
    the current launch, and the order must not depend on which piece was
    last."""

    def __init__(self, pieces, mistake=None):
        self.n, self.mistake = pieces, mistake
        self.partial = [None] * pieces
        self.count = 0
        self._lock = threading.Lock()
        self.result = None

    def piece(self, launch, i, jitter, store_delay=0.0):
        value = (launch, i)
        if self.mistake == "ticket_before_store":
            # the ticket goes out while the partial is still being written
            ticket = self._ticket()
            if ticket != self.n - 1:
                time.sleep(store_delay)
            self.partial[i] = value
        else:
            _yield(jitter)
            self.partial[i] = value
            ticket = self._ticket()
        if ticket == self.n - 1:
            with self._lock:
                self.count = 0
            order = range(self.n) if self.mistake != "arrival_order" else [i] + [j for j in range(self.n) if j != i]
            self.result = [self.partial[j] for j in order]

    def _ticket(self):
        with self._lock:
            t = self.count
            self.count += 1
            return t

    def launch(self, launch, jitter=0.3, store_delay=0.0):
        self.result = None
        ths = [threading.Thread(target=self.piece, args=(launch, i, jitter, store_delay)) for i in range(self.n)]
        random.shuffle(ths)
        for th in ths:
            th.start()
        for th in ths:
            th.join()
        return self.result
