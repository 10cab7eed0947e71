"""Relay protocol on a CPU thread model (oracle/relay_model.py).

Invariants (the reference's flag design: kernels/kr_sync_common.h:1-6,
kr_wait_aic.cpp, kr_publish_aic.cpp): counters zeroed once and monotone
across replays; each wait consumes exactly one publish; status in {1, 2};
a never-published edge reports 2. The device protocol (kr_relay.h) must in
addition never let a consumer read a row before the current replay wrote it,
under 1:1 and m:n row geometry. Planted mistakes in the model must be caught.
"""

import random
import threading

import pytest

from oracle import relay_model as RM


def _monotone(seq):
    return all(a <= b for a, b in zip(seq, seq[1:]))


def test_reference_edge_replays():
    random.seed(1)
    ctrl = RM.Ctrl(2)
    edge = RM.RefEdge(ctrl, 1)
    statuses = []
    for r in range(25):
        def producer():
            for _ in range(random.randint(0, 20)):
                threading.Event().wait(1e-5)
            edge.publish()
        th = threading.Thread(target=producer)
        th.start()
        statuses.append(edge.wait(max_spins=10 ** 7, jitter=0.3))
        th.join()
        assert ctrl.load(1, RM.OFF_CONSUMED) == ctrl.load(1, RM.OFF_PUBLISHED) == r + 1
    assert statuses == [1] * 25
    assert _monotone(ctrl.history[(1, RM.OFF_PUBLISHED)])
    assert _monotone(ctrl.history[(1, RM.OFF_CONSUMED)])
    assert ctrl.w[:RM.K_WORDS] == [0] * RM.K_WORDS  # other edges untouched


def test_reference_edge_never_published_reports_timeout():
    ctrl = RM.Ctrl(1)
    edge = RM.RefEdge(ctrl, 0)
    assert edge.wait(max_spins=50) == 2
    # the wait still consumes its target: one timeout shifts the edge by one
    assert ctrl.load(0, RM.OFF_CONSUMED) == 1 and ctrl.load(0, RM.OFF_PUBLISHED) == 0
    edge.publish()
    assert edge.wait(max_spins=50) == 2  # target 2, published 1
    edge.publish()
    edge.publish()
    assert edge.wait(max_spins=50) == 1  # back in step once published catches up


def _check_replays(relay, replays, **kw):
    for r in range(replays):
        seen = relay.replay(r, **kw)
        stale = [(g, row, got) for g, row, got, want in seen if got != want]
        assert not stale, "rows read before this replay wrote them: %s" % stale[:5]
    return seen


@pytest.mark.parametrize("arrivals", [1, 3])
def test_tile_relay_one_to_one(arrivals):
    random.seed(2 + arrivals)
    tiles, rows = 4, 12
    launch = {"group": 0, "ranges": RM.even_ranges(tiles * rows, tiles), "adv": (0, tiles)}
    relay = RM.TileRelay(tiles, rows, arrivals, [launch])
    _check_replays(relay, 12)
    c = relay.ctrl
    for t in range(tiles):
        assert c.load(t, RM.OFF_PUBLISHED) == 12
        st = relay.state0(0) + t
        assert c.load(st, RM.OFF_CONSUMED) == 12 and c.load(st, RM.OFF_STATUS) == 1
        assert _monotone(c.history[(t, RM.OFF_PUBLISHED)])
        assert _monotone(c.history[(st, RM.OFF_CONSUMED)])
        assert c.load(t, RM.OFF_ARRIVE) == 0 and c.load(st, RM.OFF_DONE) == 0


def _m_to_n_launches(total, kp, kc, groups_per_launch, group=0):
    """kc consumer launches over a producer split into kp tiles; launch j
    advances the producer tiles it is the last waiter of (the plan
    executor's last_waiter rule, kr_plan.cpp)."""
    prod = total // kp
    bounds = [total * j // kc for j in range(kc + 1)]
    launches = []
    for j in range(kc):
        lo, hi = bounds[j], bounds[j + 1]
        k0, k1 = lo // prod, (hi - 1) // prod
        nxt0 = bounds[j + 1] // prod if j + 1 < kc else kp
        adv = (k0, min(k1 + 1, nxt0)) if j + 1 < kc else (k0, k1 + 1)
        local = RM.even_ranges(hi - lo, groups_per_launch)
        launches.append({"group": group, "ranges": local, "row_off": lo, "adv": adv})
    return launches


@pytest.mark.parametrize("kp,kc", [(2, 3), (4, 3), (3, 4), (4, 2)])
def test_tile_relay_m_to_n_exactly_once(kp, kc):
    random.seed(10 * kp + kc)
    total = 48
    launches = _m_to_n_launches(total, kp, kc, groups_per_launch=2)
    # a second consumer of the same producer (fan-out) with its own states
    launches += [{"group": 1, "ranges": RM.even_ranges(total, 5), "adv": (0, kp)}]
    relay = RM.TileRelay(kp, total // kp, 2, launches)
    _check_replays(relay, 8)
    c = relay.ctrl
    for g in (0, 1):
        for t in range(kp):
            st = relay.state0(g) + t
            assert c.load(st, RM.OFF_CONSUMED) == 8, (g, t)
            assert c.load(st, RM.OFF_STATUS) == 1


def test_tile_relay_unreleased_tile_reports_timeout():
    launch = {"group": 0, "ranges": RM.even_ranges(16, 2), "adv": (0, 2)}
    relay = RM.TileRelay(2, 8, 1, [launch], max_spins=200)
    relay.replay(0, jitter=0.0, skip_tiles=(1,))
    c = relay.ctrl
    st = relay.state0(0)
    assert c.load(st, RM.OFF_STATUS) == 1  # status is per tile
    assert c.load(st + 1, RM.OFF_STATUS) == 2
    assert c.load(st + 1, RM.OFF_TIMED_OUT) == 0  # cleared by the done ticket
    assert c.load(st + 1, RM.OFF_CONSUMED) == 1


# ---- planted mistakes: each must be caught by the checks above ----

@pytest.mark.parametrize("mistake", ["target_no_plus_one", "publish_before_store"])
def test_planted_ordering_mistakes_read_stale_rows(mistake):
    random.seed(7)
    launch = {"group": 0, "ranges": RM.even_ranges(16, 2), "adv": (0, 2)}
    relay = RM.TileRelay(2, 8, 1, [launch], mistake=mistake)
    with pytest.raises(AssertionError, match="rows read before"):
        _check_replays(relay, 3, jitter=0.0, producer_delay=0.01)


def test_planted_ticket_mistake_times_out():
    launch = {"group": 0, "ranges": RM.even_ranges(16, 2), "adv": (0, 2)}
    relay = RM.TileRelay(2, 8, 2, [launch], max_spins=300, mistake="ticket_off_by_one")
    relay.replay(0, jitter=0.0)
    st = relay.state0(0)
    assert relay.ctrl.load(st, RM.OFF_STATUS) == 2
    assert relay.ctrl.load(0, RM.OFF_PUBLISHED) == 0


def test_correct_model_survives_the_same_delays():
    launch = {"group": 0, "ranges": RM.even_ranges(16, 2), "adv": (0, 2)}
    relay = RM.TileRelay(2, 8, 1, [launch])
    _check_replays(relay, 3, jitter=0.0, producer_delay=0.01)


# ------------------------- the consumer inside the producer's workgroups ----

@pytest.mark.parametrize("tiles,arrivals", [(1, 5), (4, 3), (2, 8)])
def test_in_producer_relay_reads_every_row_once_per_replay(tiles, arrivals):
    """The o/down GEMM's Add+RMSNorm relay: every row of a tile is read once
    per replay, only after this replay wrote it, whichever order the
    workgroups arrive in; the counters advance by one per replay with status
    1 and the tickets reset."""
    random.seed(40 + tiles)
    rows = 24
    relay = RM.InProducerRelay(tiles, rows, arrivals)
    for r in range(6):
        seen = relay.replay(r)
        assert sorted(row for row, _, _ in seen) == list(range(tiles * rows))
        assert all(got == want for _, got, want in seen), [s for s in seen if s[1] != s[2]][:4]
        for t in range(tiles):
            assert relay.ctrl.load(t, RM.OFF_PUBLISHED) == relay.ctrl.load(t, RM.OFF_CONSUMED) == r + 1
            assert relay.ctrl.load(t, RM.OFF_STATUS) == 1
            assert relay.ctrl.load(t, RM.OFF_ARRIVE) == relay.ctrl.load(t, RM.OFF_DONE) == 0


def test_in_producer_relay_planted_mistake_no_wait():
    """Without the wait, the first workgroups read rows the later ones have
    not written in this replay yet."""
    random.seed(7)
    relay = RM.InProducerRelay(1, 32, 8, mistake="no_wait")
    seen = relay.replay(0, jitter=0.0, write_delay=2e-3)
    assert any(got != want for _, got, want in seen)
    # and the correct protocol under the same delays reads nothing stale
    ok = RM.InProducerRelay(1, 32, 8)
    assert all(got == want for _, got, want in ok.replay(0, jitter=0.0, write_delay=2e-3))


# ----------------------------------------- the last-arrival fix-up ----

@pytest.mark.parametrize("pieces", [2, 4, 7])
def test_piece_fixup_sums_current_partials_in_piece_order(pieces):
    random.seed(pieces)
    f = RM.PieceFixup(pieces)
    for launch in range(20):
        assert f.launch(launch) == [(launch, i) for i in range(pieces)]
        assert f.count == 0


def test_piece_fixup_planted_mistakes():
    """A ticket taken before the partial is stored lets the finisher sum
    partials still being written (a previous launch's values); summing in
    arrival order makes the order depend on which piece finished last."""
    random.seed(3)
    bad = RM.PieceFixup(6, mistake="ticket_before_store")
    res = bad.launch(0, store_delay=5e-3)
    assert res != [(0, i) for i in range(6)]
    order = RM.PieceFixup(6, mistake="arrival_order")
    results = [order.launch(l) for l in range(30)]
    assert any(r != [(l, i) for i in range(6)] for l, r in enumerate(results))
