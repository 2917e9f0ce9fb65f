"""NetStim with one Random123 stream per instance: the Philox4x32-10 block against
Random123's published known-answer vectors (in the library and in the oracle), the
stream's mapping of ids and draws, closed forms of noiseless trains, and the library's
host-side trains against the oracle's queue-driven NetStim (netstim.cpp semantics)."""
import math

import numpy as np
import pytest

import oracle
from heliox_amd import netstim_train, philox4x32
from heliox_amd.spec import MechSpec, ModelSpec, NetConSpec

# Random123 known-answer vectors for philox4x32 with 10 rounds: (counter, key, output)
KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]
DT = 0.025


@pytest.mark.parametrize("ctr,key,want", KAT)
def test_philox_known_answers(ctr, key, want):
    assert philox4x32(ctr, key) == list(want)
    assert oracle.philox4x32(ctr, key) == list(want)


def step_times(n, dt=DT):
    """t of every step, accumulated as Simulate::fadvance does (two half steps)."""
    t = [0.0]
    for _ in range(n):
        x = t[-1]
        x += 0.5 * dt
        x += 0.5 * dt
        t.append(x)
    return np.array(t)


def delivered(train, dt=DT):
    """Step time at which each self event is delivered (first t_m with t_m + dt/2 >= T)."""
    tt = step_times(int(math.ceil(max(train, default=0.0) / dt)) + 4, dt)
    out, m = [], 0
    for T in train:
        while tt[m] + dt / 2 < T:
            m += 1
        out.append(tt[m])
    return np.array(out)


def test_stream_draws_follow_the_counter_layout():
    """ids (id1, id2, id3) sit in counter words 2, 3, 1; draws are the block's words in
    order, then the next sequence number; uniform = (u + 1) / (2^32 + 1)."""
    ids = (7, 3, 5)
    w = philox4x32((0, ids[2], ids[0], ids[1]), (0, 0)) + philox4x32((1, ids[2], ids[0], ids[1]), (0, 0))
    u = [(x + 1.0) * (1.0 / 4294967297.0) for x in w]
    # noise 1, interval 1, start 0: T0 = invl = -log(u0); then T_k = t_m + (-log(u_k))
    tr = netstim_train(DT, 50.0, interval=1.0, number=6, start=0.0, noise=1.0, ids=ids)
    assert tr.size == 6
    assert tr[0] == -math.log(u[0])
    dl = delivered(tr)
    for k in range(1, 6):
        assert tr[k] == dl[k - 1] + (-math.log(u[k]))


def test_noiseless_train_closed_form():
    tr = netstim_train(DT, 500.0, interval=10.0, number=25, start=20.0, noise=0.0)
    assert tr.size == 25
    np.testing.assert_allclose(tr, 20.0 + 10.0 * np.arange(25), atol=1e-9)
    # number is compared as a real: 2.5 -> three spikes; 0 or a negative start -> none
    assert netstim_train(DT, 500.0, number=2.5, start=5.0).size == 3
    assert netstim_train(DT, 500.0, number=0, start=5.0).size == 0
    assert netstim_train(DT, 500.0, number=4, start=-1.0).size == 0
    # the horizon cuts the train
    assert netstim_train(DT, 45.0, interval=10.0, number=25, start=20.0).size == 3


def test_nonpositive_interval_uses_0_01_and_fires_within_one_step():
    """invl() replaces an interval <= 0 by 0.01 ms (netstim.cpp:140-145); the first event is
    start + 0.01 - interval; later events fall inside the same delivery window."""
    tr = netstim_train(DT, 100.0, interval=-1.0, number=5, start=3.0, noise=0.0)
    assert tr.size == 5
    assert tr[0] == 3.0 + 0.01 + 1.0
    dl = delivered(tr)
    assert np.all(dl == dl[0])


def netstim_model(params, ids=None, tstop=300.0):
    """One passive compartment with an ExpSyn per NetStim instance (netcon delay 1 ms)."""
    n = len(params)
    spec = ModelSpec(ncell=1, parent=np.array([-1], np.int32), a=np.zeros(1), b=np.zeros(1),
                     area=np.array([1256.6]), cm=np.ones(1), dt=DT)
    spec.mechs["pas"] = MechSpec(np.zeros(1, np.int32), {"g_pas": np.array([1e-4]), "e_pas": np.array([-65.0])})
    spec.mechs["ExpSyn"] = MechSpec(np.zeros(n, np.int32), {"tau": np.full(n, 2.0), "e": np.zeros(n)})
    cols = {k: np.array([p[k] for p in params], float) for k in ("interval", "number", "start", "noise")}
    if ids is not None:
        for j, k in enumerate(("id1", "id2", "id3")):
            cols[k] = np.array([x[j] for x in ids], float)
    spec.mechs["NetStim"] = MechSpec(np.zeros(n, np.int32), cols)
    spec.netcons["ExpSyn"] = NetConSpec(inst=np.arange(n, dtype=np.int32), src_kind=np.full(n, 2, np.int8),
                                        src=np.arange(n, dtype=np.int32), weight=np.full(n, 1e-3),
                                        delay=np.full(n, 1.0))
    spec._tstop = tstop
    return spec


PARAMS = [dict(interval=10.0, number=12, start=5.0, noise=0.0),
          dict(interval=4.0, number=40, start=0.0, noise=0.5),
          dict(interval=2.5, number=1e9, start=12.3, noise=1.0),
          dict(interval=7.0, number=3.5, start=50.0, noise=0.2)]


def test_library_trains_match_the_oracle_queue():
    """The oracle runs NetStim through its event queue (INITIAL, init event, self events,
    per-instance streams); the spikes it emits are the library's trains delivered at step
    times, bit for bit."""
    tstop = 300.0
    spec = netstim_model(PARAMS, tstop=tstop)
    o = oracle.OracleSim(spec, monitors=[])
    o.finitialize(-65.0)
    o.run(tstop)
    ot, oi = o.netstim_spikes()
    for j, p in enumerate(PARAMS):
        got = ot[oi == j]
        tr = netstim_train(DT, tstop, ids=(j, 0, 0), **p)
        want = delivered(tr)
        want = want[want <= o.t]
        n = min(got.size, want.size)
        assert n > 2 and abs(got.size - want.size) <= 1, (j, got.size, want.size)
        assert np.array_equal(got[:n], want[:n]), j


def test_explicit_stream_ids():
    p = PARAMS[1]
    a = netstim_train(DT, 300.0, ids=(11, 2, 9), **p)
    spec = netstim_model([p], ids=[(11, 2, 9)])
    o = oracle.OracleSim(spec, monitors=[])
    o.finitialize(-65.0)
    o.run(300.0)
    ot, _ = o.netstim_spikes()
    want = delivered(a)
    want = want[want <= o.t]
    n = min(ot.size, want.size)
    assert n > 10 and np.array_equal(ot[:n], want[:n])
    # other ids, another stream
    assert not np.array_equal(a, netstim_train(DT, 300.0, ids=(12, 2, 9), **p))


def test_noisy_intervals_are_exponential():
    """noise 1: intervals are interval * Exp(1) on top of the step quantisation."""
    tr = netstim_train(DT, 2e5, interval=5.0, number=1e9, start=0.0, noise=1.0, ids=(1, 0, 0))
    gaps = np.diff(delivered(tr))
    assert gaps.size > 30000
    assert abs(gaps.mean() - 5.0) < 0.1
    # P(gap > 5) = exp(-1) up to the dt/2 rounding of each delivery
    assert abs(np.mean(gaps > 5.0) - math.exp(-1.0)) < 0.01


# ---------------------------------------------------------------------------
# NetStims that receive events (netstim.cpp:262-274): a netcon into a NetStim turns it
# on (weight > 0, when it is off) or off (weight < 0); the weight is truncated to an int
# ---------------------------------------------------------------------------
def gated_model(ns_params, triggers, weights, delays, chain=None):
    """NetStim instances each driven by one VecStim (its own trigger times); every NetStim
    drives an ExpSyn on one passive compartment.  chain: (src NetStim, dst NetStim, w, delay)
    netcons between NetStims, replacing the VecStim netcon of dst."""
    n = len(ns_params)
    spec = ModelSpec(ncell=1, parent=np.array([-1], np.int32), a=np.zeros(1), b=np.zeros(1),
                     area=np.array([1256.6]), cm=np.ones(1), dt=DT)
    spec.mechs["pas"] = MechSpec(np.zeros(1, np.int32), {"g_pas": np.array([1e-4]), "e_pas": np.array([-65.0])})
    spec.mechs["ExpSyn"] = MechSpec(np.zeros(n, np.int32), {"tau": np.full(n, 2.0), "e": np.zeros(n)})
    cols = {k: np.array([p[k] for p in ns_params], float) for k in ("interval", "number", "start", "noise")}
    spec.mechs["NetStim"] = MechSpec(np.zeros(n, np.int32), cols)
    spec.mechs["VecStim"] = MechSpec(np.zeros(n, np.int32), {})
    spec.vecstim_offsets = np.concatenate([[0], np.cumsum([len(t) for t in triggers])]).astype(np.int64)
    spec.vecstim_times = np.concatenate([np.asarray(t, float) for t in triggers])
    spec.netcons["ExpSyn"] = NetConSpec(inst=np.arange(n, dtype=np.int32), src_kind=np.full(n, 2, np.int8),
                                        src=np.arange(n, dtype=np.int32), weight=np.full(n, 1e-3),
                                        delay=np.full(n, 1.0))
    kind = np.full(n, 1, np.int8)
    src = np.arange(n, dtype=np.int32)
    w = np.asarray(weights, float)
    d = np.asarray(delays, float)
    for (a, b, wc, dc) in (chain or []):
        kind[b], src[b], w[b], d[b] = 2, a, wc, dc
    spec.netcons["NetStim"] = NetConSpec(inst=np.arange(n, dtype=np.int32), src_kind=kind, src=src, weight=w, delay=d)
    return spec


def run_oracle(spec, tstop):
    o = oracle.OracleSim(spec, monitors=[])
    o.finitialize(-65.0)
    o.run(tstop)
    return o


def chain_after(t0, interval, count):
    """Step times of a noiseless burst started at step time t0: each next self event at
    the previous spike's step time + interval, delivered at the first step reaching it."""
    tt = step_times(int(math.ceil((t0 + interval * count) / DT)) + 4)
    out = [t0]
    for _ in range(count - 1):
        T = out[-1] + interval
        m = int(np.searchsorted(tt + DT / 2, T))
        out.append(tt[m])
    return out


def test_trigger_starts_a_burst_and_is_ignored_while_on():
    """start < 0: the NetStim waits; a positive event while it is off starts a burst of
    `number` spikes, the first in the delivering step (event = invl - interval = 0), the
    next every `interval`; an event while it is on does nothing; after the last spike it is
    off again and the next trigger starts a new burst."""
    p = dict(interval=2.0, number=3, start=-1.0, noise=0.0)
    spec = gated_model([p], [[10.0, 11.0, 30.0]], [1.0], [0.5])
    o = run_oracle(spec, 60.0)
    ot, oi = o.netstim_spikes()
    t1, t3 = delivered([10.5])[0], delivered([30.5])[0]
    want = chain_after(t1, 2.0, 3) + chain_after(t3, 2.0, 3)
    assert np.array_equal(ot, np.array(want)), (ot, want)
    assert o.get("NetStim", "on", 0) == 0.0 and o.get("NetStim", "ispike", 0) == 3.0


@pytest.mark.parametrize("noise", [1.0, 0.5])
def test_noisy_trigger_draws_the_first_interval(noise):
    """A positive event turning a noisy NetStim on draws the first interval and removes
    its deterministic part (event = invl(interval) - interval (1 - noise), netstim.cpp:262-274):
    the first spike comes noise * interval * (-log u0) after the delivering step, the next
    ones invl(interval) = (1 - noise) interval + noise interval (-log u_k) apart, with u_k
    the instance's stream (ids (0, 0, 0), no draw at INITIAL since start < 0)."""
    interval = 2.0
    p = dict(interval=interval, number=3, start=-1.0, noise=noise)
    spec = gated_model([p], [[10.0]], [1.0], [0.5])
    o = run_oracle(spec, 40.0)
    ot, _ = o.netstim_spikes()
    w = philox4x32((0, 0, 0, 0), (0, 0))
    u = [(x + 1.0) * (1.0 / 4294967297.0) for x in w]
    t1 = delivered([10.5])[0]
    want, T = [], t1 + noise * interval * (-math.log(u[0]))
    for k in range(3):
        want.append(delivered([T])[0])
        T = want[-1] + (1.0 - noise) * interval + noise * interval * (-math.log(u[k + 1]))
    assert np.array_equal(ot, np.array(want)), (ot, want)
    assert o.get("NetStim", "on", 0) == 0.0 and o.get("NetStim", "ispike", 0) == 3.0


def test_negative_event_turns_a_running_netstim_off():
    p = dict(interval=10.0, number=100, start=5.0, noise=0.0)
    spec = gated_model([p], [[52.0]], [-1.0], [0.0])
    o = run_oracle(spec, 150.0)
    ot, _ = o.netstim_spikes()
    want = delivered([5.0 + 10.0 * k for k in range(5)])
    assert np.array_equal(ot, want), (ot, want)
    assert o.get("NetStim", "on", 0) == 0.0 and o.get("NetStim", "ispike", 0) == 5.0


def test_fractional_weights_truncate_to_zero():
    """The weight is read as an int: 0.9 starts nothing, -0.9 stops nothing."""
    off = dict(interval=2.0, number=3, start=-1.0, noise=0.0)
    running = dict(interval=10.0, number=6, start=5.0, noise=0.0)
    spec = gated_model([off, running], [[10.0], [22.0]], [0.9, -0.9], [0.0, 0.0])
    o = run_oracle(spec, 100.0)
    ot, oi = o.netstim_spikes()
    assert ot[oi == 0].size == 0
    assert ot[oi == 1].size == 6


def test_netstim_chain_within_one_step():
    """A (running) drives B (waiting) with delay 0: B's burst starts in the step of each of
    A's spikes, including the one at t = 0 delivered during finitialize."""
    a = dict(interval=10.0, number=3, start=0.0, noise=0.0)
    b = dict(interval=1.0, number=2, start=-1.0, noise=0.0)
    spec = gated_model([a, b], [[], []], [0.0, 0.0], [0.0, 0.0], chain=[(0, 1, 1.0, 0.0)])
    o = run_oracle(spec, 60.0)
    ot, oi = o.netstim_spikes()
    ta = delivered([0.0, 10.0, 20.0])
    assert np.array_equal(ot[oi == 0], ta)
    want_b = sum((chain_after(t, 1.0, 2) for t in ta), [])
    assert np.array_equal(ot[oi == 1], np.array(want_b)), (ot[oi == 1], want_b)
