"""A stepping call that returns with its last state update pending (close deferral),
and on a model whose density mechanisms all run in the node kernel with that kernel's
assigned outputs made on demand, gives the same bits as one that ends with the closing
state pass: voltage traces, spikes and every column of every mechanism, read after the
last call, between calls, and after writes, a fusion switch or a restarted run between
calls."""
import dataclasses

import numpy as np
import pytest

from heliox_amd import Sim, build_config, mechanisms

pytestmark = pytest.mark.gpu

DT = 0.025


def make(spec, deferral, groups=0):
    g = Sim()
    g.set_close_deferral(deferral)
    g.set_cell_groups(groups)
    g.load_model_from_spec(spec)
    g.finitialize(-65.0)
    return g


def assert_same(spec, a, b):
    assert np.array_equal(a.get_array("node", "v"), b.get_array("node", "v"))
    cols = {m.name: m.columns for m in mechanisms()}
    checked = 0
    for mech in spec.mechs:
        if mech in ("VecStim", "NetStim"):
            continue
        for c in cols[mech]:
            x, y = a.get_array(mech, c), b.get_array(mech, c)
            assert np.array_equal(x, y, equal_nan=True), f"{mech}.{c}"
            checked += 1
    at, ag = a.spikes()
    bt, bg = b.spikes()
    assert sorted(zip(at, ag)) == sorted(zip(bt, bg))
    if a.traces().size:
        assert np.array_equal(a.traces(), b.traces())
    return checked


@pytest.mark.parametrize("config,ncell,monitors", [(3, 4, True), (2, 6, False), (4, 12, True), (5, 4, False),
                                                   (1, 3, True)])
def test_deferred_close_same_bits(gpu_lib, config, ncell, monitors):
    chunks = [40 * DT, 1 * DT, 17.25 * DT]
    spec = build_config(config, ncell, 2.0)
    if not monitors:
        spec = dataclasses.replace(spec, monitors=[])
    print(f"case deferral config={config} ncell={ncell} monitors={monitors}", flush=True)
    a, b = make(spec, True), make(spec, False)
    for c in chunks:
        a.continue_run(c)
        b.continue_run(c)
        # nothing read between these calls: the pending update carries over (the split
        # schedule, chosen for a model whose VecPlay drives a node variable, has none)
        assert a.info("state_pending") == a.info("fused") and b.info("state_pending") == 0
        # config 3 runs every density mechanism in the node kernel: its last step's
        # outputs are made on demand
        assert a.info("outputs_pending") == (1 if config == 3 else 0)
        assert b.info("outputs_pending") == 0
    a.fadvance()
    b.fadvance()
    n = assert_same(spec, a, b)
    assert a.info("state_pending") == 0      # the reads above completed it
    print(f"  {n} columns", flush=True)
    assert n > 5


@pytest.mark.parametrize("config,ncell", [(3, 16), (2, 24)])
def test_deferred_close_with_cell_groups(gpu_lib, config, ncell):
    spec = build_config(config, ncell, 2.0)      # two groups need 16 cells or more
    a, b = make(spec, True, groups=2), make(spec, False, groups=2)
    for c in (10 * DT, 3 * DT, 10 * DT):
        a.continue_run(c)
        b.continue_run(c)
        # the kernel timers are host state: switching them leaves the update pending
        for g in (a, b):
            g.set_profiling(True, classes=["mech"])
        assert a.info("state_pending") == 1
    a.kernel_time("mech")
    assert a.info("state_pending") == 1                             # reading the timers too
    assert a.info("multi_stream") == 1 and a.info("state_pending") == 1
    assert a.info("outputs_pending") == (1 if config == 3 else 0)
    assert assert_same(spec, a, b) > 10
    assert a.info("outputs_pending") == 0


@pytest.mark.parametrize("config,ncell", [(2, 6), (3, 2)])
def test_reads_and_writes_between_deferred_calls(gpu_lib, config, ncell):
    spec = dataclasses.replace(build_config(config, ncell, 2.0), monitors=[])
    a, b = make(spec, True), make(spec, False)
    for g in (a, b):
        g.continue_run(12 * DT)
        m0 = g.get_array("hh", "m")            # completes the pending update first
        g.set_variable_value(0.5 * float(m0[0]) + 0.1, "hh", "m", 0)
        g.continue_run(8 * DT)
        h = g.get_variable_handle("pas", "g", 3)
        g.continue_run(4 * DT)
        g.set_variable_by_handle(h, 2e-4)
        g.set_fusion(False)                   # split passes from here on
        g.continue_run(5 * DT)
        g.set_fusion(True)
        g.continue_run(5 * DT)
        g.run(6 * DT)                          # restarts t at 0 from the current state
    assert a.get_t() == b.get_t()
    assert assert_same(spec, a, b) > 10


def test_monitor_added_after_a_deferred_call(gpu_lib):
    spec = dataclasses.replace(build_config(3, 2, 2.0), monitors=[])
    a, b = make(spec, True), make(spec, False)
    for g in (a, b):
        g.continue_run(9 * DT)
        g.add_monitor("global", "v", 0)
        g.add_monitor("hh", "m", 5)            # a state monitor: calls end with the closing pass
        g.continue_run(7 * DT)
    assert a.info("state_pending") == 0
    assert assert_same(spec, a, b) > 20
