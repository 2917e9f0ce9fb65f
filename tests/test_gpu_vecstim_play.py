"""VecStim.play through call_mech_func (SimWrapper.cpp:461-468; the FunctionRegistry
entry of vecevent.h:42-45, VecEvent::update_sequence vecevent.cpp:280-309) against the
oracle making the same calls at the same points of the run.

Instances are given four kinds of old train so that each branch of the reference's
element() (vecevent.cpp:123-156) is reached when a new train arrives in the middle of a
run: a dense train still running (it delivers its queued element, then continues from
the new train at the position reached), a short train already read past its end (the
new train is ignored until finitialize), a train whose first element is still queued
(the new train's elements before it then all fire in the step that delivers it), and
an empty train (never reads anything).  Tolerances: soma voltages within 1e-4 mV,
synaptic conductances within 1e-9 relative, identical spike counts, spike times within
one dt."""
import copy
import ctypes
import dataclasses

import numpy as np
import pytest

import oracle
from heliox_amd import Sim, build_config
from heliox_amd.sim import HelioxError
from parity_util import V_TOL, compare_spikes

pytestmark = pytest.mark.gpu


def old_train(k):
    kind = k % 4
    if kind == 0:
        return np.arange(2.0, 30.0, 0.6)
    if kind == 1:
        return np.array([1.0, 3.0])
    if kind == 2:
        return np.array([15.05, 16.0, 17.5])
    return np.zeros(0)


def new_train(k):
    x = np.arange(0.3 + 0.05 * (k % 3), 45.0, 0.45)
    if k % 5 == 0:                        # one pair out of order
        x[10], x[11] = x[11], x[10]
    return x


def model(ncell):
    spec = build_config(2, ncell, 40.0)
    nvs = spec.n_vecstim
    trains = [old_train(k) for k in range(nvs)]
    off = np.zeros(nvs + 1, np.int64)
    off[1:] = np.cumsum([t.size for t in trains])
    spec = dataclasses.replace(spec, vecstim_offsets=off, vecstim_times=np.concatenate(trains))
    # strong synapses, so that every delivered event moves the soma
    nc = copy.deepcopy(spec.netcons)
    nc["ExpSyn"].weight = np.full(nc["ExpSyn"].weight.size, 4e-3)
    return dataclasses.replace(spec, netcons=nc)


def play_all(sim_play, nvs, skip_empty_call=1):
    for k in range(nvs):
        if k == skip_empty_call:
            sim_play(k, [])                # an empty vector changes nothing
        else:
            sim_play(k, new_train(k))


def both(spec, groups):
    o = oracle.OracleSim(spec)
    g = Sim()
    g.set_cell_groups(groups)
    g.load_model_from_spec(spec)
    return o, g


def check(o, g, spec):
    ot, gt = o.traces(), g.traces()
    assert ot.shape == gt.shape
    err = float(np.max(np.abs(ot - gt)))
    print(f"  max |dv| {err:.3e} mV", flush=True)
    assert err < V_TOL
    og, gg = o.array("ExpSyn", "g"), g.get_array("ExpSyn", "g")
    assert np.allclose(gg, og, rtol=1e-9, atol=1e-15)
    compare_spikes(o, g, spec.dt)


@pytest.mark.parametrize("ncell,groups", [(2, 1), (24, 2)])
def test_play_in_the_middle_of_a_run(gpu_lib, ncell, groups):
    spec = model(ncell)
    print(f"play mid-run: {ncell} cells, {groups} groups, {spec.n_vecstim} VecStims", flush=True)
    o, g = both(spec, groups)
    o.finitialize(-65.0)
    g.finitialize(-65.0)
    o.continue_run(12.0)
    g.continue_run(12.0)
    play_all(o.vecstim_play, spec.n_vecstim)
    play_all(lambda k, x: g.call_mech_func("VecStim", "play", k, x), spec.n_vecstim)
    o.continue_run(20.0)
    g.continue_run(20.0)
    check(o, g, spec)
    # the same calls once more, later in the same run, on the trains the first calls left
    play_all(o.vecstim_play, spec.n_vecstim, skip_empty_call=2)
    play_all(lambda k, x: g.call_mech_func("VecStim", "play", k, x), spec.n_vecstim, skip_empty_call=2)
    o.continue_run(8.0)
    g.continue_run(8.0)
    check(o, g, spec)


def test_play_between_runs_and_right_after_finitialize(gpu_lib):
    spec = model(2)
    o, g = both(spec, 1)
    for sim in (o, g):
        sim.finitialize(-65.0)
        sim.continue_run(10.0)
    # between runs: the next finitialize reads the new trains from their first element
    play_all(o.vecstim_play, spec.n_vecstim)
    play_all(lambda k, x: g.call_mech_func("VecStim", "play", k, x), spec.n_vecstim)
    for sim in (o, g):
        sim.finitialize(-65.0)
        sim.continue_run(15.0)
    check(o, g, spec)
    # right after finitialize: its delivery window (t <= dt/2) has already read the first
    # element of the trains it holds, so those stay queued
    for sim in (o, g):
        sim.finitialize(-65.0)
    play_all(lambda k, x: o.vecstim_play(k, np.asarray(x) + 0.2), spec.n_vecstim, skip_empty_call=0)
    play_all(lambda k, x: g.call_mech_func("VecStim", "play", k, np.asarray(x) + 0.2), spec.n_vecstim,
             skip_empty_call=0)
    for sim in (o, g):
        sim.continue_run(15.0)
    check(o, g, spec)


def test_unregistered_function_and_bad_arguments(gpu_lib):
    spec = model(2)
    g = Sim()
    g.load_model_from_spec(spec)
    g.finitialize(-65.0)
    with pytest.raises(HelioxError, match="not registered"):
        g.call_mech_func("VecStim", "stop", 0, [1.0])
    with pytest.raises(HelioxError, match="not registered"):
        g.call_mech_func("ExpSyn", "play", 0, [1.0])
    with pytest.raises(HelioxError, match="2 arguments"):
        g.call_mech_func("VecStim", "play", [1.0])
    with pytest.raises(HelioxError, match="does not exist"):
        g.call_mech_func("VecStim", "play", spec.n_vecstim, [1.0])
    # through the C ABI an unregistered name is -1 with a message
    x = np.array([1.0])
    rc = gpu_lib.hx_call_mech_func(g._h, b"VecStim", b"stop", 0, 1, x.ctypes.data_as(ctypes.POINTER(ctypes.c_double)))
    assert rc == -1 and "not registered" in g.last_error()
