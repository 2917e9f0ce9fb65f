"""NetStim-driven runs on the GPU against the oracle's queue-driven NetStim: trains made
on the host (and made longer as runs go past their horizon), delivered through the
device event ring, and the same bits with cell groups on their own streams."""
import dataclasses

import numpy as np
import pytest

import oracle
from heliox_amd import Sim, build_config
from heliox_amd.spec import MechSpec, NetConSpec
from parity_util import V_TOL
from test_netstim import PARAMS, netstim_model

pytestmark = pytest.mark.gpu


def gpu_run(spec, pieces, groups=0, mons=None):
    g = Sim()
    g.set_cell_groups(groups)
    g.load_model_from_spec(dataclasses.replace(spec, monitors=list(mons or spec.monitors)))
    g.finitialize(-65.0)
    for tp in pieces:
        g.continue_run(tp)
    return g


def oracle_run(spec, pieces, mons):
    o = oracle.OracleSim(spec, monitors=mons)
    o.finitialize(-65.0)
    for tp in pieces:
        o.continue_run(tp)
    return o


@pytest.mark.parametrize("pieces", [[300.0], [60.0, 60.0, 60.0, 120.0]])
def test_netstim_synapses_match_oracle(gpu_lib, pieces):
    # 300 ms = 12000 steps: past the 4096-step trains made at finitialize
    spec = netstim_model(PARAMS, tstop=300.0)
    mons = [("global", "v", 0), ("ExpSyn", "g", 1), ("ExpSyn", "g", 2)]
    print(f"case netstim pieces={pieces}", flush=True)
    g = gpu_run(spec, pieces, mons=mons)
    o = oracle_run(spec, pieces, mons)
    assert g.get_t() == o.t
    err = float(np.max(np.abs(o.traces() - g.traces())))
    print(f"  max |diff| {err:.3e}", flush=True)
    assert err < V_TOL
    assert np.max(np.abs(o.array("ExpSyn", "g") - g.get_array("ExpSyn", "g"))) < 1e-12
    # every instance fired: its synapse conductance moved
    assert np.all(np.max(np.abs(g.traces()[1:, :]), axis=1) > 0)


def netstim_network(ncell=16, tstop=40.0):
    """Config 2 with each VecStim input replaced by a NetStim of the same rate (10 Hz),
    half of them noisy."""
    spec = build_config(2, ncell, tstop)
    nvs = spec.n_vecstim
    n = nvs
    rng = np.random.default_rng(3)
    spec.mechs.pop("VecStim")
    spec.mechs["NetStim"] = MechSpec(np.zeros(n, np.int32), {
        "interval": np.full(n, 100.0), "number": np.full(n, 1e9), "start": rng.uniform(0, 20, n),
        "noise": np.where(np.arange(n) % 2 == 0, 1.0, 0.0)})
    spec.vecstim_offsets = np.zeros(1, np.int64)
    spec.vecstim_times = np.zeros(0)
    nc = spec.netcons["ExpSyn"]
    kind = nc.src_kind.copy()
    kind[kind == 1] = 2
    spec.netcons["ExpSyn"] = NetConSpec(nc.inst, kind, nc.src, nc.weight * 20, nc.delay)
    return spec


def test_netstim_network_groups_and_oracle(gpu_lib):
    spec = netstim_network(16, 40.0)
    mons = [("global", "v", c) for c in range(16)]
    print("case netstim network ncell=16", flush=True)
    multi = gpu_run(spec, [40.0], groups=0, mons=mons)
    single = gpu_run(spec, [40.0], groups=1, mons=mons)
    assert multi.info("cell_groups") == 2 and multi.info("multi_stream") == 1
    assert np.array_equal(multi.traces(), single.traces())
    o = oracle_run(spec, [40.0], mons)
    err = float(np.max(np.abs(o.traces() - multi.traces())))
    print(f"  max |dv| vs oracle {err:.3e}", flush=True)
    assert err < V_TOL
    assert np.max(np.abs(o.array("ExpSyn", "g") - multi.get_array("ExpSyn", "g"))) < 1e-12


# ---------------------------------------------------------------------------
# NetStims that receive events: run on the device by k_netstim
# ---------------------------------------------------------------------------
def compare_gated(spec, tstop, mons, groups=0):
    print(f"case gated tstop={tstop} nns={spec.mechs['NetStim'].n}", flush=True)
    g = gpu_run(spec, [tstop], groups=groups, mons=mons)
    o = oracle_run(spec, [tstop], mons)
    ot, oi = o.netstim_spikes()
    order = np.lexsort((oi, ot))
    ot, oi = ot[order], oi[order]
    gt, gi = g.netstim_spikes()
    print(f"  netstim spikes oracle {ot.size} gpu {gt.size}", flush=True)
    assert np.array_equal(oi, gi) and np.array_equal(ot, gt)
    err = float(np.max(np.abs(o.traces() - g.traces())))
    print(f"  max |diff| {err:.3e}", flush=True)
    assert err < V_TOL
    assert np.max(np.abs(o.array("ExpSyn", "g") - g.get_array("ExpSyn", "g"))) < 1e-12
    return o, g


def test_gated_netstims_match_oracle(gpu_lib):
    """Triggered bursts (an event while on ignored), a running NetStim switched off,
    noisy bursts with two triggers in one step, fractional weights."""
    from test_netstim import gated_model
    ps = [dict(interval=2.0, number=3, start=-1.0, noise=0.0),
          dict(interval=10.0, number=100, start=5.0, noise=0.0),
          dict(interval=3.0, number=4, start=-1.0, noise=0.6),
          dict(interval=2.0, number=3, start=-1.0, noise=0.0),
          dict(interval=10.0, number=6, start=5.0, noise=0.0)]
    trig = [[10.0, 11.0, 30.0], [52.0], [4.0, 20.0, 20.01, 45.0], [10.0], [22.0]]
    spec = gated_model(ps, trig, [1.0, -1.0, 2.5, 0.9, -0.9], [0.5, 0.0, 0.0, 0.0, 0.0])
    o, g = compare_gated(spec, 80.0, [("global", "v", 0), ("ExpSyn", "g", 0), ("ExpSyn", "g", 2)])
    for j in range(len(ps)):
        for var in ("on", "ispike", "event"):
            assert g.get_variable_value("NetStim", var, j) == o.get("NetStim", var, j), (j, var)


@pytest.mark.parametrize("delay", [0.0, 0.0125, 0.3])
def test_netstim_chains(gpu_lib, delay):
    """A running NetStim triggers a waiting one, which triggers a third: with delay 0 and
    dt/2 the bursts start within the step of the spike that triggers them (later passes of
    the step's delivery loop), including at t = 0 during finitialize."""
    from test_netstim import gated_model
    ps = [dict(interval=10.0, number=4, start=0.0, noise=0.0),
          dict(interval=1.0, number=2, start=-1.0, noise=0.0),
          dict(interval=0.5, number=3, start=-1.0, noise=0.5)]
    spec = gated_model(ps, [[], [], []], [0.0, 0.0, 0.0], [0.0, 0.0, 0.0],
                       chain=[(0, 1, 1.0, delay), (1, 2, 1.0, delay)])
    compare_gated(spec, 60.0, [("ExpSyn", "g", 1), ("ExpSyn", "g", 2)])


def test_cell_driven_netstims(gpu_lib):
    """Detected spikes of IClamp-driven cells trigger NetStims (one waits for triggers,
    one runs until a cell's spike turns it off) that drive synapses on the other cells."""
    spec = build_config(1, 4, 80.0)
    n = 5
    spec.mechs["NetStim"] = MechSpec(np.zeros(n, np.int32), {
        "interval": np.array([2.5, 3.0, 4.0, 2.0, 3.0]), "number": np.array([2, 3, 2, 1e9, 1e9]),
        "start": np.array([-1.0, -1.0, -1.0, 0.0, 1.0]), "noise": np.array([0.0, 0.4, 1.0, 0.0, 0.3])})
    soma = np.arange(spec.ncell, dtype=np.int32)
    spec.mechs["ExpSyn"] = MechSpec(np.array([1, 2, 3, 0, 2], np.int32),
                                    {"tau": np.full(n, 2.0), "e": np.zeros(n)})
    spec.netcons["ExpSyn"] = NetConSpec(inst=np.arange(n, dtype=np.int32), src_kind=np.full(n, 2, np.int8),
                                        src=np.arange(n, dtype=np.int32), weight=np.full(n, 0.02),
                                        delay=np.full(n, 0.7))
    spec.netcons["NetStim"] = NetConSpec(inst=np.arange(n, dtype=np.int32), src_kind=np.zeros(n, np.int8),
                                         src=np.array([0, 1, 2, 3, 0], np.int32),
                                         weight=np.array([1.0, 1.0, 1.0, -1.0, -1.0]),
                                         delay=np.array([1.5, 0.0, 0.4, 2.0, 0.0]))
    o, g = compare_gated(spec, 80.0, [("global", "v", int(s)) for s in soma])
    from parity_util import compare_spikes
    nsp = compare_spikes(o, g, spec.dt)
    gt, gi = g.netstim_spikes()
    print(f"  cell spikes {nsp}, netstim spikes per instance {np.bincount(gi, minlength=n)}", flush=True)
    assert nsp > 4 and np.all(np.bincount(gi, minlength=n)[:3] > 0)
