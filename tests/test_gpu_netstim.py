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
