"""Models read from CoreNEURON exports run on the GPU with the same bits as the same
models built in memory (so the export path inherits the in-memory path's parity with
the oracle), and the configuration-4 network (cells, gaps, VecPlay, IClamp) read from
its export matches the oracle within the voltage tolerance."""
import dataclasses

import numpy as np
import pytest

import oracle
from coredat_writer import write_export
from heliox_amd import Sim
from parity_util import V_TOL, compare_spikes
from test_coredat import CASES, complete

pytestmark = pytest.mark.gpu

RUN_MS = {"config1": 30.0, "config2": 30.0, "config3": 5.0, "config4": 30.0, "config5": 30.0, "netstim": 30.0}


def from_export(path, mons, groups=0):
    g = Sim()
    g.set_cell_groups(groups)
    assert g.set_data_path(str(path)) == 0
    for m in mons:
        assert g.add_monitor(*m) >= 0
    assert g.load_model() == 0, g.last_error()
    return g


@pytest.mark.parametrize("case", sorted(CASES))
def test_export_runs_the_same_bits(gpu_lib, case, tmp_path):
    spec = complete(CASES[case]())
    mons = list(spec.monitors)[:8] + [("global", "v", spec.nnode - 1)]
    print(f"case coredat {case} nnode={spec.nnode}", flush=True)
    write_export(spec, tmp_path, seed=3)
    a = Sim()
    a.load_model_from_spec(dataclasses.replace(spec, monitors=mons))
    b = from_export(tmp_path, mons)
    for g in (a, b):
        g.finitialize(-65.0)
        g.run(RUN_MS[case])
    assert a.get_t() == b.get_t()
    assert np.array_equal(a.traces(), b.traces())
    ta, ga = a.spikes()
    tb, gb = b.spikes()
    assert np.array_equal(ta, tb) and np.array_equal(ga, gb)


def test_config4_export_matches_oracle(gpu_lib, tmp_path):
    spec = complete(CASES["config4"]())
    for vp in spec.vecplay:       # a stronger played clamp, so that the 8-cell net spikes in 60 ms
        vp.yvec = vp.yvec * 40.0
    mons = [("global", "v", c) for c in range(spec.ncell)]
    write_export(spec, tmp_path)
    g = from_export(tmp_path, mons)
    g.finitialize(-65.0)
    g.run(60.0)
    o = oracle.OracleSim(spec, monitors=mons)
    o.finitialize(-65.0)
    o.run(60.0)
    err = float(np.max(np.abs(o.traces() - g.traces())))
    print(f"  config4 from export: max |dv| vs oracle {err:.3e}", flush=True)
    assert err < V_TOL
    assert compare_spikes(o, g, spec.dt) > 0
