"""Solve units: the tree solve packs consecutive cells into one wavefront.  The
per-chunk arithmetic and the order of every sum are the same whatever the unit
size, so whole runs give the same bits, and the oracle's values."""
import dataclasses

import numpy as np
import pytest

import oracle
from heliox_amd import Sim, build_config
from parity_util import V_TOL, compare_spikes

pytestmark = pytest.mark.gpu


def run(spec, tstop, unit_cells, groups, mons, waves=0):
    g = Sim()
    g.set_solve_unit_cells(unit_cells)
    g.set_solve_waves(waves)
    g.set_cell_groups(groups)
    g.load_model_from_spec(dataclasses.replace(spec, monitors=list(mons)))
    g.finitialize(-65.0)
    g.run(tstop)
    return g


@pytest.mark.parametrize("config,ncell,tstop,sizes", [(3, 6, 8.0, (2,)), (2, 16, 30.0, (4, 16)),
                                                     (5, 8, 20.0, (2, 8))])
def test_unit_sizes_give_identical_runs(gpu_lib, config, ncell, tstop, sizes):
    spec = build_config(config, ncell, tstop)
    mons = [("global", "v", c) for c in range(ncell)]
    print(f"case units config={config} ncell={ncell} sizes={sizes}", flush=True)
    base = run(spec, tstop, 1, 1, mons)
    assert base.info("solve_unit_cells") == 1 and base.info("solve_units") == ncell
    for u in sizes:
        for groups in (1, 0):
            g = run(spec, tstop, u, groups, mons)
            assert g.info("solve_unit_cells") == u
            assert np.array_equal(g.traces(), base.traces()), (u, groups)
            assert np.array_equal(g.get_array("global", "v"), base.get_array("global", "v")), (u, groups)
            t1, g1 = g.spikes()
            t0, g0 = base.spikes()
            assert sorted(zip(t1, g1)) == sorted(zip(t0, g0))
    o = oracle.OracleSim(spec, monitors=mons)
    o.finitialize(-65.0)
    o.run(tstop)
    assert float(np.max(np.abs(o.traces() - base.traces()))) < V_TOL
    compare_spikes(o, base, spec.dt)


def test_default_unit_size_follows_cell_count(gpu_lib):
    spec = build_config(2, 3000, 1.0)
    g = Sim()
    g.load_model_from_spec(spec)
    # about one unit per 1024th of the cells: 3000 cells -> 3 per unit
    assert g.info("solve_unit_cells") == 3
    assert g.info("solve_units") == 1000


@pytest.mark.parametrize("config,ncell,unit_cells", [(2, 22, 2), (3, 7, 1)])
def test_units_per_workgroup_give_identical_runs(gpu_lib, config, ncell, unit_cells):
    """One, two, three or four solve units per workgroup (the last workgroup partly
    empty where the unit count does not divide), with and without cell groups: the
    same bits."""
    tstop = 10.0
    spec = build_config(config, ncell, tstop)
    mons = [("global", "v", c) for c in range(ncell)]
    print(f"case solve waves config={config} ncell={ncell} unit_cells={unit_cells}", flush=True)
    base = run(spec, tstop, unit_cells, 1, mons, waves=1)
    assert base.info("solve_waves") == 1
    for waves in (2, 3, 4):
        for groups in (1, 0):
            g = run(spec, tstop, unit_cells, groups, mons, waves=waves)
            assert g.info("solve_waves") == waves
            assert np.array_equal(g.traces(), base.traces()), (waves, groups)
            assert np.array_equal(g.get_array("global", "v"), base.get_array("global", "v")), (waves, groups)
            assert np.array_equal(g.get_array("global", "d"), base.get_array("global", "d")), (waves, groups)

