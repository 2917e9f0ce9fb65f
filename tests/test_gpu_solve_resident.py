"""The tree solve with each unit held whole in LDS (k_solve_res) against the solve that
streams its rounds from HBM (k_solve): the same bits for traces, spikes, v, the pivots
left in d and the solution left in rhs, on every configuration whose cells fit, with
several cells per unit, with cell groups on their own streams, and for the adjoint's
transposed solve; a unit too large for the budget is streamed."""
import dataclasses

import numpy as np
import pytest

import oracle
from heliox_amd import Sim, build_config
from heliox_amd.synth import perturb_config5
from parity_util import V_TOL

pytestmark = pytest.mark.gpu


def run(spec, resident, tstop, unit_cells=0, groups=1, chunks=2):
    g = Sim()
    g.set_cell_groups(groups)
    g.set_solve_unit_cells(unit_cells)
    g.set_solve_resident(resident)
    mons = [("global", "v", c) for c in range(spec.ncell)]
    g.load_model_from_spec(dataclasses.replace(spec, monitors=mons))
    g.finitialize(-65.0)
    for _ in range(chunks):
        g.continue_run(tstop / chunks)
    return g


def same_bits(a, b):
    assert np.array_equal(a.traces(), b.traces())
    sa, sb = a.spikes(), b.spikes()
    assert sorted(zip(sa[0], sa[1])) == sorted(zip(sb[0], sb[1]))
    for k in ("v", "d", "rhs"):
        assert np.array_equal(a.get_array("global", k), b.get_array("global", k)), k


@pytest.mark.parametrize("config,ncell,tstop,unit_cells", [
    (1, 12, 20.0, 0), (2, 12, 20.0, 0), (4, 16, 20.0, 0), (5, 8, 20.0, 0),
    (1, 12, 20.0, 5), (4, 16, 20.0, 3), (4, 16, 20.0, 4)])
def test_resident_solve_gives_the_streamed_bits(gpu_lib, config, ncell, tstop, unit_cells):
    spec = build_config(config, ncell, tstop)
    print(f"case resident config={config} ncell={ncell} unit_cells={unit_cells}", flush=True)
    res = run(spec, True, tstop, unit_cells)
    strm = run(spec, False, tstop, unit_cells)
    assert res.info("solve_resident") == 1
    assert strm.info("solve_resident") == 0
    same_bits(res, strm)
    o = oracle.OracleSim(spec, monitors=[("global", "v", c) for c in range(ncell)])
    o.finitialize(-65.0)
    for _ in range(2):
        o.continue_run(tstop / 2)
    assert float(np.max(np.abs(o.traces() - res.traces()))) < V_TOL


def test_resident_solve_with_cell_groups(gpu_lib):
    spec = build_config(5, 24, 20.0)
    print("case resident groups config=5 ncell=24", flush=True)
    res = run(spec, True, 20.0, groups=2)
    strm = run(spec, False, 20.0, groups=2)
    assert res.info("cell_groups") == 2 and res.info("multi_stream") == 1
    assert res.info("solve_resident") == 1
    same_bits(res, strm)


def test_large_units_stream(gpu_lib):
    """A config-3 cell (5000 nodes) needs about 200 KB held whole: it is streamed."""
    spec = build_config(3, 1, 2.0)
    g = run(spec, True, 2.0)
    assert g.info("solve_resident") == 0


def test_adjoint_transposed_solve_same_bits(gpu_lib):
    tstop = 20.0
    base = build_config(5, 2, tstop)
    mons = [("global", "v", i) for i in range(base.ncell)]
    o = oracle.OracleSim(perturb_config5(base, seed=3), monitors=mons)
    o.finitialize(-65.0)
    o.run(tstop)
    target = o.traces()[:, 1:].T
    out = []
    for resident in (True, False):
        print(f"case resident adjoint resident={resident}", flush=True)
        g = Sim()
        g.set_solve_resident(resident)
        g.load_model_from_spec(base, add_monitors=False)
        assert g.info("solve_resident") == int(resident)
        g.tape_begin(target.shape[0])
        g.finitialize(-65.0)
        g.run(tstop)
        loss = g.adjoint(np.arange(base.ncell), target)
        out.append((loss, {k: g.gradient(*k) for k in [("hh", "gnabar"), ("pas", "g_pas"), ("ExpSyn", "weight")]}))
    assert out[0][0] == out[1][0]
    for k in out[0][1]:
        np.testing.assert_array_equal(out[0][1][k], out[1][1][k], err_msg=str(k))
