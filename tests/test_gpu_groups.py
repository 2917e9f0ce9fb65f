"""Cell groups on separate streams: the same results as one stream, bit for bit,
and the oracle's within the parity tolerances."""
import dataclasses

import numpy as np
import pytest

import oracle
from heliox_amd import Sim, build_config
from parity_util import V_TOL, compare_spikes

pytestmark = pytest.mark.gpu


def run_gpu(spec, tstop, groups, monitors):
    g = Sim()
    g.set_cell_groups(groups)
    g.load_model_from_spec(dataclasses.replace(spec, monitors=list(monitors)))
    g.finitialize(-65.0)
    g.run(tstop)
    return g


@pytest.mark.parametrize("config,ncell,tstop", [(2, 24, 40.0), (3, 16, 8.0), (5, 20, 30.0)])
def test_groups_match_single_stream_and_oracle(gpu_lib, config, ncell, tstop):
    spec = build_config(config, ncell, tstop)
    if "ExpSyn" in spec.netcons:
        spec.netcons["ExpSyn"].weight = spec.netcons["ExpSyn"].weight * 10
    mons = [("global", "v", c) for c in range(ncell)]
    print(f"case groups config={config} ncell={ncell}", flush=True)
    multi = run_gpu(spec, tstop, 0, mons)
    single = run_gpu(spec, tstop, 1, mons)
    assert multi.info("cell_groups") == 2 and multi.info("multi_stream") == 1
    assert single.info("cell_groups") == 1 and single.info("multi_stream") == 0
    assert np.array_equal(multi.traces(), single.traces())
    for mech, cols in (("hh", ("m", "h", "n")), ("Exp2Syn", ("A", "B")), ("ExpSyn", ("g",))):
        if mech in spec.mechs:
            for c in cols:
                assert np.array_equal(multi.get_array(mech, c), single.get_array(mech, c)), (mech, c)
    mt, mg = multi.spikes()
    st, sg = single.spikes()
    assert sorted(zip(mt, mg)) == sorted(zip(st, sg))
    o = oracle.OracleSim(spec, monitors=mons)
    o.finitialize(-65.0)
    o.run(tstop)
    err = float(np.max(np.abs(o.traces() - multi.traces())))
    print(f"  max |dv| vs oracle {err:.3e}, spikes {mt.size}", flush=True)
    assert err < V_TOL
    compare_spikes(o, multi, spec.dt)


@pytest.mark.parametrize("config,ncell,tstop", [(2, 24, 30.0), (5, 40, 30.0)])
def test_groups_on_one_stream_share_event_launches(gpu_lib, config, ncell, tstop):
    """Cell groups issued on the library stream (group streams off, as under taping) take
    their VecStim input and delivery in one launch each: the same bits as the groups on
    their own streams and as one group."""
    spec = build_config(config, ncell, tstop)
    mons = [("global", "v", c) for c in range(ncell)]
    print(f"case shared event launches config={config} ncell={ncell}", flush=True)
    out = []
    for groups, streams in ((0, False), (0, True), (1, True)):
        g = Sim()
        g.set_cell_groups(groups)
        g.load_model_from_spec(dataclasses.replace(spec, monitors=list(mons)))
        g.set_group_streams(streams)
        g.finitialize(-65.0)
        g.run(tstop)
        assert g.info("multi_stream") == int(groups == 0 and streams)
        out.append(g)
    assert out[0].info("cell_groups") > 1
    for other in out[1:]:
        assert np.array_equal(out[0].traces(), other.traces())
        for mech, col in (("ExpSyn", "g"), ("Exp2Syn", "A"), ("Exp2Syn", "B")):
            if mech in spec.mechs:
                assert np.array_equal(out[0].get_array(mech, col), other.get_array(mech, col)), (mech, col)
        a, b = out[0].spikes(), other.spikes()
        assert sorted(zip(a[0], a[1])) == sorted(zip(b[0], b[1]))


def test_groups_fall_back_to_one_stream_with_state_monitors(gpu_lib):
    spec = build_config(2, 24, 10.0)
    mons = [("global", "v", 0), ("hh", "m", 3)]
    g = run_gpu(spec, 10.0, 0, mons)
    assert g.info("cell_groups") == 2 and g.info("multi_stream") == 0
    o = oracle.OracleSim(spec, monitors=mons)
    o.finitialize(-65.0)
    o.run(10.0)
    assert np.max(np.abs(o.traces() - g.traces())) < 1e-9


def test_groups_stepping_apis(gpu_lib):
    """run, continue_run in pieces and fadvance on the grouped path agree with one stream."""
    spec = build_config(2, 24, 30.0)
    mons = [("global", "v", c) for c in range(0, 24, 5)]
    out = []
    for groups in (0, 1):
        g = Sim()
        g.set_cell_groups(groups)
        g.load_model_from_spec(dataclasses.replace(spec, monitors=mons))
        g.finitialize(-65.0)
        g.continue_run(5.0)
        g.continue_run(2.5)
        for _ in range(7):
            g.fadvance()
        g.continue_run(10.0)
        out.append((g.traces().copy(), g.get_t(), g.get_array("global", "v")))
    assert out[0][1] == out[1][1]
    assert np.array_equal(out[0][0], out[1][0])
    assert np.array_equal(out[0][2], out[1][2])
