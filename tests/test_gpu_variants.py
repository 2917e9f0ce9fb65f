"""Launch variants that change no result.

The node kernel's compile-time steady-step instances (every density mechanism of the
pyramidal-cell model on every node; pas alone) give the same bits as the generic kernel:
traces, spikes and every column after a run, across configurations, cell groups, fusion
off (never steady), a monitor on an assigned variable (never steady) and chunked calls.
The cell groups' node passes taking turns on every step (events between the group streams)
give the same bits as ordering only a run's first step.  A model with IClamp and HalfGap
instances adds both currents in one launch over the nodes that carry either, and matches the
oracle."""
import dataclasses

import numpy as np
import pytest

from heliox_amd import Sim, build_config
from parity_util import V_TOL, compare_spikes, run_both

pytestmark = pytest.mark.gpu


def run(spec, steady, chunks=(5.0,), groups=1, mons=None, fusion=True, turns=True):
    g = Sim()
    g.set_cell_groups(groups)
    g.load_model_from_spec(spec if mons is None else dataclasses.replace(spec, monitors=list(mons)))
    g.set_dense_steady(steady)
    g.set_group_turns(turns)
    g.set_fusion(fusion)
    g.finitialize(-65.0)
    t = 0.0
    for c in chunks:
        t += c
        g.continue_run(t)
    return g


def columns(spec, g):
    from heliox_amd import mechanisms
    cols = {m.name: m.columns for m in mechanisms() if m.kind == "builtin"}
    out = {}
    for name in spec.mechs:
        if name in ("VecStim", "NetStim"):
            continue
        for col in cols[name]:
            out[(name, col)] = g.get_array(name, col)
    return out


def same_everything(spec, a, b):
    assert np.array_equal(a.traces(), b.traces())
    # the spike record of cell groups on their own streams interleaves in launch order
    sa, sb = a.spikes(), b.spikes()
    assert sorted(zip(sa[0], sa[1])) == sorted(zip(sb[0], sb[1]))
    ca, cb = columns(spec, a), columns(spec, b)
    assert ca.keys() == cb.keys()
    for k in ca:
        assert np.array_equal(ca[k], cb[k], equal_nan=True), k
    for k in ("v", "d", "rhs"):
        assert np.array_equal(a.get_array("global", k), b.get_array("global", k)), k


@pytest.mark.parametrize("config,ncell,groups", [(3, 3, 1), (3, 16, 2), (2, 3, 1), (5, 2, 1), (1, 4, 1),
                                                 (4, 12, 1)])
def test_steady_instance_same_bits(gpu_lib, config, ncell, groups):
    spec = build_config(config, ncell, 6.0)
    print(f"case steady instance config {config} ncell {ncell} groups {groups}", flush=True)
    a = run(spec, True, chunks=(2.0, 3.0), groups=groups)
    b = run(spec, False, chunks=(2.0, 3.0), groups=groups)
    assert a.info("cell_groups") == groups
    assert b.info("steady_launches") == 0
    if config == 3:
        # every density mechanism on every node: the pyramidal set has an instance
        assert a.info("steady_launches") > 0
    same_everything(spec, a, b)


def test_pyramidal_set_runs_its_instance_on_most_steps(gpu_lib):
    spec = build_config(3, 2, 4.0)
    print("case steady launches counted, config 3", flush=True)
    a = run(spec, True, chunks=(2.0,))
    nstep = int(round(2.0 / spec.dt))
    # finitialize's pass, the first step's current pass and each call's last step run the
    # generic kernel (they store outputs or have no state update before them)
    assert nstep - 3 <= a.info("steady_launches") <= nstep


def test_no_steady_instance_when_fusion_is_off_or_an_output_is_sampled(gpu_lib):
    spec = build_config(3, 2, 4.0)
    print("case steady instance off: split schedule, assigned monitor", flush=True)
    a = run(spec, True, fusion=False)
    assert a.info("steady_launches") == 0
    mons = list(spec.monitors) + [("hh", "ina", 5)]
    b = run(spec, True, mons=mons)
    c = run(spec, False, mons=mons)
    assert b.info("steady_launches") == 0
    same_everything(spec, b, c)


@pytest.mark.parametrize("groups", [2, 3])
def test_group_turns_same_bits(gpu_lib, groups):
    # groups hold at least 8 cells each
    spec = build_config(3, 8 * groups, 6.0)
    print(f"case group turns, config 3, {groups} groups", flush=True)
    a = run(spec, True, chunks=(1.0, 2.5, 0.5), groups=groups, turns=True)
    b = run(spec, True, chunks=(1.0, 2.5, 0.5), groups=groups, turns=False)
    assert a.info("cell_groups") == groups and a.info("multi_stream") == 1
    same_everything(spec, a, b)


def test_iclamp_and_halfgap_in_one_launch(gpu_lib):
    spec = build_config(4, 40, 20.0)
    assert spec.mechs["IClamp"].n > 0 and spec.mechs["HalfGap"].n > 0
    print("case electrode currents in one launch, config 4, 40 cells", flush=True)
    o, g = run_both(spec, 20.0)
    nodes = np.union1d(spec.mechs["IClamp"].nodes, spec.mechs["HalfGap"].nodes).size
    assert g.info("electrode_nodes") == nodes
    assert np.max(np.abs(o.traces() - g.traces())) < V_TOL
    compare_spikes(o, g, spec.dt)
    for col in ("i", "vgap"):
        assert np.max(np.abs(o.array("HalfGap", col) - g.get_array("HalfGap", col))) < 1e-9
    assert np.max(np.abs(o.array("IClamp", "i") - g.get_array("IClamp", "i"))) < 1e-12


def test_halfgap_named_by_two_gaps_takes_the_last(gpu_lib):
    """The reference copies gap transfers one after the other, so an instance named twice
    ends with the later gap's source; the oracle does the same."""
    spec = build_config(4, 16, 10.0)
    hg0 = int(spec.gap_halfgap[0])
    other = int(np.setdiff1d(np.arange(spec.ncell), [spec.gap_src_node[0], spec.mechs["HalfGap"].nodes[hg0]])[0])
    spec.gap_src_node = np.append(spec.gap_src_node, np.int32(other))
    spec.gap_halfgap = np.append(spec.gap_halfgap, np.int32(hg0))
    print("case HalfGap named by two gaps, config 4, 16 cells", flush=True)
    o, g = run_both(spec, 10.0)
    assert np.max(np.abs(o.traces() - g.traces())) < V_TOL
    assert np.max(np.abs(o.array("HalfGap", "vgap") - g.get_array("HalfGap", "vgap"))) < 1e-9
