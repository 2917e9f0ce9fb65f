"""Parameter columns holding one value are read by the node kernels as that value: the
same bits as reading every instance's copy, and a handle into such a column (a write
through set_variable_value here) returns the column to per-instance reads before the
next step, so the written value takes effect (checked against the oracle with the same
change)."""
import dataclasses

import numpy as np
import pytest

import oracle
from heliox_amd import Sim, build_config
from parity_util import V_TOL

pytestmark = pytest.mark.gpu


def run(spec, tstop, uniform=True, mons=None, edit=None):
    g = Sim()
    g.set_cell_groups(1)
    g.load_model_from_spec(dataclasses.replace(spec, monitors=list(mons or spec.monitors)))
    g.set_uniform_columns(uniform)
    if edit:
        edit(g)
    g.finitialize(-65.0)
    g.run(tstop)
    return g


def test_scalar_reads_give_the_same_bits(gpu_lib):
    """With CaDynamics_E2 per instance (one gamma moved by 1e-7), the other uniform
    columns read as scalars give the same bits as per-instance reads."""
    spec = build_config(3, 2, 5.0)
    g = spec.mechs["CaDynamics_E2"].params["gamma"]
    g[0] *= 1.0000001
    mons = [("global", "v", 0), ("global", "v", spec.nnode - 1), ("hh", "m", 7), ("CaDynamics_E2", "cai", 9)]
    print("case uniform columns config3 2 cells", flush=True)
    a = run(spec, 5.0, True, mons)
    b = run(spec, 5.0, False, mons)
    # config 3: pas g/e, hh gl/el, hd_la vhalfl/tau, Ca_HVA gbar, CaDynamics_E2
    # decay/depth/minCai (gamma made per instance here), and the erev of na and k (style 0:
    # no kernel writes it); ca's conco, which finitialize sets to 2 mM everywhere (style 04)
    # and nothing writes after that; and the capacitance cm, one value on every node
    assert a.info("uniform_columns") == 14
    assert b.info("uniform_columns") == 0
    assert a.info("uniform_bytes") == 14 * 8 * spec.nnode
    assert np.array_equal(a.traces(), b.traces())


def test_uniform_calcium_constants_agree_to_rounding(gpu_lib):
    """With all four CaDynamics_E2 parameters one value over the model, its update uses
    constants made once on the host (1 - exp(-dt/decay) and the drive factor): the same
    results as the per-instance form to rounding."""
    spec = build_config(3, 2, 5.0)
    mons = [("global", "v", 0), ("global", "v", spec.nnode - 1), ("CaDynamics_E2", "cai", 9),
            ("CaDynamics_E2", "cai", spec.nnode - 3)]
    print("case uniform CaDynamics_E2 constants", flush=True)
    a = run(spec, 5.0, True, mons)
    b = run(spec, 5.0, False, mons)
    assert a.info("uniform_columns") == 15
    ta, tb = a.traces(), b.traces()
    assert np.max(np.abs(ta[:2] - tb[:2])) < 1e-9
    assert np.max(np.abs(ta[2:] - tb[2:]) / np.abs(tb[2:])) < 1e-12


def test_handle_write_returns_the_column_to_instance_reads(gpu_lib):
    spec = build_config(2, 3, 40.0)
    n_pas = spec.mechs["pas"].n
    mons = [("global", "v", c) for c in range(3)] + [("global", "v", 100)]
    assert int(spec.mechs["na_ion"].iontype.max()) == 0
    node = int(spec.mechs["pas"].nodes[100])
    print("case uniform column written through a handle", flush=True)

    na_nodes = spec.mechs["na_ion"].nodes
    k_na = 1
    na_node = int(na_nodes[k_na])

    def edit(g):
        before = g.info("uniform_columns")
        assert g.set_variable_value(3e-3, "pas", "g_pas", 100) == 0
        assert g.info("uniform_columns") == before - 1
        assert g.set_variable_value(65.0, "na_ion", "erev", na_node) == 0     # ions: by node
        assert g.info("uniform_columns") == before - 2
        assert g.set_variable_value(1.5, "capacitance", "cm", 100) == 0       # a node array
        assert g.info("uniform_columns") == before - 3

    g = run(spec, 40.0, True, mons, edit)
    ref = dataclasses.replace(spec, mechs=dict(spec.mechs))
    ref.mechs["pas"] = dataclasses.replace(spec.mechs["pas"], params=dict(spec.mechs["pas"].params))
    gp = ref.mechs["pas"].params["g_pas"].copy()
    gp[100] = 3e-3
    ref.mechs["pas"].params["g_pas"] = gp
    ref.mechs["na_ion"] = dataclasses.replace(spec.mechs["na_ion"], params=dict(spec.mechs["na_ion"].params))
    ena = ref.mechs["na_ion"].params["erev"].copy()
    ena[k_na] = 65.0
    ref.mechs["na_ion"].params["erev"] = ena
    ref.cm = spec.cm.copy()
    ref.cm[100] = 1.5
    o = oracle.OracleSim(ref, monitors=mons)
    o.finitialize(-65.0)
    o.run(40.0)
    err = float(np.max(np.abs(o.traces() - g.traces())))
    print(f"  max |dv| vs oracle {err:.3e} (node {node})", flush=True)
    assert err < V_TOL
    # and the change is visible: the untouched model differs at that node
    u = run(spec, 40.0, True, mons)
    assert np.max(np.abs(u.traces()[3] - g.traces()[3])) > 1e-3
    assert n_pas > 100


def test_conco_written_after_finitialize_takes_effect(gpu_lib):
    """ca_ion's conco is one value after finitialize (style 04 sets it) and read as that
    value; a write through a handle after finitialize returns it to per-instance reads,
    and the changed Nernst potential shows in the trace as in the oracle's."""
    spec = build_config(3, 2, 5.0)
    node = spec.nnode - 7
    mons = [("global", "v", 0), ("global", "v", node), ("CaDynamics_E2", "cai", node)]
    print("case conco written after finitialize", flush=True)
    g = Sim()
    g.set_cell_groups(1)
    g.load_model_from_spec(dataclasses.replace(spec, monitors=mons))
    before = g.info("uniform_columns")
    g.finitialize(-65.0)
    assert g.set_variable_value(8.0, "ca_ion", "conco", node) == 0
    assert g.info("uniform_columns") == before - 1
    g.run(5.0)
    o = oracle.OracleSim(spec, monitors=mons)
    o.finitialize(-65.0)
    o.set("ca_ion", "conco", node, 8.0)
    o.run(5.0)
    err = float(np.max(np.abs(o.traces()[:2] - g.traces()[:2])))
    print(f"  max |dv| vs oracle {err:.3e}", flush=True)
    assert err < V_TOL
    assert np.max(np.abs(o.traces()[2] - g.traces()[2]) / o.traces()[2]) < 1e-9
    # the unchanged model differs at that node (ica depends on eca)
    u = run(spec, 5.0, True, mons)
    assert np.max(np.abs(u.traces()[1] - g.traces()[1])) > 1e-9


def test_conco_with_mixed_styles(gpu_lib):
    """conco counts as one value only if it is one value as the steps read it: instances
    whose style lacks 04 keep their loaded conco.  With one such instance at 3 mM the
    column is read per instance (and matches the oracle); with that instance at the init
    default (2 mM) it is one value again.  One CaDynamics_E2 gamma is moved by 1e-7 so its
    per-model constants stay off and scalar and per-instance reads give the same bits."""
    spec = build_config(3, 2, 4.0)
    spec.mechs["CaDynamics_E2"].params["gamma"][0] *= 1.0000001
    node = 11
    mons = [("global", "v", 0), ("global", "v", node), ("CaDynamics_E2", "cai", node)]

    def variant(conco):
        ca = spec.mechs["ca_ion"]
        it = ca.iontype.copy()
        it[node] = 0o40 | 0o100                    # no 04: finitialize leaves conco as loaded
        params = dict(ca.params)
        co = params["conco"].copy()
        co[node] = conco
        params["conco"] = co
        mechs = dict(spec.mechs)
        mechs["ca_ion"] = dataclasses.replace(ca, params=params, iontype=it)
        return dataclasses.replace(spec, mechs=mechs)

    print("case conco with mixed styles", flush=True)
    mixed = variant(3.0)
    a = run(mixed, 4.0, True, mons)
    b = run(mixed, 4.0, False, mons)
    same = run(variant(2.0), 4.0, True, mons)
    ref = run(spec, 4.0, True, mons)
    assert a.info("uniform_columns") == ref.info("uniform_columns") - 1
    assert same.info("uniform_columns") == ref.info("uniform_columns")
    assert np.array_equal(a.traces(), b.traces())
    o = oracle.OracleSim(mixed, monitors=mons)
    o.finitialize(-65.0)
    o.run(4.0)
    assert float(np.max(np.abs(o.traces()[:2] - a.traces()[:2]))) < V_TOL
    assert np.max(np.abs(o.traces()[2] - a.traces()[2]) / o.traces()[2]) < 1e-9
