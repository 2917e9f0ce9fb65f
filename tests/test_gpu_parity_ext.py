"""Wider parity cases of the HIP path against the CPU oracle: active networks,
events at the delivery-window boundaries, gap junctions, VecPlay, state
columns, split-mode monitors, handles, stepping APIs and full-size models."""
import dataclasses

import numpy as np
import pytest

import oracle
from heliox_amd import Sim, build_config
from heliox_amd.spec import MechSpec, NetConSpec
from parity_util import V_TOL, compare_spikes, run_both

pytestmark = pytest.mark.gpu


def active_network(ncell=60, seed=5, tstop=60.0, wscale=3.0):
    """Config-4 wiring made active: 1 ms current pulses every 10 ms on a third
    of the cells, recurrent weights rescaled, delays spread down to 0 and
    exactly dt/2."""
    spec = build_config(4, ncell, tstop)
    rng = np.random.default_rng(seed)
    nc = spec.netcons["ExpSyn"]
    nc.weight = nc.weight * wscale
    d = nc.delay.copy()
    d[::7] = 0.0
    d[3::11] = 0.0125
    d[5::13] = rng.uniform(0.0, 0.1, d[5::13].size)
    nc.delay = d
    drive = np.arange(0, ncell, 3, dtype=np.int32)
    starts = np.arange(2.0, tstop, 10.0)
    nodes = np.repeat(drive, starts.size)
    dl = np.tile(starts, drive.size) + rng.uniform(0, 3, nodes.size)
    ic = spec.mechs["IClamp"]
    spec.mechs["IClamp"] = MechSpec(np.concatenate([ic.nodes, nodes]),
                                    {"delay": np.concatenate([ic.params["delay"], dl]),
                                     "dur": np.concatenate([ic.params["dur"], np.full(nodes.size, 1.0)]),
                                     "amp": np.concatenate([ic.params["amp"], np.full(nodes.size, 2.0)])})
    return spec


@pytest.mark.parametrize("fusion", [True, False])
def test_active_network_with_gaps_and_vecplay(gpu_lib, fusion):
    spec = active_network()
    print(f"case active network ncell={spec.ncell} fusion={fusion}", flush=True)
    o, g = run_both(spec, 60.0, fusion=fusion)
    n = compare_spikes(o, g, spec.dt)
    assert n > 50, "the network should be active"
    err = float(np.max(np.abs(o.traces() - g.traces())))
    print(f"  spikes {n}, max |dv| {err:.3e}", flush=True)
    assert err < V_TOL
    assert np.max(np.abs(o.array("ExpSyn", "g") - g.get_array("ExpSyn", "g"))) < 1e-12
    assert np.max(np.abs(o.array("HalfGap", "vgap") - g.get_array("HalfGap", "vgap"))) < V_TOL


def test_vecstim_boundary_delays(gpu_lib):
    spec = build_config(2, 8, 80.0)
    nc = spec.netcons["ExpSyn"]
    rng = np.random.default_rng(2)
    nc.delay = rng.choice([0.0, 0.0125, 0.025, 0.0375, 0.3, 2.5], nc.delay.size)
    nc.weight = nc.weight * 30
    # force some trains to have elements inside one window and out of order
    t = spec.vecstim_times.copy()
    t[::5] = np.round(t[::5] / 0.0125) * 0.0125
    spec.vecstim_times = t
    print("case vecstim boundary delays", flush=True)
    o, g = run_both(spec, 80.0)
    assert np.max(np.abs(o.traces() - g.traces())) < V_TOL
    assert np.max(np.abs(o.array("ExpSyn", "g") - g.get_array("ExpSyn", "g"))) < 1e-12
    compare_spikes(o, g, spec.dt)


@pytest.mark.parametrize("config,ncell", [(3, 2), (2, 4), (4, 30)])
def test_state_columns(gpu_lib, config, ncell):
    spec = build_config(config, ncell, 30.0)
    print(f"case state columns config={config}", flush=True)
    o, g = run_both(spec, 30.0)
    checks = {"hh": ("m", "h", "n"), "Exp2Syn": ("A", "B"), "ExpSyn": ("g",), "hd_la": ("l",), "Ca_HVA": ("m", "h")}
    for mech, cols in checks.items():
        if mech not in spec.mechs:
            continue
        for c in cols:
            err = np.max(np.abs(o.array(mech, c) - g.get_array(mech, c)))
            assert err < 1e-9, f"{mech}.{c}: {err}"
    if "ca_ion" in spec.mechs:
        assert np.max(np.abs(o.array("ca_ion", "conci") - g.get_array("ca_ion", "conci"))) < 1e-12
        assert np.max(np.abs(o.array("ca_ion", "erev") - g.get_array("ca_ion", "erev"))) < 1e-8


def test_monitors_on_assigned_variables_use_split_schedule(gpu_lib):
    spec = build_config(3, 1, 20.0)
    mons = [("global", "v", 0), ("hh", "ina", 0), ("hh", "minf", 5), ("Ca_HVA", "ica", 11), ("ca_ion", "cur", 3),
            ("hd_la", "i", 7), ("pas", "i", 2), ("CaDynamics_E2", "cai", 9), ("Exp2Syn", "g", 0)]
    print("case assigned-variable monitors", flush=True)
    o, g = run_both(spec, 20.0, monitors=mons)
    assert g.info("fused") == 0
    to, tg = o.traces(), g.traces()
    for i, m in enumerate(mons):
        scale = max(1.0, float(np.max(np.abs(to[i]))))
        err = np.max(np.abs(to[i] - tg[i])) / scale
        assert err < 1e-9, f"monitor {m}: {err}"


def test_state_monitors_keep_fused_schedule(gpu_lib):
    spec = build_config(3, 1, 20.0)
    mons = [("global", "v", 0), ("hh", "m", 0), ("hd_la", "l", 40), ("ca_ion", "conci", 3)]
    o, g = run_both(spec, 20.0, monitors=mons)
    assert g.info("fused") == 1
    assert np.max(np.abs(o.traces() - g.traces())) < 1e-9


def test_point_process_monitors_use_split_schedule(gpu_lib):
    """Event delivery runs before the deferred state update in the fused
    schedule, so a monitor on a synapse variable selects the split schedule,
    where it samples at the reference's record point."""
    spec = build_config(3, 1, 20.0)
    mons = [("global", "v", 0), ("Exp2Syn", "A", 0), ("Exp2Syn", "B", 3), ("hh", "m", 0)]
    o, g = run_both(spec, 20.0, monitors=mons)
    assert g.info("fused") == 0
    assert np.max(np.abs(o.traces() - g.traces())) < 1e-9


def test_stepping_apis_agree(gpu_lib):
    """run, continue_run in chunks and fadvance give the same trajectory."""
    spec = build_config(2, 3, 30.0)
    o, g = run_both(spec, 0.0, chunks=[5.0, 2.5, 7.5])
    for _ in range(12):
        o.fadvance()
        g.fadvance()
    assert o.t == g.get_t()
    assert np.max(np.abs(o.traces() - g.traces())) < V_TOL


def test_handles_and_reinitialisation(gpu_lib):
    spec = build_config(1, 3, 40.0)
    o, g = run_both(spec, 20.0)
    # change a parameter through a handle on both and continue
    h = g.get_variable_handle("IClamp", "amp", 1)
    assert h >= 0
    g.set_variable_by_handle(h, 0.9)
    o.set("IClamp", "amp", 1, 0.9)
    assert g.get_variable_by_handle(h) == 0.9
    hv = g.get_variable_handle("global", "v", 1)
    assert abs(g.get_variable_by_handle(hv) - o.get("global", "v", 1)) < V_TOL
    g.set_variable_value(0.0, "IClamp", "delay", 2)
    o.set("IClamp", "delay", 2, 0.0)
    o.continue_run(20.0)
    g.continue_run(20.0)
    assert np.max(np.abs(o.traces() - g.traces())) < V_TOL
    compare_spikes(o, g, spec.dt)
    # finitialize + run twice reproduces the same trajectory on the GPU
    g.finitialize(-65.0)
    g.continue_run(40.0)
    first = g.traces().copy()
    g.finitialize(-65.0)
    g.continue_run(40.0)
    assert np.array_equal(first, g.traces())


@pytest.mark.parametrize("config,ncell,nref", [(3, 2000, 3), (2, 10000, 4), (5, 1000, 4), (1, 1000, 6)])
def test_full_size_prefix(gpu_lib, config, ncell, nref):
    """Cells of configs 1, 2, 3 and 5 are independent, so the first cells of the
    full-size GPU model must match an oracle model of just those cells."""
    tstop = 5.0
    full = build_config(config, ncell, tstop)
    small = build_config(config, nref, tstop)
    mons = [("global", "v", i) for i in range(nref)]
    print(f"case full-size prefix config={config} ncell={ncell}", flush=True)
    g = Sim()
    g.load_model_from_spec(dataclasses.replace(full, monitors=mons))
    g.finitialize(-65.0)
    g.run(tstop)
    o = oracle.OracleSim(small, monitors=mons)
    o.finitialize(-65.0)
    o.run(tstop)
    assert np.max(np.abs(o.traces() - g.traces())) < V_TOL
    v = g.get_array("global", "v")
    assert np.all(np.isfinite(v))


@pytest.mark.parametrize("config,ncell", [(3, 2000), (2, 10000), (5, 1000)])
def test_full_size_cells_across_groups(gpu_lib, config, ncell):
    """At full size the cells run as two groups on two streams, in solve units of a few
    cells.  The first cell, the cells either side of the groups' boundary and the last two
    cells, each against an oracle model of that cell alone (the cells are independent and
    each has its own random stream, so build_config(first_cell=c) is cell c)."""
    tstop = 5.0
    picks = [0, ncell // 2 - 1, ncell // 2, ncell - 2, ncell - 1]
    full = build_config(config, ncell, tstop)
    mons = [("global", "v", c) for c in picks]          # node c is cell c's root
    print(f"case full-size cells across groups config={config} ncell={ncell} cells={picks}", flush=True)
    g = Sim()
    g.load_model_from_spec(dataclasses.replace(full, monitors=mons))
    g.finitialize(-65.0)
    g.run(tstop)
    assert g.info("cell_groups") == 2 and g.info("multi_stream") == 1
    tr = g.traces()
    for k, c in enumerate(picks):
        o = oracle.OracleSim(build_config(config, 1, tstop, first_cell=c), monitors=[("global", "v", 0)])
        o.finitialize(-65.0)
        o.run(tstop)
        ot = o.traces()
        assert ot.shape == (1, tr.shape[1])
        err = float(np.max(np.abs(ot[0] - tr[k])))
        print(f"  cell {c}: max |dv| {err:.3e}", flush=True)
        assert err < V_TOL, (c, err)


def test_axial_coefficient_writes_reach_the_solver(gpu_lib):
    """a and b written through handles mid-run: the solve runs on each cell's
    centre-rooted tree, where the links between the model root and the centre
    are reversed, so the writes must reach the solver's own coefficients."""
    spec = build_config(2, 2, 30.0)
    mons = [("global", "v", i) for i in range(2)]
    o, g = run_both(spec, 10.0, monitors=mons)
    cell = spec.cell_of_node()
    rng = np.random.default_rng(7)
    # every link of cell 0, which includes the reversed ones; a few of cell 1
    nodes = [int(i) for i in np.nonzero(cell == 0)[0][1:]] + [int(i) for i in np.nonzero(cell == 1)[0][1:6]]
    for i in nodes:
        for var in ("a", "b"):
            x = o.get("global", var, i) * float(rng.uniform(0.5, 2.0))
            o.set("global", var, i, x)
            h = g.get_variable_handle("global", var, i)
            g.set_variable_by_handle(h, x)
            assert g.get_variable_by_handle(h) == x
    o.continue_run(20.0)
    g.continue_run(20.0)
    err = float(np.max(np.abs(o.traces() - g.traces())))
    print(f"  max |dv| after a/b writes {err:.3e}", flush=True)
    assert err < V_TOL


def test_spike_file_matches_reference_format(gpu_lib, tmp_path):
    """spk.dat as Simulate::output_spikes writes it (simulate.cpp:892-909): the oracle's
    spikes sorted by (time, gid) and printed with "%.8g\\t%d"."""
    spec = active_network(ncell=30, tstop=40.0)
    print("case spike file ncell=30", flush=True)
    o, g = run_both(spec, 40.0)
    compare_spikes(o, g, spec.dt)
    path = g.output_spikes(str(tmp_path / "out"))
    got = open(path).read()
    ot, og = o.spikes()
    order = np.lexsort((og, ot))
    want = "".join("%.8g\t%d\n" % (ot[i], og[i]) for i in order if og[i] > -1)
    assert len(want) > 0
    assert got == want


@pytest.mark.parametrize("groups", [1, 0])
def test_calcium_update_in_the_current_pass_is_exact(gpu_lib, groups):
    """CaDynamics_E2 updated right after its ica (the default) against the separate state
    pass (selected by a monitor on ca_ion): the same bits."""
    spec = build_config(3, 16, 10.0)
    vm = [("global", "v", c) for c in range(0, 16, 3)]
    runs = []
    for extra in ([], [("ca_ion", "conci", 7)]):
        g = Sim()
        g.set_cell_groups(groups)
        g.load_model_from_spec(dataclasses.replace(spec, monitors=vm + extra))
        g.finitialize(-65.0)
        g.continue_run(4.0)
        g.continue_run(6.0)
        runs.append(g)
    a, b = runs
    assert np.array_equal(a.traces(), b.traces()[: len(vm)])
    assert np.array_equal(a.get_array("ca_ion", "conci"), b.get_array("ca_ion", "conci"))
    assert np.array_equal(a.get_array("ca_ion", "cur"), b.get_array("ca_ion", "cur"))


def test_cadynamics_get_array_at_size(gpu_lib):
    """get_array of CaDynamics_E2 cai / ica over 300k instances reads the ca_ion columns
    once (one copy and a host gather), matches the oracle, and leaves the scalar
    reading of uniform columns alone."""
    import time
    spec = build_config(3, 60, 0.25)
    print(f"case CaDynamics get_array at {spec.nnode} nodes", flush=True)
    o, g = run_both(spec, 0.25)
    for var in ("cai", "ica"):
        t0 = time.perf_counter()
        got = g.get_array("CaDynamics_E2", var)
        took = time.perf_counter() - t0
        ref = o.array("CaDynamics_E2", var)
        assert got.shape == ref.shape == (spec.nnode,)
        assert np.max(np.abs(got - ref)) <= 1e-9 * np.max(np.abs(ref)), var
        assert took < 2.0, f"get_array {var} took {took:.2f} s"
    # the same values through the ion's own column, by node
    conci = g.get_array("ca_ion", "conci")
    assert np.array_equal(np.sort(conci), np.sort(g.get_array("CaDynamics_E2", "cai")))


@pytest.mark.parametrize("config,ncell,chunks", [(3, 2, [10.0, 0.5, 7.25]), (2, 4, [12.0]), (5, 4, [3.0, 3.0])])
def test_every_column_after_a_run(gpu_lib, config, ncell, chunks):
    """With no monitor or handle on an assigned variable, a call's last step and its closing
    state pass store every column once: currents and their assigned outputs from the last
    current evaluation, rates from the closing state update, ion dcurdv as 0.  Every column
    of every mechanism then reads back as the oracle's after its last step."""
    from heliox_amd import mechanisms
    spec = build_config(config, ncell, sum(chunks))
    print(f"case every column config={config} chunks={chunks}", flush=True)
    o, g = run_both(spec, sum(chunks), chunks=chunks)
    cols = {m.name: m.columns for m in mechanisms() if m.kind == "builtin"}
    checked = 0
    for mech in spec.mechs:
        if mech in ("VecStim", "NetStim"):
            continue
        for c in cols[mech]:
            try:
                ref = o.array(mech, c)
            except Exception:
                continue                    # a column the oracle does not keep
            got = g.get_array(mech, c)
            scale = max(1.0, float(np.max(np.abs(ref))))
            err = float(np.max(np.abs(got - ref)))
            assert err <= 1e-9 * scale, f"{mech}.{c}: {err}"
            checked += 1
    print(f"  {checked} columns", flush=True)
    assert checked > 20
