"""The mechanism plugin seam on the GPU: Im (csrc/mechs/Im.hip), registered by name at
library load, inserted into seeded models next to the built-in mechanisms and run
against the oracle's restatement of Im (user-mech/Im.cu:9-130)."""
import numpy as np
import pytest

import oracle
from heliox_amd import HelioxError, MechSpec, Sim, build_config
from parity_util import V_TOL, compare_spikes, run_both

pytestmark = pytest.mark.gpu


def with_im(spec, soma_g=2e-3, other_g=3e-4):
    """Im on every node that has k_ion, stronger on the somata (roots)."""
    nodes = spec.mechs["k_ion"].nodes.copy()
    g = np.where(nodes < spec.ncell, soma_g, other_g)
    spec.mechs["Im"] = MechSpec(nodes, {"gImbar": g})
    return spec


@pytest.mark.parametrize("config,ncell,tstop", [(1, 4, 100.0), (3, 2, 40.0)])
@pytest.mark.parametrize("fusion", [True, False])
def test_im_plugin_parity(gpu_lib, config, ncell, tstop, fusion):
    spec = with_im(build_config(config, ncell, tstop))
    print(f"case config={config} ncell={ncell} tstop={tstop} fusion={fusion} nIm={spec.mechs['Im'].n}",
          flush=True)
    o, g = run_both(spec, tstop, fusion=fusion)
    err = float(np.max(np.abs(o.traces() - g.traces())))
    print(f"  max |dv| = {err:.3e} mV", flush=True)
    assert err < V_TOL
    compare_spikes(o, g, spec.dt)
    for var in ("m", "ik", "gIm", "mTau"):
        a, b = o.array("Im", var), g.get_array("Im", var)
        scale = max(1e-30, float(np.max(np.abs(a))))
        assert np.max(np.abs(a - b)) <= 1e-6 * scale, var
    kc_o, kc_g = o.array("k_ion", "cur"), g.get_array("k_ion", "cur")
    assert np.max(np.abs(kc_o - kc_g)) <= 1e-6 * float(np.max(np.abs(kc_o)))


def test_im_changes_the_trace(gpu_lib):
    """The plugin's current reaches the membrane: with Im the spike count drops."""
    spec = build_config(1, 4, 100.0)
    g0 = Sim()
    g0.load_model_from_spec(spec)
    g0.finitialize(-65.0)
    g0.run(100.0)
    g1 = Sim()
    g1.load_model_from_spec(with_im(build_config(1, 4, 100.0), soma_g=0.02, other_g=0.02))
    g1.finitialize(-65.0)
    g1.run(100.0)
    n0, n1 = g0.spikes()[0].size, g1.spikes()[0].size
    print(f"  spikes without Im {n0}, with Im {n1}", flush=True)
    assert n1 < n0


def test_im_parameter_through_handles(gpu_lib):
    """gImbar set through the variable API after finitialize takes effect as in the oracle."""
    spec = with_im(build_config(1, 4, 60.0))
    o = oracle.OracleSim(spec)
    o.finitialize(-65.0)
    g = Sim()
    g.load_model_from_spec(spec)
    g.finitialize(-65.0)
    for i in range(spec.mechs["Im"].n):
        val = 5e-3 * (i + 1)
        o.set("Im", "gImbar", i, val)
        assert g.set_variable_value(val, "Im", "gImbar", i) == 0
        assert g.get_variable_value("Im", "gImbar", i) == val
    h = g.get_variable_handle("Im", "m", 0)
    assert h >= 0
    o.run(60.0)
    g.run(60.0)
    assert np.max(np.abs(o.traces() - g.traces())) < V_TOL
    assert abs(g.get_variable_by_handle(h) - o.get("Im", "m", 0)) < 1e-9
    compare_spikes(o, g, spec.dt)


def test_im_without_k_ion_is_refused(gpu_lib):
    spec = build_config(1, 4, 10.0)
    knodes = set(spec.mechs["k_ion"].nodes.tolist())
    bare = np.array([i for i in range(spec.nnode) if i not in knodes][:1], np.int32)
    assert bare.size == 1
    spec.mechs["Im"] = MechSpec(bare, {"gImbar": np.array([1e-3])})
    g = Sim()
    with pytest.raises(HelioxError, match="k_ion"):
        g.load_model_from_spec(spec)


def test_adjoint_refuses_plugins(gpu_lib):
    g = Sim()
    g.load_model_from_spec(with_im(build_config(1, 4, 10.0)))
    with pytest.raises(HelioxError, match="plugin"):
        g.tape_begin(10)


# ---------------------------------------------------------------------------
# syn_record (user_postsyn_mech/syn_record.cuh): a synapse plugin that netcons target
# ---------------------------------------------------------------------------
SR_TAUS = {"AMPA_tau1": 0.2, "AMPA_tau2": 1.7, "NMDA_tau1": 2.0, "NMDA_tau2": 30.0, "GABA_tau1": 0.5,
           "GABA_tau2": 6.0}


def with_syn_record(spec, nsyn_per_cell=6, seed=5, drive="vecstim"):
    """syn_record instances on random nodes of every cell, two thirds excitatory; driven by
    VecStim trains (drive="vecstim") or by the other cells' detectors (drive="cells")."""
    from heliox_amd.spec import NetConSpec
    rng = np.random.default_rng(seed)
    cell = spec.cell_of_node()
    nodes = []
    for c in range(spec.ncell):
        own = np.nonzero(cell == c)[0]
        nodes.extend(rng.choice(own, nsyn_per_cell, replace=False))
    nodes = np.sort(np.array(nodes, np.int32))
    n = nodes.size
    p = {k: np.full(n, v) for k, v in SR_TAUS.items()}
    w = np.where(rng.random(n) < 2 / 3, 1.0, -1.0)
    p.update({"w": w, "r_na": np.full(n, 2.0), "NMDA_C": np.full(n, 0.28), "NMDA_rho": np.full(n, 0.062),
              "AMPA_e": np.zeros(n), "NMDA_e": np.zeros(n), "GABA_e": np.full(n, -80.0)})
    spec.mechs["syn_record"] = MechSpec(nodes, p)
    weight = rng.uniform(0.002, 0.01, n)
    delay = rng.uniform(0.5, 2.0, n)
    if drive == "vecstim":
        spec.mechs["VecStim"] = MechSpec(np.zeros(n, np.int32), {})
        trains = [np.sort(rng.uniform(1.0, 80.0, rng.integers(3, 9))) for _ in range(n)]
        spec.vecstim_offsets = np.concatenate([[0], np.cumsum([t.size for t in trains])]).astype(np.int64)
        spec.vecstim_times = np.concatenate(trains)
        kind, src = np.ones(n, np.int8), np.arange(n, dtype=np.int32)
    else:
        kind = np.zeros(n, np.int8)
        src = ((cell[nodes] + 1) % spec.ncell).astype(np.int32)   # the next cell's detector
    spec.netcons["syn_record"] = NetConSpec(inst=np.arange(n, dtype=np.int32), src_kind=kind, src=src,
                                            weight=weight, delay=delay)
    return spec


@pytest.mark.parametrize("drive", ["vecstim", "cells"])
@pytest.mark.parametrize("fusion", [True, False])
def test_syn_record_plugin_parity(gpu_lib, drive, fusion):
    spec = with_syn_record(build_config(1, 4, 100.0), drive=drive)
    print(f"case syn_record drive={drive} fusion={fusion} n={spec.mechs['syn_record'].n}", flush=True)
    o, g = run_both(spec, 100.0, fusion=fusion)
    err = float(np.max(np.abs(o.traces() - g.traces())))
    print(f"  max |dv| = {err:.3e} mV", flush=True)
    assert err < V_TOL
    compare_spikes(o, g, spec.dt)
    for var in ("AMPA_A", "AMPA_B", "NMDA_B", "GABA_B", "i", "AMPA_factor", "didv", "dgdv"):
        a, b = o.array("syn_record", var), g.get_array("syn_record", var)
        scale = max(1e-30, float(np.max(np.abs(a))))
        assert np.max(np.abs(a - b)) <= 1e-6 * scale, var
    # the synapses received events: their conductance states moved
    assert np.max(g.get_array("syn_record", "NMDA_B")) > 0


def test_netcon_into_a_non_synapse_plugin_is_refused(gpu_lib):
    from heliox_amd.spec import NetConSpec
    spec = with_im(build_config(1, 4, 10.0))
    spec.mechs["VecStim"] = MechSpec(np.zeros(1, np.int32), {})
    spec.vecstim_offsets = np.array([0, 1], np.int64)
    spec.vecstim_times = np.array([1.0])
    spec.netcons["Im"] = NetConSpec(inst=np.array([0], np.int32), src_kind=np.array([1], np.int8),
                                    src=np.array([0], np.int32), weight=np.array([1.0]), delay=np.array([0.0]))
    g = Sim()
    with pytest.raises(HelioxError, match="synapse plugin"):
        g.load_model_from_spec(spec)
