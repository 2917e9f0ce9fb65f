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
