"""The HIP path against the committed golden fixtures (oracle outputs recorded
in tests/golden): traces within 1e-4 mV, identical spike counts with times
within one step, node states within 1e-9."""
import os

import numpy as np
import pytest

from golden.make_fixtures import STATE_CASES, TRACE_CASES
from heliox_amd import Sim, build_config
from parity_util import V_TOL

pytestmark = pytest.mark.gpu
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.mark.parametrize("name,config,ncell,tstop,mons", TRACE_CASES, ids=[c[0] for c in TRACE_CASES])
def test_gpu_traces_match_fixture(gpu_lib, name, config, ncell, tstop, mons):
    ref = load(name)
    spec = build_config(config, ncell, tstop)
    spec.monitors = list(mons)
    print(f"case golden {name}", flush=True)
    g = Sim()
    g.load_model_from_spec(spec)
    g.finitialize(-65.0)
    g.run(tstop)
    tr = g.traces()
    assert tr.shape == ref["traces"].shape
    nv = sum(1 for m in mons if m[0] == "global")
    assert np.max(np.abs(tr[:nv] - ref["traces"][:nv])) < V_TOL
    assert np.max(np.abs(tr[nv:] - ref["traces"][nv:])) < 1e-9
    st, sg = g.spikes()
    assert st.size == ref["spike_t"].size
    for gid in np.unique(ref["spike_gid"]):
        a = np.sort(ref["spike_t"][ref["spike_gid"] == gid])
        b = np.sort(st[sg == gid])
        assert a.size == b.size and np.all(np.abs(a - b) <= spec.dt * (1 + 1e-9))


@pytest.mark.parametrize("name,config,ncell,nstep", STATE_CASES, ids=[c[0] for c in STATE_CASES])
def test_gpu_state_matches_fixture(gpu_lib, name, config, ncell, nstep):
    ref = load(name)
    spec = build_config(config, ncell, nstep * build_config(config, 1, 1.0).dt + 1.0)
    g = Sim()
    g.load_model_from_spec(spec, add_monitors=False)
    g.finitialize(-65.0)
    np.testing.assert_allclose(g.get_array("global", "v"), ref["v_init"], atol=1e-12)
    for _ in range(nstep):
        g.fadvance()
    assert np.max(np.abs(g.get_array("global", "v") - ref["v"])) < V_TOL
    for key, (mech, var) in {"hh_m": ("hh", "m"), "hh_h": ("hh", "h"), "hh_n": ("hh", "n"),
                             "cahva_m": ("Ca_HVA", "m"), "hd_l": ("hd_la", "l"), "cai": ("ca_ion", "conci"),
                             "e2_A": ("Exp2Syn", "A"), "e2_B": ("Exp2Syn", "B")}.items():
        assert np.max(np.abs(g.get_array(mech, var) - ref[key])) < 1e-9, key
