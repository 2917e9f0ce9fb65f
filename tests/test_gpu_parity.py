"""Parity of the HIP step loop against the CPU oracle on the same seeded models."""
import numpy as np
import pytest

from heliox_amd import build_config
from parity_util import V_TOL, compare_spikes, run_both

pytestmark = pytest.mark.gpu

CASES = [
    # (config, ncell, tstop ms)
    (1, 4, 100.0),
    (2, 6, 100.0),
    (3, 2, 40.0),
    (4, 40, 100.0),
    (5, 4, 60.0),
]


@pytest.mark.parametrize("config,ncell,tstop", CASES)
@pytest.mark.parametrize("fusion", [True, False])
def test_traces_and_spikes(gpu_lib, config, ncell, tstop, fusion):
    spec = build_config(config, ncell, tstop)
    print(f"case config={config} ncell={ncell} tstop={tstop} fusion={fusion} nnode={spec.nnode}", flush=True)
    o, g = run_both(spec, tstop, fusion=fusion)
    to = o.traces()
    tg = g.traces()
    assert to.shape == tg.shape
    err = float(np.max(np.abs(to - tg)))
    print(f"  max |dv| = {err:.3e} mV", flush=True)
    assert err < V_TOL
    vo = o.array("global", "v")
    vg = g.get_array("global", "v")
    assert np.max(np.abs(vo - vg)) < V_TOL
    compare_spikes(o, g, spec.dt)
    assert abs(o.t - g.get_t()) == 0.0
