"""Boundary semantics on the HIP path against the CPU oracle: the IClamp pulse window
when del and del + dur fall exactly on mid-step times (dt = 1/32, so every step time is
exact in binary), and the strict threshold on a slow voltage ramp.  Each model is a pure
capacitor (pas with g = 0) driven by an IClamp."""
import numpy as np
import pytest

import oracle
from heliox_amd import Sim
from heliox_amd.spec import MechSpec, ModelSpec

pytestmark = pytest.mark.gpu


def capacitor(dt, amp, delay, dur, area=500.0):
    spec = ModelSpec(ncell=1, parent=np.array([-1], np.int32), a=np.zeros(1), b=np.zeros(1),
                     area=np.array([area]), cm=np.ones(1), dt=dt)
    n = np.array([0], np.int32)
    spec.mechs["pas"] = MechSpec(n, {"g_pas": np.array([0.0]), "e_pas": np.array([-65.0])})
    spec.mechs["IClamp"] = MechSpec(n.copy(), {"delay": np.array([delay]), "dur": np.array([dur]),
                                               "amp": np.array([amp])})
    spec.monitors = [("global", "v", 0)]
    return spec


def both(spec, tstop):
    o = oracle.OracleSim(spec)
    o.finitialize(-65.0)
    o.run(tstop)
    g = Sim()
    g.load_model_from_spec(spec)
    g.finitialize(-65.0)
    g.run(tstop)
    return o, g


@pytest.mark.parametrize("fusion", [True, False])
def test_iclamp_window_on_exact_mid_step_times(gpu_lib, fusion):
    dt = 1.0 / 32
    spec = capacitor(dt, 0.004, 10.5 * dt, 6 * dt)
    print(f"case iclamp window fusion={fusion}", flush=True)
    o = oracle.OracleSim(spec)
    o.finitialize(-65.0)
    o.run(24 * dt)
    g = Sim()
    g.set_fusion(fusion)
    g.load_model_from_spec(spec)
    g.finitialize(-65.0)
    g.run(24 * dt)
    v = g.traces()[0]
    assert v.size == 25
    # steps 10..15 charge the capacitor, no other
    assert v[10] == -65.0 and v[11] > -65.0 and v[15] < v[16] and v[16] == v[17] == v[24]
    assert np.max(np.abs(v - o.traces()[0])) < 1e-12


def test_threshold_is_strict_on_a_slow_ramp(gpu_lib):
    dt, step, area = 0.025, 0.1, 500.0
    amp = step * (1e-3 / dt) * area / 1e2
    spec = capacitor(dt, amp, 0.0, 1e9, area)
    spec.presyn_gid = np.array([3], np.int32)
    spec.presyn_node = np.array([0], np.int32)
    spec.presyn_thr = np.array([-65.0 + 20.5 * step])
    print("case threshold ramp", flush=True)
    o, g = both(spec, 40 * dt)
    gt, gg = g.spikes()
    ot, og = o.spikes()
    assert list(gg) == [3] and list(og) == [3]
    assert gt[0] == ot[0]
    t = 0.0
    for _ in range(21):
        t += 0.5 * dt
        t += 0.5 * dt
    assert gt[0] == t
