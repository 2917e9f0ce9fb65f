"""The solve for the new voltage (the node kernel stores rhs + d v, the solve never reads v)
against the reference's solve for the change x = v_new - v: both against the oracle to the
voltage tolerance and to each other to rounding, with one cell group and with cell groups
on their own streams, through the resident and the streamed solve; rhs holds x after a
call either way; models where a later kernel adds to d or rhs keep the reference's form."""
import dataclasses

import numpy as np
import pytest

import oracle
from heliox_amd import Sim, build_config
from heliox_amd.spec import MechSpec
from parity_util import V_TOL

pytestmark = pytest.mark.gpu

# the forms differ by rounding alone (about |v| eps per step), which a spiking network
# carries along as it carries the oracle's different summation order
FORM_TOL = 1e-6     # mV


def hh_everywhere(spec):
    """The model with hh and its ions on every node (config 5 has them on the somas): every
    density mechanism then covers the whole model, and config 5's cells fit a resident unit."""
    mechs = dict(spec.mechs)
    every = np.arange(spec.nnode, dtype=np.int32)
    for name in ("hh", "na_ion", "k_ion"):
        m = mechs[name]
        ion = None if m.iontype is None else np.full(spec.nnode, m.iontype[0], m.iontype.dtype)
        mechs[name] = MechSpec(every.copy(), {k: np.full(spec.nnode, v[0]) for k, v in m.params.items()},
                               dict(m.globals), ion)
    return dataclasses.replace(spec, mechs=mechs)


def model(config, ncell, tstop):
    return hh_everywhere(build_config(5, ncell, tstop)) if config == "5hh" else build_config(config, ncell, tstop)


def run(spec, voltage, tstop, groups=1, resident=True):
    g = Sim()
    g.set_cell_groups(groups)
    g.set_solve_resident(resident)
    g.set_solve_voltage(voltage)
    mons = [("global", "v", c) for c in range(spec.ncell)]
    g.load_model_from_spec(dataclasses.replace(spec, monitors=mons))
    g.finitialize(-65.0)
    g.continue_run(tstop / 2)     # a duration
    g.continue_run(tstop / 2)
    return g


def oracle_traces(spec, tstop):
    o = oracle.OracleSim(spec, monitors=[("global", "v", c) for c in range(spec.ncell)])
    o.finitialize(-65.0)
    o.continue_run(tstop / 2)
    o.continue_run(tstop / 2)
    return o


@pytest.mark.parametrize("config,ncell,tstop,groups,resident", [
    (3, 2, 10.0, 1, True), (3, 16, 4.0, 2, True), ("5hh", 8, 20.0, 1, True), ("5hh", 24, 20.0, 2, True),
    ("5hh", 8, 20.0, 1, False)])
def test_voltage_form_matches_the_change_form(gpu_lib, config, ncell, tstop, groups, resident):
    spec = model(config, ncell, tstop)
    print(f"case solve voltage config={config} ncell={ncell} groups={groups} resident={resident}", flush=True)
    y = run(spec, True, tstop, groups, resident)
    x = run(spec, False, tstop, groups, resident)
    assert y.info("solve_voltage") == 1
    assert x.info("solve_voltage") == 0
    assert y.info("cell_groups") == groups
    assert y.info("solve_resident") == int(resident and config != 3)
    o = oracle_traces(spec, tstop)
    ey = float(np.max(np.abs(o.traces() - y.traces())))
    ex = float(np.max(np.abs(o.traces() - x.traces())))
    exy = float(np.max(np.abs(x.traces() - y.traces())))
    print(f"  |oracle - voltage form| {ey:.3e}  |oracle - change form| {ex:.3e}  between {exy:.3e}", flush=True)
    assert ey < V_TOL and ex < V_TOL
    assert exy < FORM_TOL
    sy, sx = y.spikes(), x.spikes()
    assert sorted(zip(sy[0], sy[1])) == sorted(zip(sx[0], sx[1]))
    ot, og = o.spikes()
    assert sorted(zip(sy[0], sy[1])) == sorted(zip(ot, og))
    # the call's last step leaves x = v_new - v in rhs and the pivots in d in both forms
    for k in ("rhs", "d", "v"):
        dev = float(np.max(np.abs(y.get_array("global", k) - x.get_array("global", k))))
        print(f"  {k}: between forms {dev:.3e}", flush=True)
        assert dev < FORM_TOL, (k, dev)
    assert float(np.max(np.abs(o.array("global", "rhs") - y.get_array("global", "rhs")))) < V_TOL


@pytest.mark.parametrize("config", [1, 4, 5])
def test_later_current_kernels_keep_the_change_form(gpu_lib, config):
    """IClamp (config 1), HalfGap (config 4) and hh on the somas only (config 5, on its own
    kernel) add to rhs or d after the node kernel."""
    spec = build_config(config, 4, 5.0)
    print(f"case solve voltage off config={config}", flush=True)
    g = run(spec, True, 5.0)
    assert g.info("solve_voltage") == 0


def test_switch_between_calls(gpu_lib):
    """The form may change between calls; each step uses one form throughout."""
    spec = model("5hh", 8, 20.0)
    print("case solve voltage switched between calls", flush=True)
    g = Sim()
    g.load_model_from_spec(dataclasses.replace(spec, monitors=[("global", "v", c) for c in range(8)]))
    g.finitialize(-65.0)
    g.continue_run(5.0)
    g.set_solve_voltage(False)
    assert g.info("solve_voltage") == 0
    g.continue_run(5.0)
    g.set_solve_voltage(True)
    assert g.info("solve_voltage") == 1
    g.continue_run(10.0)
    o = oracle_traces(spec, 20.0)
    assert float(np.max(np.abs(o.traces() - g.traces()))) < V_TOL
