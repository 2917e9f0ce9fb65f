"""Configuration 4 at full size (10,000 cells x 200 compartments, 1e6 netcons, 500 gap
pairs, VecPlay into 500 cells) against the oracle, with every cell driven to fire at
about the same time and every netcon delay set to 1 ms, so the deliveries of one burst
land on the same few steps (up to a million events in a step).  ExpSyn conductances do
not decay here (tau 1e9 ms), so each synapse's g / w counts the events it received."""
import numpy as np
import pytest

from heliox_amd.spec import MechSpec
from heliox_amd import build_config
from parity_util import V_TOL, compare_spikes, run_both

pytestmark = pytest.mark.gpu


def burst_network(ncell=10000, tstop=3.0):
    spec = build_config(4, ncell, tstop)
    nc = spec.netcons["ExpSyn"]
    nc.delay = np.full(nc.delay.size, 1.0)
    es = spec.mechs["ExpSyn"]
    es.params["tau"] = np.full(es.n, 1e9)
    ic = spec.mechs["IClamp"]
    soma = np.arange(ncell, dtype=np.int32)
    spec.mechs["IClamp"] = MechSpec(np.concatenate([ic.nodes, soma]),
                                    {"delay": np.concatenate([ic.params["delay"], np.full(ncell, 0.1)]),
                                     "dur": np.concatenate([ic.params["dur"], np.full(ncell, 0.5)]),
                                     "amp": np.concatenate([ic.params["amp"], np.full(ncell, 2.0)])})
    spec.monitors = [("global", "v", int(c)) for c in range(0, ncell, 200)]
    return spec


def test_full_size_burst_matches_oracle(gpu_lib):
    tstop, dt = 3.0, 0.025
    spec = burst_network(tstop=tstop)
    nc = spec.netcons["ExpSyn"]
    print(f"case config 4 full size burst: {spec.ncell} cells, {spec.nnode} nodes, {nc.inst.size} netcons", flush=True)
    o, g = run_both(spec, tstop)
    nspk = compare_spikes(o, g, dt)
    assert nspk >= 0.9 * spec.ncell, "the pulse should make almost every cell fire"
    err = float(np.max(np.abs(o.traces() - g.traces())))
    print(f"  spikes {nspk}, max |dv| {err:.3e} mV", flush=True)
    assert err < V_TOL
    go, gg = o.array("ExpSyn", "g"), g.get_array("ExpSyn", "g")
    assert np.max(np.abs(go - gg)) <= 1e-12 * max(1.0, float(np.max(np.abs(go))))
    # delivered events: each synapse's g / w against the spikes of its source x fan-out
    w = np.zeros(spec.mechs["ExpSyn"].n)
    w[nc.inst] = nc.weight
    got = int(np.rint(gg / w).sum())
    t_spk, gid = g.spikes()
    gid_to_pre = {int(x): i for i, x in enumerate(spec.presyn_gid)}
    fanout = np.bincount(nc.src[nc.src_kind == 0], minlength=spec.presyn_gid.size)
    last = (int(round(tstop / dt)) - 1) * dt     # start time of the last step, which delivers up to last + dt/2
    due = t_spk + 1.0 <= last + dt / 2
    expected = int(sum(fanout[gid_to_pre[int(x)]] for x in gid[due]))
    print(f"  deliveries {got} (expected {expected}) from {int(due.sum())} spikes", flush=True)
    assert expected > 500000 and got == expected
