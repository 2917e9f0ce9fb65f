"""Writes the golden fixtures of this directory from the CPU oracle.

    python tests/golden/make_fixtures.py

Each fixture is an .npz of plain arrays (no pickled objects): the model is
rebuilt by heliox_amd.build_config from (config, ncell, tstop), so a fixture
holds only the run's outputs.  The tests compare the oracle (CPU suite) and the
HIP path (GPU suite) against these files, so a change to either that moves a
result shows up against a fixed record.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402
from heliox_amd import build_config  # noqa: E402

# (name, config, ncell, tstop, monitored variables)
TRACE_CASES = [
    ("c1_3cells_60ms", 1, 3, 60.0, [("global", "v", i) for i in range(3)] + [("hh", "m", 0), ("hh", "n", 2)]),
    ("c2_2cells_40ms", 2, 2, 40.0, [("global", "v", i) for i in range(2)] + [("ExpSyn", "g", 3)]),
    ("c3_1cell_15ms", 3, 1, 15.0, [("global", "v", 0), ("hd_la", "l", 100), ("ca_ion", "conci", 7),
                                    ("Exp2Syn", "A", 5)]),
]
# (name, config, ncell, steps): node arrays after finitialize and after the given steps
STATE_CASES = [
    ("c3_1cell_state", 3, 1, 40),
]


def trace_case(config, ncell, tstop, mons):
    spec = build_config(config, ncell, tstop)
    o = oracle.OracleSim(spec, monitors=mons)
    o.finitialize(-65.0)
    o.run(tstop)
    st, sg = o.spikes()
    return {"traces": o.traces(), "spike_t": st, "spike_gid": sg,
            "monitors": np.array(["%s.%s[%d]" % m for m in mons])}


def state_case(config, ncell, nstep):
    spec = build_config(config, ncell, nstep * spec_dt(config) + 1.0)
    o = oracle.OracleSim(spec, monitors=[])
    o.finitialize(-65.0)
    out = {"v_init": o.array("global", "v").copy(), "d_init": o.array("global", "d").copy(),
           "rhs_init": o.array("global", "rhs").copy()}
    o.nsteps(nstep)
    out.update({"v": o.array("global", "v"), "hh_m": o.array("hh", "m"), "hh_h": o.array("hh", "h"),
                "hh_n": o.array("hh", "n"), "cahva_m": o.array("Ca_HVA", "m"), "hd_l": o.array("hd_la", "l"),
                "cai": o.array("ca_ion", "conci"), "e2_A": o.array("Exp2Syn", "A"), "e2_B": o.array("Exp2Syn", "B")})
    return out


def spec_dt(config):
    return build_config(config, 1, 1.0).dt


def adam_case():
    rng = np.random.default_rng(11)
    w = rng.normal(size=5)
    gsz = np.array([1, 3, 2, 1, 4], np.int32)
    m = np.zeros(5)
    v = np.zeros(5)
    grads = rng.normal(size=(3, gsz.sum()))
    ws = [w.copy()]
    for step in range(1, 4):
        oracle.adam_step(w, grads[step - 1], gsz, m, v, step, 1e-3, 0.5, 2.0)
        ws.append(w.copy())
    return {"w": np.array(ws), "grads": grads, "group_size": gsz, "m": m, "v": v}


def main():
    oracle.build()
    for name, config, ncell, tstop, mons in TRACE_CASES:
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **trace_case(config, ncell, tstop, mons))
    for name, config, ncell, nstep in STATE_CASES:
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **state_case(config, ncell, nstep))
    np.savez_compressed(os.path.join(HERE, "adam_3steps.npz"), **adam_case())
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))


if __name__ == "__main__":
    main()
