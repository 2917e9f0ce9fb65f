"""Adjoint gradients on a model with config 4's features (gap junctions between somas,
an IClamp driven by VecPlay, detector netcons into ExpSyn synapses, hh on the somas and
pas everywhere) against central finite differences of the same loss computed with the
CPU oracle.  The IClamp's drive is raised so that its cell fires inside the window.

The loss is the mean over steps 1..N and cells of (soma v - target)^2, the target coming
from the same model with the gap conductances, the cells' g_pas and the netcon weights
scaled by U(0.8, 1.2).  Checked: the loss against the oracle's, the tied g_pas of two
cells, the gap conductance of the three most influential HalfGap instances, and the
three most influential netcon weights, each to 1e-6 relative."""
import copy

import numpy as np
import pytest

import oracle
from heliox_amd import Sim, build_config
from heliox_amd.synth import cell_rng

pytestmark = pytest.mark.gpu

NCELL = 16
TSTOP = 20.0
REL_TOL = 1e-6


def soma_trace(spec, tstop):
    mons = [("global", "v", i) for i in range(spec.ncell)]
    o = oracle.OracleSim(spec, monitors=mons)
    o.finitialize(-65.0)
    o.run(tstop)
    return o.traces()[:, 1:].T


def loss_of(spec, target):
    v = soma_trace(spec, TSTOP)
    return float(np.mean((v - target) ** 2))


def perturbed(spec, seed=7):
    out = copy.deepcopy(spec)
    rng = cell_rng(4, 0x5EED00 + seed)
    hg = out.mechs["HalfGap"]
    hg.params["g"] = hg.params["g"] * rng.uniform(0.8, 1.2, hg.n)
    cell = spec.cell_of_node()
    f = rng.uniform(0.8, 1.2, spec.ncell)
    pas = out.mechs["pas"]
    pas.params["g_pas"] = pas.params["g_pas"] * f[cell[pas.nodes]]
    nc = out.netcons["ExpSyn"]
    nc.weight = nc.weight * rng.uniform(0.8, 1.2, nc.weight.size)
    return out


def scaled(spec, mech, var, mask, factor):
    s = copy.deepcopy(spec)
    if mech == "ExpSyn":
        s.netcons["ExpSyn"].weight = np.where(mask, s.netcons["ExpSyn"].weight * factor, s.netcons["ExpSyn"].weight)
    else:
        p = s.mechs[mech].params
        p[var] = np.where(mask, p[var] * factor, p[var])
    return s


def fd_relative(spec, target, mech, var, mask, h=1e-4):
    lp = loss_of(scaled(spec, mech, var, mask, 1.0 + h), target)
    lm = loss_of(scaled(spec, mech, var, mask, 1.0 - h), target)
    return (lp - lm) / (2.0 * h)


def driven_model():
    """Config 4 at 16 cells with its VecPlay-driven IClamp raised to a 3 nA sinusoid, so the
    driven cell fires and its netcons deliver events inside the window."""
    base = build_config(4, NCELL, TSTOP)
    for vp in base.vecplay:
        vp.yvec = vp.yvec * 15.0
    return base


@pytest.fixture(scope="module")
def problem():
    base = driven_model()
    assert base.mechs["HalfGap"].n > 0 and len(base.vecplay) > 0
    target = soma_trace(perturbed(base), TSTOP)
    nstep = target.shape[0]
    g = Sim()
    g.load_model_from_spec(base, add_monitors=False)
    g.tape_begin(nstep)
    g.finitialize(-65.0)
    g.run(TSTOP)
    assert g.tape_length() == nstep
    loss = g.adjoint(np.arange(base.ncell), target)
    grads = {k: g.gradient(*k) for k in [("pas", "g_pas"), ("HalfGap", "g"), ("ExpSyn", "weight")]}
    return base, target, loss, grads


def test_loss_matches_oracle(problem):
    base, target, loss, _ = problem
    print("case adjoint network loss, config 4, 16 cells", flush=True)
    ref = loss_of(base, target)
    assert abs(loss - ref) <= 1e-9 * abs(ref)


def test_tied_pas_gradient_matches_fd(problem):
    base, target, _, grads = problem
    cell = base.cell_of_node()
    ms = base.mechs["pas"]
    vals = ms.params["g_pas"]
    for c in (0, 5):
        mask = cell[ms.nodes] == c
        adj = float(np.sum(vals[mask] * grads[("pas", "g_pas")][mask]))
        fd = fd_relative(base, target, "pas", "g_pas", mask)
        print(f"  g_pas cell {c}: adjoint {adj:.12e} fd {fd:.12e}", flush=True)
        assert abs(adj - fd) <= REL_TOL * abs(fd), (adj, fd)


def test_gap_conductance_gradients_match_fd(problem):
    base, target, _, grads = problem
    hg = base.mechs["HalfGap"]
    gg = grads[("HalfGap", "g")]
    infl = np.abs(gg * hg.params["g"])
    assert np.count_nonzero(infl) >= 3
    for j in np.argsort(-infl)[:3]:
        mask = np.arange(hg.n) == j
        adj = float(hg.params["g"][j] * gg[j])
        fd = fd_relative(base, target, "HalfGap", "g", mask)
        print(f"  HalfGap g {j}: adjoint {adj:.12e} fd {fd:.12e}", flush=True)
        assert fd != 0.0 and abs(adj - fd) <= REL_TOL * abs(fd), (j, adj, fd)


def test_netcon_weight_gradients_match_fd(problem):
    base, target, _, grads = problem
    nc = base.netcons["ExpSyn"]
    gw = grads[("ExpSyn", "weight")]
    infl = np.abs(gw[nc.inst] * nc.weight)
    assert np.count_nonzero(infl) >= 3, "too few synapses received events in the window"
    for k in np.argsort(-infl)[:3]:
        mask = np.arange(nc.weight.size) == k
        adj = float(nc.weight[k] * gw[nc.inst[k]])
        fd = fd_relative(base, target, "ExpSyn", "weight", mask)
        print(f"  weight {k}: adjoint {adj:.12e} fd {fd:.12e}", flush=True)
        assert fd != 0.0 and abs(adj - fd) <= REL_TOL * abs(fd), (k, adj, fd)
