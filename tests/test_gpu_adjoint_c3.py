"""Adjoint gradients on the headline model's mechanisms (config 3: hh, pas, Ih (hd_la),
Ca_HVA with CaDynamics_E2 and eca from cai every step, Exp2Syn driven by VecStim) against
central finite differences of the same loss through the CPU oracle.

One config-3 cell (5000 compartments), 25 ms.  Ca_HVA's gbar is raised tenfold so that
calcium, through ica -> cai -> eca, moves the soma voltage by much more than the
finite differences' own error.  The loss is the mean over steps and the soma of
(v - target)^2, the target coming from the same cell with gbar, ghdbar, gnabar and the
synaptic weights perturbed.  Tolerance: 1e-6 relative on every checked gradient."""
import copy

import numpy as np
import pytest

import oracle
from heliox_amd import Sim, build_config

pytestmark = pytest.mark.gpu

TSTOP = 25.0
REL_TOL = 1e-6


def base_model(variant):
    spec = build_config(3, 1, TSTOP)
    ch = spec.mechs["Ca_HVA"]
    ch.params["gbar"] = ch.params["gbar"] * 10.0
    if variant == "strong calcium":
        # calcium accumulates twenty times faster: cai rises several-fold within the run and
        # eca (Nernst every step) falls by tens of mV, so the cai -> eca feedback carries weight
        cd = spec.mechs["CaDynamics_E2"]
        cd.params["gamma"] = cd.params["gamma"] * 20.0
    elif variant == "fixed eca":
        ca = spec.mechs["ca_ion"]
        ca.iontype = np.full(ca.n, 0o4 | 0o40, np.int32)
    return spec


def perturbed(spec):
    out = copy.deepcopy(spec)
    rng = np.random.default_rng(33)
    out.mechs["Ca_HVA"].params["gbar"] *= 1.15
    out.mechs["hd_la"].params["ghdbar"] *= 0.9
    out.mechs["hh"].params["gnabar"] *= 1.1
    nc = out.netcons["Exp2Syn"]
    nc.weight = nc.weight * rng.uniform(0.8, 1.2, nc.weight.size)
    return out


def soma_trace(spec):
    o = oracle.OracleSim(spec, monitors=[("global", "v", 0)])
    o.finitialize(-65.0)
    o.run(TSTOP)
    return o.traces()[:, 1:].T


def loss_of(spec, target):
    return float(np.mean((soma_trace(spec) - target) ** 2))


def scaled(spec, mech, var, mask, factor):
    s = copy.deepcopy(spec)
    if var == "weight":
        nc = s.netcons[mech]
        nc.weight = np.where(mask, nc.weight * factor, nc.weight)
    else:
        p = s.mechs[mech].params
        p[var] = np.where(mask, p[var] * factor, p[var])
    return s


def fd_relative(spec, target, mech, var, mask, h=1e-4):
    lp = loss_of(scaled(spec, mech, var, mask, 1.0 + h), target)
    lm = loss_of(scaled(spec, mech, var, mask, 1.0 - h), target)
    return (lp - lm) / (2.0 * h)


TIED = [("Ca_HVA", "gbar"), ("hd_la", "ghdbar"), ("hh", "gnabar"), ("hh", "gkbar"), ("pas", "g_pas")]


@pytest.fixture(scope="module", params=["config 3", "strong calcium", "fixed eca"])
def problem(request, gpu_lib):
    base = base_model(request.param)
    print(f"case config-3 adjoint, {request.param}", flush=True)
    target = soma_trace(perturbed(base))
    nstep = target.shape[0]
    g = Sim()
    g.load_model_from_spec(base, add_monitors=False)
    g.tape_begin(nstep)
    g.finitialize(-65.0)
    g.run(TSTOP)
    assert g.tape_length() == nstep
    loss = g.adjoint(np.array([0]), target)
    grads = {k: g.gradient(*k) for k in TIED + [("Exp2Syn", "weight")]}
    return base, target, loss, grads, g


def test_loss_matches_oracle(problem):
    base, target, loss, _, _ = problem
    ref = loss_of(base, target)
    print(f"case config-3 adjoint loss {loss:.12e} oracle {ref:.12e}", flush=True)
    assert abs(loss - ref) <= 1e-9 * abs(ref)


@pytest.mark.parametrize("mech,var", TIED)
def test_tied_gradients_match_fd(problem, mech, var):
    base, target, _, grads, _ = problem
    vals = base.mechs[mech].params[var]
    mask = np.ones(vals.size, bool)
    adj = float(np.sum(vals * grads[(mech, var)]))     # d/d alpha of param *= (1 + alpha)
    fd = fd_relative(base, target, mech, var, mask)
    print(f"  {mech}.{var}: adjoint {adj:.12e} fd {fd:.12e}", flush=True)
    assert fd != 0.0 and abs(adj - fd) <= REL_TOL * abs(fd), (adj, fd)


def test_exp2syn_weight_gradients_match_fd(problem):
    base, target, _, grads, _ = problem
    nc = base.netcons["Exp2Syn"]
    gw = grads[("Exp2Syn", "weight")]
    infl = np.abs(gw[nc.inst] * nc.weight)
    assert np.count_nonzero(infl) >= 4, "too few synapses received events in the window"
    for k in np.argsort(-infl)[:4]:
        mask = np.arange(nc.weight.size) == k
        adj = float(nc.weight[k] * gw[nc.inst[k]])
        fd = fd_relative(base, target, "Exp2Syn", "weight", mask)
        print(f"  Exp2Syn weight {k}: adjoint {adj:.12e} fd {fd:.12e}", flush=True)
        assert fd != 0.0 and abs(adj - fd) <= REL_TOL * abs(fd), (k, adj, fd)
    quiet = np.nonzero(infl == 0)[0]
    if quiet.size:
        assert fd_relative(base, target, "Exp2Syn", "weight", np.arange(nc.weight.size) == quiet[0]) == 0.0


def test_node_parallel_kernels_give_the_same_bits(problem):
    """Every density mechanism of this model has an instance on every node, so the backward
    step runs them and the synapses in its two node-parallel kernels; each mechanism's own kernels
    (hx_set_fusion(0)) give the same loss and gradients, bit for bit, on the same tape."""
    _, target, loss, grads, g = problem
    every = 0b1111                      # pas, hh, Ca_HVA, hd_la
    gates = 0b11110                     # hh, Ca_HVA, hd_la and CaDynamics_E2
    synapses = 1 << 24                  # Exp2Syn's decay, conductance and parameter terms too
    loss_term = 1 << 25                 # and the loss term
    assert g.info("adjoint_fused") == (gates | every << 8 | every << 16 | synapses | loss_term), \
        hex(g.info("adjoint_fused"))
    g.set_fusion(False)
    try:
        loss2 = g.adjoint(np.array([0]), target)
        assert g.info("adjoint_fused") == 0
        assert loss2 == loss
        for k, v in grads.items():
            np.testing.assert_array_equal(g.gradient(*k), v, err_msg=str(k))
    finally:
        g.set_fusion(True)
    assert g.adjoint(np.array([0]), target) == loss
