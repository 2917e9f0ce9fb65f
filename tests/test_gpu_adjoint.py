"""Adjoint (VJP) gradients of the config-5 loss on the GPU against central finite
differences of the same loss computed with the CPU oracle, and the device Adam
step against the Kingma-Ba update.

The loss is the mean over steps 1..N and cells of (soma v - target)^2, the
target coming from the config-5 model with perturbed parameters.  Tolerance:
1e-6 relative on every checked gradient."""
import copy

import numpy as np
import pytest

import oracle
from heliox_amd import Sim, build_config
from heliox_amd.synth import perturb_config5

pytestmark = pytest.mark.gpu

NCELL = 2
TSTOP = 40.0
REL_TOL = 1e-6


def soma_trace(spec, tstop):
    mons = [("global", "v", i) for i in range(spec.ncell)]
    o = oracle.OracleSim(spec, monitors=mons)
    o.finitialize(-65.0)
    o.run(tstop)
    return o.traces()[:, 1:].T          # samples after steps 1..N, shape (N, ncell)


def loss_of(spec, target, tstop):
    v = soma_trace(spec, tstop)
    return float(np.mean((v - target) ** 2))


@pytest.fixture(scope="module")
def problem():
    base = build_config(5, NCELL, TSTOP)
    target = soma_trace(perturb_config5(base, seed=3), TSTOP)
    nstep = target.shape[0]
    g = Sim()
    g.load_model_from_spec(base, add_monitors=False)
    g.tape_begin(nstep)
    g.finitialize(-65.0)
    g.run(TSTOP)
    assert g.tape_length() == nstep
    loss = g.adjoint(np.arange(base.ncell), target)
    grads = {k: g.gradient(*k) for k in [("hh", "gnabar"), ("hh", "gkbar"), ("pas", "g_pas"), ("ExpSyn", "weight")]}
    return base, target, loss, grads, g


def scaled(spec, mech, var, mask, factor):
    s = copy.deepcopy(spec)
    if mech == "ExpSyn":
        s.netcons["ExpSyn"].weight = np.where(mask, s.netcons["ExpSyn"].weight * factor,
                                              s.netcons["ExpSyn"].weight)
    else:
        p = s.mechs[mech].params
        p[var] = np.where(mask, p[var] * factor, p[var])
    return s


def fd_relative(spec, target, mech, var, mask, h=1e-4):
    """d loss / d alpha for param *= (1 + alpha) on the masked instances."""
    lp = loss_of(scaled(spec, mech, var, mask, 1.0 + h), target, TSTOP)
    lm = loss_of(scaled(spec, mech, var, mask, 1.0 - h), target, TSTOP)
    return (lp - lm) / (2.0 * h)


def test_loss_matches_oracle(problem):
    base, target, loss, _, _ = problem
    ref = loss_of(base, target, TSTOP)
    assert abs(loss - ref) <= 1e-9 * abs(ref)


@pytest.mark.parametrize("mech,var", [("hh", "gnabar"), ("hh", "gkbar"), ("pas", "g_pas")])
def test_tied_conductance_gradients_match_fd(problem, mech, var):
    base, target, _, grads, _ = problem
    cell = base.cell_of_node()
    ms = base.mechs[mech]
    vals = ms.params[var]
    for c in range(base.ncell):
        mask = cell[ms.nodes] == c
        adj = float(np.sum(vals[mask] * grads[(mech, var)][mask]))   # d/d alpha of the tied scale
        fd = fd_relative(base, target, mech, var, mask)
        print(f"  {mech}.{var} cell {c}: adjoint {adj:.12e} fd {fd:.12e}", flush=True)
        assert abs(adj - fd) <= REL_TOL * abs(fd), (adj, fd)


def test_synaptic_weight_gradients_match_fd(problem):
    base, target, _, grads, _ = problem
    nc = base.netcons["ExpSyn"]
    gw = grads[("ExpSyn", "weight")]
    checked = 0
    infl = np.abs(gw[nc.inst] * nc.weight)
    assert np.count_nonzero(infl) >= 4, "too few synapses received events in the window"
    for k in np.argsort(-infl)[:4]:   # the four most influential weights
        mask = np.arange(nc.weight.size) == k
        adj = float(nc.weight[k] * gw[nc.inst[k]])
        fd = fd_relative(base, target, "ExpSyn", "weight", mask)
        print(f"  weight {k}: adjoint {adj:.12e} fd {fd:.12e}", flush=True)
        assert fd != 0.0 and abs(adj - fd) <= REL_TOL * abs(fd), (k, adj, fd)
        checked += 1
    assert checked == 4
    # a synapse that received no event in the window has no gradient
    quiet = np.nonzero(infl == 0)[0]
    if quiet.size:
        k = quiet[0]
        assert fd_relative(base, target, "ExpSyn", "weight", np.arange(nc.weight.size) == k) == 0.0


def test_node_parallel_kernels_give_the_same_bits(problem):
    """pas is on every node and hh on the somas only: the backward step's node-parallel
    kernels take pas's conductance and parameter term, hh keeps its own kernels.  Each
    mechanism's own kernels (hx_set_fusion(0)) give the same bits on the same tape."""
    base, target, loss, grads, g = problem
    assert g.info("adjoint_fused") == (1 << 8 | 1 << 16 | 1 << 25), hex(g.info("adjoint_fused"))
    g.set_fusion(False)
    try:
        loss2 = g.adjoint(np.arange(base.ncell), target)
        assert g.info("adjoint_fused") == 0
        assert loss2 == loss
        for k, v in grads.items():
            np.testing.assert_array_equal(g.gradient(*k), v, err_msg=str(k))
    finally:
        g.set_fusion(True)
    assert g.adjoint(np.arange(base.ncell), target) == loss


def test_adam_step_on_tied_groups(problem):
    base, _, _, grads, g = problem
    cell = base.cell_of_node()
    hh = base.mechs["hh"]
    opt = g.adam_create(0.9, 0.999, 1e-8)
    groups = [np.nonzero(cell[hh.nodes] == c)[0] for c in range(base.ncell)]
    for inst in groups:
        g.adam_add_group(opt, "hh", "gnabar", inst, impedance=1.0)
    w0 = g.get_array("hh", "gnabar").copy()
    lr, inv = 1e-3, 0.5
    g.adam_step(opt, lr, inv)
    w1 = g.get_array("hh", "gnabar")
    # the same update from the oracle's restatement of AdamOptimizer::step_cpu
    ww = np.array([w0[i[0]] for i in groups])
    gsz = np.array([i.size for i in groups], np.int32)
    m = np.zeros(len(groups))
    v = np.zeros(len(groups))
    oracle.adam_step(ww, np.concatenate([grads[("hh", "gnabar")][i] for i in groups]), gsz, m, v, 1, lr, inv)
    for k, inst in enumerate(groups):
        assert np.allclose(w1[inst], ww[k], rtol=1e-14, atol=0)
    step, mg, vg = g.adam_state(opt, len(groups))
    assert step == 1 and np.allclose(mg, m, rtol=1e-14) and np.allclose(vg, v, rtol=1e-14)
    # a step zeroes the gradients it used: a second step only decays the moments
    g.adam_step(opt, lr, inv)
    _, mg2, _ = g.adam_state(opt, len(groups))
    assert np.allclose(mg2, 0.9 * mg, rtol=1e-14)


def test_repeated_loss_node_matches_fd(problem):
    """A node listed twice in the loss counts twice: soma 0 appears as loss columns 0 and
    2 with different targets; the gradient matches the oracle's finite differences of the
    same loss, and the loss the host reports."""
    base, target, _, _, _ = problem
    nodes = np.array([0, 1, 0])
    tgt = np.stack([target[:, 0], target[:, 1], target[:, 0] + 0.7], axis=1)
    nstep = target.shape[0]
    g = Sim()
    g.load_model_from_spec(base, add_monitors=False)
    g.tape_begin(nstep)
    g.finitialize(-65.0)
    g.run(TSTOP)
    loss = g.adjoint(nodes, tgt)
    grad = g.gradient("hh", "gnabar")

    def loss_rep(spec):
        v = soma_trace(spec, TSTOP)[:, nodes]
        return float(np.mean((v - tgt) ** 2))

    assert abs(loss - loss_rep(base)) <= 1e-9 * abs(loss)
    cell = base.cell_of_node()
    hh = base.mechs["hh"]
    for c in range(base.ncell):
        mask = cell[hh.nodes] == c
        adj = float(np.sum(hh.params["gnabar"][mask] * grad[mask]))
        h = 1e-4
        fd = (loss_rep(scaled(base, "hh", "gnabar", mask, 1 + h)) -
              loss_rep(scaled(base, "hh", "gnabar", mask, 1 - h))) / (2 * h)
        print(f"  repeated loss node, hh.gnabar cell {c}: adjoint {adj:.12e} fd {fd:.12e}", flush=True)
        assert abs(adj - fd) <= REL_TOL * abs(fd), (adj, fd)


def test_training_loop_holds_its_device_memory(problem):
    """Twenty tape / run / adjoint / optimizer cycles after two warm-up cycles leave the
    free device memory where it was: the per-call buffers are reused."""
    from parity_util import device_free_bytes

    base, target, _, _, _ = problem
    nstep = target.shape[0]
    g = Sim()
    g.load_model_from_spec(base, add_monitors=False)
    opt = g.adam_create(0.9, 0.999, 1e-8)
    cell = base.cell_of_node()
    hh = base.mechs["hh"]
    for c in range(base.ncell):
        g.adam_add_group(opt, "hh", "gnabar", np.nonzero(cell[hh.nodes] == c)[0], impedance=1.0)

    def cycle():
        g.tape_begin(nstep)
        g.finitialize(-65.0)
        g.run(TSTOP)
        g.adjoint(np.arange(base.ncell), target)
        g.adam_step(opt, 1e-6, 1.0)

    cycle()
    cycle()
    free0 = device_free_bytes()
    for _ in range(20):
        cycle()
    free1 = device_free_bytes()
    print(f"  free device memory before {free0} after {free1}", flush=True)
    assert free1 == free0


def test_full_tape_stops_before_the_step(gpu_lib):
    """A run longer than the tape stops at the first step that would not fit, before that
    step issues anything: the tape holds its steps and the backward sweep runs on them."""
    spec = build_config(5, 2, 5.0)
    g = Sim()
    g.load_model_from_spec(spec, add_monitors=False)
    g.tape_begin(10)
    g.finitialize(-65.0)
    with pytest.raises(Exception, match="tape full"):
        g.run(1.0)
    assert g.tape_length() == 10
    loss = g.adjoint(np.arange(spec.ncell), np.full((10, spec.ncell), -65.0))
    assert np.isfinite(loss)
    assert np.all(np.isfinite(g.gradient("pas", "g_pas")))
