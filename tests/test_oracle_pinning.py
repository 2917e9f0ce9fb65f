"""Pin the CPU oracle against mathematics it must reproduce.

The reference ships no golden vectors for this path (its tests need NEURON and a
CUDA build), so each oracle function is checked against a closed form, an
independent textbook restatement, an invariant, or brute force -- chosen so that
a plausible transcription mistake (sign, index, dropped term, swapped operand)
fails.
"""
import math

import numpy as np
import pytest

import oracle
from heliox_amd.spec import MechSpec, ModelSpec, NetConSpec, VecPlaySpec

F = 1.602176634e-19 * 6.02214076e23
R = 1.380649e-23 * 6.02214076e23


def single_compartment(area=1000.0, cm=1.0, dt=0.025, celsius=6.3):
    return ModelSpec(ncell=1, parent=np.array([-1], np.int32), a=np.zeros(1), b=np.zeros(1),
                     area=np.array([area]), cm=np.array([cm]), dt=dt, celsius=celsius)


# ---------------------------------------------------------------------------
# tree solve (simulate.cpp:558-581)
# ---------------------------------------------------------------------------
def random_forest(rng, ncell, n):
    parent = -np.ones(n, np.int32)
    for i in range(ncell, n):
        parent[i] = rng.integers(0, i)
    a = -rng.uniform(0.1, 2.0, n)
    b = -rng.uniform(0.1, 2.0, n)
    a[:ncell] = 0
    b[:ncell] = 0
    return parent, a, b


def dense_matrix(parent, a, b, d):
    n = len(parent)
    M = np.diag(d.copy())
    for i in range(n):
        p = parent[i]
        if p >= 0:
            M[i, p] = b[i]
            M[p, i] = a[i]
    return M


@pytest.mark.parametrize("seed", range(6))
def test_solve_serial_equals_dense_solve(seed):
    rng = np.random.default_rng(seed)
    ncell = int(rng.integers(1, 4))
    n = int(rng.integers(ncell + 1, 64))
    parent, a, b = random_forest(rng, ncell, n)
    # the reference's matrix: d holds the full diagonal, a/b the off-diagonals
    d = rng.uniform(5.0, 10.0, n)
    rhs = rng.normal(size=n)
    x = oracle.solve_serial(ncell, parent, a, b, d, rhs)
    x_dense = np.linalg.solve(dense_matrix(parent, a, b, d), rhs)
    assert np.allclose(x, x_dense, rtol=1e-12, atol=1e-12)


def test_solve_serial_single_node():
    x = oracle.solve_serial(1, np.array([-1]), np.zeros(1), np.zeros(1), np.array([4.0]), np.array([2.0]))
    assert x[0] == 0.5


def test_solve_serial_relabel_invariant():
    """Renumbering nodes (keeping parent < child) permutes the solution."""
    rng = np.random.default_rng(7)
    n = 40
    parent, a, b = random_forest(rng, 1, n)
    d = rng.uniform(5, 9, n)
    rhs = rng.normal(size=n)
    x = oracle.solve_serial(1, parent, a, b, d, rhs)
    # a different topological order: breadth-first relabelling
    children = [[] for _ in range(n)]
    for i in range(1, n):
        children[parent[i]].append(i)
    order = [0]
    for u in order:
        order.extend(children[u][::-1])
    new = np.empty(n, int)
    new[order] = np.arange(n)
    p2 = np.array([-1] + [new[parent[u]] for u in order[1:]], np.int32)
    x2 = oracle.solve_serial(1, p2, a[order], b[order], d[order], rhs[order])
    assert np.allclose(x2, x[order], rtol=1e-12)


# ---------------------------------------------------------------------------
# passive compartment + IClamp (capacitance capac.cpp:54-80, backward Euler)
# ---------------------------------------------------------------------------
def test_passive_iclamp_backward_euler_closed_form():
    dt, area, cm, g, e, amp = 0.025, 800.0, 1.3, 2e-4, -70.0, 0.2
    spec = single_compartment(area=area, cm=cm, dt=dt)
    spec.mechs["pas"] = MechSpec(np.array([0], np.int32), {"g_pas": np.array([g]), "e_pas": np.array([e])})
    spec.mechs["IClamp"] = MechSpec(np.array([0], np.int32), {"delay": np.array([1.0]), "dur": np.array([2.0]),
                                                              "amp": np.array([amp])})
    spec.monitors = [("global", "v", 0)]
    o = oracle.OracleSim(spec)
    o.finitialize(-65.0)
    o.run(5.0)
    v = o.traces()[0]
    cfac = 1e-3 / dt
    iscale = amp * 1e2 / area
    vv, t, ref = -65.0, 0.0, [-65.0]
    for _ in range(len(v) - 1):
        tmid = t + 0.5 * dt
        inj = iscale if (1.0 <= tmid < 3.0) else 0.0
        vv = (cfac * cm * vv + g * e + inj) / (g + cfac * cm)
        t = tmid + 0.5 * dt
        ref.append(vv)
    assert np.allclose(v, ref, rtol=0, atol=1e-10)


def test_iclamp_window_on_exact_step_times():
    """The pulse is on while the mid-step time t satisfies del <= t < del + dur
    (iclamp.cu:18).  With dt = 1/32 every mid-step time is exact in binary, so del and
    del + dur can sit exactly on mid-step times: the pulse then covers steps 10..15 and
    no other, which the capacitor charging C dv/dt = I (pas with g = 0) shows one step
    at a time."""
    dt, area, cm, amp = 1.0 / 32, 500.0, 1.0, 0.004
    spec = single_compartment(area=area, cm=cm, dt=dt)
    n = np.array([0], np.int32)
    spec.mechs["pas"] = MechSpec(n, {"g_pas": np.array([0.0]), "e_pas": np.array([-65.0])})
    spec.mechs["IClamp"] = MechSpec(n.copy(), {"delay": np.array([10.5 * dt]), "dur": np.array([6 * dt]),
                                               "amp": np.array([amp])})
    spec.monitors = [("global", "v", 0)]
    o = oracle.OracleSim(spec)
    o.finitialize(-65.0)
    o.run(24 * dt)
    v = o.traces()[0]
    step = amp * 1e2 / area / (1e-3 / dt * cm)
    expect = [-65.0]
    for k in range(24):
        expect.append(expect[-1] + (step if 10 <= k <= 15 else 0.0))
    assert len(v) == 25
    assert np.allclose(v, expect, rtol=0, atol=1e-12)
    assert v[10] == -65.0 and v[11] > -65.0 and v[16] == v[17] == v[24]


def test_sealed_cable_steady_state():
    """A long passive cable with current injected at one end reaches the
    analytic sealed-end profile V(x) ~ cosh((L - x)/lambda) / cosh(L/lambda)."""
    nseg, L, diam, Ra, g, e = 200, 1000.0, 2.0, 100.0, 1e-4, -65.0
    dx = L / nseg
    area = np.full(nseg, math.pi * diam * dx)
    rhalf = 1e-2 * Ra * (dx / 2) / (math.pi * (diam / 2) ** 2)
    gax = 1.0 / (2 * rhalf)
    parent = np.arange(-1, nseg - 1, dtype=np.int32)
    a = np.full(nseg, -1e2 * gax / area[0])
    b = np.full(nseg, -1e2 * gax / area[0])
    a[0] = b[0] = 0
    spec = ModelSpec(ncell=1, parent=parent, a=a, b=b, area=area, cm=np.ones(nseg), dt=0.1)
    spec.mechs["pas"] = MechSpec(np.arange(nseg, dtype=np.int32), {"g_pas": np.full(nseg, g), "e_pas": np.full(nseg, e)})
    spec.mechs["IClamp"] = MechSpec(np.array([0], np.int32), {"delay": np.array([0.0]), "dur": np.array([1e9]),
                                                              "amp": np.array([0.05])})
    o = oracle.OracleSim(spec, monitors=[])
    o.finitialize(e)
    o.run(500.0)
    v = o.array("global", "v") - e
    lam = math.sqrt((diam * 1e-4) / (4 * Ra * g)) * 1e4     # um
    x = (np.arange(nseg) + 0.5) * dx
    shape = np.cosh((L - x) / lam)
    shape = shape / shape[0] * v[0]
    assert np.max(np.abs(v - shape)) / v[0] < 2e-2


# ---------------------------------------------------------------------------
# axial assembly with unequal areas (simulate.cpp:541-554): a[i] carries the
# parent's area and b[i] the node's own, so every check below has a != b
# ---------------------------------------------------------------------------
def axial_coefficients(parent, gax, area):
    """The model arrays for edge conductances gax[i] (uS, node i to its parent):
    a[i] = -1e2 gax / area[parent], b[i] = -1e2 gax / area[i]."""
    a = np.zeros(len(parent))
    b = np.zeros(len(parent))
    for i, p in enumerate(parent):
        if p >= 0:
            a[i] = -1e2 * gax[i] / area[p]
            b[i] = -1e2 * gax[i] / area[i]
    return a, b


def physics_step(parent, gax, area, cm, gpas, epas, v, inj, dt):
    """One backward-Euler step written from the membrane equation of each
    compartment k (current densities in mA/cm2, areas in um2, gax in uS):
        1e-3 cm_k (v'_k - v_k) / dt = -gpas (v'_k - e) + sum_j 1e2 gax_kj / A_k (v'_j - v'_k) + inj_k
    solved as a dense linear system."""
    n = len(parent)
    M = np.diag(1e-3 * cm / dt + gpas)
    r = 1e-3 * cm / dt * v + gpas * epas + inj
    for i, p in enumerate(parent):
        if p < 0:
            continue
        for k, j in ((i, p), (p, i)):
            c = 1e2 * gax[i] / area[k]
            M[k, k] += c
            M[k, j] -= c
    return np.linalg.solve(M, r)


def passive_tree_spec(parent, gax, area, cm, gpas, epas, amp, dt):
    a, b = axial_coefficients(parent, gax, area)
    n = len(parent)
    spec = ModelSpec(ncell=1, parent=np.asarray(parent, np.int32), a=a, b=b, area=np.asarray(area, float),
                     cm=np.asarray(cm, float), dt=dt)
    spec.mechs["pas"] = MechSpec(np.arange(n, dtype=np.int32), {"g_pas": np.full(n, gpas), "e_pas": np.full(n, epas)})
    spec.mechs["IClamp"] = MechSpec(np.array([0], np.int32), {"delay": np.array([0.5]), "dur": np.array([1.0]),
                                                              "amp": np.array([amp])})
    return spec


def test_two_compartments_unequal_areas_backward_euler():
    """Soma (A0) and one dendritic compartment (A1 = A0 / 5) coupled by gax:
    each compartment's coupling term is 1e2 gax / A_k, so the two rows differ
    by the area ratio; IClamp at the soma from 0.5 to 1.5 ms."""
    dt, gax, gpas, epas, amp = 0.025, 0.03, 2e-4, -70.0, 0.4
    parent, area, cm = [-1, 0], np.array([1500.0, 300.0]), np.array([1.0, 1.7])
    spec = passive_tree_spec(parent, [0.0, gax], area, cm, gpas, epas, amp, dt)
    spec.monitors = [("global", "v", 0), ("global", "v", 1)]
    o = oracle.OracleSim(spec)
    o.finitialize(-62.0)
    o.run(2.0)
    got = o.traces()
    # the two rows written out by hand
    v, t, ref = np.array([-62.0, -62.0]), 0.0, [np.array([-62.0, -62.0])]
    c0, c1 = 1e-3 * cm / dt
    g0, g1 = 1e2 * gax / area[0], 1e2 * gax / area[1]
    for _ in range(got.shape[1] - 1):
        tmid = t + 0.5 * dt
        inj = amp * 1e2 / area[0] if 0.5 <= tmid < 1.5 else 0.0
        M = np.array([[c0 + gpas + g0, -g0], [-g1, c1 + gpas + g1]])
        v = np.linalg.solve(M, [c0 * v[0] + gpas * epas + inj, c1 * v[1] + gpas * epas])
        t = tmid + 0.5 * dt
        ref.append(v)
    ref = np.array(ref).T
    assert np.max(np.abs(got - ref)) < 1e-10
    # the dendrite moved, and far more than the tolerance
    assert abs(got[1].max() - got[1, 0]) > 1.0


def tapered_tree(rng, n):
    parent = np.array([-1] + [int(rng.integers(max(0, i - 4), i)) for i in range(1, n)], np.int32)
    diam = np.linspace(4.0, 0.5, n) * rng.uniform(0.8, 1.2, n)
    L = rng.uniform(5.0, 40.0, n)
    area = math.pi * diam * L
    Ra = 150.0
    gax = np.zeros(n)
    for i in range(1, n):
        # half-segment resistances in series (Mohm), conductance in uS
        r = 1e-2 * Ra * (L[i] / 2 / (math.pi * (diam[i] / 2) ** 2) + L[parent[i]] / 2 / (math.pi * (diam[parent[i]] / 2) ** 2))
        gax[i] = 1.0 / r
    return parent, gax, area


@pytest.mark.parametrize("seed", range(3))
def test_tapered_tree_backward_euler_and_charge_conservation(seed):
    """A branched tree with tapering diameters (a != b on every edge): every
    step equals the dense backward-Euler solve of the membrane equations, and
    the area-weighted sum of capacitive and membrane currents equals the
    injected current (the axial currents cancel in pairs)."""
    rng = np.random.default_rng(seed)
    n, dt, gpas, epas, amp = 40, 0.025, 1e-4, -65.0, 0.3
    parent, gax, area = tapered_tree(rng, n)
    cm = rng.uniform(0.8, 2.0, n)
    spec = passive_tree_spec(parent, gax, area, cm, gpas, epas, amp, dt)
    o = oracle.OracleSim(spec, monitors=[])
    o.finitialize(-60.0)
    v = o.array("global", "v").copy()
    t = 0.0
    for step in range(80):
        tmid = t + 0.5 * dt
        on = 0.5 <= tmid < 1.5
        inj = np.zeros(n)
        inj[0] = amp * 1e2 / area[0] if on else 0.0
        o.fadvance()
        got = o.array("global", "v").copy()
        ref = physics_step(parent, gax, area, cm, gpas, epas, v, inj, dt)
        assert np.max(np.abs(got - ref)) < 1e-10, step
        # sum_k A_k (C dv/dt + I_m) = injected current (um2 mA/cm2 = 1e-2 nA)
        imem = 1e-3 * cm * (got - v) / dt + gpas * (got - epas)
        total = float(np.sum(area * imem)) * 1e-2
        assert abs(total - (amp if on else 0.0)) < 1e-9 * max(1.0, float(np.sum(area * np.abs(imem))) * 1e-2), step
        v, t = got, tmid + 0.5 * dt
    assert np.max(np.abs(v - (-60.0))) > 0.1


# ---------------------------------------------------------------------------
# hh (hh_templated.cu) against the textbook Hodgkin-Huxley rate functions
# ---------------------------------------------------------------------------
def hh_textbook(v, celsius=6.3):
    q10 = 3.0 ** ((celsius - 6.3) / 10)

    def lin(x, y):   # x / (1 - exp(-x/y)) with its limit y at x = 0
        return y if abs(x) < 1e-12 else x / (1 - math.exp(-x / y))

    am = 0.1 * lin(v + 40, 10)
    bm = 4 * math.exp(-(v + 65) / 18)
    ah = 0.07 * math.exp(-(v + 65) / 20)
    bh = 1 / (1 + math.exp(-(v + 35) / 10))
    an = 0.01 * lin(v + 55, 10)
    bn = 0.125 * math.exp(-(v + 65) / 80)
    return (am / (am + bm), 1 / (q10 * (am + bm)), ah / (ah + bh), 1 / (q10 * (ah + bh)),
            an / (an + bn), 1 / (q10 * (an + bn)))


def hh_cell(v_init, celsius=6.3):
    spec = single_compartment(celsius=celsius)
    n = np.array([0], np.int32)
    spec.mechs["hh"] = MechSpec(n, {"gnabar": np.array([0.12]), "gkbar": np.array([0.036]), "gl": np.array([3e-4]),
                                    "el": np.array([-54.3])})
    spec.mechs["na_ion"] = MechSpec(n.copy(), {"erev": np.array([50.0])}, iontype=np.zeros(1, np.int32))
    spec.mechs["k_ion"] = MechSpec(n.copy(), {"erev": np.array([-77.0])}, iontype=np.zeros(1, np.int32))
    return spec


@pytest.mark.parametrize("v0", [-80.0, -65.0, -40.0, -20.0, 10.0])
@pytest.mark.parametrize("celsius", [6.3, 16.3])
def test_hh_init_matches_textbook_rates(v0, celsius):
    o = oracle.OracleSim(hh_cell(v0, celsius), monitors=[])
    o.finitialize(v0)
    got = [o.get("hh", k, 0) for k in ("minf", "mtau", "hinf", "htau", "ninf", "ntau")]
    ref = hh_textbook(v0, celsius)
    assert np.allclose(got, ref, rtol=1e-12)
    assert o.get("hh", "m", 0) == got[0] and o.get("hh", "h", 0) == got[2] and o.get("hh", "n", 0) == got[4]


def test_hh_fd_jacobian_equals_conductance():
    """The FD Jacobian (I(v+0.001)-I(v))/0.001 of hh is gna+gk+gl because the
    current is linear in v at fixed gates (mech_template.cuh:616-626)."""
    o = oracle.OracleSim(hh_cell(-60.0), monitors=[])
    o.finitialize(-60.0)
    m, h, n = (o.get("hh", k, 0) for k in ("m", "h", "n"))
    g = 0.12 * m ** 3 * h + 0.036 * n ** 4 + 3e-4
    cfac = 1e-3 / 0.025
    d = o.array("global", "d")[0]        # after finitialize: mech g + capacitance
    assert abs((d - cfac) - g) / g < 1e-6
    i = 0.12 * m ** 3 * h * (-60 - 50) + 0.036 * n ** 4 * (-60 + 77) + 3e-4 * (-60 + 54.3)
    assert abs(o.array("global", "rhs")[0] + i) < 1e-12


def test_hh_gates_fixed_point_at_clamp():
    """With v held (huge capacitance), gates initialised at x_inf stay there."""
    spec = hh_cell(-30.0)
    spec.cm[:] = 1e12
    o = oracle.OracleSim(spec, monitors=[("hh", "m", 0), ("hh", "n", 0)])
    o.finitialize(-30.0)
    o.run(5.0)
    m = o.monitor(0)
    n = o.monitor(1)
    assert np.max(np.abs(m - m[0])) < 1e-9 and np.max(np.abs(n - n[0])) < 1e-9


# A capacitance of 1e15 uF/cm2 holds v: the largest membrane current here moves it by
# about 1e-12 mV per step, so gates see a constant voltage and cnexp is exact.
CLAMP_CM = 1e15


def relaxation(x0, xinf, tau, nsamp, dt=0.025):
    """Sample k of a first-order relaxation started at x0 (sample 0 = x0)."""
    k = np.arange(nsamp)
    return xinf + (x0 - xinf) * np.exp(-k * dt / tau)


def clamp_step(o, v0, v1, tstop):
    """finitialize at v0 (gates at x_inf(v0)), then hold v at v1 for tstop ms."""
    o.finitialize(v0)
    o.set("global", "v", 0, v1)
    o.run(tstop)


@pytest.mark.parametrize("v1", [-90.0, -55.0, -30.0, 5.0])
@pytest.mark.parametrize("celsius", [6.3, 16.3])
def test_hh_gate_relaxation_under_clamp(v1, celsius):
    """Gates started at x_inf(v0) and held at v1 follow x_inf + (x0 - x_inf) exp(-t/tau)
    with x_inf and tau of the textbook rates at v1 and the temperature's q10
    (hh_templated.cu:151-164).  A wrong tau, q10, sign or rate fails."""
    v0 = -65.0
    spec = hh_cell(v0, celsius)
    spec.cm[:] = CLAMP_CM
    o = oracle.OracleSim(spec, monitors=[("hh", "m", 0), ("hh", "h", 0), ("hh", "n", 0), ("global", "v", 0)])
    clamp_step(o, v0, v1, 6.0)
    v = o.monitor(3)
    assert np.max(np.abs(v[1:] - v1)) < 1e-9
    r0 = hh_textbook(v0, celsius)
    r1 = hh_textbook(v1, celsius)
    for j, name in enumerate("mhn"):
        x = o.monitor(j)
        ref = relaxation(r0[2 * j], r1[2 * j], r1[2 * j + 1], x.size)
        assert np.max(np.abs(x - ref)) < 1e-10, name
        # the relaxation is visible: it moved the gate by more than the tolerance
        assert abs(x[-1] - x[0]) > 1e-4 or abs(r0[2 * j] - r1[2 * j]) < 1e-4


def test_hh_ion_currents_under_clamp():
    """ina = gnabar m^3 h (v - ena) and ik = gkbar n^4 (v - ek) accumulate into the ions'
    cur (hh_templated.cu:120-140)."""
    v0, v1 = -65.0, -20.0
    spec = hh_cell(v0)
    spec.cm[:] = CLAMP_CM
    o = oracle.OracleSim(spec, monitors=[("hh", "m", 0), ("hh", "h", 0), ("hh", "n", 0),
                                         ("na_ion", "cur", 0), ("k_ion", "cur", 0)])
    clamp_step(o, v0, v1, 1.0)
    m, h, n, ina, ik = (o.monitor(j) for j in range(5))
    # the current of step k uses the gates of sample k-1 (states update after the solve)
    assert np.allclose(ina[1:], 0.12 * m[:-1] ** 3 * h[:-1] * (v1 - 50.0), rtol=1e-9, atol=0)
    assert np.allclose(ik[1:], 0.036 * n[:-1] ** 4 * (v1 + 77.0), rtol=1e-9, atol=0)


def cahva_textbook(v):
    """Ca_HVA rates of Reuveni et al. (1993) as distributed with the BBP models:
    (mInf, mTau, hInf, hTau)."""
    x = -27.0 - v
    ma = 0.055 * (3.8 if abs(x) < 1e-9 else x / (math.exp(x / 3.8) - 1))
    mb = 0.94 * math.exp((-75.0 - v) / 17.0)
    ha = 0.000457 * math.exp((-13.0 - v) / 50.0)
    hb = 0.0065 / (math.exp((-v - 15.0) / 28.0) + 1.0)
    return ma / (ma + mb), 1 / (ma + mb), ha / (ha + hb), 1 / (ha + hb)


def hdla_textbook(v, celsius, vhalfl=-81.0, tau=1.0):
    """Ih of Larkum (hd_la): linf and taul with the mechanism's default globals
    (kl -8, vhalft -75, a0t 0.011, zetat 2.2, gmt 0.4, q10 4.5, qtl 1)."""
    qt = 4.5 ** ((celsius - 33.0) / 10.0)
    a = math.exp(0.0378 * 2.2 * (v + 75.0))
    b = math.exp(0.0378 * 2.2 * 0.4 * (v + 75.0))
    linf = 1.0 / (1.0 + math.exp((v - vhalfl) / 8.0))
    return linf, tau * b / (1.0 * qt * 0.011 * (1.0 + a))


def calcium_cell(gbar, iontype, cadyn_params, celsius=6.3, hd=None):
    spec = single_compartment(celsius=celsius)
    spec.cm[:] = CLAMP_CM
    n = np.array([0], np.int32)
    spec.mechs["ca_ion"] = MechSpec(n, {"conci": np.array([5e-5]), "conco": np.array([2.0])},
                                    iontype=np.array([iontype], np.int32))
    spec.mechs["Ca_HVA"] = MechSpec(n.copy(), {"gbar": np.array([gbar])})
    if cadyn_params is not None:
        spec.mechs["CaDynamics_E2"] = MechSpec(n.copy(), {k: np.array([v]) for k, v in cadyn_params.items()})
    if hd is not None:
        spec.mechs["hd_la"] = MechSpec(n.copy(), {k: np.array([v]) for k, v in hd.items()})
    return spec


@pytest.mark.parametrize("v1", [-70.0, -35.0, -10.0, 20.0])
def test_cahva_gate_relaxation_under_clamp(v1):
    """Ca_HVA m and h relax with mTau, hTau of the published rates (CA_HVA.cu:97-178)."""
    v0 = -65.0
    spec = calcium_cell(1e-4, 0o4 | 0o40 | 0o100, None)
    o = oracle.OracleSim(spec, monitors=[("Ca_HVA", "m", 0), ("Ca_HVA", "h", 0)])
    clamp_step(o, v0, v1, 20.0)
    r0 = cahva_textbook(v0)
    r1 = cahva_textbook(v1)
    m, h = o.monitor(0), o.monitor(1)
    assert np.max(np.abs(m - relaxation(r0[0], r1[0], r1[1], m.size))) < 1e-10
    assert np.max(np.abs(h - relaxation(r0[2], r1[2], r1[3], h.size))) < 1e-10
    # both gates moved by at least 1e4 times the tolerance
    assert abs(m[-1] - m[0]) > 1e-6
    assert abs(h[-1] - h[0]) > 1e-6
    # the assigned time constants are the rates' own
    assert abs(o.get("Ca_HVA", "mTau", 0) / r1[1] - 1) < 1e-9
    assert abs(o.get("Ca_HVA", "hTau", 0) / r1[3] - 1) < 1e-9


@pytest.mark.parametrize("v1", [-100.0, -81.0, -60.0])
@pytest.mark.parametrize("celsius", [6.3, 34.0])
def test_hdla_gate_relaxation_under_clamp(v1, celsius):
    """Ih's l relaxes with taul = tau bett / (qtl qt a0t (1 + alpt)) (hd_la.cu:80-128),
    here with a per-instance vhalfl and tau away from their defaults."""
    v0 = -65.0
    spec = calcium_cell(0.0, 0o4 | 0o40 | 0o100, None, celsius=celsius,
                        hd={"ghdbar": 1e-4, "vhalfl": -78.0, "tau": 1.7})
    o = oracle.OracleSim(spec, monitors=[("hd_la", "l", 0)])
    clamp_step(o, v0, v1, 100.0)
    l0, _ = hdla_textbook(v0, celsius, -78.0, 1.7)
    l1, t1 = hdla_textbook(v1, celsius, -78.0, 1.7)
    x = o.monitor(0)
    assert np.max(np.abs(x - relaxation(l0, l1, t1, x.size))) < 1e-10
    assert abs(x[-1] - x[0]) > 1e-3


@pytest.mark.parametrize("ehd", [-30.0, -47.0])
@pytest.mark.parametrize("l0", [0.05, 0.6])
def test_hdla_current_moves_v_toward_ehd(ehd, l0):
    """Ih's current i = ghdbar l (v - ehd) (hd_la.cu:113-115) with ehd set as a
    global and l started away from linf(v): a compartment carrying only Ih
    follows the backward-Euler recurrence
        v' = v - ghdbar l (v - ehd) / (1e-3 cm / dt + ghdbar l),
    with l advanced after each solve by the pinned relaxation
    l' = l + (1 - exp(-dt / taul(v'))) (linf(v') - l)."""
    dt, cm, ghdbar, v0 = 0.025, 1.0, 2e-3, -70.0
    spec = single_compartment(cm=cm, dt=dt)
    spec.mechs["hd_la"] = MechSpec(np.array([0], np.int32), {"ghdbar": np.array([ghdbar])}, globals={"ehd": ehd})
    o = oracle.OracleSim(spec, monitors=[])
    o.finitialize(v0)
    assert abs(o.get("hd_la", "l", 0) - hdla_textbook(v0, 6.3)[0]) < 1e-14
    o.set("hd_la", "l", 0, l0)
    v, l = v0, l0
    for step in range(40):
        o.fadvance()
        # the step's current uses the state before the step's update
        assert abs(o.get("hd_la", "i", 0) - ghdbar * l * (v - ehd)) < 1e-13, step
        v = v - ghdbar * l * (v - ehd) / (1e-3 * cm / dt + ghdbar * l)
        linf, taul = hdla_textbook(v, 6.3)
        l = l + (1 - math.exp(-dt / taul)) * (linf - l)
        assert abs(o.array("global", "v")[0] - v) < 1e-10, step
        assert abs(o.get("hd_la", "l", 0) - l) < 1e-12, step
    # v moved toward ehd by far more than the tolerance
    assert abs(v - v0) > 0.5 and abs(v - ehd) < abs(v0 - ehd)


def im_textbook(v):
    """Im of Hay et al. 2011 as a logistic and a hyperbolic secant: with
    alpha, beta = 3.3e-3 exp(+-0.1 (v + 35)), m_inf = 1 / (1 + exp(-0.2 (v + 35))) and
    tau = 1 / (6.6e-3 cosh(0.1 (v + 35)) qt), qt = 2.3^((34 - 21) / 10) (Im.cu:63-70)."""
    x = v + 35.0
    qt = 2.3 ** 1.3
    return 1.0 / (1.0 + math.exp(-0.2 * x)), 1.0 / (6.6e-3 * math.cosh(0.1 * x) * qt)


def im_cell(gimbar, ek=-85.0):
    spec = single_compartment()
    spec.cm[:] = CLAMP_CM
    n = np.array([0], np.int32)
    spec.mechs["k_ion"] = MechSpec(n, {"erev": np.array([ek])}, iontype=np.zeros(1, np.int32))
    spec.mechs["Im"] = MechSpec(n.copy(), {"gImbar": np.array([gimbar])})
    return spec


@pytest.mark.parametrize("v1", [-80.0, -50.0, -35.0, -10.0, 20.0])
def test_im_gate_relaxation_and_ik_under_clamp(v1):
    """Im's m relaxes to m_inf(v1) with tau(v1), and ik = gImbar m (v - ek) of the gate
    before each step's state update lands in k_ion.cur (Im.cu:72-100)."""
    v0, gimbar, ek = -65.0, 2e-3, -85.0
    o = oracle.OracleSim(im_cell(gimbar, ek), monitors=[("Im", "m", 0), ("k_ion", "cur", 0), ("Im", "ek", 0)])
    clamp_step(o, v0, v1, 200.0)
    m, ik, ekr = o.monitor(0), o.monitor(1), o.monitor(2)
    m0, _ = im_textbook(v0)
    m1, t1 = im_textbook(v1)
    assert np.max(np.abs(m - relaxation(m0, m1, t1, m.size))) < 1e-10
    assert abs(m[-1] - m[0]) > 1e-3
    assert np.allclose(ik[1:], gimbar * m[:-1] * (v1 - ek), rtol=1e-12, atol=0)
    assert np.all(ekr == ek)
    # the clamp holds v to ~1e-10 mV, which moves tau by a few parts in 1e12
    assert abs(o.get("Im", "mTau", 0) / t1 - 1) < 1e-9


@pytest.mark.parametrize("v0,gbar", [(-10.0, 1e-3), (-30.0, 5e-4), (10.0, 2e-3)])
def test_cadynamics_drive_under_constant_ica(v0, gbar):
    """With v held and eca fixed at its initial Nernst value (ion style 04|040, no
    per-step Nernst), Ca_HVA's ica is constant and lands in ca_ion.cur as
    gbar m^2 h (v - eca); cai then follows the linear ODE
    dcai/dt = -1e4 ica gamma / (2 F depth) - (cai - minCai) / decay, whose solution is
    c_inf + (c0 - c_inf) exp(-t/decay) with c_inf = minCai - decay 1e4 ica gamma / (2 F depth)
    (CaDynamics_E2.cu:101-139, CA_HVA.cu:150-165)."""
    gamma, decay, depth, minCai = 0.07, 60.0, 0.2, 2e-4
    celsius = 6.3
    spec = calcium_cell(gbar, 0o4 | 0o40, {"gamma": gamma, "decay": decay, "depth": depth, "minCai": minCai})
    o = oracle.OracleSim(spec, monitors=[("ca_ion", "conci", 0), ("ca_ion", "cur", 0), ("ca_ion", "erev", 0)])
    o.finitialize(v0)
    o.run(150.0)
    cai, cur, erev = o.monitor(0), o.monitor(1), o.monitor(2)
    eca = 1000 * R * (celsius + 273.15) / F / 2 * math.log(2.0 / 5e-5)
    assert np.max(np.abs(erev - eca)) < 1e-12
    minf, _, hinf, _ = cahva_textbook(v0)
    ica = gbar * minf ** 2 * hinf * (v0 - eca)
    assert np.max(np.abs(cur[1:] - ica)) < 1e-12 * abs(ica) + 1e-15
    cinf = minCai - decay * 1e4 * ica * gamma / (2 * F * depth)
    ref = relaxation(5e-5, cinf, decay, cai.size)
    assert np.max(np.abs(cai - ref)) < 1e-10 * abs(cinf)
    assert cai[-1] > 10 * 5e-5          # the drive moved calcium far from its start


def test_cahva_ica_follows_nernst_each_step():
    """With style 0100 eca is recomputed from cai every step, and ica in ca_ion.cur is
    gbar m^2 h (v - eca) with that step's eca (eion.cuh:155-166, CA_HVA.cu:150-165)."""
    v0, gbar = -10.0, 1e-3
    spec = calcium_cell(gbar, 0o4 | 0o40 | 0o100, {"decay": 80.0})
    o = oracle.OracleSim(spec, monitors=[("ca_ion", "conci", 0), ("ca_ion", "cur", 0), ("ca_ion", "erev", 0)])
    o.finitialize(v0)
    o.run(20.0)
    cai, cur, erev = o.monitor(0), o.monitor(1), o.monitor(2)
    minf, _, hinf, _ = cahva_textbook(v0)
    nernst = 1000 * R * (6.3 + 273.15) / F / 2 * np.log(2.0 / cai)
    # the erev sampled after step k is Nernst of the cai that step k's current phase saw
    assert np.allclose(erev[1:], nernst[:-1], rtol=1e-12)
    assert np.allclose(cur[1:], gbar * minf ** 2 * hinf * (v0 - erev[1:]), rtol=1e-12)
    assert erev[-1] < erev[0] - 1.0


# ---------------------------------------------------------------------------
# synapses: cnexp decays are exact exponentials; Exp2Syn peak is normalised
# ---------------------------------------------------------------------------
def synapse_cell(mech, params, times, weight, delay=0.0):
    spec = single_compartment()
    n = np.array([0], np.int32)
    spec.mechs["pas"] = MechSpec(n, {"g_pas": np.array([1e-4]), "e_pas": np.array([-65.0])})
    spec.mechs[mech] = MechSpec(n.copy(), {k: np.array([v]) for k, v in params.items()})
    spec.mechs["VecStim"] = MechSpec(n.copy(), {})
    spec.vecstim_offsets = np.array([0, len(times)])
    spec.vecstim_times = np.asarray(times, float)
    spec.netcons[mech] = NetConSpec(np.array([0], np.int32), np.array([1], np.int8), np.array([0], np.int32),
                                    np.array([weight]), np.array([delay]))
    return spec


def test_expsyn_decay_closed_form():
    tau, w = 2.0, 0.003
    spec = synapse_cell("ExpSyn", {"tau": tau, "e": 0.0}, [0.1], w, delay=0.0)
    o = oracle.OracleSim(spec, monitors=[("ExpSyn", "g", 0)])
    o.finitialize(-65.0)
    o.run(20.0)
    g = o.monitor(0)
    k0 = int(np.argmax(g > 0))
    n = np.arange(len(g) - k0)
    ref = g[k0] * np.exp(-n * 0.025 / tau)
    assert np.allclose(g[k0:], ref, rtol=1e-12)
    # the event (weight w) lands before the first state update of its step
    assert abs(g[k0] - w * math.exp(-0.025 / tau)) < 1e-15


def backward_euler_pas_syn(v0, gsyn_per_step, esyn, gp=1e-4, ep=-65.0, area=1000.0, cm=1.0, dt=0.025):
    """Backward Euler of one compartment with pas and a synaptic conductance (uS) that is
    constant within each step: v' = (C v + gp ep + G esyn) / (C + gp + G), C = 1e-3 cm / dt,
    G = gsyn * 1e2 / area (a point process's nA -> mA/cm2)."""
    c = 1e-3 * cm / dt
    v = [v0]
    for gs in gsyn_per_step:
        G = gs * 1e2 / area
        v.append((c * v[-1] + gp * ep + G * esyn) / (c + gp + G))
    return np.array(v)


def test_expsyn_current_backward_euler():
    """ExpSyn's current g (v - e) enters the membrane as a point process: its conductance
    during step k is the sampled g undone by one decay factor (the event lands before
    the current, the decay after the solve) (expsyn.cu:40-70)."""
    tau, w, esyn = 3.0, 0.004, -10.0
    spec = synapse_cell("ExpSyn", {"tau": tau, "e": esyn}, [0.5, 3.0], w)
    o = oracle.OracleSim(spec, monitors=[("ExpSyn", "g", 0), ("global", "v", 0)])
    o.finitialize(-65.0)
    o.run(15.0)
    g, v = o.monitor(0), o.monitor(1)
    gstep = g[1:] * math.exp(0.025 / tau)
    ref = backward_euler_pas_syn(-65.0, gstep, esyn)
    assert np.max(np.abs(v - ref)) < 1e-9
    assert v.max() > -60.0            # the synapse moved v by several mV


def test_exp2syn_current_backward_euler():
    """Exp2Syn's conductance is B - A, each undone by its own decay factor (exp2syn_temp.cuh:46-67)."""
    t1, t2, w, esyn = 0.5, 5.0, 0.003, 0.0
    spec = synapse_cell("Exp2Syn", {"tau1": t1, "tau2": t2, "e": esyn}, [0.5], w)
    o = oracle.OracleSim(spec, monitors=[("Exp2Syn", "A", 0), ("Exp2Syn", "B", 0), ("global", "v", 0)])
    o.finitialize(-65.0)
    o.run(15.0)
    A, B, v = o.monitor(0), o.monitor(1), o.monitor(2)
    gstep = B[1:] * math.exp(0.025 / t2) - A[1:] * math.exp(0.025 / t1)
    ref = backward_euler_pas_syn(-65.0, gstep, esyn)
    assert np.max(np.abs(v - ref)) < 1e-9
    assert v.max() > -60.0


def test_halfgap_pair_lagged_coupling():
    """Two compartments joined by a HalfGap pair: each step the ELECTRODE current
    (vgap - v) g, with g implicit in v and vgap the partner's voltage after the
    previous update (simulate.cpp:436-438, 953-966; HalfGap.cu:61-68), gives
    v' = v + [G (vgap - v) - gp (v - e)] / (C + gp + G)."""
    area, g, gp, dt = 1000.0, 1e-3, 1e-4, 0.025
    e = np.array([-65.0, -40.0])
    spec = ModelSpec(ncell=2, parent=np.array([-1, -1], np.int32), a=np.zeros(2), b=np.zeros(2),
                     area=np.full(2, area), cm=np.ones(2), dt=dt)
    nodes = np.array([0, 1], np.int32)
    spec.mechs["pas"] = MechSpec(nodes, {"g_pas": np.full(2, gp), "e_pas": e.copy()})
    spec.mechs["HalfGap"] = MechSpec(nodes.copy(), {"g": np.full(2, g)})
    spec.gap_src_node = np.array([1, 0], np.int32)       # HalfGap 0 (on cell 0) sees cell 1
    spec.gap_halfgap = np.array([0, 1], np.int32)
    o = oracle.OracleSim(spec, monitors=[("global", "v", 0), ("global", "v", 1), ("HalfGap", "vgap", 0)])
    o.finitialize(-65.0)
    o.run(30.0)
    v0, v1, vg = o.monitor(0), o.monitor(1), o.monitor(2)
    c = 1e-3 / dt
    G = g * 1e2 / area
    ref = np.zeros((v0.size, 2))
    ref[0] = -65.0
    for k in range(1, v0.size):
        v = ref[k - 1]
        vgap = v[::-1]
        ref[k] = v + (G * (vgap - v) - gp * (v - e)) / (c + gp + G)
    assert np.max(np.abs(v0 - ref[:, 0])) < 1e-10
    assert np.max(np.abs(v1 - ref[:, 1])) < 1e-10
    assert np.array_equal(vg, v1)                 # the transfer after each update
    # the coupling is visible: without it cell 0 would stay at its rest
    assert v0[-1] > -64.0


def test_exp2syn_peak_is_weight():
    t1, t2, w = 0.5, 5.0, 0.002
    spec = synapse_cell("Exp2Syn", {"tau1": t1, "tau2": t2, "e": 0.0}, [0.1], w)
    o = oracle.OracleSim(spec, monitors=[("Exp2Syn", "A", 0), ("Exp2Syn", "B", 0)])
    o.finitialize(-65.0)
    o.run(30.0)
    g = o.monitor(1) - o.monitor(0)
    tp = t1 * t2 / (t2 - t1) * math.log(t2 / t1)
    assert abs(g.max() / w - 1) < 2e-3        # sampled within one dt of the peak
    k0 = int(np.argmax(g > 0))
    n = np.arange(len(g) - k0) + 1
    f = 1 / (math.exp(-tp / t2) - math.exp(-tp / t1))
    ref = w * f * (np.exp(-n * 0.025 / t2) - np.exp(-n * 0.025 / t1))
    assert np.allclose(g[k0:], ref, rtol=1e-9, atol=1e-18)


# ---------------------------------------------------------------------------
# ions and calcium dynamics
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("celsius", [6.3, 34.0])
def test_nernst_closed_form(celsius):
    spec = single_compartment(celsius=celsius)
    n = np.array([0], np.int32)
    spec.mechs["ca_ion"] = MechSpec(n, {"conci": np.array([5e-5]), "conco": np.array([2.0])},
                                    iontype=np.array([0o4 | 0o40 | 0o100], np.int32))
    spec.mechs["CaDynamics_E2"] = MechSpec(n.copy(), {})
    o = oracle.OracleSim(spec, monitors=[])
    o.finitialize(-65.0)
    ref = 1000 * R * (celsius + 273.15) / F / 2 * math.log(2.0 / 5e-5)
    assert abs(o.get("ca_ion", "erev", 0) - ref) < 1e-12


def test_cadynamics_relaxation_closed_form():
    """With no calcium current, cai relaxes to minCai with time constant decay."""
    spec = single_compartment()
    n = np.array([0], np.int32)
    spec.mechs["ca_ion"] = MechSpec(n, {"conci": np.array([5e-5]), "conco": np.array([2.0])},
                                    iontype=np.array([0o4 | 0o40 | 0o100], np.int32))
    spec.mechs["CaDynamics_E2"] = MechSpec(n.copy(), {"decay": np.array([80.0]), "minCai": np.array([1e-4])})
    o = oracle.OracleSim(spec, monitors=[("ca_ion", "conci", 0)])
    o.finitialize(-65.0)
    o.run(100.0)
    c = o.monitor(0)
    k = np.arange(len(c))
    ref = 1e-4 + (5e-5 - 1e-4) * np.exp(-k * 0.025 / 80.0)
    assert np.allclose(c, ref, rtol=1e-11)


def test_cahva_and_ih_steady_states():
    """Gates start at their steady state (Ca_HVA mInf/hInf, hd_la linf) at v_init."""
    spec = single_compartment()
    n = np.array([0], np.int32)
    spec.mechs["ca_ion"] = MechSpec(n, {}, iontype=np.array([0o4 | 0o40 | 0o100], np.int32))
    spec.mechs["Ca_HVA"] = MechSpec(n.copy(), {"gbar": np.array([1e-4])})
    spec.mechs["hd_la"] = MechSpec(n.copy(), {"ghdbar": np.array([1e-4])})
    o = oracle.OracleSim(spec, monitors=[])
    v = -52.0
    o.finitialize(v)
    ma = 0.055 * (-27 - v) / (math.exp((-27 - v) / 3.8) - 1)
    mb = 0.94 * math.exp((-75 - v) / 17)
    ha = 0.000457 * math.exp((-13 - v) / 50)
    hb = 0.0065 / (math.exp((-v - 15) / 28) + 1)
    assert abs(o.get("Ca_HVA", "m", 0) - ma / (ma + mb)) < 1e-14
    assert abs(o.get("Ca_HVA", "h", 0) - ha / (ha + hb)) < 1e-14
    linf = 1 / (1 + math.exp(-(v + 81) / -8))
    assert abs(o.get("hd_la", "l", 0) - linf) < 1e-14
    qt = 4.5 ** ((6.3 - 33) / 10)
    a = math.exp(0.0378 * 2.2 * (v + 75))
    taul = math.exp(0.0378 * 2.2 * 0.4 * (v + 75)) / (qt * 0.011 * (1 + a))
    assert abs(o.get("hd_la", "taul", 0) / taul - 1) < 1e-13


# ---------------------------------------------------------------------------
# spike delivery: brute force of the receive rule (postsyn.cpp:43-61)
# ---------------------------------------------------------------------------
def step_times(dt, nstep):
    t = [0.0]
    for _ in range(nstep):
        x = t[-1]
        x += 0.5 * dt
        x += 0.5 * dt
        t.append(x)
    return np.array(t)


@pytest.mark.parametrize("delay", [0.0, 0.0125, 0.0126, 0.5, 1.0, 1.37])
def test_vecstim_delivery_step_rule(delay):
    dt = 0.025
    times = [0.3, 0.31, 2.0125, 4.7]
    spec = synapse_cell("ExpSyn", {"tau": 1e9, "e": 0.0}, times, 1e-3, delay=delay)
    o = oracle.OracleSim(spec, monitors=[("ExpSyn", "g", 0)])
    o.finitialize(-65.0)
    o.run(8.0)
    g = o.monitor(0)
    # brute force: a VecStim element e fires at the first step k with e <= t_k + dt/2,
    # stamped t_k; its target receives at the first step m >= k with t_k + delay <= t_m + dt/2
    t = step_times(dt, len(g))
    expect = np.zeros(len(g))
    for e in times:
        k = int(np.argmax(e <= t + dt / 2))
        m = k + int(np.argmax(t[k] + delay <= t[k:] + dt / 2))
        expect[m + 1:] += 1e-3   # sample j is taken at the end of step j-1: step m's delivery shows in sample m+1
    assert np.allclose(g, expect, atol=1e-15)


def test_threshold_detection_and_netcon_delay():
    """A driven hh cell spikes (stamped with the step-start time, no
    interpolation, presyn.cpp:150) and its netcon delivers after the delay."""
    spec = hh_cell(-65.0)
    n = np.array([0], np.int32)
    spec.mechs["IClamp"] = MechSpec(n.copy(), {"delay": np.array([1.0]), "dur": np.array([5.0]),
                                               "amp": np.array([0.5])})
    spec.mechs["ExpSyn"] = MechSpec(n.copy(), {"tau": np.array([1e9]), "e": np.array([0.0])})
    spec.presyn_gid = np.array([7], np.int32)
    spec.presyn_node = np.array([0], np.int32)
    spec.presyn_thr = np.array([0.0])
    spec.netcons["ExpSyn"] = NetConSpec(np.array([0], np.int32), np.array([0], np.int8), np.array([0], np.int32),
                                        np.array([1e-9]), np.array([1.0]))
    spec.monitors = [("global", "v", 0), ("ExpSyn", "g", 0)]
    o = oracle.OracleSim(spec)
    o.finitialize(-65.0)
    o.run(10.0)
    v = o.monitor(0)
    g = o.monitor(1)
    ts, gid = o.spikes()
    assert len(ts) >= 1 and np.all(gid == 7)
    t = step_times(0.025, len(v))
    # spike at step k: v at the start of step k (sample k) exceeds 0 for the first time
    k = int(np.argmax(v > 0.0))
    assert abs(ts[0] - t[k]) < 1e-12
    m = k + int(np.argmax(t[k] + 1.0 <= t[k:] + 0.0125))
    assert g[m] == 0.0 and g[m + 1] > 0.0


def test_threshold_is_strict_on_a_slow_ramp():
    """Detection fires at the first step whose starting voltage is above the threshold
    (pre_v > thr, presyn.cpp:140-157), stamped with that step's start time: a capacitor
    charged at a constant 0.1 mV per step from -65 mV reaches -65 + 0.1 k after k steps,
    and the threshold sits between steps 20 and 21."""
    dt, area, cm = 0.025, 500.0, 1.0
    step = 0.1
    amp = step * (1e-3 / dt * cm) * area / 1e2
    spec = single_compartment(area=area, cm=cm, dt=dt)
    n = np.array([0], np.int32)
    spec.mechs["pas"] = MechSpec(n, {"g_pas": np.array([0.0]), "e_pas": np.array([-65.0])})
    spec.mechs["IClamp"] = MechSpec(n.copy(), {"delay": np.array([0.0]), "dur": np.array([1e9]),
                                               "amp": np.array([amp])})
    spec.presyn_gid = np.array([3], np.int32)
    spec.presyn_node = np.array([0], np.int32)
    spec.presyn_thr = np.array([-65.0 + 20.5 * step])
    spec.monitors = [("global", "v", 0)]
    o = oracle.OracleSim(spec)
    o.finitialize(-65.0)
    o.run(40 * dt)
    v = o.monitor(0)
    assert np.allclose(v, -65.0 + step * np.arange(v.size), rtol=0, atol=1e-9)
    ts, gid = o.spikes()
    t = step_times(dt, 40)
    assert list(gid) == [3]
    assert ts[0] == t[21]


# ---------------------------------------------------------------------------
# VecPlay: linear interpolation (vecplay.cu:57-79)
# ---------------------------------------------------------------------------
def test_vecplay_linear_interpolation():
    spec = single_compartment()
    n = np.array([0], np.int32)
    spec.mechs["pas"] = MechSpec(n, {})
    spec.mechs["IClamp"] = MechSpec(n.copy(), {"delay": np.array([0.0]), "dur": np.array([1e9])})
    tv = np.array([0.0, 1.0, 1.0, 3.0, 10.0])
    yv = np.array([0.0, 2.0, 4.0, -1.0, 6.0])
    spec.vecplay = [VecPlaySpec("IClamp", "amp", 0, tv, yv)]
    o = oracle.OracleSim(spec, monitors=[("IClamp", "amp", 0)])
    o.finitialize(-65.0)
    o.run(12.0)
    amp = o.monitor(0)
    t = step_times(0.025, len(amp) - 1)

    def interp(x):
        if x <= tv[0]:
            return yv[0]
        if x >= tv[-1]:     # past the last point the reference keeps extrapolating the last segment
            return yv[-2] + (yv[-1] - yv[-2]) * (x - tv[-2]) / (tv[-1] - tv[-2])
        j = int(np.searchsorted(tv, x, side="right"))
        return yv[j - 1] + (yv[j] - yv[j - 1]) * (x - tv[j - 1]) / (tv[j] - tv[j - 1])

    ref = np.array([interp(x) for x in t])
    assert np.allclose(amp, ref, atol=1e-12)


# ---------------------------------------------------------------------------
# Adam (optimizer.cpp:351-393) against Kingma & Ba
# ---------------------------------------------------------------------------
def test_adam_closed_form():
    rng = np.random.default_rng(3)
    w = rng.normal(size=4)
    w0 = w.copy()
    m = np.zeros(4)
    v = np.zeros(4)
    gsz = np.array([1, 2, 3, 1], np.int32)
    lr, b1, b2, eps, imp, inv = 1e-3, 0.9, 0.999, 1e-8, 2.0, 0.5
    mr = np.zeros(4)
    vr = np.zeros(4)
    wr = w0.copy()
    for step in range(1, 6):
        grads = rng.normal(size=gsz.sum())
        oracle.adam_step(w, grads, gsz, m, v, step, lr, inv, imp, b1, b2, eps)
        g = np.add.reduceat(grads, np.r_[0, np.cumsum(gsz)[:-1]]) / gsz * imp * inv
        mr = b1 * mr + (1 - b1) * g
        vr = b2 * vr + (1 - b2) * g * g
        wr = wr - lr * (mr / (1 - b1 ** step)) / (np.sqrt(vr / (1 - b2 ** step)) + eps)
    assert np.allclose(w, wr, rtol=1e-14)


# ---------------------------------------------------------------------------
# syn_record (user_postsyn_mech/syn_record.cuh), run by the library as a synapse plugin
# ---------------------------------------------------------------------------
def syn_record_cell(v1, w_syn, weight, t_event, taus, rna=2.0, nmda_c=0.28, nmda_rho=0.062):
    spec = single_compartment()
    spec.cm[:] = CLAMP_CM
    n = np.array([0], np.int32)
    p = {k: np.array([val]) for k, val in taus.items()}
    p.update({"w": np.array([w_syn]), "r_na": np.array([rna]), "NMDA_C": np.array([nmda_c]),
              "NMDA_rho": np.array([nmda_rho]), "AMPA_e": np.array([0.0]), "NMDA_e": np.array([0.0]),
              "GABA_e": np.array([-80.0])})
    spec.mechs["syn_record"] = MechSpec(n, p)
    spec.mechs["VecStim"] = MechSpec(n.copy(), {})
    spec.vecstim_offsets = np.array([0, 1], np.int64)
    spec.vecstim_times = np.array([t_event])
    spec.netcons["syn_record"] = NetConSpec(inst=np.array([0], np.int32), src_kind=np.array([1], np.int8),
                                            src=np.array([0], np.int32), weight=np.array([weight]),
                                            delay=np.array([0.0]))
    return spec


def two_exp_factor(t1, t2):
    """1 / peak of exp(-t/t2) - exp(-t/t1): the normalisation that makes a unit event peak at 1."""
    tp = t1 * t2 / (t2 - t1) * math.log(t2 / t1)
    return 1.0 / (math.exp(-tp / t2) - math.exp(-tp / t1))


TAUS = {"AMPA_tau1": 0.2, "AMPA_tau2": 1.7, "NMDA_tau1": 2.0, "NMDA_tau2": 30.0, "GABA_tau1": 0.5, "GABA_tau2": 6.0}


@pytest.mark.parametrize("v1", [-70.0, -30.0, 10.0])
def test_syn_record_excitatory_event_closed_form(v1):
    """An event of weight W splits W / (1 + r_na) to AMPA and W r_na / (1 + r_na) to NMDA;
    each conductance is then the normalised difference of exponentials (peak = its share),
    and i = |w| (g_AMPA (v - e_AMPA) + g_NMDA sigma(v) (v - e_NMDA)) with the Jahr-Stevens
    block sigma(v) = 1 / (1 + C exp(-rho v)), from the conductances before each step's decay."""
    W, t_ev, dt = 0.004, 1.0, 0.025
    spec = syn_record_cell(v1, 1.0, W, t_ev, TAUS)
    o = oracle.OracleSim(spec, monitors=[("syn_record", "AMPA_g", 0), ("syn_record", "NMDA_g", 0),
                                         ("syn_record", "i", 0), ("syn_record", "AMPA_A", 0)])
    clamp_step(o, -65.0, v1, 20.0)
    ga, gn, i, aa = (o.monitor(j) for j in range(4))
    # AMPA_A just after the delivering step's state update, then one decay per step
    kd = int(np.argmax(aa > 0))
    assert kd > 0 and aa[kd - 1] == 0.0
    n = np.arange(aa.size - kd)
    fa = two_exp_factor(0.2, 1.7)
    a0 = W * fa / 3.0
    assert np.allclose(aa[kd:], a0 * np.exp(-(n + 1) * dt / 0.2), rtol=1e-12, atol=1e-300)
    # a step's g is B - A before that step's decay, n steps after the delivering one
    # (0 in the delivering step itself)
    ga_ref = a0 * (np.exp(-n * dt / 1.7) - np.exp(-n * dt / 0.2))
    assert ga[kd] == 0.0 and np.allclose(ga[kd:], ga_ref, rtol=1e-9, atol=1e-18)
    fn = two_exp_factor(2.0, 30.0)
    gn_ref = W * 2.0 / 3.0 * fn * (np.exp(-n * dt / 30.0) - np.exp(-n * dt / 2.0))
    assert np.allclose(gn[kd:], gn_ref, rtol=1e-9, atol=1e-18)
    # the peaks are the shares of W (to the step's sampling)
    assert abs(ga.max() / (W / 3.0) - 1) < 0.02 and abs(gn.max() / (2 * W / 3.0) - 1) < 0.01
    sig = 1.0 / (1.0 + 0.28 * math.exp(-0.062 * v1))
    assert np.allclose(i[kd:], ga[kd:] * v1 + gn[kd:] * sig * v1, rtol=1e-9, atol=1e-18)


def test_syn_record_inhibitory_event_and_tau_clamp():
    """w <= 0 routes the event to GABA with its own factor; tau1 >= 0.9999 tau2 is lowered to
    0.9999 tau2 at INITIAL (syn_record.cuh:108-110)."""
    W, dt = 0.003, 0.025
    taus = dict(TAUS, GABA_tau1=6.0, GABA_tau2=6.0)
    spec = syn_record_cell(-50.0, -1.0, W, 2.0, taus)
    o = oracle.OracleSim(spec, monitors=[("syn_record", "GABA_g", 0), ("syn_record", "i", 0)])
    clamp_step(o, -65.0, -50.0, 30.0)
    assert o.get("syn_record", "GABA_tau1", 0) == 0.9999 * 6.0
    assert o.get("syn_record", "Use", 0) == 1.0
    g, i = o.monitor(0), o.monitor(1)
    k0 = int(np.argmax(g > 0))                # one step after the delivering one
    n = np.arange(1, g.size - k0 + 1)
    t1, t2 = 0.9999 * 6.0, 6.0
    ref = W * two_exp_factor(t1, t2) * (np.exp(-n * dt / t2) - np.exp(-n * dt / t1))
    assert np.allclose(g[k0:], ref, rtol=1e-6, atol=1e-18)
    assert np.allclose(i[k0:], g[k0:] * (-50.0 + 80.0), rtol=1e-9, atol=1e-18)
