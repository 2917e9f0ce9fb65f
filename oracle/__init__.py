"""CPU oracle for parity checks -- TEST INFRASTRUCTURE ONLY.

Python binding over ``liboracle.so`` (built from ``oracle.cpp`` by the Makefile
in this directory), the C++ restatement of the reference's CPU step loop.
Only tests, the smoke check and the CPU-baseline leg of the benchmark use it.

Parity status of each oracle function (``tests/test_oracle_pinning.py`` unless named):
  solve_serial ......... pinned: dense-solve equality, relabel invariance,
                         single-node closed form
  passive + IClamp ..... pinned: one-compartment backward-Euler closed form,
                         sealed-cable steady state
  hh ................... pinned: textbook rates at init (two temperatures), gate
                         relaxation x_inf + (x0 - x_inf) exp(-t/tau) under a voltage
                         clamp at four voltages and two temperatures, ina/ik into
                         the ion currents, FD Jacobian vs analytic g
  Ca_HVA ............... pinned: m/h relaxation with the published mTau/hTau under
                         clamp; ica = gbar m^2 h (v - eca) in ca_ion.cur, with a
                         fixed eca and with eca from the per-step Nernst
  hd_la (Ih) ........... pinned: l relaxation with taul under clamp (two
                         temperatures, per-instance vhalfl and tau)
  CaDynamics_E2 ........ pinned: cai under a constant non-zero ica against the
                         linear-ODE solution c_inf + (c0 - c_inf) exp(-t/decay),
                         c_inf = minCai - decay 1e4 ica gamma / (2 F depth); and
                         relaxation to minCai with no current
  Nernst ............... pinned: closed form with CODATA constants
  ExpSyn / Exp2Syn ..... pinned: decay closed forms, Exp2Syn peak = weight, the
                         synaptic current in a backward-Euler compartment
  HalfGap .............. pinned: a two-compartment pair against the lagged
                         coupling recurrence
  spikes / delivery .... pinned: brute-force delivery-step rule on tiny inputs
  VecPlay .............. pinned: closed-form linear interpolation
  Adam ................. pinned: Kingma-Ba closed form
  NetStim .............. pinned (tests/test_netstim.py): Philox4x32-10 against
                         Random123's published known-answer vectors, the stream's
                         id/draw layout against those blocks, noiseless trains
                         against start + k interval, noisy intervals against the
                         exponential law; netcon events against closed-form
                         bursts (trigger while off, ignored while on, switched off,
                         int-truncated weights, chains within one step)
  Im ................... pinned: m relaxation to the logistic m_inf with the
                         sech-form tau under clamp, ik into k_ion.cur
  syn_record ........... pinned: an event's AMPA / NMDA (or GABA) share, the
                         normalised two-exponential conductances, the
                         Jahr-Stevens block in the current, the tau clamp
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_D = C.POINTER(C.c_double)
_I = C.POINTER(C.c_int)


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (g++, -ffp-contract=off)."""
    if force or not os.path.exists(_LIB_PATH) or \
            os.path.getmtime(_LIB_PATH) < os.path.getmtime(os.path.join(_HERE, "oracle.cpp")):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "all"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        L.hxo_create.restype = C.c_void_p
        L.hxo_create.argtypes = [C.c_double, C.c_double]
        L.hxo_destroy.argtypes = [C.c_void_p]
        L.hxo_set_nodes.argtypes = [C.c_void_p, C.c_int, C.c_int, _I, _D, _D, _D, _D]
        L.hxo_insert.argtypes = [C.c_void_p, C.c_char_p, C.c_int, _I]
        L.hxo_set_param.argtypes = [C.c_void_p, C.c_char_p, C.c_char_p, C.c_int, _D]
        L.hxo_set_global.argtypes = [C.c_void_p, C.c_char_p, C.c_char_p, C.c_double]
        L.hxo_set_iontype.argtypes = [C.c_void_p, C.c_char_p, C.c_int, _I]
        L.hxo_add_presyn.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_double]
        L.hxo_set_vecstim.argtypes = [C.c_void_p, C.c_int, C.c_int, _D]
        L.hxo_vecstim_play.argtypes = [C.c_void_p, C.c_int, C.c_int, _D]
        L.hxo_add_netcon.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_char_p, C.c_int, C.c_double, C.c_double]
        L.hxo_add_vecplay.argtypes = [C.c_void_p, C.c_char_p, C.c_char_p, C.c_int, C.c_int, _D, _D]
        L.hxo_add_gap.argtypes = [C.c_void_p, C.c_int, C.c_int]
        L.hxo_add_monitor.argtypes = [C.c_void_p, C.c_char_p, C.c_char_p, C.c_int]
        L.hxo_finalize.argtypes = [C.c_void_p]
        L.hxo_finitialize.argtypes = [C.c_void_p, C.c_double]
        L.hxo_fadvance.argtypes = [C.c_void_p]
        L.hxo_run.argtypes = [C.c_void_p, C.c_double]
        L.hxo_continue_run.argtypes = [C.c_void_p, C.c_double]
        L.hxo_nsteps.argtypes = [C.c_void_p, C.c_int]
        L.hxo_get_t.restype = C.c_double
        L.hxo_get_t.argtypes = [C.c_void_p]
        L.hxo_monitor_len.argtypes = [C.c_void_p, C.c_int]
        L.hxo_get_monitor.argtypes = [C.c_void_p, C.c_int, _D, C.c_int]
        L.hxo_n_spikes.argtypes = [C.c_void_p]
        L.hxo_get_spikes.argtypes = [C.c_void_p, _D, _I, C.c_int]
        L.hxo_get_var.argtypes = [C.c_void_p, C.c_char_p, C.c_char_p, C.c_int, _D]
        L.hxo_set_var.argtypes = [C.c_void_p, C.c_char_p, C.c_char_p, C.c_int, C.c_double]
        L.hxo_get_array.argtypes = [C.c_void_p, C.c_char_p, C.c_char_p, _D, C.c_int]
        L.hxo_solve_serial.argtypes = [C.c_int, C.c_int, _I, _D, _D, _D, _D]
        L.hxo_adam_step.argtypes = [_D, _D, _I, C.c_int, _D, _D, C.c_longlong, C.c_double, C.c_double,
                                    C.c_double, C.c_double, C.c_double, C.c_double]
        L.hxo_philox4x32.argtypes = [C.POINTER(C.c_uint32), C.POINTER(C.c_uint32), C.POINTER(C.c_uint32)]
        L.hxo_netstim_spikes.argtypes = [C.c_void_p, _D, _I, C.c_int]
        _lib = L
    return _lib


def philox4x32(ctr, key):
    """The oracle's Philox4x32-10 block (known-answer checks)."""
    c = (C.c_uint32 * 4)(*[int(x) for x in ctr])
    k = (C.c_uint32 * 2)(*[int(x) for x in key])
    out = (C.c_uint32 * 4)()
    lib().hxo_philox4x32(c, k, out)
    return [int(x) for x in out]


def _dp(a):
    return a.ctypes.data_as(_D)


def _ip(a):
    return a.ctypes.data_as(_I)


def _check(rc, what):
    if rc < 0:
        raise RuntimeError(f"oracle: {what} failed")
    return rc


class OracleSim:
    """The reference CPU step loop, restated, loaded from a ``ModelSpec``."""

    def __init__(self, spec, monitors=None):
        L = lib()
        self.spec = spec
        self.h = L.hxo_create(spec.dt, spec.celsius)
        self._keep = []
        n = spec.nnode
        parent = np.ascontiguousarray(spec.parent, np.int32)
        arrs = [np.ascontiguousarray(x, np.float64) for x in (spec.a, spec.b, spec.area, spec.cm)]
        self._keep += [parent] + arrs
        _check(L.hxo_set_nodes(self.h, spec.ncell, n, _ip(parent), *[_dp(x) for x in arrs]), "set_nodes")
        # ions first so other mechanisms can bind to them
        order = sorted(spec.mechs.keys(), key=lambda k: 0 if k.endswith("_ion") else 1)
        for name in order:
            m = spec.mechs[name]
            nodes = np.ascontiguousarray(m.nodes, np.int32)
            self._keep.append(nodes)
            _check(L.hxo_insert(self.h, name.encode(), m.n, _ip(nodes)), f"insert {name}")
            for k, v in m.params.items():
                v = np.ascontiguousarray(v, np.float64)
                self._keep.append(v)
                _check(L.hxo_set_param(self.h, name.encode(), k.encode(), m.n, _dp(v)), f"param {name}.{k}")
            for k, v in m.globals.items():
                _check(L.hxo_set_global(self.h, name.encode(), k.encode(), float(v)), f"global {name}.{k}")
            if m.iontype is not None:
                it = np.ascontiguousarray(m.iontype, np.int32)
                self._keep.append(it)
                _check(L.hxo_set_iontype(self.h, name.encode(), m.n, _ip(it)), f"iontype {name}")
        for gid, nd, thr in zip(spec.presyn_gid, spec.presyn_node, spec.presyn_thr):
            _check(L.hxo_add_presyn(self.h, int(gid), int(nd), float(thr)), "presyn")
        for k in range(spec.n_vecstim):
            tr = np.ascontiguousarray(spec.vecstim_train(k), np.float64)
            if tr.size:
                _check(L.hxo_set_vecstim(self.h, k, tr.size, _dp(tr)), "vecstim")
        _check(L.hxo_finalize(self.h), "finalize")
        for tgt, nc in spec.netcons.items():
            for i in range(nc.inst.shape[0]):
                _check(L.hxo_add_netcon(self.h, int(nc.src_kind[i]), int(nc.src[i]), tgt.encode(),
                                        int(nc.inst[i]), float(nc.weight[i]), float(nc.delay[i])), "netcon")
        for vp in spec.vecplay:
            tv = np.ascontiguousarray(vp.tvec, np.float64)
            yv = np.ascontiguousarray(vp.yvec, np.float64)
            _check(L.hxo_add_vecplay(self.h, vp.mech.encode(), vp.var.encode(), vp.idx, tv.size, _dp(tv), _dp(yv)),
                   "vecplay")
        for s, g in zip(spec.gap_src_node, spec.gap_halfgap):
            _check(L.hxo_add_gap(self.h, int(s), int(g)), "gap")
        self.monitors = []
        for mech, var, idx in (spec.monitors if monitors is None else monitors):
            self.monitors.append(_check(L.hxo_add_monitor(self.h, mech.encode(), var.encode(), int(idx)),
                                        f"monitor {mech}.{var}[{idx}]"))

    def __del__(self):
        if getattr(self, "h", None):
            lib().hxo_destroy(self.h)
            self.h = None

    def finitialize(self, v_init: float = -65.0):
        _check(lib().hxo_finitialize(self.h, v_init), "finitialize")

    def fadvance(self):
        lib().hxo_fadvance(self.h)

    def run(self, tstop: float):
        lib().hxo_run(self.h, tstop)

    def continue_run(self, runtime: float):
        lib().hxo_continue_run(self.h, runtime)

    def nsteps(self, n: int):
        lib().hxo_nsteps(self.h, int(n))

    @property
    def t(self) -> float:
        return lib().hxo_get_t(self.h)

    def monitor(self, handle: int) -> np.ndarray:
        L = lib()
        n = L.hxo_monitor_len(self.h, handle)
        out = np.empty(max(n, 0))
        L.hxo_get_monitor(self.h, handle, _dp(out), n)
        return out

    def traces(self) -> np.ndarray:
        return np.stack([self.monitor(h) for h in self.monitors]) if self.monitors else np.zeros((0, 0))

    def netstim_spikes(self):
        """(time, instance) of every NetStim spike since finitialize, in emission order."""
        L = lib()
        n = L.hxo_netstim_spikes(self.h, None, None, 0)
        t = np.empty(max(n, 1))
        i = np.empty(max(n, 1), np.int32)
        L.hxo_netstim_spikes(self.h, _dp(t), _ip(i), n)
        return t[:n], i[:n]

    def spikes(self):
        L = lib()
        n = L.hxo_n_spikes(self.h)
        t = np.empty(n)
        g = np.empty(n, np.int32)
        L.hxo_get_spikes(self.h, _dp(t), _ip(g), n)
        return t, g

    def get(self, mech: str, var: str, idx: int) -> float:
        out = np.zeros(1)
        _check(lib().hxo_get_var(self.h, mech.encode(), var.encode(), idx, _dp(out)), f"get {mech}.{var}")
        return float(out[0])

    def set(self, mech: str, var: str, idx: int, val: float):
        _check(lib().hxo_set_var(self.h, mech.encode(), var.encode(), idx, float(val)), f"set {mech}.{var}")

    def vecstim_play(self, inst: int, times) -> None:
        """VecStim.play(inst, times) at the current point of the run (vecevent.cpp:280-309)."""
        tr = np.ascontiguousarray(np.asarray(times, np.float64).ravel())
        _check(lib().hxo_vecstim_play(self.h, int(inst), tr.size, _dp(tr)), "vecstim_play")

    def array(self, mech: str, var: str) -> np.ndarray:
        n = self.spec.nnode if mech in ("global", "node") else self.spec.mechs[mech].n
        out = np.empty(n)
        _check(lib().hxo_get_array(self.h, mech.encode(), var.encode(), _dp(out), n), f"array {mech}.{var}")
        return out


def solve_serial(ncell, parent, a, b, d, rhs):
    """Reference serial Hines solve (simulate.cpp:558-581); returns the solution."""
    parent = np.ascontiguousarray(parent, np.int32)
    a = np.ascontiguousarray(a, np.float64)
    b = np.ascontiguousarray(b, np.float64)
    d = np.array(d, np.float64)
    rhs = np.array(rhs, np.float64)
    lib().hxo_solve_serial(int(ncell), int(parent.size), _ip(parent), _dp(a), _dp(b), _dp(d), _dp(rhs))
    return rhs


def adam_step(w, grads, group_size, m, v, step, lr, inv_record_steps=1.0, impedance=1.0,
              beta1=0.9, beta2=0.999, eps=1e-8):
    """Reference Adam update for tied parameter groups (optimizer.cpp:351-393); in place."""
    gs = np.ascontiguousarray(group_size, np.int32)
    g = np.ascontiguousarray(grads, np.float64)
    lib().hxo_adam_step(_dp(w), _dp(g), _ip(gs), int(w.size), _dp(m), _dp(v), int(step), lr,
                        inv_record_steps, impedance, beta1, beta2, eps)
