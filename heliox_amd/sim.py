"""Python surface of the MI355X simulation core.

``Sim`` mirrors the reference's ``heliox.Sim`` (src/python_api/PyBindings.cpp:15-266,
SimWrapper.h) for the step-loop path: ``set_device``, ``set_dt``/``get_dt``,
``finitialize``, ``run``, ``continue_run``, ``fadvance``, ``get_t``,
``add_monitor``/``get_monitor_data``/``get_multiple_monitor_data``,
``get_variable_handle``/``get_variable_by_handle``/``set_variable_by_handle``
(and their batched forms), ``get_variable_value``/``set_variable_value``,
``add_vecplay``/``update_vecplay``/``remove_vecplay``/``has_vecplay``,
``get_spk_by_gid``, and ``add_gap_source``/``add_gap_target``.  Methods
return 0 / -1 like the reference; ``RuntimeError`` is raised only where the
reference raises.  The model comes from a ``ModelSpec`` (``load_model_from_spec``)
instead of a CoreNEURON export directory.

Every call goes through the C ABI of ``libheliox_amd.so`` (include/heliox.h);
there is no CPU fallback: without the library (or without a GPU) the calls
fail.
"""
from __future__ import annotations

import ctypes as C
import dataclasses
import os
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

from .spec import ModelSpec, register_mechanism

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libheliox_amd.so")
_lib = None

_D = C.POINTER(C.c_double)
_I = C.POINTER(C.c_int)
_F = C.POINTER(C.c_float)
_P = C.c_void_p
_S = C.c_char_p

# name: (restype, argtypes) for every entry point of include/heliox.h
SIGNATURES = {
    "hx_create": (C.c_int, [C.POINTER(_P)]),
    "hx_destroy": (None, [_P]),
    "hx_last_error": (C.c_char_p, [_P]),
    "hx_set_device": (C.c_int, [_P, _S]),
    "hx_set_dt": (C.c_int, [_P, C.c_double]),
    "hx_get_dt": (C.c_double, [_P]),
    "hx_set_celsius": (C.c_int, [_P, C.c_double]),
    "hx_model_set_nodes": (C.c_int, [_P, C.c_int, C.c_int, _I, _D, _D, _D]),
    "hx_model_insert": (C.c_int, [_P, _S, C.c_int, _I]),
    "hx_model_set_param": (C.c_int, [_P, _S, _S, C.c_int, _D]),
    "hx_model_set_global": (C.c_int, [_P, _S, _S, C.c_double]),
    "hx_model_set_iontype": (C.c_int, [_P, _S, C.c_int, _I]),
    "hx_model_add_presyn": (C.c_int, [_P, C.c_int, C.c_int, C.c_double]),
    "hx_model_set_vecstim": (C.c_int, [_P, C.c_int, C.c_int, _D]),
    "hx_call_mech_func": (C.c_int, [_P, C.c_char_p, C.c_char_p, C.c_int, C.c_int, _D]),
    "hx_model_add_netcon": (C.c_int, [_P, C.c_int, C.c_int, _S, C.c_int, C.c_double, C.c_double]),
    "hx_model_add_gap": (C.c_int, [_P, C.c_int, C.c_int]),
    "hx_load_model": (C.c_int, [_P]),
    "hx_set_data_path": (C.c_int, [_P, _S]),
    "hx_set_user_mod_num": (C.c_int, [_P, C.c_int]),
    "hx_model_read_export": (C.c_int, [_P]),
    "hx_model_digest": (C.c_int, [_P, C.c_char_p, C.c_int]),
    "hx_mechanism_names": (C.c_int, [C.c_char_p, C.c_int]),
    "hx_finitialize": (C.c_int, [_P, C.c_double]),
    "hx_run": (C.c_int, [_P, C.c_double]),
    "hx_continue_run": (C.c_int, [_P, C.c_double]),
    "hx_fadvance": (C.c_int, [_P]),
    "hx_get_t": (C.c_double, [_P]),
    "hx_add_monitor": (C.c_int, [_P, _S, _S, C.c_int]),
    "hx_get_monitor_len": (C.c_int, [_P, C.c_int]),
    "hx_get_monitor_data": (C.c_int, [_P, C.c_int, _D, C.c_int]),
    "hx_flush_recorders": (C.c_int, [_P]),
    "hx_get_variable_handle": (C.c_int, [_P, _S, _S, C.c_int]),
    "hx_get_variable_by_handle": (C.c_int, [_P, C.c_int, _D]),
    "hx_set_variable_by_handle": (C.c_int, [_P, C.c_int, C.c_double]),
    "hx_get_variables_by_handles": (C.c_int, [_P, C.c_int, _I, _D]),
    "hx_get_variables_by_handles_f32_into": (C.c_int, [_P, C.c_int, _I, _F]),
    "hx_set_variables_by_handles": (C.c_int, [_P, C.c_int, _I, _D]),
    "hx_get_variable_value": (C.c_int, [_P, _S, _S, C.c_int, _D]),
    "hx_set_variable_value": (C.c_int, [_P, C.c_double, _S, _S, C.c_int]),
    "hx_get_array": (C.c_int, [_P, _S, _S, _D, C.c_int]),
    "hx_add_vecplay": (C.c_int, [_P, _S, _S, C.c_int, C.c_int, _D, _D]),
    "hx_update_vecplay": (C.c_int, [_P, _S, _S, C.c_int, C.c_int, _D, _D]),
    "hx_remove_vecplay": (C.c_int, [_P, _S, _S, C.c_int]),
    "hx_has_vecplay": (C.c_int, [_P, _S, _S, C.c_int]),
    "hx_get_spike_count": (C.c_int, [_P]),
    "hx_get_spikes": (C.c_int, [_P, _D, _I, C.c_int]),
    "hx_get_netstim_spikes": (C.c_int, [_P, _D, _I, C.c_int]),
    "hx_get_spk_by_gid": (C.c_int, [_P, C.c_int, _D, C.c_int]),
    "hx_set_event_capacity": (C.c_int, [_P, C.c_int]),
    "hx_set_fusion": (C.c_int, [_P, C.c_int]),
    "hx_set_dense_steady": (C.c_int, [_P, C.c_int]),
    "hx_set_group_turns": (C.c_int, [_P, C.c_int]),
    "hx_set_close_deferral": (C.c_int, [_P, C.c_int]),
    "hx_set_uniform_columns": (C.c_int, [_P, C.c_int]),
    "hx_set_profiling": (C.c_int, [_P, C.c_int]),
    "hx_set_profiling_classes": (C.c_int, [_P, _S]),
    "hx_tape_begin": (C.c_int, [_P, C.c_int]),
    "hx_tape_length": (C.c_int, [_P]),
    "hx_adjoint": (C.c_int, [_P, C.c_int, _I, _D, C.c_int, _D]),
    "hx_get_gradient": (C.c_int, [_P, _S, _S, _D, C.c_int]),
    "hx_adam_create": (C.c_int, [_P, C.c_double, C.c_double, C.c_double]),
    "hx_adam_add_group": (C.c_int, [_P, C.c_int, _S, _S, C.c_int, _I, C.c_double]),
    "hx_adam_step": (C.c_int, [_P, C.c_int, C.c_double, C.c_double]),
    "hx_adam_get_state": (C.c_int, [_P, C.c_int, C.POINTER(C.c_longlong), _D, _D, C.c_int]),
    "hx_get_kernel_time": (C.c_int, [_P, _S, _D, C.POINTER(C.c_longlong)]),
    "hx_measure_stream": (C.c_int, [C.c_int, C.c_int, C.c_longlong, C.c_int, _D]),
    "hx_get_info": (C.c_longlong, [_P, _S]),
    "hx_emulate_tree_solve": (C.c_int, [C.c_int, C.c_int, _I, _D, _D, _D, C.c_double, _D, _D, _D, _I, _I]),
    "hx_set_dense_blocks_f32": (C.c_int, [_P, C.c_int, C.POINTER(_F), _I, _I]),
    "hx_clear_dense_blocks": (C.c_int, [_P]),
    "hx_simulate_output_vs_into": (C.c_int, [_P, _F, C.c_int, C.c_int, _I, C.c_double, C.c_double]),
    "hx_simulate_and_capture_mapped_signals_cached": (
        C.c_int, [_P, _F, C.c_int, C.c_int, _I, C.c_int, _I, _I, _F, C.c_int, _I, _I, _F, C.c_int, _I, _I, _F,
                  C.c_double, C.c_int, C.c_int, C.c_double]),
    "hx_simulate_and_capture_mapped_signals_into": (
        C.c_int, [_P, _F, C.c_int, C.c_int, _F, _F, _F, C.c_int, C.c_int, _I, C.c_int, _I, _I, _F, C.c_int, _I, _I,
                  _F, C.c_int, _I, _I, _F, C.c_double, C.c_int, C.c_int, C.c_double]),
    "hx_replay_compute_dw_from_cached_signals_into": (
        C.c_int, [_P, _F, C.c_int, C.c_int, _I, _I, C.c_int, _F, C.c_double, C.c_int, C.c_double, C.c_double,
                  C.c_double, C.c_int, C.c_int]),
    "hx_replay_compute_dw_dx_from_cached_signals_into": (
        C.c_int, [_P, _F, C.c_int, C.c_int, _I, _I, C.c_int, _I, C.c_int, _F, _F, C.c_double, C.c_int, C.c_double,
                  C.c_double, C.c_double, C.c_int, C.c_int]),
    "hx_replay_compute_dw_dx_from_signals_into": (
        C.c_int, [_P, _F, _F, _F, C.c_int, C.c_int, _F, C.c_int, C.c_int, _I, _I, C.c_int, _I, _F, _F, C.c_double,
                  C.c_int, C.c_double, C.c_double, C.c_double, C.c_int, C.c_int]),
    "hx_replay_compute_dw_dx_from_signals_into_noalloc": (
        C.c_int, [_P, _F, _F, _F, C.c_int, C.c_int, _F, C.c_int, C.c_int, _I, _I, C.c_int, _I, _F, _F, C.c_double,
                  C.c_int, C.c_double, C.c_double, C.c_double, C.c_int, C.c_int]),
    "hx_simulate_and_replay_dw_dx_streaming_into": (
        C.c_int, [_P, _F, C.c_int, C.c_int, _I, _I, C.c_int, C.c_int, _I, _F, _F, C.c_int, _I, _I, _F, C.c_int, _I,
                  _I, _F, C.c_int, _I, _I, _F, C.c_double, C.c_int, C.c_int, C.c_double, C.c_double, C.c_double,
                  C.c_double, C.c_double, C.c_int, C.c_int]),
    "hx_set_hdf5_enabled": (C.c_int, [_P, C.c_int]),
    "hx_is_hdf5_enabled": (C.c_int, [_P]),
    "hx_set_replay_timing": (C.c_int, [_P, C.c_int]),
    "hx_set_cell_groups": (C.c_int, [_P, C.c_int]),
    "hx_set_group_streams": (C.c_int, [_P, C.c_int]),
    "hx_set_solver_root": (C.c_int, [_P, C.c_int]),
    "hx_set_solve_unit_cells": (C.c_int, [_P, C.c_int]),
    "hx_set_solve_waves": (C.c_int, [_P, C.c_int]),
    "hx_set_solve_resident": (C.c_int, [_P, C.c_int]),
    "hx_set_solve_voltage": (C.c_int, [_P, C.c_int]),
    "hx_output_spikes": (C.c_int, [_P, C.c_char_p]),
    "hx_set_spike_output_enabled": (C.c_int, [_P, C.c_int]),
    "hx_is_spike_output_enabled": (C.c_int, [_P]),
    "hx_set_output_dir": (C.c_int, [_P, C.c_char_p]),
    "hx_add_gap_source": (C.c_int, [_P, C.c_int, C.c_char_p, C.c_char_p, C.c_int]),
    "hx_add_gap_target": (C.c_int, [_P, C.c_int, C.c_char_p, C.c_char_p, C.c_int]),
    "hx_clear_all_gap_junctions": (C.c_int, [_P]),
    "hx_get_next_available_sid": (C.c_int, [_P]),
    "hx_get_gap_junction_sids": (C.c_int, [_P, _I, C.c_int]),
    "hx_get_gap_junction": (C.c_int, [_P, C.c_int, C.c_char_p, C.c_int, C.c_char_p, C.c_int, _I, _I]),
    "hx_get_monitor_handle": (C.c_int, [_P, C.c_char_p, C.c_char_p, C.c_int]),
    "hx_get_vecplay_keys": (C.c_int, [_P, C.c_char_p, C.c_int]),
    "hx_create_optimizer": (C.c_int, [_P, C.c_char_p]),
    "hx_configure_optimizer": (C.c_int, [_P, C.c_int, C.c_double, C.c_double, C.c_double, C.c_double]),
    "hx_optimizer_add_param": (C.c_int, [_P, C.c_int, C.c_int, C.c_int, C.c_double]),
    "hx_optimizer_add_param_batch": (C.c_int, [_P, C.c_int, C.c_int, _I, _I, C.c_double]),
    "hx_optimizer_step": (C.c_int, [_P, C.c_int, C.c_double, C.c_double, C.c_double]),
    "hx_optimizer_step_with_inv_record_steps": (C.c_int, [_P, C.c_int, C.c_double, C.c_double]),
    "hx_optimizer_add_external_grads": (C.c_int, [_P, C.c_int, C.c_int, _I, C.c_double]),
    "hx_optimizer_set_external_grads_f32": (C.c_int, [_P, C.c_int, C.c_int, _F]),
    "hx_optimizer_clear_external_grads": (C.c_int, [_P, C.c_int]),
    "hx_optimizer_reset_state": (C.c_int, [_P, C.c_int]),
    "hx_optimizer_get_adam_state": (C.c_int, [_P, C.c_int, C.POINTER(C.c_longlong), _D, _D, C.c_int, _D, _D, _D]),
    "hx_optimizer_set_adam_state": (C.c_int, [_P, C.c_int, C.c_longlong, C.c_int, _D, _D, C.c_double, C.c_double,
                                              C.c_double]),
    "hx_random123_philox4x32": (C.c_int, [C.POINTER(C.c_uint32), C.POINTER(C.c_uint32), C.POINTER(C.c_uint32)]),
    "hx_fastmath_log": (C.c_int, [C.POINTER(C.c_double), C.POINTER(C.c_double), C.c_int]),
    "hx_netstim_train": (C.c_int, [C.c_double, C.c_double, C.c_double, C.c_double, C.c_double, C.c_double,
                                   C.c_uint, C.c_uint, C.c_uint, _D, C.c_int]),
    "hx_emulate_tree_solve_units": (C.c_int, [C.c_int, C.c_int, _I, _D, _D, _D, C.c_double, _D, _D, _D, C.c_int,
                                              _I, _I]),
    "hx_get_replay_kernel_time": (C.c_int, [_P, _D, C.POINTER(C.c_longlong)]),
}


def lib() -> C.CDLL:
    """Load ``libheliox_amd.so``; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m heliox_amd.build`")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
        for m in mechanisms():
            if m.kind == "plugin":
                register_mechanism(m.name, m.columns[: m.nparam])
    return _lib


@dataclasses.dataclass(frozen=True)
class MechanismInfo:
    """One mechanism the library can insert: its columns are its parameters, then its
    states, then its assigned variables."""
    name: str
    kind: str             # "builtin" or "plugin"
    nparam: int
    nstate: int
    columns: Tuple[str, ...]


def mechanisms() -> List[MechanismInfo]:
    """Every mechanism the library knows, built-in ones first, then plugins in
    registration order (hx_mechanism_names)."""
    L = _lib if _lib is not None else lib()
    n = L.hx_mechanism_names(None, 0)
    buf = C.create_string_buffer(n)
    L.hx_mechanism_names(buf, n)
    out = []
    for line in buf.value.decode().splitlines():
        name, kind, npar, nst, cols = line.split("\t")
        out.append(MechanismInfo(name, kind, int(npar), int(nst), tuple(c for c in cols.split(",") if c)))
    return out


def _dp(a: np.ndarray):
    return a.ctypes.data_as(_D)


def _ip(a: np.ndarray):
    return a.ctypes.data_as(_I)


def _b(s: str) -> bytes:
    return s.encode()


def _fp(a: np.ndarray):
    return a.ctypes.data_as(_F)


def _f32(a, ndim=None) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    if ndim is not None and a.ndim != ndim:
        raise ValueError(f"expected a {ndim}-D float32 array")
    return a


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, np.int32).reshape(-1))


def _out_f32(a: np.ndarray, name: str) -> np.ndarray:
    """Caller-owned output buffer: C-contiguous float32, written in place."""
    if not isinstance(a, np.ndarray) or a.dtype != np.float32 or not a.flags.c_contiguous:
        raise TypeError(f"{name} must be a C-contiguous float32 ndarray")
    return a


class HelioxError(RuntimeError):
    pass


class Sim:
    """One model on one GPU (the reference keeps one model group per process)."""

    def __init__(self):
        L = lib()
        h = _P()
        if L.hx_create(C.byref(h)) != 0:
            raise HelioxError("hx_create failed")
        self._h = h
        self._gap_sources: Dict[int, int] = {}
        self._next_sid = 0
        self.spec: Optional[ModelSpec] = None

    def __del__(self):
        h = getattr(self, "_h", None)
        if h and _lib is not None:
            try:
                _lib.hx_destroy(h)
            except Exception:   # interpreter shutdown
                pass
            self._h = None

    # --------------------------------------------------------------- helpers
    @property
    def handle(self):
        return self._h

    def last_error(self) -> str:
        py = getattr(self, "_py_err", None)
        if py:
            return py
        return lib().hx_last_error(self._h).decode()

    def _pyfail(self, msg: str) -> int:
        """Argument check failed before reaching the library (the reference prints and returns -1)."""
        self._py_err = msg
        return -1

    def _chk(self, rc: int, what: str) -> int:
        self._py_err = None
        if rc < 0:
            raise HelioxError(f"{what}: {self.last_error()}")
        return rc

    def _rc(self, rc: int) -> int:
        """Reference convention: return 0 / -1 and keep the message for last_error()."""
        self._py_err = None
        return 0 if rc >= 0 else -1

    # --------------------------------------------------------------- settings
    def set_device(self, dev: str) -> int:
        return self._rc(lib().hx_set_device(self._h, _b(dev)))

    def set_dt(self, dt: float) -> int:
        return self._rc(lib().hx_set_dt(self._h, float(dt)))

    def get_dt(self) -> float:
        return lib().hx_get_dt(self._h)

    def set_celsius(self, c: float) -> int:
        return self._rc(lib().hx_set_celsius(self._h, float(c)))

    def set_event_capacity(self, n: int) -> int:
        return self._rc(lib().hx_set_event_capacity(self._h, int(n)))

    def set_fusion(self, enable: bool) -> int:
        return self._rc(lib().hx_set_fusion(self._h, 1 if enable else 0))

    def set_group_turns(self, enable: bool) -> int:
        """Make the cell groups' node passes take turns on every step (default on; same
        results either way)."""
        return self._rc(lib().hx_set_group_turns(self._h, 1 if enable else 0))

    def set_dense_steady(self, enable: bool) -> int:
        """Run steady node-kernel steps through their compile-time instance (default on;
        same results either way)."""
        return self._rc(lib().hx_set_dense_steady(self._h, 1 if enable else 0))

    def set_close_deferral(self, enable: bool) -> int:
        return self._rc(lib().hx_set_close_deferral(self._h, 1 if enable else 0))

    def set_uniform_columns(self, enable: bool) -> int:
        """Read parameter columns holding one value as scalars (default on)."""
        return self._rc(lib().hx_set_uniform_columns(self._h, 1 if enable else 0))

    # --------------------------------------------------------------- model
    def load_model_from_spec(self, spec: ModelSpec, add_monitors: bool = True) -> int:
        """Build the model of ``spec`` and upload it (set_data_path + load_model with
        in-memory arrays instead of an export)."""
        self.build_model_from_spec(spec, add_monitors)
        self._chk(lib().hx_load_model(self._h), "load_model")
        self.spec = spec
        return 0

    def build_model_from_spec(self, spec: ModelSpec, add_monitors: bool = True) -> int:
        """The model builder's calls for ``spec`` (no GPU); load_model uploads it."""
        spec.validate()
        L = lib()
        h = self._h
        self._keep = []
        self._spec = spec
        self._chk(L.hx_set_dt(h, spec.dt), "set_dt")
        self._chk(L.hx_set_celsius(h, spec.celsius), "set_celsius")
        parent = np.ascontiguousarray(spec.parent, np.int32)
        arrs = [np.ascontiguousarray(x, np.float64) for x in (spec.a, spec.b, spec.area)]
        self._chk(L.hx_model_set_nodes(h, spec.ncell, spec.nnode, _ip(parent), *[_dp(x) for x in arrs]), "set_nodes")
        cm = np.ascontiguousarray(spec.cm, np.float64)
        self._chk(L.hx_model_set_param(h, b"capacitance", b"cm", spec.nnode, _dp(cm)), "cm")
        order = sorted(spec.mechs.keys(), key=lambda k: 0 if k.endswith("_ion") else 1)
        for name in order:
            m = spec.mechs[name]
            nodes = np.ascontiguousarray(m.nodes, np.int32)
            self._chk(L.hx_model_insert(h, _b(name), m.n, _ip(nodes)), f"insert {name}")
            for k, v in m.params.items():
                v = np.ascontiguousarray(v, np.float64)
                self._chk(L.hx_model_set_param(h, _b(name), _b(k), m.n, _dp(v)), f"{name}.{k}")
            for k, v in m.globals.items():
                self._chk(L.hx_model_set_global(h, _b(name), _b(k), float(v)), f"global {name}.{k}")
            if m.iontype is not None:
                it = np.ascontiguousarray(m.iontype, np.int32)
                self._chk(L.hx_model_set_iontype(h, _b(name), m.n, _ip(it)), f"iontype {name}")
        for gid, nd, thr in zip(spec.presyn_gid, spec.presyn_node, spec.presyn_thr):
            self._chk(L.hx_model_add_presyn(h, int(gid), int(nd), float(thr)), "presyn")
        for k in range(spec.n_vecstim):
            tr = np.ascontiguousarray(spec.vecstim_train(k), np.float64)
            if tr.size:
                self._chk(L.hx_model_set_vecstim(h, k, tr.size, _dp(tr)), "vecstim")
        for tgt, nc in spec.netcons.items():
            tb = _b(tgt)
            for i in range(nc.inst.shape[0]):
                self._chk(L.hx_model_add_netcon(h, int(nc.src_kind[i]), int(nc.src[i]), tb, int(nc.inst[i]),
                                                float(nc.weight[i]), float(nc.delay[i])), "netcon")
        for s, g in zip(spec.gap_src_node, spec.gap_halfgap):
            self._chk(L.hx_model_add_gap(h, int(s), int(g)), "gap")
        for vp in spec.vecplay:
            tv = np.ascontiguousarray(vp.tvec, np.float64)
            yv = np.ascontiguousarray(vp.yvec, np.float64)
            self._chk(L.hx_add_vecplay(h, _b(vp.mech), _b(vp.var), vp.idx, tv.size, _dp(tv), _dp(yv)), "vecplay")
        self.monitor_handles: List[int] = []
        if add_monitors:
            for mech, var, idx in spec.monitors:
                self.monitor_handles.append(self._chk(L.hx_add_monitor(h, _b(mech), _b(var), int(idx)),
                                                      f"monitor {mech}.{var}[{idx}]"))
        return 0

    def info(self, key: str) -> int:
        return int(lib().hx_get_info(self._h, _b(key)))

    # --------------------------------------------------------------- stepping
    def finitialize(self, v_init: float = -65.0) -> int:
        return self._chk(lib().hx_finitialize(self._h, float(v_init)), "finitialize")

    def run(self, tstop: float) -> int:
        return self._chk(lib().hx_run(self._h, float(tstop)), "run")

    def continue_run(self, runtime: float) -> int:
        return self._chk(lib().hx_continue_run(self._h, float(runtime)), "continue_run")

    def fadvance(self) -> int:
        return self._chk(lib().hx_fadvance(self._h), "fadvance")

    def get_t(self) -> float:
        return lib().hx_get_t(self._h)

    # --------------------------------------------------------------- monitors
    def add_monitor(self, mech: str, var: str, idx: int) -> int:
        h = lib().hx_add_monitor(self._h, _b(mech), _b(var), int(idx))
        if h >= 0:
            if not hasattr(self, "monitor_handles"):
                self.monitor_handles = []
            self.monitor_handles.append(h)
        return h

    def add_monitor_with_array(self, mech: str, var: str, idx: int, array_index: int) -> int:
        """Variables here are scalars: array_index must be 0."""
        if int(array_index) != 0:
            return self._pyfail(f"{mech}.{var} is not an array variable (array_index {array_index})")
        return self.add_monitor(mech, var, idx)

    def get_monitor_handle(self, mech: str, var: str, idx: int) -> int:
        return lib().hx_get_monitor_handle(self._h, _b(mech), _b(var), int(idx))

    def get_monitor_handle_with_array(self, mech: str, var: str, idx: int, array_index: int) -> int:
        if int(array_index) != 0:
            return self._pyfail(f"{mech}.{var} is not an array variable (array_index {array_index})")
        return self.get_monitor_handle(mech, var, idx)

    def flush_recorders(self) -> int:
        return self._rc(lib().hx_flush_recorders(self._h))

    def get_monitor_data(self, handle: int) -> List[float]:
        return self.monitor_array(handle).tolist()

    def monitor_array(self, handle: int) -> np.ndarray:
        L = lib()
        n = L.hx_get_monitor_len(self._h, handle)
        if n < 0:
            return np.zeros(0)
        out = np.empty(n)
        L.hx_get_monitor_data(self._h, handle, _dp(out), n)
        return out

    def get_multiple_monitor_data(self, handles: Sequence[int]) -> Dict[int, List[float]]:
        return {h: self.get_monitor_data(h) for h in handles}

    def traces(self) -> np.ndarray:
        hs = getattr(self, "monitor_handles", [])
        return np.stack([self.monitor_array(h) for h in hs]) if hs else np.zeros((0, 0))

    # --------------------------------------------------------------- variables
    def get_variable_handle(self, mech: str, var: str, idx: int) -> int:
        return lib().hx_get_variable_handle(self._h, _b(mech), _b(var), int(idx))

    def get_variable_handle_with_array(self, mech: str, var: str, idx: int, array_index: int) -> int:
        if int(array_index) != 0:
            return self._pyfail(f"{mech}.{var} is not an array variable (array_index {array_index})")
        return self.get_variable_handle(mech, var, idx)

    def get_variable_value_with_array(self, mech: str, var: str, idx: int, array_index: int) -> float:
        if int(array_index) != 0:
            raise HelioxError(f"{mech}.{var} is not an array variable (array_index {array_index})")
        return self.get_variable_value(mech, var, idx)

    def set_variable_value_with_array(self, val: float, mech: str, var: str, idx: int, array_index: int) -> int:
        if int(array_index) != 0:
            return self._pyfail(f"{mech}.{var} is not an array variable (array_index {array_index})")
        return self.set_variable_value(val, mech, var, idx)

    def get_variable_by_handle(self, handle: int) -> float:
        out = np.zeros(1)
        self._chk(lib().hx_get_variable_by_handle(self._h, int(handle), _dp(out)), "get_variable_by_handle")
        return float(out[0])

    def set_variable_by_handle(self, handle: int, value: float) -> int:
        return self._rc(lib().hx_set_variable_by_handle(self._h, int(handle), float(value)))

    def get_variables_by_handles(self, handles: Sequence[int]) -> List[float]:
        hs = np.ascontiguousarray(handles, np.int32)
        out = np.zeros(hs.size)
        self._chk(lib().hx_get_variables_by_handles(self._h, hs.size, _ip(hs), _dp(out)), "get_variables_by_handles")
        return out.tolist()

    def get_variables_by_handles_f32_into(self, handles: np.ndarray, out: np.ndarray) -> int:
        hs = np.ascontiguousarray(handles, np.int32)
        if out.dtype != np.float32 or not out.flags.c_contiguous or out.size < hs.size:
            raise ValueError("out must be a C-contiguous float32 array of at least len(handles)")
        return self._rc(lib().hx_get_variables_by_handles_f32_into(self._h, hs.size, _ip(hs),
                                                                    out.ctypes.data_as(_F)))

    def set_variables_by_handles(self, handles: Sequence[int], values: Sequence[float]) -> int:
        hs = np.ascontiguousarray(handles, np.int32)
        vs = np.ascontiguousarray(values, np.float64)
        return self._rc(lib().hx_set_variables_by_handles(self._h, hs.size, _ip(hs), _dp(vs)))

    def get_variable_value(self, mech: str, var: str, idx: int) -> float:
        out = np.zeros(1)
        self._chk(lib().hx_get_variable_value(self._h, _b(mech), _b(var), int(idx), _dp(out)), "get_variable_value")
        return float(out[0])

    def set_variable_value(self, val: float, mech: str, var: str, idx: int) -> int:
        return self._rc(lib().hx_set_variable_value(self._h, float(val), _b(mech), _b(var), int(idx)))

    def get_array(self, mech: str, var: str) -> np.ndarray:
        n = self.spec.nnode if mech in ("global", "node", "capacitance") else self.spec.mechs[mech].n
        out = np.empty(n)
        self._chk(lib().hx_get_array(self._h, _b(mech), _b(var), _dp(out), n), f"get_array {mech}.{var}")
        return out

    # --------------------------------------------------------------- vecplay
    def add_vecplay(self, mech: str, var: str, idx: int, tvec, yvec) -> int:
        tv = np.ascontiguousarray(tvec, np.float64)
        yv = np.ascontiguousarray(yvec, np.float64)
        if tv.size != yv.size:
            return -1
        return self._rc(lib().hx_add_vecplay(self._h, _b(mech), _b(var), int(idx), tv.size, _dp(tv), _dp(yv)))

    def update_vecplay(self, mech: str, var: str, idx: int, tvec, yvec) -> int:
        tv = np.ascontiguousarray(tvec, np.float64)
        yv = np.ascontiguousarray(yvec, np.float64)
        return self._rc(lib().hx_update_vecplay(self._h, _b(mech), _b(var), int(idx), tv.size, _dp(tv), _dp(yv)))

    def remove_vecplay(self, mech: str, var: str, idx: int) -> int:
        return self._rc(lib().hx_remove_vecplay(self._h, _b(mech), _b(var), int(idx)))

    def get_all_vecplay_keys(self) -> List[List[str]]:
        L = lib()
        n = L.hx_get_vecplay_keys(self._h, None, 0)
        buf = C.create_string_buffer(max(n, 1))
        L.hx_get_vecplay_keys(self._h, buf, len(buf))
        return [line.split("\t") for line in buf.value.decode().splitlines() if line]

    def has_vecplay(self, mech: str, var: str, idx: int) -> bool:
        return lib().hx_has_vecplay(self._h, _b(mech), _b(var), int(idx)) == 1

    # --------------------------------------------------------------- spikes
    def spikes(self):
        L = lib()
        n = L.hx_get_spike_count(self._h)
        t = np.empty(n)
        g = np.empty(n, np.int32)
        L.hx_get_spikes(self._h, _dp(t), _ip(g), n)
        return t, g

    def netstim_spikes(self):
        """(times, NetStim instances) of every NetStim spike since finitialize, ordered by
        time then instance."""
        L = lib()
        n = self._chk(L.hx_get_netstim_spikes(self._h, None, None, 0), "netstim_spikes")
        t = np.empty(n)
        i = np.empty(n, np.int32)
        if n:
            self._chk(L.hx_get_netstim_spikes(self._h, _dp(t), _ip(i), n), "netstim_spikes")
        return t, i

    def output_spikes(self, folder: str) -> str:
        """Write ``<folder>/spk.dat`` in the reference's format (Simulate::output_spikes);
        returns the file's path."""
        self._chk(lib().hx_output_spikes(self._h, _b(folder)), "output_spikes")
        return os.path.join(folder, "spk.dat")

    def set_spike_output_enabled(self, enable: bool) -> int:
        """Write spk.dat into the output directory after every run / continue_run."""
        return self._rc(lib().hx_set_spike_output_enabled(self._h, int(bool(enable))))

    def is_spike_output_enabled(self) -> bool:
        return bool(lib().hx_is_spike_output_enabled(self._h))

    def set_hdf5_enabled(self, enable: bool) -> int:
        """Monitor samples to <output_dir>/sim_out.h5 at /group_0/<mech>/<var>/<idx>
        (created at the next finitialize, appended by every run call)."""
        return self._rc(lib().hx_set_hdf5_enabled(self._h, int(bool(enable))))

    def is_hdf5_enabled(self) -> bool:
        return bool(lib().hx_is_hdf5_enabled(self._h))

    def set_output_dir(self, dir: str) -> int:
        return self._rc(lib().hx_set_output_dir(self._h, _b(dir)))

    def get_spk_by_gid(self, gid: int) -> List[float]:
        L = lib()
        n = L.hx_get_spike_count(self._h)
        out = np.empty(max(n, 1))
        k = L.hx_get_spk_by_gid(self._h, int(gid), _dp(out), out.size)
        return out[:k].tolist()

    # --------------------------------------------------------------- profiling
    def set_profiling(self, enable: bool, classes: Optional[Sequence[str]] = None) -> int:
        """Per-kernel-class HIP-event timing; ``classes`` limits it to those classes."""
        if enable and classes is not None:
            return self._rc(lib().hx_set_profiling_classes(self._h, _b(",".join(classes))))
        return self._rc(lib().hx_set_profiling(self._h, 1 if enable else 0))

    # ---- adjoint and Adam ----
    def tape_begin(self, max_steps: int) -> int:
        """Record the next run for the adjoint (call before finitialize)."""
        return self._chk(lib().hx_tape_begin(self._h, int(max_steps)), "tape_begin")

    def tape_length(self) -> int:
        return lib().hx_tape_length(self._h)

    def adjoint(self, loss_nodes, target) -> float:
        """Backward sweep for loss = mean((v[loss_nodes] after each taped step - target)^2);
        target has shape (tape_length, len(loss_nodes)).  Returns the loss."""
        nodes = np.ascontiguousarray(loss_nodes, np.int32)
        tgt = np.ascontiguousarray(target, np.float64)
        if tgt.ndim != 2 or tgt.shape[1] != nodes.size:
            raise ValueError("target must have shape (steps, len(loss_nodes))")
        out = C.c_double()
        self._chk(lib().hx_adjoint(self._h, int(nodes.size), _ip(nodes), _dp(tgt), int(tgt.shape[0]),
                                   C.byref(out)), "adjoint")
        return out.value

    def gradient(self, mech: str, var: str) -> np.ndarray:
        n = self._spec_count(mech)
        out = np.zeros(max(n, 1))
        k = self._chk(lib().hx_get_gradient(self._h, _b(mech), _b(var), _dp(out), out.size), "get_gradient")
        return out[:k]

    def _spec_count(self, mech: str) -> int:
        spec = getattr(self, "_spec", None)
        if spec is not None and mech in spec.mechs:
            return spec.mechs[mech].nodes.size
        return 1 << 22

    def adam_create(self, beta1: float = 0.9, beta2: float = 0.999, eps: float = 1e-8) -> int:
        return self._chk(lib().hx_adam_create(self._h, beta1, beta2, eps), "adam_create")

    def adam_add_group(self, opt: int, mech: str, var: str, instances, impedance: float = 1.0) -> int:
        inst = np.ascontiguousarray(instances, np.int32)
        return self._chk(lib().hx_adam_add_group(self._h, opt, _b(mech), _b(var), int(inst.size), _ip(inst),
                                                 impedance), "adam_add_group")

    def adam_step(self, opt: int, lr: float, inv_record_steps: float = 1.0) -> int:
        return self._chk(lib().hx_adam_step(self._h, opt, lr, inv_record_steps), "adam_step")

    def adam_state(self, opt: int, ngroup: int):
        step = C.c_longlong()
        m = np.zeros(max(ngroup, 1))
        v = np.zeros(max(ngroup, 1))
        self._chk(lib().hx_adam_get_state(self._h, opt, C.byref(step), _dp(m), _dp(v), m.size), "adam_state")
        return step.value, m[:ngroup], v[:ngroup]

    # ---- learn gradient surface (SimWrapper.cpp:533-1183; PyBindings.cpp:88-200).
    # Like the reference's bindings these return 0 / -1; last_error() holds the message.
    # --------------------------------------------------------------- optimizers
    def create_optimizer(self, optimizer_type: str) -> int:
        """"sgd", "momentum" or "adam"; returns the optimizer id (-1 on error)."""
        return lib().hx_create_optimizer(self._h, _b(optimizer_type))

    def configure_optimizer(self, optimizer_id: int, momentum: float = 0.9, beta1: float = 0.9,
                            beta2: float = 0.999, epsilon: float = 1e-8) -> int:
        return self._rc(lib().hx_configure_optimizer(self._h, int(optimizer_id), float(momentum), float(beta1),
                                                     float(beta2), float(epsilon)))

    def optimizer_add_param(self, optimizer_id: int, weight_handle: int, grad_handle: int,
                            impedance: float = 1.0) -> int:
        return lib().hx_optimizer_add_param(self._h, int(optimizer_id), int(weight_handle), int(grad_handle),
                                            float(impedance))

    def optimizer_add_param_batch(self, optimizer_id: int, weight_handles: Sequence[int],
                                  grad_handles: Sequence[int], impedance: float = 1.0) -> int:
        w = np.ascontiguousarray(weight_handles, np.int32)
        g = np.ascontiguousarray(grad_handles, np.int32)
        if w.size != g.size or w.size == 0:
            return self._pyfail("optimizer_add_param_batch: handle lists must be non-empty and have equal length")
        return lib().hx_optimizer_add_param_batch(self._h, int(optimizer_id), w.size, _ip(w), _ip(g),
                                                  float(impedance))

    def optimizer_step(self, optimizer_id: int, learning_rate: float, record_time: float, dt: float) -> int:
        return self._rc(lib().hx_optimizer_step(self._h, int(optimizer_id), float(learning_rate),
                                                float(record_time), float(dt)))

    def optimizer_step_with_inv_record_steps(self, optimizer_id: int, learning_rate: float,
                                             inv_record_steps: float) -> int:
        return self._rc(lib().hx_optimizer_step_with_inv_record_steps(self._h, int(optimizer_id),
                                                                      float(learning_rate),
                                                                      float(inv_record_steps)))

    def optimizer_add_external_grads(self, optimizer_id: int, weight_handles: Sequence[int],
                                     impedance: float = 1.0) -> int:
        w = np.ascontiguousarray(weight_handles, np.int32)
        return self._rc(lib().hx_optimizer_add_external_grads(self._h, int(optimizer_id), w.size, _ip(w),
                                                              float(impedance)))

    def optimizer_set_external_grads_f32(self, optimizer_id: int, grads: np.ndarray) -> int:
        g = np.asarray(grads)
        if g.dtype != np.float32 or g.ndim != 1 or not g.flags.c_contiguous:
            raise TypeError("grads must be a 1-D C-contiguous float32 array")
        return self._rc(lib().hx_optimizer_set_external_grads_f32(self._h, int(optimizer_id), g.size,
                                                                  g.ctypes.data_as(_F)))

    def optimizer_clear_external_grads(self, optimizer_id: int) -> int:
        return self._rc(lib().hx_optimizer_clear_external_grads(self._h, int(optimizer_id)))

    def optimizer_reset_state(self, optimizer_id: int) -> int:
        return self._rc(lib().hx_optimizer_reset_state(self._h, int(optimizer_id)))

    def optimizer_get_adam_state(self, optimizer_id: int):
        """(step_count, m, v, beta1, beta2, epsilon); the defaults with empty m, v if the
        optimizer is not Adam (as SimWrapper::optimizer_get_adam_state)."""
        L = lib()
        step = C.c_longlong(0)
        b1, b2, ep = np.zeros(1), np.zeros(1), np.zeros(1)
        n = L.hx_optimizer_get_adam_state(self._h, int(optimizer_id), C.byref(step), None, None, 0,
                                          _dp(b1), _dp(b2), _dp(ep))
        if n < 0:
            return 0, [], [], 0.9, 0.999, 1e-8
        m, v = np.zeros(max(n, 1)), np.zeros(max(n, 1))
        L.hx_optimizer_get_adam_state(self._h, int(optimizer_id), C.byref(step), _dp(m), _dp(v), n,
                                      _dp(b1), _dp(b2), _dp(ep))
        return int(step.value), m[:n].tolist(), v[:n].tolist(), float(b1[0]), float(b2[0]), float(ep[0])

    def optimizer_set_adam_state(self, optimizer_id: int, step_count: int, m: Sequence[float], v: Sequence[float],
                                 beta1: float = 0.9, beta2: float = 0.999, epsilon: float = 1e-8) -> int:
        mm = np.ascontiguousarray(m, np.float64)
        vv = np.ascontiguousarray(v, np.float64)
        if mm.size != vv.size:
            return self._pyfail("optimizer_set_adam_state: m and v differ in length")
        return self._rc(lib().hx_optimizer_set_adam_state(self._h, int(optimizer_id), int(step_count), mm.size,
                                                          _dp(mm), _dp(vv), float(beta1), float(beta2),
                                                          float(epsilon)))

    # --------------------------------------------------------------- gap junctions
    def add_gap_source(self, sid: int, src_mech: str, src_var: str, src_idx: int) -> int:
        return lib().hx_add_gap_source(self._h, int(sid), _b(src_mech), _b(src_var), int(src_idx))

    def add_gap_target(self, sid: int, tgt_mech: str, tgt_var: str, tgt_idx: int) -> int:
        return self._rc(lib().hx_add_gap_target(self._h, int(sid), _b(tgt_mech), _b(tgt_var), int(tgt_idx)))

    def clear_all_gap_junctions(self) -> int:
        return self._rc(lib().hx_clear_all_gap_junctions(self._h))

    def get_next_available_sid(self) -> int:
        return lib().hx_get_next_available_sid(self._h)

    def get_gap_junction(self, sid: int) -> Dict[str, object]:
        mech = C.create_string_buffer(256)
        var = C.create_string_buffer(256)
        idx = C.c_int(0)
        nt = C.c_int(0)
        if lib().hx_get_gap_junction(self._h, int(sid), mech, 256, var, 256, C.byref(idx), C.byref(nt)) != 0:
            return {}
        return {"src_mech": mech.value.decode(), "src_var": var.value.decode(), "src_idx": idx.value,
                "num_targets": nt.value, "is_dynamic": True}

    def get_all_gap_junctions(self) -> Dict[int, Dict[str, object]]:
        L = lib()
        n = L.hx_get_gap_junction_sids(self._h, None, 0)
        sids = np.zeros(max(n, 1), np.int32)
        L.hx_get_gap_junction_sids(self._h, _ip(sids), n)
        return {int(s): self.get_gap_junction(int(s)) for s in sids[:n]}

    # --------------------------------------------------------------- input batches
    def register_netstim_batch(self, handle_triplets, interval_scale: float = 1.0, start_base: float = 0.0,
                               epsilon: float = 1e-6, number: float = 1.0) -> int:
        """NetStim inputs driven by pixel values (SimRuntimeCore.cpp:694-790): triplets of
        (interval, start, number) variable handles; see set_input_batch_pixels."""
        trip = [tuple(int(x) for x in t) for t in handle_triplets]
        if not trip:
            return self._pyfail("register_netstim_batch: handle list is empty")
        nh = lib().hx_get_info(self._h, b"handles")
        if any(h < 0 or h >= nh for t in trip for h in t):
            return self._pyfail("register_netstim_batch: invalid handle")
        return self._add_batch(("NetStim", trip, float(interval_scale), float(start_base), float(epsilon),
                                float(number)))

    def register_vecstim_batch(self, mech_indices, spike_scale: float = 1.0, start_base: float = 0.0,
                               epsilon: float = 1e-6, spike_count: int = 1) -> int:
        """VecStim inputs driven by pixel values (SimRuntimeCore.cpp:791-826): one VecStim
        instance per pixel."""
        idx = [int(i) for i in mech_indices]
        if not idx:
            return self._pyfail("register_vecstim_batch: mech list is empty")
        if any(i < 0 for i in idx):
            return self._pyfail("register_vecstim_batch: invalid mech index")
        return self._add_batch(("VecStim", idx, float(spike_scale), float(start_base), float(epsilon),
                                int(spike_count)))

    def _add_batch(self, b) -> int:
        if not hasattr(self, "_batches"):
            self._batches = []
        self._batches.append(b)
        return len(self._batches) - 1

    def set_input_batch_pixels(self, batch_id: int, pixels) -> int:
        """Encode one input image (SimRuntimeCore.cpp:827-915): with d = max(pixel + eps, eps),
        NetStim interval = interval_scale / d, start = start_base + interval, number as given;
        VecStim spikes at start_base + k * spike_scale / d for k = 1..spike_count.  NetStim
        and VecStim inputs take the new values at the next finitialize."""
        bs = getattr(self, "_batches", [])
        if not 0 <= int(batch_id) < len(bs):
            return self._pyfail(f"set_input_batch_pixels: batch {batch_id} not found")
        kind, items, scale, base, eps, count = bs[int(batch_id)]
        px = np.asarray(pixels, np.float64).ravel()
        if px.size != len(items):
            return self._pyfail(f"set_input_batch_pixels: size mismatch batch={len(items)}, got={px.size}")
        d = np.maximum(px + eps, eps)
        if kind == "NetStim":
            for (hi, hs, hn), dv in zip(items, d):
                interval = scale / dv
                for h, val in ((hi, interval), (hs, base + interval), (hn, count)):
                    if self.set_variable_by_handle(h, val) != 0:
                        return -1
            return 0
        L = lib()
        for mi, dv in zip(items, d):
            step = scale / dv
            times = np.ascontiguousarray(base + step * np.arange(1, count + 1, dtype=np.float64))
            if L.hx_model_set_vecstim(self._h, mi, times.size, _dp(times)) != 0:
                return -1
        return 0

    # --------------------------------------------------------------- CoreNEURON exports
    def set_data_path(self, path: str) -> int:
        """Directory of a CoreNEURON export read by the next load_model (SimWrapper.cpp:18)."""
        return self._rc(lib().hx_set_data_path(self._h, _b(str(path))))

    def load_model(self) -> int:
        """Read the export at the data path and upload the model (SimWrapper.cpp:26-31).
        Monitors added before the call are resolved against the loaded model."""
        rc = lib().hx_load_model(self._h)
        if rc >= 0:
            self.spec = None
        return self._rc(rc)

    def read_export(self) -> int:
        """Only the read half of load_model: the export into the model builder (no GPU)."""
        return self._rc(lib().hx_model_read_export(self._h))

    def model_digest(self) -> str:
        """Counts and hashes of what the model builder holds (no reference counterpart)."""
        n = lib().hx_model_digest(self._h, None, 0)
        buf = C.create_string_buffer(n)
        lib().hx_model_digest(self._h, buf, n)
        return buf.value.decode()

    def set_permute_type(self, permute_type: int) -> int:
        """Accepted for compatibility: the solver uses its own node order (solve units)."""
        if int(permute_type) not in (0, 1, 2, 3):
            return self._pyfail(f"set_permute_type: unknown type {permute_type}")
        self._permute_type = int(permute_type)
        return 0

    def set_user_mod_num(self, num: int) -> None:
        """Numbering of artificial presyns in an export: -(type + index * num) (SimWrapper.cpp:481)."""
        self._user_mod_num = int(num)
        if lib().hx_set_user_mod_num(self._h, int(num)) < 0:
            raise HelioxError(f"set_user_mod_num: {self.last_error()}")

    def call_mech_func(self, mech_name: str, func_name: str, *args) -> float:
        """A registered mechanism function (SimWrapper.cpp:461-468, FunctionRegistry
        func_table.cuh:97-130).  The one the reference registers is
        ``VecStim.play(index, times)`` (vecevent.h:42-45, vecevent.cpp:280-309): the
        instance's spike times become ``times``; an empty list changes nothing.  The next
        finitialize reads the new times from the first; in a run already initialised the
        instance delivers the event it has queued and then continues from the new times at
        the position it has reached (``hx_call_mech_func``).  Returns 0.  As the reference's
        registry throws, an unregistered name or a wrong argument count raises
        ``RuntimeError``."""
        self._py_err = None
        if (mech_name, func_name) != ("VecStim", "play"):
            raise HelioxError(f"function not registered: {mech_name}.{func_name}")
        if len(args) != 2:
            raise HelioxError(f"{mech_name}.{func_name}: takes 2 arguments (index, times), got {len(args)}")
        idx, times = args
        if isinstance(times, (int, float)):
            times = [times]
        tr = np.ascontiguousarray(np.asarray(times, dtype=np.float64).ravel())
        rc = lib().hx_call_mech_func(self._h, _b(mech_name), _b(func_name), int(idx), tr.size, _dp(tr))
        self._chk(rc, f"call_mech_func {mech_name}.{func_name}")
        return 0.0

    def set_dense_blocks_f32(self, blocks) -> int:
        """Upload (bn, bn, K_len) float32 blocks; returns K_len or -1 (SimWrapper.cpp:533-572)."""
        self._py_err = None
        arrs = [np.ascontiguousarray(b, np.float32) for b in blocks]
        for a in arrs:
            if a.ndim != 3 or a.shape[0] != a.shape[1]:
                return self._pyfail("set_dense_blocks_f32: blocks must be (bn, bn, K_len)")
        ptrs = (_F * max(len(arrs), 1))(*[_fp(a) for a in arrs])
        bn = _i32([a.shape[0] for a in arrs] or [0])
        kl = _i32([a.shape[2] for a in arrs] or [0])
        self._blocks_keepalive = arrs
        return lib().hx_set_dense_blocks_f32(self._h, len(arrs), ptrs, _ip(bn), _ip(kl))

    def clear_dense_blocks(self) -> None:
        self._chk(lib().hx_clear_dense_blocks(self._h), "clear_dense_blocks")

    def simulate_output_vs_into(self, output_vs_tn: np.ndarray, output_v_handles, tstop_ms: float,
                                v_init: float) -> int:
        self._py_err = None
        out = _out_f32(output_vs_tn, "output_vs_tn")
        if out.ndim != 2:
            return self._pyfail("simulate_output_vs_into: output_vs_tn must be 2D")
        hs = _i32(output_v_handles)
        if hs.size != out.shape[1]:
            return self._pyfail("simulate_output_vs_into: output handles mismatch")
        return self._rc(lib().hx_simulate_output_vs_into(self._h, _fp(out), out.shape[0], hs.size, _ip(hs),
                                                         tstop_ms, v_init))

    @staticmethod
    def _channel(handles, dest, scale):
        h, d, sc = _i32(handles), _i32(dest), _f32(np.asarray(scale).reshape(-1))
        if not (h.size == d.size == sc.size):
            raise ValueError("handles/dest/scale size mismatch")
        return h, d, sc

    def simulate_and_capture_mapped_signals_cached(self, output_vs_tn, output_v_handles, pure_i_handles,
                                                   pure_i_dest, pure_i_scale, didv_handles, didv_dest, didv_scale,
                                                   didvpre_handles, didvpre_dest, didvpre_scale, tstop_ms: float,
                                                   k_mul: int, percise: bool, v_init: float) -> int:
        self._py_err = None
        out = _out_f32(output_vs_tn, "output_vs_tn")
        hs = _i32(output_v_handles)
        try:
            ch = [self._channel(pure_i_handles, pure_i_dest, pure_i_scale),
                  self._channel(didv_handles, didv_dest, didv_scale),
                  self._channel(didvpre_handles, didvpre_dest, didvpre_scale)]
        except ValueError as e:
            return self._pyfail(f"simulate_and_capture_mapped_signals_cached: {e}")
        if out.ndim != 2 or out.shape[1] != hs.size:
            return self._pyfail("simulate_and_capture_mapped_signals_cached: output_v_handles size mismatch")
        args = []
        for h, d, sc in ch:
            args += [h.size, _ip(h), _ip(d), _fp(sc)]
        return self._rc(lib().hx_simulate_and_capture_mapped_signals_cached(
            self._h, _fp(out), out.shape[0], hs.size, _ip(hs), *args, tstop_ms, int(k_mul), int(bool(percise)),
            v_init))

    def simulate_and_capture_mapped_signals_into(self, output_vs_tn, it_lr_tn, ditdv_lr_tn, ditdvpre_lr_tn,
                                                 output_v_handles, pure_i_handles, pure_i_dest, pure_i_scale,
                                                 didv_handles, didv_dest, didv_scale, didvpre_handles, didvpre_dest,
                                                 didvpre_scale, tstop_ms: float, k_mul: int, percise: bool,
                                                 v_init: float) -> int:
        self._py_err = None
        out = _out_f32(output_vs_tn, "output_vs_tn")
        bufs = [_out_f32(b, n) for b, n in ((it_lr_tn, "it_lr_tn"), (ditdv_lr_tn, "ditdv_lr_tn"),
                                             (ditdvpre_lr_tn, "ditdvpre_lr_tn"))]
        if any(b.ndim != 2 or b.shape != bufs[0].shape for b in bufs) or out.ndim != 2:
            return self._pyfail("simulate_and_capture_mapped_signals_into: outputs must be 2D arrays")
        hs = _i32(output_v_handles)
        if out.shape[1] != hs.size:
            return self._pyfail("simulate_and_capture_mapped_signals_into: output_vs_tn shape mismatch")
        try:
            ch = [self._channel(pure_i_handles, pure_i_dest, pure_i_scale),
                  self._channel(didv_handles, didv_dest, didv_scale),
                  self._channel(didvpre_handles, didvpre_dest, didvpre_scale)]
        except ValueError as e:
            return self._pyfail(f"simulate_and_capture_mapped_signals_into: {e}")
        args = []
        for h, d, sc in ch:
            args += [h.size, _ip(h), _ip(d), _fp(sc)]
        T, N = bufs[0].shape
        return self._rc(lib().hx_simulate_and_capture_mapped_signals_into(
            self._h, _fp(out), out.shape[0], hs.size, _fp(bufs[0]), _fp(bufs[1]), _fp(bufs[2]), T, N, _ip(hs),
            *args, tstop_ms, int(k_mul), int(bool(percise)), v_init))

    def replay_compute_dw_from_cached_signals_into(self, dLtdv_lr_ot, poutput, pre_of_col, dw_out_n, dt_ms: float,
                                                   percise: bool, grad_scale: float = 1.0, eps: float = 1e-6,
                                                   grad_l2norm_threshold: float = 1e6, clip_strategy: int = 1,
                                                   clip_check_every: int = 1) -> int:
        self._py_err = None
        dl = _f32(dLtdv_lr_ot, 2)
        po, pre = _i32(poutput), _i32(pre_of_col)
        dw = _out_f32(dw_out_n, "dw_out_n")
        if dw.size != pre.size:
            return self._pyfail("replay_compute_dw_from_cached_signals_into: dw_out_n must have N entries")
        return self._rc(lib().hx_replay_compute_dw_from_cached_signals_into(
            self._h, _fp(dl), dl.shape[0], po.size, _ip(po), _ip(pre), pre.size, _fp(dw), dt_ms,
            int(bool(percise)), grad_scale, eps, grad_l2norm_threshold, int(clip_strategy), int(clip_check_every)))

    def replay_compute_dw_dx_from_cached_signals_into(self, dLtdv_lr_ot, poutput, pinput, pre_of_col, dw_out_n,
                                                      dx_lr_it, dt_ms: float, percise: bool, grad_scale: float = 1.0,
                                                      eps: float = 1e-6, grad_l2norm_threshold: float = 1e6,
                                                      clip_strategy: int = 1, clip_check_every: int = 1) -> int:
        self._py_err = None
        dl = _f32(dLtdv_lr_ot, 2)
        po, pin, pre = _i32(poutput), _i32(pinput), _i32(pre_of_col)
        dw = _out_f32(dw_out_n, "dw_out_n")
        dx = _out_f32(dx_lr_it, "dx_lr_it")
        if dw.size != pre.size or dx.shape != (pin.size, dl.shape[0]):
            return self._pyfail("replay_compute_dw_dx_from_cached_signals_into: output shape mismatch")
        return self._rc(lib().hx_replay_compute_dw_dx_from_cached_signals_into(
            self._h, _fp(dl), dl.shape[0], po.size, _ip(po), _ip(pin), pin.size, _ip(pre), pre.size, _fp(dw),
            _fp(dx), dt_ms, int(bool(percise)), grad_scale, eps, grad_l2norm_threshold, int(clip_strategy),
            int(clip_check_every)))

    def replay_compute_dw_dx_from_signals_into(self, it_lr_nt, ditdv_lr_nt, ditdvpre_lr_nt, dLtdv_lr_to, poutput,
                                               pinput, pre_of_col, dw_out_n, dx_lr_it, dt_ms: float, percise: bool,
                                               grad_scale: float = 1.0, eps: float = 1e-6,
                                               grad_l2norm_threshold: float = 1e6, clip_strategy: int = 1,
                                               clip_check_every: int = 1, noalloc: bool = False) -> int:
        """noalloc: the entry point that allocates no device memory (its buffers come from the
        library's fixed per-GPU scratch array; larger problems are refused)."""
        self._py_err = None
        it = _f32(it_lr_nt, 2)
        dv = _f32(ditdv_lr_nt, 2) if ditdv_lr_nt is not None else None
        dp = _f32(ditdvpre_lr_nt, 2) if ditdvpre_lr_nt is not None else None
        dl = _f32(dLtdv_lr_to, 2)
        po, pin, pre = _i32(poutput), _i32(pinput), _i32(pre_of_col)
        dw = _out_f32(dw_out_n, "dw_out_n")
        dx = _out_f32(dx_lr_it, "dx_lr_it")
        N, T = it.shape
        for a in (dv, dp):
            if a is not None and a.shape != it.shape:
                return self._pyfail("replay_compute_dw_dx_from_signals_into: signal shape mismatch")
        if pre.size != N or dw.size != N or dx.shape != (pin.size, dl.shape[0]):
            return self._pyfail("replay_compute_dw_dx_from_signals_into: output shape mismatch")
        null = C.cast(None, _F)
        fn = lib().hx_replay_compute_dw_dx_from_signals_into_noalloc if noalloc else \
            lib().hx_replay_compute_dw_dx_from_signals_into
        return self._rc(fn(
            self._h, _fp(it), _fp(dv) if dv is not None else null, _fp(dp) if dp is not None else null, N, T,
            _fp(dl), dl.shape[0], po.size, _ip(po), _ip(pin), pin.size, _ip(pre), _fp(dw), _fp(dx), dt_ms,
            int(bool(percise)), grad_scale, eps, grad_l2norm_threshold, int(clip_strategy), int(clip_check_every)))

    def simulate_and_replay_dw_dx_streaming_into(self, dLtdv_lr_ot, poutput, pinput, pre_of_col, dw_out_n, dx_lr_it,
                                                 pure_i_handles, pure_i_dest, pure_i_scale, didv_handles, didv_dest,
                                                 didv_scale, didvpre_handles, didvpre_dest, didvpre_scale,
                                                 tstop_ms: float, k_mul: int, percise: bool, v_init: float,
                                                 dt_ms: float, grad_scale: float = 1.0, eps: float = 1e-6,
                                                 grad_l2norm_threshold: float = 1e6, clip_strategy: int = 1,
                                                 clip_check_every: int = 1) -> int:
        self._py_err = None
        dl = _f32(dLtdv_lr_ot, 2)
        po, pin, pre = _i32(poutput), _i32(pinput), _i32(pre_of_col)
        dw = _out_f32(dw_out_n, "dw_out_n")
        dx = _out_f32(dx_lr_it, "dx_lr_it")
        if dw.size != pre.size or dx.shape != (pin.size, dl.shape[0]):
            return self._pyfail("simulate_and_replay_dw_dx_streaming_into: output shape mismatch")
        try:
            ch = [self._channel(pure_i_handles, pure_i_dest, pure_i_scale),
                  self._channel(didv_handles, didv_dest, didv_scale),
                  self._channel(didvpre_handles, didvpre_dest, didvpre_scale)]
        except ValueError as e:
            return self._pyfail(f"simulate_and_replay_dw_dx_streaming_into: {e}")
        args = []
        for h, d, sc in ch:
            args += [h.size, _ip(h), _ip(d), _fp(sc)]
        return self._rc(lib().hx_simulate_and_replay_dw_dx_streaming_into(
            self._h, _fp(dl), dl.shape[0], po.size, _ip(po), _ip(pin), pin.size, pre.size, _ip(pre), _fp(dw),
            _fp(dx), *args, tstop_ms, int(k_mul), int(bool(percise)), v_init, dt_ms, grad_scale, eps,
            grad_l2norm_threshold, int(clip_strategy), int(clip_check_every)))

    def set_cell_groups(self, ngroup: int) -> None:
        """Cell groups issued on separate streams when nothing couples them (0 automatic, 1 off).
        Call before loading the model."""
        self._chk(lib().hx_set_cell_groups(self._h, int(ngroup)), "set_cell_groups")

    def set_solver_root(self, centre: bool) -> None:
        """Root each cell's tree solve at the midpoint of its longest path (default) or at
        the model root.  Call before loading the model."""
        self._chk(lib().hx_set_solver_root(self._h, int(bool(centre))), "set_solver_root")

    def set_solve_unit_cells(self, cells: int) -> None:
        """Cells per solve unit (one wavefront each); 0 lets the library choose.  Call
        before loading the model; results do not depend on it."""
        self._chk(lib().hx_set_solve_unit_cells(self._h, int(cells)), "set_solve_unit_cells")

    def set_solve_waves(self, waves: int) -> None:
        """Solve units per workgroup (one wavefront each); 0 lets the library choose.  Call
        before loading the model; results do not depend on it."""
        self._chk(lib().hx_set_solve_waves(self._h, int(waves)), "set_solve_waves")

    def set_solve_resident(self, enable: bool) -> None:
        """Hold each solve unit whole in LDS when it fits (the default) or always stream its
        rounds from HBM.  Call before loading the model; the same bits either way."""
        self._chk(lib().hx_set_solve_resident(self._h, int(bool(enable))), "set_solve_resident")

    def set_solve_voltage(self, enable: bool) -> None:
        """Let a model whose node kernel makes every term of d and rhs solve for the new
        voltage directly (the default), or always solve for the change, as the reference
        does.  The two agree to rounding."""
        self._chk(lib().hx_set_solve_voltage(self._h, int(bool(enable))), "set_solve_voltage")

    def set_group_streams(self, enable: bool) -> None:
        """Allow the cell groups' own streams in the following runs (same results either way)."""
        self._chk(lib().hx_set_group_streams(self._h, int(bool(enable))), "set_group_streams")

    def set_replay_timing(self, enable: bool) -> None:
        self._chk(lib().hx_set_replay_timing(self._h, int(bool(enable))), "set_replay_timing")

    def replay_kernel_time(self):
        ms = C.c_double()
        n = C.c_longlong()
        self._chk(lib().hx_get_replay_kernel_time(self._h, C.byref(ms), C.byref(n)), "replay_kernel_time")
        return ms.value, n.value

    def kernel_time(self, kernel: str):
        ms = C.c_double()
        n = C.c_longlong()
        self._chk(lib().hx_get_kernel_time(self._h, _b(kernel), C.byref(ms), C.byref(n)), "kernel_time")
        return ms.value, n.value


def philox4x32(ctr, key):
    """One Philox4x32-10 block of the library's NetStim streams (diagnostic)."""
    c = (C.c_uint32 * 4)(*[int(x) for x in ctr])
    k = (C.c_uint32 * 2)(*[int(x) for x in key])
    out = (C.c_uint32 * 4)()
    if lib().hx_random123_philox4x32(c, k, out) != 0:
        raise HelioxError("hx_random123_philox4x32 failed")
    return [int(x) for x in out]


def netstim_train(dt, t_end, interval=10.0, number=10.0, start=50.0, noise=0.0, ids=(0, 0, 0)):
    """Self-event times of one NetStim instance as the library makes them (diagnostic)."""
    L = lib()
    args = (float(dt), float(t_end), float(interval), float(number), float(start), float(noise),
            int(ids[0]), int(ids[1]), int(ids[2]))
    n = L.hx_netstim_train(*args, None, 0)
    if n < 0:
        raise HelioxError("hx_netstim_train failed")
    out = np.empty(max(n, 1))
    L.hx_netstim_train(*args, _dp(out), n)
    return out[:n]


def emulate_tree_solve(ncell, parent, a, b, cm, cfac, v, d, rhs, unit_cells=0):
    """Host emulation of the device tree solve (same chunk schedule); returns (v_new, nchunk_max, nround_max).
    unit_cells: cells per solve unit (0: the library's choice)."""
    L = lib()
    parent = np.ascontiguousarray(parent, np.int32)
    a, b, cm, d, rhs = (np.ascontiguousarray(x, np.float64) for x in (a, b, cm, d, rhs))
    vv = np.array(v, np.float64)
    nc = C.c_int()
    nr = C.c_int()
    rc = L.hx_emulate_tree_solve_units(int(ncell), parent.size, _ip(parent), _dp(a), _dp(b), _dp(cm),
                                       float(cfac), _dp(vv), _dp(d), _dp(rhs), int(unit_cells), C.byref(nc),
                                       C.byref(nr))
    if rc == -2:
        raise HelioxError("hx_emulate_tree_solve: the round length bound changed a result")
    if rc != 0:
        raise HelioxError("hx_emulate_tree_solve failed")
    return vv, nc.value, nr.value
