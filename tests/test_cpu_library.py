"""CPU-side checks of the HIP library: exported C ABI, host-side solver schedule,
workload generator, and error behaviour that needs no GPU."""
import os
import re

import numpy as np
import pytest

import oracle
from heliox_amd import Sim, build_config, emulate_tree_solve, lib
from heliox_amd.sim import SIGNATURES

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    text = open(os.path.join(ROOT, "include", "heliox.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hx_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    L = lib()
    syms = header_symbols()
    assert len(syms) > 40
    for s in syms:
        assert hasattr(L, s), f"{s} declared in include/heliox.h but not exported"
    # and the Python binding types every one of them
    assert set(syms) == set(SIGNATURES), set(syms) ^ set(SIGNATURES)


def test_entry_points_complete_a_deferred_state_update():
    """A stepping call may return with its last state update pending; every other
    entry point that takes a handle must complete it (HX_SETTLE) before it reads or
    changes the model.  The exempt ones read only host-side values."""
    src = open(os.path.join(ROOT, "heliox_amd", "csrc", "runtime.cpp")).read()
    stepping = {"hx_run", "hx_continue_run", "hx_fadvance"}
    host_only = {"hx_destroy", "hx_last_error", "hx_get_dt", "hx_get_t", "hx_get_info",
                 "hx_is_spike_output_enabled", "hx_is_hdf5_enabled", "hx_get_spike_count",
                 "hx_tape_length", "hx_get_spikes", "hx_get_spk_by_gid", "hx_output_spikes",
                 "hx_set_profiling", "hx_set_profiling_classes", "hx_get_kernel_time"}
    seen = set()
    for m in re.finditer(r"^(?:int|void|double|long long|const char\*) (hx_\w+)\(\s*hx_sim\* sim", src, re.M):
        name = m.group(1)
        seen.add(name)
        body = src[src.find("{", m.end()):][:200]
        first = body[1:].strip().split("\n")[0]
        if name in stepping:
            assert "DeferScope" in src[m.end():src.find("\n}\n", m.end())], name
        elif name not in host_only:
            assert first == "HX_SETTLE(sim);", f"{name} does not complete a deferred state update first"
    assert stepping <= seen and len(seen) > 80


def test_nm_exports_match_header():
    so = os.path.join(ROOT, "heliox_amd", "libheliox_amd.so")
    out = os.popen(f"nm -D --defined-only {so}").read()
    exported = set(re.findall(r"\b(hx_[a-z0-9_]+)\b", out))
    assert set(header_symbols()) <= exported


# ---------------------------------------------------------------------------
# solver schedule (host emulation of the device tree solve)
# ---------------------------------------------------------------------------
def assemble_and_solve_reference(spec, v, dm, rm, cfac):
    n = spec.nnode
    d = dm + cfac * spec.cm
    rhs = rm.copy()
    p = spec.parent
    for i in range(spec.ncell, n):
        dv = v[p[i]] - v[i]
        rhs[i] -= spec.b[i] * dv
        rhs[p[i]] += spec.a[i] * dv
    for i in range(spec.ncell, n):
        d[i] -= spec.b[i]
        d[p[i]] -= spec.a[i]
    return v + oracle.solve_serial(spec.ncell, p, spec.a, spec.b, d, rhs)


@pytest.mark.parametrize("config,ncell", [(1, 3), (2, 4), (3, 2), (4, 6), (5, 2)])
def test_emulated_chunk_solve_matches_serial_hines(config, ncell):
    spec = build_config(config, ncell, 1.0)
    rng = np.random.default_rng(config)
    n = spec.nnode
    v = rng.uniform(-80, 20, n)
    dm = rng.uniform(0.5, 2.0, n) * 1e-3
    rm = rng.normal(0, 1e-3, n)
    cfac = 1e-3 / 0.025
    ref = assemble_and_solve_reference(spec, v, dm, rm, cfac)
    got, nchunk, nround = emulate_tree_solve(spec.ncell, spec.parent, spec.a, spec.b, spec.cm, cfac, v, dm, rm)
    dx = ref - v
    assert np.max(np.abs(got - ref)) <= 1e-12 * max(1.0, np.max(np.abs(dx)))
    assert nchunk > 0 and nround > 0


@pytest.mark.parametrize("config,ncell,sizes", [(2, 7, (2, 3, 7)), (3, 3, (2,)), (4, 9, (2, 4, 9))])
def test_solve_units_change_no_bit(config, ncell, sizes):
    """Cells packed into solve units of several sizes (one schedule per unit, the
    cells' chunks interleaved in shared rounds) give the same bits as one cell per
    unit, and the serial Hines solve's values."""
    spec = build_config(config, ncell, 1.0)
    rng = np.random.default_rng(10 + config)
    n = spec.nnode
    v = rng.uniform(-80, 20, n)
    dm = rng.uniform(0.5, 2.0, n) * 1e-3
    rm = rng.normal(0, 1e-3, n)
    cfac = 1e-3 / 0.025
    ref = assemble_and_solve_reference(spec, v, dm, rm, cfac)
    one, _, rounds1 = emulate_tree_solve(spec.ncell, spec.parent, spec.a, spec.b, spec.cm, cfac, v, dm, rm,
                                         unit_cells=1)
    assert np.max(np.abs(one - ref)) <= 1e-12 * max(1.0, np.max(np.abs(ref - v)))
    for u in sizes:
        got, _, rounds = emulate_tree_solve(spec.ncell, spec.parent, spec.a, spec.b, spec.cm, cfac, v, dm, rm,
                                            unit_cells=u)
        assert np.array_equal(got, one), u
        assert rounds >= rounds1


def test_solve_unit_request_beyond_lds_budget_is_refused():
    # three config-3 cells hold about 1860 chunks: 16 B each plus the stage exceed 40 KB
    spec = build_config(3, 3, 1.0)
    n = spec.nnode
    with pytest.raises(Exception):
        emulate_tree_solve(spec.ncell, spec.parent, spec.a, spec.b, spec.cm, 40.0, np.zeros(n), np.ones(n),
                           np.zeros(n), unit_cells=3)


@pytest.mark.parametrize("seed", range(8))
def test_emulated_chunk_solve_random_trees(seed):
    """Random shapes: chains longer than a chunk, bushy nodes, single-node cells."""
    rng = np.random.default_rng(100 + seed)
    ncell = int(rng.integers(1, 6))
    sizes = rng.integers(1, 120, ncell)
    parent = [-1] * ncell
    a, b = [0.0] * ncell, [0.0] * ncell
    for c in range(ncell):
        local = [c]
        for j in range(1, int(sizes[c])):
            mode = rng.random()
            if mode < 0.5:
                p = local[-1]                       # extend a chain
            elif mode < 0.8:
                p = local[int(rng.integers(0, len(local)))]
            else:
                p = local[0]                        # many children on the root
            parent.append(p)
            local.append(len(parent) - 1)
            a.append(-rng.uniform(0.05, 3))
            b.append(-rng.uniform(0.05, 3))
    # renumber so that roots come first and parent < child
    n = len(parent)
    parent = np.array(parent, np.int32)
    order = list(range(ncell)) + [i for i in range(n) if i >= ncell]
    assert all(parent[i] < i for i in range(ncell, n))
    from heliox_amd.spec import ModelSpec
    spec = ModelSpec(ncell=ncell, parent=parent, a=np.array(a), b=np.array(b), area=np.ones(n), cm=np.ones(n))
    v = rng.uniform(-80, 20, n)
    dm = rng.uniform(0.5, 2.0, n) * 1e-3
    rm = rng.normal(0, 1e-3, n)
    cfac = 40.0
    ref = assemble_and_solve_reference(spec, v, dm, rm, cfac)
    got, _, _ = emulate_tree_solve(ncell, parent, spec.a, spec.b, spec.cm, cfac, v, dm, rm)
    assert np.max(np.abs(got - ref)) <= 1e-12 * max(1.0, np.max(np.abs(ref - v)))


# ---------------------------------------------------------------------------
# workload generator
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("config,ncell,nper", [(1, 5, 101), (2, 3, 500), (3, 2, 5000), (4, 4, 200), (5, 3, 500)])
def test_generator_shapes(config, ncell, nper):
    spec = build_config(config, ncell, 50.0)
    spec.validate()
    assert spec.ncell == ncell and spec.nnode == ncell * nper
    cell = spec.cell_of_node()
    assert np.all(np.bincount(cell) == nper)
    assert np.all(spec.area > 0) and np.all(spec.a[spec.ncell:] < 0) and np.all(spec.b[spec.ncell:] < 0)


def test_generator_cells_do_not_depend_on_model_size():
    small = build_config(3, 2, 20.0)
    big = build_config(3, 5, 20.0)
    cs = small.cell_of_node()
    cb = big.cell_of_node()
    for c in range(2):
        assert np.array_equal(small.a[cs == c], big.a[cb == c])
        assert np.array_equal(small.b[cs == c], big.b[cb == c])
    assert np.array_equal(small.vecstim_times, big.vecstim_times[: small.vecstim_times.size])


def test_generator_is_deterministic():
    x = build_config(2, 3, 100.0)
    y = build_config(2, 3, 100.0)
    assert np.array_equal(x.parent, y.parent) and np.array_equal(x.a, y.a)
    assert np.array_equal(x.vecstim_times, y.vecstim_times)
    assert np.array_equal(x.netcons["ExpSyn"].weight, y.netcons["ExpSyn"].weight)


# ---------------------------------------------------------------------------
# error behaviour (reference convention: -1 and a message, never an abort)
# ---------------------------------------------------------------------------
def test_error_paths_without_gpu():
    s = Sim()
    assert s.set_device("cpu") == -1 and "gpu" in s.last_error()
    L = lib()
    h = s.handle
    # mechanisms need nodes first; unknown mechanism names are rejected
    nodes = np.array([0], np.int32)
    assert L.hx_model_insert(h, b"hh", 1, nodes.ctypes.data_as(__import__("ctypes").POINTER(__import__("ctypes").c_int))) == -1
    parent = np.array([-1, 0], np.int32)
    a = np.array([0.0, -1.0])
    C = __import__("ctypes")
    dp = lambda x: x.ctypes.data_as(C.POINTER(C.c_double))
    ip = lambda x: x.ctypes.data_as(C.POINTER(C.c_int))
    bad_parent = np.array([-1, 1], np.int32)
    assert L.hx_model_set_nodes(h, 1, 2, ip(bad_parent), dp(a), dp(a), dp(a)) == -1
    assert L.hx_model_set_nodes(h, 1, 2, ip(parent), dp(a), dp(a), dp(np.array([1.0, 1.0]))) == 0
    assert L.hx_model_insert(h, b"not_a_mech", 1, ip(nodes)) == -1
    assert "unknown mechanism" in s.last_error()
    assert L.hx_model_insert(h, b"pas", 2, ip(np.array([0, 0], np.int32))) == -1   # density mech twice on a node
    assert L.hx_model_insert(h, b"pas", 2, ip(np.array([0, 1], np.int32))) == 0
    assert L.hx_model_set_param(h, b"pas", b"nope", 2, dp(a)) == -1
    assert L.hx_model_add_netcon(h, 0, 0, b"ExpSyn", 0, 1.0, 1.0) == -1
    assert L.hx_finitialize(h, -65.0) == -1 and "not loaded" in s.last_error()
    assert s.get_variable_handle("global", "v", 0) == -1


def test_plugin_mechanisms_are_listed_and_accepted():
    """Mechanisms added through the plugin seam are registered by name at library load,
    reported after the built-in ones, and accepted by model specs."""
    import heliox_amd
    from heliox_amd.spec import MECH_PARAMS
    ms = heliox_amd.mechanisms()
    kinds = [m.kind for m in ms]
    assert kinds == sorted(kinds)            # "builtin" rows, then "plugin" rows
    im = [m for m in ms if m.name == "Im"]
    assert len(im) == 1 and im[0].kind == "plugin"
    assert im[0].columns[:2] == ("gImbar", "m") and im[0].nparam == 1 and im[0].nstate == 1
    assert MECH_PARAMS["Im"] == ("gImbar",)
    for m in ms:
        if m.kind == "builtin" and m.name in MECH_PARAMS:
            assert set(MECH_PARAMS[m.name]) <= set(m.columns), m.name
    with pytest.raises(ValueError):
        heliox_amd.register_mechanism("Im", ("other",))
