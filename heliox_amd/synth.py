"""Seeded synthetic workloads for the five benchmark configurations.

Every cell draws from its own stream, seeded with
``splitmix64(S ^ (config << 56) ^ cell_id)`` with master seed ``S = 20261201``,
so a cell's morphology and inputs do not depend on how many cells are built
(small parity models are prefixes of the benchmark models).

Geometry follows NEURON's cable discretisation, the source of the reference's
exported ``a``/``b``/``area`` arrays: each section of length ``L`` is split into
``nseg`` cylinders; the axial conductance between a compartment and its parent
is ``1/(r_half(child) + r_half(parent))`` with
``r_half = 1e-2 * Ra * (L/nseg/2) / (pi (d/2)^2)`` [MOhm], and
``a[i] = -1e2 g / area[parent]``, ``b[i] = -1e2 g / area[i]`` (S/cm2).

Configurations (see the benchmark description):
  1  ball-and-stick cells, hh soma + passive dendrite, IClamp at the soma
  2  random binary trees of 500 compartments, hh soma+axon, pas, 10 ExpSyn
     driven by 10 Hz Poisson VecStim trains
  3  pyramidal-like cells of 5000 compartments (trunk, obliques, tuft, 4 basal
     trees), hh + pas + Ih (hd_la) + Ca_HVA + CaDynamics_E2 on every
     compartment, 200 Exp2Syn driven by 5 Hz Poisson trains
  4  recurrent network of 200-compartment cells, 100 ExpSyn netcons per cell,
     500 gap-junction pairs, sinusoidal IClamp VecPlay on 5% of cells
  5  config-2 morphology with 1000 cells (training workload)
"""
from __future__ import annotations

import math
from typing import Dict, List, Optional, Tuple

import numpy as np

from .spec import MechSpec, ModelSpec, NetConSpec, VecPlaySpec

MASTER_SEED = 20261201
RA = 100.0          # ohm cm
CM = 1.0            # uF/cm2
CELSIUS = 6.3
DT = 0.025
ENA, EK = 50.0, -77.0   # NEURON's default reversal potentials (hh with na/k ions)
NC_DELAY_INPUT = 1.0    # ms, NEURON's default NetCon delay, used for VecStim inputs
DEFAULT_THRESHOLD = 10.0  # mV, NEURON's default NetCon threshold

_M64 = (1 << 64) - 1


def splitmix64(x: int) -> int:
    x = (x + 0x9E3779B97F4A7C15) & _M64
    z = x
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _M64
    return z ^ (z >> 31)


def cell_rng(config: int, cell: int) -> np.random.Generator:
    return np.random.default_rng(splitmix64(MASTER_SEED ^ ((config & 0xFF) << 56) ^ cell))


# ---------------------------------------------------------------------------
# Morphology builder: sections -> compartments
# ---------------------------------------------------------------------------
class _Cell:
    """Per-cell section list; section 0 is the one-compartment soma."""

    def __init__(self):
        self.sec_parent: List[int] = [-1]
        self.sec_L: List[float] = [20.0]
        self.sec_nseg: List[int] = [1]
        self.sec_d0: List[float] = [20.0]
        self.sec_d1: List[float] = [20.0]
        self.sec_kind: List[int] = [0]
        self.sec_order: List[int] = [0]
        self.nnode = 1

    def add(self, parent: int, L: float, nseg: int, d0: float, d1: float, kind: int) -> int:
        self.sec_parent.append(parent)
        self.sec_L.append(L)
        self.sec_nseg.append(nseg)
        self.sec_d0.append(d0)
        self.sec_d1.append(d1)
        self.sec_kind.append(kind)
        self.sec_order.append(self.sec_order[parent] + (1 if kind != 0 else 0))
        self.nnode += nseg
        return len(self.sec_parent) - 1

    def expand(self):
        """Return per-compartment (parent_local, Lseg, diam0, kind, path, sec_index)."""
        ns = np.asarray(self.sec_nseg, np.int64)
        nsec = ns.shape[0]
        start = np.zeros(nsec, np.int64)
        start[1:] = np.cumsum(ns)[:-1]
        total = int(ns.sum())
        sec_of = np.repeat(np.arange(nsec), ns)
        pos = np.arange(total) - start[sec_of]
        Lseg_sec = np.asarray(self.sec_L) / ns
        Lseg = Lseg_sec[sec_of]
        frac = (pos + 0.5) / ns[sec_of]
        d0 = np.asarray(self.sec_d0)[sec_of]
        d1 = np.asarray(self.sec_d1)[sec_of]
        diam = d0 + (d1 - d0) * frac
        parent = np.arange(total) - 1
        sp = np.asarray(self.sec_parent)
        last = start + ns - 1
        first_par = np.where(sp >= 0, last[np.maximum(sp, 0)], -1)
        parent[start] = first_par
        # path distance from the soma centre to each compartment centre
        path_end = np.zeros(nsec)
        path0 = np.zeros(nsec)
        for s in range(1, nsec):
            p = self.sec_parent[s]
            base = path_end[p] if p > 0 else 10.0   # soma centre to soma(1)
            path0[s] = base
            path_end[s] = base + self.sec_L[s]
        path = path0[sec_of] + Lseg * (pos + 0.5)
        path[0] = 0.0
        kind = np.asarray(self.sec_kind, np.int8)[sec_of]
        return parent, Lseg, diam, kind, path, sec_of


def _grow_tree(cell: _Cell, rng: np.random.Generator, attach: int, budget: int, max_order: int,
               kind: int, mode: str, Lrange=(20.0, 200.0), seg_len=10.0) -> None:
    """Grow a binary tree of exactly ``budget`` compartments from section ``attach``.

    mode 'bfs' expands terminals first-in-first-out (balanced); 'random' picks a
    random terminal each time (deeper, unbalanced trees).
    """
    frontier = [attach]
    first = True
    remaining = budget
    while remaining > 0:
        if not frontier:
            raise RuntimeError("tree depth limit reached before the compartment budget")
        if mode == "bfs" or first:
            par = frontier.pop(0)
        else:
            par = frontier.pop(int(rng.integers(len(frontier))))
        nchild = 1 if first else 2
        first = False
        for _ in range(nchild):
            if remaining <= 0:
                break
            L = float(rng.uniform(*Lrange))
            nseg = max(1, int(round(L / seg_len)))
            if nseg > remaining:
                L = L * remaining / nseg
                nseg = remaining
            s = cell.add(par, L, nseg, 1.0, 1.0, kind)
            remaining -= nseg
            if cell.sec_order[s] < max_order:
                frontier.append(s)


def _taper(diam_kind_mask, path, rng, dmax, dmin, noise=0.1, floor=0.3):
    sel = np.nonzero(diam_kind_mask)[0]
    out = np.zeros(sel.shape[0])
    if sel.size == 0:
        return sel, out
    pf = path[sel] / max(path[sel].max(), 1e-12)
    d = dmax + (dmin - dmax) * pf
    d = d * (1.0 + noise * rng.standard_normal(sel.shape[0]))
    return sel, np.maximum(d, floor)


def _geometry(parent_local, Lseg, diam):
    """NEURON cylinders: area, and a/b from the half-compartment resistances."""
    area = math.pi * diam * Lseg
    rhalf = 1e-2 * RA * (Lseg / 2.0) / (math.pi * (diam / 2.0) ** 2)
    a = np.zeros_like(Lseg)
    b = np.zeros_like(Lseg)
    nz = parent_local >= 0
    p = parent_local[nz]
    g = 1.0 / (rhalf[nz] + rhalf[p])
    a[nz] = -1e2 * g / area[p]
    b[nz] = -1e2 * g / area[nz]
    return area, a, b


# per-config cell builders: return dict with local arrays
def _cell_c1(rng):
    c = _Cell()
    L = float(rng.uniform(200, 600))
    d = float(rng.uniform(1, 3))
    c.add(0, L, 100, d, d, 2)
    parent, Lseg, diam, kind, path, _ = c.expand()
    amp = float(rng.uniform(0.1, 0.5))
    return dict(parent=parent, Lseg=Lseg, diam=diam, kind=kind, path=path, amp=amp)


def _cell_tree(rng, n_dend: int, axon_nodes: int, max_order: int, mode: str):
    c = _Cell()
    if axon_nodes:
        c.add(0, 10.0 * axon_nodes, axon_nodes, 1.0, 1.0, 1)
    _grow_tree(c, rng, 0, n_dend, max_order + 1, 2, mode)
    parent, Lseg, diam, kind, path, _ = c.expand()
    sel, d = _taper(kind == 2, path, rng, 4.0, 0.5)
    diam = diam.copy()
    diam[sel] = d
    return dict(parent=parent, Lseg=Lseg, diam=diam, kind=kind, path=path)


def _cell_c3(rng):
    c = _Cell()
    trunk = []
    par = 0
    for k in range(20):           # apical trunk: 20 sections x 10 compartments
        L = float(rng.uniform(40, 60))
        d0 = 3.0 - 1.5 * k / 20
        d1 = 3.0 - 1.5 * (k + 1) / 20
        par = c.add(par, L, 10, d0, d1, 3)
        trunk.append(par)
    for s in trunk[:-1]:          # one oblique tree per trunk junction
        _grow_tree(c, rng, s, 63, 60, 4, "random", Lrange=(20.0, 120.0))
    _grow_tree(c, rng, trunk[-1], 1602, 60, 5, "random", Lrange=(20.0, 150.0))   # tuft
    for _ in range(4):                                                          # basal trees
        _grow_tree(c, rng, 0, 500, 60, 2, "random", Lrange=(20.0, 150.0))
    parent, Lseg, diam, kind, path, _ = c.expand()
    assert parent.shape[0] == 5000
    diam = diam.copy()
    for kd in (2, 4, 5):
        sel, d = _taper(kind == kd, path, rng, 2.0, 0.4)
        diam[sel] = d
    return dict(parent=parent, Lseg=Lseg, diam=diam, kind=kind, path=path,
                max_order=max(c.sec_order))


def _assemble(cells: List[dict]):
    """Roots first, then each cell's non-root compartments in local order."""
    ncell = len(cells)
    sizes = np.array([c["parent"].shape[0] for c in cells], np.int64)
    nnode = int(sizes.sum())
    base = np.zeros(ncell, np.int64)
    base[1:] = np.cumsum(sizes - 1)[:-1]
    base += ncell
    parent = np.empty(nnode, np.int32)
    a = np.empty(nnode)
    b = np.empty(nnode)
    area = np.empty(nnode)
    gmap = []          # local->global node index per cell
    for ci, c in enumerate(cells):
        n = c["parent"].shape[0]
        g = np.empty(n, np.int64)
        g[0] = ci
        g[1:] = base[ci] + np.arange(n - 1)
        ar, aa, bb = _geometry(c["parent"], c["Lseg"], c["diam"])
        pl = c["parent"]
        parent[g] = np.where(pl >= 0, g[np.maximum(pl, 0)], -1)
        a[g] = aa
        b[g] = bb
        area[g] = ar
        gmap.append(g)
    return ncell, parent, a, b, area, gmap


def _poisson_trains(rng, n: int, rate_hz: float, tstop: float):
    lam = rate_hz * tstop / 1000.0
    K = int(lam + 6 * math.sqrt(lam) + 10)
    while True:
        isi = rng.exponential(1000.0 / rate_hz, size=(n, K))
        t = np.cumsum(isi, axis=1)
        if n == 0 or np.all(t[:, -1] > tstop):
            break
        K *= 2
    keep = t <= tstop
    counts = keep.sum(axis=1)
    return [t[i, : counts[i]] for i in range(n)]


def build_config(config: int, ncell: Optional[int] = None, tstop: Optional[float] = None,
                 first_cell: int = 0) -> ModelSpec:
    """Build configuration ``config`` (1..5) with ``ncell`` cells (default: full size).

    ``first_cell`` selects cells ``first_cell .. first_cell + ncell - 1`` of the full
    configuration (each cell has its own random stream); configuration 4 wires cells to
    each other and only accepts 0."""
    full = {1: 1000, 2: 10000, 3: 2000, 4: 10000, 5: 1000}
    tdef = {1: 100.0, 2: 500.0, 3: 1000.0, 4: 1000.0, 5: 200.0}
    if config not in full:
        raise ValueError("config must be 1..5")
    ncell = full[config] if ncell is None else int(ncell)
    tstop = tdef[config] if tstop is None else float(tstop)
    if first_cell and config == 4:
        raise ValueError("configuration 4 connects its cells: first_cell must be 0")
    rngs = [cell_rng(config, first_cell + c) for c in range(ncell)]
    if config == 1:
        cells = [_cell_c1(r) for r in rngs]
    elif config in (2, 5):
        cells = [_cell_tree(r, 450, 49, 20, "bfs") for r in rngs]
    elif config == 3:
        cells = [_cell_c3(r) for r in rngs]
    else:
        cells = [_cell_tree(r, 150, 49, 20, "bfs") for r in rngs]
    ncell_, parent, a, b, area, gmap = _assemble(cells)
    nnode = parent.shape[0]
    spec = ModelSpec(ncell=ncell_, parent=parent, a=a, b=b, area=area, cm=np.full(nnode, CM),
                     celsius=CELSIUS, dt=DT, name=f"config{config}")
    kind = np.empty(nnode, np.int8)
    path = np.empty(nnode)
    for c, g in zip(cells, gmap):
        kind[g] = c["kind"]
        path[g] = c["path"]
    spec._kind = kind   # compartment class: 0 soma, 1 axon, 2 basal/dendrite, 3 trunk, 4 oblique, 5 tuft
    spec._path = path
    spec._tstop = tstop
    soma = np.arange(ncell_, dtype=np.int32)

    def ions(nodes, erev_na=ENA, erev_k=EK):
        n = nodes.shape[0]
        spec.mechs["na_ion"] = MechSpec(nodes, {"erev": np.full(n, erev_na), "conci": np.full(n, 10.0),
                                                "conco": np.full(n, 140.0)}, iontype=np.zeros(n, np.int32))
        spec.mechs["k_ion"] = MechSpec(nodes.copy(), {"erev": np.full(n, erev_k), "conci": np.full(n, 140.0),
                                                      "conco": np.full(n, 4.0)}, iontype=np.zeros(n, np.int32))

    if config == 1:
        n = ncell_
        spec.mechs["hh"] = MechSpec(soma.copy(), {"gnabar": np.full(n, 0.12), "gkbar": np.full(n, 0.036),
                                                  "gl": np.full(n, 3e-4), "el": np.full(n, -54.3)})
        ions(soma.copy())
        dend = np.arange(ncell_, nnode, dtype=np.int32)
        spec.mechs["pas"] = MechSpec(dend, {"g_pas": np.full(dend.size, 1e-4), "e_pas": np.full(dend.size, -65.0)})
        amps = np.array([c["amp"] for c in cells])
        spec.mechs["IClamp"] = MechSpec(soma.copy(), {"delay": np.full(n, 5.0), "dur": np.full(n, 40.0),
                                                      "amp": amps})
        spec.presyn_gid = np.arange(n, dtype=np.int32)
        spec.presyn_node = soma.copy()
        spec.presyn_thr = np.full(n, DEFAULT_THRESHOLD)
        spec.monitors = [("global", "v", int(i)) for i in soma]
        return spec

    if config in (2, 4, 5):
        act = np.nonzero(kind <= 1)[0].astype(np.int32)      # soma + axon
        n = act.size
        spec.mechs["hh"] = MechSpec(act, {"gnabar": np.full(n, 0.12), "gkbar": np.full(n, 0.036),
                                          "gl": np.full(n, 3e-4), "el": np.full(n, -54.3)})
        ions(act.copy())
        allnodes = np.arange(nnode, dtype=np.int32)
        spec.mechs["pas"] = MechSpec(allnodes, {"g_pas": np.full(nnode, 1e-4), "e_pas": np.full(nnode, -65.0)})
        thr = -20.0 if config == 4 else DEFAULT_THRESHOLD
        spec.presyn_gid = np.arange(ncell_, dtype=np.int32)
        spec.presyn_node = soma.copy()
        spec.presyn_thr = np.full(ncell_, thr)
        cell_nodes = [g for g in gmap]
        if config in (2, 5):
            nsyn = 10
            syn_nodes, w, trains = [], [], []
            for ci, r in enumerate(rngs):
                g = cell_nodes[ci]
                dend_local = np.nonzero(cells[ci]["kind"] == 2)[0]
                syn_nodes.append(g[r.choice(dend_local, nsyn)])
                w.append(r.uniform(0.0, 2.0, nsyn) * 1e-3)
                trains.extend(_poisson_trains(r, nsyn, 10.0, tstop))
            syn_nodes = np.concatenate(syn_nodes).astype(np.int32)
            ns = syn_nodes.size
            spec.mechs["ExpSyn"] = MechSpec(syn_nodes, {"tau": np.full(ns, 2.0), "e": np.zeros(ns)})
            spec.mechs["VecStim"] = MechSpec(syn_nodes.copy(), {})
            _set_trains(spec, trains)
            spec.netcons["ExpSyn"] = NetConSpec(np.arange(ns, dtype=np.int32), np.ones(ns, np.int8),
                                                np.arange(ns, dtype=np.int32), np.concatenate(w),
                                                np.full(ns, NC_DELAY_INPUT))
            spec.monitors = [("global", "v", int(i)) for i in soma[: min(ncell_, 1000)]]
            return spec
        # config 4: recurrent network
        nin = 100
        syn_nodes, src, w, e, dl = [], [], [], [], []
        for ci, r in enumerate(rngs):
            g = cell_nodes[ci]
            dend_local = np.nonzero(cells[ci]["kind"] == 2)[0]
            syn_nodes.append(g[r.choice(dend_local, nin)])
            s = r.integers(0, max(ncell_ - 1, 1), nin)
            s = np.where(s >= ci, s + 1, s) if ncell_ > 1 else np.zeros(nin, np.int64)
            src.append(s)
            w.append(r.lognormal(-1.0, 0.5, nin) * 1e-3)
            e.append(np.where(r.random(nin) < 0.8, 0.0, -80.0))
            dl.append(r.uniform(1.0, 5.0, nin))
        syn_nodes = np.concatenate(syn_nodes).astype(np.int32)
        ns = syn_nodes.size
        spec.mechs["ExpSyn"] = MechSpec(syn_nodes, {"tau": np.full(ns, 2.0), "e": np.concatenate(e)})
        spec.netcons["ExpSyn"] = NetConSpec(np.arange(ns, dtype=np.int32), np.zeros(ns, np.int8),
                                            np.concatenate(src).astype(np.int32), np.concatenate(w),
                                            np.concatenate(dl))
        # gap junctions between random soma pairs (HalfGap g = 1 nS)
        gr = cell_rng(config, 0xFFFFFF)
        npair = min(500, ncell_ // 2)
        if npair > 0:
            perm = gr.permutation(ncell_)[: 2 * npair].astype(np.int32)
            hg_nodes = perm                              # HalfGap k sits on cell perm[k]
            partner = np.empty_like(perm)
            partner[0::2] = perm[1::2]
            partner[1::2] = perm[0::2]
            spec.mechs["HalfGap"] = MechSpec(hg_nodes.copy(), {"g": np.full(hg_nodes.size, 1e-3)})
            spec.gap_src_node = partner.astype(np.int32)
            spec.gap_halfgap = np.arange(hg_nodes.size, dtype=np.int32)
        # sinusoidal IClamp on 5% of cells, played with VecPlay at dt resolution
        nic = max(1, ncell_ // 20)
        ic_cells = gr.choice(ncell_, nic, replace=False).astype(np.int32)
        ic_cells.sort()
        spec.mechs["IClamp"] = MechSpec(ic_cells, {"delay": np.zeros(nic), "dur": np.full(nic, 1e9),
                                                   "amp": np.zeros(nic)})
        tv = np.arange(int(round(tstop / DT)) + 1) * DT
        yv = 0.2 * np.sin(2.0 * math.pi * 8.0 * tv / 1000.0)
        spec.vecplay = [VecPlaySpec("IClamp", "amp", k, tv, yv) for k in range(nic)]
        spec.monitors = [("global", "v", int(i)) for i in soma[: min(ncell_, 100)]]
        return spec

    # config 3
    n = nnode
    allnodes = np.arange(nnode, dtype=np.int32)
    is_soma = kind == 0
    spec.mechs["hh"] = MechSpec(allnodes.copy(), {"gnabar": np.where(is_soma, 0.12, 0.03),
                                                  "gkbar": np.where(is_soma, 0.036, 0.01),
                                                  "gl": np.zeros(n), "el": np.full(n, -54.3)})
    ions(allnodes.copy())
    spec.mechs["pas"] = MechSpec(allnodes.copy(), {"g_pas": np.full(n, 1e-4), "e_pas": np.full(n, -65.0)})
    cell = spec.cell_of_node()
    dmax = np.zeros(ncell_)
    np.maximum.at(dmax, cell, path)
    gh = 1e-4 + (1e-2 - 1e-4) * path / np.maximum(dmax[cell], 1e-12)
    spec.mechs["hd_la"] = MechSpec(allnodes.copy(), {"ghdbar": gh, "vhalfl": np.full(n, -81.0),
                                                     "tau": np.ones(n)})
    spec.mechs["Ca_HVA"] = MechSpec(allnodes.copy(), {"gbar": np.full(n, 5e-5)})
    spec.mechs["CaDynamics_E2"] = MechSpec(allnodes.copy(), {"gamma": np.full(n, 0.05), "decay": np.full(n, 80.0),
                                                             "depth": np.full(n, 0.1),
                                                             "minCai": np.full(n, 1e-4)})
    spec.mechs["ca_ion"] = MechSpec(allnodes.copy(), {"erev": np.zeros(n), "conci": np.full(n, 5e-5),
                                                      "conco": np.full(n, 2.0)},
                                    iontype=np.full(n, 0o4 | 0o40 | 0o100, np.int32))
    nsyn = 200
    syn_nodes, w, trains = [], [], []
    for ci, r in enumerate(rngs):
        g = gmap[ci]
        dend_local = np.nonzero(cells[ci]["kind"] >= 2)[0]
        syn_nodes.append(g[r.choice(dend_local, nsyn)])
        w.append(r.uniform(0.0, 1.0, nsyn) * 1e-3)
        trains.extend(_poisson_trains(r, nsyn, 5.0, tstop))
    syn_nodes = np.concatenate(syn_nodes).astype(np.int32)
    ns = syn_nodes.size
    spec.mechs["Exp2Syn"] = MechSpec(syn_nodes, {"tau1": np.full(ns, 0.5), "tau2": np.full(ns, 5.0),
                                                 "e": np.zeros(ns)})
    spec.mechs["VecStim"] = MechSpec(syn_nodes.copy(), {})
    _set_trains(spec, trains)
    spec.netcons["Exp2Syn"] = NetConSpec(np.arange(ns, dtype=np.int32), np.ones(ns, np.int8),
                                         np.arange(ns, dtype=np.int32), np.concatenate(w),
                                         np.full(ns, NC_DELAY_INPUT))
    spec.presyn_gid = np.arange(ncell_, dtype=np.int32)
    spec.presyn_node = soma.copy()
    spec.presyn_thr = np.full(ncell_, DEFAULT_THRESHOLD)
    spec.monitors = [("global", "v", int(i)) for i in soma[: min(ncell_, 100)]]
    spec._max_order = max(c["max_order"] for c in cells)
    return spec


def _set_trains(spec: ModelSpec, trains: List[np.ndarray]) -> None:
    counts = np.array([t.shape[0] for t in trains], np.int64)
    off = np.zeros(counts.shape[0] + 1, np.int64)
    off[1:] = np.cumsum(counts)
    spec.vecstim_offsets = off
    spec.vecstim_times = np.concatenate(trains) if trains else np.zeros(0)


def perturb_config5(spec: ModelSpec, seed: int = 1) -> ModelSpec:
    """The config-5 target model: per cell, gnabar, gkbar and g_pas (each tied
    over the cell's instances) and each of the cell's ExpSyn netcon weights are
    scaled by U(0.8, 1.2).  Returns a new spec; ``spec`` is unchanged."""
    import copy
    out = copy.deepcopy(spec)
    cell = spec.cell_of_node()
    rng = cell_rng(5, 0x7A1F00 + seed)
    f = rng.uniform(0.8, 1.2, (spec.ncell, 3))
    hh = out.mechs["hh"]
    hc = cell[hh.nodes]
    hh.params["gnabar"] = hh.params["gnabar"] * f[hc, 0]
    hh.params["gkbar"] = hh.params["gkbar"] * f[hc, 1]
    pas = out.mechs["pas"]
    pas.params["g_pas"] = pas.params["g_pas"] * f[cell[pas.nodes], 2]
    nc = out.netcons["ExpSyn"]
    nc.weight = nc.weight * rng.uniform(0.8, 1.2, nc.weight.size)
    return out
