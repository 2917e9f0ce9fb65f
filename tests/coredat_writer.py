"""Writes a ModelSpec as a CoreNEURON export (test fixture generator).

The layout is the one the reference's reader takes apart (read_coredat.cpp:138-1141,
global_vars.cpp:12-88): bbcore_mech.dat and files.dat as text, <id>_1.dat and
<id>_2.dat as text count lines and arrays framed by "chkpnt N" lines (N running on
from the first file into the second), <id>_gap.dat with its own count from 0, and
globals.dat as "name value" lines up to "0 0".  Each mechanism instance is a row of
`dsize` doubles with the loaded variables at the offsets of the reference's
read_data_from_coredat; the other slots hold seeded filler so that a reader that
takes a wrong offset reads a wrong value.
"""
from __future__ import annotations

import os
from typing import Dict, List, Optional, Tuple

import numpy as np

from heliox_amd.spec import ModelSpec

# name -> (pnttype, is_art, is_ion, dsize, pdsize, charge, {var: offset})
# types are numbered from 2 in this order (NEURON's built-ins first, as it numbers them)
MECHS: List[Tuple[str, int, int, int, int, int, float, Dict[str, int]]] = [
    ("morphology", 0, 0, 0, 1, 0, 0.0, {}),
    ("capacitance", 0, 0, 0, 2, 0, 0.0, {"cm": 0}),
    ("pas", 0, 0, 0, 3, 0, 0.0, {"g_pas": 0, "e_pas": 1}),
    ("IClamp", 1, 0, 0, 4, 2, 0.0, {"delay": 0, "dur": 1, "amp": 2}),
    ("ExpSyn", 2, 0, 0, 8, 2, 0.0, {"tau": 0, "e": 1}),
    ("Exp2Syn", 3, 0, 0, 11, 2, 0.0, {"tau1": 0, "tau2": 1, "e": 2}),
    ("na_ion", 0, 0, 1, 5, 1, 1.0, {"erev": 0, "conci": 1, "conco": 2}),
    ("k_ion", 0, 0, 1, 5, 1, 1.0, {"erev": 0, "conci": 1, "conco": 2}),
    ("hh", 0, 0, 0, 23, 6, 0.0, {"gnabar": 0, "gkbar": 1, "gl": 2, "el": 3}),
    ("NetStim", 4, 1, 0, 8, 3, 0.0, {"interval": 0, "number": 1, "start": 2, "noise": 3}),
    ("ca_ion", 0, 0, 1, 5, 1, 2.0, {"erev": 0, "conci": 1, "conco": 2}),
    ("Ca_HVA", 0, 0, 0, 16, 3, 0.0, {"gbar": 0}),
    ("CaDynamics_E2", 0, 0, 0, 8, 2, 0.0, {"gamma": 0, "decay": 1, "depth": 2, "minCai": 3}),
    ("hd_la", 0, 0, 0, 11, 0, 0.0, {"ghdbar": 0, "vhalfl": 1, "tau": 2}),
    ("HalfGap", 5, 0, 0, 5, 2, 0.0, {"g": 0, "vgap": 1}),
    ("VecStim", 6, 1, 0, 4, 3, 0.0, {}),
]
TYPE = {m[0]: i + 2 for i, m in enumerate(MECHS)}
INFO = {m[0]: m for m in MECHS}
RECEIVE = {"ExpSyn": 1, "Exp2Syn": 1}
HD_LA_GLOBALS = ("ehd", "kl", "vhalft", "a0t", "zetat", "gmt", "q10", "qtl")


class _Out:
    """Text lines and chkpnt-framed arrays of one data file."""

    def __init__(self, path: str, chk: List[int]):
        self.f = open(path, "wb")
        self.chk = chk

    def line(self, s: str) -> None:
        self.f.write((s + "\n").encode())

    def arr(self, a, dtype) -> None:
        self.f.write(f"chkpnt {self.chk[0]}\n".encode())
        self.chk[0] += 1
        self.f.write(np.ascontiguousarray(a, dtype).tobytes())

    def close(self) -> None:
        self.f.close()


def write_export(spec: ModelSpec, out: str, version: str = "1.8", group: int = 7, mod_num: int = 1000,
                 seed: int = 0, dead_netcons: Optional[List[Tuple[str, int]]] = None,
                 pointer2type: bool = False, shuffle_netcons: bool = True, dt: Optional[float] = None,
                 extra_globals: Optional[Dict[str, float]] = None) -> None:
    """Write `spec` to directory `out`.

    dead_netcons: (target, instance) pairs that get one more netcon, written last in
    presyn order, from a real-cell presyn without a detector (output_vindex -1).
    pointer2type: write a non-empty pointer2type array for the first mechanism with
    dparams (format 1.8), to exercise the chkpnt count past it.
    """
    rng = np.random.default_rng(seed)
    os.makedirs(out, exist_ok=True)
    v18 = tuple(int(x) for x in version.split(".")) >= (1, 8)
    nnode, ncell = spec.nnode, spec.ncell

    # ---- bbcore_mech.dat
    with open(os.path.join(out, "bbcore_mech.dat"), "w") as f:
        f.write(f"{version}\n{len(MECHS) + 2}\n")
        for name, pnt, art, ion, dsz, pdsz, charge, _ in MECHS:
            f.write(f"{name} {TYPE[name]} {pnt} {art} {ion} {dsz} {pdsz}")
            if v18:
                f.write(" " + " ".join([str(dsz)] + ["1"] * dsz))
            if ion:
                f.write(f" {charge}")
            f.write("\n")

    # ---- mechanisms of the model, in type order, capacitance on every node
    present = ["capacitance"] + [m for m in TYPE if m in spec.mechs]
    present.sort(key=lambda m: TYPE[m])
    rows: Dict[str, np.ndarray] = {}
    nodes: Dict[str, np.ndarray] = {}
    pdata: Dict[str, np.ndarray] = {}
    npnt = 0
    for m in present:
        _, pnt, art, ion, dsz, pdsz, _, offs = INFO[m]
        if m == "capacitance":
            nd = np.arange(nnode, dtype=np.int32)
            vals = {"cm": np.asarray(spec.cm, float)}
        else:
            ms = spec.mechs[m]
            nd = np.asarray(ms.nodes, np.int32)
            vals = {k: np.asarray(v, float) for k, v in ms.params.items()}
        n = nd.size
        row = rng.uniform(-500.0, 500.0, (n, dsz))
        for k, off in offs.items():
            if k in vals:
                row[:, off] = vals[k]
            elif k != "vgap":
                raise ValueError(f"{m}.{k}: the writer needs every loaded variable set")
        rows[m], nodes[m] = row, nd
        if pdsz:
            pd = rng.integers(0, 1 << 20, (n, pdsz)).astype(np.int32)
            if ion:
                pd[:, 0] = np.asarray(spec.mechs[m].iontype if spec.mechs[m].iontype is not None
                                      else np.zeros(n), np.int32)
            if pnt:
                pd[:, 1] = npnt + np.arange(n)
            pdata[m] = pd
        if pnt:
            npnt += n

    # ---- presyns: real cells first, then one per artificial source used by a netcon
    def art_code(mech: str, k: int) -> int:
        return -(TYPE[mech] + mod_num * k)

    real_gid = [int(g) for g in spec.presyn_gid]
    real_node = [int(x) for x in spec.presyn_node]
    real_thr = [float(x) for x in spec.presyn_thr]
    dead_gid = None
    if dead_netcons:
        dead_gid = (max(real_gid) + 1) if real_gid else 0
        real_gid.append(dead_gid)
        real_node.append(-1)
        real_thr.append(rng.uniform(-30, 30))
    n_real = len(real_gid)
    nc_rows = []     # (srcgid, target, inst, weight, delay)
    art_used: List[Tuple[str, int]] = []
    for tgt, nc in spec.netcons.items():
        for i in range(nc.inst.shape[0]):
            kind, src = int(nc.src_kind[i]), int(nc.src[i])
            if kind == 0:
                sg = int(spec.presyn_gid[src])
            else:
                am = "VecStim" if kind == 1 else "NetStim"
                if (am, src) not in art_used:
                    art_used.append((am, src))
                sg = art_code(am, src)
            nc_rows.append((sg, tgt, int(nc.inst[i]), float(nc.weight[i]), float(nc.delay[i])))
    order = rng.permutation(len(nc_rows)) if shuffle_netcons else np.arange(len(nc_rows))
    nc_rows = [nc_rows[k] for k in order]
    for tgt, inst in dead_netcons or []:
        nc_rows.append((dead_gid, tgt, inst, 1.0, 1.0))
    out_gid = real_gid + [art_code(m, k) for m, k in art_used]
    out_vindex = real_node + [art_code(m, k) for m, k in art_used]

    # ---- files.dat
    gaps = len(spec.gap_src_node) > 0
    with open(os.path.join(out, "files.dat"), "w") as f:
        f.write(f"{version}\n")
        if gaps:
            f.write("-1\n")
        f.write(f"1\n{group}\n")

    chk = [0]
    # ---- <group>_1.dat
    o = _Out(os.path.join(out, f"{group}_1.dat"), chk)
    o.line(version)
    o.line(f"{len(out_gid)} npresyn")
    o.line(f"{len(nc_rows)} nnetcon")
    o.arr(out_gid, np.int32)
    o.arr([r[0] for r in nc_rows], np.int32)
    o.close()

    # ---- <group>_2.dat
    o = _Out(os.path.join(out, f"{group}_2.dat"), chk)
    o.line(version)
    if v18:
        o.line(f"{ncell} ncell")
    o.line(f"{len(out_gid)} ngid")
    o.line(f"{n_real} n_real_output")
    o.line(f"{nnode} nnode")
    o.line("0 ndiam")
    o.line(f"{len(present)} nmech")
    for m in present:
        o.line(str(TYPE[m]))
        o.line(str(nodes[m].size))
    nweight = sum(RECEIVE.get(r[1], 0) for r in nc_rows)
    o.line("0 nidata")
    o.line(f"{npnt} nvdata")
    o.line(f"{nweight} nweight")
    parent = np.asarray(spec.parent, np.int32).copy()
    parent[:ncell] = -1
    o.arr(parent, np.int32)
    o.arr(spec.a, np.float64)
    o.arr(spec.b, np.float64)
    o.arr(spec.area, np.float64)
    o.arr(np.full(nnode, -65.0), np.float64)
    p2t_done = False
    for m in present:
        _, pnt, art, ion, dsz, pdsz, _, _ = INFO[m]
        if not art:
            o.arr(nodes[m], np.int32)
        o.arr(rows[m].reshape(-1), np.float64)
        if pdsz:
            o.arr(pdata[m].reshape(-1), np.int32)
        if v18 and pdsz > 0:
            if pointer2type and not p2t_done:
                o.line("2")
                o.arr([-1, -1], np.int32)
                o.line("3")
                o.arr([1, 2, 3], np.uint32)
                p2t_done = True
            else:
                o.line("0")
                o.line("0")
    o.arr(out_vindex, np.int32)
    o.arr(real_thr, np.float64)
    o.arr([TYPE[r[1]] for r in nc_rows], np.int32)
    o.arr([r[2] for r in nc_rows], np.int32)
    o.arr([r[3] for r in nc_rows if RECEIVE.get(r[1], 0)], np.float64)
    o.arr([r[4] for r in nc_rows], np.float64)
    o.line(f"{npnt} npnt")
    if "VecStim" in present:
        nvs = nodes["VecStim"].size
        counts = np.array([spec.vecstim_train(k).size for k in range(nvs)], np.int32)
        times = np.concatenate([spec.vecstim_train(k) for k in range(nvs)]) if nvs else np.zeros(0)
        o.line(str(TYPE["VecStim"]))
        o.line(str(nvs))
        o.line(str(times.size))
        if nvs:
            o.arr(counts, np.int32)
        if times.size:
            o.arr(times, np.float64)
    o.line(f"{len(spec.vecplay)} n_vecplay")
    for vp in spec.vecplay:
        dsz = INFO[vp.mech][4]
        o.line("4")
        o.line(str(TYPE[vp.mech]))
        o.line(str(vp.idx * dsz + INFO[vp.mech][7][vp.var]))
        o.line(str(len(vp.tvec)))
        o.arr(vp.yvec, np.float64)
        o.arr(vp.tvec, np.float64)
    o.close()

    # ---- <group>_gap.dat
    if gaps:
        g = _Out(os.path.join(out, f"{group}_gap.dat"), [0])
        g.line(version)
        g.line("4 sidt_size")
        n = len(spec.gap_src_node)
        g.line(f"{n} ntar")
        g.line(f"{n} nsrc")
        sids = 100 + 3 * np.arange(n)
        g.arr(sids, np.int32)
        g.arr(np.full(n, -1), np.int32)
        g.arr(spec.gap_src_node, np.int32)
        perm = rng.permutation(n)
        g.arr(sids[perm], np.int32)
        g.arr(np.full(n, TYPE["HalfGap"]), np.int32)
        hg = np.asarray(spec.gap_halfgap, np.int64)[perm]
        g.arr(hg * INFO["HalfGap"][4] + 1, np.int32)
        g.close()

    # ---- globals.dat
    with open(os.path.join(out, "globals.dat"), "w") as f:
        f.write(f"{version}\n")
        f.write(f"celsius {float(spec.celsius)!r}\n")
        f.write(f"dt {float(spec.dt if dt is None else dt)!r}\n")
        f.write("secondorder_unused_array[2]\n1.5\n2.5\n")
        if "hd_la" in spec.mechs:
            for k in HD_LA_GLOBALS:
                f.write(f"{k}_hd_la {float(spec.mechs['hd_la'].globals[k])!r}\n")
        for k, v in (extra_globals or {}).items():
            f.write(f"{k} {float(v)!r}\n")
        f.write("0 0\n")
        f.write("secondorder 0\n")
        f.write("Random123_globalindex 0\n")
