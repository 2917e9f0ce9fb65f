"""Backend-neutral description of a compartmental model.

The reference builds its in-memory model from a CoreNEURON export
(src/io/read_coredat.cpp:36-87 -> src/io/coredat_to_innerdat.cpp:591-603):
node arrays (parent, a, b, area), per-mechanism instance lists with their
node indices and parameter columns, presyn detectors, netcons and VecStim
payloads.  ``ModelSpec`` holds exactly that information as numpy arrays so the
same model can be handed to the HIP runtime (``heliox_amd.Sim``) and to any
other consumer.

Conventions (same as the reference's in-memory layout):
  * roots first: nodes ``[0, ncell)`` are the cell roots (parent -1), and every
    other node has ``parent[i] < i`` (permute_order.cpp:436-463);
  * units: um, mV, ms, S/cm2, uS for synaptic weights, nA for IClamp;
  * ion instances are addressed by node index (eion.cuh:270-300).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import numpy as np

# Mechanisms of the hot path and their per-instance parameter columns
# (names follow the reference's VarNames enums).
MECH_PARAMS: Dict[str, Tuple[str, ...]] = {
    "pas": ("g_pas", "e_pas"),
    "hh": ("gnabar", "gkbar", "gl", "el"),
    "IClamp": ("delay", "dur", "amp"),
    "Ca_HVA": ("gbar",),
    "hd_la": ("ghdbar", "vhalfl", "tau"),
    "CaDynamics_E2": ("gamma", "decay", "depth", "minCai"),
    "HalfGap": ("g",),
    "ExpSyn": ("tau", "e"),
    "Exp2Syn": ("tau1", "tau2", "e"),
    "VecStim": (),
    "NetStim": ("interval", "number", "start", "noise", "id1", "id2", "id3"),
    "na_ion": ("erev", "conci", "conco"),
    "k_ion": ("erev", "conci", "conco"),
    "ca_ion": ("erev", "conci", "conco"),
    # added to the library through its mechanism plugin seam (csrc/mechs/Im.hip)
    "Im": ("gImbar",),
}
ION_NAMES = ("na_ion", "k_ion", "ca_ion")
POINT_PROCESSES = ("IClamp", "HalfGap", "ExpSyn", "Exp2Syn", "VecStim", "NetStim")


def register_mechanism(name: str, params: Tuple[str, ...]) -> None:
    """Accept ``name`` in model specs, with its parameter columns.

    For a mechanism compiled into the library through its plugin seam (registered by
    name there, as the reference's MechanismFactory does, mechanism.h:125-197);
    loading the library registers every plugin it reports.  Re-registering a name
    with other columns is an error.
    """
    params = tuple(params)
    old = MECH_PARAMS.get(name)
    if old is not None and old != params:
        raise ValueError(f"mechanism {name} is already known with parameters {old}")
    MECH_PARAMS[name] = params


@dataclass
class MechSpec:
    nodes: np.ndarray                                   # int32 node index per instance
    params: Dict[str, np.ndarray] = field(default_factory=dict)   # float64 per instance
    globals: Dict[str, float] = field(default_factory=dict)
    iontype: Optional[np.ndarray] = None                # ions only (int32 style bits)

    @property
    def n(self) -> int:
        return int(self.nodes.shape[0])


@dataclass
class NetConSpec:
    """Netcons into one synapse mechanism: one source per synapse instance."""
    inst: np.ndarray      # int32 target instance
    src_kind: np.ndarray  # int8: 0 = real presyn index, 1 = VecStim instance, 2 = NetStim instance
    src: np.ndarray       # int32
    weight: np.ndarray    # float64 (uS)
    delay: np.ndarray     # float64 (ms)


@dataclass
class VecPlaySpec:
    mech: str
    var: str
    idx: int
    tvec: np.ndarray
    yvec: np.ndarray


@dataclass
class ModelSpec:
    ncell: int
    parent: np.ndarray            # int32, -1 for roots
    a: np.ndarray
    b: np.ndarray
    area: np.ndarray
    cm: np.ndarray
    celsius: float = 6.3
    dt: float = 0.025
    mechs: Dict[str, MechSpec] = field(default_factory=dict)
    presyn_gid: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int32))
    presyn_node: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int32))
    presyn_thr: np.ndarray = field(default_factory=lambda: np.zeros(0, np.float64))
    netcons: Dict[str, NetConSpec] = field(default_factory=dict)
    vecstim_offsets: np.ndarray = field(default_factory=lambda: np.zeros(1, np.int64))
    vecstim_times: np.ndarray = field(default_factory=lambda: np.zeros(0, np.float64))
    vecplay: List[VecPlaySpec] = field(default_factory=list)
    gap_src_node: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int32))
    gap_halfgap: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int32))
    monitors: List[Tuple[str, str, int]] = field(default_factory=list)
    name: str = "model"

    @property
    def nnode(self) -> int:
        return int(self.parent.shape[0])

    def cell_of_node(self) -> np.ndarray:
        """Cell id of every node (roots are cells 0..ncell-1)."""
        up = self.parent.astype(np.int64).copy()
        up[: self.ncell] = np.arange(self.ncell)
        while True:                      # pointer jumping: O(log depth) passes
            nxt = up[up]
            if np.array_equal(nxt, up):
                return up
            up = nxt

    def validate(self) -> None:
        n = self.nnode
        if self.ncell <= 0 or n < self.ncell:
            raise ValueError("need at least one cell and ncell <= nnode")
        if np.any(self.parent[: self.ncell] != -1):
            raise ValueError("nodes [0, ncell) must be roots (parent -1)")
        idx = np.arange(self.ncell, n)
        pp = self.parent[self.ncell:]
        if np.any(pp < 0) or np.any(pp >= idx):
            raise ValueError("non-root nodes need 0 <= parent[i] < i")
        for arr, nm in ((self.a, "a"), (self.b, "b"), (self.area, "area"), (self.cm, "cm")):
            if arr.shape != (n,):
                raise ValueError(f"{nm} must have shape ({n},)")
        for nm, m in self.mechs.items():
            if nm not in MECH_PARAMS:
                raise ValueError(f"unknown mechanism {nm}")
            if m.n and (m.nodes.min() < 0 or m.nodes.max() >= n):
                raise ValueError(f"{nm}: node index out of range")
            for k, v in m.params.items():
                if v.shape != (m.n,):
                    raise ValueError(f"{nm}.{k}: wrong length")

    def vecstim_train(self, k: int) -> np.ndarray:
        o = self.vecstim_offsets
        return self.vecstim_times[o[k]: o[k + 1]]

    @property
    def n_vecstim(self) -> int:
        return int(self.vecstim_offsets.shape[0] - 1)
