"""MI355X-native HelioX simulation core: HIP kernels behind a C ABI
(include/heliox.h), a ``heliox.Sim``-compatible Python surface and seeded
synthetic workloads."""
from .spec import MechSpec, ModelSpec, NetConSpec, VecPlaySpec, register_mechanism
from .synth import build_config
from .sim import (HelioxError, MechanismInfo, Sim, emulate_tree_solve, lib, mechanisms, netstim_train,
                  philox4x32)

__all__ = ["MechSpec", "ModelSpec", "NetConSpec", "VecPlaySpec", "build_config", "Sim", "HelioxError",
           "MechanismInfo", "emulate_tree_solve", "lib", "mechanisms", "netstim_train", "philox4x32",
           "register_mechanism"]
