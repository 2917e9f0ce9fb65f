"""Monitor output to sim_out.h5 (the reference's recorder file, simulate.cpp:185-269):
switching it on and off on the CPU, and on the GPU the file read back through the HDF5
C library against get_monitor_data, across run calls and a second finitialize."""
import numpy as np
import pytest

import h5read
from heliox_amd import Sim, build_config

needs_hdf5 = pytest.mark.skipif(h5read.lib() is None, reason="the HDF5 C library is not installed here")


@needs_hdf5
def test_enable_and_disable():
    s = Sim()
    assert not s.is_hdf5_enabled()
    assert s.set_hdf5_enabled(True) == 0
    assert s.is_hdf5_enabled()
    assert s.set_hdf5_enabled(False) == 0
    assert not s.is_hdf5_enabled()


@needs_hdf5
@pytest.mark.gpu
def test_monitor_file_matches_monitor_data(gpu_lib, tmp_path):
    spec = build_config(1, 2, 30.0)
    mons = [("global", "v", 0), ("hh", "m", 0), ("na_ion", "cur", 0), ("global", "v", 101)]
    g = Sim()
    g.load_model_from_spec(spec)
    hs = [g.add_monitor(*m) for m in mons]
    hs.append(g.add_monitor("global", "v", 0))        # the same variable twice: one dataset
    g.set_output_dir(str(tmp_path / "out"))
    assert g.set_hdf5_enabled(True) == 0
    print("case hdf5 monitors: finitialize, run 10 ms, continue 5 ms, finitialize, run 4 ms", flush=True)
    g.finitialize(-65.0)
    g.run(10.0)
    g.continue_run(5.0)
    path = str(tmp_path / "out" / "sim_out.h5")
    first = [np.array(g.get_monitor_data(h)) for h in hs]
    assert first[0].size == 601
    for (mech, var, idx), data in zip(mons, first):
        got, maxd, chunk = h5read.read_dataset(path, f"/group_0/{mech}/{var}/{idx}")
        assert np.array_equal(got, data), (mech, var, idx)
        assert maxd == 2 ** 64 - 1 and chunk == 100       # unlimited, chunks of 100
    # a second finitialize keeps appending to the same datasets
    g.finitialize(-65.0)
    g.run(4.0)
    assert g.flush_recorders() == 0
    second = [np.array(g.get_monitor_data(h)) for h in hs]
    for (mech, var, idx), a, b in zip(mons, first, second):
        got, _, _ = h5read.read_dataset(path, f"/group_0/{mech}/{var}/{idx}")
        assert np.array_equal(got, np.concatenate([a, b])), (mech, var, idx)
    assert g.set_hdf5_enabled(False) == 0     # closes the file
