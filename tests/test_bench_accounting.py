"""The benchmark's byte accounting and the cell ranges its all-core CPU sample uses."""
import numpy as np

import bench
from heliox_amd import build_config


def test_step_bytes_config3_per_compartment():
    # 84 node bytes + pas 16 + hh 96 + hd_la 40 + Ca_HVA 40 + CaDynamics_E2 56, and
    # 200 Exp2Syn per 5000-compartment cell at 108 B each (4.32 B per compartment)
    spec = build_config(3, 2, 1.0)
    out = bench.step_bytes(spec, 1.0)
    assert out["alg_bytes_per_compartment"] == 336.32
    assert out["alg_bytes_per_step"] == 3363200
    assert abs(out["achieved"] - 3363200 / 1e-3 / 1e9) < 0.1


def test_step_bytes_less_uniform_columns():
    """Columns served as one value are taken out of the step's algorithmic bytes: config 3's
    13 uniform columns (pas 2, hh gl/el, hd_la 2, Ca_HVA 1, CaDynamics_E2 4, na/k erev) are
    104 B per compartment, which leaves 232.32."""
    spec = build_config(3, 2, 1.0)
    out = bench.step_bytes(spec, 1.0, not_read=13 * 8 * spec.nnode)
    assert out["alg_bytes_per_compartment"] == 232.32
    assert out["alg_bytes_per_step"] == 3363200 - 1040000


def test_first_cell_selects_disjoint_cells():
    whole = build_config(3, 3, 1.0)
    tail = build_config(3, 1, 1.0, first_cell=2)
    # the third cell of the whole model is the only cell of the tail model
    n = tail.nnode
    assert np.array_equal(whole.a[-(n - 1):], tail.a[1:])
    # roots come first: the tail cell's soma is node 2 of the whole model
    gw, gt = whole.mechs["hd_la"].params["ghdbar"], tail.mechs["hd_la"].params["ghdbar"]
    assert gw[2] == gt[0] and np.array_equal(gw[-(n - 1):], gt[1:])
    k = tail.n_vecstim
    for j in range(k):
        assert np.array_equal(whole.vecstim_train(whole.n_vecstim - k + j), tail.vecstim_train(j))


def test_host_threads_respects_omp(monkeypatch):
    monkeypatch.setenv("OMP_NUM_THREADS", "1")
    assert bench.host_threads() == 1
    monkeypatch.delenv("OMP_NUM_THREADS")
    assert bench.host_threads() >= 1
