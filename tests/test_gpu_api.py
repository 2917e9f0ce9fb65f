"""The heliox.Sim surface beyond stepping (PyBindings.cpp:15-266): optimizers on
variable handles (SGD, momentum, Adam against their closed forms, tied groups,
external gradients, state export), gap junctions added at run time (the same bits
as the model's own HalfGap transfer), spike-file output, monitor and VecPlay
lookups, and pixel-driven input batches."""
import dataclasses
import math
import os

import numpy as np
import pytest

from heliox_amd import Sim, build_config
from heliox_amd.spec import MechSpec

pytestmark = pytest.mark.gpu


def small_sim(spec, mons=()):
    g = Sim()
    g.set_cell_groups(1)
    g.load_model_from_spec(dataclasses.replace(spec, monitors=list(mons)))
    g.finitialize(-65.0)
    return g


def test_optimizers_match_closed_forms(gpu_lib):
    spec = build_config(2, 2, 5.0)
    g = small_sim(spec)
    n_pas = spec.mechs["pas"].n
    idx = [0, 3, 7]
    w0 = np.array([g.get_variable_value("pas", "g_pas", i) for i in idx])
    wh = [g.get_variable_handle("pas", "g_pas", i) for i in idx]
    gh = [g.get_variable_handle("pas", "grad_g_pas", i) for i in idx]
    assert min(wh + gh) >= 0 and idx[-1] < n_pas

    def set_grads(vals):
        for h, x in zip(gh, vals):
            assert g.set_variable_by_handle(h, x) == 0

    lr, imp, inv = 1e-5, 2.0, 0.25
    # SGD: one tied group of three weights; the update uses the mean gradient
    sgd = g.create_optimizer("SGD")
    assert sgd >= 0 and g.optimizer_add_param_batch(sgd, wh, gh, imp) == 0
    gr = [1e-3, 3e-3, 2e-3]
    set_grads(gr)
    assert g.optimizer_step_with_inv_record_steps(sgd, lr, inv) == 0
    w1 = w0[0] - lr * np.mean(gr) * imp * inv
    assert all(g.get_variable_by_handle(h) == pytest.approx(w1, rel=1e-14) for h in wh)
    assert all(g.get_variable_by_handle(h) == 0.0 for h in gh)      # gradients zeroed after the step
    # momentum on the same handles, record_time / dt form
    mom = g.create_optimizer("momentum")
    assert g.configure_optimizer(mom, 0.8, 0.9, 0.999, 1e-8) == 0
    assert g.optimizer_add_param_batch(mom, wh, gh, 1.0) == 0
    vel, w = 0.0, w1
    for gv in ([4e-3] * 3, [-2e-3] * 3):
        set_grads(gv)
        assert g.optimizer_step(mom, lr, 10.0, 0.025) == 0
        vel = 0.8 * vel - lr * gv[0] * (0.025 / 10.0)
        w = w + vel
        assert g.get_variable_by_handle(wh[1]) == pytest.approx(w, rel=1e-13)
    # Adam: one group per weight
    adam = g.create_optimizer("adam")
    b1, b2, eps = 0.9, 0.999, 1e-8
    for a, b in zip(wh, gh):
        assert g.optimizer_add_param(adam, a, b, 1.0) >= 0
    ws = np.array([g.get_variable_by_handle(h) for h in wh])
    m = np.zeros(3)
    v = np.zeros(3)
    for step in (1, 2, 3):
        gv = np.array([1e-3, -2e-3, 5e-4]) * step
        set_grads(gv)
        assert g.optimizer_step_with_inv_record_steps(adam, 1e-4, 1.0) == 0
        m = b1 * m + (1 - b1) * gv
        v = b2 * v + (1 - b2) * gv * gv
        ws = ws - 1e-4 * (m / (1 - b1 ** step)) / (np.sqrt(v / (1 - b2 ** step)) + eps)
    got = np.array([g.get_variable_by_handle(h) for h in wh])
    np.testing.assert_allclose(got, ws, rtol=1e-13)
    st, mm, vv, sb1, sb2, seps = g.optimizer_get_adam_state(adam)
    assert st == 3 and np.allclose(mm, m, rtol=1e-14) and np.allclose(vv, v, rtol=1e-14)
    assert (sb1, sb2, seps) == (b1, b2, eps)
    assert g.optimizer_get_adam_state(sgd) == (0, [], [], 0.9, 0.999, 1e-8)   # not Adam
    assert g.optimizer_reset_state(adam) == 0
    assert g.optimizer_get_adam_state(adam)[0] == 0
    assert g.optimizer_set_adam_state(adam, 7, [1.0, 2.0, 3.0], [4.0, 5.0, 6.0], 0.8, 0.99, 1e-6) == 0
    assert g.optimizer_get_adam_state(adam) == (7, [1.0, 2.0, 3.0], [4.0, 5.0, 6.0], 0.8, 0.99, 1e-6)
    assert g.optimizer_set_adam_state(adam, 1, [1.0], [1.0]) == -1
    assert g.create_optimizer("lbfgs") == -1


def test_external_gradients_on_netcon_weights(gpu_lib):
    spec = build_config(2, 2, 5.0)
    g = small_sim(spec)
    wh = [g.get_variable_handle("ExpSyn", "weight", i) for i in range(4)]
    w0 = np.array([g.get_variable_by_handle(h) for h in wh])
    opt = g.create_optimizer("sgd")
    assert g.optimizer_add_external_grads(opt, wh, 3.0) == 0
    grads = np.array([1.0, -2.0, 0.5, 4.0], np.float32)
    assert g.optimizer_set_external_grads_f32(opt, grads) == 0
    assert g.optimizer_step_with_inv_record_steps(opt, 1e-4, 0.5) == 0
    got = np.array([g.get_variable_by_handle(h) for h in wh])
    np.testing.assert_allclose(got, w0 - 1e-4 * grads.astype(float) * 3.0 * 0.5, rtol=1e-14)
    assert g.optimizer_set_external_grads_f32(opt, grads[:2]) == -1
    assert g.optimizer_clear_external_grads(opt) == 0
    assert g.optimizer_step_with_inv_record_steps(opt, 1e-4, 0.5) == 0
    np.testing.assert_array_equal(np.array([g.get_variable_by_handle(h) for h in wh]), got)


def test_runtime_gap_equals_model_gap(gpu_lib):
    """A HalfGap fed by add_gap_source/add_gap_target gives the same bits as the same
    HalfGap fed by the model's gap list; clearing stops both kinds of transfer."""
    spec = build_config(1, 2, 30.0)
    spec.mechs["HalfGap"] = MechSpec(np.array([1], np.int32), {"g": np.array([5e-3])})
    mons = [("global", "v", 0), ("global", "v", 1), ("HalfGap", "vgap", 0)]
    static = dataclasses.replace(spec, gap_src_node=np.array([0], np.int32), gap_halfgap=np.array([0], np.int32))
    a = small_sim(static, mons)
    a.continue_run(30.0)
    b = small_sim(spec, mons)
    sid = b.add_gap_source(-1, "global", "v", 0)
    assert sid == 0 and b.get_next_available_sid() == 1
    assert b.add_gap_target(sid, "HalfGap", "vgap", 0) == 0
    assert b.add_gap_target(42, "HalfGap", "vgap", 0) == -1
    assert b.get_gap_junction(sid) == {"src_mech": "global", "src_var": "v", "src_idx": 0, "num_targets": 1,
                                       "is_dynamic": True}
    assert list(b.get_all_gap_junctions()) == [0]
    b.finitialize(-65.0)
    b.continue_run(30.0)
    assert np.array_equal(a.traces(), b.traces())
    # clearing: vgap keeps its last value
    for s in (a, b):
        assert s.clear_all_gap_junctions() == 0
        last = s.get_variable_value("HalfGap", "vgap", 0)
        s.continue_run(5.0)
        assert s.get_variable_value("HalfGap", "vgap", 0) == last
    assert b.get_all_gap_junctions() == {}


def test_spike_output_monitor_and_vecplay_lookups(gpu_lib, tmp_path):
    spec = build_config(1, 3, 60.0)
    g = small_sim(spec, [("global", "v", 1)])
    assert not g.is_spike_output_enabled()
    out = tmp_path / "spk_out"
    assert g.set_output_dir(str(out)) == 0 and g.set_spike_output_enabled(True) == 0
    g.run(60.0)
    text = open(out / "spk.dat").read()
    t, gid = g.spikes()
    assert t.size > 0 and len(text.splitlines()) == t.size
    assert g.get_monitor_handle("global", "v", 1) == 0
    assert g.get_monitor_handle("global", "v", 2) == -1
    assert g.get_monitor_handle_with_array("global", "v", 1, 0) == 0
    assert g.add_monitor_with_array("global", "v", 2, 1) == -1
    assert g.get_variable_handle_with_array("global", "v", 1, 0) >= 0
    assert g.add_vecplay("IClamp", "amp", 1, [0.0, 10.0], [0.0, 1.0]) == 0
    assert g.get_all_vecplay_keys() == [["IClamp", "amp", "1"]]


def test_input_batches_encode_pixels(gpu_lib):
    """NetStim batch: interval = scale / max(p + eps, eps), start = base + interval;
    VecStim batch: spikes at base + k * scale / max(p + eps, eps)."""
    spec = build_config(2, 2, 5.0)
    n = 3
    spec.mechs["NetStim"] = MechSpec(np.zeros(n, np.int32), {"interval": np.full(n, 10.0)})
    g = small_sim(spec)
    trip = [tuple(g.get_variable_handle("NetStim", v, i) for v in ("interval", "start", "number")) for i in range(n)]
    b = g.register_netstim_batch(trip, interval_scale=20.0, start_base=5.0, epsilon=1e-3, number=4)
    assert b == 0
    px = [0.5, 0.0, 1.0]
    assert g.set_input_batch_pixels(b, px) == 0
    for i, p in enumerate(px):
        iv = 20.0 / max(p + 1e-3, 1e-3)
        assert g.get_variable_value("NetStim", "interval", i) == pytest.approx(iv)
        assert g.get_variable_value("NetStim", "start", i) == pytest.approx(5.0 + iv)
        assert g.get_variable_value("NetStim", "number", i) == 4
    assert g.set_input_batch_pixels(b, px[:2]) == -1
    vb = g.register_vecstim_batch([0, 1], spike_scale=4.0, start_base=1.0, epsilon=1e-3, spike_count=3)
    assert vb == 1 and g.set_input_batch_pixels(vb, [1.0, 0.25]) == 0
    assert g.register_vecstim_batch([]) == -1
