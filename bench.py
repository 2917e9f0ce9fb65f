"""Benchmark of the per-timestep simulation core on one MI355X.

Workload: configuration 3 -- 2000 pyramidal-like cells x 5000 compartments
(1e7 compartments), fp64, hh + pas + Ih (hd_la) + Ca_HVA + CaDynamics_E2 on
every compartment, 200 Exp2Syn per cell driven by 5 Hz Poisson VecStim trains,
dt = 0.025 ms.  A step is one fadvance of the whole model; inputs and state are
resident in HBM before the timed region starts.

Prints one JSON line:
  value ........ compartment-steps/s of the whole job (1e7 x steps / wall time)
  roofline ..... the dominant kernel (the fused mechanism kernel): algorithmic
                 bytes per launch / its mean launch time from HIP events on the
                 library's stream, against MI355X's 8 TB/s HBM peak
  cpu_baseline . the CPU oracle (a restatement of the reference CPU step loop)
                 on a bounded sample of the same workload, one host core
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "compartment-steps/s (2000×5000-comp fp64) + achieved HBM GB/s"

# Algorithmic bytes per compartment for the fused mechanism kernel on this
# workload: every per-compartment input read once, every state read and
# written once, d and rhs written once (fp64):
#   v, cm 16 + (d, rhs) 16 + pas (g, e) 16 + hh (m,h,n r/w 48; gnabar, gkbar, gl,
#   el 32; ena, ek 16) 96 + Ca_HVA (m,h r/w 32; gbar 8) 40 + hd_la (l r/w 16;
#   ghdbar, vhalfl, tau 24) 40 + CaDynamics_E2 + ca_ion (cai r/w 16; gamma, decay,
#   depth, minCai 32; cao 8) 56  =  280 B
MECH_BYTES_PER_COMP = 280


# Algorithmic bytes per instance and step over the whole step (node kernel and tree
# solve), following the compulsory-traffic accounting of the workload definition:
# states read and written once, parameters and ion inputs read once, plus index,
# area and scattered rhs/d read-modify-write for point processes.  hh reads gl and
# el per instance here (96 rather than 80); CaDynamics_E2 includes its ca_ion.
STEP_BYTES_PER_INSTANCE = {"pas": 16, "hh": 96, "hd_la": 40, "Ca_HVA": 40, "CaDynamics_E2": 56,
                           "Exp2Syn": 108, "ExpSyn": 76, "IClamp": 52}
# per node: node kernel reads v, cm and writes rhs, d (32); the solve reads rhs, d,
# a, b, v and the parent index and writes v (52).  Solving for the new voltage (rhs + d v
# from the node kernel), the solve does not read v (44).
STEP_BYTES_PER_NODE = 84
SOLVE_V_BYTES = 8


def step_bytes(spec, ms_per_step: float, not_read: int = 0, solve_voltage: bool = False):
    """Algorithmic HBM bytes of one whole step and the rate they imply at the measured
    step time (against the HBM peak): an end-to-end figure beside the node kernel's.
    not_read: bytes of parameter columns served as one value (not read per instance);
    solve_voltage: the solve yields the new voltage without reading v."""
    per_node = STEP_BYTES_PER_NODE - (SOLVE_V_BYTES if solve_voltage else 0)
    total = per_node * spec.nnode - not_read
    for name, m in spec.mechs.items():
        total += STEP_BYTES_PER_INSTANCE.get(name, 0) * m.n
    gbs = total / (ms_per_step * 1e-3) / 1e9
    return {"alg_bytes_per_step": total, "alg_bytes_per_compartment": round(total / spec.nnode, 2),
            "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4)}


def _traffic_from_profiles():
    """HBM bytes of one node-kernel pass over the whole model, from the committed rocprof
    counter summary (copy-calibrated FETCH_SIZE + WRITE_SIZE)."""
    path = os.path.join(ROOT, "profiles", "k_dense_config3_counters.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_full_pass:"):
            try:
                return float(line.split(":", 1)[1].strip())
            except ValueError:
                return None
    return None


def cpu_baseline(ncell: int, nstep: int):
    import oracle
    from heliox_amd import build_config

    spec = build_config(3, ncell, nstep * 0.025 + 1.0)
    o = oracle.OracleSim(spec, monitors=[])
    o.finitialize(-65.0)
    t0 = time.perf_counter()
    o.nsteps(nstep)
    el = time.perf_counter() - t0
    rate = spec.nnode * nstep / el
    return {"value": rate, "unit": "compartment-steps/s", "cores": 1, "kind": "port",
            "sample": f"config 3, first {ncell} cells x 5000 compartments, {nstep} steps "
                      f"({spec.nnode * nstep:.3g} compartment-steps, {el:.1f} s on one core)"}


def cpu_baseline_all_cores(ncell: int, nstep: int, threads: int):
    """The same port on every host core: the cells of config 3 are independent (VecStim
    input only), so each thread steps its own range of ``ncell`` cells; ctypes releases
    the GIL for the duration of each oracle call."""
    import oracle
    from concurrent.futures import ThreadPoolExecutor
    from heliox_amd import build_config

    sims, nnode = [], 0
    for k in range(threads):
        spec = build_config(3, ncell, nstep * 0.025 + 1.0, first_cell=k * ncell)
        o = oracle.OracleSim(spec, monitors=[])
        o.finitialize(-65.0)
        sims.append(o)
        nnode += spec.nnode
    with ThreadPoolExecutor(threads) as ex:
        t0 = time.perf_counter()
        list(ex.map(lambda o: o.nsteps(nstep), sims))
        el = time.perf_counter() - t0
    return {"value": nnode * nstep / el, "unit": "compartment-steps/s", "cores": threads, "kind": "port",
            "sample": f"config 3, cells 0..{threads * ncell - 1} ({ncell} per thread) x 5000 compartments, "
                      f"{nstep} steps ({nnode * nstep:.3g} compartment-steps, {el:.1f} s on {threads} threads)"}


def host_threads() -> int:
    """Threads for the all-core baseline: the process's CPU affinity, capped by
    OMP_NUM_THREADS when that is set (the share of a shared host this job owns)."""
    n = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def perturb_config3(spec, seed: int = 1):
    """Target model for the config-3 training step: per cell, Ca_HVA gbar, hd_la ghdbar and
    hh gnabar (each tied over the cell) scaled by U(0.8, 1.2), and every Exp2Syn netcon
    weight by U(0.8, 1.2)."""
    import copy
    import numpy as np
    out = copy.deepcopy(spec)
    cell = spec.cell_of_node()
    rng = np.random.default_rng(0x3C3 + seed)
    f = rng.uniform(0.8, 1.2, (spec.ncell, 3))
    for k, (mech, var) in enumerate((("Ca_HVA", "gbar"), ("hd_la", "ghdbar"), ("hh", "gnabar"))):
        m = out.mechs[mech]
        m.params[var] = m.params[var] * f[cell[m.nodes], k]
    nc = out.netcons["Exp2Syn"]
    nc.weight = nc.weight * rng.uniform(0.8, 1.2, nc.weight.size)
    return out


def solver_options(sim, args):
    """Tree-solve options of the command line (the layouts change no result; the two solve
    forms agree to rounding)."""
    if args.unit_cells:
        sim.set_solve_unit_cells(args.unit_cells)
    if args.solve_waves:
        sim.set_solve_waves(args.solve_waves)
    if args.solve_streamed:
        sim.set_solve_resident(False)
    if args.solve_change:
        sim.set_solve_voltage(False)


def train_bench(args):
    """One differentiable training step = taped forward run, adjoint backward pass for the
    soma-v MSE against the perturbed model's trace, and one Adam step (lr 1e-3).
    Config 5 (default): 1000 cells x 500 compartments, 200 ms; gnabar, gkbar, g_pas tied
    per cell and the 10 ExpSyn weights of each cell.  --train-config 3: config-3 cells
    (5000 compartments, --train-cells of them, 25 ms by default); Ca_HVA gbar, hd_la ghdbar,
    hh gnabar, gkbar and pas g tied per cell and the 200 Exp2Syn weights of each cell."""
    import numpy as np
    import torch
    from heliox_amd import Sim, build_config
    from heliox_amd.synth import perturb_config5

    c3 = args.train_config == 3
    tstop = args.train_tstop if args.train_tstop > 0 else (25.0 if c3 else 200.0)
    base = build_config(3 if c3 else 5, args.train_cells, tstop)
    nstep = int(round(tstop / base.dt))
    soma = list(range(base.ncell))
    tg = Sim()
    tg.load_model_from_spec(perturb_config3(base) if c3 else perturb_config5(base, seed=1), add_monitors=False)
    for c in soma:
        tg.add_monitor("global", "v", c)
    tg.finitialize(-65.0)
    tg.run(tstop)
    target = np.ascontiguousarray(tg.traces()[:, 1:].T)
    del tg
    g = Sim()
    solver_options(g, args)
    g.load_model_from_spec(base, add_monitors=False)
    g.tape_begin(nstep)
    cell = base.cell_of_node()

    def forward_backward():
        t0 = time.perf_counter()
        g.finitialize(-65.0)
        g.run(tstop)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        loss = g.adjoint(soma, target)
        return loss, t1 - t0, time.perf_counter() - t1

    forward_backward()                           # warm-up (no parameter update)
    opt = g.adam_create(0.9, 0.999, 1e-8)
    tied = (("Ca_HVA", "gbar"), ("hd_la", "ghdbar"), ("hh", "gnabar"), ("hh", "gkbar"), ("pas", "g_pas")) if c3 \
        else (("hh", "gnabar"), ("hh", "gkbar"), ("pas", "g_pas"))
    for mech, var in tied:
        cn = cell[base.mechs[mech].nodes]
        for c in range(base.ncell):
            g.adam_add_group(opt, mech, var, np.nonzero(cn == c)[0])
    syn = "Exp2Syn" if c3 else "ExpSyn"
    for k in range(base.mechs[syn].nodes.size):
        g.adam_add_group(opt, syn, "weight", [k])
    loss, tf, tb = forward_backward()
    t2 = time.perf_counter()
    g.adam_step(opt, 1e-3, 1.0)
    ta = time.perf_counter() - t2
    total = tf + tb + ta
    ncomp = base.nnode // base.ncell
    name = f"config-{3 if c3 else 5} training steps/s ({base.ncell}x{ncomp}-comp fp64, {tstop:g} ms forward + adjoint + Adam)"
    print(json.dumps({"metric": name, "value": 1.0 / total, "unit": "training steps/s", "n_gpus": 1, "steps": 1,
                      "warmup": 1, "ms_per_step": total * 1e3, "higher_is_better": True, "scaling": "weak",
                      "vs_baseline": None, "dtype": "f64", "data": "synthetic",
                      "config": {"workload": f"config {3 if c3 else 5}: {base.ncell} cells x {ncomp} compartments, "
                                             f"{nstep} steps",
                                 "forward_s": tf, "adjoint_s": tb, "adam_s": ta, "loss": loss,
                                 "adjoint_us_per_step": tb * 1e6 / nstep}}))


MFMA_F32_PEAK_TFS = 157.3


def lrds_problem(N, bn, K_len, ksteps, n_out, n_in, seed=0):
    import numpy as np
    rng = np.random.default_rng(seed)
    T = ksteps + 1
    blocks = [(rng.normal(0, 1, (bn, bn, K_len)) * 0.5 / np.sqrt(bn)).astype(np.float32) for _ in range(N // bn)]
    it = rng.normal(0, 1, (N, T)).astype(np.float32)
    dv = rng.normal(0, 0.3, (N, T)).astype(np.float32)
    dp = rng.normal(0, 0.3, (N, T)).astype(np.float32)
    it[:, 0] = dv[:, 0] = dp[:, 0] = 0
    pre = np.where(rng.random(N) < 0.6, rng.integers(0, N, N), -1).astype(np.int32)
    po = np.sort(rng.choice(N, n_out, replace=False)).astype(np.int32)
    pin = np.sort(rng.choice(N, n_in, replace=False)).astype(np.int32)
    dL = rng.normal(0, 1, (ksteps, n_out)).astype(np.float32)
    return blocks, it, dv, dp, pre, po, pin, dL


def lrds_cpu_baseline(N, bn, K_len, ksteps, rows):
    """The oracle replay (fp64 numpy, one BLAS thread) on a row subset over every
    tick: rows of dv/dw are independent recurrences, so the full-problem rate is
    the subset rate x rows / N."""
    import numpy as np
    from threadpoolctl import threadpool_limits
    from oracle import lrds
    blocks, it, dv, dp, pre, po, pin, dL = lrds_problem(N, bn, K_len, ksteps, 64, 16)
    sel = np.linspace(0, N - 1, rows).astype(np.int64)
    with threadpool_limits(limits=1):
        t0 = time.perf_counter()
        lrds.replay(it, dv, dp, blocks, dL, po, pre, dt=0.025, percise=True, clip_strategy=0, rows=sel)
        el = time.perf_counter() - t0
    return {"value": ksteps * rows / N / el, "unit": "LR ticks/s", "cores": 1, "kind": "port",
            "sample": f"oracle replay of {rows} of {N} rows over all {ksteps} ticks ({el:.1f} s on one core; "
                      f"dx and clipping need every row and are left out of the sample)"}


def lrds_bench(args):
    """LRDS replay (the learn gradient surface): N = 2048 columns in 16 dense blocks
    of 128, K_len = 64, 256 LR ticks, precise correction, dw and dx for 16 inputs,
    Frobenius clip checked every tick (the reference's defaults).  Signals are
    uploaded once; a step is one LR tick of the replay."""
    import numpy as np
    import torch
    from heliox_amd import Sim, build_config

    N, bn, K_len, ks = args.lrds_n, 128, 64, args.lrds_ticks
    blocks, it, dv, dp, pre, po, pin, dL = lrds_problem(N, bn, K_len, ks, 64, 16)
    g = Sim()
    g.load_model_from_spec(build_config(1, 1, 1.0), add_monitors=False)
    assert g.set_dense_blocks_f32(blocks) == K_len
    dw = np.zeros(N, np.float32)
    dx = np.zeros((pin.size, ks), np.float32)

    def replay():
        rc = g.replay_compute_dw_dx_from_signals_into(it, dv, dp, dL, po, pin, pre, dw, dx, 0.025, True)
        if rc != 0:
            raise RuntimeError(g.last_error())

    replay()                                    # warm-up: workspace and signal upload paths
    # timed: the replay loop only (signals uploaded inside the call are part of it)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    replay()
    wall = time.perf_counter() - t0
    g.set_replay_timing(True)
    replay()
    corr_ms, launches = g.replay_kernel_time()
    g.set_replay_timing(False)
    # algorithmic flops of the correction GEMM: 2 N bn^2 tw per block per tick
    flops = sum(2.0 * N * bn * bn * min(t, K_len) * (N // bn) for t in range(1, ks + 1))
    achieved = flops / (corr_ms / 1e3) / 1e12
    roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": MFMA_F32_PEAK_TFS, "unit": "TFLOP/s",
                "frac": round(achieved / MFMA_F32_PEAK_TFS, 4), "traffic": None,
                "kernel": "k_rp_corr (fp32 MFMA 32x32x2 correction GEMM)",
                "alg_flops_per_launch": flops / ks, "us_per_launch": corr_ms * 1e3 / launches}
    cpu = None if args.no_cpu_baseline else lrds_cpu_baseline(N, bn, K_len, ks, args.lrds_cpu_rows)
    print(json.dumps({
        "metric": "LRDS replay LR ticks/s (N=2048, 16x128 blocks, K_len 64, precise, fp32)",
        "value": ks / wall, "unit": "LR ticks/s", "n_gpus": 1, "steps": ks, "warmup": 1,
        "ms_per_step": wall * 1e3 / ks, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"LRDS replay: N={N} columns, {N // bn} blocks of {bn}, K_len {K_len}, {ks} ticks, "
                               f"precise, 64 outputs, 16 inputs, clip every tick",
                   "replay_s": wall},
        "roofline": roofline, "cpu_baseline": cpu}))


VECPLAY_BYTES_PER_ITEM = 136   # item record read and written (2 x 48), tvec/yvec reads (32), target (8)


def network_bench(args):
    """Config 4 at full size: 10,000 cells x 200 compartments, 100 netcons per cell (1e6,
    delays 1-5 ms), 500 gap-junction pairs, VecPlay current into 500 cells.  A step is one
    step of the whole network; the line reports the step rate and each kernel class's
    time per launch (HIP events on the library stream), VecPlay among them."""
    import torch
    from heliox_amd import Sim, build_config
    dt = 0.025
    spec = build_config(4, args.network_cells, (args.warmup + args.steps + 10) * dt)
    sim = Sim()
    solver_options(sim, args)
    sim.load_model_from_spec(spec, add_monitors=False)
    sim.finitialize(-65.0)
    sim.continue_run((args.warmup + 0.5) * dt)
    sim.set_profiling(False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    sim.continue_run((args.steps + 0.5) * dt)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    spikes = sim.spikes()[0].size
    sim.set_profiling(True)
    sim.continue_run((args.steps + 0.5) * dt)
    kernels = {}
    for k in ("mech", "sparse", "point", "solve", "spike", "events", "other"):
        ms, n = sim.kernel_time(k)
        if n:
            kernels[k] = {"ms_total": ms, "launches": n, "us_per_launch": ms * 1e3 / n}
    nvp = len(spec.vecplay)
    print(json.dumps({
        "metric": "compartment-steps/s (config 4 network, 10000x200-comp fp64)",
        "value": spec.nnode * args.steps / wall, "unit": "compartment-steps/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": wall * 1e3 / args.steps, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f64", "data": "synthetic",
        "config": {"workload": f"config 4: {spec.ncell} cells x {spec.nnode // spec.ncell} compartments, "
                               f"{spec.netcons['ExpSyn'].inst.size} netcons, {spec.gap_src_node.size} gap halves, "
                               f"{nvp} VecPlay items", "spikes_in_timed_steps": spikes,
                   "solve_unit_cells": sim.info("solve_unit_cells")},
        "kernel_times": kernels,
        "vecplay": {"items": nvp, "alg_bytes_per_launch": nvp * VECPLAY_BYTES_PER_ITEM}}))


def calibrate_copy(gib: float = 1.0, reps: int = 5):
    """A plain device copy of known size, for scaling rocprof FETCH_SIZE / WRITE_SIZE."""
    import torch
    n = int(gib * (1 << 30) // 8)
    x = torch.ones(n, dtype=torch.float64, device="cuda")
    y = torch.empty_like(x)
    y.copy_(x)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        y.copy_(x)
    e1.record()
    torch.cuda.synchronize()
    s = e0.elapsed_time(e1) / 1e3 / reps
    out = {"copy_bytes_read": n * 8, "copy_bytes_written": n * 8, "reps": reps + 1,
           "copy_GBps_read_plus_written": round(2 * n * 8 / s / 1e9, 1)}
    # the node kernel's own access mix through a streaming kernel of the library: one
    # group launch's 5e6 compartments, 11 columns read and 9 written per compartment
    # (160 B), and the same with every parameter column read (26 + 9, 280 B)
    import ctypes
    from heliox_amd import lib
    for nr, nw in ((11, 9), (26, 9), (1, 1)):
        n_el = 5000192 if nr > 1 else n
        ms = ctypes.c_double()
        if lib().hx_measure_stream(nr, nw, n_el, 20, ctypes.byref(ms)) == 0:
            out[f"stream_{nr}r{nw}w_GBps"] = round((nr + nw) * 8 * n_el / (ms.value * 1e-3) / 1e9, 1)
            out[f"stream_{nr}r{nw}w_us"] = round(ms.value * 1e3, 1)
    print(json.dumps(out))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--ncell", type=int, default=2000, help="cells of config 3 (2000 = the benchmark)")
    ap.add_argument("--cpu-cells", type=int, default=12)
    ap.add_argument("--cpu-steps", type=int, default=1000)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-kernel-timing", action="store_true")
    ap.add_argument("--no-streamed-segment", action="store_true",
                    help="skip the segment timed with every parameter column read per instance")
    ap.add_argument("--all-kernel-timing", action="store_true",
                    help="time every kernel class (adds event records to the timed region)")
    ap.add_argument("--calibrate-copy", action="store_true")
    ap.add_argument("--train", action="store_true", help="time the config-5 training step instead")
    ap.add_argument("--train-cells", type=int, default=1000)
    ap.add_argument("--train-config", type=int, default=5, choices=(3, 5),
                    help="model of the training step: 5 (default) or 3 (its calcium and Exp2Syn mechanisms)")
    ap.add_argument("--train-tstop", type=float, default=0.0, help="forward run of the training step (ms)")
    ap.add_argument("--cell-groups", type=int, default=0,
                    help="cell groups issued on separate streams (0: the library's choice, 1: one stream)")
    ap.add_argument("--unit-cells", type=int, default=0,
                    help="cells per tree-solve wavefront (0: the library's choice)")
    ap.add_argument("--solve-waves", type=int, default=0,
                    help="tree-solve wavefronts per workgroup (0: the library's choice)")
    ap.add_argument("--solve-streamed", action="store_true",
                    help="stream every solve unit's rounds from HBM, also where the unit fits in LDS "
                         "(same results)")
    ap.add_argument("--solve-change", action="store_true",
                    help="solve for the change in voltage, as the reference does, also where the node "
                         "kernel makes every term of the matrix (the forms agree to rounding)")
    ap.add_argument("--no-group-turns", action="store_true",
                    help="order the cell groups' node passes only on a run's first step (same results)")
    ap.add_argument("--generic-node-kernel", action="store_true",
                    help="run every node-kernel launch through the generic kernel (no compile-time "
                         "steady-step instance; same results)")
    ap.add_argument("--model-root", action="store_true",
                    help="solve each cell toward its model root instead of its centre")
    ap.add_argument("--network", action="store_true", help="time the full-size config-4 network instead")
    ap.add_argument("--network-cells", type=int, default=10000)
    ap.add_argument("--lrds", action="store_true", help="time the LRDS replay of the learn surface instead")
    ap.add_argument("--lrds-n", type=int, default=2048)
    ap.add_argument("--lrds-ticks", type=int, default=256)
    ap.add_argument("--lrds-cpu-rows", type=int, default=1)
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (cells would be sharded "
              "across GPUs with spike exchange; see the design notes). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    if args.calibrate_copy:
        calibrate_copy()
        return
    if args.train:
        train_bench(args)
        return
    if args.lrds:
        lrds_bench(args)
        return
    if args.network:
        network_bench(args)
        return

    from heliox_amd import Sim, build_config

    t_build = time.perf_counter()
    tstop_needed = (args.warmup + args.steps + 10) * 0.025
    spec = build_config(3, args.ncell, tstop_needed)
    sim = Sim()
    sim.set_cell_groups(args.cell_groups)
    sim.set_solver_root(not args.model_root)
    solver_options(sim, args)
    if args.generic_node_kernel:
        sim.set_dense_steady(False)
    if args.no_group_turns:
        sim.set_group_turns(False)
    sim.load_model_from_spec(spec)
    t_build = time.perf_counter() - t_build
    groups = sim.info("cell_groups")
    nnode = spec.nnode
    dt = spec.dt
    # parameter columns with one value over the model are read as that value
    uniform_cols = sim.info("uniform_columns")
    uniform_bytes = sim.info("uniform_bytes")

    sim.finitialize(-65.0)
    if args.warmup:
        sim.continue_run((args.warmup + 0.5) * dt)
    # only the dominant kernel is timed with events on the stream (each timed
    # class adds two event records per step to the timed region)
    sim.set_profiling(not args.no_kernel_timing, classes=None if args.all_kernel_timing else ["mech"])
    # the warm-up call's last state update, if it waits, is applied by the timed call's first
    # node pass, as every step applies the previous one's
    carried_in = sim.info("state_pending")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    sim.continue_run((args.steps + 0.5) * dt)      # returns after the stream is synchronized
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # the timed call's last state update may wait for the next call (the first node pass of
    # the timed call applied the warm-up call's in the same way): 1 if it did
    deferred = sim.info("state_pending")
    outputs_deferred = sim.info("outputs_pending")

    value = nnode * args.steps / wall
    ms_per_step = wall * 1e3 / args.steps
    multi = sim.info("multi_stream")
    kernels = {}
    for k in ("mech", "sparse", "point", "solve", "spike", "events", "other"):
        ms, n = sim.kernel_time(k)
        if n:
            kernels[k] = {"ms_total": ms, "launches": n, "us_per_launch": ms * 1e3 / n}

    def node_kernel_roofline(mech, parts, not_read=uniform_bytes):
        # a step runs the node kernel once per part (cell group); a launch covers
        # nnode / parts compartments and reads no uniform parameter column per instance
        per_launch_s = mech["ms_total"] / mech["launches"] / 1e3
        alg = (MECH_BYTES_PER_COMP * nnode - not_read) / parts
        achieved = alg / per_launch_s / 1e9
        traffic = _traffic_from_profiles()
        if not_read != uniform_bytes:
            traffic = None      # the committed counter summary is of the default (uniform-column) reads
        return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": None if traffic is None else traffic / parts,
                "kernel": "k_dense (fused hh/pas/Ih/Ca_HVA/CaDynamics_E2 state+current)",
                "alg_bytes_per_launch": alg}

    roofline = None
    alone = None
    if "mech" in kernels:
        parts = groups if multi else 1
        roofline = node_kernel_roofline(kernels["mech"], parts)
        if multi:
            # the same kernel with the whole GPU to itself: a short single-stream
            # segment after the timed region (its launches cover the whole model)
            roofline["note"] = ("launch time measured while the other cell group's tree solve runs "
                                "beside it on its own stream")
            sim.set_group_streams(False)
            sim.set_profiling(True, classes=["mech"])
            sim.continue_run(100.5 * dt)
            ms, n = sim.kernel_time("mech")
            sim.set_group_streams(True)
            if n:
                alone = node_kernel_roofline({"ms_total": ms, "launches": n}, 1)
    # the same model with every parameter column read per instance (as the reference
    # reads them): a shorter timed segment after the main one
    streamed = None
    if uniform_cols and not args.no_streamed_segment:
        nseg = max(50, args.steps // 4)
        sim.set_uniform_columns(False)
        sim.set_profiling(not args.no_kernel_timing, classes=["mech"])
        sim.continue_run(20.5 * dt)
        torch.cuda.synchronize()
        sim.set_profiling(not args.no_kernel_timing, classes=["mech"])
        t1 = time.perf_counter()
        sim.continue_run((nseg + 0.5) * dt)
        torch.cuda.synchronize()
        w1 = time.perf_counter() - t1
        sim.set_uniform_columns(True)
        ms1, n1 = sim.kernel_time("mech")
        streamed = {"steps": nseg, "ms_per_step": w1 * 1e3 / nseg, "value": nnode * nseg / w1}
        if n1:
            streamed["roofline"] = node_kernel_roofline({"ms_total": ms1, "launches": n1},
                                                        groups if multi else 1, not_read=0)
    print(json.dumps({"kernel_times": kernels, "build_s": round(t_build, 2), "nnode": nnode,
                      "cell_groups": groups, "multi_stream": sim.info("multi_stream"),
                      "spikes": sim.spikes()[0].size, "t_end": sim.get_t()}), file=sys.stderr)

    cpu = cpu_all = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(args.cpu_cells, args.cpu_steps)
        cpu_all = cpu_baseline_all_cores(args.cpu_cells, args.cpu_steps // 2, host_threads())

    out = {
        "metric": METRIC,
        "value": value,
        "unit": "compartment-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64",
        "data": "synthetic",
        "config": {"workload": f"config 3: {args.ncell} pyramidal-like cells x 5000 compartments, fp64, "
                               f"hh+pas+Ih+Ca_HVA+CaDynamics_E2 everywhere, 200 Exp2Syn/cell with 5 Hz "
                               f"Poisson VecStim input, dt 0.025 ms",
                   "ncell": args.ncell, "compartments": nnode, "dt_ms": dt, "cell_groups": groups,
                   "solve_voltage": sim.info("solve_voltage"),
                   "wall_s_per_simulated_s": ms_per_step * 40.0},
        "state_update_carried_in": bool(carried_in),
        "state_update_deferred": bool(deferred),
        "last_step_outputs_on_demand": bool(outputs_deferred),
        "roofline": roofline,
        "roofline_single_stream": alone,
        "step_bytes": step_bytes(spec, ms_per_step, uniform_bytes, bool(sim.info("solve_voltage"))),
        "uniform_columns": {"columns": uniform_cols, "bytes_per_step_not_read": uniform_bytes,
                            "all_columns_read": streamed},
        "cpu_baseline": cpu,
        "cpu_baseline_all_cores": cpu_all,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
