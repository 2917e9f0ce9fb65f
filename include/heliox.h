/*
 * heliox.h -- C ABI of the MI355X (gfx950) HelioX simulation core.
 *
 * One opaque handle holds one model (the reference keeps one model group per
 * process: read_coredat.cpp:43, simulate.cpp:201).  All calls are made from a
 * single host thread per handle.  Every entry point returns 0 (or a
 * non-negative handle / count) on success and -1 on failure, like the
 * reference's SimWrapper (SimWrapper.cpp: `printf` + `return -1`); the failure
 * text is available from hx_last_error().  No call throws across the ABI.
 *
 * Units follow the reference: ms, mV, um, S/cm2, uS (synaptic weights), nA.
 * Variables are addressed as in the reference's VarDescriptor
 * (utils.h, Simulate::getVarPtr simulate.cpp:143-184):
 *   mech "global" (or "node"), var "v" | "d" | "rhs" | "a" | "b" | "area", idx = node
 *   mech "capacitance", var "cm", idx = node
 *   mech "na_ion" | "k_ion" | "ca_ion", var "erev" | "conci" | "conco" | "cur" | "dcurdv",
 *        idx = NODE index (eion.cuh:270-300)
 *   any other mechanism, var = column name, idx = instance index
 *   mechanism globals (e.g. "hd_la" "ehd") through hx_model_set_global.
 *
 * The replacement binds to the reference's Python surface (heliox.Sim,
 * src/python_api/PyBindings.cpp:15-266) through heliox_amd/sim.py.
 */
#ifndef HELIOX_AMD_H
#define HELIOX_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct hx_sim hx_sim;

/* SimWrapper::SimWrapper / ~SimWrapper (SimWrapper.cpp:18-36). */
int hx_create(hx_sim** out);
void hx_destroy(hx_sim* sim);
/* Text of the last failure on this handle ("" if none). */
const char* hx_last_error(hx_sim* sim);

/* SimWrapper::set_device (SimWrapper.cpp): only "gpu" is served by this library. */
int hx_set_device(hx_sim* sim, const char* dev);
/* SimWrapper::set_dt / get_dt. */
int hx_set_dt(hx_sim* sim, double dt);
double hx_get_dt(hx_sim* sim);
/* Model temperature (globals.dat "celsius", global_vars.cpp:12-88). */
int hx_set_celsius(hx_sim* sim, double celsius);

/* ---- model construction: replaces set_data_path + load_model, i.e. the
 *      CoreNEURON reader read_coredat.cpp:36-1141 and
 *      coredat_to_innerdat.cpp:42-603, with in-memory arrays.              */
/* Node arrays: nodes [0, ncell) are roots (parent -1); parent[i] < i otherwise. */
int hx_model_set_nodes(hx_sim* sim, int ncell, int nnode, const int* parent, const double* a,
                       const double* b, const double* area);
/* Mechanism instances by name (MechanismFactory::createMechanism, mechanism.h:125-164). */
int hx_model_insert(hx_sim* sim, const char* mech, int n, const int* node_indices);
/* One parameter column, n values in instance order (read_data_from_coredat). */
int hx_model_set_param(hx_sim* sim, const char* mech, const char* var, int n, const double* values);
/* Every mechanism hx_model_insert accepts (MechanismFactory's registry, mechanism.h:125-164):
 * the built-in set and the plugins registered in the library's build (plugin.h,
 * HX_REGISTER_MECHANISM, the reference's REGISTER_MECHANISM mechanism.h:167-171), one
 * "name<TAB>builtin|plugin<TAB>nparam<TAB>nstate<TAB>col,col,...\n" line each (columns:
 * parameters, then states, then assigned variables).  Writes up to cap bytes
 * (NUL-terminated) and returns the length needed including the NUL. */
int hx_mechanism_names(char* buf, int cap);
/* Mechanism global (GlobalVarNames, e.g. hd_la ehd/kl/vhalft/a0t/zetat/gmt/q10/qtl). */
int hx_model_set_global(hx_sim* sim, const char* mech, const char* var, double value);
/* Ion style bits per ion instance (eion.cuh:155-197: 04 conc init, 040 erev init, 0100 erev each step). */
int hx_model_set_iontype(hx_sim* sim, const char* ion, int n, const int* iontype);
/* Threshold detector of a real cell (PreSyn, presyn.cpp:133-177); returns the detector index. */
int hx_model_add_presyn(hx_sim* sim, int gid, int node, double threshold);
/* VecStim spike times of one instance (VecEvent::update_sequence, vecevent.cpp:292-309),
 * read from the first by the next finitialize (an empty array leaves no spikes). */
int hx_model_set_vecstim(hx_sim* sim, int inst, int n, const double* times);
/* SimWrapper::call_mech_func (SimWrapper.cpp:461-468) through FunctionRegistry
 * (func_table.cuh:97-130), whose one registered function is VecStim.play (vecevent.h:42-45,
 * VecEvent::play -> update_sequence, vecevent.cpp:280-309): mech "VecStim", func "play",
 * inst the VecStim instance, times[n] its new spike times.  n <= 0 changes nothing.  The
 * next finitialize reads the new times from the first.  In a run already initialised the
 * instance keeps what it has read, as the reference's element() does: after D deliveries it
 * has read D + 1 elements and queued the last, so it delivers that one and then
 * times[D + 1], times[D + 2], ...; an instance that has read past its end takes nothing
 * more until finitialize.  Any other name returns -1 ("function not registered"). */
int hx_call_mech_func(hx_sim* sim, const char* mech, const char* func, int inst, int n, const double* times);
/* NetCon into synapse `target` instance `inst` (ExpSyn / Exp2Syn).  src_kind 0: detector index,
 * 1: VecStim instance, 2: NetStim instance.  One source per synapse instance; a later netcon
 * replaces an earlier one (coredat_to_innerdat.cpp:356-364).
 * NetStim (netstim.cpp:211-330) is inserted like any mechanism, with parameters interval,
 * number, start, noise (defaults 10, 10, 50, 0) and id1, id2, id3, the ids of its own
 * Random123 Philox4x32 stream (id1 < 0, the default: the instance index).  A NetStim that no
 * netcon targets runs from a train made on the host at finitialize and as runs need them;
 * one that netcons target runs on the device, taking its incoming events as NET_RECEIVE
 * does (netstim.cpp:247-290: start, stop by a negative weight, weights truncated).  The
 * reference draws every instance from one shared stream and redraws all instances' intervals
 * on any event (netstim.cpp:118-161); here each instance draws only its own intervals from
 * its own stream, restarted at sequence 0 by every finitialize.  Parameter writes through
 * handles take effect at the next finitialize. */
int hx_model_add_netcon(hx_sim* sim, int src_kind, int src, const char* target, int inst, double weight,
                        double delay);
/* Gap-junction transfer after each update: HalfGap[halfgap_inst].vgap = v[src_node]
 * (Simulate::add_gap_source/add_gap_target, simulate.cpp:953-966). */
int hx_model_add_gap(hx_sim* sim, int src_node, int halfgap_inst);
/* SimWrapper::set_data_path (SimWrapper.cpp:18, SimRuntime.cpp:28-36): a directory holding
 * a CoreNEURON export (files.dat, bbcore_mech.dat, <id>_1.dat, <id>_2.dat, optional
 * <id>_gap.dat, globals.dat), read by the next hx_load_model.  Formats 1.8 and older,
 * one group, as read_coredat.cpp:36-1141 reads them. */
int hx_set_data_path(hx_sim* sim, const char* path);
/* SimWrapper::set_user_mod_num (SimWrapper.cpp:481): artificial presyns of the export are
 * numbered -(type + index * num); 1000 by default (100 for older HelioX test models). */
int hx_set_user_mod_num(hx_sim* sim, int num);
/* The read half of load_model (read_coredat + data_format_trans,
 * SimRuntimeCore.cpp:109-147): reads the export at the data path into the model builder,
 * as the hx_model_* calls would build it, without building the layout or touching the
 * GPU.  hx_load_model calls it when a data path is set.  On an error the builder is left
 * empty and the message names the file and the record. */
int hx_model_read_export(hx_sim* sim);
/* No reference counterpart: a text summary of the model builder (counts and FNV-1a
 * hashes of every array; netcons reduced to the last one per synapse instance), for
 * comparing two ways of building one model.  Writes up to cap bytes (NUL-terminated)
 * and returns the length needed including the NUL. */
int hx_model_digest(hx_sim* sim, char* out, int cap);
/* SimWrapper::load_model: reads the export at the data path when one is set, then builds
 * the solver layout and uploads the model to HBM. */
int hx_load_model(hx_sim* sim);

/* ---- step API (Simulate::finitialize/run/continue_run/fadvance, simulate.h:17-76) ---- */
int hx_finitialize(hx_sim* sim, double v_init);
int hx_run(hx_sim* sim, double tstop);
int hx_continue_run(hx_sim* sim, double runtime);
int hx_fadvance(hx_sim* sim);
double hx_get_t(hx_sim* sim);

/* ---- monitors (SimWrapper::add_monitor / get_monitor_data / flush_recorders) ---- */
int hx_add_monitor(hx_sim* sim, const char* mech, const char* var, int idx);
int hx_get_monitor_len(hx_sim* sim, int handle);
int hx_get_monitor_data(hx_sim* sim, int handle, double* out, int cap);
int hx_flush_recorders(hx_sim* sim);

/* ---- variable handles (SimRuntimeCore handle cache, SimRuntimeCore.h:197-205) ---- */
int hx_get_variable_handle(hx_sim* sim, const char* mech, const char* var, int idx);
int hx_get_variable_by_handle(hx_sim* sim, int handle, double* out);
int hx_set_variable_by_handle(hx_sim* sim, int handle, double value);
int hx_get_variables_by_handles(hx_sim* sim, int n, const int* handles, double* out);
int hx_get_variables_by_handles_f32_into(hx_sim* sim, int n, const int* handles, float* out);
int hx_set_variables_by_handles(hx_sim* sim, int n, const int* handles, const double* values);
int hx_get_variable_value(hx_sim* sim, const char* mech, const char* var, int idx, double* out);
int hx_set_variable_value(hx_sim* sim, double value, const char* mech, const char* var, int idx);
/* Whole column in instance (or node) order; returns the count written. */
int hx_get_array(hx_sim* sim, const char* mech, const char* var, double* out, int cap);

/* ---- VecPlay (SimWrapper::add_vecplay/update_vecplay/remove_vecplay/has_vecplay) ---- */
int hx_add_vecplay(hx_sim* sim, const char* mech, const char* var, int idx, int n, const double* tvec,
                   const double* yvec);
int hx_update_vecplay(hx_sim* sim, const char* mech, const char* var, int idx, int n, const double* tvec,
                      const double* yvec);
int hx_remove_vecplay(hx_sim* sim, const char* mech, const char* var, int idx);
int hx_has_vecplay(hx_sim* sim, const char* mech, const char* var, int idx);

/* ---- spikes (Simulate::output_spikes simulate.cpp:892-909, get_spk_by_gid) ----
 * The record (time, gid) of every threshold crossing since the model was loaded: like the
 * reference's rec_spikes and per-gid spk_output (simulate.cpp:880, presyn.cpp:155), it is
 * not cleared by finitialize. */
int hx_get_spike_count(hx_sim* sim);
int hx_get_spikes(hx_sim* sim, double* t, int* gid, int cap);
/* Spikes of every NetStim since finitialize, ordered by time then instance: the
   NetStim's own spike record (netstim.cpp:278-330, net_event at the delivering step's
   time).  Returns the total count (-1 on error) and fills at most cap of them. */
int hx_get_netstim_spikes(hx_sim* sim, double* t, int* inst, int cap);
int hx_get_spk_by_gid(hx_sim* sim, int gid, double* out, int cap);
/* Simulate::output_spikes (simulate.cpp:892-909): writes <folder>/spk.dat (the folder is
 * created if needed) with one "%.8g<TAB>%d" line per spike of the spikes recorded so far,
 * ordered by time and then gid; spikes of negative gids are left out. */
int hx_output_spikes(hx_sim* sim, const char* folder);

/* Monitor output to <output_dir>/sim_out.h5 (the reference's recorder file:
 * SimRuntimeCore's enable_hdf5 / main.cpp's watch points select BufferEnable::HDF5,
 * SimRuntimeCore.cpp:125-128; layout simulate.cpp:185-269; append on flush
 * variable_recorder.h:142-156).  Enabled, the file is created (truncated) at the next
 * hx_finitialize with the group /group_0, and every call that brings monitor samples
 * back (run, continue_run, fadvance, flush_recorders, finitialize) appends them to the
 * dataset /group_0/<mech>/<var>/<idx> of each monitor: double, one dimension,
 * unlimited, chunks of 100.  Later hx_finitialize calls keep appending to the same
 * file, as the reference's recorder does.  The HDF5 C library (1.10 or later) is
 * loaded at run time; without it enabling fails and nothing else changes.  Default: off. */
int hx_set_hdf5_enabled(hx_sim* sim, int enable);
int hx_is_hdf5_enabled(hx_sim* sim);

/* spk.dat after every hx_run / hx_continue_run (SimWrapper::run, continue_run,
 * SimWrapper.cpp:46-84; set_spike_output_enabled, set_output_dir).  Default: off, folder
 * "output" (simulate.cpp:30). */
int hx_set_spike_output_enabled(hx_sim* sim, int enable);
int hx_is_spike_output_enabled(hx_sim* sim);
int hx_set_output_dir(hx_sim* sim, const char* dir);

/* ---- gap junctions added at run time (Simulate::add_gap_source / add_gap_target /
 *      clear_all_gap_junctions / get_gap_junction / get_next_available_sid,
 *      simulate.cpp:998-1100).  After each update (and at finitialize) every target
 *      variable receives its source variable's value.  sid < 0 picks the next free id;
 *      the call returns the sid.  Clearing also stops the model's own HalfGap transfers,
 *      as the reference's does.  Runs with such transfers stay on one stream, and the
 *      adjoint refuses them. ---- */
int hx_add_gap_source(hx_sim* sim, int sid, const char* mech, const char* var, int idx);
int hx_add_gap_target(hx_sim* sim, int sid, const char* mech, const char* var, int idx);
int hx_clear_all_gap_junctions(hx_sim* sim);
int hx_get_next_available_sid(hx_sim* sim);
/* Ids of all gap junctions (up to cap written); returns their count. */
int hx_get_gap_junction_sids(hx_sim* sim, int* sids, int cap);
/* Source of gap junction sid and its number of targets; -1 if there is no such sid. */
int hx_get_gap_junction(hx_sim* sim, int sid, char* mech, int mech_cap, char* var, int var_cap, int* idx,
                        int* num_targets);

/* Handle of the monitor on (mech, var, idx), -1 if none (SimRuntimeCore get_monitor_handle). */
int hx_get_monitor_handle(hx_sim* sim, const char* mech, const char* var, int idx);
/* All VecPlay keys as "mech\tvar\tidx\n" lines into buf; returns the size needed. */
int hx_get_vecplay_keys(hx_sim* sim, char* buf, int cap);

/* ---- optimizers (SimWrapper.cpp:159-460, simulate.cpp:1150-1260, optimizer.cpp:102-457).
 * type "sgd", "momentum" (or "sgdmomentum", "sgd_momentum") or "adam"; returns the id.
 * A parameter batch is one tied group: the update uses the mean of its gradients times
 * impedance times inv_record_steps and writes the same value to all its weights; the
 * gradients are zeroed after each step.  Weights and gradients are variable handles: any
 * variable, including ExpSyn/Exp2Syn "weight" (netcon weights) and the adjoint's gradients
 * hh "grad_gnabar" / "grad_gkbar", pas "grad_g_pas", Ca_HVA "grad_gbar", hd_la "grad_ghdbar"
 * and ExpSyn / Exp2Syn "grad_weight". ---- */
int hx_create_optimizer(hx_sim* sim, const char* type);
int hx_configure_optimizer(hx_sim* sim, int opt, double momentum, double beta1, double beta2, double eps);
int hx_optimizer_add_param(hx_sim* sim, int opt, int weight_handle, int grad_handle, double impedance);
int hx_optimizer_add_param_batch(hx_sim* sim, int opt, int n, const int* weight_handles, const int* grad_handles,
                                 double impedance);
/* inv_record_steps = dt / record_time (simulate.cpp:1198-1211). */
int hx_optimizer_step(hx_sim* sim, int opt, double lr, double record_time, double dt);
int hx_optimizer_step_with_inv_record_steps(hx_sim* sim, int opt, double lr, double inv_record_steps);
/* One group per weight handle with a library-owned gradient, set by
 * hx_optimizer_set_external_grads_f32 (n values, the handles' order). */
int hx_optimizer_add_external_grads(hx_sim* sim, int opt, int n, const int* weight_handles, double impedance);
int hx_optimizer_set_external_grads_f32(hx_sim* sim, int opt, int n, const float* grads);
int hx_optimizer_clear_external_grads(hx_sim* sim, int opt);
int hx_optimizer_reset_state(hx_sim* sim, int opt);
/* Adam only: step count, per-group m and v (up to cap), and the hyperparameters; returns the
 * group count. */
int hx_optimizer_get_adam_state(hx_sim* sim, int opt, long long* step, double* m, double* v, int cap, double* beta1,
                                double* beta2, double* eps);
int hx_optimizer_set_adam_state(hx_sim* sim, int opt, long long step, int n, const double* m, const double* v,
                                double beta1, double beta2, double eps);

/* ---- capacity and diagnostics ---- */
/* Event-ring capacity per delivery step (default sized from the model). */
int hx_set_event_capacity(hx_sim* sim, int per_step);
/* enable = 1 (default): fold each step's state update into the next step's current pass when that is
 * exact; 0: always run the reference's separate current and state passes. */
int hx_set_fusion(hx_sim* sim, int enable);
/* No reference counterpart.  enable = 1 (default): a node-kernel launch of a steady step (state
 * update and currents, nothing stored but states, d and rhs) whose dense mechanism set has a
 * compile-time instance (pas, hh, Ca_HVA, Ih, CaDynamics_E2 and the three ions on every node;
 * pas alone) runs that instance; 0: always the generic kernel.  Same bits either way. */
int hx_set_dense_steady(hx_sim* sim, int enable);
/* No reference counterpart.  enable = 1 (default): hx_run, hx_continue_run and hx_fadvance may
 * return with their last step's state update (nrn_state) still pending when no monitor, tape or
 * signal capture samples the states; the next stepping call's first node pass applies it, as every
 * step applies the previous one, and any other entry point first completes it with the pass the
 * call would have ended with.  When every density mechanism runs in the fused node kernel, that
 * kernel's assigned outputs of the last step are made the same way, on the first entry point that
 * is not a stepping call.  Results are the same bits either way; 0: every call ends with that
 * pass and stores its outputs. */
int hx_set_close_deferral(hx_sim* sim, int enable);
/* No reference counterpart.  enable = 1 (default): a mechanism parameter column that holds
 * one value for every instance at hx_load_model is read by the node kernels as that value
 * instead of once per instance from HBM (the full column stays in HBM and is what handles,
 * get_array and the other kernels use; any handle into a column ends its scalar reading).
 * 0: every column is read per instance.  Takes effect from the next step. */
int hx_set_uniform_columns(hx_sim* sim, int enable);
/* Per-kernel timing with HIP events on the library's stream: enable, then read
 * accumulated milliseconds and launch counts for a kernel class
 * ("mech", "sparse", "point", "solve", "spike", "events", "other"). */
int hx_set_profiling(hx_sim* sim, int enable);
/* Time only the listed classes (comma-separated, e.g. "mech"); "" turns timing off.
 * Fewer timed classes means fewer events on the stream, so less perturbation. */
int hx_set_profiling_classes(hx_sim* sim, const char* classes);
int hx_get_kernel_time(hx_sim* sim, const char* kernel, double* ms, long long* launches);
/* Measurement helper (no counterpart in the reference): the mean time in ms of `reps`
 * launches of a streaming kernel that reads `nread` and writes `nwrite` fp64 arrays of n
 * elements at each thread's index with non-temporal hints -- the practical HBM rate of the
 * node kernel's access mix.  (nread, nwrite) is (1, 1), (11, 9) (the node kernel's config-3
 * columns) or (26, 9) (the same with every parameter column read); anything else returns
 * -1.  Allocates and frees its own arrays. */
int hx_measure_stream(int nread, int nwrite, long long n, int reps, double* ms);
/* Cell groups (no counterpart in the reference; an MI355X scheduling choice).  When
 * nothing couples cells across groups -- no detector-driven netcons, gaps or point
 * currents outside the node kernel, every density mechanism in the node kernel -- the
 * cells are split into ngroup contiguous groups and, in runs without VecPlay, taping,
 * capture or non-voltage monitors, each group's step chain is issued on its own HIP
 * stream, so one group's latency-bound tree solve overlaps another group's HBM-bound
 * node pass.  Results are identical to a single group.  0 (default) picks 2 (the
 * fastest on config 3: 3 and 4 groups are slower); 1 turns it off.  Call before
 * hx_load_model. */
int hx_set_cell_groups(hx_sim* sim, int ngroup);
/* Root of each cell's tree solve (no counterpart in the reference: its solve always
 * eliminates toward the model root).  centre != 0 (default): the midpoint of the cell's
 * longest path, which shortens the solve's chain of dependent rounds; 0: the model's
 * root.  The solution is the same up to rounding; after a step, d holds the pivots of
 * the order used.  Call before hx_load_model. */
int hx_set_solver_root(hx_sim* sim, int centre);
/* Cells per solve unit (no counterpart in the reference, whose solve packs cells into
 * 32-thread groups, permute_order.cpp:971-1170): the tree solve runs one wavefront per
 * unit of `cells` consecutive cells, solved together as a forest.  A wavefront issues
 * the same instructions however many of its lanes carry work, so fewer, fuller
 * wavefronts shorten the solve.  0 (default): about ncell / 1024 cells per unit (one
 * wavefront per SIMD), fewer where a unit's schedule would exceed 40 KB of LDS.  Results
 * do not depend on it.  Call before hx_load_model. */
int hx_set_solve_unit_cells(hx_sim* sim, int cells);
/* Solve units per workgroup (no counterpart in the reference): the tree solve's workgroup
 * holds this many units, one wavefront each, which the CU spreads over its SIMDs.  0
 * (default): 4, fewer where their LDS would exceed a workgroup's.  Results do not depend
 * on it.  Call before hx_load_model. */
int hx_set_solve_waves(hx_sim* sim, int waves);
/* Tree solve kernel (no counterpart in the reference): enable = 1 (default) holds each
 * solve unit whole in LDS when the largest unit's nodes, rounds and chunks fit 40 KB
 * (cells of up to about 900 nodes at one cell per unit): d, rhs, a, b and v are read once
 * into one record per node and v is written once, every intermediate stays in LDS.  0, or
 * a larger unit: the rounds are streamed through LDS from HBM.  The same bits either way;
 * hx_get_info("solve_resident") reports the choice.  Call before hx_load_model. */
int hx_set_solve_resident(hx_sim* sim, int enable);
/* Tree solve unknown (no counterpart in the reference): enable = 1 (default) lets a model
 * whose node kernel makes every term of d and rhs (no density mechanism on its own kernel,
 * no IClamp or HalfGap instance, no plugin) store rhs + d v, so that the solve yields the
 * new voltage directly and never reads v (the axial terms cancel); the reference's form
 * solves for x = v_new - v and adds it.  The two agree to rounding (about 1e-13 mV per
 * step); rhs still holds x wherever it is read.  hx_get_info("solve_voltage") reports the
 * form in use.  May be called at any time. */
int hx_set_solve_voltage(hx_sim* sim, int enable);
/* Allow (1, default) or forbid (0) issuing the cell groups on their own streams in the
 * following runs; with 0 every launch goes to the library stream.  Same results. */
int hx_set_group_streams(hx_sim* sim, int enable);
/* No reference counterpart.  enable = 1 (default): with the cell groups on their own streams,
 * every step's node passes take turns (group g waits for group g-1's node pass, group 0 for the
 * last group's pass of the step before), so each group's tree solve runs beside the next group's
 * node pass; 0: only a run's first step is ordered that way.  Same results either way. */
int hx_set_group_turns(hx_sim* sim, int enable);
/* Layout facts: "nnode", "ncell", "nchunk_max", "nround_max", "dense_mask", "fused",
 * "cell_groups", "multi_stream" (1 if the last run used per-group streams), "state_pending"
 * (1 while the last stepping call's state update waits, see hx_set_close_deferral),
 * "outputs_pending" (1 while its node-kernel outputs wait), "adjoint_fused" (the mechanisms the
 * last hx_adjoint ran in its node-parallel kernels: bits 0-7 gate adjoints, 8-15 conductances,
 * 16-23 parameter terms; bit 0 pas, 1 hh, 2 Ca_HVA, 3 hd_la, 4 CaDynamics_E2; bit 24: the synapses
 * too; bit 25: the loss term too), "steady_launches" (node-kernel launches so far that ran a
 * compile-time steady-step instance, see hx_set_dense_steady), "electrode_nodes" (nodes whose
 * IClamp and HalfGap currents one launch adds when the model has both). */
long long hx_get_info(hx_sim* sim, const char* key);

/* ---- adjoint (VJP) backward pass: no reference counterpart.  It produces the
 *      parameter gradients that the reference's learn surface feeds its optimizer
 *      (LearnRuntime::replay_compute_dw_from_cached_signals_into,
 *      LearnRuntime.cpp:2298-2457), here as the exact gradient of a voltage loss
 *      through the fixed-step simulation.  Models: pas, hh, Ca_HVA, hd_la (Ih),
 *      CaDynamics_E2, ExpSyn, Exp2Syn (VecStim, NetStim or detector sources), IClamp
 *      (also driven by VecPlay), HalfGap gap junctions of the model; na/k ions with fixed
 *      reversal potentials, ca_ion with a fixed eca or eca from cai every step (style
 *      0100).  Not: VecPlay into other variables, gap transfers added at run time,
 *      plugin mechanisms. ---- */
/* Record the next run into HBM, up to max_steps steps (0 stops and frees the tape).
 * Call before hx_finitialize: deliveries at finitialize belong to step 0. */
int hx_tape_begin(hx_sim* sim, int max_steps);
/* Steps on the tape. */
int hx_tape_length(hx_sim* sim);
/* Loss = mean over samples s = 1..nsample (v after step s) and the nloss nodes of
 * (v - target[(s-1)*nloss + j])^2; nsample must equal the tape length.  Runs the
 * backward sweep and leaves per-instance gradients for hx_get_gradient. */
int hx_adjoint(hx_sim* sim, int nloss, const int* loss_nodes, const double* target, int nsample, double* loss);
/* dLoss/dparam per instance (user order): ("hh","gnabar"), ("hh","gkbar"),
 * ("pas","g_pas"), ("Ca_HVA","gbar"), ("hd_la","ghdbar"), ("HalfGap","g"), ("ExpSyn","weight")
 * and ("Exp2Syn","weight") (the weight of the netcon into that instance).  The same values
 * are the variables "grad_<var>" of the mechanism, e.g. ("Ca_HVA", "grad_gbar", i). */
int hx_get_gradient(hx_sim* sim, const char* mech, const char* var, double* out, int cap);

/* ---- Adam over tied parameter groups (AdamOptimizer::step_gpu, optimizer.cpp:351-457;
 *      SimWrapper::create_optimizer / configure_optimizer / optimizer_add_param_batch /
 *      optimizer_step_with_inv_record_steps, SimWrapper.cpp:159-283).  Gradients are
 *      the ones hx_adjoint left; a step zeroes them. ---- */
int hx_adam_create(hx_sim* sim, double beta1, double beta2, double eps);
/* One tied group: instances inst[0..n) of (mech, var) share one moment pair; the step
 * uses the mean of their gradients x impedance x inv_record_steps and writes the same
 * new value to all of them.  Returns the group index. */
int hx_adam_add_group(hx_sim* sim, int opt, const char* mech, const char* var, int n, const int* inst,
                      double impedance);
int hx_adam_step(hx_sim* sim, int opt, double lr, double inv_record_steps);
int hx_adam_get_state(hx_sim* sim, int opt, long long* step, double* m, double* v, int cap);

/* ---- Learn gradient surface: learning-signal capture and LRDS replay
 *      (LearnRuntime.cpp:197-2457, kernels replay_dw_dx.cu:9-731; Python surface
 *      heliox_learn/signals.py:102-276).  Signals and gradients are fp32. ---- */
/* LearnRuntime::set_dense_blocks_f32 (LearnRuntime.cpp:197-244; SimWrapper.cpp:533-572):
 * block b is a C-contiguous (bn[b], bn[b], k_len[b]) fp32 array; all k_len equal.
 * Blocks partition the replay columns in order.  Drops any cached capture.
 * Returns K_len (0 for nblk 0) or -1. */
int hx_set_dense_blocks_f32(hx_sim* sim, int nblk, const float* const* blocks, const int* bn, const int* k_len);
/* LearnRuntime::clear_dense_blocks (LearnRuntime.cpp:246-257) */
int hx_clear_dense_blocks(hx_sim* sim);
/* LearnRuntime::simulate_output_vs_into (LearnRuntime.cpp:259-370): finitialize(v_init),
 * then t_steps_plus1 - 1 steps; output_vs_tn[(t_steps_plus1, n_output)] receives the
 * handles' values (fp32) after finitialize and after every step. */
int hx_simulate_output_vs_into(hx_sim* sim, float* output_vs_tn, int t_steps_plus1, int n_output,
                               const int* output_v_handles, double tstop_ms, double v_init);
/* LearnRuntime::simulate_and_capture_mapped_signals_cached (LearnRuntime.cpp:1619-1984):
 * as hx_simulate_output_vs_into, and every k_mul steps each mapped channel (pure_i; with
 * percise also didv and didvpre) gathers its handles' values, rounds them to fp32,
 * multiplies by scale and sums them into column dest of the cached (T, N) signal,
 * T = (total_steps_plus1 - 1) / k_mul + 1, N = max(pure_i_dest) + 1. */
int hx_simulate_and_capture_mapped_signals_cached(
    hx_sim* sim, float* output_vs_tn, int total_steps_plus1, int n_output, const int* output_v_handles, int n_pure_i,
    const int* pure_i_handles, const int* pure_i_dest, const float* pure_i_scale, int n_didv, const int* didv_handles,
    const int* didv_dest, const float* didv_scale, int n_didvpre, const int* didvpre_handles, const int* didvpre_dest,
    const float* didvpre_scale, double tstop_ms, int k_mul, int percise, double v_init);
/* LearnRuntime::simulate_and_capture_mapped_signals_into (LearnRuntime.cpp:1289-1618): the
 * same capture with N and T = ksteps_total_plus1 given, written to the host (T, N) arrays
 * it/ditdv/ditdvpre (zeros for the dIt channels without percise); the cache is untouched. */
int hx_simulate_and_capture_mapped_signals_into(
    hx_sim* sim, float* output_vs_tn, int total_steps_plus1, int n_output, float* it_lr_tn, float* ditdv_lr_tn,
    float* ditdvpre_lr_tn, int ksteps_total_plus1, int N, const int* output_v_handles, int n_pure_i,
    const int* pure_i_handles, const int* pure_i_dest, const float* pure_i_scale, int n_didv, const int* didv_handles,
    const int* didv_dest, const float* didv_scale, int n_didvpre, const int* didvpre_handles, const int* didvpre_dest,
    const float* didvpre_scale, double tstop_ms, int k_mul, int percise, double v_init);
/* LearnRuntime::replay_compute_dw_from_cached_signals_into (LearnRuntime.cpp:2329-2359):
 * dLtdv_lr_to is (ksteps_total, n_output); pre_of_col has n_pre == N entries (-1: none);
 * dw_out_n receives N values.  Index arrays are range-checked. */
int hx_replay_compute_dw_from_cached_signals_into(hx_sim* sim, const float* dLtdv_lr_to, int ksteps_total,
                                                  int n_output, const int* poutput, const int* pre_of_col, int n_pre,
                                                  float* dw_out_n, double dt_ms, int percise, double grad_scale,
                                                  double eps, double grad_l2norm_threshold, int clip_strategy,
                                                  int clip_check_every);
/* LearnRuntime::replay_compute_dw_dx_from_cached_signals_into (LearnRuntime.cpp:2298-2328):
 * as above, plus dx_lr_it[(n_input, ksteps_total)] for the input columns pinput. */
int hx_replay_compute_dw_dx_from_cached_signals_into(hx_sim* sim, const float* dLtdv_lr_to, int ksteps_total,
                                                     int n_output, const int* poutput, const int* pinput, int n_input,
                                                     const int* pre_of_col, int n_pre, float* dw_out_n,
                                                     float* dx_lr_it, double dt_ms, int percise, double grad_scale,
                                                     double eps, double grad_l2norm_threshold, int clip_strategy,
                                                     int clip_check_every);
/* LearnRuntime::replay_compute_dw_dx_from_signals_into (LearnRuntime.cpp:372-727): the same
 * replay over host signals it/ditdv/ditdvpre given as (N, T) arrays. */
int hx_replay_compute_dw_dx_from_signals_into(hx_sim* sim, const float* it_lr_nt, const float* ditdv_lr_nt,
                                              const float* ditdvpre_lr_nt, int N, int T, const float* dLtdv_lr_to,
                                              int ksteps_total, int n_output, const int* poutput, const int* pinput,
                                              int n_input, const int* pre_of_col, float* dw_out_n, float* dx_lr_it,
                                              double dt_ms, int percise, double grad_scale, double eps,
                                              double grad_l2norm_threshold, int clip_strategy, int clip_check_every);
/* No counterpart in the reference: hx_replay_compute_dw_dx_from_signals_into for callers
 * that cannot allocate device memory (tight serving or training loops, harnesses that
 * forbid hipMalloc).  It cannot be captured into a HIP graph: it copies the host signals in
 * and the results back synchronously and synchronises the library's stream before it
 * returns.  Same arguments, checks and results;
 * every device buffer (the signals, the dv/dw history ring, the per-tick vectors) is
 * carved from one fixed 64 MiB device array that the library holds on each GPU it runs
 * on until the process ends, so the call makes no hipMalloc/hipFree.  A problem whose
 * buffers do not fit (about 8 (K_len + 1) N^2 + 16 N T bytes with percise) is refused
 * with an error.  The dense blocks must already be set.  Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (from several threads) race. */
int hx_replay_compute_dw_dx_from_signals_into_noalloc(
    hx_sim* sim, const float* it_lr_nt, const float* ditdv_lr_nt, const float* ditdvpre_lr_nt, int N, int T,
    const float* dLtdv_lr_to, int ksteps_total, int n_output, const int* poutput, const int* pinput, int n_input,
    const int* pre_of_col, float* dw_out_n, float* dx_lr_it, double dt_ms, int percise, double grad_scale, double eps,
    double grad_l2norm_threshold, int clip_strategy, int clip_check_every);
/* LearnRuntime::simulate_and_replay_dw_dx_streaming_into (LearnRuntime.cpp:729-1288):
 * finitialize(v_init), ksteps_total * k_mul steps with the mapped channels captured every
 * k_mul steps into N columns, then the replay (cached clip schedule) into dw_out_n[N] and
 * dx_lr_it[(n_input, ksteps_total)].  dt_ms > 0 must match the model's dt. */
int hx_simulate_and_replay_dw_dx_streaming_into(
    hx_sim* sim, const float* dLtdv_lr_to, int ksteps_total, int n_output, const int* poutput, const int* pinput,
    int n_input, int N, const int* pre_of_col, float* dw_out_n, float* dx_lr_it, int n_pure_i,
    const int* pure_i_handles, const int* pure_i_dest, const float* pure_i_scale, int n_didv, const int* didv_handles,
    const int* didv_dest, const float* didv_scale, int n_didvpre, const int* didvpre_handles, const int* didvpre_dest,
    const float* didvpre_scale, double tstop_ms, int k_mul, int percise, double v_init, double dt_ms,
    double grad_scale, double eps, double grad_l2norm_threshold, int clip_strategy, int clip_check_every);
/* Timing of the replay's correction-GEMM launches with HIP events on the library stream
 * (no counterpart in the reference; used by the benchmark). */
int hx_set_replay_timing(hx_sim* sim, int enable);
int hx_get_replay_kernel_time(hx_sim* sim, double* ms, long long* launches);

/* Host emulation of the device tree solve (no counterpart in the reference;
 * a diagnostic for CPU-only checks of the solver schedule): capacitance and
 * axial assembly, elimination and back substitution over the same chunk
 * schedule the kernel uses, then v += dv.  Arrays are in node order; d and rhs
 * hold the membrane-mechanism diagonal and right-hand side.  Every chunk is
 * also solved without its round's length bound; returns -2 if the two differ
 * in any bit (the bound may only skip padding). */
int hx_emulate_tree_solve(int ncell, int nnode, const int* parent, const double* a, const double* b,
                          const double* cm, double cfac, double* v, const double* d, const double* rhs,
                          int* nchunk_max, int* nround_max);

/* Philox4x32-10 block (no counterpart in the reference's API; the generator of its vendored
 * Random123, src/third_party/Random123/philox.h, as published by Salmon et al., SC11): out =
 * philox(ctr[4], key[2]).  A diagnostic for known-answer checks of the NetStim streams. */
int hx_random123_philox4x32(const uint32_t* ctr, const uint32_t* key, uint32_t* out);
/* No reference counterpart: the node kernel's logarithm (the per-step Nernst potential), built
 * for the host from the same source, for CPU checks of its accuracy.  y[i] = ln x[i] for n
 * positive, finite, normal x; returns -1 (nothing defined) if any x is outside that range. */
int hx_fastmath_log(const double* x, double* y, int n);
/* The self-event times of one NetStim instance up to t_end with step dt, as the library makes
 * them at finitialize (see hx_model_add_netcon): a diagnostic of the host-side generator.
 * Writes up to cap times to out and returns their total count (-1 on error). */
int hx_netstim_train(double dt, double t_end, double interval, double number, double start, double noise,
                     unsigned id1, unsigned id2, unsigned id3, double* out, int cap);

/* The same with an explicit solve unit size: unit_cells consecutive cells
 * share one schedule (0: the library's choice, as hx_emulate_tree_solve). */
int hx_emulate_tree_solve_units(int ncell, int nnode, const int* parent, const double* a, const double* b,
                                const double* cm, double cfac, double* v, const double* d, const double* rhs,
                                int unit_cells, int* nchunk_max, int* nround_max);

#ifdef __cplusplus
}
#endif
#endif /* HELIOX_AMD_H */
