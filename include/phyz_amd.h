/* phyz_amd.h — C ABI of the MI355X batched rigid-body stepper.
 *
 * Drop-in for the batched-world surface of the reference's phyz-gpu:
 * BatchSim<B: KernelBackend> (crates/phyz-gpu/src/cuda/mod.rs:430-1377), the
 * surface it shares with the wgpu GpuBatchSimulator
 * (crates/phyz-gpu/src/gpu_batch_simulator.rs). One fused HIP kernel per step
 * span replaces the reference's four passes launched through KernelBackend
 * (launch_pd / launch_contact / launch_aba / launch_integrate,
 * crates/phyz-gpu/src/cuda/mod.rs:260-311, bodies in
 * crates/phyz-gpu/cuda/phyz_kernels.cu:464-1421).
 *
 * Conventions
 *   - Every function returns 0 on success and nonzero on error; the message is
 *     in phz_last_error(sim) (phz_last_error(NULL) after a failed create). This
 *     replaces the reference's Result<_, String>.
 *   - Host arrays are f64 and world-major, the reference wire layout
 *     (crates/phyz-gpu/src/layout.rs:327-373): q[w * nq + j], v[w * nv + j].
 *   - Tables keep the reference slot meanings (crates/phyz-gpu/src/layout.rs:19-93)
 *     in f64; integer slots (parent, joint type, offsets, indices) are exact
 *     integer-valued doubles rather than bit casts.
 *   - A sim owns its device buffers and one HIP stream; it is not thread-safe
 *     (use one sim per thread). Work is ordered on the sim's stream; readbacks
 *     synchronize.
 */
#ifndef PHYZ_AMD_H
#define PHYZ_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct phz_sim phz_sim;

enum { PHZ_F32 = 0, PHZ_F64 = 1 };
enum { PHZ_NOISE_NORMAL = 0, PHZ_NOISE_UNIFORM = 1 };

#define PHZ_BODY_STRIDE 36  /* layout.rs:19-38 BODY_STRIDE */
#define PHZ_GEOM_STRIDE 24  /* layout.rs:40-62 GEOM_STRIDE */
#define PHZ_PD_DOF_STRIDE 8 /* layout.rs:83-93 PD_DOF_STRIDE */
#define PHZ_CONTACT_ROW 8   /* layout.rs:68-81 CONTACT_STATE_STRIDE slots 0..8 */
#define PHZ_MAX_BODIES 32   /* layout.rs:95-100 MAX_BODIES */

/* BatchSim::with_backend / CudaBatchSimulator::on_device (mod.rs:477-543).
 * body_table: nb x 36 f64. Rejects nb > 32 and nq != nv like the reference.
 * device_ordinal -1 creates a host-only sim that can configure and compile its
 * kernel (phz_compile) but not step. */
int phz_sim_create(const double* body_table, uint32_t nb, uint32_t nq, uint32_t nv, const double gravity[3],
                   double dt, uint32_t nworld, int precision, int device_ordinal, phz_sim** out);
void phz_sim_destroy(phz_sim* sim);
const char* phz_last_error(const phz_sim* sim);

/* BatchSim::set_model (mod.rs:573-597): same body count and widths, new constants. */
int phz_set_model(phz_sim* sim, const double* body_table, uint32_t nb, uint32_t nq, uint32_t nv,
                  const double gravity[3], double dt);

/* BatchSim::enable_ground_contact (mod.rs:605-624): one global stiffness and
 * damping. geom_table: nb x 24 f64 shapes (slots 8 and 9 are overwritten with
 * k and d). Writes the collidable-body count; errors when it is zero. */
int phz_enable_ground_contact(phz_sim* sim, double ground_height, double stiffness, double damping,
                              double friction, const double* geom_table, uint32_t* collidable_out);
/* BatchSim::enable_ground_contact_per_body (mod.rs:630-640): gains nb x 2 (k, d). */
int phz_enable_ground_contact_per_body(phz_sim* sim, double ground_height, double friction, const double* gains,
                                       const double* geom_table, uint32_t* collidable_out);
/* BatchSim::enable_ground_contact_with_plane / enable_contact_terrain
 * (mod.rs:642-680): per-body gains (nb x 2: k, d) over the flat ground or a
 * heightfield, with an optional body-attached plane.
 *   plane         NULL, or [body, offset, max_depth, half_x, half_y] (BodyPlane,
 *                 contact_pipeline.rs:300-353); plane_exclude lists bodies that
 *                 never touch it (the plane body never does)
 *   hf, heights   NULL, or [nx, ny, origin x, origin y, origin z, cell] and the
 *                 ny x nx heights, row-major (phyz_model::Heightfield); the node
 *                 buffer is sized to this first field
 * Writes the collidable-body count; errors when it is zero. */
int phz_enable_contact_terrain(phz_sim* sim, double ground_height, double friction, const double* gains,
                               const double* geom_table, const double* plane, const uint32_t* plane_exclude,
                               uint32_t n_exclude, const double* hf, const double* heights, uint32_t* collidable_out);
/* BatchSim::enable_contact_impulse (mod.rs:680-701): the velocity-level impulse
 * solve, contact_sweeps x [contact, ABA] per step, warm-started from the last.
 * Same arguments as phz_enable_contact_terrain, plus solver: NULL for the
 * reference's values (restitution 0, threshold 0.05, solref erp from
 * timeconst 0.02 / dampratio 1 at the model's dt, margin 0.001, SolImp
 * 0.9 / 0.95 / 0.001 / 0.5 / 2), or those 9 numbers in that order (extension). */
int phz_enable_contact_impulse(phz_sim* sim, double ground_height, double friction, const double* gains,
                               const double* geom_table, const double* plane, const uint32_t* plane_exclude,
                               uint32_t n_exclude, const double* hf, const double* heights, const double* solver,
                               uint32_t* collidable_out);
/* BatchSim::set_heightfield (mod.rs:743-760): new terrain up to the node count
 * contact was enabled with. */
int phz_set_heightfield(phz_sim* sim, const double* hf, const double* heights);
/* BatchSim::contact_sweeps, a public field (mod.rs:450-451); default 16. */
int phz_set_contact_sweeps(phz_sim* sim, uint32_t sweeps);
int phz_contact_sweeps(const phz_sim* sim);
/* Extensions for checking and checkpointing the contact solver: the whole
 * contact state, [nworld][nb][56] (layout.rs:68-81: readback row, ground
 * impulses, plane impulses), and the per-body contact forces [nworld][nb][6]
 * the next impulse-mode step starts from (ext may be NULL). */
int phz_readback_contact_state(phz_sim* sim, double* cs, double* ext);
int phz_load_contact_state(phz_sim* sim, const double* cs, const double* ext);
/* BatchSim::enable_pd_control (mod.rs:765-786): dofs n x 8 (PD_DOF_STRIDE slots). */
int phz_enable_pd_control(phz_sim* sim, const double* dofs, uint32_t n);
/* BatchSim::set_position_targets (mod.rs:789-796): rows [nworld][n]. */
int phz_set_position_targets(phz_sim* sim, const double* rows);

/* No reference counterpart: a device-side control stream that writes
 * ctrl[v_indices[k]] every step, before PD (uniform: a + (b - a) u; normal:
 * a + b z, Box-Muller). Per-world seed world_seed(seed, w) and xorshift64
 * draws as the reference's KernelRng (crates/phyz-gpu/src/policy_pipeline.rs:417-456).
 * Generates the benchmark workloads' per-step torques without a host upload. */
int phz_enable_control_noise(phz_sim* sim, uint64_t seed, int dist, double a, double b,
                             const uint32_t* v_indices, uint32_t n);

/* Terms of the reference's CPU model (phyz_model::Model) that its device body
 * table has no slots for, applied as the CPU dynamics apply them
 * (crates/phyz-rigid/src/actuation.rs:18-39, crates/phyz-model/src/joint.rs:196-247):
 *   joint terms  nb x 8: [limited, lo, hi, limit_stiffness, limit_damping,
 *                friction_loss, 0, 0] per body (Joint::limits, limit_stiffness,
 *                limit_damping, friction_loss); one-DOF joints only. NULL clears.
 * A batched simulator built from a Model with limits or friction loss calls
 * this once after create. */
int phz_set_joint_terms(phz_sim* sim, const double* table);
/* Model::actuators (crates/phyz-model/src/model.rs:18-82, actuator_forces_at
 * 203-231): n x 16 [joint (body index), gear, gain, bias_q, bias_v,
 * has_ctrl_range, ctrl_lo, ctrl_hi, has_force_range, force_lo, force_hi, 0...];
 * each drives the first DOF of its joint with gear (gain clamp(ctrl) +
 * bias_q q + bias_v v), then the force range. With n > 0 the controls of
 * load_states / set_controls / readback_controls and the control-noise indices
 * are one per actuator (Model::nu) instead of one per DOF, and are zeroed
 * here. PD servos write per-DOF controls, so they and actuators exclude each
 * other. n = 0 clears. */
int phz_set_actuators(phz_sim* sim, const double* table, uint32_t n);
/* Controls per world: the actuator count, or nv without actuators. */
int phz_nctrl(const phz_sim* sim);

/* BatchSim::load_states (mod.rs:799-807) and set_controls (mod.rs:810-815).
 * ctrl may be NULL (zeros). Loading states also reseeds the control stream. */
int phz_load_states(phz_sim* sim, const double* q, const double* v, const double* ctrl);
int phz_set_controls(phz_sim* sim, const double* ctrl);

/* BatchSim::try_step / step_many (mod.rs:818-875): n steps, replayed from a
 * cached hipGraph when graphs are enabled; bit-identical either way. */
int phz_step(phz_sim* sim);
int phz_step_many(phz_sim* sim, uint32_t n);
int phz_set_graphs_enabled(phz_sim* sim, int on); /* BatchSim::set_graphs_enabled (mod.rs:549-555) */
int phz_graphs_enabled(const phz_sim* sim);        /* BatchSim::graphs_enabled (mod.rs:557-559) */
int phz_synchronize(phz_sim* sim);

/* BatchSim::readback_states (mod.rs:978-983): q [nworld][nq], v [nworld][nv]. */
int phz_readback_states(phz_sim* sim, double* q, double* v);
/* No counterpart in the reference. For callers that cannot allocate device
 * memory (tight serving loops, harnesses that forbid hipMalloc):
 * phz_readback_states staged through the library's static 32 MiB per-GPU
 * scratch array instead of the sim's lazily allocated staging buffer, so no
 * call allocates. Rejects nworld * max(nq, nv) * 8 bytes above 32 MiB.
 * Synchronizes the sim's stream, so it returns an error while that stream is
 * capturing a graph. All calls on one GPU share its array and take turns on a
 * per-device host mutex (two threads or two sims on one GPU are serialized). */
int phz_readback_states_noalloc(phz_sim* sim, double* q, double* v);
/* BatchSim::readback_contacts (mod.rs:988-997): [nworld][nb][8] = touching,
 * penetration, point (x, y, z), force (x, y, z); errors before contact is enabled. */
int phz_readback_contacts(phz_sim* sim, double* rows);
/* Extensions for checking and checkpointing: the ctrl buffer (including what PD
 * and the control stream wrote), the last step's qdd, and the per-world
 * control-stream states. */
int phz_readback_controls(phz_sim* sim, double* ctrl);
int phz_readback_qdd(phz_sim* sim, double* qdd);
int phz_readback_rng(phz_sim* sim, uint64_t* states);
int phz_load_rng(phz_sim* sim, const uint64_t* states);
/* BatchSim::collidable_bodies (mod.rs:1000-1003). */
int phz_collidable_bodies(const phz_sim* sim);

/* Compile the step kernel (and the control-loop kernels, once kinematics or
 * the policy are enabled) for the current configuration now; otherwise each is
 * compiled at its first launch. Works on host-only sims. */
int phz_compile(phz_sim* sim);
/* Measurement: `reps` spans of n steps (n >= 1) on the sim's stream, each
 * timed by hipEvents that its first and last launch stamp with their own start
 * and end (hipExtModuleLaunchKernel): ms_per_rep[reps] receives the kernels'
 * execution time from the first start to the last end, without the dispatch
 * around them. */
int phz_time_step_many(phz_sim* sim, uint32_t n, uint32_t reps, double* ms_per_rep);
/* Kernel resource use of the compiled step kernel that a launch of [5] steps
 * runs: [0] VGPRs per lane (arch), [1] AGPRs, [2] SGPRs, [3] private
 * (scratch) bytes per lane, [4] block size, [5] max steps per launch. A large
 * launch of a kernel above 256 registers may run a second build of the same
 * arithmetic for two resident waves per SIMD (spilling to scratch) in its
 * launches of 16 steps or more; shorter launches run the one-wave build. */
int phz_kernel_info(phz_sim* sim, int64_t* info);
/* Lanes per world of the compiled step kernel: 1, or 2 or 4 when a small
 * launch splits each world's revolute-joint sincos over several lanes; -1 on
 * error. No counterpart in the reference (its kernel is one thread per world,
 * crates/phyz-gpu/cuda/phyz_kernels.cu); it reports this build's launch
 * layout. Works on host-only sims. */
int phz_lanes_per_world(phz_sim* sim);

/* ── Device-resident control loop (mod.rs:1004-1376; policy_pipeline.rs) ──── */

#define PHZ_XF_STRIDE 18      /* policy_pipeline.rs:21-29 XF_STRIDE */
#define PHZ_OBS_OP_STRIDE 4   /* policy_pipeline.rs:31-32 OBS_OP_STRIDE */
#define PHZ_POLICY_MAX_IN 128 /* policy_pipeline.rs:34-42 */
#define PHZ_POLICY_MAX_H 256
#define PHZ_POLICY_MAX_OUT 32

/* BatchSim::enable_kinematics / compute_kinematics / readback_kinematics
 * (mod.rs:1004-1040). The readout is [nworld][nb][18]: rotation world->body
 * (row-major), body origin in world, angular and linear velocity in the body
 * frame. compute runs FK over the current q, v on the device. */
int phz_enable_kinematics(phz_sim* sim);
int phz_compute_kinematics(phz_sim* sim);
int phz_readback_kinematics(phz_sim* sim, double* rows);

/* BatchSim::enable_policy (mod.rs:1045-1140) with PolicySpec
 * (policy_pipeline.rs:300-416) passed flat:
 *   ops        n_in x 4 rows [kind, a, b, c] of ObsOp::pack (policy_pipeline.rs:115-137)
 *   aux        n_aux values of pack_obs_ops' aux buffer (ComOverSupport payloads)
 *   hidden     width of both hidden layers
 *   act_slots  n_out PD servo slots (registration order) receiving base + clamp(action)
 *   act_clamp  scalar clamp, used when act_clamp_slots is NULL
 *   act_clamp_slots  n_out per-action clamps, or NULL
 *   noise_rho  AR(1) coefficient of the exploration noise
 *   input_noise  n_in per-input noise scales
 *   history_steps  control steps of observation/action history kept on device
 * Needs PD control. Re-enabling with the same widths and history keeps the
 * weights, std, streams and history buffers, like the reference. */
int phz_enable_policy(phz_sim* sim, const double* ops, uint32_t n_in, const double* aux, uint32_t n_aux,
                      uint32_t hidden, const uint32_t* act_slots, uint32_t n_out, double act_clamp,
                      const double* act_clamp_slots, double noise_rho, const double* input_noise,
                      uint32_t history_steps);
/* BatchSim::set_policy_weights (mod.rs:1149-1162): n_in*h + h + h*h + h + h*n_out + n_out
 * values, W1 b1 W2 b2 W3 b3, each W row-major [out][in]. */
int phz_set_policy_weights(phz_sim* sim, const double* weights, uint64_t n);
/* BatchSim::set_policy_std (mod.rs:1164-1177): n_out standard deviations. */
int phz_set_policy_std(phz_sim* sim, const double* stdv, uint32_t n);
/* BatchSim::set_policy_base_targets (mod.rs:1179-1186): [nworld][n_pd] rows. */
int phz_set_policy_base_targets(phz_sim* sim, const double* rows);
/* BatchSim::seed_policy (mod.rs:1188-1203): world_seed(seed, w) streams, AR(1) state zeroed. */
int phz_seed_policy(phz_sim* sim, uint64_t seed);
/* BatchSim::run_policy (mod.rs:1205-1270): FK, observation row `step`, MLP,
 * Gaussian sample into action row `step` and the PD targets. */
int phz_run_policy(phz_sim* sim, uint32_t step);
/* BatchSim::readback_policy_history (mod.rs:1272-1302) for steps [start, end):
 * obs [step][nworld][n_in], out [step][nworld][n_out + 1] (actions, then log-prob). */
int phz_readback_policy_history(phz_sim* sim, uint32_t start, uint32_t end, double* obs, double* out);
/* BatchSim::readback_targets (mod.rs:1304-1309): [nworld][n_pd]. */
int phz_readback_targets(phz_sim* sim, double* rows);

/* BatchSim::enable_state_history / record_state / readback_state_history
 * (mod.rs:1313-1376): q [slot][nworld][nq], v [slot][nworld][nv]. */
int phz_enable_state_history(phz_sim* sim, uint32_t slots);
int phz_record_state(phz_sim* sim, uint32_t slot);
int phz_readback_state_history(phz_sim* sim, uint32_t start, uint32_t end, double* q, double* v);

/* Extension: a collector's rollout as one call, the loop of
 * docs/design/cuda-backend.md section 7 — for c in [0, n_control):
 * run_policy(first + c); step_many(control_every); if record_states,
 * record_state(first + c). Captured into one hipGraph when graphs are enabled. */
int phz_rollout(phz_sim* sim, uint32_t first_step, uint32_t n_control, uint32_t control_every, int record_states);
/* Measurement: reps rollouts (as phz_rollout), each bracketed by hipEvents.
 * The first rollout of a new shape captures its graph: warm up with
 * phz_rollout first to keep capture out of the timed region. */
int phz_time_rollout(phz_sim* sim, uint32_t first_step, uint32_t n_control, uint32_t control_every,
                     int record_states, uint32_t reps, double* ms_per_rep);
/* Measurement: reps launches of one control-loop kernel (0 = FK/observation,
 * 1 = policy) for history row `step`, each bracketed by hipEvents. */
int phz_time_control_kernel(phz_sim* sim, int which, uint32_t step, uint32_t reps, double* ms_per_rep);
/* Resource use of a control-loop kernel (0 = FK/observation, 1 = policy), as
 * phz_kernel_info; [4] is the block size, [5] the worlds per workgroup. */
int phz_control_kernel_info(phz_sim* sim, int which, int64_t* info);

/* ── PPO update on the device: the reference's TrainPipeline
 * (crates/phyz-gpu/src/cuda/train.rs:523-805; kernels
 * crates/phyz-gpu/cuda/phyz_train.cu:95-362). Two three-layer tanh MLPs (an
 * actor with a global log_std after b3, a critic with one output), flat
 * parameters in tang's Mlp::to_flat order (W1 [n_h][n_in], b1, W2 [n_h][n_h],
 * b2, W3 [n_out][n_h], b3), Adam with f64 master weights and moments. ── */
typedef struct phz_train phz_train;

/* NetDims (train.rs:53-100). */
typedef struct { uint64_t n_in, n_h, n_out; } phz_net_dims;
/* AdamCfg (train.rs:102-129); TrainPipeline::new's default is
 * {3e-4, 0.9, 0.999, 1e-8, 0}. */
typedef struct { double lr, beta1, beta2, epsilon, weight_decay; } phz_adam_cfg;
/* KlMode (train.rs:150-156). */
#define PHZ_KL_CUMULATIVE 0
#define PHZ_KL_MINIBATCH 1
/* PpoUpdateCfg (train.rs:131-148). target_kl = +inf never brakes. */
typedef struct {
  double clip, entropy_coef, vdelta;
  uint64_t minibatch, epochs;
  double target_kl, kl_scale;
  int32_t kl_mode;
} phz_ppo_cfg;
/* UpdateStats (train.rs:158-172). */
typedef struct {
  double policy_loss, value_loss, kl;
  uint64_t grad_steps;
  int32_t stopped_early;
} phz_update_stats;

/* TrainPipeline::new (train.rs:570-626): same limits and messages (hidden
 * width <= 256, output width <= 64, critic output 1). capacity: most samples
 * per upload; max_b: largest minibatch. */
int phz_train_create(phz_net_dims actor, phz_net_dims critic, uint64_t capacity, uint64_t max_b, int device_ordinal,
                     phz_train** out);
void phz_train_destroy(phz_train* t);
/* The last error's message; with NULL, the last failed create's. */
const char* phz_train_last_error(const phz_train* t);
/* TrainPipeline::device_name (train.rs:628-631). */
int phz_train_device_name(const phz_train* t, char* buf, uint64_t len);
/* Parameter count of network 0 (actor, log_std included) or 1 (critic). */
uint64_t phz_train_param_count(const phz_train* t, int net);
/* Rows of a minibatch per workgroup tile (chosen at create from LDS size). */
uint32_t phz_train_rows_per_tile(const phz_train* t);
/* TrainPipeline::set_adam (train.rs:795-803): moments and step counters persist. */
int phz_train_set_adam(phz_train* t, const phz_adam_cfg* actor, const phz_adam_cfg* critic);
/* set_actor_params / set_critic_params (train.rs:633-643): f64 flat arrays;
 * both the master copy and the f32 mirror are set. */
int phz_train_set_actor_params(phz_train* t, const double* flat, uint64_t n);
int phz_train_set_critic_params(phz_train* t, const double* flat, uint64_t n);
/* actor_params / critic_params (train.rs:645-653): the f64 master weights. */
int phz_train_actor_params(phz_train* t, double* out, uint64_t n);
int phz_train_critic_params(phz_train* t, double* out, uint64_t n);
/* upload_batch (train.rs:655-690) of one SampleBatch (train.rs:509-522), f32
 * row-major columns with their lengths: obs_a [n][actor n_in], obs_c
 * [n][critic n_in], act [n][actor n_out], logp_old, adv, ret [n]. */
int phz_train_upload_batch(phz_train* t, uint64_t n_rows, const float* obs_a, uint64_t obs_a_len, const float* obs_c,
                           uint64_t obs_c_len, const float* act, uint64_t act_len, const float* logp_old,
                           uint64_t logp_old_len, const float* adv, uint64_t adv_len, const float* ret, uint64_t ret_len);
/* update (train.rs:692-791): cfg->epochs passes, epoch e visiting the batch in
 * order[e] (order_lens[e] entries, a permutation of 0..n_rows) in minibatches
 * of cfg->minibatch. Stops after the first minibatch whose brake reading
 * exceeds cfg->target_kl. All shuffles are validated before anything runs. */
int phz_train_update(phz_train* t, const uint32_t* const* order, const uint64_t* order_lens, uint64_t n_order,
                     const phz_ppo_cfg* cfg, phz_update_stats* out);
/* Measurement: phz_train_update with hipEvents around every launch on the
 * pipeline's stream; ms_kernels[2] receives the summed times of the tile
 * kernel and of the Adam kernel (which also applies the KL brake),
 * *minibatches the minibatches launched. Waits for each minibatch, so its
 * wall time is not the update's. */
int phz_train_time_update(phz_train* t, const uint32_t* const* order, const uint64_t* order_lens, uint64_t n_order,
                          const phz_ppo_cfg* cfg, phz_update_stats* out, double* ms_kernels, uint64_t* minibatches);

#ifdef __cplusplus
}
#endif

#endif /* PHYZ_AMD_H */
