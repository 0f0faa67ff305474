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

/* Compile the step kernel for the current configuration now (otherwise it is
 * compiled at the first step). Works on host-only sims. */
int phz_compile(phz_sim* sim);
/* Measurement: `reps` spans of n steps, each bracketed by hipEvents on the
 * sim's stream; ms_per_rep[reps] receives the event times. */
int phz_time_step_many(phz_sim* sim, uint32_t n, uint32_t reps, double* ms_per_rep);
/* Kernel resource use of the compiled step kernel: [0] VGPRs per lane (arch),
 * [1] AGPRs, [2] SGPRs, [3] private (scratch) bytes per lane, [4] block size,
 * [5] max steps per launch. */
int phz_kernel_info(phz_sim* sim, int64_t* info);

#ifdef __cplusplus
}
#endif

#endif /* PHYZ_AMD_H */
