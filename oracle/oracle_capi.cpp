// oracle_capi.cpp — C ABI over phz_oracle.hpp for the Python test harness.
//
// TEST INFRASTRUCTURE ONLY (see phz_oracle.hpp). Loaded by tests/ and by the
// cpu_baseline leg of bench.py through oracle/oracle.py; never by the product.
//
// Arrays are world-major, matching the reference wire format
// (crates/phyz-gpu/src/layout.rs:340-356): q[w * nq + j], v[w * nv + j].
#include <atomic>
#include <cstdio>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "phz_oracle.hpp"

using namespace phzo;

struct orc_model {
  Model m;
};

static void set_err(char* err, int len, const char* msg) {
  if (err && len > 0) { std::snprintf(err, (size_t)len, "%s", msg); }
}

extern "C" {

orc_model* orc_model_create(const double* bodies, int nb, int nq, int nv, const double* g, double dt, char* err,
                            int errlen) {
  auto* o = new orc_model();
  const char* e = model_from_table(o->m, bodies, nb, nq, nv, g, dt);
  if (e[0]) { set_err(err, errlen, e); delete o; return nullptr; }
  return o;
}
void orc_model_destroy(orc_model* o) { delete o; }

int orc_set_contact(orc_model* o, const double* geom, double ground_h, double mu) {
  geoms_from_table(o->m, geom);
  o->m.contact = true;
  o->m.ground_h = ground_h;
  o->m.mu = mu;
  return 0;
}
// Impulse mode, body-attached plane and heightfield (ContactParams,
// contact_pipeline.rs:17-100). prm: restitution, restitution_threshold, erp,
// margin, solimp dmin, dmax, width, midpoint, power. plane: offset, max_depth,
// half_x, half_y. hf: origin x, y, z, cell; heights [ny][nx] (nullable when
// hf_nx == 0). Geometry slot 7 carries the per-body plane exclusion.
int orc_set_contact_cfg(orc_model* o, int solve_mode, int sweeps, const double* prm, int plane_body,
                        const double* plane, int hf_nx, int hf_ny, const double* hf, const double* heights) {
  ContactCfg& c = o->m.cc;
  c.solve_mode = solve_mode;
  c.sweeps = sweeps;
  c.restitution = prm[0]; c.restitution_threshold = prm[1]; c.erp = prm[2]; c.margin = prm[3];
  c.solimp_dmin = prm[4]; c.solimp_dmax = prm[5]; c.solimp_width = prm[6]; c.solimp_mid = prm[7]; c.solimp_power = prm[8];
  c.plane_body = plane_body;
  if (plane_body >= 0) {
    c.plane_offset = plane[0]; c.plane_max_depth = plane[1]; c.plane_half_x = plane[2]; c.plane_half_y = plane[3];
  }
  c.hf_nx = hf_nx;
  c.hf_ny = hf_ny;
  if (hf_nx > 0) {
    c.hf_ox = hf[0]; c.hf_oy = hf[1]; c.hf_oz = hf[2]; c.hf_cell = hf[3];
    c.hf.assign(heights, heights + (size_t)hf_nx * hf_ny);
  } else {
    c.hf.clear();
  }
  return 0;
}
// Joint terms, nb x 8: [limited, lo, hi, limit_k, limit_d, friction_loss, 0, 0].
int orc_set_joint_terms(orc_model* o, const double* t) {
  Model& m = o->m;
  m.jterms.assign(m.nb, JointTerms());
  for (int i = 0; i < m.nb; i++) {
    const double* r = t + i * 8;
    JointTerms& j = m.jterms[i];
    j.limited = r[0] != 0.0;
    j.lo = r[1]; j.hi = r[2]; j.limit_k = r[3]; j.limit_d = r[4]; j.friction_loss = r[5];
  }
  return 0;
}
// Actuators, n x 16: [body, gear, gain, bias_q, bias_v, has_ctrl_range, ctrl_lo,
// ctrl_hi, has_force_range, force_lo, force_hi, 0...]; each drives the first
// DOF of its body's joint. n = 0 removes them.
int orc_set_actuators(orc_model* o, const double* t, int n) {
  Model& m = o->m;
  m.acts.clear();
  for (int a = 0; a < n; a++) {
    const double* r = t + a * 16;
    Actuator A;
    A.body = (int)r[0];
    if (A.body < 0 || A.body >= m.nb || joint_ndof(m.bodies[A.body].jtype) == 0) return 1;
    A.qidx = m.bodies[A.body].qoff;
    A.vidx = m.bodies[A.body].voff;
    A.gear = r[1]; A.gain = r[2]; A.bias_q = r[3]; A.bias_v = r[4];
    A.has_ctrl_range = r[5] != 0.0; A.ctrl_lo = r[6]; A.ctrl_hi = r[7];
    A.has_force_range = r[8] != 0.0; A.force_lo = r[9]; A.force_hi = r[10];
    m.acts.push_back(A);
  }
  return 0;
}

int orc_set_pd(orc_model* o, const double* dofs, int n) {
  o->m.pd.clear();
  for (int i = 0; i < n; i++) {
    const double* r = dofs + i * PD_STRIDE;
    o->m.pd.push_back(PdDof{(int)r[0], (int)r[1], r[2], r[3], r[4]});
  }
  return 0;
}
int orc_set_noise(orc_model* o, uint64_t seed, int dist, double a, double b, const int* vidx, int n) {
  o->m.noise = n > 0;
  o->m.noise_seed = seed;
  o->m.noise_dist = dist;
  o->m.noise_a = a;
  o->m.noise_b = b;
  o->m.noise_dofs.assign(vidx, vidx + n);
  return 0;
}

static std::vector<SV<double>> ext_from(const Model& m, const double* ext) {
  std::vector<SV<double>> e(m.nb);
  for (int i = 0; i < m.nb; i++)
    for (int k = 0; k < 6; k++) e[i].set(k, ext[i * 6 + k]);
  return e;
}

// qdd = ABA(q, v, ctrl, ext). mode 0: aba_struct, 1: aba_dense.
int orc_aba(orc_model* o, const double* q, const double* v, const double* ctrl, const double* ext, double* qdd, int mode) {
  std::vector<SV<double>> e;
  if (ext) e = ext_from(o->m, ext);
  if (mode == 1) aba_dense<double>(o->m, q, v, ctrl, ext ? e.data() : nullptr, qdd);
  else aba_struct<double>(o->m, q, v, ctrl, ext ? e.data() : nullptr, qdd);
  return 0;
}
// f32 arithmetic through the same restatement (diagnostics: f32 rounding floor).
int orc_aba_f32(orc_model* o, const float* q, const float* v, const float* ctrl, const float* ext, float* qdd) {
  std::vector<SV<float>> e(o->m.nb);
  if (ext) for (int i = 0; i < o->m.nb; i++) for (int k = 0; k < 6; k++) e[i].set(k, ext[i * 6 + k]);
  aba_struct<float>(o->m, q, v, ctrl, ext ? e.data() : nullptr, qdd);
  return 0;
}
// FK + contact + ABA entirely in f32 arithmetic (diagnostic: the f32 rounding
// floor of one step's qdd for a given state and control).
int orc_qdd_f32(orc_model* o, const float* q, const float* v, const float* ctrl, float* qdd) {
  const Model& m = o->m;
  std::vector<SV<float>> ext(m.nb);
  if (m.contact) {
    std::vector<FK<float>> fk(m.nb);
    forward_kinematics<float>(m, q, v, fk.data());
    ground_contact<float>(m, fk.data(), ext.data(), nullptr);
  }
  aba_struct<float>(m, q, v, ctrl, m.contact ? ext.data() : nullptr, qdd);
  return 0;
}
// tau = RNEA(q, v, qdd, ext): pure rigid-body inverse dynamics, no passive terms.
int orc_rnea(orc_model* o, const double* q, const double* v, const double* qdd, const double* ext, double* tau) {
  std::vector<SV<double>> e;
  if (ext) e = ext_from(o->m, ext);
  rnea<double>(o->m, q, v, qdd, ext ? e.data() : nullptr, tau);
  return 0;
}
// Joint-space inertia, armature and dt*damping on the diagonal (nv x nv).
int orc_crba(orc_model* o, const double* q, double* M) {
  crba<double>(o->m, q, M);
  return 0;
}
// Passive + ctrl generalized force (actuation.rs:18-39 subset).
int orc_generalized_forces(orc_model* o, const double* q, const double* v, const double* ctrl, double* qfrc) {
  generalized_forces<double>(o->m, q, v, ctrl, qfrc);
  return 0;
}
// FK rows per body: w_rot (body->world, row-major 9), w_pos (3), body-frame
// spatial velocity (6) — 18 doubles.
int orc_fk(orc_model* o, const double* q, const double* v, double* out) {
  std::vector<FK<double>> fk(o->m.nb);
  forward_kinematics<double>(o->m, q, v, fk.data());
  for (int i = 0; i < o->m.nb; i++) {
    double* r = out + i * 18;
    for (int a = 0; a < 3; a++) for (int b = 0; b < 3; b++) r[a * 3 + b] = fk[i].w_rot.m[a][b];
    for (int k = 0; k < 3; k++) r[9 + k] = fk[i].w_pos[k];
    for (int k = 0; k < 6; k++) r[12 + k] = fk[i].vel.get(k);
  }
  return 0;
}
// orc_fk over nworld world-major states (out: [nworld][nb][18]), worlds split
// over `threads` threads (0: all hardware threads).
int orc_fk_batch(orc_model* o, int nworld, const double* q, const double* v, double* out, int threads) {
  const Model& m = o->m;
  if (threads <= 0) threads = (int)std::max(1u, std::thread::hardware_concurrency());
  threads = std::min(threads, std::max(1, nworld));
  auto work = [&](int w0, int w1) {
    for (int w = w0; w < w1; w++)
      orc_fk(o, q + (size_t)w * m.nq, v + (size_t)w * m.nv, out + (size_t)w * m.nb * 18);
  };
  if (threads == 1) { work(0, nworld); return 0; }
  std::vector<std::thread> pool;
  int chunk = (nworld + threads - 1) / threads;
  for (int t = 0; t < threads; t++) {
    int w0 = t * chunk, w1 = std::min(nworld, w0 + chunk);
    if (w0 >= w1) break;
    pool.emplace_back(work, w0, w1);
  }
  for (auto& th : pool) th.join();
  return 0;
}
int orc_contact(orc_model* o, const double* q, const double* v, double* ext_out, double* rows_out) {
  if (!o->m.contact) return 1;
  std::vector<FK<double>> fk(o->m.nb);
  std::vector<SV<double>> ext(o->m.nb);
  forward_kinematics<double>(o->m, q, v, fk.data());
  ground_contact<double>(o->m, fk.data(), ext.data(), rows_out);
  for (int i = 0; i < o->m.nb; i++) for (int k = 0; k < 6; k++) ext_out[i * 6 + k] = ext[i].get(k);
  return 0;
}
// One contact pass from (q, v) with the solver state cs (nb x 56, read and
// written; nullable in penalty mode). v is the velocity the pass sees: the
// free velocity v + dt qdd in impulse mode.
int orc_contact_pass(orc_model* o, const double* q, const double* v, double* ext_out, double* cs, double* rows_out) {
  if (!o->m.contact) return 1;
  std::vector<FK<double>> fk(o->m.nb);
  std::vector<SV<double>> ext(o->m.nb);
  forward_kinematics<double>(o->m, q, v, fk.data());
  contact_pass<double>(o->m, fk.data(), ext.data(), cs, rows_out);
  for (int i = 0; i < o->m.nb; i++) for (int k = 0; k < 6; k++) ext_out[i * 6 + k] = ext[i].get(k);
  return 0;
}
int orc_integrate(orc_model* o, double* q, double* v, const double* qdd) {
  integrate<double>(o->m, q, v, qdd);
  return 0;
}
uint64_t orc_world_seed(uint64_t seed, uint64_t world) { return world_seed(seed, world); }

int orc_quat_exp_log(const double* w, double* quat_out, double* log_out) {
  Q<double> qq = quat_exp(V3<double>{w[0], w[1], w[2]});
  quat_out[0] = qq.w; quat_out[1] = qq.x; quat_out[2] = qq.y; quat_out[3] = qq.z;
  V3<double> l = quat_log(qq);
  log_out[0] = l.x; log_out[1] = l.y; log_out[2] = l.z;
  return 0;
}

// Step nworld worlds nsteps times, in place. rng: per-world xorshift state
// (nullable when noise is off). targets: [nworld][n_pd]. qdd_last:
// [nworld][nv] (nullable). contact_rows: [nworld][nb][8] of the last step
// (nullable). threads <= 0 uses hardware concurrency. mode 0 struct, 1 dense.
// ext_state [nworld][nb][6] and cs_state [nworld][nb][56]: impulse-mode solver
// state carried from step to step (nullable: start from zero, not returned).
int orc_step_batch(orc_model* o, int nworld, int nsteps, double* q, double* v, double* ctrl, const double* targets,
                   uint64_t* rng, double* qdd_last, double* contact_rows, int threads, int mode, double* ext_state,
                   double* cs_state) {
  const Model& m = o->m;
  if (threads <= 0) threads = (int)std::max(1u, std::thread::hardware_concurrency());
  threads = std::min(threads, std::max(1, nworld));
  const int npd = (int)m.pd.size();
  auto work = [&](int w0, int w1) {
    WorldScratch<double> ws;
    std::vector<double> rows(m.nb * CONTACT_ROW);
    for (int w = w0; w < w1; w++) {
      double* qw = q + (size_t)w * m.nq;
      double* vw = v + (size_t)w * m.nv;
      double* cw = ctrl + (size_t)w * m.nctrl();
      const double* tw = npd ? targets + (size_t)w * npd : nullptr;
      uint64_t* rw = rng ? rng + w : nullptr;
      ws.reset(m);
      double* ew = ext_state ? ext_state + (size_t)w * m.nb * 6 : nullptr;
      double* sw = cs_state ? cs_state + (size_t)w * m.nb * CS_STRIDE : nullptr;
      if (ew) for (int i = 0; i < m.nb; i++) for (int k = 0; k < 6; k++) ws.ext[i].set(k, ew[i * 6 + k]);
      if (sw) std::memcpy(ws.cs.data(), sw, sizeof(double) * m.nb * CS_STRIDE);
      for (int s = 0; s < nsteps; s++) {
        double* cr = (contact_rows && s == nsteps - 1) ? contact_rows + (size_t)w * m.nb * CONTACT_ROW : nullptr;
        step_world<double>(m, qw, vw, cw, tw, rw, ws, cr, mode == 1);
      }
      if (ew) for (int i = 0; i < m.nb; i++) for (int k = 0; k < 6; k++) ew[i * 6 + k] = ws.ext[i].get(k);
      if (sw) std::memcpy(sw, ws.cs.data(), sizeof(double) * m.nb * CS_STRIDE);
      if (qdd_last && nsteps > 0) std::memcpy(qdd_last + (size_t)w * m.nv, ws.qdd.data(), sizeof(double) * m.nv);
    }
  };
  if (threads == 1) { work(0, nworld); return 0; }
  std::vector<std::thread> pool;
  int chunk = (nworld + threads - 1) / threads;
  for (int t = 0; t < threads; t++) {
    int w0 = t * chunk, w1 = std::min(nworld, w0 + chunk);
    if (w0 >= w1) break;
    pool.emplace_back(work, w0, w1);
  }
  for (auto& th : pool) th.join();
  return 0;
}

// Count operations of one world-step at the given state (struct formulation
// when mode 0, dense when mode 1). counts: 5 phases x 6 counters
// (add, mul, div, sqrt, trans, other), phases: noise, pd, contact, aba, integrate.
// ext0 [nb][6] / cs0 [nb][56]: impulse-mode carried state (nullable: zero);
// its values count as state.
int orc_count_ops(orc_model* o, const double* q0, const double* v0, const double* ctrl0, const double* targets0,
                  uint64_t rng_state, int mode, uint64_t* counts, const double* ext0, const double* cs0) {
  const Model& m = o->m;
  std::vector<OpScalar> q(m.nq), v(m.nv), ctrl(m.nctrl()), tg(m.pd.size());
  for (int j = 0; j < m.nq; j++) q[j] = OpScalar::state(q0[j]);
  for (int j = 0; j < m.nv; j++) v[j] = OpScalar::state(v0[j]);
  for (int j = 0; j < m.nctrl(); j++) ctrl[j] = OpScalar::state(ctrl0[j]);
  for (size_t d = 0; d < m.pd.size(); d++) tg[d] = OpScalar::state(targets0[d]);
  OpCount c;
  OpCount* prev = op_counter();
  op_counter() = &c;
  OpCount last;
  auto hook = [&](int phase) {
    uint64_t* out = counts + phase * 6;
    out[0] += c.add - last.add; out[1] += c.mul - last.mul; out[2] += c.div - last.div;
    out[3] += c.sqrt - last.sqrt; out[4] += c.trans - last.trans; out[5] += c.other - last.other;
    last = c;
  };
  WorldScratch<OpScalar> ws;
  ws.reset(m);
  if (ext0) for (int i = 0; i < m.nb; i++) for (int k = 0; k < 6; k++) ws.ext[i].set(k, OpScalar::state(ext0[i * 6 + k]));
  if (cs0) for (size_t k = 0; k < ws.cs.size(); k++) ws.cs[k] = OpScalar::state(cs0[k]);
  uint64_t r = rng_state;
  step_world<OpScalar>(m, q.data(), v.data(), ctrl.data(), tg.data(), m.noise ? &r : nullptr, ws, nullptr, mode == 1,
                       hook);
  op_counter() = prev;
  return 0;
}

}  // extern "C"
