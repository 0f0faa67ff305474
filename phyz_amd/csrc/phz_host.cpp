// phz_host.cpp — host side of the MI355X batched stepper: the BatchSim object
// behind the C ABI of include/phyz_amd.h.
//
// Mirrors crates/phyz-gpu/src/cuda/mod.rs (BatchSim<B>) and the packing rules of
// crates/phyz-gpu/src/layout.rs, with a HIP runtime in place of
// KernelBackend/CudaBackend (crates/phyz-gpu/src/cuda/nvrtc.rs). Where the
// reference compiles one generic kernel source with NVRTC and launches four
// passes per step, this compiles phz_device.h with hiprtc against the uploaded
// model (every body loop unrolled, model constants folded) and launches one
// fused kernel per span of steps.
#include <dlfcn.h>
#include <hip/hip_ext.h>
#include <hip/hip_runtime_api.h>
#include <hip/hiprtc.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <memory>
#include <map>
#include <mutex>
#include <sstream>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/phyz_amd.h"

// Text of phz_device.h and phz_control.h, embedded at build time.
static const char* const kDeviceSrc =
#include "phz_device_src.inc"
    ;
static const char* const kControlSrc =
#include "phz_control_src.inc"
    ;

extern "C" {
hipError_t phz_io_pack(const double* src, void* dst, int nworld, int width, int stride, int f64, hipStream_t s);
hipError_t phz_io_unpack(const void* src, double* dst, int nworld, int width, int stride, int f64, hipStream_t s);
hipError_t phz_io_zero(void* dst, size_t bytes, hipStream_t s);
hipError_t phz_io_seed(uint64_t* rng, uint64_t seed, int nworld, hipStream_t s);
hipError_t phz_io_copy(void* dst, const void* src, size_t bytes, hipStream_t s);
hipError_t phz_io_scratch(void** ptr, size_t* bytes, int* device);
}
std::mutex& phz_io_scratch_mutex(int device);

namespace {

constexpr int kBodyStride = PHZ_BODY_STRIDE;
constexpr int kGeomStride = PHZ_GEOM_STRIDE;
constexpr int kPdStride = PHZ_PD_DOF_STRIDE;
constexpr int kMaxBodies = PHZ_MAX_BODIES;
// Launches of at least this many steps run the two-waves-per-SIMD build of the
// step kernel where there is one (phz_sim::two_waves_pay): it saves about 1.4
// us per step at 131072 ant worlds and costs about 14 us more per launch, so
// it breaks even near 10 steps.
constexpr int kTwoWaveMinSteps = 16;

thread_local std::string g_create_error;

std::string fmt(const char* f, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, f);
  std::vsnprintf(buf, sizeof(buf), f, ap);
  va_end(ap);
  return buf;
}

int ndof_of(int jt) { return jt == 2 ? 0 : (jt == 3 ? 3 : (jt == 4 ? 6 : 1)); }

struct BodyD {
  int parent, jtype, qoff, voff;
  double mass, com[3], inertia[6], ptj_rot[9], ptj_pos[3], axis[3], damping, stiffness, spring_ref, armature;
};
struct ModelD {
  int nb = 0, nq = 0, nv = 0;
  std::vector<BodyD> b;
  double g[3] = {0, 0, 0};
  double dt = 0;
};

bool is_int(double x) { return std::isfinite(x) && x == std::floor(x); }

// Unpack and validate a body table (layout.rs:19-38 slots). The checks are the
// reference's (mod.rs:498-510: body cap, nq == nv) plus what a device kernel
// needs to be safe: topological order, offsets inside nq/nv, finite values.
bool parse_model(const double* t, uint32_t nb, uint32_t nq, uint32_t nv, const double* g, double dt, ModelD& m,
                 std::string& err) {
  if (!t || !g) { err = "null body table or gravity"; return false; }
  if (nb == 0) { err = "model has no bodies"; return false; }
  if (nb > (uint32_t)kMaxBodies) {
    err = fmt("model has %u bodies but the kernels hold at most %d per world", nb, kMaxBodies);
    return false;
  }
  if (nq != nv) {
    err = fmt("kernels assume nq == nv (exponential-coordinate ball/free joints); model has nq %u nv %u", nq, nv);
    return false;
  }
  if (!(std::isfinite(dt) && dt > 0)) { err = "dt must be finite and positive"; return false; }
  m.nb = (int)nb; m.nq = (int)nq; m.nv = (int)nv; m.dt = dt;
  for (int k = 0; k < 3; k++) {
    if (!std::isfinite(g[k])) { err = "gravity must be finite"; return false; }
    m.g[k] = g[k];
  }
  m.b.assign(nb, BodyD{});
  int nsum = 0;
  for (uint32_t i = 0; i < nb; i++) {
    const double* r = t + (size_t)i * kBodyStride;
    for (int k = 0; k < 33; k++)
      if (!std::isfinite(r[k])) { err = fmt("body %u: non-finite value in slot %d", i, k); return false; }
    if (!is_int(r[0]) || !is_int(r[1]) || !is_int(r[2]) || !is_int(r[3])) {
      err = fmt("body %u: parent, joint type and offsets must be integers", i);
      return false;
    }
    BodyD& b = m.b[i];
    b.parent = (int)r[0]; b.jtype = (int)r[1]; b.qoff = (int)r[2]; b.voff = (int)r[3];
    if (b.parent < -1 || b.parent >= (int)i) {
      err = fmt("body %u: parent %d breaks topological order (parent < child)", i, b.parent);
      return false;
    }
    if (b.jtype < 0 || b.jtype > 4) { err = fmt("body %u: unknown joint type %d", i, b.jtype); return false; }
    const int nd = ndof_of(b.jtype);
    if (b.qoff < 0 || b.voff < 0 || b.qoff + nd > (int)nq || b.voff + nd > (int)nv) {
      err = fmt("body %u: joint offsets (q %d, v %d, %d DOF) exceed nq %u / nv %u", i, b.qoff, b.voff, nd, nq, nv);
      return false;
    }
    nsum += nd;
    b.mass = r[4];
    for (int k = 0; k < 3; k++) b.com[k] = r[5 + k];
    for (int k = 0; k < 6; k++) b.inertia[k] = r[8 + k];
    for (int k = 0; k < 9; k++) b.ptj_rot[k] = r[14 + k];
    for (int k = 0; k < 3; k++) b.ptj_pos[k] = r[23 + k];
    for (int k = 0; k < 3; k++) b.axis[k] = r[26 + k];
    b.damping = r[29]; b.stiffness = r[30]; b.spring_ref = r[31]; b.armature = r[32];
  }
  if (nsum != (int)nv) { err = fmt("joint DOFs sum to %d but nv is %u", nsum, nv); return false; }
  // Every velocity slot belongs to exactly one joint.
  std::vector<int> used(nv, 0);
  for (const BodyD& b : m.b)
    for (int k = 0; k < ndof_of(b.jtype); k++)
      if (used[b.voff + k]++) { err = "joint velocity offsets overlap"; return false; }
  return true;
}

struct Features {
  bool contact = false;
  double ground_h = 0, mu = 0;
  std::vector<double> geom;  // nb x 24 (slot 7: excluded from the body-attached plane)
  int collidable = 0;
  // Contact solver and terrain (ContactParams, crates/phyz-gpu/src/contact_pipeline.rs:17-100).
  int cmode = 0;             // 0 penalty, 1 velocity-level impulse solve
  int sweeps = 16;           // [contact, ABA] sweeps per step in impulse mode (DEFAULT_CONTACT_SWEEPS)
  double prm[9] = {0.0, 0.05, 0.001 / (2.0 * 0.02 + 0.001), 0.001, 0.9, 0.95, 0.001, 0.5, 2.0};
  int plane_body = -1;       // body-attached plane: body, offset, max depth, half x, half y
  double plane[4] = {0, 0, 0, 0};
  int hf_nx = 0, hf_ny = 0;  // heightfield header; the nodes live in a device buffer
  double hf_o[3] = {0, 0, 0}, hf_cell = 1.0;
  int npd = 0;
  std::vector<double> pd;  // npd x 8
  bool noise = false;
  uint64_t seed = 0;
  int dist = 0;
  double a = 0, b = 1;
  std::vector<int> noise_dofs;
  // The launch's workgroups of 64 worlds and the device's CUs (phz_sim_create),
  // for the partition plan.
  int wgs = 0, cus = 256;
  bool f64 = false;  // the sim's precision (the planner keeps f64 subtrees one per wave)
  bool host_only = false;  // a sim without a device (device ordinal -1): code generation only
  // Terms of the CPU model that the device body table has no slots for
  // (joint.rs:27-104, model.rs:18-82): the soft position limit and dry friction
  // of one-DOF joints (one entry per body; empty: none), and actuators (empty:
  // ctrl is a per-DOF generalized force; otherwise one control per actuator).
  struct JointTerm { bool limited = false; double lo = 0, hi = 0, k = 1000, d = 60, floss = 0; };
  std::vector<JointTerm> jterms;
  struct Act {
    int body = 0, q = 0, v = 0;
    double gear = 1, gain = 1, bq = 0, bv = 0;
    bool cr = false, fr = false;
    double clo = 0, chi = 0, flo = 0, fhi = 0;  // sorted bounds
  };
  std::vector<Act> acts;
};

// ── code generation ──────────────────────────────────────────────────────────
std::string num(double x) {
  char buf[40];
  std::snprintf(buf, sizeof(buf), "%.17g", x);
  std::string s(buf);
  if (s.find_first_of(".eEn") == std::string::npos) s += ".0";
  return s;
}
template <class F> std::string arr1(int n, F f) {
  std::string s = "{";
  for (int i = 0; i < n; i++) { if (i) s += ", "; s += f(i); }
  return s + "}";
}
template <class F> std::string arr2(int n, int m, F f) {
  std::string s = "{";
  for (int i = 0; i < n; i++) {
    if (i) s += ", ";
    s += "{";
    for (int j = 0; j < m; j++) { if (j) s += ", "; s += f(i, j); }
    s += "}";
  }
  return s + "}";
}

// How the step kernel splits a world's bodies over the waves of a workgroup
// (see the PMODE comment in phz_device.h).
struct Plan {
  int mode = 0;
  std::vector<int> trunk;                // topological order
  std::vector<std::vector<int>> groups;  // bodies owned by each wave, topological order
};

Plan plan_partition(const ModelD& m, const Features& f) {
  const int nb = m.nb;
  Plan pl;
  // PHZ_HOST_LIFT_GUARDS=1 lifts the two guards below (f64 plans keep one
  // subtree per wave; no plan has exactly three waves) on host-only sims,
  // whose kernels are only generated: the host emulation of the step kernel
  // (tests/host_emulation.py) builds the guarded plans for the CPU. A device
  // sim always keeps both guards.
  const char* lift_env = std::getenv("PHZ_HOST_LIFT_GUARDS");
  const bool lift_guards = f.host_only && lift_env && lift_env[0] == '1';
  std::vector<int> all(nb);
  for (int i = 0; i < nb; i++) all[i] = i;
  const char* env = std::getenv("PHZ_PARTITION");
  const std::string want = env ? env : "auto";
  auto lane_per_world = [&]() { pl = Plan{}; pl.groups.push_back(all); return pl; };
  if (want == "0") return lane_per_world();
  // Impulse sweeps and the body-attached plane couple bodies across subtrees
  // every sweep: they run one lane per world.
  if (f.contact && (f.cmode == 1 || f.plane_body >= 0)) return lane_per_world();
  std::vector<std::vector<int>> kids(nb);
  for (int i = 0; i < nb; i++) if (m.b[i].parent >= 0) kids[m.b[i].parent].push_back(i);
  std::vector<int> size(nb, 1);
  for (int i = nb - 1; i >= 0; i--) if (m.b[i].parent >= 0) size[m.b[i].parent] += size[i];
  std::vector<char> trunk(nb, 0);
  // Fixed trunk: the bodies welded to the world through fixed joints.
  bool any_fixed = false;
  for (int i = 0; i < nb; i++) {
    const BodyD& b = m.b[i];
    trunk[i] = b.jtype == 2 && (b.parent < 0 || trunk[b.parent]);
    any_fixed = any_fixed || trunk[i];
  }
  int mode = 1;
  // Floating trunk: every body on a path from a root to a branch point (a body
  // with two or more children whose subtrees hold two or more bodies). Also
  // used when the welded bodies have a single articulated subtree (a fixed
  // forearm under a wrist and a palm): the trunk then runs through the wrist.
  auto floating = [&]() {
    mode = 2;
    trunk.assign(nb, 0);
    for (int i = 0; i < nb; i++) {
      int heavy = 0;
      for (int c : kids[i]) heavy += size[c] >= 2;
      if (heavy >= 2)
        for (int j = i; j >= 0; j = m.b[j].parent) trunk[j] = 1;
    }
  };
  auto collect = [&]() {
    std::vector<std::vector<int>> parts;
    for (int i = 0; i < nb; i++) {
      if (trunk[i] || m.b[i].parent < 0 || !trunk[m.b[i].parent]) continue;
      std::vector<int> part;
      for (int j = i; j < nb; j++) {
        int a = j;
        while (a >= 0 && a != i && !trunk[a]) a = m.b[a].parent;
        if (a == i) part.push_back(j);
      }
      parts.push_back(part);
    }
    for (int i = 0; i < nb; i++)  // floating roots outside any trunk (several independent trees)
      if (!trunk[i] && m.b[i].parent < 0) {
        std::vector<int> part;
        for (int j = i; j < nb; j++) {
          int a = j;
          while (a >= 0 && a != i) a = m.b[a].parent;
          if (a == i) part.push_back(j);
        }
        parts.push_back(part);
      }
    return parts;
  };
  if (!any_fixed) floating();
  std::vector<std::vector<int>> parts = collect();
  if (mode == 1 && parts.size() < 2 && want != "1") {
    floating();
    parts = collect();
  }
  const bool forced = want == "1" || want == "2";
  if (parts.size() < 2) return lane_per_world();
  if (mode == 2 && !forced && nb < 14) return lane_per_world();
  // Waves per world group, from a model of a step's length in body weights
  // (a hinge, slide or ball body 4, a free body 8, a body without DOFs 2):
  //  - A wave's own bodies run passes 1-3 in its own instruction stream; wave 0
  //    also runs the trunk's ground contacts.
  //  - Every wave recomputes the floating trunk's pass 1, half a trunk body's
  //    weight per wave.
  //  - Between the two barriers wave 0 runs the trunk's passes 2 and 3 while
  //    the others wait: three quarters of the trunk's weight, on every wave's
  //    clock. A fixed trunk costs nothing (its values are constants).
  //  - The step kernels hold more than 256 registers, one wave per SIMD: with
  //    g <= 4 waves floor(4 / g) workgroups share a CU at a time; 5-8 waves run
  //    one workgroup per CU with waves k and k + 4 on one SIMD. The launch's
  //    workgroups per CU beyond that run in further rounds.
  // A round lasts as long as its busiest SIMD plus the serial trunk section.
  // Measured on MI355X against this model (f32, 1000-step launches): builder
  // humanoid, 32768 worlds, 2 waves 9.74 ms / 4 waves 13.91 ms (model 55 / 78);
  // MJCF humanoid 2 waves 13.01 ms / 4 waves 15.53 ms (65 / 82); MJCF hand,
  // 16384 worlds, 4 waves 7.54 ms / 5 waves 8.12 / 2 waves 11.32 (47 / 53 /
  // 63). Each cap of 8, 4 and 2 is packed to its cheapest assignment
  // (exhaustive over parts -> groups when small, else largest first into the
  // lightest group); the cheapest plan over the caps is kept, ties keeping
  // more waves. PHZ_MAX_GROUPS forces a cap (rounded down to 1, 2, 4 or 8).
  // Ground contact adds 2 per contact point (a box 8 points, other shapes 1);
  // the trunk's contacts run on wave 0 only.
  auto contact_weight = [&](int i) {
    if (!f.contact) return 0.0;
    const int gt = (int)f.geom[(size_t)i * kGeomStride];
    return gt == 0 ? 0.0 : gt == 2 ? 16.0 : 2.0;
  };
  auto weight = [&](int i) {
    const int jt = m.b[i].jtype;
    return (jt == 4 ? 8.0 : jt == 2 ? 2.0 : 4.0) + contact_weight(i);
  };
  double twt = 0, tcontact = 0;
  for (int i = 0; i < nb; i++)
    if (trunk[i]) { twt += weight(i) - contact_weight(i); tcontact += contact_weight(i); }
  if (mode != 2) tcontact = 0;
  const double pass1 = mode == 2 ? 0.5 * twt : 0.0, serial = mode == 2 ? 0.75 * twt : 0.0;
  std::vector<double> pw(parts.size(), 0.0);
  for (size_t k = 0; k < parts.size(); k++) for (int i : parts[k]) pw[k] += weight(i);
  auto cost = [&](const std::vector<double>& load) {
    const int ng = (int)load.size(), cus = std::max(f.cus, 1);
    const long per_cu = std::max(1, (f.wgs + cus - 1) / cus);
    const long conc = ng <= 4 ? 4 / ng : 1;
    const long rounds = (per_cu + conc - 1) / conc;
    double simd[4] = {0, 0, 0, 0};
    for (int k = 0; k < ng; k++) simd[k % 4] += load[k] + pass1 + (k == 0 ? tcontact : 0.0);
    return (double)rounds * (*std::max_element(simd, simd + 4) + serial);
  };
  // Cheapest assignment of the parts to at most cap groups (empty groups
  // dropped, no plan of exactly three groups), as group -> part indices.
  auto pack = [&](int cap) {
    const int n = (int)parts.size();
    std::vector<std::vector<int>> best;
    double best_cost = -1;
    auto consider = [&](const std::vector<int>& owner) {
      std::vector<std::vector<int>> g(cap);
      for (int k = 0; k < n; k++) g[owner[k]].push_back(k);
      std::vector<std::vector<int>> h;
      for (auto& x : g) if (!x.empty()) h.push_back(x);
      if (h.size() == 3 && !lift_guards) return;
      std::vector<double> load;
      for (auto& x : h) { double l = 0; for (int k : x) l += pw[k]; load.push_back(l); }
      const double c = cost(load);
      if (best_cost < 0 || c < best_cost - 1e-9) { best_cost = c; best = h; }
    };
    double combos = 1;
    for (int k = 0; k < n; k++) combos *= cap;
    if (combos <= 2e5) {
      std::vector<int> owner(n, 0);
      for (;;) {
        consider(owner);
        int k = 0;
        while (k < n && ++owner[k] == cap) owner[k++] = 0;
        if (k == n) break;
      }
    } else {
      std::vector<int> order(n);
      for (int k = 0; k < n; k++) order[k] = k;
      std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return pw[a] > pw[b]; });
      std::vector<int> owner(n, 0);
      std::vector<double> load(cap, 0.0);
      for (int k : order) {
        const int j = (int)(std::min_element(load.begin(), load.end()) - load.begin());
        owner[k] = j;
        load[j] += pw[k];
      }
      consider(owner);
      if (best.empty()) {  // three groups: the two-group split of the same greedy order
        std::fill(load.begin(), load.end(), 0.0);
        for (int k : order) {
          const int j = load[0] <= load[1] ? 0 : 1;
          owner[k] = j;
          load[j] += pw[k];
        }
        consider(owner);
      }
    }
    return std::make_pair(best, best_cost);
  };
  auto as_bodies = [&](const std::vector<std::vector<int>>& g) {
    std::vector<std::vector<int>> out;
    for (auto& x : g) {
      std::vector<int> bodies;
      for (int k : x) bodies.insert(bodies.end(), parts[k].begin(), parts[k].end());
      out.push_back(bodies);
    }
    return out;
  };
  // One part per wave, the lightest first (waves 0 and 4 share a SIMD).
  std::vector<int> by_weight(parts.size());
  for (size_t k = 0; k < parts.size(); k++) by_weight[k] = (int)k;
  std::stable_sort(by_weight.begin(), by_weight.end(), [&](int a, int b) { return pw[a] < pw[b]; });
  std::vector<std::vector<int>> unmerged;
  for (int k : by_weight) unmerged.push_back(parts[k]);
  if (const char* e = std::getenv("PHZ_MAX_GROUPS")) {
    // Rounded down to 1, 2, 4 or 8, the caps the planner itself tries (3
    // stays 3 when the guards are lifted, for the host emulation).
    const int want = std::atoi(e);
    const int cap = (lift_guards && want == 3) ? 3 : want >= 8 ? 8 : want >= 4 ? 4 : want >= 2 ? 2 : 1;
    parts = as_bodies(pack(cap).first);
  } else {
    std::vector<std::vector<int>> best;
    double best_cost = -1;
    for (int cap : {8, 4, 2}) {
      auto pc = pack(cap);
      if (!pc.first.empty() && (best_cost < 0 || pc.second < best_cost - 1e-9)) {
        best_cost = pc.second;
        best = pc.first;
      }
    }
    parts = as_bodies(best);
  }
  if (parts.size() == 3 && !lift_guards) return lane_per_world();  // unreachable: pack(2) holds at most two
  if (parts.size() < 2) return lane_per_world();
  // f64: no wave runs two subtrees. Merged f64 plans of the MJCF humanoid (two
  // and three waves) gave NaN or launch-varying results from launches of many
  // steps while the same binaries stepped one step per launch matched the
  // lane-per-world kernel; their kernels spill several hundred bytes per lane.
  // The unmerged plan (one subtree per wave) is taken instead when it has a
  // wave count the planner uses, else one lane per world.
  if (f.f64 && parts.size() < unmerged.size() && !lift_guards) {
    if (unmerged.size() == 2 || unmerged.size() == 4 || (unmerged.size() > 4 && unmerged.size() <= 8)) {
      parts = unmerged;
    } else {
      return lane_per_world();
    }
  }
  pl.mode = mode;
  for (int i = 0; i < nb; i++) if (trunk[i]) pl.trunk.push_back(i);
  for (auto& p : parts) {
    std::sort(p.begin(), p.end());
    pl.groups.push_back(p);
  }
  return pl;
}

// Lanes per world of the step kernel. A launch of few worlds leaves most SIMDs
// idle (4096 worlds are 64 waves on 1024 SIMDs), and a one-lane kernel then
// runs at the latency of its own instruction stream: such launches can give
// each world 2 or 4 lanes that split the revolute joints' sincos (see
// trig_prepass in phz_device.h). Every lane still runs the rest of the step,
// so the split pays only where the sincos is a large share of it. Measured on
// MI355X (event time per 200- or 100-step span against PHZ_LANES=1):
//  - two revolute joints (the double pendulum, 2 lanes): 7-15% faster at
//    1024-32768 worlds in f64 and in f32, where the split waves fit one per
//    SIMD;
//  - chain7 (4 lanes): f32, whose sincos is the hardware's, 6-17% slower at
//    every size from 1024 to 16384 worlds; f64 (table sincos) 4-6% faster up
//    to 4096 worlds (one split wave per CU), even at 8192, 9% slower at 16384.
// So 2 lanes go wherever the split waves fit one per SIMD, 4 lanes only to f64
// kernels whose split waves fit one per CU. Contact, partitioned plans and
// trees with fewer than two revolute joints keep one lane. PHZ_LANES=1 turns
// the split off; PHZ_LANES=2 or 4 (any value above 1) splits wherever the
// model allows it, whatever the size and precision (tests, tuning).
int lanes_per_world(const ModelD& m, const Features& f, const Plan& pl) {
  bool forced = false;
  if (const char* e = std::getenv("PHZ_LANES")) {
    if (std::atoi(e) <= 1) return 1;
    forced = true;
  }
  if (pl.mode != 0 || pl.groups.size() != 1 || f.contact) return 1;
  int nrev = 0;
  for (int i = 0; i < m.nb; i++) nrev += m.b[i].jtype == 0;
  if (nrev < 2) return 1;
  const int L = nrev == 2 ? 2 : 4;
  if (forced) return L;
  const long waves = (long)std::max(f.wgs, 1) * L, cus = std::max(f.cus, 1);
  if (L == 2) return waves <= 4 * cus ? 2 : 1;
  return f.f64 && waves <= cus ? 4 : 1;
}

// Whether body i's joint-space inertia D = S^T I_A S + (armature + dt
// damping) 1 can never give an LDL pivot below the singular test's 1e-20
// (aba.rs:210 skips such a body), for any configuration: I_A is the body's
// own spatial inertia plus its children's articulated inertias, which are
// positive semidefinite, so every pivot of D is at least the least pivot
// bound of D0 = S^T I_i S + (armature + dt damping) 1, and D0 - tau 1 >= 0
// (a Cholesky factorisation that succeeds) bounds every pivot by tau. tau
// adds to 1e-20 a rounding margin of 1e3 unit roundoffs times the trace of
// an upper bound of the subtree's composite inertia about the joint
// (sum of tr Ic_j + m_j (3 + 2 R_j^2), R_j the joint-to-COM distance along
// the fixed link offsets). A slide or free joint inside the subtree leaves
// R unbounded: no bound then. With the bound the kernel drops the test and
// the branch around the parent update.
bool pivots_bounded(const ModelD& m, int i, bool f64) {
  const int nb = m.nb;
  // Distance bound from body i's joint to each descendant's frame origin.
  std::vector<double> reach(nb, -1.0);
  reach[i] = 0.0;
  double trace = 0.0;
  for (int j = i; j < nb; j++) {
    if (j != i) {
      const int pj = m.b[j].parent;
      if (pj < 0 || reach[pj] < 0.0) continue;
      if (m.b[j].jtype == 1 || m.b[j].jtype == 4) return false;
      const double* t = m.b[j].ptj_pos;
      reach[j] = reach[pj] + std::sqrt(t[0] * t[0] + t[1] * t[1] + t[2] * t[2]);
    }
    const BodyD& b = m.b[j];
    const double rc = reach[j] + std::sqrt(b.com[0] * b.com[0] + b.com[1] * b.com[1] + b.com[2] * b.com[2]);
    trace += b.inertia[0] + b.inertia[1] + b.inertia[2] + b.mass * (3.0 + 2.0 * rc * rc);
  }
  const double eps = f64 ? 0x1p-53 : 0x1p-24;
  const double tau = 1e-20 + 1e3 * eps * trace;
  const BodyD& b = m.b[i];
  const double cx = b.com[0], cy = b.com[1], cz = b.com[2], mm = b.mass;
  const double c2 = cx * cx + cy * cy + cz * cz;
  const double Ic[9] = {b.inertia[0], b.inertia[3], b.inertia[4], b.inertia[3], b.inertia[1],
                        b.inertia[5], b.inertia[4], b.inertia[5], b.inertia[2]};
  const double c[3] = {cx, cy, cz};
  double Is[6][6] = {};  // spatial inertia at the body frame, angular rows first
  for (int r = 0; r < 3; r++)
    for (int k = 0; k < 3; k++) Is[r][k] = Ic[r * 3 + k] + mm * ((r == k ? c2 : 0.0) - c[r] * c[k]);
  const double X[9] = {0, -cz, cy, cz, 0, -cx, -cy, cx, 0};  // [c]x
  for (int r = 0; r < 3; r++)
    for (int k = 0; k < 3; k++) {
      Is[r][3 + k] = mm * X[r * 3 + k];
      Is[3 + k][r] = mm * X[r * 3 + k];
    }
  for (int r = 0; r < 3; r++) Is[3 + r][3 + r] = mm;
  int nd = 0;
  double S[6][6] = {};  // columns of the motion subspace
  if (b.jtype == 0 || b.jtype == 1) {
    for (int k = 0; k < 3; k++) S[(b.jtype == 0 ? 0 : 3) + k][0] = b.axis[k];
    nd = 1;
  } else if (b.jtype == 3) {
    for (int k = 0; k < 3; k++) S[k][k] = 1.0;
    nd = 3;
  } else if (b.jtype == 4) {
    for (int k = 0; k < 6; k++) S[k][k] = 1.0;
    nd = 6;
  } else {
    return true;  // a fixed joint has no pivots
  }
  double D[6][6];
  for (int r = 0; r < nd; r++)
    for (int k = 0; k < nd; k++) {
      double acc = 0.0;
      for (int a = 0; a < 6; a++)
        for (int e = 0; e < 6; e++) acc += S[a][r] * Is[a][e] * S[e][k];
      D[r][k] = acc + (r == k ? b.armature + m.dt * b.damping - tau : 0.0);
    }
  for (int k = 0; k < nd; k++) {  // Cholesky of D0 - tau 1
    for (int t = 0; t < k; t++) D[k][k] -= D[k][t] * D[k][t];
    if (!(D[k][k] > 0.0)) return false;
    D[k][k] = std::sqrt(D[k][k]);
    for (int r = k + 1; r < nd; r++) {
      for (int t = 0; t < k; t++) D[r][k] -= D[r][t] * D[k][t];
      D[r][k] /= D[k][k];
    }
  }
  return true;
}

std::string gen_model(const ModelD& m, const Features& f) {
  const int nb = m.nb;
  // Rigid spatial inertia [[Ic + m cx cx^T, m cx], [m cx^T, m 1]] as symmetric blocks.
  std::vector<double> A(nb * 6), B(nb * 9), C(nb * 6), iinv(nb * 6), K(nb * 9), K2(nb * 9);
  std::vector<int> ptj_id(nb), need_world(nb, 0);
  int maxnd = 0;
  for (int i = 0; i < nb; i++) {
    const BodyD& b = m.b[i];
    maxnd = std::max(maxnd, ndof_of(b.jtype));
    const double mm = b.mass, cx = b.com[0], cy = b.com[1], cz = b.com[2];
    double X[9] = {0, -cz, cy, cz, 0, -cx, -cy, cx, 0};
    double XXt[9];
    for (int r = 0; r < 3; r++)
      for (int c = 0; c < 3; c++) XXt[r * 3 + c] = X[r * 3] * X[c * 3] + X[r * 3 + 1] * X[c * 3 + 1] + X[r * 3 + 2] * X[c * 3 + 2];
    double Ic[9] = {b.inertia[0], b.inertia[3], b.inertia[4], b.inertia[3], b.inertia[1],
                    b.inertia[5], b.inertia[4], b.inertia[5], b.inertia[2]};
    const int up[6][2] = {{0, 0}, {0, 1}, {0, 2}, {1, 1}, {1, 2}, {2, 2}};
    for (int k = 0; k < 6; k++) {
      const int r = up[k][0], c = up[k][1];
      A[i * 6 + k] = Ic[r * 3 + c] + XXt[r * 3 + c] * mm;
      C[i * 6 + k] = r == c ? mm : 0.0;
    }
    for (int k = 0; k < 9; k++) B[i * 9 + k] = X[k] * mm;
    // Cofactor inverse of the COM inertia (phyz_kernels.cu:545-560).
    const double xx = b.inertia[0], yy = b.inertia[1], zz = b.inertia[2], xy = b.inertia[3], xz = b.inertia[4],
                 yz = b.inertia[5];
    const double c00 = yy * zz - yz * yz, c01 = xz * yz - xy * zz, c02 = xy * yz - xz * yy;
    const double det = xx * c00 + xy * c01 + xz * c02;
    if (std::fabs(det) < 1e-20) {
      for (int k = 0; k < 6; k++) iinv[i * 6 + k] = 0.0;
    } else {
      const double c11 = xx * zz - xz * xz, c12 = xy * xz - xx * yz, c22 = xx * yy - xy * xy, inv = 1.0 / det;
      const double v[6] = {inv * c00, inv * c01, inv * c02, inv * c11, inv * c12, inv * c22};
      for (int k = 0; k < 6; k++) iinv[i * 6 + k] = v[k];
    }
    // Rodrigues at -q (joint.rs:255-262): E_J = I + K s + K^2 (1 - c), s = sin(-q), c = cos(-q).
    const double ax = b.axis[0], ay = b.axis[1], az = b.axis[2];
    const double k9[9] = {0, -az, ay, az, 0, -ax, -ay, ax, 0};
    for (int k = 0; k < 9; k++) K[i * 9 + k] = k9[k];
    for (int r = 0; r < 3; r++)
      for (int c = 0; c < 3; c++)
        K2[i * 9 + r * 3 + c] = k9[r * 3] * k9[c] + k9[r * 3 + 1] * k9[3 + c] + k9[r * 3 + 2] * k9[6 + c];
    const double id[9] = {1, 0, 0, 0, 1, 0, 0, 0, 1};
    ptj_id[i] = 1;
    for (int k = 0; k < 9; k++) if (b.ptj_rot[k] != id[k]) ptj_id[i] = 0;
  }
  if (f.contact) {
    for (int i = 0; i < nb; i++)
      if ((int)f.geom[i * kGeomStride] != 0)
        for (int j = i; j >= 0; j = m.b[j].parent) need_world[j] = 1;
    if (f.plane_body >= 0)
      for (int j = f.plane_body; j >= 0; j = m.b[j].parent) need_world[j] = 1;
  }

  const Plan pl = plan_partition(m, f);
  const int ng = (int)pl.groups.size();
  int maxg = 1;
  for (auto& g : pl.groups) maxg = std::max(maxg, (int)g.size());
  std::vector<int> is_trunk(nb, 0), owner(nb, 0);
  for (int i : pl.trunk) is_trunk[i] = 1;
  for (int g = 0; g < ng; g++) for (int i : pl.groups[g]) owner[i] = g;
  std::vector<int> dof_group(m.nv, 0), dof_owner(m.nv, 0), tdof(m.nv, -1);
  int ntd = 0;
  for (int i = 0; i < nb; i++)
    for (int k = 0; k < ndof_of(m.b[i].jtype); k++) {
      const int j = m.b[i].voff + k;
      dof_group[j] = is_trunk[i] ? -1 : owner[i];
      dof_owner[j] = is_trunk[i] ? 0 : owner[i];
      if (is_trunk[i]) tdof[j] = ntd++;
    }
  // LDS slots (floating trunk): 27 per (group, trunk body) pair through which
  // a group other than 0 hands its subtrees' summed contributions to group 0,
  // 6 per trunk body whose acceleration other groups read, 2 per trunk DOF.
  // A group's subtree roots under one trunk body share the slot: pass 2 runs
  // them in decreasing body order, so the highest-numbered root starts the sum
  // (contrib_first) and the lowest stores it (contrib_put).
  std::vector<int> slot_contrib(nb, -1), slot_acc(nb, -1), contrib_first(nb, 0), contrib_put(nb, 0);
  int nslot = 0;
  if (pl.mode == 2) {
    std::map<std::pair<int, int>, std::vector<int>> roots;  // (group, trunk parent) -> roots, ascending
    for (int i = 0; i < nb; i++)
      if (!is_trunk[i] && m.b[i].parent >= 0 && is_trunk[m.b[i].parent] && owner[i] != 0)
        roots[{owner[i], m.b[i].parent}].push_back(i);
    for (auto& kv : roots) {
      for (int i : kv.second) slot_contrib[i] = nslot;
      nslot += 27;
      contrib_first[kv.second.back()] = 1;
      contrib_put[kv.second.front()] = 1;
      if (slot_acc[kv.first.second] < 0) slot_acc[kv.first.second] = -2;
    }
    for (int i = 0; i < nb; i++) if (slot_acc[i] == -2) { slot_acc[i] = nslot; nslot += 6; }
  }
  const int slot_state = nslot;
  if (pl.mode == 2) nslot += 2 * ntd;
  // Control noise of a floating-trunk plan: one wave other than wave 0 (the
  // one with the fewest bodies) draws the next step's values for every DOF
  // between the two barriers, while wave 0 runs the trunk, and hands them to
  // the other waves through LDS (NOISE_G; -1: each wave draws for itself).
  const int nn = f.noise ? (int)f.noise_dofs.size() : 0;
  int noise_g = -1;
  if (pl.mode == 2 && nn > 0 && ng > 1) {
    noise_g = 1;
    for (int g = 2; g < ng; g++)
      if (pl.groups[g].size() < pl.groups[noise_g].size()) noise_g = g;
  }
  const int slot_noise = nslot;
  if (noise_g >= 0) nslot += nn;

  std::ostringstream o;
  const int npd = f.npd;
  o << "struct Model {\n";
  o << "  static constexpr int NB = " << nb << ", NQ = " << m.nq << ", NV = " << m.nv
    << ", MAXD = " << std::max(maxnd, 1) << ";\n";
  o << "  static constexpr int PMODE = " << pl.mode << ", NG = " << ng << ", NTRUNK = " << pl.trunk.size()
    << ", MAXG = " << maxg << ", NSLOT = " << nslot << ", slot_state = " << slot_state << ";\n";
  o << "  static constexpr int NOISE_G = " << noise_g << ", slot_noise = " << slot_noise << ";\n";
  {
    std::vector<int> rev;
    for (int i = 0; i < nb; i++) if (m.b[i].jtype == 0) rev.push_back(i);
    const int nr = std::max((int)rev.size(), 1);
    o << "  static constexpr int LANES = " << lanes_per_world(m, f, pl) << ", NREV = " << rev.size() << ";\n";
    o << "  static constexpr int rev_body[" << nr << "] = "
      << arr1(nr, [&](int k) { return std::to_string(rev.empty() ? 0 : rev[k]); }) << ";\n";
  }
  const int nta = std::max((int)pl.trunk.size(), 1);
  o << "  static constexpr int tlist[" << nta << "] = "
    << arr1(nta, [&](int k) { return std::to_string(pl.trunk.empty() ? 0 : pl.trunk[k]); }) << ";\n";
  o << "  static constexpr int glen[" << ng << "] = " << arr1(ng, [&](int g) { return std::to_string(pl.groups[g].size()); })
    << ";\n";
  o << "  static constexpr int glist[" << ng << "][" << maxg << "] = "
    << arr2(ng, maxg, [&](int g, int k) { return std::to_string(k < (int)pl.groups[g].size() ? pl.groups[g][k] : 0); })
    << ";\n";
  o << "  static constexpr int dof_group[" << m.nv << "] = " << arr1(m.nv, [&](int j) { return std::to_string(dof_group[j]); })
    << ";\n";
  o << "  static constexpr int dof_owner[" << m.nv << "] = " << arr1(m.nv, [&](int j) { return std::to_string(dof_owner[j]); })
    << ";\n";
  o << "  static constexpr int tdof[" << m.nv << "] = " << arr1(m.nv, [&](int j) { return std::to_string(tdof[j]); })
    << ";\n";
  o << "  static constexpr bool HAS_CONTACT = " << (f.contact ? "true" : "false") << ";\n";
  o << "  static constexpr int CMODE = " << (f.contact ? f.cmode : 0) << ", SWEEPS = " << f.sweeps
    << ", PLANE = " << (f.contact ? f.plane_body : -1) << ";\n";
  o << "  static constexpr bool HAS_HF = " << (f.contact && f.hf_nx > 0 ? "true" : "false") << ";\n";
  o << "  static constexpr double c_rest = " << num(f.prm[0]) << ", c_rest_v = " << num(f.prm[1]) << ", c_erp = "
    << num(f.prm[2]) << ", c_margin = " << num(f.prm[3]) << ";\n";
  {
    // SolImp's clamps (phyz_kernels.cu:595-607), evaluated once here.
    const double dmin = std::clamp(f.prm[4], 1e-4, 1.0 - 1e-9), dmax = std::clamp(f.prm[5], 1e-4, 1.0 - 1e-9);
    const double mid = std::clamp(f.prm[7], 1e-6, 1.0 - 1e-6), pw = std::max(f.prm[8], 1.0);
    o << "  static constexpr double c_dmin = " << num(dmin) << ", c_dmax = " << num(dmax) << ", c_width = "
      << num(f.prm[6]) << ", c_mid = " << num(mid) << ", c_power = " << num(pw) << ";\n";
    o << "  static constexpr double c_mid_pow = " << num(std::pow(mid, pw - 1.0)) << ", c_omid_pow = "
      << num(std::pow(1.0 - mid, pw - 1.0)) << ";\n";
  }
  o << "  static constexpr double plane_offset = " << num(f.plane[0]) << ", plane_depth = " << num(f.plane[1])
    << ", plane_hx = " << num(f.plane[2]) << ", plane_hy = " << num(f.plane[3]) << ";\n";
  o << "  static constexpr int NPD = " << npd << ", NNOISE = " << nn << ", noise_dist = " << f.dist << ";\n";
  o << "  static constexpr double dt = " << num(m.dt) << ";\n";
  o << "  static constexpr double gravity[3] = " << arr1(3, [&](int k) { return num(m.g[k]); }) << ";\n";
  o << "  static constexpr double ground_h = " << num(f.ground_h) << ", mu = " << num(f.mu) << ";\n";
  o << "  static constexpr double noise_a = " << num(f.a) << ", noise_b = " << num(f.b) << ";\n";
  auto ib = [&](const char* name, auto get) {
    o << "  static constexpr int " << name << "[" << nb << "] = " << arr1(nb, [&](int i) { return std::to_string(get(i)); }) << ";\n";
  };
  auto bb = [&](const char* name, auto get) {
    o << "  static constexpr bool " << name << "[" << nb << "] = "
      << arr1(nb, [&](int i) { return std::string(get(i) ? "true" : "false"); }) << ";\n";
  };
  auto db = [&](const char* name, auto get) {
    o << "  static constexpr double " << name << "[" << nb << "] = " << arr1(nb, [&](int i) { return num(get(i)); }) << ";\n";
  };
  auto d2 = [&](const char* name, int w, auto get) {
    o << "  static constexpr double " << name << "[" << nb << "][" << w << "] = "
      << arr2(nb, w, [&](int i, int k) { return num(get(i, k)); }) << ";\n";
  };
  ib("parent", [&](int i) { return m.b[i].parent; });
  bb("is_trunk", [&](int i) { return is_trunk[i]; });
  ib("slot_contrib", [&](int i) { return slot_contrib[i]; });
  ib("slot_acc", [&](int i) { return slot_acc[i]; });
  bb("contrib_first", [&](int i) { return contrib_first[i]; });
  bb("contrib_put", [&](int i) { return contrib_put[i]; });
  ib("jtype", [&](int i) { return m.b[i].jtype; });
  ib("qoff", [&](int i) { return m.b[i].qoff; });
  ib("voff", [&](int i) { return m.b[i].voff; });
  bb("ptj_identity", [&](int i) { return ptj_id[i]; });
  bb("need_world", [&](int i) { return need_world[i]; });
  d2("ptj_rot", 9, [&](int i, int k) { return m.b[i].ptj_rot[k]; });
  d2("ptj_pos", 3, [&](int i, int k) { return m.b[i].ptj_pos[k]; });
  d2("axis", 3, [&](int i, int k) { return m.b[i].axis[k]; });
  d2("rev_k", 9, [&](int i, int k) { return K[i * 9 + k]; });
  d2("rev_k2", 9, [&](int i, int k) { return K2[i * 9 + k]; });
  db("damping", [&](int i) { return m.b[i].damping; });
  db("stiffness", [&](int i) { return m.b[i].stiffness; });
  db("spring_ref", [&](int i) { return m.b[i].spring_ref; });
  db("armature", [&](int i) { return m.b[i].armature; });
  // The component of a one-DOF joint's axis along which I_a S = 0 makes a
  // row and column of I_a vanish (see body_solve in phz_device.h): a
  // coordinate axis (one entry +-1), no armature and no damping, so that
  // D = S^T I_A S exactly. -1 otherwise.
  ib("zero_axis", [&](int i) {
    const BodyD& b = m.b[i];
    if ((b.jtype != 0 && b.jtype != 1) || b.armature != 0.0 || b.damping != 0.0) return -1;
    int k = -1, nz = 0;
    for (int c = 0; c < 3; c++)
      if (b.axis[c] != 0.0) { nz++; k = c; }
    if (nz != 1 || std::fabs(b.axis[k]) != 1.0) return -1;
    return b.jtype == 0 ? k : 3 + k;
  });
  // A revolute joint about a coordinate axis with no rotation from the
  // parent (X.E a rotation about that axis, see sym_xtix): the axis, else -1.
  ib("rot_axis", [&](int i) {
    const BodyD& b = m.b[i];
    if (b.jtype != 0 || !ptj_id[i]) return -1;
    int k = -1, nz = 0;
    for (int c = 0; c < 3; c++)
      if (b.axis[c] != 0.0) { nz++; k = c; }
    return nz == 1 && std::fabs(b.axis[k]) == 1.0 ? k : -1;
  });
  // Not for an f64 kernel of several waves: the MJCF humanoid's four-wave
  // f64 kernel without the branch returned non-finite worlds on gfx950 where
  // its host emulation (ASan, TSan, finite-math -O3) and the oracle agree.
  // PHZ_PIVOT_BOUND=0 keeps the test everywhere (tuning, tests). A host-only
  // sim with PHZ_HOST_LIFT_PIVOT=1 generates the refused kernel (for the host
  // emulation, as PHZ_HOST_LIFT_GUARDS does for the refused plans).
  const char* lift_env = std::getenv("PHZ_HOST_LIFT_PIVOT");
  const bool multi_f64 = f.f64 && pl.groups.size() > 1 && !(f.host_only && lift_env && lift_env[0] == '1');
  const char* pb_env = std::getenv("PHZ_PIVOT_BOUND");
  const bool pb_off = pb_env && pb_env[0] == '0';
  bb("piv_ok", [&](int i) { return !multi_f64 && !pb_off && pivots_bounded(m, i, f.f64); });
  db("mass", [&](int i) { return m.b[i].mass; });
  d2("com", 3, [&](int i, int k) { return m.b[i].com[k]; });
  d2("inA", 6, [&](int i, int k) { return A[i * 6 + k]; });
  d2("inB", 9, [&](int i, int k) { return B[i * 9 + k]; });
  d2("inC", 6, [&](int i, int k) { return C[i * 6 + k]; });
  d2("iinv", 6, [&](int i, int k) { return iinv[i * 6 + k]; });
  auto g = [&](int i, int s) { return f.contact ? f.geom[i * kGeomStride + s] : 0.0; };
  ib("gtype", [&](int i) { return f.contact ? (int)g(i, 0) : 0; });
  d2("gp", 6, [&](int i, int k) { return g(i, 1 + k); });
  db("gk", [&](int i) { return g(i, 8); });
  db("gd", [&](int i) { return g(i, 9); });
  d2("gopos", 3, [&](int i, int k) { return g(i, 10 + k); });
  d2("gorot", 9, [&](int i, int k) { return f.contact ? g(i, 13 + k) : (k % 4 == 0 ? 1.0 : 0.0); });
  bb("gskip", [&](int i) { return f.contact && g(i, 7) != 0.0; });
  const int npa = std::max(npd, 1), nna = std::max(nn, 1);
  auto pdv = [&](int d, int s) { return npd ? f.pd[d * kPdStride + s] : 0.0; };
  o << "  static constexpr int pd_q[" << npa << "] = " << arr1(npa, [&](int d) { return std::to_string((int)pdv(d, 0)); }) << ";\n";
  o << "  static constexpr int pd_v[" << npa << "] = " << arr1(npa, [&](int d) { return std::to_string((int)pdv(d, 1)); }) << ";\n";
  o << "  static constexpr double pd_kp[" << npa << "] = " << arr1(npa, [&](int d) { return num(pdv(d, 2)); }) << ";\n";
  o << "  static constexpr double pd_kd[" << npa << "] = " << arr1(npa, [&](int d) { return num(pdv(d, 3)); }) << ";\n";
  o << "  static constexpr double pd_max[" << npa << "] = " << arr1(npa, [&](int d) { return num(pdv(d, 4)); }) << ";\n";
  o << "  static constexpr int noise_dof[" << nna << "] = "
    << arr1(nna, [&](int k) { return std::to_string(nn ? f.noise_dofs[k] : 0); }) << ";\n";
  // Actuators and joint limits / dry friction.
  const int nu = (int)f.acts.size(), nctrl = nu ? nu : m.nv, nua = std::max(nu, 1);
  const Features::Act act0;
  auto act = [&](int a) -> const Features::Act& { return nu ? f.acts[a] : act0; };
  o << "  static constexpr int NU = " << nu << ", NCTRL = " << nctrl << ";\n";
  auto ia = [&](const char* name, auto get) {
    o << "  static constexpr int " << name << "[" << nua << "] = " << arr1(nua, [&](int a) { return std::to_string(get(act(a))); }) << ";\n";
  };
  auto ba = [&](const char* name, auto get) {
    o << "  static constexpr bool " << name << "[" << nua << "] = "
      << arr1(nua, [&](int a) { return std::string(get(act(a)) ? "true" : "false"); }) << ";\n";
  };
  auto da = [&](const char* name, auto get) {
    o << "  static constexpr double " << name << "[" << nua << "] = " << arr1(nua, [&](int a) { return num(get(act(a))); }) << ";\n";
  };
  ia("act_v", [](const Features::Act& x) { return x.v; });
  ia("act_q", [](const Features::Act& x) { return x.q; });
  da("act_gear", [](const Features::Act& x) { return x.gear; });
  da("act_gain", [](const Features::Act& x) { return x.gain; });
  da("act_bq", [](const Features::Act& x) { return x.bq; });
  da("act_bv", [](const Features::Act& x) { return x.bv; });
  ba("act_cr", [](const Features::Act& x) { return x.cr; });
  da("act_clo", [](const Features::Act& x) { return x.clo; });
  da("act_chi", [](const Features::Act& x) { return x.chi; });
  ba("act_fr", [](const Features::Act& x) { return x.fr; });
  da("act_flo", [](const Features::Act& x) { return x.flo; });
  da("act_fhi", [](const Features::Act& x) { return x.fhi; });
  o << "  static constexpr int ctrl_group[" << nctrl << "] = "
    << arr1(nctrl, [&](int c) { return std::to_string(dof_group[nu ? f.acts[c].v : c]); }) << ";\n";
  o << "  static constexpr int ctrl_owner[" << nctrl << "] = "
    << arr1(nctrl, [&](int c) { return std::to_string(dof_owner[nu ? f.acts[c].v : c]); }) << ";\n";
  const bool jt = !f.jterms.empty();
  bb("lim_on", [&](int i) { return jt && f.jterms[i].limited && ndof_of(m.b[i].jtype) == 1; });
  db("lim_lo", [&](int i) { return jt ? f.jterms[i].lo : 0.0; });
  db("lim_hi", [&](int i) { return jt ? f.jterms[i].hi : 0.0; });
  db("lim_k", [&](int i) { return jt ? f.jterms[i].k : 0.0; });
  db("lim_d", [&](int i) { return jt ? f.jterms[i].d : 0.0; });
  db("floss", [&](int i) { return jt && ndof_of(m.b[i].jtype) == 1 ? f.jterms[i].floss : 0.0; });
  o << "};\n";
  return o.str();
}

// One workgroup = NG waves over the same 64 worlds; wave g runs group g.
// two_waves: ask the compiler for two resident waves per SIMD (at most 256
// registers per lane, spilling what does not fit).
std::string gen_source(const ModelD& m, const Features& f, bool f64, int* ngroups, int* lanes,
                       bool two_waves = false) {
  const Plan pl = plan_partition(m, f);
  const int ng = (int)pl.groups.size();
  *ngroups = ng;
  *lanes = lanes_per_world(m, f, pl);
  const std::string T = f64 ? "double" : "float";
  std::string s = kDeviceSrc;
  s += "\n// ---- model-specialised instantiation ----\n";
  s += gen_model(m, f);
  s += "extern \"C\" __global__ void __launch_bounds__(" + std::to_string(64 * ng) + ")" +
       (two_waves ? " __attribute__((amdgpu_waves_per_eu(2, 2)))" : "") + " phz_step(phz::StepArgs a) {\n";
  s += "  __shared__ " + T + " lds[(Model::NSLOT > 0 ? Model::NSLOT : 1) * 64];\n";
  s += "  const int g = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);\n";
  s += "  const int lane = threadIdx.x & 63;\n";
  s += "  switch (g) {\n";
  for (int g = 0; g < ng; g++)
    s += "    case " + std::to_string(g) + ": phz::run_group<Model, " + T + ", " + std::to_string(g) + ">(a, lane, lds); break;\n";
  s += "    default: break;\n  }\n}\n";
  return s;
}

// ── hiprtc compile with an in-process and on-disk cache ────────────────────
uint64_t fnv1a(const std::string& s, uint64_t h = 1469598103934665603ull) {
  for (unsigned char c : s) { h ^= c; h *= 1099511628211ull; }
  return h;
}
// Step, observation and policy kernels assume finite values
// (-ffinite-math-only), which lets products with the model's constant zeros
// fold away: about 45% fewer instructions. The one exception is the f64
// impulse-mode step kernel, built with IEEE semantics: with the finite-values
// assumption the f64 terrain + impulse ant computed wrong accelerations
// (relative error 1e5, the same on every launch) at -O3 on gfx950, while the
// identical source was right without it, right at -O1, right on the host
// under the same flags and sanitizer-clean there. IEEE builds are not the
// default for f64 because several other f64 kernels built that way gave
// results that changed from launch to launch on identical inputs (finite-math
// builds of the same sources are bit-reproducible and match the oracle).
//
// Reassoc is the finite-math build with PHZ_REASSOC defined: the spatial
// algebra and the articulated-body passes of phz_device.h may then be
// reassociated (sums folded into FMAs, products with the model's constants
// regrouped), 5-8% fewer VALU instructions per step. The random stream and the
// closed-form sines, cosines and logarithms keep their written order either
// way. A step kernel that spills under Reassoc is built Finite instead.
enum class Build { Finite, Ieee, Reassoc };
const std::vector<std::string>& compile_options(Build b) {
  static const std::vector<std::string> finite_opts = {
      "--offload-arch=gfx950", "-O3", "-std=c++17", "-ffinite-math-only", "-fno-signed-zeros",
      // Packed FP32 (v_pk_*_f32) stays off in every kernel of this library.
      "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
      "-Rpass-analysis=kernel-resource-usage"};
  static const std::vector<std::string> reassoc_opts = [] {
    std::vector<std::string> o = finite_opts;
    o.push_back("-DPHZ_REASSOC=1");
    return o;
  }();
  static const std::vector<std::string> ieee_opts = {
      "--offload-arch=gfx950", "-O3", "-std=c++17", "-fno-signed-zeros",
      "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
      "-Rpass-analysis=kernel-resource-usage"};
  return b == Build::Ieee ? ieee_opts : (b == Build::Reassoc ? reassoc_opts : finite_opts);
}
std::string cache_dir() {
  if (const char* e = std::getenv("PHZ_KERNEL_CACHE")) return e;
  Dl_info info;
  if (dladdr((void*)&cache_dir, &info) && info.dli_fname) {
    std::string p = info.dli_fname;
    auto slash = p.rfind('/');
    std::string d = (slash == std::string::npos ? std::string(".") : p.substr(0, slash)) + "/_kcache";
    mkdir(d.c_str(), 0755);
    if (access(d.c_str(), W_OK) == 0) return d;
  }
  std::string d = "/tmp/phyz_amd_kcache";
  mkdir(d.c_str(), 0755);
  return d;
}

struct CodeObject {
  std::vector<char> code;
  std::string log;
};
std::mutex g_compile_mu;
std::unordered_map<uint64_t, std::shared_ptr<CodeObject>> g_code_cache;

// The compiler that hiprtc calls resolve to. A process that loaded another
// ROCm's libhiprtc.so.7 first (a Python wheel may bundle one under the same
// soname) compiles with that one, which generates different code for the same
// source: the cache key includes it, so code objects from two compilers never
// meet in one process.
const std::string& compiler_id() {
  static const std::string id = [] {
    int major = 0, minor = 0;
    std::string s = hiprtcVersion(&major, &minor) == HIPRTC_SUCCESS ? fmt("hiprtc %d.%d", major, minor) : "hiprtc ?";
    Dl_info info;
    if (dladdr((void*)&hiprtcCompileProgram, &info) && info.dli_fname) s += std::string(" ") + info.dli_fname;
    return s;
  }();
  return id;
}

std::shared_ptr<CodeObject> compile_source(const std::string& src, Build build, std::string& err) {
  std::string key_text = src;
  for (const auto& o : compile_options(build)) key_text += "\n" + o;
  key_text += "\n" + compiler_id();
  const uint64_t key = fnv1a(key_text);
  std::lock_guard<std::mutex> lk(g_compile_mu);
  auto it = g_code_cache.find(key);
  if (it != g_code_cache.end()) return it->second;
  const std::string dir = cache_dir();
  const std::string path = dir + fmt("/%016llx.co", (unsigned long long)key);
  // PHZ_KERNEL_REBUILD=1 ignores cached code objects (the build step uses it).
  const char* rebuild = std::getenv("PHZ_KERNEL_REBUILD");
  if (!(rebuild && rebuild[0] == '1')) {
    std::ifstream in(path, std::ios::binary);
    if (in) {
      auto co = std::make_shared<CodeObject>();
      co->code.assign(std::istreambuf_iterator<char>(in), std::istreambuf_iterator<char>());
      std::ifstream lg(path + ".log");
      if (lg) co->log.assign(std::istreambuf_iterator<char>(lg), std::istreambuf_iterator<char>());
      if (!co->code.empty()) { g_code_cache[key] = co; return co; }
    }
  }
  hiprtcProgram prog;
  if (hiprtcCreateProgram(&prog, src.c_str(), "phz_step.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS) {
    err = "hiprtcCreateProgram failed";
    return nullptr;
  }
  std::vector<const char*> opts;
  for (const auto& o : compile_options(build)) opts.push_back(o.c_str());
  hiprtcResult rc = hiprtcCompileProgram(prog, (int)opts.size(), opts.data());
  size_t log_size = 0;
  hiprtcGetProgramLogSize(prog, &log_size);
  std::string log(log_size, '\0');
  if (log_size) hiprtcGetProgramLog(prog, &log[0]);
  if (rc != HIPRTC_SUCCESS) {
    err = std::string("hiprtc compile failed: ") + hiprtcGetErrorString(rc) + "\n" + log;
    hiprtcDestroyProgram(&prog);
    return nullptr;
  }
  size_t code_size = 0;
  hiprtcGetCodeSize(prog, &code_size);
  auto co = std::make_shared<CodeObject>();
  co->code.resize(code_size);
  hiprtcGetCode(prog, co->code.data());
  co->log = log;
  hiprtcDestroyProgram(&prog);
  const std::string tmp = path + fmt(".tmp%d", (int)getpid());
  {
    std::ofstream out(tmp, std::ios::binary);
    out.write(co->code.data(), (std::streamsize)co->code.size());
  }
  std::rename(tmp.c_str(), path.c_str());
  {
    std::ofstream out(path + ".log");
    out << co->log;
  }
  g_code_cache[key] = co;
  return co;
}

// Parse "VGPRs: N", "AGPRs: N", "SGPRs: N", "ScratchSize [bytes/lane]: N" from the remarks.
int64_t remark_value(const std::string& log, const char* label) {
  auto p = log.find(label);
  if (p == std::string::npos) return -1;
  p += std::strlen(label);
  while (p < log.size() && (log[p] == ' ' || log[p] == ':')) p++;
  return std::strtoll(log.c_str() + p, nullptr, 10);
}

struct StepArgs {  // must match phz::StepArgs in phz_device.h
  void* q;
  void* v;
  void* ctrl;
  void* qdd;
  const void* targets;
  uint64_t* rng;
  void* contact_rows;
  void* ext;
  void* imp;
  const void* hf;
  double hf_ox, hf_oy, hf_oz, hf_cell;
  int hf_nx, hf_ny;
  int nworld;
  int stride;
  int nsteps;
  int write_contacts;
};

int env_int(const char* name, int def) {
  const char* e = std::getenv(name);
  return e ? std::atoi(e) : def;
}

// ── control loop: policy spec, code generation, weight layout ───────────────
// PolicySpec (crates/phyz-gpu/src/policy_pipeline.rs:300-416), flat.
struct PolicyD {
  int n_in = 0, hidden = 0, n_out = 0, history = 0;
  std::vector<double> ops;    // n_in x 4, ObsOp::pack rows
  std::vector<double> aux;    // ComOverSupport payloads
  std::vector<double> noise;  // n_in
  std::vector<double> clamp;  // n_out (the scalar broadcast when no per-slot clamp, PolicySpec::clamp_row)
  std::vector<int> slots;     // n_out
  double rho = 0;
  int nhb() const { return (hidden + 15) / 16; }
  int nob() const { return (n_out + 15) / 16; }
  int ku() const { return (n_in + 15) / 16; }  // 16-input groups of layer 1
  // Worlds per wave = 16 * cb: as many 16-world column blocks as keep both
  // hidden layers' tiles (2 x nhb x cb x 4 floats per lane) within ~290 registers.
  int cb() const { return std::max(1, std::min(4, 36 / nhb())); }
  size_t n_weights() const {
    const size_t i = n_in, h = hidden, o = n_out;
    return i * h + h + h * h + h + h * o + o;
  }
  // Fragment buffer (floats): W1 [ku][nhb][64][4], W2 [nhb][nhb][64][4],
  // W3 [nhb][nob][64][4] (input block major, the order the kernel streams
  // them), then the biases.
  size_t off_w2() const { return (size_t)ku() * nhb() * 256; }
  size_t off_w3() const { return off_w2() + (size_t)nhb() * nhb() * 256; }
  size_t off_bias() const { return off_w3() + (size_t)nhb() * nob() * 256; }
  size_t frag_floats() const { return off_bias() + 16 * (size_t)(2 * nhb() + nob()); }
  bool same_shape(const PolicyD& o) const {
    return n_in == o.n_in && hidden == o.hidden && n_out == o.n_out && history == o.history;
  }
};

// The MLP weights in the policy kernel's MFMA fragment order (see
// policy_wave in phz_control.h). Input order is the reference's flat
// W1 b1 W2 b2 W3 b3 with each W row-major [out][in] (policy_pipeline.rs:460-481).
void policy_fragments(const PolicyD& p, const double* w, std::vector<float>& out) {
  const int NI = p.n_in, NH = p.hidden, NO = p.n_out, NHB = p.nhb(), NOB = p.nob(), KU = p.ku();
  const double* W1 = w;
  const double* b1 = W1 + (size_t)NH * NI;
  const double* W2 = b1 + NH;
  const double* b2 = W2 + (size_t)NH * NH;
  const double* W3 = b2 + NH;
  const double* b3 = W3 + (size_t)NO * NH;
  out.assign(p.frag_floats(), 0.0f);
  // Layer 1: component s of fragment (u, hb), lane l = W1[16 hb + l%16][16 u + 4 s + l/16].
  for (int u = 0; u < KU; u++)
    for (int hb = 0; hb < NHB; hb++)
      for (int l = 0; l < 64; l++)
        for (int s = 0; s < 4; s++) {
          const int n = hb * 16 + (l & 15), i = 16 * u + 4 * s + (l >> 4);
          if (n < NH && i < NI) out[(((size_t)u * NHB + hb) * 64 + l) * 4 + s] = (float)W1[(size_t)n * NI + i];
        }
  // Layers 2 and 3: component s of fragment (kb, ob), lane l = W[16 ob + l%16][16 kb + 4 (l/16) + s].
  for (int kb = 0; kb < NHB; kb++)
    for (int hb = 0; hb < NHB; hb++)
      for (int l = 0; l < 64; l++)
        for (int s = 0; s < 4; s++) {
          const int n2 = hb * 16 + (l & 15), n1 = kb * 16 + 4 * (l >> 4) + s;
          if (n2 < NH && n1 < NH) out[p.off_w2() + (((size_t)kb * NHB + hb) * 64 + l) * 4 + s] = (float)W2[(size_t)n2 * NH + n1];
        }
  for (int kb = 0; kb < NHB; kb++)
    for (int ob = 0; ob < NOB; ob++)
      for (int l = 0; l < 64; l++)
        for (int s = 0; s < 4; s++) {
          const int k = ob * 16 + (l & 15), n = kb * 16 + 4 * (l >> 4) + s;
          if (k < NO && n < NH) out[p.off_w3() + (((size_t)kb * NOB + ob) * 64 + l) * 4 + s] = (float)W3[(size_t)k * NH + n];
        }
  for (int n = 0; n < NH; n++) {
    out[p.off_bias() + n] = (float)b1[n];
    out[p.off_bias() + 16 * NHB + n] = (float)b2[n];
  }
  for (int k = 0; k < NO; k++) out[p.off_bias() + 32 * NHB + k] = (float)b3[k];
}

// Debug form of a packed op for error messages (the reference prints ObsOp's Debug).
std::string describe_op(const double* r, const std::vector<double>& aux) {
  const int kind = (int)r[0];
  const char* names[] = {"Const", "QMinus", "V", "BodyPitch", "BodyRoll", "BodyYawError", "BodyPosZ", "BodyPos",
                         "ComOverSupport"};
  if (kind < 0 || kind > 8) return fmt("Unknown(%g)", r[0]);
  switch (kind) {
    case 0: return fmt("Const(%g)", r[3]);
    case 1: return fmt("QMinus(%d, %g)", (int)r[1], r[3]);
    case 5: return fmt("BodyYawError(%d, %g)", (int)r[1], r[3]);
    case 7: return fmt("BodyPos { body: %d, axis: %d }", (int)r[1], (int)r[2]);
    case 8: {
      const size_t a = (size_t)r[1];
      std::string h = a + 1 < aux.size() && aux[a] != 0.0 ? fmt("Some(%d)", (int)aux[a + 1]) : std::string("None");
      return fmt("ComOverSupport { support: %d points, heading_body: %s, axis: %d }", (int)r[2], h.c_str(), (int)r[3]);
    }
    default: return fmt("%s(%d)", names[kind], (int)r[1]);
  }
}

// PolicySpec::validate (policy_pipeline.rs:357-416) and ObsOp::check (153-183)
// on the packed form.
bool validate_policy(const PolicyD& p, int nq, int nv, int nb, int npd, std::string& err) {
  if (p.n_in < 1 || p.n_in > PHZ_POLICY_MAX_IN) { err = fmt("policy input width %d not in 1..=%d", p.n_in, PHZ_POLICY_MAX_IN); return false; }
  if (p.hidden < 1 || p.hidden > PHZ_POLICY_MAX_H) { err = fmt("policy hidden width %d not in 1..=%d", p.hidden, PHZ_POLICY_MAX_H); return false; }
  if (p.n_out < 1 || p.n_out > PHZ_POLICY_MAX_OUT) { err = fmt("policy output width %d not in 1..=%d", p.n_out, PHZ_POLICY_MAX_OUT); return false; }
  if (p.history < 1) { err = "policy history_steps must be at least 1"; return false; }
  for (int k = 0; k < p.n_in; k++) {
    const double* r = &p.ops[(size_t)k * 4];
    bool ok = is_int(r[0]) && r[0] >= 0 && r[0] <= 8 && is_int(r[1]) && r[1] >= 0 && is_int(r[2]) && r[2] >= 0 &&
              std::isfinite(r[3]);
    if (ok) {
      const int kind = (int)r[0], a = (int)r[1], b = (int)r[2];
      switch (kind) {
        case 0: break;
        case 1: ok = a < nq; break;
        case 2: ok = a < nv; break;
        case 3: case 4: case 5: case 6: ok = a < nb; break;
        case 7: ok = a < nb && b < 3; break;
        case 8: {
          ok = is_int(r[3]) && r[3] >= 0 && r[3] < 3 && (size_t)a + 2 + 4 * (size_t)b <= p.aux.size();
          if (ok) {
            const double flag = p.aux[a], h = p.aux[a + 1];
            if (flag != 0.0) ok = is_int(h) && h >= 0 && h < nb;
            for (int j = 0; ok && j < b; j++) {
              const double* sp = &p.aux[a + 2 + 4 * (size_t)j];
              ok = is_int(sp[0]) && sp[0] >= 0 && sp[0] < nb && std::isfinite(sp[1]) && std::isfinite(sp[2]) &&
                   std::isfinite(sp[3]);
            }
          }
          break;
        }
      }
    }
    if (!ok) {
      err = fmt("observation op %s out of range (nq %d, nv %d, nbodies %d)", describe_op(r, p.aux).c_str(), nq, nv, nb);
      return false;
    }
  }
  for (int k = 0; k < p.n_out; k++)
    if (p.slots[k] >= npd) { err = fmt("action slot %d exceeds the %d registered PD servos", p.slots[k], npd); return false; }
  for (double x : p.noise) if (!std::isfinite(x)) { err = "policy input noise must be finite"; return false; }
  for (double x : p.clamp) if (!std::isfinite(x)) { err = "policy action clamp must be finite"; return false; }
  if (!std::isfinite(p.rho)) { err = "policy noise_rho must be finite"; return false; }
  return true;
}

// FK + observation kernel: the model's kinematic constants and the op table.
std::string gen_obs_source(const ModelD& m, const PolicyD* p, bool f64) {
  const std::string T = f64 ? "double" : "float";
  std::string s = kDeviceSrc;
  s += "\n";
  s += kControlSrc;
  s += "\n// ---- model and observation table ----\n";
  s += gen_model(m, Features{});
  const int n = p ? p->n_in : 0, na = std::max(n, 1);
  const std::vector<double> empty;
  const std::vector<double>& aux = p ? p->aux : empty;
  const int naux = std::max<int>((int)aux.size(), 1);
  auto op = [&](int k, int slot) { return n ? p->ops[(size_t)k * 4 + slot] : 0.0; };
  std::ostringstream o;
  o << "struct Obs {\n  static constexpr int N = " << n << ";\n";
  o << "  static constexpr int kind[" << na << "] = " << arr1(na, [&](int k) { return std::to_string((int)op(k, 0)); }) << ";\n";
  o << "  static constexpr int a[" << na << "] = " << arr1(na, [&](int k) { return std::to_string((int)op(k, 1)); }) << ";\n";
  o << "  static constexpr int b[" << na << "] = " << arr1(na, [&](int k) { return std::to_string((int)op(k, 2)); }) << ";\n";
  o << "  static constexpr double c[" << na << "] = " << arr1(na, [&](int k) { return num(op(k, 3)); }) << ";\n";
  o << "  static constexpr double aux[" << naux << "] = "
    << arr1(naux, [&](int k) { return num(aux.empty() ? 0.0 : aux[k]); }) << ";\n};\n";
  s += o.str();
  s += "extern \"C\" __global__ void __launch_bounds__(64) phz_obs(phz::ObsArgs a) {\n";
  if (f64) s += "  phz::fill_tables(threadIdx.x);\n  __syncthreads();\n";  // f64 FK's joint sines and cosines
  s += "  const int w = blockIdx.x * 64 + threadIdx.x;\n";
  s += "  if (w < a.nworld) phz::obs_world<Model, Obs, " + T + ">(a, w);\n}\n";
  return s;
}

// Policy kernel: widths, action wiring and noise scales compiled in.
// two_waves: as gen_source's, two resident waves per SIMD.
std::string gen_policy_source(const PolicyD& p, int npd, bool f64, bool two_waves = false) {
  const std::string T = f64 ? "double" : "float";
  std::string s = kDeviceSrc;
  s += "\n";
  s += kControlSrc;
  const int cb = p.cb();
  const int lds = 16 * cb * std::max(16 * p.ku() + 1, 16 * p.nob() + 1);
  std::ostringstream o;
  o << "\n// ---- policy shape ----\nstruct Pol {\n";
  o << "  static constexpr int NI = " << p.n_in << ", NH = " << p.hidden << ", NO = " << p.n_out << ", NHB = " << p.nhb()
    << ", NOB = " << p.nob() << ", KU = " << p.ku() << ", CB = " << cb << ", NPD = " << npd << ", LDS = " << lds << ";\n";
  o << "  static constexpr double rho = " << num(p.rho) << ";\n";
  o << "  static constexpr double noise[" << p.n_in << "] = " << arr1(p.n_in, [&](int k) { return num(p.noise[k]); }) << ";\n";
  o << "  static constexpr double clamp[" << p.n_out << "] = " << arr1(p.n_out, [&](int k) { return num(p.clamp[k]); }) << ";\n";
  o << "  static constexpr int slot[" << p.n_out << "] = " << arr1(p.n_out, [&](int k) { return std::to_string(p.slots[k]); })
    << ";\n};\n";
  s += o.str();
  s += std::string("extern \"C\" __global__ void __launch_bounds__(64)") +
       (two_waves ? " __attribute__((amdgpu_waves_per_eu(2, 2)))" : "") + " phz_policy(phz::PolicyArgs a) {\n";
  s += "  __shared__ float lds[Pol::LDS];\n";
  s += "  phz::fill_tables(threadIdx.x);\n  __syncthreads();\n";  // the normals' f64 log, sine and cosine tables
  s += "  phz::policy_wave<Pol, " + T + ">(a, lds);\n}\n";
  return s;
}

struct ObsArgs {  // must match phz::ObsArgs in phz_control.h
  const void* q;
  const void* v;
  void* kin;
  float* obs;
  int nworld;
  int stride;
  int write_kin;
  int write_obs;
};

struct PolicyArgs {  // must match phz::PolicyArgs in phz_control.h
  const void* w1;
  const void* w2;
  const void* w3;
  const float* bias;
  const float* stdv;
  float* obs;
  float* out;
  uint64_t* rng;
  float* z;
  const void* base;
  void* targets;
  int nworld;
  int stride;
};

// A hiprtc-built kernel with its module, tagged with the configuration epoch it was built for.
struct Kern {
  std::shared_ptr<CodeObject> code;
  hipModule_t mod = nullptr;
  hipFunction_t fn = nullptr;
  uint64_t epoch = 0;
  void reset() {
    if (mod) hipModuleUnload(mod);
    mod = nullptr;
    fn = nullptr;
    code.reset();
    epoch = 0;
  }
};

}  // namespace

struct phz_sim {
  ModelD model;
  Features feat;
  int ctrl_rows = 0;  // rows the ctrl buffer holds (nv at create; grows for actuators)
  int nctrl() const { return feat.acts.empty() ? model.nv : (int)feat.acts.size(); }
  int nworld = 0, stride = 0;
  bool f64 = false;
  int device = -1;
  int block = 64;
  int lanes = 1;  // lanes per world of the step kernel
  int max_steps = 1000;
  hipStream_t stream = nullptr;
  void *q = nullptr, *v = nullptr, *ctrl = nullptr, *qdd = nullptr, *targets = nullptr, *rows = nullptr;
  void *ext_buf = nullptr, *imp_buf = nullptr, *hf_buf = nullptr;  // impulse solver state; heightfield nodes (f64)
  size_t hf_cap = 0;                                                // node capacity of hf_buf
  uint64_t* rng = nullptr;
  double* staging = nullptr;
  size_t staging_bytes = 0;
  std::shared_ptr<CodeObject> code;
  hipModule_t module = nullptr;
  hipFunction_t fn = nullptr;
  // The same kernel built for two resident waves per SIMD (two_waves_pay),
  // for launches of at least kTwoWaveMinSteps steps; null where it does not pay.
  std::shared_ptr<CodeObject> code2;
  hipModule_t module2 = nullptr;
  hipFunction_t fn2 = nullptr;
  bool graphs = true;
  hipGraphExec_t gexec = nullptr;
  uint32_t graph_steps = 0;
  uint64_t graph_epoch = 0;
  uint64_t epoch = 1;
  std::string err;

  // Device-resident control loop (mod.rs:1004-1376).
  bool kin_on = false;
  void* kin = nullptr;          // [nb * 18][stride] T, FK readout
  Kern obs_k, pol_k;
  uint64_t ctl_epoch = 1;       // bumped when the model, PD table or policy spec changes
  bool policy_on = false;
  PolicyD pol;
  float* pw = nullptr;          // weight fragments and biases
  float* pstd = nullptr;        // [n_out]
  float* obs_hist = nullptr;    // [history][n_in][stride]
  float* out_hist = nullptr;    // [history][n_out + 1][stride]
  float* pz = nullptr;          // [n_out][stride]
  uint64_t* prng = nullptr;     // [stride]
  void* pbase = nullptr;        // [npd][stride] T
  int pbase_npd = 0;
  int hist_slots = 0;
  void *hq = nullptr, *hv = nullptr;  // [slots][nq | nv][stride] T
  hipGraphExec_t rexec = nullptr;     // captured rollout
  uint64_t rkey[6] = {0, 0, 0, 0, 0, 0};

  size_t esize() const { return f64 ? 8 : 4; }
  bool has_device() const { return device >= 0; }

  int fail(const std::string& e) { err = e; return 1; }
  bool hip_ok(hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    err = fmt("%s: %s", what, hipGetErrorString(e));
    return false;
  }
  void drop_graph() {
    if (gexec) { hipGraphExecDestroy(gexec); gexec = nullptr; }
    graph_steps = 0;
    if (rexec) { hipGraphExecDestroy(rexec); rexec = nullptr; }
  }
  void invalidate() {  // a new kernel or buffer: recompile lazily, re-capture
    if (stream) hipStreamSynchronize(stream);  // nothing in flight uses the modules unloaded below
    drop_graph();
    if (module) { hipModuleUnload(module); module = nullptr; fn = nullptr; }
    if (module2) { hipModuleUnload(module2); module2 = nullptr; fn2 = nullptr; }
    code.reset();
    code2.reset();
    epoch++;
    ctl_epoch++;
  }
  bool alloc(void** p, size_t bytes, const char* what) {
    if (!hip_ok(hipMalloc(p, std::max<size_t>(bytes, 256)), what)) return false;
    return hip_ok(phz_io_zero(*p, std::max<size_t>(bytes, 256), stream), what);
  }
  bool ensure_staging(size_t bytes) {
    if (bytes <= staging_bytes) return true;
    // A pack or unpack kernel queued on the stream may still read the old buffer.
    if (staging && !hip_ok(hipStreamSynchronize(stream), "staging sync")) return false;
    if (staging) hipFree(staging);
    staging = nullptr;
    staging_bytes = 0;
    if (!hip_ok(hipMalloc((void**)&staging, bytes), "staging alloc")) return false;
    staging_bytes = bytes;
    return true;
  }
  // host [nworld][width] f64 -> device SoA
  bool upload_rows(const double* host, void* dst, int width, const char* what) {
    if (width <= 0) return true;
    const size_t bytes = (size_t)nworld * width * sizeof(double);
    if (!ensure_staging(bytes)) return false;
    if (!hip_ok(hipMemcpyAsync(staging, host, bytes, hipMemcpyHostToDevice, stream), what)) return false;
    return hip_ok(phz_io_pack(staging, dst, nworld, width, stride, f64 ? 1 : 0, stream), what);
  }
  // elem: 1 = f64, 0 = f32 source; -1 = the sim's precision.
  bool download_rows(const void* src, double* host, int width, const char* what, int elem = -1) {
    if (width <= 0) return true;
    const size_t bytes = (size_t)nworld * width * sizeof(double);
    if (!ensure_staging(bytes)) return false;
    const int src_f64 = elem < 0 ? (f64 ? 1 : 0) : elem;
    if (!hip_ok(phz_io_unpack(src, staging, nworld, width, stride, src_f64, stream), what)) return false;
    if (!hip_ok(hipMemcpyAsync(host, staging, bytes, hipMemcpyDeviceToHost, stream), what)) return false;
    return hip_ok(hipStreamSynchronize(stream), what);
  }

  bool compile() {
    if (code) return true;
    std::string e;
    int ng = 1;
    const std::string src = gen_source(model, feat, f64, &ng, &lanes);
    block = 64 * ng;
    if (const char* dump = std::getenv("PHZ_DUMP_SOURCE")) {
      std::ofstream out(dump);
      out << src;
    }
    if (f64 && feat.cmode == 1) {
      code = compile_source(src, Build::Ieee, e);
    } else {
      Build b = Build::Reassoc;
      code = compile_source(src, b, e);
      if (code && remark_value(code->log, "ScratchSize [bytes/lane]:") > 0) {
        b = Build::Finite;
        code = compile_source(src, b, e);
      }
      if (code && ng == 1 && two_waves_pay(code->log)) {
        // The same build as the one-wave kernel (the same arithmetic: a launch
        // gives the same bits whichever of the two runs it), kept while its
        // spills stay small: 512 bytes per lane reassociated, 768 in order,
        // 128 in f64. An f32 kernel whose reassociated rebuild spills more
        // takes the in-order build for both kernels when that rebuild fits.
        int ng2 = 1, lanes2 = 1;
        const std::string src2 = gen_source(model, feat, f64, &ng2, &lanes2, true);
        auto spills = [](const std::shared_ptr<CodeObject>& c) {
          return c ? remark_value(c->log, "ScratchSize [bytes/lane]:") : (int64_t)-1;
        };
        auto fits = [&](const std::shared_ptr<CodeObject>& c, Build bb) {
          const int64_t sc = spills(c);
          return sc >= 0 && sc <= (f64 ? 128 : bb == Build::Reassoc ? 512 : 768);
        };
        std::string e2;
        auto c2 = compile_source(src2, b, e2);
        if (fits(c2, b)) {
          code2 = c2;
        } else if (!f64 && b == Build::Reassoc) {
          auto c2f = compile_source(src2, Build::Finite, e2);
          auto c1f = fits(c2f, Build::Finite) ? compile_source(src, Build::Finite, e2) : nullptr;
          if (c1f && spills(c1f) == 0) {
            code = c1f;
            code2 = c2f;
          }
        }
      }
    }
    if (!code) { err = e; return false; }
    return true;
  }
  // Whether the one-wave-per-world-group kernel compiled to `log` gets a
  // second build for two resident waves per SIMD: it holds more than 256
  // registers (one wave per SIMD), and the launch has more waves than the
  // device has SIMDs, so that at one per SIMD they run in rounds with nothing
  // to cover a wave's latencies. The rebuild spills registers to scratch and
  // pays a fixed cost per launch (about 14 us more at 131072 ant worlds), so
  // launches of fewer than kTwoWaveMinSteps steps keep the one-wave kernel.
  // Measured on MI355X (ms per 1000 steps, one launch): the ant at 131072
  // worlds 9.03 -> 7.22 (404 B of spills per lane), at 98304 9.16 -> 7.59, at
  // 262144 18.02 -> 14.22, but 4.54 -> 4.94 at 65536 (one wave per SIMD either
  // way); the MJCF ant reassociated 16.30 -> 16.54 (960 B, not taken), in
  // order 17.39 -> 12.91 (612 B: both kernels in order, its 1- and 5-step
  // launches 6% slower than the reassociated one-wave kernel); chain7 f64 at
  // 131072 6.51 -> 8.46 (284 B of 8-byte spills, not taken). Per launch at
  // 131072 ant worlds: 1 step 21.2 -> 33.8 us, 5 steps 62.2 -> 65.6, 20 steps
  // 210.6 -> 191.2. PHZ_TWO_WAVES=0 keeps one wave per SIMD (and the
  // reassociated build).
  bool two_waves_pay(const std::string& log) const {
    if (const char* e = std::getenv("PHZ_TWO_WAVES"))
      if (e[0] == '0') return false;
    const int64_t regs = remark_value(log, "VGPRs:") + std::max<int64_t>(remark_value(log, "AGPRs:"), 0);
    const long waves = (long)std::max(feat.wgs, 1) * lanes;
    return regs > 256 && waves > 4L * std::max(feat.cus, 1);
  }
  bool load_kernel() {
    if (fn) return true;
    if (!compile()) return false;
    if (code2) {
      if (!hip_ok(hipModuleLoadData(&module2, code2->code.data()), "hipModuleLoadData")) return false;
      if (!hip_ok(hipModuleGetFunction(&fn2, module2, "phz_step"), "hipModuleGetFunction")) return false;
    }
    if (!hip_ok(hipModuleLoadData(&module, code->code.data()), "hipModuleLoadData")) return false;
    return hip_ok(hipModuleGetFunction(&fn, module, "phz_step"), "hipModuleGetFunction");
  }
  // start / stop: events stamped with this launch's own start and end
  // (hipExtModuleLaunchKernel), for timing; null otherwise.
  bool launch(int nsteps, hipEvent_t start = nullptr, hipEvent_t stop = nullptr) {
    StepArgs a{q,       v,       ctrl,    qdd,          targets,          rng,        rows,       ext_buf, imp_buf,
               hf_buf,  feat.hf_o[0], feat.hf_o[1], feat.hf_o[2], feat.hf_cell, feat.hf_nx, feat.hf_ny, nworld,
               stride,  nsteps,  feat.contact ? 1 : 0};
    void* params[] = {&a};
    const unsigned grid = (unsigned)(((long)nworld * lanes + 63) / 64);
    hipFunction_t fn = fn2 && nsteps >= kTwoWaveMinSteps ? fn2 : this->fn;
    if (start || stop) {
      // hipExtModuleLaunchKernel takes the grid in work-items (32 bits);
      // beyond that the events bracket the launch on the stream instead.
      if ((uint64_t)grid * (uint64_t)block <= 0xffffffffull)
        return hip_ok(hipExtModuleLaunchKernel(fn, grid * (unsigned)block, 1, 1, (unsigned)block, 1, 1, 0, stream,
                                               params, nullptr, start, stop, 0),
                      "step kernel launch");
      if (start && !hip_ok(hipEventRecord(start, stream), "hipEventRecord")) return false;
      if (!hip_ok(hipModuleLaunchKernel(fn, grid, 1, 1, (unsigned)block, 1, 1, 0, stream, params, nullptr),
                  "step kernel launch"))
        return false;
      return !stop || hip_ok(hipEventRecord(stop, stream), "hipEventRecord");
    }
    return hip_ok(hipModuleLaunchKernel(fn, grid, 1, 1, (unsigned)block, 1, 1, 0, stream, params, nullptr),
                  "step kernel launch");
  }
  // The span's launches; start is stamped by the first one and stop by the last.
  bool issue(uint32_t n, hipEvent_t start = nullptr, hipEvent_t stop = nullptr) {
    for (uint32_t done = 0; done < n;) {
      const uint32_t k = std::min<uint32_t>(n - done, (uint32_t)max_steps);
      const bool last = done + k == n;
      if (!launch((int)k, done == 0 ? start : nullptr, last ? stop : nullptr)) return false;
      done += k;
    }
    return true;
  }
  // What every step span needs before a launch: a device, a sweep count in
  // impulse mode and the loaded kernel. `launch` is false (and the call a
  // successful no-op) for zero steps or zero worlds.
  bool span_ready(uint32_t n, bool& launch) {
    launch = false;
    if (feat.contact && feat.cmode == 1 && feat.sweeps < 1) {
      err = "impulse contact needs at least one contact sweep per step";
      return false;
    }
    if (n == 0 || nworld == 0) return true;
    if (!has_device()) { err = "host-only sim (device_ordinal -1) cannot step"; return false; }
    if (!load_kernel()) return false;
    launch = true;
    return true;
  }

  bool step_many(uint32_t n) {
    bool launch = false;
    if (!span_ready(n, launch)) return false;
    if (!launch) return true;
    // A span of one launch goes straight to the stream: replaying a one-node
    // graph costs about 5 us more per span on MI355X (86.5 against 81.8 us
    // wall for 20 chain steps at 65536 worlds).
    if (!graphs || n <= (uint32_t)max_steps) return issue(n);
    if (!(gexec && graph_steps == n && graph_epoch == epoch)) {
      drop_graph();
      if (!hip_ok(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture"))
        return false;
      const bool issued = issue(n);
      hipGraph_t graph = nullptr;
      // End the capture even when a launch failed (mod.rs:862-867).
      hipError_t ec = hipStreamEndCapture(stream, &graph);
      if (!issued) { if (graph) hipGraphDestroy(graph); return false; }
      if (!hip_ok(ec, "hipStreamEndCapture")) return false;
      hipError_t ei = hipGraphInstantiate(&gexec, graph, nullptr, nullptr, 0);
      hipGraphDestroy(graph);
      if (!hip_ok(ei, "hipGraphInstantiate")) { gexec = nullptr; return false; }
      graph_steps = n;
      graph_epoch = epoch;
    }
    return hip_ok(hipGraphLaunch(gexec, stream), "hipGraphLaunch");
  }

  // ── control loop ──
  float* obs_row(uint32_t step) const { return obs_hist + (size_t)step * pol.n_in * stride; }
  float* out_row(uint32_t step) const { return out_hist + (size_t)step * (pol.n_out + 1) * stride; }

  // Compile (and with `load`, load) the FK/observation or the policy kernel
  // for the current configuration epoch.
  bool ensure_ctl(bool policy_kernel, bool load) {
    Kern& k = policy_kernel ? pol_k : obs_k;
    if (k.code && k.epoch != ctl_epoch) {
      if (stream) hipStreamSynchronize(stream);
      if (rexec) { hipGraphExecDestroy(rexec); rexec = nullptr; }
      k.reset();
    }
    if (!k.code) {
      const std::string src = policy_kernel ? gen_policy_source(pol, feat.npd, f64)
                                            : gen_obs_source(model, policy_on ? &pol : nullptr, f64);
      std::string e;
      k.code = compile_source(src, Build::Finite, e);
      if (!k.code) { err = e; return false; }
      // The policy kernel holds about 370 registers at CB = 2, one wave per
      // SIMD, and its per-world VALU work (the normals, tanh) then does not
      // overlap the matrix cores. With more waves than SIMDs, a build for
      // two resident waves per SIMD (the same build: the same bits) overlaps
      // one wave's VALU work with another's MFMAs: on the ant control workload
      // (131072 worlds, 4096 waves) 0.255 -> 0.224 ms per launch with 164 B
      // of spills per lane, rollout 16.99 -> 15.35 ms. Taken while it spills
      // at most 512 B per lane; PHZ_TWO_WAVES=0 keeps one wave per SIMD.
      const char* tw = std::getenv("PHZ_TWO_WAVES");
      const long waves = ((long)nworld + 16L * pol.cb() - 1) / (16L * pol.cb());
      const int64_t regs = remark_value(k.code->log, "VGPRs:") + std::max<int64_t>(remark_value(k.code->log, "AGPRs:"), 0);
      if (policy_kernel && !(tw && tw[0] == '0') && regs > 256 && waves > 4L * std::max(feat.cus, 1)) {
        std::string e2;
        auto c2 = compile_source(gen_policy_source(pol, feat.npd, f64, true), Build::Finite, e2);
        const int64_t sc = c2 ? remark_value(c2->log, "ScratchSize [bytes/lane]:") : -1;
        if (sc >= 0 && sc <= 512) k.code = c2;
      }
      k.epoch = ctl_epoch;
    }
    if (load && !k.fn) {
      if (!hip_ok(hipModuleLoadData(&k.mod, k.code->code.data()), "hipModuleLoadData")) return false;
      if (!hip_ok(hipModuleGetFunction(&k.fn, k.mod, policy_kernel ? "phz_policy" : "phz_obs"), "hipModuleGetFunction"))
        return false;
    }
    return true;
  }
  bool launch_obs(float* obs, bool write_kin) {
    ObsArgs a{q, v, write_kin ? kin : nullptr, obs, nworld, stride, write_kin ? 1 : 0, obs ? 1 : 0};
    void* params[] = {&a};
    const unsigned grid = (unsigned)((nworld + 63) / 64);
    return hip_ok(hipModuleLaunchKernel(obs_k.fn, grid, 1, 1, 64, 1, 1, 0, stream, params, nullptr), "obs kernel launch");
  }
  bool launch_policy(uint32_t step) {
    const int wpw = 16 * pol.cb();
    PolicyArgs a{pw, pw + pol.off_w2(), pw + pol.off_w3(), pw + pol.off_bias(), pstd, obs_row(step), out_row(step),
                 prng, pz, pbase, targets, nworld, stride};
    void* params[] = {&a};
    const unsigned grid = (unsigned)((nworld + wpw - 1) / wpw);
    return hip_ok(hipModuleLaunchKernel(pol_k.fn, grid, 1, 1, 64, 1, 1, 0, stream, params, nullptr),
                  "policy kernel launch");
  }
  // Everything run_policy needs, checked on the host (mod.rs:1209-1231).
  bool policy_ready(uint32_t last_step) {
    if (!policy_on) { err = "policy pass not enabled — call enable_policy first"; return false; }
    if (feat.npd == 0) { err = "policy pass needs PD control"; return false; }
    if (last_step >= (uint32_t)pol.history) {
      err = fmt("policy step %u exceeds history_steps %d", last_step, pol.history);
      return false;
    }
    if (!has_device()) { err = "host-only sim (device_ordinal -1) cannot run the policy"; return false; }
    for (int k = 0; k < pol.n_out; k++)
      if (pol.slots[k] >= feat.npd) {
        err = fmt("action slot %d exceeds the %d registered PD servos", pol.slots[k], feat.npd);
        return false;
      }
    if (pbase_npd != feat.npd) {  // the PD table was re-registered with another servo count
      if (pbase) hipFree(pbase);
      pbase = nullptr;
      if (!alloc(&pbase, (size_t)feat.npd * stride * esize(), "base targets alloc")) return false;
      pbase_npd = feat.npd;
    }
    return ensure_ctl(false, true) && ensure_ctl(true, true);
  }
  bool record(uint32_t slot) {
    const size_t E = esize(), S = stride;
    return hip_ok(phz_io_copy((char*)hq + (size_t)slot * model.nq * S * E, q, (size_t)model.nq * S * E, stream),
                  "record_state q") &&
           hip_ok(phz_io_copy((char*)hv + (size_t)slot * model.nv * S * E, v, (size_t)model.nv * S * E, stream),
                  "record_state v");
  }
  bool issue_rollout(uint32_t first, uint32_t n, uint32_t every, bool rec) {
    for (uint32_t c = 0; c < n; c++) {
      if (!launch_obs(obs_row(first + c), true) || !launch_policy(first + c) || !issue(every)) return false;
      if (rec && !record(first + c)) return false;
    }
    return true;
  }
  bool rollout(uint32_t first, uint32_t n, uint32_t every, bool rec) {
    if (n == 0) return true;
    if (!policy_ready(first + n - 1)) return false;
    if (rec) {
      if (!hist_slots) { err = "state history not enabled — call enable_state_history first"; return false; }
      if (first + n > (uint32_t)hist_slots) {
        err = fmt("history slot %u exceeds %d slots", first + n - 1, hist_slots);
        return false;
      }
    }
    if (every > 0 && !load_kernel()) return false;
    if (nworld == 0) return true;
    if (!graphs) return issue_rollout(first, n, every, rec);
    const uint64_t key[6] = {first, n, every, rec ? 1u : 0u, epoch, ctl_epoch};
    if (!(rexec && std::equal(key, key + 6, rkey))) {
      if (rexec) { hipGraphExecDestroy(rexec); rexec = nullptr; }
      if (!hip_ok(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture")) return false;
      const bool issued = issue_rollout(first, n, every, rec);
      hipGraph_t graph = nullptr;
      hipError_t ec = hipStreamEndCapture(stream, &graph);
      if (!issued) { if (graph) hipGraphDestroy(graph); return false; }
      if (!hip_ok(ec, "hipStreamEndCapture")) return false;
      hipError_t ei = hipGraphInstantiate(&rexec, graph, nullptr, nullptr, 0);
      hipGraphDestroy(graph);
      if (!hip_ok(ei, "hipGraphInstantiate")) { rexec = nullptr; return false; }
      std::copy(key, key + 6, rkey);
    }
    return hip_ok(hipGraphLaunch(rexec, stream), "hipGraphLaunch");
  }
  void free_policy_buffers() {
    for (void* p : {(void*)pw, (void*)pstd, (void*)obs_hist, (void*)out_hist, (void*)pz, (void*)prng, pbase})
      if (p) hipFree(p);
    pw = pstd = obs_hist = out_hist = pz = nullptr;
    prng = nullptr;
    pbase = nullptr;
    pbase_npd = 0;
  }

  ~phz_sim() {
    if (has_device()) {
      hipSetDevice(device);
      if (stream) hipStreamSynchronize(stream);
      drop_graph();
      if (module) hipModuleUnload(module);
      if (module2) hipModuleUnload(module2);
      obs_k.reset();
      pol_k.reset();
      free_policy_buffers();
      for (void* p : {q, v, ctrl, qdd, targets, rows, (void*)rng, (void*)staging, kin, hq, hv, ext_buf, imp_buf, hf_buf})
        if (p) hipFree(p);
      if (stream) hipStreamDestroy(stream);
    }
  }
};

namespace {
bool set_device(phz_sim* s) { return !s->has_device() || s->hip_ok(hipSetDevice(s->device), "hipSetDevice"); }

template <class F> int time_reps(phz_sim* s, uint32_t reps, double* ms_per_rep, F body) {
  std::vector<hipEvent_t> ev(2 * (size_t)reps);
  for (auto& e : ev)
    if (!s->hip_ok(hipEventCreate(&e), "hipEventCreate")) return 1;
  bool ok = true;
  for (uint32_t r = 0; r < reps && ok; r++)
    ok = s->hip_ok(hipEventRecord(ev[2 * r], s->stream), "hipEventRecord") && body() &&
         s->hip_ok(hipEventRecord(ev[2 * r + 1], s->stream), "hipEventRecord");
  ok = ok && s->hip_ok(hipStreamSynchronize(s->stream), "timing sync");
  for (uint32_t r = 0; r < reps && ok; r++) {
    float ms = 0;
    ok = s->hip_ok(hipEventElapsedTime(&ms, ev[2 * r], ev[2 * r + 1]), "hipEventElapsedTime");
    ms_per_rep[r] = ms;
  }
  for (auto& e : ev) (void)hipEventDestroy(e);
  return ok ? 0 : 1;
}

// Everything enable_contact takes (crates/phyz-gpu/src/cuda/mod.rs:704-733):
// ground or terrain, penalty or impulse, an optional body-attached plane.
struct ContactSpec {
  double ground_h = 0, friction = 0;
  const double* geom = nullptr;
  const double* gains = nullptr;  // nb x 2 (k, d), or the global k, d below
  double k = 0, d = 0;
  int cmode = 0;
  const double* solver = nullptr;  // 9 solver parameters, or the defaults
  const double* plane = nullptr;   // body, offset, max depth, half x, half y
  const uint32_t* exclude = nullptr;
  uint32_t n_exclude = 0;
  const double* hf = nullptr;      // nx, ny, origin x, y, z, cell
  const double* heights = nullptr; // [ny][nx]
};

// validate_heightfield (crates/phyz-gpu/src/contact_pipeline.rs:652-671).
bool check_heightfield(phz_sim* s, const double* hf, const double* heights, int& nx, int& ny) {
  if (!hf) return true;
  if (!(is_int(hf[0]) && is_int(hf[1])) || hf[0] < 1 || hf[1] < 1 || hf[0] > (1 << 15) || hf[1] > (1 << 15)) {
    s->err = "heightfield needs at least one node per axis";
    return false;
  }
  if (!(std::isfinite(hf[5]) && hf[5] > 0.0)) { s->err = fmt("heightfield cell must be positive, got %g", hf[5]); return false; }
  for (int k = 2; k < 5; k++)
    if (!std::isfinite(hf[k])) { s->err = "heightfield origin must be finite"; return false; }
  if (!heights) { s->err = "null heightfield heights"; return false; }
  nx = (int)hf[0];
  ny = (int)hf[1];
  for (size_t k = 0; k < (size_t)nx * ny; k++)
    if (!std::isfinite(heights[k])) { s->err = "heightfield heights must be finite"; return false; }
  return true;
}

// The nodes stay f64 on the device in every precision: the kernels evaluate
// the terrain in f64 (see Terrain in phz_device.h).
bool upload_heightfield(phz_sim* s, const double* heights, size_t n) {
  if (!s->has_device()) return true;
  if (!s->hip_ok(hipMemcpyAsync(s->hf_buf, heights, n * sizeof(double), hipMemcpyHostToDevice, s->stream),
                 "upload heightfield"))
    return false;
  return s->hip_ok(hipStreamSynchronize(s->stream), "upload heightfield");
}

int set_contact(phz_sim* s, const ContactSpec& cs, uint32_t* collidable_out) {
  if (!cs.geom) return s->fail("null geometry table");
  if (!(std::isfinite(cs.ground_h) && std::isfinite(cs.friction))) return s->fail("ground height and friction must be finite");
  const int nb = s->model.nb;
  if (cs.plane) {
    if (!is_int(cs.plane[0]) || cs.plane[0] < 0 || cs.plane[0] >= nb)
      return s->fail(fmt("plane body %g out of range for a model with %d bodies", cs.plane[0], nb));
    for (int k = 1; k < 5; k++) if (!std::isfinite(cs.plane[k])) return s->fail("plane parameters must be finite");
    for (uint32_t k = 0; k < cs.n_exclude; k++)
      if (cs.exclude[k] >= (uint32_t)nb) return s->fail(fmt("plane exclude body %u out of range", cs.exclude[k]));
  }
  int nx = 0, ny = 0;
  if (!check_heightfield(s, cs.hf, cs.heights, nx, ny)) return 1;
  if (cs.solver)
    for (int k = 0; k < 9; k++) if (!std::isfinite(cs.solver[k])) return s->fail("contact solver parameters must be finite");
  std::vector<double> g(cs.geom, cs.geom + (size_t)nb * kGeomStride);
  int collidable = 0;
  for (int i = 0; i < nb; i++) {
    double* r = &g[(size_t)i * kGeomStride];
    if (!is_int(r[0]) || r[0] < 0 || r[0] > 5) return s->fail(fmt("body %d: unknown geometry type %g", i, r[0]));
    if (cs.gains) { r[8] = cs.gains[i * 2]; r[9] = cs.gains[i * 2 + 1]; }
    else { r[8] = cs.k; r[9] = cs.d; }
    r[7] = 0.0;
    for (int q = 1; q < 22; q++)
      if (!std::isfinite(r[q])) return s->fail(fmt("body %d: non-finite geometry slot %d", i, q));
    if ((int)r[0] != 0) collidable++;
  }
  if (cs.plane) {  // pack_contact_geometry: the plane body and the excluded bodies never touch the plane
    g[(size_t)cs.plane[0] * kGeomStride + 7] = 1.0;
    for (uint32_t k = 0; k < cs.n_exclude; k++) g[(size_t)cs.exclude[k] * kGeomStride + 7] = 1.0;
  }
  if (collidable == 0)
    return s->fail("ground contact enabled but no body has GPU-collidable geometry "
                   "(supported: sphere, box, capsule, cylinder, mesh)");
  if (!set_device(s)) return 1;
  Features& f = s->feat;
  f.contact = true;
  f.ground_h = cs.ground_h;
  f.mu = cs.friction;
  f.geom = std::move(g);
  f.collidable = collidable;
  f.cmode = cs.cmode;
  const double dt = s->model.dt;
  const double defaults[9] = {0.0, 0.05, cs.cmode == 1 ? dt / (2.0 * 0.02 * 1.0 + dt) : 0.001 / (2.0 * 0.02 + 0.001),
                              0.001, 0.9, 0.95, 0.001, 0.5, 2.0};
  for (int k = 0; k < 9; k++) f.prm[k] = cs.solver ? cs.solver[k] : defaults[k];
  f.plane_body = cs.plane ? (int)cs.plane[0] : -1;
  for (int k = 0; k < 4; k++) f.plane[k] = cs.plane ? cs.plane[1 + k] : 0.0;
  f.hf_nx = nx;
  f.hf_ny = ny;
  for (int k = 0; k < 3; k++) f.hf_o[k] = cs.hf ? cs.hf[2 + k] : 0.0;
  f.hf_cell = cs.hf ? cs.hf[5] : 1.0;
  if (s->has_device()) {
    const size_t E = s->esize(), S = s->stride;
    if (!s->rows && !s->alloc(&s->rows, (size_t)nb * 8 * S * E, "contact rows alloc")) return 1;
    if (cs.cmode == 1) {
      if (!s->ext_buf && !s->alloc(&s->ext_buf, (size_t)nb * 6 * S * E, "contact force state alloc")) return 1;
      if (!s->imp_buf && !s->alloc(&s->imp_buf, (size_t)nb * 48 * S * E, "impulse state alloc")) return 1;
    }
    // Node buffer sized to this first field (set_heightfield may shrink, not grow, it).
    const size_t nodes = (size_t)std::max(nx, 1) * std::max(ny, 1);
    if (s->hf_buf) { s->invalidate(); hipFree(s->hf_buf); s->hf_buf = nullptr; }
    if (!s->alloc(&s->hf_buf, nodes * sizeof(double), "heightfield alloc")) return 1;
    s->hf_cap = nx > 0 ? nodes : 0;
    if (nx > 0 && !upload_heightfield(s, cs.heights, nodes)) return 1;
  } else {
    s->hf_cap = (size_t)nx * ny;
  }
  s->invalidate();
  if (collidable_out) *collidable_out = (uint32_t)collidable;
  return 0;
}
}  // namespace

extern "C" {

int phz_sim_create(const double* body_table, uint32_t nb, uint32_t nq, uint32_t nv, const double gravity[3],
                   double dt, uint32_t nworld, int precision, int device_ordinal, phz_sim** out) {
  g_create_error.clear();
  if (!out) { g_create_error = "null output pointer"; return 1; }
  *out = nullptr;
  if (precision != PHZ_F32 && precision != PHZ_F64) { g_create_error = "precision must be PHZ_F32 or PHZ_F64"; return 1; }
  if (nworld > (1u << 28)) { g_create_error = "nworld too large"; return 1; }
  auto s = std::make_unique<phz_sim>();
  if (!parse_model(body_table, nb, nq, nv, gravity, dt, s->model, g_create_error)) return 1;
  s->nworld = (int)nworld;
  s->stride = (int)((nworld + 63) / 64 * 64);
  s->f64 = precision == PHZ_F64;
  s->device = device_ordinal;
  s->max_steps = std::max(1, env_int("PHZ_MAX_STEPS_PER_LAUNCH", 1000));
  const char* ge = std::getenv("PHZ_HIP_GRAPHS");
  s->graphs = !(ge && (!std::strcmp(ge, "0") || !std::strcmp(ge, "off") || !std::strcmp(ge, "false")));
  if (device_ordinal >= 0) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0) { g_create_error = "no HIP device available"; return 1; }
    if (device_ordinal >= count) { g_create_error = fmt("device ordinal %d out of range (%d devices)", device_ordinal, count); return 1; }
    if (!s->hip_ok(hipSetDevice(device_ordinal), "hipSetDevice")) { g_create_error = s->err; return 1; }
    if (!s->hip_ok(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking), "hipStreamCreate")) {
      g_create_error = s->err;
      return 1;
    }
    const size_t E = s->esize(), S = (size_t)s->stride;
    if (!s->alloc(&s->q, (size_t)nq * S * E, "alloc q") || !s->alloc(&s->v, (size_t)nv * S * E, "alloc v") ||
        !s->alloc(&s->ctrl, (size_t)std::max(nv, 1u) * S * E, "alloc ctrl") || !s->alloc(&s->qdd, (size_t)nv * S * E, "alloc qdd") ||
        !s->alloc((void**)&s->rng, S * 8, "alloc rng") ||
        !s->hip_ok(hipStreamSynchronize(s->stream), "create sync")) {
      g_create_error = s->err;
      return 1;
    }
    s->ctrl_rows = (int)std::max(nv, 1u);
  }
  {
    int cus = 256;
    if (device_ordinal >= 0 && hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device_ordinal) != hipSuccess)
      cus = 256;
    s->feat.wgs = s->stride / 64;
    s->feat.cus = std::max(cus, 1);
    s->feat.f64 = s->f64;
    s->feat.host_only = device_ordinal < 0;
  }
  *out = s.release();
  return 0;
}

void phz_sim_destroy(phz_sim* sim) {
  if (sim) { set_device(sim); delete sim; }
}

const char* phz_last_error(const phz_sim* sim) { return sim ? sim->err.c_str() : g_create_error.c_str(); }

int phz_set_model(phz_sim* s, const double* body_table, uint32_t nb, uint32_t nq, uint32_t nv, const double gravity[3],
                  double dt) {
  if (!s) return 1;
  ModelD m;
  std::string e;
  if (!parse_model(body_table, nb, nq, nv, gravity, dt, m, e)) return s->fail(e);
  if (m.nb != s->model.nb || m.nq != s->model.nq || m.nv != s->model.nv)
    return s->fail(fmt("set_model: shape changed (%d bodies, nq %d, nv %d vs %d bodies, nq %d, nv %d); build a new simulator",
                       m.nb, m.nq, m.nv, s->model.nb, s->model.nq, s->model.nv));
  s->model = m;
  s->invalidate();
  return 0;
}

int phz_enable_ground_contact(phz_sim* s, double ground_height, double stiffness, double damping, double friction,
                              const double* geom_table, uint32_t* collidable_out) {
  if (!s) return 1;
  if (!(std::isfinite(stiffness) && std::isfinite(damping))) return s->fail("stiffness and damping must be finite");
  ContactSpec cs;
  cs.ground_h = ground_height;
  cs.friction = friction;
  cs.geom = geom_table;
  cs.k = stiffness;
  cs.d = damping;
  return set_contact(s, cs, collidable_out);
}

int phz_enable_ground_contact_per_body(phz_sim* s, double ground_height, double friction, const double* gains,
                                       const double* geom_table, uint32_t* collidable_out) {
  if (!s) return 1;
  if (!gains) return s->fail("null gains table");
  ContactSpec cs;
  cs.ground_h = ground_height;
  cs.friction = friction;
  cs.geom = geom_table;
  cs.gains = gains;
  return set_contact(s, cs, collidable_out);
}

namespace {
int enable_contact_with(phz_sim* s, int cmode, double ground_height, double friction, const double* gains,
                        const double* geom_table, const double* plane, const uint32_t* plane_exclude, uint32_t n_exclude,
                        const double* hf, const double* heights, const double* solver, uint32_t* collidable_out) {
  if (!gains) return s->fail("null gains table");
  if (n_exclude && !plane_exclude) return s->fail("null plane exclude list");
  ContactSpec cs;
  cs.ground_h = ground_height;
  cs.friction = friction;
  cs.geom = geom_table;
  cs.gains = gains;
  cs.cmode = cmode;
  cs.solver = solver;
  cs.plane = plane;
  cs.exclude = plane_exclude;
  cs.n_exclude = plane ? n_exclude : 0;
  cs.hf = hf;
  cs.heights = heights;
  return set_contact(s, cs, collidable_out);
}
}  // namespace

int phz_enable_contact_terrain(phz_sim* s, double ground_height, double friction, const double* gains,
                               const double* geom_table, const double* plane, const uint32_t* plane_exclude,
                               uint32_t n_exclude, const double* hf, const double* heights, uint32_t* collidable_out) {
  if (!s) return 1;
  return enable_contact_with(s, 0, ground_height, friction, gains, geom_table, plane, plane_exclude, n_exclude, hf,
                             heights, nullptr, collidable_out);
}

int phz_enable_contact_impulse(phz_sim* s, double ground_height, double friction, const double* gains,
                               const double* geom_table, const double* plane, const uint32_t* plane_exclude,
                               uint32_t n_exclude, const double* hf, const double* heights, const double* solver,
                               uint32_t* collidable_out) {
  if (!s) return 1;
  return enable_contact_with(s, 1, ground_height, friction, gains, geom_table, plane, plane_exclude, n_exclude, hf,
                             heights, solver, collidable_out);
}

int phz_set_heightfield(phz_sim* s, const double* hf, const double* heights) {
  if (!s) return 1;
  if (!s->feat.contact) return s->fail("contact not enabled — call enable_contact_terrain first");
  if (!hf) return s->fail("null heightfield");
  int nx = 0, ny = 0;
  if (!check_heightfield(s, hf, heights, nx, ny)) return 1;
  const size_t nodes = (size_t)nx * ny;
  if (s->feat.hf_nx == 0)
    return s->fail("contact was enabled without a heightfield; enable contact with one to use terrain");
  if (nodes > s->hf_cap)
    return s->fail(fmt("heightfield has %zu nodes but the buffer was sized for %zu; enable contact with the largest "
                       "grid first", nodes, s->hf_cap));
  if (!set_device(s)) return 1;
  if (s->stream) hipStreamSynchronize(s->stream);
  s->feat.hf_nx = nx;
  s->feat.hf_ny = ny;
  for (int k = 0; k < 3; k++) s->feat.hf_o[k] = hf[2 + k];
  s->feat.hf_cell = hf[5];
  s->drop_graph();  // the header is a launch argument: re-capture
  return upload_heightfield(s, heights, nodes) ? 0 : 1;
}

int phz_set_contact_sweeps(phz_sim* s, uint32_t sweeps) {
  if (!s) return 1;
  if (sweeps > 1024) return s->fail("contact_sweeps above 1024");
  if (s->feat.sweeps != (int)sweeps) {
    if (!set_device(s)) return 1;
    s->feat.sweeps = (int)sweeps;
    s->invalidate();
  }
  return 0;
}
int phz_contact_sweeps(const phz_sim* s) { return s ? s->feat.sweeps : 0; }

int phz_readback_contact_state(phz_sim* s, double* cs, double* ext) {
  if (!s) return 1;
  if (!s->feat.contact) return s->fail("ground contact not enabled — call enable_ground_contact first");
  if (!cs) return s->fail("null output");
  if (!s->has_device()) return s->fail("host-only sim has no device buffers");
  if (!set_device(s)) return 1;
  const int nb = s->model.nb;
  const size_t W = (size_t)s->nworld;
  std::vector<double> rows(W * nb * 8), imp;
  if (!s->download_rows(s->rows, rows.data(), nb * 8, "readback contact rows")) return 1;
  if (s->imp_buf) {
    imp.resize(W * nb * 48);
    if (!s->download_rows(s->imp_buf, imp.data(), nb * 48, "readback impulses")) return 1;
  }
  for (size_t w = 0; w < W; w++)
    for (int i = 0; i < nb; i++) {
      double* o = cs + (w * nb + i) * 56;
      std::memcpy(o, &rows[(w * nb + i) * 8], 8 * sizeof(double));
      for (int k = 0; k < 48; k++) o[8 + k] = imp.empty() ? 0.0 : imp[(w * nb + i) * 48 + k];
    }
  if (ext) {
    if (s->ext_buf) return s->download_rows(s->ext_buf, ext, nb * 6, "readback contact forces") ? 0 : 1;
    std::memset(ext, 0, W * nb * 6 * sizeof(double));
  }
  return 0;
}

int phz_load_contact_state(phz_sim* s, const double* cs, const double* ext) {
  if (!s) return 1;
  if (!s->feat.contact || s->feat.cmode != 1)
    return s->fail("impulse contact not enabled — call enable_contact_impulse first");
  if (!cs) return s->fail("null contact state");
  if (!s->has_device()) return s->fail("host-only sim has no device buffers");
  if (!set_device(s)) return 1;
  const int nb = s->model.nb;
  const size_t W = (size_t)s->nworld;
  std::vector<double> rows(W * nb * 8), imp(W * nb * 48);
  for (size_t w = 0; w < W; w++)
    for (int i = 0; i < nb; i++) {
      const double* c = cs + (w * nb + i) * 56;
      std::memcpy(&rows[(w * nb + i) * 8], c, 8 * sizeof(double));
      std::memcpy(&imp[(w * nb + i) * 48], c + 8, 48 * sizeof(double));
    }
  if (!s->upload_rows(rows.data(), s->rows, nb * 8, "load contact rows") ||
      !s->upload_rows(imp.data(), s->imp_buf, nb * 48, "load impulses"))
    return 1;
  if (ext && !s->upload_rows(ext, s->ext_buf, nb * 6, "load contact forces")) return 1;
  if (!ext && !s->hip_ok(phz_io_zero(s->ext_buf, (size_t)nb * 6 * s->stride * s->esize(), s->stream), "zero forces"))
    return 1;
  return s->hip_ok(hipStreamSynchronize(s->stream), "load_contact_state") ? 0 : 1;
}

int phz_enable_pd_control(phz_sim* s, const double* dofs, uint32_t n) {
  if (!s) return 1;
  if (n == 0 || !dofs) return s->fail("PD pipeline needs at least one servoed DOF");
  if (!s->feat.acts.empty())
    return s->fail("PD servos write per-DOF controls, but this model's controls drive its actuators");
  for (uint32_t d = 0; d < n; d++) {
    const double* r = dofs + (size_t)d * kPdStride;
    if (!is_int(r[0]) || !is_int(r[1]) || r[0] < 0 || r[1] < 0 || r[0] >= s->model.nq || r[1] >= s->model.nv)
      return s->fail(fmt("PD DOF out of range: q_index %g (nq %d), v_index %g (nv %d)", r[0], s->model.nq, r[1], s->model.nv));
    for (int k = 2; k < 5; k++) if (!std::isfinite(r[k])) return s->fail("PD gains must be finite");
  }
  if (!set_device(s)) return 1;
  const bool same = s->feat.npd == (int)n;
  s->feat.pd.assign(dofs, dofs + (size_t)n * kPdStride);
  // Re-enabling with the same servo count keeps the targets (mod.rs:772-778).
  if (s->has_device() && !same) {
    if (s->targets) { hipFree(s->targets); s->targets = nullptr; }
    if (!s->alloc(&s->targets, (size_t)n * s->stride * s->esize(), "targets alloc")) return 1;
  }
  s->feat.npd = (int)n;
  s->invalidate();
  return 0;
}

int phz_set_position_targets(phz_sim* s, const double* rows) {
  if (!s) return 1;
  if (s->feat.npd == 0) return s->fail("PD control not enabled — call enable_pd_control first");
  if (!rows) return s->fail("null targets");
  if (!s->has_device()) return s->fail("host-only sim has no device buffers");
  if (!set_device(s)) return 1;
  return s->upload_rows(rows, s->targets, s->feat.npd, "upload targets") ? 0 : 1;
}

int phz_enable_control_noise(phz_sim* s, uint64_t seed, int dist, double a, double b, const uint32_t* v_indices,
                             uint32_t n) {
  if (!s) return 1;
  if (dist != PHZ_NOISE_NORMAL && dist != PHZ_NOISE_UNIFORM) return s->fail("unknown noise distribution");
  if (!(std::isfinite(a) && std::isfinite(b))) return s->fail("noise parameters must be finite");
  if (n > 0 && !v_indices) return s->fail("null DOF list");
  std::vector<int> dofs;
  for (uint32_t k = 0; k < n; k++) {
    if (v_indices[k] >= (uint32_t)s->nctrl())
      return s->fail(fmt("noise control %u out of range (%d controls)", v_indices[k], s->nctrl()));
    dofs.push_back((int)v_indices[k]);
  }
  if (!set_device(s)) return 1;
  s->feat.noise = n > 0;
  s->feat.seed = seed;
  s->feat.dist = dist;
  s->feat.a = a;
  s->feat.b = b;
  s->feat.noise_dofs = dofs;
  if (s->has_device() && !s->hip_ok(phz_io_seed(s->rng, seed, s->nworld, s->stream), "seed rng")) return 1;
  s->invalidate();
  return 0;
}

int phz_set_joint_terms(phz_sim* s, const double* table) {
  if (!s) return 1;
  const int nb = s->model.nb;
  std::vector<Features::JointTerm> jt;
  if (table) {
    jt.resize(nb);
    for (int i = 0; i < nb; i++) {
      const double* r = table + (size_t)i * 8;
      for (int k = 0; k < 6; k++)
        if (!std::isfinite(r[k])) return s->fail(fmt("joint terms of body %d: non-finite value in slot %d", i, k));
      if (r[3] < 0 || r[4] < 0 || r[5] < 0)
        return s->fail(fmt("joint terms of body %d: limit stiffness, damping and friction loss must be >= 0", i));
      jt[i] = Features::JointTerm{r[0] != 0.0, r[1], r[2], r[3], r[4], r[5]};
    }
  }
  s->feat.jterms = jt;
  s->invalidate();
  return 0;
}

int phz_set_actuators(phz_sim* s, const double* table, uint32_t n) {
  if (!s) return 1;
  if (n > 0 && !table) return s->fail("null actuator table");
  if (n > 0 && s->feat.npd > 0)
    return s->fail("PD servos write per-DOF controls; a model with actuators cannot also have PD servos");
  std::vector<Features::Act> acts(n);
  for (uint32_t a = 0; a < n; a++) {
    const double* r = table + (size_t)a * 16;
    for (int k = 0; k < 11; k++)
      if (!std::isfinite(r[k])) return s->fail(fmt("actuator %u: non-finite value in slot %d", a, k));
    if (!is_int(r[0]) || r[0] < 0 || r[0] >= s->model.nb)
      return s->fail(fmt("actuator %u: joint %g out of range (%d joints)", a, r[0], s->model.nb));
    const BodyD& b = s->model.b[(int)r[0]];
    if (ndof_of(b.jtype) == 0) return s->fail(fmt("actuator %u drives joint %d, which has no DOF", a, (int)r[0]));
    Features::Act& x = acts[a];
    x.body = (int)r[0]; x.q = b.qoff; x.v = b.voff;
    x.gear = r[1]; x.gain = r[2]; x.bq = r[3]; x.bv = r[4];
    x.cr = r[5] != 0.0; x.clo = std::min(r[6], r[7]); x.chi = std::max(r[6], r[7]);
    x.fr = r[8] != 0.0; x.flo = std::min(r[9], r[10]); x.fhi = std::max(r[9], r[10]);
  }
  const int nctrl = n ? (int)n : s->model.nv;
  if (s->feat.noise)
    for (int d : s->feat.noise_dofs)
      if (d >= nctrl) return s->fail(fmt("noise control %d out of range (%d controls)", d, nctrl));
  if (!set_device(s)) return 1;
  if (s->has_device()) {
    const size_t bytes = (size_t)std::max(nctrl, 1) * s->stride * s->esize();
    if (nctrl > s->ctrl_rows) {
      s->invalidate();
      if (!s->hip_ok(hipStreamSynchronize(s->stream), "actuators sync")) return 1;
      hipFree(s->ctrl);
      s->ctrl = nullptr;
      if (!s->alloc(&s->ctrl, bytes, "ctrl alloc")) return 1;
      s->ctrl_rows = nctrl;
    }
    // Controls change meaning (per DOF <-> per actuator): start from zero.
    if (!s->hip_ok(phz_io_zero(s->ctrl, bytes, s->stream), "zero ctrl") ||
        !s->hip_ok(hipStreamSynchronize(s->stream), "actuators sync"))
      return 1;
  }
  s->feat.acts = acts;
  s->invalidate();
  return 0;
}
int phz_nctrl(const phz_sim* s) { return s ? s->nctrl() : 0; }

int phz_load_states(phz_sim* s, const double* q, const double* v, const double* ctrl) {
  if (!s) return 1;
  if (!q || !v) return s->fail("null q or v");
  if (!s->has_device()) return s->fail("host-only sim has no device buffers");
  if (!set_device(s)) return 1;
  if (!s->upload_rows(q, s->q, s->model.nq, "upload q") || !s->upload_rows(v, s->v, s->model.nv, "upload v")) return 1;
  if (ctrl) {
    if (!s->upload_rows(ctrl, s->ctrl, s->nctrl(), "upload ctrl")) return 1;
  } else if (!s->hip_ok(phz_io_zero(s->ctrl, (size_t)s->nctrl() * s->stride * s->esize(), s->stream), "zero ctrl")) {
    return 1;
  }
  if (s->feat.noise && !s->hip_ok(phz_io_seed(s->rng, s->feat.seed, s->nworld, s->stream), "seed rng")) return 1;
  return s->hip_ok(hipStreamSynchronize(s->stream), "load_states") ? 0 : 1;
}

int phz_set_controls(phz_sim* s, const double* ctrl) {
  if (!s) return 1;
  if (!ctrl) return s->fail("null ctrl");
  if (!s->has_device()) return s->fail("host-only sim has no device buffers");
  if (!set_device(s)) return 1;
  if (!s->upload_rows(ctrl, s->ctrl, s->nctrl(), "upload ctrl")) return 1;
  return s->hip_ok(hipStreamSynchronize(s->stream), "set_controls") ? 0 : 1;
}

int phz_step(phz_sim* s) { return phz_step_many(s, 1); }

int phz_step_many(phz_sim* s, uint32_t n) {
  if (!s) return 1;
  if (!set_device(s)) return 1;
  return s->step_many(n) ? 0 : 1;
}

int phz_set_graphs_enabled(phz_sim* s, int on) {
  if (!s) return 1;
  s->graphs = on != 0;
  if (!s->graphs) s->drop_graph();
  return 0;
}
int phz_graphs_enabled(const phz_sim* s) { return s && s->graphs ? 1 : 0; }

int phz_synchronize(phz_sim* s) {
  if (!s) return 1;
  if (!s->has_device()) return 0;
  if (!set_device(s)) return 1;
  // Poll the stream for up to 200 us before blocking: a blocking wait wakes
  // the host about 10 us after a short span ends.
  const auto t0 = std::chrono::steady_clock::now();
  for (;;) {
    const hipError_t e = hipStreamQuery(s->stream);
    if (e == hipSuccess) return 0;
    if (e != hipErrorNotReady) return s->hip_ok(e, "synchronize") ? 0 : 1;
    if (std::chrono::steady_clock::now() - t0 > std::chrono::microseconds(200)) break;
  }
  return s->hip_ok(hipStreamSynchronize(s->stream), "synchronize") ? 0 : 1;
}

int phz_readback_states(phz_sim* s, double* q, double* v) {
  if (!s) return 1;
  if (!s->has_device()) return s->fail("host-only sim has no device buffers");
  if (!set_device(s)) return 1;
  if (q && !s->download_rows(s->q, q, s->model.nq, "readback q")) return 1;
  if (v && !s->download_rows(s->v, v, s->model.nv, "readback v")) return 1;
  return 0;
}
// phz_readback_states through the library's static per-GPU scratch array
// instead of the sim's staging buffer: no device allocation on any call.
int phz_readback_states_noalloc(phz_sim* s, double* q, double* v) {
  if (!s) return 1;
  if (!s->has_device()) return s->fail("host-only sim has no device buffers");
  if (!set_device(s)) return 1;
  // Every step here (a kernel launch, a pageable device-to-host copy, a
  // stream synchronize) is illegal inside stream capture: refuse it plainly.
  hipStreamCaptureStatus cap_state = hipStreamCaptureStatusNone;
  if (!s->hip_ok(hipStreamIsCapturing(s->stream, &cap_state), "readback_states_noalloc: capture query")) return 1;
  if (cap_state != hipStreamCaptureStatusNone)
    return s->fail("readback_states_noalloc: the sim's stream is capturing a graph; a readback synchronizes and "
                   "cannot be captured");
  void* scr = nullptr;
  size_t cap = 0;
  int dev = -1;
  if (!s->hip_ok(phz_io_scratch(&scr, &cap, &dev), "readback_states_noalloc: scratch lookup")) return 1;
  // One caller at a time per GPU, from staging to the end of the copy out.
  std::lock_guard<std::mutex> use(phz_io_scratch_mutex(dev));
  const int width = std::max(s->model.nq, s->model.nv);
  const size_t need = (size_t)s->nworld * (size_t)width * sizeof(double);
  if (need > cap)
    return s->fail(fmt("readback_states_noalloc: %d worlds x %d values need %zu bytes of staging, above the %zu-byte "
                       "scratch; use phz_readback_states", s->nworld, width, need, cap));
  const std::pair<const void*, double*> parts[2] = {{s->q, q}, {s->v, v}};
  const int widths[2] = {s->model.nq, s->model.nv};
  for (int k = 0; k < 2; k++) {
    if (!parts[k].second || widths[k] <= 0 || s->nworld == 0) continue;
    const size_t bytes = (size_t)s->nworld * widths[k] * sizeof(double);
    if (!s->hip_ok(phz_io_unpack(parts[k].first, (double*)scr, s->nworld, widths[k], s->stride, s->f64 ? 1 : 0,
                                 s->stream), "readback_states_noalloc: unpack") ||
        !s->hip_ok(hipMemcpyAsync(parts[k].second, scr, bytes, hipMemcpyDeviceToHost, s->stream),
                   "readback_states_noalloc: copy") ||
        !s->hip_ok(hipStreamSynchronize(s->stream), "readback_states_noalloc: sync"))
      return 1;
  }
  return 0;
}

int phz_readback_controls(phz_sim* s, double* ctrl) {
  if (!s || !ctrl) return 1;
  if (!s->has_device()) return s->fail("host-only sim has no device buffers");
  if (!set_device(s)) return 1;
  return s->download_rows(s->ctrl, ctrl, s->nctrl(), "readback ctrl") ? 0 : 1;
}
int phz_readback_qdd(phz_sim* s, double* qdd) {
  if (!s || !qdd) return 1;
  if (!s->has_device()) return s->fail("host-only sim has no device buffers");
  if (!set_device(s)) return 1;
  return s->download_rows(s->qdd, qdd, s->model.nv, "readback qdd") ? 0 : 1;
}
int phz_readback_contacts(phz_sim* s, double* rows) {
  if (!s) return 1;
  if (!s->feat.contact) return s->fail("ground contact not enabled — call enable_ground_contact first");
  if (!rows) return s->fail("null output");
  if (!s->has_device()) return s->fail("host-only sim has no device buffers");
  if (!set_device(s)) return 1;
  return s->download_rows(s->rows, rows, s->model.nb * 8, "readback contacts") ? 0 : 1;
}
int phz_readback_rng(phz_sim* s, uint64_t* states) {
  if (!s || !states) return 1;
  if (!s->has_device()) return s->fail("host-only sim has no device buffers");
  if (!set_device(s)) return 1;
  if (!s->hip_ok(hipMemcpyAsync(states, s->rng, (size_t)s->nworld * 8, hipMemcpyDeviceToHost, s->stream), "readback rng"))
    return 1;
  return s->hip_ok(hipStreamSynchronize(s->stream), "readback rng") ? 0 : 1;
}
int phz_load_rng(phz_sim* s, const uint64_t* states) {
  if (!s || !states) return 1;
  if (!s->has_device()) return s->fail("host-only sim has no device buffers");
  if (!set_device(s)) return 1;
  if (!s->hip_ok(hipMemcpyAsync(s->rng, states, (size_t)s->nworld * 8, hipMemcpyHostToDevice, s->stream), "load rng"))
    return 1;
  return s->hip_ok(hipStreamSynchronize(s->stream), "load rng") ? 0 : 1;
}
int phz_collidable_bodies(const phz_sim* s) { return s && s->feat.contact ? s->feat.collidable : 0; }

int phz_compile(phz_sim* s) {
  if (!s) return 1;
  if (!s->compile()) return 1;
  if ((s->kin_on || s->policy_on) && !s->ensure_ctl(false, false)) return 1;
  if (s->policy_on && !s->ensure_ctl(true, false)) return 1;
  return 0;
}

int phz_time_step_many(phz_sim* s, uint32_t n, uint32_t reps, double* ms_per_rep) {
  if (!s || !ms_per_rep) return 1;
  if (n == 0) return s->fail("time_step_many needs at least one step");
  if (s->nworld == 0) return s->fail("time_step_many needs at least one world");
  if (!set_device(s)) return 1;
  bool launch = false;
  if (!s->span_ready(n, launch)) return 1;  // sweeps, device, kernel
  std::vector<hipEvent_t> ev(2 * (size_t)reps);
  for (auto& e : ev)
    if (!s->hip_ok(hipEventCreate(&e), "hipEventCreate")) return 1;
  // Each span's launches go straight to the stream, the first stamping the
  // start event with its own start and the last the stop event with its own
  // end: the time from the first kernel's start to the last one's end.
  bool ok = true;
  for (uint32_t r = 0; r < reps && ok; r++) ok = s->issue(n, ev[2 * r], ev[2 * r + 1]);
  ok = ok && s->hip_ok(hipStreamSynchronize(s->stream), "timing sync");
  for (uint32_t r = 0; r < reps && ok; r++) {
    float ms = 0;
    ok = s->hip_ok(hipEventElapsedTime(&ms, ev[2 * r], ev[2 * r + 1]), "hipEventElapsedTime");
    ms_per_rep[r] = ms;
  }
  for (auto& e : ev) hipEventDestroy(e);
  return ok ? 0 : 1;
}

int phz_lanes_per_world(phz_sim* s) {
  if (!s) return -1;
  if (!s->compile()) return -1;
  return s->lanes;
}

int phz_kernel_info(phz_sim* s, int64_t* info) {
  if (!s || !info) return 1;
  if (!s->compile()) return 1;
  const std::string& log = (s->code2 ? s->code2 : s->code)->log;
  info[0] = remark_value(log, "VGPRs:");
  info[1] = remark_value(log, "AGPRs:");
  info[2] = remark_value(log, "SGPRs:");
  info[3] = remark_value(log, "ScratchSize [bytes/lane]:");
  info[4] = s->block;
  info[5] = s->max_steps;
  return 0;
}


// ── device-resident control loop (mod.rs:1004-1376) ──────────────────────────

int phz_enable_kinematics(phz_sim* s) {
  if (!s) return 1;
  if (!set_device(s)) return 1;
  if (s->has_device() && !s->kin &&
      !s->alloc(&s->kin, (size_t)s->model.nb * PHZ_XF_STRIDE * s->stride * s->esize(), "kinematics alloc"))
    return 1;
  s->kin_on = true;
  return 0;
}

int phz_compute_kinematics(phz_sim* s) {
  if (!s) return 1;
  if (!s->kin_on) return s->fail("kinematics not enabled — call enable_kinematics first");
  if (!s->has_device()) return s->fail("host-only sim (device_ordinal -1) cannot compute kinematics");
  if (!set_device(s)) return 1;
  if (!s->ensure_ctl(false, true)) return 1;
  if (s->nworld == 0) return 0;
  return s->launch_obs(nullptr, true) ? 0 : 1;
}

int phz_readback_kinematics(phz_sim* s, double* rows) {
  if (!s) return 1;
  if (!s->kin_on) return s->fail("kinematics not enabled");
  if (!rows) return s->fail("null output");
  if (!s->has_device()) return s->fail("host-only sim has no device buffers");
  if (!set_device(s)) return 1;
  return s->download_rows(s->kin, rows, s->model.nb * PHZ_XF_STRIDE, "readback kinematics") ? 0 : 1;
}

int phz_enable_policy(phz_sim* s, const double* ops, uint32_t n_in, const double* aux, uint32_t n_aux, uint32_t hidden,
                      const uint32_t* act_slots, uint32_t n_out, double act_clamp, const double* act_clamp_slots,
                      double noise_rho, const double* input_noise, uint32_t history_steps) {
  if (!s) return 1;
  if (s->feat.npd == 0) return s->fail("policy pass needs PD control — call enable_pd_control first");
  if ((n_in && (!ops || !input_noise)) || (n_out && !act_slots) || (n_aux && !aux)) return s->fail("null policy table");
  PolicyD p;
  p.n_in = (int)std::min<uint32_t>(n_in, 1u << 20);
  p.hidden = (int)std::min<uint32_t>(hidden, 1u << 20);
  p.n_out = (int)std::min<uint32_t>(n_out, 1u << 20);
  p.history = (int)std::min<uint32_t>(history_steps, 1u << 30);
  if (n_in <= PHZ_POLICY_MAX_IN) {
    p.ops.assign(ops, ops + (size_t)n_in * PHZ_OBS_OP_STRIDE);
    p.noise.assign(input_noise, input_noise + n_in);
  }
  if (n_aux) p.aux.assign(aux, aux + n_aux);
  if (n_out <= PHZ_POLICY_MAX_OUT) {
    for (uint32_t k = 0; k < n_out; k++) {
      p.slots.push_back((int)std::min<uint32_t>(act_slots[k], 1u << 20));
      p.clamp.push_back(act_clamp_slots ? act_clamp_slots[k] : act_clamp);
    }
  }
  p.rho = noise_rho;
  std::string e;
  if (!validate_policy(p, s->model.nq, s->model.nv, s->model.nb, s->feat.npd, e)) return s->fail(e);
  if (phz_enable_kinematics(s)) return 1;
  if (!set_device(s)) return 1;
  const bool reuse = s->policy_on && s->pol.same_shape(p);
  if (s->stream) hipStreamSynchronize(s->stream);
  if (s->rexec) { hipGraphExecDestroy(s->rexec); s->rexec = nullptr; }
  s->pol = p;
  s->policy_on = true;
  s->ctl_epoch++;
  if (s->has_device() && !reuse) {
    s->free_policy_buffers();
    const size_t S = (size_t)s->stride;
    if (!s->alloc((void**)&s->pw, p.frag_floats() * 4, "policy weights alloc") ||
        !s->alloc((void**)&s->pstd, (size_t)p.n_out * 4, "policy std alloc") ||
        !s->alloc((void**)&s->prng, S * 8, "policy rng alloc") ||
        !s->alloc((void**)&s->pz, (size_t)p.n_out * S * 4, "policy noise state alloc") ||
        !s->alloc(&s->pbase, (size_t)s->feat.npd * S * s->esize(), "base targets alloc") ||
        !s->alloc((void**)&s->obs_hist, (size_t)p.history * p.n_in * S * 4, "observation history alloc") ||
        !s->alloc((void**)&s->out_hist, (size_t)p.history * (p.n_out + 1) * S * 4, "action history alloc")) {
      s->free_policy_buffers();
      s->policy_on = false;
      return 1;
    }
    s->pbase_npd = s->feat.npd;
    if (!s->hip_ok(hipStreamSynchronize(s->stream), "enable_policy")) return 1;
  }
  return 0;
}

int phz_set_policy_weights(phz_sim* s, const double* weights, uint64_t n) {
  if (!s) return 1;
  if (!s->policy_on) return s->fail("policy pass not enabled — call enable_policy first");
  if (n != s->pol.n_weights())
    return s->fail(fmt("policy expects %zu weights, got %llu", s->pol.n_weights(), (unsigned long long)n));
  if (!weights) return s->fail("null weights");
  if (!s->has_device()) return s->fail("host-only sim has no device buffers");
  if (!set_device(s)) return 1;
  std::vector<float> frag;
  policy_fragments(s->pol, weights, frag);
  if (!s->hip_ok(hipMemcpyAsync(s->pw, frag.data(), frag.size() * 4, hipMemcpyHostToDevice, s->stream), "upload weights"))
    return 1;
  return s->hip_ok(hipStreamSynchronize(s->stream), "upload weights") ? 0 : 1;
}

int phz_set_policy_std(phz_sim* s, const double* stdv, uint32_t n) {
  if (!s) return 1;
  if (!s->policy_on) return s->fail("policy pass not enabled — call enable_policy first");
  if ((int)n != s->pol.n_out) return s->fail(fmt("policy has %d actions, got %u stds", s->pol.n_out, n));
  if (!stdv) return s->fail("null std");
  // The reference uploads any value; a Gaussian needs std > 0, and the kernel's
  // log-probability (log std, (a - mean) / std) must stay finite.
  for (uint32_t k = 0; k < n; k++)
    if (!(std::isfinite(stdv[k]) && (float)stdv[k] > 0.0f))
      return s->fail(fmt("policy std %u must be finite and positive, got %g", k, stdv[k]));
  if (!s->has_device()) return s->fail("host-only sim has no device buffers");
  if (!set_device(s)) return 1;
  std::vector<float> f(stdv, stdv + n);
  if (!s->hip_ok(hipMemcpyAsync(s->pstd, f.data(), n * 4, hipMemcpyHostToDevice, s->stream), "upload std")) return 1;
  return s->hip_ok(hipStreamSynchronize(s->stream), "upload std") ? 0 : 1;
}

int phz_set_policy_base_targets(phz_sim* s, const double* rows) {
  if (!s) return 1;
  if (!s->policy_on) return s->fail("policy pass not enabled — call enable_policy first");
  if (!rows) return s->fail("null base targets");
  if (!s->has_device()) return s->fail("host-only sim has no device buffers");
  if (!set_device(s)) return 1;
  if (s->pbase_npd != s->feat.npd) {
    if (s->pbase) hipFree(s->pbase);
    s->pbase = nullptr;
    if (!s->alloc(&s->pbase, (size_t)s->feat.npd * s->stride * s->esize(), "base targets alloc")) return 1;
    s->pbase_npd = s->feat.npd;
  }
  if (!s->upload_rows(rows, s->pbase, s->feat.npd, "upload base targets")) return 1;
  return s->hip_ok(hipStreamSynchronize(s->stream), "set_policy_base_targets") ? 0 : 1;
}

int phz_seed_policy(phz_sim* s, uint64_t seed) {
  if (!s) return 1;
  if (!s->policy_on) return s->fail("policy pass not enabled — call enable_policy first");
  if (!s->has_device()) return s->fail("host-only sim has no device buffers");
  if (!set_device(s)) return 1;
  if (!s->hip_ok(phz_io_seed(s->prng, seed, s->nworld, s->stream), "seed policy") ||
      !s->hip_ok(phz_io_zero(s->pz, (size_t)s->pol.n_out * s->stride * 4, s->stream), "zero noise state"))
    return 1;
  return s->hip_ok(hipStreamSynchronize(s->stream), "seed_policy") ? 0 : 1;
}

int phz_run_policy(phz_sim* s, uint32_t step) {
  if (!s) return 1;
  if (!set_device(s)) return 1;
  if (!s->policy_ready(step)) return 1;
  if (s->nworld == 0) return 0;
  return s->launch_obs(s->obs_row(step), true) && s->launch_policy(step) ? 0 : 1;
}

int phz_readback_policy_history(phz_sim* s, uint32_t start, uint32_t end, double* obs, double* out) {
  if (!s) return 1;
  if (!s->policy_on) return s->fail("policy pass not enabled");
  if (end > (uint32_t)s->pol.history || start > end)
    return s->fail(fmt("policy history range %u..%u outside 0..%d", start, end, s->pol.history));
  if (!s->has_device()) return s->fail("host-only sim has no device buffers");
  if (!set_device(s)) return 1;
  const size_t W = (size_t)s->nworld;
  for (uint32_t k = start; k < end; k++) {
    if (obs && !s->download_rows(s->obs_row(k), obs + (k - start) * W * s->pol.n_in, s->pol.n_in, "readback obs", 0))
      return 1;
    if (out && !s->download_rows(s->out_row(k), out + (k - start) * W * (s->pol.n_out + 1), s->pol.n_out + 1,
                                 "readback actions", 0))
      return 1;
  }
  return 0;
}

int phz_readback_targets(phz_sim* s, double* rows) {
  if (!s) return 1;
  if (s->feat.npd == 0) return s->fail("PD control not enabled");
  if (!rows) return s->fail("null output");
  if (!s->has_device()) return s->fail("host-only sim has no device buffers");
  if (!set_device(s)) return 1;
  return s->download_rows(s->targets, rows, s->feat.npd, "readback targets") ? 0 : 1;
}

int phz_enable_state_history(phz_sim* s, uint32_t slots) {
  if (!s) return 1;
  if (slots == 0) return s->fail("state history needs at least one slot");
  if (slots > (1u << 20)) return s->fail("state history slot count too large");
  if (s->hist_slots == (int)slots) return 0;
  if (!set_device(s)) return 1;
  if (s->has_device()) {
    if (s->stream) hipStreamSynchronize(s->stream);
    if (s->rexec) { hipGraphExecDestroy(s->rexec); s->rexec = nullptr; }
    for (void** p : {&s->hq, &s->hv}) { if (*p) hipFree(*p); *p = nullptr; }
    const size_t E = s->esize(), S = s->stride;
    if (!s->alloc(&s->hq, (size_t)slots * s->model.nq * S * E, "state history alloc") ||
        !s->alloc(&s->hv, (size_t)slots * s->model.nv * S * E, "state history alloc")) {
      s->hist_slots = 0;
      return 1;
    }
  }
  s->hist_slots = (int)slots;
  return 0;
}

int phz_record_state(phz_sim* s, uint32_t slot) {
  if (!s) return 1;
  if (!s->hist_slots) return s->fail("state history not enabled — call enable_state_history first");
  if (slot >= (uint32_t)s->hist_slots) return s->fail(fmt("history slot %u exceeds %d slots", slot, s->hist_slots));
  if (!s->has_device()) return s->fail("host-only sim has no device buffers");
  if (!set_device(s)) return 1;
  return s->record(slot) ? 0 : 1;
}

int phz_readback_state_history(phz_sim* s, uint32_t start, uint32_t end, double* q, double* v) {
  if (!s) return 1;
  if (!s->hist_slots) return s->fail("state history not enabled");
  if (end > (uint32_t)s->hist_slots || start > end)
    return s->fail(fmt("history range %u..%u outside 0..%d", start, end, s->hist_slots));
  if (!s->has_device()) return s->fail("host-only sim has no device buffers");
  if (!set_device(s)) return 1;
  const size_t W = (size_t)s->nworld, E = s->esize(), S = s->stride;
  const int nq = s->model.nq, nv = s->model.nv;
  for (uint32_t k = start; k < end; k++) {
    if (q && !s->download_rows((char*)s->hq + k * nq * S * E, q + (k - start) * W * nq, nq, "readback history q"))
      return 1;
    if (v && !s->download_rows((char*)s->hv + k * nv * S * E, v + (k - start) * W * nv, nv, "readback history v"))
      return 1;
  }
  return 0;
}

int phz_rollout(phz_sim* s, uint32_t first_step, uint32_t n_control, uint32_t control_every, int record_states) {
  if (!s) return 1;
  if (!set_device(s)) return 1;
  return s->rollout(first_step, n_control, control_every, record_states != 0) ? 0 : 1;
}


int phz_time_rollout(phz_sim* s, uint32_t first_step, uint32_t n_control, uint32_t control_every, int record_states,
                     uint32_t reps, double* ms_per_rep) {
  if (!s || !ms_per_rep) return 1;
  if (!set_device(s)) return 1;
  return time_reps(s, reps, ms_per_rep, [&] { return s->rollout(first_step, n_control, control_every, record_states != 0); });
}

int phz_time_control_kernel(phz_sim* s, int which, uint32_t step, uint32_t reps, double* ms_per_rep) {
  if (!s || !ms_per_rep) return 1;
  if (which != 0 && which != 1) return s->fail("kernel must be 0 (observation) or 1 (policy)");
  if (!set_device(s)) return 1;
  if (!s->policy_ready(step)) return 1;
  if (s->nworld == 0) return s->fail("no worlds");
  return time_reps(s, reps, ms_per_rep,
                   [&] { return which == 0 ? s->launch_obs(s->obs_row(step), true) : s->launch_policy(step); });
}

int phz_control_kernel_info(phz_sim* s, int which, int64_t* info) {
  if (!s || !info) return 1;
  if (which != 0 && which != 1) return s->fail("kernel must be 0 (observation) or 1 (policy)");
  if (which == 1 && !s->policy_on) return s->fail("policy pass not enabled — call enable_policy first");
  if (!s->ensure_ctl(which == 1, false)) return 1;
  const std::string& log = (which == 1 ? s->pol_k : s->obs_k).code->log;
  info[0] = remark_value(log, "VGPRs:");
  info[1] = remark_value(log, "AGPRs:");
  info[2] = remark_value(log, "SGPRs:");
  info[3] = remark_value(log, "ScratchSize [bytes/lane]:");
  info[4] = 64;
  info[5] = which == 1 ? 16 * s->pol.cb() : 64;
  return 0;
}

}  // extern "C"
