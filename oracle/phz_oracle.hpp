// phz_oracle.hpp — CPU oracle for the batched rigid-body step.
//
// TEST INFRASTRUCTURE ONLY. Nothing in the product (the HIP library under
// phyz_amd/) includes, links or calls this file. Only tests/, the smoke check
// in __graft_entry__.py and the cpu_baseline leg of bench.py use it, and only
// as the checker.
//
// A scalar-templated f64 restatement of the reference's per-step semantics:
//   * spatial algebra conventions      crates/phyz-math/src/spatial.rs:9-42,
//                                      mirrored explicitly in
//                                      crates/phyz-gpu/cuda/phyz_kernels.cu:110-359
//   * joint maps / motion subspaces    crates/phyz-model/src/joint.rs:253-360
//   * generalized forces               crates/phyz-rigid/src/actuation.rs:18-54,
//                                      crates/phyz-model/src/joint.rs:232-247
//   * ABA (3 passes)                   crates/phyz-rigid/src/aba.rs:117-385
//   * semi-implicit Euler              crates/phyz-rigid/src/integrate.rs:41-92
//   * quat exp/log                     crates/phyz-math/src/lib.rs:43-72
//   * ground penalty contact law       crates/phyz-gpu/cuda/phyz_kernels.cu:542-580,
//                                      691-802, 804-980 (penalty branch 939-965)
//   * PD servo law                     crates/phyz-gpu/src/pd_pipeline.rs:8-13,
//                                      crates/phyz-gpu/cuda/phyz_kernels.cu:464-483
//   * body / geometry / PD tables      crates/phyz-gpu/src/layout.rs:19-93
//   * per-world RNG seed and stream    crates/phyz-gpu/src/policy_pipeline.rs:417-456
//
// Two ABA formulations live here:
//   aba_dense  — follows aba.rs line for line: dense 6x6 SpatialMat algebra,
//                X^T I X as two dense 6x6 products, D recomputed in pass 3.
//   aba_struct — the structure-exploiting formulation the HIP kernels use:
//                symmetric articulated inertias, X^T I X as a rotation then a
//                translation, U / D^-1 / u carried from pass 2 to pass 3,
//                LDL^T for multi-DOF joints. Its operation count (through
//                OpScalar below) is the algorithmic FLOP figure per world-step.
// Independent CRBA + RNEA (Featherstone, RBDA ch. 5-6) cross-check both.
#pragma once

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <type_traits>
#include <vector>

namespace phzo {

// ─────────────────────────────────────────────────────────────────────────────
// Operation-counting scalar. A value is either a model constant (`k`, known
// when the model is uploaded and therefore foldable) or state-dependent. Only
// operations with at least one state-dependent operand are counted, and
// operations with an exact constant 0 or +-1 operand are folded away, so the
// count is what a kernel specialised to the model must execute.
// ─────────────────────────────────────────────────────────────────────────────
struct OpCount {
  uint64_t add = 0, mul = 0, div = 0, sqrt = 0, trans = 0, other = 0;
  uint64_t flops() const { return add + mul + div + sqrt; }
};
inline OpCount*& op_counter() {
  static thread_local OpCount* c = nullptr;
  return c;
}
inline void count_add() { if (op_counter()) op_counter()->add++; }
inline void count_mul() { if (op_counter()) op_counter()->mul++; }
inline void count_div() { if (op_counter()) op_counter()->div++; }
inline void count_sqrt() { if (op_counter()) op_counter()->sqrt++; }
inline void count_trans(int n = 1) { if (op_counter()) op_counter()->trans += n; }
inline void count_other() { if (op_counter()) op_counter()->other++; }

struct OpScalar {
  double v = 0.0;
  bool k = true;  // model constant
  OpScalar() = default;
  OpScalar(double x) : v(x), k(true) {}  // literals and model data are constants
  static OpScalar state(double x) { OpScalar s; s.v = x; s.k = false; return s; }
  explicit operator double() const { return v; }
};
inline bool is_c(const OpScalar& a, double x) { return a.k && a.v == x; }
inline OpScalar operator-(const OpScalar& a) { OpScalar r = a; r.v = -a.v; return r; }
inline OpScalar operator+(const OpScalar& a, const OpScalar& b) {
  if (a.k && b.k) return OpScalar(a.v + b.v);
  if (is_c(a, 0.0)) return b;
  if (is_c(b, 0.0)) return a;
  count_add();
  return OpScalar::state(a.v + b.v);
}
inline OpScalar operator-(const OpScalar& a, const OpScalar& b) {
  if (a.k && b.k) return OpScalar(a.v - b.v);
  if (is_c(b, 0.0)) return a;
  if (is_c(a, 0.0)) return -b;
  count_add();
  return OpScalar::state(a.v - b.v);
}
inline OpScalar operator*(const OpScalar& a, const OpScalar& b) {
  if (a.k && b.k) return OpScalar(a.v * b.v);
  if (is_c(a, 0.0) || is_c(b, 0.0)) return OpScalar(0.0);
  if (is_c(a, 1.0)) return b;
  if (is_c(b, 1.0)) return a;
  if (is_c(a, -1.0)) return -b;
  if (is_c(b, -1.0)) return -a;
  count_mul();
  return OpScalar::state(a.v * b.v);
}
inline OpScalar operator/(const OpScalar& a, const OpScalar& b) {
  if (a.k && b.k) return OpScalar(a.v / b.v);
  if (is_c(a, 0.0)) return OpScalar(0.0);
  if (is_c(b, 1.0)) return a;
  count_div();
  return OpScalar::state(a.v / b.v);
}
inline OpScalar& operator+=(OpScalar& a, const OpScalar& b) { a = a + b; return a; }
inline OpScalar& operator-=(OpScalar& a, const OpScalar& b) { a = a - b; return a; }
inline OpScalar& operator*=(OpScalar& a, const OpScalar& b) { a = a * b; return a; }
inline OpScalar& operator/=(OpScalar& a, const OpScalar& b) { a = a / b; return a; }
inline bool operator<(const OpScalar& a, const OpScalar& b) { return a.v < b.v; }
inline bool operator>(const OpScalar& a, const OpScalar& b) { return a.v > b.v; }
inline bool operator<=(const OpScalar& a, const OpScalar& b) { return a.v <= b.v; }
inline bool operator>=(const OpScalar& a, const OpScalar& b) { return a.v >= b.v; }
inline bool operator==(const OpScalar& a, const OpScalar& b) { return a.v == b.v; }
inline bool operator!=(const OpScalar& a, const OpScalar& b) { return a.v != b.v; }

// Scalar math dispatch: plain floating types use <cmath>; OpScalar counts.
inline double s_val(double x) { return x; }
inline float s_val(float x) { return x; }
inline double s_val(const OpScalar& x) { return x.v; }

inline double s_sqrt(double x) { return std::sqrt(x); }
inline float s_sqrt(float x) { return std::sqrt(x); }
inline OpScalar s_sqrt(const OpScalar& x) {
  if (x.k) return OpScalar(std::sqrt(x.v));
  count_sqrt();
  return OpScalar::state(std::sqrt(x.v));
}
inline double s_sin(double x) { return std::sin(x); }
inline double s_cos(double x) { return std::cos(x); }
inline double s_atan2(double y, double x) { return std::atan2(y, x); }
inline double s_log(double x) { return std::log(x); }
inline float s_sin(float x) { return std::sin(x); }
inline float s_cos(float x) { return std::cos(x); }
inline float s_atan2(float y, float x) { return std::atan2(y, x); }
inline float s_log(float x) { return std::log(x); }
// sin and cos of one argument share range reduction: one transcendental
// evaluation for the pair.
inline void s_sincos(double x, double* s, double* c) { *s = std::sin(x); *c = std::cos(x); }
inline void s_sincos(float x, float* s, float* c) { *s = std::sin(x); *c = std::cos(x); }
inline OpScalar s_sin(const OpScalar& x) {
  if (x.k) return OpScalar(std::sin(x.v));
  count_trans();
  return OpScalar::state(std::sin(x.v));
}
inline OpScalar s_cos(const OpScalar& x) {
  if (x.k) return OpScalar(std::cos(x.v));
  count_trans();
  return OpScalar::state(std::cos(x.v));
}
inline void s_sincos(const OpScalar& x, OpScalar* s, OpScalar* c) {
  if (x.k) { *s = OpScalar(std::sin(x.v)); *c = OpScalar(std::cos(x.v)); return; }
  count_trans();
  *s = OpScalar::state(std::sin(x.v));
  *c = OpScalar::state(std::cos(x.v));
}
inline OpScalar s_atan2(const OpScalar& y, const OpScalar& x) {
  if (y.k && x.k) return OpScalar(std::atan2(y.v, x.v));
  count_trans();
  return OpScalar::state(std::atan2(y.v, x.v));
}
inline OpScalar s_log(const OpScalar& x) {
  if (x.k) return OpScalar(std::log(x.v));
  count_trans();
  return OpScalar::state(std::log(x.v));
}
inline double s_tanh(double x) { return std::tanh(x); }
inline float s_tanh(float x) { return std::tanh(x); }
inline OpScalar s_tanh(const OpScalar& x) {
  if (x.k) return OpScalar(std::tanh(x.v));
  count_trans();
  return OpScalar::state(std::tanh(x.v));
}
template <class S> inline S s_abs(const S& x) {
  if constexpr (std::is_same<S, OpScalar>::value) { if (!x.k) count_other(); OpScalar r = x; r.v = std::fabs(x.v); return r; }
  else return std::fabs(x);
}
template <class S> inline S s_max(const S& a, const S& b) {
  if constexpr (std::is_same<S, OpScalar>::value) {
    if (a.k && b.k) return OpScalar(std::max(a.v, b.v));
    count_other();
    return OpScalar::state(a.v > b.v ? a.v : b.v);
  } else return a > b ? a : b;
}
template <class S> inline S s_min(const S& a, const S& b) {
  if constexpr (std::is_same<S, OpScalar>::value) {
    if (a.k && b.k) return OpScalar(std::min(a.v, b.v));
    count_other();
    return OpScalar::state(a.v < b.v ? a.v : b.v);
  } else return a < b ? a : b;
}
template <class S> inline S s_clamp(const S& x, const S& lo, const S& hi) { return s_min(s_max(x, lo), hi); }

template <class S> constexpr double s_eps();
template <> constexpr double s_eps<double>() { return std::numeric_limits<double>::epsilon(); }
template <> constexpr double s_eps<OpScalar>() { return std::numeric_limits<double>::epsilon(); }
// The f32 device path uses 1e-6 as its small-angle threshold
// (crates/phyz-gpu/cuda/phyz_kernels.cu:248-253, 281-287).
template <> constexpr double s_eps<float>() { return 1e-6; }

// ─────────────────────────────────────────────────────────────────────────────
// 3-vectors, 3x3 matrices (row-major), spatial vectors [angular; linear]
// ─────────────────────────────────────────────────────────────────────────────
template <class S> struct V3 {
  S x, y, z;
  V3() : x(0.0), y(0.0), z(0.0) {}
  V3(S a, S b, S c) : x(a), y(b), z(c) {}
  S& operator[](int i) { return i == 0 ? x : (i == 1 ? y : z); }
  const S& operator[](int i) const { return i == 0 ? x : (i == 1 ? y : z); }
};
template <class S> V3<S> operator+(const V3<S>& a, const V3<S>& b) { return {a.x + b.x, a.y + b.y, a.z + b.z}; }
template <class S> V3<S> operator-(const V3<S>& a, const V3<S>& b) { return {a.x - b.x, a.y - b.y, a.z - b.z}; }
template <class S> V3<S> operator-(const V3<S>& a) { return {-a.x, -a.y, -a.z}; }
template <class S> V3<S> operator*(const V3<S>& a, const S& s) { return {a.x * s, a.y * s, a.z * s}; }
template <class S> S dot(const V3<S>& a, const V3<S>& b) { return a.x * b.x + a.y * b.y + a.z * b.z; }
template <class S> V3<S> cross(const V3<S>& a, const V3<S>& b) {
  return {a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x};
}
template <class S> S norm(const V3<S>& a) { return s_sqrt(dot(a, a)); }

template <class S> struct M3 {
  S m[3][3];
  M3() { for (int i = 0; i < 3; i++) for (int j = 0; j < 3; j++) m[i][j] = S(0.0); }
  static M3 identity() { M3 r; r.m[0][0] = S(1.0); r.m[1][1] = S(1.0); r.m[2][2] = S(1.0); return r; }
};
template <class S> M3<S> operator*(const M3<S>& a, const M3<S>& b) {
  M3<S> r;
  for (int i = 0; i < 3; i++)
    for (int j = 0; j < 3; j++) r.m[i][j] = a.m[i][0] * b.m[0][j] + a.m[i][1] * b.m[1][j] + a.m[i][2] * b.m[2][j];
  return r;
}
template <class S> V3<S> operator*(const M3<S>& a, const V3<S>& v) {
  return {a.m[0][0] * v.x + a.m[0][1] * v.y + a.m[0][2] * v.z,
          a.m[1][0] * v.x + a.m[1][1] * v.y + a.m[1][2] * v.z,
          a.m[2][0] * v.x + a.m[2][1] * v.y + a.m[2][2] * v.z};
}
template <class S> M3<S> operator+(const M3<S>& a, const M3<S>& b) {
  M3<S> r; for (int i = 0; i < 3; i++) for (int j = 0; j < 3; j++) r.m[i][j] = a.m[i][j] + b.m[i][j]; return r;
}
template <class S> M3<S> operator-(const M3<S>& a, const M3<S>& b) {
  M3<S> r; for (int i = 0; i < 3; i++) for (int j = 0; j < 3; j++) r.m[i][j] = a.m[i][j] - b.m[i][j]; return r;
}
template <class S> M3<S> operator*(const M3<S>& a, const S& s) {
  M3<S> r; for (int i = 0; i < 3; i++) for (int j = 0; j < 3; j++) r.m[i][j] = a.m[i][j] * s; return r;
}
template <class S> M3<S> transpose(const M3<S>& a) {
  M3<S> r; for (int i = 0; i < 3; i++) for (int j = 0; j < 3; j++) r.m[i][j] = a.m[j][i]; return r;
}
template <class S> V3<S> tmul(const M3<S>& a, const V3<S>& v) {  // a^T v
  return {a.m[0][0] * v.x + a.m[1][0] * v.y + a.m[2][0] * v.z,
          a.m[0][1] * v.x + a.m[1][1] * v.y + a.m[2][1] * v.z,
          a.m[0][2] * v.x + a.m[1][2] * v.y + a.m[2][2] * v.z};
}
template <class S> M3<S> skew(const V3<S>& a) {
  M3<S> r;
  r.m[0][1] = -a.z; r.m[0][2] = a.y;
  r.m[1][0] = a.z;  r.m[1][2] = -a.x;
  r.m[2][0] = -a.y; r.m[2][1] = a.x;
  return r;
}

template <class S> struct SV {
  V3<S> ang, lin;
  S get(int i) const { return i < 3 ? ang[i] : lin[i - 3]; }
  void set(int i, S x) { if (i < 3) ang[i] = x; else lin[i - 3] = x; }
};
template <class S> SV<S> operator+(const SV<S>& a, const SV<S>& b) { return {a.ang + b.ang, a.lin + b.lin}; }
template <class S> SV<S> operator-(const SV<S>& a, const SV<S>& b) { return {a.ang - b.ang, a.lin - b.lin}; }
template <class S> SV<S> operator*(const SV<S>& a, const S& s) { return {a.ang * s, a.lin * s}; }
template <class S> S dot(const SV<S>& a, const SV<S>& b) { return dot(a.ang, b.ang) + dot(a.lin, b.lin); }
// v x m (motion cross motion), v x* f (motion cross force): spatial.rs / phyz_kernels.cu:111-124.
template <class S> SV<S> cross_motion(const SV<S>& v, const SV<S>& m) {
  return {cross(v.ang, m.ang), cross(v.ang, m.lin) + cross(v.lin, m.ang)};
}
template <class S> SV<S> cross_force(const SV<S>& v, const SV<S>& f) {
  return {cross(v.ang, f.ang) + cross(v.lin, f.lin), cross(v.ang, f.lin)};
}

// Dense 6x6 spatial matrix in four 3x3 blocks, as tang's SpatialMat.
template <class S> struct SM {
  M3<S> ul, ur, ll, lr;
  S get(int i, int j) const {
    const M3<S>& b = i < 3 ? (j < 3 ? ul : ur) : (j < 3 ? ll : lr);
    return b.m[i % 3][j % 3];
  }
  void set(int i, int j, S x) {
    M3<S>& b = i < 3 ? (j < 3 ? ul : ur) : (j < 3 ? ll : lr);
    b.m[i % 3][j % 3] = x;
  }
};
template <class S> SM<S> operator+(const SM<S>& a, const SM<S>& b) { return {a.ul + b.ul, a.ur + b.ur, a.ll + b.ll, a.lr + b.lr}; }
template <class S> SM<S> operator-(const SM<S>& a, const SM<S>& b) { return {a.ul - b.ul, a.ur - b.ur, a.ll - b.ll, a.lr - b.lr}; }
template <class S> SM<S> operator*(const SM<S>& a, const S& s) { return {a.ul * s, a.ur * s, a.ll * s, a.lr * s}; }
template <class S> SV<S> mul(const SM<S>& a, const SV<S>& v) {
  return {a.ul * v.ang + a.ur * v.lin, a.ll * v.ang + a.lr * v.lin};
}
template <class S> SM<S> mul(const SM<S>& a, const SM<S>& b) {
  return {a.ul * b.ul + a.ur * b.ll, a.ul * b.ur + a.ur * b.lr, a.ll * b.ul + a.lr * b.ll, a.ll * b.ur + a.lr * b.lr};
}
template <class S> SM<S> transpose(const SM<S>& a) { return {transpose(a.ul), transpose(a.ll), transpose(a.ur), transpose(a.lr)}; }
template <class S> SM<S> outer(const SV<S>& a, const SV<S>& b) {
  SM<S> r;
  for (int i = 0; i < 6; i++) for (int j = 0; j < 6; j++) r.set(i, j, a.get(i) * b.get(j));
  return r;
}

// Plucker transform {rot E, pos r}: spatial.rs:24-35, phyz_kernels.cu:292-320.
template <class S> struct Xf {
  M3<S> rot;
  V3<S> pos;
  static Xf identity() { return {M3<S>::identity(), V3<S>()}; }
};
// a.compose(b): rot = a.rot b.rot, pos = b.pos + b.rot^T a.pos (phyz_kernels.cu:292-298)
template <class S> Xf<S> compose(const Xf<S>& a, const Xf<S>& b) { return {a.rot * b.rot, b.pos + tmul(b.rot, a.pos)}; }
// X v = [E w; E (v - r x w)]
template <class S> SV<S> apply_motion(const Xf<S>& x, const SV<S>& v) {
  return {x.rot * v.ang, x.rot * (v.lin - cross(x.pos, v.ang))};
}
// X^T f = [E^T tau + r x E^T f; E^T f]
template <class S> SV<S> inv_apply_force(const Xf<S>& x, const SV<S>& f) {
  V3<S> rf = tmul(x.rot, f.lin);
  return {tmul(x.rot, f.ang) + cross(x.pos, rf), rf};
}
// Motion matrix [E, 0; -E r x, E] (phyz_kernels.cu:180-200)
template <class S> SM<S> motion_matrix(const Xf<S>& x) {
  SM<S> r;
  r.ul = x.rot;
  r.lr = x.rot;
  r.ll = (x.rot * skew(x.pos)) * S(-1.0);
  return r;
}

// Quaternion (w, x, y, z), Hamilton product (phyz_kernels.cu:260-289).
template <class S> struct Q { S w, x, y, z; };
template <class S> Q<S> qmul(const Q<S>& a, const Q<S>& b) {
  return {a.w * b.w - a.x * b.x - a.y * b.y - a.z * b.z,
          a.w * b.x + a.x * b.w + a.y * b.z - a.z * b.y,
          a.w * b.y - a.x * b.z + a.y * b.w + a.z * b.x,
          a.w * b.z + a.x * b.y - a.y * b.x + a.z * b.w};
}
template <class S> Q<S> qnormalize(const Q<S>& q) {
  S n = s_sqrt(q.w * q.w + q.x * q.x + q.y * q.y + q.z * q.z);
  return {q.w / n, q.x / n, q.y / n, q.z / n};
}
// quat_exp: phyz-math/src/lib.rs:43-59
template <class S> Q<S> quat_exp(const V3<S>& w) {
  S angle = norm(w);
  if (angle < S(s_eps<S>())) return {S(1.0), w.x * S(0.5), w.y * S(0.5), w.z * S(0.5)};
  S s, c;
  s_sincos(angle * S(0.5), &s, &c);
  S f = s / angle;
  return {c, w.x * f, w.y * f, w.z * f};
}
// quat_log: phyz-math/src/lib.rs:65-72
template <class S> V3<S> quat_log(const Q<S>& q) {
  V3<S> v{q.x, q.y, q.z};
  S n = norm(v);
  if (n < S(s_eps<S>())) return v * S(2.0);
  S angle = S(2.0) * s_atan2(n, q.w);
  return v * (angle / n);
}
template <class S> M3<S> quat_to_matrix(const Q<S>& q) {
  M3<S> r;
  S w = q.w, x = q.x, y = q.y, z = q.z;
  r.m[0][0] = S(1.0) - S(2.0) * (y * y + z * z); r.m[0][1] = S(2.0) * (x * y - w * z); r.m[0][2] = S(2.0) * (x * z + w * y);
  r.m[1][0] = S(2.0) * (x * y + w * z); r.m[1][1] = S(1.0) - S(2.0) * (x * x + z * z); r.m[1][2] = S(2.0) * (y * z - w * x);
  r.m[2][0] = S(2.0) * (x * z - w * y); r.m[2][1] = S(2.0) * (y * z + w * x); r.m[2][2] = S(1.0) - S(2.0) * (x * x + y * y);
  return r;
}
// Rotate p by unit q: p + w t + u x t, t = 2 u x p (phyz_kernels.cu:284-289)
template <class S> V3<S> qrotate(const Q<S>& q, const V3<S>& p) {
  V3<S> u{q.x, q.y, q.z};
  V3<S> t = cross(u, p) * S(2.0);
  return p + t * q.w + cross(u, t);
}

// ─────────────────────────────────────────────────────────────────────────────
// Model: the f64 body table with layout.rs:19-38 slot meanings.
// ─────────────────────────────────────────────────────────────────────────────
enum JType { J_REVOLUTE = 0, J_PRISMATIC = 1, J_FIXED = 2, J_BALL = 3, J_FREE = 4 };
enum GType { G_NONE = 0, G_SPHERE = 1, G_BOX = 2, G_CAPSULE = 3, G_CYLINDER = 4, G_MESH = 5 };
constexpr int BODY_STRIDE = 36;
constexpr int GEOM_STRIDE = 24;
constexpr int PD_STRIDE = 8;
constexpr int CONTACT_ROW = 8;
constexpr int MAX_BODIES = 32;

inline int joint_ndof(int jt) { return jt == J_FIXED ? 0 : (jt == J_BALL ? 3 : (jt == J_FREE ? 6 : 1)); }

struct Body {
  int parent, jtype, qoff, voff;
  double mass, com[3], inertia[6];  // inertia about COM: xx yy zz xy xz yz
  double ptj_rot[9], ptj_pos[3], axis[3];
  double damping, stiffness, spring_ref, armature;
};
// Joint terms of the reference's CPU model that its device body table does not
// carry (crates/phyz-model/src/joint.rs:27-72): the soft position limit and dry
// friction of a one-DOF joint.
struct JointTerms {
  bool limited = false;
  double lo = 0.0, hi = 0.0;
  double limit_k = 1000.0, limit_d = 60.0;  // DEFAULT_LIMIT_STIFFNESS / _DAMPING (joint.rs:96-104)
  double friction_loss = 0.0;
};
// An actuator driving the first DOF of one joint (crates/phyz-model/src/model.rs:18-82).
struct Actuator {
  int body = 0, qidx = 0, vidx = 0;
  double gear = 1.0, gain = 1.0, bias_q = 0.0, bias_v = 0.0;
  bool has_ctrl_range = false, has_force_range = false;
  double ctrl_lo = 0.0, ctrl_hi = 0.0, force_lo = 0.0, force_hi = 0.0;
};
struct Geom {
  int type;
  double p[6];            // [1..7): shape parameters / mesh AABB
  bool skip_plane;        // [7]: never contacts the body-attached plane
  double k, d;            // per-body penalty gains
  double o_pos[3], o_rot[9];
};
// Contact configuration beyond the flat-ground penalty law: the fields of
// ContactParams (crates/phyz-gpu/src/contact_pipeline.rs:17-100) with the
// defaults of GroundContactParams::default (197-222).
struct ContactCfg {
  int solve_mode = 0;  // 0 penalty, 1 velocity-level impulse solve
  int sweeps = 16;     // [contact, ABA] sweeps per step in impulse mode (DEFAULT_CONTACT_SWEEPS)
  double restitution = 0.0, restitution_threshold = 0.05;
  double erp = 0.001 / (2.0 * 0.02 + 0.001), margin = 0.001;
  double solimp_dmin = 0.9, solimp_dmax = 0.95, solimp_width = 0.001, solimp_mid = 0.5, solimp_power = 2.0;
  int plane_body = -1;  // body-attached contact plane (contact_pipeline.rs:300-353)
  double plane_offset = 0.0, plane_max_depth = 0.0, plane_half_x = 0.0, plane_half_y = 0.0;
  int hf_nx = 0, hf_ny = 0;  // heightfield terrain; nx == 0 is the flat plane at ground_h
  double hf_ox = 0.0, hf_oy = 0.0, hf_oz = 0.0, hf_cell = 1.0;
  std::vector<double> hf;  // heights[iy * nx + ix]
};
constexpr int CS_STRIDE = 56;      // contact state per body: 8 readback + 24 ground + 24 plane impulses
constexpr int CS_IMPULSE_OFF = 8;
constexpr int CS_PLANE_OFF = 32;
struct PdDof { int q_index, v_index; double kp, kd, max_force; };
enum NoiseDist { NOISE_NORMAL = 0, NOISE_UNIFORM = 1 };

struct Model {
  int nb = 0, nq = 0, nv = 0;
  std::vector<Body> bodies;
  double gravity[3] = {0, 0, -9.81};
  double dt = 1e-3;
  // contact
  bool contact = false;
  double ground_h = 0.0, mu = 0.0;
  std::vector<Geom> geoms;
  ContactCfg cc;
  // PD servos
  std::vector<PdDof> pd;
  // per-step control noise (the synthetic torque stream of the benchmark workloads)
  bool noise = false;
  uint64_t noise_seed = 0;
  int noise_dist = NOISE_NORMAL;
  double noise_a = 0.0, noise_b = 1.0;
  std::vector<int> noise_dofs;
  // limits, friction loss (per body; empty: none) and actuators (empty: ctrl is
  // a per-DOF generalized force, otherwise one control per actuator)
  std::vector<JointTerms> jterms;
  std::vector<Actuator> acts;
  int nctrl() const { return acts.empty() ? nv : (int)acts.size(); }
};

// Unpack a body table; returns an error string or "" on success.
inline const char* model_from_table(Model& m, const double* t, int nb, int nq, int nv, const double g[3], double dt) {
  if (nb <= 0 || nb > MAX_BODIES) return "body count out of range";
  m.nb = nb; m.nq = nq; m.nv = nv; m.dt = dt;
  for (int k = 0; k < 3; k++) m.gravity[k] = g[k];
  m.bodies.resize(nb);
  for (int i = 0; i < nb; i++) {
    const double* r = t + i * BODY_STRIDE;
    Body& b = m.bodies[i];
    b.parent = (int)r[0]; b.jtype = (int)r[1]; b.qoff = (int)r[2]; b.voff = (int)r[3];
    b.mass = r[4];
    for (int k = 0; k < 3; k++) b.com[k] = r[5 + k];
    for (int k = 0; k < 6; k++) b.inertia[k] = r[8 + k];
    for (int k = 0; k < 9; k++) b.ptj_rot[k] = r[14 + k];
    for (int k = 0; k < 3; k++) b.ptj_pos[k] = r[23 + k];
    for (int k = 0; k < 3; k++) b.axis[k] = r[26 + k];
    b.damping = r[29]; b.stiffness = r[30]; b.spring_ref = r[31]; b.armature = r[32];
    if (b.parent >= i || b.parent < -1) return "bodies must be topologically ordered (parent < child)";
    if (b.jtype < 0 || b.jtype > 4) return "unknown joint type";
    int nd = joint_ndof(b.jtype);
    if (b.qoff + nd > nq || b.voff + nd > nv) return "joint offsets exceed nq/nv";
  }
  if (nq != nv) return "nq must equal nv (exponential-coordinate ball/free joints)";
  return "";
}
inline void geoms_from_table(Model& m, const double* t) {
  m.geoms.resize(m.nb);
  for (int i = 0; i < m.nb; i++) {
    const double* r = t + i * GEOM_STRIDE;
    Geom& g = m.geoms[i];
    g.type = (int)r[0];
    for (int k = 0; k < 6; k++) g.p[k] = r[1 + k];
    g.skip_plane = r[7] != 0.0;
    g.k = r[8]; g.d = r[9];
    for (int k = 0; k < 3; k++) g.o_pos[k] = r[10 + k];
    for (int k = 0; k < 9; k++) g.o_rot[k] = r[13 + k];
  }
}

template <class S> V3<S> cv3(const double* a) { return {S(a[0]), S(a[1]), S(a[2])}; }
template <class S> M3<S> cm3(const double* a) {
  M3<S> r; for (int i = 0; i < 3; i++) for (int j = 0; j < 3; j++) r.m[i][j] = S(a[i * 3 + j]); return r;
}

// SpatialInertia::to_matrix: [[Ic + m[c]x[c]x^T, m[c]x], [m[c]x^T, m 1]]
template <class S> SM<S> rigid_inertia(const Body& b) {
  S m = S(b.mass);
  V3<S> c = cv3<S>(b.com);
  M3<S> ic;
  ic.m[0][0] = S(b.inertia[0]); ic.m[1][1] = S(b.inertia[1]); ic.m[2][2] = S(b.inertia[2]);
  ic.m[0][1] = ic.m[1][0] = S(b.inertia[3]);
  ic.m[0][2] = ic.m[2][0] = S(b.inertia[4]);
  ic.m[1][2] = ic.m[2][1] = S(b.inertia[5]);
  M3<S> cx = skew(c);
  SM<S> r;
  r.ul = ic + (cx * transpose(cx)) * m;
  r.ur = cx * m;
  r.ll = transpose(cx) * m;
  r.lr = M3<S>::identity() * m;
  return r;
}

// Joint transform (joint.rs:253-315): revolute Rodrigues at -q, prismatic
// axis*q, ball/free exp(w)^T (+ pos for free).
template <class S> Xf<S> joint_transform(const Body& b, const S* q) {
  Xf<S> x = Xf<S>::identity();
  switch (b.jtype) {
    case J_REVOLUTE: {
      S s, c;
      s_sincos(-q[b.qoff], &s, &c);
      M3<S> K = skew(cv3<S>(b.axis));
      x.rot = M3<S>::identity() + K * s + (K * K) * (S(1.0) - c);
      break;
    }
    case J_PRISMATIC: x.pos = cv3<S>(b.axis) * q[b.qoff]; break;
    case J_BALL: {
      V3<S> w{q[b.qoff], q[b.qoff + 1], q[b.qoff + 2]};
      x.rot = transpose(quat_to_matrix(quat_exp(w)));
      break;
    }
    case J_FREE: {
      V3<S> w{q[b.qoff], q[b.qoff + 1], q[b.qoff + 2]};
      x.rot = transpose(quat_to_matrix(quat_exp(w)));
      x.pos = V3<S>{q[b.qoff + 3], q[b.qoff + 4], q[b.qoff + 5]};
      break;
    }
    default: break;
  }
  return x;
}
template <class S> Xf<S> tree_transform(const Body& b, const S* q) {
  Xf<S> ptj{cm3<S>(b.ptj_rot), cv3<S>(b.ptj_pos)};
  return compose(joint_transform(b, q), ptj);
}
// Column k of the motion subspace (joint.rs:326-360).
template <class S> SV<S> subspace_col(const Body& b, int k) {
  SV<S> s;
  if (b.jtype == J_REVOLUTE) s.ang = cv3<S>(b.axis);
  else if (b.jtype == J_PRISMATIC) s.lin = cv3<S>(b.axis);
  else if (b.jtype == J_BALL || b.jtype == J_FREE) s.set(k, S(1.0));
  return s;
}
template <class S> SV<S> joint_velocity(const Body& b, const S* v) {
  SV<S> r;
  int nd = joint_ndof(b.jtype);
  for (int k = 0; k < nd; k++) r = r + subspace_col<S>(b, k) * v[b.voff + k];
  return r;
}

// Generalized force (actuation.rs:18-39 with no actuators): ctrl passes
// through per DOF, plus passive -damping*qd on every DOF and the spring
// -k(q - q_ref) on single-DOF joints (joint.rs:232-247). Limits and
// friction_loss are not representable in the body table, so they are zero.
// Soft joint-limit force of a one-DOF joint (joint.rs:196-226): a one-sided
// spring-damper on the violation depth whose damping only resists motion
// deeper into the limit.
template <class S> S limit_force(const JointTerms& t, const S& q, const S& qd) {
  if (!t.limited) return S(0.0);
  S depth, sign;
  if (q < S(t.lo)) { depth = S(t.lo) - q; sign = S(1.0); }
  else if (q > S(t.hi)) { depth = q - S(t.hi); sign = S(-1.0); }
  else return S(0.0);
  S inward = s_max(S(0.0) - sign * qd, S(0.0));
  return sign * (S(t.limit_k) * depth + S(t.limit_d) * inward);
}
// Actuator law f = gear (gain clamp(ctrl) + bias_q q + bias_v v), then the
// force range (model.rs:57-82).
template <class S> S actuator_force(const Actuator& a, const S& ctrl, const S& q, const S& v) {
  S c = ctrl;
  if (a.has_ctrl_range) c = s_clamp(c, S(std::min(a.ctrl_lo, a.ctrl_hi)), S(std::max(a.ctrl_lo, a.ctrl_hi)));
  S f = S(a.gear) * (S(a.gain) * c + S(a.bias_q) * q + S(a.bias_v) * v);
  if (a.has_force_range) f = s_clamp(f, S(std::min(a.force_lo, a.force_hi)), S(std::max(a.force_lo, a.force_hi)));
  return f;
}
// qfrc = actuator forces (or ctrl per DOF without actuators, model.rs:175-231)
// + the passive terms of each DOF (actuation.rs:18-39, joint.rs:232-247):
// damping, and on one-DOF joints the spring, the soft limit and the dry
// friction -f_loss tanh(qd / 1e-3).
template <class S> void generalized_forces(const Model& m, const S* q, const S* v, const S* ctrl, S* qfrc) {
  if (m.acts.empty()) {
    for (int j = 0; j < m.nv; j++) qfrc[j] = ctrl[j];
  } else {
    for (int j = 0; j < m.nv; j++) qfrc[j] = S(0.0);
    for (size_t a = 0; a < m.acts.size(); a++) {
      const Actuator& A = m.acts[a];
      qfrc[A.vidx] = qfrc[A.vidx] + actuator_force(A, ctrl[a], q[A.qidx], v[A.vidx]);
    }
  }
  for (int i = 0; i < m.nb; i++) {
    const Body& b = m.bodies[i];
    int nd = joint_ndof(b.jtype);
    for (int k = 0; k < nd; k++) {
      S f = -(S(b.damping) * v[b.voff + k]);
      if (nd == 1) {
        f = f - S(b.stiffness) * (q[b.qoff] - S(b.spring_ref));
        if (!m.jterms.empty()) {
          const JointTerms& t = m.jterms[i];
          f = f + limit_force(t, q[b.qoff], v[b.voff]);
          if (t.friction_loss > 0.0) f = f - S(t.friction_loss) * s_tanh(v[b.voff] / S(1e-3));
        }
      }
      qfrc[b.voff + k] = qfrc[b.voff + k] + f;
    }
  }
}

// Small dense inverse, Gauss-Jordan with partial pivoting (row-major n x n).
// Singular (pivot magnitude < 1e-20) returns false: the reference's
// invert_small (phyz_kernels.cu:382-419); tang-la's try_inverse plays the
// same role on the CPU (aba.rs:256-259).
template <class S> bool invert_small(S* a, int n) {
  S inv[36];
  for (int r = 0; r < n; r++) for (int c = 0; c < n; c++) inv[r * n + c] = S(r == c ? 1.0 : 0.0);
  for (int col = 0; col < n; col++) {
    int piv = col;
    S best = s_abs(a[col * n + col]);
    for (int r = col + 1; r < n; r++) { S x = s_abs(a[r * n + col]); if (x > best) { best = x; piv = r; } }
    if (best < S(1e-20)) return false;
    if (piv != col)
      for (int c = 0; c < n; c++) { std::swap(a[col * n + c], a[piv * n + c]); std::swap(inv[col * n + c], inv[piv * n + c]); }
    S d = a[col * n + col];
    for (int c = 0; c < n; c++) { a[col * n + c] = a[col * n + c] / d; inv[col * n + c] = inv[col * n + c] / d; }
    for (int r = 0; r < n; r++) {
      if (r == col) continue;
      S f = a[r * n + col];
      if (f == S(0.0)) continue;
      for (int c = 0; c < n; c++) { a[r * n + c] = a[r * n + c] - f * a[col * n + c]; inv[r * n + c] = inv[r * n + c] - f * inv[col * n + c]; }
    }
  }
  for (int i = 0; i < n * n; i++) a[i] = inv[i];
  return true;
}

// ─────────────────────────────────────────────────────────────────────────────
// aba_dense: crates/phyz-rigid/src/aba.rs:117-368, line for line.
// ext (nullable) is nb spatial forces in body frame.
// ─────────────────────────────────────────────────────────────────────────────
template <class S> void aba_dense(const Model& m, const S* q, const S* v, const S* ctrl, const SV<S>* ext, S* qdd) {
  const int nb = m.nb;
  std::vector<S> qfrc(m.nv);
  generalized_forces(m, q, v, ctrl, qfrc.data());
  std::vector<Xf<S>> xt(nb);
  std::vector<SV<S>> vel(nb), cb(nb), pa(nb), acc(nb);
  std::vector<SM<S>> ia(nb);
  SV<S> a0;
  a0.lin = V3<S>{S(-m.gravity[0]), S(-m.gravity[1]), S(-m.gravity[2])};
  for (int j = 0; j < m.nv; j++) qdd[j] = S(0.0);

  for (int i = 0; i < nb; i++) {  // pass 1 (aba.rs:141-178)
    const Body& b = m.bodies[i];
    xt[i] = tree_transform<S>(b, q);
    SV<S> vj = joint_velocity<S>(b, v);
    if (b.parent < 0) { vel[i] = vj; cb[i] = SV<S>(); }
    else { vel[i] = apply_motion(xt[i], vel[b.parent]) + vj; cb[i] = cross_motion(vel[i], vj); }
    ia[i] = rigid_inertia<S>(b);
    pa[i] = cross_force(vel[i], mul(ia[i], vel[i]));
    if (ext) pa[i] = pa[i] - ext[i];
  }
  for (int i = nb - 1; i >= 0; i--) {  // pass 2 (aba.rs:181-285)
    const Body& b = m.bodies[i];
    int nd = joint_ndof(b.jtype);
    S imp = S(m.dt) * S(b.damping);
    if (nd == 0) {
      if (b.parent >= 0) {
        SM<S> xm = motion_matrix(xt[i]);
        ia[b.parent] = ia[b.parent] + mul(mul(transpose(xm), ia[i]), xm);
        pa[b.parent] = pa[b.parent] + inv_apply_force(xt[i], pa[i]);
      }
      continue;
    }
    if (nd == 1) {
      SV<S> s = subspace_col<S>(b, 0);
      S u = qfrc[b.voff] - dot(s, pa[i]);
      S d = dot(s, mul(ia[i], s)) + S(b.armature) + imp;
      if (s_abs(d) < S(1e-20)) continue;
      S uid = u / d;
      SV<S> ias = mul(ia[i], s);
      if (b.parent >= 0) {
        SM<S> inew = ia[i] - outer(ias, mul(ia[i], s)) * (S(1.0) / d);
        SV<S> pnew = pa[i] + mul(inew, cb[i]) + ias * uid;
        SM<S> xm = motion_matrix(xt[i]);
        ia[b.parent] = ia[b.parent] + mul(mul(transpose(xm), inew), xm);
        pa[b.parent] = pa[b.parent] + inv_apply_force(xt[i], pnew);
      }
    } else {
      S U[36], D[36], u[6];
      for (int k = 0; k < nd; k++) {
        SV<S> sk = subspace_col<S>(b, k);
        SV<S> uk = mul(ia[i], sk);
        for (int r = 0; r < 6; r++) U[r * nd + k] = uk.get(r);
        u[k] = qfrc[b.voff + k] - dot(sk, pa[i]);
      }
      for (int r = 0; r < nd; r++)
        for (int c = 0; c < nd; c++) {
          SV<S> sr = subspace_col<S>(b, r);
          S acc0 = S(0.0);
          for (int t = 0; t < 6; t++) acc0 = acc0 + sr.get(t) * U[t * nd + c];
          D[r * nd + c] = acc0;
        }
      for (int k = 0; k < nd; k++) D[k * nd + k] = D[k * nd + k] + S(b.armature) + imp;
      if (!invert_small(D, nd)) continue;
      if (b.parent >= 0) {
        S UD[36];
        for (int r = 0; r < 6; r++)
          for (int c = 0; c < nd; c++) {
            S s0 = S(0.0);
            for (int k = 0; k < nd; k++) s0 = s0 + U[r * nd + k] * D[k * nd + c];
            UD[r * nd + c] = s0;
          }
        SM<S> inew = ia[i];
        for (int r = 0; r < 6; r++)
          for (int c = 0; c < 6; c++) {
            S s0 = S(0.0);
            for (int k = 0; k < nd; k++) s0 = s0 + UD[r * nd + k] * U[c * nd + k];
            inew.set(r, c, inew.get(r, c) - s0);
          }
        S du[6];
        for (int r = 0; r < nd; r++) { S s0 = S(0.0); for (int k = 0; k < nd; k++) s0 = s0 + D[r * nd + k] * u[k]; du[r] = s0; }
        SV<S> udu;
        for (int r = 0; r < 6; r++) { S s0 = S(0.0); for (int k = 0; k < nd; k++) s0 = s0 + U[r * nd + k] * du[k]; udu.set(r, s0); }
        SV<S> pnew = pa[i] + (mul(inew, cb[i]) + udu);
        SM<S> xm = motion_matrix(xt[i]);
        ia[b.parent] = ia[b.parent] + mul(mul(transpose(xm), inew), xm);
        pa[b.parent] = pa[b.parent] + inv_apply_force(xt[i], pnew);
      }
    }
  }
  for (int i = 0; i < nb; i++) {  // pass 3 (aba.rs:288-365)
    const Body& b = m.bodies[i];
    int nd = joint_ndof(b.jtype);
    S imp = S(m.dt) * S(b.damping);
    SV<S> ap = b.parent < 0 ? apply_motion(xt[i], a0) : apply_motion(xt[i], acc[b.parent]);
    if (nd == 0) { acc[i] = ap + cb[i]; continue; }
    if (nd == 1) {
      SV<S> s = subspace_col<S>(b, 0);
      S d = dot(s, mul(ia[i], s)) + S(b.armature) + imp;
      if (s_abs(d) < S(1e-20)) { acc[i] = ap + cb[i]; continue; }
      S u = qfrc[b.voff] - dot(s, pa[i]);
      S x = (u - dot(mul(ia[i], ap + cb[i]), s)) / d;
      qdd[b.voff] = x;
      acc[i] = ap + cb[i] + s * x;
    } else {
      S U[36], D[36], u[6];
      for (int k = 0; k < nd; k++) {
        SV<S> sk = subspace_col<S>(b, k);
        SV<S> uk = mul(ia[i], sk);
        for (int r = 0; r < 6; r++) U[r * nd + k] = uk.get(r);
      }
      for (int r = 0; r < nd; r++)
        for (int c = 0; c < nd; c++) {
          SV<S> sr = subspace_col<S>(b, r);
          S acc0 = S(0.0);
          for (int t = 0; t < 6; t++) acc0 = acc0 + sr.get(t) * U[t * nd + c];
          D[r * nd + c] = acc0;
        }
      for (int k = 0; k < nd; k++) D[k * nd + k] = D[k * nd + k] + S(b.armature) + imp;
      if (!invert_small(D, nd)) { acc[i] = ap + cb[i]; continue; }
      for (int k = 0; k < nd; k++) u[k] = qfrc[b.voff + k] - dot(subspace_col<S>(b, k), pa[i]);
      SV<S> at = ap + cb[i];
      SV<S> iat = mul(ia[i], at);
      S rhs[6];
      for (int k = 0; k < nd; k++) rhs[k] = u[k] - dot(subspace_col<S>(b, k), iat);
      SV<S> a_new = at;
      for (int k = 0; k < nd; k++) {
        S x = S(0.0);
        for (int j = 0; j < nd; j++) x = x + D[k * nd + j] * rhs[j];
        qdd[b.voff + k] = x;
        a_new = a_new + subspace_col<S>(b, k) * x;
      }
      acc[i] = a_new;
    }
  }
}

// ─────────────────────────────────────────────────────────────────────────────
// aba_struct: the kernels' formulation (same equations, structure exploited).
//   symmetric articulated inertia: blocks A (ul, symmetric), B (ur), C (lr, symmetric)
//   X^T I X = T^T (R^T I R) T, T = [1 0; -r x 1]:
//       A' = E^T A E, B' = E^T B E, C' = E^T C E
//       B'' = B' + r x C',  A'' = A' - B' r x + r x B''^T,  C'' = C'
//   multi-DOF D solved by LDL^T (D is SPD for a physical inertia)
// ─────────────────────────────────────────────────────────────────────────────
template <class S> struct SymI {  // symmetric 6x6 in blocks
  S a[6];    // A upper triangle: 00 01 02 11 12 22
  S b[9];    // B full, row-major
  S c[6];    // C upper triangle
};
inline int sidx(int i, int j) {  // 3x3 symmetric upper-triangle index
  if (i > j) std::swap(i, j);
  return i == 0 ? j : (i == 1 ? 2 + j : 5);
}
template <class S> S sym_get(const SymI<S>& I, int i, int j) {
  if (i < 3 && j < 3) return I.a[sidx(i, j)];
  if (i >= 3 && j >= 3) return I.c[sidx(i - 3, j - 3)];
  if (i < 3) return I.b[i * 3 + (j - 3)];
  return I.b[j * 3 + (i - 3)];
}
template <class S> SymI<S> sym_from(const SM<S>& m) {
  SymI<S> r;
  for (int i = 0; i < 3; i++) for (int j = i; j < 3; j++) { r.a[sidx(i, j)] = m.ul.m[i][j]; r.c[sidx(i, j)] = m.lr.m[i][j]; }
  for (int i = 0; i < 3; i++) for (int j = 0; j < 3; j++) r.b[i * 3 + j] = m.ur.m[i][j];
  return r;
}
template <class S> SV<S> sym_mul(const SymI<S>& I, const SV<S>& v) {
  SV<S> r;
  for (int i = 0; i < 6; i++) {
    S s0 = S(0.0);
    for (int j = 0; j < 6; j++) s0 = s0 + sym_get(I, i, j) * v.get(j);
    r.set(i, s0);
  }
  return r;
}
// E^T M E for symmetric M (upper triangle in, upper triangle out)
template <class S> void sym_rot(const S* m, const M3<S>& E, S* out) {
  S T[3][3];  // T = M E
  for (int i = 0; i < 3; i++)
    for (int j = 0; j < 3; j++) T[i][j] = m[sidx(i, 0)] * E.m[0][j] + m[sidx(i, 1)] * E.m[1][j] + m[sidx(i, 2)] * E.m[2][j];
  for (int i = 0; i < 3; i++)
    for (int j = i; j < 3; j++) out[sidx(i, j)] = E.m[0][i] * T[0][j] + E.m[1][i] * T[1][j] + E.m[2][i] * T[2][j];
}
template <class S> SymI<S> sym_xtix(const SymI<S>& I, const Xf<S>& X) {
  const M3<S>& E = X.rot;
  SymI<S> r;
  S A1[6], C1[6];
  sym_rot(I.a, E, A1);
  sym_rot(I.c, E, C1);
  S T[3][3], B1[3][3];  // B1 = E^T B E
  for (int i = 0; i < 3; i++)
    for (int j = 0; j < 3; j++) T[i][j] = I.b[i * 3 + 0] * E.m[0][j] + I.b[i * 3 + 1] * E.m[1][j] + I.b[i * 3 + 2] * E.m[2][j];
  for (int i = 0; i < 3; i++)
    for (int j = 0; j < 3; j++) B1[i][j] = E.m[0][i] * T[0][j] + E.m[1][i] * T[1][j] + E.m[2][i] * T[2][j];
  const V3<S>& p = X.pos;
  // rx C1 column by column: (r x C)_{:,j} = r x C_{:,j}
  S B2[3][3];
  for (int j = 0; j < 3; j++) {
    V3<S> cj{C1[sidx(0, j)], C1[sidx(1, j)], C1[sidx(2, j)]};
    V3<S> rc = cross(p, cj);
    B2[0][j] = B1[0][j] + rc.x; B2[1][j] = B1[1][j] + rc.y; B2[2][j] = B1[2][j] + rc.z;
  }
  // A2 = A1 - B1 rx + rx B2^T ; (B1 rx)_{ij} = -(r x B1_{i,:})_j ; (rx B2^T)_{ij} = (r x B2_{j,:})_i
  V3<S> rb1[3], rb2[3];
  for (int i = 0; i < 3; i++) {
    rb1[i] = cross(p, V3<S>{B1[i][0], B1[i][1], B1[i][2]});
    rb2[i] = cross(p, V3<S>{B2[i][0], B2[i][1], B2[i][2]});
  }
  for (int i = 0; i < 3; i++)
    for (int j = i; j < 3; j++) r.a[sidx(i, j)] = A1[sidx(i, j)] + rb1[i][j] + rb2[j][i];
  for (int i = 0; i < 3; i++) for (int j = 0; j < 3; j++) r.b[i * 3 + j] = B2[i][j];
  for (int k = 0; k < 6; k++) r.c[k] = C1[k];
  return r;
}
template <class S> SymI<S> sym_add(const SymI<S>& x, const SymI<S>& y) {
  SymI<S> r;
  for (int k = 0; k < 6; k++) { r.a[k] = x.a[k] + y.a[k]; r.c[k] = x.c[k] + y.c[k]; }
  for (int k = 0; k < 9; k++) r.b[k] = x.b[k] + y.b[k];
  return r;
}

// What a second solve with other external forces can reuse (q, v, ctrl fixed):
// transforms, velocities, bias forces, the joint factorizations and I_a c.
template <class S> struct AbaCache {
  std::vector<S> qfrc;
  std::vector<Xf<S>> xt;
  std::vector<SV<S>> vel, cb, bias, iac;
  struct JointSolve { S U[36]; S L[36]; S Dd[6]; S u[6]; bool ok; };  // Dd holds 1/d_j
  std::vector<JointSolve> js;
};

// The structure-exploiting ABA (same equations as aba.rs:117-368): symmetric
// articulated inertias, X^T I X as rotate-then-translate, LDL^T joint solves.
// Fills `c` for aba_delta.
template <class S>
void aba_factor(const Model& m, const S* q, const S* v, const S* ctrl, const SV<S>* ext, S* qdd, AbaCache<S>& c) {
  const int nb = m.nb;
  c.qfrc.assign(m.nv, S(0.0));
  std::vector<S>& qfrc = c.qfrc;
  generalized_forces(m, q, v, ctrl, qfrc.data());
  c.xt.assign(nb, Xf<S>());
  c.vel.assign(nb, SV<S>());
  c.cb.assign(nb, SV<S>());
  c.bias.assign(nb, SV<S>());
  c.iac.assign(nb, SV<S>());
  c.js.assign(nb, typename AbaCache<S>::JointSolve());
  std::vector<Xf<S>>& xt = c.xt;
  std::vector<SV<S>>& vel = c.vel;
  std::vector<SV<S>>& cb = c.cb;
  std::vector<SV<S>> pa(nb), acc(nb);
  std::vector<SymI<S>> ia(nb);
  auto& js = c.js;
  SV<S> a0;
  a0.lin = V3<S>{S(-m.gravity[0]), S(-m.gravity[1]), S(-m.gravity[2])};
  for (int j = 0; j < m.nv; j++) qdd[j] = S(0.0);

  for (int i = 0; i < nb; i++) {
    const Body& b = m.bodies[i];
    xt[i] = tree_transform<S>(b, q);
    SV<S> vj = joint_velocity<S>(b, v);
    if (b.parent < 0) { vel[i] = vj; cb[i] = SV<S>(); }
    else { vel[i] = apply_motion(xt[i], vel[b.parent]) + vj; cb[i] = cross_motion(vel[i], vj); }
    SM<S> I = rigid_inertia<S>(b);
    pa[i] = cross_force(vel[i], mul(I, vel[i]));
    c.bias[i] = pa[i];
    if (ext) pa[i] = pa[i] - ext[i];
    ia[i] = sym_from(I);
  }
  for (int i = nb - 1; i >= 0; i--) {
    const Body& b = m.bodies[i];
    int nd = joint_ndof(b.jtype);
    auto& J = js[i];
    J.ok = true;
    SymI<S> Ia = ia[i];
    SV<S> pA = pa[i];
    if (nd > 0) {
      S imp = S(m.dt) * S(b.damping);
      // U = I_A S (6 x nd, column-major by DOF), D = S^T U + diag
      for (int k = 0; k < nd; k++) {
        SV<S> uk = sym_mul(ia[i], subspace_col<S>(b, k));
        for (int r = 0; r < 6; r++) J.U[k * 6 + r] = uk.get(r);
        J.u[k] = qfrc[b.voff + k] - dot(subspace_col<S>(b, k), pa[i]);
      }
      S D[36];
      for (int r = 0; r < nd; r++)
        for (int c = 0; c <= r; c++) {
          SV<S> sr = subspace_col<S>(b, r);
          S s0 = S(0.0);
          for (int t = 0; t < 6; t++) s0 = s0 + sr.get(t) * J.U[c * 6 + t];
          D[r * nd + c] = s0;
        }
      for (int k = 0; k < nd; k++) D[k * nd + k] = D[k * nd + k] + S(b.armature) + imp;
      // LDL^T: D = L diag(d) L^T, L unit lower (row-major, below diagonal).
      // E[r][j] = L[r][j] d_j is kept so each update is one multiply-add.
      S dpiv[6], E[36];
      for (int j = 0; j < nd && J.ok; j++) {
        S dj = D[j * nd + j];
        for (int k = 0; k < j; k++) dj = dj - J.L[j * nd + k] * E[j * nd + k];
        if (s_abs(dj) < S(1e-20)) { J.ok = false; break; }
        dpiv[j] = dj;
        J.Dd[j] = S(1.0) / dj;
        for (int r = j + 1; r < nd; r++) {
          S erj = D[r * nd + j];
          for (int k = 0; k < j; k++) erj = erj - J.L[r * nd + k] * E[j * nd + k];
          E[r * nd + j] = erj;
          J.L[r * nd + j] = erj * J.Dd[j];
        }
      }
      (void)dpiv;
      if (!J.ok) continue;  // singular: no propagation (aba.rs:210-212, 256-259)
      if (b.parent < 0) continue;
      // W = U D^-1 (solve per row of U): W^T = D^-1 U^T
      S W[36];
      for (int r = 0; r < 6; r++) {
        S y[6];
        for (int k = 0; k < nd; k++) { y[k] = J.U[k * 6 + r]; for (int t = 0; t < k; t++) y[k] = y[k] - J.L[k * nd + t] * y[t]; }
        for (int k = 0; k < nd; k++) y[k] = y[k] * J.Dd[k];
        for (int k = nd - 1; k >= 0; k--) for (int t = k + 1; t < nd; t++) y[k] = y[k] - J.L[t * nd + k] * y[t];
        for (int k = 0; k < nd; k++) W[k * 6 + r] = y[k];
      }
      // Ia = I_A - W U^T (symmetric)
      for (int r = 0; r < 3; r++)
        for (int c = r; c < 3; c++) {
          S s0 = S(0.0), s1 = S(0.0);
          for (int k = 0; k < nd; k++) { s0 = s0 + W[k * 6 + r] * J.U[k * 6 + c]; s1 = s1 + W[k * 6 + 3 + r] * J.U[k * 6 + 3 + c]; }
          Ia.a[sidx(r, c)] = Ia.a[sidx(r, c)] - s0;
          Ia.c[sidx(r, c)] = Ia.c[sidx(r, c)] - s1;
        }
      for (int r = 0; r < 3; r++)
        for (int c = 0; c < 3; c++) {
          S s0 = S(0.0);
          for (int k = 0; k < nd; k++) s0 = s0 + W[k * 6 + r] * J.U[k * 6 + 3 + c];
          Ia.b[r * 3 + c] = Ia.b[r * 3 + c] - s0;
        }
      // pa = p_A + Ia c + W u
      SV<S> wu;
      for (int r = 0; r < 6; r++) { S s0 = S(0.0); for (int k = 0; k < nd; k++) s0 = s0 + W[k * 6 + r] * J.u[k]; wu.set(r, s0); }
      c.iac[i] = sym_mul(Ia, cb[i]);
      pA = pA + c.iac[i] + wu;
    } else if (b.parent < 0) {
      continue;
    }
    ia[b.parent] = sym_add(ia[b.parent], sym_xtix(Ia, xt[i]));
    pa[b.parent] = pa[b.parent] + inv_apply_force(xt[i], pA);
  }
  for (int i = 0; i < nb; i++) {
    const Body& b = m.bodies[i];
    int nd = joint_ndof(b.jtype);
    SV<S> ap = apply_motion(xt[i], b.parent < 0 ? a0 : acc[b.parent]) + cb[i];
    const auto& J = js[i];
    if (nd == 0 || !J.ok) { acc[i] = ap; continue; }
    S y[6];
    for (int k = 0; k < nd; k++) {
      S uta = S(0.0);
      for (int t = 0; t < 6; t++) uta = uta + J.U[k * 6 + t] * ap.get(t);
      y[k] = J.u[k] - uta;
      for (int t = 0; t < k; t++) y[k] = y[k] - J.L[k * nd + t] * y[t];
    }
    for (int k = 0; k < nd; k++) y[k] = y[k] * J.Dd[k];
    for (int k = nd - 1; k >= 0; k--) for (int t = k + 1; t < nd; t++) y[k] = y[k] - J.L[t * nd + k] * y[t];
    for (int k = 0; k < nd; k++) { qdd[b.voff + k] = y[k]; ap = ap + subspace_col<S>(b, k) * y[k]; }
    acc[i] = ap;
  }
}

template <class S> void aba_struct(const Model& m, const S* q, const S* v, const S* ctrl, const SV<S>* ext, S* qdd) {
  AbaCache<S> c;
  aba_factor(m, q, v, ctrl, ext, qdd, c);
}

// The ABA's response dqdd to a change dext of the external forces with q, v,
// ctrl fixed: the solve is affine in the forces, so qdd(ext0 + dext) =
// qdd(ext0) + dqdd. Passes 2 and 3 run on the force change alone with the
// cached factorization: dp_A = -dext, du = -S^T dp_A, dp_a = dp_A + U D^-1 du;
// da = X da_parent (zero at the root), dqdd = D^-1 (du - U^T da), da += S dqdd.
template <class S> void aba_delta(const Model& m, AbaCache<S>& c, const SV<S>* dext, S* dqdd) {
  const int nb = m.nb;
  std::vector<SV<S>> pa(nb), acc(nb);
  for (int i = 0; i < nb; i++) pa[i] = SV<S>() - dext[i];
  for (int i = nb - 1; i >= 0; i--) {
    const Body& b = m.bodies[i];
    const int nd = joint_ndof(b.jtype);
    auto& J = c.js[i];
    SV<S> pA = pa[i];
    if (nd > 0) {
      for (int k = 0; k < nd; k++) J.u[k] = S(0.0) - dot(subspace_col<S>(b, k), pa[i]);
      if (!J.ok || b.parent < 0) continue;
      S y[6];
      for (int k = 0; k < nd; k++) { y[k] = J.u[k]; for (int t = 0; t < k; t++) y[k] = y[k] - J.L[k * nd + t] * y[t]; }
      for (int k = 0; k < nd; k++) y[k] = y[k] * J.Dd[k];
      for (int k = nd - 1; k >= 0; k--) for (int t = k + 1; t < nd; t++) y[k] = y[k] - J.L[t * nd + k] * y[t];
      SV<S> wu;
      for (int r = 0; r < 6; r++) { S s0 = S(0.0); for (int k = 0; k < nd; k++) s0 = s0 + J.U[k * 6 + r] * y[k]; wu.set(r, s0); }
      pA = pA + wu;
    } else if (b.parent < 0) {
      continue;
    }
    pa[b.parent] = pa[b.parent] + inv_apply_force(c.xt[i], pA);
  }
  for (int i = 0; i < nb; i++) {
    const Body& b = m.bodies[i];
    const int nd = joint_ndof(b.jtype);
    SV<S> ap = b.parent < 0 ? SV<S>() : apply_motion(c.xt[i], acc[b.parent]);
    const auto& J = c.js[i];
    if (nd == 0) { acc[i] = ap; continue; }
    if (!J.ok) { for (int k = 0; k < nd; k++) dqdd[b.voff + k] = S(0.0); acc[i] = ap; continue; }
    S y[6];
    for (int k = 0; k < nd; k++) {
      S uta = S(0.0);
      for (int t = 0; t < 6; t++) uta = uta + J.U[k * 6 + t] * ap.get(t);
      y[k] = J.u[k] - uta;
      for (int t = 0; t < k; t++) y[k] = y[k] - J.L[k * nd + t] * y[t];
    }
    for (int k = 0; k < nd; k++) y[k] = y[k] * J.Dd[k];
    for (int k = nd - 1; k >= 0; k--) for (int t = k + 1; t < nd; t++) y[k] = y[k] - J.L[t * nd + k] * y[t];
    for (int k = 0; k < nd; k++) { dqdd[b.voff + k] = y[k]; ap = ap + subspace_col<S>(b, k) * y[k]; }
    acc[i] = ap;
  }
}

// ─────────────────────────────────────────────────────────────────────────────
// Independent referee: CRBA (joint-space inertia) + RNEA (inverse dynamics),
// Featherstone RBDA tables 5.1 and 6.2. M includes armature and the implicit
// damping term dt*c on the diagonal, as aba.rs:207-208, 247-249 add them to D.
// ─────────────────────────────────────────────────────────────────────────────
template <class S> void rnea(const Model& m, const S* q, const S* v, const S* qdd, const SV<S>* ext, S* tau) {
  const int nb = m.nb;
  std::vector<Xf<S>> xt(nb);
  std::vector<SV<S>> vel(nb), acc(nb), f(nb);
  SV<S> a0;
  a0.lin = V3<S>{S(-m.gravity[0]), S(-m.gravity[1]), S(-m.gravity[2])};
  for (int i = 0; i < nb; i++) {
    const Body& b = m.bodies[i];
    xt[i] = tree_transform<S>(b, q);
    SV<S> vj = joint_velocity<S>(b, v);
    SV<S> aj = joint_velocity<S>(b, qdd);
    SV<S> vp = b.parent < 0 ? SV<S>() : vel[b.parent];
    SV<S> ap = b.parent < 0 ? a0 : acc[b.parent];
    vel[i] = apply_motion(xt[i], vp) + vj;
    acc[i] = apply_motion(xt[i], ap) + aj + cross_motion(vel[i], vj);
    SM<S> I = rigid_inertia<S>(b);
    f[i] = mul(I, acc[i]) + cross_force(vel[i], mul(I, vel[i]));
    if (ext) f[i] = f[i] - ext[i];
  }
  for (int j = 0; j < m.nv; j++) tau[j] = S(0.0);
  for (int i = nb - 1; i >= 0; i--) {
    const Body& b = m.bodies[i];
    int nd = joint_ndof(b.jtype);
    for (int k = 0; k < nd; k++) tau[b.voff + k] = dot(subspace_col<S>(b, k), f[i]);
    if (b.parent >= 0) f[b.parent] = f[b.parent] + inv_apply_force(xt[i], f[i]);
  }
}
template <class S> void crba(const Model& m, const S* q, S* M /* nv x nv row-major */) {
  const int nb = m.nb, nv = m.nv;
  std::vector<Xf<S>> xt(nb);
  std::vector<SM<S>> ic(nb);
  for (int i = 0; i < nb; i++) { xt[i] = tree_transform<S>(m.bodies[i], q); ic[i] = rigid_inertia<S>(m.bodies[i]); }
  for (int i = 0; i < nv * nv; i++) M[i] = S(0.0);
  for (int i = nb - 1; i >= 0; i--) {
    const Body& b = m.bodies[i];
    if (b.parent >= 0) {
      SM<S> xm = motion_matrix(xt[i]);
      ic[b.parent] = ic[b.parent] + mul(mul(transpose(xm), ic[i]), xm);
    }
  }
  for (int i = 0; i < nb; i++) {
    const Body& b = m.bodies[i];
    int nd = joint_ndof(b.jtype);
    for (int k = 0; k < nd; k++) {
      SV<S> F = mul(ic[i], subspace_col<S>(b, k));
      for (int kk = 0; kk < nd; kk++) M[(b.voff + k) * nv + b.voff + kk] = dot(subspace_col<S>(b, kk), F);
      int j = i;
      while (m.bodies[j].parent >= 0) {
        F = inv_apply_force(xt[j], F);
        j = m.bodies[j].parent;
        const Body& bj = m.bodies[j];
        int ndj = joint_ndof(bj.jtype);
        for (int kk = 0; kk < ndj; kk++) {
          S h = dot(subspace_col<S>(bj, kk), F);
          M[(b.voff + k) * nv + bj.voff + kk] = h;
          M[(bj.voff + kk) * nv + b.voff + k] = h;
        }
      }
    }
  }
  for (const Body& b : m.bodies) {
    int nd = joint_ndof(b.jtype);
    for (int k = 0; k < nd; k++) M[(b.voff + k) * nv + b.voff + k] = M[(b.voff + k) * nv + b.voff + k] + S(b.armature) + S(m.dt) * S(b.damping);
  }
}

// ─────────────────────────────────────────────────────────────────────────────
// Forward kinematics and ground penalty contact (phyz_kernels.cu:748-980,
// penalty branch 939-965; contact_eff_mass 545-571; caps 574-578).
// ─────────────────────────────────────────────────────────────────────────────
template <class S> struct FK {
  M3<S> w_rot;   // body -> world
  V3<S> w_pos;   // body origin in world
  SV<S> vel;     // body-frame spatial velocity
};
template <class S> void forward_kinematics(const Model& m, const S* q, const S* v, FK<S>* out) {
  for (int i = 0; i < m.nb; i++) {
    const Body& b = m.bodies[i];
    Xf<S> x = tree_transform<S>(b, q);
    SV<S> vj = joint_velocity<S>(b, v);
    M3<S> rt = transpose(x.rot);
    if (b.parent < 0) { out[i].w_rot = rt; out[i].w_pos = x.pos; out[i].vel = vj; }
    else {
      const FK<S>& p = out[b.parent];
      out[i].w_rot = p.w_rot * rt;
      out[i].w_pos = p.w_pos + p.w_rot * x.pos;
      out[i].vel = apply_motion(x, p.vel) + vj;
    }
  }
}
// Body velocities for other joint velocities at the same q: the tree
// transforms (and out[].w_rot / w_pos) are reused.
template <class S> void fk_velocity(const Model& m, const std::vector<Xf<S>>& xt, const S* v, FK<S>* out) {
  for (int i = 0; i < m.nb; i++) {
    const Body& b = m.bodies[i];
    SV<S> vj = joint_velocity<S>(b, v);
    out[i].vel = b.parent < 0 ? vj : apply_motion(xt[i], out[b.parent].vel) + vj;
  }
}
inline double fsign(double x) { return x > 0.0 ? 1.0 : (x < 0.0 ? -1.0 : 0.0); }
template <class S> S ssign(const S& x) { return S(fsign(s_val(x))); }

template <class S> V3<S> inertia_solve(const Body& b, const V3<S>& w) {
  double xx = b.inertia[0], yy = b.inertia[1], zz = b.inertia[2], xy = b.inertia[3], xz = b.inertia[4], yz = b.inertia[5];
  double c00 = yy * zz - yz * yz, c01 = xz * yz - xy * zz, c02 = xy * yz - xz * yy;
  double det = xx * c00 + xy * c01 + xz * c02;
  if (std::fabs(det) < 1e-20) return V3<S>();
  double c11 = xx * zz - xz * xz, c12 = xy * xz - xx * yz, c22 = xx * yy - xy * xy;
  double inv = 1.0 / det;
  return {S(inv * c00) * w.x + S(inv * c01) * w.y + S(inv * c02) * w.z,
          S(inv * c01) * w.x + S(inv * c11) * w.y + S(inv * c12) * w.z,
          S(inv * c02) * w.x + S(inv * c12) * w.y + S(inv * c22) * w.z};
}
template <class S> S contact_eff_mass(const Body& b, const V3<S>& r, const V3<S>& u) {
  if (b.mass <= 0.0) return S(1e30);
  V3<S> rc = r - cv3<S>(b.com);
  V3<S> a = cross(rc, u);
  S ang = s_max(dot(a, inertia_solve(b, a)), S(0.0));
  return S(1.0) / (S(1.0 / b.mass) + ang);
}
template <class S> S max_damping(const S& meff, double dt) { return meff / S(std::max(dt, 1e-9)); }
template <class S> S max_stiffness(const S& meff, double dt) { double d = std::max(dt, 1e-9); return S(4.0) * meff / S(d * d); }

// Support point of body i's shape against body-frame direction n (phyz_kernels.cu:691-725)
template <class S> V3<S> support_point(const Geom& g, const V3<S>& n_body) {
  M3<S> o_r = cm3<S>(g.o_rot);
  V3<S> o_p = cv3<S>(g.o_pos);
  V3<S> n = o_r * n_body;
  V3<S> s;
  if (g.type == G_SPHERE) s = n * S(-g.p[0]);
  else if (g.type == G_BOX) s = V3<S>{S(-g.p[0]) * ssign(n.x), S(-g.p[1]) * ssign(n.y), S(-g.p[2]) * ssign(n.z)};
  else if (g.type == G_CAPSULE) s = V3<S>{S(0.0), S(0.0), S(-g.p[1] * 0.5) * ssign(n.z)} - n * S(g.p[0]);
  else if (g.type == G_CYLINDER) {
    V3<S> radial{-n.x, -n.y, S(0.0)};
    S rl = norm(radial);
    V3<S> rim;
    if (rl > S(1e-6)) rim = radial * (S(g.p[0]) / rl);
    s = rim + V3<S>{S(0.0), S(0.0), S(-g.p[1] * 0.5) * ssign(n.z)};
  } else if (g.type == G_MESH) {
    V3<S> mc{S(0.5 * (g.p[0] + g.p[3])), S(0.5 * (g.p[1] + g.p[4])), S(0.5 * (g.p[2] + g.p[5]))};
    V3<S> mh{S(0.5 * (g.p[3] - g.p[0])), S(0.5 * (g.p[4] - g.p[1])), S(0.5 * (g.p[5] - g.p[2]))};
    s = mc - V3<S>{mh.x * ssign(n.x), mh.y * ssign(n.y), mh.z * ssign(n.z)};
  }
  return o_p + tmul(o_r, s);
}
template <class S> V3<S> box_corner(const Geom& g, int c) {
  V3<S> corner{S(g.p[0] * ((c & 1) ? 1.0 : -1.0)), S(g.p[1] * ((c & 2) ? 1.0 : -1.0)), S(g.p[2] * ((c & 4) ? 1.0 : -1.0))};
  return cv3<S>(g.o_pos) + tmul(cm3<S>(g.o_rot), corner);
}

template <class S> inline S s_pow(const S& x, double p) {
  if constexpr (std::is_same<S, OpScalar>::value) {
    if (x.k) return OpScalar(std::pow(x.v, p));
    count_trans();
    return OpScalar::state(std::pow(x.v, p));
  } else return S(std::pow(x, S(p)));
}
template <class S> V3<S> normalize3(const V3<S>& a) {
  S l = norm(a);
  return l > S(0.0) ? a * (S(1.0) / l) : a;
}

// Terrain height and unit normal at world (x, y): the flat plane at ground_h,
// or the bilinear heightfield with its cell-wise gradient (phyz_kernels.cu:641-664;
// crates/phyz-model/src/heightfield.rs).
template <class S> S terrain(const Model& m, const S& px, const S& py, V3<S>& n_out) {
  const ContactCfg& c = m.cc;
  if (c.hf_nx == 0) { n_out = V3<S>{S(0.0), S(0.0), S(1.0)}; return S(m.ground_h); }
  auto locate = [&](const S& w, double o, int n, int& i, S& t) {
    if (n < 2) { i = 0; t = S(0.0); return; }
    S u = s_clamp((w - S(o)) / S(c.hf_cell), S(0.0), S(double(n - 1)));
    const double uv = s_val(u);
    int ii = std::isfinite(uv) ? (int)uv : 0;  // a diverged world reads cell 0
    ii = std::max(0, std::min(ii, n - 2));
    i = ii;
    t = u - S(double(ii));
  };
  int ix, iy;
  S tx, ty;
  locate(px, c.hf_ox, c.hf_nx, ix, tx);
  locate(py, c.hf_oy, c.hf_ny, iy, ty);
  const int ix1 = std::min(ix + 1, c.hf_nx - 1), iy1 = std::min(iy + 1, c.hf_ny - 1);
  auto node = [&](int x, int y) { return S(c.hf_oz + c.hf[(size_t)y * c.hf_nx + x]); };
  const S h00 = node(ix, iy), h10 = node(ix1, iy), h01 = node(ix, iy1), h11 = node(ix1, iy1);
  const S one(1.0);
  S h = (h00 * (one - tx) + h10 * tx) * (one - ty) + (h01 * (one - tx) + h11 * tx) * ty;
  S dhdx(0.0), dhdy(0.0);
  const double span_x = double(c.hf_nx - 1) * c.hf_cell, span_y = double(c.hf_ny - 1) * c.hf_cell;
  if (c.hf_nx >= 2 && s_val(px) >= c.hf_ox && s_val(px) <= c.hf_ox + span_x)
    dhdx = ((h10 - h00) * (one - ty) + (h11 - h01) * ty) / S(c.hf_cell);
  if (c.hf_ny >= 2 && s_val(py) >= c.hf_oy && s_val(py) <= c.hf_oy + span_y)
    dhdy = ((h01 - h00) * (one - tx) + (h11 - h10) * tx) / S(c.hf_cell);
  n_out = normalize3(V3<S>{-dhdx, -dhdy, one});
  return h;
}

// SolImp impedance and its margin taper, smoothstep restitution, contact
// tangents (phyz_kernels.cu:581-633; phyz_contact's material and cone frame).
template <class S> S solimp_impedance(const ContactCfg& c, const S& r) {
  const double dmin = std::clamp(c.solimp_dmin, 1e-4, 1.0 - 1e-9), dmax = std::clamp(c.solimp_dmax, 1e-4, 1.0 - 1e-9);
  if (c.solimp_width <= 0.0) return S(dmax);
  S x = s_clamp(s_abs(r) / S(c.solimp_width), S(0.0), S(1.0));
  const double mid = std::clamp(c.solimp_mid, 1e-6, 1.0 - 1e-6), pw = std::max(c.solimp_power, 1.0);
  S y = x <= S(mid) ? s_pow(x, pw) / S(std::pow(mid, pw - 1.0))
                    : S(1.0) - s_pow(S(1.0) - x, pw) / S(std::pow(1.0 - mid, pw - 1.0));
  return S(dmin) + y * S(dmax - dmin);
}
template <class S> S impedance_at(const ContactCfg& c, const S& depth) {
  if (depth >= S(0.0)) return solimp_impedance(c, depth);
  S gap = -depth;
  if (c.margin <= 0.0 || gap >= S(c.margin)) return S(0.0);
  S sc = S(1.0) - gap / S(c.margin);
  return sc * sc * (S(3.0) - S(2.0) * sc) * solimp_impedance(c, S(0.0));
}
template <class S> S effective_restitution(const ContactCfg& c, double e, const S& approach) {
  const double vr = c.restitution_threshold;
  if (vr <= 0.0) return S(e);
  S sp = s_abs(approach);
  if (sp <= S(vr)) return S(0.0);
  if (sp >= S(2.0 * vr)) return S(e);
  S t = (sp - S(vr)) / S(vr);
  return S(e) * t * t * (S(3.0) - S(2.0) * t);
}
template <class S> void contact_tangents(const V3<S>& n, V3<S>& u, V3<S>& w) {
  V3<S> a{S(1.0), S(0.0), S(0.0)};
  if (s_abs(n.x) > S(0.9)) a = V3<S>{S(0.0), S(1.0), S(0.0)};
  u = normalize3(cross(n, a));
  w = cross(n, u);
}

template <class S> void plane_pass(const Model& m, const FK<S>* fk, SV<S>* ext, S* cs);

// One contact pass over a world (phyz_kernels.cu:804-1132): ground or terrain
// contacts per body, then the body-attached plane. Penalty mode applies the
// bounded Kelvin-Voigt law; impulse mode makes one warm-started Coulomb update
// per contact slot, from the velocities in `fk` (the free velocity v + dt qdd).
// ext is overwritten (body-frame spatial forces). cs (nb x 56: readback row,
// ground impulses, plane impulses) is read and written in impulse mode and may
// be null in penalty mode; rows (nb x 8) receives the readback rows.
template <class S> void contact_pass(const Model& m, const FK<S>* fk, SV<S>* ext, S* cs, S* rows) {
  const ContactCfg& c = m.cc;
  const bool imp = c.solve_mode == 1;
  const double dt = m.dt, dtc = std::max(dt, 1e-9);
  for (int i = 0; i < m.nb; i++) ext[i] = SV<S>();
  auto zero_body = [&](int i) {
    if (cs) for (int k = 0; k < CS_STRIDE; k++) cs[i * CS_STRIDE + k] = S(0.0);
    if (rows) for (int k = 0; k < CONTACT_ROW; k++) rows[i * CONTACT_ROW + k] = S(0.0);
  };
  for (int i = 0; i < m.nb; i++) {
    const Geom& g = m.geoms[i];
    if (g.type == G_NONE) { zero_body(i); continue; }
    const Body& b = m.bodies[i];
    const M3<S>& R = fk[i].w_rot;
    V3<S> z_body{R.m[2][0], R.m[2][1], R.m[2][2]};  // R^T z
    const int npts = g.type == G_BOX ? 8 : 1;
    const double pt_scale = g.type == G_BOX ? 0.25 : 1.0;
    auto point = [&](int cp) { return g.type == G_BOX ? box_corner<S>(g, cp) : support_point<S>(g, z_body); };
    int n_active = 0;
    if (imp) {
      for (int cq = 0; cq < npts; cq++) {
        V3<S> sq_w = fk[i].w_pos + R * point(cq);
        V3<S> tn;
        S th = terrain(m, sq_w.x, sq_w.y, tn);
        if (tn.z * (th - sq_w.z) > S(-c.margin)) n_active++;
      }
      if (n_active < 1) n_active = 1;
    }
    V3<S> f_total, deepest_w;
    S deepest(0.0);
    bool any = false;
    for (int cp = 0; cp < npts; cp++) {
      V3<S> sup = point(cp);
      V3<S> sup_w = fk[i].w_pos + R * sup;
      V3<S> n_w;
      S terr_h = terrain(m, sup_w.x, sup_w.y, n_w);
      S pen = n_w.z * (terr_h - sup_w.z);
      const bool in = imp ? pen > S(-c.margin) : pen > S(0.0);
      if (!in) {
        if (imp && cs) for (int k = 0; k < 3; k++) cs[i * CS_STRIDE + CS_IMPULSE_OFF + cp * 3 + k] = S(0.0);
        continue;
      }
      V3<S> n_body = tmul(R, n_w);
      V3<S> v_pt = fk[i].vel.lin + cross(fk[i].vel.ang, sup);
      S v_n = dot(v_pt, n_body);
      if (imp) {
        S* slot = cs + i * CS_STRIDE + CS_IMPULSE_OFF + cp * 3;
        V3<S> tu, tw;
        contact_tangents(n_body, tu, tw);
        S b_u = dot(v_pt, tu), b_w = dot(v_pt, tw);
        S m_n = contact_eff_mass<S>(b, sup, n_body) / S(double(n_active));
        S a_nn = S(1.0) / s_max(m_n, S(1e-9));
        S bias = impedance_at(c, pen) * S(c.erp) * s_max(pen, S(0.0)) / S(dtc);
        S e = effective_restitution(c, c.restitution, s_min(v_n, S(0.0)));
        S r_n = v_n * (S(1.0) + e) - a_nn * slot[0];
        S fn = s_max((bias - r_n) / a_nn, S(0.0));
        S a_uu = S(double(n_active)) / s_max(contact_eff_mass<S>(b, sup, tu), S(1e-9));
        S a_ww = S(double(n_active)) / s_max(contact_eff_mass<S>(b, sup, tw), S(1e-9));
        S ftu = -(b_u - a_uu * slot[1]) / a_uu;
        S ftw = -(b_w - a_ww * slot[2]) / a_ww;
        S limit = S(m.mu) * fn;
        S tn = s_sqrt(ftu * ftu + ftw * ftw);
        if (tn > limit) {
          S scl = tn > S(0.0) ? limit / tn : S(0.0);
          ftu = ftu * scl;
          ftw = ftw * scl;
        }
        slot[0] = fn; slot[1] = ftu; slot[2] = ftw;
        V3<S> fb = (n_body * fn + tu * ftu + tw * ftw) * (S(1.0) / S(dtc));
        ext[i].ang = ext[i].ang + cross(sup, fb);
        ext[i].lin = ext[i].lin + fb;
        f_total = f_total + R * fb;
        any = true;
        if (pen > deepest) { deepest = pen; deepest_w = sup_w; }
        continue;
      }
      S m_n = contact_eff_mass<S>(b, sup, n_body);
      S k_b = s_min(S(pt_scale * g.k), max_stiffness(m_n, dt));
      S d_b = s_min(S(pt_scale * g.d), max_damping(m_n, dt));
      S f_n = s_max(k_b * pen - d_b * v_n, S(0.0));
      V3<S> v_tan = v_pt - n_body * v_n;
      S vt = norm(v_tan);
      V3<S> fb = n_body * f_n;
      if (vt > S(1e-6)) {
        V3<S> t_dir = v_tan * (S(1.0) / vt);
        S coul = S(m.mu) * f_n * s_min(S(1.0), vt / S(1e-3));
        S f_t = s_min(coul, max_damping(contact_eff_mass<S>(b, sup, t_dir), dt) * vt);
        fb = fb - t_dir * f_t;
      }
      ext[i].ang = ext[i].ang + cross(sup, fb);
      ext[i].lin = ext[i].lin + fb;
      f_total = f_total + R * fb;
      any = true;
      if (pen > deepest) { deepest = pen; deepest_w = V3<S>{sup_w.x, sup_w.y, terr_h}; }
    }
    if (!any) { zero_body(i); continue; }
    S row[CONTACT_ROW] = {S(1.0), deepest, deepest_w.x, deepest_w.y, deepest_w.z, f_total.x, f_total.y, f_total.z};
    for (int k = 0; k < CONTACT_ROW; k++) {
      if (cs) cs[i * CS_STRIDE + k] = row[k];
      if (rows) rows[i * CONTACT_ROW + k] = row[k];
    }
  }

  plane_pass(m, fk, ext, cs);
}

// Body-attached plane: the plane body's local +Z face at plane_offset,
// acting on every other collidable body not excluded, forces on both
// (phyz_kernels.cu:982-1132). Adds to ext; cs as in contact_pass.
template <class S> void plane_pass(const Model& m, const FK<S>* fk, SV<S>* ext, S* cs) {
  const ContactCfg& c = m.cc;
  const bool imp = c.solve_mode == 1;
  const double dt = m.dt, dtc = std::max(dt, 1e-9);
  if (c.plane_body < 0) return;
  const int pb = c.plane_body;
  const M3<S>& Rp = fk[pb].w_rot;
  const V3<S> Pp = fk[pb].w_pos;
  const V3<S> n_w = Rp * V3<S>{S(0.0), S(0.0), S(1.0)};
  const V3<S> p0_w = Pp + Rp * V3<S>{S(0.0), S(0.0), S(c.plane_offset)};
  const Body& bp = m.bodies[pb];
  for (int i = 0; i < m.nb; i++) {
    if (i == pb) continue;
    const Geom& g = m.geoms[i];
    if (g.type == G_NONE || g.skip_plane) continue;
    const Body& b = m.bodies[i];
    const M3<S>& R = fk[i].w_rot;
    const V3<S> n_body = tmul(R, n_w);
    const int npts = g.type == G_BOX ? 8 : 1;
    const double pt_scale = g.type == G_BOX ? 0.25 : 1.0;
    auto point = [&](int cp) { return g.type == G_BOX ? box_corner<S>(g, cp) : support_point<S>(g, n_body); };
    S lo_x(1e30), lo_y(1e30), hi_x(-1e30), hi_y(-1e30);
    for (int cp = 0; cp < npts; cp++) {
      V3<S> rp = tmul(Rp, fk[i].w_pos + R * point(cp) - Pp);
      lo_x = s_min(lo_x, rp.x); lo_y = s_min(lo_y, rp.y);
      hi_x = s_max(hi_x, rp.x); hi_y = s_max(hi_y, rp.y);
    }
    const S ov_lo_x = s_max(lo_x, S(-c.plane_half_x)), ov_lo_y = s_max(lo_y, S(-c.plane_half_y));
    const S ov_hi_x = s_min(hi_x, S(c.plane_half_x)), ov_hi_y = s_min(hi_y, S(c.plane_half_y));
    if (ov_lo_x > ov_hi_x || ov_lo_y > ov_hi_y) continue;
    int n_act = 1;
    if (imp) {
      int cnt = 0;
      for (int cq = 0; cq < npts; cq++) {
        S d = -dot(fk[i].w_pos + R * point(cq) - p0_w, n_w);
        if (d > S(0.0) && d <= S(c.plane_max_depth)) cnt++;
      }
      n_act = cnt > 1 ? cnt : 1;
    }
    for (int cp = 0; cp < npts; cp++) {
      V3<S> sup_w0 = fk[i].w_pos + R * point(cp);
      S pen = -dot(sup_w0 - p0_w, n_w);
      if (pen <= S(0.0) || pen > S(c.plane_max_depth)) {
        if (imp && cs) for (int k = 0; k < 3; k++) cs[i * CS_STRIDE + CS_PLANE_OFF + cp * 3 + k] = S(0.0);
        continue;
      }
      V3<S> r_p = tmul(Rp, sup_w0 - Pp);
      r_p.x = s_clamp(r_p.x, ov_lo_x, ov_hi_x);
      r_p.y = s_clamp(r_p.y, ov_lo_y, ov_hi_y);
      V3<S> sup_w = Pp + Rp * r_p;
      V3<S> sup_c = tmul(R, sup_w - fk[i].w_pos);
      V3<S> v_i_w = R * (fk[i].vel.lin + cross(fk[i].vel.ang, sup_c));
      V3<S> v_p_w = Rp * (fk[pb].vel.lin + cross(fk[pb].vel.ang, r_p));
      V3<S> v_rel = v_i_w - v_p_w;
      S v_n = dot(v_rel, n_w);
      auto series = [&](const V3<S>& d_w) {
        return S(1.0) / (S(1.0) / contact_eff_mass<S>(b, sup_c, tmul(R, d_w)) +
                         S(1.0) / contact_eff_mass<S>(bp, r_p, tmul(Rp, d_w)));
      };
      S m_n = series(n_w);
      V3<S> f_w;
      if (imp) {
        S* slot = cs + i * CS_STRIDE + CS_PLANE_OFF + cp * 3;
        V3<S> pu, pw;
        contact_tangents(n_w, pu, pw);
        S bu = dot(v_rel, pu), bw = dot(v_rel, pw);
        S ann = S(double(n_act)) / s_max(m_n, S(1e-9));
        S bias = impedance_at(c, pen) * S(c.erp) * s_max(pen, S(0.0)) / S(dtc);
        S ee = effective_restitution(c, c.restitution, s_min(v_n, S(0.0)));
        S nf = s_max((bias - (v_n * (S(1.0) + ee) - ann * slot[0])) / ann, S(0.0));
        S auu = S(double(n_act)) / s_max(series(pu), S(1e-9));
        S aww = S(double(n_act)) / s_max(series(pw), S(1e-9));
        S ptu = -(bu - auu * slot[1]) / auu;
        S ptw = -(bw - aww * slot[2]) / aww;
        S plim = S(m.mu) * nf;
        S ptn = s_sqrt(ptu * ptu + ptw * ptw);
        if (ptn > plim) {
          S psc = ptn > S(0.0) ? plim / ptn : S(0.0);
          ptu = ptu * psc;
          ptw = ptw * psc;
        }
        slot[0] = nf; slot[1] = ptu; slot[2] = ptw;
        f_w = (n_w * nf + pu * ptu + pw * ptw) * (S(1.0) / S(dtc));
      } else {
        S k_b = s_min(S(pt_scale * g.k), max_stiffness(m_n, dt));
        S d_b = s_min(S(pt_scale * g.d), max_damping(m_n, dt));
        S f_n = s_max(k_b * pen - d_b * v_n, S(0.0));
        V3<S> v_tan = v_rel - n_w * v_n;
        S vt = norm(v_tan);
        f_w = n_w * f_n;
        if (vt > S(1e-6)) {
          V3<S> t_dir = v_tan * (S(1.0) / vt);
          S f_t = s_min(S(m.mu) * f_n * s_min(S(1.0), vt / S(1e-3)), max_damping(series(t_dir), dt) * vt);
          f_w = f_w - t_dir * f_t;
        }
      }
      V3<S> f_i = tmul(R, f_w);
      ext[i].ang = ext[i].ang + cross(sup_c, f_i);
      ext[i].lin = ext[i].lin + f_i;
      V3<S> f_p = tmul(Rp, -f_w);
      ext[pb].ang = ext[pb].ang + cross(r_p, f_p);
      ext[pb].lin = ext[pb].lin + f_p;
    }
  }
}

// Penalty-mode contact of one world (no persistent solver state).
template <class S> void ground_contact(const Model& m, const FK<S>* fk, SV<S>* ext, S* rows /* nb x 8, nullable */) {
  contact_pass<S>(m, fk, ext, nullptr, rows);
}

// Impulse-mode ground/terrain contact split the way the kernels run it. Within
// one step q is fixed, so everything about a contact point except its velocity
// is the same in every sweep: support point, terrain height and normal,
// penetration, tangent frame, the three effective masses and the SolImp bias.
// ground_prepare computes those once per step; ground_sweep makes the
// velocity-dependent update per sweep. With m' = max(m_n / n_active, 1e-9),
// c_t = max(m_t, 1e-9) / n_active, the update of contact_pass reads
//   f_n = max((bias - v_n (1 + e)) m' + s_n, 0),  f_t = s_t - b_t c_t,
// the same quantity as (bias - r_n) / a_nn and -(b_t - a_tt s_t) / a_tt.
template <class S> struct GroundPoint {
  V3<S> sup, nb, tu, tw;  // body-frame point, normal, tangents
  S mn, cu, cw, bias;
  bool in;
};
template <class S> struct GroundPrep {
  std::vector<GroundPoint<S>> pts;
  std::vector<int> off, np;
  std::vector<char> any;
  std::vector<S> row5;  // nb x 5: touching, deepest, deepest point (x, y, z)
};
template <class S> void ground_prepare(const Model& m, const FK<S>* fk, GroundPrep<S>& gp) {
  const ContactCfg& c = m.cc;
  const double dtc = std::max(m.dt, 1e-9);
  gp.pts.clear();
  gp.off.assign(m.nb, 0);
  gp.np.assign(m.nb, 0);
  gp.any.assign(m.nb, 0);
  gp.row5.assign((size_t)m.nb * 5, S(0.0));
  for (int i = 0; i < m.nb; i++) {
    const Geom& g = m.geoms[i];
    gp.off[i] = (int)gp.pts.size();
    if (g.type == G_NONE) continue;
    const Body& b = m.bodies[i];
    const M3<S>& R = fk[i].w_rot;
    V3<S> z_body{R.m[2][0], R.m[2][1], R.m[2][2]};
    const int npts = g.type == G_BOX ? 8 : 1;
    gp.np[i] = npts;
    GroundPoint<S> pt[8];
    S pen[8];
    V3<S> supw[8];
    int n_active = 0;
    for (int cp = 0; cp < npts; cp++) {
      pt[cp].sup = g.type == G_BOX ? box_corner<S>(g, cp) : support_point<S>(g, z_body);
      supw[cp] = fk[i].w_pos + R * pt[cp].sup;
      V3<S> n_w;
      S th = terrain(m, supw[cp].x, supw[cp].y, n_w);
      pen[cp] = n_w.z * (th - supw[cp].z);
      pt[cp].in = pen[cp] > S(-c.margin);
      pt[cp].nb = tmul(R, n_w);
      if (pt[cp].in) n_active++;
    }
    const S na(double(n_active < 1 ? 1 : n_active));
    S deepest(0.0);
    V3<S> dw;
    for (int cp = 0; cp < npts; cp++) {
      GroundPoint<S>& p = pt[cp];
      if (p.in) {
        contact_tangents(p.nb, p.tu, p.tw);
        p.mn = s_max(contact_eff_mass<S>(b, p.sup, p.nb) / na, S(1e-9));
        p.cu = s_max(contact_eff_mass<S>(b, p.sup, p.tu), S(1e-9)) / na;
        p.cw = s_max(contact_eff_mass<S>(b, p.sup, p.tw), S(1e-9)) / na;
        p.bias = impedance_at(c, pen[cp]) * S(c.erp) * s_max(pen[cp], S(0.0)) / S(dtc);
        gp.any[i] = 1;
        if (pen[cp] > deepest) { deepest = pen[cp]; dw = supw[cp]; }
      }
      gp.pts.push_back(p);
    }
    if (gp.any[i]) {
      S* r = &gp.row5[(size_t)i * 5];
      r[0] = S(1.0); r[1] = deepest; r[2] = dw.x; r[3] = dw.y; r[4] = dw.z;
    }
  }
}
// One sweep of the prepared ground contacts at the body velocities in fk,
// then the plane (contact_pass's order). ext is overwritten; cs and rows as in
// contact_pass; the row's force is R times the body's summed ground force.
template <class S> void ground_sweep(const Model& m, const GroundPrep<S>& gp, const FK<S>* fk, SV<S>* ext, S* cs,
                                     S* rows) {
  const ContactCfg& c = m.cc;
  const double dtc = std::max(m.dt, 1e-9);
  for (int i = 0; i < m.nb; i++) {
    ext[i] = SV<S>();
    if (!gp.any[i]) {
      if (cs) for (int k = 0; k < CS_STRIDE; k++) cs[i * CS_STRIDE + k] = S(0.0);
      if (rows) for (int k = 0; k < CONTACT_ROW; k++) rows[i * CONTACT_ROW + k] = S(0.0);
      continue;
    }
    for (int cp = 0; cp < gp.np[i]; cp++) {
      const GroundPoint<S>& p = gp.pts[gp.off[i] + cp];
      S* slot = cs + i * CS_STRIDE + CS_IMPULSE_OFF + cp * 3;
      if (!p.in) { for (int k = 0; k < 3; k++) slot[k] = S(0.0); continue; }
      V3<S> v_pt = fk[i].vel.lin + cross(fk[i].vel.ang, p.sup);
      S v_n = dot(v_pt, p.nb);
      S e = effective_restitution(c, c.restitution, s_min(v_n, S(0.0)));
      S fn = s_max((p.bias - v_n * (S(1.0) + e)) * p.mn + slot[0], S(0.0));
      S ftu = slot[1] - dot(v_pt, p.tu) * p.cu;
      S ftw = slot[2] - dot(v_pt, p.tw) * p.cw;
      S limit = S(m.mu) * fn;
      S tn = s_sqrt(ftu * ftu + ftw * ftw);
      if (tn > limit) {
        S scl = tn > S(0.0) ? limit / tn : S(0.0);
        ftu = ftu * scl;
        ftw = ftw * scl;
      }
      slot[0] = fn; slot[1] = ftu; slot[2] = ftw;
      V3<S> fb = (p.nb * fn + p.tu * ftu + p.tw * ftw) * (S(1.0) / S(dtc));
      ext[i].ang = ext[i].ang + cross(p.sup, fb);
      ext[i].lin = ext[i].lin + fb;
    }
    V3<S> f_total = fk[i].w_rot * ext[i].lin;
    const S* r5 = &gp.row5[(size_t)i * 5];
    S row[CONTACT_ROW] = {r5[0], r5[1], r5[2], r5[3], r5[4], f_total.x, f_total.y, f_total.z};
    for (int k = 0; k < CONTACT_ROW; k++) {
      if (cs) cs[i * CS_STRIDE + k] = row[k];
      if (rows) rows[i * CONTACT_ROW + k] = row[k];
    }
  }
  plane_pass(m, fk, ext, cs);
}

// ─────────────────────────────────────────────────────────────────────────────
// Semi-implicit Euler (integrate.rs:41-92): v += dt qdd, then q from the new v.
// ─────────────────────────────────────────────────────────────────────────────
template <class S> void integrate(const Model& m, S* q, S* v, const S* qdd) {
  S dt = S(m.dt);
  for (int j = 0; j < m.nv; j++) v[j] = v[j] + dt * qdd[j];
  for (const Body& b : m.bodies) {
    int qo = b.qoff, vo = b.voff;
    if (b.jtype == J_REVOLUTE || b.jtype == J_PRISMATIC) q[qo] = q[qo] + dt * v[vo];
    else if (b.jtype == J_BALL || b.jtype == J_FREE) {
      V3<S> w{v[vo], v[vo + 1], v[vo + 2]};
      Q<S> cur = quat_exp(V3<S>{q[qo], q[qo + 1], q[qo + 2]});
      if (b.jtype == J_FREE) {
        V3<S> wl = qrotate(cur, V3<S>{v[vo + 3], v[vo + 4], v[vo + 5]});
        q[qo + 3] = q[qo + 3] + dt * wl.x;
        q[qo + 4] = q[qo + 4] + dt * wl.y;
        q[qo + 5] = q[qo + 5] + dt * wl.z;
      }
      V3<S> lg = quat_log(qnormalize(qmul(cur, quat_exp(w * dt))));
      q[qo] = lg.x; q[qo + 1] = lg.y; q[qo + 2] = lg.z;
    }
  }
}

// ─────────────────────────────────────────────────────────────────────────────
// Per-world RNG: SplitMix64 seed mix then xorshift64 (policy_pipeline.rs:417-456).
// Uniform u = (x >> 11) 2^-53 in [0, 1). Normals by Box-Muller, both outputs
// used: r = sqrt(-2 ln(1 - u1)), (r cos 2 pi u2, r sin 2 pi u2).
// ─────────────────────────────────────────────────────────────────────────────
inline uint64_t world_seed(uint64_t seed, uint64_t world) {
  uint64_t z = seed + 0x9E3779B97F4A7C15ull * (world + 1);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z = z ^ (z >> 31);
  return z ? z : 1;
}
inline uint64_t xorshift64(uint64_t& s) {
  uint64_t x = s;
  x ^= x << 13; x ^= x >> 7; x ^= x << 17;
  s = x;
  return x;
}
inline double rng_uniform(uint64_t& s) { return (double)(xorshift64(s) >> 11) * (1.0 / 9007199254740992.0); }
template <class S> S as_state(double x) {
  if constexpr (std::is_same<S, OpScalar>::value) return OpScalar::state(x);
  else return S(x);
}
// Write the step's control draws into ctrl, in DOF-list order. Uniform:
// a + (b - a) u. Normal: a + b z.
template <class S> void noise_apply(const Model& m, uint64_t& s, S* ctrl) {
  const int n = (int)m.noise_dofs.size();
  if (m.noise_dist == NOISE_UNIFORM) {
    for (int k = 0; k < n; k++) {
      S u = as_state<S>(rng_uniform(s));
      ctrl[m.noise_dofs[k]] = S(m.noise_a) + S(m.noise_b - m.noise_a) * u;
    }
    return;
  }
  for (int k = 0; k < n; k += 2) {
    S u1 = as_state<S>(rng_uniform(s)), u2 = as_state<S>(rng_uniform(s));
    S r = s_sqrt(S(-2.0) * s_log(S(1.0) - u1));
    S sn, cs;
    s_sincos(S(6.283185307179586) * u2, &sn, &cs);
    ctrl[m.noise_dofs[k]] = S(m.noise_a) + S(m.noise_b) * (r * cs);
    if (k + 1 < n) ctrl[m.noise_dofs[k + 1]] = S(m.noise_a) + S(m.noise_b) * (r * sn);
  }
}

// ─────────────────────────────────────────────────────────────────────────────
// One full step of one world, in the reference order
// (crates/phyz-gpu/src/cuda/mod.rs:879-945): control noise, PD, contact, ABA,
// integrate. ctrl persists between steps exactly as the device ctrl buffer.
// ─────────────────────────────────────────────────────────────────────────────
template <class S> struct WorldScratch {
  std::vector<FK<S>> fk;
  std::vector<SV<S>> ext;  // impulse mode: persists from step to step (the leading ABA reads it)
  std::vector<S> qdd;
  std::vector<S> cs;       // impulse mode: nb x 56 contact state with warm-start impulses, persistent
  std::vector<S> vfree;
  AbaCache<S> cache;       // impulse mode: the step's ABA factorization, reused by the sweeps
  GroundPrep<S> gprep;     // impulse mode: the step's contact geometry, reused by the sweeps
  void reset(const Model& m) {
    fk.assign(m.nb, FK<S>());
    ext.assign(m.nb, SV<S>());
    qdd.assign(m.nv, S(0.0));
    cs.assign((size_t)m.nb * CS_STRIDE, S(0.0));
    vfree.assign(m.nv, S(0.0));
  }
};
// Phase hooks let the op counter attribute work to each phase; a phase may
// report more than once per step (impulse sweeps), so counts accumulate.
struct NoHooks { void operator()(int) const {} };
enum Phase { PH_NOISE = 0, PH_PD = 1, PH_CONTACT = 2, PH_ABA = 3, PH_INTEGRATE = 4 };
template <class S, class Hooks = NoHooks>
void step_world(const Model& m, S* q, S* v, S* ctrl, const S* targets, uint64_t* rng, WorldScratch<S>& ws,
                S* contact_rows, bool dense, const Hooks& hook = Hooks()) {
  if (m.noise && rng) noise_apply(m, *rng, ctrl);
  hook(PH_NOISE);
  for (size_t d = 0; d < m.pd.size(); d++) {
    const PdDof& p = m.pd[d];
    S tau = S(p.kp) * (targets[d] - q[p.q_index]) - S(p.kd) * v[p.v_index];
    ctrl[p.v_index] = s_clamp(tau, S(-p.max_force), S(p.max_force));
  }
  hook(PH_PD);
  if (ws.qdd.size() != (size_t)m.nv) ws.reset(m);
  auto aba = [&](const SV<S>* ext) {
    if (dense) aba_dense(m, q, v, ctrl, ext, ws.qdd.data());
    else aba_struct(m, q, v, ctrl, ext, ws.qdd.data());
  };
  if (m.contact && m.cc.solve_mode == 1) {
    // Impulse mode (mod.rs:899-928): a leading ABA with the previous step's
    // contact forces, then `sweeps` x [contact at the free velocity
    // v + dt qdd, ABA]; each contact pass warm-starts from the last.
    // dense: every sweep is a full contact pass and a full solve (the
    // reference's sequencing); otherwise the kernels' split form: transforms,
    // bias forces, joint factorizations and contact geometry once, then per
    // sweep only the velocities at v + dt qdd, the velocity-dependent contact
    // update (ground_sweep) and the ABA's response to the force change (aba_delta).
    if (dense) {
      aba(ws.ext.data());
      hook(PH_ABA);
      for (int sw = 0; sw < m.cc.sweeps; sw++) {
        for (int k = 0; k < m.nv; k++) ws.vfree[k] = v[k] + S(m.dt) * ws.qdd[k];
        forward_kinematics(m, q, ws.vfree.data(), ws.fk.data());
        contact_pass(m, ws.fk.data(), ws.ext.data(), ws.cs.data(), contact_rows);
        hook(PH_CONTACT);
        aba(ws.ext.data());
        hook(PH_ABA);
      }
    } else {
      aba_factor(m, q, v, ctrl, ws.ext.data(), ws.qdd.data(), ws.cache);
      forward_kinematics(m, q, v, ws.fk.data());
      std::vector<S> qdd0(ws.qdd), dqdd(m.nv);
      std::vector<SV<S>> ext0(ws.ext), dext(m.nb);
      hook(PH_ABA);
      ground_prepare(m, ws.fk.data(), ws.gprep);
      hook(PH_CONTACT);
      for (int sw = 0; sw < m.cc.sweeps; sw++) {
        for (int k = 0; k < m.nv; k++) ws.vfree[k] = v[k] + S(m.dt) * ws.qdd[k];
        fk_velocity(m, ws.cache.xt, ws.vfree.data(), ws.fk.data());
        ground_sweep(m, ws.gprep, ws.fk.data(), ws.ext.data(), ws.cs.data(), contact_rows);
        hook(PH_CONTACT);
        for (int i = 0; i < m.nb; i++) dext[i] = ws.ext[i] - ext0[i];
        aba_delta(m, ws.cache, dext.data(), dqdd.data());
        for (int k = 0; k < m.nv; k++) ws.qdd[k] = qdd0[k] + dqdd[k];
        hook(PH_ABA);
      }
    }
  } else {
    const SV<S>* ext = nullptr;
    if (m.contact) {
      forward_kinematics(m, q, v, ws.fk.data());
      contact_pass(m, ws.fk.data(), ws.ext.data(), (S*)nullptr, contact_rows);
      ext = ws.ext.data();
    }
    hook(PH_CONTACT);
    aba(ext);
    hook(PH_ABA);
  }
  integrate(m, q, v, ws.qdd.data());
  hook(PH_INTEGRATE);
}

}  // namespace phzo
