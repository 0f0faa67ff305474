// phz_device.h — fused per-step device code for gfx950 (CDNA4).
//
// One lane advances one world. A launch runs `nsteps` steps with the world's
// q, v and ctrl held in registers and touches HBM only to load the state at
// the start and store it at the end. Each step is, in the reference's order
// (crates/phyz-gpu/src/cuda/mod.rs:879-945):
//   control noise -> PD servo -> FK + ground penalty contact -> ABA -> integrate
//
// The model is not read from memory: the host emits a `struct Model` of
// constexpr tables (body tree, joint types, inertias, transforms, geometry,
// gains) and compiles this header against it with hiprtc. Every loop over
// bodies is unrolled at compile time (sfor/rfor below), so per-body state lives
// in registers and zero / unit entries of axes, transforms and inertias fold
// away (the kernel is built with -ffinite-math-only -fno-signed-zeros so that
// x*0 and x+0 fold).
//
// Formulation (same equations as crates/phyz-rigid/src/aba.rs:117-368 and the
// reference kernels crates/phyz-gpu/cuda/phyz_kernels.cu:1175-1421, structure
// exploited):
//   pass 1  X_i = X_J(q) X_ptj, v_i = X_i v_p + S qd, c_i = v_i x S qd,
//           p_i = v_i x* (I_i v_i) - f_ext_i   (contact computed here, FK shared)
//   pass 2  U = I_A S, D = S^T U + armature + dt damping, u = tau - S^T p_A;
//           I_a = I_A - U D^-1 U^T, p_a = p_A + I_a c + U D^-1 u;
//           I_A[p] += X^T I_a X (rotation then translation, symmetric blocks),
//           p_A[p] += X^T p_a
//   pass 3  a' = X a_p + c, qdd = D^-1 (u - U^T a'), a = a' + S qdd
//   integrate  v += dt qdd; hinge/slide q += dt v; ball/free quaternion
//              compose-and-relog (crates/phyz-rigid/src/integrate.rs:41-92)
#pragma once

#if !defined(__HIPCC_RTC__)
#include <hip/hip_runtime.h>
#endif

namespace phz {

typedef unsigned long long u64;

template <int V> struct ic { static constexpr int value = V; };
template <int I, int N, class F> __device__ __forceinline__ void sfor(F&& f) {
  if constexpr (I < N) { f(ic<I>{}); sfor<I + 1, N>(f); }
}
template <int N, class F> __device__ __forceinline__ void rfor(F&& f) {
  if constexpr (N > 0) { f(ic<N - 1>{}); rfor<N - 1>(f); }
}

enum { J_REV = 0, J_PRIS = 1, J_FIXED = 2, J_BALL = 3, J_FREE = 4 };
enum { G_NONE = 0, G_SPHERE = 1, G_BOX = 2, G_CAPSULE = 3, G_CYLINDER = 4, G_MESH = 5 };
constexpr int ndof_of(int jt) { return jt == J_FIXED ? 0 : (jt == J_BALL ? 3 : (jt == J_FREE ? 6 : 1)); }

// ── math ─────────────────────────────────────────────────────────────────────
// Kernels are compiled with -ffinite-math-only (the f64 impulse-mode step
// kernel excepted), which lets 0 * x fold away against the model's constant
// zeros. It also makes a NaN or inf anywhere in a floating-point select
// poison, the arm not taken included, and the compiler evaluates both arms. So
// no expression may produce one even on a discarded path: a division whose
// denominator can vanish divides by dmax(d, floor), with the floor below the
// select's own threshold so that the bound cannot be folded back into d.
// Truncation to int by the hardware conversion, which saturates and maps NaN
// to 0. A C cast of a NaN or out-of-range value is undefined, and under
// -ffinite-math-only the float clamps before it may be dropped, so an index
// that addresses memory or selects a quadrant is converted here and clamped as an integer.
__device__ __forceinline__ int cvt_sat_i32(float x) {
  int r;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(x));
  return r;
}
__device__ __forceinline__ int cvt_sat_i32(double x) {
  int r;
  asm("v_cvt_i32_f64 %0, %1" : "=v"(r) : "v"(x));
  return r;
}

__device__ __forceinline__ void angle_sincos(double x, double* s, double* c);
// f64 joint angles take the closed form below (reduction exact for |x| < 1.6e6)
// rather than the library routine and its large-argument branch.
__device__ __forceinline__ void dsincos(double x, double* s, double* c) { angle_sincos(x, s, c); }
__device__ __forceinline__ void angle_sincos(float x, float* s, float* c);
__device__ __forceinline__ void dsincos(float x, float* s, float* c) { angle_sincos(x, s, c); }
__device__ __forceinline__ double dsqrt(double x) { return sqrt(x); }
// sin and cos of x (f64): x = k*pi/2 + r with k the integer nearest 2x/pi,
// taken as t - M for t = 2x/pi + M, M = 1.5 * 2^52 (the addition rounds to
// an integer; the low word of t then holds k mod 2^32, the quadrant, with no
// conversion). pi/2 is split as hi + lo, hi holding 33 significant bits, so
// that k*hi and x - k*hi are exact for |k| < 2^20 (|x| < 1.6e6); |r| <= pi/4
// and the split's residual is 3.5e-27. With u = -r^2: sin r = r + r u P(u),
// P through u^7 (the Taylor series through r^17), and cos r = 1 + u Q(u), Q
// through u^7 (through r^16); the truncations stay below 1e-19 and 3e-18 of
// the value on |r| <= pi/4. P and Q are evaluated in Estrin's form (pairs,
// then u^2, then u^4), about half the dependent chain of Horner's form.
// Used for the f64 quaternion exponential of a free joint (in an IEEE build
// of the chain kernel the library sincos gave a Box-Muller sine a sign that
// varied from launch to launch, its optimised IR correct; the revolute
// angles and the Box-Muller angle now take tab_sincos below).
__device__ __forceinline__ void angle_sincos(double x, double* s, double* c) {
  constexpr double M = 6755399441055744.0;  // 1.5 * 2^52
  const double t = fma(x, 0x1.45f306dc9c883p-1, M);
  const double k = t - M;
  const double r = fma(-k, 0x1.0b4611a626331p-34, fma(-k, 0x1.921fb54400000p+0, x));
  const double u = -(r * r);
  const double u2 = u * u;
  const double u4 = u2 * u2;
  // P(u) = sum_j u^j / (2j+3)!, Q(u) = sum_j u^j / (2j+2)!  (j = 0..7)
  const double p01 = fma(u, 1.0 / 120.0, 1.0 / 6.0);
  const double p23 = fma(u, 1.0 / 362880.0, 1.0 / 5040.0);
  const double p45 = fma(u, 1.0 / 6227020800.0, 1.0 / 39916800.0);
  const double p67 = fma(u, 1.0 / 355687428096000.0, 1.0 / 1307674368000.0);
  const double q01 = fma(u, 1.0 / 24.0, 0.5);
  const double q23 = fma(u, 1.0 / 40320.0, 1.0 / 720.0);
  const double q45 = fma(u, 1.0 / 479001600.0, 1.0 / 3628800.0);
  const double q67 = fma(u, 1.0 / 20922789888000.0, 1.0 / 87178291200.0);
  const double p = fma(u4, fma(u2, p67, p45), fma(u2, p23, p01));
  const double q = fma(u4, fma(u2, q67, q45), fma(u2, q23, q01));
  const double sr = fma(r * u, p, r);
  const double cr = fma(u, q, 1.0);
  // Quadrant n = k mod 4: sin x = +-(n odd ? cos r : sin r), negative for
  // n = 2, 3; cos x = +-(n odd ? sin r : cos r), negative for n = 1, 2.
  const unsigned n = (unsigned)__builtin_bit_cast(unsigned long long, t);
  const bool odd = n & 1u;
  const unsigned long long ss = (unsigned long long)(n & 2u) << 62;
  const unsigned long long cs = (unsigned long long)((n + 1u) & 2u) << 62;
  *s = __builtin_bit_cast(double, __builtin_bit_cast(unsigned long long, odd ? cr : sr) ^ ss);
  *c = __builtin_bit_cast(double, __builtin_bit_cast(unsigned long long, odd ? sr : cr) ^ cs);
}
// sin and cos of an f64 angle from a table in LDS (the f64 kernels' revolute
// joint angles and Box-Muller angles): x = 2 pi k / 64
// + r with k = rint(64 x / 2 pi) and r reduced by a two-part 2 pi / 64 (the
// high part has 25 significant bits, so k times it is exact for |k| < 2^28);
// sin x = s_k cos r + c_k sin r, cos x = c_k cos r - s_k sin r with (c_k, s_k)
// the table's exactly rounded cosine and sine of 2 pi k / 64, and on
// |r| <= pi/64 the Taylor series of sin r through r^7 and of cos r through
// r^8 (truncation below 4.5e-18 and 2.5e-20). Within about 2 ulp, in about 19
// VALU instructions, one LDS read and ten constants, against about 30
// instructions and twenty constants for angle_sincos. At k = 0 the table
// entry is (1, 0) exactly, so a small angle keeps its relative accuracy.
// The kernel fills the table once per launch (fill_tables) before any use.
__shared__ __attribute__((aligned(16))) double phz_sc_tab[128];
// The table of tab_log below: (invc, logc) for each of its 64 intervals.
__shared__ __attribute__((aligned(16))) double phz_log_tab[128];
// Both tables, entry pair `lane` of each, from the 64 lanes of one wave.
__device__ __forceinline__ void fill_tables(int lane) {
  static constexpr double lg[128] = {
    0x1.702e05c0b8170p+0, -0x1.741d876c67bb1p-2,
    0x1.6c16c16c16c17p+0, -0x1.68ac83e9c6a15p-2,
    0x1.6816816816817p+0, -0x1.5d5bddf595f31p-2,
    0x1.642c8590b2164p+0, -0x1.522ae0738a3d7p-2,
    0x1.6058160581606p+0, -0x1.4718dc271c41cp-2,
    0x1.5c9882b931057p+0, -0x1.3c25277333183p-2,
    0x1.58ed2308158edp+0, -0x1.314f1e1d35ce3p-2,
    0x1.5555555555555p+0, -0x1.269621134db91p-2,
    0x1.51d07eae2f815p+0, -0x1.1bf99635a6b95p-2,
    0x1.4e5e0a72f0539p+0, -0x1.1178e8227e47ap-2,
    0x1.4afd6a052bf5bp+0, -0x1.07138604d5864p-2,
    0x1.47ae147ae147bp+0, -0x1.f991c6cb3b37ap-3,
    0x1.446f86562d9fbp+0, -0x1.e530effe71013p-3,
    0x1.4141414141414p+0, -0x1.d1037f2655e7bp-3,
    0x1.3e22cbce4a902p+0, -0x1.bd087383bd8aap-3,
    0x1.3b13b13b13b14p+0, -0x1.a93ed3c8ad9e5p-3,
    0x1.3813813813814p+0, -0x1.95a5adcf70182p-3,
    0x1.3521cfb2b78c1p+0, -0x1.823c16551a3c0p-3,
    0x1.323e34a2b10bfp+0, -0x1.6f0128b756ab9p-3,
    0x1.2f684bda12f68p+0, -0x1.5bf406b543db0p-3,
    0x1.2c9fb4d812ca0p+0, -0x1.4913d8333b563p-3,
    0x1.29e4129e4129ep+0, -0x1.365fcb0159014p-3,
    0x1.27350b8812735p+0, -0x1.23d712a49c201p-3,
    0x1.2492492492492p+0, -0x1.1178e8227e47ap-3,
    0x1.21fb78121fb78p+0, -0x1.fe89139dbd565p-4,
    0x1.1f7047dc11f70p+0, -0x1.da7276384469ep-4,
    0x1.1cf06ada2811dp+0, -0x1.b6ac88dad5b1dp-4,
    0x1.1a7b9611a7b96p+0, -0x1.9335e5d594988p-4,
    0x1.1811811811812p+0, -0x1.700d30aeac0e8p-4,
    0x1.15b1e5f75270dp+0, -0x1.4d3115d207eacp-4,
    0x1.135c81135c811p+0, -0x1.2aa04a44717a1p-4,
    0x1.1111111111111p+0, -0x1.08598b59e3a06p-4,
    0x1.0ecf56be69c90p+0, -0x1.ccb73cdddb2d0p-5,
    0x1.0c9714fbcda3bp+0, -0x1.894aa149fb34bp-5,
    0x1.0a6810a6810a7p+0, -0x1.466aed42de3f9p-5,
    0x1.0842108421084p+0, -0x1.0415d89e74440p-5,
    0x1.0624dd2f1a9fcp+0, -0x1.8492528c8cac5p-6,
    0x1.0410410410410p+0, -0x1.0205658935837p-6,
    0x1.0204081020408p+0, -0x1.010157588de69p-7,
    0x1.0000000000000p+0, 0x0.0p+0,
    0x1.f81f81f81f820p-1, 0x1.fc0a8b0fc03c4p-7,
    0x1.f07c1f07c1f08p-1, 0x1.f829b0e7832f8p-6,
    0x1.e9131abf0b767p-1, 0x1.77458f632dcffp-5,
    0x1.e1e1e1e1e1e1ep-1, 0x1.f0a30c01162a8p-5,
    0x1.dae6076b981dbp-1, 0x1.341d7961bd1d0p-4,
    0x1.d41d41d41d41dp-1, 0x1.6f0d28ae56b4ep-4,
    0x1.cd85689039b0bp-1, 0x1.a926d3a4ad562p-4,
    0x1.c71c71c71c71cp-1, 0x1.e27076e2af2eap-4,
    0x1.c0e070381c0e0p-1, 0x1.0d77e7cd08e5bp-3,
    0x1.bacf914c1bad0p-1, 0x1.29552f81ff521p-3,
    0x1.b4e81b4e81b4fp-1, 0x1.44d2b6ccb7d1cp-3,
    0x1.af286bca1af28p-1, 0x1.5ff3070a793d6p-3,
    0x1.a98ef606a63bep-1, 0x1.7ab890210d907p-3,
    0x1.a41a41a41a41ap-1, 0x1.9525a9cf456b6p-3,
    0x1.9ec8e951033d9p-1, 0x1.af3c94e80bff3p-3,
    0x1.999999999999ap-1, 0x1.c8ff7c79a9a20p-3,
    0x1.948b0fcd6e9e0p-1, 0x1.e27076e2af2e8p-3,
    0x1.8f9c18f9c18fap-1, 0x1.fb9186d5e3e29p-3,
    0x1.8acb90f6bf3aap-1, 0x1.0a324e27390e2p-2,
    0x1.8618618618618p-1, 0x1.1675cababa60fp-2,
    0x1.8181818181818p-1, 0x1.22941fbcf7966p-2,
    0x1.7d05f417d05f4p-1, 0x1.2e8e2bae11d31p-2,
    0x1.78a4c8178a4c8p-1, 0x1.3a64c556945eap-2,
    0x1.745d1745d1746p-1, 0x1.4618bc21c5ec2p-2};
  static constexpr double k[128] = {
    0x1.0000000000000p+0, 0x0.0p+0,
    0x1.fd88da3d12526p-1, 0x1.917a6bc29b42cp-4,
    0x1.f6297cff75cb0p-1, 0x1.8f8b83c69a60bp-3,
    0x1.e9f4156c62ddap-1, 0x1.294062ed59f06p-2,
    0x1.d906bcf328d46p-1, 0x1.87de2a6aea963p-2,
    0x1.c38b2f180bdb1p-1, 0x1.e2b5d3806f63bp-2,
    0x1.a9b66290ea1a3p-1, 0x1.1c73b39ae68c8p-1,
    0x1.8bc806b151741p-1, 0x1.44cf325091dd6p-1,
    0x1.6a09e667f3bcdp-1, 0x1.6a09e667f3bcdp-1,
    0x1.44cf325091dd6p-1, 0x1.8bc806b151741p-1,
    0x1.1c73b39ae68c8p-1, 0x1.a9b66290ea1a3p-1,
    0x1.e2b5d3806f63bp-2, 0x1.c38b2f180bdb1p-1,
    0x1.87de2a6aea963p-2, 0x1.d906bcf328d46p-1,
    0x1.294062ed59f06p-2, 0x1.e9f4156c62ddap-1,
    0x1.8f8b83c69a60bp-3, 0x1.f6297cff75cb0p-1,
    0x1.917a6bc29b42cp-4, 0x1.fd88da3d12526p-1,
    0.0, 0x1.0000000000000p+0,
    -0x1.917a6bc29b42cp-4, 0x1.fd88da3d12526p-1,
    -0x1.8f8b83c69a60bp-3, 0x1.f6297cff75cb0p-1,
    -0x1.294062ed59f06p-2, 0x1.e9f4156c62ddap-1,
    -0x1.87de2a6aea963p-2, 0x1.d906bcf328d46p-1,
    -0x1.e2b5d3806f63bp-2, 0x1.c38b2f180bdb1p-1,
    -0x1.1c73b39ae68c8p-1, 0x1.a9b66290ea1a3p-1,
    -0x1.44cf325091dd6p-1, 0x1.8bc806b151741p-1,
    -0x1.6a09e667f3bcdp-1, 0x1.6a09e667f3bcdp-1,
    -0x1.8bc806b151741p-1, 0x1.44cf325091dd6p-1,
    -0x1.a9b66290ea1a3p-1, 0x1.1c73b39ae68c8p-1,
    -0x1.c38b2f180bdb1p-1, 0x1.e2b5d3806f63bp-2,
    -0x1.d906bcf328d46p-1, 0x1.87de2a6aea963p-2,
    -0x1.e9f4156c62ddap-1, 0x1.294062ed59f06p-2,
    -0x1.f6297cff75cb0p-1, 0x1.8f8b83c69a60bp-3,
    -0x1.fd88da3d12526p-1, 0x1.917a6bc29b42cp-4,
    -0x1.0000000000000p+0, 0.0,
    -0x1.fd88da3d12526p-1, -0x1.917a6bc29b42cp-4,
    -0x1.f6297cff75cb0p-1, -0x1.8f8b83c69a60bp-3,
    -0x1.e9f4156c62ddap-1, -0x1.294062ed59f06p-2,
    -0x1.d906bcf328d46p-1, -0x1.87de2a6aea963p-2,
    -0x1.c38b2f180bdb1p-1, -0x1.e2b5d3806f63bp-2,
    -0x1.a9b66290ea1a3p-1, -0x1.1c73b39ae68c8p-1,
    -0x1.8bc806b151741p-1, -0x1.44cf325091dd6p-1,
    -0x1.6a09e667f3bcdp-1, -0x1.6a09e667f3bcdp-1,
    -0x1.44cf325091dd6p-1, -0x1.8bc806b151741p-1,
    -0x1.1c73b39ae68c8p-1, -0x1.a9b66290ea1a3p-1,
    -0x1.e2b5d3806f63bp-2, -0x1.c38b2f180bdb1p-1,
    -0x1.87de2a6aea963p-2, -0x1.d906bcf328d46p-1,
    -0x1.294062ed59f06p-2, -0x1.e9f4156c62ddap-1,
    -0x1.8f8b83c69a60bp-3, -0x1.f6297cff75cb0p-1,
    -0x1.917a6bc29b42cp-4, -0x1.fd88da3d12526p-1,
    0.0, -0x1.0000000000000p+0,
    0x1.917a6bc29b42cp-4, -0x1.fd88da3d12526p-1,
    0x1.8f8b83c69a60bp-3, -0x1.f6297cff75cb0p-1,
    0x1.294062ed59f06p-2, -0x1.e9f4156c62ddap-1,
    0x1.87de2a6aea963p-2, -0x1.d906bcf328d46p-1,
    0x1.e2b5d3806f63bp-2, -0x1.c38b2f180bdb1p-1,
    0x1.1c73b39ae68c8p-1, -0x1.a9b66290ea1a3p-1,
    0x1.44cf325091dd6p-1, -0x1.8bc806b151741p-1,
    0x1.6a09e667f3bcdp-1, -0x1.6a09e667f3bcdp-1,
    0x1.8bc806b151741p-1, -0x1.44cf325091dd6p-1,
    0x1.a9b66290ea1a3p-1, -0x1.1c73b39ae68c8p-1,
    0x1.c38b2f180bdb1p-1, -0x1.e2b5d3806f63bp-2,
    0x1.d906bcf328d46p-1, -0x1.87de2a6aea963p-2,
    0x1.e9f4156c62ddap-1, -0x1.294062ed59f06p-2,
    0x1.f6297cff75cb0p-1, -0x1.8f8b83c69a60bp-3,
    0x1.fd88da3d12526p-1, -0x1.917a6bc29b42cp-4};
  phz_sc_tab[lane] = k[lane];
  phz_sc_tab[64 + lane] = k[64 + lane];
  phz_log_tab[lane] = lg[lane];
  phz_log_tab[64 + lane] = lg[64 + lane];
}
__device__ __forceinline__ void tab_sincos_at(double r, int i, double* s, double* c) {
  const double ck = phz_sc_tab[2 * i], sk = phz_sc_tab[2 * i + 1];
  const double r2 = r * r;
  const double ps = fma(r2, fma(r2, -1.0 / 5040.0, 1.0 / 120.0), -1.0 / 6.0);
  const double sr = fma(r * r2, ps, r);
  const double qc = fma(r2, fma(r2, fma(r2, 1.0 / 40320.0, -1.0 / 720.0), 1.0 / 24.0), -0.5);
  const double cr = fma(r2, qc, 1.0);
  *s = fma(sk, cr, ck * sr);
  *c = fma(ck, cr, -(sk * sr));
}
__device__ __forceinline__ void tab_sincos(double x, double* s, double* c) {
  const double t = x * 0x1.45f306dc9c883p+3;  // 64 / 2 pi
  const double k = rint(t);
  const double r = fma(-k, 0x1.110b4611a6263p-30, fma(-k, 0x1.921fb50000000p-4, x));
  tab_sincos_at(r, cvt_sat_i32(k) & 63, s, c);  // a diverged world's NaN reads entry 0
}
// sin and cos of an f32 angle x: the reduction of the f64 angle_sincos (x is
// exact in f64), then in f32 the Taylor series of sin r through r^9 and of
// cos r through r^10 (truncation below 3e-9 on |r| <= pi/4) in Horner's form
// (each step one fma with a literal), and the quadrant from the low word of t.
// No large-argument branch: the reduction is exact for |x| < 1.6e6.
__device__ __forceinline__ void angle_sincos(float xf, float* s, float* c) {
  constexpr double M = 6755399441055744.0;  // 1.5 * 2^52
  const double x = xf;
  const double t = fma(x, 0x1.45f306dc9c883p-1, M);
  const double k = t - M;
  const float r = (float)fma(-k, 0x1.0b4611a626331p-34, fma(-k, 0x1.921fb54400000p+0, x));
  const float u = -(r * r);
  float p = fmaf(u, 1.0f / 362880.0f, 1.0f / 5040.0f);
  p = fmaf(u, p, 1.0f / 120.0f);
  p = fmaf(u, p, 1.0f / 6.0f);
  const float sr = fmaf(r * u, p, r);
  float q = fmaf(u, 1.0f / 3628800.0f, 1.0f / 40320.0f);
  q = fmaf(u, q, 1.0f / 720.0f);
  q = fmaf(u, q, 1.0f / 24.0f);
  q = fmaf(u, q, 0.5f);
  const float cr = fmaf(u, q, 1.0f);
  const unsigned n = (unsigned)__builtin_bit_cast(unsigned long long, t);
  const bool odd = n & 1u;
  const unsigned ss = (n & 2u) << 30, cs = ((n + 1u) & 2u) << 30;
  *s = __builtin_bit_cast(float, __builtin_bit_cast(unsigned, odd ? cr : sr) ^ ss);
  *c = __builtin_bit_cast(float, __builtin_bit_cast(unsigned, odd ? sr : cr) ^ cs);
}
// sin and cos of a revolute joint's f32 angle, for its rotation matrix, where
// the absolute error is what counts: x in turns, t = x / 2pi in f64 (its
// rounding 1e-16 relative), reduced to its fractional part in [-1/2, 1/2] in
// f64 and rounded to f32 (3e-8 turns), then the hardware v_sin_f32 /
// v_cos_f32, which take turns: their largest error measured on gfx950 was
// 1.25e-7 absolute, over [0, 1) turns and over joint angles in [-60, 60] rad.
// About 3e-7 absolute in all, against 6e-8 for angle_sincos, in seven
// instructions instead of about twenty. angle_sincos stays where a small
// angle's relative error matters (a free joint's quaternion exponential).
__device__ __forceinline__ void rev_sincos(float xf, float* s, float* c) {
  const double t = (double)xf * 0.15915494309189535;
  const float x = (float)(t - rint(t));
  *s = __builtin_amdgcn_sinf(x);
  *c = __builtin_amdgcn_cosf(x);
}
__device__ __forceinline__ void rev_sincos(double x, double* s, double* c) { tab_sincos(x, s, c); }
// ln x for a normal x > 0 from the LDS table phz_log_tab (Tang's method),
// within about 1 ulp: the f64 Box-Muller logarithms (the step kernels'
// ln(1 - u), the policy kernel's ln u1). From x's
// high word h by integer arithmetic alone: t = h - 0x3FE62000, k = t >> 20
// (arithmetic) and z = x / 2^k, so that z lies in [OFF, 2 OFF), OFF =
// 0x1.62p-1 (about 0.691); bits 14..19 of t pick one of 64 intervals of z,
// 2^-7 wide below 1 and 2^-6 above. The table holds for each interval invc,
// the double nearest 1 / (its midpoint), and logc, the double nearest
// -ln invc; the interval around 1, [1 - 2^-8, 1 + 2^-7), has invc = 1 and
// logc = 0 exactly, so that x near 1 keeps its relative accuracy. Then
// r = z invc - 1 by one fma (|r| <= 2^-7, rounded once), ln x = k ln2 + logc
// + log1p r, log1p r through r^8 in Estrin's form (truncation below 2^-59
// of r). About 20 VALU instructions and one LDS read, where an atanh series
// on [sqrt(1/2), sqrt(2)) takes about 33 and the library log about 90.
__device__ __forceinline__ double tab_log(double x) {
  const u64 b = __builtin_bit_cast(u64, x);
  const unsigned h = (unsigned)(b >> 32);
  const int t = (int)(h - 0x3FE62000u);
  const int k = t >> 20;
  const int i = (t >> 14) & 63;
  const unsigned zh = h - ((unsigned)t & 0xFFF00000u);
  const double z = __builtin_bit_cast(double, ((u64)zh << 32) | (b & 0xFFFFFFFFull));
  const double invc = phz_log_tab[2 * i], logc = phz_log_tab[2 * i + 1];
  const double r = fma(z, invc, -1.0);
  const double r2 = r * r;
  const double r4 = r2 * r2;
  const double a = fma(r, 1.0 / 3.0, -0.5);
  const double bq = fma(r, 1.0 / 5.0, -0.25);
  const double c = fma(r2, -0.125, fma(r, 1.0 / 7.0, -1.0 / 6.0));
  const double p = fma(r2, fma(r4, c, fma(r2, bq, a)), r);
  const double fk = (double)k;
  return fma(fk, 0x1.62e42fefa3800p-1, logc) + fma(fk, 0x1.ef35793c76730p-45, p);
}
// sqrt y (f64) for y = 0 or a normal y >= 2^-1000: the hardware v_rsq_f64
// estimate of 1 / sqrt y, one Goldschmidt step for g ~ sqrt y and h ~
// 1 / (2 sqrt y), then two corrections g += (y - g^2) h, each residual one
// fma; correctly rounded but for rare near-ties. The library routine adds a
// rescaling for tiny and huge y and a class test for 0 and inf; here y = 0
// takes the estimate of 2^-1000 and comes out 0 exactly (g = 0 * a).
__device__ __forceinline__ double nr_sqrt(double y) {
  const double a = __builtin_amdgcn_rsq(fmax(y, 0x1p-1000));
  double g = y * a, h = 0.5 * a;
  const double e = fma(-g, h, 0.5);
  g = fma(g, e, g);
  h = fma(h, e, h);
  g = fma(fma(-g, g, y), h, g);
  return fma(fma(-g, g, y), h, g);
}
// The f32 Box-Muller radius sqrt(-2 ln(1 - u)) of a uniform u in [0, 1): the
// hardware log2 and square root (1 - u >= 2^-24, never denormal), a few ulp
// from the correctly rounded value, for the synthetic control stream. The
// f64 radius is box_muller(u64&, double*, ...) below.
__device__ __forceinline__ float bm_radius(float u) {
  return __builtin_amdgcn_sqrtf(-1.3862943611198906f * __builtin_amdgcn_logf(1.0f - u));
}
// sin and cos of the f32 Box-Muller angle 2 pi u for a uniform u in [0, 1): u
// is the angle in turns, which the hardware v_sin_f32 / v_cos_f32 take as they
// are (1.25e-7 absolute at most, see angle_sincos(float)).
__device__ __forceinline__ void turn_sincos(float u, float* s, float* c) {
  *s = __builtin_amdgcn_sinf(u);
  *c = __builtin_amdgcn_cosf(u);
}
// sin and cos of a joint angle in f64 for the f32 kernels' penetration chain:
// tab_sincos from the LDS table, which those kernels fill as the f64 kernels
// do (within 2 ulp; the Taylor form through r^13 it replaced truncated at
// 3e-14 and took about 35 VALU instructions and thirteen constants).
__device__ __forceinline__ void joint_sincos64(double x, double* s, double* c) { tab_sincos(x, s, c); }
__device__ __forceinline__ float dsqrt(float x) { return sqrtf(x); }
__device__ __forceinline__ double dlog(double x) { return log(x); }
__device__ __forceinline__ float dlog(float x) { return logf(x); }
__device__ __forceinline__ double datan2(double y, double x) { return atan2(y, x); }
__device__ __forceinline__ double dpow(double x, double y) { return pow(x, y); }
__device__ __forceinline__ float dpow(float x, float y) { return powf(x, y); }
__device__ __forceinline__ double dtanh(double x) { return tanh(x); }
__device__ __forceinline__ float dtanh(float x) { return tanhf(x); }
__device__ __forceinline__ float datan2(float y, float x) { return atan2f(y, x); }
// Reciprocal on the ABA and penalty-contact paths. f32: the hardware
// v_rcp_f32 (within 1 ulp) in place of the correctly rounded division's
// eleven-instruction expansion; the f32 kernels' per-step bound is 1e-4 and
// one ulp is 6e-8. f64: the hardware v_rcp_f64 estimate refined by two Newton
// steps r += r (1 - x r), within about 1 ulp for a normal x, five
// instructions against the correctly rounded division's eleven (its scaling
// for extreme exponents and final fixup); the f64 bound is 1e-10 per step and
// one ulp 1.1e-16. The impulse solve and the heightfield cell lookup keep
// their correctly rounded divisions.
__device__ __forceinline__ float frcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ double frcp(double x) {
  double r = __builtin_amdgcn_rcp(x);
  r = fma(fma(-x, r, 1.0), r, r);
  return fma(fma(-x, r, 1.0), r, r);
}
// a / b: f32 through the hardware reciprocal (about 2 ulp); f64 q = a frcp(b)
// and one residual correction q += (a - b q) frcp(b) (about 1 ulp).
__device__ __forceinline__ float fdiv(float a, float b) { return a * __builtin_amdgcn_rcpf(b); }
__device__ __forceinline__ double fdiv(double a, double b) {
  const double r = frcp(b);
  const double q = a * r;
  return fma(fma(-b, q, a), r, q);
}
// Square root on the penalty-contact path: f32 the hardware v_sqrt_f32 (within
// 1 ulp, no correction sequence), f64 nr_sqrt (0 or a normal x >= 2^-1000; a
// smaller positive x gives a result below 2^-499 rather than its root).
__device__ __forceinline__ float fsqrt(float x) { return __builtin_amdgcn_sqrtf(x); }
__device__ __forceinline__ double fsqrt(double x) { return nr_sqrt(x); }
// 1 / sqrt(x): f32 the hardware v_rsq_f32 (about 1 ulp); f64 the hardware
// v_rsq_f64 estimate refined by two Newton steps y += y (1/2 - (x/2) y^2)
// (about 2 ulp, x normal).
__device__ __forceinline__ float frsqrt(float x) { return __builtin_amdgcn_rsqf(x); }
__device__ __forceinline__ double frsqrt(double x) {
  const double h = 0.5 * x;
  double y = __builtin_amdgcn_rsq(x);
  y = fma(y, fma(-(h * y), y, 0.5), y);
  return fma(y, fma(-(h * y), y, 0.5), y);
}
// The friction-loss argument qd / 1e-3: f32 multiplies by 1e3 (within an ulp
// of the quotient), f64 divides as the oracle does.
__device__ __forceinline__ float per_milli(float x) { return x * 1e3f; }
__device__ __forceinline__ double per_milli(double x) { return x / 1e-3; }
template <class T> __device__ __forceinline__ T dmax(T a, T b) { return a > b ? a : b; }
template <class T> __device__ __forceinline__ T dmin(T a, T b) { return a < b ? a : b; }
template <class T> __device__ __forceinline__ T dabs(T a) { return a < T(0) ? -a : a; }
template <class T> __device__ __forceinline__ T dsign(T a) { return a > T(0) ? T(1) : (a < T(0) ? T(-1) : T(0)); }
// Small-angle thresholds of quat exp/log: f64::EPSILON on the f64 path
// (crates/phyz-math/src/lib.rs:48, 67), 1e-6 on the f32 path
// (crates/phyz-gpu/cuda/phyz_kernels.cu:250, 282).
template <class T> struct Eps;
template <> struct Eps<double> { static constexpr double v = 2.220446049250313e-16; };
template <> struct Eps<float> { static constexpr float v = 1e-6f; };

// From here to the end of the file (vector and spatial algebra, contact laws,
// the articulated-body passes, integration) a kernel built with PHZ_REASSOC
// lets the compiler reassociate floating-point sums and products: a change at
// the rounding level, since nothing below relies on the order of its
// operations (no compensated sums, no magic-number rounding, no argument
// reduction). The closed-form sines, cosines and logarithms above keep their
// written order in every build.
#if PHZ_REASSOC
#pragma clang fp reassociate(on)
#endif
template <class T> struct V3 { T x, y, z; };
template <class T> __device__ __forceinline__ V3<T> v3(T x, T y, T z) { return V3<T>{x, y, z}; }
template <class T> __device__ __forceinline__ V3<T> operator+(V3<T> a, V3<T> b) { return {a.x + b.x, a.y + b.y, a.z + b.z}; }
template <class T> __device__ __forceinline__ V3<T> operator-(V3<T> a, V3<T> b) { return {a.x - b.x, a.y - b.y, a.z - b.z}; }
template <class T> __device__ __forceinline__ V3<T> operator*(V3<T> a, T s) { return {a.x * s, a.y * s, a.z * s}; }
template <class T> __device__ __forceinline__ T dot(V3<T> a, V3<T> b) { return a.x * b.x + a.y * b.y + a.z * b.z; }
template <class T> __device__ __forceinline__ V3<T> cross(V3<T> a, V3<T> b) {
  return {a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x};
}
// Component-wise select: a struct-valued ?: can become a select between two
// stack addresses, which keeps the operands out of registers.
template <class T> __device__ __forceinline__ V3<T> sel(bool c, V3<T> a, V3<T> b) {
  return {c ? a.x : b.x, c ? a.y : b.y, c ? a.z : b.z};
}
template <class T> struct SV { V3<T> a, l; };  // [angular; linear]
template <class T> __device__ __forceinline__ SV<T> operator+(SV<T> x, SV<T> y) { return {x.a + y.a, x.l + y.l}; }
template <class T> __device__ __forceinline__ SV<T> operator-(SV<T> x, SV<T> y) { return {x.a - y.a, x.l - y.l}; }
template <class T> __device__ __forceinline__ SV<T> operator*(SV<T> x, T s) { return {x.a * s, x.l * s}; }
template <class T> __device__ __forceinline__ T sv_get(const SV<T>& s, int k) {
  return k == 0 ? s.a.x : k == 1 ? s.a.y : k == 2 ? s.a.z : k == 3 ? s.l.x : k == 4 ? s.l.y : s.l.z;
}
template <class T> __device__ __forceinline__ void sv_set(SV<T>& s, int k, T v) {
  if (k == 0) s.a.x = v; else if (k == 1) s.a.y = v; else if (k == 2) s.a.z = v;
  else if (k == 3) s.l.x = v; else if (k == 4) s.l.y = v; else s.l.z = v;
}
template <class T> __device__ __forceinline__ T dot(const SV<T>& x, const SV<T>& y) { return dot(x.a, y.a) + dot(x.l, y.l); }
template <class T> __device__ __forceinline__ SV<T> cross_motion(const SV<T>& v, const SV<T>& m) {
  return {cross(v.a, m.a), cross(v.a, m.l) + cross(v.l, m.a)};
}
template <class T> __device__ __forceinline__ SV<T> cross_force(const SV<T>& v, const SV<T>& f) {
  return {cross(v.a, f.a) + cross(v.l, f.l), cross(v.a, f.l)};
}

// Row-major 3x3.
template <class T> struct R3 { T m[9]; };
template <class T> __device__ __forceinline__ V3<T> mul(const R3<T>& r, V3<T> v) {
  return {r.m[0] * v.x + r.m[1] * v.y + r.m[2] * v.z, r.m[3] * v.x + r.m[4] * v.y + r.m[5] * v.z,
          r.m[6] * v.x + r.m[7] * v.y + r.m[8] * v.z};
}
template <class T> __device__ __forceinline__ V3<T> tmul(const R3<T>& r, V3<T> v) {
  return {r.m[0] * v.x + r.m[3] * v.y + r.m[6] * v.z, r.m[1] * v.x + r.m[4] * v.y + r.m[7] * v.z,
          r.m[2] * v.x + r.m[5] * v.y + r.m[8] * v.z};
}
template <class T> __device__ __forceinline__ R3<T> mul(const R3<T>& a, const R3<T>& b) {
  R3<T> r;
#pragma unroll
  for (int i = 0; i < 3; i++)
#pragma unroll
    for (int j = 0; j < 3; j++) r.m[i * 3 + j] = a.m[i * 3] * b.m[j] + a.m[i * 3 + 1] * b.m[3 + j] + a.m[i * 3 + 2] * b.m[6 + j];
  return r;
}
template <class T> __device__ __forceinline__ R3<T> mul_bt(const R3<T>& a, const R3<T>& b) {  // a b^T
  R3<T> r;
#pragma unroll
  for (int i = 0; i < 3; i++)
#pragma unroll
    for (int j = 0; j < 3; j++)
      r.m[i * 3 + j] = a.m[i * 3] * b.m[j * 3] + a.m[i * 3 + 1] * b.m[j * 3 + 1] + a.m[i * 3 + 2] * b.m[j * 3 + 2];
  return r;
}
template <class T> __device__ __forceinline__ R3<T> transpose(const R3<T>& a) {
  return R3<T>{{a.m[0], a.m[3], a.m[6], a.m[1], a.m[4], a.m[7], a.m[2], a.m[5], a.m[8]}};
}

// Plucker transform: X v = [E w; E (v - r x w)], X^T f = [E^T t + r x E^T f; E^T f].
template <class T> struct Xf { R3<T> E; V3<T> r; };
template <class T> __device__ __forceinline__ SV<T> apply_motion(const Xf<T>& x, const SV<T>& v) {
  return {mul(x.E, v.a), mul(x.E, v.l - cross(x.r, v.a))};
}
template <class T> __device__ __forceinline__ SV<T> inv_apply_force(const Xf<T>& x, const SV<T>& f) {
  V3<T> rf = tmul(x.E, f.l);
  return {tmul(x.E, f.a) + cross(x.r, rf), rf};
}

// Symmetric 6x6 as blocks [A B; B^T C]; A and C stored as upper triangles
// (00 01 02 11 12 22), B full row-major.
template <class T> struct Sym { T a[6]; T b[9]; T c[6]; };
__device__ __forceinline__ constexpr int sx(int i, int j) {
  return i <= j ? (i == 0 ? j : (i == 1 ? 2 + j : 5)) : (j == 0 ? i : (j == 1 ? 2 + i : 5));
}
template <class T> __device__ __forceinline__ T sym_get(const Sym<T>& s, int i, int j) {
  if (i < 3 && j < 3) return s.a[sx(i, j)];
  if (i >= 3 && j >= 3) return s.c[sx(i - 3, j - 3)];
  if (i < 3) return s.b[i * 3 + (j - 3)];
  return s.b[j * 3 + (i - 3)];
}
template <class T> __device__ __forceinline__ SV<T> sym_mul(const Sym<T>& s, const SV<T>& v) {
  SV<T> r;
#pragma unroll
  for (int i = 0; i < 6; i++) {
    T acc = sym_get(s, i, 0) * sv_get(v, 0);
#pragma unroll
    for (int j = 1; j < 6; j++) acc = acc + sym_get(s, i, j) * sv_get(v, j);
    sv_set(r, i, acc);
  }
  return r;
}
template <class T> __device__ __forceinline__ void sym_add(Sym<T>& d, const Sym<T>& s) {
#pragma unroll
  for (int k = 0; k < 6; k++) { d.a[k] = d.a[k] + s.a[k]; d.c[k] = d.c[k] + s.c[k]; }
#pragma unroll
  for (int k = 0; k < 9; k++) d.b[k] = d.b[k] + s.b[k];
}
// E^T M E for symmetric M (upper triangles).
template <class T> __device__ __forceinline__ void sym_rot(const T* m, const R3<T>& E, T* out) {
  T t[9];
#pragma unroll
  for (int i = 0; i < 3; i++)
#pragma unroll
    for (int j = 0; j < 3; j++) t[i * 3 + j] = m[sx(i, 0)] * E.m[j] + m[sx(i, 1)] * E.m[3 + j] + m[sx(i, 2)] * E.m[6 + j];
#pragma unroll
  for (int i = 0; i < 3; i++)
#pragma unroll
    for (int j = i; j < 3; j++) out[sx(i, j)] = E.m[i] * t[j] + E.m[3 + i] * t[3 + j] + E.m[6 + i] * t[6 + j];
}
// E^T M E for E a rotation about coordinate axis k: E_kk = 1, no other
// entries in row or column k, and on the plane (u, w) = (k + 1, k + 2) mod 3
// the block [[c, s], [-s, c]]. The plane block of E^T M E turns by twice the
// angle: with h = (m_uu + m_ww) / 2, d = (m_uu - m_ww) / 2,
//   m'_uu = h + d cos2 - m_uw sin2,  m'_ww = h - d cos2 + m_uw sin2,
//   m'_uw = d sin2 + m_uw cos2,
// and the plane entries of column k turn by the angle itself. c2h, s2h are
// cos2 / 2 = 1/2 - s^2 and sin2 / 2 = c s.
template <class T, int k>
__device__ __forceinline__ void sym_rot_axis(const T* m, T c, T s, T c2h, T s2h, T* out) {
  constexpr int u = (k + 1) % 3, w = (k + 2) % 3;
  const T muu = m[sx(u, u)], mww = m[sx(w, w)], muw = m[sx(u, w)];
  const T h2 = muu + mww, d2 = muu - mww;
  const T t = d2 * c2h - muw * (s2h + s2h);
  out[sx(u, u)] = T(0.5) * h2 + t;
  out[sx(w, w)] = T(0.5) * h2 - t;
  out[sx(u, w)] = d2 * s2h + muw * (c2h + c2h);
  const T muk = m[sx(u, k)], mwk = m[sx(w, k)];
  out[sx(u, k)] = c * muk - s * mwk;
  out[sx(w, k)] = s * muk + c * mwk;
  out[sx(k, k)] = m[sx(k, k)];
}
// The same for a general 3x3 M (row-major): with p, r, t, q the halved sums
// m_uu + m_ww, m_uu - m_ww, m_uw + m_wu, m_uw - m_wu, the plane block is
//   m'_uu = p + (r cos2 - t sin2),  m'_ww = p - (r cos2 - t sin2),
//   m'_uw = q + (r sin2 + t cos2),  m'_wu = -q + (r sin2 + t cos2);
// row k and column k turn by the angle.
template <class T, int k>
__device__ __forceinline__ void gen_rot_axis(const T* m, T c, T s, T c2h, T s2h, T* out) {
  constexpr int u = (k + 1) % 3, w = (k + 2) % 3;
  const T muu = m[u * 3 + u], mww = m[w * 3 + w], muw = m[u * 3 + w], mwu = m[w * 3 + u];
  const T p2 = muu + mww, r2 = muu - mww, t2 = muw + mwu, q2 = muw - mwu;
  const T rr = r2 * c2h - t2 * s2h, tt = r2 * s2h + t2 * c2h;
  out[u * 3 + u] = T(0.5) * p2 + rr;
  out[w * 3 + w] = T(0.5) * p2 - rr;
  out[u * 3 + w] = T(0.5) * q2 + tt;
  out[w * 3 + u] = tt - T(0.5) * q2;
  out[u * 3 + k] = c * m[u * 3 + k] - s * m[w * 3 + k];
  out[w * 3 + k] = s * m[u * 3 + k] + c * m[w * 3 + k];
  out[k * 3 + u] = c * m[k * 3 + u] - s * m[k * 3 + w];
  out[k * 3 + w] = s * m[k * 3 + u] + c * m[k * 3 + w];
  out[k * 3 + k] = m[k * 3 + k];
}
// X^T I X = T^T (Rot^T I Rot) T with T = [1 0; -r x 1]:
//   A1 = E^T A E, B1 = E^T B E, C1 = E^T C E
//   B2 = B1 + r x C1,  A2 = A1 - B1 r x + r x B2^T,  C2 = C1
// KAX >= 0: X.E is a rotation about coordinate axis KAX (see sym_rot_axis).
template <class T, int KAX = -1> __device__ __forceinline__ Sym<T> sym_xtix(const Sym<T>& I, const Xf<T>& X) {
  const R3<T>& E = X.E;
  Sym<T> o;
  T b1[9];
  if constexpr (KAX >= 0) {
    constexpr int u = (KAX + 1) % 3, w = (KAX + 2) % 3;
    const T c = E.m[u * 3 + u], s = E.m[u * 3 + w];
    const T c2h = T(0.5) - s * s, s2h = c * s;
    sym_rot_axis<T, KAX>(I.a, c, s, c2h, s2h, o.a);
    sym_rot_axis<T, KAX>(I.c, c, s, c2h, s2h, o.c);
    gen_rot_axis<T, KAX>(I.b, c, s, c2h, s2h, b1);
  } else {
    sym_rot(I.a, E, o.a);
    sym_rot(I.c, E, o.c);
    T t[9];
#pragma unroll
    for (int i = 0; i < 3; i++)
#pragma unroll
      for (int j = 0; j < 3; j++) t[i * 3 + j] = I.b[i * 3] * E.m[j] + I.b[i * 3 + 1] * E.m[3 + j] + I.b[i * 3 + 2] * E.m[6 + j];
#pragma unroll
    for (int i = 0; i < 3; i++)
#pragma unroll
      for (int j = 0; j < 3; j++) b1[i * 3 + j] = E.m[i] * t[j] + E.m[3 + i] * t[3 + j] + E.m[6 + i] * t[6 + j];
  }
  const V3<T> r = X.r;
#pragma unroll
  for (int j = 0; j < 3; j++) {
    V3<T> rc = cross(r, v3(o.c[sx(0, j)], o.c[sx(1, j)], o.c[sx(2, j)]));
    o.b[j] = b1[j] + rc.x;
    o.b[3 + j] = b1[3 + j] + rc.y;
    o.b[6 + j] = b1[6 + j] + rc.z;
  }
  V3<T> rb1[3], rb2[3];
#pragma unroll
  for (int i = 0; i < 3; i++) {
    rb1[i] = cross(r, v3(b1[i * 3], b1[i * 3 + 1], b1[i * 3 + 2]));
    rb2[i] = cross(r, v3(o.b[i * 3], o.b[i * 3 + 1], o.b[i * 3 + 2]));
  }
  auto comp = [](const V3<T>& v, int k) { return k == 0 ? v.x : (k == 1 ? v.y : v.z); };
#pragma unroll
  for (int i = 0; i < 3; i++)
#pragma unroll
    for (int j = i; j < 3; j++) o.a[sx(i, j)] = o.a[sx(i, j)] + comp(rb1[i], j) + comp(rb2[j], i);
  return o;
}

// Quaternions (w, x, y, z).
template <class T> struct Q { T w, x, y, z; };
template <class T> __device__ __forceinline__ Q<T> qmul(const Q<T>& a, const Q<T>& b) {
  return {a.w * b.w - a.x * b.x - a.y * b.y - a.z * b.z, a.w * b.x + a.x * b.w + a.y * b.z - a.z * b.y,
          a.w * b.y - a.x * b.z + a.y * b.w + a.z * b.x, a.w * b.z + a.x * b.y - a.y * b.x + a.z * b.w};
}
template <class T> __device__ __forceinline__ Q<T> quat_exp(V3<T> w) {
  T ang = fsqrt(dot(w, w));
  T s, c;
  dsincos(ang * T(0.5), &s, &c);
  const bool small = ang < T(Eps<T>::v);
  T f = small ? T(0.5) : fdiv(s, dmax(ang, T(0.5) * T(Eps<T>::v)));
  return {small ? T(1) : c, w.x * f, w.y * f, w.z * f};
}
// Rotation vector of q. Outside the small-angle branch any positive scale of
// a unit quaternion gives the same result; the products of unit quaternions
// that the integration passes are unit to rounding.
template <class T> __device__ __forceinline__ V3<T> quat_log(const Q<T>& q) {
  V3<T> v = v3(q.x, q.y, q.z);
  T n = fsqrt(dot(v, v));
  const bool small = n < T(Eps<T>::v);
  T f = small ? T(2) : fdiv(T(2) * datan2(n, q.w), dmax(n, T(0.5) * T(Eps<T>::v)));
  return v * f;
}
// Rotation matrix of unit q (active), row-major.
template <class T> __device__ __forceinline__ R3<T> quat_mat(const Q<T>& q) {
  T w = q.w, x = q.x, y = q.y, z = q.z;
  return R3<T>{{T(1) - T(2) * (y * y + z * z), T(2) * (x * y - w * z), T(2) * (x * z + w * y),
                T(2) * (x * y + w * z), T(1) - T(2) * (x * x + z * z), T(2) * (y * z - w * x),
                T(2) * (x * z - w * y), T(2) * (y * z + w * x), T(1) - T(2) * (x * x + y * y)}};
}
template <class T> __device__ __forceinline__ V3<T> qrotate(const Q<T>& q, V3<T> p) {
  V3<T> u = v3(q.x, q.y, q.z);
  V3<T> t = cross(u, p) * T(2);
  return p + t * q.w + cross(u, t);
}

// ── per-world RNG: SplitMix64 world seed + xorshift64 ───────────────────────
// (crates/phyz-gpu/src/policy_pipeline.rs:417-456)
__device__ __forceinline__ u64 xorshift64(u64& s) {
  u64 x = s;
  x ^= x << 13;
  x ^= x >> 7;
  x ^= x << 17;
  s = x;
  return x;
}
// Uniform on [0, 1): 53 bits on the f64 path, 24 bits on the f32 path (both
// exact). f64: (x >> 11) 2^-53 = hi 2^-32 + (lo >> 11) 2^-53 for the 32-bit
// words hi, lo of x, one fma of two exact conversions, the sum exact.
__device__ __forceinline__ double uniform01(u64& s, double) {
  const u64 x = xorshift64(s);
  return fma((double)(unsigned)(x >> 32), 0x1p-32, (double)((unsigned)x >> 11) * 0x1p-53);
}
__device__ __forceinline__ float uniform01(u64& s, float) { return (float)(unsigned)(xorshift64(s) >> 40) * 0x1.0p-24f; }
// One Box-Muller pair from two uniforms u1, u2 (drawn in that order): the
// radius sqrt(-2 ln(1 - u1)) and the sine and cosine of 2 pi u2. f64: 1 - u1
// is formed exactly from the words of the draw (1 - (lo >> 11) 2^-53 is exact,
// and so is the fma that takes hi 2^-32 from it), ln by tab_log, sqrt by
// nr_sqrt; the angle is reduced in turns, where it is exact: t = 64 u2 (no
// rounding), k = rint(t), and r = (t - k) 2 pi / 64 (t - k exact, one
// rounding in the product), then tab_sincos_at.
__device__ __forceinline__ void box_muller(u64& s, float* r, float* sn, float* cs) {
  const float u1 = uniform01(s, 0.0f);
  const float u2 = uniform01(s, 0.0f);
  *r = bm_radius(u1);
  turn_sincos(u2, sn, cs);
}
__device__ __forceinline__ void box_muller(u64& s, double* r, double* sn, double* cs) {
  const u64 x1 = xorshift64(s);
  const u64 x2 = xorshift64(s);
  const double om = fma(-(double)(unsigned)(x1 >> 32), 0x1p-32, fma(-(double)((unsigned)x1 >> 11), 0x1p-53, 1.0));
  *r = nr_sqrt(-2.0 * tab_log(om));
  const double t = fma((double)(unsigned)(x2 >> 32), 0x1p-26, (double)((unsigned)x2 >> 11) * 0x1p-47);
  const double k = rint(t);
  tab_sincos_at((t - k) * 0x1.921fb54442d18p-4, cvt_sat_i32(k) & 63, sn, cs);
}

// ── kernel arguments ─────────────────────────────────────────────────────────
// Structure-of-arrays state: element (j, w) at j * stride + w.
struct StepArgs {
  void* q;             // [nq][stride]
  void* v;             // [nv][stride]
  void* ctrl;          // [nctrl][stride]: one row per actuator, or per DOF without actuators
  void* qdd;           // [nv][stride], last step's accelerations
  const void* targets; // [npd][stride]
  u64* rng;            // [stride]
  void* contact_rows;  // [nb * 8][stride], last step's contact readback
  void* ext;           // [nb * 6][stride], contact forces carried between steps (impulse mode)
  void* imp;           // [nb * 48][stride], warm-start impulses: 24 ground, 24 plane per body (impulse mode)
  const void* hf;      // heightfield nodes [ny][nx], f64 in every kernel
  double hf_ox, hf_oy, hf_oz, hf_cell;
  int hf_nx, hf_ny;
  int nworld;
  int stride;
  int nsteps;
  int write_contacts;
};

// Model-derived constants evaluated in double on the host side of the
// compiler, then rounded once to T.
template <class M, int i> struct BodyK {
  static constexpr int jt = M::jtype[i];
  static constexpr int nd = ndof_of(jt);
  static constexpr int parent = M::parent[i];
};

// ── f64 penetration chain of the f32 kernels ────────────────────────────────
// A contact's penetration depth is the small difference of two heights of
// order a metre: the ground's and the contact point's, which sums the joint
// offsets of the whole chain from the root. At a penalty stiffness of 1e4 N/m
// the f32 rounding of that sum (1e-7 m) is a force error of 1e-3 N, and on
// light feet at rest a per-step qdd error above 1e-4 of max|qdd|. So the f32
// kernels with contact carry, beside their f32 transforms, the world z-axis in
// each contact-path body's frame (the third row of its body->world rotation)
// and the world height of its origin in f64, and evaluate the depth from
// them. Everything else about the contact, and the dynamics, stays f32.
template <class M, class T> constexpr bool pen64() { return M::HAS_CONTACT && sizeof(T) == 4; }
// Over a heightfield the depth also needs the contact point's world x and y,
// and against a body-attached plane the plane's whole frame: such kernels
// carry the chain's other two rows and origins too.
template <class M, class T> constexpr bool full64() { return pen64<M, T>() && (M::HAS_HF || M::PLANE >= 0); }
// Ground contact points of body i (a box's 8 corners, one support point
// otherwise) and where they start in the per-world list of contact points.
template <class M> constexpr int ground_pts(int i) {
  return M::gtype[i] == G_NONE ? 0 : (M::gtype[i] == G_BOX ? 8 : 1);
}
template <class M> constexpr int ground_off(int i) {
  int s = 0;
  for (int k = 0; k < i; k++) s += ground_pts<M>(k);
  return s;
}


template <class M, class T, int i> __device__ __forceinline__ Sym<T> rigid_inertia() {
  Sym<T> s;
#pragma unroll
  for (int k = 0; k < 6; k++) { s.a[k] = T(M::inA[i][k]); s.c[k] = T(M::inC[i][k]); }
#pragma unroll
  for (int k = 0; k < 9; k++) s.b[k] = T(M::inB[i][k]);
  return s;
}
template <class M, class T, int i> __device__ __forceinline__ SV<T> subspace(int k) {
  constexpr int jt = M::jtype[i];
  SV<T> s = {v3(T(0), T(0), T(0)), v3(T(0), T(0), T(0))};
  if constexpr (jt == J_REV) s.a = v3(T(M::axis[i][0]), T(M::axis[i][1]), T(M::axis[i][2]));
  else if constexpr (jt == J_PRIS) s.l = v3(T(M::axis[i][0]), T(M::axis[i][1]), T(M::axis[i][2]));
  else sv_set(s, k, T(1));
  return s;
}

// Effective mass of body i at body-frame offset r along unit direction u
// (crates/phyz-gpu/cuda/phyz_kernels.cu:545-571): 1 / (1/m + a . I_c^-1 a),
// a = (r - com) x u. FAST takes the reciprocal with frcp (penalty contact).
template <class M, class T, int i, bool FAST = false> __device__ __forceinline__ T eff_mass(V3<T> r, V3<T> u) {
  if constexpr (!(M::mass[i] > 0.0)) {
    return T(1e30);
  } else {
    V3<T> rc = r - v3(T(M::com[i][0]), T(M::com[i][1]), T(M::com[i][2]));
    V3<T> a = cross(rc, u);
    // Cofactor inverse of the COM inertia, upper triangle (zeros if singular).
    V3<T> ia = v3(T(M::iinv[i][0]) * a.x + T(M::iinv[i][1]) * a.y + T(M::iinv[i][2]) * a.z,
                  T(M::iinv[i][1]) * a.x + T(M::iinv[i][3]) * a.y + T(M::iinv[i][4]) * a.z,
                  T(M::iinv[i][2]) * a.x + T(M::iinv[i][4]) * a.y + T(M::iinv[i][5]) * a.z);
    T ang = dmax(dot(a, ia), T(0));
    const T den = T(1.0 / M::mass[i]) + ang;
    if constexpr (FAST) return frcp(den);
    else return T(1) / den;
  }
}

// Heightfield terrain: nodes h[iy * nx + ix] and the header, uniform over a
// launch. Always f64, in f32 kernels too: the terrain's height and normal are
// evaluated in f64 at the contact point's f64 position, so that which side of
// a contact threshold a point lies on, and which cell it is in, is decided as
// the f64 oracle decides it.
template <class T> struct Terrain {
  const double* h;
  double ox, oy, oz, cell;
  int nx, ny;
};

// Cell and fraction along one axis, clamped to the grid. The cell index is in
// [0, n - 2] whatever w holds (a diverged world's NaN or inf included).
// Grid coordinate of w along one axis, clamped to the grid.
template <class T> __device__ __forceinline__ T hf_u(T w, T o, int n, T cell) {
  return n < 2 ? T(0) : dmin(dmax((w - o) / cell, T(0)), T(n - 1));
}
template <class T> __device__ __forceinline__ void hf_locate(T w, T o, int n, T cell, int& i, T& t) {
  if (n < 2) { i = 0; t = T(0); return; }
  const T u = hf_u(w, o, n, cell);
  int ii = cvt_sat_i32(u);
  ii = ii < 0 ? 0 : (ii > n - 2 ? n - 2 : ii);
  i = ii;
  t = u - T(ii);
}

// Terrain height and unit normal at world (x, y): the flat ground, or the
// bilinear heightfield with its cell-wise gradient (phyz_kernels.cu:641-664).
// hf_cell finds the cell, the fractions in it and whether x and y lie over the
// grid (outside it the height is the edge's and the gradient along that axis
// zero); hf_eval evaluates the patch. terrain_at does both in f64.
struct HfCell {
  int ix, iy;
  bool inx, iny;
};
template <class T, class S>
__device__ __forceinline__ HfCell hf_cell(const Terrain<T>& tr, S px, S py, S& tx, S& ty) {
  HfCell c;
  hf_locate(px, S(tr.ox), tr.nx, S(tr.cell), c.ix, tx);
  hf_locate(py, S(tr.oy), tr.ny, S(tr.cell), c.iy, ty);
  c.inx = tr.nx >= 2 && px >= S(tr.ox) && px <= S(tr.ox + double(tr.nx - 1) * tr.cell);
  c.iny = tr.ny >= 2 && py >= S(tr.oy) && py <= S(tr.oy + double(tr.ny - 1) * tr.cell);
  return c;
}
template <class T, class S>
__device__ __forceinline__ S hf_eval(const Terrain<T>& tr, const HfCell& c, S tx, S ty, S* grad) {
  const int ix1 = c.ix + 1 < tr.nx - 1 ? c.ix + 1 : tr.nx - 1;
  const int iy1 = c.iy + 1 < tr.ny - 1 ? c.iy + 1 : tr.ny - 1;
  const S oz = S(tr.oz);
  const S h00 = oz + S(tr.h[c.iy * tr.nx + c.ix]), h10 = oz + S(tr.h[c.iy * tr.nx + ix1]);
  const S h01 = oz + S(tr.h[iy1 * tr.nx + c.ix]), h11 = oz + S(tr.h[iy1 * tr.nx + ix1]);
  const S h = (h00 * (S(1) - tx) + h10 * tx) * (S(1) - ty) + (h01 * (S(1) - tx) + h11 * tx) * ty;
  const S cell = S(tr.cell);
  grad[0] = c.inx ? -(((h10 - h00) * (S(1) - ty) + (h11 - h01) * ty) / cell) : S(0);
  grad[1] = c.iny ? -(((h01 - h00) * (S(1) - tx) + (h11 - h10) * tx) / cell) : S(0);
  return h;
}
template <class M, class T>
__device__ __forceinline__ double terrain_at(const Terrain<T>& tr, double px, double py, V3<double>& n,
                                             HfCell* cell_out = nullptr) {
  if constexpr (!M::HAS_HF) {
    n = v3(0.0, 0.0, 1.0);
    return M::ground_h;
  } else {
    double tx, ty, g[2];
    const HfCell c = hf_cell(tr, px, py, tx, ty);
    const double h = hf_eval(tr, c, tx, ty, g);
    const V3<double> gv = v3(g[0], g[1], 1.0);
    n = gv * (1.0 / sqrt(dot(gv, gv)));  // |g| >= 1
    if (cell_out) *cell_out = c;
    return h;
  }
}
// A cell packed in one word: ix (15 bits), iy (15 bits), the two over-grid
// flags (the host limits heightfields to 32768 nodes per axis).
__device__ __forceinline__ int pack_cell(const HfCell& c) {
  return c.ix | (c.iy << 15) | (c.inx ? 1 << 30 : 0) | (c.iny ? int(1u << 31) : 0);
}
__device__ __forceinline__ HfCell unpack_cell(int w) {
  return HfCell{w & 0x7fff, (w >> 15) & 0x7fff, ((w >> 30) & 1) != 0, w < 0};
}
template <class T> __device__ __forceinline__ V3<T> to_t(const V3<double>& a) { return v3(T(a.x), T(a.y), T(a.z)); }

// A depth computed in f64 and kept in f32 for the contact law, on the same
// side of the law's activation threshold (0 in penalty mode, -margin in
// impulse mode) as the f64 value: the f32 rounding moves it by at most one
// ulp of the threshold, where the law's force is continuous in the depth
// (impulse mode's impedance vanishes at -margin), so only the decision is
// carried, not a new value.
__device__ __forceinline__ float next_above(float t) {
  if (t == 0.0f) return 1.17549435e-38f;
  const int b = __builtin_bit_cast(int, t);
  return __builtin_bit_cast(float, t > 0.0f ? b + 1 : b - 1);
}
template <class M, class T> __device__ __forceinline__ T pen_decided(double pen) {
  constexpr double thr = M::CMODE == 1 ? -M::c_margin : 0.0;
  const T t = T(thr);
  T p = T(pen);
  if constexpr (sizeof(T) == 4) {
    const bool in = pen > thr;
    p = (in && !(p > t)) ? next_above(t) : p;
    p = (!in && p > t) ? t : p;
  }
  return p;
}

// Contact point cp of body i's shape, body frame: a box corner, or the
// support point against body-frame direction d (phyz_kernels.cu:667-730).
// The shape's sign and threshold tests (which end of a capsule or cylinder,
// which corner of a mesh box, whether a cylinder's rim is defined) read dd, the
// same direction in precision D: f32 kernels with the f64 height chain pass
// the chain's f64 direction, so that the point is the one whose depth the chain
// computed. A capsule lying within f32 rounding of level would otherwise touch
// at one end and take its force at the other.
template <class M, class T, int i, class D = T>
__device__ __forceinline__ V3<T> contact_point(int cp, V3<T> d, V3<D> dd) {
  constexpr int gt = M::gtype[i];
  const R3<T> oR = R3<T>{{T(M::gorot[i][0]), T(M::gorot[i][1]), T(M::gorot[i][2]), T(M::gorot[i][3]), T(M::gorot[i][4]),
                          T(M::gorot[i][5]), T(M::gorot[i][6]), T(M::gorot[i][7]), T(M::gorot[i][8])}};
  const V3<T> oP = v3(T(M::gopos[i][0]), T(M::gopos[i][1]), T(M::gopos[i][2]));
  if constexpr (gt == G_BOX) {
    V3<T> corner = v3(T(M::gp[i][0] * ((cp & 1) ? 1.0 : -1.0)), T(M::gp[i][1] * ((cp & 2) ? 1.0 : -1.0)),
                      T(M::gp[i][2] * ((cp & 4) ? 1.0 : -1.0)));
    return oP + tmul(oR, corner);
  } else {
    const R3<D> oRd = R3<D>{{D(M::gorot[i][0]), D(M::gorot[i][1]), D(M::gorot[i][2]), D(M::gorot[i][3]),
                             D(M::gorot[i][4]), D(M::gorot[i][5]), D(M::gorot[i][6]), D(M::gorot[i][7]),
                             D(M::gorot[i][8])}};
    const V3<T> n = mul(oR, d);
    const V3<D> nd = mul(oRd, dd);
    V3<T> sp;
    if constexpr (gt == G_SPHERE) {
      sp = n * T(-M::gp[i][0]);
    } else if constexpr (gt == G_CAPSULE) {
      sp = v3(T(0), T(0), T(-0.5 * M::gp[i][1]) * T(dsign(nd.z))) - n * T(M::gp[i][0]);
    } else if constexpr (gt == G_CYLINDER) {
      const D rl = dsqrt(nd.x * nd.x + nd.y * nd.y);
      const T f = rl > D(1e-6) ? T(D(M::gp[i][0]) / dmax(rl, D(5e-7))) : T(0);
      sp = v3(-n.x * f, -n.y * f, T(-0.5 * M::gp[i][1]) * T(dsign(nd.z)));
    } else {  // mesh AABB
      sp = v3(T(0.5 * (M::gp[i][0] + M::gp[i][3])) - T(0.5 * (M::gp[i][3] - M::gp[i][0])) * T(dsign(nd.x)),
              T(0.5 * (M::gp[i][1] + M::gp[i][4])) - T(0.5 * (M::gp[i][4] - M::gp[i][1])) * T(dsign(nd.y)),
              T(0.5 * (M::gp[i][2] + M::gp[i][5])) - T(0.5 * (M::gp[i][5] - M::gp[i][2])) * T(dsign(nd.z)));
    }
    return oP + tmul(oR, sp);
  }
}
template <class M, class T, int i> __device__ __forceinline__ V3<T> contact_point(int cp, V3<T> d) {
  return contact_point<M, T, i, T>(cp, d, d);
}

// SolImp impedance with the margin taper, smoothstep restitution, and the
// contact tangent frame (phyz_kernels.cu:581-633), constants from the model.
template <class M, class T> __device__ __forceinline__ T solimp_pow(T x) {
  if constexpr (M::c_power == 1.0) return x;
  else if constexpr (M::c_power == 2.0) return x * x;
  else if constexpr (M::c_power == 3.0) return x * x * x;
  else return dpow(x, T(M::c_power));
}
// Model constants arrive clamped as SolImp clamps them: c_dmin, c_dmax in
// [1e-4, 1 - 1e-9], c_mid in [1e-6, 1 - 1e-6], c_power >= 1, and
// c_mid_pow = mid^(power-1), c_omid_pow = (1-mid)^(power-1).
template <class M, class T> __device__ __forceinline__ T solimp_at(T r) {
  if constexpr (M::c_width <= 0.0) {
    return T(M::c_dmax);
  } else {
    const T x = dmin(dmax(dabs(r) / T(M::c_width), T(0)), T(1));
    const T lo = solimp_pow<M, T>(x) / T(M::c_mid_pow);
    const T hi = T(1) - solimp_pow<M, T>(T(1) - x) / T(M::c_omid_pow);
    const T y = x <= T(M::c_mid) ? lo : hi;
    return T(M::c_dmin) + y * T(M::c_dmax - M::c_dmin);
  }
}
template <class M, class T> __device__ __forceinline__ T impedance_at(T depth) {
  if (depth >= T(0)) return solimp_at<M, T>(depth);
  if constexpr (M::c_margin <= 0.0) {
    return T(0);
  } else {
    const T gap = -depth;
    const T sc = T(1) - gap / T(M::c_margin);
    const T val = sc * sc * (T(3) - T(2) * sc) * solimp_at<M, T>(T(0));
    return gap >= T(M::c_margin) ? T(0) : val;
  }
}
template <class M, class T> __device__ __forceinline__ T restitution_at(T approach) {
  if constexpr (M::c_rest == 0.0) {
    return T(0);  // every branch below is c_rest times a finite factor
  } else if constexpr (M::c_rest_v <= 0.0) {
    return T(M::c_rest);
  } else {
    const T sp = dabs(approach);
    const T t = (sp - T(M::c_rest_v)) / T(M::c_rest_v);
    const T ramp = T(M::c_rest) * t * t * (T(3) - T(2) * t);
    return sp <= T(M::c_rest_v) ? T(0) : (sp >= T(2.0 * M::c_rest_v) ? T(M::c_rest) : ramp);
  }
}
template <class T> __device__ __forceinline__ void tangent_frame(V3<T> n, V3<T>& u, V3<T>& w) {
  const bool ax = dabs(n.x) > T(0.9);
  const V3<T> a = v3(ax ? T(0) : T(1), ax ? T(1) : T(0), T(0));
  const V3<T> c = cross(n, a);
  const T l2 = dot(c, c);
  u = sel(l2 > T(0), c * frsqrt(dmax(l2, T(1e-36))), c);
  w = cross(n, u);
}

// One warm-started Coulomb update of a contact slot (impulse mode,
// phyz_kernels.cu:874-937 and 1058-1096): normal response with SolImp/solref
// bias and restitution, tangential response clipped to the friction cone.
// a_* are the Delassus diagonals, b_* the free contact velocity components;
// slot holds (normal, tangent u, tangent w) impulses in and out.
template <class M, class T>
__device__ __forceinline__ void impulse_update(T pen, T b_n, T b_u, T b_w, T a_nn, T a_uu, T a_ww, T* slot) {
  const double dtc = M::dt > 1e-9 ? M::dt : 1e-9;
  const T bias = impedance_at<M, T>(pen) * T(M::c_erp) * dmax(pen, T(0)) / T(dtc);
  const T e = restitution_at<M, T>(dmin(b_n, T(0)));
  const T r_n = b_n * (T(1) + e) - a_nn * slot[0];
  const T fn = dmax((bias - r_n) / a_nn, T(0));
  T tu = -(b_u - a_uu * slot[1]) / a_uu;
  T tw = -(b_w - a_ww * slot[2]) / a_ww;
  const T limit = T(M::mu) * fn;
  const T tn = dsqrt(tu * tu + tw * tw);
  const T sc = tn > limit ? (tn > T(0) ? limit / dmax(tn, T(1e-30)) : T(0)) : T(1);
  slot[0] = fn;
  slot[1] = tu * sc;
  slot[2] = tw * sc;
}

template <class M, class T> struct WS;

// Depth, terrain height and unit normal (world) at contact point cp of body i.
// The f32 kernels take them from pass 1's f64 chain (pen64): over a
// heightfield the values pass 1 evaluated in f64 at the point's f64 position,
// on flat ground the ground height minus the point's f64 height; the depth is
// kept on the f64 side of the law's threshold (pen_decided), so the f32
// kernels switch a contact on and off where the f64 oracle does. The f64
// kernels evaluate them from supw.
template <class M, class T, int i>
__device__ __forceinline__ void contact_depth(const WS<M, T>& ws, const Terrain<T>& tr, int cp, const V3<T>& supw,
                                              T& pen, T& th, V3<T>& nw) {
  const int k = ground_off<M>(i) + cp;
  if constexpr (pen64<M, T>() && M::HAS_HF) {
    // Height and normal in f32 in the cell pass 1 chose in f64: continuous
    // in the point's position, so the f32 position serves.
    pen = ws.hf_pen[k];
    const HfCell c = unpack_cell(ws.hf_cellw[k]);
    T g[2];
    const T tx = hf_u(supw.x, T(tr.ox), tr.nx, T(tr.cell)) - T(c.ix);
    const T ty = hf_u(supw.y, T(tr.oy), tr.ny, T(tr.cell)) - T(c.iy);
    th = hf_eval(tr, c, tx, ty, g);
    const V3<T> gv = v3(g[0], g[1], T(1));
    nw = gv * frsqrt(dot(gv, gv));
  } else if constexpr (pen64<M, T>()) {
    pen = pen_decided<M, T>(M::ground_h - ws.cz64[k]);
    th = T(M::ground_h);
    nw = v3(T(0), T(0), T(1));
  } else {
    V3<double> n64;
    const double th64 = terrain_at<M, T>(tr, double(supw.x), double(supw.y), n64);
    pen = T(n64.z * (th64 - double(supw.z)));
    th = T(th64);
    nw = to_t<T>(n64);
  }
}

// Ground penalty contact of body i (crates/phyz-gpu/cuda/phyz_kernels.cu:804-980,
// penalty branch 939-965). Rw: body->world rotation, pw: body origin in world,
// vel: body-frame spatial velocity. Returns the body-frame spatial force. When
// `write` is set, stores the readback row (touching, deepest penetration,
// point (x, y, h), summed world force) at out[k * S], k = 8 i .. 8 i + 7.
template <class M, class T, int i>
__device__ __forceinline__ SV<T> contact_body(const R3<T>& Rw, V3<T> pw, const SV<T>& vel, const WS<M, T>& ws,
                                              const Terrain<T>& tr, T* out, int S, bool write) {
  constexpr int gt = M::gtype[i];
  constexpr int npts = gt == G_BOX ? 8 : 1;
  constexpr double sc = gt == G_BOX ? 0.25 : 1.0;
  const double dtc = M::dt > 1e-9 ? M::dt : 1e-9;
  V3<T> zb = v3(Rw.m[6], Rw.m[7], Rw.m[8]);  // world +Z in the body frame
  SV<T> ext = {v3(T(0), T(0), T(0)), v3(T(0), T(0), T(0))};
  V3<T> ftot = v3(T(0), T(0), T(0));
  T deepest = T(0);
  T dx = T(0), dy = T(0), dz = T(0);
  bool any = false;
#pragma unroll
  for (int cp = 0; cp < npts; cp++) {
    V3<T> sup;
    if constexpr (pen64<M, T>()) sup = contact_point<M, T, i, double>(cp, zb, ws.zb64[i]);
    else sup = contact_point<M, T, i>(cp, zb);
    V3<T> supw = pw + mul(Rw, sup);
    T pen, th;
    V3<T> nw;
    contact_depth<M, T, i>(ws, tr, cp, supw, pen, th, nw);
    const V3<T> nb = M::HAS_HF ? tmul(Rw, nw) : zb;
    const bool in = pen > T(0);
    V3<T> vpt = vel.l + cross(vel.a, sup);
    T vn = dot(vpt, nb);
    T mn = eff_mass<M, T, i, true>(sup, nb);
    T kb = dmin(T(sc * M::gk[i]), T(4.0 / (dtc * dtc)) * mn);
    T db = dmin(T(sc * M::gd[i]), T(1.0 / dtc) * mn);
    T fn = dmax(kb * pen - db * vn, T(0));
    V3<T> vt3 = vpt - nb * vn;
    T vt = fsqrt(dot(vt3, vt3));
    const bool slip = vt > T(1e-6);
    T ivt = slip ? frcp(dmax(vt, T(5e-7))) : T(0);
    V3<T> td = vt3 * ivt;
    T coul = T(M::mu) * fn * dmin(T(1), vt * T(1e3));
    T ft = dmin(coul, T(1.0 / dtc) * eff_mass<M, T, i, true>(sup, td) * vt);
    ft = slip ? ft : T(0);
    V3<T> fb = nb * fn - td * ft;
    fb = in ? fb : v3(T(0), T(0), T(0));
    ext.a = ext.a + cross(sup, fb);
    ext.l = ext.l + fb;
    if (write) {
      ftot = ftot + mul(Rw, fb);
      const bool deeper = in && pen > deepest;
      deepest = deeper ? pen : deepest;
      dx = deeper ? supw.x : dx;
      dy = deeper ? supw.y : dy;
      dz = deeper ? th : dz;
      any = any || in;
    }
  }
  if (write) {
    T* o = out + 8 * i * S;
    o[0] = any ? T(1) : T(0);
    o[S] = any ? deepest : T(0);
    o[2 * S] = any ? dx : T(0);
    o[3 * S] = any ? dy : T(0);
    o[4 * S] = any ? dz : T(0);
    o[5 * S] = any ? ftot.x : T(0);
    o[6 * S] = any ? ftot.y : T(0);
    o[7 * S] = any ? ftot.z : T(0);
  }
  return ext;
}

// Impulse-mode ground/terrain contact (phyz_kernels.cu:845-937), split in two.
// Within a step q is fixed, so a contact point's support point, terrain height
// and normal, penetration, tangent frame, effective masses and SolImp bias are
// the same in every sweep: ground_prepare computes them once per step and
// ground_sweep makes the velocity-dependent warm-started update per sweep.
// With m' = max(m_n / n_active, 1e-9) and c_t = max(m_t, 1e-9) / n_active the
// reference's update (bias - r_n) / a_nn and -(b_t - a_tt s_t) / a_tt reads
//   f_n = max((bias - v_n (1 + e)) m' + s_n, 0),  f_t = s_t - b_t c_t.
template <class M, class T> struct GroundPrep {
  static constexpr int N = ground_off<M>(M::NB) > 0 ? ground_off<M>(M::NB) : 1;
  V3<T> sup[N], nb[N], tu[N];  // body frame; the second tangent is nb x tu (tangent_frame)
  T mn[N], cu[N], cw[N], bias[N];
  bool in[N];
  bool any[M::NB];
};

// Body i's contact geometry; writes the position part of its readback row
// (touching, deepest penetration, deepest point) when `write`.
template <class M, class T, int i>
__device__ __forceinline__ void ground_prepare(const R3<T>& Rw, V3<T> pw, const WS<M, T>& ws, const Terrain<T>& tr,
                                               GroundPrep<M, T>& gp, T* out, int S, bool write) {
  const V3<double>& zb64 = ws.zb64[i];
  constexpr int n = ground_pts<M>(i), o = ground_off<M>(i);
  const double dtc = M::dt > 1e-9 ? M::dt : 1e-9;
  const V3<T> zb = v3(Rw.m[6], Rw.m[7], Rw.m[8]);  // world +Z in the body frame
  V3<T> supw[n];
  T pen[n];
  int nact = 0;
#pragma unroll
  for (int cp = 0; cp < n; cp++) {
    if constexpr (pen64<M, T>()) gp.sup[o + cp] = contact_point<M, T, i, double>(cp, zb, zb64);
    else gp.sup[o + cp] = contact_point<M, T, i>(cp, zb);
    supw[cp] = pw + mul(Rw, gp.sup[o + cp]);
    T th;
    V3<T> nw;
    contact_depth<M, T, i>(ws, tr, cp, supw[cp], pen[cp], th, nw);
    gp.in[o + cp] = pen[cp] > T(-M::c_margin);
    gp.nb[o + cp] = M::HAS_HF ? tmul(Rw, nw) : zb;
    nact += gp.in[o + cp] ? 1 : 0;
  }
  const T na = n == 1 ? T(1) : T(nact < 1 ? 1 : nact);
  T deepest = T(0);
  V3<T> dw = v3(T(0), T(0), T(0));
  bool any = false;
#pragma unroll
  for (int cp = 0; cp < n; cp++) {
    const int k = o + cp;
    V3<T> tw;
    tangent_frame(gp.nb[k], gp.tu[k], tw);
    gp.mn[k] = dmax(eff_mass<M, T, i>(gp.sup[k], gp.nb[k]) / na, T(1e-9));
    gp.cu[k] = dmax(eff_mass<M, T, i>(gp.sup[k], gp.tu[k]), T(1e-9)) / na;
    gp.cw[k] = dmax(eff_mass<M, T, i>(gp.sup[k], tw), T(1e-9)) / na;
    gp.bias[k] = impedance_at<M, T>(pen[cp]) * T(M::c_erp) * dmax(pen[cp], T(0)) / T(dtc);
    const bool in = gp.in[k];
    any = any || in;
    const bool deeper = in && pen[cp] > deepest;
    deepest = deeper ? pen[cp] : deepest;
    dw = sel(deeper, supw[cp], dw);
  }
  gp.any[i] = any;
  if (write) {
    T* r = out + 8 * i * S;
    r[0] = any ? T(1) : T(0);
    r[S] = any ? deepest : T(0);
    r[2 * S] = any ? dw.x : T(0);
    r[3 * S] = any ? dw.y : T(0);
    r[4 * S] = any ? dw.z : T(0);
  }
}

// One sweep of body i's prepared ground contacts at body-frame velocity vel;
// slot holds its ground impulses (3 per point). Returns the body-frame force.
template <class M, class T, int i>
__device__ __forceinline__ SV<T> ground_sweep(const GroundPrep<M, T>& gp, const SV<T>& vel, T* slot) {
  constexpr int n = ground_pts<M>(i), o = ground_off<M>(i);
  const double dtc = M::dt > 1e-9 ? M::dt : 1e-9;
  SV<T> ext = {v3(T(0), T(0), T(0)), v3(T(0), T(0), T(0))};
#pragma unroll
  for (int cp = 0; cp < n; cp++) {
    const int k = o + cp;
    const V3<T> vpt = vel.l + cross(vel.a, gp.sup[k]);
    const V3<T> gtw = cross(gp.nb[k], gp.tu[k]);  // as tangent_frame forms it
    const T b_n = dot(vpt, gp.nb[k]);
    const T e = restitution_at<M, T>(dmin(b_n, T(0)));
    const T fn = dmax((gp.bias[k] - b_n * (T(1) + e)) * gp.mn[k] + slot[3 * cp], T(0));
    const T tu = slot[3 * cp + 1] - dot(vpt, gp.tu[k]) * gp.cu[k];
    const T tw = slot[3 * cp + 2] - dot(vpt, gtw) * gp.cw[k];
    const T limit = T(M::mu) * fn;
    T sc;
    if constexpr (sizeof(T) == 4) {
      // Slip when |t| > limit, compared as squares; the scale limit / |t|
      // from the hardware reciprocal square root (about 1 ulp): no rooted
      // or divided expansion in the sweep loop, which runs for every contact
      // point SWEEPS times a step. limit >= 0, so slipping implies |t| > 0.
      const T t2 = tu * tu + tw * tw;
      sc = t2 > limit * limit ? limit * __builtin_amdgcn_rsqf(dmax(t2, T(1e-36))) : T(1);
    } else {
      const T tn = dsqrt(tu * tu + tw * tw);
      sc = tn > limit ? (tn > T(0) ? limit / dmax(tn, T(1e-30)) : T(0)) : T(1);
    }
    const bool in = gp.in[k];
    slot[3 * cp] = in ? fn : T(0);
    slot[3 * cp + 1] = in ? tu * sc : T(0);
    slot[3 * cp + 2] = in ? tw * sc : T(0);
    const V3<T> fb = (gp.nb[k] * slot[3 * cp] + gp.tu[k] * slot[3 * cp + 1] + gtw * slot[3 * cp + 2]) * T(1.0 / dtc);
    ext.a = ext.a + cross(gp.sup[k], fb);
    ext.l = ext.l + fb;
  }
  return ext;
}

// Contacts on the body-attached plane (phyz_kernels.cu:982-1132): the plane
// body's local +Z face at plane_offset, finite in x and y, against every other
// collidable body not excluded. Forces land on both bodies (added to f). In
// impulse mode pslot[i] holds body i's plane impulses.
// The plane contacts' decisions, made once per step after pass 1 from the
// f64 chain (f32 kernels; full64): for each body, bits 0-7 say which of its
// contact points lie within the plane's depth range, bit 8 whether its
// footprint overlaps the plane's face. The f32 contact law below then
// switches each contact on and off where the f64 oracle does; the depths and
// points it applies stay f32 (the law is continuous in them otherwise).
template <class M, class T>
__device__ __forceinline__ void plane_decide(const WS<M, T>& ws, int (&mask)[M::NB]) {
  constexpr int pb = M::PLANE;
  const V3<double> nw = v3(ws.xb64[pb].z, ws.yb64[pb].z, ws.zb64[pb].z);
  const V3<double> ppb = v3(ws.px64[pb], ws.py64[pb], ws.pz64[pb]);
  const V3<double> p0 = ppb + nw * M::plane_offset;
  const V3<double> c0 = v3(ws.xb64[pb].x, ws.yb64[pb].x, ws.zb64[pb].x);  // the plane body's x and y axes, world
  const V3<double> c1 = v3(ws.xb64[pb].y, ws.yb64[pb].y, ws.zb64[pb].y);
  sfor<0, M::NB>([&](auto I) {
    constexpr int i = decltype(I)::value;
    mask[i] = 0;
    if constexpr (i != pb && M::gtype[i] != G_NONE && !M::gskip[i]) {
      constexpr int npts = M::gtype[i] == G_BOX ? 8 : 1;
      const V3<double> nbi = ws.xb64[i] * nw.x + ws.yb64[i] * nw.y + ws.zb64[i] * nw.z;
      double lox = 1e30, loy = 1e30, hix = -1e30, hiy = -1e30;
      int m = 0;
#pragma unroll
      for (int cp = 0; cp < npts; cp++) {
        const V3<double> sp = contact_point<M, double, i>(cp, nbi);
        const V3<double> spw = v3(ws.px64[i] + dot(ws.xb64[i], sp), ws.py64[i] + dot(ws.yb64[i], sp),
                                  ws.pz64[i] + dot(ws.zb64[i], sp));
        const V3<double> d = spw - ppb;
        const double rx = dot(c0, d), ry = dot(c1, d);
        lox = dmin(lox, rx); loy = dmin(loy, ry);
        hix = dmax(hix, rx); hiy = dmax(hiy, ry);
        const double pen = -dot(spw - p0, nw);
        m |= (pen > 0.0 && pen <= M::plane_depth) ? 1 << cp : 0;
      }
      const bool over = !(dmax(lox, -M::plane_hx) > dmin(hix, M::plane_hx) || dmax(loy, -M::plane_hy) > dmin(hiy, M::plane_hy));
      mask[i] = m | (over ? 1 << 8 : 0);
    }
  });
}

template <class M, class T, bool IMP>
__device__ __forceinline__ void plane_contacts(const R3<T>* Rw, const V3<T>* Pw, const SV<T>* vel, T (*pslot)[24],
                                               SV<T>* f, const int* mask64) {
  constexpr int pb = M::PLANE;
  const double dtc = M::dt > 1e-9 ? M::dt : 1e-9;
  const V3<T> nw = v3(Rw[pb].m[2], Rw[pb].m[5], Rw[pb].m[8]);  // the face normal, world
  const V3<T> p0 = Pw[pb] + nw * T(M::plane_offset);
  sfor<0, M::NB>([&](auto I) {
    constexpr int i = decltype(I)::value;
    if constexpr (i != pb && M::gtype[i] != G_NONE && !M::gskip[i]) {
      constexpr int gt = M::gtype[i];
      constexpr int npts = gt == G_BOX ? 8 : 1;
      constexpr double sc = gt == G_BOX ? 0.25 : 1.0;
      const V3<T> nbi = tmul(Rw[i], nw);
      V3<T> spw[npts];
      T lox = T(1e30), loy = T(1e30), hix = T(-1e30), hiy = T(-1e30);
      int cnt = 0;
#pragma unroll
      for (int cp = 0; cp < npts; cp++) {
        spw[cp] = Pw[i] + mul(Rw[i], contact_point<M, T, i>(cp, nbi));
        const V3<T> rp = tmul(Rw[pb], spw[cp] - Pw[pb]);
        lox = dmin(lox, rp.x); loy = dmin(loy, rp.y);
        hix = dmax(hix, rp.x); hiy = dmax(hiy, rp.y);
        const T d = -dot(spw[cp] - p0, nw);
        if constexpr (pen64<M, T>()) cnt += (mask64[i] >> cp) & 1;
        else cnt += (d > T(0) && d <= T(M::plane_depth)) ? 1 : 0;
      }
      const T olx = dmax(lox, T(-M::plane_hx)), oly = dmax(loy, T(-M::plane_hy));
      const T ohx = dmin(hix, T(M::plane_hx)), ohy = dmin(hiy, T(M::plane_hy));
      bool over;
      if constexpr (pen64<M, T>()) over = ((mask64[i] >> 8) & 1) != 0;
      else over = !(olx > ohx || oly > ohy);
      if (over) {
        const T na = T(cnt > 1 ? cnt : 1);
#pragma unroll
        for (int cp = 0; cp < npts; cp++) {
          const T pen = -dot(spw[cp] - p0, nw);
          bool in;
          if constexpr (pen64<M, T>()) in = ((mask64[i] >> cp) & 1) != 0;
          else in = pen > T(0) && pen <= T(M::plane_depth);
          V3<T> rpp = tmul(Rw[pb], spw[cp] - Pw[pb]);
          rpp.x = dmin(dmax(rpp.x, olx), ohx);
          rpp.y = dmin(dmax(rpp.y, oly), ohy);
          const V3<T> sw = Pw[pb] + mul(Rw[pb], rpp);
          const V3<T> sc_i = tmul(Rw[i], sw - Pw[i]);
          const V3<T> vrel = mul(Rw[i], vel[i].l + cross(vel[i].a, sc_i)) - mul(Rw[pb], vel[pb].l + cross(vel[pb].a, rpp));
          const T vn = dot(vrel, nw);
          auto series = [&](V3<T> d) {
            return T(1) / (T(1) / eff_mass<M, T, i>(sc_i, tmul(Rw[i], d)) + T(1) / eff_mass<M, T, pb>(rpp, tmul(Rw[pb], d)));
          };
          V3<T> fw;
          if constexpr (IMP) {
            V3<T> pu, pwv;
            tangent_frame(nw, pu, pwv);
            T* sl = pslot[i] + 3 * cp;
            T upd[3] = {sl[0], sl[1], sl[2]};
            impulse_update<M, T>(pen, vn, dot(vrel, pu), dot(vrel, pwv), na / dmax(series(nw), T(1e-9)),
                                 na / dmax(series(pu), T(1e-9)), na / dmax(series(pwv), T(1e-9)), upd);
#pragma unroll
            for (int k = 0; k < 3; k++) sl[k] = in ? upd[k] : T(0);
            fw = (nw * sl[0] + pu * sl[1] + pwv * sl[2]) * T(1.0 / dtc);
          } else {
            const T mn = series(nw);
            const T kb = dmin(T(sc * M::gk[i]), T(4.0 / (dtc * dtc)) * mn);
            const T db = dmin(T(sc * M::gd[i]), T(1.0 / dtc) * mn);
            const T fn = dmax(kb * pen - db * vn, T(0));
            const V3<T> vt3 = vrel - nw * vn;
            const T vt = dsqrt(dot(vt3, vt3));
            const bool slip = vt > T(1e-6);
            const V3<T> td = vt3 * (slip ? T(1) / dmax(vt, T(5e-7)) : T(0));
            T ft = dmin(T(M::mu) * fn * dmin(T(1), vt * T(1e3)), T(1.0 / dtc) * series(td) * vt);
            ft = slip ? ft : T(0);
            fw = nw * fn - td * ft;
            fw = sel(in, fw, v3(T(0), T(0), T(0)));
          }
          const V3<T> fi = tmul(Rw[i], fw);
          f[i].a = f[i].a + cross(sc_i, fi);
          f[i].l = f[i].l + fi;
          const V3<T> fp = tmul(Rw[pb], v3(T(0), T(0), T(0)) - fw);
          f[pb].a = f[pb].a + cross(rpp, fp);
          f[pb].l = f[pb].l + fp;
        }
      }
    }
  });
}

// ── per-world step, organised by body groups ────────────────────────────────
// The host partitions the tree (Model::PMODE):
//   0  one group owns every body: one lane per world, no exchange.
//   1  fixed trunk: the trunk is the chain of fixed joints from the world; its
//      transforms, velocities and accelerations are constants, so every group
//      recomputes them (they fold away) and the subtrees below it are
//      independent. One wave per subtree group, no exchange.
//   2  floating trunk: group 0 owns the trunk (the bodies above the branch
//      points); the other groups own subtrees. Every group recomputes the
//      trunk's pass 1 from its own copy of the trunk state; subtree groups hand
//      their articulated inertia and bias force contributions to group 0
//      through LDS, group 0 finishes the trunk and hands back the branch-point
//      accelerations and the new trunk state. Two workgroup barriers per step.
// A workgroup is NG waves over the same 64 worlds; wave g runs group g's code.
// f32 kernels with the f64 height chain compute a ball or free joint's
// quaternion in f64 in pass 1; the integration takes its rounding instead of
// a second, f32 exponential of the same rotation vector.
template <class M, class T, int i> constexpr bool quat_from_pass1() {
  return pen64<M, T>() && M::need_world[i] && (M::jtype[i] == J_BALL || M::jtype[i] == J_FREE);
}
template <class M, class T> struct WS {
  Xf<T> X[M::NB];
  SV<T> vel[M::NB], cb[M::NB], pA[M::NB], acc[M::NB];
  R3<T> Rw[M::NB];
  V3<T> Pw[M::NB];
  Sym<T> IA[M::NB];
  T U[M::NB][M::MAXD][6];
  T Lm[M::NB][M::MAXD][M::MAXD];
  T Dinv[M::NB][M::MAXD];
  T uu[M::NB][M::MAXD];
  bool ok[M::NB];
  V3<double> zb64[M::NB];  // f64 penetration chain (f32 kernels with contact)
  double pz64[M::NB];
  double cz64[ground_off<M>(M::NB) > 0 ? ground_off<M>(M::NB) : 1];  // contact points' world heights
  // The chain's other two rows and origins (heightfield or body-attached plane):
  // contact points' world x, y, and the plane's frame, in f64.
  V3<double> xb64[M::NB], yb64[M::NB];
  double px64[M::NB], py64[M::NB];
  // Over a heightfield, each contact point's depth (pen_decided) and terrain
  // cell (pack_cell), both decided in pass 1 in f64.
  T hf_pen[ground_off<M>(M::NB) > 0 ? ground_off<M>(M::NB) : 1];
  int hf_cellw[ground_off<M>(M::NB) > 0 ? ground_off<M>(M::NB) : 1];
  T ts[M::NB], tc[M::NB];  // revolute joints' sin and cos of -q (split-lane kernels)
  Sym<T> cI[M::NB];        // a group's summed subtree contributions to trunk body p (groups other than 0)
  SV<T> cP[M::NB];
  Q<T> qj[M::NB];          // a ball or free joint's quaternion from pass 1's f64 transform (quat_from_pass1)
};

// Column k, entry r of U = I_A S of body i. A free joint's S is the identity,
// so its U is I_A itself, read from the symmetric storage (21 values live
// through the impulse sweeps instead of 36).
template <class M, class T, int i> __device__ __forceinline__ T Uv(const WS<M, T>& ws, int k, int r) {
  if constexpr (M::jtype[i] == J_FREE) return sym_get(ws.IA[i], r, k);
  else return ws.U[i][k][r];
}

// A revolute joint's transform from s, c = sin, cos of -q (Rodrigues' form
// with the axis terms precomputed on the host) and its joint velocity.
template <class M, class T, int i>
__device__ __forceinline__ void rev_xf(T s, T c, const T* v, Xf<T>& X, SV<T>& vj) {
  const R3<T> Rp = R3<T>{{T(M::ptj_rot[i][0]), T(M::ptj_rot[i][1]), T(M::ptj_rot[i][2]), T(M::ptj_rot[i][3]),
                          T(M::ptj_rot[i][4]), T(M::ptj_rot[i][5]), T(M::ptj_rot[i][6]), T(M::ptj_rot[i][7]),
                          T(M::ptj_rot[i][8])}};
  const T omc = T(1) - c;
  R3<T> EJ;
#pragma unroll
  for (int k = 0; k < 9; k++) EJ.m[k] = T(k % 4 == 0 ? 1.0 : 0.0) + T(M::rev_k[i][k]) * s + T(M::rev_k2[i][k]) * omc;
  X.E = M::ptj_identity[i] ? EJ : mul(EJ, Rp);
  X.r = v3(T(M::ptj_pos[i][0]), T(M::ptj_pos[i][1]), T(M::ptj_pos[i][2]));
  vj = SV<T>{v3(T(M::axis[i][0]), T(M::axis[i][1]), T(M::axis[i][2])) * v[M::voff[i]], v3(T(0), T(0), T(0))};
}

// Joint transform X = X_J(q) X_ptj of body i and its joint velocity S qd
// (crates/phyz-model/src/joint.rs:253-360 maps; the same for FK and ABA).
template <class M, class T, int i>
__device__ __forceinline__ void joint_xf(const T* q, const T* v, Xf<T>& X, SV<T>& vj) {
  constexpr int jt = M::jtype[i];
  constexpr int qo = M::qoff[i], vo = M::voff[i];
  const R3<T> Rp = R3<T>{{T(M::ptj_rot[i][0]), T(M::ptj_rot[i][1]), T(M::ptj_rot[i][2]), T(M::ptj_rot[i][3]),
                          T(M::ptj_rot[i][4]), T(M::ptj_rot[i][5]), T(M::ptj_rot[i][6]), T(M::ptj_rot[i][7]),
                          T(M::ptj_rot[i][8])}};
  const V3<T> pp = v3(T(M::ptj_pos[i][0]), T(M::ptj_pos[i][1]), T(M::ptj_pos[i][2]));
  vj = SV<T>{v3(T(0), T(0), T(0)), v3(T(0), T(0), T(0))};
  if constexpr (jt == J_REV) {
    T s, c;
    rev_sincos(-q[qo], &s, &c);
    rev_xf<M, T, i>(s, c, v, X, vj);
  } else if constexpr (jt == J_PRIS) {
    X.E = Rp;
    X.r = pp + tmul(Rp, v3(T(M::axis[i][0]), T(M::axis[i][1]), T(M::axis[i][2])) * q[qo]);
    vj.l = v3(T(M::axis[i][0]), T(M::axis[i][1]), T(M::axis[i][2])) * v[vo];
  } else if constexpr (jt == J_BALL || jt == J_FREE) {
    R3<T> EJ = transpose(quat_mat(quat_exp(v3(q[qo], q[qo + 1], q[qo + 2]))));
    X.E = M::ptj_identity[i] ? EJ : mul(EJ, Rp);
    if constexpr (jt == J_FREE) {
      X.r = pp + tmul(Rp, v3(q[qo + 3], q[qo + 4], q[qo + 5]));
      vj.l = v3(v[vo + 3], v[vo + 4], v[vo + 5]);
    } else {
      X.r = pp;
    }
    vj.a = v3(v[vo], v[vo + 1], v[vo + 2]);
  } else {
    X.E = Rp;
    X.r = pp;
  }
}


template <class T> __device__ __forceinline__ Q<double> quat_exp64(V3<T> wf) {
  const V3<double> w = v3(double(wf.x), double(wf.y), double(wf.z));
  const double ang = sqrt(dot(w, w));
  double s, c;
  joint_sincos64(0.5 * ang, &s, &c);
  const bool small = ang < Eps<double>::v;
  const double f = small ? 0.5 : s / dmax(ang, 0.5 * Eps<double>::v);
  return {small ? 1.0 : c, w.x * f, w.y * f, w.z * f};
}

// Body i's joint rotation and offset (joint_xf's X.E and X.r) in f64.
template <class M, class T, int i>
__device__ __forceinline__ void joint_xf64(const T* q, R3<double>& E, V3<double>& r, Q<double>* qj = nullptr) {
  constexpr int jt = M::jtype[i];
  constexpr int qo = M::qoff[i];
  const R3<double> Rp = R3<double>{{M::ptj_rot[i][0], M::ptj_rot[i][1], M::ptj_rot[i][2], M::ptj_rot[i][3],
                                    M::ptj_rot[i][4], M::ptj_rot[i][5], M::ptj_rot[i][6], M::ptj_rot[i][7],
                                    M::ptj_rot[i][8]}};
  const V3<double> pp = v3(M::ptj_pos[i][0], M::ptj_pos[i][1], M::ptj_pos[i][2]);
  if constexpr (jt == J_REV) {
    double s, c;
    joint_sincos64(-double(q[qo]), &s, &c);
    const double omc = 1.0 - c;
    R3<double> EJ;
#pragma unroll
    for (int k = 0; k < 9; k++) EJ.m[k] = (k % 4 == 0 ? 1.0 : 0.0) + M::rev_k[i][k] * s + M::rev_k2[i][k] * omc;
    E = M::ptj_identity[i] ? EJ : mul(EJ, Rp);
    r = pp;
  } else if constexpr (jt == J_PRIS) {
    E = Rp;
    r = pp + tmul(Rp, v3(M::axis[i][0], M::axis[i][1], M::axis[i][2]) * double(q[qo]));
  } else if constexpr (jt == J_BALL || jt == J_FREE) {
    const Q<double> qq = quat_exp64(v3(q[qo], q[qo + 1], q[qo + 2]));
    if (qj) *qj = qq;
    R3<double> EJ = transpose(quat_mat(qq));
    E = M::ptj_identity[i] ? EJ : mul(EJ, Rp);
    if constexpr (jt == J_FREE) r = pp + tmul(Rp, v3(double(q[qo + 3]), double(q[qo + 4]), double(q[qo + 5])));
    else r = pp;
  } else {
    E = Rp;
    r = pp;
  }
}

// Body i's joint velocity S qd (joint_xf's vj).
template <class M, class T, int i> __device__ __forceinline__ SV<T> joint_vel(const T* v) {
  constexpr int jt = M::jtype[i];
  constexpr int vo = M::voff[i];
  SV<T> vj = {v3(T(0), T(0), T(0)), v3(T(0), T(0), T(0))};
  if constexpr (jt == J_REV) vj.a = v3(T(M::axis[i][0]), T(M::axis[i][1]), T(M::axis[i][2])) * v[vo];
  else if constexpr (jt == J_PRIS) vj.l = v3(T(M::axis[i][0]), T(M::axis[i][1]), T(M::axis[i][2])) * v[vo];
  else if constexpr (jt == J_BALL || jt == J_FREE) {
    vj.a = v3(v[vo], v[vo + 1], v[vo + 2]);
    if constexpr (jt == J_FREE) vj.l = v3(v[vo + 3], v[vo + 4], v[vo + 5]);
  }
  return vj;
}

template <class M, class T, int i>
__device__ __forceinline__ void body_pass1(WS<M, T>& ws, const T* q, const T* v, T* rows, int S, bool write_rows,
                                           bool do_contact, const Terrain<T>& tr) {
  constexpr int p = M::parent[i];
  Xf<T>& X = ws.X[i];
  SV<T> vj;
  if constexpr (pen64<M, T>() && M::need_world[i]) {
    // The joint transform once, in f64: the height chain uses it as it is and
    // the f32 dynamics its rounding (so no f32 sincos of this joint).
    // Rw_i = Rw_p X.E^T: third row zb_i = X.E zb_p; Pw_i = Pw_p + Rw_p X.r.
    R3<double> E64;
    V3<double> r64;
    Q<double> q64;
    joint_xf64<M, T, i>(q, E64, r64, &q64);
    if constexpr (quat_from_pass1<M, T, i>()) ws.qj[i] = Q<T>{T(q64.w), T(q64.x), T(q64.y), T(q64.z)};
#pragma unroll
    for (int k = 0; k < 9; k++) X.E.m[k] = T(E64.m[k]);
    X.r = v3(T(r64.x), T(r64.y), T(r64.z));
    vj = joint_vel<M, T, i>(v);
    if constexpr (p < 0) {
      ws.zb64[i] = v3(E64.m[2], E64.m[5], E64.m[8]);
      ws.pz64[i] = r64.z;
      if constexpr (full64<M, T>()) {
        ws.xb64[i] = v3(E64.m[0], E64.m[3], E64.m[6]);
        ws.yb64[i] = v3(E64.m[1], E64.m[4], E64.m[7]);
        ws.px64[i] = r64.x;
        ws.py64[i] = r64.y;
      }
    } else {
      ws.zb64[i] = mul(E64, ws.zb64[p]);
      ws.pz64[i] = ws.pz64[p] + dot(ws.zb64[p], r64);
      if constexpr (full64<M, T>()) {
        ws.xb64[i] = mul(E64, ws.xb64[p]);
        ws.yb64[i] = mul(E64, ws.yb64[p]);
        ws.px64[i] = ws.px64[p] + dot(ws.xb64[p], r64);
        ws.py64[i] = ws.py64[p] + dot(ws.yb64[p], r64);
      }
    }
    // Only the contact points' world heights (and over a heightfield their
    // x, y) outlive the body's children.
#pragma unroll
    for (int cp = 0; cp < ground_pts<M>(i); cp++) {
      const int k = ground_off<M>(i) + cp;
      const V3<double> sp = contact_point<M, double, i>(cp, ws.zb64[i]);
      const double cz = ws.pz64[i] + dot(ws.zb64[i], sp);
      if constexpr (M::HAS_HF) {
        V3<double> n64;
        HfCell c;
        const double th =
            terrain_at<M, T>(tr, ws.px64[i] + dot(ws.xb64[i], sp), ws.py64[i] + dot(ws.yb64[i], sp), n64, &c);
        ws.hf_pen[k] = pen_decided<M, T>(n64.z * (th - cz));
        ws.hf_cellw[k] = pack_cell(c);
      } else {
        ws.cz64[k] = cz;
      }
    }
  } else if constexpr (M::LANES > 1 && M::jtype[i] == J_REV) {
    rev_xf<M, T, i>(ws.ts[i], ws.tc[i], v, X, vj);
  } else {
    joint_xf<M, T, i>(q, v, X, vj);
  }
  if constexpr (p < 0) {
    ws.vel[i] = vj;
    ws.cb[i] = SV<T>{v3(T(0), T(0), T(0)), v3(T(0), T(0), T(0))};
  } else {
    ws.vel[i] = apply_motion(X, ws.vel[p]) + vj;
    ws.cb[i] = cross_motion(ws.vel[i], vj);
  }
  ws.pA[i] = cross_force(ws.vel[i], sym_mul(rigid_inertia<M, T, i>(), ws.vel[i]));
  if constexpr (M::need_world[i]) {
    if constexpr (p < 0) {
      ws.Rw[i] = transpose(X.E);
      ws.Pw[i] = X.r;
    } else {
      ws.Rw[i] = mul_bt(ws.Rw[p], X.E);
      ws.Pw[i] = ws.Pw[p] + mul(ws.Rw[p], X.r);
    }
  }
  if constexpr (M::gtype[i] != G_NONE) {
    if (do_contact) {
      SV<T> f = contact_body<M, T, i>(ws.Rw[i], ws.Pw[i], ws.vel[i], ws, tr, rows, S, write_rows);
      ws.pA[i] = ws.pA[i] - f;
    }
  }
}

// Generalized force on DOF k of body i's joint: the actuators driving it (or
// the DOF's own ctrl entry when the model has none, model.rs:175-231), then the
// passive terms (actuation.rs:18-39, joint.rs:196-247): damping, and on a
// one-DOF joint the spring, the soft position limit and dry friction.
template <class M, class T, int a> __device__ __forceinline__ T actuator_force(T c, T qj, T vj) {
  if constexpr (M::act_cr[a]) c = dmin(dmax(c, T(M::act_clo[a])), T(M::act_chi[a]));
  T f = T(M::act_gear[a]) * (T(M::act_gain[a]) * c + T(M::act_bq[a]) * qj + T(M::act_bv[a]) * vj);
  if constexpr (M::act_fr[a]) f = dmin(dmax(f, T(M::act_flo[a])), T(M::act_fhi[a]));
  return f;
}
template <class M, class T, int i, int k>
__device__ __forceinline__ T dof_force(const T* q, const T* v, const T* ctrl) {
  constexpr int nd = ndof_of(M::jtype[i]);
  constexpr int vo = M::voff[i], qo = M::qoff[i];
  T tau;
  if constexpr (M::NU == 0) {
    tau = ctrl[vo + k];
  } else {
    tau = T(0);
    sfor<0, M::NU>([&](auto A) {
      constexpr int a = decltype(A)::value;
      if constexpr (M::act_v[a] == vo + k) tau = tau + actuator_force<M, T, a>(ctrl[a], q[M::act_q[a]], v[vo + k]);
    });
  }
  T f = -(T(M::damping[i]) * v[vo + k]);
  if constexpr (nd == 1) {
    f = f - T(M::stiffness[i]) * (q[qo] - T(M::spring_ref[i]));
    if constexpr (M::lim_on[i]) {
      const T x = q[qo], xd = v[vo];
      const bool below = x < T(M::lim_lo[i]), above = x > T(M::lim_hi[i]);
      const T depth = below ? T(M::lim_lo[i]) - x : x - T(M::lim_hi[i]);
      const T sign = below ? T(1) : T(-1);
      const T lf = sign * (T(M::lim_k[i]) * depth + T(M::lim_d[i]) * dmax(-(sign * xd), T(0)));
      f = f + ((below || above) ? lf : T(0));
    }
    if constexpr (M::floss[i] > 0.0) f = f - T(M::floss[i]) * dtanh(per_milli(v[vo]));
  }
  return tau + f;
}

// Joint solve of body i (U, D = LDL^T, u) and its articulated inertia / bias
// force as seen by the parent (I_a, p_a), from I_A and p_A. Returns false for
// a body without DOFs (then Ia, pa are I_A, p_A unchanged).
template <class M, class T, int i>
__device__ __forceinline__ void body_solve(WS<M, T>& ws, const T* q, const T* v, const T* ctrl, Sym<T>& Ia,
                                           SV<T>& pa) {
  constexpr int nd = ndof_of(M::jtype[i]);
  constexpr int p = M::parent[i];
  constexpr int vo = M::voff[i], qo = M::qoff[i];
  constexpr int MAXD = M::MAXD;
  ws.ok[i] = true;
  Ia = ws.IA[i];
  pa = ws.pA[i];
  if constexpr (nd > 0) {
    sfor<0, nd>([&](auto K) {
      constexpr int k = decltype(K)::value;
      if constexpr (M::jtype[i] != J_FREE) {
        SV<T> uk = sym_mul(ws.IA[i], subspace<M, T, i>(k));
        ws.U[i][k][0] = uk.a.x; ws.U[i][k][1] = uk.a.y; ws.U[i][k][2] = uk.a.z;
        ws.U[i][k][3] = uk.l.x; ws.U[i][k][4] = uk.l.y; ws.U[i][k][5] = uk.l.z;
      }
      ws.uu[i][k] = dof_force<M, T, i, k>(q, v, ctrl) - dot(subspace<M, T, i>(k), ws.pA[i]);
    });
    T D[MAXD][MAXD];
#pragma unroll
    for (int r = 0; r < nd; r++)
#pragma unroll
      for (int c = 0; c <= r; c++) {
        SV<T> sr = subspace<M, T, i>(r);
        SV<T> ucol = {v3(Uv<M, T, i>(ws, c, 0), Uv<M, T, i>(ws, c, 1), Uv<M, T, i>(ws, c, 2)), v3(Uv<M, T, i>(ws, c, 3), Uv<M, T, i>(ws, c, 4), Uv<M, T, i>(ws, c, 5))};
        D[r][c] = dot(sr, ucol) + (r == c ? T(M::armature[i] + M::dt * M::damping[i]) : T(0));
      }
    // LDL^T with the pivots stored inverted (same singular test as aba.rs:210).
    T E[MAXD][MAXD];
#pragma unroll
    for (int j = 0; j < nd; j++) {
      T dj = D[j][j];
#pragma unroll
      for (int k = 0; k < j; k++) dj = dj - ws.Lm[i][j][k] * E[j][k];
      // piv_ok: the host has bounded every pivot of this joint away from the
      // test, so ok stays true at compile time and the parent updates guarded
      // by it need no branch.
      if constexpr (!M::piv_ok[i]) ws.ok[i] = ws.ok[i] && !(dabs(dj) < T(1e-20));
      ws.Dinv[i][j] = frcp(!M::piv_ok[i] && dabs(dj) < T(1e-20) ? T(1) : dj);
#pragma unroll
      for (int r = j + 1; r < nd; r++) {
        T e = D[r][j];
#pragma unroll
        for (int k = 0; k < j; k++) e = e - ws.Lm[i][r][k] * E[j][k];
        E[r][j] = e;
        ws.Lm[i][r][j] = e * ws.Dinv[i][j];
      }
    }
    if constexpr (p >= 0) {
      // W = U D^-1, one row of U at a time.
      T W[MAXD][6];
#pragma unroll
      for (int r = 0; r < 6; r++) {
        T y[MAXD];
#pragma unroll
        for (int k = 0; k < nd; k++) {
          y[k] = Uv<M, T, i>(ws, k, r);
#pragma unroll
          for (int t = 0; t < k; t++) y[k] = y[k] - ws.Lm[i][k][t] * y[t];
        }
#pragma unroll
        for (int k = 0; k < nd; k++) y[k] = y[k] * ws.Dinv[i][k];
#pragma unroll
        for (int k = nd - 1; k >= 0; k--)
#pragma unroll
          for (int t = k + 1; t < nd; t++) y[k] = y[k] - ws.Lm[i][t][k] * y[t];
#pragma unroll
        for (int k = 0; k < nd; k++) W[k][r] = y[k];
      }
#pragma unroll
      for (int r = 0; r < 3; r++)
#pragma unroll
        for (int c = r; c < 3; c++) {
          T s0 = W[0][r] * Uv<M, T, i>(ws, 0, c), s1 = W[0][3 + r] * Uv<M, T, i>(ws, 0, 3 + c);
#pragma unroll
          for (int k = 1; k < nd; k++) { s0 = s0 + W[k][r] * Uv<M, T, i>(ws, k, c); s1 = s1 + W[k][3 + r] * Uv<M, T, i>(ws, k, 3 + c); }
          Ia.a[sx(r, c)] = Ia.a[sx(r, c)] - s0;
          Ia.c[sx(r, c)] = Ia.c[sx(r, c)] - s1;
        }
#pragma unroll
      for (int r = 0; r < 3; r++)
#pragma unroll
        for (int c = 0; c < 3; c++) {
          T s0 = W[0][r] * Uv<M, T, i>(ws, 0, 3 + c);
#pragma unroll
          for (int k = 1; k < nd; k++) s0 = s0 + W[k][r] * Uv<M, T, i>(ws, k, 3 + c);
          Ia.b[r * 3 + c] = Ia.b[r * 3 + c] - s0;
        }
      if constexpr (M::zero_axis[i] >= 0) {
        // I_a S = U - U D^-1 S^T U = 0 when D = S^T U (no armature or
        // damping): for S a coordinate axis z, row and column z of I_a are
        // zero in exact arithmetic, and set so here (the computed values are
        // rounding residue). The zeros then fold through X^T I_a X and I_a c.
        constexpr int z = M::zero_axis[i];
#pragma unroll
        for (int j = 0; j < 6; j++) {
          if (z < 3 && j < 3) Ia.a[sx(z, j)] = T(0);
          if (z < 3 && j >= 3) Ia.b[z * 3 + (j - 3)] = T(0);
          if (z >= 3 && j >= 3) Ia.c[sx(z - 3, j - 3)] = T(0);
          if (z >= 3 && j < 3) Ia.b[j * 3 + (z - 3)] = T(0);
        }
      }
      SV<T> wu;
#pragma unroll
      for (int r = 0; r < 6; r++) {
        T s0 = W[0][r] * ws.uu[i][0];
#pragma unroll
        for (int k = 1; k < nd; k++) s0 = s0 + W[k][r] * ws.uu[i][k];
        sv_set(wu, r, s0);
      }
      pa = pa + sym_mul(Ia, ws.cb[i]) + wu;
    }
  }
}

template <class M, class T, int i> __device__ __forceinline__ void body_pass3(WS<M, T>& ws, T* qdd) {
  constexpr int nd = ndof_of(M::jtype[i]);
  constexpr int p = M::parent[i];
  constexpr int vo = M::voff[i];
  constexpr int MAXD = M::MAXD;
  SV<T> ap;
  if constexpr (p < 0) {
    SV<T> a0 = {v3(T(0), T(0), T(0)), v3(T(-M::gravity[0]), T(-M::gravity[1]), T(-M::gravity[2]))};
    ap = apply_motion(ws.X[i], a0) + ws.cb[i];
  } else {
    ap = apply_motion(ws.X[i], ws.acc[p]) + ws.cb[i];
  }
  if constexpr (nd > 0) {
    T y[MAXD];
#pragma unroll
    for (int k = 0; k < nd; k++) {
      T uta = Uv<M, T, i>(ws, k, 0) * ap.a.x + Uv<M, T, i>(ws, k, 1) * ap.a.y + Uv<M, T, i>(ws, k, 2) * ap.a.z + Uv<M, T, i>(ws, k, 3) * ap.l.x +
              Uv<M, T, i>(ws, k, 4) * ap.l.y + Uv<M, T, i>(ws, k, 5) * ap.l.z;
      y[k] = ws.uu[i][k] - uta;
#pragma unroll
      for (int t = 0; t < k; t++) y[k] = y[k] - ws.Lm[i][k][t] * y[t];
    }
#pragma unroll
    for (int k = 0; k < nd; k++) y[k] = y[k] * ws.Dinv[i][k];
#pragma unroll
    for (int k = nd - 1; k >= 0; k--)
#pragma unroll
      for (int t = k + 1; t < nd; t++) y[k] = y[k] - ws.Lm[i][t][k] * y[t];
#pragma unroll
    for (int k = 0; k < nd; k++) {
      y[k] = ws.ok[i] ? y[k] : T(0);
      qdd[vo + k] = y[k];
      ap = ap + subspace<M, T, i>(k) * y[k];
    }
  }
  ws.acc[i] = ap;
}

// Semi-implicit Euler for body i's joint (integrate.rs:41-92); v += dt qdd first.
template <class M, class T, int i, bool QJ = false>
__device__ __forceinline__ void body_integrate(T* q, T* v, const T* qdd, const Q<T>& qj = Q<T>{}) {
  constexpr int jt = M::jtype[i];
  constexpr int nd = ndof_of(jt);
  constexpr int qo = M::qoff[i], vo = M::voff[i];
  const T dt = T(M::dt);
#pragma unroll
  for (int k = 0; k < nd; k++) v[vo + k] = v[vo + k] + dt * qdd[vo + k];
  if constexpr (jt == J_REV || jt == J_PRIS) {
    q[qo] = q[qo] + dt * v[vo];
  } else if constexpr (jt == J_BALL || jt == J_FREE) {
    Q<T> cur;
    if constexpr (QJ) cur = qj;
    else cur = quat_exp(v3(q[qo], q[qo + 1], q[qo + 2]));
    if constexpr (jt == J_FREE) {
      V3<T> wl = qrotate(cur, v3(v[vo + 3], v[vo + 4], v[vo + 5]));
      q[qo + 3] = q[qo + 3] + dt * wl.x;
      q[qo + 4] = q[qo + 4] + dt * wl.y;
      q[qo + 5] = q[qo + 5] + dt * wl.z;
    }
    // The product is not normalised: it is unit to rounding, and quat_log is
    // scale-free (atan2(s n, s w) = atan2(n, w), v / |v|), so the reference's
    // normalisation would move the result by rounding only.
    Q<T> nx = qmul(cur, quat_exp(v3(v[vo], v[vo + 1], v[vo + 2]) * dt));
    V3<T> lg = quat_log(nx);
    q[qo] = lg.x;
    q[qo + 1] = lg.y;
    q[qo + 2] = lg.z;
  }
}

// Articulated inertia / bias force of body i propagated to its parent:
// I_A[p] += X^T I_a X, p_A[p] += X^T p_a.
template <class M, class T, int i>
__device__ __forceinline__ void propagate(WS<M, T>& ws, const Sym<T>& Ia, const SV<T>& pa, Sym<T>& dI, SV<T>& dp) {
  dI = sym_xtix<T, M::rot_axis[i]>(Ia, ws.X[i]);
  dp = inv_apply_force(ws.X[i], pa);
}

// LDS exchange slots (floating trunk): slot s holds 64 lanes of T.
template <class T> __device__ __forceinline__ void lds_put(T* lds, int slot, int lane, T x) { lds[slot * 64 + lane] = x; }
template <class T> __device__ __forceinline__ T lds_get(const T* lds, int slot, int lane) { return lds[slot * 64 + lane]; }
template <class T> __device__ __forceinline__ void put_sym(T* lds, int s, int lane, const Sym<T>& I, const SV<T>& p) {
#pragma unroll
  for (int k = 0; k < 6; k++) { lds_put(lds, s + k, lane, I.a[k]); lds_put(lds, s + 6 + k, lane, I.c[k]); }
#pragma unroll
  for (int k = 0; k < 9; k++) lds_put(lds, s + 12 + k, lane, I.b[k]);
  lds_put(lds, s + 21, lane, p.a.x); lds_put(lds, s + 22, lane, p.a.y); lds_put(lds, s + 23, lane, p.a.z);
  lds_put(lds, s + 24, lane, p.l.x); lds_put(lds, s + 25, lane, p.l.y); lds_put(lds, s + 26, lane, p.l.z);
}
template <class T> __device__ __forceinline__ void add_sym(const T* lds, int s, int lane, Sym<T>& I, SV<T>& p) {
#pragma unroll
  for (int k = 0; k < 6; k++) { I.a[k] = I.a[k] + lds_get(lds, s + k, lane); I.c[k] = I.c[k] + lds_get(lds, s + 6 + k, lane); }
#pragma unroll
  for (int k = 0; k < 9; k++) I.b[k] = I.b[k] + lds_get(lds, s + 12 + k, lane);
  p.a = p.a + v3(lds_get(lds, s + 21, lane), lds_get(lds, s + 22, lane), lds_get(lds, s + 23, lane));
  p.l = p.l + v3(lds_get(lds, s + 24, lane), lds_get(lds, s + 25, lane), lds_get(lds, s + 26, lane));
}

// Control noise and PD servos of group G's DOFs, before the dynamics.
template <class M, class T, int G>
__device__ __forceinline__ void apply_controls(const T (&q)[M::NQ], const T (&v)[M::NV], T (&ctrl)[M::NCTRL], const T* tgt,
                                               u64& rng, const T* lds, int lane) {
  // ── control noise: every group advances the whole stream; values only for its DOFs ──
  if constexpr (M::NNOISE > 0 && M::NOISE_G >= 0) {
    // Drawn by wave NOISE_G during the previous step (draw_shared_noise).
    sfor<0, M::NNOISE>([&](auto K) {
      constexpr int k = decltype(K)::value;
      if constexpr (M::ctrl_owner[M::noise_dof[k]] == G) ctrl[M::noise_dof[k]] = lds_get(lds, M::slot_noise + k, lane);
    });
  } else if constexpr (M::NNOISE > 0) {
    if constexpr (M::noise_dist == 1) {
      sfor<0, M::NNOISE>([&](auto K) {
        constexpr int k = decltype(K)::value;
        T u = uniform01(rng, T(0));
        if constexpr (M::ctrl_owner[M::noise_dof[k]] == G)
          ctrl[M::noise_dof[k]] = T(M::noise_a) + T(M::noise_b - M::noise_a) * u;
      });
    } else {
      sfor<0, (M::NNOISE + 1) / 2>([&](auto K) {
        constexpr int k = 2 * decltype(K)::value;
        constexpr bool mine0 = M::ctrl_owner[M::noise_dof[k]] == G;
        constexpr bool mine1 = k + 1 < M::NNOISE && M::ctrl_owner[M::noise_dof[k + 1 < M::NNOISE ? k + 1 : k]] == G;
        T r, sn, cs;
        box_muller(rng, &r, &sn, &cs);  // the pair's radius and angle
        if constexpr (mine0 || mine1) {
          if constexpr (mine0) ctrl[M::noise_dof[k]] = T(M::noise_a) + T(M::noise_b) * (r * cs);
          if constexpr (mine1) ctrl[M::noise_dof[k + 1]] = T(M::noise_a) + T(M::noise_b) * (r * sn);
        }
      });
    }
  }
  // ── PD servo (crates/phyz-gpu/cuda/phyz_kernels.cu:464-483) ──
  sfor<0, M::NPD>([&](auto K) {
    constexpr int d = decltype(K)::value;
    if constexpr (M::dof_owner[M::pd_v[d]] == G) {
      T tau = T(M::pd_kp[d]) * (tgt[d] - q[M::pd_q[d]]) - T(M::pd_kd[d]) * v[M::pd_v[d]];
      ctrl[M::pd_v[d]] = dmin(dmax(tau, T(-M::pd_max[d])), T(M::pd_max[d]));
    }
  });

}

// Floating-trunk plans (NOISE_G >= 0): wave NOISE_G draws one step's noise
// for every DOF into the LDS slots, the draws and transforms of
// apply_controls in the same order, so every value is the one-lane kernel's.
// It runs between the two barriers, while wave 0 runs the trunk and the other
// waves wait, instead of every wave advancing the whole stream each step.
template <class M, class T> __device__ __forceinline__ void draw_shared_noise(u64& rng, T* lds, int lane) {
  if constexpr (M::noise_dist == 1) {
    sfor<0, M::NNOISE>([&](auto K) {
      constexpr int k = decltype(K)::value;
      T u = uniform01(rng, T(0));
      lds_put(lds, M::slot_noise + k, lane, T(M::noise_a) + T(M::noise_b - M::noise_a) * u);
    });
  } else {
    sfor<0, (M::NNOISE + 1) / 2>([&](auto K) {
      constexpr int k = 2 * decltype(K)::value;
      T r, sn, cs;
      box_muller(rng, &r, &sn, &cs);
      lds_put(lds, M::slot_noise + k, lane, T(M::noise_a) + T(M::noise_b) * (r * cs));
      if constexpr (k + 1 < M::NNOISE) lds_put(lds, M::slot_noise + k + 1, lane, T(M::noise_a) + T(M::noise_b) * (r * sn));
    });
  }
}

// Value x of lane o of each aligned group of L lanes (L = 2 or 4), for every
// lane of the group: one DPP quad permutation per 32-bit half.
template <int L, int o> __device__ __forceinline__ int lane_bcast32(int x) {
  static_assert(L == 2 || L == 4, "lane groups of 2 or 4");
  constexpr int a = o, b = L == 2 ? 2 + o : o;
  return __builtin_amdgcn_mov_dpp(x, a | (a << 2) | (b << 4) | (b << 6), 0xf, 0xf, false);
}
template <int L, int o> __device__ __forceinline__ float lane_bcast(float x) {
  return __builtin_bit_cast(float, lane_bcast32<L, o>(__builtin_bit_cast(int, x)));
}
template <int L, int o> __device__ __forceinline__ double lane_bcast(double x) {
  const unsigned long long u = __builtin_bit_cast(unsigned long long, x);
  const int lo = lane_bcast32<L, o>((int)(unsigned)u), hi = lane_bcast32<L, o>((int)(unsigned)(u >> 32));
  return __builtin_bit_cast(double, ((unsigned long long)(unsigned)hi << 32) | (unsigned)lo);
}

// Split-lane kernels (LANES > 1: small launches, one lane per world would
// leave most SIMDs idle): a world's LANES lanes hold its whole state and run
// the whole step redundantly, except the revolute joints' sines and cosines,
// the step's transcendental work: lane o of the group takes joints o, o +
// LANES, ... and the results are broadcast within the group. Every lane then
// holds the same bits as the one-lane kernel computes.
template <class M, class T> __device__ __forceinline__ void trig_prepass(WS<M, T>& ws, const T* q, int lane) {
  constexpr int L = M::LANES;
  const int sub = lane & (L - 1);
  sfor<0, (M::NREV + L - 1) / L>([&](auto U) {
    constexpr int u = decltype(U)::value;
    T ang = -q[M::qoff[M::rev_body[u * L]]];
    sfor<1, L>([&](auto O) {
      constexpr int o = decltype(O)::value;
      if constexpr (u * L + o < M::NREV) {
        if (sub == o) ang = -q[M::qoff[M::rev_body[u * L + o]]];
      }
    });
    T sn, cs;
    rev_sincos(ang, &sn, &cs);
    sfor<0, L>([&](auto O) {
      constexpr int o = decltype(O)::value;
      if constexpr (u * L + o < M::NREV) {
        constexpr int b = M::rev_body[u * L + o];
        ws.ts[b] = lane_bcast<L, o>(sn);
        ws.tc[b] = lane_bcast<L, o>(cs);
      }
    });
  });
}

// One step of group G for one world (lane). State arrays are in registers; a
// group reads and writes only the DOFs of its own bodies (plus the trunk's).
template <class M, class T, int G>
__device__ __forceinline__ void step_group(T (&q)[M::NQ], T (&v)[M::NV], T (&ctrl)[M::NCTRL], T (&qdd)[M::NV],
                                           const T* tgt, u64& rng, T* rows, int S, bool write_rows, T* lds, int lane,
                                           const Terrain<T>& tr, bool draw_next) {
  constexpr int NB = M::NB;
  constexpr int NL = M::glen[G];
  constexpr int NT = M::NTRUNK;
  constexpr bool FLOAT = M::PMODE == 2;
  apply_controls<M, T, G>(q, v, ctrl, tgt, rng, lds, lane);

  WS<M, T> ws;
  if constexpr (M::LANES > 1) trig_prepass<M, T>(ws, q, lane);
  // ── pass 1: trunk (every group), then own bodies ──
  sfor<0, NT>([&](auto K) {
    constexpr int i = M::tlist[decltype(K)::value];
    body_pass1<M, T, i>(ws, q, v, rows, S, write_rows, G == 0, tr);
  });
  sfor<0, NL>([&](auto K) {
    constexpr int i = M::glist[G][decltype(K)::value];
    body_pass1<M, T, i>(ws, q, v, rows, S, write_rows, true, tr);
  });
  if constexpr (M::HAS_CONTACT && M::PLANE >= 0) {
    // Body-attached plane, penalty law (one group owns every body here).
    SV<T> fp[NB];
    sfor<0, NB>([&](auto I) { constexpr int i = decltype(I)::value; fp[i] = SV<T>{v3(T(0), T(0), T(0)), v3(T(0), T(0), T(0))}; });
    int pmask[NB];
    if constexpr (pen64<M, T>()) plane_decide<M, T>(ws, pmask);
    plane_contacts<M, T, false>(ws.Rw, ws.Pw, ws.vel, (T(*)[24]) nullptr, fp, pmask);
    sfor<0, NB>([&](auto I) { constexpr int i = decltype(I)::value; ws.pA[i] = ws.pA[i] - fp[i]; });
  }
  // ── pass 2: own bodies, leaves first ──
  sfor<0, NB>([&](auto I) { constexpr int i = decltype(I)::value; ws.IA[i] = rigid_inertia<M, T, i>(); });
  rfor<NL>([&](auto K) {
    constexpr int i = M::glist[G][decltype(K)::value];
    constexpr int p = M::parent[i];
    Sym<T> Ia;
    SV<T> pa;
    body_solve<M, T, i>(ws, q, v, ctrl, Ia, pa);
    if constexpr (p >= 0) {
      if constexpr (M::is_trunk[p] && M::PMODE == 1) {
        // A fixed trunk absorbs the subtree: nothing above it moves.
      } else if constexpr (M::is_trunk[p] && FLOAT && G != 0) {
        Sym<T> dI;
        SV<T> dp;
        propagate<M, T, i>(ws, Ia, pa, dI, dp);
        if (!ws.ok[i]) { dI = Sym<T>{}; dp = SV<T>{v3(T(0), T(0), T(0)), v3(T(0), T(0), T(0))}; }
        if constexpr (M::contrib_first[i]) {
          ws.cI[p] = dI;
          ws.cP[p] = dp;
        } else {
          sym_add(ws.cI[p], dI);
          ws.cP[p] = ws.cP[p] + dp;
        }
        if constexpr (M::contrib_put[i]) put_sym(lds, M::slot_contrib[i], lane, ws.cI[p], ws.cP[p]);
      } else {
        if (ws.ok[i]) {
          Sym<T> dI;
          SV<T> dp;
          propagate<M, T, i>(ws, Ia, pa, dI, dp);
          sym_add(ws.IA[p], dI);
          ws.pA[p] = ws.pA[p] + dp;
        }
      }
    }
  });
  if constexpr (FLOAT) {
    __syncthreads();
    if constexpr (M::NOISE_G == G) {
      // Every wave has read this step's noise before the barrier above; the
      // next step's is read after the one below.
      if (draw_next) draw_shared_noise<M, T>(rng, lds, lane);
    }
    if constexpr (G == 0) {
      // The other groups' summed subtree contributions, in body order.
      sfor<0, NB>([&](auto I) {
        constexpr int i = decltype(I)::value;
        if constexpr (M::slot_contrib[i] >= 0 && M::contrib_put[i])
          add_sym(lds, M::slot_contrib[i], lane, ws.IA[M::parent[i]], ws.pA[M::parent[i]]);
      });
      rfor<NT>([&](auto K) {
        constexpr int i = M::tlist[decltype(K)::value];
        constexpr int p = M::parent[i];
        Sym<T> Ia;
        SV<T> pa;
        body_solve<M, T, i>(ws, q, v, ctrl, Ia, pa);
        if constexpr (p >= 0) {
          if (ws.ok[i]) {
            Sym<T> dI;
            SV<T> dp;
            propagate<M, T, i>(ws, Ia, pa, dI, dp);
            sym_add(ws.IA[p], dI);
            ws.pA[p] = ws.pA[p] + dp;
          }
        }
      });
      // Trunk accelerations, then the trunk's new state, for the other groups.
      sfor<0, NT>([&](auto K) {
        constexpr int i = M::tlist[decltype(K)::value];
        body_pass3<M, T, i>(ws, qdd);
        if constexpr (M::slot_acc[i] >= 0) {
          const int s = M::slot_acc[i];
          lds_put(lds, s, lane, ws.acc[i].a.x); lds_put(lds, s + 1, lane, ws.acc[i].a.y); lds_put(lds, s + 2, lane, ws.acc[i].a.z);
          lds_put(lds, s + 3, lane, ws.acc[i].l.x); lds_put(lds, s + 4, lane, ws.acc[i].l.y); lds_put(lds, s + 5, lane, ws.acc[i].l.z);
        }
        body_integrate<M, T, i, quat_from_pass1<M, T, i>()>(q, v, qdd, ws.qj[i]);
      });
      sfor<0, M::NQ>([&](auto J) {
        constexpr int j = decltype(J)::value;
        if constexpr (M::dof_group[j] == -1) {
          lds_put(lds, M::slot_state + 2 * M::tdof[j], lane, q[j]);
          lds_put(lds, M::slot_state + 2 * M::tdof[j] + 1, lane, v[j]);
        }
      });
    }
    __syncthreads();
    if constexpr (G != 0) {
      sfor<0, NT>([&](auto K) {
        constexpr int i = M::tlist[decltype(K)::value];
        if constexpr (M::slot_acc[i] >= 0) {
          const int s = M::slot_acc[i];
          ws.acc[i] = SV<T>{v3(lds_get(lds, s, lane), lds_get(lds, s + 1, lane), lds_get(lds, s + 2, lane)),
                            v3(lds_get(lds, s + 3, lane), lds_get(lds, s + 4, lane), lds_get(lds, s + 5, lane))};
        }
      });
      sfor<0, M::NQ>([&](auto J) {
        constexpr int j = decltype(J)::value;
        if constexpr (M::dof_group[j] == -1) {
          q[j] = lds_get(lds, M::slot_state + 2 * M::tdof[j], lane);
          v[j] = lds_get(lds, M::slot_state + 2 * M::tdof[j] + 1, lane);
        }
      });
    }
  } else {
    // Trunk accelerations (constants for a fixed trunk; the whole tree otherwise empty).
    sfor<0, NT>([&](auto K) {
      constexpr int i = M::tlist[decltype(K)::value];
      body_pass3<M, T, i>(ws, qdd);
    });
  }
  // ── pass 3 and integration: own bodies ──
  sfor<0, NL>([&](auto K) {
    constexpr int i = M::glist[G][decltype(K)::value];
    body_pass3<M, T, i>(ws, qdd);
    body_integrate<M, T, i, quat_from_pass1<M, T, i>()>(q, v, qdd, ws.qj[i]);
  });
}

// The ABA's response to a change of the external forces with q, v and ctrl
// fixed (the impulse sweeps). The articulated-body solve is affine in the
// external forces, so with the step's factorization (X, U, L, D^-1, ok) kept,
// qdd(ext) = qdd(ext0) + dqdd(ext - ext0), where dqdd runs passes 2 and 3 on
// the force change alone: dp_A = -(ext - ext0), du = -S^T dp_A,
// dp_a = dp_A + U D^-1 du up the tree; da = X da_parent (zero at the root:
// gravity and the velocity-product terms are in qdd(ext0)),
// dqdd = D^-1 (du - U^T da), da += S dqdd down the tree.
template <class M, class T, int i> __device__ __forceinline__ void body_delta_up(WS<M, T>& ws, SV<T> (&dp)[M::NB]) {
  constexpr int nd = ndof_of(M::jtype[i]);
  constexpr int p = M::parent[i];
  constexpr int MAXD = M::MAXD;
  SV<T> pa = dp[i];
  if constexpr (nd > 0) {
#pragma unroll
    for (int k = 0; k < nd; k++) ws.uu[i][k] = -dot(subspace<M, T, i>(k), dp[i]);
    if constexpr (p >= 0) {
      T y[MAXD];
#pragma unroll
      for (int k = 0; k < nd; k++) {
        y[k] = ws.uu[i][k];
#pragma unroll
        for (int t = 0; t < k; t++) y[k] = y[k] - ws.Lm[i][k][t] * y[t];
      }
#pragma unroll
      for (int k = 0; k < nd; k++) y[k] = y[k] * ws.Dinv[i][k];
#pragma unroll
      for (int k = nd - 1; k >= 0; k--)
#pragma unroll
        for (int t = k + 1; t < nd; t++) y[k] = y[k] - ws.Lm[i][t][k] * y[t];
#pragma unroll
      for (int k = 0; k < nd; k++) {
        const SV<T> uk = {v3(Uv<M, T, i>(ws, k, 0), Uv<M, T, i>(ws, k, 1), Uv<M, T, i>(ws, k, 2)), v3(Uv<M, T, i>(ws, k, 3), Uv<M, T, i>(ws, k, 4), Uv<M, T, i>(ws, k, 5))};
        pa = pa + uk * y[k];
      }
    }
  }
  if constexpr (p >= 0) {
    if (ws.ok[i]) dp[p] = dp[p] + inv_apply_force(ws.X[i], pa);
  }
}
template <class M, class T, int i> __device__ __forceinline__ void body_delta_down(WS<M, T>& ws, T* dqdd) {
  constexpr int nd = ndof_of(M::jtype[i]);
  constexpr int p = M::parent[i];
  constexpr int vo = M::voff[i];
  constexpr int MAXD = M::MAXD;
  SV<T> ap;
  if constexpr (p < 0) ap = SV<T>{v3(T(0), T(0), T(0)), v3(T(0), T(0), T(0))};
  else ap = apply_motion(ws.X[i], ws.acc[p]);
  if constexpr (nd > 0) {
    T y[MAXD];
#pragma unroll
    for (int k = 0; k < nd; k++) {
      T uta = Uv<M, T, i>(ws, k, 0) * ap.a.x + Uv<M, T, i>(ws, k, 1) * ap.a.y + Uv<M, T, i>(ws, k, 2) * ap.a.z + Uv<M, T, i>(ws, k, 3) * ap.l.x +
              Uv<M, T, i>(ws, k, 4) * ap.l.y + Uv<M, T, i>(ws, k, 5) * ap.l.z;
      y[k] = ws.uu[i][k] - uta;
#pragma unroll
      for (int t = 0; t < k; t++) y[k] = y[k] - ws.Lm[i][k][t] * y[t];
    }
#pragma unroll
    for (int k = 0; k < nd; k++) y[k] = y[k] * ws.Dinv[i][k];
#pragma unroll
    for (int k = nd - 1; k >= 0; k--)
#pragma unroll
      for (int t = k + 1; t < nd; t++) y[k] = y[k] - ws.Lm[i][t][k] * y[t];
#pragma unroll
    for (int k = 0; k < nd; k++) {
      y[k] = ws.ok[i] ? y[k] : T(0);
      dqdd[vo + k] = y[k];
      ap = ap + subspace<M, T, i>(k) * y[k];
    }
  }
  ws.acc[i] = ap;
}

template <class M> struct HasExt {
  template <int i> static constexpr bool at() { return M::gtype[i] != G_NONE || i == M::PLANE; }
};

// One impulse-mode step of one world (crates/phyz-gpu/src/cuda/mod.rs:899-928):
// controls; FK, velocities and bias forces once; a full ABA against the
// contact forces carried from the previous step; the contact geometry; then
// SWEEPS x [contact at the free velocity v + dt qdd (warm-started), the ABA's
// response to the change of the contact forces]; integrate.
// ext, impg (ground) and impp (plane) persist between steps.
template <class M, class T>
__device__ __forceinline__ void step_impulse(T (&q)[M::NQ], T (&v)[M::NV], T (&ctrl)[M::NCTRL], T (&qdd)[M::NV],
                                             const T* tgt, u64& rng, SV<T> (&ext)[M::NB], T (&impg)[M::NB][24],
                                             T (&impp)[M::NB][24], const Terrain<T>& tr, T* rows, int S,
                                             bool write_rows) {
  constexpr int NB = M::NB;
  apply_controls<M, T, 0>(q, v, ctrl, tgt, rng, nullptr, 0);
  WS<M, T> ws;
  sfor<0, NB>([&](auto I) {
    constexpr int i = decltype(I)::value;
    body_pass1<M, T, i>(ws, q, v, rows, S, false, false, tr);
  });
  // The contacts' geometry depends on q alone: prepared straight after pass 1,
  // so the world transforms it reads need not outlive passes 2 and 3.
  int pmask[NB];
  if constexpr (M::PLANE >= 0 && pen64<M, T>()) plane_decide<M, T>(ws, pmask);
  GroundPrep<M, T> gp;
  sfor<0, NB>([&](auto I) {
    constexpr int i = decltype(I)::value;
    if constexpr (M::gtype[i] != G_NONE) ground_prepare<M, T, i>(ws.Rw[i], ws.Pw[i], ws, tr, gp, rows, S, write_rows);
  });
  sfor<0, NB>([&](auto I) {
    constexpr int i = decltype(I)::value;
    if constexpr (HasExt<M>::template at<i>()) ws.pA[i] = ws.pA[i] - ext[i];
    ws.IA[i] = rigid_inertia<M, T, i>();
  });
  rfor<NB>([&](auto I) {
    constexpr int i = decltype(I)::value;
    constexpr int p = M::parent[i];
    Sym<T> Ia;
    SV<T> pa;
    body_solve<M, T, i>(ws, q, v, ctrl, Ia, pa);
    if constexpr (p >= 0) {
      if (ws.ok[i]) {
        Sym<T> dI;
        SV<T> dp;
        propagate<M, T, i>(ws, Ia, pa, dI, dp);
        sym_add(ws.IA[p], dI);
        ws.pA[p] = ws.pA[p] + dp;
      }
    }
  });
  sfor<0, NB>([&](auto I) { body_pass3<M, T, decltype(I)::value>(ws, qdd); });
  // Each sweep moves qdd by the ABA's response to that sweep's change of the
  // contact forces (the solve is affine in them): qdd and ext carry from one
  // sweep to the next, so neither the step's first qdd nor its first forces
  // stay live through the loop.
  // A plain loop: compact and exact at every sweep count. Left to the
  // compiler's own unrolling choice, the f64 kernel of an 8-corner box gave
  // wrong impulses from the fourth sweep on (checked across sweep counts in
  // tests/test_gpu_contact_modes.py).
#pragma unroll 1
  for (int sw = 0; sw < M::SWEEPS; sw++) {
    // Body velocities at the free joint velocity v + dt qdd.
    T vv[M::NV];
#pragma unroll
    for (int j = 0; j < M::NV; j++) vv[j] = v[j] + T(M::dt) * qdd[j];
    SV<T> vf[NB];
    sfor<0, NB>([&](auto I) {
      constexpr int i = decltype(I)::value;
      constexpr int p = M::parent[i];
      const SV<T> vj = joint_vel<M, T, i>(vv);
      if constexpr (p < 0) vf[i] = vj;
      else vf[i] = apply_motion(ws.X[i], vf[p]) + vj;
    });
    const bool wr = write_rows && sw == M::SWEEPS - 1;
    SV<T> dp[NB];  // the previous sweep's forces, then their change
    sfor<0, NB>([&](auto I) {
      constexpr int i = decltype(I)::value;
      if constexpr (HasExt<M>::template at<i>()) dp[i] = ext[i];
      else dp[i] = SV<T>{v3(T(0), T(0), T(0)), v3(T(0), T(0), T(0))};
    });
    sfor<0, NB>([&](auto I) {
      constexpr int i = decltype(I)::value;
      if constexpr (M::gtype[i] != G_NONE) {
        ext[i] = ground_sweep<M, T, i>(gp, vf[i], impg[i]);
        if constexpr (M::PLANE >= 0) {
          // The reference clears a body's whole contact state, plane impulses
          // included, when it is off the ground; the plane pass then starts
          // those from zero in every sweep.
          if (!gp.any[i]) {
#pragma unroll
            for (int k = 0; k < 3 * ground_pts<M>(i); k++) impp[i][k] = T(0);
          }
          if (wr) {
            const V3<T> ft = mul(ws.Rw[i], ext[i].l);  // summed ground force, world frame
            T* r = rows + 8 * i * S;
            r[5 * S] = gp.any[i] ? ft.x : T(0);
            r[6 * S] = gp.any[i] ? ft.y : T(0);
            r[7 * S] = gp.any[i] ? ft.z : T(0);
          }
        }
      } else if constexpr (i == M::PLANE) {
        ext[i] = SV<T>{v3(T(0), T(0), T(0)), v3(T(0), T(0), T(0))};
      }
    });
    if constexpr (M::PLANE >= 0) plane_contacts<M, T, true>(ws.Rw, ws.Pw, vf, impp, ext, pmask);
    sfor<0, NB>([&](auto I) {
      constexpr int i = decltype(I)::value;
      if constexpr (HasExt<M>::template at<i>()) dp[i] = dp[i] - ext[i];
    });
    rfor<NB>([&](auto I) { body_delta_up<M, T, decltype(I)::value>(ws, dp); });
    T dqdd[M::NV];
    sfor<0, NB>([&](auto I) { body_delta_down<M, T, decltype(I)::value>(ws, dqdd); });
#pragma unroll
    for (int j = 0; j < M::NV; j++) qdd[j] = qdd[j] + dqdd[j];
  }
  if constexpr (M::PLANE < 0) {
    // Without a plane, ext holds the last sweep's ground forces: the readback
    // rows' world force, with the body rotations recomputed here (rows are
    // written on a launch's last step only, and the rotations do not stay live
    // through the sweeps).
    if (write_rows) {
      R3<T> Rw[NB];
      sfor<0, NB>([&](auto I) {
        constexpr int i = decltype(I)::value;
        constexpr int p = M::parent[i];
        if constexpr (M::need_world[i]) {
          R3<T> E = ws.X[i].E;
#pragma unroll
          for (int k = 0; k < 9; k++) asm volatile("" : "+v"(E.m[k]));  // recompute, not reuse pass 1's
          Rw[i] = p < 0 ? transpose(E) : mul_bt(Rw[p < 0 ? 0 : p], E);
        }
        if constexpr (M::gtype[i] != G_NONE) {
          const V3<T> ft = mul(Rw[i], ext[i].l);
          T* r = rows + 8 * i * S;
          r[5 * S] = gp.any[i] ? ft.x : T(0);
          r[6 * S] = gp.any[i] ? ft.y : T(0);
          r[7 * S] = gp.any[i] ? ft.z : T(0);
        }
      });
    }
  }
  sfor<0, NB>([&](auto I) { body_integrate<M, T, decltype(I)::value>(q, v, qdd); });
}

// Kernel body for group G: load the world's state, run nsteps, store. A group
// loads the DOFs it owns and the trunk's; it stores only the DOFs it owns
// (group 0 also stores the trunk's and the RNG state).
template <class M, class T, int G> __device__ __forceinline__ void run_group(const StepArgs& a, int lane, T* lds) {
  if constexpr (sizeof(T) == 8 || pen64<M, T>()) {
    // The f64 sine / cosine and log tables (f64 kernels, and the f32 contact
    // kernels' f64 penetration chain), before any lane of the workgroup returns.
    if constexpr (G == 0) fill_tables(lane);
    __syncthreads();
  }
  // Split-lane kernels give each world LANES consecutive lanes.
  const int w = (int)(blockIdx.x * 64 + lane) / M::LANES;
  const bool live = w < a.nworld;
  if constexpr (M::PMODE != 2) {
    if (!live) return;
  }
  const int wl = live ? w : a.nworld - 1;  // out-of-range lanes shadow the last world (no stores)
  const int S = a.stride;
  T* gq = (T*)a.q;
  T* gv = (T*)a.v;
  T* gc = (T*)a.ctrl;
  T q[M::NQ], v[M::NV], ctrl[M::NCTRL], qdd[M::NV];
  sfor<0, M::NQ>([&](auto J) {
    constexpr int j = decltype(J)::value;
    if constexpr (M::dof_group[j] == G || M::dof_group[j] == -1) {
      q[j] = gq[j * S + wl];
      v[j] = gv[j * S + wl];
    } else {
      q[j] = T(0); v[j] = T(0);
    }
    qdd[j] = T(0);
  });
  sfor<0, M::NCTRL>([&](auto J) {
    constexpr int j = decltype(J)::value;
    if constexpr (M::ctrl_group[j] == G || M::ctrl_group[j] == -1) ctrl[j] = gc[j * S + wl];
    else ctrl[j] = T(0);
  });
  T tgt[M::NPD > 0 ? M::NPD : 1];
  sfor<0, M::NPD>([&](auto K) {
    constexpr int d = decltype(K)::value;
    if constexpr (M::dof_owner[M::pd_v[d]] == G) tgt[d] = ((const T*)a.targets)[d * S + wl];
    else tgt[d] = T(0);
  });
  u64 rng = 0;
  if constexpr (M::NNOISE > 0) rng = a.rng[wl];
  T* rows = M::HAS_CONTACT ? (T*)a.contact_rows + wl : nullptr;
  const Terrain<T> tr{(const double*)a.hf, a.hf_ox, a.hf_oy, a.hf_oz, a.hf_cell, a.hf_nx, a.hf_ny};
  const int n = a.nsteps;
  if constexpr (M::HAS_CONTACT && M::CMODE == 1) {
    // Impulse mode: one group (checked on the host); the solver state persists.
    SV<T> ext[M::NB];
    T impg[M::NB][24], impp[M::NB][24];
    const T* ge = (const T*)a.ext;
    const T* gi = (const T*)a.imp;
    sfor<0, M::NB>([&](auto I) {
      constexpr int i = decltype(I)::value;
      constexpr int np3 = 3 * (M::gtype[i] == G_BOX ? 8 : 1);
      if constexpr (HasExt<M>::template at<i>()) {
        ext[i] = SV<T>{v3(ge[(6 * i) * S + wl], ge[(6 * i + 1) * S + wl], ge[(6 * i + 2) * S + wl]),
                       v3(ge[(6 * i + 3) * S + wl], ge[(6 * i + 4) * S + wl], ge[(6 * i + 5) * S + wl])};
      }
      if constexpr (M::gtype[i] != G_NONE) {
#pragma unroll
        for (int k = 0; k < np3; k++) {
          impg[i][k] = gi[(48 * i + k) * S + wl];
          impp[i][k] = M::PLANE >= 0 ? gi[(48 * i + 24 + k) * S + wl] : T(0);
        }
      }
    });
    for (int s = 0; s < n; s++) {
      const bool last = (s == n - 1) && a.write_contacts && live;
      step_impulse<M, T>(q, v, ctrl, qdd, tgt, rng, ext, impg, impp, tr, rows, S, last);
    }
    if (live) {
      T* he = (T*)a.ext;
      T* hi = (T*)a.imp;
      asm volatile("" : "+s"(he), "+s"(hi));  // fresh addresses (see below)
      sfor<0, M::NB>([&](auto I) {
        constexpr int i = decltype(I)::value;
        constexpr int np3 = 3 * (M::gtype[i] == G_BOX ? 8 : 1);
        if constexpr (HasExt<M>::template at<i>()) {
          he[(6 * i) * S + w] = ext[i].a.x; he[(6 * i + 1) * S + w] = ext[i].a.y; he[(6 * i + 2) * S + w] = ext[i].a.z;
          he[(6 * i + 3) * S + w] = ext[i].l.x; he[(6 * i + 4) * S + w] = ext[i].l.y; he[(6 * i + 5) * S + w] = ext[i].l.z;
        }
        if constexpr (M::gtype[i] != G_NONE) {
#pragma unroll
          for (int k = 0; k < np3; k++) {
            hi[(48 * i + k) * S + w] = impg[i][k];
            if constexpr (M::PLANE >= 0) hi[(48 * i + 24 + k) * S + w] = impp[i][k];
          }
        }
      });
    }
  } else {
    if constexpr (M::NOISE_G >= 0) {
      if constexpr (G == M::NOISE_G) draw_shared_noise<M, T>(rng, lds, lane);
      __syncthreads();
    }
    for (int s = 0; s < n; s++) {
      const bool last = (s == n - 1) && a.write_contacts && live;
      step_group<M, T, G>(q, v, ctrl, qdd, tgt, rng, rows, S, last, lds, lane, tr, s + 1 < n);
    }
  }
  if (!live) return;
  if constexpr (M::LANES > 1) {
    if ((lane & (M::LANES - 1)) != 0) return;  // the group's first lane stores
  }
  // Addresses for the final stores computed afresh: reusing the loads' per-DOF
  // addresses would keep them live through every step of the launch.
  asm volatile("" : "+s"(gq), "+s"(gv), "+s"(gc));
  sfor<0, M::NQ>([&](auto J) {
    constexpr int j = decltype(J)::value;
    if constexpr (M::dof_group[j] == G || (G == 0 && M::dof_group[j] == -1)) {
      gq[j * S + w] = q[j];
      gv[j * S + w] = v[j];
      ((T*)a.qdd)[j * S + w] = qdd[j];
    }
  });
  sfor<0, M::NCTRL>([&](auto J) {
    constexpr int j = decltype(J)::value;
    if constexpr (M::ctrl_group[j] == G || (G == 0 && M::ctrl_group[j] == -1)) gc[j * S + w] = ctrl[j];
  });
  if constexpr (M::NNOISE > 0 && G == (M::NOISE_G >= 0 ? M::NOISE_G : 0)) a.rng[w] = rng;
}

#if PHZ_REASSOC
#pragma clang fp reassociate(off)
#endif
}  // namespace phz
