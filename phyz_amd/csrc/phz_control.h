// phz_control.h — the device-resident control loop for gfx950 (CDNA4):
// FK readout, observation ops and the MLP policy pass.
//
// Behaviour follows crates/phyz-gpu/src/policy_pipeline.rs (ObsOp, PolicySpec,
// observe_reference, policy_reference, KernelRng) and the reference passes
// crates/phyz-gpu/cuda/phyz_kernels.cu:1423-1715 (fk_thread, obs_thread,
// policy_thread). The layout here is this library's own:
//
//   phz_obs     one lane per world, model and op table compiled in (the host
//               emits `struct Model` and `struct Obs` of constexpr tables).
//               FK in registers; the FK readout rows and the observation row
//               are stored structure-of-arrays ([j][stride]) so a wave's
//               stores coalesce.
//   phz_policy  one wave per 16*CB worlds. The three MLP layers run on f32
//               MFMA (v_mfma_f32_16x16x4f32) with the weights as the A
//               operand and the activations as the B operand, so a layer's
//               16x16 output tiles are already laid out as the next layer's
//               B fragments: hidden activations never leave registers. Only
//               the per-world prologue (input noise) and epilogue (Gaussian
//               sample, log-prob, PD targets) go through LDS, because each
//               world's random stream is sequential and lives in one lane.
#pragma once

namespace phz {

// ── FK readout and observations ──────────────────────────────────────────────

// Observation op kinds: the packed table row [kind, a, b, c] of ObsOp::pack
// (crates/phyz-gpu/src/policy_pipeline.rs:115-137).
enum {
  OBS_CONST = 0,    // c
  OBS_QMINUS = 1,   // q[a] - c
  OBS_V = 2,        // v[a]
  OBS_PITCH = 3,    // atan2(-r02, r22), r = world->body rotation of body a
  OBS_ROLL = 4,     // atan2(r12, r22)
  OBS_YAWERR = 5,   // wrap(c - atan2(r01, r00))
  OBS_POSZ = 6,     // body a origin z, world
  OBS_POS = 7,      // body a origin, world axis b
  OBS_COM_SUPPORT = 8  // centre of mass minus mean support point, axis c; aux window (a, b)
};

constexpr int XF_STRIDE = 18;  // rotation world->body (9, row-major), origin (3), omega (3), v (3), body frame

struct ObsArgs {
  const void* q;  // [nq][stride] T
  const void* v;  // [nv][stride] T
  void* kin;      // [nb * XF_STRIDE][stride] T, written when write_kin
  float* obs;     // [n_in][stride] f32, the history row of this control step, written when write_obs
  int nworld;
  int stride;
  int write_kin;
  int write_obs;
};

template <class M, class T> struct FKState {
  R3<T> Rw[M::NB];  // body -> world rotation
  V3<T> Pw[M::NB];  // body origin in world
  SV<T> vel[M::NB]; // body-frame spatial velocity
};

// Forward kinematics of every body (crates/phyz-rigid/src/kinematics.rs:10-50,
// the same chain as the reference's fk_world).
template <class M, class T> __device__ __forceinline__ void fk_all(const T* q, const T* v, FKState<M, T>& f) {
  sfor<0, M::NB>([&](auto I) {
    constexpr int i = decltype(I)::value;
    constexpr int p = M::parent[i];
    Xf<T> X;
    SV<T> vj;
    joint_xf<M, T, i>(q, v, X, vj);
    if constexpr (p < 0) {
      f.vel[i] = vj;
      f.Rw[i] = transpose(X.E);
      f.Pw[i] = X.r;
    } else {
      f.vel[i] = apply_motion(X, f.vel[p]) + vj;
      f.Rw[i] = mul_bt(f.Rw[p], X.E);
      f.Pw[i] = f.Pw[p] + mul(f.Rw[p], X.r);
    }
  });
}

template <class T> __device__ __forceinline__ T wrap_pi(T a) {
  const T pi = T(3.14159265358979323846);
  while (a > pi) a -= T(2) * pi;
  while (a < -pi) a += T(2) * pi;
  return a;
}

template <class T> __device__ __forceinline__ T axis_of(V3<T> p, int axis) {
  return axis == 0 ? p.x : (axis == 1 ? p.y : p.z);
}

// One feature (ObsOp::eval, policy_pipeline.rs:189-249). The world->body
// rotation r is Rw^T, so r[i][j] = Rw.m[3 j + i].
template <class M, class O, class T, int k>
__device__ __forceinline__ T obs_feature(const T* q, const T* v, const FKState<M, T>& f) {
  constexpr int kind = O::kind[k], a = O::a[k], b = O::b[k];
  if constexpr (kind == OBS_CONST) {
    return T(O::c[k]);
  } else if constexpr (kind == OBS_QMINUS) {
    return q[a] - T(O::c[k]);
  } else if constexpr (kind == OBS_V) {
    return v[a];
  } else if constexpr (kind == OBS_PITCH) {
    return datan2(-f.Rw[a].m[6], f.Rw[a].m[8]);
  } else if constexpr (kind == OBS_ROLL) {
    return datan2(f.Rw[a].m[7], f.Rw[a].m[8]);
  } else if constexpr (kind == OBS_YAWERR) {
    return wrap_pi(T(O::c[k]) - datan2(f.Rw[a].m[3], f.Rw[a].m[0]));
  } else if constexpr (kind == OBS_POSZ) {
    return f.Pw[a].z;
  } else if constexpr (kind == OBS_POS) {
    return axis_of(f.Pw[a], b > 2 ? 2 : b);
  } else {
    // ComOverSupport: aux window [heading_flag, heading_body, (body, ox, oy, oz) x b] at a.
    if constexpr (b == 0) {
      return T(0);
    } else {
      V3<T> com = v3(T(0), T(0), T(0));
      T mt = T(0);
      sfor<0, M::NB>([&](auto I) {
        constexpr int i = decltype(I)::value;
        if constexpr (M::mass[i] > 0.0) {
          const V3<T> c = v3(T(M::com[i][0]), T(M::com[i][1]), T(M::com[i][2]));
          com = com + (f.Pw[i] + mul(f.Rw[i], c)) * T(M::mass[i]);
          mt = mt + T(M::mass[i]);
        }
      });
      if (mt > T(0)) com = com * (T(1) / dmax(mt, T(1e-30)));
      V3<T> tgt = v3(T(0), T(0), T(0));
      sfor<0, b>([&](auto J) {
        constexpr int base = a + 2 + 4 * decltype(J)::value;
        constexpr int body = (int)O::aux[base];
        const V3<T> o = v3(T(O::aux[base + 1]), T(O::aux[base + 2]), T(O::aux[base + 3]));
        tgt = tgt + f.Pw[body] + mul(f.Rw[body], o);
      });
      const V3<T> e = com - tgt * (T(1) / T(b));
      constexpr int axis = (int)O::c[k];
      if constexpr (O::aux[a] != 0.0) {
        constexpr int h = (int)O::aux[a + 1];
        const T yaw = datan2(f.Rw[h].m[3], f.Rw[h].m[0]);
        T sy, cy;
        dsincos(yaw, &sy, &cy);
        if constexpr (axis == 0) return cy * e.x + sy * e.y;
        else if constexpr (axis == 1) return -sy * e.x + cy * e.y;
        else return e.z;
      } else {
        return axis_of(e, axis);
      }
    }
  }
}

template <class M, class O, class T> __device__ __forceinline__ void obs_world(const ObsArgs& a, int w) {
  const T* gq = (const T*)a.q;
  const T* gv = (const T*)a.v;
  const int S = a.stride;
  T q[M::NQ], v[M::NV];
#pragma unroll
  for (int j = 0; j < M::NQ; j++) q[j] = gq[j * S + w];
#pragma unroll
  for (int j = 0; j < M::NV; j++) v[j] = gv[j * S + w];
  FKState<M, T> f;
  fk_all<M, T>(q, v, f);
  if (a.write_kin) {
    T* kin = (T*)a.kin;
    sfor<0, M::NB>([&](auto I) {
      constexpr int i = decltype(I)::value;
      T* r = kin + (size_t)(i * XF_STRIDE) * S + w;
      const R3<T> wb = transpose(f.Rw[i]);
#pragma unroll
      for (int k = 0; k < 9; k++) r[k * S] = wb.m[k];
      r[9 * S] = f.Pw[i].x;
      r[10 * S] = f.Pw[i].y;
      r[11 * S] = f.Pw[i].z;
      r[12 * S] = f.vel[i].a.x;
      r[13 * S] = f.vel[i].a.y;
      r[14 * S] = f.vel[i].a.z;
      r[15 * S] = f.vel[i].l.x;
      r[16 * S] = f.vel[i].l.y;
      r[17 * S] = f.vel[i].l.z;
    });
  }
  if constexpr (O::N > 0) {
    if (a.write_obs) {
      sfor<0, O::N>([&](auto K) {
        constexpr int k = decltype(K)::value;
        a.obs[(size_t)k * S + w] = (float)obs_feature<M, O, T, k>(q, v, f);
      });
    }
  }
}

// ── policy: two-hidden-layer tanh MLP, diagonal Gaussian, PD targets ─────────

typedef float f32x4 __attribute__((ext_vector_type(4)));

struct PolicyArgs {
  const f32x4* w1;     // [KU][NHB][64] x 4 fragments of W1 (host re-layout, zero padded)
  const f32x4* w2;     // [NHB][NHB][64] x 4 fragments of W2, input block major
  const f32x4* w3;     // [NHB][NOB][64] x 4 fragments of W3, input block major
  const float* bias;   // b1[NHB*16] b2[NHB*16] b3[NOB*16], zero padded
  const float* stdv;   // [NO]
  float* obs;          // [NI][stride], this control step's history row (noised in place)
  float* out;          // [NO + 1][stride], actions then log-prob
  u64* rng;            // [stride] policy streams
  float* z;            // [NO][stride] AR(1) noise state
  const void* base;    // [NPD][stride] T, base PD targets
  void* targets;       // [NPD][stride] T, PD targets the step kernel reads
  int nworld;
  int stride;
};

// KernelRng::uniform / normal (policy_pipeline.rs:441-456): 53-bit uniform,
// Box-Muller on two uniforms, cosine branch, in double: sqrt(-2 ln u1) cos(2 pi
// u2) with u1 >= 1e-300. The uniforms come from the draws' 32-bit words in one
// exact fma each; ln is tab_log and the root nr_sqrt (the step kernels' f64
// Box-Muller, within 1 ulp each); the cosine is taken in turns, where the
// reduction is exact (t = 64 u2, k = rint(t), r = (t - k) 2 pi / 64) and the
// LDS table gives cos(2 pi k / 64), within 2 ulp of the cosine of the exact
// angle. These 37 normals per world and control step are the part of the
// policy kernel that does not overlap its MFMAs; the kernel fills the tables
// at its start.
__device__ __forceinline__ void policy_uniforms(u64& s, double& u1, double& t) {
  const u64 x1 = xorshift64(s);
  const u64 x2 = xorshift64(s);
  u1 = fma((double)(unsigned)(x1 >> 32), 0x1p-32, (double)((unsigned)x1 >> 11) * 0x1p-53);
  t = fma((double)(unsigned)(x2 >> 32), 0x1p-26, (double)((unsigned)x2 >> 11) * 0x1p-47);
}
__device__ __forceinline__ double policy_transform(double u1, double t) {
  const double k = rint(t);
  double sn, cs;
  tab_sincos_at((t - k) * 0x1.921fb54442d18p-4, cvt_sat_i32(k) & 63, &sn, &cs);
  return nr_sqrt(-2.0 * tab_log(fmax(u1, 1e-300))) * cs;
}
__device__ __forceinline__ double policy_normal(u64& s) {
  double u1, t;
  policy_uniforms(s, u1, t);
  return policy_transform(u1, t);
}

// A double from lane `lane ^ 32`, the other half of the wave (ds_bpermute,
// which every lane of the wave executes).
__device__ __forceinline__ double from_other_half(double v, int lane) {
  const u64 b = __builtin_bit_cast(u64, v);
  const int addr = (lane ^ 32) << 2;
  const unsigned lo = (unsigned)__builtin_amdgcn_ds_bpermute(addr, (int)(unsigned)b);
  const unsigned hi = (unsigned)__builtin_amdgcn_ds_bpermute(addr, (int)(unsigned)(b >> 32));
  return __builtin_bit_cast(double, ((u64)hi << 32) | lo);
}

// The next N normals of the stream in lanes 0..31 (one world each; lanes
// 32..63 own none), the same values as N calls of policy_normal there. The
// world's lane draws every pair of uniforms in order; the transforms, the
// costly part, run two at a time: normal 2j in the world's lane and normal
// 2j + 1 in lane + 32, whose uniforms and result cross the wave's halves.
// Lanes 32..63 advance a stream of their own that nothing reads. Every lane
// of the wave calls it, outside any branch.
template <int N> __device__ __forceinline__ void policy_normals_paired(u64& s, int lane, double (&n)[N]) {
#pragma unroll
  for (int j = 0; j < N; j += 2) {
    double u1a, ta, u1b = 0.5, tb = 0.0;
    policy_uniforms(s, u1a, ta);
    if (j + 1 < N) policy_uniforms(s, u1b, tb);
    const double pu = from_other_half(u1b, lane), pt = from_other_half(tb, lane);
    const bool upper = lane >= 32;
    const double r = policy_transform(upper ? pu : u1a, upper ? pt : ta);
    n[j] = r;
    if (j + 1 < N) n[j + 1] = from_other_half(r, lane);
  }
}

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// tanh without branches, from tanh|x| = (1 - t) / (1 + t), t = e^(-2|x|) = 2^(-2|x| log2 e)
// (hardware exp2 and reciprocal, about 1 ulp each), and the odd series
// x - x^3/3 + 2x^5/15 - 17x^7/315 below |x| = 1/16, where 1 - t cancels; the
// series' first omitted term is under 1e-12 relative there. Absolute error
// stays near 2e-7 over the whole range; NaN propagates.
__device__ __forceinline__ float tanh_mlp(float x) {
  const float ax = fabsf(x);
  const float t = __builtin_amdgcn_exp2f(-2.88539008177792681f * ax);
  const float big = (1.0f - t) * __builtin_amdgcn_rcpf(1.0f + t);
  const float x2 = x * x;
  const float small = ax * (1.0f + x2 * (-0.333333333333f + x2 * (0.133333333333f + x2 * -0.0539682539683f)));
  return copysignf(ax < 0.0625f ? small : big, x);
}

template <int NB_, int CB> __device__ __forceinline__ void bias_tiles(const float* bias, int g, f32x4 (&acc)[NB_][CB]) {
#pragma unroll
  for (int ob = 0; ob < NB_; ob++) {
    f32x4 b0;
#pragma unroll
    for (int j = 0; j < 4; j++) b0[j] = bias[ob * 16 + 4 * g + j];
#pragma unroll
    for (int cb = 0; cb < CB; cb++) acc[ob][cb] = b0;
  }
}

template <int NB_, int CB> __device__ __forceinline__ void tanh_tiles(f32x4 (&h)[NB_][CB]) {
#pragma unroll
  for (int ob = 0; ob < NB_; ob++)
#pragma unroll
    for (int cb = 0; cb < CB; cb++)
#pragma unroll
      for (int j = 0; j < 4; j++) h[ob][cb][j] = tanh_mlp(h[ob][cb][j]);
}

// acc[ob][cb] += sum over k of W[ob block][k] B[k][cb block]. The weights are
// fragments [kb][ob][lane] x 4 (component s = k-step s of input block kb), read
// in that order as one contiguous stream with PF fragments in flight; the
// sched_barrier keeps the compiler from sinking the prefetches to their use,
// which would expose a full L2 round trip per fragment. bfrag(kb, s, cb) is
// the B operand (this lane's input value) of k-step s of block kb for world
// block cb.
template <int NKB, int NOB_, int CB, class BF>
__device__ __forceinline__ void mfma_layer(const f32x4* __restrict__ w, int lane, f32x4 (&acc)[NOB_][CB], BF bfrag) {
  constexpr int NT = NKB * NOB_;
  constexpr int PF = NT < 6 ? NT : 6;
  f32x4 ring[PF];
#pragma unroll
  for (int t = 0; t < PF; t++) ring[t] = w[t * 64 + lane];
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const int kb = t / NOB_, ob = t % NOB_;
    const f32x4 wa = ring[t % PF];
    if (t + PF < NT) ring[t % PF] = w[(t + PF) * 64 + lane];
#pragma unroll
    for (int s = 0; s < 4; s++)
#pragma unroll
      for (int cb = 0; cb < CB; cb++) acc[ob][cb] = mfma4(wa[s], bfrag(kb, s, cb), acc[ob][cb]);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// v_mfma_f32_16x16x4f32 lane layout: A[i][k] in lane i + 16 k, B[k][j] in
// lane j + 16 k, D[i][j] in lane j + 16 (i / 4), register i % 4.
// Layer l computes H_l^T = tanh(W_l H_{l-1}^T + b_l): rows are neurons, columns
// worlds. For the next layer, k-step s of input block kb uses register s of
// the previous output tile, i.e. lane j + 16 g supplies neuron 16 kb + 4 g + s
// of world j; the host lays W out to match (phz_host.cpp, policy_fragments).
// Inputs with observation noise, the prologue's normals per world.
template <class P> constexpr int noised_inputs() {
  int c = 0;
  for (int i = 0; i < P::NI; i++) c += P::noise[i] != 0.0 ? 1 : 0;
  return c;
}

template <class P, class T> __device__ __forceinline__ void policy_wave(const PolicyArgs& a, float* lds) {
  constexpr int NI = P::NI, NO = P::NO, CB = P::CB, NHB = P::NHB, NOB = P::NOB, KU = P::KU, NPD = P::NPD;
  constexpr int WPW = 16 * CB;     // worlds per wave
  constexpr int XS = 16 * KU + 1;  // LDS row stride of the input tile (floats)
  constexpr int MS = 16 * NOB + 1; // LDS row stride of the output tile
  const int lane = threadIdx.x & 63;
  const int w0 = blockIdx.x * WPW;
  const int S = a.stride;
  const int my = w0 + lane;
  const bool own = lane < WPW && my < a.nworld;
  u64 rs = 0;

  // Prologue: world w0 + lane reads its observation row, adds input noise in
  // index order (the noised value is what the history keeps), stages x in LDS.
  if constexpr (WPW == 32) {
    // Half the lanes own a world: the normals' transforms are paired across
    // the wave's halves (policy_normals_paired).
    constexpr int NN = noised_inputs<P>();
    if (own) rs = a.rng[my];
    float x[16 * KU];
#pragma unroll
    for (int i = 0; i < 16 * KU; i++) x[i] = (i < NI && own) ? a.obs[(size_t)i * S + my] : 0.0f;
    if constexpr (NN > 0) {
      double nz[NN];
      policy_normals_paired<NN>(rs, lane, nz);
      int c = 0;
#pragma unroll
      for (int i = 0; i < NI; i++)
        if (P::noise[i] != 0.0) {
          x[i] += float(P::noise[i]) * (float)nz[c++];
          if (own) a.obs[(size_t)i * S + my] = x[i];
        }
    }
    if (lane < WPW) {
#pragma unroll
      for (int i = 0; i < 16 * KU; i++) lds[lane * XS + i] = x[i];
    }
  } else if (lane < WPW) {
    if (own) rs = a.rng[my];
#pragma unroll
    for (int i = 0; i < 16 * KU; i++) {
      float x = 0.0f;
      if (i < NI && own) {
        x = a.obs[(size_t)i * S + my];
        if (P::noise[i] != 0.0) {
          x += float(P::noise[i]) * (float)policy_normal(rs);
          a.obs[(size_t)i * S + my] = x;
        }
      }
      lds[lane * XS + i] = x;
    }
  }
  __syncthreads();

  const int r = lane & 15, g = lane >> 4;
  // Layer 1: B = the input tile in LDS; k-step s of input group u is inputs
  // 16 u + 4 s + g in lane group g.
  f32x4 h[NHB][CB];
  bias_tiles<NHB, CB>(a.bias, g, h);
  mfma_layer<KU, NHB, CB>(a.w1, lane, h, [&](int kb, int s, int cb) { return lds[(cb * 16 + r) * XS + 16 * kb + 4 * s + g]; });
  tanh_tiles<NHB, CB>(h);
  // Layer 2: B = layer 1's output tiles, straight from registers.
  f32x4 h2[NHB][CB];
  bias_tiles<NHB, CB>(a.bias + 16 * NHB, g, h2);
  mfma_layer<NHB, NHB, CB>(a.w2, lane, h2, [&](int kb, int s, int cb) { return h[kb][cb][s]; });
  tanh_tiles<NHB, CB>(h2);
  // Layer 3: the action means.
  f32x4 m[NOB][CB];
  bias_tiles<NOB, CB>(a.bias + 32 * NHB, g, m);
  mfma_layer<NHB, NOB, CB>(a.w3, lane, m, [&](int kb, int s, int cb) { return h2[kb][cb][s]; });
  // Means to LDS, world-major, for the per-world epilogue.
  __syncthreads();
#pragma unroll
  for (int ob = 0; ob < NOB; ob++)
#pragma unroll
    for (int cb = 0; cb < CB; cb++)
#pragma unroll
      for (int j = 0; j < 4; j++) lds[(cb * 16 + r) * MS + ob * 16 + 4 * g + j] = m[ob][cb][j];
  __syncthreads();

  // Epilogue (policy_reference, policy_pipeline.rs:488-520): every servo gets
  // its base target, then each action k: AR(1) noise, sample, log-prob, the
  // clamped action onto its slot's base. With half the lanes owning a world
  // the actions' normals are drawn first, paired across the halves.
  double na[NO];
  if constexpr (WPW == 32) policy_normals_paired<NO>(rs, lane, na);
  if (own) {
    const T* base = (const T*)a.base;
    T* tgt = (T*)a.targets;
#pragma unroll
    for (int j = 0; j < NPD; j++) tgt[(size_t)j * S + my] = base[(size_t)j * S + my];
    const float rho = float(P::rho);
    const float keep = sqrtf(fmaxf(0.0f, 1.0f - rho * rho));
    const float half_ln_2pi = 0.91893853320467274178f;
    float logp = 0.0f;
#pragma unroll
    for (int k = 0; k < NO; k++) {
      const float mk = lds[lane * MS + k];
      const float zk = rho * a.z[(size_t)k * S + my] + keep * (float)(WPW == 32 ? na[k] : policy_normal(rs));
      a.z[(size_t)k * S + my] = zk;
      const float sd = a.stdv[k];
      const float act = mk + sd * zk;
      const float zi = (act - mk) / sd;
      logp += -0.5f * zi * zi - logf(sd) - half_ln_2pi;
      a.out[(size_t)k * S + my] = act;
      const float lim = float(P::clamp[k]);
      // clamp(-lim, lim) that passes NaN through, as f64::clamp does.
      const float applied = act < -lim ? -lim : (act > lim ? lim : act);
      const int slot = P::slot[k];
      tgt[(size_t)slot * S + my] = base[(size_t)slot * S + my] + T(applied);
    }
    a.out[(size_t)NO * S + my] = logp;
    a.rng[my] = rs;
  }
}

}  // namespace phz
