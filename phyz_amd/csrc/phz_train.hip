// phz_train.hip — the PPO update pass on gfx950 (kernels and their C ABI).
//
// The update half of a reinforcement-learning iteration, as the reference's
// TrainPipeline runs it (crates/phyz-gpu/src/cuda/train.rs:523-791, kernels
// crates/phyz-gpu/cuda/phyz_train.cu:95-362): epochs x minibatches of a
// clipped-surrogate PPO step over a three-layer tanh MLP actor with a global
// learned log_std and a three-layer tanh MLP critic, Adam on both (f64 master
// weights and moments, f32 mirror for the forward pass), and a per-minibatch
// KL brake.
//
// Layout of the work on the device (one stream, no host round trip inside an
// update):
//   ppo_tiles  grid (tiles, 2): one workgroup per tile of R minibatch rows and
//              per network (y = 0 actor, 1 critic). The tile's rows are
//              gathered into LDS, and forward, loss gradient and backward all
//              run out of LDS. Each workgroup writes its tile's partial weight
//              and bias gradients in f64 (part[tile][param]) and its partial
//              statistics (stats_part[tile][4]).
//   ppo_adam   one thread per parameter of both networks: the tile partials
//              summed in tile order in f64, rounded to f32 (the gradient the
//              reference hands Adam is f32), then Adam in f64. Writes the f64
//              master, the row-major f32 mirror (backward) and a transposed
//              f32 mirror of each weight matrix (forward: lanes over output
//              neurons read consecutive words).
//   ppo_brake  one thread: the minibatch's statistics into the update's
//              running sums, and the KL brake. When it trips, it sets a flag
//              that every later launch of the update checks first, so the
//              loop stops after that minibatch exactly as the reference's
//              host loop does, without the reference's per-minibatch readback.
// Every sum has a fixed order (rows within a tile, then tiles ascending), so
// an update is bit-reproducible run to run.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "../../include/phyz_amd.h"

namespace {

constexpr int kThreads = 256;   // threads per workgroup of every training launch
constexpr int kRowBlock = 8;    // rows a thread carries through one dense-layer item
constexpr uint32_t kMaxHidden = 256;  // TRAIN_MAX_H (train.rs:46)
constexpr uint32_t kMaxOut = 64;      // TRAIN_MAX_OUT (train.rs:50)

// ── parameter layout: tang's Mlp::to_flat order (phyz_train.cu:62-93) ───────
struct Dims {
  uint32_t n_in, n_h, n_out;
  __host__ __device__ uint32_t oW1() const { return 0; }
  __host__ __device__ uint32_t ob1() const { return n_h * n_in; }
  __host__ __device__ uint32_t oW2() const { return ob1() + n_h; }
  __host__ __device__ uint32_t ob2() const { return oW2() + n_h * n_h; }
  __host__ __device__ uint32_t oW3() const { return ob2() + n_h; }
  __host__ __device__ uint32_t ob3() const { return oW3() + n_out * n_h; }
  __host__ __device__ uint32_t mlp_params() const { return ob3() + n_out; }
  // Transposed mirror: W1t [n_in][n_h], W2t [n_h][n_h], W3t [n_h][n_out].
  __host__ __device__ uint32_t tW2() const { return n_h * n_in; }
  __host__ __device__ uint32_t tW3() const { return tW2() + n_h * n_h; }
  __host__ __device__ uint32_t t_size() const { return tW3() + n_h * n_out; }
};

// LDS of one tile workgroup, in floats: X [R][n_in], H1 [R][n_h], H2 [R][n_h],
// DA [R][n_h], DB [R][n_h], OUT [R][n_out] (the output, then dL/dout),
// DLS [R][n_out] (per-row dL/dlog_std), RS [R][4] (per-row statistics),
// SD [n_out], LSD [n_out].
struct Lds {
  uint32_t X, H1, H2, DA, DB, OUT, DLS, RS, SD, LSD, total;
  __host__ __device__ Lds(const Dims& d, uint32_t R) {
    X = 0;
    H1 = X + R * d.n_in;
    H2 = H1 + R * d.n_h;
    DA = H2 + R * d.n_h;
    DB = DA + R * d.n_h;
    OUT = DB + R * d.n_h;
    DLS = OUT + R * d.n_out;
    RS = DLS + R * d.n_out;
    SD = RS + R * 4;
    LSD = SD + d.n_out;
    total = LSD + d.n_out;
  }
};

struct TileArgs {
  const float* x[2];      // obs_a [n_rows][n_in], obs_c [n_rows][n_in]
  const float* w[2];      // row-major f32 mirrors
  const float* wt[2];     // transposed f32 mirrors of the weight matrices
  double* part[2];        // [tile][n_param] f64 partial gradients
  Dims dims[2];
  uint32_t n_param[2];
  const uint32_t* idx;    // this minibatch's sample indices
  uint32_t b;             // rows in this minibatch
  uint32_t R;             // rows per tile
  const float* act;       // [n_rows][actor n_out]
  const float* logp_old;  // [n_rows]
  const float* adv;       // [n_rows]
  const float* ret;       // [n_rows]
  float clip, entropy_coef, vdelta;
  double* stats_part;     // [tile][4]
  const int* stopped;     // the update's KL-brake flag
};

// tanh rounded once to f32 from an f64 evaluation. Near saturation the
// backward pass uses 1 - h^2, whose relative error is the activation's error
// over (1 - |h|): a few-ulp f32 tanh there visibly perturbs the gradients of
// the layer above, which a correctly rounded activation does not.
__device__ inline float act_tanh(float x) { return (float)tanh((double)x); }

// Y[r][j] = act(b[j] + sum_i Wt[i][j] X[r][i]) for rows r < R, neurons j < N.
// Lanes run over neurons (coalesced Wt reads, LDS broadcasts of X); each item
// carries kRowBlock rows. The sum starts from the bias and adds inputs in
// order, as the reference's per-row loop does (phyz_train.cu:115-132).
template <bool TANH>
__device__ void dense_forward(const float* __restrict__ X, uint32_t K, const float* __restrict__ Wt,
                              const float* __restrict__ bias, uint32_t N, float* __restrict__ Y, uint32_t R) {
  const uint32_t NP = (N + 63u) & ~63u;
  const uint32_t items = (R / kRowBlock) * NP;
  for (uint32_t it = threadIdx.x; it < items; it += kThreads) {
    const uint32_t j = it % NP, r0 = (it / NP) * kRowBlock;
    if (j >= N) continue;
    float acc[kRowBlock];
    const float bj = bias[j];
#pragma unroll
    for (int rr = 0; rr < kRowBlock; rr++) acc[rr] = bj;
    for (uint32_t i = 0; i < K; i++) {
      const float wij = Wt[i * N + j];
#pragma unroll
      for (int rr = 0; rr < kRowBlock; rr++) acc[rr] += wij * X[(r0 + rr) * K + i];
    }
#pragma unroll
    for (int rr = 0; rr < kRowBlock; rr++) Y[(r0 + rr) * N + j] = TANH ? act_tanh(acc[rr]) : acc[rr];
  }
}

// dH[r][j] = (sum_k D[r][k] W[k][j]) (1 - H[r][j]^2), W row-major [K][N]
// (phyz_train.cu:212-222).
__device__ void dense_backward_hidden(const float* __restrict__ D, uint32_t K, const float* __restrict__ W,
                                      const float* __restrict__ H, uint32_t N, float* __restrict__ DH, uint32_t R) {
  const uint32_t NP = (N + 63u) & ~63u;
  const uint32_t items = (R / kRowBlock) * NP;
  for (uint32_t it = threadIdx.x; it < items; it += kThreads) {
    const uint32_t j = it % NP, r0 = (it / NP) * kRowBlock;
    if (j >= N) continue;
    float acc[kRowBlock];
#pragma unroll
    for (int rr = 0; rr < kRowBlock; rr++) acc[rr] = 0.0f;
    for (uint32_t k = 0; k < K; k++) {
      const float wkj = W[k * N + j];
#pragma unroll
      for (int rr = 0; rr < kRowBlock; rr++) acc[rr] += D[(r0 + rr) * K + k] * wkj;
    }
#pragma unroll
    for (int rr = 0; rr < kRowBlock; rr++) {
      const float a = H[(r0 + rr) * N + j];
      DH[(r0 + rr) * N + j] = acc[rr] * (1.0f - a * a);
    }
  }
}

// Tile partials of a linear layer's gradients: Gw[o][i] = sum_r D[r][o] X[r][i]
// and Gb[o] = sum_r D[r][o] over the tile's valid rows, in f64 (the
// reference's row loops accumulate in double, phyz_train.cu:226-260).
__device__ void dense_grad(const float* __restrict__ D, uint32_t O, const float* __restrict__ X, uint32_t I,
                           uint32_t rows, double* __restrict__ Gw, double* __restrict__ Gb) {
  for (uint32_t it = threadIdx.x; it < O * I; it += kThreads) {
    const uint32_t o = it / I, i = it % I;
    double acc = 0.0;
    for (uint32_t r = 0; r < rows; r++) acc += (double)D[r * O + o] * (double)X[r * I + i];
    Gw[it] = acc;
  }
  for (uint32_t o = threadIdx.x; o < O; o += kThreads) {
    double acc = 0.0;
    for (uint32_t r = 0; r < rows; r++) acc += (double)D[r * O + o];
    Gb[o] = acc;
  }
}

__device__ inline float clampf(float x, float lo, float hi) { return x < lo ? lo : (x > hi ? hi : x); }

__global__ void __launch_bounds__(kThreads) ppo_tiles(TileArgs a) {
  if (*a.stopped) return;
  extern __shared__ float lds[];
  const int net = blockIdx.y;
  const Dims d = a.dims[net];
  const uint32_t R = a.R;
  const uint32_t row0 = blockIdx.x * R;
  const uint32_t rows = row0 >= a.b ? 0u : std::min(R, a.b - row0);
  const Lds L(d, R);
  float* X = lds + L.X;
  float* H1 = lds + L.H1;
  float* H2 = lds + L.H2;
  float* DA = lds + L.DA;
  float* DB = lds + L.DB;
  float* OUT = lds + L.OUT;
  float* DLS = lds + L.DLS;
  float* RS = lds + L.RS;
  float* SD = lds + L.SD;
  float* LSD = lds + L.LSD;
  const float* w = a.w[net];
  const float* wt = a.wt[net];
  double* part = a.part[net] + (size_t)blockIdx.x * a.n_param[net];
  const float* x = a.x[net];

  // ── gather the tile's rows (the minibatch is an index list into the batch) ──
  for (uint32_t e = threadIdx.x; e < R * d.n_in; e += kThreads) {
    const uint32_t r = e / d.n_in, i = e % d.n_in;
    X[e] = r < rows ? x[(size_t)a.idx[row0 + r] * d.n_in + i] : 0.0f;
  }
  if (net == 0) {
    for (uint32_t k = threadIdx.x; k < d.n_out; k += kThreads) {
      const float s = expf(w[d.mlp_params() + k]);
      SD[k] = s;
      LSD[k] = logf(s);
    }
  }
  __syncthreads();

  // ── forward (phyz_train.cu:101-133) ──
  dense_forward<true>(X, d.n_in, wt, w + d.ob1(), d.n_h, H1, R);
  __syncthreads();
  dense_forward<true>(H1, d.n_h, wt + d.tW2(), w + d.ob2(), d.n_h, H2, R);
  __syncthreads();
  dense_forward<false>(H2, d.n_h, wt + d.tW3(), w + d.ob3(), d.n_out, OUT, R);
  __syncthreads();

  // ── loss gradient per row; OUT becomes dL/dout ──
  const float fb = (float)a.b;
  if (net == 0) {
    // Clipped surrogate with the gradient through the active branch only and
    // the entropy bonus folded into dlog_std (phyz_train.cu:150-196).
    const float LN_2PI = 1.8378770664093453f;
    for (uint32_t r = threadIdx.x; r < R; r += kThreads) {
      float* o = OUT + r * d.n_out;
      float* dls = DLS + r * d.n_out;
      if (r >= rows) {
        for (uint32_t k = 0; k < d.n_out; k++) { o[k] = 0.0f; dls[k] = 0.0f; }
        RS[r * 4 + 0] = RS[r * 4 + 1] = RS[r * 4 + 2] = 0.0f;
        continue;
      }
      const uint32_t s = a.idx[row0 + r];
      const float* act = a.act + (size_t)s * d.n_out;
      float logp = 0.0f;
      for (uint32_t k = 0; k < d.n_out; k++) {
        const float z = (act[k] - o[k]) / SD[k];
        logp += -0.5f * z * z - LSD[k] - 0.5f * LN_2PI;
      }
      const float adv = a.adv[s];
      const float log_ratio = logp - a.logp_old[s];
      const float ratio = expf(log_ratio);
      const float clipped = clampf(ratio, 1.0f - a.clip, 1.0f + a.clip);
      const float uo = ratio * adv, co = clipped * adv;
      RS[r * 4 + 0] = -(uo < co ? uo : co);
      RS[r * 4 + 1] = a.logp_old[s] - logp;
      RS[r * 4 + 2] = ratio - 1.0f - log_ratio;
      const bool active = uo <= co + 1e-12f;
      const float coef = -adv * ratio / fb;
      for (uint32_t k = 0; k < d.n_out; k++) {
        if (!active) {
          o[k] = 0.0f;
          dls[k] = -a.entropy_coef / fb;
        } else {
          const float z = (act[k] - o[k]) / SD[k];
          o[k] = coef * (z / SD[k]);
          dls[k] = coef * (z * z - 1.0f) - a.entropy_coef / fb;
        }
      }
    }
  } else {
    // Squared error to the return with the gradient Huber-clipped at vdelta;
    // the statistic stays the plain squared error (phyz_train.cu:198-208).
    for (uint32_t r = threadIdx.x; r < R; r += kThreads) {
      if (r >= rows) {
        OUT[r] = 0.0f;
        RS[r * 4 + 3] = 0.0f;
        continue;
      }
      const float err = OUT[r] - a.ret[a.idx[row0 + r]];
      RS[r * 4 + 3] = err * err;
      OUT[r] = 2.0f * clampf(err, -a.vdelta, a.vdelta) / fb;
    }
  }
  __syncthreads();

  // ── layer 3 gradients, tile statistics, dL/dh2 ──
  dense_grad(OUT, d.n_out, H2, d.n_h, rows, part + d.oW3(), part + d.ob3());
  if (net == 0) {
    for (uint32_t k = threadIdx.x; k < d.n_out; k += kThreads) {
      double acc = 0.0;
      for (uint32_t r = 0; r < rows; r++) acc += (double)DLS[r * d.n_out + k];
      part[d.mlp_params() + k] = acc;
    }
  }
  if (threadIdx.x < 4 && (net == 0) == (threadIdx.x < 3)) {
    double acc = 0.0;
    for (uint32_t r = 0; r < rows; r++) acc += (double)RS[r * 4 + threadIdx.x];
    a.stats_part[(size_t)blockIdx.x * 4 + threadIdx.x] = acc;
  }
  dense_backward_hidden(OUT, d.n_out, w + d.oW3(), H2, d.n_h, DA, R);
  __syncthreads();

  // ── layer 2 gradients, dL/dh1 ──
  dense_grad(DA, d.n_h, H1, d.n_h, rows, part + d.oW2(), part + d.ob2());
  dense_backward_hidden(DA, d.n_h, w + d.oW2(), H1, d.n_h, DB, R);
  __syncthreads();

  // ── layer 1 gradients (input: the gathered rows) ──
  dense_grad(DB, d.n_h, X, d.n_in, rows, part + d.oW1(), part + d.ob1());
}

struct AdamArgs {
  const double* part[2];
  double* p[2];
  double* m[2];
  double* v[2];
  float* w[2];
  float* wt[2];
  Dims dims[2];
  uint32_t n_param[2];
  uint32_t tiles;
  double lr[2], beta1[2], beta2[2], eps[2], wd[2], bc1[2], bc2[2];
  const int* stopped;
};

// tang's ModuleAdam step, elementwise (phyz_train.cu:268-288), on the sum of
// the tile partials.
__global__ void __launch_bounds__(kThreads) ppo_adam(AdamArgs a) {
  if (*a.stopped) return;
  const uint32_t t = blockIdx.x * kThreads + threadIdx.x;
  if (t >= a.n_param[0] + a.n_param[1]) return;
  const int net = t < a.n_param[0] ? 0 : 1;
  const uint32_t q = net == 0 ? t : t - a.n_param[0];
  const uint32_t np = a.n_param[net];
  const double* part = a.part[net];
  double g = 0.0;
  for (uint32_t k = 0; k < a.tiles; k++) g += part[(size_t)k * np + q];
  const double gr = (double)(float)g;
  double x = a.p[net][q];
  const double lr = a.lr[net];
  if (a.wd[net] > 0.0) x = x * (1.0 - lr * a.wd[net]);
  const double b1 = a.beta1[net], b2 = a.beta2[net];
  const double mt = b1 * a.m[net][q] + (1.0 - b1) * gr;
  const double vt = b2 * a.v[net][q] + (1.0 - b2) * gr * gr;
  a.m[net][q] = mt;
  a.v[net][q] = vt;
  const double m_hat = mt / a.bc1[net];
  const double v_hat = vt / a.bc2[net];
  x -= lr * m_hat / (sqrt(v_hat) + a.eps[net]);
  a.p[net][q] = x;
  const float xf = (float)x;
  a.w[net][q] = xf;
  const Dims d = a.dims[net];
  if (q < d.ob1()) {
    const uint32_t j = q / d.n_in, i = q % d.n_in;
    a.wt[net][i * d.n_h + j] = xf;
  } else if (q >= d.oW2() && q < d.ob2()) {
    const uint32_t e = q - d.oW2(), j = e / d.n_h, i = e % d.n_h;
    a.wt[net][d.tW2() + i * d.n_h + j] = xf;
  } else if (q >= d.oW3() && q < d.ob3()) {
    const uint32_t e = q - d.oW3(), k = e / d.n_h, i = e % d.n_h;
    a.wt[net][d.tW3() + i * d.n_out + k] = xf;
  }
}

// The update's running sums on the device (train.rs:620-627).
struct UpdateState {
  double policy_acc, value_acc, brake_acc, kl_acc;
  uint64_t kl_rows, batches;
  int stopped;
  int pad;
};

struct BrakeArgs {
  const double* stats_part;
  uint32_t tiles;
  uint32_t b;
  int kl_mode;  // PHZ_KL_CUMULATIVE / PHZ_KL_MINIBATCH
  double kl_scale, target_kl;
  UpdateState* st;
};

// The four statistic columns reduced (rounded to f32, as the reference's
// reduce_stats output is), then the brake (train.rs:757-777).
__global__ void ppo_brake(BrakeArgs a) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  UpdateState* st = a.st;
  if (st->stopped) return;
  double s[4] = {0.0, 0.0, 0.0, 0.0};
  for (uint32_t k = 0; k < a.tiles; k++)
    for (int c = 0; c < 4; c++) s[c] += a.stats_part[(size_t)k * 4 + c];
  const double ploss = (double)(float)s[0], kl_sum = (double)(float)s[1];
  const double k3_sum = (double)(float)s[2], vloss = (double)(float)s[3];
  const double b = (double)a.b;
  st->policy_acc += ploss / b;
  st->value_acc += vloss / b;
  st->kl_acc += kl_sum;
  st->kl_rows += a.b;
  const double rows = (double)(st->kl_rows > 0 ? st->kl_rows : 1);
  const double brake = (a.kl_mode == PHZ_KL_CUMULATIVE ? fabs(st->kl_acc / rows) : k3_sum / b) / a.kl_scale;
  st->brake_acc += brake;
  st->batches += 1;
  if (brake > a.target_kl) st->stopped = 1;
}

// ── host side ───────────────────────────────────────────────────────────────
std::string fmt(const char* f, ...) __attribute__((format(printf, 1, 2)));
std::string fmt(const char* f, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, f);
  vsnprintf(buf, sizeof buf, f, ap);
  va_end(ap);
  return buf;
}

thread_local std::string g_train_create_error;

// beta^t by binary exponentiation (t >= 1).
double powi(double beta, uint64_t t) {
  double r = 1.0;
  while (t) {
    if (t & 1) r *= beta;
    t >>= 1;
    if (t) beta *= beta;
  }
  return r;
}

Dims to_dims(const phz_net_dims& d) { return Dims{(uint32_t)d.n_in, (uint32_t)d.n_h, (uint32_t)d.n_out}; }

}  // namespace

struct phz_train {
  int device = 0;
  std::string err;
  hipStream_t stream = nullptr;
  Dims dims[2];
  uint32_t n_param[2];   // the actor's includes log_std
  uint64_t capacity = 0, max_b = 0, n_rows = 0;
  uint32_t R = 0, max_tiles = 0;
  size_t lds_bytes = 0;
  phz_adam_cfg adam[2];
  uint64_t t[2] = {0, 0};
  // device buffers
  float* w[2] = {nullptr, nullptr};
  float* wt[2] = {nullptr, nullptr};
  double* p[2] = {nullptr, nullptr};
  double* m[2] = {nullptr, nullptr};
  double* v[2] = {nullptr, nullptr};
  double* part[2] = {nullptr, nullptr};
  float* obs[2] = {nullptr, nullptr};
  float* act = nullptr;
  float* logp_old = nullptr;
  float* adv = nullptr;
  float* ret = nullptr;
  double* stats_part = nullptr;
  UpdateState* state = nullptr;
  uint32_t* order = nullptr;
  uint64_t order_cap = 0;
  std::vector<void*> allocs;

  int fail(const std::string& e) { err = e; return 1; }
  bool hip_ok(hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    err = fmt("%s: %s", what, hipGetErrorString(e));
    return false;
  }
  template <class T> bool alloc(T** ptr, size_t count, const char* what) {
    void* q = nullptr;
    if (!hip_ok(hipMalloc(&q, std::max<size_t>(count, 1) * sizeof(T)), what)) return false;
    allocs.push_back(q);
    if (!hip_ok(hipMemsetAsync(q, 0, std::max<size_t>(count, 1) * sizeof(T), stream), what)) return false;
    *ptr = (T*)q;
    return true;
  }
  ~phz_train() {
    if (stream) hipStreamSynchronize(stream);
    for (void* q : allocs) hipFree(q);
    if (order) hipFree(order);
    if (stream) hipStreamDestroy(stream);
  }
};

namespace {

bool set_device(phz_train* t) { return t->hip_ok(hipSetDevice(t->device), "hipSetDevice"); }

// Rows per tile: the most (64, 32, 16 or 8) whose LDS fits 64 KiB, else the
// most that fits the device's per-workgroup LDS.
bool choose_tile(phz_train* t, size_t lds_limit, std::string& e) {
  auto bytes = [&](uint32_t R) {
    size_t worst = 0;
    for (int n = 0; n < 2; n++) worst = std::max<size_t>(worst, Lds(t->dims[n], R).total);
    return worst * sizeof(float);
  };
  for (size_t limit : {size_t(65536), lds_limit}) {
    for (uint32_t R : {64u, 32u, 16u, 8u}) {
      if (bytes(R) <= limit) {
        t->R = R;
        t->lds_bytes = bytes(R);
        return true;
      }
    }
  }
  e = fmt("networks too wide for one tile: 8 rows need %zu bytes of LDS, the device has %zu", bytes(8), lds_limit);
  return false;
}

bool upload_params(phz_train* t, int net, const double* flat) {
  const Dims& d = t->dims[net];
  const uint32_t np = t->n_param[net];
  std::vector<float> mirror(np), tr(d.t_size());
  for (uint32_t q = 0; q < np; q++) mirror[q] = (float)flat[q];
  for (uint32_t j = 0; j < d.n_h; j++)
    for (uint32_t i = 0; i < d.n_in; i++) tr[i * d.n_h + j] = mirror[d.oW1() + j * d.n_in + i];
  for (uint32_t j = 0; j < d.n_h; j++)
    for (uint32_t i = 0; i < d.n_h; i++) tr[d.tW2() + i * d.n_h + j] = mirror[d.oW2() + j * d.n_h + i];
  for (uint32_t k = 0; k < d.n_out; k++)
    for (uint32_t i = 0; i < d.n_h; i++) tr[d.tW3() + i * d.n_out + k] = mirror[d.oW3() + k * d.n_h + i];
  return t->hip_ok(hipMemcpyAsync(t->p[net], flat, np * sizeof(double), hipMemcpyHostToDevice, t->stream), "upload params") &&
         t->hip_ok(hipMemcpyAsync(t->w[net], mirror.data(), np * sizeof(float), hipMemcpyHostToDevice, t->stream), "upload params") &&
         t->hip_ok(hipMemcpyAsync(t->wt[net], tr.data(), tr.size() * sizeof(float), hipMemcpyHostToDevice, t->stream), "upload params") &&
         t->hip_ok(hipStreamSynchronize(t->stream), "upload params");
}

int set_params(phz_train* t, int net, const double* flat, uint64_t n) {
  if (!t) return 1;
  t->err.clear();
  if (n != t->n_param[net])
    return t->fail(fmt("parameter array is %llu long, network wants %u", (unsigned long long)n, t->n_param[net]));
  if (!flat) return t->fail("null parameter array");
  if (!set_device(t)) return 1;
  return upload_params(t, net, flat) ? 0 : 1;
}

int get_params(phz_train* t, int net, double* out, uint64_t n) {
  if (!t) return 1;
  t->err.clear();
  if (n != t->n_param[net])
    return t->fail(fmt("output array is %llu long, network has %u parameters", (unsigned long long)n, t->n_param[net]));
  if (!out) return t->fail("null output array");
  if (!set_device(t)) return 1;
  return t->hip_ok(hipMemcpyAsync(out, t->p[net], n * sizeof(double), hipMemcpyDeviceToHost, t->stream), "read params") &&
                 t->hip_ok(hipStreamSynchronize(t->stream), "read params")
             ? 0
             : 1;
}

}  // namespace

extern "C" {

int phz_train_create(phz_net_dims actor, phz_net_dims critic, uint64_t capacity, uint64_t max_b, int device_ordinal,
                     phz_train** out) {
  g_train_create_error.clear();
  if (!out) { g_train_create_error = "null output pointer"; return 1; }
  *out = nullptr;
  const char* what[2] = {"actor", "critic"};
  const phz_net_dims nd[2] = {actor, critic};
  for (int n = 0; n < 2; n++) {
    if (nd[n].n_h > kMaxHidden) {
      g_train_create_error = fmt("%s hidden width %llu exceeds TRAIN_MAX_H %u", what[n], (unsigned long long)nd[n].n_h, kMaxHidden);
      return 1;
    }
    if (nd[n].n_out > kMaxOut) {
      g_train_create_error = fmt("%s output width %llu exceeds TRAIN_MAX_OUT %u", what[n], (unsigned long long)nd[n].n_out, kMaxOut);
      return 1;
    }
    if (nd[n].n_in == 0 || nd[n].n_h == 0 || nd[n].n_out == 0) {
      g_train_create_error = fmt("%s has a zero-width layer", what[n]);
      return 1;
    }
    if (nd[n].n_in > (1u << 16)) {
      g_train_create_error = fmt("%s input width %llu is too large", what[n], (unsigned long long)nd[n].n_in);
      return 1;
    }
  }
  if (critic.n_out != 1) {
    g_train_create_error = fmt("critic must have one output, got %llu", (unsigned long long)critic.n_out);
    return 1;
  }
  if (max_b == 0 || max_b > (1u << 24)) { g_train_create_error = "max_b must be in 1..2^24"; return 1; }
  if (capacity > (1ull << 32) - 1) { g_train_create_error = "capacity must fit 32-bit sample indices"; return 1; }
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count == 0) { g_train_create_error = "no HIP device available"; return 1; }
  if (device_ordinal < 0 || device_ordinal >= count) {
    g_train_create_error = fmt("device ordinal %d out of range (%d devices)", device_ordinal, count);
    return 1;
  }
  auto* t = new phz_train();
  t->device = device_ordinal;
  t->capacity = capacity;
  t->max_b = max_b;
  t->dims[0] = to_dims(actor);
  t->dims[1] = to_dims(critic);
  t->n_param[0] = t->dims[0].mlp_params() + t->dims[0].n_out;
  t->n_param[1] = t->dims[1].mlp_params();
  for (int n = 0; n < 2; n++) t->adam[n] = phz_adam_cfg{3e-4, 0.9, 0.999, 1e-8, 0.0};
  auto bail = [&](const std::string& e) {
    g_train_create_error = e;
    delete t;
    return 1;
  };
  if (!set_device(t) || !t->hip_ok(hipStreamCreateWithFlags(&t->stream, hipStreamNonBlocking), "hipStreamCreate"))
    return bail(t->err);
  int lds_limit = 0;
  if (!t->hip_ok(hipDeviceGetAttribute(&lds_limit, hipDeviceAttributeMaxSharedMemoryPerBlock, device_ordinal), "LDS limit"))
    return bail(t->err);
  std::string e;
  if (!choose_tile(t, (size_t)lds_limit, e)) return bail(e);
  if (t->lds_bytes > 65536 &&
      !t->hip_ok(hipFuncSetAttribute((const void*)ppo_tiles, hipFuncAttributeMaxDynamicSharedMemorySize, (int)t->lds_bytes),
                 "LDS attribute"))
    return bail(t->err);
  t->max_tiles = (uint32_t)((max_b + t->R - 1) / t->R);
  bool ok = true;
  for (int n = 0; n < 2 && ok; n++) {
    const uint32_t np = t->n_param[n];
    ok = t->alloc(&t->w[n], np, "alloc weights") && t->alloc(&t->wt[n], t->dims[n].t_size(), "alloc weights") &&
         t->alloc(&t->p[n], np, "alloc master weights") && t->alloc(&t->m[n], np, "alloc Adam moments") &&
         t->alloc(&t->v[n], np, "alloc Adam moments") &&
         t->alloc(&t->part[n], (size_t)t->max_tiles * np, "alloc gradient partials") &&
         t->alloc(&t->obs[n], capacity * t->dims[n].n_in, "alloc batch");
  }
  ok = ok && t->alloc(&t->act, capacity * actor.n_out, "alloc batch") && t->alloc(&t->logp_old, capacity, "alloc batch") &&
       t->alloc(&t->adv, capacity, "alloc batch") && t->alloc(&t->ret, capacity, "alloc batch") &&
       t->alloc(&t->stats_part, (size_t)t->max_tiles * 4, "alloc statistics") &&
       t->alloc(&t->state, 1, "alloc update state") && t->hip_ok(hipStreamSynchronize(t->stream), "create");
  if (!ok) return bail(t->err);
  *out = t;
  return 0;
}

void phz_train_destroy(phz_train* t) {
  if (!t) return;
  hipSetDevice(t->device);
  delete t;
}

const char* phz_train_last_error(const phz_train* t) { return t ? t->err.c_str() : g_train_create_error.c_str(); }

int phz_train_device_name(const phz_train* t, char* buf, uint64_t len) {
  if (!t || !buf || len == 0) return 1;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, t->device) != hipSuccess) return 1;
  snprintf(buf, (size_t)len, "%s (%s)", prop.name, prop.gcnArchName);
  return 0;
}

uint64_t phz_train_param_count(const phz_train* t, int net) { return t && (net == 0 || net == 1) ? t->n_param[net] : 0; }

uint32_t phz_train_rows_per_tile(const phz_train* t) { return t ? t->R : 0; }

int phz_train_set_adam(phz_train* t, const phz_adam_cfg* actor, const phz_adam_cfg* critic) {
  if (!t) return 1;
  t->err.clear();
  if (!actor || !critic) return t->fail("null Adam configuration");
  t->adam[0] = *actor;
  t->adam[1] = *critic;
  return 0;
}

int phz_train_set_actor_params(phz_train* t, const double* flat, uint64_t n) { return set_params(t, 0, flat, n); }
int phz_train_set_critic_params(phz_train* t, const double* flat, uint64_t n) { return set_params(t, 1, flat, n); }
int phz_train_actor_params(phz_train* t, double* out, uint64_t n) { return get_params(t, 0, out, n); }
int phz_train_critic_params(phz_train* t, double* out, uint64_t n) { return get_params(t, 1, out, n); }

int phz_train_upload_batch(phz_train* t, uint64_t n_rows, const float* obs_a, uint64_t obs_a_len, const float* obs_c,
                           uint64_t obs_c_len, const float* act, uint64_t act_len, const float* logp_old,
                           uint64_t logp_old_len, const float* adv, uint64_t adv_len, const float* ret, uint64_t ret_len) {
  if (!t) return 1;
  t->err.clear();
  if (n_rows > t->capacity)
    return t->fail(fmt("%llu samples into a pipeline built for %llu", (unsigned long long)n_rows,
                       (unsigned long long)t->capacity));
  struct Col { const char* name; const float* src; uint64_t got, want; void* dst; } cols[6] = {
      {"obs_a", obs_a, obs_a_len, n_rows * t->dims[0].n_in, t->obs[0]},
      {"obs_c", obs_c, obs_c_len, n_rows * t->dims[1].n_in, t->obs[1]},
      {"act", act, act_len, n_rows * t->dims[0].n_out, t->act},
      {"logp_old", logp_old, logp_old_len, n_rows, t->logp_old},
      {"adv", adv, adv_len, n_rows, t->adv},
      {"ret", ret, ret_len, n_rows, t->ret}};
  for (const Col& c : cols) {
    if (c.got != c.want)
      return t->fail(fmt("%s is %llu long, expected %llu", c.name, (unsigned long long)c.got, (unsigned long long)c.want));
    if (c.want && !c.src) return t->fail(fmt("null %s", c.name));
  }
  if (!set_device(t)) return 1;
  for (const Col& c : cols)
    if (c.want && !t->hip_ok(hipMemcpyAsync(c.dst, c.src, c.want * sizeof(float), hipMemcpyHostToDevice, t->stream),
                             "upload batch"))
      return 1;
  if (!t->hip_ok(hipStreamSynchronize(t->stream), "upload batch")) return 1;
  t->n_rows = n_rows;
  return 0;
}

int phz_train_update(phz_train* t, const uint32_t* const* order, const uint64_t* order_lens, uint64_t n_order,
                     const phz_ppo_cfg* cfg, phz_update_stats* out) {
  if (!t) return 1;
  t->err.clear();
  if (!cfg || !out) return t->fail("null configuration or output");
  *out = phz_update_stats{0.0, 0.0, 0.0, 0, 0};
  if (t->n_rows == 0) return 0;
  if (cfg->minibatch > t->max_b)
    return t->fail(fmt("minibatch %llu exceeds the pipeline's %llu", (unsigned long long)cfg->minibatch,
                       (unsigned long long)t->max_b));
  if (cfg->minibatch == 0) return t->fail("minibatch must be at least 1");
  if (n_order < cfg->epochs)
    return t->fail(fmt("%llu shuffles for %llu epochs", (unsigned long long)n_order, (unsigned long long)cfg->epochs));
  if (cfg->kl_mode != PHZ_KL_CUMULATIVE && cfg->kl_mode != PHZ_KL_MINIBATCH) return t->fail("unknown KL mode");
  const uint64_t n = t->n_rows, epochs = cfg->epochs;
  if (epochs == 0) return 0;
  if (!order || !order_lens) return t->fail("null shuffle list");
  // Every shuffle is checked before anything runs: its length, and that its
  // indices address the batch (a stray index would be a stray device read).
  for (uint64_t e = 0; e < epochs; e++) {
    if (order_lens[e] != n)
      return t->fail(fmt("shuffle is %llu long, batch is %llu", (unsigned long long)order_lens[e], (unsigned long long)n));
    if (!order[e]) return t->fail("null shuffle");
    for (uint64_t r = 0; r < n; r++)
      if (order[e][r] >= n)
        return t->fail(fmt("shuffle %llu holds index %u, batch is %llu", (unsigned long long)e, order[e][r],
                           (unsigned long long)n));
  }
  if (!set_device(t)) return 1;
  if (epochs * n > t->order_cap) {
    if (t->order) hipFree(t->order);
    t->order = nullptr;
    t->order_cap = 0;
    if (!t->hip_ok(hipMalloc(&t->order, epochs * n * sizeof(uint32_t)), "alloc shuffles")) return 1;
    t->order_cap = epochs * n;
  }
  for (uint64_t e = 0; e < epochs; e++)
    if (!t->hip_ok(hipMemcpyAsync(t->order + e * n, order[e], n * sizeof(uint32_t), hipMemcpyHostToDevice, t->stream),
                   "upload shuffles"))
      return 1;
  if (!t->hip_ok(hipMemsetAsync(t->state, 0, sizeof(UpdateState), t->stream), "reset update state")) return 1;

  TileArgs ta{};
  AdamArgs aa{};
  BrakeArgs ba{};
  for (int k = 0; k < 2; k++) {
    ta.x[k] = t->obs[k];
    ta.w[k] = t->w[k];
    ta.wt[k] = t->wt[k];
    ta.part[k] = t->part[k];
    ta.dims[k] = t->dims[k];
    ta.n_param[k] = t->n_param[k];
    aa.part[k] = t->part[k];
    aa.p[k] = t->p[k];
    aa.m[k] = t->m[k];
    aa.v[k] = t->v[k];
    aa.w[k] = t->w[k];
    aa.wt[k] = t->wt[k];
    aa.dims[k] = t->dims[k];
    aa.n_param[k] = t->n_param[k];
    aa.lr[k] = t->adam[k].lr;
    aa.beta1[k] = t->adam[k].beta1;
    aa.beta2[k] = t->adam[k].beta2;
    aa.eps[k] = t->adam[k].epsilon;
    aa.wd[k] = t->adam[k].weight_decay;
  }
  ta.R = t->R;
  ta.act = t->act;
  ta.logp_old = t->logp_old;
  ta.adv = t->adv;
  ta.ret = t->ret;
  ta.clip = (float)cfg->clip;
  ta.entropy_coef = (float)cfg->entropy_coef;
  ta.vdelta = (float)cfg->vdelta;
  ta.stats_part = t->stats_part;
  ta.stopped = &t->state->stopped;
  aa.stopped = &t->state->stopped;
  ba.stats_part = t->stats_part;
  ba.kl_mode = cfg->kl_mode;
  ba.kl_scale = cfg->kl_scale;
  ba.target_kl = cfg->target_kl;
  ba.st = t->state;
  const uint32_t n_all = t->n_param[0] + t->n_param[1];
  uint64_t j = 0;  // minibatch counter within this update
  for (uint64_t e = 0; e < epochs; e++) {
    for (uint64_t s = 0; s < n; s += cfg->minibatch, j++) {
      const uint32_t b = (uint32_t)std::min<uint64_t>(cfg->minibatch, n - s);
      const uint32_t tiles = (b + t->R - 1) / t->R;
      ta.idx = t->order + e * n + s;
      ta.b = b;
      hipLaunchKernelGGL(ppo_tiles, dim3(tiles, 2), dim3(kThreads), t->lds_bytes, t->stream, ta);
      aa.tiles = tiles;
      for (int k = 0; k < 2; k++) {
        // The step this minibatch would be, if it runs: every earlier one ran.
        aa.bc1[k] = 1.0 - powi(t->adam[k].beta1, t->t[k] + j + 1);
        aa.bc2[k] = 1.0 - powi(t->adam[k].beta2, t->t[k] + j + 1);
      }
      hipLaunchKernelGGL(ppo_adam, dim3((n_all + kThreads - 1) / kThreads), dim3(kThreads), 0, t->stream, aa);
      ba.tiles = tiles;
      ba.b = b;
      hipLaunchKernelGGL(ppo_brake, dim3(1), dim3(64), 0, t->stream, ba);
    }
  }
  if (!t->hip_ok(hipGetLastError(), "launch update")) return 1;
  UpdateState st;
  if (!t->hip_ok(hipMemcpyAsync(&st, t->state, sizeof st, hipMemcpyDeviceToHost, t->stream), "read update state") ||
      !t->hip_ok(hipStreamSynchronize(t->stream), "update"))
    return 1;
  const double nb = (double)std::max<uint64_t>(st.batches, 1);
  out->policy_loss = st.policy_acc / nb;
  out->value_loss = st.value_acc / nb;
  out->kl = st.brake_acc / nb;
  out->grad_steps = st.batches;
  out->stopped_early = st.stopped;
  t->t[0] += st.batches;
  t->t[1] += st.batches;
  return 0;
}

}  // extern "C"
