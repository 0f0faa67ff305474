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
//              Each layer's weights are staged through LDS when they fit.
//   ppo_adam   one thread per parameter of both networks: the tile partials
//              summed in a fixed order in f64, rounded to f32 (the gradient
//              the reference hands Adam is f32), then Adam in f64. Writes the
//              f64 master, the row-major f32 mirror (backward) and a
//              transposed f32 mirror of each weight matrix (forward: lanes
//              over output neurons read consecutive words). Its first wave
//              also folds the minibatch's statistics into the update's
//              running sums and applies the KL brake: when it trips, it sets
//              the next minibatch's stop flag, which every later launch of the
//              update checks first. The loop thus stops after that minibatch,
//              as the reference's host loop does, without the reference's
//              per-minibatch readback.
// Every sum has a fixed order, so an update is bit-reproducible run to run.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "../../include/phyz_amd.h"

namespace {

constexpr int kTileThreads = 512;  // 8 waves per tile workgroup (2 per SIMD)
constexpr int kAdamThreads = 64;   // one wave per Adam workgroup: spread over every CU
constexpr int kAdamLanes = 4;      // lanes that share one parameter's sum over the tiles
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

__host__ __device__ inline uint32_t pad4(uint32_t x) { return (x + 3u) & ~3u; }
// A tile's row of f64 gradient partials, padded to whole 128-byte lines: the
// Adam kernel's wave reads 16 consecutive parameters of a row at once, one
// line when rows start on line boundaries (two when they do not).
__host__ __device__ inline uint32_t part_stride(uint32_t n_param) { return (n_param + 15u) & ~15u; }
// LDS row stride of a row of k values, in floats: k rounded up to whole
// 16-column blocks (the matrix-core loops read 16 columns per step, so the
// padding must exist and hold zeros), then the first value = 20 (mod 32)
// beyond it. An odd number of float4s puts the 16 rows that one ds_read_b128
// of a 16 x 16 block touches in distinct bank groups, and the offset 20
// keeps the 4 consecutive rows that one ds_read_b32 of the gradient blocks
// touches apart (one row stride of 64 floats had put all 16 rows of a block
// on one bank).
__host__ __device__ inline uint32_t row_stride(uint32_t k) {
  const uint32_t s = ((k + 15u) & ~15u) + 4u;
  return s % 32u == 4u ? s + 16u : s;
}

// How a tile workgroup reads the weights: all five matrices staged into LDS
// at the start (one load phase), one layer at a time through a staging buffer,
// or straight from the mirrors in HBM (networks too wide for the LDS).
enum { STAGE_ALL = 0, STAGE_LAYER = 1, STAGE_NONE = 2 };

// A network's weights as the tile kernels hold them in LDS: W1 [n_h][lx],
// W2 [n_h][lh], W3 [n_out][lh] (forward: rows along the summed input), W3t
// [n_h][lo], W2t [n_h][lh] (backprop), each row padded with zeros to its
// row_stride, then the biases b1, b2 [n_h] and b3 [n_out], each padded to a
// float4. The Adam kernel keeps a copy of this image in HBM, so a tile
// stages it with coalesced 16-byte loads and no index arithmetic.
struct WImg {
  uint32_t lx, lh, lo, w_1, w_2, w_3, w_3t, w_2t, b_1, b_2, b_3, size;
  __host__ __device__ explicit WImg(const Dims& d)
      : lx(row_stride(d.n_in)), lh(row_stride(d.n_h)), lo(row_stride(d.n_out)) {
    w_1 = 0;
    w_2 = w_1 + d.n_h * lx;
    w_3 = w_2 + d.n_h * lh;
    w_3t = w_3 + d.n_out * lh;
    w_2t = w_3t + d.n_h * lo;
    b_1 = w_2t + d.n_h * lh;
    b_2 = b_1 + pad4(d.n_h);
    b_3 = b_2 + pad4(d.n_h);
    size = b_3 + pad4(d.n_out);
  }
};

// LDS of one tile workgroup, in floats; row strides from row_stride:
// X [R][lx], H1, H2, DA, DB [R][lh], OUT [R][lo] (the output, then dL/dout),
// ACT [R][lo] (the rows' actions), DLS [R][lo] (per-row dL/dlog_std), RV
// [R][4] (per-row advantage, old log-prob, return), RS [R][4] (per-row
// statistics), SD and LSD [lo] (std and log std), then the weights, each
// matrix with rows along the summed index and zero padding:
// STAGE_ALL  W1 [n_h][lx], W2 [n_h][lh], W3 [n_out][lh] (forward),
//            W3t [n_h][lo], W2t [n_h][lh] (backprop) at WB + w_*;
// STAGE_LAYER one of them at a time at WB.
struct Lds {
  uint32_t lx, lh, lo;
  uint32_t X, H1, H2, DA, DB, OUT, ACT, DLS, RV, RS, SD, LSD, WB, total;
  uint32_t w_1, w_2, w_3, w_3t, w_2t, b_1, b_2, b_3;
  __host__ __device__ Lds(const Dims& d, uint32_t R, int mode) {
    lx = row_stride(d.n_in);
    lh = row_stride(d.n_h);
    lo = row_stride(d.n_out);
    X = 0;
    H1 = X + R * lx;
    H2 = H1 + R * lh;
    DA = H2 + R * lh;
    DB = DA + R * lh;
    OUT = DB + R * lh;
    ACT = OUT + R * lo;
    DLS = ACT + R * lo;
    RV = DLS + R * lo;
    RS = RV + R * 4;
    SD = RS + R * 4;
    LSD = SD + lo;
    WB = LSD + lo;
    const WImg im(d);
    w_1 = im.w_1;
    w_2 = im.w_2;
    w_3 = im.w_3;
    w_3t = im.w_3t;
    w_2t = im.w_2t;
    b_1 = im.b_1;
    b_2 = im.b_2;
    b_3 = im.b_3;
    const uint32_t all = im.size;
    uint32_t one = d.n_h * (lx > lh ? lx : lh);  // the largest staged matrix
    one = one > d.n_out * lh ? one : d.n_out * lh;
    one = one > d.n_h * lo ? one : d.n_h * lo;
    total = WB + (mode == STAGE_ALL ? all : mode == STAGE_LAYER ? one : 0u);
  }
};

struct TileArgs {
  const float* x[2];      // obs_a [n_rows][n_in], obs_c [n_rows][n_in]
  const float* w[2];      // row-major f32 mirrors
  const float* wt[2];     // transposed f32 mirrors of the weight matrices
  const float* img[2];    // padded weight images (WImg)
  double* part[2];        // [tile][part_stride(n_param)] f64 partial gradients
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
  const int* skip;        // nonzero: the KL brake stopped the update before this minibatch
};

// tanh(x) = sign(x) t / (t + 2) with t = expm1(2|x|): within 3 ulp and
// correctly rounded for 86% of f32 inputs (glibc's tanhf, 65%), and tight
// near saturation, where the backward pass's 1 - h^2 magnifies an
// activation's error by 1 / (1 - |h|). Past |x| = 9 tanh rounds to +-1 in f32.
__device__ inline float act_tanh(float x) {
  const float ax = fabsf(x);
  const float t = expm1f(2.0f * (ax < 9.0f ? ax : 9.0f));
  const float h = ax < 9.0f ? t / (t + 2.0f) : 1.0f;
  return x != x ? x : copysignf(h, x);
}

// n / d for n * d < 2^32 by one multiply-high (m = ceil(2^32 / d)).
struct FastDiv {
  uint64_t m;
  uint32_t d;
  __device__ explicit FastDiv(uint32_t d_) : m(((1ull << 32) + d_ - 1) / d_), d(d_) {}
  __device__ uint32_t div(uint32_t n) const { return (uint32_t)(((uint64_t)n * m) >> 32); }
};

enum { EPI_TANH = 0, EPI_LINEAR = 1, EPI_DTANH = 2 };

typedef float float4_t __attribute__((ext_vector_type(4)));

// Y[r][j] for rows r < R, columns j < N of
//   EPI_TANH    tanh(b[j] + sum_k X[r][k] Wkn[k][j])
//   EPI_LINEAR  b[j] + sum_k X[r][k] Wkn[k][j]
//   EPI_DTANH   (sum_k X[r][k] Wkn[k][j]) (1 - H[r][j]^2)
// Wkn is [K][N] row-major: the transposed mirror for a forward layer, the
// row-major weights for a backprop. On the matrix cores: each wave takes 16 x
// 16 (r, j) blocks, its accumulators start from the bias, and one
// v_mfma_f32_16x16x4 per four inputs adds the products. Lane l feeds
// A = X[r0 + l%16][k0 + l/16] and B = Wkn[k0 + l/16][j0 + l%16] and holds
// Y[r0 + 4(l/16) + v][j0 + l%16] in accumulator v. Inputs past K are zero
// (the rows' padding columns are never written, so they are masked, not
// read); rows past R and columns past N read clamped in-range values and are
// not stored.
template <int EPI>
__device__ void dense(const float* __restrict__ X, uint32_t ldx, uint32_t K, const float* __restrict__ Wkn,
                      uint32_t N, const float* __restrict__ bias, const float* __restrict__ H, uint32_t ldh,
                      float* __restrict__ Y, uint32_t ldy, uint32_t R) {
  const uint32_t wave = threadIdx.x / 64u, lane = threadIdx.x % 64u;
  const uint32_t lr = lane / 16u, lc = lane % 16u;
  const uint32_t RB = (R + 15u) / 16u, NB = (N + 15u) / 16u;
  for (uint32_t blk = wave; blk < RB * NB; blk += kTileThreads / 64u) {
    const uint32_t rb = blk / NB, r0 = rb * 16u, j0 = (blk - rb * NB) * 16u;
    const uint32_t ra = r0 + lc < R ? r0 + lc : R - 1u;
    const uint32_t jb = j0 + lc < N ? j0 + lc : N - 1u;
    const float init = EPI == EPI_DTANH ? 0.0f : bias[jb];
    float4_t acc = {init, init, init, init};
    for (uint32_t k0 = 0; k0 < K; k0 += 4u) {
      const uint32_t k = k0 + lr;
      const float av = k < K ? X[ra * ldx + k] : 0.0f;
      const float bv = k < K ? Wkn[k * N + jb] : 0.0f;
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc, 0, 0, 0);
    }
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const uint32_t r = r0 + 4u * lr + v, j = j0 + lc;
      if (r >= R || j >= N) continue;
      float y = acc[v];
      if (EPI == EPI_TANH) y = act_tanh(y);
      if (EPI == EPI_DTANH) {
        const float h = H[r * ldh + j];
        y = y * (1.0f - h * h);
      }
      Y[r * ldy + j] = y;
    }
  }
}

// The same layer with both operands in LDS (staged modes), four inputs per
// lane per load: Wr is [N][ldw], row j holding output j's weights along the
// summed index (the row-major matrix for a forward layer, the transposed one
// for a backprop), X is [R][ldx]; both have zeros from K up to the next
// multiple of 16. For each 16 inputs k0..k0+15, lane l loads the float4s
// X[r0 + l%16][k0 + 4(l/16) ..] and Wr[j0 + l%16][k0 + 4(l/16) ..] (one
// ds_read_b128 each) and component s feeds the s-th of four
// v_mfma_f32_16x16x4: that product sums k0 + 4q + s over q = 0..3, so the four
// cover the 16 inputs once. Blocks are dealt to the waves in row-major order
// without a division.
template <int EPI>
__device__ void dense4(const float* __restrict__ X, uint32_t ldx, uint32_t K, const float* __restrict__ Wr,
                       uint32_t ldw, uint32_t N, const float* __restrict__ bias, const float* __restrict__ H,
                       uint32_t ldh, float* __restrict__ Y, uint32_t ldy, uint32_t R) {
  const uint32_t wave = threadIdx.x / 64u, lane = threadIdx.x % 64u;
  const uint32_t lr = lane / 16u, lc = lane % 16u;
  constexpr uint32_t kWaves = kTileThreads / 64u;
  uint32_t blk = 0;
  for (uint32_t r0 = 0; r0 < R; r0 += 16u)
    for (uint32_t j0 = 0; j0 < N; j0 += 16u, blk++) {
      if (blk % kWaves != wave) continue;
      const uint32_t ra = r0 + lc < R ? r0 + lc : R - 1u;
      const uint32_t jb = j0 + lc < N ? j0 + lc : N - 1u;
      const float init = EPI == EPI_DTANH ? 0.0f : bias[jb];
      // Two accumulators (components 0, 2 and 1, 3) halve the chain of
      // dependent MFMAs; the next 16 inputs load while these multiply (the
      // last prefetch re-reads the final block, in bounds).
      float4_t acc = {init, init, init, init}, acc2 = {0.0f, 0.0f, 0.0f, 0.0f};
      const float* xa = X + ra * ldx + 4u * lr;
      const float* wb = Wr + jb * ldw + 4u * lr;
      float4_t a = *reinterpret_cast<const float4_t*>(xa);
      float4_t b = *reinterpret_cast<const float4_t*>(wb);
      for (uint32_t k0 = 0; k0 < K; k0 += 16u) {
        const uint32_t kn = k0 + 16u < K ? k0 + 16u : k0;
        const float4_t an = *reinterpret_cast<const float4_t*>(xa + kn);
        const float4_t bn = *reinterpret_cast<const float4_t*>(wb + kn);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[0], b[0], acc, 0, 0, 0);
        acc2 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[1], b[1], acc2, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[2], b[2], acc, 0, 0, 0);
        acc2 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[3], b[3], acc2, 0, 0, 0);
        a = an;
        b = bn;
      }
      acc += acc2;
#pragma unroll
      for (int v = 0; v < 4; v++) {
        const uint32_t r = r0 + 4u * lr + v, j = j0 + lc;
        if (r >= R || j >= N) continue;
        float y = acc[v];
        if (EPI == EPI_TANH) y = act_tanh(y);
        if (EPI == EPI_DTANH) {
          const float h = H[r * ldh + j];
          y = y * (1.0f - h * h);
        }
        Y[r * ldy + j] = y;
      }
    }
}

typedef double double4_t __attribute__((ext_vector_type(4)));

// Tile partials of a linear layer's gradients, Gw[o][i] = sum_r D[r][o] X[r][i]
// and Gb[o] = sum_r D[r][o], in f64 (the reference's row loops accumulate in
// double, phyz_train.cu:226-260), on the matrix cores: each wave takes 16 x 16
// (o, i) blocks and runs one v_mfma_f64_16x16x4 per four rows over all R rows.
// Lane l feeds A = D[r0 + l/16][o0 + l%16] and B = X[r0 + l/16][i0 + l%16] and
// holds Gw[o0 + l/16 + 4v][i0 + l%16] in accumulator v. Rows past the
// minibatch have D = 0 (and finite X), so they add nothing; outputs and
// inputs past O and I read clamped in-range values and are not stored. Every
// sum is an f64 sum in an order fixed by the hardware, so a tile's partials
// are reproducible. The bias sums use four lanes per output: rows p, p + 4,
// ... for lane p, combined by a fixed butterfly. The partials are stored
// non-temporally: each is written once here and read once by ppo_adam,
// mostly on another XCD, so holding them in this XCD's L2 only slowed the
// stores (31 -> 25 us per tile launch at the timing shape).
__device__ void dense_grad(const float* __restrict__ D, uint32_t ldd, uint32_t O, const float* __restrict__ X,
                           uint32_t ldx, uint32_t I, uint32_t R, double* __restrict__ Gw, double* __restrict__ Gb) {
  const uint32_t wave = threadIdx.x / 64u, lane = threadIdx.x % 64u;
  const uint32_t lr = lane / 16u, lc = lane % 16u;
  constexpr uint32_t kWaves = kTileThreads / 64u;
  uint32_t blk = 0;
  for (uint32_t o0 = 0; o0 < O; o0 += 16u)
    for (uint32_t i0 = 0; i0 < I; i0 += 16u, blk++) {
      if (blk % kWaves != wave) continue;
      const uint32_t oa = o0 + lc < O ? o0 + lc : O - 1u;
      const uint32_t ia = i0 + lc < I ? i0 + lc : I - 1u;
      // Sixteen rows per round: the eight LDS reads first, then four MFMAs
      // alternating between two accumulators (R is a multiple of 8).
      double4_t acc = {0.0, 0.0, 0.0, 0.0}, acc2 = {0.0, 0.0, 0.0, 0.0};
      for (uint32_t r0 = 0; r0 < R; r0 += 16u) {
        double av[4], bv[4];
#pragma unroll
        for (uint32_t q = 0; q < 4u; q++) {
          const uint32_t r = r0 + 4u * q + lr < R ? r0 + 4u * q + lr : lr;
          av[q] = (double)D[r * ldd + oa];
          bv[q] = (double)X[r * ldx + ia];
        }
        acc = __builtin_amdgcn_mfma_f64_16x16x4f64(av[0], bv[0], acc, 0, 0, 0);
        acc2 = __builtin_amdgcn_mfma_f64_16x16x4f64(av[1], bv[1], acc2, 0, 0, 0);
        if (r0 + 8u < R) {
          acc = __builtin_amdgcn_mfma_f64_16x16x4f64(av[2], bv[2], acc, 0, 0, 0);
          acc2 = __builtin_amdgcn_mfma_f64_16x16x4f64(av[3], bv[3], acc2, 0, 0, 0);
        }
      }
      acc += acc2;
#pragma unroll
      for (int v = 0; v < 4; v++) {
        const uint32_t o = o0 + lr + 4u * v, i = i0 + lc;
        if (o < O && i < I) __builtin_nontemporal_store(acc[v], &Gw[(size_t)o * I + i]);
      }
    }
  for (uint32_t t = threadIdx.x; t < 4u * ((O + 15u) & ~15u); t += kTileThreads) {
    const uint32_t o = t / 4u, p = t % 4u;
    double acc = 0.0;
    if (o < O)
      for (uint32_t r = p; r < R; r += 4u) acc += (double)D[r * ldd + o];
    acc += __shfl_xor(acc, 1, 64);
    acc += __shfl_xor(acc, 2, 64);
    if (p == 0 && o < O) __builtin_nontemporal_store(acc, &Gb[o]);
  }
}

// count floats (a multiple of 4, 16-byte aligned at both ends) from global
// memory into LDS, eight 16-byte loads in flight per thread.
__device__ void copy4(float* __restrict__ dst, const float* __restrict__ src, uint32_t count) {
  constexpr uint32_t U = 8;
  const uint32_t n4 = count / 4u;
  const float4_t* s4 = reinterpret_cast<const float4_t*>(src);
  float4_t* d4 = reinterpret_cast<float4_t*>(dst);
  for (uint32_t base = threadIdx.x; base < n4; base += U * kTileThreads) {
    float4_t v[U];
#pragma unroll
    for (uint32_t u = 0; u < U; u++) {
      const uint32_t e = base + u * kTileThreads;
      v[u] = s4[e < n4 ? e : 0u];
    }
#pragma unroll
    for (uint32_t u = 0; u < U; u++) {
      const uint32_t e = base + u * kTileThreads;
      if (e < n4) d4[e] = v[u];
    }
  }
}

__device__ inline float clampf(float x, float lo, float hi) { return x < lo ? lo : (x > hi ? hi : x); }

// One workgroup per (tile of R minibatch rows, network); MODE as above.
template <int MODE>
__global__ void __launch_bounds__(kTileThreads) ppo_tiles(TileArgs a) {
  // The stop flag is read here and tested once the tile's first loads are in
  // flight, so its round trip overlaps theirs; a stopped minibatch's loads
  // stay in bounds (its index list was validated) and it stores nothing.
  const int stopped = *a.skip;
  extern __shared__ __align__(16) float lds[];
  const int net = blockIdx.y;
  const Dims d = a.dims[net];
  const uint32_t R = a.R;
  const uint32_t row0 = blockIdx.x * R;
  const uint32_t rows = row0 >= a.b ? 0u : std::min(R, a.b - row0);
  const Lds L(d, R, MODE);
  float* X = lds + L.X;
  float* H1 = lds + L.H1;
  float* H2 = lds + L.H2;
  float* DA = lds + L.DA;
  float* DB = lds + L.DB;
  float* OUT = lds + L.OUT;
  float* ACT = lds + L.ACT;
  float* DLS = lds + L.DLS;
  float* RV = lds + L.RV;
  float* RS = lds + L.RS;
  float* SD = lds + L.SD;
  float* LSD = lds + L.LSD;
  float* WB = lds + L.WB;
  const float* w = a.w[net];
  const float* wt = a.wt[net];
  double* part = a.part[net] + (size_t)blockIdx.x * part_stride(a.n_param[net]);
  const float* x = a.x[net];
  const float* img = a.img[net];
  // A forward layer's weights for the matrix-core loop: the LDS copy
  // (STAGE_ALL) or the staging buffer, loaded here from the weight image
  // (STAGE_LAYER; every wave is past the previous layer's reads at the first
  // barrier).
  auto staged = [&](uint32_t off, uint32_t rows_, uint32_t ld) -> const float* {
    if (MODE == STAGE_ALL) return WB + off;
    __syncthreads();
    copy4(WB, img + off, rows_ * ld);
    __syncthreads();
    return WB;
  };

  // A layer's biases: the image's LDS copy (STAGE_ALL) or the f32 mirror.
  auto bias = [&](uint32_t off, uint32_t q) -> const float* { return MODE == STAGE_ALL ? WB + off : w + q; };

  // ── the tile's inputs: its rows (the minibatch is an index list into the
  //    batch), their actions and scalars, and the weight image. Every global
  //    load of the first batch is issued before any LDS store. ──
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64u), lane = threadIdx.x % 64u;
  constexpr uint32_t kWaves = kTileThreads / 64u;
  constexpr uint32_t kImgU = 12;  // float4s of the image per thread in the first batch
  const float4_t* img4 = reinterpret_cast<const float4_t*>(img);
  float4_t* WB4 = reinterpret_cast<float4_t*>(WB);
  const uint32_t n4 = MODE == STAGE_ALL ? WImg(d).size / 4u : 0u;
  float4_t wv[kImgU];
#pragma unroll
  for (uint32_t u = 0; u < kImgU; u++) {
    const uint32_t e = threadIdx.x + u * kTileThreads;
    wv[u] = img4[e < n4 ? e : 0u];
  }
  // Zero H1, H2, DA, DB and OUT, whose padding columns the matrix-core loops
  // read (against zero weights, but an uninitialised NaN would survive the
  // product); nothing else writes them before the barrier below.
  for (uint32_t e = L.H1 + 4u * threadIdx.x; e < L.ACT; e += 4u * kTileThreads)
    *reinterpret_cast<float4_t*>(lds + e) = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
  // Rows: wave w takes rows w, w + 8, ...; its lanes run over 64-column chunks.
  const uint32_t nchunk = (L.lx + 63u) / 64u, nrw = (R + kWaves - 1u) / kWaves;
  const uint32_t nt = nrw * nchunk;
  float sdv = 0.0f;
  if (net == 0 && threadIdx.x < d.n_out) sdv = w[d.mlp_params() + threadIdx.x];
  // t = q * nchunk + ch runs over this wave's (row, chunk) pairs; q and ch
  // are stepped, not divided out.
  uint32_t q0 = 0, ch0 = 0;
  for (uint32_t t0 = 0; t0 < nt; t0 += 8u) {
    float xv[8], av[8], rv[8];
    uint32_t q = q0, ch = ch0;
#pragma unroll
    for (uint32_t u = 0; u < 8u; u++) {
      const uint32_t t = t0 + u, i = ch * 64u + lane, r = wave + kWaves * q;
      const bool live = t < nt && r < rows;
      const uint32_t sidx = live ? a.idx[row0 + r] : 0u;
      xv[u] = live && i < d.n_in ? x[(size_t)sidx * d.n_in + i] : 0.0f;
      const bool first = ch == 0u;  // one chunk per row fetches the row's extras
      av[u] = net == 0 && live && first && lane < d.n_out ? a.act[(size_t)sidx * d.n_out + lane] : 0.0f;
      const float* sc = net == 0 ? (lane == 0 ? a.adv : a.logp_old) : a.ret;
      rv[u] = live && first && lane < (net == 0 ? 2u : 1u) ? sc[sidx] : 0.0f;
      if (++ch == nchunk) { ch = 0u; ++q; }
    }
    q = q0;
    ch = ch0;
#pragma unroll
    for (uint32_t u = 0; u < 8u; u++) {
      const uint32_t t = t0 + u, i = ch * 64u + lane, r = wave + kWaves * q;
      if (t < nt && r < R) {
        if (i < L.lx) X[r * L.lx + i] = xv[u];  // zero past n_in
        if (ch == 0u) {
          if (net == 0 && lane < d.n_out) ACT[r * L.lo + lane] = av[u];
          if (lane < (net == 0 ? 2u : 1u)) RV[r * 4 + (net == 0 ? lane : 2u)] = rv[u];
        }
      }
      if (++ch == nchunk) { ch = 0u; ++q; }
    }
    q0 = q;
    ch0 = ch;
  }
  if (stopped) return;  // uniform over the workgroup, before its first barrier
  if (net == 0 && threadIdx.x < d.n_out) {
    const float sd = expf(sdv);
    SD[threadIdx.x] = sd;
    LSD[threadIdx.x] = logf(sd);
  }
#pragma unroll
  for (uint32_t u = 0; u < kImgU; u++) {
    const uint32_t e = threadIdx.x + u * kTileThreads;
    if (e < n4) WB4[e] = wv[u];
  }
  for (uint32_t e = threadIdx.x + kImgU * kTileThreads; e < n4; e += kTileThreads) WB4[e] = img4[e];
  __syncthreads();

  // ── forward (phyz_train.cu:101-133) ──
  if (MODE == STAGE_NONE) {
    dense<EPI_TANH>(X, L.lx, d.n_in, wt, d.n_h, w + d.ob1(), nullptr, 0, H1, L.lh, R);
    __syncthreads();
    dense<EPI_TANH>(H1, L.lh, d.n_h, wt + d.tW2(), d.n_h, w + d.ob2(), nullptr, 0, H2, L.lh, R);
    __syncthreads();
    dense<EPI_LINEAR>(H2, L.lh, d.n_h, wt + d.tW3(), d.n_out, w + d.ob3(), nullptr, 0, OUT, L.lo, R);
  } else {
    dense4<EPI_TANH>(X, L.lx, d.n_in, staged(L.w_1, d.n_h, L.lx), L.lx, d.n_h, bias(L.b_1, d.ob1()),
                     nullptr, 0, H1, L.lh, R);
    if (MODE == STAGE_ALL) __syncthreads();
    dense4<EPI_TANH>(H1, L.lh, d.n_h, staged(L.w_2, d.n_h, L.lh), L.lh, d.n_h, bias(L.b_2, d.ob2()),
                     nullptr, 0, H2, L.lh, R);
    if (MODE == STAGE_ALL) __syncthreads();
    dense4<EPI_LINEAR>(H2, L.lh, d.n_h, staged(L.w_3, d.n_out, L.lh), L.lh, d.n_out,
                       bias(L.b_3, d.ob3()), nullptr, 0, OUT, L.lo, R);
  }
  __syncthreads();

  // ── loss gradient; OUT becomes dL/dout ──
  const float fb = (float)a.b;
  if (net == 0) {
    // Clipped surrogate with the gradient through the active branch only and
    // the entropy bonus folded into dlog_std (phyz_train.cu:150-196), in three
    // passes: the standardized actions z of every (row, dim) in parallel (DLS
    // holds them), each row's log-prob summed over dims in order with its
    // ratio and branch, then every (row, dim) gradient in parallel.
    const float LN_2PI = 1.8378770664093453f;
    const FastDiv byOut(d.n_out);
    for (uint32_t e = threadIdx.x; e < rows * d.n_out; e += kTileThreads) {
      const uint32_t r = byOut.div(e), k = e - r * d.n_out;
      DLS[r * L.lo + k] = (ACT[r * L.lo + k] - OUT[r * L.lo + k]) / SD[k];
    }
    __syncthreads();
    for (uint32_t r = threadIdx.x; r < R; r += kTileThreads) {
      if (r >= rows) {
        RS[r * 4 + 0] = RS[r * 4 + 1] = RS[r * 4 + 2] = 0.0f;
        continue;
      }
      const float* z = DLS + r * L.lo;
      float logp = 0.0f;
      for (uint32_t k = 0; k < d.n_out; k++) logp += -0.5f * z[k] * z[k] - LSD[k] - 0.5f * LN_2PI;
      const float adv = RV[r * 4 + 0], lp_old = RV[r * 4 + 1];
      const float log_ratio = logp - lp_old;
      const float ratio = expf(log_ratio);
      const float clipped = clampf(ratio, 1.0f - a.clip, 1.0f + a.clip);
      const float uo = ratio * adv, co = clipped * adv;
      RS[r * 4 + 0] = -(uo < co ? uo : co);
      RS[r * 4 + 1] = lp_old - logp;
      RS[r * 4 + 2] = ratio - 1.0f - log_ratio;
      // The row's gradient scale, and whether the unclipped branch is the
      // active one (an actor row has no use for the critic's column 3).
      RV[r * 4 + 3] = -adv * ratio / fb;
      RS[r * 4 + 3] = uo <= co + 1e-12f ? 1.0f : 0.0f;
    }
    __syncthreads();
    for (uint32_t e = threadIdx.x; e < R * d.n_out; e += kTileThreads) {
      const uint32_t r = byOut.div(e), k = e - r * d.n_out;
      float dm = 0.0f, dl = 0.0f;
      if (r < rows) {
        if (RS[r * 4 + 3] == 0.0f) {
          dl = -a.entropy_coef / fb;
        } else {
          const float coef = RV[r * 4 + 3], z = DLS[r * L.lo + k];
          dm = coef * (z / SD[k]);
          dl = coef * (z * z - 1.0f) - a.entropy_coef / fb;
        }
      }
      OUT[r * L.lo + k] = dm;
      DLS[r * L.lo + k] = dl;
    }
  } else {
    // Squared error to the return with the gradient Huber-clipped at vdelta;
    // the statistic stays the plain squared error (phyz_train.cu:198-208).
    for (uint32_t r = threadIdx.x; r < R; r += kTileThreads) {
      if (r >= rows) {
        OUT[r * L.lo] = 0.0f;
        RS[r * 4 + 3] = 0.0f;
        continue;
      }
      const float err = OUT[r * L.lo] - RV[r * 4 + 2];
      RS[r * 4 + 3] = err * err;
      OUT[r * L.lo] = 2.0f * clampf(err, -a.vdelta, a.vdelta) / fb;
    }
  }
  if (MODE == STAGE_LAYER) copy4(WB, img + L.w_3t, d.n_h * L.lo);  // W3 transposed, for dL/dh2
  __syncthreads();

  // ── layer 3 gradients, tile statistics, dL/dh2 ──
  dense_grad(OUT, L.lo, d.n_out, H2, L.lh, d.n_h, R, part + d.oW3(), part + d.ob3());
  // The column sums of dlog_std and of the statistics, on the last threads
  // (the gradient items above start from thread 0).
  const uint32_t back = kTileThreads - 1u - threadIdx.x;
  if (net == 0) {
    for (uint32_t k = back; k < d.n_out; k += kTileThreads) {
      double acc = 0.0;
      for (uint32_t r = 0; r < rows; r++) acc += (double)DLS[r * L.lo + k];
      part[d.mlp_params() + k] = acc;
    }
  }
  if (back >= 32u && back < 36u && (net == 0) == (back < 35u)) {
    const uint32_t c = back - 32u;
    double acc = 0.0;
    for (uint32_t r = 0; r < rows; r++) acc += (double)RS[r * 4 + c];
    a.stats_part[(size_t)blockIdx.x * 4 + c] = acc;
  }
  if (MODE == STAGE_NONE)
    dense<EPI_DTANH>(OUT, L.lo, d.n_out, w + d.oW3(), d.n_h, nullptr, H2, L.lh, DA, L.lh, R);
  else
    dense4<EPI_DTANH>(OUT, L.lo, d.n_out, MODE == STAGE_ALL ? WB + L.w_3t : WB, L.lo, d.n_h, nullptr, H2, L.lh, DA,
                      L.lh, R);
  if (MODE == STAGE_LAYER) {  // W2 transposed, for dL/dh1
    __syncthreads();
    copy4(WB, img + L.w_2t, d.n_h * L.lh);
  }
  __syncthreads();

  // ── layer 2 gradients, dL/dh1 ──
  dense_grad(DA, L.lh, d.n_h, H1, L.lh, d.n_h, R, part + d.oW2(), part + d.ob2());
  if (MODE == STAGE_NONE)
    dense<EPI_DTANH>(DA, L.lh, d.n_h, w + d.oW2(), d.n_h, nullptr, H1, L.lh, DB, L.lh, R);
  else
    dense4<EPI_DTANH>(DA, L.lh, d.n_h, MODE == STAGE_ALL ? WB + L.w_2t : WB, L.lh, d.n_h, nullptr, H1, L.lh, DB, L.lh,
                      R);
  __syncthreads();

  // ── layer 1 gradients (input: the gathered rows) ──
  dense_grad(DB, L.lh, d.n_h, X, L.lx, d.n_in, R, part + d.oW1(), part + d.ob1());
}

// The update's running sums on the device (train.rs:620-627).
struct UpdateState {
  double policy_acc, value_acc, brake_acc, kl_acc;
  uint64_t kl_rows, batches;
  int stopped;
  int pad;
};

struct AdamArgs {
  const double* part[2];
  double* p[2];
  double* m[2];
  double* v[2];
  float* w[2];
  float* wt[2];
  float* img[2];
  Dims dims[2];
  uint32_t n_param[2];
  uint32_t tiles;
  double lr[2], beta1[2], beta2[2], eps[2], wd[2], bc1[2], bc2[2];
  // The minibatch's statistics and the KL brake (train.rs:757-777).
  const double* stats_part;  // [tile][4]
  uint32_t b;
  int kl_mode;               // PHZ_KL_CUMULATIVE / PHZ_KL_MINIBATCH
  double kl_scale, target_kl;
  UpdateState* st;
  int* skip;                 // skip[j]: minibatch j does not run; this one is skip[0], the next skip[1]
};

// Wave 0 of workgroup 0: the four statistic columns summed over the tiles
// (lane l takes tiles l, l + 64, ..., then a fixed butterfly across lanes),
// rounded to f32 as the reference's reduce_stats output is, into the running
// sums; then the brake, which decides whether the next minibatch runs. The
// first two tiles of each lane come preloaded (`pre`, loaded at kernel entry
// beside the gradient partials), and so does the update's state (`s0`); the
// rest of the tiles are read here, in the same order.
constexpr uint32_t kStatPre = 2;
__device__ void brake(const AdamArgs& a, const double (&pre)[kStatPre][4], const UpdateState& s0) {
  const uint32_t lane = threadIdx.x;
  double s[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
  for (uint32_t r = 0; r < kStatPre; r++)
    if (lane + 64u * r < a.tiles)
      for (int c = 0; c < 4; c++) s[c] += pre[r][c];
  for (uint32_t k = lane + 64u * kStatPre; k < a.tiles; k += 64)
    for (int c = 0; c < 4; c++) s[c] += a.stats_part[(size_t)k * 4 + c];
  for (int c = 0; c < 4; c++)
    for (int off = 32; off > 0; off >>= 1) s[c] += __shfl_xor(s[c], off, 64);
  if (lane != 0) return;
  UpdateState* st = a.st;
  const double ploss = (double)(float)s[0], kl_sum = (double)(float)s[1];
  const double k3_sum = (double)(float)s[2], vloss = (double)(float)s[3];
  const double b = (double)a.b;
  const double kl_acc = s0.kl_acc + kl_sum;
  const uint64_t kl_rows = s0.kl_rows + a.b;
  st->policy_acc = s0.policy_acc + ploss / b;
  st->value_acc = s0.value_acc + vloss / b;
  st->kl_acc = kl_acc;
  st->kl_rows = kl_rows;
  const double rows = (double)(kl_rows > 0 ? kl_rows : 1);
  const double reading = (a.kl_mode == PHZ_KL_CUMULATIVE ? fabs(kl_acc / rows) : k3_sum / b) / a.kl_scale;
  st->brake_acc = s0.brake_acc + reading;
  st->batches = s0.batches + 1;
  if (reading > a.target_kl) {
    st->stopped = 1;
    a.skip[1] = 1;
  }
}

// tang's ModuleAdam step, elementwise (phyz_train.cu:268-288), on the sum of
// the tile partials. Four lanes share a parameter: lane s sums tiles s, s + 4,
// ... in eight interleaved chains, chain j taking tiles s + 4j, s + 4j + 32,
// ..., added as a fixed tree; a fixed xor butterfly gives all four the same
// total, and the first applies the step. Each lane issues the loads of up to
// four rounds of its chains (32 partials, 128 tiles) before the first add, so
// a minibatch of up to 128 tiles per network costs one memory round trip; the
// grid holds about one wave per SIMD, so the kernel asks for the registers of
// two resident waves, not the compiler's default of five (which kept only 22
// of the 32 loads in flight).
__global__ void __launch_bounds__(kAdamThreads) __attribute__((amdgpu_waves_per_eu(1, 2))) ppo_adam(AdamArgs a) {
  // The stop flag is tested once the partial sums' loads are in flight (as
  // in ppo_tiles); a stopped minibatch's tiles stored nothing, so what they
  // read is never used.
  const int stopped = *a.skip;
  // Loaded for every lane at a clamped, in-range tile (tiles >= 1); the brake
  // adds only those of tiles that exist.
  double pre[kStatPre][4];
#pragma unroll
  for (uint32_t r = 0; r < kStatPre; r++) {
    const uint32_t k = threadIdx.x + 64u * r;
    const double* sp = a.stats_part + (size_t)(k < a.tiles ? k : 0u) * 4;
#pragma unroll
    for (int c = 0; c < 4; c++) pre[r][c] = sp[c];
  }
  const uint32_t gt = blockIdx.x * kAdamThreads + threadIdx.x;
  const uint32_t t = gt / kAdamLanes, sub = gt % kAdamLanes;
  // Parameter slots: the actor's padded to a multiple of 16, then the
  // critic's, so that every wave's 16 parameters lie in one network and start
  // on a 128-byte line of each partial row.
  const uint32_t lead = part_stride(a.n_param[0]);
  const int net = t >= lead ? 1 : 0;
  const uint32_t qt = net == 0 ? t : t - lead;
  const bool valid = qt < a.n_param[net];
  const uint32_t q = valid ? qt : 0u;
  const uint32_t np = part_stride(a.n_param[net]);
  const double* part = a.part[net] + q;
  // The parameter's master weight and Adam moments, loaded beside the partials
  // (the four lanes of a parameter read the same words; lanes past the last
  // parameter read slot 0 and store nothing), and the update's state for the
  // brake (every workgroup reads the same 48 bytes; workgroup 0 uses them).
  const double p0 = a.p[net][q], m0 = a.m[net][q], v0 = a.v[net][q];
  const UpdateState s0 = *a.st;
  constexpr uint32_t kChains = 8, kRounds = 4;
  double gc[kChains];
#pragma unroll
  for (uint32_t j = 0; j < kChains; j++) gc[j] = 0.0;
  if (valid) {
    uint32_t k = sub;
    for (; k + (kRounds * kChains - 1) * kAdamLanes < a.tiles; k += kRounds * kChains * kAdamLanes) {
      double x[kRounds][kChains];
#pragma unroll
      for (uint32_t r = 0; r < kRounds; r++)
#pragma unroll
        for (uint32_t j = 0; j < kChains; j++) x[r][j] = part[(size_t)(k + (r * kChains + j) * kAdamLanes) * np];
#pragma unroll
      for (uint32_t r = 0; r < kRounds; r++)
#pragma unroll
        for (uint32_t j = 0; j < kChains; j++) gc[j] += x[r][j];
    }
    for (; k + (kChains - 1) * kAdamLanes < a.tiles; k += kChains * kAdamLanes) {
#pragma unroll
      for (uint32_t j = 0; j < kChains; j++) gc[j] += part[(size_t)(k + j * kAdamLanes) * np];
    }
#pragma unroll
    for (uint32_t j = 0; j < kChains; j++)
      if (k + j * kAdamLanes < a.tiles) gc[j] += part[(size_t)(k + j * kAdamLanes) * np];
  }
  if (stopped) {
    if (blockIdx.x == 0 && threadIdx.x == 0) a.skip[1] = 1;  // a stopped update stays stopped
    return;
  }
  if (blockIdx.x == 0) brake(a, pre, s0);
  double g = ((gc[0] + gc[1]) + (gc[2] + gc[3])) + ((gc[4] + gc[5]) + (gc[6] + gc[7]));
  for (int off = 1; off < kAdamLanes; off <<= 1) g += __shfl_xor(g, off, 64);
  if (!valid || sub != 0) return;
  const double gr = (double)(float)g;
  double x = p0;
  const double lr = a.lr[net];
  if (a.wd[net] > 0.0) x = x * (1.0 - lr * a.wd[net]);
  const double b1 = a.beta1[net], b2 = a.beta2[net];
  const double mt = b1 * m0 + (1.0 - b1) * gr;
  const double vt = b2 * v0 + (1.0 - b2) * gr * gr;
  a.m[net][q] = mt;
  a.v[net][q] = vt;
  const double m_hat = mt / a.bc1[net];
  const double v_hat = vt / a.bc2[net];
  x -= lr * m_hat / (sqrt(v_hat) + a.eps[net]);
  a.p[net][q] = x;
  const float xf = (float)x;
  a.w[net][q] = xf;
  const Dims d = a.dims[net];
  const WImg im(d);
  float* img = a.img[net];
  if (q < d.ob1()) {
    const uint32_t j = q / d.n_in, i = q % d.n_in;
    a.wt[net][i * d.n_h + j] = xf;
    img[im.w_1 + j * im.lx + i] = xf;
  } else if (q >= d.oW2() && q < d.ob2()) {
    const uint32_t e = q - d.oW2(), j = e / d.n_h, i = e % d.n_h;
    a.wt[net][d.tW2() + i * d.n_h + j] = xf;
    img[im.w_2 + j * im.lh + i] = xf;
    img[im.w_2t + i * im.lh + j] = xf;
  } else if (q >= d.oW3() && q < d.ob3()) {
    const uint32_t e = q - d.oW3(), k2 = e / d.n_h, i = e % d.n_h;
    a.wt[net][d.tW3() + i * d.n_out + k2] = xf;
    img[im.w_3 + k2 * im.lh + i] = xf;
    img[im.w_3t + i * im.lo + k2] = xf;
  } else if (q >= d.ob1() && q < d.oW2()) {
    img[im.b_1 + q - d.ob1()] = xf;
  } else if (q >= d.ob2() && q < d.oW3()) {
    img[im.b_2 + q - d.ob2()] = xf;
  } else if (q >= d.ob3() && q < d.mlp_params()) {
    img[im.b_3 + q - d.ob3()] = xf;
  }
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
  int mode = STAGE_ALL;
  size_t lds_bytes = 0;
  phz_adam_cfg adam[2];
  uint64_t t[2] = {0, 0};
  // device buffers
  float* w[2] = {nullptr, nullptr};
  float* wt[2] = {nullptr, nullptr};
  float* img[2] = {nullptr, nullptr};  // padded weight images (WImg)
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
  int* skip = nullptr;      // per-minibatch stop flags of the current update
  uint64_t skip_cap = 0;
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
    if (skip) hipFree(skip);
    if (stream) hipStreamDestroy(stream);
  }
};

namespace {

bool set_device(phz_train* t) { return t->hip_ok(hipSetDevice(t->device), "hipSetDevice"); }

// Rows per tile and weight staging, the first option whose workgroup fits the
// device's LDS: 32 rows with every weight matrix staged (one load phase), 16
// rows likewise, then one layer at a time, then weights from HBM; and 8-row
// tiles as the last resort. PHZ_TRAIN_TILE_ROWS=8|16|32|64 restricts the
// choice to that row count (tuning, tests).
bool choose_tile(phz_train* t, size_t lds_limit, std::string& e) {
  auto bytes = [&](uint32_t R, int mode) {
    size_t worst = 0;
    for (int n = 0; n < 2; n++) worst = std::max<size_t>(worst, Lds(t->dims[n], R, mode).total);
    return worst * sizeof(float);
  };
  uint32_t only = 0;
  if (const char* env = std::getenv("PHZ_TRAIN_TILE_ROWS")) {
    only = (uint32_t)std::atoi(env);
    if (only != 8 && only != 16 && only != 32 && only != 64) {
      e = fmt("PHZ_TRAIN_TILE_ROWS must be 8, 16, 32 or 64, not '%s'", env);
      return false;
    }
  }
  struct Option { uint32_t R; int mode; };
  const Option options[] = {{32, STAGE_ALL},  {16, STAGE_ALL},   {64, STAGE_ALL},  {32, STAGE_LAYER},
                            {16, STAGE_LAYER}, {64, STAGE_LAYER}, {32, STAGE_NONE}, {16, STAGE_NONE},
                            {8, STAGE_ALL},   {8, STAGE_LAYER},  {8, STAGE_NONE}};
  for (const Option& o : options) {
    if (only && o.R != only) continue;
    if (bytes(o.R, o.mode) <= lds_limit) {
      t->R = o.R;
      t->mode = o.mode;
      t->lds_bytes = bytes(o.R, o.mode);
      return true;
    }
  }
  const uint32_t R = only ? only : 8;
  e = fmt("networks too wide for one tile: %u rows need %zu bytes of LDS, the device has %zu", R, bytes(R, STAGE_NONE),
          lds_limit);
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
  const WImg im(d);
  std::vector<float> img(im.size, 0.0f);
  for (uint32_t j = 0; j < d.n_h; j++)
    for (uint32_t i = 0; i < d.n_in; i++) img[im.w_1 + j * im.lx + i] = mirror[d.oW1() + j * d.n_in + i];
  for (uint32_t j = 0; j < d.n_h; j++)
    for (uint32_t i = 0; i < d.n_h; i++) {
      img[im.w_2 + j * im.lh + i] = mirror[d.oW2() + j * d.n_h + i];
      img[im.w_2t + i * im.lh + j] = mirror[d.oW2() + j * d.n_h + i];
    }
  for (uint32_t k = 0; k < d.n_out; k++)
    for (uint32_t i = 0; i < d.n_h; i++) {
      img[im.w_3 + k * im.lh + i] = mirror[d.oW3() + k * d.n_h + i];
      img[im.w_3t + i * im.lo + k] = mirror[d.oW3() + k * d.n_h + i];
    }
  for (uint32_t j = 0; j < d.n_h; j++) {
    img[im.b_1 + j] = mirror[d.ob1() + j];
    img[im.b_2 + j] = mirror[d.ob2() + j];
  }
  for (uint32_t k = 0; k < d.n_out; k++) img[im.b_3 + k] = mirror[d.ob3() + k];
  return t->hip_ok(hipMemcpyAsync(t->img[net], img.data(), img.size() * sizeof(float), hipMemcpyHostToDevice, t->stream),
                   "upload params") &&
         t->hip_ok(hipMemcpyAsync(t->p[net], flat, np * sizeof(double), hipMemcpyHostToDevice, t->stream), "upload params") &&
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
    if (nd[n].n_in > (1u << 14)) {  // keeps every in-kernel index product below 2^32
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
  if (t->lds_bytes > 65536) {
    const void* fns[3] = {(const void*)ppo_tiles<STAGE_ALL>, (const void*)ppo_tiles<STAGE_LAYER>,
                          (const void*)ppo_tiles<STAGE_NONE>};
    if (!t->hip_ok(hipFuncSetAttribute(fns[t->mode], hipFuncAttributeMaxDynamicSharedMemorySize, (int)t->lds_bytes),
                   "LDS attribute"))
      return bail(t->err);
  }
  t->max_tiles = (uint32_t)((max_b + t->R - 1) / t->R);
  bool ok = true;
  for (int n = 0; n < 2 && ok; n++) {
    const uint32_t np = t->n_param[n];
    ok = t->alloc(&t->w[n], np, "alloc weights") && t->alloc(&t->wt[n], t->dims[n].t_size(), "alloc weights") &&
         t->alloc(&t->img[n], WImg(t->dims[n]).size, "alloc weights") &&
         t->alloc(&t->p[n], np, "alloc master weights") && t->alloc(&t->m[n], np, "alloc Adam moments") &&
         t->alloc(&t->v[n], np, "alloc Adam moments") &&
         t->alloc(&t->part[n], (size_t)t->max_tiles * part_stride(np), "alloc gradient partials") &&
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

}  // extern "C"

namespace {

// Per-kernel hipEvent time over one update (measurement only).
// An event-timed update: three events per minibatch (before the tile kernel,
// between the two kernels, after the Adam kernel), all recorded as the
// launches are queued and read after the update's final synchronisation, so
// no host wait falls between a launch and its events.
struct KernelTimes {
  std::vector<hipEvent_t> ev;
  double ms[2] = {0.0, 0.0};
  uint64_t launches = 0;
  ~KernelTimes() {
    for (auto e : ev) hipEventDestroy(e);
  }
};

int run_update(phz_train* t, const uint32_t* const* order, const uint64_t* order_lens, uint64_t n_order,
               const phz_ppo_cfg* cfg, phz_update_stats* out, KernelTimes* tm) {
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
  if (tm) {
    const uint64_t total = epochs * ((n + cfg->minibatch - 1) / cfg->minibatch);
    tm->ev.assign(4 * total, nullptr);
    for (auto& e : tm->ev)
      if (!t->hip_ok(hipEventCreate(&e), "hipEventCreate")) return 1;
  }
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
  uint64_t total = 0;  // minibatches this update can launch
  for (uint64_t e = 0; e < epochs; e++) total += (n + cfg->minibatch - 1) / cfg->minibatch;
  if (total + 1 > t->skip_cap) {
    if (t->skip) hipFree(t->skip);
    t->skip = nullptr;
    t->skip_cap = 0;
    if (!t->hip_ok(hipMalloc(&t->skip, (total + 1) * sizeof(int)), "alloc stop flags")) return 1;
    t->skip_cap = total + 1;
  }
  if (!t->hip_ok(hipMemsetAsync(t->state, 0, sizeof(UpdateState), t->stream), "reset update state") ||
      !t->hip_ok(hipMemsetAsync(t->skip, 0, (total + 1) * sizeof(int), t->stream), "reset stop flags"))
    return 1;

  TileArgs ta{};
  AdamArgs aa{};
  for (int k = 0; k < 2; k++) {
    ta.x[k] = t->obs[k];
    ta.w[k] = t->w[k];
    ta.wt[k] = t->wt[k];
    ta.img[k] = t->img[k];
    ta.part[k] = t->part[k];
    ta.dims[k] = t->dims[k];
    ta.n_param[k] = t->n_param[k];
    aa.part[k] = t->part[k];
    aa.p[k] = t->p[k];
    aa.m[k] = t->m[k];
    aa.v[k] = t->v[k];
    aa.w[k] = t->w[k];
    aa.wt[k] = t->wt[k];
    aa.img[k] = t->img[k];
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
  aa.stats_part = t->stats_part;
  aa.kl_mode = cfg->kl_mode;
  aa.kl_scale = cfg->kl_scale;
  aa.target_kl = cfg->target_kl;
  aa.st = t->state;
  const uint32_t n_all = part_stride(t->n_param[0]) + t->n_param[1];  // ppo_adam's parameter slots
  auto tiles_kernel = t->mode == STAGE_ALL ? ppo_tiles<STAGE_ALL>
                      : t->mode == STAGE_LAYER ? ppo_tiles<STAGE_LAYER> : ppo_tiles<STAGE_NONE>;
  uint64_t j = 0;  // minibatch counter within this update
  for (uint64_t e = 0; e < epochs; e++) {
    for (uint64_t s = 0; s < n; s += cfg->minibatch, j++) {
      const uint32_t b = (uint32_t)std::min<uint64_t>(cfg->minibatch, n - s);
      const uint32_t tiles = (b + t->R - 1) / t->R;
      ta.idx = t->order + e * n + s;
      ta.b = b;
      ta.skip = t->skip + j;
      aa.tiles = tiles;
      aa.b = b;
      aa.skip = t->skip + j;
      for (int k = 0; k < 2; k++) {
        // The step this minibatch would be, if it runs: every earlier one ran.
        aa.bc1[k] = 1.0 - powi(t->adam[k].beta1, t->t[k] + j + 1);
        aa.bc2[k] = 1.0 - powi(t->adam[k].beta2, t->t[k] + j + 1);
      }
      // Timed updates pass events to the launch itself: HIP stamps them with
      // the kernel's own start and end, so they measure its execution and not
      // the dispatch around it.
      hipEvent_t* ev = tm ? &tm->ev[4 * j] : nullptr;
      hipExtLaunchKernelGGL(tiles_kernel, dim3(tiles, 2), dim3(kTileThreads), (uint32_t)t->lds_bytes, t->stream,
                            ev ? ev[0] : nullptr, ev ? ev[1] : nullptr, 0u, ta);
      hipExtLaunchKernelGGL(ppo_adam, dim3((n_all * kAdamLanes + kAdamThreads - 1) / kAdamThreads), dim3(kAdamThreads),
                            0u, t->stream, ev ? ev[2] : nullptr, ev ? ev[3] : nullptr, 0u, aa);
    }
  }
  if (!t->hip_ok(hipGetLastError(), "launch update")) return 1;
  UpdateState st;
  if (!t->hip_ok(hipMemcpyAsync(&st, t->state, sizeof st, hipMemcpyDeviceToHost, t->stream), "read update state") ||
      !t->hip_ok(hipStreamSynchronize(t->stream), "update"))
    return 1;
  if (tm) {
    for (uint64_t i = 0; i < j; i++)
      for (int k = 0; k < 2; k++) {
        float ms = 0.0f;
        if (!t->hip_ok(hipEventElapsedTime(&ms, tm->ev[4 * i + 2 * k], tm->ev[4 * i + 2 * k + 1]), "time update")) return 1;
        tm->ms[k] += ms;
      }
    tm->launches = j;
  }
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

}  // namespace

extern "C" {

int phz_train_update(phz_train* t, const uint32_t* const* order, const uint64_t* order_lens, uint64_t n_order,
                     const phz_ppo_cfg* cfg, phz_update_stats* out) {
  return run_update(t, order, order_lens, n_order, cfg, out, nullptr);
}

int phz_train_time_update(phz_train* t, const uint32_t* const* order, const uint64_t* order_lens, uint64_t n_order,
                          const phz_ppo_cfg* cfg, phz_update_stats* out, double* ms_kernels, uint64_t* minibatches) {
  if (!t) return 1;
  if (!ms_kernels || !minibatches) return t->fail("null timing output");
  if (!set_device(t)) return 1;
  KernelTimes tm;
  const int rc = run_update(t, order, order_lens, n_order, cfg, out, &tm);
  for (int k = 0; k < 2; k++) ms_kernels[k] = tm.ms[k];
  *minibatches = tm.launches;
  return rc;
}

}  // extern "C"
