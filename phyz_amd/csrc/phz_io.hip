// phz_io.hip — state layout kernels (ahead-of-time compiled for gfx950).
//
// The C ABI hands over world-major f64 rows (the reference wire layout,
// crates/phyz-gpu/src/layout.rs:327-373); the step kernel keeps state as
// structure-of-arrays [j][stride] in the sim's precision so that lane-per-world
// loads and stores coalesce. These kernels convert between the two on device,
// so a host upload or readback is one contiguous copy plus one launch.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

namespace {

// dst[j * stride + w] = (T) src[w * width + j]
template <class T>
__global__ void pack_rows(const double* __restrict__ src, T* __restrict__ dst, int nworld, int width, int stride) {
  const int w = blockIdx.x * blockDim.x + threadIdx.x;
  if (w >= nworld) return;
  for (int j = 0; j < width; j++) dst[(size_t)j * stride + w] = (T)src[(size_t)w * width + j];
}

// dst[w * width + j] = (double) src[j * stride + w]
template <class T>
__global__ void unpack_rows(const T* __restrict__ src, double* __restrict__ dst, int nworld, int width, int stride) {
  const int w = blockIdx.x * blockDim.x + threadIdx.x;
  if (w >= nworld) return;
  for (int j = 0; j < width; j++) dst[(size_t)w * width + j] = (double)src[(size_t)j * stride + w];
}

template <class T> __global__ void fill_zero(T* __restrict__ dst, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = T(0);
}

// SplitMix64 world seeds (crates/phyz-gpu/src/policy_pipeline.rs:417-424).
__global__ void seed_worlds(uint64_t* __restrict__ rng, uint64_t seed, int nworld) {
  const int w = blockIdx.x * blockDim.x + threadIdx.x;
  if (w >= nworld) return;
  uint64_t z = seed + 0x9E3779B97F4A7C15ull * (uint64_t)(w + 1);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z = z ^ (z >> 31);
  rng[w] = z ? z : 1;
}

// dst[i] = src[i], 4-byte words (state snapshots; a kernel rather than a
// memcpy node so that a captured rollout holds only kernel nodes).
__global__ void copy_words(uint32_t* __restrict__ dst, const uint32_t* __restrict__ src, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = src[i];
}

constexpr int kBlock = 256;
inline int blocks(size_t n) { return (int)((n + kBlock - 1) / kBlock); }

constexpr size_t kScratchBytes = size_t(32) << 20;
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
std::mutex g_scratch_use[kMaxDevices];

}  // namespace

// Held by a caller across its whole use of device `dev`'s scratch array
// (stage, copy out, synchronize), so calls from several threads or sims on
// one GPU take turns instead of overwriting each other's rows.
std::mutex& phz_io_scratch_mutex(int dev) { return g_scratch_use[dev]; }

// Staging rows for callers that cannot allocate device memory
// (phz_readback_states_noalloc): 32 MiB per GPU, held until the process ends.
// Every call on a GPU shares that GPU's copy; callers serialize their use of
// it with phz_io_scratch_mutex. In host code `scratch` names a host-side stand-in, never the device
// memory: use the address phz_io_scratch returns.
static __device__ __align__(256) double scratch[kScratchBytes / sizeof(double)];

extern "C" {

hipError_t phz_io_pack(const double* src, void* dst, int nworld, int width, int stride, int f64, hipStream_t s) {
  if (nworld <= 0 || width <= 0) return hipSuccess;
  if (f64) hipLaunchKernelGGL(pack_rows<double>, dim3(blocks(nworld)), dim3(kBlock), 0, s, src, (double*)dst, nworld, width, stride);
  else hipLaunchKernelGGL(pack_rows<float>, dim3(blocks(nworld)), dim3(kBlock), 0, s, src, (float*)dst, nworld, width, stride);
  return hipGetLastError();
}

hipError_t phz_io_unpack(const void* src, double* dst, int nworld, int width, int stride, int f64, hipStream_t s) {
  if (nworld <= 0 || width <= 0) return hipSuccess;
  if (f64) hipLaunchKernelGGL(unpack_rows<double>, dim3(blocks(nworld)), dim3(kBlock), 0, s, (const double*)src, dst, nworld, width, stride);
  else hipLaunchKernelGGL(unpack_rows<float>, dim3(blocks(nworld)), dim3(kBlock), 0, s, (const float*)src, dst, nworld, width, stride);
  return hipGetLastError();
}

// Zero-fill with a kernel (no hipMemsetAsync, so a captured graph stays valid).
hipError_t phz_io_zero(void* dst, size_t bytes, hipStream_t s) {
  if (bytes == 0) return hipSuccess;
  const size_t n = bytes / 4;
  hipLaunchKernelGGL(fill_zero<uint32_t>, dim3(blocks(n)), dim3(kBlock), 0, s, (uint32_t*)dst, n);
  return hipGetLastError();
}

hipError_t phz_io_copy(void* dst, const void* src, size_t bytes, hipStream_t s) {
  if (bytes == 0) return hipSuccess;
  const size_t n = bytes / 4;
  hipLaunchKernelGGL(copy_words, dim3(blocks(n)), dim3(kBlock), 0, s, (uint32_t*)dst, (const uint32_t*)src, n);
  return hipGetLastError();
}

// The device address of the current device's scratch array, its size and the
// device's ordinal, looked up once per device (with that device current) and
// kept.
hipError_t phz_io_scratch(void** ptr, size_t* bytes, int* device) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  *bytes = kScratchBytes;
  *device = dev;
  return hipSuccess;
}

hipError_t phz_io_seed(uint64_t* rng, uint64_t seed, int nworld, hipStream_t s) {
  if (nworld <= 0) return hipSuccess;
  hipLaunchKernelGGL(seed_worlds, dim3(blocks(nworld)), dim3(kBlock), 0, s, rng, seed, nworld);
  return hipGetLastError();
}

}  // extern "C"
