// HBM read-stream calibration for the benchmark (not part of the attention
// ABI): the practical ceiling of a kernel that only reads, against which the
// decode split kernel (a read-only stream over the K/V cache) is compared.
// Each block streams 32 KB chunks (eight 16-byte loads in flight per thread),
// grid-stride over the buffer, and keeps a running sum, written once per
// thread at the end so the loads cannot be dropped.
#include <hip/hip_runtime.h>

#include <cstddef>

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void read_stream_kernel(const f4* __restrict__ x, size_t n4,
                                                          float* __restrict__ out) {
  // block-contiguous 32 KB chunks (8 loads of 16 B in flight per thread), grid-stride over chunks
  constexpr int U = 8;
  const size_t chunk = (size_t)U * 256;
  f4 acc[U];
#pragma unroll
  for (int u = 0; u < U; ++u) acc[u] = f4{0.f, 0.f, 0.f, 0.f};
  size_t c = (size_t)blockIdx.x * chunk;
  for (; c + chunk <= n4; c += (size_t)gridDim.x * chunk) {
    f4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = x[c + threadIdx.x + 256 * u];
#pragma unroll
    for (int u = 0; u < U; ++u) acc[u] += v[u];
  }
  // the tail chunk (partial), element by element
  for (size_t i = c + threadIdx.x; c < n4 && i < n4 && i < c + chunk; i += 256) acc[0] += x[i];
  f4 t = acc[0];
#pragma unroll
  for (int u = 1; u < U; ++u) t += acc[u];
  out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = (t.x + t.y) + (t.z + t.w);
}

}  // namespace

extern "C" {

// Reads n4 float4 of x once; out holds blocks * 256 floats.  Returns a
// hipError_t code.
int whp_read_stream(const void* x, size_t n4, float* out, int blocks, void* stream) {
  if (x == nullptr || out == nullptr || blocks <= 0) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(read_stream_kernel, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const f4*>(x), n4, out);
  return (int)hipGetLastError();
}

}  // extern "C"
