// HBM read-stream calibration for the benchmark (not part of the attention
// ABI): the practical ceiling of a kernel that only reads, against which the
// decode split kernel (a read-only stream over the K/V cache) is compared.
// Each thread streams 16-byte loads grid-stride over the buffer and keeps a
// running sum, written once at the end so the loads cannot be dropped.
#include <hip/hip_runtime.h>

#include <cstddef>

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void read_stream_kernel(const f4* __restrict__ x, size_t n4,
                                                          float* __restrict__ out) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  f4 a = {0.f, 0.f, 0.f, 0.f}, b = a;
  // two loads in flight per iteration
  for (; i + stride < n4; i += 2 * stride) {
    const f4 u = x[i];
    const f4 v = x[i + stride];
    a += u;
    b += v;
  }
  if (i < n4) {
    const f4 u = x[i];
    a += u;
  }
  out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = (a.x + a.y) + (a.z + a.w) + (b.x + b.y) + (b.z + b.w);
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
