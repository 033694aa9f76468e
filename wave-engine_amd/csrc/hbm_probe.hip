// HBM read-stream calibration for the benchmark (not part of the attention
// ABI): the practical ceiling of a kernel that only reads, against which the
// decode split kernel (a read-only stream over the K/V cache) is compared.
// Each block streams chunks of U * 4 KB (U 16-byte loads in flight per
// thread), grid-stride over the buffer, and keeps a running sum, written once
// per thread at the end so the loads cannot be dropped.  The benchmark sweeps
// the unroll U, the grid and plain against non-temporal loads and keeps the
// fastest, so the ceiling is a property of the memory system rather than of
// one launch shape.
#include <hip/hip_runtime.h>

#include <cstddef>

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

// S = 2: the buffer is read as two halves at once (the U loads alternate
// between them), as the decode kernel reads its K and V streams.
template <int U, bool NT, int S>
__global__ __launch_bounds__(256) void read_stream_kernel(const f4* __restrict__ x, size_t n4,
                                                          float* __restrict__ out) {
  const size_t chunk = (size_t)U * 256;  // float4 per block and iteration (over the S streams)
  const size_t half = n4 / S;            // float4 per stream
  f4 acc[U];
#pragma unroll
  for (int u = 0; u < U; ++u) acc[u] = f4{0.f, 0.f, 0.f, 0.f};
  size_t c = (size_t)blockIdx.x * (chunk / S);
  for (; c + chunk / S <= half; c += (size_t)gridDim.x * (chunk / S)) {
    f4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const f4* p = x + (u % S) * half + c + threadIdx.x + 256 * (u / S);
      v[u] = NT ? __builtin_nontemporal_load(p) : *p;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc[u] += v[u];
  }
  // the tail of each stream (partial chunk), element by element
  for (int s = 0; s < S; ++s)
    for (size_t i = c + threadIdx.x; c < half && i < half && i < c + chunk / S; i += 256) acc[0] += x[s * half + i];
  f4 t = acc[0];
#pragma unroll
  for (int u = 1; u < U; ++u) t += acc[u];
  out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = (t.x + t.y) + (t.z + t.w);
}

template <int U, bool NT>
hipError_t launch(const void* x, size_t n4, float* out, int blocks, int streams, hipStream_t s) {
  if (streams == 2)
    hipLaunchKernelGGL((read_stream_kernel<U, NT, 2>), dim3((unsigned)blocks), dim3(256), 0, s,
                       static_cast<const f4*>(x), n4, out);
  else
    hipLaunchKernelGGL((read_stream_kernel<U, NT, 1>), dim3((unsigned)blocks), dim3(256), 0, s,
                       static_cast<const f4*>(x), n4, out);
  return hipGetLastError();
}

}  // namespace

extern "C" {

// Reads n4 float4 of x once with `unroll` (4, 8 or 16) loads in flight per
// thread, as one stream or two (the halves of x at once: streams = 2, n4
// even), non-temporal loads when nontemporal != 0; out holds blocks * 256
// floats.  Returns a hipError_t code.
int whp_read_stream_v(const void* x, size_t n4, float* out, int blocks, int unroll, int nontemporal, int streams,
                      void* stream) {
  if (x == nullptr || out == nullptr || blocks <= 0) return (int)hipErrorInvalidValue;
  if (streams != 1 && (streams != 2 || n4 % 2 != 0)) return (int)hipErrorInvalidValue;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool nt = nontemporal != 0;
  switch (unroll) {
    case 4:
      return (int)(nt ? launch<4, true>(x, n4, out, blocks, streams, s)
                      : launch<4, false>(x, n4, out, blocks, streams, s));
    case 8:
      return (int)(nt ? launch<8, true>(x, n4, out, blocks, streams, s)
                      : launch<8, false>(x, n4, out, blocks, streams, s));
    case 16:
      return (int)(nt ? launch<16, true>(x, n4, out, blocks, streams, s)
                      : launch<16, false>(x, n4, out, blocks, streams, s));
    default: return (int)hipErrorInvalidValue;
  }
}

// The eight-load plain single-stream form.
int whp_read_stream(const void* x, size_t n4, float* out, int blocks, void* stream) {
  return whp_read_stream_v(x, n4, out, blocks, 8, 0, 1, stream);
}

}  // extern "C"
