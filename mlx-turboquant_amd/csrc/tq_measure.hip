// Measurement hook of bench.py, not part of the ABI (include/tq_abi.h does not
// declare it): a streaming read of `bytes` bytes of device memory, the
// reference point for the decode kernels' achieved bandwidth on the same box.
// Each thread sums 16-byte pieces, four in flight per step (grid-strided, so
// every step reads one contiguous range of the buffer), and writes one float
// per workgroup so the loads cannot be dropped.

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int RT = 256;  // threads per workgroup
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(RT) void read_kernel(const v4u* __restrict__ src, size_t n16, float* out) {
  const size_t stride = (size_t)gridDim.x * RT;
  size_t i = (size_t)blockIdx.x * RT + threadIdx.x;
  uint32_t acc = 0;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const v4u a = __builtin_nontemporal_load(src + i);
    const v4u b = __builtin_nontemporal_load(src + i + stride);
    const v4u c = __builtin_nontemporal_load(src + i + 2 * stride);
    const v4u d = __builtin_nontemporal_load(src + i + 3 * stride);
    acc += (a.x ^ b.y) + (c.z ^ d.w) + (a.y ^ b.z) + (c.w ^ d.x) + (a.z ^ b.w) + (c.x ^ d.y) + (a.w ^ b.x) + (c.y ^ d.z);
  }
  for (; i < n16; i += stride) {
    const v4u a = src[i];
    acc += a.x + a.y + a.z + a.w;
  }
  __shared__ uint32_t red[RT / 64];
  for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) out[blockIdx.x] = (float)(red[0] + red[1] + red[2] + red[3]);
}

}  // namespace

extern "C" int tq_measure_read(const void* src, size_t bytes, float* out, int nwg, void* stream) {
  if (!src || !out || nwg <= 0 || (reinterpret_cast<uintptr_t>(src) & 15) || (bytes & 15)) return -1;
  hipLaunchKernelGGL(read_kernel, dim3(nwg), dim3(RT), 0, static_cast<hipStream_t>(stream),
                     static_cast<const v4u*>(src), bytes / 16, out);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}
