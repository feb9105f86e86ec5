// Shared device/host helpers for the TurboQuant HIP library (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/tq_abi.h"

namespace tq {

// Records a message for tq_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...);

// Validates a codec description on the host. Returns TQ_OK or an error code.
int check_codec(const tq_codec* c);

// Bytes of one packed row for `dims` codes at `bits` bits.
__host__ __device__ inline int row_bytes(int dims, int bits) { return dims * bits / 8; }

// Writes 32 codes of `BITS` bits as a little-endian LSB-first bitstream into
// BITS consecutive dwords: code k occupies bits [BITS*k, BITS*k + BITS).
template <int BITS>
__device__ inline void pack32(const uint32_t (&code)[32], uint32_t (&w)[BITS]) {
#pragma unroll
  for (int i = 0; i < BITS; ++i) w[i] = 0u;
#pragma unroll
  for (int k = 0; k < 32; ++k) {
    const int p = BITS * k;
    w[p >> 5] |= code[k] << (p & 31);
    if ((p & 31) + BITS > 32) w[(p >> 5) + 1] |= code[k] >> (32 - (p & 31));
  }
}

// Inverse of pack32.
template <int BITS>
__device__ inline void unpack32(const uint32_t (&w)[BITS], uint32_t (&code)[32]) {
  constexpr uint32_t mask = (1u << BITS) - 1u;
#pragma unroll
  for (int k = 0; k < 32; ++k) {
    const int p = BITS * k;
    uint32_t v = w[p >> 5] >> (p & 31);
    if ((p & 31) + BITS > 32) v |= w[(p >> 5) + 1] << (32 - (p & 31));
    code[k] = v & mask;
  }
}

__device__ inline float half_bits_to_float(uint16_t h) {
  return __half2float(__ushort_as_half(h));
}

// Element i of a TQ_F16 / TQ_BF16 / TQ_F32 array as float32 (exact).
__device__ inline float load_elem(const void* p, int64_t i, int dtype) {
  if (dtype == TQ_F32) return static_cast<const float*>(p)[i];
  const uint16_t h = static_cast<const uint16_t*>(p)[i];
  if (dtype == TQ_BF16) return __uint_as_float(static_cast<uint32_t>(h) << 16);
  return half_bits_to_float(h);
}

inline int dtype_bytes(int dtype) { return dtype == TQ_F32 ? 4 : 2; }

}  // namespace tq

#define TQ_LAUNCH_CHECK(name)                                                  \
  do {                                                                         \
    hipError_t _e = hipGetLastError();                                         \
    if (_e != hipSuccess)                                                      \
      return tq::set_error(TQ_ERR_LAUNCH, "%s launch failed: %s", name,        \
                           hipGetErrorString(_e));                             \
  } while (0)
