// MFMA / VALU overlap probe on gfx950 (a design measurement, not part of the
// library; build with `make probe`).
// 256 workgroups of W waves (W = 4: one wave per SIMD; W = 8: two per SIMD).
// Per loop iteration each wave runs 4 groups of {1 MFMA 16x16x32 f16, K VALU}
// (the order pinned with sched_group_barrier), or only the MFMAs, or only the
// VALU ops. VALU ops: independent fp32 FMA chains (F) or integer v_perm/xor
// chains (P). Prints microseconds per launch.
#include <hip/hip_runtime.h>
#include <stdio.h>
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
constexpr int IT = 1024;

template <int MODE, int K, bool INT>
__global__ void k(float* out, float s) {
  half8 a, b;
  for (int e = 0; e < 8; ++e) { a[e] = (_Float16)(s * (threadIdx.x + e)); b[e] = (_Float16)(s * e); }
  f4 c[4];
  for (int j = 0; j < 4; ++j) c[j] = f4{0.f, 0.f, 0.f, 0.f};
  float x[8];
  uint32_t u[8];
  for (int j = 0; j < 8; ++j) { x[j] = s * (threadIdx.x + j); u[j] = threadIdx.x * 2654435761u + j; }
  const float y = s * 0.5f, z = s * 0.25f;
  const uint32_t sel = 0x05040100u + (threadIdx.x & 3);
  for (int it = 0; it < IT; ++it) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      if (MODE != 1) c[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c[g], 0, 0, 0);
      if (MODE != 0) {
#pragma unroll
        for (int v = 0; v < K; ++v) {
          const int j = (g * K + v) & 7;
          if (INT) u[j] = __builtin_amdgcn_perm(u[j], u[(j + 1) & 7], sel) ^ (uint32_t)it;
          else x[j] = fmaf(x[j], y, z);
        }
      }
      if (MODE == 2) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, INT ? 2 * K : K, 0);
      }
    }
  }
  float r = 0.f;
  for (int j = 0; j < 4; ++j) r += c[j][0] + c[j][1] + c[j][2] + c[j][3];
  for (int j = 0; j < 8; ++j) r += x[j] + (float)u[j];
  out[blockIdx.x * blockDim.x + threadIdx.x] = r;
}

template <int MODE, int K, bool INT>
float run(float* out, int waves) {
  hipEvent_t e0, e1;
  (void)hipEventCreate(&e0);
  (void)hipEventCreate(&e1);
  for (int i = 0; i < 3; ++i) hipLaunchKernelGGL((k<MODE, K, INT>), dim3(256), dim3(64 * waves), 0, 0, out, 1e-3f);
  (void)hipEventRecord(e0);
  for (int i = 0; i < 10; ++i) hipLaunchKernelGGL((k<MODE, K, INT>), dim3(256), dim3(64 * waves), 0, 0, out, 1e-3f);
  (void)hipEventRecord(e1);
  (void)hipEventSynchronize(e1);
  float ms;
  (void)hipEventElapsedTime(&ms, e0, e1);
  return ms * 100.f;
}

template <int K, bool INT>
void row(float* out, int waves) {
  const float m = run<0, K, INT>(out, waves), v = run<1, K, INT>(out, waves), b = run<2, K, INT>(out, waves);
  printf("waves/SIMD %d  %s K=%d per MFMA: MFMA only %7.1f us  VALU only %7.1f us  interleaved %7.1f us  "
         "(sum %7.1f, max %7.1f)  overlap %.0f%%\n",
         waves / 4, INT ? "perm+xor" : "fma     ", K, m, v, b, m + v, m > v ? m : v,
         100.f * (m + v - b) / (m < v ? m : v));
}

int main() {
  float* out;
  (void)hipMalloc(&out, 256 * 512 * 4);
  for (int waves : {4, 8}) {
    row<1, false>(out, waves);
    row<2, false>(out, waves);
    row<4, false>(out, waves);
    row<8, false>(out, waves);
    row<1, true>(out, waves);
    row<2, true>(out, waves);
    row<4, true>(out, waves);
  }
  (void)hipFree(out);
  return 0;
}
