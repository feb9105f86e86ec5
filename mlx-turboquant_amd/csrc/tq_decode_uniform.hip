// K4/V2 instantiations of the uniform-batch decode kernels (the kernel
// templates and their design notes are in tq_decode_uniform.h).

#include "tq_decode_uniform.h"

namespace tq {

template <int G, bool QB, bool BF>
static void launch_u(const UniformArgs& a, int merge, hipStream_t s) {
  if (a.bpw > FAST_WAVES * 4)
    hipLaunchKernelGGL((uk::uniform_decode_kernel<G, QB, 8, 4, 2, BF>), dim3(a.nwg, a.hkv, a.batch), dim3(uk::FT), 0,
                       s, a);
  else
    hipLaunchKernelGGL((uk::uniform_decode_kernel<G, QB, 4, 4, 2, BF>), dim3(a.nwg, a.hkv, a.batch), dim3(uk::FT), 0,
                       s, a);
  if (merge) hipLaunchKernelGGL((uk::uniform_merge_kernel<G>), dim3(a.hq, a.batch), dim3(uk::MT), 0, s, a);
}

template <bool BF>
static int launch_ub(const UniformArgs& a, int G, bool qb, int merge, hipStream_t s) {
  switch (G * 2 + (qb ? 1 : 0)) {
    case 2: launch_u<1, false, BF>(a, merge, s); break;
    case 3: launch_u<1, true, BF>(a, merge, s); break;
    case 4: launch_u<2, false, BF>(a, merge, s); break;
    case 5: launch_u<2, true, BF>(a, merge, s); break;
    case 8: launch_u<4, false, BF>(a, merge, s); break;
    case 9: launch_u<4, true, BF>(a, merge, s); break;
    case 16: launch_u<8, false, BF>(a, merge, s); break;
    case 17: launch_u<8, true, BF>(a, merge, s); break;
    default: return -1;
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_uniform_decode(const UniformArgs& a, int G, bool qb, int merge, hipStream_t s, bool bf16_kv) {
  return bf16_kv ? launch_ub<true>(a, G, qb, merge, s) : launch_ub<false>(a, G, qb, merge, s);
}

}  // namespace tq

