// Uniform-batch decode kernels for the integer widths other than K4/V2 (key
// and value bits in 2..4): the templates of tq_decode_uniform.h with their
// width parameters, and the same merge kernel.

#include "tq_decode_uniform.h"

namespace tq {

template <int G, int KB, int VB>
static void launch_w(const UniformArgs& a, int merge, hipStream_t s) {
  if (a.bpw > FAST_WAVES * 4)
    hipLaunchKernelGGL((uk::uniform_decode_kernel<G, false, 8, KB, VB>), dim3(a.nwg, a.hkv, a.batch), dim3(uk::FT), 0,
                       s, a);
  else
    hipLaunchKernelGGL((uk::uniform_decode_kernel<G, false, 4, KB, VB>), dim3(a.nwg, a.hkv, a.batch), dim3(uk::FT), 0,
                       s, a);
  if (merge) hipLaunchKernelGGL((uk::uniform_merge_kernel<G>), dim3(a.hq, a.batch), dim3(uk::MT), 0, s, a);
}

template <int KB, int VB>
static int launch_kv(const UniformArgs& a, int G, int merge, hipStream_t s) {
  switch (G) {
    case 1: launch_w<1, KB, VB>(a, merge, s); break;
    case 2: launch_w<2, KB, VB>(a, merge, s); break;
    case 4: launch_w<4, KB, VB>(a, merge, s); break;
    case 8: launch_w<8, KB, VB>(a, merge, s); break;
    default: return -1;
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_uniform_widths(const UniformArgs& a, int G, int kb, int vb, int merge, hipStream_t s) {
  switch (kb * 8 + vb) {
    case 2 * 8 + 2: return launch_kv<2, 2>(a, G, merge, s);
    case 2 * 8 + 3: return launch_kv<2, 3>(a, G, merge, s);
    case 2 * 8 + 4: return launch_kv<2, 4>(a, G, merge, s);
    case 3 * 8 + 2: return launch_kv<3, 2>(a, G, merge, s);
    case 3 * 8 + 3: return launch_kv<3, 3>(a, G, merge, s);
    case 3 * 8 + 4: return launch_kv<3, 4>(a, G, merge, s);
    case 4 * 8 + 3: return launch_kv<4, 3>(a, G, merge, s);
    case 4 * 8 + 4: return launch_kv<4, 4>(a, G, merge, s);
    default: return -1;
  }
}

}  // namespace tq
