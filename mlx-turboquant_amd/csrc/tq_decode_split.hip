// Fractional-width instantiations of the uniform-batch decode kernels (key
// and value codebooks split at dim 64: 4 / 3 bits for 3.5, 3 / 2 for 2.5; the
// kernel template and its design notes are in tq_decode_split.h).

#include "tq_decode_split.h"

namespace tq {

template <int G, int KH, int VH>
static void launch_s(const UniformArgs& a, int merge, hipStream_t s) {
  if (a.bpw > FAST_WAVES * 4)
    hipLaunchKernelGGL((uk::split_decode_kernel<G, 8, KH, KH - 1, VH, VH - 1>), dim3(a.nwg, a.hkv, a.batch),
                       dim3(uk::FT), 0, s, a);
  else
    hipLaunchKernelGGL((uk::split_decode_kernel<G, 4, KH, KH - 1, VH, VH - 1>), dim3(a.nwg, a.hkv, a.batch),
                       dim3(uk::FT), 0, s, a);
  if (merge) hipLaunchKernelGGL((uk::uniform_merge_kernel<G>), dim3(a.hq, a.batch), dim3(uk::MT), 0, s, a);
}

template <int KH, int VH>
static int launch_skv(const UniformArgs& a, int G, int merge, hipStream_t s) {
  switch (G) {
    case 1: launch_s<1, KH, VH>(a, merge, s); break;
    case 2: launch_s<2, KH, VH>(a, merge, s); break;
    case 4: launch_s<4, KH, VH>(a, merge, s); break;
    case 8: launch_s<8, KH, VH>(a, merge, s); break;
    default: return -1;
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_uniform_split(const UniformArgs& a, int G, int kh, int vh, int merge, hipStream_t s) {
  switch (kh * 8 + vh) {
    case 4 * 8 + 4: return launch_skv<4, 4>(a, G, merge, s);
    case 4 * 8 + 3: return launch_skv<4, 3>(a, G, merge, s);
    case 3 * 8 + 4: return launch_skv<3, 4>(a, G, merge, s);
    case 3 * 8 + 3: return launch_skv<3, 3>(a, G, merge, s);
    default: return -1;
  }
}

}  // namespace tq
