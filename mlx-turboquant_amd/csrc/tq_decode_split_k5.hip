// Split-codebook decode kernels with 2.5-bit keys (3 / 2 bits split at dim 64)
// and every value width (tq_decode_split.h).

#include "tq_decode_split.h"

namespace tq {

int launch_split_k5(const UniformArgs& a, int G, int vkind, int merge, hipStream_t s) {
  return launch_split_v<3, 2, false>(a, G, vkind, merge, s);
}

}  // namespace tq
