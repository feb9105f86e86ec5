// Split-codebook decode kernels with 3.5-bit keys (4 / 3 bits split at dim 64)
// and every value width (the kernel template and its design notes are in
// tq_decode_split.h); the dispatch over key widths.

#include "tq_decode_split.h"

namespace tq {

int launch_split_k7(const UniformArgs& a, int G, int vkind, int merge, hipStream_t s) {
  return launch_split_v<4, 3, false>(a, G, vkind, merge, s);
}

// kind = 2 * bits for fractional widths (3.5 -> 7, 2.5 -> 5), bits for integer ones
int launch_uniform_split(const UniformArgs& a, int G, int kkind, int vkind, int merge, hipStream_t s) {
  if (kkind == 7) return launch_split_k7(a, G, vkind, merge, s);
  if (kkind == 5) return launch_split_k5(a, G, vkind, merge, s);
  if (kkind >= 2 && kkind <= 4 && (vkind == 5 || vkind == 7)) return launch_split_ki(a, G, kkind, vkind, merge, s);
  return -1;
}

}  // namespace tq
