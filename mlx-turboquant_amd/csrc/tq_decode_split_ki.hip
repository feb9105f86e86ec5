// Split-codebook decode kernels with integer keys (2-4 bits, one row per
// token) and fractional values (tq_decode_split.h).

#include "tq_decode_split.h"

namespace tq {

int launch_split_ki(const UniformArgs& a, int G, int kkind, int vkind, int merge, hipStream_t s) {
  switch (kkind) {
    case 2: return launch_split_v<2, 2, true>(a, G, vkind, merge, s);
    case 3: return launch_split_v<3, 3, true>(a, G, vkind, merge, s);
    case 4: return launch_split_v<4, 4, true>(a, G, vkind, merge, s);
    default: return -1;
  }
}

}  // namespace tq
