// Kernel instantiations for f32 q/k/v inputs.

#include "gdn_fwd_kernel.h"

namespace gdn {

int launch_f32(const KArgs& a, int K, int C, int bv, int grid, hipStream_t s) {
  return launch_k<float>(a, K, C, bv, grid, s);
}

}  // namespace gdn
