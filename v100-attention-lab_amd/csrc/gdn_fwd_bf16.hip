// Kernel instantiations for bf16 q/k/v inputs.

#include "gdn_fwd_kernel.h"
#include "gdn_fwd_pipe.h"

namespace gdn {

int launch_bf16(const KArgs& a, int K, int C, int bv, int grid, hipStream_t s) {
  return launch_k<bf16_t>(a, K, C, bv, grid, s);
}

int launch_pipe_bf16(const KArgs& a, int K, int bv, int grid, hipStream_t s) {
  return launch_pipe_k<bf16_t>(a, K, bv, grid, s);
}

}  // namespace gdn
