// Instantiates the split-operand band kernels (split_band.h) for phase
// fwd, bf16 operands (one term).
#include "split_band.h"

namespace tension {

void launch_split_fwd_bf16(const BandParams& p, hipStream_t st, unsigned n) {
  split::launch<1, 1, 0>(p, st, n);
}

}  // namespace tension
