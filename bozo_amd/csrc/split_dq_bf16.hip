// Instantiates the split-operand band kernels (split_band.h) for phase
// dq, bf16 operands (one term).
#include "split_band.h"

namespace tension {

void launch_split_dq_bf16(const BandParams& p, hipStream_t st, unsigned n) {
  split::launch<1, 1, 1>(p, st, n);
}

}  // namespace tension
