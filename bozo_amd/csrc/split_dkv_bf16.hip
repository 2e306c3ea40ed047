// Instantiates the split-operand band kernels (split_band.h) for phase
// dkv, bf16 operands (one term).
#include "split_band.h"

namespace tension {

void launch_split_dkv_bf16(const BandParams& p, hipStream_t st, unsigned n) {
  split::launch<1, 1, 2>(p, st, n);
}

}  // namespace tension
