// Instantiates the split-operand band kernels (split_band.h) for phase
// dq, float16 Q / K / V / dOut (two bf16 terms per value).
#include "split_band.h"

namespace tension {

void launch_split_dq_f16(const BandParams& p, hipStream_t st, unsigned n) {
  split::launch<2, 2, 1>(p, st, n);
}

}  // namespace tension
