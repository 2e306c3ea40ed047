// Instantiates the split-operand band kernels (split_band.h) for phase
// dq, float32 Q / K / V / dOut (three bf16 terms per value).
#include "split_band.h"

namespace tension {

void launch_split_dq_f32v(const BandParams& p, hipStream_t st, unsigned n) {
  split::launch<3, 3, 1>(p, st, n);
}

}  // namespace tension
