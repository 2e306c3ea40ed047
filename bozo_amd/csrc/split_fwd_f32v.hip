// Instantiates the split-operand band kernels (split_band.h) for phase
// fwd, float32 Q / K / V / dOut (three bf16 terms per value).
#include "split_band.h"

namespace tension {

void launch_split_fwd_f32v(const BandParams& p, hipStream_t st, unsigned n) {
  split::launch<3, 3, 0>(p, st, n);
}

}  // namespace tension
