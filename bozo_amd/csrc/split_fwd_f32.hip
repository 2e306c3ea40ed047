// Instantiates the split-operand band kernels (split_band.h) for phase
// fwd, float32 Q / K / dOut with a bf16 V (three bf16 terms per
// float32 value).
#include "split_band.h"

namespace tension {

void launch_split_fwd_f32(const BandParams& p, hipStream_t st, unsigned n) {
  split::launch<3, 1, 0>(p, st, n);
}

}  // namespace tension
