// Instantiates the split-operand band kernels (split_band.h) for phase
// dkv, float32 Q / K / V / dOut (three bf16 terms per value).
#include "split_band.h"

namespace tension {

void launch_split_dkv_f32v(const BandParams& p, hipStream_t st, unsigned n) {
  split::launch<3, 3, 2>(p, st, n);
}

}  // namespace tension
