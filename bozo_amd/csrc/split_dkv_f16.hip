// Instantiates the split-operand band kernels (split_band.h) for phase
// dkv, float16 Q / K / V / dOut (two bf16 terms per value).
#include "split_band.h"

namespace tension {

void launch_split_dkv_f16(const BandParams& p, hipStream_t st, unsigned n) {
  split::launch<2, 2, 2>(p, st, n);
}

}  // namespace tension
