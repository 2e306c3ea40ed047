// The exact band kernel of phase fwd with accumulator float (exact_launch).
#include "exact_impl.h"

namespace tension {

int launch_exact_fwd_f32(const BandParams& p, hipStream_t st, hipError_t* err) {
  return exact_launch<float, 0>(p, st, err);
}

}  // namespace tension
