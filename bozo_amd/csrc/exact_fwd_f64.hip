// The exact band kernel of phase fwd with accumulator double (exact_launch).
#include "exact_impl.h"

namespace tension {

int launch_exact_fwd_f64(const BandParams& p, hipStream_t st, hipError_t* err) {
  return exact_launch<double, 0>(p, st, err);
}

}  // namespace tension
