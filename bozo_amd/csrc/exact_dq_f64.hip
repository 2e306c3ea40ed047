// The exact band kernel of phase dq with accumulator double (exact_launch).
#include "exact_impl.h"

namespace tension {

int launch_exact_dq_f64(const BandParams& p, hipStream_t st, hipError_t* err) {
  return exact_launch<double, 1>(p, st, err);
}

}  // namespace tension
