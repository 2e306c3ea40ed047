// The exact band kernel of phase dkv with accumulator float (exact_launch).
#include "exact_impl.h"

namespace tension {

int launch_exact_dkv_f32(const BandParams& p, hipStream_t st, hipError_t* err) {
  return exact_launch<float, 2>(p, st, err);
}

}  // namespace tension
