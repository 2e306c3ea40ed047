// Dispatch of the exact band kernels (instantiated in exact_<phase>_<acc>.hip).
#include "kernels.h"

namespace tension {

int launch_exact_fwd_f32(const BandParams&, hipStream_t, hipError_t*);
int launch_exact_dq_f32(const BandParams&, hipStream_t, hipError_t*);
int launch_exact_dkv_f32(const BandParams&, hipStream_t, hipError_t*);
int launch_exact_fwd_f64(const BandParams&, hipStream_t, hipError_t*);
int launch_exact_dq_f64(const BandParams&, hipStream_t, hipError_t*);
int launch_exact_dkv_f64(const BandParams&, hipStream_t, hipError_t*);

int launch_exact(int phase, bool f64, const BandParams& p, hipStream_t st, hipError_t* err) {
  switch (phase) {
    case 0: return f64 ? launch_exact_fwd_f64(p, st, err) : launch_exact_fwd_f32(p, st, err);
    case 1: return f64 ? launch_exact_dq_f64(p, st, err) : launch_exact_dq_f32(p, st, err);
    case 2: return f64 ? launch_exact_dkv_f64(p, st, err) : launch_exact_dkv_f32(p, st, err);
    default: return -1;
  }
}

}  // namespace tension
