// Instantiates the exact band kernels for accumulator float and phase fwd.
#include "exact_impl.h"

namespace tension {

template <int D>
static void launch_d(const BandParams& p, hipStream_t st, unsigned grid) {
  hipLaunchKernelGGL((exact_fwd<float, D>), dim3(grid), dim3(128), 0, st, p);
}

int launch_exact_fwd_f32(const BandParams& p, hipStream_t st, hipError_t* err) {
  const int64_t total = (int64_t)p.B * p.H * p.T;
  if ((total + 127) / 128 > 0x7fffffff) return kGridTooLarge;
  const unsigned grid = (unsigned)((total + 127) / 128);
  switch (p.D) {
    case 8: launch_d<8>(p, st, grid); break;
    case 16: launch_d<16>(p, st, grid); break;
    case 32: launch_d<32>(p, st, grid); break;
    case 64: launch_d<64>(p, st, grid); break;
    case 128: launch_d<128>(p, st, grid); break;
    default: return -1;
  }
  *err = hipGetLastError();
  return 0;
}

}  // namespace tension
