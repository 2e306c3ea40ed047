// Dispatch of the bf16 MFMA band kernels (mfma_fwd.hip, mfma_dq.hip,
// mfma_dkv.hip): grid size and the normalisation mode of the template.
#include <atomic>

#include "mfma_common.h"

namespace tension {

void launch_mfma_fwd(const BandParams& p, hipStream_t st, unsigned nwg, int norm);
void launch_mfma_dq(const BandParams& p, hipStream_t st, unsigned nwg, int norm);
void launch_mfma_dkv(const BandParams& p, hipStream_t st, unsigned nwg, int norm);
void launch_mfma_bwd_fused(const BandParams& p, hipStream_t st, unsigned nwg, int norm);

// Workgroups the fused backward aims for per CU: two resident (76 KB of LDS
// each).
#ifndef TENSION_BWD_WG_PER_CU
#define TENSION_BWD_WG_PER_CU 2
#endif

// Compute units of the current device (256 on MI355X), queried once per
// device: the band kernels' grids are sized to whole rounds of resident
// workgroups.
int device_cus() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

int launch_mfma(int phase, const BandParams& p_in, hipStream_t st, hipError_t* err) {
  BandArgs probe;
  if (!band_args(p_in, &probe)) return -1;  // the kernels take 32-bit strides
  BandParams p = p_in;
  p.ntiles = (p.T + kTile - 1) / kTile;
  const int64_t nwg = (int64_t)p.B * p.H * p.ntiles;
  // ring kernels: consecutive tiles per workgroup, sized so the grid still
  // offers about three workgroups per CU
  const int64_t cus = device_cus();
  p.chunk = 1;
#ifdef TENSION_FWD_CHUNK
  p.chunk = TENSION_FWD_CHUNK;
#else
  while (p.chunk < 4 && (int64_t)p.B * p.H * ((p.ntiles + 2 * p.chunk - 1) / (2 * p.chunk)) >= 3 * cus)
    p.chunk *= 2;
#endif
  if (nwg <= 0) return -1;
  if (nwg > 0x7fffffff) return kGridTooLarge;
  const int norm = (p.flags & TENSION_NORM_MASS)    ? NORM_MASS_
                   : (p.flags & TENSION_NORM_COUNT) ? NORM_COUNT_
                                                    : NORM_RAW;
  if (phase == 3) {
    // fused backward (local window <= 64): p.chunk = runs of tiles per (b,h)
    const int64_t bh = (int64_t)p.B * p.H;
    int64_t runs = (TENSION_BWD_WG_PER_CU * cus + bh / 2) / bh;
    if (runs < 1) runs = 1;
    if (runs > p.ntiles) runs = p.ntiles;
    if (bh * runs > 0x7fffffff) return kGridTooLarge;
    p.chunk = (int)runs;
    launch_mfma_bwd_fused(p, st, (unsigned)(bh * runs), norm);
    *err = hipGetLastError();
    return 0;
  }
  switch (phase) {
    case 0: launch_mfma_fwd(p, st, (unsigned)nwg, norm); break;
    case 1: launch_mfma_dq(p, st, (unsigned)nwg, norm); break;
    case 2: launch_mfma_dkv(p, st, (unsigned)nwg, norm); break;
    default: return -1;
  }
  *err = hipGetLastError();
  return 0;
}

}  // namespace tension
