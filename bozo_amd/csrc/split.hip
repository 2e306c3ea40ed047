// Dispatch of the split-operand band kernels (split_band.h): grid size and
// the per-phase, per-precision instantiation units.
#include "kernels.h"

namespace tension {

void launch_split_fwd_bf16(const BandParams& p, hipStream_t st, unsigned n);
void launch_split_dq_bf16(const BandParams& p, hipStream_t st, unsigned n);
void launch_split_dkv_bf16(const BandParams& p, hipStream_t st, unsigned n);
void launch_split_fwd_f32(const BandParams& p, hipStream_t st, unsigned n);
void launch_split_dq_f32(const BandParams& p, hipStream_t st, unsigned n);
void launch_split_dkv_f32(const BandParams& p, hipStream_t st, unsigned n);
void launch_split_fwd_f32v(const BandParams& p, hipStream_t st, unsigned n);
void launch_split_dq_f32v(const BandParams& p, hipStream_t st, unsigned n);
void launch_split_dkv_f32v(const BandParams& p, hipStream_t st, unsigned n);
void launch_split_fwd_f16(const BandParams& p, hipStream_t st, unsigned n);
void launch_split_dq_f16(const BandParams& p, hipStream_t st, unsigned n);
void launch_split_dkv_f16(const BandParams& p, hipStream_t st, unsigned n);

int launch_split(int phase, int flow, const BandParams& p_in, hipStream_t st, hipError_t* err) {
  if (flow < SPLIT_FLOW_BF16 || flow > SPLIT_FLOW_F16) return -1;
  if (phase < 0 || phase > 2) return -1;
  BandArgs probe;
  if (!band_args(p_in, &probe)) return -1;  // the kernels take 32-bit strides
  BandParams p = p_in;
  if (p.D != 32 && p.D != 64) return -1;
  p.ntiles = (p.T + 63) / 64;
  int64_t nwg = (int64_t)p.B * p.H * p.ntiles;
  if (nwg <= 0) return -1;
  if (nwg > 0x7fffffff) return kGridTooLarge;
  // p.chunk > 0: runs of consecutive tiles per workgroup (p.chunk runs per
  // (b, h)) for a local window W <= 64: the forward, sized for about three
  // resident workgroups per CU, and the backward kernels for about two: dK /
  // dV except with a float32 V at head dim 64 (there its run kernel holds
  // 272 registers, one wave per SIMD, and one tile per workgroup measured
  // faster: 134 against 142 us per float32 step at B8 H12 T1024 W64), dQ
  // for float32 Q / K with a bf16 V at head dim 32 without dTau (where its
  // run kernel measured faster); 0: one tile per workgroup
  p.chunk = 0;
  const bool dq_runs = flow == SPLIT_FLOW_F32 && p.D == 32 && p.dtau.p == nullptr;
  const bool dkv_runs = !(flow == SPLIT_FLOW_F32V && p.D == 64);
  if ((phase == 0 || (phase == 2 && dkv_runs) || (phase == 1 && dq_runs)) && !p.glob && p.win >= 1 &&
      p.win <= 64) {
    const int64_t bh = (int64_t)p.B * p.H;
    const int64_t per_cu = phase == 0 ? 3 : 2;
    int64_t runs = (per_cu * (int64_t)device_cus() + bh / 2) / bh;
    if (runs < 1) runs = 1;
    if (runs < p.ntiles) {
      p.chunk = (int)runs;
      nwg = bh * runs;
    }
  }
  const unsigned n = (unsigned)nwg;
  typedef void (*Launch)(const BandParams&, hipStream_t, unsigned);
  static const Launch table[4][3] = {
      {launch_split_fwd_bf16, launch_split_dq_bf16, launch_split_dkv_bf16},
      {launch_split_fwd_f32, launch_split_dq_f32, launch_split_dkv_f32},
      {launch_split_fwd_f32v, launch_split_dq_f32v, launch_split_dkv_f32v},
      {launch_split_fwd_f16, launch_split_dq_f16, launch_split_dkv_f16}};
  table[flow][phase](p, st, n);
  *err = hipGetLastError();
  return 0;
}

}  // namespace tension
