// Launcher declarations and parameter blocks shared by the C API and the
// kernel translation units.
#pragma once

#include "band.h"

namespace tension {

struct DecodeParams {
  Buf q, kn, vn, kc, vc, out, tau;
  const int32_t* pos_in;
  int32_t* pos_out;
  int N, H, D, W;
  double scale;
  float inv_scale;  // (float)(1 / scale)
  int flags;
};

struct RopeParams {
  Buf x, y;
  const float* cos;
  const float* sin;
  int B, T, H, D;
  int64_t pos_offset;
  int inverse;
};

// tau export reductions: up to kMaxLayers layers of tau [B, T, H, W] per call
constexpr int kMaxLayers = 32;

struct TauStatParams {
  Buf tau[kMaxLayers];
  float* stats;  // [L, H, 4]: mean, p99, peak_pos, concentration
  int L, B, T, H, W;
  int valid_only;
};

struct TauAggParams {
  Buf tau[kMaxLayers];
  const int32_t* mask;  // [L, H], nonzero = selected
  float* agg;           // [T, W]
  int L, B, T, H, W;
};

// graph-bias builder: content-pair hash table and bias fill
struct BiasTableParams {
  const unsigned long long* in_keys;
  const double* in_vals;
  int64_t n;
  unsigned long long* keys;  // [2^log2cap], empty = ~0
  double* vals;
  int log2cap;
};

struct BiasBuildParams {
  const int32_t* ids;  // [T] content ids, -1 = no edges
  const unsigned long long* keys;
  const double* vals;
  int log2cap;
  double alpha;
  void* out;            // [B, T, K], element strides os0, os1, 1
  int64_t os0, os1;
  int B, T, K;          // K = W (window) or T (global)
  int global;
  double* stats;        // [3] hits, weight sum, weight max (nullable)
};

// fused tau regularisers: per-row passes over up to kMaxLayers layers
struct AuxLossParams {
  Buf tau[kMaxLayers];
  Buf dtau[kMaxLayers];   // backward output
  double* acc;            // forward: [L, blocks, 4] partial sums
  const float* coef;      // backward: [L, 3] diversity, consistency, entropy
  int L, B, T, H, W;
};

// phase: 0 forward, 1 dQ, 2 dK/dV.  Return 0 when launched (HIP status in
// *err), -1 when no kernel exists for the request, kGridTooLarge when the
// grid would exceed 2^31 - 1 workgroups (band.h).
int launch_exact(int phase, bool f64, const BandParams& p, hipStream_t st, hipError_t* err);
int launch_mfma(int phase, const BandParams& p, hipStream_t st, hipError_t* err);
// decode step by flow: DECODE_EXACT (any dtype / head dim), or the fast
// kernel (head dim 64, W <= 1024) for bf16 throughout (DECODE_BF16), float32
// q / K / out with a bf16 V (DECODE_KF32), float32 throughout (DECODE_F32),
// float16 throughout (DECODE_F16)
enum { DECODE_EXACT = 0, DECODE_BF16 = 1, DECODE_KF32 = 2, DECODE_F32 = 3, DECODE_F16 = 4 };
int launch_decode(int flow, bool f64, const DecodeParams& p, hipStream_t st, hipError_t* err);
// split-operand kernels (split_band.h), by flow: SPLIT_FLOW_BF16 bf16
// throughout, SPLIT_FLOW_F32 float32 Q / K / dOut with a bfloat16 V,
// SPLIT_FLOW_F32V float32 Q / K / V / dOut, SPLIT_FLOW_F16 float16
// throughout; head dim 32 or 64; phase 0 forward, 1 dQ, 2 dK / dV
enum { SPLIT_FLOW_BF16 = 0, SPLIT_FLOW_F32 = 1, SPLIT_FLOW_F32V = 2, SPLIT_FLOW_F16 = 3 };
int launch_split(int phase, int flow, const BandParams& p, hipStream_t st, hipError_t* err);
// Compute units of the current device (queried once per device).
int device_cus();
int launch_rope(bool f64, const RopeParams& p, hipStream_t st, hipError_t* err);
// bf16 / float32 rows (x_f32, y_f32), D % 16 == 0, 16-byte aligned rows and tables
int launch_rope_vec(bool x_f32, bool y_f32, const RopeParams& p, hipStream_t st, hipError_t* err);
int launch_tau_stats(const TauStatParams& p, hipStream_t st, hipError_t* err);
int launch_tau_aggregate(const TauAggParams& p, hipStream_t st, hipError_t* err);
int launch_bias_insert(const BiasTableParams& p, hipStream_t st, hipError_t* err);
// rows per aux-loss workgroup, and the workgroups (partial-sum slots) per layer
constexpr int kAuxRowsPerBlock = 1024;
inline int64_t aux_loss_blocks(int64_t nrow) { return (nrow + kAuxRowsPerBlock - 1) / kAuxRowsPerBlock; }
int launch_aux_loss(bool bwd, const AuxLossParams& p, hipStream_t st, hipError_t* err);
int launch_bias_build(int out_dtype, const BiasBuildParams& p, hipStream_t st, hipError_t* err);

}  // namespace tension
