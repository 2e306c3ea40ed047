// Streaming decode step over a ring K/V cache, and the RoPE rotation.
//
// Decode is a pure HBM stream: every step reads the whole cache of each
// (sequence, head) once (2 * W * D * 2 bytes) and does 4*D flops per slot.
// One 8-wave workgroup owns one (n, h): every lane issues all of its cache
// loads before any arithmetic, eight lanes cover one 128-byte cache row (1 KB
// of contiguous cache per wave load instruction), and the sums are folded with
// DPP lane moves and one LDS pass.
#include "kernels.h"

namespace tension {

// Window slot w (0 = oldest) of ring slot `slot` when `pos` tokens are cached.
__device__ __forceinline__ int ring_w(int slot, int pos, int W) {
  int w = (slot - pos) % W;
  return w < 0 ? w + W : w;
}

// Normaliser of one decode output row: tau mass, number of keys, or 1.
__device__ __forceinline__ float decode_norm(int flags, float mass, int keys) {
  if (flags & TENSION_NORM_MASS) return 1.f / (mass > kMassEps ? mass : kMassEps);
  if (flags & TENSION_NORM_COUNT) return 1.f / (float)(keys > 1 ? keys : 1);
  return 1.f;
}

// Fast path: bf16 q / cache / out, D = 64, W <= 8 * NW * NP.
//
// NW waves per workgroup; pass i covers cache rows 8 * NW * i .. + 8 * NW - 1,
// eight lanes per 128-byte row, so each wave load instruction reads 1 KB of
// contiguous cache.  Every lane issues its NP K loads and NP V loads before
// any arithmetic, as raw buffer loads over the (n, h) slab of W rows: rows
// past W fall outside the descriptor's range and read as zero with no memory
// access, so no load sits behind a branch and the compiler waits for pass i
// alone (vmcnt) before computing on it.  The 8-lane row dot products reduce
// through DPP lane moves instead of LDS shuffles.
namespace {

constexpr int kRawBufWord3 = 0x00020000;  // raw 32-bit data format (buffer descriptor word 3)

// Cache rows are read once per step: non-temporal loads (buffer cache policy
// bit nt) keep them from displacing reusable lines in L2.
#ifdef TENSION_DECODE_TEMPORAL
constexpr int kCacheAux = 0;
#else
constexpr int kCacheAux = 2;
#endif

}  // namespace

// KF32: q, k_new, the K cache and out in float32 with a bf16 V cache (the
// reference's autocast dtype flow: rotated Q / K promoted to float32); a K
// row is then 256 bytes, two 16-byte loads per lane, and the dot products
// are float32 products.  Not with TENSION_DECODE_SELF.
// SELF: TENSION_DECODE_SELF (a compile-time choice: with the flag read at
// run time the compiler waited for the position counter, which only the
// self-key step's descriptor range needs, before issuing any cache load).
// Arguments of the fast kernel: row pointers and 32-bit element strides, 43
// dwords against the 96 of DecodeParams, so the kernel argument reads that
// precede the cache loads take fewer dependent rounds of scalar loads.  The
// host takes the fast path only when every stride fits in 32 bits.
struct DecodeFastArgs {
  const void* q;
  const void* kn;
  const void* vn;
  void* kc;
  void* vc;
  void* out;
  void* tau;
  const int32_t* pos_in;
  int32_t* pos_out;
  int q_n, q_h, kn_n, kn_h, vn_n, vn_h;
  int kc_n, kc_h, kc_w, vc_n, vc_h, vc_w;
  int out_n, out_h, tau_n, tau_h, tau_dt;
  int H, W, flags;
  float inv_scale;
};

// FLOW (the element types of one step): kDecodeBF16 -- bf16 throughout;
// kDecodeKF32 -- float32 q / K / out, bf16 V (KF32 above); kDecodeF32 --
// float32 throughout (the reference's flow without autocast: V rows of 256
// bytes too); kDecodeF16 -- float16 throughout (the bf16 layout, float16
// arithmetic conversions).  SELF with bf16 or float16 only.
enum { kDecodeBF16 = 0, kDecodeKF32 = 1, kDecodeF32 = 2, kDecodeF16 = 3 };

template <int NW, int NP, int FLOW, bool SELF>
__device__ __forceinline__ void decode_d64_body(const DecodeFastArgs& p) {
  constexpr bool KF32 = FLOW == kDecodeKF32 || FLOW == kDecodeF32;
  constexpr bool VF32 = FLOW == kDecodeF32;
  constexpr bool H16 = FLOW == kDecodeF16;  // the 16-bit element is float16
  static_assert(!(SELF && KF32), "the self-key step takes 16-bit rows");
  constexpr int kRows = 8 * NW;  // cache rows per pass
  constexpr int kKBytes = KF32 ? 4 : 2;   // bytes per K / q / out element
  constexpr int kKChunks = KF32 ? 16 : 8;  // 16-byte chunks of a K row
  constexpr int kVBytes = VF32 ? 4 : 2;   // bytes per V element
  constexpr int kVChunks = VF32 ? 16 : 8;  // 16-byte chunks of a V row
  using VE = typename std::conditional<VF32, float, bf16>::type;  // V addressing (16-bit: bf16 or float16)
  __shared__ float red[NW * 4][64];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int ch = lane & 7, rw = lane >> 3;  // d-chunk, row within a pass
  const int n = blockIdx.x / p.H, h = blockIdx.x % p.H;
  const int W = p.W;

  // this lane's 8 query features (8 ch .. +7)
  u16x8 qbits, qbits2;
  if constexpr (KF32) {
    const float* qrow = (const float*)p.q + (int64_t)n * p.q_n + (int64_t)h * p.q_h + 8 * ch;
    qbits = *(const u16x8*)qrow;
    qbits2 = *(const u16x8*)(qrow + 4);
  } else {
    const bf16* qrow = (const bf16*)p.q + (int64_t)n * p.q_n + (int64_t)h * p.q_h;
    qbits = *(const u16x8*)(qrow + 8 * ch);
  }
  // The new token's K / V rows are appended after the reduction, but fetched
  // now so their latency hides under the cache stream: lanes a = tid - 64 in
  // [0, kKChunks) hold 16-byte chunk a of k_new, the next 8 chunk
  // a - kKChunks of v_new.  The descriptors span one row; every other lane's
  // offset is out of range and reads zero without a memory access, so the
  // loads need no branch.
  const int ai = tid - 64;
  const __amdgpu_buffer_rsrc_t knr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const char*)p.kn + ((int64_t)n * p.kn_n + (int64_t)h * p.kn_h) * kKBytes), (short)0, 16 * kKChunks,
      kRawBufWord3);
  const __amdgpu_buffer_rsrc_t vnr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const VE*)p.vn + (int64_t)n * p.vn_n + (int64_t)h * p.vn_h), (short)0, 16 * kVChunks, kRawBufWord3);
  const u16x8 knew = __builtin_bit_cast(u16x8, __builtin_amdgcn_raw_buffer_load_b128(
      knr, (ai >= 0 && ai < kKChunks) ? 16 * ai : 16 * kKChunks, 0, 0));
  const u16x8 vnew = __builtin_bit_cast(u16x8, __builtin_amdgcn_raw_buffer_load_b128(
      vnr, (ai >= kKChunks && ai < kKChunks + kVChunks) ? 16 * (ai - kKChunks) : 16 * kVChunks, 0, 0));

  // One descriptor per cache slab; loads of rows past its range return
  // zeros.  The range is W rows, or, for a self-key step (a global layer's
  // cache, filled from slot 0 and never wrapped), the live rows only: that
  // cache is long and partly empty, and the position read it needs first
  // costs little there.  Window caches keep the loads ahead of that read.
  constexpr bool self_key = SELF;
  int rows = W;
  if (self_key) {
    const int pe = p.pos_in[n] > 0 ? p.pos_in[n] : 0;
    rows = pe < W ? pe : W;
  }
  const char* kbase = (const char*)p.kc + ((int64_t)n * p.kc_n + (int64_t)h * p.kc_h) * kKBytes;
  const VE* vbase = (const VE*)p.vc + (int64_t)n * p.vc_n + (int64_t)h * p.vc_h;
  const __amdgpu_buffer_rsrc_t kr_ = __builtin_amdgcn_make_buffer_rsrc(
      (void*)kbase, (short)0, (int)((int64_t)rows * p.kc_w * kKBytes), kRawBufWord3);
  const __amdgpu_buffer_rsrc_t vr_ = __builtin_amdgcn_make_buffer_rsrc(
      (void*)vbase, (short)0, (int)((int64_t)rows * p.vc_w * kVBytes), kRawBufWord3);
  const uint32_t row0 = (uint32_t)(wave * 8 + rw);
  const uint32_t kstep = (uint32_t)(kRows * p.kc_w * kKBytes), vstep = (uint32_t)(kRows * p.vc_w * kVBytes);
  const uint32_t koff = row0 * (uint32_t)(p.kc_w * kKBytes) + 8 * kKBytes * ch;
  const uint32_t voff = row0 * (uint32_t)(p.vc_w * kVBytes) + 8 * kVBytes * ch;
  u16x8 kr[NP], kr2[KF32 ? NP : 1], vr[NP], vr2[VF32 ? NP : 1];
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    kr[i] = __builtin_bit_cast(u16x8, __builtin_amdgcn_raw_buffer_load_b128(kr_, (int)(koff + i * kstep), 0, kCacheAux));
    if constexpr (KF32)
      kr2[i] = __builtin_bit_cast(u16x8, __builtin_amdgcn_raw_buffer_load_b128(kr_, (int)(koff + i * kstep + 16), 0,
                                                                               kCacheAux));
  }
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    vr[i] = __builtin_bit_cast(u16x8, __builtin_amdgcn_raw_buffer_load_b128(vr_, (int)(voff + i * vstep), 0, kCacheAux));
    if constexpr (VF32)
      vr2[i] = __builtin_bit_cast(u16x8, __builtin_amdgcn_raw_buffer_load_b128(vr_, (int)(voff + i * vstep + 16), 0,
                                                                               kCacheAux));
  }

  const int pos = p.pos_in[n] > 0 ? p.pos_in[n] : 0;
  const int live = pos < W ? pos : W;  // slots [0, live) hold tokens
  // Whole-vector bit casts only: a bit cast of one subscripted vector
  // element (bit_cast<bf16>(v[i])) compiles to element 0 for every i.
  float q[8];
  if constexpr (KF32) {
    const f32x4 qa = __builtin_bit_cast(f32x4, qbits), qb = __builtin_bit_cast(f32x4, qbits2);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      q[e] = qa[e] * p.inv_scale;
      q[4 + e] = qb[e] * p.inv_scale;
    }
  } else if constexpr (H16) {
    const f16x8 qv = __builtin_bit_cast(f16x8, qbits);
#pragma unroll
    for (int e = 0; e < 8; ++e) q[e] = (float)qv[e] * p.inv_scale;
  } else {
    const bf16x8 qv = __builtin_bit_cast(bf16x8, qbits);
#pragma unroll
    for (int e = 0; e < 8; ++e) q[e] = (float)qv[e] * p.inv_scale;
  }
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float msum = 0.f;
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int slot = i * kRows + (int)row0;
    float part = 0.f;
    if constexpr (KF32) {
      const f32x4 ka = __builtin_bit_cast(f32x4, kr[i]), kb = __builtin_bit_cast(f32x4, kr2[i]);
#pragma unroll
      for (int e = 0; e < 4; ++e) part += q[e] * ka[e] + q[4 + e] * kb[e];
    } else if constexpr (H16) {
      const f16x8 kv = __builtin_bit_cast(f16x8, kr[i]);
#pragma unroll
      for (int e = 0; e < 8; ++e) part += q[e] * (float)kv[e];
    } else {
      const bf16x8 kv = __builtin_bit_cast(bf16x8, kr[i]);
#pragma unroll
      for (int e = 0; e < 8; ++e) part += q[e] * (float)kv[e];
    }
    part = row_sum8(part);
    const float tau = slot < live ? sigmoid_fast(part) : 0.f;
    if (p.tau && ch == 0 && slot < W) {
      const int64_t to = (int64_t)n * p.tau_n + (int64_t)h * p.tau_h + ring_w(slot, pos, W);
      switch (p.tau_dt) {
        case TENSION_F32: ((float*)p.tau)[to] = tau; break;
        case TENSION_BF16: ((bf16*)p.tau)[to] = (bf16)tau; break;
        case TENSION_F16: ((f16*)p.tau)[to] = (f16)tau; break;
        default: ((double*)p.tau)[to] = (double)tau; break;
      }
    }
    msum += tau;
    if constexpr (VF32) {
      const f32x4 va = __builtin_bit_cast(f32x4, vr[i]), vb = __builtin_bit_cast(f32x4, vr2[i]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[e] += tau * va[e];
        acc[4 + e] += tau * vb[e];
      }
    } else if constexpr (H16) {
      const f16x8 vv = __builtin_bit_cast(f16x8, vr[i]);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += tau * (float)vv[e];
    } else {
      const bf16x8 vv = __builtin_bit_cast(bf16x8, vr[i]);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += tau * (float)vv[e];
    }
  }
  // TENSION_DECODE_SELF: the new token is a key too (global layers attend to
  // s <= t).  Wave 1 holds its k row in lanes 0-7 and its v row in lanes
  // 8-15 (chunk = lane & 7, the same chunk of q each lane holds): lanes 0-7
  // form the dot, lanes 8-15 take its sigmoid through the row rotate and
  // scale their v chunk; the results meet the cache sums in LDS.
  __shared__ float sred[65];
  if (!KF32 && self_key && wave == 1) {
    float kx[8], vx[8];
    if constexpr (H16) {
      const f16x8 kv = __builtin_bit_cast(f16x8, knew), vv = __builtin_bit_cast(f16x8, vnew);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        kx[e] = (float)kv[e];
        vx[e] = (float)vv[e];
      }
    } else {
      const bf16x8 kv = __builtin_bit_cast(bf16x8, knew), vv = __builtin_bit_cast(bf16x8, vnew);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        kx[e] = (float)kv[e];
        vx[e] = (float)vv[e];
      }
    }
    float part = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) part += q[e] * kx[e];
    const float ts = sigmoid_fast(row_sum8(part));
    const float tv = dpp_move<0x128>(ts);  // lanes 8-15 <- lanes 0-7
    if (lane >= 8 && lane < 16) {
#pragma unroll
      for (int e = 0; e < 8; ++e) sred[8 * (lane - 8) + e] = tv * vx[e];
    }
    if (lane == 0) sred[64] = ts;
  }
  // Fold row pairs (lanes 8 apart) with a DPP rotate; then lane ch of every
  // 16-lane row holds the sums over rows rw = 2r, 2r + 1 of its wave, and the
  // NW * 4 row partials meet in LDS.  tau, hence msum, is equal on the 8 lanes
  // of a row, so one lane per 16-lane row stores it.
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] += dpp_move<0x128>(acc[e]);  // row_ror:8
  msum += dpp_move<0x128>(msum);
  __shared__ float mred[NW * 4];
  if ((lane & 8) == 0) {
    const int r = wave * 4 + (lane >> 4);
#pragma unroll
    for (int e = 0; e < 8; ++e) red[r][8 * ch + e] = acc[e];
    if (ch == 0) mred[r] = msum;
  }
  __syncthreads();  // every cache read of this (n, h) is complete past here
  if (tid < 64) {
    float o = 0.f, m = 0.f;
#pragma unroll
    for (int r = 0; r < NW * 4; ++r) {
      o += red[r][tid];
      m += mred[r];
    }
    if (self_key) {
      o += sred[tid];
      m += sred[64];
    }
    const float inv = decode_norm(p.flags, m, live + (self_key ? 1 : 0));
    if constexpr (KF32) {
      ((float*)p.out)[(int64_t)n * p.out_n + (int64_t)h * p.out_h + tid] = o * inv;
    } else if constexpr (H16) {
      f16* orow = (f16*)p.out + (int64_t)n * p.out_n + (int64_t)h * p.out_h;
      orow[tid] = (f16)(o * inv);
    } else {
      bf16* orow = (bf16*)p.out + (int64_t)n * p.out_n + (int64_t)h * p.out_h;
      orow[tid] = (bf16)(o * inv);
    }
  } else if (ai < kKChunks + kVChunks) {
    // append k_new / v_new at slot pos % W (16 bytes per lane)
    const int slot = pos % W;
    if (ai < kKChunks) {
      char* dst = (char*)p.kc + ((int64_t)n * p.kc_n + (int64_t)h * p.kc_h + (int64_t)slot * p.kc_w) * kKBytes;
      *(u16x8*)(dst + 16 * ai) = knew;
    } else {
      VE* dst = (VE*)p.vc + (int64_t)n * p.vc_n + (int64_t)h * p.vc_h + (int64_t)slot * p.vc_w;
      *(u16x8*)(dst + (16 / kVBytes) * (ai - kKChunks)) = vnew;
    }
  } else if (ai == kKChunks + kVChunks && h == 0 && p.pos_out) {
    p.pos_out[n] = pos + 1;
  }
}

template <int NW, int NP, bool KF32 = false, bool SELF = false>
__global__ __launch_bounds__(64 * NW) void decode_bf16_d64(DecodeFastArgs p) {
  decode_d64_body<NW, NP, KF32 ? kDecodeKF32 : kDecodeBF16, SELF>(p);
}

// The fast path for the float32 (FLOW kDecodeF32) and float16 (kDecodeF16)
// flows.
template <int NW, int NP, int FLOW, bool SELF = false>
__global__ __launch_bounds__(64 * NW) void decode_d64(DecodeFastArgs p) {
  decode_d64_body<NW, NP, FLOW, SELF>(p);
}

// Exact path: any dtype, any D <= 256, any W; one thread per (n, h).  The
// thread reads every slot before it overwrites slot pos % W, so the
// read-before-write order holds within the thread.
template <typename A>
__global__ __launch_bounds__(64) void decode_exact(DecodeParams p) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= p.N * p.H) return;
  const int n = idx / p.H, h = idx % p.H;
  const int pos = p.pos_in[n] > 0 ? p.pos_in[n] : 0;
  const int W = p.W, D = p.D;
  const A scale = (A)p.scale;
  A acc[256];
  for (int d = 0; d < D; ++d) acc[d] = A(0);
  A msum = A(0);
  const int64_t qo = n * p.q.s0 + h * p.q.s1;
  for (int slot = 0; slot < W; ++slot) {
    const bool ok = pos >= W || slot < pos;
    A tau = A(0);
    if (ok) {
      const int64_t ko = n * p.kc.s0 + h * p.kc.s1 + (int64_t)slot * p.kc.s2;
      const int64_t vo = n * p.vc.s0 + h * p.vc.s1 + (int64_t)slot * p.vc.s2;
      A dot = A(0);
      for (int d = 0; d < D; ++d) dot += ld<A>(p.q, qo + d) * ld<A>(p.kc, ko + d);
      tau = sigmoid_exact(dot / scale);
      for (int d = 0; d < D; ++d) acc[d] += tau * ld<A>(p.vc, vo + d);
    }
    msum += tau;
    if (p.tau.p) st<A>(p.tau, n * p.tau.s0 + h * p.tau.s1 + ring_w(slot, pos, W), tau);
  }
  const int64_t no = n * p.kn.s0 + h * p.kn.s1;
  const int64_t nvo = n * p.vn.s0 + h * p.vn.s1;
  const bool self_key = (p.flags & TENSION_DECODE_SELF) != 0;
  if (self_key) {  // the new token as a key (s <= t)
    A dot = A(0);
    for (int d = 0; d < D; ++d) dot += ld<A>(p.q, qo + d) * ld<A>(p.kn, no + d);
    const A tau = sigmoid_exact(dot / scale);
    for (int d = 0; d < D; ++d) acc[d] += tau * ld<A>(p.vn, nvo + d);
    msum += tau;
  }
  A inv = A(1);
  if (p.flags & TENSION_NORM_MASS) {
    inv = A(1) / (msum > A(kMassEps) ? msum : A(kMassEps));
  } else if (p.flags & TENSION_NORM_COUNT) {
    const int keys = (pos < W ? pos : W) + (self_key ? 1 : 0);
    inv = A(1) / A(keys > 1 ? keys : 1);
  }
  const int64_t oo = n * p.out.s0 + h * p.out.s1;
  for (int d = 0; d < D; ++d) st<A>(p.out, oo + d, acc[d] * inv);
  const int slot = pos % W;
  const int64_t ko = n * p.kc.s0 + h * p.kc.s1 + (int64_t)slot * p.kc.s2;
  const int64_t vo = n * p.vc.s0 + h * p.vc.s1 + (int64_t)slot * p.vc.s2;
  for (int d = 0; d < D; ++d) {
    st<A>(p.kc, ko + d, ld<A>(p.kn, no + d));
    st<A>(p.vc, vo + d, ld<A>(p.vn, nvo + d));
  }
  if (h == 0 && p.pos_out) p.pos_out[n] = pos + 1;
}

namespace {

bool fits32(int64_t s) { return s >= 0 && s <= 0x7fffffff; }

// The fast kernel's arguments, or false when a stride needs 64 bits.
bool fast_args(const DecodeParams& p, DecodeFastArgs* a) {
  const int64_t st[] = {p.q.s0, p.q.s1, p.kn.s0, p.kn.s1, p.vn.s0, p.vn.s1, p.kc.s0, p.kc.s1, p.kc.s2,
                        p.vc.s0, p.vc.s1, p.vc.s2, p.out.s0, p.out.s1, p.tau.s0, p.tau.s1};
  for (int64_t x : st)
    if (!fits32(x)) return false;
  a->q = p.q.p; a->kn = p.kn.p; a->vn = p.vn.p;
  a->kc = (void*)p.kc.p; a->vc = (void*)p.vc.p; a->out = (void*)p.out.p; a->tau = (void*)p.tau.p;
  a->pos_in = p.pos_in; a->pos_out = p.pos_out;
  a->q_n = (int)p.q.s0; a->q_h = (int)p.q.s1; a->kn_n = (int)p.kn.s0; a->kn_h = (int)p.kn.s1;
  a->vn_n = (int)p.vn.s0; a->vn_h = (int)p.vn.s1;
  a->kc_n = (int)p.kc.s0; a->kc_h = (int)p.kc.s1; a->kc_w = (int)p.kc.s2;
  a->vc_n = (int)p.vc.s0; a->vc_h = (int)p.vc.s1; a->vc_w = (int)p.vc.s2;
  a->out_n = (int)p.out.s0; a->out_h = (int)p.out.s1;
  a->tau_n = (int)p.tau.s0; a->tau_h = (int)p.tau.s1; a->tau_dt = p.tau.dt;
  a->H = p.H; a->W = p.W; a->flags = p.flags; a->inv_scale = p.inv_scale;
  return true;
}

}  // namespace

int launch_decode(int flow, bool f64, const DecodeParams& p_in, hipStream_t st, hipError_t* err) {
  DecodeFastArgs p;
  bool fast = flow != DECODE_EXACT && !(flow == DECODE_F32 && p_in.W > 512);
  if (fast && !fast_args(p_in, &p)) fast = false;
  const bool kf32 = fast && flow == DECODE_KF32;
  if (fast && (flow == DECODE_F32 || flow == DECODE_F16)) {
    // float32 throughout (no self key; W <= 512: sixteen passes of float32
    // K and V rows would not fit the registers), or float16 throughout
    // (W <= 1024); D == 64
    const dim3 grid((unsigned)(p_in.N * p_in.H));
#define DECODE_WIDE(FL, SELF, TOP)                                                         \
  do {                                                                                     \
    if (p.W <= 32)                                                                         \
      hipLaunchKernelGGL((decode_d64<4, 1, FL, SELF>), grid, dim3(256), 0, st, p);         \
    else if (p.W <= 64)                                                                    \
      hipLaunchKernelGGL((decode_d64<8, 1, FL, SELF>), grid, dim3(512), 0, st, p);         \
    else if (p.W <= 128)                                                                   \
      hipLaunchKernelGGL((decode_d64<8, 2, FL, SELF>), grid, dim3(512), 0, st, p);         \
    else if (p.W <= 256)                                                                   \
      hipLaunchKernelGGL((decode_d64<4, 8, FL, SELF>), grid, dim3(256), 0, st, p);         \
    else if (p.W <= 512 || TOP == 8)                                                       \
      hipLaunchKernelGGL((decode_d64<8, 8, FL, SELF>), grid, dim3(512), 0, st, p);         \
    else                                                                                   \
      hipLaunchKernelGGL((decode_d64<8, TOP, FL, SELF>), grid, dim3(512), 0, st, p);       \
  } while (0)
    if (flow == DECODE_F32) {
      DECODE_WIDE(kDecodeF32, false, 8);
    } else if (p.flags & TENSION_DECODE_SELF) {
      DECODE_WIDE(kDecodeF16, true, 16);
    } else {
      DECODE_WIDE(kDecodeF16, false, 16);
    }
#undef DECODE_WIDE
  } else if (fast && kf32) {
    // float32 q / K / out, bf16 V (D == 64, W <= 1024, no self key)
    const dim3 grid((unsigned)(p_in.N * p_in.H));
    if (p.W <= 32)
      hipLaunchKernelGGL((decode_bf16_d64<4, 1, true>), grid, dim3(256), 0, st, p);
    else if (p.W <= 64)
      hipLaunchKernelGGL((decode_bf16_d64<8, 1, true>), grid, dim3(512), 0, st, p);
    else if (p.W <= 128)
      hipLaunchKernelGGL((decode_bf16_d64<8, 2, true>), grid, dim3(512), 0, st, p);
    else if (p.W <= 256)
      hipLaunchKernelGGL((decode_bf16_d64<8, 4, true>), grid, dim3(512), 0, st, p);
    else if (p.W <= 512)
      hipLaunchKernelGGL((decode_bf16_d64<8, 8, true>), grid, dim3(512), 0, st, p);
    else
      hipLaunchKernelGGL((decode_bf16_d64<8, 16, true>), grid, dim3(512), 0, st, p);
  } else if (fast) {
    // fast requires D == 64, W <= 1024
    const dim3 grid((unsigned)(p_in.N * p_in.H));
#define DECODE_FAST(SELF)                                                                    \
  do {                                                                                       \
    if (p.W <= 32)                                                                           \
      hipLaunchKernelGGL((decode_bf16_d64<4, 1, false, SELF>), grid, dim3(256), 0, st, p);  \
    else if (p.W <= 64)                                                                      \
      hipLaunchKernelGGL((decode_bf16_d64<8, 1, false, SELF>), grid, dim3(512), 0, st, p);  \
    else if (p.W <= 128)                                                                     \
      hipLaunchKernelGGL((decode_bf16_d64<8, 2, false, SELF>), grid, dim3(512), 0, st, p);  \
    else if (p.W <= 256) /* 4 waves x 8 passes: 2% faster than 8 x 4 at config 4 */         \
      hipLaunchKernelGGL((decode_bf16_d64<4, 8, false, SELF>), grid, dim3(256), 0, st, p);  \
    else if (p.W <= 512)                                                                     \
      hipLaunchKernelGGL((decode_bf16_d64<8, 8, false, SELF>), grid, dim3(512), 0, st, p);  \
    else                                                                                     \
      hipLaunchKernelGGL((decode_bf16_d64<8, 16, false, SELF>), grid, dim3(512), 0, st, p); \
  } while (0)
    if (p.flags & TENSION_DECODE_SELF) DECODE_FAST(true);
    else DECODE_FAST(false);
#undef DECODE_FAST
  } else {
    const unsigned grid = (unsigned)((p_in.N * p_in.H + 63) / 64);
    if (f64)
      hipLaunchKernelGGL(decode_exact<double>, dim3(grid), dim3(64), 0, st, p_in);
    else
      hipLaunchKernelGGL(decode_exact<float>, dim3(grid), dim3(64), 0, st, p_in);
  }
  *err = hipGetLastError();
  return 0;
}

// ------------------------------------------------------------------ RoPE

// y[i]      = x[i] cos - x[i+half] sin      (model.py:81)
// y[i+half] = x[i] sin + x[i+half] cos
// inverse: the transpose (rotation by -theta).  One thread per (row, i<half);
// each thread reads both halves before writing, so y may alias x.
template <typename A>
__global__ __launch_bounds__(256) void rope_kernel(RopeParams p) {
  const int half = p.D >> 1;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)p.B * p.T * p.H * half;
  if (idx >= total) return;
  const int i = (int)(idx % half);
  int64_t r = idx / half;
  const int h = (int)(r % p.H);
  r /= p.H;
  const int t = (int)(r % p.T);
  const int b = (int)(r / p.T);
  const int64_t xo = b * p.x.s0 + (int64_t)t * p.x.s1 + h * p.x.s2;
  const int64_t yo = b * p.y.s0 + (int64_t)t * p.y.s1 + h * p.y.s2;
  const int64_t to = (p.pos_offset + t) * half + i;
  const A c = (A)p.cos[to], s = p.inverse ? -(A)p.sin[to] : (A)p.sin[to];
  const A x1 = ld<A>(p.x, xo + i), x2 = ld<A>(p.x, xo + i + half);
  st<A>(p.y, yo + i, x1 * c - x2 * s);
  st<A>(p.y, yo + i + half, x1 * s + x2 * c);
}

// bf16 / float32 in and out (the four pairs), D a multiple of 16, 16-byte
// aligned rows and tables: one thread rotates 8 pairs (16 or 32 bytes of each
// half, 32 bytes of each table row), so a row of D = 64 is 4 consecutive
// threads reading whole 16-byte pieces.  float32 arithmetic, as rope_kernel;
// both halves are read before either is written (y may alias x).
template <typename T>
__device__ __forceinline__ void rope_load8(const T* p, float* v) {
  if constexpr (sizeof(T) == 2) {
    const bf16x8 x = __builtin_bit_cast(bf16x8, *(const u16x8*)p);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (float)x[e];
  } else {
    const f32x4 x0 = *(const f32x4*)p, x1 = *(const f32x4*)(p + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = x0[e];
      v[4 + e] = x1[e];
    }
  }
}

template <typename T>
__device__ __forceinline__ void rope_store8(T* p, const float* v) {
  if constexpr (sizeof(T) == 2) {
    bf16x8 y;
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = (bf16)v[e];
    *(u16x8*)p = __builtin_bit_cast(u16x8, y);
  } else {
    *(f32x4*)p = f32x4{v[0], v[1], v[2], v[3]};
    *(f32x4*)(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
  }
}

template <typename XT, typename YT>
__global__ __launch_bounds__(256) void rope_vec(RopeParams p) {
  const int half = p.D >> 1, nq = half >> 3;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)p.B * p.T * p.H * nq;
  if (idx >= total) return;
  const int q = (int)(idx % nq);
  int64_t r = idx / nq;
  const int h = (int)(r % p.H);
  r /= p.H;
  const int t = (int)(r % p.T);
  const int b = (int)(r / p.T);
  const XT* xr = (const XT*)p.x.p + b * p.x.s0 + (int64_t)t * p.x.s1 + h * p.x.s2 + 8 * q;
  YT* yr = (YT*)p.y.p + b * p.y.s0 + (int64_t)t * p.y.s1 + h * p.y.s2 + 8 * q;
  float x1[8], x2[8], y1[8], y2[8];
  rope_load8(xr, x1);
  rope_load8(xr + half, x2);
  const int64_t to = (p.pos_offset + t) * half + 8 * q;
  const f32x4 c0 = *(const f32x4*)(p.cos + to), c1 = *(const f32x4*)(p.cos + to + 4);
  const f32x4 s0 = *(const f32x4*)(p.sin + to), s1 = *(const f32x4*)(p.sin + to + 4);
  const float sg = p.inverse ? -1.f : 1.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float c = e < 4 ? c0[e & 3] : c1[e & 3];
    const float sn = sg * (e < 4 ? s0[e & 3] : s1[e & 3]);
    y1[e] = x1[e] * c - x2[e] * sn;
    y2[e] = x1[e] * sn + x2[e] * c;
  }
  rope_store8(yr, y1);
  rope_store8(yr + half, y2);
}

int launch_rope_vec(bool x_f32, bool y_f32, const RopeParams& p, hipStream_t st, hipError_t* err) {
  const int64_t total = (int64_t)p.B * p.T * p.H * (p.D / 16);
  const dim3 grid((unsigned)((total + 255) / 256));
  if (x_f32) {
    if (y_f32) hipLaunchKernelGGL((rope_vec<float, float>), grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((rope_vec<float, bf16>), grid, dim3(256), 0, st, p);
  } else {
    if (y_f32) hipLaunchKernelGGL((rope_vec<bf16, float>), grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((rope_vec<bf16, bf16>), grid, dim3(256), 0, st, p);
  }
  *err = hipGetLastError();
  return 0;
}

int launch_rope(bool f64, const RopeParams& p, hipStream_t st, hipError_t* err) {
  const int64_t total = (int64_t)p.B * p.T * p.H * (p.D / 2);
  const unsigned grid = (unsigned)((total + 255) / 256);
  if (f64)
    hipLaunchKernelGGL(rope_kernel<double>, dim3(grid), dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL(rope_kernel<float>, dim3(grid), dim3(256), 0, st, p);
  *err = hipGetLastError();
  return 0;
}

}  // namespace tension
