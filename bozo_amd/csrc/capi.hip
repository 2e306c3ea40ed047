// extern "C" entry points of libtension_hip.so: argument validation,
// kernel selection (MFMA bf16 path or exact path) and error reporting.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "kernels.h"

using namespace tension;

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int ok() {
  g_err.clear();
  return TENSION_OK;
}

int launched(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(TENSION_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return ok();
}

#define TRY(x)         \
  do {                 \
    int _r = (x);      \
    if (_r) return _r; \
  } while (0)

bool dtype_ok(int dt) { return dt >= TENSION_F32 && dt <= TENSION_F64; }

// A required or optional tensor; `unit` is the index of the stride that must
// be 1 (the innermost one), or -1.
int check_buf(const tension_buf* b, const char* what, bool required, int unit) {
  if (!b) return required ? fail(TENSION_ERR_ARG, "%s is required", what) : 0;
  if (!b->ptr) return fail(TENSION_ERR_ARG, "%s: null data pointer", what);
  if (!dtype_ok(b->dtype)) return fail(TENSION_ERR_ARG, "%s: bad dtype code %d", what, b->dtype);
  if (unit >= 0 && b->s[unit] != 1)
    return fail(TENSION_ERR_ARG, "%s: innermost stride must be 1 (got %lld)", what, (long long)b->s[unit]);
  return 0;
}

bool is_f64(const tension_buf* b) { return b && b->dtype == TENSION_F64; }

// Kernels that address one (b, h) sequence through a 32-bit buffer view need
// every row offset up to T + 128 rows to fit in 32 bits.
bool rows_fit_u32(const tension_buf* b, int64_t T) {
  return b && rows_fit_view(T + 128, b->s[1]);
}

bool any_f64(const tension_buf* a, const tension_buf* b, const tension_buf* c) {
  return is_f64(a) || is_f64(b) || is_f64(c);
}

bool aligned_rows16(const tension_buf* b, int32_t dtype) {
  if (!b || b->dtype != dtype) return false;
  if (((uintptr_t)b->ptr & 15) != 0) return false;
  return (b->s[0] % 8 == 0) && (b->s[1] % 8 == 0) && (b->s[2] % 8 == 0);
}

bool aligned_bf16_rows(const tension_buf* b) { return aligned_rows16(b, TENSION_BF16); }
bool aligned_f16_rows(const tension_buf* b) { return aligned_rows16(b, TENSION_F16); }

hipStream_t hs(tension_stream_t s) { return (hipStream_t)s; }

struct Shape {
  int64_t B, T, H, D;
};

// Shape and scale checks; sets *empty when there is nothing to compute (then
// the data pointers are not inspected: an empty tensor may have none).
int check_shape(Shape sh, double scale, bool* empty) {
  if (sh.B < 0 || sh.T < 0 || sh.H < 0 || sh.D <= 0)
    return fail(TENSION_ERR_ARG, "bad shape B=%lld T=%lld H=%lld D=%lld", (long long)sh.B, (long long)sh.T,
                (long long)sh.H, (long long)sh.D);
  constexpr int64_t kMaxRows = (int64_t)1 << 40;
  if (sh.T > 0x3fffffff || sh.H > 0x3fffffff || sh.B > 0x3fffffff || sh.D > 0x3fffffff ||
      mul_cap(mul_cap(sh.B, sh.H, kMaxRows), sh.T, kMaxRows) < 0)
    return fail(TENSION_ERR_ARG, "shape too large");
  if (!(std::isfinite(scale) && scale != 0.0)) return fail(TENSION_ERR_ARG, "scale must be finite and non-zero");
  *empty = sh.B * sh.H * sh.T == 0;
  return 0;
}

BandParams band_common(Shape sh, double scale, int flags) {
  BandParams p;
  memset(&p, 0, sizeof p);
  p.B = (int)sh.B;
  p.T = (int)sh.T;
  p.H = (int)sh.H;
  p.D = (int)sh.D;
  p.scale = scale;
  p.flags = flags;
  return p;
}

void set_local(BandParams& p, int64_t W) {
  p.win = (int)W;
  p.diag = 0;
  p.glob = 0;
  p.W = (int)W;
  p.Wtau = (int)W;
}

void set_global(BandParams& p, int64_t Wl) {
  p.win = p.T + 1;
  p.diag = 1;
  p.glob = 1;
  p.W = 0;
  p.Wtau = (int)Wl;
}

// 16-byte aligned float32 rows (head dim multiple of 4, unit innermost stride)
bool aligned_f32_rows(const tension_buf* b) {
  if (!b || b->dtype != TENSION_F32) return false;
  if (((uintptr_t)b->ptr & 15) != 0) return false;
  return (b->s[0] % 4 == 0) && (b->s[1] % 4 == 0) && (b->s[2] % 4 == 0);
}

// Split-operand MFMA kernels (split_band.h), head dim 32 or 64, any window,
// local or global, every float32 value carried as three bf16 terms:
// float32 Q / K with a bfloat16 V -- the reference's autocast flow,
// float32 out / dOut / dQ / dK, bf16 dV -- (SPLIT_F32), float32 throughout
// (SPLIT_F32V), float16 throughout as two terms per value (SPLIT_F16), or
// bf16 everywhere (SPLIT_BF16) for what the dedicated bf16 kernels (head
// dim 64) do not take.
enum { SPLIT_NONE = 0, SPLIT_BF16 = 1, SPLIT_F32 = 2, SPLIT_F32V = 3, SPLIT_F16 = 4 };

int split_kind(const tension_buf* q, const tension_buf* k, const tension_buf* v, const tension_buf* bias,
               int64_t D, int flags) {
  if ((flags & TENSION_FORCE_EXACT) || (D != 32 && D != 64)) return SPLIT_NONE;
  if (bias && bias->dtype != TENSION_F32) return SPLIT_NONE;
  if (aligned_f32_rows(q) && aligned_f32_rows(k)) {
    if (aligned_bf16_rows(v)) return SPLIT_F32;
    if (aligned_f32_rows(v)) return SPLIT_F32V;
    return SPLIT_NONE;
  }
  if (aligned_bf16_rows(q) && aligned_bf16_rows(k) && aligned_bf16_rows(v)) return SPLIT_BF16;
  if (aligned_f16_rows(q) && aligned_f16_rows(k) && aligned_f16_rows(v)) return SPLIT_F16;
  return SPLIT_NONE;
}

// Q's dtype in a split kernel
int32_t split_qk_dtype(int kind) {
  return kind == SPLIT_BF16 ? TENSION_BF16 : kind == SPLIT_F16 ? TENSION_F16 : TENSION_F32;
}

// A further operand of a split kernel: rows in Q's dtype (outputs and
// gradients of Q / K / out).
bool split_rows(int kind, const tension_buf* b) {
  const int32_t dt = split_qk_dtype(kind);
  return dt == TENSION_F32 ? aligned_f32_rows(b) : aligned_rows16(b, dt);
}

// dV of a split kernel: rows in V's dtype.
bool split_dv_rows(int kind, const tension_buf* b) {
  return kind == SPLIT_F32V ? aligned_f32_rows(b) : kind == SPLIT_F16 ? aligned_f16_rows(b) : aligned_bf16_rows(b);
}

// tau / dtau of a split kernel: absent, or in Q's dtype (the kernels index
// them as typed rows).
bool split_side(int kind, const tension_buf* b) { return !b || b->dtype == split_qk_dtype(kind); }

// Local windows wider than one 64-row tile run on the split kernels in bf16
// too: 14-20% faster per fwd+bwd step than the dedicated band kernels'
// W > 64 path (mfma_fwd / mfma_dq / mfma_dkv), measured at W = 100, 128,
// 256, tau-mass and valid-count.  TENSION_WIDE_ON_BAND_KERNELS keeps them
// on the band kernels (for A/B runs).
bool wide_on_split(bool global, int64_t W) {
#ifdef TENSION_WIDE_ON_BAND_KERNELS
  (void)global;
  (void)W;
  return false;
#else
  return !global && W > 64;
#endif
}

enum {
  KERNEL_EXACT = 0,
  KERNEL_MFMA = 1,
  KERNEL_SPLIT_BF16 = 2,
  KERNEL_SPLIT_F32 = 3,
  KERNEL_SPLIT_F32V = 4,
  KERNEL_SPLIT_F16 = 5
};

thread_local int g_last_kernel = -1;

int run_band(int phase, int kind, bool f64, const BandParams& p, tension_stream_t stream, const char* what) {
  hipError_t e = hipSuccess;
  // the MFMA and split kernels take 32-bit strides (BandArgs); a tensor with
  // a larger one runs on the exact kernels
  BandArgs probe;
  if (kind != KERNEL_EXACT && phase != 3 && !band_args(p, &probe)) kind = KERNEL_EXACT;
  int r = kind == KERNEL_SPLIT_F16    ? launch_split(phase, SPLIT_FLOW_F16, p, hs(stream), &e)
          : kind == KERNEL_SPLIT_F32V ? launch_split(phase, SPLIT_FLOW_F32V, p, hs(stream), &e)
          : kind == KERNEL_SPLIT_F32  ? launch_split(phase, SPLIT_FLOW_F32, p, hs(stream), &e)
          : kind == KERNEL_SPLIT_BF16 ? launch_split(phase, SPLIT_FLOW_BF16, p, hs(stream), &e)
          : kind == KERNEL_MFMA       ? launch_mfma(phase, p, hs(stream), &e)
                                      : launch_exact(phase, f64, p, hs(stream), &e);
  if (r == kGridTooLarge)
    return fail(TENSION_ERR_UNSUPPORTED, "%s: B*H*T = %lld rows need a grid beyond 2^31 - 1 workgroups", what,
                (long long)p.B * p.H * p.T);
  if (r != 0)
    return fail(TENSION_ERR_UNSUPPORTED, "%s: head dim %d not supported (exact path: 8,16,32,64,128)", what, p.D);
  g_last_kernel = kind;
  return launched(e, what);
}

int split_kernel(int kind) {
  return kind == SPLIT_F16    ? KERNEL_SPLIT_F16
         : kind == SPLIT_F32V ? KERNEL_SPLIT_F32V
         : kind == SPLIT_F32  ? KERNEL_SPLIT_F32
                              : KERNEL_SPLIT_BF16;
}

// ---------------------------------------------------------------- forward

int band_fwd(const tension_buf* q, const tension_buf* k, const tension_buf* v, const tension_buf* out,
             const tension_buf* tau, const tension_buf* bias, const tension_buf* mass, Shape sh, int64_t Wparam,
             double scale, int32_t flags, tension_stream_t stream, bool global) {
  const char* what = global ? "tension_global_fwd" : "tension_window_fwd";
  bool empty = false;
  TRY(check_shape(sh, scale, &empty));
  if (!global && (Wparam < 1 || Wparam > 0x3fffffff))
    return fail(TENSION_ERR_ARG, "window must be >= 1 (got %lld)", (long long)Wparam);
  if (global && tau && (Wparam < 1 || Wparam > sh.T))
    return fail(TENSION_ERR_ARG, "tau_local width must be in [1, T]");
  if ((flags & TENSION_NORM_MASS) && (flags & TENSION_NORM_COUNT))
    return fail(TENSION_ERR_ARG, "NORM_MASS and NORM_COUNT are exclusive");
  if ((flags & TENSION_GLOBAL) && !global)
    return fail(TENSION_ERR_ARG, "use tension_global_fwd for the global block");
  if (global && (flags & TENSION_NORM_COUNT))
    return fail(TENSION_ERR_ARG, "global block is tau-mass normalised only");
  if (empty) return ok();
  TRY(check_buf(q, "q", true, 3));
  TRY(check_buf(k, "k", true, 3));
  TRY(check_buf(v, "v", true, 3));
  TRY(check_buf(out, "out", true, 3));
  TRY(check_buf(tau, global ? "tau_local" : "tau", false, 3));
  TRY(check_buf(bias, "bias", false, 2));
  TRY(check_buf(mass, "mass", false, -1));
  if (mass && mass->dtype != TENSION_F32 && mass->dtype != TENSION_F64)
    return fail(TENSION_ERR_ARG, "mass must be f32 or f64");
  if (global) flags |= TENSION_NORM_MASS | TENSION_GLOBAL;
  BandParams p = band_common(sh, scale, flags);
  if (global) set_global(p, tau ? Wparam : 0); else set_local(p, Wparam);
  p.q = make_buf(q); p.k = make_buf(k); p.v = make_buf(v);
  p.out = make_buf(out); p.tau = make_buf(tau); p.bias = make_buf(bias); p.mass = make_buf(mass);
  bool mf = !(flags & TENSION_FORCE_EXACT) && sh.D == 64 && aligned_bf16_rows(q) && aligned_bf16_rows(k) &&
                  aligned_bf16_rows(v) && aligned_bf16_rows(out) && (!bias || bias->dtype == TENSION_F32);
  if (wide_on_split(global, Wparam)) mf = false;
  const int sk = mf ? SPLIT_NONE : split_kind(q, k, v, bias, sh.D, flags);
  const bool sp = sk != SPLIT_NONE && split_rows(sk, out) && split_side(sk, tau);
  return run_band(0, sp ? split_kernel(sk) : mf ? KERNEL_MFMA : KERNEL_EXACT, any_f64(q, k, v), p, stream, what);
}

// ---------------------------------------------------------------- backward

// The workspace holds the per-query coefficients a_t, c_t of the tau-mass
// backward (dtau = a_t * dP - c_t + dTau): fp32, or f64 when any activation
// is f64.
// -1 for sizes that check_shape rejects (negative, or B*T*H above 2^40).
int64_t ws_bytes(int64_t B, int64_t T, int64_t H, int32_t dtype_acc, int32_t flags) {
  if (!(flags & TENSION_NORM_MASS)) return 0;
  const int64_t el = dtype_acc == TENSION_F64 ? 8 : 4;
  constexpr int64_t kMaxRows = (int64_t)1 << 40;
  const int64_t rows = mul_cap(mul_cap(B, T, kMaxRows), H, kMaxRows);
  return rows < 0 ? -1 : 2 * rows * el;
}

int check_bwd(const tension_buf* q, const tension_buf* k, const tension_buf* v, const tension_buf* dout,
              const tension_buf* dtau, const tension_buf* bias, Shape sh, int64_t Wparam, double scale,
              int32_t flags, void* ws, bool global, bool* empty) {
  TRY(check_shape(sh, scale, empty));
  if (!global && (Wparam < 1 || Wparam > 0x3fffffff))
    return fail(TENSION_ERR_ARG, "window must be >= 1 (got %lld)", (long long)Wparam);
  if (global && dtau && (Wparam < 1 || Wparam > sh.T))
    return fail(TENSION_ERR_ARG, "tau_local width must be in [1, T]");
  if ((flags & TENSION_NORM_MASS) && (flags & TENSION_NORM_COUNT))
    return fail(TENSION_ERR_ARG, "NORM_MASS and NORM_COUNT are exclusive");
  if (global && (flags & TENSION_NORM_COUNT))
    return fail(TENSION_ERR_ARG, "global block is tau-mass normalised only");
  if (*empty) return 0;
  TRY(check_buf(q, "q", true, 3));
  TRY(check_buf(k, "k", true, 3));
  TRY(check_buf(v, "v", true, 3));
  TRY(check_buf(dout, "dout", true, 3));
  TRY(check_buf(dtau, global ? "dtau_local" : "dtau", false, 3));
  TRY(check_buf(bias, "bias", false, 2));
  if (((flags & TENSION_NORM_MASS) || global) && !ws)
    return fail(TENSION_ERR_ARG, "workspace is required with tau-mass normalisation");
  return 0;
}

bool mfma_ok_bwd(const tension_buf* q, const tension_buf* k, const tension_buf* v, const tension_buf* dout,
                 const tension_buf* bias, const tension_buf* o1, const tension_buf* o2, int64_t D, int flags) {
  if (flags & TENSION_FORCE_EXACT) return false;
  if (D != 64) return false;
  if (!aligned_bf16_rows(q) || !aligned_bf16_rows(k) || !aligned_bf16_rows(v) || !aligned_bf16_rows(dout))
    return false;
  if (o1 && !aligned_bf16_rows(o1)) return false;
  if (o2 && !aligned_bf16_rows(o2)) return false;
  if (bias && bias->dtype != TENSION_F32) return false;
  return true;
}

BandParams bwd_params(const tension_buf* q, const tension_buf* k, const tension_buf* v, const tension_buf* dout,
                      const tension_buf* dtau, const tension_buf* bias, void* ws, Shape sh, int64_t Wparam,
                      double scale, int32_t flags, bool global) {
  if (global) flags |= TENSION_NORM_MASS | TENSION_GLOBAL;
  BandParams p = band_common(sh, scale, flags);
  if (global) set_global(p, dtau ? Wparam : 0); else set_local(p, Wparam);
  p.q = make_buf(q); p.k = make_buf(k); p.v = make_buf(v);
  p.dout = make_buf(dout); p.dtau = make_buf(dtau); p.bias = make_buf(bias); p.ws = ws;
  return p;
}

int band_bwd_dq(const tension_buf* q, const tension_buf* k, const tension_buf* v, const tension_buf* dout,
                const tension_buf* dtau, const tension_buf* bias, const tension_buf* dq, void* ws, Shape sh,
                int64_t Wparam, double scale, int32_t flags, tension_stream_t stream, bool global,
                const tension_buf* out = nullptr, const tension_buf* mass = nullptr) {
  bool empty = false;
  TRY(check_bwd(q, k, v, dout, dtau, bias, sh, Wparam, scale, flags, ws, global, &empty));
  if (empty) return ok();
  TRY(check_buf(dq, "dq", true, 3));
  BandParams p = bwd_params(q, k, v, dout, dtau, bias, ws, sh, Wparam, scale, flags, global);
  p.dq = make_buf(dq);
  bool mf = mfma_ok_bwd(q, k, v, dout, bias, dq, nullptr, sh.D, flags);
  if (wide_on_split(global, Wparam)) mf = false;
  const int sk = mf ? SPLIT_NONE : split_kind(q, k, v, bias, sh.D, flags);
  const bool sp = sk != SPLIT_NONE && split_rows(sk, dout) && split_rows(sk, dq) && split_side(sk, dtau);
  // the forward's saved output rows and tau mass (the tau-mass coefficients
  // come from them instead of a pass over the band): the global bf16
  // kernels, and the split kernels with float32 rows (whose dO . out does
  // not cancel the way a bf16 out would); every other kernel ignores them
  if (out && mass) {
    TRY(check_buf(out, "out", true, 3));
    TRY(check_buf(mass, "mass", true, -1));
    const bool f32_mass = mass->dtype == TENSION_F32;
    const bool rows_mf = mf && global && aligned_bf16_rows(out) && f32_mass;
    const bool rows_sp = sp && (sk == SPLIT_F32 || sk == SPLIT_F32V) && ((flags & TENSION_NORM_MASS) || global) &&
                         aligned_f32_rows(out) && f32_mass;
    if (rows_mf || rows_sp) {
      p.out = make_buf(out);
      p.mass = make_buf(mass);
      p.coef_pre = 1;
    }
  }
  return run_band(1, sp ? split_kernel(sk) : mf ? KERNEL_MFMA : KERNEL_EXACT, any_f64(q, k, v), p, stream,
                  global ? "tension_global_bwd(dq)" : "tension_window_bwd_dq");
}

int band_bwd_dkv(const tension_buf* q, const tension_buf* k, const tension_buf* v, const tension_buf* dout,
                 const tension_buf* dtau, const tension_buf* bias, const tension_buf* dk, const tension_buf* dv,
                 void* ws, Shape sh, int64_t Wparam, double scale, int32_t flags, tension_stream_t stream,
                 bool global) {
  bool empty = false;
  TRY(check_bwd(q, k, v, dout, dtau, bias, sh, Wparam, scale, flags, ws, global, &empty));
  if (empty) return ok();
  TRY(check_buf(dk, "dk", true, 3));
  TRY(check_buf(dv, "dv", true, 3));
  BandParams p = bwd_params(q, k, v, dout, dtau, bias, ws, sh, Wparam, scale, flags, global);
  p.dk = make_buf(dk);
  p.dv = make_buf(dv);
  bool mf = mfma_ok_bwd(q, k, v, dout, bias, dk, dv, sh.D, flags);
  if (wide_on_split(global, Wparam)) mf = false;
  const int sk = mf ? SPLIT_NONE : split_kind(q, k, v, bias, sh.D, flags);
  const bool sp = sk != SPLIT_NONE && split_rows(sk, dout) && split_rows(sk, dk) && split_dv_rows(sk, dv) &&
                  split_side(sk, dtau);
  return run_band(2, sp ? split_kernel(sk) : mf ? KERNEL_MFMA : KERNEL_EXACT, any_f64(q, k, v), p, stream,
                  global ? "tension_global_bwd(dkv)" : "tension_window_bwd_dkv");
}

}  // namespace

// ---------------------------------------------------------------- fixed scratch
// Device workspace of tension_global_bwd_noalloc: one copy of this array per
// GPU the library runs on, held until the process ends.  Host code reaches it
// only through the address hipGetSymbolAddress returns for the current device
// (the array's name in host code is not a device address).
static __device__ __align__(256) unsigned char scratch[TENSION_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch`, per device

// Address of the current device's copy of `scratch`, looked up once per
// device (the first call with that device current).
int scratch_ptr(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(TENSION_ERR_LAUNCH, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(TENSION_ERR_UNSUPPORTED, "device %d: the fixed scratch supports devices 0..%d", dev, kMaxDevices - 1);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(TENSION_ERR_LAUNCH, "hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

}  // namespace

extern "C" {

const char* tension_last_error(void) { return g_err.c_str(); }

int tension_last_kernel(void) { return g_last_kernel; }

const char* tension_version(void) { return "tension_hip 0.1 (gfx950)"; }

int tension_window_fwd(const tension_buf* q, const tension_buf* k, const tension_buf* v, const tension_buf* out,
                       const tension_buf* tau, const tension_buf* bias, const tension_buf* mass, int64_t B,
                       int64_t T, int64_t H, int64_t D, int64_t W, double scale, int32_t flags,
                       tension_stream_t stream) {
  return band_fwd(q, k, v, out, tau, bias, mass, Shape{B, T, H, D}, W, scale, flags, stream, false);
}

int64_t tension_window_bwd_workspace(int64_t B, int64_t T, int64_t H, int32_t dtype_acc, int32_t flags) {
  return ws_bytes(B, T, H, dtype_acc, flags);
}

int tension_window_bwd_dq(const tension_buf* q, const tension_buf* k, const tension_buf* v,
                          const tension_buf* dout, const tension_buf* dtau, const tension_buf* bias,
                          const tension_buf* dq, void* ws, int64_t B, int64_t T, int64_t H, int64_t D, int64_t W,
                          double scale, int32_t flags, tension_stream_t stream) {
  return band_bwd_dq(q, k, v, dout, dtau, bias, dq, ws, Shape{B, T, H, D}, W, scale, flags, stream, false);
}

int tension_window_bwd_dkv(const tension_buf* q, const tension_buf* k, const tension_buf* v,
                           const tension_buf* dout, const tension_buf* dtau, const tension_buf* bias,
                           const tension_buf* dk, const tension_buf* dv, void* ws, int64_t B, int64_t T,
                           int64_t H, int64_t D, int64_t W, double scale, int32_t flags,
                           tension_stream_t stream) {
  return band_bwd_dkv(q, k, v, dout, dtau, bias, dk, dv, ws, Shape{B, T, H, D}, W, scale, flags, stream, false);
}

}  // extern "C"

namespace {

// tension_window_bwd with, optionally, the forward's output rows and tau
// mass (see band_bwd_dq).
int window_bwd(const tension_buf* q, const tension_buf* k, const tension_buf* v, const tension_buf* dout,
               const tension_buf* dtau, const tension_buf* bias, const tension_buf* out, const tension_buf* mass,
               const tension_buf* dq, const tension_buf* dk, const tension_buf* dv, void* ws, int64_t B,
               int64_t T, int64_t H, int64_t D, int64_t W, double scale, int32_t flags, tension_stream_t stream) {
  const Shape sh{B, T, H, D};
  if (W >= 1 && W <= 64) {
    // one fused kernel (no workspace traffic) when the MFMA path applies
    bool empty = false;
    TRY(check_bwd(q, k, v, dout, dtau, bias, sh, W, scale, flags, ws, false, &empty));
    if (empty) return ok();
    TRY(check_buf(dq, "dq", true, 3));
    TRY(check_buf(dk, "dk", true, 3));
    TRY(check_buf(dv, "dv", true, 3));
    bool fit = true;
    for (const tension_buf* t : {q, k, v, dout, dq, dk, dv}) fit = fit && rows_fit_u32(t, sh.T);
    if (fit && mfma_ok_bwd(q, k, v, dout, bias, dq, dk, sh.D, flags) && aligned_bf16_rows(dv)) {
      BandParams p = bwd_params(q, k, v, dout, dtau, bias, ws, sh, W, scale, flags, false);
      p.dq = make_buf(dq);
      p.dk = make_buf(dk);
      p.dv = make_buf(dv);
      BandArgs probe;  // 32-bit strides, else the split pair below
      if (band_args(p, &probe)) return run_band(3, KERNEL_MFMA, false, p, stream, "tension_window_bwd");
    }
  }
  TRY(band_bwd_dq(q, k, v, dout, dtau, bias, dq, ws, sh, W, scale, flags, stream, false, out, mass));
  return band_bwd_dkv(q, k, v, dout, dtau, bias, dk, dv, ws, sh, W, scale, flags, stream, false);
}

}  // namespace

extern "C" {

int tension_window_bwd(const tension_buf* q, const tension_buf* k, const tension_buf* v, const tension_buf* dout,
                       const tension_buf* dtau, const tension_buf* bias, const tension_buf* dq,
                       const tension_buf* dk, const tension_buf* dv, void* ws, int64_t B, int64_t T, int64_t H,
                       int64_t D, int64_t W, double scale, int32_t flags, tension_stream_t stream) {
  return window_bwd(q, k, v, dout, dtau, bias, nullptr, nullptr, dq, dk, dv, ws, B, T, H, D, W, scale, flags,
                    stream);
}

int tension_window_bwd_saved(const tension_buf* q, const tension_buf* k, const tension_buf* v,
                             const tension_buf* dout, const tension_buf* dtau, const tension_buf* bias,
                             const tension_buf* out, const tension_buf* mass, const tension_buf* dq,
                             const tension_buf* dk, const tension_buf* dv, void* ws, int64_t B, int64_t T,
                             int64_t H, int64_t D, int64_t W, double scale, int32_t flags,
                             tension_stream_t stream) {
  if (!out || !mass) return fail(TENSION_ERR_ARG, "tension_window_bwd_saved: out and mass are required");
  return window_bwd(q, k, v, dout, dtau, bias, out, mass, dq, dk, dv, ws, B, T, H, D, W, scale, flags, stream);
}

int tension_global_fwd(const tension_buf* q, const tension_buf* k, const tension_buf* v, const tension_buf* out,
                       const tension_buf* tau_local, const tension_buf* bias, const tension_buf* mass, int64_t B,
                       int64_t T, int64_t H, int64_t D, int64_t Wl, double scale, int32_t flags,
                       tension_stream_t stream) {
  return band_fwd(q, k, v, out, tau_local, bias, mass, Shape{B, T, H, D}, Wl, scale, flags, stream, true);
}

int64_t tension_global_bwd_workspace(int64_t B, int64_t T, int64_t H, int32_t dtype_acc, int32_t flags) {
  return ws_bytes(B, T, H, dtype_acc, flags | TENSION_NORM_MASS);
}

int tension_global_bwd(const tension_buf* q, const tension_buf* k, const tension_buf* v, const tension_buf* dout,
                       const tension_buf* dtau_local, const tension_buf* bias, const tension_buf* out,
                       const tension_buf* mass, const tension_buf* dq, const tension_buf* dk,
                       const tension_buf* dv, void* ws, int64_t B, int64_t T, int64_t H, int64_t D, int64_t Wl,
                       double scale, int32_t flags, tension_stream_t stream) {
  const Shape sh{B, T, H, D};
  TRY(band_bwd_dq(q, k, v, dout, dtau_local, bias, dq, ws, sh, Wl, scale, flags, stream, true, out, mass));
  return band_bwd_dkv(q, k, v, dout, dtau_local, bias, dk, dv, ws, sh, Wl, scale, flags, stream, true);
}

int tension_global_bwd_noalloc(const tension_buf* q, const tension_buf* k, const tension_buf* v,
                               const tension_buf* dout, const tension_buf* dtau_local, const tension_buf* bias,
                               const tension_buf* out, const tension_buf* mass, const tension_buf* dq,
                               const tension_buf* dk, const tension_buf* dv, int64_t B, int64_t T, int64_t H,
                               int64_t D, int64_t Wl, double scale, int32_t flags, tension_stream_t stream) {
  const Shape sh{B, T, H, D};
  bool empty = false;
  TRY(check_shape(sh, scale, &empty));
  if (empty) return ok();
  const int32_t acc = any_f64(q, k, v) ? TENSION_F64 : TENSION_F32;
  const int64_t need = ws_bytes(B, T, H, acc, flags | TENSION_NORM_MASS);
  if (need > (int64_t)TENSION_NOALLOC_SCRATCH_BYTES)
    return fail(TENSION_ERR_ARG,
                "tension_global_bwd_noalloc: B*T*H = %lld queries need %lld bytes of workspace, more than the "
                "fixed scratch of %lld bytes (use tension_global_bwd with a caller workspace)",
                (long long)(B * T * H), (long long)need, (long long)TENSION_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  TRY(scratch_ptr(&ws));
  TRY(band_bwd_dq(q, k, v, dout, dtau_local, bias, dq, ws, sh, Wl, scale, flags, stream, true, out, mass));
  return band_bwd_dkv(q, k, v, dout, dtau_local, bias, dk, dv, ws, sh, Wl, scale, flags, stream, true);
}

int tension_decode_step(const tension_buf* q, const tension_buf* k_new, const tension_buf* v_new,
                        const tension_buf* k_cache, const tension_buf* v_cache, const tension_buf* out,
                        const tension_buf* tau, const int32_t* pos_in, int32_t* pos_out, int64_t N, int64_t H,
                        int64_t D, int64_t W, double scale, int32_t flags, tension_stream_t stream) {
  if (N < 0 || H < 0 || D <= 0 || D > 256 || W < 1 || W > 0x3fffffff || mul_cap(N, H, 0x3fffffff) < 0)
    return fail(TENSION_ERR_ARG, "decode: bad sizes N=%lld H=%lld D=%lld W=%lld", (long long)N, (long long)H,
                (long long)D, (long long)W);
  if (!(std::isfinite(scale) && scale != 0.0)) return fail(TENSION_ERR_ARG, "scale must be finite and non-zero");
  if (N * H == 0) return ok();
  TRY(check_buf(q, "q", true, 2));
  TRY(check_buf(k_new, "k_new", true, 2));
  TRY(check_buf(v_new, "v_new", true, 2));
  TRY(check_buf(out, "out", true, 2));
  TRY(check_buf(k_cache, "k_cache", true, 3));
  TRY(check_buf(v_cache, "v_cache", true, 3));
  TRY(check_buf(tau, "tau", false, 2));
  if (!pos_in) return fail(TENSION_ERR_ARG, "pos_in is required");
  if (pos_out && pos_out == pos_in) return fail(TENSION_ERR_ARG, "pos_out must not alias pos_in");
  if (k_cache->dtype != k_new->dtype || v_cache->dtype != v_new->dtype)
    return fail(TENSION_ERR_ARG, "cache and new-token dtypes must match");
  if ((flags & TENSION_NORM_MASS) && (flags & TENSION_NORM_COUNT))
    return fail(TENSION_ERR_ARG, "decode: TENSION_NORM_MASS and TENSION_NORM_COUNT are exclusive");
  if ((flags & TENSION_DECODE_SELF) && tau && tau->ptr)
    return fail(TENSION_ERR_ARG, "decode: tau output is not supported with TENSION_DECODE_SELF");
  DecodeParams p;
  memset(&p, 0, sizeof p);
  p.q = make_buf(q); p.kn = make_buf(k_new); p.vn = make_buf(v_new);
  p.kc = make_buf(k_cache); p.vc = make_buf(v_cache); p.out = make_buf(out); p.tau = make_buf(tau);
  p.pos_in = pos_in; p.pos_out = pos_out;
  p.N = (int)N; p.H = (int)H; p.D = (int)D; p.W = (int)W;
  p.scale = scale; p.inv_scale = (float)(1.0 / scale); p.flags = flags;
  // 16-byte aligned rows of a 16-bit dtype (bf16 or float16)
  auto a16 = [](const tension_buf* b, bool four, int32_t dt) {
    if (b->dtype != dt || ((uintptr_t)b->ptr & 15)) return false;
    return b->s[0] % 8 == 0 && b->s[1] % 8 == 0 && (!four || b->s[2] % 8 == 0);
  };
  // 16-byte aligned float32 rows
  auto a32 = [](const tension_buf* b, bool four) {
    if (b->dtype != TENSION_F32 || ((uintptr_t)b->ptr & 15)) return false;
    return b->s[0] % 4 == 0 && b->s[1] % 4 == 0 && (!four || b->s[2] % 4 == 0);
  };
  // the fast kernel reads each (n, h) cache slab through a buffer descriptor
  // of W * row_stride * element bytes (31-bit range, rows of at least 64
  // elements)
  auto slab_fits = [&](const tension_buf* b, int el) {
    return b->s[2] >= 64 && mul_cap(W, b->s[2], ((int64_t)1 << 31) / el - 1) >= 0;
  };
  auto all16 = [&](int32_t dt) {
    return a16(q, false, dt) && a16(k_new, false, dt) && a16(v_new, false, dt) && a16(out, false, dt) &&
           a16(k_cache, true, dt) && a16(v_cache, true, dt) && slab_fits(k_cache, 2) && slab_fits(v_cache, 2);
  };
  const bool f32qk = a32(q, false) && a32(k_new, false) && a32(out, false) && a32(k_cache, true) &&
                     slab_fits(k_cache, 4);
  int flow = DECODE_EXACT;
  if (!(flags & TENSION_FORCE_EXACT) && D == 64 && W <= 1024) {
    if (all16(TENSION_BF16)) {
      flow = DECODE_BF16;
    } else if (all16(TENSION_F16)) {
      flow = DECODE_F16;
    } else if (f32qk && !(flags & TENSION_DECODE_SELF)) {
      // the reference's autocast flow: float32 q / K (promoted by RoPE), bf16
      // V; or float32 throughout (no autocast)
      if (a16(v_new, false, TENSION_BF16) && a16(v_cache, true, TENSION_BF16) && slab_fits(v_cache, 2))
        flow = DECODE_KF32;
      else if (W <= 512 && a32(v_new, false) && a32(v_cache, true) && slab_fits(v_cache, 4))
        flow = DECODE_F32;
    }
  }
  hipError_t e = hipSuccess;
  launch_decode(flow, is_f64(q) || is_f64(k_cache) || is_f64(v_cache), p, hs(stream), &e);
  return launched(e, "tension_decode_step");
}

int tension_rope(const tension_buf* x, const tension_buf* y, const float* cos, const float* sin,
                 int64_t table_rows, int64_t B, int64_t T, int64_t H, int64_t D, int64_t pos_offset,
                 int32_t inverse, tension_stream_t stream) {
  bool empty = false;
  TRY(check_shape(Shape{B, T, H, D}, 1.0, &empty));
  if (D % 2) return fail(TENSION_ERR_ARG, "rope: head dim must be even");
  if (pos_offset < 0) return fail(TENSION_ERR_ARG, "rope: negative position offset");
  if (T > table_rows || pos_offset > table_rows - T)
    return fail(TENSION_ERR_ARG, "rope: table has %lld rows, positions %lld + [0, %lld) requested",
                (long long)table_rows, (long long)pos_offset, (long long)T);
  if (empty) return ok();
  TRY(check_buf(x, "x", true, 3));
  TRY(check_buf(y, "y", true, 3));
  if (!cos || !sin) return fail(TENSION_ERR_ARG, "rope: cos/sin tables are required");
  RopeParams p;
  memset(&p, 0, sizeof p);
  p.x = make_buf(x); p.y = make_buf(y); p.cos = cos; p.sin = sin;
  p.B = (int)B; p.T = (int)T; p.H = (int)H; p.D = (int)D;
  p.pos_offset = pos_offset; p.inverse = inverse;
  hipError_t e = hipSuccess;
  // 16-byte pieces of bf16 / float32 rows and of the float tables
  auto v16 = [](const tension_buf* b) {
    const int64_t per = b->dtype == TENSION_BF16 ? 8 : b->dtype == TENSION_F32 ? 4 : 0;
    return per && ((uintptr_t)b->ptr & 15) == 0 && b->s[0] % per == 0 && b->s[1] % per == 0 &&
           b->s[2] % per == 0;
  };
  if (D % 16 == 0 && v16(x) && v16(y) && ((uintptr_t)cos & 15) == 0 && ((uintptr_t)sin & 15) == 0)
    launch_rope_vec(x->dtype == TENSION_F32, y->dtype == TENSION_F32, p, hs(stream), &e);
  else
    launch_rope(is_f64(x) || is_f64(y), p, hs(stream), &e);
  return launched(e, "tension_rope");
}

namespace {

int check_taus(const tension_buf* taus, int32_t L, int64_t B, int64_t T, int64_t H, int64_t W, Buf* out) {
  if (!taus) return fail(TENSION_ERR_ARG, "taus is required");
  if (L < 1 || L > kMaxLayers) return fail(TENSION_ERR_ARG, "tau export: L=%d outside [1, %d]", L, kMaxLayers);
  if (B < 1 || T < 1 || H < 1 || W < 1 || mul_cap(T, W, 0x3fffffff) < 0 ||
      mul_cap(mul_cap(mul_cap(B, T, (int64_t)1 << 40), H, (int64_t)1 << 40), W, (int64_t)1 << 40) < 0)
    return fail(TENSION_ERR_ARG, "tau export: bad sizes B=%lld T=%lld H=%lld W=%lld", (long long)B,
                (long long)T, (long long)H, (long long)W);
  for (int l = 0; l < L; ++l) {
    TRY(check_buf(&taus[l], "tau", true, 3));
    out[l] = make_buf(&taus[l]);
  }
  return 0;
}

}  // namespace

int tension_tau_head_stats(const tension_buf* taus, int32_t L, int64_t B, int64_t T, int64_t H, int64_t W,
                           float* stats, int32_t flags, tension_stream_t stream) {
  TauStatParams p;
  memset(&p, 0, sizeof p);
  TRY(check_taus(taus, L, B, T, H, W, p.tau));
  if (!stats) return fail(TENSION_ERR_ARG, "stats is required");
  p.stats = stats;
  p.L = L; p.B = (int)B; p.T = (int)T; p.H = (int)H; p.W = (int)W;
  p.valid_only = (flags & TENSION_TAU_VALID_ONLY) ? 1 : 0;
  hipError_t e = hipSuccess;
  launch_tau_stats(p, hs(stream), &e);
  return launched(e, "tension_tau_head_stats");
}

int tension_tau_aggregate(const tension_buf* taus, int32_t L, int64_t B, int64_t T, int64_t H, int64_t W,
                          const int32_t* head_mask, float* agg, tension_stream_t stream) {
  TauAggParams p;
  memset(&p, 0, sizeof p);
  TRY(check_taus(taus, L, B, T, H, W, p.tau));
  if (H > 64) return fail(TENSION_ERR_UNSUPPORTED, "tau aggregate: H=%lld > 64", (long long)H);
  if (!head_mask || !agg) return fail(TENSION_ERR_ARG, "head_mask and agg are required");
  p.mask = head_mask; p.agg = agg;
  p.L = L; p.B = (int)B; p.T = (int)T; p.H = (int)H; p.W = (int)W;
  hipError_t e = hipSuccess;
  launch_tau_aggregate(p, hs(stream), &e);
  return launched(e, "tension_tau_aggregate");
}

int64_t tension_aux_loss_partials(int64_t B, int64_t T, int64_t H) {
  const int64_t nrow = mul_cap(mul_cap(B, T, (int64_t)1 << 40), H, (int64_t)1 << 40);
  return nrow > 0 ? aux_loss_blocks(nrow) : 0;
}

int tension_aux_loss_fwd(const tension_buf* taus, int32_t L, int64_t B, int64_t T, int64_t H, int64_t W,
                         double* partials, tension_stream_t stream) {
  AuxLossParams p;
  memset(&p, 0, sizeof p);
  TRY(check_taus(taus, L, B, T, H, W, p.tau));
  if (W > 256) return fail(TENSION_ERR_UNSUPPORTED, "aux loss: W=%lld > 256", (long long)W);
  if (!partials) return fail(TENSION_ERR_ARG, "partials is required");
  if (B * T * H * 8 > 0x7fffffffll * 256) return fail(TENSION_ERR_ARG, "aux loss: too many rows");
  p.acc = partials;
  p.L = L; p.B = (int)B; p.T = (int)T; p.H = (int)H; p.W = (int)W;
  hipError_t e = hipSuccess;
  launch_aux_loss(false, p, hs(stream), &e);
  return launched(e, "tension_aux_loss_fwd");
}

int tension_aux_loss_bwd(const tension_buf* taus, const tension_buf* dtaus, int32_t L, int64_t B, int64_t T,
                         int64_t H, int64_t W, const float* coef, tension_stream_t stream) {
  AuxLossParams p;
  memset(&p, 0, sizeof p);
  TRY(check_taus(taus, L, B, T, H, W, p.tau));
  TRY(check_taus(dtaus, L, B, T, H, W, p.dtau));
  if (W > 256) return fail(TENSION_ERR_UNSUPPORTED, "aux loss: W=%lld > 256", (long long)W);
  if (!coef) return fail(TENSION_ERR_ARG, "coef is required");
  if (B * T * H * 8 > 0x7fffffffll * 256) return fail(TENSION_ERR_ARG, "aux loss: too many rows");
  p.coef = coef;
  p.L = L; p.B = (int)B; p.T = (int)T; p.H = (int)H; p.W = (int)W;
  hipError_t e = hipSuccess;
  launch_aux_loss(true, p, hs(stream), &e);
  return launched(e, "tension_aux_loss_bwd");
}

int tension_bias_table_insert(const uint64_t* keys_in, const double* vals_in, int64_t n, uint64_t* table_keys,
                              double* table_vals, int32_t log2cap, tension_stream_t stream) {
  if (log2cap < 1 || log2cap > 40) return fail(TENSION_ERR_ARG, "bias table: log2cap=%d outside [1, 40]", log2cap);
  if (n < 0 || n > ((int64_t)1 << log2cap) / 2)
    return fail(TENSION_ERR_ARG, "bias table: %lld keys need a capacity of at least twice that (have 2^%d)",
                (long long)n, log2cap);
  if (n == 0) return ok();
  if (!keys_in || !vals_in || !table_keys || !table_vals) return fail(TENSION_ERR_ARG, "bias table: null pointer");
  BiasTableParams p;
  p.in_keys = (const unsigned long long*)keys_in; p.in_vals = vals_in; p.n = n;
  p.keys = (unsigned long long*)table_keys; p.vals = table_vals; p.log2cap = log2cap;
  hipError_t e = hipSuccess;
  launch_bias_insert(p, hs(stream), &e);
  return launched(e, "tension_bias_table_insert");
}

int tension_bias_build(const int32_t* content_ids, int64_t B, int64_t T, int64_t W, const uint64_t* table_keys,
                       const double* table_vals, int32_t log2cap, double alpha, const tension_buf* bias,
                       double* stats, tension_stream_t stream) {
  // the launch covers T * K (K = W, or T for the global [B, T, T] bias)
  // elements in 256-thread blocks: at most 2^38 of them
  if (B < 1 || T < 0 || W < 0 || B > 0x3fffffff || T > 0x7fffffff / 2 || W > 0x3fffffff ||
      mul_cap(T, W > 0 ? W : T, 0x3fffffffffll) < 0)
    return fail(TENSION_ERR_ARG, "bias build: bad sizes B=%lld T=%lld W=%lld", (long long)B, (long long)T,
                (long long)W);
  if (log2cap < 1 || log2cap > 40) return fail(TENSION_ERR_ARG, "bias build: log2cap=%d outside [1, 40]", log2cap);
  if (!std::isfinite(alpha)) return fail(TENSION_ERR_ARG, "bias build: alpha must be finite");
  if (T == 0) return ok();
  TRY(check_buf(bias, "bias", true, 2));
  if (!content_ids || !table_keys || !table_vals) return fail(TENSION_ERR_ARG, "bias build: null pointer");
  BiasBuildParams p;
  memset(&p, 0, sizeof p);
  p.ids = content_ids; p.keys = (const unsigned long long*)table_keys; p.vals = table_vals;
  p.log2cap = log2cap; p.alpha = alpha; p.out = bias->ptr; p.os0 = bias->s[0]; p.os1 = bias->s[1];
  p.B = (int)B; p.T = (int)T; p.K = (int)(W > 0 ? W : T); p.global = W == 0; p.stats = stats;
  hipError_t e = hipSuccess;
  launch_bias_build(bias->dtype, p, hs(stream), &e);
  return launched(e, "tension_bias_build");
}

}  // extern "C"
