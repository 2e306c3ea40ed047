// extern "C" entry points of libtension_hip.so: argument validation,
// kernel selection (MFMA bf16 path or exact path) and error reporting.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
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

bool dtype_ok(int dt) { return dt >= TENSION_F32 && dt <= TENSION_F64; }

// A required or optional [.., .., .., D] tensor with unit innermost stride.
int check4(const tension_buf* b, const char* what, bool required) {
  if (!b) return required ? fail(TENSION_ERR_ARG, "%s is required", what) : 0;
  if (!b->ptr) return fail(TENSION_ERR_ARG, "%s: null data pointer", what);
  if (!dtype_ok(b->dtype)) return fail(TENSION_ERR_ARG, "%s: bad dtype code %d", what, b->dtype);
  if (b->s[3] != 1) return fail(TENSION_ERR_ARG, "%s: innermost stride must be 1 (got %lld)", what, (long long)b->s[3]);
  return 0;
}

int check3(const tension_buf* b, const char* what, bool required, bool unit_last) {
  if (!b) return required ? fail(TENSION_ERR_ARG, "%s is required", what) : 0;
  if (!b->ptr) return fail(TENSION_ERR_ARG, "%s: null data pointer", what);
  if (!dtype_ok(b->dtype)) return fail(TENSION_ERR_ARG, "%s: bad dtype code %d", what, b->dtype);
  if (unit_last && b->s[2] != 1) return fail(TENSION_ERR_ARG, "%s: innermost stride must be 1", what);
  return 0;
}

bool is_f64(const tension_buf* b) { return b && b->dtype == TENSION_F64; }

bool aligned_bf16_rows(const tension_buf* b) {
  if (!b || b->dtype != TENSION_BF16) return false;
  if (((uintptr_t)b->ptr & 15) != 0) return false;
  return (b->s[0] % 8 == 0) && (b->s[1] % 8 == 0) && (b->s[2] % 8 == 0);
}

hipStream_t hs(tension_stream_t s) { return (hipStream_t)s; }

struct Shape {
  int64_t B, T, H, D;
};

int check_shape(Shape sh, double scale) {
  if (sh.B < 0 || sh.T < 0 || sh.H < 0 || sh.D <= 0)
    return fail(TENSION_ERR_ARG, "bad shape B=%lld T=%lld H=%lld D=%lld", (long long)sh.B,
                (long long)sh.T, (long long)sh.H, (long long)sh.D);
  if (sh.T > 0x3fffffff || sh.H > 0x3fffffff || sh.B > 0x3fffffff || sh.B * sh.H * sh.T > (int64_t)1 << 40)
    return fail(TENSION_ERR_ARG, "shape too large");
  if (!(std::isfinite(scale) && scale != 0.0)) return fail(TENSION_ERR_ARG, "scale must be finite and non-zero");
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

// MFMA path: bf16 activations, D = 64, 16-byte aligned rows, fp32 side tensors.
bool mfma_ok_fwd(const tension_buf* q, const tension_buf* k, const tension_buf* v,
                 const tension_buf* out, const tension_buf* bias, const tension_buf* mass, int64_t D,
                 int flags) {
  if (flags & TENSION_FORCE_EXACT) return false;
  if (D != 64) return false;
  if (!aligned_bf16_rows(q) || !aligned_bf16_rows(k) || !aligned_bf16_rows(v) || !aligned_bf16_rows(out))
    return false;
  if (bias && bias->dtype != TENSION_F32) return false;
  if (mass && mass->dtype != TENSION_F32) return false;
  return true;
}

int run_band(int phase, bool mfma, bool f64, const BandParams& p, tension_stream_t stream, const char* what) {
  if ((int64_t)p.B * p.H * p.T == 0) return ok();
  hipError_t e = hipSuccess;
  int r = mfma ? launch_mfma(phase, p, hs(stream), &e) : launch_exact(phase, f64, p, hs(stream), &e);
  if (r != 0) return fail(TENSION_ERR_UNSUPPORTED, "%s: head dim %d not supported (exact path: 8,16,32,64,128)", what, p.D);
  return launched(e, what);
}

#define TRY(x)            \
  do {                    \
    int _r = (x);         \
    if (_r) return _r;    \
  } while (0)

int validate_fwd(const tension_buf* q, const tension_buf* k, const tension_buf* v, const tension_buf* out,
                 const tension_buf* tau, const tension_buf* bias, const tension_buf* mass, Shape sh,
                 double scale, int32_t flags, bool global) {
  TRY(check_shape(sh, scale));
  TRY(check4(q, "q", true));
  TRY(check4(k, "k", true));
  TRY(check4(v, "v", true));
  TRY(check4(out, "out", true));
  TRY(check4(tau, global ? "tau_local" : "tau", false));
  TRY(check3(bias, "bias", false, true));
  TRY(check3(mass, "mass", false, false));
  if ((flags & TENSION_NORM_MASS) && (flags & TENSION_NORM_COUNT))
    return fail(TENSION_ERR_ARG, "NORM_MASS and NORM_COUNT are exclusive");
  if (mass && mass->dtype != TENSION_F32 && mass->dtype != TENSION_F64)
    return fail(TENSION_ERR_ARG, "mass must be f32 or f64");
  return 0;
}

int validate_bwd_common(const tension_buf* q, const tension_buf* k, const tension_buf* v,
                        const tension_buf* dout, const tension_buf* dtau, const tension_buf* bias,
                        const tension_buf* out, const tension_buf* mass, Shape sh, double scale,
                        int32_t flags, void* ws, bool need_out) {
  TRY(check_shape(sh, scale));
  TRY(check4(q, "q", true));
  TRY(check4(k, "k", true));
  TRY(check4(v, "v", true));
  TRY(check4(dout, "dout", true));
  TRY(check4(dtau, "dtau", false));
  TRY(check3(bias, "bias", false, true));
  if ((flags & TENSION_NORM_MASS) && (flags & TENSION_NORM_COUNT))
    return fail(TENSION_ERR_ARG, "NORM_MASS and NORM_COUNT are exclusive");
  if (flags & TENSION_NORM_MASS) {
    if (need_out) {
      TRY(check4(out, "out (saved forward output)", true));
      TRY(check3(mass, "mass (saved forward mass)", true, false));
    }
    if (!ws) return fail(TENSION_ERR_ARG, "workspace is required with TENSION_NORM_MASS");
  }
  return 0;
}

bool any_f64(const tension_buf* a, const tension_buf* b, const tension_buf* c) {
  return is_f64(a) || is_f64(b) || is_f64(c);
}

bool mfma_ok_bwd(const tension_buf* q, const tension_buf* k, const tension_buf* v, const tension_buf* dout,
                 const tension_buf* bias, const tension_buf* out, const tension_buf* mass,
                 const tension_buf* o1, const tension_buf* o2, int64_t D, int flags) {
  if (flags & TENSION_FORCE_EXACT) return false;
  if (D != 64) return false;
  if (!aligned_bf16_rows(q) || !aligned_bf16_rows(k) || !aligned_bf16_rows(v) || !aligned_bf16_rows(dout))
    return false;
  if (o1 && !aligned_bf16_rows(o1)) return false;
  if (o2 && !aligned_bf16_rows(o2)) return false;
  if (bias && bias->dtype != TENSION_F32) return false;
  if (flags & TENSION_NORM_MASS) {
    if (!aligned_bf16_rows(out)) return false;
    if (!mass || mass->dtype != TENSION_F32) return false;
  }
  return true;
}

// The workspace element type follows the path: fp32 for the MFMA path and
// for non-f64 exact calls, f64 when any activation is f64.
int64_t ws_bytes(int64_t B, int64_t T, int64_t H, int32_t dtype_acc, int32_t flags) {
  if (!(flags & TENSION_NORM_MASS)) return 0;
  const int64_t el = dtype_acc == TENSION_F64 ? 8 : 4;
  return 2 * B * T * H * el;
}

int band_bwd_dq(const tension_buf* q, const tension_buf* k, const tension_buf* v, const tension_buf* dout,
                const tension_buf* dtau, const tension_buf* bias, const tension_buf* out,
                const tension_buf* mass, const tension_buf* dq, void* ws, Shape sh, int64_t Wparam,
                double scale, int32_t flags, tension_stream_t stream, bool global) {
  TRY(validate_bwd_common(q, k, v, dout, dtau, bias, out, mass, sh, scale, flags, ws, true));
  TRY(check4(dq, "dq", true));
  if (global) flags |= TENSION_NORM_MASS;
  BandParams p = band_common(sh, scale, flags);
  if (global) set_global(p, Wparam); else set_local(p, Wparam);
  p.q = make_buf(q); p.k = make_buf(k); p.v = make_buf(v);
  p.dout = make_buf(dout); p.dtau = make_buf(dtau); p.bias = make_buf(bias);
  p.out = make_buf(out); p.mass = make_buf(mass); p.dq = make_buf(dq); p.ws = ws;
  const bool mf = mfma_ok_bwd(q, k, v, dout, bias, out, mass, dq, nullptr, sh.D, flags);
  return run_band(1, mf, any_f64(q, k, v), p, stream, global ? "tension_global_bwd(dq)" : "tension_window_bwd_dq");
}

int band_bwd_dkv(const tension_buf* q, const tension_buf* k, const tension_buf* v, const tension_buf* dout,
                 const tension_buf* dtau, const tension_buf* bias, const tension_buf* out,
                 const tension_buf* mass, const tension_buf* dk, const tension_buf* dv, void* ws, Shape sh,
                 int64_t Wparam, double scale, int32_t flags, tension_stream_t stream, bool global) {
  TRY(validate_bwd_common(q, k, v, dout, dtau, bias, out, mass, sh, scale, flags, ws, false));
  TRY(check4(dk, "dk", true));
  TRY(check4(dv, "dv", true));
  if (global) flags |= TENSION_NORM_MASS;
  BandParams p = band_common(sh, scale, flags);
  if (global) set_global(p, Wparam); else set_local(p, Wparam);
  p.q = make_buf(q); p.k = make_buf(k); p.v = make_buf(v);
  p.dout = make_buf(dout); p.dtau = make_buf(dtau); p.bias = make_buf(bias);
  p.dk = make_buf(dk); p.dv = make_buf(dv); p.ws = ws;
  // The dkv kernel reads the saved out/mass only through the workspace
  // (fp32 unless an activation is f64, on either path).
  const bool mf = mfma_ok_bwd(q, k, v, dout, bias, nullptr, nullptr, dk, dv, sh.D, flags & ~TENSION_NORM_MASS);
  return run_band(2, mf, any_f64(q, k, v), p, stream, global ? "tension_global_bwd(dkv)" : "tension_window_bwd_dkv");
}

}  // namespace

extern "C" {

const char* tension_last_error(void) { return g_err.c_str(); }

const char* tension_version(void) { return "tension_hip 0.1 (gfx950)"; }

int tension_window_fwd(const tension_buf* q, const tension_buf* k, const tension_buf* v, const tension_buf* out,
                       const tension_buf* tau, const tension_buf* bias, const tension_buf* mass, int64_t B,
                       int64_t T, int64_t H, int64_t D, int64_t W, double scale, int32_t flags,
                       tension_stream_t stream) {
  const Shape sh{B, T, H, D};
  TRY(validate_fwd(q, k, v, out, tau, bias, mass, sh, scale, flags, false));
  if (W < 1 || W > 0x3fffffff) return fail(TENSION_ERR_ARG, "window must be >= 1 (got %lld)", (long long)W);
  if ((flags & TENSION_NORM_MASS) && !mass) return fail(TENSION_ERR_ARG, "NORM_MASS needs a mass output");
  if (flags & TENSION_GLOBAL) return fail(TENSION_ERR_ARG, "use tension_global_fwd for the global block");
  BandParams p = band_common(sh, scale, flags);
  set_local(p, W);
  p.q = make_buf(q); p.k = make_buf(k); p.v = make_buf(v);
  p.out = make_buf(out); p.tau = make_buf(tau); p.bias = make_buf(bias); p.mass = make_buf(mass);
  const bool mf = mfma_ok_fwd(q, k, v, out, bias, mass, D, flags);
  return run_band(0, mf, any_f64(q, k, v), p, stream, "tension_window_fwd");
}

int64_t tension_window_bwd_workspace(int64_t B, int64_t T, int64_t H, int32_t dtype_acc, int32_t flags) {
  return ws_bytes(B, T, H, dtype_acc, flags);
}

int tension_window_bwd_dq(const tension_buf* q, const tension_buf* k, const tension_buf* v,
                          const tension_buf* dout, const tension_buf* dtau, const tension_buf* bias,
                          const tension_buf* out, const tension_buf* mass, const tension_buf* dq, void* ws,
                          int64_t B, int64_t T, int64_t H, int64_t D, int64_t W, double scale, int32_t flags,
                          tension_stream_t stream) {
  if (W < 1 || W > 0x3fffffff) return fail(TENSION_ERR_ARG, "window must be >= 1 (got %lld)", (long long)W);
  return band_bwd_dq(q, k, v, dout, dtau, bias, out, mass, dq, ws, Shape{B, T, H, D}, W, scale, flags, stream,
                     false);
}

int tension_window_bwd_dkv(const tension_buf* q, const tension_buf* k, const tension_buf* v,
                           const tension_buf* dout, const tension_buf* dtau, const tension_buf* bias,
                           const tension_buf* dk, const tension_buf* dv, void* ws, int64_t B, int64_t T,
                           int64_t H, int64_t D, int64_t W, double scale, int32_t flags,
                           tension_stream_t stream) {
  if (W < 1 || W > 0x3fffffff) return fail(TENSION_ERR_ARG, "window must be >= 1 (got %lld)", (long long)W);
  return band_bwd_dkv(q, k, v, dout, dtau, bias, nullptr, nullptr, dk, dv, ws, Shape{B, T, H, D}, W, scale,
                      flags, stream, false);
}

int tension_window_bwd(const tension_buf* q, const tension_buf* k, const tension_buf* v, const tension_buf* dout,
                       const tension_buf* dtau, const tension_buf* bias, const tension_buf* out,
                       const tension_buf* mass, const tension_buf* dq, const tension_buf* dk,
                       const tension_buf* dv, void* ws, int64_t B, int64_t T, int64_t H, int64_t D, int64_t W,
                       double scale, int32_t flags, tension_stream_t stream) {
  if (W < 1 || W > 0x3fffffff) return fail(TENSION_ERR_ARG, "window must be >= 1 (got %lld)", (long long)W);
  const Shape sh{B, T, H, D};
  TRY(check4(dk, "dk", true));
  TRY(check4(dv, "dv", true));
  TRY(band_bwd_dq(q, k, v, dout, dtau, bias, out, mass, dq, ws, sh, W, scale, flags, stream, false));
  return band_bwd_dkv(q, k, v, dout, dtau, bias, out, mass, dk, dv, ws, sh, W, scale, flags, stream, false);
}

int tension_global_fwd(const tension_buf* q, const tension_buf* k, const tension_buf* v, const tension_buf* out,
                       const tension_buf* tau_local, const tension_buf* bias, const tension_buf* mass, int64_t B,
                       int64_t T, int64_t H, int64_t D, int64_t Wl, double scale, int32_t flags,
                       tension_stream_t stream) {
  const Shape sh{B, T, H, D};
  TRY(validate_fwd(q, k, v, out, tau_local, bias, mass, sh, scale, flags, true));
  if (!mass) return fail(TENSION_ERR_ARG, "tension_global_fwd: mass output is required");
  if (flags & TENSION_NORM_COUNT) return fail(TENSION_ERR_ARG, "global block is tau-mass normalised only");
  if (tau_local && (Wl < 1 || Wl > T)) return fail(TENSION_ERR_ARG, "tau_local width must be in [1, T]");
  BandParams p = band_common(sh, scale, flags | TENSION_NORM_MASS | TENSION_GLOBAL);
  set_global(p, tau_local ? Wl : 0);
  p.q = make_buf(q); p.k = make_buf(k); p.v = make_buf(v);
  p.out = make_buf(out); p.tau = make_buf(tau_local); p.bias = make_buf(bias); p.mass = make_buf(mass);
  const bool mf = mfma_ok_fwd(q, k, v, out, bias, mass, D, flags);
  return run_band(0, mf, any_f64(q, k, v), p, stream, "tension_global_fwd");
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
  if (flags & TENSION_NORM_COUNT) return fail(TENSION_ERR_ARG, "global block is tau-mass normalised only");
  if (dtau_local && (Wl < 1 || Wl > T)) return fail(TENSION_ERR_ARG, "tau_local width must be in [1, T]");
  const int64_t wl = dtau_local ? Wl : 0;
  TRY(check4(dk, "dk", true));
  TRY(check4(dv, "dv", true));
  TRY(band_bwd_dq(q, k, v, dout, dtau_local, bias, out, mass, dq, ws, sh, wl, scale, flags | TENSION_NORM_MASS,
                  stream, true));
  return band_bwd_dkv(q, k, v, dout, dtau_local, bias, out, mass, dk, dv, ws, sh, wl, scale,
                      flags | TENSION_NORM_MASS, stream, true);
}

int tension_decode_step(const tension_buf* q, const tension_buf* k_new, const tension_buf* v_new,
                        const tension_buf* k_cache, const tension_buf* v_cache, const tension_buf* out,
                        const tension_buf* tau, const int32_t* pos_in, int32_t* pos_out, int64_t N, int64_t H,
                        int64_t D, int64_t W, double scale, int32_t flags, tension_stream_t stream) {
  if (N < 0 || H < 0 || D <= 0 || D > 256 || W < 1 || N * H > 0x3fffffff)
    return fail(TENSION_ERR_ARG, "decode: bad sizes N=%lld H=%lld D=%lld W=%lld", (long long)N, (long long)H,
                (long long)D, (long long)W);
  if (!(std::isfinite(scale) && scale != 0.0)) return fail(TENSION_ERR_ARG, "scale must be finite and non-zero");
  TRY(check3(q, "q", true, true));
  TRY(check3(k_new, "k_new", true, true));
  TRY(check3(v_new, "v_new", true, true));
  TRY(check3(out, "out", true, true));
  TRY(check4(k_cache, "k_cache", true));
  TRY(check4(v_cache, "v_cache", true));
  if (tau) TRY(check3(tau, "tau", true, true));
  if (!pos_in) return fail(TENSION_ERR_ARG, "pos_in is required");
  if (pos_out && pos_out == pos_in) return fail(TENSION_ERR_ARG, "pos_out must not alias pos_in");
  if (k_cache->dtype != k_new->dtype || v_cache->dtype != v_new->dtype)
    return fail(TENSION_ERR_ARG, "cache and new-token dtypes must match");
  if (N * H == 0) return ok();
  DecodeParams p;
  memset(&p, 0, sizeof p);
  p.q = make_buf(q); p.kn = make_buf(k_new); p.vn = make_buf(v_new);
  p.kc = make_buf(k_cache); p.vc = make_buf(v_cache); p.out = make_buf(out); p.tau = make_buf(tau);
  p.pos_in = pos_in; p.pos_out = pos_out;
  p.N = (int)N; p.H = (int)H; p.D = (int)D; p.W = (int)W;
  p.scale = scale; p.flags = flags;
  auto a16 = [](const tension_buf* b, bool four) {
    if (b->dtype != TENSION_BF16 || ((uintptr_t)b->ptr & 15)) return false;
    return b->s[0] % 8 == 0 && b->s[1] % 8 == 0 && (!four || b->s[2] % 8 == 0);
  };
  const bool fast = !(flags & TENSION_FORCE_EXACT) && D == 64 && W % 32 == 0 && W <= 512 && a16(q, false) &&
                    a16(k_new, false) && a16(v_new, false) && a16(out, false) && a16(k_cache, true) &&
                    a16(v_cache, true);
  hipError_t e = hipSuccess;
  launch_decode(fast, is_f64(q) || is_f64(k_cache) || is_f64(v_cache), p, hs(stream), &e);
  return launched(e, "tension_decode_step");
}

int tension_rope(const tension_buf* x, const tension_buf* y, const float* cos, const float* sin,
                 int64_t table_rows, int64_t B, int64_t T, int64_t H, int64_t D, int64_t pos_offset,
                 int32_t inverse, tension_stream_t stream) {
  TRY(check_shape(Shape{B, T, H, D}, 1.0));
  if (D % 2) return fail(TENSION_ERR_ARG, "rope: head dim must be even");
  if (pos_offset < 0) return fail(TENSION_ERR_ARG, "rope: negative position offset");
  if (pos_offset + T > table_rows)
    return fail(TENSION_ERR_ARG, "rope: table has %lld rows, positions up to %lld requested",
                (long long)table_rows, (long long)(pos_offset + T));
  TRY(check4(x, "x", true));
  TRY(check4(y, "y", true));
  if (!cos || !sin) return fail(TENSION_ERR_ARG, "rope: cos/sin tables are required");
  if (B * T * H == 0) return ok();
  RopeParams p;
  memset(&p, 0, sizeof p);
  p.x = make_buf(x); p.y = make_buf(y); p.cos = cos; p.sin = sin;
  p.B = (int)B; p.T = (int)T; p.H = (int)H; p.D = (int)D;
  p.pos_offset = pos_offset; p.inverse = inverse;
  hipError_t e = hipSuccess;
  launch_rope(is_f64(x) || is_f64(y), p, hs(stream), &e);
  return launched(e, "tension_rope");
}

}  // extern "C"
