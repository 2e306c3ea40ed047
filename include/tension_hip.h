/*
 * tension_hip.h -- C ABI of the MI355X (gfx950) sigmoid-tension library
 * (libtension_hip.so).
 *
 * The reference has no native FFI for this path: its boundary is the Python
 * autograd op `causal_tension(Q, K, V, window, scale, return_tau=False,
 * bias=None)` (triton_tension/ops.py:192-224), which launches three Triton
 * kernels with raw pointers, sizes and strides (ops.py:104-112,165-182;
 * kernel.py:42-55,131-144,233-246).  The entry points below replace those
 * launches one for one; the Python host layer (bozo_amd/ops.py) binds them
 * with ctypes.
 *
 * Conventions
 *  - Every tensor is described by a tension_buf: device pointer, dtype code,
 *    and element strides.  4-D activations are [B,T,H,D] with strides
 *    s[0..3] for (B,T,H,D); s[3] must be 1.  tau is [B,T,H,W] (s[3] == 1),
 *    bias [B,T,W] (local) or [B,T,T] (global) uses s[0..2] and needs
 *    s[2] == 1; mass is [B,T,H] (s[0..2]).
 *  - A NULL tension_buf pointer means "absent" (no tau, no bias, ...).
 *  - The library never allocates device memory.  Work is enqueued on the
 *    given stream; no call synchronises the device.  All functions are
 *    reentrant; the only global state is the per-thread error string and
 *    the fixed device scratch of tension_global_bwd_noalloc.
 *  - Return value: TENSION_OK or a TENSION_ERR_* code; tension_last_error()
 *    describes the last failure on the calling thread.  Nothing throws
 *    across the ABI.
 */
#ifndef TENSION_HIP_H
#define TENSION_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* tension_stream_t; /* == hipStream_t */

/* dtype codes */
enum {
  TENSION_F32 = 0,
  TENSION_BF16 = 1,
  TENSION_F16 = 2,
  TENSION_F64 = 3
};

/* status codes */
enum {
  TENSION_OK = 0,
  TENSION_ERR_ARG = 1,         /* bad pointer / shape / stride / dtype combination */
  TENSION_ERR_UNSUPPORTED = 2, /* valid request this build has no kernel for (e.g. D) */
  TENSION_ERR_LAUNCH = 3       /* hipGetLastError() after the launch was not hipSuccess */
};

/* flags */
enum {
  /* out = msg / max(sum_w tau, 1e-6)        (model.py:257-258,281-282) */
  TENSION_NORM_MASS = 1 << 0,
  /* out = msg / max(min(t, W), 1)            (model.py:159-163,264) */
  TENSION_NORM_COUNT = 1 << 1,
  /* bias is [B,T,T] indexed by key position (global block, model.py:224-225) */
  TENSION_GLOBAL = 1 << 2,
  /* force the exact (non-MFMA) kernels even when the MFMA path applies */
  TENSION_FORCE_EXACT = 1 << 3,
  /* decode: the new token is also a key (keys s <= t, the global block's
   * diagonal, model.py:221) */
  TENSION_DECODE_SELF = 1 << 4
};

typedef struct tension_buf {
  void* ptr;
  int32_t dtype;
  int32_t reserved;
  int64_t s[4];
} tension_buf;

/* ---------------------------------------------------------------------------
 * Local window forward.  Replaces `_fwd_kernel` (kernel.py:41-125) launched by
 * `_CausalTensionFn.forward` (ops.py:75-124).
 *   tau[b,t,h,w] = sigmoid(q_t . k_s / scale + bias[b,t,w]),  s = t-(W-w),
 *                  0 where s < 0;  msg = sum_w tau * v_s.
 *   out = msg (raw, the reference contract), or normalised per flags.
 *   q,k,v,out: [B,T,H,D]; tau (nullable, out): [B,T,H,W], written fully
 *   (zeros on empty slots); bias (nullable): [B,T,W];
 *   mass (nullable, out): [B,T,H] = sum_w tau (unclamped), f32 or f64.
 * ------------------------------------------------------------------------- */
int tension_window_fwd(const tension_buf* q, const tension_buf* k,
                       const tension_buf* v, const tension_buf* out,
                       const tension_buf* tau, const tension_buf* bias,
                       const tension_buf* mass, int64_t B, int64_t T,
                       int64_t H, int64_t D, int64_t W, double scale,
                       int32_t flags, tension_stream_t stream);

/* Bytes of device workspace tension_window_bwd needs (0 if none; -1 for
 * sizes the entry points reject: negative, or B*T*H above 2^40). */
int64_t tension_window_bwd_workspace(int64_t B, int64_t T, int64_t H,
                                     int32_t dtype_acc, int32_t flags);

/* ---------------------------------------------------------------------------
 * Local window backward.  Replaces `_bwd_dq_kernel` + `_bwd_dkv_kernel`
 * (kernel.py:130-341) launched by `_CausalTensionFn.backward`
 * (ops.py:126-187).  For windows W <= 64 with bf16 rows (head dim 64,
 * 16-byte aligned rows) it launches one kernel that produces dQ, dK and
 * dV in a single pass; otherwise tension_window_bwd_dq then
 * tension_window_bwd_dkv on `stream`.  Recomputes tau from q, k (and
 * bias); nothing from the forward is needed besides the inputs.
 *   dout: grad of out (of the raw msg without a NORM flag, of the
 *   normalised output with one); dtau (nullable): grad of tau [B,T,H,W];
 *   bias: as in the forward (sigma' is taken at the biased argument,
 *   kernel.py:24-29; bias gets no gradient).  dq/dk/dv are written, not
 *   accumulated, in their own dtypes.
 *   workspace: tension_window_bwd_workspace() bytes (NULL if that is 0);
 *   with TENSION_NORM_MASS it carries per-query coefficients from the dq
 *   kernel to the dkv kernel (the single-pass kernel forms them in
 *   registers and leaves the workspace untouched; it is required either
 *   way, so callers need not know which kernel runs).
 * ------------------------------------------------------------------------- */
int tension_window_bwd(const tension_buf* q, const tension_buf* k,
                       const tension_buf* v, const tension_buf* dout,
                       const tension_buf* dtau, const tension_buf* bias,
                       const tension_buf* dq, const tension_buf* dk,
                       const tension_buf* dv, void* workspace, int64_t B,
                       int64_t T, int64_t H, int64_t D, int64_t W,
                       double scale, int32_t flags, tension_stream_t stream);

/* tension_window_bwd with the forward's output rows `out` ([B,T,H,D], as
 * written by tension_window_fwd) and tau mass `mass` ([B,T,H] f32, the
 * forward's `mass` output), both required.  No counterpart in the reference
 * (its backward recomputes everything, ops.py:126-187): with
 * TENSION_NORM_MASS on the float32-Q/K split kernels and a window wider
 * than 64 the per-query coefficients then come from these rows --
 * a = 1/max(m, 1e-6), c = dout.out * a (0 where m < 1e-6) -- in one pass
 * over the band instead of two; every other case computes them as
 * tension_window_bwd does.  Same results to float32 rounding. */
int tension_window_bwd_saved(const tension_buf* q, const tension_buf* k,
                             const tension_buf* v, const tension_buf* dout,
                             const tension_buf* dtau, const tension_buf* bias,
                             const tension_buf* out, const tension_buf* mass,
                             const tension_buf* dq, const tension_buf* dk,
                             const tension_buf* dv, void* workspace, int64_t B,
                             int64_t T, int64_t H, int64_t D, int64_t W,
                             double scale, int32_t flags, tension_stream_t stream);

/* The two halves of tension_window_bwd, one kernel each.  _dq fills the
 * workspace that _dkv reads, so on one stream _dq must precede _dkv.
 * Counterparts: kernel.py:130-227 (dQ) and kernel.py:232-341 (dK/dV). */
int tension_window_bwd_dq(const tension_buf* q, const tension_buf* k,
                          const tension_buf* v, const tension_buf* dout,
                          const tension_buf* dtau, const tension_buf* bias,
                          const tension_buf* dq, void* workspace, int64_t B,
                          int64_t T, int64_t H, int64_t D, int64_t W,
                          double scale, int32_t flags, tension_stream_t stream);
int tension_window_bwd_dkv(const tension_buf* q, const tension_buf* k,
                           const tension_buf* v, const tension_buf* dout,
                           const tension_buf* dtau, const tension_buf* bias,
                           const tension_buf* dk, const tension_buf* dv,
                           void* workspace, int64_t B, int64_t T, int64_t H,
                           int64_t D, int64_t W, double scale, int32_t flags,
                           tension_stream_t stream);

/* ---------------------------------------------------------------------------
 * Global (full causal, diagonal included) block, tau-mass normalised.
 * Replaces the PyTorch einsum path of the global layer (model.py:217-238);
 * the reference has no kernel for it.
 *   bias (nullable): [B,T,T] indexed [b,t,s].
 *   tau_local (nullable, out): [B,T,H,Wl] with slot j = key s = T-1-j
 *   (model.py:231-237), zero where s > t.  mass (nullable, out): [B,T,H]
 *   = sum_s tau (unclamped).
 * ------------------------------------------------------------------------- */
int tension_global_fwd(const tension_buf* q, const tension_buf* k,
                       const tension_buf* v, const tension_buf* out,
                       const tension_buf* tau_local, const tension_buf* bias,
                       const tension_buf* mass, int64_t B, int64_t T,
                       int64_t H, int64_t D, int64_t Wl, double scale,
                       int32_t flags, tension_stream_t stream);

/* Bytes of device workspace tension_global_bwd needs (-1 as above). */
int64_t tension_global_bwd_workspace(int64_t B, int64_t T, int64_t H,
                                     int32_t dtype_acc, int32_t flags);

/* Backward of tension_global_fwd: dout (grad of out), dtau_local
 * (nullable, grad of tau_local [B,T,H,Wl]); recomputes tau like the local
 * backward.  workspace: tension_global_bwd_workspace() bytes (required).
 *   out, mass (nullable, in): the forward's output and mass.  When both are
 *   given (bf16 out, f32 mass, the bf16 head-dim-64 kernels), the per-query
 *   coefficients 1/m_t and dO_t.out_t/m_t come from one pass over these rows
 *   instead of a recompute of the whole causal band; otherwise they are
 *   ignored and the band is recomputed. */
int tension_global_bwd(const tension_buf* q, const tension_buf* k,
                       const tension_buf* v, const tension_buf* dout,
                       const tension_buf* dtau_local, const tension_buf* bias,
                       const tension_buf* out, const tension_buf* mass,
                       const tension_buf* dq, const tension_buf* dk,
                       const tension_buf* dv, void* workspace, int64_t B,
                       int64_t T, int64_t H, int64_t D, int64_t Wl,
                       double scale, int32_t flags, tension_stream_t stream);

/* ---------------------------------------------------------------------------
 * tension_global_bwd without a caller workspace.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments and results as tension_global_bwd minus
 * `workspace`; the per-query coefficients live in a fixed device array inside
 * the library, TENSION_NOALLOC_SCRATCH_BYTES per GPU (one copy per device,
 * held until the process ends; its address is looked up on the first call
 * with that device current).  The call allocates nothing.  It needs
 * 2 * B * T * H * 4 bytes (8 with f64 activations) of that array; larger
 * requests return TENSION_ERR_ARG.  Every call on one GPU shares the array:
 * calls that overlap on one GPU (several streams, several host threads) race
 * and must be serialised by the caller.
 * ------------------------------------------------------------------------- */
#define TENSION_NOALLOC_SCRATCH_BYTES (8 << 20)

int tension_global_bwd_noalloc(const tension_buf* q, const tension_buf* k,
                               const tension_buf* v, const tension_buf* dout,
                               const tension_buf* dtau_local,
                               const tension_buf* bias, const tension_buf* out,
                               const tension_buf* mass, const tension_buf* dq,
                               const tension_buf* dk, const tension_buf* dv,
                               int64_t B, int64_t T, int64_t H, int64_t D,
                               int64_t Wl, double scale, int32_t flags,
                               tension_stream_t stream);

/* ---------------------------------------------------------------------------
 * Streaming decode step over a ring K/V cache (no reference kernel: the
 * reference re-runs the whole forward per token, model.py:617-652,719-768;
 * the streaming exporter reads tau[:, -1], ts_bridge/streaming.py:125-127).
 *   q, k_new, v_new, out: [N,H,D] (s[0..2] used, s[2] == 1).
 *   k_cache, v_cache: [N,H,W,D] (s[0..3], s[3] == 1), updated in place:
 *   after attending, k_new/v_new are written to slot pos[n] % W.
 *   pos_in: device int32 [N], tokens already cached per sequence.
 *   pos_out (nullable): device int32 [N], receives pos_in + 1 (must not
 *   alias pos_in).  tau (nullable, out): [N,H,W], w=0 oldest.
 *   Attends to the min(pos, W) most recent cached tokens (strictly past),
 *   plus the new token itself with TENSION_DECODE_SELF (a global layer's
 *   step: the cache then holds every earlier token, W >= positions; tau
 *   must be null).
 *   flags: TENSION_NORM_MASS (tau-mass normalised), TENSION_NORM_COUNT
 *   (divided by the number of keys, max(min(pos, W), 1) for a local layer,
 *   the valid count of model.py:159-163,264) or neither (raw); optionally
 *   TENSION_DECODE_SELF.
 * ------------------------------------------------------------------------- */
int tension_decode_step(const tension_buf* q, const tension_buf* k_new,
                        const tension_buf* v_new, const tension_buf* k_cache,
                        const tension_buf* v_cache, const tension_buf* out,
                        const tension_buf* tau, const int32_t* pos_in,
                        int32_t* pos_out, int64_t N, int64_t H, int64_t D,
                        int64_t W, double scale, int32_t flags,
                        tension_stream_t stream);

/* ---------------------------------------------------------------------------
 * RoPE (half-split rotation, model.py:54-81).  y = R(pos) x, or R(pos)^T x
 * when inverse != 0 (the backward).  cos/sin: contiguous float32
 * [table_rows, D/2] tables (the model's buffers); rows
 * pos_offset .. pos_offset+T-1 are used and must exist.
 * x, y: [B,T,H,D]; y may alias x.  A negative pos_in entry of
 * tension_decode_step is read as 0.
 * ------------------------------------------------------------------------- */
int tension_rope(const tension_buf* x, const tension_buf* y, const float* cos,
                 const float* sin, int64_t table_rows, int64_t B, int64_t T,
                 int64_t H, int64_t D, int64_t pos_offset, int32_t inverse,
                 tension_stream_t stream);

/* ---------------------------------------------------------------------------
 * tau export reductions (replace the host numpy passes of the reference's
 * graph exporter over .cpu() copies of tau).  taus: L <= 32 buffers of
 * tau [B,T,H,W] (s[3] == 1, any float dtype), one per local layer; every
 * statistic reads the batch mean of tau.
 *
 * tension_tau_head_stats -- ts_bridge/head_filter.py:98-130 (profile_heads)
 *   and, with TENSION_TAU_VALID_ONLY (cells with t + w < W read as 0),
 *   ts_bridge/corpus_profile.py:58-98 (_per_head_stats).  stats: device
 *   float [L,H,4] = mean over (t, w); 0.99 quantile over (t, w) (linear
 *   interpolation, numpy's default); mean over t of the first arg-max over
 *   w; mean over t of the max over w.
 * ------------------------------------------------------------------------- */
enum { TENSION_TAU_VALID_ONLY = 1 << 5 };

int tension_tau_head_stats(const tension_buf* taus, int32_t L, int64_t B,
                           int64_t T, int64_t H, int64_t W, float* stats,
                           int32_t flags, tension_stream_t stream);

/* tension_tau_aggregate -- ts_bridge/export.py:185-200 (and the per-step
 *   form of streaming.py:127-146): agg[t,w] (device float [T,W]) = mean over
 *   the selected (layer, head) pairs of tau; head_mask: device int32 [L,H],
 *   nonzero = selected; all pairs when none is.  H <= 64. */
int tension_tau_aggregate(const tension_buf* taus, int32_t L, int64_t B,
                          int64_t T, int64_t H, int64_t W,
                          const int32_t* head_mask, float* agg,
                          tension_stream_t stream);

/* ---------------------------------------------------------------------------
 * The model's tau regularisers (model.py:498-611: tension_diversity_loss,
 * constraint_consistency_loss, tension_entropy_loss) over the tau of L <= 32
 * layers, each [B,T,H,W] (W <= 256, s[3] == 1), computed in fp32.
 *
 * tension_aux_loss_fwd: partials (device double [L, P, 4], P =
 *   tension_aux_loss_partials(B,T,H)) receives, per layer and workgroup, the
 *   sums of: row entropy -sum p log(p + 1e-8) with p = tau / (sum tau +
 *   1e-8); the consistency terms relu(tau[r,w1-1] tau[r-1,0] - tau[r,w1])
 *   (w1 = 1..min(W-2,4), w1+1 <= r <= w1+T-min(W-2,4)-1); relu(0.05 - m);
 *   relu(m - 0.8), m the row mean.  The caller sums over P and forms the
 *   losses.
 * tension_aux_loss_bwd: dtaus[l] = k_div[l] d(row entropy)/dtau
 *   + k_cons[l] d(consistency terms)/dtau + k_ent[l] d(relu sums)/dtau,
 *   coef = device float [L, 3] (k_div, k_cons, k_ent); every element of
 *   every dtau is written.
 * ------------------------------------------------------------------------- */
int64_t tension_aux_loss_partials(int64_t B, int64_t T, int64_t H);

int tension_aux_loss_fwd(const tension_buf* taus, int32_t L, int64_t B,
                         int64_t T, int64_t H, int64_t W, double* partials,
                         tension_stream_t stream);

int tension_aux_loss_bwd(const tension_buf* taus, const tension_buf* dtaus,
                         int32_t L, int64_t B, int64_t T, int64_t H,
                         int64_t W, const float* coef,
                         tension_stream_t stream);

/* ---------------------------------------------------------------------------
 * Graph-bias builder (ts_bridge/bias.py:125-233 GraphBias.local_bias /
 * global_bias, whose O(T W) / O(T^2) host loops look up a content-pair ->
 * weight map per (query, key)).  The map lives on the device as an
 * open-addressing table: keys uint64 (src_id << 32 | dst_id), values double,
 * capacity 2^log2cap, empty slots hold ~0 (fill table_keys with 0xff bytes
 * first).  Hash: slot = (key * 0x9E3779B97F4A7C15) >> (64 - log2cap) (mod
 * 2^64), linear probing.
 *
 * tension_bias_table_insert: insert n distinct keys (2 n <= capacity).
 * tension_bias_build: content_ids device int32 [T] (-1 = no entry); bias
 *   [B,T,W] (W > 0, key s = t - (W - w), zero where s < 0) or [B,T,T]
 *   (W == 0, keys s < t), s[2] == 1, any float dtype; every element written:
 *   alpha * weight(ids[s] -> ids[t]) where the weight is > 0, else 0.
 *   stats (nullable, device double [3], caller-zeroed): += hits, += sum of
 *   the hit weights, max of the hit weights.
 * ------------------------------------------------------------------------- */
int tension_bias_table_insert(const uint64_t* keys_in, const double* vals_in,
                              int64_t n, uint64_t* table_keys,
                              double* table_vals, int32_t log2cap,
                              tension_stream_t stream);

int tension_bias_build(const int32_t* content_ids, int64_t B, int64_t T,
                       int64_t W, const uint64_t* table_keys,
                       const double* table_vals, int32_t log2cap,
                       double alpha, const tension_buf* bias, double* stats,
                       tension_stream_t stream);

/* Message for the last non-OK return on the calling thread ("" if none). */
const char* tension_last_error(void);

/* Library version string. */
const char* tension_version(void);

/* Kernel family of the last band launch (window / global forward, dq, dkv)
 * on the calling thread: TENSION_KERNEL_* below, or -1 before the first.
 * No counterpart in the reference (its router picks Triton or PyTorch,
 * ops.py:217-219); it lets callers and tests see which path ran. */
enum {
  TENSION_KERNEL_EXACT = 0,      /* one thread per row, any dtype / head dim */
  TENSION_KERNEL_MFMA = 1,       /* dedicated bf16 kernels, head dim 64 */
  TENSION_KERNEL_SPLIT_BF16 = 2, /* split-operand kernels, bf16, head dim 32 / 64 */
  TENSION_KERNEL_SPLIT_F32 = 3,  /* split-operand kernels, float32 Q / K with bf16 V */
  TENSION_KERNEL_SPLIT_F32V = 4, /* split-operand kernels, float32 Q / K / V */
  TENSION_KERNEL_SPLIT_F16 = 5   /* split-operand kernels, float16 Q / K / V */
};
int tension_last_kernel(void);

#ifdef __cplusplus
}
#endif

#endif /* TENSION_HIP_H */
