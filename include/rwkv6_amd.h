/*
 * rwkv6_amd.h — C ABI of the MI355X (gfx950) RWKV-6 time-mix hot path.
 *
 * One shared library, librwkv6_amd.so, built from the .hip sources in rwkv-megatron_amd/csrc.
 * Plain pointers and sizes only: no torch or C++ types cross this boundary.
 *
 * Conventions shared by every entry point
 *   - All pointers are device pointers, owned by the caller (the library never
 *     allocates, frees or synchronises the host).  Work is enqueued on `stream`
 *     (a hipStream_t; NULL = the default stream).
 *   - Tensors are dense, row-major, and 16-byte aligned.
 *   - Outputs (workspace included) must not overlap inputs or each other; an entry point
 *     that finds an overlap returns RWKV6_ERR_INVALID_ARG without launching.
 *   - Return value: RWKV6_OK or an rwkv6_status code; rwkv6_strerror() maps it
 *     to text.  Validation failures never launch anything.
 *   - Calls are re-entrant: no mutable global state; the same inputs give
 *     bit-identical outputs (no floating-point atomics anywhere).
 *
 * Reference interface each group replaces (TimeMobius/RWKV-Megatron):
 *   WKV6      fla `fused_recurrent_rwkv6` / `chunk_rwkv6` as called at
 *             rwkv_megatron/rwkv6_layer_specs.py:339 (layout glue :330-341)
 *   mix       token shift + lerp + data-dependent lerp of RWKV6TimeMix.forward,
 *             rwkv6_layer_specs.py:290-300 and :440-452 (bias of :195 folded in)
 *   gn_gate   GroupNorm (rwkv6_layer_specs.py:90-97) applied at :461-465, times
 *             the silu gate of :458, the product formed at :466
 *   lora      LoRA up-projections of RWKV6Bottleneck (:177-195) fused with the ddlerp
 *             of :447-452 or the decay bias of :454
 *   cmix      token shift + static lerp, relu^2 and sigmoid gate of
 *             RWKV6ChannelMix.forward, rwkv6_layer_specs.py:512-536
 */
#ifndef RWKV6_AMD_H
#define RWKV6_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RWKV6_ABI_VERSION 3

enum rwkv6_status {
    RWKV6_OK = 0,
    RWKV6_ERR_INVALID_ARG = 1, /* null pointer, bad size, bad dtype code */
    RWKV6_ERR_UNSUPPORTED = 2, /* e.g. head size other than 64 */
    RWKV6_ERR_LAUNCH = 3,      /* hipGetLastError() after a launch */
    RWKV6_ERR_ALIGNMENT = 4    /* a tensor pointer is not 16-byte aligned */
};

enum rwkv6_dtype { RWKV6_F32 = 0, RWKV6_BF16 = 1 };

int rwkv6_abi_version(void);
const char* rwkv6_strerror(int code);

/* ------------------------------------------------------------------------
 * WKV6.  Replaces fla.ops.rwkv6.fused_recurrent_rwkv6 / chunk_rwkv6
 * (call site rwkv_megatron/rwkv6_layer_specs.py:339).
 *   r, k, w : [B,H,T,K] bf16 (w = log-space decay, as the caller passes -exp(decay), :336)
 *   v, o    : [B,H,T,V] bf16
 *   u       : [H,K] in u_dtype (f32 or bf16; time_first viewed per head, :337)
 *   h0, hT  : [B,H,K,V] f32, each nullable (initial_state / output_final_state)
 *   scale   : multiplies r (the reference passes 1.0)
 * Only K == V == 64 (RWKV-6 head size) is supported; T >= 0 arbitrary.
 * Per-token log-decay is floored at -10 (decay factor 4.5e-5; the chunked evaluation
 * keeps 8-token decay products inside the bf16 exponent range): tokens below the floor
 * change outputs and states by less than that factor; their dw (d_decay in the
 * sequence-first entry) is 0, the derivative of the floored forward.
 * `saved` (rwkv6_wkv_saved_bytes) receives the bf16 state entering every chunk
 * (and the final state), which the backward consumes; keep it alive until
 * rwkv6_wkv_bwd.  `workspace` (rwkv6_wkv_workspace_bytes) is scratch for the duration
 * of one call.
 * ---------------------------------------------------------------------- */
size_t rwkv6_wkv_saved_bytes(int64_t B, int64_t H, int64_t T, int64_t K, int64_t V);
size_t rwkv6_wkv_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t K, int64_t V,
                                 int for_bwd);

int rwkv6_wkv_fwd(const void* r, const void* k, const void* v, const void* w, const void* u,
                  int u_dtype, const float* h0, void* o, float* hT, void* saved,
                  void* workspace, int64_t B, int64_t H, int64_t T, int64_t K, int64_t V,
                  float scale, void* stream);

/* Gradients of rwkv6_wkv_fwd for loss terms on o (dO, bf16 [B,H,T,V]) and on the
 * final state (dhT, f32 [B,H,K,V], nullable = zero).  dr, dk, dw: [B,H,T,K] bf16;
 * dv: [B,H,T,V] bf16; du: [H,K] in u_dtype; dh0: [B,H,K,V] f32, nullable. */
int rwkv6_wkv_bwd(const void* r, const void* k, const void* v, const void* w, const void* u,
                  int u_dtype, const void* dO, const float* dhT, const void* saved, void* dr,
                  void* dk, void* dv, void* dw, void* du, float* dh0, void* workspace,
                  int64_t B, int64_t H, int64_t T, int64_t K, int64_t V, float scale,
                  void* stream);

/* Sequence-first variant for the time-mix module (the layout of WKV6.forward's inputs
 * before its rearranges, rwkv6_layer_specs.py:330-336): r, k, v and `decay` are
 * [T,B,H*K] bf16 straight from the linear layers, the log-decay w = -exp(decay) of :336 is
 * evaluated inside the kernels, o and dO stay head-first [B,H,T,V] (the layout
 * rwkv6_gn_gate_* reads with head_first=1).  The backward writes dr, dk, dv and
 * d_decay = dw * w in [T,B,H*K].  Same `saved` / `workspace` sizes as the head-first calls. */
int rwkv6_wkv_fwd_seqfirst(const void* r, const void* k, const void* v, const void* decay,
                           const void* u, int u_dtype, const float* h0, void* o, float* hT,
                           void* saved, void* workspace, int64_t B, int64_t H, int64_t T,
                           int64_t K, int64_t V, float scale, void* stream);
int rwkv6_wkv_bwd_seqfirst(const void* r, const void* k, const void* v, const void* decay,
                           const void* u, int u_dtype, const void* dO, const float* dhT,
                           const void* saved, void* dr, void* dk, void* dv, void* d_decay,
                           void* du, float* dh0, void* workspace, int64_t B, int64_t H,
                           int64_t T, int64_t K, int64_t V, float scale, void* stream);

/* ------------------------------------------------------------------------
 * Token shift and static lerp of RWKV6TimeMix.forward, sequence-first [T,B,C] bf16.
 *   shift(x)[t] = x[t-1], shift(x)[0] = 0              (rwkv6_layer_specs.py:294-300)
 *   xxx         = x + (shift(x) - x) * maa              (:443-444), maa [C] in param_dtype
 * C must be a multiple of 8.  The data-dependent lerp of :446-452 is written by
 * rwkv6_ddlerp_lora_fwd below, whose backward (with rwkv6_shift_lerp_bwd) covers both lerps.
 * ---------------------------------------------------------------------- */
int rwkv6_shift_lerp_fwd(const void* x, const void* maa, int param_dtype, void* xxx,
                         int64_t T, int64_t B, int64_t C, void* stream);

/* ------------------------------------------------------------------------
 * LoRA up-projections fused with their consumers (RWKV6Bottleneck.forward,
 * rwkv6_layer_specs.py:177-195, as used at :446-454).  The caller computes
 * neck = tanh(input @ W_down) as [N, E*R] bf16 (N = T*B tokens, a hipBLASLt GEMM) and passes
 * W_up transposed: w_up_t [E, C, R] bf16 (w_up_t[e][c][r] = weight_up[e][r][c]).  R must be a
 * multiple of 32 (E = 5: R = 32; E = 1: R <= 128) and C a multiple of 64.  bias [E, C] in
 * param_dtype.
 *   ddlerp_lora: E = 5, mixed[e] = x + (shift(x) - x) * (neck_e @ W_up[e] + bias[e]), the five
 *                mixes written straight to `mixed` (host array of 5 device pointers, [T,B,C])
 *   lora_bias:   E = 1 or 5, out[n][e] = neck_e[n] @ W_up[e] + bias[e]: the bottleneck's own
 *                output [N, E, C] (:195); for E = 1 the decay of :454 ([N, C])
 * ---------------------------------------------------------------------- */
int rwkv6_ddlerp_lora_fwd(const void* x, const void* neck, const void* w_up_t, const void* bias,
                          int param_dtype, void* const* mixed, int64_t T, int64_t B, int64_t C,
                          int64_t R, void* stream);
int rwkv6_lora_bias_fwd(const void* neck, const void* w_up_t, const void* bias, int param_dtype,
                        void* out, int64_t N, int64_t E, int64_t C, int64_t R, void* stream);
/* Backward of rwkv6_ddlerp_lora_fwd for d_mixed (5 device pointers, [T,B,C] bf16):
 *   d_mexp [5,N,C] bf16 = d_mixed * (shift(x) - x)   (the LoRA up-projection's output gradient)
 *   d_delta_part [N,C] bf16 = sum_e d_mixed_e (m_e + bias_e),   d_sum [N,C] bf16 = sum_e d_mixed_e
 *   (summed in fp32, rounded once), d_bias [5,C] (param_dtype).  m is recomputed on MFMA from
 *   neck and w_up_t. */
size_t rwkv6_ddlerp_lora_bwd_workspace_bytes(int64_t T, int64_t B, int64_t C);
int rwkv6_ddlerp_lora_bwd(const void* x, const void* neck, const void* w_up_t, const void* bias,
                          int param_dtype, const void* const* d_mixed, void* d_mexp,
                          void* d_delta_part, void* d_sum, void* d_bias, void* workspace,
                          int64_t T, int64_t B, int64_t C, int64_t R, void* stream);
/* Backward of the bottleneck's tanh (autograd of torch.tanh at rwkv6_layer_specs.py:195):
 *   d_pre[n][e*R + r] = d_neck(e, n, r) * (1 - neck[n][e*R + r]^2)
 * with d_neck(e, n, r) at d_neck + e*sE + n*sN + r (bf16; sE = N*R, sN = R for the batched
 * [E,N,R] GEMM output, sE = R, sN = E*R for [N,E,R]), neck and d_pre [N, E*R] bf16.  R, sE,
 * sN multiples of 8. */
int rwkv6_lora_tanh_bwd(const void* d_neck, int64_t sE, int64_t sN, const void* neck, void* d_pre,
                        int64_t N, int64_t E, int64_t R, void* stream);
/* out[m] = sum_n x[n][m] for x [N, M] bf16 (M a multiple of 8), summed in fp32 in a fixed order
 * and written in param_dtype: the bias gradient of a bottleneck (autograd of the `+ bias` at
 * rwkv6_layer_specs.py:195), N = tokens, M = E*C. */
size_t rwkv6_col_sum_workspace_bytes(int64_t N, int64_t M);
int rwkv6_col_sum(const void* x, int64_t N, int64_t M, int param_dtype, void* out,
                  void* workspace, void* stream);
/* Input gradient of the time-mix token mixing given d_xxx [T,B,C] bf16 (the gradient of
 * xxx = x + (shift(x) - x) * maa, :443-444, from the LoRA down-projection) and the two sums of
 * rwkv6_ddlerp_lora_bwd:  d_delta = d_delta_part + d_xxx * maa,
 * dx = d_sum + d_xxx - d_delta + shift^T(d_delta) -> dx [T,B,C] bf16, d_maa [C] (param_dtype). */
size_t rwkv6_shift_lerp_bwd_workspace_bytes(int64_t T, int64_t B, int64_t C);
int rwkv6_shift_lerp_bwd(const void* x, const void* maa, int param_dtype, const void* d_delta_part,
                         const void* d_sum, const void* d_xxx, void* dx, void* d_maa,
                         void* workspace, int64_t T, int64_t B, int64_t C, void* stream);

/* ------------------------------------------------------------------------
 * Channel mix (RWKV6ChannelMix.forward, rwkv6_layer_specs.py:512-536), [T,B,C] bf16.
 *   mixed[e] = x + (shift(x) - x) * mix[e]    (:513-520), mix = mix_coeffs [2,C] in
 *              param_dtype; `mixed` is a host array of 2 device pointers, each [T,B,C]:
 *              e = 0 feeds linear_up, e = 1 linear_gate (d_mixed likewise)
 *   h        = relu(up)^2                     (:524), up = linear_up output
 *   y        = out * sigmoid(gate_pre)        (:533-536), out = linear_down output
 * The elementwise entries take n = element count (a multiple of 8).
 * ---------------------------------------------------------------------- */
int rwkv6_cmix_lerp_fwd(const void* x, const void* mix, int param_dtype, void* const* mixed,
                        int64_t T, int64_t B, int64_t C, void* stream);
/* d_mixed 2 x [T,B,C] -> dx [T,B,C] and d_mix [2,C] (param_dtype). */
size_t rwkv6_cmix_lerp_bwd_workspace_bytes(int64_t T, int64_t B, int64_t C);
int rwkv6_cmix_lerp_bwd(const void* x, const void* mix, int param_dtype,
                        const void* const* d_mixed, void* dx, void* d_mix, void* workspace,
                        int64_t T, int64_t B, int64_t C, void* stream);
int rwkv6_relu_sq_fwd(const void* up, void* h, int64_t n, void* stream);
/* d_up = 2 relu(up) dh */
int rwkv6_relu_sq_bwd(const void* up, const void* dh, void* d_up, int64_t n, void* stream);
int rwkv6_sigmoid_gate_fwd(const void* out, const void* gate_pre, void* y, int64_t n,
                           void* stream);
/* d_out = dy sigmoid(gate_pre); d_gate_pre = dy out sigmoid'(gate_pre) */
int rwkv6_sigmoid_gate_bwd(const void* out, const void* gate_pre, const void* dy, void* d_out,
                           void* d_gate_pre, int64_t n, void* stream);

/* out[i] = sum_{j < S} part[j*n + i] in fp32, j in order, written in out_dtype (RWKV6_F32 or
 * RWKV6_BF16); n a multiple of 8, 1 <= S <= 64.  No counterpart in the reference: the weight
 * gradient of each projection (autograd of linear_proj / linear_up / ... in
 * rwkv6_layer_specs.py) is computed here as S token-split partial GEMMs (to fill the device),
 * and this sums them in one pass. */
int rwkv6_sum_partials(const float* part, int64_t S, int64_t n, int out_dtype, void* out,
                       void* stream);

/* ------------------------------------------------------------------------
 * GroupNorm(per head) * silu(gate), fused with the head-first -> sequence-first
 * layout change of rwkv6_layer_specs.py:341 and :461-465.
 *   o      : WKV output, [B,H,T,K] bf16 (head_first=1) or [T,B,H*K] (head_first=0)
 *   g_pre  : [T,B,H*K] bf16, linear_gate output before silu (:458); nullable: without a
 *            gate, y = GN(o) is the reference's GroupNorm.forward over [N, C] (:90-97),
 *            called with head_first = 0, T = N, B = 1 (group size 64 only)
 *   gamma, beta : [H*K] in param_dtype; eps = config.layernorm_epsilon (:68)
 *   y      : [T,B,H*K] bf16 = GN(o) * silu(g_pre)
 *   mean, rstd : [T*B*H] f32 statistics saved for the backward
 * ---------------------------------------------------------------------- */
int rwkv6_gn_gate_fwd(const void* o, int head_first, const void* g_pre, const void* gamma,
                      const void* beta, int param_dtype, float eps, void* y, float* mean,
                      float* rstd, int64_t T, int64_t B, int64_t H, int64_t K, void* stream);
size_t rwkv6_gn_gate_bwd_workspace_bytes(int64_t T, int64_t B, int64_t H, int64_t K);
/* dy [T,B,H*K] -> d_o (layout of o), d_g_pre [T,B,H*K] (NULL exactly when g_pre is NULL),
 * dgamma, dbeta [H*K] (param_dtype). */
int rwkv6_gn_gate_bwd(const void* o, int head_first, const void* g_pre, const void* gamma,
                      const void* beta, int param_dtype, const float* mean, const float* rstd,
                      const void* dy, void* d_o, void* d_g_pre, void* dgamma, void* dbeta,
                      void* workspace, int64_t T, int64_t B, int64_t H, int64_t K,
                      void* stream);

/* ------------------------------------------------------------------------
 * Forward without a workspace argument.  No counterpart in the reference: for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Same arguments and results as rwkv6_wkv_fwd minus `workspace`:
 * the forward's scratch (the pre-pass pieces' states, at most 256, and the segments' start
 * states) lives in a library-owned device array of 8,454,144 bytes (8.06 MiB: 256 x (two fp32
 * 64x64 states + one fp32 64-vector)) per GPU (enough for every shape; larger needs return
 * RWKV6_ERR_UNSUPPORTED).  The call allocates nothing.  The first call on a GPU looks the
 * array's address up and raises the kernels' LDS limits (host API calls, once per GPU): make
 * that first call eagerly, before capturing later calls into a HIP graph.  A failed look-up is
 * retried by the next call.  Calls on one GPU share the array: they must not overlap in time
 * (concurrent calls on two streams of one GPU race).  The caller still provides o, hT and
 * `saved` (rwkv6_wkv_saved_bytes), which rwkv6_wkv_bwd consumes as after rwkv6_wkv_fwd.
 * ---------------------------------------------------------------------- */
int rwkv6_wkv_fwd_noalloc(const void* r, const void* k, const void* v, const void* w,
                          const void* u, int u_dtype, const float* h0, void* o, float* hT,
                          void* saved, int64_t B, int64_t H, int64_t T, int64_t K, int64_t V,
                          float scale, void* stream);

/* ------------------------------------------------------------------------
 * Measurement variants (no counterpart in the reference): identical to
 * rwkv6_wkv_fwd / rwkv6_wkv_bwd, and additionally record caller-created timing
 * hipEvent_t objects around each kernel phase on `stream` (phase_events may be
 * NULL, and so may any entry).  Index pairs (2p, 2p+1) bracket phase p:
 *   fwd: 0 segment-state pre-pass (only when B*H alone cannot fill the device),
 *        1 unused (empty), 2 the output walk
 *   bwd: 0 chunk-local dstates (chunk-parallel form only), 1 the reverse dstate walk or
 *        the dstate scan, 2 chunk gradients, 3 du reduction
 * ---------------------------------------------------------------------- */
int rwkv6_wkv_fwd_ex(const void* r, const void* k, const void* v, const void* w, const void* u,
                     int u_dtype, const float* h0, void* o, float* hT, void* saved,
                     void* workspace, int64_t B, int64_t H, int64_t T, int64_t K, int64_t V,
                     float scale, void* stream, void* const* phase_events);
int rwkv6_wkv_bwd_ex(const void* r, const void* k, const void* v, const void* w, const void* u,
                     int u_dtype, const void* dO, const float* dhT, const void* saved, void* dr,
                     void* dk, void* dv, void* dw, void* du, float* dh0, void* workspace,
                     int64_t B, int64_t H, int64_t T, int64_t K, int64_t V, float scale,
                     void* stream, void* const* phase_events);

#ifdef __cplusplus
}
#endif

#endif /* RWKV6_AMD_H */
