/*
 * pm_delta.h — C ABI of libpmdelta.so, the MI355X (gfx950) delta-rule
 * linear-attention forward and its single-token decode step.
 *
 * Recurrence (decay gate 1), per (batch b, head h), state S is d_k x d_v:
 *     S_t = (I - beta_t k_t k_t^T) S_{t-1} + beta_t k_t v_t^T
 *     o_t = q_t S_t                              (o_t[e] = sum_d q_t[d] S_t[d][e])
 *
 * Reference interfaces this ABI stands behind (teddytennant/prometheus):
 *   kernels/__init__.py:661-689  chunked_delta_rule_fwd   -> pm_delta_fwd
 *   kernels/__init__.py:591-619  chunked_delta_rule       -> pm_delta_fwd
 *   kernels/__init__.py:357-376  _delta_step_np/_jax      -> pm_delta_step
 *   kernels/__init__.py:692-719  chunked_delta_rule_bwd   -> pm_delta_bwd
 *   (no reference counterpart)   packed cu_seqlens batch  -> pm_delta_fwd_varlen
 * The reference has no FFI of its own: its call surface is Python
 * (kernels/__init__.py).  prometheus_amd/kernels binds these entry points
 * with ctypes under the reference's names.
 *
 * Layouts (all row-major, contiguous, device pointers):
 *   q, k, v  (B, T, H, D)        element type in_dtype
 *   beta     (B, T, H)           fp32
 *   s0/s_out (B, H, D, D)        fp32, [d_k][d_v]
 *   o        (B, T, H, D)        element type out_dtype
 * Varlen: q, k, v are (total_T, H, D), beta (total_T, H), cu_seqlens int32
 * (n_seqs + 1) exclusive prefix with cu_seqlens[0] == 0 and
 * cu_seqlens[n_seqs] == total_T; s0/s_out are (n_seqs, H, D, D).
 *
 * Return codes: 0 on success; a negative PM_E* value for an invalid
 * argument (nothing was launched); a positive hipError_t when a launch
 * failed.  pm_last_error() gives a thread-local message for the last
 * nonzero return on the calling thread.
 *
 * All launches are asynchronous on `stream` (a hipStream_t; NULL is the
 * default stream).  The library never synchronises the host and allocates
 * no device memory (pm_delta_bwd_noalloc's scratch is a static array).
 * Inputs and outputs must not alias, except that pm_delta_step updates
 * s_inout in place by design.
 */
#ifndef PM_DELTA_H
#define PM_DELTA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PM_DELTA_ABI_VERSION 13

/* element types */
#define PM_DTYPE_F32 0
#define PM_DTYPE_BF16 1

/* negative return codes */
#define PM_E_NULL (-1)        /* required pointer is NULL               */
#define PM_E_SHAPE (-2)       /* dimension out of range / inconsistent  */
#define PM_E_DTYPE (-3)       /* unknown or unsupported element type    */
#define PM_E_ALIGN (-4)       /* pointer not aligned for vector access  */
#define PM_E_WORKSPACE (-5)   /* workspace too small                    */
#define PM_E_UNSUPPORTED (-6) /* valid request this build cannot serve  */

/* Largest head dimension any entry point accepts. */
#define PM_DELTA_MAX_D 256

/*
 * Delta-rule forward over (B, T, H, D) inputs.
 * Replaces kernels/__init__.py:661-689 (chunked_delta_rule_fwd) and
 * :591-619 (chunked_delta_rule): same inputs, same (O, S) outputs.
 * s0 may be NULL (zero initial state, as `state=None` at :349-351).
 * chunk >= 1 is accepted as in the reference (:676-677); like the
 * reference it does not change the mathematical result (:92).
 * T == 0 gives no output rows and s_out = s0 (or zeros).
 * workspace/ws_bytes: optional device memory (16-byte aligned) of at least
 * pm_delta_workspace_bytes(B, T, H, D, in_dtype) bytes, which is nonzero
 * exactly when the call would run the split form of the chunked kernel: a
 * parallel pass builds every chunk's T diag(beta), T = (I + A)^-1, into the
 * workspace and the chunk recurrence loads it instead of building it.  By
 * default (pm_delta_set_path(0)) that is the case for bf16 inputs at D in
 * {64, 128} when B*H*(D/32) < 256 (the chunked kernel's 16-column tiles),
 * where the split form is the faster one.  Without the workspace the
 * single-stage chunked kernel runs, which needs none; the two agree within
 * the bf16 parity bound.  fp32 inputs at D in {64, 128} (16-byte aligned
 * q, k, v) run the chunked forward on fp32 MFMA, whose parallel pass writes
 * every 16-token chunk's (-T diag(beta))^T into the workspace (1 KiB per
 * (b, h) and chunk); without the workspace they run the per-token fp32
 * kernel.  Both are fp32 arithmetic (fp32 parity).  The library never
 * allocates.
 */
int pm_delta_fwd(const void* q, const void* k, const void* v, const float* beta,
                 const float* s0, void* o, float* s_out, int B, int T, int H, int D,
                 int in_dtype, int out_dtype, int chunk, void* workspace, size_t ws_bytes,
                 void* stream);

/*
 * Packed variable-length forward: n_seqs independent sequences
 * concatenated along the token axis, state reset at every boundary
 * (each segment equals a B=1 pm_delta_fwd call with s0 = NULL, bit for bit).
 * No reference counterpart: the reference's equivalent is n_seqs separate
 * chunked_delta_rule calls (kernels/__init__.py:591-619) with B=1.
 * s0 may be NULL (zeros) or (n_seqs, H, D, D).
 * workspace/ws_bytes as pm_delta_fwd, sized by pm_delta_varlen_workspace_bytes.
 * Where the single-stage bf16 kernel runs, its workgroups take the sequences
 * longest first (by chunk count, ties in index order): up to 64 sequences
 * ranked inside the kernel; beyond that the workspace holds the order
 * (computed on the device), and without it they go in cu_seqlens order.
 * Only the schedule changes: the results are the same bits either way.
 */
int pm_delta_fwd_varlen(const void* q, const void* k, const void* v, const float* beta,
                        const int32_t* cu_seqlens, int n_seqs, int total_T,
                        const float* s0, void* o, float* s_out, int H, int D,
                        int in_dtype, int out_dtype, int chunk, void* workspace,
                        size_t ws_bytes, void* stream);

/*
 * Device-side check of a packed batch's offsets, for callers whose cu_seqlens
 * already live on the device: no host copy and no synchronisation, so it can
 * be captured in a graph with the forward it guards.  One small kernel on
 * `stream` ORs into *flag (a device int32 the caller owns and reads when it
 * chooses):
 *   1: cu_seqlens[0] != 0            2: cu_seqlens[n_seqs] != total_T
 *   4: a decreasing pair             8: an offset outside [0, total_T]
 * pm_delta_fwd_varlen itself clamps every segment into [0, total_T], so bad
 * offsets never reach outside the buffers; this entry point reports them.
 * No reference counterpart: the reference has no packed batch, and its
 * callers' offsets would be host values checked in Python
 * (kernels/__init__.py:308-338 is where the reference validates shapes).
 */
int pm_varlen_check(const int32_t* cu_seqlens, int n_seqs, int total_T, int32_t* flag,
                    void* stream);

/*
 * One recurrent decode step for B*H sequences, state updated in place.
 * Replaces kernels/__init__.py:357-376 (_delta_step_np / _delta_step_jax):
 *   S' = S - beta k (k^T S) + beta k v^T ;  o = q S'
 * q, k, v: (B, H, D) in_dtype; beta (B, H) fp32; s_inout (B, H, D, D) fp32;
 * o: (B, H, D) fp32.
 */
int pm_delta_step(float* s_inout, const void* q, const void* k, const void* v,
                  const float* beta, float* o, int B, int H, int D, int in_dtype,
                  void* stream);

/*
 * The gated delta rule (Gated DeltaNet; the reference names it as its
 * model's intent, spec/03-model.md:12, and has no code for it:
 * PROGRESS.md:109).  No reference counterpart: the recurrence of
 * pm_delta_fwd with a per-(token, head) log-gate g, alpha = exp(g):
 *   S_t = alpha_t (I - beta_t k_t k_t^T) S_{t-1} + beta_t k_t v_t^T,  o_t = q_t S_t
 * g (B, T, H) fp32, NULL only when B*T*H == 0; everything else as
 * pm_delta_fwd (chunk 64).  bf16 q/k/v with D in {64, 128} run the chunked
 * MFMA kernel (in-chunk decays exp(G_t - G_s), at most 1 when g <= 0);
 * other inputs run the fp32 per-token kernel.
 */
int pm_gated_delta_fwd(const void* q, const void* k, const void* v, const float* beta,
                       const float* g, const float* s0, void* o, float* s_out, int B, int T, int H,
                       int D, int in_dtype, int out_dtype, void* stream);

/*
 * One gated step: S' = alpha (S - beta k (k^T S)) + beta k v^T, o = q S',
 * alpha = exp(g), g (B, H) fp32; otherwise as pm_delta_step.
 */
int pm_gated_delta_step(float* s_inout, const void* q, const void* k, const void* v,
                        const float* beta, const float* g, float* o, int B, int H, int D,
                        int in_dtype, void* stream);

/*
 * The delta rule with a decay per key channel (KDA, Kimi Delta Attention; the
 * reference's model names the "Gated DeltaNet / KDA family",
 * spec/03-model.md:12 and kernels/__init__.py:6, and has code for neither
 * gate).  No reference counterpart:
 *   S_t = (I - beta_t k_t k_t^T) Diag(alpha_t) S_{t-1} + beta_t k_t v_t^T,  o_t = q_t S_t,
 * alpha_t = exp(g_t) with g (B, T, H, D) fp32 (one log-gate per key channel,
 * i.e. per row of S), NULL only when B*T*H == 0.  With g constant along D
 * this is pm_gated_delta_fwd.
 *   * bf16 q/k/v with D in {64, 128}, 16-byte aligned q/k/v/o, and a workspace of
 *     pm_kda_delta_workspace_bytes (16-byte aligned): the chunked WY form on bf16
 *     MFMA (a parallel pass writes every chunk's decayed operands, T and P into the
 *     workspace, then the chunk recurrence).  It clamps each log-gate into [-10, 1]
 *     (alpha >= 4.5e-5: a difference below bf16 resolution).
 *   * otherwise, without a large enough workspace, and under path 1: the fp32
 *     per-token kernel, every in_dtype and D <= 256, g as given.
 * Path 2 or 3 (chunked kernel required) returns PM_E_UNSUPPORTED for inputs the
 * chunked form does not take and PM_E_WORKSPACE without the workspace.
 * Everything else as pm_delta_fwd.
 */
int pm_kda_delta_fwd(const void* q, const void* k, const void* v, const float* beta,
                     const float* g, const float* s0, void* o, float* s_out, int B, int T, int H,
                     int D, int in_dtype, int out_dtype, void* workspace, size_t ws_bytes,
                     void* stream);

/* Workspace bytes of pm_kda_delta_fwd's chunked form (0 where the call runs the
 * per-token kernel): 61 KiB (D = 128) or 37 KiB (D = 64) per 64-token chunk of every
 * (b, h). */
size_t pm_kda_delta_workspace_bytes(int B, int T, int H, int D, int in_dtype);

/*
 * One KDA step: S' = (I - beta k k^T) Diag(exp(g)) S + beta k v^T, o = q S',
 * g (B, H, D) fp32; otherwise as pm_delta_step.
 */
int pm_kda_delta_step(float* s_inout, const void* q, const void* k, const void* v,
                      const float* beta, const float* g, float* o, int B, int H, int D,
                      int in_dtype, void* stream);

/*
 * Decode step over a serving-side state cache (no reference counterpart in
 * code: the consumer the reference's serving spec names, spec/13-serving.md
 * item 4 and sglang-fork/sglang_fork/model_def.py, whose linear layers keep
 * a fixed-size state per request).  The step of pm_delta_step
 * (kernels/__init__.py:357-376) for B requests, request b updating the
 * state pool[slots[b]] in place:
 *   pool  (n_slots, H, D, D) fp32, 16-byte aligned;  slots (B,) int32;
 *   q, k, v (B, H, D) fp32 or bf16 (in_dtype);  beta (B, H) fp32;
 *   o (B, H, D) fp32, 16-byte aligned.
 * A slot outside [0, n_slots) is skipped: the pool is not touched and the
 * request's output row is zero (padding in fixed-size, graph-captured
 * batches).  Two requests naming the same slot race.  D in {32, 64, 128}.
 */
int pm_delta_step_slots(float* pool, const int32_t* slots, int n_slots, const void* q,
                        const void* k, const void* v, const float* beta, float* o, int B, int H,
                        int D, int in_dtype, void* stream);

/*
 * The model's linear attention (Gated DeltaNet / KDA family, beta = 1).
 * Replaces the recurrence of model.linear_attention (model/__init__.py:
 * 393-432, called by model._linear_attn :726-734): per (b, h) and token,
 *   q^ = q / max(||q||, 1e-6),  k^ = k / max(||k||, 1e-6)   (:203-205)
 *   S_t = (I - k^ k^^T) S_{t-1} + k^ v^T,   o_t = q^ S_t
 * with the normalisation done inside the kernel (no normalised copies in
 * memory).  Shapes, dtypes and state handling as pm_delta_fwd without beta.
 * Kernels as pm_delta_fwd chooses them (pm_delta_set_path): bf16 q/k/v with
 * D in {64, 128} run the chunked MFMA kernel, which folds the norms into its
 * Gram tiles and row scalings (bf16 parity); everything else runs the fp32
 * per-token kernel, which normalises the rows as it stages them (fp32 parity).
 */
int pm_linear_attention(const void* q, const void* k, const void* v, const float* s0, void* o,
                        float* s_out, int B, int T, int H, int D, int in_dtype, int out_dtype,
                        void* stream);

/*
 * pm_linear_attention with a workspace: fp32 q/k/v at D in {64, 128}
 * (16-byte aligned) run the fp32 chunked forward on fp32 MFMA in its
 * normalised mode when workspace holds pm_linear_attention_workspace_bytes
 * bytes (16-byte aligned); without it, the per-token kernel.  Everything
 * else as pm_linear_attention (same replaced interface, model/__init__.py:
 * 393-432; the workspace has no reference counterpart).
 */
int pm_linear_attention_ws(const void* q, const void* k, const void* v, const float* s0, void* o,
                           float* s_out, int B, int T, int H, int D, int in_dtype, int out_dtype,
                           void* workspace, size_t ws_bytes, void* stream);
/* Workspace bytes pm_linear_attention_ws uses (1088 bytes per (b, h) and
 * 16-token chunk for fp32 inputs at D in {64, 128}; otherwise 0). */
size_t pm_linear_attention_workspace_bytes(int B, int T, int H, int D, int in_dtype);

/*
 * Workspace bytes pm_delta_fwd uses: the split form of the bf16 chunked
 * kernel (6 KiB per (b, h) and 64-token chunk) or the fp32 chunked forward
 * (1 KiB per (b, h) and 16-token chunk); 0 when the call, under the calling
 * thread's pm_delta_set_path / pm_delta_set_tile setting, would use neither.
 * No reference counterpart: the reference's scan keeps no per-chunk state
 * (kernels/__init__.py:421-458).
 */
size_t pm_delta_workspace_bytes(int B, int T, int H, int D, int in_dtype);
/* The same for pm_delta_fwd_varlen (per head: 6 KiB per slot, with
 * ceil(total_T / 64) + n_seqs slots; fp32: 1 KiB per slot, with
 * ceil(total_T / 16) + n_seqs slots; the single-stage bf16 kernel: 4 bytes
 * per sequence for 65 to 8192 sequences, the sequence order). */
size_t pm_delta_varlen_workspace_bytes(int n_seqs, int total_T, int H, int D, int in_dtype);

/*
 * Reverse mode of the forward: gradients of L with respect to (q, k, v,
 * beta, s0) given go = dL/dO and gs = dL/dS_T.
 * Replaces kernels/__init__.py:692-719 (chunked_delta_rule_bwd, which runs
 * _delta_vjp_np :460-527 / _delta_vjp_jax :529-588): same inputs as the
 * residual (q, k, v, beta, s0), same grads (go, gs), same five fp32 outputs
 * in the order (gq, gk, gv, gbeta, gs0).
 *   go (B, T, H, D) fp32 or NULL (zeros); gs (B, H, D, D) fp32 or NULL (zeros);
 *   s0 NULL means a zero initial state;
 *   gq, gk, gv (B, T, H, D), gbeta (B, T, H), gs0 (B, H, D, D): fp32 outputs.
 * q, k, v are fp32 or bf16 (in_dtype); 1 <= D <= 256.
 * Three kernels, chosen as the forward's are (pm_delta_set_path):
 *   - bf16 q/k/v with D in {64, 128}: the chunked backward on bf16 MFMA
 *     (the forward's chunked kernel in reverse; bf16 parity, rel-L2 <= 2e-2
 *     against the fp32 reference).  q, k, v, go, gq, gk, gv and
 *     workspace 16-byte aligned.  Workspace, per (b, h) and 64-token chunk: the chunk's start
 *     state and end state gradient and W (bf16), and the packed 64x64 T:
 *     2 * B * H * ceil(T / 64) * (2 * D * D + 64 * D + 3072) bytes.
 *   - fp32 q/k/v with D in {64, 128}: the chunked backward on fp32 MFMA
 *     (16-token chunks; fp32 parity).  q, k, v, go, gq, gk, gv and workspace
 *     16-byte aligned.  Workspace (fp32, each region rounded up to 256
 *     bytes), per (b, h): 256 + 784 values per 16-token chunk (the chunk's
 *     T and P factors), D * D values per 256-token span and one more (the
 *     state at every span start and at the end), D * D per span (the state
 *     gradient at every span end) and 2 * T * D (W and U); 475 MB at B4
 *     T4096 H16 D128.
 *   - otherwise the per-token fp32 backward (fp32 parity).  Workspace:
 *     per-token u = v - S^T k and the state every 8 tokens, 4 * B * H *
 *     (T * D + ceil(T / 8) * D * D) bytes, and for D > 32 the partial sums
 *     of gq, gk and gbeta over column tiles of the state (32 columns for
 *     D <= 128, 16 above), 4 * B * H * T * n_tiles * (2 * D + 1) bytes more.
 * workspace: device memory of at least pm_delta_bwd_workspace_bytes(B, T,
 * H, D, in_dtype) bytes (queried under the same path setting), 4-byte
 * aligned, contents undefined on entry and exit.
 * T == 0 gives gs0 = gs (or zeros).
 */
int pm_delta_bwd(const void* q, const void* k, const void* v, const float* beta,
                 const float* s0, const float* go, const float* gs, float* gq, float* gk,
                 float* gv, float* gbeta, float* gs0, int B, int T, int H, int D, int in_dtype,
                 void* workspace, size_t ws_bytes, void* stream);

/* Workspace bytes pm_delta_bwd needs for these shapes and in_dtype under the
 * current path setting (0 for invalid shapes, dtypes or D > 256). */
size_t pm_delta_bwd_workspace_bytes(int B, int T, int H, int D, int in_dtype);

/*
 * Reverse mode of pm_gated_delta_fwd (the gated delta rule, alpha = exp(g)
 * per token and head).  No reference counterpart: the reference's model
 * names the variant (spec/03-model.md:12) and has no code for it
 * (PROGRESS.md:109); every primitive on its path has a VJP
 * (kernels/__init__.py:591-658), and this is that VJP for the gated forward.
 * Arguments as pm_delta_bwd, plus g (B, T, H) fp32, the forward's log-gates,
 * and gg (B, T, H) fp32, dL/dg.  With P_t = alpha_t S_{t-1}, per token in
 * reverse: y = P_t w, dL/dg_t = <G - beta_t k_t w^T, P_t>, G <- alpha_t (G -
 * beta_t k_t w^T), the other gradients as pm_delta_bwd's.  Runs the
 * per-token fp32 kernels (any D <= 256, fp32 or bf16 q/k/v); each 8-token
 * checkpoint block is recomputed forward from its start state, never walked
 * back (which would divide by alpha).  Path 2 (chunked backward required)
 * returns PM_E_UNSUPPORTED.  workspace: pm_gated_delta_bwd_workspace_bytes.
 */
int pm_gated_delta_bwd(const void* q, const void* k, const void* v, const float* beta,
                       const float* g, const float* s0, const float* go, const float* gs, float* gq,
                       float* gk, float* gv, float* gbeta, float* gg, float* gs0, int B, int T,
                       int H, int D, int in_dtype, void* workspace, size_t ws_bytes, void* stream);

/* Workspace bytes pm_gated_delta_bwd needs (0 for invalid shapes, dtypes or D > 256):
 * pm_delta_bwd's per-token workspace plus, for D > 32, the partial sums of gg. */
size_t pm_gated_delta_bwd_workspace_bytes(int B, int T, int H, int D, int in_dtype);

/*
 * Reverse mode of pm_kda_delta_fwd (a log-gate per key channel).  No reference
 * counterpart (the reference names the KDA family, spec/03-model.md:12, and has no
 * code for it).  Arguments as pm_gated_delta_bwd, with g and gg (B, T, H, D) fp32.
 * With P_t = Diag(alpha_t) S_{t-1}, per token in reverse: y = P_t w,
 * dL/dg_t[d] = <G_P[d, :], P_t[d, :]> with G_P = G - beta_t k_t w^T, and
 * G <- Diag(alpha_t) G_P; the other gradients as pm_delta_bwd's.  The per-token fp32
 * kernels (any D <= 256, fp32 or bf16 q/k/v), each 8-token checkpoint block
 * recomputed forward from its start state.  Path 2 returns PM_E_UNSUPPORTED.
 * workspace: pm_kda_delta_bwd_workspace_bytes.
 */
int pm_kda_delta_bwd(const void* q, const void* k, const void* v, const float* beta,
                     const float* g, const float* s0, const float* go, const float* gs, float* gq,
                     float* gk, float* gv, float* gbeta, float* gg, float* gs0, int B, int T,
                     int H, int D, int in_dtype, void* workspace, size_t ws_bytes, void* stream);

/* Workspace bytes pm_kda_delta_bwd needs (0 for invalid shapes, dtypes or D > 256):
 * pm_delta_bwd's per-token workspace plus, for D > 32, the partial sums of gg per
 * column tile. */
size_t pm_kda_delta_bwd_workspace_bytes(int B, int T, int H, int D, int in_dtype);

/*
 * pm_delta_bwd without a caller workspace and without any allocation.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving or training loops,
 * harnesses that forbid hipMalloc).  The kernels and results are those of
 * pm_delta_bwd; the workspace is a fixed scratch array inside the library,
 * one per GPU, held until the process ends: PM_DELTA_NOALLOC_SCRATCH_BYTES.
 * A call whose pm_delta_bwd_workspace_bytes exceeds it returns
 * PM_E_WORKSPACE before launching anything.  Every call on one GPU uses that
 * GPU's scratch: calls that overlap on one GPU (other streams, other threads)
 * race and must be ordered by the caller.  Arguments as pm_delta_bwd.
 */
#define PM_DELTA_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int pm_delta_bwd_noalloc(const void* q, const void* k, const void* v, const float* beta,
                         const float* s0, const float* go, const float* gs, float* gq, float* gk,
                         float* gv, float* gbeta, float* gs0, int B, int T, int H, int D,
                         int in_dtype, void* stream);

/* Thread-local message for the last nonzero return on this thread. */
const char* pm_last_error(void);

/* PM_DELTA_ABI_VERSION of the loaded library. */
int pm_abi_version(void);

/*
 * Kernel selection for pm_delta_fwd, pm_delta_fwd_varlen, pm_delta_bwd and
 * pm_linear_attention, for tests and benchmarks: 0 = automatic (chunked MFMA
 * kernel where the shape and dtype allow, else the per-token kernel; the
 * plain forward in split form where that is faster and a workspace is
 * given; fp32 inputs on the fp32 chunked forward where a workspace is
 * given), 1 = always the per-token kernel, 2 = chunked kernel required
 * (PM_E_UNSUPPORTED when it cannot serve the call; for fp32 inputs the fp32
 * chunked forward, PM_E_WORKSPACE without its workspace), single-stage form,
 * 3 = as 2, with the plain bf16 forward always in split form (PM_E_WORKSPACE
 * without a workspace of pm_delta_workspace_bytes bytes).  The previous value is
 * returned.  The setting is per calling thread: a
 * workspace-size query and the call it sizes, made on one thread, always see
 * the same setting.
 */
int pm_delta_set_path(int path);

/*
 * Column-tile width (d_v columns per workgroup) the chunked kernel uses:
 * 0 = automatic (32 when B*H*(D/32) >= 256, else 16), else 16, 32 or 64;
 * 64 is accepted and served with 32-column workgroups.  Returns the previous
 * value.  Per calling thread, as pm_delta_set_path.
 */
int pm_delta_set_tile(int dv_tile);

#ifdef __cplusplus
}
#endif

#endif /* PM_DELTA_H */
