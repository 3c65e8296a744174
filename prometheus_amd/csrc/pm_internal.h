// pm_internal.h — launcher interfaces between the C ABI layer and kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace pm {

// Per-token kernel (K4). Fixed-length mode: n_pairs = B*H sequences of T
// tokens. Varlen mode (cu_seqlens != nullptr): n_pairs = n_seqs*H and T is
// the packed token count (segment offsets are clamped into [0, T]).
struct RecurrentArgs {
    const void* q;
    const void* k;
    const void* v;
    const float* beta;  // nullable: beta = 1
    const float* s0;    // nullable; may alias s_out
    void* o;
    float* s_out;
    const int32_t* cu_seqlens;  // nullable
    int n_pairs;
    int T, H, D;
    bool in_bf16, out_bf16;
    bool l2norm = false;  // q and k divided by max(||.||_2, 1e-6) per token on load
    const float* g = nullptr;  // gated variant: log-gates per (token, head), alpha = exp(g)
    // per-channel variant (KDA; takes precedence over g): log-gates per (token, head, key
    // channel), S <- Diag(exp(g)) S before each token; 16-byte aligned for vector loads
    const float* gk = nullptr;
};
hipError_t launch_recurrent(const RecurrentArgs& a, hipStream_t st);

// Decode step (K3) for D in {32, 64, 128}: s updated in place.
struct StepArgs {
    float* s;
    const void* q;
    const void* k;
    const void* v;
    const float* beta;
    float* o;
    int n_pairs, D;
    bool in_bf16;
    // State-cache mode (nullable): request b = pair / H updates the state of slot
    // slots[b] in a pool of n_slots x H states; a slot outside [0, n_slots)
    // leaves the pool untouched and gets a zero output row.
    const int32_t* slots = nullptr;
    int H = 1, n_slots = 0;
    const float* g = nullptr;  // gated variant: log-gate per (b, h), alpha = exp(g)
    const float* gk = nullptr; // per-channel variant (KDA): log-gates per (b, h, key channel)
};
bool step_supported(int D);
hipError_t launch_step(const StepArgs& a, hipStream_t st);

// Chunked WY/UT forward (K1 / K2 when cu_seqlens != nullptr), bf16 inputs.
struct ChunkedArgs {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const float* beta;
    const float* s0;  // nullable
    void* o;
    float* s_out;
    const int32_t* cu_seqlens;  // nullable
    int n_seq;                  // B, or n_seqs in varlen mode
    int T, H, D;                // varlen: T = packed token count
    bool out_bf16;
    int dv_tile;  // 0 = automatic
    // The model's linear attention: beta = 1 (beta unused) and q, k divided by
    // max(||.||, 1e-6) per token inside the kernel.
    bool norm = false;
    // Gated variant (not with norm): log-gates per (token, head), alpha = exp(g)
    // (g <= 0 keeps every in-chunk decay factor at most 1).
    const float* g = nullptr;
    // Packed batches (cu_seqlens): a permutation of the n_seq sequences, longest first
    // (launch_varlen_order), in which the workgroups take them; nullptr: the kernel ranks
    // up to 64 sequences itself and keeps cu_seqlens order beyond.  Only the schedule
    // changes: every sequence's results are the same bits either way.
    const int32_t* seq_order = nullptr;
};
bool chunked_supported(int D, int H);  // D in {64, 128}, H*D <= 2^24
// d_v columns per workgroup of the chunked forward: 32 (two chain waves) unless that
// leaves CUs idle; `requested` 16 or 32 forces it (64 is served as 32).
int chunked_pick_tile(int D, long n_pairs, int requested);
hipError_t launch_chunked(const ChunkedArgs& a, hipStream_t st);
// The plain forward (no norm, no gates) in split form (delta_chunked_split.hip): a
// parallel pass builds every chunk's T diag(beta) into `t_ws` (chunked_split_ws_bytes
// bytes, 16-byte aligned), then the chunk recurrence loads it instead of building it.
// Same algebra as the single-stage kernel, rounded differently (bf16 parity).
size_t chunked_split_ws_bytes(bool varlen, int n_seq, int T, int H);

// The per-channel gated (KDA) forward in chunked form (kda_chunked.hip): bf16 q/k/v, D in
// {64, 128}, fixed length; g (B, T, H, D) fp32 log-gates, clamped into [-10, 1].  A
// parallel pass writes every chunk's decayed operands, T'' and P into `workspace`
// (kda_chunked_ws_bytes, 16-byte aligned), then the chunk recurrence copies them in.
struct KdaChunkedArgs {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const float* beta;
    const float* g;
    const float* s0;  // nullable
    void* o;
    float* s_out;
    int B, T, H, D;
    bool out_bf16;
    void* workspace;
};
size_t kda_chunked_ws_bytes(int B, int T, int H, int D);
hipError_t launch_kda_chunked(const KdaChunkedArgs& a, hipStream_t st);
hipError_t launch_chunked_split(const ChunkedArgs& a, int dv, void* t_ws, hipStream_t st);
// Chunked forward for fp32 q/k/v on fp32 MFMA (delta_chunked_f32.hip), D in {64, 128},
// plain (no norm, no gates): a parallel pass writes every 16-token chunk's (T'')^T and
// P^T into `ws` (chunked_f32_ws_bytes bytes, 16-byte aligned), then the recurrence runs
// on them.  fp32 arithmetic throughout.
struct ChunkedF32Args {
    const float* q;
    const float* k;
    const float* v;
    const float* beta;
    const float* s0;  // nullable
    void* o;
    float* s_out;
    const int32_t* cu_seqlens;  // nullable
    int n_seq;                  // B, or n_seqs in varlen mode
    int T, H, D;                // varlen: T = packed token count
    bool out_bf16;
    int dv_tile;  // 0 = automatic
    // The model's linear attention: beta = 1 (beta unused), q and k divided by
    // max(||.||, 1e-6) per token inside the kernels.
    bool norm = false;
};
size_t chunked_f32_ws_bytes(bool varlen, int n_seq, int T, int H, bool norm = false);
int chunked_f32_pick_tile(int D, long n_pairs, int requested);
hipError_t launch_chunked_f32(const ChunkedF32Args& a, void* ws, hipStream_t st);
// The same kernel writing, instead of O and the final state, the state at
// the start of every chunk as bf16 rows of S^T (fixed-length batches only):
// s_hist holds n_seq*H x ceil(T/64) x D x D values.
hipError_t launch_chunked_states(const ChunkedArgs& a, uint16_t* s_hist, hipStream_t st);

// The fp32 chunked backward (K9; fixed-length batches, fp32 q/k/v, D in {64, 128}).
// Chunks of kC16 = 16 tokens; the state S and its gradient G are kept at the start and
// the end of every span of kF32Span chunks (256 tokens).  Workspace regions (bytes, each
// 256-byte aligned), per (b, h):
//   t2     (T'')^T per chunk, 256 floats (the fp32 forward's own workspace layout)
//   rec    T, K K^T, beta and P = lower_incl(Q K^T) per chunk, kF32BwdRec floats
//   s_hist S at every span start and at the end, g_hist G at every span end: D x D floats
//          each, as accumulator registers (column block of 16, tile of 16 rows, lane,
//          register)
//   w, u   W = dL/dX and U per token, (B, T, H, D) floats each
constexpr int kF32Span = 16;
constexpr int kF32BwdRec = 784;
struct F32BwdWs {
    size_t t2, rec, s_hist, g_hist, w, u, bytes;
};
F32BwdWs f32_bwd_ws(long n_pairs, int T, int D);
bool f32_bwd_supported(int D, int H);
// K9p: the backward's records ((T'')^T, and T, K K^T, beta, P; fixed-length batches).
hipError_t launch_f32_bwd_prep(const float* q, const float* k, const float* beta, int n_pairs, int T, int H, int D,
                               float* ws_t2, float* ws_rec, hipStream_t st);

// Reverse mode (K5, fp32): fixed-length batch of n_pairs = B*H sequences of
// T tokens, D <= 256.  workspace holds bwd_workspace_floats(n_pairs, T, D)
// floats: u (n_pairs x T x D), the checkpoints (n_pairs x ceil(T/8) x D x D),
// then for D > 32 the per-column-tile partial sums of gq, gk (n_tiles x
// n_pairs x T x D each) and gbeta (n_tiles x n_pairs x T), n_tiles = ceil(D/32)
// for D <= 128 and ceil(D/16) above.
struct BwdArgs {
    const void* q;
    const void* k;
    const void* v;
    const float* beta;
    const float* s0;  // nullable
    const float* go;  // nullable (zeros)
    const float* gs;  // nullable (zeros)
    float* gq;
    float* gk;
    float* gv;
    float* gbeta;
    float* gs0;
    float* workspace;
    int n_pairs, T, H, D;
    bool in_bf16;
    // gated variant (per-token fp32 kernels only): log-gates per (token, head), alpha =
    // exp(g), and their gradient gg (B, T, H)
    const float* g = nullptr;
    float* gg = nullptr;
    // with g: one log-gate per (token, head, key channel) (KDA), g and gg (B, T, H, D)
    bool per_channel = false;
};
constexpr int kBwdMaxD = 256;
// gm: 0 ungated, 1 gated, 2 per-channel gated
size_t bwd_workspace_floats(long n_pairs, int T, int D, int gm = 0);
hipError_t launch_bwd(const BwdArgs& a, hipStream_t st);

// Chunked reverse mode (K6, bf16 MFMA): bf16 q/k/v and chunked_supported(D,
// H).  a.workspace is a byte buffer of chunked_bwd_ws(...).bytes bytes (16-byte
// aligned) holding, per chunk of every (b, h), the start state and the end
// gradient of the state (bf16 rows of S^T and G^T), W (bf16 rows of W^T) and
// the packed T.
struct ChunkedBwdWs {
    size_t s_hist, g_hist, w_hist, tp, bytes;
};
ChunkedBwdWs chunked_bwd_ws(long n_pairs, int T, int D);
bool chunked_bwd_supported(int D, int H);  // chunked_supported and H*D <= 2^23 (fp32 dO rows)
hipError_t launch_bwd_chunked(const BwdArgs& a, hipStream_t st);
// K9 (the fp32 chunked backward): a.workspace holds f32_bwd_ws(...).bytes bytes.
// K9a + K9b in one launch: the state history (s_hist, U into u_out) and the gradient sweep
// (gv, gs0, W into w_out, g_hist), from K9p's records.
hipError_t launch_f32_hist_sweep(const BwdArgs& a, const float* t2, const float* rec, float* w_out, float* s_hist,
                                 float* g_hist, float* u_out, hipStream_t st);
hipError_t launch_bwd_chunked_f32(const BwdArgs& a, hipStream_t st);

// Zero fill (used instead of hipMemsetAsync so callers may graph-capture).
hipError_t launch_fill_zero(float* p, size_t n, hipStream_t st);
hipError_t launch_copy_f32(float* dst, const float* src, size_t n, hipStream_t st);
// One workgroup checks a packed batch's offsets and ORs error bits into *flag.
hipError_t launch_varlen_check(const int32_t* cu, int n_seqs, int total, int32_t* flag, hipStream_t st);
// order[r] = the sequence of rank r by chunk count, largest first, ties in index order
// (cu_seqlens clamped as the chunked kernels clamp them); at most kVarlenOrderMax sequences
constexpr int kVarlenOrderMax = 8192;
hipError_t launch_varlen_order(const int32_t* cu, int n_seqs, int total, int32_t* order, hipStream_t st);

}  // namespace pm
