// pm_delta_abi.hip — the extern "C" boundary of libpmdelta.so.
//
// Validates every argument before anything is launched (negative PM_E_*
// codes, thread-local message), then dispatches to the gfx950 kernels:
//   K1/K2 delta_chunked.hip    chunked WY/UT forward on bf16 MFMA
//   K3    delta_step.hip       decode step, HBM-streaming
//   K4    delta_recurrent.hip  per-token fp32 recurrence (generic shapes)
//   K5    delta_bwd.hip        reverse mode, fp32, checkpointed
//   K6    delta_chunked_bwd.hip     chunked reverse mode, bf16 inputs
//   K7    delta_chunked_f32.hip     chunked forward on fp32 MFMA, fp32 inputs
//   K8    kda_chunked.hip           chunked forward with a decay per key channel
//   K9    delta_chunked_f32_bwd.hip chunked reverse mode on fp32 MFMA, fp32 inputs
// Mirrors the checks of kernels/__init__.py:308-338 (shapes), :613-614 and
// :676-677 (chunk >= 1); shapes arrive as integers, so the Python layer
// (prometheus_amd/kernels) raises KernelError for the tensor-level checks
// before it calls in.

#include <stdarg.h>
#include <stdio.h>

#include <atomic>
#include <mutex>

#include "pm_common.h"
#include "pm_internal.h"
#include "../../include/pm_delta.h"

namespace pm {

__global__ void fill_zero_kernel(float* __restrict__ p, size_t n) {
    size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (; i < n; i += stride) p[i] = 0.f;
}

__global__ void copy_f32_kernel(float* __restrict__ d, const float* __restrict__ s, size_t n) {
    size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (; i < n; i += stride) d[i] = s[i];
}

static unsigned grid_for(size_t n) {
    size_t g = (n + 255) / 256;
    if (g > 65536) g = 65536;
    return static_cast<unsigned>(g < 1 ? 1 : g);
}

hipError_t launch_fill_zero(float* p, size_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(fill_zero_kernel, dim3(grid_for(n)), dim3(256), 0, st, p, n);
    return hipGetLastError();
}

// Offsets of a packed batch checked on the device: one workgroup ORs what it finds into
// *flag (bit 1: cu[0] != 0; 2: cu[n] != total; 4: a decreasing pair; 8: an offset outside
// [0, total]).  The workgroup combines its lanes' bits in LDS and one lane updates the
// flag, so the word is read and written by a single thread of a single launch.
__global__ __launch_bounds__(256) void varlen_check_kernel(const int32_t* __restrict__ cu, int n_seqs,
                                                           int total, int32_t* __restrict__ flag) {
    __shared__ int found;
    if (threadIdx.x == 0) found = 0;
    __syncthreads();
    int bits = 0;
    for (int i = threadIdx.x; i <= n_seqs; i += blockDim.x) {
        const int a = cu[i];
        if (a < 0 || a > total) bits |= 8;
        if (i == 0 && a != 0) bits |= 1;
        if (i == n_seqs && a != total) bits |= 2;
        if (i < n_seqs && cu[i + 1] < a) bits |= 4;
    }
    if (bits) atomicOr(&found, bits);
    __syncthreads();
    if (threadIdx.x == 0 && found) flag[0] |= found;
}

hipError_t launch_varlen_check(const int32_t* cu, int n_seqs, int total, int32_t* flag, hipStream_t st) {
    hipLaunchKernelGGL(varlen_check_kernel, dim3(1), dim3(256), 0, st, cu, n_seqs, total, flag);
    return hipGetLastError();
}

// The order in which the chunked forward takes the sequences of a packed batch: its
// workgroups are dispatched in block order, one per CU, and a long sequence whose blocks
// come late starts only when earlier, shorter ones have finished.  Ranked by chunk count
// (the recurrence walks chunks in order), largest first, ties in index order, so the
// ranks are a permutation and every order slot is written once.  One thread per
// sequence, the counts compared through LDS in tiles of 1024.
__global__ __launch_bounds__(256) void varlen_order_kernel(const int32_t* __restrict__ cu, int n_seqs,
                                                           int total, int32_t* __restrict__ order) {
    constexpr int kTile = 1024;
    __shared__ int nc[kTile];
    auto chunks = [&](int j) {  // clamped as the chunked kernels clamp the offsets
        const int a = min(max(cu[j], 0), total);
        const int z = min(max(cu[j + 1], a), total);
        return (z - a + 63) / 64;  // 64-token chunks
    };
    const int i = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
    const int mine = i < n_seqs ? chunks(i) : 0;
    int rank = 0;
    for (int j0 = 0; j0 < n_seqs; j0 += kTile) {
        const int m = min(kTile, n_seqs - j0);
        __syncthreads();
        for (int t = static_cast<int>(threadIdx.x); t < m; t += 256) nc[t] = chunks(j0 + t);
        __syncthreads();
        if (i < n_seqs) {
            for (int t = 0; t < m; ++t) rank += nc[t] > mine || (nc[t] == mine && j0 + t < i);
        }
    }
    if (i < n_seqs) order[rank] = i;
}

hipError_t launch_varlen_order(const int32_t* cu, int n_seqs, int total, int32_t* order, hipStream_t st) {
    if (n_seqs <= 0 || n_seqs > kVarlenOrderMax) return hipErrorInvalidValue;
    hipLaunchKernelGGL(varlen_order_kernel, dim3(static_cast<unsigned>((n_seqs + 255) / 256)), dim3(256), 0, st,
                       cu, n_seqs, total, order);
    return hipGetLastError();
}

hipError_t launch_copy_f32(float* dst, const float* src, size_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(copy_f32_kernel, dim3(grid_for(n)), dim3(256), 0, st, dst, src, n);
    return hipGetLastError();
}

}  // namespace pm

namespace {

thread_local char g_err[512] = "";
// Kernel-selection knobs (pm_delta_set_path / pm_delta_set_tile): per calling
// thread, so that a workspace-size query and the call it sizes always see the
// same setting, whatever other threads select meanwhile.
thread_local int g_path = 0;
thread_local int g_tile = 0;

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

// Scratch of pm_delta_bwd_noalloc: a file-scope device array, one copy per GPU,
// held until the process ends.  Host code never uses `scratch` itself (its
// host-side name is not a device address): the device address comes from
// hipGetSymbolAddress, once per device with that device current.
constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;
__device__ __attribute__((aligned(256))) unsigned char scratch[kNoAllocScratchBytes];
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

int hip_fail(hipError_t e, const char* what);

// Device address of this GPU's scratch (looked up on the first call on the device).
int scratch_address(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return fail(PM_E_UNSUPPORTED, "device %d beyond %d", dev, kMaxDevices);
    void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
        if (!p) {
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
            if (!p) return fail(PM_E_NULL, "hipGetSymbolAddress(scratch) gave NULL");
            g_scratch_ptr[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return 0;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(static_cast<int>(e), "%s: HIP error %d (%s)", what, static_cast<int>(e),
                hipGetErrorString(e));
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// The split form of the chunked forward runs under path 3, and by default (path 0) where
// even 16-column tiles leave CUs idle: fewer than 256 workgroups of the single-stage
// kernel (n_pairs * D / 16 < 256).  There its fully parallel T pass and lighter recurrence
// win (measured 9-32 % faster); from 256 workgroups on, the single-stage kernel is faster
// or level (cfg3, 256 workgroups: 656 against 706 us).
bool split_chosen(int path, int D, long n_pairs) {
    return path == 3 || (path == 0 && pm::chunked_pick_tile(D, n_pairs, g_tile) == 16 &&
                         n_pairs * (D / 16) < 256);
}

int check_dtypes(int in_dtype, int out_dtype) {
    if (in_dtype != PM_DTYPE_F32 && in_dtype != PM_DTYPE_BF16)
        return fail(PM_E_DTYPE, "in_dtype %d is not PM_DTYPE_F32 or PM_DTYPE_BF16", in_dtype);
    if (out_dtype != PM_DTYPE_F32 && out_dtype != PM_DTYPE_BF16)
        return fail(PM_E_DTYPE, "out_dtype %d is not PM_DTYPE_F32 or PM_DTYPE_BF16", out_dtype);
    return 0;
}

// Common forward dispatch. cu == nullptr: fixed length (n_seq = B, T).
int forward(const void* q, const void* k, const void* v, const float* beta, const float* s0,
            void* o, float* s_out, const int32_t* cu, int n_seq, int T, int total_T, int H,
            int D, int in_dtype, int out_dtype, int chunk, hipStream_t st,
            const float* g = nullptr, void* workspace = nullptr, size_t ws_bytes = 0,
            const float* gk = nullptr) {
    const bool varlen = cu != nullptr;
    const long n_pairs = static_cast<long>(n_seq) * H;
    const long n_tok = varlen ? static_cast<long>(total_T) : static_cast<long>(n_seq) * T;
    if (n_pairs == 0) return 0;
    if (!s_out) return fail(PM_E_NULL, "s_out is NULL");
    if (n_tok > 0 && (!q || !k || !v || !beta || !o))
        return fail(PM_E_NULL, "q, k, v, beta and o must be non-NULL");
    if (!aligned(s_out, 4) || (s0 && !aligned(s0, 4)) || (beta && !aligned(beta, 4)))
        return fail(PM_E_ALIGN, "fp32 buffers must be 4-byte aligned");
    if (n_pairs > (1L << 30) || n_tok > (1L << 40))
        return fail(PM_E_SHAPE, "problem too large");

    const size_t s_elems = static_cast<size_t>(n_pairs) * D * D;
    if (n_tok == 0) {
        // no tokens: every state passes through unchanged (reference :456-457)
        hipError_t e = s0 ? pm::launch_copy_f32(s_out, s0, s_elems, st)
                          : pm::launch_fill_zero(s_out, s_elems, st);
        return e == hipSuccess ? 0 : hip_fail(e, "state copy");
    }

    const int path = g_path;
    const bool in_bf16 = in_dtype == PM_DTYPE_BF16;
    const bool want_chunked = path != 1;
    // per-channel gates (gk): the per-token kernel only
    if (gk && path >= 2)
        return fail(PM_E_UNSUPPORTED, "the per-channel gated forward runs on the per-token kernel only "
                    "(path %d asks for the chunked one)", path);
    const bool can_chunked = !gk && in_bf16 && pm::chunked_supported(D, H) && aligned(q, 16) &&
                             aligned(k, 16) && aligned(v, 16) &&
                             (out_dtype == PM_DTYPE_F32 ? aligned(o, 16) : aligned(o, 8));
    // fp32 q/k/v: the chunked forward on fp32 MFMA (plain forward only)
    const bool can_f32 = !in_bf16 && !g && !gk && pm::chunked_supported(D, H) && aligned(q, 16) && aligned(k, 16) &&
                         aligned(v, 16) && (out_dtype == PM_DTYPE_F32 ? aligned(o, 4) : aligned(o, 2));
    if (path >= 2 && !can_chunked && !can_f32)
        return fail(PM_E_UNSUPPORTED,
                    "chunked kernel needs bf16 (or, for the plain forward, fp32) inputs, D in {64, 128} "
                    "and 16-byte aligned q/k/v (got in_dtype %d, D %d)",
                    in_dtype, D);
    if (want_chunked && can_f32) {
        const size_t need = pm::chunked_f32_ws_bytes(varlen, n_seq, varlen ? total_T : T, H);
        if (workspace && ws_bytes >= need && aligned(workspace, 16)) {
            pm::ChunkedF32Args a{static_cast<const float*>(q), static_cast<const float*>(k),
                                 static_cast<const float*>(v), beta, s0, o, s_out, cu, n_seq,
                                 varlen ? total_T : T, H, D, out_dtype == PM_DTYPE_BF16, g_tile};
            hipError_t e = pm::launch_chunked_f32(a, workspace, st);
            return e == hipSuccess ? 0 : hip_fail(e, "fp32 chunked forward launch");
        }
        if (path >= 2)
            return fail(PM_E_WORKSPACE, "the fp32 chunked forward needs a 16-byte aligned workspace of %zu bytes "
                        "(got %zu)", need, workspace ? ws_bytes : static_cast<size_t>(0));
    }
    if (want_chunked && can_chunked) {
        pm::ChunkedArgs a{static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                          static_cast<const uint16_t*>(v), beta, s0, o, s_out, cu, n_seq,
                          varlen ? total_T : T, H, D,
                          out_dtype == PM_DTYPE_BF16, g_tile};
        a.g = g;
        // the split form (T built by a parallel pass into the caller's workspace) for the
        // plain forward where it is the faster form (split_chosen), or always under path 3
        if (!g && split_chosen(path, D, n_pairs)) {
            const size_t need = pm::chunked_split_ws_bytes(varlen, n_seq, varlen ? total_T : T, H);
            if (workspace && ws_bytes >= need && aligned(workspace, 16)) {
                hipError_t e = pm::launch_chunked_split(a, pm::chunked_pick_tile(D, n_pairs, g_tile), workspace, st);
                return e == hipSuccess ? 0 : hip_fail(e, "chunked forward launch");
            }
            if (path == 3)
                return fail(PM_E_WORKSPACE, "path 3 needs a 16-byte aligned workspace of %zu bytes (got %zu)",
                            need, workspace ? ws_bytes : static_cast<size_t>(0));
        }
        // packed batches: the sequences go longest first, ranked inside the kernel up to 64
        // sequences and, beyond, through an order the rank kernel writes into the workspace
        if (varlen && !g && n_seq > 64 && n_seq <= pm::kVarlenOrderMax && workspace &&
            ws_bytes >= static_cast<size_t>(n_seq) * 4 && aligned(workspace, 4)) {
            int32_t* order = static_cast<int32_t*>(workspace);
            hipError_t e = pm::launch_varlen_order(cu, n_seq, total_T, order, st);
            if (e != hipSuccess) return hip_fail(e, "sequence order launch");
            a.seq_order = order;
        }
        hipError_t e = pm::launch_chunked(a, st);
        return e == hipSuccess ? 0 : hip_fail(e, "chunked forward launch");
    }
    (void)chunk;
    pm::RecurrentArgs a{q, k, v, beta, s0, o, s_out, cu, static_cast<int>(n_pairs),
                        varlen ? total_T : T, H, D,
                        in_bf16, out_dtype == PM_DTYPE_BF16};
    a.g = g;
    a.gk = gk;
    hipError_t e = pm::launch_recurrent(a, st);
    return e == hipSuccess ? 0 : hip_fail(e, "recurrent forward launch");
}

// The decode step, plain (g == gk == NULL), gated (g) or per-channel gated (gk).
int step(float* s_inout, const void* q, const void* k, const void* v, const float* beta,
         const float* g, float* o, int B, int H, int D, int in_dtype, void* stream,
         const float* gk = nullptr) {
    g_err[0] = '\0';
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (B < 0 || H < 0) return fail(PM_E_SHAPE, "B, H must be >= 0 (got %d, %d)", B, H);
    if (D < 1 || D > PM_DELTA_MAX_D)
        return fail(PM_E_SHAPE, "D must be in [1, %d] (got %d)", PM_DELTA_MAX_D, D);
    if (in_dtype != PM_DTYPE_F32 && in_dtype != PM_DTYPE_BF16)
        return fail(PM_E_DTYPE, "in_dtype %d is not PM_DTYPE_F32 or PM_DTYPE_BF16", in_dtype);
    const long n_pairs = static_cast<long>(B) * H;
    if (n_pairs == 0) return 0;
    if (n_pairs > (1L << 30)) return fail(PM_E_SHAPE, "problem too large");
    if (!s_inout || !q || !k || !v || !beta || !o)
        return fail(PM_E_NULL, "s_inout, q, k, v, beta and o must be non-NULL");
    if (pm::step_supported(D) && aligned(s_inout, 16) && aligned(o, 16)) {
        pm::StepArgs a{s_inout, q, k, v, beta, o, static_cast<int>(n_pairs), D,
                       in_dtype == PM_DTYPE_BF16};
        a.H = H;
        a.g = g;
        a.gk = gk;
        hipError_t e = pm::launch_step(a, st);
        return e == hipSuccess ? 0 : hip_fail(e, "decode step launch");
    }
    if (!aligned(s_inout, 4) || !aligned(o, 4))
        return fail(PM_E_ALIGN, "fp32 buffers must be 4-byte aligned");
    // a (B, H, D) token is a length-1 (B, 1, H, D) sequence; K4 runs it in place
    pm::RecurrentArgs a{q, k, v, beta, s_inout, o, s_inout, nullptr, static_cast<int>(n_pairs), 1,
                        H, D, in_dtype == PM_DTYPE_BF16, false};
    a.g = g;
    a.gk = gk;
    hipError_t e = pm::launch_recurrent(a, st);
    return e == hipSuccess ? 0 : hip_fail(e, "decode step launch");
}

// Which backward serves (B, T, H, D, in_dtype) under the current path setting:
// the chunked kernel for bf16 inputs with D in {64, 128}, else the per-token one.
bool bwd_chunked(int H, int D, int in_dtype) {
    return g_path != 1 && in_dtype == PM_DTYPE_BF16 && pm::chunked_bwd_supported(D, H);
}
// ... and the fp32 chunked backward (K9) for fp32 inputs with D in {64, 128}
bool bwd_chunked_f32(int H, int D, int in_dtype) {
    return g_path != 1 && in_dtype == PM_DTYPE_F32 && pm::f32_bwd_supported(D, H);
}

// gm: 0 ungated, 1 gated (a log-gate per token and head), 2 per-channel gated (KDA)
size_t bwd_ws_bytes(int B, int T, int H, int D, int in_dtype, int gm = 0) {
    const long n_pairs = static_cast<long>(B) * H;
    if (gm == 0 && bwd_chunked(H, D, in_dtype)) return pm::chunked_bwd_ws(n_pairs, T, D).bytes;
    if (gm == 0 && bwd_chunked_f32(H, D, in_dtype)) return pm::f32_bwd_ws(n_pairs, T, D).bytes;
    return sizeof(float) * pm::bwd_workspace_floats(n_pairs, T, D, gm);
}

// Common backward dispatch; g != NULL: a gated variant (per-token kernels, gg out), with
// per_channel its KDA form (g and gg (B, T, H, D)).
int backward(const void* q, const void* k, const void* v, const float* beta, const float* g,
             const float* s0, const float* go, const float* gs, float* gq, float* gk, float* gv,
             float* gbeta, float* gg, float* gs0, int B, int T, int H, int D, int in_dtype,
             void* workspace, size_t ws_bytes, void* stream, bool per_channel = false) {
    if (B < 0 || T < 0 || H < 0)
        return fail(PM_E_SHAPE, "B, T, H must be >= 0 (got %d, %d, %d)", B, T, H);
    if (D < 1 || D > pm::kBwdMaxD)
        return fail(PM_E_SHAPE, "backward D must be in [1, %d] (got %d)", pm::kBwdMaxD, D);
    if (in_dtype != PM_DTYPE_F32 && in_dtype != PM_DTYPE_BF16)
        return fail(PM_E_DTYPE, "in_dtype %d is not PM_DTYPE_F32 or PM_DTYPE_BF16", in_dtype);
    const long n_pairs = static_cast<long>(B) * H;
    const long n_tok = static_cast<long>(B) * T;
    if (n_pairs == 0) return 0;
    if (n_pairs > (1L << 30) || n_tok > (1L << 40)) return fail(PM_E_SHAPE, "problem too large");
    if (!gs0) return fail(PM_E_NULL, "gs0 is NULL");
    if (n_tok > 0 && (!q || !k || !v || !beta || !gq || !gk || !gv || !gbeta))
        return fail(PM_E_NULL, "q, k, v, beta, gq, gk, gv and gbeta must be non-NULL");
    const bool gated = g != nullptr || gg != nullptr;
    if (gated && n_tok > 0 && (!g || !gg)) return fail(PM_E_NULL, "g and gg must be non-NULL");
    const void* f32s[] = {beta, g, s0, go, gs, gq, gk, gv, gbeta, gg, gs0, workspace};
    for (const void* p : f32s)
        if (p && !aligned(p, 4)) return fail(PM_E_ALIGN, "fp32 buffers must be 4-byte aligned");
    const bool chunked16 = !gated && bwd_chunked(H, D, in_dtype);
    const bool chunked32 = !gated && bwd_chunked_f32(H, D, in_dtype);
    const bool chunked = chunked16 || chunked32;
    if (g_path >= 2 && !chunked)
        return fail(PM_E_UNSUPPORTED,
                    gated ? "the gated backward runs on the per-token kernels only (path 2 asks for the chunked one)"
                          : "chunked backward needs D in {64, 128} (got in_dtype %d, D %d)",
                    in_dtype, D);
    if (chunked && n_tok > 0) {
        const void* v16[] = {q, k, v, go, gq, gk, gv, workspace};
        for (const void* p : v16)
            if (p && !aligned(p, 16))
                return fail(PM_E_ALIGN,
                            "chunked backward: q, k, v, go, gq, gk, gv and workspace must be 16-byte aligned");
    }
    const size_t need = bwd_ws_bytes(B, T, H, D, in_dtype, !gated ? 0 : per_channel ? 2 : 1);
    if (need > 0 && (!workspace || ws_bytes < need))
        return fail(PM_E_WORKSPACE, "workspace of %zu bytes needed (got %zu)", need,
                    workspace ? ws_bytes : static_cast<size_t>(0));
    pm::BwdArgs a{q, k, v, beta, s0, go, gs, gq, gk, gv, gbeta, gs0,
                  static_cast<float*>(workspace), static_cast<int>(n_pairs), T, H, D,
                  in_dtype == PM_DTYPE_BF16};
    a.g = g;
    a.gg = gg;
    a.per_channel = per_channel;
    hipError_t e = chunked16   ? pm::launch_bwd_chunked(a, static_cast<hipStream_t>(stream))
                   : chunked32 ? pm::launch_bwd_chunked_f32(a, static_cast<hipStream_t>(stream))
                               : pm::launch_bwd(a, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? 0 : hip_fail(e, "backward launch");
}

// The forward's workspace: the split form's T blocks (bf16 inputs, where split_chosen), the
// fp32 chunked forward's (T'')^T and P^T (fp32 inputs), or a packed batch's sequence order
// for the single-stage kernel (bf16 inputs, 65 to kVarlenOrderMax sequences); else 0.
size_t fwd_ws_bytes(bool varlen, int n_seq, int T, int H, int D, int in_dtype) {
    if (n_seq < 0 || T < 0 || H < 0 || !pm::chunked_supported(D, H) || g_path == 1) return 0;
    const long n_pairs = static_cast<long>(n_seq) * H;
    if (n_pairs > (1L << 30)) return 0;
    if (in_dtype == PM_DTYPE_F32) return pm::chunked_f32_ws_bytes(varlen, n_seq, T, H);
    if (in_dtype != PM_DTYPE_BF16) return 0;
    if (split_chosen(g_path, D, n_pairs)) return pm::chunked_split_ws_bytes(varlen, n_seq, T, H);
    // the single-stage kernel: a packed batch's sequence order (longest first) beyond the 64
    // sequences the kernel ranks itself
    if (varlen && n_seq > 64 && n_seq <= pm::kVarlenOrderMax) return static_cast<size_t>(n_seq) * 4;
    return 0;
}

}  // namespace

extern "C" {

int pm_abi_version(void) { return PM_DELTA_ABI_VERSION; }

const char* pm_last_error(void) { return g_err; }

size_t pm_delta_workspace_bytes(int B, int T, int H, int D, int in_dtype) {
    return fwd_ws_bytes(false, B, T, H, D, in_dtype);
}

size_t pm_delta_varlen_workspace_bytes(int n_seqs, int total_T, int H, int D, int in_dtype) {
    return fwd_ws_bytes(true, n_seqs, total_T, H, D, in_dtype);
}

size_t pm_delta_bwd_workspace_bytes(int B, int T, int H, int D, int in_dtype) {
    if (B < 0 || T < 0 || H < 0 || D < 1 || D > pm::kBwdMaxD) return 0;
    if (in_dtype != PM_DTYPE_F32 && in_dtype != PM_DTYPE_BF16) return 0;
    return bwd_ws_bytes(B, T, H, D, in_dtype);
}

int pm_delta_bwd(const void* q, const void* k, const void* v, const float* beta,
                 const float* s0, const float* go, const float* gs, float* gq, float* gk,
                 float* gv, float* gbeta, float* gs0, int B, int T, int H, int D, int in_dtype,
                 void* workspace, size_t ws_bytes, void* stream) {
    g_err[0] = '\0';
    return backward(q, k, v, beta, nullptr, s0, go, gs, gq, gk, gv, gbeta, nullptr, gs0, B, T, H, D,
                    in_dtype, workspace, ws_bytes, stream);
}

size_t pm_gated_delta_bwd_workspace_bytes(int B, int T, int H, int D, int in_dtype) {
    if (B < 0 || T < 0 || H < 0 || D < 1 || D > pm::kBwdMaxD) return 0;
    if (in_dtype != PM_DTYPE_F32 && in_dtype != PM_DTYPE_BF16) return 0;
    return bwd_ws_bytes(B, T, H, D, in_dtype, 1);
}

size_t pm_kda_delta_bwd_workspace_bytes(int B, int T, int H, int D, int in_dtype) {
    if (B < 0 || T < 0 || H < 0 || D < 1 || D > pm::kBwdMaxD) return 0;
    if (in_dtype != PM_DTYPE_F32 && in_dtype != PM_DTYPE_BF16) return 0;
    return bwd_ws_bytes(B, T, H, D, in_dtype, 2);
}

int pm_kda_delta_bwd(const void* q, const void* k, const void* v, const float* beta,
                     const float* g, const float* s0, const float* go, const float* gs, float* gq,
                     float* gk, float* gv, float* gbeta, float* gg, float* gs0, int B, int T,
                     int H, int D, int in_dtype, void* workspace, size_t ws_bytes, void* stream) {
    g_err[0] = '\0';
    if (static_cast<long>(B) * T * H > 0 && (!g || !gg)) return fail(PM_E_NULL, "g and gg must be non-NULL");
    return backward(q, k, v, beta, g, s0, go, gs, gq, gk, gv, gbeta, gg, gs0, B, T, H, D, in_dtype,
                    workspace, ws_bytes, stream, true);
}

int pm_gated_delta_bwd(const void* q, const void* k, const void* v, const float* beta,
                       const float* g, const float* s0, const float* go, const float* gs, float* gq,
                       float* gk, float* gv, float* gbeta, float* gg, float* gs0, int B, int T,
                       int H, int D, int in_dtype, void* workspace, size_t ws_bytes, void* stream) {
    g_err[0] = '\0';
    if (static_cast<long>(B) * T * H > 0 && (!g || !gg)) return fail(PM_E_NULL, "g and gg must be non-NULL");
    return backward(q, k, v, beta, g, s0, go, gs, gq, gk, gv, gbeta, gg, gs0, B, T, H, D, in_dtype,
                    workspace, ws_bytes, stream);
}

int pm_delta_bwd_noalloc(const void* q, const void* k, const void* v, const float* beta,
                         const float* s0, const float* go, const float* gs, float* gq, float* gk,
                         float* gv, float* gbeta, float* gs0, int B, int T, int H, int D,
                         int in_dtype, void* stream) {
    g_err[0] = '\0';
    if (B < 0 || T < 0 || H < 0)
        return fail(PM_E_SHAPE, "B, T, H must be >= 0 (got %d, %d, %d)", B, T, H);
    if (D < 1 || D > pm::kBwdMaxD)
        return fail(PM_E_SHAPE, "backward D must be in [1, %d] (got %d)", pm::kBwdMaxD, D);
    if (in_dtype != PM_DTYPE_F32 && in_dtype != PM_DTYPE_BF16)
        return fail(PM_E_DTYPE, "in_dtype %d is not PM_DTYPE_F32 or PM_DTYPE_BF16", in_dtype);
    const size_t need = bwd_ws_bytes(B, T, H, D, in_dtype);
    if (need > kNoAllocScratchBytes)
        return fail(PM_E_WORKSPACE,
                    "the backward needs %zu bytes of workspace; the no-allocation entry point holds "
                    "%zu (use pm_delta_bwd with a caller workspace)",
                    need, kNoAllocScratchBytes);
    void* ws = nullptr;
    if (need > 0 && static_cast<long>(B) * H > 0) {
        if (int rc = scratch_address(&ws)) return rc;
    }
    return pm_delta_bwd(q, k, v, beta, s0, go, gs, gq, gk, gv, gbeta, gs0, B, T, H, D, in_dtype, ws,
                        ws ? kNoAllocScratchBytes : 0, stream);
}

int pm_delta_set_path(int path) {
    if (path < 0 || path > 3) return fail(PM_E_UNSUPPORTED, "path %d not in {0, 1, 2, 3}", path);
    const int old = g_path;
    g_path = path;
    return old;
}

int pm_delta_set_tile(int dv_tile) {
    if (dv_tile != 0 && dv_tile != 16 && dv_tile != 32 && dv_tile != 64)
        return fail(PM_E_UNSUPPORTED, "dv_tile %d not in {0, 16, 32, 64}", dv_tile);
    const int old = g_tile;
    g_tile = dv_tile;
    return old;
}

int pm_delta_fwd(const void* q, const void* k, const void* v, const float* beta,
                 const float* s0, void* o, float* s_out, int B, int T, int H, int D,
                 int in_dtype, int out_dtype, int chunk, void* workspace, size_t ws_bytes,
                 void* stream) {
    g_err[0] = '\0';
    if (B < 0 || T < 0 || H < 0)
        return fail(PM_E_SHAPE, "B, T, H must be >= 0 (got %d, %d, %d)", B, T, H);
    if (D < 1 || D > PM_DELTA_MAX_D)
        return fail(PM_E_SHAPE, "D must be in [1, %d] (got %d)", PM_DELTA_MAX_D, D);
    if (chunk < 1) return fail(PM_E_SHAPE, "chunk must be >= 1, got %d", chunk);
    if (int rc = check_dtypes(in_dtype, out_dtype)) return rc;
    return forward(q, k, v, beta, s0, o, s_out, nullptr, B, T, 0, H, D, in_dtype, out_dtype,
                   chunk, static_cast<hipStream_t>(stream), nullptr, workspace, ws_bytes);
}

int pm_delta_fwd_varlen(const void* q, const void* k, const void* v, const float* beta,
                        const int32_t* cu_seqlens, int n_seqs, int total_T, const float* s0,
                        void* o, float* s_out, int H, int D, int in_dtype, int out_dtype,
                        int chunk, void* workspace, size_t ws_bytes, void* stream) {
    g_err[0] = '\0';
    if (n_seqs < 0 || total_T < 0 || H < 0)
        return fail(PM_E_SHAPE, "n_seqs, total_T, H must be >= 0 (got %d, %d, %d)", n_seqs,
                    total_T, H);
    if (D < 1 || D > PM_DELTA_MAX_D)
        return fail(PM_E_SHAPE, "D must be in [1, %d] (got %d)", PM_DELTA_MAX_D, D);
    if (chunk < 1) return fail(PM_E_SHAPE, "chunk must be >= 1, got %d", chunk);
    if (int rc = check_dtypes(in_dtype, out_dtype)) return rc;
    if (n_seqs > 0 && !cu_seqlens) return fail(PM_E_NULL, "cu_seqlens is NULL");
    if (cu_seqlens && !aligned(cu_seqlens, 4))
        return fail(PM_E_ALIGN, "cu_seqlens must be 4-byte aligned");
    return forward(q, k, v, beta, s0, o, s_out, cu_seqlens, n_seqs, 0, total_T, H, D, in_dtype,
                   out_dtype, chunk, static_cast<hipStream_t>(stream), nullptr, workspace, ws_bytes);
}

int pm_varlen_check(const int32_t* cu_seqlens, int n_seqs, int total_T, int32_t* flag, void* stream) {
    g_err[0] = '\0';
    if (n_seqs < 0 || total_T < 0)
        return fail(PM_E_SHAPE, "n_seqs and total_T must be >= 0 (got %d, %d)", n_seqs, total_T);
    if (!cu_seqlens || !flag) return fail(PM_E_NULL, "cu_seqlens and flag must be non-NULL");
    if (!aligned(cu_seqlens, 4) || !aligned(flag, 4))
        return fail(PM_E_ALIGN, "cu_seqlens and flag must be 4-byte aligned");
    hipError_t e = pm::launch_varlen_check(cu_seqlens, n_seqs, total_T, flag, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? 0 : hip_fail(e, "cu_seqlens check launch");
}

int pm_delta_step_slots(float* pool, const int32_t* slots, int n_slots, const void* q,
                        const void* k, const void* v, const float* beta, float* o, int B, int H,
                        int D, int in_dtype, void* stream) {
    g_err[0] = '\0';
    if (B < 0 || H < 0 || n_slots < 0)
        return fail(PM_E_SHAPE, "B, H, n_slots must be >= 0 (got %d, %d, %d)", B, H, n_slots);
    if (!pm::step_supported(D))
        return fail(PM_E_UNSUPPORTED, "slot-indexed decode step needs D in {32, 64, 128} (got %d)", D);
    if (in_dtype != PM_DTYPE_F32 && in_dtype != PM_DTYPE_BF16)
        return fail(PM_E_DTYPE, "in_dtype %d is not PM_DTYPE_F32 or PM_DTYPE_BF16", in_dtype);
    const long n_pairs = static_cast<long>(B) * H;
    if (n_pairs == 0) return 0;
    if (n_pairs > (1L << 30) || static_cast<long>(n_slots) * H > (1L << 30))
        return fail(PM_E_SHAPE, "problem too large");
    if (!slots || !q || !k || !v || !beta || !o || (n_slots > 0 && !pool))
        return fail(PM_E_NULL, "slots, q, k, v, beta, o (and pool when n_slots > 0) must be non-NULL");
    if ((pool && !aligned(pool, 16)) || !aligned(o, 16) || !aligned(slots, 4) || !aligned(beta, 4))
        return fail(PM_E_ALIGN, "pool and o must be 16-byte aligned, slots and beta 4-byte aligned");
    pm::StepArgs a{pool, q, k, v, beta, o, static_cast<int>(n_pairs), D, in_dtype == PM_DTYPE_BF16,
                   slots, H, n_slots};
    hipError_t e = pm::launch_step(a, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? 0 : hip_fail(e, "slot decode step launch");
}

size_t pm_linear_attention_workspace_bytes(int B, int T, int H, int D, int in_dtype) {
    if (B < 0 || T < 0 || H < 0 || in_dtype != PM_DTYPE_F32 || !pm::chunked_supported(D, H) || g_path == 1)
        return 0;
    if (static_cast<long>(B) * H > (1L << 30)) return 0;
    return pm::chunked_f32_ws_bytes(false, B, T, H, true);
}

int pm_linear_attention(const void* q, const void* k, const void* v, const float* s0, void* o,
                        float* s_out, int B, int T, int H, int D, int in_dtype, int out_dtype,
                        void* stream) {
    return pm_linear_attention_ws(q, k, v, s0, o, s_out, B, T, H, D, in_dtype, out_dtype, nullptr, 0, stream);
}

int pm_linear_attention_ws(const void* q, const void* k, const void* v, const float* s0, void* o,
                           float* s_out, int B, int T, int H, int D, int in_dtype, int out_dtype,
                           void* workspace, size_t ws_bytes, void* stream) {
    g_err[0] = '\0';
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (B < 0 || T < 0 || H < 0)
        return fail(PM_E_SHAPE, "B, T, H must be >= 0 (got %d, %d, %d)", B, T, H);
    if (D < 1 || D > PM_DELTA_MAX_D)
        return fail(PM_E_SHAPE, "D must be in [1, %d] (got %d)", PM_DELTA_MAX_D, D);
    if (int rc = check_dtypes(in_dtype, out_dtype)) return rc;
    const long n_pairs = static_cast<long>(B) * H;
    const long n_tok = static_cast<long>(B) * T;
    if (n_pairs == 0) return 0;
    if (n_pairs > (1L << 30) || n_tok > (1L << 40)) return fail(PM_E_SHAPE, "problem too large");
    if (!s_out) return fail(PM_E_NULL, "s_out is NULL");
    if (n_tok > 0 && (!q || !k || !v || !o))
        return fail(PM_E_NULL, "q, k, v and o must be non-NULL");
    if (!aligned(s_out, 4) || (s0 && !aligned(s0, 4)))
        return fail(PM_E_ALIGN, "fp32 buffers must be 4-byte aligned");
    if (n_tok == 0) {
        const size_t s_elems = static_cast<size_t>(n_pairs) * D * D;
        hipError_t e = s0 ? pm::launch_copy_f32(s_out, s0, s_elems, st)
                          : pm::launch_fill_zero(s_out, s_elems, st);
        return e == hipSuccess ? 0 : hip_fail(e, "state copy");
    }
    const int path = g_path;
    const bool can_chunked = in_dtype == PM_DTYPE_BF16 && pm::chunked_supported(D, H) &&
                             aligned(q, 16) && aligned(k, 16) && aligned(v, 16) &&
                             (out_dtype == PM_DTYPE_F32 ? aligned(o, 16) : aligned(o, 8));
    // fp32 q/k/v: the fp32 chunked forward in its normalised mode, with the workspace
    const bool can_f32 = in_dtype == PM_DTYPE_F32 && pm::chunked_supported(D, H) && aligned(q, 16) &&
                         aligned(k, 16) && aligned(v, 16) && (out_dtype == PM_DTYPE_F32 ? aligned(o, 4) : aligned(o, 2));
    if (path >= 2 && !can_chunked && !can_f32)
        return fail(PM_E_UNSUPPORTED,
                    "chunked kernel needs bf16 or fp32 inputs, D in {64, 128} and 16-byte aligned "
                    "q/k/v (got in_dtype %d, D %d)",
                    in_dtype, D);
    if (path != 1 && can_chunked) {
        pm::ChunkedArgs a{static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                          static_cast<const uint16_t*>(v), nullptr, s0, o, s_out, nullptr, B, T, H, D,
                          out_dtype == PM_DTYPE_BF16, g_tile, true};
        hipError_t e = pm::launch_chunked(a, st);
        return e == hipSuccess ? 0 : hip_fail(e, "chunked linear attention launch");
    }
    if (path != 1 && can_f32) {
        const size_t need = pm::chunked_f32_ws_bytes(false, B, T, H, true);
        if (workspace && ws_bytes >= need && aligned(workspace, 16)) {
            pm::ChunkedF32Args a{static_cast<const float*>(q), static_cast<const float*>(k),
                                 static_cast<const float*>(v), nullptr, s0, o, s_out, nullptr, B, T, H, D,
                                 out_dtype == PM_DTYPE_BF16, g_tile};
            a.norm = true;
            hipError_t e = pm::launch_chunked_f32(a, workspace, st);
            return e == hipSuccess ? 0 : hip_fail(e, "fp32 chunked linear attention launch");
        }
        if (path >= 2)
            return fail(PM_E_WORKSPACE, "the fp32 chunked linear attention needs a 16-byte aligned workspace of "
                        "%zu bytes (got %zu)", need, workspace ? ws_bytes : static_cast<size_t>(0));
    }
    pm::RecurrentArgs a{q, k, v, nullptr, s0, o, s_out, nullptr, static_cast<int>(n_pairs), T, H, D,
                        in_dtype == PM_DTYPE_BF16, out_dtype == PM_DTYPE_BF16, true};
    hipError_t e = pm::launch_recurrent(a, st);
    return e == hipSuccess ? 0 : hip_fail(e, "linear attention launch");
}

int pm_delta_step(float* s_inout, const void* q, const void* k, const void* v,
                  const float* beta, float* o, int B, int H, int D, int in_dtype, void* stream) {
    return step(s_inout, q, k, v, beta, nullptr, o, B, H, D, in_dtype, stream);
}

int pm_gated_delta_step(float* s_inout, const void* q, const void* k, const void* v,
                        const float* beta, const float* g, float* o, int B, int H, int D,
                        int in_dtype, void* stream) {
    g_err[0] = '\0';
    if (static_cast<long>(B) * H > 0 && !g) return fail(PM_E_NULL, "g is NULL");
    if (g && !aligned(g, 4)) return fail(PM_E_ALIGN, "g must be 4-byte aligned");
    return step(s_inout, q, k, v, beta, g, o, B, H, D, in_dtype, stream);
}

int pm_gated_delta_fwd(const void* q, const void* k, const void* v, const float* beta,
                       const float* g, const float* s0, void* o, float* s_out, int B, int T, int H,
                       int D, int in_dtype, int out_dtype, void* stream) {
    g_err[0] = '\0';
    if (B < 0 || T < 0 || H < 0)
        return fail(PM_E_SHAPE, "B, T, H must be >= 0 (got %d, %d, %d)", B, T, H);
    if (D < 1 || D > PM_DELTA_MAX_D)
        return fail(PM_E_SHAPE, "D must be in [1, %d] (got %d)", PM_DELTA_MAX_D, D);
    if (int rc = check_dtypes(in_dtype, out_dtype)) return rc;
    if (static_cast<long>(B) * T * H > 0 && !g) return fail(PM_E_NULL, "g is NULL");
    if (g && !aligned(g, 4)) return fail(PM_E_ALIGN, "g must be 4-byte aligned");
    return forward(q, k, v, beta, s0, o, s_out, nullptr, B, T, 0, H, D, in_dtype, out_dtype, 64,
                   static_cast<hipStream_t>(stream), g);
}

size_t pm_kda_delta_workspace_bytes(int B, int T, int H, int D, int in_dtype) {
    if (B < 0 || T < 0 || H < 0 || in_dtype != PM_DTYPE_BF16 || !pm::chunked_supported(D, H) || g_path == 1)
        return 0;
    if (static_cast<long>(B) * H > (1L << 30)) return 0;
    return pm::kda_chunked_ws_bytes(B, T, H, D);
}

int pm_kda_delta_fwd(const void* q, const void* k, const void* v, const float* beta,
                     const float* g, const float* s0, void* o, float* s_out, int B, int T, int H,
                     int D, int in_dtype, int out_dtype, void* workspace, size_t ws_bytes, void* stream) {
    g_err[0] = '\0';
    if (B < 0 || T < 0 || H < 0)
        return fail(PM_E_SHAPE, "B, T, H must be >= 0 (got %d, %d, %d)", B, T, H);
    if (D < 1 || D > PM_DELTA_MAX_D)
        return fail(PM_E_SHAPE, "D must be in [1, %d] (got %d)", PM_DELTA_MAX_D, D);
    if (int rc = check_dtypes(in_dtype, out_dtype)) return rc;
    const long n_pairs = static_cast<long>(B) * H, n_tok = static_cast<long>(B) * T;
    if (n_pairs * T > 0 && !g) return fail(PM_E_NULL, "g is NULL");
    if (g && !aligned(g, 4)) return fail(PM_E_ALIGN, "g must be 4-byte aligned");
    hipStream_t st = static_cast<hipStream_t>(stream);
    // the chunked form (bf16 q/k/v, D in {64, 128}) with the caller's workspace; otherwise,
    // and always under path 1, the per-token kernel
    const bool can_chunked = in_dtype == PM_DTYPE_BF16 && pm::chunked_supported(D, H) && aligned(q, 16) &&
                             aligned(k, 16) && aligned(v, 16) &&
                             (out_dtype == PM_DTYPE_F32 ? aligned(o, 16) : aligned(o, 8));
    if (g_path != 1 && can_chunked && n_pairs > 0 && n_tok > 0 && n_pairs <= (1L << 30)) {
        if (!s_out || !q || !k || !v || !beta || !o) return fail(PM_E_NULL, "q, k, v, beta, o and s_out must be non-NULL");
        if (!aligned(beta, 4) || !aligned(s_out, 4) || (s0 && !aligned(s0, 4)))
            return fail(PM_E_ALIGN, "fp32 buffers must be 4-byte aligned");
        const size_t need = pm::kda_chunked_ws_bytes(B, T, H, D);
        if (workspace && ws_bytes >= need && aligned(workspace, 16)) {
            pm::KdaChunkedArgs a{static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                                 static_cast<const uint16_t*>(v), beta, g, s0, o, s_out, B, T, H, D,
                                 out_dtype == PM_DTYPE_BF16, workspace};
            hipError_t e = pm::launch_kda_chunked(a, st);
            return e == hipSuccess ? 0 : hip_fail(e, "KDA chunked forward launch");
        }
        if (g_path >= 2)
            return fail(PM_E_WORKSPACE, "the KDA chunked forward needs a 16-byte aligned workspace of %zu bytes "
                        "(got %zu)", need, workspace ? ws_bytes : static_cast<size_t>(0));
    } else if (g_path >= 2 && n_pairs > 0 && n_tok > 0) {
        return fail(PM_E_UNSUPPORTED,
                    "the KDA chunked forward needs bf16 q/k/v, D in {64, 128} and 16-byte aligned q/k/v/o "
                    "(got in_dtype %d, D %d)", in_dtype, D);
    }
    // per-token kernel: forward() with the per-channel gates, as path 1
    const int old = g_path;
    g_path = 1;
    const int rc = forward(q, k, v, beta, s0, o, s_out, nullptr, B, T, 0, H, D, in_dtype, out_dtype, 64, st,
                           nullptr, nullptr, 0, g);
    g_path = old;
    return rc;
}

int pm_kda_delta_step(float* s_inout, const void* q, const void* k, const void* v,
                      const float* beta, const float* g, float* o, int B, int H, int D,
                      int in_dtype, void* stream) {
    g_err[0] = '\0';
    if (static_cast<long>(B) * H > 0 && !g) return fail(PM_E_NULL, "g is NULL");
    if (g && !aligned(g, 4)) return fail(PM_E_ALIGN, "g must be 4-byte aligned");
    return step(s_inout, q, k, v, beta, nullptr, o, B, H, D, in_dtype, stream, g);
}

}  // extern "C"
