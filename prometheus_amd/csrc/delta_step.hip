// delta_step.hip — K3: single-token recurrent decode step, S updated in place.
//
// Same step algebra as the reference (kernels/__init__.py:357-376):
//   kS = k^T S ;  S' = S + beta k (v - kS)^T ;  o = q S'
// The step is HBM-bound (about 0.74 flop per byte at D=128): S is streamed
// in once and out once with 128-bit non-temporal accesses and every column
// of S stays in VGPRs between the two reductions (k^T S, then q^T S').
//
// Mapping (D=128): one 256-thread workgroup per (b, h), on a (H, B) grid so that no
// division is needed to find b.  Thread t owns
// columns 4*(t % 32) .. +3 and rows (t / 32) + 8*i, i < 16, so each wave
// instruction reads or writes two whole 512-byte rows (1 KiB contiguous).
// Column partial sums are reduced across the row groups of a wave with
// cross-lane shuffles, then across the 4 waves through LDS.
//
// State-cache mode (slots != NULL): the serving side keeps every request's
// fixed-size state in a pool of n_slots x H x D x D and decodes a batch
// through a slot table; request b updates pool[slots[b]].  A slot outside
// [0, n_slots) (padding in a fixed-size, graph-captured batch) is skipped:
// no state is read or written and the output row is zero.

#include "pm_common.h"
#include "pm_internal.h"

namespace pm {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// GM 1 (gated): S' = alpha (S - beta k (k^T S)) + beta k v^T with alpha = exp(g[b, h]).
// GM 2 (per-channel, KDA): S is first decayed row by row, S <- Diag(exp(g[b, h, :])) S,
// and the ungated step runs on the decayed state.
template <int D, typename InT, int GM>
__global__ __launch_bounds__(256) void delta_step_kernel(float* __restrict__ s,
                                                         const InT* __restrict__ q,
                                                         const InT* __restrict__ k,
                                                         const InT* __restrict__ v,
                                                         const float* __restrict__ beta,
                                                         float* __restrict__ o,
                                                         const int32_t* __restrict__ slots,
                                                         int b0, int n_slots,
                                                         const float* __restrict__ gate) {
    constexpr int NT = 256;
    constexpr int CG = D / 4;      // column groups of 4
    constexpr int RG = NT / CG;    // row groups
    constexpr int RPT = D / RG;    // rows per thread
    constexpr int NW = NT / 64;    // waves
    static_assert(CG <= 64 && RPT >= 1, "unsupported D");

    constexpr bool GATED = GM == 1, CHAN = GM == 2;
    __shared__ float sk[D], sq[D], sv[D], sa[CHAN ? D : 1];
    __shared__ f32x4 red[2][NW][CG];

    const int H = static_cast<int>(gridDim.x), bi = b0 + static_cast<int>(blockIdx.y);
    const int pair = bi * H + static_cast<int>(blockIdx.x);
    const int t = threadIdx.x;
    const int cg = t % CG, rg = t / CG;
    const int lane = t & 63, w = t >> 6;

    // the token's q, k, v and beta do not depend on the slot: their loads go out first
    InT kq = InT(), qq = InT(), vq = InT();
    float gq = 0.f;
    if (t < D) {
        const size_t a = static_cast<size_t>(pair) * D + t;
        kq = k[a];
        qq = q[a];
        vq = v[a];
        if constexpr (CHAN) gq = gate[a];
    }
    const float b = beta[pair];
    size_t state = pair;
    if (slots) {
        const int slot = slots[bi];
        if (slot < 0 || slot >= n_slots) {
            if (t < CG) {
                const f32x4 z = {0.f, 0.f, 0.f, 0.f};
                reinterpret_cast<f32x4*>(o + static_cast<size_t>(pair) * D)[cg] = z;
            }
            return;
        }
        state = static_cast<size_t>(slot) * H + blockIdx.x;
    }
    f32x4* sp = reinterpret_cast<f32x4*>(s + state * D * D);
    f32x4 S[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i)
        S[i] = __builtin_nontemporal_load(sp + (rg + RG * i) * CG + cg);

    if (t < D) {
        sk[t] = to_f32(kq);
        sq[t] = to_f32(qq);
        sv[t] = to_f32(vq);
        if constexpr (CHAN) sa[t] = expf(gq);
    }
    __syncthreads();
    if constexpr (CHAN) {
#pragma unroll
        for (int i = 0; i < RPT; ++i) S[i] *= sa[rg + RG * i];
    }

    f32x4 kp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < RPT; ++i) kp += sk[rg + RG * i] * S[i];
#pragma unroll
    for (int m = CG; m < 64; m <<= 1) {
        kp.x += __shfl_xor(kp.x, m);
        kp.y += __shfl_xor(kp.y, m);
        kp.z += __shfl_xor(kp.z, m);
        kp.w += __shfl_xor(kp.w, m);
    }
    if (lane < CG) red[0][w][cg] = kp;
    __syncthreads();
    f32x4 ks = red[0][0][cg];
#pragma unroll
    for (int j = 1; j < NW; ++j) ks += red[0][j][cg];

    const f32x4 vv = {sv[4 * cg], sv[4 * cg + 1], sv[4 * cg + 2], sv[4 * cg + 3]};
    float al = 1.f;
    if constexpr (GATED) al = expf(gate[pair]);
    const f32x4 u = GATED ? b * (vv - al * ks) : b * (vv - ks);
    f32x4 op = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
        const int row = rg + RG * i;
        if constexpr (GATED) S[i] = al * S[i] + sk[row] * u;
        else S[i] += sk[row] * u;
        op += sq[row] * S[i];
        __builtin_nontemporal_store(S[i], sp + row * CG + cg);
    }
#pragma unroll
    for (int m = CG; m < 64; m <<= 1) {
        op.x += __shfl_xor(op.x, m);
        op.y += __shfl_xor(op.y, m);
        op.z += __shfl_xor(op.z, m);
        op.w += __shfl_xor(op.w, m);
    }
    if (lane < CG) red[1][w][cg] = op;
    __syncthreads();
    if (t < CG) {
        f32x4 acc = red[1][0][cg];
#pragma unroll
        for (int j = 1; j < NW; ++j) acc += red[1][j][cg];
        reinterpret_cast<f32x4*>(o + static_cast<size_t>(pair) * D)[cg] = acc;
    }
}

bool step_supported(int D) { return D == 32 || D == 64 || D == 128; }

template <int D, int GM>
static hipError_t launch_step_g(const StepArgs& a, hipStream_t st) {
    // grid (H, rows of b), at most 65535 rows per launch
    const int n_b = a.n_pairs / a.H;
    for (int b0 = 0; b0 < n_b; b0 += 65535) {
        const dim3 grid(static_cast<unsigned>(a.H), static_cast<unsigned>(min(65535, n_b - b0)));
        if (a.in_bf16) {
            hipLaunchKernelGGL((delta_step_kernel<D, uint16_t, GM>), grid, dim3(256), 0, st, a.s,
                               static_cast<const uint16_t*>(a.q), static_cast<const uint16_t*>(a.k),
                               static_cast<const uint16_t*>(a.v), a.beta, a.o, a.slots, b0, a.n_slots,
                               GM == 2 ? a.gk : a.g);
        } else {
            hipLaunchKernelGGL((delta_step_kernel<D, float, GM>), grid, dim3(256), 0, st, a.s,
                               static_cast<const float*>(a.q), static_cast<const float*>(a.k),
                               static_cast<const float*>(a.v), a.beta, a.o, a.slots, b0, a.n_slots,
                               GM == 2 ? a.gk : a.g);
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

template <int D>
static hipError_t launch_step_d(const StepArgs& a, hipStream_t st) {
    if (a.gk) return launch_step_g<D, 2>(a, st);
    return a.g ? launch_step_g<D, 1>(a, st) : launch_step_g<D, 0>(a, st);
}

hipError_t launch_step(const StepArgs& a, hipStream_t st) {
    if (a.n_pairs == 0) return hipSuccess;
    switch (a.D) {
        case 32: return launch_step_d<32>(a, st);
        case 64: return launch_step_d<64>(a, st);
        case 128: return launch_step_d<128>(a, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace pm
