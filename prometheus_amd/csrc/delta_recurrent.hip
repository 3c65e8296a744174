// delta_recurrent.hip — K4: per-token delta-rule recurrence for any D <= 256.
//
// The reference's own algorithm (kernels/__init__.py:357-376 step,
// sequential over tokens as in :379-395 / :421-458), in fp32 on the VALU:
//   kS = k^T S ;  u = beta (v - kS) ;  S += k u^T ;  o = q S
// It serves fp32 inputs (parity at 1e-5 against the fp32 reference), every
// head dimension the chunked MFMA kernel does not cover (the reference's
// own tests use D = 2..8), the varlen form of those, and pm_delta_step for
// D outside the specialised decode kernel.
//
// Mapping: one workgroup per (sequence, head).  Thread (e, r) holds rows
// [r*RPT, r*RPT + RPT) of column e of S in registers (RS = row slices per
// column, adjacent lanes, reduced with DPP quad permutes).  Tokens are
// staged into LDS STEPS at a time so the inner loop has no barriers.
// S is read once at the start and written once at the end, so s0 may alias
// s_out (the decode step runs in place).
//
// The model's linear attention (model/__init__.py:393-432) runs here too:
// with l2norm, each staged q and k row is divided by max(||row||_2, 1e-6)
// (its _l2_normalize, :203-205) before use, and a NULL beta means beta = 1.
//
// Gated variant (log-gates g, alpha = exp(g) per token and head):
//   S_t = alpha_t (I - beta_t k_t k_t^T) S_{t-1} + beta_t k_t v_t^T,
// i.e. u = beta (v - alpha k^T S), S = alpha S + k u^T.  Without g, alpha = 1
// and the arithmetic is exactly the ungated step.

#include "pm_common.h"
#include "pm_internal.h"

namespace pm {

constexpr int kRecSteps = 16;

// Sum over the RS adjacent lanes that hold one column (RS in {1, 2, 4}): DPP quad
// permutes, no LDS round trip.
__device__ __forceinline__ float quad_xor(float x, int ctrl) {
    const int xi = __float_as_int(x);
    return __int_as_float(ctrl == 1 ? __builtin_amdgcn_update_dpp(xi, xi, 0xB1, 0xF, 0xF, false)
                                    : __builtin_amdgcn_update_dpp(xi, xi, 0x4E, 0xF, 0xF, false));
}
__device__ __forceinline__ float col_sum(float x, int RS) {
    if (RS >= 2) x += quad_xor(x, 1);  // lanes i, i ^ 1
    if (RS >= 4) x += quad_xor(x, 2);  // lanes i, i ^ 2
    return x;
}
// Dot product of a row slice with four independent accumulators (RPT % 4 == 0), so the
// dependent chain is RPT / 4 FMAs long.
template <int RPT>
__device__ __forceinline__ float dot4(const float* a, const float (&b)[RPT]) {
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
    for (int i = 0; i < RPT; i += 4) {
        s0 = fmaf(a[i], b[i], s0);
        s1 = fmaf(a[i + 1], b[i + 1], s1);
        s2 = fmaf(a[i + 2], b[i + 2], s2);
        s3 = fmaf(a[i + 3], b[i + 3], s3);
    }
    return (s0 + s1) + (s2 + s3);
}

// D <= 128 runs at most 512 threads (RPT 32, 4 slices); only D > 128 needs
// 1024 threads, where the 64-row slices do not fit the register budget and
// part of S spills (a rare shape, kept for generality).
template <int RPT, typename InT, typename OutT>
__global__ __launch_bounds__(RPT >= 64 ? 1024 : 512) void delta_recurrent_kernel(
    const InT* __restrict__ q, const InT* __restrict__ k, const InT* __restrict__ v,
    const float* __restrict__ beta, const float* s0, OutT* __restrict__ o, float* s_out,
    const int32_t* __restrict__ cu_seqlens, int T, int H, int D, int RS, int l2norm,
    const float* __restrict__ gate) {
    extern __shared__ float lds[];
    const int DP = RS * RPT;  // padded row count per column
    float* sk = lds;                          // [kRecSteps][DP]
    float* sq = sk + kRecSteps * DP;          // [kRecSteps][DP]
    float* sv = sq + kRecSteps * DP;          // [kRecSteps][DP]
    float* sb = sv + kRecSteps * DP;          // [kRecSteps]
    float* sa = sb + kRecSteps;               // [kRecSteps] alpha

    const int pair = blockIdx.x;
    const int seq = pair / H, h = pair % H;
    long tok0;
    int len;
    if (cu_seqlens) {
        // varlen: T is the packed token count; offsets are clamped into it
        const int a = min(max(cu_seqlens[seq], 0), T);
        const int z = min(max(cu_seqlens[seq + 1], a), T);
        tok0 = a;
        len = z - a;
    } else {
        tok0 = static_cast<long>(seq) * T;
        len = T;
    }

    const int tid = threadIdx.x;
    const int e = tid / RS;
    const int r = tid % RS;
    const bool col_ok = e < D;
    const size_t sbase = static_cast<size_t>(pair) * D * D;

    float S[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
        const int d = r * RPT + i;
        S[i] = (s0 && col_ok && d < D) ? s0[sbase + static_cast<size_t>(d) * D + e] : 0.0f;
    }

    for (int t0 = 0; t0 < len; t0 += kRecSteps) {
        const int nst = min(kRecSteps, len - t0);
        __syncthreads();
        for (int idx = tid; idx < kRecSteps * DP; idx += blockDim.x) {
            const int j = idx / DP, d = idx % DP;
            float kv = 0.f, qv = 0.f, vv = 0.f;
            if (j < nst && d < D) {
                const size_t a = (static_cast<size_t>(tok0 + t0 + j) * H + h) * D + d;
                kv = to_f32(k[a]);
                qv = to_f32(q[a]);
                vv = to_f32(v[a]);
            }
            sk[idx] = kv;
            sq[idx] = qv;
            sv[idx] = vv;
        }
        for (int j = tid; j < kRecSteps; j += blockDim.x) {
            const size_t a = static_cast<size_t>(tok0 + t0 + j) * H + h;
            sb[j] = (j >= nst) ? 0.f : beta ? beta[a] : 1.f;
            sa[j] = (j < nst && gate) ? expf(gate[a]) : 1.f;
        }
        __syncthreads();
        if (l2norm) {
            // one wave per staged row (k rows, then q rows): x / max(||x||, 1e-6)
            const int lane = tid & 63, nw = blockDim.x >> 6;
            for (int row = tid >> 6; row < 2 * nst; row += nw) {
                float* x = (row < nst ? sk : sq) + (row % nst) * DP;
                float ss = 0.f;
                for (int d = lane; d < D; d += 64) ss = fmaf(x[d], x[d], ss);
                for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m);
                const float den = fmaxf(sqrtf(ss), 1e-6f);
                for (int d = lane; d < D; d += 64) x[d] = x[d] / den;
            }
            __syncthreads();
        }

        for (int j = 0; j < nst; ++j) {
            const float* kr = sk + j * DP + r * RPT;
            const float* qr = sq + j * DP + r * RPT;
            const float ks = col_sum(dot4<RPT>(kr, S), RS);
            const float al = sa[j];
            const float u = sb[j] * ((col_ok ? sv[j * DP + e] : 0.f) - al * ks);
#pragma unroll
            for (int i = 0; i < RPT; ++i) S[i] = fmaf(kr[i], u, al * S[i]);
            const float os = col_sum(dot4<RPT>(qr, S), RS);
            if (r == 0 && col_ok)
                o[(static_cast<size_t>(tok0 + t0 + j) * H + h) * D + e] = from_f32<OutT>(os);
        }
    }

    if (col_ok) {
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
            const int d = r * RPT + i;
            if (d < D) s_out[sbase + static_cast<size_t>(d) * D + e] = S[i];
        }
    }
}

// Picks rows-per-thread and the row-slice count for head dimension D.
// (RS <= 4 for every D <= 256, as col_sum needs.)
static void recurrent_geometry(int D, int* rpt, int* rs) {
    int r = (D <= 8) ? 8 : (D <= 16) ? 16 : (D <= 128) ? 32 : 64;
    int s = 1;
    while (r * s < D) s <<= 1;
    *rpt = r;
    *rs = s;
}

template <int RPT, typename InT, typename OutT>
static hipError_t launch_rec_t(const RecurrentArgs& a, int rs, hipStream_t st) {
    const int threads = ((a.D * rs + 63) / 64) * 64;
    const size_t lds = sizeof(float) * (3 * kRecSteps * rs * RPT + 2 * kRecSteps);
    hipLaunchKernelGGL((delta_recurrent_kernel<RPT, InT, OutT>), dim3(a.n_pairs), dim3(threads),
                       lds, st, static_cast<const InT*>(a.q), static_cast<const InT*>(a.k),
                       static_cast<const InT*>(a.v), a.beta, a.s0, static_cast<OutT*>(a.o),
                       a.s_out, a.cu_seqlens, a.T, a.H, a.D, rs, a.l2norm ? 1 : 0, a.g);
    return hipGetLastError();
}

template <typename InT, typename OutT>
static hipError_t launch_rec_io(const RecurrentArgs& a, hipStream_t st) {
    int rpt, rs;
    recurrent_geometry(a.D, &rpt, &rs);
    switch (rpt) {
        case 8: return launch_rec_t<8, InT, OutT>(a, rs, st);
        case 16: return launch_rec_t<16, InT, OutT>(a, rs, st);
        case 32: return launch_rec_t<32, InT, OutT>(a, rs, st);
        default: return launch_rec_t<64, InT, OutT>(a, rs, st);
    }
}

hipError_t launch_recurrent(const RecurrentArgs& a, hipStream_t st) {
    if (a.n_pairs == 0) return hipSuccess;
    if (a.in_bf16) {
        return a.out_bf16 ? launch_rec_io<uint16_t, uint16_t>(a, st)
                          : launch_rec_io<uint16_t, float>(a, st);
    }
    return a.out_bf16 ? launch_rec_io<float, uint16_t>(a, st) : launch_rec_io<float, float>(a, st);
}

}  // namespace pm
