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
// Mapping.  Given k, v and beta, the columns of S evolve independently
// (column e: kS_e = k . S[:, e], u_e = beta (v_e - kS_e), S[:, e] += k u_e,
// o_e = q . S[:, e]), so each (sequence, head) is split into column groups of
// CW = 256 / RS columns, one 256-thread workgroup per group.  Thread (el, r)
// holds rows [r*RPT, r*RPT + RPT) of column c*CW + el in registers; the RS
// row slices of a column are adjacent lanes of one 16-lane DPP row and are
// summed with DPP (no LDS round trip).  A column's arithmetic depends on RPT
// and RS only (fixed by D), never on the group width or the grid.
//
// Per token, k.S and q.S are both taken from the state before the update, and
//   o = q.S_new = alpha (q.S) + (q.k) u
// with q.k formed once per token while staging: the two dot products and their
// lane sums run side by side, and only the rank-1 update waits for u.
//
// Tokens are staged into LDS 16 at a time, double-buffered with one barrier
// per block: the q/k/v/beta/gate loads of block b + 1 are issued into
// registers before block b's token loop and written to LDS after it, and a
// block's outputs leave through LDS as row segments one block later.  Row
// slices sit at a stride of RPT + 4 floats, so the 16-byte slice reads of a
// wave hit distinct banks.  Workgroups of one (sequence, head) are numbered
// 8 apart, so they run on one XCD and share its L2 copy of q and k.
// S is read once at the start and written once at the end, column group by
// column group, so s0 may alias s_out (the decode step runs in place).
//
// The model's linear attention (model/__init__.py:393-432) runs here too:
// with l2norm, each staged q and k row is divided by max(||row||_2, 1e-6)
// (its _l2_normalize, :203-205) before use, and a NULL beta means beta = 1.
//
// Gated variant (log-gates g, alpha = exp(g) per token and head):
//   S_t = alpha_t (I - beta_t k_t k_t^T) S_{t-1} + beta_t k_t v_t^T,
// i.e. u = beta (v - alpha k^T S), S = alpha S + k u^T.  With g = 0, alpha = 1
// and the arithmetic is exactly the ungated step.
//
// Per-channel variant (KDA: log-gates g per token, head and key channel,
// alpha_t = exp(g_t) a d_k-vector):
//   S_t = (I - beta_t k_t k_t^T) Diag(alpha_t) S_{t-1} + beta_t k_t v_t^T.
// Row d of S is the key channel d, so a thread scales its RPT rows by their
// own alpha before the token's dot products, and the rest is the ungated step
// on the decayed state.  The alpha rows are staged like the k rows (one more
// [16][DPL] array per buffer, after the per-token scalars).

#include "pm_common.h"
#include "pm_internal.h"
#include "pm_rec.h"

namespace pm {

// One (sequence, head) column group per workgroup; blockIdx = (slot * ncg + c) * 8 + x
// for pair = pair0 + slot * 8 + x and column group c.
// GM: 0 no gate, 1 a log-gate per (token, head), 2 one per (token, head, key channel).
template <int RPT, int RS, int GM, typename InT, typename OutT>
__global__ __launch_bounds__(kRecThreads) void delta_recurrent_kernel(
    const InT* __restrict__ q, const InT* __restrict__ k, const InT* __restrict__ v,
    const float* __restrict__ beta, const float* s0, OutT* __restrict__ o, float* s_out,
    const int32_t* __restrict__ cu_seqlens, int pair0, int n_pairs, int ncg, int T, int H, int D,
    int l2norm, int vec, const float* __restrict__ gate) {
    using G = RecGeo<RPT, RS>;
    constexpr int CW = G::CW, DP = G::DP, SL = G::SL, DPL = G::DPL;
    constexpr int KB = kRecSteps, NT = kRecThreads;
    constexpr bool GATED = GM == 1, CHAN = GM == 2;
    constexpr int BUFX = G::BUF + (CHAN ? KB * DPL : 0);  // floats of one staging buffer
    constexpr int NG = KB * DP / 4;           // 4-element groups in a staged q or k block
    constexpr int NPF = (NG + NT - 1) / NT;   // groups per thread
    constexpr int NPV = KB * CW / NT;         // staged v elements per thread (16 / RS)
    static_assert(RPT % 4 == 0 && RS <= 16 && NPV * NT == KB * CW, "recurrent geometry");
    extern __shared__ float4 lds4[];
    float* const lds = reinterpret_cast<float*>(lds4);

    const int xs = blockIdx.x & 7, rest = blockIdx.x >> 3;
    const int c = rest % ncg;
    const int pair = pair0 + (rest / ncg) * 8 + xs;
    if (pair >= n_pairs) return;  // whole workgroup, before any barrier
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
    const int el = tid / RS, r = tid % RS;
    const int e = c * CW + el;
    const bool col_ok = e < D;
    const size_t sbase = static_cast<size_t>(pair) * D * D;

    float S[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
        const int d = r * RPT + i;
        S[i] = (s0 && col_ok && d < D) ? s0[sbase + static_cast<size_t>(d) * D + e] : 0.0f;
    }

    auto row = [&](int t) { return (static_cast<size_t>(tok0 + t) * H + h) * D; };

    // ---- prefetch registers for one block ----
    Raw4<InT> pk[NPF], pq[NPF];
    Raw4<float> pa[CHAN ? NPF : 1];
    InT pv[NPV];
    float pb = 0.f, pg = 0.f;
    auto prefetch = [&](int t0, int nst) {
#pragma unroll
        for (int s = 0; s < NPF; ++s) {
            const int grp = s * NT + tid;
            const int j = grp * 4 / DP, d = grp * 4 % DP;
            int n = 0;
            size_t a = 0;
            if (grp < NG && j < nst) {
                n = max(0, min(4, D - d));
                a = row(t0 + j) + d;
            }
            pk[s].load(k + a, n, vec);
            pq[s].load(q + a, n, vec);
            if constexpr (CHAN) pa[s].load(gate + a, n, vec);
        }
#pragma unroll
        for (int s = 0; s < NPV; ++s) {
            const int idx = s * NT + tid;
            const int j = idx / CW, e2 = c * CW + idx % CW;
            pv[s] = (j < nst && e2 < D) ? v[row(t0 + j) + e2] : InT(0);
        }
        if (tid < KB) {
            const size_t a = static_cast<size_t>(tok0 + t0 + tid) * H + h;
            pb = tid < nst ? (beta ? beta[a] : 1.f) : 0.f;
            if constexpr (GATED) pg = tid < nst ? gate[a] : 0.f;
        }
    };

    // ---- registers -> LDS buffer (q and k rows normalised first under l2norm) ----
    auto stage = [&](float* buf) {
        float* sk = buf;
        float* sq = sk + KB * DPL;
        float* sv = sq + KB * DPL;
        float* sc = sv + 2 * KB * CW;  // [KB] x {beta, q.k, alpha, 0}
#pragma unroll
        for (int s = 0; s < NPF; ++s) {
            const int grp = s * NT + tid;
            const int j = grp * 4 / DP, d = grp * 4 % DP;
            float xk[4], xq[4];
            pk[s].get(xk, vec);
            pq[s].get(xq, vec);
            if (l2norm) {
                // a row is DP / 4 adjacent lanes (DP / 4 divides 64)
                float ssk = 0.f, ssq = 0.f;
#pragma unroll
                for (int c2 = 0; c2 < 4; ++c2) {
                    ssk = fmaf(xk[c2], xk[c2], ssk);
                    ssq = fmaf(xq[c2], xq[c2], ssq);
                }
                ssk = lane_sum<DP / 4>(ssk);
                ssq = lane_sum<DP / 4>(ssq);
                const float dk = fmaxf(sqrtf(ssk), 1e-6f), dq = fmaxf(sqrtf(ssq), 1e-6f);
#pragma unroll
                for (int c2 = 0; c2 < 4; ++c2) {
                    xk[c2] = xk[c2] / dk;
                    xq[c2] = xq[c2] / dq;
                }
            }
            float qk = 0.f;
#pragma unroll
            for (int c2 = 0; c2 < 4; ++c2) qk = fmaf(xq[c2], xk[c2], qk);
            qk = lane_sum<DP / 4>(qk);
            if (grp < NG) {
                const int pos = j * DPL + (d / RPT) * SL + d % RPT;
                *reinterpret_cast<float4*>(sk + pos) = make_float4(xk[0], xk[1], xk[2], xk[3]);
                *reinterpret_cast<float4*>(sq + pos) = make_float4(xq[0], xq[1], xq[2], xq[3]);
                if constexpr (CHAN) {
                    float xa[4];
                    pa[s].get(xa, true);
                    // past the row end g = 0: alpha 1 on rows of S that stay zero
                    *reinterpret_cast<float4*>(buf + G::BUF + pos) =
                        make_float4(expf(xa[0]), expf(xa[1]), expf(xa[2]), expf(xa[3]));
                }
                if (d == 0) sc[4 * j + 1] = qk;
            }
        }
#pragma unroll
        for (int s = 0; s < NPV; ++s) sv[s * NT + tid] = to_f32(pv[s]);
        if (tid < KB) {
            sc[4 * tid] = pb;
            sc[4 * tid + 2] = GATED ? expf(pg) : 1.f;  // alpha: 1 past the sequence end
        }
    };

    // ---- the recurrence over one staged block ----
    auto tokens = [&](const float* buf, int nst) {
        const float* sk = buf;
        const float* sq = sk + KB * DPL;
        const float* sv = sq + KB * DPL;
        float* so = const_cast<float*>(sv) + KB * CW;
        const float4* sc = reinterpret_cast<const float4*>(so + KB * CW);
        auto body = [&](int j) {
            float kk[RPT], qq[RPT];
            const float4* kp = reinterpret_cast<const float4*>(sk + j * DPL + r * SL);
            const float4* qp = reinterpret_cast<const float4*>(sq + j * DPL + r * SL);
#pragma unroll
            for (int i = 0; i < RPT / 4; ++i) {
                const float4 t = kp[i], w = qp[i];
                kk[4 * i] = t.x, kk[4 * i + 1] = t.y, kk[4 * i + 2] = t.z, kk[4 * i + 3] = t.w;
                qq[4 * i] = w.x, qq[4 * i + 1] = w.y, qq[4 * i + 2] = w.z, qq[4 * i + 3] = w.w;
            }
            if constexpr (CHAN) {
                // decay each row by its channel's alpha first: S <- Diag(alpha) S
                const float4* ap = reinterpret_cast<const float4*>(buf + G::BUF + j * DPL + r * SL);
#pragma unroll
                for (int i = 0; i < RPT / 4; ++i) {
                    const float4 t = ap[i];
                    S[4 * i] *= t.x, S[4 * i + 1] *= t.y, S[4 * i + 2] *= t.z, S[4 * i + 3] *= t.w;
                }
            }
            float ks, qs;
            row_dot2<RPT>(kk, qq, S, ks, qs);
            col_sum2<RS>(ks, qs);
            const float4 cj = sc[j];  // beta, q.k, alpha
            const float vv = sv[j * CW + el];
            float os;
            if constexpr (GATED) {
                const float u = cj.x * (vv - cj.z * ks);
                os = fmaf(cj.y, u, cj.z * qs);
#pragma unroll
                for (int i = 0; i < RPT; ++i) S[i] = fmaf(kk[i], u, cj.z * S[i]);
            } else {
                const float u = cj.x * (vv - ks);
                os = fmaf(cj.y, u, qs);
#pragma unroll
                for (int i = 0; i < RPT; ++i) S[i] = fmaf(kk[i], u, S[i]);
            }
            so[j * CW + el] = os;  // the RS lanes of a column store the same bits
        };
        if (nst == KB) {
#pragma unroll
            for (int j = 0; j < KB; ++j) body(j);
        } else {
            for (int j = 0; j < nst; ++j) body(j);
        }
    };

    // ---- a block's outputs, from LDS, as row segments of CW columns ----
    auto store_o = [&](const float* buf, int t0, int nst) {
        const float* so = buf + 2 * KB * DPL + KB * CW;
#pragma unroll
        for (int s = 0; s < NPV; ++s) {
            const int idx = s * NT + tid;
            const int j = idx / CW, e2 = c * CW + idx % CW;
            if (j < nst && e2 < D) o[row(t0 + j) + e2] = from_f32<OutT>(so[idx]);
        }
    };

    const int nblk = (len + KB - 1) / KB;
    if (nblk > 0) prefetch(0, min(KB, len));
    for (int b = 0; b < nblk; ++b) {
        float* buf = lds + (b & 1) * BUFX;
        const int t0 = b * KB, nst = min(KB, len - t0);
        // buf was last read by block b - 2's token loop, before the previous barrier
        stage(buf);
        __syncthreads();
        if (b + 1 < nblk) prefetch(t0 + KB, min(KB, len - t0 - KB));
        if (b > 0) store_o(lds + ((b - 1) & 1) * BUFX, t0 - KB, KB);
        tokens(buf, nst);
    }
    if (nblk > 0) {
        __syncthreads();
        const int t0 = (nblk - 1) * KB;
        store_o(lds + ((nblk - 1) & 1) * BUFX, t0, len - t0);
    }

    if (col_ok) {
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
            const int d = r * RPT + i;
            if (d < D) s_out[sbase + static_cast<size_t>(d) * D + e] = S[i];
        }
    }
}

// Rows per thread and row slices per column for head dimension D: RPT 8 up to
// D = 128, 16 above; RS the smallest power of two with RS * RPT >= D (<= 16).
static void recurrent_geometry(int D, int* rpt, int* rs) {
    const int r = D <= 128 ? 8 : 16;
    int s = 1;
    while (r * s < D) s <<= 1;
    *rpt = r;
    *rs = s;
}

static bool is_aligned(const void* p, size_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

template <int RPT, int RS, int GM, typename InT, typename OutT>
static hipError_t launch_rec_t(const RecurrentArgs& a, hipStream_t st) {
    using G = RecGeo<RPT, RS>;
    auto kern = delta_recurrent_kernel<RPT, RS, GM, InT, OutT>;
    // the per-channel gate stages one more [kRecSteps][DPL] array per buffer
    constexpr size_t BYTES = G::BYTES + (GM == 2 ? 2 * sizeof(float) * kRecSteps * G::DPL : 0);
    if (BYTES > 64 * 1024) {
        // the dynamic-LDS limit is a per-device function attribute
        int dev = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e != hipSuccess) return e;
        static bool attr_set[64] = {};
        if (dev < 0 || dev >= 64 || !attr_set[dev]) {
            e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(BYTES));
            if (e != hipSuccess) return e;
            if (dev >= 0 && dev < 64) attr_set[dev] = true;
        }
    }
    const int ncg = (a.D + G::CW - 1) / G::CW;
    // 16-byte (fp32) or 8-byte (bf16) row loads when every q/k row group is aligned
    const size_t vb = sizeof(InT) * 4;
    const int vec = (a.D % 4 == 0) && is_aligned(a.q, vb) && is_aligned(a.k, vb) &&
                    (GM != 2 || is_aligned(a.gk, 16));
    // at most 2^22 workgroups (2^30 work-items) per launch
    const long per = ((1L << 22) / (8L * ncg)) * 8;
    for (long p0 = 0; p0 < a.n_pairs; p0 += per) {
        const long np = a.n_pairs - p0 < per ? a.n_pairs - p0 : per;
        const dim3 grid(static_cast<unsigned>((np + 7) / 8 * 8 * ncg));
        hipLaunchKernelGGL(kern, grid, dim3(kRecThreads), BYTES, st, static_cast<const InT*>(a.q),
                           static_cast<const InT*>(a.k), static_cast<const InT*>(a.v), a.beta, a.s0,
                           static_cast<OutT*>(a.o), a.s_out, a.cu_seqlens, static_cast<int>(p0), a.n_pairs,
                           ncg, a.T, a.H, a.D, a.l2norm ? 1 : 0, vec, GM == 2 ? a.gk : a.g);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

template <int RPT, int RS, typename InT, typename OutT>
static hipError_t launch_rec_g(const RecurrentArgs& a, hipStream_t st) {
    if (a.gk) return launch_rec_t<RPT, RS, 2, InT, OutT>(a, st);
    return a.g ? launch_rec_t<RPT, RS, 1, InT, OutT>(a, st) : launch_rec_t<RPT, RS, 0, InT, OutT>(a, st);
}

template <typename InT, typename OutT>
static hipError_t launch_rec_io(const RecurrentArgs& a, hipStream_t st) {
    int rpt, rs;
    recurrent_geometry(a.D, &rpt, &rs);
    if (rpt == 16) return launch_rec_g<16, 16, InT, OutT>(a, st);
    switch (rs) {
        case 1: return launch_rec_g<8, 1, InT, OutT>(a, st);
        case 2: return launch_rec_g<8, 2, InT, OutT>(a, st);
        case 4: return launch_rec_g<8, 4, InT, OutT>(a, st);
        case 8: return launch_rec_g<8, 8, InT, OutT>(a, st);
        default: return launch_rec_g<8, 16, InT, OutT>(a, st);
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
