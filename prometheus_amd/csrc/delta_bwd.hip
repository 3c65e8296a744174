// delta_bwd.hip — K5: reverse mode of the delta-rule recurrence, fp32.
//
// Gradients of the reference's backward (kernels/__init__.py:692-719 ->
// _delta_vjp_np :460-527 / _delta_vjp_jax :529-588) without its state
// history.  With u_t = v_t - S_{t-1}^T k_t (so S_t = S_{t-1} + beta_t k_t
// u_t^T) and the output gradient G (dL/dS, d_k x d_v), per token in reverse:
//
//   G += q_t go_t^T            w = G^T k_t           x = G u_t
//   gq_t = S_t go_t            gv_t = beta_t w       gbeta_t = k_t . x
//   S_{t-1} = S_t - beta_t k_t u_t^T                 y = S_{t-1} w
//   gk_t = beta_t (x - y)      G -= beta_t k_t w^T
//
// (the reference's g_A = G S_{t-1}^T enters only as g_A k = G (v - u) and
// g_A^T k = S_{t-1} w, which fold into x and y).  S is walked back within
// blocks of kCk tokens and restarted from a checkpoint at every block end,
// so the only memory beyond inputs and outputs is a workspace of u (T x D
// per sequence) and the checkpoints (ceil(T / kCk) x D x D).  Walking back
// subtracts terms of the size of S: where S grows (|1 - beta |k|^2| > 1,
// unnormalised keys) the fp32 error grows with the walk, so the walk is
// kept short: kCk = 8 holds the reference's own growing test case
// (tests/test_kernels.py:1537-1548) at 1e-6, where 16 reaches 3e-5.
//
// The recurrence is separable along the columns of S and G (d_v): a
// workgroup owns a tile of NC columns of one (b, h) (NC = min(D, 32) for
// D <= 128, 16 above), so B*H*ceil(D/NC) workgroups run (256 at cfg1
// instead of 64).  gv and gS0 are
// per column; gq, gk and gbeta sum over all columns (x, y and S go are row
// sums), so with several tiles each writes its partial sums and a final
// pass adds them (in a fixed order: results do not depend on scheduling).
//
// K5a (checkpoint pass) runs the forward recurrence in the per-token
// forward kernel's layout (column groups of 256 threads), writing u and the
// block-end states.  K5b (reverse pass) holds three fp32 matrices of the
// tile on chip: G by columns (thread (e, rc): rows rc*8.. of column e, for
// w = G^T k), G by rows and S by rows (thread (d, rr): tile columns rr*8..
// of row d, for x = G u, S go and S w); every product is a per-thread
// partial sum reduced over adjacent lanes with DPP.  w moves from the
// column to the row layout through LDS: one LDS-only barrier per token,
// after which the next token's operands are read.  A checkpoint block's
// inputs (k, q, go, u, beta and the checkpoint) are loaded into registers
// one block ahead and staged into double-buffered LDS (slices at a stride
// of kRpt + 4 floats: 16-byte reads in distinct banks); the block's outputs
// collect in LDS and go out coalesced at the next block, before that
// block's loads, so that waiting for loads never waits for stores.

#include "pm_common.h"
#include "pm_internal.h"
#include "pm_rec.h"

namespace pm {

constexpr int kBwdSteps = 8;  // tokens staged in LDS at a time
constexpr int kCk = 8;        // tokens between state checkpoints (multiple of kBwdSteps)
constexpr int kRpt = 8;       // elements of a row or column slice per thread
constexpr int kTileCols = 32; // columns per workgroup when 32 < D <= 128
constexpr int kTileColsWide = 16;  // ... when D > 128 (512 threads: 32 row slices x 16 columns)
static_assert(kCk == kBwdSteps, "the reverse pass stages one checkpoint block at a time");

// Workgroup barrier for LDS traffic only: global stores still in flight are not
// waited for (no other thread reads them).
__device__ __forceinline__ void lds_sync() { __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

struct BwdGeo {
    int nc, n_tiles;  // tile columns, tiles per (b, h)
    int rsc, rsr;     // row slices per column (column layout), column slices per row (row layout)
    int threads;
};
static int pow2_at_least(int x) {
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}
static BwdGeo bwd_geo(int D) {
    BwdGeo g;
    g.nc = D <= kTileCols ? D : (D <= 128 ? kTileCols : kTileColsWide);
    g.n_tiles = (D + g.nc - 1) / g.nc;
    g.rsc = pow2_at_least((D + kRpt - 1) / kRpt);
    g.rsr = pow2_at_least((g.nc + kRpt - 1) / kRpt);
    const int t = max(g.nc * g.rsc, D * g.rsr);
    g.threads = ((t + 63) / 64) * 64;
    return g;
}

// ---------------- K5a: forward pass writing u and block-end states ----------------
// The forward recurrence in the per-token forward kernel's layout (256 threads per
// group of CW = 256 / RS columns, thread (el, r) holding rows [r*RPT, r*RPT + RPT)
// of its column, DPP column sums, tokens staged 16 at a time with the next block's
// loads in flight), writing u_t = v_t - S_{t-1}^T k_t per token (through LDS, one
// block later) and S after every kCk-th token and after the last.
// GM: 0 ungated, 1 a log-gate per (token, head), 2 one per (token, head, key channel),
// where P = Diag(alpha) S: each thread decays its rows before the token's dot product.
template <int RPT, int RS, typename InT, int GM>
__global__ __launch_bounds__(kRecThreads) void delta_bwd_ckpt_kernel(
    const InT* __restrict__ k, const InT* __restrict__ v, const float* __restrict__ beta,
    const float* __restrict__ gate, const float* __restrict__ s0, float* __restrict__ u_ws,
    float* __restrict__ ck_ws, int pair0, int n_pairs, int ncg, int T, int H, int D, int vec) {
    using G = RecGeo<RPT, RS>;
    constexpr int CW = G::CW, DP = G::DP, SL = G::SL, DPL = G::DPL;
    constexpr int KB = kRecSteps, NT = kRecThreads;
    constexpr int NG = KB * DP / 4, NPF = (NG + NT - 1) / NT, NPV = KB * CW / NT;
    constexpr bool GATED = GM == 1, CHAN = GM == 2;
    // k rows, v, u, beta (and alpha), then (CHAN) the alpha rows in the k rows' layout
    constexpr int BUF0 = KB * DPL + 2 * KB * CW + 4 * KB;
    constexpr int BUF = BUF0 + (CHAN ? KB * DPL : 0);
    static_assert(KB % kCk == 0, "checkpoints fall inside a staged block");
    extern __shared__ float4 lds4[];
    float* const lds = reinterpret_cast<float*>(lds4);

    const int xs = blockIdx.x & 7, rest = blockIdx.x >> 3;
    const int c = rest % ncg;
    const int pair = pair0 + (rest / ncg) * 8 + xs;
    if (pair >= n_pairs) return;  // whole workgroup, before any barrier
    const int seq = pair / H, h = pair % H;
    const long tok0 = static_cast<long>(seq) * T;
    const int tid = threadIdx.x;
    const int el = tid / RS, r = tid % RS;
    const int e = c * CW + el;
    const bool col_ok = e < D;
    const size_t sbase = static_cast<size_t>(pair) * D * D;
    const int n_ck = (T + kCk - 1) / kCk;
    float* u_p = u_ws + static_cast<size_t>(pair) * T * D;
    float* ck_p = ck_ws + static_cast<size_t>(pair) * n_ck * D * D;

    float S[RPT];  // S[r*RPT + i][e]
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
        const int d = r * RPT + i;
        S[i] = (s0 && col_ok && d < D) ? s0[sbase + static_cast<size_t>(d) * D + e] : 0.f;
    }
    auto row = [&](int t) { return (static_cast<size_t>(tok0 + t) * H + h) * D; };

    Raw4<InT> pk[NPF];
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
            if constexpr (CHAN) pa[s].load(gate + a, n, vec);
        }
#pragma unroll
        for (int s = 0; s < NPV; ++s) {
            const int idx = s * NT + tid;
            const int j = idx / CW, e2 = c * CW + idx % CW;
            pv[s] = (j < nst && e2 < D) ? v[row(t0 + j) + e2] : InT(0);
        }
        if (tid < KB) pb = tid < nst ? beta[static_cast<size_t>(tok0 + t0 + tid) * H + h] : 0.f;
        if (GATED && tid < KB) pg = tid < nst ? gate[static_cast<size_t>(tok0 + t0 + tid) * H + h] : 0.f;
    };
    auto stage = [&](float* buf) {
        float* sk = buf;
        float* sv = sk + KB * DPL;
        float* sb = sv + 2 * KB * CW;  // beta, then (GATED) alpha = exp(g)
#pragma unroll
        for (int s = 0; s < NPF; ++s) {
            const int grp = s * NT + tid;
            const int j = grp * 4 / DP, d = grp * 4 % DP;
            float xk[4];
            pk[s].get(xk, vec);
            if (grp < NG) {
                const int pos = j * DPL + (d / RPT) * SL + d % RPT;
                *reinterpret_cast<float4*>(sk + pos) = make_float4(xk[0], xk[1], xk[2], xk[3]);
                if constexpr (CHAN) {
                    float xa[4];
                    pa[s].get(xa, true);
                    *reinterpret_cast<float4*>(buf + BUF0 + pos) =
                        make_float4(expf(xa[0]), expf(xa[1]), expf(xa[2]), expf(xa[3]));
                }
            }
        }
#pragma unroll
        for (int s = 0; s < NPV; ++s) sv[s * NT + tid] = to_f32(pv[s]);
        if (tid < KB) sb[tid] = pb;
        if (GATED && tid < KB) sb[KB + tid] = expf(pg);
    };
    auto checkpoint = [&](int t) {
        float* cp = ck_p + static_cast<size_t>(t / kCk) * D * D;
        if (col_ok) {
#pragma unroll
            for (int i = 0; i < RPT; ++i) {
                const int d = r * RPT + i;
                if (d < D) cp[static_cast<size_t>(d) * D + e] = S[i];
            }
        }
    };
    auto tokens = [&](float* buf, int t0, int nst, int len) {
        const float* sk = buf;
        const float* sv = sk + KB * DPL;
        float* su = buf + KB * DPL + KB * CW;
        const float* sb = su + KB * CW;
        auto body = [&](int j) {
            float kk[RPT];
            const float4* kp = reinterpret_cast<const float4*>(sk + j * DPL + r * SL);
#pragma unroll
            for (int i = 0; i < RPT / 4; ++i) {
                const float4 t = kp[i];
                kk[4 * i] = t.x, kk[4 * i + 1] = t.y, kk[4 * i + 2] = t.z, kk[4 * i + 3] = t.w;
            }
            if constexpr (CHAN) {
                // P = Diag(alpha) S, row by row
                const float4* ap = reinterpret_cast<const float4*>(buf + BUF0 + j * DPL + r * SL);
#pragma unroll
                for (int i = 0; i < RPT / 4; ++i) {
                    const float4 t = ap[i];
                    S[4 * i] *= t.x, S[4 * i + 1] *= t.y, S[4 * i + 2] *= t.z, S[4 * i + 3] *= t.w;
                }
            }
            const float ks = col_sum<RS>(row_dot<RPT>(kk, S));
            // GATED: the decayed state P = alpha S enters both the prediction and the update
            const float a = GATED ? sb[KB + j] : 1.f;
            const float u = sv[j * CW + el] - (GATED ? a * ks : ks);
            su[j * CW + el] = u;  // the RS lanes of a column store the same bits
            const float bu = sb[j] * u;
#pragma unroll
            for (int i = 0; i < RPT; ++i) S[i] = fmaf(kk[i], bu, GATED ? a * S[i] : S[i]);
            // t0 is a multiple of kCk
            if ((j + 1) % kCk == 0 || t0 + j + 1 == len) checkpoint(t0 + j);
        };
        if (nst == KB) {
#pragma unroll
            for (int j = 0; j < KB; ++j) body(j);
        } else {
            for (int j = 0; j < nst; ++j) body(j);
        }
    };
    auto store_u = [&](const float* buf, int t0, int nst) {
        const float* su = buf + KB * DPL + KB * CW;
#pragma unroll
        for (int s = 0; s < NPV; ++s) {
            const int idx = s * NT + tid;
            const int j = idx / CW, e2 = c * CW + idx % CW;
            if (j < nst && e2 < D) u_p[static_cast<size_t>(t0 + j) * D + e2] = su[idx];
        }
    };

    const int len = T;
    const int nblk = (len + KB - 1) / KB;
    if (nblk > 0) prefetch(0, min(KB, len));
    for (int b = 0; b < nblk; ++b) {
        float* buf = lds + (b & 1) * BUF;
        const int t0 = b * KB, nst = min(KB, len - t0);
        stage(buf);
        __syncthreads();
        if (b + 1 < nblk) prefetch(t0 + KB, min(KB, len - t0 - KB));
        if (b > 0) store_u(lds + ((b - 1) & 1) * BUF, t0 - KB, KB);
        tokens(buf, t0, nst, len);
    }
    if (nblk > 0) {
        __syncthreads();
        const int t0 = (nblk - 1) * KB;
        store_u(lds + ((nblk - 1) & 1) * BUF, t0, len - t0);
    }
}

template <int RPT, int RS, typename InT, int GM>
static hipError_t launch_ckpt_t(const BwdArgs& a, float* u_ws, float* ck_ws, hipStream_t st) {
    using G = RecGeo<RPT, RS>;
    constexpr size_t kBytes = 2 * sizeof(float) * ((GM == 2 ? 2 : 1) * kRecSteps * G::DPL +
                                                   2 * kRecSteps * G::CW + 4 * kRecSteps);
    auto kern = delta_bwd_ckpt_kernel<RPT, RS, InT, GM>;
    if (kBytes > 64 * 1024) {
        // the dynamic-LDS limit is a per-device function attribute
        int dev = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e != hipSuccess) return e;
        static bool attr_set[64] = {};
        if (dev < 0 || dev >= 64 || !attr_set[dev]) {
            e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kBytes));
            if (e != hipSuccess) return e;
            if (dev >= 0 && dev < 64) attr_set[dev] = true;
        }
    }
    const int ncg = (a.D + G::CW - 1) / G::CW;
    const size_t vb = sizeof(InT) * 4;
    const int vec = (a.D % 4 == 0) && reinterpret_cast<uintptr_t>(a.k) % vb == 0 &&
                    (GM != 2 || reinterpret_cast<uintptr_t>(a.g) % 16 == 0);
    // at most 2^22 workgroups (2^30 work-items) per launch
    const long per = ((1L << 22) / (8L * ncg)) * 8;
    for (long p0 = 0; p0 < a.n_pairs; p0 += per) {
        const long np = a.n_pairs - p0 < per ? a.n_pairs - p0 : per;
        const dim3 grid(static_cast<unsigned>((np + 7) / 8 * 8 * ncg));
        hipLaunchKernelGGL(kern, grid, dim3(kRecThreads), kBytes, st, static_cast<const InT*>(a.k),
                           static_cast<const InT*>(a.v), a.beta, a.g, a.s0, u_ws, ck_ws, static_cast<int>(p0),
                           a.n_pairs, ncg, a.T, a.H, a.D, vec);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// RPT 8 and RS the smallest power of two with 8 RS >= D for D <= 128; RPT 16 and RS 16
// above (the per-token forward's geometry).
template <typename InT, int GM>
static hipError_t launch_ckpt(const BwdArgs& a, float* u_ws, float* ck_ws, hipStream_t st) {
    if (a.D > 128) return launch_ckpt_t<16, 16, InT, GM>(a, u_ws, ck_ws, st);
    int rs = 1;
    while (8 * rs < a.D) rs <<= 1;
    switch (rs) {
        case 1: return launch_ckpt_t<8, 1, InT, GM>(a, u_ws, ck_ws, st);
        case 2: return launch_ckpt_t<8, 2, InT, GM>(a, u_ws, ck_ws, st);
        case 4: return launch_ckpt_t<8, 4, InT, GM>(a, u_ws, ck_ws, st);
        case 8: return launch_ckpt_t<8, 8, InT, GM>(a, u_ws, ck_ws, st);
        default: return launch_ckpt_t<8, 16, InT, GM>(a, u_ws, ck_ws, st);
    }
}

// LDS layout of K5b's staged vectors: slice i of kRpt elements starts at i * kSl, so
// slices are 16-byte aligned and the slices read by one wave start in different banks.
constexpr int kSl = kRpt + 4;
__device__ __forceinline__ int spad(int x) { return (x / kRpt) * kSl + x % kRpt; }
__device__ __forceinline__ void load_slice(const float* p, float (&x)[kRpt]) {
    const float4* p4 = reinterpret_cast<const float4*>(p);
#pragma unroll
    for (int i = 0; i < kRpt / 4; ++i) {
        const float4 t = p4[i];
        x[4 * i] = t.x, x[4 * i + 1] = t.y, x[4 * i + 2] = t.z, x[4 * i + 3] = t.w;
    }
}
// Dot product of two register slices, one accumulator (see row_dot).
__device__ __forceinline__ float slice_dot(const float (&a)[kRpt], const float (&b)[kRpt]) { return row_dot<kRpt>(a, b); }

// ---------------- K5b: reverse pass over one column tile ----------------
// gq/gk/gb receive this tile's sums over its columns: the outputs themselves
// when n_tiles == 1, else this tile's slot of the partial-sum buffers.
// RSC row slices per column (column layout), RSR column slices per row (row layout), NCT
// the tile width the geometry is sized for (the fewest threads a launch has is NCT RSC).
//
// GATED (log-gates g, alpha = exp(g)): with P_t = alpha_t S_{t-1} the step is
// S_t = P_t + beta_t k_t u_t^T, and per token in reverse
//   y = P_t w,   dL/dg_t = <G_P, P_t> with G_P = G - beta_t k_t w^T,   G <- alpha_t G_P.
// Walking S back would divide by alpha (unbounded error for strong decay), so each
// checkpoint block is first recomputed forward from its start state (the previous
// block's end, or S0), its states before every token kept in registers, and the
// reverse walk reads them.
//
// GM = 2 (a log-gate per key channel, P_t = Diag(alpha_t) S_{t-1}): the same walk with
// row d scaled by alpha_t[d]: y_d = alpha_t[d] (S_{t-1} w)_d, dL/dg_t[d] = alpha_t[d]
// <G_P[d, :], S_{t-1}[d, :]> (a per-row output like gk, no sum over d), and
// G <- Diag(alpha_t) G_P (the column layout scales each of its rows by its own alpha).
template <typename InT, int RSC, int RSR, int NCT, int GM>
__global__ __launch_bounds__(512) void delta_bwd_kernel(
    const InT* __restrict__ q, const InT* __restrict__ k, const float* __restrict__ beta,
    const float* __restrict__ gate, const float* __restrict__ s0,
    const float* __restrict__ go, const float* __restrict__ gs, const float* __restrict__ u_ws,
    const float* __restrict__ ck_ws, float* __restrict__ gq, float* __restrict__ gk,
    float* __restrict__ gv, float* __restrict__ gb, float* __restrict__ gg, float* __restrict__ gs0,
    int T, int H, int D, int NC, int n_tiles, size_t part_stride_e, size_t part_stride_b) {
    extern __shared__ float lds[];
    constexpr int DP = RSC * kRpt;   // padded rows (column layout)
    constexpr int CP = RSR * kRpt;   // padded tile columns (row layout)
    constexpr int DPL = RSC * kSl;   // their LDS strides (spad positions)
    constexpr int CPL = RSR * kSl;
    constexpr int KB = kBwdSteps;
    // per-thread staging slots, for the fewest threads a launch of this geometry has
    constexpr int NTMIN = NCT * RSC < 64 ? 64 : NCT * RSC;
    constexpr int MK = (KB * DP + NTMIN - 1) / NTMIN, MG = (KB * CP + NTMIN - 1) / NTMIN;
    constexpr bool GATED = GM != 0, CHAN = GM == 2;  // GATED: any decay
    // one staging buffer: k, q, go, u, beta and alpha, then (CHAN) the alpha rows
    constexpr int SB0 = 2 * KB * DPL + 2 * KB * CPL + 2 * KB;
    constexpr int SB = SB0 + (CHAN ? KB * DPL : 0);
    const int NT = blockDim.x, NWV = NT / 64;
    // outputs of a block, written out one block later: by block parity,
    // [KB][D] gbeta terms k[d] x[d], [KB][D] gq, [KB][D] gk, [KB][NC] gv
    // (GATED: then [KB][D] gate terms, summed over d when written out)
    const int OB = (GATED ? 4 : 3) * KB * D + KB * NC;
    float* sw = lds + 2 * SB;           // [2][CPL]       w, by token parity
    float* so0 = sw + 2 * CPL;          // [2][OB]

    const int tile = blockIdx.x % n_tiles, pair = blockIdx.x / n_tiles, col0 = tile * NC;
    const int seq = pair / H, h = pair % H;
    const long tok0 = static_cast<long>(seq) * T;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    // column layout: tile column e, rows rc*kRpt..; row layout: row d, tile columns rr*kRpt..
    const int e = tid / RSC, rc = tid % RSC;
    const int d = tid / RSR, rr = tid % RSR;
    const bool ok_c = e < NC && col0 + e < D;
    const bool ok_r = d < D;
    const size_t sbase = static_cast<size_t>(pair) * D * D;
    const int n_ck = (T + kCk - 1) / kCk;
    const float* u_p = u_ws + static_cast<size_t>(pair) * T * D;
    const float* ck_p = ck_ws + static_cast<size_t>(pair) * n_ck * D * D;
    float* gq_t = gq + tile * part_stride_e;
    float* gk_t = gk + tile * part_stride_e;
    float* gb_t = gb + tile * part_stride_b;
    float* gg_t = GATED ? gg + tile * (CHAN ? part_stride_e : part_stride_b) : nullptr;

    // w's padding entries (tile columns past NC or D) are read as zeros, never written
    for (int x = tid; x < 2 * CPL; x += NT) sw[x] = 0.f;

    float Gc[kRpt], Gr[kRpt], Sr[kRpt];  // G[rc*R+i][col0+e], G[d][col0+rr*R+i], S[d][col0+rr*R+i]
#pragma unroll
    for (int i = 0; i < kRpt; ++i) {
        const int row = rc * kRpt + i, c = rr * kRpt + i;
        Gc[i] = (gs && ok_c && row < D) ? gs[sbase + static_cast<size_t>(row) * D + col0 + e] : 0.f;
        Gr[i] = (gs && ok_r && c < NC && col0 + c < D)
                    ? gs[sbase + static_cast<size_t>(d) * D + col0 + c] : 0.f;
    }

    // ---- one checkpoint block's inputs, loaded a block ahead into registers ----
    InT pk[MK], pq[MK];
    float pg[MG], pu[MG], ps[kRpt], pb = 0.f, pa = 0.f, pac[CHAN ? MK : 1];
    auto prefetch = [&](int blk) {
        const int lo = blk * kCk, nst = min(T, lo + kCk) - lo;
#pragma unroll
        for (int s = 0; s < MK; ++s) {
            const int idx = s * NT + tid;
            const int j = idx / DP, x = idx % DP;
            const bool ok = idx < KB * DP && j < nst && x < D;
            const size_t a = ok ? (static_cast<size_t>(tok0 + lo + j) * H + h) * D + x : 0;
            pk[s] = ok ? k[a] : InT(0);
            pq[s] = ok ? q[a] : InT(0);
            if constexpr (CHAN) pac[s] = ok ? gate[a] : 0.f;
        }
#pragma unroll
        for (int s = 0; s < MG; ++s) {
            const int idx = s * NT + tid;
            const int j = idx / CP, c = idx % CP;
            const bool ok = idx < KB * CP && j < nst && c < NC && col0 + c < D;
            pg[s] = (ok && go) ? go[(static_cast<size_t>(tok0 + lo + j) * H + h) * D + col0 + c] : 0.f;
            pu[s] = ok ? u_p[static_cast<size_t>(lo + j) * D + col0 + c] : 0.f;
        }
        if (tid < KB) pb = tid < nst ? beta[static_cast<size_t>(tok0 + lo + tid) * H + h] : 0.f;
        if (GM == 1 && tid < KB) pa = tid < nst ? gate[static_cast<size_t>(tok0 + lo + tid) * H + h] : 0.f;
        // the block's end state, walked back (GATED: its start state, recomputed forward)
        const float* cp = !GATED      ? ck_p + static_cast<size_t>(blk) * D * D
                          : blk > 0   ? ck_p + static_cast<size_t>(blk - 1) * D * D
                          : s0        ? s0 + sbase
                                      : nullptr;
#pragma unroll
        for (int i = 0; i < kRpt; ++i) {
            const int c = rr * kRpt + i;
            ps[i] = (cp && ok_r && c < NC && col0 + c < D) ? cp[static_cast<size_t>(d) * D + col0 + c] : 0.f;
        }
    };
    auto stage = [&](float* buf) {
        float* sk = buf;
        float* sq = sk + KB * DPL;
        float* sg = sq + KB * DPL;
        float* su = sg + KB * CPL;
        float* sb = su + KB * CPL;
#pragma unroll
        for (int s = 0; s < MK; ++s) {
            const int idx = s * NT + tid;
            if (idx < KB * DP) {
                const int pos = (idx / DP) * DPL + spad(idx % DP);
                sk[pos] = to_f32(pk[s]);
                sq[pos] = to_f32(pq[s]);
                if constexpr (CHAN) buf[SB0 + pos] = expf(pac[s]);  // 1 past the row or block
            }
        }
#pragma unroll
        for (int s = 0; s < MG; ++s) {
            const int idx = s * NT + tid;
            if (idx < KB * CP) {
                const int pos = (idx / CP) * CPL + spad(idx % CP);
                sg[pos] = pg[s];
                su[pos] = pu[s];
            }
        }
        if (tid < KB) sb[tid] = pb;
        if (GM == 1 && tid < KB) sb[KB + tid] = expf(pa);
#pragma unroll
        for (int i = 0; i < kRpt; ++i) Sr[i] = ps[i];
    };
    // a block's outputs: gq, gk and gv rows, and gbeta (one wave per token)
    auto flush_out = [&](const float* so, int lo, int nst) {
        const float* soq = so + KB * D;
        const float* sok = soq + KB * D;
        const float* sov = sok + KB * D;
        [[maybe_unused]] const float* sog = sok + KB * D + KB * NC;  // GATED: the gate terms
        for (int idx = tid; idx < nst * D; idx += NT) {
            const int j = idx / D, x = idx % D;
            const size_t a = (static_cast<size_t>(tok0 + lo + j) * H + h) * D + x;
            gq_t[a] = soq[idx];
            gk_t[a] = sok[idx];
            if constexpr (CHAN) gg_t[a] = sog[idx];
        }
        for (int idx = tid; idx < nst * NC; idx += NT) {
            const int j = idx / NC, c = idx % NC;
            if (col0 + c < D) gv[(static_cast<size_t>(tok0 + lo + j) * H + h) * D + col0 + c] = sov[idx];
        }
        for (int j = wave; j < nst; j += NWV) {
            float sum = 0.f;
            for (int x = lane; x < D; x += 64) sum += so[j * D + x];
            sum = wave_sum_row3(sum);
            if (lane == 63) gb_t[static_cast<size_t>(tok0 + lo + j) * H + h] = sum;
        }
        if constexpr (GM == 1) {
            for (int j = wave; j < nst; j += NWV) {
                float sum = 0.f;
                for (int x = lane; x < D; x += 64) sum += sog[j * D + x];
                sum = wave_sum_row3(sum);
                if (lane == 63) gg_t[static_cast<size_t>(tok0 + lo + j) * H + h] = sum;
            }
        }
    };

    if (n_ck > 0) prefetch(n_ck - 1);
    for (int blk = n_ck - 1, it = 0; blk >= 0; --blk, ++it) {
        float* buf = lds + (it & 1) * SB;
        const int lo = blk * kCk, nst = min(T, lo + kCk) - lo;
        // buf was last read by the token loop two blocks back, before the previous barrier
        stage(buf);
        __syncthreads();
        // the previous block's stores go out before this block's loads, so that waiting
        // for the loads never waits for stores issued after them
        if (it > 0) flush_out(so0 + ((it - 1) & 1) * OB, lo + kCk, min(T, lo + 2 * kCk) - lo - kCk);
        if (blk > 0) prefetch(blk - 1);
        const float* sk = buf;
        const float* sq = sk + KB * DPL;
        const float* sg = sq + KB * DPL;
        const float* su = sg + KB * CPL;
        const float* sb = su + KB * CPL;
        float* sgb = so0 + (it & 1) * OB;  // gbeta terms, then gq, gk, gv (GATED: gate terms)
        float* soq = sgb + KB * D;
        float* sok = soq + KB * D;
        float* sov = sok + KB * D;
        float* sog = sov + KB * NC;
        // CHAN: alpha of token j for row d (row layout)
        const float* sar = buf + SB0;
        auto alpha_row = [&](int j) { return CHAN ? (ok_r ? sar[j * DPL + spad(d)] : 1.f) : sb[KB + j]; };
        // GATED: the block recomputed forward from its start state; Sh[j] = S before token lo + j
        float Sh[GATED ? KB : 1][kRpt];
        if constexpr (GATED) {
#pragma unroll
            for (int j = 0; j < KB; ++j) {
                if (j < nst) {
                    float ur[kRpt];
                    load_slice(su + j * CPL + rr * kSl, ur);
                    const float a = alpha_row(j), bkd = sb[j] * (ok_r ? sk[j * DPL + spad(d)] : 0.f);
#pragma unroll
                    for (int i = 0; i < kRpt; ++i) {
                        Sh[j][i] = Sr[i];
                        Sr[i] = fmaf(bkd, ur[i], a * Sr[i]);
                    }
                }
            }
        }
        {
            // a token's operands; the next token's are loaded while this one finishes
            float b, ge, kd, qd, kc[kRpt], qc[kRpt], gr[kRpt], ur[kRpt];
            auto load_tok = [&](int j) {
                b = sb[j];
                load_slice(sk + j * DPL + rc * kSl, kc);  // k[rc*R + i]      (column layout)
                load_slice(sq + j * DPL + rc * kSl, qc);  // q[rc*R + i]
                load_slice(sg + j * CPL + rr * kSl, gr);  // go[col0 + rr*R + i] (row layout)
                load_slice(su + j * CPL + rr * kSl, ur);  // u[col0 + rr*R + i]
                ge = ok_c ? sg[j * CPL + spad(e)] : 0.f;  // go[col0 + e]
                kd = ok_r ? sk[j * DPL + spad(d)] : 0.f;  // k[d]
                qd = ok_r ? sq[j * DPL + spad(d)] : 0.f;  // q[d]
            };
            if (nst > 0) load_tok(nst - 1);
            auto step = [&](int j) __attribute__((always_inline)) {
                const int t = lo + j;
                // G += q go^T (both layouts); S_t go over the tile's columns (row layout)
#pragma unroll
                for (int i = 0; i < kRpt; ++i) {
                    Gc[i] = fmaf(qc[i], ge, Gc[i]);
                    Gr[i] = fmaf(qd, gr[i], Gr[i]);
                }
                float gqp = slice_dot(gr, Sr);
                // w = G^T k (column layout), x = G u over the tile's columns (row layout)
                float wp = slice_dot(kc, Gc);
                float xp = slice_dot(ur, Gr);
                wp = lane_sum<RSC>(wp);
                gqp = col_sum<RSR>(gqp);
                xp = col_sum<RSR>(xp);
                float* swp = sw + (t & 1) * CPL;
                if (rc == 0 && ok_c) {
                    swp[spad(e)] = wp;
                    sov[j * NC + e] = b * wp;
                }
                if (rr == 0 && ok_r) soq[j * D + d] = gqp;
                // S_{t-1} = S_t - b k u^T (row layout); GATED: the recomputed S_{t-1}
                const float bkd = b * kd;
                const float at = GATED ? alpha_row(j) : 1.f;
#pragma unroll
                for (int i = 0; i < kRpt; ++i) Sr[i] = GATED ? Sh[GATED ? j : 0][i] : fmaf(-bkd, ur[i], Sr[i]);
                // what the rest of this token needs from its operands
                const float bt = b, kdt = kd;
                float bk[kRpt];
#pragma unroll
                for (int i = 0; i < kRpt; ++i) bk[i] = -b * kc[i];
                lds_sync();  // w visible to the row layout
                float wr[kRpt];
                load_slice(swp + rr * kSl, wr);  // w[col0 + rr*R + i]
                if (j > 0) load_tok(j - 1);
                // y = P w with P = alpha S_{t-1}
                const float yp = (GATED ? at : 1.f) * col_sum<RSR>(slice_dot(wr, Sr));
                if (rr == 0 && ok_r) {
                    sok[j * D + d] = bt * (xp - yp);
                    sgb[j * D + d] = kdt * xp;  // gbeta = k . x, summed when written out
                }
                // G -= b k w^T (both layouts)
#pragma unroll
                for (int i = 0; i < kRpt; ++i) {
                    Gc[i] = fmaf(bk[i], wp, Gc[i]);
                    Gr[i] = fmaf(-bkd, wr[i], Gr[i]);
                }
                if constexpr (GATED) {
                    // dL/dg_t = <G_P, alpha S_{t-1}> (row d's share; summed over d when written
                    // out), then G <- alpha G_P
                    const float gp = col_sum<RSR>(slice_dot(Gr, Sr));
                    if (rr == 0 && ok_r) sog[j * D + d] = at * gp;
                    if constexpr (CHAN) {
                        float ac[kRpt];
                        load_slice(sar + j * DPL + rc * kSl, ac);  // alpha[rc*R + i]
#pragma unroll
                        for (int i = 0; i < kRpt; ++i) {
                            Gc[i] *= ac[i];
                            Gr[i] *= at;
                        }
                    } else {
#pragma unroll
                        for (int i = 0; i < kRpt; ++i) {
                            Gc[i] *= at;
                            Gr[i] *= at;
                        }
                    }
                }
            };
            if constexpr (GATED) {
                // unrolled, so that the recomputed states Sh[j] stay in registers
#pragma unroll
                for (int j = KB - 1; j >= 0; --j)
                    if (j < nst) step(j);
            } else {
                for (int j = nst - 1; j >= 0; --j) step(j);
            }
        }
    }
    if (n_ck > 0) {
        __syncthreads();
        flush_out(so0 + ((n_ck - 1) & 1) * OB, 0, min(T, kCk));
    }
    if (ok_c) {
#pragma unroll
        for (int i = 0; i < kRpt; ++i) {
            const int row = rc * kRpt + i;
            if (row < D) gs0[sbase + static_cast<size_t>(row) * D + col0 + e] = Gc[i];
        }
    }
}

// out[i] = sum over tiles of part[tile * stride + i], tiles in order
__global__ void bwd_reduce_kernel(float* __restrict__ out, const float* __restrict__ part,
                                  size_t n, size_t stride, int n_tiles) {
    size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t step = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (; i < n; i += step) {
        float s = part[i];
        for (int t = 1; t < n_tiles; ++t) s += part[t * stride + i];
        out[i] = s;
    }
}

// The same sum four floats at a time (n4 = n / 4 groups, stride4 = stride / 4).
__global__ void bwd_reduce4_kernel(float4* __restrict__ out, const float4* __restrict__ part, size_t n4,
                                   size_t stride4, int n_tiles) {
    size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t step = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (; i < n4; i += step) {
        float4 s = part[i];
        for (int t = 1; t < n_tiles; ++t) {
            const float4 x = part[t * stride4 + i];
            s.x += x.x, s.y += x.y, s.z += x.z, s.w += x.w;
        }
        out[i] = s;
    }
}

static hipError_t launch_reduce(float* out, const float* part, size_t n, size_t stride, int n_tiles,
                                hipStream_t st) {
    if (n == 0) return hipSuccess;
    const bool vec = n % 4 == 0 && stride % 4 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(part) % 16 == 0;
    const size_t m = vec ? n / 4 : n;
    size_t g = (m + 255) / 256;
    if (g > 65536) g = 65536;
    if (vec) {
        hipLaunchKernelGGL(bwd_reduce4_kernel, dim3(static_cast<unsigned>(g)), dim3(256), 0, st,
                           reinterpret_cast<float4*>(out), reinterpret_cast<const float4*>(part), m, stride / 4,
                           n_tiles);
    } else {
        hipLaunchKernelGGL(bwd_reduce_kernel, dim3(static_cast<unsigned>(g)), dim3(256), 0, st, out, part, n,
                           stride, n_tiles);
    }
    return hipGetLastError();
}

size_t bwd_workspace_floats(long n_pairs, int T, int D, int gm) {
    const BwdGeo g = bwd_geo(D);
    const long n_ck = (T + kCk - 1) / kCk;
    const size_t e = static_cast<size_t>(n_pairs) * T * D, bt = static_cast<size_t>(n_pairs) * T;
    size_t f = e + static_cast<size_t>(n_pairs) * n_ck * D * D;
    // per tile: gq and gk partial sums, gbeta's, and gg's (per token, or per channel)
    if (g.n_tiles > 1) f += static_cast<size_t>(g.n_tiles) * (2 * e + bt + (gm == 1 ? bt : gm == 2 ? e : 0));
    return f;
}

template <typename InT, int GM>
static hipError_t launch_bwd_in(const BwdArgs& a, hipStream_t st) {
    constexpr bool GATED = GM != 0;
    const BwdGeo g = bwd_geo(a.D);
    const size_t e = static_cast<size_t>(a.n_pairs) * a.T * a.D;
    const size_t bt = static_cast<size_t>(a.n_pairs) * a.T;
    const long n_ck = (a.T + kCk - 1) / kCk;
    float* u_ws = a.workspace;
    float* ck_ws = u_ws + e;
    float* part = ck_ws + static_cast<size_t>(a.n_pairs) * n_ck * a.D * a.D;
    const unsigned grid = static_cast<unsigned>(a.n_pairs) * g.n_tiles;

    hipError_t err = launch_ckpt<InT, GM>(a, u_ws, ck_ws, st);
    if (err != hipSuccess) return err;

    const bool split = g.n_tiles > 1;
    float* gq = split ? part : a.gq;
    float* gk = split ? part + static_cast<size_t>(g.n_tiles) * e : a.gk;
    float* gb = split ? part + static_cast<size_t>(2 * g.n_tiles) * e : a.gbeta;
    float* gg = !GATED ? nullptr : split ? part + static_cast<size_t>(2 * g.n_tiles) * e + g.n_tiles * bt : a.gg;
    const size_t gg_n = GM == 2 ? e : bt;  // gg per channel or per token
    const int dp = g.rsc * kSl, cp = g.rsr * kSl;
    constexpr int NO = GATED ? 4 : 3;  // [KB][D] output arrays per block
    constexpr int NR = GM == 2 ? 3 : 2;  // [KB][DPL] arrays per staging buffer (k, q, alpha)
    auto lds_bytes = [&](int dpx, int cpx, int nc, int D) {
        return sizeof(float) * (2 * (NR * kBwdSteps * dpx + 2 * kBwdSteps * cpx + 2 * kBwdSteps) + 2 * cpx +
                                2 * (NO * kBwdSteps * D + kBwdSteps * nc));
    };
    const size_t lds_b = lds_bytes(dp, cp, g.nc, a.D);
    // with kRpt 8 and tiles of min(D, 32) columns, RSR = min(RSC, 4) for every D <= 128;
    // above, 16-column tiles: RSC 32, RSR 2
    const bool wide = a.D > 128;
    if (wide ? (g.rsc != 32 || g.rsr != 2 || g.nc != kTileColsWide)
             : (g.rsr != (g.rsc < 4 ? g.rsc : 4) || g.rsc > 16))
        return hipErrorInvalidValue;
    auto kern = delta_bwd_kernel<InT, 16, 4, kTileCols, GM>;
    int which = 4;  // the kernel's slot among the geometries below
    switch (g.rsc) {
        case 1: kern = delta_bwd_kernel<InT, 1, 1, kTileCols, GM>, which = 0; break;
        case 2: kern = delta_bwd_kernel<InT, 2, 2, kTileCols, GM>, which = 1; break;
        case 4: kern = delta_bwd_kernel<InT, 4, 4, kTileCols, GM>, which = 2; break;
        case 8: kern = delta_bwd_kernel<InT, 8, 4, kTileCols, GM>, which = 3; break;
        case 32: kern = delta_bwd_kernel<InT, 32, 2, kTileColsWide, GM>, which = 5; break;
        default: break;
    }
    if (lds_b > 64 * 1024) {
        // the dynamic-LDS limit is a per-device function attribute: set it once per kernel,
        // to what the largest D of its geometry needs (128, or 256 for the wide tiles)
        const size_t lds_max = wide ? lds_bytes(32 * kSl, 2 * kSl, kTileColsWide, 256)
                                    : lds_bytes(dp, cp, g.nc, 128);
        if (lds_b > lds_max) return hipErrorInvalidValue;
        int dev = 0;
        if ((err = hipGetDevice(&dev)) != hipSuccess) return err;
        static bool attr_set[6][64] = {};
        if (dev < 0 || dev >= 64 || !attr_set[which][dev]) {
            err = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds_max));
            if (err != hipSuccess) return err;
            if (dev >= 0 && dev < 64) attr_set[which][dev] = true;
        }
    }
    hipLaunchKernelGGL(kern, dim3(grid), dim3(g.threads), lds_b, st, static_cast<const InT*>(a.q),
                       static_cast<const InT*>(a.k), a.beta, a.g, a.s0, a.go, a.gs, u_ws, ck_ws, gq, gk,
                       a.gv, gb, gg, a.gs0, a.T, a.H, a.D, g.nc, g.n_tiles, split ? e : 0, split ? bt : 0);
    err = hipGetLastError();
    if (err != hipSuccess || !split) return err;
    if ((err = launch_reduce(a.gq, gq, e, e, g.n_tiles, st)) != hipSuccess) return err;
    if ((err = launch_reduce(a.gk, gk, e, e, g.n_tiles, st)) != hipSuccess) return err;
    if (GATED && (err = launch_reduce(a.gg, gg, gg_n, gg_n, g.n_tiles, st)) != hipSuccess) return err;
    return launch_reduce(a.gbeta, gb, bt, bt, g.n_tiles, st);
}

hipError_t launch_bwd(const BwdArgs& a, hipStream_t st) {
    if (a.n_pairs == 0) return hipSuccess;
    if (a.g && a.per_channel)
        return a.in_bf16 ? launch_bwd_in<uint16_t, 2>(a, st) : launch_bwd_in<float, 2>(a, st);
    if (a.g)
        return a.in_bf16 ? launch_bwd_in<uint16_t, 1>(a, st) : launch_bwd_in<float, 1>(a, st);
    return a.in_bf16 ? launch_bwd_in<uint16_t, 0>(a, st) : launch_bwd_in<float, 0>(a, st);
}

}  // namespace pm
