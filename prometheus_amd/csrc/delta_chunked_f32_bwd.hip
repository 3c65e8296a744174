// delta_chunked_f32_bwd.hip — K9: the chunked backward for fp32 q/k/v on fp32 MFMA
// (v_mfma_f32_16x16x4f32), D in {64, 128}, fixed-length batches.  Every product is
// fp32 x fp32 with fp32 accumulation.
//
// The reference's VJP (kernels/__init__.py:460-527, :529-588) in the WY/UT chunk form,
// chunks of C = 16 tokens.  Per chunk with start state S, T = (I + A)^-1,
// A = strict_lower(diag(beta) K K^T), T'' = -T diag(beta), X' = K S - V, U = T'' X',
// P = lower_incl(Q K^T), the forward is O = Q S + P U, S' = S + K^T U.  Given
// G = dL/dS' and dO:
//   W  = T^T (K G + P^T dO)                      (= dL/d(diag(beta)(V - K S)))
//   G <- G + Q^T dO - K^T diag(beta) W           (dL/dS)
//   dV = diag(beta) W
//   dP = lower_incl(dO U^T),  dA = -strict_lower(W U^T)
//   dQ = dO S^T + dP K
//   dK = U G^T + dP^T Q - diag(beta) W S^T + diag(beta) dA K + dA^T diag(beta) K
//   dbeta_t = -W_t . X'_t + sum_s dA_ts (k_t . k_s)
// Only G travels backwards from chunk to chunk, only S forwards.
//
// Launches (on the caller's stream):
//   K9p (delta_chunked_f32.hip): (T'')^T, T, K K^T, beta and P per chunk.
//   K9a + K9b (delta_chunked_f32.hip, one launch, one workgroup of eight waves per (b, h,
//     32 columns of d_v)): the forward in its history mode, storing S at the start of
//     every span of kF32Span chunks and at the end of the sequence; beside it the G
//     recurrence backwards over all chunks, storing W and dV per token, G at the end of
//     every span, dS0.
//   K9c (span, one workgroup per (b, h, span)): from the span's start state, the forward
//     again (X', U, with U kept in LDS for the whole span), then backwards from the
//     span's end state and end gradient: S reconstructed as S - K^T U (no growth: U is
//     the stored forward value), G as in K9b, and dQ, dK, dbeta.
// Column ownership differs by phase: the recurrences over S and G keep their columns
// independent (a wave owns 16 columns of d_v), while the products contracting over d_v
// (dO S^T, U G^T, ...) need all of them: K9c's forward keeps S by columns (j), its
// reverse keeps S^T and G^T by rows of d (a wave owns 16 of them), and the two small
// products that contract over d_v inside a chunk (dO U^T, W U^T) are summed over the
// waves in LDS, in a fixed order.

#include "pm_cdna4.h"
#include "pm_f32mfma.h"
#include "pm_internal.h"

namespace pm {
namespace {

__device__ __forceinline__ f32x4_t ld4(const unsigned char* p) { return *reinterpret_cast<const f32x4_t*>(p); }
__device__ __forceinline__ void st4(unsigned char* p, f32x4_t x) { *reinterpret_cast<f32x4_t*>(p) = x; }
__device__ __forceinline__ void fence() { __builtin_amdgcn_sched_barrier(0); }

// ---------------------------------------------------------------- K9c
template <int D>
struct SpGeo {
    static constexpr int NW = D / 16;              // waves; wave w owns rows 16 w .. of d
    static constexpr int NT = D / 16;
    static constexpr int NI = kC16 * D * 4 / 1024; // 1 KiB copies per row tile
    static constexpr int TILE = kC16 * D * 4;
    static constexpr int B_K = 0;                  // row tiles (f32_chunk): K, Q, dO, W, U, V
    static constexpr int B_Q = B_K + TILE;
    static constexpr int B_O = B_Q + TILE;
    static constexpr int B_W = B_O + TILE;
    static constexpr int B_U = B_W + TILE;
    static constexpr int B_V = B_U + TILE;
    static constexpr int B_G = B_V + TILE;         // K K^T, accumulator registers
    static constexpr int B_B = B_G + 1024;         // beta (64 bytes; the copy fills 1 KiB)
    static constexpr int BUF = B_B + 1024;
    static constexpr int OFF_DB = 2 * BUF;                     // dbeta parts: 2 slots x NW x 16
    static constexpr int OFF_PP = OFF_DB + 2 * NW * 64;        // per wave: dO U^T, W U^T parts [t][s]
    static constexpr int OFF_TR = OFF_PP + NW * 2048;          // totals dP, dA as rows [t][s]
    static constexpr int OFF_TC = OFF_TR + 2048;               // totals dP, dA as columns [s][t], stride 20
    static constexpr int BYTES = OFF_TC + 2 * 16 * 20 * 4;
    static constexpr int NC = 6 * NI + 2;                      // copies per chunk
    static_assert(BYTES <= 160 * 1024, "LDS");
};

// s_waitcnt vmcnt(n) for a wave-uniform n in [0, 20] (more waits for 20)
__device__ __forceinline__ void wait_vm_upto(int n) {
    switch (n) {
        case 0: wait_vm_n<0>(); break;
        case 1: wait_vm_n<1>(); break;
        case 2: wait_vm_n<2>(); break;
        case 3: wait_vm_n<3>(); break;
        case 4: wait_vm_n<4>(); break;
        case 5: wait_vm_n<5>(); break;
        case 6: wait_vm_n<6>(); break;
        case 7: wait_vm_n<7>(); break;
        case 8: wait_vm_n<8>(); break;
        case 9: wait_vm_n<9>(); break;
        case 10: wait_vm_n<10>(); break;
        case 11: wait_vm_n<11>(); break;
        case 12: wait_vm_n<12>(); break;
        case 13: wait_vm_n<13>(); break;
        case 14: wait_vm_n<14>(); break;
        case 15: wait_vm_n<15>(); break;
        case 16: wait_vm_n<16>(); break;
        case 17: wait_vm_n<17>(); break;
        case 18: wait_vm_n<18>(); break;
        case 19: wait_vm_n<19>(); break;
        default: wait_vm_n<20>(); break;
    }
}

// One workgroup of NW waves per (b, h, span of kF32Span chunks), the span's chunks
// backwards from its end state and end gradient (S^T and G^T by rows of d: wave w holds
// S^T[16 i + 4 g + v][16 w + r] in tile i, G^T likewise, gathered from the histories).
// Per chunk, from the chunk's K, Q, dO, W, U (the forward's, stored by the history pass)
// and V rows:
//   S^T -= U^T K (S^T at the chunk's start: U is the forward's own value, so the
//   subtraction does not amplify error); dQ = dO S^T; WS = W S^T; dK = U G^T -
//   diag(beta) WS; G^T += dO^T Q - (diag(beta) W)^T K; this wave's parts of dO U^T and
//   W U^T, and of -W.X' = -sum_d K WS + W.V (X' = K S - V);
// a barrier; each wave sums 1/NW of the parts' entries (in a fixed order) and masks them
// into dP and dA; a barrier; dQ += dP K, dK += dP^T Q + diag(beta) dA K + dA^T diag(beta)
// K; wave 0 forms dbeta.  Staging: two chunk buffers; chunk m - 2's copies are issued
// once every wave has read chunk m (after the first barrier) and waited for before the
// second barrier of chunk m - 1.
template <int D>
__global__ __launch_bounds__(D * 4) void f32_bwd_span_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ go, const float* __restrict__ rec, const float* __restrict__ s_hist,
    const float* __restrict__ g_hist, const float* __restrict__ w_in, const float* __restrict__ u_in,
    float* __restrict__ gq, float* __restrict__ gk, float* __restrict__ gbeta, int T, int H, int n_ch, int n_span) {
    using G = SpGeo<D>;
    constexpr int NW = G::NW, NT = G::NT;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

    const int pair = blockIdx.x / n_span, span = blockIdx.x % n_span;
    const int seq = pair / H, h = pair % H;
    const long tok0 = static_cast<long>(seq) * T;
    const int c0 = span * kF32Span;
    const int nm = min(kF32Span, n_ch - c0);  // chunks in this span
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = static_cast<int>(uniform(static_cast<unsigned>(tid >> 6)));
    const int r = lane & 15, g = lane >> 4;
    const size_t tstride = static_cast<size_t>(H) * D;
    const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};

    auto buf = [=](int m) { return smem + (m & 1) * G::BUF; };
    auto col_read = [=](const unsigned char* tileb, int t, int d) {  // X[t][d] of a row tile
        return reinterpret_cast<const float*>(tileb)[4 * f32_chunk<D>(t, d >> 2) + (d & 3)];
    };
    auto row_read = [=](const unsigned char* tileb, int i) {  // X[r][16 i + 4 g ..]
        return ld4(tileb + 16 * f32_chunk<D>(r, 4 * i + g));
    };
    auto row0_of = [=](int m, int col) {
        return static_cast<size_t>(tok0 + (c0 + m) * kC16) * tstride + static_cast<size_t>(h) * D + col;
    };
    auto bytes_of = [=](int m, int row_floats) {
        const int clen = min(kC16, T - (c0 + m) * kC16);
        return static_cast<unsigned>(((clen - 1) * tstride + row_floats) * 4);
    };
    // copy number x of chunk m (one branch per source: a selected pointer would become a
    // table in scratch); wave w issues x = w, w + NW, ...
    auto copy_one = [=](int m, int x, unsigned char* b) __attribute__((always_inline)) {
        const size_t cslot = static_cast<size_t>(pair) * n_ch + c0 + m;
        if (x < 6 * G::NI) {
            const int which = x / G::NI, i = x % G::NI;
            const int qc = 64 * i + lane, t = qc / (D / 4), p = (qc % (D / 4)) ^ t;
            const unsigned vo = static_cast<unsigned>(t * tstride * 4 + 16 * p);
            const size_t r0 = row0_of(m, 0);
            const unsigned nb = bytes_of(m, D);
            if (which == 0) {
                dma16_asm(make_rsrc(k + r0, nb), uniform_ptr(b + G::B_K + 1024 * i), vo);
            } else if (which == 1) {
                dma16_asm(make_rsrc(q + r0, nb), uniform_ptr(b + G::B_Q + 1024 * i), vo);
            } else if (which == 2) {
                // a null dO reads zeros (a zero-length range)
                dma16_asm(make_rsrc(go ? go + r0 : go, go ? nb : 0u), uniform_ptr(b + G::B_O + 1024 * i), vo);
            } else if (which == 3) {
                dma16_asm(make_rsrc(w_in + r0, nb), uniform_ptr(b + G::B_W + 1024 * i), vo);
            } else if (which == 4) {
                dma16_asm(make_rsrc(u_in + r0, nb), uniform_ptr(b + G::B_U + 1024 * i), vo);
            } else {
                dma16_asm(make_rsrc(v + r0, nb), uniform_ptr(b + G::B_V + 1024 * i), vo);
            }
        } else if (x == 6 * G::NI) {
            dma16_asm(make_rsrc(rec + cslot * kF32BwdRec + 256, 1024), uniform_ptr(b + G::B_G),
                      static_cast<unsigned>(16 * lane));
        } else {
            dma16_asm(make_rsrc(rec + cslot * kF32BwdRec + 512, 64), uniform_ptr(b + G::B_B),
                      static_cast<unsigned>(16 * lane));
        }
    };
    auto issue = [=](int m) __attribute__((always_inline)) {
        if (m < 0) return;
        unsigned char* b = buf(m);
        for (int x = w; x < G::NC; x += NW) copy_one(m, x, b);
    };
    const int n_mine = (G::NC - w + NW - 1) / NW;  // copies this wave issues per chunk

    // ---- the span's end state and end gradient, by rows of d, gathered from the column-
    // block layout of the histories: S^T[16 i + 4 g + e][16 w + r] = S[16 w + r][16 i + 4 g + e]
    // is in column block i, tile w, lane 16 (r >> 2) + 4 g + e, register r & 3 ----
    f32x4_t St[NT], Gt[NT];
    {
        const float* sp = s_hist + (static_cast<size_t>(pair) * (n_span + 1) + span + 1) * D * D;
        const float* gp = g_hist + (static_cast<size_t>(pair) * n_span + span) * D * D;
#pragma unroll
        for (int i = 0; i < NT; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const size_t o = (static_cast<size_t>(i) * NT + w) * 256 + 4 * (16 * (r >> 2) + 4 * g + e) + (r & 3);
                St[i][e] = sp[o];
                Gt[i][e] = gp[o];
            }
    }
    issue(nm - 1);
    issue(nm - 2);
    wait_vm_n<0>();
    lds_barrier();

    for (int m = nm - 1; m >= 0; --m) {
        const unsigned char* b = buf(m);
        const int dbs = m & 1;  // the dbeta parts' slot
        // B operands for this wave's rows 16 w + r of d; beta; K K^T
        f32x4_t kc, qc, wj, vj;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            kc[e] = col_read(b + G::B_K, 4 * g + e, 16 * w + r);
            qc[e] = col_read(b + G::B_Q, 4 * g + e, 16 * w + r);
            wj[e] = col_read(b + G::B_W, 4 * g + e, 16 * w + r);  // W, V at columns 16 w + r of d_v
            vj[e] = col_read(b + G::B_V, 4 * g + e, 16 * w + r);
        }
        const f32x4_t b4 = ld4(b + G::B_B + 16 * g);
        const float br = reinterpret_cast<const float*>(b + G::B_B)[r];
        const f32x4_t gram = ld4(b + G::B_G + 16 * lane);  // K K^T[4 g + v][r] = K K^T[r][4 g + v]
        fence();
        // S^T -= U^T K: S^T at the chunk's start
#pragma unroll
        for (int i = 0; i < NT; ++i) {
            float uc[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) uc[e] = col_read(b + G::B_U, 4 * g + e, 16 * i + r);
#pragma unroll
            for (int e = 0; e < 4; ++e) St[i] = mfma4(uc[e], -kc[e], St[i]);
        }
        // dQ = dO S^T, WS = W S^T, U G^T, and this wave's parts of dO U^T, W U^T
        f32x4_t qa[2] = {zero, zero}, wa[2] = {zero, zero}, ka[2] = {zero, zero};
        f32x4_t pp = zero, pa = zero;
#pragma unroll
        for (int i = 0; i < NT; ++i) {
            const f32x4_t dor = row_read(b + G::B_O, i);
            const f32x4_t wrw = row_read(b + G::B_W, i);
            const f32x4_t ur = row_read(b + G::B_U, i);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                qa[e & 1] = mfma4(dor[e], St[i][e], qa[e & 1]);
                wa[e & 1] = mfma4(wrw[e], St[i][e], wa[e & 1]);
                ka[e & 1] = mfma4(ur[e], Gt[i][e], ka[e & 1]);
            }
            if (i == w) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    pp = mfma4(ur[e], dor[e], pp);  // (U dO^T)[4 g + v][r] = (dO U^T)[r][4 g + v]
                    pa = mfma4(ur[e], wrw[e], pa);
                }
            }
        }
        const f32x4_t WS = wa[0] + wa[1];  // W S^T[4 g + v][16 w + r]
        f32x4_t dK = ka[0] + ka[1] - b4 * WS;
        // this wave's part of -W.X' per token 4 g + v: -sum over its d of K WS, plus W.V over
        // its 16 columns of d_v
        {
            f32x4_t x = wj * vj - kc * WS;
#pragma unroll
            for (int sh = 1; sh < 16; sh <<= 1)
#pragma unroll
                for (int e = 0; e < 4; ++e) x[e] += __shfl_xor(x[e], sh);
            if (r == 0) st4(smem + G::OFF_DB + (dbs * NW + w) * 64 + 16 * g, x);
        }
        unsigned char* part = smem + G::OFF_PP + w * 2048;
        // row t = r, entries s = 4 g .. 4 g + 3 of each [t][s] part (16 bytes)
        st4(part + 16 * (4 * r + g), pp);
        st4(part + 1024 + 16 * (4 * r + g), pa);
        // G^T += dO^T Q - (diag(beta) W)^T K (after its use above)
#pragma unroll
        for (int i = 0; i < NT; ++i) {
            float dc[4], wc[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                dc[e] = col_read(b + G::B_O, 4 * g + e, 16 * i + r);
                wc[e] = -b4[e] * col_read(b + G::B_W, 4 * g + e, 16 * i + r);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                Gt[i] = mfma4(dc[e], qc[e], Gt[i]);
                Gt[i] = mfma4(wc[e], kc[e], Gt[i]);
            }
        }
        lds_barrier();  // Y: the parts are in LDS; every wave is done reading chunk m
        issue(m - 2);   // into chunk m's buffer
        for (int x = tid; x < 512; x += NW * 64) {
            const int mat = x >> 8, t = (x >> 4) & 15, s = x & 15;
            float sum = 0.f;
#pragma unroll
            for (int ww = 0; ww < NW; ++ww)
                sum += reinterpret_cast<const float*>(smem + G::OFF_PP + ww * 2048 + mat * 1024)[16 * t + s];
            const float val = mat == 0 ? (s <= t ? sum : 0.f) : (s < t ? -sum : 0.f);
            reinterpret_cast<float*>(smem + G::OFF_TR + mat * 1024)[16 * t + s] = val;
            reinterpret_cast<float*>(smem + G::OFF_TC + mat * 1280)[20 * s + t] = val;
        }
        // chunk m - 1's copies have landed (issued after the previous chunk's first barrier);
        // still in flight may be the previous chunk's stores and chunk m - 2's copies
        if (m >= 1) wait_vm_upto((m + 1 < nm ? 8 + (w == 0 ? 1 : 0) : 0) + (m >= 2 ? n_mine : 0));
        lds_barrier();  // Z: totals in LDS, chunk m - 1 in its buffer
        // dQ += dP K; dK += dP^T Q + diag(beta) dA K + dA^T diag(beta) K
        const f32x4_t dpr = ld4(smem + G::OFF_TR + 16 * (4 * r + g));            // dP[r][4 g ..]
        const f32x4_t dar = ld4(smem + G::OFF_TR + 1024 + 16 * (4 * r + g));     // dA[r][4 g ..]
        const f32x4_t dpc = ld4(smem + G::OFF_TC + 4 * (20 * r + 4 * g));        // dP[4 g ..][r]
        const f32x4_t dac = ld4(smem + G::OFF_TC + 1280 + 4 * (20 * r + 4 * g)); // dA[4 g ..][r]
        f32x4_t dQ = qa[0] + qa[1];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            dQ = mfma4(dpr[e], kc[e], dQ);
            dK = mfma4(dpc[e], qc[e], dK);
            dK = mfma4(br * dar[e], kc[e], dK);
            dK = mfma4(dac[e] * b4[e], kc[e], dK);
        }
        // rows 4 g + v of dQ and dK, columns 16 w + r
        {
            const size_t row0 = row0_of(m, 16 * w);
            const unsigned nb = bytes_of(m, 16);
            const __amdgpu_buffer_rsrc_t rq = make_rsrc(gq + row0, nb), rk = make_rsrc(gk + row0, nb);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const unsigned off = static_cast<unsigned>(((4 * g + e) * tstride + r) * 4);
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(dQ[e]), rq, off, 0, 0);
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(dK[e]), rk, off, 0, 0);
            }
        }
        if (w == 0) {
            // dbeta_t = -W_t . X'_t + sum_s dA_ts (k_t . k_s), t = r
            float sdg = dar[0] * gram[0] + dar[1] * gram[1] + dar[2] * gram[2] + dar[3] * gram[3];
            sdg += __shfl_xor(sdg, 16);
            sdg += __shfl_xor(sdg, 32);
            float wx = 0.f;
#pragma unroll
            for (int ww = 0; ww < NW; ++ww)
                wx += reinterpret_cast<const float*>(smem + G::OFF_DB + (dbs * NW + ww) * 64)[r];
            const int clen = min(kC16, T - (c0 + m) * kC16);
            const __amdgpu_buffer_rsrc_t rb = make_rsrc(gbeta + (tok0 + (c0 + m) * kC16) * H + h,
                                                        static_cast<unsigned>(((clen - 1) * H + 1) * 4));
            // every lane stores (lanes r of each group write the same value), one store per wave
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(wx + sdg), rb, static_cast<unsigned>(r * H * 4), 0,
                                                  0);
        }
    }
}

template <typename Kern>
hipError_t set_lds(Kern kern, int bytes) {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

template <int D>
hipError_t launch_d(const BwdArgs& a, hipStream_t st) {
    const int n_ch = (a.T + kC16 - 1) / kC16;
    const int n_span = (n_ch + kF32Span - 1) / kF32Span;
    const F32BwdWs ws = f32_bwd_ws(a.n_pairs, a.T, D);
    unsigned char* base = reinterpret_cast<unsigned char*>(a.workspace);
    float* t2 = reinterpret_cast<float*>(base + ws.t2);
    float* rec = reinterpret_cast<float*>(base + ws.rec);
    float* s_hist = reinterpret_cast<float*>(base + ws.s_hist);
    float* g_hist = reinterpret_cast<float*>(base + ws.g_hist);
    float* w_ws = reinterpret_cast<float*>(base + ws.w);
    float* u_ws = reinterpret_cast<float*>(base + ws.u);
    const float* q = static_cast<const float*>(a.q);
    const float* k = static_cast<const float*>(a.k);
    const float* v = static_cast<const float*>(a.v);
    hipError_t e;
    if ((e = set_lds(f32_bwd_span_kernel<D>, SpGeo<D>::BYTES)) != hipSuccess) return e;
    if (n_ch > 0 && (e = launch_f32_bwd_prep(q, k, a.beta, a.n_pairs, a.T, a.H, D, t2, rec, st)) != hipSuccess) return e;
    if ((e = launch_f32_hist_sweep(a, t2, rec, w_ws, s_hist, g_hist, u_ws, st)) != hipSuccess) return e;
    if (n_ch == 0) return hipSuccess;
    hipLaunchKernelGGL(f32_bwd_span_kernel<D>, dim3(static_cast<unsigned>(a.n_pairs * n_span)), dim3(D * 4),
                       SpGeo<D>::BYTES, st, q, k, v, a.go, rec, s_hist, g_hist, w_ws, u_ws, a.gq, a.gk, a.gbeta, a.T,
                       a.H, n_ch, n_span);
    return hipGetLastError();
}

}  // namespace

F32BwdWs f32_bwd_ws(long n_pairs, int T, int D) {
    const size_t n_ch = static_cast<size_t>((T + kC16 - 1) / kC16);
    const size_t n_span = (n_ch + kF32Span - 1) / kF32Span;
    const size_t np = static_cast<size_t>(n_pairs);
    auto al = [](size_t x) { return (x + 255) & ~static_cast<size_t>(255); };
    F32BwdWs w;
    w.t2 = 0;
    w.rec = al(w.t2 + np * n_ch * 256 * 4);
    w.s_hist = al(w.rec + np * n_ch * kF32BwdRec * 4);
    w.g_hist = al(w.s_hist + np * (n_span + 1) * D * D * 4);
    w.w = al(w.g_hist + np * n_span * D * D * 4);
    w.u = al(w.w + np * static_cast<size_t>(T) * D * 4);
    w.bytes = al(w.u + np * static_cast<size_t>(T) * D * 4);
    return w;
}

// 32-bit buffer offsets: a chunk of fp32 rows spans 16 token rows of H*D values.
bool f32_bwd_supported(int D, int H) { return (D == 64 || D == 128) && static_cast<long>(H) * D <= (1L << 24); }

hipError_t launch_bwd_chunked_f32(const BwdArgs& a, hipStream_t st) {
    if (a.n_pairs == 0) return hipSuccess;
    if (a.in_bf16 || !f32_bwd_supported(a.D, a.H)) return hipErrorInvalidValue;
    return a.D == 128 ? launch_d<128>(a, st) : launch_d<64>(a, st);
}

}  // namespace pm
