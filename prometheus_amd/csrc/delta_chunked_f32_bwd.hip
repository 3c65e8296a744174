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
//   K9p + K9a (delta_chunked_f32.hip): (T'')^T, T, K K^T, beta and P per chunk; the forward
//     in its history mode, storing S at the start of every span of kF32Span chunks and
//     at the end of the sequence.
//   K9b (sweep, one workgroup per (b, h, 32 columns of d_v)): the G recurrence backwards
//     over all chunks; stores W and dV per token, G at the end of every span, dS0.
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

#include <mutex>

#include "pm_cdna4.h"
#include "pm_f32mfma.h"
#include "pm_internal.h"

namespace pm {
namespace {

__device__ __forceinline__ f32x4_t ld4(const unsigned char* p) { return *reinterpret_cast<const f32x4_t*>(p); }
__device__ __forceinline__ void st4(unsigned char* p, f32x4_t x) { *reinterpret_cast<f32x4_t*>(p) = x; }
__device__ __forceinline__ void fence() { __builtin_amdgcn_sched_barrier(0); }

// ---------------------------------------------------------------- K9b
template <int D>
struct SwGeo {
    static constexpr int NT = D / 16;              // G accumulator tiles per chain wave
    static constexpr int NI = kC16 * D * 4 / 1024; // 1 KiB copies per K or Q tile
    static constexpr int NB = 4;                   // rotating chunk buffers
    static constexpr int B_K = 0;                  // K rows (f32_chunk)
    static constexpr int B_Q = B_K + kC16 * D * 4; // Q rows
    static constexpr int B_O = B_Q + kC16 * D * 4; // dO columns of the tile: two [16 t][16] blocks
    static constexpr int B_T = B_O + 2048;         // T, accumulator registers
    static constexpr int B_P = B_T + 1024;         // P, accumulator registers
    static constexpr int B_B = B_P + 1024;         // beta (64 bytes; the copy fills 1 KiB)
    static constexpr int BUF = B_B + 1024;
    static constexpr int OFF_H = NB * BUF;                   // 2 slots x 2 chain waves: Q^T dO (NT tiles)
    static constexpr int OFF_W = OFF_H + 2 * 2 * NT * 1024;  // 2 slots x 2 chain waves: W, -beta W
    static constexpr int BYTES = OFF_W + 2 * 2 * 2048;
    static constexpr int NCP = 2 * NI + 5;  // the copy wave's copies per chunk
    static constexpr int NST = 2;           // ... and its stores (W and dV rows)
    static_assert(BYTES <= 160 * 1024 && NCP + NST <= 63, "LDS / vmcnt");
};

// Waves 2 and 3 (chain) carry G for the columns col0 + 16 (w - 2) + [0, 16) as NT
// accumulator tiles (rows 16 m ..).  Iteration i runs chunk c = n - i on the chain
// (i >= 1): Y = K G, dU = Y + P^T dO, W = T^T dU, and G += Q^T dO - K^T diag(beta) W,
// with Q^T dO built one iteration earlier by waves 0 and 1 (helper w serves chain wave
// 2 + w) and P, T, beta taken from the prep's record.  The helpers store the W and dV rows the chain
// handed over through LDS one iteration later (iteration n + 1 stores chunk 0's); wave 1
// copies chunk n - 3 - i (two iterations ahead of its first use).  One LDS-only barrier
// per iteration 0 .. n.
template <int D>
__global__ __launch_bounds__(256) void f32_bwd_sweep_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ go,
    const float* __restrict__ gs, float* __restrict__ gv, float* __restrict__ gs0, const float* __restrict__ rec,
    float* __restrict__ w_out, float* __restrict__ g_hist, int n_pairs, int T, int H, int n_tiles, int n_ch,
    int n_span) {
    using G = SwGeo<D>;
    constexpr int NT = G::NT;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

    // XCD-aware placement: the n_tiles workgroups of a pair share bid % 8
    const int bid = blockIdx.x;
    const int xcd = bid & 7, bslot = bid >> 3;
    const int tile = bslot % n_tiles;
    const int pair = (bslot / n_tiles) * 8 + xcd;
    if (pair >= n_pairs) return;
    const int seq = pair / H, h = pair % H;
    const long tok0 = static_cast<long>(seq) * T;
    const int col0 = tile * 32;
    const int lane = threadIdx.x & 63;
    const int w = static_cast<int>(uniform(static_cast<unsigned>(threadIdx.x >> 6)));
    const int r = lane & 15, g = lane >> 4;
    // roles: waves 2 and 3 chain, 0 and 1 helpers (wave 1 copies), so that beside a
    // workgroup of the history pass (chain waves 0 and 1) the four chains of a CU spread
    // over its four SIMDs (waves of a workgroup go to the SIMDs in turn)
    const bool chain_wave = w >= 2;
    const int cw = w & 1;  // the 16 columns col0 + 16 cw + [0, 16) this wave works on
    const bool copy_wave = w == 1;
    const size_t tstride = static_cast<size_t>(H) * D;
    const size_t sbase = static_cast<size_t>(pair) * D * D;
    const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};

    auto buf = [&](int c) { return smem + (c % G::NB) * G::BUF; };
    auto hslot = [&](int c, int which) { return smem + G::OFF_H + ((c & 1) * 2 + which) * NT * 1024; };
    auto wslot = [&](int c, int which) { return smem + G::OFF_W + ((c & 1) * 2 + which) * 2048; };
    auto col_read = [&](const unsigned char* tileb, int t, int d) {  // X[t][d] of a row tile
        return reinterpret_cast<const float*>(tileb)[4 * f32_chunk<D>(t, d >> 2) + (d & 3)];
    };

    // ---- HBM -> LDS copies of chunk c ----
    auto row0_of = [&](int c, int col) {
        return static_cast<size_t>(tok0 + c * kC16) * tstride + static_cast<size_t>(h) * D + col;
    };
    auto bytes_of = [&](int c, int row_floats) {
        const int clen = min(kC16, T - c * kC16);
        return static_cast<unsigned>(((clen - 1) * tstride + row_floats) * 4);
    };
    auto copy_tile = [&](const float* base, int c, unsigned char* dst) __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(base + row0_of(c, 0), bytes_of(c, D));
        unsigned char* d0 = uniform_ptr(dst);
#pragma unroll
        for (int i = 0; i < G::NI; ++i) {
            const int qc = 64 * i + lane;
            const int t = qc / (D / 4), p = (qc % (D / 4)) ^ t;
            dma16_asm(rs, d0 + 1024 * i, static_cast<unsigned>(t * tstride * 4 + 16 * p));
        }
    };
    auto copies = [&](int c) __attribute__((always_inline)) {
        unsigned char* b = buf(c);
        copy_tile(k, c, b + G::B_K);
        copy_tile(q, c, b + G::B_Q);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            // a null dO reads zeros (a zero-length range)
            const __amdgpu_buffer_rsrc_t rs =
                make_rsrc(go ? go + row0_of(c, col0 + 16 * j) : go, go ? bytes_of(c, 16) : 0u);
            const int t = lane >> 2, p = lane & 3;
            dma16_asm(rs, uniform_ptr(b + G::B_O + 1024 * j), static_cast<unsigned>(t * tstride * 4 + 16 * p));
        }
        const float* rc = rec + (static_cast<size_t>(pair) * n_ch + c) * kF32BwdRec;
        dma16_asm(make_rsrc(rc, 1024), uniform_ptr(b + G::B_T), static_cast<unsigned>(16 * lane));
        dma16_asm(make_rsrc(rc + 528, 1024), uniform_ptr(b + G::B_P), static_cast<unsigned>(16 * lane));
        dma16_asm(make_rsrc(rc + 512, 64), uniform_ptr(b + G::B_B), static_cast<unsigned>(16 * lane));
    };

    if (n_ch > 0 && copy_wave) {
        copies(n_ch - 1);
        if (n_ch > 1) {
            copies(n_ch - 2);
            wait_vm_n<G::NCP>();
        } else {
            wait_vm_n<0>();
        }
    }
    if (n_ch > 0) lds_barrier();  // B0

    if (chain_wave) {
        // ============ chain wave ============
        const int ecol = col0 + 16 * cw + r;
        f32x4_t Gm[NT];
#pragma unroll
        for (int m = 0; m < NT; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                Gm[m][e] = gs ? gs[sbase + static_cast<size_t>(16 * m + 4 * g + e) * D + ecol] : 0.f;
        // vmcnt(0) as the intrinsic: the gs loads settle here, not inside the loop
        __builtin_amdgcn_s_waitcnt(0x0F70);
        // Iteration i runs chunk n - i from operands read from its buffer in iteration i - 1
        // (that buffer has landed by then: the helpers use it in iteration i - 1), so that no
        // LDS latency starts the chain's chunk; only Q^T dO (built in iteration i - 1) is read
        // in iteration i.
        f32x4_t kf[NT], dOc = zero, ta = zero, b4 = zero, pp = zero;
        float kt[4][NT];
        auto fetch = [&](int c) __attribute__((always_inline)) {
            const unsigned char* b = buf(c);
#pragma unroll
            for (int m = 0; m < NT; ++m) kf[m] = ld4(b + G::B_K + 16 * f32_chunk<D>(r, 4 * m + g));
            const float* Of = reinterpret_cast<const float*>(b + G::B_O + 1024 * cw);
#pragma unroll
            for (int e = 0; e < 4; ++e) dOc[e] = Of[(4 * g + e) * 16 + r];
            ta = ld4(b + G::B_T + 16 * lane);
            b4 = ld4(b + G::B_B + 16 * g);
            pp = ld4(b + G::B_P + 16 * lane);
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int m = 0; m < NT; ++m) kt[e][m] = col_read(b + G::B_K, 4 * g + e, 16 * m + r);
        };
        for (int i = 0; i <= n_ch; ++i) {
            if (i >= 1) {
                const int c = n_ch - i;
                if (c == n_ch - 1 || c % kF32Span == kF32Span - 1) {
                    float* hp = g_hist + ((static_cast<size_t>(pair) * n_span + c / kF32Span) * (D / 16) + col0 / 16 +
                                          cw) * NT * 256;
#pragma unroll
                    for (int m = 0; m < NT; ++m) *reinterpret_cast<f32x4_t*>(hp + m * 256 + 4 * lane) = Gm[m];
                }
                f32x4_t hq[NT];
#pragma unroll
                for (int m = 0; m < NT; ++m) hq[m] = ld4(hslot(c, cw) + 1024 * m + 16 * lane);
                // Y = K G (accumulator e takes the steps (m, e))
                f32x4_t ya[4] = {zero, zero, zero, zero};
#pragma unroll
                for (int m = 0; m < NT; ++m)
#pragma unroll
                    for (int e = 0; e < 4; ++e) ya[e] = mfma4(kf[m][e], Gm[m][e], ya[e]);
                const f32x4_t dU = mm16(pp, dOc, (ya[0] + ya[1]) + (ya[2] + ya[3]));  // + P^T dO
                const f32x4_t W = mm16(ta, dU);                                        // T^T dU
                const f32x4_t nbW = -(W * b4);                                         // -diag(beta) W
                st4(wslot(c, cw) + 16 * lane, W);
                st4(wslot(c, cw) + 1024 + 16 * lane, nbW);
                // G += Q^T dO - K^T diag(beta) W
#pragma unroll
                for (int e = 0; e < 4; ++e)
#pragma unroll
                    for (int m = 0; m < NT; ++m) Gm[m] = mfma4(kt[e][m], nbW[e], Gm[m]);
#pragma unroll
                for (int m = 0; m < NT; ++m) Gm[m] += hq[m];
            }
            if (n_ch - 1 - i >= 0) fetch(n_ch - 1 - i);
            // (iteration n_ch too: the helpers store its W after one more barrier)
            if (n_ch > 0) lds_barrier();
        }
#pragma unroll
        for (int m = 0; m < NT; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e) gs0[sbase + static_cast<size_t>(16 * m + 4 * g + e) * D + ecol] = Gm[m][e];
    } else if (n_ch > 0) {
        // ============ helper waves ============
        const int hw = w;
        for (int i = 0; i <= n_ch + 1; ++i) {
            const bool cp = copy_wave && n_ch - 3 - i >= 0;
            if (cp) copies(n_ch - 3 - i);
            const int ch = n_ch - 1 - i;
            if (ch >= 0) {
                const unsigned char* b = buf(ch);
                const float* Of = reinterpret_cast<const float*>(b + G::B_O + 1024 * hw);
                f32x4_t dOc;
#pragma unroll
                for (int e = 0; e < 4; ++e) dOc[e] = Of[(4 * g + e) * 16 + r];
                // Q^T dO for chain wave hw's columns: tile m = rows 16 m .. of d
                f32x4_t hq[NT];
#pragma unroll
                for (int m = 0; m < NT; ++m) {
                    float qt[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) qt[e] = col_read(b + G::B_Q, 4 * g + e, 16 * m + r);
                    hq[m] = zero;
#pragma unroll
                    for (int e = 0; e < 4; ++e) hq[m] = mfma4(qt[e], dOc[e], hq[m]);
                }
#pragma unroll
                for (int m = 0; m < NT; ++m) st4(hslot(ch, hw) + 1024 * m + 16 * lane, hq[m]);
            }
            // the W and dV rows of the chunk the chain ran in the last iteration: lane
            // (t, p) stores columns 4 p .. 4 p + 3 of row t
            const int cs = n_ch - i + 1;
            const bool st = i >= 2;
            if (st) {
                const float* wsrc = reinterpret_cast<const float*>(wslot(cs, hw));
                const int t = lane >> 2, p = lane & 3;
                f32x4_t wv, dv;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int ln = 16 * (t >> 2) + 4 * p + e;
                    wv[e] = wsrc[4 * ln + (t & 3)];
                    dv[e] = -wsrc[256 + 4 * ln + (t & 3)];
                }
                const size_t row0 = row0_of(cs, col0 + 16 * hw);
                const unsigned nb = bytes_of(cs, 16);
                const unsigned off = static_cast<unsigned>((t * tstride + 4 * p) * 4);
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, wv), make_rsrc(w_out + row0, nb),
                                                       off, 0, 0);
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, dv), make_rsrc(gv + row0, nb),
                                                       off, 0, 0);
            }
            if (i <= n_ch) {
                // the copies of chunk ch - 1 (the helpers' next) have landed; the newer copies
                // and this iteration's stores may still be in flight
                if (copy_wave && ch - 1 >= 0) {
                    if (cp && st) wait_vm_n<G::NCP + G::NST>();
                    else if (cp) wait_vm_n<G::NCP>();
                    else if (st) wait_vm_n<G::NST>();
                    else wait_vm_n<0>();
                }
                lds_barrier();
            }
        }
    }
}

// ---------------------------------------------------------------- K9c
template <int D>
struct SpGeo {
    static constexpr int NW = D / 16;              // waves; wave w owns columns (forward) or rows (reverse) 16 w ..
    static constexpr int NT = D / 16;
    static constexpr int NI = kC16 * D * 4 / 1024; // 1 KiB copies per row tile
    static constexpr int TILE = kC16 * D * 4;
    static constexpr int B_K = 0;                  // K rows (f32_chunk)
    static constexpr int B_Q = B_K + TILE;         // Q rows (reverse)
    static constexpr int B_O = B_Q + TILE;         // dO rows (reverse)
    static constexpr int B_W = B_O + TILE;         // W rows (reverse)
    static constexpr int B_T = B_W + TILE;         // (T'')^T (forward)
    static constexpr int B_G = B_T + 1024;         // K K^T, accumulator registers (reverse)
    static constexpr int B_B = B_G + 1024;         // beta (reverse; 64 bytes, the copy fills 1 KiB)
    static constexpr int BUF = B_B + 1024;
    static constexpr int OFF_U = 2 * BUF;                            // U rows of the span's chunks
    static constexpr int OFF_DB = OFF_U + kF32Span * TILE;           // -W.X' partials [chunk][wave][16]
    static constexpr int OFF_PP = OFF_DB + kF32Span * NW * 64;       // per wave: dO U^T, W U^T partials [t][s]
    static constexpr int OFF_TR = OFF_PP + NW * 2048;                // totals dP, dA as rows [t][s]
    static constexpr int OFF_TC = OFF_TR + 2048;                     // totals dP, dA as columns [s][t], stride 20
    static constexpr int BYTES = OFF_TC + 2 * 16 * 20 * 4;
    static constexpr int NCF = NI + 1;      // forward copies per chunk (K, (T'')^T)
    static constexpr int NCR = 4 * NI + 2;  // reverse copies per chunk (K, Q, dO, W, K K^T, beta)
    static_assert(BYTES <= 160 * 1024, "LDS");
};

// One workgroup of NW waves per (b, h, span of kF32Span chunks).  Forward, chunk by chunk
// (wave w: columns 16 w .. of S, D/16 accumulator tiles): X' = K S - V, U = T'' X' and
// U^T = X'^T T''^T, U's rows to LDS, this wave's part of W.X', S += K^T U.  Reverse,
// chunk by chunk backwards (wave w: rows 16 w .. of d; S^T and G^T as D/16 accumulator
// tiles over the columns): S^T -= U^T K (S^T at the chunk's start), dQ = dO S^T,
// dK = U G^T - diag(beta) W S^T, G^T += dO^T Q - (diag(beta) W)^T K, this wave's parts of
// dO U^T and W U^T; after a barrier the parts are summed (each wave sums 1/NW of the
// entries, in a fixed order) and masked into dP and dA; after another, dQ += dP K,
// dK += dP^T Q + diag(beta) dA K + dA^T diag(beta) K, and wave 0 forms dbeta.
// Staging: two chunk buffers; every wave issues a share of the next chunk's copies right
// after the barrier that frees its buffer and waits for them before the next barrier.
template <int D>
__global__ __launch_bounds__(D * 4) void f32_bwd_span_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ go, const float* __restrict__ t2, const float* __restrict__ rec,
    const float* __restrict__ s_hist, const float* __restrict__ g_hist, const float* __restrict__ w_in,
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

    auto buf = [=](int f) { return smem + (f & 1) * G::BUF; };
    auto uh = [=](int m) { return smem + G::OFF_U + m * G::TILE; };
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
    // copy number x of a chunk's list; wave w issues x = w, w + NW, ...
    auto copy_one = [=](int m, bool fwd, int x, unsigned char* b) __attribute__((always_inline)) {
        const size_t cslot = static_cast<size_t>(pair) * n_ch + c0 + m;
        if (fwd) {
            if (x < G::NI) {
                const int qc = 64 * x + lane, t = qc / (D / 4), p = (qc % (D / 4)) ^ t;
                dma16_asm(make_rsrc(k + row0_of(m, 0), bytes_of(m, D)), uniform_ptr(b + G::B_K + 1024 * x),
                          static_cast<unsigned>(t * tstride * 4 + 16 * p));
            } else {
                dma16_asm(make_rsrc(t2 + cslot * 256, 1024), uniform_ptr(b + G::B_T), static_cast<unsigned>(16 * lane));
            }
            return;
        }
        if (x < 4 * G::NI) {
            // one branch per source (a selected pointer would become a table in scratch)
            const int which = x / G::NI, i = x % G::NI;
            const int qc = 64 * i + lane, t = qc / (D / 4), p = (qc % (D / 4)) ^ t;
            const unsigned vo = static_cast<unsigned>(t * tstride * 4 + 16 * p);
            if (which == 0) {
                dma16_asm(make_rsrc(k + row0_of(m, 0), bytes_of(m, D)), uniform_ptr(b + G::B_K + 1024 * i), vo);
            } else if (which == 1) {
                dma16_asm(make_rsrc(q + row0_of(m, 0), bytes_of(m, D)), uniform_ptr(b + G::B_Q + 1024 * i), vo);
            } else if (which == 2) {
                // a null dO reads zeros (a zero-length range)
                dma16_asm(make_rsrc(go ? go + row0_of(m, 0) : go, go ? bytes_of(m, D) : 0u),
                          uniform_ptr(b + G::B_O + 1024 * i), vo);
            } else {
                dma16_asm(make_rsrc(w_in + row0_of(m, 0), bytes_of(m, D)), uniform_ptr(b + G::B_W + 1024 * i), vo);
            }
        } else if (x == 4 * G::NI) {
            dma16_asm(make_rsrc(rec + cslot * kF32BwdRec + 256, 1024), uniform_ptr(b + G::B_G),
                      static_cast<unsigned>(16 * lane));
        } else {
            dma16_asm(make_rsrc(rec + cslot * kF32BwdRec + 512, 64), uniform_ptr(b + G::B_B),
                      static_cast<unsigned>(16 * lane));
        }
    };
    // staged chunk f of the span's sequence: forward m = f (f < nm), reverse m = 2 nm - 1 - f
    auto issue = [=](int f) __attribute__((always_inline)) {
        if (f >= 2 * nm) return;
        const bool fwd = f < nm;
        const int m = fwd ? f : 2 * nm - 1 - f;
        const int n = fwd ? G::NCF : G::NCR;
        unsigned char* b = buf(f);
        for (int x = w; x < n; x += NW) copy_one(m, fwd, x, b);
    };
    // this wave's V and W columns of forward chunk m: X[4 g + e][16 w + r]
    auto load_cols = [=](const float* base, int m) {
        f32x4_t x = zero;
        if (!base || m >= nm) return x;
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(base + row0_of(m, 16 * w), bytes_of(m, 16));
#pragma unroll
        for (int e = 0; e < 4; ++e)
            x[e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                rs, static_cast<unsigned>(((4 * g + e) * tstride + r) * 4), 0, 0));
        return x;
    };

    // ---- forward: S by columns (wave w: S[16 m + 4 g + v][16 w + r], tile m) ----
    f32x4_t S[NT];
    {
        const float* hp = s_hist + ((static_cast<size_t>(pair) * (n_span + 1) + span) * (D / 16) + w) * NT * 256;
#pragma unroll
        for (int m = 0; m < NT; ++m) S[m] = *reinterpret_cast<const f32x4_t*>(hp + m * 256 + 4 * lane);
    }
    issue(0);
    f32x4_t vnext = load_cols(v, 0), wnext = load_cols(w_in, 0);
    f32x4_t St[NT], Gt[NT];  // reverse: S^T[16 i + 4 g + v][16 w + r], G^T likewise (tile i)
    wait_vm_n<0>();
    lds_barrier();
    for (int f = 0; f < nm; ++f) {
        issue(f + 1);
        const f32x4_t vr = vnext, wr = wnext;
        vnext = load_cols(v, f + 1);
        wnext = load_cols(w_in, f + 1);
        const unsigned char* b = buf(f);
        f32x4_t kf[NT];
#pragma unroll
        for (int m = 0; m < NT; ++m) kf[m] = row_read(b + G::B_K, m);
        const f32x4_t tt = ld4(b + G::B_T + 16 * lane);
        fence();
        f32x4_t xa[4] = {-vr, zero, zero, zero};
#pragma unroll
        for (int m = 0; m < NT; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e) xa[e] = mfma4(kf[m][e], S[m][e], xa[e]);
        float kt[4][NT];
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int m = 0; m < NT; ++m) kt[e][m] = col_read(b + G::B_K, 4 * g + e, 16 * m + r);
        const f32x4_t X = (xa[0] + xa[1]) + (xa[2] + xa[3]);  // X'[4 g + v][16 w + r]
        const f32x4_t U = mm16(tt, X);                          // T'' X'
        const f32x4_t Ut = mm16(X, tt);                         // U^T: U[r][16 w + 4 g + v]
        st4(uh(f) + 16 * f32_chunk<D>(r, 4 * w + g), Ut);
        // -W.X' over this wave's columns, per token 4 g + v
        f32x4_t wx = -(X * wr);
#pragma unroll
        for (int sh = 1; sh < 16; sh <<= 1)
#pragma unroll
            for (int e = 0; e < 4; ++e) wx[e] += __shfl_xor(wx[e], sh);
        if (r == 0) st4(smem + G::OFF_DB + (f * NW + w) * 64 + 16 * g, wx);
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int m = 0; m < NT; ++m) S[m] = mfma4(kt[e][m], U[e], S[m]);
        wait_vm_n<0>();
        lds_barrier();
    }

    // ---- reverse: chunk m = nm - 1 .. 0 (staged sequence f = 2 nm - 1 - m) ----
    {
        // S^T and G^T at the span's end, gathered from the column-block layout of the histories:
        // S^T[16 i + 4 g + e][16 w + r] = S[16 w + r][16 i + 4 g + e] is in column block i,
        // tile w, lane 16 (r >> 2) + 4 g + e, register r & 3
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
    for (int m = nm - 1; m >= 0; --m) {
        const int f = 2 * nm - 1 - m;
        issue(f + 1);
        const unsigned char* b = buf(f);
        const unsigned char* ub = uh(m);
        // B operands of this wave's rows 16 w + r of d: K, Q columns; beta of 4 g + e
        f32x4_t kc, qc;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            kc[e] = col_read(b + G::B_K, 4 * g + e, 16 * w + r);
            qc[e] = col_read(b + G::B_Q, 4 * g + e, 16 * w + r);
        }
        const f32x4_t b4 = ld4(b + G::B_B + 16 * g);
        const float br = reinterpret_cast<const float*>(b + G::B_B)[r];
        fence();
        // S^T -= U^T K: S^T at the chunk's start
#pragma unroll
        for (int i = 0; i < NT; ++i) {
            float uc[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) uc[e] = col_read(ub, 4 * g + e, 16 * i + r);
#pragma unroll
            for (int e = 0; e < 4; ++e) St[i] = mfma4(uc[e], -kc[e], St[i]);
        }
        // dQ = dO S^T, dK = U G^T - diag(beta) W S^T, and this wave's parts of dO U^T, W U^T
        f32x4_t qa[2] = {zero, zero}, ka[2] = {zero, zero};
        f32x4_t pp = zero, pa = zero;
#pragma unroll
        for (int i = 0; i < NT; ++i) {
            const f32x4_t dor = row_read(b + G::B_O, i);
            const f32x4_t wrw = row_read(b + G::B_W, i);
            const f32x4_t ur = row_read(ub, i);
            const f32x4_t nbw = wrw * -br;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                qa[e & 1] = mfma4(dor[e], St[i][e], qa[e & 1]);
                ka[e & 1] = mfma4(nbw[e], St[i][e], ka[e & 1]);
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
        // operands of the step after the next barrier, read while this chunk's buffer holds them
        const f32x4_t gram = ld4(b + G::B_G + 16 * lane);  // K K^T[4 g + v][r] = K K^T[r][4 g + v]
        lds_barrier();  // Y: the parts are in LDS
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
        wait_vm_n<0>();  // this wave's copies of the next staged chunk
        lds_barrier();   // Z: totals in LDS, the next chunk's copies landed
        // dQ += dP K; dK += dP^T Q + diag(beta) dA K + dA^T diag(beta) K
        const f32x4_t dpr = ld4(smem + G::OFF_TR + 16 * (4 * r + g));           // dP[r][4 g ..]
        const f32x4_t dar = ld4(smem + G::OFF_TR + 1024 + 16 * (4 * r + g));    // dA[r][4 g ..]
        const f32x4_t dpc = ld4(smem + G::OFF_TC + 4 * (20 * r + 4 * g));       // dP[4 g ..][r]
        const f32x4_t dac = ld4(smem + G::OFF_TC + 1280 + 4 * (20 * r + 4 * g)); // dA[4 g ..][r]
        f32x4_t dQ = qa[0] + qa[1], dK = ka[0] + ka[1];
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
            for (int ww = 0; ww < NW; ++ww) wx += reinterpret_cast<const float*>(smem + G::OFF_DB + (m * NW + ww) * 64)[r];
            if (g == 0) {
                const int clen = min(kC16, T - (c0 + m) * kC16);
                const __amdgpu_buffer_rsrc_t rb = make_rsrc(gbeta + (tok0 + (c0 + m) * kC16) * H + h,
                                                            static_cast<unsigned>(((clen - 1) * H + 1) * 4));
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(wx + sdg), rb, static_cast<unsigned>(r * H * 4),
                                                      0, 0);
            }
        }
    }
}

template <typename Kern>
hipError_t set_lds(Kern kern, int bytes) {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

// The history pass (K9a) and the sweep (K9b) are independent (both read only the
// records of K9p), and one workgroup of each fits on a CU (33 + 122 KiB of LDS at
// D = 128): K9a runs on a side stream of the library's (default priority, one per
// device, created on first use) between two events, forked from and joined back to the
// caller's stream, which also keeps the pair capturable in a graph.  The enqueueing is
// serialised across host threads; without the side stream the two run in order.
struct Side {
    hipStream_t s = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
    bool ok = false, tried = false;
};
std::mutex g_side_mu;
Side g_side[64];

Side* side_for_current_device() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    Side& sd = g_side[dev];
    if (!sd.tried) {
        sd.tried = true;
        sd.ok = hipStreamCreateWithFlags(&sd.s, hipStreamNonBlocking) == hipSuccess &&
                hipEventCreateWithFlags(&sd.fork, hipEventDisableTiming) == hipSuccess &&
                hipEventCreateWithFlags(&sd.join, hipEventDisableTiming) == hipSuccess;
    }
    return sd.ok ? &sd : nullptr;
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
    const float* q = static_cast<const float*>(a.q);
    const float* k = static_cast<const float*>(a.k);
    const float* v = static_cast<const float*>(a.v);
    hipError_t e;
    if ((e = set_lds(f32_bwd_sweep_kernel<D>, SwGeo<D>::BYTES)) != hipSuccess) return e;
    if ((e = set_lds(f32_bwd_span_kernel<D>, SpGeo<D>::BYTES)) != hipSuccess) return e;
    if (n_ch > 0 && (e = launch_f32_bwd_prep(q, k, a.beta, a.n_pairs, a.T, a.H, D, t2, rec, st)) != hipSuccess) return e;
    const int n_tiles = D / 32, slots = (a.n_pairs + 7) / 8;
    {
        std::lock_guard<std::mutex> lock(g_side_mu);
        Side* sd = n_ch > 0 ? side_for_current_device() : nullptr;
        if (sd) {
            if ((e = hipEventRecord(sd->fork, st)) != hipSuccess) return e;
            if ((e = hipStreamWaitEvent(sd->s, sd->fork, 0)) != hipSuccess) return e;
        }
        if (n_ch > 0 && (e = launch_f32_history(k, v, a.s0, a.n_pairs, a.T, a.H, D, t2, s_hist, sd ? sd->s : st)) !=
                            hipSuccess)
            return e;
        hipLaunchKernelGGL(f32_bwd_sweep_kernel<D>, dim3(static_cast<unsigned>(slots * n_tiles * 8)), dim3(256),
                           SwGeo<D>::BYTES, st, q, k, a.go, a.gs, a.gv, a.gs0, rec, w_ws, g_hist, a.n_pairs, a.T, a.H,
                           n_tiles, n_ch, n_span);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        if (sd) {
            if ((e = hipEventRecord(sd->join, sd->s)) != hipSuccess) return e;
            if ((e = hipStreamWaitEvent(st, sd->join, 0)) != hipSuccess) return e;
        }
    }
    if (n_ch == 0) return hipSuccess;
    hipLaunchKernelGGL(f32_bwd_span_kernel<D>, dim3(static_cast<unsigned>(a.n_pairs * n_span)), dim3(D * 4),
                       SpGeo<D>::BYTES, st, q, k, v, a.go, t2, rec, s_hist, g_hist, w_ws, a.gq, a.gk, a.gbeta, a.T,
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
    w.bytes = al(w.w + np * static_cast<size_t>(T) * D * 4);
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
