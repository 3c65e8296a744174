// delta_chunked_f32.hip — K7: the chunked forward for fp32 q/k/v on fp32 MFMA
// (v_mfma_f32_16x16x4f32), D in {64, 128}, in chunks of C = 16 tokens.
//
// The reference's recurrence (kernels/__init__.py:357-376 per token, :421-458 over
// the sequence) in the WY/UT chunk form, per chunk with start state S:
//   A = strict_lower(diag(beta) K K^T)     T = (I + A)^-1     T'' = -T diag(beta)
//   X = K S - V     U = T'' X  (= T diag(beta) (V - K S))
//   O = Q S + lower_incl_diag(Q K^T) U     S <- S + K^T U
// every product on fp32 MFMA with fp32 accumulation: fp32 arithmetic throughout.
//
// MFMA layout (lane l = 16 g + r): A operand A[r][g], B operand B[g][r], accumulator
// register v = D[4 g + v][r].  Each product's contraction index is mapped so that an
// operand which is itself a product comes straight from accumulator registers:
//   * over d (X = K S, Y = Q S): step (m, v) covers d = 16 m + 4 g + v, so register v
//     of S's accumulator tile m (rows 16 m ..) is the B operand, and lane (g, r) reads
//     K[r][16 m + 4 g .. + 3] as one float4 for the four steps of tile m;
//   * over tokens (U = T'' X, S += K^T U, O += P U): step v covers token 4 g + v, so
//     register v of X's or U's accumulator is the B operand, and the A operand M[r][4 g
//     + v] is register v of the accumulator of M^T.
//
// K7p (prep, one wave per (sequence, head, chunk), all chunks at once): G = K K^T and
// P^T = K Q^T from K and Q rows read straight into operand registers, N = -A and N^T
// from G (which is symmetric), and T^T = ((I+N)(I+N^2)(I+N^4)(I+N^8))^T (N is strictly
// lower triangular, so N^16 = 0) as products of accumulators with transposed
// accumulators.  It writes (T'')^T and (lower_incl P)^T as accumulator registers, 1 KiB
// each per chunk: the A operands of U = T'' X and of P U, lane-linear.
//
// K7 (recurrence): one workgroup per (sequence, head, d_v tile of DV columns) with DV/16
// chain waves and as many output waves.  Chain wave w owns the S columns col0 + 16 w +
// [0, 16) as D/16 accumulator tiles and runs chunk i (X, U, S: 68 MFMAs at D = 128),
// handing S_i (before its update) and U_i to output wave w through LDS; output wave w
// runs chunk i - 1 (Y = Q S, O = Y + P U) and stores O.  HBM -> LDS copies
// (buffer_load ... lds) run two chunks ahead: the output waves copy K and Q rows and
// P^T, the chain waves their V columns and (wave 0) T''^T.  One LDS-only barrier per
// chunk.

#include "pm_cdna4.h"
#include "pm_internal.h"

namespace pm {
namespace {

constexpr int kC16 = 16;          // tokens per chunk
constexpr int kWsFloats = 512;    // workspace floats per chunk: (T'')^T, then P^T

__device__ __forceinline__ f32x4_t mfma4(float a, float b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
// Left * Right over a 16-token contraction, given the accumulators of Left^T and Right.
__device__ __forceinline__ f32x4_t mm16(f32x4_t lt, f32x4_t r) {
    f32x4_t a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int v = 0; v < 4; ++v) a = mfma4(lt[v], r[v], a);
    return a;
}

// Workspace slots (16-token chunks), as the split form's: fixed length, row = pair, slot
// = c; varlen, row = h and slot = floor(tok0 / 16) + seq + c (consecutive sequences never
// share a slot).
__host__ __device__ inline int f32_n_slot(bool varlen, int T, int n_seq) {
    return varlen ? (T + kC16 - 1) / kC16 + n_seq : (T + kC16 - 1) / kC16;
}

// LDS tile of 16 fp32 token rows of D values: the 16-byte chunk p of row t is stored at
// chunk t * (D / 4) + (p ^ t).  With it the float4 operand reads (lane (g, r): row r,
// chunk 4 m + g) and the column reads of K^T (lane (g, r): row 4 g + v, element 16 m + r)
// fall in distinct banks across each quarter wave.
template <int D>
__device__ __forceinline__ int f32_chunk(int t, int p) {
    return t * (D / 4) + (p ^ t);
}

// ---------------------------------------------------------------- K7p
template <int D>
__global__ __launch_bounds__(256) void delta_f32_prep_kernel(const float* __restrict__ q,
                                                             const float* __restrict__ k,
                                                             const float* __restrict__ beta,
                                                             const int32_t* __restrict__ cu_seqlens,
                                                             int n_seq, int T, int H, int n_slot, long n_items,
                                                             float* __restrict__ ws) {
    constexpr int NJ = D / 16;
    const int lane = threadIdx.x & 63;
    const long item = static_cast<long>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (item >= n_items) return;
    const int row = static_cast<int>(item / n_slot), slot = static_cast<int>(item % n_slot);
    int seq, h, c, len;
    long tok0;
    if (cu_seqlens) {
        h = row;
        // the sequence whose slot range starts at or before `slot`: the largest s with
        // floor(cu[s] / 16) + s <= slot (non-decreasing in s)
        int lo = 0, hi = n_seq - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            const int a = min(max(cu_seqlens[mid], 0), T);
            if (a / kC16 + mid <= slot) lo = mid; else hi = mid - 1;
        }
        seq = lo;
        const int a = min(max(cu_seqlens[seq], 0), T);
        const int z = min(max(cu_seqlens[seq + 1], a), T);
        tok0 = a;
        len = z - a;
        c = slot - (a / kC16 + seq);
        if (c < 0 || c * kC16 >= len) return;
    } else {
        seq = row / H;
        h = row % H;
        tok0 = static_cast<long>(seq) * T;
        len = T;
        c = slot;
    }
    const int r = lane & 15, g = lane >> 4;
    const int base = c * kC16, clen = min(kC16, len - base);
    const size_t tstride = static_cast<size_t>(H) * D;
    const size_t row0 = static_cast<size_t>(tok0 + base) * tstride + static_cast<size_t>(h) * D;
    const unsigned nb = static_cast<unsigned>(((clen - 1) * tstride + D) * 4);
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(k + row0, nb), rq = make_rsrc(q + row0, nb);
    const __amdgpu_buffer_rsrc_t rb =
        make_rsrc(beta + (tok0 + base) * H + h, static_cast<unsigned>(((clen - 1) * H + 1) * 4));
    f32x4_t kf[NJ], qf[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const unsigned vo = static_cast<unsigned>((r * tstride + 16 * j + 4 * g) * 4);
        kf[j] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rk, vo, 0, 0));
        qf[j] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rq, vo, 0, 0));
    }
    const float bc = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rb, static_cast<unsigned>(r * H * 4), 0, 0));
    f32x4_t bt;
#pragma unroll
    for (int v = 0; v < 4; ++v)
        bt[v] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rb, static_cast<unsigned>((4 * g + v) * H * 4), 0, 0));

    // G = K K^T and P^T = K Q^T (two accumulators each, summed at the end)
    const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
    f32x4_t g0 = zero, g1 = zero, p0 = zero, p1 = zero;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            if (j & 1) {
                g1 = mfma4(kf[j][v], kf[j][v], g1);
                p1 = mfma4(kf[j][v], qf[j][v], p1);
            } else {
                g0 = mfma4(kf[j][v], kf[j][v], g0);
                p0 = mfma4(kf[j][v], qf[j][v], p0);
            }
        }
    }
    const f32x4_t G = g0 + g1, Pt = p0 + p1;
    // N[i][j] = -beta_i G[i][j] (i > j), N^T[i][j] = -beta_j G[i][j] (j > i); i = 4 g + v, j = r
    f32x4_t N, Nt, eye;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int i = 4 * g + v;
        N[v] = i > r ? -bt[v] * G[v] : 0.f;
        Nt[v] = r > i ? -bc * G[v] : 0.f;
        eye[v] = i == r ? 1.f : 0.f;
    }
    const f32x4_t N2 = mm16(Nt, N), N2t = mm16(N, Nt);
    const f32x4_t N4 = mm16(N2t, N2), N4t = mm16(N2, N2t);
    const f32x4_t N8 = mm16(N4t, N4);
    const f32x4_t F1t = mm16(eye + N2, eye + Nt);   // ((I+N)(I+N^2))^T
    const f32x4_t F2t = mm16(eye + N4, F1t);        // (... (I+N^4))^T
    const f32x4_t Tt = mm16(eye + N8, F2t);         // T^T
    f32x4_t tw, pw;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        tw[v] = -bt[v] * Tt[v];                     // (T'')^T[i][j] = -beta_i T[j][i]
        pw[v] = (4 * g + v <= r) ? Pt[v] : 0.f;     // P^T[i][j] = P[j][i], kept for i <= j
    }
    float* out = ws + (static_cast<size_t>(row) * n_slot + slot) * kWsFloats + lane * 4;
    *reinterpret_cast<f32x4_t*>(out) = tw;
    *reinterpret_cast<f32x4_t*>(out + 256) = pw;
}

// ---------------------------------------------------------------- K7
template <int D, int DV>
struct F32Geo {
    static constexpr int NCW = DV / 16;            // chain waves 0 .. NCW-1, output waves NCW ..
    static constexpr int NT = D / 16;              // S accumulator tiles per chain wave
    static constexpr int NI = kC16 * D * 4 / 1024; // 1 KiB copies per K or Q tile
    static constexpr int NB = 4;                   // rotating chunk buffers
    // one chunk buffer: K rows, Q rows, P^T, (T'')^T, V columns of each chain wave
    static constexpr int B_K = 0;
    static constexpr int B_Q = B_K + kC16 * D * 4;
    static constexpr int B_P = B_Q + kC16 * D * 4;
    static constexpr int B_T = B_P + 1024;
    static constexpr int B_V = B_T + 1024;
    static constexpr int BUF = B_V + NCW * 1024;
    static constexpr int OFF_S = NB * BUF;                     // 2 slots x NCW x NT KiB: S_i
    static constexpr int OFF_U = OFF_S + 2 * NCW * NT * 1024;  // 2 slots x NCW KiB: U_i
    static constexpr int BYTES = OFF_U + 2 * NCW * 1024;
    // copies per chunk: output wave 0 (K, P^T and, with one output wave, Q), output wave 1
    // (Q); chain wave 0 (V, T''), chain wave 1 (V)
    static constexpr int NCP_O0 = NI + 1 + (NCW == 1 ? NI : 0);
    static constexpr int NCP_O1 = NI;
    static constexpr int NST = 4;  // O stores per output wave per chunk
    static_assert(D == 64 || D == 128, "D");
    static_assert(DV == 16 || DV == 32, "DV");
    static_assert(BYTES <= 160 * 1024 && NCP_O0 + NST <= 63, "LDS / vmcnt");
};

template <int D, int DV, bool OUT_BF16>
__global__ __launch_bounds__(DV == 32 ? 256 : 128) void delta_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ s0, void* __restrict__ o_out, float* __restrict__ s_out,
    const int32_t* __restrict__ cu_seqlens, const float* __restrict__ ws, int n_pairs, int T, int H,
    int n_tiles, int n_slot) {
    using G = F32Geo<D, DV>;
    constexpr int NCW = G::NCW, NT = G::NT;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

    // XCD-aware placement: the n_tiles workgroups of a pair share bid % 8
    const int bid = blockIdx.x;
    const int xcd = bid & 7, bslot = bid >> 3;
    const int tile = bslot % n_tiles;
    const int pair = (bslot / n_tiles) * 8 + xcd;
    if (pair >= n_pairs) return;
    const int seq = pair / H, h = pair % H;
    long tok0;
    int len;
    if (cu_seqlens) {
        const int a = min(max(cu_seqlens[seq], 0), T);
        const int z = min(max(cu_seqlens[seq + 1], a), T);
        tok0 = a;
        len = z - a;
    } else {
        tok0 = static_cast<long>(seq) * T;
        len = T;
    }
    const int col0 = tile * DV;
    const int n_chunks = (len + kC16 - 1) / kC16;
    const int ws_row = cu_seqlens ? h : pair;
    const int ws_slot0 = cu_seqlens ? static_cast<int>(tok0 / kC16) + seq : 0;

    const int lane = threadIdx.x & 63;
    const int w = static_cast<int>(uniform(static_cast<unsigned>(threadIdx.x >> 6)));
    const int r = lane & 15, g = lane >> 4;
    const bool chain = w < NCW;
    const int cw = chain ? w : w - NCW;  // the 16 columns this wave works on
    const size_t tstride = static_cast<size_t>(H) * D;
    const size_t sbase = static_cast<size_t>(pair) * D * D;
    const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};

    auto buf = [&](int c) { return smem + (c % G::NB) * G::BUF; };
    auto sslot = [&](int c, int which) { return smem + G::OFF_S + ((c & 1) * NCW + which) * NT * 1024; };
    auto uslot = [&](int c, int which) { return smem + G::OFF_U + ((c & 1) * NCW + which) * 1024; };
    auto ld4 = [&](const unsigned char* p) { return *reinterpret_cast<const f32x4_t*>(p); };
    auto st4 = [&](unsigned char* p, f32x4_t x) { *reinterpret_cast<f32x4_t*>(p) = x; };

    // ---- HBM -> LDS copies of chunk c (c < n_chunks) ----
    auto chunk_rsrc = [&](const float* base, int c, int row_floats, int col) {
        const int clen = min(kC16, len - c * kC16);
        const size_t row0 = static_cast<size_t>(tok0 + c * kC16) * tstride + static_cast<size_t>(h) * D + col;
        return make_rsrc(base + row0, static_cast<unsigned>(((clen - 1) * tstride + row_floats) * 4));
    };
    auto copy_tile = [&](const float* base, int c, unsigned char* dst) __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t rs = chunk_rsrc(base, c, D, 0);
        unsigned char* d0 = uniform_ptr(dst);
#pragma unroll
        for (int i = 0; i < G::NI; ++i) {
            const int qc = 64 * i + lane;  // LDS chunk
            const int t = qc / (D / 4), p = (qc % (D / 4)) ^ t;
            dma16_asm(rs, d0 + 1024 * i, static_cast<unsigned>(t * tstride * 4 + 16 * p));
        }
    };
    auto copy_ws = [&](int c, int part, unsigned char* dst) __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(
            ws + (static_cast<size_t>(ws_row) * n_slot + ws_slot0 + c) * kWsFloats + 256 * part, 1024);
        dma16_asm(rs, uniform_ptr(dst), static_cast<unsigned>(16 * lane));
    };
    auto copy_v = [&](int c, unsigned char* dst) __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t rs = chunk_rsrc(v, c, 16, col0 + 16 * cw);
        const int t = lane >> 2, p = lane & 3;
        dma16_asm(rs, uniform_ptr(dst), static_cast<unsigned>(t * tstride * 4 + 16 * p));
    };
    // this wave's copies of chunk c
    auto copies = [&](int c) __attribute__((always_inline)) {
        unsigned char* b = buf(c);
        if (chain) {
            copy_v(c, b + G::B_V + 1024 * cw);
            if (cw == 0) copy_ws(c, 0, b + G::B_T);
        } else if (cw == 0) {
            copy_tile(k, c, b + G::B_K);
            copy_ws(c, 1, b + G::B_P);
            if (NCW == 1) copy_tile(q, c, b + G::B_Q);
        } else {
            copy_tile(q, c, b + G::B_Q);
        }
    };
    // wait until chunk c's copies (issued before `extra` later operations) have landed
    auto wait_own = [&](int extra_stores, bool extra_copies) __attribute__((always_inline)) {
        if (chain) {
            if (!extra_copies) wait_vm_n<0>();
            else if (cw == 0) wait_vm_n<2>();
            else wait_vm_n<1>();
        } else if (cw == 0) {
            if (extra_copies && extra_stores) wait_vm_n<G::NCP_O0 + G::NST>();
            else if (extra_copies) wait_vm_n<G::NCP_O0>();
            else if (extra_stores) wait_vm_n<G::NST>();
            else wait_vm_n<0>();
        } else {
            if (extra_copies && extra_stores) wait_vm_n<G::NCP_O1 + G::NST>();
            else if (extra_copies) wait_vm_n<G::NCP_O1>();
            else if (extra_stores) wait_vm_n<G::NST>();
            else wait_vm_n<0>();
        }
    };

    if (n_chunks > 0) {
        copies(0);
        if (n_chunks > 1) copies(1);
        wait_own(0, n_chunks > 1);
        lds_barrier();  // B0
    }

    if (chain) {
        // ============ chain wave: S columns col0 + 16 cw + [0, 16) ============
        const int ecol = col0 + 16 * cw + r;
        f32x4_t S[NT];
#pragma unroll
        for (int m = 0; m < NT; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                S[m][e] = s0 ? s0[sbase + static_cast<size_t>(16 * m + 4 * g + e) * D + ecol] : 0.f;
        for (int i = 0; i < n_chunks; ++i) {
            const bool cp = i + 2 < n_chunks;
            if (cp) copies(i + 2);
            const unsigned char* b = buf(i);
            const float* Kf = reinterpret_cast<const float*>(b + G::B_K);
            const float* Vf = reinterpret_cast<const float*>(b + G::B_V + 1024 * cw);
            // X = K S - V (two accumulators over alternate tiles)
            f32x4_t x0, x1 = zero;
#pragma unroll
            for (int e = 0; e < 4; ++e) x0[e] = -Vf[(4 * g + e) * 16 + r];
#pragma unroll
            for (int m = 0; m < NT; ++m) {
                const f32x4_t kf = ld4(b + G::B_K + 16 * f32_chunk<D>(r, 4 * m + g));
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (m & 1) x1 = mfma4(kf[e], S[m][e], x1);
                    else x0 = mfma4(kf[e], S[m][e], x0);
                }
            }
            const f32x4_t X = x0 + x1;
            // U = T'' X
            const f32x4_t tt = ld4(b + G::B_T + 16 * lane);
            const f32x4_t U = mm16(tt, X);
            // hand S_i and U_i to the output wave
            unsigned char* ss = sslot(i, cw);
#pragma unroll
            for (int m = 0; m < NT; ++m) st4(ss + 1024 * m + 16 * lane, S[m]);
            st4(uslot(i, cw) + 16 * lane, U);
            // S += K^T U: A operand K[4 g + e][16 m + r]
#pragma unroll
            for (int m = 0; m < NT; ++m) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int t = 4 * g + e, d = 16 * m + r;
                    const float kt = Kf[4 * f32_chunk<D>(t, d >> 2) + (d & 3)];
                    S[m] = mfma4(kt, U[e], S[m]);
                }
            }
            if (i + 1 < n_chunks) wait_own(0, cp);
            lds_barrier();
        }
#pragma unroll
        for (int m = 0; m < NT; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e) s_out[sbase + static_cast<size_t>(16 * m + 4 * g + e) * D + ecol] = S[m][e];
    } else if (n_chunks > 0) {
        // ============ output wave: O of chunk i - 1 for the columns of chain wave cw ============
        constexpr int ES = OUT_BF16 ? 2 : 4;
        for (int i = 0; i <= n_chunks; ++i) {
            const bool cp = i + 2 < n_chunks;
            if (cp) copies(i + 2);
            const bool st = i >= 1;
            if (st) {
                const int c = i - 1;
                const unsigned char* b = buf(c);
                const unsigned char* ss = sslot(c, cw);
                f32x4_t y0 = zero, y1 = zero;
#pragma unroll
                for (int m = 0; m < NT; ++m) {
                    const f32x4_t qf = ld4(b + G::B_Q + 16 * f32_chunk<D>(r, 4 * m + g));
                    const f32x4_t sc = ld4(ss + 1024 * m + 16 * lane);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if (m & 1) y1 = mfma4(qf[e], sc[e], y1);
                        else y0 = mfma4(qf[e], sc[e], y0);
                    }
                }
                const f32x4_t pt = ld4(b + G::B_P + 16 * lane);
                const f32x4_t u = ld4(uslot(c, cw) + 16 * lane);
                f32x4_t O = y0 + y1;
#pragma unroll
                for (int e = 0; e < 4; ++e) O = mfma4(pt[e], u[e], O);
                // lane (g, r) holds O[4 g + e][16 cw + r]; rows past the end are dropped by
                // the range-checked stores
                const int clen = min(kC16, len - c * kC16);
                const size_t rowe = static_cast<size_t>(tok0 + c * kC16) * tstride + static_cast<size_t>(h) * D +
                                    col0 + 16 * cw;
                const __amdgpu_buffer_rsrc_t ro = make_rsrc(static_cast<unsigned char*>(o_out) + rowe * ES,
                                                            static_cast<unsigned>(((clen - 1) * tstride + 16) * ES));
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const unsigned off = static_cast<unsigned>(((4 * g + e) * tstride + r) * ES);
                    if constexpr (OUT_BF16)
                        __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(O[e]), ro, off, 0, 0);
                    else
                        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(O[e]), ro, off, 0, 0);
                }
            }
            if (i < n_chunks) {
                if (i + 1 < n_chunks) wait_own(st, cp);
                lds_barrier();
            }
        }
    }
}

template <typename K>
hipError_t set_lds_f32(K kern, int bytes) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    static bool done[64] = {};
    if (dev >= 0 && dev < 64 && done[dev]) return hipSuccess;
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess && dev >= 0 && dev < 64) done[dev] = true;
    return e;
}

template <int D, int DV, bool OB>
hipError_t launch_f32_t(const ChunkedF32Args& a, float* ws, hipStream_t st) {
    using G = F32Geo<D, DV>;
    const bool varlen = a.cu_seqlens != nullptr;
    const int n_pairs = a.n_seq * a.H;
    const int n_slot = f32_n_slot(varlen, a.T, a.n_seq);
    const long n_items = static_cast<long>(varlen ? a.H : n_pairs) * n_slot;
    const float *q = a.q, *k = a.k, *v = a.v;
    if (n_items > 0) {
        hipLaunchKernelGGL(delta_f32_prep_kernel<D>, dim3(static_cast<unsigned>((n_items + 3) / 4)), dim3(256), 0,
                           st, q, k, a.beta, a.cu_seqlens, a.n_seq, a.T, a.H, n_slot, n_items, ws);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    auto kern = delta_f32_kernel<D, DV, OB>;
    hipError_t e = set_lds_f32(kern, G::BYTES);
    if (e != hipSuccess) return e;
    const int n_tiles = D / DV;
    const int slots = (n_pairs + 7) / 8;
    hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(slots * n_tiles * 8)), dim3(128 * G::NCW), G::BYTES, st, q, k,
                       v, a.s0, a.o, a.s_out, a.cu_seqlens, ws, n_pairs, a.T, a.H, n_tiles, n_slot);
    return hipGetLastError();
}

template <int D, int DV>
hipError_t launch_f32_dv(const ChunkedF32Args& a, float* ws, hipStream_t st) {
    return a.out_bf16 ? launch_f32_t<D, DV, true>(a, ws, st) : launch_f32_t<D, DV, false>(a, ws, st);
}

}  // namespace

size_t chunked_f32_ws_bytes(bool varlen, int n_seq, int T, int H) {
    const long rows = varlen ? H : static_cast<long>(n_seq) * H;
    return static_cast<size_t>(rows) * f32_n_slot(varlen, T, n_seq) * kWsFloats * 4;
}

int chunked_f32_pick_tile(int D, long n_pairs, int requested) {
    if (requested == 16 || requested == 32) return requested;
    if (requested == 64) return 32;
    return n_pairs * (D / 32) >= 256 ? 32 : 16;
}

hipError_t launch_chunked_f32(const ChunkedF32Args& a, void* ws, hipStream_t st) {
    if (a.n_seq == 0 || a.H == 0) return hipSuccess;
    float* w = static_cast<float*>(ws);
    const int dv = chunked_f32_pick_tile(a.D, static_cast<long>(a.n_seq) * a.H, a.dv_tile);
    if (a.D == 128) return dv == 16 ? launch_f32_dv<128, 16>(a, w, st) : launch_f32_dv<128, 32>(a, w, st);
    return dv == 16 ? launch_f32_dv<64, 16>(a, w, st) : launch_f32_dv<64, 32>(a, w, st);
}

}  // namespace pm
