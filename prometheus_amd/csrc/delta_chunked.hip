// delta_chunked.hip — K1/K2: chunked WY/UT delta-rule forward on bf16 MFMA.
//
// Same recurrence as the reference (kernels/__init__.py:357-376 per token,
// :421-458 over the sequence), restated per chunk of C = 64 tokens with
// start state S (d_k x d_v), rows K, V, Q and gates beta:
//
//   A = strict_lower(diag(beta) K K^T)      T = (I + A)^-1   (unit lower)
//   U = T diag(beta) (V - K S)              u_t = beta_t (v_t - S_{t-1}^T k_t)
//   O = Q S + lower_incl_diag(Q K^T) U      o_t = q_t S_t
//   S <- S + K^T U
//
// (DeltaNet chunk form, Yang et al. 2024; W = T diag(beta) K is never
// formed: T is applied to diag(beta)(V - K S), which keeps every per-chunk
// product that depends on K alone independent of the d_v columns.)
//
// Work split.  The recurrence is separable along d_v: columns of S, U, V
// and O never mix.  One 256-thread workgroup owns (sequence, head, d_v tile
// of DV columns) and walks that sequence's chunks in order; the DV/16
// "chain" waves each own 16 columns of S in MFMA accumulators.  All four
// waves build the column-independent chunk data (K K^T, Q K^T, T) in LDS.
// Workgroups of one (sequence, head) are placed on one XCD (blocks are
// dispatched round-robin over the 8 XCDs) so their shared Q/K reads hit
// the same L2.
//
// Register-resident chain.  v_mfma_f32_16x16x32_bf16 contracts 32 values
// per lane group; since the contraction is invariant under any permutation
// of its index applied to both operands, lane group g's 8 slots are mapped
// to indices {4g..4g+3} and {16+4g..16+4g+3} of each 32-block.  With that
// mapping two stacked 16x16 fp32 accumulator tiles, converted to bf16, are
// exactly the B operand of the next product: S -> K S, R -> T R,
// U -> P U and K^T U need no LDS round trip.  A operands are read from LDS
// as two 8-byte pieces per lane with the same mapping.  (The 16x16x16 form
// used for T has 4 slots, and an accumulator tile is its B operand as is.)
//
// Numerics: q/k/v bf16, every product fp32-accumulated; T, P, R, U and the
// MFMA copy of S are rounded to bf16; S itself is carried in fp32.

#include "pm_common.h"
#include "pm_internal.h"

namespace pm {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kC = 64;  // chunk length (tokens)

__device__ __forceinline__ f32x4_t mfma32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4_t mfma16(u32x2_t a, u32x2_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(bf16x4_t, a),
                                                     __builtin_bit_cast(bf16x4_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ uint16_t bf16_bits(float x) {
    return __builtin_bit_cast(uint16_t, (__bf16)x);
}
// bf16 operands are assembled from 16-bit patterns packed into 32-bit
// words and bit-cast to the MFMA vector type only at the call: element
// access on bf16 vectors (extract or insert) is avoided on purpose, since
// hipcc (ROCm 7.2) miscompiled an element extract feeding a 16-bit LDS store.
__device__ __forceinline__ unsigned pack2(float a, float b) {
    return static_cast<unsigned>(bf16_bits(a)) | (static_cast<unsigned>(bf16_bits(b)) << 16);
}
__device__ __forceinline__ u32x2_t cvt4(f32x4_t x) {
    const u32x2_t r = {pack2(x.x, x.y), pack2(x.z, x.w)};
    return r;
}
// Two stacked accumulator tiles (rows 0-15 and 16-31 of a 32-block) as a B operand.
__device__ __forceinline__ bf16x8_t acc_to_b(f32x4_t lo, f32x4_t hi) {
    const u32x4_t r = {pack2(lo.x, lo.y), pack2(lo.z, lo.w), pack2(hi.x, hi.y), pack2(hi.z, hi.w)};
    return __builtin_bit_cast(bf16x8_t, r);
}

// A operand of a 16x16x32 product from a row-major bf16 LDS matrix:
// row `row`, contraction block starting at k0, lane group g.
__device__ __forceinline__ bf16x8_t lds_a(const uint16_t* m, int pitch, int row, int k0, int g) {
    const uint16_t* p = m + row * pitch + k0 + 4 * g;
    const u32x2_t lo = *reinterpret_cast<const u32x2_t*>(p);
    const u32x2_t hi = *reinterpret_cast<const u32x2_t*>(p + 16);
    const u32x4_t v = {lo.x, lo.y, hi.x, hi.y};
    return __builtin_bit_cast(bf16x8_t, v);
}

__device__ __forceinline__ void wave_lds_fence() {
    // orders this wave's LDS writes before its later LDS reads
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

__device__ __forceinline__ uint16_t half_of(u32x4_t v, int j) {
    const unsigned w = v[j >> 1];
    return static_cast<uint16_t>((j & 1) ? (w >> 16) : (w & 0xffffu));
}

template <int D, int DV>
struct Geo {
    static constexpr int NCW = DV / 16;         // chain waves
    static constexpr int PK = D + 8;            // Ks/Qs pitch (bf16)
    static constexpr int PT = kC + 8;           // Kt/Vt/Tm/Pm pitch (bf16)
    static constexpr int PA = kC + 4;           // Af pitch (fp32)
    static constexpr int PD = 24;               // Dw pitch (bf16)
    static constexpr int TPT = D / 32;          // K/Q tokens per thread per chunk
    static constexpr int DG = D / 8;            // 16-byte groups per token row
    static constexpr int VG = DV / 8;           // 16-byte groups per V tile row
    static constexpr int VPT = (kC * VG + 255) / 256;
    static constexpr int OFF_KS = 0;
    static constexpr int OFF_QS = OFF_KS + kC * PK * 2;
    static constexpr int OFF_KT = OFF_QS + kC * PK * 2;
    static constexpr int OFF_VT = OFF_KT + D * PT * 2;
    static constexpr int OFF_TM = OFF_VT + DV * PT * 2;
    static constexpr int OFF_PM = OFF_TM + kC * PT * 2;
    static constexpr int OFF_AF = OFF_PM + kC * PT * 2;
    static constexpr int OFF_BS = OFF_AF + kC * PA * 4;
    static constexpr int OFF_DW = OFF_BS + kC * 4;
    static constexpr int BYTES = OFF_DW + 4 * 4 * 16 * PD * 2;
    static_assert(D % 32 == 0 && D <= 128, "D");
    static_assert(DV % 16 == 0 && DV <= 64 && D % DV == 0, "DV");
    static_assert(kC * DG == 256 * TPT, "K/Q load split");
};

template <int D, int DV, bool OUT_BF16>
__global__ __launch_bounds__(256) void delta_chunked_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const float* __restrict__ beta,
    const float* __restrict__ s0, void* __restrict__ o_out, float* __restrict__ s_out,
    const int32_t* __restrict__ cu_seqlens, int n_pairs, int T, int H, int n_tiles) {
    using G = Geo<D, DV>;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    uint16_t* Ks = reinterpret_cast<uint16_t*>(smem + G::OFF_KS);
    uint16_t* Qs = reinterpret_cast<uint16_t*>(smem + G::OFF_QS);
    uint16_t* Kt = reinterpret_cast<uint16_t*>(smem + G::OFF_KT);
    uint16_t* Vt = reinterpret_cast<uint16_t*>(smem + G::OFF_VT);
    uint16_t* Tm = reinterpret_cast<uint16_t*>(smem + G::OFF_TM);
    uint16_t* Pm = reinterpret_cast<uint16_t*>(smem + G::OFF_PM);
    float* Af = reinterpret_cast<float*>(smem + G::OFF_AF);
    float* Bs = reinterpret_cast<float*>(smem + G::OFF_BS);
    uint16_t* Dw = reinterpret_cast<uint16_t*>(smem + G::OFF_DW);

    // XCD-aware placement: the n_tiles workgroups of a pair share bid % 8.
    const int bid = blockIdx.x;
    const int xcd = bid & 7, slot = bid >> 3;
    const int tile = slot % n_tiles;
    const int pair = (slot / n_tiles) * 8 + xcd;
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

    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int l16 = lane & 15, lg = lane >> 4;
    const bool chain = w < G::NCW;
    const size_t sbase = static_cast<size_t>(pair) * D * D;
    const size_t tstride = static_cast<size_t>(H) * D;  // elements between tokens

    // ---- state: chain wave w owns columns col0 + 16w + [0, 16) ----
    f32x4_t S[D / 16];
    const int ecol = col0 + 16 * w + l16;
#pragma unroll
    for (int md = 0; md < D / 16; ++md) {
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            const int d = 16 * md + 4 * lg + ii;
            S[md][ii] = (chain && s0) ? s0[sbase + static_cast<size_t>(d) * D + ecol] : 0.f;
        }
    }
    bf16x8_t Sb[D / 32];
#pragma unroll
    for (int kb = 0; kb < D / 32; ++kb) Sb[kb] = acc_to_b(S[2 * kb], S[2 * kb + 1]);

    // ---- chunk input staging (global -> registers -> LDS) ----
    const int dg = tid % G::DG, tg = tid / G::DG;
    u32x4_t kr[G::TPT], qr[G::TPT], vr[G::VPT];
    float br = 0.f;
    auto load_chunk = [&](int c) {
        const int base = c * kC;
        const int clen = min(kC, len - base);
#pragma unroll
        for (int i = 0; i < G::TPT; ++i) {
            const int t = tg * G::TPT + i;
            const u32x4_t z = {0u, 0u, 0u, 0u};
            kr[i] = z;
            qr[i] = z;
            if (t < clen) {
                const size_t a = (tok0 + base + t) * tstride + static_cast<size_t>(h) * D + dg * 8;
                kr[i] = *reinterpret_cast<const u32x4_t*>(k + a);
                qr[i] = *reinterpret_cast<const u32x4_t*>(q + a);
            }
        }
#pragma unroll
        for (int i = 0; i < G::VPT; ++i) {
            const int idx = tid + 256 * i;
            const int t = idx / G::VG, cv = idx % G::VG;
            const u32x4_t z = {0u, 0u, 0u, 0u};
            vr[i] = z;
            if (idx < kC * G::VG && t < clen) {
                const size_t a = (tok0 + base + t) * tstride + static_cast<size_t>(h) * D + col0 + cv * 8;
                vr[i] = *reinterpret_cast<const u32x4_t*>(v + a);
            }
        }
        br = (tid < clen) ? beta[(tok0 + base + tid) * H + h] : 0.f;
    };
    auto store_chunk = [&]() {
#pragma unroll
        for (int i = 0; i < G::TPT; ++i) {
            const int t = tg * G::TPT + i;
            *reinterpret_cast<u32x4_t*>(Ks + t * G::PK + dg * 8) = kr[i];
            *reinterpret_cast<u32x4_t*>(Qs + t * G::PK + dg * 8) = qr[i];
        }
        // K^T: d-major rows, the TPT tokens of this thread contiguous
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint16_t* dst = Kt + (dg * 8 + j) * G::PT + tg * G::TPT;
            if constexpr (G::TPT == 4) {
                const u32x2_t pk = {half_of(kr[0], j) | (static_cast<unsigned>(half_of(kr[1], j)) << 16),
                                    half_of(kr[2], j) | (static_cast<unsigned>(half_of(kr[3], j)) << 16)};
                *reinterpret_cast<u32x2_t*>(dst) = pk;
            } else {
                static_assert(G::TPT == 2, "TPT");
                *reinterpret_cast<unsigned*>(dst) =
                    half_of(kr[0], j) | (static_cast<unsigned>(half_of(kr[1], j)) << 16);
            }
        }
#pragma unroll
        for (int i = 0; i < G::VPT; ++i) {
            const int idx = tid + 256 * i;
            if (idx < kC * G::VG) {
                const int t = idx / G::VG, cv = idx % G::VG;
#pragma unroll
                for (int j = 0; j < 8; ++j) Vt[(cv * 8 + j) * G::PT + t] = half_of(vr[i], j);
            }
        }
        if (tid < kC) Bs[tid] = br;
    };

    const int n_chunks = (len + kC - 1) / kC;
    if (n_chunks > 0) load_chunk(0);

    for (int c = 0; c < n_chunks; ++c) {
        const int base = c * kC;
        const int clen = min(kC, len - base);
        __syncthreads();  // previous chunk's LDS reads are done
        store_chunk();
        if (c + 1 < n_chunks) load_chunk(c + 1);
        __syncthreads();

        // ---- phase G: row block w of G = K K^T and P = Q K^T (lower blocks) ----
        {
            bf16x8_t aK[D / 32], aQ[D / 32];
#pragma unroll
            for (int kb = 0; kb < D / 32; ++kb) {
                aK[kb] = lds_a(Ks, G::PK, 16 * w + l16, 32 * kb, lg);
                aQ[kb] = lds_a(Qs, G::PK, 16 * w + l16, 32 * kb, lg);
            }
#pragma unroll
            for (int bj = 0; bj < 4; ++bj) {
                if (bj > w) break;
                f32x4_t g = {0.f, 0.f, 0.f, 0.f}, p = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kb = 0; kb < D / 32; ++kb) {
                    const bf16x8_t bK = lds_a(Ks, G::PK, 16 * bj + l16, 32 * kb, lg);
                    g = mfma32(aK[kb], bK, g);
                    p = mfma32(aQ[kb], bK, p);
                }
                const int col = 16 * bj + l16;
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) {
                    const int row = 16 * w + 4 * lg + ii;
                    Af[row * G::PA + col] = (row > col) ? Bs[row] * g[ii] : 0.f;
                    Pm[row * G::PT + col] = (row >= col) ? bf16_bits(p[ii]) : uint16_t(0);
                }
            }
            if ((w & 1) == 0) {  // upper block (w, w+1) of P is read by O = P U
#pragma unroll
                for (int ii = 0; ii < 4; ++ii)
                    Pm[(16 * w + 4 * lg + ii) * G::PT + 16 * (w + 1) + l16] = 0;
            }
        }
        // chain waves: X = K S and Y = Q S for their 16 columns
        f32x4_t X[4], Y[4];
        if (chain) {
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                f32x4_t x = {0.f, 0.f, 0.f, 0.f}, y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kb = 0; kb < D / 32; ++kb) {
                    x = mfma32(lds_a(Ks, G::PK, 16 * m + l16, 32 * kb, lg), Sb[kb], x);
                    y = mfma32(lds_a(Qs, G::PK, 16 * m + l16, 32 * kb, lg), Sb[kb], y);
                }
                X[m] = x;
                Y[m] = y;
            }
        }
        __syncthreads();

        // ---- phase T: wave j builds column block j of T = (I + A)^-1 ----
        {
            // rows of the four 16x16 diagonal inverses, lane group g = block
            float yv[16];
#pragma unroll
            for (int cc = 0; cc < 16; ++cc) yv[cc] = (cc == l16) ? 1.f : 0.f;
            const float* Ablk = Af + (16 * lg) * G::PA + 16 * lg;
#pragma unroll
            for (int cc = 14; cc >= 0; --cc) {
                float acc = yv[cc];
#pragma unroll
                for (int kk = cc + 1; kk < 16; ++kk) acc = fmaf(-Ablk[kk * G::PA + cc], yv[kk], acc);
                yv[cc] = acc;
            }
            uint16_t* dw = Dw + ((w * 4 + lg) * 16 + l16) * G::PD;
            u32x4_t r0, r1;
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                r0[cc] = bf16_bits(yv[2 * cc]) | (static_cast<unsigned>(bf16_bits(yv[2 * cc + 1])) << 16);
                r1[cc] = bf16_bits(yv[8 + 2 * cc]) |
                         (static_cast<unsigned>(bf16_bits(yv[8 + 2 * cc + 1])) << 16);
            }
            *reinterpret_cast<u32x4_t*>(dw) = r0;
            *reinterpret_cast<u32x4_t*>(dw + 8) = r1;
            if (lg == w) {  // diagonal block of T
                uint16_t* tdst = Tm + (16 * w + l16) * G::PT + 16 * w;
                *reinterpret_cast<u32x4_t*>(tdst) = r0;
                *reinterpret_cast<u32x4_t*>(tdst + 8) = r1;
            }
            if ((w & 1) == 1 && lg == 0) {  // upper block (w-1, w) of T is read by U = T R
                const u32x4_t z = {0u, 0u, 0u, 0u};
                uint16_t* tdst = Tm + (16 * (w - 1) + l16) * G::PT + 16 * w;
                *reinterpret_cast<u32x4_t*>(tdst) = z;
                *reinterpret_cast<u32x4_t*>(tdst + 8) = z;
            }
            wave_lds_fence();

            // X_i = T[16i.., 16j..]: X_j = D_j, X_i = -D_i sum_{k=j}^{i-1} A_ik X_k.
            // xb[i] holds X_i as a 16x16x16 B operand (slot s <-> row 4g+s);
            // every slot starts as X_j and slots i > j are overwritten in order.
            const int j = w;
            u32x2_t xb[4];
            {
                const uint16_t* dj = Dw + ((w * 4 + j) * 16) * G::PD + l16;
                xb[0].x = dj[(4 * lg) * G::PD] | (static_cast<unsigned>(dj[(4 * lg + 1) * G::PD]) << 16);
                xb[0].y = dj[(4 * lg + 2) * G::PD] | (static_cast<unsigned>(dj[(4 * lg + 3) * G::PD]) << 16);
#pragma unroll
                for (int i = 1; i < 4; ++i) xb[i] = xb[0];
            }
#pragma unroll
            for (int i = 1; i < 4; ++i) {
                if (i <= j) continue;
                f32x4_t z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kk = 0; kk < 3; ++kk) {
                    if (kk < j || kk >= i) continue;
                    const f32x4_t af =
                        *reinterpret_cast<const f32x4_t*>(Af + (16 * i + l16) * G::PA + 16 * kk + 4 * lg);
                    z = mfma16(cvt4(af), xb[kk], z);
                }
                const uint16_t* di = Dw + ((w * 4 + i) * 16 + l16) * G::PD + 4 * lg;
                const u32x2_t dv = *reinterpret_cast<const u32x2_t*>(di);
                const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
                const f32x4_t x = -mfma16(dv, cvt4(z), zero);
                xb[i] = cvt4(x);
                uint16_t* tcol = Tm + (16 * i + 4 * lg) * G::PT + 16 * j + l16;
                tcol[0] = static_cast<uint16_t>(xb[i].x & 0xffffu);
                tcol[G::PT] = static_cast<uint16_t>(xb[i].x >> 16);
                tcol[2 * G::PT] = static_cast<uint16_t>(xb[i].y & 0xffffu);
                tcol[3 * G::PT] = static_cast<uint16_t>(xb[i].y >> 16);
            }
        }
        __syncthreads();

        // ---- phase U: chain waves finish the chunk for their 16 columns ----
        if (chain) {
            const int lc = 16 * w + l16;  // column inside the tile
            f32x4_t R[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const u32x2_t vv = *reinterpret_cast<const u32x2_t*>(Vt + lc * G::PT + 16 * m + 4 * lg);
                const f32x4_t bs = *reinterpret_cast<const f32x4_t*>(Bs + 16 * m + 4 * lg);
                const f32x4_t vf = {bf16_to_f32(vv.x & 0xffffu), bf16_to_f32(vv.x >> 16),
                                    bf16_to_f32(vv.y & 0xffffu), bf16_to_f32(vv.y >> 16)};
                R[m] = bs * (vf - X[m]);
            }
            const bf16x8_t Rb0 = acc_to_b(R[0], R[1]), Rb1 = acc_to_b(R[2], R[3]);
            f32x4_t U[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                f32x4_t u = {0.f, 0.f, 0.f, 0.f};
                u = mfma32(lds_a(Tm, G::PT, 16 * m + l16, 0, lg), Rb0, u);
                if (m >= 2) u = mfma32(lds_a(Tm, G::PT, 16 * m + l16, 32, lg), Rb1, u);
                U[m] = u;
            }
            const bf16x8_t Ub0 = acc_to_b(U[0], U[1]), Ub1 = acc_to_b(U[2], U[3]);
            // O = Y + P U
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                f32x4_t ov = Y[m];
                ov = mfma32(lds_a(Pm, G::PT, 16 * m + l16, 0, lg), Ub0, ov);
                if (m >= 2) ov = mfma32(lds_a(Pm, G::PT, 16 * m + l16, 32, lg), Ub1, ov);
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) {
                    const int t = 16 * m + 4 * lg + ii;
                    if (t < clen) {
                        const size_t a = (tok0 + base + t) * tstride + static_cast<size_t>(h) * D + ecol;
                        if constexpr (OUT_BF16)
                            static_cast<uint16_t*>(o_out)[a] = f32_to_bf16(ov[ii]);
                        else
                            static_cast<float*>(o_out)[a] = ov[ii];
                    }
                }
            }
            // S += K^T U
#pragma unroll
            for (int md = 0; md < D / 16; ++md) {
                S[md] = mfma32(lds_a(Kt, G::PT, 16 * md + l16, 0, lg), Ub0, S[md]);
                S[md] = mfma32(lds_a(Kt, G::PT, 16 * md + l16, 32, lg), Ub1, S[md]);
            }
#pragma unroll
            for (int kb = 0; kb < D / 32; ++kb) Sb[kb] = acc_to_b(S[2 * kb], S[2 * kb + 1]);
        }
    }

    if (chain) {
#pragma unroll
        for (int md = 0; md < D / 16; ++md) {
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
                const int d = 16 * md + 4 * lg + ii;
                s_out[sbase + static_cast<size_t>(d) * D + ecol] = S[md][ii];
            }
        }
    }
}

template <int D, int DV, bool OB>
hipError_t launch_t(const ChunkedArgs& a, hipStream_t st) {
    using G = Geo<D, DV>;
    auto kern = delta_chunked_kernel<D, DV, OB>;
    static bool attr_set = false;  // per instantiation
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, G::BYTES);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const int n_pairs = a.n_seq * a.H;
    const int n_tiles = D / DV;
    const int slots = (n_pairs + 7) / 8;
    const dim3 grid(static_cast<unsigned>(slots * 8 * n_tiles));
    hipLaunchKernelGGL(kern, grid, dim3(256), G::BYTES, st, a.q, a.k, a.v, a.beta, a.s0, a.o,
                       a.s_out, a.cu_seqlens, n_pairs, a.T, a.H, n_tiles);
    return hipGetLastError();
}

template <int D, int DV>
hipError_t launch_dv(const ChunkedArgs& a, hipStream_t st) {
    return a.out_bf16 ? launch_t<D, DV, true>(a, st) : launch_t<D, DV, false>(a, st);
}

// Tile width: enough workgroups to cover the 256 CUs, as few column tiles
// as that allows (every tile repeats the column-independent chunk work).
int pick_tile(int D, long n_pairs, int requested) {
    if (requested == 16 || requested == 32 || requested == 64) return requested > D ? D : requested;
    int dv = D < 64 ? D : 64;
    while (dv > 16 && n_pairs * (D / dv) < 256) dv /= 2;
    return dv;
}

}  // namespace

bool chunked_supported(int D) { return D == 64 || D == 128; }

hipError_t launch_chunked(const ChunkedArgs& a, hipStream_t st) {
    const long n_pairs = static_cast<long>(a.n_seq) * a.H;
    if (n_pairs == 0) return hipSuccess;
    const int dv = pick_tile(a.D, n_pairs, a.dv_tile);
    if (a.D == 128) {
        if (dv == 16) return launch_dv<128, 16>(a, st);
        if (dv == 32) return launch_dv<128, 32>(a, st);
        return launch_dv<128, 64>(a, st);
    }
    if (a.D == 64) {
        if (dv == 16) return launch_dv<64, 16>(a, st);
        if (dv == 32) return launch_dv<64, 32>(a, st);
        return launch_dv<64, 64>(a, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace pm
