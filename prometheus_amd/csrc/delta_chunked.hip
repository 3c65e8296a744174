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
// (DeltaNet chunk form, Yang et al. 2024.  W = T diag(beta) K is never
// formed: T is applied to diag(beta)(V - K S), so the per-chunk work that
// depends on K and Q alone does not depend on the d_v columns.)
//
// Work split.  The recurrence is separable along d_v.  A 256-thread
// workgroup owns (sequence, head, d_v tile of DV columns) and walks the
// sequence's chunks in order, as a three-stage software pipeline:
//   * DV/16 "chain" waves own 16 columns of S each (fp32 MFMA
//     accumulators) and run chunk c: K S, Q S, R, U = T R, O = Q S + P U,
//     S += K^T U;
//   * "producer" waves build chunk c+1's T (producer 0) and P (producer 1)
//     in registers and stage chunk c+2 from HBM into LDS.
// Two LDS-only barriers per chunk; only producers touch global loads, so
// no barrier waits on memory traffic.  The workgroups of one (sequence,
// head) share bid % 8, i.e. one XCD and its L2 (blocks go round-robin
// over the 8 XCDs), so their common Q/K reads are served by that L2.
//
// Register-resident algebra.  v_mfma_f32_16x16x32_bf16 contracts 32
// values per lane group; the contraction is invariant under any
// permutation of its index applied to both operands, so lane group g's 8
// slots are mapped to indices {4g..4g+3, 16+4g..16+4g+3} of each 32-block.
// With that mapping two stacked fp32 accumulator tiles, rounded to bf16,
// are the B operand of the next product (contraction over the tile rows),
// and one accumulator tile used as an A operand is its own transpose.
// T is built without LDS:
//   * diagonal 16x16 blocks (I + L)^-1 = (I+N)(I+N^2)(I+N^4)(I+N^8), N = -L,
//     on v_mfma_f32_16x16x16_bf16, each factor kept both as itself and as
//     its transpose (K K^T is symmetric, so one accumulator tile of K K^T
//     yields L and L^T);
//   * off-diagonal blocks T_ij = -D_i sum_{k=j}^{i-1} A_ik T_kj, with A_ik
//     taken from the upper tile (k, i) of K K^T (again by symmetry).
// T and P are stored in LDS in MFMA A-operand order (one 16-byte read per
// operand per lane, contiguous across the wave).
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
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
// Two floats -> packed bf16 pair (round to nearest even) in one v_cvt_pk_bf16_f32.
__device__ __forceinline__ unsigned pack2(float a, float b) {
    const f32x2_t v = {a, b};
    return __builtin_bit_cast(unsigned, __builtin_convertvector(v, bf16x2_t));
}
__device__ __forceinline__ unsigned pack_rne(float a, float b) {
    return static_cast<unsigned>(f32_to_bf16(a)) | (static_cast<unsigned>(f32_to_bf16(b)) << 16);
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

// LDS swizzles (bank-conflict-free 8-byte accesses).  Rows are stored in
// 8-byte blocks of 4 bf16; the physical block is the logical block XORed
// with a per-row value:
//   K/Q rows (token-major):      block ^ ((row >> 3) & 1)   -- rows r and r+8
//                                land on different banks; a 16-byte chunk keeps
//                                its place with its two halves swapped;
//   K^T / V^T rows (d/e-major):  block ^ ((row >> 3) & 15)  -- the staging
//                                writes of 16 lanes (16 different rows 8
//                                apart, one token block) hit 16 different banks.
__device__ __forceinline__ int swz_kq(int row) { return (row >> 3) & 1; }
__device__ __forceinline__ int swz_t(int row) { return (row >> 3) & 15; }

// A operand of a 16x16x32 product from a swizzled bf16 LDS matrix:
// row `row`, contraction block starting at k0 (multiple of 32), lane group g.
__device__ __forceinline__ bf16x8_t lds_a_sw(const uint16_t* m, int pitch, int row, int k0, int g,
                                             int sw) {
    const uint16_t* r = m + row * pitch;
    const int b = (k0 >> 2) + g;
    const u32x2_t lo = *reinterpret_cast<const u32x2_t*>(r + 4 * (b ^ sw));
    const u32x2_t hi = *reinterpret_cast<const u32x2_t*>(r + 4 * ((b + 4) ^ sw));
    const u32x4_t v = {lo.x, lo.y, hi.x, hi.y};
    return __builtin_bit_cast(bf16x8_t, v);
}
__device__ __forceinline__ bf16x8_t lds_a_kq(const uint16_t* m, int pitch, int row, int k0, int g) {
    return lds_a_sw(m, pitch, row, k0, g, swz_kq(row));
}
__device__ __forceinline__ bf16x8_t lds_a_t(const uint16_t* m, int pitch, int row, int k0, int g) {
    return lds_a_sw(m, pitch, row, k0, g, swz_t(row));
}

// Packed operand layout of the 64x64 lower-triangular T and P: operand
// block q holds rows 16m.. and contraction block kb (32 columns) for
// (m, kb) in (0,0) (1,0) (2,0) (2,1) (3,0) (3,1); lane L's 8 values are
// contiguous at q*512 + L*8 (bf16 elements).
__device__ __forceinline__ int qblk(int m, int kb) { return m < 2 ? m : 2 * m - 2 + kb; }

__device__ __forceinline__ bf16x8_t packed_a(const uint16_t* buf, int q, int lane) {
    return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(buf + q * 512 + lane * 8));
}

// Store block (i, j) of a 64x64 matrix M into the packed operand layout,
// given the accumulator tile of its transpose (lane (g, l16) holds
// M[16i+l16][16j+4g+r], r<4): those are exactly this lane's operand slots
// 4(j&1)..4(j&1)+3, so one 8-byte write per lane, contiguous across the wave.
__device__ __forceinline__ void store_packed_t(uint16_t* buf, int i, int j, f32x4_t acc_t, int lane) {
    *reinterpret_cast<u32x2_t*>(buf + qblk(i, j >> 1) * 512 + lane * 8 + 4 * (j & 1)) = cvt4(acc_t);
}
// Zero the upper 16-column half of operand block q (T/P blocks (0,1), (2,3)).
__device__ __forceinline__ void zero_upper_half(uint16_t* buf, int q, int lane) {
    const u32x2_t z = {0u, 0u};
    *reinterpret_cast<u32x2_t*>(buf + q * 512 + lane * 8 + 4) = z;
}

// Element j of four 8-element rows r[0..3], packed as 4 consecutive bf16
// (a column of a 4x8 block), with v_perm_b32 selecting 16-bit halves.
__device__ __forceinline__ u32x2_t column4(const u32x4_t* r, int j) {
    const unsigned sel = (j & 1) ? 0x07060302u : 0x05040100u;
    const u32x2_t out = {__builtin_amdgcn_perm(r[1][j >> 1], r[0][j >> 1], sel),
                         __builtin_amdgcn_perm(r[3][j >> 1], r[2][j >> 1], sel)};
    return out;
}

// LDS-only workgroup barrier: waits for this wave's LDS traffic, never for
// global loads or stores still in flight.
__device__ __forceinline__ void lds_barrier() {
    __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int D, int DV>
struct Geo {
    static constexpr int NCW = DV / 16;   // chain waves
    static constexpr int NPW = 4 - NCW;   // producer waves
    static constexpr int PK = D + 8;      // Ks/Qs pitch (bf16)
    static constexpr int PT = kC + 8;     // Kt/Vt pitch (bf16)
    static constexpr int DG = D / 8;      // 16-byte groups per token row
    static constexpr int VG = DV / 8;     // 16-byte groups per V tile row
    static constexpr int NU = 16 * DG;    // K/Q staging units (4 tokens x 8 d)
    static constexpr int NVU = 16 * VG;   // V staging units (4 tokens x 8 columns)
    static constexpr int UPL = (NU + NPW * 64 - 1) / (NPW * 64);   // units per producer lane
    static constexpr int VPL = (NVU + NPW * 64 - 1) / (NPW * 64);
    // one RAW buffer: Ks, Qs, Kt, Vt (bf16), Bs (fp32)
    static constexpr int R_KS = 0;
    static constexpr int R_QS = R_KS + kC * PK * 2;
    static constexpr int R_KT = R_QS + kC * PK * 2;
    static constexpr int R_VT = R_KT + D * PT * 2;
    static constexpr int R_BS = R_VT + DV * PT * 2;
    static constexpr int RAW = R_BS + kC * 4;
    // one TP buffer: T and P, 6 operand blocks of 1 KiB each
    static constexpr int TP = 2 * 6 * 1024;
    static constexpr int BYTES = 2 * RAW + 2 * TP;
    static_assert(D % 32 == 0 && D <= 128, "D");
    static_assert(DV == 16 || DV == 32, "DV");
    static_assert(RAW % 16 == 0, "RAW alignment");
    static_assert(BYTES <= 160 * 1024, "LDS budget");
};

template <int D, int DV, bool OUT_BF16>
__global__ __launch_bounds__(256) void delta_chunked_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const float* __restrict__ beta,
    const float* __restrict__ s0, void* __restrict__ o_out, float* __restrict__ s_out,
    const int32_t* __restrict__ cu_seqlens, int n_pairs, int T, int H, int n_tiles) {
    using G = Geo<D, DV>;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

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
    const int n_chunks = (len + kC - 1) / kC;

    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int l16 = lane & 15, lg = lane >> 4;
    const bool chain = w < G::NCW;
    const int pw = w - G::NCW;  // producer index (valid when !chain)
    const int plane = pw * 64 + lane;
    const size_t sbase = static_cast<size_t>(pair) * D * D;
    const size_t tstride = static_cast<size_t>(H) * D;  // elements between tokens

    auto raw = [&](int c) { return smem + (c & 1) * G::RAW; };
    auto tpb = [&](int c) { return reinterpret_cast<uint16_t*>(smem + 2 * G::RAW + (c & 1) * G::TP); };

    // ---------------- producer state: staged chunk in registers ----------------
    u32x4_t kr[G::UPL][4], qr[G::UPL][4], vr[G::VPL][4];
    float br = 0.f;
    auto stage_load = [&](int c) {
        const int base = c * kC;
        const int clen = min(kC, len - base);
        const u32x4_t z = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int u = 0; u < G::UPL; ++u) {
            const int unit = plane + u * G::NPW * 64;
            const int dg = unit % G::DG, tg = unit / G::DG;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = 4 * tg + i;
                kr[u][i] = z;
                qr[u][i] = z;
                if (unit < G::NU && t < clen) {
                    const size_t a = (tok0 + base + t) * tstride + static_cast<size_t>(h) * D + dg * 8;
                    kr[u][i] = *reinterpret_cast<const u32x4_t*>(k + a);
                    qr[u][i] = *reinterpret_cast<const u32x4_t*>(q + a);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < G::VPL; ++u) {
            const int unit = plane + u * G::NPW * 64;
            const int tg = unit % 16, cv = unit / 16;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = 4 * tg + i;
                vr[u][i] = z;
                if (unit < G::NVU && t < clen) {
                    const size_t a =
                        (tok0 + base + t) * tstride + static_cast<size_t>(h) * D + col0 + cv * 8;
                    vr[u][i] = *reinterpret_cast<const u32x4_t*>(v + a);
                }
            }
        }
        br = (plane < clen) ? beta[(tok0 + base + plane) * H + h] : 0.f;
    };
    auto stage_store = [&](int c) {
        unsigned char* rb = raw(c);
        uint16_t* Ks = reinterpret_cast<uint16_t*>(rb + G::R_KS);
        uint16_t* Qs = reinterpret_cast<uint16_t*>(rb + G::R_QS);
        uint16_t* Kt = reinterpret_cast<uint16_t*>(rb + G::R_KT);
        uint16_t* Vt = reinterpret_cast<uint16_t*>(rb + G::R_VT);
        float* Bs = reinterpret_cast<float*>(rb + G::R_BS);
#pragma unroll
        for (int u = 0; u < G::UPL; ++u) {
            const int unit = plane + u * G::NPW * 64;
            if (unit < G::NU) {
                const int dg = unit % G::DG, tg = unit / G::DG;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = 4 * tg + i;
                    const bool swap = swz_kq(r) != 0;  // 16-byte chunk with its halves swapped
                    const u32x4_t kv = swap ? u32x4_t{kr[u][i].z, kr[u][i].w, kr[u][i].x, kr[u][i].y} : kr[u][i];
                    const u32x4_t qv = swap ? u32x4_t{qr[u][i].z, qr[u][i].w, qr[u][i].x, qr[u][i].y} : qr[u][i];
                    *reinterpret_cast<u32x4_t*>(Ks + r * G::PK + dg * 8) = kv;
                    *reinterpret_cast<u32x4_t*>(Qs + r * G::PK + dg * 8) = qv;
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int d = dg * 8 + j;
                    *reinterpret_cast<u32x2_t*>(Kt + d * G::PT + 4 * (tg ^ swz_t(d))) = column4(kr[u], j);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < G::VPL; ++u) {
            const int unit = plane + u * G::NPW * 64;
            if (unit < G::NVU) {
                const int tg = unit % 16, cv = unit / 16;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int e = cv * 8 + j;
                    *reinterpret_cast<u32x2_t*>(Vt + e * G::PT + 4 * (tg ^ swz_t(e))) = column4(vr[u], j);
                }
            }
        }
        if (plane < kC) Bs[plane] = br;
    };

    // ---------------- producer 0: T = (I + A)^-1 in packed operand order ----------------
    auto build_t = [&](int c) {
        unsigned char* rb = raw(c);
        const uint16_t* Ks = reinterpret_cast<const uint16_t*>(rb + G::R_KS);
        const float* Bs = reinterpret_cast<const float*>(rb + G::R_BS);
        uint16_t* Tp = tpb(c);
        const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
        // G = K K^T: diagonal tiles gd[b] and upper tiles gu(k, i), k < i
        f32x4_t gd[4], gu[6];
#pragma unroll
        for (int b = 0; b < 4; ++b) gd[b] = zero;
#pragma unroll
        for (int x = 0; x < 6; ++x) gu[x] = zero;
#pragma unroll
        for (int kb = 0; kb < D / 32; ++kb) {
            bf16x8_t f[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) f[r] = lds_a_kq(Ks, G::PK, 16 * r + l16, 32 * kb, lg);
#pragma unroll
            for (int b = 0; b < 4; ++b) gd[b] = mfma32(f[b], f[b], gd[b]);
            gu[0] = mfma32(f[0], f[1], gu[0]);  // (0,1)
            gu[1] = mfma32(f[0], f[2], gu[1]);  // (0,2)
            gu[2] = mfma32(f[1], f[2], gu[2]);  // (1,2)
            gu[3] = mfma32(f[0], f[3], gu[3]);  // (0,3)
            gu[4] = mfma32(f[1], f[3], gu[4]);  // (1,3)
            gu[5] = mfma32(f[2], f[3], gu[5]);  // (2,3)
        }
        // beta of the rows this lane holds in accumulator form (br4) and in A-operand form (bc)
        f32x4_t br4[4];
        float bc[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            br4[b] = *reinterpret_cast<const f32x4_t*>(Bs + 16 * b + 4 * lg);
            bc[b] = Bs[16 * b + l16];
        }
        f32x4_t eye;
#pragma unroll
        for (int r = 0; r < 4; ++r) eye[r] = (4 * lg + r == l16) ? 1.f : 0.f;
        // diagonal inverses D_b = (I+N)(I+N^2)(I+N^4)(I+N^8), N = -L_b (dd = D_b, ddt = D_b^T),
        // one level at a time over the four independent blocks
        u32x2_t cn[4], cnt[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            f32x4_t n, nt;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = 4 * lg + r;
                n[r] = (row > l16) ? -br4[b][r] * gd[b][r] : 0.f;   // N[row][l16]
                nt[r] = (l16 > row) ? -bc[b] * gd[b][r] : 0.f;      // N[l16][row]
            }
            cn[b] = cvt4(n);
            cnt[b] = cvt4(nt);
        }
        f32x4_t n2[4], n2t[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            n2[b] = mfma16(cnt[b], cn[b], zero);
            n2t[b] = mfma16(cn[b], cnt[b], zero);
        }
        u32x2_t cn2[4], cn2t[4], ci2[4], cet[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            cn2[b] = cvt4(n2[b]);
            cn2t[b] = cvt4(n2t[b]);
            ci2[b] = cvt4(n2[b] + eye);
        }
        f32x4_t n4[4], n4t[4], ft[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            // cet = (I + N)^T as an accumulator, rebuilt from cnt's source values
            f32x4_t nt;
#pragma unroll
            for (int r = 0; r < 4; ++r) nt[r] = (l16 > 4 * lg + r) ? -bc[b] * gd[b][r] : 0.f;
            cet[b] = cvt4(nt + eye);
            n4[b] = mfma16(cn2t[b], cn2[b], zero);
            n4t[b] = mfma16(cn2[b], cn2t[b], zero);
            ft[b] = mfma16(ci2[b], cet[b], zero);       // ((I+N)(I+N^2))^T
        }
        u32x2_t cn4[4], cn4t[4], ci4[4], cft[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            cn4[b] = cvt4(n4[b]);
            cn4t[b] = cvt4(n4t[b]);
            ci4[b] = cvt4(n4[b] + eye);
            cft[b] = cvt4(ft[b]);
        }
        f32x4_t n8[4], f2t[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            n8[b] = mfma16(cn4t[b], cn4[b], zero);
            f2t[b] = mfma16(ci4[b], cft[b], zero);      // (...(I+N^4))^T
        }
        f32x4_t dd[4], ddt[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const u32x2_t ci8 = cvt4(n8[b] + eye), cf2t = cvt4(f2t[b]);
            dd[b] = mfma16(cf2t, ci8, zero);            // ...(I+N^8)
            ddt[b] = mfma16(ci8, cf2t, zero);
        }
        // A_ik as an A operand: upper tile (k, i) of K K^T, rows scaled by beta_{16i+l16}
        auto a_op = [&](int x, int i) { return cvt4(bc[i] * gu[x]); };
        const u32x2_t cd0 = cvt4(dd[0]), cd1 = cvt4(dd[1]), cd2 = cvt4(dd[2]);
        const u32x2_t cdt1 = cvt4(ddt[1]), cdt2 = cvt4(ddt[2]), cdt3 = cvt4(ddt[3]);
        const u32x2_t a10 = a_op(0, 1), a20 = a_op(1, 2), a21 = a_op(2, 2);
        const u32x2_t a30 = a_op(3, 3), a31 = a_op(4, 3), a32 = a_op(5, 3);
        // T_ij = -D_i Z_ij with Z_ij = sum_k A_ik T_kj; cdt_i is D_i as an A operand and
        // D_i^T as a B operand, so -mfma(Z, cdt_i) is T_ij^T (what the packed store takes)
        // level 1
        const u32x2_t z10 = cvt4(mfma16(a10, cd0, zero));
        const u32x2_t z21 = cvt4(mfma16(a21, cd1, zero));
        const u32x2_t z32 = cvt4(mfma16(a32, cd2, zero));
        const u32x2_t cx10 = cvt4(-mfma16(cdt1, z10, zero));
        const u32x2_t cx21 = cvt4(-mfma16(cdt2, z21, zero));
        const f32x4_t x10t = -mfma16(z10, cdt1, zero);
        const f32x4_t x21t = -mfma16(z21, cdt2, zero);
        const f32x4_t x32t = -mfma16(z32, cdt3, zero);
        // level 2
        const u32x2_t z20 = cvt4(mfma16(a21, cx10, mfma16(a20, cd0, zero)));
        const u32x2_t z31 = cvt4(mfma16(a32, cx21, mfma16(a31, cd1, zero)));
        const u32x2_t cx20 = cvt4(-mfma16(cdt2, z20, zero));
        const f32x4_t x20t = -mfma16(z20, cdt2, zero);
        const f32x4_t x31t = -mfma16(z31, cdt3, zero);
        // level 3
        const u32x2_t z30 = cvt4(mfma16(a32, cx20, mfma16(a31, cx10, mfma16(a30, cd0, zero))));
        const f32x4_t x30t = -mfma16(z30, cdt3, zero);
        store_packed_t(Tp, 0, 0, ddt[0], lane);
        store_packed_t(Tp, 1, 0, x10t, lane);
        store_packed_t(Tp, 1, 1, ddt[1], lane);
        store_packed_t(Tp, 2, 0, x20t, lane);
        store_packed_t(Tp, 2, 1, x21t, lane);
        store_packed_t(Tp, 2, 2, ddt[2], lane);
        store_packed_t(Tp, 3, 0, x30t, lane);
        store_packed_t(Tp, 3, 1, x31t, lane);
        store_packed_t(Tp, 3, 2, x32t, lane);
        store_packed_t(Tp, 3, 3, ddt[3], lane);
        zero_upper_half(Tp, qblk(0, 0), lane);
        zero_upper_half(Tp, qblk(2, 1), lane);
    };

    // ---------------- producer 1: P = lower_incl_diag(Q K^T) in packed operand order ----------------
    auto build_p = [&](int c) {
        unsigned char* rb = raw(c);
        const uint16_t* Ks = reinterpret_cast<const uint16_t*>(rb + G::R_KS);
        const uint16_t* Qs = reinterpret_cast<const uint16_t*>(rb + G::R_QS);
        uint16_t* Pp = tpb(c) + 6 * 512;
        const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
        f32x4_t p[10];
#pragma unroll
        for (int x = 0; x < 10; ++x) p[x] = zero;
#pragma unroll
        for (int kb = 0; kb < D / 32; ++kb) {
            bf16x8_t fk[4], fq[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                fk[r] = lds_a_kq(Ks, G::PK, 16 * r + l16, 32 * kb, lg);
                fq[r] = lds_a_kq(Qs, G::PK, 16 * r + l16, 32 * kb, lg);
            }
            // accumulator of (P_ij)^T = K_j Q_i^T: lane holds P[16i+l16][16j+4g+r]
            int x = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j <= i; ++j, ++x) p[x] = mfma32(fk[j], fq[i], p[x]);
        }
        int x = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j <= i; ++j, ++x) {
                f32x4_t t = p[x];
                if (i == j) {  // keep t >= s: row l16, column 4g+r
#pragma unroll
                    for (int r = 0; r < 4; ++r) t[r] = (l16 >= 4 * lg + r) ? t[r] : 0.f;
                }
                store_packed_t(Pp, i, j, t, lane);
            }
        zero_upper_half(Pp, qblk(0, 0), lane);
        zero_upper_half(Pp, qblk(2, 1), lane);
    };

    // ---------------- chain state: wave w owns columns col0 + 16w + [0, 16) ----------------
    f32x4_t S[D / 16];
    const int ecol = col0 + 16 * w + l16;
#pragma unroll
    for (int md = 0; md < D / 16; ++md) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int d = 16 * md + 4 * lg + r;
            S[md][r] = (chain && s0) ? s0[sbase + static_cast<size_t>(d) * D + ecol] : 0.f;
        }
    }
    bf16x8_t Sb[D / 32];
#pragma unroll
    for (int kb = 0; kb < D / 32; ++kb) Sb[kb] = acc_to_b(S[2 * kb], S[2 * kb + 1]);

    auto run_chunk = [&](int c) {
        unsigned char* rb = raw(c);
        const uint16_t* Ks = reinterpret_cast<const uint16_t*>(rb + G::R_KS);
        const uint16_t* Qs = reinterpret_cast<const uint16_t*>(rb + G::R_QS);
        const uint16_t* Kt = reinterpret_cast<const uint16_t*>(rb + G::R_KT);
        const uint16_t* Vt = reinterpret_cast<const uint16_t*>(rb + G::R_VT);
        const float* Bs = reinterpret_cast<const float*>(rb + G::R_BS);
        const uint16_t* Tp = tpb(c);
        const uint16_t* Pp = Tp + 6 * 512;
        const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
        const int base = c * kC;
        const int clen = min(kC, len - base);
        // X = K S (token rows) and Y^T = S^T Q^T (column rows: lane holds 4 columns of a token)
        f32x4_t X[4], Y[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            X[m] = zero;
            Y[m] = zero;
        }
#pragma unroll
        for (int kb = 0; kb < D / 32; ++kb) {
            bf16x8_t fk[4], fq[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                fk[m] = lds_a_kq(Ks, G::PK, 16 * m + l16, 32 * kb, lg);
                fq[m] = lds_a_kq(Qs, G::PK, 16 * m + l16, 32 * kb, lg);
            }
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                X[m] = mfma32(fk[m], Sb[kb], X[m]);
                Y[m] = mfma32(Sb[kb], fq[m], Y[m]);
            }
        }
        // R = beta (V - X)
        const int lc = 16 * w + l16;
        f32x4_t R[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const u32x2_t vv =
                *reinterpret_cast<const u32x2_t*>(Vt + lc * G::PT + 4 * ((4 * m + lg) ^ swz_t(lc)));
            const f32x4_t bs = *reinterpret_cast<const f32x4_t*>(Bs + 16 * m + 4 * lg);
            const f32x4_t vf = {bf16_to_f32(vv.x & 0xffffu), bf16_to_f32(vv.x >> 16),
                                bf16_to_f32(vv.y & 0xffffu), bf16_to_f32(vv.y >> 16)};
            R[m] = bs * (vf - X[m]);
        }
        const bf16x8_t Rb0 = acc_to_b(R[0], R[1]), Rb1 = acc_to_b(R[2], R[3]);
        // U = T R
        f32x4_t U[4];
        U[0] = mfma32(packed_a(Tp, 0, lane), Rb0, zero);
        U[1] = mfma32(packed_a(Tp, 1, lane), Rb0, zero);
        U[2] = mfma32(packed_a(Tp, 3, lane), Rb1, mfma32(packed_a(Tp, 2, lane), Rb0, zero));
        U[3] = mfma32(packed_a(Tp, 5, lane), Rb1, mfma32(packed_a(Tp, 4, lane), Rb0, zero));
        const bf16x8_t Ub0 = acc_to_b(U[0], U[1]), Ub1 = acc_to_b(U[2], U[3]);
        // S += K^T U
#pragma unroll
        for (int h4 = 0; h4 < D / 64; ++h4) {
            bf16x8_t f0[4], f1[4];
#pragma unroll
            for (int x = 0; x < 4; ++x) {
                f0[x] = lds_a_t(Kt, G::PT, 16 * (4 * h4 + x) + l16, 0, lg);
                f1[x] = lds_a_t(Kt, G::PT, 16 * (4 * h4 + x) + l16, 32, lg);
            }
#pragma unroll
            for (int x = 0; x < 4; ++x) {
                S[4 * h4 + x] = mfma32(f0[x], Ub0, S[4 * h4 + x]);
                S[4 * h4 + x] = mfma32(f1[x], Ub1, S[4 * h4 + x]);
            }
        }
        // O^T = Y^T + U^T P^T (U tiles as the A operand give U^T; the packed P rows are the
        // B operand P^T); lane (g, l16) holds O[16m+l16][4g..4g+3] of its 16 columns
        f32x4_t O[4];
        O[0] = mfma32(Ub0, packed_a(Pp, 0, lane), Y[0]);
        O[1] = mfma32(Ub0, packed_a(Pp, 1, lane), Y[1]);
        O[2] = mfma32(Ub1, packed_a(Pp, 3, lane), mfma32(Ub0, packed_a(Pp, 2, lane), Y[2]));
        O[3] = mfma32(Ub1, packed_a(Pp, 5, lane), mfma32(Ub0, packed_a(Pp, 4, lane), Y[3]));
#pragma unroll
        for (int kb = 0; kb < D / 32; ++kb) Sb[kb] = acc_to_b(S[2 * kb], S[2 * kb + 1]);
        const int ocol = col0 + 16 * w + 4 * lg;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int t = 16 * m + l16;
            if (t < clen) {
                const size_t a = (tok0 + base + t) * tstride + static_cast<size_t>(h) * D + ocol;
                if constexpr (OUT_BF16) {
                    const u32x2_t ob = {pack_rne(O[m].x, O[m].y), pack_rne(O[m].z, O[m].w)};
                    *reinterpret_cast<u32x2_t*>(static_cast<uint16_t*>(o_out) + a) = ob;
                } else {
                    *reinterpret_cast<f32x4_t*>(static_cast<float*>(o_out) + a) = O[m];
                }
            }
        }
    };

    // ---------------- pipeline: chain(c) || prep(c+1), staging c+2 ----------------
    // Each role runs its own loop (so registers are allocated per role) with
    // the same sequence of barriers: one after the prologue, two per chunk.
    if (n_chunks > 0) {
        if (chain) {
            lds_barrier();
            for (int c = 0; c < n_chunks; ++c) {
                lds_barrier();  // T/P of chunk c ready; chunk c-1 no longer read
                lds_barrier();  // chunk c+1 staged
                run_chunk(c);
            }
        } else {
            stage_load(0);
            stage_store(0);
            if (n_chunks > 1) stage_load(1);
            lds_barrier();
            if (pw == 0) {
                build_t(0);
            } else if (pw == 1) {
                build_p(0);
            }
            for (int c = 0; c < n_chunks; ++c) {
                lds_barrier();
                if (c + 1 < n_chunks) {
                    stage_store(c + 1);
                    if (c + 2 < n_chunks) stage_load(c + 2);
                }
                lds_barrier();
                if (c + 1 < n_chunks) {
                    if (pw == 0) {
                        build_t(c + 1);
                    } else if (pw == 1) {
                        build_p(c + 1);
                    }
                }
            }
        }
    }

    if (chain) {
#pragma unroll
        for (int md = 0; md < D / 16; ++md) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int d = 16 * md + 4 * lg + r;
                s_out[sbase + static_cast<size_t>(d) * D + ecol] = S[md][r];
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

// Tile width: 32 columns (two chain waves) unless that leaves CUs idle.
int pick_tile(int D, long n_pairs, int requested) {
    if (requested == 16 || requested == 32) return requested;
    if (requested == 64) return 32;
    return n_pairs * (D / 32) >= 256 ? 32 : 16;
}

}  // namespace

bool chunked_supported(int D) { return D == 64 || D == 128; }

hipError_t launch_chunked(const ChunkedArgs& a, hipStream_t st) {
    const long n_pairs = static_cast<long>(a.n_seq) * a.H;
    if (n_pairs == 0) return hipSuccess;
    const int dv = pick_tile(a.D, n_pairs, a.dv_tile);
    if (a.D == 128) return dv == 16 ? launch_dv<128, 16>(a, st) : launch_dv<128, 32>(a, st);
    if (a.D == 64) return dv == 16 ? launch_dv<64, 16>(a, st) : launch_dv<64, 32>(a, st);
    return hipErrorInvalidValue;
}

}  // namespace pm
