// pm_cdna4.h — gfx950 building blocks of the chunked delta-rule kernels:
// MFMA wrappers, bf16 packing, the swizzled LDS token tiles and their
// operand reads (plain and transposed), the packed operand layout of 64x64
// triangular blocks, buffer -> LDS copies, and the T = (I + A)^-1 builder.
// Everything is internal to the translation unit that includes it.
#pragma once

#include "pm_common.h"

namespace pm {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));

constexpr int kC = 64;  // chunk length (tokens)
// Buffer descriptor word 3 for raw (untyped, unswizzled) gfx9 buffer access.
constexpr int kRsrcWord3 = 0x00020000;

__device__ __forceinline__ f32x4_t mfma32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4_t mfma16(u32x2_t a, u32x2_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(bf16x4_t, a),
                                                     __builtin_bit_cast(bf16x4_t, b), c, 0, 0, 0);
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
__device__ __forceinline__ f32x4_t widen4(u32x2_t v) {
    const f32x4_t r = {__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u),
                       __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xffff0000u)};
    return r;
}

// LDS layout of a token-major tile (K or Q: D bf16 per row, V: DV per row).
// Rows have no padding; the 16-byte chunk c of row r is stored at chunk
// c ^ f(r), with f depending on r mod 16 only.  The copies (1 KiB contiguous
// per instruction) are conflict-free for any f.  f was chosen by measuring
// SQ_LDS_BANK_CONFLICT on gfx950 for the two patterns that read these tiles:
//   * 16-byte MFMA operand reads (lane (g, l16): row l16, chunk (4kb+g) ^ f);
//   * 8-byte transpose reads of K^T (lanes 4j+cc of group g: row 4g+j,
//     chunk (4kb+cc) ^ f).
// D = 128 (16 chunks per row): the table below makes the operand reads
// conflict-free (3.9 LDS cycles per instruction instead of 7.7) and costs the
// transpose reads 5.8 cycles instead of 3.9; no f of the 4096 tried makes
// both conflict-free, and the operand reads are twice as frequent.
// D = 64 (8 chunks per row): f(r) = r mod 8 makes both conflict-free.
template <int D>
__device__ __forceinline__ int kq_f(int r) {
    if constexpr (D == 128) return static_cast<int>((0x45AD27F936E8CB01ull >> (4 * (r & 15))) & 15);
    else return r & 7;
}
template <int DV>
__device__ __forceinline__ int v_f(int r) {
    if constexpr (DV == 32) return 2 * ((r >> 2) & 1);  // rows r and r+4 share banks
    else return 0;                                       // 8 rows of 32 bytes cover all banks
}

// Contraction over d.  In every product that contracts over d (X = K S,
// Y^T = S^T Q^T, K K^T, Q K^T) lane group g's 8 slots of 32-block kb are
// d = 32 kb + 8 g + [0, 8): one 16-byte chunk of a K/Q row.  To match,
// accumulator tile md = 2 kb + h of S holds the rows
//     d = 32 kb + 8 (r / 4) + 4 h + r % 4,   r = 0..15,
// so that acc_to_b(S[2 kb], S[2 kb + 1]) puts exactly those d in the slots.
__device__ __forceinline__ int s_row_d(int md, int r) {
    return 32 * (md >> 1) + 8 * (r >> 2) + 4 * (md & 1) + (r & 3);
}
// Operand (A or B) over d from a swizzled K/Q tile: row `row`, 32-block kb, lane group g.
template <int D>
__device__ __forceinline__ bf16x8_t lds_op_kq(const uint16_t* m, int row, int kb, int g) {
    return __builtin_bit_cast(bf16x8_t,
                              *reinterpret_cast<const u32x4_t*>(m + row * D + 8 * ((4 * kb + g) ^ kq_f<D>(row))));
}

// ds_read_b64_tr_b16: within each 16-lane group, the four 4-element rows
// addressed by lanes 4j..4j+3 (16 consecutive elements of row j) are
// transposed: lane i receives element i of rows 0..3.
//
// Issued as inline asm: the compiler's intrinsic for it carries no LDS
// memory operand, so hipcc (ROCm 7.2) puts a vmcnt(0) wait -- for every
// pending global store -- in front of it.  The asm form is asynchronous:
// results are valid only after lds_wait() takes them as operands.
__device__ __forceinline__ unsigned lds_addr(const void* p) {
    typedef __attribute__((address_space(3))) const void lds_cvoid_t;
    return static_cast<unsigned>(reinterpret_cast<uintptr_t>((lds_cvoid_t*)(p)));
}
template <int OFFSET>
__device__ __forceinline__ u32x2_t lds_tr16_issue(unsigned addr) {
    u32x2_t r;
    __asm__ volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFFSET) : "memory");
    return r;
}
// Wait for all of this wave's LDS reads; x's registers are tied to the wait
// so that no use of them is scheduled before it.
__device__ __forceinline__ void lds_wait(u32x2_t& a, u32x2_t& b, u32x2_t& c, u32x2_t& d) {
    __asm__ volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : : "memory");
}
__device__ __forceinline__ void lds_wait(u32x4_t& a, u32x4_t& b, u32x4_t& c, u32x4_t& d, u32x4_t& e,
                                         u32x4_t& f, u32x4_t& g, u32x4_t& h) {
    __asm__ volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(a), "+v"(b), "+v"(c), "+v"(d), "+v"(e), "+v"(f), "+v"(g), "+v"(h)
                     :
                     : "memory");
}
// A operand of K^T for S tile md (rows d = s_row_d(md, l16), contraction
// over tokens K0 + {4g..4g+3, 16+4g..16+4g+3}) from the token-major K
// tile: two transpose reads, 16 rows apart (kq_f(t + 16) == kq_f(t)); the
// four lanes 4j + cc of a group address d = 32 kb + 8 cc + 4 h + [0, 4).
template <int D, int K0>
__device__ __forceinline__ u32x4_t lds_kt_issue(const uint16_t* Ks, int md, int lane) {
    const int g = lane >> 4, j = (lane >> 2) & 3, cc = lane & 3;
    const int t = K0 + 4 * g + j;
    const unsigned a = lds_addr(Ks + t * D + 8 * ((4 * (md >> 1) + cc) ^ kq_f<D>(t)) + 4 * (md & 1));
    const u32x2_t lo = lds_tr16_issue<0>(a), hi = lds_tr16_issue<16 * D * 2>(a);
    const u32x4_t v = {lo.x, lo.y, hi.x, hi.y};
    return v;
}
// V in accumulator layout: lane (g, l16) gets V[16m + 4g + i][16w + l16], i < 4
// (bf16 pairs; widen4 after lds_wait).
template <int DV>
__device__ __forceinline__ u32x2_t lds_v_issue(const uint16_t* Vs, int m, int w, int lane) {
    const int g = lane >> 4, j = (lane >> 2) & 3, cc = lane & 3;
    const int t = 16 * m + 4 * g + j;
    return lds_tr16_issue<0>(lds_addr(Vs + t * DV + 8 * ((2 * w + (cc >> 1)) ^ v_f<DV>(t)) + 4 * (cc & 1)));
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

// I + X in bf16 operand form for a strictly lower X (or its transpose) held as a 16x16
// accumulator tile converted with cvt4 (lane (g, l16) holds rows 4g + [0, 4) of column
// l16; halves (r0, r1) and (r2, r3)).  X's diagonal entries are exact zeros (+0 or -0),
// so cvt4(X + I) equals cvt4(X) with the diagonal halves replaced by bf16 1.0 (0x3F80):
// two bit operations per word instead of four adds and two conversions.
struct EyeBits {
    u32x2_t one;   // 0x3F80 in the halves on the diagonal
    u32x2_t keep;  // 0xFFFF in the halves off the diagonal
};
__device__ __forceinline__ EyeBits eye_bits(int lane) {
    const int r = (lane & 15) - 4 * (lane >> 4);  // the component on the diagonal, if in [0, 4)
    EyeBits e = {{0u, 0u}, {~0u, ~0u}};
    if (r >= 0 && r < 4) {
        const int sh = 16 * (r & 1);
        if (r < 2) {
            e.one.x = 0x3F80u << sh;
            e.keep.x = ~(0xFFFFu << sh);
        } else {
            e.one.y = 0x3F80u << sh;
            e.keep.y = ~(0xFFFFu << sh);
        }
    }
    return e;
}
// (Plain C on purpose: these words feed MFMA operands, and hipcc inserts the wait states
// between a VALU write and an MFMA read only for instructions it generated itself.)
__device__ __forceinline__ u32x2_t with_eye(u32x2_t x, const EyeBits& e) { return (x & e.keep) | e.one; }

// Wave-uniform values made visibly uniform (SGPRs), so that buffer
// descriptors and role branches are scalar rather than per-lane.
__device__ __forceinline__ unsigned uniform(unsigned x) { return __builtin_amdgcn_readfirstlane(x); }
template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
    const unsigned long long u = reinterpret_cast<unsigned long long>(p);
    const unsigned long long lo = uniform(static_cast<unsigned>(u));
    const unsigned long long hi = uniform(static_cast<unsigned>(u >> 32));
    return reinterpret_cast<T*>((hi << 32) | lo);
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(const_cast<void*>(base)), 0, uniform(bytes),
                                             kRsrcWord3);
}

// Asynchronous copy of 16 (or 4) bytes per lane from a buffer to LDS:
// lane L's bytes land at dst + L * size (dst wave-uniform).
__device__ __forceinline__ void copy_to_lds(__amdgpu_buffer_rsrc_t rsrc, void* dst, int size,
                                            unsigned voffset) {
    typedef __attribute__((address_space(3))) void lds_void_t;
    if (size == 16)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t*)(dst), 16, voffset, 0, 0, 0);
    else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t*)(dst), 4, voffset, 0, 0, 0);
}

// LDS-only workgroup barrier: waits for this wave's LDS traffic, never for
// global loads or stores still in flight.
__device__ __forceinline__ void lds_barrier() {
    __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
// Wait for this wave's outstanding buffer loads (and so its LDS copies).
__device__ __forceinline__ void wait_copies() { __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// Wait until at most N vector-memory operations of this wave are outstanding
// (they complete in issue order).
template <int N>
__device__ __forceinline__ void wait_vm_n() {
    __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// A 16-byte-per-lane buffer -> LDS copy that the compiler does not see (lane L's
// bytes land at lds_dst + 16 L): no compiler-inserted waits before later LDS reads;
// the caller waits with wait_vm_n and a barrier.
__device__ __forceinline__ void dma16_asm(__amdgpu_buffer_rsrc_t rs, const void* lds_dst, unsigned voffset) {
    const unsigned m0 = uniform(lds_addr(lds_dst));
    __asm__ volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voffset), "s"(rs), "{m0}"(m0) : "memory");
}

// 2^x in one v_exp_f32 (about 1 ulp; 0 for x below the fp32 range).
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// The ten lower 16x16 blocks of T = (I + A)^-1, A = strict_lower(diag(beta) K K^T),
// for one 64-token chunk, each as the accumulator tile of its transpose (lane (g, l16)
// holds T[16i + l16][16j + 4g + r], r < 4), in the order (0,0) (1,0) (1,1) (2,0) (2,1)
// (2,2) (3,0) (3,1) (3,2) (3,3): the form store_packed_t takes.  One wave, from
//   f[r][kb]: K token row 16 r + l16, d = 32 kb + 8 g + [0, 8) (the operand order of
//             lds_op_kq), rows past the chunk's end zero;
//   bc[b] = beta of token 16 b + l16;  br4[b][r] = beta of token 16 b + 4 g + r.
// The forward kernel keeps the same algebra inline in its T producer, with its NORM and
// GATED scalings (called through a function instead, it compiled to 5 more VGPRs and
// about 190 more instructions, in its most time-critical role); for plain inputs the two
// give equal bits.
//
// t_from_gram is the part after the Gram matrix, for a Gram that need not be symmetric
// (the per-channel decayed one): with A'[t][s] the matrix whose strict lower part times
// diag(beta) is A, gd[b] holds diagonal block b as accumulator tile (lane (g, l16):
// A'[16b + 4g + r][16b + l16]), gdt[b] the same block transposed (A'[16b + l16][16b + 4g
// + r]), and gu[x] the off-diagonal block (k, i), k < i, in the order (0,1) (0,2) (1,2)
// (0,3) (1,3) (2,3), as the tile of A'[16i + l16][16k + 4g + r] at (g, l16).  t_blocks
// passes K K^T (gdt = gd).  tn gets the same blocks untransposed (lane (g, l16) holds
// T[16i + 4g + r][16j + l16], the diagonal blocks with exact zeros above the diagonal):
// two of those stacked, T_{2kb, m} over T_{2kb+1, m}, are block (m, kb) of T^T in packed
// operand order (acc_to_b).  Callers that do not read tn leave its products to dead-code
// elimination.
__device__ __forceinline__ void t_from_gram(const f32x4_t (&gd)[4], const f32x4_t (&gdt)[4],
                                            const f32x4_t (&gu)[6], const float (&bc)[4],
                                            const f32x4_t (&br4)[4], int lane, f32x4_t (&tb)[10],
                                            f32x4_t (&tn)[10]) {
    const int l16 = lane & 15, lg = lane >> 4;
    const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
    const EyeBits eyeb = eye_bits(lane);
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
            nt[r] = (l16 > row) ? -bc[b] * gdt[b][r] : 0.f;     // N[l16][row]
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
        ci2[b] = with_eye(cn2[b], eyeb);
    }
    f32x4_t n4[4], n4t[4], ft[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        cet[b] = with_eye(cnt[b], eyeb);  // (I + N)^T
        n4[b] = mfma16(cn2t[b], cn2[b], zero);
        n4t[b] = mfma16(cn2[b], cn2t[b], zero);
        ft[b] = mfma16(ci2[b], cet[b], zero);       // ((I+N)(I+N^2))^T
    }
    u32x2_t cn4[4], cn4t[4], ci4[4], cft[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        cn4[b] = cvt4(n4[b]);
        cn4t[b] = cvt4(n4t[b]);
        ci4[b] = with_eye(cn4[b], eyeb);
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
        const u32x2_t ci8 = with_eye(cvt4(n8[b]), eyeb), cf2t = cvt4(f2t[b]);
        dd[b] = mfma16(cf2t, ci8, zero);            // ...(I+N^8)
        ddt[b] = mfma16(ci8, cf2t, zero);
    }
    // -A_ik as an A operand: upper tile (k, i) of K K^T, rows scaled by -beta_{16i+l16} (the
    // minus folded in here, so that every product below comes out with T's sign; rounding
    // to nearest is symmetric, so negating an operand negates the rounded result exactly)
    auto a_op = [&](int x, int i) { return cvt4(-bc[i] * gu[x]); };
    const u32x2_t cd0 = cvt4(dd[0]), cd1 = cvt4(dd[1]), cd2 = cvt4(dd[2]);
    const u32x2_t cdt1 = cvt4(ddt[1]), cdt2 = cvt4(ddt[2]), cdt3 = cvt4(ddt[3]);
    const u32x2_t a10 = a_op(0, 1), a20 = a_op(1, 2), a21 = a_op(2, 2);
    const u32x2_t a30 = a_op(3, 3), a31 = a_op(4, 3), a32 = a_op(5, 3);
    // T_ij = D_i Z_ij with Z_ij = -sum_k A_ik T_kj (the a_op operands carry the minus);
    // cdt_i is D_i as an A operand and D_i^T as a B operand, so mfma(Z, cdt_i) is T_ij^T
    // (what the packed store takes)
    // level 1
    const u32x2_t z10 = cvt4(mfma16(a10, cd0, zero));
    const u32x2_t z21 = cvt4(mfma16(a21, cd1, zero));
    const u32x2_t z32 = cvt4(mfma16(a32, cd2, zero));
    const u32x2_t cx10 = cvt4(mfma16(cdt1, z10, zero));
    const u32x2_t cx21 = cvt4(mfma16(cdt2, z21, zero));
    tb[1] = mfma16(z10, cdt1, zero);  // (1,0)
    tb[4] = mfma16(z21, cdt2, zero);  // (2,1)
    tb[8] = mfma16(z32, cdt3, zero);  // (3,2)
    // level 2
    const u32x2_t z20 = cvt4(mfma16(a21, cx10, mfma16(a20, cd0, zero)));
    const u32x2_t z31 = cvt4(mfma16(a32, cx21, mfma16(a31, cd1, zero)));
    const u32x2_t cx20 = cvt4(mfma16(cdt2, z20, zero));
    tb[3] = mfma16(z20, cdt2, zero);  // (2,0)
    tb[7] = mfma16(z31, cdt3, zero);  // (3,1)
    // level 3
    const u32x2_t z30 = cvt4(mfma16(a32, cx20, mfma16(a31, cx10, mfma16(a30, cd0, zero))));
    tb[6] = mfma16(z30, cdt3, zero);  // (3,0)
    tb[0] = ddt[0];
    tb[2] = ddt[1];
    tb[5] = ddt[2];
    tb[9] = ddt[3];
    // mfma(cdt_i, Z_ij) = T_ij: the products above with the operands swapped (the same
    // products summed in the same order, so each element has the bits of tb's)
    tn[1] = mfma16(cdt1, z10, zero);
    tn[4] = mfma16(cdt2, z21, zero);
    tn[8] = mfma16(cdt3, z32, zero);
    tn[3] = mfma16(cdt2, z20, zero);
    tn[7] = mfma16(cdt3, z31, zero);
    tn[6] = mfma16(cdt3, z30, zero);
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) tn[b * (b + 3) / 2][r] = (4 * lg + r >= l16) ? dd[b][r] : 0.f;
}

template <int D>
__device__ __forceinline__ void t_blocks(const bf16x8_t (&f)[4][D / 32], const float (&bc)[4],
                                         const f32x4_t (&br4)[4], int lane, f32x4_t (&tb)[10],
                                         f32x4_t (&tn)[10]) {
    const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
    // G = K K^T: diagonal tiles gd[b] and upper tiles gu(k, i), k < i
    f32x4_t gd[4], gu[6];
#pragma unroll
    for (int b = 0; b < 4; ++b) gd[b] = zero;
#pragma unroll
    for (int x = 0; x < 6; ++x) gu[x] = zero;
#pragma unroll
    for (int kb = 0; kb < D / 32; ++kb) {
#pragma unroll
        for (int b = 0; b < 4; ++b) gd[b] = mfma32(f[b][kb], f[b][kb], gd[b]);
        gu[0] = mfma32(f[0][kb], f[1][kb], gu[0]);  // (0,1)
        gu[1] = mfma32(f[0][kb], f[2][kb], gu[1]);  // (0,2)
        gu[2] = mfma32(f[1][kb], f[2][kb], gu[2]);  // (1,2)
        gu[3] = mfma32(f[0][kb], f[3][kb], gu[3]);  // (0,3)
        gu[4] = mfma32(f[1][kb], f[3][kb], gu[4]);  // (1,3)
        gu[5] = mfma32(f[2][kb], f[3][kb], gu[5]);  // (2,3)
    }
    t_from_gram(gd, gd, gu, bc, br4, lane, tb, tn);
}

}  // namespace
}  // namespace pm
