// delta_chunked_bwd.hip — K6: reverse mode of the chunked forward on bf16
// MFMA (bf16 q/k/v, D in {64, 128}).
//
// Gradients of the reference's backward (kernels/__init__.py:692-719 ->
// _delta_vjp_np :460-527) restated per chunk of C = 64 tokens.  With the
// chunk's start state S, T = (I + A)^-1, A = strict_lower(diag(beta) K K^T),
// X = diag(beta)(V - K S), U = T X, P = lower_incl(Q K^T), the forward is
//     O = Q S + P U,      S_next = S + K^T U.
// Given G = dL/dS_next and dO, the reverse of one chunk is
//     W   = T^T (K G + P^T dO)                  (= dL/dX)
//     dS  = G + Q^T dO - K^T diag(beta) W       (G of the previous chunk)
//     dV  = diag(beta) W
//     dP  = lower_incl(dO U^T),   dA = -strict_lower(W U^T)
//     dQ  = dO S^T + dP K
//     dK  = U G^T + dP^T Q - diag(beta) W S^T + diag(beta) dA K + dA^T diag(beta) K
//     dbeta_t = W_t . (v_t - S^T k_t) + sum_{s<t} dA_ts (k_t . k_s)
// (dT = dU X^T and dA = -T^T dT T^T = -W U^T.)  Only the state gradient G
// is carried from chunk to chunk; everything else is local to a chunk once
// its start state S and end gradient G are known.  Three launches:
//   1. the forward kernel in its state-history mode writes every chunk's S
//      (bf16, as rows of S^T);
//   2. bwd_rev_kernel walks the chunks backwards per (b, h, 32 columns of
//      d_v) carrying G in fp32 MFMA accumulators (the columns of G are
//      independent) in two waves, while a third copies K, Q and beta of the
//      chunks ahead and builds their T^T and P^T (T by the forward's
//      builder) in packed MFMA operand order and a fourth copies dO and
//      stores dV; it writes G_c and W (bf16, in the packed order below),
//      the packed T, dV and finally dS_0;
//   3. bwd_grad_kernel, all chunks in parallel (one persistent workgroup
//      per CU, the next chunk's inputs fetched during the last two phases):
//      dQ, dK and dbeta from S_c, G_c, W and the chunk's q/k/v/beta.
// Numerics as in the forward: bf16 operands, fp32 accumulation; G and the
// outputs stay fp32.
//
// Operand orders.  An MFMA A (B) operand gives lane (g, l16) 8 values of row
// (column) l16 along the contraction.  Operands read from LDS use the
// natural order (slots = 8g .. 8g+7 of a 32-block): rows read directly
// (16 bytes, lds_op_kq) and columns read through the LDS transpose
// (lds_col_issue).  Operands built from accumulators (acc_to_b) and the
// packed 64x64 blocks use the order {4g..4g+3, 16+4g..16+4g+3}, and are only
// ever paired with each other or with the forward's K^T reads (lds_kt_issue).

#include "pm_cdna4.h"
#include "pm_internal.h"

namespace pm {
namespace {

constexpr int kPacked = 6 * 512;  // bf16 elements of one packed 64x64 triangular operand

// Packed index of the upper-triangular operands (T^T, P^T): block (m, kb)
// for (0,0) (0,1) (1,0) (1,1) (2,1) (3,1).
__device__ __forceinline__ int qblk_u(int m, int kb) { return m < 2 ? 2 * m + kb : m + 2; }

// Ties registers filled by asynchronous LDS reads to a wait for all of them.
__device__ __forceinline__ void lds_wait_all() { __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
template <typename V>
__device__ __forceinline__ void tie(V& x) {
    __asm__ volatile("" : "+v"(x));
}

// Natural-order column operand from a swizzled tile with rows of RL
// elements: lane (g, l16) gets M[r0 + 8g + i][c0 + l16], i < 8 (two
// transpose reads; valid after lds_wait_all + tie).
template <int RL>
__device__ __forceinline__ u32x4_t lds_col_issue(const uint16_t* M, int r0, int c0, int lane) {
    const int g = lane >> 4, j = (lane >> 2) & 3, cc = lane & 3;
    const int col = c0 + 4 * cc;
    const int ra = r0 + 8 * g + j, rb = ra + 4;
    const u32x2_t lo = lds_tr16_issue<0>(lds_addr(M + ra * RL + 8 * ((col >> 3) ^ kq_f<RL>(ra)) + (col & 7)));
    const u32x2_t hi = lds_tr16_issue<0>(lds_addr(M + rb * RL + 8 * ((col >> 3) ^ kq_f<RL>(rb)) + (col & 7)));
    const u32x4_t v = {lo.x, lo.y, hi.x, hi.y};
    return v;
}
// Accumulator-layout tile: lane (g, l16) gets M[r0 + 4g + i][c0 + l16], i < 4.
template <int RL>
__device__ __forceinline__ u32x2_t lds_acc_issue(const uint16_t* M, int r0, int c0, int lane) {
    const int g = lane >> 4, j = (lane >> 2) & 3, cc = lane & 3;
    const int col = c0 + 4 * cc, r = r0 + 4 * g + j;
    return lds_tr16_issue<0>(lds_addr(M + r * RL + 8 * ((col >> 3) ^ kq_f<RL>(r)) + (col & 7)));
}
// Element offset of M[r][c .. c+3] in a swizzled tile (c a multiple of 4).
template <int RL>
__device__ __forceinline__ int swz(int r, int c) {
    return r * RL + 8 * ((c >> 3) ^ kq_f<RL>(r)) + (c & 7);
}
__device__ __forceinline__ bf16x8_t as_b(u32x4_t x) { return __builtin_bit_cast(bf16x8_t, x); }

// Packed order of a chunk's W and G in the workspace (written by the reverse sweep in its
// accumulator layout, so each store instruction covers one contiguous block).  Block
// (jt, x) holds column tile jt (columns j = 16 jt + l16) and contraction block x; the piece
// of lane (g, l16) goes to slot w_slot / g_slot, a bijection on 0..63 chosen so that the
// gradient kernel's transposing reads hit every LDS bank once:
//   W (x = m):  4-element pieces W[16m + 4g .. +4][16jt + l16], blocks of 256 elements;
//   G (x = kb): 8-element pieces G[32kb + 8g .. +8][16jt + l16], blocks of 512 elements.
__device__ __forceinline__ int w_slot(int g, int l16) { return 16 * g + (l16 ^ (4 * (g >> 1))); }
__device__ __forceinline__ int g_slot(int g, int l16) { return 16 * g + (l16 ^ (4 * (g & 1))); }
// From the packed W: lane (g, l16) gets W[16m + l16][32kb + 8g + i], i < 8 (two transposing
// reads; valid after lds_wait_all + tie).
__device__ __forceinline__ u32x4_t w_col_issue(const uint16_t* Wp, int kb, int m, int lane) {
    const int g = lane >> 4, jp = (lane >> 2) & 3, cc = lane & 3;
    const int ja = 32 * kb + 8 * g + jp, jb = ja + 4;
    const u32x2_t lo = lds_tr16_issue<0>(lds_addr(Wp + (((ja >> 4) * 4 + m) * 64 + w_slot(cc, ja & 15)) * 4));
    const u32x2_t hi = lds_tr16_issue<0>(lds_addr(Wp + (((jb >> 4) * 4 + m) * 64 + w_slot(cc, jb & 15)) * 4));
    const u32x4_t v = {lo.x, lo.y, hi.x, hi.y};
    return v;
}
// From the packed G: lane (g, l16) gets G[16dt + l16][32kb + 8g + i], i < 8.
template <int D>
__device__ __forceinline__ u32x4_t g_col_issue(const uint16_t* Gp, int kb, int dt, int lane) {
    const int g = lane >> 4, jp = (lane >> 2) & 3, cc = lane & 3;
    const int ja = 32 * kb + 8 * g + jp, jb = ja + 4;
    const int d = 16 * dt + 4 * cc;
    const int e = ((d >> 5) * 64) * 8 + 4 * ((d >> 2) & 1);  // contraction block and half piece
    const int gg = (d & 31) >> 3;
    const u32x2_t lo = lds_tr16_issue<0>(lds_addr(Gp + (ja >> 4) * (D / 32) * 512 + e + g_slot(gg, ja & 15) * 8));
    const u32x2_t hi = lds_tr16_issue<0>(lds_addr(Gp + (jb >> 4) * (D / 32) * 512 + e + g_slot(gg, jb & 15) * 8));
    const u32x4_t v = {lo.x, lo.y, hi.x, hi.y};
    return v;
}

// Copy n_instr KiB of a tile of rows of RL bf16 (rows src_row_bytes apart
// in the buffer) into a swizzled LDS tile; instruction ii (taken by wave
// ii % nw) fills LDS bytes [1024 ii, +1024).
template <int RL>
__device__ __forceinline__ void copy_rows(__amdgpu_buffer_rsrc_t rs, unsigned char* dst, int n_instr,
                                          unsigned src_row_bytes, int w, int nw, int lane) {
    for (int ii = w; ii < n_instr; ii += nw) {
        const int pos = 512 * ii + 8 * lane;
        const int r = pos / RL, p = (pos % RL) / 8;
        copy_to_lds(rs, dst + 1024 * ii, 16, static_cast<unsigned>(r) * src_row_bytes + 16u * (p ^ kq_f<RL>(r)));
    }
}
// Copy n_instr contiguous KiB (no swizzle).
__device__ __forceinline__ void copy_flat(__amdgpu_buffer_rsrc_t rs, unsigned char* dst, int n_instr, int w,
                                          int nw, int lane) {
    for (int ii = w; ii < n_instr; ii += nw)
        copy_to_lds(rs, dst + 1024 * ii, 16, static_cast<unsigned>(1024 * ii + 16 * lane));
}

// ---------------------------------------------------------------------------
// 2. reverse sweep over chunks: G, W, T, dV, dS_0
// ---------------------------------------------------------------------------
template <int D>
struct RevGeo {
    static constexpr int KS = 0;
    static constexpr int QS = KS + kC * D * 2;
    static constexpr int TT = QS + kC * D * 2;  // packed T^T, then packed P^T (built here)
    static constexpr int PT = TT + kPacked * 2;
    static constexpr int NC = 32;                // columns per workgroup (16 per chain wave)
    static constexpr int DO = PT + kPacked * 2;  // dO tile, fp32 [t][NC], 16-byte chunks swizzled
    static constexpr int BS = DO + kC * NC * 4;
    static constexpr int BUF = BS + kC * 4;
    static constexpr int NBUF = 3;  // the loaders run two chunks ahead
    // two ints: the oldest chunk whose K and beta, and whose Q, have landed in LDS
    static constexpr int FLAG = NBUF * BUF;
    static constexpr int BYTES = FLAG + 16;
    static constexpr int THREADS = 320;  // five waves
    // copy instructions per chunk (all by wave 2): K, Q, beta and dO
    static constexpr int N_KQ = kC * D * 2 / 1024, N_DO = kC * NC * 4 / 1024;
    // most memory operations wave 2 has in flight (vmcnt counts to 63): a chunk's dV stores,
    // the next chunk's copies and the one after's, and that one's dV stores
    static_assert(2 * N_KQ + 1 + N_DO + 2 * N_DO <= 63, "vmcnt range");
    static_assert(BUF % 16 == 0 && BYTES <= 160 * 1024, "layout");
};
// dO tile (rows of 32 fp32 = 128 bytes, half the banks): 16-byte chunk p of token row t
// sits at chunk p ^ fdo(t).  The operand reads touch rows 4g + i (same parity) and 16
// consecutive columns per lane group g; the XOR puts odd and even g in different
// bank halves (2-way, the least two 128-byte rows of one parity allow).
__device__ __forceinline__ int fdo(int t) { return 4 * ((t >> 2) & 1); }

template <int D>
__global__ __launch_bounds__(320) __attribute__((amdgpu_waves_per_eu(2, 2))) void bwd_rev_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const float* __restrict__ beta,
    const float* __restrict__ go, const float* __restrict__ gs, uint16_t* __restrict__ t_ws,
    uint16_t* __restrict__ g_hist, uint16_t* __restrict__ w_hist, float* __restrict__ gv,
    float* __restrict__ gs0, int n_pairs, int T, int H, int n_ch, int n_tiles) {
    using G = RevGeo<D>;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    // the n_tiles workgroups of a pair share bid % 8 (one XCD, one L2)
    const int bid = blockIdx.x;
    const int xcd = bid & 7, slot = bid >> 3;
    const int tile = slot % n_tiles;
    const int pair = (slot / n_tiles) * 8 + xcd;
    if (pair >= n_pairs) return;
    const int seq = pair / H, h = pair % H;
    const long tok0 = static_cast<long>(seq) * T;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = static_cast<int>(uniform(static_cast<unsigned>(tid >> 6)));
    const int l16 = lane & 15, lg = lane >> 4;
    // waves 0 and 1 (the chain) carry G (16 columns each) and store G and W.  For the chunks
    // ahead, wave 2 copies K, beta, Q and dO, marks in an LDS flag each chunk whose copies
    // have landed, and stores dV; wave 3 then builds the chunk's T^T (and T), wave 4 its
    // P^T.  No chain wave waits on a copy, a build or a dV store, and no builder's MFMA work
    // queues behind memory instructions.
    const int j = tile * G::NC + 16 * (w & 1) + l16;  // this lane's column of G (chain waves)
    const int jt = j >> 4;                             // its 16-column tile
    const size_t tstride = static_cast<size_t>(H) * D;
    const size_t sbase = static_cast<size_t>(pair) * D * D;

    const int col0 = tile * G::NC;
    auto buf = [&](int c) { return smem + ((n_ch - 1 - c) % G::NBUF) * G::BUF; };
    const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
    auto put = [&](uint16_t* dst, int x, f32x4_t lo, f32x4_t hi) {
        *reinterpret_cast<bf16x8_t*>(dst + x * 512 + lane * 8) = acc_to_b(lo, hi);
    };
    // Wave 2 copies K, beta and then Q of chunk c, and its dO (rows past the chunk's end
    // fall outside the buffer ranges and read as zeros)
    auto issue_kq = [&](int c, bool kpart, bool qpart) {
        const int base = c * kC, clen = min(kC, T - base);
        const size_t row0 = (tok0 + base) * tstride + static_cast<size_t>(h) * D;
        const unsigned n_kq = static_cast<unsigned>(((clen - 1) * tstride + D) * 2);
        unsigned char* b = uniform_ptr(buf(c));
        if (kpart) {
            copy_rows<D>(make_rsrc(k + row0, n_kq), b + G::KS, G::N_KQ, static_cast<unsigned>(tstride * 2), 0, 1,
                         lane);
            copy_to_lds(make_rsrc(beta + (tok0 + base) * H + h, static_cast<unsigned>(((clen - 1) * H + 1) * 4)),
                        b + G::BS, 4, static_cast<unsigned>(lane * H * 4));
        }
        if (qpart)
            copy_rows<D>(make_rsrc(q + row0, n_kq), b + G::QS, G::N_KQ, static_cast<unsigned>(tstride * 2), 0, 1,
                         lane);
    };
    auto issue_do = [&](int c) {
        const int base = c * kC, clen = min(kC, T - base);
        const size_t row0 = (tok0 + base) * tstride + static_cast<size_t>(h) * D;
        unsigned char* b = uniform_ptr(buf(c));
        // dO (fp32): rows of NC values from column col0; a NULL go reads as zeros
        const unsigned n_do = go ? static_cast<unsigned>(((clen - 1) * tstride + G::NC) * 4) : 0u;
        const __amdgpu_buffer_rsrc_t rd = make_rsrc(go ? go + row0 + col0 : go, n_do);
        for (int ii = 0; ii < G::N_DO; ++ii) {
            const int pos = 1024 * ii + 16 * lane;  // byte in the LDS tile
            const int r = pos / (G::NC * 4), p = (pos % (G::NC * 4)) / 16;
            copy_to_lds(rd, b + G::DO + 1024 * ii, 16,
                        static_cast<unsigned>(r * tstride * 4) + 16u * static_cast<unsigned>(p ^ fdo(r)));
        }
    };
    // Wave 3: T^T of chunk c, from its K and beta in LDS, into the chunk's buffer in packed
    // operand order, and T itself (packed, the gradient kernel's operand) into tp.  The
    // forward's builder gives T's blocks both
    // transposed (tb, for T) and not (tn): T^T's packed block (m, kb) is T_(2kb, m) over
    // T_(2kb+1, m) as untransposed tiles, a zero tile where 2kb < m.
    auto build_t = [&](int c, u32x4_t (&tp)[6]) {
        unsigned char* b = uniform_ptr(buf(c));
        const uint16_t* Ks = reinterpret_cast<const uint16_t*>(b + G::KS);
        const float* Bs = reinterpret_cast<const float*>(b + G::BS);
        bf16x8_t f[4][D / 32];
#pragma unroll
        for (int kb = 0; kb < D / 32; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) f[r][kb] = lds_op_kq<D>(Ks, 16 * r + l16, kb, lg);
        f32x4_t br4[4];
        float bc[4];
#pragma unroll
        for (int x = 0; x < 4; ++x) {
            br4[x] = *reinterpret_cast<const f32x4_t*>(Bs + 16 * x + 4 * lg);
            bc[x] = Bs[16 * x + l16];
        }
        f32x4_t tb[10], tn[10];
        t_blocks<D>(f, bc, br4, lane, tb, tn);
        // block (i, j), j <= i, is number i (i + 1) / 2 + j of tb and tn
        uint16_t* TTp = reinterpret_cast<uint16_t*>(b + G::TT);
        put(TTp, qblk_u(0, 0), tn[0], tn[1]);  // T00, T10
        put(TTp, qblk_u(0, 1), tn[3], tn[6]);  // T20, T30
        put(TTp, qblk_u(1, 0), zero, tn[2]);   // T01 = 0, T11
        put(TTp, qblk_u(1, 1), tn[4], tn[7]);  // T21, T31
        put(TTp, qblk_u(2, 1), tn[5], tn[8]);  // T22, T32
        put(TTp, qblk_u(3, 1), zero, tn[9]);   // T23 = 0, T33
        // packed T (block q = qblk(i, kb) holds T_(i, 2kb) and T_(i, 2kb+1) transposed)
        auto pk = [](f32x4_t lo, f32x4_t hi) { return __builtin_bit_cast(u32x4_t, acc_to_b(lo, hi)); };
        tp[qblk(0, 0)] = pk(tb[0], zero);
        tp[qblk(1, 0)] = pk(tb[1], tb[2]);
        tp[qblk(2, 0)] = pk(tb[3], tb[4]);
        tp[qblk(2, 1)] = pk(tb[5], zero);
        tp[qblk(3, 0)] = pk(tb[6], tb[7]);
        tp[qblk(3, 1)] = pk(tb[8], tb[9]);
    };
    // the first tile's workgroup writes T of chunk c for the gradient kernel
    auto store_t = [&](int c, const u32x4_t (&tp)[6]) {
        if (tile != 0) return;
        uint16_t* dst = t_ws + (static_cast<size_t>(pair) * n_ch + c) * kPacked;
#pragma unroll
        for (int x = 0; x < 6; ++x) *reinterpret_cast<u32x4_t*>(dst + x * 512 + lane * 8) = tp[x];
    };
    // Wave 4: P^T of chunk c from its K and Q in LDS.  The accumulator tile of Q_j K_i^T
    // (lane: P[16j + 4g + r][16i + l16]) is the (i, j) part of P^T's packed block (i, j / 2);
    // parts with j < i are zero.  Two column blocks j at a time, stored as soon as formed.
    auto build_p = [&](int c) {
        unsigned char* b = uniform_ptr(buf(c));
        const uint16_t* Ks = reinterpret_cast<const uint16_t*>(b + G::KS);
        const uint16_t* Qs = reinterpret_cast<const uint16_t*>(b + G::QS);
        uint16_t* PTp = reinterpret_cast<uint16_t*>(b + G::PT);
        bf16x8_t f[4][D / 32];
#pragma unroll
        for (int kb = 0; kb < D / 32; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) f[r][kb] = lds_op_kq<D>(Ks, 16 * r + l16, kb, lg);
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
            f32x4_t pa[4][2];
#pragma unroll
            for (int i = 0; i < 4; ++i) pa[i][0] = pa[i][1] = zero;
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const int j = 2 * jb + jj;
#pragma unroll
                for (int kb = 0; kb < D / 32; ++kb) {
                    const bf16x8_t qa = lds_op_kq<D>(Qs, 16 * j + l16, kb, lg);
#pragma unroll
                    for (int i = 0; i <= j; ++i) pa[i][jj] = mfma32(qa, f[i][kb], pa[i][jj]);
                }
            }
#pragma unroll
            for (int i = 2 * jb; i < 2 * jb + 2; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) pa[i][i - 2 * jb][r] = (4 * lg + r >= l16) ? pa[i][i - 2 * jb][r] : 0.f;
            if (jb == 0) {
                put(PTp, qblk_u(0, 0), pa[0][0], pa[0][1]);
                put(PTp, qblk_u(1, 0), zero, pa[1][1]);
            } else {
                put(PTp, qblk_u(0, 1), pa[0][0], pa[0][1]);
                put(PTp, qblk_u(1, 1), pa[1][0], pa[1][1]);
                put(PTp, qblk_u(2, 1), pa[2][0], pa[2][1]);
                put(PTp, qblk_u(3, 1), zero, pa[3][1]);
            }
        }
    };
    // dO as a B operand over tokens 32kb + {4g..4g+3, 16+4g..16+4g+3}, column j
    const int jl = 16 * (w & 1) + l16;  // column within the tile
    auto do_op = [&](const float* Ds, int kb) {
        float f[8];
#pragma unroll
        for (int y = 0; y < 8; ++y) {
            const int t = 32 * kb + (y < 4 ? 4 * lg + y : 12 + 4 * lg + y);
            f[y] = Ds[t * G::NC + 4 * ((jl >> 2) ^ fdo(t)) + (jl & 3)];
        }
        const u32x4_t v = {pack2(f[0], f[1]), pack2(f[2], f[3]), pack2(f[4], f[5]), pack2(f[6], f[7])};
        return as_b(v);
    };

    // Stores that scatter over many rows stall a chain wave while copies are in flight.  So
    // G and W go out in packed order (one contiguous block per instruction), W at the start
    // of the next iteration next to G; and dV, whose rows are 64 bytes per chain wave, is
    // staged in the chunk's dO space (dead once the chain has its dO operands; each wave
    // overwrites only the bytes of its own dO columns) and stored by wave 2 in whole 128-byte
    // rows in the next iteration, before that buffer is refilled.
    u32x2_t w_pend[4];
    uint16_t* wp_pend = nullptr;
    auto store_w = [&] {
#pragma unroll
        for (int m = 0; m < 4; ++m) *reinterpret_cast<u32x2_t*>(wp_pend + m * 256) = w_pend[m];
    };
    // dV of chunk cc from its staging tile (rows of 32 fp32 in the dO tile's order) to gv, in
    // two steps so that copies into the same buffer can be issued between them (the reads
    // complete first); rows past the chunk's end fall outside the buffer range and are
    // dropped (offsets fit 32 bits since H D <= 2^23)
    auto read_dv = [&](int cc, u32x4_t (&x)[G::N_DO]) {
        const float* Ds = reinterpret_cast<const float*>(buf(cc) + G::DO);
#pragma unroll
        for (int ii = 0; ii < G::N_DO; ++ii) {
            const int r = 8 * ii + (lane >> 3), p = lane & 7;
            x[ii] = *reinterpret_cast<const u32x4_t*>(Ds + r * G::NC + 4 * (p ^ fdo(r)));
        }
        lds_wait_all();
#pragma unroll
        for (int ii = 0; ii < G::N_DO; ++ii) tie(x[ii]);
    };
    auto write_dv = [&](int cc, const u32x4_t (&x)[G::N_DO]) {
        const int cb = cc * kC, cl = min(kC, T - cb);
        const __amdgpu_buffer_rsrc_t rv =
            make_rsrc(gv + (tok0 + cb) * tstride + static_cast<size_t>(h) * D + col0,
                      static_cast<unsigned>(((cl - 1) * tstride + G::NC) * 4));
#pragma unroll
        for (int ii = 0; ii < G::N_DO; ++ii) {
            const int r = 8 * ii + (lane >> 3), p = lane & 7;
            __builtin_amdgcn_raw_buffer_store_b128(x[ii], rv, static_cast<unsigned>((r * tstride + 4 * p) * 4), 0, 0);
        }
    };
    // One LDS-only barrier per chunk: by then the chunk the chain takes next is in LDS with
    // its T^T and P^T, and the chain's stores need not complete.  In iteration c (the chain
    // on chunk c) wave 2 waits for chunk c - 1's copies (issued an iteration earlier),
    // marking K and beta as soon as they have landed and then Q, and issues chunk c - 2's;
    // wave 3 waits for the first mark and builds chunk c - 1's T^T, wave 4 for the second
    // and builds its P^T.  The iteration before the chain's first (c = n_ch) does the
    // same for chunk n_ch - 1.  Each role runs its own loop, with the same barriers, so that
    // no value of the chain is live through the builders' code.
    // (an LDS pointer, so that its accesses are ds_ reads and writes, not flat ones, which
    // would wait on the vector memory counter too)
    typedef __attribute__((address_space(3))) volatile int lds_int;
    lds_int* flag = (lds_int*)(smem + G::FLAG);  // [0]: K and beta, [1]: Q
    if (w == 2 && lane < 2) flag[lane] = n_ch;   // nothing landed yet
    lds_barrier();
    // Waves 3 and 4: wait until chunk c's K, Q and beta have landed.  Wave 2 marks every
    // chunk in turn, after its vmcnt wait for the copies and before the barrier that ends
    // the iteration, so the wait ends; its bound only keeps it finite by construction.
    auto wait_mark = [&](int c, int which) {
        for (int spin = 0; spin < (1 << 20); ++spin) {
            if (__builtin_amdgcn_readfirstlane(flag[which]) <= c) break;
            __builtin_amdgcn_s_sleep(1);
        }
    };
    if (w == 2) {
        // chunk c's copies in issue order: K and beta, Q, dO; in iteration c they are waited
        // for one part at a time (each mark as soon as its part has landed), with chunk
        // c + 2's dV stores (issued last in the iteration before, when there was one) still
        // in flight behind them
        if (n_ch > 0) {
            issue_kq(n_ch - 1, true, true);
            issue_do(n_ch - 1);
        }
        constexpr int NK = G::N_KQ + 1, NQ = G::N_KQ, ND = G::N_DO;  // copies of K + beta, Q, dO
        for (int c = n_ch; c > 0; --c) {
            // The newer chunk's K and beta go out as soon as the older chunk's have landed, and
            // its Q once the older Q has: each wait counts what was issued after the part it
            // waits for.  In flight at the top: chunk c - 1's K + beta, Q, dO, then chunk c + 2's
            // dV stores when the last iteration stored (c <= n_ch - 3).
            const bool more = c >= 2;
            if (c <= n_ch - 3) {
                wait_vm_n<NQ + 2 * ND>();
                if (lane == 0) flag[0] = c - 1;
                if (more) {
                    issue_kq(c - 2, true, false);
                    wait_vm_n<2 * ND + NK>();
                    if (lane == 0) flag[1] = c - 1;
                    issue_kq(c - 2, false, true);
                    wait_vm_n<ND + NK + NQ>();  // its dO
                } else {
                    wait_vm_n<2 * ND>();
                    if (lane == 0) flag[1] = c - 1;
                    wait_vm_n<ND>();
                }
            } else {
                wait_vm_n<NQ + ND>();
                if (lane == 0) flag[0] = c - 1;
                if (more) {
                    issue_kq(c - 2, true, false);
                    wait_vm_n<ND + NK>();
                    if (lane == 0) flag[1] = c - 1;
                    issue_kq(c - 2, false, true);
                    wait_vm_n<NK + NQ>();       // its dO
                } else {
                    wait_vm_n<ND>();
                    if (lane == 0) flag[1] = c - 1;
                    wait_copies();
                }
            }
            if (c <= n_ch - 2) {             // dV of chunk c + 1, whose buffer chunk c - 2 takes
                u32x4_t x[G::N_DO];
                read_dv(c + 1, x);
                if (c >= 2) issue_do(c - 2);
                write_dv(c + 1, x);
            } else if (c >= 2) {
                issue_do(c - 2);
            }
            lds_barrier();
        }
        u32x4_t x[G::N_DO];
        if (n_ch > 1) {
            read_dv(1, x);
            write_dv(1, x);
        }
        if (n_ch > 0) {
            lds_barrier();  // chunk 0's dV is staged
            read_dv(0, x);
            write_dv(0, x);
        }
        return;
    }
    if (w == 3) {
        u32x4_t tp[6];
        for (int c = n_ch; c > 0; --c) {
            wait_mark(c - 1, 0);
            build_t(c - 1, tp);
            wait_copies();                   // the last chunk's T stores, long complete
            store_t(c - 1, tp);
            lds_barrier();
        }
        if (n_ch > 0) lds_barrier();
        return;
    }
    if (w == 4) {
        for (int c = n_ch; c > 0; --c) {
            wait_mark(c - 1, 1);
            build_p(c - 1);
            lds_barrier();
        }
        if (n_ch > 0) lds_barrier();
        return;
    }
    // chain waves
    if (n_ch > 0) lds_barrier();  // chunk n_ch - 1 is ready
    f32x4_t Gm[D / 16];
#pragma unroll
    for (int md = 0; md < D / 16; ++md)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            Gm[md][r] = gs ? gs[sbase + static_cast<size_t>(s_row_d(md, 4 * lg + r)) * D + j] : 0.f;
    bf16x8_t Gb[D / 32];
#pragma unroll
    for (int kb = 0; kb < D / 32; ++kb) Gb[kb] = acc_to_b(Gm[2 * kb], Gm[2 * kb + 1]);

    for (int c = n_ch - 1; c >= 0; --c) {
        unsigned char* b = buf(c);
        const uint16_t* Ks = reinterpret_cast<const uint16_t*>(b + G::KS);
        const uint16_t* Qs = reinterpret_cast<const uint16_t*>(b + G::QS);
        const uint16_t* TTp = reinterpret_cast<const uint16_t*>(b + G::TT);
        const uint16_t* PTp = reinterpret_cast<const uint16_t*>(b + G::PT);
        const float* Bs = reinterpret_cast<const float*>(b + G::BS);
        const float* Ds = reinterpret_cast<const float*>(b + G::DO);
        // G_c, the gradient of the state at the end of chunk c, in packed order (Gb[kb] holds
        // G[32kb + 8g .. +8][j], j in column tile jt)
        {
            uint16_t* hp = g_hist + (static_cast<size_t>(pair) * n_ch + c) * D * D + static_cast<size_t>(jt) * D * 16 +
                           g_slot(lg, l16) * 8;
#pragma unroll
            for (int kb = 0; kb < D / 32; ++kb) *reinterpret_cast<bf16x8_t*>(hp + kb * 512) = Gb[kb];
        }
        if (c < n_ch - 1) store_w();
        const bf16x8_t d0 = do_op(Ds, 0), d1 = do_op(Ds, 1);
        // beta of tokens 16m + 4g + [0, 4) (the state update) and 16m + l16 (dV), read now so
        // that the stores below wait on no LDS read
        f32x4_t bq[4];
        float bt[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            bq[m] = *reinterpret_cast<const f32x4_t*>(Bs + 16 * m + 4 * lg);
            bt[m] = Bs[16 * m + l16];
        }
        // Y = K G + P^T dO
        f32x4_t Y[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) Y[m] = zero;
#pragma unroll
        for (int kb = 0; kb < D / 32; ++kb) {
            bf16x8_t fk[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) fk[m] = lds_op_kq<D>(Ks, 16 * m + l16, kb, lg);
#pragma unroll
            for (int m = 0; m < 4; ++m) Y[m] = mfma32(fk[m], Gb[kb], Y[m]);
        }
        Y[0] = mfma32(packed_a(PTp, qblk_u(0, 1), lane), d1, mfma32(packed_a(PTp, qblk_u(0, 0), lane), d0, Y[0]));
        Y[1] = mfma32(packed_a(PTp, qblk_u(1, 1), lane), d1, mfma32(packed_a(PTp, qblk_u(1, 0), lane), d0, Y[1]));
        Y[2] = mfma32(packed_a(PTp, qblk_u(2, 1), lane), d1, Y[2]);
        Y[3] = mfma32(packed_a(PTp, qblk_u(3, 1), lane), d1, Y[3]);
        // G += Q^T dO: it does not depend on W, so its products fill the wait for Y and W
        // (Y took G through Gb, so Gm is free to change)
#pragma unroll
        for (int h4 = 0; h4 < D / 64; ++h4) {
            u32x4_t e0 = lds_kt_issue<D, 0>(Qs, 4 * h4 + 0, lane), f0 = lds_kt_issue<D, 32>(Qs, 4 * h4 + 0, lane);
            u32x4_t e1 = lds_kt_issue<D, 0>(Qs, 4 * h4 + 1, lane), f1 = lds_kt_issue<D, 32>(Qs, 4 * h4 + 1, lane);
            u32x4_t e2 = lds_kt_issue<D, 0>(Qs, 4 * h4 + 2, lane), f2 = lds_kt_issue<D, 32>(Qs, 4 * h4 + 2, lane);
            u32x4_t e3 = lds_kt_issue<D, 0>(Qs, 4 * h4 + 3, lane), f3 = lds_kt_issue<D, 32>(Qs, 4 * h4 + 3, lane);
            lds_wait(e0, f0, e1, f1, e2, f2, e3, f3);
            const u32x4_t qa[4] = {e0, e1, e2, e3}, qb[4] = {f0, f1, f2, f3};
#pragma unroll
            for (int x = 0; x < 4; ++x) {
                Gm[4 * h4 + x] = mfma32(as_b(qa[x]), d0, Gm[4 * h4 + x]);
                Gm[4 * h4 + x] = mfma32(as_b(qb[x]), d1, Gm[4 * h4 + x]);
            }
        }
        // W = T^T Y
        const bf16x8_t Yb0 = acc_to_b(Y[0], Y[1]), Yb1 = acc_to_b(Y[2], Y[3]);
        f32x4_t W[4];
        W[0] = mfma32(packed_a(TTp, qblk_u(0, 1), lane), Yb1, mfma32(packed_a(TTp, qblk_u(0, 0), lane), Yb0, zero));
        W[1] = mfma32(packed_a(TTp, qblk_u(1, 1), lane), Yb1, mfma32(packed_a(TTp, qblk_u(1, 0), lane), Yb0, zero));
        W[2] = mfma32(packed_a(TTp, qblk_u(2, 1), lane), Yb1, zero);
        W[3] = mfma32(packed_a(TTp, qblk_u(3, 1), lane), Yb1, zero);
        // W^T = Y^T T, the same product with the operands swapped: lane (g, l16) holds
        // W[16m + l16][4g .. 4g+3] of its 16 columns, so dV = beta W goes out in 16-byte rows
        f32x4_t WT[4];
        WT[0] = mfma32(Yb1, packed_a(TTp, qblk_u(0, 1), lane), mfma32(Yb0, packed_a(TTp, qblk_u(0, 0), lane), zero));
        WT[1] = mfma32(Yb1, packed_a(TTp, qblk_u(1, 1), lane), mfma32(Yb0, packed_a(TTp, qblk_u(1, 0), lane), zero));
        WT[2] = mfma32(Yb1, packed_a(TTp, qblk_u(2, 1), lane), zero);
        WT[3] = mfma32(Yb1, packed_a(TTp, qblk_u(3, 1), lane), zero);
        // W^T rows (bf16) for the gradient kernel; the state update takes -beta W
        f32x4_t NBW[4];
        float* Dst = reinterpret_cast<float*>(b + G::DO);  // dV staging (the chain's own dO columns)
        wp_pend = w_hist + (static_cast<size_t>(pair) * n_ch + c) * D * kC + static_cast<size_t>(jt) * 4 * 256 +
                  w_slot(lg, l16) * 4;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            NBW[m] = -(bq[m] * W[m]);
            w_pend[m] = cvt4(W[m]);
            const int t = 16 * m + l16;
            *reinterpret_cast<f32x4_t*>(Dst + t * G::NC + 4 * ((4 * (w & 1) + lg) ^ fdo(t))) = bt[m] * WT[m];
        }
        // G -= K^T diag(beta) W (Q^T dO was added above)
        const bf16x8_t nb0 = acc_to_b(NBW[0], NBW[1]), nb1 = acc_to_b(NBW[2], NBW[3]);
#pragma unroll
        for (int h4 = 0; h4 < D / 64; ++h4) {
            u32x4_t a0 = lds_kt_issue<D, 0>(Ks, 4 * h4 + 0, lane), b0 = lds_kt_issue<D, 32>(Ks, 4 * h4 + 0, lane);
            u32x4_t a1 = lds_kt_issue<D, 0>(Ks, 4 * h4 + 1, lane), b1 = lds_kt_issue<D, 32>(Ks, 4 * h4 + 1, lane);
            u32x4_t a2 = lds_kt_issue<D, 0>(Ks, 4 * h4 + 2, lane), b2 = lds_kt_issue<D, 32>(Ks, 4 * h4 + 2, lane);
            u32x4_t a3 = lds_kt_issue<D, 0>(Ks, 4 * h4 + 3, lane), b3 = lds_kt_issue<D, 32>(Ks, 4 * h4 + 3, lane);
            lds_wait(a0, b0, a1, b1, a2, b2, a3, b3);
            const u32x4_t ka[4] = {a0, a1, a2, a3}, kb_[4] = {b0, b1, b2, b3};
#pragma unroll
            for (int x = 0; x < 4; ++x) {
                Gm[4 * h4 + x] = mfma32(as_b(ka[x]), nb0, Gm[4 * h4 + x]);
                Gm[4 * h4 + x] = mfma32(as_b(kb_[x]), nb1, Gm[4 * h4 + x]);
            }
        }
#pragma unroll
        for (int kb = 0; kb < D / 32; ++kb) Gb[kb] = acc_to_b(Gm[2 * kb], Gm[2 * kb + 1]);
        if (c > 0) lds_barrier();
    }
    if (n_ch > 0) {
        lds_barrier();  // chunk 0's dV is staged
        store_w();
    }
#pragma unroll
    for (int md = 0; md < D / 16; ++md)
#pragma unroll
        for (int r = 0; r < 4; ++r) gs0[sbase + static_cast<size_t>(s_row_d(md, 4 * lg + r)) * D + j] = Gm[md][r];
}

// ---------------------------------------------------------------------------
// 3. per-chunk gradients dQ, dK, dbeta (all chunks in parallel)
// ---------------------------------------------------------------------------
template <int D>
struct GradGeo {
    static constexpr int KS = 0;                   // K  [t][d]
    static constexpr int QS = KS + kC * D * 2;     // Q  [t][d]
    static constexpr int VS = QS + kC * D * 2;     // V  [t][j], later U^T [j][t]
    static constexpr int DO = VS + kC * D * 2;     // dO [t][j] (bf16)
    static constexpr int ST = DO + kC * D * 2;     // S^T [j][d]
    static constexpr int GT = ST + D * D * 2;      // G (packed), later dP^T, (beta dA)^T [s][t]
    static constexpr int GT_BYTES = D * D * 2 > 4 * kC * kC ? D * D * 2 : 4 * kC * kC;
    static constexpr int WT = GT + GT_BYTES;       // W (packed)
    static constexpr int TP = WT + D * kC * 2;     // packed T
    static constexpr int BS = TP + kPacked * 2;    // beta
    static constexpr int DB = BS + kC * 4;         // dbeta partial sums [2][4][kC]
    static constexpr int BS2 = DB + 2 * 4 * kC * 4;  // beta of every other chunk
    static constexpr int BYTES = BS2 + kC * 4;
    static constexpr int JW = D / 64;              // 16-column tiles per wave
    static_assert(BYTES <= 160 * 1024, "LDS budget");
};

template <int D>
__global__ __launch_bounds__(256) void bwd_grad_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const float* __restrict__ beta, const float* __restrict__ go, const uint16_t* __restrict__ s_hist,
    const uint16_t* __restrict__ g_hist, const uint16_t* __restrict__ w_hist,
    const uint16_t* __restrict__ tp_ws, float* __restrict__ gq, float* __restrict__ gk,
    float* __restrict__ gbeta, int T, int H, int n_ch, int n_total) {
    using G = GradGeo<D>;
    constexpr int JW = G::JW;
    constexpr int NDO = kC * D / 4 / 256;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = static_cast<int>(uniform(static_cast<unsigned>(tid >> 6)));
    const int l16 = lane & 15, lg = lane >> 4;
    const size_t tstride = static_cast<size_t>(H) * D;

    // beta alternates between two buffers by chunk, so the next chunk's is copied while
    // phase 3 still reads the current one
    int par = 0;
    uint16_t* Ks = reinterpret_cast<uint16_t*>(smem + G::KS);
    uint16_t* Qs = reinterpret_cast<uint16_t*>(smem + G::QS);
    uint16_t* Vs = reinterpret_cast<uint16_t*>(smem + G::VS);
    uint16_t* Ut = Vs;
    uint16_t* DOs = reinterpret_cast<uint16_t*>(smem + G::DO);
    uint16_t* St = reinterpret_cast<uint16_t*>(smem + G::ST);
    uint16_t* Gt = reinterpret_cast<uint16_t*>(smem + G::GT);
    uint16_t* dPt = Gt;
    uint16_t* dAt = Gt + kC * kC;
    uint16_t* Wt = reinterpret_cast<uint16_t*>(smem + G::WT);
    const uint16_t* Tp = reinterpret_cast<const uint16_t*>(smem + G::TP);
    const float* Bs = reinterpret_cast<const float*>(smem + G::BS);
    auto set_par = [&](int p) {
        par = p;
        Bs = reinterpret_cast<const float*>(smem + (p ? G::BS2 : G::BS));
    };
    float* db1 = reinterpret_cast<float*>(smem + G::DB);  // [wave][t]: W . (V - K S)
    float* db2 = db1 + 4 * kC;                             // [wave][t]: sum_s dA (k_t . k_s)

    // Persistent: workgroup b takes chunks b, b + gridDim.x, ...  Memory stays busy through
    // all three phases:
    //   * phase 1: this chunk's G and Q, and the previous chunk's dQ/dK stores;
    //   * phase 2 (reads U^T, W, S^T, G, dO): the next chunk's K, beta, T and dO (phase 1
    //     read K and T last; phase 3's K operands are taken into registers before it);
    //   * phase 3 (reads K's registers, Q, dP^T, dA^T, beta): the next chunk's V, S^T, W.
    // The one barrier between chunks waits for LDS traffic only, so the dQ/dK stores run
    // on into the next chunk.
    struct Ref {
        long tok0;
        int h, base, clen;
        size_t row0, cidx;
    };
    auto ref_of = [&](int idx) {
        Ref r;
        const int pair = idx / n_ch, c = idx % n_ch;
        r.h = pair % H;
        r.tok0 = static_cast<long>(pair / H) * T;
        r.base = c * kC;
        r.clen = min(kC, T - r.base);
        r.row0 = (r.tok0 + r.base) * tstride + static_cast<size_t>(r.h) * D;
        r.cidx = static_cast<size_t>(pair) * n_ch + c;
        return r;
    };
    // dO (fp32) into registers with buffer loads (rows past the chunk's end, and a NULL
    // go, read as zeros); written to LDS as bf16 token rows once they have landed
    f32x4_t xdo[NDO];
    auto load_do = [&](const Ref& r) {
        const __amdgpu_buffer_rsrc_t rgo = make_rsrc(
            go ? go + r.row0 : nullptr, go ? static_cast<unsigned>(((r.clen - 1) * tstride + D) * 4) : 0u);
#pragma unroll
        for (int i = 0; i < NDO; ++i) {
            const int e = tid + 256 * i, t = e / (D / 4), d = 4 * (e % (D / 4));
            xdo[i] = __builtin_bit_cast(
                f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rgo, static_cast<unsigned>((t * tstride + d) * 4), 0, 0));
        }
    };
    auto store_do = [&]() {
#pragma unroll
        for (int i = 0; i < NDO; ++i) {
            const int e = tid + 256 * i, t = e / (D / 4), d = 4 * (e % (D / 4));
            *reinterpret_cast<u32x2_t*>(DOs + swz<D>(t, d)) = cvt4(xdo[i]);
        }
    };
    // the inputs phase 3 does not read: V (later U^T), S^T, W^T
    auto copy_a = [&](const Ref& r) {
        const unsigned n_kq = static_cast<unsigned>(((r.clen - 1) * tstride + D) * 2);
        const unsigned rb = static_cast<unsigned>(tstride * 2);
        copy_rows<D>(make_rsrc(v + r.row0, n_kq), smem + G::VS, kC * D * 2 / 1024, rb, w, 4, lane);
        copy_rows<D>(make_rsrc(s_hist + r.cidx * D * D, D * D * 2), smem + G::ST, D * D * 2 / 1024, D * 2, w, 4, lane);
        copy_flat(make_rsrc(w_hist + r.cidx * D * kC, D * kC * 2), smem + G::WT, D * kC * 2 / 1024, w, 4, lane);
    };
    auto copy_t = [&](const Ref& r) {
        copy_flat(make_rsrc(tp_ws + r.cidx * kPacked, kPacked * 2), smem + G::TP, kPacked * 2 / 1024, w, 4, lane);
    };
    // K and beta, copied while phase 2 runs: K over the K that phase 1 read last, beta into
    // the other buffer (phase 3 still reads the current one)
    auto copy_k = [&](const Ref& r, int p) {
        const unsigned n_kq = static_cast<unsigned>(((r.clen - 1) * tstride + D) * 2);
        const unsigned rb = static_cast<unsigned>(tstride * 2);
        copy_rows<D>(make_rsrc(k + r.row0, n_kq), smem + G::KS, kC * D * 2 / 1024, rb, w, 4, lane);
        if (w == 3)
            copy_to_lds(make_rsrc(beta + (r.tok0 + r.base) * H + r.h, static_cast<unsigned>(((r.clen - 1) * H + 1) * 4)),
                        smem + (p ? G::BS2 : G::BS), 4, static_cast<unsigned>(lane * H * 4));
    };
    // G (read in phase 2) and Q (read in phase 3), into space phase 3 of the chunk before
    // read last, copied while phase 1 runs
    auto copy_qg = [&](const Ref& r) {
        const unsigned n_kq = static_cast<unsigned>(((r.clen - 1) * tstride + D) * 2);
        const unsigned rb = static_cast<unsigned>(tstride * 2);
        copy_flat(make_rsrc(g_hist + r.cidx * D * D, D * D * 2), smem + G::GT, D * D * 2 / 1024, w, 4, lane);
        copy_rows<D>(make_rsrc(q + r.row0, n_kq), smem + G::QS, kC * D * 2 / 1024, rb, w, 4, lane);
    };

    int idx = blockIdx.x;
    if (idx >= n_total) return;  // whole workgroup, before any barrier
    Ref cur = ref_of(idx);
    load_do(cur);
    copy_k(cur, 0);
    copy_a(cur);
    copy_t(cur);
    store_do();
    wait_copies();
    __syncthreads();
    for (;;) {
        const long tok0 = cur.tok0;
        const int h = cur.h, base = cur.base, clen = cur.clen;
        const size_t row0 = cur.row0;
        const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
        copy_qg(cur);

        // ---- phase 1: R' = V - K S and U = T diag(beta) R' for this wave's columns ----
        // The lower 16x16 tiles (m, st), m >= st, numbered 0..9 row by row, go to waves by
        // number mod 4 (wave w takes tiles w, w + 4, w + 8): KK = K K^T here in phase 1, from
        // the K operands X = K S reads anyway; dP = dO U^T and dA = -W U^T in phase 2.
        constexpr int kTiles = 3;
        auto tile_m = [](int idx) { return idx >= 6 ? 3 : idx >= 3 ? 2 : idx >= 1 ? 1 : 0; };
        auto tile_s = [&](int idx) { const int m = tile_m(idx); return idx - m * (m + 1) / 2; };
        const int nt = w < 2 ? 3 : 2;
        int tm[kTiles], ts[kTiles];
#pragma unroll
        for (int x = 0; x < kTiles; ++x) {
            const int idx = min(w + 4 * x, 9);
            tm[x] = tile_m(idx);
            ts[x] = tile_s(idx);
        }
        f32x4_t KK[kTiles];
#pragma unroll
        for (int x = 0; x < kTiles; ++x) KK[x] = zero;
        f32x4_t U[4][JW];
        {
            f32x4_t X[4][JW];
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int jj = 0; jj < JW; ++jj) X[m][jj] = zero;
#pragma unroll
            for (int kb = 0; kb < D / 32; ++kb) {
                bf16x8_t fk[4], fs[JW];
#pragma unroll
                for (int m = 0; m < 4; ++m) fk[m] = lds_op_kq<D>(Ks, 16 * m + l16, kb, lg);
#pragma unroll
                for (int jj = 0; jj < JW; ++jj) fs[jj] = lds_op_kq<D>(St, 16 * (JW * w + jj) + l16, kb, lg);
#pragma unroll
                for (int m = 0; m < 4; ++m)
#pragma unroll
                    for (int jj = 0; jj < JW; ++jj) X[m][jj] = mfma32(fk[m], fs[jj], X[m][jj]);
#pragma unroll
                for (int x = 0; x < kTiles; ++x) {
                    if (x < nt) {
                        // rows tm[x] and ts[x] of K without dynamic register indexing
                        bf16x8_t ka = fk[0], kc = fk[0];
#pragma unroll
                        for (int m = 1; m < 4; ++m) {
                            if (tm[x] == m) ka = fk[m];
                            if (ts[x] == m) kc = fk[m];
                        }
                        KK[x] = mfma32(ka, kc, KK[x]);
                    }
                }
            }
            f32x4_t dbp[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) dbp[m] = zero;
#pragma unroll
            for (int jj = 0; jj < JW; ++jj) {
                const int jt = JW * w + jj;
                u32x2_t vv0 = lds_acc_issue<D>(Vs, 0, 16 * jt, lane), vv1 = lds_acc_issue<D>(Vs, 16, 16 * jt, lane);
                u32x2_t vv2 = lds_acc_issue<D>(Vs, 32, 16 * jt, lane), vv3 = lds_acc_issue<D>(Vs, 48, 16 * jt, lane);
                lds_wait(vv0, vv1, vv2, vv3);
                const u32x2_t vv[4] = {vv0, vv1, vv2, vv3};
                f32x4_t R[4];
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const int t0 = 16 * m + 4 * lg;
                    const f32x4_t rp = widen4(vv[m]) - X[m][jj];  // V - K S
                    const f32x4_t wv = widen4(*reinterpret_cast<const u32x2_t*>(Wt + ((jt * 4 + m) * 64 + w_slot(lg, l16)) * 4));
                    dbp[m] += wv * rp;
                    R[m] = *reinterpret_cast<const f32x4_t*>(Bs + t0) * rp;
                }
                const bf16x8_t Rb0 = acc_to_b(R[0], R[1]), Rb1 = acc_to_b(R[2], R[3]);
                U[0][jj] = mfma32(packed_a(Tp, 0, lane), Rb0, zero);
                U[1][jj] = mfma32(packed_a(Tp, 1, lane), Rb0, zero);
                U[2][jj] = mfma32(packed_a(Tp, 3, lane), Rb1, mfma32(packed_a(Tp, 2, lane), Rb0, zero));
                U[3][jj] = mfma32(packed_a(Tp, 5, lane), Rb1, mfma32(packed_a(Tp, 4, lane), Rb0, zero));
            }
            // dbeta, first term: sum over this wave's columns (lanes l16, then its tiles)
#pragma unroll
            for (int m = 0; m < 4; ++m) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    dbp[m][r] = row16_sum(dbp[m][r]);
                }
                if (l16 == 0) *reinterpret_cast<f32x4_t*>(db1 + w * kC + 16 * m + 4 * lg) = dbp[m];
            }
        }
        // phase 3's K operands, taken into registers now: the next chunk's K lands over
        // them while phase 2 runs
        u32x4_t fkc[2][JW];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int dd = 0; dd < JW; ++dd) fkc[kb][dd] = lds_col_issue<D>(Ks, 32 * kb, 16 * (JW * w + dd), lane);
        lds_wait_all();
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int dd = 0; dd < JW; ++dd) tie(fkc[kb][dd]);
        wait_copies();    // Q and G (and the previous chunk's dQ/dK stores)
        __syncthreads();  // V is dead: its space takes U^T; K and T are free
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int jj = 0; jj < JW; ++jj)
                *reinterpret_cast<u32x2_t*>(Ut + swz<kC>(16 * (JW * w + jj) + l16, 16 * m + 4 * lg)) = cvt4(U[m][jj]);
        __syncthreads();
        // the next chunk's K, beta, T and dO, fetched while phase 2 runs
        const int nidx = idx + static_cast<int>(gridDim.x);
        const bool more = nidx < n_total;
        Ref nxt{};
        if (more) {
            nxt = ref_of(nidx);
            load_do(nxt);
            copy_k(nxt, par ^ 1);
            copy_t(nxt);
        }

        // ---- phase 2: products contracting over the d_v index j ----
        // dQ1 = dO S^T, dKa = U G^T, dKb = W S^T for this wave's d tiles; dP = dO U^T and
        // dA = -W U^T for its lower tiles.
        f32x4_t dQ[4][JW], dKa[4][JW], dKb[4][JW];
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int dd = 0; dd < JW; ++dd) {
                dQ[m][dd] = zero;
                dKa[m][dd] = zero;
                dKb[m][dd] = zero;
            }
        f32x4_t dP[kTiles], dA[kTiles];
#pragma unroll
        for (int x = 0; x < kTiles; ++x) dP[x] = dA[x] = zero;
#pragma unroll
        for (int kb = 0; kb < D / 32; ++kb) {
            u32x4_t fu[4], fw[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                fu[m] = lds_col_issue<kC>(Ut, 32 * kb, 16 * m, lane);
                fw[m] = w_col_issue(Wt, kb, m, lane);
            }
            u32x4_t fst[JW], fgt[JW];
#pragma unroll
            for (int dd = 0; dd < JW; ++dd) {
                fst[dd] = lds_col_issue<D>(St, 32 * kb, 16 * (JW * w + dd), lane);
                fgt[dd] = g_col_issue<D>(Gt, kb, JW * w + dd, lane);
            }
            bf16x8_t fdo[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) fdo[m] = lds_op_kq<D>(DOs, 16 * m + l16, kb, lg);
            lds_wait_all();
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                tie(fu[m]);
                tie(fw[m]);
            }
#pragma unroll
            for (int dd = 0; dd < JW; ++dd) {
                tie(fst[dd]);
                tie(fgt[dd]);
            }
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int dd = 0; dd < JW; ++dd) {
                    // operands swapped: the tiles hold dQ^T, dK^T (lane: 4 consecutive d of a token)
                    dQ[m][dd] = mfma32(as_b(fst[dd]), fdo[m], dQ[m][dd]);
                    dKa[m][dd] = mfma32(as_b(fgt[dd]), as_b(fu[m]), dKa[m][dd]);
                    dKb[m][dd] = mfma32(as_b(fst[dd]), as_b(fw[m]), dKb[m][dd]);
                }
#pragma unroll
            for (int x = 0; x < kTiles; ++x) {
                if (x < nt) {
                    // select row block tm[x] and column block ts[x] without dynamic register indexing
                    bf16x8_t ado = fdo[0];
                    u32x4_t aw = fw[0], bu = fu[0];
#pragma unroll
                    for (int m = 1; m < 4; ++m) {
                        if (tm[x] == m) {
                            ado = fdo[m];
                            aw = fw[m];
                        }
                        if (ts[x] == m) bu = fu[m];
                    }
                    dP[x] = mfma32(ado, as_b(bu), dP[x]);
                    dA[x] = mfma32(as_b(aw), as_b(bu), dA[x]);
                }
            }
        }
        // masks, dbeta second term, beta dA
        f32x4_t db2p[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) db2p[m] = zero;
#pragma unroll
        for (int x = 0; x < kTiles; ++x) {
            if (x < nt) {
                const int m = tm[x], st = ts[x];
                const int t0 = 16 * m + 4 * lg, s = 16 * st + l16;
                const f32x4_t bs = *reinterpret_cast<const f32x4_t*>(Bs + t0);
                f32x4_t e = zero;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (t0 + r < s) dP[x][r] = 0.f;
                    const float a = (t0 + r > s) ? -dA[x][r] : 0.f;
                    e[r] = a * KK[x][r];
                    dA[x][r] = bs[r] * a;
                }
#pragma unroll
                for (int mm = 0; mm < 4; ++mm)
                    if (mm == m) db2p[mm] += e;
            }
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                db2p[m][r] = row16_sum(db2p[m][r]);
            }
            if (l16 == 0) *reinterpret_cast<f32x4_t*>(db2 + w * kC + 16 * m + 4 * lg) = db2p[m];
        }
        __syncthreads();  // G^T is dead: its space takes dP^T and (beta dA)^T
#pragma unroll
        for (int x = 0; x < kTiles; ++x) {
            if (x < nt) {
                const int o = swz<kC>(16 * ts[x] + l16, 16 * tm[x] + 4 * lg);
                *reinterpret_cast<u32x2_t*>(dPt + o) = cvt4(dP[x]);
                *reinterpret_cast<u32x2_t*>(dAt + o) = cvt4(dA[x]);
            }
        }
        {
            // the upper tiles (m < st) are zero; 6 of them, numbered row by row, by number mod 4
            int idx = 0;
            const u32x2_t z2 = {0u, 0u};
            for (int m = 0; m < 4; ++m)
                for (int st = m + 1; st < 4; ++st, ++idx)
                    if ((idx & 3) == w) {
                        const int o = swz<kC>(16 * st + l16, 16 * m + 4 * lg);
                        *reinterpret_cast<u32x2_t*>(dPt + o) = z2;
                        *reinterpret_cast<u32x2_t*>(dAt + o) = z2;
                    }
        }
        __syncthreads();

        // the next chunk's V, S^T and W^T, into space phase 3 does not read
        if (more) copy_a(nxt);

        // ---- phase 3: products contracting over tokens ----
        // dQ += dP K;  dKc = dP^T Q + (beta dA)^T K + (beta dA) K
        f32x4_t dKc[4][JW];
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int dd = 0; dd < JW; ++dd) dKc[m][dd] = zero;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            u32x4_t fqc[JW], fpc[4], fac[4];
#pragma unroll
            for (int dd = 0; dd < JW; ++dd) fqc[dd] = lds_col_issue<D>(Qs, 32 * kb, 16 * (JW * w + dd), lane);
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                fpc[m] = lds_col_issue<kC>(dPt, 32 * kb, 16 * m, lane);
                fac[m] = lds_col_issue<kC>(dAt, 32 * kb, 16 * m, lane);
            }
            bf16x8_t fpr[4], far[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                fpr[m] = lds_op_kq<kC>(dPt, 16 * m + l16, kb, lg);
                far[m] = lds_op_kq<kC>(dAt, 16 * m + l16, kb, lg);
            }
            lds_wait_all();
#pragma unroll
            for (int dd = 0; dd < JW; ++dd) tie(fqc[dd]);
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                tie(fpc[m]);
                tie(fac[m]);
            }
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int dd = 0; dd < JW; ++dd) {
                    dQ[m][dd] = mfma32(as_b(fkc[kb][dd]), as_b(fpc[m]), dQ[m][dd]);
                    dKc[m][dd] = mfma32(as_b(fqc[dd]), fpr[m], dKc[m][dd]);
                    dKc[m][dd] = mfma32(as_b(fkc[kb][dd]), far[m], dKc[m][dd]);
                    dKc[m][dd] = mfma32(as_b(fkc[kb][dd]), as_b(fac[m]), dKc[m][dd]);
                }
        }
        // outputs: lane (g, l16) holds d = 16 dt + 4g + [0, 4) of token 16m + l16 (16-byte
        // stores).  Range-checked buffer stores (rows past the chunk's end are dropped), so
        // every wave issues exactly kStores of them whatever the chunk's length.
        constexpr int kStores = 2 * 4 * JW;
        {
            const unsigned nb = static_cast<unsigned>(((clen - 1) * tstride + D) * 4);
            const __amdgpu_buffer_rsrc_t rq = make_rsrc(gq + row0, nb), rk = make_rsrc(gk + row0, nb);
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const int t = 16 * m + l16;
                const float bt = Bs[t];
#pragma unroll
                for (int dd = 0; dd < JW; ++dd) {
                    const int d0 = 16 * (JW * w + dd) + 4 * lg;
                    const f32x4_t kk = dKa[m][dd] - bt * dKb[m][dd] + dKc[m][dd];
                    const unsigned off = static_cast<unsigned>((t * tstride + d0) * 4);
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, dQ[m][dd]), rq, off, 0, 0);
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, kk), rk, off, 0, 0);
                }
            }
        }
        auto store_gbeta = [&]() {
            if (tid < clen) {
                float s = 0.f;
#pragma unroll
                for (int x = 0; x < 4; ++x) s += db1[x * kC + tid];
#pragma unroll
                for (int x = 0; x < 4; ++x) s += db2[x * kC + tid];
                gbeta[(tok0 + base + tid) * H + h] = s;
            }
        };
        if (!more) {
            store_gbeta();
            break;
        }
        // No barrier before these: phase 3 reads neither dO's space nor the next chunk's
        // copies, and the dbeta sums were complete at the barrier before phase 3.  The
        // dQ/dK stores stay in flight into the next chunk.
        store_do();            // waits for this wave's dO loads only
        wait_vm_n<kStores>();  // and its copies, issued before the stores
        store_gbeta();
        lds_barrier();         // every wave's copies have landed; db1/db2 and dO are free
        idx = nidx;
        cur = nxt;
        set_par(par ^ 1);
    }
}

template <typename Kern>
hipError_t set_lds(Kern kern, int bytes) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                               bytes);
}

template <int D>
hipError_t launch_d(const BwdArgs& a, hipStream_t st) {
    const int n_ch = (a.T + kC - 1) / kC;
    const ChunkedBwdWs ws = chunked_bwd_ws(a.n_pairs, a.T, D);
    unsigned char* base = reinterpret_cast<unsigned char*>(a.workspace);
    uint16_t* s_hist = reinterpret_cast<uint16_t*>(base + ws.s_hist);
    uint16_t* g_hist = reinterpret_cast<uint16_t*>(base + ws.g_hist);
    uint16_t* w_hist = reinterpret_cast<uint16_t*>(base + ws.w_hist);
    uint16_t* tp = reinterpret_cast<uint16_t*>(base + ws.tp);
    const uint16_t* q = static_cast<const uint16_t*>(a.q);
    const uint16_t* k = static_cast<const uint16_t*>(a.k);
    const uint16_t* v = static_cast<const uint16_t*>(a.v);
    hipError_t e;
    if (n_ch > 0) {
        ChunkedArgs f{q, k, v, a.beta, a.s0, nullptr, nullptr, nullptr, a.n_pairs / a.H, a.T, a.H, D, false, 0};
        if ((e = launch_chunked_states(f, s_hist, st)) != hipSuccess) return e;
    }
    const int n_tiles = D / RevGeo<D>::NC;
    const int slots = (a.n_pairs + 7) / 8;
    if ((e = set_lds(bwd_rev_kernel<D>, RevGeo<D>::BYTES)) != hipSuccess) return e;
    hipLaunchKernelGGL(bwd_rev_kernel<D>, dim3(static_cast<unsigned>(slots * 8 * n_tiles)), dim3(RevGeo<D>::THREADS),
                       RevGeo<D>::BYTES, st, q, k, a.beta, a.go, a.gs, tp, g_hist, w_hist, a.gv, a.gs0,
                       a.n_pairs, a.T, a.H, n_ch, n_tiles);
    if ((e = hipGetLastError()) != hipSuccess || n_ch == 0) return e;
    if ((e = set_lds(bwd_grad_kernel<D>, GradGeo<D>::BYTES)) != hipSuccess) return e;
    // persistent: one workgroup per CU (its LDS allows no more), each taking every
    // gridDim.x-th chunk
    int dev = 0, n_cu = 0;
    if ((e = hipGetDevice(&dev)) != hipSuccess) return e;
    if ((e = hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
    const long n_total = static_cast<long>(a.n_pairs) * n_ch;
    if (n_total > (1L << 30)) return hipErrorInvalidValue;  // chunk indices stay in int
    const long grid = n_total < n_cu ? n_total : (n_cu > 0 ? n_cu : 1);
    hipLaunchKernelGGL(bwd_grad_kernel<D>, dim3(static_cast<unsigned>(grid)), dim3(256), GradGeo<D>::BYTES, st, q,
                       k, v, a.beta, a.go, s_hist, g_hist, w_hist, tp, a.gq, a.gk, a.gbeta, a.T, a.H, n_ch,
                       static_cast<int>(n_total));
    return hipGetLastError();
}

}  // namespace

ChunkedBwdWs chunked_bwd_ws(long n_pairs, int T, int D) {
    const size_t n = static_cast<size_t>(n_pairs) * ((T + kC - 1) / kC);
    ChunkedBwdWs w;
    w.s_hist = 0;
    w.g_hist = w.s_hist + n * D * D * 2;
    w.w_hist = w.g_hist + n * D * D * 2;
    w.tp = w.w_hist + n * D * kC * 2;
    w.bytes = w.tp + n * kPacked * 2;
    return w;
}

// 32-bit buffer offsets: a chunk of fp32 dO spans 64 token rows of H*D values.
bool chunked_bwd_supported(int D, int H) {
    return chunked_supported(D, H) && static_cast<long>(H) * D <= (1L << 23);
}

hipError_t launch_bwd_chunked(const BwdArgs& a, hipStream_t st) {
    if (a.n_pairs == 0) return hipSuccess;
    if (!a.in_bf16 || !chunked_bwd_supported(a.D, a.H)) return hipErrorInvalidValue;
    return a.D == 128 ? launch_d<128>(a, st) : launch_d<64>(a, st);
}

}  // namespace pm
