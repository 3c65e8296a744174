// kda_chunked.hip — K8: the delta rule with a decay per key channel (KDA) in
// chunked WY form on bf16 MFMA, for bf16 q/k/v and D in {64, 128}.
//
// Per token, with alpha_t = exp(g_t) a d_k-vector (g (B, T, H, D) log-gates):
//   S_t = (I - beta_t k_t k_t^T) Diag(alpha_t) S_{t-1} + beta_t k_t v_t^T,  o_t = q_t S_t.
// Per chunk of C = 64 tokens with start state S and G_t = sum_{j <= t} g_j (per channel,
// from the chunk's start), unrolling the recurrence gives
//   A'[t][s] = sum_d k_t[d] k_s[d] exp(G_t[d] - G_s[d])   (s < t)
//   T = (I + strict_lower(diag(beta) A'))^-1,   U = T diag(beta) (V - K^ S)
//   O = Q^ S + P U,   P[t][s] = sum_d q_t[d] k_s[d] exp(G_t[d] - G_s[d])   (s <= t)
//   S <- Diag(exp(G_C)) S + K-^T U
// with K^ = K exp(G), Q^ = Q exp(G) and K- = K exp(G_C - G) (row t scaled per channel).
// Every factor in K^, Q^, K- is at most 1 (g <= 0).  A' and P are Gram matrices whose
// entries need exp(G_t - G_s) inside the sum over d, so each 16x16 block is one MFMA
// product of two operands scaled against a reference token r between them:
//   k_t exp(G_t - G_r)  and  k_s exp(G_r - G_s).
// Off-diagonal blocks (s in block j < i, t in block i) take r = the last token of block
// j: both factors are at most 1.  Diagonal blocks take r = 16 b + 7 (mid-block): the
// factors reach exp(8 |g|) for the tokens on the far side of r (only the products with
// s <= t are kept, and each of those is at most 1).  The kernel clamps g into [-10, 1],
// which keeps every factor below 2^116 (fp32 and bf16 share that range); a log-gate
// below -10 keeps alpha = exp(-10) = 4.5e-5 of the state instead of less, a difference
// below bf16 resolution.  The per-token kernel (delta_recurrent.hip) takes g as given.
//
// K8p (prepass, 256-thread workgroups, two per CU, each walking (b, h, chunk) items with
// the next item's K and Q loaded during the current one; all chunks independent):
// the clamped prefix sums G (LDS), then T'' = -T diag(beta) (the decayed Gram blocks on
// waves 0 and 1, t_from_gram on wave 0), P (waves 2 and 3) and the recurrence's operands
// K^, Q^, K-^T and exp(G_C), all written to the workspace in MFMA operand order (1 KiB
// blocks, 16 bytes per lane), so that the recurrence only copies them.
// K8s (recurrence, one workgroup of four waves per (b, h, 32 columns of d_v)): two
// chain waves own 16 columns of S each as fp32 accumulators and two output waves form O
// for the same columns; chunk c + 1's workspace image and V tile are copied HBM -> LDS
// (buffer_load ... lds) while chunk c runs from LDS: X = K^ S - V, U = T'' bf16(X),
// S = exp(G_C) S + K-^T U on the chain, O^T = S^T Q^T + U^T P^T on the output waves
// (stored as rows).  Two LDS-only barriers per chunk (U handed over, chunk done).

#include "pm_cdna4.h"
#include "pm_internal.h"

namespace pm {
namespace {

constexpr float kKdaGMin = -10.f, kKdaGMax = 1.f;
constexpr float kLog2E = 1.44269504088896341f;

// One chunk's slot in the workspace (byte offsets): operand blocks of 1 KiB.
template <int D>
struct KdaWs {
    static constexpr int NKB = D / 32;
    static constexpr int NOP = NKB * 4;        // blocks of K^, Q^ or K-^T
    static constexpr int KH = 0;               // K^: block kb * 4 + m
    static constexpr int QH = KH + NOP * 1024; // Q^: same
    static constexpr int KT = QH + NOP * 1024; // K-^T: block md * 2 + half
    static constexpr int TT = KT + NOP * 1024; // T'' packed (6 blocks)
    static constexpr int PP = TT + 6 * 1024;   // P packed (6 blocks)
    static constexpr int DEC = PP + 6 * 1024;  // exp(G_C): [g][md][r] fp32 (D floats), rest zero
    static constexpr int BYTES = DEC + 1024;
    static constexpr int NBLK = BYTES / 1024;
};

// ---------------------------------------------------------------- K8p
// Every decayed operand factors into a per-element part and a per-channel part.  With
// m(b) = 16 b + 7 the middle of block b and e(b) = 16 b + 15 its last token, per element
// of block b (G in log2 units)
//   a_t = exp2(G_t - G_{m(b)}),   r_t = exp2(G_{m(b)} - G_t),
// which the clamp keeps within 2^(+-116) (kept as bf16, which has fp32's exponent range):
//   diagonal left / right    k_t a_t,  k_s r_s          (q_t a_t for P)
//   off-diagonal left        k_t a_t cX(i, k),   cX = exp2(G_{m(i)} - G_{e(k)})   (k < i)
//   off-diagonal right       k_s r_s cE(k),      cE = exp2(G_{e(k)} - G_{m(k)})
//   K^, Q^                   x_t a_t cH(b),      cH = exp2(G_{m(b)})
//   K-                       k_t r_t cB(b),      cB = exp2(G_C - G_{m(b)})
// Every channel vector is at most 1 (g <= 0), so where one underflows the product it
// stands for is below 2^-48 (a and r stay above 2^-116).  The prepass forms, once per
// element, the bf16 tiles K a, K r and Q a (two exponentials per element): the diagonal
// blocks' operands are then plain reads, every other operand one product with a channel
// vector (18 of them).
template <int D>
struct KdaPrepLds {
    static constexpr int NCV = 18;                // channel vectors (see cvec)
    static constexpr int KA = 0;                  // K a, K r, Q a: bf16 [64][D], 16-byte chunk c
    static constexpr int KR = KA + kC * D * 2;    // of row t at c ^ (t mod D/8)
    static constexpr int QA = KR + kC * D * 2;
    static constexpr int GS = KA;                 // G fp32 [64][D] until K a and K r replace it
    static constexpr int CV = QA + kC * D * 2;    // channel vectors fp32 [NCV][D]
    static constexpr int BS = CV + NCV * D * 4;   // beta
    static constexpr int GU = BS + kC * 4;        // the six off-diagonal Gram tiles, wave 1 -> wave 0
    static constexpr int TOT = GU + 6 * 1024;
    static_assert(2 * TOT <= 160 * 1024, "two workgroups per CU");
};
// channel vectors: cX for the pairs (k, i) = (0,1) (0,2) (1,2) (0,3) (1,3) (2,3), cE(0..2),
// cH(0..3), cB(0..3), exp2(G_C)
constexpr int kCvX = 0, kCvE = 6, kCvH = 9, kCvB = 13, kCvD = 17;
// index of the pair (k, i), k < i, in that order
__host__ __device__ constexpr int kda_pair(int k, int i) { return i == 1 ? 0 : i == 2 ? 1 + k : 3 + k; }

template <int D>
__device__ __forceinline__ int kda_swz(int t) { return t & (D / 8 - 1); }
// 16 bytes (8 elements from d0 = 8 c) of row t of a swizzled bf16 tile
template <int D>
__device__ __forceinline__ u32x4_t kda_row16(const uint16_t* base, int t, int c) {
    return *reinterpret_cast<const u32x4_t*>(base + t * D + 8 * (c ^ kda_swz<D>(t)));
}
// x (bf16) * cv (fp32, or x itself when cv is null), rounded to bf16: an operand fragment
__device__ __forceinline__ bf16x8_t kda_mul(u32x4_t x, const float* cv) {
    if (!cv) return __builtin_bit_cast(bf16x8_t, x);
    const f32x4_t p0 = widen4(u32x2_t{x.x, x.y}) * *reinterpret_cast<const f32x4_t*>(cv);
    const f32x4_t p1 = widen4(u32x2_t{x.z, x.w}) * *reinterpret_cast<const f32x4_t*>(cv + 4);
    const u32x4_t o = {pack2(p0.x, p0.y), pack2(p0.z, p0.w), pack2(p1.x, p1.y), pack2(p1.z, p1.w)};
    return __builtin_bit_cast(bf16x8_t, o);
}
// the products of 8 bf16 values with 8 floats, rounded to bf16
__device__ __forceinline__ u32x4_t kda_mul8(u32x4_t x, const float (&f)[8]) {
    const f32x4_t x0 = widen4(u32x2_t{x.x, x.y}), x1 = widen4(u32x2_t{x.z, x.w});
    const u32x4_t o = {pack2(x0.x * f[0], x0.y * f[1]), pack2(x0.z * f[2], x0.w * f[3]),
                       pack2(x1.x * f[4], x1.y * f[5]), pack2(x1.z * f[6], x1.w * f[7])};
    return o;
}

// Roles, after the factors: wave 0 the diagonal Gram tiles and, after one barrier, T from
// all of them; wave 1 the off-diagonal Gram tiles (handed to wave 0 through LDS); waves 2
// and 3 the ten P tiles; waves 1-3 the recurrence's operand blocks; wave 0 exp(G_C).
template <int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void kda_prep_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                                       const float* __restrict__ beta, const float* __restrict__ gate,
                                                       int T, int H, int n_chunks, long n_items,
                                                       unsigned char* __restrict__ ws) {
    using W = KdaWs<D>;
    using L = KdaPrepLds<D>;
    constexpr int NKB = W::NKB, NCH = D / 8;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    uint16_t* KAs = reinterpret_cast<uint16_t*>(smem + L::KA);
    uint16_t* KRs = reinterpret_cast<uint16_t*>(smem + L::KR);
    uint16_t* QAs = reinterpret_cast<uint16_t*>(smem + L::QA);
    float* Gs = reinterpret_cast<float*>(smem + L::GS);
    float* Cv = reinterpret_cast<float*>(smem + L::CV);
    float* Bs = reinterpret_cast<float*>(smem + L::BS);
    unsigned char* Gu = smem + L::GU;

    const size_t tstride = static_cast<size_t>(H) * D;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = static_cast<int>(uniform(static_cast<unsigned>(tid >> 6)));
    const int l16 = lane & 15, lg = lane >> 4;
    const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
    constexpr int NV = kC * NCH;  // 16-byte chunks per K or Q tile
    constexpr int NKQ = NV / 256, NSEG = 256 / D, SEG = kC / NSEG;
    const int gd_ = tid % D, gsg = tid / D;  // this thread's channel and token segment of G

    // An item's K and Q rows (zeros past the chunk's end) and beta, loaded one whole item
    // ahead into registers, so that they arrive during the previous item's work (the
    // workgroup walks items blockIdx.x, + gridDim.x, ...); its log-gates load at its start.
    u32x4_t pk[NKQ], pq[NKQ];
    float pgv[SEG], pb = 0.f;
    auto prefetch = [&](long it) __attribute__((always_inline)) {
        const int pr = static_cast<int>(it / n_chunks), cc = static_cast<int>(it % n_chunks);
        const long t0 = static_cast<long>(pr / H) * T + static_cast<long>(cc) * kC;
        const int cl = min(kC, T - cc * kC);
        const size_t r0 = static_cast<size_t>(t0) * tstride + static_cast<size_t>(pr % H) * D;
#pragma unroll
        for (int i = 0; i < NKQ; ++i) {
            const int x = tid + 256 * i, t = x / NCH, ch = x % NCH;
            const u32x4_t z = {0u, 0u, 0u, 0u};
            pk[i] = t < cl ? *reinterpret_cast<const u32x4_t*>(k + r0 + t * tstride + 8 * ch) : z;
            pq[i] = t < cl ? *reinterpret_cast<const u32x4_t*>(q + r0 + t * tstride + 8 * ch) : z;
        }
        if (tid < kC) pb = tid < cl ? beta[static_cast<size_t>(t0 + tid) * H + pr % H] : 0.f;
    };
    // An item's log-gates, at the item's start: through a buffer resource whose range ends
    // at the chunk's last valid row (later rows read as zeros), with the token's offset a
    // wave-uniform scalar and the channel the lane's (per-token 64-bit addresses, hoisted
    // out of the item loop, had held 64 VGPRs through the whole kernel)
    auto load_gates = [&](long it) __attribute__((always_inline)) {
        const int pr = static_cast<int>(it / n_chunks), cc = static_cast<int>(it % n_chunks);
        const long t0 = static_cast<long>(pr / H) * T + static_cast<long>(cc) * kC;
        const int cl = min(kC, T - cc * kC);
        const size_t r0 = static_cast<size_t>(t0) * tstride + static_cast<size_t>(pr % H) * D;
        const __amdgpu_buffer_rsrc_t rg =
            make_rsrc(gate + r0, static_cast<unsigned>(((cl - 1) * tstride + D) * 4));
        const int seg0 = static_cast<int>(uniform(static_cast<unsigned>(gsg))) * SEG;
#pragma unroll
        for (int j = 0; j < SEG; ++j)
            pgv[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                rg, static_cast<unsigned>(gd_ * 4), static_cast<unsigned>((seg0 + j) * tstride * 4), 0));
    };

    long item = blockIdx.x;
    if (item >= n_items) return;
    prefetch(item);
    for (; item < n_items; item += gridDim.x) {
    unsigned char* out = ws + static_cast<size_t>(item) * W::BYTES;
    load_gates(item);

    // ---- stage the item: beta and the prefix sums G of the log-gates (K and Q stay in
    // registers until the scaled tiles are formed) ----
    if (tid < kC) Bs[tid] = pb;
    {
        // clamped log-gates in log2 units, running sum over this thread's token segment
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < SEG; ++j) {
            acc += fminf(fmaxf(pgv[j], kKdaGMin), kKdaGMax) * kLog2E;
            Gs[(gsg * SEG + j) * D + gd_] = acc;
        }
    }
    __syncthreads();
    {
        // each segment adds the sums of the segments before it (read before any is changed)
        float off = 0.f;
        for (int s2 = 0; s2 < gsg; ++s2) off += Gs[(s2 * SEG + SEG - 1) * D + gd_];
        __syncthreads();
        if (gsg > 0)
            for (int j = 0; j < SEG; ++j) Gs[(gsg * SEG + j) * D + gd_] += off;
    }
    __syncthreads();

    // ---- the scaled tiles K a, K r, Q a (bf16) over G's storage, and the channel vectors ----
    {
        // the tiles are formed into registers while G is still in LDS, and written over it
        // after the barrier (element chunk i of a thread lies in block i)
        constexpr int NE = NV / 256;  // 8-element chunks per thread
        u32x4_t tka[NE], tkr[NE], tqa[NE];
#pragma unroll
        for (int i = 0; i < NE; ++i) {
            const int x = tid + 256 * i, t = x / NCH, ch = x % NCH, b = t / 16;
            float av[8], rv[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int d = 8 * ch + j;
                const float gv = Gs[t * D + d], gm = Gs[(16 * b + 7) * D + d];
                av[j] = exp2_hw(gv - gm);
                rv[j] = exp2_hw(gm - gv);
            }
            tka[i] = kda_mul8(pk[i], av);
            tkr[i] = kda_mul8(pk[i], rv);
            tqa[i] = kda_mul8(pq[i], av);
        }
        for (int x = tid; x < L::NCV * D; x += 256) {
            const int v = x / D, d = x % D;
            auto G = [&](int t) { return Gs[t * D + d]; };
            // (no table lookups with a runtime index here: such a table is read from global
            // memory, and its wait would also wait for the next item's loads)
            const int pi = v < 1 ? 1 : v < 3 ? 2 : 3, pk = v - (pi == 1 ? 0 : pi == 2 ? 1 : 3);
            float e;
            if (v < kCvE) e = G(16 * pi + 7) - G(16 * pk + 15);                  // cX(k, i)
            else if (v < kCvH) e = G(16 * (v - kCvE) + 15) - G(16 * (v - kCvE) + 7);  // cE(k)
            else if (v < kCvB) e = G(16 * (v - kCvH) + 7);                        // cH(b)
            else if (v < kCvD) e = G(kC - 1) - G(16 * (v - kCvB) + 7);           // cB(b)
            else e = G(kC - 1);                                                   // exp(G_C)
            Cv[x] = exp2_hw(e);
        }
        __syncthreads();  // every read of G is done
#pragma unroll
        for (int i = 0; i < NE; ++i) {
            const int x = tid + 256 * i, t = x / NCH, ch = x % NCH;
            const int pos = t * D + 8 * (ch ^ kda_swz<D>(t));
            *reinterpret_cast<u32x4_t*>(KAs + pos) = tka[i];
            *reinterpret_cast<u32x4_t*>(KRs + pos) = tkr[i];
            *reinterpret_cast<u32x4_t*>(QAs + pos) = tqa[i];
        }
    }
    // the next item's K, Q and beta, in flight through this item's work (the gates load at
    // the item's start: held as well, they would not fit two workgroups per CU)
    if (item + gridDim.x < n_items) prefetch(item + gridDim.x);
    __syncthreads();

    auto cvec = [&](int v, int kb) { return Cv + v * D + 32 * kb + 8 * lg; };
    auto frag = [&](const uint16_t* X, int t, int kb, int v) {
        return kda_mul(kda_row16<D>(X, t, 4 * kb + lg), v < 0 ? nullptr : cvec(v, kb));
    };

    f32x4_t gd[4], gdt[4];
    if (w == 0) {
#pragma unroll
        for (int b = 0; b < 4; ++b) gd[b] = gdt[b] = zero;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int t = 16 * b + l16;
                const bf16x8_t lm = frag(KAs, t, kb, -1);
                const bf16x8_t rm = frag(KRs, t, kb, -1);
                gd[b] = mfma32(lm, rm, gd[b]);
                gdt[b] = mfma32(rm, lm, gdt[b]);
            }
    } else if (w == 1) {
        // block (k, i), k < i, in the order (0,1) (0,2) (1,2) (0,3) (1,3) (2,3)
        constexpr int pk[6] = {0, 0, 1, 0, 1, 2}, pi[6] = {1, 2, 2, 3, 3, 3};
        f32x4_t gu[6];
#pragma unroll
        for (int x = 0; x < 6; ++x) gu[x] = zero;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int kk = 0; kk < 3; ++kk) {
                const bf16x8_t rk = frag(KRs, 16 * kk + l16, kb, kCvE + kk);
#pragma unroll
                for (int x = 0; x < 6; ++x) {
                    if (pk[x] != kk) continue;
                    gu[x] = mfma32(rk, frag(KAs, 16 * pi[x] + l16, kb, kCvX + x), gu[x]);
                }
            }
#pragma unroll
        for (int x = 0; x < 6; ++x) *reinterpret_cast<f32x4_t*>(Gu + x * 1024 + lane * 16) = gu[x];
    } else {
        // P = lower_incl(decayed Q K^T): wave 2 tiles (0,0) (1,0) (1,1) (2,0) (2,1), wave 3
        // (2,2) (3,0) (3,1) (3,2) (3,3)
        uint16_t* pp = reinterpret_cast<uint16_t*>(out + W::PP);
        constexpr int pi[10] = {0, 1, 1, 2, 2, 2, 3, 3, 3, 3}, pj[10] = {0, 0, 1, 0, 1, 2, 0, 1, 2, 3};
#pragma unroll
        for (int x = 0; x < 10; ++x) {
            if ((x < 5) != (w == 2)) continue;
            const int i = pi[x], j = pj[x];
            f32x4_t acc = zero;
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
                const bf16x8_t rj = frag(KRs, 16 * j + l16, kb, i == j ? -1 : kCvE + j);
                const bf16x8_t li = frag(QAs, 16 * i + l16, kb, i == j ? -1 : kCvX + kda_pair(j, i));
                acc = mfma32(rj, li, acc);  // lane: P[16i + l16][16j + 4g + r]
            }
            if (i == j) {
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) acc[rr] = (l16 >= 4 * lg + rr) ? acc[rr] : 0.f;
            }
            store_packed_t(pp, i, j, acc, lane);
            if (i == 0 && j == 0) zero_upper_half(pp, qblk(0, 0), lane);
            if (i == 2 && j == 2) zero_upper_half(pp, qblk(2, 1), lane);
        }
    }
    __syncthreads();  // the off-diagonal Gram tiles are in LDS

    if (w == 0) {
        // ---- T'' = -T diag(beta) ----
        f32x4_t gu[6];
#pragma unroll
        for (int x = 0; x < 6; ++x) gu[x] = *reinterpret_cast<const f32x4_t*>(Gu + x * 1024 + lane * 16);
        float bc[4];
        f32x4_t br4[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            bc[b] = Bs[16 * b + l16];
            br4[b] = *reinterpret_cast<const f32x4_t*>(Bs + 16 * b + 4 * lg);
        }
        f32x4_t tb[10], tn[10];
        t_from_gram(gd, gdt, gu, bc, br4, lane, tb, tn);
        // block (i, j) holds T[16i + l16][16j + 4g + r] in this lane
        constexpr int ib[10] = {0, 1, 1, 2, 2, 2, 3, 3, 3, 3}, jb[10] = {0, 0, 1, 0, 1, 2, 0, 1, 2, 3};
        uint16_t* tt = reinterpret_cast<uint16_t*>(out + W::TT);
#pragma unroll
        for (int x = 0; x < 10; ++x) store_packed_t(tt, ib[x], jb[x], tb[x] * -br4[jb[x]], lane);
        zero_upper_half(tt, qblk(0, 0), lane);
        zero_upper_half(tt, qblk(2, 1), lane);
        // ---- exp(G_C) in the recurrence's accumulator row order: [g][md][r] ----
        float* dec = reinterpret_cast<float*>(out + W::DEC);
        for (int x = lane; x < 256; x += 64) {
            float val = 0.f;
            if (x < D) {
                const int g = x / (D / 4), rem = x % (D / 4);
                val = Cv[kCvD * D + s_row_d(rem / 4, 4 * g + rem % 4)];
            }
            dec[x] = val;
        }
    } else {
        // ---- the recurrence's operands: K^, Q^ (block kb * 4 + m), K-^T (block md * 2 + half) ----
        for (int x = w - 1; x < 3 * W::NOP; x += 3) {
            const int arr = x / W::NOP, blk = x % W::NOP;
            bf16x8_t v;
            if (arr < 2) {
                const int kb = blk / 4, m = blk % 4;
                v = frag(arr == 0 ? KAs : QAs, 16 * m + l16, kb, kCvH + m);
            } else {
                // lane (g, l16): K-[K0 + 4g + i][d] (slots 0-3) and K-[K0 + 16 + 4g + i][d]
                // (slots 4-7), d = s_row_d(md, l16); K- = k r cB(block).  The k r values come
                // from two transposing reads of the K r tile, 16 rows apart (the swizzle
                // repeats every 16 rows): lanes 4 j + cc of group g address row K0 + 4 g + j,
                // d = 32 kb + 8 cc + 4 h + [0, 4) (md = 2 kb + h); then one channel value
                // per lane for each 16-token block.
                const int md = blk / 2, k0 = 32 * (blk % 2);
                const int d = s_row_d(md, l16);
                const int jj = (lane >> 2) & 3, cc = lane & 3, t = k0 + 4 * lg + jj;
                const unsigned ad = lds_addr(KRs + t * D + 8 * ((4 * (md >> 1) + cc) ^ kda_swz<D>(t)) + 4 * (md & 1));
                u32x2_t lo = lds_tr16_issue<0>(ad), hi = lds_tr16_issue<16 * D * 2>(ad);
                const float c0 = Cv[(kCvB + k0 / 16) * D + d], c1 = Cv[(kCvB + k0 / 16 + 1) * D + d];
                __asm__ volatile("s_waitcnt lgkmcnt(0)" : "+v"(lo), "+v"(hi) : : "memory");
                const f32x4_t e0 = widen4(lo) * c0, e1 = widen4(hi) * c1;
                const u32x4_t o = {pack2(e0.x, e0.y), pack2(e0.z, e0.w), pack2(e1.x, e1.y), pack2(e1.z, e1.w)};
                v = __builtin_bit_cast(bf16x8_t, o);
            }
            const int base = arr == 0 ? W::KH : arr == 1 ? W::QH : W::KT;
            *reinterpret_cast<bf16x8_t*>(out + base + blk * 1024 + lane * 16) = v;
        }
    }
    __syncthreads();  // every read of this item's LDS is done before the next item is staged
    }
}

// ---------------------------------------------------------------- K8s
template <int D>
struct KdaRecLds {
    static constexpr int NKB = D / 32;
    static constexpr int WS = KdaWs<D>::BYTES;
    static constexpr int VS = WS;                  // V tile: 64 rows x 32 bf16 (swizzled)
    static constexpr int BUF = VS + kC * 32 * 2;   // one chunk's buffer
    static constexpr int SB = 2 * BUF;             // per chain wave: bf16 S at the chunk's start
    static constexpr int UB = SB + 2 * NKB * 1024; // per chain wave: bf16 U
    static constexpr int BYTES = UB + 2 * 2048;
    static constexpr int NCP_WS = KdaWs<D>::NBLK;  // 1 KiB copies of the workspace image
    static constexpr int NCP = NCP_WS + kC * 32 * 2 / 1024;  // ... plus the V tile's
    static_assert(BYTES <= 160 * 1024, "LDS");
    static_assert((NCP + 3) / 4 + 4 <= 63, "vmcnt range");
};

// Waves 0 and 1 (chain) own columns col0 + 16 w + [0, 16) of S; waves 2 and 3 (output)
// form O for the same columns.  Per chunk c, between barrier A(c) and B(c): the chain
// computes X and U and hands U over; the output wave computes Y^T = S^T Q^T from the S
// handed over at the end of chunk c - 1.  Between B(c) and A(c + 1): the chain updates S
// and hands bf16 S_{c+1} over; the output wave forms O = Y + P U and stores it.  Every
// wave copies a quarter of chunk c + 1's image during chunk c.
template <int D, bool OUT_BF16>
__global__ __launch_bounds__(256) void kda_chunk_kernel(const uint16_t* __restrict__ v, const float* __restrict__ s0,
                                                        void* __restrict__ o_out, float* __restrict__ s_out,
                                                        const unsigned char* __restrict__ ws, int n_pairs, int T,
                                                        int H, int n_tiles, int n_chunks) {
    using W = KdaWs<D>;
    using L = KdaRecLds<D>;
    constexpr int NKB = W::NKB, DV = 32;
    constexpr int NCPW = (L::NCP + 3) / 4;  // copies per wave (the last wave may issue fewer)
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

    // XCD-aware placement: the n_tiles workgroups of a pair share bid % 8
    const int bid = blockIdx.x;
    const int xcd = bid & 7, slot = bid >> 3;
    const int tile = slot % n_tiles;
    const int pair = (slot / n_tiles) * 8 + xcd;
    if (pair >= n_pairs) return;
    const int seq = pair / H, h = pair % H;
    const long tok0 = static_cast<long>(seq) * T;
    const int col0 = tile * DV;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = static_cast<int>(uniform(static_cast<unsigned>(tid >> 6)));
    const int cw = w & 1;  // the column half (chain wave cw, output wave 2 + cw)
    const bool chain = w < 2;
    const int l16 = lane & 15, lg = lane >> 4;
    const size_t sbase = static_cast<size_t>(pair) * D * D;
    const size_t tstride = static_cast<size_t>(H) * D;
    const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
    auto buf = [&](int c) { return smem + (c & 1) * L::BUF; };
    unsigned char* sbslot = smem + L::SB + cw * NKB * 1024;
    unsigned char* uslot = smem + L::UB + cw * 2048;
    auto ld16 = [&](const unsigned char* p) { return *reinterpret_cast<const bf16x8_t*>(p + lane * 16); };
    auto st16 = [&](unsigned char* p, bf16x8_t x) { *reinterpret_cast<bf16x8_t*>(p + lane * 16) = x; };

    // chunk c's copies (workspace image, then the V tile's 4 blocks): wave w issues
    // [w NCPW, (w + 1) NCPW), as inline asm with exact vmcnt waits
    const int i0 = w * NCPW, i1 = min(L::NCP, i0 + NCPW);
    auto issue_copies = [&](int c) __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t rw =
            make_rsrc(ws + (static_cast<size_t>(pair) * n_chunks + c) * W::BYTES, W::BYTES);
        const int clen = min(kC, T - c * kC);
        const size_t vrow0 = static_cast<size_t>(tok0 + static_cast<long>(c) * kC) * tstride +
                             static_cast<size_t>(h) * D + col0;
        const __amdgpu_buffer_rsrc_t rv = make_rsrc(v + vrow0, static_cast<unsigned>(((clen - 1) * tstride + DV) * 2));
        unsigned char* b = uniform_ptr(buf(c));
        for (int i = i0; i < i1; ++i) {
            if (i < L::NCP_WS) {
                dma16_asm(rw, b + 1024 * i, static_cast<unsigned>(1024 * i + 16 * lane));
            } else {
                const int j = i - L::NCP_WS;  // V block: row r, 16-byte chunk p of the row
                const int pos = 512 * j + 8 * lane;
                const int r = pos / DV, p = (pos % DV) / 8;
                dma16_asm(rv, b + L::VS + 1024 * j, static_cast<unsigned>(r * tstride * 2) + 16u * (p ^ v_f<DV>(r)));
            }
        }
    };

    f32x4_t S[D / 16];
    bf16x8_t Sb[NKB];
    const int ecol = col0 + 16 * cw + l16;
    if (chain) {
#pragma unroll
        for (int md = 0; md < D / 16; ++md)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int d = s_row_d(md, 4 * lg + r);
                S[md][r] = s0 ? s0[sbase + static_cast<size_t>(d) * D + ecol] : 0.f;
            }
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
            Sb[kb] = acc_to_b(S[2 * kb], S[2 * kb + 1]);
            st16(sbslot + kb * 1024, Sb[kb]);
        }
    }
    if (n_chunks > 0) {
        issue_copies(0);
        wait_vm_n<0>();
    }
    lds_barrier();  // A(0)
    for (int c = 0; c < n_chunks; ++c) {
        const bool more = c + 1 < n_chunks;
        if (more) issue_copies(c + 1);
        const unsigned char* B = buf(c);
        if (chain) {
            // X = K^ S - V (the accumulators start at -V)
            u32x2_t vv[4];
            const uint16_t* Vs = reinterpret_cast<const uint16_t*>(B + L::VS);
#pragma unroll
            for (int m = 0; m < 4; ++m) vv[m] = lds_v_issue<DV>(Vs, m, cw, lane);
            lds_wait(vv[0], vv[1], vv[2], vv[3]);
            f32x4_t X[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) X[m] = -widen4(vv[m]);
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int m = 0; m < 4; ++m) X[m] = mfma32(ld16(B + W::KH + (kb * 4 + m) * 1024), Sb[kb], X[m]);
            // U = T'' bf16(X) = T diag(beta) (V - K^ S)
            const bf16x8_t Rb0 = acc_to_b(X[0], X[1]), Rb1 = acc_to_b(X[2], X[3]);
            bf16x8_t tt[6];
#pragma unroll
            for (int x = 0; x < 6; ++x) tt[x] = ld16(B + W::TT + x * 1024);
            f32x4_t U[4];
            U[0] = mfma32(tt[0], Rb0, zero);
            U[1] = mfma32(tt[1], Rb0, zero);
            U[2] = mfma32(tt[3], Rb1, mfma32(tt[2], Rb0, zero));
            U[3] = mfma32(tt[5], Rb1, mfma32(tt[4], Rb0, zero));
            const bf16x8_t Ub0 = acc_to_b(U[0], U[1]), Ub1 = acc_to_b(U[2], U[3]);
            st16(uslot, Ub0);
            st16(uslot + 1024, Ub1);
            lds_barrier();  // B(c): U handed over
            // S = Diag(exp(G_C)) S + K-^T U
            const float* dec = reinterpret_cast<const float*>(B + W::DEC) + lg * (D / 4);
#pragma unroll
            for (int md = 0; md < D / 16; ++md) {
                const f32x4_t dv = *reinterpret_cast<const f32x4_t*>(dec + 4 * md);
                S[md] = S[md] * dv;
                S[md] = mfma32(ld16(B + W::KT + (2 * md) * 1024), Ub0, S[md]);
                S[md] = mfma32(ld16(B + W::KT + (2 * md + 1) * 1024), Ub1, S[md]);
            }
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
                Sb[kb] = acc_to_b(S[2 * kb], S[2 * kb + 1]);
                st16(sbslot + kb * 1024, Sb[kb]);
            }
            if (more) wait_vm_n<0>();  // this wave's copies of chunk c + 1
        } else {
            // Y^T = S^T Q^T: lane (g, l16) holds Y[16m + l16][16 cw + 4g .. +4)
            bf16x8_t sb[NKB];
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) sb[kb] = ld16(sbslot + kb * 1024);
            f32x4_t Y[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) Y[m] = zero;
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int m = 0; m < 4; ++m) Y[m] = mfma32(sb[kb], ld16(B + W::QH + (kb * 4 + m) * 1024), Y[m]);
            bf16x8_t pp[6];
#pragma unroll
            for (int x = 0; x < 6; ++x) pp[x] = ld16(B + W::PP + x * 1024);
            lds_barrier();  // B(c)
            const bf16x8_t Ub0 = ld16(uslot), Ub1 = ld16(uslot + 1024);
            f32x4_t O[4];
            O[0] = mfma32(Ub0, pp[0], Y[0]);
            O[1] = mfma32(Ub0, pp[1], Y[1]);
            O[2] = mfma32(Ub1, pp[3], mfma32(Ub0, pp[2], Y[2]));
            O[3] = mfma32(Ub1, pp[5], mfma32(Ub0, pp[4], Y[3]));
            // O rows by range-checked buffer stores (rows past the sequence's end are dropped)
            const int clen = min(kC, T - c * kC);
            constexpr int ES = OUT_BF16 ? 2 : 4;
            const size_t rowe = static_cast<size_t>(tok0 + static_cast<long>(c) * kC) * tstride +
                                static_cast<size_t>(h) * D + col0;
            const __amdgpu_buffer_rsrc_t ro = make_rsrc(static_cast<unsigned char*>(o_out) + rowe * ES,
                                                        static_cast<unsigned>(((clen - 1) * tstride + DV) * ES));
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const unsigned off = static_cast<unsigned>(((16 * m + l16) * tstride + 16 * cw + 4 * lg) * ES);
                if constexpr (OUT_BF16) {
                    const u32x2_t ob = {pack_rne(O[m].x, O[m].y), pack_rne(O[m].z, O[m].w)};
                    __builtin_amdgcn_raw_buffer_store_b64(ob, ro, off, 0, 0);
                } else {
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, O[m]), ro, off, 0, 0);
                }
            }
            // this wave's copies of chunk c + 1 have landed (its 4 O stores, issued after
            // them, may not have)
            if (more) wait_vm_n<4>();
        }
        lds_barrier();  // A(c + 1)
    }
    if (chain) {
#pragma unroll
        for (int md = 0; md < D / 16; ++md)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int d = s_row_d(md, 4 * lg + r);
                s_out[sbase + static_cast<size_t>(d) * D + ecol] = S[md][r];
            }
    }
}

template <auto KERN>
hipError_t kda_set_lds_once(int bytes) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    static bool done[64] = {};
    if (dev >= 0 && dev < 64 && done[dev]) return hipSuccess;
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(KERN), hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess && dev >= 0 && dev < 64) done[dev] = true;
    return e;
}

template <int D, bool OB>
hipError_t launch_kda_t(const KdaChunkedArgs& a, hipStream_t st) {
    const int n_pairs = a.B * a.H;
    const int n_chunks = (a.T + kC - 1) / kC;
    const long n_items = static_cast<long>(n_pairs) * n_chunks;
    if (n_items == 0) return hipSuccess;
    unsigned char* ws = static_cast<unsigned char*>(a.workspace);
    constexpr int PREP = KdaPrepLds<D>::TOT;
    hipError_t e;
    if ((e = kda_set_lds_once<kda_prep_kernel<D>>(PREP)) != hipSuccess) return e;
    // persistent: two workgroups per CU (the LDS limit), each walking items
    int dev = 0, n_cu = 0;
    if ((e = hipGetDevice(&dev)) != hipSuccess) return e;
    if ((e = hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
    const long grid = std::min<long>(n_items, 2L * std::max(n_cu, 1));
    hipLaunchKernelGGL(kda_prep_kernel<D>, dim3(static_cast<unsigned>(grid)), dim3(256), PREP, st, a.q, a.k,
                       a.beta, a.g, a.T, a.H, n_chunks, n_items, ws);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    using L = KdaRecLds<D>;
    if ((e = kda_set_lds_once<kda_chunk_kernel<D, OB>>(L::BYTES)) != hipSuccess) return e;
    const int n_tiles = D / 32;
    const int slots = (n_pairs + 7) / 8;
    hipLaunchKernelGGL((kda_chunk_kernel<D, OB>), dim3(static_cast<unsigned>(slots * 8 * n_tiles)), dim3(256),
                       L::BYTES, st, a.v, a.s0, a.o, a.s_out, ws, n_pairs, a.T, a.H, n_tiles, n_chunks);
    return hipGetLastError();
}

}  // namespace

size_t kda_chunked_ws_bytes(int B, int T, int H, int D) {
    const size_t n = static_cast<size_t>(B) * H * ((T + kC - 1) / kC);
    return n * (D == 128 ? KdaWs<128>::BYTES : KdaWs<64>::BYTES);
}

hipError_t launch_kda_chunked(const KdaChunkedArgs& a, hipStream_t st) {
    if (a.D == 128) return a.out_bf16 ? launch_kda_t<128, true>(a, st) : launch_kda_t<128, false>(a, st);
    return a.out_bf16 ? launch_kda_t<64, true>(a, st) : launch_kda_t<64, false>(a, st);
}

}  // namespace pm
