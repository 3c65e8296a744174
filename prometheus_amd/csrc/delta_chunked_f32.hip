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
// K7p (prep, one wave per (sequence, head, chunk), all chunks at once): G = K K^T from K
// rows read straight into operand registers, N = -A and N^T from G (which is symmetric),
// and T^T = ((I+N)(I+N^2)(I+N^4)(I+N^8))^T (N is strictly lower triangular, so N^16 = 0)
// as products of accumulators with transposed accumulators.  It writes (T'')^T as
// accumulator registers, 1 KiB per chunk: the A operand of U = T'' X, lane-linear.
//
// K7 (recurrence): one workgroup per (sequence, head, d_v tile of DV columns) with DV/16
// chain waves and as many output waves.  Chain wave w owns the S columns col0 + 16 w +
// [0, 16) as D/16 accumulator tiles and runs chunk i (X, U, S: 68 MFMAs at D = 128),
// handing S_i (before its update) and U_i to output wave w through LDS; output wave w
// runs chunk i - 1 (Y = Q S, P^T = K Q^T, O = Y + P U: 68 MFMAs at D = 128, as many as
// the chain's) and stores O.  Products of one accumulator are spread over several
// accumulators (a dependent MFMA waits for its predecessor's result), summed at the end.
// HBM -> LDS copies (buffer_load ... lds) run two chunks ahead: the output waves copy K
// and Q rows, the chain waves their V columns and (wave 0) T''^T.  One LDS-only barrier
// per chunk.

#include <type_traits>

#include "pm_cdna4.h"
#include "pm_f32mfma.h"
#include "pm_internal.h"

namespace pm {
namespace {

constexpr int kBwdRec = kF32BwdRec;  // floats per chunk of the backward's record: T, K K^T, beta, P
// workspace floats per chunk: (T'')^T, then (normalised mode) the 16 keys' 1 / max(||k||, 1e-6)
template <bool NORM>
constexpr int ws_floats() { return NORM ? 256 + 16 : 256; }


// Workspace slots (16-token chunks), as the split form's: fixed length, row = pair, slot
// = c; varlen, row = h and slot = floor(tok0 / 16) + seq + c (consecutive sequences never
// share a slot).
__host__ __device__ inline int f32_n_slot(bool varlen, int T, int n_seq) {
    return varlen ? (T + kC16 - 1) / kC16 + n_seq : (T + kC16 - 1) / kC16;
}


// ---------------------------------------------------------------- K7p
template <int D, bool NORM, bool BWD = false>
__global__ __launch_bounds__(256) void delta_f32_prep_kernel(const float* __restrict__ k,
                                                             const float* __restrict__ beta,
                                                             const int32_t* __restrict__ cu_seqlens,
                                                             int n_seq, int T, int H, int n_slot, long n_items,
                                                             float* __restrict__ ws, float* __restrict__ ws_b = nullptr,
                                                             const float* __restrict__ q = nullptr) {
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
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(k + row0, nb);
    f32x4_t kf[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const unsigned vo = static_cast<unsigned>((r * tstride + 16 * j + 4 * g) * 4);
        kf[j] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rk, vo, 0, 0));
    }
    // beta of this lane's column token r (bc) and of its accumulator rows 4 g + v (bt); in the
    // normalised mode beta = 1 and sk / s4 are the keys' 1 / max(||k||, 1e-6) instead
    float bc = 1.f, sk = 1.f;
    f32x4_t bt = {1.f, 1.f, 1.f, 1.f}, s4 = {1.f, 1.f, 1.f, 1.f};
    if constexpr (NORM) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int v = 0; v < 4; ++v) ss = fmaf(kf[j][v], kf[j][v], ss);
        ss += __shfl_xor(ss, 16);  // row r's four slices (every lane of the row gets equal bits)
        ss += __shfl_xor(ss, 32);
        sk = 1.f / fmaxf(sqrtf(ss), 1e-6f);
#pragma unroll
        for (int v = 0; v < 4; ++v) s4[v] = __shfl(sk, 4 * g + v);
    } else {
        const __amdgpu_buffer_rsrc_t rb =
            make_rsrc(beta + (tok0 + base) * H + h, static_cast<unsigned>(((clen - 1) * H + 1) * 4));
        bc = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rb, static_cast<unsigned>(r * H * 4), 0, 0));
#pragma unroll
        for (int v = 0; v < 4; ++v)
            bt[v] = __uint_as_float(
                __builtin_amdgcn_raw_buffer_load_b32(rb, static_cast<unsigned>((4 * g + v) * H * 4), 0, 0));
    }

    // G = K K^T (one accumulator per step of a tile, summed at the end)
    const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
    f32x4_t ga[4] = {zero, zero, zero, zero};
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) ga[v] = mfma4(kf[j][v], kf[j][v], ga[v]);
    f32x4_t G = (ga[0] + ga[1]) + (ga[2] + ga[3]);
    if constexpr (NORM) G = G * s4 * sk;  // Gram matrix of the normalised keys
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
    f32x4_t tw;
#pragma unroll
    for (int v = 0; v < 4; ++v) tw[v] = -bt[v] * Tt[v];  // (T'')^T[i][j] = -beta_i T[j][i]
    float* out = ws + (static_cast<size_t>(row) * n_slot + slot) * ws_floats<NORM>();
    *reinterpret_cast<f32x4_t*>(out + lane * 4) = tw;
    if constexpr (BWD) {
        // the backward's record: T (accumulator registers: T[4 g + v][r]), the Gram matrix
        // K K^T (symmetric, so its registers are also those of its transpose), beta and P
        const f32x4_t Tacc = mm16(F2t, eye + N8);  // (I+N)(I+N^2)(I+N^4) (I+N^8)
        float* ob = ws_b + (static_cast<size_t>(row) * n_slot + slot) * kBwdRec;
        *reinterpret_cast<f32x4_t*>(ob + lane * 4) = Tacc;
        *reinterpret_cast<f32x4_t*>(ob + 256 + lane * 4) = G;
        if (g == 0) ob[512 + r] = bc;
        // P = lower_incl(Q K^T): P[4 g + v][r] = q_{4 g + v} . k_r, kept for r <= 4 g + v
        const __amdgpu_buffer_rsrc_t rq = make_rsrc(q + row0, nb);
        f32x4_t pa[4] = {zero, zero, zero, zero};
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const unsigned vo = static_cast<unsigned>((r * tstride + 16 * j + 4 * g) * 4);
            const f32x4_t qf = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rq, vo, 0, 0));
#pragma unroll
            for (int v = 0; v < 4; ++v) pa[v] = mfma4(qf[v], kf[j][v], pa[v]);
        }
        f32x4_t P = (pa[0] + pa[1]) + (pa[2] + pa[3]);
#pragma unroll
        for (int v = 0; v < 4; ++v) P[v] = (r <= 4 * g + v) ? P[v] : 0.f;
        *reinterpret_cast<f32x4_t*>(ob + 528 + lane * 4) = P;
    }
    if constexpr (NORM) {
        if (g == 0) out[256 + r] = sk;
    }
}

// ---------------------------------------------------------------- K7
// HIST (the history mode) keeps no Q and no hand-off slots, and three chunk buffers
// (the chain's, the one in flight, the one being copied): 33 KiB at D = 128, DV = 32, so
// that a workgroup of the backward's sweep fits beside it on a CU.
template <int D, int DV, bool NORM, bool HIST = false>
struct F32Geo {
    static constexpr int NCW = DV / 16;            // chain waves 0 .. NCW-1, output waves NCW ..
    static constexpr int NT = D / 16;              // S accumulator tiles per chain wave
    static constexpr int NI = kC16 * D * 4 / 1024; // 1 KiB copies per K or Q tile
    static constexpr int NB = HIST ? 3 : 4;        // rotating chunk buffers
    // one chunk buffer: K rows, Q rows, (T'')^T, V columns of each chain wave
    static constexpr int B_K = 0;
    static constexpr int B_Q = B_K + kC16 * D * 4;
    static constexpr int B_T = B_Q + (HIST ? 0 : kC16 * D * 4);
    static constexpr int B_V = B_T + (NORM ? 2048 : 1024);  // (T'')^T, then the keys' scales
    static constexpr int BUF = B_V + NCW * 1024;
    static constexpr int OFF_S = NB * BUF;                                  // 2 slots x NCW x NT KiB: S_i
    static constexpr int OFF_U = OFF_S + (HIST ? 0 : 2 * NCW * NT * 1024);  // 2 slots x NCW KiB: U_i
    static constexpr int PSLOT = NORM ? 1024 + 64 : 1024;                   // P^T, then the queries' scales
    static constexpr int OFF_P = OFF_U + (HIST ? 0 : 2 * NCW * 1024);       // 2 slots: P^T of a chunk
    static constexpr int BYTES = OFF_P + (HIST ? 0 : 2 * PSLOT);
    // the last output wave (the copy wave) issues every copy of a chunk: K and Q rows,
    // (T'')^T and the V columns of each chain wave
    static constexpr int NCP = (HIST ? NI : 2 * NI) + 1 + NCW + (NORM ? 1 : 0);
    static constexpr int NST = 4;  // O stores per output wave per chunk
    static_assert(D == 64 || D == 128, "D");
    static_assert(DV == 16 || DV == 32, "DV");
    static_assert(BYTES <= 160 * 1024 && NCP + NST <= 63, "LDS / vmcnt");
};

// HIST (the backward's history pass, fixed-length batches): no O and no final state; the
// chain waves store the state at the start of every kF32Span-th chunk and at the end
// instead (n_span = the number of spans + 1 states per pair), as accumulator registers:
// hist[pair][index][column block 16 jb][tile m][lane][4] holds S[16 m + 4 g + v][16 jb + r]
// at lane 16 g + r, register v; and every chunk's U as rows (u_out, laid out like v).  The
// copy wave then copies no Q.
// Work a caller adds to the history mode's non-chain waves, once per chunk i (before
// the chunk's barrier): none by default.
struct NoExtra {
    __device__ void operator()(int, int) const {}
};

template <int D, int DV, bool OUT_BF16, bool NORM, bool HIST, typename Extra = NoExtra>
__device__ __forceinline__ void f32_fwd_body(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ s0, void* __restrict__ o_out, float* __restrict__ s_out,
    const int32_t* __restrict__ cu_seqlens, const float* __restrict__ ws, int n_pairs, int T, int H,
    int n_tiles, int n_slot, float* __restrict__ hist, int n_span, unsigned char* __restrict__ smem, int w,
    float* __restrict__ u_out = nullptr, Extra extra = Extra{}) {
    using G = F32Geo<D, DV, NORM, HIST>;
    constexpr int NCW = G::NCW, NT = G::NT;
    constexpr int NCP = G::NCP;                          // copies per chunk
    constexpr int NST = HIST ? 0 : G::NST;               // O stores per output wave per chunk
    constexpr int WSF = ws_floats<NORM>();

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
    const int r = lane & 15, g = lane >> 4;
    const bool chain = w < NCW;
    const int cw = chain ? w : w - NCW;  // the 16 columns this wave works on
    const bool p_wave = w == NCW;         // builds P^T for every output wave
    const bool copy_wave = w == 2 * NCW - 1;
    const size_t tstride = static_cast<size_t>(H) * D;
    const size_t sbase = static_cast<size_t>(pair) * D * D;
    const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
    auto fence = []() __attribute__((always_inline)) { __builtin_amdgcn_sched_barrier(0); };

    auto buf = [&](int c) { return smem + (c % G::NB) * G::BUF; };
    auto sslot = [&](int c, int which) { return smem + G::OFF_S + ((c & 1) * NCW + which) * NT * 1024; };
    auto uslot = [&](int c, int which) { return smem + G::OFF_U + ((c & 1) * NCW + which) * 1024; };
    auto pslot = [&](int c) { return smem + G::OFF_P + (c & 1) * G::PSLOT; };
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
    auto copy_ws = [&](int c, unsigned char* dst) __attribute__((always_inline)) {
        const float* src = ws + (static_cast<size_t>(ws_row) * n_slot + ws_slot0 + c) * WSF;
        dma16_asm(make_rsrc(src, 1024), uniform_ptr(dst), static_cast<unsigned>(16 * lane));
        // the keys' scales: 64 bytes (lanes past them read zeros)
        if constexpr (NORM) dma16_asm(make_rsrc(src + 256, 64), uniform_ptr(dst + 1024), static_cast<unsigned>(16 * lane));
    };
    auto copy_v = [&](int c, int j, unsigned char* dst) __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t rs = chunk_rsrc(v, c, 16, col0 + 16 * j);
        const int t = lane >> 2, p = lane & 3;
        dma16_asm(rs, uniform_ptr(dst), static_cast<unsigned>(t * tstride * 4 + 16 * p));
    };
    // the copy wave's copies of chunk c
    auto copies = [&](int c) __attribute__((always_inline)) {
        unsigned char* b = buf(c);
        copy_tile(k, c, b + G::B_K);
        if constexpr (!HIST) copy_tile(q, c, b + G::B_Q);
        copy_ws(c, b + G::B_T);
#pragma unroll
        for (int j = 0; j < NCW; ++j) copy_v(c, j, b + G::B_V + 1024 * j);
    };
    // the copy wave: wait until the next chunk's copies have landed, with the operations
    // issued after them (this and the last iteration's O stores, the copies of the chunk
    // after next) possibly in flight
    auto wait_next = [&](bool extra_stores, bool extra_copies) __attribute__((always_inline)) {
        if (extra_copies && extra_stores) wait_vm_n<NCP + NST>();
        else if (extra_copies) wait_vm_n<NCP>();
        else if (extra_stores) wait_vm_n<NST>();
        else wait_vm_n<0>();
    };

    if (n_chunks > 0) {
        if (copy_wave) {
            copies(0);
            if (n_chunks > 1) copies(1);
            wait_next(false, n_chunks > 1);
        }
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
        // s_waitcnt vmcnt(0) as the intrinsic, which the compiler's wait insertion sees: with
        // the S0 loads settled here it puts no wait for them inside the loop, where a
        // vmcnt(0) would also wait for the copies of two chunks ahead
        __builtin_amdgcn_s_waitcnt(0x0F70);
        // Iteration i (after barrier B_i) finishes chunk i - 1 (S += K^T U, its K^T operands
        // read before the barrier) and runs chunk i up to U, so the state update of one chunk
        // and X of the next run back to back on the MFMA pipe; the LDS reads of each phase
        // are issued ahead of it, in groups fenced by sched_barrier (left to itself the
        // compiler reads each operand right before its MFMA and waits out the LDS latency).
        float kt[4][NT];  // K^T operand of chunk i - 1: K[4 g + e][16 m + r]
        f32x4_t Up = zero;
        for (int i = 0; i <= n_chunks; ++i) {
            const bool run = i < n_chunks;
            const unsigned char* b = buf(run ? i : 0);
            const float* Vf = reinterpret_cast<const float*>(b + G::B_V + 1024 * cw);
            f32x4_t kf[NT], xa[4] = {zero, zero, zero, zero}, tt = zero, vr = zero;
            if (run) {
#pragma unroll
                for (int m = 0; m < NT; ++m) kf[m] = ld4(b + G::B_K + 16 * f32_chunk<D>(r, 4 * m + g));
#pragma unroll
                for (int e = 0; e < 4; ++e) vr[e] = Vf[(4 * g + e) * 16 + r];
                tt = ld4(b + G::B_T + 16 * lane);
            }
            fence();
            // S += K^T U of chunk i - 1 (consecutive MFMAs go to different tiles)
            if (i > 0) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
#pragma unroll
                    for (int m = 0; m < NT; ++m) S[m] = mfma4(kt[e][m], Up[e], S[m]);
            }
            if (!run) break;
            if constexpr (HIST) {
                if (i % kF32Span == 0) {
                    float* hp = hist + ((static_cast<size_t>(pair) * n_span + i / kF32Span) * (D / 16) +
                                        col0 / 16 + cw) * NT * 256;
#pragma unroll
                    for (int m = 0; m < NT; ++m) *reinterpret_cast<f32x4_t*>(hp + m * 256 + 4 * lane) = S[m];
                }
            }
            fence();
            if constexpr (!NORM) xa[0] = -vr;  // (negated only here: a use right after the read would wait for it)
            // X = K S - V (accumulator e takes the steps (m, e))
#pragma unroll
            for (int m = 0; m < NT; ++m)
#pragma unroll
                for (int e = 0; e < 4; ++e) xa[e] = mfma4(kf[m][e], S[m][e], xa[e]);
            f32x4_t X = (xa[0] + xa[1]) + (xa[2] + xa[3]);
            // normalised mode: X = diag(s) K S - V with s the keys' scales (rows 4 g + e)
            f32x4_t skc = {1.f, 1.f, 1.f, 1.f};
            if constexpr (NORM) {
                skc = ld4(b + G::B_T + 1024 + 16 * g);
                X = X * skc - vr;
            }
            // U = T'' X (normalised mode: the state update and P U take diag(s) U)
            Up = mm16(tt, X);
            if constexpr (NORM) Up = Up * skc;
            if constexpr (HIST) {
                // U's rows for the backward, from U^T = X^T T''^T: lane (g, r) holds
                // U[r][col0 + 16 cw + 4 g ..] (rows past the end dropped by the range)
                const f32x4_t Ut = mm16(X, tt);
                const int clen = min(kC16, len - i * kC16);
                const size_t rowu = static_cast<size_t>(tok0 + i * kC16) * tstride + static_cast<size_t>(h) * D +
                                    col0 + 16 * cw;
                __builtin_amdgcn_raw_buffer_store_b128(
                    __builtin_bit_cast(u32x4_t, Ut),
                    make_rsrc(u_out + rowu, static_cast<unsigned>(((clen - 1) * tstride + 16) * 4)),
                    static_cast<unsigned>((r * tstride + 4 * g) * 4), 0, 0);
            }
            // hand S_i and U_i to the output wave
            if constexpr (!HIST) {
                unsigned char* ss = sslot(i, cw);
#pragma unroll
                for (int m = 0; m < NT; ++m) st4(ss + 1024 * m + 16 * lane, S[m]);
                st4(uslot(i, cw) + 16 * lane, Up);
            }
            // K^T operand of chunk i, for the next iteration's state update
            const float* Kf = reinterpret_cast<const float*>(b + G::B_K);
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int m = 0; m < NT; ++m) {
                    const int t = 4 * g + e, d = 16 * m + r;
                    kt[e][m] = Kf[4 * f32_chunk<D>(t, d >> 2) + (d & 3)];
                }
            // lgkmcnt(0) as the intrinsic, so that the compiler knows kt has landed and puts
            // no wait for it after the barrier (where it would also wait for the new reads)
            __builtin_amdgcn_s_waitcnt(0xC07F);
            lds_barrier();
        }
        if constexpr (!HIST) {
#pragma unroll
            for (int m = 0; m < NT; ++m)
#pragma unroll
                for (int e = 0; e < 4; ++e) s_out[sbase + static_cast<size_t>(16 * m + 4 * g + e) * D + ecol] = S[m][e];
        } else {
            // the state at the end of the sequence closes the last span
            float* hp = hist + ((static_cast<size_t>(pair) * n_span + n_span - 1) * (D / 16) + col0 / 16 + cw) * NT * 256;
#pragma unroll
            for (int m = 0; m < NT; ++m) *reinterpret_cast<f32x4_t*>(hp + m * 256 + 4 * lane) = S[m];
        }
    } else if (HIST && n_chunks > 0) {
        // the copy wave keeps two chunks ahead; the other output waves only keep the barriers
        for (int i = 0; i < n_chunks; ++i) {
            if (copy_wave && i + 2 < n_chunks) copies(i + 2);
            extra(i, w);
            if (copy_wave && i + 1 < n_chunks) wait_next(false, i + 2 < n_chunks);
            lds_barrier();
        }
    } else if (n_chunks > 0) {
        // ============ output waves: O of chunk i - 1 for the columns of chain wave cw ============
        // Iteration i: the P wave builds P^T of chunk i (for the next iteration, into LDS);
        // every output wave forms Y = Q S and O = Y + P U of chunk i - 1 and stores O; the
        // copy wave issues chunk i + 2's copies.
        constexpr int ES = OUT_BF16 ? 2 : 4;
        for (int i = 0; i <= n_chunks; ++i) {
            const bool cp = copy_wave && i + 2 < n_chunks;
            if (cp) copies(i + 2);
            const bool st = i >= 1;
            const bool pp = p_wave && i < n_chunks;
            // accumulator e takes the steps (m, e); each tile's operand reads are issued two
            // tiles ahead.  One straight-line body per combination of the two products.
            f32x4_t ya[4] = {zero, zero, zero, zero}, pa[4] = {zero, zero, zero, zero};
            float qss = 0.f;  // normalised mode: this lane's part of ||q_r||^2 of chunk i
            const unsigned char* by = buf(st ? i - 1 : 0);
            const unsigned char* bp = buf(i);
            const unsigned char* ss = sslot(st ? i - 1 : 0, cw);
            auto products = [&](auto ST, auto PP) __attribute__((always_inline)) {
                constexpr bool DO_Y = decltype(ST)::value, DO_P = decltype(PP)::value;
                f32x4_t qy[NT], sc[NT], qp[NT], kp[NT];
                auto rd = [&](int m) __attribute__((always_inline)) {
                    if constexpr (DO_Y) {
                        qy[m] = ld4(by + G::B_Q + 16 * f32_chunk<D>(r, 4 * m + g));
                        sc[m] = ld4(ss + 1024 * m + 16 * lane);
                    }
                    if constexpr (DO_P) {
                        qp[m] = ld4(bp + G::B_Q + 16 * f32_chunk<D>(r, 4 * m + g));
                        kp[m] = ld4(bp + G::B_K + 16 * f32_chunk<D>(r, 4 * m + g));
                    }
                };
                rd(0);
                rd(1);
                fence();
#pragma unroll
                for (int m = 0; m < NT; ++m) {
                    if (m + 2 < NT) rd(m + 2);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if constexpr (DO_Y) ya[e] = mfma4(qy[m][e], sc[m][e], ya[e]);
                        if constexpr (DO_P) pa[e] = mfma4(kp[m][e], qp[m][e], pa[e]);
                        if constexpr (DO_P && NORM) qss = fmaf(qp[m][e], qp[m][e], qss);
                    }
                    fence();
                }
            };
            using T_ = std::true_type;
            using F_ = std::false_type;
            if (st && pp) products(T_{}, T_{});
            else if (st) products(T_{}, F_{});
            else if (pp) products(F_{}, T_{});
            if (pp) {
                // P^T[i][j] = P[j][i] = q_j . k_i, kept for i <= j (lower_incl P)
                const f32x4_t pq = (pa[0] + pa[1]) + (pa[2] + pa[3]);
                f32x4_t pt;
#pragma unroll
                for (int e = 0; e < 4; ++e) pt[e] = (4 * g + e <= r) ? pq[e] : 0.f;
                st4(pslot(i) + 16 * lane, pt);
                if constexpr (NORM) {
                    // the queries' scales 1 / max(||q||, 1e-6) of chunk i, from the Q operands
                    // just used (a row's four slices are lanes r, r + 16, r + 32, r + 48)
                    float ss = qss;
                    ss += __shfl_xor(ss, 16);
                    ss += __shfl_xor(ss, 32);
                    if (g == 0) reinterpret_cast<float*>(pslot(i) + 1024)[r] = 1.f / fmaxf(sqrtf(ss), 1e-6f);
                }
            }
            if (st) {
                const int c = i - 1;
                const f32x4_t pt = ld4(pslot(c) + 16 * lane);
                const f32x4_t u = ld4(uslot(c, cw) + 16 * lane);
                f32x4_t O = mm16(pt, u, (ya[0] + ya[1]) + (ya[2] + ya[3]));
                if constexpr (NORM) O = O * ld4(pslot(c) + 1024 + 16 * g);  // rows scaled by the queries' scales
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
                if (copy_wave && i + 1 < n_chunks) wait_next(st, cp);
                lds_barrier();
            }
        }
    }
}

template <int D, int DV, bool OUT_BF16, bool NORM, bool HIST = false>
__global__ __launch_bounds__(DV == 32 ? 256 : 128) void delta_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ s0, void* __restrict__ o_out, float* __restrict__ s_out,
    const int32_t* __restrict__ cu_seqlens, const float* __restrict__ ws, int n_pairs, int T, int H,
    int n_tiles, int n_slot, float* __restrict__ hist = nullptr, int n_span = 0) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    f32_fwd_body<D, DV, OUT_BF16, NORM, HIST>(q, k, v, s0, o_out, s_out, cu_seqlens, ws, n_pairs, T, H, n_tiles,
                                              n_slot, hist, n_span, smem,
                                              static_cast<int>(uniform(static_cast<unsigned>(threadIdx.x >> 6))));
}

// ---------------------------------------------------------------- K9b: the backward's gradient sweep
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
// Q^T dO of chunk ch for chain wave c's 16 columns, tiles m0 .. m1 - 1 (rows 16 m .. of d),
// from the chunk's buffer into its slot (sw: the sweep's LDS).
template <int D>
__device__ __forceinline__ void sweep_qtdo(unsigned char* sw, int ch, int c, int m0, int m1) {
    using G = SwGeo<D>;
    const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
    const unsigned char* b = sw + (ch % G::NB) * G::BUF;
    const float* Of = reinterpret_cast<const float*>(b + G::B_O + 1024 * c);
    const float* Qf = reinterpret_cast<const float*>(b + G::B_Q);
    f32x4_t dOc;
#pragma unroll
    for (int e = 0; e < 4; ++e) dOc[e] = Of[(4 * g + e) * 16 + r];
    unsigned char* slot = sw + G::OFF_H + ((ch & 1) * 2 + c) * G::NT * 1024;
#pragma unroll
    for (int m = 0; m < G::NT; ++m) {
        if (m < m0 || m >= m1) continue;
        float qt[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int t = 4 * g + e, d = 16 * m + r;
            qt[e] = Qf[4 * f32_chunk<D>(t, d >> 2) + (d & 3)];
        }
        f32x4_t hq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 4; ++e) hq = mfma4(qt[e], dOc[e], hq);
        *reinterpret_cast<f32x4_t*>(slot + 1024 * m + 16 * lane) = hq;
    }
}

// SPLIT: the helper forms the first half of its chain's Q^T dO tiles (the caller's other
// waves form the second half in the same iteration).
template <int D, bool SPLIT = false>
__device__ __forceinline__ void f32_sweep_body(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ go,
    const float* __restrict__ gs, float* __restrict__ gv, float* __restrict__ gs0, const float* __restrict__ rec,
    float* __restrict__ w_out, float* __restrict__ g_hist, int n_pairs, int T, int H, int n_tiles, int n_ch,
    int n_span, unsigned char* __restrict__ smem, int w) {
    using G = SwGeo<D>;
    constexpr int NT = G::NT;
    auto ld4 = [](const unsigned char* p) { return *reinterpret_cast<const f32x4_t*>(p); };
    auto st4 = [](unsigned char* p, f32x4_t x) { *reinterpret_cast<f32x4_t*>(p) = x; };

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
            // Q^T dO for chain wave hw's columns: tile m = rows 16 m .. of d
            if (ch >= 0) sweep_qtdo<D>(smem, ch, hw, 0, SPLIT ? NT / 2 : NT);
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


// K9a + K9b in one workgroup of eight waves per (b, h, 32 columns of d_v): waves 0-3 run
// the forward in its history mode, waves 4-7 the gradient sweep, two independent
// recurrences over the same chunks in opposite directions.  Waves w and w + 4 share a
// SIMD, so the four chain waves (0, 1, 6, 7) take the four SIMDs.  The two halves share
// the workgroup's barriers: the sweep passes one more (n + 2 against n + 1), which the
// history half adds at its end.  LDS: the history half's 33 KiB, then the sweep's.
template <int D>
__global__ __launch_bounds__(512) void f32_hist_sweep_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ s0, const float* __restrict__ go, const float* __restrict__ gs, float* __restrict__ gv,
    float* __restrict__ gs0, const float* __restrict__ t2, const float* __restrict__ rec, float* __restrict__ w_out,
    float* __restrict__ s_hist, float* __restrict__ g_hist, float* __restrict__ u_out, int n_pairs, int T, int H,
    int n_ch, int n_span) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    using GH = F32Geo<D, 32, false, true>;
    constexpr int OFF2 = (GH::BYTES + 255) & ~255;
    constexpr int n_tiles = D / 32;
    const int w8 = static_cast<int>(uniform(static_cast<unsigned>(threadIdx.x >> 6)));
    if (w8 < 4) {
        // the history half's two non-chain waves (2, 3: SIMDs 2, 3, beside the sweep's chains
        // on waves 6, 7) form the second half of each sweep chain's Q^T dO, the sweep's
        // helpers (4, 5: SIMDs 0, 1, beside the history's chains) the first
        unsigned char* sw = smem + OFF2;
        auto extra = [=](int i, int wl) {
            const int ch = n_ch - 1 - i;
            if (wl >= 2 && ch >= 0) sweep_qtdo<D>(sw, ch, wl - 2, SwGeo<D>::NT / 2, SwGeo<D>::NT);
        };
        f32_fwd_body<D, 32, false, false, true>(nullptr, k, v, s0, nullptr, nullptr, nullptr, t2, n_pairs, T, H,
                                                n_tiles, n_ch, s_hist, n_span + 1, smem, w8, u_out, extra);
        const int bslot = static_cast<int>(blockIdx.x) >> 3;
        const int pair = (bslot / n_tiles) * 8 + (static_cast<int>(blockIdx.x) & 7);
        if (pair < n_pairs && n_ch > 0) lds_barrier();
    } else {
        f32_sweep_body<D, true>(q, k, go, gs, gv, gs0, rec, w_out, g_hist, n_pairs, T, H, n_tiles, n_ch, n_span,
                                smem + OFF2, w8 - 4);
    }
}


// The dynamic-LDS limit is a per-device function attribute, set once per device for each
// kernel (KERN: one static flag array per kernel, not per signature).
template <auto KERN>
hipError_t set_lds_f32(int bytes) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    static bool done[64] = {};
    if (dev >= 0 && dev < 64 && done[dev]) return hipSuccess;
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(KERN), hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess && dev >= 0 && dev < 64) done[dev] = true;
    return e;
}

template <int D, int DV, bool OB, bool NORM>
hipError_t launch_f32_t(const ChunkedF32Args& a, float* ws, hipStream_t st) {
    using G = F32Geo<D, DV, NORM>;
    const bool varlen = a.cu_seqlens != nullptr;
    const int n_pairs = a.n_seq * a.H;
    const int n_slot = f32_n_slot(varlen, a.T, a.n_seq);
    const long n_items = static_cast<long>(varlen ? a.H : n_pairs) * n_slot;
    const float *q = a.q, *k = a.k, *v = a.v;
    if (n_items > 0) {
        hipLaunchKernelGGL((delta_f32_prep_kernel<D, NORM>), dim3(static_cast<unsigned>((n_items + 3) / 4)), dim3(256), 0,
                           st, k, a.beta, a.cu_seqlens, a.n_seq, a.T, a.H, n_slot, n_items, ws, nullptr, nullptr);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    auto kern = delta_f32_kernel<D, DV, OB, NORM>;
    hipError_t e = set_lds_f32<delta_f32_kernel<D, DV, OB, NORM>>(G::BYTES);
    if (e != hipSuccess) return e;
    const int n_tiles = D / DV;
    const int slots = (n_pairs + 7) / 8;
    hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(slots * n_tiles * 8)), dim3(128 * G::NCW), G::BYTES, st, q, k,
                       v, a.s0, a.o, a.s_out, a.cu_seqlens, ws, n_pairs, a.T, a.H, n_tiles, n_slot, nullptr, 0);
    return hipGetLastError();
}

template <int D, int DV, bool NORM>
hipError_t launch_f32_n(const ChunkedF32Args& a, float* ws, hipStream_t st) {
    return a.out_bf16 ? launch_f32_t<D, DV, true, NORM>(a, ws, st) : launch_f32_t<D, DV, false, NORM>(a, ws, st);
}
template <int D, int DV>
hipError_t launch_f32_dv(const ChunkedF32Args& a, float* ws, hipStream_t st) {
    return a.norm ? launch_f32_n<D, DV, true>(a, ws, st) : launch_f32_n<D, DV, false>(a, ws, st);
}

}  // namespace

size_t chunked_f32_ws_bytes(bool varlen, int n_seq, int T, int H, bool norm) {
    const long rows = varlen ? H : static_cast<long>(n_seq) * H;
    return static_cast<size_t>(rows) * f32_n_slot(varlen, T, n_seq) * (norm ? ws_floats<true>() : ws_floats<false>()) * 4;
}

int chunked_f32_pick_tile(int D, long n_pairs, int requested) {
    if (requested == 16 || requested == 32) return requested;
    if (requested == 64) return 32;
    return n_pairs * (D / 32) >= 256 ? 32 : 16;
}

hipError_t launch_f32_bwd_prep(const float* q, const float* k, const float* beta, int n_pairs, int T, int H, int D,
                               float* ws_t2, float* ws_rec, hipStream_t st) {
    if (n_pairs == 0 || T == 0) return hipSuccess;
    const int n_slot = f32_n_slot(false, T, 0);
    const long n_items = static_cast<long>(n_pairs) * n_slot;
    const dim3 grid(static_cast<unsigned>((n_items + 3) / 4));
    if (D == 128)
        hipLaunchKernelGGL((delta_f32_prep_kernel<128, false, true>), grid, dim3(256), 0, st, k, beta, nullptr,
                           n_pairs / H, T, H, n_slot, n_items, ws_t2, ws_rec, q);
    else
        hipLaunchKernelGGL((delta_f32_prep_kernel<64, false, true>), grid, dim3(256), 0, st, k, beta, nullptr,
                           n_pairs / H, T, H, n_slot, n_items, ws_t2, ws_rec, q);
    return hipGetLastError();
}

namespace {
template <int D>
hipError_t launch_hist_sweep_t(const BwdArgs& a, const float* t2, const float* rec, float* w_out, float* s_hist,
                               float* g_hist, float* u_out, hipStream_t st) {
    constexpr int OFF2 = (F32Geo<D, 32, false, true>::BYTES + 255) & ~255;
    constexpr int BYTES = OFF2 + SwGeo<D>::BYTES;
    static_assert(BYTES <= 160 * 1024, "LDS");
    hipError_t e = set_lds_f32<f32_hist_sweep_kernel<D>>(BYTES);
    if (e != hipSuccess) return e;
    const int n_ch = (a.T + kC16 - 1) / kC16;
    const int n_span = (n_ch + kF32Span - 1) / kF32Span;
    const int slots = (a.n_pairs + 7) / 8;
    hipLaunchKernelGGL(f32_hist_sweep_kernel<D>, dim3(static_cast<unsigned>(slots * (D / 32) * 8)), dim3(512), BYTES,
                       st, static_cast<const float*>(a.q), static_cast<const float*>(a.k),
                       static_cast<const float*>(a.v), a.s0, a.go, a.gs, a.gv, a.gs0, t2, rec, w_out, s_hist, g_hist,
                       u_out, a.n_pairs, a.T, a.H, n_ch, n_span);
    return hipGetLastError();
}
}  // namespace

hipError_t launch_f32_hist_sweep(const BwdArgs& a, const float* t2, const float* rec, float* w_out, float* s_hist,
                                 float* g_hist, float* u_out, hipStream_t st) {
    if (a.n_pairs == 0) return hipSuccess;
    return a.D == 128 ? launch_hist_sweep_t<128>(a, t2, rec, w_out, s_hist, g_hist, u_out, st)
                      : launch_hist_sweep_t<64>(a, t2, rec, w_out, s_hist, g_hist, u_out, st);
}

hipError_t launch_chunked_f32(const ChunkedF32Args& a, void* ws, hipStream_t st) {
    if (a.n_seq == 0 || a.H == 0) return hipSuccess;
    float* w = static_cast<float*>(ws);
    const int dv = chunked_f32_pick_tile(a.D, static_cast<long>(a.n_seq) * a.H, a.dv_tile);
    if (a.D == 128) return dv == 16 ? launch_f32_dv<128, 16>(a, w, st) : launch_f32_dv<128, 32>(a, w, st);
    return dv == 16 ? launch_f32_dv<64, 16>(a, w, st) : launch_f32_dv<64, 32>(a, w, st);
}

}  // namespace pm
