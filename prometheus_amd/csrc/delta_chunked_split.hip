// delta_chunked_split.hip — K1 in split form: a fully parallel pass that builds
// every chunk's T (K1t), then the chunk recurrence (K1s) that copies T in with
// the chunk's token rows instead of building it.
//
// Same algebra as the single-stage kernel (delta_chunked.hip) and the
// reference's recurrence (kernels/__init__.py:357-376 per token, :421-458 over
// the sequence), per chunk of C = 64 tokens with start state S:
//
//   A = strict_lower(diag(beta) K K^T)      T = (I + A)^-1   (unit lower)
//   U = T diag(beta) (V - K S)              O = Q S + lower_incl_diag(Q K^T) U
//   S <- S + K^T U
//
// T depends on the chunk's K and beta only, so K1t builds it for every
// (sequence, head, chunk) at once (one wave each, K rows straight from global
// memory into MFMA operand registers) and writes T'' = -T diag(beta), packed in
// MFMA operand order, to the forward's workspace (6 KiB per chunk).  With it
//   U = T'' (K S - V)
// and the recurrence's dependent steps per chunk shrink to X = K S - V (the
// accumulators start at -V), U = T'' bf16(X), S += K^T U.
//
// K1s: one 256-thread workgroup per (sequence, head, d_v tile of DV columns)
// walks the sequence's chunks; every iteration ends with one LDS-only barrier.
//   * chain waves (DV / 16; wave w owns columns col0 + 16 w + [0, 16) of S as
//     fp32 MFMA accumulators) run chunk c from registers (K operand rows, K^T,
//     V loaded from LDS during chunk c - 1; T'' loaded from the workspace two
//     chunks ahead), hand U(c) and bf16 S_{c+1} to the output wave through LDS,
//     and copy the V columns of chunk c + 3;
//   * the output wave, one chunk behind, forms Y = Q S and O = Y + P U and
//     stores O with range-checked buffer stores; it copies chunk i + 2's Q rows;
//   * the P wave builds P = lower_incl_diag(Q K^T) into LDS and copies chunk
//     i + 2's K rows.
// The copies are HBM -> LDS (buffer_load ... lds); each wave waits for its own
// share of the next chunk's before the barrier.  The chain waves issue their T
// loads and V copies as inline asm with exact vmcnt waits (the compiler's
// conservative waits stalled the chain on copies issued in the same iteration).
// The products are the single-stage kernel's, except that T diag(beta) is
// applied as one bf16 operand and U = T'' bf16(K S - V) instead of
// T bf16(diag(beta)(V - K S)); results agree within bf16 rounding, not bitwise.

#include "pm_cdna4.h"
#include "pm_internal.h"

namespace pm {
namespace {

constexpr int kTElems = 6 * 512;  // bf16 elements of one packed T (6 KiB)

// Where chunk c of pair (seq, h) keeps its T in the workspace.  Fixed length:
// row = pair, slot = c, n_slot = ceil(T / 64).  Varlen: row = h and slot =
// floor(tok0 / 64) + seq + c, n_slot = ceil(total / 64) + n_seq; slots of
// consecutive sequences never overlap (the floor loses less than one chunk
// per sequence, and the + seq term gives each sequence one spare slot).
__host__ __device__ inline int split_n_slot(bool varlen, int T, int n_seq) {
    return varlen ? (T + kC - 1) / kC + n_seq : (T + kC - 1) / kC;
}

// ---------------------------------------------------------------- K1t
// One wave per (row, slot).  Waves whose slot holds no chunk (varlen gaps) exit.
template <int D>
__global__ __launch_bounds__(256) void delta_t_prep_kernel(const uint16_t* __restrict__ k,
                                                           const float* __restrict__ beta,
                                                           const int32_t* __restrict__ cu_seqlens,
                                                           int n_seq, int T, int H, int n_slot,
                                                           long n_items, uint16_t* __restrict__ tws) {
    constexpr int NKB = D / 32;
    const int lane = threadIdx.x & 63;
    const long item = static_cast<long>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (item >= n_items) return;
    const int row = static_cast<int>(item / n_slot), slot = static_cast<int>(item % n_slot);
    int seq, h, c;
    long tok0;
    int len;
    if (cu_seqlens) {
        h = row;
        // the sequence whose slot range starts at or before `slot`: the largest s with
        // floor(cu[s] / 64) + s <= slot (non-decreasing in s)
        int lo = 0, hi = n_seq - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            const int a = min(max(cu_seqlens[mid], 0), T);
            if (a / kC + mid <= slot) lo = mid; else hi = mid - 1;
        }
        seq = lo;
        const int a = min(max(cu_seqlens[seq], 0), T);
        const int z = min(max(cu_seqlens[seq + 1], a), T);
        tok0 = a;
        len = z - a;
        c = slot - (a / kC + seq);
        if (c < 0 || c * kC >= len) return;
    } else {
        const int pair = row;
        seq = pair / H;
        h = pair % H;
        tok0 = static_cast<long>(seq) * T;
        len = T;
        c = slot;
    }
    const int l16 = lane & 15, lg = lane >> 4;
    const int base = c * kC, clen = min(kC, len - base);
    const size_t tstride = static_cast<size_t>(H) * D;
    const size_t row0 = static_cast<size_t>(tok0 + base) * tstride + static_cast<size_t>(h) * D;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(k + row0, static_cast<unsigned>(((clen - 1) * tstride + D) * 2));
    const __amdgpu_buffer_rsrc_t rb =
        make_rsrc(beta + (tok0 + base) * H + h, static_cast<unsigned>(((clen - 1) * H + 1) * 4));
    bf16x8_t f[4][NKB];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
            const unsigned vo = static_cast<unsigned>((16 * r + l16) * tstride * 2) + 2u * (32 * kb + 8 * lg);
            f[r][kb] = __builtin_bit_cast(bf16x8_t, __builtin_amdgcn_raw_buffer_load_b128(rk, vo, 0, 0));
        }
    float bc[4];
    f32x4_t br4[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        bc[b] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rb, static_cast<unsigned>((16 * b + l16) * H * 4), 0, 0));
#pragma unroll
        for (int r = 0; r < 4; ++r)
            br4[b][r] = __uint_as_float(
                __builtin_amdgcn_raw_buffer_load_b32(rb, static_cast<unsigned>((16 * b + 4 * lg + r) * H * 4), 0, 0));
    }
    f32x4_t tb[10], tn[10];
    t_blocks<D>(f, bc, br4, lane, tb, tn);
    // T'' = -T diag(beta): block (i, j) holds T[16i + l16][16j + 4g + r] in this lane, so its
    // columns scale by -beta of token 16j + 4g + r
    {
        const int jb[10] = {0, 0, 1, 0, 1, 2, 0, 1, 2, 3};
#pragma unroll
        for (int x = 0; x < 10; ++x) tb[x] = tb[x] * -br4[jb[x]];
    }
    // packed operand block q = qblk(i, kb) holds blocks (i, 2 kb) and (i, 2 kb + 1)
    uint16_t* out = tws + (static_cast<size_t>(row) * n_slot + slot) * kTElems + lane * 8;
    const u32x2_t z = {0u, 0u};
    auto put = [&](int q, u32x2_t lo, u32x2_t hi) {
        const u32x4_t v = {lo.x, lo.y, hi.x, hi.y};
        *reinterpret_cast<u32x4_t*>(out + q * 512) = v;
    };
    put(0, cvt4(tb[0]), z);               // (0,0) | 0
    put(1, cvt4(tb[1]), cvt4(tb[2]));     // (1,0) | (1,1)
    put(2, cvt4(tb[3]), cvt4(tb[4]));     // (2,0) | (2,1)
    put(3, cvt4(tb[5]), z);               // (2,2) | 0
    put(4, cvt4(tb[6]), cvt4(tb[7]));     // (3,0) | (3,1)
    put(5, cvt4(tb[8]), cvt4(tb[9]));     // (3,2) | (3,3)
}

// ---------------------------------------------------------------- K1s
template <int D, int DV>
struct SplitGeo {
    static constexpr int NCW = DV / 16;               // chain waves (waves 0 .. NCW - 1)
    static constexpr int OW = 2;                      // the output wave
    static constexpr int PW = 3;                      // the P wave
    static constexpr int NKB = D / 32;
    static constexpr int NI_KQ = kC * D * 2 / 1024;   // 1 KiB copies per K or Q tile
    static constexpr int NI_V = kC * DV * 2 / 1024;   // ... per V tile
    static constexpr int NCP_P = NI_KQ;               // copies the P wave issues per chunk (K)
    static constexpr int NCP_O = NI_KQ;               // ... the output wave (Q)
    static constexpr int NST_O = NCW * 4;             // O stores of the output wave per chunk
    static constexpr int NVH = NI_V / NCW;            // V copies of each chain wave (its columns)
    // one chunk buffer: K, Q, V (bf16 token rows, swizzled)
    static constexpr int R_KS = 0;
    static constexpr int R_QS = R_KS + kC * D * 2;
    static constexpr int R_VS = R_QS + kC * D * 2;
    static constexpr int RAW = R_VS + kC * DV * 2;
    static constexpr int NRAW = 3;
    static constexpr int OFF_P = NRAW * RAW;                   // two packed P slots
    static constexpr int OFF_SB = OFF_P + 2 * kTElems * 2;     // two slots: bf16 S per chain wave
    static constexpr int SBSLOT = NCW * NKB * 1024;
    static constexpr int OFF_U = OFF_SB + 2 * SBSLOT;          // two slots: bf16 U per chain wave
    static constexpr int USLOT = NCW * 2 * 1024;
    static constexpr int BYTES = OFF_U + 2 * USLOT;
    static_assert(D == 64 || D == 128, "D");
    static_assert(DV == 16 || DV == 32, "DV");
    static_assert(2 * NVH + 6 <= 63 && NCP_O + NST_O <= 63 && NCP_P <= 63, "vmcnt range");
    static_assert(RAW % 16 == 0 && BYTES <= 160 * 1024, "LDS layout");
};

// A chain wave issues its T loads and its share of the copies as inline asm (dma16_asm,
// load16_asm), which the compiler does not see, and orders them with its own exact vmcnt
// waits: the compiler's wait insertion, merging loop iterations conservatively, would
// otherwise wait for copies issued in the same iteration.
__device__ __forceinline__ bf16x8_t load16_asm(__amdgpu_buffer_rsrc_t rs, unsigned voffset) {
    u32x4_t r;
    __asm__ volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen" : "=v"(r) : "v"(voffset), "s"(rs) : "memory");
    return __builtin_bit_cast(bf16x8_t, r);
}
// Wait until at most N of this wave's vector-memory operations are outstanding, with the
// registers of an asynchronous load tied to the wait.
template <int N>
__device__ __forceinline__ void vm_tie(bf16x8_t (&t)[6]) {
    __asm__ volatile("s_waitcnt vmcnt(%6)"
                     : "+v"(t[0]), "+v"(t[1]), "+v"(t[2]), "+v"(t[3]), "+v"(t[4]), "+v"(t[5])
                     : "n"(N)
                     : "memory");
}

// Tie registers filled by asynchronous LDS reads (inline asm) to a wait, so that the
// compiler neither reads nor copies them before their data has arrived.
__device__ __forceinline__ void lds_tie(u32x4_t (&a)[8]) {
    __asm__ volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]), "+v"(a[6]),
                       "+v"(a[7])
                     :
                     : "memory");
}
__device__ __forceinline__ void lds_tie(u32x2_t (&a)[4]) {
    __asm__ volatile("s_waitcnt lgkmcnt(0)" : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]) : : "memory");
}

template <int D, int DV, bool OUT_BF16>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void delta_chunked_split_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const float* __restrict__ s0, void* __restrict__ o_out, float* __restrict__ s_out,
    const int32_t* __restrict__ cu_seqlens, const uint16_t* __restrict__ tws, int n_pairs, int T, int H,
    int n_tiles, int n_slot) {
    using G = SplitGeo<D, DV>;
    constexpr int NKB = G::NKB;
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
    // this pair's T blocks: chunk c at tws + (t_row * n_slot + t_slot0 + c) * kTElems
    const int t_row = cu_seqlens ? h : pair;
    const int t_slot0 = cu_seqlens ? static_cast<int>(tok0 / kC) + seq : 0;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = static_cast<int>(uniform(static_cast<unsigned>(tid >> 6)));  // wave index
    const int l16 = lane & 15, lg = lane >> 4;
    const bool chain = w < G::NCW;
    const size_t sbase = static_cast<size_t>(pair) * D * D;
    const size_t tstride = static_cast<size_t>(H) * D;  // elements between tokens
    const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
    auto fence = []() __attribute__((always_inline)) { __builtin_amdgcn_sched_barrier(0); };

    auto raw = [&](int c) { return smem + (c % G::NRAW) * G::RAW; };
    auto pslot = [&](int c) { return reinterpret_cast<uint16_t*>(smem + G::OFF_P + (c & 1) * kTElems * 2); };
    auto sbslot = [&](int c, int cw) { return smem + G::OFF_SB + (c & 1) * G::SBSLOT + cw * NKB * 1024; };
    auto uslot = [&](int c, int cw) { return smem + G::OFF_U + (c & 1) * G::USLOT + cw * 2048; };
    // lane-linear 16-byte LDS accesses of a 1 KiB operand block
    auto st16 = [&](unsigned char* p, bf16x8_t x) { *reinterpret_cast<bf16x8_t*>(p + lane * 16) = x; };
    auto ld16 = [&](const unsigned char* p) { return *reinterpret_cast<const bf16x8_t*>(p + lane * 16); };

    // ---------------- HBM -> LDS copies of chunk c ----------------
    // Copy instruction i, lane L fills LDS bytes [1024 i + 16 L, +16) of a tile: row r,
    // stored chunk p, i.e. logical chunk p ^ f(r) of token row r.  Rows past the end of the
    // sequence read as zeros (buffer range check).
    // instructions [i0, i1) of the copy of chunk c's rows (a chunk past the end copies zeros:
    // the range is empty)
    auto copy_rows = [&](const uint16_t* base_ptr, int row_elems, unsigned char* dst, int i0, int i1, int c,
                         bool is_v, bool via_asm) __attribute__((always_inline)) {
        const int clen = c < n_chunks ? min(kC, len - c * kC) : 0;
        const size_t row0 = static_cast<size_t>(tok0 + (c < n_chunks ? c : 0) * kC) * tstride + static_cast<size_t>(h) * D;
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(
            base_ptr + row0 + (is_v ? col0 : 0),
            clen > 0 ? static_cast<unsigned>(((clen - 1) * tstride + row_elems) * 2) : 0u);
        unsigned char* rbuf = uniform_ptr(dst);
#pragma unroll
        for (int i = i0; i < i1; ++i) {
            const int pos = 512 * i + 8 * lane;  // element position in the tile
            const int r = pos / row_elems, p = (pos % row_elems) / 8;
            const int f = is_v ? v_f<DV>(r) : kq_f<D>(r);
            const unsigned vo = static_cast<unsigned>(r * tstride * 2) + 16u * (p ^ f);
            if (via_asm) dma16_asm(rs, rbuf + 1024 * i, vo);
            else copy_to_lds(rs, rbuf + 1024 * i, 16, vo);
        }
    };
    // the P wave copies K, the output wave Q, and chain wave w the V rows of its columns
    auto copy_k = [&](int c) __attribute__((always_inline)) {
        copy_rows(k, D, raw(c) + G::R_KS, 0, G::NI_KQ, c, false, false);
    };
    auto copy_q = [&](int c) __attribute__((always_inline)) {
        copy_rows(q, D, raw(c) + G::R_QS, 0, G::NI_KQ, c, false, false);
    };
    auto copy_v = [&](int c) __attribute__((always_inline)) {
        copy_rows(v, DV, raw(c) + G::R_VS, w * G::NVH, (w + 1) * G::NVH, c, true, true);
    };

    // chain waves: T'' of chunk c (clamped into the sequence) straight from the workspace into
    // registers, two chunks ahead of use (ttA for even chunks, ttB for odd)
    bf16x8_t ttA[6], ttB[6];
    auto load_t = [&](int c, bf16x8_t (&tt)[6]) __attribute__((always_inline)) {
        const int cc = min(c, n_chunks - 1);
        const __amdgpu_buffer_rsrc_t rt =
            make_rsrc(tws + (static_cast<size_t>(t_row) * n_slot + t_slot0 + cc) * kTElems, kTElems * 2);
#pragma unroll
        for (int x = 0; x < 6; ++x) tt[x] = load16_asm(rt, static_cast<unsigned>(1024 * x + 16 * lane));
    };
    // A chain wave's vector-memory operations come in one order, so that every wait
    // counts exactly: before B0, V(0), T(0), V(1); between B0 and B1, T(1), V(2); in the
    // iteration of chunk c (between B(c+1) and B(c+2)), T(c + 2) and V(c + 3) after U.
    // Before U(c): wait for T(c) (V(c+1), T(c+1), V(c+2) may be in flight); before the
    // iteration's barrier: wait for V(c+2) (T(c+2), V(c+3) may be in flight).

    if (n_chunks > 0) {
        // ---- prologue: chunks 0 and 1 in flight, chunk 0 landed at barrier B0 (the chain
        // waves' T loads join their copies in the steady-state order, see below)
        if (w == G::PW) {
            copy_k(0);
            copy_k(1);
            wait_vm_n<G::NCP_P>();
        } else if (w == G::OW) {
            copy_q(0);
            copy_q(1);
            wait_vm_n<G::NCP_O>();
        } else if (chain) {
            copy_v(0);
            load_t(0, ttA);
            copy_v(1);
            wait_vm_n<6 + G::NVH>();
        }
        lds_barrier();  // B0
    }

    if (chain) {
        // ============ chain wave: columns col0 + 16 w + [0, 16) of S ============
        f32x4_t S[D / 16];
        const int ecol = col0 + 16 * w + l16;
#pragma unroll
        for (int md = 0; md < D / 16; ++md) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int d = s_row_d(md, 4 * lg + r);
                S[md][r] = s0 ? s0[sbase + static_cast<size_t>(d) * D + ecol] : 0.f;
            }
        }
        bf16x8_t Sb[NKB];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) Sb[kb] = acc_to_b(S[2 * kb], S[2 * kb + 1]);
        if (n_chunks > 0) {
            bf16x8_t fk[NKB][4];
            u32x4_t kt[D / 64][8];  // K^T operands: [h4][x] (token half 0) and [h4][4 + x] (half 1)
            u32x2_t vv[4];
            auto tie_async = [&]() __attribute__((always_inline)) {
                lds_tie(vv);
#pragma unroll
                for (int h4 = 0; h4 < D / 64; ++h4) lds_tie(kt[h4]);
            };
            // chunk 0's operands, T(0) and T(1), and the start state for the output wave
            {
                const uint16_t* K0 = reinterpret_cast<const uint16_t*>(raw(0) + G::R_KS);
                const uint16_t* V0 = reinterpret_cast<const uint16_t*>(raw(0) + G::R_VS);
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                    for (int m = 0; m < 4; ++m) fk[kb][m] = lds_op_kq<D>(K0, 16 * m + l16, kb, lg);
#pragma unroll
                for (int h4 = 0; h4 < D / 64; ++h4)
#pragma unroll
                    for (int x = 0; x < 4; ++x) {
                        kt[h4][x] = lds_kt_issue<D, 0>(K0, 4 * h4 + x, lane);
                        kt[h4][4 + x] = lds_kt_issue<D, 32>(K0, 4 * h4 + x, lane);
                    }
#pragma unroll
                for (int m = 0; m < 4; ++m) vv[m] = lds_v_issue<DV>(V0, m, w, lane);
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb) st16(sbslot(0, w) + kb * 1024, Sb[kb]);
                load_t(1, ttB);
                copy_v(2);
                tie_async();
                wait_vm_n<6 + G::NVH>();  // V(1)
            }
            lds_barrier();  // B1

            // Chunk c (its operands in registers), loading chunk c + 1's from LDS as each
            // register falls free (after the last chunk, from a buffer whose contents are
            // never used: the body is one branch-free block), and T(c + 2) into tt after U.
            // Hand-scheduled in groups fenced by sched_barrier, one MFMA per group with at
            // most a few other instructions in its shadow, along the dependency chain
            // X -> R -> U -> S.  U(c) and bf16 S_{c+1} go to the output wave through LDS.
            auto run_chunk = [&](int c, bf16x8_t (&tt)[6]) __attribute__((always_inline)) {
                const unsigned char* rn = raw(c + 1);
                const uint16_t* Kn = reinterpret_cast<const uint16_t*>(rn + G::R_KS);
                const uint16_t* Vn = reinterpret_cast<const uint16_t*>(rn + G::R_VS);
                // X = K S - V (the accumulators start at -V)
                f32x4_t X[4];
#pragma unroll
                for (int m = 0; m < 4; ++m) X[m] = -widen4(vv[m]);
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
                    for (int m = 0; m < 4; ++m) {
                        X[m] = mfma32(fk[kb][m], Sb[kb], X[m]);
                        if (kb > 0) fk[kb - 1][m] = lds_op_kq<D>(Kn, 16 * m + l16, kb - 1, lg);
                        if (kb == 0) vv[m] = lds_v_issue<DV>(Vn, m, w, lane);
                        fence();
                    }
                }
                // R = bf16(K S - V); U = T'' R with T'' = -T diag(beta), so U = T diag(beta)(V - K S)
                const bf16x8_t Rb0 = acc_to_b(X[0], X[1]), Rb1 = acc_to_b(X[2], X[3]);
                vm_tie<2 * G::NVH + 6>(tt);  // T(c) has landed
                f32x4_t U[4];
                const f32x4_t u2a = mfma32(tt[2], Rb0, zero);
                fk[NKB - 1][0] = lds_op_kq<D>(Kn, l16, NKB - 1, lg);
                fence();
                const f32x4_t u3a = mfma32(tt[4], Rb0, zero);
                fk[NKB - 1][1] = lds_op_kq<D>(Kn, 16 + l16, NKB - 1, lg);
                fence();
                U[0] = mfma32(tt[0], Rb0, zero);
                fk[NKB - 1][2] = lds_op_kq<D>(Kn, 32 + l16, NKB - 1, lg);
                fence();
                U[1] = mfma32(tt[1], Rb0, zero);
                fk[NKB - 1][3] = lds_op_kq<D>(Kn, 48 + l16, NKB - 1, lg);
                fence();
                U[2] = mfma32(tt[3], Rb1, u2a);
                fence();
                U[3] = mfma32(tt[5], Rb1, u3a);
                fence();
                const bf16x8_t Ub0 = acc_to_b(U[0], U[1]), Ub1 = acc_to_b(U[2], U[3]);
                st16(uslot(c, w), Ub0);
                st16(uslot(c, w) + 1024, Ub1);
                load_t(c + 2, tt);
                copy_v(c + 3);
                fence();
                // S += K^T U; each K^T operand refilled after its product
#pragma unroll
                for (int h4 = 0; h4 < D / 64; ++h4) {
#pragma unroll
                    for (int x = 0; x < 4; ++x) {
                        S[4 * h4 + x] = mfma32(__builtin_bit_cast(bf16x8_t, kt[h4][x]), Ub0, S[4 * h4 + x]);
                        kt[h4][x] = lds_kt_issue<D, 0>(Kn, 4 * h4 + x, lane);
                        fence();
                        S[4 * h4 + x] = mfma32(__builtin_bit_cast(bf16x8_t, kt[h4][4 + x]), Ub1, S[4 * h4 + x]);
                        kt[h4][4 + x] = lds_kt_issue<D, 32>(Kn, 4 * h4 + x, lane);
                        fence();
                    }
                }
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb) {
                    Sb[kb] = acc_to_b(S[2 * kb], S[2 * kb + 1]);
                    st16(sbslot(c + 1, w) + kb * 1024, Sb[kb]);
                }
                tie_async();
                wait_vm_n<6 + G::NVH>();  // V(c + 2)
            };
            // iteration c + 1 runs chunk c; every iteration ends with a barrier (B2 .. B(n+1))
            for (int c = 0; c < n_chunks; c += 2) {
                run_chunk(c, ttA);
                lds_barrier();
                if (c + 1 < n_chunks) {
                    run_chunk(c + 1, ttB);
                    lds_barrier();
                }
            }
            wait_vm_n<0>();
        }
#pragma unroll
        for (int md = 0; md < D / 16; ++md) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int d = s_row_d(md, 4 * lg + r);
                s_out[sbase + static_cast<size_t>(d) * D + ecol] = S[md][r];
            }
        }
    } else if (w == G::OW && n_chunks > 0) {
        // ============ output wave: Y = Q S and O = Y + P U, one chunk behind the chain ============
        // Iteration i (after barrier Bi): O(i - 2) from Y(i - 2), P(i - 2) (registers) and
        // U(i - 2) (LDS); Y(i - 1) = Q(i - 1) S_{i-1} and P(i - 1) into registers; chunk i's Q
        // rows into registers.  Iterations 0 .. n_chunks end
        // with barriers B1 .. B(n+1); iteration n_chunks + 1 only finishes O(n_chunks - 1).
        // It also copies chunk i + 2's Q rows.
        bf16x8_t fq[NKB][4], pp[6];
        f32x4_t Y[G::NCW][4];
        auto load_q = [&](int c) __attribute__((always_inline)) {
            const uint16_t* Qs = reinterpret_cast<const uint16_t*>(raw(c) + G::R_QS);
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int m = 0; m < 4; ++m) fq[kb][m] = lds_op_kq<D>(Qs, 16 * m + l16, kb, lg);
        };
        // O(c) by range-checked buffer stores (rows past the end of the sequence are dropped
        // by the hardware)
        auto out_chunk = [&](int c) __attribute__((always_inline)) {
            const int clen = min(kC, len - c * kC);
            constexpr int ES = OUT_BF16 ? 2 : 4;
            const size_t rowe = static_cast<size_t>(tok0 + c * kC) * tstride + static_cast<size_t>(h) * D + col0;
            const __amdgpu_buffer_rsrc_t ro = make_rsrc(static_cast<unsigned char*>(o_out) + rowe * ES,
                                                        static_cast<unsigned>(((clen - 1) * tstride + DV) * ES));
#pragma unroll
            for (int cw = 0; cw < G::NCW; ++cw) {
                const bf16x8_t Ub0 = ld16(uslot(c, cw)), Ub1 = ld16(uslot(c, cw) + 1024);
                f32x4_t O[4];
                const f32x4_t o2a = mfma32(Ub0, pp[2], Y[cw][2]);
                const f32x4_t o3a = mfma32(Ub0, pp[4], Y[cw][3]);
                O[0] = mfma32(Ub0, pp[0], Y[cw][0]);
                O[1] = mfma32(Ub0, pp[1], Y[cw][1]);
                O[2] = mfma32(Ub1, pp[3], o2a);
                O[3] = mfma32(Ub1, pp[5], o3a);
                // lane (g, l16) holds O[16m + l16][16 cw + 4g .. +4)
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
            }
        };
        // Y(c) = Q(c) S_c (column rows: lane holds 4 columns of a token) and P(c)
        auto y_chunk = [&](int c) __attribute__((always_inline)) {
#pragma unroll
            for (int cw = 0; cw < G::NCW; ++cw) {
                bf16x8_t sb[NKB];
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb) sb[kb] = ld16(sbslot(c, cw) + kb * 1024);
#pragma unroll
                for (int m = 0; m < 4; ++m) Y[cw][m] = zero;
#pragma unroll
                for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                    for (int m = 0; m < 4; ++m) Y[cw][m] = mfma32(sb[kb], fq[kb][m], Y[cw][m]);
            }
            const uint16_t* Pp = pslot(c);
#pragma unroll
            for (int x = 0; x < 6; ++x) pp[x] = packed_a(Pp, x, lane);
        };
        for (int i = 0; i <= n_chunks + 1; ++i) {
            const bool cp = i + 2 < n_chunks;
            if (cp) copy_q(i + 2);
            const bool st = i >= 2;
            if (st) out_chunk(i - 2);
            if (i >= 1 && i <= n_chunks) y_chunk(i - 1);
            if (i < n_chunks) load_q(i);
            if (i <= n_chunks) {
                // chunk i + 1's Q (issued in iteration i - 1) has landed; the stores issued
                // after it are range-checked buffer stores, NST_O per iteration
                if (cp && st) wait_vm_n<G::NCP_O + G::NST_O>();
                else if (cp) wait_vm_n<G::NCP_O>();
                else if (st) wait_vm_n<G::NST_O>();
                else wait_vm_n<0>();
                lds_barrier();
            }
        }
    } else if (w == G::PW && n_chunks > 0) {
        // ============ P wave: P = lower_incl_diag(Q K^T) in packed operand order ============
        auto build_p = [&](int c) __attribute__((always_inline)) {
            const unsigned char* rb = raw(c);
            const uint16_t* Ks = reinterpret_cast<const uint16_t*>(rb + G::R_KS);
            const uint16_t* Qs = reinterpret_cast<const uint16_t*>(rb + G::R_QS);
            uint16_t* Pp = pslot(c);
            f32x4_t p[10];
#pragma unroll
            for (int x = 0; x < 10; ++x) p[x] = zero;
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
                bf16x8_t fk[4], fq[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    fk[r] = lds_op_kq<D>(Ks, 16 * r + l16, kb, lg);
                    fq[r] = lds_op_kq<D>(Qs, 16 * r + l16, kb, lg);
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
        // iteration j (after barrier Bj): P(j); chunk j + 2's K copies; barriers B1 .. B(n+1)
        for (int j = 0; j <= n_chunks; ++j) {
            const bool cp = j + 2 < n_chunks;
            if (cp) copy_k(j + 2);
            if (j < n_chunks) build_p(j);
            if (cp) wait_vm_n<G::NCP_P>(); else wait_vm_n<0>();
            lds_barrier();
        }
    } else if (n_chunks > 0) {
        for (int i = 0; i <= n_chunks; ++i) lds_barrier();  // an idle wave (one chain wave)
    }
}

// The dynamic-LDS limit is a per-device function attribute, set once per device for each
// kernel (KERN: one static flag array per kernel, not per signature).
template <auto KERN>
hipError_t set_lds_once(int bytes) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    static bool done[64] = {};
    if (dev >= 0 && dev < 64 && done[dev]) return hipSuccess;
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(KERN), hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess && dev >= 0 && dev < 64) done[dev] = true;
    return e;
}

template <int D, int DV, bool OB>
hipError_t launch_split_t(const ChunkedArgs& a, uint16_t* tws, hipStream_t st) {
    using G = SplitGeo<D, DV>;
    const bool varlen = a.cu_seqlens != nullptr;
    const int n_pairs = a.n_seq * a.H;
    const int n_slot = split_n_slot(varlen, a.T, a.n_seq);
    const long n_items = static_cast<long>(varlen ? a.H : n_pairs) * n_slot;
    hipLaunchKernelGGL(delta_t_prep_kernel<D>, dim3(static_cast<unsigned>((n_items + 3) / 4)), dim3(256), 0, st,
                       a.k, a.beta, a.cu_seqlens, a.n_seq, a.T, a.H, n_slot, n_items, tws);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    auto kern = delta_chunked_split_kernel<D, DV, OB>;
    if ((e = set_lds_once<delta_chunked_split_kernel<D, DV, OB>>(G::BYTES)) != hipSuccess) return e;
    const int n_tiles = D / DV;
    const int slots = (n_pairs + 7) / 8;
    hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(slots * 8 * n_tiles)), dim3(256), G::BYTES, st, a.q, a.k,
                       a.v, a.s0, a.o, a.s_out, a.cu_seqlens, tws, n_pairs, a.T, a.H, n_tiles, n_slot);
    return hipGetLastError();
}

template <int D, int DV>
hipError_t launch_split_dv(const ChunkedArgs& a, uint16_t* tws, hipStream_t st) {
    return a.out_bf16 ? launch_split_t<D, DV, true>(a, tws, st) : launch_split_t<D, DV, false>(a, tws, st);
}

}  // namespace

size_t chunked_split_ws_bytes(bool varlen, int n_seq, int T, int H) {
    const long rows = varlen ? H : static_cast<long>(n_seq) * H;
    return static_cast<size_t>(rows) * split_n_slot(varlen, T, n_seq) * kTElems * 2;
}

hipError_t launch_chunked_split(const ChunkedArgs& a, int dv, void* tws, hipStream_t st) {
    uint16_t* t = static_cast<uint16_t*>(tws);
    if (a.D == 128) return dv == 16 ? launch_split_dv<128, 16>(a, t, st) : launch_split_dv<128, 32>(a, t, st);
    return dv == 16 ? launch_split_dv<64, 16>(a, t, st) : launch_split_dv<64, 32>(a, t, st);
}

}  // namespace pm
