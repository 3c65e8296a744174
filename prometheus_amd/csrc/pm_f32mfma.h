// pm_f32mfma.h — fp32 MFMA (v_mfma_f32_16x16x4f32) building blocks shared by the fp32
// chunked forward and backward: the product wrappers and the swizzled LDS tile of 16
// fp32 token rows.  Internal to the translation unit that includes it (after
// pm_cdna4.h).
//
// Layout (lane l = 16 g + r): A operand A[r][g], B operand B[g][r], accumulator register
// v = D[4 g + v][r].  The accumulator registers of a 16x16 matrix M therefore serve as
//   * the B operand of a product contracting over M's rows (step v takes row 4 g + v), and
//   * the A operand of a product with M^T on the left, contracting over the same index,
// and a product contracting over M's columns needs the registers of M^T instead.
#pragma once

namespace pm {
namespace {

constexpr int kC16 = 16;  // tokens per chunk

__device__ __forceinline__ f32x4_t mfma4(float a, float b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
// Left * Right over a 16-token contraction, given the accumulators of Left^T and Right
// (plus c), in two accumulators.
__device__ __forceinline__ f32x4_t mm16(f32x4_t lt, f32x4_t r, f32x4_t c = f32x4_t{0.f, 0.f, 0.f, 0.f}) {
    const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
    f32x4_t a0 = mfma4(lt[0], r[0], c), a1 = mfma4(lt[1], r[1], z);
    a0 = mfma4(lt[2], r[2], a0);
    a1 = mfma4(lt[3], r[3], a1);
    return a0 + a1;
}

// LDS tile of 16 fp32 token rows of D values: the 16-byte chunk p of row t is stored at
// chunk t * (D / 4) + (p ^ t).  With it the float4 operand reads (lane (g, r): row r,
// chunk 4 m + g) and the column reads of K^T (lane (g, r): row 4 g + v, element 16 m + r)
// fall in distinct banks across each quarter wave.
template <int D>
__device__ __forceinline__ int f32_chunk(int t, int p) {
    return t * (D / 4) + (p ^ t);
}

}  // namespace
}  // namespace pm
