// Device helpers shared by the GEMM kernels' epilogues (gemm.hip,
// gemm_ring.hip): activations and the LayerNorm fold terms.
#pragma once

#include "fh_common.h"

namespace fh_epi {

// Rounds an epilogue value to binary16 from its f32 value.  The empty asm
// hides how x was produced, so the compiler cannot fold a final fma into a
// mixed-precision fma (v_fma_mix: one rounding straight to binary16): every
// GEMM kernel rounds the same f32 value to the same binary16.
__device__ __forceinline__ f16 to_f16(float x) {
    asm("" : "+v"(x));
    return (f16)x;
}

// erf-GELU, 0.5·x·(1 + erf(x/√2)) (native/mathf32.go:96-107), with the
// hardware reciprocal and exp.
__device__ __forceinline__ float gelu_erf(float x) {
    // x·Φ(x) with erfc(z) = t·P(t)·exp(−z²), t = 1/(1 + p·z), z = |x|/√2
    // (Abramowitz & Stegun 7.1.26, |error| ≤ 1.5e-7).  Constants folded:
    // p/√2, ½·a_i, and exp(−x²/2) = 2^(−x²·½·log2 e).
    const float t = __builtin_amdgcn_rcpf(fmaf(fabsf(x), 0.23164190f, 1.0f));
    float q = 0.53070271f;
    q = fmaf(q, t, -0.72657601f);
    q = fmaf(q, t, 0.71070687f);
    q = fmaf(q, t, -0.14224837f);
    q = fmaf(q, t, 0.12741480f);
    const float e = __builtin_amdgcn_exp2f((x * x) * -0.72134752f);
    // h = ½·x·erfc(|x|/√2) = x·(q·t)·e has the sign of x, so x·Φ(x), which is
    // h for x < 0 and x − h otherwise, is max(x, 0) − |x·q·t|·e.
    return fmaf(-fabsf(x * (q * t)), e, fmaxf(x, 0.f));
}
__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

// The LayerNorm terms below spell out every rounding (explicit fmaf and
// uncontracted products), so that each GEMM kernel computes them bit for bit
// alike whatever the compiler's contraction choices in its context.

// LN_IN fold of one 4-column group: rstd·(acc − mean·c1) + c2.
__device__ __forceinline__ f32x4 ln_fold_v(f32x4 v, f32x2 rs, f32x4 c1, f32x4 c2) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = fmaf(rs[1], fmaf(-rs[0], c1[i], v[i]), c2[i]);
    return v;
}
__device__ __forceinline__ f32x4 ln_fold(const GemmArgs &g, int col, f32x4 v, f32x2 rs) {
    return ln_fold_v(v, rs, *(const f32x4 *)(g.c1 + col), *(const f32x4 *)(g.c2 + col));
}
// RES_LN residual of 4 columns: (y − mean)·rstd·γ + β.
__device__ __forceinline__ f32x4 ln_resid_v(f16x4 y, f32x2 st, f32x4 gm, f32x4 bt) {
    f32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = fmaf(__fmul_rn((float)y[i] - st[0], st[1]), gm[i], bt[i]);
    return r;
}
__device__ __forceinline__ f32x4 ln_resid(const GemmArgs &g, f32x2 st, int col, f16x4 y) {
    return ln_resid_v(y, st, *(const f32x4 *)(g.ln_g + col), *(const f32x4 *)(g.ln_b + col));
}

}  // namespace fh_epi
