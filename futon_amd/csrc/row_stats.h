// LayerNorm row statistics shared by the row-statistics kernel (rowops.hip)
// and the fused feed-forward kernel (mlp.hip): both reduce in exactly this
// order, so they produce the same bits for the same row.
#pragma once

#include "fh_common.h"

namespace fh_rs {

// Sum over each 16-lane DPP row (xor 1, xor 2, half-row mirror, row mirror:
// the row total lands in all 16 lanes), in float64 as two 32-bit halves.
template <int CTRL>
__device__ __forceinline__ double dpp_step_f64(double v) {
    const int lo = __builtin_amdgcn_update_dpp(0, (int)__double2loint(v), CTRL, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)__double2hiint(v), CTRL, 0xF, 0xF, false);
    return v + __hiloint2double(hi, lo);
}
__device__ __forceinline__ double row16_sum_f64(double v) {
    v = dpp_step_f64<0xB1>(v);
    v = dpp_step_f64<0x4E>(v);
    v = dpp_step_f64<0x141>(v);
    return dpp_step_f64<0x140>(v);
}

// (mean, rstd) of one binary16 row of width 128·C held by the 16 lanes of a
// DPP row: lane l16 holds the row's 16-byte chunks c·16 + l16 (c < C) in
// v[c].  Σy and Σy² in float64 (Σy exact for binary16 data, each y² exact),
// mean = Σy/H, var = Σy²/H − mean², then float32(mean) and
// float32(1/sqrt(var + eps)): layerNormRows' (native/model.go:741-770)
// float64 statistics.  Every lane of the DPP row gets the result.
template <int C>
__device__ __forceinline__ f32x2 row_stats16(const f16x8 (&v)[C], float eps) {
    constexpr int H = 128 * C;
    double s1 = 0.0, s2 = 0.0;
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const double x = (double)(float)v[c][e];
            s1 += x;
            s2 = fma(x, x, s2);
        }
    s1 = row16_sum_f64(s1);
    s2 = row16_sum_f64(s2);
    const double mean = s1 / H;
    const double var = fmax(s2 / H - mean * mean, 0.0);
    return (f32x2){(float)mean, (float)(1.0 / sqrt(var + (double)eps))};
}

}  // namespace fh_rs
