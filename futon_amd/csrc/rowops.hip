// Row-wise, HBM-bound kernels of the encoder forward: embedding gather +
// LayerNorm, (residual already added) LayerNorm, CLS-row gather, per-row
// int8 activation quantization, and pooling + Matryoshka + L2.
//
// LayerNorm statistics follow native/model.go:743-769: two-pass mean and
// variance accumulated in float64, inv = float32(1/sqrt(var + eps)),
// y = (x - float32(mean))·inv·γ + β.  One wavefront per row.
#include "fh_common.h"
#include "row_stats.h"

namespace {

constexpr int MAXV = 16;  // values per lane: H ≤ 1024

// LN over v[0..n) held by one wave (element e = lane + 64·j); writes x32/x16 row.
__device__ __forceinline__ void ln_row(float (&v)[MAXV], int H, const float *gamma,
                                       const float *beta, float eps, float *o32, f16 *o16) {
    const int lane = threadIdx.x & 63;
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
        const int e = lane + 64 * j;
        if (e < H) s += (double)v[j];
    }
    const double mean = wave_sum_f64(s) / (double)H;
    double q = 0.0;
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
        const int e = lane + 64 * j;
        if (e < H) {
            const double dd = (double)v[j] - mean;
            q += dd * dd;
        }
    }
    const double var = wave_sum_f64(q) / (double)H;
    const float inv = (float)(1.0 / sqrt(var + (double)eps));
    const float mf = (float)mean;
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
        const int e = lane + 64 * j;
        if (e < H) {
            const float y = gamma ? __fadd_rn(__fmul_rn(__fmul_rn(__fsub_rn(v[j], mf), inv), gamma[e]), beta[e])
                                  : __fmul_rn(__fsub_rn(v[j], mf), inv);
            if (o32) o32[e] = y;
            if (o16) o16[e] = (f16)y;
        }
    }
}

// x[t] = LN(word[id_t] + type[0] + pos[t]) — native/model.go:384-396.
// grid = (ceil(max_len/4), nseq), 4 waves per block, one token per wave.
__global__ __launch_bounds__(256) void embed_ln_kernel(const int32_t *ids, const int32_t *offsets,
                                                       const float *word, const float *type0,
                                                       const float *pos, const float *gamma,
                                                       const float *beta, float eps, int H,
                                                       float *x32, f16 *x16) {
    const int seq = blockIdx.y;
    const int start = offsets[seq], L = offsets[seq + 1] - start;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= L) return;
    const int lane = threadIdx.x & 63;
    const size_t row = (size_t)(start + t);
    const float *w = word + (size_t)ids[row] * H;
    float v[MAXV];
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
        const int e = lane + 64 * j;
        float x = 0.f;
        if (e < H) {
            x = w[e];
            if (type0) x = __fadd_rn(x, type0[e]);
            if (pos) x = __fadd_rn(x, pos[(size_t)t * H + e]);
        }
        v[j] = x;
    }
    ln_row(v, H, gamma, beta, eps, x32 ? x32 + row * H : nullptr, x16 + row * H);
}

// x = LN(y) per row (y already holds proj + bias + residual) — model.go:596-599, 631-633.
template <class T>
__global__ __launch_bounds__(256) void layer_norm_kernel(const T *y, int M, int H,
                                                         const float *gamma, const float *beta,
                                                         float eps, float *x32, f16 *x16) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    const int lane = threadIdx.x & 63;
    const T *src = y + (size_t)row * H;
    float v[MAXV];
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
        const int e = lane + 64 * j;
        v[j] = e < H ? (float)src[e] : 0.f;
    }
    ln_row(v, H, gamma, beta, eps, x32 ? x32 + (size_t)row * H : nullptr, x16 ? x16 + (size_t)row * H : nullptr);
}

// xc[i] = x[offsets[i]]: the CLS rows the last layer computes (model.go:403-410),
// from the f32 and/or f16 stream.
__global__ void gather_rows_kernel(const float *x32, const f16 *x16, const f32x2 *st, const int32_t *offsets, int H,
                                   float *xc32, f16 *xc16, f32x2 *stc) {
    const int seq = blockIdx.x;
    const size_t src = (size_t)offsets[seq] * H, dst = (size_t)seq * H;
    if (st && threadIdx.x == 0) stc[seq] = st[offsets[seq]];
    for (int e = threadIdx.x; e < H; e += blockDim.x) {
        if (x32) xc32[dst + e] = x32[src + e];
        if (x16) xc16[dst + e] = x16[src + e];
    }
}

__global__ __launch_bounds__(256) void quantize_rows_kernel(const float *x, int M, int K, int ldx,
                                                            int8_t *q, float *scale) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    const int lane = threadIdx.x & 63;
    const float *src = x + (size_t)row * ldx;
    float amax = 0.f;
    for (int e = lane; e < K; e += 64) amax = fmaxf(amax, fabsf(src[e]));
    amax = wave_max(amax);
    int8_t *dst = q + (size_t)row * K;
    if (amax == 0.f) {
        for (int e = lane; e < K; e += 64) dst[e] = 0;
        if (lane == 0) scale[row] = 0.f;
        return;
    }
    const double inv = 127.0 / (double)amax;
    for (int e = lane; e < K; e += 64) {
        double c = round((double)src[e] * inv);
        c = fmin(127.0, fmax(-127.0, c));
        dst[e] = (int8_t)c;
    }
    if (lane == 0) scale[row] = __fdiv_rn(amax, 127.0f);
}

// Width-specialized LayerNorm for H = 64·VPL (VPL even).  A lane owns VPL
// elements of its row: the first 256·(VPL/4) in 4-element chunks
// (elements 4·(64·c + lane) .. +3 of chunk c), then, when VPL % 4 == 2, the
// next 128 in pairs (256·(VPL/4) + 2·lane .. +1), so every access is a
// 16/8-byte (f32) or 8/4-byte (f16) vector and a wave covers contiguous
// memory.  Statistics in float32, two-pass (mean, then centered variance),
// which keeps the relative error of the normalized values near 1e-7.
// Wave sum without LDS traffic: DPP butterflies inside each 16-lane row
// (xor 1, xor 2, half-row mirror, row mirror leave the row sum in every lane
// of the row), then the four row sums read out as scalars.
template <int CTRL>
__device__ __forceinline__ float dpp_step(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_sum_f32(float v) {
    v = dpp_step<0xB1>(v);   // quad_perm [1,0,3,2]
    v = dpp_step<0x4E>(v);   // quad_perm [2,3,0,1]
    v = dpp_step<0x141>(v);  // row_half_mirror
    v = dpp_step<0x140>(v);  // row_mirror
    const int b = __builtin_bit_cast(int, v);
    return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16))) +
           (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48)));
}

template <int VPL>
__device__ __forceinline__ void ld_row(const float *p, int lane, float (&v)[VPL]) {
    constexpr int N4 = VPL / 4;
#pragma unroll
    for (int c = 0; c < N4; ++c) {
        const f32x4 t = *(const f32x4 *)(p + 4 * (64 * c + lane));
#pragma unroll
        for (int i = 0; i < 4; ++i) v[4 * c + i] = t[i];
    }
    if (VPL % 4) {
        const f32x2 t = *(const f32x2 *)(p + 256 * N4 + 2 * lane);
        v[4 * N4] = t[0];
        v[4 * N4 + 1] = t[1];
    }
}
template <int VPL>
__device__ __forceinline__ void ld_row(const f16 *p, int lane, float (&v)[VPL]) {
    constexpr int N4 = VPL / 4;
#pragma unroll
    for (int c = 0; c < N4; ++c) {
        const f16x4 t = *(const f16x4 *)(p + 4 * (64 * c + lane));
#pragma unroll
        for (int i = 0; i < 4; ++i) v[4 * c + i] = (float)t[i];
    }
    if (VPL % 4) {
        const f16x2 t = *(const f16x2 *)(p + 256 * N4 + 2 * lane);
        v[4 * N4] = (float)t[0];
        v[4 * N4 + 1] = (float)t[1];
    }
}
template <int VPL>
__device__ __forceinline__ void st_row(float *o32, f16 *o16, int lane, const float (&y)[VPL]) {
    constexpr int N4 = VPL / 4;
#pragma unroll
    for (int c = 0; c < N4; ++c) {
        const int e = 4 * (64 * c + lane);
        if (o32) *(f32x4 *)(o32 + e) = (f32x4){y[4 * c], y[4 * c + 1], y[4 * c + 2], y[4 * c + 3]};
        if (o16) *(f16x4 *)(o16 + e) = (f16x4){(f16)y[4 * c], (f16)y[4 * c + 1], (f16)y[4 * c + 2], (f16)y[4 * c + 3]};
    }
    if (VPL % 4) {
        const int e = 256 * N4 + 2 * lane;
        if (o32) *(f32x2 *)(o32 + e) = (f32x2){y[4 * N4], y[4 * N4 + 1]};
        if (o16) *(f16x2 *)(o16 + e) = (f16x2){(f16)y[4 * N4], (f16)y[4 * N4 + 1]};
    }
}

// Per-row int8 codes of a row held in ld_row's layout (quantizeRowQ8,
// native/quant.go:42-70, as the activation quantizer of matMulTQ8,
// quant.go:104-110): scale = float32(amax)/127; code =
// round-half-away(float64(v)·(127/float64(amax))) clamped to ±127; a zero
// row gives zero codes and scale 0.  Four codes per 32-bit store.
template <int VPL>
__device__ __forceinline__ void quant_row_v(const float (&v)[VPL], int lane, int8_t *q, float *scale) {
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) amax = fmaxf(amax, fabsf(v[j]));
    amax = wave_max(amax);
    const double inv = amax == 0.f ? 0.0 : 127.0 / (double)amax;
    auto code = [&](float x) -> uint32_t {
        const double c = fmin(127.0, fmax(-127.0, round((double)x * inv)));
        return (uint32_t)(uint8_t)(int8_t)(int)c;
    };
    constexpr int N4 = VPL / 4;
#pragma unroll
    for (int c = 0; c < N4; ++c)
        *(uint32_t *)(q + 4 * (64 * c + lane)) =
            code(v[4 * c]) | code(v[4 * c + 1]) << 8 | code(v[4 * c + 2]) << 16 | code(v[4 * c + 3]) << 24;
    if (VPL % 4) *(uint16_t *)(q + 256 * N4 + 2 * lane) = (uint16_t)(code(v[4 * N4]) | code(v[4 * N4 + 1]) << 8);
    if (lane == 0) *scale = amax == 0.f ? 0.f : __fdiv_rn(amax, 127.0f);
}

// One row per wave, held in registers between the absmax and the codes.
template <int VPL>
__global__ __launch_bounds__(256) void quantize_rows_v_kernel(const float *x, int M, int ldx, int8_t *q,
                                                              float *scale) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    const int lane = threadIdx.x & 63;
    float v[VPL];
    ld_row<VPL>(x + (size_t)row * ldx, lane, v);
    quant_row_v<VPL>(v, lane, q + (size_t)row * (64 * VPL), scale + row);
}

// Normalizes v (a row in ld_row's layout) in place with statistics of the
// row; gw/gb hold this lane's γ/β elements.
template <int VPL>
__device__ __forceinline__ void ln_norm_v(float (&v)[VPL], const float (&gw)[VPL], const float (&gb)[VPL], float eps) {
    constexpr int H = 64 * VPL;
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) s += v[j];
    const float mean = wave_sum_f32(s) * (1.0f / H);
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        const float d = v[j] - mean;
        q += d * d;
    }
    const float var = wave_sum_f32(q) * (1.0f / H);
    const float inv = 1.0f / sqrtf(var + eps);
#pragma unroll
    for (int j = 0; j < VPL; ++j) v[j] = (v[j] - mean) * inv * gw[j] + gb[j];
}
// ln_norm_v, then the row written out.
template <int VPL>
__device__ __forceinline__ void ln_row_v(float (&v)[VPL], const float (&gw)[VPL], const float (&gb)[VPL], float eps,
                                         float *o32, f16 *o16) {
    ln_norm_v<VPL>(v, gw, gb, eps);
    st_row<VPL>(o32, o16, threadIdx.x & 63, v);
}
// Column of element j of a lane's row in ld_row's layout.
template <int VPL>
__device__ __forceinline__ int row_col(int j, int lane) {
    constexpr int N4 = VPL / 4;
    return j < 4 * N4 ? 4 * (64 * (j >> 2) + lane) + (j & 3) : 256 * N4 + 2 * lane + (j - 4 * N4);
}

// (mean, rstd) per row of binary16 y [M, 128·C]: 16 lanes per row, C
// 16-byte chunks per lane, four rows per wave.  Σy and Σy² in float64
// (Σy exact for binary16 data), mean = Σy/H, var = Σy²/H − mean² in float64,
// then float32(mean) and float32(1/sqrt(var + eps)): layerNormRows'
// (native/model.go:741-770) float64 statistics, for the folded GEMMs.
template <int C>
__global__ __launch_bounds__(256) void row_stats_kernel(const f16 *y, int M, float eps, f32x2 *st) {
    constexpr int H = 128 * C;
    const int lane = threadIdx.x & 63;
    const int row = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 4 + (lane >> 4);
    const int r = min(row, M - 1);
    const int l16 = lane & 15;
    f16x8 v[C];
#pragma unroll
    for (int c = 0; c < C; ++c) v[c] = *(const f16x8 *)(y + (size_t)r * H + (c * 16 + l16) * 8);
    const f32x2 s = fh_rs::row_stats16<C>(v, eps);
    if (l16 == 0 && row < M) st[row] = s;
}

// Two rows per wave: both rows and γ/β are requested before any reduction,
// so one memory latency covers the pair.
// q non-null: also the int8 codes and scale of each normalized row (the
// activation quantizer of the next int8 GEMM, quant_row_v).
template <int VPL, class T>
__global__ __launch_bounds__(256) void layer_norm_v_kernel(const T *y, int M, const float *gamma,
                                                           const float *beta, float eps, float *x32, f16 *x16,
                                                           int8_t *q, float *qs) {
    constexpr int H = 64 * VPL;
    const int row = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 2;
    if (row >= M) return;
    const bool two = row + 1 < M;
    const int lane = threadIdx.x & 63;
    float v0[VPL], v1[VPL], gw[VPL], gb[VPL];
    ld_row<VPL>(y + (size_t)row * H, lane, v0);
    if (two) ld_row<VPL>(y + (size_t)(row + 1) * H, lane, v1);
    ld_row<VPL>(gamma, lane, gw);
    ld_row<VPL>(beta, lane, gb);
    ln_row_v<VPL>(v0, gw, gb, eps, x32 ? x32 + (size_t)row * H : nullptr, x16 ? x16 + (size_t)row * H : nullptr);
    if (q) quant_row_v<VPL>(v0, lane, q + (size_t)row * H, qs + row);
    if (two) {
        ln_row_v<VPL>(v1, gw, gb, eps, x32 ? x32 + (size_t)(row + 1) * H : nullptr,
                      x16 ? x16 + (size_t)(row + 1) * H : nullptr);
        if (q) quant_row_v<VPL>(v1, lane, q + (size_t)(row + 1) * H, qs + row + 1);
    }
}
// With gamma null: the un-normalized sum in binary16 for a consumer that
// folds this LayerNorm, and, when st is set, its rows' (mean, rstd) as
// row_stats_kernel computes them from those binary16 values: the block's four
// rows are staged in LDS and wave 0 reduces them with row_stats' lane layout
// (16 lanes a row), so the statistics are the same bits without a second
// pass over the rows.  (Each wave reducing its own row, every 16-lane group
// the same one, measured slower: four times the float64 work a block.)
template <int VPL>
__global__ __launch_bounds__(256) void embed_ln_v_kernel(const int32_t *ids, const int32_t *offsets,
                                                         const float *word, const float *type0, const float *pos,
                                                         const float *gamma, const float *beta, float eps,
                                                         float *x32, f16 *x16, int8_t *q, float *qs, f32x2 *st) {
    constexpr int H = 64 * VPL;
    __shared__ __attribute__((aligned(16))) f16 srow[4][H];
    const int seq = blockIdx.y;
    const int start = offsets[seq], L = offsets[seq + 1] - start;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    const bool stats = H % 128 == 0 && !gamma && st;  // block-uniform: every wave reaches the barrier below
    if (t >= L && !stats) return;
    const int lane = threadIdx.x & 63;
    const size_t row = (size_t)(start + t);
    if (t < L) {
        float v[VPL], u[VPL];
        ld_row<VPL>(word + (size_t)ids[row] * H, lane, v);
        if (type0) {
            ld_row<VPL>(type0, lane, u);
#pragma unroll
            for (int j = 0; j < VPL; ++j) v[j] += u[j];
        }
        if (pos) {
            ld_row<VPL>(pos + (size_t)t * H, lane, u);
#pragma unroll
            for (int j = 0; j < VPL; ++j) v[j] += u[j];
        }
        if (!gamma) {  // un-normalized sum, for a consumer that folds this LayerNorm
            st_row<VPL>(nullptr, x16 + row * H, lane, v);
            if (stats) st_row<VPL>(nullptr, srow[threadIdx.x >> 6], lane, v);
        } else {
            float gw[VPL], gb[VPL];
            ld_row<VPL>(gamma, lane, gw);
            ld_row<VPL>(beta, lane, gb);
            ln_row_v<VPL>(v, gw, gb, eps, x32 ? x32 + row * H : nullptr, x16 + row * H);
            if (q) quant_row_v<VPL>(v, lane, q + row * H, qs + row);
        }
    }
    if constexpr (H % 128 == 0) {
        if (!stats) return;
        __syncthreads();
        if (threadIdx.x < 64) {
            constexpr int C = H / 128;
            const int r = lane >> 4, l16 = lane & 15, tr = blockIdx.x * 4 + r;
            f16x8 w8[C];
#pragma unroll
            for (int c = 0; c < C; ++c) w8[c] = *(const f16x8 *)&srow[r][(c * 16 + l16) * 8];
            const f32x2 rs = fh_rs::row_stats16<C>(w8, eps);
            if (l16 == 0 && tr < L) st[start + tr] = rs;
        }
    }
}

__device__ double block_sum_f64(double v, double *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    v = wave_sum_f64(v);
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    double t = 0.0;
    for (int w = 0; w < nw; ++w) t += red[w];
    return t;
}

// Mean pooling, first stage: the float32 column sums of each POOL_SEG-token
// segment of each sequence, in token order, over the whole chip (one block
// per (segment, sequence), 4 columns per thread).  Segment j of sequence q
// goes to partial row fh::pool_part_row(offsets[q], q) + j: the rows of
// different sequences never overlap, and a sequence's sums do not depend
// on the rest of the batch.
__global__ __launch_bounds__(256) void pool_partial_kernel(const float *__restrict__ x32,
                                                           const int32_t *__restrict__ offsets, int H,
                                                           float *__restrict__ part) {
    const int seq = blockIdx.y, j = blockIdx.x;
    const int start = offsets[seq], L = offsets[seq + 1] - start;
    const int t0 = j * fh::POOL_SEG;
    if (t0 >= L) return;
    const int t1 = min(L, t0 + fh::POOL_SEG);
    float *dst = part + (size_t)(fh::pool_part_row(start, seq) + j) * H;
    // Rows are loaded 16 at a time ahead of the in-order adds: one 64-token
    // segment is then 4 load latencies instead of a chain of 64.
    constexpr int RB = 16;
    for (int c = threadIdx.x * 4; c < H; c += blockDim.x * 4) {
        const float *src = x32 + (size_t)(start + t0) * H + c;
        f32x4 acc = *(const f32x4 *)src;
        int t = t0 + 1;
        for (; t + RB <= t1; t += RB) {
            f32x4 v[RB];
#pragma unroll
            for (int r = 0; r < RB; ++r) v[r] = *(const f32x4 *)(src + (size_t)(t - t0 + r) * H);
#pragma unroll
            for (int r = 0; r < RB; ++r)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[i] = __fadd_rn(acc[i], v[r][i]);
        }
        for (; t < t1; ++t) {
            const f32x4 v = *(const f32x4 *)(src + (size_t)(t - t0) * H);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = __fadd_rn(acc[i], v[i]);
        }
        *(f32x4 *)(dst + c) = acc;
    }
}

// The last LayerNorm fused with mean pooling's first stage, for the pooled
// rows only: block (segment j, sequence q) with 8 waves; wave w normalizes
// rows t0 + 8w .. t0 + 8w + 7 of the segment (layer_norm_v's arithmetic,
// ln_norm_v) and adds them up per column in token order, then the waves'
// sums are added in wave order into the segment's partial row (pool_part_row,
// as pool_partial_kernel).  The normalized rows are never written: the
// float32 hidden state of every token (4H bytes a token) is neither stored
// nor read back.  The order of the sums depends only on the sequence, not on
// the rest of the batch.
template <int VPL, class T>
__global__ __launch_bounds__(512) void ln_pool_partial_kernel(const T *__restrict__ y,
                                                              const int32_t *__restrict__ offsets,
                                                              const float *__restrict__ gamma,
                                                              const float *__restrict__ beta, float eps,
                                                              float *__restrict__ part) {
    constexpr int H = 64 * VPL, NWV = 8, RW = fh::POOL_SEG / NWV;
    __shared__ float wsum[NWV][H];
    const int seq = blockIdx.y, j = blockIdx.x;
    const int start = offsets[seq], L = offsets[seq + 1] - start;
    const int t0 = j * fh::POOL_SEG;
    if (t0 >= L) return;  // the whole block
    const int t1 = min(L, t0 + fh::POOL_SEG);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r0 = t0 + wave * RW, n = min(t1 - r0, RW);  // this wave's rows (none when n ≤ 0)
    if (n > 0) {
        float gw[VPL], gb[VPL], v[RW][VPL], acc[VPL];
        ld_row<VPL>(gamma, lane, gw);
        ld_row<VPL>(beta, lane, gb);
#pragma unroll
        for (int r = 0; r < RW; ++r)
            if (r < n) ld_row<VPL>(y + (size_t)(start + r0 + r) * H, lane, v[r]);
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            if (r < n) {
                ln_norm_v<VPL>(v[r], gw, gb, eps);
#pragma unroll
                for (int i = 0; i < VPL; ++i) acc[i] = r == 0 ? v[0][i] : __fadd_rn(acc[i], v[r][i]);
            }
        }
#pragma unroll
        for (int i = 0; i < VPL; ++i) wsum[wave][row_col<VPL>(i, lane)] = acc[i];
    }
    __syncthreads();
    const int nw = (t1 - t0 + RW - 1) / RW;  // waves that had rows
    float *dst = part + (size_t)(fh::pool_part_row(start, seq) + j) * H;
    for (int c = threadIdx.x; c < H; c += NWV * 64) {
        float sum = wsum[0][c];
        for (int w = 1; w < nw; ++w) sum = __fadd_rn(sum, wsum[w][c]);
        dst[c] = sum;
    }
}

// Pool → Matryoshka → L2 — native/model.go:417-453.  One block per sequence.
// CLS reads row seq of the compact last-layer buffer; mean adds the
// sequence's segment sums (pool_partial_kernel) in segment order in float32
// and scales by float32(1/L).
// Matryoshka truncation (with its LayerNorm when asked) and L2 of the pooled
// row in pooled[0..H) (every thread of the block calls it), into out[0..n).
__device__ void finish_pooled(float *pooled, double *red, int H, int mat_ln, int out_dim, int normalize,
                              float *out) {
    int n = H;
    if (out_dim != H) {
        if (mat_ln) {
            double s = 0.0;
            for (int e = threadIdx.x; e < H; e += blockDim.x) s += (double)pooled[e];
            const double mu = block_sum_f64(s, red) / (double)H;
            double q = 0.0;
            for (int e = threadIdx.x; e < H; e += blockDim.x) {
                const double dd = (double)pooled[e] - mu;
                q += dd * dd;
            }
            const double var = block_sum_f64(q, red) / (double)H;
            const float inv = (float)(1.0 / sqrt(var + (double)1e-5f));
            const float mf = (float)mu;
            __syncthreads();
            for (int e = threadIdx.x; e < H; e += blockDim.x)
                pooled[e] = __fmul_rn(__fsub_rn(pooled[e], mf), inv);
            __syncthreads();
        }
        n = out_dim;
    }
    float inv = 1.0f;
    if (normalize) {
        double ss = 0.0;
        for (int e = threadIdx.x; e < n; e += blockDim.x) ss += (double)pooled[e] * (double)pooled[e];
        ss = block_sum_f64(ss, red);
        if (ss > 0) inv = (float)(1.0 / sqrt(ss));
    }
    for (int e = threadIdx.x; e < n; e += blockDim.x) out[e] = normalize ? __fmul_rn(pooled[e], inv) : pooled[e];
}

__global__ __launch_bounds__(256) void pool_kernel(const float *x32, const float *part, const int32_t *offsets,
                                                   int H, int cls_compact, int mean, int mat_ln, int out_dim,
                                                   int normalize, float *out) {
    __shared__ float pooled[1024];
    __shared__ double red[4];
    const int seq = blockIdx.x;
    const int start = offsets[seq], L = offsets[seq + 1] - start;
    for (int e = threadIdx.x; e < H; e += blockDim.x) {
        float p;
        if (mean) {
            const int nseg = (L + fh::POOL_SEG - 1) / fh::POOL_SEG;
            const float *col = part + (size_t)fh::pool_part_row(start, seq) * H + e;
            p = col[0];
            for (int j = 1; j < nseg; ++j) p = __fadd_rn(p, col[(size_t)j * H]);
            p = __fmul_rn(p, __fdiv_rn(1.0f, (float)L));
        } else {
            p = x32[(size_t)(cls_compact ? seq : start) * H + e];
        }
        pooled[e] = p;
    }
    __syncthreads();
    finish_pooled(pooled, red, H, mat_ln, out_dim, normalize, out + (size_t)seq * (out_dim != H ? out_dim : H));
}

// CLS pooling of the compact last-layer rows yc [nseq, H] (binary16, or
// float32 on the Q8 path) with their LayerNorm: one wave normalizes the row
// with layer_norm_v's arithmetic (ln_norm_v) into LDS, then finish_pooled.
// The same values as the LayerNorm kernel followed by pool_kernel, without
// the float32 row written and read back or the launch between them.
template <int VPL, class T>
__global__ __launch_bounds__(256) void ln_cls_pool_kernel(const T *__restrict__ yc, const float *__restrict__ gamma,
                                                          const float *__restrict__ beta, float eps, int mat_ln,
                                                          int out_dim, int normalize, float *out) {
    constexpr int H = 64 * VPL;
    __shared__ float pooled[H];
    __shared__ double red[4];
    const int seq = blockIdx.x;
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        float v[VPL], gw[VPL], gb[VPL];
        ld_row<VPL>(yc + (size_t)seq * H, lane, v);
        ld_row<VPL>(gamma, lane, gw);
        ld_row<VPL>(beta, lane, gb);
        ln_norm_v<VPL>(v, gw, gb, eps);
#pragma unroll
        for (int i = 0; i < VPL; ++i) pooled[row_col<VPL>(i, lane)] = v[i];
    }
    __syncthreads();
    finish_pooled(pooled, red, H, mat_ln, out_dim, normalize, out + (size_t)seq * (out_dim != H ? out_dim : H));
}

}  // namespace

namespace fh {
bool embed_stats_ok(int H) { return H % 128 == 0 && (H / 64 == 4 || H / 64 == 6 || H / 64 == 8 || H / 64 == 12 || H / 64 == 16); }
hipError_t embed_ln(const int32_t *ids, const int32_t *offsets, int nseq, int max_len,
                    const float *word, const float *type0, const float *pos, const float *gamma,
                    const float *beta, float eps, int H, float *x32, f16 *x16, hipStream_t s, int8_t *q,
                    float *qs, int T, f32x2 *st) {
    if (nseq <= 0) return hipSuccess;
    if (st && (gamma || !embed_stats_ok(H))) return hipErrorInvalidValue;
    const dim3 grid((max_len + 3) / 4, nseq);
#define FH_EMB_V(V)                                                                                          \
    case V: hipLaunchKernelGGL(embed_ln_v_kernel<V>, grid, dim3(256), 0, s, ids, offsets, word, type0, pos, gamma, \
                               beta, eps, x32, x16, gamma ? q : nullptr, qs, st);                            \
        return hipGetLastError();
    if (H % 64 == 0) {
        switch (H / 64) {
            FH_EMB_V(4) FH_EMB_V(6) FH_EMB_V(8) FH_EMB_V(12) FH_EMB_V(16)
        default: break;
        }
    }
#undef FH_EMB_V
    hipLaunchKernelGGL(embed_ln_kernel, grid, dim3(256), 0, s, ids, offsets, word, type0, pos, gamma, beta, eps, H,
                       x32, x16);
    if (q && x32) return quantize_rows(x32, T, H, H, q, qs, s);
    return hipGetLastError();
}
hipError_t layer_norm(const float *y32, const f16 *y16, int M, int H, const float *gamma, const float *beta,
                      float eps, float *x32, f16 *x16, hipStream_t s, int8_t *q, float *qs) {
    if (M <= 0) return hipSuccess;
    const dim3 grid((M + 3) / 4), grid2((M + 7) / 8);
#define FH_LN_V(V)                                                                                             \
    case V:                                                                                                    \
        if (y16) hipLaunchKernelGGL((layer_norm_v_kernel<V, f16>), grid2, dim3(256), 0, s, y16, M, gamma, beta, eps, \
                                    x32, x16, q, qs);                                                          \
        else hipLaunchKernelGGL((layer_norm_v_kernel<V, float>), grid2, dim3(256), 0, s, y32, M, gamma, beta, eps, \
                                x32, x16, q, qs);                                                              \
        return hipGetLastError();
    if (H % 64 == 0 && gamma) {
        switch (H / 64) {
            FH_LN_V(4) FH_LN_V(6) FH_LN_V(8) FH_LN_V(12) FH_LN_V(16)
        default: break;
        }
    }
#undef FH_LN_V
    if (y16) hipLaunchKernelGGL(layer_norm_kernel<f16>, grid, dim3(256), 0, s, y16, M, H, gamma, beta, eps, x32, x16);
    else hipLaunchKernelGGL(layer_norm_kernel<float>, grid, dim3(256), 0, s, y32, M, H, gamma, beta, eps, x32, x16);
    if (q) {
        if (!x32) return hipErrorInvalidValue;
        return quantize_rows(x32, M, H, H, q, qs, s);
    }
    return hipGetLastError();
}
hipError_t row_stats(const f16 *y, int M, int H, float eps, f32x2 *st, hipStream_t s) {
    if (M <= 0) return hipSuccess;
    const dim3 grid((M + 15) / 16);
#define FH_RS_C(C)                                                                                  \
    case 128 * C: hipLaunchKernelGGL(row_stats_kernel<C>, grid, dim3(256), 0, s, y, M, eps, st); \
        return hipGetLastError();
    switch (H) {
        FH_RS_C(2) FH_RS_C(3) FH_RS_C(4) FH_RS_C(6) FH_RS_C(8)
    default: break;
    }
#undef FH_RS_C
    return hipErrorInvalidValue;
}
hipError_t gather_rows(const float *x32, const f16 *x16, const f32x2 *st, const int32_t *offsets, int nseq, int H,
                       float *xc32, f16 *xc16, f32x2 *stc, hipStream_t s) {
    if (nseq <= 0) return hipSuccess;
    hipLaunchKernelGGL(gather_rows_kernel, dim3(nseq), dim3(128), 0, s, x32, x16, st, offsets, H, xc32, xc16, stc);
    return hipGetLastError();
}
hipError_t quantize_rows(const float *x, int M, int K, int ldx, int8_t *q, float *scale,
                         hipStream_t s) {
    if (M <= 0) return hipSuccess;
#define FH_Q_V(V)                                                                                           \
    case V: hipLaunchKernelGGL(quantize_rows_v_kernel<V>, dim3((M + 3) / 4), dim3(256), 0, s, x, M, ldx, q, scale); \
        return hipGetLastError();
    if (K % 64 == 0 && ldx % 4 == 0) {
        switch (K / 64) {
            FH_Q_V(4) FH_Q_V(6) FH_Q_V(8) FH_Q_V(12) FH_Q_V(16) FH_Q_V(24) FH_Q_V(32) FH_Q_V(48)
        default: break;
        }
    }
#undef FH_Q_V
    hipLaunchKernelGGL(quantize_rows_kernel, dim3((M + 3) / 4), dim3(256), 0, s, x, M, K, ldx, q, scale);
    return hipGetLastError();
}
bool ln_pool_ok(int H) { return H % 64 == 0 && (H / 64 == 4 || H / 64 == 6 || H / 64 == 8 || H / 64 == 12 || H / 64 == 16); }
hipError_t ln_pool(const float *y32, const f16 *y16, const int32_t *offsets, int nseq, int max_len, int H,
                   const float *gamma, const float *beta, float eps, int matryoshka_ln, int out_dim, int normalize,
                   float *part, float *out, hipStream_t s) {
    if (nseq <= 0) return hipSuccess;
    if (!ln_pool_ok(H) || !part || max_len <= 0 || !gamma || !beta || !(y32 || y16)) return hipErrorInvalidValue;
    const dim3 grid((max_len + POOL_SEG - 1) / POOL_SEG, nseq);
#define FH_LNP(V)                                                                                                  \
    case V:                                                                                                        \
        if (y16) hipLaunchKernelGGL((ln_pool_partial_kernel<V, f16>), grid, dim3(512), 0, s, y16, offsets, gamma,   \
                                    beta, eps, part);                                                              \
        else hipLaunchKernelGGL((ln_pool_partial_kernel<V, float>), grid, dim3(512), 0, s, y32, offsets, gamma,     \
                                beta, eps, part);                                                                  \
        break;
    switch (H / 64) {
        FH_LNP(4) FH_LNP(6) FH_LNP(8) FH_LNP(12) FH_LNP(16)
    default: return hipErrorInvalidValue;
    }
#undef FH_LNP
    hipLaunchKernelGGL(pool_kernel, dim3(nseq), dim3(256), 0, s, (const float *)nullptr, part, offsets, H, 0, 1,
                       matryoshka_ln, out_dim, normalize, out);
    return hipGetLastError();
}
hipError_t ln_cls_pool(const float *y32, const f16 *y16, int nseq, int H, const float *gamma, const float *beta,
                       float eps, int matryoshka_ln, int out_dim, int normalize, float *out, hipStream_t s) {
    if (nseq <= 0) return hipSuccess;
    if (!ln_pool_ok(H) || !gamma || !beta || !(y32 || y16)) return hipErrorInvalidValue;
#define FH_LNC(V)                                                                                                \
    case V:                                                                                                      \
        if (y16) hipLaunchKernelGGL((ln_cls_pool_kernel<V, f16>), dim3(nseq), dim3(256), 0, s, y16, gamma, beta, \
                                    eps, matryoshka_ln, out_dim, normalize, out);                                \
        else hipLaunchKernelGGL((ln_cls_pool_kernel<V, float>), dim3(nseq), dim3(256), 0, s, y32, gamma, beta,   \
                                eps, matryoshka_ln, out_dim, normalize, out);                                    \
        break;
    switch (H / 64) {
        FH_LNC(4) FH_LNC(6) FH_LNC(8) FH_LNC(12) FH_LNC(16)
    default: return hipErrorInvalidValue;
    }
#undef FH_LNC
    return hipGetLastError();
}
hipError_t pool(const float *x32, const int32_t *offsets, int nseq, int max_len, int H, int cls_compact, int mean,
                int matryoshka_ln, int out_dim, int normalize, float *part, float *out, hipStream_t s) {
    if (nseq <= 0) return hipSuccess;
    if (mean) {
        if (!part || H % 4 || max_len <= 0) return hipErrorInvalidValue;
        hipLaunchKernelGGL(pool_partial_kernel, dim3((max_len + POOL_SEG - 1) / POOL_SEG, nseq), dim3(256), 0, s, x32,
                           offsets, H, part);
    }
    hipLaunchKernelGGL(pool_kernel, dim3(nseq), dim3(256), 0, s, x32, part, offsets, H, cls_compact, mean,
                       matryoshka_ln, out_dim, normalize, out);
    return hipGetLastError();
}
}  // namespace fh
