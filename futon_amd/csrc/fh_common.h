// Shared device types and launch plumbing for the futon MI355X (gfx950) encoder.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

// 64-lane wavefront helpers (CDNA).
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Kernel launch parameter blocks.  Every pointer is device memory.
struct GemmArgs {
    const void *A;       // [M, K] row-major activations (f16, or i8 codes)
    const void *B;       // [N, K] row-major weights (nn.Linear layout)
    const float *bias;   // [N] or null
    const float *resid;  // [M, ldr] f32 residual added in the epilogue, or null
    const f16 *resid_h;  // [M, ldr] f16 residual (used when resid is null), or null
    const float *a_scale;  // Q8: [M] per-row activation scales
    const float *b_scale;  // Q8: [N] per-row weight scales
    void *C;             // [M, ldc] output (f16 or f32)
    int M, N, K;
    int lda, ldb, ldc, ldr;
    int epi_lds;         // set by the launcher: stage the epilogue through LDS
    // LayerNorm folded into the binary16 GEMMs (A and resid_h hold the
    // un-normalized LN input y; x = (y − mean)·rstd·γ + β is never stored):
    const float *c1;     // LN_IN: [N] Σ_k B[n,k] (B = W·diag(γ), as stored)
    const float *c2;     // LN_IN: [N] Σ_k W[n,k]·β[k] + bias[n]
    const f32x2 *stats_in;      // [M] (mean, rstd) of A's rows (LN_IN) or of resid_h's rows (RES_LN)
    const float *ln_g, *ln_b;   // RES_LN: γ, β of resid_h's LayerNorm
    // Tiled kernel only: output row r takes its residual (and, with RES_LN,
    // its statistics) from row res_map[r] of resid/resid_h (stats_in), or
    // from row r when null.
    const int32_t *res_map;
};

// Fused feed-forward block (mlp.hip), hidden width 384:
// out = GELU(rstd·(y·W1ᵀ − mean·c1) + c2)·W2ᵀ + b2 + ((y − mean)·rstd·γ + β).
struct MlpArgs {
    const f16 *y;              // [M, 384] un-normalized LayerNorm input
    const f32x2 *stats;        // [M] (mean, rstd) of y's rows, or null: computed from y (row_stats' order)
    const f16 *w1;             // fc1 weights [I, 384] scaled by γ, fragment-ordered (mlp_w1_unit)
    const float *c1, *c2;      // [I] LayerNorm fold terms of fc1 (c2 includes fc1's bias)
    const f16 *w2;             // fc2 weights [384, I], fragment-ordered (mlp_w2_unit)
    const float *b2;           // [384] fc2 bias, or null
    const float *ln_g, *ln_b;  // [384] γ, β of y's LayerNorm (the residual)
    f16 *out;                  // [M, 384]
    f32x2 *stats_out;          // [M] (mean, rstd) of out's rows, or null
    // Optional output projection ahead of the block (attn non-null): y is
    // then yB = attn·Woᵀ + bo + ((ya − mean)·rstd·γa + βa), built on-chip
    // (y itself is unused and stats must be null).
    const f16 *attn;           // [M, 384] attention output, or null
    const f16 *wo;             // Wo [384, 384], fragment-ordered (mlp_w2_unit)
    const float *bo;           // [384] or null
    const f16 *ya;             // [M, 384] un-normalized input of the attention block's LayerNorm
    const f32x2 *stats_a;      // [M] (mean, rstd) of ya's rows
    const float *ga, *ba;      // [384] γ, β of that LayerNorm
    // Optional QKV projection of the next layer after the block (wq
    // non-null): qkv = f16(rstd·(out·Wq'ᵀ − mean·c1q) + c2q) with out's own
    // statistics (the LN_IN fold of the QKV GEMM).
    const f16 *wq;             // [1152, 384] γ-scaled, fragment-ordered (mlp_w2_unit)
    const float *c1q, *c2q;    // [1152]
    f16 *qkv;                  // [M, 1152]
    float eps;                 // LayerNorm epsilon of both statistics
    int M, I;
};

struct AttnArgs {
    const f16 *qkv;        // [T, 3H] f16: q | k | v, heads-major inside each
    const int32_t *offsets;  // [nseq + 1] packed sequence starts
    const float *rope_cos;   // [maxpos, d/2] or null
    const float *rope_sin;
    void *out;             // [T or nseq, ldo]
    int H, d, ldo;
    int seq0;              // first sequence of this launch (blockIdx.z counts from it)
    int q_limit;           // queries per sequence that produce output (1 = CLS row)
    int compact;           // output row = sequence index (CLS mode)
    float scale_log2e;     // (1/sqrt(d)) * log2(e)
};

// Host-side launchers (defined next to their kernels).
namespace fh {
// ACT_RES16 is internal to the GEMM launcher: no activation, binary16 output
// with a binary16 residual added in f32 before the single rounding.
enum Act { ACT_NONE = 0, ACT_GELU = 1, ACT_SWIGLU = 2, ACT_RES16 = 3 };
// LayerNorm folding of a binary16 GEMM: LN_IN — A is the LN input y, B the
// weights scaled by γ, and the epilogue forms rstd·(acc − mean·c1) + c2 with
// y's row statistics from stats_in (row_stats); RES_LN — the residual is
// LN(resid_h) rebuilt from stats_in, γ, β (binary16 output with ACT_NONE).
enum LnMode { LN_NONE = 0, LN_IN = 1, RES_LN = 2 };
hipError_t gemm_f16(const GemmArgs &a, int act, bool out_f32, hipStream_t s, int ln = LN_NONE);
hipError_t gemm_i8(const GemmArgs &a, int act, bool out_f32, hipStream_t s);
// Persistent LDS-ring GEMM (gemm_ring.hip).  B must be packed with
// ring_pack_row (rows permuted inside each 64-row block); gemm_ring_ok says
// whether a problem fits it (binary16, N % 128 == 0, K % 64 == 0; SwiGLU
// with binary16 output only).
bool gemm_ring_ok(const GemmArgs &a, int act, bool out_f32, int ln);
// The int8 form of the ring GEMM (A, B int8 codes with a_scale/b_scale, B
// rows in ring_pack_row order; f32 or binary16 output, an f32 residual with
// f32 output; act NONE or GELU): the same bits as gemm_i8.  K % 128 == 0.
bool gemm_ring_q8_ok(const GemmArgs &a, int act, bool out_f32);
hipError_t gemm_ring_q8(const GemmArgs &a, int act, bool out_f32, hipStream_t s);
// Whether an M×N problem has enough rows for the ring to beat the tiled GEMM.
bool gemm_ring_worth(int M, int N);
hipError_t gemm_ring(const GemmArgs &a, int act, bool out_f32, hipStream_t s, int ln = LN_NONE);
// out = B with rows in ring_pack_row order (N % 64 == 0, K % 8 == 0).
hipError_t ring_pack(const f16 *B, f16 *out, int N, int K, hipStream_t s);
// Row of the unpacked weight matrix stored at packed row r.
__host__ __device__ inline int ring_pack_row(int r) {
    const int p = r & 63, tn = p >> 4, g = (p >> 2) & 3, e = p & 3;
    return (r & ~63) | ((tn >> 1) * 32 + g * 8 + (tn & 1) * 4 + e);
}
// Fragment-ordered weight copies for mlp(): a sequence of 1-KB MFMA operand
// fragments (16 rows × 32 columns, lane l holding row l%16, columns
// 8·(l/16) .. +7), ordered the way each of the kernel's MLP_NW waves consumes
// them.  mlp_w1_unit / mlp_w2_unit give, for 16-byte unit u of the packed
// copy, the source row and first column of its 8 binary16 values.
constexpr int MLP_NW = 8;                          // waves per fused block
constexpr int MLP_NT1 = 128 / MLP_NW / 16;         // fc1 16-row tiles per wave and 128-feature chunk
constexpr int MLP_NT2 = 384 / MLP_NW / 16;         // fc2 16-row tiles per wave
// fc1 [I, K]: fragment f = (g·(K/32) + ks)·NT1 + tn for 16·NT1-row group g,
// k-step ks, tile tn; MFMA row 16tn + 4a + e of a group is its row
// 4·NT1·a + 4tn + e, so each lane ends with 4·NT1 consecutive features.
__host__ __device__ inline void mlp_w1_unit(long u, int K, int &row, int &col) {
    const int l = (int)(u & 63);
    long f = u >> 6;
    const int tn = (int)(f % MLP_NT1);
    f /= MLP_NT1;
    const int ks = (int)(f % (K / 32)), grp = (int)(f / (K / 32));
    const int p = 16 * tn + (l & 15);
    row = grp * 16 * MLP_NT1 + 4 * MLP_NT1 * ((p >> 2) & 3) + 4 * (p >> 4) + (p & 3);
    col = ks * 32 + (l >> 4) * 8;
}
// fc2 [384, I] (and each 384-row block of a taller matrix, one after the
// other: the output projection, the next layer's QKV): per 128-column chunk
// j, wave w (16·NT2 output rows), k-step ks, tile t:
// f = ((j·NW + w)·4 + ks)·NT2 + t; MFMA row 16t + 4a + e of a wave's rows
// is its row 4·NT2·a + 4t + e, so each lane ends with 4·NT2 consecutive
// outputs.
__host__ __device__ inline void mlp_w2_unit(long u, int K, int &row, int &col) {
    const long ub = 384L * K / 8;  // units per 384-row block
    const int blk = (int)(u / ub);
    u -= blk * ub;
    const int l = (int)(u & 63);
    long f = u >> 6;
    const int t = (int)(f % MLP_NT2);
    f /= MLP_NT2;
    const int ks = (int)(f % 4);
    f /= 4;
    const int w = (int)(f % MLP_NW), j = (int)(f / MLP_NW);
    const int p = 16 * t + (l & 15);
    row = 384 * blk + 16 * MLP_NT2 * w + 4 * MLP_NT2 * ((p >> 2) & 3) + 4 * (p >> 4) + (p & 3);
    col = j * 128 + ks * 32 + (l >> 4) * 8;
}
// out = the fragment-ordered copy of B [N, K]: kind 1 (fc1, K % 32 == 0,
// N % (16·MLP_NT1) == 0) or kind 2 (N % 384 == 0, K % 128 == 0).
// Compute units of the current device (queried once per process; 0 when
// the query fails).
int cu_count();
hipError_t mlp_pack(int kind, const f16 *B, f16 *out, int N, int K, hipStream_t s);
// Whether mlp() takes an M-row problem with intermediate width I, and
// whether it can also write the next layer's Q/K/V for M rows (32-bit
// buffer offsets into the [M, 1152] output).
bool mlp_ok(int M, int H, int I);
bool mlp_qkv_ok(int M);
hipError_t mlp(const MlpArgs &a, hipStream_t s);
// Sequences of at most ATTN_ONE_BLOCK_KEYS tokens take attention's
// one-key-block path (each query tile's softmax over all keys at once);
// longer ones the multi-block path (64-key blocks, online rescaling).  The
// two round differently, so a batch that mixes them is split (fh_encode).
constexpr int ATTN_ONE_BLOCK_KEYS = 128;
hipError_t attention(const AttnArgs &a, int nseq, int max_len, bool out_f32, hipStream_t s);
// rotateHalf of every token's Q and K in place (binary16 qkv [T, 3H], head
// width d, cos/sin tables [max_len, d/2]), with the rounding the attention
// kernels apply when they rotate: attention then runs without RoPE and gives
// the same bits.  Needs (d/2) % 8 == 0 (rope_qk_ok).
bool rope_qk_ok(int H, int d);
hipError_t rope_qk(f16 *qkv, const int32_t *offsets, int nseq, int max_len, int H, int d, const float *cos_t,
                   const float *sin_t, hipStream_t s);
// gamma == null (only for H/64 in {4, 6, 8, 12, 16}) writes the un-normalized
// binary16 sum to x16 instead, for a consumer that folds this LayerNorm.
// q non-null (with gamma and x32): also the int8 codes and scales of the
// normalized rows, as quantize_rows would compute them from x32 (T = total
// rows, for the separate pass the generic kernel needs).
hipError_t embed_ln(const int32_t *ids, const int32_t *offsets, int nseq, int max_len,
                    const float *word, const float *type0, const float *pos, const float *gamma,
                    const float *beta, float eps, int H, float *x32, f16 *x16, hipStream_t s, int8_t *q = nullptr,
                    float *qs = nullptr, int T = 0, f32x2 *st = nullptr);
// Whether embed_ln can also write the un-normalized rows' (mean, rstd) (st,
// gamma null: row_stats' values, eps the LayerNorm's).
bool embed_stats_ok(int H);
// y32 or y16 (exactly one non-null) holds proj + bias + residual; q
// non-null (with x32): also the normalized rows' int8 codes and scales.
hipError_t layer_norm(const float *y32, const f16 *y16, int M, int H, const float *gamma, const float *beta,
                      float eps, float *x32, f16 *x16, hipStream_t s, int8_t *q = nullptr, float *qs = nullptr);
// (mean, rstd) of each binary16 row of y [M, H] (H in {256, 384, 512, 768,
// 1024}): float64 Σy and Σy², rounded to float32 like layerNormRows' float64
// statistics.
hipError_t row_stats(const f16 *y, int M, int H, float eps, f32x2 *st, hipStream_t s);
// Sequence i's first row (and its (mean, rstd) when st is non-null) → row i.
hipError_t gather_rows(const float *x32, const f16 *x16, const f32x2 *st, const int32_t *offsets, int nseq, int H,
                       float *xc32, f16 *xc16, f32x2 *stc, hipStream_t s);
hipError_t quantize_rows(const float *x, int M, int K, int ldx, int8_t *q, float *scale,
                         hipStream_t s);
// Mean pooling sums each sequence in POOL_SEG-token segments (token order
// inside a segment), then the segments in order.  `part` holds the segment
// sums: pool_part_rows(T, nseq) rows of H floats; sequence q's segments
// start at row pool_part_row(offsets[q], q) (≥ the previous sequence's
// last segment + 1, since ⌊a/G⌋ + ⌈L/G⌉ ≤ ⌊(a+L)/G⌋ + 1).
constexpr int POOL_SEG = 64;
__host__ __device__ inline int64_t pool_part_row(int64_t start, int64_t seq) { return start / POOL_SEG + seq; }
inline int64_t pool_part_rows(int64_t T, int64_t nseq) { return T / POOL_SEG + nseq + 1; }
hipError_t pool(const float *x32, const int32_t *offsets, int nseq, int max_len, int H, int cls_compact,
                int mean, int matryoshka_ln, int out_dim, int normalize, float *part, float *out, hipStream_t s);
// Mean pooling straight from the un-normalized last hidden state (binary16
// y16 or float32 y32, [T, H]): its LayerNorm (γ, β, eps) fused with the
// segment sums, then pool's per-sequence stage.  H / 64 ∈ {4, 6, 8, 12, 16}
// (ln_pool_ok).
bool ln_pool_ok(int H);
hipError_t ln_pool(const float *y32, const f16 *y16, const int32_t *offsets, int nseq, int max_len, int H,
                   const float *gamma, const float *beta, float eps, int matryoshka_ln, int out_dim, int normalize,
                   float *part, float *out, hipStream_t s);
// CLS pooling of the compact last-layer rows [nseq, H] with their LayerNorm
// (the same values as layer_norm then pool with cls_compact); H as ln_pool.
hipError_t ln_cls_pool(const float *y32, const f16 *y16, int nseq, int H, const float *gamma, const float *beta,
                       float eps, int matryoshka_ln, int out_dim, int normalize, float *out, hipStream_t s);
}  // namespace fh
