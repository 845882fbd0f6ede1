/*
 * futon_hip_ops.h — per-kernel C entry points of the gfx950 encoder, on
 * device pointers.  They expose each kernel that fh_encode chains, so every
 * step of the forward can be checked in isolation; the GEMM entry is the
 * device form of the reference's Kernel seam.
 *
 * All pointers are device pointers; `stream` is a hipStream_t (NULL = the
 * null stream).  Calls are asynchronous.  Return FH_OK or FH_E* (see
 * futon_hip.h); shapes outside a kernel's limits are FH_EINVAL.
 */
#ifndef FUTON_HIP_OPS_H
#define FUTON_HIP_OPS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FH_OP_F16 0 /* A, B binary16 */
#define FH_OP_I8 1  /* A, B int8 codes with per-row scales */

#define FH_OP_ACT_NONE 0
#define FH_OP_ACT_GELU 1
#define FH_OP_ACT_SWIGLU 2 /* B rows interleaved: 16 fc1 rows, 16 gate rows, … */

/* C[M,N'] = act(A[M,K] · B[N,K]ᵀ (· sA[m]·sB[n] for I8) + bias[N]) + resid[M,N'],
 * N' = N (N/2 for SwiGLU).  Output f32 when out_f32, else binary16.
 * resid is f32, or binary16 when resid_f16 (F16, no activation, binary16
 * output only: the sum is formed in f32 and rounded once).
 * Requires K % 16 == 0 for I8, K % 8 == 0 for F16, N % 4 == 0 (N % 32 for SwiGLU).
 * Replaces: Kernel.MatMulT / MatMulTF16 (native/kernel.go:26-43) and
 * q8Kernel.MatMulTQ8 (native/quant.go:92-137). */
int fh_op_gemm(int32_t dtype, const void *A, const void *B, const float *bias, const void *resid,
               int32_t resid_f16, const float *a_scale, const float *b_scale, void *C, int32_t M, int32_t N,
               int32_t K, int32_t act, int32_t out_f32, void *stream);

/* The same contraction on the persistent LDS-ring kernel (binary16 only):
 * B_packed is B with its rows permuted by fh_op_ring_pack.  Requires
 * N % 128 == 0 and K % 64 == 0; act is NONE, GELU or SWIGLU (SwiGLU:
 * binary16 output [M, N/2], no residual).  Gives the same bits as
 * fh_op_gemm on the unpacked B.
 * Replaces: Kernel.MatMulTF16 (native/kernel.go:26-43). */
int fh_op_gemm_ring(const void *A, const void *B_packed, const float *bias, const void *resid, int32_t resid_f16,
                    void *C, int32_t M, int32_t N, int32_t K, int32_t act, int32_t out_f32, void *stream);

/* The int8 contraction of fh_op_gemm (dtype I8: int8 codes A [M,K] and
 * B [N,K] with per-row scales, f32 output C [M,N], bias and f32 residual
 * optional) on the persistent LDS-ring kernel: B_packed is B's codes with
 * their rows permuted by fh_op_ring_pack (which moves 16-byte units, so it
 * takes the codes as a binary16 matrix of K/2 columns).  Requires
 * N % 128 == 0 and K % 128 == 0; act is NONE or GELU.  Gives the same bits
 * as fh_op_gemm with dtype I8.
 * Replaces: q8Kernel.MatMulTQ8 (native/quant.go:92-137). */
int fh_op_gemm_ring_q8(const void *A, const void *B_packed, const float *a_scale, const float *b_scale,
                       const float *bias, const float *resid, float *C, int32_t M, int32_t N, int32_t K,
                       int32_t act, void *stream);

/* The folded-LayerNorm forms of the binary16 GEMM (K % 64 == 0), on the
 * tiled kernel (ring = 0, B as is) or the ring kernel (ring = 1, B packed);
 * stats holds [M] (mean, rstd) float pairs (fh_op_row_stats):
 *  ln_mode 1 (LN_IN):  C = act(rstd·(A·Bᵀ − mean·c1) + c2) with A's row
 *                      statistics; act NONE or GELU, or SWIGLU (B, c1
 *                      and c2 interleaved as for fh_op_gemm, N % 128 == 0,
 *                      C [M, N/2]).
 *  ln_mode 2 (RES_LN): C = A·Bᵀ + bias + (resid_h − mean)·rstd·ln_g + ln_b
 *                      with resid_h's row statistics, rounded once.
 * C is binary16 [M, N].  These are the model's LayerNorm folds of
 * native/model.go:555-633 (LN(x)·Wᵀ and the residual LN). */
int fh_op_gemm_ln(int32_t ring, int32_t ln_mode, const void *A, const void *B, const float *c1, const float *c2,
                  const float *bias, const void *resid_h, const void *stats, const float *ln_g, const float *ln_b,
                  void *C, int32_t M, int32_t N, int32_t K, int32_t act, void *stream);

/* Per-row LayerNorm statistics of binary16 y [M, H] (H in 256, 384, 512,
 * 768, 1024): stats[r] = (mean, 1/sqrt(var + eps)) from float64 Σy and Σy²,
 * rounded to float32 — the float64 statistics of layerNormRows
 * (native/model.go:741-770) — for the folded GEMMs. */
int fh_op_row_stats(const void *y, int32_t M, int32_t H, float eps, void *stats, void *stream);

/* Row permutation of a binary16 [N, K] weight matrix (N % 64 == 0, K % 8 == 0)
 * into the order fh_op_gemm_ring reads: inside each 64-row block, packed row
 * 16·t + 4·g + e holds row 32·(t/2) + 8·g + 4·(t%2) + e.  No reference
 * counterpart (a layout of this build). */
int fh_op_ring_pack(const void *B, void *out, int32_t N, int32_t K, void *stream);

/* Fragment-ordered copy of a binary16 [N, K] weight matrix for fh_op_mlp: a
 * sequence of 1-KB MFMA operand fragments (16 rows × 32 columns; 16-byte
 * unit u holds row r, columns c .. c+7 with lane l = u % 64 taking row
 * l % 16 of its tile and columns 8·(l/16) ..).  kind 1 (fc1 [I, 384], N % 16
 * == 0, K % 32 == 0): fragment f = u / 64 is 16-row tile f / (K/32), k-step
 * f % (K/32).  kind 2 (fc2 [384, I] and any [384·n, K], K % 128 == 0; each
 * 384-row block packed in turn): f = ((8j + w)·4 + ks)·3 + t for 128-column
 * chunk j, 48-row group w, k-step ks, tile t, and MFMA row 16t + 4g + e of a
 * group is row 12g + 4t + e.  No reference counterpart (a layout of this
 * build). */
int fh_op_mlp_pack(int32_t kind, const void *B, void *out, int32_t N, int32_t K, void *stream);

/* The encoder layer's feed-forward block in one kernel, hidden width H = 384,
 * GELU, I % 128 == 0, I <= 2048:
 *   out = GELU(rstd·(y·W1ᵀ − mean·c1) + c2)·W2ᵀ + b2 + (y − mean)·rstd·ln_g + ln_b
 * y [M, 384] binary16 (un-normalized); stats [M] (mean, rstd) float pairs of
 * y's rows, or NULL to compute them in the kernel (the same bits as
 * fh_op_row_stats with eps); w1_packed = fh_op_mlp_pack kind 1 of W1
 * [I, 384], w2_packed = kind 2 of W2 [384, I], b2 may be NULL; out [M, 384]
 * binary16; stats_out, when not NULL, receives fh_op_row_stats(out, eps).
 * The intermediate GELU output never reaches memory; the result has the same
 * bits as fh_op_gemm_ln LN_IN + GELU followed by RES_LN.
 * Replaces: the MLP block of the encoder layer (native/model.go:607-633) and
 * the statistics of the LayerNorms on either side (:741-770). */
int fh_op_mlp(const void *y, const void *stats, const void *w1_packed, const float *c1, const float *c2,
              const void *w2_packed, const float *b2, const float *ln_g, const float *ln_b, void *out,
              void *stats_out, float eps, int32_t M, int32_t H, int32_t I, void *stream);

/* The rest of an encoder layer after attention, in one kernel (hidden 384,
 * GELU): yB = attn·Woᵀ + bo + (ya − mean_a)·rstd_a·ga + ba is built on-chip
 * (Wo = fh_op_mlp_pack kind 2 of the [384, 384] projection, bo may be NULL,
 * stats_a the (mean, rstd) of ya's rows), then out = fh_op_mlp's block of
 * yB with yB's statistics computed in the kernel.  With wq_packed (kind 2 of
 * the next layer's γ-scaled [1152, 384] QKV weights) it also writes
 * qkv [M, 1152] = the LN_IN fold of out with c1q/c2q and out's statistics.
 * Gives the same bits as fh_op_gemm_ln RES_LN for yB, fh_op_mlp, then
 * fh_op_gemm_ln LN_IN for qkv.  out may alias ya and stats_out stats_a.
 * Replaces: native/model.go:596-633 (output projection, residual + norm1, FFN,
 * residual) and the next layer's QKV projection (:555). */
int fh_op_outproj_mlp(const void *attn, const void *wo_packed, const float *bo, const void *ya, const void *stats_a,
                      const float *ga, const float *ba, const void *w1_packed, const float *c1, const float *c2,
                      const void *w2_packed, const float *b2, const float *ln_g, const float *ln_b, void *out,
                      void *stats_out, float eps, const void *wq_packed, const float *c1q, const float *c2q, void *qkv,
                      int32_t M, int32_t H, int32_t I, void *stream);

/* Multi-head attention over packed sequences: qkv [T, 3H] binary16 (q | k | v,
 * heads-major), offsets [nseq+1].  Output [T, H] (or [nseq, H] when compact,
 * holding each sequence's first q_limit=1 query row), f32 or binary16.
 * rope_cos/sin: [max_len, head_dim/2] tables or NULL.
 * Replaces: attendHead + softmaxScaled + rotateHalf (native/model.go:646-739). */
int fh_op_attention(const void *qkv, const int32_t *offsets, int32_t nseq, int32_t max_len, int32_t H,
                    int32_t heads, const float *rope_cos, const float *rope_sin, void *out,
                    int32_t q_limit, int32_t compact, int32_t out_f32, void *stream);

/* x32/x16[M,H] = LN(y) with γ, β (NULL γ = parameter-free); y is f32, or
 * binary16 when y_f16.
 * Replaces: layerNormRows (native/model.go:743-769). */
int fh_op_layer_norm(const void *y, int32_t y_f16, int32_t M, int32_t H, const float *gamma,
                     const float *beta, float eps, float *x32, void *x16, void *stream);

/* Per-row int8 codes + scales of x[M,K] (row stride K).
 * Replaces: quantizeRowQ8 over activation rows (native/quant.go:42-70, :104-110). */
int fh_op_quantize_rows(const float *x, int32_t M, int32_t K, int8_t *q, float *scale, void *stream);

/* x32/x16[T,H] = LN(word[id] + type0 + pos[t]).  type0/pos may be NULL.
 * Replaces: the embedding block of EncodeTokensKernel (native/model.go:384-396). */
int fh_op_embed_ln(const int32_t *ids, const int32_t *offsets, int32_t nseq, int32_t max_len,
                   const float *word, const float *type0, const float *pos, const float *gamma,
                   const float *beta, float eps, int32_t H, float *x32, void *x16, void *stream);

/* out[nseq, out_dim] = L2(Matryoshka(pool(x))).  cls_compact: x is [nseq, H]
 * holding CLS rows; otherwise mean over each sequence's rows of x [T, H].
 * Replaces: pooling, Matryoshka and L2 of EncodeTokensKernel (native/model.go:417-453). */
int fh_op_pool(const float *x32, const int32_t *offsets, int32_t nseq, int32_t H, int32_t cls_compact,
               int32_t matryoshka_ln, int32_t out_dim, int32_t normalize, float *out, void *stream);

/* Which kernels a layer of the binary16 (LayerNorm-folded) forward runs for
 * M rows of a pack with this hidden width, intermediate width and
 * activation: FH_ROUTE_* bits (0 = every GEMM on the tiled kernel, or a
 * width the fold does not cover).  Host-only, no device needed.  A
 * projection leaves the persistent ring GEMM, and the layer tail the fused
 * kernel, when its rows no longer fit 32-bit buffer offsets; the tiled GEMM
 * (64-bit indices) then computes the same bits.  No reference counterpart:
 * routing diagnostics. */
#define FH_ROUTE_RING_QKV 1
#define FH_ROUTE_RING_OUT 2
#define FH_ROUTE_RING_FFN1 4
#define FH_ROUTE_RING_FC2 8
#define FH_ROUTE_MLP 16      /* out projection + FFN fused (last layer) */
#define FH_ROUTE_MLP_QKV 32  /* ... and the next layer's QKV projection */
int32_t fh_route_flags(int32_t hidden, int32_t inter, int32_t swiglu, int32_t M);

#ifdef __cplusplus
}
#endif
#endif /* FUTON_HIP_OPS_H */
