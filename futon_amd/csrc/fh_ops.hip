// Per-kernel C entry points (include/futon_hip_ops.h): argument checks,
// then the same launchers fh_encode uses.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <vector>
#include <cmath>

#include "../../include/futon_hip.h"
#include "../../include/futon_hip_ops.h"
#include "fh_common.h"

namespace {
int code_of(hipError_t e) { return e == hipSuccess ? FH_OK : FH_EHIP; }
}  // namespace

extern "C" int fh_op_gemm(int32_t dtype, const void *A, const void *B, const float *bias, const void *resid,
                          int32_t resid_f16, const float *a_scale, const float *b_scale, void *C, int32_t M,
                          int32_t N, int32_t K, int32_t act, int32_t out_f32, void *stream) {
    if (!A || !B || !C || M < 0 || N <= 0 || K <= 0) return FH_EINVAL;
    if (resid && resid_f16 && (out_f32 || act != FH_OP_ACT_NONE || dtype != FH_OP_F16)) return FH_EINVAL;
    if (N % 4 || (act == FH_OP_ACT_SWIGLU && N % 32) || act < 0 || act > 2) return FH_EINVAL;
    if (dtype == FH_OP_I8 ? (K % 16 || !a_scale || !b_scale) : (dtype != FH_OP_F16 || K % 8)) return FH_EINVAL;
    GemmArgs g{};
    g.A = A;
    g.B = B;
    g.bias = bias;
    g.resid = resid_f16 ? nullptr : (const float *)resid;
    g.resid_h = resid_f16 ? (const f16 *)resid : nullptr;
    g.a_scale = a_scale;
    g.b_scale = b_scale;
    g.C = C;
    g.M = M;
    g.N = N;
    g.K = K;
    g.lda = K;
    g.ldb = K;
    g.ldc = act == FH_OP_ACT_SWIGLU ? N / 2 : N;
    g.ldr = g.ldc;
    hipStream_t s = (hipStream_t)stream;
    return code_of(dtype == FH_OP_I8 ? fh::gemm_i8(g, act, out_f32 != 0, s) : fh::gemm_f16(g, act, out_f32 != 0, s));
}

extern "C" int fh_op_gemm_ring(const void *A, const void *B_packed, const float *bias, const void *resid,
                               int32_t resid_f16, void *C, int32_t M, int32_t N, int32_t K, int32_t act,
                               int32_t out_f32, void *stream) {
    if (!A || !B_packed || !C || M < 0 || N <= 0 || K <= 0) return FH_EINVAL;
    if (act != FH_OP_ACT_NONE && act != FH_OP_ACT_GELU && act != FH_OP_ACT_SWIGLU) return FH_EINVAL;
    if (resid && resid_f16 && (out_f32 || act != FH_OP_ACT_NONE)) return FH_EINVAL;
    if (act == FH_OP_ACT_SWIGLU && (out_f32 || resid)) return FH_EINVAL;
    if (M == 0) return FH_OK;
    GemmArgs g{};
    g.A = A;
    g.B = B_packed;
    g.bias = bias;
    g.resid = resid_f16 ? nullptr : (const float *)resid;
    g.resid_h = resid_f16 ? (const f16 *)resid : nullptr;
    g.C = C;
    g.M = M;
    g.N = N;
    g.K = K;
    g.lda = K;
    g.ldb = K;
    g.ldc = act == FH_OP_ACT_SWIGLU ? N / 2 : N;
    g.ldr = N;
    const int a = act == FH_OP_ACT_NONE && !out_f32 && g.resid_h ? fh::ACT_RES16 : act;
    if (!fh::gemm_ring_ok(g, a, out_f32 != 0, fh::LN_NONE)) return FH_EINVAL;
    return code_of(fh::gemm_ring(g, act, out_f32 != 0, (hipStream_t)stream));
}

extern "C" int fh_op_gemm_ring_q8(const void *A, const void *B_packed, const float *a_scale, const float *b_scale,
                                  const float *bias, const float *resid, float *C, int32_t M, int32_t N, int32_t K,
                                  int32_t act, void *stream) {
    if (!A || !B_packed || !a_scale || !b_scale || !C || M < 0 || N <= 0 || K <= 0) return FH_EINVAL;
    if (act != FH_OP_ACT_NONE && act != FH_OP_ACT_GELU) return FH_EINVAL;
    if (M == 0) return FH_OK;
    GemmArgs g{};
    g.A = A;
    g.B = B_packed;
    g.a_scale = a_scale;
    g.b_scale = b_scale;
    g.bias = bias;
    g.resid = resid;
    g.C = C;
    g.M = M;
    g.N = N;
    g.K = K;
    g.lda = K;
    g.ldb = K;
    g.ldc = N;
    g.ldr = N;
    if (!fh::gemm_ring_q8_ok(g, act, true)) return FH_EINVAL;
    return code_of(fh::gemm_ring_q8(g, act, true, (hipStream_t)stream));
}

extern "C" int fh_op_gemm_ln(int32_t ring, int32_t ln_mode, const void *A, const void *B, const float *c1,
                             const float *c2, const float *bias, const void *resid_h, const void *stats,
                             const float *ln_g, const float *ln_b, void *C, int32_t M, int32_t N, int32_t K,
                             int32_t act, void *stream) {
    if (!A || !B || !C || !stats || M < 0 || N <= 0 || K <= 0 || K % 64 || N % 4) return FH_EINVAL;
    GemmArgs g{};
    g.A = A;
    g.B = B;
    g.C = C;
    g.M = M;
    g.N = N;
    g.K = K;
    g.lda = K;
    g.ldb = K;
    g.ldc = N;
    g.ldr = N;
    g.stats_in = (const f32x2 *)stats;
    int a;
    if (ln_mode == fh::LN_IN) {
        if (!c1 || !c2 || act < FH_OP_ACT_NONE || act > FH_OP_ACT_SWIGLU) return FH_EINVAL;
        if (act == FH_OP_ACT_SWIGLU && N % 128) return FH_EINVAL;
        g.c1 = c1;
        g.c2 = c2;
        g.ldc = act == FH_OP_ACT_SWIGLU ? N / 2 : N;
        a = act;
    } else if (ln_mode == fh::RES_LN) {
        if (!resid_h || !ln_g || !ln_b || act != FH_OP_ACT_NONE) return FH_EINVAL;
        g.bias = bias;
        g.resid_h = (const f16 *)resid_h;
        g.ln_g = ln_g;
        g.ln_b = ln_b;
        a = fh::ACT_RES16;
    } else {
        return FH_EINVAL;
    }
    if (M == 0) return FH_OK;
    hipStream_t s = (hipStream_t)stream;
    if (ring) {
        if (!fh::gemm_ring_ok(g, a, false, ln_mode)) return FH_EINVAL;
        return code_of(fh::gemm_ring(g, a, false, s, ln_mode));
    }
    return code_of(fh::gemm_f16(g, ln_mode == fh::RES_LN ? (int)fh::ACT_NONE : a, false, s, ln_mode));
}

extern "C" int fh_op_row_stats(const void *y, int32_t M, int32_t H, float eps, void *stats, void *stream) {
    if (!y || !stats || M < 0 || (H != 256 && H != 384 && H != 512 && H != 768 && H != 1024)) return FH_EINVAL;
    return code_of(fh::row_stats((const f16 *)y, M, H, eps, (f32x2 *)stats, (hipStream_t)stream));
}

extern "C" int fh_op_ring_pack(const void *B, void *out, int32_t N, int32_t K, void *stream) {
    if (!B || !out || N <= 0 || K <= 0 || N % 64 || K % 8) return FH_EINVAL;
    return code_of(fh::ring_pack((const f16 *)B, (f16 *)out, N, K, (hipStream_t)stream));
}

extern "C" int fh_op_mlp_pack(int32_t kind, const void *B, void *out, int32_t N, int32_t K, void *stream) {
    if (!B || !out || N <= 0 || K <= 0) return FH_EINVAL;
    if (kind == 1 ? N % 16 || K % 32 : kind != 2 || N % 384 || K % 128) return FH_EINVAL;
    return code_of(fh::mlp_pack(kind, (const f16 *)B, (f16 *)out, N, K, (hipStream_t)stream));
}

extern "C" int fh_op_mlp(const void *y, const void *stats, const void *w1_packed, const float *c1, const float *c2,
                         const void *w2_packed, const float *b2, const float *ln_g, const float *ln_b, void *out,
                         void *stats_out, float eps, int32_t M, int32_t H, int32_t I, void *stream) {
    if (!y || !w1_packed || !c1 || !c2 || !w2_packed || !ln_g || !ln_b || !out || M < 0) return FH_EINVAL;
    if (M == 0) return FH_OK;
    if (!fh::mlp_ok(M, H, I)) return FH_EINVAL;
    MlpArgs g{};
    g.y = (const f16 *)y;
    g.stats = (const f32x2 *)stats;
    g.w1 = (const f16 *)w1_packed;
    g.c1 = c1;
    g.c2 = c2;
    g.w2 = (const f16 *)w2_packed;
    g.b2 = b2;
    g.ln_g = ln_g;
    g.ln_b = ln_b;
    g.out = (f16 *)out;
    g.stats_out = (f32x2 *)stats_out;
    g.eps = eps;
    g.M = M;
    g.I = I;
    return code_of(fh::mlp(g, (hipStream_t)stream));
}

extern "C" int fh_op_outproj_mlp(const void *attn, const void *wo_packed, const float *bo, const void *ya,
                                 const void *stats_a, const float *ga, const float *ba, const void *w1_packed,
                                 const float *c1, const float *c2, const void *w2_packed, const float *b2,
                                 const float *ln_g, const float *ln_b, void *out, void *stats_out, float eps,
                                 const void *wq_packed, const float *c1q, const float *c2q, void *qkv, int32_t M,
                                 int32_t H, int32_t I, void *stream) {
    if (!attn || !wo_packed || !ya || !stats_a || !ga || !ba || !w1_packed || !c1 || !c2 || !w2_packed || !ln_g ||
        !ln_b || !out || M < 0)
        return FH_EINVAL;
    if (M == 0) return FH_OK;
    if (!fh::mlp_ok(M, H, I)) return FH_EINVAL;
    MlpArgs g{};
    g.attn = (const f16 *)attn;
    g.wo = (const f16 *)wo_packed;
    g.bo = bo;
    g.ya = (const f16 *)ya;
    g.stats_a = (const f32x2 *)stats_a;
    g.ga = ga;
    g.ba = ba;
    g.w1 = (const f16 *)w1_packed;
    g.c1 = c1;
    g.c2 = c2;
    g.w2 = (const f16 *)w2_packed;
    g.b2 = b2;
    g.ln_g = ln_g;
    g.ln_b = ln_b;
    g.out = (f16 *)out;
    g.stats_out = (f32x2 *)stats_out;
    g.eps = eps;
    g.wq = (const f16 *)wq_packed;
    g.c1q = c1q;
    g.c2q = c2q;
    g.qkv = (f16 *)qkv;
    g.M = M;
    g.I = I;
    return code_of(fh::mlp(g, (hipStream_t)stream));
}

extern "C" int fh_op_attention(const void *qkv, const int32_t *offsets, int32_t nseq, int32_t max_len, int32_t H,
                               int32_t heads, const float *rope_cos, const float *rope_sin, void *out,
                               int32_t q_limit, int32_t compact, int32_t out_f32, void *stream) {
    if (!qkv || !offsets || !out || nseq < 0 || max_len <= 0 || heads <= 0 || H % heads) return FH_EINVAL;
    const int d = H / heads;
    if (d % 8 || d > 128 || (rope_cos && !rope_sin)) return FH_EINVAL;
    AttnArgs a{};
    a.qkv = (const f16 *)qkv;
    a.offsets = offsets;
    a.rope_cos = rope_cos;
    a.rope_sin = rope_sin;
    a.out = out;
    a.H = H;
    a.d = d;
    a.ldo = H;
    a.q_limit = q_limit > 0 ? q_limit : INT_MAX;
    a.compact = compact;
    a.scale_log2e = (float)(1.0 / std::sqrt((double)d)) * 1.4426950408889634f;
    return code_of(fh::attention(a, nseq, max_len, out_f32 != 0, (hipStream_t)stream));
}

extern "C" int fh_op_layer_norm(const void *y, int32_t y_f16, int32_t M, int32_t H, const float *gamma,
                                const float *beta, float eps, float *x32, void *x16, void *stream) {
    if (!y || !x32 || H <= 0 || H > 1024 || (gamma && !beta)) return FH_EINVAL;
    return code_of(fh::layer_norm(y_f16 ? nullptr : (const float *)y, y_f16 ? (const f16 *)y : nullptr, M, H, gamma,
                                  beta, eps, x32, (f16 *)x16, (hipStream_t)stream));
}

extern "C" int fh_op_quantize_rows(const float *x, int32_t M, int32_t K, int8_t *q, float *scale, void *stream) {
    if (!x || !q || !scale || K <= 0) return FH_EINVAL;
    return code_of(fh::quantize_rows(x, M, K, K, q, scale, (hipStream_t)stream));
}

extern "C" int fh_op_embed_ln(const int32_t *ids, const int32_t *offsets, int32_t nseq, int32_t max_len,
                              const float *word, const float *type0, const float *pos, const float *gamma,
                              const float *beta, float eps, int32_t H, float *x32, void *x16, void *stream) {
    if (!ids || !offsets || !word || !gamma || !beta || !x32 || !x16 || H <= 0 || H > 1024) return FH_EINVAL;
    return code_of(fh::embed_ln(ids, offsets, nseq, max_len, word, type0, pos, gamma, beta, eps, H, x32, (f16 *)x16,
                                (hipStream_t)stream));
}

extern "C" int fh_op_pool(const float *x32, const int32_t *offsets, int32_t nseq, int32_t H, int32_t cls_compact,
                          int32_t matryoshka_ln, int32_t out_dim, int32_t normalize, float *out, void *stream) {
    if (!x32 || !offsets || !out || H <= 0 || H > 1024 || H % 4 || out_dim <= 0 || out_dim > H || nseq < 0)
        return FH_EINVAL;
    if (nseq == 0) return FH_OK;
    // Mean pooling needs its segment-sum buffer: sized from the offsets (a
    // test entry point, so it reads them back and allocates here).
    std::vector<int32_t> h((size_t)nseq + 1);
    hipStream_t s = (hipStream_t)stream;
    if (hipMemcpyAsync(h.data(), offsets, h.size() * 4, hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
        return FH_EHIP;
    int max_len = 0;
    for (int i = 0; i < nseq; i++) max_len = std::max(max_len, h[(size_t)i + 1] - h[(size_t)i]);
    float *part = nullptr;
    if (!cls_compact && hipMalloc(&part, (size_t)fh::pool_part_rows(h[(size_t)nseq], nseq) * H * 4) != hipSuccess)
        return FH_ENOMEM;
    const hipError_t e = fh::pool(x32, offsets, nseq, std::max(max_len, 1), H, cls_compact, cls_compact ? 0 : 1,
                                  matryoshka_ln, out_dim, normalize, part, out, s);
    if (part) {
        hipStreamSynchronize(s);
        hipFree(part);
    }
    return code_of(e);
}
