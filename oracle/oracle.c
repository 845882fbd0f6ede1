/*
 * CPU oracle for the futon encoder forward pass — TEST INFRASTRUCTURE ONLY.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * it, to compare against; the product never does.
 *
 * Restates, in C, the reference's Go forward (native/model.go), its float32
 * transcendentals (native/mathf32.go), the amd64 AVX2 GEMM's per-element
 * order (native/kernel_avx2_amd64.go + .s) and the Q8 scheme
 * (native/quant.go).  Built with -ffp-contract=off so that, like Go on amd64,
 * no a*b+c is fused except where fmaf() is written (the VFMADD231PS lanes).
 */
#include "oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ── native/mathf32.go:22-35 ─────────────────────────────────────────────── */
#define EXP_OVERFLOW_F32 88.72283f
#define EXP_UNDERFLOW_F32 -87.33654f
#define EXP_CLAMP_LO -104.0f
#define LOG2E_F32 ((float)1.4426950408889634)
#define LN2_HI_F32 0.693145751953125f
#define LN2_LO_F32 1.428606820309417e-06f
#define ROUND_MAGIC_F32 12582912.0f

static float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

/* native/mathf32.go:40-68 — Cephes single-precision exp with the
 * reference's range reduction and two-step 2^k scaling. */
float fo_exp_f32(float x) {
    if (x < EXP_UNDERFLOW_F32) return 0.0f;
    float kf = (x * LOG2E_F32 + ROUND_MAGIC_F32) - ROUND_MAGIC_F32;
    int32_t k = (int32_t)kf;
    float r = x - kf * LN2_HI_F32;
    r -= kf * LN2_LO_F32;
    float p = 1.9875691500e-4f;
    p = p * r + 1.3981999507e-3f;
    p = p * r + 8.3334519073e-3f;
    p = p * r + 4.1665795894e-2f;
    p = p * r + 1.6666665459e-1f;
    p = p * r + 5.0000001201e-1f;
    p = (p * r + 1.0f) * r + 1.0f;
    int32_t e = k + 127;
    if (e <= 0) return 0.0f;
    if (e >= 255) return p * bits_f32((uint32_t)(e - 1) << 23) * 2.0f;
    return p * bits_f32((uint32_t)e << 23);
}

/* native/mathf32.go:73-90 — Numerical Recipes erfcc Chebyshev fit. */
float fo_erfc_pos(float a) {
    float t = 1.0f / (1.0f + 0.5f * a);
    float p = 0.17087277f;
    p = p * t - 0.82215223f;
    p = p * t + 1.48851587f;
    p = p * t - 1.13520398f;
    p = p * t + 0.27886807f;
    p = p * t - 0.18628806f;
    p = p * t + 0.09678418f;
    p = p * t + 0.37409196f;
    p = p * t + 1.00002368f;
    p = p * t - 1.26551223f;
    float e = p - a * a;
    if (e < EXP_CLAMP_LO) e = EXP_CLAMP_LO;
    return t * fo_exp_f32(e);
}

/* native/mathf32.go:96-107 — exact-erf GELU through erfc. */
float fo_gelu_f32(float x) {
    float a = x * (float)0.7071067811865476;
    if (a < 0) a = -a;
    float c = fo_erfc_pos(a);
    if (x < 0) return 0.5f * x * c;
    return 0.5f * x * (2.0f - c);
}

/* native/mathf32.go:111-120 */
float fo_sigmoid_f32(float x) {
    float e = -x;
    if (e < EXP_CLAMP_LO) e = EXP_CLAMP_LO;
    if (e > EXP_OVERFLOW_F32) return 0.0f;
    return 1.0f / (1.0f + fo_exp_f32(e));
}

/* ── native/safetensors.go:226-289 ───────────────────────────────────────── */
float fo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (uint32_t)(h >> 10) & 0x1f;
    uint32_t mant = (uint32_t)h & 0x3ff;
    if (exp == 0) {
        if (mant == 0) return bits_f32(sign);
        uint32_t e = 127 - 15 + 1;
        while ((mant & 0x400) == 0) {
            mant <<= 1;
            e--;
        }
        mant &= 0x3ff;
        return bits_f32(sign | e << 23 | mant << 13);
    }
    if (exp == 0x1f) return bits_f32(sign | 0xffu << 23 | mant << 13);
    return bits_f32(sign | (exp + 127 - 15) << 23 | mant << 13);
}

uint16_t fo_f32_to_f16(float f) {
    uint32_t b = f32_bits(f);
    uint16_t sign = (uint16_t)(b >> 16) & 0x8000;
    int32_t exp32 = (int32_t)(b >> 23 & 0xff);
    uint32_t mant = b & 0x7fffff;
    int32_t exp = exp32 - 127 + 15;
    if (exp32 == 0xff) return mant ? (sign | 0x7e00) : (sign | 0x7c00);
    if (exp >= 0x1f) return sign | 0x7c00;
    if (exp <= 0) {
        if (exp < -10) return sign;
        mant |= 0x800000;
        uint32_t shift = (uint32_t)(14 - exp);
        uint32_t half = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (half & 1))) half++;
        return sign | (uint16_t)half;
    }
    uint16_t half = (uint16_t)((uint32_t)exp << 10 | (mant >> 13));
    uint32_t rem = mant & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (half & 1))) half++;
    return sign | half;
}

/* ── native/quant.go:42-70 ───────────────────────────────────────────────── */
float fo_quantize_row_q8(int8_t *dst, const float *src, int n) {
    float amax = 0.0f;
    for (int i = 0; i < n; i++) {
        float v = src[i];
        if (v < 0) v = -v;
        if (v > amax) amax = v;
    }
    if (amax == 0.0f) {
        memset(dst, 0, (size_t)n);
        return 0.0f;
    }
    float scale = amax / 127.0f;
    double inv = 127.0 / (double)amax;
    for (int i = 0; i < n; i++) {
        double q = round((double)src[i] * inv); /* math.Round: half away from zero */
        if (q > 127) q = 127;
        else if (q < -127) q = -127;
        dst[i] = (int8_t)q;
    }
    return scale;
}

/* ── GEMM: native/kernel_avx2_amd64.go:47-90 + kernel_avx2_amd64.s:78-93 ──
 * Per output element: 8 FMA lanes over k8 = k&~7 (VFMADD231PS), the fixed
 * REDUCE1 fold ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)) (.s:20-25), then the
 * unfused scalar k-tail, then the bias.  Computed as the reference's 4×2
 * panel so the oracle also serves as a fast-enough CPU baseline. */
static inline float reduce8(const float *l) {
    float v0 = l[0] + l[4], v1 = l[1] + l[5], v2 = l[2] + l[6], v3 = l[3] + l[7];
    return (v0 + v1) + (v2 + v3);
}

/* Threads one GEMM splits its 4-row panels over (each output element is
 * still computed whole by one thread, in the order above): 1 inside
 * fo_encode_batch's per-sequence workers, all of them when a batch has fewer
 * sequences than threads (the reference's parallelTiles, kernel.go:106-127,
 * splits one GEMM the same way without changing any element's order). */
static int inner_threads = 1;

void fo_matmul_t(float *dst, const float *a, const float *b, int m, int n, int k,
                 const float *bias) {
    const int k8 = k & ~7;
#pragma omp parallel for schedule(static) num_threads(inner_threads) if (inner_threads > 1 && m >= 32)
    for (int i = 0; i < m; i += 4) {
        const int rows = (m - i) < 4 ? (m - i) : 4;
        const float *ar[4];
        for (int r = 0; r < 4; r++) ar[r] = a + (size_t)((i + r) < m ? (i + r) : (m - 1)) * k;
        for (int j = 0; j < n; j += 2) {
            const int j1 = (j + 1 < n) ? j + 1 : j;
            const float *b0 = b + (size_t)j * k, *b1 = b + (size_t)j1 * k;
            float acc[4][2][8];
            memset(acc, 0, sizeof acc);
            for (int p = 0; p < k8; p += 8) {
                for (int r = 0; r < 4; r++) {
                    for (int l = 0; l < 8; l++) {
                        acc[r][0][l] = fmaf(ar[r][p + l], b0[p + l], acc[r][0][l]);
                        acc[r][1][l] = fmaf(ar[r][p + l], b1[p + l], acc[r][1][l]);
                    }
                }
            }
            for (int r = 0; r < rows; r++) {
                float s0 = reduce8(acc[r][0]), s1 = reduce8(acc[r][1]);
                for (int p = k8; p < k; p++) {
                    s0 += ar[r][p] * b0[p];
                    s1 += ar[r][p] * b1[p];
                }
                if (bias) {
                    s0 += bias[j];
                    s1 += bias[j1];
                }
                dst[(size_t)(i + r) * n + j] = s0;
                if (j1 != j) dst[(size_t)(i + r) * n + j1] = s1;
            }
        }
    }
}

/* native/kernel_avx2_amd64.go:92-135: identical order with the weight read
 * through the exact binary16 conversion (VCVTPH2PS). */
void fo_matmul_t_f16(float *dst, const float *a, const uint16_t *b, int m, int n, int k,
                     const float *bias) {
    float *bf = (float *)malloc((size_t)n * k * sizeof(float));
    for (size_t i = 0; i < (size_t)n * k; i++) bf[i] = fo_f16_to_f32(b[i]);
    fo_matmul_t(dst, a, bf, m, n, k, bias);
    free(bf);
}

/* native/quant.go:99-137: per-row dynamic activation quantization, exact
 * int32 dot, one float32 rescale float32(sum)*(sA*scale[j]) (+bias). */
void fo_matmul_t_q8(float *dst, const float *a, const int8_t *qb, const float *scales,
                    int m, int n, int k, const float *bias) {
    int8_t *qa = (int8_t *)malloc((size_t)m * k);
    float *as = (float *)malloc((size_t)m * sizeof(float));
    for (int i = 0; i < m; i++) as[i] = fo_quantize_row_q8(qa + (size_t)i * k, a + (size_t)i * k, k);
    for (int i = 0; i < m; i++) {
        const int8_t *ai = qa + (size_t)i * k;
        for (int j = 0; j < n; j++) {
            const int8_t *bj = qb + (size_t)j * k;
            int32_t sum = 0;
            for (int p = 0; p < k; p++) sum += (int32_t)ai[p] * (int32_t)bj[p];
            float s = (float)sum * (as[i] * scales[j]);
            if (bias) s += bias[j];
            dst[(size_t)i * n + j] = s;
        }
    }
    free(qa);
    free(as);
}

/* ── native/model.go:717-739 ─────────────────────────────────────────────── */
void fo_softmax_scaled(float *row, int n, float scale) {
    float maxv = row[0];
    for (int i = 1; i < n; i++)
        if (row[i] > maxv) maxv = row[i];
    maxv *= scale;
    double sum = 0.0;
    for (int i = 0; i < n; i++) {
        float d = row[i] * scale - maxv;
        if (d < EXP_CLAMP_LO) d = EXP_CLAMP_LO;
        float e = fo_exp_f32(d);
        row[i] = e;
        sum += (double)e;
    }
    float inv = (float)(1.0 / sum);
    for (int i = 0; i < n; i++) row[i] *= inv;
}

/* ── native/model.go:743-769: float64 two-pass statistics ─────────────────── */
void fo_layer_norm_rows(float *x, int rows, int h, const float *weight, const float *bias,
                        float eps) {
    for (int r = 0; r < rows; r++) {
        float *row = x + (size_t)r * h;
        double mean = 0.0;
        for (int i = 0; i < h; i++) mean += (double)row[i];
        mean /= (double)h;
        double var = 0.0;
        for (int i = 0; i < h; i++) {
            double d = (double)row[i] - mean;
            var += d * d;
        }
        var /= (double)h;
        float inv = (float)(1.0 / sqrt(var + (double)eps));
        float mf = (float)mean;
        if (weight) {
            for (int i = 0; i < h; i++) row[i] = (row[i] - mf) * inv * weight[i] + bias[i];
        } else {
            for (int i = 0; i < h; i++) row[i] = (row[i] - mf) * inv;
        }
    }
}

/* ── Model container: native/model.go:24-103, 134-295 ─────────────────────── */
typedef struct {
    float *w;    /* float storage (f16 packs converted exactly at load) */
    int8_t *q8;  /* Q8 codes when cfg.q8 (native/model.go:269-289) */
    float *q8s;  /* per-row scales */
} fo_mat;

typedef struct {
    fo_mat qkv, out, fc1, gate, fc2;
    float *qkv_b, *out_b, *fc1_b, *gate_b, *fc2_b;
    float *n1w, *n1b, *n2w, *n2b;
} fo_layer;

struct fo_model {
    fo_config cfg;
    int hd;
    float *word, *pos, *type, *emb_w, *emb_b;
    fo_layer *layers;
    float *rope_cos, *rope_sin;
    int rope_len;
    void **owned;
    int nowned;
};

static void *own(fo_model *m, void *p) {
    m->owned = (void **)realloc(m->owned, sizeof(void *) * (size_t)(m->nowned + 1));
    m->owned[m->nowned++] = p;
    return p;
}

typedef struct {
    int n;
    const char *const *names;
    const void *const *data;
    const int *dtypes;
    const int64_t *numel;
    char *used;
} tensor_set;

static int find_tensor(const tensor_set *ts, const char *name) {
    for (int i = 0; i < ts->n; i++)
        if (strcmp(ts->names[i], name) == 0) return i;
    return -1;
}

/* need/opt (native/model.go:143-184): f16 converted exactly to float32. */
static float *take(fo_model *m, tensor_set *ts, const char *name, int64_t numel, int required,
                   char *err, int errlen, int *fail) {
    int i = find_tensor(ts, name);
    if (i < 0) {
        if (required) {
            snprintf(err, (size_t)errlen, "pack %s: missing tensor \"%s\"", "oracle", name);
            *fail = 1;
        }
        return NULL;
    }
    ts->used[i] = 1;
    if (ts->numel[i] != numel) {
        snprintf(err, (size_t)errlen, "tensor \"%s\" has %lld elements, want %lld", name,
                 (long long)ts->numel[i], (long long)numel);
        *fail = 1;
        return NULL;
    }
    float *out = (float *)own(m, malloc((size_t)numel * sizeof(float)));
    if (ts->dtypes[i] == FO_F16) {
        const uint16_t *src = (const uint16_t *)ts->data[i];
        for (int64_t e = 0; e < numel; e++) out[e] = fo_f16_to_f32(src[e]);
    } else {
        memcpy(out, ts->data[i], (size_t)numel * sizeof(float));
    }
    return out;
}

static void quantize_mat(fo_model *m, fo_mat *w, int n, int k) {
    if (!w->w) return;
    w->q8 = (int8_t *)own(m, malloc((size_t)n * k));
    w->q8s = (float *)own(m, malloc((size_t)n * sizeof(float)));
    for (int j = 0; j < n; j++)
        w->q8s[j] = fo_quantize_row_q8(w->q8 + (size_t)j * k, w->w + (size_t)j * k, k);
    w->w = NULL; /* float storage dropped, as native/model.go:286 */
}

fo_model *fo_model_create(const fo_config *cfg, int ntensors, const char *const *names,
                          const void *const *data, const int *dtypes, const int64_t *numel,
                          char *err, int errlen) {
    fo_model *m = (fo_model *)calloc(1, sizeof *m);
    m->cfg = *cfg;
    m->hd = cfg->hidden / cfg->heads;
    const int64_t h = cfg->hidden, I = cfg->inter;
    tensor_set ts = {ntensors, names, data, dtypes, numel, (char *)calloc((size_t)ntensors + 1, 1)};
    int fail = 0;
    char nm[128];

    m->word = take(m, &ts, "embeddings.word", (int64_t)cfg->vocab * h, 1, err, errlen, &fail);
    if (!cfg->rope)
        m->pos = take(m, &ts, "embeddings.position", (int64_t)cfg->max_seq_len * h, 1, err, errlen, &fail);
    if (cfg->type_vocab > 0)
        m->type = take(m, &ts, "embeddings.token_type", (int64_t)cfg->type_vocab * h, 1, err, errlen, &fail);
    m->emb_w = take(m, &ts, "embeddings.norm.weight", h, 1, err, errlen, &fail);
    m->emb_b = take(m, &ts, "embeddings.norm.bias", h, 1, err, errlen, &fail);
    m->layers = (fo_layer *)own(m, calloc((size_t)cfg->layers, sizeof(fo_layer)));
    for (int li = 0; li < cfg->layers && !fail; li++) {
        fo_layer *L = &m->layers[li];
#define T(field, suffix, cnt, req)                                   \
    snprintf(nm, sizeof nm, "layers.%d.%s", li, suffix);             \
    field = take(m, &ts, nm, cnt, req, err, errlen, &fail);
        T(L->qkv.w, "attn.qkv.weight", 3 * h * h, 1)
        T(L->qkv_b, "attn.qkv.bias", 3 * h, 0)
        T(L->out.w, "attn.out.weight", h * h, 1)
        T(L->out_b, "attn.out.bias", h, 0)
        T(L->n1w, "norm1.weight", h, 1)
        T(L->n1b, "norm1.bias", h, 1)
        T(L->fc1.w, "mlp.fc1.weight", I * h, 1)
        T(L->fc1_b, "mlp.fc1.bias", I, 0)
        if (cfg->swiglu) {
            T(L->gate.w, "mlp.gate.weight", I * h, 1)
            T(L->gate_b, "mlp.gate.bias", I, 0)
        }
        T(L->fc2.w, "mlp.fc2.weight", h * I, 1)
        T(L->fc2_b, "mlp.fc2.bias", h, 0)
        T(L->n2w, "norm2.weight", h, 1)
        T(L->n2b, "norm2.bias", h, 1)
#undef T
    }
    for (int i = 0; i < ntensors && !fail; i++) {
        if (!ts.used[i]) {
            snprintf(err, (size_t)errlen, "unexpected tensor \"%s\" (pack/config mismatch)", names[i]);
            fail = 1;
        }
    }
    free(ts.used);
    if (fail) {
        fo_model_destroy(m);
        return NULL;
    }
    if (cfg->q8) {
        for (int li = 0; li < cfg->layers; li++) {
            fo_layer *L = &m->layers[li];
            quantize_mat(m, &L->qkv, 3 * (int)h, (int)h);
            quantize_mat(m, &L->out, (int)h, (int)h);
            quantize_mat(m, &L->fc1, (int)I, (int)h);
            quantize_mat(m, &L->gate, (int)I, (int)h);
            quantize_mat(m, &L->fc2, (int)h, (int)I);
        }
    }
    if (cfg->rope) {
        /* native/model.go:306-318: float64 angles, float32 tables. */
        int eff = (cfg->max_trained > 0 && cfg->max_trained < cfg->max_seq_len) ? cfg->max_trained
                                                                                 : cfg->max_seq_len;
        int half = m->hd / 2;
        m->rope_len = eff;
        m->rope_cos = (float *)own(m, malloc((size_t)eff * half * sizeof(float)));
        m->rope_sin = (float *)own(m, malloc((size_t)eff * half * sizeof(float)));
        for (int t = 0; t < eff; t++) {
            for (int i = 0; i < half; i++) {
                double freq = 1.0 / pow(cfg->rope_theta, (double)(2 * i) / (double)m->hd);
                double angle = (double)t * freq;
                m->rope_cos[t * half + i] = (float)cos(angle);
                m->rope_sin[t * half + i] = (float)sin(angle);
            }
        }
    }
    return m;
}

void fo_model_destroy(fo_model *m) {
    if (!m) return;
    for (int i = 0; i < m->nowned; i++) free(m->owned[i]);
    free(m->owned);
    free(m);
}

/* mmT (native/model.go:74-88). */
static void mmt(float *dst, const float *a, const fo_mat *w, int rows, int n, int k,
                const float *bias) {
    if (w->q8) fo_matmul_t_q8(dst, a, w->q8, w->q8s, rows, n, k, bias);
    else fo_matmul_t(dst, a, w->w, rows, n, k, bias);
}

/* native/model.go:705-712 */
static void rotate_half(float *x, const float *c, const float *s, int half) {
    for (int i = 0; i < half; i++) {
        float x1 = x[i], x2 = x[i + half];
        x[i] = x1 * c[i] - x2 * s[i];
        x[i + half] = x2 * c[i] + x1 * s[i];
    }
}

typedef struct {
    float *x, *pooled, *qkv, *attn_cat, *attn_out, *ffn_h, *ffn_gate, *ffn_out;
    float *q, *k, *vT, *scores, *head_out;
} scratch;

static int eff_max(const fo_config *c) {
    return (c->max_trained > 0 && c->max_trained < c->max_seq_len) ? c->max_trained : c->max_seq_len;
}

/* attendHead, native/model.go:646-701 (serial over heads). */
static void attend_head(const fo_model *m, scratch *s, int head, int seq, int rows) {
    const int h = m->cfg.hidden, hd = m->hd, half = hd / 2;
    const float scale = (float)(1.0 / sqrt((double)hd));
    const int kp = (seq + 7) & ~7;
    memset(s->k, 0, (size_t)kp * hd * sizeof(float));
    memset(s->vT, 0, (size_t)hd * kp * sizeof(float));
    const int qo = head * hd, ko = h + head * hd, vo = 2 * h + head * hd;
    for (int t = 0; t < seq; t++) {
        const float *row = s->qkv + (size_t)t * 3 * h;
        if (t < rows) memcpy(s->q + (size_t)t * hd, row + qo, (size_t)hd * sizeof(float));
        memcpy(s->k + (size_t)t * hd, row + ko, (size_t)hd * sizeof(float));
        for (int d = 0; d < hd; d++) s->vT[(size_t)d * kp + t] = row[vo + d];
    }
    if (m->cfg.rope) {
        for (int t = 0; t < seq; t++) {
            const float *c = m->rope_cos + (size_t)t * half, *sn = m->rope_sin + (size_t)t * half;
            if (t < rows) rotate_half(s->q + (size_t)t * hd, c, sn, half);
            rotate_half(s->k + (size_t)t * hd, c, sn, half);
        }
    }
    fo_matmul_t(s->scores, s->q, s->k, rows, kp, hd, NULL);
    for (int t = 0; t < rows; t++) {
        float *row = s->scores + (size_t)t * kp;
        fo_softmax_scaled(row, seq, scale);
        memset(row + seq, 0, (size_t)(kp - seq) * sizeof(float));
    }
    fo_matmul_t(s->head_out, s->scores, s->vT, rows, hd, kp, NULL);
    for (int t = 0; t < rows; t++)
        memcpy(s->attn_cat + (size_t)t * h + head * hd, s->head_out + (size_t)t * hd,
               (size_t)hd * sizeof(float));
}

/* layerForward, native/model.go:550-635. */
static void layer_forward(const fo_model *m, const fo_layer *L, scratch *s, int seq, int rows) {
    const fo_config *c = &m->cfg;
    const int h = c->hidden, I = c->inter;
    const float eps = (float)c->eps;
    mmt(s->qkv, s->x, &L->qkv, seq, 3 * h, h, L->qkv_b);
    for (int head = 0; head < c->heads; head++) attend_head(m, s, head, seq, rows);
    mmt(s->attn_out, s->attn_cat, &L->out, rows, h, h, L->out_b);
    for (int i = 0; i < rows * h; i++) s->attn_out[i] += s->x[i];
    memcpy(s->x, s->attn_out, (size_t)rows * h * sizeof(float));
    fo_layer_norm_rows(s->x, rows, h, L->n1w, L->n1b, eps);
    if (!c->swiglu) {
        mmt(s->ffn_h, s->x, &L->fc1, rows, I, h, L->fc1_b);
        for (size_t i = 0; i < (size_t)rows * I; i++) s->ffn_h[i] = fo_gelu_f32(s->ffn_h[i]);
    } else {
        mmt(s->ffn_h, s->x, &L->fc1, rows, I, h, L->fc1_b);
        mmt(s->ffn_gate, s->x, &L->gate, rows, I, h, L->gate_b);
        for (size_t i = 0; i < (size_t)rows * I; i++) {
            float g = s->ffn_gate[i];
            s->ffn_h[i] *= g * fo_sigmoid_f32(g);
        }
    }
    mmt(s->ffn_out, s->ffn_h, &L->fc2, rows, h, I, L->fc2_b);
    for (int i = 0; i < rows * h; i++) s->ffn_out[i] += s->x[i];
    memcpy(s->x, s->ffn_out, (size_t)rows * h * sizeof(float));
    fo_layer_norm_rows(s->x, rows, h, L->n2w, L->n2b, eps);
}

/* EncodeTokensKernel, native/model.go:346-457. */
int fo_encode(const fo_model *m, const int32_t *ids, int len, int out_dim, float *out,
              char *err, int errlen) {
    const fo_config *c = &m->cfg;
    if (len == 0) {
        snprintf(err, (size_t)errlen, "native: empty token sequence");
        return -1;
    }
    if (len > eff_max(c)) {
        snprintf(err, (size_t)errlen,
                 "native: sequence length %d exceeds effective max_seq_len %d (declared %d, trained %d)",
                 len, eff_max(c), c->max_seq_len, c->max_trained);
        return -1;
    }
    if (out_dim < 0 || out_dim > c->hidden) {
        snprintf(err, (size_t)errlen, "native: requested dim %d outside [1,%d]", out_dim, c->hidden);
        return -1;
    }
    if (out_dim != 0 && out_dim != c->hidden && !c->matryoshka) {
        snprintf(err, (size_t)errlen, "native: pack does not support matryoshka truncation to %d", out_dim);
        return -1;
    }
    for (int t = 0; t < len; t++) {
        if (ids[t] < 0 || ids[t] >= c->vocab) {
            snprintf(err, (size_t)errlen, "native: token id %d outside vocab of %d", ids[t], c->vocab);
            return -1;
        }
    }
    const int seq = len, h = c->hidden, I = c->inter, hd = m->hd, kp = (seq + 7) & ~7;
    scratch s;
    float *block = (float *)malloc(sizeof(float) *
                                   ((size_t)seq * h * 4 + (size_t)h + (size_t)seq * 3 * h +
                                    (size_t)seq * I * 2 + (size_t)seq * hd * 2 + (size_t)kp * hd * 2 +
                                    (size_t)seq * kp));
    float *p = block;
#define CARVE(f, cnt) s.f = p; p += (cnt);
    CARVE(x, (size_t)seq * h)
    CARVE(pooled, (size_t)h)
    CARVE(qkv, (size_t)seq * 3 * h)
    CARVE(attn_cat, (size_t)seq * h)
    CARVE(attn_out, (size_t)seq * h)
    CARVE(ffn_h, (size_t)seq * I)
    CARVE(ffn_gate, (size_t)seq * I)
    CARVE(ffn_out, (size_t)seq * h)
    CARVE(q, (size_t)seq * hd)
    CARVE(head_out, (size_t)seq * hd)
    CARVE(k, (size_t)kp * hd)
    CARVE(vT, (size_t)kp * hd)
    CARVE(scores, (size_t)seq * kp)
#undef CARVE

    /* Embeddings (native/model.go:384-396). */
    for (int t = 0; t < seq; t++) {
        float *row = s.x + (size_t)t * h;
        memcpy(row, m->word + (size_t)ids[t] * h, (size_t)h * sizeof(float));
        if (m->type)
            for (int i = 0; i < h; i++) row[i] += m->type[i];
        if (m->pos)
            for (int i = 0; i < h; i++) row[i] += m->pos[(size_t)t * h + i];
    }
    fo_layer_norm_rows(s.x, seq, h, m->emb_w, m->emb_b, (float)c->eps);

    /* Layers; CLS pooling computes only row 0 in the last one (:403-410). */
    for (int li = 0; li < c->layers; li++) {
        int rows = (li == c->layers - 1 && c->pool_cls) ? 1 : seq;
        layer_forward(m, &m->layers[li], &s, seq, rows);
    }

    /* Pooling (:417-430). */
    memset(s.pooled, 0, (size_t)h * sizeof(float));
    if (c->pool_cls) {
        memcpy(s.pooled, s.x, (size_t)h * sizeof(float));
    } else {
        for (int t = 0; t < seq; t++)
            for (int i = 0; i < h; i++) s.pooled[i] += s.x[(size_t)t * h + i];
        float inv = 1.0f / (float)seq;
        for (int i = 0; i < h; i++) s.pooled[i] *= inv;
    }
    int n = h;
    /* Matryoshka (:433-439): parameter-free LN, eps float32(1e-5). */
    if (out_dim != 0 && out_dim != h) {
        if (c->matryoshka_ln) fo_layer_norm_rows(s.pooled, 1, h, NULL, NULL, 1e-5f);
        n = out_dim;
    }
    /* L2 (:442-453): float64 sum of squares, skipped when zero. */
    if (c->normalize) {
        double ss = 0.0;
        for (int i = 0; i < n; i++) ss += (double)s.pooled[i] * (double)s.pooled[i];
        if (ss > 0) {
            float inv = (float)(1.0 / sqrt(ss));
            for (int i = 0; i < n; i++) s.pooled[i] *= inv;
        }
    }
    memcpy(out, s.pooled, (size_t)n * sizeof(float));
    free(block);
    return 0;
}

int fo_encode_batch(const fo_model *m, const int32_t *ids, const int32_t *offsets, int nseq,
                    int out_dim, float *out, int threads, char *err, int errlen) {
    const int od = out_dim == 0 ? m->cfg.hidden : out_dim;
    int failed = 0;
    if (threads > 1 && nseq < threads) {
        /* Fewer sequences than threads (long-context batches): one sequence
         * at a time, its GEMMs split over the threads. */
        inner_threads = threads;
        for (int i = 0; i < nseq && !failed; i++) {
            char e[256];
            if (fo_encode(m, ids + offsets[i], offsets[i + 1] - offsets[i], out_dim, out + (size_t)i * od, e,
                          sizeof e) != 0) {
                snprintf(err, (size_t)errlen, "native: batch item %d: %s", i, e);
                failed = 1;
            }
        }
        inner_threads = 1;
        return failed ? -1 : 0;
    }
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1)
    for (int i = 0; i < nseq; i++) {
        char e[256];
        if (fo_encode(m, ids + offsets[i], offsets[i + 1] - offsets[i], out_dim, out + (size_t)i * od,
                      e, sizeof e) != 0) {
#pragma omp critical
            {
                if (!failed) snprintf(err, (size_t)errlen, "native: batch item %d: %s", i, e);
                failed = 1;
            }
        }
    }
    return failed ? -1 : 0;
}
