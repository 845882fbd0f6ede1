/*
 * CPU oracle for the futon encoder forward pass — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's Go CPU path, used by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg, to compare against.
 * Nothing in the product (futon_amd/) links, loads or calls this code.
 *
 * Every function cites the reference file:line it follows.  Floating-point
 * evaluation order mirrors the Go source: the file is compiled with
 * -ffp-contract=off (Go on amd64 never fuses a*b+c), and the GEMM uses
 * explicit fmaf() exactly where the reference's AVX2 kernel issues
 * VFMADD231PS, so the lane/reduction order is the default amd64 kernel's.
 */
#ifndef FUTON_ORACLE_H
#define FUTON_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* native/mathf32.go:40-120 */
float fo_exp_f32(float x);
float fo_erfc_pos(float a);
float fo_gelu_f32(float x);
float fo_sigmoid_f32(float x);

/* native/safetensors.go:226-289 */
float fo_f16_to_f32(uint16_t h);
uint16_t fo_f32_to_f16(float f);

/* native/quant.go:42-70 */
float fo_quantize_row_q8(int8_t *dst, const float *src, int n);

/* native/kernel_avx2_amd64.go:47-135 (+ .s:78-111): dst = a·bᵀ (+bias) */
void fo_matmul_t(float *dst, const float *a, const float *b, int m, int n, int k,
                 const float *bias);
void fo_matmul_t_f16(float *dst, const float *a, const uint16_t *b, int m, int n, int k,
                     const float *bias);
/* native/quant.go:99-137 */
void fo_matmul_t_q8(float *dst, const float *a, const int8_t *qb, const float *scales,
                    int m, int n, int k, const float *bias);

/* native/model.go:717-739 */
void fo_softmax_scaled(float *row, int n, float scale);
/* native/model.go:743-769; weight/bias may be NULL (parameter-free norm) */
void fo_layer_norm_rows(float *x, int rows, int h, const float *weight, const float *bias,
                        float eps);

/* Architecture options; mirrors native/config.go:54-102. */
typedef struct {
    int hidden, layers, heads, inter, vocab, type_vocab, max_seq_len, max_trained;
    double eps;
    int rope;          /* 0 absolute, 1 rope */
    double rope_theta;
    int swiglu;        /* 0 gelu, 1 swiglu */
    int pool_cls;      /* 0 mean, 1 cls */
    int normalize;
    int matryoshka;    /* pack declares matryoshka support */
    int matryoshka_ln; /* parameter-free LN before truncation */
    int q8;            /* FUTON_NATIVE_Q8=1 load-time quantization */
} fo_config;

enum { FO_F32 = 0, FO_F16 = 1 };

typedef struct fo_model fo_model;

/* Builds a model from named tensors (canonical pack names, see
 * native/model.go:189-256).  Returns NULL and fills err on failure. */
fo_model *fo_model_create(const fo_config *cfg, int ntensors, const char *const *names,
                          const void *const *data, const int *dtypes,
                          const int64_t *numel, char *err, int errlen);
void fo_model_destroy(fo_model *m);

/* native/model.go:346-457.  Returns 0, or -1 with err filled (same
 * validation messages as the reference). */
int fo_encode(const fo_model *m, const int32_t *ids, int len, int out_dim, float *out,
              char *err, int errlen);

/* Independent forwards over a packed batch, threads workers (OpenMP), one
 * forward per worker (the reference's batchPlan at large batch sizes,
 * native/provider.go:127-140).  out is nseq × out_dim (out_dim 0 = hidden). */
int fo_encode_batch(const fo_model *m, const int32_t *ids, const int32_t *offsets,
                    int nseq, int out_dim, float *out, int threads, char *err, int errlen);

#ifdef __cplusplus
}
#endif
#endif
