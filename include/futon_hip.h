/*
 * futon_hip.h — C ABI of the MI355X (gfx950) futon encoder forward pass.
 *
 * This is the device boundary the reference's Go host would bind through
 * cgo behind a `hip` build tag.  It replaces, for a whole batch, the body of
 *
 *   native.Model.EncodeTokensKernel   native/model.go:346-457
 *   (+ the Kernel seam it drives)     native/kernel.go:26-43, native/quant.go:92-96
 *
 * while every Go-side validation (manifest, safetensors, config, tensor
 * names/shapes) stays where it is: fh_model_create receives tensors the
 * host already validated, and fh_encode receives token ids the host
 * tokenizer (native/tokenizer.go:146-176) produced.
 *
 * Conventions: plain C types, row-major tensors, no ownership transfer.
 * Every function returns FH_OK (0) or a negative FH_E* code; the thread-local
 * detail of the last failure is available from fh_last_error().
 */
#ifndef FUTON_HIP_H
#define FUTON_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define FH_OK 0
#define FH_EINVAL (-22)      /* bad argument (shape, id range, length, dims) */
#define FH_ENOMEM (-12)      /* device or host allocation failed */
#define FH_EHIP (-5)         /* HIP runtime error */
#define FH_ECANCELED (-125)  /* cancel flag observed at a checkpoint */
#define FH_ETOOLONG (-36)    /* sequence longer than the effective max_seq_len */
#define FH_ENODEV (-19)      /* no usable gfx950 device */

/* Option values (native/config.go:14-30). */
#define FH_POS_ABSOLUTE 0
#define FH_POS_ROPE 1
#define FH_ACT_GELU 0
#define FH_ACT_SWIGLU 1
#define FH_POOL_MEAN 0
#define FH_POOL_CLS 1

/* Tensor element types of a pack (native/safetensors.go:31-34). */
#define FH_DTYPE_F32 0
#define FH_DTYPE_F16 1

/* Architecture description; mirrors native.PackConfig (native/config.go:54-102)
 * plus the load-time switches the reference reads from the environment. */
typedef struct fh_config {
    int32_t hidden_size;
    int32_t num_layers;
    int32_t num_heads;
    int32_t intermediate_size;
    int32_t vocab_size;
    int32_t type_vocab_size;       /* 0 = no token-type table */
    int32_t max_seq_len;
    int32_t max_trained_positions; /* 0 = unset; clamps max_seq_len (config.go:111-116) */
    double layer_norm_eps;
    int32_t position_encoding;     /* FH_POS_* */
    double rope_theta;
    int32_t activation;            /* FH_ACT_* */
    int32_t pooling;               /* FH_POOL_* */
    int32_t normalize;             /* L2-normalize the pooled vector */
    int32_t matryoshka;            /* pack declares Matryoshka support */
    int32_t matryoshka_layernorm;  /* parameter-free LN (eps 1e-5) before truncation */
    int32_t q8;                    /* FUTON_NATIVE_Q8=1: int8 per-row layer weights (quant.go:30) */
} fh_config;

/* One named tensor in host memory (canonical pack names, model.go:189-256). */
typedef struct fh_tensor {
    const char *name;
    int32_t dtype;     /* FH_DTYPE_* */
    int32_t rank;
    int64_t shape[4];
    const void *data;  /* host pointer, row-major, valid for the duration of the call */
} fh_tensor;

typedef struct fh_model fh_model;

/* Uploads a validated pack to `device` (weights converted once: GEMM weights
 * to fp16, or to int8 + per-row scales when cfg->q8; norms/biases/tables to
 * f32; RoPE tables computed in float64 exactly as native/model.go:306-318).
 * Checks the tensor-name set and every shape like newModel
 * (native/model.go:134-263): a missing, misshapen or unexpected tensor is
 * FH_EINVAL.  Host tensors may be freed when this returns.
 * Replaces: native.newModel (native/model.go:134-295). */
int fh_model_create(const fh_config *cfg, const fh_tensor *tensors, int32_t n_tensors,
                    int32_t device, fh_model **out);

/* Releases the model's device memory.  NULL is a no-op.
 * Replaces: Provider.Close's release of the weights (native/provider.go:276-281). */
void fh_model_destroy(fh_model *m);

/* Encodes a packed batch: sequence i is ids[seq_offsets[i] .. seq_offsets[i+1]),
 * already wrapped in [CLS] … [SEP] (no padding ids).  Writes nseq × out_dim
 * floats to out (out_dim 0 = hidden_size).  Each vector equals an independent
 * unpadded forward of its sequence, independent of the rest of the batch.
 * `cancel` (may be NULL) is polled at the reference's checkpoints — before
 * each layer and between attention and FFN (model.go:400, :603); a non-zero
 * value aborts with FH_ECANCELED and out untouched.
 * Validation (same rules and order as model.go:348-365): empty sequence or
 * out_dim/id out of range → FH_EINVAL, too long → FH_ETOOLONG.
 * Safe to call concurrently on one model (calls are serialized per model).
 * Replaces: native.Model.EncodeTokensKernel (native/model.go:346-457), once
 * per sequence, as driven by Provider.EmbedBatch (native/provider.go:152-202). */
int fh_encode(fh_model *m, const int32_t *ids, const int32_t *seq_offsets, int32_t nseq,
              int32_t out_dim, float *out, const volatile int32_t *cancel);

/* fh_encode on device-resident inputs: d_ids, d_offsets and d_out are device
 * pointers; total_tokens and max_len describe the batch (the host keeps
 * them while the ids live on the device).  Enqueued on `stream` (a
 * hipStream_t; NULL = the model's own stream) and NOT synchronized.  The
 * caller guarantees the ids were validated.  h_offsets (nullable) is a host
 * copy of d_offsets, for the profiler's FLOP accounting and the attention
 * split: when it shows a longest-first batch that mixes sequences of at most
 * 128 tokens with longer ones, each class runs its own attention path, so
 * every vector equals its single-sequence forward (as fh_encode, which sorts
 * the batch itself, always does); otherwise one attention launch sized by
 * max_len serves the whole batch.  For throughput harnesses whose inputs
 * already reside in HBM.
 * Replaces: the same as fh_encode. */
int fh_encode_device(fh_model *m, const int32_t *d_ids, const int32_t *d_offsets, int32_t nseq,
                     int32_t total_tokens, int32_t max_len, int32_t out_dim, float *d_out,
                     void *stream, const int32_t *h_offsets);

/* fh_encode_device without any device allocation: the same forward, same
 * bits, with its workspace in a fixed scratch array that each device holds
 * from model creation until the process ends (fh_noalloc_scratch_bytes,
 * 64 MiB: ≈ 6.6k tokens of a hidden-384 pack, ≈ 3.3k of hidden 768).  A
 * batch whose workspace exceeds it is FH_EINVAL and nothing runs.  Calls no
 * hipMalloc/hipFree and creates nothing (not profiled).  Every call on a
 * device shares that device's array: calls are queued behind the previous
 * call that used it (an event, whatever the stream or model), so they never
 * overlap on the GPU; a caller must not expect two such calls to run
 * concurrently.  No counterpart in the reference: for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). */
int fh_encode_device_noalloc(fh_model *m, const int32_t *d_ids, const int32_t *d_offsets, int32_t nseq,
                             int32_t total_tokens, int32_t max_len, int32_t out_dim, float *d_out,
                             void *stream, const int32_t *h_offsets);
int64_t fh_noalloc_scratch_bytes(void);

/* Per-kernel-class timing with HIP events around every launch of
 * fh_encode_device (off by default).  fh_profile_read copies up to `cap`
 * entries: names (static strings), total milliseconds, launch counts, and
 * algorithmic FLOPs / bytes summed over those launches; returns the number
 * of classes.  fh_profile_reset clears the totals.  No reference
 * counterpart: measurement support. */
int fh_profile_enable(fh_model *m, int32_t on);
int fh_profile_reset(fh_model *m);
int fh_profile_read(fh_model *m, const char **names, double *ms, int64_t *launches, double *flops,
                    double *bytes, int32_t cap);

/* Test hook: the n-th checkpoint (0-based) of every later fh_encode sees a
 * cancellation, n < 0 disables.  Mirrors the reference's cancelAfterN
 * context (native/model_test.go:203-214). */
int fh_debug_cancel_after(fh_model *m, int32_t n);

/* Number of cancellation checkpoints one fh_encode call passes. */
int fh_checkpoints_per_call(const fh_model *m);

/* Static description of an FH_* code. */
const char *fh_strerror(int code);

/* Copies the calling thread's last error detail into buf (NUL-terminated);
 * returns its full length. */
int fh_last_error(char *buf, size_t len);

/* Device memory currently held by the model (weights + workspace), bytes. */
int64_t fh_model_device_bytes(const fh_model *m);

#ifdef __cplusplus
}
#endif
#endif /* FUTON_HIP_H */
