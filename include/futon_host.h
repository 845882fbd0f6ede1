/*
 * futon_host.h — C ABI of the host side (pack loading, tokenizer,
 * provider) that sits above futon_hip.h, for FFI callers (Python ctypes,
 * cgo).  The C++ API with the reference's names is futon_native.hpp; every
 * function here is a thin wrapper over it.  Return values are FH_OK or a
 * negative FH_E* code (futon_hip.h), with the reference's message available
 * from fh_last_error().
 */
#ifndef FUTON_HOST_H
#define FUTON_HOST_H

#include <stddef.h>
#include <stdint.h>

#include "futon_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct fh_tokenizer fh_tokenizer;
typedef struct fh_pack fh_pack;
typedef struct fh_provider fh_provider;

/* Tokenizer options (native.TokenizerConfig, native/tokenizer.go:15-33);
 * NULL strings and 0 mean the reference's defaults. */
typedef struct fh_tokenizer_config {
    int32_t do_lower_case;
    int32_t tokenize_chinese_chars;
    int32_t max_input_chars_per_word;
    const char *cls_token, *sep_token, *unk_token, *pad_token, *mask_token;
} fh_tokenizer_config;

/* native.NewTokenizer (native/tokenizer.go:94-138). */
int fh_tokenizer_new(const char *vocab_path, const fh_tokenizer_config *cfg, fh_tokenizer **out);
/* Tokenizer.Encode (native/tokenizer.go:146-176): text[0..len) → [CLS] … [SEP]
 * ids, at most max_seq_len of them.  Writes min(n, cap) ids and stores n. */
int fh_tokenizer_encode(const fh_tokenizer *t, const char *text, size_t len, int32_t max_seq_len, int32_t *ids,
                        int32_t cap, int32_t *n_out);
int32_t fh_tokenizer_vocab_size(const fh_tokenizer *t);
void fh_tokenizer_free(fh_tokenizer *t);

/* The host half of native.LoadModel (native/model.go:112-131): manifest
 * verification, config.json, model_id agreement, strict safetensors parse,
 * tensor-name check.  No device is touched. */
int fh_pack_load(const char *dir, fh_pack **out);
/* native.LoadPackConfig (native/config.go:174-187) alone. */
int fh_pack_config_load(const char *dir, fh_config *cfg, int32_t *effective_max_seq_len);
/* The loaded pack's config, as the device config (q8 as given). */
int fh_pack_config(const fh_pack *p, int32_t q8, fh_config *cfg);
int fh_pack_model_id(const fh_pack *p, char *buf, size_t len);
int32_t fh_pack_tensor_count(const fh_pack *p);
/* newModel on the device (native/model.go:134-295) from a loaded pack. */
int fh_pack_create_model(const fh_pack *p, int32_t q8, int32_t device, fh_model **out);
void fh_pack_free(fh_pack *p);
/* native.ParseSafetensors (native/safetensors.go:106-221) over a memory
 * image, for validation only: returns the tensor count or an error. */
int fh_safetensors_check(const void *data, size_t len, int32_t *n_tensors);

/* native.New (native/provider.go:70-111): pack_dir, dimensions (0 = model
 * width), threads (kept for API parity; the forward runs on the GPU). */
int fh_provider_new(const char *pack_dir, int32_t dimensions, int32_t threads, fh_provider **out);
/* Provider.Embed (native/provider.go:115-121): out holds dimensions floats. */
int fh_provider_embed(fh_provider *p, const char *text, size_t len, float *out, const volatile int32_t *cancel);
/* Provider.EmbedBatch (native/provider.go:152-202): texts[i][0..lens[i]),
 * out is n × dimensions floats, index-aligned.  Host tokenization, then one
 * device call per token-budget chunk; the whole batch fails on the first
 * error. */
int fh_provider_embed_batch(fh_provider *p, const char *const *texts, const size_t *lens, int32_t n, float *out,
                            const volatile int32_t *cancel);
int32_t fh_provider_dimensions(const fh_provider *p);
/* Provider.ModelName (native/provider.go:251-264): "native/<model_id>". */
int fh_provider_model_name(const fh_provider *p, char *buf, size_t len);
/* Provider.IsAvailable / Close (native/provider.go:266-282); Close is idempotent. */
int32_t fh_provider_is_available(const fh_provider *p);
int fh_provider_close(fh_provider *p);
void fh_provider_free(fh_provider *p);

/* futon.New (futon.go:84-98) with local packs: model_path, or
 * models_dir/model (defaults: $FUTON_HOME/models or ~/.futon/models, and
 * bge-small-en-v1.5).  Returns a provider handle. */
int fh_futon_new(const char *model, const char *models_dir, const char *model_path, int32_t dimensions,
                 int32_t threads, fh_provider **out);

#ifdef __cplusplus
}
#endif
#endif /* FUTON_HOST_H */
