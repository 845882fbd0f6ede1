// Provider (native/provider.go), futon.New (futon.go) and the host C ABI
// (include/futon_host.h).  EmbedBatch keeps the reference's contract —
// index-aligned results, whole-batch failure on the first error, batch
// vector == single vector — but replaces its per-text worker pool with host
// tokenization followed by one packed device call per token-budget chunk.
#include <sys/stat.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <thread>

#include "../../../include/futon_host.h"
#include "../../../include/futon_native.hpp"
#include "host_common.h"

namespace futon {
namespace native {

using fh::raise;

namespace {
// Tokens per device call; a larger batch is split into consecutive chunks
// (each sequence's vector does not depend on the chunking).
constexpr size_t kChunkTokens = 1u << 20;
}  // namespace

std::unique_ptr<Provider> Provider::New(const Options &opts) {
    if (opts.PackDir.empty()) raise(FH_EINVAL, "native: PackDir is required (no downloading in this phase)");
    auto p = std::unique_ptr<Provider>(new Provider());
    p->model_ = LoadModel(opts.PackDir, opts.Threads);
    const PackConfig &cfg = p->model_->Config();
    p->tok_ = std::make_unique<Tokenizer>(fh::join_path(opts.PackDir, "vocab.txt"), cfg.Tokenizer);
    if (p->tok_->VocabSize() > cfg.VocabSize)
        raise(FH_EINVAL, "native: vocab.txt has %d entries but pack declares vocab_size %lld", p->tok_->VocabSize(),
              (long long)cfg.VocabSize);
    int dims = opts.Dimensions;
    if (dims == 0) dims = (int)cfg.HiddenSize;
    if (dims != cfg.HiddenSize) {
        if (!cfg.Matryoshka)
            raise(FH_EINVAL, "native: pack %s does not support truncation to %d dimensions", cfg.ModelID.c_str(), dims);
        if (dims < 1 || dims > cfg.HiddenSize)
            raise(FH_EINVAL, "native: dimensions %d outside [1,%lld]", dims, (long long)cfg.HiddenSize);
    }
    p->dims_ = dims;
    int threads = opts.Threads;
    if (threads < 1) threads = (int)std::max(1u, std::thread::hardware_concurrency());
    p->threads_ = threads;
    return p;
}

void Provider::checkOpen() const {
    std::lock_guard<std::mutex> g(mu_);
    if (closed_) raise(FH_EINVAL, "native: provider is closed");
}

bool Provider::IsAvailable() const {
    std::lock_guard<std::mutex> g(mu_);
    return !closed_;
}

void Provider::Close() {
    std::lock_guard<std::mutex> g(mu_);
    closed_ = true;
}

std::string Provider::ModelName() const { return std::string(NativeModelNamePrefix) + model_->Config().ModelID; }

std::vector<float> Provider::Embed(const Context *ctx, const std::string &text) {
    checkOpen();
    const std::vector<int> ids = tok_->Encode(text, (int)model_->Config().EffectiveMaxSeqLen());
    return model_->EncodeTokens(ctx, ids, dims_);
}

std::vector<std::vector<float>> Provider::EmbedBatch(const Context *ctx, const std::vector<std::string> &texts) {
    checkOpen();
    std::vector<std::vector<float>> result;
    if (texts.empty()) return result;
    const int maxSeq = (int)model_->Config().EffectiveMaxSeqLen();
    std::vector<std::vector<int>> ids(texts.size());
    // Host tokenization on up to `threads` workers (read-only tokenizer).
    const size_t nw = std::min<size_t>((size_t)threads_, (texts.size() + 63) / 64);
    if (nw <= 1) {
        for (size_t i = 0; i < texts.size(); i++) ids[i] = tok_->Encode(texts[i], maxSeq);
    } else {
        std::vector<std::thread> pool;
        for (size_t w = 0; w < nw; w++)
            pool.emplace_back([&, w]() {
                for (size_t i = w; i < texts.size(); i += nw) ids[i] = tok_->Encode(texts[i], maxSeq);
            });
        for (auto &t : pool) t.join();
    }
    result.resize(texts.size());
    size_t i = 0;
    while (i < texts.size()) {
        size_t j = i, tokens = 0;
        std::vector<std::vector<int>> chunk;
        while (j < texts.size() && (j == i || tokens + ids[j].size() <= kChunkTokens)) {
            tokens += ids[j].size();
            chunk.push_back(std::move(ids[j]));
            j++;
        }
        if (ctx && ctx->Canceled()) raise(FH_ECANCELED, "native: batch item %zu: context canceled", i);
        std::vector<std::vector<float>> vecs;
        try {
            vecs = model_->EncodeBatch(ctx, chunk, dims_);
        } catch (const fh::Error &e) {
            if (e.code == FH_ECANCELED) raise(FH_ECANCELED, "native: batch item %zu: context canceled", i);
            raise(e.code, "native: batch item %zu: %s", i, e.what());
        }
        for (size_t k = 0; k < vecs.size(); k++) result[i + k] = std::move(vecs[k]);
        i = j;
    }
    return result;
}

}  // namespace native

std::string DefaultModelsDir() {
    if (const char *home = getenv("FUTON_HOME"); home && *home) return fh::join_path(home, "models");
    const char *h = getenv("HOME");
    if (!h || !*h) return ".futon/models";
    return fh::join_path(fh::join_path(h, ".futon"), "models");
}

namespace {

using fh::raise;

class NativeEmbedder : public Embedder {
  public:
    explicit NativeEmbedder(std::unique_ptr<native::Provider> p) : p_(std::move(p)) {}
    std::vector<float> Embed(const Context *ctx, const std::string &text) override { return p_->Embed(ctx, text); }
    std::vector<std::vector<float>> EmbedBatch(const Context *ctx, const std::vector<std::string> &texts) override {
        return p_->EmbedBatch(ctx, texts);
    }
    int Dimensions() const override { return p_->Dimensions(); }
    std::string ModelName() const override { return p_->ModelName(); }
    void Close() override { p_->Close(); }
    native::Provider &provider() { return *p_; }

  private:
    std::unique_ptr<native::Provider> p_;
};

// packs.Resolve (packs/packs.go:84-113) for an installed pack directory.
std::string resolve_pack(const std::string &modelsDir, const std::string &id) {
    if (id.empty() || id.find('/') != std::string::npos || id.find('\\') != std::string::npos || id == "." ||
        id == ".." || id[0] == '.')
        raise(FH_EINVAL, "packs: invalid pack id \"%s\"", id.c_str());
    if (modelsDir.empty()) raise(FH_EINVAL, "packs: models dir is required");
    const std::string dir = fh::join_path(modelsDir, id);
    struct stat st;
    if (stat(fh::join_path(dir, "manifest.json").c_str(), &st) != 0)
        raise(FH_EINVAL,
              "futon: packs: pack \"%s\" is not installed: install a weight-pack archive (.futonpack) with "
              "packs.Install, or load a pack directory with packs.LoadDir",
              id.c_str());
    return dir;
}

}  // namespace

std::string packDir(const Options &opts) {
    if (!opts.ModelPath.empty()) return opts.ModelPath;
    return resolve_pack(opts.ModelsDir.empty() ? DefaultModelsDir() : opts.ModelsDir,
                        opts.Model.empty() ? DefaultModel : opts.Model);
}

int threadBudget(int requested) {
    const int avail = (int)std::max(1u, std::thread::hardware_concurrency());
    if (requested < 1) requested = 6;
    return std::min(requested, avail);
}

std::unique_ptr<Embedder> New(const Options &opts) {
    native::Options no;
    no.PackDir = packDir(opts);
    no.Dimensions = opts.Dimensions;
    no.Threads = threadBudget(opts.Threads);
    return std::make_unique<NativeEmbedder>(native::Provider::New(no));
}

}  // namespace futon

// ───────────────────────────── C ABI ─────────────────────────────

using futon::native::Pack;
using futon::native::Provider;
using futon::native::Tokenizer;

struct fh_tokenizer {
    std::unique_ptr<Tokenizer> t;
};
struct fh_pack {
    Pack p;
};
struct fh_provider {
    std::unique_ptr<Provider> p;
};

namespace {

template <class F>
int guarded(F &&f) {
    try {
        return f();
    } catch (const fh::Error &e) {
        return fh::fail(e.code, "%s", e.what());
    } catch (const std::bad_alloc &) {
        return fh::fail(FH_ENOMEM, "out of host memory");
    } catch (const std::exception &e) {
        return fh::fail(FH_EINVAL, "%s", e.what());
    }
}

int copy_str(const std::string &s, char *buf, size_t len) {
    if (buf && len) {
        const size_t n = std::min(len - 1, s.size());
        memcpy(buf, s.data(), n);
        buf[n] = 0;
    }
    return (int)s.size();
}

fh_config to_device_config(const futon::native::PackConfig &c, bool q8) {
    fh_config d{};
    d.hidden_size = (int32_t)c.HiddenSize;
    d.num_layers = (int32_t)c.NumLayers;
    d.num_heads = (int32_t)c.NumHeads;
    d.intermediate_size = (int32_t)c.IntermediateSize;
    d.vocab_size = (int32_t)c.VocabSize;
    d.type_vocab_size = (int32_t)c.TypeVocabSize;
    d.max_seq_len = (int32_t)c.MaxSeqLen;
    d.max_trained_positions = (int32_t)c.MaxTrainedPositions;
    d.layer_norm_eps = c.LayerNormEps;
    d.position_encoding = c.PositionEncoding == "rope" ? FH_POS_ROPE : FH_POS_ABSOLUTE;
    d.rope_theta = c.RoPETheta;
    d.activation = c.Activation == "swiglu" ? FH_ACT_SWIGLU : FH_ACT_GELU;
    d.pooling = c.Pooling == "cls" ? FH_POOL_CLS : FH_POOL_MEAN;
    d.normalize = c.Normalize;
    d.matryoshka = c.Matryoshka.has_value();
    d.matryoshka_layernorm = c.Matryoshka && c.Matryoshka->LayerNorm;
    d.q8 = q8;
    return d;
}

}  // namespace

extern "C" int fh_tokenizer_new(const char *vocab_path, const fh_tokenizer_config *cfg, fh_tokenizer **out) {
    return guarded([&] {
        if (!vocab_path || !out) return fh::fail(FH_EINVAL, "fh_tokenizer_new: null argument");
        *out = nullptr;
        futon::native::TokenizerConfig tc;
        if (cfg) {
            tc.DoLowerCase = cfg->do_lower_case != 0;
            tc.TokenizeChineseChars = cfg->tokenize_chinese_chars != 0;
            tc.MaxInputCharsPerWord = cfg->max_input_chars_per_word;
            if (cfg->cls_token) tc.ClsToken = cfg->cls_token;
            if (cfg->sep_token) tc.SepToken = cfg->sep_token;
            if (cfg->unk_token) tc.UnkToken = cfg->unk_token;
            if (cfg->pad_token) tc.PadToken = cfg->pad_token;
            if (cfg->mask_token) tc.MaskToken = cfg->mask_token;
        }
        auto t = std::make_unique<fh_tokenizer>();
        t->t = std::make_unique<Tokenizer>(vocab_path, tc);
        *out = t.release();
        return FH_OK;
    });
}

extern "C" int fh_tokenizer_encode(const fh_tokenizer *t, const char *text, size_t len, int32_t max_seq_len,
                                   int32_t *ids, int32_t cap, int32_t *n_out) {
    return guarded([&] {
        if (!t || (!text && len) || !n_out || (cap > 0 && !ids)) return fh::fail(FH_EINVAL, "fh_tokenizer_encode: null argument");
        const std::vector<int> v = t->t->Encode(std::string(text ? text : "", len), max_seq_len);
        *n_out = (int32_t)v.size();
        for (int32_t i = 0; i < cap && i < (int32_t)v.size(); i++) ids[i] = v[(size_t)i];
        return FH_OK;
    });
}

extern "C" int32_t fh_tokenizer_vocab_size(const fh_tokenizer *t) { return t ? t->t->VocabSize() : 0; }
extern "C" void fh_tokenizer_free(fh_tokenizer *t) { delete t; }

extern "C" int fh_pack_load(const char *dir, fh_pack **out) {
    return guarded([&] {
        if (!dir || !out) return fh::fail(FH_EINVAL, "fh_pack_load: null argument");
        *out = nullptr;
        auto p = std::make_unique<fh_pack>();
        p->p = futon::native::LoadPack(dir);
        *out = p.release();
        return FH_OK;
    });
}

extern "C" int fh_pack_config_load(const char *dir, fh_config *cfg, int32_t *effective_max_seq_len) {
    return guarded([&] {
        if (!dir) return fh::fail(FH_EINVAL, "fh_pack_config_load: null argument");
        const futon::native::PackConfig c = futon::native::LoadPackConfig(dir);
        if (cfg) *cfg = to_device_config(c, false);
        if (effective_max_seq_len) *effective_max_seq_len = (int32_t)c.EffectiveMaxSeqLen();
        return FH_OK;
    });
}

extern "C" int fh_pack_config(const fh_pack *p, int32_t q8, fh_config *cfg) {
    if (!p || !cfg) return fh::fail(FH_EINVAL, "fh_pack_config: null argument");
    *cfg = to_device_config(p->p.Config, q8 != 0);
    return FH_OK;
}

extern "C" int fh_pack_model_id(const fh_pack *p, char *buf, size_t len) {
    return p ? copy_str(p->p.Config.ModelID, buf, len) : fh::fail(FH_EINVAL, "fh_pack_model_id: null pack");
}

extern "C" int32_t fh_pack_tensor_count(const fh_pack *p) { return p ? (int32_t)p->p.Tensors.size() : 0; }

extern "C" int fh_pack_create_model(const fh_pack *p, int32_t q8, int32_t device, fh_model **out) {
    return guarded([&] {
        if (!p || !out) return fh::fail(FH_EINVAL, "fh_pack_create_model: null argument");
        *out = nullptr;
        const fh_config dc = to_device_config(p->p.Config, q8 != 0);
        std::vector<fh_tensor> ts;
        for (const auto &kv : p->p.Tensors) {
            const futon::native::Tensor &t = kv.second;
            if (t.Shape.size() > 4) return fh::fail(FH_EINVAL, "pack: tensor \"%s\" has rank %zu", t.Name.c_str(), t.Shape.size());
            fh_tensor d{};
            d.name = t.Name.c_str();
            d.rank = (int32_t)t.Shape.size();
            for (size_t i = 0; i < t.Shape.size(); i++) d.shape[i] = t.Shape[i];
            d.dtype = t.F16.empty() ? FH_DTYPE_F32 : FH_DTYPE_F16;
            d.data = t.F16.empty() ? (const void *)t.Data.data() : (const void *)t.F16.data();
            ts.push_back(d);
        }
        return fh_model_create(&dc, ts.data(), (int32_t)ts.size(), device, out);
    });
}

extern "C" void fh_pack_free(fh_pack *p) { delete p; }

extern "C" int fh_safetensors_check(const void *data, size_t len, int32_t *n_tensors) {
    return guarded([&] {
        if (!data && len) return fh::fail(FH_EINVAL, "fh_safetensors_check: null data");
        const auto m = futon::native::ParseSafetensors(std::string((const char *)data, len), true);
        if (n_tensors) *n_tensors = (int32_t)m.size();
        return FH_OK;
    });
}

extern "C" int fh_provider_new(const char *pack_dir, int32_t dimensions, int32_t threads, fh_provider **out) {
    return guarded([&] {
        if (!out) return fh::fail(FH_EINVAL, "fh_provider_new: null argument");
        *out = nullptr;
        futon::native::Options o;
        o.PackDir = pack_dir ? pack_dir : "";
        o.Dimensions = dimensions;
        o.Threads = threads;
        auto p = std::make_unique<fh_provider>();
        p->p = Provider::New(o);
        *out = p.release();
        return FH_OK;
    });
}

extern "C" int fh_provider_embed(fh_provider *p, const char *text, size_t len, float *out,
                                 const volatile int32_t *cancel) {
    const char *texts[1] = {text};
    const size_t lens[1] = {len};
    return fh_provider_embed_batch(p, texts, lens, 1, out, cancel);
}

extern "C" int fh_provider_embed_batch(fh_provider *p, const char *const *texts, const size_t *lens, int32_t n,
                                       float *out, const volatile int32_t *cancel) {
    return guarded([&] {
        if (!p || n < 0 || (n > 0 && (!texts || !lens || !out)))
            return fh::fail(FH_EINVAL, "fh_provider_embed_batch: null argument");
        std::vector<std::string> v((size_t)n);
        for (int32_t i = 0; i < n; i++) {
            if (!texts[i] && lens[i]) return fh::fail(FH_EINVAL, "fh_provider_embed_batch: null text %d", i);
            v[(size_t)i].assign(texts[i] ? texts[i] : "", lens[i]);
        }
        futon::Context ctx(cancel);
        const auto res = p->p->EmbedBatch(cancel ? &ctx : nullptr, v);
        const int dim = p->p->Dimensions();
        for (size_t i = 0; i < res.size(); i++) memcpy(out + i * (size_t)dim, res[i].data(), (size_t)dim * 4);
        return FH_OK;
    });
}

extern "C" int32_t fh_provider_dimensions(const fh_provider *p) { return p ? p->p->Dimensions() : 0; }

extern "C" int fh_provider_model_name(const fh_provider *p, char *buf, size_t len) {
    return p ? copy_str(p->p->ModelName(), buf, len) : fh::fail(FH_EINVAL, "fh_provider_model_name: null provider");
}

extern "C" int32_t fh_provider_is_available(const fh_provider *p) { return p && p->p->IsAvailable() ? 1 : 0; }

extern "C" int fh_provider_close(fh_provider *p) {
    if (!p) return fh::fail(FH_EINVAL, "fh_provider_close: null provider");
    p->p->Close();
    return FH_OK;
}

extern "C" void fh_provider_free(fh_provider *p) { delete p; }

extern "C" int fh_futon_new(const char *model, const char *models_dir, const char *model_path, int32_t dimensions,
                            int32_t threads, fh_provider **out) {
    return guarded([&] {
        if (!out) return fh::fail(FH_EINVAL, "fh_futon_new: null argument");
        *out = nullptr;
        futon::Options o;
        o.Model = model ? model : "";
        o.ModelsDir = models_dir ? models_dir : "";
        o.ModelPath = model_path ? model_path : "";
        futon::native::Options no;
        no.PackDir = futon::packDir(o);
        no.Dimensions = dimensions;
        no.Threads = futon::threadBudget(threads);
        auto p = std::make_unique<fh_provider>();
        p->p = Provider::New(no);
        *out = p.release();
        return FH_OK;
    });
}
