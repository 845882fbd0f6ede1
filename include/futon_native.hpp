/*
 * futon_native.hpp — C++ host side of the MI355X futon encoder.
 *
 * The reference's host side is Go (package native and package futon); this
 * header restates the part of it that sits on the forward path, with the
 * same names, argument meanings and error behaviour, above the device C ABI
 * (futon_hip.h):
 *
 *   PackConfig, Validate, EffectiveMaxSeqLen, LoadPackConfig   native/config.go:34-187
 *   Tensor, ParseSafetensors, LoadSafetensors(Raw)              native/safetensors.go:36-221
 *   PackManifest, loadAndVerifyManifest, verifyTensorNames      native/manifest.go:1-117
 *   TokenizerConfig, Tokenizer, NewTokenizer, Encode            native/tokenizer.go:1-361
 *   Model, LoadModel, EncodeTokens                              native/model.go:112-457
 *   Options, Provider, New, Embed, EmbedBatch, ModelName, Close native/provider.go:29-290
 *   futon::Options, futon::Embedder, futon::New                 futon.go:32-154
 *
 * Where Go returns (value, error), these functions return the value and
 * throw fh::Error (code = an FH_E* value from futon_hip.h, what() = the
 * reference's message).  A Context carries cancellation, as Go's ctx does.
 */
#ifndef FUTON_NATIVE_HPP
#define FUTON_NATIVE_HPP

#include <atomic>
#include <cstdint>
#include <map>
#include <memory>
#include <mutex>
#include <optional>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "futon_hip.h"

namespace fh {
struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string &msg) : std::runtime_error(msg), code(c) {}
};
}  // namespace fh

namespace futon {

// Cancellation flag polled by the device forward at the reference's
// checkpoints (before each layer, between attention and FFN).
// A Context owns its flag (Cancel sets it) or watches a caller's flag.
class Context {
  public:
    Context() = default;
    explicit Context(const volatile int32_t *external) : ext_(external) {}
    void Cancel() { flag_.store(1); }
    bool Canceled() const { return ext_ ? *ext_ != 0 : flag_.load() != 0; }
    const volatile int32_t *flag() const {
        return ext_ ? ext_ : reinterpret_cast<const volatile int32_t *>(&flag_);
    }

  private:
    std::atomic<int32_t> flag_{0};
    const volatile int32_t *ext_ = nullptr;
};

namespace native {

constexpr int PackFormatVersion = 1;
constexpr const char *NativeModelNamePrefix = "native/";
constexpr const char *PackNomicEmbedTextV15 = "nomic-embed-text-v1.5";
constexpr const char *PackBGESmallENV15 = "bge-small-en-v1.5";
constexpr const char *PackArcticEmbedMLong = "snowflake-arctic-embed-m-long";

struct MatryoshkaConfig {
    bool LayerNorm = false;
    std::vector<int64_t> Dims;
};

struct TokenizerConfig {
    bool DoLowerCase = false;
    bool TokenizeChineseChars = false;
    int64_t MaxInputCharsPerWord = 0;
    std::string ClsToken, SepToken, UnkToken, PadToken, MaskToken;
};

struct PackConfig {
    int64_t PackFormat = 0;
    std::string ModelID;
    int64_t HiddenSize = 0, NumLayers = 0, NumHeads = 0, IntermediateSize = 0, VocabSize = 0, TypeVocabSize = 0,
            MaxSeqLen = 0;
    double LayerNormEps = 0;
    std::string PositionEncoding;
    double RoPETheta = 0;
    int64_t MaxTrainedPositions = 0;
    std::string Activation;
    bool PreNorm = false;
    std::string Pooling;
    bool Normalize = false;
    std::optional<MatryoshkaConfig> Matryoshka;
    TokenizerConfig Tokenizer;
    std::map<std::string, std::string> Prefixes;

    int64_t EffectiveMaxSeqLen() const;
    void Validate() const;  // throws fh::Error(FH_EINVAL)
};
PackConfig ParsePackConfig(const std::string &json);  // decode + Validate
PackConfig LoadPackConfig(const std::string &dir);

struct Tensor {
    std::string Name;
    std::vector<int64_t> Shape;
    std::vector<float> Data;    // row-major float32 (F32, or F16 dequantized)
    std::vector<uint16_t> F16;  // raw binary16 bits (raw mode only)
    int64_t Numel() const;
};
using TensorMap = std::map<std::string, Tensor>;
TensorMap ParseSafetensors(const std::string &raw, bool keepF16 = false);
TensorMap LoadSafetensors(const std::string &path);
TensorMap LoadSafetensorsRaw(const std::string &path);

struct PackManifest {
    struct Member {
        std::string SHA256;
        int64_t Size = 0;
    };
    int64_t PackFormat = 0;
    std::string ModelID;
    std::map<std::string, Member> Members;
    std::optional<std::vector<std::string>> TensorNames;
    void verifyTensorNames(const TensorMap &tensors) const;
};
PackManifest loadAndVerifyManifest(const std::string &dir);

class Tokenizer {
  public:
    Tokenizer(const std::string &vocabPath, TokenizerConfig cfg);  // NewTokenizer
    std::vector<int> Encode(const std::string &text, int maxSeqLen) const;
    int VocabSize() const { return (int)vocab_.size(); }
    int PadID() const { return padID_; }

  private:
    struct Segment {
        std::string text;
        int specialID;
    };
    std::vector<Segment> splitSpecials(const std::string &text) const;
    std::vector<std::string> basicTokenize(const std::string &text) const;
    void wordPiece(const std::string &word, std::vector<int> &out) const;

    TokenizerConfig cfg_;
    std::unordered_map<std::string, int> vocab_;
    int clsID_ = 0, sepID_ = 0, unkID_ = 0, padID_ = 0, maskID_ = 0;
    std::vector<std::pair<std::string, int>> specials_;
};

// The validated host half of LoadModel: config, manifest, tensors.
struct Pack {
    std::string Dir;
    PackConfig Config;
    PackManifest Manifest;
    TensorMap Tensors;
};
Pack LoadPack(const std::string &dir);  // manifest → config → model_id → safetensors → tensor names

// A pack resident on one GPU.  Safe for concurrent use.
class Model {
  public:
    Model(const Pack &pack, bool q8, int device = 0);
    ~Model();
    Model(const Model &) = delete;
    Model &operator=(const Model &) = delete;

    const PackConfig &Config() const { return cfg_; }
    bool Q8() const { return q8_; }
    fh_model *Handle() const { return h_; }
    std::vector<float> EncodeTokens(const Context *ctx, const std::vector<int> &ids, int outDim) const;
    // One device call for the whole batch; vectors are index-aligned and
    // bit-identical to EncodeTokens of each sequence.
    std::vector<std::vector<float>> EncodeBatch(const Context *ctx, const std::vector<std::vector<int>> &batch,
                                                int outDim) const;

  private:
    PackConfig cfg_;
    bool q8_ = false;
    fh_model *h_ = nullptr;
};
// LoadModel (model.go:112-132); Q8 weights when FUTON_NATIVE_Q8=1.
std::shared_ptr<Model> LoadModel(const std::string &dir, int threads = 0);

struct Options {
    std::string PackDir;
    int Dimensions = 0;
    int Threads = 0;
};

class Provider {
  public:
    static std::unique_ptr<Provider> New(const Options &opts);  // native.New
    std::vector<float> Embed(const Context *ctx, const std::string &text);
    std::vector<std::vector<float>> EmbedBatch(const Context *ctx, const std::vector<std::string> &texts);
    int Dimensions() const { return dims_; }
    std::string ModelName() const;
    bool IsAvailable() const;
    void Close();
    const Tokenizer &Tok() const { return *tok_; }
    const Model &Mdl() const { return *model_; }

  private:
    void checkOpen() const;
    std::shared_ptr<Model> model_;
    std::unique_ptr<Tokenizer> tok_;
    int dims_ = 0, threads_ = 1;
    mutable std::mutex mu_;
    bool closed_ = false;
};

}  // namespace native

constexpr const char *DefaultModel = "bge-small-en-v1.5";

struct Options {
    std::string Model, ModelsDir, ModelPath;
    int Dimensions = 0;
    int Threads = 0;
};

class Embedder {
  public:
    virtual ~Embedder() = default;
    virtual std::vector<float> Embed(const Context *ctx, const std::string &text) = 0;
    virtual std::vector<std::vector<float>> EmbedBatch(const Context *ctx, const std::vector<std::string> &texts) = 0;
    virtual int Dimensions() const = 0;
    virtual std::string ModelName() const = 0;
    virtual void Close() = 0;
};

std::unique_ptr<Embedder> New(const Options &opts);  // futon.New (local packs only)
std::string DefaultModelsDir();
// futon.go:100-119 and packs.Resolve (packs/packs.go:84-113): the pack
// directory New loads (ModelPath, else ModelsDir/Model with defaults).
std::string packDir(const Options &opts);
// futon.go:131-154: requested threads (default 6) clamped to the CPUs.
int threadBudget(int requested);

}  // namespace futon

#endif /* FUTON_NATIVE_HPP */
