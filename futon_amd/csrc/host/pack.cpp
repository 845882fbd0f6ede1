// Pack loading on the host: config.json (native/config.go), the strict
// safetensors reader (native/safetensors.go), manifest verification
// (native/manifest.go), and the Model wrapper that hands the validated
// tensors to the device (native/model.go:112-132, :335-366).
#include <sys/stat.h>

#include <algorithm>
#include <cerrno>
#include <climits>
#include <cstdlib>
#include <cstring>

#include "../../../include/futon_hip.h"
#include "../../../include/futon_native.hpp"
#include "host_common.h"

namespace futon {
namespace native {

using fh::Json;
using fh::raise;

// ───────────────────────── config (native/config.go) ─────────────────────────

int64_t PackConfig::EffectiveMaxSeqLen() const {
    if (MaxTrainedPositions > 0 && MaxTrainedPositions < MaxSeqLen) return MaxTrainedPositions;
    return MaxSeqLen;
}

void PackConfig::Validate() const {
    const char *mid = ModelID.c_str();
    if (PackFormat != PackFormatVersion)
        raise(FH_EINVAL, "pack: unsupported pack_format %lld (loader supports %d)", (long long)PackFormat,
              PackFormatVersion);
    if (ModelID.empty()) raise(FH_EINVAL, "pack: model_id missing");
    if (HiddenSize <= 0 || NumLayers <= 0 || NumHeads <= 0 || IntermediateSize <= 0)
        raise(FH_EINVAL, "pack %s: non-positive architecture dimension", mid);
    if (HiddenSize % NumHeads != 0)
        raise(FH_EINVAL, "pack %s: hidden_size %lld not divisible by num_heads %lld", mid, (long long)HiddenSize,
              (long long)NumHeads);
    if (VocabSize <= 0 || MaxSeqLen <= 2) raise(FH_EINVAL, "pack %s: invalid vocab_size/max_seq_len", mid);
    if (MaxTrainedPositions < 0 || (MaxTrainedPositions > 0 && MaxTrainedPositions <= 2))
        raise(FH_EINVAL, "pack %s: invalid max_trained_positions %lld", mid, (long long)MaxTrainedPositions);
    if (LayerNormEps <= 0) raise(FH_EINVAL, "pack %s: layer_norm_eps must be positive", mid);
    if (PositionEncoding == "rope") {
        if (RoPETheta <= 0) raise(FH_EINVAL, "pack %s: rope position encoding requires rope_theta > 0", mid);
    } else if (PositionEncoding != "absolute") {
        raise(FH_EINVAL, "pack %s: unknown position_encoding \"%s\"", mid, PositionEncoding.c_str());
    }
    if (Activation != "gelu" && Activation != "swiglu")
        raise(FH_EINVAL, "pack %s: unknown activation \"%s\"", mid, Activation.c_str());
    if (Pooling != "mean" && Pooling != "cls") raise(FH_EINVAL, "pack %s: unknown pooling \"%s\"", mid, Pooling.c_str());
    if (PreNorm)
        raise(FH_EINVAL,
              "pack %s: pre_norm is declared but not yet implemented — refusing to run the wrong architecture", mid);
    if (Matryoshka) {
        for (int64_t d : Matryoshka->Dims)
            if (d <= 0 || d > HiddenSize)
                raise(FH_EINVAL, "pack %s: matryoshka dim %lld outside (0,%lld]", mid, (long long)d,
                      (long long)HiddenSize);
    }
}

namespace {

void need_object(const Json &v, const char *type) {
    if (v.kind != Json::Object && v.kind != Json::Null)
        raise(FH_EINVAL, "json: cannot unmarshal %s into Go value of type %s",
              v.kind == Json::Array ? "array" : v.kind == Json::String ? "string" : v.kind == Json::Number ? "number" : "bool",
              type);
}

void int_list(const Json *v, const char *field, std::vector<int64_t> &dst) {
    if (!v || v->kind == Json::Null) return;
    if (v->kind != Json::Array) raise(FH_EINVAL, "json: cannot unmarshal into field %s of type []int", field);
    dst.clear();
    for (const Json &e : v->arr) {
        int64_t x = 0;
        fh::json_int(&e, field, x);
        dst.push_back(x);
    }
}

void decode_config(const Json &j, PackConfig &c) {
    need_object(j, "native.PackConfig");
    if (j.kind == Json::Null) return;
    fh::json_int(j.get("pack_format"), "pack_format", c.PackFormat);
    fh::json_string(j.get("model_id"), "model_id", c.ModelID);
    fh::json_int(j.get("hidden_size"), "hidden_size", c.HiddenSize);
    fh::json_int(j.get("num_layers"), "num_layers", c.NumLayers);
    fh::json_int(j.get("num_heads"), "num_heads", c.NumHeads);
    fh::json_int(j.get("intermediate_size"), "intermediate_size", c.IntermediateSize);
    fh::json_int(j.get("vocab_size"), "vocab_size", c.VocabSize);
    fh::json_int(j.get("type_vocab_size"), "type_vocab_size", c.TypeVocabSize);
    fh::json_int(j.get("max_seq_len"), "max_seq_len", c.MaxSeqLen);
    fh::json_float(j.get("layer_norm_eps"), "layer_norm_eps", c.LayerNormEps);
    fh::json_string(j.get("position_encoding"), "position_encoding", c.PositionEncoding);
    fh::json_float(j.get("rope_theta"), "rope_theta", c.RoPETheta);
    fh::json_int(j.get("max_trained_positions"), "max_trained_positions", c.MaxTrainedPositions);
    fh::json_string(j.get("activation"), "activation", c.Activation);
    fh::json_bool(j.get("pre_norm"), "pre_norm", c.PreNorm);
    fh::json_string(j.get("pooling"), "pooling", c.Pooling);
    fh::json_bool(j.get("normalize"), "normalize", c.Normalize);
    if (const Json *m = j.get("matryoshka")) {
        if (m->kind != Json::Null) {
            need_object(*m, "native.MatryoshkaConfig");
            MatryoshkaConfig mc;
            fh::json_bool(m->get("layernorm"), "matryoshka.layernorm", mc.LayerNorm);
            int_list(m->get("dims"), "matryoshka.dims", mc.Dims);
            c.Matryoshka = mc;
        }
    }
    if (const Json *t = j.get("tokenizer")) {
        need_object(*t, "native.TokenizerConfig");
        if (t->kind == Json::Object) {
            TokenizerConfig &tc = c.Tokenizer;
            fh::json_bool(t->get("do_lower_case"), "tokenizer.do_lower_case", tc.DoLowerCase);
            fh::json_bool(t->get("tokenize_chinese_chars"), "tokenizer.tokenize_chinese_chars",
                          tc.TokenizeChineseChars);
            fh::json_int(t->get("max_input_chars_per_word"), "tokenizer.max_input_chars_per_word",
                         tc.MaxInputCharsPerWord);
            fh::json_string(t->get("cls_token"), "tokenizer.cls_token", tc.ClsToken);
            fh::json_string(t->get("sep_token"), "tokenizer.sep_token", tc.SepToken);
            fh::json_string(t->get("unk_token"), "tokenizer.unk_token", tc.UnkToken);
            fh::json_string(t->get("pad_token"), "tokenizer.pad_token", tc.PadToken);
            fh::json_string(t->get("mask_token"), "tokenizer.mask_token", tc.MaskToken);
        }
    }
    if (const Json *p = j.get("prefixes")) {
        if (p->kind != Json::Null) {
            need_object(*p, "map[string]string");
            for (const auto &kv : p->obj) {
                std::string v;
                fh::json_string(&kv.second, "prefixes", v);
                c.Prefixes[kv.first] = v;
            }
        }
    }
}

}  // namespace

PackConfig ParsePackConfig(const std::string &raw) {
    PackConfig cfg;
    try {
        decode_config(fh::parse_json(raw.data(), raw.size(), "json"), cfg);
    } catch (const fh::Error &e) {
        raise(FH_EINVAL, "pack: parse config: %s", e.what());
    }
    cfg.Validate();
    return cfg;
}

PackConfig LoadPackConfig(const std::string &dir) {
    std::string raw, err;
    if (!fh::read_file(fh::join_path(dir, "config.json"), raw, err)) raise(FH_EINVAL, "pack: read config: %s", err.c_str());
    return ParsePackConfig(raw);
}

// ───────────────────── safetensors (native/safetensors.go) ─────────────────────

namespace {

constexpr uint64_t kMaxHeaderBytes = 16ull << 20;  // maxHeaderBytes, native/safetensors.go:39

float f16_bits_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31, exp = (h >> 10) & 0x1f, mant = h & 0x3ff, bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            uint32_t e = 127 - 15 + 1;
            while (!(mant & 0x400)) {
                mant <<= 1;
                e--;
            }
            bits = sign | e << 23 | (mant & 0x3ff) << 13;
        }
    } else if (exp == 0x1f) {
        bits = sign | 0xffu << 23 | mant << 13;
    } else {
        bits = sign | (exp + 127 - 15) << 23 | mant << 13;
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

std::string shape_str(const std::vector<int64_t> &s) {
    std::string o = "[";
    for (size_t i = 0; i < s.size(); i++) {
        if (i) o += " ";
        o += std::to_string(s[i]);
    }
    return o + "]";
}

}  // namespace

int64_t Tensor::Numel() const {
    int64_t n = 1;
    for (int64_t d : Shape) n *= d;
    return n;
}

TensorMap ParseSafetensors(const std::string &raw, bool keepF16) {
    if (raw.size() < 8) raise(FH_EINVAL, "safetensors: file too small (%zu bytes) for header length prefix", raw.size());
    uint64_t hl = 0;
    for (int i = 7; i >= 0; i--) hl = hl << 8 | (uint8_t)raw[(size_t)i];
    if (hl > kMaxHeaderBytes)
        raise(FH_EINVAL, "safetensors: header length %llu exceeds limit %llu", (unsigned long long)hl,
              (unsigned long long)kMaxHeaderBytes);
    if (raw.size() < 8 + hl)
        raise(FH_EINVAL, "safetensors: declared header length %llu exceeds file size %zu", (unsigned long long)hl,
              raw.size());
    Json header;
    try {
        header = fh::parse_json(raw.data() + 8, (size_t)hl, "json");
    } catch (const fh::Error &e) {
        raise(FH_EINVAL, "safetensors: parse header JSON: %s", e.what());
    }
    if (header.kind != Json::Object && header.kind != Json::Null)
        raise(FH_EINVAL, "safetensors: parse header JSON: json: cannot unmarshal into map[string]json.RawMessage");
    const char *data = raw.data() + 8 + hl;
    const int64_t dlen = (int64_t)(raw.size() - 8 - hl);

    // Last occurrence of a key wins, as for a Go map.
    std::map<std::string, const Json *> entries;
    for (const auto &kv : header.obj) entries[kv.first] = &kv.second;

    struct Span {
        int64_t begin, end;
        std::string name;
    };
    std::vector<Span> spans;
    TensorMap tensors;
    for (const auto &kv : entries) {
        const std::string &name = kv.first;
        if (name == "__metadata__") continue;
        const Json &e = *kv.second;
        std::string dtype;
        std::vector<int64_t> shape;
        int64_t offs[2] = {0, 0};
        try {
            if (e.kind != Json::Object && e.kind != Json::Null)
                raise(FH_EINVAL, "json: cannot unmarshal into Go value of type native.stHeaderEntry");
            if (e.kind == Json::Object) {
                fh::json_string(e.get("dtype"), "dtype", dtype);
                int_list(e.get("shape"), "shape", shape);
                if (const Json *o = e.get("data_offsets")) {
                    if (o->kind == Json::Array) {
                        for (size_t i = 0; i < o->arr.size(); i++) {
                            int64_t x = 0;
                            fh::json_int(&o->arr[i], "data_offsets", x);
                            if (i < 2) offs[i] = x;
                        }
                    } else if (o->kind != Json::Null) {
                        raise(FH_EINVAL, "json: cannot unmarshal into field data_offsets of type [2]int");
                    }
                }
            }
        } catch (const fh::Error &err) {
            raise(FH_EINVAL, "safetensors: tensor \"%s\": parse entry: %s", name.c_str(), err.what());
        }
        int64_t esz;
        if (dtype == "F32") esz = 4;
        else if (dtype == "F16") esz = 2;
        else
            raise(FH_EINVAL, "safetensors: tensor \"%s\": unsupported dtype \"%s\" (want F32 or F16)", name.c_str(),
                  dtype.c_str());
        unsigned __int128 elems = 1;
        for (int64_t d : shape) {
            if (d < 0) raise(FH_EINVAL, "safetensors: tensor \"%s\": negative dimension %lld", name.c_str(), (long long)d);
            elems *= (uint64_t)d;
            if (elems >> 64)
                raise(FH_EINVAL, "safetensors: tensor \"%s\": shape %s element count overflows", name.c_str(),
                      shape_str(shape).c_str());
        }
        if ((uint64_t)elems > (uint64_t)INT64_MAX / (uint64_t)esz)
            raise(FH_EINVAL, "safetensors: tensor \"%s\": shape %s byte size overflows", name.c_str(),
                  shape_str(shape).c_str());
        const int64_t n = (int64_t)elems, b = offs[0], en = offs[1];
        if (b < 0 || en < b || en > dlen)
            raise(FH_EINVAL, "safetensors: tensor \"%s\": offsets [%lld,%lld) outside data section of %lld bytes",
                  name.c_str(), (long long)b, (long long)en, (long long)dlen);
        if (en - b != n * esz)
            raise(FH_EINVAL, "safetensors: tensor \"%s\": shape %s × %s needs %lld bytes, offsets span %lld",
                  name.c_str(), shape_str(shape).c_str(), dtype.c_str(), (long long)(n * esz), (long long)(en - b));
        Tensor t;
        t.Name = name;
        t.Shape = shape;
        const char *buf = data + b;
        if (esz == 4) {
            t.Data.resize((size_t)n);
            memcpy(t.Data.data(), buf, (size_t)n * 4);  // little-endian host
        } else if (keepF16) {
            t.F16.resize((size_t)n);
            memcpy(t.F16.data(), buf, (size_t)n * 2);
        } else {
            t.Data.resize((size_t)n);
            for (int64_t i = 0; i < n; i++) {
                uint16_t h;
                memcpy(&h, buf + 2 * i, 2);
                t.Data[(size_t)i] = f16_bits_to_f32(h);
            }
        }
        tensors[name] = std::move(t);
        spans.push_back({b, en, name});
    }
    // Spans tile the data section exactly: no overlap, gap or trailing bytes.
    std::stable_sort(spans.begin(), spans.end(), [](const Span &x, const Span &y) { return x.begin < y.begin; });
    int64_t cursor = 0;
    for (const Span &s : spans) {
        if (s.begin != cursor)
            raise(FH_EINVAL, "safetensors: tensor \"%s\" begins at %lld, expected %lld (overlap or gap)", s.name.c_str(),
                  (long long)s.begin, (long long)cursor);
        cursor = s.end;
    }
    if (cursor != dlen)
        raise(FH_EINVAL, "safetensors: data section is %lld bytes but tensors cover %lld", (long long)dlen,
              (long long)cursor);
    return tensors;
}

TensorMap LoadSafetensors(const std::string &path) {
    std::string raw, err;
    if (!fh::read_file(path, raw, err)) raise(FH_EINVAL, "safetensors: read %s: %s", path.c_str(), err.c_str());
    return ParseSafetensors(raw, false);
}

TensorMap LoadSafetensorsRaw(const std::string &path) {
    std::string raw, err;
    if (!fh::read_file(path, raw, err)) raise(FH_EINVAL, "safetensors: read %s: %s", path.c_str(), err.c_str());
    return ParseSafetensors(raw, true);
}

// ───────────────────────── manifest (native/manifest.go) ─────────────────────────

PackManifest loadAndVerifyManifest(const std::string &dir) {
    std::string raw, err;
    if (!fh::read_file(fh::join_path(dir, "manifest.json"), raw, err))
        raise(FH_EINVAL, "pack %s: manifest.json unreadable (refusing to load an unverifiable pack): %s", dir.c_str(),
              err.c_str());
    PackManifest man;
    try {
        const Json j = fh::parse_json(raw.data(), raw.size(), "json");
        need_object(j, "native.PackManifest");
        if (j.kind == Json::Object) {
            fh::json_int(j.get("pack_format"), "pack_format", man.PackFormat);
            fh::json_string(j.get("model_id"), "model_id", man.ModelID);
            if (const Json *m = j.get("members"); m && m->kind != Json::Null) {
                need_object(*m, "map[string]struct");
                for (const auto &kv : m->obj) {
                    need_object(kv.second, "struct");
                    PackManifest::Member mem;
                    if (kv.second.kind == Json::Object) {
                        fh::json_string(kv.second.get("sha256"), "sha256", mem.SHA256);
                        fh::json_int(kv.second.get("size"), "size", mem.Size);
                    }
                    man.Members[kv.first] = mem;
                }
            }
            if (const Json *t = j.get("tensor_names"); t && t->kind != Json::Null) {
                if (t->kind != Json::Array) raise(FH_EINVAL, "json: cannot unmarshal into field tensor_names of type []string");
                std::vector<std::string> names;
                for (const Json &e : t->arr) {
                    std::string s;
                    fh::json_string(&e, "tensor_names", s);
                    names.push_back(s);
                }
                man.TensorNames = names;
            }
        }
    } catch (const fh::Error &e) {
        raise(FH_EINVAL, "pack %s: manifest.json malformed: %s", dir.c_str(), e.what());
    }
    for (const char *member : {"config.json", "model.safetensors", "vocab.txt"}) {
        auto it = man.Members.find(member);
        if (it == man.Members.end()) raise(FH_EINVAL, "pack %s: manifest records no entry for %s", dir.c_str(), member);
        const std::string path = fh::join_path(dir, member);
        struct stat st;
        if (stat(path.c_str(), &st) != 0)
            raise(FH_EINVAL, "pack %s: member %s: stat %s: %s", dir.c_str(), member, path.c_str(), strerror(errno));
        if ((int64_t)st.st_size != it->second.Size)
            raise(FH_EINVAL, "pack %s: member %s is %lld bytes, manifest records %lld", dir.c_str(), member,
                  (long long)st.st_size, (long long)it->second.Size);
        std::string got;
        try {
            got = fh::sha256_file_hex(path);
        } catch (const fh::Error &e) {
            raise(FH_EINVAL, "pack %s: member %s: %s", dir.c_str(), member, e.what());
        }
        if (got != it->second.SHA256)
            raise(FH_EINVAL,
                  "pack %s: member %s sha256 %s does not match manifest %s (tampered or corrupt — rebuild the pack)",
                  dir.c_str(), member, got.c_str(), it->second.SHA256.c_str());
    }
    return man;
}

void PackManifest::verifyTensorNames(const TensorMap &tensors) const {
    if (!TensorNames) return;  // pre-tensor_names manifest; the member hashes still cover the bytes
    std::vector<std::string> got, want = *TensorNames;
    for (const auto &kv : tensors) got.push_back(kv.first);
    std::sort(got.begin(), got.end());
    std::sort(want.begin(), want.end());
    if (got.size() != want.size())
        raise(FH_EINVAL, "pack %s: %zu tensors on disk, manifest records %zu — tensor set drifted", ModelID.c_str(),
              got.size(), want.size());
    for (size_t i = 0; i < got.size(); i++)
        if (got[i] != want[i])
            raise(FH_EINVAL, "pack %s: tensor set drifted from manifest (first difference: \"%s\" vs recorded \"%s\")",
                  ModelID.c_str(), got[i].c_str(), want[i].c_str());
}

// ───────────────────────── model (native/model.go) ─────────────────────────

Pack LoadPack(const std::string &dir) {
    Pack p;
    p.Dir = dir;
    p.Manifest = loadAndVerifyManifest(dir);
    p.Config = LoadPackConfig(dir);
    if (p.Manifest.ModelID != p.Config.ModelID)
        raise(FH_EINVAL, "pack %s: manifest is for \"%s\" — mixed pack contents", p.Config.ModelID.c_str(),
              p.Manifest.ModelID.c_str());
    try {
        p.Tensors = LoadSafetensorsRaw(fh::join_path(dir, "model.safetensors"));
    } catch (const fh::Error &e) {
        raise(e.code, "pack %s: %s", p.Config.ModelID.c_str(), e.what());
    }
    p.Manifest.verifyTensorNames(p.Tensors);
    return p;
}

namespace {

[[noreturn]] void raise_device(int rc) {
    throw fh::Error(rc, std::string("native: ") + fh::last_error());
}

fh_config device_config(const PackConfig &c, bool q8) {
    auto i32 = [&](int64_t v, const char *what) {
        if (v < INT_MIN || v > INT_MAX) raise(FH_EINVAL, "pack %s: %s %lld out of range", c.ModelID.c_str(), what, (long long)v);
        return (int32_t)v;
    };
    fh_config d{};
    d.hidden_size = i32(c.HiddenSize, "hidden_size");
    d.num_layers = i32(c.NumLayers, "num_layers");
    d.num_heads = i32(c.NumHeads, "num_heads");
    d.intermediate_size = i32(c.IntermediateSize, "intermediate_size");
    d.vocab_size = i32(c.VocabSize, "vocab_size");
    d.type_vocab_size = i32(c.TypeVocabSize, "type_vocab_size");
    d.max_seq_len = i32(c.MaxSeqLen, "max_seq_len");
    d.max_trained_positions = i32(c.MaxTrainedPositions, "max_trained_positions");
    d.layer_norm_eps = c.LayerNormEps;
    d.position_encoding = c.PositionEncoding == "rope" ? FH_POS_ROPE : FH_POS_ABSOLUTE;
    d.rope_theta = c.RoPETheta;
    d.activation = c.Activation == "swiglu" ? FH_ACT_SWIGLU : FH_ACT_GELU;
    d.pooling = c.Pooling == "cls" ? FH_POOL_CLS : FH_POOL_MEAN;
    d.normalize = c.Normalize ? 1 : 0;
    d.matryoshka = c.Matryoshka ? 1 : 0;
    d.matryoshka_layernorm = c.Matryoshka && c.Matryoshka->LayerNorm ? 1 : 0;
    d.q8 = q8 ? 1 : 0;
    return d;
}

}  // namespace

Model::Model(const Pack &pack, bool q8, int device) : cfg_(pack.Config), q8_(q8) {
    const fh_config dc = device_config(cfg_, q8);
    std::vector<fh_tensor> ts;
    ts.reserve(pack.Tensors.size());
    for (const auto &kv : pack.Tensors) {
        const Tensor &t = kv.second;
        if (t.Shape.size() > 4)
            raise(FH_EINVAL, "pack %s: tensor \"%s\" has rank %zu", cfg_.ModelID.c_str(), t.Name.c_str(), t.Shape.size());
        fh_tensor d{};
        d.name = t.Name.c_str();
        d.rank = (int32_t)t.Shape.size();
        for (size_t i = 0; i < t.Shape.size(); i++) d.shape[i] = t.Shape[i];
        if (!t.F16.empty()) {
            d.dtype = FH_DTYPE_F16;
            d.data = t.F16.data();
        } else {
            d.dtype = FH_DTYPE_F32;
            d.data = t.Data.data();
        }
        ts.push_back(d);
    }
    const int rc = fh_model_create(&dc, ts.data(), (int32_t)ts.size(), device, &h_);
    if (rc != FH_OK) raise_device(rc);
}

Model::~Model() { fh_model_destroy(h_); }

std::vector<std::vector<float>> Model::EncodeBatch(const Context *ctx, const std::vector<std::vector<int>> &batch,
                                                   int outDim) const {
    std::vector<std::vector<float>> res;
    if (batch.empty()) return res;
    const int dim = outDim == 0 ? (int)cfg_.HiddenSize : outDim;
    std::vector<int32_t> ids, offs;
    offs.reserve(batch.size() + 1);
    size_t total = 0;
    for (const auto &s : batch) total += s.size();
    ids.reserve(total);
    for (const auto &s : batch) {
        offs.push_back((int32_t)ids.size());
        for (int id : s) ids.push_back((int32_t)id);
    }
    offs.push_back((int32_t)ids.size());
    std::vector<float> out((size_t)batch.size() * (size_t)std::max(dim, 1));
    const int rc = fh_encode(h_, ids.data(), offs.data(), (int32_t)batch.size(), (int32_t)outDim, out.data(),
                             ctx ? ctx->flag() : nullptr);
    if (rc != FH_OK) raise_device(rc);
    res.resize(batch.size());
    for (size_t i = 0; i < batch.size(); i++) res[i].assign(out.begin() + (long)(i * dim), out.begin() + (long)((i + 1) * dim));
    return res;
}

std::vector<float> Model::EncodeTokens(const Context *ctx, const std::vector<int> &ids, int outDim) const {
    return EncodeBatch(ctx, {ids}, outDim)[0];
}

std::shared_ptr<Model> LoadModel(const std::string &dir, int threads) {
    (void)threads;  // the device forward has no host thread budget
    const Pack p = LoadPack(dir);
    const char *q = getenv("FUTON_NATIVE_Q8");
    return std::make_shared<Model>(p, q && std::string(q) == "1");
}

}  // namespace native
}  // namespace futon
