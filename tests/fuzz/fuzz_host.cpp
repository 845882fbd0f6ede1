// Seeded fuzz driver for the host parsers that read untrusted bytes: the
// safetensors reader (ParseSafetensors), the pack-config JSON decoder
// (ParsePackConfig) and the WordPiece tokenizer (Tokenizer::Encode).  Built
// with AddressSanitizer + UndefinedBehaviorSanitizer by tests/test_sanitize.py
// from the host sources only (no device code).
//
//   fuzz_host safetensors <seed.safetensors> <iterations> <seed>
//   fuzz_host config      <config.json>      <iterations> <seed>
//   fuzz_host tokenizer   <vocab.txt>        <iterations> <seed>
//
// Parsers must either succeed or throw fh::Error; the tokenizer must return
// a well-formed [CLS] … [SEP] sequence within bounds for any byte soup, the
// same ids twice (native/tokenizer_test.go:130-168).  Exit status 0 = no
// property failed (sanitizer reports abort the process).
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>
#include <string>
#include <vector>

#include "futon_native.hpp"

// The device half of the C ABI is not part of this build: model creation
// reports no device, which the parsers never reach.
extern "C" {
int fh_model_create(const fh_config *, const fh_tensor *, int32_t, int32_t, fh_model **out) {
    if (out) *out = nullptr;
    return FH_ENODEV;
}
void fh_model_destroy(fh_model *) {}
int fh_encode(fh_model *, const int32_t *, const int32_t *, int32_t, int32_t, float *, const volatile int32_t *) {
    return FH_ENODEV;
}
}

namespace {

uint64_t rng_state = 1;
uint64_t next() {  // splitmix64
    uint64_t z = (rng_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
size_t below(size_t n) { return n ? (size_t)(next() % n) : 0; }

std::string read_all(const char *path) {
    std::ifstream f(path, std::ios::binary);
    std::stringstream ss;
    ss << f.rdbuf();
    return ss.str();
}

// Byte-level mutations, plus edits aimed at the formats' numbers and
// structure: digits rewritten, lengths grown or shrunk, JSON punctuation.
std::string mutate(const std::string &in, bool textual) {
    std::string s = in;
    const int edits = 1 + (int)below(8);
    static const char *tokens[] = {"\"", "{", "}", "[", "]", ",", ":", "null", "-1", "1e308", "18446744073709551615",
                                   "9223372036854775807", "0", "\"F16\"", "\"F32\"", "\"I8\"", "\\u0000", "\\ud800",
                                   "true", "1.5", "[]", "{}", " "};
    for (int e = 0; e < edits; e++) {
        const size_t n = s.size();
        switch (below(textual ? 9 : 7)) {
        case 0:
            if (n) s[below(n)] ^= (char)(1u << below(8));
            break;
        case 1:
            if (n) s[below(n)] = (char)next();
            break;
        case 2:
            if (n) s.resize(below(n + 1));
            break;
        case 3:
            s.insert(below(n + 1), 1 + below(16), (char)next());
            break;
        case 4:
            if (n) s.erase(below(n), 1 + below(32));
            break;
        case 5: {  // rewrite a run of digits
            for (int tries = 0; tries < 16 && n; tries++) {
                const size_t p = below(n);
                if (s[p] >= '0' && s[p] <= '9') {
                    size_t q = p;
                    while (q < s.size() && s[q] >= '0' && s[q] <= '9') q++;
                    s.replace(p, q - p, std::to_string((long long)(next() % 2 ? next() : next() % 1000)));
                    break;
                }
            }
            break;
        }
        case 6:  // the 8-byte little-endian header length of a safetensors image
            if (n >= 8) {
                uint64_t v = below(4) == 0 ? next() : (uint64_t)(n - 8 + below(64)) - 32;
                memcpy(&s[0], &v, 8);
            }
            break;
        default: {
            const char *t = tokens[below(sizeof tokens / sizeof *tokens)];
            s.insert(below(n + 1), t);
        }
        }
    }
    return s;
}

int fuzz_safetensors(const std::string &seed, long iters) {
    long ok = 0, rejected = 0;
    for (long i = 0; i < iters; i++) {
        const std::string img = i == 0 ? seed : mutate(seed, below(2) == 0);
        for (int raw = 0; raw < 2; raw++) {
            try {
                const auto m = futon::native::ParseSafetensors(img, raw != 0);
                for (const auto &kv : m) {  // every accepted tensor is whole
                    const auto &t = kv.second;
                    const size_t have = raw && !t.F16.empty() ? t.F16.size() : t.Data.size();
                    if ((int64_t)have != t.Numel()) {
                        fprintf(stderr, "tensor %s: %zu values for %lld elements\n", kv.first.c_str(), have,
                                (long long)t.Numel());
                        return 1;
                    }
                }
                ok++;
            } catch (const fh::Error &) {
                rejected++;
            }
        }
    }
    printf("safetensors: %ld accepted, %ld rejected\n", ok, rejected);
    return 0;
}

int fuzz_config(const std::string &seed, long iters) {
    long ok = 0, rejected = 0;
    for (long i = 0; i < iters; i++) {
        const std::string js = i == 0 ? seed : mutate(seed, true);
        try {
            const auto c = futon::native::ParsePackConfig(js);
            const int64_t eff = c.EffectiveMaxSeqLen();
            if (eff <= 0 || eff > c.MaxSeqLen) {
                fprintf(stderr, "accepted config with EffectiveMaxSeqLen %lld (max_seq_len %lld)\n", (long long)eff,
                        (long long)c.MaxSeqLen);
                return 1;
            }
            ok++;
        } catch (const fh::Error &) {
            rejected++;
        }
    }
    printf("config: %ld accepted, %ld rejected\n", ok, rejected);
    return 0;
}

int fuzz_tokenizer(const char *vocab, long iters) {
    futon::native::TokenizerConfig cfg;
    cfg.DoLowerCase = true;
    cfg.TokenizeChineseChars = true;
    cfg.ClsToken = "[CLS]";
    cfg.SepToken = "[SEP]";
    cfg.UnkToken = "[UNK]";
    cfg.PadToken = "[PAD]";
    cfg.MaskToken = "[MASK]";
    futon::native::Tokenizer tok(vocab, cfg);
    const std::vector<std::string> seeds = {"", " ", "hello world", "\xC3\x89lodie caf\xC3\xA9 \xE2\x98\x83",
                                            "\xE8\x87\xAA\xE7\x84\xB6\xE8\xA8\x80\xE8\xAA\x9E", "(((([[{{}}]]))))",
                                            std::string("a\x00b\x07" "c", 5), "\xff\xfe invalid utf8",
                                            "buffalo buffalo buffalo", "x", "[CLS] injected [SEP]",
                                            "e\xCC\x81\xCC\x81\xCC\x81 combining", std::string(300, 'a')};
    for (long i = 0; i < iters; i++) {
        std::string text = seeds[below(seeds.size())];
        if (i >= (long)seeds.size()) {
            text = mutate(text, true);
            if (below(4) == 0) {  // random code points, valid and not
                const int n = (int)below(64);
                for (int k = 0; k < n; k++) {
                    const uint32_t cp = below(3) == 0 ? (uint32_t)below(0x110000) : (uint32_t)below(0x3000);
                    if (cp < 0x80) {
                        text += (char)cp;
                    } else if (cp < 0x800) {
                        text += (char)(0xC0 | (cp >> 6));
                        text += (char)(0x80 | (cp & 0x3F));
                    } else if (cp < 0x10000) {
                        text += (char)(0xE0 | (cp >> 12));
                        text += (char)(0x80 | ((cp >> 6) & 0x3F));
                        text += (char)(0x80 | (cp & 0x3F));
                    } else {
                        text += (char)(0xF0 | (cp >> 18));
                        text += (char)(0x80 | ((cp >> 12) & 0x3F));
                        text += (char)(0x80 | ((cp >> 6) & 0x3F));
                        text += (char)(0x80 | (cp & 0x3F));
                    }
                }
            }
        }
        const int maxLen = (int)(next() % 1024) + 2;
        const auto ids = tok.Encode(text, maxLen);
        if (ids.size() < 2 || (int)ids.size() > maxLen || ids.front() != 101 || ids.back() != 102) {
            fprintf(stderr, "malformed encoding of a %zu-byte text (maxLen %d): %zu ids\n", text.size(), maxLen,
                    ids.size());
            return 1;
        }
        for (int id : ids)
            if (id < 0 || id >= tok.VocabSize()) {
                fprintf(stderr, "id %d outside vocab %d\n", id, tok.VocabSize());
                return 1;
            }
        if (tok.Encode(text, maxLen) != ids) {
            fprintf(stderr, "non-deterministic encode\n");
            return 1;
        }
    }
    printf("tokenizer: %ld texts\n", iters);
    return 0;
}

}  // namespace

int main(int argc, char **argv) {
    if (argc != 5) {
        fprintf(stderr, "usage: %s safetensors|config|tokenizer <seed-file> <iterations> <seed>\n", argv[0]);
        return 2;
    }
    const std::string mode = argv[1];
    const long iters = atol(argv[3]);
    rng_state = strtoull(argv[4], nullptr, 10);
    if (mode == "safetensors") return fuzz_safetensors(read_all(argv[2]), iters);
    if (mode == "config") return fuzz_config(read_all(argv[2]), iters);
    if (mode == "tokenizer") return fuzz_tokenizer(argv[2], iters);
    fprintf(stderr, "unknown mode %s\n", mode.c_str());
    return 2;
}
