// Host WordPiece tokenizer: native/tokenizer.go restated in C++.  The
// pipeline is the HF BERT one the reference implements — literal special
// tokens split first on the raw text, then clean (drop NUL, U+FFFD and
// controls, canonicalize whitespace, isolate CJK ideographs), lowercase +
// NFD + drop Mn, split on whitespace and punctuation, greedy longest-match
// WordPiece with "##" continuations — and the ids are pinned bit-exact by
// the reference's tokenizer fixtures.
//
// Text is iterated the way Go's `for range` iterates a string: UTF-8
// decoded rune by rune, an invalid byte yielding U+FFFD (then dropped by
// the cleaner).  Case mapping is Go's unicode.ToLower (the simple mapping),
// decomposition the canonical (NFD) one with canonical reordering.
#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <unordered_map>

#include "../../../include/futon_hip.h"
#include "../../../include/futon_native.hpp"
#include "host_common.h"

namespace {
#include "unicode_tables.inc"

constexpr uint32_t kCtrl = 1, kPunct = 2, kZs = 4, kMn = 8;

uint32_t uclass(uint32_t r) {
    size_t lo = 0, hi = sizeof kClassRanges / sizeof kClassRanges[0];
    while (lo < hi) {
        const size_t mid = (lo + hi) / 2;
        if (kClassRanges[mid][1] < r) lo = mid + 1;
        else hi = mid;
    }
    if (lo < sizeof kClassRanges / sizeof kClassRanges[0] && kClassRanges[lo][0] <= r) return kClassRanges[lo][2];
    return 0;
}

template <size_t N, size_t W>
const uint32_t *find_cp(const uint32_t (&tab)[N][W], uint32_t r) {
    size_t lo = 0, hi = N;
    while (lo < hi) {
        const size_t mid = (lo + hi) / 2;
        if (tab[mid][0] < r) lo = mid + 1;
        else hi = mid;
    }
    return lo < N && tab[lo][0] == r ? tab[lo] : nullptr;
}

uint32_t to_lower(uint32_t r) {
    if (r < 0x80) return (r >= 'A' && r <= 'Z') ? r + 32 : r;
    const uint32_t *e = find_cp(kLower, r);
    return e ? e[1] : r;
}

uint32_t ccc(uint32_t r) {
    if (r < 0x300) return 0;
    const uint32_t *e = find_cp(kCcc, r);
    return e ? e[1] : 0;
}

// Go's utf8.DecodeRuneInString: invalid or overlong sequences, surrogates
// and values above U+10FFFF decode as U+FFFD with width 1.
uint32_t decode_rune(const std::string &s, size_t i, size_t &width) {
    const unsigned char c0 = (unsigned char)s[i];
    width = 1;
    if (c0 < 0x80) return c0;
    const size_t n = s.size() - i;
    auto cont = [&](size_t k) { return k < n && ((unsigned char)s[i + k] & 0xC0) == 0x80; };
    if (c0 >= 0xC2 && c0 <= 0xDF) {
        if (!cont(1)) return 0xFFFD;
        width = 2;
        return (uint32_t)(c0 & 0x1F) << 6 | ((unsigned char)s[i + 1] & 0x3F);
    }
    if (c0 >= 0xE0 && c0 <= 0xEF) {
        if (!cont(1) || !cont(2)) return 0xFFFD;
        const unsigned char c1 = (unsigned char)s[i + 1];
        if ((c0 == 0xE0 && c1 < 0xA0) || (c0 == 0xED && c1 > 0x9F)) return 0xFFFD;  // overlong / surrogate
        width = 3;
        return (uint32_t)(c0 & 0x0F) << 12 | (uint32_t)(c1 & 0x3F) << 6 | ((unsigned char)s[i + 2] & 0x3F);
    }
    if (c0 >= 0xF0 && c0 <= 0xF4) {
        if (!cont(1) || !cont(2) || !cont(3)) return 0xFFFD;
        const unsigned char c1 = (unsigned char)s[i + 1];
        if ((c0 == 0xF0 && c1 < 0x90) || (c0 == 0xF4 && c1 > 0x8F)) return 0xFFFD;
        width = 4;
        return (uint32_t)(c0 & 0x07) << 18 | (uint32_t)(c1 & 0x3F) << 12 |
               (uint32_t)((unsigned char)s[i + 2] & 0x3F) << 6 | ((unsigned char)s[i + 3] & 0x3F);
    }
    return 0xFFFD;
}

std::vector<uint32_t> runes_of(const std::string &s) {
    std::vector<uint32_t> out;
    out.reserve(s.size());
    for (size_t i = 0; i < s.size();) {
        size_t w;
        out.push_back(decode_rune(s, i, w));
        i += w;
    }
    return out;
}

void put_utf8(std::string &o, uint32_t cp) {
    if (cp < 0x80) {
        o += (char)cp;
    } else if (cp < 0x800) {
        o += (char)(0xC0 | cp >> 6);
        o += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
        o += (char)(0xE0 | cp >> 12);
        o += (char)(0x80 | (cp >> 6 & 0x3F));
        o += (char)(0x80 | (cp & 0x3F));
    } else {
        o += (char)(0xF0 | cp >> 18);
        o += (char)(0x80 | (cp >> 12 & 0x3F));
        o += (char)(0x80 | (cp >> 6 & 0x3F));
        o += (char)(0x80 | (cp & 0x3F));
    }
}

// Canonical decomposition (NFD) of a rune sequence, with canonical ordering
// of each run of non-starters.
void nfd(const std::vector<uint32_t> &in, std::vector<uint32_t> &out) {
    out.clear();
    for (uint32_t r : in) {
        if (r >= 0xAC00 && r <= 0xD7A3) {  // Hangul syllable: L V (T)
            const uint32_t s = r - 0xAC00;
            out.push_back(0x1100 + s / 588);
            out.push_back(0x1161 + (s % 588) / 28);
            if (s % 28) out.push_back(0x11A7 + s % 28);
        } else if (const uint32_t *e = r < 0xC0 ? nullptr : find_cp(kDecomp, r)) {
            for (uint32_t k = 0; k < e[2]; k++) out.push_back(kDecompPool[e[1] + k]);
        } else {
            out.push_back(r);
        }
    }
    for (size_t i = 0; i < out.size();) {
        if (!ccc(out[i])) {
            i++;
            continue;
        }
        size_t j = i;
        while (j < out.size() && ccc(out[j])) j++;
        std::stable_sort(out.begin() + (long)i, out.begin() + (long)j,
                         [](uint32_t a, uint32_t b) { return ccc(a) < ccc(b); });
        i = j;
    }
}

// tokenizer.go:327-333 — space, \t, \n, \r or Zs.
bool is_whitespace(uint32_t r) { return r == ' ' || r == '\t' || r == '\n' || r == '\r' || (uclass(r) & kZs); }
// tokenizer.go:337-344 — Go's unicode.C (Cc, Cf, Co, Cs) except \t \n \r.
bool is_control(uint32_t r) { return r != '\t' && r != '\n' && r != '\r' && (uclass(r) & kCtrl); }
// tokenizer.go:349-354 — the four ASCII symbol/punct ranges plus P*.
bool is_punct(uint32_t r) {
    if ((r >= 33 && r <= 47) || (r >= 58 && r <= 64) || (r >= 91 && r <= 96) || (r >= 123 && r <= 126)) return true;
    return uclass(r) & kPunct;
}
// tokenizer.go:358-371 — CJK ideograph blocks.
bool is_cjk(uint32_t r) {
    return (r >= 0x4E00 && r <= 0x9FFF) || (r >= 0x3400 && r <= 0x4DBF) || (r >= 0x20000 && r <= 0x2A6DF) ||
           (r >= 0x2A700 && r <= 0x2B73F) || (r >= 0x2B740 && r <= 0x2B81F) || (r >= 0x2B820 && r <= 0x2CEAF) ||
           (r >= 0xF900 && r <= 0xFAFF) || (r >= 0x2F800 && r <= 0x2FA1F);
}
// Go's unicode.IsSpace, which strings.Fields splits on.
bool go_is_space(uint32_t r) {
    if (r <= 0xFF) return r == '\t' || r == '\n' || r == '\v' || r == '\f' || r == '\r' || r == ' ' || r == 0x85 || r == 0xA0;
    return r == 0x1680 || (r >= 0x2000 && r <= 0x200A) || r == 0x2028 || r == 0x2029 || r == 0x202F || r == 0x205F ||
           r == 0x3000;
}

}  // namespace

namespace futon {
namespace native {

using fh::raise;

Tokenizer::Tokenizer(const std::string &vocabPath, TokenizerConfig cfg) : cfg_(std::move(cfg)) {
    std::string raw, err;
    if (!fh::read_file(vocabPath, raw, err)) raise(FH_EINVAL, "tokenizer: open vocab: %s", err.c_str());
    // applyDefaults (tokenizer.go:35-54)
    if (cfg_.MaxInputCharsPerWord == 0) cfg_.MaxInputCharsPerWord = 100;
    if (cfg_.ClsToken.empty()) cfg_.ClsToken = "[CLS]";
    if (cfg_.SepToken.empty()) cfg_.SepToken = "[SEP]";
    if (cfg_.UnkToken.empty()) cfg_.UnkToken = "[UNK]";
    if (cfg_.PadToken.empty()) cfg_.PadToken = "[PAD]";
    if (cfg_.MaskToken.empty()) cfg_.MaskToken = "[MASK]";
    // One token per line (bufio.ScanLines: '\n'-separated, a final line
    // without newline kept when non-empty), trailing "\r\n" trimmed; a
    // repeated token keeps its last line number.
    int id = 0;
    size_t pos = 0;
    while (pos < raw.size()) {
        size_t nl = raw.find('\n', pos);
        const bool last = nl == std::string::npos;
        if (last) nl = raw.size();
        if (nl - pos > (1u << 20)) raise(FH_EINVAL, "tokenizer: scan vocab: bufio.Scanner: token too long");
        std::string tok = raw.substr(pos, nl - pos);
        while (!tok.empty() && (tok.back() == '\r' || tok.back() == '\n')) tok.pop_back();
        vocab_[tok] = id++;
        pos = last ? raw.size() : nl + 1;
    }
    if (id == 0) raise(FH_EINVAL, "tokenizer: vocab %s is empty", vocabPath.c_str());
    const std::pair<const std::string *, int *> sp[] = {{&cfg_.ClsToken, &clsID_},
                                                         {&cfg_.SepToken, &sepID_},
                                                         {&cfg_.UnkToken, &unkID_},
                                                         {&cfg_.PadToken, &padID_},
                                                         {&cfg_.MaskToken, &maskID_}};
    for (const auto &s : sp) {
        auto it = vocab_.find(*s.first);
        if (it == vocab_.end()) raise(FH_EINVAL, "tokenizer: special token \"%s\" not in vocab", s.first->c_str());
        *s.second = it->second;
        specials_.emplace_back(*s.first, it->second);
    }
}

// tokenizer.go:183-214: leftmost literal match on the raw bytes, the longer
// literal winning a tie; text between matches is an independent segment.
std::vector<Tokenizer::Segment> Tokenizer::splitSpecials(const std::string &text) const {
    std::vector<Segment> segs;
    size_t at = 0;
    while (at < text.size()) {
        size_t best = std::string::npos, bestLen = 0;
        int bestID = -1;
        for (const auto &sp : specials_) {
            const size_t i = text.find(sp.first, at);
            if (i != std::string::npos &&
                (best == std::string::npos || i < best || (i == best && sp.first.size() > bestLen))) {
                best = i;
                bestID = sp.second;
                bestLen = sp.first.size();
            }
        }
        if (best == std::string::npos) {
            segs.push_back({text.substr(at), -1});
            break;
        }
        if (best > at) segs.push_back({text.substr(at, best - at), -1});
        segs.push_back({std::string(), bestID});
        at = best + bestLen;
    }
    return segs;
}

// tokenizer.go:218-264
std::vector<std::string> Tokenizer::basicTokenize(const std::string &text) const {
    std::vector<uint32_t> cleaned;
    cleaned.reserve(text.size() + text.size() / 4);
    for (size_t i = 0; i < text.size();) {
        size_t w;
        const uint32_t r = decode_rune(text, i, w);
        i += w;
        if (r == 0 || r == 0xFFFD || is_control(r)) continue;
        if (is_whitespace(r)) {
            cleaned.push_back(' ');
        } else if (cfg_.TokenizeChineseChars && is_cjk(r)) {
            cleaned.push_back(' ');
            cleaned.push_back(r);
            cleaned.push_back(' ');
        } else {
            cleaned.push_back(r);
        }
    }
    if (cfg_.DoLowerCase) {
        for (uint32_t &r : cleaned) r = to_lower(r);
        std::vector<uint32_t> d;
        nfd(cleaned, d);
        cleaned.clear();
        for (uint32_t r : d)
            if (!(uclass(r) & kMn)) cleaned.push_back(r);
    }
    std::vector<std::string> words;
    std::string cur;
    bool open = false;
    auto flush = [&]() {
        if (open) words.push_back(cur);
        cur.clear();
        open = false;
    };
    for (uint32_t r : cleaned) {
        if (go_is_space(r)) {
            flush();
        } else if (is_punct(r)) {
            flush();
            std::string p;
            put_utf8(p, r);
            words.push_back(p);
        } else {
            put_utf8(cur, r);
            open = true;
        }
    }
    flush();
    return words;
}

// tokenizer.go:270-298
void Tokenizer::wordPiece(const std::string &word, std::vector<int> &out) const {
    const std::vector<uint32_t> rs = runes_of(word);
    if ((int64_t)rs.size() > cfg_.MaxInputCharsPerWord) {
        out.push_back(unkID_);
        return;
    }
    std::vector<size_t> off(rs.size() + 1, 0);  // byte offset of rune i in word
    for (size_t i = 0, b = 0; i < rs.size(); i++) {
        size_t w;
        decode_rune(word, b, w);
        b += w;
        off[i + 1] = b;
    }
    const size_t mark = out.size();
    size_t start = 0;
    std::string sub;
    while (start < rs.size()) {
        size_t end = rs.size();
        int curID = -1;
        while (end > start) {
            sub.assign(start > 0 ? "##" : "");
            sub.append(word, off[start], off[end] - off[start]);
            auto it = vocab_.find(sub);
            if (it != vocab_.end()) {
                curID = it->second;
                break;
            }
            end--;
        }
        if (curID < 0) {
            out.resize(mark);
            out.push_back(unkID_);
            return;
        }
        out.push_back(curID);
        start = end;
    }
}

// tokenizer.go:146-176
std::vector<int> Tokenizer::Encode(const std::string &text, int maxSeqLen) const {
    if (maxSeqLen < 2) maxSeqLen = 2;
    std::vector<int> ids;
    ids.reserve(64);
    ids.push_back(clsID_);
    const int budget = maxSeqLen - 2;
    std::vector<int> pieces;
    for (const Segment &seg : splitSpecials(text)) {
        if (seg.specialID >= 0) {
            if ((int)ids.size() - 1 >= budget) break;
            ids.push_back(seg.specialID);
            continue;
        }
        bool stop = false;
        for (const std::string &w : basicTokenize(seg.text)) {
            if ((int)ids.size() - 1 >= budget) {
                stop = true;
                break;
            }
            pieces.clear();
            wordPiece(w, pieces);
            for (int p : pieces) {
                if ((int)ids.size() - 1 >= budget) {
                    stop = true;
                    break;
                }
                ids.push_back(p);
            }
            if (stop) break;
        }
        if (stop) break;
    }
    ids.push_back(sepID_);
    return ids;
}

}  // namespace native
}  // namespace futon
