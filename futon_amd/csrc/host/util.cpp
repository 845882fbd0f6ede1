// JSON reader, SHA-256 and file helpers for the host layer.
#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "../../../include/futon_hip.h"
#include "host_common.h"

namespace fh {

// ───────────────────────────── JSON ─────────────────────────────

namespace {

struct Parser {
    const char *p, *end, *begin;
    std::string what;
    int depth = 0;

    [[noreturn]] void bad(const char *msg) {
        raise(FH_EINVAL, "%s: %s at offset %ld", what.c_str(), msg, (long)(p - begin));
    }
    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
    }
    bool lit(const char *s) {
        const size_t n = strlen(s);
        if ((size_t)(end - p) >= n && memcmp(p, s, n) == 0) {
            p += n;
            return true;
        }
        return false;
    }
    static void put_utf8(std::string &o, uint32_t cp) {
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
    int hex4() {
        if (end - p < 4) bad("truncated \\u escape");
        int v = 0;
        for (int i = 0; i < 4; i++) {
            const char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= c - '0';
            else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
            else bad("invalid \\u escape");
        }
        return v;
    }
    std::string str() {
        if (p >= end || *p != '"') bad("expected string");
        p++;
        std::string o;
        for (;;) {
            if (p >= end) bad("unterminated string");
            const unsigned char c = (unsigned char)*p;
            if (c == '"') {
                p++;
                return o;
            }
            if (c < 0x20) bad("control character in string");
            if (c != '\\') {
                o += (char)c;
                p++;
                continue;
            }
            p++;
            if (p >= end) bad("unterminated escape");
            const char e = *p++;
            switch (e) {
            case '"': o += '"'; break;
            case '\\': o += '\\'; break;
            case '/': o += '/'; break;
            case 'b': o += '\b'; break;
            case 'f': o += '\f'; break;
            case 'n': o += '\n'; break;
            case 'r': o += '\r'; break;
            case 't': o += '\t'; break;
            case 'u': {
                uint32_t cp = (uint32_t)hex4();
                if (cp >= 0xD800 && cp < 0xDC00) {
                    const char *save = p;
                    if (end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
                        p += 2;
                        const uint32_t lo = (uint32_t)hex4();
                        if (lo >= 0xDC00 && lo < 0xE000) {
                            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                        } else {
                            p = save;
                            cp = 0xFFFD;
                        }
                    } else {
                        cp = 0xFFFD;
                    }
                } else if (cp >= 0xDC00 && cp < 0xE000) {
                    cp = 0xFFFD;
                }
                put_utf8(o, cp);
                break;
            }
            default: bad("invalid escape");
            }
        }
    }
    std::string number() {
        const char *s = p;
        if (p < end && *p == '-') p++;
        if (p >= end) bad("truncated number");
        if (*p == '0') {
            p++;
        } else if (*p >= '1' && *p <= '9') {
            while (p < end && *p >= '0' && *p <= '9') p++;
        } else {
            bad("invalid number");
        }
        if (p < end && *p == '.') {
            p++;
            if (p >= end || !(*p >= '0' && *p <= '9')) bad("invalid number");
            while (p < end && *p >= '0' && *p <= '9') p++;
        }
        if (p < end && (*p == 'e' || *p == 'E')) {
            p++;
            if (p < end && (*p == '+' || *p == '-')) p++;
            if (p >= end || !(*p >= '0' && *p <= '9')) bad("invalid number");
            while (p < end && *p >= '0' && *p <= '9') p++;
        }
        return std::string(s, p);
    }
    Json value() {
        if (++depth > 1000) bad("nesting too deep");
        ws();
        if (p >= end) bad("unexpected end of input");
        Json v;
        const char c = *p;
        if (c == '{') {
            p++;
            v.kind = Json::Object;
            ws();
            if (p < end && *p == '}') {
                p++;
            } else {
                for (;;) {
                    ws();
                    std::string k = str();
                    ws();
                    if (p >= end || *p != ':') bad("expected ':'");
                    p++;
                    Json m = value();
                    v.obj.emplace_back(std::move(k), std::move(m));
                    ws();
                    if (p < end && *p == ',') {
                        p++;
                        continue;
                    }
                    if (p < end && *p == '}') {
                        p++;
                        break;
                    }
                    bad("expected ',' or '}'");
                }
            }
        } else if (c == '[') {
            p++;
            v.kind = Json::Array;
            ws();
            if (p < end && *p == ']') {
                p++;
            } else {
                for (;;) {
                    v.arr.push_back(value());
                    ws();
                    if (p < end && *p == ',') {
                        p++;
                        continue;
                    }
                    if (p < end && *p == ']') {
                        p++;
                        break;
                    }
                    bad("expected ',' or ']'");
                }
            }
        } else if (c == '"') {
            v.kind = Json::String;
            v.s = str();
        } else if (c == 't' || c == 'f' || c == 'n') {
            if (lit("true")) {
                v.kind = Json::Bool;
                v.b = true;
            } else if (lit("false")) {
                v.kind = Json::Bool;
            } else if (lit("null")) {
                v.kind = Json::Null;
            } else {
                bad("invalid literal");
            }
        } else {
            v.kind = Json::Number;
            v.s = number();
        }
        depth--;
        return v;
    }
};

bool ieq(const std::string &a, const std::string &b) {
    if (a.size() != b.size()) return false;
    for (size_t i = 0; i < a.size(); i++) {
        char x = a[i], y = b[i];
        if (x >= 'A' && x <= 'Z') x = (char)(x - 'A' + 'a');
        if (y >= 'A' && y <= 'Z') y = (char)(y - 'A' + 'a');
        if (x != y) return false;
    }
    return true;
}

const char *kind_name(Json::Kind k) {
    switch (k) {
    case Json::Null: return "null";
    case Json::Bool: return "bool";
    case Json::Number: return "number";
    case Json::String: return "string";
    case Json::Array: return "array";
    default: return "object";
    }
}

}  // namespace

const Json *Json::get(const std::string &key) const {
    const Json *exact = nullptr, *fold = nullptr;
    for (const auto &kv : obj) {
        if (kv.first == key) exact = &kv.second;
        else if (ieq(kv.first, key)) fold = &kv.second;
    }
    return exact ? exact : fold;
}

Json parse_json(const char *data, size_t len, const std::string &what) {
    Parser ps{data, data + len, data, what};
    Json v = ps.value();
    ps.ws();
    if (ps.p != ps.end) ps.bad("invalid character after top-level value");
    return v;
}

void json_int(const Json *v, const char *field, int64_t &dst) {
    if (!v || v->kind == Json::Null) return;
    if (v->kind != Json::Number)
        raise(FH_EINVAL, "json: cannot unmarshal %s into field %s of type int", kind_name(v->kind), field);
    errno = 0;
    char *e = nullptr;
    const long long x = strtoll(v->s.c_str(), &e, 10);
    if (errno || !e || *e)
        raise(FH_EINVAL, "json: cannot unmarshal number %s into field %s of type int", v->s.c_str(), field);
    dst = x;
}

void json_float(const Json *v, const char *field, double &dst) {
    if (!v || v->kind == Json::Null) return;
    if (v->kind != Json::Number)
        raise(FH_EINVAL, "json: cannot unmarshal %s into field %s of type float64", kind_name(v->kind), field);
    errno = 0;
    char *e = nullptr;
    const double x = strtod(v->s.c_str(), &e);
    if (errno == ERANGE && (x > 1.0 || x < -1.0))
        raise(FH_EINVAL, "json: cannot unmarshal number %s into field %s of type float64", v->s.c_str(), field);
    dst = x;
}

void json_bool(const Json *v, const char *field, bool &dst) {
    if (!v || v->kind == Json::Null) return;
    if (v->kind != Json::Bool)
        raise(FH_EINVAL, "json: cannot unmarshal %s into field %s of type bool", kind_name(v->kind), field);
    dst = v->b;
}

void json_string(const Json *v, const char *field, std::string &dst) {
    if (!v || v->kind == Json::Null) return;
    if (v->kind != Json::String)
        raise(FH_EINVAL, "json: cannot unmarshal %s into field %s of type string", kind_name(v->kind), field);
    dst = v->s;
}

// ───────────────────────────── SHA-256 ─────────────────────────────

namespace {

struct Sha256 {
    uint32_t h[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a, 0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    uint8_t buf[64];
    size_t nbuf = 0;
    uint64_t total = 0;

    static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
    void block(const uint8_t *b) {
        static const uint32_t K[64] = {
            0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
            0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
            0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
            0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
            0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
            0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
            0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
            0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};
        uint32_t w[64];
        for (int i = 0; i < 16; i++)
            w[i] = (uint32_t)b[4 * i] << 24 | (uint32_t)b[4 * i + 1] << 16 | (uint32_t)b[4 * i + 2] << 8 | b[4 * i + 3];
        for (int i = 16; i < 64; i++) {
            const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
            const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
            w[i] = w[i - 16] + s0 + w[i - 7] + s1;
        }
        uint32_t a = h[0], bb = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
        for (int i = 0; i < 64; i++) {
            const uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
            const uint32_t ch = (e & f) ^ (~e & g);
            const uint32_t t1 = hh + S1 + ch + K[i] + w[i];
            const uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
            const uint32_t mj = (a & bb) ^ (a & c) ^ (bb & c);
            const uint32_t t2 = S0 + mj;
            hh = g;
            g = f;
            f = e;
            e = d + t1;
            d = c;
            c = bb;
            bb = a;
            a = t1 + t2;
        }
        h[0] += a;
        h[1] += bb;
        h[2] += c;
        h[3] += d;
        h[4] += e;
        h[5] += f;
        h[6] += g;
        h[7] += hh;
    }
    void update(const uint8_t *d, size_t n) {
        total += n;
        if (nbuf) {
            const size_t k = std::min<size_t>(64 - nbuf, n);
            memcpy(buf + nbuf, d, k);
            nbuf += k;
            d += k;
            n -= k;
            if (nbuf == 64) {
                block(buf);
                nbuf = 0;
            }
        }
        while (n >= 64) {
            block(d);
            d += 64;
            n -= 64;
        }
        if (n) {
            memcpy(buf, d, n);
            nbuf = n;
        }
    }
    std::string hex() {
        const uint64_t bits = total * 8;
        const uint8_t one = 0x80, zero = 0;
        update(&one, 1);
        while (nbuf != 56) update(&zero, 1);
        uint8_t len[8];
        for (int i = 0; i < 8; i++) len[i] = (uint8_t)(bits >> (56 - 8 * i));
        update(len, 8);
        static const char *dig = "0123456789abcdef";
        std::string o;
        for (int i = 0; i < 8; i++)
            for (int sh = 28; sh >= 0; sh -= 4) o += dig[(h[i] >> sh) & 0xF];
        return o;
    }
};

}  // namespace

std::string sha256_hex(const void *data, size_t len) {
    Sha256 s;
    s.update((const uint8_t *)data, len);
    return s.hex();
}

std::string sha256_file_hex(const std::string &path) {
    FILE *f = fopen(path.c_str(), "rb");
    if (!f) raise(FH_EINVAL, "open %s: %s", path.c_str(), strerror(errno));
    Sha256 s;
    std::vector<uint8_t> buf(1 << 20);
    size_t n;
    while ((n = fread(buf.data(), 1, buf.size(), f)) > 0) s.update(buf.data(), n);
    const bool err = ferror(f) != 0;
    fclose(f);
    if (err) raise(FH_EINVAL, "read %s: I/O error", path.c_str());
    return s.hex();
}

bool read_file(const std::string &path, std::string &out, std::string &err) {
    FILE *f = fopen(path.c_str(), "rb");
    if (!f) {
        err = "open " + path + ": " + strerror(errno);
        return false;
    }
    out.clear();
    char buf[1 << 16];
    size_t n;
    while ((n = fread(buf, 1, sizeof buf, f)) > 0) out.append(buf, n);
    const bool bad = ferror(f) != 0;
    fclose(f);
    if (bad) {
        err = "read " + path + ": I/O error";
        return false;
    }
    return true;
}

std::string join_path(const std::string &dir, const std::string &name) {
    if (dir.empty()) return name;
    return dir.back() == '/' ? dir + name : dir + "/" + name;
}

}  // namespace fh
