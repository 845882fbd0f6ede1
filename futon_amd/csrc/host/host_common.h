// Internal plumbing shared by the host-side C++ layer (pack loading,
// tokenizer, provider) and the device orchestrator: thread-local error
// detail, a small JSON reader with Go encoding/json field semantics, and
// SHA-256 for manifest verification.
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "../../../include/futon_native.hpp"  // fh::Error

namespace fh {

// Records printf-style detail for fh_last_error() and returns code.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
const std::string &last_error();

// Throws fh::Error(code, printf-style message).
[[noreturn]] void raise(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

// ── JSON ──
struct Json {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    std::string s;  // String value, or the literal text of a Number
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;  // in document order

    // Member lookup as Go's encoding/json resolves a struct field: the last
    // exact-case match, else the last case-insensitive match; null if absent.
    const Json *get(const std::string &key) const;
};
// Parses a complete JSON document; throws Error(FH_EINVAL) with a message
// prefixed by `what` on malformed input.
Json parse_json(const char *data, size_t len, const std::string &what);

// Field decoding with encoding/json's rules: a JSON null (or absent member)
// leaves the destination unchanged; a wrong type is an error naming field.
void json_int(const Json *v, const char *field, int64_t &dst);
void json_float(const Json *v, const char *field, double &dst);
void json_bool(const Json *v, const char *field, bool &dst);
void json_string(const Json *v, const char *field, std::string &dst);

// ── SHA-256 (FIPS 180-4) ──
std::string sha256_file_hex(const std::string &path);  // throws on I/O error
std::string sha256_hex(const void *data, size_t len);

bool read_file(const std::string &path, std::string &out, std::string &err);
std::string join_path(const std::string &dir, const std::string &name);

}  // namespace fh
