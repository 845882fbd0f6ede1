// futon_embed: the `futon embed` command (cmd/futon/main.go:68-111) on the
// MI355X path, built from the C++ host layer for hosts without Go.
//
//   futon_embed [-model id] [-models-dir dir] [-dims n] [text ...]
//
// Prints one JSON array per input text, in encoding/json's float32 format;
// with no text arguments it reads one text per line from standard input.
// Errors go to standard error as "futon: <message>" with exit status 1; a
// bad flag prints the usage with exit status 2.  SIGINT cancels the forward
// at its next layer boundary (signal.NotifyContext in the reference).
#include <csignal>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <charconv>
#include <cmath>
#include <iostream>
#include <string>
#include <vector>

#include "futon_native.hpp"

namespace {

volatile int32_t g_interrupted = 0;
void on_sigint(int) { g_interrupted = 1; }

void usage() {
    fputs("usage:\n  futon_embed [-model id] [-models-dir dir] [-dims n] [text ...]\n", stderr);
}

// encoding/json's float32 encoding (the shortest round-trip form: 'f' for
// 1e-6 <= |x| < 1e21, else 'e' with a one-digit negative exponent written
// without its leading zero).
void append_float32(std::string &out, float f) {
    char buf[64];
    const float a = std::fabs(f);
    const bool sci = a != 0.f && (a < 1e-6f || a >= 1e21f);
    auto r = std::to_chars(buf, buf + sizeof buf, f, sci ? std::chars_format::scientific : std::chars_format::fixed);
    std::string s(buf, r.ptr);
    if (sci) {
        const size_t n = s.size();
        if (n >= 4 && s[n - 4] == 'e' && s[n - 3] == '-' && s[n - 2] == '0') s.erase(n - 2, 1);
    }
    out += s;
}

// Go's flag package: -name value, -name=value, --name forms; parsing stops
// at the first non-flag argument or after "--".
bool parse_flags(int argc, char **argv, futon::Options &o, std::vector<std::string> &rest) {
    int i = 1;
    for (; i < argc; ++i) {
        std::string a = argv[i];
        if (a == "--") {
            ++i;
            break;
        }
        if (a.size() < 2 || a[0] != '-') break;
        std::string name = a.substr(a[1] == '-' ? 2 : 1), val;
        bool has_val = false;
        if (const size_t eq = name.find('='); eq != std::string::npos) {
            val = name.substr(eq + 1);
            name = name.substr(0, eq);
            has_val = true;
        }
        if (name == "h" || name == "help") {
            usage();
            exit(0);
        }
        if (name != "model" && name != "models-dir" && name != "dims") {
            fprintf(stderr, "flag provided but not defined: -%s\n", name.c_str());
            return false;
        }
        if (!has_val) {
            if (i + 1 >= argc) {
                fprintf(stderr, "flag needs an argument: -%s\n", name.c_str());
                return false;
            }
            val = argv[++i];
        }
        if (name == "model") {
            o.Model = val;
        } else if (name == "models-dir") {
            o.ModelsDir = val;
        } else {
            char *end = nullptr;
            const long d = strtol(val.c_str(), &end, 0);
            if (val.empty() || *end || d < INT32_MIN || d > INT32_MAX) {
                fprintf(stderr, "invalid value \"%s\" for flag -dims: parse error\n", val.c_str());
                return false;
            }
            o.Dimensions = (int)d;
        }
    }
    for (; i < argc; ++i) rest.emplace_back(argv[i]);
    return true;
}

}  // namespace

int main(int argc, char **argv) {
    futon::Options opts;
    opts.Model = futon::DefaultModel;
    std::vector<std::string> texts;
    if (!parse_flags(argc, argv, opts, texts)) {
        usage();
        return 2;
    }
    try {
        if (texts.empty()) {
            std::string line;
            while (std::getline(std::cin, line)) {
                if (!line.empty() && line.back() == '\r') line.pop_back();  // bufio.ScanLines
                texts.push_back(line);
            }
        }
        if (texts.empty()) throw fh::Error(FH_EINVAL, "no text to embed");
        auto e = futon::New(opts);
        std::signal(SIGINT, on_sigint);
        futon::Context ctx(&g_interrupted);
        const auto vecs = e->EmbedBatch(&ctx, texts);
        e->Close();
        std::string out;
        for (const auto &v : vecs) {
            out.clear();
            out += '[';
            for (size_t j = 0; j < v.size(); ++j) {
                if (j) out += ',';
                append_float32(out, v[j]);
            }
            out += "]\n";
            fwrite(out.data(), 1, out.size(), stdout);
        }
        fflush(stdout);
    } catch (const std::exception &ex) {
        fprintf(stderr, "futon: %s\n", ex.what());
        return 1;
    }
    return 0;
}
