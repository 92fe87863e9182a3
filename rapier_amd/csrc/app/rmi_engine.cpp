// rmi_engine - the engine executable: the reference's qwythos command line (flags of qw:2815-2900) over librapier_mi.
//
//   rmi_engine --model FILE.gguf --serve                  JSON-lines serving on stdin/stdout (rmi_serve_engine)
//   rmi_engine --model FILE.gguf --tokens id,id --n N     ingest the prompt, generate N tokens (greedy MTP), print them
//
// Other flags: --device D (default: the device with the most memory), --eos ID (the id that ends a served generation,
// 248046 by default).  --split (the reference's two-GPU layer split) is rejected.  Every flag also takes the
// --flag=value form.
// Environment, as the reference reads it: QWYTHOS_MAXCTX (context length, 1024..65536, default 65536), QWYTHOS_BN
// (ingest chunk, 2..16), QWYTHOS_NOBATCH (token-by-token ingest), QWYTHOS_NOMTP (the CLI generates without MTP).
#include <hip/hip_runtime_api.h>

#include <cerrno>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../../include/rapier_mi.h"
#include "../../../include/rapier_mi_engine.h"

namespace {

// ---- command line -------------------------------------------------------------------------------------------------
// The flags are rows of one table; a row names the option, what its value parses as and where the value goes.  The
// parser walks argv once, looks each word up in the table and hands the value text to the row's converter, so a new
// flag is one row.

struct Options {
    std::string model;
    std::vector<int> tokens;
    bool serve = false;
    long ngen = 32;
    long device = -1;
    double split = 0.0;
    long eos = -1;
};

enum class Kind { Text, Integer, Real, Switch, IdList };

struct Flag {
    const char* name;
    Kind kind;
    const char* meta;  // value placeholder in the usage text ("" for a switch)
    void* (*slot)(Options&);
};

const Flag kFlags[] = {
    {"--model", Kind::Text, "FILE.gguf", [](Options& o) -> void* { return &o.model; }},
    {"--serve", Kind::Switch, "", [](Options& o) -> void* { return &o.serve; }},
    {"--tokens", Kind::IdList, "ID,ID,...", [](Options& o) -> void* { return &o.tokens; }},
    {"--n", Kind::Integer, "N", [](Options& o) -> void* { return &o.ngen; }},
    {"--device", Kind::Integer, "D", [](Options& o) -> void* { return &o.device; }},
    {"--eos", Kind::Integer, "ID", [](Options& o) -> void* { return &o.eos; }},
    {"--split", Kind::Real, "FRAC", [](Options& o) -> void* { return &o.split; }},
};

void usage(FILE* f) {
    std::fprintf(f, "usage: rmi_engine");
    for (const Flag& fl : kFlags) std::fprintf(f, " [%s%s%s]", fl.name, *fl.meta ? " " : "", fl.meta);
    std::fprintf(f, "\n  needs --model and either --serve or --tokens\n");
}

bool to_long(const char* s, long* out) {
    if (!*s) return false;
    char* end = nullptr;
    errno = 0;
    const long v = std::strtol(s, &end, 10);
    if (errno || *end) return false;
    *out = v;
    return true;
}

// Stores `text` into the row's slot; false (with a message) when the text is not a value of the row's kind.
bool assign(const Flag& fl, const char* text, Options& o) {
    void* p = fl.slot(o);
    switch (fl.kind) {
        case Kind::Text:
            *static_cast<std::string*>(p) = text;
            return true;
        case Kind::Switch:
            *static_cast<bool*>(p) = true;
            return true;
        case Kind::Integer:
            if (to_long(text, static_cast<long*>(p))) return true;
            break;
        case Kind::Real: {
            char* end = nullptr;
            const double v = std::strtod(text, &end);
            if (*text && !*end) {
                *static_cast<double*>(p) = v;
                return true;
            }
            break;
        }
        case Kind::IdList: {
            auto* ids = static_cast<std::vector<int>*>(p);
            std::string word;
            for (const char* c = text;; ++c) {
                if (*c && *c != ',') {
                    word.push_back(*c);
                    continue;
                }
                long id = 0;
                if (!to_long(word.c_str(), &id) || id < 0 || id > 0x7fffffffL) {
                    std::fprintf(stderr, "rmi_engine: %s: '%s' is not a token id\n", fl.name, word.c_str());
                    return false;
                }
                ids->push_back(static_cast<int>(id));
                word.clear();
                if (!*c) return true;
            }
        }
    }
    std::fprintf(stderr, "rmi_engine: %s: bad value '%s'\n", fl.name, text);
    return false;
}

// 0 on success, otherwise the process exit code (2, a usage error).
int parse(int argc, char** argv, Options& o) {
    int k = 1;
    while (k < argc) {
        const char* word = argv[k++];
        const char* eq = std::strchr(word, '=');
        const size_t len = eq ? static_cast<size_t>(eq - word) : std::strlen(word);
        const Flag* fl = nullptr;
        for (const Flag& cand : kFlags)
            if (std::strlen(cand.name) == len && std::strncmp(cand.name, word, len) == 0) fl = &cand;
        if (!fl) {
            std::fprintf(stderr, "rmi_engine: unrecognised option '%s'\n", word);
            usage(stderr);
            return 2;
        }
        const char* value = "";
        if (fl->kind == Kind::Switch) {
            if (eq) {
                std::fprintf(stderr, "rmi_engine: %s takes no value\n", fl->name);
                return 2;
            }
        } else if (eq) {
            value = eq + 1;
        } else if (k < argc) {
            value = argv[k++];
        } else {
            std::fprintf(stderr, "rmi_engine: %s needs a value (%s)\n", fl->name, fl->meta);
            return 2;
        }
        if (!assign(*fl, value, o)) return 2;
    }
    return 0;
}

int env_int(const char* name, int lo, int hi, int dflt) {
    const char* s = std::getenv(name);
    long v = 0;
    if (!s || !to_long(s, &v)) return dflt;
    return v >= lo && v <= hi ? static_cast<int>(v) : dflt;
}

// ---- device --------------------------------------------------------------------------------------------------------
// Without --device the engine runs on the GPU with the largest memory; among equals the lowest ordinal wins.  Returns
// the ordinal, or -1 with a message.
int choose_device(long requested) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count < 1) {
        std::fprintf(stderr, "rmi_engine: no GPU\n");
        return -1;
    }
    if (requested >= 0) {
        if (requested >= count) {
            std::fprintf(stderr, "rmi_engine: --device %ld, but only %d GPU(s) are visible\n", requested, count);
            return -1;
        }
        return static_cast<int>(requested);
    }
    std::vector<size_t> mem(static_cast<size_t>(count), 0);
    for (int d = 0; d < count; ++d) {
        size_t bytes = 0;
        if (hipDeviceTotalMem(&bytes, d) == hipSuccess) mem[static_cast<size_t>(d)] = bytes;
    }
    int pick = 0;
    for (int d = 1; d < count; ++d)
        if (mem[static_cast<size_t>(d)] > mem[static_cast<size_t>(pick)]) pick = d;
    return pick;
}

int die(const char* what) {
    std::fprintf(stderr, "rmi_engine: %s: %s\n", what, rmi_last_error());
    return 1;
}

}  // namespace

int main(int argc, char** argv) {
    Options o;
    if (const int rc = parse(argc, argv, o)) return rc;
    if (o.model.empty() || (!o.serve && (o.tokens.empty() || o.ngen < 1))) {
        usage(stderr);
        return 2;
    }
    if (o.split > 0.0) {
        std::fprintf(stderr, "--split: the two-GPU layer split is not supported; the engine runs on one GPU\n");
        return 2;
    }
    rmi_serve_options opt = rmi_serve_default_options();
    if (o.eos >= 0) opt.eos = static_cast<int>(o.eos);
    const int device = choose_device(o.device);
    if (device < 0) return 2;
    if (hipSetDevice(device) != hipSuccess) {
        std::fprintf(stderr, "rmi_engine: cannot select device %d\n", device);
        return 1;
    }
    const int max_ctx = env_int("QWYTHOS_MAXCTX", 1024, 65536, 65536);
    opt.batch = std::getenv("QWYTHOS_NOBATCH") ? 1 : env_int("QWYTHOS_BN", 2, 16, 16);
    const int ngen = static_cast<int>(o.ngen);

    const auto t0 = std::chrono::steady_clock::now();
    rmi_engine* e = nullptr;
    if (rmi_engine_create_gguf(o.model.c_str(), max_ctx, nullptr, &e) != RMI_OK) return die("load");
    const double load_s = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    if (o.serve) {
        std::fprintf(stderr, "rapier serve: ready (load %.2f s)\n", load_s);
        std::fflush(stderr);
        const int rc = rmi_serve_engine(e, &opt, 0, 1);
        rmi_engine_destroy(e);
        if (rc != RMI_OK) {
            std::fprintf(stderr, "rmi_engine: serve ended: %s\n", rmi_last_error());
            return 1;
        }
        return 0;
    }
    const auto t1 = std::chrono::steady_clock::now();
    int first = 0;
    if (rmi_engine_prefill_batch(e, o.tokens.data(), static_cast<int>(o.tokens.size()), opt.batch, &first) != RMI_OK)
        return die("prefill");
    const double prefill_s = std::chrono::duration<double>(std::chrono::steady_clock::now() - t1).count();
    std::vector<int> out(static_cast<size_t>(ngen));
    out[0] = first;
    rmi_gen_stats st{};
    if (ngen > 1) {
        rmi_gen_request req{};
        req.mode = std::getenv("QWYTHOS_NOMTP") ? RMI_GEN_GREEDY : RMI_GEN_MTP;
        req.n_gen = ngen - 1;
        req.use_graph = 1;
        if (rmi_engine_generate(e, &req, out.data() + 1, &st) != RMI_OK) return die("generate");
    }
    std::printf("{\"load_s\":%.3f,\"prefill_s\":%.3f,\"prompt\":%zu,\"tokens\":[", load_s, prefill_s,
                o.tokens.size());
    for (int i = 0; i < ngen; ++i) std::printf("%s%d", i ? "," : "", out[static_cast<size_t>(i)]);
    std::printf("],\"gen_ms\":%.3f,\"tok_s\":%.1f,\"rounds\":%d,\"accepted\":%d}\n", st.gpu_ms,
                st.gpu_ms > 0 ? (ngen - 1) / (st.gpu_ms / 1e3) : 0.0, st.rounds, st.accepted);
    rmi_engine_destroy(e);
    return 0;
}
