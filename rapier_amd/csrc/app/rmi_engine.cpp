// rmi_engine - the engine executable: the reference's qwythos command line (qw:2815-2900) over librapier_mi.
//
//   rmi_engine --model FILE.gguf --serve                  JSON-lines serving on stdin/stdout (rmi_serve_engine)
//   rmi_engine --model FILE.gguf --tokens id,id --n N     ingest the prompt, generate N tokens (greedy MTP), print them
//
// Other flags: --device D (default: the device with the most memory, as the reference picks it), --eos ID (the id that
// ends a served generation, 248046 by default).  --split (the reference's two-GPU layer split) is rejected.
// Environment, as the reference reads it: QWYTHOS_MAXCTX (context length, 1024..65536, default 65536), QWYTHOS_BN
// (ingest chunk, 2..16), QWYTHOS_NOBATCH (token-by-token ingest), QWYTHOS_NOMTP (the CLI generates without MTP).
#include <hip/hip_runtime_api.h>

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "../../../include/rapier_mi.h"
#include "../../../include/rapier_mi_engine.h"

namespace {

int env_int(const char* name, int lo, int hi, int dflt) {
    const char* s = std::getenv(name);
    if (!s) return dflt;
    const int v = std::atoi(s);
    return v >= lo && v <= hi ? v : dflt;
}

int die(const char* what) {
    std::fprintf(stderr, "rmi_engine: %s: %s\n", what, rmi_last_error());
    return 1;
}

}  // namespace

int main(int argc, char** argv) {
    std::string model;
    std::vector<int> tokens;
    bool serve = false;
    int ngen = 32, device = -1;
    float split = 0.0f;
    rmi_serve_options opt = rmi_serve_default_options();
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        auto need = [&](const char* flag) {
            if (i + 1 >= argc) {
                std::fprintf(stderr, "missing value for %s\n", flag);
                std::exit(2);
            }
            return std::string(argv[++i]);
        };
        if (a == "--model") model = need("--model");
        else if (a == "--n") ngen = std::atoi(need("--n").c_str());
        else if (a == "--split") split = static_cast<float>(std::atof(need("--split").c_str()));
        else if (a == "--device") device = std::atoi(need("--device").c_str());
        else if (a == "--eos") opt.eos = std::atoi(need("--eos").c_str());
        else if (a == "--serve") serve = true;
        else if (a == "--tokens") {
            const std::string s = need("--tokens");
            for (size_t p = 0; p < s.size();) {
                size_t c = s.find(',', p);
                if (c == std::string::npos) c = s.size();
                tokens.push_back(std::atoi(s.substr(p, c - p).c_str()));
                p = c + 1;
            }
        } else {
            std::fprintf(stderr, "unknown arg %s\n", a.c_str());
            return 2;
        }
    }
    if (model.empty() || (!serve && (tokens.empty() || ngen < 1))) {
        std::fprintf(stderr, "usage: rmi_engine --model file.gguf (--serve | --tokens id,id --n 32) [--device N] "
                             "[--eos ID]\n");
        return 2;
    }
    if (split > 0.0f) {
        std::fprintf(stderr, "--split: the two-GPU layer split is not supported; the engine runs on one GPU\n");
        return 2;
    }
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1) {
        std::fprintf(stderr, "rmi_engine: no GPU\n");
        return 1;
    }
    if (device < 0) {
        size_t best = 0;
        device = 0;
        for (int i = 0; i < ndev; ++i) {
            hipDeviceProp_t p{};
            if (hipGetDeviceProperties(&p, i) == hipSuccess && p.totalGlobalMem >= best) {
                best = p.totalGlobalMem;
                device = i;
            }
        }
    }
    if (device >= ndev) {
        std::fprintf(stderr, "device %d out of %d\n", device, ndev);
        return 2;
    }
    if (hipSetDevice(device) != hipSuccess) {
        std::fprintf(stderr, "rmi_engine: cannot select device %d\n", device);
        return 1;
    }
    const int max_ctx = env_int("QWYTHOS_MAXCTX", 1024, 65536, 65536);
    opt.batch = std::getenv("QWYTHOS_NOBATCH") ? 1 : env_int("QWYTHOS_BN", 2, 16, 16);

    const auto t0 = std::chrono::steady_clock::now();
    rmi_engine* e = nullptr;
    if (rmi_engine_create_gguf(model.c_str(), max_ctx, nullptr, &e) != RMI_OK) return die("load");
    const double load_s = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    if (serve) {
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
    if (rmi_engine_prefill_batch(e, tokens.data(), static_cast<int>(tokens.size()), opt.batch, &first) != RMI_OK)
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
    std::printf("{\"load_s\":%.3f,\"prefill_s\":%.3f,\"prompt\":%zu,\"tokens\":[", load_s, prefill_s, tokens.size());
    for (int i = 0; i < ngen; ++i) std::printf("%s%d", i ? "," : "", out[static_cast<size_t>(i)]);
    std::printf("],\"gen_ms\":%.3f,\"tok_s\":%.1f,\"rounds\":%d,\"accepted\":%d}\n", st.gpu_ms,
                st.gpu_ms > 0 ? (ngen - 1) / (st.gpu_ms / 1e3) : 0.0, st.rounds, st.accepted);
    rmi_engine_destroy(e);
    return 0;
}
