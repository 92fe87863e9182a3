// serve.cpp - the engine's --serve protocol: one JSON object per line in, one JSON object per line out (reference
// src/qwythos.cpp: protocol qw:2139-2148, serve_loop qw:2593-2813, topk_out qw:2513-2531).
//
//   {"op":"reset"}                                  -> {"ok":true,"op":"reset"}   (empty context, position 0)
//   {"op":"run","tokens":[..],"gen":N,"mtp":B}      -> ingest the tokens at the current position, then N tokens:
//        {"id":I,"top":[[id,logit],..]}   per generated token (the list: the k largest logits that chose I, k = 40;
//                                         under "mtp":true only the first token has one, later ones have "top":[])
//        {"done":true,"pos":P}           P = the context length after the run
//   errors: {"error":"need tokens and gen"}, {"error":"context full; send op reset"}, {"error":<engine message>}
//
// The generation loops are the reference's, step for step: greedy emits the current token, stops after the
// end-of-sequence id, otherwise feeds it (so the last emitted token is in the context); MTP emits c0 (and c1 when the
// draft was accepted and the budget allows) per verify round and checks the end-of-sequence id on the round's current
// token.  Requests are parsed as JSON (the reference matches substrings of the compact JSON its server sends; both read
// those lines the same way).  An optional "topk":K (0..64) sets the list length, 40 when absent.
//
// The loop talks to the engine through rmi_serve_backend (function pointers), so the protocol logic runs the same over
// the real engine (rmi_serve_engine) and over any other backend.
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/rapier_mi.h"
#include "../../include/rapier_mi_engine.h"

namespace {

constexpr int kStopped = -1;   // the request ended with an error line; the loop goes on

#define RMI_SERVE_TRY(expr)            \
    do {                               \
        const int rc_ = (expr);        \
        if (rc_ != RMI_OK) return rc_; \
    } while (0)

// ---- a small JSON reader: the request objects (string keys; string, number, bool, null, array, object values) ----
struct Json {
    const char* p;
    const char* end;
    std::string err;

    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\r' || *p == '\n')) ++p;
    }
    bool lit(const char* s) {
        const size_t n = std::strlen(s);
        if (static_cast<size_t>(end - p) < n || std::strncmp(p, s, n) != 0) return false;
        p += n;
        return true;
    }
    bool fail(const char* what) {
        if (err.empty()) err = what;
        return false;
    }
    bool string(std::string* out) {
        if (p >= end || *p != '"') return fail("expected a string");
        ++p;
        while (p < end && *p != '"') {
            char c = *p++;
            if (c == '\\') {
                if (p >= end) return fail("bad escape");
                c = *p++;
                if (c == 'u') {
                    if (end - p < 4) return fail("bad escape");
                    p += 4;          // keys and ops are ASCII; a \u escape is kept as '?'
                    c = '?';
                } else if (c == 'n') c = '\n';
                else if (c == 't') c = '\t';
                else if (c == 'r') c = '\r';
                else if (c == 'b') c = '\b';
                else if (c == 'f') c = '\f';
                else if (c != '"' && c != '\\' && c != '/') return fail("bad escape");
            } else if (static_cast<unsigned char>(c) < 0x20) {
                return fail("control character in a string");
            }
            if (out) out->push_back(c);
        }
        if (p >= end) return fail("unterminated string");
        ++p;
        return true;
    }
    // a JSON number; *is_int: no fraction or exponent
    bool number(double* out, bool* is_int) {
        const char* s = p;
        if (p < end && *p == '-') ++p;
        if (p >= end || *p < '0' || *p > '9') return fail("bad number");
        if (*p == '0') ++p;
        else while (p < end && *p >= '0' && *p <= '9') ++p;
        bool integral = true;
        if (p < end && *p == '.') {
            integral = false;
            ++p;
            if (p >= end || *p < '0' || *p > '9') return fail("bad number");
            while (p < end && *p >= '0' && *p <= '9') ++p;
        }
        if (p < end && (*p == 'e' || *p == 'E')) {
            integral = false;
            ++p;
            if (p < end && (*p == '+' || *p == '-')) ++p;
            if (p >= end || *p < '0' || *p > '9') return fail("bad number");
            while (p < end && *p >= '0' && *p <= '9') ++p;
        }
        *out = std::strtod(std::string(s, p).c_str(), nullptr);
        *is_int = integral;
        return true;
    }
    bool skip_value(int depth = 0) {
        if (depth > 32) return fail("nested too deep");
        ws();
        if (p >= end) return fail("expected a value");
        if (*p == '"') return string(nullptr);
        if (*p == '{') return object(nullptr, depth + 1);
        if (*p == '[') {
            ++p;
            ws();
            if (p < end && *p == ']') {
                ++p;
                return true;
            }
            for (;;) {
                if (!skip_value(depth + 1)) return false;
                ws();
                if (p < end && *p == ',') { ++p; continue; }
                if (p < end && *p == ']') { ++p; return true; }
                return fail("bad array");
            }
        }
        if (lit("true") || lit("false") || lit("null")) return true;
        double d;
        bool i;
        return number(&d, &i);
    }
    template <typename F>
    bool object(F* on_key, int depth = 0) {
        ws();
        if (p >= end || *p != '{') return fail("expected an object");
        ++p;
        ws();
        if (p < end && *p == '}') {
            ++p;
            return true;
        }
        for (;;) {
            ws();
            std::string key;
            if (!string(&key)) return false;
            ws();
            if (p >= end || *p != ':') return fail("expected ':'");
            ++p;
            ws();
            if (on_key) {
                if (!(*on_key)(key)) return false;
            } else if (!skip_value(depth)) {
                return false;
            }
            ws();
            if (p < end && *p == ',') { ++p; continue; }
            if (p < end && *p == '}') { ++p; return true; }
            return fail("expected ',' or '}'");
        }
    }
    bool object(std::nullptr_t, int depth) {
        auto skip = [&](const std::string&) { return skip_value(depth); };
        return object(&skip, depth);
    }
};

struct Request {
    bool reset = false;
    bool has_tokens = false;
    std::vector<int> tokens;
    long long gen = -1;          // -1: absent
    bool mtp = false;
    int topk = -1;               // -1: absent
};

// parses one request line; "" on success, else the reason
std::string parse_request(const char* line, size_t len, Request* r) {
    Json j{line, line + len, {}};
    auto on_key = [&](const std::string& key) -> bool {
        if (key == "op") {
            std::string op;
            if (!j.string(&op)) return false;
            r->reset = op == "reset";
            return true;
        }
        if (key == "tokens") {
            if (j.p >= j.end || *j.p != '[') return j.fail("tokens must be an array");
            ++j.p;
            j.ws();
            r->has_tokens = true;
            if (j.p < j.end && *j.p == ']') {
                ++j.p;
                return true;
            }
            for (;;) {
                j.ws();
                double d;
                bool integral;
                if (!j.number(&d, &integral)) return false;
                if (!integral || d < -2147483648.0 || d > 2147483647.0) return j.fail("tokens must be integers");
                r->tokens.push_back(static_cast<int>(d));
                j.ws();
                if (j.p < j.end && *j.p == ',') { ++j.p; continue; }
                if (j.p < j.end && *j.p == ']') { ++j.p; return true; }
                return j.fail("bad tokens array");
            }
        }
        if (key == "gen" || key == "topk") {
            double d;
            bool integral;
            if (!j.number(&d, &integral)) return false;
            if (!integral || std::fabs(d) > 9.0e15) return j.fail("gen and topk must be integers");
            if (key == "gen") r->gen = static_cast<long long>(d);
            else r->topk = d < 0 ? -2 : d > 1e6 ? 1000000 : static_cast<int>(d);
            return true;
        }
        if (key == "mtp") {
            if (j.lit("true")) r->mtp = true;
            else if (j.lit("false")) r->mtp = false;
            else return j.fail("mtp must be true or false");
            return true;
        }
        return j.skip_value();
    };
    if (!j.object(&on_key)) return j.err;
    j.ws();
    if (j.p != j.end) return "trailing characters after the object";
    return "";
}

std::string json_escape(const char* s) {
    std::string o;
    for (; *s; ++s) {
        const unsigned char c = static_cast<unsigned char>(*s);
        if (c == '"' || c == '\\') {
            o.push_back('\\');
            o.push_back(static_cast<char>(c));
        } else if (c < 0x20) {
            char b[8];
            std::snprintf(b, sizeof b, "\\u%04x", c);
            o += b;
        } else {
            o.push_back(static_cast<char>(c));
        }
    }
    return o;
}

// one generated token: {"id":I,"top":[[id,logit],..]} with %.5f logits, as topk_out prints them
std::string token_line(int id, const int* ids, const float* logits, int k) {
    std::string s = "{\"id\":" + std::to_string(id) + ",\"top\":[";
    char b[64];
    for (int i = 0; i < k; ++i) {
        std::snprintf(b, sizeof b, "%s[%d,%.5f]", i ? "," : "", ids[i], static_cast<double>(logits[i]));
        s += b;
    }
    return s + "]}";
}

class Loop {
public:
    Loop(const rmi_serve_backend* b, const rmi_serve_options* o, int out_fd) : b_(b), o_(*o), out_(out_fd) {}

    // handles one line; RMI_OK, or the code of a device or output failure (the loop ends)
    int line(const char* text, size_t len) {
        const int rc = handle(text, len);
        return rc == kStopped ? RMI_OK : rc;
    }

private:
    int handle(const char* text, size_t len) {
        if (len == 0) return RMI_OK;
        Request r;
        const std::string perr = parse_request(text, len, &r);
        if (!perr.empty()) return error(("bad request: " + perr).c_str());
        if (r.reset) {
            const int rc = b_->reset(b_->user);
            if (rc != RMI_OK) return engine_error(rc);
            return emit("{\"ok\":true,\"op\":\"reset\"}");
        }
        if (r.tokens.empty() || r.gen <= 0) return error("need tokens and gen");
        int pos = 0;
        int rc = b_->position(b_->user, &pos);
        if (rc != RMI_OK) return engine_error(rc);
        if (static_cast<long long>(pos) + static_cast<long long>(r.tokens.size()) + r.gen + 8 >=
            static_cast<long long>(b_->max_ctx))
            return error("context full; send op reset");
        const int k = r.topk == -1 ? o_.topk : r.topk;
        if (k < 0 || k > 64) return error("topk must be 0..64");
        int cur = 0;
        rc = b_->ingest(b_->user, r.tokens.data(), static_cast<int>(r.tokens.size()), o_.batch, &cur);
        if (rc != RMI_OK) return engine_error(rc);
        return r.mtp ? run_mtp(cur, r.gen, k) : run_greedy(cur, r.gen, k);
    }

    // serve_loop's greedy path (qw:2748-2759)
    int run_greedy(int cur, long long gen, int k) {
        int rc = b_->gen_begin(b_->user, RMI_GEN_GREEDY);
        if (rc != RMI_OK) return engine_error(rc);
        for (long long out = 0; out < gen;) {
            RMI_SERVE_TRY(emit_with_top(cur, k));
            ++out;
            if (cur == o_.eos) break;
            int toks[2], n = 0;
            rc = b_->gen_step(b_->user, toks, &n);
            if (rc != RMI_OK) return engine_error(rc);
            cur = toks[0];
        }
        return done();
    }

    // serve_loop's MTP path (qw:2761-2808): the first token with its list, then verify rounds
    int run_mtp(int cur, long long gen, int k) {
        RMI_SERVE_TRY(emit_with_top(cur, k));
        long long emitted = 1;
        if (cur != o_.eos && emitted < gen) {
            int rc = b_->gen_begin(b_->user, RMI_GEN_MTP);
            if (rc != RMI_OK) return engine_error(rc);
            while (emitted < gen) {
                int toks[2], n = 0;
                rc = b_->gen_step(b_->user, toks, &n);
                if (rc != RMI_OK) return engine_error(rc);
                RMI_SERVE_TRY(emit(token_line(toks[0], nullptr, nullptr, 0)));
                ++emitted;
                if (n == 2) {
                    if (emitted < gen) {
                        RMI_SERVE_TRY(emit(token_line(toks[1], nullptr, nullptr, 0)));
                        ++emitted;
                        cur = toks[1];
                    } else {
                        cur = toks[0];
                    }
                } else {
                    cur = toks[0];
                }
                if (cur == o_.eos) break;
            }
        }
        return done();
    }

    int emit_with_top(int id, int k) {
        int ids[64];
        float logits[64];
        if (k > 0) {
            const int rc = b_->topk(b_->user, k, ids, logits);
            if (rc != RMI_OK) return engine_error(rc);
        }
        return emit(token_line(id, ids, logits, k));
    }

    int done() {
        int pos = 0;
        const int rc = b_->position(b_->user, &pos);
        if (rc != RMI_OK) return engine_error(rc);
        return emit("{\"done\":true,\"pos\":" + std::to_string(pos) + "}");
    }

    int error(const char* msg) { return emit("{\"error\":\"" + json_escape(msg) + "\"}"); }

    // an engine failure ends the request with an error line; a device failure (a failed launch or HIP call) also ends
    // the loop, as the reference exits on one
    int engine_error(int rc) {
        const char* m = b_->error ? b_->error(b_->user) : nullptr;
        const int wr = error(m && *m ? m : "engine error");
        if (rc == RMI_ERR_LAUNCH || wr != RMI_OK) return rc == RMI_ERR_LAUNCH ? rc : wr;
        return kStopped;
    }

    int emit(const std::string& s) {
        std::string l = s + "\n";
        const char* p = l.data();
        size_t left = l.size();
        while (left > 0) {
            const ssize_t w = ::write(out_, p, left);
            if (w < 0 && errno == EINTR) continue;
            if (w <= 0) return RMI_ERR_STATE;
            p += w;
            left -= static_cast<size_t>(w);
        }
        return RMI_OK;
    }

    const rmi_serve_backend* b_;
    rmi_serve_options o_;
    int out_;
};

// ---- the backend over the engine's C API ----
int eng_reset(void* u) { return rmi_engine_reset(static_cast<rmi_engine*>(u)); }
int eng_ingest(void* u, const int* t, int n, int batch, int* first) {
    return rmi_engine_ingest(static_cast<rmi_engine*>(u), t, n, batch, first);
}
int eng_topk(void* u, int k, int* ids, float* logits) {
    return rmi_engine_topk(static_cast<rmi_engine*>(u), 0, k, ids, logits);
}
int eng_gen_begin(void* u, int mode) { return rmi_engine_gen_begin(static_cast<rmi_engine*>(u), mode); }
int eng_gen_step(void* u, int* t, int* n) { return rmi_engine_gen_step(static_cast<rmi_engine*>(u), t, n); }
int eng_position(void* u, int* pos) {
    int cur = 0;
    return rmi_engine_state(static_cast<rmi_engine*>(u), pos, &cur);
}
const char* eng_error(void*) { return rmi_last_error(); }

}  // namespace

extern "C" rmi_serve_options rmi_serve_default_options(void) {
    rmi_serve_options o;
    o.eos = 248046;   // the qwen35 vocabulary's end-of-turn id, as serve_loop compares it (qw:2752, 2765, 2807)
    o.batch = 16;
    o.topk = 40;      // TOPK of the reference server and topk_out's k (qw:2746)
    return o;
}

extern "C" int rmi_serve_fd(const rmi_serve_backend* b, const rmi_serve_options* o, int in_fd, int out_fd) {
    if (!b || !o || !b->reset || !b->ingest || !b->topk || !b->gen_begin || !b->gen_step || !b->position)
        return RMI_ERR_POINTER;
    if (o->batch < 1 || o->batch > 16 || o->topk < 0 || o->topk > 64) return RMI_ERR_SHAPE;
    Loop loop(b, o, out_fd);
    std::string buf;
    char chunk[65536];
    for (;;) {
        const ssize_t r = ::read(in_fd, chunk, sizeof chunk);
        if (r < 0 && errno == EINTR) continue;
        if (r < 0) return RMI_ERR_STATE;
        if (r == 0) break;
        buf.append(chunk, static_cast<size_t>(r));
        size_t start = 0;
        for (size_t nl; (nl = buf.find('\n', start)) != std::string::npos; start = nl + 1) {
            size_t len = nl - start;
            if (len > 0 && buf[start + len - 1] == '\r') --len;
            const int rc = loop.line(buf.data() + start, len);
            if (rc != RMI_OK) return rc;
        }
        buf.erase(0, start);
    }
    if (!buf.empty()) {   // a last line without its newline
        const int rc = loop.line(buf.data(), buf.size());
        if (rc != RMI_OK) return rc;
    }
    return RMI_OK;
}

extern "C" int rmi_serve_engine(rmi_engine* e, const rmi_serve_options* o, int in_fd, int out_fd) {
    if (!e || !o) return RMI_ERR_POINTER;
    rmi_engine_info_t info;
    const int rc = rmi_engine_info(e, &info);
    if (rc != RMI_OK) return rc;
    rmi_serve_backend b;
    b.user = e;
    b.max_ctx = info.max_ctx;
    b.reset = eng_reset;
    b.ingest = eng_ingest;
    b.topk = eng_topk;
    b.gen_begin = eng_gen_begin;
    b.gen_step = eng_gen_step;
    b.position = eng_position;
    b.error = eng_error;
    return rmi_serve_fd(&b, o, in_fd, out_fd);
}
