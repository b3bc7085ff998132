// engine_mm3: run an MMCF container on the GPU from the command line.
//
//   engine_mm3 --model M.mmcf --prompt-ids 12,7,99 --gen 64 [--seq 256] [--kv q16|q8]
//   engine_mm3 --model M.mmcf --prompt-random 32 --gen 64 --seed 0
//   engine_mm3 --model M.mmcf --prompt-ids ... --save-prefix P.mmkv   (MMKV1 of the prompt but its last token)
//   engine_mm3 --model M.mmcf --prompt-ids ... --prefix-cache P.mmkv  (resume from it)
//   engine_mm3 --model M.mmcf --worker [--prefix-cache P.mmkv]
//
// Flag names follow the reference CLI (engine/src/cli.cpp:26-77: --model,
// --gen, --greedy, --prefix-cache, --worker; KV=q16|q8 is the reference's
// environment switch, engine/src/gpu_attn.cpp:59-61).  Text needs the
// tokenizer, which is outside this build: prompts are token ids, and the
// command-line generation is greedy.
//
// --worker speaks the reference's line protocol (engine/src/worker.cpp:81-435,
// server/README.md "Worker protocol"): control lines {"op":"load"|"stats"|
// "cancel"} and tab-separated request lines base64(prompt) \t max_tokens \t
// temperature \t top_p \t seed [\t repetition \t frequency \t presence \t
// no_repeat_ngram \t min_p \t (chat JSON) \t top_k \t request id \t
// logprobs], answered with one JSON event per line (ready, loaded, stats,
// start, token, done, cancelled, error).  In this build the decoded prompt is
// a list of token ids ("12 7 99" or "12,7,99"), a token event's text is the id
// followed by a space, and a chat-JSON column is answered with an error.
// Temperature <= 0 decodes greedily on the device; above it each step's
// logits (or, with --top-k-candidates and a top_k, its top-k candidates) are
// sampled on the host with the request's seed, as the reference samples.
// The rolling prefix reuse is the reference's: the
// common prefix with the previous request (or the loaded prefix cache) is not
// prefilled again -- except on a hybrid model, whose conv history only
// matches the whole previous sequence, so a partial reuse prefills from 0.
#include <poll.h>
#include <unistd.h>

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "vgx.h"
#include "vgx_engine.h"

static void usage() {
    std::fprintf(stderr,
                 "usage: engine_mm3 --model PATH (--prompt-ids a,b,c | --prompt-random N | --worker) [--gen N]\n"
                 "                  [--seq N] [--kv q16|q8] [--device D] [--seed S] [--greedy]\n"
                 "                  [--top-k N] [--top-k-candidates]  (worker sampling defaults)\n"
                 "                  [--prefix-cache P.mmkv] [--save-prefix P.mmkv]\n");
}

static std::vector<int> parse_ids(const std::string& s, bool* ok) {
    std::vector<int> v;
    *ok = true;
    size_t i = 0;
    while (i < s.size()) {
        while (i < s.size() && (s[i] == ' ' || s[i] == ',' || s[i] == '\n' || s[i] == '\t')) ++i;
        if (i >= s.size()) break;
        if (s[i] < '0' || s[i] > '9') { *ok = false; return v; }
        long x = 0;
        while (i < s.size() && s[i] >= '0' && s[i] <= '9') {
            x = x * 10 + (s[i] - '0');
            if (x > 1 << 30) { *ok = false; return v; }
            ++i;
        }
        v.push_back((int)x);
    }
    return v;
}

// ---------------------------------------------------------------------------
// worker

namespace {

std::string g_inbuf;  // stdin bytes not yet consumed as lines

bool stdin_fill(int timeout_ms) {
    struct pollfd fd = {0, POLLIN, 0};
    if (poll(&fd, 1, timeout_ms) <= 0) return false;
    char tmp[4096];
    const ssize_t n = read(0, tmp, sizeof(tmp));
    if (n <= 0) return false;
    g_inbuf.append(tmp, (size_t)n);
    return true;
}

// timeout_ms < 0 blocks until a line or the end of the stream.
bool stdin_line(std::string& line, int timeout_ms) {
    for (;;) {
        const size_t nl = g_inbuf.find('\n');
        if (nl != std::string::npos) {
            line = g_inbuf.substr(0, nl);
            g_inbuf.erase(0, nl + 1);
            if (!line.empty() && line.back() == '\r') line.pop_back();
            return true;
        }
        if (!stdin_fill(timeout_ms)) {
            if (timeout_ms >= 0 || g_inbuf.empty()) return false;
            line.swap(g_inbuf);
            g_inbuf.clear();
            return true;
        }
    }
}

// A cancel waiting at the head of the input is consumed; a request that
// arrived early stays queued.
bool take_pending_cancel() {
    const size_t nl = g_inbuf.find('\n');
    if (nl == std::string::npos) return false;
    const std::string head = g_inbuf.substr(0, nl);
    if (head.find("\"op\"") == std::string::npos || head.find("cancel") == std::string::npos) return false;
    g_inbuf.erase(0, nl + 1);
    return true;
}

std::string json_str(const std::string& s) {
    std::string o = "\"";
    for (unsigned char c : s) {
        if (c == '"' || c == '\\') { o += '\\'; o += (char)c; }
        else if (c == '\n') o += "\\n";
        else if (c == '\t') o += "\\t";
        else if (c < 0x20) { char b[8]; std::snprintf(b, sizeof(b), "\\u%04x", c); o += b; }
        else o += (char)c;
    }
    return o + "\"";
}

// The string value of "key" in a one-level JSON object line ("" if absent).
std::string json_field(const std::string& line, const char* key) {
    const std::string k = std::string("\"") + key + "\"";
    size_t p = line.find(k);
    if (p == std::string::npos) return "";
    p = line.find(':', p + k.size());
    if (p == std::string::npos) return "";
    p = line.find('"', p);
    if (p == std::string::npos) return "";
    std::string v;
    for (size_t i = p + 1; i < line.size() && line[i] != '"'; ++i) {
        if (line[i] == '\\' && i + 1 < line.size()) ++i;
        v += line[i];
    }
    return v;
}

std::string base64_decode(const std::string& in) {
    auto val = [](char c) -> int {
        if (c >= 'A' && c <= 'Z') return c - 'A';
        if (c >= 'a' && c <= 'z') return c - 'a' + 26;
        if (c >= '0' && c <= '9') return c - '0' + 52;
        if (c == '+' || c == '-') return 62;
        if (c == '/' || c == '_') return 63;
        return -1;
    };
    std::string out;
    int acc = 0, bits = 0;
    for (char c : in) {
        const int v = val(c);
        if (v < 0) continue;
        acc = (acc << 6) | v;
        bits += 6;
        if (bits >= 8) {
            bits -= 8;
            out += (char)((acc >> bits) & 0xFF);
        }
    }
    return out;
}

struct Worker {
    vgx_engine* e = nullptr;
    std::string model;
    int device = 0, seq = 0, kv = 16, vocab = 0, kvlen = 0;
    std::string prefix_path;
    std::vector<int> cache_tokens;  // what the KV cache holds, positions 0..
    std::string req_id;
    const std::chrono::steady_clock::time_point t0 = std::chrono::steady_clock::now();

    void emit(const std::string& j) { std::printf("%s\n", j.c_str()); std::fflush(stdout); }
    void emit_req(std::string j) {
        if (!req_id.empty()) j = j.substr(0, j.size() - 1) + ",\"id\":" + json_str(req_id) + "}";
        emit(j);
    }
    void emit_error(const std::string& m) {
        emit_req("{\"event\":\"error\",\"message\":" + json_str(m) + "}");
    }

    bool open_model(const std::string& path) {
        if (e) vgx_engine_close(e);
        e = nullptr;
        if (vgx_engine_open(path.c_str(), device, seq, kv, &e)) return false;
        int dim, layers;
        vgx_engine_info(e, &dim, &layers, &vocab, &kvlen);
        model_is_hybrid = vgx_engine_conv_layers(e) > 0;
        model = path;
        cache_tokens.clear();
        if (!prefix_path.empty()) {
            std::vector<int> t((size_t)kvlen);
            int n = 0;
            if (vgx_engine_load_prefix(e, prefix_path.c_str(), t.data(), kvlen, &n) == 0) {
                t.resize((size_t)n);
                cache_tokens = t;
            } else {
                std::fprintf(stderr, "PREFIX_CACHE ignored %s: %s\n", prefix_path.c_str(), vgx_engine_last_error());
            }
        }
        return true;
    }

    // Process defaults a request may override: --top-k and
    // --top-k-candidates (engine/src/cli.cpp:45-48); the penalties are off.
    int top_k = 0;
    bool top_k_candidates = false;

    // One request (engine/src/worker.cpp:200-409).  Greedy requests
    // (temperature <= 0, no penalties, no logprobs) keep the token on the
    // device: the prompt is prefilled in batches and each step's argmax feeds
    // the next.  Sampled requests read each step's logits -- or, with
    // --top-k-candidates and a top_k, only its top-k candidates -- and draw on
    // the host with the request's seed.
    void request(const std::vector<std::string>& f) {
        bool ok = false;
        const std::vector<int> tokens = parse_ids(base64_decode(f[0]), &ok);
        int max_new = std::atoi(f[1].c_str());
        if (max_new < 0) max_new = 0;
        const float temp = (float)std::atof(f[2].c_str());
        float top_p = (float)std::atof(f[3].c_str());
        if (top_p <= 0.0f || top_p > 1.0f) top_p = 0.9f;
        const uint32_t seed = (uint32_t)std::strtoul(f[4].c_str(), nullptr, 10);
        // columns 6..10: penalties, clamped as the reference clamps them
        auto col = [&](size_t i) -> const char* { return f.size() > i && !f[i].empty() ? f[i].c_str() : nullptr; };
        auto clampf = [](float v, float lo, float hi) { return v < lo ? lo : v > hi ? hi : v; };
        const float rep = col(5) ? clampf((float)std::atof(col(5)), 0.5f, 2.0f) : 1.0f;
        const float freq = col(6) ? clampf((float)std::atof(col(6)), -2.0f, 2.0f) : 0.0f;
        const float pres = col(7) ? clampf((float)std::atof(col(7)), -2.0f, 2.0f) : 0.0f;
        int ngram = col(8) ? std::atoi(col(8)) : 0;
        ngram = ngram < 0 ? 0 : ngram > 8 ? 8 : ngram;
        const float min_p = col(9) ? clampf((float)std::atof(col(9)), 0.0f, 1.0f) : 0.0f;
        if (col(10)) { emit_error("this build takes token ids as the prompt (no chat template)"); return; }
        int req_top_k = col(11) ? std::atoi(col(11)) : top_k;
        if (req_top_k < 0) req_top_k = 0;
        const bool want_logprobs = col(13) && std::atoi(col(13)) != 0;
        const bool penalties = rep != 1.0f || freq != 0.0f || pres != 0.0f || ngram > 1 || min_p > 0.0f;
        const bool greedy = temp <= 0.0f;
        const bool fast_greedy = greedy && !want_logprobs && !penalties;
        bool cand_mode = top_k_candidates && req_top_k > 0 && !greedy && !penalties && !want_logprobs;
        if (!ok) { emit_error("this build takes token ids as the prompt (no tokenizer)"); return; }
        if (tokens.empty()) { emit_error("empty prompt"); return; }
        for (int t : tokens)
            if (t >= vocab) { emit_error("prompt token outside the vocabulary"); return; }
        const int n = (int)tokens.size();
        if (n >= kvlen) { emit_error("context full"); return; }
        int common = 0;
        while (common < (int)cache_tokens.size() && common < n && cache_tokens[common] == tokens[common]) ++common;
        // A hybrid's conv history is that of the whole cached sequence, and a
        // position run twice would step it twice: only an exact extension of
        // the cache is resumed.
        if (model_is_hybrid && (common < (int)cache_tokens.size() || common >= n)) common = 0;
        const int from = common < n ? common : n - 1;
        emit_req("{\"event\":\"start\",\"prompt_tokens\":" + std::to_string(n) + ",\"cached_tokens\":" +
                 std::to_string(common) + ",\"prefill_tokens\":" + std::to_string(n - from) + "}");
        std::vector<float> logits((size_t)vocab);
        std::vector<int16_t> q16((size_t)vocab);
        std::vector<float> cval((size_t)(req_top_k > 0 ? req_top_k : 1));
        std::vector<int> ctok(cval.size());
        int ncand = 0, complete = 0;
        float cstats[3] = {0.0f, 0.0f, 0.0f};
        // one position: the argmax (greedy), the candidates, or the logits
        auto step = [&](int tok, int p, int* next) -> bool {
            int st;
            if (fast_greedy) {
                st = vgx_engine_step(e, tok, p, nullptr, next);
            } else if (cand_mode) {
                st = vgx_engine_step_candidates(e, tok, p, req_top_k, temp, top_p, cval.data(), ctok.data(),
                                                (int)cval.size(), &ncand, cstats, &complete, logits.data());
                if (!st && !complete) cand_mode = false;  // the full logits came back instead
            } else {
                st = vgx_engine_step(e, tok, p, q16.data(), nullptr);
                for (int i = 0; !st && i < vocab; ++i) logits[(size_t)i] = (float)q16[(size_t)i] / 256.0f;
            }
            return st == 0;
        };
        int next = 0;
        bool fine = true;
        if (fast_greedy) {
            fine = vgx_engine_prefill(e, tokens.data() + from, n - from, from, nullptr, &next) == 0;
        } else {
            // the prompt but its last position in batches, the last for its logits
            if (n - 1 > from) fine = vgx_engine_prefill(e, tokens.data() + from, n - 1 - from, from, nullptr, nullptr) == 0;
            if (fine) fine = step(tokens[(size_t)n - 1], n - 1, nullptr);
        }
        if (!fine) {
            emit_error(vgx_engine_last_error());
            cache_tokens.clear();
            return;
        }
        vgx_sampler* rng = nullptr;
        vgx_sampler_create(seed, &rng);
        std::vector<int> all = tokens, recent;
        std::string full, finish = "length", lp_rows;
        int pos = n, generated = 0;
        if (max_new > kvlen - pos) max_new = kvlen - pos;
        bool cancelled = false;
        for (int i = 0; i < max_new; ++i) {
            if (i % 4 == 0 && stdin_fill(0) && take_pending_cancel()) {
                cancelled = true;
                finish = "cancelled";
                break;
            }
            float lp = 0.0f;
            if (!fast_greedy) {
                if (!cand_mode)
                    vgx_apply_penalties(logits.data(), vocab, recent.data(), (int)recent.size(), rep, freq, pres, ngram,
                                        min_p);
                if (want_logprobs) {
                    if (greedy) vgx_argmax_report(logits.data(), vocab, &next, &lp);
                    else vgx_sample_logits(rng, logits.data(), vocab, temp, top_p, req_top_k, &next, &lp);
                } else if (greedy) {
                    vgx_argmax_report(logits.data(), vocab, &next, nullptr);
                } else if (cand_mode) {
                    vgx_sample_candidates(rng, cval.data(), ctok.data(), ncand, 1, cstats[0], temp, top_p, req_top_k,
                                          &next);
                } else {
                    vgx_sample_logits(rng, logits.data(), vocab, temp, top_p, req_top_k, &next, nullptr);
                }
            }
            // no special ids stated: 1 and 2 end a sequence (engine/src/worker.cpp:361-363)
            if (next == 1 || next == 2) {
                if (pos < kvlen && vgx_engine_step(e, next, pos++, nullptr, nullptr) == 0) all.push_back(next);
                finish = "stop";
                break;
            }
            const std::string piece = std::to_string(next) + " ";
            full += piece;
            emit_req("{\"event\":\"token\",\"text\":" + json_str(piece) + "}");
            if (want_logprobs) {
                char b[64];
                std::snprintf(b, sizeof b, "%.9g", lp);
                lp_rows += std::string(lp_rows.empty() ? "" : ",") + "{\"id\":" + std::to_string(next) +
                           ",\"text\":" + json_str(piece) + ",\"lp\":" + b + "}";
            }
            ++generated;
            all.push_back(next);
            recent.push_back(next);
            if (i + 1 < max_new && pos < kvlen) {
                if (!step(next, pos++, &next)) {
                    emit_error(vgx_engine_last_error());
                    cache_tokens.clear();
                    vgx_sampler_free(rng);
                    return;
                }
            }
        }
        vgx_sampler_free(rng);
        // the KV holds every token run through the model: the prompt and each
        // generated token but the last (it was emitted, not yet run)
        if (!all.empty() && (int)all.size() > pos) all.resize((size_t)pos);
        cache_tokens = all;
        if (cancelled) emit("{\"event\":\"cancelled\",\"id\":" + json_str(req_id) + "}");
        emit_req("{\"event\":\"done\",\"text\":" + json_str(full) + ",\"finish_reason\":" + json_str(finish) +
                 ",\"prompt_tokens\":" + std::to_string(n) + ",\"completion_tokens\":" + std::to_string(generated) +
                 ",\"cached_tokens\":" + std::to_string(common) + ",\"prefill_tokens\":" + std::to_string(n - from) +
                 (want_logprobs ? ",\"logprobs\":[" + lp_rows + "]" : std::string()) + "}");
    }

    bool model_is_hybrid = false;

    int run() {
        emit("{\"event\":\"ready\",\"prefix_cache_tokens\":" + std::to_string(cache_tokens.size()) +
             ",\"template\":\"plain\",\"chat_template\":false}");
        std::string line;
        while (stdin_line(line, -1)) {
            if (line.empty()) continue;
            req_id.clear();
            if (line[0] == '{') {
                const std::string op = json_field(line, "op");
                if (op == "cancel") {
                    emit("{\"event\":\"cancelled\",\"id\":" + json_str(json_field(line, "id")) + ",\"idle\":true}");
                } else if (op == "stats") {
                    const long long up = std::chrono::duration_cast<std::chrono::milliseconds>(
                                             std::chrono::steady_clock::now() - t0).count();
                    emit("{\"event\":\"stats\",\"seq\":" + std::to_string(kvlen) + ",\"kv_pack\":" +
                         std::to_string(kv) + ",\"template\":\"plain\",\"uptime_ms\":" + std::to_string(up) + "}");
                } else if (op == "load") {
                    const std::string want = json_field(line, "model");
                    if (want.empty()) { emit_error("load: no model path"); continue; }
                    const auto tl = std::chrono::steady_clock::now();
                    if (!open_model(want)) {
                        emit_error("load: cannot read " + want + ": " + vgx_engine_last_error());
                        return 1;  // no model is loaded any more
                    }
                    const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - tl)
                                          .count();
                    emit("{\"event\":\"loaded\",\"model\":" + json_str(want) + ",\"load_ms\":" + std::to_string(ms) +
                         ",\"template\":\"plain\",\"chat_template\":false,\"seq\":" + std::to_string(kvlen) + "}");
                } else {
                    emit_error("unknown op \"" + op + "\"");
                }
                continue;
            }
            std::vector<std::string> f;
            size_t start = 0;
            while (start <= line.size()) {
                const size_t tab = line.find('\t', start);
                f.push_back(line.substr(start, tab == std::string::npos ? std::string::npos : tab - start));
                if (tab == std::string::npos) break;
                start = tab + 1;
            }
            if (f.size() < 5) { emit_error("bad request line"); continue; }
            if (f.size() > 12) req_id = f[12];
            request(f);
        }
        return 0;
    }
};

}  // namespace

int main(int argc, char** argv) {
    std::string model, ids, save_prefix, prefix_cache;
    int gen = 8, seq = 0, device = 0, rnd = 0, kv = 0;
    bool worker = false, top_k_candidates = false;
    unsigned seed = 0;
    int top_k = 0;
    if (const char* k = std::getenv("KV")) kv = !std::strcmp(k, "q8") ? 8 : 16;
    if (const char* m = std::getenv("MODEL")) model = m;
    for (int i = 1; i < argc; ++i) {
        std::string a = argv[i];
        auto next = [&]() -> const char* {
            if (i + 1 >= argc) { usage(); std::exit(2); }
            return argv[++i];
        };
        if (a == "--model") model = next();
        else if (a == "--prompt-ids") ids = next();
        else if (a == "--prompt-random") rnd = std::atoi(next());
        else if (a == "--gen") gen = std::atoi(next());
        else if (a == "--seq") seq = std::atoi(next());
        else if (a == "--device") device = std::atoi(next());
        else if (a == "--seed") seed = (unsigned)std::atoi(next());
        else if (a == "--kv") { std::string v = next(); kv = v == "q8" ? 8 : v == "q16" ? 16 : -1; }
        else if (a == "--save-prefix") save_prefix = next();
        else if (a == "--prefix-cache") prefix_cache = next();
        else if (a == "--worker") worker = true;
        else if (a == "--greedy") {}
        else if (a == "--top-k") top_k = std::atoi(next());
        else if (a == "--top-k-candidates") top_k_candidates = true;
        else { usage(); return 2; }
    }
    if (model.empty() || kv < 0 || (!worker && ids.empty() && rnd <= 0)) { usage(); return 2; }
    if (worker) {
        Worker w;
        w.device = device;
        w.seq = seq;
        w.kv = kv ? kv : 16;
        w.prefix_path = prefix_cache;
        w.top_k = top_k < 0 ? 0 : top_k;
        // a candidate pass keeps top_k candidates: none without a top_k (engine/src/engine.cpp:82-86)
        w.top_k_candidates = top_k_candidates && w.top_k > 0;
        if (!w.open_model(model)) { std::fprintf(stderr, "engine_mm3: %s\n", vgx_engine_last_error()); return 1; }
        const int rc = w.run();
        vgx_engine_close(w.e);
        return rc;
    }
    vgx_engine* e = nullptr;
    int st = vgx_engine_open(model.c_str(), device, seq, kv ? kv : 16, &e);
    if (st) { std::fprintf(stderr, "engine_mm3: %s\n", vgx_engine_last_error()); return 1; }
    int dim, layers, vocab, kvlen;
    vgx_engine_info(e, &dim, &layers, &vocab, &kvlen);
    std::vector<int> prompt;
    if (!ids.empty()) {
        bool ok = false;
        prompt = parse_ids(ids, &ok);
        if (!ok) { usage(); vgx_engine_close(e); return 2; }
    } else {
        std::mt19937 rng(seed);
        std::uniform_int_distribution<int> d(0, vocab - 1);
        for (int i = 0; i < rnd; ++i) prompt.push_back(d(rng));
    }
    // --prefix-cache: resume from the cached prefix the prompt starts with
    int cached = 0;
    if (!prefix_cache.empty()) {
        std::vector<int> t((size_t)kvlen);
        int n = 0;
        if (vgx_engine_load_prefix(e, prefix_cache.c_str(), t.data(), kvlen, &n) == 0) {
            while (cached < n && cached < (int)prompt.size() && t[cached] == prompt[cached]) ++cached;
            if (cached < n) cached = 0;  // the prompt must extend the whole cached prefix
            // the prompt's last token is run for its logits: a KV row is
            // rewritten unchanged, but a conv history would step twice
            if (cached >= (int)prompt.size()) cached = vgx_engine_conv_layers(e) > 0 ? 0 : (int)prompt.size() - 1;
        } else {
            std::fprintf(stderr, "PREFIX_CACHE ignored %s: %s\n", prefix_cache.c_str(), vgx_engine_last_error());
        }
    }
    std::vector<int> out(gen);
    double pf = 0, dc = 0;
    if (!save_prefix.empty() && (int)prompt.size() - 1 > cached) {
        // the prompt but its last token, saved (a later run of a prompt that
        // extends it prefills only the rest), then generation resumes from it
        const int m = (int)prompt.size() - 1;
        st = vgx_engine_prefill(e, prompt.data() + cached, m - cached, cached, nullptr, nullptr);
        if (!st) st = vgx_engine_save_prefix(e, save_prefix.c_str(), prompt.data(), m, 0, 0);
        if (!st) cached = m;
    }
    if (!st) st = vgx_engine_generate_from(e, prompt.data(), (int)prompt.size(), cached, gen, out.data(), &pf, &dc);
    if (st) { std::fprintf(stderr, "engine_mm3: %s\n", vgx_engine_last_error()); vgx_engine_close(e); return 1; }
    for (int i = 0; i < gen; ++i) std::printf("%d%c", out[i], i + 1 < gen ? ' ' : '\n');
    const double per = gen > 1 ? dc / (gen - 1) : 0.0;
    std::fprintf(stderr, "TIMING prefill=%.3fms (%zu tokens, %d cached) decode_avg=%.4fms/token (%.1f tokens/s) gen=%d\n",
                 pf, prompt.size(), cached, per, per > 0 ? 1000.0 / per : 0.0, gen);
    vgx_engine_close(e);
    return 0;
}
