// engine_mm3: run an MMCF container on the GPU from the command line.
//
//   engine_mm3 --model M.mmcf --prompt-ids 12,7,99 --gen 64 [--seq 256] [--kv q16|q8]
//   engine_mm3 --model M.mmcf --prompt-random 32 --gen 64 --seed 0
//
// Flag names follow the reference CLI (engine/src/cli.cpp:26-77: --model,
// --gen, --greedy; KV=q16|q8 is the reference's environment switch,
// engine/src/gpu_attn.cpp:59-61).  Text prompts need the tokenizer, which is
// outside this build: prompts are token ids.  Decoding is greedy.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "vgx.h"
#include "vgx_engine.h"

extern "C" const char* vgx_engine_last_error(void);

static void usage() {
    std::fprintf(stderr,
                 "usage: engine_mm3 --model PATH (--prompt-ids a,b,c | --prompt-random N) [--gen N]\n"
                 "                  [--seq N] [--kv q16|q8] [--device D] [--seed S] [--greedy]\n");
}

int main(int argc, char** argv) {
    std::string model, ids;
    int gen = 8, seq = 0, device = 0, rnd = 0, kv = 0;
    unsigned seed = 0;
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
        else if (a == "--greedy") {}
        else { usage(); return 2; }
    }
    if (model.empty() || kv < 0 || (ids.empty() && rnd <= 0)) { usage(); return 2; }
    vgx_engine* e = nullptr;
    int st = vgx_engine_open(model.c_str(), device, seq, kv ? kv : 16, &e);
    if (st) { std::fprintf(stderr, "engine_mm3: %s\n", vgx_engine_last_error()); return 1; }
    int dim, layers, vocab, kvlen;
    vgx_engine_info(e, &dim, &layers, &vocab, &kvlen);
    std::vector<int> prompt;
    if (!ids.empty()) {
        for (const char* p = ids.c_str(); *p;) {
            prompt.push_back(std::atoi(p));
            while (*p && *p != ',') ++p;
            if (*p == ',') ++p;
        }
    } else {
        std::mt19937 rng(seed);
        std::uniform_int_distribution<int> d(0, vocab - 1);
        for (int i = 0; i < rnd; ++i) prompt.push_back(d(rng));
    }
    std::vector<int> out(gen);
    double pf = 0, dc = 0;
    st = vgx_engine_generate(e, prompt.data(), (int)prompt.size(), gen, out.data(), &pf, &dc);
    if (st) { std::fprintf(stderr, "engine_mm3: %s\n", vgx_engine_last_error()); vgx_engine_close(e); return 1; }
    for (int i = 0; i < gen; ++i) std::printf("%d%c", out[i], i + 1 < gen ? ' ' : '\n');
    const double per = gen > 1 ? dc / (gen - 1) : 0.0;
    std::fprintf(stderr, "TIMING prefill=%.3fms (%zu tokens) decode_avg=%.4fms/token (%.1f tokens/s) gen=%d\n", pf,
                 prompt.size(), per, per > 0 ? 1000.0 / per : 0.0, gen);
    vgx_engine_close(e);
    return 0;
}
