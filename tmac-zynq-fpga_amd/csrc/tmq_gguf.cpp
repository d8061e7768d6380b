// tmq_gguf -- command-line engine over libtmq.so, the counterpart of the
// reference's `tmac_gguf` (sim/tmac_gguf.cpp:2050-2181).
//
//   tmq_gguf <model.tmac> [--generate N] [--max-seq N] [--perf] [--no-graphs]
//            [--fpga-q8 --fpga-q5-0 --fpga-q4k --fpga-q6-k --fpga]
//
// Prompt token ids are read from stdin.  Without --generate the top-10
// logits of the last prompt position are printed as JSON,
// [{"id":…,"logit":%.3f},…] (:2156-2165); with --generate N the N greedily
// chosen ids are printed one per line (the reference samples top-k with
// rand(); greedy is this engine's choice).  All quantized formats always run
// on the GPU, so the --fpga-* flags are accepted and change nothing.
// --perf prints a timing summary (prompt, per-token decode) to stderr.
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../../include/tmq.h"

namespace {

double now_ms() {
    using namespace std::chrono;
    return duration<double, std::milli>(steady_clock::now().time_since_epoch()).count();
}

int die(const char* what) {
    fprintf(stderr, "[ERROR] %s: %s\n", what, tmq_last_error());
    return 1;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 2) {
        fprintf(stderr,
                "Usage: %s <model.tmac> [--generate N] [--max-seq N] [--perf] [--no-graphs]\n"
                "  Prompt tokens read from stdin; top-10 logits JSON, or N greedy tokens, to stdout.\n",
                argv[0]);
        return 1;
    }
    int generate_n = 0, max_seq = 512;
    bool perf = false, graphs = true;
    for (int i = 2; i < argc; i++) {
        if (!strcmp(argv[i], "--generate") && i + 1 < argc) generate_n = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--max-seq") && i + 1 < argc) max_seq = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--perf")) perf = true;
        else if (!strcmp(argv[i], "--no-graphs")) graphs = false;
        else if (!strncmp(argv[i], "--fpga", 6)) continue;
        else {
            fprintf(stderr, "[ERROR] unknown option %s\n", argv[i]);
            return 1;
        }
    }
    std::vector<int32_t> tokens;
    int tok;
    while (scanf("%d", &tok) == 1) tokens.push_back(tok);
    if (tokens.empty()) {
        fprintf(stderr, "[ERROR] No prompt tokens\n");
        return 1;
    }
    tmq_ctx* ctx = nullptr;
    if (tmq_open(0, &ctx) != TMQ_OK) return die("tmq_open");
    const double t0 = now_ms();
    tmq_model* m = nullptr;
    if (tmq_model_load(ctx, argv[1], max_seq, &m) != TMQ_OK) return die("load");
    tmq_model_set_graphs(m, graphs ? 1 : 0);
    tmq_model_config cfg;
    tmq_model_get_config(m, &cfg);
    const double t1 = now_ms();
    if (tmq_model_prompt(m, tokens.data(), (int)tokens.size()) != TMQ_OK) return die("prompt");
    const double t2 = now_ms();
    double t3 = t2;
    if (generate_n > 0) {
        std::vector<int32_t> out(generate_n);
        if (tmq_model_generate(m, generate_n, out.data()) != TMQ_OK) return die("generate");
        t3 = now_ms();
        for (int v : out) printf("%d\n", v);
    } else {
        std::vector<float> logits(cfg.vocab);
        if (tmq_model_logits(m, logits.data()) != TMQ_OK) return die("logits");
        t3 = now_ms();
        std::vector<int> idx(cfg.vocab);
        for (int i = 0; i < cfg.vocab; i++) idx[i] = i;
        const int k = std::min(10, cfg.vocab);
        std::partial_sort(idx.begin(), idx.begin() + k, idx.end(), [&](int a, int b) {
            return logits[a] != logits[b] ? logits[a] > logits[b] : a < b;
        });
        printf("[");
        for (int i = 0; i < k; i++) printf("{\"id\":%d,\"logit\":%.3f}%s", idx[i], logits[idx[i]], i + 1 < k ? "," : "");
        printf("]\n");
    }
    fflush(stdout);
    if (perf) {
        fprintf(stderr, "[PERF] load %.1f ms (%.1f MB of weights, %d layers)\n", t1 - t0,
                tmq_model_weight_bytes(m) / 1e6, cfg.n_layers);
        fprintf(stderr, "[PERF] prompt %zu tokens: %.3f ms (%.3f ms/token)\n", tokens.size(), t2 - t1,
                (t2 - t1) / tokens.size());
        if (generate_n > 0)
            fprintf(stderr, "[PERF] generate %d tokens: %.3f ms (%.3f ms/token, %.1f tok/s, %.1f GB/s weights)\n",
                    generate_n, t3 - t2, (t3 - t2) / generate_n, 1e3 * generate_n / (t3 - t2),
                    tmq_model_weight_bytes(m) * (double)generate_n / ((t3 - t2) * 1e-3) / 1e9);
        else
            fprintf(stderr, "[PERF] logits: %.3f ms\n", t3 - t2);
    }
    tmq_model_free(m);
    tmq_close(ctx);
    return 0;
}
