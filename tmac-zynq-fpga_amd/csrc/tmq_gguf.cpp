// tmq_gguf -- command-line engine over libtmq.so, the counterpart of the
// reference's `tmac_gguf` (sim/tmac_gguf.cpp:2050-2181).
//
//   tmq_gguf <model.tmac> [--generate N] [--max-seq N] [--perf] [--trace PATH]
//            [--prefill N | --no-prefill] [--no-graphs]
//            [--fpga] [--fpga-int16] [--fpga-q8] [--fpga-q4k] [--fpga-q5-0] [--fpga-q6-k]
//
// Prompt token ids are read from stdin.  Without --generate the top-10
// logits of the last prompt position are printed as JSON,
// [{"id":…,"logit":%.3f},…] (:2156-2165); with --generate N the N greedily
// chosen ids are printed one per line (the reference samples top-k with
// rand(); greedy is this engine's choice).  The --fpga* flags set what the
// reference's flags set (:2085-2091) and route every matmul the way its
// `matmul` does (:473-493), all on the GPU: a type whose --fpga-<type> flag
// is given takes its quantized kernel, the others matmul_fpga_int16 when
// any --fpga flag is given, and without any flag every matmul is the FP32
// loop; the logits are get_logits_q8 only under --fpga-q8 (:2151-2155).
// The prompt runs through the batched prefill in chunks of --prefill N
// tokens (default 512); --no-prefill runs it one token at a time.
// --dump-tiles N, --dump-tiles-q5-0 N, --dump-tiles-q6-k N write the first N
// Q8_0 / Q5_0 / Q6_K tiles of the run's matmuls in the reference's
// cosimulation layouts (:1046-1065, :1282-1298, :1478-1495) to
// <cosim-dir>/cosim_tiles{,_q5_0,_q6_k}.bin (default /tmp); --fpga-phaseb
// sets every --fpga flag and records the PhaseB descriptor chain of the
// run's Q5_0/Q4_K/Q6_K matmuls until the reference's 1 GiB DDR is full,
// replays it on the GPU and verifies it (:834-880); --dump-phaseb writes
// tb_phaseb.bin/.hdr (:609-708) to the same directory.  While any of these
// records, positions run one at a time with their matmul inputs captured.
// --perf prints host timings (load, prompt, per-token decode) to stderr, then
// profiles up to 8 more decode steps launch by launch on the GPU and prints
// the reference's pipeline timing breakdown (:79-134) per operation, and
// writes the launches as a Chrome trace (:55-76) to --trace PATH (default
// /tmp/pipeline_trace.json, the reference's path).  Any --fpga* flag prints
// the reference's [FPGA TIMING SUMMARY] with GPU figures to stderr at the end
// (timing_summary).
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "../../include/tmq.h"
#include "tmq_cosim.h"

namespace {

double now_ms() {
    using namespace std::chrono;
    return duration<double, std::milli>(steady_clock::now().time_since_epoch()).count();
}

int die(const char* what) {
    fprintf(stderr, "[ERROR] %s: %s\n", what, tmq_last_error());
    return 1;
}

// Per-operation totals of a GPU launch profile, in the reference's table
// layout, and the launches as Chrome trace events.
void perf_report(const std::vector<tmq_launch_time>& lt, int steps, const char* trace_path) {
    struct Agg {
        const char* name;
        double ms;
        long calls;
    };
    std::vector<Agg> agg;
    double total = 0.0;
    for (const tmq_launch_time& t : lt) {
        const double ms = t.end_ms - t.start_ms;
        total += ms;
        auto it = std::find_if(agg.begin(), agg.end(), [&](const Agg& a) { return !strcmp(a.name, t.name); });
        if (it == agg.end()) agg.push_back({t.name, ms, 1});
        else {
            it->ms += ms;
            it->calls++;
        }
    }
    std::sort(agg.begin(), agg.end(), [](const Agg& a, const Agg& b) { return a.ms > b.ms; });
    fprintf(stderr, "\n[PERF — PIPELINE TIMING BREAKDOWN] (GPU, %d decode steps, launch by launch)\n", steps);
    fprintf(stderr, "  %-24s %12s %8s %10s %8s\n", "Operation", "Time (ms)", "Calls", "Avg (ms)", "Share");
    fprintf(stderr, "  %s\n", std::string(69, '-').c_str());
    for (const Agg& a : agg)
        fprintf(stderr, "  %-24s %10.3f %8ld %8.4f %6.1f%%\n", a.name, a.ms, a.calls, a.ms / a.calls,
                total > 0 ? 100.0 * a.ms / total : 0.0);
    fprintf(stderr, "  %s\n", std::string(69, '-').c_str());
    fprintf(stderr, "  %-24s %10.3f\n", "TOTAL", total);
    if (!agg.empty())
        fprintf(stderr, "\n  >> Hottest: %s (%.3f ms, %.1f%%)\n\n", agg[0].name, agg[0].ms,
                total > 0 ? 100.0 * agg[0].ms / total : 0.0);
    FILE* f = fopen(trace_path, "w");
    if (!f) {
        fprintf(stderr, "[TRACE] cannot write %s\n", trace_path);
        return;
    }
    fprintf(f, "{\"traceEvents\":[\n");
    for (size_t i = 0; i < lt.size(); i++) {
        fprintf(f, "{\"ph\":\"B\",\"name\":\"%s\",\"cat\":\"gpu\",\"ts\":%.3f,\"pid\":1,\"tid\":1},\n", lt[i].name,
                lt[i].start_ms * 1e3);
        fprintf(f, "{\"ph\":\"E\",\"name\":\"%s\",\"cat\":\"gpu\",\"ts\":%.3f,\"pid\":1,\"tid\":1}%s\n", lt[i].name,
                lt[i].end_ms * 1e3, i + 1 < lt.size() ? "," : "");
    }
    fprintf(f, "]}\n");
    fclose(f);
    fprintf(stderr, "[TRACE] Wrote Chrome trace: %s\n", trace_path);
}

// Tiles and MACs of one decode step's matmuls (the seven projections of
// every layer) and of one logits call under flags, counted as the reference's
// matmul_fpga_* count them (tmq_matmul_tiles).
struct StepCounts {
    int64_t step_tiles = 0, step_macs = 0, logit_tiles = 0, logit_macs = 0;
};
bool step_counts(const tmq_model* m, const tmq_model_config& cfg, uint32_t flags, StepCounts* out) {
    static const char* proj[7] = {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"};
    auto add = [&](const char* name, int64_t* tiles, int64_t* macs) {
        const tmq_tensor* t = tmq_model_tensor(m, name);
        uint32_t type = 0;
        uint64_t rows = 0, cols = 0, bytes = 0;
        int64_t tl = 0, mc = 0;
        if (!t || tmq_tensor_info(t, &type, &rows, &cols, &bytes) != TMQ_OK ||
            tmq_matmul_tiles(type, flags, rows, cols, &tl, &mc) != TMQ_OK)
            return false;
        *tiles += tl;
        *macs += mc;
        return true;
    };
    for (int l = 0; l < cfg.n_layers; l++)
        for (const char* p : proj) {
            char name[64];
            snprintf(name, sizeof(name), "blk.%d.%s.weight", l, p);
            if (!add(name, &out->step_tiles, &out->step_macs)) return false;
        }
    return add("token_embd.weight", &out->logit_tiles, &out->logit_macs);
}

// The reference's [FPGA TIMING SUMMARY] (sim/fpga_sim.hpp:156-172, printed
// when g_use_fpga is set, sim/tmac_gguf.cpp:2168-2171) for the GPU: the
// run's tiles and MACs in the reference's tilings, the wall time of its
// prompt and decode calls and MACs over that time ("NAIVE", as the
// reference divides by the host time of its matmul calls); then `steps`
// more decode steps profiled launch by launch (tmq_model_profile): kernel
// time per step, its MACs over that time and its weight bytes over that
// time.  To stderr, which carries the engine's other reports.
int timing_summary(tmq_model* m, const tmq_model_config& cfg, uint32_t flags, int64_t positions,
                   int64_t logit_calls, double wall_ms) {
    StepCounts c;
    if (!step_counts(m, cfg, flags, &c)) return die("timing summary");
    const int64_t tiles = c.step_tiles * positions + c.logit_tiles * logit_calls;
    const int64_t macs = c.step_macs * positions + c.logit_macs * logit_calls;
    if (tiles == 0) return 0;  // as the reference: nothing ran on the accelerator
    fprintf(stderr, "\n[FPGA TIMING SUMMARY] (GPU)\n");
    fprintf(stderr, "  Tiles: %-8lld  MACs: %-10lld  GPU: %.2f ms  NAIVE: %.2f Gop/s\n", (long long)tiles,
            (long long)macs, wall_ms, wall_ms > 0 ? macs / (wall_ms / 1000.0) / 1e9 : 0.0);
    const int steps = std::min(4, cfg.max_seq - 1 - tmq_model_position(m));
    if (steps <= 0) return 0;
    std::vector<tmq_launch_time> lt((size_t)steps * (3 + 6 * (size_t)cfg.n_layers));
    int n = 0;
    if (tmq_model_profile(m, steps, lt.data(), (int)lt.size(), &n) != TMQ_OK) return die("profile");
    double kern_ms = 0.0;
    for (int i = 0; i < n; i++) kern_ms += lt[i].end_ms - lt[i].start_ms;
    const double us = 1e3 * kern_ms / steps;
    const int64_t st = c.step_tiles + c.logit_tiles, sm = c.step_macs + c.logit_macs;
    fprintf(stderr, "  GPU: %d decode steps profiled, %.2f us of kernels per step (%lld tiles, %lld MACs): "
                    "%.2f Gop/s, %.1f GB/s of weights\n",
            steps, us, (long long)st, (long long)sm, sm / (us * 1e-6) / 1e9,
            tmq_model_weight_bytes(m) / (us * 1e-6) / 1e9);
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 2) {
        fprintf(stderr,
                "Usage: %s <model.tmac> [--generate N] [--max-seq N] [--perf] [--trace PATH]\n"
                "       [--prefill N | --no-prefill] [--no-graphs] [--dump-layers] [--dump-dir DIR]\n"
                "       [--fpga] [--fpga-int16] [--fpga-q8] [--fpga-q4k] [--fpga-q5-0] [--fpga-q6-k]\n"
                "  Prompt tokens read from stdin; top-10 logits JSON, or N greedy tokens, to stdout.\n",
                argv[0]);
        return 1;
    }
    int generate_n = 0, max_seq = 512, prefill = 512;
    bool perf = false, graphs = true, dump_layers = false;
    uint32_t flags = 0;  // the reference's g_use_fpga / g_fpga_* (all off by default)
    bool phaseb = false, dump_phaseb = false;
    int dump_tiles[3] = {0, 0, 0};  // Q8_0, Q5_0, Q6_K
    std::string cosim_dir = "/tmp";
    const char* trace_path = "/tmp/pipeline_trace.json";
    const char* dump_dir = "/tmp";
    for (int i = 2; i < argc; i++) {
        if (!strcmp(argv[i], "--generate") && i + 1 < argc) generate_n = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--max-seq") && i + 1 < argc) max_seq = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--perf")) perf = true;
        else if (!strcmp(argv[i], "--trace") && i + 1 < argc) trace_path = argv[++i];
        else if (!strcmp(argv[i], "--prefill") && i + 1 < argc) prefill = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--no-prefill")) prefill = 0;
        else if (!strcmp(argv[i], "--no-graphs")) graphs = false;
        else if (!strcmp(argv[i], "--dump-layers")) dump_layers = true;
        else if (!strcmp(argv[i], "--dump-dir") && i + 1 < argc) dump_dir = argv[++i];
        else if (!strcmp(argv[i], "--fpga") || !strcmp(argv[i], "--fpga-int16")) flags |= TMQ_FLAG_FPGA;
        else if (!strcmp(argv[i], "--fpga-q8")) flags |= TMQ_FLAG_FPGA | TMQ_FLAG_Q8_0;
        else if (!strcmp(argv[i], "--fpga-q4k")) flags |= TMQ_FLAG_FPGA | TMQ_FLAG_Q4_K;
        else if (!strcmp(argv[i], "--fpga-q5-0")) flags |= TMQ_FLAG_FPGA | TMQ_FLAG_Q5_0;
        else if (!strcmp(argv[i], "--fpga-q6-k")) flags |= TMQ_FLAG_FPGA | TMQ_FLAG_Q6_K;
        else if (!strcmp(argv[i], "--fpga-phaseb")) {
            phaseb = true;
            flags = TMQ_FLAGS_ALL;
        } else if (!strcmp(argv[i], "--dump-phaseb")) dump_phaseb = true;
        else if (!strcmp(argv[i], "--dump-tiles") && i + 1 < argc) dump_tiles[0] = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--dump-tiles-q5-0") && i + 1 < argc) dump_tiles[1] = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--dump-tiles-q6-k") && i + 1 < argc) dump_tiles[2] = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--cosim-dir") && i + 1 < argc) cosim_dir = argv[++i];
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
    if (tmq_model_set_flags(m, flags) != TMQ_OK) return die("flags");
    if (prefill > 0 && flags != TMQ_FLAGS_ALL) prefill = 0;  // batched prefill: the all-flags arithmetic only
    if (tmq_model_set_prefill(m, prefill) != TMQ_OK) {
        fprintf(stderr, "[WARN] %s; the prompt runs one token at a time\n", tmq_last_error());
        tmq_model_set_prefill(m, 0);
    }
    tmq_model_config cfg;
    tmq_model_get_config(m, &cfg);
    // per-matmul recorders (tile dumps, PhaseB): the .tmac bytes of every
    // weight, and the inputs of every matmul captured position by position
    tmq_cli::TmacFile tf;
    std::unique_ptr<tmq_cli::Recorder> rec;
    if (phaseb || dump_tiles[0] > 0 || dump_tiles[1] > 0 || dump_tiles[2] > 0) {
        std::string err;
        if (!tf.load(argv[1], &err)) {
            fprintf(stderr, "[ERROR] %s\n", err.c_str());
            return 1;
        }
        rec.reset(new tmq_cli::Recorder(ctx, m, &tf, flags));
        static const char* names[3] = {"/cosim_tiles.bin", "/cosim_tiles_q5_0.bin", "/cosim_tiles_q6_k.bin"};
        for (int k = 0; k < 3; k++)
            if (!rec->open_tiles(k, dump_tiles[k], cosim_dir + names[k])) {
                fprintf(stderr, "[ERROR] cannot write %s%s\n", cosim_dir.c_str(), names[k]);
                return 1;
            }
        if (phaseb) {
            rec->enable_phaseb();
            fprintf(stderr, "[PHASEB] Descriptor chain mode enabled\n");
        }
    }
    const size_t cap_n = (size_t)cfg.n_layers * (3 * (size_t)cfg.hidden + cfg.inter);
    std::vector<float> acts;
    // one position with its matmul inputs offered to the recorders
    auto feed_rec = [&](int32_t t) -> int {
        acts.resize(cap_n);
        if (tmq_model_feed_capture(m, t, acts.data()) != TMQ_OK) return die("feed_capture");
        return rec->offer_position(acts.data(), cfg.n_layers, cfg.hidden, cfg.inter) ? 1 : 0;
    };
    // the logits (get_logits_q8 / get_logits) with their input offered
    auto logits_rec = [&](std::vector<float>& lg) -> int {
        std::vector<float> x(cfg.hidden);
        if (tmq_model_logits_capture(m, lg.data(), x.data()) != TMQ_OK) return die("logits_capture");
        if (flags & TMQ_FLAG_Q8_0) return rec->offer({"token_embd.weight", x.data()}) ? 1 : 0;
        return 0;
    };
    const double t1 = now_ms();
    if (rec && rec->active() && !dump_layers) {
        // process_prompt one token at a time while the recorders take calls
        if (tmq_model_reset(m) != TMQ_OK) return die("reset");
        size_t i = 0;
        for (; i < tokens.size() && rec->active(); i++)
            if (feed_rec(tokens[i])) return 1;
        for (; i < tokens.size(); i++)
            if (tmq_model_feed(m, tokens[i]) != TMQ_OK) return die("feed");
    } else if (!dump_layers) {
        if (tmq_model_prompt(m, tokens.data(), (int)tokens.size()) != TMQ_OK) return die("prompt");
    } else {
        // process_prompt with dump_layers (sim/tmac_gguf.cpp:2001-2018): the
        // embedding as cpp_layer_0.bin (the last token's, as each token
        // overwrites it) and the hidden state after each layer of the last
        // token as cpp_layer_<l+1>.bin, hidden fp32 values each
        const int n = (int)tokens.size();
        if (n > 1 && tmq_model_prompt(m, tokens.data(), n - 1) != TMQ_OK) return die("prompt");
        std::vector<float> layers((size_t)(cfg.n_layers + 1) * cfg.hidden);
        if (tmq_model_feed_dump(m, tokens[n - 1], layers.data()) != TMQ_OK) return die("feed_dump");
        for (int l = 0; l <= cfg.n_layers; l++) {
            char path[4096];
            snprintf(path, sizeof(path), "%s/cpp_layer_%d.bin", dump_dir, l);
            FILE* f = fopen(path, "wb");
            if (!f || fwrite(layers.data() + (size_t)l * cfg.hidden, sizeof(float), cfg.hidden, f) != (size_t)cfg.hidden) {
                fprintf(stderr, "[ERROR] cannot write %s\n", path);
                if (f) fclose(f);
                return 1;
            }
            fclose(f);
        }
    }
    const double t2 = now_ms();
    double t3 = t2;
    // greedy choice of generate: the first index of the largest logit
    auto argmax = [](const std::vector<float>& lg) {
        return (int32_t)(std::max_element(lg.begin(), lg.end()) - lg.begin());
    };
    if (generate_n > 0) {
        std::vector<int32_t> out(generate_n);
        int g = 0;
        std::vector<float> lg(cfg.vocab);
        // generate (:2025-2045): logits, choice, then the chosen token fed
        for (; g < generate_n && rec && rec->active(); g++) {
            if (logits_rec(lg)) return 1;
            out[g] = argmax(lg);
            if (feed_rec(out[g])) return 1;
        }
        if (g < generate_n && tmq_model_generate(m, generate_n - g, out.data() + g) != TMQ_OK) return die("generate");
        t3 = now_ms();
        for (int v : out) printf("%d\n", v);
    } else {
        std::vector<float> logits(cfg.vocab);
        if (rec && rec->active()) {
            if (logits_rec(logits)) return 1;
        } else if (tmq_model_logits(m, logits.data()) != TMQ_OK) return die("logits");
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
    const int run_positions = tmq_model_position(m);  // before --perf advances it
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
        const int steps = std::min(8, cfg.max_seq - 1 - tmq_model_position(m));
        if (steps > 0) {
            std::vector<tmq_launch_time> lt((size_t)steps * (3 + 6 * (size_t)cfg.n_layers));
            int n = 0;
            if (tmq_model_profile(m, steps, lt.data(), (int)lt.size(), &n) != TMQ_OK) return die("profile");
            lt.resize(n);
            perf_report(lt, steps, trace_path);
        }
    }
    int64_t logit_calls = generate_n > 0 ? generate_n : 1;
    if (flags & TMQ_FLAG_FPGA) {
        if (timing_summary(m, cfg, flags, run_positions, logit_calls, t3 - t1)) return 1;
    }
    int rc = 0;
    if (rec && phaseb) {
        // phaseb_verify (:834-880), then phaseb_dump_files (:609-708)
        if (rec->phaseb_verify() < 0) rc = 1;
        if (!rc && dump_phaseb && rec->phaseb_dump(cosim_dir) < 0) rc = 1;
    }
    rec.reset();
    tmq_model_free(m);
    tmq_close(ctx);
    return rc;
}
