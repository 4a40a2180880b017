// velox_hip_timeline: per-workgroup timeline of one graph-replayed single-sequence decode step,
// from the timeline build of the library (velox_amd.build --timeline, -DVX_TIMELINE). Every GEMV and
// attention workgroup stamps s_memrealtime (100 MHz) at its start, after its activations are staged
// (GEMV) or after its first barrier (attention), and at its end; the step is replayed from a HIP
// graph as the runner replays it. Prints, per launch kind, the launch span, the gap from the previous
// launch's last workgroup end to this launch's first workgroup start, and workgroup medians.
//
//   velox_hip_timeline [--model llama3_8b] [--pos 133] [--reps 20] [--dump FILE]
// --dump writes every stamped workgroup of the last replay as CSV (launch, workgroup, start, staged,
// end, mark3, mark4; us from the step's first stamp).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "velox_hip.h"

extern "C" void velox_hip_timeline_set(unsigned long long* d_buf);

namespace {

double median(std::vector<double> v) {
    if (v.empty()) return 0.0;
    std::sort(v.begin(), v.end());
    return v[v.size() / 2];
}

int fail(const char* what) {
    std::fprintf(stderr, "velox_hip_timeline: %s failed (status %d)\n", what, velox_hip_last_error());
    return 1;
}

}  // namespace

int main(int argc, char** argv) {
    std::string model = "llama3_8b";
    uint32_t pos = 133;
    int reps = 20;
    std::string dump;
    for (int i = 1; i < argc; ++i) {
        const std::string f = argv[i];
        if (i + 1 >= argc) { std::fprintf(stderr, "missing value for %s\n", f.c_str()); return 2; }
        if (f == "--model") model = argv[++i];
        else if (f == "--pos") pos = (uint32_t)std::strtoul(argv[++i], nullptr, 10);
        else if (f == "--reps") reps = std::max(1, std::atoi(argv[++i]));
        else if (f == "--dump") dump = argv[++i];
        else { std::fprintf(stderr, "unknown flag %s\n", f.c_str()); return 2; }
    }
    VeloxHipModelConfig cfg;
    if (velox_hip_builtin_config(model.c_str(), std::max<uint32_t>(512u, pos + 1u), &cfg)) return fail("builtin_config");
    VeloxHipModel* M = nullptr;
    if (velox_hip_model_create(&cfg, &M)) return fail("model_create");
    VeloxHipArena A;
    if (velox_hip_arena_create(M, &A)) return fail("arena_create");
    hipStream_t st;
    if (hipStreamCreate(&st) != hipSuccess) return 1;
    velox_hip_synthesize_model(&A, 1234, 0.02f, 0.0f, st);
    for (uint32_t l = 0; l < cfg.num_layers; ++l) velox_hip_fill_kv(&A, l, pos, 7, 1.0f, st);
    velox_hip_set_state(&A, pos, 17, st);
    // the fused QKV + attention launch (one per layer) where the step uses it: its GEMV and attention
    // workgroups are tabulated apart (the first na workgroups attend)
    uint32_t fsplits = 0, ferr = 0;
    if (velox_hip_fused_attention_status(&A, &fsplits, &ferr)) return fail("fused_attention_status");
    const size_t na = (size_t)fsplits * cfg.num_kv_heads;
    const size_t per_layer = fsplits ? 4 : 5, nlaunch = per_layer * cfg.num_layers + 1, slots = nlaunch * 1024;
    unsigned long long* tl = nullptr;
    if (hipMalloc(&tl, slots * 64) != hipSuccess || hipMemset(tl, 0, slots * 64) != hipSuccess) return 1;
    velox_hip_timeline_set(tl);
    hipGraph_t g;
    hipGraphExec_t ex;
    if (hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal) != hipSuccess) return 1;
    velox_hip_decode_graph_step(&A, 1, st);
    if (hipStreamEndCapture(st, &g) != hipSuccess || hipGraphInstantiate(&ex, g, nullptr, nullptr, 0) != hipSuccess)
        return 1;
    hipEvent_t e0, e1;
    (void)hipEventCreate(&e0);
    (void)hipEventCreate(&e1);
    for (int r = 0; r < 5; ++r) (void)hipGraphLaunch(ex, st);
    (void)hipEventRecord(e0, st);
    for (int r = 0; r < reps; ++r) (void)hipGraphLaunch(ex, st);
    (void)hipEventRecord(e1, st);
    if (hipStreamSynchronize(st) != hipSuccess || velox_hip_last_error()) return fail("decode step");
    float ms = 0.0f;
    (void)hipEventElapsedTime(&ms, e0, e1);
    std::vector<unsigned long long> h(slots * 8);
    if (hipMemcpy(h.data(), tl, slots * 64, hipMemcpyDeviceToHost) != hipSuccess) return 1;
    velox_hip_timeline_set(nullptr);

    std::printf("model %s, position %u: step %.1f us (event-timed mean of %d graph replays; the stamps are the last "
                "replay's)\n", model.c_str(), pos, ms * 1000.0 / reps, reps);
    // kinds: 0 qkv (GEMV workgroups of the fused launch), 1 attn (its attention workgroups), 2 o_proj,
    // 3 gate_up, 4 down, 5 lm_head
    const char* names[6] = {"qkv", "attn", "o_proj", "gate_up", "down", "lm_head"};
    if (fsplits) {
        names[0] = "qkv|f";
        names[1] = "attn|f";
        std::printf("fused QKV + attention: %u splits per KV head (%zu attention workgroups per launch)\n", fsplits, na);
    }
    unsigned long long base = ~0ull;
    for (size_t i = 0; i < slots; ++i)
        if (h[8 * i]) base = std::min(base, h[8 * i]);
    if (!dump.empty()) {
        FILE* fd = std::fopen(dump.c_str(), "w");
        if (!fd) return fail("--dump file");
        std::fprintf(fd, "launch,wg,start,staged,end,mark3,mark4\n");
        for (size_t i = 0; i < slots; ++i) {
            const unsigned long long* e = &h[8 * i];
            if (!e[0]) continue;
            auto us = [&](unsigned long long t) { return t ? (double)(t - base) * 0.01 : -1.0; };
            std::fprintf(fd, "%zu,%zu,%.2f,%.2f,%.2f,%.2f,%.2f\n", i / 1024, i % 1024, us(e[0]), us(e[1]), us(e[2]),
                         us(e[3]), us(e[4]));
        }
        std::fclose(fd);
    }
    // per kind: span, gap before, median prologue (start -> staged / first barrier), median rest,
    // median workgroup, first workgroup end, last workgroup start, attention: median loop end, merge
    double sums[6][9] = {{0}};
    int cnt[6] = {0};
    double prev_end = -1.0, last_end = 0.0;
    std::printf("\nlayer 0 and the head (us from the step's first stamp):\n");
    std::printf("%-8s %5s %8s %8s %6s %6s %9s %7s %7s %8s %8s\n", "launch", "wgs", "start", "end", "span", "gap",
                "prologue", "rest", "wg", "1st_end", "last_st");
    // (launch, part): part 1 of a fused launch is its attention workgroups
    for (size_t LP = 0; LP < 2 * nlaunch; ++LP) {
        const size_t L = LP / 2, part = LP % 2;
        const bool fused_launch = fsplits && L < nlaunch - 1 && L % per_layer == 0;
        if (part == 1 && !fused_launch) continue;
        std::vector<double> t0, t1, t2, t3, t4;
        for (size_t b = 0; b < 1024; ++b) {
            const unsigned long long* e = &h[8 * (L * 1024 + b)];
            if (!e[0]) continue;
            if (fused_launch && (b < na) != (part == 1)) continue;
            t0.push_back((double)(e[0] - base) * 0.01);
            t1.push_back((double)(e[1] - base) * 0.01);
            t2.push_back((double)(e[2] - base) * 0.01);
            t3.push_back(e[3] ? (double)(e[3] - e[0]) * 0.01 : 0.0);
            t4.push_back(e[4] ? (double)(e[4] - e[0]) * 0.01 : 0.0);
        }
        if (t0.empty()) continue;
        const int kind = L == nlaunch - 1 ? 5 : fused_launch ? (int)part : (int)(L % per_layer) + (fsplits ? 1 : 0);
        std::vector<double> pro, rest, wg;
        for (size_t i = 0; i < t0.size(); ++i) {
            pro.push_back(t1[i] - t0[i]);
            rest.push_back(t2[i] - t1[i]);
            wg.push_back(t2[i] - t0[i]);
        }
        const double fs = *std::min_element(t0.begin(), t0.end()), le = *std::max_element(t2.begin(), t2.end());
        const double fe = *std::min_element(t2.begin(), t2.end()), ls = *std::max_element(t0.begin(), t0.end());
        const double gap = prev_end < 0 || part == 1 ? 0.0 : fs - prev_end;
        if (L < per_layer || L == nlaunch - 1)
            std::printf("%-8s %5zu %8.2f %8.2f %6.2f %6.2f %9.2f %7.2f %7.2f %8.2f %8.2f\n", names[kind], t0.size(), fs,
                        le, le - fs, gap, median(pro), median(rest), median(wg), fe - fs, ls - fs);
        const double v[9] = {le - fs, gap, median(pro), median(rest), median(wg), fe - fs, ls - fs, median(t3), median(t4)};
        if (L >= per_layer) {  // layer 0 (cold first launch of the step) left out of the averages
            for (int k = 0; k < 9; ++k) sums[kind][k] += v[k];
            ++cnt[kind];
        }
        if (fused_launch && part == 0) {  // the launch ends with the later of its two parts
            double le_all = le;
            for (size_t b = 0; b < na; ++b) {
                const unsigned long long* e = &h[8 * (L * 1024 + b)];
                if (e[0]) le_all = std::max(le_all, (double)(e[2] - base) * 0.01);
            }
            prev_end = le_all;
            last_end = le_all;
        } else if (part == 0) {
            prev_end = le;
            last_end = le;
        }
    }
    std::printf("\nmeans over layers 1..%u and the head (us): span, gap before, workgroup medians\n", cfg.num_layers - 1);
    std::printf("%-8s %6s %6s %9s %7s %7s %8s %8s %9s %7s\n", "kind", "span", "gap", "prologue", "rest", "wg", "1st_end",
                "last_st", "loop_end", "merge");
    double layer = 0.0;
    for (int k = 0; k < 6; ++k) {
        if (!cnt[k]) continue;
        double m[9];
        for (int j = 0; j < 9; ++j) m[j] = sums[k][j] / cnt[k];
        if (k < 5 && !(fsplits && k == 1)) layer += m[0] + m[1];  // (fused: the attention part overlaps)
        std::printf("%-8s %6.2f %6.2f %9.2f %7.2f %7.2f %8.2f %8.2f %9.2f %7.2f\n", names[k], m[0], m[1], m[2], m[3], m[4],
                    m[5], m[6], m[7], m[8]);
    }
    std::printf("\nlayer (spans + gaps): %.2f us; stamped step: %.1f us\n", layer, last_end);
    (void)hipGraphExecDestroy(ex);
    (void)hipGraphDestroy(g);
    (void)hipFree(tl);
    velox_hip_arena_destroy(&A);
    velox_hip_model_destroy(M);
    return 0;
}
