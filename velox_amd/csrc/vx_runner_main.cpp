// velox_hip_runner -- command-line runner over the C ABI, with the argv and stdout report of the
// reference's runner (src/runners/velox_cuda_runner.cu:327-726), so that `veloxc --run`
// (src/cli.rs:640-770, "[Step N] Token: id" parsing at :706-733) and the benchmark regexes
// (benchmarks/run_sota_roofline_benchmarks.py:278-292) keep working.
//
//   velox_hip_runner [--model llama3_8b | --model-file MODEL.vlx] [--weights synthetic|FILE.gguf]
//                    [--tokens 1,2,3 | --prompt-len N]
//                    [--context-len N] [--steps N] [--warmup N] [--seed S] [--layers L]
//                    [--prefill-chunk N] [--unquantized f32|f16] [--quantize MODE] [--no-cuda-graph]
//                    [--verbose]
//
// --model-file MODEL.vlx reads the model from its .vlx source (the `model` header, weight
// declarations and `target hardware` budget; what `velox build MODEL.vlx` compiles into the
// reference's emitted runner) instead of a builtin configuration.
// --prefill-chunk N (2..128) prefills the prompt N positions per batched step (one weight pass per
// chunk) instead of the reference's one decode step per prompt token; TTFT reports either.
// --unquantized f32|f16 keeps the synthetic weights as fp32 / fp16 rows (the reference's quant_mode
// 0 / 1, a build without --quantize) instead of Q4_0.
// --quantize MODE (or --quantize=MODE) takes the reference runner's fp32 model and converts it at
// load as that runner does (velox_cuda_runner.cu:356-372): f16 / fp16 to fp16 rows, q4_0 / int4 /
// w4a16 to its group-64 format, any other value keeps fp32 rows.
//
// Weights are the seeded synthetic Q4_0 model (`--weights synthetic`, what src/cli.rs:654 passes
// through) or a GGUF Q4_0 checkpoint (`--weights FILE.gguf`, whose metadata then defines the model,
// as the K2 runner's --weights does); other checkpoint formats are refused with exit 1.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "velox_hip.h"

int main(int argc, char** argv) {
    std::string model = "llama3_8b", weights, model_file;
    uint32_t unquantized = 0;
    std::vector<uint32_t> tokens;
    uint32_t prompt_len = 128, steps = 32, warmup = 0, layers = 0, context_len = 0, prefill_chunk = 0;
    uint64_t seed = 1234;
    bool graph = true, verbose = false;
    for (int i = 1; i < argc; ++i) {
        const char* a = argv[i];
        auto next = [&]() -> const char* {
            if (i + 1 >= argc) { std::fprintf(stderr, "Error: %s needs a value\n", a); std::exit(1); }
            return argv[++i];
        };
        if (!std::strcmp(a, "--model")) model = next();
        else if (!std::strcmp(a, "--model-file")) model_file = next();
        else if (!std::strcmp(a, "--unquantized")) {
            const char* f = next();
            if (!std::strcmp(f, "f32")) unquantized = 1;
            else if (!std::strcmp(f, "f16")) unquantized = 2;
            else { std::fprintf(stderr, "Error: --unquantized takes f32 or f16\n"); return 1; }
        }
        else if (!std::strcmp(a, "--quantize") || !std::strncmp(a, "--quantize=", 11)) {
            const char* f = a[10] == '=' ? a + 11 : next();
            if (!std::strcmp(f, "f16") || !std::strcmp(f, "fp16")) unquantized = 2;
            else if (!std::strcmp(f, "q4_0") || !std::strcmp(f, "int4") || !std::strcmp(f, "w4a16")) unquantized = 3;
            else unquantized = 1;
        }
        else if (!std::strcmp(a, "--tokens")) {
            std::string s = next();
            size_t p = 0;
            while (p < s.size()) {
                size_t q = s.find(',', p);
                if (q == std::string::npos) q = s.size();
                const std::string t = s.substr(p, q - p);
                char* end = nullptr;
                const unsigned long v = std::strtoul(t.c_str(), &end, 10);
                if (t.empty() || *end != '\0' || v > 0xFFFFFFFFul) {
                    std::fprintf(stderr, "Error: bad token id '%s' in --tokens\n", t.c_str());
                    return 1;
                }
                tokens.push_back((uint32_t)v);
                p = q + 1;
            }
            if (tokens.empty()) { std::fprintf(stderr, "Error: --tokens is empty\n"); return 1; }
        } else if (!std::strcmp(a, "--prompt-len")) prompt_len = (uint32_t)std::atoi(next());
        else if (!std::strcmp(a, "--steps")) steps = (uint32_t)std::atoi(next());
        else if (!std::strcmp(a, "--warmup")) warmup = (uint32_t)std::atoi(next());
        else if (!std::strcmp(a, "--seed")) seed = std::strtoull(next(), nullptr, 10);
        else if (!std::strcmp(a, "--layers")) layers = (uint32_t)std::atoi(next());
        else if (!std::strcmp(a, "--prefill-chunk")) {
            prefill_chunk = (uint32_t)std::atoi(next());
            if (prefill_chunk < 2 || prefill_chunk > 128) {
                std::fprintf(stderr, "Error: --prefill-chunk takes 2..128 positions\n");
                return 1;
            }
        }
        else if (!std::strcmp(a, "--no-cuda-graph") || !std::strcmp(a, "--no-graph")) graph = false;
        else if (!std::strcmp(a, "--verbose")) verbose = true;
        else if (!std::strcmp(a, "--weights")) {
            const char* w = next();
            const size_t n = std::strlen(w);
            if (n > 5 && !std::strcmp(w + n - 5, ".gguf")) {
                weights = w;
            } else if (std::strcmp(w, "synthetic") != 0) {
                std::fprintf(stderr, "Error: --weights %s is not supported (synthetic or a .gguf Q4_0 file)\n", w);
                return 1;
            }
        } else if (!std::strcmp(a, "--context-len")) {
            context_len = (uint32_t)std::atoi(next());
        } else if (!std::strcmp(a, "--speculative") ||
                   !std::strcmp(a, "--draft-len") || !std::strcmp(a, "--spec-ema")) {
            std::fprintf(stderr, "Error: %s is not supported by this runner\n", a);
            return 1;
        } else {
            std::fprintf(stderr, "Error: unknown argument %s\n", a);
            return 1;
        }
    }
    if (!tokens.empty()) prompt_len = (uint32_t)tokens.size();
    if (context_len && prompt_len != 1) {
        if (!tokens.empty()) {
            std::fprintf(stderr, "Error: --context-len continues from one token; pass a single --tokens id\n");
            return 1;
        }
        prompt_len = 1;
    }
    if (steps == 0 || prompt_len == 0) { std::fprintf(stderr, "Error: --steps and --prompt-len must be > 0\n"); return 1; }

    VeloxHipRunOptions opt;
    std::memset(&opt, 0, sizeof(opt));
    opt.model = model.c_str();
    opt.model_file = model_file.empty() ? nullptr : model_file.c_str();
    opt.unquantized = unquantized;
    opt.prompt_len = prompt_len;
    opt.warmup = warmup;
    // the first generated token comes from the prefill; steps-1 decode steps are timed
    opt.steps = steps > 1 ? steps - 1 : 1;
    opt.seed = seed;
    opt.sigma = 0.02f;
    opt.use_graph = graph ? 1 : 0;
    opt.num_layers = layers;
    opt.verbose = verbose ? 1 : 0;
    opt.prompt_tokens = tokens.empty() ? nullptr : tokens.data();
    opt.context_len = context_len;
    opt.weights_path = weights.empty() ? nullptr : weights.c_str();
    opt.prefill_chunk = context_len ? 0 : prefill_chunk;
    std::vector<uint32_t> out(prompt_len + warmup + opt.steps + 8);
    VeloxHipRunReport rep;
    const int rc = velox_hip_run(&opt, out.data(), (uint32_t)out.size(), &rep);
    if (rc != 0) {
        std::fprintf(stderr, "HIP error detected: status %d%s\n", rc,
                     rc == VELOX_HIP_EINVAL ? " (invalid argument: token id >= vocab or unsupported shape)" : "");
        return 1;
    }
    // ring[p] = argmax after position p; generated tokens start at p = prompt_len - 1
    const uint32_t first = prompt_len - 1;
    const uint32_t n_gen = (uint32_t)std::min<size_t>(rep.n_tokens - first, (size_t)warmup + opt.steps + 1);
    for (uint32_t s = 0; s < n_gen; ++s) std::printf("[Step %u] Token: %u\n", s, out[first + s]);
    std::printf("================================================================================\n");
    std::printf("VELOX MI355X HIP RUNTIME EXECUTION REPORT\n");
    std::printf("================================================================================\n");
    if (weights.empty()) {
        const char* fmt = unquantized == 1   ? "fp32 rows"
                          : unquantized == 2 ? "fp16 rows"
                          : unquantized == 3 ? "group-64 4-bit"
                                             : "Q4_0";
        std::printf("Model                  : %s (synthetic %s, seed %llu)\n",
                    model_file.empty() ? model.c_str() : model_file.c_str(), fmt, (unsigned long long)seed);
        std::printf("Weight Synthesis       : %.2f ms\n", rep.load_ms);
    } else {
        std::printf("Model                  : %s (GGUF Q4_0)\n", weights.c_str());
        std::printf("Weight Load            : %.2f ms\n", rep.load_ms);
    }
    std::printf("TTFT (Prefill Latency) : %.3f ms (%u prompt tokens, %s)\n", rep.prefill_ms, prompt_len,
                opt.prefill_chunk ? "batched prefill" : "token by token");
    std::printf("Decode Latency (%u tok): %.3f ms (%.2f tok/s, %.3f ms/tok)\n", opt.steps, rep.decode_ms, rep.tok_per_s,
                rep.decode_ms / opt.steps);
    std::printf("Achieved HBM Bandwidth : %.1f GB/s (%.2f%% of 8000 GB/s)\n", rep.hbm_gbps, rep.hbm_gbps / 80.0);
    std::printf("Dynamic Heap Allocs    : 0 (no hipMalloc/hipFree during generation)\n");
    std::printf("================================================================================\n");
    return 0;
}
