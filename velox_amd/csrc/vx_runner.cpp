// vx_runner.cpp -- velox_hip_runner_main, the command-line runner over the C ABI (the generic
// velox_hip_runner and every runner `velox_amd.build --model X.vlx` generates call it), with the
// argv and stdout report of the reference's runner (src/runners/velox_cuda_runner.cu:327-726), so that `veloxc --run`
// (src/cli.rs:640-770, "[Step N] Token: id" parsing at :706-733) and the benchmark regexes
// (benchmarks/run_sota_roofline_benchmarks.py:278-292) keep working.
//
//   velox_hip_runner [--model llama3_8b | --model-file MODEL.vlx] [--weights synthetic|FILE]
//                    [--tokens 1,2,3 | --prompt-len N]
//                    [--context-len N] [--steps N] [--warmup N] [--seed S] [--layers L]
//                    [--prefill-chunk N] [--unquantized f32|f16] [--quantize MODE] [--no-cuda-graph]
//                    [--attn-splits N] [--verbose]
//
// --weights FILE is what src/cli.rs:653-654 passes on every run: the checkpoint the model's source
// binds (src/cli.rs:1400-1414). A safetensors file (the reference runner's format,
// velox_cuda_runner.cu:154-199, Hugging Face tensor names) runs on the --model / --model-file
// configuration, or without either on the builtin configuration its tensor shapes match; a GGUF
// Q4_0 file (recognized by its magic) defines the model by its metadata, as the K2 runner's
// --weights does. `--weights synthetic` (or no --weights) runs the seeded synthetic model.
// --model-file MODEL.vlx reads the model from its .vlx source (the `model` header, weight
// declarations and `target hardware` budget; what `velox build MODEL.vlx` compiles into the
// reference's emitted runner) instead of a builtin configuration; without --weights, the source's
// first safetensors("file", ...) binding is loaded when that file exists (beside the source or in
// the working directory), else the synthetic model runs.
// --prefill-chunk N (2..128) prefills the prompt N positions per batched step (one weight pass per
// chunk) instead of the reference's one decode step per prompt token; TTFT reports either.
// --quantize MODE (or --quantize=MODE) converts fp32 weights at load as the reference runner does
// (velox_cuda_runner.cu:356-372): f16 / fp16 to fp16 rows, q4_0 / int4 / w4a16 to its group-64
// format, any other value keeps fp32 rows; ggml_q4_0 quantizes to GGML Q4_0 on the device. Without
// it a safetensors checkpoint keeps fp32 rows (the reference runner's default) and the synthetic
// model is GGML Q4_0 (the benchmark format). --unquantized f32|f16 keeps the synthetic weights as
// fp32 / fp16 rows.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "velox_hip.h"

namespace {
bool file_exists(const std::string& p) {
    FILE* f = std::fopen(p.c_str(), "rb");
    if (!f) return false;
    std::fclose(f);
    return true;
}

bool is_gguf(const std::string& p) {
    FILE* f = std::fopen(p.c_str(), "rb");
    if (!f) return false;
    char m[4] = {0, 0, 0, 0};
    const size_t n = std::fread(m, 1, 4, f);
    std::fclose(f);
    return n == 4 && !std::memcmp(m, "GGUF", 4);
}
}  // namespace

extern "C" int velox_hip_runner_main(int argc, char** argv, const VeloxHipModelConfig* baked,
                                     void (*step)(VeloxHipArena*, uint64_t, hipStream_t)) {
    std::string model = "llama3_8b", weights, model_file;
    bool model_given = false;
    int qsel = -1;  // weight format: -1 the default of the weight source, else VeloxHipRunOptions.unquantized
    std::vector<uint32_t> tokens;
    uint32_t prompt_len = 128, steps = 32, warmup = 0, layers = 0, context_len = 0, prefill_chunk = 0, attn_splits = 0;
    uint64_t seed = 1234;
    bool graph = true, verbose = false;
    for (int i = 1; i < argc; ++i) {
        const char* a = argv[i];
        auto next = [&]() -> const char* {
            if (i + 1 >= argc) { std::fprintf(stderr, "Error: %s needs a value\n", a); std::exit(1); }
            return argv[++i];
        };
        if (baked && (!std::strcmp(a, "--model") || !std::strcmp(a, "--model-file"))) {
            std::fprintf(stderr, "Error: this runner is built for model %s (%s is not taken)\n", baked->name, a);
            return 1;
        }
        if (!std::strcmp(a, "--model")) { model = next(); model_given = true; }
        else if (!std::strcmp(a, "--model-file")) model_file = next();
        else if (!std::strcmp(a, "--unquantized")) {
            const char* f = next();
            if (!std::strcmp(f, "f32")) qsel = 1;
            else if (!std::strcmp(f, "f16")) qsel = 2;
            else { std::fprintf(stderr, "Error: --unquantized takes f32 or f16\n"); return 1; }
        }
        else if (!std::strcmp(a, "--quantize") || !std::strncmp(a, "--quantize=", 11)) {
            const char* f = a[10] == '=' ? a + 11 : next();
            if (!std::strcmp(f, "f16") || !std::strcmp(f, "fp16")) qsel = 2;
            else if (!std::strcmp(f, "q4_0") || !std::strcmp(f, "int4") || !std::strcmp(f, "w4a16")) qsel = 3;
            else if (!std::strcmp(f, "ggml_q4_0")) qsel = 0;
            else qsel = 1;
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
        else if (!std::strcmp(a, "--attn-splits")) attn_splits = (uint32_t)std::atoi(next());
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
            weights = std::strcmp(w, "synthetic") ? w : "";
            if (!weights.empty() && !file_exists(weights)) {
                std::fprintf(stderr, "Error: failed to open weights file '%s'\n", w);
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
    if (weights.empty() && !model_file.empty()) {
        // the source's own weight binding, as the CLI resolves it (src/cli.rs:1400-1414)
        VeloxHipModelConfig c;
        VeloxHipVlxTarget t;
        if (velox_hip_vlx_load(model_file.c_str(), 0, &c, &t) == 0 && t.weights_file[0]) {
            const std::string dir = model_file.find('/') == std::string::npos
                                        ? std::string(".")
                                        : model_file.substr(0, model_file.rfind('/'));
            for (const std::string& cand : {dir + "/" + t.weights_file, std::string(t.weights_file)})
                if (file_exists(cand)) { weights = cand; break; }
        }
    }
    const bool gguf = !weights.empty() && is_gguf(weights);
    const bool st_file = !weights.empty() && !gguf;
    const uint32_t unquantized = qsel >= 0 ? (uint32_t)qsel : st_file ? 1u : 0u;

    VeloxHipRunOptions opt;
    std::memset(&opt, 0, sizeof(opt));
    opt.model = st_file && !model_given ? nullptr : model.c_str();
    opt.model_config = baked;
    opt.attn_splits = attn_splits;
    opt.decode_step = step;
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
        const char* why = rc == VELOX_HIP_EINVAL     ? " (invalid argument: token id >= vocab, unsupported shape or "
                                                       "malformed file)"
                          : rc == VELOX_HIP_ETENSOR  ? " ([E013] checkpoint tensor missing or outside the file)"
                          : rc == VELOX_HIP_EDTYPE   ? " ([E014] checkpoint tensor dtype not F32, F16 or BF16)"
                          : rc == VELOX_HIP_ESHAPE   ? " (checkpoint tensor shape does not match the model)"
                          : rc == VELOX_HIP_ENOMEM   ? " ([E002] plan exceeds the VRAM budget)"
                          : rc == VELOX_HIP_ENOTLOADED ? " (file could not be read)"
                                                       : "";
        std::fprintf(stderr, "HIP error detected: status %d%s\n", rc, why);
        return 1;
    }
    // ring[p] = argmax after position p; generated tokens start at p = prompt_len - 1
    const uint32_t first = prompt_len - 1;
    const uint32_t n_gen = (uint32_t)std::min<size_t>(rep.n_tokens - first, (size_t)warmup + opt.steps + 1);
    for (uint32_t s = 0; s < n_gen; ++s) std::printf("[Step %u] Token: %u\n", s, out[first + s]);
    std::printf("================================================================================\n");
    std::printf("VELOX MI355X HIP RUNTIME EXECUTION REPORT\n");
    std::printf("================================================================================\n");
    const char* fmt = unquantized == 1   ? "fp32 rows"
                      : unquantized == 2 ? "fp16 rows"
                      : unquantized == 3 ? "group-64 4-bit"
                                         : "Q4_0";
    if (weights.empty()) {
        std::printf("Model                  : %s (synthetic %s, seed %llu)\n",
                    baked ? baked->name : model_file.empty() ? model.c_str() : model_file.c_str(), fmt,
                    (unsigned long long)seed);
        std::printf("Weight Synthesis       : %.2f ms\n", rep.load_ms);
    } else if (gguf) {
        std::printf("Model                  : %s (GGUF Q4_0)\n", weights.c_str());
        std::printf("Weight Load            : %.2f ms\n", rep.load_ms);
    } else {
        std::printf("Model                  : %s (safetensors, %s)\n", weights.c_str(), fmt);
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
