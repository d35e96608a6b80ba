// Runs the reference's GPT model (src/model/gpt.cpp, unchanged) forward and
// backward on three backends from the same weights and tokens and writes the
// 16 weight gradients of each, packed as in gpt_weights:
//   the reference CPUBackend (src/backend/cpu/cpu_backend.cpp),
//   HipAttnBackend (gpt_amd/adapter/hip_attn_backend.*: the attention op pair
//     on the GPU through libgpt_hip_attn.so, every other op the CPU backend's),
//   HipBackend (gpt_amd/adapter/hip_backend.*: every op on the GPU).
//
// TEST INFRASTRUCTURE ONLY (tests/test_gpt_grads_d64_gpu.py). It repeats the
// sequence of the reference's gpt_test run_and_download_grads
// (src/model/gpt_test.cpp:148-164: zero_grad, forward, backward, loss) for a
// config given on the command line, so that the model's attention runs at
// head_dim 64 (the hot path's MFMA kernels) instead of gpt_test's 8. Inputs
// are tokens[0 .. B*T), labels tokens[1 .. B*T], as gpt_test shifts them.
//
// Usage: gpt_grad_check cpu|gpu V VP L H D F S B T tokens.bin weights.bin out_prefix
//   cpu: the CPU backend only (out_prefix + "cpu.bin"); gpu: the two HIP
//   backends (out_prefix + "attn.bin", "full.bin"); one loss line each
#include "cpu_backend.h"
#include "gpt.h"
#include "hip_attn_backend.h"
#include "hip_backend.h"

#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

static bool run(IGPTBackend *be, const gpt_config &cfg, int B, int T, const std::vector<int> &tokens,
                const char *weights, const std::string &out, const char *label)
{
    GPT model(be, const_cast<gpt_config *>(&cfg), true);
    if (!model.load_checkpoint(weights))
        return false;
    model.set_size(B, T);
    int *dev = nullptr;
    be->device_malloc((void **)&dev, tokens.size() * sizeof(int));
    be->device_memcpy_h2d(dev, tokens.data(), tokens.size() * sizeof(int));
    model.zero_grad();
    model.forward(dev);
    model.backward(dev, dev + 1);
    const float loss = model.loss(dev + 1);
    const gpt_weights *g = model.grad_weights();
    std::vector<float> host(g->buffer_count_);
    be->device_memcpy_d2h(host.data(), g->buffer_, host.size() * sizeof(float));
    be->device_free(dev);
    FILE *fp = std::fopen(out.c_str(), "wb");
    if (!fp || std::fwrite(host.data(), sizeof(float), host.size(), fp) != host.size())
    {
        std::fprintf(stderr, "cannot write %s\n", out.c_str());
        return false;
    }
    std::fclose(fp);
    std::printf("%s loss %.7f gradients %zu\n", label, loss, host.size());
    std::fflush(stdout);
    return true;
}

int main(int argc, char **argv)
{
    if (argc != 14 || (std::string(argv[1]) != "cpu" && std::string(argv[1]) != "gpu"))
    {
        std::fprintf(stderr, "usage: %s cpu|gpu V VP L H D F S B T tokens.bin weights.bin out_prefix\n", argv[0]);
        return 2;
    }
    const bool cpu = std::string(argv[1]) == "cpu";
    ++argv;
    gpt_config cfg;
    cfg.vocab_size = std::atoi(argv[1]);
    cfg.vocab_size_padded = std::atoi(argv[2]);
    cfg.num_layers = std::atoi(argv[3]);
    cfg.num_heads = std::atoi(argv[4]);
    cfg.d_model = std::atoi(argv[5]);
    cfg.d_ffn = std::atoi(argv[6]);
    cfg.max_seq_len = std::atoi(argv[7]);
    const int B = std::atoi(argv[8]), T = std::atoi(argv[9]);
    const std::string prefix = argv[12];

    std::vector<int> tokens((size_t)B * T + 1);
    FILE *fp = std::fopen(argv[10], "rb");
    if (!fp || std::fread(tokens.data(), sizeof(int), tokens.size(), fp) != tokens.size())
    {
        std::fprintf(stderr, "cannot read %s\n", argv[10]);
        return 1;
    }
    std::fclose(fp);

    if (cpu)
    {
        CPUBackend be;
        return run(&be, cfg, B, T, tokens, argv[11], prefix + "cpu.bin", "cpu") ? 0 : 1;
    }
    {
        HipAttnBackend be;
        if (!run(&be, cfg, B, T, tokens, argv[11], prefix + "attn.bin", "attn"))
            return 1;
    }
    {
        HipBackend be;
        if (!run(&be, cfg, B, T, tokens, argv[11], prefix + "full.bin", "full"))
            return 1;
    }
    return 0;
}
