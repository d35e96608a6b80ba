// Runs the reference's GPT model (src/model/gpt.cpp) on the reference's
// CPUBackend (src/backend/cpu/cpu_backend.cpp) for the gpt_test config and
// writes the 16 weight gradients, packed as in gpt_weights, to a file.
//
// TEST INFRASTRUCTURE ONLY: used to pin the independent PyTorch restatement
// in tests/golden/make_gpt_fixtures.py against the reference model on the
// CPU. It repeats the sequence of gpt_test's run_and_download_grads
// (src/model/gpt_test.cpp:148-164): zero_grad, forward, backward, loss.
//
// Usage: gpt_cpu_grads <tokens.bin> <weights.bin> <grads_out.bin>
#include "cpu_backend.h"
#include "gpt.h"

#include <cstdio>
#include <cstdlib>
#include <vector>

int main(int argc, char **argv)
{
    if (argc != 4)
    {
        std::fprintf(stderr, "usage: %s tokens.bin weights.bin grads_out.bin\n", argv[0]);
        return 2;
    }
    gpt_config cfg;
    cfg.max_seq_len = 64;
    cfg.vocab_size = 507;
    cfg.vocab_size_padded = 512;
    cfg.num_layers = 4;
    cfg.num_heads = 4;
    cfg.d_model = 32;
    cfg.d_ffn = 256;
    const int T = cfg.max_seq_len;

    std::vector<int> tokens(T + 1);
    FILE *fp = std::fopen(argv[1], "rb");
    if (!fp || std::fread(tokens.data(), sizeof(int), T + 1, fp) != (size_t)(T + 1))
    {
        std::fprintf(stderr, "cannot read %s\n", argv[1]);
        return 1;
    }
    std::fclose(fp);

    CPUBackend be;
    GPT model(&be, &cfg, true);
    if (!model.load_checkpoint(argv[2]))
        return 1;
    model.set_size(1, T);
    model.zero_grad();
    model.forward(tokens.data());
    model.backward(tokens.data(), tokens.data() + 1);
    const float loss = model.loss(tokens.data() + 1);

    const gpt_weights *g = model.grad_weights();
    fp = std::fopen(argv[3], "wb");
    if (!fp || std::fwrite(g->buffer_, sizeof(float), g->buffer_count_, fp) != g->buffer_count_)
    {
        std::fprintf(stderr, "cannot write %s\n", argv[3]);
        return 1;
    }
    std::fclose(fp);
    std::printf("loss %.6f, %zu gradients\n", loss, g->buffer_count_);
    return 0;
}
