// parity_audit.cpp - the reference's parity-audit program (src/parity_audit.cu) on this
// build: the same file protocol, so the same data directory drives both.
//
//   data_dir/config.txt          B T C L H V (whitespace separated; d_ff = 4C, d_head = C/H)
//   data_dir/pytorch_params.bin  the flat fp32 parameter buffer (src/model.cu:185-217 order)
//   data_dir/inputs.bin          B*T int32 tokens
//   data_dir/targets.bin         B*T int32 targets
// writes
//   data_dir/cuda_logits.bin     (B*T, V) fp32 logits of the forward
//   data_dir/cuda_loss.bin       one fp32: the mean cross-entropy
//   data_dir/cuda_grads.bin      the flat fp32 gradient buffer
//
// Attention: the reference's default materialised mode; --tiled_attn the tiled launcher
// sequence (as the reference's flag); --fused_attn this build's fused path; --fused_x3_attn
// the fused path on the bf16 matrix cores with three-plane fp32 operands.
#include <cstdio>
#include <fstream>
#include <iostream>
#include <string>
#include <vector>

#include "common.h"
#include "gpt_capi.h"

namespace {

bool read_file(const std::string& path, void* dst, size_t bytes) {
    std::ifstream in(path, std::ios::binary);
    if (!in) return false;
    in.read(static_cast<char*>(dst), static_cast<std::streamsize>(bytes));
    return static_cast<size_t>(in.gcount()) == bytes;
}

bool write_file(const std::string& path, const void* src, size_t bytes) {
    std::ofstream out(path, std::ios::binary);
    out.write(static_cast<const char*>(src), static_cast<std::streamsize>(bytes));
    return static_cast<bool>(out);
}

int fail(const std::string& what) {
    std::cerr << "[Parity Audit] error: " << what << "\n";
    return 1;
}

}  // namespace

int main(int argc, char** argv) {
    std::string data_dir = "tests/parity_data";
    int mode = GPT_ATTN_MATERIALIZED;
    for (int i = 1; i < argc; ++i) {
        const std::string arg = argv[i];
        if (arg == "--tiled_attn") mode = GPT_ATTN_TILED_SPLIT;
        else if (arg == "--fused_attn") mode = GPT_ATTN_FUSED;
        else if (arg == "--fused_x3_attn") mode = GPT_ATTN_FUSED_X3;
        else if (arg.rfind("--", 0) != 0) data_dir = arg;
        else return fail("unknown flag " + arg);
    }
    std::ifstream cfg_in(data_dir + "/config.txt");
    if (!cfg_in) return fail("cannot open " + data_dir + "/config.txt");
    int B = 0, T = 0, C = 0, L = 0, H = 0, V = 0;
    cfg_in >> B >> T >> C >> L >> H >> V;
    if (!cfg_in || B <= 0 || T <= 0 || C <= 0 || L <= 0 || H <= 0 || V <= 0)
        return fail("malformed config.txt");
    gpt_config cfg;
    gpt_default_config(&cfg, V, T, C, L, H, 4 * C, B);
    cfg.attention_mode = mode;
    std::cout << "[Parity Audit] Loading config: B=" << B << ", T=" << T << ", C=" << C
              << ", L=" << L << ", H=" << H << ", V=" << V << ", attention="
              << (mode == GPT_ATTN_FUSED          ? "fused"
                  : mode == GPT_ATTN_FUSED_X3     ? "fused_x3"
                  : mode == GPT_ATTN_TILED_SPLIT  ? "tiled"
                                                  : "materialized")
              << "\n";
    gpt_model* model = nullptr;
    int st = gpt_create(&cfg, &model);
    if (st != 0) return fail("gpt_create status " + std::to_string(st));
    const long long n = gpt_num_parameters(model);
    std::vector<float> params(n);
    if (!read_file(data_dir + "/pytorch_params.bin", params.data(), n * sizeof(float)))
        return fail("pytorch_params.bin does not hold " + std::to_string(n) + " floats");
    if (gpt_set_parameters(model, params.data(), n) != 0) return fail("gpt_set_parameters");
    const size_t tokens = static_cast<size_t>(B) * T;
    std::vector<int> h_in(tokens), h_tg(tokens);
    if (!read_file(data_dir + "/inputs.bin", h_in.data(), tokens * sizeof(int)) ||
        !read_file(data_dir + "/targets.bin", h_tg.data(), tokens * sizeof(int)))
        return fail("inputs.bin / targets.bin");
    int *d_in = nullptr, *d_tg = nullptr;
    float* d_loss = nullptr;
    HIP_CHECK(hipMalloc(&d_in, tokens * sizeof(int)));
    HIP_CHECK(hipMalloc(&d_tg, tokens * sizeof(int)));
    HIP_CHECK(hipMalloc(&d_loss, sizeof(float)));
    HIP_CHECK(hipMemcpy(d_in, h_in.data(), tokens * sizeof(int), hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(d_tg, h_tg.data(), tokens * sizeof(int), hipMemcpyHostToDevice));
    st = gpt_forward_backward(model, d_in, d_tg, d_loss, nullptr);
    if (st != 0) return fail("gpt_forward_backward status " + std::to_string(st));
    HIP_CHECK(hipDeviceSynchronize());
    std::vector<float> logits(tokens * static_cast<size_t>(V));
    if (gpt_get_logits(model, logits.data(), static_cast<long long>(logits.size())) != 0)
        return fail("gpt_get_logits");
    float loss = 0.0f;
    HIP_CHECK(hipMemcpy(&loss, d_loss, sizeof(float), hipMemcpyDeviceToHost));
    std::vector<float> grads(n);
    if (gpt_get_gradients(model, grads.data(), n) != 0) return fail("gpt_get_gradients");
    if (!write_file(data_dir + "/cuda_logits.bin", logits.data(), logits.size() * sizeof(float)) ||
        !write_file(data_dir + "/cuda_loss.bin", &loss, sizeof(float)) ||
        !write_file(data_dir + "/cuda_grads.bin", grads.data(), grads.size() * sizeof(float)))
        return fail("writing outputs");
    std::cout << "[Parity Audit] Completed forward & backward pass. Loss: " << loss << "\n";
    std::cout << "[Parity Audit] Tensors written to " << data_dir << "\n";
    (void)hipFree(d_in);
    (void)hipFree(d_tg);
    (void)hipFree(d_loss);
    gpt_destroy(model);
    return 0;
}
