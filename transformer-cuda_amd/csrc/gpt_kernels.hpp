// gpt_kernels.hpp - launchers of the GPT training-step harness kernels (gpt_kernels.hip).
// All tensors row-major fp32 device buffers; every launcher enqueues on stream s.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

namespace tcamd {
namespace gpt {

struct AdamWParams {
    float lr, beta1, beta2, eps, weight_decay, max_norm;
    float bc1, bc2;  // bias corrections 1 - beta^step
};

void embedding_forward(const int* tokens, const float* tok_emb, const float* pos_emb, float* out,
                       int B, int T, int C, hipStream_t s);
// d_tok_emb is accumulated into (zeroed by the caller); d_pos_emb is written.
void embedding_backward(const int* tokens, const float* dx, float* d_tok_emb, float* d_pos_emb,
                        float* scratch, int B, int T, int C, hipStream_t s);

// out[n] = sum_r x[r, n]; scratch: column_sum_scratch(R, N) floats.
size_t column_sum_scratch(int R, int N);
void column_sum(const float* x, int R, int N, float* out, float* scratch, hipStream_t s);
// out[i] = sum_j x[j * n + i] over nslice slices of n floats.
void sum_slices(const float* x, int nslice, int n, float* out, hipStream_t s);

void layernorm_forward(const float* x, const float* gamma, const float* beta, float* y,
                       float* mean, float* rstd, int R, int C, float eps, hipStream_t s);
// dx written (or added to when accumulate); dgamma, dbeta written.
void layernorm_backward(const float* dy, const float* x, const float* gamma, const float* mean,
                        const float* rstd, float* dx, float* dgamma, float* dbeta, float* scratch,
                        int R, int C, bool accumulate, hipStream_t s);

void add_bias(float* y, const float* b, int R, int N, hipStream_t s);
void bias_residual(const float* res, const float* y, const float* b, float* out, int R, int N,
                   hipStream_t s);
void bias_gelu_forward(const float* y, const float* b, float* out, int R, int N, hipStream_t s);
void bias_gelu_backward(const float* dout, const float* y, const float* b, float* dy, int R,
                        int N, hipStream_t s);

// Mean cross-entropy into *loss (device), dlogits = (softmax - onehot) / rows.
void cross_entropy(const float* logits, const int* targets, float* dlogits, float* row_loss,
                   float* loss, int rows, int V, hipStream_t s);

// Global-norm clip + AdamW (decoupled weight decay) + zero the gradient, one pass over the
// flat buffers; norm_scratch holds 1 + adamw_norm_blocks() floats (norm first).
int adamw_norm_blocks();
void clip_adamw_zero(float* params, float* grads, float* m, float* v, float* norm_scratch,
                     long long n, const AdamWParams& a, hipStream_t s);

}  // namespace gpt
}  // namespace tcamd
