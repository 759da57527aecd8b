// gpt_kernels.hip - the element-wise and reduction kernels of the GPT training-step harness
// around the attention path (fp32): embedding, LayerNorm, bias + GELU, bias + residual,
// column sums (bias and LayerNorm parameter gradients), fused cross-entropy, and the fused
// gradient-clip + AdamW + zero-grad update.
//
// Reference (behaviour, one kernel family each): src/kernels/embedding.cu (token + position
// gather, scatter-add backward), src/kernels/layernorm.cu:29-303 (biased variance, eps inside
// the square root), src/kernels/ffn.cu:8-166 (tanh-approximated GELU), src/kernels/loss.cu:
// 24-125 (mean cross-entropy, dlogits = (softmax - onehot) / (B*T)), src/optimizer.cu:117-154
// (global-norm clip folded into AdamW with decoupled weight decay, then zero the gradient).
//
// Row kernels run one wave64 per row with shuffle reductions; reductions over rows (bias,
// gamma, beta and position-embedding gradients) are two-stage and deterministic: partial sums
// over fixed row chunks, then a sum of the chunks in chunk order.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "gpt_kernels.hpp"

namespace tcamd {
namespace gpt {
namespace {

constexpr int kWave = 64;
constexpr int kBlock = 256;
constexpr int kRowsPerBlock = kBlock / kWave;

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int off = kWave / 2; off >= 1; off >>= 1) x += __shfl_xor(x, off, kWave);
    return x;
}
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int off = kWave / 2; off >= 1; off >>= 1) x = fmaxf(x, __shfl_xor(x, off, kWave));
    return x;
}

inline unsigned blocks_for(long long n, int per_block) {
    return static_cast<unsigned>((n + per_block - 1) / per_block);
}

// ---- embedding ------------------------------------------------------------------------
__global__ void embedding_fwd_kernel(const int* __restrict__ tokens,
                                     const float* __restrict__ tok_emb,
                                     const float* __restrict__ pos_emb, float* __restrict__ out,
                                     int BT, int T, int C) {
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<long long>(BT) * C) return;
    const int row = static_cast<int>(i / C), c = static_cast<int>(i % C);
    out[i] = tok_emb[static_cast<long long>(tokens[row]) * C + c] +
             pos_emb[static_cast<long long>(row % T) * C + c];
}

// d_tok_emb[token] += dx[row] (tokens repeat: atomic adds).
__global__ void embedding_tok_bwd_kernel(const int* __restrict__ tokens,
                                         const float* __restrict__ dx,
                                         float* __restrict__ d_tok_emb, int BT, int C) {
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<long long>(BT) * C) return;
    const int row = static_cast<int>(i / C), c = static_cast<int>(i % C);
    atomicAdd(&d_tok_emb[static_cast<long long>(tokens[row]) * C + c], dx[i]);
}

// ---- column sums: out[n] = sum_r x[r, n] (beta: out = sum + beta*out) -----------------
constexpr int kChunkRows = 128;

// partial[chunk][n] = sum over the chunk's rows; with ln_x != nullptr the summand is
// x[r,n] times the normalised input (ln_x[r,n] - mean[r]) * rstd[r] (the LayerNorm gamma
// gradient).  A block covers 64 columns (one wave's lanes, 256 contiguous bytes per row)
// and the chunk's rows split over its 4 waves, two rows in flight per thread; the 4 partial
// sums of a column meet in LDS.
constexpr int kColTile = kWave;
constexpr int kColLanes = kBlock / kColTile;
__global__ __launch_bounds__(kBlock) void colsum_partial_kernel(
    const float* __restrict__ x, int R, int N, const float* __restrict__ ln_x,
    const float* __restrict__ ln_mean, const float* __restrict__ ln_rstd,
    float* __restrict__ partial) {
    __shared__ float red[kColLanes][kColTile];
    const int c = threadIdx.x % kColTile, j = threadIdx.x / kColTile;
    const int n = blockIdx.x * kColTile + c;
    const int r0 = blockIdx.y * kChunkRows, r1 = min(R, r0 + kChunkRows);
    auto term = [&](int r) {
        const long long i = static_cast<long long>(r) * N + n;
        return ln_x != nullptr ? x[i] * ((ln_x[i] - ln_mean[r]) * ln_rstd[r]) : x[i];
    };
    float s0 = 0.0f, s1 = 0.0f;
    if (n < N) {
        int r = r0 + j;
        for (; r + kColLanes < r1; r += 2 * kColLanes) {
            s0 += term(r);
            s1 += term(r + kColLanes);
        }
        if (r < r1) s0 += term(r);
    }
    red[j][c] = s0 + s1;
    __syncthreads();
    if (j == 0 && n < N) {
        float t = red[0][c];
#pragma unroll
        for (int i = 1; i < kColLanes; ++i) t += red[i][c];
        partial[static_cast<long long>(blockIdx.y) * N + n] = t;
    }
}

// out[n] = sum over the nchunk partial rows: a block covers 16 columns, its 16 lanes per
// column stride over the chunks.
constexpr int kFinCols = 16;
constexpr int kFinLanes = kBlock / kFinCols;
__global__ __launch_bounds__(kBlock) void colsum_final_kernel(const float* __restrict__ partial,
                                                              int nchunk, int N,
                                                              float* __restrict__ out) {
    __shared__ float red[kFinLanes][kFinCols + 1];
    const int c = threadIdx.x % kFinCols, j = threadIdx.x / kFinCols;
    const int n = blockIdx.x * kFinCols + c;
    float s = 0.0f;
    if (n < N) {
        for (int k = j; k < nchunk; k += kFinLanes) s += partial[static_cast<long long>(k) * N + n];
    }
    red[j][c] = s;
    __syncthreads();
    if (j == 0 && n < N) {
        float t = red[0][c];
        for (int i = 1; i < kFinLanes; ++i) t += red[i][c];
        out[n] = t;
    }
}

// out[i] = sum_j x[j*n + i]: one thread per element (n large, few slices).
__global__ __launch_bounds__(kBlock) void slice_sum_kernel(const float* __restrict__ x,
                                                           int nslice, int n,
                                                           float* __restrict__ out) {
    const int i = blockIdx.x * kBlock + threadIdx.x;
    if (i >= n) return;
    float s = 0.0f;
    for (int j = 0; j < nslice; ++j) s += x[static_cast<long long>(j) * n + i];
    out[i] = s;
}

// ---- LayerNorm ---------------------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void layernorm_fwd_kernel(
    const float* __restrict__ x, const float* __restrict__ gamma,
    const float* __restrict__ beta, float* __restrict__ y, float* __restrict__ mean_out,
    float* __restrict__ rstd_out, int R, int C, float eps) {
    const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    if (row >= R) return;
    const float* xr = x + static_cast<long long>(row) * C;
    float s = 0.0f;
    for (int c = lane; c < C; c += kWave) s += xr[c];
    const float mean = wave_sum(s) / C;
    float v = 0.0f;
    for (int c = lane; c < C; c += kWave) {
        const float d = xr[c] - mean;
        v = fmaf(d, d, v);
    }
    const float rstd = 1.0f / sqrtf(wave_sum(v) / C + eps);
    float* yr = y + static_cast<long long>(row) * C;
    for (int c = lane; c < C; c += kWave) yr[c] = fmaf((xr[c] - mean) * rstd, gamma[c], beta[c]);
    if (lane == 0) {
        mean_out[row] = mean;
        rstd_out[row] = rstd;
    }
}

// dx = rstd * (g - mean(g) - xhat * mean(g * xhat)), g = dy * gamma; dx is added to
// (accumulate) or written.
__global__ __launch_bounds__(kBlock) void layernorm_bwd_kernel(
    const float* __restrict__ dy, const float* __restrict__ x, const float* __restrict__ gamma,
    const float* __restrict__ mean, const float* __restrict__ rstd, float* __restrict__ dx,
    int R, int C, int accumulate) {
    const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    if (row >= R) return;
    const long long base = static_cast<long long>(row) * C;
    const float mu = mean[row], rs = rstd[row];
    float sg = 0.0f, sgx = 0.0f;
    for (int c = lane; c < C; c += kWave) {
        const float g = dy[base + c] * gamma[c];
        sg += g;
        sgx = fmaf(g, (x[base + c] - mu) * rs, sgx);
    }
    const float mg = wave_sum(sg) / C, mgx = wave_sum(sgx) / C;
    for (int c = lane; c < C; c += kWave) {
        const float g = dy[base + c] * gamma[c];
        const float xh = (x[base + c] - mu) * rs;
        const float d = rs * (g - mg - xh * mgx);
        dx[base + c] = accumulate ? dx[base + c] + d : d;
    }
}

// ---- bias, residual, GELU -------------------------------------------------------------------
__global__ void add_bias_kernel(float* __restrict__ y, const float* __restrict__ b, long long n,
                                int N) {
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) y[i] += b[i % N];
}

// out = res + y + b
__global__ void bias_residual_kernel(const float* __restrict__ res, const float* __restrict__ y,
                                     const float* __restrict__ b, float* __restrict__ out,
                                     long long n, int N) {
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) out[i] = res[i] + y[i] + b[i % N];
}

constexpr float kGeluC = 0.7978845608028654f;  // sqrt(2/pi)
constexpr float kGeluA = 0.044715f;

// out = gelu_tanh(y + b)
__global__ void bias_gelu_fwd_kernel(const float* __restrict__ y, const float* __restrict__ b,
                                     float* __restrict__ out, long long n, int N) {
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float x = y[i] + b[i % N];
    const float t = tanhf(kGeluC * (x + kGeluA * x * x * x));
    out[i] = 0.5f * x * (1.0f + t);
}

// dy = dout * gelu_tanh'(y + b)
__global__ void bias_gelu_bwd_kernel(const float* __restrict__ dout, const float* __restrict__ y,
                                     const float* __restrict__ b, float* __restrict__ dy,
                                     long long n, int N) {
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float x = y[i] + b[i % N];
    const float u = kGeluC * (x + kGeluA * x * x * x);
    const float t = tanhf(u);
    const float du = kGeluC * (1.0f + 3.0f * kGeluA * x * x);
    dy[i] = dout[i] * (0.5f * (1.0f + t) + 0.5f * x * (1.0f - t * t) * du);
}

// ---- cross-entropy ----------------------------------------------------------------------
// One workgroup per row: loss_row = logsumexp(z) - z[target]; dz = (softmax(z) - onehot)
// * inv_rows.  Row losses are summed by a second pass (deterministic).
__global__ __launch_bounds__(kBlock) void cross_entropy_kernel(
    const float* __restrict__ logits, const int* __restrict__ targets,
    float* __restrict__ dlogits, float* __restrict__ row_loss, int V, float inv_rows) {
    __shared__ float red[kBlock / kWave];
    const int row = blockIdx.x;
    const int tid = threadIdx.x, lane = tid % kWave, w = tid / kWave;
    const float* z = logits + static_cast<long long>(row) * V;
    // one pass for the maximum and the sum of exponentials (a thread's running sum is
    // rescaled when its maximum grows), then the thread sums are brought to the row maximum
    float tm = -INFINITY, ts = 0.0f;
    for (int i = tid; i < V; i += kBlock) {
        const float zi = z[i];
        if (zi > tm) {
            ts = ts * expf(tm - zi) + 1.0f;
            tm = zi;
        } else {
            ts += expf(zi - tm);
        }
    }
    float mx = wave_max(tm);
    if (lane == 0) red[w] = mx;
    __syncthreads();
    mx = red[0];
    for (int i = 1; i < kBlock / kWave; ++i) mx = fmaxf(mx, red[i]);
    __syncthreads();
    float s = tm == -INFINITY ? 0.0f : ts * expf(tm - mx);
    s = wave_sum(s);
    if (lane == 0) red[w] = s;
    __syncthreads();
    s = 0.0f;
    for (int i = 0; i < kBlock / kWave; ++i) s += red[i];
    const float lse = mx + logf(s);
    const int tgt = targets[row];
    float* dz = dlogits + static_cast<long long>(row) * V;
    for (int i = tid; i < V; i += kBlock) {
        const float p = expf(z[i] - lse);
        dz[i] = (p - (i == tgt ? 1.0f : 0.0f)) * inv_rows;
    }
    if (tid == 0) row_loss[row] = lse - z[tgt];
}

__global__ void mean_kernel(const float* __restrict__ x, int n, float* __restrict__ out) {
    __shared__ float red[kBlock / kWave];
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += kBlock) s += x[i];
    s = wave_sum(s);
    if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = 0.0f;
        for (int i = 0; i < kBlock / kWave; ++i) t += red[i];
        *out = t / n;
    }
}

// ---- gradient norm + AdamW ------------------------------------------------------------------
__global__ __launch_bounds__(kBlock) void sumsq_partial_kernel(const float* __restrict__ g,
                                                               long long n,
                                                               float* __restrict__ partial) {
    __shared__ float red[kBlock / kWave];
    float s = 0.0f;
    for (long long i = static_cast<long long>(blockIdx.x) * kBlock + threadIdx.x; i < n;
         i += static_cast<long long>(gridDim.x) * kBlock)
        s = fmaf(g[i], g[i], s);
    s = wave_sum(s);
    if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = 0.0f;
        for (int i = 0; i < kBlock / kWave; ++i) t += red[i];
        partial[blockIdx.x] = t;
    }
}

__global__ void norm_final_kernel(const float* __restrict__ partial, int n,
                                  float* __restrict__ norm) {
    __shared__ float red[kBlock / kWave];
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += kBlock) s += partial[i];
    s = wave_sum(s);
    if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = 0.0f;
        for (int i = 0; i < kBlock / kWave; ++i) t += red[i];
        *norm = sqrtf(t);
    }
}

__global__ void adamw_kernel(float* __restrict__ p, float* __restrict__ g, float* __restrict__ m,
                             float* __restrict__ v, const float* __restrict__ norm, long long n,
                             AdamWParams a) {
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float nrm = *norm;
    float gi = g[i];
    if (nrm > a.max_norm && nrm > 1e-6f) gi *= a.max_norm / nrm;
    const float mt = a.beta1 * m[i] + (1.0f - a.beta1) * gi;
    const float vt = a.beta2 * v[i] + (1.0f - a.beta2) * gi * gi;
    m[i] = mt;
    v[i] = vt;
    const float mh = mt / a.bc1, vh = vt / a.bc2;
    const float pi = p[i];
    p[i] = pi - a.lr * (mh / (sqrtf(vh) + a.eps) + a.weight_decay * pi);
    g[i] = 0.0f;
}

}  // namespace

void embedding_forward(const int* tokens, const float* tok_emb, const float* pos_emb, float* out,
                       int B, int T, int C, hipStream_t s) {
    const long long n = static_cast<long long>(B) * T * C;
    hipLaunchKernelGGL(embedding_fwd_kernel, dim3(blocks_for(n, kBlock)), dim3(kBlock), 0, s,
                       tokens, tok_emb, pos_emb, out, B * T, T, C);
}

void embedding_backward(const int* tokens, const float* dx, float* d_tok_emb, float* d_pos_emb,
                        float* scratch, int B, int T, int C, hipStream_t s) {
    const long long n = static_cast<long long>(B) * T * C;
    hipLaunchKernelGGL(embedding_tok_bwd_kernel, dim3(blocks_for(n, kBlock)), dim3(kBlock), 0, s,
                       tokens, dx, d_tok_emb, B * T, C);
    // d_pos_emb[t, c] = sum_b dx[b, t, c]: column sums of a (B, T*C) matrix
    column_sum(dx, B, T * C, d_pos_emb, scratch, s);
}

size_t column_sum_scratch(int R, int N) {
    return static_cast<size_t>((R + kChunkRows - 1) / kChunkRows) * N;
}

void column_sum(const float* x, int R, int N, float* out, float* scratch, hipStream_t s) {
    const int nchunk = (R + kChunkRows - 1) / kChunkRows;
    hipLaunchKernelGGL(colsum_partial_kernel, dim3(blocks_for(N, kColTile), nchunk),
                       dim3(kBlock), 0, s, x, R, N, nullptr, nullptr, nullptr, scratch);
    hipLaunchKernelGGL(colsum_final_kernel, dim3(blocks_for(N, kFinCols)), dim3(kBlock), 0, s,
                       scratch, nchunk, N, out);
}

void sum_slices(const float* x, int nslice, int n, float* out, hipStream_t s) {
    hipLaunchKernelGGL(slice_sum_kernel, dim3(blocks_for(n, kBlock)), dim3(kBlock), 0, s, x,
                       nslice, n, out);
}

void layernorm_forward(const float* x, const float* gamma, const float* beta, float* y,
                       float* mean, float* rstd, int R, int C, float eps, hipStream_t s) {
    hipLaunchKernelGGL(layernorm_fwd_kernel, dim3(blocks_for(R, kRowsPerBlock)), dim3(kBlock), 0,
                       s, x, gamma, beta, y, mean, rstd, R, C, eps);
}

void layernorm_backward(const float* dy, const float* x, const float* gamma, const float* mean,
                        const float* rstd, float* dx, float* dgamma, float* dbeta, float* scratch,
                        int R, int C, bool accumulate, hipStream_t s) {
    hipLaunchKernelGGL(layernorm_bwd_kernel, dim3(blocks_for(R, kRowsPerBlock)), dim3(kBlock), 0,
                       s, dy, x, gamma, mean, rstd, dx, R, C, accumulate ? 1 : 0);
    const int nchunk = (R + kChunkRows - 1) / kChunkRows;
    hipLaunchKernelGGL(colsum_partial_kernel, dim3(blocks_for(C, kColTile), nchunk),
                       dim3(kBlock), 0, s, dy, R, C, x, mean, rstd, scratch);
    hipLaunchKernelGGL(colsum_final_kernel, dim3(blocks_for(C, kFinCols)), dim3(kBlock), 0, s,
                       scratch, nchunk, C, dgamma);
    column_sum(dy, R, C, dbeta, scratch, s);
}

void add_bias(float* y, const float* b, int R, int N, hipStream_t s) {
    const long long n = static_cast<long long>(R) * N;
    hipLaunchKernelGGL(add_bias_kernel, dim3(blocks_for(n, kBlock)), dim3(kBlock), 0, s, y, b, n,
                       N);
}

void bias_residual(const float* res, const float* y, const float* b, float* out, int R, int N,
                   hipStream_t s) {
    const long long n = static_cast<long long>(R) * N;
    hipLaunchKernelGGL(bias_residual_kernel, dim3(blocks_for(n, kBlock)), dim3(kBlock), 0, s, res,
                       y, b, out, n, N);
}

void bias_gelu_forward(const float* y, const float* b, float* out, int R, int N, hipStream_t s) {
    const long long n = static_cast<long long>(R) * N;
    hipLaunchKernelGGL(bias_gelu_fwd_kernel, dim3(blocks_for(n, kBlock)), dim3(kBlock), 0, s, y,
                       b, out, n, N);
}

void bias_gelu_backward(const float* dout, const float* y, const float* b, float* dy, int R,
                        int N, hipStream_t s) {
    const long long n = static_cast<long long>(R) * N;
    hipLaunchKernelGGL(bias_gelu_bwd_kernel, dim3(blocks_for(n, kBlock)), dim3(kBlock), 0, s,
                       dout, y, b, dy, n, N);
}

void cross_entropy(const float* logits, const int* targets, float* dlogits, float* row_loss,
                   float* loss, int rows, int V, hipStream_t s) {
    hipLaunchKernelGGL(cross_entropy_kernel, dim3(rows), dim3(kBlock), 0, s, logits, targets,
                       dlogits, row_loss, V, 1.0f / static_cast<float>(rows));
    hipLaunchKernelGGL(mean_kernel, dim3(1), dim3(kBlock), 0, s, row_loss, rows, loss);
}

int adamw_norm_blocks() { return 1024; }

void clip_adamw_zero(float* params, float* grads, float* m, float* v, float* norm_scratch,
                     long long n, const AdamWParams& a, hipStream_t s) {
    const int nb = adamw_norm_blocks();
    hipLaunchKernelGGL(sumsq_partial_kernel, dim3(nb), dim3(kBlock), 0, s, grads, n,
                       norm_scratch + 1);
    hipLaunchKernelGGL(norm_final_kernel, dim3(1), dim3(kBlock), 0, s, norm_scratch + 1, nb,
                       norm_scratch);
    hipLaunchKernelGGL(adamw_kernel, dim3(blocks_for(n, kBlock)), dim3(kBlock), 0, s, params,
                       grads, m, v, norm_scratch, n, a);
}

}  // namespace gpt
}  // namespace tcamd
