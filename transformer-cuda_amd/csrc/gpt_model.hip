// gpt_model.hip - the GPT training-step harness (include/gpt_capi.h): the reference's
// TransformerModel forward/backward (src/model.cu:248-704) and its fused clip + AdamW step
// (src/optimizer.cu:117-154), with the attention of every block on this build's path.
//
// Differences from the reference that a caller sees: fp32 GEMMs run on rocBLAS (the
// reference uses cuBLAS / cuBLASLt); the attention runs in one of four modes
// (gpt_config.attention_mode): the fused path of this build (attention from the packed QKV
// projection output straight into the merged-heads layout, three launches per layer and
// direction) on the fp32 MFMA or, fused_x3, on the bf16 MFMA with fp32 operands as three
// bf16 planes (a plane workspace per layer, kept from the forward to the backward, and one
// dS area for all layers), the reference's tiled launcher sequence (split-transpose, tiled
// attention, head merge), or the reference's default materialised sequence (T x T scores).
#include <hip/hip_runtime.h>
#include <math.h>
#include <rocblas/rocblas.h>
#include <stdint.h>

#include <algorithm>
#include <new>
#include <vector>

#include "../../include/attn_capi.h"
#include "../../include/gpt_capi.h"
#include "gpt_kernels.hpp"

namespace {

using namespace tcamd::gpt;

struct Layer {  // parameter (or gradient) views into a flat buffer
    float *ln1_g, *ln1_b, *qkv_w, *qkv_b, *proj_w, *proj_b, *ln2_g, *ln2_b, *ffn1_w, *ffn1_b,
        *ffn2_w, *ffn2_b;
};
struct Params {
    float *tok_emb, *pos_emb, *lnf_g, *lnf_b, *head_w;
    std::vector<Layer> layers;
};

struct LayerActs {
    float *ln1, *ln1_mean, *ln1_rstd, *qkv, *merged, *attn_m, *attn_l, *res1, *ln2, *ln2_mean,
        *ln2_rstd, *ffn1, *gelu, *out;
    float *q, *k, *v, *attn_out;  // tiled-split and materialised modes
    float* probs;                 // materialised mode (B, H, T, T)
    float* planes;                // fused_x3 mode: the layer's plane workspace
};

long long param_count(const gpt_config& c) {
    const long long V = c.vocab_size, T = c.max_seq_len, C = c.d_model, F = c.d_ff;
    const long long per_layer = 2 * C + C * 3 * C + 3 * C + C * C + C + 2 * C + C * F + F +
                                F * C + C;
    return V * C + T * C + c.num_layers * per_layer + 2 * C + C * V;
}

Params map_params(float* p, const gpt_config& c) {
    const long long V = c.vocab_size, T = c.max_seq_len, C = c.d_model, F = c.d_ff;
    Params r;
    r.tok_emb = p; p += V * C;
    r.pos_emb = p; p += T * C;
    r.layers.resize(c.num_layers);
    for (Layer& l : r.layers) {
        l.ln1_g = p; p += C;
        l.ln1_b = p; p += C;
        l.qkv_w = p; p += C * 3 * C;
        l.qkv_b = p; p += 3 * C;
        l.proj_w = p; p += C * C;
        l.proj_b = p; p += C;
        l.ln2_g = p; p += C;
        l.ln2_b = p; p += C;
        l.ffn1_w = p; p += C * F;
        l.ffn1_b = p; p += F;
        l.ffn2_w = p; p += F * C;
        l.ffn2_b = p; p += C;
    }
    r.lnf_g = p; p += C;
    r.lnf_b = p; p += C;
    r.head_w = p;
    return r;
}

}  // namespace

struct gpt_model {
    gpt_config cfg{};
    long long n_params = 0;
    float *params = nullptr, *grads = nullptr, *adam_m = nullptr, *adam_v = nullptr;
    Params P, G;
    std::vector<LayerActs> acts;
    float *emb = nullptr, *lnf = nullptr, *lnf_mean = nullptr, *lnf_rstd = nullptr,
          *logits = nullptr, *dlogits = nullptr, *row_loss = nullptr;
    // backward scratch shared by the layers
    float *d_x = nullptr, *d_ln = nullptr, *d_qkv = nullptr, *d_merged = nullptr,
          *d_ffn_a = nullptr, *d_ffn_b = nullptr, *ws = nullptr, *colsum = nullptr, *splitk = nullptr,
          *attn_ds = nullptr,  // fused modes: the backward's dS, shared by the layers (null
                               // where the shape takes the two-stage backward)
          *norm = nullptr, *proj = nullptr;
    float *dq = nullptr, *dk = nullptr, *dv = nullptr, *d_attn_out = nullptr;  // split modes
    float *scores = nullptr, *dprobs = nullptr, *dscores = nullptr;          // materialised
    std::vector<void*> allocations;
    rocblas_handle blas = nullptr;
    int step = 0;
    bool timing = false;
    std::vector<hipEvent_t> ev;  // pairs around attention launches
    int ev_used = 0;
};

namespace {

int alloc(gpt_model* m, float** p, long long n) {
    void* q = nullptr;
    if (hipMalloc(&q, static_cast<size_t>(n > 0 ? n : 1) * sizeof(float)) != hipSuccess)
        return ATTN_ERROR_LAUNCH;
    m->allocations.push_back(q);
    *p = static_cast<float*>(q);
    return ATTN_SUCCESS;
}

// Row-major C (M x N) = alpha * op(A) * op(B) + beta * C, A (M x K) or stored (K x M) when
// ta, B (K x N) or stored (N x K) when tb: the column-major product C^T = op(B)^T op(A)^T.
int gemm(rocblas_handle h, bool ta, bool tb, int M, int N, int K, const float* A, const float* B,
         float* C, float beta = 0.0f) {
    const float alpha = 1.0f;
    const rocblas_status st = rocblas_sgemm(
        h, tb ? rocblas_operation_transpose : rocblas_operation_none,
        ta ? rocblas_operation_transpose : rocblas_operation_none, N, M, K, &alpha, B,
        tb ? K : N, A, ta ? M : K, &beta, C, N);
    return st == rocblas_status_success ? ATTN_SUCCESS : ATTN_ERROR_LAUNCH;
}

// Row-major C (M x N) = A (M x K) * B^T with B stored (N x K), as gemm(false, true, ...), with
// K cut into ks slices: one strided-batched product writes the ks partial products to ws
// (ks * M * N floats), a sum over the slices writes C, and one more product adds the K % ks
// remainder.  For a long contraction over a small output (the output head's input gradient,
// K = vocabulary), where a single product runs on a few dozen workgroups.
int gemm_nt_splitk(rocblas_handle h, int M, int N, int K, const float* A, const float* B,
                   float* C, float* ws, int ks, hipStream_t s) {
    const float one = 1.0f, zero = 0.0f;
    const int kc = K / ks, rem = K - kc * ks;
    const rocblas_stride mn = static_cast<rocblas_stride>(M) * N;
    rocblas_status st = rocblas_sgemm_strided_batched(
        h, rocblas_operation_transpose, rocblas_operation_none, N, M, kc, &one, B, K, kc, A, K,
        kc, &zero, ws, N, mn, ks);
    if (st != rocblas_status_success) return ATTN_ERROR_LAUNCH;
    sum_slices(ws, ks, static_cast<int>(mn), C, s);
    if (rem > 0) {
        const size_t off = static_cast<size_t>(kc) * ks;
        st = rocblas_sgemm(h, rocblas_operation_transpose, rocblas_operation_none, N, M, rem, &one,
                           B + off, K, A + off, K, &one, C, N);
    }
    return st == rocblas_status_success ? ATTN_SUCCESS : ATTN_ERROR_LAUNCH;
}

// Row-major C (M x N) = A^T B with A stored (K x M) and B (K x N), as gemm(true, false, ...),
// with K cut into ks slices as in gemm_nt_splitk.  For the weight gradients, whose K is the
// batch of tokens (B*T) and whose outputs (C x 3C, C x F, F x C, C x C) fill few tiles.
int gemm_tn_splitk(rocblas_handle h, int M, int N, int K, const float* A, const float* B,
                   float* C, float* ws, int ks, hipStream_t s) {
    const float one = 1.0f, zero = 0.0f;
    const int kc = K / ks, rem = K - kc * ks;
    const rocblas_stride mn = static_cast<rocblas_stride>(M) * N;
    rocblas_status st = rocblas_sgemm_strided_batched(
        h, rocblas_operation_none, rocblas_operation_transpose, N, M, kc, &one, B, N,
        static_cast<rocblas_stride>(kc) * N, A, M, static_cast<rocblas_stride>(kc) * M, &zero,
        ws, N, mn, ks);
    if (st != rocblas_status_success) return ATTN_ERROR_LAUNCH;
    sum_slices(ws, ks, static_cast<int>(mn), C, s);
    if (rem > 0) {
        const size_t off = static_cast<size_t>(kc) * ks;
        st = rocblas_sgemm(h, rocblas_operation_none, rocblas_operation_transpose, N, M, rem,
                           &one, B + off * N, N, A + off * M, M, &one, C, N);
    }
    return st == rocblas_status_success ? ATTN_SUCCESS : ATTN_ERROR_LAUNCH;
}

// Weight-gradient slices: measured on the MI355X at B*T = 8192, four slices take the C x F
// and F x C gradients from 450 to 275-310 us and the C x C one from 116 to 93 us.
constexpr int kWeightSplitK = 4;
constexpr long long kWeightSplitMaxOut = 1LL << 22;  // outputs up to 4 M floats
bool weight_splitk(const gpt_config& c) {
    return static_cast<long long>(c.batch_size) * c.max_seq_len >= 4096;
}
long long weight_splitk_floats(const gpt_config& c) {
    const long long C = c.d_model, F = c.d_ff;
    long long mn = 0;
    for (long long x : {3 * C * C, C * F, C * C})
        if (x <= kWeightSplitMaxOut) mn = std::max(mn, x);
    return kWeightSplitK * mn;
}

// A weight gradient dW (M x N) = X^T dY over the B*T tokens: sliced when the token count
// and the output size call for it.
int gemm_dw(gpt_model* m, int M, int N, int K, const float* X, const float* dY, float* dW,
            hipStream_t s) {
    if (weight_splitk(m->cfg) && static_cast<long long>(M) * N <= kWeightSplitMaxOut)
        return gemm_tn_splitk(m->blas, M, N, K, X, dY, dW, m->splitk, kWeightSplitK, s);
    return gemm(m->blas, true, false, M, N, K, X, dY, dW);
}

// Slices of the vocabulary contraction, used when V >= 16 C (a long contraction against a
// BT x C output); the partial products take kHeadSplitK * BT * C floats of their own.
constexpr int kHeadSplitK = 8;
bool head_splitk(const gpt_config& c) {
    return c.vocab_size >= 16 * c.d_model &&
           static_cast<long long>(c.batch_size) * c.max_seq_len * c.d_model < (1LL << 31);
}

#define TRY(x)                                 \
    do {                                       \
        const int _st = (x);                   \
        if (_st != ATTN_SUCCESS) return _st;   \
    } while (0)

void attn_mark(gpt_model* m, hipStream_t s) {
    if (!m->timing) return;
    if (m->ev_used == static_cast<int>(m->ev.size())) {
        hipEvent_t e;
        (void)hipEventCreate(&e);
        m->ev.push_back(e);
    }
    (void)hipEventRecord(m->ev[m->ev_used++], s);
}

int attention_forward(gpt_model* m, LayerActs& a, hipStream_t s) {
    const gpt_config& c = m->cfg;
    const int B = c.batch_size, T = c.max_seq_len, H = c.num_heads, d = c.d_model / H;
    const float scale = 1.0f / sqrtf(static_cast<float>(d));
    attn_mark(m, s);
    switch (c.attention_mode) {
        case GPT_ATTN_FUSED:
            TRY(attn_fused_causal_forward_f32(a.qkv, a.merged, B, H, T, d, scale, a.attn_m,
                                              a.attn_l, s));
            break;
        case GPT_ATTN_FUSED_X3:
            TRY(attn_fused_causal_forward_f32x3(a.qkv, a.merged, B, H, T, d, scale, a.attn_m,
                                                a.attn_l, a.planes, s));
            break;
        case GPT_ATTN_TILED_SPLIT:
            TRY(attn_qkv_split_transpose_forward_f32(a.qkv, a.q, a.k, a.v, B, T, H, d, s));
            TRY(attn_tiled_causal_forward_f32(a.q, a.k, a.v, a.attn_out, B, H, T, d, scale,
                                              a.attn_m, a.attn_l, s));
            TRY(attn_head_merge_transpose_forward_f32(a.attn_out, a.merged, B, H, T, d, s));
            break;
        default:
            TRY(attn_qkv_split_transpose_forward_f32(a.qkv, a.q, a.k, a.v, B, T, H, d, s));
            TRY(attn_materialized_causal_forward_f32(a.q, a.k, a.v, m->scores, a.probs,
                                                     a.attn_out, B, H, T, d, scale, s));
            TRY(attn_head_merge_transpose_forward_f32(a.attn_out, a.merged, B, H, T, d, s));
            break;
    }
    attn_mark(m, s);
    return ATTN_SUCCESS;
}

// d_merged (B, T, C) -> d_qkv (B, T, 3C)
int attention_backward(gpt_model* m, LayerActs& a, hipStream_t s) {
    const gpt_config& c = m->cfg;
    const int B = c.batch_size, T = c.max_seq_len, H = c.num_heads, d = c.d_model / H;
    const float scale = 1.0f / sqrtf(static_cast<float>(d));
    attn_mark(m, s);
    switch (c.attention_mode) {
        case GPT_ATTN_FUSED:
            if (m->attn_ds != nullptr)  // dS-first: dK/dV write dS, dQ is computed from it
                TRY(attn_fused_causal_backward_ds_f32(a.qkv, a.merged, m->d_merged, a.attn_m,
                                                      a.attn_l, m->d_qkv, m->ws, m->attn_ds, B, H,
                                                      T, d, scale, s));
            else  // dS above its size limit: the two-stage order, no T^2 workspace
                TRY(attn_fused_causal_backward_f32(a.qkv, a.merged, m->d_merged, a.attn_m,
                                                   a.attn_l, m->d_qkv, m->ws, B, H, T, d, scale,
                                                   s));
            break;
        case GPT_ATTN_FUSED_X3:  // the layer's qkv and planes are the forward's
            TRY(attn_fused_causal_backward_ds_f32x3(a.qkv, a.merged, m->d_merged, a.attn_m,
                                                    a.attn_l, m->d_qkv, m->ws, m->attn_ds, B, H, T,
                                                    d, scale, a.planes, 1, s));
            break;
        case GPT_ATTN_TILED_SPLIT:
            TRY(attn_head_merge_transpose_backward_f32(m->d_merged, m->d_attn_out, B, H, T, d,
                                                       s));
            TRY(attn_tiled_causal_backward_f32(a.q, a.k, a.v, a.attn_out, m->d_attn_out,
                                               a.attn_m, a.attn_l, m->dq, m->dk, m->dv, m->ws, B,
                                               H, T, d, scale, s));
            TRY(attn_qkv_split_transpose_backward_f32(m->dq, m->dk, m->dv, m->d_qkv, B, T, H, d,
                                                      s));
            break;
        default:
            TRY(attn_head_merge_transpose_backward_f32(m->d_merged, m->d_attn_out, B, H, T, d,
                                                       s));
            TRY(attn_materialized_causal_backward_f32(a.q, a.k, a.v, a.probs, m->d_attn_out,
                                                      m->dprobs, m->dscores, m->dq, m->dk,
                                                      m->dv, B, H, T, d, scale, s));
            TRY(attn_qkv_split_transpose_backward_f32(m->dq, m->dk, m->dv, m->d_qkv, B, T, H, d,
                                                      s));
            break;
    }
    attn_mark(m, s);
    return ATTN_SUCCESS;
}

int check_config(const gpt_config& c) {
    if (c.vocab_size <= 0 || c.max_seq_len <= 0 || c.d_model <= 0 || c.num_layers <= 0 ||
        c.num_heads <= 0 || c.d_ff <= 0 || c.batch_size <= 0)
        return ATTN_ERROR_INVALID_DIM;
    if (c.d_model % c.num_heads != 0) return ATTN_ERROR_INVALID_DIM;
    if (c.attention_mode < GPT_ATTN_FUSED || c.attention_mode > GPT_ATTN_FUSED_X3)
        return ATTN_ERROR_INVALID_VALUE;
    const int d = c.d_model / c.num_heads;  // the materialised mode takes any head dimension
    if (c.attention_mode != GPT_ATTN_MATERIALIZED && d != 32 && d != 64 && d != 128)
        return ATTN_ERROR_UNSUPPORTED_HEAD_DIM;
    if (c.attention_mode == GPT_ATTN_FUSED_X3 && d == 128) return ATTN_ERROR_UNSUPPORTED_HEAD_DIM;
    const long long rows = static_cast<long long>(c.batch_size) * c.max_seq_len;
    if (rows * c.vocab_size > 2147483647LL * 8 || rows > 2147483647LL)
        return ATTN_ERROR_INVALID_DIM;
    if (!(c.layernorm_eps > 0.0f) || !(c.learning_rate >= 0.0f) || !(c.adam_eps > 0.0f))
        return ATTN_ERROR_INVALID_VALUE;
    return ATTN_SUCCESS;
}

int create(const gpt_config& c, gpt_model* m) {
    m->cfg = c;
    m->n_params = param_count(c);
    const long long B = c.batch_size, T = c.max_seq_len, C = c.d_model, F = c.d_ff,
                    V = c.vocab_size, H = c.num_heads, BT = B * T;
    TRY(alloc(m, &m->params, m->n_params));
    TRY(alloc(m, &m->grads, m->n_params));
    TRY(alloc(m, &m->adam_m, m->n_params));
    TRY(alloc(m, &m->adam_v, m->n_params));
    for (float* p : {m->params, m->grads, m->adam_m, m->adam_v})
        if (hipMemset(p, 0, m->n_params * sizeof(float)) != hipSuccess) return ATTN_ERROR_LAUNCH;
    m->P = map_params(m->params, c);
    m->G = map_params(m->grads, c);
    m->acts.resize(c.num_layers);
    for (LayerActs& a : m->acts) {
        a = LayerActs{};
        TRY(alloc(m, &a.ln1, BT * C));
        TRY(alloc(m, &a.ln1_mean, BT));
        TRY(alloc(m, &a.ln1_rstd, BT));
        TRY(alloc(m, &a.qkv, BT * 3 * C));
        TRY(alloc(m, &a.merged, BT * C));
        TRY(alloc(m, &a.attn_m, B * H * T));
        TRY(alloc(m, &a.attn_l, B * H * T));
        TRY(alloc(m, &a.res1, BT * C));
        TRY(alloc(m, &a.ln2, BT * C));
        TRY(alloc(m, &a.ln2_mean, BT));
        TRY(alloc(m, &a.ln2_rstd, BT));
        TRY(alloc(m, &a.ffn1, BT * F));
        TRY(alloc(m, &a.gelu, BT * F));
        TRY(alloc(m, &a.out, BT * C));
        if (c.attention_mode == GPT_ATTN_FUSED_X3) {  // the planes only: dS is shared below
            const size_t bytes = attn_f32x3_planes_bytes(static_cast<int>(B), static_cast<int>(H),
                                                         static_cast<int>(T),
                                                         static_cast<int>(C / H));
            TRY(alloc(m, &a.planes, static_cast<long long>((bytes + 3) / 4)));
        }
        if (c.attention_mode == GPT_ATTN_TILED_SPLIT ||
            c.attention_mode == GPT_ATTN_MATERIALIZED) {
            TRY(alloc(m, &a.q, BT * C));
            TRY(alloc(m, &a.k, BT * C));
            TRY(alloc(m, &a.v, BT * C));
            TRY(alloc(m, &a.attn_out, BT * C));
        }
        if (c.attention_mode == GPT_ATTN_MATERIALIZED) TRY(alloc(m, &a.probs, B * H * T * T));
    }
    TRY(alloc(m, &m->emb, BT * C));
    TRY(alloc(m, &m->lnf, BT * C));
    TRY(alloc(m, &m->lnf_mean, BT));
    TRY(alloc(m, &m->lnf_rstd, BT));
    TRY(alloc(m, &m->logits, BT * V));
    TRY(alloc(m, &m->dlogits, BT * V));
    TRY(alloc(m, &m->row_loss, BT));
    TRY(alloc(m, &m->d_x, BT * C));
    TRY(alloc(m, &m->d_ln, BT * C));
    TRY(alloc(m, &m->d_qkv, BT * 3 * C));
    TRY(alloc(m, &m->d_merged, BT * C));
    TRY(alloc(m, &m->d_ffn_a, BT * F));
    TRY(alloc(m, &m->d_ffn_b, BT * F));
    TRY(alloc(m, &m->proj, BT * C));
    TRY(alloc(m, &m->ws, B * H * T));
    {
        // One dS area for all layers (dS lives within one layer's backward call), where the
        // shape takes the dS-first order: the fp32 MFMA backward up to its 16 GiB limit, the
        // three-plane backward where attn_f32x3_ds_workspace_bytes is not 0.
        const int iB = static_cast<int>(B), iH = static_cast<int>(H), iT = static_cast<int>(T),
                  id = static_cast<int>(C / H);
        size_t bytes = 0;
        if (c.attention_mode == GPT_ATTN_FUSED && attn_f32_backward_uses_ds(iB, iH, iT, id))
            bytes = attn_f32_ds_workspace_bytes(iB, iH, iT, id);
        if (c.attention_mode == GPT_ATTN_FUSED_X3)
            bytes = attn_f32x3_ds_workspace_bytes(iB, iH, iT, id);
        if (bytes > 0) TRY(alloc(m, &m->attn_ds, static_cast<long long>((bytes + 3) / 4)));
    }
    long long sk = head_splitk(c) ? static_cast<long long>(kHeadSplitK) * BT * C : 0;
    if (weight_splitk(c)) sk = std::max(sk, weight_splitk_floats(c));
    if (sk > 0) TRY(alloc(m, &m->splitk, sk));
    long long cs = 0;
    for (long long n : {3 * C, F, C}) cs = std::max<long long>(cs, column_sum_scratch(BT, n));
    cs = std::max<long long>(cs, column_sum_scratch(B, T * C));
    TRY(alloc(m, &m->colsum, cs));
    TRY(alloc(m, &m->norm, 1 + adamw_norm_blocks()));
    if (c.attention_mode == GPT_ATTN_TILED_SPLIT || c.attention_mode == GPT_ATTN_MATERIALIZED) {
        TRY(alloc(m, &m->dq, BT * C));
        TRY(alloc(m, &m->dk, BT * C));
        TRY(alloc(m, &m->dv, BT * C));
        TRY(alloc(m, &m->d_attn_out, BT * C));
    }
    if (c.attention_mode == GPT_ATTN_MATERIALIZED) {
        TRY(alloc(m, &m->scores, B * H * T * T));
        TRY(alloc(m, &m->dprobs, B * H * T * T));
        TRY(alloc(m, &m->dscores, B * H * T * T));
    }
    if (rocblas_create_handle(&m->blas) != rocblas_status_success) return ATTN_ERROR_LAUNCH;
    return ATTN_SUCCESS;
}

int forward(gpt_model* m, const int* tokens, hipStream_t s) {
    const gpt_config& c = m->cfg;
    const int B = c.batch_size, T = c.max_seq_len, C = c.d_model, F = c.d_ff, V = c.vocab_size;
    const int BT = B * T;
    embedding_forward(tokens, m->P.tok_emb, m->P.pos_emb, m->emb, B, T, C, s);
    const float* x = m->emb;
    for (int li = 0; li < c.num_layers; ++li) {
        const Layer& p = m->P.layers[li];
        LayerActs& a = m->acts[li];
        layernorm_forward(x, p.ln1_g, p.ln1_b, a.ln1, a.ln1_mean, a.ln1_rstd, BT, C,
                          c.layernorm_eps, s);
        TRY(gemm(m->blas, false, false, BT, 3 * C, C, a.ln1, p.qkv_w, a.qkv));
        add_bias(a.qkv, p.qkv_b, BT, 3 * C, s);
        TRY(attention_forward(m, a, s));
        TRY(gemm(m->blas, false, false, BT, C, C, a.merged, p.proj_w, m->proj));
        bias_residual(x, m->proj, p.proj_b, a.res1, BT, C, s);
        layernorm_forward(a.res1, p.ln2_g, p.ln2_b, a.ln2, a.ln2_mean, a.ln2_rstd, BT, C,
                          c.layernorm_eps, s);
        TRY(gemm(m->blas, false, false, BT, F, C, a.ln2, p.ffn1_w, a.ffn1));
        bias_gelu_forward(a.ffn1, p.ffn1_b, a.gelu, BT, F, s);
        TRY(gemm(m->blas, false, false, BT, C, F, a.gelu, p.ffn2_w, m->proj));
        bias_residual(a.res1, m->proj, p.ffn2_b, a.out, BT, C, s);
        x = a.out;
    }
    layernorm_forward(x, m->P.lnf_g, m->P.lnf_b, m->lnf, m->lnf_mean, m->lnf_rstd, BT, C,
                      c.layernorm_eps, s);
    return gemm(m->blas, false, false, BT, V, C, m->lnf, m->P.head_w, m->logits);
}

int backward(gpt_model* m, const int* tokens, const int* targets, float* loss, hipStream_t s) {
    const gpt_config& c = m->cfg;
    const int B = c.batch_size, T = c.max_seq_len, C = c.d_model, F = c.d_ff, V = c.vocab_size;
    const int BT = B * T;
    cross_entropy(m->logits, targets, m->dlogits, m->row_loss, loss, BT, V, s);
    TRY(gemm(m->blas, true, false, C, V, BT, m->lnf, m->dlogits, m->G.head_w));
    if (head_splitk(c))
        TRY(gemm_nt_splitk(m->blas, BT, C, V, m->dlogits, m->P.head_w, m->d_ln, m->splitk,
                           kHeadSplitK, s));
    else
        TRY(gemm(m->blas, false, true, BT, C, V, m->dlogits, m->P.head_w, m->d_ln));
    const float* x_top = c.num_layers > 0 ? m->acts.back().out : m->emb;
    layernorm_backward(m->d_ln, x_top, m->P.lnf_g, m->lnf_mean, m->lnf_rstd, m->d_x, m->G.lnf_g,
                       m->G.lnf_b, m->colsum, BT, C, false, s);
    for (int li = c.num_layers - 1; li >= 0; --li) {
        const Layer& p = m->P.layers[li];
        const Layer& g = m->G.layers[li];
        LayerActs& a = m->acts[li];
        const float* x_in = li > 0 ? m->acts[li - 1].out : m->emb;
        // out = res1 + gelu(ln2 W1 + b1) W2 + b2; d_x holds d(out)
        column_sum(m->d_x, BT, C, g.ffn2_b, m->colsum, s);
        TRY(gemm_dw(m, F, C, BT, a.gelu, m->d_x, g.ffn2_w, s));
        TRY(gemm(m->blas, false, true, BT, F, C, m->d_x, p.ffn2_w, m->d_ffn_a));
        bias_gelu_backward(m->d_ffn_a, a.ffn1, p.ffn1_b, m->d_ffn_b, BT, F, s);
        column_sum(m->d_ffn_b, BT, F, g.ffn1_b, m->colsum, s);
        TRY(gemm_dw(m, C, F, BT, a.ln2, m->d_ffn_b, g.ffn1_w, s));
        TRY(gemm(m->blas, false, true, BT, C, F, m->d_ffn_b, p.ffn1_w, m->d_ln));
        layernorm_backward(m->d_ln, a.res1, p.ln2_g, a.ln2_mean, a.ln2_rstd, m->d_x, g.ln2_g,
                           g.ln2_b, m->colsum, BT, C, true, s);
        // res1 = x_in + merged Wproj + bproj; d_x holds d(res1)
        column_sum(m->d_x, BT, C, g.proj_b, m->colsum, s);
        TRY(gemm_dw(m, C, C, BT, a.merged, m->d_x, g.proj_w, s));
        TRY(gemm(m->blas, false, true, BT, C, C, m->d_x, p.proj_w, m->d_merged));
        TRY(attention_backward(m, a, s));
        column_sum(m->d_qkv, BT, 3 * C, g.qkv_b, m->colsum, s);
        TRY(gemm_dw(m, C, 3 * C, BT, a.ln1, m->d_qkv, g.qkv_w, s));
        TRY(gemm(m->blas, false, true, BT, C, 3 * C, m->d_qkv, p.qkv_w, m->d_ln));
        layernorm_backward(m->d_ln, x_in, p.ln1_g, a.ln1_mean, a.ln1_rstd, m->d_x, g.ln1_g,
                           g.ln1_b, m->colsum, BT, C, true, s);
    }
    if (hipMemsetAsync(m->G.tok_emb, 0, static_cast<size_t>(V) * C * sizeof(float), s) !=
        hipSuccess)
        return ATTN_ERROR_LAUNCH;
    embedding_backward(tokens, m->d_x, m->G.tok_emb, m->G.pos_emb, m->colsum, B, T, C, s);
    return hipGetLastError() == hipSuccess ? ATTN_SUCCESS : ATTN_ERROR_LAUNCH;
}

}  // namespace

extern "C" {

void gpt_default_config(gpt_config* cfg, int vocab_size, int max_seq_len, int d_model,
                        int num_layers, int num_heads, int d_ff, int batch_size) {
    if (cfg == nullptr) return;
    *cfg = gpt_config{};
    cfg->vocab_size = vocab_size;
    cfg->max_seq_len = max_seq_len;
    cfg->d_model = d_model;
    cfg->num_layers = num_layers;
    cfg->num_heads = num_heads;
    cfg->d_ff = d_ff;
    cfg->batch_size = batch_size;
    cfg->layernorm_eps = 1e-5f;   // include/config.h:16-22
    cfg->learning_rate = 3e-4f;
    cfg->weight_decay = 0.01f;
    cfg->beta1 = 0.9f;
    cfg->beta2 = 0.999f;
    cfg->adam_eps = 1e-8f;
    cfg->grad_clip = 1.0f;
    cfg->attention_mode = GPT_ATTN_FUSED;
}

int gpt_create(const gpt_config* cfg, gpt_model** out) {
    if (cfg == nullptr || out == nullptr) return ATTN_ERROR_NULL_POINTER;
    *out = nullptr;
    const int st = check_config(*cfg);
    if (st != ATTN_SUCCESS) return st;
    gpt_model* m = new (std::nothrow) gpt_model;
    if (m == nullptr) return ATTN_ERROR_LAUNCH;
    const int cs = create(*cfg, m);
    if (cs != ATTN_SUCCESS) {
        gpt_destroy(m);
        return cs;
    }
    *out = m;
    return ATTN_SUCCESS;
}

void gpt_destroy(gpt_model* m) {
    if (m == nullptr) return;
    if (m->blas != nullptr) rocblas_destroy_handle(m->blas);
    for (hipEvent_t e : m->ev) (void)hipEventDestroy(e);
    for (void* p : m->allocations) (void)hipFree(p);
    delete m;
}

long long gpt_num_parameters(const gpt_model* m) { return m == nullptr ? 0 : m->n_params; }

int gpt_set_parameters(gpt_model* m, const float* host, long long n) {
    if (m == nullptr || host == nullptr) return ATTN_ERROR_NULL_POINTER;
    if (n != m->n_params) return ATTN_ERROR_INVALID_DIM;
    return hipMemcpy(m->params, host, n * sizeof(float), hipMemcpyHostToDevice) == hipSuccess
               ? ATTN_SUCCESS
               : ATTN_ERROR_LAUNCH;
}

int gpt_get_parameters(const gpt_model* m, float* host, long long n) {
    if (m == nullptr || host == nullptr) return ATTN_ERROR_NULL_POINTER;
    if (n != m->n_params) return ATTN_ERROR_INVALID_DIM;
    return hipMemcpy(host, m->params, n * sizeof(float), hipMemcpyDeviceToHost) == hipSuccess
               ? ATTN_SUCCESS
               : ATTN_ERROR_LAUNCH;
}

int gpt_get_gradients(const gpt_model* m, float* host, long long n) {
    if (m == nullptr || host == nullptr) return ATTN_ERROR_NULL_POINTER;
    if (n != m->n_params) return ATTN_ERROR_INVALID_DIM;
    return hipMemcpy(host, m->grads, n * sizeof(float), hipMemcpyDeviceToHost) == hipSuccess
               ? ATTN_SUCCESS
               : ATTN_ERROR_LAUNCH;
}

int gpt_get_logits(const gpt_model* m, float* host, long long n) {
    if (m == nullptr || host == nullptr) return ATTN_ERROR_NULL_POINTER;
    const long long want =
        static_cast<long long>(m->cfg.batch_size) * m->cfg.max_seq_len * m->cfg.vocab_size;
    if (n != want) return ATTN_ERROR_INVALID_DIM;
    return hipMemcpy(host, m->logits, n * sizeof(float), hipMemcpyDeviceToHost) == hipSuccess
               ? ATTN_SUCCESS
               : ATTN_ERROR_LAUNCH;
}

int gpt_forward_backward(gpt_model* m, const int* tokens, const int* targets, float* loss,
                         hipStream_t stream) {
    if (m == nullptr || tokens == nullptr || targets == nullptr || loss == nullptr)
        return ATTN_ERROR_NULL_POINTER;
    if (rocblas_set_stream(m->blas, stream) != rocblas_status_success) return ATTN_ERROR_LAUNCH;
    m->ev_used = 0;
    (void)hipGetLastError();
    TRY(forward(m, tokens, stream));
    return backward(m, tokens, targets, loss, stream);
}

int gpt_optimizer_step(gpt_model* m, hipStream_t stream) {
    if (m == nullptr) return ATTN_ERROR_NULL_POINTER;
    const gpt_config& c = m->cfg;
    m->step += 1;
    AdamWParams a;
    a.lr = c.learning_rate;
    a.beta1 = c.beta1;
    a.beta2 = c.beta2;
    a.eps = c.adam_eps;
    a.weight_decay = c.weight_decay;
    a.max_norm = c.grad_clip;
    a.bc1 = 1.0f - powf(c.beta1, static_cast<float>(m->step));
    a.bc2 = 1.0f - powf(c.beta2, static_cast<float>(m->step));
    (void)hipGetLastError();
    clip_adamw_zero(m->params, m->grads, m->adam_m, m->adam_v, m->norm, m->n_params, a, stream);
    return hipGetLastError() == hipSuccess ? ATTN_SUCCESS : ATTN_ERROR_LAUNCH;
}

int gpt_set_attention_timing(gpt_model* m, int on) {
    if (m == nullptr) return ATTN_ERROR_NULL_POINTER;
    m->timing = on != 0;
    return ATTN_SUCCESS;
}

int gpt_last_attention_ms(gpt_model* m, float* ms) {
    if (m == nullptr || ms == nullptr) return ATTN_ERROR_NULL_POINTER;
    float total = 0.0f;
    for (int i = 0; i + 1 < m->ev_used; i += 2) {
        if (hipEventSynchronize(m->ev[i + 1]) != hipSuccess) return ATTN_ERROR_LAUNCH;
        float t = 0.0f;
        if (hipEventElapsedTime(&t, m->ev[i], m->ev[i + 1]) != hipSuccess)
            return ATTN_ERROR_LAUNCH;
        total += t;
    }
    *ms = total;
    return ATTN_SUCCESS;
}

}  // extern "C"
