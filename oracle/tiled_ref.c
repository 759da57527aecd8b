/*
 * tiled_ref.c - plain-C restatement of the reference's attention kernels
 * (src/kernels/attention.cu), executed sequentially on the CPU.  TEST INFRASTRUCTURE ONLY:
 * nothing in the product links this file.
 *
 * Each function evaluates, per output element, the arithmetic the reference's kernel
 * thread performs (same fp32 operations in the same order per row), so its results are
 * what the reference CUDA path computes up to fp32 contraction choices of nvcc.
 * Built with -ffp-contract=off so every multiply and add rounds separately.
 */
#include <float.h>
#include <math.h>
#include <stddef.h>
#include <stdint.h>

/* Row (b, t, s, h) of the (B, T, S, H, d) tensor <-> row (b, h, t) of tensor s of the
 * S head-major (B, H, T, d) tensors.  attention.cu:36-49 (S = 3), :320-327 (S = 1). */
static size_t rm_offset(int b, int t, int s, int h, int T, int S, int H, int d) {
    return ((((size_t)b * T + t) * S + s) * H + h) * (size_t)d;
}
static size_t hm_offset(int b, int h, int t, int H, int T, int d) {
    return (((size_t)b * H + h) * T + t) * (size_t)d;
}

/* attention.cu:54-82 */
void oracle_qkv_split_fwd(const float* qkv, float* q, float* k, float* v, int B, int T, int H,
                          int d) {
    float* outs[3] = {q, k, v};
    for (int b = 0; b < B; ++b)
        for (int t = 0; t < T; ++t)
            for (int s = 0; s < 3; ++s)
                for (int h = 0; h < H; ++h) {
                    const float* src = qkv + rm_offset(b, t, s, h, T, 3, H, d);
                    float* dst = outs[s] + hm_offset(b, h, t, H, T, d);
                    for (int e = 0; e < d; ++e) dst[e] = src[e];
                }
}

/* attention.cu:115-143 */
void oracle_qkv_split_bwd(const float* dq, const float* dk, const float* dv, float* dqkv,
                          int B, int T, int H, int d) {
    const float* ins[3] = {dq, dk, dv};
    for (int b = 0; b < B; ++b)
        for (int t = 0; t < T; ++t)
            for (int s = 0; s < 3; ++s)
                for (int h = 0; h < H; ++h) {
                    const float* src = ins[s] + hm_offset(b, h, t, H, T, d);
                    float* dst = dqkv + rm_offset(b, t, s, h, T, 3, H, d);
                    for (int e = 0; e < d; ++e) dst[e] = src[e];
                }
}

/* attention.cu:325-340: (B, H, T, d) -> (B, T, H*d) */
void oracle_head_merge_fwd(const float* in, float* out, int B, int H, int T, int d) {
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h)
            for (int t = 0; t < T; ++t) {
                const float* src = in + hm_offset(b, h, t, H, T, d);
                float* dst = out + rm_offset(b, t, 0, h, T, 1, H, d);
                for (int e = 0; e < d; ++e) dst[e] = src[e];
            }
}

/* attention.cu:362-379: (B, T, H*d) -> (B, H, T, d) */
void oracle_head_merge_bwd(const float* dout, float* din, int B, int H, int T, int d) {
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h)
            for (int t = 0; t < T; ++t) {
                const float* src = dout + rm_offset(b, t, 0, h, T, 1, H, d);
                float* dst = din + hm_offset(b, h, t, H, T, d);
                for (int e = 0; e < d; ++e) dst[e] = src[e];
            }
}

/* attention.cu:147-238: max over j <= i of s*scale (masked = -FLT_MAX), e = expf(s*scale -
 * max), p = e * (1 / (sum + 1e-12)), zeros above the diagonal. */
void oracle_causal_softmax_fwd(const float* scores, float* probs, int B, int H, int T,
                               float scale) {
    const size_t rows = (size_t)B * H * T;
    for (size_t r = 0; r < rows; ++r) {
        const int i = (int)(r % (size_t)T);
        const float* s = scores + r * (size_t)T;
        float* p = probs + r * (size_t)T;
        float mx = -FLT_MAX;
        for (int j = 0; j <= i; ++j) {
            const float x = s[j] * scale;
            if (x > mx) mx = x;
        }
        float sum = 0.0f;
        for (int j = 0; j < T; ++j) {
            if (j <= i) {
                const float e = expf(s[j] * scale - mx);
                p[j] = e;
                sum += e;
            } else {
                p[j] = 0.0f;
            }
        }
        const float inv = 1.0f / (sum + 1e-12f);
        for (int j = 0; j <= i; ++j) p[j] *= inv;
    }
}

/* attention.cu:242-305: ds = scale * p * (dp - sum_{j<=i} dp*p) for j <= i, else 0. */
void oracle_causal_softmax_bwd(const float* dprobs, const float* probs, float* dscores, int B,
                               int H, int T, float scale) {
    const size_t rows = (size_t)B * H * T;
    for (size_t r = 0; r < rows; ++r) {
        const int i = (int)(r % (size_t)T);
        const float* dp = dprobs + r * (size_t)T;
        const float* p = probs + r * (size_t)T;
        float* ds = dscores + r * (size_t)T;
        float dot = 0.0f;
        for (int j = 0; j <= i; ++j) dot += dp[j] * p[j];
        for (int j = 0; j < T; ++j) ds[j] = (j <= i) ? scale * p[j] * (dp[j] - dot) : 0.0f;
    }
}

/* attention.cu:518-624: per query, keys in order, online softmax with two expf per key;
 * O = o * (1 / (l + 1e-12)); stats m, l. */
void oracle_tiled_fwd(const float* q, const float* k, const float* v, float* out, int B, int H,
                      int T, int d, float scale, float* m_out, float* l_out) {
    float o[512];
    for (int bh = 0; bh < B * H; ++bh) {
        const size_t base = (size_t)bh * T * d;
        for (int i = 0; i < T; ++i) {
            const float* qi = q + base + (size_t)i * d;
            float m = -FLT_MAX, l = 0.0f;
            for (int e = 0; e < d; ++e) o[e] = 0.0f;
            for (int j = 0; j <= i; ++j) {
                const float* kj = k + base + (size_t)j * d;
                const float* vj = v + base + (size_t)j * d;
                float score = 0.0f;
                for (int e = 0; e < d; ++e) score += qi[e] * kj[e];
                score *= scale;
                const float m_new = score > m ? score : m;
                const float alpha = expf(m - m_new);
                const float beta = expf(score - m_new);
                l = l * alpha + beta;
                for (int e = 0; e < d; ++e) o[e] = o[e] * alpha + beta * vj[e];
                m = m_new;
            }
            const float inv_l = (l > 0.0f) ? 1.0f / (l + 1e-12f) : 0.0f;
            for (int e = 0; e < d; ++e) out[base + (size_t)i * d + e] = o[e] * inv_l;
            if (m_out) m_out[(size_t)bh * T + i] = m;
            if (l_out) l_out[(size_t)bh * T + i] = l;
        }
    }
}

/* attention.cu:659-677 */
void oracle_dot_do_o(const float* dO, const float* O, float* D, int64_t rows, int d) {
    for (int64_t r = 0; r < rows; ++r) {
        float sum = 0.0f;
        for (int e = 0; e < d; ++e) sum += dO[r * d + e] * O[r * d + e];
        D[r] = sum;
    }
}

/* attention.cu:696-812: p = expf(s - m) * inv_l, dp = dO.v, ds = scale * p * (dp - D),
 * dq += ds * k, keys in order. */
void oracle_tiled_bwd_dq(const float* q, const float* k, const float* v, const float* dO,
                         const float* m, const float* l, const float* D, float* dq, int B,
                         int H, int T, int d, float scale) {
    float acc[512];
    for (int bh = 0; bh < B * H; ++bh) {
        const size_t base = (size_t)bh * T * d;
        for (int i = 0; i < T; ++i) {
            const float* qi = q + base + (size_t)i * d;
            const float* doi = dO + base + (size_t)i * d;
            const float mi = m[(size_t)bh * T + i];
            const float li = l[(size_t)bh * T + i];
            const float di = D[(size_t)bh * T + i];
            const float inv_l = (li > 0.0f) ? 1.0f / (li + 1e-12f) : 0.0f;
            for (int e = 0; e < d; ++e) acc[e] = 0.0f;
            for (int j = 0; j <= i; ++j) {
                const float* kj = k + base + (size_t)j * d;
                const float* vj = v + base + (size_t)j * d;
                float s = 0.0f;
                for (int e = 0; e < d; ++e) s += qi[e] * kj[e];
                s *= scale;
                const float p = expf(s - mi) * inv_l;
                float dp = 0.0f;
                for (int e = 0; e < d; ++e) dp += doi[e] * vj[e];
                const float ds = scale * p * (dp - di);
                for (int e = 0; e < d; ++e) acc[e] += ds * kj[e];
            }
            for (int e = 0; e < d; ++e) dq[base + (size_t)i * d + e] = acc[e];
        }
    }
}

/* attention.cu:816-955: per key j, queries i >= j in order: dv += p * dO_i,
 * dk += ds * q_i. */
void oracle_tiled_bwd_dkdv(const float* q, const float* k, const float* v, const float* dO,
                           const float* m, const float* l, const float* D, float* dk,
                           float* dv, int B, int H, int T, int d, float scale) {
    float dka[512], dva[512];
    for (int bh = 0; bh < B * H; ++bh) {
        const size_t base = (size_t)bh * T * d;
        for (int j = 0; j < T; ++j) {
            const float* kj = k + base + (size_t)j * d;
            const float* vj = v + base + (size_t)j * d;
            for (int e = 0; e < d; ++e) {
                dka[e] = 0.0f;
                dva[e] = 0.0f;
            }
            for (int i = j; i < T; ++i) {
                const float* qi = q + base + (size_t)i * d;
                const float* doi = dO + base + (size_t)i * d;
                const float mi = m[(size_t)bh * T + i];
                const float li = l[(size_t)bh * T + i];
                const float di = D[(size_t)bh * T + i];
                const float inv_l = (li > 0.0f) ? 1.0f / (li + 1e-12f) : 0.0f;
                float s = 0.0f;
                for (int e = 0; e < d; ++e) s += qi[e] * kj[e];
                s *= scale;
                const float p = expf(s - mi) * inv_l;
                for (int e = 0; e < d; ++e) dva[e] += p * doi[e];
                float dp = 0.0f;
                for (int e = 0; e < d; ++e) dp += doi[e] * vj[e];
                const float ds = scale * p * (dp - di);
                for (int e = 0; e < d; ++e) dka[e] += ds * qi[e];
            }
            for (int e = 0; e < d; ++e) {
                dk[base + (size_t)j * d + e] = dka[e];
                dv[base + (size_t)j * d + e] = dva[e];
            }
        }
    }
}
