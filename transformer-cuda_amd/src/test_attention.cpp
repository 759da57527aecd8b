// test_attention.cpp - C++ host tests of the attention launchers (include/kernels/attention.h),
// the counterpart of the reference's tests/test_kernels.cu.  Each test uses inputs with an
// exact closed-form answer:
//   * causal softmax on all-equal scores (reference KAT, tests/test_kernels.cu:91-120):
//     row i is 1/(i+1) on j <= i, 0 above;
//   * the reference's tiled KAT (tests/test_kernels.cu:210-284: T=8, d=32, q=k=0.1, v=1,
//     dO=0.5), strengthened from "finite" to the exact values: O = 1, dQ = dK = 0 and
//     dV_j = 0.5 * sum_{i=j}^{T-1} 1/(i+1);
//   * Q = 0 at T not a multiple of the tile: P_ij = 1/(i+1), O_i = mean(v_0..v_i),
//     m_i = 0, l_i = i+1;
//   * QKV split followed by its backward is the identity (bitwise), head merge likewise;
//   * the packed launchers (attention straight from qkv, gradient straight into dqkv) equal
//     split + tiled + split-back bitwise, and the fused launchers (output and its gradient in
//     the merged-heads layout) equal them with the head merge applied;
//   * the materialised mode driven with the reference's own call text (src/model.cu:314-332,
//     618-650: a GEMM handle first, then the matmul.cuh:44-58 parameter list) equals the
//     library's materialised sequences bitwise, and the defaults of matmul_batched_strided
//     (no transposes, alpha 1, beta 0) equal the explicit arguments;
//   * the no-alloc backward (no caller workspace) equals the workspace backward bitwise;
//   * an unsupported head dimension throws instead of silently doing nothing.
// Exit status 0 iff every test passes.
#include <cmath>
#include <cstdio>
#include <stdexcept>
#include <utility>
#include <vector>

#include "common.h"
#include "kernels/attention.h"
#include "kernels/matmul.h"

namespace {

int g_failures = 0;

#define EXPECT(cond, ...)                                   \
    do {                                                    \
        if (!(cond)) {                                      \
            std::printf("    FAILED %s:%d: ", __FILE__, __LINE__); \
            std::printf(__VA_ARGS__);                       \
            std::printf("\n");                              \
            ++g_failures;                                   \
            return false;                                   \
        }                                                   \
    } while (0)

struct DevBuf {
    float* p = nullptr;
    size_t n = 0;
    explicit DevBuf(size_t count) : n(count) { HIP_CHECK(hipMalloc(&p, n * sizeof(float))); }
    ~DevBuf() { (void)hipFree(p); }
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    void upload(const std::vector<float>& h) {
        HIP_CHECK(hipMemcpy(p, h.data(), n * sizeof(float), hipMemcpyHostToDevice));
    }
    std::vector<float> download() const {
        std::vector<float> h(n);
        HIP_CHECK(hipMemcpy(h.data(), p, n * sizeof(float), hipMemcpyDeviceToHost));
        return h;
    }
};

bool test_causal_softmax() {
    std::printf("[Test] causal softmax, all-equal scores (reference KAT)...\n");
    const int B = 1, H = 1, T = 4;
    DevBuf scores(T * T), probs(T * T);
    scores.upload(std::vector<float>(T * T, 1.0f));
    causal_softmax_forward(scores.p, probs.p, B, H, T, 1.0f);
    HIP_CHECK(hipDeviceSynchronize());
    const std::vector<float> p = probs.download();
    for (int i = 0; i < T; ++i)
        for (int j = 0; j < T; ++j) {
            const float want = (j <= i) ? 1.0f / (i + 1) : 0.0f;
            EXPECT(std::fabs(p[i * T + j] - want) <= 1e-6f, "p[%d][%d] = %g, want %g", i, j,
                   p[i * T + j], want);
        }
    return true;
}

bool test_tiled_kat(int d_head) {
    std::printf("[Test] tiled causal attention KAT (T=8, d=%d, q=k=0.1, v=1, dO=0.5)...\n",
                d_head);
    const int B = 1, H = 1, T = 8;
    const size_t n = static_cast<size_t>(B) * H * T * d_head;
    const size_t r = static_cast<size_t>(B) * H * T;
    DevBuf q(n), k(n), v(n), o(n), dO(n), dq(n), dk(n), dv(n), m(r), l(r), ws(r);
    q.upload(std::vector<float>(n, 0.1f));
    k.upload(std::vector<float>(n, 0.1f));
    v.upload(std::vector<float>(n, 1.0f));
    dO.upload(std::vector<float>(n, 0.5f));
    const float scale = 1.0f / std::sqrt(static_cast<float>(d_head));
    tiled_causal_attention_forward(q.p, k.p, v.p, o.p, B, H, T, d_head, scale, m.p, l.p);
    tiled_causal_attention_backward(q.p, k.p, v.p, o.p, dO.p, m.p, l.p, dq.p, dk.p, dv.p, ws.p,
                                    B, H, T, d_head, scale);
    HIP_CHECK(hipDeviceSynchronize());
    const auto ho = o.download(), hdq = dq.download(), hdk = dk.download(), hdv = dv.download();
    const auto hl = l.download();
    for (size_t i = 0; i < n; ++i) {
        EXPECT(std::fabs(ho[i] - 1.0f) <= 1e-6f, "O[%zu] = %.9g, want 1", i, ho[i]);
        EXPECT(std::fabs(hdq[i]) <= 1e-6f, "dQ[%zu] = %g, want 0", i, hdq[i]);
        EXPECT(std::fabs(hdk[i]) <= 1e-6f, "dK[%zu] = %g, want 0", i, hdk[i]);
    }
    for (int t = 0; t < T; ++t) {
        EXPECT(std::fabs(hl[t] - (t + 1)) <= 1e-5f, "l[%d] = %g, want %d", t, hl[t], t + 1);
        double want = 0.0;
        for (int i = t; i < T; ++i) want += 0.5 / (i + 1);
        for (int e = 0; e < d_head; ++e) {
            const float got = hdv[t * d_head + e];
            EXPECT(std::fabs(got - want) <= 1e-6 * want + 1e-7, "dV[%d][%d] = %.9g, want %.9g", t,
                   e, got, want);
        }
    }
    return true;
}

bool test_zero_query(int d_head, int T) {
    std::printf("[Test] Q = 0 closed form (T=%d, d=%d): prefix means of V...\n", T, d_head);
    const int B = 2, H = 3;
    const size_t n = static_cast<size_t>(B) * H * T * d_head;
    const size_t r = static_cast<size_t>(B) * H * T;
    std::vector<float> hv(n), hk(n);
    uint32_t state = 12345u;
    for (size_t i = 0; i < n; ++i) {
        state = state * 1664525u + 1013904223u;
        hv[i] = static_cast<float>(static_cast<int>(state >> 9) % 2001 - 1000) / 1000.0f;
        state = state * 1664525u + 1013904223u;
        hk[i] = static_cast<float>(static_cast<int>(state >> 9) % 2001 - 1000) / 500.0f;
    }
    DevBuf q(n), k(n), v(n), o(n), m(r), l(r);
    q.upload(std::vector<float>(n, 0.0f));
    k.upload(hk);
    v.upload(hv);
    tiled_causal_attention_forward(q.p, k.p, v.p, o.p, B, H, T, d_head,
                                   1.0f / std::sqrt(static_cast<float>(d_head)), m.p, l.p);
    HIP_CHECK(hipDeviceSynchronize());
    const auto ho = o.download(), hm = m.download(), hl = l.download();
    for (int bh = 0; bh < B * H; ++bh) {
        std::vector<double> sum(d_head, 0.0);
        for (int t = 0; t < T; ++t) {
            const size_t row = static_cast<size_t>(bh) * T + t;
            EXPECT(hm[row] == 0.0f, "m[%zu] = %g, want 0", row, hm[row]);
            EXPECT(std::fabs(hl[row] - (t + 1)) <= 1e-6f * (t + 1), "l[%zu] = %g, want %d", row,
                   hl[row], t + 1);
            for (int e = 0; e < d_head; ++e) {
                sum[e] += hv[row * d_head + e];
                const double want = sum[e] / (t + 1);
                const float got = ho[row * d_head + e];
                EXPECT(std::fabs(got - want) <= 2e-6, "O[%zu][%d] = %.9g, want %.9g", row, e,
                       got, want);
            }
        }
    }
    return true;
}

bool test_split_roundtrip() {
    std::printf("[Test] QKV split-transpose fwd -> bwd is the identity; head merge too...\n");
    const int B = 2, T = 37, H = 3, d = 64;
    const size_t n = static_cast<size_t>(B) * T * H * d;
    std::vector<float> h(3 * n);
    for (size_t i = 0; i < h.size(); ++i) h[i] = static_cast<float>(i) * 0.25f - 7.0f;
    DevBuf qkv(3 * n), q(n), k(n), v(n), back(3 * n), merged(n), unmerged(n);
    qkv.upload(h);
    qkv_split_transpose_forward(qkv.p, q.p, k.p, v.p, B, T, H, d);
    qkv_split_transpose_backward(q.p, k.p, v.p, back.p, B, T, H, d);
    head_merge_transpose_forward(q.p, merged.p, B, H, T, d);
    head_merge_transpose_backward(merged.p, unmerged.p, B, H, T, d);
    HIP_CHECK(hipDeviceSynchronize());
    const auto hb = back.download();
    for (size_t i = 0; i < h.size(); ++i) EXPECT(hb[i] == h[i], "dqkv[%zu] = %g != %g", i, hb[i], h[i]);
    const auto hq = q.download();
    // q[b,h,t,e] = qkv[b,t,0*C + h*d + e]
    for (int b = 0; b < B; ++b)
        for (int hh = 0; hh < H; ++hh)
            for (int t = 0; t < T; ++t)
                for (int e = 0; e < d; ++e) {
                    const size_t hm_i = ((static_cast<size_t>(b) * H + hh) * T + t) * d + e;
                    const size_t rm_i = (static_cast<size_t>(b) * T + t) * 3 * H * d + hh * d + e;
                    EXPECT(hq[hm_i] == h[rm_i], "q mismatch at %zu", hm_i);
                }
    const auto hu = unmerged.download();
    for (size_t i = 0; i < n; ++i) EXPECT(hu[i] == hq[i], "head merge round trip at %zu", i);
    return true;
}

bool test_packed_matches_split(int d, int T) {
    std::printf("[Test] packed / fused launchers == split + tiled + split-back, bitwise (T=%d, d=%d)...\n",
                T, d);
    const int B = 2, H = 3;
    const size_t n = static_cast<size_t>(B) * H * T * d;
    const size_t r = static_cast<size_t>(B) * H * T;
    const float scale = 1.0f / std::sqrt(static_cast<float>(d));
    std::vector<float> hqkv(3 * n), hdo(n);
    uint32_t state = 777u + static_cast<uint32_t>(T);
    auto next = [&state]() {
        state = state * 1664525u + 1013904223u;
        return static_cast<float>(static_cast<int>(state >> 9) % 2001 - 1000) / 700.0f;
    };
    for (auto& x : hqkv) x = next();
    for (auto& x : hdo) x = next();
    DevBuf qkv(3 * n), dO(n), q(n), k(n), v(n), o1(n), m1(r), l1(r), dq(n), dk(n), dv(n),
        dqkv1(3 * n), ws1(r), o2(n), m2(r), l2(r), dqkv2(3 * n), ws2(r);
    qkv.upload(hqkv);
    dO.upload(hdo);
    qkv_split_transpose_forward(qkv.p, q.p, k.p, v.p, B, T, H, d);
    tiled_causal_attention_forward(q.p, k.p, v.p, o1.p, B, H, T, d, scale, m1.p, l1.p);
    tiled_causal_attention_backward(q.p, k.p, v.p, o1.p, dO.p, m1.p, l1.p, dq.p, dk.p, dv.p,
                                    ws1.p, B, H, T, d, scale);
    qkv_split_transpose_backward(dq.p, dk.p, dv.p, dqkv1.p, B, T, H, d);
    packed_causal_attention_forward(qkv.p, o2.p, B, H, T, d, scale, m2.p, l2.p);
    packed_causal_attention_backward(qkv.p, o2.p, dO.p, m2.p, l2.p, dqkv2.p, ws2.p, B, H, T, d,
                                     scale);
    HIP_CHECK(hipDeviceSynchronize());
    // Fused: O written in the merged-heads layout, dO read from it (the head merge is a
    // permutation, so the comparison is bitwise too).
    DevBuf om(n), dOm(n), m3(r), l3(r), dqkv3(3 * n), ws3(r), om_ref(n);
    head_merge_transpose_forward(dO.p, dOm.p, B, H, T, d);
    head_merge_transpose_forward(o1.p, om_ref.p, B, H, T, d);
    fused_causal_attention_forward(qkv.p, om.p, B, H, T, d, scale, m3.p, l3.p);
    fused_causal_attention_backward(qkv.p, om.p, dOm.p, m3.p, l3.p, dqkv3.p, ws3.p, B, H, T, d,
                                    scale);
    HIP_CHECK(hipDeviceSynchronize());
    const std::pair<const DevBuf*, const DevBuf*> pairs[] = {
        {&o1, &o2}, {&m1, &m2}, {&l1, &l2}, {&dqkv1, &dqkv2}, {&ws1, &ws2},
        {&om_ref, &om}, {&m1, &m3}, {&l1, &l3}, {&dqkv1, &dqkv3}, {&ws1, &ws3}};
    const char* names[] = {"O", "m", "l", "dqkv", "D",
                           "fused O", "fused m", "fused l", "fused dqkv", "fused D"};
    for (int t = 0; t < 10; ++t) {
        const auto a = pairs[t].first->download(), b = pairs[t].second->download();
        for (size_t i = 0; i < a.size(); ++i)
            EXPECT(std::isfinite(a[i]) && a[i] == b[i], "%s[%zu]: split %.9g, packed %.9g",
                   names[t], i, a[i], b[i]);
    }
    return true;
}

// The reference's layer buffers, by the member names src/model.cu uses (include/model.h:42-49,
// 84-93).
struct LayerActs {
    float *q, *k, *v, *attn_scores, *attn_probs, *attn_out;
};
struct LayerGrads {
    float *d_attn_out, *d_attn_probs, *d_attn_scores, *d_q, *d_k, *d_v;
};

bool test_materialized_reference_call_text() {
    std::printf("[Test] materialised mode through the reference's call text == library sequences...\n");
    const int B = 2, H = 3, T = 70, d_head = 64;
    const size_t n = static_cast<size_t>(B) * H * T * d_head;
    const size_t nn = static_cast<size_t>(B) * H * T * T;
    const float scale = 1.0f / std::sqrt(static_cast<float>(d_head));
    uint32_t state = 4242u;
    auto next = [&state]() {
        state = state * 1664525u + 1013904223u;
        return static_cast<float>(static_cast<int>(state >> 9) % 2001 - 1000) / 700.0f;
    };
    std::vector<float> hq(n), hk(n), hv(n), hdo(n);
    for (auto* h : {&hq, &hk, &hv, &hdo})
        for (auto& x : *h) x = next();
    DevBuf q(n), k(n), v(n), dO(n), s1(nn), p1(nn), o1(n), dp1(nn), ds1(nn), dq1(n), dk1(n),
        dv1(n), s2(nn), p2(nn), o2(n), dp2(nn), ds2(nn), dq2(n), dk2(n), dv2(n), dv3(n);
    q.upload(hq);
    k.upload(hk);
    v.upload(hv);
    dO.upload(hdo);
    gemm_handle_t cublas_handle = nullptr;
    gemm_create(&cublas_handle);
    hipStream_t stream = nullptr;
    LayerActs la{q.p, k.p, v.p, s1.p, p1.p, o1.p};
    LayerGrads grads{dO.p, dp1.p, ds1.p, dq1.p, dk1.p, dv1.p};
    // src/model.cu:314-332, verbatim apart from the buffers' owners
    matmul_batched_strided(
        cublas_handle,
        la.q, la.k, la.attn_scores,
        T, T, d_head,
        T * d_head, T * d_head, T * T,
        B * H, false, true, 1.0f, 0.0f, stream
    );
    causal_softmax_forward(la.attn_scores, la.attn_probs, B, H, T, scale, stream);
    matmul_batched_strided(
        cublas_handle,
        la.attn_probs, la.v, la.attn_out,
        T, d_head, T,
        T * T, T * d_head, T * d_head,
        B * H, false, false, 1.0f, 0.0f, stream
    );
    // src/model.cu:618-650
    matmul_batched_strided(
        cublas_handle,
        grads.d_attn_out, la.v, grads.d_attn_probs,
        T, T, d_head,
        T * d_head, T * d_head, T * T,
        B * H, false, true, 1.0f, 0.0f, stream
    );
    matmul_batched_strided(
        cublas_handle,
        la.attn_probs, grads.d_attn_out, grads.d_v,
        T, d_head, T,
        T * T, T * d_head, T * d_head,
        B * H, true, false, 1.0f, 0.0f, stream
    );
    causal_softmax_backward(grads.d_attn_probs, la.attn_probs, grads.d_attn_scores, B, H, T, scale, stream);
    matmul_batched_strided(
        cublas_handle,
        grads.d_attn_scores, la.k, grads.d_q,
        T, d_head, T,
        T * T, T * d_head, T * d_head,
        B * H, false, false, 1.0f, 0.0f, stream
    );
    matmul_batched_strided(
        cublas_handle,
        grads.d_attn_scores, la.q, grads.d_k,
        T, d_head, T,
        T * T, T * d_head, T * d_head,
        B * H, true, false, 1.0f, 0.0f, stream
    );
    // defaults: no transposes, alpha 1, beta 0, null stream
    matmul_batched_strided(cublas_handle, la.attn_probs, la.v, dv3.p, T, d_head, T, T * T,
                           T * d_head, T * d_head, B * H);
    materialized_causal_attention_forward(q.p, k.p, v.p, s2.p, p2.p, o2.p, B, H, T, d_head, scale);
    materialized_causal_attention_backward(q.p, k.p, v.p, p2.p, dO.p, dp2.p, ds2.p, dq2.p, dk2.p,
                                           dv2.p, B, H, T, d_head, scale);
    HIP_CHECK(hipDeviceSynchronize());
    EXPECT(attn_gemm_device(cublas_handle) >= 0, "handle not bound to a device");
    gemm_destroy(cublas_handle);
    const std::pair<const DevBuf*, const DevBuf*> pairs[] = {
        {&s1, &s2}, {&p1, &p2}, {&o1, &o2}, {&dp1, &dp2}, {&ds1, &ds2},
        {&dq1, &dq2}, {&dk1, &dk2}, {&dv1, &dv2}, {&o1, &dv3}};
    const char* names[] = {"scores", "probs", "out", "dprobs", "dscores", "dq", "dk", "dv",
                           "defaults (probs V)"};
    for (int t = 0; t < 9; ++t) {
        const auto a = pairs[t].first->download(), b = pairs[t].second->download();
        for (size_t i = 0; i < a.size(); ++i)
            EXPECT(std::isfinite(a[i]) && a[i] == b[i], "%s[%zu]: call text %.9g, library %.9g",
                   names[t], i, a[i], b[i]);
    }
    bool threw = false;
    try {
        matmul_batched_strided(static_cast<gemm_handle_t>(nullptr), la.q, la.k, la.attn_scores,
                               T, T, d_head, T * d_head, T * d_head, T * T, B * H, false, true);
    } catch (const std::runtime_error&) {
        threw = true;
    }
    EXPECT(threw, "a null GEMM handle did not throw");
    return true;
}

bool test_noalloc_backward() {
    std::printf("[Test] no-alloc backward == workspace backward, bitwise, two calls...\n");
    for (int pass = 0; pass < 2; ++pass) {
        const int B = pass == 0 ? 2 : 1, H = pass == 0 ? 4 : 3, T = pass == 0 ? 300 : 65;
        const int d = pass == 0 ? 64 : 128;
        const size_t n = static_cast<size_t>(B) * H * T * d, r = static_cast<size_t>(B) * H * T;
        const float scale = 1.0f / std::sqrt(static_cast<float>(d));
        uint32_t state = 99u + static_cast<uint32_t>(pass);
        auto next = [&state]() {
            state = state * 1664525u + 1013904223u;
            return static_cast<float>(static_cast<int>(state >> 9) % 2001 - 1000) / 700.0f;
        };
        std::vector<float> h(n);
        DevBuf q(n), k(n), v(n), dO(n), o(n), m(r), l(r), ws(r), dq1(n), dk1(n), dv1(n), dq2(n),
            dk2(n), dv2(n);
        for (DevBuf* b : {&q, &k, &v, &dO}) {
            for (auto& x : h) x = next();
            b->upload(h);
        }
        tiled_causal_attention_forward(q.p, k.p, v.p, o.p, B, H, T, d, scale, m.p, l.p);
        tiled_causal_attention_backward(q.p, k.p, v.p, o.p, dO.p, m.p, l.p, dq1.p, dk1.p, dv1.p,
                                        ws.p, B, H, T, d, scale);
        tiled_causal_attention_backward_noalloc(q.p, k.p, v.p, o.p, dO.p, m.p, l.p, dq2.p, dk2.p,
                                                dv2.p, B, H, T, d, scale);
        HIP_CHECK(hipDeviceSynchronize());
        const std::pair<const DevBuf*, const DevBuf*> pairs[] = {{&dq1, &dq2}, {&dk1, &dk2},
                                                                 {&dv1, &dv2}};
        const char* names[] = {"dq", "dk", "dv"};
        for (int t = 0; t < 3; ++t) {
            const auto a = pairs[t].first->download(), b = pairs[t].second->download();
            for (size_t i = 0; i < a.size(); ++i)
                EXPECT(std::isfinite(a[i]) && a[i] == b[i], "%s[%zu]: workspace %.9g, no-alloc %.9g",
                       names[t], i, a[i], b[i]);
        }
    }
    return true;
}

bool test_bad_head_dim() {
    std::printf("[Test] unsupported d_head is an error, not a silent no-op...\n");
    DevBuf buf(1024);
    bool threw = false;
    try {
        tiled_causal_attention_forward(buf.p, buf.p, buf.p, buf.p, 1, 1, 8, 48, 0.1f);
    } catch (const std::runtime_error&) {
        threw = true;
    }
    EXPECT(threw, "d_head = 48 did not throw");
    return true;
}

}  // namespace

int main() {
    std::printf("========================================\n");
    std::printf(" MI355X attention host test suite\n");
    std::printf("========================================\n");
    std::fflush(stdout);
    test_causal_softmax();
    for (int d : {32, 64, 128}) test_tiled_kat(d);
    test_zero_query(64, 100);
    test_zero_query(128, 33);
    test_zero_query(32, 257);
    test_split_roundtrip();
    test_packed_matches_split(64, 77);
    test_packed_matches_split(128, 130);
    test_materialized_reference_call_text();
    test_noalloc_backward();
    test_bad_head_dim();
    if (g_failures == 0) {
        std::printf("All host tests passed.\n");
        return 0;
    }
    std::printf("%d host test(s) failed.\n", g_failures);
    return 1;
}
