// causal_softmax.hip - fused scaled causal softmax over materialised (B*H*T, T) rows.
//
// Forward (reference semantics, src/kernels/attention.cu:147-238):
//     M = max_{j<=i} scale*s_j,  e_j = exp(scale*s_j - M),  p_j = e_j / (sum_j e_j + 1e-12)
//     for j <= i and p_j = 0 for j > i, where i = row mod T.
// Backward (src/kernels/attention.cu:242-305):
//     ds_j = scale * p_j * (dp_j - sum_{j'<=i} dp_j' p_j')  for j <= i, else 0.
//
// One wavefront per row.  Only the causal prefix j <= i is read; the masked suffix is
// written as zeros without reading it, which halves the read traffic of a full-row pass.
// With zero_block = Z > 0 the zeros stop at the end of the Z-column block that holds the
// diagonal, (i / Z + 1) * Z: the materialised attention's products read a probability row
// only up to there, so the rest of the suffix is neither read nor written.
// Rows up to kCacheCols columns stay in registers (one read per element); longer rows
// take a streaming two-pass path (online max/sum, then normalise).
#include <float.h>

#include "device_common.hpp"
#include "launch.hpp"

namespace tcamd {
namespace {

constexpr int kWavesPerBlock = 4;
constexpr int kChunks = 8;  // float4 chunks per lane kept in registers: 64*4*8 = 2048 cols

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
    return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
    return x;
}

template <int VEC>
struct Vec;
template <>
struct Vec<4> {
    using T = f32x4;
    __device__ static T load(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
    __device__ static void store(float* p, T x) { *reinterpret_cast<f32x4*>(p) = x; }
    __device__ static float get(const T& x, int e) { return x[e]; }
    __device__ static void set(T& x, int e, float v) { x[e] = v; }
};
template <>
struct Vec<1> {
    using T = float;
    __device__ static T load(const float* p) { return *p; }
    __device__ static void store(float* p, T x) { *p = x; }
    __device__ static float get(const T& x, int) { return x; }
    __device__ static void set(T& x, int, float v) { x = v; }
};

// Zero columns [from, T) of a row; `from` need not be VEC-aligned.  Columns past the last
// multiple of VEC below T are written one by one, so T need not be VEC-aligned.
template <int VEC>
__device__ __forceinline__ void zero_suffix(float* row, int from, int T, int lane) {
    using V = Vec<VEC>;
    const int first_chunk = from / VEC;
    const int nchunks = (T + VEC - 1) / VEC;
    for (int c = first_chunk + lane; c < nchunks; c += kWave) {
        const int j0 = c * VEC;
        if (j0 >= from && j0 + VEC <= T) {
            typename V::T z;
#pragma unroll
            for (int e = 0; e < VEC; ++e) V::set(z, e, 0.0f);
            V::store(row + j0, z);
        } else {
            for (int e = 0; e < VEC; ++e) {
                const int j = j0 + e;
                if (j >= from && j < T) row[j] = 0.0f;
            }
        }
    }
}

template <int VEC>
__global__ __launch_bounds__(kWave* kWavesPerBlock) void causal_softmax_fwd_kernel(
    const float* __restrict__ scores, float* __restrict__ probs, int64_t rows, int T,
    float scale, int zero_block) {
    using V = Vec<VEC>;
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t r = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
    if (r >= rows) return;
    const int i = static_cast<int>(r % T);
    const float* s_row = scores + r * T;
    float* p_row = probs + r * T;
    const int n = i + 1;  // valid columns
    const int nchunks = (n + VEC - 1) / VEC;
    const int zend = zero_block > 0 ? min(T, (i / zero_block + 1) * zero_block) : T;

    if (nchunks <= kChunks * kWave) {
        typename V::T x[kChunks];
        float mx = -FLT_MAX;
#pragma unroll
        for (int u = 0; u < kChunks; ++u) {
            const int c = lane + u * kWave;
            if (c < nchunks) {
                x[u] = V::load(s_row + c * VEC);
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    const float val = (c * VEC + e < n) ? V::get(x[u], e) * scale : -FLT_MAX;
                    V::set(x[u], e, val);
                    mx = fmaxf(mx, val);
                }
            }
        }
        mx = wave_max(mx);
        float sum = 0.0f;
#pragma unroll
        for (int u = 0; u < kChunks; ++u) {
            const int c = lane + u * kWave;
            if (c < nchunks) {
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    const float ev = (c * VEC + e < n) ? expf(V::get(x[u], e) - mx) : 0.0f;
                    V::set(x[u], e, ev);
                    sum += ev;
                }
            }
        }
        sum = wave_sum(sum);
        const float inv = 1.0f / (sum + 1e-12f);
#pragma unroll
        for (int u = 0; u < kChunks; ++u) {
            const int c = lane + u * kWave;
            if (c < nchunks) {
#pragma unroll
                for (int e = 0; e < VEC; ++e) V::set(x[u], e, V::get(x[u], e) * inv);
                if (c * VEC + VEC <= T) {
                    V::store(p_row + c * VEC, x[u]);
                } else {
                    for (int e = 0; e < VEC && c * VEC + e < T; ++e) p_row[c * VEC + e] = V::get(x[u], e);
                }
            }
        }
        // Columns of the last valid chunk beyond n were written as exp(-inf) * inv = 0.
        zero_suffix<VEC>(p_row, nchunks * VEC, zend, lane);
        return;
    }

    // Streaming path: per-lane online (max, sum), merged across the wave.
    float m = -FLT_MAX, l = 0.0f;
    for (int c = lane; c < nchunks; c += kWave) {
        const typename V::T x = V::load(s_row + c * VEC);
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            if (c * VEC + e < n) {
                const float val = V::get(x, e) * scale;
                if (val > m) {
                    l = l * expf(m - val) + 1.0f;
                    m = val;
                } else {
                    l += expf(val - m);
                }
            }
        }
    }
    const float mx = wave_max(m);
    float sum = (l > 0.0f) ? l * expf(m - mx) : 0.0f;
    sum = wave_sum(sum);
    const float inv = 1.0f / (sum + 1e-12f);
    for (int c = lane; c < nchunks; c += kWave) {
        typename V::T x = V::load(s_row + c * VEC);
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            const float pv = (c * VEC + e < n) ? expf(V::get(x, e) * scale - mx) * inv : 0.0f;
            V::set(x, e, pv);
        }
        if (c * VEC + VEC <= T) {
            V::store(p_row + c * VEC, x);
        } else {
            for (int e = 0; e < VEC && c * VEC + e < T; ++e) p_row[c * VEC + e] = V::get(x, e);
        }
    }
    zero_suffix<VEC>(p_row, nchunks * VEC, zend, lane);
}

template <int VEC>
__global__ __launch_bounds__(kWave* kWavesPerBlock) void causal_softmax_bwd_kernel(
    const float* __restrict__ dprobs, const float* __restrict__ probs,
    float* __restrict__ dscores, int64_t rows, int T, float scale, int zero_block) {
    using V = Vec<VEC>;
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t r = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
    if (r >= rows) return;
    const int i = static_cast<int>(r % T);
    const float* dp_row = dprobs + r * T;
    const float* p_row = probs + r * T;
    float* ds_row = dscores + r * T;
    const int n = i + 1;
    const int nchunks = (n + VEC - 1) / VEC;
    const int zend = zero_block > 0 ? min(T, (i / zero_block + 1) * zero_block) : T;

    if (nchunks <= kChunks * kWave) {
        typename V::T pv[kChunks], dpv[kChunks];
        float dot = 0.0f;
#pragma unroll
        for (int u = 0; u < kChunks; ++u) {
            const int c = lane + u * kWave;
            if (c < nchunks) {
                pv[u] = V::load(p_row + c * VEC);
                dpv[u] = V::load(dp_row + c * VEC);
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    if (c * VEC + e < n) dot += V::get(pv[u], e) * V::get(dpv[u], e);
                }
            }
        }
        dot = wave_sum(dot);
#pragma unroll
        for (int u = 0; u < kChunks; ++u) {
            const int c = lane + u * kWave;
            if (c < nchunks) {
                typename V::T o;
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    const float val =
                        (c * VEC + e < n)
                            ? scale * V::get(pv[u], e) * (V::get(dpv[u], e) - dot)
                            : 0.0f;
                    V::set(o, e, val);
                }
                if (c * VEC + VEC <= T) {
                    V::store(ds_row + c * VEC, o);
                } else {
                    for (int e = 0; e < VEC && c * VEC + e < T; ++e) ds_row[c * VEC + e] = V::get(o, e);
                }
            }
        }
        zero_suffix<VEC>(ds_row, nchunks * VEC, zend, lane);
        return;
    }

    float dot = 0.0f;
    for (int c = lane; c < nchunks; c += kWave) {
        const typename V::T pv = V::load(p_row + c * VEC);
        const typename V::T dpv = V::load(dp_row + c * VEC);
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            if (c * VEC + e < n) dot += V::get(pv, e) * V::get(dpv, e);
        }
    }
    dot = wave_sum(dot);
    for (int c = lane; c < nchunks; c += kWave) {
        const typename V::T pv = V::load(p_row + c * VEC);
        const typename V::T dpv = V::load(dp_row + c * VEC);
        typename V::T o;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            const float val =
                (c * VEC + e < n) ? scale * V::get(pv, e) * (V::get(dpv, e) - dot) : 0.0f;
            V::set(o, e, val);
        }
        if (c * VEC + VEC <= T) {
            V::store(ds_row + c * VEC, o);
        } else {
            for (int e = 0; e < VEC && c * VEC + e < T; ++e) ds_row[c * VEC + e] = V::get(o, e);
        }
    }
    zero_suffix<VEC>(ds_row, nchunks * VEC, zend, lane);
}

bool vec4_ok(const void* a, const void* b, const void* c, int T) {
    const uintptr_t bits = reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
                           reinterpret_cast<uintptr_t>(c);
    return (T % 4 == 0) && (bits & 15u) == 0;
}

}  // namespace

void launch_causal_softmax_fwd_f32(const float* scores, float* probs, int64_t rows, int T,
                                   float scale, hipStream_t stream, int zero_block) {
    const dim3 grid(static_cast<unsigned>((rows + kWavesPerBlock - 1) / kWavesPerBlock));
    const dim3 block(kWave * kWavesPerBlock);
    if (vec4_ok(scores, probs, probs, T)) {
        hipLaunchKernelGGL(causal_softmax_fwd_kernel<4>, grid, block, 0, stream, scores, probs,
                           rows, T, scale, zero_block);
    } else {
        hipLaunchKernelGGL(causal_softmax_fwd_kernel<1>, grid, block, 0, stream, scores, probs,
                           rows, T, scale, zero_block);
    }
}

void launch_causal_softmax_bwd_f32(const float* dprobs, const float* probs, float* dscores,
                                   int64_t rows, int T, float scale, hipStream_t stream,
                                   int zero_block) {
    const dim3 grid(static_cast<unsigned>((rows + kWavesPerBlock - 1) / kWavesPerBlock));
    const dim3 block(kWave * kWavesPerBlock);
    if (vec4_ok(dprobs, probs, dscores, T)) {
        hipLaunchKernelGGL(causal_softmax_bwd_kernel<4>, grid, block, 0, stream, dprobs, probs,
                           dscores, rows, T, scale, zero_block);
    } else {
        hipLaunchKernelGGL(causal_softmax_bwd_kernel<1>, grid, block, 0, stream, dprobs, probs,
                           dscores, rows, T, scale, zero_block);
    }
}

}  // namespace tcamd
