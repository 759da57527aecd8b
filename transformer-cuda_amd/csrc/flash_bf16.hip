// flash_bf16.hip - tiled causal attention backward, bf16 fast path, on
// v_mfma_f32_32x32x16_bf16 (the forward is in flash_bf16_fwd.hip).
//
// Same algorithm, wave/tile structure and statistics contract as flash_f32.hip (reference:
// src/kernels/attention.cu:518-955), with bf16 operands and fp32 accumulation:
//   * softmax runs in the log2 domain: scores are scaled by scale*log2(e) with one FMA and
//     exponentiated with v_exp_f32 (exp2); m_out/l_out are converted back to the natural
//     domain so the reference contract P = exp(scale*q.k - m)/l holds;
//   * P and dS are rounded to bf16 as MFMA B operands; O/dQ/dK/dV are rounded once, at
//     the store.
// A 32x32x16 MFMA takes eight consecutive k per lane.  Products that contract over the
// head dimension read 16 contiguous bytes per lane from a row-major LDS tile.  Products
// that contract over the sequence (O^T += V^T P^T, dQ^T += K^T dS^T, dV^T += dO^T P,
// dK^T += Q^T dS) take their A operand from a transposed LDS copy of the tile, written
// while staging: the eight k of a lane are then two 8-byte runs that match the rows the
// accumulator layout gives to P / dS (acc_row(8u..8u+7, half)).
#include <math.h>

#include "device_common.hpp"
#include "launch.hpp"

namespace tcamd {
namespace {

constexpr int kTile = 32;
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kTStride = kTile + 4;  // transposed tiles: 72-byte rows, conflict-free 8-B reads

__device__ __forceinline__ bf16x8 as_bf16x8(u16x8 x) { return __builtin_bit_cast(bf16x8, x); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// 32 rows x D bf16: global (16-byte chunks) -> registers -> LDS row-major, stride RS.
template <int D, int NT, int RS>
struct RowTile {
    static constexpr int kChunksPerRow = D / 8;
    static constexpr int kChunks = kTile * kChunksPerRow;
    static constexpr int kPerThread = (kChunks + NT - 1) / NT;
    u16x8 r[kPerThread];

    __device__ __forceinline__ void load(const uint16_t* __restrict__ head, int row0, int T,
                                         int tid) {
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            const int idx = tid + i * NT;
            const int row = idx / kChunksPerRow;
            const int c = idx - row * kChunksPerRow;
            if ((kChunks % NT == 0 || idx < kChunks) && row0 + row < T) {
                r[i] = *reinterpret_cast<const u16x8*>(head + (row0 + row) * D + c * 8);
            } else {
                r[i] = u16x8{};
            }
        }
    }
    __device__ __forceinline__ void store(uint16_t* lds, int tid) const {
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            const int idx = tid + i * NT;
            if (kChunks % NT == 0 || idx < kChunks) {
                const int row = idx / kChunksPerRow;
                const int c = idx - row * kChunksPerRow;
                *reinterpret_cast<u16x8*>(lds + row * RS + c * 8) = r[i];
            }
        }
    }
};

// 32 rows x D bf16 -> LDS transposed (D rows of kTStride), element (row, c) at
// lds[c*kTStride + row].  A thread owns a pair of rows and CW columns; it writes packed
// (row 2p, row 2p+1) dwords.
template <int D, int NT>
struct TransTile {
    static constexpr int kThreadsPerPair = NT / (kTile / 2);
    static constexpr int CW = D / kThreadsPerPair;  // columns per thread
    static_assert(CW >= 2 && CW % 2 == 0 && CW <= 8, "transposed tile split");
    typedef uint16_t vec_t __attribute__((ext_vector_type(CW)));
    vec_t a, b;

    __device__ __forceinline__ void load(const uint16_t* __restrict__ head, int row0, int T,
                                         int tid) {
        const int p = tid / kThreadsPerPair;
        const int c0 = (tid - p * kThreadsPerPair) * CW;
        const int r = row0 + 2 * p;
        a = (r < T) ? *reinterpret_cast<const vec_t*>(head + r * D + c0) : vec_t{};
        b = (r + 1 < T) ? *reinterpret_cast<const vec_t*>(head + (r + 1) * D + c0) : vec_t{};
    }
    __device__ __forceinline__ void store(uint16_t* lds, int tid) const {
        const int p = tid / kThreadsPerPair;
        const int c0 = (tid - p * kThreadsPerPair) * CW;
#pragma unroll
        for (int e = 0; e < CW; ++e) {
            const uint32_t w = static_cast<uint32_t>(a[e]) | (static_cast<uint32_t>(b[e]) << 16);
            *reinterpret_cast<uint32_t*>(lds + (c0 + e) * kTStride + 2 * p) = w;
        }
    }
};

// Lane (col, half) loads its row: dst[j] = row[16j + 8*half .. +8], zeros if row >= T.
template <int D>
__device__ __forceinline__ void load_row(bf16x8 (&dst)[D / 16], const uint16_t* __restrict__ head,
                                         int row, int T, int half) {
#pragma unroll
    for (int j = 0; j < D / 16; ++j) {
        dst[j] = (row < T) ? as_bf16x8(*reinterpret_cast<const u16x8*>(head + row * D + 16 * j +
                                                                        8 * half))
                           : as_bf16x8(u16x8{});
    }
}

// acc += (row-major LDS tile rows) x breg, contracting over the head dimension.
//   lds_row = lds + (lane%32)*RS + 8*half
template <int D>
__device__ __forceinline__ f32x16 mma_rows(const uint16_t* lds_row, const bf16x8 (&breg)[D / 16],
                                           f32x16 acc) {
#pragma unroll
    for (int j = 0; j < D / 16; ++j) {
        const bf16x8 a = as_bf16x8(*reinterpret_cast<const u16x8*>(lds_row + 16 * j));
        acc = mfma_32x32x16_bf16(a, breg[j], acc);
    }
    return acc;
}

// Pack accumulator rows acc_row(8u .. 8u+7, half) of a 32x32 fp32 tile into a B operand.
__device__ __forceinline__ bf16x8 pack_b(const f32x16& x, int u) {
    bf16x8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = static_cast<__bf16>(x[8 * u + e]);
    return r;
}

// acc[dt] += X^T * Y over the 32 sequence rows of a tile: A from the transposed tile
// (row dt*32 + col), B = packed Y rows (pb[u] = rows acc_row(8u..8u+7, half)).
template <int D>
__device__ __forceinline__ void mma_cols(const uint16_t* ldsT, int col, int half,
                                         const bf16x8 (&pb)[2], f32x16 (&acc)[D / 32]) {
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
        const uint16_t* rowp = ldsT + (dt * 32 + col) * kTStride + 4 * half;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const u16x4 lo = *reinterpret_cast<const u16x4*>(rowp + 16 * u);
            const u16x4 hi = *reinterpret_cast<const u16x4*>(rowp + 16 * u + 8);
            const u16x8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            acc[dt] = mfma_32x32x16_bf16(as_bf16x8(a), pb[u], acc[dt]);
        }
    }
}

template <int D>
__device__ __forceinline__ void store_acc_row(uint16_t* __restrict__ head, int row, int half,
                                              const f32x16 (&acc)[D / 32], float mul) {
    uint16_t* p = head + row * D + 4 * half;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            u16x4 o;
            o[0] = f32_to_bf16_bits(acc[dt][4 * g + 0] * mul);
            o[1] = f32_to_bf16_bits(acc[dt][4 * g + 1] * mul);
            o[2] = f32_to_bf16_bits(acc[dt][4 * g + 2] * mul);
            o[3] = f32_to_bf16_bits(acc[dt][4 * g + 3] * mul);
            *reinterpret_cast<u16x4*>(p + dt * 32 + 8 * g) = o;
        }
    }
}

// ---------------------------------------------------------------------------------------
// Backward stage 1 (query-parallel): D = rowsum(dO*O) (fp32) and dQ.
// LDS: K row-major (S^T), V row-major (dP^T), K transposed (dQ^T += K^T dS^T).
// ---------------------------------------------------------------------------------------
template <int D, int NW>
__global__ __launch_bounds__(kWave* NW) void flash_bwd_dq_bf16_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint16_t* __restrict__ o,
    const uint16_t* __restrict__ dO, const float* __restrict__ m, const float* __restrict__ l,
    uint16_t* __restrict__ dq, float* __restrict__ Dws, int BH, int T, float scale, int nqt) {
    constexpr int NT = kWave * NW;
    constexpr int RS = D + 8;
    __shared__ __attribute__((aligned(16))) uint16_t Ks[2][kTile * RS];
    __shared__ __attribute__((aligned(16))) uint16_t Vs[2][kTile * RS];
    __shared__ __attribute__((aligned(16))) uint16_t Kt[2][D * kTStride];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid >> 6;
    const int col = lane & 31;
    const int half = lane >> 5;

    const int id = blockIdx.x;
    const int qt = nqt - 1 - id / BH;
    const int bh = id - (id / BH) * BH;
    const int q0 = qt * kTile * NW;
    const int qw = q0 + kTile * wave;
    const int qi = qw + col;
    const bool wave_live = qw < T;
    const bool row_ok = qi < T;

    const size_t head_off = static_cast<size_t>(bh) * T * D;
    const size_t stat_off = static_cast<size_t>(bh) * T;

    bf16x8 qreg[D / 16];
    bf16x8 doreg[D / 16];
    load_row<D>(qreg, q + head_off, qi, T, half);
    load_row<D>(doreg, dO + head_off, qi, T, half);

    float Dval;
    {
        bf16x8 orow[D / 16];
        load_row<D>(orow, o + head_off, qi, T, half);
        float part = 0.0f;
#pragma unroll
        for (int j = 0; j < D / 16; ++j) {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                part = fmaf(static_cast<float>(doreg[j][e]), static_cast<float>(orow[j][e]), part);
        }
        Dval = xhalf_sum(part);
    }
    if (row_ok && half == 0) Dws[stat_off + qi] = Dval;
    const float c = scale * kLog2e;
    const float lse2 = row_ok ? m[stat_off + qi] * kLog2e + log2f(l[stat_off + qi]) : INFINITY;

    f32x16 acc[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) acc[dt] = f32x16{};

    const int kend = min(T, q0 + kTile * NW);
    const int ntiles = (kend + kTile - 1) / kTile;
    const int wave_last = qw / kTile;

    const uint16_t* kh = k + head_off;
    const uint16_t* vh = v + head_off;
    RowTile<D, NT, RS> kcp, vcp;
    TransTile<D, NT> ktcp;
    kcp.load(kh, 0, T, tid);
    vcp.load(vh, 0, T, tid);
    ktcp.load(kh, 0, T, tid);
    kcp.store(Ks[0], tid);
    vcp.store(Vs[0], tid);
    ktcp.store(Kt[0], tid);
    __syncthreads();

    for (int t = 0; t < ntiles; ++t) {
        const int buf = t & 1;
        if (t + 1 < ntiles) {
            kcp.load(kh, (t + 1) * kTile, T, tid);
            vcp.load(vh, (t + 1) * kTile, T, tid);
            ktcp.load(kh, (t + 1) * kTile, T, tid);
        }
        if (wave_live && t <= wave_last) {
            const int rbase = col * RS + 8 * half;
            f32x16 s = mma_rows<D>(Ks[buf] + rbase, qreg, f32x16{});
            f32x16 dp = mma_rows<D>(Vs[buf] + rbase, doreg, f32x16{});
            const bool diag = (t == wave_last);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float p = fast_exp2(fmaf(s[r], c, -lse2));
                if (diag && t * kTile + acc_row(r, half) > qi) p = 0.0f;
                s[r] = p * (dp[r] - Dval);
            }
            const bf16x8 pb[2] = {pack_b(s, 0), pack_b(s, 1)};
            mma_cols<D>(Kt[buf], col, half, pb, acc);
        }
        if (t + 1 < ntiles) {
            kcp.store(Ks[buf ^ 1], tid);
            vcp.store(Vs[buf ^ 1], tid);
            ktcp.store(Kt[buf ^ 1], tid);
        }
        __syncthreads();
    }

    if (wave_live && row_ok) store_acc_row<D>(dq + head_off, qi, half, acc, scale);
}

// ---------------------------------------------------------------------------------------
// Backward stage 2 (key-parallel): dK, dV.  Wave = 32 keys (K, V in VGPRs).
// LDS: Q and dO row-major (S, dP) and transposed (dK^T, dV^T); per-query lse2 and D.
// ---------------------------------------------------------------------------------------
template <int D, int NW>
__global__ __launch_bounds__(kWave* NW) void flash_bwd_dkdv_bf16_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint16_t* __restrict__ dO,
    const float* __restrict__ m, const float* __restrict__ l, const float* __restrict__ Dws,
    uint16_t* __restrict__ dk, uint16_t* __restrict__ dv, int BH, int T, float scale, int nkt) {
    constexpr int NT = kWave * NW;
    constexpr int RS = D + 8;
    __shared__ __attribute__((aligned(16))) uint16_t Qs[2][kTile * RS];
    __shared__ __attribute__((aligned(16))) uint16_t Gs[2][kTile * RS];  // dO
    __shared__ __attribute__((aligned(16))) uint16_t Qt[2][D * kTStride];
    __shared__ __attribute__((aligned(16))) uint16_t Gt[2][D * kTStride];
    __shared__ float St[2][2][kTile];  // lse2, D

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid >> 6;
    const int col = lane & 31;
    const int half = lane >> 5;

    const int id = blockIdx.x;
    const int kt = id / BH;
    const int bh = id - kt * BH;
    const int k0 = kt * kTile * NW;
    const int kw = k0 + kTile * wave;
    const int kj = kw + col;
    const bool wave_live = kw < T;

    const size_t head_off = static_cast<size_t>(bh) * T * D;
    const size_t stat_off = static_cast<size_t>(bh) * T;

    bf16x8 kreg[D / 16];
    bf16x8 vreg[D / 16];
    load_row<D>(kreg, k + head_off, kj, T, half);
    load_row<D>(vreg, v + head_off, kj, T, half);

    f32x16 dk_acc[D / 32], dv_acc[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
        dk_acc[dt] = f32x16{};
        dv_acc[dt] = f32x16{};
    }
    const float c = scale * kLog2e;

    const int qt_first = k0 / kTile;
    const int nqt = (T + kTile - 1) / kTile;
    const int wave_first = kw / kTile;

    const uint16_t* qh = q + head_off;
    const uint16_t* doh = dO + head_off;
    RowTile<D, NT, RS> qcp, gcp;
    TransTile<D, NT> qtcp, gtcp;
    const int st_kind = tid >> 5;  // 0: lse2, 1: D  (tid < 64)
    const int st_row = tid & 31;
    auto load_stat = [&](int row0) -> float {
        const int r = row0 + st_row;
        if (tid >= 2 * kTile) return 0.0f;
        if (r >= T) return st_kind == 0 ? INFINITY : 0.0f;  // exp2(-inf) = 0: padded queries
        if (st_kind == 0) return m[stat_off + r] * kLog2e + log2f(l[stat_off + r]);
        return Dws[stat_off + r];
    };

    const int r0 = qt_first * kTile;
    qcp.load(qh, r0, T, tid);
    gcp.load(doh, r0, T, tid);
    qtcp.load(qh, r0, T, tid);
    gtcp.load(doh, r0, T, tid);
    float st = load_stat(r0);
    qcp.store(Qs[0], tid);
    gcp.store(Gs[0], tid);
    qtcp.store(Qt[0], tid);
    gtcp.store(Gt[0], tid);
    if (tid < 2 * kTile) St[0][st_kind][st_row] = st;
    __syncthreads();

    for (int t = qt_first; t < nqt; ++t) {
        const int buf = (t - qt_first) & 1;
        if (t + 1 < nqt) {
            const int rn = (t + 1) * kTile;
            qcp.load(qh, rn, T, tid);
            gcp.load(doh, rn, T, tid);
            qtcp.load(qh, rn, T, tid);
            gtcp.load(doh, rn, T, tid);
            st = load_stat(rn);
        }
        if (wave_live && t >= wave_first) {
            const int rbase = col * RS + 8 * half;
            f32x16 s = mma_rows<D>(Qs[buf] + rbase, kreg, f32x16{});
            f32x16 dp = mma_rows<D>(Gs[buf] + rbase, vreg, f32x16{});
            const float* sl = St[buf][0];
            const float* sd = St[buf][1];
            f32x16 ds;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int qr = acc_row(r, half);
                float p = fast_exp2(fmaf(s[r], c, -sl[qr]));
                if (t * kTile + qr < kj) p = 0.0f;
                s[r] = p;
                ds[r] = p * (dp[r] - sd[qr]);
            }
            const bf16x8 pb[2] = {pack_b(s, 0), pack_b(s, 1)};
            const bf16x8 db[2] = {pack_b(ds, 0), pack_b(ds, 1)};
            mma_cols<D>(Gt[buf], col, half, pb, dv_acc);
            mma_cols<D>(Qt[buf], col, half, db, dk_acc);
        }
        if (t + 1 < nqt) {
            qcp.store(Qs[buf ^ 1], tid);
            gcp.store(Gs[buf ^ 1], tid);
            qtcp.store(Qt[buf ^ 1], tid);
            gtcp.store(Gt[buf ^ 1], tid);
            if (tid < 2 * kTile) St[buf ^ 1][st_kind][st_row] = st;
        }
        __syncthreads();
    }

    if (wave_live && kj < T) {
        store_acc_row<D>(dk + head_off, kj, half, dk_acc, scale);
        store_acc_row<D>(dv + head_off, kj, half, dv_acc, 1.0f);
    }
}

constexpr int kWaves = 4;

template <int D>
void dq_dispatch(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* o,
                 const uint16_t* dO, const float* m, const float* l, uint16_t* dq, float* Dws,
                 int BH, int T, float scale, hipStream_t stream) {
    const int nqt = (T + kTile * kWaves - 1) / (kTile * kWaves);
    hipLaunchKernelGGL((flash_bwd_dq_bf16_kernel<D, kWaves>), dim3(BH * nqt),
                       dim3(kWave * kWaves), 0, stream, q, k, v, o, dO, m, l, dq, Dws, BH, T,
                       scale, nqt);
}

template <int D>
void dkdv_dispatch(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* dO,
                   const float* m, const float* l, const float* Dws, uint16_t* dk, uint16_t* dv,
                   int BH, int T, float scale, hipStream_t stream) {
    const int nkt = (T + kTile * kWaves - 1) / (kTile * kWaves);
    hipLaunchKernelGGL((flash_bwd_dkdv_bf16_kernel<D, kWaves>), dim3(BH * nkt),
                       dim3(kWave * kWaves), 0, stream, q, k, v, dO, m, l, Dws, dk, dv, BH, T,
                       scale, nkt);
}

}  // namespace

void launch_flash_bwd_dq_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                              const uint16_t* o, const uint16_t* dO, const float* m,
                              const float* l, uint16_t* dq, float* Dws, int BH, int T, int d,
                              float scale, hipStream_t stream) {
    switch (d) {
        case 32: dq_dispatch<32>(q, k, v, o, dO, m, l, dq, Dws, BH, T, scale, stream); break;
        case 64: dq_dispatch<64>(q, k, v, o, dO, m, l, dq, Dws, BH, T, scale, stream); break;
        default: dq_dispatch<128>(q, k, v, o, dO, m, l, dq, Dws, BH, T, scale, stream); break;
    }
}

void launch_flash_bwd_dkdv_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                const uint16_t* dO, const float* m, const float* l,
                                const float* Dws, uint16_t* dk, uint16_t* dv, int BH, int T,
                                int d, float scale, hipStream_t stream) {
    switch (d) {
        case 32: dkdv_dispatch<32>(q, k, v, dO, m, l, Dws, dk, dv, BH, T, scale, stream); break;
        case 64: dkdv_dispatch<64>(q, k, v, dO, m, l, Dws, dk, dv, BH, T, scale, stream); break;
        default: dkdv_dispatch<128>(q, k, v, dO, m, l, Dws, dk, dv, BH, T, scale, stream); break;
    }
}

}  // namespace tcamd
