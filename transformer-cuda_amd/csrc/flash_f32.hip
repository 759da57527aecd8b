// flash_f32.hip - tiled causal attention, fp32 parity path, on v_mfma_f32_32x32x2_f32.
//
// Algorithm (reference: src/kernels/attention.cu:518-624 forward, :659-692 D = rowsum(dO*O),
// :696-812 dQ, :816-955 dK/dV).  Same maths and the same m/l statistics contract,
//     P_ij = exp(scale*q_i.k_j - m_i) / l_i,
// re-laid out for CDNA4: a wavefront owns 32 rows (queries, or keys in the dK/dV kernel)
// and every contraction is a 32x32 MFMA tile.
//
// The orientation of each product is chosen so that the softmax state never crosses
// lanes except between the two wave halves:
//   * forward / dQ compute S^T = K Q^T (keys = MFMA rows, queries = MFMA columns), so
//     lane l holds 16 scores of query l%32; row max / row sum are 15 in-lane ops plus
//     one v_permlane32_swap.  The S^T accumulator registers are, unchanged, the B operand
//     of O^T += V^T P^T (and dQ^T += K^T dS^T): no LDS round trip for P.
//   * dK/dV compute S = Q K^T (keys = columns), so P and dS are the B operands of
//     dV^T += dO^T P and dK^T += Q^T dS.
// Operands that a wave reuses for its whole life (its Q rows, or its K and V rows) sit in
// VGPRs; tiles shared by the workgroup's waves (K/V, or Q/dO/stats) are staged through LDS
// from coalesced 16-byte global loads, double-buffered so that the next tile's loads are
// in flight while the current one is multiplied.  Causal skipping is per wave (a wave
// stops at its diagonal tile) and per workgroup (tiles past the last query are never
// loaded).  Workgroups are issued heaviest-first to shorten the causal tail.
#include <math.h>

#include "device_common.hpp"
#include "launch.hpp"

namespace tcamd {
namespace {

constexpr int kTile = 32;  // rows per wave and per LDS tile

// 32 rows x D floats, global -> registers -> LDS (row stride STRIDE floats).
template <int D, int NTHREADS, int STRIDE>
struct TileCopy {
    static constexpr int kF4PerRow = D / 4;
    static constexpr int kPerThread = kTile * kF4PerRow / NTHREADS;
    static_assert(kPerThread >= 1 && kTile * kF4PerRow % NTHREADS == 0, "tile split");
    f32x4 r[kPerThread];

    __device__ __forceinline__ void load(const float* __restrict__ head, int row0, int T,
                                         int tid) {
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            const int idx = tid + i * NTHREADS;
            const int row = idx / kF4PerRow;
            const int c4 = idx - row * kF4PerRow;
            if (row0 + row < T) {
                r[i] = *reinterpret_cast<const f32x4*>(head + (row0 + row) * D + c4 * 4);
            } else {
                r[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }
    }
    __device__ __forceinline__ void store(float* lds, int tid) const {
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            const int idx = tid + i * NTHREADS;
            const int row = idx / kF4PerRow;
            const int c4 = idx - row * kF4PerRow;
            *reinterpret_cast<f32x4*>(lds + row * STRIDE + c4 * 4) = r[i];
        }
    }
};

// Lane (col, half) loads its row's half: dst[j] = src[row][half*D/2 + j], zeros if row >= T.
template <int D>
__device__ __forceinline__ void load_row_half(float (&dst)[D / 2], const float* __restrict__ head,
                                              int row, int T, int half) {
    if (row < T) {
        const float* p = head + row * D + half * (D / 2);
#pragma unroll
        for (int j = 0; j < D / 2; j += 4) {
            const f32x4 x = *reinterpret_cast<const f32x4*>(p + j);
            dst[j] = x[0];
            dst[j + 1] = x[1];
            dst[j + 2] = x[2];
            dst[j + 3] = x[3];
        }
    } else {
#pragma unroll
        for (int j = 0; j < D / 2; ++j) dst[j] = 0.0f;
    }
}

// acc += A * B where A row i = LDS row i (k over the lane half's D/2 columns) and B column j
// = breg of lane j: the contraction over the head dimension.
//   lds_row = lds + (lane%32)*STRIDE + half*D/2
template <int D>
__device__ __forceinline__ f32x16 mma_rows(const float* lds_row, const float (&breg)[D / 2],
                                           f32x16 acc) {
#pragma unroll
    for (int j = 0; j < D / 2; j += 4) {
        const f32x4 a = *reinterpret_cast<const f32x4*>(lds_row + j);
        acc = mfma_32x32x2_f32(a[0], breg[j], acc);
        acc = mfma_32x32x2_f32(a[1], breg[j + 1], acc);
        acc = mfma_32x32x2_f32(a[2], breg[j + 2], acc);
        acc = mfma_32x32x2_f32(a[3], breg[j + 3], acc);
    }
    return acc;
}

// acc[dt] += X^T(32 x 32 tile dt of the head dim) * Y where Y is a 32x32 accumulator tile
// held in MFMA layout (bacc) whose rows index the contraction dimension:
//   acc[dt][i = c][j] += sum_r lds[r][dt*32 + c] * Y[r][j]
// Step s feeds row acc_row(s, half) of Y: lane (c, half) supplies A = lds[acc_row(s,half)]
// [dt*32 + c] and B = bacc[s], which is Y[acc_row(s, half)][col].
template <int D, int STRIDE>
__device__ __forceinline__ void mma_cols(const float* lds, int col, int half, const f32x16& bacc,
                                         f32x16 (&acc)[D / 32]) {
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const float a = lds[acc_row(s, half) * STRIDE + dt * 32 + col];
            acc[dt] = mfma_32x32x2_f32(a, bacc[s], acc[dt]);
        }
    }
}

// Store a (D x 32) transposed accumulator: acc[dt][v] is element (row, dt*32 + acc_row(v,
// half)) of a row-major (T, D) tensor, row = this lane's row.  Four float4 per 32 columns.
template <int D>
__device__ __forceinline__ void store_acc_row(float* __restrict__ head, int row, int half,
                                              const f32x16 (&acc)[D / 32], float mul) {
    float* p = head + row * D + 4 * half;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            f32x4 o;
            o[0] = acc[dt][4 * g + 0] * mul;
            o[1] = acc[dt][4 * g + 1] * mul;
            o[2] = acc[dt][4 * g + 2] * mul;
            o[3] = acc[dt][4 * g + 3] * mul;
            *reinterpret_cast<f32x4*>(p + dt * 32 + 8 * g) = o;
        }
    }
}

// Compensated (Kahan) running sum of per-tile partial products: sum += x with the rounding
// error carried in comp.  Each tile's contraction is accumulated by the MFMA into a fresh
// zero accumulator (16 fp32 adds per element per tile) and only tile totals enter the
// running sum, so the rounding error no longer grows with the sequence length.  Used for
// d_head <= 64; at d_head = 128 the compensation terms do not fit the register file of the
// dK/dV kernel, which then adds the tile totals without compensation (two-level sum).
template <int D>
constexpr bool kCompensated = D <= 64;

template <int N>
__device__ __forceinline__ void plain_add(f32x16 (&sum)[N], const f32x16 (&x)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) sum[i] += x[i];
}

template <int N>
__device__ __forceinline__ void kahan_add(f32x16 (&sum)[N], f32x16 (&comp)[N],
                                          const f32x16 (&x)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const f32x16 y = x[i] - comp[i];
        const f32x16 t = sum[i] + y;
        comp[i] = (t - sum[i]) - y;
        sum[i] = t;
    }
}

// --------------------------------------------------------------------------------------
// Forward.  Workgroup = NW waves = 32*NW queries of one (b, h); wave w owns queries
// [q0 + 32w, q0 + 32w + 32).  grid = BH * nqt, heaviest query tile first.
// --------------------------------------------------------------------------------------
template <int D, int NW>
__global__ __launch_bounds__(kWave* NW) void flash_fwd_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    float* __restrict__ o, float* __restrict__ m_out, float* __restrict__ l_out, int BH, int T,
    float scale, int nqt) {
    constexpr int NT = kWave * NW;
    constexpr int KS = D + 4;  // K rows: 16-byte reads along a row
    constexpr int VS = D + 8;  // V rows: read down a column by the two wave halves
    __shared__ float Ks[2][kTile * KS];
    __shared__ float Vs[2][kTile * VS];

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

    const size_t head_off = static_cast<size_t>(bh) * T * D;
    const float* qh = q + head_off;
    const float* kh = k + head_off;
    const float* vh = v + head_off;

    float qreg[D / 2];
    load_row_half<D>(qreg, qh, qi, T, half);

    f32x16 acc[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) acc[dt] = f32x16{};
    float m_i = -INFINITY;
    float l_i = 0.0f;

    const int kend = min(T, q0 + kTile * NW);
    const int ntiles = (kend + kTile - 1) / kTile;
    const int wave_last = qw / kTile;  // diagonal tile of this wave

    TileCopy<D, NT, KS> kcp;
    TileCopy<D, NT, VS> vcp;
    kcp.load(kh, 0, T, tid);
    vcp.load(vh, 0, T, tid);
    kcp.store(Ks[0], tid);
    vcp.store(Vs[0], tid);
    __syncthreads();

    for (int t = 0; t < ntiles; ++t) {
        const int buf = t & 1;
        if (t + 1 < ntiles) {
            kcp.load(kh, (t + 1) * kTile, T, tid);
            vcp.load(vh, (t + 1) * kTile, T, tid);
        }
        if (wave_live && t <= wave_last) {
            f32x16 s = mma_rows<D>(Ks[buf] + col * KS + half * (D / 2), qreg, f32x16{});
            if (t == wave_last) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    if (t * kTile + acc_row(r, half) > qi) s[r] = -INFINITY;
                }
            }
            float mx = s[0];
#pragma unroll
            for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
            mx = xhalf_max(mx);
            const float m_new = fmaxf(m_i, mx * scale);
            const float alpha = expf(m_i - m_new);
            float rs = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                s[r] = expf(fmaf(s[r], scale, -m_new));
                rs += s[r];
            }
            rs = xhalf_sum(rs);
            l_i = l_i * alpha + rs;
            m_i = m_new;
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) acc[dt] *= alpha;
            mma_cols<D, VS>(Vs[buf], col, half, s, acc);
        }
        if (t + 1 < ntiles) {
            kcp.store(Ks[buf ^ 1], tid);
            vcp.store(Vs[buf ^ 1], tid);
        }
        __syncthreads();
    }

    if (wave_live && qi < T) {
        const float inv_l = 1.0f / l_i;  // l_i >= 1 (the row maximum contributes exp(0))
        store_acc_row<D>(o + head_off, qi, half, acc, inv_l);
        if (half == 0) {
            if (m_out != nullptr) m_out[static_cast<size_t>(bh) * T + qi] = m_i;
            if (l_out != nullptr) l_out[static_cast<size_t>(bh) * T + qi] = l_i;
        }
    }
}

// --------------------------------------------------------------------------------------
// D[r] = sum_e dO[r,e] * O[r,e]  (the reference's standalone launcher).  16 lanes per row.
// --------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void dot_do_o_f32_kernel(const float* __restrict__ dO,
                                                           const float* __restrict__ O,
                                                           float* __restrict__ D,
                                                           int64_t rows, int d) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 16 + (threadIdx.x >> 4);
    const int sub = threadIdx.x & 15;
    float acc = 0.0f;
    if (row < rows) {
        const float* a = dO + row * d;
        const float* b = O + row * d;
        for (int e = sub; e < d; e += 16) acc = fmaf(a[e], b[e], acc);
    }
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 16);
    if (row < rows && sub == 0) D[row] = acc;
}

// --------------------------------------------------------------------------------------
// Backward stage 1 (query-parallel): D = rowsum(dO*O) and
//     dQ_i = scale * sum_j P_ij (dP_ij - D_i) k_j,   dP = dO V^T.
// Wave = 32 queries; K/V tiles through LDS.
// --------------------------------------------------------------------------------------
template <int D, int NW>
__global__ __launch_bounds__(kWave* NW) void flash_bwd_dq_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ o, const float* __restrict__ dO, const float* __restrict__ m,
    const float* __restrict__ l, float* __restrict__ dq, float* __restrict__ Dws, int BH,
    int T, float scale, int nqt) {
    constexpr int NT = kWave * NW;
    constexpr int KS = D + 4;
    __shared__ float Ks[2][kTile * KS];
    __shared__ float Vs[2][kTile * KS];

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

    float qreg[D / 2];
    float doreg[D / 2];
    load_row_half<D>(qreg, q + head_off, qi, T, half);
    load_row_half<D>(doreg, dO + head_off, qi, T, half);

    // D_i from this lane's half row of O, completed across the halves.
    float Dval;
    {
        float orow[D / 2];
        load_row_half<D>(orow, o + head_off, qi, T, half);
        float part = 0.0f;
#pragma unroll
        for (int j = 0; j < D / 2; ++j) part = fmaf(doreg[j], orow[j], part);
        Dval = xhalf_sum(part);
    }
    if (row_ok && half == 0) Dws[stat_off + qi] = Dval;
    const float m_row = row_ok ? m[stat_off + qi] : 0.0f;
    const float inv_l = row_ok ? 1.0f / l[stat_off + qi] : 0.0f;

    f32x16 acc[D / 32], comp[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
        acc[dt] = f32x16{};
        comp[dt] = f32x16{};
    }

    const int kend = min(T, q0 + kTile * NW);
    const int ntiles = (kend + kTile - 1) / kTile;
    const int wave_last = qw / kTile;

    const float* kh = k + head_off;
    const float* vh = v + head_off;
    TileCopy<D, NT, KS> kcp;
    TileCopy<D, NT, KS> vcp;
    kcp.load(kh, 0, T, tid);
    vcp.load(vh, 0, T, tid);
    kcp.store(Ks[0], tid);
    vcp.store(Vs[0], tid);
    __syncthreads();

    for (int t = 0; t < ntiles; ++t) {
        const int buf = t & 1;
        if (t + 1 < ntiles) {
            kcp.load(kh, (t + 1) * kTile, T, tid);
            vcp.load(vh, (t + 1) * kTile, T, tid);
        }
        if (wave_live && t <= wave_last) {
            const int rbase = col * KS + half * (D / 2);
            f32x16 s = mma_rows<D>(Ks[buf] + rbase, qreg, f32x16{});
            f32x16 dp = mma_rows<D>(Vs[buf] + rbase, doreg, f32x16{});
            const bool diag = (t == wave_last);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float p = expf(fmaf(s[r], scale, -m_row)) * inv_l;
                if (diag && t * kTile + acc_row(r, half) > qi) p = 0.0f;
                s[r] = p * (dp[r] - Dval);  // dS^T (without the scale)
            }
            f32x16 part[D / 32];
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) part[dt] = f32x16{};
            mma_cols<D, KS>(Ks[buf], col, half, s, part);
            if constexpr (kCompensated<D>) {
                kahan_add(acc, comp, part);
            } else {
                plain_add(acc, part);
            }
        }
        if (t + 1 < ntiles) {
            kcp.store(Ks[buf ^ 1], tid);
            vcp.store(Vs[buf ^ 1], tid);
        }
        __syncthreads();
    }

    if (wave_live && row_ok) store_acc_row<D>(dq + head_off, qi, half, acc, scale);
}

// --------------------------------------------------------------------------------------
// Backward stage 2 (key-parallel):
//     dV_j = sum_i P_ij dO_i,   dK_j = scale * sum_i P_ij (dP_ij - D_i) q_i.
// Wave = 32 keys (K and V rows in VGPRs); Q/dO tiles and per-query m, 1/l, D through LDS.
// grid = BH * nkt, lowest key tile (most queries) first.
// --------------------------------------------------------------------------------------
template <int D, int NW>
__global__ __launch_bounds__(kWave* NW) void flash_bwd_dkdv_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ dO, const float* __restrict__ m, const float* __restrict__ l,
    const float* __restrict__ Dws, float* __restrict__ dk, float* __restrict__ dv, int BH,
    int T, float scale, int nkt) {
    constexpr int NT = kWave * NW;
    constexpr int QS = D + 4;
    __shared__ float Qs[2][kTile * QS];
    __shared__ float Ps[2][kTile * QS];  // dO tile
    __shared__ float St[2][3][kTile];    // m, 1/l, D of the tile's queries

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

    float kreg[D / 2];
    float vreg[D / 2];
    load_row_half<D>(kreg, k + head_off, kj, T, half);
    load_row_half<D>(vreg, v + head_off, kj, T, half);

    f32x16 dk_acc[D / 32], dv_acc[D / 32], dk_comp[D / 32], dv_comp[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
        dk_acc[dt] = f32x16{};
        dv_acc[dt] = f32x16{};
        dk_comp[dt] = f32x16{};
        dv_comp[dt] = f32x16{};
    }

    const int qt_first = k0 / kTile;
    const int nqt = (T + kTile - 1) / kTile;
    const int wave_first = kw / kTile;  // diagonal query tile of this wave

    const float* qh = q + head_off;
    const float* doh = dO + head_off;
    TileCopy<D, NT, QS> qcp;
    TileCopy<D, NT, QS> docp;
    // Stats: threads [0, 96) each stage one value (m, 1/l or D) of one query row.
    const int st_kind = tid >> 5;  // 0: m, 1: 1/l, 2: D (only tid < 96)
    const int st_row = tid & 31;
    auto load_stat = [&](int row0) -> float {
        const int r = row0 + st_row;
        if (tid >= 3 * kTile || r >= T) return 0.0f;
        if (st_kind == 0) return m[stat_off + r];
        if (st_kind == 1) return 1.0f / l[stat_off + r];
        return Dws[stat_off + r];
    };

    qcp.load(qh, qt_first * kTile, T, tid);
    docp.load(doh, qt_first * kTile, T, tid);
    float st = load_stat(qt_first * kTile);
    qcp.store(Qs[0], tid);
    docp.store(Ps[0], tid);
    if (tid < 3 * kTile) St[0][st_kind][st_row] = st;
    __syncthreads();

    for (int t = qt_first; t < nqt; ++t) {
        const int buf = (t - qt_first) & 1;
        if (t + 1 < nqt) {
            qcp.load(qh, (t + 1) * kTile, T, tid);
            docp.load(doh, (t + 1) * kTile, T, tid);
            st = load_stat((t + 1) * kTile);
        }
        if (wave_live && t >= wave_first) {
            const int rbase = col * QS + half * (D / 2);
            f32x16 s = mma_rows<D>(Qs[buf] + rbase, kreg, f32x16{});
            f32x16 dp = mma_rows<D>(Ps[buf] + rbase, vreg, f32x16{});
            const float* sm = St[buf][0];
            const float* sl = St[buf][1];
            const float* sd = St[buf][2];
            f32x16 ds;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int qr = acc_row(r, half);
                float p = expf(fmaf(s[r], scale, -sm[qr])) * sl[qr];
                if (t * kTile + qr < kj) p = 0.0f;
                s[r] = p;
                ds[r] = p * (dp[r] - sd[qr]);
            }
            f32x16 part[D / 32];
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) part[dt] = f32x16{};
            mma_cols<D, QS>(Ps[buf], col, half, s, part);
            if constexpr (kCompensated<D>) {
                kahan_add(dv_acc, dv_comp, part);
            } else {
                plain_add(dv_acc, part);
            }
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) part[dt] = f32x16{};
            mma_cols<D, QS>(Qs[buf], col, half, ds, part);
            if constexpr (kCompensated<D>) {
                kahan_add(dk_acc, dk_comp, part);
            } else {
                plain_add(dk_acc, part);
            }
        }
        if (t + 1 < nqt) {
            qcp.store(Qs[buf ^ 1], tid);
            docp.store(Ps[buf ^ 1], tid);
            if (tid < 3 * kTile) St[buf ^ 1][st_kind][st_row] = st;
        }
        __syncthreads();
    }

    if (wave_live && kj < T) {
        store_acc_row<D>(dk + head_off, kj, half, dk_acc, scale);
        store_acc_row<D>(dv + head_off, kj, half, dv_acc, 1.0f);
    }
}

constexpr int kWavesFwd = 4;
constexpr int kWavesBwd = 4;

template <int D>
void fwd_dispatch(const float* q, const float* k, const float* v, float* o, float* m_out,
                  float* l_out, int BH, int T, float scale, hipStream_t stream) {
    const int nqt = (T + kTile * kWavesFwd - 1) / (kTile * kWavesFwd);
    hipLaunchKernelGGL((flash_fwd_f32_kernel<D, kWavesFwd>), dim3(BH * nqt),
                       dim3(kWave * kWavesFwd), 0, stream, q, k, v, o, m_out, l_out, BH, T,
                       scale, nqt);
}

template <int D>
void dq_dispatch(const float* q, const float* k, const float* v, const float* o,
                 const float* dO, const float* m, const float* l, float* dq, float* Dws, int BH,
                 int T, float scale, hipStream_t stream) {
    const int nqt = (T + kTile * kWavesBwd - 1) / (kTile * kWavesBwd);
    hipLaunchKernelGGL((flash_bwd_dq_f32_kernel<D, kWavesBwd>), dim3(BH * nqt),
                       dim3(kWave * kWavesBwd), 0, stream, q, k, v, o, dO, m, l, dq, Dws, BH,
                       T, scale, nqt);
}

template <int D>
void dkdv_dispatch(const float* q, const float* k, const float* v, const float* dO,
                   const float* m, const float* l, const float* Dws, float* dk, float* dv,
                   int BH, int T, float scale, hipStream_t stream) {
    const int nkt = (T + kTile * kWavesBwd - 1) / (kTile * kWavesBwd);
    hipLaunchKernelGGL((flash_bwd_dkdv_f32_kernel<D, kWavesBwd>), dim3(BH * nkt),
                       dim3(kWave * kWavesBwd), 0, stream, q, k, v, dO, m, l, Dws, dk, dv, BH,
                       T, scale, nkt);
}

}  // namespace

void launch_flash_fwd_f32(const float* q, const float* k, const float* v, float* o,
                          float* m_out, float* l_out, int BH, int T, int d, float scale,
                          hipStream_t stream) {
    switch (d) {
        case 32: fwd_dispatch<32>(q, k, v, o, m_out, l_out, BH, T, scale, stream); break;
        case 64: fwd_dispatch<64>(q, k, v, o, m_out, l_out, BH, T, scale, stream); break;
        default: fwd_dispatch<128>(q, k, v, o, m_out, l_out, BH, T, scale, stream); break;
    }
}

void launch_dot_do_o_f32(const float* dO, const float* O, float* D, int64_t rows, int d,
                         hipStream_t stream) {
    const unsigned blocks = static_cast<unsigned>((rows + 15) / 16);
    hipLaunchKernelGGL(dot_do_o_f32_kernel, dim3(blocks), dim3(256), 0, stream, dO, O, D, rows,
                       d);
}

void launch_flash_bwd_dq_f32(const float* q, const float* k, const float* v, const float* o,
                             const float* dO, const float* m, const float* l, float* dq,
                             float* Dws, int BH, int T, int d, float scale,
                             hipStream_t stream) {
    switch (d) {
        case 32: dq_dispatch<32>(q, k, v, o, dO, m, l, dq, Dws, BH, T, scale, stream); break;
        case 64: dq_dispatch<64>(q, k, v, o, dO, m, l, dq, Dws, BH, T, scale, stream); break;
        default: dq_dispatch<128>(q, k, v, o, dO, m, l, dq, Dws, BH, T, scale, stream); break;
    }
}

void launch_flash_bwd_dkdv_f32(const float* q, const float* k, const float* v,
                               const float* dO, const float* m, const float* l,
                               const float* Dws, float* dk, float* dv, int BH, int T, int d,
                               float scale, hipStream_t stream) {
    switch (d) {
        case 32: dkdv_dispatch<32>(q, k, v, dO, m, l, Dws, dk, dv, BH, T, scale, stream); break;
        case 64: dkdv_dispatch<64>(q, k, v, dO, m, l, Dws, dk, dv, BH, T, scale, stream); break;
        default: dkdv_dispatch<128>(q, k, v, dO, m, l, Dws, dk, dv, BH, T, scale, stream); break;
    }
}

}  // namespace tcamd
