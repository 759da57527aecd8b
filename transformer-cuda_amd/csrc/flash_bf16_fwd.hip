// flash_bf16_fwd.hip - tiled causal attention forward, bf16 fast path, on
// v_mfma_f32_32x32x16_bf16 with fp32 accumulation.
//
// Algorithm: the reference's tiled online-softmax forward (src/kernels/attention.cu:518-624),
// with the same statistics contract P_ij = exp(scale*q_i.k_j - m_i) / l_i.
//
// Layout of the work.  A workgroup of 4 waves (one per SIMD of a CU) owns 256 queries of one
// (b, h) head, as 8 sub-blocks of 32; wave w computes sub-blocks w and 7-w, so the causal
// work of the four waves is equal.  K and V stream through LDS in 64-key tiles, double
// buffered and shared by the four waves; each K fragment read from LDS feeds the MFMAs of
// both sub-blocks of a wave.  Workgroups are issued heaviest query block first, with every
// block of a head on one XCD when the number of heads is a multiple of 8.
//
// Per 32-key half tile and sub-block:
//   S^T = K Q^T       4 MFMAs at d = 64; A = K rows from LDS (16-byte reads), B = Q in VGPRs
//   online softmax    lane l holds 16 scores of query l%32: 15 in-lane max/sum steps and one
//                     v_permlane32_swap; exponentials on v_exp_f32 in the log2 domain
//   O^T += V^T P^T    4 MFMAs; B = P straight from the S^T accumulator (rounded to bf16),
//                     A = V^T read from the row-major V tile with ds_read_tr16_b64, which
//                     hands each lane 4 consecutive keys of one head dimension: the two
//                     reads per MFMA carry exactly the keys the accumulator layout gives P.
// The running maximum used for the exponentials is only raised when a row's maximum grows by
// more than 2^8 (in exponent units), which leaves p <= 256 and the fp32 sums exact in form
// while skipping the O rescale on almost every tile; the true maximum is tracked beside it
// and the exported (m, l) are converted to it.
//
// Staging.  Tiles are copied HBM -> LDS with global_load_lds_dwordx4 (1 KB per wave
// instruction) into rows whose 16-byte chunks are XOR-swizzled by row, with padding after
// every 8 rows, so that both the row reads of K and the transposing reads of V hit distinct
// banks (bf16_tile.hpp).
#include <math.h>

#include "device_common.hpp"
#include "bf16_tile.hpp"
#include "launch.hpp"

namespace tcamd {
namespace {

using namespace bf16t;

constexpr int kKeyTile = kRowTile;    // keys per LDS tile
constexpr float kRescaleLog2 = 8.0f;  // raise the running max only beyond p = 2^8

template <int D>
struct FwdSmem {
    uint16_t k[2][Swz<D>::kBytes / 2];
    uint16_t v[2][Swz<D>::kBytes / 2];
};

// Maximum and sum of a lane's 16 scores as balanced trees (dependency depth 3 and 4 instead
// of 8 and 16 for a running reduction).
__device__ __forceinline__ float max_tree16(const f32x16& s) {
    const float a = fmaxf(fmaxf(s[0], s[1]), s[2]), b = fmaxf(fmaxf(s[3], s[4]), s[5]);
    const float c = fmaxf(fmaxf(s[6], s[7]), s[8]), d = fmaxf(fmaxf(s[9], s[10]), s[11]);
    const float e = fmaxf(fmaxf(s[12], s[13]), s[14]);
    return fmaxf(fmaxf(fmaxf(a, b), c), fmaxf(fmaxf(d, e), s[15]));
}
__device__ __forceinline__ float sum_tree16(const f32x16& s) {
    float t[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) t[i] = s[2 * i] + s[2 * i + 1];
#pragma unroll
    for (int i = 0; i < 4; ++i) t[i] += t[i + 4];
    return (t[0] + t[2]) + (t[1] + t[3]);
}

// Per-wave softmax state of one 32-query sub-block.
template <int D>
struct SubState {
    f32x16 acc[D / 32];  // O^T accumulator
    float m_used;        // max the exponentials are taken against
    float m_true;        // running max of the raw scores q.k
    float l;             // running sum of 2^(s*c - m_used*c)
};

// Masks S^T for keys kb.. against queries qj + col, runs the online-softmax update of `st`,
// and packs P as the two B operands of the PV products.
template <int D>
__device__ __forceinline__ void softmax_step(f32x16& s, SubState<D>& st, bf16x8 (&pb)[2],
                                             int kb, int qj, int col, int half, float c) {
    if (kb + 31 > qj) {  // the half tile crosses the diagonal of this sub-block
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if (kb + acc_row(r, half) > qj + col) s[r] = -INFINITY;
    }
    float mx = max_tree16(s);
    mx = xhalf_max(mx);
    st.m_true = fmaxf(st.m_true, mx);
    if (__builtin_amdgcn_ballot_w64((mx - st.m_used) * c > kRescaleLog2) != 0) {
        const float m_new = fmaxf(st.m_used, mx);
        const float alpha = exp2_fast((st.m_used - m_new) * c);  // 0 at the start
        st.l *= alpha;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) st.acc[dt] *= alpha;
        st.m_used = m_new;
    }
    const float mc = st.m_used * c;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = exp2_fast(fmaf(s[r], c, -mc));
    st.l += xhalf_sum(sum_tree16(s));
    pb[0] = pack_b(s, 0);
    pb[1] = pack_b(s, 1);
}

// One 32-key half tile (keys kb..kb+31, tile rows 32h..) for sub-block 1, and sub-block 0
// too when BOTH.  ka[st] / va[dt]: this lane's LDS read addresses in the current tiles for
// the K chunk of step st and the V^T fragment of head-dim tile dt (half 0, keys 0..).
template <int D, bool BOTH>
__device__ __forceinline__ void half_step(int kb, const uint32_t (&ka)[D / 16],
                                          const uint32_t (&va)[D / 32], const bf16x8 (&q0)[D / 16],
                                          const bf16x8 (&q1)[D / 16], SubState<D>& st0,
                                          SubState<D>& st1, int qj0, int qj1, int col, int half,
                                          float c) {
    f32x16 s0 = f32x16{}, s1 = f32x16{};
#pragma unroll
    for (int st = 0; st < D / 16; ++st) {
        const bf16x8 a = lds_b128(ka[st]);
        s1 = mfma_32x32x16_bf16(a, q1[st], s1);
        if constexpr (BOTH) s0 = mfma_32x32x16_bf16(a, q0[st], s0);
    }
    bf16x8 p0[2], p1[2];
    softmax_step<D>(s1, st1, p1, kb, qj1, col, half, c);
    if constexpr (BOTH) softmax_step<D>(s0, st0, p0, kb, qj0, col, half, c);
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const bf16x8 a = lds_tr(va[dt] + u * Swz<D>::rows(16), Swz<D>::rows(8));
            st1.acc[dt] = mfma_32x32x16_bf16(a, p1[u], st1.acc[dt]);
            if constexpr (BOTH) st0.acc[dt] = mfma_32x32x16_bf16(a, p0[u], st0.acc[dt]);
        }
    }
}

// NSUB = 2: 256 queries per workgroup, wave w owns sub-blocks w (0) and 7-w (1).
// NSUB = 1: 128 queries per workgroup, wave w owns sub-block w (1) (small grids).
template <int D, int NSUB>
__global__ __launch_bounds__(kWave* kWaves) void flash_fwd_bf16_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, uint16_t* __restrict__ o, float* __restrict__ m_out,
    float* __restrict__ l_out, int BH, int T, float scale, int nblk, HeadView xv,
    HeadView ov) {
    using S = Swz<D>;
    __shared__ __attribute__((aligned(1024))) FwdSmem<D> sm;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 31;
    const int half = lane >> 5;
    int bh, blk;
    map_block(blockIdx.x, BH, nblk, true, bh, blk);
    constexpr int kBlock = kWaves * NSUB * kSub;
    const int q0 = blk * kBlock;
    const int qj0 = q0 + kSub * wave;                                     // sub-block 0
    const int qj1 = NSUB == 2 ? q0 + kSub * (2 * kWaves - 1 - wave) : qj0;  // sub-block 1
    const size_t xoff = xv.off(bh), ooff = ov.off(bh);  // q, k, v head / o head
    const int xrs = xv.row, ors = ov.row;
    const uint16_t* kh = k + xoff;
    const uint16_t* vh = v + xoff;
    const float c = scale * kLog2e;

    bf16x8 qr0[D / 16], qr1[D / 16];
    if constexpr (NSUB == 2) load_rowop<D>(qr0, q + xoff, qj0 + col, T, half, xrs);
    load_rowop<D>(qr1, q + xoff, qj1 + col, T, half, xrs);

    const int kend = min(T, q0 + kBlock);
    const int ntile = (kend + kKeyTile - 1) / kKeyTile;
    const uint32_t k_lds = lds_addr(sm.k[0]);
    const uint32_t v_lds = lds_addr(sm.v[0]);
    dma_tile<D>(kh, 0, T, k_lds, wave, lane, xrs);
    dma_tile<D>(vh, 0, T, v_lds, wave, lane, xrs);

    // Lane read offsets within a tile (K row reads, V transposing reads).
    uint32_t koff[D / 16], voff[D / 32];
    lane_offsets<D>(lane, koff, voff);

    SubState<D> st0, st1;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
        st0.acc[dt] = f32x16{};
        st1.acc[dt] = f32x16{};
    }
    st0.m_used = st1.m_used = -INFINITY;
    st0.m_true = st1.m_true = -INFINITY;
    st0.l = st1.l = 0.0f;

    // Half tiles hh = 0 .. 2*ntile-1 (keys 32*hh ..).  Sub-block w is active for
    // hh < hA, sub-block 7-w for hh < hB; every wave takes part in every tile's barrier and
    // copy.  Three straight loops keep the accumulators out of any control-flow join.
    const int nhalf_t = (T + 31) / 32;
    const int hA = NSUB == 2 ? min(qj0 / 32 + 1, nhalf_t) : 0;
    const int hB = min(qj1 / 32 + 1, nhalf_t);
    const int hend = 2 * ntile;
    uint32_t ka[D / 16], va[D / 32];
    auto tile_sync = [&](int hh) {
        const int kt = hh >> 1;
        if ((hh & 1) == 0) {
            wait_vm<0>();     // this wave's copies of tile kt landed ...
            __syncthreads();  // ... and every wave's; tile kt-1 is no longer read by anyone
            if (kt + 1 < ntile) {
                const uint32_t nbuf = static_cast<uint32_t>((kt + 1) & 1) * S::kBytes;
                dma_tile<D>(kh, (kt + 1) * kKeyTile, T, k_lds + nbuf, wave, lane, xrs);
                dma_tile<D>(vh, (kt + 1) * kKeyTile, T, v_lds + nbuf, wave, lane, xrs);
            }
        }
        const uint32_t base = static_cast<uint32_t>(kt & 1) * S::kBytes +
                              static_cast<uint32_t>(hh & 1) * S::rows(32);
#pragma unroll
        for (int st = 0; st < D / 16; ++st) ka[st] = k_lds + base + koff[st];
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) va[dt] = v_lds + base + voff[dt];
    };
    int hh = 0;
    for (; hh < hA; ++hh) {
        tile_sync(hh);
        half_step<D, true>(32 * hh, ka, va, qr0, qr1, st0, st1, qj0, qj1, col, half, c);
    }
    for (; hh < hB; ++hh) {
        tile_sync(hh);
        half_step<D, false>(32 * hh, ka, va, qr0, qr1, st0, st1, qj0, qj1, col, half, c);
    }
    for (; hh < hend; ++hh) tile_sync(hh);

#pragma unroll
    for (int j = 2 - NSUB; j < 2; ++j) {
        const SubState<D>& st = j == 0 ? st0 : st1;
        const int qi = (j == 0 ? qj0 : qj1) + col;
        if (qi < T) {
            store_row<D>(o + ooff, qi, half, st.acc, 1.0f / st.l, ors);  // l >= 1
            if (half == 0) {
                const size_t r = static_cast<size_t>(bh) * T + qi;
                // m = scale * max_j q.k; l relative to that maximum
                if (m_out != nullptr) m_out[r] = st.m_true * scale;
                if (l_out != nullptr) l_out[r] = st.l * exp2_fast((st.m_used - st.m_true) * c);
            }
        }
    }
}

template <int D, int NSUB>
void fwd_launch(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o,
                float* m_out, float* l_out, int BH, int T, float scale, const HeadView& xv,
                const HeadView& ov, hipStream_t stream) {
    constexpr int kBlock = kWaves * NSUB * kSub;
    const int nblk = (T + kBlock - 1) / kBlock;
    hipLaunchKernelGGL((flash_fwd_bf16_kernel<D, NSUB>), dim3(BH * nblk), dim3(kWave * kWaves),
                       0, stream, q, k, v, o, m_out, l_out, BH, T, scale, nblk, xv, ov);
}

template <int D>
void fwd_dispatch(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o,
                  float* m_out, float* l_out, int BH, int T, float scale, const HeadView& xv,
                  const HeadView& ov, hipStream_t stream) {
    // d = 128: one sub-block per wave fits two waves per SIMD (two sub-blocks do not)
    if (D >= 128 || use_single_subblock(BH, T))
        fwd_launch<D, 1>(q, k, v, o, m_out, l_out, BH, T, scale, xv, ov, stream);
    else
        fwd_launch<D, 2>(q, k, v, o, m_out, l_out, BH, T, scale, xv, ov, stream);
}

}  // namespace

void launch_flash_fwd_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                           uint16_t* o, float* m_out, float* l_out, int BH, int T, int d,
                           float scale, const HeadView& xv, const HeadView& ov,
                           hipStream_t stream) {
    switch (d) {
        case 32: fwd_dispatch<32>(q, k, v, o, m_out, l_out, BH, T, scale, xv, ov, stream); break;
        case 64: fwd_dispatch<64>(q, k, v, o, m_out, l_out, BH, T, scale, xv, ov, stream); break;
        default: fwd_dispatch<128>(q, k, v, o, m_out, l_out, BH, T, scale, xv, ov, stream); break;
    }
}

}  // namespace tcamd
