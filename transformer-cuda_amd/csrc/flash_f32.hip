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
//
// Work decomposition.  The kernels are persistent: as many workgroups as fit resident are
// launched, and each pulls (head, block) tasks heaviest first from a per-XCD atomic queue
// (sched.hpp), which balances the very unequal causal blocks across CUs and keeps a head's
// K/V in one XCD's L2.  A workgroup is four wavefronts, one per SIMD; the four split the
// task's tiles into contiguous ranges, each with private LDS tiles, and merge their partial
// results through LDS at the end of the task (the only workgroup barriers).  The forward also
// has a form on shared tiles (flash_fwd_f32_shared_kernel: 128 queries per workgroup, K/V
// tiles double-buffered and shared by the four waves, XCD-aware static block order), which
// runs where it measures faster (fwd_on_shared_tiles); so do the two backward stages
// (flash_bwd_dq_f32_shared_kernel, flash_bwd_dkdv_f32_shared_kernel: 128 queries or keys
// per workgroup, the streamed tiles shared the same way).
//
// Staging.  The 32-row tiles streamed over the sequence (K/V, or Q/dO) are copied from HBM
// straight into LDS with global_load_lds_dwordx4 (16 bytes per lane, 1 KB of the tile per
// wave instruction, each lane's source offsets precomputed once per kernel), bypassing
// VGPRs, into rows padded to a bank-conflict-free stride.  Each
// tensor has one LDS tile: the next tile's copy is issued as soon as the current tile's
// last LDS read has returned, and waited for (vmcnt) just before its first read, so the
// copy overlaps the other tensor's contraction and the softmax; a second resident wave on
// the SIMD covers what remains.  In the dQ kernel a tile starts with the V contraction, so
// the K copy issued at the end of the previous tile lands behind it.
//
// Summation.  The backward kernels accumulate each 32-row tile's contraction in a fresh
// MFMA accumulator and add the tile totals into the running sum (two-level summation), so
// the fp32 rounding error grows with the number of tiles, not with the sequence length.
//
// The backward also runs in the dS-first order: D alone (d_rows_f32_kernel, the dQ
// kernel's sums), the dK/dV kernel writing dS as well (its DS form), then dQ = scale * dS K
// from the stored dS (flash_bwd_dq_ds_f32_kernel), which leaves out the dQ kernel's second
// computation of S and dP.
#include <math.h>

#include <type_traits>

#include "bf16_tile.hpp"
#include "device_common.hpp"
#include "launch.hpp"
#include "lds_dma.hpp"
#include "sched.hpp"

namespace tcamd {
namespace {

constexpr int kTile = 32;  // rows per wave and per LDS tile
constexpr float kLog2e = 1.4426950408889634f;

// 2^x on the transcendental unit (v_exp_f32).  The softmax runs in the log2 domain:
// exp(scale*s - m) = 2^(s*c - m*log2 e) with c = scale*log2 e folded into one FMA.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// A 32-row tile of a (T, D) head copied into LDS rows of STRIDE floats with 16-byte copies:
// copy instruction i writes LDS bytes [1024 i, 1024 i + 1024) of the tile, lane l the 16
// bytes at 1024 i + 16 l, i.e. byte b of row r with (r, b) = divmod(1024 i + 16 l, 4 STRIDE).
// Lanes that land on a row's padding copy the row's first 16 bytes there (never read);
// lanes past the tile's end, in the last instruction only, are off.  In a partial last tile
// (rows at or beyond T) those rows read the last 16 bytes of row T - 1 instead: every read
// stays inside the head and the padding rows hold finite values, which the kernels mask.
template <int D, int STRIDE>
struct TileShape {
    static constexpr int kRowBytes = 4 * STRIDE;
    static constexpr int kBytes = kTile * kRowBytes;
    static constexpr int kInst = (kBytes + 1023) / 1024;
    static_assert(STRIDE % 4 == 0 && D % 4 == 0, "16-byte chunks");
    // Row r and source byte (0 for padding) of lane `lane` in instruction i.
    __device__ static void row_byte(int i, int lane, int& r, int& b) {
        const int o = 1024 * i + 16 * lane;
        r = o / kRowBytes;
        b = o - r * kRowBytes;
        if (b >= 4 * D) b = 0;
    }
    __device__ static bool active(int i, int lane) {
        return i + 1 < kInst || 1024 * i + 16 * lane < kBytes;
    }
    // Largest in-bounds offset from row0 when the tile is partial.
    __device__ static uint32_t last(int row0, int T, int rs) {
        return static_cast<uint32_t>((T - 1 - row0) * rs * 4 + 4 * D - 16);
    }
};

// Copy plan for one row stride rs: voff[i] is the lane's source byte offset from the tile's
// first row, the same for every tile, so a whole tile costs no VALU.
template <int D, int STRIDE>
struct TileCopy : TileShape<D, STRIDE> {
    using S = TileShape<D, STRIDE>;
    uint32_t voff[S::kInst];

    __device__ void init(int lane, int rs) {
#pragma unroll
        for (int i = 0; i < S::kInst; ++i) {
            int r, b;
            S::row_byte(i, lane, r, b);
            voff[i] = static_cast<uint32_t>(r * rs * 4 + b);
        }
    }
    // Copy rows [row0, row0 + kTile) of a head (rows rs floats apart; rs is the init's) into
    // the tile at LDS byte address lds.
    __device__ void copy(const float* __restrict__ head, int row0, int T, uint32_t lds, int lane,
                         int rs) const {
        const float* base = head + static_cast<size_t>(row0) * rs;
        const bool whole = row0 + kTile <= T;
        const uint32_t last = S::last(row0, T, rs);
#pragma unroll
        for (int i = 0; i < S::kInst; ++i)
            if (S::active(i, lane))
                dma_dwordx4(base, lds + static_cast<uint32_t>(1024 * i),
                            whole ? voff[i] : min(voff[i], last));
    }
};

// Copy plan for any row stride: rb[i] = r | (b / 16) << 24, and every copy forms
// r * 4 rs + b = mul_u24(rb, 4 rs) + (rb >> 20) (bits 20-23 are zero) in two VALU
// instructions.  One plan serves two tiles whose rows are strided differently.  The two
// instructions are asm so that the optimiser cannot hoist them out of the tile loop into one
// register per instruction and stride.
template <int D, int STRIDE>
struct TileCopyAnyStride : TileShape<D, STRIDE> {
    using S = TileShape<D, STRIDE>;
    static_assert(kTile < (1 << 20) && S::kRowBytes / 16 < 256, "fields of rb");
    uint32_t rb[S::kInst];

    __device__ void init(int lane) {
#pragma unroll
        for (int i = 0; i < S::kInst; ++i) {
            int r, b;
            S::row_byte(i, lane, r, b);
            rb[i] = static_cast<uint32_t>(r) | static_cast<uint32_t>(b / 16) << 24;
        }
    }
    __device__ static uint32_t offset(uint32_t p, uint32_t rs4) {
        uint32_t off, t;
        asm volatile(
            "v_lshrrev_b32 %1, 20, %2\n\t"
            "v_mad_u32_u24 %0, %2, %3, %1"
            : "=v"(off), "=&v"(t)
            : "v"(p), "s"(rs4));
        return off;
    }
    __device__ void copy(const float* __restrict__ head, int row0, int T, uint32_t lds, int lane,
                         int rs) const {
        const float* base = head + static_cast<size_t>(row0) * rs;
        const uint32_t rs4 = static_cast<uint32_t>(rs) * 4u;
        if (row0 + kTile <= T) {
#pragma unroll
            for (int i = 0; i < S::kInst; ++i)
                if (S::active(i, lane))
                    dma_dwordx4(base, lds + static_cast<uint32_t>(1024 * i), offset(rb[i], rs4));
        } else {
            const uint32_t last = S::last(row0, T, rs);
#pragma unroll
            for (int i = 0; i < S::kInst; ++i)
                if (S::active(i, lane))
                    dma_dwordx4(base, lds + static_cast<uint32_t>(1024 * i),
                                min(offset(rb[i], rs4), last));
        }
    }
};

// Copy instructions per tile (every tile of the kernels has kTile rows of D + 4 or D + 8
// floats; both give the same count).
template <int D>
constexpr int kTileDma = TileShape<D, D + 4>::kInst;
static_assert(TileShape<32, 36>::kInst == TileShape<32, 40>::kInst &&
              TileShape<64, 68>::kInst == TileShape<64, 72>::kInst &&
              TileShape<128, 132>::kInst == TileShape<128, 136>::kInst,
              "the copy waits count one instruction total per tile");

// Lane (col, half) loads its row's half: dst[j] = src[row][half*D/2 + j], zeros if row >= T
// (rows rs floats apart).
template <int D>
__device__ __forceinline__ void load_row_half(float (&dst)[D / 2], const float* __restrict__ head,
                                              int row, int T, int half, int rs) {
    if (row < T) {
        const float* p = head + static_cast<size_t>(row) * rs + half * (D / 2);
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
                                              const f32x16 (&acc)[D / 32], float mul, int rs) {
    float* p = head + static_cast<size_t>(row) * rs + 4 * half;
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

template <int N>
__device__ __forceinline__ void zero(f32x16 (&x)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] = f32x16{};
}

template <int N>
__device__ __forceinline__ void add_into(f32x16 (&sum)[N], const f32x16 (&x)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) sum[i] += x[i];
}

// A wave's accumulator tiles in LDS, lane-major (conflict-free): element (i, r) of lane l at
// part[(i*16 + r)*64 + l].
template <int N>
__device__ __forceinline__ void put_part(float* part, const f32x16 (&x)[N], int lane) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) part[(i * 16 + r) * kWave + lane] = x[i][r];
    }
}
// Store element (i, r) of an accumulator set, i.e. column i*32 + acc_row(r, half) of row
// `row` of a row-major (T, D) tensor, for the flat indices f = i*16 + r in [f0, f0 + 8):
// two float4 stores (f0 is a multiple of 8, so the 8 elements are rows acc_row(8u..8u+7)).
template <int D>
__device__ __forceinline__ void store_slice8(float* __restrict__ head, int row, int half,
                                             int f0, const float (&x)[8], float mul, int rs) {
    const int i = f0 >> 4;
    const int u = (f0 & 15) >> 3;  // which 8 of the 16 accumulator rows
    float* p = head + static_cast<size_t>(row) * rs + i * 32 + 16 * u + 4 * half;
    f32x4 a, b;
    a[0] = x[0] * mul; a[1] = x[1] * mul; a[2] = x[2] * mul; a[3] = x[3] * mul;
    b[0] = x[4] * mul; b[1] = x[5] * mul; b[2] = x[6] * mul; b[3] = x[7] * mul;
    *reinterpret_cast<f32x4*>(p) = a;
    *reinterpret_cast<f32x4*>(p + 8) = b;
}

// Work split of a task over the NW waves of a workgroup: wave w takes the contiguous tile
// range [n*w/NW, n*(w+1)/NW) of the task's n tiles, and the workgroup waits at the merge
// for the wave with the most tiles.  The forward and dK/dV kernels use 4 waves (one per
// SIMD); the dQ kernel uses 2, which halves that wait when a task's tiles do not split
// evenly (its per-wave LDS tiles still leave room for two waves per SIMD).
constexpr int kFwdWaves = 4, kDqWaves = 2, kDkdvWaves = 4;
template <int NW>
__device__ __forceinline__ void wave_range(int n, int wave, int& t0, int& t1) {
    t0 = n * wave / NW;
    t1 = n * (wave + 1) / NW;
}

#define TCAMD_F32_KERNEL(NW) __global__ __launch_bounds__(kWave*(NW))

// The next task is fetched by lane 0 of wave 0, right after that wave's first tile copies
// are issued, so the atomic's round trip overlaps the chunk's work.
struct Fetch {
    const TaskQueue* q;  // non-null only for the fetching wave
    unsigned value;
    unsigned cur;        // the task being processed
    __device__ __forceinline__ void issue(int lane) {
        if (q != nullptr && lane == 0) value = q->fetch(cur);
    }
};

// --------------------------------------------------------------------------------------
// Forward.  Task = query block qb (32 queries) of one (b, h); wave w of the workgroup
// runs key tiles [n*w/4, n*(w+1)/4) of the qb+1 tiles with Q in VGPRs and its own K/V
// LDS tiles, and the four partial (O, m, l) are merged through LDS by wave 0.
// --------------------------------------------------------------------------------------
template <int D>
struct FwdLds {
    static constexpr int KS = D + 4;  // K rows: 16-byte reads along a row
    static constexpr int VS = D + 8;  // V rows: read down a column by the two wave halves
    float k[kTile * KS];
    float v[kTile * VS];
};
static_assert(sizeof(FwdLds<32>) >= (32 * 32 + 128) * 4, "partial exchange fits");

template <int D>
__device__ __forceinline__ void fwd_chunk(const float* __restrict__ kh,
                                          const float* __restrict__ vh, int T, int stride,
                                          float c, int qb,
                                          int t0, int t1, const float (&qreg)[D / 2],
                                          FwdLds<D>& L, int lane, Fetch& fetch,
                                          const TileCopy<D, FwdLds<D>::KS>& kc,
                                          const TileCopy<D, FwdLds<D>::VS>& vc,
                                          f32x16 (&acc)[D / 32], float& m_raw, float& l_i) {
    constexpr int KS = FwdLds<D>::KS;
    constexpr int VS = FwdLds<D>::VS;
    const float* Ks = L.k;
    const float* Vs = L.v;
    const int col = lane & 31;
    const int half = lane >> 5;
    const int qi = qb * kTile + col;
    zero(acc);
    m_raw = -INFINITY;  // running max of the raw scores q.k (scale > 0)
    l_i = 0.0f;
    if (t0 >= t1) {
        fetch.issue(lane);
        return;
    }
    kc.copy(kh, t0 * kTile, T, lds_addr(L.k), lane, stride);
    vc.copy(vh, t0 * kTile, T, lds_addr(L.v), lane, stride);
    fetch.issue(lane);

    for (int t = t0; t < t1; ++t) {
        const bool more = t + 1 < t1;
        wait_vm<kTileDma<D>>();  // K tile t landed
        f32x16 s = mma_rows<D>(Ks + col * KS + half * (D / 2), qreg, f32x16{});
        wait_lds();
        if (more) kc.copy(kh, (t + 1) * kTile, T, lds_addr(L.k), lane, stride);
        if (t == qb) {  // diagonal tile
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                if (t * kTile + acc_row(r, half) > qi) s[r] = -INFINITY;
            }
        }
        float mx = s[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
        mx = xhalf_max(mx);
        const float m_new = fmaxf(m_raw, mx);
        const float alpha = exp2_fast((m_raw - m_new) * c);  // 0 on the first tile
        const float mc = m_new * c;
        float rs = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            s[r] = exp2_fast(fmaf(s[r], c, -mc));
            rs += s[r];
        }
        rs = xhalf_sum(rs);
        l_i = l_i * alpha + rs;
        m_raw = m_new;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) acc[dt] *= alpha;
        if (more) {
            wait_vm<kTileDma<D>>();  // V tile t (K t+1 in flight)
        } else {
            wait_vm<0>();
        }
        mma_cols<D, VS>(Vs, col, half, s, acc);
        wait_lds();
        if (more) vc.copy(vh, (t + 1) * kTile, T, lds_addr(L.v), lane, stride);
    }
}

template <int D>
TCAMD_F32_KERNEL(kFwdWaves) void flash_fwd_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    float* __restrict__ o, float* __restrict__ m_out, float* __restrict__ l_out, int BH, int T,
    float scale, int nqb, QueueSlot* slot, int per_xcd, HeadView xv, HeadView ov) {
    __shared__ FwdLds<D> L[kFwdWaves];
    __shared__ unsigned s_next;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 31;
    const int half = lane >> 5;
    const float c = scale * kLog2e;
    const TaskQueue tq = TaskQueue::bind(slot, BH, nqb, per_xcd != 0);
    TileCopy<D, FwdLds<D>::KS> kc;
    TileCopy<D, FwdLds<D>::VS> vc;
    kc.init(lane, xv.row);
    vc.init(lane, xv.row);
    unsigned task = tq.first();
    while (task < tq.n_tasks) {
        int bh, rank;
        tq.decode(task, bh, rank);
        const int qb = nqb - 1 - rank;
        const int qi = qb * kTile + col;
        const size_t xoff = wave_uniform(xv.off(bh)), ooff = wave_uniform(ov.off(bh));
        int t0, t1;
        wave_range<kFwdWaves>(qb + 1, wave, t0, t1);

        float qreg[D / 2];
        load_row_half<D>(qreg, q + xoff, qi, T, half, xv.row);
        Fetch fetch{wave == 0 ? &tq : nullptr, 0u, task};
        f32x16 acc[D / 32];
        float m_raw, l_i;
        fwd_chunk<D>(k + xoff, v + xoff, T, xv.row, c, qb, t0, t1, qreg, L[wave], lane, fetch,
                     kc, vc, acc, m_raw, l_i);

        // Merge: every wave publishes (acc, m, l) over its own tiles; then wave w reduces
        // and stores the 8-element chunks w, w+4, ... of the flat accumulator.
        constexpr int NP = D / 2;  // accumulator floats per lane (a multiple of 8)
        float* part = reinterpret_cast<float*>(&L[wave]);
        put_part(part, acc, lane);
        part[D * 32 + lane] = m_raw;
        part[D * 32 + kWave + lane] = l_i;
        if (wave == 0 && lane == 0) s_next = fetch.value;
        __syncthreads();
        float mw[kFwdWaves], m_tot = -INFINITY;
#pragma unroll
        for (int w = 0; w < kFwdWaves; ++w) {
            mw[w] = reinterpret_cast<const float*>(&L[w])[D * 32 + lane];
            m_tot = fmaxf(m_tot, mw[w]);
        }
        float aw[kFwdWaves], l_tot = 0.0f;
#pragma unroll
        for (int w = 0; w < kFwdWaves; ++w) {
            aw[w] = exp2_fast((mw[w] - m_tot) * c);  // 0 for an empty chunk
            l_tot += reinterpret_cast<const float*>(&L[w])[D * 32 + kWave + lane] * aw[w];
        }
#pragma unroll 1
        for (int f0 = wave * 8; f0 < NP; f0 += 8 * kFwdWaves) {  // 8-element chunks, round robin
            float x[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float sum = 0.0f;
#pragma unroll
                for (int w = 0; w < kFwdWaves; ++w)
                    sum += reinterpret_cast<const float*>(&L[w])[(f0 + e) * kWave + lane] * aw[w];
                x[e] = sum;
            }
            if (qi < T) store_slice8<D>(o + ooff, qi, half, f0, x, 1.0f / l_tot, ov.row);
        }
        if (wave == 0 && half == 0 && qi < T) {
            // max_j scale*s_j = scale * max_j s_j exactly (rounding is monotone); l_tot >= 1
            if (m_out != nullptr) m_out[static_cast<size_t>(bh) * T + qi] = m_tot * scale;
            if (l_out != nullptr) l_out[static_cast<size_t>(bh) * T + qi] = l_tot;
        }
        __syncthreads();
        task = __builtin_amdgcn_readfirstlane(s_next);  // the same in every lane
    }
}

// --------------------------------------------------------------------------------------
// Forward on shared tiles.  A workgroup owns 128 queries of one (b, h), wave w the 32 at
// q0 + 32w; the 32-key K and V tiles are double-buffered in LDS and shared by the four
// waves, which copy each tile together (copy instructions w, w + 4, ... of it) one tile
// ahead, with one barrier per tile.  Wave w runs key tiles 0 .. its diagonal tile and then
// only joins the barriers; it owns its queries' (O, m, l), so nothing is merged.  Per tile
// and wave: S^T = K Q^T (D/2 MFMAs), the online softmax of mma_rows' accumulator, and
// O^T += V^T P^T (D/2 MFMAs), as in the per-wave kernel above.
// --------------------------------------------------------------------------------------
template <int D>
struct FwdSharedLds {
    static constexpr int KS = FwdLds<D>::KS;
    static constexpr int VS = FwdLds<D>::VS;
    float k[2][kTile * KS];
    float v[2][kTile * VS];
};
constexpr int kFwdSharedWaves = 4;

// Copy instructions i = wave, wave + 4, ... of one tile's plan (TileShape), this lane's
// source offsets precomputed.
template <int D, int STRIDE>
struct SharedTileCopy : TileShape<D, STRIDE> {
    using S = TileShape<D, STRIDE>;
    static constexpr int kPer = (S::kInst + kFwdSharedWaves - 1) / kFwdSharedWaves;
    uint32_t voff[kPer];
    __device__ void init(int wave, int lane, int rs) {
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            int r, b;
            S::row_byte(min(wave + kFwdSharedWaves * j, S::kInst - 1), lane, r, b);
            voff[j] = static_cast<uint32_t>(r * rs * 4 + b);
        }
    }
    __device__ void copy(const float* __restrict__ head, int row0, int T, uint32_t lds, int wave,
                         int lane, int rs) const {
        const float* base = head + static_cast<size_t>(row0) * rs;
        const bool whole = row0 + kTile <= T;
        const uint32_t last = S::last(row0, T, rs);
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int i = wave + kFwdSharedWaves * j;
            if (i < S::kInst && S::active(i, lane))
                dma_dwordx4(base, lds + static_cast<uint32_t>(1024 * i),
                            whole ? voff[j] : min(voff[j], last));
        }
    }
};

template <int D>
__global__ __launch_bounds__(kWave* kFwdSharedWaves) void flash_fwd_f32_shared_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    float* __restrict__ o, float* __restrict__ m_out, float* __restrict__ l_out, int BH, int T,
    float scale, int nblk, HeadView xv, HeadView ov, int serp) {
    using L_t = FwdSharedLds<D>;
    constexpr int KS = L_t::KS, VS = L_t::VS;
    __shared__ __attribute__((aligned(1024))) L_t L;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 31;
    const int half = lane >> 5;
    int bh, blk;
    if (serp < 0)
        bf16t::map_block_grouped(blockIdx.x, BH, nblk, -serp, true, bh, blk);
    else
        bf16t::map_block(blockIdx.x, BH, nblk, true, serp != 0, bh, blk);
    const int q0 = blk * kTile * kFwdSharedWaves;
    const int qj = q0 + kTile * wave;
    const int qi = qj + col;
    const size_t xoff = wave_uniform(xv.off(bh)), ooff = wave_uniform(ov.off(bh));
    const float* kh = k + xoff;
    const float* vh = v + xoff;
    const float c = scale * kLog2e;

    SharedTileCopy<D, KS> kc;
    SharedTileCopy<D, VS> vc;
    kc.init(wave, lane, xv.row);
    vc.init(wave, lane, xv.row);
    const int ntile = (min(T, q0 + kTile * kFwdSharedWaves) + kTile - 1) / kTile;
    const uint32_t k_lds = lds_addr(&L.k[0][0]), v_lds = lds_addr(&L.v[0][0]);
    constexpr uint32_t kKBuf = kTile * KS * 4, kVBuf = kTile * VS * 4;
    auto copy_tile = [&](int t) {
        const uint32_t b = static_cast<uint32_t>(t & 1);
        kc.copy(kh, t * kTile, T, k_lds + b * kKBuf, wave, lane, xv.row);
        vc.copy(vh, t * kTile, T, v_lds + b * kVBuf, wave, lane, xv.row);
    };
    copy_tile(0);

    float qreg[D / 2];
    load_row_half<D>(qreg, q + xoff, qi, T, half, xv.row);
    f32x16 acc[D / 32];
    zero(acc);
    float m_raw = -INFINITY;  // running max of the raw scores q.k (scale > 0)
    float l_i = 0.0f;
    // this wave's last key tile (its diagonal one); none if its queries start at or past T
    const int tlast = qj < T ? qj / kTile : -1;
    for (int t = 0; t < ntile; ++t) {
        wait_vm<0>();     // this wave's copies of tile t landed ...
        __syncthreads();  // ... and every wave's; tile t-1 is no longer read by anyone
        if (t + 1 < ntile) copy_tile(t + 1);
        if (t > tlast) continue;
        const float* Ks = &L.k[t & 1][0];
        const float* Vs = &L.v[t & 1][0];
        f32x16 s = mma_rows<D>(Ks + col * KS + half * (D / 2), qreg, f32x16{});
        if (t == tlast) {  // diagonal tile
#pragma unroll
            for (int r = 0; r < 16; ++r)
                if (t * kTile + acc_row(r, half) > qi) s[r] = -INFINITY;
        }
        float mx = s[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
        mx = xhalf_max(mx);
        const float m_new = fmaxf(m_raw, mx);
        const float alpha = exp2_fast((m_raw - m_new) * c);  // 0 on the first tile
        const float mc = m_new * c;
        float rs = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            s[r] = exp2_fast(fmaf(s[r], c, -mc));
            rs += s[r];
        }
        rs = xhalf_sum(rs);
        l_i = l_i * alpha + rs;
        m_raw = m_new;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) acc[dt] *= alpha;
        mma_cols<D, VS>(Vs, col, half, s, acc);
    }
    if (qi < T) {
        store_acc_row<D>(o + ooff, qi, half, acc, 1.0f / l_i, ov.row);
        if (half == 0) {
            // max_j scale*s_j = scale * max_j s_j exactly (rounding is monotone)
            if (m_out != nullptr) m_out[static_cast<size_t>(bh) * T + qi] = m_raw * scale;
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
// Task = query block qb; wave w of the two runs key tiles [n*w/2, n*(w+1)/2) of the qb+1
// tiles with Q, dO in VGPRs and its own K/V LDS tiles; the partial dQ are summed in LDS.
// --------------------------------------------------------------------------------------
template <int D>
struct DqLds {
    static constexpr int KS = D + 4;  // K: row reads (S^T) and column reads (dQ^T)
    static constexpr int VS = D + 4;  // V: row reads (dP^T)
    float k[kTile * KS];
    float v[kTile * VS];
};

template <int D>
__device__ __forceinline__ void dq_chunk(const float* __restrict__ kh,
                                         const float* __restrict__ vh, int T, int stride,
                                         float c,
                                         float lse2, float Dval, int qb, int t0, int t1,
                                         const float (&qreg)[D / 2],
                                         const float (&doreg)[D / 2], DqLds<D>& L, int lane,
                                         Fetch& fetch, const TileCopy<D, DqLds<D>::KS>& kc,
                                         f32x16 (&acc)[D / 32]) {
    constexpr int KS = DqLds<D>::KS;
    constexpr int VS = DqLds<D>::VS;
    const float* Ks = L.k;
    const float* Vs = L.v;
    const int col = lane & 31;
    const int half = lane >> 5;
    const int qi = qb * kTile + col;
    zero(acc);
    if (t0 >= t1) {
        fetch.issue(lane);
        return;
    }
    // V before K: the V copy of a tile is always the older one in flight, so each tile
    // starts with dP (V) while the K copy issued at the end of the previous tile lands.
    kc.copy(vh, t0 * kTile, T, lds_addr(L.v), lane, stride);
    kc.copy(kh, t0 * kTile, T, lds_addr(L.k), lane, stride);
    fetch.issue(lane);

    for (int t = t0; t < t1; ++t) {
        const bool more = t + 1 < t1;
        wait_vm<kTileDma<D>>();  // V tile t landed (K tile t may still be in flight)
        f32x16 dp = mma_rows<D>(Vs + col * VS + half * (D / 2), doreg, f32x16{});
        wait_lds();
        if (more) {
            kc.copy(vh, (t + 1) * kTile, T, lds_addr(L.v), lane, stride);
            wait_vm<kTileDma<D>>();  // K tile t landed (V tile t+1 in flight)
        } else {
            wait_vm<0>();
        }
        f32x16 s = mma_rows<D>(Ks + col * KS + half * (D / 2), qreg, f32x16{});
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            float p = exp2_fast(fmaf(s[r], c, -lse2));
            if (t == qb && t * kTile + acc_row(r, half) > qi) p = 0.0f;
            s[r] = p * (dp[r] - Dval);  // dS^T (without the scale)
        }
        f32x16 part[D / 32];
        zero(part);
        mma_cols<D, KS>(Ks, col, half, s, part);
        add_into(acc, part);
        wait_lds();
        if (more) kc.copy(kh, (t + 1) * kTile, T, lds_addr(L.k), lane, stride);
    }
}

template <int D>
TCAMD_F32_KERNEL(kDqWaves) void flash_bwd_dq_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ o, const float* __restrict__ dO, const float* __restrict__ m,
    const float* __restrict__ l, float* __restrict__ dq, float* __restrict__ Dws, int BH,
    int T, float scale, int nqb, QueueSlot* slot, int per_xcd, HeadView xv, HeadView ov,
    HeadView gv) {
    __shared__ DqLds<D> L[kDqWaves];
    __shared__ unsigned s_next;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 31;
    const int half = lane >> 5;
    const float c = scale * kLog2e;
    const TaskQueue tq = TaskQueue::bind(slot, BH, nqb, per_xcd != 0);
    static_assert(DqLds<D>::KS == DqLds<D>::VS, "K and V tiles share one copy plan");
    TileCopy<D, DqLds<D>::KS> kc;
    kc.init(lane, xv.row);
    unsigned task = tq.first();
    while (task < tq.n_tasks) {
        int bh, rank;
        tq.decode(task, bh, rank);
        const int qb = nqb - 1 - rank;
        const int qi = qb * kTile + col;
        const bool row_ok = qi < T;
        const size_t xoff = wave_uniform(xv.off(bh)), ooff = wave_uniform(ov.off(bh)),
                     goff = wave_uniform(gv.off(bh));
        const size_t stat_off = static_cast<size_t>(bh) * T;
        int t0, t1;
        wave_range<kDqWaves>(qb + 1, wave, t0, t1);

        float qreg[D / 2];
        float doreg[D / 2];
        load_row_half<D>(qreg, q + xoff, qi, T, half, xv.row);
        load_row_half<D>(doreg, dO + ooff, qi, T, half, ov.row);
        // D_i from this lane's half row of O, completed across the halves.
        float Dval;
        {
            float orow[D / 2];
            load_row_half<D>(orow, o + ooff, qi, T, half, ov.row);
            float pd = 0.0f;
#pragma unroll
            for (int j = 0; j < D / 2; ++j) pd = fmaf(doreg[j], orow[j], pd);
            Dval = xhalf_sum(pd);
        }
        // P_ij = exp(scale*s - m)/l = 2^(s*c - lse2), lse2 = m*log2 e + log2 l; +inf on
        // padded rows
        const float lse2 =
            row_ok ? fmaf(m[stat_off + qi], kLog2e, __builtin_amdgcn_logf(l[stat_off + qi]))
                   : INFINITY;
        Fetch fetch{wave == 0 ? &tq : nullptr, 0u, task};
        f32x16 acc[D / 32];
        dq_chunk<D>(k + xoff, v + xoff, T, xv.row, c, lse2, Dval, qb, t0, t1, qreg, doreg,
                    L[wave], lane, fetch, kc, acc);

        // Merge: every wave publishes its partial dQ; wave w sums (in wave order) and stores
        // the 8-element chunks w, w+2, ... of the flat accumulator.
        constexpr int NP = D / 2;
        put_part(reinterpret_cast<float*>(&L[wave]), acc, lane);
        if (wave == 0 && lane == 0) s_next = fetch.value;
        __syncthreads();
#pragma unroll 1
        for (int f0 = wave * 8; f0 < NP; f0 += 8 * kDqWaves) {  // 8-element chunks, round robin
            float x[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float sum = reinterpret_cast<const float*>(&L[0])[(f0 + e) * kWave + lane];
#pragma unroll
                for (int w = 1; w < kDqWaves; ++w)
                    sum += reinterpret_cast<const float*>(&L[w])[(f0 + e) * kWave + lane];
                x[e] = sum;
            }
            if (row_ok) store_slice8<D>(dq + goff, qi, half, f0, x, scale, gv.row);
        }
        if (wave == 0 && half == 0 && row_ok) Dws[stat_off + qi] = Dval;
        __syncthreads();
        task = __builtin_amdgcn_readfirstlane(s_next);  // the same in every lane
    }
}

// --------------------------------------------------------------------------------------
// Backward stage 1 on shared tiles.  A workgroup owns 128 queries of one (b, h), wave w the
// 32 at q0 + 32w; the 32-key K and V tiles are double-buffered in LDS and shared by the four
// waves, which copy each tile together one tile ahead, with one barrier per tile.  Wave w
// runs key tiles 0 .. its diagonal tile with Q, dO in VGPRs; the per-tile products are those
// of dq_chunk (each in a fresh accumulator, added into the running sum).  No merge: each wave
// owns its queries' dQ and D.
// --------------------------------------------------------------------------------------
template <int D>
struct DqSharedLds {
    static constexpr int KS = DqLds<D>::KS;
    float k[2][kTile * KS];
    float v[2][kTile * KS];
};

template <int D>
__global__ __launch_bounds__(kWave* kFwdSharedWaves) void flash_bwd_dq_f32_shared_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ o, const float* __restrict__ dO, const float* __restrict__ m,
    const float* __restrict__ l, float* __restrict__ dq, float* __restrict__ Dws, int BH,
    int T, float scale, int nblk, HeadView xv, HeadView ov, HeadView gv, int serp) {
    using L_t = DqSharedLds<D>;
    constexpr int KS = L_t::KS;
    static_assert(DqLds<D>::KS == DqLds<D>::VS, "K and V tiles share one copy plan");
    __shared__ __attribute__((aligned(1024))) L_t L;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 31;
    const int half = lane >> 5;
    int bh, blk;
    if (serp < 0)
        bf16t::map_block_grouped(blockIdx.x, BH, nblk, -serp, true, bh, blk);
    else
        bf16t::map_block(blockIdx.x, BH, nblk, true, serp != 0, bh, blk);
    const int q0 = blk * kTile * kFwdSharedWaves;
    const int qj = q0 + kTile * wave;
    const int qi = qj + col;
    const bool row_ok = qi < T;
    const size_t xoff = wave_uniform(xv.off(bh)), ooff = wave_uniform(ov.off(bh)),
                 goff = wave_uniform(gv.off(bh));
    const size_t stat_off = static_cast<size_t>(bh) * T;
    const float* kh = k + xoff;
    const float* vh = v + xoff;
    const float c = scale * kLog2e;

    SharedTileCopy<D, KS> kc;
    kc.init(wave, lane, xv.row);
    const int ntile = (min(T, q0 + kTile * kFwdSharedWaves) + kTile - 1) / kTile;
    const uint32_t k_lds = lds_addr(&L.k[0][0]), v_lds = lds_addr(&L.v[0][0]);
    constexpr uint32_t kBuf = kTile * KS * 4;
    auto copy_tile = [&](int t) {
        const uint32_t b = static_cast<uint32_t>(t & 1) * kBuf;
        kc.copy(kh, t * kTile, T, k_lds + b, wave, lane, xv.row);
        kc.copy(vh, t * kTile, T, v_lds + b, wave, lane, xv.row);
    };
    copy_tile(0);

    float qreg[D / 2];
    float doreg[D / 2];
    load_row_half<D>(qreg, q + xoff, qi, T, half, xv.row);
    load_row_half<D>(doreg, dO + ooff, qi, T, half, ov.row);
    // D_i from this lane's half row of O, completed across the halves (the same fma chains
    // as the per-wave kernel's, so the same bits).
    float Dval;
    {
        float orow[D / 2];
        load_row_half<D>(orow, o + ooff, qi, T, half, ov.row);
        float pd = 0.0f;
#pragma unroll
        for (int j = 0; j < D / 2; ++j) pd = fmaf(doreg[j], orow[j], pd);
        Dval = xhalf_sum(pd);
    }
    // P_ij = 2^(s*c - lse2), lse2 = m*log2 e + log2 l; +inf on padded rows
    const float lse2 =
        row_ok ? fmaf(m[stat_off + qi], kLog2e, __builtin_amdgcn_logf(l[stat_off + qi]))
               : INFINITY;
    f32x16 acc[D / 32];
    zero(acc);
    // this wave's last key tile (its diagonal one); none if its queries start at or past T
    const int tlast = qj < T ? qj / kTile : -1;
    for (int t = 0; t < ntile; ++t) {
        wait_vm<0>();     // this wave's copies of tile t landed ...
        __syncthreads();  // ... and every wave's; tile t-1 is no longer read by anyone
        if (t + 1 < ntile) copy_tile(t + 1);
        if (t > tlast) continue;
        const float* Ks = &L.k[t & 1][0];
        const float* Vs = &L.v[t & 1][0];
        f32x16 dp = mma_rows<D>(Vs + col * KS + half * (D / 2), doreg, f32x16{});
        f32x16 s = mma_rows<D>(Ks + col * KS + half * (D / 2), qreg, f32x16{});
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            float p = exp2_fast(fmaf(s[r], c, -lse2));
            if (t == tlast && t * kTile + acc_row(r, half) > qi) p = 0.0f;
            s[r] = p * (dp[r] - Dval);  // dS^T (without the scale)
        }
        f32x16 part[D / 32];
        zero(part);
        mma_cols<D, KS>(Ks, col, half, s, part);
        add_into(acc, part);
    }
    if (row_ok) {
        store_acc_row<D>(dq + goff, qi, half, acc, scale, gv.row);
        if (half == 0) Dws[stat_off + qi] = Dval;
    }
}

// --------------------------------------------------------------------------------------
// Backward stage 2 (key-parallel):
//     dV_j = sum_i P_ij dO_i,   dK_j = scale * sum_i P_ij (dP_ij - D_i) q_i.
// Task = key block kb (query tiles kb .. nb-1); wave w runs query tiles kb + [n*w/4,
// n*(w+1)/4) of the n = nb - kb tiles with K, V in VGPRs and its own Q/dO/statistics LDS
// tiles; the four partial dK/dV are summed by wave 0.  Key blocks are issued lowest kb
// (most work) first.
// --------------------------------------------------------------------------------------
template <int D>
struct DkdvLds {
    static constexpr int QS = D + 4;
    static constexpr int GS = D + 4;  // dO tile
    float q[kTile * QS];
    float g[kTile * GS];
    float st[2][kTile];  // per query of the tile: lse2, D
};

template <int D, bool DS>
__device__ __forceinline__ void dkdv_chunk(const float* __restrict__ qh,
                                           const float* __restrict__ doh,
                                           const float* __restrict__ m,
                                           const float* __restrict__ l,
                                           const float* __restrict__ Dws, size_t stat_off,
                                           int T, int qstride, int gstride, float c, int kb, int t0,
                                           int t1,
                                           const float (&kreg)[D / 2],
                                           const float (&vreg)[D / 2], DkdvLds<D>& L, int lane,
                                           Fetch& fetch,
                                           const TileCopyAnyStride<D, DkdvLds<D>::QS>& tc,
                                           f32x16 (&dk_acc)[D / 32],
                                           f32x16 (&dv_acc)[D / 32], float* ds_head = nullptr,
                                           int ds_n = 0) {
    constexpr int QS = DkdvLds<D>::QS;
    constexpr int GS = DkdvLds<D>::GS;
    const float* Qs = L.q;
    const float* Gs = L.g;
    auto& St = L.st;
    const int col = lane & 31;
    const int half = lane >> 5;
    zero(dk_acc);
    zero(dv_acc);
    if (t0 >= t1) {
        fetch.issue(lane);
        return;
    }
    // Lane (col, half) fetches statistic `half` of query row0 + col: 0: lse2 = m*log2 e +
    // log2 l, so that P = 2^(s*c - lse2); 1: D.  Padded query rows get lse2 = +inf (P = 0)
    // and D = 0.
    auto load_stat = [&](int row0) -> float {
        const int r = row0 + col;
        if (r >= T) return half == 0 ? INFINITY : 0.0f;
        if (half == 0)
            return fmaf(m[stat_off + r], kLog2e, __builtin_amdgcn_logf(l[stat_off + r]));
        return Dws[stat_off + r];
    };
    St[half][col] = load_stat(t0 * kTile);
    tc.copy(qh, t0 * kTile, T, lds_addr(L.q), lane, qstride);
    tc.copy(doh, t0 * kTile, T, lds_addr(L.g), lane, gstride);
    fetch.issue(lane);

    for (int t = t0; t < t1; ++t) {
        const bool more = t + 1 < t1;
        wait_vm<0>();  // Q and dO tiles t landed
        const float st_n = more ? load_stat((t + 1) * kTile) : 0.0f;
        f32x16 s = mma_rows<D>(Qs + col * QS + half * (D / 2), kreg, f32x16{});
        f32x16 dp = mma_rows<D>(Gs + col * GS + half * (D / 2), vreg, f32x16{});
        f32x16 ds;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int qr = acc_row(r, half);
            float p = exp2_fast(fmaf(s[r], c, -St[0][qr]));
            if (t == kb && qr < col) p = 0.0f;  // diagonal tile: query < key
            s[r] = p;
            ds[r] = p * (dp[r] - St[1][qr]);
        }
        if constexpr (DS) {
            // dS tile (t, kb) of the head (ds_tile): row acc_row(r, half), column col; a 32-lane
            // store covers one query's 32 keys (128 bytes).  Keys past T get zeros.
            const int kj = kb * kTile + col;
            float* tile = ds_head + ds_tile(0, ds_n, t, kb);
            const uint32_t loff = static_cast<uint32_t>(4 * half * kTile + col);
#pragma unroll
            for (int r = 0; r < 16; ++r)
                tile[(8 * (r / 4) + r % 4) * kTile + loff] = kj < T ? ds[r] : 0.0f;
        }
        f32x16 part[D / 32];
        zero(part);
        mma_cols<D, GS>(Gs, col, half, s, part);
        add_into(dv_acc, part);
        zero(part);
        mma_cols<D, QS>(Qs, col, half, ds, part);
        add_into(dk_acc, part);
        wait_lds();
        if (more) {
            St[half][col] = st_n;
            tc.copy(qh, (t + 1) * kTile, T, lds_addr(L.q), lane, qstride);
            tc.copy(doh, (t + 1) * kTile, T, lds_addr(L.g), lane, gstride);
        }
    }
}

// DS: dS written out as well (the tiles of ds_tile at or below the diagonal, ds_n = T
// rounded up to 32), for the dQ-from-dS kernel below.
template <int D, bool DS>
TCAMD_F32_KERNEL(kDkdvWaves) void flash_bwd_dkdv_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ dO, const float* __restrict__ m, const float* __restrict__ l,
    const float* __restrict__ Dws, float* __restrict__ dk, float* __restrict__ dv, int BH,
    int T, float scale, int nkb, QueueSlot* slot, int per_xcd, HeadView xv, HeadView ov,
    HeadView gv, float* __restrict__ ds, int ds_n) {
    __shared__ DkdvLds<D> L[kDkdvWaves];
    __shared__ unsigned s_next;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 31;
    const int half = lane >> 5;
    const float c = scale * kLog2e;
    const TaskQueue tq = TaskQueue::bind(slot, BH, nkb, per_xcd != 0);
    static_assert(DkdvLds<D>::QS == DkdvLds<D>::GS, "Q and dO tiles share one copy plan");
    TileCopyAnyStride<D, DkdvLds<D>::QS> tc;
    tc.init(lane);
    unsigned task = tq.first();
    while (task < tq.n_tasks) {
        int bh, kb;
        tq.decode(task, bh, kb);
        const int kj = kb * kTile + col;
        const size_t xoff = wave_uniform(xv.off(bh)), ooff = wave_uniform(ov.off(bh)),
                     goff = wave_uniform(gv.off(bh));
        const size_t stat_off = static_cast<size_t>(bh) * T;
        int t0, t1;
        wave_range<kDkdvWaves>(nkb - kb, wave, t0, t1);

        float kreg[D / 2];
        float vreg[D / 2];
        load_row_half<D>(kreg, k + xoff, kj, T, half, xv.row);
        load_row_half<D>(vreg, v + xoff, kj, T, half, xv.row);
        Fetch fetch{wave == 0 ? &tq : nullptr, 0u, task};
        f32x16 dk_acc[D / 32], dv_acc[D / 32];
        float* ds_head = nullptr;
        if constexpr (DS) ds_head = ds + static_cast<size_t>(bh) * ds_n * ds_n;
        dkdv_chunk<D, DS>(q + xoff, dO + ooff, m, l, Dws, stat_off, T, xv.row, ov.row, c, kb,
                          kb + t0, kb + t1, kreg, vreg, L[wave], lane, fetch, tc, dk_acc, dv_acc,
                          ds_head, ds_n);

        // Merge: every wave publishes its partial dK, dV; wave w sums (in wave order) and
        // stores the 8-element chunks w, w+4, ... of the concatenated (dK, dV) accumulators.
        constexpr int NP = D;  // D/2 floats of dK then D/2 of dV per lane
        float* part = reinterpret_cast<float*>(&L[wave]);
        put_part(part, dk_acc, lane);
        put_part(part + D * 32, dv_acc, lane);
        if (wave == 0 && lane == 0) s_next = fetch.value;
        __syncthreads();
#pragma unroll 1
        for (int f0 = wave * 8; f0 < NP; f0 += 8 * kDkdvWaves) {  // 8-element chunks, round robin
            float x[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float sum = reinterpret_cast<const float*>(&L[0])[(f0 + e) * kWave + lane];
#pragma unroll
                for (int w = 1; w < kDkdvWaves; ++w)
                    sum += reinterpret_cast<const float*>(&L[w])[(f0 + e) * kWave + lane];
                x[e] = sum;
            }
            if (kj < T) {
                if (f0 < D / 2) {
                    store_slice8<D>(dk + goff, kj, half, f0, x, scale, gv.row);
                } else {
                    store_slice8<D>(dv + goff, kj, half, f0 - D / 2, x, 1.0f, gv.row);
                }
            }
        }
        __syncthreads();
        task = __builtin_amdgcn_readfirstlane(s_next);  // the same in every lane
    }
}

// --------------------------------------------------------------------------------------
// dK/dV on shared tiles.  A workgroup owns 128 keys of one (b, h), wave w the 32 at
// k0 + 32w; the 32-query Q and dO tiles are double-buffered in LDS and shared by the four
// waves, which copy each tile together one tile ahead, with one barrier per tile.  Wave w
// starts at its diagonal tile (t0 + w) and runs to the last; the per-tile products are those
// of dkdv_chunk (each in a fresh accumulator, added into the running sums), the statistics
// of a tile staged in LDS by wave 0.  No merge: each wave owns its keys' dK and dV.
// --------------------------------------------------------------------------------------
template <int D>
struct DkdvSharedLds {
    static constexpr int QS = DkdvLds<D>::QS;
    float q[2][kTile * QS];
    float g[2][kTile * QS];
    float st[2][2][kTile];  // [buffer][lse2, D][query of the tile]
};

template <int D, bool DS>
__global__ __launch_bounds__(kWave* kFwdSharedWaves) void flash_bwd_dkdv_f32_shared_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ dO, const float* __restrict__ m, const float* __restrict__ l,
    const float* __restrict__ Dws, float* __restrict__ dk, float* __restrict__ dv, int BH,
    int T, float scale, int nblk, HeadView xv, HeadView ov, HeadView gv,
    float* __restrict__ ds, int ds_n, int serp) {
    using L_t = DkdvSharedLds<D>;
    constexpr int QS = L_t::QS;
    __shared__ __attribute__((aligned(1024))) L_t L;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 31;
    const int half = lane >> 5;
    int bh, blk;
    bf16t::map_block(blockIdx.x, BH, nblk, false, serp != 0, bh, blk);  // block 0: every query
    const int k0 = blk * kTile * kFwdSharedWaves;
    const int kw = k0 + kTile * wave;
    const int kj = kw + col;
    const size_t xoff = wave_uniform(xv.off(bh)), ooff = wave_uniform(ov.off(bh)),
                 goff = wave_uniform(gv.off(bh));
    const size_t stat_off = static_cast<size_t>(bh) * T;
    const float* qh = q + xoff;
    const float* gh = dO + ooff;
    const float c = scale * kLog2e;

    SharedTileCopy<D, QS> qc, gc;
    qc.init(wave, lane, xv.row);
    gc.init(wave, lane, ov.row);
    const int t0 = k0 / kTile;
    const int ntile = (T + kTile - 1) / kTile;
    const uint32_t q_lds = lds_addr(&L.q[0][0]), g_lds = lds_addr(&L.g[0][0]);
    constexpr uint32_t kBuf = kTile * QS * 4;
    auto copy_tile = [&](int t) {
        const uint32_t b = static_cast<uint32_t>(t & 1) * kBuf;
        qc.copy(qh, t * kTile, T, q_lds + b, wave, lane, xv.row);
        gc.copy(gh, t * kTile, T, g_lds + b, wave, lane, ov.row);
    };
    // Lane (col, half) of wave 0: statistic `half` of query row0 + col: 0: lse2 = m*log2 e +
    // log2 l, so that P = 2^(s*c - lse2); 1: D.  Padded query rows: lse2 = +inf (P = 0), D = 0.
    auto load_stat = [&](int row0) -> float {
        const int r = row0 + col;
        if (r >= T) return half == 0 ? INFINITY : 0.0f;
        if (half == 0)
            return fmaf(m[stat_off + r], kLog2e, __builtin_amdgcn_logf(l[stat_off + r]));
        return Dws[stat_off + r];
    };
    if (wave == 0) L.st[t0 & 1][half][col] = load_stat(t0 * kTile);
    copy_tile(t0);

    float kreg[D / 2], vreg[D / 2];
    load_row_half<D>(kreg, k + xoff, kj, T, half, xv.row);
    load_row_half<D>(vreg, v + xoff, kj, T, half, xv.row);
    f32x16 dk_acc[D / 32], dv_acc[D / 32];
    zero(dk_acc);
    zero(dv_acc);
    float* ds_head = nullptr;
    if constexpr (DS) ds_head = ds + static_cast<size_t>(bh) * ds_n * ds_n;
    // this wave's first query tile (its diagonal one); none if its keys start at or past T
    const int tw = kw < T ? kw / kTile : ntile;
    for (int t = t0; t < ntile; ++t) {
        const bool more = t + 1 < ntile;
        wait_vm<0>();     // this wave's copies (and statistics) of tile t landed ...
        __syncthreads();  // ... and every wave's; tile t-1 is no longer read by anyone
        float st_n = 0.0f;
        if (more) {
            if (wave == 0) st_n = load_stat((t + 1) * kTile);
            copy_tile(t + 1);
        }
        if (t >= tw) {
            const float* Qs = &L.q[t & 1][0];
            const float* Gs = &L.g[t & 1][0];
            const float* St0 = &L.st[t & 1][0][0];
            const float* St1 = &L.st[t & 1][1][0];
            f32x16 s = mma_rows<D>(Qs + col * QS + half * (D / 2), kreg, f32x16{});
            f32x16 dp = mma_rows<D>(Gs + col * QS + half * (D / 2), vreg, f32x16{});
            f32x16 dsv;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int qr = acc_row(r, half);
                float p = exp2_fast(fmaf(s[r], c, -St0[qr]));
                if (t == tw && qr < col) p = 0.0f;  // diagonal tile: query < key
                s[r] = p;
                dsv[r] = p * (dp[r] - St1[qr]);
            }
            if constexpr (DS) {
                // dS tile (t, kw/32) of the head (ds_tile): row acc_row(r, half), column col; a
                // 32-lane store covers one query's 32 keys (128 bytes).  Keys past T get zeros.
                float* tile = ds_head + ds_tile(0, ds_n, t, kw / kTile);
                const uint32_t loff = static_cast<uint32_t>(4 * half * kTile + col);
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    tile[(8 * (r / 4) + r % 4) * kTile + loff] = kj < T ? dsv[r] : 0.0f;
            }
            f32x16 part[D / 32];
            zero(part);
            mma_cols<D, QS>(Gs, col, half, s, part);
            add_into(dv_acc, part);
            zero(part);
            mma_cols<D, QS>(Qs, col, half, dsv, part);
            add_into(dk_acc, part);
        }
        if (more && wave == 0) L.st[(t + 1) & 1][half][col] = st_n;
    }
    if (kj < T) {
        store_acc_row<D>(dk + goff, kj, half, dk_acc, scale, gv.row);
        store_acc_row<D>(dv + goff, kj, half, dv_acc, 1.0f, gv.row);
    }
}

// --------------------------------------------------------------------------------------
// The dS-first backward order: D first (the dQ kernel's sums, alone), then dK/dV writing dS
// (DS = true above), then dQ = scale * dS K from the stored dS, whose products (one of the
// dQ kernel's three) are then all that dQ costs.
// --------------------------------------------------------------------------------------

// D = rowsum(dO o O): two lanes per row, lane `half` an fma chain over elements
// half*D/2 .. in order, the two halves added: the dQ kernel's D, bitwise.  nrows = B*H*T.
template <int D>
__global__ __launch_bounds__(256) void d_rows_f32_kernel(const float* __restrict__ dO,
                                                         const float* __restrict__ O,
                                                         HeadView ov, float* __restrict__ Dws,
                                                         int nrows, int T) {
    const int gid = blockIdx.x * 256 + threadIdx.x;
    const int row = gid >> 1;
    const int half = gid & 1;
    float pd = 0.0f;
    if (row < nrows) {
        const int bh = row / T;
        const int t = row - bh * T;
        const size_t off = ov.off(bh) + static_cast<size_t>(t) * ov.row + half * (D / 2);
#pragma unroll
        for (int j = 0; j < D / 2; j += 4) {
            const f32x4 a = *reinterpret_cast<const f32x4*>(dO + off + j);
            const f32x4 b = *reinterpret_cast<const f32x4*>(O + off + j);
#pragma unroll
            for (int e = 0; e < 4; ++e) pd = fmaf(a[e], b[e], pd);
        }
    }
    const float sum = pd + __shfl_xor(pd, 1);
    if (row < nrows && half == 0) Dws[row] = sum;
}

// dQ^T += K^T dS^T over 32-key tiles: 128 queries per workgroup, one 32-query sub-block per
// wave, on v_mfma_f32_32x32x2_f32 with the backward kernels' two-level summation (each
// tile's products in a fresh accumulator).  K tiles (fp32 rows, bank-conflict-free stride)
// stream through LDS in three buffers, two tiles ahead, the copy instructions of a tile
// shared out over the four waves; each wave copies its 32 queries' dS rows of a tile (32 keys,
// 128 bytes each, 8 lanes per row) into its own LDS slot (two slots), two tiles ahead, and a
// lane reads back the 16 keys of its query that its accumulator-layout B operand holds (four
// runs of 4, XOR-swizzled so that the reads are conflict-free).  Key tiles past a wave's
// diagonal are skipped (dS is not written there); the diagonal tile holds the zeros of the
// causal mask.  The copies retire in issue order: a step waits for tile kt's K copies
// before the barrier and for its own dS copies after it.
template <int D>
__global__ __launch_bounds__(kWave * 4) void flash_bwd_dq_ds_f32_kernel(
    const float* __restrict__ k, HeadView kv, const float* __restrict__ ds, int ds_n,
    float* __restrict__ dq, HeadView gv, int BH, int T, float scale, int nblk) {
    constexpr int kWv = 4;                 // waves per workgroup
    constexpr int KS = D + 4;              // K row stride in LDS (floats)
    using Sh = TileShape<D, KS>;
    constexpr int NB = 3;                  // K buffers
    constexpr int kLoads = 4;              // dS copies per wave and tile: 32 rows x 128 bytes
    constexpr uint32_t kSlot = kLoads * 1024;
    __shared__ __attribute__((aligned(16))) float smk[NB][kTile * KS];
    __shared__ __attribute__((aligned(1024))) float sms[kWv][2][kLoads * 256];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 31;
    const int half = lane >> 5;
    // heaviest query block first; every block of a head on one XCD when BH % 8 == 0
    int bh, rank;
    if ((BH & 7) == 0) {
        const int hpx = BH >> 3;
        const int slot = blockIdx.x >> 3;
        bh = (blockIdx.x & 7) * hpx + slot % hpx;
        rank = slot / hpx;
    } else {
        bh = blockIdx.x % BH;
        rank = blockIdx.x / BH;
    }
    const int q0 = (nblk - 1 - rank) * kWv * kTile;
    const int qj = q0 + kTile * wave;
    const float* kh = k + kv.off(bh);
    const int krs = kv.row;
    // K tile copies: instruction i of a tile is issued by wave i % 4
    uint32_t voff[Sh::kInst];
#pragma unroll
    for (int i = 0; i < Sh::kInst; ++i) {
        int r, b;
        Sh::row_byte(i, lane, r, b);
        voff[i] = static_cast<uint32_t>(r * krs * 4 + b);
    }
    int ncopy = 0;
#pragma unroll
    for (int i = 0; i < Sh::kInst; ++i) ncopy += i % kWv == wave ? 1 : 0;
    constexpr int kMaxCopy = (Sh::kInst + kWv - 1) / kWv;  // ncopy of wave 0
    static_assert(2 * kLoads + kMaxCopy <= 15 && kLoads + 2 * kMaxCopy <= 15,
                  "wait_vm_at_most's counts");
    auto copy_tile = [&](int kt, uint32_t buf) {
        const int row0 = kt * kTile;
        const float* base = kh + static_cast<size_t>(row0) * krs;
        const bool whole = row0 + kTile <= T;
        const uint32_t last = Sh::last(row0, T, krs);
#pragma unroll
        for (int i = 0; i < Sh::kInst; ++i)
            if (i % kWv == wave && Sh::active(i, lane))
                dma_dwordx4(base, buf + static_cast<uint32_t>(1024 * i),
                            whole ? voff[i] : min(voff[i], last));
    };
    const int kend = min(T, q0 + kWv * kTile);
    const int ntile = (kend + kTile - 1) / kTile;
    // key tiles 0 .. qj/32 (the last one the diagonal); none when the wave's queries start past
    // T.  Rows qj + col < ds_n when qj < T.
    const int nmine = qj < T ? min(qj / kTile + 1, ntile) : 0;
    const float* sbase = ds + ds_tile(bh, ds_n, min(qj, ds_n - kTile) / kTile, 0);
    // A slot holds the tile's 32 query rows of 32 keys; 16-byte chunk c of row r at
    // r*128 + 16*(c ^ ((r/2) % 8)).  Copy j: lane i fills slot bytes 1024j + 16i, row 8j + i/8
    // (one contiguous 1 KB of the tile).
    uint32_t soff[kLoads];
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
        const int r = 8 * j + lane / 8;
        const int c = (lane % 8) ^ ((r >> 1) & 7);
        soff[j] = static_cast<uint32_t>((r * kTile + 4 * c) * 4);
    }
    const uint32_t s_lds = lds_addr(sms[wave][0]);
    auto copy_ds = [&](int kt) {
        const float* b = sbase + static_cast<size_t>(kt) * 1024;  // tile (qj/32, kt)
#pragma unroll
        for (int j = 0; j < kLoads; ++j)
            dma_dwordx4(b, s_lds + static_cast<uint32_t>(kt & 1) * kSlot + 1024 * j, soff[j]);
    };
    copy_tile(0, lds_addr(smk[0]));
    if (0 < nmine) copy_ds(0);
    if (1 < ntile) copy_tile(1, lds_addr(smk[1]));
    if (1 < nmine) copy_ds(1);
    f32x16 acc[D / 32];
    zero(acc);
    // Every wave issues kMaxCopy copies per K tile when the tile's copy instructions divide
    // evenly among the waves.  STEADY: kt + 2 < nmine (the wave has two more tiles of its own,
    // and nmine <= ntile), so the copies in flight, and the waits, are constants; the steps
    // before the last two of the wave's own run in a loop of their own, without the general
    // case's branches.
    constexpr bool kEven = Sh::kInst % kWv == 0;
    auto step = [&](int kt, auto steady_c) {
        constexpr bool steady = decltype(steady_c)::value && kEven;
        // this wave's copies of K tile kt landed: outstanding may be only its dS of tile kt
        // and tile kt+1's copies ...
        if constexpr (steady)
            wait_vm<2 * kLoads + kMaxCopy>();
        else
            wait_vm_at_most((kt < nmine ? kLoads : 0) + (kt + 1 < ntile ? ncopy : 0) +
                            (kt + 1 < nmine ? kLoads : 0));
        __syncthreads();  // ... and every wave's; tile kt-1's buffer is no longer read
        if (steady || kt + 2 < ntile) copy_tile(kt + 2, lds_addr(smk[(kt + 2) % NB]));
        if (!steady && kt >= nmine) return;
        // dS of tile kt landed: outstanding may be only tile kt+1's and K tile kt+2's copies
        if constexpr (steady)
            wait_vm<kLoads + 2 * kMaxCopy>();
        else
            wait_vm_at_most((kt + 1 < ntile ? ncopy : 0) + (kt + 1 < nmine ? kLoads : 0) +
                            (kt + 2 < ntile ? ncopy : 0));
        // B operand in accumulator layout: element r = key acc_row(r, half) = 8(r/4) +
        // 4 half + r%4 of this lane's query: run j = r/4, chunk 2j + half of the row
        f32x16 sb;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const f32x4 x = *(TCAMD_LDS const f32x4*)(uintptr_t)(
                s_lds + static_cast<uint32_t>(kt & 1) * kSlot + 128 * col +
                16 * ((2 * j + half) ^ ((col >> 1) & 7)));
#pragma unroll
            for (int e = 0; e < 4; ++e) sb[4 * j + e] = x[e];
        }
        if (steady || kt + 2 < nmine) {
            wait_lds();  // the slot's reads are done before the copy into it starts
            copy_ds(kt + 2);
        }
        f32x16 part[D / 32];
        zero(part);
        mma_cols<D, KS>(smk[kt % NB], col, half, sb, part);
        add_into(acc, part);
    };
    int kt = 0;
    for (; kt + 2 < nmine; ++kt) step(kt, std::true_type{});
    for (; kt < ntile; ++kt) step(kt, std::false_type{});
    const int qi = qj + col;
    if (qi < T) store_acc_row<D>(dq + gv.off(bh), qi, half, acc, scale, gv.row);
}

__device__ QueueSlot g_fwd_queue[kQueueSlots];
__device__ QueueSlot g_dq_queue[kQueueSlots];
__device__ QueueSlot g_dkdv_queue[kQueueSlots];
std::atomic<unsigned> g_fwd_ticket{0};
std::atomic<unsigned> g_dq_ticket{0};
std::atomic<unsigned> g_dkdv_ticket{0};

// Device address of a queue array on the current device (the host-side name of a
// __device__ array is not a device address).
enum class Family { Fwd = 0, Dq = 1, Dkdv = 2 };
QueueSlot* queue_base(Family f) {
    constexpr int kMaxDev = 64;
    static std::atomic<QueueSlot*> cache[3][kMaxDev] = {};
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (dev < 0 || dev >= kMaxDev) dev = 0;
    QueueSlot* p = cache[static_cast<int>(f)][dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        void* addr = nullptr;
        hipError_t e = hipErrorInvalidSymbol;
        switch (f) {
            case Family::Fwd: e = hipGetSymbolAddress(&addr, HIP_SYMBOL(g_fwd_queue)); break;
            case Family::Dq: e = hipGetSymbolAddress(&addr, HIP_SYMBOL(g_dq_queue)); break;
            case Family::Dkdv: e = hipGetSymbolAddress(&addr, HIP_SYMBOL(g_dkdv_queue)); break;
        }
        if (e != hipSuccess) return nullptr;
        p = static_cast<QueueSlot*>(addr);
        cache[static_cast<int>(f)][dev].store(p, std::memory_order_release);
    }
    return p;
}

// The queue slot of a launch of family f on `stream`: null (static schedule) under graph
// capture.  Sets `ok` to false if the queue array's address cannot be found; the caller
// then launches nothing and the C ABI reports a launch error.
QueueSlot* launch_slot(Family f, std::atomic<unsigned>& ticket, hipStream_t stream, bool& ok) {
    ok = true;
    if (stream_is_capturing(stream)) return nullptr;
    QueueSlot* base = queue_base(f);
    if (base == nullptr) {
        ok = false;
        note_launch_failure();
        return nullptr;
    }
    return base + next_queue_slot(ticket);
}

// The forward on shared tiles (flash_fwd_f32_shared_kernel) where it is the faster one, else
// the persistent per-wave kernel.  Measured forward (one process, us, per-wave -> shared):
// d = 64: B16 H12 T512 92 -> 79, B8 H12 T1024 142 -> 134, B8 H16 T2048 623 -> 562,
// B4 H12 T2048 237 -> 239, B2 H12 T4096 439 -> 464, B1 H12 T8192 886 -> 1086 (its static
// block order balances long causal ranges worse than the persistent queue); d = 128:
// B8 H12 T1024 314 -> 249, B2 H16 T2048 355 -> 299, B1 H16 T8192 2443 -> 2349; d = 32:
// B8 H12 T1024 72 -> 74.
bool fwd_on_shared_tiles(int D, int T) { return D == 128 || (D == 64 && T <= 2048); }
constexpr bool kDkdvShared = true;
// The dQ stage on shared tiles under the same rule; measured dQ (us, per-wave -> shared):
// d = 64: B8 H12 T1024 197 -> 196, B16 H12 T512 123 -> 117, B4 H12 T2048 355 -> 345,
// B8 H16 T2048 861 -> 876; d = 128: B2 H16 T2048 484 -> 454, B8 H12 T1024 390 -> 386.
constexpr bool kDqShared = true;

template <int D>
void fwd_dispatch(const float* q, const float* k, const float* v, float* o, float* m_out,
                  float* l_out, int BH, int T, float scale, const HeadView& xv,
                  const HeadView& ov, hipStream_t stream) {
    if (fwd_on_shared_tiles(D, T)) {
        constexpr int kBlock = kTile * kFwdSharedWaves;
        const int nblk = (T + kBlock - 1) / kBlock;
        const auto kernel = flash_fwd_f32_shared_kernel<D>;
        const int res = resident_capacity(kernel, kWave * kFwdSharedWaves, 0);
        const int serp = BH * nblk <= res ? 1 : -head_group(BH, nblk, res);
        hipLaunchKernelGGL(kernel, dim3(BH * nblk), dim3(kWave * kFwdSharedWaves), 0, stream, q,
                           k, v, o, m_out, l_out, BH, T, scale, nblk, xv, ov, serp);
        return;
    }
    const int nqb = (T + kTile - 1) / kTile;
    bool ok = true;
    QueueSlot* slot = launch_slot(Family::Fwd, g_fwd_ticket, stream, ok);
    if (!ok) return;
    const int grid = persistent_grid(flash_fwd_f32_kernel<D>, kWave * kFwdWaves, 0,
                                     static_cast<long long>(BH) * nqb);
    hipLaunchKernelGGL(flash_fwd_f32_kernel<D>, dim3(grid), dim3(kWave * kFwdWaves), 0, stream, q, k, v, o,
                       m_out, l_out, BH, T, scale, nqb, slot, (BH % kXcds) == 0 ? 1 : 0, xv, ov);
}

template <int D>
void dq_dispatch(const float* q, const float* k, const float* v, const float* o,
                 const float* dO, const float* m, const float* l, float* dq, float* Dws, int BH,
                 int T, float scale, const HeadView& xv, const HeadView& ov, const HeadView& gv,
                 hipStream_t stream) {
    if (kDqShared && fwd_on_shared_tiles(D, T)) {
        constexpr int kBlock = kTile * kFwdSharedWaves;
        const int nblk = (T + kBlock - 1) / kBlock;
        const auto kernel = flash_bwd_dq_f32_shared_kernel<D>;
        const int res = resident_capacity(kernel, kWave * kFwdSharedWaves, 0);
        const int serp = BH * nblk <= res ? 1 : -head_group(BH, nblk, res);
        hipLaunchKernelGGL(kernel, dim3(BH * nblk), dim3(kWave * kFwdSharedWaves), 0, stream, q,
                           k, v, o, dO, m, l, dq, Dws, BH, T, scale, nblk, xv, ov, gv, serp);
        return;
    }
    const int nqb = (T + kTile - 1) / kTile;
    bool ok = true;
    QueueSlot* slot = launch_slot(Family::Dq, g_dq_ticket, stream, ok);
    if (!ok) return;
    const int grid = persistent_grid(flash_bwd_dq_f32_kernel<D>, kWave * kDqWaves, 0,
                                     static_cast<long long>(BH) * nqb);
    hipLaunchKernelGGL(flash_bwd_dq_f32_kernel<D>, dim3(grid), dim3(kWave * kDqWaves), 0, stream, q, k, v,
                       o, dO, m, l, dq, Dws, BH, T, scale, nqb, slot,
                       (BH % kXcds) == 0 ? 1 : 0, xv, ov, gv);
}

template <int D, bool DS>
void dkdv_launch(const float* q, const float* k, const float* v, const float* dO,
                 const float* m, const float* l, const float* Dws, float* dk, float* dv, int BH,
                 int T, float scale, const HeadView& xv, const HeadView& ov, const HeadView& gv,
                 float* ds, hipStream_t stream) {
    if (kDkdvShared && fwd_on_shared_tiles(D, T)) {
        constexpr int kBlock = kTile * kFwdSharedWaves;
        const int nblk = (T + kBlock - 1) / kBlock;
        const auto kernel = flash_bwd_dkdv_f32_shared_kernel<D, DS>;
        const int serp = BH * nblk <= resident_capacity(kernel, kWave * kFwdSharedWaves, 0);
        hipLaunchKernelGGL(kernel, dim3(BH * nblk), dim3(kWave * kFwdSharedWaves), 0, stream, q,
                           k, v, dO, m, l, Dws, dk, dv, BH, T, scale, nblk, xv, ov, gv, ds,
                           ds_rows(T), serp);
        return;
    }
    const int nkb = (T + kTile - 1) / kTile;
    bool ok = true;
    QueueSlot* slot = launch_slot(Family::Dkdv, g_dkdv_ticket, stream, ok);
    if (!ok) return;
    const int grid = persistent_grid(flash_bwd_dkdv_f32_kernel<D, DS>, kWave * kDkdvWaves, 0,
                                     static_cast<long long>(BH) * nkb);
    hipLaunchKernelGGL((flash_bwd_dkdv_f32_kernel<D, DS>), dim3(grid), dim3(kWave * kDkdvWaves), 0,
                       stream, q, k, v, dO, m, l, Dws, dk, dv, BH, T, scale, nkb, slot,
                       (BH % kXcds) == 0 ? 1 : 0, xv, ov, gv, ds, ds_rows(T));
}

template <int D>
void dkdv_dispatch(const float* q, const float* k, const float* v, const float* dO,
                   const float* m, const float* l, const float* Dws, float* dk, float* dv,
                   int BH, int T, float scale, const HeadView& xv, const HeadView& ov,
                   const HeadView& gv, float* ds, hipStream_t stream) {
    if (ds != nullptr)
        dkdv_launch<D, true>(q, k, v, dO, m, l, Dws, dk, dv, BH, T, scale, xv, ov, gv, ds, stream);
    else
        dkdv_launch<D, false>(q, k, v, dO, m, l, Dws, dk, dv, BH, T, scale, xv, ov, gv, ds,
                              stream);
}

}  // namespace

void launch_flash_fwd_f32(const float* q, const float* k, const float* v, float* o,
                          float* m_out, float* l_out, int BH, int T, int d, float scale,
                          const HeadView& xv, const HeadView& ov, hipStream_t stream) {
    switch (d) {
        case 32: fwd_dispatch<32>(q, k, v, o, m_out, l_out, BH, T, scale, xv, ov, stream); break;
        case 64: fwd_dispatch<64>(q, k, v, o, m_out, l_out, BH, T, scale, xv, ov, stream); break;
        default: fwd_dispatch<128>(q, k, v, o, m_out, l_out, BH, T, scale, xv, ov, stream); break;
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
                             float* Dws, int BH, int T, int d, float scale, const HeadView& xv,
                             const HeadView& ov, const HeadView& gv, hipStream_t stream) {
    switch (d) {
        case 32: dq_dispatch<32>(q, k, v, o, dO, m, l, dq, Dws, BH, T, scale, xv, ov, gv, stream); break;
        case 64: dq_dispatch<64>(q, k, v, o, dO, m, l, dq, Dws, BH, T, scale, xv, ov, gv, stream); break;
        default: dq_dispatch<128>(q, k, v, o, dO, m, l, dq, Dws, BH, T, scale, xv, ov, gv, stream); break;
    }
}

void launch_flash_bwd_dkdv_f32(const float* q, const float* k, const float* v,
                               const float* dO, const float* m, const float* l,
                               const float* Dws, float* dk, float* dv, int BH, int T, int d,
                               float scale, const HeadView& xv, const HeadView& ov,
                               const HeadView& gv, hipStream_t stream, float* ds) {
    switch (d) {
        case 32: dkdv_dispatch<32>(q, k, v, dO, m, l, Dws, dk, dv, BH, T, scale, xv, ov, gv, ds, stream); break;
        case 64: dkdv_dispatch<64>(q, k, v, dO, m, l, Dws, dk, dv, BH, T, scale, xv, ov, gv, ds, stream); break;
        default: dkdv_dispatch<128>(q, k, v, dO, m, l, Dws, dk, dv, BH, T, scale, xv, ov, gv, ds, stream); break;
    }
}

void launch_bwd_d_rows_f32(const float* dO, const float* O, const HeadView& ov, float* Dws,
                           int BH, int T, int d, hipStream_t stream) {
    const int nrows = BH * T;
    const unsigned blocks = static_cast<unsigned>((2LL * nrows + 255) / 256);
    switch (d) {
        case 32: hipLaunchKernelGGL((d_rows_f32_kernel<32>), dim3(blocks), dim3(256), 0, stream, dO, O, ov, Dws, nrows, T); break;
        case 64: hipLaunchKernelGGL((d_rows_f32_kernel<64>), dim3(blocks), dim3(256), 0, stream, dO, O, ov, Dws, nrows, T); break;
        default: hipLaunchKernelGGL((d_rows_f32_kernel<128>), dim3(blocks), dim3(256), 0, stream, dO, O, ov, Dws, nrows, T); break;
    }
}

void launch_flash_bwd_dq_ds_f32(const float* k, const HeadView& kv, const float* ds, float* dq,
                                const HeadView& gv, int BH, int T, int d, float scale,
                                hipStream_t stream) {
    constexpr int kBlock = 4 * kTile;
    const int nblk = (T + kBlock - 1) / kBlock;
    const dim3 grid(BH * nblk), block(kWave * 4);
    const int n = ds_rows(T);
    switch (d) {
        case 32: hipLaunchKernelGGL((flash_bwd_dq_ds_f32_kernel<32>), grid, block, 0, stream, k, kv, ds, n, dq, gv, BH, T, scale, nblk); break;
        case 64: hipLaunchKernelGGL((flash_bwd_dq_ds_f32_kernel<64>), grid, block, 0, stream, k, kv, ds, n, dq, gv, BH, T, scale, nblk); break;
        default: hipLaunchKernelGGL((flash_bwd_dq_ds_f32_kernel<128>), grid, block, 0, stream, k, kv, ds, n, dq, gv, BH, T, scale, nblk); break;
    }
}

}  // namespace tcamd
