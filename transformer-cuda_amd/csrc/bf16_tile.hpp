// bf16_tile.hpp - LDS tiles and MFMA operand helpers shared by the bf16 attention kernels.
//
// A K/V/Q/dO tile is 64 rows (sequence positions) x D bf16, copied HBM -> LDS with
// global_load_lds_dwordx4 into rows whose 16-byte chunks are XOR-swizzled by row:
//   * 16-byte reads of one chunk index by 32 lanes on 32 rows (the A operand of a product
//     that contracts over the head dimension) hit distinct banks;
//   * ds_read_tr16_b64, which hands lane i of a 16-lane group element i%4 of the 8-byte
//     read of lane 4e + i/4 (e = 0..3), turns a row-major tile into the A operand of a
//     product that contracts over the sequence: two reads 8 rows apart give a lane the
//     positions 16u + 4g + {0..3} and 16u + 8 + 4g + {0..3} of one head dimension,
//     exactly the k-slots of the B operand packed from a 32x32 accumulator (pack_b).
#pragma once

#include <math.h>

#include "device_common.hpp"
#include "lds_dma.hpp"

namespace tcamd {
namespace bf16t {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kWaves = 4;      // waves per workgroup, one per SIMD of a CU
constexpr int kSub = 32;       // rows per sub-block (MFMA width)
constexpr int kRowTile = 64;   // sequence rows per LDS tile

typedef short s16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// A 64-row x D bf16 tile in LDS.  Rows are grouped in blocks of 8; row r, 16-byte chunk c
// is at byte (r/8)*B + (r%8)*2D + 16*(c ^ swz(r)), where B = 8 rows + kPad bytes.
//   * d = 64 (a row is half a 256-byte bank line): swz(r) = 2*(r%4) + (r/4)%2 gives the 8
//     rows of a block 8 distinct chunk slots, and the 4 rows x 2 chunks that a 16-lane group
//     of a transposing read touches (rows inside one block) 8 distinct slots; consecutive
//     rows sit on alternate halves of the bank line.
//   * d = 128 (a row is a whole bank line, so every row of a block starts on bank 0): with
//     i = r%8 = (i2 i1 i0), swz = 8*i1 + 4*i0 + 2*i2 + i1, i.e. 0 4 9 13 2 6 11 15.  Its low
//     three bits differ over the 8 rows of a block (row reads, below), and its high two
//     bits over rows 0-3 and over rows 4-7, so the 4 rows x 4 chunks of the 32 lanes of a
//     transposing read (chunks 4m .. 4m+3, swizzled to 4-chunk groups m ^ (swz/4)) cover 16
//     distinct slots, all 64 banks (2*(r%4) + (r/4)%2 put rows r and r^1 on the same four
//     slots there: two-way conflicts).
//   * The LDS serves 16 lanes of a 16-byte read per cycle (64 banks x 4 bytes), so a row
//     read (lane i: row i, same chunk) covers 16 rows, i.e. two blocks; kPad = 128 bytes
//     after each block (d >= 64) moves the second block's rows by half a bank line, where
//     they meet no slot of the first block.
// Both the swizzle and the padding repeat every 8 rows, so a row offset that is a multiple
// of 8 is a constant byte offset (rows()).
template <int D, int ROWS = kRowTile>
struct Swz {
    static constexpr int kCpr = D / 8;  // 16-byte chunks per row
    static constexpr int kRowBytes = 2 * D;
    static constexpr int kPad = D >= 64 ? 128 : 0;
    static constexpr int kBlockData = 8 * kRowBytes;
    static constexpr int kBlockBytes = kBlockData + kPad;
    static constexpr int kBytes = (ROWS / 8) * kBlockBytes;  // one tile of ROWS rows
    static constexpr int kDma = ROWS * kRowBytes / 1024;     // wave instructions per tile
    static_assert(kPad == 0 || kBlockData % 1024 == 0, "a copy instruction stays in a block");
    // Byte offset of row n (a multiple of 8).
    static constexpr uint32_t rows(int n) { return static_cast<uint32_t>((n / 8) * kBlockBytes); }
    // Byte offset of the 1 KB that copy instruction i writes (tile bytes i*1024 ..).
    static constexpr uint32_t dma_off(int i) {
        return static_cast<uint32_t>((i * 1024 / kBlockData) * kBlockBytes + (i * 1024) % kBlockData);
    }
    __device__ static int swz(int r) {
        if constexpr (kCpr >= 16) {
            const int i0 = r & 1, i1 = (r >> 1) & 1, i2 = (r >> 2) & 1;
            return 8 * i1 + 4 * i0 + 2 * i2 + i1;
        } else {
            return kCpr >= 8 ? 2 * (r & 3) + ((r >> 2) & 1) : (r & (kCpr - 1));
        }
    }
    __device__ static uint32_t off(int r, int c) {
        return static_cast<uint32_t>((r >> 3) * kBlockBytes + (r & 7) * kRowBytes +
                                     ((c ^ swz(r)) << 4));
    }
};

// Wave `wave` of NW issues its share of the copy of rows [row0, row0 + ROWS) of a head (T
// rows of D bf16, consecutive rows rs elements apart) into the tile at LDS byte address lds.
// Rows past T are read from row T-1 (finite values; every consumer masks or zero-weights
// them).
template <int D, int NW = kWaves, int ROWS = kRowTile>
__device__ __forceinline__ void dma_tile(const uint16_t* __restrict__ head, int row0, int T,
                                         uint32_t lds, int wave, int lane, int rs) {
    using S = Swz<D, ROWS>;
    const uint16_t* base = head + static_cast<size_t>(row0) * rs;
#pragma unroll
    for (int i = wave; i < S::kDma; i += NW) {
        const int p = i * kWave + lane;  // 16-byte slot of the tile
        const int r = p / S::kCpr;
        const int c = (p % S::kCpr) ^ S::swz(r);
        const int gr = min(r, T - 1 - row0);
        dma_dwordx4(base, lds + S::dma_off(i), static_cast<uint32_t>(gr * rs * 2 + c * 16));
    }
}

// Lane (col, half) loads row `row` as a B operand over the head dimension:
// dst[s] = row[16s + 8*half .. +8], zeros if row >= T (rows rs elements apart).
template <int D>
__device__ __forceinline__ void load_rowop(bf16x8 (&dst)[D / 16],
                                          const uint16_t* __restrict__ head, int row, int T,
                                          int half, int rs) {
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
        u16x8 x = u16x8{};
        if (row < T)
            x = *reinterpret_cast<const u16x8*>(head + static_cast<size_t>(row) * rs + 16 * s +
                                                8 * half);
        dst[s] = __builtin_bit_cast(bf16x8, x);
    }
}

// Pack accumulator rows acc_row(8u .. 8u+7, half) of a 32x32 fp32 tile into a B operand.
__device__ __forceinline__ bf16x8 pack_b(const f32x16& x, int u) {
    bf16x8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = static_cast<__bf16>(x[8 * u + e]);
    return r;
}

// Store a (D x 32) transposed accumulator (acc[dt][v] = element (row, dt*32 +
// acc_row(v, half))) of a head (rows rs elements apart) in bf16, times mul.
template <int D>
__device__ __forceinline__ void store_row(uint16_t* __restrict__ head, int row, int half,
                                          const f32x16 (&acc)[D / 32], float mul, int rs) {
    uint16_t* p = head + static_cast<size_t>(row) * rs + 4 * half;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            u16x4 o;
            o[0] = f32_to_bf16_bits(acc[dt][4 * g + 0] * mul);
            o[1] = f32_to_bf16_bits(acc[dt][4 * g + 1] * mul);
            o[2] = f32_to_bf16_bits(acc[dt][4 * g + 2] * mul);
            o[3] = f32_to_bf16_bits(acc[dt][4 * g + 3] * mul);
            __builtin_nontemporal_store(o, reinterpret_cast<u16x4*>(p + dt * 32 + 8 * g));
        }
    }
}

// ---------------------------------------------------------------------------------------
// fp32 operands as bf16 planes.  An fp32 value x is carried as NP bf16 values (planes)
// x_0 + x_1 + ... with x_0 = bf16(x), x_i = bf16(x - x_0 - ... - x_{i-1}) (round to nearest
// even).  NP = 1 is the bf16 path itself.  NP = 3 keeps 3 x 8 significant bits, all of
// fp32's 24, and a product a*b is taken as the six plane products a_i*b_j with i + j <= 2;
// the three left out are below 2^-23 |a*b| together, about one fp32 rounding.
// ---------------------------------------------------------------------------------------

// c + A*B over planes, the small products first.
template <int NP>
__device__ __forceinline__ f32x16 mma_planes(const bf16x8 (&a)[NP], const bf16x8 (&b)[NP],
                                             f32x16 c) {
    static_assert(NP == 1 || NP == 3, "1 or 3 planes");
    if constexpr (NP == 1) {
        return mfma_32x32x16_bf16(a[0], b[0], c);
    } else {
        c = mfma_32x32x16_bf16(a[2], b[0], c);
        c = mfma_32x32x16_bf16(a[1], b[1], c);
        c = mfma_32x32x16_bf16(a[0], b[2], c);
        c = mfma_32x32x16_bf16(a[1], b[0], c);
        c = mfma_32x32x16_bf16(a[0], b[1], c);
        return mfma_32x32x16_bf16(a[0], b[0], c);
    }
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// The planes of 8 fp32 values (round to nearest even).  Three planes go two values at a
// time: one conversion of the pair (v_cvt_pk_bf16_f32), then the pair's bf16 values back in
// fp32 by a shift (low half) and a mask (high half) for the residuals -- the same planes as
// converting each value alone, in 5.5 instead of 7.5 VALU instructions per value (config 2
// three-plane dK/dV 171 -> 160 us, step -3.5%).
template <int NP>
__device__ __forceinline__ void split_planes(const float (&x)[8], bf16x8 (&p)[NP]) {
    if constexpr (NP == 1) {
#pragma unroll
        for (int e = 0; e < 8; ++e) p[0][e] = static_cast<__bf16>(x[e]);
    } else {
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            float r0 = x[e], r1 = x[e + 1];
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const f32x2 r = {r0, r1};
                const bf16x2 h = __builtin_convertvector(r, bf16x2);
                p[i][e] = h[0];
                p[i][e + 1] = h[1];
                if (i + 1 < NP) {
                    const uint32_t bits = __builtin_bit_cast(uint32_t, h);
                    r0 -= __builtin_bit_cast(float, bits << 16);
                    r1 -= __builtin_bit_cast(float, bits & 0xffff0000u);
                }
            }
        }
    }
}

// pack_b over planes: accumulator rows acc_row(8u .. 8u+7, half) as NP B operands.
template <int NP>
__device__ __forceinline__ void pack_planes(const f32x16& x, int u, bf16x8 (&p)[NP]) {
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = x[8 * u + e];
    split_planes<NP>(v, p);
}

// load_rowop over planes: dst[s][i] = chunk s of plane i of row `row`; plane i lies
// pstride elements after plane i-1.
template <int D, int NP>
__device__ __forceinline__ void load_rowop_planes(bf16x8 (&dst)[D / 16][NP],
                                                  const uint16_t* __restrict__ head,
                                                  size_t pstride, int row, int T, int half,
                                                  int rs) {
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        bf16x8 t[D / 16];
        load_rowop<D>(t, head + i * pstride, row, T, half, rs);
#pragma unroll
        for (int st = 0; st < D / 16; ++st) dst[st][i] = t[st];
    }
}

// load_rowop_planes from fp32 rows: the planes of row `row` of an fp32 head (rows rs
// floats apart), split in registers.
template <int D, int NP>
__device__ __forceinline__ void load_rowop_split(bf16x8 (&dst)[D / 16][NP],
                                                 const float* __restrict__ head, int row, int T,
                                                 int half, int rs) {
#pragma unroll
    for (int st = 0; st < D / 16; ++st) {
        float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (row < T) {
            const float* p = head + static_cast<size_t>(row) * rs + 16 * st + 8 * half;
            const f32x4 a = *reinterpret_cast<const f32x4*>(p);
            const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                x[e] = a[e];
                x[e + 4] = b[e];
            }
        }
        split_planes<NP>(x, dst[st]);
    }
}

// The planes of a row operand (as load_rowop_planes / load_rowop_split give them) back to
// NP head-major plane tensors (rows D elements apart, planes pstride elements apart); rows
// at or beyond T are skipped.
template <int D, int NP>
__device__ __forceinline__ void store_planes(uint16_t* __restrict__ head, size_t pstride,
                                             const bf16x8 (&x)[D / 16][NP], int row, int T,
                                             int half) {
    if (row >= T) return;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        uint16_t* p = head + i * pstride + static_cast<size_t>(row) * D + 8 * half;
#pragma unroll
        for (int st = 0; st < D / 16; ++st)
            __builtin_nontemporal_store(__builtin_bit_cast(u16x8, x[st][i]), reinterpret_cast<u16x8*>(p + 16 * st));
    }
}

// store_row in fp32.
template <int D>
__device__ __forceinline__ void store_row(float* __restrict__ head, int row, int half,
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
            __builtin_nontemporal_store(o, reinterpret_cast<f32x4*>(p + dt * 32 + 8 * g));
        }
    }
}

// ---------------------------------------------------------------------------------------
// Row stores through LDS.  Stored straight from the MFMA register layout, a wave's 32-row
// sub-block leaves as 32 bytes of each of 32 rows per store instruction (two lanes per row).
// Staged in a wave-private LDS area and read back row by row, it leaves as whole rows,
// 1 KB per wave instruction.  Stage layout: row r, 16-byte chunk c at
// r*RB + 16*(c ^ swz(r)), swz(r) = (r / max(1, 256/RB)) % min(RB/16, 16), so that the 16
// rows x one chunk that 16 lanes write, and the 256 bytes of whole rows that 16 lanes read
// back, each cover the 64 banks once.
// ---------------------------------------------------------------------------------------

template <int RB>  // bytes per staged row
struct RowStage {
    static_assert(RB >= 64 && RB % 64 == 0, "rows of whole 64-byte groups");
    static constexpr int kCpr = RB / 16;
    static constexpr int kRp = RB >= 256 ? 1 : 256 / RB;
    static constexpr int kSwzMask = (kCpr < 16 ? kCpr : 16) - 1;
    static constexpr uint32_t kBytes = 32u * RB;  // one wave's stage
    __device__ static uint32_t off(int r, int c) {
        return static_cast<uint32_t>(r * RB + 16 * (c ^ ((r / kRp) & kSwzMask)));
    }
};

__device__ __forceinline__ void lds_put16(uint32_t addr, u16x8 v) {
    *(TCAMD_LDS u16x8*)(uintptr_t)addr = v;
}
__device__ __forceinline__ void lds_put8(uint32_t addr, u16x4 v) {
    *(TCAMD_LDS u16x4*)(uintptr_t)addr = v;
}

// Wave-wide: the staged rows row0 .. row0+31 that lie below T, to rows rs_bytes apart from
// base; lane l moves chunk (64 i + l) % (RB/16) of row (64 i + l) / (RB/16) in step i.
// The row stores of the attention outputs are nontemporal: no kernel reads them back, and
// L2 stays with the K/V (or Q/dO) tiles that the blocks of a head share.
template <int RB>
__device__ __forceinline__ void stage_flush(uint32_t stage, char* __restrict__ base, int row0,
                                            int T, size_t rs_bytes, int lane) {
    using St = RowStage<RB>;
#pragma unroll
    for (int i = 0; i < 32 * St::kCpr / kWave; ++i) {
        const int g = i * kWave + lane;
        const int r = g / St::kCpr;
        const int c = g % St::kCpr;
        const u16x8 v = *(TCAMD_LDS const u16x8*)(uintptr_t)(stage + St::off(r, c));
        if (row0 + r < T)
            __builtin_nontemporal_store(v, reinterpret_cast<u16x8*>(base + static_cast<size_t>(row0 + r) * rs_bytes + 16 * c));
    }
}

// A wave's stage inside a pair of idle tile buffers (lo, hi: LDS byte addresses, each at
// least 2 * bytes long): waves 0, 1 in lo, waves 2, 3 in hi.
__device__ __forceinline__ uint32_t wave_stage(uint32_t lo, uint32_t hi, int wave,
                                               uint32_t bytes) {
    return (wave < 2 ? lo : hi) + static_cast<uint32_t>(wave & 1) * bytes;
}

// store_planes for the sub-block of rows row0 .. row0+31, through the wave's stage of
// RowStage<2D>::kBytes bytes: the same values, stored as whole rows.
template <int D, int NP>
__device__ __forceinline__ void store_planes_staged(uint16_t* __restrict__ head, size_t pstride,
                                                    const bf16x8 (&x)[D / 16][NP], int row0,
                                                    int T, int lane, uint32_t stage) {
    using St = RowStage<2 * D>;
    const int col = lane & 31;
    const int half = lane >> 5;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
#pragma unroll
        for (int st = 0; st < D / 16; ++st)
            lds_put16(stage + St::off(col, 2 * st + half), __builtin_bit_cast(u16x8, x[st][i]));
        stage_flush<2 * D>(stage, reinterpret_cast<char*>(head + i * pstride), row0, T, 2 * D,
                           lane);
    }
}

// store_row (bf16) for the sub-block of rows row0 .. row0+31, through the wave's stage of
// RowStage<2D>::kBytes bytes.
template <int D>
__device__ __forceinline__ void store_row_staged(uint16_t* __restrict__ head, int row0, int T,
                                                 int lane, const f32x16 (&acc)[D / 32],
                                                 float mul, int rs, uint32_t stage) {
    using St = RowStage<2 * D>;
    const int col = lane & 31;
    const int half = lane >> 5;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            u16x4 o;
            o[0] = f32_to_bf16_bits(acc[dt][4 * g + 0] * mul);
            o[1] = f32_to_bf16_bits(acc[dt][4 * g + 1] * mul);
            o[2] = f32_to_bf16_bits(acc[dt][4 * g + 2] * mul);
            o[3] = f32_to_bf16_bits(acc[dt][4 * g + 3] * mul);
            lds_put8(stage + St::off(col, 4 * dt + g) + 8 * half, o);
        }
    }
    stage_flush<2 * D>(stage, reinterpret_cast<char*>(head), row0, T,
                       static_cast<size_t>(rs) * 2, lane);
}

// store_row (fp32) for the sub-block of rows row0 .. row0+31, through the wave's stage of
// RowStage<128>::kBytes bytes: one 32-column slice (128 bytes of each row) at a time.
template <int D>
__device__ __forceinline__ void store_row_staged(float* __restrict__ head, int row0, int T,
                                                 int lane, const f32x16 (&acc)[D / 32],
                                                 float mul, int rs, uint32_t stage) {
    using St = RowStage<128>;
    const int col = lane & 31;
    const int half = lane >> 5;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            f32x4 o;
            o[0] = acc[dt][4 * g + 0] * mul;
            o[1] = acc[dt][4 * g + 1] * mul;
            o[2] = acc[dt][4 * g + 2] * mul;
            o[3] = acc[dt][4 * g + 3] * mul;
            lds_put16(stage + St::off(col, 2 * g + half), __builtin_bit_cast(u16x8, o));
        }
        stage_flush<128>(stage, reinterpret_cast<char*>(head + 32 * dt), row0, T,
                         static_cast<size_t>(rs) * 4, lane);
    }
}

// Bytes of one wave's stage for the staged stores of a D-wide row operand (planes, bf16 or
// fp32 rows).
template <int D, int NP>
constexpr uint32_t kStageBytes = NP == 1 ? RowStage<2 * D>::kBytes
                                         : (RowStage<2 * D>::kBytes > RowStage<128>::kBytes
                                                ? RowStage<2 * D>::kBytes
                                                : RowStage<128>::kBytes);

// ---------------------------------------------------------------------------------------
// Per-row statistics as one more contraction step: a product over 16 more k-slots, where the
// A (or B) operand is (1, 1, [1,] 0, ...) and the other carries the terms of the statistic,
// adds the statistic to every element of the row.
// ---------------------------------------------------------------------------------------

// Terms of a statistic chunk: (hi, lo) carries 16 significant bits, enough next to bf16
// operands; fp32 operands take three.
template <int NP>
constexpr int kStatTerms = NP == 1 ? 2 : 3;

// The terms of x: x_0 = bf16(x), x_i = bf16(x - x_0 - ... - x_{i-1}).
template <int NP>
__device__ __forceinline__ u16x4 stat_terms(float x) {
    u16x4 v = u16x4{};
#pragma unroll
    for (int i = 0; i < kStatTerms<NP>; ++i) {
        v[i] = f32_to_bf16_bits(x);
        x -= bf16_bits_to_f32(v[i]);
    }
    return v;
}

// The B or A operand (1, 1, [1,] 0, ...) of a contraction step that adds a per-row
// statistic chunk to a product: lanes of k-group 1 hold zeros.
template <int NP>
__device__ __forceinline__ bf16x8 ones_chunk(int half) {
    bf16x8 one = bf16x8{};
    if (half == 0) {
#pragma unroll
        for (int i = 0; i < kStatTerms<NP>; ++i) one[i] = static_cast<__bf16>(1.0f);
    }
    return one;
}

// The statistic chunk (terms of x, 0, ...) of a lane's row (zeros in k-group 1).
template <int NP>
__device__ __forceinline__ bf16x8 stat_chunk(float x, int half) {
    u16x8 v = u16x8{};
    if (half == 0) {
        const u16x4 t = stat_terms<NP>(x);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = t[i];
    }
    return __builtin_bit_cast(bf16x8, v);
}

// CUs per XCD of the MI355X (256 CUs in 8 XCDs).
constexpr int kCusPerXcd = 32;

// Workgroup id -> (head bh, block b) in rank order: b = nb-1-rank when `descending`, else
// b = rank, so the heaviest causal blocks start first.  When BH % 8 == 0, every block of a
// head is on one XCD (workgroup i runs on XCD i % 8), so a head's tiles stay in one L2.
// `serpentine` (wave-uniform; for grids the device holds at once): the XCD's workgroups take
// the heaviest-first order in rounds of one per CU with every other full round reversed, so
// a CU, which then holds the j-th workgroups of consecutive rounds, pairs heavy blocks with
// light ones (at config 2, three blocks per CU: causal work 12-14 units per CU instead of
// 10-17).  Grids that do not fit at once keep the plain order: there the heaviest blocks
// must start first.
__host__ __device__ __forceinline__ void map_block(int id, int BH, int nb, bool descending,
                                                   bool serpentine, int& bh, int& b) {
    int rank;
    if ((BH & 7) == 0) {
        const int hpx = BH >> 3;
        int slot = id >> 3;
        const int round = slot / kCusPerXcd;
        if (serpentine && (round & 1) && (round + 1) * kCusPerXcd <= hpx * nb)
            slot = round * kCusPerXcd + (kCusPerXcd - 1 - slot % kCusPerXcd);
        bh = (id & 7) * hpx + slot % hpx;
        rank = slot / hpx;
    } else {
        bh = id % BH;
        rank = id / BH;
    }
    b = descending ? nb - 1 - rank : rank;
}

// map_block's plain order (rank order, one XCD per head when BH % 8 == 0) with the XCD's
// heads taken G at a time: each group's blocks, heaviest first (the last block first when
// descending), before the next group's, so that fewer heads' tiles compete for the XCD's L2.
// G = 0, or heads per XCD not a multiple of G: map_block's order.
__host__ __device__ __forceinline__ void map_block_grouped(int id, int BH, int nb, int G,
                                                           bool descending, int& bh, int& b) {
    const int hpx = BH >> 3;
    if (G > 0 && (BH & 7) == 0 && hpx % G == 0) {
        const int slot = id >> 3;
        const int g = slot / (G * nb), r = slot % (G * nb);
        bh = (id & 7) * hpx + g * G + r % G;
        b = descending ? nb - 1 - r / G : r / G;
    } else {
        map_block(id, BH, nb, descending, false, bh, b);
    }
}

// 16 bytes from LDS at a byte address.
__device__ __forceinline__ bf16x8 lds_b128(uint32_t addr) {
    return __builtin_bit_cast(bf16x8, *(TCAMD_LDS const u16x8*)(uintptr_t)addr);
}
// 16 bytes of fp32 from LDS at a byte address.
__device__ __forceinline__ f32x4 lds_f32x4(uint32_t addr) {
    return *(TCAMD_LDS const f32x4*)(uintptr_t)addr;
}
// A operand of a product contracting over the 16 sequence rows 16u.. of a tile (see
// above): two transposing reads, 8 rows apart.
__device__ __forceinline__ bf16x8 lds_tr(uint32_t addr, uint32_t row8_bytes) {
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((TCAMD_LDS s16x4*)(uintptr_t)addr);
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (TCAMD_LDS s16x4*)(uintptr_t)(addr + row8_bytes));
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}
// This lane's byte offsets within a tile: row reads (row col, chunk 2*st + half) and the
// transposing reads of head-dim tile dt (16-lane group G reads dims d0(G) + 4*(j%4) .. of
// rows 4*(G/2) + j/4).
template <int D>
__device__ __forceinline__ void lane_offsets(int lane, uint32_t (&roff)[D / 16],
                                             uint32_t (&troff)[D / 32]) {
    using S = Swz<D>;
    const int col = lane & 31;
    const int half = lane >> 5;
#pragma unroll
    for (int st = 0; st < D / 16; ++st) roff[st] = S::off(col, 2 * st + half);
    const int G = lane >> 4;
    const int j16 = lane & 15;
    const int tr_row = 4 * (G >> 1) + (j16 >> 2);
    const int tr_dim = 16 * (G & 1) + 4 * (j16 & 3);
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
        const int d = dt * 32 + tr_dim;
        troff[dt] = S::off(tr_row, d >> 3) + static_cast<uint32_t>((d & 7) << 1);
    }
}

// Host side: whether a query-parallel kernel should run one 32-query sub-block per wave
// (128 queries per workgroup) instead of two (256): when 256-query blocks would give fewer
// than two workgroups per CU, halving the block doubles the parallelism.
inline bool use_single_subblock(int BH, int T) {
    static thread_local int cached_dev = -1, cached_cus = 256;
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (dev != cached_dev) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
            cus > 0)
            cached_cus = cus;
        cached_dev = dev;
    }
    const long long blocks = static_cast<long long>(BH) * ((T + 255) / 256);
    return blocks < 2LL * cached_cus;
}

}  // namespace bf16t
}  // namespace tcamd
