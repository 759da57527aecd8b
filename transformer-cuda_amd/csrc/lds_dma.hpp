// lds_dma.hpp - HBM -> LDS copies (global_load_lds) and the waits that order them.
//
// The copies are issued as inline asm so that the compiler's wait-count pass, which cannot
// tell different LDS tiles apart, does not insert a full vmcnt(0) before every LDS read
// that follows a copy into another tile.  The kernels order copies against their reads
// themselves: wait_vm<N>() before the first read of a tile (vector-memory operations return
// in issue order, so it waits for every copy but the last N), and wait_lds() before a tile
// that is still being read is overwritten.  Both are asm with a memory clobber, so no LDS
// access is moved across them.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define TCAMD_LDS __attribute__((address_space(3)))

// LDS byte address of a __shared__ object.
#define lds_addr(obj) \
    static_cast<uint32_t>(reinterpret_cast<uintptr_t>((TCAMD_LDS const void*)(obj)))

namespace tcamd {

template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N < 63 ? N : 63) : "memory");  // 6-bit field
}
__device__ __forceinline__ void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Wait until at most n (wave-uniform, 0 .. 15) vector-memory operations of this wave are
// outstanding (larger n: 15, which waits longer, always safe).
__device__ __forceinline__ void wait_vm_at_most(int n) {
    switch (n) {
        case 0: wait_vm<0>(); break;
        case 1: wait_vm<1>(); break;
        case 2: wait_vm<2>(); break;
        case 3: wait_vm<3>(); break;
        case 4: wait_vm<4>(); break;
        case 5: wait_vm<5>(); break;
        case 6: wait_vm<6>(); break;
        case 7: wait_vm<7>(); break;
        case 8: wait_vm<8>(); break;
        case 9: wait_vm<9>(); break;
        case 10: wait_vm<10>(); break;
        case 11: wait_vm<11>(); break;
        case 12: wait_vm<12>(); break;
        case 13: wait_vm<13>(); break;
        case 14: wait_vm<14>(); break;
        default: wait_vm<15>(); break;
    }
}

// A 64-bit value that is the same in every lane, moved to SGPRs (the copies take their base
// address from SGPRs).
__device__ __forceinline__ size_t wave_uniform(size_t v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
    return (static_cast<size_t>(hi) << 32) | lo;
}

// M0 carries the LDS address.  These asm statements are the only users of M0 in the kernels
// (gfx9-class LDS instructions do not read it), so declaring it clobbered is exact; the
// compiler's generic warning about clobbering a reserved register is silenced.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"

// Lane i copies 4 bytes from row_ptr + voff_i (row_ptr wave-uniform) to LDS byte address
// lds_byte + 4*i.
__device__ __forceinline__ void dma_dword(const void* row_ptr, uint32_t lds_byte, uint32_t voff) {
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dword %1, %2"
        :
        : "s"(lds_byte), "v"(voff), "s"(row_ptr)
        : "memory", "m0");
}

// Lane i copies 16 bytes from base + voff_i (base wave-uniform) to LDS byte address
// lds_byte + 16*i: one instruction fills 1 KB of LDS.
__device__ __forceinline__ void dma_dwordx4(const void* base, uint32_t lds_byte, uint32_t voff) {
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %2"
        :
        : "s"(lds_byte), "v"(voff), "s"(base)
        : "memory", "m0");
}
#pragma clang diagnostic pop

}  // namespace tcamd
