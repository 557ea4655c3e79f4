// Direct-to-LDS staging helpers shared by the attention and selection
// kernels (gfx950).
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace hba {

// Byte offset of an LDS object within the workgroup's LDS (for M0).
__device__ __forceinline__ uint32_t lds_offset(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// One 1 KB direct-to-LDS copy: lane l's 16 bytes land at lds + 16*l.  Written
// as inline asm so that the compiler does not serialise a ring on it (it would
// wait for every outstanding LDS DMA before each LDS read); the callers order
// it by hand: s_waitcnt vmcnt + barrier before a slot is read, a barrier before
// a slot is refilled.
__device__ __forceinline__ void dma16(const void *src, uint32_t lds_addr) {
    const uint32_t a = __builtin_amdgcn_readfirstlane(lds_addr);   // wave-uniform by construction
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(a), "v"(src)
                 : "memory");
}

// vmcnt(N) with the other counters left alone (gfx9 s_waitcnt encoding)
template <int N>
__device__ __forceinline__ void wait_vm() {
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// vmcnt(c) for a wave-uniform runtime c in [0, 24] (larger values wait for
// everything: always safe, only slower)
__device__ __forceinline__ void wait_vm_n(int c) {
    switch (c) {
#define HBA_VMW(N) \
    case N: wait_vm<N>(); break;
        HBA_VMW(1) HBA_VMW(2) HBA_VMW(3) HBA_VMW(4) HBA_VMW(5) HBA_VMW(6) HBA_VMW(7) HBA_VMW(8)
        HBA_VMW(9) HBA_VMW(10) HBA_VMW(11) HBA_VMW(12) HBA_VMW(13) HBA_VMW(14) HBA_VMW(15) HBA_VMW(16)
        HBA_VMW(17) HBA_VMW(18) HBA_VMW(19) HBA_VMW(20) HBA_VMW(21) HBA_VMW(22) HBA_VMW(23) HBA_VMW(24)
#undef HBA_VMW
        default: wait_vm<0>(); break;
    }
}

}  // namespace hba
