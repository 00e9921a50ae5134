// LDS DMA and wait helpers shared by the MFMA attention kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace gtmfma {

// One global_load_lds_dwordx4: lane l copies 16 bytes from gbase + voff to LDS byte address
// lds + 16 l.  Issued from assembly so that the compiler does not see an LDS write it would
// have to wait for (vmcnt(0)) before every later LDS read, which would serialise the prefetch
// of later tiles with the compute of the current one; the kernel waits for it explicitly
// (vmcnt + barrier) before reading the destination.  m0 is saved and restored.  An LDS DMA
// that reads m0 right after a scalar write of it needs one wait state (the compiler inserts
// that s_nop itself around its own LDS DMA; inside assembly it cannot).
__device__ inline void lds_dma16(uint32_t lds, const void *gbase, uint32_t voff) {
    uint32_t save;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %2, %3\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(save)
        : "s"(lds), "v"(voff), "s"(gbase)
        : "memory");
}

// One global_load_lds_dword: lane l copies 4 bytes from gbase + voff to LDS byte address
// lds + 4 l.
__device__ inline void lds_dma4(uint32_t lds, const void *gbase, uint32_t voff) {
    uint32_t save;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dword %2, %3\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(save)
        : "s"(lds), "v"(voff), "s"(gbase)
        : "memory");
}

__device__ inline uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// s_waitcnt vmcnt(n) (expcnt and lgkmcnt left alone), n a compile-time constant < 64: vmcnt's
// low 4 bits sit in bits 3:0 of the encoding, its high 2 bits in bits 15:14
template <int N>
__device__ inline void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt(0x0f70 | (N & 15) | ((N >> 4) << 14));
}

}  // namespace gtmfma
