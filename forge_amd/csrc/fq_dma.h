// fq_dma.h -- copies from global memory straight into LDS, counted by hand.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fq {

// Global memory straight into LDS: 16 bytes per lane, to lds + 16 lane (lds
// is wave-uniform, in M0).  Issued as inline assembly on purpose: the
// compiler cannot tell which LDS bytes the builtin's copy writes, so it waits
// for every outstanding load (vmcnt(0)) before the next LDS read, which would
// serialise a kernel's loads with its compute.  The kernel counts the copies
// itself (wait_vm) before it reads what they wrote.  The compiler does not
// see these copies either when it counts its own loads, so its waits for
// register loads issued before a copy only ever wait longer than needed.
__device__ __forceinline__ void dma16(const uint8_t* g, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(g), "{m0}"(lds) : "memory");
}

// The same copy from base + off: base wave-uniform (a scalar register pair),
// off a 32-bit per-lane byte offset, so a loop that moves base keeps the
// per-lane part in one register and its address arithmetic on the scalar
// unit.
__device__ __forceinline__ void dma16s(uint32_t off, const uint8_t* base, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(off), "s"(base), "{m0}"(lds)
                 : "memory");
}

// Wait until at most N vector-memory loads of this wave are outstanding.
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// The LDS address of p as the 32-bit value M0 takes.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)p;
}

}  // namespace fq
