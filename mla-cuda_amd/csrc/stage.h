// Direct-to-LDS staging shared by the kernels that stream the cache or the weights through
// LDS (flash.hip, wgemm.hip): buffer descriptors, the buffer_load ... lds instruction,
// vector-memory waits and an LDS-only workgroup barrier.
#pragma once

#include "common.h"

namespace mla {

typedef __attribute__((address_space(3))) void lds_t;

template <int N>
__device__ __forceinline__ void wait_vm() {
    // vmcnt(N) with lgkmcnt and expcnt left at their maxima (gfx9 encoding)
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier for LDS data only: this wave's LDS accesses are complete (lgkmcnt(0)),
// then s_barrier.  __syncthreads() would also wait for every outstanding global load
// (vmcnt(0)), i.e. drain the ring of direct-to-LDS prefetches.  The empty asm statements
// and scheduling barriers keep the compiler from moving instructions across the barrier.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0), vmcnt/expcnt at their maxima
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

typedef int32_t v4i __attribute__((ext_vector_type(4)));

// 16 bytes per lane from buffer offset soff + voff into LDS at lds + 16*lane (gfx950
// buffer_load_dwordx4 ... lds).  Written as asm so that the compiler neither tracks it
// (it would otherwise wait for every such load before any LDS read it cannot prove
// disjoint) nor reorders memory accesses across it; the kernel waits with explicit vmcnt.
// voff >= kRsrcRange (kOob) returns zeros without a memory access.
// (m0 is a reserved register: the compiler keeps no value in it across this statement;
// nothing else in these kernels uses m0.)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(v4i rsrc, uint32_t lds, uint32_t voff, uint32_t soff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(lds), "v"(voff), "s"(rsrc), "s"(soff)
                 : "memory", "m0");
}
// The same with soffset 0 and an immediate offset OFF (< 4096), which the instruction adds
// to both addresses: the bytes at voff + OFF land at lds + OFF + 16*lane.
template <int OFF>
__device__ __forceinline__ void dma16_imm(v4i rsrc, uint32_t lds, uint32_t voff) {
    static_assert(OFF >= 0 && OFF < 4096, "12-bit buffer offset");
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen offset:%3 lds"
                 :
                 : "s"(lds), "v"(voff), "s"(rsrc), "i"(OFF)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)reinterpret_cast<uintptr_t>((const lds_t*)p);
}

// Descriptor words of `bytes` bytes at base + off (off in bytes); wave-uniform arguments
// (readfirstlane keeps the words in scalar registers, as the load instruction needs).
__device__ __forceinline__ v4i rsrc_span(uint64_t base, uint32_t off, uint32_t bytes) {
    const uint64_t p = base + off;
    return v4i{__builtin_amdgcn_readfirstlane((int32_t)(uint32_t)p),
               __builtin_amdgcn_readfirstlane((int32_t)((uint32_t)(p >> 32) & 0xffff)),
               __builtin_amdgcn_readfirstlane((int32_t)bytes), 0x00020000};
}

}  // namespace mla
