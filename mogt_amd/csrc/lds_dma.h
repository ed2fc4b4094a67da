// Direct global-to-LDS loads for the bf16 GEMMs (swiglu_gemm.hip,
// wgrad_gemm.hip): buffer descriptors, the 16-byte-per-lane load that writes
// LDS without staging registers, and the explicit wait on outstanding vector
// memory operations that such loads need (the compiler's own waits for
// LDS-bound loads drain all of them before any LDS read).
#pragma once

#include "common.h"

namespace mogt {

typedef int lds_i32x4 __attribute__((ext_vector_type(4)));

// raw buffer descriptor over [base, base + bytes): loads at offsets past
// `bytes` return zero
__device__ __forceinline__ lds_i32x4 lds_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    lds_i32x4 r;
    r[0] = __builtin_amdgcn_readfirstlane(static_cast<int>(a & 0xffffffffu));
    r[1] = __builtin_amdgcn_readfirstlane(static_cast<int>(a >> 32));   // stride 0
    r[2] = __builtin_amdgcn_readfirstlane(static_cast<int>(bytes));
    r[3] = 0x00020000;
    return r;
}

// 64 lanes x 16 bytes from (rsrc, voff + soff) into LDS at lds .. lds + 1023,
// lane L's bytes at lds + 16 L.  m0 carries the LDS address; it is written
// here and read only by the load that follows.
__device__ __forceinline__ void lds_dma16(lds_i32x4 rsrc, int voff, int soff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(lds), "v"(voff), "s"(rsrc), "s"(soff)
                 : "memory", "m0");
}

// wait until at most N vector memory operations of this wave are outstanding
template <int N>
__device__ __forceinline__ void lds_wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// LDS address (32-bit) of a __shared__ array
template <typename T>
__device__ __forceinline__ uint32_t lds_addr(T* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) char*)p));
}

}  // namespace mogt
