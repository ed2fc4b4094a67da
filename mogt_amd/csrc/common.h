// Shared device/host helpers for the MOGT scan kernels (gfx950, wave64).
//
// Everything here is plain HIP for CDNA4: no CUDA-compat headers, no second
// backend.  Numeric types crossing the C ABI are identified by the small
// integer codes of include/mogt_scan.h (MOGT_F32 / MOGT_BF16).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/mogt_scan.h"

namespace mogt {

// ---------------------------------------------------------------------------
// Error reporting: every entry point returns 0 or a negative code and leaves a
// message in a thread-local buffer readable through mogt_last_error().
// ---------------------------------------------------------------------------
int set_error(int code, const char* fmt, ...);
void clear_error();
int check_launch(const char* what);

// ---------------------------------------------------------------------------
// bf16 <-> f32.  Storage is the raw 16-bit pattern.  f32 -> bf16 uses
// round-to-nearest-even on the upper half of the IEEE-754 word (the standard
// bit-level method; NaNs are kept quiet).
// ---------------------------------------------------------------------------
typedef uint16_t bf16_t;

__device__ __forceinline__ float bf16_to_f32(bf16_t x) {
    return __uint_as_float(static_cast<uint32_t>(x) << 16);
}

__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<bf16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<bf16_t>(u >> 16);
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

template <typename T> struct IO;
template <> struct IO<float> {
    __device__ __forceinline__ static float ld(float x) { return x; }
    __device__ __forceinline__ static float st(float x) { return x; }
};
template <> struct IO<bf16_t> {
    __device__ __forceinline__ static float ld(bf16_t x) { return bf16_to_f32(x); }
    __device__ __forceinline__ static bf16_t st(float x) { return f32_to_bf16(x); }
};

// N consecutive elements moved as one vector memory instruction.
template <typename T, int N> struct alignas(sizeof(T) * N) Pack { T v[N]; };

template <typename T, int N>
__device__ __forceinline__ void load_vec(const T* __restrict__ p, float (&out)[N]) {
    Pack<T, N> pk = *reinterpret_cast<const Pack<T, N>*>(p);
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = IO<T>::ld(pk.v[i]);
}

template <typename T, int N>
__device__ __forceinline__ void store_vec(T* __restrict__ p, const float (&in)[N]) {
    Pack<T, N> pk;
#pragma unroll
    for (int i = 0; i < N; ++i) pk.v[i] = IO<T>::st(in[i]);
    *reinterpret_cast<Pack<T, N>*>(p) = pk;
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

// ---------------------------------------------------------------------------
// Decoupled look-back workspace protocol (shared by every single-pass scan).
//
//   hdr[0]  ticket counter: work-groups take chunk ids in the order they start,
//           so a chunk only ever waits on chunks that are already resident.
//   hdr[1]  done counter: the last work-group to finish resets hdr[0..1] and
//           advances the epoch, so the buffer is reusable by the next launch
//           without a memset (also inside a captured HIP graph).
//   hdr[2]  epoch (30 bits).
//   hdr[3]  count of bounded waits that gave up (must stay 0; a non-zero value
//           means the protocol was violated and the output is not valid).
//
// Every published value is a 64-bit word {tag:32 | f32 bits:32} written with a
// single agent-scope atomic store, tag = epoch << 2 | status.  A reader accepts
// a word only if its tag matches, so payloads need no release/acquire fences
// (an agent-scope release fence on gfx950 writes back the whole L2).  Per-chunk
// status flags are hints that tell the look-back how far back to read.
// ---------------------------------------------------------------------------
constexpr uint32_t ST_AGG = 1u;   // chunk aggregate published
constexpr uint32_t ST_INC = 2u;   // inclusive prefix published
constexpr size_t WS_HDR_BYTES = 256;

__device__ __forceinline__ uint32_t ld_relaxed(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_relaxed(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_relaxed(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_relaxed(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t fetch_add_relaxed(uint32_t* p, uint32_t v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t pack_word(float v, uint32_t tag) {
    return (static_cast<uint64_t>(tag) << 32) | __float_as_uint(v);
}
__device__ __forceinline__ uint32_t word_tag(uint64_t w) { return static_cast<uint32_t>(w >> 32); }
__device__ __forceinline__ float word_val(uint64_t w) { return __uint_as_float(static_cast<uint32_t>(w)); }

__device__ __forceinline__ uint32_t make_tag(uint32_t epoch, uint32_t status) {
    return (epoch << 2) | status;
}

// Every wait is bounded so a kernel always drains, whatever the workspace
// holds: after MAX_SPIN polls (about a second) the wait gives up and counts
// the failure in hdr[3].
constexpr uint32_t MAX_SPIN = 1u << 20;

__device__ __forceinline__ void note_timeout(uint32_t* hdr) { fetch_add_relaxed(&hdr[3], 1u); }

// Spin until the tagged word at p carries `tag`; return its value.
__device__ __forceinline__ float wait_word(const uint64_t* p, uint32_t tag, uint32_t* hdr) {
    uint64_t w = ld_relaxed(p);
    uint32_t n = 0;
    while (word_tag(w) != tag) {
        if (++n > MAX_SPIN) {
            note_timeout(hdr);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
        w = ld_relaxed(p);
    }
    return word_val(w);
}

// Work-group start: take a ticket and read the epoch (thread 0, broadcast).
__device__ __forceinline__ void ws_begin(uint32_t* hdr, int* s_ticket, uint32_t* s_epoch) {
    if (threadIdx.x == 0) {
        *s_ticket = static_cast<int>(fetch_add_relaxed(&hdr[0], 1u));
        *s_epoch = ld_relaxed(&hdr[2]);
    }
    __syncthreads();
}

// Work-group end: the last one resets the ticket/done counters and advances
// the epoch for the next launch.
__device__ __forceinline__ void ws_end(uint32_t* hdr, uint32_t epoch) {
    if (threadIdx.x == 0) {
        uint32_t total = gridDim.x * gridDim.y * gridDim.z;
        uint32_t old = fetch_add_relaxed(&hdr[1], 1u);
        if (old == total - 1) {
            st_relaxed(&hdr[0], 0u);
            st_relaxed(&hdr[1], 0u);
            st_relaxed(&hdr[2], (epoch + 1u) & 0x3fffffffu);
        }
    }
}

inline size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

}  // namespace mogt
