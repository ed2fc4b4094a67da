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
// compute units of the current device (queried once per device); MOGT_OK or
// MOGT_E_LAUNCH with the HIP error
int device_cu_count(int& cus);

// ---------------------------------------------------------------------------
// bf16 <-> f32.  Storage is the raw 16-bit pattern.  f32 -> bf16 rounds to
// nearest even (the hardware conversion of gfx950).
// ---------------------------------------------------------------------------
typedef uint16_t bf16_t;

__device__ __forceinline__ float bf16_to_f32(bf16_t x) {
    return __uint_as_float(static_cast<uint32_t>(x) << 16);
}

__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
    // one v_cvt_pk_bf16_f32 on gfx950 (round to nearest even, NaN stays NaN)
    return __builtin_bit_cast(bf16_t, static_cast<__bf16>(f));
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

// sigmoid(a) = 1 / (1 + 2^(-a log2 e)) on the hardware exponential and
// reciprocal (v_exp_f32, v_rcp_f32; about 2 ulp): a = -inf gives 0, +inf 1.
__device__ __forceinline__ float sigmoid_hw(float a) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(a * -1.4426950408889634f));
}

// ---------------------------------------------------------------------------
// Decoupled look-back workspace protocol (shared by every single-pass scan).
//
// Chunk ids are blockIdx.x: work-groups are dispatched in increasing id order,
// so the lowest unfinished chunk is always resident and never waits on an
// unstarted one.  (A global atomic ticket would make this independent of the
// dispatcher, but one same-address atomic per work-group costs more than the
// whole scan on an 8-XCD part; every wait below is bounded instead.)
//
//   hdr[2]  epoch (30 bits), read once by every work-group.
//   hdr[3]  count of bounded waits that gave up (must stay 0; a non-zero value
//           means the protocol was violated and the output is not valid).
//           A look-back that gives up also writes NaN into its chunk's carry,
//           so the affected outputs are visibly invalid; the count is read
//           back with mogt_workspace_faults().
//
// Every published value is a 64-bit word {tag:32 | f32 bits:32} written with a
// single agent-scope atomic store, tag = epoch << 2 | status.  A reader accepts
// a word only if its tag matches, so payloads need no release/acquire fences
// (an agent-scope release fence on gfx950 writes back the whole L2).  Each
// chunk also publishes one status flag word (same tag) that tells the
// look-back how far back to read.
//
// Reuse without clearing: the last work-group waits until every chunk flag
// carries the current epoch's tag (each work-group writes its flag right after
// it read the epoch), then advances the epoch.  Tagged words of older launches
// of the same layout can never match a newer tag, so repeated launches of one
// layout never clear the buffer, also inside a captured HIP graph.  Words of
// another layout, or plain data of other kernels, could in principle hold a
// current tag's bit pattern: the host keeps look-back workspaces apart from
// plain-data scratch and clears the region past the header whenever the
// layout of a buffer's launches changes (mogt_amd/ops.py, workspace()).
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

// Work-group start: read the launch's epoch (thread 0, broadcast via LDS).
__device__ __forceinline__ uint32_t ws_epoch(uint32_t* hdr, uint32_t* s_epoch) {
    if (threadIdx.x == 0) *s_epoch = ld_relaxed(&hdr[2]);
    __syncthreads();
    return *s_epoch;
}

// Last work-group of the grid: once all n_flags chunk flags carry the tag
// `want` (make_tag(epoch, status): never 0, so a zero-filled word never
// passes), advance the epoch for the next launch.
__device__ __forceinline__ void ws_finish(uint32_t* hdr, const uint32_t* flags, int64_t n_flags,
                                          uint32_t epoch, uint32_t want) {
    const uint64_t lin = blockIdx.x + static_cast<uint64_t>(gridDim.x) *
                                          (blockIdx.y + static_cast<uint64_t>(gridDim.y) * blockIdx.z);
    if (lin != static_cast<uint64_t>(gridDim.x) * gridDim.y * gridDim.z - 1) return;
    for (int64_t i = threadIdx.x; i < n_flags; i += blockDim.x) {
        uint32_t n = 0;
        while (ld_relaxed(&flags[i]) != want) {
            if (++n > MAX_SPIN) {
                note_timeout(hdr);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) st_relaxed(&hdr[2], (epoch + 1u) & 0x3fffffffu);
}

// Streaming (non-temporal) vector loads/stores of N consecutive elements: the
// scan touches every byte exactly once, so keep it out of the caches.
template <int BYTES> struct WordVec;
template <> struct WordVec<4> { typedef uint32_t type; };
template <> struct WordVec<8> { typedef uint32_t type __attribute__((ext_vector_type(2))); };
template <> struct WordVec<16> { typedef uint32_t type __attribute__((ext_vector_type(4))); };

template <typename T, int N>
__device__ __forceinline__ void load_stream(const T* __restrict__ p, float (&out)[N]) {
    constexpr int BYTES = static_cast<int>(sizeof(T)) * N;
    if constexpr (BYTES == 2) {
        out[0] = IO<T>::ld(__builtin_nontemporal_load(p));
    } else {
        typedef typename WordVec<BYTES>::type W;
        union { W w; T v[N]; } u;
        u.w = __builtin_nontemporal_load(reinterpret_cast<const W*>(p));
#pragma unroll
        for (int i = 0; i < N; ++i) out[i] = IO<T>::ld(u.v[i]);
    }
}

// Raw 16-bit patterns of N consecutive bf16 values (zero-extended).
template <int N>
__device__ __forceinline__ void load_bits16(const bf16_t* __restrict__ p, uint32_t (&out)[N]) {
    constexpr int BYTES = 2 * N;
    if constexpr (BYTES == 2) {
        out[0] = __builtin_nontemporal_load(p);
    } else {
        typedef typename WordVec<BYTES>::type W;
        union { W w; bf16_t v[N]; } u;
        u.w = __builtin_nontemporal_load(reinterpret_cast<const W*>(p));
#pragma unroll
        for (int i = 0; i < N; ++i) out[i] = u.v[i];
    }
}

// BYTES consecutive bytes (2, 4, 8 or 16) as raw 32-bit words, streaming
// (non-temporal) or cached.  No value is extracted, so a run of these loads
// issues back to back without waiting.
template <int BYTES, bool NT>
__device__ __forceinline__ void load_raw_impl(const void* p, uint32_t (&w)[(BYTES + 3) / 4]) {
    if constexpr (BYTES == 2) {
        const uint16_t* q = static_cast<const uint16_t*>(p);
        w[0] = NT ? __builtin_nontemporal_load(q) : *q;
    } else if constexpr (BYTES == 4) {
        const uint32_t* q = static_cast<const uint32_t*>(p);
        w[0] = NT ? __builtin_nontemporal_load(q) : *q;
    } else {
        typedef typename WordVec<BYTES>::type W;
        const W* q = static_cast<const W*>(p);
        const W x = NT ? __builtin_nontemporal_load(q) : *q;
#pragma unroll
        for (int i = 0; i < BYTES / 4; ++i) w[i] = x[i];
    }
}
template <int BYTES>
__device__ __forceinline__ void load_raw(const void* p, uint32_t (&w)[(BYTES + 3) / 4]) {
    load_raw_impl<BYTES, true>(p, w);
}
template <int BYTES>
__device__ __forceinline__ void load_raw_cached(const void* p, uint32_t (&w)[(BYTES + 3) / 4]) {
    load_raw_impl<BYTES, false>(p, w);
}

template <typename T, int N>
__device__ __forceinline__ void store_stream(T* __restrict__ p, const float (&in)[N]) {
    constexpr int BYTES = static_cast<int>(sizeof(T)) * N;
    if constexpr (BYTES == 2) {
        __builtin_nontemporal_store(IO<T>::st(in[0]), p);
    } else {
        typedef typename WordVec<BYTES>::type W;
        union { W w; T v[N]; } u;
#pragma unroll
        for (int i = 0; i < N; ++i) u.v[i] = IO<T>::st(in[i]);
        __builtin_nontemporal_store(u.w, reinterpret_cast<W*>(p));
    }
}

inline size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

}  // namespace mogt
