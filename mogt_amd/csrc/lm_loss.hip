// Row kernels of the chunked tied-head cross-entropy (chunked_lm_loss.py:5-80).
// For one [rows, vocab] block of logits x (one chunk of tokens against the
// whole tied embedding) and integer labels:
//   forward   lse_r  = log sum_j exp(x_rj),   loss_r = lse_r - x_r[label_r]
//   backward  g_rj   = s * (exp(x_rj - lse_r) - [j == label_r]),  s = *scale
// Rows whose label equals ignore_index give loss 0 and a zero gradient row
// (the forward of F.cross_entropy, whose default ignore_index is -100); any
// other label outside [0, vocab) gives a NaN loss and a NaN gradient row.
//
// The logits GEMMs stay with the BLAS library.  These kernels replace the
// softmax / cross-entropy / one-hot / scale passes over each logits block: the
// forward reads the block once (running maximum and rescaled sum of
// exponentials per thread, merged across the work-group), the backward reads
// it once and writes the gradient, in place when the caller passes the same
// buffer.  One 256-thread work-group per row; the row's interior moves in
// 16-byte vectors, its unaligned head and tail element-wise.  Exponentials run
// in base 2 on the hardware unit (v_exp_f32): exp(x - m) = 2^((x - m) log2 e),
// the difference taken first so the row maximum's term is exactly 1; terms
// below 2^-126 of the row maximum flush to zero.
#include "common.h"

#include <math.h>

namespace mogt {

constexpr int CE_THREADS = 256;
constexpr float CE_LOG2E = 1.4426950408889634f;

// Running (max, sum of exp(x - max)) of a thread.  An empty or all -inf state
// has m = -inf and s = 0; NaN inputs reach s through exp2(NaN).
struct RowMS {
    float m = -INFINITY, s = 0.0f;

    template <int N>
    __device__ __forceinline__ void add(const float (&v)[N]) {
        float vm = v[0];
#pragma unroll
        for (int i = 1; i < N; ++i) vm = fmaxf(vm, v[i]);
        if (vm > m) {
            s *= __builtin_amdgcn_exp2f((m - vm) * CE_LOG2E);   // m = -inf: s is 0 and stays 0
            m = vm;
        }
        const float mm = m == -INFINITY ? 0.0f : m;   // all -inf so far: every term is 0
#pragma unroll
        for (int i = 0; i < N; ++i) s += __builtin_amdgcn_exp2f((v[i] - mm) * CE_LOG2E);
    }
    __device__ __forceinline__ void merge(float m2, float s2) {
        const float M = fmaxf(m, m2);
        if (M == -INFINITY) {
            s += s2;
            return;
        }
        s = s * __builtin_amdgcn_exp2f((m - M) * CE_LOG2E) + s2 * __builtin_amdgcn_exp2f((m2 - M) * CE_LOG2E);
        m = M;
    }
};

// Elements of a row before its first 16-byte boundary (row pointers are
// element-aligned).
template <typename T>
__device__ __forceinline__ int64_t head_elems(const T* p, int64_t n) {
    const int64_t mis = static_cast<int64_t>(reinterpret_cast<uintptr_t>(p) & 15);
    const int64_t h = mis ? (16 - mis) / static_cast<int64_t>(sizeof(T)) : 0;
    return h < n ? h : n;
}

template <typename TL>
__global__ __launch_bounds__(CE_THREADS) void ce_fwd_kernel(const TL* __restrict__ logits, int64_t ld,
                                                            const int64_t* __restrict__ labels, int64_t vocab,
                                                            int64_t ignore, float* __restrict__ loss,
                                                            float* __restrict__ lse) {
    constexpr int VEC = 16 / sizeof(TL);
    __shared__ float sM[CE_THREADS / 64], sS[CE_THREADS / 64];
    const int64_t row = blockIdx.x;
    const TL* x = logits + row * ld;
    const int tid = threadIdx.x;
    RowMS acc;
    const int64_t h = head_elems(x, vocab);
    const int64_t nv = (vocab - h) / VEC;
    for (int64_t j = tid; j < h; j += CE_THREADS) {
        const float v[1] = {IO<TL>::ld(x[j])};
        acc.add(v);
    }
    const TL* xv = x + h;
    for (int64_t i = tid; i < nv; i += CE_THREADS) {
        float v[VEC];
        load_vec<TL, VEC>(xv + i * VEC, v);
        acc.add(v);
    }
    for (int64_t j = h + nv * VEC + tid; j < vocab; j += CE_THREADS) {
        const float v[1] = {IO<TL>::ld(x[j])};
        acc.add(v);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc.merge(__shfl_xor(acc.m, off, 64), __shfl_xor(acc.s, off, 64));
    if ((tid & 63) == 0) {
        sM[tid >> 6] = acc.m;
        sS[tid >> 6] = acc.s;
    }
    __syncthreads();
    if (tid == 0) {
        RowMS r;
#pragma unroll
        for (int w = 0; w < CE_THREADS / 64; ++w) r.merge(sM[w], sS[w]);
        const float l = r.m + logf(r.s);
        const int64_t lab = labels[row];
        float out;
        if (lab == ignore)
            out = 0.0f;
        else if (lab < 0 || lab >= vocab)
            out = __builtin_nanf("");
        else
            out = l - IO<TL>::ld(x[lab]);
        loss[row] = out;
        lse[row] = l;
    }
}

template <typename TL, typename TG>
__global__ __launch_bounds__(CE_THREADS) void ce_bwd_kernel(const TL* logits, int64_t ld,
                                                            const int64_t* __restrict__ labels,
                                                            const float* __restrict__ lse, int64_t vocab,
                                                            int64_t ignore, const float* __restrict__ scale,
                                                            TG* grad, int64_t ldg) {
    constexpr int VEC = 16 / sizeof(TL);
    const int64_t row = blockIdx.x;
    const TL* x = logits + row * ld;
    TG* g = grad + row * ldg;
    const int tid = threadIdx.x;
    const int64_t lab = labels[row];
    // exp(x - lse) = 2^((x - lse) log2 e); an ignored row is all zero, a label
    // outside the vocabulary poisons the row
    const bool skip = lab == ignore;
    const float bad = (!skip && (lab < 0 || lab >= vocab)) ? __builtin_nanf("") : 0.0f;
    const float lr = lse[row];
    const float sc = *scale;
    auto one = [&](int64_t j, float v) {
        const float p = __builtin_amdgcn_exp2f((v - lr) * CE_LOG2E) - (j == lab ? 1.0f : 0.0f);
        return skip ? 0.0f : p * sc + bad;
    };
    // both rows share one alignment only when the dtypes and strides agree; the
    // vector path needs the logits and gradient rows aligned together
    const int64_t h = head_elems(x, vocab);
    const bool vec_ok = sizeof(TL) == sizeof(TG) &&
                        ((reinterpret_cast<uintptr_t>(g + h) & 15) == 0);
    const int64_t nv = vec_ok ? (vocab - h) / VEC : 0;
    const int64_t h_end = vec_ok ? h : vocab;
    for (int64_t j = tid; j < h_end; j += CE_THREADS) g[j] = IO<TG>::st(one(j, IO<TL>::ld(x[j])));
    if (vec_ok) {
        for (int64_t i = tid; i < nv; i += CE_THREADS) {
            const int64_t j0 = h + i * VEC;
            float v[VEC], o[VEC];
            load_vec<TL, VEC>(x + j0, v);
#pragma unroll
            for (int e = 0; e < VEC; ++e) o[e] = one(j0 + e, v[e]);
            store_vec<TG, VEC>(g + j0, o);
        }
        for (int64_t j = h + nv * VEC + tid; j < vocab; j += CE_THREADS)
            g[j] = IO<TG>::st(one(j, IO<TL>::ld(x[j])));
    }
}

namespace {

bool ce_dt(int d) { return d == MOGT_F32 || d == MOGT_BF16; }

int ce_check(int64_t rows, int64_t vocab, int64_t ld, const char* what) {
    if (rows < 0 || vocab <= 0) return set_error(MOGT_E_INVALID, "%s: rows must be >= 0 and vocab > 0", what);
    if (ld < vocab) return set_error(MOGT_E_INVALID, "%s: row stride %lld < vocab %lld", what, (long long)ld,
                                     (long long)vocab);
    if (rows > 0x7fffffffLL) return set_error(MOGT_E_INVALID, "%s: more than 2^31 - 1 rows", what);
    return MOGT_OK;
}

}  // namespace
}  // namespace mogt

using namespace mogt;

extern "C" int mogt_lm_ce_fwd(const void* logits, int64_t ld, int logits_dtype, const int64_t* labels,
                              int64_t rows, int64_t vocab, int64_t ignore_index, float* loss_rows,
                              float* lse_rows, void* stream) {
    clear_error();
    int rc = ce_check(rows, vocab, ld, "lm_ce_fwd");
    if (rc) return rc;
    if (!ce_dt(logits_dtype)) return set_error(MOGT_E_INVALID, "lm_ce_fwd: logits dtype");
    if (rows == 0) return MOGT_OK;
    if (!logits || !labels || !loss_rows || !lse_rows) return set_error(MOGT_E_INVALID, "lm_ce_fwd: null pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid(static_cast<unsigned>(rows));
    if (logits_dtype == MOGT_F32)
        hipLaunchKernelGGL((ce_fwd_kernel<float>), grid, dim3(CE_THREADS), 0, st, static_cast<const float*>(logits),
                           ld, labels, vocab, ignore_index, loss_rows, lse_rows);
    else
        hipLaunchKernelGGL((ce_fwd_kernel<bf16_t>), grid, dim3(CE_THREADS), 0, st,
                           static_cast<const bf16_t*>(logits), ld, labels, vocab, ignore_index, loss_rows, lse_rows);
    return check_launch("ce_fwd_kernel");
}

extern "C" int mogt_lm_ce_bwd(const void* logits, int64_t ld, int logits_dtype, const int64_t* labels,
                              const float* lse_rows, int64_t rows, int64_t vocab, int64_t ignore_index,
                              const float* scale, void* grad, int64_t ld_grad, int grad_dtype, void* stream) {
    clear_error();
    int rc = ce_check(rows, vocab, ld, "lm_ce_bwd");
    if (rc) return rc;
    if (ld_grad < vocab) return set_error(MOGT_E_INVALID, "lm_ce_bwd: gradient row stride < vocab");
    if (!ce_dt(logits_dtype) || !ce_dt(grad_dtype)) return set_error(MOGT_E_INVALID, "lm_ce_bwd: dtype");
    if (grad == logits && (grad_dtype != logits_dtype || ld_grad != ld))
        return set_error(MOGT_E_INVALID, "lm_ce_bwd: in place needs the logits' dtype and row stride");
    if (rows == 0) return MOGT_OK;
    if (!logits || !labels || !lse_rows || !scale || !grad)
        return set_error(MOGT_E_INVALID, "lm_ce_bwd: null pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid(static_cast<unsigned>(rows));
#define MOGT_CE_BWD(TL, TG)                                                                           \
    hipLaunchKernelGGL((ce_bwd_kernel<TL, TG>), grid, dim3(CE_THREADS), 0, st, static_cast<const TL*>(logits), \
                       ld, labels, lse_rows, vocab, ignore_index, scale, static_cast<TG*>(grad), ld_grad)
    if (logits_dtype == MOGT_F32 && grad_dtype == MOGT_F32) MOGT_CE_BWD(float, float);
    else if (logits_dtype == MOGT_F32) MOGT_CE_BWD(float, bf16_t);
    else if (grad_dtype == MOGT_F32) MOGT_CE_BWD(bf16_t, float);
    else MOGT_CE_BWD(bf16_t, bf16_t);
#undef MOGT_CE_BWD
    return check_launch("ce_bwd_kernel");
}
