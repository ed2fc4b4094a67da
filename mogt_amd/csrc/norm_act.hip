// Fused row-wise kernels of the MOGT block (model_mogt.py:9-30, 238-256):
//   rmsnorm       out = (x * rsqrt(mean(x^2) + eps)).type_as(x) * w
//   add_rmsnorm   x' = x + round(s * z);  out = rmsnorm(x') * w   (residual + norm)
//   silu_mul      out = silu(y[:, :H]) * y[:, H:]                   (SwiGLU gate)
// Each rounds to bf16 at the points where the reference's bf16 tensors do, so
// results track the reference's autocast dtype flow; statistics are fp32.
// One wave per row: lanes hold 4-element vectors of the row (coalesced 16 B
// loads), the sum of squares is reduced across the wave with cross-lane
// shuffles, and the row is written once.
#include "common.h"

#include <initializer_list>

namespace mogt {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

template <typename T> __device__ __forceinline__ float rnd(float v) { return IO<T>::ld(IO<T>::st(v)); }

constexpr int NA_WAVES = 4;   // rows per work-group

// VPL = 4-element vectors per lane (row length <= 256 * VPL).
// ROWSCALE (with ADD): z is a read-out computed from an unnormalised input
// row, zr = W diag(w_out) h; the row's RMSNorm factor r = rsqrt(sum of the
// n_stat partial sums of squares of h / D + stat_eps) turns it into
// Z = round(r zr) = theta_read(norm_out(h)) before the residual update.
template <typename TX, typename TZ, typename TO, int VPL, bool ADD, bool ROWSCALE = false>
__global__ __launch_bounds__(64 * NA_WAVES) void rmsnorm_kernel(
    const TX* __restrict__ x, const TZ* __restrict__ z, float scale, const float* __restrict__ w,
    float* __restrict__ x_out, TO* __restrict__ out, int64_t rows, int D, float eps,
    const float* __restrict__ rowstat = nullptr, int n_stat = 0, float stat_eps = 0.0f) {
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * NA_WAVES + (threadIdx.x >> 6);
    if (row >= rows) return;
    const TX* xr = x + row * D;
    float zscale = 1.0f;
    if constexpr (ROWSCALE) {
        float t = 0.0f;
        for (int i = lane; i < n_stat; i += 64) t += rowstat[row * n_stat + i];
        zscale = rsqrtf(wave_sum(t) / static_cast<float>(D) + stat_eps);
    }
    float v[VPL][4];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        const int c = (k * 64 + lane) * 4;
        if (c < D) {
            load_vec<TX, 4>(xr + c, v[k]);
            if constexpr (ADD) {
                float zz[4];
                load_vec<TZ, 4>(z + row * D + c, zz);
                if constexpr (ROWSCALE) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) zz[e] = rnd<TZ>(zscale * zz[e]);
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) v[k][e] += rnd<TZ>(scale * zz[e]);
                if (x_out) store_vec<float, 4>(x_out + row * D + c, v[k]);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) ss = fmaf(v[k][e], v[k][e], ss);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[k][e] = 0.0f;
        }
    }
    const float inv = rsqrtf(wave_sum(ss) / static_cast<float>(D) + eps);
    TO* orow = out + row * D;
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        const int c = (k * 64 + lane) * 4;
        if (c < D) {
            float ww[4], o[4];
            load_vec<float, 4>(w + c, ww);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                // .type_as(x): the normalised value takes the input's dtype first
                const float nrm = ADD ? v[k][e] * inv : rnd<TX>(v[k][e] * inv);
                o[e] = nrm * ww[e];
            }
            store_vec<TO, 4>(orow + c, o);
        }
    }
}

// The SwiGLU row kernels walk the flattened [rows, H / VEC] vector index with a
// grid stride; a thread's first (row, column) is one division and later ones
// advance by the stride's quotient and remainder (no 64-bit division per
// vector: these kernels are otherwise VALU-bound on the division alone).
struct RowWalk {
    int64_t i, r, c, S, sq, sr, hv;
    __device__ RowWalk(int64_t hv_) : hv(hv_) {
        S = static_cast<int64_t>(gridDim.x) * blockDim.x;
        i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
        r = i / hv;
        c = i - r * hv;
        sq = S / hv;
        sr = S - sq * hv;
    }
    __device__ __forceinline__ void next() {
        i += S;
        r += sq;
        c += sr;
        if (c >= hv) {
            c -= hv;
            ++r;
        }
    }
};

// SwiGLU gate (model_mogt.py:29-30): out = silu(a) * b for y = [a | b] rows.
template <typename T, int VEC>
__global__ __launch_bounds__(256) void silu_mul_kernel(const T* __restrict__ y, T* __restrict__ out,
                                                       int64_t rows, int64_t H) {
    const int64_t nvec = rows * (H / VEC);
    for (RowWalk w(H / VEC); w.i < nvec; w.next()) {
        const T* ya = y + w.r * 2 * H + w.c * VEC;
        float a[VEC], b[VEC], o[VEC];
        load_vec<T, VEC>(ya, a);
        load_vec<T, VEC>(ya + H, b);
#pragma unroll
        for (int k = 0; k < VEC; ++k) o[k] = rnd<T>(a[k] * sigmoid_hw(a[k])) * b[k];   // F.silu on T
        store_vec<T, VEC>(out + w.r * H + w.c * VEC, o);
    }
}

// Backward of rmsnorm / add_rmsnorm (model_mogt.py:15-20).  With r =
// rsqrt(mean(x^2) + eps), n = x r, n_t = n rounded to x's dtype (the
// .type_as(x); a no-op for the fp32 residual of add_rmsnorm) and y = n_t w:
//   dw = sum over rows of dy n_t
//   dx = r (dn - n mean(dn n)) + dres,   dn = dy w
// (the rounding of n_t passes the gradient straight through, as autograd of
// the reference's expression does).  One wave per group of rows_per_wave rows:
// each lane keeps its columns' dw sums in registers and the wave writes one
// partial row, which the caller sums; dres (the residual stream's own
// gradient, add_rmsnorm) may be null.
template <typename TX, typename TG, int VPL>
__global__ __launch_bounds__(64 * NA_WAVES) void rmsnorm_bwd_kernel(
    const TX* __restrict__ x, const float* __restrict__ w, const TG* __restrict__ dy,
    const float* __restrict__ dres, TX* __restrict__ dx, float* __restrict__ dw_part, int64_t rows, int D,
    float eps, int rows_per_wave, void* __restrict__ dz, float dz_scale, int dz_bf16) {
    extern __shared__ float dw_lds[];   // [NA_WAVES][D]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t gw = static_cast<int64_t>(blockIdx.x) * NA_WAVES + wave;
    const int64_t r0 = gw * rows_per_wave;
    // a wave past the last row has no rows but still joins the group's dw sum
    const int64_t r1 = r0 >= rows ? r0 : (r0 + rows_per_wave < rows ? r0 + rows_per_wave : rows);
    float ww[VPL][4], acc[VPL][4];
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        const int c = (k * 64 + lane) * 4;
#pragma unroll
        for (int e = 0; e < 4; ++e) ww[k][e] = acc[k][e] = 0.0f;
        if (c < D) load_vec<float, 4>(w + c, ww[k]);
    }
    const float inv_d = 1.0f / static_cast<float>(D);
    // x, dy and dres of a row (zeros past D); the next row's are in flight
    // while the current one reduces
    auto load_row = [&](int64_t row, float (&v)[VPL][4], float (&g)[VPL][4], float (&rr)[VPL][4]) {
#pragma unroll
        for (int k = 0; k < VPL; ++k) {
            const int c = (k * 64 + lane) * 4;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[k][e] = g[k][e] = rr[k][e] = 0.0f;
            if (c < D) {
                load_vec<TX, 4>(x + row * D + c, v[k]);
                load_vec<TG, 4>(dy + row * D + c, g[k]);
                if (dres) load_vec<float, 4>(dres + row * D + c, rr[k]);
            }
        }
    };
    float v[VPL][4], g[VPL][4], rr[VPL][4];
    if (r0 < r1) load_row(r0, v, g, rr);
    for (int64_t row = r0; row < r1; ++row) {
        float vn[VPL][4], gn[VPL][4], rn[VPL][4];
        if (row + 1 < r1) load_row(row + 1, vn, gn, rn);
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < VPL; ++k)
#pragma unroll
            for (int e = 0; e < 4; ++e) ss = fmaf(v[k][e], v[k][e], ss);
        const float r = rsqrtf(wave_sum(ss) * inv_d + eps);
        float dot = 0.0f;
#pragma unroll
        for (int k = 0; k < VPL; ++k)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float n = v[k][e] * r;
                acc[k][e] = fmaf(g[k][e], rnd<TX>(n), acc[k][e]);
                g[k][e] *= ww[k][e];   // dn
                dot = fmaf(g[k][e], n, dot);
            }
        const float mdot = wave_sum(dot) * inv_d;
#pragma unroll
        for (int k = 0; k < VPL; ++k) {
            const int c = (k * 64 + lane) * 4;
            if (c < D) {
                float o[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = r * (g[k][e] - v[k][e] * r * mdot) + rr[k][e];
                store_vec<TX, 4>(dx + row * D + c, o);
                if (dz) {   // the gradient of the scaled term: (dx * scale) in z's dtype
                    float oz[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) oz[e] = rnd<TX>(o[e]) * dz_scale;
                    if (dz_bf16)
                        store_vec<bf16_t, 4>(static_cast<bf16_t*>(dz) + row * D + c, oz);
                    else
                        store_vec<float, 4>(static_cast<float*>(dz) + row * D + c, oz);
                }
            }
        }
        if (row + 1 < r1) {
#pragma unroll
            for (int k = 0; k < VPL; ++k)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[k][e] = vn[k][e];
                    g[k][e] = gn[k][e];
                    rr[k][e] = rn[k][e];
                }
        }
    }
    // the group's waves' dw partials summed in wave order (deterministic):
    // one partial per work-group and feature, stored feature-major
    // ([D][groups]) so the caller's sum runs along contiguous memory
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        const int c = (k * 64 + lane) * 4;
        if (c < D) store_vec<float, 4>(dw_lds + wave * D + c, acc[k]);
    }
    __syncthreads();
    for (int c = threadIdx.x; c < D; c += 64 * NA_WAVES) {
        float t = dw_lds[c];
#pragma unroll
        for (int q = 1; q < NA_WAVES; ++q) t += dw_lds[q * D + c];
        dw_part[static_cast<int64_t>(c) * gridDim.x + blockIdx.x] = t;
    }
}

// Backward of silu_mul: with a = y[:, :H], b = y[:, H:], s = silu(a) rounded to
// the tensor dtype (as in the forward), out = s b:
//   db = d s,   ds = d b,   da = ds sigmoid(a) (1 + a (1 - sigmoid(a)))
// each rounded to the dtype where torch's bf16 autograd rounds (mul backward,
// then silu_backward in fp32 and cast).  dy = [da | db], the gradient of the
// fused [w1; w2] projection's output.
template <typename T, int VEC>
__global__ __launch_bounds__(256) void silu_mul_bwd_kernel(const T* __restrict__ y, const T* __restrict__ dout,
                                                           T* __restrict__ dy, int64_t rows, int64_t H) {
    const int64_t nvec = rows * (H / VEC);
    for (RowWalk w(H / VEC); w.i < nvec; w.next()) {
        const int64_t ia = w.r * 2 * H + w.c * VEC;
        float a[VEC], b[VEC], d[VEC], da[VEC], db[VEC];
        load_vec<T, VEC>(y + ia, a);
        load_vec<T, VEC>(y + ia + H, b);
        load_vec<T, VEC>(dout + w.r * H + w.c * VEC, d);
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
            const float sg = sigmoid_hw(a[k]);
            db[k] = d[k] * rnd<T>(a[k] * sg);
            const float ds = rnd<T>(d[k] * b[k]);
            da[k] = ds * sg * (1.0f + a[k] * (1.0f - sg));
        }
        store_vec<T, VEC>(dy + ia, da);
        store_vec<T, VEC>(dy + ia + H, db);
    }
}

namespace {

bool dt_ok(int d) { return d == MOGT_F32 || d == MOGT_BF16; }

// Widest vector (elements, at most 16 bytes) that divides the hidden width and
// that every pointer is aligned to.
int swiglu_vec(int64_t hidden, size_t esz, std::initializer_list<const void*> ptrs) {
    for (int v : {8, 4, 2}) {
        if (v * esz > 16 || hidden % v) continue;
        bool ok = true;
        for (const void* p : ptrs) ok = ok && reinterpret_cast<uintptr_t>(p) % (v * esz) == 0;
        if (ok) return v;
    }
    return 1;
}
dim3 swiglu_grid(int64_t rows, int64_t hidden, int vec) {
    const int64_t nvec = rows * (hidden / vec);
    return dim3(static_cast<unsigned>(nvec / 256 + 1 < 8192 ? nvec / 256 + 1 : 8192));
}

template <typename TX, typename TG>
int launch_norm_bwd(const void* x, const float* w, const void* dy, const float* dres, void* dx, float* dw_part,
                    int64_t rows, int D, float eps, int rpw, void* dz, float dz_scale, int dz_bf16,
                    hipStream_t st) {
    const int vpl = (D + 255) / 256;
    const int64_t waves = (rows + rpw - 1) / rpw;
    const dim3 grid(static_cast<unsigned>((waves + NA_WAVES - 1) / NA_WAVES));
    const dim3 block(64 * NA_WAVES);
    const size_t lds = static_cast<size_t>(NA_WAVES) * D * sizeof(float);
    const TX* xp = static_cast<const TX*>(x);
    const TG* gp = static_cast<const TG*>(dy);
    TX* dxp = static_cast<TX*>(dx);
#define MOGT_NORM_BWD_CASE(V)                                                                     \
    if (vpl <= V) {                                                                                \
        hipLaunchKernelGGL((rmsnorm_bwd_kernel<TX, TG, V>), grid, block, lds, st, xp, w, gp, dres, dxp, \
                           dw_part, rows, D, eps, rpw, dz, dz_scale, dz_bf16);                      \
        return check_launch("rmsnorm_bwd_kernel");                                                 \
    }
    MOGT_NORM_BWD_CASE(1)
    MOGT_NORM_BWD_CASE(2)
    MOGT_NORM_BWD_CASE(3)
    MOGT_NORM_BWD_CASE(4)
    MOGT_NORM_BWD_CASE(8)
    MOGT_NORM_BWD_CASE(16)
#undef MOGT_NORM_BWD_CASE
    return set_error(MOGT_E_INVALID, "rmsnorm_bwd: row length %d > 4096", D);
}

template <typename TX, typename TZ, typename TO, bool ADD, bool ROWSCALE = false>
int launch_norm(const void* x, const void* z, float scale, const float* w, float* x_out, void* out,
                int64_t rows, int D, float eps, hipStream_t st, const float* rowstat = nullptr, int n_stat = 0,
                float stat_eps = 0.0f) {
    const int vpl = (D + 255) / 256;
    const dim3 grid(static_cast<unsigned>((rows + NA_WAVES - 1) / NA_WAVES));
    const dim3 block(64 * NA_WAVES);
    const TX* xp = static_cast<const TX*>(x);
    const TZ* zp = static_cast<const TZ*>(z);
    TO* op = static_cast<TO*>(out);
#define MOGT_NORM_CASE(V)                                                                            \
    if (vpl <= V) {                                                                                   \
        hipLaunchKernelGGL((rmsnorm_kernel<TX, TZ, TO, V, ADD, ROWSCALE>), grid, block, 0, st, xp, zp, \
                           scale, w, x_out, op, rows, D, eps, rowstat, n_stat, stat_eps);             \
        return check_launch("rmsnorm_kernel");                                                        \
    }
    MOGT_NORM_CASE(1)
    MOGT_NORM_CASE(2)
    MOGT_NORM_CASE(3)
    MOGT_NORM_CASE(4)
    MOGT_NORM_CASE(8)
    MOGT_NORM_CASE(16)
#undef MOGT_NORM_CASE
    return set_error(MOGT_E_INVALID, "rmsnorm: row length %d > 4096", D);
}

int check_norm_args(int64_t rows, int64_t dim) {
    if (rows < 0 || dim <= 0) return set_error(MOGT_E_INVALID, "rmsnorm: bad shape");
    if (dim % 4 != 0) return set_error(MOGT_E_INVALID, "rmsnorm: row length must be a multiple of 4");
    if (dim > 4096) return set_error(MOGT_E_INVALID, "rmsnorm: row length %lld > 4096", (long long)dim);
    return MOGT_OK;
}

}  // namespace
}  // namespace mogt

using namespace mogt;

extern "C" int mogt_rmsnorm_fwd(const void* x, const float* weight, void* out, int64_t rows, int64_t dim,
                                float eps, int x_dtype, int out_dtype, void* stream) {
    clear_error();
    int rc = check_norm_args(rows, dim);
    if (rc) return rc;
    if (!dt_ok(x_dtype) || !dt_ok(out_dtype)) return set_error(MOGT_E_INVALID, "rmsnorm: dtype");
    if (rows == 0) return MOGT_OK;
    if (!x || !weight || !out) return set_error(MOGT_E_INVALID, "rmsnorm: null pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int D = static_cast<int>(dim);
    if (x_dtype == MOGT_F32 && out_dtype == MOGT_F32)
        return launch_norm<float, float, float, false>(x, nullptr, 0.f, weight, nullptr, out, rows, D, eps, st);
    if (x_dtype == MOGT_F32 && out_dtype == MOGT_BF16)
        return launch_norm<float, float, bf16_t, false>(x, nullptr, 0.f, weight, nullptr, out, rows, D, eps, st);
    if (x_dtype == MOGT_BF16 && out_dtype == MOGT_F32)
        return launch_norm<bf16_t, float, float, false>(x, nullptr, 0.f, weight, nullptr, out, rows, D, eps, st);
    return launch_norm<bf16_t, float, bf16_t, false>(x, nullptr, 0.f, weight, nullptr, out, rows, D, eps, st);
}

extern "C" int mogt_add_rmsnorm_fwd(const float* x, const void* z, float scale, const float* weight,
                                    float* x_out, void* out, int64_t rows, int64_t dim, float eps,
                                    int z_dtype, int out_dtype, void* stream) {
    clear_error();
    int rc = check_norm_args(rows, dim);
    if (rc) return rc;
    if (!dt_ok(z_dtype) || !dt_ok(out_dtype)) return set_error(MOGT_E_INVALID, "add_rmsnorm: dtype");
    if (rows == 0) return MOGT_OK;
    if (!x || !z || !weight || !out) return set_error(MOGT_E_INVALID, "add_rmsnorm: null pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int D = static_cast<int>(dim);
    if (z_dtype == MOGT_F32 && out_dtype == MOGT_F32)
        return launch_norm<float, float, float, true>(x, z, scale, weight, x_out, out, rows, D, eps, st);
    if (z_dtype == MOGT_F32 && out_dtype == MOGT_BF16)
        return launch_norm<float, float, bf16_t, true>(x, z, scale, weight, x_out, out, rows, D, eps, st);
    if (z_dtype == MOGT_BF16 && out_dtype == MOGT_F32)
        return launch_norm<float, bf16_t, float, true>(x, z, scale, weight, x_out, out, rows, D, eps, st);
    return launch_norm<float, bf16_t, bf16_t, true>(x, z, scale, weight, x_out, out, rows, D, eps, st);
}

extern "C" int mogt_add_rmsnorm_rowscale_fwd(const float* x, const void* z, const float* row_stats,
                                             int64_t n_stats, float stat_eps, float scale, const float* weight,
                                             float* x_out, void* out, int64_t rows, int64_t dim, float eps,
                                             int z_dtype, int out_dtype, void* stream) {
    clear_error();
    int rc = check_norm_args(rows, dim);
    if (rc) return rc;
    if (!dt_ok(z_dtype) || !dt_ok(out_dtype)) return set_error(MOGT_E_INVALID, "add_rmsnorm_rowscale: dtype");
    if (n_stats <= 0 || n_stats > 4096)
        return set_error(MOGT_E_INVALID, "add_rmsnorm_rowscale: 1 <= n_stats <= 4096");
    if (rows == 0) return MOGT_OK;
    if (!x || !z || !row_stats || !weight || !x_out || !out)
        return set_error(MOGT_E_INVALID, "add_rmsnorm_rowscale: null pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int D = static_cast<int>(dim), ns = static_cast<int>(n_stats);
    if (z_dtype == MOGT_F32 && out_dtype == MOGT_F32)
        return launch_norm<float, float, float, true, true>(x, z, scale, weight, x_out, out, rows, D, eps, st,
                                                            row_stats, ns, stat_eps);
    if (z_dtype == MOGT_F32 && out_dtype == MOGT_BF16)
        return launch_norm<float, float, bf16_t, true, true>(x, z, scale, weight, x_out, out, rows, D, eps, st,
                                                             row_stats, ns, stat_eps);
    if (z_dtype == MOGT_BF16 && out_dtype == MOGT_F32)
        return launch_norm<float, bf16_t, float, true, true>(x, z, scale, weight, x_out, out, rows, D, eps, st,
                                                             row_stats, ns, stat_eps);
    return launch_norm<float, bf16_t, bf16_t, true, true>(x, z, scale, weight, x_out, out, rows, D, eps, st,
                                                          row_stats, ns, stat_eps);
}

extern "C" int mogt_silu_mul_fwd(const void* y, void* out, int64_t rows, int64_t hidden, int dtype,
                                 void* stream) {
    clear_error();
    if (rows < 0 || hidden <= 0 || hidden % 4 != 0)
        return set_error(MOGT_E_INVALID, "silu_mul: hidden must be a positive multiple of 4");
    if (!dt_ok(dtype)) return set_error(MOGT_E_INVALID, "silu_mul: dtype");
    if (rows == 0) return MOGT_OK;
    if (!y || !out) return set_error(MOGT_E_INVALID, "silu_mul: null pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const size_t esz = dtype == MOGT_F32 ? 4 : 2;
    const int vec = swiglu_vec(hidden, esz, {y, out});
    const dim3 grid = swiglu_grid(rows, hidden, vec);
#define MOGT_SILU_CASE(T, V)                                                                                      \
    if (vec == V) {                                                                                               \
        hipLaunchKernelGGL((silu_mul_kernel<T, V>), grid, dim3(256), 0, st, static_cast<const T*>(y),              \
                           static_cast<T*>(out), rows, hidden);                                                   \
        return check_launch("silu_mul_kernel");                                                                   \
    }
    if (dtype == MOGT_F32) {
        MOGT_SILU_CASE(float, 4) MOGT_SILU_CASE(float, 2) MOGT_SILU_CASE(float, 1)
    } else {
        MOGT_SILU_CASE(bf16_t, 8) MOGT_SILU_CASE(bf16_t, 4) MOGT_SILU_CASE(bf16_t, 2) MOGT_SILU_CASE(bf16_t, 1)
    }
#undef MOGT_SILU_CASE
    return set_error(MOGT_E_INVALID, "silu_mul: no vector width");
}

extern "C" int mogt_rmsnorm_bwd(const void* x, const float* weight, const void* dy, const float* dres, void* dx,
                                float* dw_partial, int64_t rows, int64_t dim, float eps, int rows_per_wave,
                                int x_dtype, int dy_dtype, void* dz, float dz_scale, int dz_dtype,
                                void* stream) {
    clear_error();
    int rc = check_norm_args(rows, dim);
    if (rc) return rc;
    if (!dt_ok(x_dtype) || !dt_ok(dy_dtype) || (dz && !dt_ok(dz_dtype)))
        return set_error(MOGT_E_INVALID, "rmsnorm_bwd: dtype");
    if (rows_per_wave <= 0) return set_error(MOGT_E_INVALID, "rmsnorm_bwd: rows_per_wave must be positive");
    if (dres && x_dtype != MOGT_F32)
        return set_error(MOGT_E_INVALID, "rmsnorm_bwd: a residual gradient needs the fp32 residual stream");
    if (rows == 0) return MOGT_OK;
    if (!x || !weight || !dy || !dx || !dw_partial) return set_error(MOGT_E_INVALID, "rmsnorm_bwd: null pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int D = static_cast<int>(dim);
    if (x_dtype == MOGT_F32 && dy_dtype == MOGT_F32)
        return launch_norm_bwd<float, float>(x, weight, dy, dres, dx, dw_partial, rows, D, eps, rows_per_wave, dz,
                                         dz_scale, dz_dtype == MOGT_BF16, st);
    if (x_dtype == MOGT_F32)
        return launch_norm_bwd<float, bf16_t>(x, weight, dy, dres, dx, dw_partial, rows, D, eps, rows_per_wave, dz,
                                         dz_scale, dz_dtype == MOGT_BF16, st);
    if (dy_dtype == MOGT_F32)
        return launch_norm_bwd<bf16_t, float>(x, weight, dy, dres, dx, dw_partial, rows, D, eps, rows_per_wave, dz,
                                         dz_scale, dz_dtype == MOGT_BF16, st);
    return launch_norm_bwd<bf16_t, bf16_t>(x, weight, dy, dres, dx, dw_partial, rows, D, eps, rows_per_wave, dz,
                                         dz_scale, dz_dtype == MOGT_BF16, st);
}

extern "C" int mogt_silu_mul_bwd(const void* y, const void* dout, void* dy, int64_t rows, int64_t hidden,
                                 int dtype, void* stream) {
    clear_error();
    if (rows < 0 || hidden <= 0 || hidden % 4 != 0)
        return set_error(MOGT_E_INVALID, "silu_mul_bwd: hidden must be a positive multiple of 4");
    if (!dt_ok(dtype)) return set_error(MOGT_E_INVALID, "silu_mul_bwd: dtype");
    if (rows == 0) return MOGT_OK;
    if (!y || !dout || !dy) return set_error(MOGT_E_INVALID, "silu_mul_bwd: null pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const size_t esz = dtype == MOGT_F32 ? 4 : 2;
    const int vec = swiglu_vec(hidden, esz, {y, dout, dy});
    const dim3 grid = swiglu_grid(rows, hidden, vec);
#define MOGT_SILU_BWD_CASE(T, V)                                                                                  \
    if (vec == V) {                                                                                               \
        hipLaunchKernelGGL((silu_mul_bwd_kernel<T, V>), grid, dim3(256), 0, st, static_cast<const T*>(y),          \
                           static_cast<const T*>(dout), static_cast<T*>(dy), rows, hidden);                       \
        return check_launch("silu_mul_bwd_kernel");                                                               \
    }
    if (dtype == MOGT_F32) {
        MOGT_SILU_BWD_CASE(float, 4) MOGT_SILU_BWD_CASE(float, 2) MOGT_SILU_BWD_CASE(float, 1)
    } else {
        MOGT_SILU_BWD_CASE(bf16_t, 8) MOGT_SILU_BWD_CASE(bf16_t, 4) MOGT_SILU_BWD_CASE(bf16_t, 2)
        MOGT_SILU_BWD_CASE(bf16_t, 1)
    }
#undef MOGT_SILU_BWD_CASE
    return set_error(MOGT_E_INVALID, "silu_mul_bwd: no vector width");
}
