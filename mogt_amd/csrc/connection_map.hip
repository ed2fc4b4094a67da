// Connection maps of the MOGT transport for gfx950: per step, the r x r
// orthogonal transport U = damping * f(s A) of a skew-symmetric generator A
// (model_mogt.py:79-102):
//   f = exp   (connection_impl "matrix_exp", torch.matrix_exp)
//   f = Cayley: U = (I - X)^{-1} (I + X), X = s A / 2   ("cayley", torch.linalg.solve)
// One wave per matrix, r <= 32 as 16 x 16 tiles on fp32 MFMA
// (v_mfma_f32_16x16x4_f32).  A tile lives in "accumulator layout": lane
// (g = lane / 16, n = lane % 16) holds M[4g + i][n], i = 0..3, in one f32x4.
// The A operand of the MFMA needs the left factor's rows along lanes, which is
// the accumulator layout of its transpose; every left factor here is a
// polynomial in a skew X, whose transpose is mostly known without moving data
// (X^T = -X, symmetric matrices are their own transpose, exp(X)^T = exp(-X));
// the Newton-Schulz iterate of the Cayley map is transposed through LDS.
//
// exp:    scaling and squaring.  With 2^-k X of Frobenius norm <= 1/2,
//         Horner's rule of the degree-8 Taylor polynomial runs on E ~ exp(X)
//         and on F ~ exp(-X) = E^T together (remainder < 2^-9 / 9! / (1 -
//         1/20) = 5.7e-9, below fp32 rounding); k squarings E <- E E use F as
//         the transposed left factor and vice versa.
// Cayley: U = M^{-1} (I + X) with M = I - X.  M^{-1} comes from Newton-Schulz
//         iterations Y <- Y (2I - M Y) from Y = c M^T: with Z = X^T X
//         (symmetric positive semi-definite, lam = ||Z||_inf >= lambda_max(Z))
//         the first residual I - c (I + Z), c = 2 / (2 + lam), has norm
//         <= lam / (2 + lam) < 1 for any X, and the residual squares every step;
//         working on M itself (not on I + Z = M M^T) keeps the condition number
//         at cond(M) = sqrt(1 + lambda_max(Z)).  Y, the left factor of its own
//         update, is transposed exactly through LDS once per step (a
//         transpose carried as a separate iteration drifts by rounding).
#include "common.h"

#include <math.h>

namespace mogt {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int RT>
struct Mat {
    f32x4 t[RT][RT];
};

template <int RT>
__device__ __forceinline__ Mat<RT> mat_scaled_identity(float d) {
    const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
    Mat<RT> m;
#pragma unroll
    for (int a = 0; a < RT; ++a)
#pragma unroll
        for (int b = 0; b < RT; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) m.t[a][b][i] = (a == b && 4 * g + i == n) ? d : 0.0f;
    return m;
}

// alpha * P + beta * Q + d * I
template <int RT>
__device__ __forceinline__ Mat<RT> mat_comb(float alpha, const Mat<RT>& P, float beta, const Mat<RT>& Q,
                                            float d) {
    Mat<RT> m = mat_scaled_identity<RT>(d);
#pragma unroll
    for (int a = 0; a < RT; ++a)
#pragma unroll
        for (int b = 0; b < RT; ++b) m.t[a][b] = m.t[a][b] + alpha * P.t[a][b] + beta * Q.t[a][b];
    return m;
}

// L R with LT = L^T in accumulator layout, R in accumulator layout.
template <int RT>
__device__ __forceinline__ Mat<RT> mat_mul(const Mat<RT>& LT, const Mat<RT>& R) {
    Mat<RT> C;
#pragma unroll
    for (int a = 0; a < RT; ++a)
#pragma unroll
        for (int b = 0; b < RT; ++b) C.t[a][b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kt = 0; kt < RT; ++kt)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
#pragma unroll
            for (int a = 0; a < RT; ++a)
#pragma unroll
                for (int b = 0; b < RT; ++b)
                    C.t[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(LT.t[kt][a][kk], R.t[kt][b][kk], C.t[a][b],
                                                                     0, 0, 0);
    return C;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
    return x;
}

template <int RT>
__device__ __forceinline__ float mat_frob2(const Mat<RT>& m) {
    float s = 0.0f;
#pragma unroll
    for (int a = 0; a < RT; ++a)
#pragma unroll
        for (int b = 0; b < RT; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) s = fmaf(m.t[a][b][i], m.t[a][b][i], s);
    return wave_sum(s);
}

constexpr int CM_WAVES = 4;   // matrices per work-group

// M^T in accumulator layout through a per-wave LDS tile (row stride 33).  LDS
// executes one wave's accesses in issue order; the wave-scope fences only keep
// the compiler from reordering them.
template <int RT>
__device__ __forceinline__ Mat<RT> mat_transpose(const Mat<RT>& m, float (*sm)[33]) {
    const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
#pragma unroll
    for (int a = 0; a < RT; ++a)
#pragma unroll
        for (int b = 0; b < RT; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) sm[16 * a + 4 * g + i][16 * b + n] = m.t[a][b][i];
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    Mat<RT> t;
#pragma unroll
    for (int a = 0; a < RT; ++a)
#pragma unroll
        for (int b = 0; b < RT; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) t.t[a][b][i] = sm[16 * b + n][16 * a + 4 * g + i];
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    return t;
}

template <int RT, int IMPL, typename TO>
__global__ __launch_bounds__(64 * CM_WAVES) void connection_map_kernel(const float* __restrict__ A,
                                                                       TO* __restrict__ U, int64_t n,
                                                                       int r, float scale, float damping) {
    __shared__ float s_tr[CM_WAVES][32][33];
    const int64_t mi = static_cast<int64_t>(blockIdx.x) * CM_WAVES + (threadIdx.x >> 6);
    if (mi >= n) return;   // whole waves only: no wave-level operation is split
    float (*sm)[33] = s_tr[threadIdx.x >> 6];
    const int lane = threadIdx.x & 63, g = lane >> 4, nn = lane & 15;
    const float* src = A + mi * r * r;
    // X = scale * A (IMPL 0) or scale * A / 2 (Cayley), zero outside r x r
    const float xs = IMPL == 0 ? scale : 0.5f * scale;
    Mat<RT> X;
#pragma unroll
    for (int a = 0; a < RT; ++a)
#pragma unroll
        for (int b = 0; b < RT; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = 16 * a + 4 * g + i, col = 16 * b + nn;
                X.t[a][b][i] = (row < r && col < r) ? xs * src[row * r + col] : 0.0f;
            }
    const Mat<RT> zero = mat_scaled_identity<RT>(0.0f);
    const float lam = mat_frob2(X);   // ||X||_F^2, uniform across the wave

    Mat<RT> out;
    if constexpr (IMPL == 0) {
        // scaling: 2^-k X with ||.||_F <= 1/2, i.e. k >= log2(||X||_F) + 1
        int k = 0;
        if (lam > 0.25f) {
            const float kf = ceilf(0.5f * log2f(lam)) + 1.0f;   // inf stays inf: capped
            k = kf < 64.0f ? static_cast<int>(kf) : 64;
        }
        const float sc = exp2f(static_cast<float>(-k));
        Mat<RT> Xn = mat_comb<RT>(-sc, X, 0.0f, zero, 0.0f);   // (2^-k X)^T = -2^-k X
        Mat<RT> Xp = mat_comb<RT>(sc, X, 0.0f, zero, 0.0f);    // (-2^-k X)^T
        Mat<RT> E = mat_scaled_identity<RT>(1.0f), F = E;
        for (int m = 8; m >= 1; --m) {
            const float inv = 1.0f / static_cast<float>(m);
            E = mat_comb<RT>(inv, mat_mul<RT>(Xn, E), 0.0f, zero, 1.0f);   // I + X E / m
            F = mat_comb<RT>(inv, mat_mul<RT>(Xp, F), 0.0f, zero, 1.0f);   // I - X F / m
        }
        for (int s = 0; s < k; ++s) {
            const Mat<RT> E2 = mat_mul<RT>(F, E);   // E^T = F
            const Mat<RT> F2 = mat_mul<RT>(E, F);
            E = E2;
            F = F2;
        }
        out = E;
    } else {
        const Mat<RT> Z = mat_mul<RT>(X, X);                       // X^T X: (X^T)^T = X
        // lam = ||Z||_inf >= lambda_max(Z): the spectrum of I + Z is in [1, 1 + lam]
        float lam = 0.0f;
        {
            float rows[RT][4];
#pragma unroll
            for (int a = 0; a < RT; ++a)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float sum = 0.0f;
#pragma unroll
                    for (int b = 0; b < RT; ++b) sum += fabsf(Z.t[a][b][i]);
                    rows[a][i] = sum;
                }
            // sum over the 16 lanes of a row group (columns), then max over rows
#pragma unroll
            for (int off = 8; off >= 1; off >>= 1)
#pragma unroll
                for (int a = 0; a < RT; ++a)
#pragma unroll
                    for (int i = 0; i < 4; ++i) rows[a][i] += __shfl_xor(rows[a][i], off, 64);
#pragma unroll
            for (int a = 0; a < RT; ++a)
#pragma unroll
                for (int i = 0; i < 4; ++i) lam = fmaxf(lam, rows[a][i]);
#pragma unroll
            for (int off = 32; off >= 16; off >>= 1) lam = fmaxf(lam, __shfl_xor(lam, off, 64));
        }
        // M^{-1} (M = I - X) by Newton-Schulz from Y_0 = c M^T, c = 2 / (2 + lam):
        // the residual I - M Y_0 = I - c (I + Z) has norm <= lam / (2 + lam) < 1
        // and squares every step.  Y is the left factor of its own update, so its
        // exact transpose is formed (LDS) once per step.
        const float c = 2.0f / (2.0f + lam);
        const float w = lam / (2.0f + lam);
        int K = 1;
        if (w > 1e-8f) K = min(30, static_cast<int>(ceilf(log2f(fmaxf(-26.0f / log2f(w), 1.0f)))) + 1);
        const Mat<RT> Mp = mat_comb<RT>(1.0f, X, 0.0f, zero, 1.0f);    // I + X = M^T
        Mat<RT> Y = mat_comb<RT>(c, Mp, 0.0f, zero, 0.0f);            // c M^T
        for (int k = 0; k < K; ++k) {
            const Mat<RT> T = mat_mul<RT>(Mp, Y);     // M Y   (M^T = I + X is M's transpose)
            Y = mat_mul<RT>(mat_transpose<RT>(Y, sm), mat_comb<RT>(-1.0f, T, 0.0f, zero, 2.0f));
        }
        out = mat_mul<RT>(mat_transpose<RT>(Y, sm), Mp);   // U = M^{-1} (I + X)
    }
    TO* dst = U + mi * r * r;
#pragma unroll
    for (int a = 0; a < RT; ++a)
#pragma unroll
        for (int b = 0; b < RT; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = 16 * a + 4 * g + i, col = 16 * b + nn;
                if (row < r && col < r) dst[row * r + col] = IO<TO>::st(damping * out.t[a][b][i]);
            }
}

template <int IMPL, typename TO>
int launch_cm(const float* A, void* U, int64_t n, int r, float scale, float damping, hipStream_t st) {
    const dim3 grid(static_cast<unsigned>((n + CM_WAVES - 1) / CM_WAVES));
    if (r <= 16)
        hipLaunchKernelGGL((connection_map_kernel<1, IMPL, TO>), grid, dim3(64 * CM_WAVES), 0, st, A,
                           static_cast<TO*>(U), n, r, scale, damping);
    else
        hipLaunchKernelGGL((connection_map_kernel<2, IMPL, TO>), grid, dim3(64 * CM_WAVES), 0, st, A,
                           static_cast<TO*>(U), n, r, scale, damping);
    return check_launch("connection_map_kernel");
}

}  // namespace
}  // namespace mogt

using namespace mogt;

extern "C" int mogt_connection_map_fwd(const void* A, void* U, int64_t count, int64_t rank, float scale,
                                       float damping, int impl, int out_dtype, void* stream) {
    clear_error();
    if (count < 0 || rank <= 0) return set_error(MOGT_E_INVALID, "A must be [N, r, r] with r >= 1");
    if (rank > 32) return set_error(MOGT_E_INVALID, "r = %lld not supported (r <= 32)", (long long)rank);
    if (impl != MOGT_CONN_EXP && impl != MOGT_CONN_CAYLEY)
        return set_error(MOGT_E_INVALID, "unknown connection map %d", impl);
    if (out_dtype != MOGT_F32 && out_dtype != MOGT_BF16) return set_error(MOGT_E_INVALID, "unsupported output dtype");
    if (count == 0) return MOGT_OK;
    if (!A || !U) return set_error(MOGT_E_INVALID, "null tensor pointer");
    if ((count + CM_WAVES - 1) / CM_WAVES > 0x7fffffffLL) return set_error(MOGT_E_INVALID, "too many matrices");
    const int r = static_cast<int>(rank);
    const float* a = static_cast<const float*>(A);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (impl == MOGT_CONN_EXP)
        return out_dtype == MOGT_F32 ? launch_cm<0, float>(a, U, count, r, scale, damping, st)
                                     : launch_cm<0, bf16_t>(a, U, count, r, scale, damping, st);
    return out_dtype == MOGT_F32 ? launch_cm<1, float>(a, U, count, r, scale, damping, st)
                                 : launch_cm<1, bf16_t>(a, U, count, r, scale, damping, st);
}
