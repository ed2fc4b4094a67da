// Rank-1 coupled write-forget scan with readout, per (batch, head):
//   S_t = f_t S_{t-1} + (1 - f_t) v_t k_t^T,   y_t = S_t q_t,   S_0 = 0
// i.e. the affine recurrence of affine_scan.py:48-55 with U_t = f_t I and the
// rank-1 write V_t = (1 - f_t) v_t k_t^T, read out through q_t.  S_t (d x d per
// step) is never written to memory.  Chunked form over T steps, with
// Lc_t = sum_{u<=t} log f_u inside the chunk and S_in the state before it:
//   y_t  = exp(Lc_t) S_in q_t + sum_{s<=t} exp(Lc_t - Lc_s) (1 - f_s) (q_t . k_s) v_s
//   S_out = exp(Lc_T) S_in + sum_s exp(Lc_T - Lc_s) (1 - f_s) v_s k_s^T
// Three launches:
//   K_A  per chunk: dS = V^T diag(w) K on bf16 MFMA (32x32x16), chunk log-decay
//   K_B  per (sequence, state element): S_in(k) = exp(LcT(k-1)) S_in(k-1) + dS(k-1)
//        -- the chunk carries compose element-wise, so this is a plain scan
//   K_C  per chunk: (Q K^T masked by the decay) V + exp(Lc) Q S_in^T on MFMA; the
//        state operand is split into bf16 hi + lo parts for fp32-level accuracy.
// Layouts: f [B, L, H]; q, k, v, y [B, L, H, DH] (the reference's flattening).
#include "common.h"

namespace mogt {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int R1_DH = 64;        // head dimension
constexpr int R1_T = 64;         // chunk length
constexpr int R1_THREADS = 256;  // 4 waves
constexpr int R1_PAD = 8;        // LDS row padding (bf16): rows of 144 B, conflict-free 16 B reads
constexpr float R1_LOG_MIN = -80.0f;

struct Rank1Params {
    const void* f;
    const void* k;
    const void* v;
    const void* q;
    void* y;
    float* dS;      // [n_seq][nch][DH*DH]
    float* lcT;     // [n_seq][nch]
    float* Sin;     // [n_seq][nch][DH*DH]
    int64_t L;
    int H, nch;
};

// 32x32 fp32 tile += A[32 x K] B[K x 32]; A rows in `a` (row stride sa, k contiguous),
// B columns in `b` (column stride sb, k contiguous), both bf16 in LDS.
__device__ __forceinline__ f32x16 mma32(const bf16_t* a, int sa, const bf16_t* b, int sb, int K, f32x16 acc) {
    const int l = threadIdx.x & 63;
    for (int k0 = 0; k0 < K; k0 += 16) {
        const bf16x8 av = *reinterpret_cast<const bf16x8*>(a + (l & 31) * sa + k0 + 8 * (l >> 5));
        const bf16x8 bv = *reinterpret_cast<const bf16x8*>(b + (l & 31) * sb + k0 + 8 * (l >> 5));
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, acc, 0, 0, 0);
    }
    return acc;
}

// Row of the 32x32 output element held in register r by this lane (column = lane & 31).
__device__ __forceinline__ int mrow(int r) { return 8 * (r >> 2) + 4 * ((threadIdx.x & 63) >> 5) + (r & 3); }

__device__ __forceinline__ f32x16 zero16() {
    f32x16 z;
#pragma unroll
    for (int r = 0; r < 16; ++r) z[r] = 0.0f;
    return z;
}

// Inclusive prefix sum over the 64 lanes of a wave (shuffle-up scan).
__device__ __forceinline__ float wave_incl_scan(float x) {
    const int l = threadIdx.x & 63;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const float y = __shfl_up(x, off, 64);
        if (l >= off) x += y;
    }
    return x;
}

// Load a T x DH tile of q/k/v rows (zero past L) into LDS, row-major or transposed.
template <typename TI, bool TRANSPOSE>
__device__ __forceinline__ void load_rows(const TI* __restrict__ src, bf16_t* dst, int64_t rowbase,
                                          int64_t t0, int64_t L, int H) {
    constexpr int SEG = R1_DH / 8;   // 8-element segments per row
    for (int e = threadIdx.x; e < R1_T * SEG; e += R1_THREADS) {
        const int t = e / SEG, sg = e - (e / SEG) * SEG;
        float x[8];
        if (t0 + t < L) {
            load_vec<TI, 8>(src + (rowbase + (t0 + t) * H) * R1_DH + sg * 8, x);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) x[i] = 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const bf16_t bv = f32_to_bf16(x[i]);
            if (TRANSPOSE) dst[(sg * 8 + i) * (R1_T + R1_PAD) + t] = bv;
            else dst[t * (R1_DH + R1_PAD) + sg * 8 + i] = bv;
        }
    }
}

// Lc (inclusive log-decay cumsum) and 1 - f of the chunk into LDS (wave 0).
template <typename TF>
__device__ __forceinline__ void chunk_decay(const TF* __restrict__ f, int64_t fbase, int64_t t0, int64_t L, int H,
                                            float* sLc, float* sOmf) {
    if (threadIdx.x < 64) {
        const int t = threadIdx.x;
        float fv = 1.0f;
        if (t0 + t < L) fv = IO<TF>::ld(f[fbase + (t0 + t) * H]);
        const float lg = fmaxf(logf(fv), R1_LOG_MIN);
        sLc[t] = wave_incl_scan(lg);
        sOmf[t] = 1.0f - fv;
    }
}

template <typename TF, typename TI>
__global__ __launch_bounds__(R1_THREADS) void rank1_summary_kernel(Rank1Params p) {
    __shared__ __attribute__((aligned(16))) bf16_t sVT[R1_DH * (R1_T + R1_PAD)];
    __shared__ __attribute__((aligned(16))) bf16_t sKT[R1_DH * (R1_T + R1_PAD)];
    __shared__ float sLc[R1_T], sOmf[R1_T];
    const int kc = blockIdx.x;               // chunk
    const int seq = blockIdx.y;              // b * H + h
    const int b = seq / p.H, h = seq - (seq / p.H) * p.H;
    const int64_t t0 = static_cast<int64_t>(kc) * R1_T;
    const int64_t rowbase = static_cast<int64_t>(b) * p.L * p.H + h;   // (b*L + t)*H + h = rowbase + t*H
    load_rows<TI, true>(static_cast<const TI*>(p.v), sVT, rowbase, t0, p.L, p.H);
    load_rows<TI, true>(static_cast<const TI*>(p.k), sKT, rowbase, t0, p.L, p.H);
    chunk_decay<TF>(static_cast<const TF*>(p.f), rowbase, t0, p.L, p.H, sLc, sOmf);
    __syncthreads();
    // scale V^T columns by w_s = exp(LcT - Lc_s) (1 - f_s)
    const float lct = sLc[R1_T - 1];
    for (int e = threadIdx.x; e < R1_DH * R1_T; e += R1_THREADS) {
        const int i = e / R1_T, s = e - (e / R1_T) * R1_T;
        bf16_t& x = sVT[i * (R1_T + R1_PAD) + s];
        x = f32_to_bf16(bf16_to_f32(x) * expf(lct - sLc[s]) * sOmf[s]);
    }
    __syncthreads();
    const int w = threadIdx.x >> 6;           // output tile (ib, jb) of dS [i][j]
    const int ib = w >> 1, jb = w & 1;
    f32x16 acc = mma32(sVT + ib * 32 * (R1_T + R1_PAD), R1_T + R1_PAD,
                       sKT + jb * 32 * (R1_T + R1_PAD), R1_T + R1_PAD, R1_T, zero16());
    float* out = p.dS + (static_cast<int64_t>(seq) * p.nch + kc) * R1_DH * R1_DH;
    const int col = jb * 32 + (threadIdx.x & 31);
#pragma unroll
    for (int r = 0; r < 16; ++r) out[(ib * 32 + mrow(r)) * R1_DH + col] = acc[r];
    if (threadIdx.x == 0) p.lcT[static_cast<int64_t>(seq) * p.nch + kc] = lct;
}

// Carries: one thread per state element, scan over the chunks of one sequence.
__global__ __launch_bounds__(256) void rank1_carry_kernel(Rank1Params p) {
    const int seq = blockIdx.y;
    const int e = blockIdx.x * 256 + threadIdx.x;   // < DH*DH
    const int64_t base = static_cast<int64_t>(seq) * p.nch;
    float S = 0.0f;
    for (int kc = 0; kc < p.nch; ++kc) {
        p.Sin[(base + kc) * R1_DH * R1_DH + e] = S;
        S = fmaf(expf(p.lcT[base + kc]), S, p.dS[(base + kc) * R1_DH * R1_DH + e]);
    }
}

template <typename TF, typename TI, typename TO>
__global__ __launch_bounds__(R1_THREADS) void rank1_output_kernel(Rank1Params p) {
    constexpr int SR = R1_DH + R1_PAD;   // row stride of [t][d] / [i][j] tiles
    constexpr int SP = R1_T + R1_PAD;    // row stride of [.][t] tiles
    __shared__ __attribute__((aligned(16))) bf16_t sQ[R1_T * SR];
    __shared__ __attribute__((aligned(16))) bf16_t sK[R1_T * SR];
    __shared__ __attribute__((aligned(16))) bf16_t sVT[R1_DH * SP];
    __shared__ __attribute__((aligned(16))) bf16_t sP[R1_T * SP];
    __shared__ __attribute__((aligned(16))) bf16_t sShi[R1_DH * SR];
    __shared__ __attribute__((aligned(16))) bf16_t sSlo[R1_DH * SR];
    __shared__ float sLc[R1_T], sOmf[R1_T];
    const int kc = blockIdx.x;
    const int seq = blockIdx.y;
    const int b = seq / p.H, h = seq - (seq / p.H) * p.H;
    const int64_t t0 = static_cast<int64_t>(kc) * R1_T;
    const int64_t rowbase = static_cast<int64_t>(b) * p.L * p.H + h;
    load_rows<TI, false>(static_cast<const TI*>(p.q), sQ, rowbase, t0, p.L, p.H);
    load_rows<TI, false>(static_cast<const TI*>(p.k), sK, rowbase, t0, p.L, p.H);
    load_rows<TI, true>(static_cast<const TI*>(p.v), sVT, rowbase, t0, p.L, p.H);
    chunk_decay<TF>(static_cast<const TF*>(p.f), rowbase, t0, p.L, p.H, sLc, sOmf);
    {
        const float* S = p.Sin + (static_cast<int64_t>(seq) * p.nch + kc) * R1_DH * R1_DH;
        for (int e = threadIdx.x; e < R1_DH * R1_DH; e += R1_THREADS) {
            const int i = e / R1_DH, j = e - (e / R1_DH) * R1_DH;
            const float x = S[e];
            const bf16_t hi = f32_to_bf16(x);
            sShi[i * SR + j] = hi;
            sSlo[i * SR + j] = f32_to_bf16(x - bf16_to_f32(hi));
        }
    }
    __syncthreads();
    const int w = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int tb = w >> 1, xb = w & 1;   // this wave's 32-row block and 32-column block
    // P = (Q K^T) o exp(Lc_t - Lc_s) (1 - f_s) on s <= t  (tile (tb, xb); s-block xb > tb is zero)
    {
        const int t_of = tb * 32, s_of = xb * 32;
        if (xb <= tb) {
            f32x16 acc = mma32(sQ + t_of * SR, SR, sK + s_of * SR, SR, R1_DH, zero16());
            const int s = s_of + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int t = t_of + mrow(r);
                const float pv = (s <= t) ? acc[r] * expf(sLc[t] - sLc[s]) * sOmf[s] : 0.0f;
                sP[t * SP + s] = f32_to_bf16(pv);
            }
        }
    }
    __syncthreads();
    // y tile (rows tb, columns xb): intra-chunk P V + decayed inter-chunk Q S_in^T
    const int t_of = tb * 32, i_of = xb * 32;
    f32x16 intra = zero16();
    for (int sb = 0; sb <= tb; ++sb)
        intra = mma32(sP + t_of * SP + sb * 32, SP, sVT + i_of * SP + sb * 32, SP, 32, intra);
    f32x16 inter = mma32(sQ + t_of * SR, SR, sShi + i_of * SR, SR, R1_DH, zero16());
    inter = mma32(sQ + t_of * SR, SR, sSlo + i_of * SR, SR, R1_DH, inter);
    TO* y = static_cast<TO*>(p.y);
    const int col = i_of + (lane & 31);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int t = t_of + mrow(r);
        if (t0 + t < p.L) {
            const float val = intra[r] + expf(sLc[t]) * inter[r];
            y[(rowbase + (t0 + t) * p.H) * R1_DH + col] = IO<TO>::st(val);
        }
    }
}

namespace {

struct R1Geo {
    int nch;
    size_t off_ds, off_lct, off_sin, bytes;
};

R1Geo r1_geometry(int64_t B, int64_t L, int64_t H) {
    R1Geo g{};
    g.nch = static_cast<int>((L + R1_T - 1) / R1_T);
    const size_t nseq = static_cast<size_t>(B) * H;
    size_t off = WS_HDR_BYTES;
    auto take = [&](size_t n) { size_t o = off; off = round_up(off + n, 256); return o; };
    g.off_ds = take(nseq * g.nch * R1_DH * R1_DH * sizeof(float));
    g.off_lct = take(nseq * g.nch * sizeof(float));
    g.off_sin = take(nseq * g.nch * R1_DH * R1_DH * sizeof(float));
    g.bytes = off;
    return g;
}

template <typename TF, typename TI, typename TO>
int run_rank1(const Rank1Params& prm, int n_seq, hipStream_t st) {
    const dim3 grid(prm.nch, n_seq);
    hipLaunchKernelGGL((rank1_summary_kernel<TF, TI>), grid, dim3(R1_THREADS), 0, st, prm);
    int rc = check_launch("rank1_summary_kernel");
    if (rc) return rc;
    hipLaunchKernelGGL(rank1_carry_kernel, dim3(R1_DH * R1_DH / 256, n_seq), dim3(256), 0, st, prm);
    rc = check_launch("rank1_carry_kernel");
    if (rc) return rc;
    hipLaunchKernelGGL((rank1_output_kernel<TF, TI, TO>), grid, dim3(R1_THREADS), 0, st, prm);
    return check_launch("rank1_output_kernel");
}

}  // namespace
}  // namespace mogt

using namespace mogt;

extern "C" size_t mogt_rank1_coupled_scan_workspace_bytes(int64_t batch, int64_t length, int64_t heads,
                                                          int64_t head_dim) {
    if (batch <= 0 || length <= 0 || heads <= 0 || head_dim != R1_DH) return WS_HDR_BYTES;
    return r1_geometry(batch, length, heads).bytes;
}

extern "C" int mogt_rank1_coupled_scan_fwd(const void* f, const void* k, const void* v, const void* q,
                                           void* y, int64_t batch, int64_t length, int64_t heads,
                                           int64_t head_dim, int f_dtype, int kvq_dtype, int out_dtype,
                                           void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    if (batch < 0 || length < 0 || heads <= 0)
        return set_error(MOGT_E_INVALID, "f must be [B, L, H] and k, v, q [B, L, H, d]");
    if (head_dim != R1_DH) return set_error(MOGT_E_INVALID, "head_dim %lld not supported (64)", (long long)head_dim);
    for (int d : {f_dtype, kvq_dtype, out_dtype})
        if (d != MOGT_F32 && d != MOGT_BF16) return set_error(MOGT_E_INVALID, "unsupported dtype code");
    if (batch == 0 || length == 0) return MOGT_OK;
    if (!f || !k || !v || !q || !y) return set_error(MOGT_E_INVALID, "null tensor pointer");
    const R1Geo g = r1_geometry(batch, length, heads);
    if (!workspace || workspace_bytes < g.bytes)
        return set_error(MOGT_E_WORKSPACE, "workspace of %zu bytes required, got %zu", g.bytes, workspace_bytes);
    if (batch * heads > 65535) return set_error(MOGT_E_INVALID, "batch * heads > 65535");
    char* base = static_cast<char*>(workspace);
    Rank1Params prm{};
    prm.f = f; prm.k = k; prm.v = v; prm.q = q; prm.y = y;
    prm.dS = reinterpret_cast<float*>(base + g.off_ds);
    prm.lcT = reinterpret_cast<float*>(base + g.off_lct);
    prm.Sin = reinterpret_cast<float*>(base + g.off_sin);
    prm.L = length; prm.H = static_cast<int>(heads); prm.nch = g.nch;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int n_seq = static_cast<int>(batch * heads);
    const bool fb = f_dtype == MOGT_BF16, ib = kvq_dtype == MOGT_BF16, ob = out_dtype == MOGT_BF16;
    if (fb && ib && ob) return run_rank1<bf16_t, bf16_t, bf16_t>(prm, n_seq, st);
    if (fb && ib && !ob) return run_rank1<bf16_t, bf16_t, float>(prm, n_seq, st);
    if (!fb && ib && ob) return run_rank1<float, bf16_t, bf16_t>(prm, n_seq, st);
    if (!fb && ib && !ob) return run_rank1<float, bf16_t, float>(prm, n_seq, st);
    if (fb && !ib && ob) return run_rank1<bf16_t, float, bf16_t>(prm, n_seq, st);
    if (fb && !ib && !ob) return run_rank1<bf16_t, float, float>(prm, n_seq, st);
    if (!fb && !ib && ob) return run_rank1<float, float, bf16_t>(prm, n_seq, st);
    return run_rank1<float, float, float>(prm, n_seq, st);
}
