// Rank-1 coupled write-forget scan with readout, per (batch, head):
//   S_t = f_t S_{t-1} + (1 - f_t) v_t k_t^T,   y_t = S_t q_t,   S_0 = 0
// i.e. the affine recurrence of affine_scan.py:48-55 with U_t = f_t I and the
// rank-1 write V_t = (1 - f_t) v_t k_t^T, read out through q_t.  S_t (d x d per
// step) is never written to memory.
//
// Chunked form.  Inside a block of steps with Lc_t = sum_{u<=t} log2 f_u (block
// local; decays are 2^(Lc_t - Lc_s), one v_exp_f32 each) and S_in the state
// before the block:
//   y_t   = 2^Lc_t S_in q_t + sum_{s<=t} 2^(Lc_t - Lc_s) (1 - f_s) (q_t . k_s) v_s
//   S_out = 2^Lc_T S_in + V^T diag(w) K,   w_s = 2^(Lc_T - Lc_s) (1 - f_s)
// Three launches over super-chunks of RS = 256 steps:
//   K_A  per super-chunk: dS = V^T diag(w) K over its 256 steps (one bf16 MFMA
//        chain, K = 256) and its total log-decay.
//   K_B  per (sequence, state element): S_in of every super-chunk -- the carries
//        compose element-wise with a scalar decay, so this is a plain scan.
//   K_C  per super-chunk: four 64-step sub-chunks in order, the 64 x 64 state
//        carried in MFMA accumulators; per sub-chunk the masked, decayed
//        (Q K^T) V plus 2^Lc Q S^T (state split into bf16 hi + lo parts for
//        fp32-level accuracy), then S <- 2^Lc_T S + V^T diag(w) K.  The next
//        sub-chunk's q, k, v are loaded into registers while this one computes.
// K_A reads k and v with ordinary (cache-allocating) loads, so K_C usually finds
// them in the Infinity Cache.  Layouts: f [B, L, H]; q, k, v, y [B, L, H, DH].
#include "lds_dma.h"

namespace mogt {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int R1_DH = 64;         // head dimension
constexpr int R1_T = 64;          // sub-chunk length
constexpr int R1_SUB = 4;         // sub-chunks per super-chunk
constexpr int R1_RS = R1_T * R1_SUB;
constexpr int R1_THREADS = 256;   // 4 waves
constexpr int R1_PAD = 8;         // LDS row padding (bf16): rows of 144 B
constexpr int R1_SR = R1_DH + R1_PAD;
constexpr float R1_LOG2_MIN = -120.0f;   // clamp of log2 f (f = 0 -> 2^-120 per step)

struct Rank1Params {
    const void* f;
    const void* k;
    const void* v;
    const void* q;
    void* y;
    float* dS;      // [n_seq][nsc][DH*DH]
    float* lcT;     // [n_seq][nsc]
    float* Sin;     // [n_seq][nsc][DH*DH]
    int64_t L;
    int H, nsc;
};

// Transposed tiles (rows d, 64 steps t per row, written by put_cols) hold
// 16-byte chunk c of row d at chunk position c ^ (d / 8 % 8).  The transposed
// 4-byte stores, whose lanes write rows 8 apart, then fall into distinct
// banks, and an MFMA operand read (8 consecutive rows, one chunk each) stays
// conflict-free through the row padding.
__device__ __forceinline__ int tsw(int row) { return (row >> 3) & 7; }

// 32x32 fp32 tile += A[32 x K] B[K x 32].  A is rows ar.. of tile `a` from
// column ac, B the columns held as rows br.. of tile `b` from column bc (k
// contiguous in both); SWA / SWB mark transposed (chunk-swizzled) tiles.
template <bool SWA, bool SWB>
__device__ __forceinline__ f32x16 mma32(const bf16_t* a, int ar, int ac, const bf16_t* b, int br, int bc, int K,
                                        f32x16 acc) {
    const int l = threadIdx.x & 63, hb = l >> 5;
    const int ra = ar + (l & 31), rb = br + (l & 31);
    const int xa = SWA ? tsw(ra) : 0, xb = SWB ? tsw(rb) : 0;
#pragma unroll
    for (int k0 = 0; k0 < K; k0 += 16) {
        const int ca = (((ac + k0) >> 3) + hb) ^ xa, cb = (((bc + k0) >> 3) + hb) ^ xb;
        const bf16x8 av = *reinterpret_cast<const bf16x8*>(a + ra * R1_SR + 8 * ca);
        const bf16x8 bv = *reinterpret_cast<const bf16x8*>(b + rb * R1_SR + 8 * cb);
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

// Inclusive prefix sum over the 64 lanes of a wave on DPP lane moves (no LDS
// round trips): shifts by 1, 2, 4, 8 inside each row of 16 lanes (lanes
// shifted past the row start add 0), then each row adds the total of the rows
// before it through row_bcast:15 (rows 1, 3) and row_bcast:31 (rows 2, 3).
template <int CTRL, int ROW_MASK, bool BOUND_ZERO>
__device__ __forceinline__ float dpp_f32(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xf, BOUND_ZERO));
}
__device__ __forceinline__ float wave_incl_scan(float x) {
    x += dpp_f32<0x111, 0xf, true>(x);   // row_shr:1
    x += dpp_f32<0x112, 0xf, true>(x);   // row_shr:2
    x += dpp_f32<0x114, 0xf, true>(x);   // row_shr:4
    x += dpp_f32<0x118, 0xf, true>(x);   // row_shr:8
    x += dpp_f32<0x142, 0xa, false>(x);  // row_bcast:15 into rows 1 and 3
    x += dpp_f32<0x143, 0xc, false>(x);  // row_bcast:31 into rows 2 and 3
    return x;
}

// One 64-step x 64-wide tile of q, k or v held in registers.  Thread e covers
// the row pair (2m, 2m + 1), m = e / 8, and segment sg = e % 8 of 8 consecutive
// elements in both rows, so 8 consecutive lanes read one 128-byte row and a
// transposed store writes both rows' elements of one column as one 4-byte
// word.  Tiles are read through a buffer descriptor whose range ends with the
// sequence's row L - 1, so rows past L read as zeros; the per-lane offsets are
// constant and the loads carry no address arithmetic.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

template <typename TI>
struct Tile8 {
    static constexpr int NW = sizeof(TI) == 2 ? 1 : 2;   // 16-byte words per segment
    u32x4 x[2][NW];
};

__device__ __forceinline__ int tile_m() { return static_cast<int>(threadIdx.x) >> 3; }
__device__ __forceinline__ int tile_sg() { return static_cast<int>(threadIdx.x) & 7; }

// Byte range of the rows t0 .. L - 1 of one (batch, head) sequence of a
// [B, L, H, n] tensor with n elements of `elem` bytes per row: the first
// element of row t0 and the span up to the end of row L - 1.  For t0 >= L (a
// padding sub-chunk past the end, which the summary kernel still prefetches)
// the span is empty and the base stays at the sequence's first row, so loads
// through it read 0 and stores are dropped.  Host and device share it, so
// mogt_rank1_check_ranges can check every range the kernels build.
struct RowsRange {
    int64_t base;   // element offset of the range's first byte
    int64_t span;   // bytes
};
__host__ __device__ inline RowsRange rows_range(int64_t rowbase, int64_t t0, int64_t L, int H, int n, int elem) {
    const int64_t strideB = static_cast<int64_t>(H) * n * elem;
    const bool live = t0 < L;
    int64_t span = live ? (L - 1 - t0) * strideB + static_cast<int64_t>(n) * elem : 0;
    if (span > 0x7fffffff) span = 0x7fffffff;
    return {(rowbase + (live ? t0 : 0) * H) * n, span};
}
template <typename T>
__device__ __forceinline__ auto seq_rsrc(const T* base, int64_t rowbase, int64_t t0, int64_t L, int H, int n) {
    const RowsRange r = rows_range(rowbase, t0, L, H, n, static_cast<int>(sizeof(T)));
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(base) + r.base, 0, static_cast<int>(r.span),
                                             0x00020000);
}

template <typename TI>
__device__ __forceinline__ Tile8<TI> load_tile(const TI* __restrict__ src, int64_t rowbase, int64_t t0,
                                               int64_t L, int H) {
    const auto rs = seq_rsrc(src, rowbase, t0, L, H, R1_DH);
    const int strideB = H * R1_DH * static_cast<int>(sizeof(TI));
    Tile8<TI> r;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int off = (2 * tile_m() + u) * strideB + tile_sg() * 8 * static_cast<int>(sizeof(TI));
#pragma unroll
        for (int j = 0; j < Tile8<TI>::NW; ++j)
            r.x[u][j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16 * j, 0, 0));
    }
    return r;
}

// The 8 elements of row 2m + u as fp32.
template <typename TI>
__device__ __forceinline__ void seg_f32(const Tile8<TI>& r, int u, float (&o)[8]) {
    if constexpr (sizeof(TI) == 2) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            o[2 * i] = __uint_as_float(r.x[u][0][i] << 16);
            o[2 * i + 1] = __uint_as_float(r.x[u][0][i] & 0xffff0000u);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) o[4 * j + i] = __uint_as_float(r.x[u][j][i]);
    }
}

// Two fp32 values as one word of two bf16 (round to nearest even): one
// v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo, hi}), bf16x2));
}

// Tile into LDS row-major [t][d] (row stride R1_SR).
template <typename TI>
__device__ __forceinline__ void put_rows(const Tile8<TI>& r, bf16_t* dst) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int t = 2 * tile_m() + u;
        u32x4 w;
        if constexpr (sizeof(TI) == 2) {
            w = r.x[u][0];
        } else {
            float o[8];
            seg_f32(r, u, o);
#pragma unroll
            for (int i = 0; i < 4; ++i) w[i] = pack_bf16(o[2 * i], o[2 * i + 1]);
        }
        *reinterpret_cast<u32x4*>(dst + t * R1_SR + tile_sg() * 8) = w;
    }
}
// Tile into LDS transposed [d][t] with the chunk swizzle of tsw();
// with SCALE, rows 2m and 2m + 1 are multiplied by s0 and s1.  Row d = 8 sg + i
// of the transposed tile gets the word (t = 2m, 2m + 1) in chunk (m / 4) ^ sg.
template <bool SCALE, typename TI>
__device__ __forceinline__ void put_cols(const Tile8<TI>& r, bf16_t* dst, float s0 = 1.0f, float s1 = 1.0f) {
    const int m = tile_m(), sg = tile_sg();
    bf16_t* base = dst + 8 * sg * R1_SR + 8 * ((m >> 2) ^ sg) + 2 * (m & 3);
    uint32_t wd[8];
    if constexpr (sizeof(TI) == 2 && !SCALE) {
        // bf16 halves regrouped by byte permutes: element 2i is the low half of
        // word i, element 2i + 1 the high half
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            wd[2 * i] = __builtin_amdgcn_perm(r.x[1][0][i], r.x[0][0][i], 0x05040100u);
            wd[2 * i + 1] = __builtin_amdgcn_perm(r.x[1][0][i], r.x[0][0][i], 0x07060302u);
        }
    } else {
        float a[8], b[8];
        seg_f32(r, 0, a);
        seg_f32(r, 1, b);
#pragma unroll
        for (int i = 0; i < 8; ++i) wd[i] = SCALE ? pack_bf16(a[i] * s0, b[i] * s1) : pack_bf16(a[i], b[i]);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) *reinterpret_cast<uint32_t*>(base + i * R1_SR) = wd[i];
}

// Raw f of step t (row L - 1 past the end; see fval).
template <typename TF>
__device__ __forceinline__ TF load_f(const TF* __restrict__ f, int64_t rowbase, int64_t t, int64_t L,
                                     int H) {
    return f[rowbase + (t < L ? t : L - 1) * H];
}
// Padding steps past L act as f = 1 with k = v = q = 0 (no write, no decay).
template <typename TF>
__device__ __forceinline__ float fval(TF raw, int64_t t, int64_t L) {
    return t < L ? IO<TF>::ld(raw) : 1.0f;
}

// 2^x on the hardware exponential (v_exp_f32); every argument here is <= 0,
// and results below 2^-126 only weight terms already below bf16 resolution.
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------------------
// K_A: dS = V^T diag(w) K over one 256-step super-chunk.
// ---------------------------------------------------------------------------
template <typename TF, typename TI>
__global__ __launch_bounds__(R1_THREADS) void rank1_summary_kernel(Rank1Params p) {
    __shared__ __attribute__((aligned(16))) bf16_t sVT[R1_DH * R1_SR];
    __shared__ __attribute__((aligned(16))) bf16_t sKT[R1_DH * R1_SR];
    __shared__ float sW[R1_RS];
    __shared__ float sWave[4];
    const int sc = blockIdx.x;
    const int seq = blockIdx.y;
    const int b = seq / p.H, h = seq - (seq / p.H) * p.H;
    const int64_t t0 = static_cast<int64_t>(sc) * R1_RS;
    const int64_t rowbase = static_cast<int64_t>(b) * p.L * p.H + h;   // (b*L + t)*H + h
    const TI* kp = static_cast<const TI*>(p.k);
    const TI* vp = static_cast<const TI*>(p.v);

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const TF fraw = load_f<TF>(static_cast<const TF*>(p.f), rowbase, t0 + tid, p.L, p.H);
    Tile8<TI> kt = load_tile<TI>(kp, rowbase, t0, p.L, p.H);
    Tile8<TI> vt = load_tile<TI>(vp, rowbase, t0, p.L, p.H);

    // block-wide inclusive log-decay cumsum over the super-chunk (one step per
    // thread; threads past it act as f = 1)
    static_assert(R1_RS <= R1_THREADS, "one thread per step of the super-chunk");
    const bool tin = tid < R1_RS;
    const float fv = tin ? fval<TF>(fraw, t0 + tid, p.L) : 1.0f;
    float lc = wave_incl_scan(fmaxf(__log2f(fv), R1_LOG2_MIN));
    if (lane == 63) sWave[w] = lc;
    __syncthreads();
    for (int i = 0; i < w; ++i) lc += sWave[i];
    const float lcT = sWave[0] + sWave[1] + sWave[2] + sWave[3];
    if (tin) sW[tid] = exp2_hw(lcT - lc) * (1.0f - fv);

    const int ib = w >> 1, jb = w & 1;   // this wave's 32x32 tile of dS[i][j]
    const int m = tile_m();
    f32x16 acc = zero16();
    for (int sub = 0; sub < R1_SUB; ++sub) {
        __syncthreads();   // previous sub-block's tiles consumed; sW visible
        put_cols<false>(kt, sKT);
        put_cols<true>(vt, sVT, sW[sub * R1_T + 2 * m], sW[sub * R1_T + 2 * m + 1]);   // V^T diag(w)
        if (sub + 1 < R1_SUB) {   // prefetch the next sub-block while this one multiplies
            kt = load_tile<TI>(kp, rowbase, t0 + (sub + 1) * R1_T, p.L, p.H);
            vt = load_tile<TI>(vp, rowbase, t0 + (sub + 1) * R1_T, p.L, p.H);
        }
        __syncthreads();
        acc = mma32<true, true>(sVT, ib * 32, 0, sKT, jb * 32, 0, R1_T, acc);
    }
    float* out = p.dS + (static_cast<int64_t>(seq) * p.nsc + sc) * R1_DH * R1_DH;
    const int col = jb * 32 + (lane & 31);
#pragma unroll
    for (int r = 0; r < 16; ++r) out[(ib * 32 + mrow(r)) * R1_DH + col] = acc[r];
    if (tid == 0) p.lcT[static_cast<int64_t>(seq) * p.nsc + sc] = lcT;
}

// ---------------------------------------------------------------------------
// K_B: carries.  One thread per state element; the summaries of up to 32
// super-chunks are loaded at once, ahead of the dependent multiply-adds.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rank1_carry_kernel(Rank1Params p) {
    const int seq = blockIdx.y;
    const int e = blockIdx.x * 256 + threadIdx.x;   // < DH*DH
    const int64_t base = static_cast<int64_t>(seq) * p.nsc;
    constexpr int64_t SZ = R1_DH * R1_DH;
    constexpr int NB = 32;
    float S = 0.0f;
    for (int c0 = 0; c0 < p.nsc; c0 += NB) {
        float d[NB], dec[NB];
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int c = min(c0 + i, p.nsc - 1);   // in-bounds, unconditional
            d[i] = p.dS[(base + c) * SZ + e];
            dec[i] = p.lcT[base + c];
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            if (c0 + i < p.nsc) {
                p.Sin[(base + c0 + i) * SZ + e] = S;
                S = fmaf(exp2f(dec[i]), S, d[i]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// K_C: outputs of one super-chunk, four sub-chunks in order.
//
// Wave w = (a, c) = (w / 2, w % 2) owns the 32 x 32 quadrant (rows 32a, columns
// 32c) of every 64 x 64 product: of P[t][s] (a >= c only), of y[t][i], and of
// the transposed state S^T[j][i], kept in MFMA accumulators.  Holding S^T
// puts four consecutive j of one row S[i][.] in each lane's register group,
// so the bf16 hi / lo halves of S go to LDS as 8-byte words.  Per sub-chunk:
//   every wave scans the 64 log-decays itself (lane = step) and stages its
//   share of q, k (rows), k^T diag(w) and v^T into LDS      | barrier
//   P = (Q K^T) o 2^(Lc_t - Lc_s) (1 - f_s), s <= t          | barrier
//   y = P V + 2^Lc_t Q S^T (S as bf16 hi + lo)               | barrier
//   S^T <- 2^Lc_T S^T + K^T diag(w) V; S halves to LDS       | barrier
// The next sub-chunk's q, k, v, f are loaded while the current one computes.
// y is written through a buffer descriptor whose range ends at the sequence's
// last row, so rows past L are dropped by the hardware.
// ---------------------------------------------------------------------------
template <typename TF, typename TI, typename TO>
__global__ __launch_bounds__(R1_THREADS) void rank1_output_kernel(Rank1Params p) {
    __shared__ __attribute__((aligned(16))) bf16_t sQ[R1_T * R1_SR];
    __shared__ __attribute__((aligned(16))) bf16_t sK[R1_T * R1_SR];
    __shared__ __attribute__((aligned(16))) bf16_t sVT[R1_DH * R1_SR];
    __shared__ __attribute__((aligned(16))) bf16_t sKTw[R1_DH * R1_SR];
    __shared__ __attribute__((aligned(16))) bf16_t sP[R1_T * R1_SR];
    __shared__ __attribute__((aligned(16))) bf16_t sShi[R1_DH * R1_SR];
    __shared__ __attribute__((aligned(16))) bf16_t sSlo[R1_DH * R1_SR];
    __shared__ __attribute__((aligned(16))) float sLc[R1_T];
    __shared__ __attribute__((aligned(16))) float sE[R1_T];
    __shared__ float sOmf[R1_T];
    const int sc = blockIdx.x;
    const int seq = blockIdx.y;
    const int b = seq / p.H, h = seq - (seq / p.H) * p.H;
    const int64_t rowbase = static_cast<int64_t>(b) * p.L * p.H + h;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int qa = w >> 1, qc = w & 1;   // this wave's quadrant: rows 32 qa, columns 32 qc
    const int m = tile_m();
    const TI* qp = static_cast<const TI*>(p.q);
    const TI* kp = static_cast<const TI*>(p.k);
    const TI* vp = static_cast<const TI*>(p.v);
    const TF* fp = static_cast<const TF*>(p.f);
    const int64_t rowStrideB = static_cast<int64_t>(p.H) * R1_DH * sizeof(TO);   // bytes between steps of y

    const int64_t tsc = static_cast<int64_t>(sc) * R1_RS;
    TF fraw = load_f<TF>(fp, rowbase, tsc + lane, p.L, p.H);
    Tile8<TI> qt = load_tile<TI>(qp, rowbase, tsc, p.L, p.H);
    Tile8<TI> kt = load_tile<TI>(kp, rowbase, tsc, p.L, p.H);
    Tile8<TI> vt = load_tile<TI>(vp, rowbase, tsc, p.L, p.H);

    // S^T quadrant (rows j = 32 qa + mrow(r), columns i = 32 qc + lane % 32) of S_in
    f32x16 ST;
    {
        const float* src = p.Sin + (static_cast<int64_t>(seq) * p.nsc + sc) * R1_DH * R1_DH;
        const int i = qc * 32 + (lane & 31);
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {   // j = 32 qa + 8 g4 + 4 (lane / 32) + 0..3: one 16-byte load
            const int j = qa * 32 + 8 * g4 + 4 * (lane >> 5);
            const f32x4 v4 = *reinterpret_cast<const f32x4*>(src + i * R1_DH + j);
#pragma unroll
            for (int q = 0; q < 4; ++q) ST[4 * g4 + q] = v4[q];
        }
    }
    // S (= transposed accumulators) as bf16 hi + lo halves into LDS rows [i][j]
    auto put_state = [&]() {
        const int i = qc * 32 + (lane & 31);
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
            const int j = qa * 32 + 8 * g4 + 4 * (lane >> 5);
            uint32_t hw[2], lw[2];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const float x0 = ST[4 * g4 + 2 * q], x1 = ST[4 * g4 + 2 * q + 1];
                hw[q] = pack_bf16(x0, x1);
                const float h0 = __uint_as_float(hw[q] << 16), h1 = __uint_as_float(hw[q] & 0xffff0000u);
                lw[q] = pack_bf16(x0 - h0, x1 - h1);
            }
            *reinterpret_cast<uint2*>(sShi + i * R1_SR + j) = uint2{hw[0], hw[1]};
            *reinterpret_cast<uint2*>(sSlo + i * R1_SR + j) = uint2{lw[0], lw[1]};
        }
    };
    put_state();

    const int nsub = static_cast<int>((p.L - tsc + R1_T - 1) / R1_T) < R1_SUB
                         ? static_cast<int>((p.L - tsc + R1_T - 1) / R1_T)
                         : R1_SUB;
    for (int sub = 0; sub < nsub; ++sub) {
        const int64_t t0 = tsc + static_cast<int64_t>(sub) * R1_T;
        // log-decays of this sub-chunk, lane = step (every wave; wave 0 publishes)
        const float fv = fval<TF>(fraw, t0 + lane, p.L);
        const float lc = wave_incl_scan(fmaxf(__log2f(fv), R1_LOG2_MIN));
        const float lcT = __shfl(lc, 63, 64);
        const float wgt = exp2_hw(lcT - lc) * (1.0f - fv);
        if (w == 0) {
            sLc[lane] = lc;
            sE[lane] = exp2_hw(lc);
            sOmf[lane] = 1.0f - fv;
        }
        // stage this sub-chunk
        put_rows(qt, sQ);
        put_rows(kt, sK);
        put_cols<true>(kt, sKTw, __shfl(wgt, 2 * m, 64), __shfl(wgt, 2 * m + 1, 64));
        put_cols<false>(vt, sVT);
        __syncthreads();
        if (sub + 1 < nsub) {   // next sub-chunk's operands, in flight while this one computes
            qt = load_tile<TI>(qp, rowbase, t0 + R1_T, p.L, p.H);
            kt = load_tile<TI>(kp, rowbase, t0 + R1_T, p.L, p.H);
            vt = load_tile<TI>(vp, rowbase, t0 + R1_T, p.L, p.H);
            fraw = load_f<TF>(fp, rowbase, t0 + R1_T + lane, p.L, p.H);
        }
        const int t_of = qa * 32, c_of = qc * 32;
        // Lc_t and 2^Lc_t of this lane's 16 rows t = t_of + mrow(r): 16-byte reads
        float lct[16], et[16];
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
            const int t = t_of + 8 * g4 + 4 * (lane >> 5);
            const f32x4 l4 = *reinterpret_cast<const f32x4*>(sLc + t);
            const f32x4 e4 = *reinterpret_cast<const f32x4*>(sE + t);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                lct[4 * g4 + q] = l4[q];
                et[4 * g4 + q] = e4[q];
            }
        }
        // P quadrant (rows t_of, columns s_of = c_of), lower triangle only
        if (qc <= qa) {
            f32x16 acc = mma32<false, false>(sQ, t_of, 0, sK, c_of, 0, R1_DH, zero16());
            const int s = c_of + (lane & 31);
            const float lcs = sLc[s], omf = sOmf[s];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int t = t_of + mrow(r);
                const float pv = (qc < qa || s <= t) ? acc[r] * exp2_hw(lct[r] - lcs) * omf : 0.0f;
                sP[t * R1_SR + s] = f32_to_bf16(pv);
            }
        }
        __syncthreads();
        // y quadrant (rows t_of, columns i = c_of): intra P V + decayed inter Q S^T
        {
            // decayed inter term first, then the intra products accumulate onto it
            f32x16 acc = mma32<false, false>(sQ, t_of, 0, sShi, c_of, 0, R1_DH, zero16());
            acc = mma32<false, false>(sQ, t_of, 0, sSlo, c_of, 0, R1_DH, acc);
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[r] *= et[r];
            for (int sb = 0; sb <= qa; ++sb)
                acc = mma32<false, true>(sP, t_of, sb * 32, sVT, c_of, sb * 32, 32, acc);
            // rows of this sub-chunk at or past L fall outside the range and are dropped
            const int64_t left = p.L - t0;   // >= 1
            const int64_t span = (left - 1) * rowStrideB + static_cast<int64_t>(R1_DH) * sizeof(TO);
            const auto ry = __builtin_amdgcn_make_buffer_rsrc(
                static_cast<TO*>(p.y) + (rowbase + t0 * p.H) * R1_DH, 0,
                static_cast<int>(span < 0x7fffffff ? span : 0x7fffffff), 0x00020000);
            const int colB = (c_of + (lane & 31)) * static_cast<int>(sizeof(TO));
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int t = t_of + mrow(r);
                const float val = acc[r];
                const int off = t * static_cast<int>(rowStrideB) + colB;
                if constexpr (sizeof(TO) == 4)
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(val), ry, off, 0, 2);
                else
                    __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(val), ry, off, 0, 2);
            }
        }
        __syncthreads();   // sQ, sP and the old state halves are consumed
        // S^T <- 2^Lc_T S^T + K^T diag(w) V
        {
            const float dec = exp2_hw(lcT);
#pragma unroll
            for (int r = 0; r < 16; ++r) ST[r] *= dec;
            ST = mma32<true, true>(sKTw, t_of, 0, sVT, c_of, 0, R1_T, ST);
            put_state();
        }
        __syncthreads();   // tiles of this sub-chunk consumed before the next staging
    }
}

// ---------------------------------------------------------------------------
// Single-pass form, for sequences of at most R1S_MAX_SC super-chunks.
//
// One work-group per super-chunk (256 steps); wave j owns sub-chunk j (64
// steps) from start to end, so the waves never take turns:
//   1. each wave loads its q, k (MFMA operand registers), v and f, scans its
//      log-decays, and stages V and K diag(w) (w relative to the sub-chunk's
//      end) into LDS as natural [step][dim] rows            | barrier
//   2. wave j: S_j^loc = the state at its sub-chunk's start from a zero state
//      at the super-chunk's start (Horner over the staged sub-chunks m < j:
//      S <- 2^LcT_m S + K_m^T diag(w) V_m); wave 0 runs all four and publishes
//      the super-chunk's aggregate; P^T = K Q^T decayed and masked;
//      y_pre = 2^Lc_t Q S_j^loc^T + P V
//   3. carries, cooperatively per sequence: once every aggregate of the
//      sequence is published, work-group c scans the element slice
//      [c E, (c + 1) E) of the states through all super-chunks and writes the
//      carried-in states' slices; once every slice is written, each
//      work-group reads its own carried-in state S_in
//   4. y = y_pre + 2^(Lc_t + Lc_start_j) Q S_in^T              -> y
// The contractions over steps (K^T V, P V) read their operands from the
// natural LDS rows with ds_read_b64_tr_b16 (gfx950's transposing LDS read):
// in each 16-lane group, lane 4r + c addresses row r, columns 4c .. 4c + 3 of
// a 4 x 16 block, and lane i receives column i of the block's 4 rows.  LDS
// rows hold their 16-byte chunks XOR-permuted by row so these reads are free
// of bank conflicts.  Operands of the contractions over the head dimension
// (K Q^T, Q S^T) come straight from registers in a contraction order that
// matches the MFMA accumulator layout (k = 16 kk + 4 (lane / 32) + 0..3, then
// + 8), so P^T and S^T accumulators feed the next products without a
// transpose.  The cross-work-group steps use the workspace epoch tags of the
// look-back protocol: payloads are written with agent-coherent (sc1) stores,
// each writer waits for its stores before its flag, readers poll the flags
// with agent-scope loads and read payloads with sc1 loads.  Every wait is
// bounded; a wait that gives up poisons the affected outputs with NaN and
// counts in the workspace header.  Forward progress needs all super-chunks of
// one sequence resident at once, which in-order dispatch guarantees for at
// most R1S_MAX_SC of them.
// ---------------------------------------------------------------------------
constexpr int R1S_MAX_SC = 64;
constexpr int R1S_GROUPS_PER_CU = 3;   // resident one-launch work-groups per CU (registers and LDS)
constexpr int R1S_NB = 16;            // aggregates loaded per batch of the slice scan
constexpr int R1_SC1 = 16;            // buffer cache policy: agent-coherent (sc1)

// One agent-coherent (sc1) dword per lane straight into LDS at lds + 4 * lane
// (no register holds it).  m0 carries the LDS address; it is written here and
// read only by the load that follows.
__device__ __forceinline__ void r1_dma4_sc1(lds_i32x4 rsrc, int voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen sc1 lds"
                 :
                 : "s"(lds), "v"(voff), "s"(rsrc)
                 : "memory", "m0");
}

struct Rank1SParams {
    const void* f;
    const void* k;
    const void* v;
    const void* q;
    void* y;
    uint32_t* hdr;
    uint64_t* flag1;   // [n_seq][nsc] {tag | total log2-decay of the super-chunk}
    uint32_t* flag2;   // [n_seq][nsc] tag: slices of the carried-in states written
    float* agg;        // [n_seq][nsc][DH*DH] aggregates (accumulator order)
    float* sin;        // [n_seq][nsc][DH*DH] carried-in states (same order)
    int64_t L;
    int H, nsc;
    int skip_agg0;       // test path: super-chunk 0 withholds its aggregate, and waits
                         // on it give up after 64 polls (every other wait: MAX_SPIN)
};

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Natural LDS tile [64 rows][64] bf16: 16-byte chunk c of row r sits at chunk
// c ^ nsw(r).  A transposing read touches rows R0 .. R0 + 3 (R0 % 4 == 0) and
// two adjacent chunks per row, which then cover all 32 banks once.
__device__ __forceinline__ int nsw(int row) { return ((row & 3) << 1) | ((row >> 2) & 1); }
__device__ __forceinline__ int noff(int row, int col) {   // element offset, col % 4 == 0
    return row * R1_DH + 8 * ((col >> 3) ^ nsw(row)) + (col & 7);
}

__device__ __forceinline__ u32x2 ds_tr(bf16_t* p) {
    const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(p));
    return __builtin_bit_cast(u32x2, r);
}

// 8-bf16 MFMA operand whose contraction runs over the rows of a natural tile:
// lane l gets column cb + l % 32 and rows 16 kk + 4 (l / 32) + 0..3 (slots
// 0-3) and the same + 8 (slots 4-7).
__device__ __forceinline__ bf16x8 tr_op(bf16_t* tile, int kk, int cb, int l = threadIdx.x & 63) {
    const int i = l & 15;
    const int col = cb + 16 * ((l >> 4) & 1) + 4 * (i & 3);
    const int r0 = 16 * kk + 4 * (l >> 5) + (i >> 2);
    const u32x2 a = ds_tr(tile + noff(r0, col));
    const u32x2 b = ds_tr(tile + noff(r0 + 8, col));
    return __builtin_bit_cast(bf16x8, (u32x4{a[0], a[1], b[0], b[1]}));
}

// Descriptor over rows t0 .. L - 1 of one (batch, head) sequence (rows_range).
template <typename T>
__device__ __forceinline__ auto rows_rsrc(const T* base, int64_t rowbase, int64_t t0, int64_t L, int H, int n) {
    return seq_rsrc(base, rowbase, t0, L, H, n);
}

// Register operand of row `row` of a [64][64] tile in global memory, head-dim
// slots 16 kk + 4 (lane / 32) + 0..3 and + 8 (the accumulator-matching order).
// Each lane loads the natural 16-byte piece d = 16 kk + 8 (lane / 32) + 0..7
// (two lanes cover 32 contiguous bytes of a row), then lanes l and l + 32
// swap half of it: the lower half-wave keeps d + 0..3 and takes the partner's
// d + 8..11, the upper one takes the partner's d + 4..7 and keeps d + 12..15.
template <typename TI, typename R>
__device__ __forceinline__ bf16x8 ld_op(R rs, int row, int kk, int strideB) {
    const int hf = (threadIdx.x & 63) >> 5;
    const int off = row * strideB + (16 * kk + 8 * hf) * static_cast<int>(sizeof(TI));
    u32x4 x;
    if constexpr (sizeof(TI) == 2) {
        x = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    } else {
        const f32x4 a = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
        const f32x4 b = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16, 0, 0));
        x = u32x4{pack_bf16(a[0], a[1]), pack_bf16(a[2], a[3]), pack_bf16(b[0], b[1]), pack_bf16(b[2], b[3])};
    }
    return __builtin_bit_cast(bf16x8, x);
}
__device__ __forceinline__ bf16x8 permute_op(bf16x8 v) {
    const u32x4 x = __builtin_bit_cast(u32x4, v);
    const bool hf = ((threadIdx.x & 63) >> 5) != 0;
    const uint32_t s0 = __shfl_xor(hf ? x[0] : x[2], 32, 64);
    const uint32_t s1 = __shfl_xor(hf ? x[1] : x[3], 32, 64);
    return __builtin_bit_cast(bf16x8, hf ? (u32x4{s0, s1, x[2], x[3]}) : (u32x4{x[0], x[1], s0, s1}));
}

// 16-byte chunk (8 consecutive elements as bf16) of row `row`, chunk `ch`.
template <typename TI, typename R>
__device__ __forceinline__ u32x4 ld_chunk(R rs, int row, int ch, int strideB) {
    const int off = row * strideB + ch * 8 * static_cast<int>(sizeof(TI));
    if constexpr (sizeof(TI) == 2) {
        return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    } else {
        const f32x4 a = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
        const f32x4 b = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16, 0, 0));
        return u32x4{pack_bf16(a[0], a[1]), pack_bf16(a[2], a[3]), pack_bf16(b[0], b[1]), pack_bf16(b[2], b[3])};
    }
}

__device__ __forceinline__ uint32_t scale_bf16x2(uint32_t wd, float s) {
    return pack_bf16(__uint_as_float(wd << 16) * s, __uint_as_float(wd & 0xffff0000u) * s);
}

// Slots 8 kh .. 8 kh + 7 of a 32x32 accumulator as bf16 hi and lo operands.
__device__ __forceinline__ void split_op(const f32x16& acc, int kh, bf16x8& hi, bf16x8& lo) {
    u32x4 hw, lw;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float x0 = acc[8 * kh + 2 * q], x1 = acc[8 * kh + 2 * q + 1];
        hw[q] = pack_bf16(x0, x1);
        const float h0 = __uint_as_float(hw[q] << 16), h1 = __uint_as_float(hw[q] & 0xffff0000u);
        lw[q] = pack_bf16(x0 - h0, x1 - h1);
    }
    hi = __builtin_bit_cast(bf16x8, hw);
    lo = __builtin_bit_cast(bf16x8, lw);
}

__device__ __forceinline__ void wait_all_memory() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// bf16 one-hot B operand that makes a 32x32x16 MFMA copy its A operand:
// slot p of k-step half kh holds 1 where the A slot's head-dim index (the
// ld_op order, 16 kh + 8 (p / 4) + 4 (lane / 32) + p % 4) equals this lane's
// output column lane % 32.  The copy C[s][n] = A[s][n] comes out in the
// accumulator layout (lane = column), i.e. transposed.
__device__ __forceinline__ bf16x8 ident_op(int kh) {
    const int l = threadIdx.x & 63, n = l & 31, hf = l >> 5;
    u32x4 w{0u, 0u, 0u, 0u};
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        const int jp = 16 * kh + 8 * (p >> 2) + 4 * hf + (p & 3);
        if (jp == n) w[p >> 1] |= 0x3F80u << (16 * (p & 1));
    }
    return __builtin_bit_cast(bf16x8, w);
}

__device__ __forceinline__ bf16x8 scale_op(bf16x8 v, float s) {
    const u32x4 x = __builtin_bit_cast(u32x4, v);
    return __builtin_bit_cast(bf16x8, (u32x4{scale_bf16x2(x[0], s), scale_bf16x2(x[1], s), scale_bf16x2(x[2], s),
                                             scale_bf16x2(x[3], s)}));
}

// Keeps a computed operand in registers where it is made: without it the
// compiler sinks the producing arithmetic (and its wider fp32 inputs) down to
// the distant use, past the carry exchange.
__device__ __forceinline__ void pin(bf16x8& v) {
    u32x4 x = __builtin_bit_cast(u32x4, v);
    asm volatile("" : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]));
    v = __builtin_bit_cast(bf16x8, x);
}

__device__ __forceinline__ bf16x8 pack_op(const f32x16& acc, int kh) {
    u32x4 wd;
#pragma unroll
    for (int q = 0; q < 4; ++q) wd[q] = pack_bf16(acc[8 * kh + 2 * q], acc[8 * kh + 2 * q + 1]);
    return __builtin_bit_cast(bf16x8, wd);
}

// Offset (floats) of accumulator register group g4 of state tile T in the
// accumulator order shared by the aggregates, the carried-in states and the
// LDS chain buffer: lane-contiguous 16-byte groups.
__device__ __forceinline__ int acc_off(int T, int g4) { return ((T * 4 + g4) * 64 + (threadIdx.x & 63)) * 4; }

template <typename TF, typename TI, typename TO>
__global__ __launch_bounds__(R1_THREADS, 3) void rank1_single_kernel(Rank1SParams p) {
    __shared__ __attribute__((aligned(16))) bf16_t sV[R1_SUB][R1_T * R1_DH];   // natural V rows
    __shared__ __attribute__((aligned(16))) float sX[R1_DH * R1_DH];          // state chain / S_in / y staging
    __shared__ __attribute__((aligned(16))) float sLc[R1_SUB][R1_T];
    __shared__ __attribute__((aligned(16))) float sOmf[R1_SUB][R1_T];
    __shared__ __attribute__((aligned(16))) float sE[R1_SUB][R1_T];
    __shared__ float sLcT[R1_SUB];
    __shared__ float sLcS[R1S_MAX_SC];
    __shared__ float sCarry[R1_THREADS];   // slice scan: value handed from one part to the next
    __shared__ uint32_t sEpoch;
    __shared__ int sFail;

    const int nsc = p.nsc;
    const int seq = blockIdx.x / nsc, c = blockIdx.x - seq * nsc;
    const int b = seq / p.H, hh = seq - (seq / p.H) * p.H;
    // wave j owns sub-chunk j (readfirstlane: uniform, so the buffer descriptors stay scalar)
    const int tid = threadIdx.x, lane = tid & 63, j = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t rowbase = static_cast<int64_t>(b) * p.L * p.H + hh;
    const int64_t t0 = static_cast<int64_t>(c) * R1_RS + j * R1_T;
    const int strideI = p.H * R1_DH * static_cast<int>(sizeof(TI));
    const TF* fp = static_cast<const TF*>(p.f);

    // ---- 1. k, v, f; decays; V rows to LDS; K diag(w) transposed ----------
    const TF fraw = fp[rowbase + (t0 + lane < p.L ? t0 + lane : p.L - 1) * p.H];
    const auto rq = rows_rsrc(static_cast<const TI*>(p.q), rowbase, t0, p.L, p.H, R1_DH);
    const auto rk = rows_rsrc(static_cast<const TI*>(p.k), rowbase, t0, p.L, p.H, R1_DH);
    const auto rv = rows_rsrc(static_cast<const TI*>(p.v), rowbase, t0, p.L, p.H, R1_DH);
    bf16x8 kop[2][4];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) kop[rt][kk] = ld_op<TI>(rk, 32 * rt + (lane & 31), kk, strideI);
    u32x4 vch[8];
#pragma unroll
    for (int n = 0; n < 8; ++n) vch[n] = ld_chunk<TI>(rv, (lane >> 3) + 8 * n, lane & 7, strideI);
    bf16x8 qop[2][4];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) qop[rt][kk] = ld_op<TI>(rq, 32 * rt + (lane & 31), kk, strideI);
    if (tid == 0) {
        sEpoch = ld_relaxed(&p.hdr[2]);
        sFail = 0;
    }
    const float fv = fval<TF>(fraw, t0 + lane, p.L);
    const float lc = wave_incl_scan(fmaxf(__log2f(fv), R1_LOG2_MIN));
    const float lcT = __shfl(lc, 63, 64);
    const float wgt = exp2_hw(lcT - lc) * (1.0f - fv);
    sLc[j][lane] = lc;
    sOmf[j][lane] = 1.0f - fv;
    sE[j][lane] = exp2_hw(lc);
    if (lane == 63) sLcT[j] = lcT;
#pragma unroll
    for (int n = 0; n < 8; ++n) {
        const int s = (lane >> 3) + 8 * n;
        *reinterpret_cast<u32x4*>(&sV[j][noff(s, 8 * (lane & 7))]) = vch[n];
    }
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) kop[rt][kk] = permute_op(kop[rt][kk]);
    // (K diag(w))^T as dS A operands kwt[sb][jb][kh]: rows j, steps s of block sb
    bf16x8 kwt[2][2][2];
    {
        const float w0 = __shfl(wgt, lane & 31, 64), w1 = __shfl(wgt, (lane & 31) + 32, 64);
        const bf16x8 id0 = ident_op(0), id1 = ident_op(1);
#pragma unroll
        for (int sb = 0; sb < 2; ++sb)
#pragma unroll
            for (int jb = 0; jb < 2; ++jb) {
                const float ws = sb ? w1 : w0;
                f32x16 cc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(scale_op(kop[sb][2 * jb], ws), id0, zero16(), 0, 0, 0);
                cc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(scale_op(kop[sb][2 * jb + 1], ws), id1, cc, 0, 0, 0);
                kwt[sb][jb][0] = pack_op(cc, 0);
                kwt[sb][jb][1] = pack_op(cc, 1);
            }
    }
    __syncthreads();
    const uint32_t epoch = sEpoch;
    float lcStart = 0.0f, lcS = 0.0f;
#pragma unroll
    for (int m = 0; m < R1_SUB; ++m) {
        if (m < j) lcStart += sLcT[m];
        lcS += sLcT[m];
    }

    // ---- P^T = K Q^T decayed and masked, tiles (sb, tb) = (0,0), (0,1), (1,1),
    // before the state exists (K, Q, P and the state together exceed the
    // register budget of three work-groups per CU)
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) qop[rt][kk] = permute_op(qop[rt][kk]);
    bf16x8 pb[3][2];
    {
        // (1,1) first: the K operand rows 32..63 die after it
        constexpr int SB[3] = {0, 0, 1}, TB[3] = {0, 1, 1};
#pragma unroll
        for (int n = 2; n >= 0; --n) {
            f32x16 acc = zero16();
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kop[SB[n]][kk], qop[TB[n]][kk], acc, 0, 0, 0);
            const int t = 32 * TB[n] + (lane & 31);
            const float lct = sLc[j][t];
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const int s0 = 32 * SB[n] + 8 * g4 + 4 * (lane >> 5);
                const f32x4 ls = *reinterpret_cast<const f32x4*>(&sLc[j][s0]);
                const f32x4 om = *reinterpret_cast<const f32x4*>(&sOmf[j][s0]);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int r = 4 * g4 + q;
                    acc[r] = (s0 + q <= t) ? acc[r] * exp2_hw(lct - ls[q]) * om[q] : 0.0f;
                }
            }
            pb[n][0] = pack_op(acc, 0);
            pb[n][1] = pack_op(acc, 1);
            pin(pb[n][0]);
            pin(pb[n][1]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // ---- 2. dS_j^T = (K diag(w))^T V_j; state chain through LDS ------------
    f32x16 S[2][2];   // [jb][ib]: dS_j^T, then S_j^loc^T (state at this sub-chunk's start)
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int e = 0; e < 2; ++e) S[a][e] = zero16();
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
            const bf16x8 v0 = tr_op(sV[j], 2 * sb + kh, 0), v1 = tr_op(sV[j], 2 * sb + kh, 32);
#pragma unroll
            for (int jb = 0; jb < 2; ++jb) {
                S[jb][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kwt[sb][jb][kh], v0, S[jb][0], 0, 0, 0);
                S[jb][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kwt[sb][jb][kh], v1, S[jb][1], 0, 0, 0);
            }
        }
    float* const aggSeq = p.agg + static_cast<int64_t>(seq) * nsc * (R1_DH * R1_DH);
    float* const sinSeq = p.sin + static_cast<int64_t>(seq) * nsc * (R1_DH * R1_DH);
    const auto rAgg = __builtin_amdgcn_make_buffer_rsrc(aggSeq, 0, nsc * R1_DH * R1_DH * 4, 0x00020000);
    const auto rSin = __builtin_amdgcn_make_buffer_rsrc(sinSeq, 0, nsc * R1_DH * R1_DH * 4, 0x00020000);
    // wave m reads X_m = S_m^loc and writes X_{m+1} = 2^LcT_m X_m + dS_m in place;
    // wave 3 turns X_4 into the super-chunk's aggregate and publishes it
    const bool publish = c + 1 < nsc && !(p.skip_agg0 && c == 0);
#pragma unroll
    for (int m = 0; m < R1_SUB; ++m) {
        if (j == m) {
            const float dec = exp2_hw(sLcT[m]);
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int e = 0; e < 2; ++e)
#pragma unroll
                    for (int g4 = 0; g4 < 4; ++g4) {
                        const int off = acc_off(2 * a + e, g4);
                        const f32x4 x = m > 0 ? *reinterpret_cast<const f32x4*>(&sX[off]) : f32x4{0.f, 0.f, 0.f, 0.f};
                        f32x4 nx;
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            nx[q] = fmaf(dec, x[q], S[a][e][4 * g4 + q]);
                            S[a][e][4 * g4 + q] = x[q];
                        }
                        if (m + 1 < R1_SUB)
                            *reinterpret_cast<f32x4*>(&sX[off]) = nx;
                        else if (publish)
                            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, nx), rAgg,
                                                                   (c * R1_DH * R1_DH + off) * 4, 0, R1_SC1);
                    }
            if (m + 1 == R1_SUB && publish) {
                wait_all_memory();
                if (lane == 0)
                    st_relaxed(&p.flag1[static_cast<int64_t>(seq) * nsc + c], pack_word(lcS, make_tag(epoch, ST_AGG)));
            }
        }
        if (m + 1 < R1_SUB) __syncthreads();
    }

    // ---- 3. carries -------------------------------------------------------
    const int64_t fbase = static_cast<int64_t>(seq) * nsc;
    if (nsc > 1) {
        if (j == 0 && lane < nsc - 1) {   // every aggregate of the sequence but the last
            const uint32_t tag = make_tag(epoch, ST_AGG);
            uint64_t wd = ld_relaxed(&p.flag1[fbase + lane]);
            const uint32_t limit = p.skip_agg0 && lane == 0 ? 64u : MAX_SPIN;
            uint32_t n = 0;
            bool ok = true;
            while (word_tag(wd) != tag) {
                if (++n > limit) {
                    note_timeout(p.hdr);
                    ok = false;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
                wd = ld_relaxed(&p.flag1[fbase + lane]);
            }
            sLcS[lane] = ok ? word_val(wd) : __builtin_nanf("");
        }
        __syncthreads();
        // slice [e0, e1) of every carried-in state: S_in(m + 1) = 2^LcS_m S_in(m) + agg_m
        const int E = (R1_DH * R1_DH + nsc - 1) / nsc;
        const int e0 = c * E, e1 = min(R1_DH * R1_DH, e0 + E);
        // Every aggregate load of a thread's part in one batch, straight into
        // LDS (the chain buffer, free until the carried-in state lands in it):
        // the aggregates are cut into parts of R1S_NB, thread (part, el) of a
        // round loads its part of element e0 + round * epr + el into
        // sX[i * R1_THREADS + tid], and the parts continue the recurrence in
        // turn from the value the previous part ended with: the same
        // operations in the same order as one thread walking every aggregate.
        const int nagg = nsc - 1, parts = (nagg + R1S_NB - 1) / R1S_NB;
        const int epr = R1_THREADS / parts, rounds = (E + epr - 1) / epr;
        const lds_i32x4 rAggD = lds_rsrc(aggSeq, static_cast<uint32_t>(nsc) * R1_DH * R1_DH * 4);
        const uint32_t sxw = lds_addr(sX) + j * 256;   // this wave's 64 slots of a row of sX
        for (int rd = 0; rd < rounds; ++rd) {
            const int part = tid / epr, el = rd * epr + (tid - part * epr);
            const bool act = part < parts && e0 + el < e1;
            const int mb = part * R1S_NB;
            // this wave's reads of its slots are done before the loads overwrite them
            __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0)
#pragma unroll
            for (int i = 0; i < R1S_NB; ++i)   // inactive lanes and past the aggregates: out of range, load 0
                r1_dma4_sc1(rAggD, ((act && mb + i < nagg ? mb + i : nsc) * R1_DH * R1_DH + (act ? e0 + el : 0)) * 4,
                            sxw + i * (R1_THREADS * 4));
            lds_wait_vm<0>();   // each thread reads only the slots its own wave loaded
            for (int q = 0; q < parts; ++q) {
                if (act && part == q) {
                    float Sv = q > 0 ? sCarry[el] : 0.0f;
                    // offsets formed here from an opaque base, so none is held across the barriers
                    int so = ((mb + 1) * R1_DH * R1_DH + e0 + el) * 4;
                    asm volatile("" : "+v"(so));
#pragma unroll
                    for (int i = 0; i < R1S_NB; ++i) {
                        const int m = mb + i;
                        if (m < nagg) {
                            Sv = fmaf(exp2_hw(sLcS[m]), Sv, sX[i * R1_THREADS + tid]);
                            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(Sv), rSin, so + i * (R1_DH * R1_DH * 4),
                                                                  0, R1_SC1);
                        }
                    }
                    if (q + 1 < parts) sCarry[el] = Sv;
                }
                if (q + 1 < parts) __syncthreads();
            }
        }
        wait_all_memory();
        __syncthreads();
        if (tid == 0) st_relaxed(&p.flag2[fbase + c], make_tag(epoch, ST_INC));
    } else if (tid == 0) {
        st_relaxed(&p.flag2[fbase + c], make_tag(epoch, ST_INC));
    }

    // ---- carried-in state: S_j = 2^Lc_start_j S_in + S_j^loc -----------------
    if (nsc > 1 && c > 0) {
        if (j == 0 && lane < nsc) {   // every slice written
            const uint32_t tag = make_tag(epoch, ST_INC);
            uint32_t n = 0;
            while (ld_relaxed(&p.flag2[fbase + lane]) != tag) {
                if (++n > MAX_SPIN) {
                    note_timeout(p.hdr);
                    sFail = 1;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        __syncthreads();
#pragma unroll
        for (int n = 0; n < 4; ++n) {   // S_in (accumulator order) into the chain buffer
            const int o = 4 * (tid + R1_THREADS * n);
            *reinterpret_cast<u32x4*>(&sX[o]) = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(rSin, (c * R1_DH * R1_DH + o) * 4, 0, R1_SC1));
        }
        __syncthreads();
        const float es = sFail ? __builtin_nanf("") : exp2_hw(lcStart);
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int e = 0; e < 2; ++e)
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const f32x4 x = *reinterpret_cast<const f32x4*>(&sX[acc_off(2 * a + e, g4)]);
#pragma unroll
                    for (int q = 0; q < 4; ++q) S[a][e][4 * g4 + q] = fmaf(es, x[q], S[a][e][4 * g4 + q]);
                }
    }
    __syncthreads();   // the chain buffer is free: y staging from here

    // ---- 4. y = 2^Lc_t Q S_j^T + P V, one column block ib at a time ---------
    constexpr int SO = static_cast<int>(sizeof(TO));
    const int strideO = p.H * R1_DH * SO;
    const auto ry = rows_rsrc(static_cast<const TO*>(p.y), rowbase, t0, p.L, p.H, R1_DH);
    bf16_t* const sy = reinterpret_cast<bf16_t*>(sX) + j * (R1_T * 32);   // [64 t][32 i] per wave
    // S_j^T as bf16 hi + lo operands, made once (the fp32 state dies here)
    bf16x8 sh[4][2], sl[4][2];   // [kk][ib]
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int ib = 0; ib < 2; ++ib) {
            split_op(S[kk >> 1][ib], kk & 1, sh[kk][ib], sl[kk][ib]);
            pin(sh[kk][ib]);
            pin(sl[kk][ib]);
        }
#pragma unroll
    for (int ib = 0; ib < 2; ++ib) {
        // The lane index made opaque here, so the LDS addresses below are
        // formed where they are used: otherwise the compiler keeps the same
        // addresses of the earlier phases alive across the carry exchange,
        // spills them and reloads them one scratch round trip at a time.
        int ol = lane;
        asm volatile("" : "+v"(ol));
        // staging offset of accumulator row group q (row t = 32 tb + 8 g4 +
        // 4 (lane / 32) + q, chunk (i / 8) ^ (t % 4)): 4 registers for all 16 rows
        int qoff[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
            qoff[q] = (4 * (ol >> 5) + q) * 32 + 8 * (((ol & 31) >> 3) ^ q) + (ol & 7);
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            f32x16 acc = zero16();
            if (j > 0 || c > 0) {
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qop[tb][kk], sh[kk][ib], acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qop[tb][kk], sl[kk][ib], acc, 0, 0, 0);
                }
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const f32x4 e4 = *reinterpret_cast<const f32x4*>(&sE[j][32 * tb + 8 * g4 + 4 * (lane >> 5)]);
#pragma unroll
                    for (int q = 0; q < 4; ++q) acc[4 * g4 + q] *= e4[q];
                }
            }
#pragma unroll
            for (int sb = 0; sb <= tb; ++sb)
#pragma unroll
                for (int kh = 0; kh < 2; ++kh)
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pb[tb == 0 ? 0 : 1 + sb][kh],
                                                                  tr_op(sV[j], 2 * sb + kh, 32 * ib, ol), acc, 0, 0, 0);
            if constexpr (SO == 2) {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    sy[(32 * tb + 8 * (r >> 2)) * 32 + qoff[r & 3]] = f32_to_bf16(acc[r]);
            } else {
                const int colB = (32 * ib + (lane & 31)) * SO;
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[r]), ry,
                                                          (32 * tb + mrow(r)) * strideO + colB, 0, 2);
            }
        }
        if constexpr (SO == 2) {   // this wave's [64 t][32 i] block as 16-byte row pieces
#pragma unroll
            for (int n = 0; n < 4; ++n) {
                const int t = (ol >> 2) + 16 * n, ch = ol & 3;
                const u32x4 x = *reinterpret_cast<const u32x4*>(&sy[t * 32 + 8 * (ch ^ (t & 3))]);
                __builtin_amdgcn_raw_buffer_store_b128(x, ry, t * strideO + (32 * ib + 8 * ch) * SO, 0, 2);
            }
        }
    }
    ws_finish(p.hdr, p.flag2, static_cast<int64_t>(gridDim.x), epoch, make_tag(epoch, ST_INC));
}

namespace {

struct R1Geo {
    int nsc;
    size_t off_ds, off_lct, off_sin, bytes;
    size_t s_flag1, s_flag2, s_agg, s_sin, s_bytes;   // single-pass layout
};

R1Geo r1_geometry(int64_t B, int64_t L, int64_t H) {
    R1Geo g{};
    g.nsc = static_cast<int>((L + R1_RS - 1) / R1_RS);
    const size_t nseq = static_cast<size_t>(B) * H;
    size_t off = WS_HDR_BYTES;
    auto take = [&](size_t n) { size_t o = off; off = round_up(off + n, 256); return o; };
    g.off_ds = take(nseq * g.nsc * R1_DH * R1_DH * sizeof(float));
    g.off_lct = take(nseq * g.nsc * sizeof(float));
    g.off_sin = take(nseq * g.nsc * R1_DH * R1_DH * sizeof(float));
    g.bytes = off;
    off = WS_HDR_BYTES;
    g.s_flag1 = take(nseq * g.nsc * sizeof(uint64_t));
    g.s_flag2 = take(nseq * g.nsc * sizeof(uint32_t));
    g.s_agg = take(nseq * g.nsc * R1_DH * R1_DH * sizeof(float));
    g.s_sin = take(nseq * g.nsc * R1_DH * R1_DH * sizeof(float));
    g.s_bytes = off;
    return g;
}

template <typename TF, typename TI, typename TO>
int run_rank1(const Rank1Params& prm, int n_seq, hipStream_t st) {
    const dim3 grid(prm.nsc, n_seq);
    hipLaunchKernelGGL((rank1_summary_kernel<TF, TI>), grid, dim3(R1_THREADS), 0, st, prm);
    int rc = check_launch("rank1_summary_kernel");
    if (rc) return rc;
    hipLaunchKernelGGL(rank1_carry_kernel, dim3(R1_DH * R1_DH / 256, n_seq), dim3(256), 0, st, prm);
    rc = check_launch("rank1_carry_kernel");
    if (rc) return rc;
    hipLaunchKernelGGL((rank1_output_kernel<TF, TI, TO>), grid, dim3(R1_THREADS), 0, st, prm);
    return check_launch("rank1_output_kernel");
}

template <typename TF, typename TI, typename TO>
int run_rank1_single(const Rank1SParams& prm, int n_seq, hipStream_t st) {
    hipLaunchKernelGGL((rank1_single_kernel<TF, TI, TO>), dim3(n_seq * prm.nsc), dim3(R1_THREADS), 0, st, prm);
    return check_launch("rank1_single_kernel");
}

// The one-launch kernel takes bf16 k, v, q only: fp32 operands would double
// its load registers past the budget of three work-groups per CU, so fp32
// k, v, q always take the three-launch path.
template <typename TF, typename TI, typename TO>
int run_path(bool single, const Rank1Params& p3, const Rank1SParams& p1, int n_seq, hipStream_t st) {
    if constexpr (sizeof(TI) == 2) {
        if (single) return run_rank1_single<TF, TI, TO>(p1, n_seq, st);
    }
    return run_rank1<TF, TI, TO>(p3, n_seq, st);
}

}  // namespace
}  // namespace mogt

using namespace mogt;

extern "C" size_t mogt_rank1_coupled_scan_workspace_bytes(int64_t batch, int64_t length, int64_t heads,
                                                          int64_t head_dim) {
    if (batch <= 0 || length <= 0 || heads <= 0 || head_dim != R1_DH) return WS_HDR_BYTES;
    const R1Geo g = r1_geometry(batch, length, heads);
    return g.bytes > g.s_bytes ? g.bytes : g.s_bytes;
}

extern "C" int mogt_rank1_coupled_scan_fwd_cfg(const void* f, const void* k, const void* v, const void* q,
                                               void* y, int64_t batch, int64_t length, int64_t heads,
                                               int64_t head_dim, int f_dtype, int kvq_dtype, int out_dtype,
                                               void* workspace, size_t workspace_bytes, int path,
                                               void* stream) {
    clear_error();
    if (batch < 0 || length < 0 || heads <= 0)
        return set_error(MOGT_E_INVALID, "f must be [B, L, H] and k, v, q [B, L, H, d]");
    if (head_dim != R1_DH) return set_error(MOGT_E_INVALID, "head_dim %lld not supported (64)", (long long)head_dim);
    for (int d : {f_dtype, kvq_dtype, out_dtype})
        if (d != MOGT_F32 && d != MOGT_BF16) return set_error(MOGT_E_INVALID, "unsupported dtype code");
    if (path < 0 || path > 3) return set_error(MOGT_E_INVALID, "path %d not in {0, 1, 2, 3}", path);
    if (batch == 0 || length == 0) return MOGT_OK;
    if (!f || !k || !v || !q || !y) return set_error(MOGT_E_INVALID, "null tensor pointer");
    if (batch * heads > 65535) return set_error(MOGT_E_INVALID, "batch * heads > 65535");
    if (length > (int64_t(1) << 40)) return set_error(MOGT_E_INVALID, "length too large");
    const R1Geo g = r1_geometry(batch, length, heads);
    const bool bf16_io = kvq_dtype == MOGT_BF16;
    // By default the one-launch form runs when all its work-groups are resident
    // together (three per CU): every further generation of work-groups pays the
    // whole carry exchange again, and the three launches then win (B = 2,
    // L = 16384, H = 12: 97 vs 94 us).
    int cus = 0;
    const int64_t n_groups = batch * heads * g.nsc;
    const bool one_gen = device_cu_count(cus) == MOGT_OK && n_groups <= int64_t(R1S_GROUPS_PER_CU) * cus;
    clear_error();
    const bool single = path == 1 || path == 3 || (path == 0 && g.nsc <= R1S_MAX_SC && bf16_io && one_gen);
    if (path == 3 && g.nsc < 2)
        return set_error(MOGT_E_INVALID, "the give-up test path needs at least 2 super-chunks (L > %d)", R1_RS);
    if (single && g.nsc > R1S_MAX_SC)
        return set_error(MOGT_E_INVALID, "single-pass rank-1 scan takes at most %d super-chunks (L <= %d)",
                         R1S_MAX_SC, R1S_MAX_SC * R1_RS);
    if (single && !bf16_io) return set_error(MOGT_E_INVALID, "single-pass rank-1 scan takes bf16 k, v, q");
    const size_t need = single ? g.s_bytes : g.bytes;
    if (!workspace || workspace_bytes < need)
        return set_error(MOGT_E_WORKSPACE, "workspace of %zu bytes required, got %zu", need, workspace_bytes);
    char* base = static_cast<char*>(workspace);
    Rank1Params p3{};
    p3.f = f; p3.k = k; p3.v = v; p3.q = q; p3.y = y;
    p3.dS = reinterpret_cast<float*>(base + g.off_ds);
    p3.lcT = reinterpret_cast<float*>(base + g.off_lct);
    p3.Sin = reinterpret_cast<float*>(base + g.off_sin);
    p3.L = length; p3.H = static_cast<int>(heads); p3.nsc = g.nsc;
    Rank1SParams p1{};
    p1.f = f; p1.k = k; p1.v = v; p1.q = q; p1.y = y;
    p1.hdr = reinterpret_cast<uint32_t*>(base);
    p1.flag1 = reinterpret_cast<uint64_t*>(base + g.s_flag1);
    p1.flag2 = reinterpret_cast<uint32_t*>(base + g.s_flag2);
    p1.agg = reinterpret_cast<float*>(base + g.s_agg);
    p1.sin = reinterpret_cast<float*>(base + g.s_sin);
    p1.L = length; p1.H = static_cast<int>(heads); p1.nsc = g.nsc;
    // path 3 (tests): super-chunk 0 withholds its aggregate; each work-group's
    // wait on it gives up after 64 polls and is counted once
    p1.skip_agg0 = path == 3;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int n_seq = static_cast<int>(batch * heads);
    const bool fb = f_dtype == MOGT_BF16, ib = kvq_dtype == MOGT_BF16, ob = out_dtype == MOGT_BF16;
    if (fb && ib && ob) return run_path<bf16_t, bf16_t, bf16_t>(single, p3, p1, n_seq, st);
    if (fb && ib && !ob) return run_path<bf16_t, bf16_t, float>(single, p3, p1, n_seq, st);
    if (!fb && ib && ob) return run_path<float, bf16_t, bf16_t>(single, p3, p1, n_seq, st);
    if (!fb && ib && !ob) return run_path<float, bf16_t, float>(single, p3, p1, n_seq, st);
    if (fb && !ib && ob) return run_path<bf16_t, float, bf16_t>(single, p3, p1, n_seq, st);
    if (fb && !ib && !ob) return run_path<bf16_t, float, float>(single, p3, p1, n_seq, st);
    if (!fb && !ib && ob) return run_path<float, float, bf16_t>(single, p3, p1, n_seq, st);
    return run_path<float, float, float>(single, p3, p1, n_seq, st);
}

extern "C" int mogt_rank1_coupled_scan_fwd(const void* f, const void* k, const void* v, const void* q,
                                           void* y, int64_t batch, int64_t length, int64_t heads,
                                           int64_t head_dim, int f_dtype, int kvq_dtype, int out_dtype,
                                           void* workspace, size_t workspace_bytes, void* stream) {
    return mogt_rank1_coupled_scan_fwd_cfg(f, k, v, q, y, batch, length, heads, head_dim, f_dtype, kvq_dtype,
                                           out_dtype, workspace, workspace_bytes, 0, stream);
}

extern "C" int mogt_rank1_check_ranges(int64_t batch, int64_t length, int64_t heads, int elem_bytes) {
    clear_error();
    if (batch <= 0 || length <= 0 || heads <= 0 || (elem_bytes != 2 && elem_bytes != 4))
        return set_error(MOGT_E_INVALID, "batch, length, heads > 0 and elem_bytes 2 or 4 expected");
    const R1Geo g = r1_geometry(batch, length, heads);
    const int64_t total = batch * length * heads * R1_DH * elem_bytes;   // bytes of one [B, L, H, 64] tensor
    const int64_t strideB = heads * R1_DH * elem_bytes;
    if (63 * strideB + R1_DH * elem_bytes > 0x7fffffff)
        return set_error(MOGT_E_INVALID, "a 64-row tile spans more than 2 GiB");
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t h = 0; h < heads; ++h) {
            const int64_t rowbase = b * length * heads + h;
            // every sub-chunk start the kernels build a descriptor for: K_A's
            // prefetches, K_C's and the one-launch kernel's sub-chunks, and the
            // tiles of a padding super-chunk past the end
            for (int64_t t0 = 0; t0 <= (static_cast<int64_t>(g.nsc) + 1) * R1_RS; t0 += R1_T) {
                const RowsRange r = rows_range(rowbase, t0, length, static_cast<int>(heads), R1_DH, elem_bytes);
                const int64_t start = r.base * elem_bytes;
                if (r.span < 0 || start < 0 || start + r.span > total)
                    return set_error(MOGT_E_INVALID,
                                     "b %lld h %lld t0 %lld: range [%lld, %lld) outside the %lld-byte tensor",
                                     (long long)b, (long long)h, (long long)t0, (long long)start,
                                     (long long)(start + r.span), (long long)total);
                // rows t0 .. min(L, t0 + 64) - 1 are read in full inside the
                // range; every later row of the tile starts past its end
                const int64_t live = t0 < length ? (length - t0 < R1_T ? length - t0 : R1_T) : 0;
                if (live > 0 && (live - 1) * strideB + R1_DH * elem_bytes > r.span)
                    return set_error(MOGT_E_INVALID, "t0 %lld: live rows cut off by the range", (long long)t0);
                if (live < R1_T && live * strideB < r.span)
                    return set_error(MOGT_E_INVALID, "t0 %lld: row %lld past L inside the range",
                                     (long long)t0, (long long)live);
            }
        }
    return MOGT_OK;
}
