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
#include "common.h"

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

// Descriptor over the rows t0 .. L - 1 of one (batch, head) sequence of a
// [B, L, H, n] tensor with n elements of T per row (t0 < L).
template <typename T>
__device__ __forceinline__ auto seq_rsrc(const T* base, int64_t rowbase, int64_t t0, int64_t L, int H, int n) {
    const int64_t strideB = static_cast<int64_t>(H) * n * sizeof(T);
    const int64_t span = (L - 1 - t0) * strideB + static_cast<int64_t>(n) * sizeof(T);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(base) + (rowbase + t0 * H) * n, 0,
                                             static_cast<int>(span < 0x7fffffff ? span : 0x7fffffff), 0x00020000);
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

namespace {

struct R1Geo {
    int nsc;
    size_t off_ds, off_lct, off_sin, bytes;
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
    if (length > (int64_t(1) << 40)) return set_error(MOGT_E_INVALID, "length too large");
    char* base = static_cast<char*>(workspace);
    Rank1Params prm{};
    prm.f = f; prm.k = k; prm.v = v; prm.q = q; prm.y = y;
    prm.dS = reinterpret_cast<float*>(base + g.off_ds);
    prm.lcT = reinterpret_cast<float*>(base + g.off_lct);
    prm.Sin = reinterpret_cast<float*>(base + g.off_sin);
    prm.L = length; prm.H = static_cast<int>(heads); prm.nsc = g.nsc;
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
