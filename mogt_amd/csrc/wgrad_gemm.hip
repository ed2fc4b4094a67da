// Weight gradient of a bias-free bf16 nn.Linear as a split-K GEMM on the
// matrix cores:
//   dW[o][i] = sum_t dY[t][o] * X[t][i]
// dY [T, d_out] (row stride ldd), X [T, d_in] (row stride ldx), bf16; dW
// [d_out, d_in] (row stride ldw), bf16 or fp32; fp32 accumulation.  This is
// the product autograd forms for the weight of the model's linear layers
// (model_mogt.py:25-27 w1, w2, w3; :57 phi_val; :61 theta_read) in the
// backward.  Torch hands it to the BLAS library as one GEMM whose output
// (d_out x d_in, e.g. 768 x 768) has too few tiles to fill 256 CUs, while its
// contraction (T = B * L = 32768 tokens) is long.
//
// Here the tokens are split into S slices.  Work-group (tile, slice) forms a
// 256 x 256 block of dW over its slice into an fp32 partial buffer
// [S, d_out, d_in]; a second kernel sums the S partials in slice order (so
// the result does not depend on scheduling) and rounds once.  S is chosen so
// that tiles x S fills the CUs.
//
// Both operands are token-major: the contraction index is the slow one, but
// the MFMA wants K-contiguous fragments.  Tiles reach LDS as they lie in
// memory (32 tokens x 256 columns per operand and stage, by direct
// buffer-to-LDS loads), and fragments are read with gfx950's transposing LDS
// read, ds_read_b64_tr_b16: within each group of 16 lanes, lanes 4r .. 4r + 3
// address row r of a 4 x 16 block (4 consecutive elements each) and lane j
// receives column j of the block, i.e. 4 consecutive tokens of one column.
// Two such reads give a lane the 8 K-values of a v_mfma_f32_32x32x16_bf16
// operand.  Which token feeds which K-slot is free (the MFMA sums over them)
// as long as both operands agree: lane half h (lane / 32), slot q ->
// token 4 (2 (q / 4) + h) + q % 4 of the 16-token K-step, so one read
// instruction covers 8 consecutive token rows.  An LDS row (one token) holds
// 256 columns, 512 B, as 8 chunks of 64 B (32 columns); chunk c of row r is
// stored at position c ^ (r % 8), so the 8 rows of one read hit 8 different
// chunk positions and every bank equally.
//
// Work-group tile 256 (o) x 256 (i), 4 waves of 128 x 128: 4 x 4 accumulator
// tiles of D[i][o] (MFMA A operand = X fragment, B = dY fragment), so a lane's
// 16 results are 4 groups of 4 consecutive i of one o, each stored as one
// 16-byte write of the partial.  The stage pipeline (four stages of 32 tokens
// in flight, fragments read one stage ahead, the next stage's loads and
// fragment reads interleaved one to one with the current stage's MFMAs) is
// that of the fused SwiGLU GEMM (swiglu_gemm.hip).
//
// Work-groups are renumbered XCD-aware (the hardware deals them round-robin
// over the 8 XCDs): each XCD gets a contiguous run of (slice, tile) pairs,
// tiles fastest, so the tiles of one slice share that XCD's L2 for their
// common dY and X rows.
#include <type_traits>

#include "lds_dma.h"

namespace mogt {
namespace {

typedef __bf16 wg_bf16x8 __attribute__((ext_vector_type(8)));
typedef short wg_i16x4 __attribute__((ext_vector_type(4)));
typedef short wg_i16x8 __attribute__((ext_vector_type(8)));
typedef float wg_f32x16 __attribute__((ext_vector_type(16)));
typedef float wg_f32x4 __attribute__((ext_vector_type(4)));
typedef float wg_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 wg_bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t wg_u32x4 __attribute__((ext_vector_type(4)));

constexpr int WG_BT = 256;                   // tile edge along d_out and d_in
constexpr int WG_BK = 32;                    // tokens per stage
constexpr int WG_NST = 4;                    // stages in LDS
constexpr int WG_THREADS = 256;              // 4 waves
constexpr int WG_ROWB = WG_BT * 2;           // bytes per LDS row (one token)
constexpr int WG_OPB = WG_BK * WG_ROWB;      // one operand of a stage (16 KB)
constexpr int WG_STB = 2 * WG_OPB;           // one stage (32 KB)
constexpr int WG_MIN_SLICE = 128;            // fewest tokens per slice (4 stages)

struct WgradParams {
    const bf16_t* dy;    // [T, d_out]
    const bf16_t* x;     // [T, d_in]
    float* part;         // [slices, d_out, d_in]
    int64_t T;
    int64_t ldd, ldx;    // elements
    int d_out, d_in;
    int n_ot, n_it;      // tiles along d_out, d_in
    int slices, slice;   // S, tokens per slice (multiple of WG_BK)
};

// block id -> (tile along d_out, tile along d_in, slice)
__device__ __forceinline__ void wg_tile(const WgradParams& p, int& ot, int& it, int& s) {
    const int tiles = p.n_ot * p.n_it;
    const int n = tiles * p.slices;
    const int bid = blockIdx.x;
    const int q = n >> 3, rem = n & 7;
    const int xcd = bid & 7, loc = bid >> 3;
    const int v = xcd < rem ? xcd * (q + 1) + loc : rem * (q + 1) + (xcd - rem) * q + loc;
    s = v / tiles;
    const int t = v - s * tiles;
    ot = t / p.n_it;
    it = t - ot * p.n_it;
}

// 4 consecutive tokens of one column, transposed out of LDS (see the header)
__device__ __forceinline__ wg_i16x4 wg_read_tr(const char* p) {
    typedef __attribute__((address_space(3))) wg_i16x4 lds_i16x4;
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_i16x4*)((__attribute__((address_space(3))) char*)(const_cast<char*>(p))));
}

__global__ __launch_bounds__(WG_THREADS) void wgrad_gemm_kernel(WgradParams p) {
    __shared__ __attribute__((aligned(1024))) char smem[WG_NST * WG_STB];   // [stage][dY | X][32 tokens][512 B]
    int ot, it, s;
    wg_tile(p, ot, it, s);
    const int o0 = ot * WG_BT, i0 = it * WG_BT;
    const int64_t t0 = static_cast<int64_t>(s) * p.slice;
    const int64_t tl = p.T - t0 < p.slice ? p.T - t0 : p.slice;   // >= 1 (host)
    const int nk = static_cast<int>((tl + WG_BK - 1) / WG_BK);
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int l32 = lane & 31, hb = lane >> 5;
    const uint32_t lds0 = lds_addr(smem);

    // Loads: wave w fills token rows 8 w .. 8 w + 7 of each operand's stage
    // tile, 2 rows (1 KB) per instruction; lane L takes row 8 w + 2 i + L / 32
    // and LDS slot L % 32 of it (16 B), which under the swizzle holds global
    // chunk ((slot / 4) ^ (row % 8)), columns + 8 (slot % 4).  The descriptors
    // end at the slice's last token (past it, and past the matrix, loads
    // return zero); columns past d_out / d_in within a row only reach outputs
    // that are not stored.  Stage offsets go into the per-lane offset, which
    // is what the range check covers.
    const lds_i32x4 rd = lds_rsrc(p.dy + t0 * p.ldd + o0, static_cast<uint32_t>(((tl - 1) * p.ldd + (p.d_out - o0)) * 2));
    const lds_i32x4 rx = lds_rsrc(p.x + t0 * p.ldx + i0, static_cast<uint32_t>(((tl - 1) * p.ldx + (p.d_in - i0)) * 2));
    int vd[4], vx[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = 8 * wave + 2 * i + (lane >> 5), q = lane & 31;
        const int col = (((q >> 2) ^ (r & 7)) << 5) + ((q & 3) << 3);
        vd[i] = static_cast<int>((r * p.ldd + col) * 2);
        vx[i] = static_cast<int>((r * p.ldx + col) * 2);
    }
    const int sd = static_cast<int>(WG_BK * p.ldd * 2), sx = static_cast<int>(WG_BK * p.ldx * 2);
    const uint32_t dd = lds0 + wave * 4096, dx = lds0 + WG_OPB + wave * 4096;
    auto issue = [&](int k) {
        const uint32_t st = (k & (WG_NST - 1)) * WG_STB;
#pragma unroll
        for (int i = 0; i < 4; ++i) lds_dma16(rd, vd[i] + k * sd, 0, dd + st + i * 1024);
#pragma unroll
        for (int i = 0; i < 4; ++i) lds_dma16(rx, vx[i] + k * sx, 0, dx + st + i * 1024);
    };

    // Fragment reads: lane l (group G = l / 16, j = l % 16, half h = l / 32)
    // reads row 4 h + j / 4 (+ 8 for the second half of its K-values, + 16
    // for the stage's second K-step) at columns 16 (G % 2) + 4 (j % 4) .. + 3
    // of a 32-column block.  Fragment f < 4: X block 4 wn + f; f >= 4: dY
    // block 4 wm + f - 4.
    int fb[8];
    {
        const int G = lane >> 4, j = lane & 15, rsel = 4 * (lane >> 5) + (j >> 2);
        const int lrow = rsel * WG_ROWB + 32 * (G & 1) + 8 * (j & 3);
#pragma unroll
        for (int f = 0; f < 8; ++f) {
            const int cb = f < 4 ? 4 * wn + f : 4 * wm + (f - 4);
            fb[f] = (f < 4 ? WG_OPB : 0) + lrow + ((cb ^ rsel) << 6);
        }
    }
    auto frag_ptr = [&](int k, int ks, int f) { return smem + (k & (WG_NST - 1)) * WG_STB + fb[f] + ks * 8192; };
    auto read_frag = [&](const char* q) {
        const wg_i16x8 v = __builtin_shufflevector(wg_read_tr(q), wg_read_tr(q + 4096), 0, 1, 2, 3, 4, 5, 6, 7);
        return __builtin_bit_cast(wg_bf16x8, v);
    };

    // [X tile][dY tile]; the first K-step's MFMAs take a zero accumulator
    wg_f32x16 acc[4][4];
    wg_f32x16 zero;
#pragma unroll
    for (int r = 0; r < 16; ++r) zero[r] = 0.0f;

    // a: a stage's first K-step; b: its second; c: the next stage's second
    // K-step, read during this stage (b and c swap roles from stage to stage)
    wg_bf16x8 a[8], b[8], c[8];   // X 0..3 | dY 0..3
    auto read_stage = [&](int k, wg_bf16x8 (&f0)[8], wg_bf16x8 (&f1)[8]) {
#pragma unroll
        for (int f = 0; f < 8; ++f) f0[f] = read_frag(frag_ptr(k, 0, f));
#pragma unroll
        for (int f = 0; f < 8; ++f) f1[f] = read_frag(frag_ptr(k, 1, f));
    };
    auto mfma_half = [&](const wg_bf16x8 (&f)[8], auto first) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[j], f[4 + i], first ? zero : acc[j][i], 0, 0, 0);
    };
    constexpr std::true_type FIRST{};
    constexpr std::false_type LATER{};
    // One stage with every later stage present: the second K-step's 16 MFMAs
    // are interleaved one to one with the 8 loads of stage k + 3 and the 16
    // fragment reads of stage k + 1 (first K-step into a, then the second into
    // `next`).  Stage k + 3 goes to the buffer of stage k - 1, whose fragments
    // every wave has consumed before the barrier.
    auto steady = [&](int k, const wg_bf16x8 (&cur)[8], wg_bf16x8 (&next)[8], auto first) {
        mfma_half(a, first);
        __builtin_amdgcn_sched_barrier(0);
        lds_wait_vm<8>();
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        const uint32_t dst = ((k + 3) & (WG_NST - 1)) * WG_STB;
        const int kn = k + 3;
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const int j = t >> 2, i = t & 3;
            acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cur[j], cur[4 + i], acc[j][i], 0, 0, 0);
            if (t < 4)
                lds_dma16(rd, vd[t] + kn * sd, 0, dd + dst + t * 1024);
            else if (t < 8)
                lds_dma16(rx, vx[t - 4] + kn * sx, 0, dx + dst + (t - 4) * 1024);
            if (t < 8)
                a[t] = read_frag(frag_ptr(k + 1, 0, t));
            else
                next[t - 8] = read_frag(frag_ptr(k + 1, 1, t - 8));
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    issue(0);
    if (nk > 1) issue(1);
    if (nk > 2) issue(2);
    if (nk > 2)
        lds_wait_vm<16>();
    else if (nk > 1)
        lds_wait_vm<8>();
    else
        lds_wait_vm<0>();
    __syncthreads();
    read_stage(0, a, b);
    int k = 0;
    if (nk > 4) {
        steady(0, b, c, FIRST);
        steady(1, c, b, LATER);
        k = 2;
    }
    for (; k + 4 < nk; k += 2) {
        steady(k, b, c, LATER);
        steady(k + 1, c, b, LATER);
    }
    if (k + 3 < nk) {
        if (k == 0)
            steady(k, b, c, FIRST);
        else
            steady(k, b, c, LATER);
#pragma unroll
        for (int f = 0; f < 8; ++f) b[f] = c[f];
        ++k;
    }
    // the last (up to) three stages
    for (; k < nk; ++k) {
        if (k == 0)
            mfma_half(a, FIRST);
        else
            mfma_half(a, LATER);
        __builtin_amdgcn_sched_barrier(0);
        if (k + 1 < nk) {
            if (k + 2 < nk)
                lds_wait_vm<8>();
            else
                lds_wait_vm<0>();
            __syncthreads();
            read_stage(k + 1, a, c);
        }
        __builtin_amdgcn_sched_barrier(0);
        mfma_half(b, LATER);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int f = 0; f < 8; ++f) b[f] = c[f];
    }

    // epilogue: lane (l32, hb), register group q of acc[j][i]: dW row
    // o = o0 + 128 wm + 32 i + l32, columns 128 wn + 32 j + 8 q + 4 hb .. + 3
    float* part = p.part + static_cast<int64_t>(s) * p.d_out * p.d_in;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int o = o0 + 128 * wm + 32 * i + l32;
        if (o >= p.d_out) continue;
        float* row = part + static_cast<int64_t>(o) * p.d_in;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int col = i0 + 128 * wn + 32 * j + 8 * q + 4 * hb;
                if (col < p.d_in)
                    *reinterpret_cast<wg_f32x4*>(row + col) =
                        wg_f32x4{acc[j][i][4 * q], acc[j][i][4 * q + 1], acc[j][i][4 * q + 2], acc[j][i][4 * q + 3]};
            }
    }
}

// dW = sum over slices of the partials, in slice order; 8 outputs per thread
template <bool F32>
__global__ __launch_bounds__(256) void wgrad_reduce_kernel(const float* __restrict__ part, void* __restrict__ out,
                                                           int64_t ldw, int slices, int d_out, int d_in) {
    const int per_row = d_in >> 3;
    const int64_t n = static_cast<int64_t>(d_out) * per_row;
    const int64_t plane = static_cast<int64_t>(d_out) * d_in;
    for (int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; g < n;
         g += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int o = static_cast<int>(g / per_row);
        const int col = static_cast<int>(g - static_cast<int64_t>(o) * per_row) << 3;
        const float* src = part + static_cast<int64_t>(o) * d_in + col;
        wg_f32x4 lo = {0.0f, 0.0f, 0.0f, 0.0f}, hi = lo;
        for (int k = 0; k < slices; ++k) {
            lo += *reinterpret_cast<const wg_f32x4*>(src + k * plane);
            hi += *reinterpret_cast<const wg_f32x4*>(src + k * plane + 4);
        }
        if constexpr (F32) {
            float* dst = static_cast<float*>(out) + static_cast<int64_t>(o) * ldw + col;
            *reinterpret_cast<wg_f32x4*>(dst) = lo;
            *reinterpret_cast<wg_f32x4*>(dst + 4) = hi;
        } else {
            auto pack = [](float a, float b) {
                return __builtin_bit_cast(uint32_t, __builtin_convertvector((wg_f32x2{a, b}), wg_bf16x2));
            };
            bf16_t* dst = static_cast<bf16_t*>(out) + static_cast<int64_t>(o) * ldw + col;
            *reinterpret_cast<wg_u32x4*>(dst) = wg_u32x4{pack(lo[0], lo[1]), pack(lo[2], lo[3]), pack(hi[0], hi[1]),
                                                         pack(hi[2], hi[3])};
        }
    }
}

struct WgradPlan {
    int64_t slices, slice, tiles;
};

// slices: the caller's count, or (<= 0) enough to give every CU one
// work-group; then each slice a whole number of stages and no slice empty
WgradPlan wgrad_plan(int64_t tokens, int64_t d_out, int64_t d_in, int64_t splits, int64_t cus) {
    WgradPlan pl{};
    pl.tiles = ((d_out + WG_BT - 1) / WG_BT) * ((d_in + WG_BT - 1) / WG_BT);
    if (tokens <= 0) return pl;
    int64_t s = splits;
    if (s <= 0) {
        s = pl.tiles >= cus ? 1 : cus / pl.tiles;
        const int64_t most = tokens / WG_MIN_SLICE;
        s = s < most ? s : (most > 1 ? most : 1);
    }
    if (s > tokens) s = tokens;
    int64_t slice = (tokens + s - 1) / s;
    slice = (slice + WG_BK - 1) / WG_BK * WG_BK;
    pl.slice = slice;
    pl.slices = (tokens + slice - 1) / slice;
    return pl;
}

int device_cus(int64_t& cus) {
    int n = 0;
    const int rc = device_cu_count(n);
    cus = n;
    return rc;
}

}  // namespace
}  // namespace mogt

using namespace mogt;

extern "C" int64_t mogt_linear_wgrad_splits(int64_t tokens, int64_t d_out, int64_t d_in, int64_t splits, int64_t cus) {
    if (tokens < 0 || d_out <= 0 || d_in <= 0) return -1;
    if (cus <= 0 && splits <= 0 && device_cus(cus) != MOGT_OK) return -1;
    return wgrad_plan(tokens, d_out, d_in, splits, cus > 0 ? cus : 1).slices;
}

extern "C" size_t mogt_linear_wgrad_workspace_bytes(int64_t tokens, int64_t d_out, int64_t d_in, int64_t splits,
                                                    int64_t cus) {
    const int64_t s = mogt_linear_wgrad_splits(tokens, d_out, d_in, splits, cus);
    return s > 0 ? static_cast<size_t>(s) * d_out * d_in * sizeof(float) : 0;
}

extern "C" int mogt_linear_wgrad(const void* dy, const void* x, void* dw, int64_t tokens, int64_t d_out,
                                 int64_t d_in, int64_t ldd, int64_t ldx, int64_t ldw, int64_t splits, int out_dtype,
                                 void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    if (out_dtype != MOGT_BF16 && out_dtype != MOGT_F32)
        return set_error(MOGT_E_INVALID, "linear_wgrad: dW must be bf16 or fp32 (dY and X are bf16)");
    if (tokens < 0 || d_out <= 0 || d_in <= 0) return set_error(MOGT_E_INVALID, "linear_wgrad: bad shape");
    if (d_out % 8 != 0 || d_in % 8 != 0)
        return set_error(MOGT_E_INVALID, "linear_wgrad: d_out and d_in must be multiples of 8");
    if (ldd < d_out || ldx < d_in || ldw < d_in || ldd % 8 != 0 || ldx % 8 != 0 || ldw % 8 != 0)
        return set_error(MOGT_E_INVALID, "linear_wgrad: row strides must cover the rows and be multiples of 8");
    if (!dw || (tokens > 0 && (!dy || !x))) return set_error(MOGT_E_INVALID, "linear_wgrad: null pointer");
    if ((reinterpret_cast<uintptr_t>(dy) | reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(dw)) & 15)
        return set_error(MOGT_E_INVALID, "linear_wgrad: dY, X and dW need 16-byte alignment");
    int64_t cus = 0;
    if (splits <= 0 && tokens > 0) {
        const int rc = device_cus(cus);
        if (rc != MOGT_OK) return rc;
    }
    const WgradPlan pl = wgrad_plan(tokens, d_out, d_in, splits, cus > 0 ? cus : 1);
    const int64_t ld = ldd > ldx ? ldd : ldx;
    // per-slice byte offsets (the last stage may reach one stage past the
    // slice) and descriptor ranges are 32-bit
    if (tokens > 0 && (pl.slice + WG_BK) * ld * 2 >= (int64_t(1) << 31))
        return set_error(MOGT_E_INVALID, "linear_wgrad: slices of %lld tokens x row stride %lld exceed 2 GiB; "
                                         "pass more splits", static_cast<long long>(pl.slice),
                         static_cast<long long>(ld));
    const int64_t n_wg = pl.tiles * pl.slices;
    if (n_wg > 0x7fffffff) return set_error(MOGT_E_INVALID, "linear_wgrad: too many tiles");
    const size_t need = static_cast<size_t>(pl.slices) * d_out * d_in * sizeof(float);
    if (need > 0 && (!workspace || workspace_bytes < need))
        return set_error(MOGT_E_WORKSPACE, "linear_wgrad: workspace of %zu bytes needed, %zu given", need,
                         workspace_bytes);
    if (need > 0 && (reinterpret_cast<uintptr_t>(workspace) & 15))
        return set_error(MOGT_E_INVALID, "linear_wgrad: workspace needs 16-byte alignment");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (pl.slices > 0) {
        WgradParams prm{};
        prm.dy = static_cast<const bf16_t*>(dy);
        prm.x = static_cast<const bf16_t*>(x);
        prm.part = static_cast<float*>(workspace);
        prm.T = tokens;
        prm.ldd = ldd;
        prm.ldx = ldx;
        prm.d_out = static_cast<int>(d_out);
        prm.d_in = static_cast<int>(d_in);
        prm.n_ot = static_cast<int>((d_out + WG_BT - 1) / WG_BT);
        prm.n_it = static_cast<int>((d_in + WG_BT - 1) / WG_BT);
        prm.slices = static_cast<int>(pl.slices);
        prm.slice = static_cast<int>(pl.slice);
        hipLaunchKernelGGL(wgrad_gemm_kernel, dim3(static_cast<unsigned>(n_wg)), dim3(WG_THREADS), 0, st, prm);
        const int rc = check_launch("wgrad_gemm_kernel");
        if (rc != MOGT_OK) return rc;
    }
    // no tokens: the reduction over zero slices writes zeros
    const int64_t groups = d_out * (d_in / 8);
    const int64_t blocks = (groups + 255) / 256 < 4096 ? (groups + 255) / 256 : 4096;
    if (out_dtype == MOGT_F32)
        hipLaunchKernelGGL(wgrad_reduce_kernel<true>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st,
                           static_cast<const float*>(workspace), dw, ldw, static_cast<int>(pl.slices),
                           static_cast<int>(d_out), static_cast<int>(d_in));
    else
        hipLaunchKernelGGL(wgrad_reduce_kernel<false>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st,
                           static_cast<const float*>(workspace), dw, ldw, static_cast<int>(pl.slices),
                           static_cast<int>(d_out), static_cast<int>(d_in));
    return check_launch("wgrad_reduce_kernel");
}
