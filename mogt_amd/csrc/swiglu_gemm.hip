// The SwiGLU gate of the feed-forward block as one bf16 GEMM with the gate in
// its epilogue (SwiGLU.forward, model_mogt.py:29-30, first half):
//   y[m][n] = silu(x[m] . w_gate[n]) * (x[m] . w_up[n])
// x [rows, K] (row stride ldx), w_gate / w_up [H, K] (nn.Linear weights), y
// [rows, H] (row stride ldy), all bf16; fp32 accumulation.  The [rows, 2H]
// pre-activations are never written.  The epilogue rounds like the unfused
// path it replaces: each linear output to bf16, silu of it to bf16, then the
// product to bf16.
//
// Tiling (v_mfma_f32_32x32x16_bf16, 4 waves, one work-group per CU):
//   work-group  256 rows of x  x  128 outputs (128 w_gate rows + the same 128
//               w_up rows)
//   wave        128 rows of x x 64 outputs: 4 x 4 accumulator tiles of
//               D[w][x] (weight row, x row) -- tiles 0, 1 gate, 2, 3 up, so a
//               gate value and its up value sit in the same lane and register
// With weight rows as the MFMA's A operand, a lane's 16 results are 4 groups
// of 4 consecutive outputs of one x row: the gate is applied in registers and
// each group leaves as one 8-byte store, no LDS round trip.
//
// Operands reach LDS by direct buffer-to-LDS loads (no staging registers) in
// stages of 32 along K, four stages in flight (128 KB): stage s is multiplied
// while stages s + 1 .. s + 3 load.  A stage holds 256 rows of x then 256 rows
// of weights, 64 B per row; the 16-byte chunk c of row r sits at chunk
// c ^ ((r / 2 ^ r / 4) % 4), so an MFMA operand read (consecutive rows, one
// chunk) is free of bank conflicts whether the LDS serves 8 lanes x 16 B or
// 16 lanes x 16 B per cycle.  One wave load instruction fills 1 KB of
// LDS (16 rows) in lane order, so the swizzle is applied to the global
// addresses.  These loads are issued from inline assembly and their
// completion is awaited with explicit vmcnt waits: the compiler's own waits
// for LDS-bound loads drain all of them before any LDS read.  Rows of x past
// `rows` are loaded as the last valid row (their outputs are dropped by the
// store descriptor's range).
//
// Work-group order is XCD-aware: the hardware deals work-groups round-robin
// over the 8 XCDs, so block b is renumbered to give each XCD a contiguous run
// of tiles, walked 8 row blocks at a time, so that one XCD's L2 keeps the x
// rows of those 8 blocks while it sweeps the weight blocks.
//
// Two schedules of the same tiles: one tile per work-group
// (swiglu_gemm_kernel), and a persistent one (swiglu_gemm_persistent_kernel,
// the default where K allows it) in which each CU's work-group streams its
// tiles' stages back to back and runs a tile's epilogue inside the next tile's
// main loop.  Both give bit-identical outputs.
#include <type_traits>
#include <vector>

#include "lds_dma.h"

namespace mogt {
namespace {

typedef __bf16 sg_bf16x8 __attribute__((ext_vector_type(8)));
typedef float sg_f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t sg_u32x2 __attribute__((ext_vector_type(2)));
typedef float sg_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 sg_bf16x2 __attribute__((ext_vector_type(2)));

constexpr int SG_BM = 256;                   // x rows per work-group
constexpr int SG_BN = 128;                   // outputs per work-group
constexpr int SG_BK = 32;                    // contraction per stage
constexpr int SG_NST = 4;                    // stages in LDS
constexpr int SG_THREADS = 256;              // 4 waves
constexpr int SG_ROWB = SG_BK * 2;           // bytes per LDS row
constexpr int SG_OPB = 256 * SG_ROWB;        // one operand of a stage (16 KB)
constexpr int SG_STB = 2 * SG_OPB;           // one stage (32 KB)
constexpr int SG_GROUP_M = 8;                // row blocks walked together per XCD

struct SwigluParams {
    const bf16_t* x;
    const bf16_t* wg;
    const bf16_t* wu;
    bf16_t* y;
    int64_t rows;
    int64_t ldx, ldy;    // elements
    int K, H;
    int n_mb, n_nb;      // row blocks, output blocks
};

__device__ __forceinline__ float sg_silu(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

// two fp32 values as one word of two bf16 (round to nearest even)
__device__ __forceinline__ uint32_t sg_pack(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((sg_f32x2{lo, hi}), sg_bf16x2));
}

// lo and hi rounded to bf16 (nearest even) with one conversion, back as fp32
__device__ __forceinline__ void sg_round2(float lo, float hi, float& rlo, float& rhi) {
    const uint32_t w = sg_pack(lo, hi);
    rlo = __uint_as_float(w << 16);
    rhi = __uint_as_float(w & 0xffff0000u);
}

// Tiles of work-group `bid` of `grid`: its XCD (ids = xcd mod 8; with fewer
// than 8 work-groups, each is its own group) owns a contiguous run of the n
// tiles, dealt to that XCD's work-groups in turn; the work-group takes tiles
// base, base + step, ... (count of them).  One tile per work-group (grid = n)
// and the persistent schedule (grid = min(n, CUs)) both use it, as does the
// host self-check (mogt_swiglu_check_schedule).
struct SgpWalk {
    int base, step, count;
};

__host__ __device__ inline SgpWalk sgp_walk(int n, int grid, int bid) {
    const int nx = grid < 8 ? grid : 8;
    const int xcd = bid % nx, loc = bid / nx;
    const int nloc = (grid - xcd + nx - 1) / nx;
    const int q = n / nx, rem = n - q * nx;
    const int first = xcd < rem ? xcd * (q + 1) : rem * (q + 1) + (xcd - rem) * q;
    const int xcount = q + (xcd < rem ? 1 : 0);
    return SgpWalk{first + loc, nloc, loc < xcount ? (xcount - loc + nloc - 1) / nloc : 0};
}

// tile index -> (row block, output block), 8 row blocks walked together
__host__ __device__ inline void sgp_block(int n_mb, int n_nb, int v, int& mb, int& nb) {
    const int group = SG_GROUP_M * n_nb;
    const int g = v / group, first = g * SG_GROUP_M;
    const int gm = (n_mb - first) < SG_GROUP_M ? (n_mb - first) : SG_GROUP_M;
    const int w = v - g * group;
    mb = first + w % gm;
    nb = w / gm;
}

// block id -> (row block, output block), one tile per work-group
__device__ __forceinline__ void sg_tile(const SwigluParams& p, int& mb, int& nb) {
    const int n = p.n_mb * p.n_nb;
    sgp_block(p.n_mb, p.n_nb, sgp_walk(n, n, static_cast<int>(blockIdx.x)).base, mb, nb);
}

__global__ __launch_bounds__(SG_THREADS) void swiglu_gemm_kernel(SwigluParams p) {
    __shared__ __attribute__((aligned(1024))) char smem[SG_NST * SG_STB];   // [stage][x | w][256][64 B]
    int mb, nb;
    sg_tile(p, mb, nb);
    const int64_t m0 = static_cast<int64_t>(mb) * SG_BM;
    const int n0 = nb * SG_BN;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int l32 = lane & 31, hb = lane >> 5;
    const uint32_t lds0 = lds_addr(smem);

    // loads: wave w fills rows 64 w .. 64 w + 63 of each operand, 16 rows
    // (1 KB) per instruction; lane L takes row 16 i + L / 4 of its block and
    // the global chunk that lands in LDS slot L % 4 under the swizzle
    const int64_t mrows = p.rows - m0 < SG_BM ? p.rows - m0 : SG_BM;
    const lds_i32x4 rx = lds_rsrc(p.x + m0 * p.ldx, static_cast<uint32_t>(mrows * p.ldx * 2));
    const lds_i32x4 rw = lds_rsrc((wave < 2 ? p.wg : p.wu) + static_cast<int64_t>(n0) * p.K,
                                static_cast<uint32_t>(SG_BN * p.K * 2));
    const int lc = (lane & 3) ^ (((lane >> 3) ^ (lane >> 4)) & 3);
    int vx[4], vw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = 64 * wave + 16 * i + (lane >> 2);
        const int rc = r < mrows ? r : static_cast<int>(mrows) - 1;
        vx[i] = static_cast<int>(rc * p.ldx * 2) + lc * 16;
        vw[i] = ((r & 127) * p.K) * 2 + lc * 16;
    }
    const uint32_t ldx_dst = lds0 + wave * 4096, ldw_dst = lds0 + SG_OPB + wave * 4096;
    const int nk = p.K / SG_BK;
    auto issue = [&](int s) {
        const uint32_t st = (s & (SG_NST - 1)) * SG_STB;
        const int kb = s * SG_ROWB;
#pragma unroll
        for (int i = 0; i < 4; ++i) lds_dma16(rx, vx[i], kb, ldx_dst + st + i * 1024);
#pragma unroll
        for (int i = 0; i < 4; ++i) lds_dma16(rw, vw[i], kb, ldw_dst + st + i * 1024);
    };

    // fragment rows: x rows wm*128 + 32 i + l32; weight rows (gate) 64 wn + 32 j
    // + l32, (up) 128 + 64 wn + 32 j + l32; every one has row % 16 == l32 % 16
    const int xrow0 = (wm * 128 + l32) * SG_ROWB;
    const int wrow0 = SG_OPB + (wn * 64 + l32) * SG_ROWB;
    const int swz = ((l32 >> 1) ^ (l32 >> 2)) & 3;

    // [weight tile][x tile]; the first K-step's MFMAs take a zero accumulator
    // operand instead of 256 register clears
    sg_f32x16 acc[4][4];
    sg_f32x16 zero;
#pragma unroll
    for (int r = 0; r < 16; ++r) zero[r] = 0.0f;

    // Fragments of a whole stage (2 K-steps: 4 x and 4 weight fragments each)
    // are read into registers one stage ahead, so the MFMAs never wait on LDS.
    // Stage s + 1 is awaited (this wave's loads, then the barrier for every
    // wave's) between the two K-steps of stage s, its fragments read, and the
    // loads of stage s + 3 issued into the buffer of stage s - 1, whose
    // fragments every wave has consumed before that barrier.
    // a: the stage's first K-step; b: its second; c: the next stage's second
    // K-step, read during this stage.  b and c swap roles from stage to stage
    // (the loop is unrolled by two), so no fragment is ever copied.
    sg_bf16x8 a[8], b[8], c[8];   // x 0..3 | w 0..3
    auto frag_ptr = [&](const char* st, int ks, int f) {
        const int cb = ((2 * ks + hb) ^ swz) << 4;
        const int row = f < 4 ? xrow0 + f * 32 * SG_ROWB : wrow0 + (((f - 4) >> 1) * 128 + ((f - 4) & 1) * 32) * SG_ROWB;
        return reinterpret_cast<const sg_bf16x8*>(st + row + cb);
    };
    auto read_stage = [&](int s, sg_bf16x8 (&f0)[8], sg_bf16x8 (&f1)[8]) {
        const char* st = smem + (s & (SG_NST - 1)) * SG_STB;
#pragma unroll
        for (int f = 0; f < 8; ++f) f0[f] = *frag_ptr(st, 0, f);
#pragma unroll
        for (int f = 0; f < 8; ++f) f1[f] = *frag_ptr(st, 1, f);
    };
    auto mfma_half = [&](const sg_bf16x8 (&f)[8], auto first) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[4 + j], f[i], first ? zero : acc[j][i], 0, 0,
                                                                    0);
    };
    constexpr std::true_type FIRST{};
    constexpr std::false_type LATER{};
    // One stage with every later stage present: the second K-step's 16 MFMAs
    // (fragments `cur`) are interleaved one to one with the 8 loads of stage
    // s + 3 and the 16 fragment reads of stage s + 1 (first K-step into a,
    // free since the first half, then the second K-step into `next`).
    auto steady = [&](int s, const sg_bf16x8 (&cur)[8], sg_bf16x8 (&next)[8], auto first) {
        mfma_half(a, first);
        __builtin_amdgcn_sched_barrier(0);
        lds_wait_vm<8>();
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        const uint32_t dst = ((s + 3) & (SG_NST - 1)) * SG_STB;
        const int kb = (s + 3) * SG_ROWB;
        const char* stn = smem + ((s + 1) & (SG_NST - 1)) * SG_STB;
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const int j = t >> 2, i = t & 3;
            acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cur[4 + j], cur[i], acc[j][i], 0, 0, 0);
            if (t < 4)
                lds_dma16(rx, vx[t], kb, ldx_dst + dst + t * 1024);
            else if (t < 8)
                lds_dma16(rw, vw[t - 4], kb, ldw_dst + dst + (t - 4) * 1024);
            if (t < 8)
                a[t] = *frag_ptr(stn, 0, t);
            else
                next[t - 8] = *frag_ptr(stn, 1, t - 8);
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
    int s = 0;
    if (nk > 4) {   // stage 0's first K-step starts the accumulators
        steady(0, b, c, FIRST);
        steady(1, c, b, LATER);
        s = 2;
    }
    for (; s + 4 < nk; s += 2) {
        steady(s, b, c, LATER);
        steady(s + 1, c, b, LATER);
    }
    if (s + 3 < nk) {
        if (s == 0)
            steady(s, b, c, FIRST);
        else
            steady(s, b, c, LATER);
#pragma unroll
        for (int f = 0; f < 8; ++f) b[f] = c[f];
        ++s;
    }
    // the last (up to) three stages
    for (; s < nk; ++s) {
        if (s == 0)
            mfma_half(a, FIRST);
        else
            mfma_half(a, LATER);
        __builtin_amdgcn_sched_barrier(0);
        if (s + 1 < nk) {
            if (s + 2 < nk)
                lds_wait_vm<8>();
            else
                lds_wait_vm<0>();
            __syncthreads();
            read_stage(s + 1, a, c);
        }
        __builtin_amdgcn_sched_barrier(0);
        mfma_half(b, LATER);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int f = 0; f < 8; ++f) b[f] = c[f];
    }

    // epilogue: lane (l32, hb), register group q: x row 32 i + l32, outputs
    // 32 j + 8 q + 4 hb .. + 3 of the wave's 64
    const auto ry = __builtin_amdgcn_make_buffer_rsrc(p.y + m0 * p.ldy, 0, static_cast<int>(mrows * p.ldy * 2),
                                                      0x00020000);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row_off = static_cast<int>((wm * 128 + 32 * i + l32) * p.ldy * 2);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                // roundings to bf16 two values per conversion
                float g[4], u[4], sg[4], o[4];
#pragma unroll
                for (int e = 0; e < 4; e += 2) {
                    sg_round2(acc[j][i][4 * q + e], acc[j][i][4 * q + e + 1], g[e], g[e + 1]);
                    sg_round2(acc[j + 2][i][4 * q + e], acc[j + 2][i][4 * q + e + 1], u[e], u[e + 1]);
                    sg_round2(sg_silu(g[e]), sg_silu(g[e + 1]), sg[e], sg[e + 1]);
                    o[e] = sg[e] * u[e];
                    o[e + 1] = sg[e + 1] * u[e + 1];
                }
                const sg_u32x2 w = {sg_pack(o[0], o[1]), sg_pack(o[2], o[3])};
                const int col = n0 + wn * 64 + 32 * j + 8 * q + 4 * hb;
                __builtin_amdgcn_raw_buffer_store_b64(w, ry, row_off + col * 2, 0, 0);
            }
        }
    }
}


// ---------------------------------------------------------------------------
// Persistent schedule (default when K % 128 == 0 and K >= 640, i.e. a multiple
// of four stages and at least 20 of them): one work-group per CU walks its
// XCD's tiles in turn as one continuous stream of stages, so a tile's last
// three stages load the next tile's first three (no prologue wait, no pipeline
// drain), and tile k's epilogue runs inside tile k + 1's main loop:
//   stage 0      each accumulator tile is rounded to bf16 pairs (`pend`, 128
//                registers: the gate and up values of 32 groups of 4 outputs)
//                right before the first K-step's MFMA restarts it;
//   stages 1-16  two groups per stage: gate math in the first K-step, the two
//                8-byte stores after the stage's loads in the second;
//   last tile    its epilogue after the loop, as in the kernel above.
// Stores never let a load wait pass early: every wait counts only the loads
// issued after the stage it waits for, and loads complete in order, so a wait
// that passes has that stage's loads done whatever the stores issued after them
// are doing (it may wait longer for those stores).  The last tile loads its own
// first stages again (in bounds, never read) so every stage has the same waits;
// the kernel ends by waiting for them.  Same roundings in the same order as the
// kernel above: the outputs are bit-identical.
constexpr int SGP_MIN_STAGES = 20;   // stage 0 + 16 epilogue stages + 3 prefetch stages

struct SgpTile {
    int64_t m0;
    int n0;
    int mrows;
};


__device__ __forceinline__ void sgp_tile(const SwigluParams& p, int v, SgpTile& t) {
    int mb, nb;
    sgp_block(p.n_mb, p.n_nb, v, mb, nb);
    t.m0 = static_cast<int64_t>(mb) * SG_BM;
    t.n0 = nb * SG_BN;
    const int64_t mr = p.rows - t.m0;
    t.mrows = static_cast<int>(mr < SG_BM ? mr : SG_BM);
}

__global__ __launch_bounds__(SG_THREADS) void swiglu_gemm_persistent_kernel(SwigluParams p) {
    __shared__ __attribute__((aligned(1024))) char smem[SG_NST * SG_STB];   // [stage][x | w][256][64 B]
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int l32 = lane & 31, hb = lane >> 5;
    const uint32_t lds0 = lds_addr(smem);

    // tiles of this work-group: its XCD's contiguous run (ids = xcd mod 8), dealt
    // to the XCD's work-groups in turn
    const SgpWalk walk = sgp_walk(p.n_mb * p.n_nb, static_cast<int>(gridDim.x), static_cast<int>(blockIdx.x));
    const int ntile = walk.count;
    if (ntile == 0) return;

    const int nk = p.K / SG_BK;
    const int lc = (lane & 3) ^ (((lane >> 3) ^ (lane >> 4)) & 3);
    int vw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) vw[i] = (((64 * wave + 16 * i + (lane >> 2)) & 127) * p.K) * 2 + lc * 16;
    const uint32_t ldx_dst = lds0 + wave * 4096, ldw_dst = lds0 + SG_OPB + wave * 4096;

    // a tile's load state: descriptors and x row offsets (rows past `rows`
    // load the last valid row, as in the kernel above)
    struct Ld {
        lds_i32x4 rx, rw;
        int vx[4];
    };
    auto make_ld = [&](const SgpTile& t, Ld& L) {
        L.rx = lds_rsrc(p.x + t.m0 * p.ldx, static_cast<uint32_t>(static_cast<int64_t>(t.mrows) * p.ldx * 2));
        L.rw = lds_rsrc((wave < 2 ? p.wg : p.wu) + static_cast<int64_t>(t.n0) * p.K,
                        static_cast<uint32_t>(SG_BN * p.K * 2));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 64 * wave + 16 * i + (lane >> 2);
            L.vx[i] = static_cast<int>((r < t.mrows ? r : t.mrows - 1) * p.ldx * 2) + lc * 16;
        }
    };
    // the 8 loads of stage `sl` of a tile into LDS buffer `buf`
    auto issue = [&](const Ld& L, int sl, int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) lds_dma16(L.rx, L.vx[i], sl * SG_ROWB, ldx_dst + buf * SG_STB + i * 1024);
#pragma unroll
        for (int i = 0; i < 4; ++i) lds_dma16(L.rw, vw[i], sl * SG_ROWB, ldw_dst + buf * SG_STB + i * 1024);
    };

    const int xrow0 = (wm * 128 + l32) * SG_ROWB;
    const int wrow0 = SG_OPB + (wn * 64 + l32) * SG_ROWB;
    const int swz = ((l32 >> 1) ^ (l32 >> 2)) & 3;
    auto frag_ptr = [&](const char* st, int ks, int f) {
        const int cb = ((2 * ks + hb) ^ swz) << 4;
        const int row = f < 4 ? xrow0 + f * 32 * SG_ROWB : wrow0 + (((f - 4) >> 1) * 128 + ((f - 4) & 1) * 32) * SG_ROWB;
        return reinterpret_cast<const sg_bf16x8*>(st + row + cb);
    };

    sg_f32x16 acc[4][4];
    sg_f32x16 zero;
#pragma unroll
    for (int r = 0; r < 16; ++r) zero[r] = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[j][i] = zero;
    // the previous tile's linear outputs in bf16, two per word; group
    // gi = 8 i + 4 j + q (x tile i, gate tile j, register group q):
    // {gate 0,1 | gate 2,3 | up 0,1 | up 2,3}
    uint32_t pend[32][4];
#pragma unroll
    for (int gi = 0; gi < 32; ++gi)
#pragma unroll
        for (int e = 0; e < 4; ++e) pend[gi][e] = 0u;

    // where the previous tile's outputs go (nowhere before the first tile)
    int64_t ym0 = 0;
    int ybytes = 0, yn0 = 0;
    const int yrow = (wm * 128 + l32) * static_cast<int>(p.ldy) * 2;

    // a, b, c: fragments as in the kernel above (b and c swap roles stage by stage)
    sg_bf16x8 a[8], b[8], c[8];
    sg_u32x2 ow[2];
    int oo[2];
    // one group of the previous tile: 4 outputs, kept for one 8-byte store
    auto epi_group = [&](auto gtag, int slot) {
        constexpr int gi = decltype(gtag)::value;
        constexpr int i = gi >> 3, j = (gi >> 2) & 1, q = gi & 3;
        float g[4], u[4], sg[4], o[4];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            g[2 * e] = __uint_as_float(pend[gi][e] << 16);
            g[2 * e + 1] = __uint_as_float(pend[gi][e] & 0xffff0000u);
            u[2 * e] = __uint_as_float(pend[gi][2 + e] << 16);
            u[2 * e + 1] = __uint_as_float(pend[gi][2 + e] & 0xffff0000u);
        }
        sg_round2(sg_silu(g[0]), sg_silu(g[1]), sg[0], sg[1]);
        sg_round2(sg_silu(g[2]), sg_silu(g[3]), sg[2], sg[3]);
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = sg[e] * u[e];
        ow[slot] = sg_u32x2{sg_pack(o[0], o[1]), sg_pack(o[2], o[3])};
        oo[slot] = yrow + i * 64 * static_cast<int>(p.ldy) + (yn0 + wn * 64 + 32 * j + 8 * q + 4 * hb) * 2;
    };
    // first K-step of a stage, with epilogue groups E0 and E0 + 1 when E0 >= 0
    auto half_a = [&](auto etag) {
        constexpr int E0 = decltype(etag)::value;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[4 + j], a[i], acc[j][i], 0, 0, 0);
        if constexpr (E0 >= 0) {
            epi_group(std::integral_constant<int, E0>{}, 0);
            epi_group(std::integral_constant<int, E0 + 1>{}, 1);
        }
    };
    // first K-step of a tile's stage 0: each accumulator tile becomes `pend`
    // just before the MFMA that starts it again from zero
    auto half_a_first = [&]() {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int gi = 8 * i + 4 * (j & 1) + q, e0 = j < 2 ? 0 : 2;
                    pend[gi][e0] = sg_pack(acc[j][i][4 * q], acc[j][i][4 * q + 1]);
                    pend[gi][e0 + 1] = sg_pack(acc[j][i][4 * q + 2], acc[j][i][4 * q + 3]);
                }
                acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[4 + j], a[i], zero, 0, 0, 0);
            }
    };
    // second K-step of a stage: wait for the next stage (buffer `bufn`), then
    // 16 MFMAs interleaved with the 8 loads of stage `sl` of load state L into
    // buffer `bufl`, the next stage's fragment reads and, with `st`, the first
    // half's two stores
    auto half_b = [&](int bufn, const Ld& L, int sl, int bufl, const sg_bf16x8 (&cur)[8], sg_bf16x8 (&next)[8],
                      auto st, __amdgpu_buffer_rsrc_t ry) {
        __builtin_amdgcn_sched_barrier(0);
        lds_wait_vm<8>();
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        const char* stn = smem + bufn * SG_STB;
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const int j = t >> 2, i = t & 3;
            acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cur[4 + j], cur[i], acc[j][i], 0, 0, 0);
            if (t < 4)
                lds_dma16(L.rx, L.vx[t], sl * SG_ROWB, ldx_dst + bufl * SG_STB + t * 1024);
            else if (t < 8)
                lds_dma16(L.rw, vw[t - 4], sl * SG_ROWB, ldw_dst + bufl * SG_STB + (t - 4) * 1024);
            if (t < 8)
                a[t] = *frag_ptr(stn, 0, t);
            else
                next[t - 8] = *frag_ptr(stn, 1, t - 8);
            if constexpr (decltype(st)::value) {
                if (t == 8 || t == 9) __builtin_amdgcn_raw_buffer_store_b64(ow[t - 8], ry, oo[t - 8], 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    SgpTile tc, tn;
    Ld lcur, lnext;
    sgp_tile(p, walk.base, tc);
    make_ld(tc, lcur);
    issue(lcur, 0, 0);
    issue(lcur, 1, 1);
    issue(lcur, 2, 2);
    lds_wait_vm<16>();
    __syncthreads();
    {
        const char* st = smem;
#pragma unroll
        for (int f = 0; f < 8; ++f) a[f] = *frag_ptr(st, 0, f);
#pragma unroll
        for (int f = 0; f < 8; ++f) b[f] = *frag_ptr(st, 1, f);
    }

    constexpr std::integral_constant<int, -1> NOEPI{};
    constexpr std::true_type ST{};
    constexpr std::false_type NOST{};
    // nk % 4 == 0: a tile's stage s sits in LDS buffer s % 4
    for (int k = 0; k < ntile; ++k) {
        const auto ry = __builtin_amdgcn_make_buffer_rsrc(p.y + ym0 * p.ldy, 0, ybytes, 0x00020000);
        half_a_first();
        half_b(1, lcur, 3, 3, b, c, NOST, ry);
#define SGP_PAIR(S)                                                              \
        half_a(std::integral_constant<int, 2 * ((S) - 1)>{});                  \
        half_b(((S) + 1) & 3, lcur, (S) + 3, ((S) + 3) & 3, c, b, ST, ry);     \
        half_a(std::integral_constant<int, 2 * (S)>{});                        \
        half_b(((S) + 2) & 3, lcur, (S) + 4, ((S) + 4) & 3, b, c, ST, ry);
        SGP_PAIR(1) SGP_PAIR(3) SGP_PAIR(5) SGP_PAIR(7) SGP_PAIR(9) SGP_PAIR(11) SGP_PAIR(13) SGP_PAIR(15)
#undef SGP_PAIR
        for (int s = 17; s + 1 <= nk - 4; s += 2) {
            half_a(NOEPI);
            half_b((s + 1) & 3, lcur, s + 3, (s + 3) & 3, c, b, NOST, ry);
            half_a(NOEPI);
            half_b((s + 2) & 3, lcur, s + 4, (s + 4) & 3, b, c, NOST, ry);
        }
        // the last three stages load the next tile's first three
        sgp_tile(p, walk.base + (k + 1 < ntile ? k + 1 : k) * walk.step, tn);
        make_ld(tn, lnext);
        half_a(NOEPI);
        half_b((nk - 2) & 3, lnext, 0, 0, c, b, NOST, ry);
        half_a(NOEPI);
        half_b((nk - 1) & 3, lnext, 1, 1, b, c, NOST, ry);
        half_a(NOEPI);
        half_b(0, lnext, 2, 2, c, b, NOST, ry);

        ym0 = tc.m0;
        ybytes = static_cast<int>(static_cast<int64_t>(tc.mrows) * p.ldy * 2);
        yn0 = tc.n0;
        tc = tn;
        lcur = lnext;
    }

    // the last tile's epilogue
    const auto ry = __builtin_amdgcn_make_buffer_rsrc(p.y + ym0 * p.ldy, 0, ybytes, 0x00020000);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float g[4], u[4], sg[4], o[4];
#pragma unroll
                for (int e = 0; e < 4; e += 2) {
                    sg_round2(acc[j][i][4 * q + e], acc[j][i][4 * q + e + 1], g[e], g[e + 1]);
                    sg_round2(acc[j + 2][i][4 * q + e], acc[j + 2][i][4 * q + e + 1], u[e], u[e + 1]);
                    sg_round2(sg_silu(g[e]), sg_silu(g[e + 1]), sg[e], sg[e + 1]);
                    o[e] = sg[e] * u[e];
                    o[e + 1] = sg[e + 1] * u[e + 1];
                }
                const sg_u32x2 w = {sg_pack(o[0], o[1]), sg_pack(o[2], o[3])};
                const int col = yn0 + wn * 64 + 32 * j + 8 * q + 4 * hb;
                __builtin_amdgcn_raw_buffer_store_b64(w, ry, yrow + i * 64 * static_cast<int>(p.ldy) + col * 2, 0, 0);
            }
        }
    }
    lds_wait_vm<0>();   // the last tile's unused loads
}

}  // namespace
}  // namespace mogt

using namespace mogt;

namespace {

// path: 0 = by shape (persistent when d_in qualifies), 1 = one tile per
// work-group, 2 = persistent
int swiglu_launch(const void* x, const void* w_gate, const void* w_up, void* y, int64_t rows, int64_t d_in,
                  int64_t hidden, int64_t ldx, int64_t ldy, int dtype, int path, void* stream) {
    clear_error();
    if (path < 0 || path > 2) return set_error(MOGT_E_INVALID, "swiglu_gate: path must be 0, 1 or 2");
    if (dtype != MOGT_BF16) return set_error(MOGT_E_INVALID, "swiglu_gate: bf16 operands only");
    if (rows < 0 || d_in <= 0 || hidden <= 0) return set_error(MOGT_E_INVALID, "swiglu_gate: bad shape");
    if (d_in % SG_BK != 0 || hidden % SG_BN != 0)
        return set_error(MOGT_E_INVALID, "swiglu_gate: d_in must be a multiple of %d and hidden of %d", SG_BK, SG_BN);
    if (ldx < d_in || ldy < hidden || ldx % 8 != 0 || ldy % 4 != 0)
        return set_error(MOGT_E_INVALID, "swiglu_gate: row strides must cover the rows (ldx %% 8 == 0, ldy %% 4 == 0)");
    if (rows == 0) return MOGT_OK;
    if (!x || !w_gate || !w_up || !y) return set_error(MOGT_E_INVALID, "swiglu_gate: null pointer");
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w_gate) | reinterpret_cast<uintptr_t>(w_up)) & 15 ||
        reinterpret_cast<uintptr_t>(y) & 7)
        return set_error(MOGT_E_INVALID, "swiglu_gate: x and weights need 16-byte, y 8-byte alignment");
    // per-block byte ranges and offsets are 32-bit
    if (static_cast<int64_t>(SG_BM) * (ldx > ldy ? ldx : ldy) * 2 >= (int64_t(1) << 31) ||
        static_cast<int64_t>(SG_BN) * d_in * 2 >= (int64_t(1) << 31))
        return set_error(MOGT_E_INVALID, "swiglu_gate: row strides too large");
    const int64_t n_mb = (rows + SG_BM - 1) / SG_BM;
    const int64_t n_nb = hidden / SG_BN;
    if (n_mb * n_nb > 0x7fffffff) return set_error(MOGT_E_INVALID, "swiglu_gate: too many tiles");
    SwigluParams prm{};
    prm.x = static_cast<const bf16_t*>(x);
    prm.wg = static_cast<const bf16_t*>(w_gate);
    prm.wu = static_cast<const bf16_t*>(w_up);
    prm.y = static_cast<bf16_t*>(y);
    prm.rows = rows;
    prm.ldx = ldx;
    prm.ldy = ldy;
    prm.K = static_cast<int>(d_in);
    prm.H = static_cast<int>(hidden);
    prm.n_mb = static_cast<int>(n_mb);
    prm.n_nb = static_cast<int>(n_nb);
    const bool fits = d_in % (SG_NST * SG_BK) == 0 && d_in / SG_BK >= SGP_MIN_STAGES;
    if (path == 2 && !fits)
        return set_error(MOGT_E_INVALID, "swiglu_gate: the persistent schedule needs d_in %% %d == 0 and d_in >= %d",
                         SG_NST * SG_BK, SGP_MIN_STAGES * SG_BK);
    if (path == 1 || !fits) {
        hipLaunchKernelGGL(swiglu_gemm_kernel, dim3(static_cast<unsigned>(n_mb * n_nb)), dim3(SG_THREADS), 0,
                           static_cast<hipStream_t>(stream), prm);
        return check_launch("swiglu_gemm_kernel");
    }
    int cus = 0;
    const int rc = device_cu_count(cus);
    if (rc != MOGT_OK) return rc;
    const int64_t grid = n_mb * n_nb < cus ? n_mb * n_nb : cus;   // one work-group per CU (128 KB of LDS)
    hipLaunchKernelGGL(swiglu_gemm_persistent_kernel, dim3(static_cast<unsigned>(grid)), dim3(SG_THREADS), 0,
                       static_cast<hipStream_t>(stream), prm);
    return check_launch("swiglu_gemm_persistent_kernel");
}

}  // namespace

extern "C" int mogt_swiglu_gate_fwd(const void* x, const void* w_gate, const void* w_up, void* y, int64_t rows,
                                    int64_t d_in, int64_t hidden, int64_t ldx, int64_t ldy, int dtype,
                                    void* stream) {
    return swiglu_launch(x, w_gate, w_up, y, rows, d_in, hidden, ldx, ldy, dtype, 0, stream);
}

extern "C" int mogt_swiglu_gate_fwd_cfg(const void* x, const void* w_gate, const void* w_up, void* y, int64_t rows,
                                        int64_t d_in, int64_t hidden, int64_t ldx, int64_t ldy, int dtype, int path,
                                        void* stream) {
    return swiglu_launch(x, w_gate, w_up, y, rows, d_in, hidden, ldx, ldy, dtype, path, stream);
}

extern "C" int mogt_swiglu_check_schedule(int64_t rows, int64_t hidden, int grid) {
    clear_error();
    if (rows <= 0 || hidden <= 0 || hidden % SG_BN != 0 || grid <= 0)
        return set_error(MOGT_E_INVALID, "swiglu_check_schedule: bad shape or grid");
    const int64_t n_mb64 = (rows + SG_BM - 1) / SG_BM, n_nb64 = hidden / SG_BN;
    if (n_mb64 * n_nb64 > (int64_t(1) << 24))
        return set_error(MOGT_E_INVALID, "swiglu_check_schedule: too many tiles");
    const int n_mb = static_cast<int>(n_mb64), n_nb = static_cast<int>(n_nb64), n = n_mb * n_nb;
    // the persistent grid, then one tile per work-group
    for (const int g : {grid, n}) {
        std::vector<int> seen_v(n, 0), seen_b(n, 0);
        for (int bid = 0; bid < g; ++bid) {
            const SgpWalk w = sgp_walk(n, g, bid);
            if (g == n && w.count != 1)
                return set_error(MOGT_E_INVALID, "swiglu schedule: work-group %d of %d has %d tiles", bid, g, w.count);
            for (int k = 0; k < w.count; ++k) {
                const int v = w.base + k * w.step;
                if (v < 0 || v >= n)
                    return set_error(MOGT_E_INVALID, "swiglu schedule: work-group %d takes tile %d of %d", bid, v, n);
                ++seen_v[v];
                int mb, nb;
                sgp_block(n_mb, n_nb, v, mb, nb);
                if (mb < 0 || mb >= n_mb || nb < 0 || nb >= n_nb)
                    return set_error(MOGT_E_INVALID, "swiglu schedule: tile %d maps to block (%d, %d)", v, mb, nb);
                ++seen_b[mb * n_nb + nb];
            }
        }
        for (int v = 0; v < n; ++v)
            if (seen_v[v] != 1 || seen_b[v] != 1)
                return set_error(MOGT_E_INVALID, "swiglu schedule (grid %d): tile %d taken %d times, block %d taken %d "
                                 "times", g, v, seen_v[v], v, seen_b[v]);
    }
    return MOGT_OK;
}
