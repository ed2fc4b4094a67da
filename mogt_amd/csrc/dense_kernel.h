// Chunk kernel of the dense affine scan H_t = U_t H_{t-1} + V_t (U_t: R x R,
// H/V: R x C) for gfx950, shared by the pass instantiation files
// (dense_pass_*.hip) and the host recursion (dense_scan.hip).
//
// Semantics: affine_scan_sequential (affine_scan.py:14-62), fp32 state, H_0 = 0,
// optional prefix products P_t = U_t ... U_1; the chunk/carry decomposition of
// affine_scan_block_reference (affine_scan.py:175-278) and the reference's
// hybrid path (triton_scan.py:232-311), re-designed so that no L x R x C
// intermediate is written and every contraction runs on fp32 MFMA.
//
// dense_chunk_kernel runs the recurrence X_t = U_t X_{t-1} + [0 | V_t] on the
// augmented state X = [P | H] over chunks of T steps, one wave per (chunk,
// column block, sequence), with X held in MFMA accumulators.  Its modes give
// every pass of the scan:
//   SUMMARY  X_0 = [I | 0]; writes the chunk's (P_T, H_T).
//   LOCAL    the same, plus every step's local (P_t, H_t) (the block-local scan;
//            any block size).
//   EXCL     X_0 = the chunk's carry (or [I | 0]); writes the state *before*
//            every step, i.e. exclusive prefixes.
//   OUTPUT   X_0 = the chunk's carry; writes H_t (and P_t) after every step.
// SUMMARY, EXCL and OUTPUT run chunks of exactly kDenseChunk steps (the last
// one ragged), which fixes the trip count of the step loop at compile time.
//
// REV (level-0 SUMMARY and OUTPUT): the reverse-time recurrence of the
// backward, G_t = X_t + U_{t+1}^T G_{t+1} (affine_scan.py:110-118), run as a
// forward scan in reversed time s = L - 1 - t: the operands of step s are
// X at memory step L - 1 - s and U at memory step L - s read transposed (zero
// at s = 0, where the state before is zero), and outputs go to memory step
// L - 1 - s.  The chunk summaries are then in reversed order already, so the
// upper levels run unchanged.
#pragma once

#include "common.h"

namespace mogt {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));


enum ChunkMode { CM_SUMMARY = 0, CM_LOCAL = 1, CM_EXCL = 2, CM_OUTPUT = 3 };

// Steps per chunk of the SUMMARY / EXCL / OUTPUT passes at every level.
constexpr int kDenseChunk = 32;

struct ChunkParams {
    const float* U;      // [B, L, R, R] fp32 (level 0) or chunk products of the level below
    const void* V;       // [B, L, R, C] (fp32 / bf16; level >= 1: fp32); null if C == 0;
                         // VK passes: the vectors v [B, L, R]
    const void* K;       // VK passes: the vectors k [B, L, C] of V_t = v_t k_t^T
    const float* carP;   // [B, nb, R, R] chunk carries (EXCL / OUTPUT); null = identity
    const float* carH;   // [B, nb, R, C]                                ; null = zero
    void* outP;          // per-step P: LOCAL fp32 / EXCL fp32 / OUTPUT TO (may be null)
    void* outH;          // per-step H: LOCAL fp32 / EXCL fp32 / OUTPUT TO
    float* sumP;         // [B, nb, R, R] chunk products (SUMMARY / LOCAL)
    float* sumH;         // [B, nb, R, C]
    int64_t L;           // steps of this level
    int R, C, T, nb;
    int withP;           // carry / write the P columns (column block 0 only)
};

// Passes with fewer waves than this at their natural width (up to 4 column
// tiles per wave) run one column tile per wave instead: the step chain of a
// wave gets shorter (fewer MFMAs per step) and more waves run in parallel,
// which is what the small upper levels of the scan are bound by.
constexpr int64_t kDenseNarrowWaves = 256;

// Chunk pass on fp32 MFMA (v_mfma_f32_16x16x4_f32), one wave per (chunk k,
// column block cb, sequence b).  X = [P | H] is padded to 16-row tiles; tile
// (rt, ct) is 4 accumulator registers, lane (g = lane/16, n = lane%16) holding
// X[16 rt + 4 g + i][16 ct + n], i = 0..3.  Per output tile, X_t = U_t X_{t-1}
// + [0 | V_t] is RT x 4 MFMAs over the contraction index j = 16 kt + 4 g + kk
// (K-step kk): with that assignment the B operand of K-step kk is accumulator
// register kk of the previous step in the same lane, so the state never moves
// between steps, and the A operand U_t[16 rt + m][16 kt + 4 g + kk] is four
// consecutive floats of one row of U_t per lane (one 16-byte load when R is a
// multiple of 4, U4).  The operands of the next D steps are always in flight.
//
// W16 (C a multiple of 8, V / H 16-byte aligned): the wave's block of V_t
// (16 RT rows x 16 CTW columns, contiguous along each row) arrives as
// coalesced 16-byte loads and reaches the accumulator layout through a small
// LDS tile; the stored H state leaves the same way, as whole 16-byte pieces
// of rows.  Otherwise V is read and H written one element at a time.
// All global accesses of the step loop go through buffer descriptors, whose
// range check zero-fills padding (see the addressing comment in the body).
template <int RT, int CTW, bool WITHP, bool U4, bool W16, typename TV, typename TO, int MODE, bool VK, bool REV>
__global__ __launch_bounds__(64) void dense_chunk_kernel(ChunkParams p) {
    static_assert(!REV || (!U4 && !VK && (MODE == CM_SUMMARY || MODE == CM_OUTPUT)),
                  "the reverse form reads U transposed, level 0 only");
    constexpr bool FIXED = MODE != CM_LOCAL;   // trip count kDenseChunk
    // OUTPUT passes write H (and P) non-temporally: lines left dirty in the
    // caches are otherwise written back while the next pass streams its
    // operands (measured: level-0 summary after an OUTPUT pass 37-39 -> 23 us
    // at R = 16, C = 48; configs[3] 540 -> 519 us).
    constexpr int kOutPolicy = MODE == CM_OUTPUT ? 2 : 0;
    constexpr int NT = RT + CTW;               // column tiles: RT of P, then CTW of H
    constexpr int D = RT == 1 ? 8 : 4;         // steps of operands in flight
    static_assert(!FIXED || kDenseChunk % D == 0, "chunk must be a multiple of the prefetch depth");
    const int k = blockIdx.x;
    const int cb = blockIdx.y;
    const int b = blockIdx.z;
    const int lane = threadIdx.x;
    const int g = lane >> 4, n = lane & 15;
    const int R = p.R, C = p.C;
    const int c0 = cb * (16 * CTW);
    // P columns are computed by every column block when WITHP (they do not
    // depend on H) and written by block 0; H tiles past C compute padding.
    const bool hasP = WITHP && cb == 0;
    const int64_t t0 = static_cast<int64_t>(k) * p.T;
    const int64_t t1 = t0 + p.T < p.L ? t0 + p.T : p.L;
    const int nv = static_cast<int>(t1 - t0);   // valid steps of this chunk
    const int64_t seq = static_cast<int64_t>(b) * p.nb + k;
    const int64_t RR = static_cast<int64_t>(R) * R;
    const TV* Vg = static_cast<const TV*>(p.V);

    auto trow = [&](int rt, int i) { return 16 * rt + 4 * g + i; };
    auto pcol = [&](int ct) { return 16 * ct + n; };               // ct < RT
    auto hcol = [&](int ct) { return c0 + 16 * (ct - RT) + n; };   // ct >= RT
    auto live = [](int ct) { return ct < RT ? WITHP : true; };   // compile-time per tile

    // ---- initial state ------------------------------------------------------
    f32x4 X[RT][NT];
    const bool fromCarry = (MODE == CM_EXCL || MODE == CM_OUTPUT) && p.carH != nullptr;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int ct = 0; ct < NT; ++ct)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = trow(rt, i);
                float x = 0.0f;
                if (ct < RT) {
                    if (fromCarry && p.carP) {
                        if (WITHP && r < R && pcol(ct) < R) x = p.carP[seq * RR + r * R + pcol(ct)];
                    } else {
                        x = (r == pcol(ct) && r < R) ? 1.0f : 0.0f;
                    }
                } else if (fromCarry && r < R && hcol(ct) < C) {
                    x = p.carH[(seq * R + r) * C + hcol(ct)];
                }
                X[rt][ct][i] = x;
            }

    // ---- addressing ---------------------------------------------------------
    // Every step's block of U, V, H (and P) is reached through a buffer
    // descriptor whose base is the block's first element (uniform, SGPRs) and
    // whose range is the block's bytes; the per-lane byte offsets inside a
    // block are fixed for the whole chunk.  Padding elements (rows / columns
    // past R / C) get the offset kOOB, past every range: the hardware returns 0
    // for such loads and drops such stores, so nothing is masked per step.  A
    // padding step of a ragged last chunk gets range 0 (zero operands, no
    // stores).
    constexpr int kOOB = 0x7ffffff0;
    auto rsrc = [](const void* base, uint32_t bytes) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes),
                                                 0x00020000);
    };
    constexpr int VW = 16 * CTW;                              // columns of the block
    constexpr int VS = VW + 4;    // LDS row stride: 16-byte aligned rows, the column reads
                                  // of the 4 row groups land 16 banks apart
    constexpr int ROWS = 16 * RT;
    constexpr int VE = 16 / static_cast<int>(sizeof(TV));     // V elements per 16-byte piece
    constexpr int OE = 16 / static_cast<int>(sizeof(TO));     // output elements per piece
    constexpr bool VBLOCK = W16 && !VK;                       // V_t block through LDS
    constexpr int NV = VBLOCK ? (ROWS * VW / VE + 63) / 64 : 1;
    constexpr bool STORES = MODE != CM_SUMMARY;
    constexpr bool STAGE_OUT = W16 && STORES;
    constexpr int NO = STAGE_OUT ? (ROWS * VW / OE + 63) / 64 : 1;
    constexpr int ES = MODE == CM_OUTPUT ? static_cast<int>(sizeof(TO)) : 4;   // stored element bytes
    const uint32_t uBytes = static_cast<uint32_t>(RR * 4);
    const uint32_t vBytes = static_cast<uint32_t>((VK ? R : R * C) * static_cast<int>(sizeof(TV)));
    const uint32_t kBytes = static_cast<uint32_t>(C * static_cast<int>(sizeof(TV)));
    const uint32_t hBytes = static_cast<uint32_t>(R * C * ES);
    const uint32_t pBytes = static_cast<uint32_t>(RR * ES);

    // per-lane offsets (bytes) of the A operand: row 16 rt + n, columns 16 kt + 4 g (+ kk)
    int offA[RT][RT][U4 ? 1 : 4];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int kt = 0; kt < RT; ++kt)
#pragma unroll
            for (int kk = 0; kk < (U4 ? 1 : 4); ++kk) {
                const int r = 16 * rt + n, c = 16 * kt + 4 * g + kk;
                offA[rt][kt][kk] = (r < R && c < R) ? (REV ? c * R + r : r * R + c) * 4 : kOOB;
            }
    // V: 16-byte pieces of the ROWS x VW block (VBLOCK) or one element per tile
    // register; VK: element i of v per tile row group and one element of k per
    // column tile (offK)
    int offV[VBLOCK ? NV : RT][VBLOCK || VK ? 1 : CTW][VBLOCK ? 1 : 4];
    int offK[VK ? CTW : 1];
#pragma unroll
    for (int j = 0; j < (VBLOCK ? NV : RT); ++j)
#pragma unroll
        for (int h = 0; h < (VBLOCK || VK ? 1 : CTW); ++h)
#pragma unroll
            for (int i = 0; i < (VBLOCK ? 1 : 4); ++i) {
                int r, c;
                if constexpr (VBLOCK) {
                    const int e = (lane + 64 * j) * VE;
                    r = e < ROWS * VW ? e / VW : R;
                    c = c0 + e % VW;
                } else {
                    r = trow(j, i);
                    c = VK ? 0 : c0 + 16 * h + n;
                }
                const int e = VK ? r : r * C + c;
                offV[j][h][i] = (r < R && c < C) ? e * static_cast<int>(sizeof(TV)) : kOOB;
            }
#pragma unroll
    for (int h = 0; h < (VK ? CTW : 1); ++h) {
        const int c = c0 + 16 * h + n;
        offK[h] = (VK && c < C) ? c * static_cast<int>(sizeof(TV)) : kOOB;
    }
    // H stores: 16-byte pieces (STAGE_OUT) or one element per tile register
    int offH[STAGE_OUT ? NO : RT][STAGE_OUT ? 1 : CTW][STAGE_OUT ? 1 : 4];
#pragma unroll
    for (int j = 0; j < (STAGE_OUT ? NO : RT); ++j)
#pragma unroll
        for (int h = 0; h < (STAGE_OUT ? 1 : CTW); ++h)
#pragma unroll
            for (int i = 0; i < (STAGE_OUT ? 1 : 4); ++i) {
                int r, c;
                if constexpr (STAGE_OUT) {
                    const int e = (lane + 64 * j) * OE;
                    r = e < ROWS * VW ? e / VW : R;
                    c = c0 + e % VW;
                } else {
                    r = trow(j, i);
                    c = c0 + 16 * h + n;
                }
                offH[j][h][i] = (STORES && r < R && c < C) ? (r * C + c) * ES : kOOB;
            }
    // P stores (column block 0 only)
    int offP[RT][RT][4];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int ct = 0; ct < RT; ++ct)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = trow(rt, i), c = pcol(ct);
                offP[rt][ct][i] = (hasP && r < R && c < R) ? (r * R + c) * ES : kOOB;
            }

    __shared__ __align__(16) float s_v[VBLOCK ? ROWS : 1][VBLOCK ? VS : 4];
    __shared__ __align__(16) float s_o[STAGE_OUT ? ROWS : 1][STAGE_OUT ? VS : 4];
    // Orders this wave's LDS writes before its reads of other lanes' data and
    // vice versa (LDS executes one wave's accesses in issue order; a wave-scope
    // fence only keeps the compiler from reordering them).
    auto lds_order = [] { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront"); };

    // ---- operands of one step: A (rows of U_t) and C (V_t) tiles ----------
    struct Ops {
        f32x4 A[RT][RT];
        f32x4 Cv[RT][CTW];
        u32x4 raw[NV];
        f32x4 vv[VK ? RT : 1];   // VK: v rows of the tile row groups
        float kk[VK ? CTW : 1];  // VK: k columns of the column tiles
    };
    const int64_t seqStep = static_cast<int64_t>(b) * p.L;
    // memory step of the operands / outputs of step t (REV: reversed time)
    auto vrow = [&](int64_t t) { return REV ? p.L - 1 - t : t; };
    auto load_ops = [&](int64_t t, bool valid, Ops& o) {
        const int64_t tu = REV ? p.L - t : t;   // REV: U_{t'+1} of memory step t' = L - 1 - t
        const auto ru = rsrc(p.U + (seqStep + (REV && t == 0 ? 0 : tu)) * RR,
                             valid && !(REV && t == 0) ? uBytes : 0u);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int kt = 0; kt < RT; ++kt) {
                if constexpr (U4) {
                    o.A[rt][kt] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(ru, offA[rt][kt][0], 0, 0));
                } else {
#pragma unroll
                    for (int kk = 0; kk < 4; ++kk)
                        o.A[rt][kt][kk] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ru, offA[rt][kt][kk], 0, 0));
                }
            }
        if (!VBLOCK && !Vg) return;   // C == 0: no V (VBLOCK implies V)
        const auto rv = rsrc(static_cast<const char*>(p.V) + (seqStep + vrow(t)) * vBytes, valid ? vBytes : 0u);
        auto ld1 = [](__amdgpu_buffer_rsrc_t r, int off) {   // one element as fp32 bits (bf16: raw)
            if constexpr (sizeof(TV) == 4) return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
            else return __uint_as_float(static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0)));
        };
        if constexpr (VK) {
            const auto rk = rsrc(static_cast<const char*>(p.K) + (seqStep + t) * kBytes, valid ? kBytes : 0u);
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int i = 0; i < 4; ++i) o.vv[rt][i] = ld1(rv, offV[rt][0][i]);
#pragma unroll
            for (int h = 0; h < CTW; ++h) o.kk[h] = ld1(rk, offK[h]);
        } else if constexpr (VBLOCK) {
#pragma unroll
            for (int j = 0; j < NV; ++j) o.raw[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, offV[j][0][0], 0, 0));
        } else {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int h = 0; h < CTW; ++h)
#pragma unroll
                    for (int i = 0; i < 4; ++i) o.Cv[rt][h][i] = ld1(rv, offV[rt][h][i]);   // bf16: raw bits
        }
    };
    // Bring a loaded operand set into the accumulator layout (fp32).
    auto convert_ops = [&](Ops& o) {
        auto widen = [](float x) {   // bf16 raw bits -> fp32
            if constexpr (sizeof(TV) == 2) return __uint_as_float(__float_as_uint(x) << 16);
            else return x;
        };
        if constexpr (VK) {
            // V_t = v_t k_t^T, one fp32 product per element (as a materialised V)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int h = 0; h < CTW; ++h)
#pragma unroll
                    for (int i = 0; i < 4; ++i) o.Cv[rt][h][i] = widen(o.vv[rt][i]) * widen(o.kk[h]);
        } else if constexpr (VBLOCK) {
            // 16-byte pieces -> LDS (fp32) -> accumulator layout
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const int e = (lane + 64 * j) * VE;
                if (ROWS * VW % (64 * VE) == 0 || e < ROWS * VW) {
                    float* dst = &s_v[e / VW][e % VW];
                    if constexpr (sizeof(TV) == 4) {
                        *reinterpret_cast<f32x4*>(dst) = __builtin_bit_cast(f32x4, o.raw[j]);
                    } else {
#pragma unroll
                        for (int q = 0; q < 2; ++q) {
                            const uint32_t w0 = o.raw[j][2 * q], w1 = o.raw[j][2 * q + 1];
                            *reinterpret_cast<f32x4*>(dst + 4 * q) =
                                f32x4{__uint_as_float(w0 << 16), __uint_as_float(w0 & 0xffff0000u),
                                      __uint_as_float(w1 << 16), __uint_as_float(w1 & 0xffff0000u)};
                        }
                    }
                }
            }
            lds_order();
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int h = 0; h < CTW; ++h)
#pragma unroll
                    for (int i = 0; i < 4; ++i) o.Cv[rt][h][i] = s_v[trow(rt, i)][16 * h + n];
            lds_order();
        } else if constexpr (sizeof(TV) == 2) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int h = 0; h < CTW; ++h)
#pragma unroll
                    for (int i = 0; i < 4; ++i) o.Cv[rt][h][i] = widen(o.Cv[rt][h][i]);
        }
    };
    // K-step-major order: consecutive MFMAs belong to different tiles, so none
    // waits on the previous one's result.
    auto step = [&](const Ops& o) {
        f32x4 acc[RT][NT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < NT; ++ct)
                acc[rt][ct] = (ct < RT || (!VBLOCK && !Vg)) ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : o.Cv[rt][ct - RT];
#pragma unroll
        for (int kt = 0; kt < RT; ++kt)
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                    for (int ct = 0; ct < NT; ++ct)
                        if (live(ct))
                            acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(o.A[rt][kt][kk], X[kt][ct][kk],
                                                                               acc[rt][ct], 0, 0, 0);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < NT; ++ct)
                if (live(ct)) X[rt][ct] = acc[rt][ct];
    };
    auto st_elem = [](__amdgpu_buffer_rsrc_t r, int off, float x) {
        if constexpr (ES == 4) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x), r, off, 0, kOutPolicy);
        else __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(x), r, off, 0, kOutPolicy);
    };
    // Per-step output of the state X to row `t` (P columns when WITHP; H
    // columns); `valid` false (a padding step) stores nothing.
    auto store_state = [&](int64_t t, bool valid) {
        const int64_t row = seqStep + vrow(t);
        if constexpr (WITHP) {
            const auto rp = rsrc(static_cast<char*>(p.outP) + row * RR * ES, valid && p.outP ? pBytes : 0u);
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int ct = 0; ct < RT; ++ct)
#pragma unroll
                    for (int i = 0; i < 4; ++i) st_elem(rp, offP[rt][ct][i], X[rt][ct][i]);
        }
        const auto rh = rsrc(static_cast<char*>(p.outH) + row * R * static_cast<int64_t>(C) * ES,
                             valid && p.outH ? hBytes : 0u);
        if constexpr (STAGE_OUT) {
            // H tiles -> LDS -> whole 16-byte pieces of rows
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int h = 0; h < CTW; ++h)
#pragma unroll
                    for (int i = 0; i < 4; ++i) s_o[trow(rt, i)][16 * h + n] = X[rt][RT + h][i];
            lds_order();
#pragma unroll
            for (int j = 0; j < NO; ++j) {
                const int e = min((lane + 64 * j) * OE, ROWS * VW - OE);
                const int r = e / VW, c = e % VW;
                const f32x4 lo = *reinterpret_cast<const f32x4*>(&s_o[r][c]);
                u32x4 piece;
                if constexpr (sizeof(TO) == 4 || MODE != CM_OUTPUT) {
                    piece = __builtin_bit_cast(u32x4, lo);
                } else {
                    const f32x4 hi = *reinterpret_cast<const f32x4*>(&s_o[r][c + 4]);
                    auto pk = [](float a, float b2) {
                        return static_cast<uint32_t>(f32_to_bf16(a)) | (static_cast<uint32_t>(f32_to_bf16(b2)) << 16);
                    };
                    piece = u32x4{pk(lo[0], lo[1]), pk(lo[2], lo[3]), pk(hi[0], hi[1]), pk(hi[2], hi[3])};
                }
                __builtin_amdgcn_raw_buffer_store_b128(piece, rh, offH[j][0][0], 0, kOutPolicy);
            }
            lds_order();
        } else if constexpr (STORES) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int h = 0; h < CTW; ++h)
#pragma unroll
                    for (int i = 0; i < 4; ++i) st_elem(rh, offH[rt][h][i], X[rt][RT + h][i]);
        }
    };

    // ---- the recurrence, operands D steps ahead ---------------------------
    Ops buf[D];
    if constexpr (FIXED) {
        // kDenseChunk steps.  Steps past nv (ragged last chunk) have zero
        // operands and store nothing: their state reaches no output (a
        // chunk's final state is consumed only as the summary of a chunk
        // that has a successor, and every chunk before the last is full).
        const int last = nv - 1;
#pragma unroll
        for (int i = 0; i < D; ++i) load_ops(t0 + min(i, last), i < nv, buf[i]);
        convert_ops(buf[0]);
        for (int s0 = 0; s0 < kDenseChunk; s0 += D) {
#pragma unroll
            for (int i = 0; i < D; ++i) {
                const int s = s0 + i;
                if constexpr (MODE == CM_EXCL) store_state(t0 + min(s, last), s < nv);
                step(buf[i]);
                if constexpr (MODE == CM_OUTPUT) store_state(t0 + min(s, last), s < nv);
                // refill this slot, then convert the next step's operands
                // while this step's MFMAs run
                load_ops(t0 + min(s + D, last), s + D < nv, buf[i]);
                convert_ops(buf[(i + 1) % D]);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < D; ++i) load_ops(t0 + min(i, nv - 1), true, buf[i]);
        for (int64_t t = t0; t < t1; t += D) {
#pragma unroll
            for (int i = 0; i < D; ++i) {
                const int64_t ti = t + i;
                if (ti >= t1) break;
                convert_ops(buf[i]);
                step(buf[i]);
                store_state(ti, true);
                load_ops(ti + D < t1 ? ti + D : t1 - 1, true, buf[i]);
            }
        }
    }

    if constexpr (MODE == CM_SUMMARY || MODE == CM_LOCAL) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < NT; ++ct)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = trow(rt, i);
                    if (r >= R || !live(ct)) continue;
                    if (ct < RT) {
                        if (hasP && pcol(ct) < R) p.sumP[seq * RR + r * R + pcol(ct)] = X[rt][ct][i];
                    } else if (hcol(ct) < C) {
                        p.sumH[(seq * R + r) * C + hcol(ct)] = X[rt][ct][i];
                    }
                }
    }
}

// ---------------------------------------------------------------------------
// Launch: tile shape from (R, C), 16-byte paths from alignment.
// ---------------------------------------------------------------------------
inline int dense_col_tiles(int64_t C) { return C <= 16 ? 1 : C <= 32 ? 2 : C <= 48 ? 3 : 4; }
inline int dense_col_blocks(int64_t C, int ctw) {
    return C == 0 ? 1 : static_cast<int>((C + 16 * ctw - 1) / (16 * ctw));
}

template <int RT, int CTW, bool U4, typename TV, typename TO, int MODE, bool VK, bool REV>
int dense_launch_ct(const ChunkParams& c, int64_t B, hipStream_t st) {
    const dim3 grid(c.nb, dense_col_blocks(c.C, CTW), static_cast<unsigned>(B));
    auto al16 = [](const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
    // W16: whole 16-byte pieces of both element types (C % 8 == 0): V blocks
    // (not VK) and staged H stores (not SUMMARY).
    const bool w16 = c.V && (VK || al16(c.V)) && c.C % 8 == 0 && c.C >= 8 && (!c.outH || al16(c.outH));
    constexpr bool alwaysP = MODE == CM_SUMMARY || MODE == CM_LOCAL;
    constexpr bool anyW16 = !(VK && MODE == CM_SUMMARY);   // VK summaries use neither path
    const bool wp = alwaysP || c.withP;
    if (wp && w16 && anyW16) hipLaunchKernelGGL((dense_chunk_kernel<RT, CTW, true, U4, anyW16, TV, TO, MODE, VK, REV>), grid, dim3(64), 0, st, c);
    else if (wp) hipLaunchKernelGGL((dense_chunk_kernel<RT, CTW, true, U4, false, TV, TO, MODE, VK, REV>), grid, dim3(64), 0, st, c);
    else if constexpr (!alwaysP) {
        if (w16) hipLaunchKernelGGL((dense_chunk_kernel<RT, CTW, false, U4, true, TV, TO, MODE, VK, REV>), grid, dim3(64), 0, st, c);
        else hipLaunchKernelGGL((dense_chunk_kernel<RT, CTW, false, U4, false, TV, TO, MODE, VK, REV>), grid, dim3(64), 0, st, c);
    }
    return check_launch("dense_chunk_kernel");
}

template <int RT, bool U4, typename TV, typename TO, int MODE, bool VK, bool REV>
int dense_launch_c(const ChunkParams& c, int64_t B, hipStream_t st) {
    const int ctw = dense_col_tiles(c.C);
    if (ctw > 1 && B * c.nb * dense_col_blocks(c.C, ctw) < kDenseNarrowWaves)
        return dense_launch_ct<RT, 1, U4, TV, TO, MODE, VK, REV>(c, B, st);
    switch (ctw) {
        case 1: return dense_launch_ct<RT, 1, U4, TV, TO, MODE, VK, REV>(c, B, st);
        case 2: return dense_launch_ct<RT, 2, U4, TV, TO, MODE, VK, REV>(c, B, st);
        case 3: return dense_launch_ct<RT, 3, U4, TV, TO, MODE, VK, REV>(c, B, st);
        default: return dense_launch_ct<RT, 4, U4, TV, TO, MODE, VK, REV>(c, B, st);
    }
}

// One pass over a level.  U4: R % 4 == 0 and 16-byte aligned rows of U (level
// >= 1 products live in the 256-byte aligned workspace).  The FIXED passes
// require c.T == kDenseChunk.  VK: V_t = v_t k_t^T from c.V = v, c.K = k.
template <typename TV, typename TO, int MODE, bool VK = false, bool REV = false>
int dense_launch_pass(const ChunkParams& c, int64_t B, hipStream_t st) {
    if (MODE != CM_LOCAL && c.T != kDenseChunk)
        return set_error(MOGT_E_INVALID, "dense pass: chunk length %d, expected %d", c.T, kDenseChunk);
    if constexpr (REV) {   // transposed U: element loads
        if (c.R <= 16) return dense_launch_c<1, false, TV, TO, MODE, VK, true>(c, B, st);
        return dense_launch_c<2, false, TV, TO, MODE, VK, true>(c, B, st);
    } else {
        const bool u4 = c.R % 4 == 0 && reinterpret_cast<uintptr_t>(c.U) % 16 == 0;
        if (c.R <= 16) return u4 ? dense_launch_c<1, true, TV, TO, MODE, VK, false>(c, B, st) : dense_launch_c<1, false, TV, TO, MODE, VK, false>(c, B, st);
        return u4 ? dense_launch_c<2, true, TV, TO, MODE, VK, false>(c, B, st) : dense_launch_c<2, false, TV, TO, MODE, VK, false>(c, B, st);
    }
}

// Instantiated once each in dense_pass_*.hip (parallel compilation).
#define MOGT_DENSE_PASSES(X)                 \
    X(float, float, CM_SUMMARY, false)       \
    X(bf16_t, float, CM_SUMMARY, false)      \
    X(float, float, CM_EXCL, false)          \
    X(float, float, CM_LOCAL, false)         \
    X(bf16_t, float, CM_LOCAL, false)        \
    X(float, float, CM_OUTPUT, false)        \
    X(float, bf16_t, CM_OUTPUT, false)       \
    X(bf16_t, float, CM_OUTPUT, false)       \
    X(bf16_t, bf16_t, CM_OUTPUT, false)      \
    X(float, float, CM_SUMMARY, true)        \
    X(bf16_t, float, CM_SUMMARY, true)       \
    X(float, float, CM_OUTPUT, true)         \
    X(float, bf16_t, CM_OUTPUT, true)        \
    X(bf16_t, float, CM_OUTPUT, true)        \
    X(bf16_t, bf16_t, CM_OUTPUT, true)
#define MOGT_DENSE_EXTERN(TV, TO, M, VK) \
    extern template int dense_launch_pass<TV, TO, M, VK>(const ChunkParams&, int64_t, hipStream_t);
MOGT_DENSE_PASSES(MOGT_DENSE_EXTERN)
#undef MOGT_DENSE_EXTERN
// the reverse-time level-0 passes (dense_pass_rev.hip)
extern template int dense_launch_pass<float, float, CM_SUMMARY, false, true>(const ChunkParams&, int64_t, hipStream_t);
extern template int dense_launch_pass<float, float, CM_OUTPUT, false, true>(const ChunkParams&, int64_t, hipStream_t);

}  // namespace mogt
