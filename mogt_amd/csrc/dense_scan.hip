// Dense affine scan H_t = U_t H_{t-1} + V_t (U_t: R x R, H/V: R x C) for gfx950.
//
// Semantics: affine_scan_sequential (affine_scan.py:14-62), fp32 state, H_0 = 0,
// optional prefix products P_t = U_t ... U_1; the chunk/carry decomposition of
// affine_scan_block_reference (affine_scan.py:175-278) and the reference's
// hybrid path (triton_scan.py:232-311), re-designed so that no L x R x C
// intermediate is written and every contraction runs on fp32 MFMA.
//
// One kernel (dense_chunk_kernel) runs the recurrence X_t = U_t X_{t-1} +
// [0 | V_t] on the augmented state X = [P | H] over chunks of T steps, one wave
// per (chunk, column block, sequence), with X held in MFMA accumulators (see
// the kernel comment).  Its modes give every pass of the scan:
//   SUMMARY  X_0 = [I | 0]; writes the chunk's (P_T, H_T).
//   LOCAL    the same, plus every step's local (P_t, H_t) (the block-local scan).
//   EXCL     X_0 = the chunk's carry (or [I | 0]); writes the state *before*
//            every step, i.e. exclusive prefixes.
//   OUTPUT   X_0 = the chunk's carry; writes H_t (and P_t) after every step.
// The carries are themselves an affine scan: (P_T, H_T) of consecutive chunks
// compose exactly like (U_t, V_t) -- the reference's affine_combine
// (affine_scan.py:4-11), (P_a, H_a) o (P_b, H_b) = (P_a P_b, P_a H_b + H_a).
// So the summaries, laid out like U and V, are scanned by the same kernel,
// recursively: summaries of summaries until one chunk remains, then EXCL passes
// back down produce every level's carries, and the OUTPUT pass of level 0
// writes H once.  Each pass is independent per chunk (no inter-chunk waits).
#include "common.h"

namespace mogt {

typedef float f32x4 __attribute__((ext_vector_type(4)));

enum ChunkMode { CM_SUMMARY = 0, CM_LOCAL = 1, CM_EXCL = 2, CM_OUTPUT = 3 };

struct ChunkParams {
    const float* U;      // [B, L, R, R] fp32 (level 0) or chunk products of the level below
    const void* V;       // [B, L, R, C] (fp32 / bf16; level >= 1: fp32); null if C == 0
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

// Chunk pass on fp32 MFMA (v_mfma_f32_16x16x4_f32), one wave per (chunk k,
// column block cb, sequence b).  X = [P | H] is padded to 16-row tiles; tile
// (rt, ct) is 4 accumulator registers, lane (g = lane/16, n = lane%16) holding
// X[16 rt + 4 g + i][16 ct + n], i = 0..3.  Per output tile, X_t = U_t X_{t-1}
// + [0 | V_t] is RT x 4 MFMAs over the contraction index j = 16 kt + 4 g + kk
// (K-step kk): with that assignment the B operand of K-step kk is accumulator
// register kk of the previous step in the same lane, so the state never moves
// between steps, and the A operand U_t[16 rt + m][16 kt + 4 g + kk] is four
// consecutive floats of one row of U_t per lane (one 16-byte load when R is a
// multiple of 4).  The operands of the next D steps are always in flight.
// Rows and columns past R / C read a clamped in-bounds address and count as 0.
template <int RT, int CTW, bool U4, typename TV, typename TO, int MODE>
__global__ __launch_bounds__(64) void dense_chunk_kernel(ChunkParams p) {
    constexpr int NT = RT + CTW;          // column tiles: RT of P, then CTW of H
    constexpr int D = RT == 1 ? 3 : 2;    // steps of operands in flight
    const int k = blockIdx.x;
    const int cb = blockIdx.y;
    const int b = blockIdx.z;
    const int lane = threadIdx.x;
    const int g = lane >> 4, n = lane & 15;
    const int R = p.R, C = p.C;
    const int c0 = cb * (16 * CTW);
    const bool hasP = cb == 0 && (MODE == CM_SUMMARY || MODE == CM_LOCAL || p.withP);
    const int nH = C <= c0 ? 0 : min(CTW, (C - c0 + 15) / 16);
    const int64_t t0 = static_cast<int64_t>(k) * p.T;
    const int64_t t1 = t0 + p.T < p.L ? t0 + p.T : p.L;
    const int64_t seq = static_cast<int64_t>(b) * p.nb + k;
    const int64_t RR = static_cast<int64_t>(R) * R;
    const TV* Vg = static_cast<const TV*>(p.V);

    auto trow = [&](int rt, int i) { return 16 * rt + 4 * g + i; };
    auto pcol = [&](int ct) { return 16 * ct + n; };               // ct < RT
    auto hcol = [&](int ct) { return c0 + 16 * (ct - RT) + n; };   // ct >= RT
    auto live = [&](int ct) { return ct < RT ? hasP : (ct - RT < nH); };

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
                        if (hasP && r < R && pcol(ct) < R) x = p.carP[seq * RR + r * R + pcol(ct)];
                    } else {
                        x = (r == pcol(ct) && r < R) ? 1.0f : 0.0f;
                    }
                } else if (fromCarry && ct - RT < nH && r < R && hcol(ct) < C) {
                    x = p.carH[(seq * R + r) * C + hcol(ct)];
                }
                X[rt][ct][i] = x;
            }

    // ---- operands of one step: A (rows of U_t) and C (V_t) tiles ----------
    struct Ops {
        f32x4 A[RT][RT];
        f32x4 Cv[RT][CTW];
    };
    auto load_ops = [&](int64_t t, Ops& o) {
        const float* Ut = p.U + (static_cast<int64_t>(b) * p.L + t) * RR;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int kt = 0; kt < RT; ++kt) {
                const int r = min(16 * rt + n, R - 1);
                if constexpr (U4) {
                    const int c = min(16 * kt + 4 * g, R - 4);
                    o.A[rt][kt] = *reinterpret_cast<const f32x4*>(Ut + r * R + c);
                } else {
#pragma unroll
                    for (int kk = 0; kk < 4; ++kk) o.A[rt][kt][kk] = Ut[r * R + min(16 * kt + 4 * g + kk, R - 1)];
                }
            }
        if (Vg) {
            const TV* Vt = Vg + (static_cast<int64_t>(b) * p.L + t) * R * static_cast<int64_t>(C);
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int h = 0; h < CTW; ++h)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int r = min(trow(rt, i), R - 1);
                        const int c = min(c0 + 16 * h + n, C - 1);
                        // raw value (bf16: its bit pattern), converted when masked
                        const TV raw = Vt[static_cast<int64_t>(r) * C + c];
                        if constexpr (sizeof(TV) == 4) o.Cv[rt][h][i] = raw;
                        else o.Cv[rt][h][i] = __uint_as_float(static_cast<uint32_t>(raw));
                    }
        }
    };
    // Convert and zero the padding of a loaded operand set (values past R / C).
    auto mask_ops = [&](Ops& o) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
            for (int kt = 0; kt < RT; ++kt)
#pragma unroll
                for (int kk = 0; kk < 4; ++kk)
                    if (16 * rt + n >= R || 16 * kt + 4 * g + kk >= R) o.A[rt][kt][kk] = 0.0f;
#pragma unroll
            for (int h = 0; h < CTW; ++h)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float v = o.Cv[rt][h][i];
                    if constexpr (sizeof(TV) == 2) v = __uint_as_float(__float_as_uint(v) << 16);
                    o.Cv[rt][h][i] = (!Vg || trow(rt, i) >= R || c0 + 16 * h + n >= C) ? 0.0f : v;
                }
        }
    };
    auto step = [&](const Ops& o) {
        f32x4 Xn[RT][NT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < NT; ++ct) {
                if (!live(ct)) { Xn[rt][ct] = X[rt][ct]; continue; }
                f32x4 acc = ct < RT ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : o.Cv[rt][ct - RT];
#pragma unroll
                for (int kt = 0; kt < RT; ++kt)
#pragma unroll
                    for (int kk = 0; kk < 4; ++kk)
                        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(o.A[rt][kt][kk], X[kt][ct][kk], acc, 0, 0, 0);
                Xn[rt][ct] = acc;
            }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < NT; ++ct) X[rt][ct] = Xn[rt][ct];
    };
    // Per-step output of the state X (LOCAL, EXCL: fp32; OUTPUT: TO).
    auto store_state = [&](int64_t t) {
        if constexpr (MODE == CM_SUMMARY) return;
        const int64_t row = static_cast<int64_t>(b) * p.L + t;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < NT; ++ct)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = trow(rt, i);
                    if (r >= R || !live(ct)) continue;
                    const float x = X[rt][ct][i];
                    if (ct < RT) {
                        if (pcol(ct) >= R || !p.outP) continue;
                        const int64_t at = (row * R + r) * R + pcol(ct);
                        if constexpr (MODE == CM_OUTPUT) static_cast<TO*>(p.outP)[at] = IO<TO>::st(x);
                        else static_cast<float*>(p.outP)[at] = x;
                    } else {
                        if (hcol(ct) >= C) continue;
                        const int64_t at = (row * R + r) * C + hcol(ct);
                        if constexpr (MODE == CM_OUTPUT) static_cast<TO*>(p.outH)[at] = IO<TO>::st(x);
                        else static_cast<float*>(p.outH)[at] = x;
                    }
                }
    };

    // ---- the recurrence, operands D steps ahead ---------------------------
    Ops buf[D];
#pragma unroll
    for (int i = 0; i < D; ++i) load_ops(t0 + i < t1 ? t0 + i : t1 - 1, buf[i]);
    for (int64_t t = t0; t < t1; t += D) {
#pragma unroll
        for (int i = 0; i < D; ++i) {
            const int64_t ti = t + i;
            if (ti >= t1) break;
            mask_ops(buf[i]);
            if constexpr (MODE == CM_EXCL) store_state(ti);
            step(buf[i]);
            if constexpr (MODE == CM_LOCAL || MODE == CM_OUTPUT) store_state(ti);
            // refill this slot (always issued; clamped to the chunk's last step)
            load_ops(ti + D < t1 ? ti + D : t1 - 1, buf[i]);
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
                        if (pcol(ct) < R) p.sumP[seq * RR + r * R + pcol(ct)] = X[rt][ct][i];
                    } else if (hcol(ct) < C) {
                        p.sumH[(seq * R + r) * C + hcol(ct)] = X[rt][ct][i];
                    }
                }
    }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
namespace {

// Steps per chunk: 32 at level 0 (long serial runs over the big operands),
// 8 above it (the summary levels are small, so parallelism matters more than
// the number of levels).
constexpr int kChunk0 = 32;
constexpr int kChunkUp = 8;
inline int chunk_len(int level) { return level == 0 ? kChunk0 : kChunkUp; }

int col_tiles(int64_t C) { return C <= 16 ? 1 : C <= 32 ? 2 : C <= 48 ? 3 : 4; }
int col_blocks(int64_t C, int ctw) {
    return C == 0 ? 1 : static_cast<int>((C + 16 * ctw - 1) / (16 * ctw));
}

template <int RT, int CTW, bool U4, typename TV, typename TO, int MODE>
int launch_ct(const ChunkParams& c, int64_t B, hipStream_t st) {
    hipLaunchKernelGGL((dense_chunk_kernel<RT, CTW, U4, TV, TO, MODE>),
                       dim3(c.nb, col_blocks(c.C, CTW), static_cast<unsigned>(B)), dim3(64), 0, st, c);
    return check_launch("dense_chunk_kernel");
}

template <int RT, bool U4, typename TV, typename TO, int MODE>
int launch_c(const ChunkParams& c, int64_t B, hipStream_t st) {
    switch (col_tiles(c.C)) {
        case 1: return launch_ct<RT, 1, U4, TV, TO, MODE>(c, B, st);
        case 2: return launch_ct<RT, 2, U4, TV, TO, MODE>(c, B, st);
        case 3: return launch_ct<RT, 3, U4, TV, TO, MODE>(c, B, st);
        default: return launch_ct<RT, 4, U4, TV, TO, MODE>(c, B, st);
    }
}

// One pass over a level.  U4: R % 4 == 0 and 16-byte aligned rows of U (level
// >= 1 products live in the 256-byte aligned workspace).
template <typename TV, typename TO, int MODE>
int launch_pass(const ChunkParams& c, int64_t B, hipStream_t st) {
    const bool u4 = c.R % 4 == 0 && reinterpret_cast<uintptr_t>(c.U) % 16 == 0;
    if (c.R <= 16) return u4 ? launch_c<1, true, TV, TO, MODE>(c, B, st) : launch_c<1, false, TV, TO, MODE>(c, B, st);
    return u4 ? launch_c<2, true, TV, TO, MODE>(c, B, st) : launch_c<2, false, TV, TO, MODE>(c, B, st);
}

// Workspace: per level l >= 0 with n_l = ceil(n_{l-1} / T) chunks (n_{-1} = L),
// the chunk products (sumP, sumH) and the chunk carries (carP, carH), fp32.
struct Level {
    int64_t n;                        // chunks of this level (= steps of the next)
    size_t sumP, sumH, carP, carH;    // byte offsets
};
struct DenseGeo {
    int depth;
    Level lv[24];
    size_t bytes;
};

DenseGeo dense_geometry(int64_t B, int64_t L, int64_t R, int64_t C) {
    DenseGeo g{};
    size_t off = WS_HDR_BYTES;
    auto take = [&](size_t nbytes) { size_t o = off; off = round_up(off + nbytes, 256); return o; };
    int64_t steps = L;
    while (steps > 1 && g.depth < 24) {
        const int T = chunk_len(g.depth);
        Level& v = g.lv[g.depth++];
        v.n = (steps + T - 1) / T;
        const size_t m = static_cast<size_t>(B) * v.n;
        v.sumP = take(m * R * R * sizeof(float));
        v.sumH = take(m * R * static_cast<size_t>(C) * sizeof(float));
        v.carP = take(m * R * R * sizeof(float));
        v.carH = take(m * R * static_cast<size_t>(C) * sizeof(float));
        steps = v.n;
    }
    g.bytes = off;
    return g;
}

// Exclusive scan of a level's (U, V) sequence of `len` steps into (outP, outH):
// the state before every step, starting from [I | 0].  Recursive over chunk
// products; lv indexes the workspace level holding this sequence's chunks.
template <typename TV>
int excl_scan(const float* U, const void* V, int64_t len, float* outP, float* outH, int64_t B,
              int64_t R, int64_t C, bool withP, char* ws, const DenseGeo& geo, int lv,
              hipStream_t st) {
    ChunkParams c{};
    c.U = U; c.V = C > 0 ? V : nullptr;
    c.L = len; c.R = static_cast<int>(R); c.C = static_cast<int>(C); c.T = chunk_len(lv);
    c.nb = static_cast<int>((len + c.T - 1) / c.T);
    c.withP = withP;
    c.outP = withP ? outP : nullptr;
    c.outH = outH;
    if (c.nb > 1) {
        const Level& v = geo.lv[lv];
        ChunkParams s = c;
        s.sumP = reinterpret_cast<float*>(ws + v.sumP);
        s.sumH = reinterpret_cast<float*>(ws + v.sumH);
        int rc = launch_pass<TV, float, CM_SUMMARY>(s, B, st);
        if (rc) return rc;
        // carries of this level's chunks: exclusive scan of the chunk products
        rc = excl_scan<float>(s.sumP, s.sumH, c.nb, reinterpret_cast<float*>(ws + v.carP),
                              reinterpret_cast<float*>(ws + v.carH), B, R, C, withP, ws, geo, lv + 1, st);
        if (rc) return rc;
        c.carP = withP ? reinterpret_cast<float*>(ws + v.carP) : nullptr;
        c.carH = reinterpret_cast<float*>(ws + v.carH);
    }
    return launch_pass<TV, float, CM_EXCL>(c, B, st);
}

template <typename TV, typename TO>
int run_levels(const float* U, const void* V, void* H, void* P, int64_t B, int64_t L, int64_t R,
               int64_t C, char* ws, const DenseGeo& geo, hipStream_t st) {
    const bool withP = P != nullptr;
    ChunkParams c{};
    c.U = U; c.V = C > 0 ? V : nullptr;
    c.L = L; c.R = static_cast<int>(R); c.C = static_cast<int>(C); c.T = chunk_len(0);
    c.nb = static_cast<int>((L + c.T - 1) / c.T);
    c.withP = withP;
    c.outP = P; c.outH = H;
    if (c.nb > 1) {
        const Level& v = geo.lv[0];
        ChunkParams s = c;
        s.sumP = reinterpret_cast<float*>(ws + v.sumP);
        s.sumH = reinterpret_cast<float*>(ws + v.sumH);
        int rc = launch_pass<TV, TO, CM_SUMMARY>(s, B, st);
        if (rc) return rc;
        rc = excl_scan<float>(s.sumP, s.sumH, c.nb, reinterpret_cast<float*>(ws + v.carP),
                              reinterpret_cast<float*>(ws + v.carH), B, R, C, withP, ws, geo, 1, st);
        if (rc) return rc;
        c.carP = withP ? reinterpret_cast<float*>(ws + v.carP) : nullptr;
        c.carH = reinterpret_cast<float*>(ws + v.carH);
    }
    return launch_pass<TV, TO, CM_OUTPUT>(c, B, st);
}

int check_dense_shapes(int64_t B, int64_t L, int64_t R, int64_t C) {
    if (B < 0 || L < 0 || R <= 0 || C < 0)
        return set_error(MOGT_E_INVALID, "U must be [B, L, R, R] and V must be [B, L, R, C]");
    if (R > 32) return set_error(MOGT_E_INVALID, "R = %lld not supported (R <= 32)", (long long)R);
    if (C > (1 << 22)) return set_error(MOGT_E_INVALID, "C too large");
    return MOGT_OK;
}

int run_dense(const float* U, const void* V, void* H, void* P, int64_t B, int64_t L, int64_t R,
              int64_t C, int v_dtype, int out_dtype, void* ws, size_t ws_bytes, void* stream) {
    clear_error();
    int rc = check_dense_shapes(B, L, R, C);
    if (rc) return rc;
    if (v_dtype != MOGT_F32 && v_dtype != MOGT_BF16) return set_error(MOGT_E_INVALID, "unsupported V dtype");
    if (out_dtype != MOGT_F32 && out_dtype != MOGT_BF16) return set_error(MOGT_E_INVALID, "unsupported output dtype");
    if (B == 0 || L == 0) return MOGT_OK;
    if (!U || (C > 0 && (!V || !H)) || (C == 0 && !P)) return set_error(MOGT_E_INVALID, "null tensor pointer");
    if (B > 65535 || (L + kChunk0 - 1) / kChunk0 > 0x7fffffffLL)
        return set_error(MOGT_E_INVALID, "problem too large for one launch");
    const DenseGeo g = dense_geometry(B, L, R, C);
    if (!ws || ws_bytes < g.bytes)
        return set_error(MOGT_E_WORKSPACE, "workspace of %zu bytes required, got %zu", g.bytes, ws_bytes);
    char* base = static_cast<char*>(ws);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (v_dtype == MOGT_F32 && out_dtype == MOGT_F32) return run_levels<float, float>(U, V, H, P, B, L, R, C, base, g, st);
    if (v_dtype == MOGT_F32 && out_dtype == MOGT_BF16) return run_levels<float, bf16_t>(U, V, H, P, B, L, R, C, base, g, st);
    if (v_dtype == MOGT_BF16 && out_dtype == MOGT_F32) return run_levels<bf16_t, float>(U, V, H, P, B, L, R, C, base, g, st);
    return run_levels<bf16_t, bf16_t>(U, V, H, P, B, L, R, C, base, g, st);
}

}  // namespace
}  // namespace mogt

using namespace mogt;

extern "C" size_t mogt_affine_scan_workspace_bytes(int64_t batch, int64_t length, int64_t rank,
                                                   int64_t channels) {
    if (batch <= 0 || length <= 0 || rank <= 0 || rank > 32 || channels < 0) return WS_HDR_BYTES;
    return dense_geometry(batch, length, rank, channels).bytes;
}

extern "C" int mogt_affine_scan_fwd(const void* U, const void* V, void* H, void* U_prefix, int64_t batch,
                                    int64_t length, int64_t rank, int64_t channels, int v_dtype,
                                    int out_dtype, void* workspace, size_t workspace_bytes,
                                    void* stream) {
    return run_dense(static_cast<const float*>(U), V, H, U_prefix, batch, length, rank, channels,
                     v_dtype, out_dtype, workspace, workspace_bytes, stream);
}

extern "C" size_t mogt_fused_scan_workspace_bytes(int64_t batch, int64_t length, int64_t rank) {
    return mogt_affine_scan_workspace_bytes(batch, length, rank, 0);
}

extern "C" int mogt_fused_scan_fwd(const void* U, void* Y, int64_t batch, int64_t length, int64_t rank,
                                   int out_dtype, void* workspace, size_t workspace_bytes,
                                   void* stream) {
    return run_dense(static_cast<const float*>(U), nullptr, nullptr, Y, batch, length, rank, 0,
                     MOGT_F32, out_dtype, workspace, workspace_bytes, stream);
}

extern "C" int mogt_affine_local_scan(const void* U, const void* V, void* U_prefix, void* H_prefix,
                                      void* U_summary, void* H_summary, int64_t batch, int64_t length,
                                      int64_t rank, int64_t channels, int64_t block_size, int v_dtype,
                                      void* stream) {
    clear_error();
    int rc = check_dense_shapes(batch, length, rank, channels);
    if (rc) return rc;
    if (block_size <= 0) return set_error(MOGT_E_INVALID, "block_size must be positive");
    if (v_dtype != MOGT_F32 && v_dtype != MOGT_BF16) return set_error(MOGT_E_INVALID, "unsupported V dtype");
    if (batch == 0 || length == 0) return MOGT_OK;
    if (!U || !U_prefix || !U_summary || (channels > 0 && (!V || !H_prefix || !H_summary)))
        return set_error(MOGT_E_INVALID, "null tensor pointer");
    const int64_t nb = (length + block_size - 1) / block_size;
    if (nb > 0x7fffffffLL || block_size > 0x7fffffffLL || batch > 65535)
        return set_error(MOGT_E_INVALID, "problem too large for one launch");
    ChunkParams c{};
    c.U = static_cast<const float*>(U);
    c.V = channels > 0 ? V : nullptr;
    c.outP = U_prefix; c.outH = H_prefix;
    c.sumP = static_cast<float*>(U_summary);
    c.sumH = static_cast<float*>(H_summary);
    c.L = length; c.R = static_cast<int>(rank); c.C = static_cast<int>(channels);
    c.T = static_cast<int>(block_size); c.nb = static_cast<int>(nb);
    c.withP = 1;
    hipStream_t st = static_cast<hipStream_t>(stream);
    return v_dtype == MOGT_BF16 ? launch_pass<bf16_t, float, CM_LOCAL>(c, batch, st)
                                : launch_pass<float, float, CM_LOCAL>(c, batch, st);
}
