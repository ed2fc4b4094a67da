// Single-pass diagonal affine scan h_t = a_t * h_{t-1} + b_t for gfx950.
//
// Semantics follow the reference's sequential recurrence (affine_scan.py:48-55,
// H_0 = 0, fp32 state, outputs cast at the end) in the per-feature R=C=1 case,
// and the coupled write-forget gate of the MOGT mixer (model_mogt.py:166-182).
//
// Design (one launch, 3 HBM streams: read a, read b, write h):
//   tile     one work-group = WT waves x 64 lanes.  A lane owns VEC consecutive
//            features (one VEC-wide vector load/store per row, rows contiguous
//            along D), a wave owns S consecutive steps of them; the WT waves of
//            a group cover T = WT*S consecutive steps of the same FW = 64*VEC
//            features.
//   level 1  each lane scans its S steps serially in registers (2 FMA/element).
//   level 2  wave summaries (prod a, h_end) go through LDS; each wave folds the
//            summaries of the waves before it to get its in-chunk carry.
//   level 3  chunks of one feature group are chained with a decoupled look-back
//            (tagged 64-bit words, see common.h): publish the chunk aggregate,
//            fold predecessors' aggregates until an inclusive prefix is found,
//            publish the inclusive prefix, then apply the carry in registers and
//            write h once.
#include "common.h"

namespace mogt {

struct DiagParams {
    const void* a;      // [B, L, D] (DIAG)            | gate logits z [B, L, R] (COUPLED)
    const void* b;      // [B, L, D]                    | v [B, L, D]
    void* h;            // [B, L, D]
    void* aprefix;      // [B, L, D] or null
    int64_t L, D;
    int n_fg;           // feature groups per batch row
    int n_ch;           // chunks along L
    int G;              // B * n_fg look-back chains
    int R, C;           // COUPLED: gate count and channels per gate (D = R*C)
    float damping;      // COUPLED: connection damping (identity connection scale)
    uint32_t* hdr;
    uint32_t* flags;    // [G][n_ch]
    uint64_t* pay;      // 4 planes of [G][n_ch][FW] words: aggA, aggH, incA, incH
    int64_t plane;      // words per plane
};

template <typename TIn, typename TZ, typename TOut, int VEC, int S, int WT, bool PREFIX,
          bool COUPLED>
__global__ __launch_bounds__(64 * WT) void diag_scan_kernel(DiagParams p) {
    constexpr int NT = 64 * WT;
    constexpr int FW = 64 * VEC;
    constexpr int T = WT * S;
    static_assert(FW <= NT, "look-back needs one thread per feature of the group");

    __shared__ int s_ticket;
    __shared__ uint32_t s_epoch;
    __shared__ float s_sumA[WT][FW];
    __shared__ float s_sumH[WT][FW];
    __shared__ float s_inA[FW];
    __shared__ float s_inH[FW];
    __shared__ int s_nfold, s_found;

    ws_begin(p.hdr, &s_ticket, &s_epoch);
    const int ticket = s_ticket;
    const uint32_t epoch = s_epoch;
    const int chunk = ticket / p.G;
    const int g = ticket - chunk * p.G;
    const int bi = g / p.n_fg;
    const int fg = g - bi * p.n_fg;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform (SGPR)
    const int64_t fbase = static_cast<int64_t>(fg) * FW;          // first feature of the group
    const int flane = lane * VEC;                                  // lane offset inside the group
    const bool fvalid = fbase + flane < p.D;
    const int64_t t0 = static_cast<int64_t>(chunk) * T + wave * S;
    const int64_t row0 = static_cast<int64_t>(bi) * p.L;
    // Wave-uniform row pointers; lanes only add their 32-bit feature offset.
    const int64_t rowoff0 = (row0 + t0) * p.D + fbase;

    // ---- load (all loads issued before any use) -------------------------
    float ra[S][VEC], rb[S][VEC];
    {
        const TIn* pa = static_cast<const TIn*>(COUPLED ? p.b : p.a) + rowoff0;
        const TIn* pb = static_cast<const TIn*>(p.b) + rowoff0;
        const TZ* pz = COUPLED ? static_cast<const TZ*>(p.a) + (row0 + t0) * p.R : nullptr;
        const int gi = COUPLED ? static_cast<int>((fbase + flane) / p.C) : 0;
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const bool tvalid = t0 + s < p.L;   // wave-uniform
            if (fvalid && tvalid) {
                if constexpr (COUPLED) {
                    const float zz = IO<TZ>::ld(pz[gi]);
                    float vv[VEC];
                    load_vec<TIn, VEC>(pb + flane, vv);
                    const float gate = sigmoidf_(zz);
                    // reference: V_t_raw * value_gate.to(V_t_raw.dtype), U * (1 - value_gate)
                    const float gate_io = IO<TIn>::ld(IO<TIn>::st(gate));
#pragma unroll
                    for (int v = 0; v < VEC; ++v) {
                        ra[s][v] = p.damping * (1.0f - gate);
                        rb[s][v] = IO<TIn>::ld(IO<TIn>::st(vv[v] * gate_io));
                    }
                } else {
                    load_vec<TIn, VEC>(pa + flane, ra[s]);
                    load_vec<TIn, VEC>(pb + flane, rb[s]);
                }
            } else {
#pragma unroll
                for (int v = 0; v < VEC; ++v) { ra[s][v] = 1.0f; rb[s][v] = 0.0f; }
            }
            pa += p.D;
            pb += p.D;
            if constexpr (COUPLED) pz += p.R;
        }
    }

    // ---- level 1: serial in-lane scan; ra <- prod a, rb <- h -------------
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
        float A = 1.0f, hh = 0.0f;
#pragma unroll
        for (int s = 0; s < S; ++s) {
            hh = fmaf(ra[s][v], hh, rb[s][v]);
            A *= ra[s][v];
            ra[s][v] = A;
            rb[s][v] = hh;
        }
        s_sumA[wave][lane * VEC + v] = A;
        s_sumH[wave][lane * VEC + v] = hh;
    }
    __syncthreads();

    // ---- level 2: carry into this wave from the waves before it ---------
    float cwA[VEC], cwH[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) { cwA[v] = 1.0f; cwH[v] = 0.0f; }
#pragma unroll
    for (int w = 0; w < WT - 1; ++w) {
        if (w < wave) {
#pragma unroll
            for (int v = 0; v < VEC; ++v) {
                const float A = s_sumA[w][lane * VEC + v];
                cwH[v] = fmaf(A, cwH[v], s_sumH[w][lane * VEC + v]);
                cwA[v] *= A;
            }
        }
    }

    // ---- level 3: decoupled look-back over chunks of this feature group --
    const uint32_t tagA = make_tag(epoch, ST_AGG);
    const uint32_t tagI = make_tag(epoch, ST_INC);
    uint64_t* aggA = p.pay;
    uint64_t* aggH = p.pay + p.plane;
    uint64_t* incA = p.pay + 2 * p.plane;
    uint64_t* incH = p.pay + 3 * p.plane;
    const int64_t gbase = static_cast<int64_t>(g) * p.n_ch;   // chunk-row of this chain

    float gA = 1.0f, gH = 0.0f;   // chunk aggregate of feature `tid`
    if (tid < FW) {
#pragma unroll
        for (int w = 0; w < WT; ++w) {
            const float A = s_sumA[w][tid];
            gH = fmaf(A, gH, s_sumH[w][tid]);
            gA *= A;
        }
        const int64_t idx = (gbase + chunk) * FW + tid;
        if (chunk == 0) {
            st_relaxed(&incA[idx], pack_word(gA, tagI));
            st_relaxed(&incH[idx], pack_word(gH, tagI));
            s_inA[tid] = 1.0f;
            s_inH[tid] = 0.0f;
        } else {
            st_relaxed(&aggA[idx], pack_word(gA, tagA));
            st_relaxed(&aggH[idx], pack_word(gH, tagA));
        }
    }
    __syncthreads();
    if (tid == 0) st_relaxed(&p.flags[gbase + chunk], make_tag(epoch, chunk == 0 ? ST_INC : ST_AGG));

    if (chunk > 0) {
        float cA = 1.0f, cH = 0.0f;   // composite of folded aggregates (feature tid)
        int p_hi = chunk - 1;
        while (true) {
            if (wave == 0) {
                // Poll up to 64 predecessor flags at once (lane i <-> chunk p_hi - i).
                uint32_t spins = 0;
                while (true) {
                    const int pc = p_hi - lane;
                    uint32_t st = 0;
                    if (pc >= 0) {
                        const uint32_t w = ld_relaxed(&p.flags[gbase + pc]);
                        st = ((w >> 2) == epoch) ? (w & 3u) : 0u;
                    }
                    const uint64_t inc_m = __ballot(pc >= 0 && st == ST_INC);
                    const uint64_t nr_m = __ballot(pc >= 0 && st == 0u);
                    bool ok;
                    int nf, found;
                    if (inc_m) {
                        const int j = __ffsll(static_cast<long long>(inc_m)) - 1;
                        const uint64_t below = (j == 0) ? 0ull : ((1ull << j) - 1ull);
                        ok = (nr_m & below) == 0ull;
                        nf = j;
                        found = 1;
                    } else {
                        ok = (nr_m == 0ull);
                        nf = 64;
                        found = 0;
                    }
                    if (!ok && ++spins > MAX_SPIN) {
                        // Give up: fold whatever is there; hdr[3] marks the result invalid.
                        if (lane == 0) note_timeout(p.hdr);
                        ok = true;
                        if (!inc_m) { nf = p_hi + 1 < 64 ? p_hi + 1 : 64; found = 0; }
                        if (p_hi - nf < 0) { nf = p_hi; found = 1; }
                    }
                    if (ok) {
                        if (lane == 0) { s_nfold = nf; s_found = found; }
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
            }
            __syncthreads();
            const int nf = s_nfold;
            const int found = s_found;
            if (tid < FW) {
                // Fold aggregates of chunks p_hi, p_hi-1, ..., p_hi-nf+1 (newest first).
                constexpr int BATCH = 8;
                for (int q0 = 0; q0 < nf; q0 += BATCH) {
                    float bA[BATCH], bH[BATCH];
#pragma unroll
                    for (int q = 0; q < BATCH; ++q) {
                        if (q0 + q < nf) {
                            const int64_t idx = (gbase + p_hi - q0 - q) * FW + tid;
                            bA[q] = wait_word(&aggA[idx], tagA, p.hdr);
                            bH[q] = wait_word(&aggH[idx], tagA, p.hdr);
                        }
                    }
#pragma unroll
                    for (int q = 0; q < BATCH; ++q) {
                        if (q0 + q < nf) {
                            cH = fmaf(cA, bH[q], cH);
                            cA *= bA[q];
                        }
                    }
                }
                if (found) {
                    const int64_t idx = (gbase + p_hi - nf) * FW + tid;
                    const float iA = wait_word(&incA[idx], tagI, p.hdr);
                    const float iH = wait_word(&incH[idx], tagI, p.hdr);
                    const float inH = fmaf(cA, iH, cH);
                    const float inA = cA * iA;
                    s_inA[tid] = inA;
                    s_inH[tid] = inH;
                    const int64_t me = (gbase + chunk) * FW + tid;
                    st_relaxed(&incA[me], pack_word(gA * inA, tagI));
                    st_relaxed(&incH[me], pack_word(fmaf(gA, inH, gH), tagI));
                }
            }
            if (found) break;
            p_hi -= nf;
            __syncthreads();   // s_nfold/s_found are rewritten by the next poll
        }
        __syncthreads();
        if (tid == 0) st_relaxed(&p.flags[gbase + chunk], make_tag(epoch, ST_INC));
    } else {
        __syncthreads();
    }

    // ---- apply carry and write each output once -------------------------
    float stH[VEC], stA[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
        const float inH = s_inH[lane * VEC + v];
        const float inA = s_inA[lane * VEC + v];
        stH[v] = fmaf(cwA[v], inH, cwH[v]);
        stA[v] = cwA[v] * inA;
    }
    {
        TOut* ph = static_cast<TOut*>(p.h) + rowoff0;
        TOut* pp = PREFIX ? static_cast<TOut*>(p.aprefix) + rowoff0 : nullptr;
#pragma unroll
        for (int s = 0; s < S; ++s) {
            if (fvalid && t0 + s < p.L) {
                float o[VEC];
#pragma unroll
                for (int v = 0; v < VEC; ++v) o[v] = fmaf(ra[s][v], stH[v], rb[s][v]);
                store_vec<TOut, VEC>(ph + flane, o);
                if constexpr (PREFIX) {
#pragma unroll
                    for (int v = 0; v < VEC; ++v) o[v] = ra[s][v] * stA[v];
                    store_vec<TOut, VEC>(pp + flane, o);
                }
            }
            ph += p.D;
            if constexpr (PREFIX) pp += p.D;
        }
    }

    ws_end(p.hdr, epoch);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
namespace {

struct TileCfg { int vec, steps, waves; };

// Tile configurations compiled into the library.
constexpr TileCfg kCfgs[] = {
    {1, 32, 4}, {1, 16, 4}, {2, 16, 4}, {2, 8, 4}, {4, 8, 4}, {4, 16, 4}, {4, 4, 4},
    {1, 32, 8}, {2, 16, 8}, {4, 8, 8},
};

bool cfg_known(int vec, int steps, int waves) {
    for (const auto& c : kCfgs)
        if (c.vec == vec && c.steps == steps && c.waves == waves) return true;
    return false;
}

struct Geometry {
    int n_fg, n_ch, G;
    int64_t plane;
    size_t flags_bytes, bytes;
};

Geometry geometry(int64_t B, int64_t L, int64_t D, int vec, int steps, int waves) {
    Geometry g{};
    const int64_t FW = 64 * vec;
    const int64_t T = static_cast<int64_t>(steps) * waves;
    g.n_fg = static_cast<int>((D + FW - 1) / FW);
    g.n_ch = static_cast<int>((L + T - 1) / T);
    g.G = static_cast<int>(B * g.n_fg);
    g.plane = static_cast<int64_t>(g.G) * g.n_ch * FW;
    g.flags_bytes = round_up(static_cast<size_t>(g.G) * g.n_ch * sizeof(uint32_t), 256);
    g.bytes = WS_HDR_BYTES + g.flags_bytes + 4 * static_cast<size_t>(g.plane) * sizeof(uint64_t);
    return g;
}

template <typename TIn, typename TZ, typename TOut, int VEC, int S, int WT, bool PREFIX, bool COUPLED>
int launch_one(const DiagParams& prm, int grid, hipStream_t stream) {
    hipLaunchKernelGGL((diag_scan_kernel<TIn, TZ, TOut, VEC, S, WT, PREFIX, COUPLED>), dim3(grid),
                       dim3(64 * WT), 0, stream, prm);
    return check_launch("diag_scan_kernel");
}

template <typename TIn, typename TZ, typename TOut, bool PREFIX, bool COUPLED>
int launch_cfg(const DiagParams& prm, int grid, int vec, int steps, int waves, hipStream_t st) {
#define MOGT_DIAG_CASE(V_, S_, W_)                                                     \
    if (vec == V_ && steps == S_ && waves == W_)                                        \
        return launch_one<TIn, TZ, TOut, V_, S_, W_, PREFIX, COUPLED>(prm, grid, st);
    MOGT_DIAG_CASE(1, 32, 4)
    MOGT_DIAG_CASE(1, 16, 4)
    MOGT_DIAG_CASE(2, 16, 4)
    MOGT_DIAG_CASE(2, 8, 4)
    MOGT_DIAG_CASE(4, 8, 4)
    MOGT_DIAG_CASE(4, 16, 4)
    MOGT_DIAG_CASE(4, 4, 4)
    MOGT_DIAG_CASE(1, 32, 8)
    MOGT_DIAG_CASE(2, 16, 8)
    MOGT_DIAG_CASE(4, 8, 8)
#undef MOGT_DIAG_CASE
    return set_error(MOGT_E_INVALID, "diag scan: tile (vec=%d, steps=%d, waves=%d) not compiled", vec,
                     steps, waves);
}

// Default tile choice: the widest vector the feature count and dtype allow.
TileCfg default_cfg(int64_t D, int in_dtype, int64_t align_elems) {
    (void)in_dtype;
    if (D % 4 == 0 && align_elems % 4 == 0) return {4, 8, 4};
    if (D % 2 == 0 && align_elems % 2 == 0) return {2, 16, 4};
    return {1, 32, 4};
}

bool dtype_ok(int d) { return d == MOGT_F32 || d == MOGT_BF16; }

int64_t ptr_align_elems(const void* p, size_t esize) {
    const uintptr_t u = reinterpret_cast<uintptr_t>(p);
    int64_t e = 1;
    while (e < 4 && (u % (esize * e * 2)) == 0) e *= 2;
    return e;
}

int run_scan(const void* a, const void* b, void* h, void* aprefix, int64_t B, int64_t L,
             int64_t D, int R, int C, float damping, int in_dtype, int z_dtype, int out_dtype,
             bool coupled, int vec, int steps, int waves, void* ws, size_t ws_bytes,
             void* stream) {
    clear_error();
    if (B < 0 || L < 0 || D < 0) return set_error(MOGT_E_INVALID, "negative size");
    if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype) || !dtype_ok(z_dtype))
        return set_error(MOGT_E_INVALID, "unsupported dtype code");
    if (B == 0 || L == 0 || D == 0) return MOGT_OK;
    if (!a || !b || !h) return set_error(MOGT_E_INVALID, "null tensor pointer");
    if (!cfg_known(vec, steps, waves))
        return set_error(MOGT_E_INVALID, "diag scan: tile (%d,%d,%d) not compiled", vec, steps, waves);
    if (D % vec != 0) return set_error(MOGT_E_INVALID, "features %lld not a multiple of vec %d",
                                       (long long)D, vec);
    if (coupled && C % vec != 0)
        return set_error(MOGT_E_INVALID, "channels %d not a multiple of vec %d", C, vec);
    const Geometry geo = geometry(B, L, D, vec, steps, waves);
    if (static_cast<int64_t>(geo.G) * geo.n_ch > 0x7fffffffLL)
        return set_error(MOGT_E_INVALID, "problem too large for one launch");
    if (!ws || ws_bytes < geo.bytes)
        return set_error(MOGT_E_WORKSPACE, "workspace of %zu bytes required, got %zu", geo.bytes,
                         ws_bytes);

    DiagParams prm{};
    prm.a = a; prm.b = b; prm.h = h; prm.aprefix = aprefix;
    prm.L = L; prm.D = D;
    prm.n_fg = geo.n_fg; prm.n_ch = geo.n_ch; prm.G = geo.G;
    prm.R = R; prm.C = C; prm.damping = damping;
    char* base = static_cast<char*>(ws);
    prm.hdr = reinterpret_cast<uint32_t*>(base);
    prm.flags = reinterpret_cast<uint32_t*>(base + WS_HDR_BYTES);
    prm.pay = reinterpret_cast<uint64_t*>(base + WS_HDR_BYTES + geo.flags_bytes);
    prm.plane = geo.plane;
    const int grid = geo.G * geo.n_ch;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool pre = aprefix != nullptr;

#define MOGT_DT(TI, TZ_, TO)                                                                   \
    if (coupled) return launch_cfg<TI, TZ_, TO, false, true>(prm, grid, vec, steps, waves, st); \
    if (pre) return launch_cfg<TI, TZ_, TO, true, false>(prm, grid, vec, steps, waves, st);     \
    return launch_cfg<TI, TZ_, TO, false, false>(prm, grid, vec, steps, waves, st);

    if (coupled) {
        if (in_dtype == MOGT_BF16 && z_dtype == MOGT_F32 && out_dtype == MOGT_F32) { MOGT_DT(bf16_t, float, float) }
        if (in_dtype == MOGT_BF16 && z_dtype == MOGT_BF16 && out_dtype == MOGT_F32) { MOGT_DT(bf16_t, bf16_t, float) }
        if (in_dtype == MOGT_BF16 && z_dtype == MOGT_F32 && out_dtype == MOGT_BF16) { MOGT_DT(bf16_t, float, bf16_t) }
        if (in_dtype == MOGT_BF16 && z_dtype == MOGT_BF16 && out_dtype == MOGT_BF16) { MOGT_DT(bf16_t, bf16_t, bf16_t) }
        if (in_dtype == MOGT_F32 && z_dtype == MOGT_F32 && out_dtype == MOGT_F32) { MOGT_DT(float, float, float) }
        if (in_dtype == MOGT_F32 && z_dtype == MOGT_BF16 && out_dtype == MOGT_F32) { MOGT_DT(float, bf16_t, float) }
        if (in_dtype == MOGT_F32 && z_dtype == MOGT_F32 && out_dtype == MOGT_BF16) { MOGT_DT(float, float, bf16_t) }
        if (in_dtype == MOGT_F32 && z_dtype == MOGT_BF16 && out_dtype == MOGT_BF16) { MOGT_DT(float, bf16_t, bf16_t) }
    } else {
        if (in_dtype == MOGT_F32 && out_dtype == MOGT_F32) { MOGT_DT(float, float, float) }
        if (in_dtype == MOGT_F32 && out_dtype == MOGT_BF16) { MOGT_DT(float, float, bf16_t) }
        if (in_dtype == MOGT_BF16 && out_dtype == MOGT_F32) { MOGT_DT(bf16_t, float, float) }
        if (in_dtype == MOGT_BF16 && out_dtype == MOGT_BF16) { MOGT_DT(bf16_t, float, bf16_t) }
    }
#undef MOGT_DT
    return set_error(MOGT_E_INVALID, "unsupported dtype combination");
}

size_t esize(int dt) { return dt == MOGT_BF16 ? 2 : 4; }

}  // namespace
}  // namespace mogt

using namespace mogt;

extern "C" size_t mogt_diag_scan_workspace_bytes_cfg(int64_t batch, int64_t length,
                                                     int64_t features, int vec, int steps,
                                                     int waves) {
    if (batch <= 0 || length <= 0 || features <= 0 || vec <= 0 || steps <= 0 || waves <= 0)
        return WS_HDR_BYTES;
    return geometry(batch, length, features, vec, steps, waves).bytes;
}

extern "C" size_t mogt_diag_scan_workspace_bytes(int64_t batch, int64_t length, int64_t features,
                                                 int in_dtype) {
    // Sized for the widest default tile any pointer alignment can select.
    size_t best = 0;
    for (int v : {1, 2, 4}) {
        TileCfg c = default_cfg(features, in_dtype, v);
        size_t s = mogt_diag_scan_workspace_bytes_cfg(batch, length, features, c.vec, c.steps,
                                                      c.waves);
        if (s > best) best = s;
    }
    return best;
}

extern "C" int mogt_diag_scan_fwd_cfg(const void* a, const void* b, void* h, void* a_prefix,
                                      int64_t batch, int64_t length, int64_t features,
                                      int in_dtype, int out_dtype, int vec, int steps, int waves,
                                      void* workspace, size_t workspace_bytes, void* stream) {
    return run_scan(a, b, h, a_prefix, batch, length, features, 1, 1, 1.0f, in_dtype, MOGT_F32,
                    out_dtype, false, vec, steps, waves, workspace, workspace_bytes, stream);
}

extern "C" int mogt_diag_scan_fwd(const void* a, const void* b, void* h, void* a_prefix,
                                  int64_t batch, int64_t length, int64_t features, int in_dtype,
                                  int out_dtype, void* workspace, size_t workspace_bytes,
                                  void* stream) {
    if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) {
        clear_error();
        return set_error(MOGT_E_INVALID, "unsupported dtype code");
    }
    int64_t al = 4;
    for (const void* ptr : {a, b, static_cast<const void*>(h), static_cast<const void*>(a_prefix)}) {
        if (!ptr) continue;
        const size_t es = (ptr == a || ptr == b) ? esize(in_dtype) : esize(out_dtype);
        const int64_t e = ptr_align_elems(ptr, es);
        if (e < al) al = e;
    }
    const TileCfg c = default_cfg(features, in_dtype, al);
    return run_scan(a, b, h, a_prefix, batch, length, features, 1, 1, 1.0f, in_dtype, MOGT_F32,
                    out_dtype, false, c.vec, c.steps, c.waves, workspace, workspace_bytes, stream);
}

extern "C" size_t mogt_coupled_rank_scan_workspace_bytes(int64_t batch, int64_t length,
                                                         int64_t rank, int64_t channels,
                                                         int v_dtype) {
    return mogt_diag_scan_workspace_bytes(batch, length, rank * channels, v_dtype);
}

extern "C" int mogt_coupled_rank_scan_fwd(const void* z, const void* v, void* h, int64_t batch,
                                          int64_t length, int64_t rank, int64_t channels,
                                          float damping, int z_dtype, int v_dtype, int out_dtype,
                                          void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    if (rank <= 0 || channels <= 0 || rank > 0x7fffffff || channels > 0x7fffffff)
        return set_error(MOGT_E_INVALID, "rank and channels must be positive");
    if (!dtype_ok(z_dtype) || !dtype_ok(v_dtype) || !dtype_ok(out_dtype))
        return set_error(MOGT_E_INVALID, "unsupported dtype code");
    const int64_t D = rank * channels;
    int64_t al = 4;
    for (const void* ptr : {v, static_cast<const void*>(h)}) {
        if (!ptr) continue;
        const size_t es = (ptr == v) ? esize(v_dtype) : esize(out_dtype);
        const int64_t e = ptr_align_elems(ptr, es);
        if (e < al) al = e;
    }
    if (channels % 4 != 0) al = al < 2 ? al : 2;
    if (channels % 2 != 0) al = 1;
    const TileCfg c = default_cfg(D, v_dtype, al);
    return run_scan(z, v, h, nullptr, batch, length, D, static_cast<int>(rank),
                    static_cast<int>(channels), damping, v_dtype, z_dtype, out_dtype, true, c.vec,
                    c.steps, c.waves, workspace, workspace_bytes, stream);
}
