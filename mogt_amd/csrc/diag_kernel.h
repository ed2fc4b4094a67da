// Single-pass diagonal affine scan h_t = a_t * h_{t-1} + b_t for gfx950, shared
// by the plain per-feature scan (diag_scan.hip) and the coupled write-forget
// mixer scan (coupled_scan.hip).
//
// Semantics follow the reference's sequential recurrence (affine_scan.py:48-55,
// H_0 = 0, fp32 state, outputs cast at the end) in the per-feature R=C=1 case,
// and the coupled write-forget gate of the MOGT mixer (model_mogt.py:166-182).
//
// Design (one launch, 3 HBM streams: read a, read b, write h):
//   tile     one work-group = WT waves x 64 lanes.  A lane owns VEC consecutive
//            features (one vector load/store per row, rows contiguous along D);
//            a wave owns S consecutive steps of them; the WT waves of a group
//            cover T = WT*S consecutive steps of the same FW = 64*VEC features.
//            Chunk id = blockIdx.x, position-major over the G = B * D/FW
//            feature-group chains, so one dispatch generation covers the same
//            stretch of every chain.
//   stash    every load is issued first; the raw inputs stay in registers in
//            the most compact exact form (fp32 pairs, packed bf16 pairs, or one
//            gate value per step for the coupled mode) until the carry is known.
//   level 1  each lane scans its S steps in registers (prod a, h from 0).
//   level 2  wave summaries go through LDS; one thread per feature folds them
//            into the chunk aggregate.
//   level 3  decoupled look-back along the chain.  Every chunk owns one pair of
//            64-bit words per feature, {tag | f32 A} and {tag | f32 H}, written
//            with single atomic stores: first the aggregate (tag AGG), then,
//            in place, the inclusive prefix (tag INC).  A reader accepts a pair
//            only when both tags agree, so no fences and no separate status
//            flags are needed, and every feature resolves independently.  One
//            look-back round reads a window of NR predecessors at once (slice
//            r of the group's threads reads predecessor hi - r), folds the
//            window newest-first up to the nearest INC, and repeats only for the
//            features whose window was incomplete.
//   output   each lane composes the chunk carry with the summaries of the waves
//            before it, re-runs its S steps from that state (same order of
//            operations as the sequential recurrence) and writes every h once.
//
// Workspace reuse without clearing: the launch epoch lives in the workspace
// header; each work-group records that it has read it (one "seen" word per
// chunk) and the last work-group advances it once every chunk has, so stale
// words of earlier launches never match a newer tag and the buffer is
// zero-filled only once (this also holds inside a captured HIP graph).
#pragma once

#include <type_traits>

#include "common.h"

namespace mogt {

// MODE_DIAG_REV: the backward recurrence of MODE_DIAG, run in reverse time
// with the decay shifted by one step: h_t = a_{t+1} h_{t+1} + b_t (a_L := 0),
// i.e. G_t = dH_t + a_{t+1} G_{t+1} of affine_scan.py:65-124 for R = C = 1.
// MODE_COUPLED_REV: the same backward recurrence for MODE_COUPLED, whose decay
// a = damping * (1 - sigmoid(z)) is formed from the gate logits (per gate,
// over its C channels) instead of being read as a [B, L, D] tensor.
enum DiagMode { MODE_DIAG = 0, MODE_COUPLED = 1, MODE_DIAG_REV = 2, MODE_COUPLED_REV = 3 };

struct DiagParams {
    const void* a;      // [B, L, D] (DIAG)            | gate logits z [B, L, R] (COUPLED)
    const void* b;      // [B, L, D]                    | v [B, L, D]
    void* h;            // [B, L, D]
    void* aprefix;      // [B, L, D] or null (DIAG only)
    int64_t L, D;
    int n_fg;           // feature groups per batch row
    int n_ch;           // chunks along L
    int G;              // B * n_fg look-back chains
    int R, C;           // COUPLED: gate count and channels per gate (D = R*C)
    float damping;      // COUPLED: connection damping (identity connection scale)
    uint32_t* hdr;
    uint32_t* seen;     // [G * n_ch] per-chunk "epoch read" words
    uint64_t* pay;      // 2 planes of [G][n_ch][FW] words: A, H
    int64_t plane;      // words per plane
    float* rowstat;     // COUPLED with ROWSTAT: [B, L, n_fg] sums of squares of h
    int64_t ldv;        // COUPLED: row stride of v in elements (D, or wider inside a projection)
    int64_t ldz;        // GATED: row stride of the gate logits (R)
};

constexpr uint32_t ST_NONE = 0u;

// Sum over the lanes of one row of a chunk (FWL consecutive lanes), returned
// in every lane of the row.  A 16-lane row is one DPP row: quad swaps, then
// the half-row and row mirrors; wider rows add cross-row shuffles.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

template <int FWL>
__device__ __forceinline__ float row_lanes_sum(float v) {
    v += dpp_f32<0xB1>(v);    // quad_perm [1,0,3,2]
    v += dpp_f32<0x4E>(v);    // quad_perm [2,3,0,1]
    v += dpp_f32<0x141>(v);   // row_half_mirror
    v += dpp_f32<0x140>(v);   // row_mirror
    if constexpr (FWL >= 32) v += __shfl_xor(v, 16, 64);
    if constexpr (FWL >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

// Waves per SIMD the register allocation must leave room for.  A 768-chunk
// launch (L = 32768, D = 768 in 512-step, 64-feature chunks) of the 8-wave,
// 16-step coupled tile with bf16 v is one full generation at three
// work-groups per CU (six waves per SIMD, <= 80 VGPRs); at the unconstrained
// 96 VGPRs two fit, and the last third of the chunks runs as a second,
// half-empty generation.  The larger stashes (bf16 diagonal a and b words;
// fp32 v; row statistics) spill at that budget and measured no faster, so
// those keep the compiler's choice.
constexpr int diag_waves_per_simd(int MODE, int S, int WT, bool BF16_IN, bool ROWSTAT) {
    return (MODE == MODE_COUPLED && S == 16 && WT == 8 && BF16_IN && !ROWSTAT) ? 6 : 1;
}

template <int MODE, typename TIn, typename TZ, typename TOut, int VEC, int FWL, int S, int WT,
          bool PREFIX, bool ROWSTAT = false>
__global__ __launch_bounds__(64 * WT) __attribute__((amdgpu_waves_per_eu(diag_waves_per_simd(MODE, S, WT, std::is_same<TIn, bf16_t>::value, ROWSTAT))))
void diag_scan_kernel(DiagParams p) {
    constexpr int NT = 64 * WT;
    constexpr int Q = 64 / FWL;       // step groups per wave (rows per vector load)
    constexpr int VW = WT * Q;        // "virtual waves": groups of S consecutive steps
    constexpr int FW = FWL * VEC;     // features per chunk (chain width)
    constexpr int T = VW * S;         // steps per chunk
    constexpr int NR = NT / FW;       // look-back window (predecessors read per round)
    static_assert(64 % FWL == 0 && FWL >= 16, "a row spans 16, 32 or 64 lanes");
    constexpr bool COUPLED = MODE == MODE_COUPLED;                 // gated write v * g
    constexpr bool GATED = COUPLED || MODE == MODE_COUPLED_REV;   // decay from gate logits
    constexpr bool REV = MODE == MODE_DIAG_REV || MODE == MODE_COUPLED_REV;
    static_assert(!(PREFIX && REV), "prefix output is a forward option");
    constexpr bool BF16_IN = std::is_same<TIn, bf16_t>::value;
    // Stash (32-bit registers per step and lane): DIAG fp32 a[VEC], b[VEC];
    // DIAG bf16 raw a and b words (two values per word); COUPLED the gate logit
    // (then the gate) and the raw v words.
    static_assert(!(PREFIX && GATED), "prefix output is a DIAG-mode option");
    // ROWSTAT: per (row, feature group) sum of squares of the fp32 outputs, the
    // statistics of the RMSNorm that reads h (model_mogt.py:240), so h can
    // leave in the GEMM's dtype without a separate normalisation pass
    static_assert(!ROWSTAT || COUPLED, "row statistics are a COUPLED-mode option");

    __shared__ int s_pending[2];
    __shared__ float s_cwA[VW][FW];   // level-1 summaries, then exclusive prefixes over VW
    __shared__ float s_cwH[VW][FW];
    __shared__ float s_lbA[NR][FW];
    __shared__ float s_lbH[NR][FW];
    __shared__ uint32_t s_lbSt[NR][FW];
    __shared__ int s_hi[FW];
    __shared__ float s_inA[FW];
    __shared__ float s_inH[FW];

    const int blk = blockIdx.x;
    // Block -> (chunk position, chain).  Position-major by default.  GATED:
    // positions in groups of 8, block b of a group at position b % 8, so the
    // chains of one position share b % 8 -- one XCD under round-robin dispatch,
    // which then fetches that position's gate-logit rows once instead of once
    // per XCD.  Either way a chain's chunks have increasing block ids.
    int pos, g;
    if constexpr (GATED) {
        const int full = (p.n_ch / 8) * 8 * p.G;   // blocks of whole groups of 8 positions
        if (blk < full) {
            const int grp = blk / (8 * p.G), rem = blk - grp * 8 * p.G;
            g = rem / 8;
            pos = 8 * grp + (rem - g * 8);
        } else {
            const int rel = blk - full;
            pos = (p.n_ch / 8) * 8 + rel / p.G;
            g = rel - (rel / p.G) * p.G;
        }
    } else {
        pos = blk / p.G;
        g = blk - pos * p.G;
    }
    const int bi = g / p.n_fg;
    const int fg = g - bi * p.n_fg;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane / FWL;                  // step group of this lane inside its wave
    const int vw = wave * Q + q;
    const int flane = (lane % FWL) * VEC;      // first feature of this lane inside the chunk
    const int64_t fbase = static_cast<int64_t>(fg) * FW;
    const bool fvalid = fbase + flane < p.D;
    const int64_t tw = static_cast<int64_t>(pos) * T + static_cast<int64_t>(wave) * (Q * S);
    const int64_t t0 = tw + q * S;             // first step of this lane
    const int64_t row0 = static_cast<int64_t>(bi) * p.L;
    const int Di = static_cast<int>(p.D);      // row stride (checked on the host)
    // Memory row of logical step t: row0 + t, or row0 + L - 1 - t in reverse
    // time (REV), where rows are walked with a negative stride.
    const int64_t rbase = REV ? row0 + p.L - 1 : row0;
    const int Ds = REV ? -Di : Di;             // signed row stride
    const bool first = REV && t0 == 0;         // REV: this lane holds step 0 (a_L := 0)

    // The launch epoch is read by every lane before the data loads are issued:
    // memory counters retire in order, so waiting for it never waits for data.
    const uint32_t epoch = __builtin_amdgcn_readfirstlane(ld_relaxed(&p.hdr[2]));

    // ---- stash: issue every load before any use --------------------------
    // Loads are unconditional (rows past L and features past D read a clamped,
    // in-bounds location) and land in raw registers, so they issue back to back
    // with no wait in between; steps outside the problem are replaced by the
    // identity (a = 1, b = 0) where the values are used.
    constexpr int NWB = BF16_IN ? (VEC + 1) / 2 : VEC;   // raw 32-bit words per row of b or v
    constexpr int NA = GATED ? 1 : (BF16_IN ? NWB : VEC);
    float ra[S][NA];      // DIAG fp32: a; DIAG bf16: raw a words; GATED: raw z, then decay
    uint32_t rb[S][NWB];  // raw words of b (DIAG) or v (COUPLED)
    int nv;               // valid steps of this lane (0 .. S)
    int gi = 0;           // GATED: rank (gate index) of this lane's features
    {
        const int64_t r = p.L - t0;
        nv = !fvalid || r <= 0 ? 0 : (r >= S ? S : static_cast<int>(r));
        const int lastrel = static_cast<int>(p.L - 1 - tw);   // last row of the problem, from tw
        const int flc = fvalid ? flane : 0;
        const int64_t wbase = (rbase + (REV ? -tw : tw)) * p.D + fbase;
        // v of the forward coupled scan may sit inside a wider projection row
        const int64_t ldb = MODE == MODE_COUPLED ? p.ldv : p.D;
        const int Dsb = MODE == MODE_COUPLED ? static_cast<int>(p.ldv) : Ds;
        // REV reads a one row later in memory (a_{t+1}), except for logical
        // step 0, whose a_L does not exist: it reads row L - 1 and uses a = 0
        // (step_a); clamped rows past the end map to step 0 too when L = 1
        const TIn* pa = static_cast<const TIn*>(p.a) + wbase;
        const TIn* pb = static_cast<const TIn*>(p.b) + (rbase + (REV ? -tw : tw)) * ldb + fbase;
        const TZ* pz = nullptr;
        if constexpr (GATED) {
            // forward: the gate row of step tw + rel; REV: the row after it in
            // memory (a_{t+1}), row L - 1 for logical step 0 (decay unused)
            pz = static_cast<const TZ*>(p.a) + (REV ? rbase - tw : row0 + tw) * p.ldz;
            gi = static_cast<int>((fbase + flc) / p.C);
        }
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int rel = min(q * S + s, lastrel);
            const int off = rel * Ds + flc;
            load_raw<sizeof(TIn) * VEC>(pb + rel * Dsb + flc, rb[s]);
            if constexpr (GATED) {
                uint32_t zw[1];
                const int zrel = REV ? ((tw + rel != 0) ? 1 - rel : -rel) : rel;
                load_raw_cached<sizeof(TZ)>(pz + zrel * p.ldz + gi, zw);
                ra[s][0] = __uint_as_float(zw[0]);
            } else {
                uint32_t aw[NA];
                load_raw<sizeof(TIn) * VEC>(pa + off + ((REV && tw + rel != 0) ? Di : 0), aw);
#pragma unroll
                for (int j = 0; j < NA; ++j) ra[s][j] = __uint_as_float(aw[j]);
            }
        }
    }

    // Coupled gate, once per step when the data arrives: g = sigmoid(z),
    // a = damping * (1 - g) replaces the logit, and b = v * g (rounded to v's
    // dtype exactly where the reference's product is) replaces v in place --
    // b is exactly representable in v's dtype, so the stash keeps its size.
    // Steps outside the problem become the identity (a = 1, b = 0).  The
    // reverse mode only forms the decay (b is the incoming gradient).
    if constexpr (GATED) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const uint32_t zb = __float_as_uint(ra[s][0]);
            const float z = std::is_same<TZ, bf16_t>::value ? __uint_as_float(zb << 16) : __uint_as_float(zb);
            const bool ok = s < nv;
            const float gg = sigmoid_hw(z);
            ra[s][0] = ok ? p.damping * (1.0f - gg) : 1.0f;
            if constexpr (COUPLED) {
                // reference: V_t_raw * value_gate.to(V_t_raw.dtype), U * (1 - value_gate)
                const float g_io = IO<TIn>::ld(IO<TIn>::st(gg));
#pragma unroll
                for (int j = 0; j < NWB; ++j) {
                    uint32_t w = rb[s][j];
                    if constexpr (BF16_IN) {
                        const uint32_t lo = f32_to_bf16(__uint_as_float(w << 16) * g_io);
                        const uint32_t hi = f32_to_bf16(__uint_as_float(w & 0xffff0000u) * g_io);
                        w = lo | (hi << 16);
                    } else {
                        w = __float_as_uint(__uint_as_float(w) * g_io);
                    }
                    rb[s][j] = ok ? w : 0u;
                }
            }
        }
    }
    // bf16 element v of a raw word array (two per word, low half first).
    auto bf16_at = [](uint32_t w, int v) -> float {
        return __uint_as_float((v & 1) ? (w & 0xffff0000u) : (w << 16));
    };
    // Element accessors (fp32 values of a and b for step s, feature v).
    auto step_a = [&](int s, int v) -> float {
        if constexpr (REV) {
            if (s == 0 && first) return 0.0f;
        }
        if constexpr (GATED) return ra[s][0];
        else if constexpr (BF16_IN) return s < nv ? bf16_at(__float_as_uint(ra[s][v >> 1]), v) : 1.0f;
        else return s < nv ? ra[s][v] : 1.0f;
    };
    auto step_b = [&](int s, int v) -> float {
        if constexpr (COUPLED) return BF16_IN ? bf16_at(rb[s][v >> 1], v) : __uint_as_float(rb[s][v]);
        else if constexpr (BF16_IN) return s < nv ? bf16_at(rb[s][v >> 1], v) : 0.0f;
        else return s < nv ? __uint_as_float(rb[s][v]) : 0.0f;
    };

    // ---- level 1: in-lane summary (prod a, h from 0) of the S steps -------
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
        float A = 1.0f, hh = 0.0f;
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const float av = step_a(s, v);
            hh = fmaf(av, hh, step_b(s, v));
            A *= av;
        }
        s_cwA[vw][flane + v] = A;
        s_cwH[vw][flane + v] = hh;
    }
    if constexpr (BF16_IN || GATED) {
        // Keep only the compact stash live across the look-back: an empty asm
        // that "rewrites" it stops the compiler from holding unpacked values.
#pragma unroll
        for (int s = 0; s < S; ++s) {
#pragma unroll
            for (int j = 0; j < NWB; ++j) asm volatile("" : "+v"(rb[s][j]));
#pragma unroll
            for (int j = 0; j < NA; ++j) asm volatile("" : "+v"(ra[s][j]));
        }
    }
    if (tid == 0) { s_pending[0] = 0; s_pending[1] = 0; }
    __syncthreads();
    // Record that this work-group has read the epoch (after the data arrived,
    // so no wave waits for this store's acknowledgement before level 1).
    if (tid == 0) st_relaxed(&p.seen[blk], make_tag(epoch, ST_AGG));
    const uint32_t tagA = make_tag(epoch, ST_AGG);
    const uint32_t tagI = make_tag(epoch, ST_INC);

    // ---- level 2: per feature, exclusive prefixes over the step groups and
    // the chunk aggregate; publish the aggregate ----------------------------
    uint64_t* PA = p.pay;
    uint64_t* PH = p.pay + p.plane;
    const int64_t gbase = static_cast<int64_t>(g) * p.n_ch;
    float gA = 1.0f, gH = 0.0f;   // chunk aggregate of feature tid (tid < FW)
    if (tid < FW) {
#pragma unroll 8
        for (int w = 0; w < VW; ++w) {
            const float A = s_cwA[w][tid];
            const float H = s_cwH[w][tid];
            s_cwA[w][tid] = gA;
            s_cwH[w][tid] = gH;
            gH = fmaf(A, gH, H);
            gA *= A;
        }
        const int64_t me = (gbase + pos) * FW + tid;
        const uint32_t tg = pos == 0 ? tagI : tagA;
        st_relaxed(&PA[me], pack_word(gA, tg));
        st_relaxed(&PH[me], pack_word(gH, tg));
        s_hi[tid] = pos - 1;   // -1: nothing to look back over
        if (pos == 0) { s_inA[tid] = 1.0f; s_inH[tid] = 0.0f; }
    }

    // ---- level 3: look-back over the predecessors of this chain ----------
    if (pos > 0) {
        float cA = 1.0f, cH = 0.0f;   // composite of the folded predecessors, per feature
        const int f = tid % FW;
        const int r = tid / FW;
        uint32_t rounds = 0;
        for (int par = 0;; par ^= 1) {
            __syncthreads();   // s_hi of the previous round visible; s_pending[par] cleared
            const int hi = s_hi[f];
            if (hi >= 0 && hi - r >= 0) {
                const int64_t idx = (gbase + hi - r) * FW + f;
                const uint64_t wA = ld_relaxed(&PA[idx]);
                const uint64_t wH = ld_relaxed(&PH[idx]);
                const uint32_t ta = word_tag(wA), th = word_tag(wH);
                s_lbSt[r][f] = (ta == th && (ta == tagI || ta == tagA)) ? (ta & 3u) : ST_NONE;
                s_lbA[r][f] = word_val(wA);
                s_lbH[r][f] = word_val(wH);
            }
            if (tid == 0) s_pending[par ^ 1] = 0;
            __syncthreads();
            if (tid < FW && hi >= 0) {
                int rr = 0;
                bool done = false;
                for (; rr < NR && hi - rr >= 0; ++rr) {
                    const uint32_t st = s_lbSt[rr][tid];
                    if (st == ST_NONE) break;
                    cH = fmaf(cA, s_lbH[rr][tid], cH);
                    cA *= s_lbA[rr][tid];
                    if (st == ST_INC) { done = true; break; }
                }
                s_hi[tid] = done ? -1 : hi - rr;
                if (!done) s_pending[par] = 1;
            }
            __syncthreads();
            if (!s_pending[par]) break;
            if (++rounds > MAX_SPIN) {
                // Gave up: the carry is unknown.  Count it and poison the
                // carry, so this chunk's outputs and every later chunk of the
                // chain (which fold this chunk's published prefix) read NaN
                // instead of a silently wrong partial carry.
                if (tid == 0) note_timeout(p.hdr);
                cA = __builtin_nanf("");
                cH = __builtin_nanf("");
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (tid < FW) {
            s_inA[tid] = cA;
            s_inH[tid] = cH;
            const int64_t me = (gbase + pos) * FW + tid;
            st_relaxed(&PA[me], pack_word(gA * cA, tagI));
            st_relaxed(&PH[me], pack_word(fmaf(gA, cH, gH), tagI));
        }
    }
    __syncthreads();

    // ---- output: state entering this step group, re-run the steps, write h
    {
        float hh[VEC], Ap[VEC];
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
            const float cwA = s_cwA[vw][flane + v];
            hh[v] = fmaf(cwA, s_inH[flane + v], s_cwH[vw][flane + v]);
            Ap[v] = cwA * s_inA[flane + v];
        }
        const int64_t wbase = (rbase + (REV ? -tw : tw)) * p.D + fbase;
        // The stores walk a row pointer from this lane's first step.  Its step
        // offset comes from a value made opaque here: otherwise the compiler
        // keeps the load phase's per-step row offsets alive until these stores,
        // or spills them and reloads each one behind a wait for every store
        // issued before it.
        int qs = q * S;
        asm volatile("" : "+v"(qs));
        const int64_t roff = static_cast<int64_t>(qs) * Ds + flane;
        TOut* const ph = static_cast<TOut*>(p.h) + wbase + roff;
        TOut* const pp = PREFIX ? static_cast<TOut*>(p.aprefix) + wbase + roff : nullptr;
        // FULL: every step of every lane of the wave is in the problem (every
        // chunk but a chain's last when D is a multiple of the chunk width), so
        // the stores need no per-step lane mask
        auto emit = [&](auto full_tag) {
            constexpr bool FULL = decltype(full_tag)::value;
            TOut* rh = ph;
            TOut* rp = pp;
#pragma unroll
            for (int s = 0; s < S; ++s) {
                float o[VEC];
#pragma unroll
                for (int v = 0; v < VEC; ++v) {
                    const float av = step_a(s, v);
                    hh[v] = fmaf(av, hh[v], step_b(s, v));
                    if constexpr (PREFIX) Ap[v] *= av;
                    o[v] = hh[v];
                }
                if constexpr (ROWSTAT) {
                    // features past D hold h = 0 (identity steps); every lane of
                    // the row takes part, the row's first lane (always a valid
                    // feature) stores the group's sum
                    float sq = 0.0f;
#pragma unroll
                    for (int v = 0; v < VEC; ++v) sq = fmaf(o[v], o[v], sq);
                    sq = row_lanes_sum<FWL>(sq);
                    if ((lane % FWL) == 0 && (FULL || s < nv))
                        p.rowstat[(row0 + t0 + s) * p.n_fg + fg] = sq;
                }
                if (FULL || s < nv) {
                    store_stream<TOut, VEC>(rh, o);
                    if constexpr (PREFIX) {
#pragma unroll
                        for (int v = 0; v < VEC; ++v) o[v] = Ap[v];
                        store_stream<TOut, VEC>(rp, o);
                    }
                }
                rh += Ds;
                if constexpr (PREFIX) rp += Ds;
            }
        };
        if (__all(nv == S))
            emit(std::true_type{});
        else
            emit(std::false_type{});
    }

    // ---- last work-group: advance the epoch once every chunk has read it --
    if (blk == static_cast<int>(gridDim.x) - 1) {
        const int64_t n = static_cast<int64_t>(p.G) * p.n_ch;
        const uint32_t want = make_tag(epoch, ST_AGG);
        for (int64_t i = tid; i < n; i += NT) {
            uint32_t spins = 0;
            while (ld_relaxed(&p.seen[i]) != want) {
                if (++spins > MAX_SPIN) {
                    note_timeout(p.hdr);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        __syncthreads();
        if (tid == 0) st_relaxed(&p.hdr[2], (epoch + 1u) & 0x3fffffffu);
    }
}

// ---------------------------------------------------------------------------
// Host side: geometry and launch of one tile configuration.
// ---------------------------------------------------------------------------
struct DiagTile { int vec, lanes, steps, waves; };   // lanes per row: 64, 32 or 16

struct DiagGeometry {
    int n_fg, n_ch, G;
    int64_t plane;
    size_t seen_bytes, bytes;
};

inline DiagGeometry diag_geometry(int64_t B, int64_t L, int64_t D, const DiagTile& t) {
    DiagGeometry g{};
    const int64_t FW = static_cast<int64_t>(t.lanes) * t.vec;
    const int64_t T = static_cast<int64_t>(t.steps) * t.waves * (64 / t.lanes);
    g.n_fg = static_cast<int>((D + FW - 1) / FW);
    g.n_ch = static_cast<int>((L + T - 1) / T);
    g.G = static_cast<int>(B * g.n_fg);
    g.plane = static_cast<int64_t>(g.G) * g.n_ch * FW;
    g.seen_bytes = round_up(static_cast<size_t>(g.G) * g.n_ch * sizeof(uint32_t), 256);
    g.bytes = WS_HDR_BYTES + g.seen_bytes + 2 * static_cast<size_t>(g.plane) * sizeof(uint64_t);
    return g;
}

inline int64_t diag_groups(int64_t B, int64_t L, int64_t D, const DiagTile& t) {
    const DiagGeometry g = diag_geometry(B, L, D, t);
    return static_cast<int64_t>(g.G) * g.n_ch;
}

// First tile of a preference list (longest chunks first) with at least 128
// work-groups; else the last (shortest).  Measured at D = 768, L = 8192: 192
// long chunks (fewer than the 256 CUs) beat 768 short ones, because short
// chunks put more chunks of one chain in flight and lengthen the look-back.
// Default tile: the first of `list` whose launch has at least its minimum
// number of work-groups (else the last).  Lists and thresholds come from
// MI355X sweeps at D = 768, L = 8K / 16K / 32K.
struct TileChoice {
    DiagTile tile;
    int64_t min_groups;
};
inline DiagTile pick_tile(int64_t B, int64_t L, int64_t D, const TileChoice* list, int n) {
    for (int i = 0; i < n - 1; ++i)
        if (diag_groups(B, L, D, list[i].tile) >= list[i].min_groups) return list[i].tile;
    return list[n - 1].tile;
}

// Default fp32 tile (forward and reverse scans; measured on MI355X, B = 1,
// D = 768, L = 8k..32k): chunks of 512 steps x 64 features, rows of 256 B, two
// features per lane where the features and pointers allow.  A launch of 384
// such chunks (1.5 generations of one group per CU) runs faster as 768 chunks
// of 256 steps (L = 16k: 32.7 -> 30.7 us); a launch of fewer than 512 chunks
// (one generation, under a group per CU) runs its 512-step chunks on 16 waves
// of one feature per lane (L = 8k: 16.6 -> 16.0 us); short problems fall back
// to shorter chunks so the grid still covers the GPU.
inline DiagTile f32_tile(int64_t B, int64_t L, int64_t D, bool vec2) {
    static const TileChoice v2[] = {{{2, 32, 32, 8}, 512}, {{2, 32, 32, 4}, 512}, {{1, 64, 32, 16}, 128},
                                    {{2, 32, 16, 8}, 128}, {{2, 32, 8, 16}, 128}, {{1, 64, 8, 16}, 0}};
    static const TileChoice v1[] = {{{1, 64, 32, 16}, 128}, {{1, 64, 16, 16}, 128}, {{1, 64, 8, 16}, 0}};
    return vec2 ? pick_tile(B, L, D, v2, 6) : pick_tile(B, L, D, v1, 3);
}

// Shape checks shared by every entry point; fills prm (except tensor pointers).
inline int diag_prepare(DiagParams& prm, int64_t B, int64_t L, int64_t D, const DiagTile& t,
                        void* ws, size_t ws_bytes) {
    const DiagGeometry geo = diag_geometry(B, L, D, t);
    if (static_cast<int64_t>(geo.G) * geo.n_ch > 0x7fffffffLL ||
        D > (1LL << 31) / (static_cast<int64_t>(t.steps) * (64 / t.lanes) + 1))
        return set_error(MOGT_E_INVALID, "problem too large for one launch");
    if (!ws || ws_bytes < geo.bytes)
        return set_error(MOGT_E_WORKSPACE, "workspace of %zu bytes required, got %zu", geo.bytes,
                         ws_bytes);
    prm.L = L;
    prm.D = D;
    prm.ldv = D;
    prm.ldz = 1;
    prm.n_fg = geo.n_fg;
    prm.n_ch = geo.n_ch;
    prm.G = geo.G;
    char* base = static_cast<char*>(ws);
    prm.hdr = reinterpret_cast<uint32_t*>(base);
    prm.seen = reinterpret_cast<uint32_t*>(base + WS_HDR_BYTES);
    prm.pay = reinterpret_cast<uint64_t*>(base + WS_HDR_BYTES + geo.seen_bytes);
    prm.plane = geo.plane;
    return MOGT_OK;
}

template <int MODE, typename TIn, typename TZ, typename TOut, int VEC, int FWL, int S, int WT,
          bool PREFIX, bool ROWSTAT = false>
int diag_launch(const DiagParams& prm, hipStream_t stream) {
    const int grid = prm.G * prm.n_ch;
    hipLaunchKernelGGL((diag_scan_kernel<MODE, TIn, TZ, TOut, VEC, FWL, S, WT, PREFIX, ROWSTAT>),
                       dim3(grid), dim3(64 * WT), 0, stream, prm);
    return check_launch("diag_scan_kernel");
}

// Tile configurations compiled into the library (features per lane, lanes per
// row, steps per lane, waves per work-group), per input family.  Every tile
// keeps rows of at least 256 contiguous bytes (narrower rows cost HBM
// efficiency) and at most 64 stash registers per lane.
#define MOGT_DIAG_F32_TILES(X) X(2, 32, 32, 8) X(2, 32, 16, 16) X(2, 32, 16, 8) X(2, 32, 32, 4) X(2, 32, 8, 16) X(1, 64, 32, 16) X(1, 64, 16, 16) X(1, 64, 8, 16)
#define MOGT_DIAG_BF16_TILES(X) X(4, 16, 16, 8) X(4, 16, 16, 16) X(4, 16, 8, 8) X(4, 32, 16, 8) X(2, 32, 16, 8) X(2, 32, 16, 16) X(2, 32, 8, 16) X(1, 64, 32, 16) X(1, 64, 16, 16) X(1, 64, 8, 16)
#define MOGT_COUPLED_TILES(X) X(4, 16, 8, 16) X(4, 16, 8, 8) X(4, 16, 16, 8) X(4, 16, 16, 16) X(4, 32, 8, 16) X(2, 32, 16, 8) X(2, 32, 16, 16) X(2, 32, 8, 16) X(1, 64, 32, 16) X(1, 64, 16, 16) X(1, 64, 8, 16)
// Reverse coupled scan (fp32 dh in, G out): the fp32 reverse tiles plus four
// channels per lane (the stash is one logit and the dh words per step)
#define MOGT_COUPLED_REV_TILES(X) X(2, 32, 32, 8) X(2, 32, 32, 4) X(2, 32, 16, 8) X(2, 32, 8, 16) X(4, 16, 16, 8) X(4, 16, 8, 16) X(4, 16, 8, 8) X(1, 64, 32, 16) X(1, 64, 16, 16) X(1, 64, 8, 16)

// Per-family launchers (diag_f32.hip, diag_bf16.hip, coupled_scan.hip).
int diag_run_f32in(const DiagParams& prm, const DiagTile& t, int out_dtype, bool prefix,
                   hipStream_t stream);
int diag_run_bf16in(const DiagParams& prm, const DiagTile& t, int out_dtype, bool prefix,
                    hipStream_t stream);
bool diag_tile_compiled(int family, const DiagTile& t);   // family: 0 f32, 1 bf16, 2 coupled, 3 coupled reverse
int diag_run_rev(const DiagParams& prm, const DiagTile& t, hipStream_t stream);   // diag_rev.hip

}  // namespace mogt
