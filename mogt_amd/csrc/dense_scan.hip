// Dense affine scan H_t = U_t H_{t-1} + V_t (U_t: R x R, H/V: R x C) for gfx950.
//
// Semantics: affine_scan_sequential (affine_scan.py:14-62), fp32 state, H_0 = 0,
// optional prefix products P_t = U_t ... U_1; the chunk/carry decomposition of
// affine_scan_block_reference (affine_scan.py:175-278) and the reference's
// hybrid path (triton_scan.py:232-311), re-designed so no L x R x C
// intermediate is written and the carry is applied in registers:
//
//   K1 chunk pass    one wave per (chunk, column block, sequence).  Lane l owns
//                    one column of the augmented state [P | H] (P columns
//                    0..R-1, then up to 64-R columns of H) and runs the chunk's
//                    recurrence serially with U_t read as wave-uniform values;
//                    writes the chunk summary (P_T, H_T) -- or, for the local
//                    scan API, every step's local prefix.
//   K2 carry pass    one work-group per group of GS consecutive chunk summaries:
//                    folds its group with the whole work-group (column-owner
//                    threads, broadcast row reads from LDS), chains the groups
//                    with the decoupled look-back of common.h, then writes the
//                    exclusive carry (state before the chunk) of every chunk.
//   K3 output pass   K1's recurrence restarted from the chunk's carry; writes
//                    H_t (and P_t) once.
//
// Composition of affine elements (the reference's affine_combine,
// affine_scan.py:4-11): (P_a, H_a) o (P_b, H_b) = (P_a P_b, P_a H_b + H_a).
#include "common.h"

namespace mogt {

struct DenseParams {
    const float* U;     // [B, L, R, R] fp32
    const void* V;      // [B, L, R, C] (fp32 or bf16); null for the transport-only scan
    void* H;            // K3: [B, L, R, C] output; K1 local mode: H_prefix (fp32)
    void* P;            // K3: [B, L, R, R] prefix output or null; K1 local: U_prefix
    float* Psum;        // [B, nb, R, R]
    float* Hsum;        // [B, nb, R, C]
    float* Pcar;        // [B, nb, R, R]   state before each chunk (exclusive carry)
    float* Hcar;        // [B, nb, R, C]
    int64_t L;
    int R, C, T, nb, Cb, n_cblk;
    int GS, n_grp;      // K2 grouping
    uint32_t* hdr;
    uint32_t* flags;    // [B * n_cblk][n_grp]
    uint64_t* pay;      // 4 planes of [B * n_cblk][n_grp][R*(R+Cb)] words
    int64_t plane;
};

enum ChunkMode { CM_SUMMARY = 0, CM_LOCAL = 1, CM_OUTPUT = 2 };

// One wave: runs the recurrence of chunk `k` of sequence `b`, column block `cb`.
// EXACT: R == RMAX at compile time (unguarded loops, wide scalar loads of U_t).
template <int RMAX, bool EXACT, typename TV, typename TO, int MODE, bool PREFIX>
__global__ __launch_bounds__(64) void dense_chunk_kernel(DenseParams p, const float* __restrict__ Ug,
                                                         const TV* __restrict__ Vb, TO* __restrict__ Ho) {
    const int k = blockIdx.x;
    const int cb = blockIdx.y;
    const int b = blockIdx.z;
    const int lane = threadIdx.x;
    const int R = EXACT ? RMAX : p.R;
    const bool isP = lane < R;
    const int hc = cb * p.Cb + (lane - R);                   // H column of this lane
    const bool isH = !isP && lane - R < p.Cb && hc < p.C;
    const bool pOwner = isP && cb == 0;                       // P written by block 0 only
    const int64_t t0 = static_cast<int64_t>(k) * p.T;
    const int64_t t1 = t0 + p.T < p.L ? t0 + p.T : p.L;
    const int64_t seq = static_cast<int64_t>(b) * p.nb + k;  // summary / carry index

    float col[RMAX];
    if constexpr (MODE == CM_OUTPUT) {
#pragma unroll
        for (int i = 0; i < RMAX; ++i) {
            float x = 0.0f;
            if (i < R) {
                if (isP) x = p.Pcar[seq * R * R + i * R + lane];
                else if (isH) x = p.Hcar[(seq * R + i) * p.C + hc];
            }
            col[i] = x;
        }
    } else {
#pragma unroll
        for (int i = 0; i < RMAX; ++i) col[i] = (isP && i == lane) ? 1.0f : 0.0f;
    }

    for (int64_t t = t0; t < t1; ++t) {
        // U_t is wave-uniform: read through the scalar data cache.
        const float* __restrict__ Ut = Ug + (static_cast<int64_t>(b) * p.L + t) * R * R;
        float nw[RMAX];
#pragma unroll
        for (int i = 0; i < RMAX; ++i) {
            float acc = 0.0f;
            if (i < R && isH && Vb) acc = IO<TV>::ld(Vb[((static_cast<int64_t>(b) * p.L + t) * R + i) * p.C + hc]);
            nw[i] = acc;
        }
#pragma unroll
        for (int i = 0; i < RMAX; ++i) {
            if (i < R) {
#pragma unroll
                for (int j = 0; j < RMAX; ++j)
                    if (j < R) nw[i] = fmaf(Ut[i * R + j], col[j], nw[i]);
            }
        }
#pragma unroll
        for (int i = 0; i < RMAX; ++i) col[i] = nw[i];

        if constexpr (MODE == CM_LOCAL) {
            float* Pl = static_cast<float*>(p.P);
            float* Hl = static_cast<float*>(p.H);
#pragma unroll
            for (int i = 0; i < RMAX; ++i) {
                if (i < R) {
                    if (pOwner) Pl[((static_cast<int64_t>(b) * p.L + t) * R + i) * R + lane] = col[i];
                    else if (isH) Hl[((static_cast<int64_t>(b) * p.L + t) * R + i) * p.C + hc] = col[i];
                }
            }
        } else if constexpr (MODE == CM_OUTPUT) {
#pragma unroll
            for (int i = 0; i < RMAX; ++i) {
                if (i < R) {
                    if (isH) Ho[((static_cast<int64_t>(b) * p.L + t) * R + i) * p.C + hc] = IO<TO>::st(col[i]);
                    if constexpr (PREFIX) {
                        if (pOwner)
                            static_cast<TO*>(p.P)[((static_cast<int64_t>(b) * p.L + t) * R + i) * R + lane] =
                                IO<TO>::st(col[i]);
                    }
                }
            }
        }
    }

    if constexpr (MODE != CM_OUTPUT) {
#pragma unroll
        for (int i = 0; i < RMAX; ++i) {
            if (i < R) {
                if (pOwner) p.Psum[seq * R * R + i * R + lane] = col[i];
                else if (isH) p.Hsum[(seq * R + i) * p.C + hc] = col[i];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// K2: carries.  Affine elements live in LDS as [P | H] with row stride W = R + Wc
// (this column block only), so a composition is one R x R by R x W product.
// ---------------------------------------------------------------------------
constexpr int K2_THREADS = 512;

// out = a o b for [R][W] elements in LDS (out must not alias a or b).
// Thread <-> (column c, row slice): b's column stays in registers, the rows of
// P_a are wave-uniform (broadcast) LDS reads.
template <int RMAX>
__device__ void compose_lds(const float* a, const float* bm, float* out, int R, int W) {
    constexpr int SLICES = K2_THREADS / 64;
    const int c = threadIdx.x & 63;
    const int sl = threadIdx.x >> 6;
    if (c < W) {
        float bc[RMAX];
#pragma unroll
        for (int kk = 0; kk < RMAX; ++kk) bc[kk] = kk < R ? bm[kk * W + c] : 0.0f;
        for (int i = sl; i < R; i += SLICES) {
            float acc = c >= R ? a[i * W + c] : 0.0f;   // + H_a on H columns
#pragma unroll
            for (int kk = 0; kk < RMAX; ++kk)
                if (kk < R) acc = fmaf(a[i * W + kk], bc[kk], acc);
            out[i * W + c] = acc;
        }
    }
}

template <int RMAX>
__global__ __launch_bounds__(K2_THREADS) void dense_carry_kernel(DenseParams p) {
    constexpr int EMAX = RMAX * 64;   // max R * W (R + Cb <= 64)
    __shared__ float s_buf[4][EMAX];
    __shared__ uint32_t s_epoch;
    __shared__ int s_nfold, s_found;

    const uint32_t epoch = ws_epoch(p.hdr, &s_epoch);
    const int grp = blockIdx.x;
    const int cb = blockIdx.y;
    const int b = blockIdx.z;
    const int R = p.R;
    const int c0 = cb * p.Cb;
    const int Wc = (p.C - c0) < p.Cb ? (p.C - c0) : p.Cb;    // H columns of this block
    const int W = R + Wc;
    const int E = R * W;
    const int k0 = grp * p.GS;
    const int k1 = (k0 + p.GS) < p.nb ? (k0 + p.GS) : p.nb;
    const int tid = threadIdx.x;

    float* grpc = s_buf[0];   // composite of this group's summaries
    float* acc = s_buf[1];    // running composite / state
    float* elt = s_buf[2];    // element being folded in
    float* tmp = s_buf[3];

    auto load_summary = [&](int k, float* dst) {
        const int64_t seq = static_cast<int64_t>(b) * p.nb + k;
        for (int e = tid; e < E; e += K2_THREADS) {
            const int i = e / W, j = e - i * W;
            dst[e] = j < R ? p.Psum[seq * R * R + i * R + j]
                           : p.Hsum[(seq * R + i) * p.C + c0 + (j - R)];
        }
    };
    auto set_identity = [&](float* dst) {
        for (int e = tid; e < E; e += K2_THREADS) {
            const int i = e / W, j = e - i * W;
            dst[e] = (j == i) ? 1.0f : 0.0f;
        }
    };
    auto swap = [](float*& x, float*& y) { float* t = x; x = y; y = t; };

    // 1. composite of this group's chunk summaries: S_{k1-1} o ... o S_{k0}.
    load_summary(k0, grpc);
    __syncthreads();
    for (int k = k0 + 1; k < k1; ++k) {
        load_summary(k, elt);
        __syncthreads();
        compose_lds<RMAX>(elt, grpc, tmp, R, W);
        __syncthreads();
        swap(grpc, tmp);
    }

    // 2. decoupled look-back over the groups of this (sequence, column block)
    //    chain; `acc` ends as the inclusive prefix before this group (carry-in).
    const uint32_t tagA = make_tag(epoch, ST_AGG);
    const uint32_t tagI = make_tag(epoch, ST_INC);
    const int64_t chain = static_cast<int64_t>(b) * p.n_cblk + cb;
    const int64_t EW = static_cast<int64_t>(R) * (R + p.Cb);   // words per group slot
    uint64_t* aggW = p.pay;
    uint64_t* incW = p.pay + p.plane;
    uint32_t* flg = p.flags + chain * p.n_grp;
    auto slot = [&](int g) { return (chain * p.n_grp + g) * EW; };

    set_identity(acc);
    if (grp == 0) {
        for (int e = tid; e < E; e += K2_THREADS) st_relaxed(&incW[slot(0) + e], pack_word(grpc[e], tagI));
        __syncthreads();
        if (tid == 0) st_relaxed(&flg[0], make_tag(epoch, ST_INC));
    } else {
        for (int e = tid; e < E; e += K2_THREADS) st_relaxed(&aggW[slot(grp) + e], pack_word(grpc[e], tagA));
        __syncthreads();
        if (tid == 0) st_relaxed(&flg[grp], make_tag(epoch, ST_AGG));
        int p_hi = grp - 1;
        while (true) {
            if (tid < 64) {
                uint32_t spins = 0;
                while (true) {
                    const int pc = p_hi - tid;
                    uint32_t st = 0;
                    if (pc >= 0) {
                        const uint32_t w = ld_relaxed(&flg[pc]);
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
                        ok = nr_m == 0ull;
                        nf = 64;
                        found = 0;
                    }
                    if (!ok && ++spins > MAX_SPIN) {
                        if (tid == 0) note_timeout(p.hdr);
                        ok = true;
                        if (!inc_m) { nf = p_hi + 1 < 64 ? p_hi + 1 : 64; found = 0; }
                        if (p_hi - nf < 0) { nf = p_hi; found = 1; }
                    }
                    if (ok) {
                        if (tid == 0) { s_nfold = nf; s_found = found; }
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
            }
            __syncthreads();
            const int nf = s_nfold;
            const int found = s_found;
            // acc <- acc o agg_{p_hi} o agg_{p_hi-1} o ... (newest first)
            for (int q = 0; q < nf; ++q) {
                const int64_t base = slot(p_hi - q);
                for (int e = tid; e < E; e += K2_THREADS) elt[e] = wait_word(&aggW[base + e], tagA, p.hdr);
                __syncthreads();
                compose_lds<RMAX>(acc, elt, tmp, R, W);
                __syncthreads();
                swap(acc, tmp);
            }
            if (found) {
                const int64_t base = slot(p_hi - nf);
                for (int e = tid; e < E; e += K2_THREADS) elt[e] = wait_word(&incW[base + e], tagI, p.hdr);
                __syncthreads();
                compose_lds<RMAX>(acc, elt, tmp, R, W);
                __syncthreads();
                swap(acc, tmp);
                break;
            }
            p_hi -= nf;
            __syncthreads();
        }
        // publish this group's inclusive prefix: grpc o acc
        compose_lds<RMAX>(grpc, acc, tmp, R, W);
        __syncthreads();
        for (int e = tid; e < E; e += K2_THREADS) st_relaxed(&incW[slot(grp) + e], pack_word(tmp[e], tagI));
        __syncthreads();
        if (tid == 0) st_relaxed(&flg[grp], make_tag(epoch, ST_INC));
    }

    // 3. exclusive carry of every chunk of the group: state before chunk k.
    for (int k = k0; k < k1; ++k) {
        const int64_t seq = static_cast<int64_t>(b) * p.nb + k;
        for (int e = tid; e < E; e += K2_THREADS) {
            const int i = e / W, j = e - i * W;
            if (j < R) {
                if (cb == 0) p.Pcar[seq * R * R + i * R + j] = acc[e];
            } else {
                p.Hcar[(seq * R + i) * p.C + c0 + (j - R)] = acc[e];
            }
        }
        if (k + 1 < k1) {
            load_summary(k, elt);
            __syncthreads();
            compose_lds<RMAX>(elt, acc, tmp, R, W);
            __syncthreads();
            swap(acc, tmp);
        }
    }

    ws_finish(p.hdr, p.flags, static_cast<int64_t>(gridDim.y) * gridDim.z * p.n_grp, epoch);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
namespace {

struct DenseGeo {
    int T, nb, Cb, n_cblk, GS, n_grp, rmax;
    size_t off_psum, off_hsum, off_pcar, off_hcar, off_flags, off_pay, bytes;
    int64_t plane;
};

int rmax_for(int R) {
    if (R <= 4) return 4;
    if (R <= 8) return 8;
    if (R <= 16) return 16;
    if (R <= 32) return 32;
    return 0;
}

DenseGeo dense_geometry(int64_t B, int64_t L, int R, int64_t C, int T) {
    DenseGeo g{};
    g.T = T;
    g.nb = static_cast<int>((L + T - 1) / T);
    g.rmax = rmax_for(R);
    const int room = 64 - R;                       // H columns per wave
    g.Cb = C == 0 ? 0 : static_cast<int>(C < room ? C : room);
    g.n_cblk = C == 0 ? 1 : static_cast<int>((C + g.Cb - 1) / g.Cb);
    g.GS = g.nb <= 64 ? 1 : (g.nb + 63) / 64;
    g.n_grp = (g.nb + g.GS - 1) / g.GS;
    size_t off = WS_HDR_BYTES;
    auto take = [&](size_t n) { size_t o = off; off = round_up(off + n, 256); return o; };
    const size_t nb = static_cast<size_t>(B) * g.nb;
    g.off_psum = take(nb * R * R * sizeof(float));
    g.off_hsum = take(nb * R * static_cast<size_t>(C) * sizeof(float));
    g.off_pcar = take(nb * R * R * sizeof(float));
    g.off_hcar = take(nb * R * static_cast<size_t>(C) * sizeof(float));
    const size_t chains = static_cast<size_t>(B) * g.n_cblk;
    g.off_flags = take(chains * g.n_grp * sizeof(uint32_t));
    g.plane = static_cast<int64_t>(chains) * g.n_grp * R * (R + g.Cb);
    g.off_pay = take(2 * static_cast<size_t>(g.plane) * sizeof(uint64_t));
    g.bytes = off;
    return g;
}

// Chunk length: short chunks give parallelism along L; the serial work per
// step is R*(R+64) FMAs per lane.
int default_chunk(int64_t B, int64_t L, int R) {
    (void)B;
    (void)R;
    return L >= 4096 ? 32 : 16;
}

template <int RMAX, typename TV, typename TO, int MODE, bool PREFIX>
int launch_chunk(const DenseParams& prm, int64_t B, hipStream_t st) {
    if (prm.R == RMAX) {
        hipLaunchKernelGGL((dense_chunk_kernel<RMAX, true, TV, TO, MODE, PREFIX>),
                           dim3(prm.nb, prm.n_cblk, static_cast<unsigned>(B)), dim3(64), 0, st, prm,
                           prm.U, static_cast<const TV*>(prm.V), static_cast<TO*>(prm.H));
        return check_launch("dense_chunk_kernel");
    }
    hipLaunchKernelGGL((dense_chunk_kernel<RMAX, false, TV, TO, MODE, PREFIX>),
                       dim3(prm.nb, prm.n_cblk, static_cast<unsigned>(B)), dim3(64), 0, st, prm,
                       prm.U, static_cast<const TV*>(prm.V), static_cast<TO*>(prm.H));
    return check_launch("dense_chunk_kernel");
}

template <int RMAX>
int launch_carry(const DenseParams& prm, int64_t B, hipStream_t st) {
    hipLaunchKernelGGL((dense_carry_kernel<RMAX>), dim3(prm.n_grp, prm.n_cblk, static_cast<unsigned>(B)),
                       dim3(K2_THREADS), 0, st, prm);
    return check_launch("dense_carry_kernel");
}

template <int RMAX, typename TV, typename TO>
int run_dense_t(DenseParams prm, int64_t B, bool prefix, hipStream_t st) {
    int rc = launch_chunk<RMAX, TV, TO, CM_SUMMARY, false>(prm, B, st);
    if (rc) return rc;
    rc = launch_carry<RMAX>(prm, B, st);
    if (rc) return rc;
    if (prefix) return launch_chunk<RMAX, TV, TO, CM_OUTPUT, true>(prm, B, st);
    return launch_chunk<RMAX, TV, TO, CM_OUTPUT, false>(prm, B, st);
}

template <typename TV, typename TO>
int run_dense_r(const DenseParams& prm, int64_t B, bool prefix, int rmax, hipStream_t st) {
    switch (rmax) {
        case 4: return run_dense_t<4, TV, TO>(prm, B, prefix, st);
        case 8: return run_dense_t<8, TV, TO>(prm, B, prefix, st);
        case 16: return run_dense_t<16, TV, TO>(prm, B, prefix, st);
        case 32: return run_dense_t<32, TV, TO>(prm, B, prefix, st);
        default: return set_error(MOGT_E_INVALID, "R must be <= 32");
    }
}

int check_dense_shapes(int64_t B, int64_t L, int64_t R, int64_t C) {
    if (B < 0 || L < 0 || R <= 0 || C < 0)
        return set_error(MOGT_E_INVALID, "U must be [B, L, R, R] and V must be [B, L, R, C]");
    if (R > 32) return set_error(MOGT_E_INVALID, "R = %lld not supported (R <= 32)", (long long)R);
    if (C > (1 << 24)) return set_error(MOGT_E_INVALID, "C too large");
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
    const int T = default_chunk(B, L, static_cast<int>(R));
    const DenseGeo g = dense_geometry(B, L, static_cast<int>(R), C, T);
    if (!ws || ws_bytes < g.bytes)
        return set_error(MOGT_E_WORKSPACE, "workspace of %zu bytes required, got %zu", g.bytes, ws_bytes);
    if (static_cast<int64_t>(g.nb) > 0x7fffffffLL || B > 65535)
        return set_error(MOGT_E_INVALID, "problem too large for one launch");
    char* base = static_cast<char*>(ws);
    DenseParams prm{};
    prm.U = U; prm.V = C > 0 ? V : nullptr; prm.H = H; prm.P = P;
    prm.Psum = reinterpret_cast<float*>(base + g.off_psum);
    prm.Hsum = reinterpret_cast<float*>(base + g.off_hsum);
    prm.Pcar = reinterpret_cast<float*>(base + g.off_pcar);
    prm.Hcar = reinterpret_cast<float*>(base + g.off_hcar);
    prm.L = L; prm.R = static_cast<int>(R); prm.C = static_cast<int>(C); prm.T = T; prm.nb = g.nb;
    prm.Cb = g.Cb; prm.n_cblk = g.n_cblk; prm.GS = g.GS; prm.n_grp = g.n_grp;
    prm.hdr = reinterpret_cast<uint32_t*>(base);
    prm.flags = reinterpret_cast<uint32_t*>(base + g.off_flags);
    prm.pay = reinterpret_cast<uint64_t*>(base + g.off_pay);
    prm.plane = g.plane;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool prefix = P != nullptr;
    if (v_dtype == MOGT_F32 && out_dtype == MOGT_F32) return run_dense_r<float, float>(prm, B, prefix, g.rmax, st);
    if (v_dtype == MOGT_F32 && out_dtype == MOGT_BF16) return run_dense_r<float, bf16_t>(prm, B, prefix, g.rmax, st);
    if (v_dtype == MOGT_BF16 && out_dtype == MOGT_F32) return run_dense_r<bf16_t, float>(prm, B, prefix, g.rmax, st);
    return run_dense_r<bf16_t, bf16_t>(prm, B, prefix, g.rmax, st);
}

template <int RMAX, typename TV>
int launch_local(const DenseParams& prm, int64_t B, hipStream_t st) {
    return launch_chunk<RMAX, TV, float, CM_LOCAL, false>(prm, B, st);
}

}  // namespace
}  // namespace mogt

using namespace mogt;

extern "C" size_t mogt_affine_scan_workspace_bytes(int64_t batch, int64_t length, int64_t rank,
                                                   int64_t channels) {
    if (batch <= 0 || length <= 0 || rank <= 0 || rank > 32 || channels < 0) return WS_HDR_BYTES;
    const int T = default_chunk(batch, length, static_cast<int>(rank));
    return dense_geometry(batch, length, static_cast<int>(rank), channels, T).bytes;
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
    const DenseGeo g = dense_geometry(batch, length, static_cast<int>(rank), channels,
                                      static_cast<int>(block_size));
    DenseParams prm{};
    prm.U = static_cast<const float*>(U);
    prm.V = channels > 0 ? V : nullptr;
    prm.H = H_prefix; prm.P = U_prefix;
    prm.Psum = static_cast<float*>(U_summary);
    prm.Hsum = static_cast<float*>(H_summary);
    prm.L = length; prm.R = static_cast<int>(rank); prm.C = static_cast<int>(channels);
    prm.T = static_cast<int>(block_size); prm.nb = static_cast<int>(nb);
    prm.Cb = g.Cb; prm.n_cblk = g.n_cblk;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool bf = v_dtype == MOGT_BF16;
    switch (g.rmax) {
        case 4: return bf ? launch_local<4, bf16_t>(prm, batch, st) : launch_local<4, float>(prm, batch, st);
        case 8: return bf ? launch_local<8, bf16_t>(prm, batch, st) : launch_local<8, float>(prm, batch, st);
        case 16: return bf ? launch_local<16, bf16_t>(prm, batch, st) : launch_local<16, float>(prm, batch, st);
        case 32: return bf ? launch_local<32, bf16_t>(prm, batch, st) : launch_local<32, float>(prm, batch, st);
        default: return set_error(MOGT_E_INVALID, "R must be <= 32");
    }
}
