// Generic dense affine scan  M_t = U_t M_{t-1} + [V_t | 0]  for any rank R <= 1024 and any
// number of channels, with the state carried in fp32 or fp64 (the reference scans'
// state_dtype argument, affine_scan.py:14-62, :127-172, :175-278).
//
// The MFMA pipeline of dense_scan.hip covers the model's shapes (R <= 32, fp32 state).
// This kernel covers everything else the reference's functions accept: a float64 state
// (the reference's own sanity check runs in float64, sanity_affine_scan.py:19-61), ranks
// above 32, fp16 / fp64 inputs and outputs.  It is a latency-bound scalar kernel, not a
// matrix-core one: every state element is one thread's running dot product over the R
// rows of the previous state, with the state in LDS.
//
// The prefix product U_prefix_t = U_t ... U_1 (return_prefix=True, affine_scan.py:43-55)
// is the same recurrence applied to R extra state columns that start at the identity and
// take no input, so one augmented state [H | U_prefix] of width C + R serves both.
//
// Three passes over chunks of `seg` steps (seg ~ sqrt(L)):
//   LOCAL   per chunk, from [0 | I]: the chunk's end state [E_j | P_j] (E_j: the
//           chunk's own contribution, P_j: the product of its transitions);
//   CARRY   per batch row, sequentially over chunks: M_in(j+1) = P_j M_in(j) + [E_j | 0],
//           M_in(0) = [0 | I] (the carry recursion of affine_scan.py:175-278);
//   OUTPUT  per chunk, from M_in(j): every step's state, written as H and U_prefix.
// One pass (OUTPUT from [0 | I]) when the whole sequence is one chunk.
//
// Reverse mode (the backward's total-gradient recursion, affine_scan.py:110-118):
// G_t = X_t + U_{t+1}^T G_{t+1}: position q of the scan is time L-1-q, its transition is
// U_{L-q}^T (the identity at q = 0, where the state is still zero).
#include "common.h"

namespace mogt {
namespace {

constexpr int GS_THREADS = 256;
constexpr int GS_EPT = 4;                          // state elements per thread
constexpr int GS_MAX_ELEMS = GS_THREADS * GS_EPT;  // R * column-tile width
constexpr int GS_MAX_R = 1024;
constexpr int GS_ULDS_MAX_R = 64;                  // transitions staged in LDS up to this rank

// A [batch][sequence][rows][cols] view of a device buffer (strides in elements).
struct GView {
    void* p;
    int64_t bs, ss, rs;
    int code;
};

struct GParams {
    GView tr;        // transitions, state dtype; column offset tr_c0
    GView in;        // inputs, columns [0, cin)
    GView init;      // initial state per (batch, chunk), state dtype; p == nullptr: [0 | I]
    GView out_h;     // state columns [0, csplit)
    GView out_p;     // state columns [csplit, W), written at column c - csplit (p may be null)
    int64_t L;       // positions in the scanned sequence
    int64_t seg;     // positions per chunk (one work-group's run)
    int nseg, ntile;
    int R, W, Cb;    // rank, state width, column-tile width
    int tr_c0, cin, cid, csplit;  // cid: first identity column of the [0 | I] start
    int every;       // 1: write the state after every step; 0: the final state at the chunk index
    int shift;       // 1: step q is written at index q + 1 and the initial state at index 0
    int rev;         // reverse, transposed transitions (see the file comment)
};

__device__ __forceinline__ int64_t at(const GView& v, int64_t b, int64_t s, int64_t r, int64_t c) {
    return b * v.bs + s * v.ss + r * v.rs + c;
}

template <typename TS>
__device__ __forceinline__ TS ld_code(const void* p, int64_t i, int code) {
    if (code == MOGT_F64) return static_cast<TS>(static_cast<const double*>(p)[i]);
    if (code == MOGT_BF16) return static_cast<TS>(bf16_to_f32(static_cast<const bf16_t*>(p)[i]));
    if (code == MOGT_F16) return static_cast<TS>(static_cast<float>(static_cast<const _Float16*>(p)[i]));
    return static_cast<TS>(static_cast<const float*>(p)[i]);
}

// Narrow outputs round from the state through fp32 (round to nearest even at each step),
// as a torch float64 -> bfloat16 / float16 conversion does.
template <typename TS>
__device__ __forceinline__ void st_code(void* p, int64_t i, int code, TS x) {
    if (code == MOGT_F64) {
        static_cast<double*>(p)[i] = static_cast<double>(x);
        return;
    }
    const float f = static_cast<float>(x);
    if (code == MOGT_BF16) static_cast<bf16_t*>(p)[i] = f32_to_bf16(f);
    else if (code == MOGT_F16) static_cast<_Float16*>(p)[i] = static_cast<_Float16>(f);
    else static_cast<float*>(p)[i] = f;
}

template <typename TS>
__device__ __forceinline__ void put(const GParams& p, int64_t b, int64_t idx, int i, int c, TS x) {
    if (c < p.csplit) {
        st_code<TS>(p.out_h.p, at(p.out_h, b, idx, i, c), p.out_h.code, x);
    } else if (p.out_p.p) {
        st_code<TS>(p.out_p.p, at(p.out_p, b, idx, i, c - p.csplit), p.out_p.code, x);
    }
}

// Row length in LDS of the staged transition and of a state column: R rounded
// up to 16 bytes, plus 16 bytes of skew between rows.
template <typename TS>
__host__ __device__ constexpr int gs_ld(int R) {
    return (R + static_cast<int>(16 / sizeof(TS)) - 1) / static_cast<int>(16 / sizeof(TS)) *
               static_cast<int>(16 / sizeof(TS)) + static_cast<int>(16 / sizeof(TS));
}

// ULDS: the step's transition staged through LDS (R <= 64), UPT of its values
// per thread; PD: steps of operands in flight.
template <typename TS, bool ULDS, int UPT, int PD, int RM = 0>
__global__ __launch_bounds__(GS_THREADS, sizeof(TS) == 4 ? 3 : 2) void generic_scan_kernel(GParams p) {
    extern __shared__ __align__(16) unsigned char gs_smem[];
    // LDS: the step's transition U [R][ld] (staged variant) then two state
    // buffers stored column-major, [Cb][ld]; ld = R rounded up to 16 bytes plus
    // 16 bytes of skew, so a thread reads 16 bytes of a U row or of its state
    // column per instruction.  Padding columns / rows stay zero.
    constexpr int VE = 16 / sizeof(TS);
    const int R = p.R, Cb = p.Cb, RCb = R * Cb;
    const int ld = gs_ld<TS>(R);
    TS* sU = reinterpret_cast<TS*>(gs_smem);
    TS* sS = sU + (ULDS ? R * ld : 0);
    const int lds_elems = (ULDS ? R * ld : 0) + 2 * Cb * ld;
    for (int e = threadIdx.x; e < lds_elems; e += GS_THREADS) sU[e] = TS(0);
    __syncthreads();

    const int tid = threadIdx.x;
    int64_t blk = blockIdx.x;
    const int ct = static_cast<int>(blk % p.ntile);
    blk /= p.ntile;
    const int j = static_cast<int>(blk % p.nseg);
    const int64_t b = blk / p.nseg;
    const int64_t q0 = static_cast<int64_t>(j) * p.seg;
    const int64_t n = min(p.seg, p.L - q0);

    int oi[GS_EPT], ocl[GS_EPT], oc[GS_EPT];
    bool own[GS_EPT], ok[GS_EPT];
#pragma unroll
    for (int m = 0; m < GS_EPT; ++m) {
        const int e = tid + m * GS_THREADS;
        own[m] = e < RCb;
        oi[m] = own[m] ? e / Cb : 0;
        ocl[m] = own[m] ? e - oi[m] * Cb : 0;
        oc[m] = ct * Cb + ocl[m];
        ok[m] = own[m] && oc[m] < p.W;
    }

    // initial state (columns past W stay zero and are never written out)
    TS acc[GS_EPT];
#pragma unroll
    for (int m = 0; m < GS_EPT; ++m) {
        TS v0 = TS(0);
        if (ok[m]) {
            if (p.init.p) v0 = ld_code<TS>(p.init.p, at(p.init, b, j, oi[m], oc[m]), p.init.code);
            else if (oc[m] >= p.cid) v0 = (oi[m] == oc[m] - p.cid) ? TS(1) : TS(0);
            if (p.shift) put<TS>(p, b, 0, oi[m], oc[m], v0);
        }
        acc[m] = v0;
        if (own[m]) sS[ocl[m] * ld + oi[m]] = v0;
    }

    // Operands of the next PD steps are in flight: slot pp of the ring holds
    // step s0 + pp of the current round and is refilled with step s0 + pp + PD
    // once its values have been consumed.
    TS ureg[PD][ULDS ? UPT : 1];
    TS vreg[PD][GS_EPT];
    auto fetch = [&](int64_t q, TS (&u)[ULDS ? UPT : 1], TS (&v)[GS_EPT]) {
        if constexpr (ULDS) {
            const bool ident = p.rev && q == 0;
            const int64_t tt = p.rev ? p.L - q : q;
#pragma unroll
            for (int m = 0; m < UPT; ++m) {
                const int idx = tid + m * GS_THREADS;
                if (idx < R * R) {
                    const int rr = idx / R, cc = idx - rr * R;
                    u[m] = ident ? TS(rr == cc ? 1 : 0)
                                 : static_cast<const TS*>(p.tr.p)[at(p.tr, b, tt, rr, p.tr_c0 + cc)];
                }
            }
        }
        const int64_t ti = p.rev ? p.L - 1 - q : q;
#pragma unroll
        for (int m = 0; m < GS_EPT; ++m)
            v[m] = (ok[m] && oc[m] < p.cin) ? ld_code<TS>(p.in.p, at(p.in, b, ti, oi[m], oc[m]), p.in.code)
                                            : TS(0);
    };

#pragma unroll
    for (int pp = 0; pp < PD; ++pp)
        if (pp < n) fetch(q0 + pp, ureg[pp], vreg[pp]);
    __syncthreads();
    int cur = 0;
    // one step: slot (u, v) holds step s; refilled with step s + PD
    auto step = [&](int64_t s, TS (&u)[ULDS ? UPT : 1], TS (&v)[GS_EPT]) {
        const int64_t q = q0 + s;
        if constexpr (ULDS) {
#pragma unroll
            for (int m = 0; m < UPT; ++m) {
                const int idx = tid + m * GS_THREADS;
                if (idx < R * R) {
                    const int rr = idx / R, cc = idx - rr * R;
                    // stored as the transition itself: row i, column k
                    if (p.rev) sU[cc * ld + rr] = u[m];
                    else sU[rr * ld + cc] = u[m];
                }
            }
        }
        TS vin[GS_EPT];
#pragma unroll
        for (int m = 0; m < GS_EPT; ++m) vin[m] = v[m];
        if (s + PD < n) fetch(q + PD, u, v);   // later steps' loads overlap this step's arithmetic
        if constexpr (ULDS) __syncthreads();

        const TS* Sc = sS + cur * Cb * ld;
        TS* Sn = sS + (cur ^ 1) * Cb * ld;
        const bool ident = p.rev && q == 0;
        const int64_t tt = p.rev ? p.L - q : q;
        const int64_t tout = (p.rev ? p.L - 1 - q : q) + p.shift;
        // every element a thread owns sits in one column (the tile width
        // divides the thread count), so each state value read serves all
        const TS* scol = Sc + ocl[0] * ld;
        TS a[GS_EPT];
#pragma unroll
        for (int m = 0; m < GS_EPT; ++m) a[m] = vin[m];
        if (ident) {
#pragma unroll
            for (int m = 0; m < GS_EPT; ++m) a[m] += scol[oi[m]];
        } else if constexpr (ULDS) {
            typedef TS vec_t __attribute__((ext_vector_type(VE)));
            auto kstep = [&](int k) {
                const vec_t sv = *reinterpret_cast<const vec_t*>(scol + k);
#pragma unroll
                for (int m = 0; m < GS_EPT; ++m) {
                    const vec_t uv = *reinterpret_cast<const vec_t*>(sU + oi[m] * ld + k);
#pragma unroll
                    for (int e = 0; e < VE; ++e) a[m] += uv[e] * sv[e];
                }
            };
            if constexpr (RM > 0) {
                // rank bounded at compile time: the whole contraction unrolled,
                // its LDS reads issued together
#pragma unroll
                for (int k = 0; k < RM; k += VE)
                    if (k < R) kstep(k);
            } else {
#pragma unroll 2
                for (int k = 0; k < R; k += VE) kstep(k);
            }
        } else {
            const TS* ut = static_cast<const TS*>(p.tr.p);
            for (int k = 0; k < R; ++k) {
                const TS sv = scol[k];
#pragma unroll
                for (int m = 0; m < GS_EPT; ++m) {
                    const int64_t ui = p.rev ? at(p.tr, b, tt, k, p.tr_c0 + oi[m]) : at(p.tr, b, tt, oi[m], p.tr_c0 + k);
                    a[m] += ut[ui] * sv;
                }
            }
        }
#pragma unroll
        for (int m = 0; m < GS_EPT; ++m) {
            if (!own[m]) continue;
            if (!ok[m]) a[m] = TS(0);
            else if (p.every) put<TS>(p, b, tout, oi[m], oc[m], a[m]);
            acc[m] = a[m];
            Sn[ocl[m] * ld + oi[m]] = a[m];
        }
        __syncthreads();
        cur ^= 1;
    };
    if constexpr (PD == 1) {
        for (int64_t s = 0; s < n; ++s) step(s, ureg[0], vreg[0]);
    } else {
        for (int64_t s0 = 0; s0 < n; s0 += PD) {
#pragma unroll
            for (int pp = 0; pp < PD; ++pp) {
                if (s0 + pp >= n) break;   // uniform over the work-group
                step(s0 + pp, ureg[pp], vreg[pp]);
            }
        }
    }
    if (!p.every) {
#pragma unroll
        for (int m = 0; m < GS_EPT; ++m)
            if (ok[m]) put<TS>(p, b, j, oi[m], oc[m], acc[m]);
    }
}

struct GGeo {
    int64_t seg, nch;
    int Wl, Wo;          // LOCAL state width (C + R), OUTPUT / CARRY width (C + R if prefix)
    size_t s_off, m_off, bytes;
};

size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

GGeo generic_geometry(int64_t B, int64_t L, int64_t R, int64_t C, int with_prefix, int state_code) {
    GGeo g{};
    g.seg = 16;
    while (g.seg * g.seg < L && g.seg < 1024) g.seg *= 2;
    g.nch = (L + g.seg - 1) / g.seg;
    g.Wl = static_cast<int>(C + R);
    g.Wo = static_cast<int>(C + (with_prefix ? R : 0));
    const size_t ts = state_code == MOGT_F64 ? 8 : 4;
    g.s_off = 0;
    g.m_off = 0;
    g.bytes = WS_HDR_BYTES;
    if (g.nch > 1) {
        g.s_off = WS_HDR_BYTES;
        g.m_off = g.s_off + align256(static_cast<size_t>(B * g.nch * R * g.Wl) * ts);
        g.bytes = g.m_off + align256(static_cast<size_t>(B * g.nch * R * g.Wo) * ts);
    }
    return g;
}

int tile_width(int R, int W) {
    int cap = 1;   // a power of two dividing the thread count (one column per thread)
    while (cap * 2 * R <= GS_MAX_ELEMS && cap < GS_THREADS) cap *= 2;
    int cb = 1;
    while (cb < W && cb < cap) cb *= 2;
    return cb;
}

template <typename TS>
int launch_generic(GParams p, int64_t batch, hipStream_t st, const char* what) {
    p.Cb = tile_width(p.R, p.W);
    p.ntile = (p.W + p.Cb - 1) / p.Cb;
    const int64_t blocks = batch * p.nseg * p.ntile;
    if (blocks <= 0) return MOGT_OK;
    if (blocks > 0x7fffffffLL) return set_error(MOGT_E_INVALID, "%s: problem too large for one launch", what);
    const bool ulds = p.R <= GS_ULDS_MAX_R;
    const int ld = gs_ld<TS>(p.R);
    const size_t lds = (static_cast<size_t>(ulds ? p.R * ld : 0) + 2 * static_cast<size_t>(p.Cb) * ld) * sizeof(TS);
    const dim3 grid(static_cast<unsigned>(blocks)), block(GS_THREADS);
    // transitions staged per thread: R^2 / 256 values (1, 4 or 16); the
    // shallower the stash, the more steps in flight
    if (p.R <= 16)
        hipLaunchKernelGGL((generic_scan_kernel<TS, true, 1, 4, 16>), grid, block, lds, st, p);
    else if (p.R <= 32)
        hipLaunchKernelGGL((generic_scan_kernel<TS, true, 4, 4>), grid, block, lds, st, p);
    else if (ulds)
        hipLaunchKernelGGL((generic_scan_kernel<TS, true, GS_ULDS_MAX_R * GS_ULDS_MAX_R / GS_THREADS, 1>), grid,
                           block, lds, st, p);
    else
        hipLaunchKernelGGL((generic_scan_kernel<TS, false, 1, 2>), grid, block, lds, st, p);
    return check_launch(what);
}

bool io_code(int c) { return c == MOGT_F32 || c == MOGT_BF16 || c == MOGT_F64 || c == MOGT_F16; }

template <typename TS>
int run_generic(const void* U, const void* V, void* H, void* P, int64_t B, int64_t L, int64_t R, int64_t C,
                int v_code, int state_code, int out_code, int reverse, void* ws, hipStream_t st) {
    const GGeo g = generic_geometry(B, L, R, C, P != nullptr, state_code);
    const int iR = static_cast<int>(R), iC = static_cast<int>(C);
    // U / V / H / U_prefix views: [B][L][R][*]
    const GView vU{const_cast<void*>(U), L * R * R, R * R, R, state_code};
    const GView vV{const_cast<void*>(V), L * R * C, R * C, C, v_code};
    const GView vH{H, L * R * C, R * C, C, out_code};
    const GView vP{P, L * R * R, R * R, R, out_code};
    const GView none{nullptr, 0, 0, 0, state_code};

    unsigned char* base = static_cast<unsigned char*>(ws);
    const GView vS{base + g.s_off, g.nch * R * g.Wl, R * g.Wl, g.Wl, state_code};   // [B][nch][R][C+R]
    const GView vM{base + g.m_off, g.nch * R * g.Wo, R * g.Wo, g.Wo, state_code};   // [B][nch][R][Wo]

    if (g.nch > 1) {
        GParams loc{};
        loc.tr = vU; loc.in = vV; loc.init = none; loc.out_h = vS; loc.out_p = none;
        loc.L = L; loc.seg = g.seg; loc.nseg = static_cast<int>(g.nch);
        loc.R = iR; loc.W = g.Wl; loc.tr_c0 = 0; loc.cin = iC; loc.cid = iC; loc.csplit = g.Wl;
        loc.every = 0; loc.shift = 0; loc.rev = reverse;
        int rc = launch_generic<TS>(loc, B, st, "generic_scan local");
        if (rc) return rc;

        GParams car{};
        car.tr = vS; car.in = vS; car.init = none; car.out_h = vM; car.out_p = none;
        car.L = g.nch - 1; car.seg = g.nch - 1; car.nseg = 1;
        car.R = iR; car.W = g.Wo; car.tr_c0 = iC; car.cin = iC; car.cid = iC; car.csplit = g.Wo;
        car.every = 1; car.shift = 1; car.rev = 0;
        rc = launch_generic<TS>(car, B, st, "generic_scan carry");
        if (rc) return rc;
    }
    GParams out{};
    out.tr = vU; out.in = vV; out.init = g.nch > 1 ? vM : none; out.out_h = vH; out.out_p = vP;
    out.L = L; out.seg = g.seg; out.nseg = static_cast<int>(g.nch);
    out.R = iR; out.W = g.Wo; out.tr_c0 = 0; out.cin = iC; out.cid = iC; out.csplit = iC;
    out.every = 1; out.shift = 0; out.rev = reverse;
    return launch_generic<TS>(out, B, st, "generic_scan output");
}

int check_generic(int64_t B, int64_t L, int64_t R, int64_t C, int v_code, int state_code, int out_code,
                  int reverse, const void* P) {
    if (B < 0 || L < 0 || R < 0 || C < 0) return set_error(MOGT_E_INVALID, "negative size");
    if (R == 0 && B > 0 && L > 0) return set_error(MOGT_E_INVALID, "rank must be positive");
    if (R > GS_MAX_R) return set_error(MOGT_E_INVALID, "rank %lld above the generic scan's limit %d",
                                       static_cast<long long>(R), GS_MAX_R);
    if (C + R > 0x3fffffffLL) return set_error(MOGT_E_INVALID, "too many channels");
    if (state_code != MOGT_F32 && state_code != MOGT_F64)
        return set_error(MOGT_E_INVALID, "state dtype must be MOGT_F32 or MOGT_F64");
    if (!io_code(v_code) || !io_code(out_code)) return set_error(MOGT_E_INVALID, "unsupported V or output dtype");
    if (reverse && P) return set_error(MOGT_E_INVALID, "the reverse scan has no prefix output");
    return MOGT_OK;
}

}  // namespace
}  // namespace mogt

using namespace mogt;

extern "C" size_t mogt_affine_scan_generic_workspace_bytes(int64_t batch, int64_t length, int64_t rank,
                                                          int64_t channels, int with_prefix, int state_dtype) {
    if (batch <= 0 || length <= 0 || rank <= 0 || rank > GS_MAX_R || channels < 0) return WS_HDR_BYTES;
    return generic_geometry(batch, length, rank, channels, with_prefix != 0, state_dtype).bytes;
}

extern "C" int mogt_affine_scan_generic_fwd(const void* U, const void* V, void* H, void* U_prefix, int64_t batch,
                                            int64_t length, int64_t rank, int64_t channels, int v_dtype,
                                            int state_dtype, int out_dtype, int reverse, void* workspace,
                                            size_t workspace_bytes, void* stream) {
    clear_error();
    int rc = check_generic(batch, length, rank, channels, v_dtype, state_dtype, out_dtype, reverse, U_prefix);
    if (rc) return rc;
    if (batch == 0 || length == 0 || (channels == 0 && !U_prefix)) return MOGT_OK;
    if (!U || (channels > 0 && (!V || !H))) return set_error(MOGT_E_INVALID, "null tensor pointer");
    const GGeo g = generic_geometry(batch, length, rank, channels, U_prefix != nullptr, state_dtype);
    if (g.nch > 1 && (!workspace || workspace_bytes < g.bytes))
        return set_error(MOGT_E_WORKSPACE, "workspace of %zu bytes needed", g.bytes);
    hipStream_t st = static_cast<hipStream_t>(stream);
    return state_dtype == MOGT_F64
               ? run_generic<double>(U, V, H, U_prefix, batch, length, rank, channels, v_dtype, state_dtype,
                                     out_dtype, reverse, workspace, st)
               : run_generic<float>(U, V, H, U_prefix, batch, length, rank, channels, v_dtype, state_dtype,
                                    out_dtype, reverse, workspace, st);
}

extern "C" int mogt_affine_local_scan_generic(const void* U, const void* V, void* U_prefix, void* H_prefix,
                                              int64_t batch, int64_t length, int64_t rank, int64_t channels,
                                              int64_t block_size, int v_dtype, int state_dtype, int out_dtype,
                                              void* stream) {
    clear_error();
    int rc = check_generic(batch, length, rank, channels, v_dtype, state_dtype, out_dtype, 0, nullptr);
    if (rc) return rc;
    if (block_size <= 0) return set_error(MOGT_E_INVALID, "block_size must be positive");
    if (batch == 0 || length == 0) return MOGT_OK;
    if (!U || !U_prefix || (channels > 0 && (!V || !H_prefix))) return set_error(MOGT_E_INVALID, "null tensor pointer");
    const int64_t nb = (length + block_size - 1) / block_size;
    if (nb > 0x7fffffffLL) return set_error(MOGT_E_INVALID, "too many blocks");
    const int iR = static_cast<int>(rank), iC = static_cast<int>(channels);
    const GView none{nullptr, 0, 0, 0, state_dtype};
    GParams loc{};
    // one pass: every block from [0 | I], every step written (the OUTPUT pass
    // with no carries)
    loc.tr = GView{const_cast<void*>(U), length * rank * rank, rank * rank, rank, state_dtype};
    loc.in = GView{const_cast<void*>(V), length * rank * channels, rank * channels, channels, v_dtype};
    loc.init = none;
    loc.out_h = GView{H_prefix, length * rank * channels, rank * channels, channels, out_dtype};
    loc.out_p = GView{U_prefix, length * rank * rank, rank * rank, rank, out_dtype};
    loc.L = length; loc.seg = block_size; loc.nseg = static_cast<int>(nb);
    loc.R = iR; loc.W = iC + iR; loc.tr_c0 = 0; loc.cin = iC; loc.cid = iC; loc.csplit = iC;
    loc.every = 1; loc.shift = 0; loc.rev = 0;
    hipStream_t st = static_cast<hipStream_t>(stream);
    return state_dtype == MOGT_F64 ? launch_generic<double>(loc, batch, st, "generic local scan")
                                   : launch_generic<float>(loc, batch, st, "generic local scan");
}
