// Coupled write-forget per-rank scan of the MOGT mixer (identity connection):
// the gate sigmoid, the coupling a = damping * (1 - g) and the gated write
// b = v * g are computed in registers inside the single-pass diagonal scan
// (diag_kernel.h), so the reference's [B, L, r, r] fp32 U, its [B, L, 3d] gate
// input and its gated V (model_mogt.py:104-182) are never written to memory.
#include "diag_kernel.h"

namespace mogt {

namespace {

template <typename TZ, typename TV, typename TO>
int coupled_dispatch(const DiagParams& prm, const DiagTile& t, hipStream_t st) {
#define MOGT_CASE(V_, F_, S_, W_)                                          \
    if (t.vec == V_ && t.lanes == F_ && t.steps == S_ && t.waves == W_) \
        return diag_launch<MODE_COUPLED, TV, TZ, TO, V_, F_, S_, W_, false>(prm, st);
    MOGT_COUPLED_TILES(MOGT_CASE)
#undef MOGT_CASE
    return set_error(MOGT_E_INVALID, "coupled scan: tile (vec=%d, lanes=%d, steps=%d, waves=%d) not compiled",
                     t.vec, t.lanes, t.steps, t.waves);
}

// Tiles of the row-statistics variant: the default tiles, all 64 features
// wide, so the statistics have one column per 64 features whatever the pick.
#define MOGT_COUPLED_STAT_TILES(X) X(4, 16, 8, 16) X(4, 16, 8, 8) X(4, 16, 16, 8) X(2, 32, 8, 16) X(2, 32, 16, 8) X(1, 64, 8, 16) \
    X(1, 64, 32, 16) X(1, 64, 16, 16)

template <typename TV, typename TO>
int coupled_stat_dispatch(const DiagParams& prm, const DiagTile& t, hipStream_t st) {
#define MOGT_CASE(V_, F_, S_, W_)                                          \
    if (t.vec == V_ && t.lanes == F_ && t.steps == S_ && t.waves == W_) \
        return diag_launch<MODE_COUPLED, TV, float, TO, V_, F_, S_, W_, false, true>(prm, st);
    MOGT_COUPLED_STAT_TILES(MOGT_CASE)
#undef MOGT_CASE
    return set_error(MOGT_E_INVALID, "coupled scan statistics: tile (vec=%d, lanes=%d, steps=%d, waves=%d) not compiled",
                     t.vec, t.lanes, t.steps, t.waves);
}

// Gate logits of the projection-fed scan: row t of the projection P holds the
// current token's pre-logits from column gate_col (R columns; `pre` points
// there) and, with gate_prev, the previous-token pre-logits in the next R
// columns, which belong to step t + 1:
//   z[b][t][i] = (P[t][gate_col + i] + (gate_prev && t > 0 ? P[t-1][gate_col + R + i] : 0))
//                + gconst[b][i]
// (phi_value_gate over [x_t, x_{t-1}, prefix], model_mogt.py:104-122, 170-171,
// with the bias and prefix terms folded into gconst).  Thread = (row, group of
// four consecutive logits), 32-bit indexing (the host bounds the count).
template <typename T>
__global__ __launch_bounds__(256) void coupled_gate_logits_kernel(const T* __restrict__ pre, int64_t ld,
                                                                  int gate_prev, const float* __restrict__ gconst,
                                                                  float* __restrict__ z, uint32_t L, int R,
                                                                  uint32_t n) {
    const uint32_t k = blockIdx.x * 256u + threadIdx.x;
    if (k >= n) return;
    const uint32_t nq = (static_cast<uint32_t>(R) + 3u) / 4u;
    const uint32_t row = k / nq;
    const int i0 = static_cast<int>(k - row * nq) * 4;
    const uint32_t b = row / L;
    const bool prev = gate_prev && row - b * L > 0;
    const T* cur = pre + static_cast<int64_t>(row) * ld;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int i = i0 + e;
        if (i < R) {
            float v = IO<T>::ld(cur[i]);
            if (prev) v = v + IO<T>::ld(cur[R + i - ld]);
            if (gconst) v = v + gconst[static_cast<int64_t>(b) * R + i];
            z[static_cast<int64_t>(row) * R + i] = v;
        }
    }
}

template <typename T>
int coupled_gate_logits(const T* pre, int64_t ld, int gate_prev, const float* gconst, float* z, int64_t B,
                        int64_t L, int R, hipStream_t st) {
    const int64_t n = B * L * ((R + 3) / 4);
    if (n > 0xffffff00LL) return set_error(MOGT_E_INVALID, "projection-fed scan: too many gate logits");
    const unsigned blocks = static_cast<unsigned>((n + 255) / 256);
    hipLaunchKernelGGL((coupled_gate_logits_kernel<T>), dim3(blocks), dim3(256), 0, st, pre, ld, gate_prev, gconst,
                       z, static_cast<uint32_t>(L), R, static_cast<uint32_t>(n));
    return check_launch("coupled_gate_logits_kernel");
}

// Workspace bytes of the fp32 gate logits [B, L, R], rounded up to 256.
size_t coupled_logit_bytes(int64_t B, int64_t L, int64_t R) {
    return (static_cast<size_t>(B * L * R) * sizeof(float) + 255) & ~static_cast<size_t>(255);
}

bool dtype_ok(int d) { return d == MOGT_F32 || d == MOGT_BF16; }

// Default tile (measured on MI355X at r = 16, c = 48, L = 8k..32k): four
// channels per lane where the channel count and the pointers allow it (the
// lanes of one vector must share a gate, so the vector must divide the channel
// count), 512-step chunks; short problems fall back to shorter chunks.
DiagTile coupled_tile(int64_t B, int64_t L, int64_t R, int64_t C, int align_elems) {
    static const TileChoice v4[] = {{{4, 16, 16, 8}, 512}, {{4, 16, 8, 8}, 128}, {{2, 32, 8, 16}, 128},
                                    {{1, 64, 8, 16}, 0}};
    static const TileChoice v2[] = {{{2, 32, 16, 8}, 128}, {{2, 32, 8, 16}, 128}, {{1, 64, 8, 16}, 0}};
    static const TileChoice v1[] = {{{1, 64, 32, 16}, 128}, {{1, 64, 16, 16}, 128}, {{1, 64, 8, 16}, 0}};
    if (C % 4 == 0 && align_elems % 4 == 0) return pick_tile(B, L, R * C, v4, 4);
    if (C % 2 == 0 && align_elems % 2 == 0) return pick_tile(B, L, R * C, v2, 3);
    return pick_tile(B, L, R * C, v1, 3);
}

// Largest vector width (4, 2 or 1 elements) both v and h are aligned to.
int coupled_alignment(const void* v, const void* h, int v_dtype, int out_dtype) {
    const uintptr_t ve = v_dtype == MOGT_BF16 ? 2 : 4, he = out_dtype == MOGT_BF16 ? 2 : 4;
    for (int n : {4, 2})
        if (reinterpret_cast<uintptr_t>(v) % (ve * n) == 0 && reinterpret_cast<uintptr_t>(h) % (he * n) == 0)
            return n;
    return 1;
}

}  // namespace

// ldv: row stride of v (0: R * C).
int coupled_run(const void* z, const void* v, void* h, int64_t B, int64_t L, int64_t R, int64_t C,
                float damping, int z_dtype, int v_dtype, int out_dtype, const DiagTile& t,
                void* ws, size_t ws_bytes, void* stream, float* row_stats = nullptr, int64_t ldv = 0) {
    const int64_t D = R * C;
    if (C % t.vec != 0)
        return set_error(MOGT_E_INVALID, "channels %lld not a multiple of vec %d", (long long)C, t.vec);
    DiagParams prm{};
    int rc = diag_prepare(prm, B, L, D, t, ws, ws_bytes);
    if (rc) return rc;
    prm.a = z;
    prm.b = v;
    prm.h = h;
    prm.aprefix = nullptr;
    prm.R = static_cast<int>(R);
    prm.C = static_cast<int>(C);
    prm.damping = damping;
    prm.rowstat = row_stats;
    prm.ldz = prm.R;
    if (ldv) prm.ldv = ldv;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool zb = z_dtype == MOGT_BF16, vb = v_dtype == MOGT_BF16, ob = out_dtype == MOGT_BF16;
    if (row_stats) {
        if (zb) return set_error(MOGT_E_INVALID, "coupled scan statistics: gate logits must be fp32");
        if (t.vec * t.lanes != 64)
            return set_error(MOGT_E_INVALID, "coupled scan statistics: tile must be 64 features wide");
        if (vb) return ob ? coupled_stat_dispatch<bf16_t, bf16_t>(prm, t, st) : coupled_stat_dispatch<bf16_t, float>(prm, t, st);
        return ob ? coupled_stat_dispatch<float, bf16_t>(prm, t, st) : coupled_stat_dispatch<float, float>(prm, t, st);
    }
    if (!zb && vb && !ob) return coupled_dispatch<float, bf16_t, float>(prm, t, st);
    if (!zb && vb && ob) return coupled_dispatch<float, bf16_t, bf16_t>(prm, t, st);
    if (zb && vb && !ob) return coupled_dispatch<bf16_t, bf16_t, float>(prm, t, st);
    if (zb && vb && ob) return coupled_dispatch<bf16_t, bf16_t, bf16_t>(prm, t, st);
    if (!zb && !vb && !ob) return coupled_dispatch<float, float, float>(prm, t, st);
    if (!zb && !vb && ob) return coupled_dispatch<float, float, bf16_t>(prm, t, st);
    if (zb && !vb && !ob) return coupled_dispatch<bf16_t, float, float>(prm, t, st);
    return coupled_dispatch<bf16_t, float, bf16_t>(prm, t, st);
}

}  // namespace mogt

using namespace mogt;

extern "C" size_t mogt_coupled_rank_scan_workspace_bytes(int64_t batch, int64_t length,
                                                         int64_t rank, int64_t channels,
                                                         int v_dtype) {
    if (batch <= 0 || length <= 0 || rank <= 0 || channels <= 0) return WS_HDR_BYTES;
    // Largest requirement over the tiles the entry point may pick.
    (void)v_dtype;
    size_t best = 0;
    for (int al : {4, 2, 1}) {
        const size_t n = diag_geometry(batch, length, rank * channels,
                                       coupled_tile(batch, length, rank, channels, al)).bytes;
        best = n > best ? n : best;
    }
    // + the projection-fed entry point's assembled gate logits
    return ((best + 255) & ~static_cast<size_t>(255)) + coupled_logit_bytes(batch, length, rank);
}

extern "C" int mogt_coupled_rank_scan_fwd(const void* z, const void* v, void* h, int64_t batch,
                                          int64_t length, int64_t rank, int64_t channels,
                                          float damping, int z_dtype, int v_dtype, int out_dtype,
                                          void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    if (batch < 0 || length < 0) return set_error(MOGT_E_INVALID, "negative size");
    if (rank <= 0 || channels <= 0 || rank > 0x7fffffff || channels > 0x7fffffff)
        return set_error(MOGT_E_INVALID, "rank and channels must be positive");
    if (!dtype_ok(z_dtype) || !dtype_ok(v_dtype) || !dtype_ok(out_dtype))
        return set_error(MOGT_E_INVALID, "unsupported dtype code");
    if (batch == 0 || length == 0) return MOGT_OK;
    if (!z || !v || !h) return set_error(MOGT_E_INVALID, "null tensor pointer");
    const DiagTile t = coupled_tile(batch, length, rank, channels,
                                    coupled_alignment(v, h, v_dtype, out_dtype));
    return coupled_run(z, v, h, batch, length, rank, channels, damping, z_dtype, v_dtype, out_dtype,
                       t, workspace, workspace_bytes, stream);
}

extern "C" int mogt_coupled_rank_scan_stats_fwd(const void* z, const void* v, void* h, float* row_stats,
                                                int64_t batch, int64_t length, int64_t rank, int64_t channels,
                                                float damping, int v_dtype, int out_dtype, void* workspace,
                                                size_t workspace_bytes, void* stream) {
    clear_error();
    if (batch < 0 || length < 0) return set_error(MOGT_E_INVALID, "negative size");
    if (rank <= 0 || channels <= 0 || rank > 0x7fffffff || channels > 0x7fffffff)
        return set_error(MOGT_E_INVALID, "rank and channels must be positive");
    if (!dtype_ok(v_dtype) || !dtype_ok(out_dtype)) return set_error(MOGT_E_INVALID, "unsupported dtype code");
    if (batch == 0 || length == 0) return MOGT_OK;
    if (!z || !v || !h || !row_stats) return set_error(MOGT_E_INVALID, "null tensor pointer");
    const DiagTile t = coupled_tile(batch, length, rank, channels, coupled_alignment(v, h, v_dtype, out_dtype));
    return coupled_run(z, v, h, batch, length, rank, channels, damping, MOGT_F32, v_dtype, out_dtype, t,
                       workspace, workspace_bytes, stream, row_stats);
}

extern "C" int mogt_coupled_rank_scan_proj_fwd(const void* proj, int64_t ld_proj, int64_t gate_col, int gate_prev,
                                               const float* gate_const, void* h, float* row_stats, float* z_out,
                                               int64_t batch, int64_t length, int64_t rank, int64_t channels,
                                               float damping, int dtype, int out_dtype, void* workspace,
                                               size_t workspace_bytes, void* stream) {
    clear_error();
    if (batch < 0 || length < 0) return set_error(MOGT_E_INVALID, "negative size");
    if (rank <= 0 || channels <= 0 || rank > 0x7fffffff || channels > 0x7fffffff)
        return set_error(MOGT_E_INVALID, "rank and channels must be positive");
    if (!dtype_ok(dtype) || !dtype_ok(out_dtype)) return set_error(MOGT_E_INVALID, "unsupported dtype code");
    if (row_stats ? out_dtype != dtype : out_dtype != MOGT_F32)
        return set_error(MOGT_E_INVALID, "projection-fed scan: h in proj's dtype with row statistics, "
                                         "else fp32");
    const int64_t D = rank * channels;
    if (gate_prev != 0 && gate_prev != 1) return set_error(MOGT_E_INVALID, "gate_prev must be 0 or 1");
    if (gate_col < D || gate_col + rank * (1 + gate_prev) > ld_proj || ld_proj > 0x7fffffff)
        return set_error(MOGT_E_INVALID, "projection row of %lld columns cannot hold v (%lld) and the gate "
                         "pre-logits at column %lld", (long long)ld_proj, (long long)D, (long long)gate_col);
    if (batch == 0 || length == 0) return MOGT_OK;
    if (!proj || !h) return set_error(MOGT_E_INVALID, "null tensor pointer");
    // the vector must divide the projection's row stride as well as the channels
    const int al = coupled_alignment(proj, h, dtype, out_dtype);
    const int vec_ok = ld_proj % 4 == 0 ? al : (ld_proj % 2 == 0 ? (al < 2 ? al : 2) : 1);
    const DiagTile t = coupled_tile(batch, length, rank, channels, vec_ok);
    // the logits go to z_out, or to the workspace's tail
    size_t scan_bytes = workspace_bytes;
    float* z = z_out;
    if (!z) {
        const size_t zbytes = coupled_logit_bytes(batch, length, rank);
        if (!workspace || workspace_bytes < zbytes)
            return set_error(MOGT_E_WORKSPACE, "workspace of %zu bytes cannot hold the %zu bytes of gate logits",
                             workspace_bytes, zbytes);
        scan_bytes = (workspace_bytes - zbytes) & ~static_cast<size_t>(255);
        z = reinterpret_cast<float*>(static_cast<char*>(workspace) + scan_bytes);
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    const size_t esz = dtype == MOGT_BF16 ? 2 : 4;
    const void* pre = static_cast<const char*>(proj) + gate_col * esz;
    const int R = static_cast<int>(rank);
    int rc = dtype == MOGT_BF16
                 ? coupled_gate_logits(static_cast<const bf16_t*>(pre), ld_proj, gate_prev, gate_const, z, batch,
                                       length, R, st)
                 : coupled_gate_logits(static_cast<const float*>(pre), ld_proj, gate_prev, gate_const, z, batch,
                                       length, R, st);
    if (rc) return rc;
    return coupled_run(z, proj, h, batch, length, rank, channels, damping, MOGT_F32, dtype, out_dtype, t, workspace,
                       scan_bytes, stream, row_stats, ld_proj);
}

// The same with an explicit tile (sweeps and tests): the tile must be one of
// mogt_diag_scan_tiles(2), its vector must divide the channel count, and v and
// h must be aligned to the vector (at most 16 bytes).  Workspace:
// mogt_diag_scan_workspace_bytes_cfg(batch, length, rank * channels, tile).
extern "C" int mogt_coupled_rank_scan_fwd_cfg(const void* z, const void* v, void* h, int64_t batch,
                                              int64_t length, int64_t rank, int64_t channels, float damping,
                                              int z_dtype, int v_dtype, int out_dtype, int vec, int lanes,
                                              int steps, int waves, void* workspace, size_t workspace_bytes,
                                              void* stream) {
    clear_error();
    if (batch < 0 || length < 0) return set_error(MOGT_E_INVALID, "negative size");
    if (rank <= 0 || channels <= 0 || rank > 0x7fffffff || channels > 0x7fffffff)
        return set_error(MOGT_E_INVALID, "rank and channels must be positive");
    if (!dtype_ok(z_dtype) || !dtype_ok(v_dtype) || !dtype_ok(out_dtype))
        return set_error(MOGT_E_INVALID, "unsupported dtype code");
    const DiagTile t{vec, lanes, steps, waves};
    if (!diag_tile_compiled(2, t))
        return set_error(MOGT_E_INVALID, "coupled scan: tile (%d,%d,%d,%d) not compiled", vec, lanes, steps, waves);
    if (batch == 0 || length == 0) return MOGT_OK;
    if (!z || !v || !h) return set_error(MOGT_E_INVALID, "null tensor pointer");
    auto aligned = [&](const void* p, int dt) {
        const uintptr_t bytes = static_cast<uintptr_t>(vec) * (dt == MOGT_BF16 ? 2 : 4);
        return reinterpret_cast<uintptr_t>(p) % (bytes < 16 ? bytes : 16) == 0;
    };
    if (!aligned(v, v_dtype) || !aligned(h, out_dtype))
        return set_error(MOGT_E_INVALID, "v and h must be aligned to the tile's vector");
    return coupled_run(z, v, h, batch, length, rank, channels, damping, z_dtype, v_dtype, out_dtype, t, workspace,
                       workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// Gradient epilogue of the coupled scan (the backward of
// mogt_coupled_rank_scan_fwd, after the reverse scan has produced
// G_t = dH_t + a_{t+1} G_{t+1}).  Per (b, t, i) with g = sigmoid(z[b,t,i]) and
// g_io = g rounded to v's dtype (the gate as multiplied into v):
//   dv[b,t,i,c] = G[b,t,i,c] * g_io                                  (v's dtype)
//   dz[b,t,i]   = g (1 - g) (sum_c G v - damping sum_c G h[b,t-1])   (fp32)
// since h_t = damping (1 - g_t) h_{t-1} + round(v_t g_t) and the rounding passes
// gradients through, as a dtype cast does under autograd.  A work-group walks
// CG_ROWS rows (b, t); per row, thread f covers features 4f .. 4f + 3 (coalesced
// 16-byte fp32 / 8-byte bf16 vectors), writes dv and leaves its two partial
// dot products in LDS, and thread i then sums rank i's C / 4 partials.
// ---------------------------------------------------------------------------
namespace mogt {

constexpr int CG_THREADS = 256;
constexpr int CG_ROWS = 8;
constexpr int CG_MAX_VEC = 1024;   // D <= 4096

// ldv: row stride of v and dv.  PROJ: v and dv live in projection rows of
// ldv elements whose gate columns (from D: R current, then R previous when
// gate_prev) receive the logit gradient -- dz[t] in row t's current columns
// and in row t - 1's previous columns (the previous-token term of step t is a
// term of row t - 1), zero in row L - 1's previous columns; dz (fp32
// [B, L, R]) may then be null.
template <typename TV, bool PROJ = false>
__global__ __launch_bounds__(CG_THREADS) void coupled_grad_kernel(const float* __restrict__ G,
                                                                  const float* __restrict__ z,
                                                                  const TV* __restrict__ v,
                                                                  const float* __restrict__ h,
                                                                  TV* __restrict__ dv, float* __restrict__ dz,
                                                                  int64_t nrows, int64_t L, int R, int C,
                                                                  float damping, int64_t ldv = 0,
                                                                  int gate_prev = 0) {
    __shared__ float s_v[CG_MAX_VEC], s_h[CG_MAX_VEC];
    const int tid = threadIdx.x;
    const int D = R * C, nvec = D / 4, vpr = C / 4;
    const int64_t ld = PROJ ? ldv : D;
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * CG_ROWS;
    const int64_t r1 = r0 + CG_ROWS < nrows ? r0 + CG_ROWS : nrows;
    for (int64_t row = r0; row < r1; ++row) {
        const bool has_prev = row % L != 0;
        const int64_t base = row * D;
        for (int f = tid; f < nvec; f += CG_THREADS) {
            const int i = f / vpr;
            const float g_io = IO<TV>::ld(IO<TV>::st(sigmoid_hw(z[row * R + i])));
            float gv[4], vv[4], hv[4] = {0.0f, 0.0f, 0.0f, 0.0f}, o[4];
            load_vec<float, 4>(G + base + 4 * f, gv);
            load_vec<TV, 4>(v + row * ld + 4 * f, vv);
            if (has_prev) load_vec<float, 4>(h + base - D + 4 * f, hv);
            float sv = 0.0f, sh = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                sv = fmaf(gv[e], vv[e], sv);
                sh = fmaf(gv[e], hv[e], sh);
                o[e] = gv[e] * g_io;
            }
            store_vec<TV, 4>(dv + row * ld + 4 * f, o);
            s_v[f] = sv;
            s_h[f] = sh;
        }
        __syncthreads();
        for (int i = tid; i < R; i += CG_THREADS) {
            float sv = 0.0f, sh = 0.0f;
            for (int k = i * vpr; k < (i + 1) * vpr; ++k) {
                sv += s_v[k];
                sh += s_h[k];
            }
            const float gg = sigmoid_hw(z[row * R + i]);
            const float g = (sv - damping * sh) * gg * (1.0f - gg);
            if (dz) dz[row * R + i] = g;
            if constexpr (PROJ) {
                dv[row * ld + D + i] = IO<TV>::st(g);
                if (gate_prev) {
                    if (has_prev) dv[(row - 1) * ld + D + R + i] = IO<TV>::st(g);
                    if (row % L == L - 1) dv[row * ld + D + R + i] = IO<TV>::st(0.0f);
                }
            }
        }
        __syncthreads();
    }
}

}  // namespace mogt

extern "C" int mogt_coupled_rank_scan_grad(const void* G, const float* z, const void* v, const float* h, void* dv,
                                           float* dz, int64_t batch, int64_t length, int64_t rank,
                                           int64_t channels, float damping, int v_dtype, void* stream) {
    clear_error();
    if (batch < 0 || length < 0) return set_error(MOGT_E_INVALID, "negative size");
    if (rank <= 0 || channels <= 0 || channels % 4 != 0 || rank * channels > 4 * CG_MAX_VEC)
        return set_error(MOGT_E_INVALID,
                         "coupled grad: channels a positive multiple of 4 and rank * channels <= 4096");
    if (!dtype_ok(v_dtype)) return set_error(MOGT_E_INVALID, "unsupported dtype code");
    if (batch == 0 || length == 0) return MOGT_OK;
    if (!G || !z || !v || !h || !dv || !dz) return set_error(MOGT_E_INVALID, "null tensor pointer");
    const int64_t nrows = batch * length;
    const int64_t blocks = (nrows + CG_ROWS - 1) / CG_ROWS;
    if (blocks > 0x7fffffffLL) return set_error(MOGT_E_INVALID, "coupled grad: problem too large");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int R = static_cast<int>(rank), C = static_cast<int>(channels);
    if (v_dtype == MOGT_F32)
        hipLaunchKernelGGL((coupled_grad_kernel<float>), dim3(static_cast<unsigned>(blocks)), dim3(CG_THREADS), 0, st,
                           static_cast<const float*>(G), z, static_cast<const float*>(v), h,
                           static_cast<float*>(dv), dz, nrows, length, R, C, damping);
    else
        hipLaunchKernelGGL((coupled_grad_kernel<bf16_t>), dim3(static_cast<unsigned>(blocks)), dim3(CG_THREADS), 0,
                           st, static_cast<const float*>(G), z, static_cast<const bf16_t*>(v), h,
                           static_cast<bf16_t*>(dv), dz, nrows, length, R, C, damping);
    return check_launch("coupled_grad_kernel");
}

extern "C" int mogt_coupled_rank_scan_proj_grad(const float* G, const float* z, const void* proj, int64_t ld_proj,
                                                int gate_prev, const float* h, void* dproj, float* dz,
                                                int64_t batch, int64_t length, int64_t rank, int64_t channels,
                                                float damping, int dtype, void* stream) {
    clear_error();
    if (batch < 0 || length < 0) return set_error(MOGT_E_INVALID, "negative size");
    if (rank <= 0 || channels <= 0 || channels % 4 != 0 || rank * channels > 4 * CG_MAX_VEC)
        return set_error(MOGT_E_INVALID,
                         "coupled grad: channels a positive multiple of 4 and rank * channels <= 4096");
    if (!dtype_ok(dtype)) return set_error(MOGT_E_INVALID, "unsupported dtype code");
    if (gate_prev != 0 && gate_prev != 1) return set_error(MOGT_E_INVALID, "gate_prev must be 0 or 1");
    const int64_t D = rank * channels;
    if (ld_proj != D + rank * (1 + gate_prev) || ld_proj % 4 != 0)
        return set_error(MOGT_E_INVALID, "projection rows must be D + R * (1 + gate_prev) elements, a multiple of 4");
    if (batch == 0 || length == 0) return MOGT_OK;
    if (!G || !z || !proj || !h || !dproj) return set_error(MOGT_E_INVALID, "null tensor pointer");
    const int64_t nrows = batch * length;
    const int64_t blocks = (nrows + CG_ROWS - 1) / CG_ROWS;
    if (blocks > 0x7fffffffLL) return set_error(MOGT_E_INVALID, "coupled grad: problem too large");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int R = static_cast<int>(rank), C = static_cast<int>(channels);
    if (dtype == MOGT_F32)
        hipLaunchKernelGGL((coupled_grad_kernel<float, true>), dim3(static_cast<unsigned>(blocks)), dim3(CG_THREADS),
                           0, st, G, z, static_cast<const float*>(proj), h, static_cast<float*>(dproj), dz, nrows,
                           length, R, C, damping, ld_proj, gate_prev);
    else
        hipLaunchKernelGGL((coupled_grad_kernel<bf16_t, true>), dim3(static_cast<unsigned>(blocks)),
                           dim3(CG_THREADS), 0, st, G, z, static_cast<const bf16_t*>(proj), h,
                           static_cast<bf16_t*>(dproj), dz, nrows, length, R, C, damping, ld_proj, gate_prev);
    return check_launch("coupled_grad_kernel");
}
