// Backward of the token embedding (nn.Embedding, model_mogt.py:262, 270):
// dW[v] = the sum of the output-gradient rows of every position holding token
// v, summed in position order, so the result does not depend on timing.
//
// The caller sorts the token ids stably (positions of equal ids keep their
// order), passes the sorted ids and the positions in that order, and
// zero-fills dW.  Positions below n1 are rows of the first gradient, the rest
// rows of a second one (a second lookup into the same table, whose gradient
// then needs no table of its own).  Pass 1: one wave per block of EB consecutive sorted
// positions walks them, summing the gradient rows of each run of equal ids: a
// run that begins and ends inside the block is written to dW directly; the
// piece of a run that began in an earlier block goes to the block's slot 0;
// a run that begins in the block and continues past it goes to slot 1.
// Pass 2: one wave per block whose last run began in it and continues adds
// that slot 1 and the slot 0 of every following block the run covers, in
// block order, and writes dW.  A frequent token's run is thus summed by many
// waves at once instead of one.
#include "common.h"

namespace mogt {
namespace {

constexpr int EB = 16;        // sorted positions per block
constexpr int EMB_WAVES = 4;  // waves (blocks) per work-group

template <typename TG, int VPL>
__global__ __launch_bounds__(64 * EMB_WAVES) void emb_bwd_blocks(const TG* __restrict__ g, int64_t ldg,
                                                                 const TG* __restrict__ g2, int64_t ldg2,
                                                                 int64_t n1, const int64_t* __restrict__ sid,
                                                                 const int64_t* __restrict__ perm, int64_t n,
                                                                 int D, int64_t V, float* __restrict__ dw,
                                                                 float* __restrict__ part) {
    const int lane = threadIdx.x & 63;
    const int64_t b = static_cast<int64_t>(blockIdx.x) * EMB_WAVES + (threadIdx.x >> 6);
    const int64_t i0 = b * EB;
    if (i0 >= n) return;
    const int64_t i1 = i0 + EB < n ? i0 + EB : n;
    float acc[VPL][4];
#pragma unroll
    for (int k = 0; k < VPL; ++k)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[k][e] = 0.0f;
    bool began_before = i0 > 0 && sid[i0 - 1] == sid[i0];
    for (int64_t i = i0; i < i1; ++i) {
        const int64_t id = sid[i];
        const int64_t row = perm[i];
        const TG* src = row < n1 ? g + row * ldg : g2 + (row - n1) * ldg2;
#pragma unroll
        for (int k = 0; k < VPL; ++k) {
            const int c = (k * 64 + lane) * 4;
            if (c < D) {
                float v[4];
                load_vec<TG, 4>(src + c, v);
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[k][e] += v[e];
            }
        }
        const bool run_ends = i + 1 == n || sid[i + 1] != id;
        if (run_ends || i + 1 == i1) {
            float* dst = nullptr;
            if (began_before)
                dst = part + (2 * b) * D;          // slot 0: a run that began earlier
            else if (!run_ends)
                dst = part + (2 * b + 1) * D;      // slot 1: begins here, continues
            else if (id >= 0 && id < V)
                dst = dw + id * D;                 // whole run inside the block
            if (dst) {
#pragma unroll
                for (int k = 0; k < VPL; ++k) {
                    const int c = (k * 64 + lane) * 4;
                    if (c < D) store_vec<float, 4>(dst + c, acc[k]);
                }
            }
#pragma unroll
            for (int k = 0; k < VPL; ++k)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[k][e] = 0.0f;
            began_before = false;
        }
    }
}

template <int VPL>
__global__ __launch_bounds__(64 * EMB_WAVES) void emb_bwd_runs(const int64_t* __restrict__ sid, int64_t n, int D,
                                                               int64_t V, const float* __restrict__ part,
                                                               float* __restrict__ dw) {
    const int lane = threadIdx.x & 63;
    const int64_t b = static_cast<int64_t>(blockIdx.x) * EMB_WAVES + (threadIdx.x >> 6);
    const int64_t i0 = b * EB;
    if (i0 >= n) return;
    const int64_t last = (i0 + EB < n ? i0 + EB : n) - 1;
    if (last + 1 >= n) return;
    const int64_t id = sid[last];
    if (sid[last + 1] != id) return;              // the block's last run ends in it
    if (i0 > 0 && sid[i0 - 1] == id) return;      // the run began in an earlier block
    float acc[VPL][4];
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        const int c = (k * 64 + lane) * 4;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[k][e] = 0.0f;
        if (c < D) load_vec<float, 4>(part + (2 * b + 1) * D + c, acc[k]);
    }
    for (int64_t bb = b + 1;; ++bb) {             // every following block the run covers
#pragma unroll
        for (int k = 0; k < VPL; ++k) {
            const int c = (k * 64 + lane) * 4;
            if (c < D) {
                float v[4];
                load_vec<float, 4>(part + (2 * bb) * D + c, v);
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[k][e] += v[e];
            }
        }
        const int64_t l = ((bb + 1) * EB < n ? (bb + 1) * EB : n) - 1;
        if (l + 1 >= n || sid[l + 1] != id) break;
    }
    if (id < 0 || id >= V) return;
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        const int c = (k * 64 + lane) * 4;
        if (c < D) store_vec<float, 4>(dw + id * D + c, acc[k]);
    }
}

template <typename TG>
int emb_bwd_launch(const TG* g, int64_t ldg, const TG* g2, int64_t ldg2, int64_t n1, const int64_t* sid,
                   const int64_t* perm, int64_t n, int D, int64_t V, float* dw, float* part, hipStream_t st) {
    const int64_t blocks = (n + EB - 1) / EB;
    const dim3 grid(static_cast<unsigned>((blocks + EMB_WAVES - 1) / EMB_WAVES));
    const dim3 block(64 * EMB_WAVES);
    const int vpl = (D + 255) / 256;
#define MOGT_EMB_CASE(VP)                                                                              \
    if (vpl <= VP) {                                                                                   \
        hipLaunchKernelGGL((emb_bwd_blocks<TG, VP>), grid, block, 0, st, g, ldg, g2, ldg2, n1, sid, perm, n, D, \
                           V, dw, part);                                                               \
        int rc = check_launch("emb_bwd_blocks");                                                       \
        if (rc) return rc;                                                                             \
        hipLaunchKernelGGL((emb_bwd_runs<VP>), grid, block, 0, st, sid, n, D, V, part, dw);             \
        return check_launch("emb_bwd_runs");                                                           \
    }
    MOGT_EMB_CASE(1)
    MOGT_EMB_CASE(2)
    MOGT_EMB_CASE(3)
    MOGT_EMB_CASE(4)
    MOGT_EMB_CASE(8)
    MOGT_EMB_CASE(16)
#undef MOGT_EMB_CASE
    return set_error(MOGT_E_INVALID, "embedding_bwd: row length %d > 4096", D);
}

}  // namespace
}  // namespace mogt

using namespace mogt;

extern "C" int mogt_embedding_bwd(const void* grad, int64_t ld_grad, const void* grad2, int64_t ld_grad2,
                                  int64_t n_first, int grad_dtype, const int64_t* sorted_ids,
                                  const int64_t* positions, int64_t n, int64_t dim, int64_t vocab, float* dweight,
                                  float* partials, void* stream) {
    clear_error();
    if (n < 0 || dim <= 0 || vocab <= 0) return set_error(MOGT_E_INVALID, "embedding_bwd: bad shape");
    if (dim % 4 != 0 || dim > 4096)
        return set_error(MOGT_E_INVALID, "embedding_bwd: row length must be a multiple of 4 and <= 4096");
    if (n_first < 0 || n_first > n || (!grad2 && n_first != n))
        return set_error(MOGT_E_INVALID, "embedding_bwd: n_first must be in [0, n], and n without a second gradient");
    if (ld_grad < dim || ld_grad % 4 != 0 || (grad2 && (ld_grad2 < dim || ld_grad2 % 4 != 0)))
        return set_error(MOGT_E_INVALID, "embedding_bwd: gradient row stride must cover the row (multiple of 4)");
    if (grad_dtype != MOGT_F32 && grad_dtype != MOGT_BF16)
        return set_error(MOGT_E_INVALID, "embedding_bwd: unsupported gradient dtype");
    if (n == 0) return MOGT_OK;
    if ((n_first > 0 && !grad) || !sorted_ids || !positions || !dweight || !partials)
        return set_error(MOGT_E_INVALID, "embedding_bwd: null pointer");
    const size_t esz = grad_dtype == MOGT_BF16 ? 2 : 4;
    if ((reinterpret_cast<uintptr_t>(grad) % (4 * esz)) || (reinterpret_cast<uintptr_t>(grad2) % (4 * esz)) ||
        (reinterpret_cast<uintptr_t>(dweight) % 16) || (reinterpret_cast<uintptr_t>(partials) % 16))
        return set_error(MOGT_E_INVALID, "embedding_bwd: gradient, dweight and partials need vector alignment");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int D = static_cast<int>(dim);
    if (grad_dtype == MOGT_BF16)
        return emb_bwd_launch<bf16_t>(static_cast<const bf16_t*>(grad), ld_grad, static_cast<const bf16_t*>(grad2),
                                      ld_grad2, n_first, sorted_ids, positions, n, D, vocab, dweight, partials, st);
    return emb_bwd_launch<float>(static_cast<const float*>(grad), ld_grad, static_cast<const float*>(grad2), ld_grad2,
                                 n_first, sorted_ids, positions, n, D, vocab, dweight, partials, st);
}
