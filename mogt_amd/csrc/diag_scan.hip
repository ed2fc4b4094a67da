// C entry points of the single-pass diagonal affine scan (kernel: diag_kernel.h;
// instantiations: diag_f32.hip, diag_bf16.hip, coupled_scan.hip).
#include <mutex>

#include "diag_kernel.h"

namespace mogt {

bool diag_tile_compiled(int family, const DiagTile& t) {
#define MOGT_MATCH(V_, F_, S_, W_) \
    if (t.vec == V_ && t.lanes == F_ && t.steps == S_ && t.waves == W_) return true;
    if (family == 0) { MOGT_DIAG_F32_TILES(MOGT_MATCH) }
    if (family == 1) { MOGT_DIAG_BF16_TILES(MOGT_MATCH) }
    if (family == 2) { MOGT_COUPLED_TILES(MOGT_MATCH) }
    if (family == 3) { MOGT_COUPLED_REV_TILES(MOGT_MATCH) }
#undef MOGT_MATCH
    return false;
}

namespace {

bool dtype_ok(int d) { return d == MOGT_F32 || d == MOGT_BF16; }

// Default tile (measured on MI355X, B = 1, D = 768, L = 8k..32k): chunks of
// 512 steps x 64 features, rows of 256 B.  fp32: f32_tile; bf16: four
// features per lane, 16 lanes per row (the packed stash holds both inputs in
// one register per element).  Vectors need D to be a multiple of the vector
// and aligned pointers; short problems fall back to shorter chunks so the
// grid still covers the GPU.
DiagTile default_tile(int64_t B, int64_t L, int64_t D, bool bf16_in, int align_elems) {
    if (bf16_in) {
        static const TileChoice v4[] = {{{4, 16, 16, 8}, 128}, {{2, 32, 8, 16}, 128}, {{1, 64, 8, 16}, 0}};
        static const TileChoice v2[] = {{{2, 32, 16, 8}, 128}, {{2, 32, 8, 16}, 128}, {{1, 64, 8, 16}, 0}};
        static const TileChoice v1[] = {{{1, 64, 32, 16}, 128}, {{1, 64, 16, 16}, 128}, {{1, 64, 8, 16}, 0}};
        if (D % 4 == 0 && align_elems % 4 == 0) return pick_tile(B, L, D, v4, 3);
        if (D % 2 == 0 && align_elems % 2 == 0) return pick_tile(B, L, D, v2, 3);
        return pick_tile(B, L, D, v1, 3);
    }
    return f32_tile(B, L, D, D % 2 == 0 && align_elems % 2 == 0);
}

// rev: the reverse-time recurrence h_t = a_{t+1} h_{t+1} + b_t (fp32 only).
int run_scan(const void* a, const void* b, void* h, void* aprefix, int64_t B, int64_t L,
             int64_t D, int in_dtype, int out_dtype, const DiagTile& t, void* ws, size_t ws_bytes,
             void* stream, bool rev = false) {
    clear_error();
    if (B < 0 || L < 0 || D < 0) return set_error(MOGT_E_INVALID, "negative size");
    if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype))
        return set_error(MOGT_E_INVALID, "unsupported dtype code");
    if (B == 0 || L == 0 || D == 0) return MOGT_OK;
    if (!a || !b || !h) return set_error(MOGT_E_INVALID, "null tensor pointer");
    const int family = in_dtype == MOGT_BF16 ? 1 : 0;
    if (!diag_tile_compiled(family, t))
        return set_error(MOGT_E_INVALID, "diag scan: tile (%d,%d,%d,%d) not compiled", t.vec,
                         t.lanes, t.steps, t.waves);
    if (D % t.vec != 0)
        return set_error(MOGT_E_INVALID, "features %lld not a multiple of vec %d", (long long)D,
                         t.vec);
    DiagParams prm{};
    const int rc = diag_prepare(prm, B, L, D, t, ws, ws_bytes);
    if (rc) return rc;
    prm.a = a;
    prm.b = b;
    prm.h = h;
    prm.aprefix = aprefix;
    prm.R = 1;
    prm.C = 1;
    prm.damping = 1.0f;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool pre = aprefix != nullptr;
    if (rev) return diag_run_rev(prm, t, st);
    return family == 1 ? diag_run_bf16in(prm, t, out_dtype, pre, st)
                       : diag_run_f32in(prm, t, out_dtype, pre, st);
}

// Largest vector width (in elements, 4, 2 or 1) every pointer is aligned to.
int common_alignment(const void* a, const void* b, const void* h, const void* p, int in_dtype,
                     int out_dtype) {
    const uintptr_t ie = in_dtype == MOGT_BF16 ? 2 : 4, oe = out_dtype == MOGT_BF16 ? 2 : 4;
    for (int v : {4, 2}) {
        auto ok = [&](const void* ptr, uintptr_t es) {
            return ptr == nullptr || reinterpret_cast<uintptr_t>(ptr) % (es * v) == 0;
        };
        if (ok(a, ie) && ok(b, ie) && ok(h, oe) && ok(p, oe)) return v;
    }
    return 1;
}

// ---------------------------------------------------------------------------
// Scratch of the no-allocation entry point: the look-back workspace lives in a
// file-scope device array, one copy per GPU, held until the process ends.
// Host code never passes `scratch` itself (in host code it names a host-side
// stand-in); it passes the device address that hipGetSymbolAddress returned
// for the current device.
// ---------------------------------------------------------------------------
constexpr size_t NOALLOC_SCRATCH_BYTES = size_t(8) << 20;
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

constexpr int NOALLOC_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[NOALLOC_MAX_DEVICES] = {};

__global__ __launch_bounds__(256) void clear_scratch_kernel(uint4* p, size_t n) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// Device address of the current device's scratch; on the first call for a
// device it is looked up and the whole array is cleared on `stream` (a fill
// kernel, so the set-up is also valid inside a captured graph).
int noalloc_scratch(hipStream_t stream, void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(MOGT_E_LAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES)
        return set_error(MOGT_E_INVALID, "device %d beyond the %d the library tracks", dev,
                         NOALLOC_MAX_DEVICES);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return set_error(MOGT_E_LAUNCH, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        const size_t n = NOALLOC_SCRATCH_BYTES / sizeof(uint4);
        hipLaunchKernelGGL(clear_scratch_kernel, dim3(1024), dim3(256), 0, stream,
                           static_cast<uint4*>(ptr), n);
        const int rc = check_launch("clear_scratch_kernel");
        if (rc) return rc;
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return MOGT_OK;
}

}  // namespace
}  // namespace mogt

using namespace mogt;

extern "C" size_t mogt_diag_scan_workspace_bytes_cfg(int64_t batch, int64_t length,
                                                     int64_t features, int vec, int lanes,
                                                     int steps, int waves) {
    if (batch <= 0 || length <= 0 || features <= 0 || vec <= 0 || steps <= 0 || waves <= 0 ||
        (lanes != 16 && lanes != 32 && lanes != 64))
        return WS_HDR_BYTES;
    return diag_geometry(batch, length, features, DiagTile{vec, lanes, steps, waves}).bytes;
}

extern "C" size_t mogt_diag_scan_workspace_bytes(int64_t batch, int64_t length, int64_t features,
                                                 int in_dtype) {
    if (batch <= 0 || length <= 0 || features <= 0) return WS_HDR_BYTES;
    // Largest requirement over the tiles the entry point may pick.
    const bool bf = in_dtype == MOGT_BF16;
    size_t best = 0;
    for (int al : {4, 2, 1}) {
        const size_t n = diag_geometry(batch, length, features,
                                       default_tile(batch, length, features, bf, al)).bytes;
        best = n > best ? n : best;
    }
    return best;
}

extern "C" int mogt_diag_scan_fwd_cfg(const void* a, const void* b, void* h, void* a_prefix,
                                      int64_t batch, int64_t length, int64_t features,
                                      int in_dtype, int out_dtype, int vec, int lanes, int steps,
                                      int waves, void* workspace, size_t workspace_bytes,
                                      void* stream) {
    return run_scan(a, b, h, a_prefix, batch, length, features, in_dtype, out_dtype,
                    DiagTile{vec, lanes, steps, waves}, workspace, workspace_bytes, stream);
}

extern "C" int mogt_diag_scan_fwd(const void* a, const void* b, void* h, void* a_prefix,
                                  int64_t batch, int64_t length, int64_t features, int in_dtype,
                                  int out_dtype, void* workspace, size_t workspace_bytes,
                                  void* stream) {
    if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) {
        clear_error();
        return set_error(MOGT_E_INVALID, "unsupported dtype code");
    }
    const int al = common_alignment(a, b, h, a_prefix, in_dtype, out_dtype);
    const DiagTile t = default_tile(batch, length, features, in_dtype == MOGT_BF16, al);
    return run_scan(a, b, h, a_prefix, batch, length, features, in_dtype, out_dtype, t, workspace,
                    workspace_bytes, stream);
}

extern "C" int mogt_diag_scan_rev_fwd(const void* a, const void* b, void* h, int64_t batch,
                                      int64_t length, int64_t features, void* workspace,
                                      size_t workspace_bytes, void* stream) {
    const int al = common_alignment(a, b, h, nullptr, MOGT_F32, MOGT_F32);
    const DiagTile t = default_tile(batch, length, features, false, al);
    return run_scan(a, b, h, nullptr, batch, length, features, MOGT_F32, MOGT_F32, t, workspace,
                    workspace_bytes, stream, true);
}

extern "C" int mogt_diag_scan_tiles(int family, int* out, int max_tiles) {
    static const DiagTile f32[] = {
#define MOGT_T(V_, F_, S_, W_) DiagTile{V_, F_, S_, W_},
        MOGT_DIAG_F32_TILES(MOGT_T)
    };
    static const DiagTile b16[] = {MOGT_DIAG_BF16_TILES(MOGT_T)};
    static const DiagTile cpl[] = {MOGT_COUPLED_TILES(MOGT_T)};
    static const DiagTile crev[] = {MOGT_COUPLED_REV_TILES(MOGT_T)};
#undef MOGT_T
    const DiagTile* list = family == 0 ? f32 : family == 1 ? b16 : family == 2 ? cpl : family == 3 ? crev : nullptr;
    const int n = family == 0   ? static_cast<int>(sizeof(f32) / sizeof(f32[0]))
                  : family == 1 ? static_cast<int>(sizeof(b16) / sizeof(b16[0]))
                  : family == 2 ? static_cast<int>(sizeof(cpl) / sizeof(cpl[0]))
                  : family == 3 ? static_cast<int>(sizeof(crev) / sizeof(crev[0]))
                                : 0;
    for (int i = 0; i < n && i < max_tiles && out; ++i) {
        out[4 * i] = list[i].vec;
        out[4 * i + 1] = list[i].lanes;
        out[4 * i + 2] = list[i].steps;
        out[4 * i + 3] = list[i].waves;
    }
    return n;
}

extern "C" int mogt_diag_scan_fwd_noalloc(const void* a, const void* b, void* h, void* a_prefix,
                                          int64_t batch, int64_t length, int64_t features,
                                          int in_dtype, int out_dtype, void* stream) {
    clear_error();
    if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype))
        return set_error(MOGT_E_INVALID, "unsupported dtype code");
    if (batch < 0 || length < 0 || features < 0) return set_error(MOGT_E_INVALID, "negative size");
    if (batch == 0 || length == 0 || features == 0) return MOGT_OK;
    const int al = common_alignment(a, b, h, a_prefix, in_dtype, out_dtype);
    const DiagTile t = default_tile(batch, length, features, in_dtype == MOGT_BF16, al);
    const size_t need = diag_geometry(batch, length, features, t).bytes;
    if (need > NOALLOC_SCRATCH_BYTES)
        return set_error(MOGT_E_INVALID,
                         "diag scan of %lld x %lld x %lld needs %zu bytes of look-back scratch; the "
                         "no-allocation entry point holds %zu (use mogt_diag_scan_fwd with a workspace)",
                         (long long)batch, (long long)length, (long long)features, need,
                         NOALLOC_SCRATCH_BYTES);
    hipStream_t st = static_cast<hipStream_t>(stream);
    void* ws = nullptr;
    const int rc = noalloc_scratch(st, &ws);
    if (rc) return rc;
    return run_scan(a, b, h, a_prefix, batch, length, features, in_dtype, out_dtype, t, ws,
                    NOALLOC_SCRATCH_BYTES, stream);
}
