// C ABI plumbing shared by all scan entry points: per-thread error text,
// launch checking and the ABI version.
#include <atomic>
#include <cstdarg>
#include <cstdio>

#include "common.h"

namespace mogt {

namespace {
thread_local char g_last_error[512] = {0};
}

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_last_error[0] = '\0'; }

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(MOGT_E_LAUNCH, "%s: %s", what, hipGetErrorString(e));
    return MOGT_OK;
}

namespace {
constexpr int MAX_DEVICES = 64;
std::atomic<int> g_cus[MAX_DEVICES];   // 0: not queried yet
}

int device_cu_count(int& cus) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(MOGT_E_LAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
    if (dev >= 0 && dev < MAX_DEVICES && (cus = g_cus[dev].load(std::memory_order_relaxed)) > 0) return MOGT_OK;
    int n = 0;
    e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return set_error(MOGT_E_LAUNCH, "CU count query: %s", hipGetErrorString(e));
    cus = n > 0 ? n : 1;
    if (dev >= 0 && dev < MAX_DEVICES) g_cus[dev].store(cus, std::memory_order_relaxed);
    return MOGT_OK;
}

}  // namespace mogt

extern "C" const char* mogt_last_error(void) { return mogt::g_last_error; }

extern "C" int mogt_abi_version(void) { return 11; }

// "name:sha256[:12];..." of the sources and compiler flags this library was
// built from, passed in by the build script (mogt_amd/_build.py).
#ifndef MOGT_BUILD_MANIFEST
#define MOGT_BUILD_MANIFEST ""
#endif
extern "C" const char* mogt_build_manifest(void) { return MOGT_BUILD_MANIFEST; }

extern "C" int mogt_workspace_faults(const void* workspace, size_t workspace_bytes, uint32_t* count,
                                     void* stream) {
    mogt::clear_error();
    if (!workspace || !count) return mogt::set_error(MOGT_E_INVALID, "null workspace or count pointer");
    if (workspace_bytes < mogt::WS_HDR_BYTES)
        return mogt::set_error(MOGT_E_WORKSPACE, "workspace of at least %zu bytes expected, got %zu",
                               mogt::WS_HDR_BYTES, workspace_bytes);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const char* hdr = static_cast<const char*>(workspace);
    // header word 3: bounded waits that gave up (common.h)
    hipError_t e = hipMemcpyAsync(count, hdr + 3 * sizeof(uint32_t), sizeof(uint32_t),
                                  hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess)
        return mogt::set_error(MOGT_E_LAUNCH, "mogt_workspace_faults: %s", hipGetErrorString(e));
    return MOGT_OK;
}
