// hx_runtime.hip — device selection, allocation, copies and error reporting for the C ABI.
#include <cctype>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "hx_common.h"
#include "hx_once.h"
#include <tuple>

namespace hx {

namespace {
thread_local char g_last_error[1024] = {0};
}

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_last_error[0] = 0; }

bool grant_dynamic_lds(const void* fn, size_t dyn_bytes, size_t static_bytes) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    static OnceMap<std::tuple<const void*, int, size_t>, bool> memo;
    return memo.get(std::make_tuple(fn, dev, dyn_bytes), [&] {
        int v = 0;
        const bool ok = hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess &&
                        (size_t)v >= dyn_bytes + static_bytes &&
                        hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)dyn_bytes) ==
                            hipSuccess;
        (void)hipGetLastError();  // a refusal is an answer, not a pending error
        return ok;
    });
}

int device_cus() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    static OnceMap<int, int> memo;
    return memo.get(dev, [&] {
        int v = 0;
        return (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) ? v
                                                                                                              : 256;
    });
}

}  // namespace hx

extern "C" {

int hx_version(void) { return (0 << 16) | (1 << 8) | 0; }

const char* hx_last_error(void) { return hx::g_last_error; }

int hx_init(int device) {
    int n = 0;
    HX_HIP_CHECK(hipGetDeviceCount(&n));
    HX_REQUIRE(device >= 0 && device < n, HX_ERR_INVALID_INPUT,
               "hx_init: device %d out of range (%d visible)", device, n);
    HX_HIP_CHECK(hipSetDevice(device));
    if (int rc = hx::scan_scratch_setup(nullptr)) return rc;
    hx::clear_error();
    return HX_OK;
}

int hx_malloc(void** ptr, size_t bytes) {
    HX_REQUIRE(ptr != nullptr, HX_ERR_INVALID_INPUT, "hx_malloc: null out-pointer");
    *ptr = nullptr;
    if (bytes == 0) return HX_OK;
    hipError_t e = hipMalloc(ptr, bytes);
    if (e != hipSuccess) {
        *ptr = nullptr;
        return hx::set_error(HX_ERR_ALLOCATION, "hx_malloc(%zu bytes): %s", bytes,
                             hipGetErrorString(e));
    }
    return HX_OK;
}

int hx_free(void* ptr) {
    if (ptr == nullptr) return HX_OK;
    HX_HIP_CHECK(hipFree(ptr));
    return HX_OK;
}

int hx_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return HX_OK;
    HX_REQUIRE(dst && src, HX_ERR_INVALID_INPUT, "hx_memcpy_h2d: null pointer");
    HX_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return HX_OK;
}

int hx_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return HX_OK;
    HX_REQUIRE(dst && src, HX_ERR_INVALID_INPUT, "hx_memcpy_d2h: null pointer");
    HX_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return HX_OK;
}

int hx_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return HX_OK;
    HX_REQUIRE(dst && src, HX_ERR_INVALID_INPUT, "hx_memcpy_d2d: null pointer");
    HX_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, hx::as_stream(stream)));
    return HX_OK;
}

int hx_sync(void) {
    HX_HIP_CHECK(hipDeviceSynchronize());
    return HX_OK;
}

int hx_device_info(int device, int* compute_units, size_t* memory_bytes) {
    hipDeviceProp_t prop;
    HX_HIP_CHECK(hipGetDeviceProperties(&prop, device));
    if (compute_units) *compute_units = prop.multiProcessorCount;
    if (memory_bytes) *memory_bytes = prop.totalGlobalMem;
    return HX_OK;
}

int hx_device_utilization(int device, double* busy_fraction) {
    HX_REQUIRE(busy_fraction != nullptr, HX_ERR_INVALID_INPUT, "hx_device_utilization: NULL output");
    *busy_fraction = 0.0;
    char bus[64] = {0};
    HX_HIP_CHECK(hipDeviceGetPCIBusId(bus, (int)sizeof(bus), device));
    for (char* c = bus; *c; ++c) *c = (char)tolower((unsigned char)*c);  // sysfs names are lower case
    char path[160];
    snprintf(path, sizeof(path), "/sys/bus/pci/devices/%s/gpu_busy_percent", bus);
    FILE* f = fopen(path, "r");
    HX_REQUIRE(f != nullptr, HX_ERR_UNSUPPORTED, "hx_device_utilization: %s is not readable", path);
    int pct = -1;
    const int got = fscanf(f, "%d", &pct);
    fclose(f);
    HX_REQUIRE(got == 1 && pct >= 0 && pct <= 100, HX_ERR_BACKEND,
               "hx_device_utilization: unexpected contents of %s", path);
    *busy_fraction = pct / 100.0;
    return HX_OK;
}

}  // extern "C"
