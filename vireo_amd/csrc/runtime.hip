// Library state: device selection, error text, and the per-device workspace
// that kernels use for intermediates (router partials, expert activations).
#include <hip/hip_runtime.h>
#include <errno.h>
#include <stdio.h>
#include <string.h>
#include "common.h"
#include "vireo_hip.h"

namespace {
constexpr int kMaxDev = 16;
struct DevState {
    void *ws = nullptr;
    size_t ws_bytes = 0;
    unsigned *ctr = nullptr;
    int ctr_n = 0;
    void *red = nullptr;
    size_t red_bytes = 0;
    int cus = 0;
};
DevState g_dev[kMaxDev];
thread_local char g_err[256];

int cur_dev() {
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= kMaxDev) return -1;
    return d;
}
}  // namespace

VhLaunchTiming g_vh_timing = {nullptr, nullptr};

int vh_check(hipError_t e) {
    if (e == hipSuccess) return 0;
    snprintf(g_err, sizeof g_err, "HIP error %d: %s", int(e), hipGetErrorString(e));
    return -EIO;
}

int vh_finish(hipStream_t s, int rc) {
    if (rc) return rc;
    int e = vh_check(hipGetLastError());
    if (e) return e;
    if (!s) return vh_check(hipStreamSynchronize(nullptr));
    return 0;
}

int vh_num_cus() {
    int d = cur_dev();
    if (d < 0) return 256;
    if (!g_dev[d].cus) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, d) != hipSuccess || n <= 0) n = 256;
        g_dev[d].cus = n;
    }
    return g_dev[d].cus;
}

// Grow-only scratch. Growing synchronises the device first, because earlier
// enqueued kernels may still read the old buffer.
int vh_device_workspace(size_t bytes, void **out) {
    int d = cur_dev();
    if (d < 0) return -ENODEV;
    DevState &st = g_dev[d];
    if (bytes > st.ws_bytes) {
        size_t nb = bytes < (size_t(1) << 20) ? (size_t(1) << 20) : bytes;
        nb = (nb + 0xffff) & ~size_t(0xffff);
        if (st.ws) {
            if (int rc = vh_check(hipDeviceSynchronize())) return rc;
            if (int rc = vh_check(hipFree(st.ws))) return rc;
            st.ws = nullptr;
            st.ws_bytes = 0;
        }
        if (int rc = vh_check(hipMalloc(&st.ws, nb))) return rc == -EIO ? -ENOMEM : rc;
        st.ws_bytes = nb;
    }
    *out = st.ws;
    return 0;
}

// Arrival counters for "last block finishes the job" kernels. They are zeroed
// once here; every kernel that uses one returns it to zero before it exits.
int vh_counters(int n, unsigned **out) {
    int d = cur_dev();
    if (d < 0) return -ENODEV;
    DevState &st = g_dev[d];
    if (n > st.ctr_n) {
        int nn = n < 4096 ? 4096 : n;
        if (st.ctr) {
            if (int rc = vh_check(hipDeviceSynchronize())) return rc;
            if (int rc = vh_check(hipFree(st.ctr))) return rc;
            st.ctr = nullptr;
            st.ctr_n = 0;
        }
        if (int rc = vh_check(hipMalloc(&st.ctr, sizeof(unsigned) * nn))) return rc;
        if (int rc = vh_check(hipMemset(st.ctr, 0, sizeof(unsigned) * nn))) return rc;
        if (int rc = vh_check(hipDeviceSynchronize())) return rc;
        st.ctr_n = nn;
    }
    *out = st.ctr;
    return 0;
}

// Grow-only scratch for the partial results of multi-workgroup reductions
// (argmax), separate from the MoE workspace.
int vh_reduce_scratch(size_t bytes, void **out) {
    int d = cur_dev();
    if (d < 0) return -ENODEV;
    DevState &st = g_dev[d];
    if (bytes > st.red_bytes) {
        const size_t nb = (bytes + 0xffff) & ~size_t(0xffff);
        if (st.red) {
            if (int rc = vh_check(hipDeviceSynchronize())) return rc;
            if (int rc = vh_check(hipFree(st.red))) return rc;
            st.red = nullptr;
            st.red_bytes = 0;
        }
        if (int rc = vh_check(hipMalloc(&st.red, nb))) return rc;
        st.red_bytes = nb;
    }
    *out = st.red;
    return 0;
}

extern "C" int vireo_hip_init(int device) {
    int n = 0;
    if (int rc = vh_check(hipGetDeviceCount(&n))) return rc;
    if (device < 0 || device >= n || device >= kMaxDev) return -EINVAL;
    return vh_check(hipSetDevice(device));
}

extern "C" const char *vireo_hip_strerror(int err) {
    if (err == -EIO && g_err[0]) return g_err;
    switch (err) {
    case 0: return "ok";
    case -EINVAL: return "invalid argument or unsupported ggml type";
    case -ENOMEM: return "out of device or host memory";
    case -ENODEV: return "no HIP device";
    case -ENOSPC: return "ExpertStore capacity below the experts that must stay resident";
    case -E2BIG: return "size exceeds a kernel limit";
    case -EIO: return "HIP runtime or I/O failure";
    default: return strerror(err < 0 ? -err : err);
    }
}

extern "C" int vireo_type_block(uint32_t t, int *be, int *bb) {
    if (!be || !bb) return -EINVAL;
    switch (t) {
    case VT_F32:  *be = 1;   *bb = 4;   return 0;
    case VT_F16:  *be = 1;   *bb = 2;   return 0;
    case VT_Q8_0: *be = 32;  *bb = 34;  return 0;
    case VT_Q4_0: *be = 32;  *bb = 18;  return 0;
    case VT_Q5_0: *be = 32;  *bb = 22;  return 0;
    case VT_Q4_K: *be = 256; *bb = 144; return 0;
    case VT_Q6_K: *be = 256; *bb = 210; return 0;
    default: return -EINVAL;
    }
}
