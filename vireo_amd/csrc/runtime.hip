// Library state: device selection, error text, and the per-device workspace
// that kernels use for intermediates (router partials, expert activations).
#include <hip/hip_runtime.h>
#include <errno.h>
#include <stdio.h>
#include <string.h>
#include "common.h"
#include "route_kernels.h"
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
    hipStream_t copy = nullptr;   // expert page-in copies
    // pinned staging for small per-call transfers: two buffers used in turn
    void *host[2] = {nullptr, nullptr};
    size_t host_bytes[2] = {0, 0};
    hipEvent_t host_done[2] = {nullptr, nullptr};
    bool host_done_set[2] = {false, false};
    int host_next = 0;            // the buffer the next call takes
    int host_cur = 0;             // the buffer the current call took
    uint32_t *status = nullptr;   // sticky device status bits (VIREO_DECODE_TIMEOUT)
    LayerXchg *xchg = nullptr;    // the layer kernel's exchange area (zeroed once)
};
unsigned g_spin_limit = 1u << 18;
DevState g_dev[kMaxDev];
thread_local char g_err[256];

int cur_dev() {
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= kMaxDev) return -1;
    return d;
}
}  // namespace

VhLaunchTiming g_vh_timing = {nullptr, nullptr};
uint64_t *g_vh_stamps = nullptr;

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

// Grow-only device buffers. A buffer that is outgrown is not freed: kernels
// already enqueued and HIP graphs captured over earlier calls keep reading
// and writing the old one, so it stays allocated until the process ends.
// Each growth at least doubles, so the retired buffers together are no
// larger than the current one.
int grow_device(void **buf, size_t *bytes, size_t need, size_t floor) {
    if (need <= *bytes) return 0;
    size_t nb = need < floor ? floor : need;
    if (nb < 2 * *bytes) nb = 2 * *bytes;
    nb = (nb + 0xffff) & ~size_t(0xffff);
    void *p = nullptr;
    if (int rc = vh_check(hipMalloc(&p, nb))) return rc == -EIO ? -ENOMEM : rc;
    *buf = p;  // the old buffer is retired, not freed
    *bytes = nb;
    return 0;
}

int vh_device_workspace(size_t bytes, void **out) {
    int d = cur_dev();
    if (d < 0) return -ENODEV;
    DevState &st = g_dev[d];
    if (int rc = grow_device(&st.ws, &st.ws_bytes, bytes, size_t(1) << 20)) return rc;
    *out = st.ws;
    return 0;
}

// Arrival counters for "last block finishes the job" kernels. Every kernel
// that uses one returns it to zero before it exits; a new (larger) set is
// zeroed once here.
int vh_counters(int n, unsigned **out) {
    int d = cur_dev();
    if (d < 0) return -ENODEV;
    DevState &st = g_dev[d];
    if (n > st.ctr_n) {
        void *p = st.ctr;
        size_t b = size_t(st.ctr_n) * sizeof(unsigned);
        const size_t need = sizeof(unsigned) * size_t(n < 4096 ? 4096 : n);
        if (int rc = grow_device(&p, &b, need, need)) return rc;
        if (int rc = vh_check(hipMemset(p, 0, b))) return rc;
        if (int rc = vh_check(hipDeviceSynchronize())) return rc;
        st.ctr = static_cast<unsigned *>(p);
        st.ctr_n = int(b / sizeof(unsigned));
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
    if (int rc = grow_device(&st.red, &st.red_bytes, bytes, size_t(1) << 16)) return rc;
    *out = st.red;
    return 0;
}

int vh_copy_stream(hipStream_t *out) {
    int d = cur_dev();
    if (d < 0) return -ENODEV;
    DevState &st = g_dev[d];
    if (!st.copy && vh_check(hipStreamCreateWithFlags(&st.copy, hipStreamNonBlocking))) {
        st.copy = nullptr;
        return -EIO;
    }
    *out = st.copy;
    return 0;
}

int vh_host_staging(size_t bytes, void **out) {
    int d = cur_dev();
    if (d < 0) return -ENODEV;
    DevState &st = g_dev[d];
    const int i = st.host_next;
    if (st.host_done_set[i]) {
        if (int rc = vh_check(hipEventSynchronize(st.host_done[i]))) return rc;
        st.host_done_set[i] = false;
    }
    if (bytes > st.host_bytes[i]) {  // nothing reads the old buffer any more (waited above)
        if (st.host[i]) (void)hipHostFree(st.host[i]);
        st.host[i] = nullptr;
        st.host_bytes[i] = 0;
        const size_t nb = bytes < (size_t(1) << 20) ? (size_t(1) << 20) : 2 * bytes;
        if (vh_check(hipHostMalloc(&st.host[i], nb, 0))) { st.host[i] = nullptr; return -ENOMEM; }
        st.host_bytes[i] = nb;
    }
    st.host_cur = i;
    st.host_next = i ^ 1;
    *out = st.host[i];
    return 0;
}

int vh_host_staging_done(hipStream_t s) {
    int d = cur_dev();
    if (d < 0) return -ENODEV;
    DevState &st = g_dev[d];
    const int i = st.host_cur;
    if (!st.host_done[i] && vh_check(hipEventCreateWithFlags(&st.host_done[i], hipEventDisableTiming))) {
        st.host_done[i] = nullptr;
        return -EIO;
    }
    if (int rc = vh_check(hipEventRecord(st.host_done[i], s))) return rc;
    st.host_done_set[i] = true;
    return 0;
}

int vh_status_word(uint32_t **out) {
    int d = cur_dev();
    if (d < 0) return -ENODEV;
    DevState &st = g_dev[d];
    if (!st.status) {
        void *p = nullptr;
        if (int rc = vh_check(hipMalloc(&p, 256))) return rc == -EIO ? -ENOMEM : rc;
        if (int rc = vh_check(hipMemset(p, 0, 256))) return rc;
        if (int rc = vh_check(hipDeviceSynchronize())) return rc;
        st.status = static_cast<uint32_t *>(p);
    }
    *out = st.status;
    return 0;
}

unsigned vh_spin_limit() { return g_spin_limit; }

int vh_layer_xchg(LayerXchg **out) {
    int d = cur_dev();
    if (d < 0) return -ENODEV;
    DevState &st = g_dev[d];
    if (!st.xchg) {
        void *p = nullptr;
        if (int rc = vh_check(hipMalloc(&p, sizeof(LayerXchg)))) return rc == -EIO ? -ENOMEM : rc;
        if (int rc = vh_check(hipMemset(p, 0, sizeof(LayerXchg)))) return rc;
        if (int rc = vh_check(hipDeviceSynchronize())) return rc;
        st.xchg = static_cast<LayerXchg *>(p);
    }
    *out = st.xchg;
    return 0;
}

// Read and clear the sticky status bits after the stream's work is done.
int vh_take_status(hipStream_t s) {
    uint32_t *w = nullptr;
    if (int rc = vh_status_word(&w)) return rc;
    if (int rc = vh_check(hipStreamSynchronize(s))) return rc;
    uint32_t v = 0;
    if (int rc = vh_check(hipMemcpy(&v, w, 4, hipMemcpyDeviceToHost))) return rc;
    if (!v) return 0;
    if (int rc = vh_check(hipMemset(w, 0, 4))) return rc;
    if (int rc = vh_check(hipDeviceSynchronize())) return rc;
    return (v & VIREO_DECODE_TIMEOUT) ? -ETIMEDOUT : 0;
}

extern "C" int vireo_hip_status(void *stream) { return vh_take_status(static_cast<hipStream_t>(stream)); }

extern "C" int vireo_hip_set_spin_limit(unsigned polls) {
    g_spin_limit = polls;
    return 0;
}

extern "C" int vireo_hip_init(int device) {
    int n = 0;
    if (int rc = vh_check(hipGetDeviceCount(&n))) return rc;
    if (device < 0 || device >= n || device >= kMaxDev) return -EINVAL;
    if (int rc = vh_check(hipSetDevice(device))) return rc;
    return vh_noalloc_setup(nullptr);  // the static scratch's address on this device
}

extern "C" const char *vireo_hip_strerror(int err) {
    if (err == -EIO && g_err[0]) return g_err;
    switch (err) {
    case 0: return "ok";
    case -EINVAL: return "invalid argument or unsupported ggml type";
    case -ENOMEM: return "out of device or host memory";
    case -ENODEV: return "no HIP device";
    case -ENOSPC: return "ExpertStore capacity below the experts that must stay resident";
    case -E2BIG: return "size exceeds a kernel limit or the fixed scratch of an entry point that allocates nothing";
    case -EIO: return "HIP runtime or I/O failure";
    case -ETIMEDOUT: return "a grid-wide wait gave up (not every workgroup was resident): results invalid";
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
