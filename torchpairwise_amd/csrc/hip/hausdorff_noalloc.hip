// Allocation-free variant of tpw_directed_hausdorff: the same kernels with their scratch in a
// static device array.  The array lives in this file's own code object, which the runtime loads
// onto a GPU only when this entry point first looks the array up there, so processes that never
// call the entry point hold no copy of it.  Every GPU the entry point runs on holds its own copy
// (at its own address) until the process ends.  Calls on one GPU share it; they are
// serialised through one event per device: each call's stream waits for the previous call's
// work (on whatever stream it ran) before its own, and records the event after it.  The kernels
// initialise every part of the scratch they read (tpw_directed_hausdorff's preset fill), so the
// previous call's contents never leak into a result.
#include <mutex>

#include "common.hpp"

namespace tpw {
namespace {

constexpr size_t kNoAllocScratchBytes = (size_t)TPW_HAUSDORFF_NOALLOC_SCRATCH_MIB << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

struct DeviceState {
    void *scratch = nullptr;  // the device address of `scratch` on this device
    hipEvent_t done = nullptr;  // recorded after each call's work
};

constexpr int kMaxDevices = 64;
std::mutex g_mu;
DeviceState g_dev[kMaxDevices];

// Set-up, once per device with that device current: the device address of `scratch` (the
// array's name is only a host-side stand-in in host code) and the serialising event.
int device_state(DeviceState **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        set_error("directed_hausdorff_noalloc: no usable current device (%s)", hipGetErrorString(e));
        return TPW_ERR_LAUNCH;
    }
    DeviceState &st = g_dev[dev];
    if (st.scratch == nullptr) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            set_error("directed_hausdorff_noalloc: hipGetSymbolAddress failed on device %d: %s", dev,
                      hipGetErrorString(e));
            return TPW_ERR_LAUNCH;
        }
        hipEvent_t ev = nullptr;
        e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (e != hipSuccess) {
            set_error("directed_hausdorff_noalloc: hipEventCreate failed on device %d: %s", dev,
                      hipGetErrorString(e));
            return TPW_ERR_LAUNCH;
        }
        st.scratch = p;
        st.done = ev;
    }
    *out = &st;
    return TPW_OK;
}

}  // namespace
}  // namespace tpw

extern "C" int tpw_directed_hausdorff_noalloc(const float *x1, const float *x2, int64_t batch, int64_t b1,
                                              int64_t p1, int64_t b2, int64_t p2, int64_t d,
                                              const int64_t *perm1, const int64_t *perm2, float *out,
                                              int64_t *idx1, int64_t *idx2, void *stream) {
    TPW_REQUIRE(batch >= 0 && b1 >= 0 && b2 >= 0 && p1 >= 0 && p2 >= 0 && d >= 0, "invalid sizes");
    const size_t need = tpw_hausdorff_workspace_size(batch, b1, p1, b2, p2, d);
    TPW_REQUIRE(need <= tpw::kNoAllocScratchBytes,
                "directed_hausdorff_noalloc: these sizes need %zu bytes of scratch, more than the %zu-byte "
                "static buffer; call tpw_directed_hausdorff with a workspace instead",
                need, tpw::kNoAllocScratchBytes);
    std::lock_guard<std::mutex> lock(tpw::g_mu);  // one host thread enqueues at a time
    tpw::DeviceState *st = nullptr;
    int rc = tpw::device_state(&st);
    if (rc != TPW_OK) return rc;
    hipStream_t s = tpw::as_stream(stream);
    // Under graph capture the order of the graph's nodes is the caller's to give: an event
    // recorded outside the capture cannot be waited on inside it.
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cap) != hipSuccess) cap = hipStreamCaptureStatusNone;
    const bool serialise = cap == hipStreamCaptureStatusNone;
    if (serialise && hipStreamWaitEvent(s, st->done, 0) != hipSuccess) {
        tpw::set_error("directed_hausdorff_noalloc: hipStreamWaitEvent failed");
        return TPW_ERR_LAUNCH;
    }
    rc = tpw_directed_hausdorff(x1, x2, batch, b1, p1, b2, p2, d, perm1, perm2, out, idx1, idx2, st->scratch,
                                stream);
    if (rc != TPW_OK) return rc;
    if (serialise && hipEventRecord(st->done, s) != hipSuccess) {
        tpw::set_error("directed_hausdorff_noalloc: hipEventRecord failed");
        return TPW_ERR_LAUNCH;
    }
    return TPW_OK;
}
