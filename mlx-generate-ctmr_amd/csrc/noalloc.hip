// ctmr_conv3d_noalloc: ctmr_conv3d with its workspace in a library-owned
// device array instead of a caller buffer, for callers that cannot allocate
// device memory (code under HIP graph capture, tight serving loops, harnesses
// that forbid hipMalloc).  The array is a file-scope __device__ variable: each
// GPU the library runs on holds its own copy, allocated when this code object
// is loaded on that device and kept until the process ends.  Its device
// address is looked up once per device (hipGetSymbolAddress, with that device
// current) and that pointer -- never the variable's host-side name -- is what
// the kernels receive.  Nothing here allocates or frees device memory.
//
// Ordering: every call on a device shares that device's array, so calls are
// chained through one per-device event (created once, at the same set-up as
// the address lookup): a call makes its stream wait for the event, enqueues
// its kernels, then records the event on its stream, all under a host lock.
// Calls from several streams or host threads therefore run one after another
// on the GPU in the order the host issued them.  Work enqueued under stream
// capture is not chained (a captured graph orders its own nodes; replays of
// several such graphs on different streams must be ordered by the caller).
#include <mutex>

#include "ctmr_common.hpp"

namespace {

constexpr size_t kScratchBytes = CTMR_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

// Workspace of every ctmr_conv3d_noalloc call on this device: the padded input
// copy, split partial planes or tap columns of the conv being run.  Kernels
// write every byte they later read, so nothing has to start at zero.
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

struct DeviceScratch {
  void* ptr = nullptr;           // device address of `scratch` on this device, null until looked up
  hipEvent_t last = nullptr;     // recorded after each chained call's kernels
  bool recorded = false;         // `last` has been recorded at least once
};

std::mutex g_scratch_lock;  // guards g_dev and serialises wait -> launch -> record
DeviceScratch g_dev[kMaxDevices];

// The device `stream` belongs to; it must be the current device (the symbol
// lookup and the kernels' launch resolve against the current device).
int stream_device(hipStream_t stream, int* out) {
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess || cur < 0 || cur >= kMaxDevices)
    return ctmr::fail(CTMR_E_LAUNCH, "ctmr_conv3d_noalloc: no current HIP device");
  if (stream) {
    int sdev = -1;
    const hipError_t e = hipStreamGetDevice(stream, &sdev);
    if (e != hipSuccess) {
      ctmr::set_error("ctmr_conv3d_noalloc: hipStreamGetDevice failed: %s", hipGetErrorString(e));
      return CTMR_E_INVALID;
    }
    if (sdev != cur) {
      ctmr::set_error("ctmr_conv3d_noalloc: the stream belongs to device %d but device %d is current; "
                      "make the stream's device current", sdev, cur);
      return CTMR_E_INVALID;
    }
  }
  *out = cur;
  return CTMR_OK;
}

// Per-device set-up, once per device with that device current: the scratch
// array's device address and the ordering event.  Caller holds g_scratch_lock.
int setup_device(int dev) {
  DeviceScratch& d = g_dev[dev];
  if (!d.ptr) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      ctmr::set_error("ctmr_conv3d_noalloc: hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
      return CTMR_E_LAUNCH;
    }
    d.ptr = ptr;
  }
  if (!d.last) {
    const hipError_t e = hipEventCreateWithFlags(&d.last, hipEventDisableTiming);
    if (e != hipSuccess) {
      d.last = nullptr;
      ctmr::set_error("ctmr_conv3d_noalloc: hipEventCreateWithFlags failed: %s", hipGetErrorString(e));
      return CTMR_E_LAUNCH;
    }
  }
  return CTMR_OK;
}

}  // namespace

extern "C" {

int ctmr_conv3d_noalloc(const ctmr_conv_desc* desc, const float* x, const void* packed, const float* bias,
                        const float* affine, const float* residual, float* y, void* stream) {
  const int64_t need = ctmr_conv3d_workspace_bytes(desc);
  if (need < 0) return (int)need;  // the descriptor's own error, message already set
  if (need > (int64_t)kScratchBytes) {
    ctmr::set_error("ctmr_conv3d_noalloc: this convolution needs %lld bytes of workspace, above the %lld-byte "
                    "scratch limit; use ctmr_conv3d with a caller workspace",
                    (long long)need, (long long)kScratchBytes);
    return CTMR_E_WORKSPACE;
  }
  const hipStream_t s = static_cast<hipStream_t>(stream);
  int dev = -1;
  int rc = stream_device(s, &dev);
  if (rc) return rc;
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &capture) != hipSuccess)
    return ctmr::fail(CTMR_E_LAUNCH, "ctmr_conv3d_noalloc: hipStreamIsCapturing failed");
  const bool chain = capture == hipStreamCaptureStatusNone;

  std::lock_guard<std::mutex> guard(g_scratch_lock);
  rc = setup_device(dev);
  if (rc) return rc;
  DeviceScratch& d = g_dev[dev];
  if (chain && d.recorded && hipStreamWaitEvent(s, d.last, 0) != hipSuccess)
    return ctmr::fail(CTMR_E_LAUNCH, "ctmr_conv3d_noalloc: hipStreamWaitEvent failed");
  rc = ctmr_conv3d(desc, x, packed, bias, affine, residual, y, d.ptr, kScratchBytes, stream);
  if (rc) return rc;
  if (chain) {
    if (hipEventRecord(d.last, s) != hipSuccess)
      return ctmr::fail(CTMR_E_LAUNCH, "ctmr_conv3d_noalloc: hipEventRecord failed");
    d.recorded = true;
  }
  return CTMR_OK;
}

}  // extern "C"
