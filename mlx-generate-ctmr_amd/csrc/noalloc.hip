// ctmr_conv3d_noalloc: ctmr_conv3d with its workspace in a library-owned
// device array instead of a caller buffer, for callers that cannot allocate
// device memory (code under HIP graph capture, tight serving loops, harnesses
// that forbid hipMalloc).  The array is a file-scope __device__ variable: each
// GPU the library runs on holds its own copy, allocated when this code object
// is loaded on that device and kept until the process ends.  Its device
// address is looked up once per device (hipGetSymbolAddress, with that device
// current) and that pointer -- never the variable's host-side name -- is what
// the kernels receive.  Nothing here allocates or frees.
#include <mutex>

#include "ctmr_common.hpp"

namespace {

constexpr size_t kScratchBytes = CTMR_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

// Workspace of every ctmr_conv3d_noalloc call on this device: the padded input
// copy, split partial planes or tap columns of the conv being run.  Kernels
// write every byte they later read, so nothing has to start at zero.
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_lock;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device, null until looked up

// Device address of this device's `scratch` (looked up on the first call on the device).
int scratch_for_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return ctmr::fail(CTMR_E_LAUNCH, "ctmr_conv3d_noalloc: no current HIP device");
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      ctmr::set_error("ctmr_conv3d_noalloc: hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
      return CTMR_E_LAUNCH;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
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
  void* ws = nullptr;
  const int rc = scratch_for_current_device(&ws);
  if (rc) return rc;
  return ctmr_conv3d(desc, x, packed, bias, affine, residual, y, ws, kScratchBytes, stream);
}

}  // extern "C"
