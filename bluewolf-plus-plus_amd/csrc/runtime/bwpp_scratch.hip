// Device-resident scratch memory for libbwpp_hip's allocation-free entry
// point (bwpp_hip_dispatch_attention_grad_noalloc).  The array below is a
// file-scope __device__ variable of this code object: each GPU the library
// runs on holds its own copy, at its own address, from the first lookup
// until the process ends.  Host code never uses the array's name as an
// address (on the host it is only a stand-in for the symbol): it asks HIP
// for the device address once per device and passes that pointer to the
// kernels, as the other entry points pass the handle's workspace.
//
// Every call on one GPU shares that GPU's copy, and a call leaves its
// contents behind: calls that overlap on one GPU (two streams, two
// handles, two threads) race on it.
#include <hip/hip_runtime.h>

#include <mutex>
#include <vector>

#include "internal.h"

static __device__ __align__(256) unsigned char scratch[BWPP_HIP_NOALLOC_SCRATCH_BYTES];

namespace {

struct DeviceScratch {
  bool looked_up = false;
  hipError_t err = hipSuccess;
  void *ptr = nullptr;
};

std::mutex g_mu;
std::vector<DeviceScratch> g_devices;

}  // namespace

// Device address of `device`'s scratch array; the caller has made `device`
// current.  The lookup runs once per device and its result (address or
// error) is kept for the life of the process.
BwppHipStatus bwpp_hip_scratch_setup(int device, void **ptr, const char **why) {
  std::lock_guard<std::mutex> lock(g_mu);
  if (device < 0) return BWPP_HIP_ERR_INVALID_ARG;
  if ((size_t)device >= g_devices.size()) g_devices.resize((size_t)device + 1);
  DeviceScratch &d = g_devices[(size_t)device];
  if (!d.looked_up) {
    void *p = nullptr;
    d.err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    d.ptr = d.err == hipSuccess ? p : nullptr;
    if (d.err != hipSuccess) (void)hipGetLastError();
    d.looked_up = true;
  }
  *ptr = d.ptr;
  if (why) *why = d.err == hipSuccess ? "" : hipGetErrorString(d.err);
  return d.ptr ? BWPP_HIP_OK : BWPP_HIP_ERR_HIP;
}
