// Host-side HIP helpers of the C ABI: error mapping, device queries and the
// status word's host memory.
#include <string.h>

#include "abi_internal.h"

namespace ssl {

constexpr size_t kStatusWordBytes = 256;

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return SSL_OK;
  return fail(SSL_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

int device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
      v = 256;
    cache[dev] = v;
  }
  return cache[dev];
}

// The checked build's status word for calls that pass none (the in-place op,
// which never waits): a file-scope device word, used through the address
// hipGetSymbolAddress gives with the device current (the name is a host-side
// stand-in in host code), once per device.
#if SSL_DEVICE_CHECKS
static __device__ unsigned long long check_word;
#endif

unsigned long long* check_word_ptr() {
#if SSL_DEVICE_CHECKS
  static unsigned long long* cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  if (!cache[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(check_word)) == hipSuccess) cache[dev] = (unsigned long long*)p;
  }
  return cache[dev];
#else
  return nullptr;
#endif
}

}  // namespace ssl

using namespace ssl;

extern "C" {

int64_t ssl_debug_check_word(void) {
#if SSL_DEVICE_CHECKS
  unsigned long long v = 0, zero = 0;
  if (hipMemcpyFromSymbol(&v, HIP_SYMBOL(check_word), sizeof v, 0, hipMemcpyDeviceToHost) != hipSuccess)
    return -1;
  if (v != 0 &&
      hipMemcpyToSymbol(HIP_SYMBOL(check_word), &zero, sizeof zero, 0, hipMemcpyHostToDevice) != hipSuccess)
    return -1;
  return (int64_t)v;
#else
  return 0;
#endif
}

int32_t ssl_device_checks(void) { return SSL_DEVICE_CHECKS; }

int ssl_status_word_alloc(void** host_ptr, void** device_ptr) {
  clear_error();
  if (!host_ptr || !device_ptr) return fail(SSL_ERR_INVALID, "status word: null output pointer");
  void* h = nullptr;
  // coherent (fine-grained): a kernel's store reaches host memory without a
  // cache write-back, so the host sees it as soon as it lands
  if (int rc = check_hip(hipHostMalloc(&h, kStatusWordBytes,
                                       hipHostMallocPortable | hipHostMallocMapped |
                                           hipHostMallocCoherent),
                         "status word allocation"))
    return rc;
  memset(h, 0, kStatusWordBytes);
  void* d = nullptr;
  if (int rc = check_hip(hipHostGetDevicePointer(&d, h, 0), "status word device address")) {
    (void)hipHostFree(h);
    return rc;
  }
  *host_ptr = h;
  *device_ptr = d;
  return SSL_OK;
}

}  // extern "C"
