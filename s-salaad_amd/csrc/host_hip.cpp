// Host-side HIP helpers of the C ABI: error mapping and device queries.
#include "abi_internal.h"

namespace ssl {

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

}  // namespace ssl
