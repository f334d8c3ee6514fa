// The fused SLR linear without caller-provided scratch, for callers that may
// not allocate device memory (code under HIP graph capture, tight serving
// loops, hosts that forbid allocation).
//
// The scratch the fused kernel needs (int32 row counters, uint64 handshake
// words, and the byte workspace for the latent and split-row partials) lives in
// one file-scope device array of kNoAllocScratchBytes per GPU. Its device
// address comes from hipGetSymbolAddress, once per device, with that device
// current; host code uses only that address, never the array's name (which on
// the host is a stand-in, not a device pointer).
//
// Every call shares its GPU's array and the array keeps the last call's
// contents, so each call first clears the counters and handshake words it will
// use, with a fill kernel on the call's stream (no memset node, so the pair of
// launches can be captured in a graph). Calls that overlap on one GPU (other
// streams, other threads) race on the array.

#include <mutex>

#include "abi_internal.h"

namespace ssl {
namespace {

constexpr int64_t kNoAllocScratchBytes = 16LL << 20;
constexpr int64_t kNoAllocCounterBytes = 256LL << 10;   // 65,536 int32 row counters
constexpr int64_t kNoAllocExchangeBytes = 512LL << 10;  // 65,536 uint64 handshake words
constexpr int64_t kNoAllocWorkspaceBytes =
    kNoAllocScratchBytes - kNoAllocCounterBytes - kNoAllocExchangeBytes;

__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
unsigned char* g_scratch[kMaxDevices] = {};

// The array's address on the current device (looked up on the first call there).
int scratch_on_current_device(unsigned char** out) {
  int dev = -1;
  if (int rc = check_hip(hipGetDevice(&dev), "hipGetDevice")) return rc;
  if (dev < 0 || dev >= kMaxDevices)
    return fail(SSL_ERR_UNSUPPORTED, "device %d beyond the %d the library tracks", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    if (int rc = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                           "hipGetSymbolAddress(scratch)"))
      return rc;
    if (!p) return fail(SSL_ERR_HIP, "hipGetSymbolAddress(scratch) returned no address");
    g_scratch[dev] = (unsigned char*)p;
  }
  *out = g_scratch[dev];
  return SSL_OK;
}

// Zero `n32` int32 words at `a` and `n64` uint64 words at `b`.
__global__ void clear_words(int32_t* a, int64_t n32, unsigned long long* b, int64_t n64) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n32) a[i] = 0;
  if (i < n64) b[i] = 0;
}

}  // namespace
}  // namespace ssl

using namespace ssl;

extern "C" {

int64_t ssl_slr_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

int ssl_slr_forward_noalloc(void* y, int64_t ldy, const void* x, int64_t ldx, const void* A,
                            const void* B, const void* bias, const int32_t* col,
                            const void* values, const int32_t* plan, int64_t n_chunks,
                            int64_t n_slots, int64_t lr_wgs, int64_t M, int64_t m, int64_t m_pad,
                            int64_t NB, int64_t r_pad, int32_t block_p, int32_t block_q,
                            int32_t dtype, void* stream) {
  clear_error();
  if (M < 0 || NB < 0 || r_pad < 0 || n_slots < 0 || m_pad < 0)
    return fail(SSL_ERR_INVALID, "negative size");
  if (M == 0 || NB == 0) return SSL_OK;
  const int64_t n_cnt = ssl_slr_counter_count(M, NB);
  const int64_t x_bytes = ssl_slr_exchange_size(M, r_pad, m_pad, dtype);
  // the workspace the call needs (the room for split prefill calls' partial
  // tiles is used when the array holds it)
  const int64_t ws = slr_workspace_min(M, NB, block_p, r_pad, m_pad, n_slots, dtype);
  if (4 * n_cnt > kNoAllocCounterBytes || x_bytes > kNoAllocExchangeBytes ||
      ws > kNoAllocWorkspaceBytes)
    return fail(SSL_ERR_CAPACITY,
                "this call needs %lld counter, %lld exchange and %lld workspace bytes; the "
                "no-allocation entry point holds at most %lld, %lld and %lld (use ssl_slr_forward "
                "with caller scratch)",
                (long long)(4 * n_cnt), (long long)x_bytes, (long long)ws,
                (long long)kNoAllocCounterBytes, (long long)kNoAllocExchangeBytes,
                (long long)kNoAllocWorkspaceBytes);
  unsigned char* base = nullptr;
  if (int rc = scratch_on_current_device(&base)) return rc;
  int32_t* counters = (int32_t*)base;
  unsigned char* exchange = base + kNoAllocCounterBytes;
  unsigned char* workspace = exchange + kNoAllocExchangeBytes;
  // The handshake words start at zero for this call's plan (the previous call
  // may have used another plan), and so do the row counters.
  const int64_t n_words = x_bytes / 8;
  const int64_t n_clear = n_cnt > n_words ? n_cnt : n_words;
  hipLaunchKernelGGL(clear_words, dim3((unsigned)((n_clear + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, counters, n_cnt, (unsigned long long*)exchange, n_words);
  if (int rc = check_hip(hipGetLastError(), "scratch clear launch")) return rc;
  return ssl_slr_forward(y, ldy, x, ldx, A, B, bias, col, values, plan, n_chunks, n_slots, lr_wgs,
                         M, m, m_pad, NB, r_pad, block_p, block_q, dtype, counters, n_cnt,
                         exchange, x_bytes, workspace, kNoAllocWorkspaceBytes, stream);
}

}  // extern "C"
