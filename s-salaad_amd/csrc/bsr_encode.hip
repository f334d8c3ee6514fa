// Dense -> BSR encoder on the device.
//
// Keep rule (ssalaad/efficient/artifact.py:28-29): a block is stored iff the sum
// of |values| over it is > 0. A sum of absolute values is > 0 exactly when the
// block holds at least one non-zero and no NaN (a NaN makes the sum NaN, and
// NaN > 0 is false), so the rule is evaluated on bit patterns and is exact for
// every dtype. Kept blocks are numbered row-major (artifact.py:36-38), values
// are copied bit for bit, and the module's int32/transposed/active-row view
// (ssalaad/efficient/ls_linear.py:89-97) is produced in the same pass.
#include "abi_internal.h"
#include "slr_common.h"

namespace ssl {
namespace {

template <int DT>
struct Bits {
  using T = typename std::conditional<DT == DT_F32, uint32_t, uint16_t>::type;
  __device__ static bool is_nan(T b) {
    if constexpr (DT == DT_F32) return (b & 0x7fffffffu) > 0x7f800000u;
    else if constexpr (DT == DT_BF16) return (b & 0x7fffu) > 0x7f80u;
    else return (b & 0x7fffu) > 0x7c00u;
  }
  __device__ static bool is_zero(T b) {
    if constexpr (DT == DT_F32) return (b & 0x7fffffffu) == 0u;
    else return (b & 0x7fffu) == 0u;
  }
};

// One wave per block: flags[by·NBK + bc] = keep.
template <int DT>
__global__ __launch_bounds__(kThreads) void bsr_flag_kernel(const void* S, int64_t lds, int NB,
                                                            int NBK, int p, int q, uint8_t* flags) {
  using T = typename Bits<DT>::T;
  const int lane = threadIdx.x & 63;
  const int64_t blk = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (blk >= (int64_t)NB * NBK) return;
  const int by = (int)(blk / NBK), bc = (int)(blk % NBK);
  const T* base = (const T*)S + (int64_t)by * p * lds + (int64_t)bc * q;
  bool nan = false, nz = false;
  for (int idx = lane; idx < p * q; idx += kWave) {
    const int i = idx / q, j = idx % q;
    const T b = base[(int64_t)i * lds + j];
    nan |= Bits<DT>::is_nan(b);
    nz |= !Bits<DT>::is_zero(b);
  }
  const bool any_nan = __any(nan);
  const bool any_nz = __any(nz);
  if (lane == 0) flags[blk] = (uint8_t)((!any_nan && any_nz) ? 1 : 0);
}

// Single workgroup: crow (exclusive scan of per-row counts), active rows, totals.
__global__ __launch_bounds__(kThreads) void bsr_scan_kernel(const uint8_t* flags, int NB, int NBK,
                                                            int32_t* crow, int32_t* active,
                                                            int32_t* totals) {
  __shared__ int s_nnz[kThreads], s_act[kThreads];
  const int t = threadIdx.x;
  const int R = (NB + kThreads - 1) / kThreads;
  const int r0 = min(t * R, NB), r1 = min(r0 + R, NB);
  auto count = [&](int by) {
    int n = 0;
    const uint8_t* f = flags + (int64_t)by * NBK;
    for (int j = 0; j < NBK; ++j) n += f[j];
    return n;
  };
  int nnz = 0, act = 0;
  for (int by = r0; by < r1; ++by) {
    const int n = count(by);
    nnz += n;
    act += (n > 0);
  }
  s_nnz[t] = nnz;
  s_act[t] = act;
  __syncthreads();
  if (t == 0) {
    int a = 0, b = 0;
    for (int i = 0; i < kThreads; ++i) {
      const int x = s_nnz[i], y = s_act[i];
      s_nnz[i] = a;
      s_act[i] = b;
      a += x;
      b += y;
    }
    crow[NB] = a;
    totals[0] = a;
    totals[1] = b;
  }
  __syncthreads();
  int off = s_nnz[t], aoff = s_act[t];
  for (int by = r0; by < r1; ++by) {
    const int n = count(by);
    crow[by] = off;
    if (n > 0) active[aoff++] = by;
    off += n;
  }
}

// One workgroup per block-row: col indices and value copies of the kept blocks.
template <int DT>
__global__ __launch_bounds__(kThreads) void bsr_fill_kernel(const void* S, int64_t lds, int NBK,
                                                            int p, int q, const uint8_t* flags,
                                                            const int32_t* crow, int32_t* col,
                                                            void* vbsr, void* vt) {
  using T = typename Bits<DT>::T;
  constexpr int SEG = 1024;
  __shared__ int s_cols[SEG];
  __shared__ int s_cnt[kThreads];
  __shared__ int s_nseg;
  const int by = blockIdx.x, t = threadIdx.x;
  const uint8_t* f = flags + (int64_t)by * NBK;
  int base = crow[by];
  for (int c0 = 0; c0 < NBK; c0 += SEG) {
    const int cn = min(SEG, NBK - c0);
    // 4 consecutive columns per thread, scanned in thread order.
    const int j0 = c0 + 4 * t;
    int mine = 0;
    for (int j = j0; j < min(j0 + 4, c0 + cn); ++j) mine += f[j];
    s_cnt[t] = mine;
    __syncthreads();
    if (t == 0) {
      int a = 0;
      for (int i = 0; i < kThreads; ++i) {
        const int x = s_cnt[i];
        s_cnt[i] = a;
        a += x;
      }
      s_nseg = a;
    }
    __syncthreads();
    int pos = s_cnt[t];
    for (int j = j0; j < min(j0 + 4, c0 + cn); ++j)
      if (f[j]) s_cols[pos++] = j;
    __syncthreads();
    const int nseg = s_nseg;
    for (int k = 0; k < nseg; ++k) {
      const int bc = s_cols[k];
      const int64_t dst = (int64_t)base + k;
      if (t == 0) col[dst] = bc;
      const T* src = (const T*)S + (int64_t)by * p * lds + (int64_t)bc * q;
      for (int idx = t; idx < p * q; idx += kThreads) {
        const int i = idx / q, j = idx % q;
        const T v = src[(int64_t)i * lds + j];
        if (vbsr) ((T*)vbsr)[dst * p * q + idx] = v;             // (p, q)
        if (vt) ((T*)vt)[dst * p * q + (int64_t)j * p + i] = v;  // (q, p)
      }
    }
    base += nseg;
    __syncthreads();
  }
}

}  // namespace
}  // namespace ssl

using namespace ssl;

extern "C" {

int ssl_bsr_encode_count(const void* S, int64_t lds, int64_t NB, int64_t NBK, int32_t block_p,
                         int32_t block_q, int32_t dtype, uint8_t* flags, int32_t* crow,
                         int32_t* active_rows, int32_t* totals, void* stream) {
  clear_error();
  if (block_p <= 0 || block_q <= 0 || NB < 0 || NBK < 0) return fail(SSL_ERR_INVALID, "bad sizes");
  if (lds < NBK * block_q) return fail(SSL_ERR_INVALID, "lds smaller than the row");
  if (!crow || !totals || (NB > 0 && (!flags || !active_rows)) || (NB * NBK > 0 && !S))
    return fail(SSL_ERR_INVALID, "null pointer");
  if (NB * NBK > 0x7fffffffLL) return fail(SSL_ERR_INVALID, "too many blocks");
  hipStream_t s = (hipStream_t)stream;
  const int64_t nblocks = NB * NBK;
  if (nblocks > 0) {
    const unsigned grid = (unsigned)((nblocks + kWaves - 1) / kWaves);
    switch (dtype) {
      case SSL_F32:
        hipLaunchKernelGGL(bsr_flag_kernel<DT_F32>, dim3(grid), dim3(kThreads), 0, s, S, lds,
                           (int)NB, (int)NBK, block_p, block_q, flags);
        break;
      case SSL_BF16:
        hipLaunchKernelGGL(bsr_flag_kernel<DT_BF16>, dim3(grid), dim3(kThreads), 0, s, S, lds,
                           (int)NB, (int)NBK, block_p, block_q, flags);
        break;
      case SSL_F16:
        hipLaunchKernelGGL(bsr_flag_kernel<DT_F16>, dim3(grid), dim3(kThreads), 0, s, S, lds,
                           (int)NB, (int)NBK, block_p, block_q, flags);
        break;
      default:
        return fail(SSL_ERR_UNSUPPORTED, "unsupported dtype %d", dtype);
    }
    int rc = check_hip(hipGetLastError(), "bsr flag launch");
    if (rc) return rc;
  } else if (!(dtype == SSL_F32 || dtype == SSL_BF16 || dtype == SSL_F16)) {
    return fail(SSL_ERR_UNSUPPORTED, "unsupported dtype %d", dtype);
  }
  hipLaunchKernelGGL(bsr_scan_kernel, dim3(1), dim3(kThreads), 0, s, flags, (int)NB, (int)NBK,
                     crow, active_rows, totals);
  return check_hip(hipGetLastError(), "bsr scan launch");
}

int ssl_bsr_encode_fill(const void* S, int64_t lds, int64_t NB, int64_t NBK, int32_t block_p,
                        int32_t block_q, int32_t dtype, const uint8_t* flags, const int32_t* crow,
                        int32_t* col, void* values_bsr, void* values_t, void* stream) {
  clear_error();
  if (block_p <= 0 || block_q <= 0 || NB < 0 || NBK < 0) return fail(SSL_ERR_INVALID, "bad sizes");
  if (lds < NBK * block_q) return fail(SSL_ERR_INVALID, "lds smaller than the row");
  if (NB == 0 || NBK == 0) return SSL_OK;
  if (!S || !flags || !crow || !col) return fail(SSL_ERR_INVALID, "null pointer");
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case SSL_F32:
      hipLaunchKernelGGL(bsr_fill_kernel<DT_F32>, dim3((unsigned)NB), dim3(kThreads), 0, s, S, lds,
                         (int)NBK, block_p, block_q, flags, crow, col, values_bsr, values_t);
      break;
    case SSL_BF16:
      hipLaunchKernelGGL(bsr_fill_kernel<DT_BF16>, dim3((unsigned)NB), dim3(kThreads), 0, s, S,
                         lds, (int)NBK, block_p, block_q, flags, crow, col, values_bsr, values_t);
      break;
    case SSL_F16:
      hipLaunchKernelGGL(bsr_fill_kernel<DT_F16>, dim3((unsigned)NB), dim3(kThreads), 0, s, S, lds,
                         (int)NBK, block_p, block_q, flags, crow, col, values_bsr, values_t);
      break;
    default:
      return fail(SSL_ERR_UNSUPPORTED, "unsupported dtype %d", dtype);
  }
  return check_hip(hipGetLastError(), "bsr fill launch");
}

}  // extern "C"
