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

// ---------------------------------------------------------------------------
// Vector paths, for blocks whose rows are whole 16-byte pieces (S, lds and q
// aligned to 16 bytes). The keep rule and the copies are the ones above.
// ---------------------------------------------------------------------------
constexpr int kFlagRounds = 4;   // blocks per lane group and wave, small blocks
constexpr int kScanThreads = 1024;
constexpr int kScanKeep = 16;    // row counts a scan thread keeps in registers

// L lanes per block (the piece count's next power of two, at most 64), 64 / L
// blocks per wave and round; a lane tests pieces li, li + L, ... of its block,
// four loads at a time.
template <int DT>
__global__ __launch_bounds__(kThreads) void bsr_flag_vec_kernel(const void* S, int64_t lds,
                                                                int64_t nblocks, int NBK, int p,
                                                                int q, int L, int rounds,
                                                                uint8_t* flags) {
  using T = typename Bits<DT>::T;
  constexpr int EB = (int)sizeof(T), VE = 16 / EB;
  const int lane = threadIdx.x & 63;
  const int per_round = kWave / L, cpr = q / VE, pieces = p * cpr;
  const int gi = lane / L, li = lane % L;
  const unsigned long long gmask = (L == kWave ? ~0ull : ((1ull << L) - 1ull)) << (gi * L);
  const int64_t wave = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  auto test = [&](const uint4& v, bool& nan, bool& nz) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      if constexpr (DT == DT_F32) {
        nan |= Bits<DT>::is_nan(w[h]);
        nz |= !Bits<DT>::is_zero(w[h]);
      } else {
        const T lo = (T)(w[h] & 0xffffu), hi = (T)(w[h] >> 16);
        nan |= Bits<DT>::is_nan(lo) || Bits<DT>::is_nan(hi);
        nz |= !Bits<DT>::is_zero(lo) || !Bits<DT>::is_zero(hi);
      }
    }
  };
  if (pieces <= L && rounds == kFlagRounds) {
    // at most one piece per lane and block: every round's load in flight at once
    uint4 v[kFlagRounds];
#pragma unroll
    for (int r = 0; r < kFlagRounds; ++r) {
      const int64_t blk = (wave * kFlagRounds + r) * per_round + gi;
      v[r] = make_uint4(0, 0, 0, 0);
      if (blk < nblocks && li < pieces) {
        const int by = (int)(blk / NBK), bc = (int)(blk % NBK);
        const char* base = (const char*)S + ((int64_t)by * p * lds + (int64_t)bc * q) * EB;
        v[r] = *(const uint4*)(base + ((int64_t)(li / cpr) * lds + (li % cpr) * VE) * EB);
      }
    }
#pragma unroll
    for (int r = 0; r < kFlagRounds; ++r) {
      const int64_t blk = (wave * kFlagRounds + r) * per_round + gi;
      bool nan = false, nz = false;
      test(v[r], nan, nz);
      const unsigned long long bn = __ballot(nan) & gmask, bz = __ballot(nz) & gmask;
      if (li == 0 && blk < nblocks) flags[blk] = (uint8_t)((bn == 0ull && bz != 0ull) ? 1 : 0);
    }
    return;
  }
  for (int r = 0; r < rounds; ++r) {
    const int64_t blk = (wave * rounds + r) * per_round + gi;
    bool nan = false, nz = false;
    if (blk < nblocks) {
      const int by = (int)(blk / NBK), bc = (int)(blk % NBK);
      const char* base = (const char*)S + ((int64_t)by * p * lds + (int64_t)bc * q) * EB;
      for (int x0 = li; x0 < pieces; x0 += 4 * L) {
        uint4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int x = x0 + u * L;
          v[u] = make_uint4(0, 0, 0, 0);
          if (x < pieces)
            v[u] = *(const uint4*)(base + ((int64_t)(x / cpr) * lds + (x % cpr) * VE) * EB);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) test(v[u], nan, nz);
      }
    }
    const unsigned long long bn = __ballot(nan) & gmask, bz = __ballot(nz) & gmask;
    if (li == 0 && blk < nblocks) flags[blk] = (uint8_t)((bn == 0ull && bz != 0ull) ? 1 : 0);
  }
}

// One wave per block-row: crow[by] = its number of kept blocks (the scan below
// turns the counts into offsets in place).
__global__ __launch_bounds__(kThreads) void bsr_rowcount_kernel(const uint8_t* flags, int NB,
                                                                int NBK, int32_t* crow) {
  const int lane = threadIdx.x & 63;
  const int64_t by = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (by >= NB) return;
  const uint8_t* f = flags + by * NBK;
  int c = 0;
  for (int j0 = 0; j0 < NBK; j0 += 4 * kWave) {
    uint8_t v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int j = j0 + u * kWave + lane;
      v[u] = j < NBK ? f[j] : 0;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) c += __popcll(__ballot(v[u] != 0));
  }
  if (lane == 0) crow[by] = c;
}

// Single workgroup: row counts → crow offsets (in place), active rows, totals.
// Thread t owns rows [t·R, (t+1)·R); it reads them all before the scan and
// writes only its own rows after it.
__global__ __launch_bounds__(kScanThreads) void bsr_scan_counts_kernel(int NB, int32_t* crow,
                                                                       int32_t* active,
                                                                       int32_t* totals) {
  __shared__ int s_w[kScanThreads / kWave][2];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int R = (NB + kScanThreads - 1) / kScanThreads;
  const int r0 = min(t * R, NB), r1 = min(r0 + R, NB);
  int cnt[kScanKeep];
  int nnz = 0, act = 0;
#pragma unroll
  for (int k = 0; k < kScanKeep; ++k) {
    cnt[k] = r0 + k < r1 ? crow[r0 + k] : 0;
    nnz += cnt[k];
    act += cnt[k] > 0;
  }
  for (int by = r0 + kScanKeep; by < r1; ++by) {
    const int c = crow[by];
    nnz += c;
    act += c > 0;
  }
  // inclusive scans of (nnz, act) over the wave, then over the waves
  int in = nnz, ia = act;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int a = __shfl_up(in, off, kWave), b = __shfl_up(ia, off, kWave);
    if (lane >= off) in += a, ia += b;
  }
  if (lane == kWave - 1) s_w[w][0] = in, s_w[w][1] = ia;
  __syncthreads();
  int bn = 0, ba = 0, tn = 0, ta = 0;
  for (int x = 0; x < kScanThreads / kWave; ++x) {
    if (x < w) bn += s_w[x][0], ba += s_w[x][1];
    tn += s_w[x][0];
    ta += s_w[x][1];
  }
  int off = bn + in - nnz, aoff = ba + ia - act;
#pragma unroll
  for (int k = 0; k < kScanKeep; ++k) {
    if (r0 + k < r1) {
      crow[r0 + k] = off;
      if (cnt[k] > 0) active[aoff++] = r0 + k;
      off += cnt[k];
    }
  }
  for (int by = r0 + kScanKeep; by < r1; ++by) {
    const int c = crow[by];
    crow[by] = off;
    if (c > 0) active[aoff++] = by;
    off += c;
  }
  if (t == kScanThreads - 1) {
    crow[NB] = tn;
    totals[0] = tn;
    totals[1] = ta;
  }
}

// gridDim.y workgroups per block-row, each wave BPW kept blocks a round (small
// blocks) or one: the (p, q) copy in 16-byte pieces; the (q, p) copy through
// LDS, whole small blocks or slabs of SR rows (a multiple of VE, at most 8 KiB
// of the block per wave): the slab's
// pieces are stored row-major, then each lane gathers VE consecutive rows of
// one column and stores them as one 16-byte piece (VT needs p a multiple of VE
// and q at most 512, so that a slab holds at least VE rows).
template <int DT>
__global__ __launch_bounds__(kThreads) void bsr_fill_vec_kernel(const void* S, int64_t lds, int NBK,
                                                                int p, int q,
                                                                const uint8_t* flags,
                                                                const int32_t* crow, int32_t* col,
                                                                void* vbsr, void* vt) {
  using T = typename Bits<DT>::T;
  constexpr int EB = (int)sizeof(T), VE = 16 / EB;
  constexpr int SEG = 1024, kSlabBytes = 8192;
  __shared__ int s_cols[SEG];
  __shared__ int s_cnt[kThreads];
  __shared__ int s_nseg;
  __shared__ uint4 s_slab[kWaves][kSlabBytes / 16];
  const int by = blockIdx.x, t = threadIdx.x, lane = t & 63, w = t >> 6;
  const uint8_t* f = flags + (int64_t)by * NBK;
  const int cpr = q / VE, pieces = p * cpr;
  // Blocks of at most half a slab: BPW whole blocks per wave and round, one
  // slab each; larger blocks: one block per wave, in slabs of SR rows.
  const int blk_bytes = p * q * EB;
  const int BPW = blk_bytes <= kSlabBytes / 2 ? min(16, kSlabBytes / blk_bytes) : 1;
  const int SR = BPW > 1 ? p : min(p, kSlabBytes / (q * EB) / VE * VE);
  const T* tile = (const T*)s_slab[w];
  int base = crow[by];
  for (int c0 = 0; c0 < NBK; c0 += SEG) {
    const int cn = min(SEG, NBK - c0);
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
    // rounds of 4·BPW blocks, the same count in every wave (the slab barriers);
    // workgroup z of the row takes rounds z, z + gridDim.y, ...; wave w takes
    // the round's blocks kw .. kw + nb - 1
    for (int k0 = blockIdx.y * kWaves * BPW; k0 < nseg; k0 += kWaves * BPW * gridDim.y) {
      const int kw = k0 + w * BPW;
      const int nb = max(0, min(BPW, nseg - kw));
      auto src_of = [&](int bi) {
        return (const char*)S + ((int64_t)by * p * lds + (int64_t)s_cols[kw + bi] * q) * EB;
      };
      if (lane < nb) col[(int64_t)base + kw + lane] = s_cols[kw + lane];
      if (vbsr) {
        const int total = nb * pieces;
        for (int x0 = lane; x0 < total; x0 += 4 * kWave) {
          uint4 v[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int x = x0 + u * kWave;
            v[u] = make_uint4(0, 0, 0, 0);
            if (x < total) {
              const int bi = x / pieces, xx = x % pieces;
              v[u] = *(const uint4*)(src_of(bi) + ((int64_t)(xx / cpr) * lds + (xx % cpr) * VE) * EB);
            }
          }
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int x = x0 + u * kWave;
            if (x < total) {
              const int bi = x / pieces, xx = x % pieces;
              *(uint4*)((char*)vbsr + ((int64_t)base + kw + bi) * blk_bytes + (int64_t)xx * 16) = v[u];
            }
          }
        }
      }
      if (vt) {
        for (int r0 = 0; r0 < p; r0 += SR) {
          const int nr = min(SR, p - r0), spieces = nr * cpr, tpc = nr / VE;
          const int total = nb * spieces;  // at most kSlabBytes / 16 pieces
          for (int x0 = lane; x0 < total; x0 += 4 * kWave) {
            uint4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const int x = x0 + u * kWave;
              v[u] = make_uint4(0, 0, 0, 0);
              if (x < total) {
                const int bi = x / spieces, xx = x % spieces;
                v[u] = *(const uint4*)(src_of(bi) + ((int64_t)(r0 + xx / cpr) * lds + (xx % cpr) * VE) * EB);
              }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
              if (x0 + u * kWave < total) s_slab[w][x0 + u * kWave] = v[u];
          }
          __syncthreads();
          const int tp = q * tpc, ttotal = nb * tp;
          for (int y = lane; y < ttotal; y += kWave) {
            const int bi = y / tp, yy = y % tp;
            const int j = yy / tpc, i0 = (yy % tpc) * VE;
            const T* tb = tile + bi * (nr * q);
            uint32_t wv[4];
#pragma unroll
            for (int e = 0; e < VE; ++e) {
              const uint32_t bits = (uint32_t)tb[(i0 + e) * q + j];
              if constexpr (VE == 4) wv[e] = bits;
              else if (e & 1) wv[e >> 1] |= bits << 16;
              else wv[e >> 1] = bits;
            }
            *(uint4*)((char*)vt + ((int64_t)base + kw + bi) * blk_bytes + ((int64_t)j * p + r0 + i0) * EB) =
                make_uint4(wv[0], wv[1], wv[2], wv[3]);
          }
          __syncthreads();
        }
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
  const int eb = (dtype == SSL_F32) ? 4 : 2;
  const bool vec = ((uintptr_t)S % 16 == 0) && (lds * eb) % 16 == 0 && (block_q * eb) % 16 == 0;
  if (nblocks > 0 && vec && (dtype == SSL_F32 || dtype == SSL_BF16 || dtype == SSL_F16)) {
    const int64_t pieces = (int64_t)block_p * (block_q * eb / 16);
    int L = 1;
    while (L < pieces && L < kWave) L <<= 1;
    const int rounds = L < kWave ? kFlagRounds : 1;
    const int64_t per_wave = (int64_t)(kWave / L) * rounds;
    const int64_t waves = (nblocks + per_wave - 1) / per_wave;
    const unsigned grid = (unsigned)((waves + kWaves - 1) / kWaves);
#define SSL_FLAG_VEC(DTC)                                                                        \
  hipLaunchKernelGGL(bsr_flag_vec_kernel<DTC>, dim3(grid), dim3(kThreads), 0, s, S, lds, nblocks, \
                     (int)NBK, block_p, block_q, L, rounds, flags)
    if (dtype == SSL_F32) SSL_FLAG_VEC(DT_F32);
    else if (dtype == SSL_BF16) SSL_FLAG_VEC(DT_BF16);
    else SSL_FLAG_VEC(DT_F16);
#undef SSL_FLAG_VEC
    int rc = check_hip(hipGetLastError(), "bsr flag launch");
    if (rc) return rc;
  } else if (nblocks > 0) {
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
  if (NB > 0)
    hipLaunchKernelGGL(bsr_rowcount_kernel, dim3((unsigned)((NB + kWaves - 1) / kWaves)),
                       dim3(kThreads), 0, s, flags, (int)NB, (int)NBK, crow);
  hipLaunchKernelGGL(bsr_scan_counts_kernel, dim3(1), dim3(kScanThreads), 0, s, (int)NB, crow,
                     active_rows, totals);
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
  const int eb = (dtype == SSL_F32) ? 4 : 2;
  const bool vec = ((uintptr_t)S % 16 == 0) && (lds * eb) % 16 == 0 &&
                   (block_q * eb) % 16 == 0 && (uintptr_t)values_bsr % 16 == 0 &&
                   (!values_t || ((uintptr_t)values_t % 16 == 0 && (block_p * eb) % 16 == 0 &&
                                  block_q <= 512));  // a slab holds 16 bytes of rows per column
  if (vec && (dtype == SSL_F32 || dtype == SSL_BF16 || dtype == SSL_F16)) {
    // enough workgroups for about four per compute unit, at most 8 per block-row
    const int64_t want = (4 * (int64_t)device_cus() + NB - 1) / NB;
    const unsigned split = (unsigned)std::max<int64_t>(1, std::min<int64_t>(want, 8));
#define SSL_FILL_VEC(DTC)                                                                         \
  hipLaunchKernelGGL(bsr_fill_vec_kernel<DTC>, dim3((unsigned)NB, split), dim3(kThreads), 0, s, S, \
                     lds, (int)NBK, block_p, block_q, flags, crow, col, values_bsr, values_t)
    if (dtype == SSL_F32) SSL_FILL_VEC(DT_F32);
    else if (dtype == SSL_BF16) SSL_FILL_VEC(DT_BF16);
    else SSL_FILL_VEC(DT_F16);
#undef SSL_FILL_VEC
    return check_hip(hipGetLastError(), "bsr fill launch");
  }
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
