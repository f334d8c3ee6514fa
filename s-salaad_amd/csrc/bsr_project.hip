// Block projection on the device: keep the n_keep blocks of largest Frobenius
// norm, the sparse step of the reference's compression loop
// (ssalaad/inference/egar.py:296-317, _project_S):
//
//   norms[b]  = Σ over block b of v², v = the input as fp32   (M.float(), .pow(2).sum)
//   keep      = the n_keep largest norms                       (topk(n_keep, largest=True))
//   out       = the input as fp32 where its block is kept, 0 elsewhere
//
// The selection is a most-significant-digit radix select over the norms' fp32
// bit patterns, which order like the values themselves because every norm is
// ≥ +0 or NaN (all NaNs are folded into one pattern above +inf, so NaN blocks
// count as the largest, as in torch.topk). Blocks whose norms are equal are
// taken in ascending block order (row-major), which makes the result
// deterministic; torch.topk leaves that order unspecified.
#include "abi_internal.h"
#include "slr_common.h"

namespace ssl {
namespace {

constexpr int kSelThreads = 1024;
constexpr uint32_t kNanKey = 0x7fc00000u;

template <int DT>
__device__ __forceinline__ float elem_f32(const void* base, int64_t i) {
  if constexpr (DT == DT_F32) return ((const float*)base)[i];
  else if constexpr (DT == DT_BF16) return bf16_to_f32(((const uint16_t*)base)[i]);
  else return f16_to_f32(((const uint16_t*)base)[i]);
}

// The many-workgroup select's workspace (32-bit words): per pass (one 8-bit
// digit of the key each, most significant first) a 256-bin histogram, then
// per workgroup its own last-pass histogram, whose bin of the threshold key T
// counts the keys equal to T in its range, for the ordered pass. The norms'
// launch zeroes the pass histograms, so each call starts from zero whatever
// the last call left.
constexpr int kSelPasses = 4;
constexpr int kWsHist = 0;  // [pass][256]
constexpr int kWsGroupHist = kWsHist + 256 * kSelPasses;
constexpr int kMaxSelGroups = 1024;
static_assert(kWsGroupHist % 4 == 0, "per-group histograms start on a 16-byte boundary");

__device__ __forceinline__ void sel_ws_init(uint32_t* ws) {
  for (int i = threadIdx.x; i < kWsGroupHist; i += blockDim.x) ws[i] = 0u;
}

// One wave per block: the fp32 sum of squares (lane-strided partial sums, then a
// fixed butterfly, so repeated runs give identical bits). A lane takes pieces
// lane, lane + 64, ... in that order, kSumsqUnroll loads at a time.
constexpr int kSumsqUnroll = 8;
template <int DT>
__global__ __launch_bounds__(kThreads) void block_sumsq_kernel(const void* S, int64_t lds, int NB,
                                                               int NBK, int p, int q, bool vec,
                                                               float* norms, uint32_t* sel_ws) {
  if (sel_ws && blockIdx.x == 0) sel_ws_init(sel_ws);
  const int lane = threadIdx.x & 63;
  const int64_t blk = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (blk >= (int64_t)NB * NBK) return;
  const int by = (int)(blk / NBK), bc = (int)(blk % NBK);
  const int64_t base = (int64_t)by * p * lds + (int64_t)bc * q;
  constexpr int EB = Elem<DT>::bytes, VE = 16 / EB;  // elements per 16-byte piece
  float acc = 0.f;
  if (vec) {
    // pieces of VE elements: cpr per block row, all rows
    const int cpr = q / VE, pieces = p * cpr;
    for (int idx0 = lane; idx0 < pieces; idx0 += kSumsqUnroll * kWave) {
      uint4 v4[kSumsqUnroll];
#pragma unroll
      for (int u = 0; u < kSumsqUnroll; ++u) {
        const int idx = idx0 + u * kWave;
        const int i = idx / cpr, j = (idx % cpr) * VE;
        v4[u] = idx < pieces ? *(const uint4*)((const char*)S + (base + (int64_t)i * lds + j) * EB)
                             : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < kSumsqUnroll; ++u) {
        const uint32_t w[4] = {v4[u].x, v4[u].y, v4[u].z, v4[u].w};
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          if constexpr (DT == DT_F32) {
            const float v = __uint_as_float(w[h]);
            acc = fmaf(v, v, acc);
          } else {
            const float lo = DT == DT_BF16 ? bf16_to_f32(w[h] & 0xffffu) : f16_to_f32(w[h] & 0xffffu);
            const float hi = DT == DT_BF16 ? bf16_to_f32(w[h] >> 16) : f16_to_f32(w[h] >> 16);
            acc = fmaf(lo, lo, acc);
            acc = fmaf(hi, hi, acc);
          }
        }
      }
    }
  } else {
    for (int idx = lane; idx < p * q; idx += kWave) {
      const int i = idx / q, j = idx % q;
      const float v = elem_f32<DT>(S, base + (int64_t)i * lds + j);
      acc = fmaf(v, v, acc);
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, kWave);
  if (lane == 0) norms[blk] = acc;
}

// Small blocks (at most 64 pieces of 16 bytes, e.g. 16×16 fp32, 8×8): lanes-per-
// block L, the next power of two of the piece count; a wave takes 64 / L blocks
// a round and kSmallRounds rounds with every load in flight at once. Each lane
// sums its piece in the order above and the L lanes of a block reduce with
// the last log2(L) steps of the same butterfly (the wider steps above would
// add lanes that hold +0), so the sums are bit-identical to the kernel above.
constexpr int kSmallRounds = 4;

template <int DT>
__global__ __launch_bounds__(kThreads) void block_sumsq_small_kernel(
    const void* S, int64_t lds, int64_t nblocks, int NBK, int p, int q, int L, float* norms,
    uint32_t* sel_ws) {
  if (sel_ws && blockIdx.x == 0) sel_ws_init(sel_ws);
  constexpr int EB = Elem<DT>::bytes, VE = 16 / EB;
  const int lane = threadIdx.x & 63;
  const int per_round = kWave / L, cpr = q / VE, pieces = p * cpr;
  const int gi = lane / L, li = lane % L;
  const int64_t wave = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  const int64_t blk0 = wave * (kSmallRounds * per_round) + gi;
  uint4 v4[kSmallRounds];
#pragma unroll
  for (int u = 0; u < kSmallRounds; ++u) {
    const int64_t blk = blk0 + (int64_t)u * per_round;
    v4[u] = make_uint4(0, 0, 0, 0);
    if (li < pieces && blk < nblocks) {
      const int by = (int)(blk / NBK), bc = (int)(blk % NBK);
      const int i = li / cpr, j = (li % cpr) * VE;
      const int64_t off = (int64_t)by * p * lds + (int64_t)bc * q + (int64_t)i * lds + j;
      v4[u] = *(const uint4*)((const char*)S + off * EB);
    }
  }
#pragma unroll
  for (int u = 0; u < kSmallRounds; ++u) {
    float acc = 0.f;
    const uint32_t w[4] = {v4[u].x, v4[u].y, v4[u].z, v4[u].w};
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      if constexpr (DT == DT_F32) {
        const float v = __uint_as_float(w[h]);
        acc = fmaf(v, v, acc);
      } else {
        const float lo = DT == DT_BF16 ? bf16_to_f32(w[h] & 0xffffu) : f16_to_f32(w[h] & 0xffffu);
        const float hi = DT == DT_BF16 ? bf16_to_f32(w[h] >> 16) : f16_to_f32(w[h] >> 16);
        acc = fmaf(lo, lo, acc);
        acc = fmaf(hi, hi, acc);
      }
    }
    for (int off = L >> 1; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, kWave);
    const int64_t blk = blk0 + (int64_t)u * per_round;
    if (li == 0 && blk < nblocks) norms[blk] = acc;
  }
}

__device__ __forceinline__ uint32_t norm_key(float v) {
  const uint32_t b = __float_as_uint(v);
  return (b & 0x7fffffffu) > 0x7f800000u ? kNanKey : b;
}

// hist[d] += 1 for each lane with `in`. Norms of one matrix mostly share their
// leading digits, so a wave's lanes usually land in one bin; then one lane adds
// the wave's count instead of 64 lanes contending for one LDS word.
__device__ __forceinline__ void hist_add(int* hist, bool in, uint32_t d) {
  const unsigned long long act = __ballot(in);
  if (act == 0ull) return;
  const int first = __ffsll((long long)act) - 1;
  const uint32_t d0 = (uint32_t)__shfl((int)d, first, kWave);
  if (__ballot(in && d == d0) == act) {
    if ((int)(threadIdx.x & 63) == first) atomicAdd(&hist[d0], __popcll(act));
  } else if (in) {
    atomicAdd(&hist[d], 1);
  }
}

// The digit of the need-th largest key among those matching the prefix, from
// a 256-bin histogram read by one wave (lane l: bins 4l .. 4l + 3). Returns the
// lane's result in d, cum (keys above bin d) and cnt (keys in bin d); exactly
// one lane's bins hold it (returns true).
__device__ __forceinline__ bool find_digit(const int (&h)[4], int need0, int& d, int& cum,
                                           int& cnt) {
  const int lane = threadIdx.x & 63;
  const int sum4 = h[0] + h[1] + h[2] + h[3];
  int incl = sum4;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int v = __shfl_down(incl, off, kWave);
    if (lane + off < kWave) incl += v;
  }
  const int above = incl - sum4;
  if (!(above < need0 && need0 <= incl)) return false;
  cum = above;
  d = 4 * lane;
  cnt = h[0];
#pragma unroll
  for (int b = 3; b >= 0; --b) {
    if (cum + h[b] >= need0) {
      d = 4 * lane + b;
      cnt = h[b];
      break;
    }
    cum += h[b];
  }
  return true;
}

// Single workgroup: keep[b] = 1 for the n_keep largest keys (ties: lowest b first).
// STAGED: the keys are copied into LDS once (n ≤ kLdsKeys) and every pass reads them there.
constexpr int kLdsKeys = 15360;  // 60 KiB of keys: within 64 KiB of LDS with the rest
constexpr int64_t kSelOneGroupMax = kLdsKeys;  // more keys: the many-workgroup select

template <bool STAGED>
__global__ __launch_bounds__(kSelThreads) void block_topk_kernel(const float* norms, int n,
                                                                 int n_keep, uint8_t* keep) {
  extern __shared__ uint32_t s_keys[];
  auto key_at = [&](int i) { return STAGED ? s_keys[i] : norm_key(norms[i]); };
  __shared__ int hist[256];
  __shared__ uint32_t s_prefix, s_mask;
  __shared__ int s_need, s_eq;
  __shared__ int s_wave[kSelThreads / kWave];
  const int t = threadIdx.x;
  if (n_keep <= 0 || n_keep >= n) {
    for (int i = t; i < n; i += kSelThreads) keep[i] = n_keep > 0 ? 1 : 0;
    return;
  }
  if (t == 0) {
    s_prefix = 0u;
    s_mask = 0u;
    s_need = n_keep;
  }
  if constexpr (STAGED)
    for (int i = t; i < n; i += kSelThreads) s_keys[i] = norm_key(norms[i]);
  __syncthreads();
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int d = t; d < 256; d += kSelThreads) hist[d] = 0;
    __syncthreads();
    const uint32_t prefix = s_prefix, mask = s_mask;
    for (int i0 = 0; i0 < n; i0 += kSelThreads) {
      const int i = i0 + t;
      const uint32_t k = i < n ? key_at(i) : 0u;
      hist_add(hist, i < n && (k & mask) == prefix, (k >> shift) & 255u);
    }
    __syncthreads();
    if (t < kWave) {
      int h[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) h[b] = hist[4 * t + b];
      const int need0 = s_need;
      int d, cum, cnt;
      if (find_digit(h, need0, d, cum, cnt)) {
        s_need = need0 - cum;
        s_eq = cnt;  // keys matching the prefix so far (after the last digit: equal to T)
        s_prefix = prefix | ((uint32_t)d << shift);
        s_mask = mask | (255u << shift);
      }
    }
    __syncthreads();
  }
  // Threshold key T: keep every key above it and the first s_need keys equal
  // to it in block order.
  const uint32_t T = s_prefix;
  const int need = s_need;
  if (need == s_eq) {
    // every key equal to T is kept: no order among them to respect
    for (int i = t; i < n; i += kSelThreads) keep[i] = key_at(i) >= T ? 1 : 0;
    return;
  }
  const int lane = t & 63, w = t >> 6;
  int taken = 0;  // equal keys already kept in earlier chunks (same in every thread)
  for (int c0 = 0; c0 < n; c0 += kSelThreads) {
    const int i = c0 + t;
    uint32_t k = 0;
    if (i < n) k = key_at(i);
    const bool eq = i < n && k == T;
    const unsigned long long bal = __ballot(eq);
    const int before = __popcll(bal & ((1ull << lane) - 1ull));
    if (lane == 0) s_wave[w] = __popcll(bal);
    __syncthreads();
    int wave_off = 0, chunk_total = 0;
    for (int v = 0; v < kSelThreads / kWave; ++v) {
      const int c = s_wave[v];
      if (v < w) wave_off += c;
      chunk_total += c;
    }
    if (i < n) keep[i] = (k > T || (eq && taken + wave_off + before < need)) ? 1 : 0;
    taken += chunk_total;
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Many-workgroup select, for more keys than one workgroup reads quickly. Four
// 8-bit digit passes, each a launch over every key: group g
// counts the digits of its range [g·chunk, (g+1)·chunk) that match the prefix
// chosen so far into an LDS histogram, adds it to the pass's histogram in the
// workspace, and the group that arrives last picks the pass's digit for the
// next launch. The last pass also leaves each group's own histogram. Then the
// marking launch keeps every key above T, and, when only some of the keys
// equal to T are kept, each group ranks its keys equal to T in block order
// from the count of them in the groups before it.
// ---------------------------------------------------------------------------
constexpr int kSelGroupThreads = 256;
constexpr int kSelUnroll = 32;       // keys per thread per round, loaded together
constexpr int kSelGroupKeys = kSelGroupThreads * kSelUnroll;  // keys per workgroup (one round),
                                                              // up to kMaxSelGroups groups
constexpr int kTiePer = 32;          // contiguous keys per thread in the ordered pass
static_assert(kSelGroupThreads == 256, "one histogram bin per thread");

__device__ __forceinline__ void group_range(int64_t n, int chunk, int64_t& i0, int64_t& i1) {
  i0 = (int64_t)blockIdx.x * chunk;
  i1 = i0 + chunk < n ? i0 + chunk : n;
}

// Block-wide exclusive prefix of v over the workgroup's 256 threads; total in tot.
__device__ __forceinline__ int group_exclusive(int v, int& tot, int* s_wave) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int u = __shfl_up(incl, off, kWave);
    if (lane >= off) incl += u;
  }
  if (lane == kWave - 1) s_wave[w] = incl;
  __syncthreads();
  int before = 0;
  tot = 0;
#pragma unroll
  for (int x = 0; x < kSelGroupThreads / kWave; ++x) {
    const int c = s_wave[x];
    if (x < w) before += c;
    tot += c;
  }
  __syncthreads();
  return before + incl - v;
}

// The select's state after `passes` passes, from the finished histograms of
// those passes (earlier launches, read device-coherently like the atomics
// that built them): wave 0 repeats the digit search of each
// pass in order, every workgroup the same way, and writes {prefix, mask, need,
// eq} to st. Reading the histograms costs one round trip, which the caller
// overlaps with its own key loads.
__device__ __forceinline__ void sel_state(const uint32_t* ws, int passes, int n_keep,
                                          uint32_t* st) {
  const int lane = threadIdx.x & 63;
  if (threadIdx.x >= kWave) return;
  int h[kSelPasses][4];
#pragma unroll
  for (int ps = 0; ps < kSelPasses; ++ps)
#pragma unroll
    for (int b = 0; b < 4; ++b)
      h[ps][b] = ps < passes ? __hip_atomic_load((const int*)ws + kWsHist + 256 * ps + 4 * lane + b,
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                             : 0;
  uint32_t prefix = 0u, mask = 0u;
  int need = n_keep, eq = 0;
#pragma unroll
  for (int ps = 0; ps < kSelPasses; ++ps) {
    if (ps >= passes) break;
    int d = 0, cum = 0, cnt = 0;
    const bool found = find_digit(h[ps], need, d, cum, cnt);
    const int src = __ffsll((long long)__ballot(found)) - 1;
    d = __shfl(d, src, kWave);
    cum = __shfl(cum, src, kWave);
    cnt = __shfl(cnt, src, kWave);
    const int shift = 24 - 8 * ps;
    prefix |= (uint32_t)d << shift;
    mask |= 255u << shift;
    need -= cum;
    eq = cnt;
  }
  if (lane == 0) {
    st[0] = prefix;
    st[1] = mask;
    st[2] = (uint32_t)need;
    st[3] = (uint32_t)eq;
  }
}

template <int PS>
__global__ __launch_bounds__(kSelGroupThreads) void topk_hist_kernel(const float* norms, int n,
                                                                     int chunk, int n_keep,
                                                                     uint32_t* ws) {
  constexpr int SHIFT = 24 - 8 * PS;
  __shared__ int hist[256];
  __shared__ uint32_t s_st[4];
  const int t = threadIdx.x;
  int64_t i0, i1;
  group_range(n, chunk, i0, i1);
  // The first round's keys are requested first, so their round trip overlaps
  // the state's (the earlier passes' histograms) and the barrier.
  constexpr int64_t kStep = kSelGroupThreads * kSelUnroll;
  uint32_t k[kSelUnroll];
  auto load_round = [&](int64_t b) {
#pragma unroll
    for (int u = 0; u < kSelUnroll; ++u) {
      const int64_t i = b + u * kSelGroupThreads + t;
      k[u] = i < i1 ? norm_key(norms[i]) : 0u;
    }
  };
  load_round(i0);
  hist[t] = 0;
  if constexpr (PS > 0) sel_state(ws, PS, n_keep, s_st);
  else if (t == 0) s_st[0] = s_st[1] = 0u;
  __syncthreads();
  const uint32_t prefix = s_st[0], mask = s_st[1];
  for (int64_t b = i0; b < i1; b += kStep) {
#pragma unroll
    for (int u = 0; u < kSelUnroll; ++u) {
      const int64_t i = b + u * kSelGroupThreads + t;
      hist_add(hist, i < i1 && (k[u] & mask) == prefix, (k[u] >> SHIFT) & 255u);
    }
    if (b + kStep < i1) load_round(b + kStep);
  }
  __syncthreads();
  const int mine = hist[t];
  if (mine)
    __hip_atomic_fetch_add((int*)ws + kWsHist + 256 * PS + t, mine, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  // this group's keys per last digit, for the ranks of keys equal to T
  if constexpr (PS == kSelPasses - 1) ws[kWsGroupHist + (int64_t)blockIdx.x * 256 + t] = mine;
}

// Ordered pass over [i0, i1): thread t takes kTiePer consecutive keys of each
// slice of kSelGroupThreads·kTiePer; keys equal to T are ranked in block order
// from `base`, and kept while their rank is below need.
__device__ __forceinline__ void tie_pass(const float* norms, int64_t i0, int64_t i1, uint32_t T,
                                         int need, int base, uint8_t* keep, int* s_wave) {
  for (int64_t s0 = i0; s0 < i1; s0 += kSelGroupThreads * kTiePer) {
    const int64_t a = s0 + (int64_t)threadIdx.x * kTiePer;
    uint32_t k[kTiePer];
    int c = 0;
#pragma unroll
    for (int u = 0; u < kTiePer; ++u) {
      k[u] = a + u < i1 ? norm_key(norms[a + u]) : 0u;
      c += (a + u < i1 && k[u] == T) ? 1 : 0;
    }
    int tot;
    int r = base + group_exclusive(c, tot, s_wave);
#pragma unroll
    for (int u = 0; u < kTiePer; ++u) {
      if (a + u < i1) {
        const bool eq = k[u] == T;
        keep[a + u] = (k[u] > T || (eq && r < need)) ? 1 : 0;
        r += eq ? 1 : 0;
      }
    }
    base += tot;
  }
}

// keep[i] for the group's range: fill ≥ 0 writes that value (n_keep ≤ 0 or
// ≥ n), else the select's result.
__global__ __launch_bounds__(kSelGroupThreads) void topk_mark_kernel(const float* norms, int n,
                                                                     int chunk, int n_keep,
                                                                     const uint32_t* ws, int fill,
                                                                     uint8_t* keep) {
  __shared__ int s_wave[kSelGroupThreads / kWave];
  __shared__ uint32_t s_st[4];
  const int t = threadIdx.x;
  int64_t i0, i1;
  group_range(n, chunk, i0, i1);
  if (fill >= 0) {
    for (int64_t i = i0 + t; i < i1; i += kSelGroupThreads) keep[i] = (uint8_t)fill;
    return;
  }
  sel_state(ws, kSelPasses, n_keep, s_st);
  __syncthreads();
  const uint32_t T = s_st[0];
  const int need = (int)s_st[2];
  if (s_st[2] == s_st[3]) {
    // every key equal to T is kept: no ranks needed
    for (int64_t b = i0; b < i1; b += kSelGroupThreads * kSelUnroll) {
      uint32_t k[kSelUnroll];
#pragma unroll
      for (int u = 0; u < kSelUnroll; ++u) {
        const int64_t i = b + u * kSelGroupThreads + t;
        k[u] = i < i1 ? norm_key(norms[i]) : 0u;
      }
#pragma unroll
      for (int u = 0; u < kSelUnroll; ++u) {
        const int64_t i = b + u * kSelGroupThreads + t;
        if (i < i1) keep[i] = k[u] >= T ? 1 : 0;
      }
    }
    return;
  }
  // keys equal to T in the ranges of the groups before this one
  const uint32_t d = T & 255u;
  int before = 0;
  for (int g = t; g < (int)blockIdx.x; g += kSelGroupThreads)
    before += (int)ws[kWsGroupHist + (int64_t)g * 256 + d];
  int tot;
  group_exclusive(before, tot, s_wave);
  tie_pass(norms, i0, i1, T, need, tot, keep, s_wave);
}

// out[i, j] = input as fp32 where block (i / p, j / q) is kept, else 0.
// vin: every run of 4 elements starting at a multiple of 4 lies in one block
// and is aligned to 4 elements, so it is one vector load (16 bytes of fp32,
// 8 of 16-bit values) under one keep flag.
template <int DT>
__global__ __launch_bounds__(kThreads) void block_mask_kernel(const void* S, int64_t lds, int n,
                                                              int m, int p, int q, int NBK,
                                                              const uint8_t* keep, float* out,
                                                              int64_t ldo, bool vec, bool vin) {
  for (int i = blockIdx.y; i < n; i += gridDim.y) {
    const uint8_t* krow = keep + (int64_t)(i / p) * NBK;
    for (int j0 = 4 * (blockIdx.x * kThreads + threadIdx.x); j0 < m; j0 += 4 * gridDim.x * kThreads) {
      float v[4];
      if (vin && j0 + 4 <= m) {
        v[0] = v[1] = v[2] = v[3] = 0.f;
        if (krow[j0 / q]) {
          const int64_t e = (int64_t)i * lds + j0;
          if constexpr (DT == DT_F32) {
            const float4 f = *(const float4*)((const float*)S + e);
            v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
          } else {
            const uint2 h = *(const uint2*)((const uint16_t*)S + e);
            v[0] = DT == DT_BF16 ? bf16_to_f32(h.x & 0xffffu) : f16_to_f32(h.x & 0xffffu);
            v[1] = DT == DT_BF16 ? bf16_to_f32(h.x >> 16) : f16_to_f32(h.x >> 16);
            v[2] = DT == DT_BF16 ? bf16_to_f32(h.y & 0xffffu) : f16_to_f32(h.y & 0xffffu);
            v[3] = DT == DT_BF16 ? bf16_to_f32(h.y >> 16) : f16_to_f32(h.y >> 16);
          }
        }
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int j = j0 + u;
          v[u] = (j < m && krow[j / q]) ? elem_f32<DT>(S, (int64_t)i * lds + j) : 0.f;
        }
      }
      if (vec && j0 + 4 <= m) {
        *(float4*)(out + (int64_t)i * ldo + j0) = make_float4(v[0], v[1], v[2], v[3]);
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (j0 + u < m) out[(int64_t)i * ldo + j0 + u] = v[u];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// N:M projection (ssalaad/inference/egar.py:284-292, _project_S_nm): in each
// run of nm_m consecutive entries of a row keep the nm_n of largest
// magnitude; out = value · (kept ? 1 : 0) in fp32. The reference multiplies by
// the mask, so a dropped negative value gives −0 and a dropped ±inf or NaN
// gives NaN; the same multiply here gives the same. An entry's order key is
// its magnitude's bit pattern (non-negative floats order like their bits),
// every NaN folded above +inf; equal keys go to the lower index. One thread
// per group; NMM ≥ nm_m bounds the unrolled group.
// ---------------------------------------------------------------------------
// VEC (nm_m == NMM, every group aligned in R, out and keep): the group is read
// with 16-byte (or, for four 16-bit values, 8-byte) loads and written with
// 16-byte stores of out and one store of its NMM keep bytes.
template <int DT, int NMM, bool VEC>
__global__ __launch_bounds__(kThreads) void nm_project_kernel(const void* R, int64_t ldr, int n,
                                                              int groups_per_row, int nm_n,
                                                              int nm_m, float* out, int64_t ldo,
                                                              uint8_t* keep, int64_t ldk) {
  constexpr int EB = Elem<DT>::bytes;
  const int64_t total = (int64_t)n * groups_per_row;
  for (int64_t g = (int64_t)blockIdx.x * kThreads + threadIdx.x; g < total;
       g += (int64_t)gridDim.x * kThreads) {
    const int64_t row = g / groups_per_row;
    const int64_t c0 = (g % groups_per_row) * nm_m;
    float v[NMM];
    uint32_t key[NMM];
    if constexpr (VEC) {
      constexpr int W = NMM * EB / 4;  // 32-bit words of the group
      uint32_t w[W];
      const char* src = (const char*)R + (row * ldr + c0) * EB;
      if constexpr (W % 4 == 0) {
#pragma unroll
        for (int x = 0; x < W / 4; ++x) {
          const uint4 q = ((const uint4*)src)[x];
          w[4 * x] = q.x, w[4 * x + 1] = q.y, w[4 * x + 2] = q.z, w[4 * x + 3] = q.w;
        }
      } else {
        const uint2 q = *(const uint2*)src;
        w[0] = q.x, w[1] = q.y;
      }
#pragma unroll
      for (int j = 0; j < NMM; ++j) {
        if constexpr (DT == DT_F32) v[j] = __uint_as_float(w[j]);
        else {
          const uint32_t h = (w[j / 2] >> (16 * (j & 1))) & 0xffffu;
          v[j] = DT == DT_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < NMM; ++j) v[j] = j < nm_m ? elem_f32<DT>(R, row * ldr + c0 + j) : 0.f;
    }
#pragma unroll
    for (int j = 0; j < NMM; ++j) {
      const uint32_t b = __float_as_uint(v[j]) & 0x7fffffffu;
      key[j] = j < nm_m ? (b > 0x7f800000u ? kNanKey : b) : 0u;
    }
    float o[NMM];
    uint8_t kb[NMM];
#pragma unroll
    for (int j = 0; j < NMM; ++j) {
      int rank = 0;
#pragma unroll
      for (int k = 0; k < NMM; ++k)
        rank += (k < nm_m && (key[k] > key[j] || (key[k] == key[j] && k < j))) ? 1 : 0;
      const bool kept = rank < nm_n;
      o[j] = v[j] * (kept ? 1.f : 0.f);
      kb[j] = kept ? 1 : 0;
    }
    if constexpr (VEC) {
      float4* dst = (float4*)(out + row * ldo + c0);
#pragma unroll
      for (int x = 0; x < NMM / 4; ++x)
        dst[x] = make_float4(o[4 * x], o[4 * x + 1], o[4 * x + 2], o[4 * x + 3]);
      if (keep) {
        uint32_t kw[NMM / 4];
#pragma unroll
        for (int x = 0; x < NMM / 4; ++x)
          kw[x] = kb[4 * x] | (kb[4 * x + 1] << 8) | (kb[4 * x + 2] << 16) |
                  ((uint32_t)kb[4 * x + 3] << 24);
        uint8_t* kd = keep + row * ldk + c0;
        if constexpr (NMM == 4) *(uint32_t*)kd = kw[0];
        else if constexpr (NMM == 8) *(uint2*)kd = make_uint2(kw[0], kw[1]);
        else {
#pragma unroll
          for (int x = 0; x < NMM / 16; ++x)
            ((uint4*)kd)[x] = make_uint4(kw[4 * x], kw[4 * x + 1], kw[4 * x + 2], kw[4 * x + 3]);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < NMM; ++j) {
        if (j >= nm_m) break;
        out[row * ldo + c0 + j] = o[j];
        if (keep) keep[row * ldk + c0 + j] = kb[j];
      }
    }
  }
}

}  // namespace
}  // namespace ssl

using namespace ssl;

extern "C" {

// Workgroups of the many-workgroup select: kSelGroupKeys keys each, at most
// kMaxSelGroups (then more keys each).
static int64_t select_groups(int64_t n_blocks) {
  return std::min<int64_t>((n_blocks + kSelGroupKeys - 1) / kSelGroupKeys, kMaxSelGroups);
}

int64_t ssl_block_topk_workspace_size(int64_t n_blocks) {
  if (n_blocks <= 0) return 0;
  const int64_t words = kWsGroupHist + select_groups(n_blocks) * 256;
  return (words * 4 + 255) / 256 * 256;
}

int ssl_block_topk(const void* S, int64_t lds, int64_t NB, int64_t NBK, int32_t block_p,
                   int32_t block_q, int32_t dtype, int64_t n_keep, float* norms, uint8_t* keep,
                   float* out, int64_t ldo, void* workspace, int64_t workspace_bytes,
                   void* stream) {
  clear_error();
  if (block_p <= 0 || block_q <= 0 || NB < 0 || NBK < 0) return fail(SSL_ERR_INVALID, "bad sizes");
  if (dtype != SSL_F32 && dtype != SSL_BF16 && dtype != SSL_F16)
    return fail(SSL_ERR_UNSUPPORTED, "unsupported dtype %d", dtype);
  const int64_t nblocks = NB * NBK;
  if (nblocks == 0) return SSL_OK;
  if (nblocks > 0x7fffffffLL || NB * block_p > 0x7fffffffLL || NBK * block_q > 0x7fffffffLL)
    return fail(SSL_ERR_INVALID, "too many blocks");
  if (lds < NBK * block_q) return fail(SSL_ERR_INVALID, "lds smaller than the row");
  if (!S || !norms || !keep) return fail(SSL_ERR_INVALID, "null pointer");
  if (out && ldo < NBK * block_q) return fail(SSL_ERR_INVALID, "ldo smaller than the row");
  if (!workspace || workspace_bytes < ssl_block_topk_workspace_size(nblocks) ||
      (uintptr_t)workspace % 16 != 0)
    return fail(SSL_ERR_WORKSPACE, "block projection workspace missing, small or not 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  const unsigned grid = (unsigned)((nblocks + kWaves - 1) / kWaves);
  const int n = (int)(NB * block_p), m = (int)(NBK * block_q);
  const int mcols = (m + 4 * kThreads - 1) / (4 * kThreads);
  const dim3 mgrid((unsigned)(mcols < 64 ? mcols : 64), (unsigned)(n < 65535 ? n : 65535));
  const int eb = elem_bytes(dtype);
  const int keep_n = (int)(n_keep < 0 ? 0 : (n_keep > nblocks ? nblocks : n_keep));
  // 16-byte pieces of the input: aligned base, row stride and block rows
  const bool vec_in = ((uintptr_t)S % 16 == 0) && (lds * eb) % 16 == 0 && (block_q * eb) % 16 == 0;
  const bool vec_out = out && ((uintptr_t)out % 16 == 0) && ldo % 4 == 0;
  const bool vec_mask_in = ((uintptr_t)S % (4 * eb) == 0) && lds % 4 == 0 && block_q % 4 == 0;
  // The select: one workgroup over keys staged in its LDS, or many workgroups
  // over kSelGroupKeys keys each (four histogram launches and the marking).
  const int64_t knob = debug_knobs().topk_groups;
  const bool many = knob == 2 || (knob == 0 && nblocks > kSelOneGroupMax);
  const bool fill = keep_n <= 0 || keep_n >= nblocks;
  const int groups = (int)select_groups(nblocks);
  const int chunk = (int)((nblocks + groups - 1) / groups);
  uint32_t* ws = (uint32_t*)workspace;
  // blocks of at most 64 pieces of 16 bytes: several blocks per wave
  const int64_t pieces = vec_in ? (int64_t)block_p * (block_q * eb / 16) : 0;
  const bool small = vec_in && pieces <= kWave;
  int lanes = 1;
  while (small && lanes < pieces) lanes <<= 1;
  const int64_t small_blocks = (int64_t)kSmallRounds * (kWave / lanes);  // per wave
  const int64_t small_waves = small ? (nblocks + small_blocks - 1) / small_blocks : 0;
  const unsigned small_grid = (unsigned)((small_waves + kWaves - 1) / kWaves);
  uint32_t* init_ws = many && !fill ? ws : nullptr;
#define SSL_PROJECT(DTC)                                                                       \
  if (small)                                                                                    \
    hipLaunchKernelGGL(block_sumsq_small_kernel<DTC>, dim3(small_grid), dim3(kThreads), 0, s, S, \
                       lds, nblocks, (int)NBK, block_p, block_q, lanes, norms, init_ws);         \
  else                                                                                          \
    hipLaunchKernelGGL(block_sumsq_kernel<DTC>, dim3(grid), dim3(kThreads), 0, s, S, lds,        \
                       (int)NB, (int)NBK, block_p, block_q, vec_in, norms, init_ws);            \
  if (!many && nblocks <= kLdsKeys)                                                              \
    hipLaunchKernelGGL(block_topk_kernel<true>, dim3(1), dim3(kSelThreads),                      \
                       (unsigned)(4 * nblocks), s, norms, (int)nblocks, keep_n, keep);           \
  else if (!many)                                                                               \
    hipLaunchKernelGGL(block_topk_kernel<false>, dim3(1), dim3(kSelThreads), 0, s, norms,        \
                       (int)nblocks, keep_n, keep);                                             \
  else if (fill)                                                                                \
    hipLaunchKernelGGL(topk_mark_kernel, dim3(groups), dim3(kSelGroupThreads), 0, s, norms,      \
                       (int)nblocks, chunk, keep_n, ws, keep_n > 0 ? 1 : 0, keep);              \
  else {                                                                                        \
    hipLaunchKernelGGL(topk_hist_kernel<0>, dim3(groups), dim3(kSelGroupThreads), 0, s, norms,   \
                       (int)nblocks, chunk, keep_n, ws);                                        \
    hipLaunchKernelGGL(topk_hist_kernel<1>, dim3(groups), dim3(kSelGroupThreads), 0, s, norms,   \
                       (int)nblocks, chunk, keep_n, ws);                                        \
    hipLaunchKernelGGL(topk_hist_kernel<2>, dim3(groups), dim3(kSelGroupThreads), 0, s, norms,   \
                       (int)nblocks, chunk, keep_n, ws);                                        \
    hipLaunchKernelGGL(topk_hist_kernel<3>, dim3(groups), dim3(kSelGroupThreads), 0, s, norms,   \
                       (int)nblocks, chunk, keep_n, ws);                                        \
    hipLaunchKernelGGL(topk_mark_kernel, dim3(groups), dim3(kSelGroupThreads), 0, s, norms,      \
                       (int)nblocks, chunk, keep_n, ws, -1, keep);                              \
  }                                                                                             \
  if (out)                                                                                      \
    hipLaunchKernelGGL(block_mask_kernel<DTC>, mgrid, dim3(kThreads), 0, s, S, lds, n, m,        \
                       block_p, block_q, (int)NBK, keep, out, ldo, vec_out, vec_mask_in);
  switch (dtype) {
    case SSL_F32: SSL_PROJECT(DT_F32) break;
    case SSL_BF16: SSL_PROJECT(DT_BF16) break;
    case SSL_F16: SSL_PROJECT(DT_F16) break;
  }
#undef SSL_PROJECT
  return check_hip(hipGetLastError(), "block projection launch");
}

int ssl_project_nm(const void* R, int64_t ldr, int64_t n, int64_t m, int32_t nm_n, int32_t nm_m,
                   int32_t dtype, float* out, int64_t ldo, uint8_t* keep, int64_t ldk,
                   void* stream) {
  clear_error();
  if (n < 0 || m < 0) return fail(SSL_ERR_INVALID, "negative size");
  if (nm_m < 1 || nm_m > 32)
    return fail(SSL_ERR_UNSUPPORTED, "group size nm_m=%d outside [1, 32]", nm_m);
  if (nm_n < 0 || nm_n > nm_m)
    return fail(SSL_ERR_INVALID, "nm_n=%d outside [0, nm_m=%d]", nm_n, nm_m);
  if (m % nm_m) return fail(SSL_ERR_INVALID, "m=%lld is not a multiple of nm_m=%d", (long long)m, nm_m);
  if (dtype != SSL_F32 && dtype != SSL_BF16 && dtype != SSL_F16)
    return fail(SSL_ERR_UNSUPPORTED, "unsupported dtype %d", dtype);
  if (n == 0 || m == 0) return SSL_OK;
  if (!R || !out) return fail(SSL_ERR_INVALID, "null pointer");
  if (ldr < m || ldo < m || (keep && ldk < m)) return fail(SSL_ERR_INVALID, "row stride smaller than the row");
  if (n > 0x7fffffffLL || m / nm_m > 0x7fffffffLL) return fail(SSL_ERR_INVALID, "too large");
  const int64_t total = n * (m / nm_m);
  const int64_t want = (total + kThreads - 1) / kThreads;
  const unsigned grid = (unsigned)(want < 8192 ? want : 8192);
  hipStream_t s = (hipStream_t)stream;
  const int gpr = (int)(m / nm_m);
  // Whole aligned groups: nm_m a power of two from 4, every group's start in R
  // aligned to its own size (at most 16 bytes), out rows to 16 bytes, keep
  // rows to the group's byte count (at most 16).
  const int eb = elem_bytes(dtype);
  const bool pow2 = nm_m == 4 || nm_m == 8 || nm_m == 16 || nm_m == 32;
  const int64_t ga = std::min<int64_t>((int64_t)nm_m * eb, 16), ka = std::min(nm_m, 16);
  const bool vec = pow2 && (uintptr_t)R % ga == 0 && (ldr * eb) % ga == 0 &&
                   (uintptr_t)out % 16 == 0 && ldo % 4 == 0 &&
                   (!keep || ((uintptr_t)keep % ka == 0 && ldk % ka == 0));
#define SSL_NM(DTC, NMM)                                                                       \
  do {                                                                                          \
    if (vec && nm_m == NMM)                                                                     \
      hipLaunchKernelGGL((nm_project_kernel<DTC, NMM, true>), dim3(grid), dim3(kThreads), 0, s,   \
                         R, ldr, (int)n, gpr, nm_n, nm_m, out, ldo, keep, ldk);                 \
    else                                                                                        \
      hipLaunchKernelGGL((nm_project_kernel<DTC, NMM, false>), dim3(grid), dim3(kThreads), 0, s,  \
                         R, ldr, (int)n, gpr, nm_n, nm_m, out, ldo, keep, ldk);                 \
  } while (0)
#define SSL_NM_DT(DTC)                   \
  if (nm_m <= 4) SSL_NM(DTC, 4);         \
  else if (nm_m <= 8) SSL_NM(DTC, 8);    \
  else if (nm_m <= 16) SSL_NM(DTC, 16);  \
  else SSL_NM(DTC, 32);
  switch (dtype) {
    case SSL_F32: SSL_NM_DT(DT_F32) break;
    case SSL_BF16: SSL_NM_DT(DT_BF16) break;
    case SSL_F16: SSL_NM_DT(DT_F16) break;
  }
#undef SSL_NM_DT
#undef SSL_NM
  return check_hip(hipGetLastError(), "N:M projection launch");
}

}  // extern "C"
