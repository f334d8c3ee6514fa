#pragma once
// Device code of the streaming SLR / BSR kernels (slr_kernel), shared by the
// per-dtype instantiation files stream_{bf16,f16,f32}.hip; the host side is
// bsr_stream.hip.
//
// Decode-shaped calls (up to 64 token rows per tile) are HBM-bound: every
// weight byte is read once per token tile and feeds a handful of MFMAs. The
// kernels are therefore organised around keeping as many weight bytes in
// flight as possible and around the few cross-workgroup exchanges that the
// computation needs, because on a loaded device each exchange (a device-coherent
// store, its acknowledgement and a counter update) costs microseconds.
//
// Row-resident workgroups. A plan (plan.cpp) gives one workgroup (8 waves) a
// whole block-row — its sparse (q, p) blocks and, for the fused linear, the
// 32-rank slices of A — unless the row is long, in which case it is split into
// a few chunks. The 8 waves take the units round-robin and issue all of their
// loads before the first MFMA (about 32 blocks of 64×64 in one batch), so a
// typical row costs one memory round trip. Weights go from HBM straight into
// registers (no LDS staging: each byte is used once per token tile); the sparse
// blocks, stored (q, p) as in the reference module, are transposed into MFMA
// fragments with register byte permutes.
//
// Reduction. The 8 wave tiles are summed in LDS in a fixed tree order; wave 0
// then runs the epilogue (bias, or the in-place add of the op) and stores the
// row tile once.
//
// Split rows. A chunk of a split row stores its fp32 tile with device-coherent
// (sc1) stores, waits for the acknowledgement and bumps the row's counter. In
// the fused linear the row's finaliser chunk (the one with the low-rank units,
// launched after all other chunks) waits for the others and sums the partials in
// chunk order; in the in-place op the chunk that arrives last does. Results are
// deterministic either way. Only exchanged data is accessed device-coherently;
// no workgroup writes back or invalidates a whole L2.
//
// The latent. The fused launch starts with one workgroup per 16-rank tile of
// t = x·Bᵀ and chunk of in_features (one batch of loads each); each stores its
// fp32 partial device-coherently and bumps the token tile's ready counter. The
// consumers sum the partials in chunk order and round once. Low-rank units
// load their A slices first and wait for that counter (bounded spin) only then.
// Only one thread per workgroup polls. Workgroups of one XCD are dispatched in
// index order, so every workgroup a chunk may wait for (latent tiles, earlier
// chunks of its row) is resident or done before it, and every wait ends. The
// latent counters are monotonic per plan (a consumer's ticket tells it which
// launch it belongs to), so no launch needs an end-of-launch reset.

#include "abi_internal.h"
#include "slr_common.h"

namespace ssl {

enum : int { MODE_OP = 0, MODE_FUSED = 1 };
enum : int { SF_BSR = 0, SF_NM24 = 1 };  // sparse block storage

constexpr int kSW = 8;            // waves per streaming workgroup
constexpr int kST = kSW * kWave;  // threads per streaming workgroup

// Polls of a counter before a wait gives up and flags an error in the status
// word (seconds; a healthy launch waits microseconds). ssl_debug_set can lower
// it for tests of the give-up path.
constexpr int kSpinLimit = 1 << 22;

// ---------------------------------------------------------------------------
// Device-coherent (agent scope) 32-bit accesses for data exchanged between
// workgroups of one launch: sc1 loads/stores, no cache-wide maintenance.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void st_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev_u32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_dev_u32(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int rmw_add(int* p, int v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int ld_int(const int* p) {
  return __hip_atomic_load(const_cast<int*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_int(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Vector forms of the same device-coherent accesses: buffer loads/stores with
// the sc1 cache policy (what the relaxed agent-scope atomics above compile to),
// N = 1, 2, 3 or 4 floats at a wave-uniform base plus a per-lane byte offset below
// 2 GiB (the host checks the workspace size).
constexpr int kSc1 = 16;  // cache-policy bit: sc1
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dev_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff,
                                           0x00020000);
}
template <int N>
__device__ __forceinline__ void ld_dev_vec(__amdgpu_buffer_rsrc_t r, int byte_off, float* v) {
  if constexpr (N == 4) {
    const auto u = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kSc1);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __uint_as_float(u[i]);
  } else if constexpr (N == 2) {
    const auto u = __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, kSc1);
    v[0] = __uint_as_float(u[0]);
    v[1] = __uint_as_float(u[1]);
  } else if constexpr (N == 3) {
#pragma unroll
    for (int i = 0; i < 3; ++i)
      v[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, byte_off + 4 * i, 0, kSc1));
  } else {
    static_assert(N == 1, "1, 2, 3 or 4 floats");
    v[0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, kSc1));
  }
}
template <int N>
__device__ __forceinline__ void st_dev_vec(__amdgpu_buffer_rsrc_t r, int byte_off, const float* v) {
  if constexpr (N == 4) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 u = {__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                     __float_as_uint(v[3])};
    __builtin_amdgcn_raw_buffer_store_b128(u, r, byte_off, 0, kSc1);
  } else if constexpr (N == 2) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 u = {__float_as_uint(v[0]), __float_as_uint(v[1])};
    __builtin_amdgcn_raw_buffer_store_b64(u, r, byte_off, 0, kSc1);
  } else if constexpr (N == 3) {
#pragma unroll
    for (int i = 0; i < 3; ++i)
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v[i]), r, byte_off + 4 * i, 0, kSc1);
  } else {
    static_assert(N == 1, "1, 2, 3 or 4 floats");
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v[0]), r, byte_off, 0, kSc1);
  }
}

// All of this thread's earlier memory operations have completed (stores are
// acknowledged by the device-coherent level).
__device__ __forceinline__ void wait_mem() { __builtin_amdgcn_s_waitcnt(0); }

typedef unsigned long long u64;
constexpr int kLatentUnits = 840;  // divisible by every latent split 1..8
__device__ __forceinline__ u64 rmw_add64(u64* p, u64 v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u64 ld_u64(const u64* p) {
  return __hip_atomic_load(const_cast<u64*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_u64(u64* p, u64 v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Spin (one lane) until *flag >= target; bounded (`polls`), sets *status on
// timeout. The caller goes on either way, so every workgroup of the launch
// still ends; a wait that gave up leaves its tile unreliable, which the status
// word reports.
template <typename T, int SLEEP = 2>
__device__ __forceinline__ void wait_at_least(const T* flag, T target, u64* status, int polls) {
  int n = 0;
  while (__hip_atomic_load(const_cast<T*>(flag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) <
         target) {
    __builtin_amdgcn_s_sleep(SLEEP);
    if (++n > polls) {
      st_u64(status, 1);
      break;
    }
  }
}

// One KE-element fragment (16 bytes) of the final latent, read device-coherently.
template <int DT, int KE>
__device__ __forceinline__ typename Mma<DT, KE>::Frag ld_dev_frag(__amdgpu_buffer_rsrc_t r,
                                                                  int byte_off) {
  static_assert(KE * Elem<DT>::bytes == 16, "16-byte fragments");
  const auto u = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kSc1);
  typename Mma<DT, KE>::Frag f;
  static_assert(sizeof(f) == 16, "fragment image");
  __builtin_memcpy(&f, &u, 16);
  return f;
}

// One KE-element fragment of x read device-coherently: in a chained launch x
// is a row tile that another workgroup of the same launch wrote. `valid`
// (0..KE) elements are read, the rest are zero.
template <int DT, int KE>
__device__ __forceinline__ typename Mma<DT, KE>::Frag ld_dev_kfrag(__amdgpu_buffer_rsrc_t r,
                                                                   int byte_off, int valid) {
  using F = typename Mma<DT, KE>::Frag;
  constexpr int EB = Elem<DT>::bytes;
  static_assert(sizeof(F) == KE * EB, "fragment image");
  F f;
  if (valid >= KE) {
    if constexpr (KE * EB == 16) {
      const auto u = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kSc1);
      __builtin_memcpy(&f, &u, 16);
    } else {
      static_assert(KE * EB == 8, "8- or 16-byte fragments");
      const auto u = __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, kSc1);
      __builtin_memcpy(&f, &u, 8);
    }
  } else if constexpr (DT == DT_F32) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      f.f[e] = e < valid ? __uint_as_float(
                               __builtin_amdgcn_raw_buffer_load_b32(r, byte_off + 4 * e, 0, kSc1))
                         : 0.f;
  } else {
#pragma unroll
    for (int d = 0; d < KE / 2; ++d) {
      const uint32_t lo =
          2 * d < valid ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, byte_off + 4 * d, 0, kSc1)
                        : 0u;
      const uint32_t hi = 2 * d + 1 < valid ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(
                                                  r, byte_off + 4 * d + 2, 0, kSc1)
                                            : 0u;
      f.d[d] = lo | (hi << 16);
    }
  }
  return f;
}

// W adjacent output elements stored device-coherently (a chained stage's
// output, read by a later stage of the same launch).
template <int DT, int W>
__device__ __forceinline__ void st_w_dev(__amdgpu_buffer_rsrc_t r, int byte_off,
                                         const float (&v)[W]) {
  if constexpr (DT == DT_F32) {
    st_dev_vec<W>(r, byte_off, v);
  } else if constexpr (W == 1 || W == 3) {
#pragma unroll
    for (int i = 0; i < W; ++i)
      __builtin_amdgcn_raw_buffer_store_b16((unsigned short)to_bits<DT>(v[i]), r, byte_off + 2 * i,
                                            0, kSc1);
  } else {
    uint32_t w[W / 2];
#pragma unroll
    for (int i = 0; i < W / 2; ++i) w[i] = to_bits<DT>(v[2 * i]) | (to_bits<DT>(v[2 * i + 1]) << 16);
    if constexpr (W == 4) {
      typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
      const u32x2 u = {w[0], w[1]};
      __builtin_amdgcn_raw_buffer_store_b64(u, r, byte_off, 0, kSc1);
    } else {
      __builtin_amdgcn_raw_buffer_store_b32(w[0], r, byte_off, 0, kSc1);
    }
  }
}

// ---------------------------------------------------------------------------
// Deterministic reduction of the kSW wave tiles into wave 0's registers. Tiles
// of up to 4 KiB (MT·W ≤ 4: decode tiles of up to 64 output features) go
// through LDS at once: waves 1..7 store, one barrier, wave 0 adds them in wave
// order (measured: the three halving rounds' six barriers took about 0.6 µs of
// a 7B decode launch's tail). Larger tiles take rounds of halving; in each
// round wave i (< half) adds wave i + half's tile, passed through LDS in groups
// of SLOTS tiles.
// ---------------------------------------------------------------------------
template <int MT, int W>
constexpr bool flat_reduce() {
  return MT * W <= 4;
}
template <int MT, int W>
constexpr int red_slots() {
  return flat_reduce<MT, W>() ? kSW - 1 : (MT * W <= 8 ? 4 : 2);  // LDS: SLOTS × MT·W KiB
}
// The LDS a launch's reductions share: its row workgroups reduce MT·W tiles,
// its latent workgroups MT·1 tiles (which may take the flat form where the row
// tiles do not).
template <int MT, int W>
constexpr int red_len() {
  constexpr int rows = red_slots<MT, W>() * MT * W * kWave;
  constexpr int lat = red_slots<MT, 1>() * MT * kWave;
  return rows > lat ? rows : lat;
}

template <int MT, int W, int NR>
__device__ __forceinline__ void tree_reduce(f32x4 (&acc)[MT][W], f32x4 (&red)[NR], int wid, int lane) {
  constexpr int SLOTS = red_slots<MT, W>();
  static_assert(SLOTS * MT * W * kWave <= NR, "the reduction's tiles fit the launch's LDS buffer");
  if constexpr (flat_reduce<MT, W>()) {
    if (wid > 0) {
      f32x4* slot = red + (wid - 1) * (MT * W * kWave);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int s = 0; s < W; ++s) slot[(mt * W + s) * kWave + lane] = acc[mt][s];
    }
    __syncthreads();
    if (wid == 0) {
#pragma unroll
      for (int k = 0; k < kSW - 1; ++k) {
        const f32x4* slot = red + k * (MT * W * kWave);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int s = 0; s < W; ++s) acc[mt][s] += slot[(mt * W + s) * kWave + lane];
      }
    }
    return;
  }
#pragma unroll
  for (int half = kSW / 2; half >= 1; half /= 2) {
#pragma unroll
    for (int g0 = 0; g0 < half; g0 += SLOTS) {
      const int g1 = g0 + SLOTS < half ? g0 + SLOTS : half;
      if (wid >= half + g0 && wid < half + g1) {
        f32x4* slot = red + (wid - half - g0) * (MT * W * kWave);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int s = 0; s < W; ++s) slot[(mt * W + s) * kWave + lane] = acc[mt][s];
      }
      __syncthreads();
      if (wid >= g0 && wid < g1) {
        const f32x4* slot = red + (wid - g0) * (MT * W * kWave);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int s = 0; s < W; ++s) acc[mt][s] += slot[(mt * W + s) * kWave + lane];
      }
      __syncthreads();
    }
  }
}

// Wave-level exchange of a row tile held in registers (lane-native layout:
// lane (c, g), element e of column tile s -> row 16·mt + 4g + e, column W·c + s).
// Partial tiles live in memory row-major [16·MT][16·W] fp32.
template <int MT, int W>
__device__ __forceinline__ void store_partial(const f32x4 (&acc)[MT][W], float* part, int Mrem,
                                              int lane) {
  constexpr int TP = 16 * W;
  const int c = lane & 15, g = lane >> 4;
  const auto r = dev_rsrc(part);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int rr = mt * 16 + 4 * g + e;
      if (rr < Mrem) {
        float v[W];
#pragma unroll
        for (int s = 0; s < W; ++s) v[s] = acc[mt][s][e];
        st_dev_vec<W>(r, (rr * TP + W * c) * 4, v);
      }
    }
}
template <int MT, int W>
__device__ __forceinline__ void add_partial(f32x4 (&tot)[MT][W], const float* part, int Mrem,
                                            int lane) {
  constexpr int TP = 16 * W;
  const int c = lane & 15, g = lane >> 4;
  const auto r = dev_rsrc(part);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int rr = mt * 16 + 4 * g + e;
      if (rr < Mrem) {
        float v[W];
        ld_dev_vec<W>(r, (rr * TP + W * c) * 4, v);
#pragma unroll
        for (int s = 0; s < W; ++s) tot[mt][s][e] += v[s];
      }
    }
}

// The same for tiles in any register layout: every lane's accumulators whole,
// lane-native (the TSZ floats of a tile are exactly MT·W f32x4 per lane).
template <int MT, int W>
__device__ __forceinline__ void store_partial_lanes(const f32x4 (&acc)[MT][W], float* part, int lane) {
  const auto r = dev_rsrc(part);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int s = 0; s < W; ++s) {
      const float v[4] = {acc[mt][s][0], acc[mt][s][1], acc[mt][s][2], acc[mt][s][3]};
      st_dev_vec<4>(r, (((mt * W + s) * kWave + lane) * 4) * 4, v);
    }
}
template <int MT, int W>
__device__ __forceinline__ void add_partial_lanes(f32x4 (&tot)[MT][W], const float* part, int lane) {
  const auto r = dev_rsrc(part);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int s = 0; s < W; ++s) {
      float v[4];
      ld_dev_vec<4>(r, (((mt * W + s) * kWave + lane) * 4) * 4, v);
      tot[mt][s] += f32x4{v[0], v[1], v[2], v[3]};
    }
}

// ---------------------------------------------------------------------------
// Kernel arguments (one struct for every mode).
// ---------------------------------------------------------------------------
struct SlrArgs {
  // activations
  const void* x;
  int64_t ldx;
  int M, m;
  // output and the streamed part
  void* y;
  int64_t ldy;
  const int32_t* col;
  const void* values;
  const int32_t* plan;
  int n_chunks;
  int NB;
  int nnz;              // stored blocks (0: not given; bounds the plan's block ranges)
  // Sparse blocks are walked in K slabs of KM rows (the MFMA's k extent):
  // block b's slab ks is KM·p contiguous values at b·blk_bytes + ks·slab_bytes.
  int q;                // block_q: input features per block
  int nks;              // slabs per block (q / KM; 1 for 2:4 storage)
  uint32_t nks_magic;   // ceil(2^32 / nks) when nks > 1: slab → block by a high multiply
  int blk_bytes;        // bytes per stored block
  int slab_bytes;       // bytes per slab
  const void* A;
  int64_t lda;
  const void* bias;
  int64_t n_slots;
  float* part_main;
  int* cnt_main;  // [MG][NB]
  // latent
  const void* B;
  int64_t ldb;
  void* t;          // final latent [MG·16·MT][ldt], activation dtype
  int64_t ldt;
  float* t_part;    // fp32 partials [n_kc][MG][n_rt][MT·256] (lane-native tiles)
  int MG;           // token tiles
  int n_rt;         // 16-rank tiles
  int n_kc;         // in_features chunks of the latent
  int ku_total;     // in_features in KM-column units
  int ku_chunk;     // KM-column units per latent chunk
  int n_lat_wgs;    // latent workgroups at the start of the grid (n_rt·n_kc·MG)
  // Handshake words, all monotonic (never reset): sync[0] is the status (1 =
  // a wait gave up); token tile mg owns sync[1 + mg·(2 + n_rt) ...]:
  //   [0], [1] unused
  //   [2 + rt] arrivals of rank tile rt's K chunks (+kLatentUnits/n_kc each,
  //       so every launch adds exactly kLatentUnits whatever its split)
  // and, in fin's 512-byte slot (mg·kFinCopies + c), c < kFinCopies, copy c of
  // token tile mg's count of final latent tiles written (word 0: +1 per rank
  // tile and launch, to every copy) and consumer tickets (word kFinTicket: +1
  // per consuming workgroup of copy c and launch). With tk_copies = kFinCopies
  // (every block-row has exactly one consuming chunk, lr_wgs = NB) the
  // consumers of block-row `row` use copy row % kFinCopies; otherwise every
  // consumer takes its ticket from copy 0 and polls copy chunk % kFinCopies.
  u64* sync;
  u64* fin;
  int tk_copies;
  int lr_wgs;       // workgroups that consume the latent (per token tile)
  int lat_weight;   // kLatentUnits / n_kc
  // Bounded waits: where a timeout is reported (the caller's status word, or
  // sync[0]), polls before giving up, and an offset added to every wait's
  // target (nonzero only when a test forces the give-up path).
  u64* status;
  int wait_polls;
  int wait_bias;
  // Chained launches (slr_chain_kernel), where x is the output of a member of
  // an earlier stage of the same launch. dep: that stage's words (below), zero
  // at rest, or null when x is an input of the launch; dep_need: the source's
  // row tiles per token tile (its NB); dep_waiters: workgroups of this stage
  // per token tile. done: the words this member's finished row tiles are
  // counted in (the dependent stage's dep), or null; a member with `done`
  // stores its output device-coherently.
  int* dep;
  int dep_need;
  int dep_waiters;
  int dep_lat_base;  // this member's first latent / row workgroup among the
  int dep_row_base;  // stage's waiters of one token tile
  int* done;
  // Fragment-order copies (chained launches, 16-bit, 32- or 64-wide blocks).
  // xf, when set, holds x's whole 32-column units as 1 KiB blocks in the order
  // the MFMA fragments take them: block (mg·MT + mt)·xf_units + u, lane
  // 16g + c's 16 bytes = row 16·mt + c of token tile mg, columns 32u + 8g ..
  // 32u + 8g + 7. A wave then reads a unit with one contiguous 1 KiB load
  // instead of 16 row segments. yf: where this member writes its own output
  // in that order (yf_units units per token row tile), for the stage reading it.
  const void* xf;
  void* yf;
  int xf_units;
  int yf_units;
};

// A stage's words, per token tile: kDepCopies slots of 512 bytes. Slot c holds
// at +0 the finished row tiles j of the source with j % kDepCopies == c, and at
// +256 bytes the waiters w with w % kDepCopies == c that have passed; slot 0
// also holds at +384 bytes the slots whose waiters have all passed. Same-address
// atomics are served one after another (tens of ns each), so each finished row
// tile makes ONE increment, spreading a source's NB increments over 64 words,
// and a waiter reads all 64 counts with one load (a lane each). Measured on
// the 1B layer: every row tile adding to 16 copies (each copy taking NB
// increments) and each waiter taking a returning "passed" ticket before it went
// on cost 1.1-2.8 µs per hand-over; one increment per tile over 16 / 32 / 64
// words: 18.67 k / 19.06 k / 19.11 k tok/s (1282 / 1312 / 1318 at one token row).
constexpr int kDepCopies = 64;
static_assert(kDepCopies <= 64, "a waiter polls the copies with one lane each");
constexpr int kDepSlotInts = 128;
constexpr int kDepPassedInts = 64;
constexpr int kDepClosedInts = 96;
constexpr int kDepSleep = 2;  // s_sleep between polls of a stage's input counts

// Increments slot c's count takes per launch when n things are dealt out by
// index modulo kDepCopies.
__device__ __forceinline__ int dep_share(int n, int c) {
  return n / kDepCopies + (c < n % kDepCopies ? 1 : 0);
}

// Chained stages: wait until the source member has finished every row tile of
// token tile mg in this launch. Wave 0 polls the kDepCopies counts, the barrier
// releases the workgroup. The bookkeeping that returns the words to zero
// (dep_close) runs when the workgroup ends, off the path to its output.
__device__ __forceinline__ void wait_dep(const SlrArgs& a, int mg) {
  if (threadIdx.x < kWave) {
    const int lane = threadIdx.x;
    const bool mine = lane < kDepCopies;
    const int* word = a.dep + ((int64_t)mg * kDepCopies + (mine ? lane : 0)) * kDepSlotInts;
    const int need = dep_share(a.dep_need, mine ? lane : 0) + a.wait_bias;
    for (int n = 0;; ++n) {
      const int v = mine ? __hip_atomic_load(const_cast<int*>(word), __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT)
                         : need;
      if (__builtin_amdgcn_ballot_w64(v < need) == 0) break;
      if (n >= a.wait_polls) {
        if (lane == 0) st_u64(a.status, 1);
        break;
      }
      __builtin_amdgcn_s_sleep(kDepSleep);
    }
  }
  __syncthreads();
}

// Called once by each waiter (wave 0, after its workgroup's work): w is its
// index among the stage's waiters of token tile mg. The waiter that passes last
// subtracts what the launch added to every word, so the words are zero at rest
// whatever the order of arrivals, a wait that gave up included.
__device__ __forceinline__ void dep_close(const SlrArgs& a, int mg, int w) {
  const int lane = threadIdx.x;
  int* base = a.dep + (int64_t)mg * kDepCopies * kDepSlotInts;
  const int c = w % kDepCopies;
  int last = 0;
  if (lane == 0) {
    last = rmw_add(base + c * kDepSlotInts + kDepPassedInts, 1) == dep_share(a.dep_waiters, c) - 1;
    if (last) {
      const int slots = a.dep_waiters < kDepCopies ? a.dep_waiters : kDepCopies;
      last = rmw_add(base + kDepClosedInts, 1) == slots - 1;
    }
  }
  if (!__builtin_amdgcn_readfirstlane(last)) return;
  if (lane < kDepCopies) {
    const int slots = a.dep_waiters < kDepCopies ? a.dep_waiters : kDepCopies;
    const int n_src = dep_share(a.dep_need, lane);
    if (n_src) rmw_add(base + lane * kDepSlotInts, -n_src);
    if (lane < slots) rmw_add(base + lane * kDepSlotInts + kDepPassedInts, -dep_share(a.dep_waiters, lane));
    if (lane == 0) rmw_add(base + kDepClosedInts, -slots);
  }
}

__device__ __forceinline__ u64* tile_sync(const SlrArgs& a, int mg) {
  return a.sync + 1 + (int64_t)mg * (2 + a.n_rt);
}

// A token tile's final-latent counts, in kFinCopies 512-byte slots: rank tile
// rt adds 1 to slot rt % kFinCopies's count when its final tile is written (one
// increment, so no count takes more than ceil(n_rt / kFinCopies) per launch),
// and a consumer reads all the counts with one load (a lane each). Word
// kFinTicket of each slot holds consumer tickets, taken by the consumers of
// block-row `row` from slot row % kFinCopies: 16 slots against 8 spread the
// tickets of a stage's hundreds of row workgroups thinner (1B stack decode
// 19.13 k → 19.36 k tok/s; 32 slots the same).
constexpr int kFinCopies = 16;
static_assert(kFinCopies <= 64, "a consumer polls the copies with one lane each");
constexpr int kFinSlotWords = 64;
constexpr int kFinTicket = 32;
__device__ __forceinline__ u64* fin_copy(const SlrArgs& a, int mg, int c) {
  return a.fin + ((int64_t)mg * kFinCopies + c) * kFinSlotWords;
}
__device__ __forceinline__ int fin_share(int n, int c) {
  return n / kFinCopies + (c < n % kFinCopies ? 1 : 0);
}

// Wave 0 of a consumer: wait until every rank tile of token tile mg has its
// final latent of launch `launch` (counted from the consumer's ticket: every
// launch adds fin_share(n_rt, c) to slot c, so launch k is complete when slot c
// holds (k + 1)·fin_share(n_rt, c)).
__device__ __forceinline__ void wait_fin(const SlrArgs& a, int mg, u64 launch) {
  const int lane = threadIdx.x;
  const bool mine = lane < kFinCopies;
  const u64* word = fin_copy(a, mg, mine ? lane : 0);
  const u64 need = (launch + 1) * (u64)fin_share(a.n_rt, mine ? lane : 0) + (u64)a.wait_bias;
  for (int n = 0;; ++n) {
    const u64 v = mine ? __hip_atomic_load(const_cast<u64*>(word), __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT)
                       : need;
    if (__builtin_amdgcn_ballot_w64(v < need) == 0) break;
    if (n >= a.wait_polls) {
      if (lane == 0) st_u64(a.status, 1);
      break;
    }
    __builtin_amdgcn_s_sleep(2);
  }
}

// ---------------------------------------------------------------------------
// Latent workgroup: t[token tile, 16-rank tile rt] over all of in_features.
// ---------------------------------------------------------------------------
// CH (chained launches): 0 = an ordinary launch; 1 = a chained member whose x
// is an input of the launch; 2 = a chained member whose x another stage of the
// launch writes: its B loads go out before it waits for x, and x is read
// device-coherently.
// TF (16-bit activations): t written in fragment order (units of 32 ranks,
// 1 KiB per 16 token rows, lane 16g + c's 16 bytes = token row c, ranks
// 8g .. 8g + 7 of the unit), the tile computed transposed so that each lane
// holds 4 adjacent ranks of one token row and stores them at once; the row
// workgroups then read each 32-rank unit of t with one contiguous load. (The
// row order took 4 two-byte stores per lane and 16 row segments per load.)
template <int DT, int MT, int CH = 0, bool FX = false, bool TF = (DT != DT_F32), int NR>
__device__ __forceinline__ void latent_wg(const SlrArgs& a, int wg, f32x4 (&red)[NR]) {
  constexpr int KE = (DT == DT_F32) ? 4 : 8;
  using MM = Mma<DT, KE>;
  using Frag = typename MM::Frag;
  constexpr int KM = MM::KM;
  constexpr int UNR = MT == 1 ? 8 : (MT == 2 ? 4 : 2);

  const int lane = threadIdx.x & (kWave - 1);
  const int wid = wave_uniform(threadIdx.x >> 6);
  const int c = lane & 15, g = lane >> 4;
  const int per_mg = a.n_rt * a.n_kc;
  const int mg = wg / per_mg, rt = (wg % per_mg) / a.n_kc, kc = wg % a.n_kc;
  const int m0 = mg * MT * 16;
  const int Mrem = min(a.M - m0, MT * 16);
  const int64_t brow = (int64_t)(rt * 16 + c) * a.ldb;
  const int ub = kc * a.ku_chunk, ue = min(ub + a.ku_chunk, a.ku_total);

  constexpr int EB = Elem<DT>::bytes;
  f32x4 acc[MT][1];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt][0] = f32x4{0.f, 0.f, 0.f, 0.f};

  const auto xr = dev_rsrc(a.x);
  const auto xfr = dev_rsrc(a.xf);
  // FX: whole units of x from its fragment-order copy (chained stages of
  // 32- and 64-wide blocks, whose source writes one)
  static_assert(!FX || (CH == 2 && DT != DT_F32 && KE == 8), "fragment-order x: 16-bit chains");
  // x fragments of K unit u for every token row tile
  auto load_x = [&](int u, Frag(&xk)[MT]) {
    const int kcol = u * KM + KE * g;
    if (u * KM + KM <= a.m) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int64_t off = (int64_t)(m0 + min(mt * 16 + c, Mrem - 1)) * a.ldx + kcol;
        if constexpr (FX)
          xk[mt] = ld_dev_kfrag<DT, KE>(xfr, (((mg * MT + mt) * a.xf_units + u) << 10) + lane * 16,
                                        KE);
        else if constexpr (CH == 2) xk[mt] = ld_dev_kfrag<DT, KE>(xr, (int)(off * EB), KE);
        else xk[mt] = load_kfrag_full<DT, KE>(a.x, off);
      }
    } else {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int rr = mt * 16 + c;
        const int valid = (rr < Mrem) ? min(KE, a.m - kcol) : 0;
        const int64_t off = (int64_t)(m0 + rr) * a.ldx + kcol;
        if constexpr (CH == 2)
          xk[mt] = (valid > 0) ? ld_dev_kfrag<DT, KE>(xr, (int)(off * EB), valid)
                               : zero_frag<DT, KE>();
        else
          xk[mt] = (valid > 0) ? load_kfrag<DT, KE>(a.x, off, valid) : zero_frag<DT, KE>();
      }
    }
  };

  int u0 = ub + wid;
  if constexpr (CH == 2) {
    // B does not depend on x: the first batch's B loads go out before the wait.
    Frag xf[UNR][MT];
    Frag bf[UNR];
#pragma unroll
    for (int k = 0; k < UNR; ++k) {
      const int u = u0 + k * kSW;
      if (u < ue) bf[k] = load_kfrag_full<DT, KE>(a.B, brow + u * KM + KE * g);
    }
    wait_dep(a, mg);
#pragma unroll
    for (int k = 0; k < UNR; ++k)
      if (u0 + k * kSW < ue) load_x(u0 + k * kSW, xf[k]);
#pragma unroll
    for (int k = 0; k < UNR; ++k) {
      if (u0 + k * kSW < ue) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          if constexpr (TF) MM::run(acc[mt][0], bf[k], xf[k][mt]);
          else MM::run(acc[mt][0], xf[k][mt], bf[k]);
        }
      }
    }
    u0 += kSW * UNR;
  }
  for (; u0 < ue; u0 += kSW * UNR) {
    Frag xf[UNR][MT];
    Frag bf[UNR];
#pragma unroll
    for (int k = 0; k < UNR; ++k) {
      const int u = u0 + k * kSW;
      if (u < ue) {
        load_x(u, xf[k]);
        bf[k] = load_kfrag_full<DT, KE>(a.B, brow + u * KM + KE * g);
      }
    }
#pragma unroll
    for (int k = 0; k < UNR; ++k) {
      if (u0 + k * kSW < ue) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          if constexpr (TF) MM::run(acc[mt][0], bf[k], xf[k][mt]);
          else MM::run(acc[mt][0], xf[k][mt], bf[k]);
        }
      }
    }
  }

  tree_reduce<MT, 1>(acc, red, wid, lane);
  if (wid != 0) return;
  // wave 0: lane (c, g) holds rows 16·mt + 4g + e of rank rt·16 + c.
  u64* sy = tile_sync(a, mg);
  if (a.n_kc > 1) {
    // Publish this K chunk's fp32 partial; the last chunk of the rank tile to
    // arrive sums all of them in chunk order (deterministic) and goes on.
    const auto pr = dev_rsrc(a.t_part);
    const int64_t slab = (int64_t)a.MG * a.n_rt * (MT * 256);  // floats per K chunk
    const int64_t tile = ((int64_t)mg * a.n_rt + rt) * (MT * 256);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      float v[4] = {acc[mt][0][0], acc[mt][0][1], acc[mt][0][2], acc[mt][0][3]};
      st_dev_vec<4>(pr, (int)((kc * slab + tile + (mt * 64 + lane) * 4) * 4), v);
    }
    wait_mem();
    int last = 0;
    if (lane == 0) {
      const u64 old = rmw_add64(sy + 2 + rt, (u64)a.lat_weight);
      last = (old + (u64)a.lat_weight) % kLatentUnits == 0;
    }
    if (!__builtin_amdgcn_readfirstlane(last)) return;
    f32x4 tot[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) tot[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < a.n_kc; ++k) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if (k == kc) {
          tot[mt] += acc[mt][0];
        } else {
          float v[4];
          ld_dev_vec<4>(pr, (int)((k * slab + tile + (mt * 64 + lane) * 4) * 4), v);
          tot[mt] += f32x4{v[0], v[1], v[2], v[3]};
        }
      }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt][0] = tot[mt];
  }
  // Final latent tile, rounded once to the activation dtype as F.linear's
  // output is. Rows past M hold finite values no output uses (their x rows
  // were read as copies of the last row, or as zeros past in_features).
  const auto tr = dev_rsrc(a.t);
  if constexpr (TF) {
    static_assert(DT != DT_F32, "fragment-order t: 16-bit");
    // lane (c, g): ranks rt·16 + 4g .. + 3 of token row 16·mt + c: 8 bytes of
    // unit rt / 2, 8-rank group 2·(rt % 2) + g / 2, half g % 2
    const int units = (int)(a.ldt >> 5);
    typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const u32x2v w = {to_bits<DT>(acc[mt][0][0]) | (to_bits<DT>(acc[mt][0][1]) << 16),
                        to_bits<DT>(acc[mt][0][2]) | (to_bits<DT>(acc[mt][0][3]) << 16)};
      const int off = (((mg * MT + mt) * units + (rt >> 1)) << 10) +
                      (16 * (2 * (rt & 1) + (g >> 1)) + c) * 16 + (g & 1) * 8;
      __builtin_amdgcn_raw_buffer_store_b64(w, tr, off, 0, kSc1);
    }
    wait_mem();
    if (lane == 0) rmw_add64(fin_copy(a, mg, rt % kFinCopies), 1);
    return;
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int off = (int)(((int64_t)(m0 + mt * 16 + 4 * g + e) * a.ldt + rt * 16 + c) * EB);
      if constexpr (DT == DT_F32) {
        float v = acc[mt][0][e];
        st_dev_vec<1>(tr, off, &v);
      } else {
        __builtin_amdgcn_raw_buffer_store_b16((unsigned short)to_bits<DT>(acc[mt][0][e]), tr, off,
                                              0, kSc1);
      }
    }
  wait_mem();
  if (lane == 0) rmw_add64(fin_copy(a, mg, rt % kFinCopies), 1);
}

// ---------------------------------------------------------------------------
// Streaming workgroup: one plan chunk for one token tile.
// ---------------------------------------------------------------------------
// SF: storage of the sparse blocks, SF_BSR (q, p) blocks or SF_NM24 packed 2:4 blocks.
// P: output features per block-row (the tile width; W = P / 16 MFMA column tiles).
// KE: k elements per lane of the sparse MFMA fragments (8 when q is a multiple
// of 32 for 16-bit activations, else 4), so one K slab is KM = 4·KE block rows
// and q (any multiple of KM) is a runtime value.
// CH: as for latent_wg (chained launches; 2 = x written by an earlier stage:
// the first batch's weight loads go out before the wait for x).
template <int DT, int P, int KE, int MT, int MODE, int UNR, int SF, int CH = 0, bool FR = false,
          int NR>
__device__ __forceinline__ void stream_wg(const SlrArgs& a, int chunk, int mg, f32x4 (&red)[NR]) {
  constexpr int W = P / 16;
  using MM = Mma<DT, KE>;
  using Frag = typename MM::Frag;
  constexpr int KM = MM::KM;
  static_assert(DT != DT_F32 || KE == 4, "fp32 fragments hold 4 k");
  static_assert(SF == SF_BSR || (P == kNmBlock && DT != DT_F32 && KE == 8),
                "2:4 blocks are 32×32, 16-bit");
  using Raw = typename std::conditional<SF == SF_NM24, NmRaw, VRawT<DT, KE, W>>::type;
  constexpr int KEL = (DT == DT_F32) ? 4 : 8;  // low-rank part: widest fragment
  using ML = Mma<DT, KEL>;
  using FragL = typename ML::Frag;
  constexpr int NLS = 32 / ML::KM;  // macro steps per 32-rank unit
  constexpr int EB = Elem<DT>::bytes;
  constexpr int TSZ = MT * 16 * P;

  const int lane = threadIdx.x & (kWave - 1);
  const int wid = wave_uniform(threadIdx.x >> 6);
  const int c = lane & 15, g = lane >> 4;
  const int32_t* d = a.plan + (int64_t)chunk * SSL_PLAN_STRIDE;
  const int row = d[0], bb = d[1], be = d[2], lb = d[3], le = d[4], seq = d[5], nseq = d[6];
  const int slot = d[7];
#if SSL_DEVICE_CHECKS
  if (!(row >= 0 && row < a.NB && bb >= 0 && bb <= be && (a.nnz <= 0 || be <= a.nnz) &&
        lb >= 0 && lb <= le && (int64_t)le * 32 <= a.lda && nseq >= 1 && seq >= 0 && seq < nseq &&
        (nseq == 1 || (slot >= 0 && slot + nseq <= a.n_slots)))) {
    if (threadIdx.x == 0) check_fail(a.status, kChkPlan);
    return;  // the whole workgroup: the entry is uniform
  }
#endif
  const int m0 = mg * MT * 16;
  const int Mrem = min(a.M - m0, MT * 16);

  f32x4 acc[MT][W];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int s = 0; s < W; ++s) acc[mt][s] = f32x4{0.f, 0.f, 0.f, 0.f};

  const bool used_t = (MODE == MODE_FUSED) && lb < le;
  // A consumer of the latent takes a ticket at once (its latency hides behind
  // the row's loads). Launch k's n consumers of a ticket copy hold its tickets
  // k·n ... and wait for (k + 1)·n_rt final tiles, so no counter is ever reset.
  u64 ticket = 0;
  const bool per_row = a.tk_copies > 1;
  const int tc = per_row ? row % kFinCopies : 0;
  if (used_t && threadIdx.x == 0) ticket = rmw_add64(fin_copy(a, mg, tc) + kFinTicket, 1);

  // The wave's first low-rank unit of A does not depend on the latent: its
  // loads go out ahead of the sparse blocks.
  FragL af0[NLS][W];
  if constexpr (MODE == MODE_FUSED) {
    if (used_t && lb + wid < le) {
#pragma unroll
      for (int ls = 0; ls < NLS; ++ls)
#pragma unroll
        for (int s = 0; s < W; ++s)
          af0[ls][s] = load_kfrag<DT, KEL>(
              a.A, (int64_t)(row * P + W * c + s) * a.lda + (lb + wid) * 32 + ls * ML::KM + KEL * g,
              KEL);
    }
  }

  // ---- sparse blocks, as K slabs: the chunk's slabs [bb·nks, be·nks) go to
  // the waves round-robin; a batch issues all its loads (x, then the slab)
  // slab by slab before the first MFMA, so each slab waits only for its own data.
  const int nks = a.nks;
  const int vb = bb * nks, ve = be * nks;
  const auto xr = dev_rsrc(a.x);
  const auto xfr = dev_rsrc(a.xf);
  // whole units of x from the fragment-order copy its source writes (chained
  // stages, 16-bit, 32- and 64-wide blocks: KE = 8, KM = 32 and every slab's
  // column is a multiple of 32)
  constexpr bool kFragIn = FR && CH == 2 && DT != DT_F32 && (P == 32 || P == 64);
  static_assert(!kFragIn || KE == 8, "fragment-order x: 32-column units");
  // Chained 16-bit members with 32- or 64-wide tiles in the kernels that pass
  // fragment-order inputs (FR) compute the transposed tile (features × tokens:
  // the weights as the MFMA's first operand), so that lane (c, g) ends with 4W
  // adjacent features, W·4g .. W·4g + 4W − 1, of token row 16·mt + c, element
  // (s, e) being feature W·(4g + e) + s: its output row segment is one vector
  // store, and for W = 2 it is exactly the lane's 16 bytes of the
  // fragment-order copy (for W = 4, two of them). (At one token row, where
  // FR kernels are not used, the transposed tile measured 4% slower.)
  constexpr bool kSwap = FR && CH > 0 && MODE == MODE_FUSED && DT != DT_F32 && (P == 32 || P == 64);
  // t in fragment order (latent_wg's TF) for 16-bit activations
  constexpr bool kTFrag = MODE == MODE_FUSED && DT != DT_F32;
  static_assert(!kTFrag || NLS == 1, "fragment-order t: one fragment per 32-rank unit");
  // the batch's column indices first, as scalar loads issued together
  auto index = [&](int v0, int(&colk)[UNR], int64_t(&voff)[UNR]) {
#pragma unroll
    for (int k = 0; k < UNR; ++k) {
      const int v = min(v0 + k * kSW, ve - 1);
      const int blk = nks == 1 ? v : (int)__umulhi((uint32_t)v, a.nks_magic);
      const int ks = v - blk * nks;
#if SSL_DEVICE_CHECKS
      // The fused linear reads x through masks at in_features, so a block past
      // it reads zeros (the padding of a ragged last block, or the all-padding
      // sub-blocks cut from a deep one): there a column must only be
      // non-negative with an offset in range. The op's x is exactly its
      // block-columns wide.
      int cb = ld_uniform(a.col, blk);
      if (cb < 0 || (MODE == MODE_OP ? (int64_t)cb * a.q >= a.m : (int64_t)cb * a.q > 0x3fffffff)) {
        if (lane == 0) check_fail(a.status, kChkColumn);
        cb = 0;
      }
      colk[k] = cb * a.q + ks * KM;
#else
      colk[k] = ld_uniform(a.col, blk) * a.q + ks * KM;
#endif
      voff[k] = (int64_t)blk * a.blk_bytes + ks * a.slab_bytes;
    }
  };
  // x fragments of the slab at input column colk for every token row tile
  auto load_x = [&](int colk, Frag(&xk)[MT]) {
    const int kcol = colk + KE * g;
    const bool full = colk + KM <= a.m;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int rr = mt * 16 + c;
      if (full) {
        const int64_t off = (int64_t)(m0 + min(rr, Mrem - 1)) * a.ldx + kcol;
        if constexpr (kFragIn)
          xk[mt] = ld_dev_kfrag<DT, KE>(
              xfr, (((mg * MT + mt) * a.xf_units + (colk >> 5)) << 10) + lane * 16, KE);
        else if constexpr (CH == 2) xk[mt] = ld_dev_kfrag<DT, KE>(xr, (int)(off * EB), KE);
        else xk[mt] = load_kfrag_full<DT, KE>(a.x, off);
      } else {
        const int valid = (rr < Mrem) ? min(KE, a.m - kcol) : 0;
        const int64_t off = (int64_t)(m0 + rr) * a.ldx + kcol;
        if constexpr (CH == 2)
          xk[mt] = (valid > 0) ? ld_dev_kfrag<DT, KE>(xr, (int)(off * EB), valid)
                               : zero_frag<DT, KE>();
        else
          xk[mt] = (valid > 0) ? load_kfrag<DT, KE>(a.x, off, valid) : zero_frag<DT, KE>();
      }
    }
  };
  auto load_w = [&](int64_t voff, Raw& rk) {
    const char* vb_ = (const char*)a.values + voff;
    if constexpr (SF == SF_NM24) load_nm(rk, vb_, lane);
    else load_vstep<DT, KE, W>(rk, vb_, P, 0, lane);
  };
  auto mma = [&](const Raw& rk, const Frag(&xk)[MT]) {
#pragma unroll
    for (int s = 0; s < W; ++s) {
      Frag vf;
      if constexpr (SF == SF_NM24) vf = nm_frag<DT>(rk, s);
      else vf = vfrag<DT, KE, W>(rk, s);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if constexpr (kSwap) MM::run(acc[mt][s], vf, xk[mt]);
        else MM::run(acc[mt][s], xk[mt], vf);
      }
    }
  };

  int v0 = vb + wid;
  if constexpr (CH == 2) {
    // The weights do not depend on x: the first batch's block loads go out
    // before the wait for the stage's input.
    Raw raw[UNR];
    Frag xf[UNR][MT];
    int colk[UNR];
    int64_t voff[UNR];
    if (v0 < ve) index(v0, colk, voff);
#pragma unroll
    for (int k = 0; k < UNR; ++k)
      if (v0 + k * kSW < ve) load_w(voff[k], raw[k]);
    wait_dep(a, mg);
#pragma unroll
    for (int k = 0; k < UNR; ++k)
      if (v0 + k * kSW < ve) load_x(colk[k], xf[k]);
#pragma unroll
    for (int k = 0; k < UNR; ++k)
      if (v0 + k * kSW < ve) mma(raw[k], xf[k]);
    v0 += kSW * UNR;
  }
  for (; v0 < ve; v0 += kSW * UNR) {
    Raw raw[UNR];
    Frag xf[UNR][MT];
    int colk[UNR];
    int64_t voff[UNR];
    index(v0, colk, voff);
#pragma unroll
    for (int k = 0; k < UNR; ++k) {
      if (v0 + k * kSW < ve) {
        load_x(colk[k], xf[k]);
        load_w(voff[k], raw[k]);
      }
    }
#pragma unroll
    for (int k = 0; k < UNR; ++k)
      if (v0 + k * kSW < ve) mma(raw[k], xf[k]);
  }

  // ---- low-rank units: 32 ranks of A per unit, t·Aᵀ. One thread of the
  // workgroup waits for this launch's final latent; the barrier releases the
  // other waves, which then read it device-coherently.
  if constexpr (MODE == MODE_FUSED) {
    if (used_t) {
      if (threadIdx.x < kWave) {
        // the ticket's launch: this copy's consumers per launch
        const int n_tc = per_row ? fin_share(a.NB, tc) : a.lr_wgs;
        const u64 tk = ((u64)__builtin_amdgcn_readfirstlane((uint32_t)(ticket >> 32)) << 32) |
                       (u64)__builtin_amdgcn_readfirstlane((uint32_t)ticket);
        wait_fin(a, mg, tk / (u64)n_tc);
      }
      __syncthreads();
      const auto tr = dev_rsrc(a.t);
      for (int u = lb + wid; u < le; u += kSW) {
        FragL af[NLS][W];
        FragL tf[NLS][MT];
#pragma unroll
        for (int ls = 0; ls < NLS; ++ls) {
          const int kr = u * 32 + ls * ML::KM + KEL * g;
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            if constexpr (kTFrag)
              tf[ls][mt] = ld_dev_frag<DT, KEL>(
                  tr, (((mg * MT + mt) * (int)(a.ldt >> 5) + u) << 10) + lane * 16);
            else
              tf[ls][mt] = ld_dev_frag<DT, KEL>(
                  tr, (int)(((int64_t)(m0 + mt * 16 + c) * a.ldt + kr) * EB));
          }
#pragma unroll
          for (int s = 0; s < W; ++s)
            af[ls][s] = (u == lb + wid)
                            ? af0[ls][s]
                            : load_kfrag<DT, KEL>(a.A, (int64_t)(row * P + W * c + s) * a.lda + kr,
                                                  KEL);
        }
#pragma unroll
        for (int ls = 0; ls < NLS; ++ls)
#pragma unroll
          for (int s = 0; s < W; ++s)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              if constexpr (kSwap) ML::run(acc[mt][s], af[ls][s], tf[ls][mt]);
              else ML::run(acc[mt][s], tf[ls][mt], af[ls][s]);
            }
      }
    }
  }

  tree_reduce<MT, W>(acc, red, wid, lane);
  if (wid != 0) return;

  // ---- wave 0: combine (split rows) and epilogue ---------------------------
  if (nseq > 1) {
    float* part_base = a.part_main + ((int64_t)mg * a.n_slots + slot) * TSZ;
    int* counter = a.cnt_main + (int64_t)mg * a.NB + row;
    const bool finaliser_mode = (MODE == MODE_FUSED) && a.n_rt > 0;
    if (finaliser_mode && used_t) {
      // the row's finaliser: wait for the other nseq - 1 chunks
      if (lane == 0) wait_at_least<int>(counter, nseq - 1 + a.wait_bias, a.status, a.wait_polls);
    } else {
      if constexpr (kSwap) store_partial_lanes<MT, W>(acc, part_base + (int64_t)seq * TSZ, lane);
      else store_partial<MT, W>(acc, part_base + (int64_t)seq * TSZ, Mrem, lane);
      wait_mem();
      int old = 0;
      if (lane == 0) old = rmw_add(counter, 1);
      old = __builtin_amdgcn_readfirstlane(old);
      if (finaliser_mode || old != nseq - 1) return;
    }
    // This chunk combines the row (the finaliser, or the op's last arrival).
    // sum the partials in chunk order, this chunk's tile at its own position
    f32x4 tot[MT][W];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int s = 0; s < W; ++s) tot[mt][s] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < nseq; ++k) {
      if (k == seq) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int s = 0; s < W; ++s) tot[mt][s] += acc[mt][s];
      } else {
        if constexpr (kSwap) add_partial_lanes<MT, W>(tot, part_base + (int64_t)k * TSZ, lane);
        else add_partial<MT, W>(tot, part_base + (int64_t)k * TSZ, Mrem, lane);
      }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int s = 0; s < W; ++s) acc[mt][s] = tot[mt][s];
    // Return the row counter to zero by subtracting the arrivals this launch
    // makes (nseq - 1 other chunks for the finaliser; all nseq in the op)
    // rather than storing 0: if a finaliser's wait gave up, the chunks still to
    // arrive bring the counter back to exactly zero by the launch's end.
    if (lane == 0) rmw_add(counter, finaliser_mode ? -(nseq - 1) : -nseq);
  }

  // epilogue: lane (c, g) owns W adjacent output columns of rows 16·mt + 4g + e
  const int j0 = row * P + W * c;
  float bv[W];
#pragma unroll
  for (int s = 0; s < W; ++s) bv[s] = 0.f;
  if constexpr (MODE == MODE_FUSED && !kSwap) {
    if (a.bias != nullptr) ld_w<DT, W>(a.bias, j0, bv);
  }
  // a chained member another stage reads stores device-coherently
  const bool dev_out = CH > 0 && a.done != nullptr;
  const auto yr = dev_rsrc(a.y);
  if constexpr (kSwap) {
    // transposed tile: lane (c, g) holds 4W adjacent features of token row
    // 16·mt + c (see kSwap). Its row segment goes out as 16-byte stores, and
    // a member another stage reads also writes it to the fragment-order copy
    // (every token row of the tile, those past M included: finite, computed
    // from copies of the last row), so the reader loads whole units.
    constexpr int NF = 4 * W;  // features per lane
    const int f0 = row * P + NF * g;
    float bw[NF];
#pragma unroll
    for (int i = 0; i < NF; ++i) bw[i] = 0.f;
    if (a.bias != nullptr) ld_w<DT, NF>(a.bias, f0, bw);
    const bool frag_out = dev_out && a.yf != nullptr;
    const auto fr = dev_rsrc(a.yf);
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int rr = mt * 16 + c;
      uint32_t w[NF / 2];
#pragma unroll
      for (int i = 0; i < NF / 2; ++i) {
        // features 2i and 2i + 1 of the lane: (s, e) = ((2i) % W, (2i) / W), ...
        const int f_lo = 2 * i, f_hi = 2 * i + 1;
        const float lo = acc[mt][f_lo % W][f_lo / W] + bw[f_lo];
        const float hi = acc[mt][f_hi % W][f_hi / W] + bw[f_hi];
        w[i] = to_bits<DT>(lo) | (to_bits<DT>(hi) << 16);
      }
#pragma unroll
      for (int q = 0; q < NF / 8; ++q) {
        const u32x4v v = {w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3]};
        if (rr < Mrem) {
          const int64_t off = ((int64_t)(m0 + rr) * a.ldy + f0 + 8 * q) * EB;
          if (dev_out) __builtin_amdgcn_raw_buffer_store_b128(v, yr, (int)off, 0, kSc1);
          else *reinterpret_cast<u32x4v*>((char*)a.y + off) = v;
        }
        if (frag_out) {
          // unit (row·P + NF·g + 8q) / 32 of the output, 8-column group
          // ((NF·g + 8q) % 32) / 8 of it
          const int col = NF * g + 8 * q;
          const int unit = row * (P / 32) + col / 32, gg = (col % 32) / 8;
          __builtin_amdgcn_raw_buffer_store_b128(
              v, fr, (((mg * MT + mt) * a.yf_units + unit) << 10) + (16 * gg + c) * 16, 0, kSc1);
        }
      }
    }
  } else {
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int rr = mt * 16 + 4 * g + e;
      if (rr < Mrem) {
        const int64_t off = (int64_t)(m0 + rr) * a.ldy + j0;
        float o[W];
        if constexpr (MODE == MODE_FUSED) {
#pragma unroll
          for (int s = 0; s < W; ++s) o[s] = acc[mt][s][e] + bv[s];
        } else {
          ld_w<DT, W>(a.y, off, o);
#pragma unroll
          for (int s = 0; s < W; ++s) o[s] += acc[mt][s][e];
        }
        if (CH > 0 && dev_out) st_w_dev<DT, W>(yr, (int)(off * EB), o);
        else st_w<DT, W>(a.y, off, o);
      }
    }
  }
  if constexpr (CH > 0) {
    // count this row tile as finished once its stores are acknowledged
    if (dev_out) {
      wait_mem();
      if (lane == 0) rmw_add(a.done + ((int64_t)mg * kDepCopies + row % kDepCopies) * kDepSlotInts, 1);
    }
  }
}

// ---------------------------------------------------------------------------
// Kernel. Grid (1-D): [latent workgroups][stream chunks × token tiles].
// ---------------------------------------------------------------------------
// A launch serves up to kMaxGroup linears that read the same x (e.g. the q, k
// and v projections): all latent workgroups first, member by member, then all
// row workgroups, member by member. Workgroup → member lookups read the
// descriptors in place from the kernel-argument segment (scalar loads).
constexpr int kMaxGroup = 4;
struct GroupArgs {
  int n;                          // members
  int lat_total;                  // latent workgroups of all members
  int lat_off[kMaxGroup + 1];     // first latent workgroup of each member
  int str_off[kMaxGroup + 1];     // first row workgroup (after lat_total) of each member
  SlrArgs m[kMaxGroup];
};

template <int DT, int P, int KE, int MT, int MODE, int UNR, int SF>
__global__ __launch_bounds__(kST, (DT != DT_F32 && P <= 32) ? 4 : 2) void slr_kernel(
    GroupArgs g_by_value) {
  (void)g_by_value;
  const GroupArgs& g = *(const GroupArgs*)__builtin_amdgcn_kernarg_segment_ptr();
  constexpr int W = P / 16;
  __shared__ f32x4 red[red_len<MT, W>()];
  const int b = blockIdx.x;
  // the member of workgroup b: every member's offsets in one batch of scalar
  // loads and a chain of selects (no dependent loads before the work starts)
  if constexpr (MODE == MODE_FUSED) {
    if (b < g.lat_total) {
      int i = 0, off = g.lat_off[0];
#pragma unroll
      for (int k = 1; k < kMaxGroup; ++k) {
        const bool in = k < g.n && b >= g.lat_off[k];
        i = in ? k : i;
        off = in ? g.lat_off[k] : off;
      }
      latent_wg<DT, MT>(g.m[i], b - off, red);
      return;
    }
  }
  const int sb = b - (MODE == MODE_FUSED ? g.lat_total : 0);
  int i = 0, off = g.str_off[0];
#pragma unroll
  for (int k = 1; k < kMaxGroup; ++k) {
    const bool in = k < g.n && sb >= g.str_off[k];
    i = in ? k : i;
    off = in ? g.str_off[k] : off;
  }
  const SlrArgs& a = g.m[i];
  const int lb = sb - off;
  const int mg = lb / a.n_chunks, chunk = lb % a.n_chunks;
  stream_wg<DT, P, KE, MT, MODE, UNR, SF>(a, chunk, mg, red);
}

// ---------------------------------------------------------------------------
// Chained launch: the linears of several dependent stages (e.g. a decoder
// layer's q,k,v -> o -> gate,up -> down projections) in ONE launch. The grid is
// the stages in order, each [latent workgroups][row workgroups] of its members
// as in slr_kernel. A stage after the first reads the output of a member of an
// earlier stage: its workgroups issue their first weight loads, then wait for
// that member's row tiles of their token tile (SlrArgs::dep), then read x
// device-coherently. Every wait is on workgroups earlier in the grid, which an
// XCD dispatches first, so every wait ends; the weight streams of a stage
// overlap the tail of the stage before it, and the launch pays one kernel
// boundary instead of one per stage.
// ---------------------------------------------------------------------------
constexpr int kMaxChain = 8;       // members of a chained launch described in its kernel arguments
constexpr int kMaxChainTab = 256;  // members of one described by a table in device memory
template <int NMAX>
struct ChainDesc {
  // the launch it describes (read by the host when launching from a table)
  int64_t grid;                 // workgroups
  int M, block_p, dtype, sf;    // token rows, kernel block width, SSL dtype, SF_*
  int fr;                       // later stages read fragment-order copies (FR kernels)
  int n_seg;                    // grid segments, in grid order
  int seg_start[2 * NMAX + 1];  // first workgroup of each segment, then the grid size
  int seg_member[2 * NMAX];     // the member a segment belongs to
  int seg_rows[2 * NMAX];       // 1: its row workgroups, 0: its latent workgroups
  SlrArgs m[NMAX];
};
using ChainArgs = ChainDesc<kMaxChain>;
using ChainTab = ChainDesc<kMaxChainTab>;
static_assert(sizeof(ChainArgs) <= 4096, "kernel arguments of a chained launch");

template <int DT, int P, int KE, int MT, int UNR, int SF, bool FR, int NMAX, int NR>
__device__ __forceinline__ void chain_wg(const ChainDesc<NMAX>& g, f32x4 (&red)[NR]) {
  constexpr bool kFrag = FR && DT != DT_F32 && (P == 32 || P == 64);
  const int b = blockIdx.x;
  // the last segment starting at or before b (empty segments share a start)
  int member, rows, start;
  if constexpr (2 * NMAX <= 16) {
    // Kernel arguments: every segment's words in one batch of scalar loads and
    // a chain of selects. A binary search's dependent loads, each a round trip
    // to L2 on a cold scalar cache, put a workgroup's first work 1.0-1.6 µs
    // after its first instruction.
    member = g.seg_member[0];
    rows = g.seg_rows[0];
    start = g.seg_start[0];
#pragma unroll
    for (int i = 1; i < 2 * NMAX; ++i) {
      const bool in = i < g.n_seg && b >= g.seg_start[i];
      member = in ? g.seg_member[i] : member;
      rows = in ? g.seg_rows[i] : rows;
      start = in ? g.seg_start[i] : start;
    }
  } else {
    int lo = 0, hi = g.n_seg - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (b >= g.seg_start[mid]) lo = mid;
      else hi = mid - 1;
    }
    member = g.seg_member[lo];
    rows = g.seg_rows[lo];
    start = g.seg_start[lo];
  }
  const SlrArgs& a = g.m[member];
  const int lb = b - start;
  if (!rows) {
    if (a.dep) {
      latent_wg<DT, MT, 2, kFrag>(a, lb, red);
      const int per_mg = a.n_rt * a.n_kc;
      if (threadIdx.x < kWave) dep_close(a, lb / per_mg, a.dep_lat_base + lb % per_mg);
    } else {
      latent_wg<DT, MT, 1>(a, lb, red);
    }
    return;
  }
  const int mg = lb / a.n_chunks, chunk = lb % a.n_chunks;
  if (a.dep) {
    stream_wg<DT, P, KE, MT, MODE_FUSED, UNR, SF, 2, FR>(a, chunk, mg, red);
    if (threadIdx.x < kWave) dep_close(a, mg, a.dep_row_base + chunk);
  } else {
    stream_wg<DT, P, KE, MT, MODE_FUSED, UNR, SF, 1, FR>(a, chunk, mg, red);
  }
}

template <int DT, int P, int KE, int MT, int UNR, int SF, bool FR>
__global__ __launch_bounds__(kST, (DT != DT_F32 && P <= 32) ? 4 : 2) void slr_chain_kernel(
    ChainArgs c_by_value) {
  (void)c_by_value;
  constexpr int W = P / 16;
  __shared__ f32x4 red[red_len<MT, W>()];
  chain_wg<DT, P, KE, MT, UNR, SF, FR, kMaxChain>(
      *(const ChainArgs*)__builtin_amdgcn_kernarg_segment_ptr(), red);
}

// The same with the descriptor in device memory (many stages, e.g. every
// layer of a model in one launch). Read through the constant address space,
// as kernel arguments are: scalar loads of uniform words.
typedef const __attribute__((address_space(4))) ChainTab* ChainTabPtr;
template <int DT, int P, int KE, int MT, int UNR, int SF, bool FR>
__global__ __launch_bounds__(kST, (DT != DT_F32 && P <= 32) ? 4 : 2) void slr_chain_tab_kernel(
    ChainTabPtr tab) {
  constexpr int W = P / 16;
  __shared__ f32x4 red[red_len<MT, W>()];
  chain_wg<DT, P, KE, MT, UNR, SF, FR, kMaxChainTab>(*(const ChainTab*)tab, red);
}

// Slabs per wave per batch. The byte budget of the square-block kernels
// (a 32-block row in one batch of the 8 waves for 32×32 and 64×64 blocks,
// fewer units for wide tiles; 16-bit kernels with P ≤ 32 stay within 128 VGPRs,
// so two workgroups share a compute unit), expressed in slabs of KM = 4·KE rows.
template <int DT, int P, int KE, int MT>
constexpr int stream_unroll() {
  constexpr int KM = 4 * KE;
  constexpr int bytes = P * P * Elem<DT>::bytes;
  constexpr int u = bytes >= 16384 ? 2 : (bytes >= 2048 ? 4 : 16);
  constexpr int d = MT >= 4 ? 4 : MT;
  constexpr int blocks = u / d > 0 ? u / d : 1;
  constexpr int slabs = blocks * P / KM;
  return slabs > 0 ? slabs : 1;
}

// One launch of slr_kernel (grid: `blocks` workgroups of kST threads) for a
// dtype; defined in stream_{bf16,f16,f32}.hip. P ∈ {16, 32, 48, 64}; KE 4 or
// 8 (4 for fp32); MT ∈ {1, 2, 4}; SF_NM24 only with P = 32, KE = 8, MODE_FUSED.
template <int DT>
hipError_t stream_launch(int mode, int sf, int P, int KE, int MT, const GroupArgs& a,
                         int64_t blocks, hipStream_t s);

template <int DT, int P, int KE, int MT, int MODE, int SF>
hipError_t stream_launch_one(const GroupArgs& a, int64_t blocks, hipStream_t s) {
  constexpr int UNR = stream_unroll<DT, P, KE, MT>();
  hipLaunchKernelGGL((slr_kernel<DT, P, KE, MT, MODE, UNR, SF>), dim3((unsigned)blocks), dim3(kST),
                     0, s, a);
  return hipGetLastError();
}

// One chained launch for a 16-bit dtype; defined in stream_{bf16,f16}.hip.
// Square blocks of 16, 32 or 64 (KE 4, 8, 8) or 2:4 blocks; MT ∈ {1, 2, 4}.
// `a` is the descriptor in kernel arguments, or else `tab` one in device memory.
template <int DT>
hipError_t chain_launch(int sf, int P, int MT, bool fr, const ChainArgs* a, const ChainTab* tab,
                        int64_t blocks, hipStream_t s);

template <int DT, int P, int KE, int MT, int SF, bool FR>
hipError_t chain_launch_one(const ChainArgs* a, const ChainTab* tab, int64_t blocks,
                            hipStream_t s) {
  constexpr int UNR = stream_unroll<DT, P, KE, MT>();
  if (a)
    hipLaunchKernelGGL((slr_chain_kernel<DT, P, KE, MT, UNR, SF, FR>), dim3((unsigned)blocks),
                       dim3(kST), 0, s, *a);
  else
    hipLaunchKernelGGL((slr_chain_tab_kernel<DT, P, KE, MT, UNR, SF, FR>), dim3((unsigned)blocks),
                       dim3(kST), 0, s, (ChainTabPtr)tab);
  return hipGetLastError();
}

// fr: the stages after the first read their input from its fragment-order
// copy (32- and 64-wide blocks). One-tile calls have both kernels; taller
// ones (MT > 1) always read fragments, and 16-wide blocks never do.
template <int DT>
hipError_t chain_dispatch(int sf, int P, int MT, bool fr, const ChainArgs* a, const ChainTab* tab,
                          int64_t blocks, hipStream_t s) {
  static_assert(DT != DT_F32, "chained launches take 16-bit activations");
#define SSL_CMT(PP, KK, SS)                                                               \
  switch (MT) {                                                                           \
    case 1:                                                                               \
      return fr ? chain_launch_one<DT, PP, KK, 1, SS, true>(a, tab, blocks, s)            \
                : chain_launch_one<DT, PP, KK, 1, SS, false>(a, tab, blocks, s);          \
    case 2: if (fr) return chain_launch_one<DT, PP, KK, 2, SS, true>(a, tab, blocks, s); \
      break;                                                                              \
    case 4: if (fr) return chain_launch_one<DT, PP, KK, 4, SS, true>(a, tab, blocks, s); \
      break;                                                                              \
  }                                                                                       \
  return hipErrorInvalidValue;
  if (sf == SF_NM24) {
    if (P != kNmBlock) return hipErrorInvalidValue;
    SSL_CMT(kNmBlock, 8, SF_NM24)
  }
  if (sf != SF_BSR) return hipErrorInvalidValue;
  switch (P) {
    case 16:
      if (fr) return hipErrorInvalidValue;
      switch (MT) {
        case 1: return chain_launch_one<DT, 16, 4, 1, SF_BSR, false>(a, tab, blocks, s);
        case 2: return chain_launch_one<DT, 16, 4, 2, SF_BSR, false>(a, tab, blocks, s);
        case 4: return chain_launch_one<DT, 16, 4, 4, SF_BSR, false>(a, tab, blocks, s);
      }
      return hipErrorInvalidValue;
    case 32: { SSL_CMT(32, 8, SF_BSR) }
    case 64: { SSL_CMT(64, 8, SF_BSR) }
  }
  return hipErrorInvalidValue;
#undef SSL_CMT
}

// The instantiation table of one dtype (expanded in its own file).
template <int DT>
hipError_t stream_dispatch(int mode, int sf, int P, int KE, int MT, const GroupArgs& a,
                           int64_t blocks, hipStream_t s) {
  if constexpr (DT != DT_F32) {
    if (sf == SF_NM24) {
      if (P != kNmBlock || KE != 8 || mode != MODE_FUSED) return hipErrorInvalidValue;
      switch (MT) {
        case 1: return stream_launch_one<DT, kNmBlock, 8, 1, MODE_FUSED, SF_NM24>(a, blocks, s);
        case 2: return stream_launch_one<DT, kNmBlock, 8, 2, MODE_FUSED, SF_NM24>(a, blocks, s);
        case 4: return stream_launch_one<DT, kNmBlock, 8, 4, MODE_FUSED, SF_NM24>(a, blocks, s);
      }
      return hipErrorInvalidValue;
    }
  }
  if (sf != SF_BSR) return hipErrorInvalidValue;
#define SSL_MT(PP, KK, MD)                                                     \
  switch (MT) {                                                                \
    case 1: return stream_launch_one<DT, PP, KK, 1, MD, SF_BSR>(a, blocks, s); \
    case 2: return stream_launch_one<DT, PP, KK, 2, MD, SF_BSR>(a, blocks, s); \
    case 4: return stream_launch_one<DT, PP, KK, 4, MD, SF_BSR>(a, blocks, s); \
  }                                                                            \
  return hipErrorInvalidValue;
#define SSL_KE(PP, MD)                           \
  if (KE == 4) { SSL_MT(PP, 4, MD) }             \
  if constexpr (DT != DT_F32) {                  \
    if (KE == 8) { SSL_MT(PP, 8, MD) }           \
  }                                              \
  return hipErrorInvalidValue;
#define SSL_P(MD)                        \
  switch (P) {                           \
    case 16: { SSL_KE(16, MD) }          \
    case 32: { SSL_KE(32, MD) }          \
    case 48: { SSL_KE(48, MD) }          \
    case 64: { SSL_KE(64, MD) }          \
  }                                      \
  return hipErrorInvalidValue;
  if (mode == MODE_FUSED) {
    SSL_P(MODE_FUSED)
  }
  SSL_P(MODE_OP)
#undef SSL_P
#undef SSL_KE
#undef SSL_MT
}

}  // namespace ssl

