// Streaming SLR / BSR kernels for gfx950.
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
#include "prefill.h"
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
// N = 1, 2 or 4 floats at a wave-uniform base plus a per-lane byte offset below
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
  } else {
    static_assert(N == 1, "1, 2 or 4 floats");
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
  } else {
    static_assert(N == 1, "1, 2 or 4 floats");
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
template <typename T>
__device__ __forceinline__ void wait_at_least(const T* flag, T target, u64* status, int polls) {
  int n = 0;
  while (__hip_atomic_load(const_cast<T*>(flag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) <
         target) {
    __builtin_amdgcn_s_sleep(2);
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

// ---------------------------------------------------------------------------
// Deterministic tree reduction of the kSW wave tiles into wave 0's registers:
// rounds of halving; in each round wave i (< half) adds wave i + half's tile,
// passed through LDS in groups of SLOTS tiles.
// ---------------------------------------------------------------------------
template <int MT, int W>
constexpr int red_slots() {
  return MT * W <= 8 ? 4 : 2;  // LDS: SLOTS × MT·W KiB
}

template <int MT, int W>
__device__ __forceinline__ void tree_reduce(f32x4 (&acc)[MT][W], f32x4* red, int wid, int lane) {
  constexpr int SLOTS = red_slots<MT, W>();
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
  //   [0] final latent tiles written (+1 per rank tile and launch)
  //   [1] consumer tickets (+1 per consuming workgroup and launch)
  //   [2 + rt] arrivals of rank tile rt's K chunks (+kLatentUnits/n_kc each,
  //       so every launch adds exactly kLatentUnits whatever its split)
  u64* sync;
  int lr_wgs;       // workgroups that consume the latent (per token tile)
  int lat_weight;   // kLatentUnits / n_kc
  // Bounded waits: where a timeout is reported (the caller's status word, or
  // sync[0]), polls before giving up, and an offset added to every wait's
  // target (nonzero only when a test forces the give-up path).
  u64* status;
  int wait_polls;
  int wait_bias;
};

__device__ __forceinline__ u64* tile_sync(const SlrArgs& a, int mg) {
  return a.sync + 1 + (int64_t)mg * (2 + a.n_rt);
}

// ---------------------------------------------------------------------------
// Latent workgroup: t[token tile, 16-rank tile rt] over all of in_features.
// ---------------------------------------------------------------------------
template <int DT, int MT>
__device__ __forceinline__ void latent_wg(const SlrArgs& a, int wg, f32x4* red) {
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

  f32x4 acc[MT][1];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt][0] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int u0 = ub + wid; u0 < ue; u0 += kSW * UNR) {
    Frag xf[UNR][MT];
    Frag bf[UNR];
#pragma unroll
    for (int k = 0; k < UNR; ++k) {
      const int u = u0 + k * kSW;
      if (u < ue) {
        const int kcol = u * KM + KE * g;
        if (u * KM + KM <= a.m) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            xf[k][mt] = load_kfrag_full<DT, KE>(
                a.x, (int64_t)(m0 + min(mt * 16 + c, Mrem - 1)) * a.ldx + kcol);
        } else {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const int rr = mt * 16 + c;
            const int valid = (rr < Mrem) ? min(KE, a.m - kcol) : 0;
            xf[k][mt] = (valid > 0)
                            ? load_kfrag<DT, KE>(a.x, (int64_t)(m0 + rr) * a.ldx + kcol, valid)
                            : zero_frag<DT, KE>();
          }
        }
        bf[k] = load_kfrag_full<DT, KE>(a.B, brow + kcol);
      }
    }
#pragma unroll
    for (int k = 0; k < UNR; ++k) {
      if (u0 + k * kSW < ue) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) MM::run(acc[mt][0], xf[k][mt], bf[k]);
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
  // output is. Rows past M hold zeros (their x rows were read as zero).
  const auto tr = dev_rsrc(a.t);
  constexpr int EB = Elem<DT>::bytes;
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
  if (lane == 0) rmw_add64(sy, 1);
}

// ---------------------------------------------------------------------------
// Streaming workgroup: one plan chunk for one token tile.
// ---------------------------------------------------------------------------
// SF: storage of the sparse blocks, SF_BSR (q, p) blocks or SF_NM24 packed 2:4 blocks.
template <int DT, int P, int MT, int MODE, int UNR, int SF>
__device__ __forceinline__ void stream_wg(const SlrArgs& a, int chunk, int mg, f32x4* red) {
  constexpr int Q = P;
  constexpr int W = P / 16;
  constexpr int KE = (DT == DT_F32) ? 4 : (Q >= 32 ? 8 : 4);
  using MM = Mma<DT, KE>;
  using Frag = typename MM::Frag;
  constexpr int KM = MM::KM;
  constexpr int NKS = Q / KM;
  static_assert(SF == SF_BSR || (P == kNmBlock && DT != DT_F32), "2:4 blocks are 32×32, 16-bit");
  using Raw = typename std::conditional<SF == SF_NM24, NmRaw, VRawT<DT, KE, W>>::type;
  constexpr int BLK_BYTES = SF == SF_NM24 ? kNmBlockBytes : P * Q * Elem<DT>::bytes;
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
  const int m0 = mg * MT * 16;
  const int Mrem = min(a.M - m0, MT * 16);

  f32x4 acc[MT][W];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int s = 0; s < W; ++s) acc[mt][s] = f32x4{0.f, 0.f, 0.f, 0.f};

  const bool used_t = (MODE == MODE_FUSED) && lb < le;
  // A consumer of the latent takes a ticket at once (its latency hides behind
  // the row's loads). Launch k's consumers hold tickets k·lr_wgs ... and wait
  // for (k + 1)·(latent workgroups) completions, so no counter is ever reset.
  u64 ticket = 0;
  if (used_t && threadIdx.x == 0) ticket = rmw_add64(tile_sync(a, mg) + 1, 1);

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

  // ---- sparse blocks: a batch issues all its loads (x, then the block) unit by
  // unit before the first MFMA, so each unit waits only for its own data.
  for (int u0 = bb + wid; u0 < be; u0 += kSW * UNR) {
    Raw raw[UNR][NKS];
    Frag xf[UNR][NKS][MT];
    // the batch's column indices first, as scalar loads issued together
    int colk[UNR];
#pragma unroll
    for (int k = 0; k < UNR; ++k) colk[k] = ld_uniform(a.col, min(u0 + k * kSW, be - 1)) * Q;
#pragma unroll
    for (int k = 0; k < UNR; ++k) {
      const int u = u0 + k * kSW;
      if (u < be) {
        const int colb = colk[k];
        const char* vb = (const char*)a.values + (int64_t)u * BLK_BYTES;
        const bool full = colb + Q <= a.m;
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
          const int kcol = colb + ks * KM + KE * g;
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const int rr = mt * 16 + c;
            if (full) {
              xf[k][ks][mt] =
                  load_kfrag_full<DT, KE>(a.x, (int64_t)(m0 + min(rr, Mrem - 1)) * a.ldx + kcol);
            } else {
              const int valid = (rr < Mrem) ? min(KE, a.m - kcol) : 0;
              xf[k][ks][mt] = (valid > 0) ? load_kfrag<DT, KE>(
                                                a.x, (int64_t)(m0 + rr) * a.ldx + kcol, valid)
                                          : zero_frag<DT, KE>();
            }
          }
          if constexpr (SF == SF_NM24) load_nm(raw[k][ks], vb, lane);
          else load_vstep<DT, KE, W>(raw[k][ks], vb, P, ks * KM, lane);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < UNR; ++k) {
      if (u0 + k * kSW < be) {
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
          for (int s = 0; s < W; ++s) {
            Frag vf;
            if constexpr (SF == SF_NM24) vf = nm_frag<DT>(raw[k][ks], s);
            else vf = vfrag<DT, KE, W>(raw[k][ks], s);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) MM::run(acc[mt][s], xf[k][ks][mt], vf);
          }
      }
    }
  }

  // ---- low-rank units: 32 ranks of A per unit, t·Aᵀ. One thread of the
  // workgroup waits for this launch's final latent; the barrier releases the
  // other waves, which then read it device-coherently.
  if constexpr (MODE == MODE_FUSED) {
    if (used_t) {
      if (threadIdx.x == 0) {
        const u64 target = (ticket / (u64)a.lr_wgs + 1) * (u64)a.n_rt;
        wait_at_least<u64>(tile_sync(a, mg), target + (u64)a.wait_bias, a.status, a.wait_polls);
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
          for (int mt = 0; mt < MT; ++mt)
            tf[ls][mt] = ld_dev_frag<DT, KEL>(
                tr, (int)(((int64_t)(m0 + mt * 16 + c) * a.ldt + kr) * EB));
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
            for (int mt = 0; mt < MT; ++mt) ML::run(acc[mt][s], tf[ls][mt], af[ls][s]);
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
      store_partial<MT, W>(acc, part_base + (int64_t)seq * TSZ, Mrem, lane);
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
        add_partial<MT, W>(tot, part_base + (int64_t)k * TSZ, Mrem, lane);
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
  if constexpr (MODE == MODE_FUSED) {
    if (a.bias != nullptr) ld_w<DT, W>(a.bias, j0, bv);
  }
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
        st_w<DT, W>(a.y, off, o);
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

template <int DT, int P, int MT, int MODE, int UNR, int SF>
__global__ __launch_bounds__(kST, (DT != DT_F32 && P <= 32) ? 4 : 2) void slr_kernel(
    GroupArgs g_by_value) {
  (void)g_by_value;
  const GroupArgs& g = *(const GroupArgs*)__builtin_amdgcn_kernarg_segment_ptr();
  constexpr int W = P / 16;
  constexpr int SLOTS = red_slots<MT, W>();
  __shared__ f32x4 red[SLOTS * MT * W * kWave];
  const int b = blockIdx.x;
  if constexpr (MODE == MODE_FUSED) {
    if (b < g.lat_total) {
      int i = 0;
      while (i + 1 < g.n && b >= g.lat_off[i + 1]) ++i;
      latent_wg<DT, MT>(g.m[i], b - g.lat_off[i], red);
      return;
    }
  }
  const int sb = b - (MODE == MODE_FUSED ? g.lat_total : 0);
  int i = 0;
  while (i + 1 < g.n && sb >= g.str_off[i + 1]) ++i;
  const SlrArgs& a = g.m[i];
  const int lb = sb - g.str_off[i];
  const int mg = lb / a.n_chunks, chunk = lb % a.n_chunks;
  stream_wg<DT, P, MT, MODE, UNR, SF>(a, chunk, mg, red);
}

// ---------------------------------------------------------------------------
// Host-side launch plumbing
// ---------------------------------------------------------------------------
namespace {

template <int DT, int P, int MT, int SF = SF_BSR>
constexpr int stream_unroll() {
  // Units per wave per batch: a 32-block row in one batch of the 8 waves for
  // 32×32 and 64×64 blocks, fewer units for wide tiles. 16-bit 32×32 kernels stay
  // within 128 VGPRs, so two workgroups share a compute unit.
  constexpr int bytes = P * P * Elem<DT>::bytes;
  constexpr int u = bytes >= 16384 ? 2 : (bytes >= 2048 ? 4 : 16);
  constexpr int d = MT >= 4 ? 4 : MT;
  return u / d > 0 ? u / d : 1;
}

template <int DT, int P, int MT, int MODE, int SF = SF_BSR>
hipError_t launch(const GroupArgs& a, int64_t blocks, hipStream_t s) {
  constexpr int UNR = stream_unroll<DT, P, MT, SF>();
  hipLaunchKernelGGL((slr_kernel<DT, P, MT, MODE, UNR, SF>), dim3((unsigned)blocks), dim3(kST), 0, s,
                     a);
  return hipGetLastError();
}

// The fused linear on 2:4 blocks: 32×32, 16-bit only.
template <int DT>
hipError_t dispatch_nm(int MT, const GroupArgs& a, int64_t blocks, hipStream_t s) {
  switch (MT) {
    case 1: return launch<DT, kNmBlock, 1, MODE_FUSED, SF_NM24>(a, blocks, s);
    case 2: return launch<DT, kNmBlock, 2, MODE_FUSED, SF_NM24>(a, blocks, s);
    case 4: return launch<DT, kNmBlock, 4, MODE_FUSED, SF_NM24>(a, blocks, s);
  }
  return hipErrorInvalidValue;
}

template <int DT, int MODE>
hipError_t dispatch_p(int P, int MT, const GroupArgs& a, int64_t blocks, hipStream_t s) {
#define SSL_CASE(PP, MM) \
  if (P == PP && MT == MM) return launch<DT, PP, MM, MODE>(a, blocks, s);
  SSL_CASE(16, 1) SSL_CASE(16, 2) SSL_CASE(16, 4)
  SSL_CASE(32, 1) SSL_CASE(32, 2) SSL_CASE(32, 4)
  SSL_CASE(64, 1) SSL_CASE(64, 2) SSL_CASE(64, 4)
#undef SSL_CASE
  return hipErrorInvalidValue;
}

template <int MODE>
hipError_t dispatch(int dtype, int P, int MT, const GroupArgs& a, int64_t blocks, hipStream_t s) {
  switch (dtype) {
    case SSL_F32: return dispatch_p<DT_F32, MODE>(P, MT, a, blocks, s);
    case SSL_BF16: return dispatch_p<DT_BF16, MODE>(P, MT, a, blocks, s);
    case SSL_F16: return dispatch_p<DT_F16, MODE>(P, MT, a, blocks, s);
  }
  return hipErrorInvalidValue;
}

// Most in_features chunks of the latent a call may use (the workspace is
// sized for this many fp32 partials). More chunks put more workgroups, and so
// more of the device's memory parallelism, on the latent that every row needs
// before it can finish; chunks stay at least 512 columns wide, and calls with
// many token rows keep few partials.
int latent_split_max(int64_t M, int64_t m_pad) {
  int64_t n = m_pad / 512;
  const int64_t by_tokens = 128 / (M > 0 ? M : 1);
  if (n > by_tokens) n = by_tokens;
  if (n > 8) n = 8;
  return n < 1 ? 1 : (int)n;
}

bool supported_block(int p, int q) { return p == q && (p == 16 || p == 32 || p == 64); }
bool supported_dtype(int dt) { return dt == SSL_F32 || dt == SSL_BF16 || dt == SSL_F16; }

// Scratch layout of one fused call. Row counters live in their own int32 array
// (zero at rest, never shared with data) and the handshake words in the plan's
// own uint64 array; the data workspace holds the latent partials, the final
// latent and the fp32 partial tiles of split rows (byte offsets).
struct Layout {
  int MT, MG;
  int n_rt, n_kc_max, ku_total;
  int64_t cnt_total;  // int32 row counters: [MG][NB]
  int64_t n_sync;     // u64 handshake words: status, then (2 + n_rt) per token tile
  int64_t t_part, t_final, part_main, total;
};

Layout slr_layout(int64_t M, int64_t NB, int p, int64_t r_pad, int64_t m_pad, int64_t n_slots,
                  int dtype) {
  Layout L{};
  L.MT = tile_mt(M);
  L.MG = (int)((M + 16 * L.MT - 1) / (16 * L.MT));
  L.n_rt = (int)(r_pad / 16);
  const int KM = dtype == SSL_F32 ? 16 : 32;
  L.ku_total = (int)(m_pad / KM);
  L.n_kc_max = latent_split_max(M, m_pad);
  L.cnt_total = (int64_t)L.MG * NB;
  L.n_sync = 1 + (int64_t)L.MG * (2 + L.n_rt);
  const int64_t rows = (int64_t)L.MG * 16 * L.MT;
  int64_t off = 0;
  L.t_part = off;
  if (M >= kPrefillMinM && dtype != SSL_F32) {
    // prefill: the latent GEMM's K-split partials
    const int ks = prefill_latent_split(M, r_pad, m_pad, device_cus());
    if (ks > 1) off = align_up(off + 4 * (int64_t)ks * rows * r_pad, 256);
  } else if (L.n_kc_max > 1) {
    off = align_up(off + 4 * (int64_t)L.n_kc_max * rows * r_pad, 256);
  }
  L.t_final = off;
  off = align_up(off + (int64_t)elem_bytes(dtype) * rows * r_pad, 256);
  L.part_main = off;
  off = align_up(off + 4 * (int64_t)L.MG * n_slots * (16 * L.MT * p), 256);
  L.total = off;
  return L;
}

// K chunks of this launch's latent: as many as the free compute units allow
// (latent workgroups — per_chunk of them per K chunk — and the n_stream row
// workgroups all resident at once), at most n_kc_max; then evened out so no
// chunk is empty.
void latent_chunks(const Layout& L, int64_t n_stream, int64_t per_chunk, int* n_kc,
                   int* ku_chunk) {
  int64_t n = per_chunk > 0 ? (device_cus() - n_stream) / per_chunk : 1;
  if (n > L.n_kc_max) n = L.n_kc_max;
  if (n < 1) n = 1;
  int ku = (int)((L.ku_total + n - 1) / n);
  if (ku < 1) ku = 1;
  *ku_chunk = ku;
  *n_kc = (L.ku_total + ku - 1) / ku;
  if (*n_kc < 1) *n_kc = 1;
}

}  // namespace
}  // namespace ssl

using namespace ssl;

extern "C" {

int64_t ssl_prefill_min_rows(void) { return kPrefillMinM; }

// Which kernels a fused call with block storage takes. The prefill kernels
// from kPrefillMinM token rows with 16-bit activations, except where the
// streaming kernel (one weight pass per 64-row token tile, the re-reads served
// by the caches) measured faster on MI355X: blocks of 32×32 or less up to 512
// rows (LLaMA-1B gate 5461×2048 at 128 / 256 / 512 rows: 34.2 / 41.8 / 65.5 µs
// prefill, 24.5 / 35.6 / 55.1 streaming), and calls of fewer than 100
// block-rows up to 128 rows (4096×4096 with 64×64 blocks: 40.7 -> 31.9 µs).
int32_t ssl_slr_takes_prefill(int64_t M, int64_t n_rows, int32_t block_p, int32_t dtype) {
  if (dtype == SSL_F32 || M < kPrefillMinM) return 0;
  if (block_p <= 32 && M <= 512) return 0;
  if (M <= kPrefillMinM && n_rows < 100) return 0;
  return 1;
}

int64_t ssl_nm24_block_bytes(void) { return kNmBlockBytes; }

int32_t ssl_prefill_group(int64_t M, int64_t n_rows, int32_t block_p) {
  if (!supported_block(block_p, block_p)) return 1;
  return prefill_group(M, n_rows, block_p, device_cus());
}

int64_t ssl_bsr_addmm_counter_count(int64_t M, int64_t NB) {
  const int MT = tile_mt(M);
  const int64_t MG = (M + 16 * MT - 1) / (16 * MT);
  return MG * NB;
}

int64_t ssl_bsr_addmm_workspace_size(int64_t M, int64_t NB, int32_t block_p, int64_t n_slots) {
  (void)NB;
  const int MT = tile_mt(M);
  const int64_t MG = (M + 16 * MT - 1) / (16 * MT);
  return align_up(4 * MG * n_slots * (16 * MT * block_p), 256);
}

int ssl_bsr_addmm_inplace(void* out, int64_t ldo, const void* x, int64_t ldx, const int32_t* col,
                          const void* values, int64_t nnz, const int32_t* plan, int64_t n_chunks,
                          int64_t n_slots, const void* values_pq, const int32_t* pf_groups,
                          const int32_t* pf_entries,
                          int64_t pf_n_groups, int32_t pf_group, int64_t M, int64_t N, int64_t K,
                          int64_t NB, int32_t block_p, int32_t block_q, int32_t dtype,
                          int32_t* counters, int64_t n_counters, void* workspace,
                          int64_t workspace_bytes, void* stream) {
  clear_error();
  if (!supported_dtype(dtype)) return fail(SSL_ERR_UNSUPPORTED, "unsupported dtype %d", dtype);
  if (!supported_block(block_p, block_q))
    return fail(SSL_ERR_UNSUPPORTED,
                "BSR kernel needs square 16, 32 or 64 blocks, got %dx%d", block_p, block_q);
  if (M < 0 || N < 0 || K < 0 || NB < 0 || n_chunks < 0 || n_slots < 0)
    return fail(SSL_ERR_INVALID, "negative size");
  if (N != NB * block_p) return fail(SSL_ERR_INVALID, "out N=%lld does not match crow/block_p", (long long)N);
  if (K % block_q) return fail(SSL_ERR_INVALID, "x K=%lld must be divisible by block_q", (long long)K);
  if (M == 0 || n_chunks == 0) return SSL_OK;
  const int MT = tile_mt(M);
  const int64_t MG = (M + 16 * MT - 1) / (16 * MT);
  if (n_chunks * MG > 0x7fffffffLL) return fail(SSL_ERR_INVALID, "grid too large");
  const int eb = elem_bytes(dtype);
  if (!out || !x || !col || !values || !plan) return fail(SSL_ERR_INVALID, "null pointer");
  if (ldx < K || ldo < N) return fail(SSL_ERR_INVALID, "leading dimension smaller than row");
  if (!aligned(x, 16) || (ldx * eb) % 16 || !aligned(values, 16))
    return fail(SSL_ERR_INVALID, "x rows and values must be 16-byte aligned");
  if (!aligned(out, 16) || (ldo * eb) % 16) return fail(SSL_ERR_INVALID, "out rows must be 16-byte aligned");
  const int64_t need = ssl_bsr_addmm_workspace_size(M, NB, block_p, n_slots);
  if (workspace_bytes < need || (need > 0 && !workspace))
    return fail(SSL_ERR_WORKSPACE, "workspace of %lld bytes needed", (long long)need);
  if (workspace && !aligned(workspace, 256))
    return fail(SSL_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  if (n_counters < ssl_bsr_addmm_counter_count(M, NB) || !counters)
    return fail(SSL_ERR_WORKSPACE, "%lld zeroed counters needed",
                (long long)ssl_bsr_addmm_counter_count(M, NB));

  if (M >= kPrefillMinM && dtype != SSL_F32) {
    if (!pf_groups || !pf_entries || pf_n_groups <= 0 || !values_pq)
      return fail(SSL_ERR_INVALID, "calls with %lld token rows need a prefill plan and (p, q) "
                  "ordered block values", (long long)M);
    if (pf_group != prefill_group(M, n_chunks, block_p, device_cus()))
      return fail(SSL_ERR_INVALID, "prefill plan built for group %d, this call needs %d", pf_group,
                  prefill_group(M, n_chunks, block_p, device_cus()));
    if (nnz < 0 || nnz * block_p * block_q * eb > 0x7fffffffLL)
      return fail(SSL_ERR_UNSUPPORTED, "block values beyond 2 GiB");
    PfArgs rows{};
    rows.x = x; rows.ldx = ldx; rows.M = (int)M; rows.m = (int)K; rows.m_pad = (int)K;
    rows.mode = PF_OP;
    rows.n = 1;
    PfMember& pm = rows.mb[0];
    pm.y = out; pm.ldy = ldo; pm.values_pq = values_pq;
    pm.values_bytes = nnz * block_p * block_q * eb;
    pm.groups = pf_groups; pm.entries = pf_entries; pm.n_groups = (int)pf_n_groups;
    const int64_t T = (M + prefill_row_tile(pf_group) - 1) / prefill_row_tile(pf_group);
    if (pf_n_groups * T > 0x7fffffffLL / 8) return fail(SSL_ERR_INVALID, "grid too large");
    rows.items = (int)(pf_n_groups * T);
    rows.off[1] = rows.items;
    return check_hip(prefill_launch_op(dtype, block_p, pf_group, rows, (hipStream_t)stream),
                     "bsr_addmm prefill launch");
  }

  GroupArgs g{};
  g.n = 1;
  g.str_off[1] = (int)(n_chunks * MG);
  SlrArgs& a = g.m[0];
  a.x = x; a.ldx = ldx; a.M = (int)M; a.m = (int)K;
  a.y = out; a.ldy = ldo; a.col = col; a.values = values; a.plan = plan;
  a.n_chunks = (int)n_chunks; a.NB = (int)NB;
  a.n_slots = n_slots; a.part_main = (float*)workspace; a.cnt_main = counters;
  return check_hip(dispatch<MODE_OP>(dtype, block_p, MT, g, n_chunks * MG, (hipStream_t)stream),
                   "bsr_addmm launch");
}

int64_t ssl_slr_counter_count(int64_t M, int64_t NB) {
  return slr_layout(M, NB, 16, 0, 64, 0, SSL_BF16).cnt_total;
}

int64_t ssl_slr_exchange_size(int64_t M, int64_t r_pad, int64_t m_pad, int32_t dtype) {
  (void)m_pad;
  (void)dtype;
  return align_up(8 * slr_layout(M, 0, 16, r_pad, 64, 0, SSL_BF16).n_sync, 256);
}

int64_t ssl_slr_workspace_size(int64_t M, int64_t NB, int32_t block_p, int64_t r_pad,
                               int64_t m_pad, int64_t n_slots, int32_t dtype) {
  return slr_layout(M, NB, block_p, r_pad, m_pad, n_slots, dtype).total;
}

int ssl_slr_forward_group(const void* x, int64_t ldx, int64_t M, int64_t m, int64_t m_pad,
                          int32_t block_p, int32_t block_q, int32_t dtype,
                          const ssl_slr_member* members, int32_t n_members, void* stream) {
  clear_error();
  if (!supported_dtype(dtype)) return fail(SSL_ERR_UNSUPPORTED, "unsupported dtype %d", dtype);
  if (!supported_block(block_p, block_q))
    return fail(SSL_ERR_UNSUPPORTED,
                "SLR kernel needs square 16, 32 or 64 blocks, got %dx%d", block_p, block_q);
  if (n_members < 1 || n_members > kMaxGroup || !members)
    return fail(SSL_ERR_INVALID, "a fused call takes 1 to %d linears, got %d", kMaxGroup, n_members);
  if (M < 0 || m < 0) return fail(SSL_ERR_INVALID, "negative size");
  if (m_pad % 64 || m_pad < m) return fail(SSL_ERR_INVALID, "m_pad must be a multiple of 64 and >= m");
  const int eb = elem_bytes(dtype);
  if (M == 0) return SSL_OK;
  if (!x || !aligned(x, 16) || ldx < m || (ldx * eb) % 16)
    return fail(SSL_ERR_INVALID, "x rows must be 16-byte aligned and at least m wide");

  GroupArgs g{};
  g.n = n_members;
  Layout L[kMaxGroup];
  int64_t n_stream = 0, rt_tiles = 0;
  const int s_format = members[0].s_format;
  if (s_format != SSL_S_BSR && s_format != SSL_S_NM24)
    return fail(SSL_ERR_INVALID, "unknown sparse storage format %d", s_format);
  if (s_format == SSL_S_NM24 && (block_p != kNmBlock || block_q != kNmBlock || dtype == SSL_F32))
    return fail(SSL_ERR_UNSUPPORTED, "2:4 blocks are 32x32 with 16-bit activations");
  for (int i = 0; i < n_members; ++i) {
    const ssl_slr_member& mb = members[i];
    if (mb.NB < 0 || mb.r_pad < 0 || mb.n_chunks < 0 || mb.n_slots < 0 || mb.lr_wgs < 0)
      return fail(SSL_ERR_INVALID, "linear %d: negative size", i);
    if (mb.s_format != s_format)
      return fail(SSL_ERR_INVALID, "linear %d: all linears of a call share the sparse storage", i);
    if (mb.r_pad % 64) return fail(SSL_ERR_INVALID, "linear %d: r_pad must be a multiple of 64", i);
    if (mb.NB == 0) {  // no output columns: nothing to launch for this linear
      L[i] = slr_layout(M, 0, block_p, 0, m_pad, 0, dtype);
      continue;
    }
    if (mb.n_chunks == 0)
      return fail(SSL_ERR_INVALID, "linear %d: empty plan for a non-empty output", i);
    if ((mb.r_pad > 0) != (mb.lr_wgs > 0) || mb.lr_wgs > mb.n_chunks)
      return fail(SSL_ERR_INVALID, "linear %d: lr_wgs must count the plan's chunks with low-rank units", i);
    if (!mb.y || !mb.plan || (mb.r_pad > 0 && (!mb.A || !mb.B)))
      return fail(SSL_ERR_INVALID, "linear %d: null pointer", i);
    if (mb.ldy < mb.NB * block_p || !aligned(mb.y, 16) || (mb.ldy * eb) % 16)
      return fail(SSL_ERR_INVALID, "linear %d: y rows must be 16-byte aligned and NB·p wide", i);
    if ((mb.A && !aligned(mb.A, 16)) || (mb.B && !aligned(mb.B, 16)) ||
        (mb.values && !aligned(mb.values, 16)))
      return fail(SSL_ERR_INVALID, "linear %d: A, B and values must be 16-byte aligned", i);
    L[i] = slr_layout(M, mb.NB, block_p, mb.r_pad, m_pad, mb.n_slots, dtype);
    if (L[i].total > 0x7fffffffLL)
      return fail(SSL_ERR_UNSUPPORTED,
                  "linear %d: workspace of %lld bytes exceeds 2 GiB; split the call by tokens", i,
                  (long long)L[i].total);
    if (mb.workspace_bytes < L[i].total || !mb.workspace)
      return fail(SSL_ERR_WORKSPACE, "linear %d: workspace of %lld bytes needed", i,
                  (long long)L[i].total);
    if (!aligned(mb.workspace, 256))
      return fail(SSL_ERR_WORKSPACE, "linear %d: workspace must be 256-byte aligned", i);
    if (mb.n_counters < L[i].cnt_total || !mb.counters)
      return fail(SSL_ERR_WORKSPACE, "linear %d: %lld zeroed counters needed", i,
                  (long long)L[i].cnt_total);
    if (mb.exchange_bytes < 8 * L[i].n_sync || !mb.exchange)
      return fail(SSL_ERR_WORKSPACE, "linear %d: exchange area of %lld bytes needed", i,
                  (long long)(8 * L[i].n_sync));
    if (!aligned(mb.exchange, 256))
      return fail(SSL_ERR_WORKSPACE, "linear %d: exchange area must be 256-byte aligned", i);
    n_stream += (mb.NB > 0 ? mb.n_chunks : 0) * L[i].MG;
    rt_tiles += (int64_t)L[i].n_rt * L[i].MG;
  }
  if (n_stream == 0) return SSL_OK;

  int64_t call_rows = 0;
  for (int i = 0; i < n_members; ++i) call_rows += members[i].NB;
  if (s_format == SSL_S_BSR && ssl_slr_takes_prefill(M, call_rows, block_p, dtype)) {
    // Many token rows: the latent GEMM (K split, then combined), then the row
    // GEMM over groups of block-rows. (2:4 blocks stay on the row-streaming
    // kernel at every M.)
    const int cus = device_cus();
    PfArgs rows{}, lat{};
    rows.x = lat.x = x; rows.ldx = lat.ldx = ldx;
    rows.M = lat.M = (int)M; rows.m = lat.m = (int)m; rows.m_pad = lat.m_pad = (int)m_pad;
    rows.rows = lat.rows = (int)((M + 63) / 64 * 64);
    rows.mode = PF_FUSED;
    rows.n = lat.n = n_members;
    const int64_t T64 = (M + 63) / 64;
    // one group size for the whole call, from all members' rows together
    int64_t total_rows = 0;
    for (int i = 0; i < n_members; ++i)
      if (members[i].NB > 0) total_rows += members[i].n_chunks;
    const int G = prefill_group(M, total_rows, block_p, cus);
    int64_t items = 0, litems = 0;
    for (int i = 0; i < n_members; ++i) {
      const ssl_slr_member& mb = members[i];
      PfMember& pm = rows.mb[i];
      rows.off[i] = (int)items;
      lat.off[i] = (int)litems;
      if (mb.NB == 0) continue;
      if (!mb.pf_groups || !mb.pf_entries || mb.pf_n_groups <= 0 || mb.pf_group != G ||
          (mb.nnz > 0 && !mb.values_pq))
        return fail(SSL_ERR_INVALID, "linear %d: calls with %lld token rows need a prefill plan "
                    "with group %d and (p, q) ordered block values", i, (long long)M, G);
      const int64_t T = (M + prefill_row_tile(G) - 1) / prefill_row_tile(G);
      if (mb.nnz < 0 || mb.nnz * block_p * block_p * eb > 0x7fffffffLL ||
          mb.NB * block_p * mb.r_pad * eb > 0x7fffffffLL)
        return fail(SSL_ERR_UNSUPPORTED, "linear %d: weights beyond 2 GiB", i);
      pm.y = mb.y; pm.ldy = mb.ldy; pm.A = mb.A; pm.lda = mb.r_pad;
      pm.A_bytes = mb.NB * block_p * mb.r_pad * eb; pm.bias = mb.bias;
      pm.values_pq = mb.values_pq; pm.values_bytes = mb.nnz * block_p * block_p * eb;
      pm.groups = mb.pf_groups; pm.entries = mb.pf_entries; pm.n_groups = (int)mb.pf_n_groups;
      pm.B = mb.B; pm.ldb = m_pad;
      pm.t = (char*)mb.workspace + L[i].t_final; pm.ldt = mb.r_pad;
      pm.tpart = (float*)((char*)mb.workspace + L[i].t_part);
      pm.r_pad = (int)mb.r_pad;
      pm.ksplit = mb.r_pad > 0 ? prefill_latent_split(M, mb.r_pad, m_pad, cus) : 1;
      lat.mb[i] = pm;
      items += mb.pf_n_groups * T;
      if (mb.r_pad > 0) litems += T64 * (mb.r_pad / 64) * pm.ksplit;
      if (items > 0x7fffffffLL / 8 || litems > 0x7fffffffLL) return fail(SSL_ERR_INVALID, "grid too large");
    }
    rows.off[n_members] = (int)items;
    lat.off[n_members] = (int)litems;
    rows.items = (int)items;
    lat.items = (int)litems;
    // combine workgroups (members with a split latent), offsets in member order
    PfArgs comb = lat;
    {
      int64_t c = 0;
      for (int i = 0; i < n_members; ++i) {
        comb.off[i] = (int)c;
        if (members[i].NB > 0 && members[i].r_pad > 0 && lat.mb[i].ksplit > 1)
          c += (rows.rows * members[i].r_pad / 4 + 255) / 256;
      }
      comb.off[n_members] = (int)c;
      comb.combine_items = (int)c;
    }
    return check_hip(prefill_launch_fused(dtype, block_p, G, rows, lat, comb, (hipStream_t)stream),
                     "slr prefill launch");
  }

  const DebugKnobs& knobs = debug_knobs();
  // One K split for the whole launch: latent and row workgroups of every
  // member resident at once.
  int n_kc = 1, ku_chunk = 1;
  latent_chunks(L[0], n_stream, rt_tiles, &n_kc, &ku_chunk);
  int64_t lat = 0, str = 0;
  for (int i = 0; i < n_members; ++i) {
    const ssl_slr_member& mb = members[i];
    g.lat_off[i] = (int)lat;
    g.str_off[i] = (int)str;
    lat += (int64_t)L[i].n_rt * n_kc * L[i].MG;
    str += (mb.NB > 0 ? mb.n_chunks : 0) * L[i].MG;
    if (lat + str > 0x7fffffffLL) return fail(SSL_ERR_INVALID, "grid too large");
    char* ws = (char*)mb.workspace;
    SlrArgs& a = g.m[i];
    a.x = x; a.ldx = ldx; a.M = (int)M; a.m = (int)m;
    a.y = mb.y; a.ldy = mb.ldy; a.col = mb.col; a.values = mb.values; a.plan = mb.plan;
    a.n_chunks = (int)mb.n_chunks; a.NB = (int)mb.NB;
    a.A = mb.A; a.lda = mb.r_pad; a.bias = mb.bias;
    a.n_slots = mb.n_slots; a.part_main = (float*)(ws + L[i].part_main); a.cnt_main = mb.counters;
    a.B = mb.B; a.ldb = m_pad; a.t = ws + L[i].t_final; a.ldt = mb.r_pad;
    a.t_part = (float*)(ws + L[i].t_part);
    a.MG = L[i].MG; a.n_rt = L[i].n_rt; a.n_kc = n_kc; a.ku_total = L[i].ku_total;
    a.ku_chunk = ku_chunk;
    a.n_lat_wgs = (int)((int64_t)L[i].n_rt * n_kc * L[i].MG);
    a.sync = (u64*)mb.exchange; a.lr_wgs = (int)mb.lr_wgs; a.lat_weight = kLatentUnits / n_kc;
    a.status = mb.status ? (u64*)mb.status : (u64*)mb.exchange;
    a.wait_polls = knobs.wait_polls > 0 ? (int)knobs.wait_polls : kSpinLimit;
    // out of reach of any launch: tickets and counters advance far less per launch
    a.wait_bias = knobs.wait_unreachable ? (1 << 30) : 0;
  }
  g.lat_off[n_members] = (int)lat;
  g.str_off[n_members] = (int)str;
  g.lat_total = (int)lat;
  if (s_format == SSL_S_NM24)
    return check_hip(dtype == SSL_BF16
                         ? dispatch_nm<DT_BF16>(L[0].MT, g, lat + str, (hipStream_t)stream)
                         : dispatch_nm<DT_F16>(L[0].MT, g, lat + str, (hipStream_t)stream),
                     "slr launch (2:4)");
  return check_hip(
      dispatch<MODE_FUSED>(dtype, block_p, L[0].MT, g, lat + str, (hipStream_t)stream),
      "slr launch");
}

int ssl_slr_forward(void* y, int64_t ldy, const void* x, int64_t ldx, const void* A, const void* B,
                    const void* bias, const int32_t* col, const void* values, const int32_t* plan,
                    int64_t n_chunks, int64_t n_slots, int64_t lr_wgs, int64_t M, int64_t m,
                    int64_t m_pad, int64_t NB, int64_t r_pad, int32_t block_p, int32_t block_q,
                    int32_t dtype, int32_t* counters, int64_t n_counters, void* exchange,
                    int64_t exchange_bytes, void* workspace, int64_t workspace_bytes, void* stream) {
  ssl_slr_member mb{};
  mb.y = y; mb.ldy = ldy; mb.A = A; mb.B = B; mb.bias = bias; mb.col = col; mb.values = values;
  mb.plan = plan; mb.n_chunks = n_chunks; mb.n_slots = n_slots; mb.lr_wgs = lr_wgs;
  mb.NB = NB; mb.r_pad = r_pad; mb.counters = counters; mb.n_counters = n_counters;
  mb.exchange = exchange; mb.exchange_bytes = exchange_bytes;
  mb.workspace = workspace; mb.workspace_bytes = workspace_bytes;
  return ssl_slr_forward_group(x, ldx, M, m, m_pad, block_p, block_q, dtype, &mb, 1, stream);
}

}  // extern "C"
