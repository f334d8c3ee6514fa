// Prefill-shaped SLR linear on gfx950: many token rows (M ≥ kPrefillMinM), 16-bit
// activations. Two LDS-tiled MFMA kernels instead of the row-streaming decode
// kernel (which re-reads each weight row once per 64-token tile):
//
//   latent  t[M, r_pad] = x · Bᵀ                   dense GEMM, rounded once to
//                                                    the activation dtype (as F.linear)
//   rows    y[:, row] = Σ_blocks x[:, col·p:+p] · V_blockᵀ + t · A[row·p:+p, :]ᵀ
//                       (+ bias, or + the old out for the in-place op)
//
// Both run one engine: a workgroup of 4 waves owns a BM × BN output tile (BM =
// 64·MTW token rows, wave w the rows [16·MTW·w, +16·MTW)) and walks a list of
// K units of width KU. Each unit stages an A tile (BM × KU, from x or t) and a
// B tile (BN × KU, k-contiguous per output column) in LDS, double buffered:
// the next units' global loads are in flight while the current one feeds the
// MFMAs. Every B tile is copied as k-contiguous rows: sparse blocks come from a
// (p, q)-ordered copy of the block values (made once per weight), low-rank and
// latent units from the rows of A or B.
//
// Token rows past M read row M − 1 (their outputs are never stored), so the
// only masked loads are x columns past in_features in a ragged last unit.
// Row workgroups are ordered XCD-major, token tile by token tile: the
// workgroups one XCD runs at a time share a token tile, so its x panel stays in
// that XCD's L2 while the block-rows stream past it.

#include "abi_internal.h"
#include "prefill.h"
#include "slr_common.h"

namespace ssl {

namespace {

constexpr int kPfThreads = 256;  // 4 waves
constexpr int kXcds = 8;

template <int DT>
__device__ __forceinline__ typename Mma<DT, 8>::Frag lds_frag8(const uint16_t* p) {
  const uint4 v = *(const uint4*)p;
  typename Mma<DT, 8>::Frag f;
  f.d[0] = v.x; f.d[1] = v.y; f.d[2] = v.z; f.d[3] = v.w;
  return f;
}
template <int DT>
__device__ __forceinline__ typename Mma<DT, 4>::Frag lds_frag4(const uint16_t* p) {
  const uint2 v = *(const uint2*)p;
  typename Mma<DT, 4>::Frag f;
  f.d[0] = v.x; f.d[1] = v.y;
  return f;
}

// Buffer-resource loads: an offset at or past the resource's size reads as
// zero with no memory access, so absent blocks need no branch and no traffic.
constexpr uint32_t kOob = 0x80000000u;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t mk_rsrc(const void* base, int64_t bytes) {
  const int n = bytes > 0x7fffffffLL ? 0x7fffffff : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}
__device__ __forceinline__ uint4 ld16_buf(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const auto u = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return make_uint4(u[0], u[1], u[2], u[3]);
}

template <int DT, int KE>
__device__ __forceinline__ typename Mma<DT, KE>::Frag zero_past(typename Mma<DT, KE>::Frag f,
                                                                 int k0, int kmax) {
  // elements k0 + e (e < KE) at or past kmax read as zero
#pragma unroll
  for (int d = 0; d < KE / 2; ++d) {
    const uint32_t lo = (k0 + 2 * d < kmax) ? (f.d[d] & 0xffffu) : 0u;
    const uint32_t hi = (k0 + 2 * d + 1 < kmax) ? (f.d[d] & 0xffff0000u) : 0u;
    f.d[d] = lo | hi;
  }
  return f;
}

// Tile geometry. A workgroup owns BM = 64·MTW token rows (wave w: the rows
// [16·MTW·w, +16·MTW)) and G block-rows of p columns ("slots"). A unit is one
// K step of width p: the A tile (x or t columns, each wave its own rows, straight
// into registers) and the B tiles of the G slots (p × p each, through LDS, shared
// by the 4 waves).
template <int DT, int P, int G, int MTW>
struct Geo {
  static constexpr int KU = P, W = P / 16, KP = P + 8;
  static constexpr int KE = P >= 32 ? 8 : 4;
  static constexpr int KM = Mma<DT, KE>::KM;
  static constexpr int NKS = P / KM;
  static constexpr int CHUNKS = G * P * P / 8;  // 16-byte pieces of the G B tiles
  static constexpr int NLD = (CHUNKS + kPfThreads - 1) / kPfThreads;
};

template <int DT, int P, int G, int MTW>
struct Stage {
  using Gm = Geo<DT, P, G, MTW>;
  typename Mma<DT, Gm::KE>::Frag a[MTW][Gm::NKS];
  uint4 b[Gm::NLD];
  int mask;
};

// Where one unit's tiles come from (all wave-uniform).
template <int G>
struct Unit {
  const uint16_t* a;  // A source: row-major, row stride lda, unit columns [ka, ka + p)
  int64_t lda;
  int ka;
  int kmax;           // A columns at and past kmax read as zero (in_features for x)
  int kread;          // last column a full fragment may start at (row length − KE)
  __amdgpu_buffer_rsrc_t br;  // B source
  uint32_t base[G];   // per slot: byte offset of its p × p tile in br, kOob if absent
  uint32_t bld;       // bytes between the k-contiguous rows [col][k] of a tile
  int mask;           // slots present
};

// LDS row of B-tile column j: column W·c + s at row 16·s + c, so the 16 lanes
// reading one column tile hit 16 consecutive rows (no bank conflict) while a
// lane still owns W adjacent output columns in the epilogue.
template <int P>
__device__ __forceinline__ int brow(int j) {
  constexpr int W = P / 16;
  return 16 * (j % W) + j / W;
}

template <int G>
__device__ __forceinline__ uint32_t slot_base(const Unit<G>& u, int g) {
  uint32_t v = kOob;
#pragma unroll
  for (int q = 0; q < G; ++q) v = (g == q) ? u.base[q] : v;
  return v;
}

template <int DT, int P, int G, int MTW>
__device__ __forceinline__ void load_unit(const Unit<G>& u, int m0, int M, int wid, int lane,
                                          Stage<DT, P, G, MTW>& st) {
  using Gm = Geo<DT, P, G, MTW>;
  constexpr int KE = Gm::KE;
  const int c = lane & 15, gq = lane >> 4;
#pragma unroll
  for (int mt = 0; mt < MTW; ++mt) {
    const int row = min(m0 + wid * 16 * MTW + mt * 16 + c, M - 1);
    const uint16_t* rp = u.a + (int64_t)row * u.lda;
#pragma unroll
    for (int ks = 0; ks < Gm::NKS; ++ks) {
      const int k = u.ka + ks * Gm::KM + KE * gq;
      const auto f = load_kfrag_full<DT, KE>(rp, min(k, u.kread));
      st.a[mt][ks] = (k + KE <= u.kmax) ? f : zero_past<DT, KE>(f, k, u.kmax);
    }
  }
  const int tid = threadIdx.x;
  constexpr int PER = P * P / 8;   // pieces per tile
  constexpr int CPR = P / 8;       // pieces per tile row
#pragma unroll
  for (int i = 0; i < Gm::NLD; ++i) {
    const int q = tid + kPfThreads * i;
    const int g = q / PER, r = q % PER;
    const int j = r / CPR, kc = (r % CPR) * 8;
    const uint32_t off =
        (q < Gm::CHUNKS ? slot_base(u, g) : kOob) + (uint32_t)j * u.bld + (uint32_t)(kc * 2);
    st.b[i] = ld16_buf(u.br, off);
  }
  st.mask = u.mask;
}

template <int DT, int P, int G, int MTW>
__device__ __forceinline__ void store_b(const Stage<DT, P, G, MTW>& st, uint16_t* sb) {
  using Gm = Geo<DT, P, G, MTW>;
  constexpr int KP = Gm::KP;
  constexpr int PER = P * P / 8, CPR = P / 8;
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < Gm::NLD; ++i) {
    const int q = tid + kPfThreads * i;
    if (Gm::CHUNKS % kPfThreads == 0 || q < Gm::CHUNKS) {
      const int g = q / PER, r = q % PER;
      const int j = r / CPR, kc = (r % CPR) * 8;
      *(uint4*)(sb + (g * P + brow<P>(j)) * KP + kc) = st.b[i];
    }
  }
}

// MFMAs of one unit for the slots present: A fragments from the stage
// registers, B from LDS; acc[g][mt][s] (column tile s, lane column c → column W·c + s).
template <int DT, int P, int G, int MTW>
__device__ __forceinline__ void compute_unit(const Stage<DT, P, G, MTW>& st, const uint16_t* sb,
                                             int lane, f32x4 (&acc)[G][MTW][P / 16]) {
  using Gm = Geo<DT, P, G, MTW>;
  constexpr int KE = Gm::KE, W = Gm::W, KP = Gm::KP;
  using MM = Mma<DT, KE>;
  const int c = lane & 15, gq = lane >> 4;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if ((st.mask >> g) & 1) {
#pragma unroll
      for (int ks = 0; ks < Gm::NKS; ++ks) {
        const int k = ks * Gm::KM + KE * gq;
        typename MM::Frag bf[W];
#pragma unroll
        for (int s = 0; s < W; ++s) {
          const uint16_t* p = sb + (g * P + 16 * s + c) * KP + k;
          if constexpr (KE == 8) bf[s] = lds_frag8<DT>(p);
          else bf[s] = lds_frag4<DT>(p);
        }
#pragma unroll
        for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
          for (int s = 0; s < W; ++s) MM::run(acc[g][mt][s], st.a[mt][ks], bf[s]);
      }
    }
  }
}

// The unit pipeline: D units in flight in registers (a ring whose slot k
// always holds a unit ≡ k mod D, a constant once the loop is unrolled); the B
// tiles of the unit being computed sit in one LDS buffer while the next unit's
// are written to the other. A unit's loads are issued D units before its MFMAs.
// Units past the end load the last unit again (never computed), so every load
// is unconditional and each wait covers exactly the loads it needs.
template <int DT, int P, int G, int MTW, int D, typename UnitFn>
__device__ __forceinline__ void run_units(const UnitFn& unit, int U, int m0, int M, uint16_t* sb0,
                                          uint16_t* sb1, int wid, int lane,
                                          f32x4 (&acc)[G][MTW][P / 16]) {
  if (U <= 0) return;
  Stage<DT, P, G, MTW> st[D];
#pragma unroll
  for (int k = 0; k < D; ++k) load_unit<DT, P, G, MTW>(unit(min(k, U - 1)), m0, M, wid, lane, st[k]);
  store_b<DT, P, G, MTW>(st[0], sb0);
  __syncthreads();
  for (int u0 = 0; u0 < U; u0 += D) {
#pragma unroll
    for (int k = 0; k < D; ++k) {
      const int u = u0 + k;
      const int s = (k + 1) % D;  // holds unit u + 1
      if (u < U) {
        compute_unit<DT, P, G, MTW>(st[k], (u & 1) ? sb1 : sb0, lane, acc);
        if (u + 1 < U) store_b<DT, P, G, MTW>(st[s], (u & 1) ? sb0 : sb1);
      }
      load_unit<DT, P, G, MTW>(unit(min(u + D, U - 1)), m0, M, wid, lane, st[k]);
      __syncthreads();
    }
  }
}

// XCD-major work order: blocks b, b + 8, b + 16, ... run on one XCD, so the
// items one XCD holds at a time are consecutive (one token tile: its x panel
// stays in that XCD's L2 while the block-rows stream past).
__device__ __forceinline__ int xcd_item(int items) {
  const int b = blockIdx.x;
  const int per_xcd = (items + kXcds - 1) / kXcds;
  return (b % kXcds) * per_xcd + b / kXcds;
}

// ---------------------------------------------------------------------------
// Row kernel: one workgroup per (token tile, group of G block-rows).
// ---------------------------------------------------------------------------
template <int DT, int P, int G, int MTW, int D>
__global__ __launch_bounds__(kPfThreads, 2) void pf_rows_kernel(PfArgs by_value) {
  (void)by_value;
  const PfArgs& a = *(const PfArgs*)__builtin_amdgcn_kernarg_segment_ptr();
  using Gm = Geo<DT, P, G, MTW>;
  constexpr int BM = 64 * MTW, W = Gm::W, KP = Gm::KP, EB = 2;
  __shared__ __align__(16) uint16_t sb[2][G * P * KP];

  const int item = xcd_item(a.items);
  if (item >= a.items) return;
  int i = 0;
  while (i + 1 < a.n && item >= a.off[i + 1]) ++i;
  const PfMember& mb = a.mb[i];
  const int local = item - a.off[i];
  const int tt = local / mb.n_groups, grp = local % mb.n_groups;
  const int m0 = tt * BM;
  const int32_t* gr = mb.groups + (int64_t)grp * (2 + G);
  const int e0 = gr[0], e1 = gr[1];
  int rowmask = 0;
#pragma unroll
  for (int g = 0; g < G; ++g) rowmask |= (gr[2 + g] >= 0) << g;
  const int nsp = e1 - e0;
  const int nlr = (a.mode == PF_FUSED) ? mb.r_pad / P : 0;
  const int U = nsp + nlr;
  const auto vr = mk_rsrc(mb.values_pq, mb.values_bytes);
  const auto ar = mk_rsrc(mb.A, mb.A_bytes);

  auto unit = [&](int u) {
    Unit<G> s;
    if (u < nsp) {
      const int32_t* e = mb.entries + (int64_t)(e0 + u) * (2 + G);
      s.a = (const uint16_t*)a.x; s.lda = a.ldx; s.ka = e[0] * P; s.kmax = a.m;
      s.kread = (int)a.ldx - Gm::KE;
      s.br = vr; s.bld = P * EB; s.mask = e[1];
#pragma unroll
      for (int g = 0; g < G; ++g)
        s.base[g] = e[2 + g] >= 0 ? (uint32_t)e[2 + g] * (uint32_t)(P * P * EB) : kOob;
    } else {
      const int k0 = (u - nsp) * P;
      s.a = (const uint16_t*)mb.t; s.lda = mb.ldt; s.ka = k0; s.kmax = 1 << 30;
      s.kread = (int)mb.ldt - Gm::KE;
      s.br = ar; s.bld = (uint32_t)(mb.lda * EB); s.mask = rowmask;
#pragma unroll
      for (int g = 0; g < G; ++g)
        s.base[g] = gr[2 + g] >= 0
                        ? (uint32_t)(((int64_t)gr[2 + g] * P * mb.lda + k0) * EB)
                        : kOob;
    }
    return s;
  };

  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  f32x4 acc[G][MTW][W];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
      for (int s = 0; s < W; ++s) acc[g][mt][s] = f32x4{0.f, 0.f, 0.f, 0.f};

  run_units<DT, P, G, MTW, D>(unit, U, m0, a.M, sb[0], sb[1], wid, lane, acc);

  // epilogue: lane (c, gq) owns W adjacent columns of rows 16·mt + 4gq + e
  const int c = lane & 15, gq = lane >> 4;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int row = gr[2 + g];
    if (row < 0) continue;
    const int j0 = row * P + W * c;
    float bv[W];
#pragma unroll
    for (int s = 0; s < W; ++s) bv[s] = 0.f;
    if (a.mode == PF_FUSED && mb.bias != nullptr) ld_w<DT, W>(mb.bias, j0, bv);
#pragma unroll
    for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = m0 + wid * 16 * MTW + mt * 16 + 4 * gq + e;
        if (r < a.M) {
          const int64_t off = (int64_t)r * mb.ldy + j0;
          float o[W];
          if (a.mode == PF_FUSED) {
#pragma unroll
            for (int s = 0; s < W; ++s) o[s] = acc[g][mt][s][e] + bv[s];
          } else {
            ld_w<DT, W>(mb.y, off, o);
#pragma unroll
            for (int s = 0; s < W; ++s) o[s] += acc[g][mt][s][e];
          }
          st_w<DT, W>(mb.y, off, o);
        }
      }
  }
}

// ---------------------------------------------------------------------------
// Latent kernel: one workgroup per (64-row token tile, 64-rank tile, K split).
// Writes the rounded latent when there is one split, else fp32 partials that
// pf_latent_combine sums in split order. Rows past M come from row M − 1.
// ---------------------------------------------------------------------------
template <int DT, int D>
__global__ __launch_bounds__(kPfThreads) void pf_latent_kernel(PfArgs by_value) {
  (void)by_value;
  const PfArgs& a = *(const PfArgs*)__builtin_amdgcn_kernarg_segment_ptr();
  constexpr int P = 64, G = 1, MTW = 1, BM = 64, EB = 2;
  using Gm = Geo<DT, P, G, MTW>;
  constexpr int W = Gm::W, KP = Gm::KP;
  __shared__ __align__(16) uint16_t sb[2][G * P * KP];

  const int b = blockIdx.x;
  int i = 0;
  while (i + 1 < a.n && b >= a.off[i + 1]) ++i;
  const PfMember& mb = a.mb[i];
  const int n_rt = mb.r_pad / P;
  const int local = b - a.off[i];
  const int ks = local % mb.ksplit, tile = local / mb.ksplit;
  const int tt = tile / n_rt, rt = tile % n_rt;
  const int m0 = tt * BM;
  const int units = a.m_pad / P;
  const int ku = (units + mb.ksplit - 1) / mb.ksplit;
  const int ub = ks * ku, ue = min(ub + ku, units);
  const auto br = mk_rsrc(mb.B, (int64_t)mb.r_pad * mb.ldb * EB);

  auto unit = [&](int u) {
    Unit<G> s;
    const int k0 = (ub + u) * P;
    s.a = (const uint16_t*)a.x; s.lda = a.ldx; s.ka = k0; s.kmax = a.m;
    s.kread = (int)a.ldx - Gm::KE;
    s.br = br; s.bld = (uint32_t)(mb.ldb * EB); s.mask = 1;
    s.base[0] = (uint32_t)(((int64_t)rt * P * mb.ldb + k0) * EB);
    return s;
  };
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  f32x4 acc[G][MTW][W];
#pragma unroll
  for (int s = 0; s < W; ++s) acc[0][0][s] = f32x4{0.f, 0.f, 0.f, 0.f};
  run_units<DT, P, G, MTW, D>(unit, ue - ub, m0, a.M, sb[0], sb[1], wid, lane, acc);

  // rows m0 + 16·wid + 4gq + e, ranks rt·64 + W·c + s
  const int c = lane & 15, gq = lane >> 4;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int r = m0 + wid * 16 + 4 * gq + e;
    float o[W];
#pragma unroll
    for (int s = 0; s < W; ++s) o[s] = acc[0][0][s][e];
    const int64_t idx = (int64_t)r * mb.ldt + rt * P + W * c;
    if (mb.ksplit == 1) {
      st_w<DT, W>(mb.t, idx, o);
    } else {
      float* pp = mb.tpart + (int64_t)ks * a.rows * mb.ldt + idx;
      *(float4*)pp = make_float4(o[0], o[1], o[2], o[3]);
    }
  }
}

// t = Σ_splits partials in split order, rounded once to the activation dtype.
template <int DT>
__global__ __launch_bounds__(kPfThreads) void pf_latent_combine(PfArgs by_value) {
  (void)by_value;
  const PfArgs& a = *(const PfArgs*)__builtin_amdgcn_kernarg_segment_ptr();
  const int b = blockIdx.x;
  int i = 0;
  while (i + 1 < a.n && b >= a.off[i + 1]) ++i;
  const PfMember& mb = a.mb[i];
  const int64_t q = (int64_t)(b - a.off[i]) * kPfThreads + threadIdx.x;  // 4-element piece
  const int64_t n = (int64_t)a.rows * mb.ldt / 4;
  if (q >= n) return;
  const int64_t slab = (int64_t)a.rows * mb.ldt;
  float4 v = *(const float4*)(mb.tpart + 4 * q);
  for (int k = 1; k < mb.ksplit; ++k) {
    const float4 w = *(const float4*)(mb.tpart + k * slab + 4 * q);
    v.x += w.x; v.y += w.y; v.z += w.z; v.w += w.w;
  }
  const float o[4] = {v.x, v.y, v.z, v.w};
  st_w<DT, 4>(mb.t, 4 * q, o);
}

// Two configurations per block size, both two waves per SIMD (≤ 256 registers):
//   wide:   128 token rows × G = 256/p block-rows (x tiles shared by G rows)
//   narrow: 64 token rows × 1 block-row (more workgroups for smaller calls)
template <int DT, int P>
hipError_t launch_rows(const PfArgs& a, int G, int bm, hipStream_t s) {
  constexpr int GM = 256 / P;
  const int per_xcd = (a.items + kXcds - 1) / kXcds;
  const dim3 grid((unsigned)(per_xcd * kXcds)), blk(kPfThreads);
  constexpr int D = P == 64 ? 2 : 3;
  if (G == GM && bm == 128) hipLaunchKernelGGL((pf_rows_kernel<DT, P, GM, 2, D>), grid, blk, 0, s, a);
  else if (G == 1 && bm == 64) hipLaunchKernelGGL((pf_rows_kernel<DT, P, 1, 1, 8>), grid, blk, 0, s, a);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

template <int DT>
hipError_t launch_rows_p(const PfArgs& rows, int P, int G, hipStream_t s) {
  if (rows.items == 0) return hipSuccess;
  const int bm = prefill_row_tile(G);
  switch (P) {
    case 16: return launch_rows<DT, 16>(rows, G, bm, s);
    case 32: return launch_rows<DT, 32>(rows, G, bm, s);
    case 64: return launch_rows<DT, 64>(rows, G, bm, s);
  }
  return hipErrorInvalidValue;
}

template <int DT>
hipError_t launch_fused(const PfArgs& rows, const PfArgs& lat, const PfArgs& comb, int P, int G,
                        hipStream_t s) {
  if (lat.items > 0) {
    hipLaunchKernelGGL((pf_latent_kernel<DT, 4>), dim3((unsigned)lat.items), dim3(kPfThreads), 0, s,
                       lat);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (comb.combine_items > 0) {
      hipLaunchKernelGGL((pf_latent_combine<DT>), dim3((unsigned)comb.combine_items),
                         dim3(kPfThreads), 0, s, comb);
      e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
  }
  return launch_rows_p<DT>(rows, P, G, s);
}

}  // namespace

int prefill_row_tile(int group) { return group > 1 ? 128 : 64; }

int prefill_group(int64_t M, int64_t n_rows, int block_p, int n_cus) {
  // the wide configuration when it still gives every CU a workgroup
  const int gmax = 256 / block_p;
  const int64_t forced = debug_knobs().prefill_group;  // test hook
  if (forced == 1) return 1;
  if (forced == 2) return gmax;
  const int64_t items = ((M + 127) / 128) * ((n_rows + gmax - 1) / gmax);
  return items >= n_cus ? gmax : 1;
}

int prefill_latent_split(int64_t M, int64_t r_pad, int64_t m_pad, int n_cus) {
  const int64_t tiles = ((M + 63) / 64) * (r_pad / 64);
  if (tiles <= 0) return 1;
  int64_t ks = (2 * n_cus) / tiles;
  const int64_t units = m_pad / 64;
  if (ks > units / 4) ks = units / 4;
  if (ks > 16) ks = 16;
  return ks < 1 ? 1 : (int)ks;
}

hipError_t prefill_launch_fused(int dtype, int P, int G, const PfArgs& rows, const PfArgs& lat,
                                const PfArgs& comb, hipStream_t stream) {
  switch (dtype) {
    case SSL_BF16: return launch_fused<DT_BF16>(rows, lat, comb, P, G, stream);
    case SSL_F16: return launch_fused<DT_F16>(rows, lat, comb, P, G, stream);
  }
  return hipErrorInvalidValue;
}

hipError_t prefill_launch_op(int dtype, int P, int G, const PfArgs& rows, hipStream_t stream) {
  switch (dtype) {
    case SSL_BF16: return launch_rows_p<DT_BF16>(rows, P, G, stream);
    case SSL_F16: return launch_rows_p<DT_F16>(rows, P, G, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace ssl
