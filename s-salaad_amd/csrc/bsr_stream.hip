// Streaming SLR / BSR kernels for gfx950.
//
// One workgroup (4 waves) executes one chunk of a work plan (plan.cpp): a
// consecutive range of the units of one block-row — sparse (q, p) blocks and,
// for the fused linear, 32-rank slices of A — for a tile of 16·MT token rows.
// The four waves take the chunk's units round-robin and stream each unit's
// weights from HBM straight into registers (no LDS staging: every weight byte
// is used exactly once per token tile), feeding v_mfma_f32_16x16x{32,16,4}.
// Partial tiles are reduced across the waves in LDS; a block-row split over
// several chunks is combined through a per-row arrival counter: each chunk
// writes its fp32 partial, and the last chunk to arrive sums all partials in
// chunk order (deterministic) and runs the epilogue.
//
// The low-rank latent t = x·Bᵀ is produced by lr_latent_kernel with the same
// machinery (chunks over the in_features dimension, combined per 64-rank group).

#include "abi_internal.h"
#include "slr_common.h"

namespace ssl {

// ---------------------------------------------------------------------------
// W-wide fp32 vectors in memory (partials) and in the output dtype (epilogue).
// ---------------------------------------------------------------------------
template <int W>
__device__ __forceinline__ void st_f32(float* p, const float (&v)[W]) {
  if constexpr (W == 4) *(float4*)p = make_float4(v[0], v[1], v[2], v[3]);
  else if constexpr (W == 2) *(float2*)p = make_float2(v[0], v[1]);
  else p[0] = v[0];
}
template <int W>
__device__ __forceinline__ void ld_f32(const float* p, float (&v)[W]) {
  if constexpr (W == 4) {
    float4 t = *(const float4*)p;
    v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
  } else if constexpr (W == 2) {
    float2 t = *(const float2*)p;
    v[0] = t.x; v[1] = t.y;
  } else {
    v[0] = p[0];
  }
}
template <int DT, int W>
__device__ __forceinline__ void st_elems(void* base, int64_t off, const float (&v)[W]) {
  if constexpr (DT == DT_F32) {
    st_f32<W>((float*)base + off, v);
  } else {
    uint16_t* p = (uint16_t*)base + off;
    if constexpr (W == 4) {
      uint2 u;
      u.x = to_bits<DT>(v[0]) | (to_bits<DT>(v[1]) << 16);
      u.y = to_bits<DT>(v[2]) | (to_bits<DT>(v[3]) << 16);
      *(uint2*)p = u;
    } else if constexpr (W == 2) {
      *(uint32_t*)p = to_bits<DT>(v[0]) | (to_bits<DT>(v[1]) << 16);
    } else {
      p[0] = (uint16_t)to_bits<DT>(v[0]);
    }
  }
}
template <int DT, int W>
__device__ __forceinline__ void ld_elems(const void* base, int64_t off, float (&v)[W]) {
  if constexpr (DT == DT_F32) {
    ld_f32<W>((const float*)base + off, v);
  } else {
    const uint16_t* p = (const uint16_t*)base + off;
    uint32_t w[(W + 1) / 2];
    if constexpr (W == 4) {
      uint2 u = *(const uint2*)p;
      w[0] = u.x; w[1] = u.y;
    } else if constexpr (W == 2) {
      w[0] = *(const uint32_t*)p;
    } else {
      w[0] = p[0];
    }
#pragma unroll
    for (int s = 0; s < W; ++s) {
      uint32_t h = (w[s >> 1] >> (16 * (s & 1))) & 0xffffu;
      v[s] = (DT == DT_BF16) ? bf16_to_f32(h) : f16_to_f32(h);
    }
  }
}

// ---------------------------------------------------------------------------
// Combine the workgroup's tile with the other chunks of the same row and run
// the epilogue once. Called by wave 0 only; `acc` is the workgroup total.
//   part_base : partial slot 0 of this row (slots seq = 0..nseq-1 follow)
//   counter   : arrival counter of this row (zero on entry, zero on exit)
// ---------------------------------------------------------------------------
template <int MT, int W, typename Store>
__device__ __forceinline__ void finish_tile(f32x4 (&acc)[MT][W], int nseq, int seq,
                                            float* part_base, int* counter, int Mrem, int lane,
                                            Store&& store) {
  constexpr int TP = 16 * W;
  constexpr int TSZ = MT * 16 * TP;
  if (nseq == 1) {
    store(acc);
    return;
  }
  const int c = lane & 15, g = lane >> 4;
  float* mine = part_base + (int64_t)seq * TSZ;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int rr = mt * 16 + 4 * g + e;
      if (rr < Mrem) {
        float v[W];
#pragma unroll
        for (int s = 0; s < W; ++s) v[s] = acc[mt][s][e];
        st_f32<W>(mine + rr * TP + W * c, v);
      }
    }
  fence_agent();
  int old = 0;
  if (lane == 0) old = atomic_inc_agent(counter);
  old = __builtin_amdgcn_readfirstlane(old);
  if (old != nseq - 1) return;
  fence_agent();
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
      const float* pk = part_base + (int64_t)k * TSZ;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int rr = mt * 16 + 4 * g + e;
          if (rr < Mrem) {
            float v[W];
            ld_f32<W>(pk + rr * TP + W * c, v);
#pragma unroll
            for (int s = 0; s < W; ++s) tot[mt][s][e] += v[s];
          }
        }
    }
  }
  if (lane == 0) atomic_store_agent(counter, 0);
  store(tot);
}

// Sum the four waves' tiles into wave 0 (fixed order). Returns false for waves 1..3.
template <int MT, int W>
__device__ __forceinline__ bool reduce_waves(f32x4 (&acc)[MT][W], int wid, int lane) {
  __shared__ f32x4 red[kWaves - 1][MT][W][kWave];
  if (wid > 0) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int s = 0; s < W; ++s) red[wid - 1][mt][s][lane] = acc[mt][s];
  }
  __syncthreads();
  if (wid != 0) return false;
#pragma unroll
  for (int w2 = 0; w2 < kWaves - 1; ++w2)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int s = 0; s < W; ++s) acc[mt][s] += red[w2][mt][s][lane];
  return true;
}

// ---------------------------------------------------------------------------
// Main streaming kernel.
//   FUSED = false : out[:, row tile] += Σ blocks           (in-place BSR addmm)
//   FUSED = true  : y[:, row tile]    = Σ blocks + t·Aᵀ + b (fused SLR linear)
// ---------------------------------------------------------------------------
struct StreamArgs {
  void* y;
  int64_t ldy;
  const void* x;
  int64_t ldx;
  const int32_t* col;
  const void* values;
  const int32_t* plan;
  const void* A;
  int64_t lda;
  const void* t;
  int64_t ldt;
  const void* bias;
  float* partials;
  int* counters;
  int64_t n_slots;
  int NB, M, m;
};

template <int DT, int P, int MT, bool FUSED, int UNR>
__global__ __launch_bounds__(kThreads) void bsr_stream_kernel(StreamArgs a) {
  constexpr int Q = P;
  constexpr int W = P / 16;
  constexpr int KE = (DT == DT_F32) ? 4 : (Q >= 32 ? 8 : 4);
  using MM = Mma<DT, KE>;
  using Frag = typename MM::Frag;
  constexpr int KM = MM::KM;
  constexpr int NKS = Q / KM;
  using Raw = VRawT<DT, KE, W>;
  constexpr int KEL = (DT == DT_F32) ? 4 : 8;  // low-rank part: widest fragment
  using ML = Mma<DT, KEL>;
  using FragL = typename ML::Frag;
  constexpr int NLS = 32 / ML::KM;  // macro steps per 32-rank unit
  constexpr int EB = Elem<DT>::bytes;

  const int lane = threadIdx.x & (kWave - 1);
  const int wid = wave_uniform(threadIdx.x >> 6);
  const int c = lane & 15, g = lane >> 4;
  const int32_t* d = a.plan + (int64_t)blockIdx.x * SSL_PLAN_STRIDE;
  const int row = d[0], ubeg = d[1], uend = d[2], seq = d[3], nseq = d[4], slot = d[5];
  const int nblk = d[6], blk0 = d[7];
  const int mg = blockIdx.y;
  const int m0 = mg * MT * 16;
  const int Mrem = min(a.M - m0, MT * 16);

  f32x4 acc[MT][W];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int s = 0; s < W; ++s) acc[mt][s] = f32x4{0.f, 0.f, 0.f, 0.f};

  // ---- sparse blocks ------------------------------------------------------
  const int se = min(uend, nblk);
  for (int u0 = ubeg + wid; u0 < se; u0 += kWaves * UNR) {
    Raw raw[UNR][NKS];
    int colb[UNR];
#pragma unroll
    for (int k = 0; k < UNR; ++k) {
      const int u = u0 + k * kWaves;
      colb[k] = 0;
      if (u < se) {
        const int blk = blk0 + u;
        colb[k] = a.col[blk] * Q;
        const char* vb = (const char*)a.values + (int64_t)blk * (P * Q * EB);
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) load_vstep<DT, KE, W>(raw[k][ks], vb, P, ks * KM, lane);
      }
    }
#pragma unroll
    for (int k = 0; k < UNR; ++k) {
      const int u = u0 + k * kWaves;
      if (u < se) {
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
          const int kcol = colb[k] + ks * KM + KE * g;
          Frag xf[MT];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const int rr = mt * 16 + c;
            int valid = (rr < Mrem) ? min(KE, a.m - kcol) : 0;
            xf[mt] = (valid > 0) ? load_kfrag<DT, KE>(a.x, (int64_t)(m0 + rr) * a.ldx + kcol, valid)
                                 : zero_frag<DT, KE>();
          }
#pragma unroll
          for (int s = 0; s < W; ++s) {
            const Frag vf = vfrag<DT, KE, W>(raw[k][ks], s);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) MM::run(acc[mt][s], xf[mt], vf);
          }
        }
      }
    }
  }

  // ---- low-rank units: 32 ranks of A per unit, t·Aᵀ -------------------------
  if constexpr (FUSED) {
    const int lb = max(ubeg, nblk);
    for (int u = lb + wid; u < uend; u += kWaves) {
      const int r0 = (u - nblk) * 32;
#pragma unroll
      for (int ls = 0; ls < NLS; ++ls) {
        const int kr = r0 + ls * ML::KM + KEL * g;
        FragL af[W];
#pragma unroll
        for (int s = 0; s < W; ++s)
          af[s] = load_kfrag<DT, KEL>(a.A, (int64_t)(row * P + W * c + s) * a.lda + kr, KEL);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int rr = mt * 16 + c;
          const FragL tf = (rr < Mrem)
                               ? load_kfrag<DT, KEL>(a.t, (int64_t)(m0 + rr) * a.ldt + kr, KEL)
                               : zero_frag<DT, KEL>();
#pragma unroll
          for (int s = 0; s < W; ++s) ML::run(acc[mt][s], tf, af[s]);
        }
      }
    }
  }

  if (!reduce_waves<MT, W>(acc, wid, lane)) return;

  auto store = [&](f32x4(&v)[MT][W]) {
    const int j0 = row * P + W * c;
    float bv[W];
#pragma unroll
    for (int s = 0; s < W; ++s) bv[s] = 0.f;
    if constexpr (FUSED) {
      if (a.bias != nullptr) {
#pragma unroll
        for (int s = 0; s < W; ++s) bv[s] = load_scalar<DT>(a.bias, j0 + s);
      }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int rr = mt * 16 + 4 * g + e;
        if (rr < Mrem) {
          const int64_t off = (int64_t)(m0 + rr) * a.ldy + j0;
          float o[W];
          if constexpr (FUSED) {
#pragma unroll
            for (int s = 0; s < W; ++s) o[s] = v[mt][s][e] + bv[s];
          } else {
            ld_elems<DT, W>(a.y, off, o);
#pragma unroll
            for (int s = 0; s < W; ++s) o[s] += v[mt][s][e];
          }
          st_elems<DT, W>(a.y, off, o);
        }
      }
  };
  constexpr int TSZ = MT * 16 * P;
  finish_tile<MT, W>(acc, nseq, seq, a.partials + ((int64_t)mg * a.n_slots + slot) * TSZ,
                     a.counters + (int64_t)mg * a.NB + row, Mrem, lane, store);
}

// ---------------------------------------------------------------------------
// Latent kernel: t[M, r_pad] = x[M, :m] · B[r_pad, :m_pad]ᵀ, rounded to the
// activation dtype. Workgroup = (64-rank group, chunk of in_features).
// ---------------------------------------------------------------------------
struct LatentArgs {
  void* t;
  int64_t ldt;
  const void* x;
  int64_t ldx;
  const void* B;
  int64_t ldb;
  float* partials;
  int* counters;
  int n_rg, n_kc, ku_total, ku_chunk;
  int M, m;
};

template <int DT, int MT, int UNR>
__global__ __launch_bounds__(kThreads) void lr_latent_kernel(LatentArgs a) {
  constexpr int KE = (DT == DT_F32) ? 4 : 8;
  using MM = Mma<DT, KE>;
  using Frag = typename MM::Frag;
  constexpr int KM = MM::KM;
  constexpr int W = 4;

  const int lane = threadIdx.x & (kWave - 1);
  const int wid = wave_uniform(threadIdx.x >> 6);
  const int c = lane & 15, g = lane >> 4;
  const int rg = blockIdx.x / a.n_kc, kc = blockIdx.x % a.n_kc;
  const int mg = blockIdx.y;
  const int m0 = mg * MT * 16;
  const int Mrem = min(a.M - m0, MT * 16);
  const int ub = kc * a.ku_chunk, ue = min(ub + a.ku_chunk, a.ku_total);

  f32x4 acc[MT][W];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int s = 0; s < W; ++s) acc[mt][s] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int u0 = ub + wid; u0 < ue; u0 += kWaves * UNR) {
    Frag bf[UNR][W];
#pragma unroll
    for (int k = 0; k < UNR; ++k) {
      const int u = u0 + k * kWaves;
      if (u < ue) {
#pragma unroll
        for (int s = 0; s < W; ++s)
          bf[k][s] = load_kfrag<DT, KE>(a.B, (int64_t)(rg * 64 + W * c + s) * a.ldb + u * KM + KE * g, KE);
      }
    }
#pragma unroll
    for (int k = 0; k < UNR; ++k) {
      const int u = u0 + k * kWaves;
      if (u < ue) {
        const int kcol = u * KM + KE * g;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int rr = mt * 16 + c;
          int valid = (rr < Mrem) ? min(KE, a.m - kcol) : 0;
          const Frag xf = (valid > 0)
                              ? load_kfrag<DT, KE>(a.x, (int64_t)(m0 + rr) * a.ldx + kcol, valid)
                              : zero_frag<DT, KE>();
#pragma unroll
          for (int s = 0; s < W; ++s) MM::run(acc[mt][s], xf, bf[k][s]);
        }
      }
    }
  }

  if (!reduce_waves<MT, W>(acc, wid, lane)) return;

  auto store = [&](f32x4(&v)[MT][W]) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int rr = mt * 16 + 4 * g + e;
        if (rr < Mrem) {
          float o[W];
#pragma unroll
          for (int s = 0; s < W; ++s) o[s] = v[mt][s][e];
          st_elems<DT, W>(a.t, (int64_t)(m0 + rr) * a.ldt + rg * 64 + W * c, o);
        }
      }
  };
  constexpr int TSZ = MT * 16 * 64;
  finish_tile<MT, W>(acc, a.n_kc, kc,
                     a.partials + ((int64_t)mg * a.n_rg + rg) * a.n_kc * TSZ,
                     a.counters + (int64_t)mg * a.n_rg + rg, Mrem, lane, store);
}

// ---------------------------------------------------------------------------
// Host-side launch plumbing
// ---------------------------------------------------------------------------
namespace {

template <int DT, int P>
constexpr int stream_unroll() {
  // Keep roughly 8–16 KiB of one wave's weight loads in flight.
  constexpr int bytes = P * P * Elem<DT>::bytes;
  return bytes >= 16384 ? 1 : (bytes >= 8192 ? 2 : (bytes >= 2048 ? 4 : 8));
}

template <int DT, int P, int MT, bool FUSED>
hipError_t launch_stream(const StreamArgs& a, int64_t n_chunks, int MG, hipStream_t s) {
  constexpr int UNR = stream_unroll<DT, P>();
  hipLaunchKernelGGL((bsr_stream_kernel<DT, P, MT, FUSED, UNR>), dim3((unsigned)n_chunks, MG),
                     dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

template <int DT, bool FUSED>
hipError_t dispatch_stream(int P, int MT, const StreamArgs& a, int64_t n_chunks, int MG,
                           hipStream_t s) {
#define SSL_CASE(PP, MM)                                                  \
  if (P == PP && MT == MM) return launch_stream<DT, PP, MM, FUSED>(a, n_chunks, MG, s);
  SSL_CASE(16, 1) SSL_CASE(16, 2) SSL_CASE(16, 4)
  SSL_CASE(32, 1) SSL_CASE(32, 2) SSL_CASE(32, 4)
  SSL_CASE(64, 1) SSL_CASE(64, 2) SSL_CASE(64, 4)
#undef SSL_CASE
  return hipErrorInvalidValue;
}

template <bool FUSED>
hipError_t dispatch_stream_dt(int dtype, int P, int MT, const StreamArgs& a, int64_t n_chunks,
                              int MG, hipStream_t s) {
  switch (dtype) {
    case SSL_F32: return dispatch_stream<DT_F32, FUSED>(P, MT, a, n_chunks, MG, s);
    case SSL_BF16: return dispatch_stream<DT_BF16, FUSED>(P, MT, a, n_chunks, MG, s);
    case SSL_F16: return dispatch_stream<DT_F16, FUSED>(P, MT, a, n_chunks, MG, s);
  }
  return hipErrorInvalidValue;
}

template <int DT, int MT>
hipError_t launch_latent(const LatentArgs& a, int MG, hipStream_t s) {
  hipLaunchKernelGGL((lr_latent_kernel<DT, MT, 2>), dim3((unsigned)(a.n_rg * a.n_kc), MG),
                     dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t dispatch_latent(int dtype, int MT, const LatentArgs& a, int MG, hipStream_t s) {
#define SSL_CASE(DD, MM) \
  if (dtype == DD && MT == MM) return launch_latent<DD, MM>(a, MG, s);
  SSL_CASE(DT_F32, 1) SSL_CASE(DT_F32, 2) SSL_CASE(DT_F32, 4)
  SSL_CASE(DT_BF16, 1) SSL_CASE(DT_BF16, 2) SSL_CASE(DT_BF16, 4)
  SSL_CASE(DT_F16, 1) SSL_CASE(DT_F16, 2) SSL_CASE(DT_F16, 4)
#undef SSL_CASE
  return hipErrorInvalidValue;
}

bool supported_block(int p, int q) { return p == q && (p == 16 || p == 32 || p == 64); }
bool supported_dtype(int dt) { return dt == SSL_F32 || dt == SSL_BF16 || dt == SSL_F16; }

// Workspace layout of one call (offsets in bytes).
struct Layout {
  int MT, MG;
  int n_rg, n_kc, ku_total, ku_chunk;
  int64_t counters_main, counters_lat, counter_end;
  int64_t t_buf, part_lat, part_main, total;
};

Layout slr_layout(int64_t M, int64_t NB, int p, int64_t r_pad, int64_t m_pad, int64_t n_slots,
                  int dtype) {
  Layout L{};
  L.MT = tile_mt(M);
  L.MG = (int)((M + 16 * L.MT - 1) / (16 * L.MT));
  L.n_rg = (int)(r_pad / 64);
  const int KM = (dtype == SSL_F32) ? 16 : 32;
  L.ku_total = (int)(m_pad / KM);
  // One token tile: split in_features so the latent kernel covers the device;
  // several tiles already give enough workgroups.
  int chunk = L.ku_total;
  if (L.MG == 1) {
    chunk = (L.ku_total + 31) / 32;
    if (chunk < 4) chunk = 4;
    if (chunk > L.ku_total) chunk = L.ku_total;
  }
  if (chunk < 1) chunk = 1;
  L.ku_chunk = chunk;
  L.n_kc = L.ku_total > 0 ? (L.ku_total + chunk - 1) / chunk : 1;
  int64_t off = 0;
  L.counters_main = off;
  off = align_up(off + 4 * (int64_t)L.MG * NB, 256);
  L.counters_lat = off;
  off = align_up(off + 4 * (int64_t)L.MG * L.n_rg, 256);
  L.counter_end = off;
  L.t_buf = off;
  off = align_up(off + (int64_t)elem_bytes(dtype) * M * r_pad, 256);
  L.part_lat = off;
  if (L.n_kc > 1) off = align_up(off + 4 * (int64_t)L.MG * L.n_rg * L.n_kc * (16 * L.MT * 64), 256);
  L.part_main = off;
  off = align_up(off + 4 * (int64_t)L.MG * n_slots * (16 * L.MT * p), 256);
  L.total = off;
  return L;
}

}  // namespace
}  // namespace ssl

using namespace ssl;

extern "C" {

int64_t ssl_bsr_addmm_counter_bytes(int64_t M, int64_t NB) {
  const int MT = tile_mt(M);
  const int64_t MG = (M + 16 * MT - 1) / (16 * MT);
  return align_up(4 * MG * NB, 256);
}

int64_t ssl_bsr_addmm_workspace_size(int64_t M, int64_t NB, int32_t block_p, int64_t n_slots) {
  const int MT = tile_mt(M);
  const int64_t MG = (M + 16 * MT - 1) / (16 * MT);
  return ssl_bsr_addmm_counter_bytes(M, NB) + align_up(4 * MG * n_slots * (16 * MT * block_p), 256);
}

int ssl_bsr_addmm_inplace(void* out, int64_t ldo, const void* x, int64_t ldx, const int32_t* col,
                          const void* values, const int32_t* plan, int64_t n_chunks,
                          int64_t n_slots, int64_t M, int64_t N, int64_t K, int64_t NB,
                          int32_t block_p, int32_t block_q, int32_t dtype, void* workspace,
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
  if (n_chunks > 0x7fffffff) return fail(SSL_ERR_INVALID, "too many chunks");
  const int eb = elem_bytes(dtype);
  if (!out || !x || !col || !values || !plan) return fail(SSL_ERR_INVALID, "null pointer");
  if (ldx < K || ldo < N) return fail(SSL_ERR_INVALID, "leading dimension smaller than row");
  if (!aligned(x, 16) || (ldx * eb) % 16 || !aligned(values, 16))
    return fail(SSL_ERR_INVALID, "x rows and values must be 16-byte aligned");
  if (!aligned(out, 16) || (ldo * eb) % 16) return fail(SSL_ERR_INVALID, "out rows must be 16-byte aligned");
  const int64_t need = ssl_bsr_addmm_workspace_size(M, NB, block_p, n_slots);
  if (workspace_bytes < need || (need > 0 && !workspace))
    return fail(SSL_ERR_WORKSPACE, "workspace of %lld bytes needed", (long long)need);
  if (!aligned(workspace, 256)) return fail(SSL_ERR_WORKSPACE, "workspace must be 256-byte aligned");

  const int MT = tile_mt(M);
  const int MG = (int)((M + 16 * MT - 1) / (16 * MT));
  StreamArgs a{};
  a.y = out; a.ldy = ldo; a.x = x; a.ldx = ldx; a.col = col; a.values = values; a.plan = plan;
  a.counters = (int*)workspace;
  a.partials = (float*)((char*)workspace + ssl_bsr_addmm_counter_bytes(M, NB));
  a.n_slots = n_slots; a.NB = (int)NB; a.M = (int)M; a.m = (int)K;
  return check_hip(dispatch_stream_dt<false>(dtype, block_p, MT, a, n_chunks, MG, (hipStream_t)stream),
                   "bsr_addmm launch");
}

int64_t ssl_slr_counter_bytes(int64_t M, int64_t NB, int64_t r_pad, int64_t m_pad) {
  return slr_layout(M, NB, 16, r_pad, m_pad, 0, SSL_BF16).counter_end;
}

int64_t ssl_slr_workspace_size(int64_t M, int64_t NB, int32_t block_p, int64_t r_pad,
                               int64_t m_pad, int64_t n_slots, int32_t dtype) {
  return slr_layout(M, NB, block_p, r_pad, m_pad, n_slots, dtype).total;
}

int ssl_slr_forward_phase(void* y, int64_t ldy, const void* x, int64_t ldx, const void* A,
                          const void* B, const void* bias, const int32_t* col, const void* values,
                          const int32_t* plan, int64_t n_chunks, int64_t n_slots, int64_t M,
                          int64_t m, int64_t m_pad, int64_t NB, int64_t r_pad, int32_t block_p,
                          int32_t block_q, int32_t dtype, void* workspace, int64_t workspace_bytes,
                          int32_t phase, void* stream) {
  if (phase < 0 || phase > 2) return fail(SSL_ERR_INVALID, "phase must be 0, 1 or 2");
  clear_error();
  if (!supported_dtype(dtype)) return fail(SSL_ERR_UNSUPPORTED, "unsupported dtype %d", dtype);
  if (!supported_block(block_p, block_q))
    return fail(SSL_ERR_UNSUPPORTED,
                "SLR kernel needs square 16, 32 or 64 blocks, got %dx%d", block_p, block_q);
  if (M < 0 || m < 0 || NB < 0 || r_pad < 0 || n_chunks < 0 || n_slots < 0)
    return fail(SSL_ERR_INVALID, "negative size");
  if (r_pad % 64 || m_pad % 64 || m_pad < m)
    return fail(SSL_ERR_INVALID, "r_pad and m_pad must be multiples of 64 with m_pad >= m");
  if (M == 0 || NB == 0) return SSL_OK;
  if (n_chunks == 0) return fail(SSL_ERR_INVALID, "empty plan for a non-empty output");
  const int eb = elem_bytes(dtype);
  if (!y || !x || !plan || (r_pad > 0 && (!A || !B))) return fail(SSL_ERR_INVALID, "null pointer");
  if (ldx < m || ldy < NB * block_p) return fail(SSL_ERR_INVALID, "leading dimension smaller than row");
  if (!aligned(x, 16) || (ldx * eb) % 16) return fail(SSL_ERR_INVALID, "x rows must be 16-byte aligned");
  if (!aligned(y, 16) || (ldy * eb) % 16) return fail(SSL_ERR_INVALID, "y rows must be 16-byte aligned");
  if ((A && !aligned(A, 16)) || (B && !aligned(B, 16)) || (values && !aligned(values, 16)))
    return fail(SSL_ERR_INVALID, "A, B and values must be 16-byte aligned");
  const Layout L = slr_layout(M, NB, block_p, r_pad, m_pad, n_slots, dtype);
  if (workspace_bytes < L.total || !workspace)
    return fail(SSL_ERR_WORKSPACE, "workspace of %lld bytes needed", (long long)L.total);
  if (!aligned(workspace, 256)) return fail(SSL_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;

  if (r_pad > 0 && phase != 2) {
    LatentArgs la{};
    la.t = ws + L.t_buf; la.ldt = r_pad; la.x = x; la.ldx = ldx; la.B = B; la.ldb = m_pad;
    la.partials = (float*)(ws + L.part_lat); la.counters = (int*)(ws + L.counters_lat);
    la.n_rg = L.n_rg; la.n_kc = L.n_kc; la.ku_total = L.ku_total; la.ku_chunk = L.ku_chunk;
    la.M = (int)M; la.m = (int)m;
    int rc = check_hip(dispatch_latent(dtype, L.MT, la, L.MG, s), "latent launch");
    if (rc) return rc;
  }
  if (phase == 1) return SSL_OK;
  StreamArgs a{};
  a.y = y; a.ldy = ldy; a.x = x; a.ldx = ldx; a.col = col; a.values = values; a.plan = plan;
  a.A = A; a.lda = r_pad; a.t = ws + L.t_buf; a.ldt = r_pad; a.bias = bias;
  a.counters = (int*)(ws + L.counters_main); a.partials = (float*)(ws + L.part_main);
  a.n_slots = n_slots; a.NB = (int)NB; a.M = (int)M; a.m = (int)m;
  return check_hip(dispatch_stream_dt<true>(dtype, block_p, L.MT, a, n_chunks, L.MG, s),
                   "slr launch");
}

int ssl_slr_forward(void* y, int64_t ldy, const void* x, int64_t ldx, const void* A, const void* B,
                    const void* bias, const int32_t* col, const void* values, const int32_t* plan,
                    int64_t n_chunks, int64_t n_slots, int64_t M, int64_t m, int64_t m_pad,
                    int64_t NB, int64_t r_pad, int32_t block_p, int32_t block_q, int32_t dtype,
                    void* workspace, int64_t workspace_bytes, void* stream) {
  return ssl_slr_forward_phase(y, ldy, x, ldx, A, B, bias, col, values, plan, n_chunks, n_slots, M,
                               m, m_pad, NB, r_pad, block_p, block_q, dtype, workspace,
                               workspace_bytes, 0, stream);
}

}  // extern "C"
