// Decode-step kernels around the SLR linears of a LLaMA / Qwen3 decoder layer:
// one new token per sequence, keys and values kept in a per-layer cache.
//
//   add_rmsnorm   h += delta (rounded to the model dtype), out = w · norm(h);
//                 or h = embed[token] first (the layer-0 input)
//   rope_kv       q/k rotary embedding (after Qwen3's per-head RMSNorm), k and v
//                 written into the cache at the sequence's position
//   attn_split    softmax(q·Kᵀ·scale)·V over one slice of a sequence's context,
//                 per wave an online softmax, the slice's partial (max, sum, o);
//                 the last slice to finish merges all of them into the output
//   silu_mul      silu(gate) · up
//
// Rounding points follow transformers' LlamaRMSNorm / apply_rotary_pos_emb /
// LlamaMLP (transformers 5.15.0, models/llama/modeling_llama.py): every torch
// operation on a 16-bit tensor rounds its fp32 result to the tensor's dtype.
// The attention itself accumulates in fp32 and rounds once at the output.
//
// Caches are [slots, kv_heads, max_ctx, head_dim] per layer; batch row b uses
// slot b. All loads of keys and values are 16-byte vectors, one row of a head
// spread over head_dim·elem/16 lanes, so a wave reads whole rows contiguously.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <algorithm>

#include "abi_internal.h"
#include "slr_common.h"

namespace ssl {
namespace {

template <int DT>
__device__ __forceinline__ float rnd(float f) {
  if constexpr (DT == DT_F32) return f;
  else if constexpr (DT == DT_BF16) return bf16_to_f32(f32_to_bf16(f));
  else return f16_to_f32(f32_to_f16(f));
}

template <int DT>
__device__ __forceinline__ void store_scalar(void* p, int64_t i, float f) {
  if constexpr (DT == DT_F32) ((float*)p)[i] = f;
  else ((uint16_t*)p)[i] = (uint16_t)to_bits<DT>(f);
}

// Device-coherent (agent scope) accesses for the attention slices' partials.
__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The same device-coherent read as a plain buffer load (cache policy sc1), so
// that many of them can be in flight at once; `r` spans the partials.
constexpr int kSc1Policy = 16;
__device__ __forceinline__ float ld_sc1(__amdgpu_buffer_rsrc_t r, int64_t idx) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)(idx * 4), 0, kSc1Policy));
}

constexpr int kMaxSplits = 256;

__device__ __forceinline__ float wave_sum(float v) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// ---------------------------------------------------------------------------
// add_rmsnorm: one workgroup per row, K elements per thread (hidden <= 256·K)
// held in registers, so every load of the row is issued before the first use.
// With `tokens` the row is first gathered from the embedding table (h =
// embed[token]; a token outside [0, vocab) gives a zero row).
// ---------------------------------------------------------------------------
template <int DT, int K>
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(
    void* __restrict__ h, int64_t ldh, const void* __restrict__ delta, int64_t ldd,
    const void* __restrict__ w, void* __restrict__ out, int64_t ldo, int hidden, float eps,
    const void* __restrict__ embed, int64_t lde, const int64_t* __restrict__ tokens,
    int64_t vocab) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const void* src = h;
  int64_t srow = row * ldh;
  bool valid = true;
  if (tokens) {
    const int64_t t = tokens[row];
    valid = t >= 0 && t < vocab;
    src = embed;
    srow = valid ? t * lde : 0;
  }
  // Loads are unconditional (indices clamped into the row) and masked
  // afterwards: a load under a per-lane condition becomes a branch that waits
  // for it, which would serialise the row.
  float v[K], d[K], wv[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int i = min(tid + 256 * k, hidden - 1);
    v[k] = load_scalar<DT>(src, srow + i);
    wv[k] = load_scalar<DT>(w, i);
  }
  if (delta) {
#pragma unroll
    for (int k = 0; k < K; ++k) d[k] = load_scalar<DT>(delta, row * ldd + min(tid + 256 * k, hidden - 1));
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const bool in = tid + 256 * k < hidden;
    if (delta) v[k] = rnd<DT>(v[k] + d[k]);
    v[k] = (in && valid) ? v[k] : 0.f;
    ss += v[k] * v[k];
  }
  if (delta || tokens) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int i = tid + 256 * k;
      if (i < hidden) store_scalar<DT>(h, row * ldh + i, v[k]);
    }
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  const float tot = red[0] + red[1] + red[2] + red[3];
  const float rs = rsqrtf(tot / (float)hidden + eps);
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int i = tid + 256 * k;
    if (i < hidden) store_scalar<DT>(out, row * ldo + i, wv[k] * rnd<DT>(v[k] * rs));
  }
}

// ---------------------------------------------------------------------------
// rope_kv: one wave per (row, head slot); slots [0, heads) are query heads,
// [heads, heads + kv_heads) key heads (whose value head is copied alongside).
// head_dim <= 256: a lane holds at most two rotary pairs (j, j + head_dim/2).
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(64) void rope_kv_kernel(
    const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv,
    const void* cos_t, const void* sin_t, const void* q_norm, const void* k_norm, float eps,
    const int32_t* pos, void* q_out, void* k_cache, void* v_cache, int heads, int kv_heads, int hd,
    int64_t max_ctx) {
  // torch rounds q·cos and rotate_half(q)·sin separately before the sum
#pragma clang fp contract(off)
  const int slot = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int lane = threadIdx.x;
  const int64_t p = pos[b];
  if (p < 0 || p >= max_ctx) return;  // the host rejects such positions before launching
  const bool is_q = slot < heads;
  const int kh = slot - heads;
  const void* src = is_q ? q : k;
  const int64_t soff = is_q ? b * ldq + (int64_t)slot * hd : b * ldk + (int64_t)kh * hd;
  void* dst = is_q ? q_out : k_cache;
  const int64_t doff = is_q ? (b * heads + slot) * hd : ((b * kv_heads + kh) * max_ctx + p) * hd;
  const void* nw = is_q ? q_norm : k_norm;
  const int half = hd >> 1;

  float x1[2], x2[2], c1[2], s1[2], c2[2], s2[2];
  float ss = 0.f;
#pragma unroll
  for (int u = 0; u < 2; ++u) {  // clamped, unconditional loads (see add_rmsnorm)
    const int j = min(lane + 64 * u, half - 1);
    x1[u] = load_scalar<DT>(src, soff + j);
    x2[u] = load_scalar<DT>(src, soff + j + half);
    c1[u] = load_scalar<DT>(cos_t, p * hd + j);
    s1[u] = load_scalar<DT>(sin_t, p * hd + j);
    c2[u] = load_scalar<DT>(cos_t, p * hd + j + half);
    s2[u] = load_scalar<DT>(sin_t, p * hd + j + half);
  }
#pragma unroll
  for (int u = 0; u < 2; ++u)
    if (lane + 64 * u < half) ss += x1[u] * x1[u] + x2[u] * x2[u];
  if (nw) {  // Qwen3: RMSNorm over the head's features before the rotation
    const float rs = rsqrtf(wave_sum(ss) / (float)hd + eps);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int j = min(lane + 64 * u, half - 1);
      x1[u] = rnd<DT>(load_scalar<DT>(nw, j) * rnd<DT>(x1[u] * rs));
      x2[u] = rnd<DT>(load_scalar<DT>(nw, j + half) * rnd<DT>(x2[u] * rs));
    }
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int j = lane + 64 * u;
    if (j < half) {  // rotate_half(x) = (-x2, x1)
      store_scalar<DT>(dst, doff + j, rnd<DT>(x1[u] * c1[u]) - rnd<DT>(x2[u] * s1[u]));
      store_scalar<DT>(dst, doff + j + half, rnd<DT>(x2[u] * c2[u]) + rnd<DT>(x1[u] * s2[u]));
    }
  }
  if (!is_q) {
    const int64_t vs = b * ldv + (int64_t)kh * hd;
    for (int j = lane; j < hd; j += 64)
      store_scalar<DT>(v_cache, doff + j, load_scalar<DT>(v, vs + j));
  }
}

// ---------------------------------------------------------------------------
// attn_split: workgroup (split, head block, row). A lane reads 16 bytes (VE
// elements) of a key/value row; LPR lanes cover a row and a wave instruction
// reads RPI whole rows. Each wave takes 4·RPI positions per step and keeps its
// own online softmax (max m, sum l, o) for the GB query heads that share one
// key/value head; the four waves are merged through LDS at the end.
// Scores are kept in base 2: s = q·k · scale · log2(e).
// ---------------------------------------------------------------------------
template <int DT>
struct Vec16 {
  static constexpr int VE = DT == DT_F32 ? 4 : 8;
  __device__ __forceinline__ static uint4 raw(const void* base, int64_t off) {
    return *(const uint4*)((const char*)base + off * Elem<DT>::bytes);
  }
  __device__ __forceinline__ static void load(float* f, const void* base, int64_t off) {
    unpack(f, raw(base, off));
  }
  __device__ __forceinline__ static void unpack(float* f, const uint4 raw) {
    if constexpr (DT == DT_F32) {
      f[0] = __uint_as_float(raw.x);
      f[1] = __uint_as_float(raw.y);
      f[2] = __uint_as_float(raw.z);
      f[3] = __uint_as_float(raw.w);
    } else {
      const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (DT == DT_BF16) {
          f[2 * i] = bf16_to_f32(w[i] & 0xffffu);
          f[2 * i + 1] = bf16_to_f32(w[i] >> 16);
        } else {
          f[2 * i] = f16_to_f32(w[i] & 0xffffu);
          f[2 * i + 1] = f16_to_f32(w[i] >> 16);
        }
      }
    }
  }
  // f holds values already rounded to DT
  __device__ __forceinline__ static uint4 pack(const float* f) {
    if constexpr (DT == DT_F32) {
      return uint4{__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]),
                   __float_as_uint(f[3])};
    } else {
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = to_bits<DT>(f[2 * i]) | (to_bits<DT>(f[2 * i + 1]) << 16);
      return uint4{w[0], w[1], w[2], w[3]};
    }
  }
};

// (a & mask) | (b & ~mask), dword by dword
__device__ __forceinline__ uint4 merge(uint32_t mask, const uint4 a, const uint4 b) {
  return uint4{(a.x & mask) | (b.x & ~mask), (a.y & mask) | (b.y & ~mask),
               (a.z & mask) | (b.z & ~mask), (a.w & mask) | (b.w & ~mask)};
}

// The q/k/v projections of the new token, for the attention launch that also
// applies the rotary embedding and appends the key and value to the cache.
struct RopeIn {
  const void* q;
  int64_t ldq;
  const void* k;
  int64_t ldk;
  const void* v;
  int64_t ldv;
  const void* cos_t;   // [max_ctx, head_dim]
  const void* sin_t;
  const void* q_norm;  // Qwen3's per-head RMSNorm weights, or null
  const void* k_norm;
  float eps;
  void* k_cache;       // the caches the launch reads, written at the new position
  void* v_cache;
};

// One head's rotary embedding in the attention layout (lane vv of a row group
// holds features vv·VE … vv·VE + VE − 1), with rope_kv_kernel's rounding
// points. The partner features (± head_dim / 2) are read from memory rather
// than exchanged between lanes (x: own, xp: partner; c, s: the tables at the
// own features; w, wp: the per-head RMSNorm weights when `norm`). Under the
// norm the sum of squares is reduced over the row group's LPR lanes. All
// operands are raw vectors, loaded by the caller before the first use.
template <int DT, int HD>
__device__ __forceinline__ void rope_apply(float* out, const uint4 xr, const uint4 xpr,
                                          const uint4 cr, const uint4 sr, bool norm,
                                          const uint4 wr, const uint4 wpr, float eps, int vv) {
#pragma clang fp contract(off)
  constexpr int VE = Vec16<DT>::VE;
  constexpr int LPR = HD / VE;
  const bool low = vv * VE < HD / 2;
  float x[VE], xp[VE], c[VE], s[VE];
  Vec16<DT>::unpack(x, xr);
  Vec16<DT>::unpack(xp, xpr);
  Vec16<DT>::unpack(c, cr);
  Vec16<DT>::unpack(s, sr);
  if (norm) {
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < VE; ++e) ss += x[e] * x[e];
#pragma unroll
    for (int off = 1; off < LPR; off <<= 1) ss += __shfl_xor(ss, off);
    const float rs = rsqrtf(ss / (float)HD + eps);
    float w[VE], wp[VE];
    Vec16<DT>::unpack(w, wr);
    Vec16<DT>::unpack(wp, wpr);
#pragma unroll
    for (int e = 0; e < VE; ++e) {
      x[e] = rnd<DT>(w[e] * rnd<DT>(x[e] * rs));
      xp[e] = rnd<DT>(wp[e] * rnd<DT>(xp[e] * rs));
    }
  }
#pragma unroll
  for (int e = 0; e < VE; ++e) {  // rotate_half(x) = (-x2, x1)
    const float a = rnd<DT>(x[e] * c[e]), bb = rnd<DT>(xp[e] * s[e]);
    out[e] = rnd<DT>(low ? a - bb : a + bb);
  }
}

constexpr int kAttnJ = 4;  // wave instructions (row groups) per step

// ROPE: 0 q read as given; 1 rotary embedding and cache append in the launch;
// 2 the same after Qwen3's per-head RMSNorm.
template <int DT, int HD, int GB, int ROPE>
__global__ __launch_bounds__(256, ROPE == 1 && GB == 1 ? 4 : 1) void attn_split_kernel(
    const void* q, const void* kc, const void* vc, const int32_t* pos, int64_t max_ctx, int heads,
    int kv_heads, int n_split, float scale_log2, float* part_o, float* part_ml, int* counters,
    void* out, int64_t ldo, RopeIn R) {
  constexpr int VE = Vec16<DT>::VE;
  constexpr int LPR = HD / VE;
  constexpr int RPI = 64 / LPR;
  constexpr int WSTEP = kAttnJ * RPI;  // positions per wave per step
  constexpr int STEP = 4 * WSTEP;      // positions per workgroup per step
  static_assert(LPR <= 64 && (LPR & (LPR - 1)) == 0, "head_dim must give a power-of-two lane count");
  __shared__ float sh_o[4][GB][HD];
  __shared__ float sh_m[4][GB];
  __shared__ float sh_l[4][GB];

  const int split = blockIdx.x;
  const int G = heads / kv_heads;
  const int n_hb = (G + GB - 1) / GB;
  const int kh = blockIdx.y / n_hb;
  const int g0 = (blockIdx.y % n_hb) * GB;
  const int ng = min(GB, G - g0);
  const int64_t b = blockIdx.z;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int rr = lane / LPR, vv = lane % LPR;

  const int64_t pcur = pos[b];
  const int64_t L = min(pcur + 1, max_ctx);
  int64_t per = (L + n_split - 1) / n_split;
  per = (per + STEP - 1) / STEP * STEP;
  const int64_t lo = (int64_t)split * per;
  const int64_t hi = min(lo + per, L);
  const int64_t head_off = (b * kv_heads + kh) * max_ctx * HD;

  float qf[GB][VE];
  uint4 kn = {0, 0, 0, 0}, vn = {0, 0, 0, 0};  // the new token's key (rotated) and value
  // Rotary embedding of the query heads and the new key. It runs in the first
  // step of the loop, after that step's key and value loads are issued, so the
  // projections' loads share their round trip.
  auto rope_prep = [&]() {
    // the host rejects positions outside [0, max_ctx); the clamp keeps table reads in bounds
    const int64_t pt = min(max(pcur, (int64_t)0), max_ctx - 1);
    const int e0 = vv * VE;
    const int ep = e0 < HD / 2 ? e0 + HD / 2 : e0 - HD / 2;
    // Buffer loads: each row base is uniform (a scalar resource) and lanes add
    // one of two 32-bit byte offsets, so these loads, whose addresses do not
    // change over the loop, hold no 64-bit address registers through it.
    const int o0 = e0 * Elem<DT>::bytes, op = ep * Elem<DT>::bytes;
    auto at = [](const void* base, int64_t elems, int off) {
      const auto r = __builtin_amdgcn_make_buffer_rsrc(
          (char*)const_cast<void*>(base) + elems * Elem<DT>::bytes, (short)0, 0x7fffffff,
          0x00020000);
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
      return uint4{v[0], v[1], v[2], v[3]};
    };
    // every load first (a use between them would wait for all earlier loads,
    // the key/value loads of the step included)
    uint4 qx[GB], qxp[GB];
#pragma unroll
    for (int g = 0; g < GB; ++g) {
      const int64_t row = b * R.ldq + ((int64_t)kh * G + g0 + (g < ng ? g : 0)) * HD;
      qx[g] = at(R.q, row, o0);
      qxp[g] = at(R.q, row, op);
    }
    const int64_t krow = b * R.ldk + (int64_t)kh * HD;
    const uint4 kx = at(R.k, krow, o0), kxp = at(R.k, krow, op);
    const uint4 cr = at(R.cos_t, pt * HD, o0), sr = at(R.sin_t, pt * HD, o0);
    vn = at(R.v, b * R.ldv + (int64_t)kh * HD, o0);
    uint4 qw0{}, qw1{}, kw0{}, kw1{};
    if constexpr (ROPE == 2) {
      // a missing weight vector (one of the two norms only) reads a table row, unused
      const void* qw = R.q_norm ? R.q_norm : R.cos_t;
      const void* kw = R.k_norm ? R.k_norm : R.cos_t;
      qw0 = at(qw, 0, o0);
      qw1 = at(qw, 0, op);
      kw0 = at(kw, 0, o0);
      kw1 = at(kw, 0, op);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int g = 0; g < GB; ++g) {
      if (g < ng) {
        rope_apply<DT, HD>(qf[g], qx[g], qxp[g], cr, sr, ROPE == 2 && R.q_norm != nullptr, qw0,
                           qw1, R.eps, vv);
      } else {
#pragma unroll
        for (int e = 0; e < VE; ++e) qf[g][e] = 0.f;
      }
    }
    float kf[VE];
    rope_apply<DT, HD>(kf, kx, kxp, cr, sr, ROPE == 2 && R.k_norm != nullptr, kw0, kw1, R.eps,
                       vv);
    kn = Vec16<DT>::pack(kf);
    // The slice that holds the new position reads its key and value from
    // registers; the first head block of that slice also writes them into the
    // cache for later steps. No other workgroup of the launch reads that
    // position, so the write needs no ordering within the launch.
    if (pcur >= lo && pcur < hi && blockIdx.y % n_hb == 0 && wave == 0 && rr == 0) {
      *(uint4*)((char*)R.k_cache + (head_off + pcur * HD + e0) * Elem<DT>::bytes) = kn;
      *(uint4*)((char*)R.v_cache + (head_off + pcur * HD + e0) * Elem<DT>::bytes) = vn;
    }
  };
  if constexpr (ROPE) {
    // an empty slice never runs the loop: its partial is empty whatever q is
#pragma unroll
    for (int g = 0; g < GB; ++g)
#pragma unroll
      for (int e = 0; e < VE; ++e) qf[g][e] = 0.f;
  } else {
#pragma unroll
    for (int g = 0; g < GB; ++g) {
      if (g < ng) {
        Vec16<DT>::load(qf[g], q, (b * heads + (int64_t)kh * G + g0 + g) * HD + vv * VE);
      } else {
#pragma unroll
        for (int e = 0; e < VE; ++e) qf[g][e] = 0.f;
      }
    }
  }
  float m[GB], l[GB], o[GB][VE];
#pragma unroll
  for (int g = 0; g < GB; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < VE; ++e) o[g][e] = 0.f;
  }

  for (int64_t p0 = lo; p0 < hi; p0 += STEP) {
    // positions past the slice are clamped to its last one (loads stay
    // unconditional, see add_rmsnorm) and masked out of the softmax
    uint4 kr[kAttnJ], vr[kAttnJ];
    bool ok[kAttnJ];
#pragma unroll
    for (int j = 0; j < kAttnJ; ++j) {
      const int64_t p = p0 + wave * WSTEP + j * RPI + rr;
      ok[j] = p < hi;
      kr[j] = Vec16<DT>::raw(kc, head_off + (ok[j] ? p : hi - 1) * HD + vv * VE);
    }
#pragma unroll
    for (int j = 0; j < kAttnJ; ++j) {
      const int64_t p = p0 + wave * WSTEP + j * RPI + rr;
      vr[j] = Vec16<DT>::raw(vc, head_off + (ok[j] ? p : hi - 1) * HD + vv * VE);
    }
    // every key and value load of the step is issued before the first use
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (ROPE) {
      if (p0 == lo) rope_prep();
#pragma unroll
      for (int j = 0; j < kAttnJ; ++j) {
        // a bitwise merge of values: `c ? kn : kr[j]` on two vector lvalues
        // selects between their addresses, which keeps both in scratch memory
        const uint32_t c = 0u - (uint32_t)(p0 + wave * WSTEP + j * RPI + rr == pcur);
        kr[j] = merge(c, kn, kr[j]);
        vr[j] = merge(c, vn, vr[j]);
      }
    }
    float kf[kAttnJ][VE], vf[kAttnJ][VE];
#pragma unroll
    for (int j = 0; j < kAttnJ; ++j) Vec16<DT>::unpack(kf[j], kr[j]);
    float s[GB][kAttnJ];
#pragma unroll
    for (int g = 0; g < GB; ++g) {
#pragma unroll
      for (int j = 0; j < kAttnJ; ++j) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < VE; ++e) d += qf[g][e] * kf[j][e];
#pragma unroll
        for (int off = 1; off < LPR; off <<= 1) d += __shfl_xor(d, off);
        s[g][j] = ok[j] ? d * scale_log2 : -INFINITY;
      }
    }
#pragma unroll
    for (int j = 0; j < kAttnJ; ++j) Vec16<DT>::unpack(vf[j], vr[j]);
#pragma unroll
    for (int g = 0; g < GB; ++g) {
      float mx = s[g][0];
#pragma unroll
      for (int j = 1; j < kAttnJ; ++j) mx = fmaxf(mx, s[g][j]);
#pragma unroll
      for (int off = LPR; off < 64; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
      const float mn = fmaxf(m[g], mx);
      if (mn == -INFINITY) continue;  // no valid position for this wave yet
      const float alpha = exp2f(m[g] - mn);
      float ps = 0.f;
      float pj[kAttnJ];
#pragma unroll
      for (int j = 0; j < kAttnJ; ++j) {
        pj[j] = ok[j] ? exp2f(s[g][j] - mn) : 0.f;
        ps += pj[j];
      }
#pragma unroll
      for (int off = LPR; off < 64; off <<= 1) ps += __shfl_xor(ps, off);
      l[g] = l[g] * alpha + ps;
      m[g] = mn;
#pragma unroll
      for (int e = 0; e < VE; ++e) {
        float acc = o[g][e] * alpha;
#pragma unroll
        for (int j = 0; j < kAttnJ; ++j) acc += pj[j] * vf[j][e];  // pj = 0 when masked
        o[g][e] = acc;
      }
    }
  }
  // sum o over the wave's row groups, then merge the four waves
#pragma unroll
  for (int g = 0; g < GB; ++g) {
#pragma unroll
    for (int e = 0; e < VE; ++e) {
      float acc = o[g][e];
#pragma unroll
      for (int off = LPR; off < 64; off <<= 1) acc += __shfl_xor(acc, off);
      o[g][e] = acc;
    }
    if (rr == 0) {
#pragma unroll
      for (int e = 0; e < VE; ++e) sh_o[wave][g][vv * VE + e] = o[g][e];
    }
    if (lane == 0) {
      sh_m[wave][g] = m[g];
      sh_l[wave][g] = l[g];
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < GB * HD; i += 256) {
    const int g = i / HD, d = i % HD;
    if (g >= ng) continue;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) mx = fmaxf(mx, sh_m[w][g]);
    float lsum = 0.f, acc = 0.f;
    if (mx != -INFINITY) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float sc = exp2f(sh_m[w][g] - mx);  // 0 for a wave with no position
        lsum += sh_l[w][g] * sc;
        acc += sh_o[w][g][d] * sc;
      }
    }
    const int64_t hrow = (b * heads + (int64_t)kh * G + g0 + g) * n_split + split;
    st_agent(part_o + hrow * HD + d, acc);
    if (d == 0) {
      st_agent(part_ml + 2 * hrow, mx);
      st_agent(part_ml + 2 * hrow + 1, lsum);
    }
  }

  // The slice that finishes last merges every slice of its heads: partials are
  // stored device-coherently and acknowledged before the arrival count, which
  // the last arriver returns to zero (the counters are zero at rest).
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  __shared__ int last;
  int* cnt = counters + (b * kv_heads + kh) * n_hb + (blockIdx.y % n_hb);
  if (threadIdx.x == 0) {
    last = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == n_split - 1;
    if (last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!last) return;
  __shared__ float cm[GB][kMaxSplits], cl[GB][kMaxSplits];
  for (int i = threadIdx.x; i < ng * n_split; i += 256) {
    const int g = i / n_split, sp = i % n_split;
    const int64_t hrow = (b * heads + (int64_t)kh * G + g0 + g) * n_split + sp;
    cm[g][sp] = ld_agent(part_ml + 2 * hrow);
    cl[g][sp] = ld_agent(part_ml + 2 * hrow + 1);
  }
  __syncthreads();
  // partials span rows·heads·n_split·HD floats (below 2 GiB: the host checks)
  const auto pr = __builtin_amdgcn_make_buffer_rsrc(part_o, (short)0, 0x7fffffff, 0x00020000);
  for (int i = threadIdx.x; i < GB * HD; i += 256) {
    const int g = i / HD, d = i % HD;
    if (g >= ng) continue;
    const int h = kh * G + g0 + g;
    const int64_t base = (b * heads + h) * n_split;
    float mx = -INFINITY;
    for (int sp = 0; sp < n_split; ++sp)
      if (cl[g][sp] > 0.f) mx = fmaxf(mx, cm[g][sp]);
    float lsum = 0.f, acc = 0.f;
#pragma unroll 8
    for (int sp = 0; sp < n_split; ++sp) {  // every slice stored its partial (zero if empty)
      const float sc = cl[g][sp] > 0.f ? exp2f(cm[g][sp] - mx) : 0.f;
      lsum += cl[g][sp] * sc;
      acc += ld_sc1(pr, (base + sp) * HD + d) * sc;
    }
    store_scalar<DT>(out, b * ldo + (int64_t)h * HD + d, lsum > 0.f ? acc / lsum : 0.f);
  }
}

// ---------------------------------------------------------------------------
// silu_mul: out = silu(gate) · up, silu rounded to the dtype first (LlamaMLP).
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(256) void silu_mul_kernel(const void* g, int64_t ldg, const void* u,
                                                       int64_t ldu, void* out, int64_t ldo,
                                                       int64_t rows, int64_t n) {
  const int64_t total = rows * n;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / n, c = i % n;
    const float gv = load_scalar<DT>(g, r * ldg + c);
    const float a = rnd<DT>(gv / (1.f + expf(-gv)));
    store_scalar<DT>(out, r * ldo + c, a * load_scalar<DT>(u, r * ldu + c));
  }
}

template <template <int> class K, typename... Args>
void launch_dt(int dtype, dim3 grid, dim3 block, hipStream_t st, Args... args) {
  if (dtype == SSL_F32) hipLaunchKernelGGL(K<DT_F32>::fn, grid, block, 0, st, args...);
  else if (dtype == SSL_BF16) hipLaunchKernelGGL(K<DT_BF16>::fn, grid, block, 0, st, args...);
  else hipLaunchKernelGGL(K<DT_F16>::fn, grid, block, 0, st, args...);
}

template <int DT>
void launch_norm(int hidden, unsigned rows, hipStream_t st, void* h, int64_t ldh,
                 const void* delta, int64_t ldd, const void* w, void* out, int64_t ldo, float eps,
                 const void* embed, int64_t lde, const int64_t* tokens, int64_t vocab) {
  const int k = (hidden + 255) / 256;
#define SSL_NORM(KK)                                                                           \
  hipLaunchKernelGGL((add_rmsnorm_kernel<DT, KK>), dim3(rows), dim3(256), 0, st, h, ldh, delta, \
                     ldd, w, out, ldo, hidden, eps, embed, lde, tokens, vocab)
  if (k <= 1) SSL_NORM(1);
  else if (k <= 2) SSL_NORM(2);
  else if (k <= 4) SSL_NORM(4);
  else if (k <= 8) SSL_NORM(8);
  else if (k <= 16) SSL_NORM(16);
  else SSL_NORM(32);
#undef SSL_NORM
}

int norm_launch(int32_t dtype, int hidden, unsigned rows, hipStream_t st, void* h, int64_t ldh,
                const void* delta, int64_t ldd, const void* w, void* out, int64_t ldo, float eps,
                const void* embed, int64_t lde, const int64_t* tokens, int64_t vocab) {
  if (dtype == SSL_F32)
    launch_norm<DT_F32>(hidden, rows, st, h, ldh, delta, ldd, w, out, ldo, eps, embed, lde, tokens, vocab);
  else if (dtype == SSL_BF16)
    launch_norm<DT_BF16>(hidden, rows, st, h, ldh, delta, ldd, w, out, ldo, eps, embed, lde, tokens, vocab);
  else
    launch_norm<DT_F16>(hidden, rows, st, h, ldh, delta, ldd, w, out, ldo, eps, embed, lde, tokens, vocab);
  return check_hip(hipGetLastError(), "rmsnorm launch");
}
template <int DT>
struct Rope { static constexpr auto fn = rope_kv_kernel<DT>; };
template <int DT>
struct SiluMul { static constexpr auto fn = silu_mul_kernel<DT>; };

template <int DT, int HD, int ROPE>
int launch_attn_hd(int GB, dim3 grid, hipStream_t st, const void* q, const void* kc,
                   const void* vc, const int32_t* pos, int64_t max_ctx, int heads, int kv_heads,
                   int n_split, float sl2, float* po, float* pml, int* cnt, void* out,
                   int64_t ldo, const RopeIn& R) {
  switch (GB) {
    case 1: hipLaunchKernelGGL((attn_split_kernel<DT, HD, 1, ROPE>), grid, dim3(256), 0, st, q, kc, vc, pos, max_ctx, heads, kv_heads, n_split, sl2, po, pml, cnt, out, ldo, R); break;
    case 2: hipLaunchKernelGGL((attn_split_kernel<DT, HD, 2, ROPE>), grid, dim3(256), 0, st, q, kc, vc, pos, max_ctx, heads, kv_heads, n_split, sl2, po, pml, cnt, out, ldo, R); break;
    case 4: hipLaunchKernelGGL((attn_split_kernel<DT, HD, 4, ROPE>), grid, dim3(256), 0, st, q, kc, vc, pos, max_ctx, heads, kv_heads, n_split, sl2, po, pml, cnt, out, ldo, R); break;
    default: hipLaunchKernelGGL((attn_split_kernel<DT, HD, 8, ROPE>), grid, dim3(256), 0, st, q, kc, vc, pos, max_ctx, heads, kv_heads, n_split, sl2, po, pml, cnt, out, ldo, R); break;
  }
  return 0;
}

template <int DT, int ROPE>
void launch_attn_rope(int hd, int GB, dim3 grid, hipStream_t st, const void* q, const void* kc,
                      const void* vc, const int32_t* pos, int64_t max_ctx, int heads, int kv_heads,
                      int n_split, float sl2, float* po, float* pml, int* cnt, void* out,
                      int64_t ldo, const RopeIn& R) {
  if (hd == 64) launch_attn_hd<DT, 64, ROPE>(GB, grid, st, q, kc, vc, pos, max_ctx, heads, kv_heads, n_split, sl2, po, pml, cnt, out, ldo, R);
  else if (hd == 128) launch_attn_hd<DT, 128, ROPE>(GB, grid, st, q, kc, vc, pos, max_ctx, heads, kv_heads, n_split, sl2, po, pml, cnt, out, ldo, R);
  else launch_attn_hd<DT, 256, ROPE>(GB, grid, st, q, kc, vc, pos, max_ctx, heads, kv_heads, n_split, sl2, po, pml, cnt, out, ldo, R);
}

template <int DT>
void launch_attn(int rope, int hd, int GB, dim3 grid, hipStream_t st, const void* q,
                 const void* kc, const void* vc, const int32_t* pos, int64_t max_ctx, int heads,
                 int kv_heads, int n_split, float sl2, float* po, float* pml, int* cnt, void* out,
                 int64_t ldo, const RopeIn& R) {
  if (rope == 2) launch_attn_rope<DT, 2>(hd, GB, grid, st, q, kc, vc, pos, max_ctx, heads, kv_heads, n_split, sl2, po, pml, cnt, out, ldo, R);
  else if (rope == 1) launch_attn_rope<DT, 1>(hd, GB, grid, st, q, kc, vc, pos, max_ctx, heads, kv_heads, n_split, sl2, po, pml, cnt, out, ldo, R);
  else launch_attn_rope<DT, 0>(hd, GB, grid, st, q, kc, vc, pos, max_ctx, heads, kv_heads, n_split, sl2, po, pml, cnt, out, ldo, R);
}

int head_block(int G) { return G >= 5 ? 8 : (G >= 3 ? 4 : G); }

int check_dtype(int32_t dtype) {
  if (dtype != SSL_F32 && dtype != SSL_BF16 && dtype != SSL_F16)
    return fail(SSL_ERR_INVALID, "unknown dtype code %d", dtype);
  return SSL_OK;
}

}  // namespace
}  // namespace ssl

using namespace ssl;

extern "C" int ssl_add_rmsnorm(void* h, int64_t ldh, const void* delta, int64_t ldd,
                               const void* weight, void* out, int64_t ldo, int64_t rows,
                               int64_t hidden, float eps, int32_t dtype, void* stream) {
  clear_error();
  if (int rc = check_dtype(dtype)) return rc;
  if (rows < 0 || rows > 65535 * 1024LL || hidden <= 0)
    return fail(SSL_ERR_INVALID, "add_rmsnorm: rows %lld, hidden %lld", (long long)rows,
                (long long)hidden);
  if (hidden > 8192) return fail(SSL_ERR_UNSUPPORTED, "add_rmsnorm: hidden %lld above 8192",
                                 (long long)hidden);
  if (rows == 0) return SSL_OK;
  if (!h || !weight || !out || ldh < hidden || ldo < hidden || (delta && ldd < hidden))
    return fail(SSL_ERR_INVALID, "add_rmsnorm: null pointer or leading dimension below hidden");
  return norm_launch(dtype, (int)hidden, (unsigned)rows, (hipStream_t)stream, h, ldh, delta, ldd,
                     weight, out, ldo, eps, nullptr, 0, nullptr, 0);
}

extern "C" int ssl_embed_rmsnorm(const void* embed, int64_t lde, int64_t vocab,
                                 const int64_t* tokens, void* h, int64_t ldh, const void* weight,
                                 void* out, int64_t ldo, int64_t rows, int64_t hidden, float eps,
                                 int32_t dtype, void* stream) {
  clear_error();
  if (int rc = check_dtype(dtype)) return rc;
  if (rows < 0 || rows > 65535 * 1024LL || hidden <= 0 || vocab <= 0)
    return fail(SSL_ERR_INVALID, "embed_rmsnorm: rows %lld, hidden %lld, vocab %lld",
                (long long)rows, (long long)hidden, (long long)vocab);
  if (hidden > 8192) return fail(SSL_ERR_UNSUPPORTED, "embed_rmsnorm: hidden %lld above 8192",
                                 (long long)hidden);
  if (rows == 0) return SSL_OK;
  if (!embed || !tokens || !h || !weight || !out || lde < hidden || ldh < hidden || ldo < hidden)
    return fail(SSL_ERR_INVALID, "embed_rmsnorm: null pointer or leading dimension below hidden");
  return norm_launch(dtype, (int)hidden, (unsigned)rows, (hipStream_t)stream, h, ldh, nullptr, 0,
                     weight, out, ldo, eps, embed, lde, tokens, vocab);
}

extern "C" int ssl_rope_kv_append(const void* q, int64_t ldq, const void* k, int64_t ldk,
                                  const void* v, int64_t ldv, const void* cos_table,
                                  const void* sin_table, const void* q_norm, const void* k_norm,
                                  float eps, const int32_t* pos, void* q_out, void* k_cache,
                                  void* v_cache, int64_t rows, int32_t heads, int32_t kv_heads,
                                  int32_t head_dim, int64_t max_ctx, int32_t dtype, void* stream) {
  clear_error();
  if (int rc = check_dtype(dtype)) return rc;
  if (heads <= 0 || kv_heads <= 0 || heads % kv_heads)
    return fail(SSL_ERR_INVALID, "rope_kv: %d heads over %d key/value heads", heads, kv_heads);
  if (head_dim <= 0 || head_dim > 256 || head_dim % 2)
    return fail(SSL_ERR_UNSUPPORTED, "rope_kv: head_dim %d (even, at most 256)", head_dim);
  if (rows < 0 || rows > 65535 || max_ctx <= 0)
    return fail(SSL_ERR_INVALID, "rope_kv: rows %lld, max_ctx %lld", (long long)rows,
                (long long)max_ctx);
  if (rows == 0) return SSL_OK;
  if (!q || !k || !v || !cos_table || !sin_table || !pos || !q_out || !k_cache || !v_cache)
    return fail(SSL_ERR_INVALID, "rope_kv: null pointer");
  if (ldq < (int64_t)heads * head_dim || ldk < (int64_t)kv_heads * head_dim ||
      ldv < (int64_t)kv_heads * head_dim)
    return fail(SSL_ERR_INVALID, "rope_kv: leading dimension below the projection width");
  launch_dt<Rope>(dtype, dim3(heads + kv_heads, (unsigned)rows), dim3(64), (hipStream_t)stream, q,
                  ldq, k, ldk, v, ldv, cos_table, sin_table, q_norm, k_norm, eps, pos, q_out,
                  k_cache, v_cache, (int)heads, (int)kv_heads, (int)head_dim, max_ctx);
  return check_hip(hipGetLastError(), "rope_kv launch");
}

extern "C" int32_t ssl_decode_attention_splits(int64_t rows, int32_t heads, int32_t kv_heads,
                                               int64_t max_ctx) {
  if (rows <= 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads || max_ctx <= 0) return 1;
  const int G = heads / kv_heads;
  const int64_t blocks = rows * kv_heads * ((G + head_block(G) - 1) / head_block(G));
  // about 1024 workgroups, each with at least 128 positions of the full context
  // (the last slice to finish merges them all, so fewer slices end sooner)
  int64_t s = (1024 + blocks - 1) / blocks;
  s = std::min<int64_t>(s, (max_ctx + 127) / 128);
  return (int32_t)std::max<int64_t>(1, std::min<int64_t>(s, 64));
}

extern "C" int64_t ssl_decode_attention_workspace_size(int64_t rows, int32_t heads,
                                                       int32_t head_dim, int32_t n_split) {
  if (rows <= 0 || heads <= 0 || head_dim <= 0 || n_split <= 0) return 0;
  return rows * heads * n_split * ((int64_t)head_dim + 2) * 4;
}

extern "C" int64_t ssl_decode_attention_counter_count(int64_t rows, int32_t heads,
                                                      int32_t kv_heads) {
  if (rows <= 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads) return 0;
  const int G = heads / kv_heads;
  return rows * kv_heads * ((G + head_block(G) - 1) / head_block(G));
}

namespace ssl {
namespace {

// Checks and launch shared by the attention entry points; R.q is set only for
// the launch that also applies the rotary embedding and appends to the cache.
int attention_launch(const char* what, const void* q, const void* k_cache, const void* v_cache,
                     const int32_t* pos, void* out, int64_t ldo, int64_t rows, int32_t heads,
                     int32_t kv_heads, int32_t head_dim, int64_t max_ctx, float scale,
                     int32_t n_split, void* workspace, int64_t workspace_bytes, int32_t* counters,
                     int64_t n_counters, int32_t dtype, void* stream, const RopeIn& R) {
  if (int rc = check_dtype(dtype)) return rc;
  if (heads <= 0 || kv_heads <= 0 || heads % kv_heads)
    return fail(SSL_ERR_INVALID, "%s: %d heads over %d key/value heads", what, heads, kv_heads);
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(SSL_ERR_UNSUPPORTED, "%s: head_dim %d (64, 128 or 256)", what, head_dim);
  if (rows < 0 || rows > 65535 || max_ctx <= 0 || n_split <= 0 || n_split > kMaxSplits)
    return fail(SSL_ERR_INVALID, "%s: rows %lld, max_ctx %lld, splits %d", what,
                (long long)rows, (long long)max_ctx, n_split);
  if (rows == 0) return SSL_OK;
  if ((!R.q && !q) || !k_cache || !v_cache || !pos || !out || ldo < (int64_t)heads * head_dim)
    return fail(SSL_ERR_INVALID, "%s: null pointer or output leading dimension too small", what);
  if ((!R.q && !aligned(q, 16)) || !aligned(k_cache, 16) || !aligned(v_cache, 16))
    return fail(SSL_ERR_INVALID, "%s: q and the caches must be 16-byte aligned", what);
  const int64_t need = ssl_decode_attention_workspace_size(rows, heads, head_dim, n_split);
  if (need > 0x7fffffffLL)
    return fail(SSL_ERR_UNSUPPORTED, "%s: partials of %lld bytes (at most 2 GiB)", what,
                (long long)need);
  if (!workspace || workspace_bytes < need || !aligned(workspace, 16))
    return fail(SSL_ERR_WORKSPACE, "%s: workspace of %lld bytes needed", what, (long long)need);
  if (!counters || n_counters < ssl_decode_attention_counter_count(rows, heads, kv_heads))
    return fail(SSL_ERR_WORKSPACE, "%s: %lld counters needed", what,
                (long long)ssl_decode_attention_counter_count(rows, heads, kv_heads));
  const int G = heads / kv_heads;
  const int GB = head_block(G);
  const int n_hb = (G + GB - 1) / GB;
  float* po = (float*)workspace;
  float* pml = po + rows * heads * n_split * head_dim;
  const float sl2 = scale * 1.4426950408889634f;
  hipStream_t st = (hipStream_t)stream;
  const int rope = !R.q ? 0 : (R.q_norm || R.k_norm) ? 2 : 1;
  dim3 grid((unsigned)n_split, (unsigned)(kv_heads * n_hb), (unsigned)rows);
  if (dtype == SSL_F32)
    launch_attn<DT_F32>(rope, head_dim, GB, grid, st, q, k_cache, v_cache, pos, max_ctx, heads,
                        kv_heads, n_split, sl2, po, pml, counters, out, ldo, R);
  else if (dtype == SSL_BF16)
    launch_attn<DT_BF16>(rope, head_dim, GB, grid, st, q, k_cache, v_cache, pos, max_ctx, heads,
                         kv_heads, n_split, sl2, po, pml, counters, out, ldo, R);
  else
    launch_attn<DT_F16>(rope, head_dim, GB, grid, st, q, k_cache, v_cache, pos, max_ctx, heads,
                        kv_heads, n_split, sl2, po, pml, counters, out, ldo, R);
  return check_hip(hipGetLastError(), "attention launch");
}

}  // namespace
}  // namespace ssl

extern "C" int ssl_decode_attention(const void* q, const void* k_cache, const void* v_cache,
                                    const int32_t* pos, void* out, int64_t ldo, int64_t rows,
                                    int32_t heads, int32_t kv_heads, int32_t head_dim,
                                    int64_t max_ctx, float scale, int32_t n_split,
                                    void* workspace, int64_t workspace_bytes, int32_t* counters,
                                    int64_t n_counters, int32_t dtype, void* stream) {
  clear_error();
  return attention_launch("attention", q, k_cache, v_cache, pos, out, ldo, rows, heads, kv_heads,
                          head_dim, max_ctx, scale, n_split, workspace, workspace_bytes,
                          counters, n_counters, dtype, stream, RopeIn{});
}

extern "C" int ssl_decode_rope_attention(
    const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v, int64_t ldv,
    const void* cos_table, const void* sin_table, const void* q_norm, const void* k_norm, float eps,
    const int32_t* pos, void* k_cache, void* v_cache, void* out, int64_t ldo, int64_t rows,
    int32_t heads, int32_t kv_heads, int32_t head_dim, int64_t max_ctx, float scale,
    int32_t n_split, void* workspace, int64_t workspace_bytes, int32_t* counters,
    int64_t n_counters, int32_t dtype, void* stream) {
  clear_error();
  if (rows > 0) {
    if (!q || !k || !v || !cos_table || !sin_table)
      return fail(SSL_ERR_INVALID, "rope_attention: null pointer");
    if (heads <= 0 || kv_heads <= 0 || ldq < (int64_t)heads * head_dim ||
        ldk < (int64_t)kv_heads * head_dim || ldv < (int64_t)kv_heads * head_dim)
      return fail(SSL_ERR_INVALID, "rope_attention: leading dimension below the projection width");
    const int64_t eb = dtype == SSL_F32 ? 4 : 2;
    // every access is a 16-byte vector of one head's features
    if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(cos_table, 16) ||
        !aligned(sin_table, 16) || (q_norm && !aligned(q_norm, 16)) ||
        (k_norm && !aligned(k_norm, 16)) || (ldq * eb) % 16 || (ldk * eb) % 16 || (ldv * eb) % 16)
      return fail(SSL_ERR_INVALID,
                  "rope_attention: q, k, v, the tables and the norm weights must be 16-byte "
                  "aligned, and so must their rows");
  }
  RopeIn R{q, ldq, k, ldk, v, ldv, cos_table, sin_table, q_norm, k_norm, eps, k_cache, v_cache};
  return attention_launch("rope_attention", nullptr, k_cache, v_cache, pos, out, ldo, rows, heads,
                          kv_heads, head_dim, max_ctx, scale, n_split, workspace, workspace_bytes,
                          counters, n_counters, dtype, stream, R);
}

extern "C" int ssl_silu_mul(const void* gate, int64_t ldg, const void* up, int64_t ldu, void* out,
                            int64_t ldo, int64_t rows, int64_t n, int32_t dtype, void* stream) {
  clear_error();
  if (int rc = check_dtype(dtype)) return rc;
  if (rows < 0 || n < 0) return fail(SSL_ERR_INVALID, "silu_mul: negative size");
  if (rows == 0 || n == 0) return SSL_OK;
  if (!gate || !up || !out || ldg < n || ldu < n || ldo < n)
    return fail(SSL_ERR_INVALID, "silu_mul: null pointer or leading dimension below n");
  const int64_t total = rows * n;
  const unsigned blocks = (unsigned)std::min<int64_t>((total + 255) / 256, 4096);
  launch_dt<SiluMul>(dtype, dim3(blocks), dim3(256), (hipStream_t)stream, gate, ldg, up, ldu, out,
                     ldo, rows, n);
  return check_hip(hipGetLastError(), "silu_mul launch");
}
