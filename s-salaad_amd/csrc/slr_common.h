// Shared device code for the gfx950 SLR-linear kernels.
//
// Matrix-core conventions (v_mfma_f32_16x16x*, wave64):
//   A operand  : lane L holds row  (L % 16) and KE consecutive k of k-group (L / 16)
//   B operand  : lane L holds col  (L % 16) and the same KE k of k-group (L / 16)
//   accumulator: lane L holds rows 4·(L/16) + e (e = 0..3) of column (L % 16)
// Only the row/column placement is relied upon. Which k a lane's element maps to
// inside the instruction does not matter for a contraction as long as the A and
// B fragments use the same assignment, and every loader below does.
//
// Output tiles are p columns wide and split into w = p/16 MFMA column tiles
// with a strided column map: column tile s, lane column c  ->  output column w·c + s.
// A lane therefore owns w adjacent output columns, which makes every epilogue
// store one contiguous w-element vector per row.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace ssl {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x16 __attribute__((ext_vector_type(16)));

enum : int { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };

constexpr int kWave = 64;
constexpr int kWaves = 4;            // waves per workgroup
constexpr int kThreads = kWave * kWaves;

// ---------------------------------------------------------------------------
// Scalar conversions (round to nearest even, NaN stays NaN)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) | 0x40u) & 0xffffu;  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h);
  return (float)v;
}
__device__ __forceinline__ uint32_t f32_to_f16(float f) {
  _Float16 v = (_Float16)f;
  return (uint32_t)__builtin_bit_cast(uint16_t, v);
}

// ---------------------------------------------------------------------------
// Data-type traits.
//   KE  : k elements per lane in one fragment (A and B alike)
//   KM  : k covered by one "macro step" (4 k-groups · KE)
//   Frag: register image of one fragment
// 16-bit types use one v_mfma_f32_16x16x32 (KE = 8) or 16x16x16 (KE = 4) per
// macro step; fp32 uses four v_mfma_f32_16x16x4f32 (KE = 4, element e in the e-th).
// ---------------------------------------------------------------------------
template <int DT, int KE>
struct Mma;

template <int KE>
struct Frag16 {  // KE 16-bit elements, packed two per dword (even k in the low half)
  uint32_t d[KE / 2];
};
struct Frag32 {  // four fp32
  float f[4];
};

template <>
struct Mma<DT_BF16, 8> {
  using Frag = Frag16<8>;
  static constexpr int KE = 8, KM = 32;
  __device__ __forceinline__ static void run(f32x4& acc, const Frag& a, const Frag& b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
  }
};
template <>
struct Mma<DT_BF16, 4> {
  using Frag = Frag16<4>;
  static constexpr int KE = 4, KM = 16;
  __device__ __forceinline__ static void run(f32x4& acc, const Frag& a, const Frag& b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a),
                                                    __builtin_bit_cast(i16x4, b), acc, 0, 0, 0);
  }
};
template <>
struct Mma<DT_F16, 8> {
  using Frag = Frag16<8>;
  static constexpr int KE = 8, KM = 32;
  __device__ __forceinline__ static void run(f32x4& acc, const Frag& a, const Frag& b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                 __builtin_bit_cast(f16x8, b), acc, 0, 0, 0);
  }
};
template <>
struct Mma<DT_F16, 4> {
  using Frag = Frag16<4>;
  static constexpr int KE = 4, KM = 16;
  __device__ __forceinline__ static void run(f32x4& acc, const Frag& a, const Frag& b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a),
                                                __builtin_bit_cast(f16x4, b), acc, 0, 0, 0);
  }
};
template <>
struct Mma<DT_F32, 4> {
  using Frag = Frag32;
  static constexpr int KE = 4, KM = 16;
  __device__ __forceinline__ static void run(f32x4& acc, const Frag& a, const Frag& b) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.f[e], b.f[e], acc, 0, 0, 0);
  }
};

template <int DT>
struct Elem {
  static constexpr int bytes = (DT == DT_F32) ? 4 : 2;
};

// Store converters: fp32 -> storage bits.
template <int DT>
__device__ __forceinline__ float load_scalar(const void* p, int64_t i) {
  if constexpr (DT == DT_F32) return ((const float*)p)[i];
  else if constexpr (DT == DT_BF16) return bf16_to_f32(((const uint16_t*)p)[i]);
  else return f16_to_f32(((const uint16_t*)p)[i]);
}
template <int DT>
__device__ __forceinline__ uint32_t to_bits(float f) {
  if constexpr (DT == DT_BF16) return f32_to_bf16(f);
  else if constexpr (DT == DT_F16) return f32_to_f16(f);
  else return __float_as_uint(f);
}

// ---------------------------------------------------------------------------
// Contiguous fragment load: KE elements starting at element `off` of `base`.
// `valid` (0..KE) elements are read, the rest are zero. Full loads are one
// 8- or 16-byte vector access; callers guarantee that alignment.
// ---------------------------------------------------------------------------
template <int DT, int KE>
__device__ __forceinline__ typename Mma<DT, KE>::Frag load_kfrag(const void* base, int64_t off,
                                                                 int valid) {
  using F = typename Mma<DT, KE>::Frag;
  F f;
  if constexpr (DT == DT_F32) {
    const float* p = (const float*)base + off;
    if (valid >= 4) {
      float4 v = *(const float4*)p;
      f.f[0] = v.x; f.f[1] = v.y; f.f[2] = v.z; f.f[3] = v.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) f.f[e] = (e < valid) ? p[e] : 0.f;
    }
  } else {
    const uint16_t* p = (const uint16_t*)base + off;
    if (valid >= KE) {
      if constexpr (KE == 8) {
        uint4 v = *(const uint4*)p;
        f.d[0] = v.x; f.d[1] = v.y; f.d[2] = v.z; f.d[3] = v.w;
      } else {
        uint2 v = *(const uint2*)p;
        f.d[0] = v.x; f.d[1] = v.y;
      }
    } else {
#pragma unroll
      for (int d = 0; d < KE / 2; ++d) {
        uint32_t lo = (2 * d < valid) ? (uint32_t)p[2 * d] : 0u;
        uint32_t hi = (2 * d + 1 < valid) ? (uint32_t)p[2 * d + 1] : 0u;
        f.d[d] = lo | (hi << 16);
      }
    }
  }
  return f;
}

// Unmasked form: KE elements known to be in range (one vector access).
template <int DT, int KE>
__device__ __forceinline__ typename Mma<DT, KE>::Frag load_kfrag_full(const void* base,
                                                                      int64_t off) {
  using F = typename Mma<DT, KE>::Frag;
  F f;
  if constexpr (DT == DT_F32) {
    const float4 v = *(const float4*)((const float*)base + off);
    f.f[0] = v.x; f.f[1] = v.y; f.f[2] = v.z; f.f[3] = v.w;
  } else if constexpr (KE == 8) {
    const uint4 v = *(const uint4*)((const uint16_t*)base + off);
    f.d[0] = v.x; f.d[1] = v.y; f.d[2] = v.z; f.d[3] = v.w;
  } else {
    const uint2 v = *(const uint2*)((const uint16_t*)base + off);
    f.d[0] = v.x; f.d[1] = v.y;
  }
  return f;
}

template <int DT, int KE>
__device__ __forceinline__ typename Mma<DT, KE>::Frag zero_frag() {
  typename Mma<DT, KE>::Frag f;
  if constexpr (DT == DT_F32) {
#pragma unroll
    for (int e = 0; e < 4; ++e) f.f[e] = 0.f;
  } else {
#pragma unroll
    for (int d = 0; d < KE / 2; ++d) f.d[d] = 0u;
  }
  return f;
}

// ---------------------------------------------------------------------------
// Block-value loader for one macro step of a (q, p) block in [k][col] layout.
// Lane (c = L%16, g = L/16) reads rows k0 + KE·g + e (e < KE), columns w·c..w·c+w-1,
// and transposes them into w B-fragments (column tile s holds column w·c + s).
// ---------------------------------------------------------------------------
template <int DT, int KE, int W>
struct VRaw;  // raw registers of one macro step

template <int KE, int W>
struct VRaw16 {
  // W = 4: two dwords per row; W = 3: columns 0, 1 in the first dword and
  // column 2 in the low half of the second; W = 2: one dword; W = 1: one
  // 16-bit value.
  uint32_t r[KE][(W + 1) / 2];
};
template <int W>
struct VRaw32 {
  float r[4][W];
};

template <int DT, int KE, int W>
using VRawT = typename std::conditional<DT == DT_F32, VRaw32<W>, VRaw16<KE, W>>::type;

template <int DT, int KE, int W>
__device__ __forceinline__ void load_vstep(VRawT<DT, KE, W>& raw, const void* blk, int p, int k0,
                                           int lane) {
  const int c = lane & 15, g = lane >> 4;
  if constexpr (DT == DT_F32) {
    const float* b = (const float*)blk + (int64_t)(k0 + 4 * g) * p + W * c;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float* q = b + (int64_t)e * p;
      if constexpr (W == 4) {
        float4 v = *(const float4*)q;
        raw.r[e][0] = v.x; raw.r[e][1] = v.y; raw.r[e][2] = v.z; raw.r[e][3] = v.w;
      } else if constexpr (W == 3) {  // 12-byte pieces: 4-byte aligned only
        raw.r[e][0] = q[0]; raw.r[e][1] = q[1]; raw.r[e][2] = q[2];
      } else if constexpr (W == 2) {
        float2 v = *(const float2*)q;
        raw.r[e][0] = v.x; raw.r[e][1] = v.y;
      } else {
        raw.r[e][0] = *q;
      }
    }
  } else {
    const uint16_t* b = (const uint16_t*)blk + (int64_t)(k0 + KE * g) * p + W * c;
#pragma unroll
    for (int e = 0; e < KE; ++e) {
      const uint16_t* q = b + (int64_t)e * p;
      if constexpr (W == 4) {
        uint2 v = *(const uint2*)q;
        raw.r[e][0] = v.x; raw.r[e][1] = v.y;
      } else if constexpr (W == 3) {  // 6-byte pieces: 2-byte aligned only
        raw.r[e][0] = (uint32_t)q[0] | ((uint32_t)q[1] << 16);
        raw.r[e][1] = (uint32_t)q[2];
      } else if constexpr (W == 2) {
        raw.r[e][0] = *(const uint32_t*)q;
      } else {
        raw.r[e][0] = (uint32_t)*q;
      }
    }
  }
}

// Build column-tile s's fragment from the raw rows.
template <int DT, int KE, int W>
__device__ __forceinline__ typename Mma<DT, KE>::Frag vfrag(const VRawT<DT, KE, W>& raw, int s) {
  typename Mma<DT, KE>::Frag f;
  if constexpr (DT == DT_F32) {
#pragma unroll
    for (int e = 0; e < 4; ++e) f.f[e] = raw.r[e][s];
  } else {
#pragma unroll
    for (int d = 0; d < KE / 2; ++d) {
      uint32_t a, b;
      if constexpr (W == 1) {
        a = raw.r[2 * d][0];
        b = raw.r[2 * d + 1][0];
        f.d[d] = (a & 0xffffu) | (b << 16);
      } else {
        a = raw.r[2 * d][s >> 1];
        b = raw.r[2 * d + 1][s >> 1];
        f.d[d] = (s & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
      }
    }
  }
  return f;
}

// ---------------------------------------------------------------------------
// 2:4 blocks (N:M sparse S, two kept values in every group of four consecutive
// input features). A stored 32×32 block (32 input features k × 32 output
// columns j, the orientation of the (q, p) blocks) is kNmBlockBytes bytes:
//   values [16][16][2] 16-bit: [c][i][s] = the i-th kept value (k ascending)
//          of output column 2c + s, i.e. group i / 2, slot i % 2
//   index  [16][8][2] bytes:   [c][grp][s] = i0 | i1 << 2, the positions
//          (0..3, i0 < i1) of the group's two kept values in column 2c + s
// Lane (c, g) of a wave covers columns 2c, 2c + 1 and k ∈ [8g, 8g + 8): one
// 16-byte piece of values at 64c + 16g and four index bytes at 1024 + 16c + 4g,
// so one load instruction reads 1 KiB contiguous.
// ---------------------------------------------------------------------------
constexpr int kNmBlock = 32;
constexpr int kNmBlockBytes = 1280;

struct NmRaw {
  uint4 v;
  uint32_t idx;
};

__device__ __forceinline__ void load_nm(NmRaw& r, const char* blk, int lane) {
  const int c = lane & 15, g = lane >> 4;
  r.v = *(const uint4*)(blk + 64 * c + 16 * g);
  r.idx = *(const uint32_t*)(blk + 1024 + 16 * c + 4 * g);
}

// The dense MFMA B fragment (8 consecutive k of output column 2c + s) of a lane's piece.
template <int DT>
__device__ __forceinline__ typename Mma<DT, 8>::Frag nm_frag(const NmRaw& r, int s) {
  typename Mma<DT, 8>::Frag f;
  const uint32_t w[4] = {r.v.x, r.v.y, r.v.z, r.v.w};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    // kept values of column s, group h: packed i = 2h, 2h + 1 → word i, half s
    const uint32_t v0 = (w[2 * h] >> (16 * s)) & 0xffffu;
    const uint32_t v1 = (w[2 * h + 1] >> (16 * s)) & 0xffffu;
    const uint32_t ix = (r.idx >> (8 * (2 * h + s))) & 0xffu;
    const uint32_t i0 = ix & 3u, i1 = (ix >> 2) & 3u;
    uint32_t e[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) e[t] = (i0 == (uint32_t)t) ? v0 : ((i1 == (uint32_t)t) ? v1 : 0u);
    f.d[2 * h] = e[0] | (e[1] << 16);
    f.d[2 * h + 1] = e[2] | (e[3] << 16);
  }
  return f;
}

__device__ __forceinline__ int wave_uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Wave-uniform read of a structure array that no kernel writes (column indices,
// plan entries). Through the constant address space it becomes a scalar load,
// counted by lgkmcnt: waiting for it does not also wait for the vector loads
// already in flight, as a vector load's vmcnt wait would (that counter retires
// in order).
__device__ __forceinline__ int ld_uniform(const int32_t* p, int64_t i) {
  return ((const __attribute__((address_space(4))) int32_t*)p)[i];
}

// ---------------------------------------------------------------------------
// Device bounds checks, compiled in by building with SSL_DEVICE_CHECKS=1 (the
// library build's checked variant). The kernels index x, the block values and
// their outputs with numbers read from device memory: plan entries, column
// indices, prefill group, step and part records. The planners check them on
// the host; a checked build checks them again where they are read. An index
// outside what a plan can hold is recorded in the call's status word (bit
// 8 + code, a plain store: the word may be host memory, where an atomic RMW
// needs PCIe atomics) and the access it would drive is dropped or clamped, so
// every kernel still ends normally. LDS offsets are compile-time expressions
// of the tile shape, bounded by static assertions, and are not re-checked.
// ---------------------------------------------------------------------------
#ifndef SSL_DEVICE_CHECKS
#define SSL_DEVICE_CHECKS 0
#endif
enum : int {
  kChkPlan = 0,      // a streaming plan entry (row, block or unit range, parts, slot)
  kChkColumn = 1,    // a block's column index
  kChkGroupRow = 2,  // a prefill group record's block-row
  kChkStep = 3,      // a prefill step record's x column or block index
  kChkPart = 4,      // a prefill part record
};
template <typename U64>
__device__ __forceinline__ void check_fail(U64* status, int code) {
  static_assert(sizeof(U64) == 8, "a 64-bit status word");
  if (status != nullptr)
    __hip_atomic_store(status, (U64)1 << (8 + code), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// W adjacent elements in the activation dtype.
// ---------------------------------------------------------------------------
template <int DT, int W>
__device__ __forceinline__ void st_w(void* base, int64_t off, const float (&v)[W]) {
  if constexpr (DT == DT_F32) {
    float* p = (float*)base + off;
    if constexpr (W == 4) *(float4*)p = make_float4(v[0], v[1], v[2], v[3]);
    else if constexpr (W == 2) *(float2*)p = make_float2(v[0], v[1]);
    else {
#pragma unroll
      for (int i = 0; i < W; ++i) p[i] = v[i];
    }
  } else {
    uint16_t* p = (uint16_t*)base + off;
    if constexpr (W == 1 || W == 3) {
#pragma unroll
      for (int i = 0; i < W; ++i) p[i] = (uint16_t)to_bits<DT>(v[i]);
    } else {
      uint32_t w[W / 2];
#pragma unroll
      for (int i = 0; i < W / 2; ++i) w[i] = to_bits<DT>(v[2 * i]) | (to_bits<DT>(v[2 * i + 1]) << 16);
      if constexpr (W == 4) *(uint2*)p = make_uint2(w[0], w[1]);
      else *(uint32_t*)p = w[0];
    }
  }
}
template <int DT, int W>
__device__ __forceinline__ void ld_w(const void* base, int64_t off, float (&v)[W]) {
  if constexpr (DT == DT_F32) {
    const float* p = (const float*)base + off;
#pragma unroll
    for (int s = 0; s < W; ++s) v[s] = p[s];
  } else {
    const uint16_t* p = (const uint16_t*)base + off;
#pragma unroll
    for (int s = 0; s < W; ++s) v[s] = (DT == DT_BF16) ? bf16_to_f32(p[s]) : f16_to_f32(p[s]);
  }
}

}  // namespace ssl
