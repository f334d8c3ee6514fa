// Prefill-shaped SLR linear on gfx950: many token rows (M ≥ kPrefillMinM), 16-bit
// or fp32 activations. Two LDS-tiled MFMA GEMM kernels replace the row-streaming
// decode kernel (which re-reads each weight row once per 64-token tile):
//
//   latent  t[M, r_pad] = x · Bᵀ                  dense GEMM (K split, fp32
//                                                   partials summed in split order),
//                                                   rounded once to the activation
//                                                   dtype, as F.linear's output is
//   rows    y[:, row] = Σ_blocks x[:, col·p:+p] · V_blockᵀ + t · A[row·p:+p, :]ᵀ
//                       (+ bias, or + the old out for the in-place op)
//
// One engine runs both. A workgroup (4 waves) owns a BM × BN output tile and
// walks a list of steps, each 128 bytes of k (64 columns of 16-bit data, 32 of
// fp32). A step stages an A tile (BM rows of x or t) and a B tile (BN rows of
// weights, k-contiguous per output feature) in LDS; wave (wm, wn) multiplies
// its TM × TN share with v_mfma_f32_16x16x32 (fp32: v_mfma_f32_16x16x4f32).
// Tiles go from global memory straight into LDS (buffer loads with the lds
// flag) through a ring of S stages: the loads of the next S − 1 steps are in
// flight while one step computes, with one barrier per step.
//
// Sparse steps. The row kernel gives a workgroup G = BN / p block-rows ("slots")
// and walks the union of their block columns, 64 / p union entries per step (the
// plan: ssl_prefill_plan_build). A step record holds a presence mask, the first
// x column of each entry and, per entry and slot, the BSR block index (−1 when
// the slot's row has no block there), laid out so that each wave's words are
// contiguous. Each wave loads its view of a record (one word per lane) into LDS
// S steps ahead of the tile loads that use it; a lane then reads the column and
// block indices of its own chunks with ordinary LDS loads. An absent block or
// entry loads from a buffer offset past the resource, which returns zeros with
// no memory traffic, and the MFMAs of a slot absent from a 32-column half of
// the step are skipped (a wave-uniform branch on the mask). The low-rank units
// follow the sparse steps: t's 64-rank slices against the slots' rows of A.
//
// Rows of x past M read row M − 1 (their outputs are never stored). Columns of x
// past in_features (a ragged last block column) are zeroed in LDS once the
// stage has landed. Workgroups are ordered XCD-major, token tile by token tile:
// the workgroups one XCD runs at a time share a token tile, so its x panel stays
// in that XCD's L2 while the weights stream past it (each weight block is read
// by every XCD at about the same time, so the 256 MB MALL serves all but the
// first read).

#include "abi_internal.h"
#include "prefill.h"
#include "slr_common.h"

namespace ssl {

namespace {

constexpr int kPfThreads = 256;  // 4 waves
constexpr int kXcds = 8;
constexpr int kK = 64;           // 16-bit units per LDS row (128 bytes)
constexpr uint32_t kOob = 0x80000000u;

enum : int { K_ROWS_OP = 0, K_ROWS_FUSED = 1, K_LATENT = 2, K_ROWS_NM = 3 };

// 2:4 blocks as the row kernel reads them (32 input × 32 output features per
// block, kNmPfBytes each): values [j][h][8] 16-bit — output feature j, half h
// of the block's 32 input features, the 8 kept values of its 4 groups in
// order (group, slot) — then index [j] uint32: for half h (bits 16h..16h+15)
// one nibble per group, i0 | i1 << 2, the kept values' positions in the group.
// Lane (i, g) of v_smfmac_f32_16x16x64 reads one 16-byte values piece (its
// feature, 16 input features) and 16 index bits: exactly these.
constexpr int kNmPfBytes = kNmPrefillBlockBytes;

// 16-byte chunk with its elements (EB bytes each) at and past `valid` set to zero.
template <int EB>
__device__ __forceinline__ uint4 keep_first(uint4 v, int valid) {
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    if constexpr (EB == 4) {
      w[d] = d < valid ? w[d] : 0u;
    } else {
      const uint32_t lo = (2 * d < valid) ? (w[d] & 0xffffu) : 0u;
      const uint32_t hi = (2 * d + 1 < valid) ? (w[d] & 0xffff0000u) : 0u;
      w[d] = lo | hi;
    }
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// 16 bytes of an activation-dtype array (16 / EB elements from element `off`,
// 16-byte aligned) as fp32, and back (rounded once to the dtype).
template <int DT>
__device__ __forceinline__ void ld16(const void* base, int64_t off, float* v) {
  if constexpr (DT == DT_F32) {
    const float4 q = *(const float4*)((const float*)base + off);
    v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
  } else {
    const uint4 q = *(const uint4*)((const uint16_t*)base + off);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t lo = (uint16_t)(w[i] & 0xffffu), hi = (uint16_t)(w[i] >> 16);
      v[2 * i] = DT == DT_BF16 ? bf16_to_f32(lo) : f16_to_f32(lo);
      v[2 * i + 1] = DT == DT_BF16 ? bf16_to_f32(hi) : f16_to_f32(hi);
    }
  }
}
template <int DT>
__device__ __forceinline__ void st16(void* base, int64_t off, const float* v) {
  if constexpr (DT == DT_F32) {
    *(float4*)((float*)base + off) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = to_bits<DT>(v[2 * i]) | (to_bits<DT>(v[2 * i + 1]) << 16);
    *(uint4*)((uint16_t*)base + off) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// Element i of an activation-dtype array as fp32 bits stored back.
template <int DT>
__device__ __forceinline__ void store_elem(void* base, int64_t i, float v) {
  if constexpr (DT == DT_F32) ((float*)base)[i] = v;
  else ((uint16_t*)base)[i] = (uint16_t)to_bits<DT>(v);
}

// D (16 × 16) += A · B with A 16 × 64 2:4-sparse (8 kept 16-bit values per
// lane, `idx` their positions) and B 64 × 16 dense (16 values per lane: k in
// [8g, 8g + 8) then [32 + 8g, 32 + 8g + 8) for lane group g).
template <int DT>
__device__ __forceinline__ void smfmac64(f32x4& acc, uint4 a, uint4 b0, uint4 b1, int idx) {
  typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));
  const u32x8 b = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
  if constexpr (DT == DT_BF16) {
    acc = __builtin_amdgcn_smfmac_f32_16x16x64_bf16(__builtin_bit_cast(bf16x8, a),
                                                     __builtin_bit_cast(bf16x16, b), acc, idx, 0, 0);
  } else {
    acc = __builtin_amdgcn_smfmac_f32_16x16x64_f16(__builtin_bit_cast(f16x8, a),
                                                    __builtin_bit_cast(f16x16, b), acc, idx, 0, 0);
  }
}

template <int BM, int BN, int WM, int WN>
struct Tile {
  static_assert(WM * WN == 4, "four waves");
  static constexpr int TM = BM / WM, TN = BN / WN;
  static constexpr int MTI = TM / 16, NTI = TN / 16;
  static constexpr int IA = BM / 32;  // A loads per wave per step (8 rows × 128 B each)
  static constexpr int IB = BN / 32;  // B loads per wave per step
  static constexpr int LDS = (BM + BN) * kK;  // elements per LDS stage (rows of 128 bytes)
};

// Row items of a member, in order: its token tiles in groups of TG; within a
// group, its row groups (or part records) one after another, each with the
// group's token tiles adjacent. The items of one XCD are a contiguous range,
// so an XCD runs a block-row's token tiles together and its L2 serves the
// block-row's weights to all of them. When D XCDs share a group of token
// tiles, the row groups are dealt to them round-robin (XCD chunk c holds row
// groups c, c + D, c + 2D, ...), so that long rows of a skewed structure
// spread over the XCDs instead of filling one contiguous range.
// Item t → token tile tt and row group / part record j of n per token tile.
// Pairs of narrow (128-token) tiles, whose x panels stay in L2 together, when
// the token tiles pair up evenly: the 7B FFN (11008×4096, 64×64 blocks) fetched
// 119 → 75 MB per call beyond L2 at 256 tokens (60.6 MB compulsory) and ran
// 81.0 / 99.9 / 145.3 → 78.3 / 97.5 / 141.0 µs at 768 / 1024 / 1536 tokens
// (best of three interleaved runs). Larger panels evict each other's x: with
// the tall tile's 2 MB panels skewed calls lost 3-6%, and with the narrow
// tile's 2.8 MB panels at 11008 input features the Zipf 10%-density calls
// lost 12% (16×16 blocks, 176 → 198 µs) and 8% (32×32). An odd token-tile
// count (384 tokens: a lone last tile) lost 8%. Those keep one token tile per
// group (TG = 1: the items in token-tile order); pairs need narrow tiles, an
// even token-tile count and panels of at most kPairPanelBytes.
constexpr int64_t kPairPanelBytes = 1 << 20;

template <int BM, int EB>
__device__ __forceinline__ void tile_of(int t, int n, int MG, int m, int& tt, int& j) {
  constexpr int TG = 2;
  if (BM > 128 || MG % TG != 0 || (int64_t)BM * m * EB > kPairPanelBytes) {
    tt = t / n;
    j = t - tt * n;
    return;
  }
  const int blk = TG * n;
  const int pg = t / blk, r = t - pg * blk;
  const int tg = min(TG, MG - pg * TG);
  const int q = r / tg;  // position of the row group within the token-tile group
  tt = pg * TG + (r - q * tg);
  const int n_pg = (MG + TG - 1) / TG;
  const int D = max(1, min(n, kXcds / n_pg));  // XCDs sharing this group of token tiles
  const int base = n / D, rem = n % D;         // chunks 0..rem-1 hold base + 1 row groups
  int c, i;
  if (q < rem * (base + 1)) {
    c = q / (base + 1);
    i = q - c * (base + 1);
  } else {
    const int q2 = q - rem * (base + 1);
    c = rem + q2 / base;
    i = q2 - (c - rem) * base;
  }
  j = c + i * D;
}

__device__ __forceinline__ int ld_word(const int32_t* p, int i) {
  return __builtin_amdgcn_readfirstlane(ld_uniform(p, i));
}

// word base + k·stride_k of `rec` for k = sel (0 ≤ sel < N, per lane): scalar
// loads and a chain of selects (no local array, which a per-lane index would
// place in scratch memory)
template <int N>
__device__ __forceinline__ int pick_word(const int32_t* rec, int base, int stride_k, int sel) {
  int x = ld_word(rec, base);
#pragma unroll
  for (int k = 1; k < N; ++k) {
    const int v = ld_word(rec, base + k * stride_k);
    x = (sel == k) ? v : x;
  }
  return x;
}

// A buffer resource as four SGPRs (base, no stride, size in bytes; loads at
// offsets past the size read zeros), for the direct-to-LDS loads below.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x4 rsrc_words(const void* base, int64_t bytes) {
  const uint64_t b = (uint64_t)(uintptr_t)base;
  const uint32_t n = bytes > 0x7fffffffLL ? 0x7fffffffu : (uint32_t)bytes;
  u32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((uint32_t)b);
  r[1] = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32) & 0xffffu);
  r[2] = __builtin_amdgcn_readfirstlane(n);
  r[3] = 0x00020000u;
  return r;
}

// Global memory straight into LDS, 16 bytes per lane: lane l of the wave
// writes LDS byte address lds + 16·l, so one instruction fills 1 KiB. The byte
// offset is voff (per lane) + soff
// (uniform); every use keeps soff inside the buffer, so the zero-fill of a
// lane rests on voff alone (an absent block or chunk: voff ≥ 2^31). Issued as
// inline assembly so that the compiler neither tracks these LDS writes nor
// inserts its own waits for them: the engine waits with explicit vmcnt counts
// (every load of the loop is unconditional, so the counts are exact) and
// orders LDS access with explicit barriers. No memory clobber: the waits and
// barriers that order LDS access around these loads are compiler barriers
// themselves.
__device__ __forceinline__ void dma16(const u32x4& r, uint32_t voff, uint32_t soff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(lds), "v"(voff), "s"(r), "s"(__builtin_amdgcn_readfirstlane(soff))
               : "m0");
}
// The same with the sc1 cache policy: device-coherent, for data another
// workgroup of the launch wrote (the latent) that a stale cache line must not
// hide.
__device__ __forceinline__ void dma16_sc1(const u32x4& r, uint32_t voff, uint32_t soff,
                                          uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen sc1 lds"
               :
               : "s"(lds), "v"(voff), "s"(r), "s"(__builtin_amdgcn_readfirstlane(soff))
               : "m0");
}

// 4 bytes a lane: lane l writes LDS byte address lds + 4·l (active lanes only).
__device__ __forceinline__ void dma4(const u32x4& r, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               :
               : "s"(lds), "v"(voff), "s"(r)
               : "m0");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p);
}

// s_waitcnt vmcnt(n) / lgkmcnt(0), also compiler barriers for memory accesses
// (LDS reads of data a direct-to-LDS load wrote must stay after the wait).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
// Workgroup barrier that is also a compiler barrier for memory accesses. It
// first waits for this wave's LDS reads (the stage the next loads overwrite
// was read by the previous step's fragment loads); loads are waited for
// explicitly.
__device__ __forceinline__ void barrier_only() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// LDS layout of a stage: rows of 64 elements (128 bytes), A rows first, then
// B rows. The 16-byte chunk kc of row R sits at position kc ^ (R % 8) of the
// row, so the 8 rows one load instruction fills and the 16 rows one fragment
// read covers spread over all banks without padding (which the 1 KiB
// contiguous direct-to-LDS writes cannot skip).
__device__ __forceinline__ int lds_chunk(int R, int kc) { return R * kK + ((kc ^ (R & 7)) << 3); }

// Cross-workgroup hand-over of the latent inside one launch. The latent's
// workgroups store their tile with the sc1 cache policy (device-coherent),
// wait for the stores to be acknowledged, and count the tile with a relaxed
// agent-scope add; a row workgroup polls that count (bounded) before its
// low-rank steps and reads the latent with sc1 loads. No cache-wide fence.
constexpr int kSc1Policy = 16;
// fp32 partial tile of a latent K chunk: 64 tokens × 64 ranks
constexpr int kLatentPartFloats = kPrefillLatentRows * 64;
__device__ __forceinline__ void st_sc1(const __amdgpu_buffer_rsrc_t& r, int off, float v, int eb,
                                       uint32_t bits16) {
  if (eb == 4) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, kSc1Policy);
  else __builtin_amdgcn_raw_buffer_store_b16((unsigned short)bits16, r, off, 0, kSc1Policy);
}

// Workgroups per compute unit that the stages' LDS allows (160 KiB per CU).
constexpr int pf_occupancy(int BM, int BN, int S) {
  return (160 * 1024) / ((BM + BN) * kK * 2 * S) > 4 ? 4 : (160 * 1024) / ((BM + BN) * kK * 2 * S);
}

// ---------------------------------------------------------------------------
// The engine. KIND: K_ROWS_OP / K_ROWS_FUSED (rows of the block-sparse linear),
// K_ROWS_NM (the fused linear with 2:4 S on v_smfmac_f32_16x16x64: its tiles
// are computed transposed, output features × tokens, because the sparse
// operand of the structured-sparse MFMA is its A) or K_LATENT (t = x·Bᵀ). P: block size (rows kernels). S: LDS stages (loads
// of S − 1 steps in flight while one step computes). A step is 128 bytes of
// every tile row: 64 k columns of 16-bit data (one v_mfma_f32_16x16x32 per
// 32 k) or 32 of fp32 (four v_mfma_f32_16x16x4f32 per 16 k, element e of a
// lane's 16-byte chunk in the e-th).
//
// Every kernel argument the step loop uses is read into a register before the
// loop: the loop's waits and barriers are compiler barriers for memory, which
// would otherwise reload them from the argument segment every step.
// ---------------------------------------------------------------------------
template <int DT, int KIND, int P, int BM, int BN, int WM, int WN, int S>
__device__ __forceinline__ void pf_body(const PfArgs& a, int bid, int n_bid,
                                        uint16_t (*lds)[Tile<BM, BN, WM, WN>::LDS]) {
  using T = Tile<BM, BN, WM, WN>;
  constexpr int IA = T::IA, IB = T::IB, MTI = T::MTI, NTI = T::NTI;
  constexpr bool ROWS = KIND != K_LATENT;
  constexpr bool NM = KIND == K_ROWS_NM;
  constexpr bool LR = KIND == K_ROWS_FUSED || NM;  // rows kernels with low-rank steps
  static_assert(!NM || (P == 32 && BN == 64 && DT != DT_F32), "2:4 tiles: 32-wide blocks, 16-bit");
  constexpr int G = ROWS ? BN / P : 1;
  constexpr int EB = Elem<DT>::bytes;
  constexpr int CE = 16 / EB;       // elements per 16-byte chunk
  constexpr int KS = 8 * CE;        // k columns per step
  static_assert(!ROWS || KS % P == 0, "a step holds whole blocks");
  constexpr int E = ROWS ? KS / P : 1;
  constexpr int kRecInts = (1 + E + 4 * IB * E + 3) / 4 * 4;  // ssl_prefill_step_ints(P, G)
  constexpr int LOADS = IA + IB;    // tile load instructions per wave per step
  // loads issued after a step's tile loads by the time that step is waited
  // on: the tile loads of the S − 2 later steps
  constexpr int kWait = (S - 2) * LOADS;
  // the rows kernels' record loads rely on every load being waited for at
  // each step
  static_assert(!ROWS || S == 2, "rows kernels run two stages");
  constexpr int NRV = 1 + E + IB * E;  // words of a wave's record view
  static_assert(NRV <= 64, "a record view is one word per lane");
  using MM = Mma<DT, DT == DT_F32 ? 4 : 8>;
  using Frag = typename MM::Frag;

  // ---- which tile
  const int items = a.items;
  int item;
  if constexpr (KIND == K_LATENT) {
    item = bid;
    if (item >= items) return;
  } else {  // XCD-major order
    const int per_xcd = (items + kXcds - 1) / kXcds;
    item = (bid % kXcds) * per_xcd + bid / kXcds;
    if (item >= items) return;
  }
  (void)n_bid;
  int mi = 0;
  while (mi + 1 < a.n && item >= a.off[mi + 1]) ++mi;
  const PfMember& mb = a.mb[mi];
  const int local = item - a.off[mi];
  const int M = a.M, m = a.m;

  int m0, s_begin, s_end;            // token tile; step range
  int n_sp = 0;                      // sparse steps (rows kernels)
  const int32_t* gr = nullptr;       // group record: {step_begin, step_end, rows[G]}
  int rt = 0;                        // latent: rank tile
  int ksplit = mb.ksplit;            // K parts of a tile (1: whole)
  int tile = local / ksplit;         // a tile's parts are adjacent items
  int kp = local - tile * ksplit;    // this workgroup's part
  int64_t part_tile = (int64_t)tile * ksplit;  // rows: its parts' first partial tile
  int arrive = tile;                 // rows: its parts' arrival word
  bool has_lr = LR;                  // rows: this part runs the low-rank steps
  if constexpr (KIND == K_LATENT) {
    const int n_rt = mb.r_pad / BN;
    rt = tile % n_rt;
    m0 = (tile / n_rt) * BM;
    s_begin = kp * mb.kchunk;
    s_end = min(a.m_pad / KS, s_begin + mb.kchunk);
  } else {
    int grp;
    if (mb.parts != nullptr) {
      // the member's part table (ssl_prefill_parts_build): per token tile,
      // its records in turn, each a group's step range and its part of them
      int tt, j;
      tile_of<BM, EB>(local, mb.n_parts, (M + BM - 1) / BM, m, tt, j);
      const int32_t* pr = mb.parts + (int64_t)j * kPartInts;
      grp = ld_word(pr, 0);
      s_begin = ld_word(pr, 1);
      n_sp = ld_word(pr, 2) - s_begin;
      kp = ld_word(pr, 3);
      ksplit = ld_word(pr, 4);
      const int first = ld_word(pr, 5);
#if SSL_DEVICE_CHECKS
      if (!(grp >= 0 && grp < mb.n_groups && ksplit >= 1 && ksplit <= 16 && kp >= 0 &&
            kp < ksplit && (ksplit == 1 || (first >= 0 && first + ksplit <= mb.split_parts)) &&
            n_sp >= 0 && s_begin >= ld_word(mb.groups + (int64_t)grp * (2 + G), 0) &&
            s_begin + n_sp <= ld_word(mb.groups + (int64_t)grp * (2 + G), 1))) {
        if (threadIdx.x == 0) check_fail(a.status, kChkPart);
        return;
      }
#endif
      part_tile = (int64_t)tt * mb.split_parts + first;
      arrive = tt * mb.n_groups + grp;
      m0 = tt * BM;
      gr = mb.groups + (int64_t)grp * (2 + G);
    } else {
      int tt;
      tile_of<BM, EB>(tile, mb.n_groups, (M + BM - 1) / BM, m, tt, grp);
      m0 = tt * BM;
      gr = mb.groups + (int64_t)grp * (2 + G);
      // part kp of the group's sparse steps; the last part also the low-rank ones
      const int g0 = ld_word(gr, 0), n_all = ld_word(gr, 1) - g0;
      const int chunk = (n_all + ksplit - 1) / ksplit;
      const int b0 = min(kp * chunk, n_all), b1 = min(b0 + chunk, n_all);
      s_begin = g0 + b0;
      n_sp = b1 - b0;
    }
#if SSL_DEVICE_CHECKS
    {
      bool ok = true;
#pragma unroll
      for (int g2 = 0; g2 < G; ++g2) {
        const int r = ld_word(gr, 2 + g2);
        ok = ok && r >= -1 && r < mb.NB;
      }
      if (!ok) {
        if (threadIdx.x == 0) check_fail(a.status, kChkGroupRow);
        return;
      }
    }
#endif
    // a member with no low-rank factor (r_pad 0) has no latent tiles to wait
    // for and no tile counters (tcnt is null): it neither waits nor departs
    has_lr = LR && kp == ksplit - 1 && mb.r_pad > 0;
    const int n_lr = has_lr ? mb.r_pad / KS : 0;
    s_end = s_begin + n_sp + n_lr;
  }
  const int U = s_end - s_begin;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wid / WN, wn = wid % WN;
  // This lane loads, in every tile load instruction, row (8·instr_row + lane / 8)
  // and the column chunk that lands at position lane % 8 of that row.
  const int lrow = lane >> 3;
  const int kc = (lane & 7) ^ lrow;
  const int e_t = (ROWS && E > 1) ? (kc * CE) / P : 0;  // rows kernels: this lane's entry of a step
  const int kin = ROWS ? (kc * CE) % P : kc * CE;  // and its column within the entry

  // ---- LDS byte addresses: stage 0's A rows 8·wid and B rows 8·wid; 2:4
  // steps: this wave's 16 rows of the values region (64 bytes a row) and its
  // 16 rows of the index region (8 bytes a row, after 4 KiB of values)
  const uint32_t la0 = lds_addr(&lds[0][8 * wid * kK]);
  const uint32_t lb0 = lds_addr(&lds[0][(BM + 8 * wid) * kK]);
  const uint32_t lnv0 = lds_addr(&lds[0][BM * kK]) + 1024u * wid;
  const uint32_t lni0 = lds_addr(&lds[0][BM * kK]) + 4096u + 128u * wid;
  constexpr uint32_t kStageBytes = T::LDS * 2, kRowBytes32 = 32 * kK * 2;

  // ---- constant parts of this lane's addresses
  const u32x4 xr = rsrc_words(a.x, (int64_t)M * a.ldx * EB);
  uint32_t ax[IA];               // x offsets of its A loads at entry column 0
#pragma unroll
  for (int i = 0; i < IA; ++i)
    ax[i] = (uint32_t)(min(m0 + 8 * (wid + 4 * i) + lrow, M - 1) * a.ldx * EB + kin * EB);
  u32x4 tr = xr, br = xr, ar = xr;
  uint32_t at_[IA];              // t offsets of its A loads (low-rank steps)
  uint32_t bconst[IB];           // B offsets that do not change per step
  uint32_t lroff[IB];            // A-matrix offsets of its B loads (low-rank steps)
  const int32_t* steps = nullptr;  // this group's first step record
  int rword = 0;                   // this lane's word of a record
  int lr_mask = 0;
  if constexpr (KIND == K_LATENT) {
    br = rsrc_words(mb.B, (int64_t)mb.r_pad * mb.ldb * EB);
#pragma unroll
    for (int i = 0; i < IB; ++i)
      bconst[i] = (uint32_t)(((int64_t)(rt * BN + 8 * (wid + 4 * i) + lrow) * mb.ldb + kc * CE) * EB);
#pragma unroll
    for (int i = 0; i < IA; ++i) at_[i] = 0;
#pragma unroll
    for (int i = 0; i < IB; ++i) lroff[i] = 0;
  } else {
    br = rsrc_words(mb.values_pq, mb.values_bytes);
#pragma unroll
    for (int i = 0; i < IB; ++i) {
      const int f = 8 * (wid + 4 * i) + lrow, j = f % P;
      bconst[i] = (uint32_t)((j * P + kin) * EB);
    }
    if constexpr (LR) {
      tr = rsrc_words(mb.t, (int64_t)M * mb.ldt * EB);
      ar = rsrc_words(mb.A, mb.A_bytes);
#pragma unroll
      for (int i = 0; i < IA; ++i)
        at_[i] = (uint32_t)((min(m0 + 8 * (wid + 4 * i) + lrow, M - 1) * mb.ldt + kc * CE) * EB);
#pragma unroll
      for (int i = 0; i < IB; ++i) {
        const int f = 8 * (wid + 4 * i) + lrow;
        const int row = ld_word(gr, 2 + (8 * (wid + 4 * i)) / P);
        lroff[i] = row < 0 ? kOob : (uint32_t)(((int64_t)(row * P + f % P) * mb.lda + kc * CE) * EB);
      }
#pragma unroll
      for (int g = 0; g < G; ++g) lr_mask |= (ld_word(gr, 2 + g) >= 0) ? (1 << g) | (1 << (G + g)) : 0;
      if constexpr (NM) lr_mask |= 1 << 30;  // a low-rank step: dense MFMAs
    } else {
#pragma unroll
      for (int i = 0; i < IA; ++i) at_[i] = 0;
#pragma unroll
      for (int i = 0; i < IB; ++i) lroff[i] = 0;
    }
    steps = mb.steps + (int64_t)s_begin * kRecInts;
    // lane j of the wave holds word j of its view {mask, col[E], W[wave][IB][E]}
    const int j = lane < NRV ? lane : 0;
    rword = j < 1 + E ? j : 1 + E + wid * IB * E + (j - 1 - E);
  }

  // ---- the wave's view of sparse step v's record, one word per lane (an
  // ordinary vector load, issued one step before the tile loads that use it;
  // with two stages every load of the previous step has been waited for when
  // it is used, so the compiler's own wait for it costs nothing)
  auto read_record = [&](int v) -> int {
    if constexpr (ROWS) {
      if (n_sp > 0) return steps[(int64_t)min(v, n_sp - 1) * kRecInts + rword];
    }
    return -1;
  };
  // word w of the view as seen by this lane: lane w's value (uniform) or, for
  // the per-entry words, the word of this lane's entry (w + e_t)
  auto view_word = [&](int rv, int w) -> int { return __builtin_amdgcn_readlane(rv, w); };
  auto view_entry = [&](int rv, int w) -> int {
    if constexpr (E == 1) return __builtin_amdgcn_readlane(rv, w);
    else return __builtin_amdgcn_ds_bpermute((w + e_t) * 4, rv);
  };

  // ---- wait until the latent tiles of this tile's token rows are written
  // (rows kernels with low-rank steps; one lane per wave polls its copy,
  // bounded). The wave counts itself in the slot's departures at its end; the
  // last of the tile's waiters on that copy returns both words to zero.
  auto wait_latent = [&]() {
    if constexpr (LR) {
      if (lane == 0) {
        const int lbm = a.lbm, target = mb.r_pad / 64 + a.wait_bias, polls = a.polls;
        const int lt1 = (min(m0 + BM, M) - 1) / lbm;
        for (int lt = m0 / lbm; lt <= lt1; ++lt) {
          int n = 0;
          const int32_t* w = mb.tcnt + ((int64_t)lt * kPfCntCopies + wid % kPfCntCopies) * kPfCntStride;
          while (__hip_atomic_load(const_cast<int32_t*>(w), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) <
                 target) {
            __builtin_amdgcn_s_sleep(2);
            if (++n > polls) {
              __hip_atomic_store(a.status, (uint64_t)1, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
              break;
            }
          }
        }
      }
    }
  };

  // ---- issue the tile loads of step u (clamped past the end) into stage `k`
  // (rv: the step's record view); returns the step's mask (uniform).
  // `ragged` is set when an x chunk of the step is cut by in_features (those
  // chunks are fixed up once they landed); `xcol` is then this lane's first x
  // column in the step.
  auto fetch = [&](int u_in, int k, int rv, int& ragged, int& xcol) -> int {
    const int u = min(u_in, U - 1);
    int mask;
    const uint32_t la = la0 + (uint32_t)k * kStageBytes, lb = lb0 + (uint32_t)k * kStageBytes;
    if constexpr (KIND == K_LATENT) {
      const int k0 = (s_begin + u) * KS;
      const int col = k0 + kc * CE;
      ragged = k0 + KS > m;
      xcol = col;
      const uint32_t xcb = col < m ? (uint32_t)(k0 * EB) : kOob;
#pragma unroll
      for (int i = 0; i < IA; ++i) dma16(xr, ax[i] + xcb, 0, la + i * kRowBytes32);
#pragma unroll
      for (int i = 0; i < IB; ++i) dma16(br, bconst[i], (uint32_t)(k0 * EB), lb + i * kRowBytes32);
      mask = 3;
    } else {
      if (u < n_sp) {
        mask = view_word(rv, 0);
#if SSL_DEVICE_CHECKS
        int c = view_entry(rv, 1);  // first x column of this lane's entry, or −1
        if (c >= a.m_pad) {
          check_fail(a.status, kChkStep);
          c = -1;
        }
#else
        const int c = view_entry(rv, 1);  // first x column of this lane's entry, or −1
#endif
        const uint32_t xcb = c >= 0 ? (uint32_t)(c * EB) : kOob;
#pragma unroll
        for (int i = 0; i < IA; ++i) dma16(xr, ax[i] + xcb, 0, la + i * kRowBytes32);
        if constexpr (NM) {
          // this wave's 16 feature rows (slot wid / 2): lane l takes row l / 4,
          // entry (l % 4) / 2, half l % 2 of the values; lanes < 32 the
          // index word of row l / 2, entry l % 2
#if SSL_DEVICE_CHECKS
          int b0 = view_word(rv, 1 + E + (wid >> 1) * E);
          int b1 = view_word(rv, 1 + E + (wid >> 1) * E + 1);
          if ((int64_t)b0 * kNmPfBytes >= mb.values_bytes || (int64_t)b1 * kNmPfBytes >= mb.values_bytes) {
            check_fail(a.status, kChkStep);
            if ((int64_t)b0 * kNmPfBytes >= mb.values_bytes) b0 = -1;
            if ((int64_t)b1 * kNmPfBytes >= mb.values_bytes) b1 = -1;
          }
#else
          const int b0 = view_word(rv, 1 + E + (wid >> 1) * E);
          const int b1 = view_word(rv, 1 + E + (wid >> 1) * E + 1);
#endif
          const uint32_t kst = (uint32_t)k * kStageBytes;
          const int bv = (lane & 2) ? b1 : b0;
          const uint32_t jv = 16 * (wid & 1) + (lane >> 2);
          dma16(br, bv < 0 ? kOob : (uint32_t)bv * kNmPfBytes + jv * 32 + (lane & 1) * 16, 0,
                lnv0 + kst);
          if (lane < 32) {
            const int bi = (lane & 1) ? b1 : b0;
            const uint32_t ji = 16 * (wid & 1) + (lane >> 1);
            dma4(br, bi < 0 ? kOob : (uint32_t)bi * kNmPfBytes + 1024 + ji * 4, lni0 + kst);
          }
        } else {
#pragma unroll
          for (int i = 0; i < IB; ++i) {
#if SSL_DEVICE_CHECKS
            int blk = view_entry(rv, 1 + E + i * E);
            if ((int64_t)blk * (P * P * EB) >= mb.values_bytes) {
              check_fail(a.status, kChkStep);
              blk = -1;
            }
#else
            const int blk = view_entry(rv, 1 + E + i * E);
#endif
            dma16(br, blk < 0 ? kOob : (uint32_t)blk * (uint32_t)(P * P * EB) + bconst[i], 0,
                  lb + i * kRowBytes32);
          }
        }
        if (m % P != 0) {  // only a ragged last block column cuts chunks
          xcol = c >= 0 ? c + kin : 0x3fffffff;
          ragged = __builtin_amdgcn_ballot_w64(xcol + CE > m) != 0;
        } else {
          xcol = 0;
          ragged = 0;
        }
      } else {
        const uint32_t k0b = (uint32_t)((u - n_sp) * KS * EB);  // ranks (K_ROWS_FUSED only)
        // before the first load of t; once (fetches past the end repeat the last
        // step, which is step n_sp itself when there is one low-rank step)
        if (u_in == n_sp) wait_latent();
#pragma unroll
        for (int i = 0; i < IA; ++i) dma16_sc1(tr, at_[i], k0b, la + i * kRowBytes32);
#pragma unroll
        for (int i = 0; i < IB; ++i) dma16(ar, lroff[i], k0b, lb + i * kRowBytes32);
        mask = lr_mask;
        ragged = 0;
        xcol = 0;
      }
    }
    return mask;
  };

  // ---- zero the x elements at and past in_features in a landed ragged stage
  auto fix_ragged = [&](int k, int xcol) {
    const int valid = m - xcol;
    if (valid < CE) {
#pragma unroll
      for (int i = 0; i < IA; ++i) {
        uint16_t* q = &lds[k][lds_chunk(8 * (wid + 4 * i) + lrow, kc)];
        *(uint4*)q = valid <= 0 ? make_uint4(0, 0, 0, 0) : keep_first<EB>(*(const uint4*)q, valid);
      }
    }
  };

  f32x4 acc[MTI][NTI];
#pragma unroll
  for (int mt = 0; mt < MTI; ++mt)
#pragma unroll
    for (int nt = 0; nt < NTI; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int c = lane & 15, gq = lane >> 4;
  // ---- the MFMAs of one step from an LDS stage
  auto compute = [&](const uint16_t* buf, int mask_in) {
    const int mask = __builtin_amdgcn_readfirstlane(mask_in);
    if constexpr (NM) {
      if (!((mask >> 30) & 1)) {
        // 2:4 step: A = the weights' kept values (features × 64 k), B = the x
        // chunks gq and 4 + gq of each token row; tiles are features × tokens
        uint4 xa[MTI][2], sv[NTI];
        int ix[NTI];
        const uint16_t* vb = buf + BM * kK;  // values region (64 bytes a feature row)
#pragma unroll
        for (int mt = 0; mt < MTI; ++mt) {
          const int row = wm * T::TM + 16 * mt + c;
          xa[mt][0] = *(const uint4*)(buf + lds_chunk(row, gq));
          xa[mt][1] = *(const uint4*)(buf + lds_chunk(row, 4 + gq));
        }
#pragma unroll
        for (int nt = 0; nt < NTI; ++nt) {
          const int f = wn * T::TN + 16 * nt + c;
          sv[nt] = *(const uint4*)(vb + f * 32 + gq * 8);
          ix[nt] = vb[2048 + f * 4 + (gq >> 1) * 2 + (gq & 1)];
        }
#pragma unroll
        for (int nt = 0; nt < NTI; ++nt) {
          const int slot = (wn * T::TN + 16 * nt) / P;
          if (((mask >> slot) | (mask >> (G + slot))) & 1) {
#pragma unroll
            for (int mt = 0; mt < MTI; ++mt)
              smfmac64<DT>(acc[mt][nt], sv[nt], xa[mt][0], xa[mt][1], ix[nt]);
          }
        }
        return;
      }
    }
    Frag af[2][MTI], bf[2][NTI];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int mt = 0; mt < MTI; ++mt) {
        const uint4 v = *(const uint4*)(buf + lds_chunk(wm * T::TM + 16 * mt + c, ks * 4 + gq));
        af[ks][mt] = __builtin_bit_cast(Frag, v);
      }
#pragma unroll
      for (int nt = 0; nt < NTI; ++nt) {
        const uint4 v =
            *(const uint4*)(buf + lds_chunk(BM + wn * T::TN + 16 * nt + c, ks * 4 + gq));
        bf[ks][nt] = __builtin_bit_cast(Frag, v);
      }
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int nt = 0; nt < NTI; ++nt) {
        const int slot = (KIND == K_LATENT) ? 0 : (wn * T::TN + 16 * nt) / P;
        if ((mask >> (ks * G + slot)) & 1) {
#pragma unroll
          for (int mt = 0; mt < MTI; ++mt) {
            if constexpr (NM) MM::run(acc[mt][nt], bf[ks][nt], af[ks][mt]);  // features × tokens
            else MM::run(acc[mt][nt], af[ks][mt], bf[ks][nt]);
          }
        }
      }
    }
  };

  if (U > 0) {
    // stage (u % S) holds step u's tiles and (rows kernels) its record view;
    // the tile loads of S − 1 steps are in flight, and the record loads of the
    // S steps after those
    int masks[S], rag[S], xcol[S];
#pragma unroll
    for (int k = 0; k < S - 1; ++k) masks[k] = fetch(k, k, read_record(k), rag[k], xcol[k]);
    int next = read_record(S - 1);  // the record of the step the loop fetches first
    for (int u0 = 0; u0 < U; u0 += S) {
#pragma unroll
      for (int k = 0; k < S; ++k) {
        const int u = u0 + k;
        if (u < U) {
          wait_vmcnt<kWait>();                    // this wave's loads of step u landed
          if (__builtin_amdgcn_readfirstlane(rag[k])) {
            fix_ragged(k, xcol[k]);
            wait_lgkm0();
          }
          barrier_only();                         // every wave's; step u − 1 computed
          const int nk = (k + S - 1) % S;         // stage of step u + S − 1 (= step u − 1's)
          masks[nk] = fetch(u + S - 1, nk, next, rag[nk], xcol[nk]);
          next = read_record(u + S);
          compute(lds[k], masks[k]);
        }
      }
    }
  }
  wait_vmcnt<0>();  // no load may still be writing LDS when the workgroup ends

  auto depart = [&]() {
    if constexpr (LR) {
      if (!has_lr) return;  // only the part that ran the low-rank steps waited
      // depart; the last waiter of a latent tile's copy: every latent tile of
      // that copy has been counted (n_rt) and every waiter has departed
      // (n_groups), so subtracting both leaves the slot at zero for the next
      // launch (also after a wait that gave up: the counts still arrive within
      // the launch). Counted here rather than past the wait, so that no returned
      // value occupies a register through the low-rank steps.
      if (lane == 0) {
        const int lt0 = m0 / a.lbm, lt1 = (min(m0 + BM, M) - 1) / a.lbm;
        for (int lt = lt0; lt <= lt1; ++lt) {
          int32_t* w = mb.tcnt + ((int64_t)lt * kPfCntCopies + wid % kPfCntCopies) * kPfCntStride;
          const int old = __hip_atomic_fetch_add(w + kPfDepartWord, 1, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
          if (old == mb.n_groups - 1) {
            __hip_atomic_fetch_add(w, -(mb.r_pad / 64), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_fetch_add(w + kPfDepartWord, -mb.n_groups, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
          }
        }
      }
    }
  };

  // ---- K parts: this part's fp32 partial tile (each thread's accumulators,
  // contiguous) stored device-coherently, then counted; the last part to
  // arrive returns the count to zero, sums every part's tile in part order
  // into acc and goes on to the epilogue (true); the others are done (false).
  auto combine = [&](float* base, int32_t* arrive) -> bool {
    constexpr int TF = MTI * NTI * 4 * kPfThreads;  // floats of a part's tile
    const __amdgpu_buffer_rsrc_t pr =
        __builtin_amdgcn_make_buffer_rsrc(base, (short)0, ksplit * TF * 4, 0x00020000);
#pragma unroll
    for (int mt = 0; mt < MTI; ++mt)
#pragma unroll
      for (int nt = 0; nt < NTI; ++nt)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[mt][nt]), pr,
                                               ((kp * kPfThreads + tid) * MTI * NTI + mt * NTI + nt) * 16,
                                               0, kSc1Policy);
    __builtin_amdgcn_s_waitcnt(0);  // this thread's stores acknowledged
    __syncthreads();                // (and every wave is past its last LDS read)
    volatile int32_t* const flag = reinterpret_cast<volatile int32_t*>(&lds[0][0]);
    if (tid == 0)
      *flag = __hip_atomic_fetch_add(arrive, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (*flag != ksplit - 1) return false;
    if (tid == 0) __hip_atomic_fetch_add(arrive, -ksplit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    f32x4 sum[MTI][NTI];
#pragma unroll
    for (int mt = 0; mt < MTI; ++mt)
#pragma unroll
      for (int nt = 0; nt < NTI; ++nt) sum[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < ksplit; ++j) {
#pragma unroll
      for (int mt = 0; mt < MTI; ++mt)
#pragma unroll
        for (int nt = 0; nt < NTI; ++nt)
          sum[mt][nt] += (j == kp) ? acc[mt][nt]
                                   : __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                         pr, ((j * kPfThreads + tid) * MTI * NTI + mt * NTI + nt) * 16,
                                         0, kSc1Policy));
    }
#pragma unroll
    for (int mt = 0; mt < MTI; ++mt)
#pragma unroll
      for (int nt = 0; nt < NTI; ++nt) acc[mt][nt] = sum[mt][nt];
    return true;
  };
  if constexpr (KIND == K_LATENT) {
    if (ksplit > 1 &&
        !combine(mb.kpart + (int64_t)tile * ksplit * kLatentPartFloats,
                 mb.tcnt + (int64_t)(m0 / BM) * kPfCntCopies * kPfCntStride + kPfLatArriveWord + rt))
      return;
  } else if constexpr (BM < 256) {
    if (ksplit > 1 && !combine(mb.kpart + part_tile * (BM * BN), mb.karrive + arrive)) {
      depart();
      return;
    }
  }

  // ---- epilogue: lane (c, gq) holds rows 16·mt + 4gq + e of column 16·nt + c.
  // The output pointers and strides are read into registers first: the
  // stores below could otherwise alias the argument segment and force a
  // reload per store.
  if constexpr (KIND == K_LATENT) {
    // the tile, rounded once to the activation dtype as F.linear's output is,
    // stored device-coherently, then counted for its token rows
    const __amdgpu_buffer_rsrc_t tr =
        __builtin_amdgcn_make_buffer_rsrc(mb.t, (short)0, 0x7fffffff, 0x00020000);
    const int64_t ldt = mb.ldt;
    int32_t* const tcnt = mb.tcnt;
#pragma unroll
    for (int mt = 0; mt < MTI; ++mt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = m0 + wm * T::TM + 16 * mt + 4 * gq + e;
        if (r >= M) continue;
#pragma unroll
        for (int nt = 0; nt < NTI; ++nt) {
          const int col = rt * BN + wn * T::TN + 16 * nt + c;
          const float v = acc[mt][nt][e];
          st_sc1(tr, (int)(((int64_t)r * ldt + col) * EB), v, EB,
                 EB == 2 ? to_bits<DT>(v) : 0u);
        }
      }
    __builtin_amdgcn_s_waitcnt(0);  // this thread's stores acknowledged
    __syncthreads();
    if (tid < kPfCntCopies)
      __hip_atomic_fetch_add(tcnt + ((int64_t)(m0 / BM) * kPfCntCopies + tid) * kPfCntStride, 1,
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    // Rows: the finished tile goes through LDS as fp32 ([BM token rows][BN + 4
    // features], the bias added for the fused linear), then out 16 bytes per
    // lane, consecutive lanes along a token row's features, so a wave writes
    // whole 128-byte feature runs. (Stored straight from the MFMA layout, one
    // 2-byte element per lane, a wave's store covered four rows in 32-byte
    // pieces, and the epilogue took as long as four low-rank steps.)
    constexpr int LDT = BN + 4;  // floats per staged row; the padding spreads the banks
    static_assert(BM * LDT * 4 <= T::LDS * 2 * 2, "the staged tile fits in the stages' LDS");
    float* const stg = reinterpret_cast<float*>(&lds[0][0]);
    const void* const bias = mb.bias;
    __syncthreads();  // every wave is past its last read of the stages
#pragma unroll
    for (int nt = 0; nt < NTI; ++nt) {
      const int row = ld_word(gr, 2 + (wn * T::TN + 16 * nt) / P);
      if (row < 0) continue;
      if constexpr (NM) {
        // lane (c, gq) holds features 4gq + e of feature tile nt for token 16·mt + c
        const int fl = wn * T::TN + 16 * nt + 4 * gq;
        float bv[4] = {0.f, 0.f, 0.f, 0.f};
        if (bias != nullptr) {
#pragma unroll
          for (int e = 0; e < 4; ++e) bv[e] = load_scalar<DT>(bias, row * P + fl % P + e);
        }
#pragma unroll
        for (int mt = 0; mt < MTI; ++mt) {
          float* const d = stg + (wm * T::TM + 16 * mt + c) * LDT + fl;
#pragma unroll
          for (int e = 0; e < 4; ++e) d[e] = acc[mt][nt][e] + bv[e];
        }
      } else {
        // lane (c, gq) holds token rows 16·mt + 4gq + e of feature 16·nt + c
        const int f = wn * T::TN + 16 * nt + c;
        float bv = 0.f;
        if (KIND == K_ROWS_FUSED && bias != nullptr) bv = load_scalar<DT>(bias, row * P + f % P);
#pragma unroll
        for (int mt = 0; mt < MTI; ++mt)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            stg[(wm * T::TM + 16 * mt + 4 * gq + e) * LDT + f] = acc[mt][nt][e] + bv;
      }
    }
    __syncthreads();
    void* const y_out = mb.y;
    const int64_t ldy = mb.ldy;
    constexpr int CO = 16 / EB;   // outputs per 16-byte store
    constexpr int CPR = BN / CO;  // stores per token row of the tile
    int srow[G];                  // the slots' block-rows (−1: absent)
#pragma unroll
    for (int g = 0; g < G; ++g) srow[g] = ld_word(gr, 2 + g);
    const int rows_here = min(BM, M - m0);
    for (int q = tid; q < rows_here * CPR; q += kPfThreads) {
      const int tr = q / CPR, f0 = (q % CPR) * CO;
      int row = srow[0];
#pragma unroll
      for (int g = 1; g < G; ++g) row = (f0 / P == g) ? srow[g] : row;
      if (row < 0) continue;
      const int64_t yi = (int64_t)(m0 + tr) * ldy + row * P + f0 % P;
      float o[CO];
      const float* const sp = stg + tr * LDT + f0;
#pragma unroll
      for (int i = 0; i < CO; i += 4) {
        const float4 v = *(const float4*)(sp + i);
        o[i] = v.x; o[i + 1] = v.y; o[i + 2] = v.z; o[i + 3] = v.w;
      }
      if constexpr (KIND == K_ROWS_OP) {  // the op accumulates onto out in fp32
        float old[CO];
        ld16<DT>(y_out, yi, old);
#pragma unroll
        for (int i = 0; i < CO; ++i) o[i] += old[i];
      }
      st16<DT>(y_out, yi, o);
    }
  }
  depart();
}

// The op's row kernel (no latent): the engine in a kernel of its own.
template <int DT, int KIND, int P, int BM, int BN, int WM, int WN, int S>
__global__ __launch_bounds__(kPfThreads, pf_occupancy(BM, BN, S)) void pf_gemm(PfArgs by_value) {
  (void)by_value;
  const PfArgs& a = *(const PfArgs*)__builtin_amdgcn_kernarg_segment_ptr();
  __shared__ __align__(1024) uint16_t lds[S][Tile<BM, BN, WM, WN>::LDS];
  pf_body<DT, KIND, P, BM, BN, WM, WN, S>(a, blockIdx.x, gridDim.x, lds);
}

// The fused linear in one launch: grid [latent workgroups (padded to a
// multiple of kXcds)][row workgroups]. Latent workgroups come first in the
// grid, so every tile a row workgroup waits for belongs to a workgroup
// dispatched before it; they never wait themselves. One LDS allocation serves
// both roles.
constexpr int kLatentStages = 3;
template <int BM, int BN, int WM, int WN>
constexpr int fused_lds() {
  return Tile<BM, BN, WM, WN>::LDS * 2 > Tile<kPrefillLatentRows, 64, 2, 2>::LDS * kLatentStages
             ? Tile<BM, BN, WM, WN>::LDS * 2
             : Tile<kPrefillLatentRows, 64, 2, 2>::LDS * kLatentStages;
}
template <int DT, int KIND, int P, int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(kPfThreads, pf_occupancy(fused_lds<BM, BN, WM, WN>() / kK, 0, 1))
void pf_fused(PfArgs rows_by_value, PfArgs lat_by_value) {
  (void)rows_by_value;
  (void)lat_by_value;
  const PfArgs* args = (const PfArgs*)__builtin_amdgcn_kernarg_segment_ptr();
  const PfArgs& rows = args[0];
  const PfArgs& lat = args[1];
  __shared__ __align__(1024) uint16_t raw[fused_lds<BM, BN, WM, WN>()];
  const int nlat = (lat.items + kXcds - 1) / kXcds * kXcds;
  const int b = blockIdx.x;
  if (b < nlat) {
    using TL = Tile<kPrefillLatentRows, 64, 2, 2>;
    pf_body<DT, K_LATENT, 64, kPrefillLatentRows, 64, 2, 2, kLatentStages>(
        lat, b, nlat, reinterpret_cast<uint16_t(*)[TL::LDS]>(raw));
  } else {
    using TR = Tile<BM, BN, WM, WN>;
    pf_body<DT, KIND, P, BM, BN, WM, WN, 2>(rows, b - nlat, (int)gridDim.x - nlat,
                                            reinterpret_cast<uint16_t(*)[TR::LDS]>(raw));
  }
}

// Row-kernel tiles: tall 256 × 64 (waves 4 × 1, 64 × 64 each; 80 KiB of LDS,
// two workgroups per compute unit), narrow 128 × 64 (waves 2 × 2, 64 × 32
// each; 48 KiB) and short 64 × 64 (waves 2 × 2, 32 × 32 each), all with two
// stages. The latent's tiles are 64 tokens × 64
// ranks (waves 2 × 2) with three stages.
template <int DT, int KIND, int P>
hipError_t launch_rows(const PfArgs& a, int G, hipStream_t s) {
  const int per_xcd = (a.items + kXcds - 1) / kXcds;
  const dim3 grid((unsigned)(per_xcd * kXcds)), blk(kPfThreads);
  if (G * P == 64 && a.bm == 256)
    hipLaunchKernelGGL((pf_gemm<DT, KIND, P, 256, 64, 4, 1, 2>), grid, blk, 0, s, a);
  else if (G * P == 64 && a.bm == 128)
    hipLaunchKernelGGL((pf_gemm<DT, KIND, P, 128, 64, 2, 2, 2>), grid, blk, 0, s, a);
  else if (G * P == 64 && a.bm == 64)
    hipLaunchKernelGGL((pf_gemm<DT, KIND, P, 64, 64, 2, 2, 2>), grid, blk, 0, s, a);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

template <int DT, int KIND>
hipError_t launch_rows_p(const PfArgs& rows, int P, int G, hipStream_t s) {
  if (rows.items == 0) return hipSuccess;
  switch (P) {
    case 16: return launch_rows<DT, KIND, 16>(rows, G, s);
    case 32: return launch_rows<DT, KIND, 32>(rows, G, s);
    case 64:
      if constexpr (DT != DT_F32) return launch_rows<DT, KIND, 64>(rows, G, s);
      break;  // fp32 steps are 32 columns: 64-wide blocks stream
  }
  return hipErrorInvalidValue;
}

// Latent and rows in one launch.
template <int DT, int KIND, int P>
hipError_t launch_fused_p(const PfArgs& rows, const PfArgs& lat, int G, hipStream_t s) {
  if (G * P != 64) return hipErrorInvalidValue;
  const int nlat = (lat.items + kXcds - 1) / kXcds * kXcds;
  const int per_xcd = (rows.items + kXcds - 1) / kXcds;
  const dim3 grid((unsigned)(nlat + per_xcd * kXcds)), blk(kPfThreads);
  if (rows.bm == 256)
    hipLaunchKernelGGL((pf_fused<DT, KIND, P, 256, 64, 4, 1>), grid, blk, 0, s, rows, lat);
  else if (rows.bm == 128)
    hipLaunchKernelGGL((pf_fused<DT, KIND, P, 128, 64, 2, 2>), grid, blk, 0, s, rows, lat);
  else if (rows.bm == 64)
    hipLaunchKernelGGL((pf_fused<DT, KIND, P, 64, 64, 2, 2>), grid, blk, 0, s, rows, lat);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

template <int DT>
hipError_t launch_fused(const PfArgs& rows, const PfArgs& lat, int P, int G, hipStream_t s) {
  switch (P) {
    case 16: return launch_fused_p<DT, K_ROWS_FUSED, 16>(rows, lat, G, s);
    case 32: return launch_fused_p<DT, K_ROWS_FUSED, 32>(rows, lat, G, s);
    case 64:
      if constexpr (DT != DT_F32) return launch_fused_p<DT, K_ROWS_FUSED, 64>(rows, lat, G, s);
      break;
  }
  return hipErrorInvalidValue;
}

}  // namespace

// Parts of fewer steps lose more to the exchange of partial tiles (a store,
// its acknowledgement, a count, a load: some µs) than they gain: 7B FFN
// 11008×4096 (32 steps a group) at 256 rows 41.1 µs whole, 53.7 in two parts;
// 4096×11008 (86 steps) 65.9 whole, 53.3 in two parts, 58.2 in three.
constexpr int64_t kRowSplitMinSteps = 40;
// Past half the CUs' worth of row groups, parts stack on compute units that
// already run one: two parts pay only when each is long or the latent is what
// they would otherwise wait for. Measured (whole -> auto parts, µs): 4096×11008
// with 64×64 blocks (86 steps a group, 172-step latent) at 384 / 512 rows 66.1
// -> 67.2 / 79.6 -> 66.7, at 640 (640 parts) 85.1 -> 96.9; with 16×16 (344
// steps) at 512 134.5 -> 95.8; 2048×5461 with 32×32 (86 steps, 86-step latent)
// at 512 / 640 / 768 rows 62.7 -> 56.1 / 65.2 -> 68.0 / 65.0 -> 70.6.
constexpr int64_t kRowSplitLongSteps = 64;

int prefill_row_split(int64_t items, int64_t steps, int64_t lat_steps, int n_cus, int bm) {
  if (bm >= 256) return 1;  // the tall tile keeps its registers for its own steps
  const int64_t forced = debug_knobs().prefill_split;  // test hook
  if (forced == 1) return 1;
  if (forced >= 2) return (int)forced;
  const int64_t slots = 2 * (int64_t)n_cus;
  if (items <= 0 || items >= slots) return 1;
  int64_t k = (slots + items - 1) / items;
  if (k > 4) k = 4;
  if (k > steps / kRowSplitMinSteps) k = steps / kRowSplitMinSteps;
  while (k >= 2 && k * items > slots) --k;
  if (k < 2) return 1;
  if (2 * items > n_cus && steps / k < kRowSplitLongSteps && 2 * lat_steps < 3 * steps) return 1;
  return (int)k;
}

// The latent's K chunks when the rows split: chunks of at least 16 steps, at
// most 256 latent workgroups in all, at most 16 chunks a tile, at most 64 rank
// tiles (their arrival words). LLaMA-7B FFN at 256 rows: 16 tiles; 4096
// in_features (64 steps) in 4 chunks, 11008 (172 steps) in 11.
PfLatentSplit prefill_latent_split(int64_t M, int64_t m_pad, int64_t r_pad, int dtype) {
  const int64_t ks = dtype == SSL_F32 ? 32 : 64;  // in_features per step
  const int64_t steps = m_pad / ks;
  const int64_t tiles = (M + kPrefillLatentRows - 1) / kPrefillLatentRows * (r_pad / 64);
  PfLatentSplit r{1, (int)steps};
  if (tiles <= 0 || steps <= 16 || r_pad / 64 > 64) return r;
  int64_t n = (steps + 15) / 16;
  if (n > 256 / tiles) n = 256 / tiles;
  if (n > 16) n = 16;
  if (n <= 1) return r;
  const int64_t chunk = (steps + n - 1) / n;
  r.split = (int)((steps + chunk - 1) / chunk);
  r.chunk = (int)chunk;
  return r;
}

// The latent's K chunks when the row groups run whole. A row workgroup waits
// for its token rows' latent tiles after its own sparse steps, so a latent
// longer than that (a call with few blocks, or none: S = 0) is the rows'
// critical path: its in_features split into chunks about a group's sparse
// steps long (at least 16 steps), at most twice the CUs' worth of latent
// workgroups, 16 chunks a tile and 64 rank tiles. Within 1.5 times a group's
// steps the exchange of partials would cost more than it saves.
PfLatentSplit prefill_latent_split_whole(int64_t M, int64_t m_pad, int64_t r_pad, int dtype,
                                         int64_t row_steps, int n_cus) {
  const int64_t ks = dtype == SSL_F32 ? 32 : 64;  // in_features per step
  const int64_t steps = m_pad / ks;
  const int64_t tiles = (M + kPrefillLatentRows - 1) / kPrefillLatentRows * (r_pad / 64);
  PfLatentSplit r{1, (int)steps};
  if (tiles <= 0 || r_pad / 64 > 64) return r;
  const int64_t target = row_steps > 16 ? row_steps : 16;
  if (2 * steps <= 3 * target) return r;
  int64_t n = (steps + target - 1) / target;
  if (n > 16) n = 16;
  if (n > 2 * (int64_t)n_cus / tiles) n = 2 * (int64_t)n_cus / tiles;
  if (n <= 1) return r;
  const int64_t chunk = (steps + n - 1) / n;
  r.split = (int)((steps + chunk - 1) / chunk);
  r.chunk = (int)chunk;
  return r;
}

int64_t prefill_split_bytes(int64_t M, int64_t NB, int block_p, int64_t m_pad, int64_t r_pad,
                            int dtype, int n_cus) {
  if (M < kPrefillMinM || NB <= 0) return 0;
  const int64_t groups = (NB + 64 / block_p - 1) / (64 / block_p);
  int64_t rows = 0;
  // row parts only while even the tall tile's grid gives fewer than two
  // workgroups per CU
  if (((M + 255) / 256) * groups < 2 * (int64_t)n_cus || debug_knobs().prefill_split != 0) {
    int64_t tiles = 4 * ((M + 63) / 64) * groups;  // part tiles: 4 parts of 64-row tiles at most
    if (tiles > 4 * (int64_t)n_cus) tiles = 4 * (int64_t)n_cus;  // automatic splits: < 4 CUs' worth
    rows = tiles * 128 * 64 * 4;  // at most 128 × 64 fp32 a part
  }
  // the latent's chunks: the most either policy takes (whole rows: a group
  // without sparse steps)
  int split = prefill_latent_split(M, m_pad, r_pad, dtype).split;
  const int whole = prefill_latent_split_whole(M, m_pad, r_pad, dtype, 0, n_cus).split;
  if (whole > split) split = whole;
  const int64_t lat = split > 1 ? prefill_latent_part_bytes(M, r_pad, split) : 0;
  return rows + lat;
}

int64_t prefill_latent_part_bytes(int64_t M, int64_t r_pad, int split) {
  return 4LL * kLatentPartFloats * split * ((M + kPrefillLatentRows - 1) / kPrefillLatentRows) *
         (r_pad / 64);
}

int prefill_group(int64_t M, int64_t n_rows, int block_p, int n_cus) {
  (void)M; (void)n_rows; (void)n_cus;
  return 64 / block_p;
}

int prefill_row_tile(int64_t M, int64_t n_rows, int group, int block_p, int n_cus, int dtype,
                     int64_t lat_items) {
  (void)block_p;
  const int64_t forced = debug_knobs().prefill_group;  // test hook
  if (forced == 1) return 128;
  if (forced == 2) return 256;
  if (forced == 3) return 64;
  const int64_t groups = (n_rows + group - 1) / group;
  const int64_t tall = ((M + 255) / 256) * groups, narrow = ((M + 127) / 128) * groups;
  // fp32 steps are latency bound (a quarter of the k of a 16-bit step per load
  // round trip): the short tile when the narrow one gives fewer than two
  // workgroups per compute unit (LLaMA-60M gate at 2048 rows: 58 -> 50 µs).
  if (dtype == SSL_F32 && narrow < 2 * n_cus) return 64;
  // A small grid: the short tile (64 × 64), twice the workgroups of the narrow
  // one (2048×2048 with 32×32 blocks at 256 rows: 26.0 -> 22.7 µs; 4096×4096
  // with 64×64 at 128 rows: 34.4 -> 31.7 µs).
  if (narrow < n_cus / 2) return 64;
  if (M <= 128) return 128;  // one token tile either way; the tall one's lower half past M
  // Rounds of the grid at the tile's workgroups per compute unit, the tall tile
  // (80 KiB of LDS: 2) against the narrow one (48 KiB: 3); a round of tall
  // workgroups moves 40 KiB a step per workgroup against 24 and costs about 1.2
  // narrow rounds. The latent's workgroups (first in the grid, short) count
  // against the narrow grid only: narrow rows that wait for their slots run a
  // whole round late, tall ones about a latent's length. Min of 3 graph
  // timings: 7B FFN 11008×4096 at 768 / 1024 rows narrow 78.5 / 92.0 µs, tall
  // 86.7 / 96.0; at 1280 / 2048 / 3072 tall 100.8 / 154.5 / 231.2, narrow
  // 114.1 / 168.1 / 245.4; 4096×11008 at 1536 / 2048 / 3072 rows tall 123.4 /
  // 169.9 / 236.1, narrow 169.6 / 195.0 / 285.2.
  return prefill_rounds_prefer_tall(tall, narrow + lat_items, n_cus) ? 256 : 128;
}

bool prefill_rounds_prefer_tall(int64_t tall, int64_t narrow, int n_cus) {
  if (debug_knobs().prefill_group != 0) return false;  // a forced tile stays
  const int64_t rt = (tall + 2 * n_cus - 1) / (2 * n_cus);
  const int64_t rn = (narrow + 3 * n_cus - 1) / (3 * n_cus);
  return 12 * rt <= 10 * rn;
}

hipError_t prefill_launch_fused(int dtype, int P, int G, const PfArgs& rows, const PfArgs& lat,
                                hipStream_t stream) {
  switch (dtype) {
    case SSL_BF16: return launch_fused<DT_BF16>(rows, lat, P, G, stream);
    case SSL_F16: return launch_fused<DT_F16>(rows, lat, P, G, stream);
    case SSL_F32: return launch_fused<DT_F32>(rows, lat, P, G, stream);
  }
  return hipErrorInvalidValue;
}

hipError_t prefill_launch_fused_nm24(int dtype, const PfArgs& rows, const PfArgs& lat,
                                     hipStream_t stream) {
  switch (dtype) {
    case SSL_BF16: return launch_fused_p<DT_BF16, K_ROWS_NM, 32>(rows, lat, 2, stream);
    case SSL_F16: return launch_fused_p<DT_F16, K_ROWS_NM, 32>(rows, lat, 2, stream);
  }
  return hipErrorInvalidValue;
}

hipError_t prefill_launch_op(int dtype, int P, int G, const PfArgs& rows, hipStream_t stream) {
  switch (dtype) {
    case SSL_BF16: return launch_rows_p<DT_BF16, K_ROWS_OP>(rows, P, G, stream);
    case SSL_F16: return launch_rows_p<DT_F16, K_ROWS_OP>(rows, P, G, stream);
    case SSL_F32: return launch_rows_p<DT_F32, K_ROWS_OP>(rows, P, G, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace ssl
