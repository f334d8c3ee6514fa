// Prefill-shaped SLR kernels (many token rows, 16-bit activations): the host
// interface between the C-ABI entry points and csrc/prefill.hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ssl {

// Calls with at least this many token rows (and 16-bit activations) take the
// LDS-tiled prefill kernels; fewer rows take the row-streaming decode kernel.
constexpr int64_t kPrefillMinM = 128;
// Copies of each latent tile counter, one per wave of a row workgroup, each in
// its own 512-byte slot: every wave of every row workgroup of a token tile
// polls its counter when it reaches its low-rank steps, and workgroups that
// started together get there together; with one word those polls queue at one
// memory location.
// A slot's word 0 counts the latent tiles written for its token tile, word
// kPfDepartWord the waiters that have passed; the last waiter returns both to
// zero, so the slots (in the call's zero-at-rest counters) need no clearing
// between launches.
constexpr int kPfCntCopies = 4;
constexpr int kPfCntStride = 128;
constexpr int kPfDepartWord = 32;

enum : int { PF_OP = 0, PF_FUSED = 1 };

struct PfMember {
  void* y;
  int64_t ldy;
  const void* A;        // [NB·p][r_pad]
  int64_t lda;
  int64_t A_bytes;
  const void* bias;
  const void* values_pq;  // the block values in (nnz, p, q) order (k-contiguous per column)
  int64_t values_bytes;
  const int32_t* groups;  // prefill plan: (2 + G) int32 per group
  const int32_t* steps;   // prefill plan: ssl_prefill_step_ints(p, G) int32 per step
  int n_groups;
  const void* B;        // [r_pad][m_pad]
  int64_t ldb;
  void* t;              // latent [M][r_pad], activation dtype
  int64_t ldt;
  int32_t* tcnt;        // latent tiles written, per latent token tile, in
                        // kPfCntCopies copies kPfCntStride int32 apart (zero at
                        // rest; the low-rank steps wait on them)
  int r_pad;
  // K parts (prefill_row_split): rows kernels split a row group's sparse steps
  // into ksplit parts (the last also takes the low-rank steps), the latent its
  // in_features into ksplit chunks of kchunk steps; every part stores its fp32
  // partial tile in kpart and counts itself, and the last to arrive sums the
  // parts in part order (the same sum whichever arrives last) and goes on.
  int ksplit, kchunk;
  float* kpart;         // ksplit > 1: [tile][part][tile elements] fp32
  int32_t* karrive;     // rows, ksplit > 1: parts arrived per (token tile,
                        // group), zero at rest (the latent's arrivals use
                        // words kPfLatArriveWord + rank tile of its tile
                        // counters' first slot)
  // Rows: a part table (ssl_prefill_parts_build) instead of `ksplit` equal
  // parts of every group: n_parts records per token tile, kPartInts int32
  // each, {group, step_begin, step_end, part, parts, first split part}. The
  // partial tiles of split groups sit at kpart [token tile][split_parts],
  // the arrivals at karrive [token tile][group].
  const int32_t* parts;
  int n_parts, split_parts;
  int NB;               // block-rows (bounds the group records' rows)
};

struct PfArgs {
  const void* x;
  int64_t ldx;
  int M, m, m_pad;
  int mode;             // PF_OP: y += x·Sᵀ on planned rows; PF_FUSED: the SLR linear
  int n;                // members
  int items;            // workgroups that do work
  int bm;               // rows kernels: token rows per tile (prefill_row_tile)
  int lbm;              // token rows per latent tile (kPrefillLatentRows)
  uint64_t* status;     // set to 1 when a bounded wait gives up
  int polls;            // polls before a wait gives up
  int wait_bias;        // added to every wait's target (test hook: out of reach)
  int off[5];           // first item of each member
  PfMember mb[4];
};

// int32 per record of a prefill part table.
constexpr int kPartInts = 8;

// Token rows per latent tile of the prefill kernels.
constexpr int kPrefillLatentRows = 64;
constexpr int kPfLatArriveWord = 64;  // rank tiles ≤ 64 (r_pad ≤ 4096) for a latent split

// K parts of a fused prefill call with few row workgroups: a grid of `items`
// row workgroups under twice the CUs splits each row group's sparse steps in
// up to 4 parts (at least 40 steps a part, `steps` the mean per group, the
// parts at most twice the CUs; past half the CUs' worth of groups only parts
// of 64 steps or more, or when the latent's steps are 1.5 times the group's),
// and then the latent's in_features too (prefill_latent_split), so neither
// leaves the other's critical path. 1 = no split.
// lat_steps: the latent's steps over in_features.
int prefill_row_split(int64_t items, int64_t steps, int64_t lat_steps, int n_cus, int bm);
struct PfLatentSplit {
  int split, chunk;
};
PfLatentSplit prefill_latent_split(int64_t M, int64_t m_pad, int64_t r_pad, int dtype);
// The latent's K chunks when the row groups run whole (no K parts): split when
// the latent is longer than 1.5 times a group's sparse steps (`row_steps`, the
// member's mean), into chunks about that long.
PfLatentSplit prefill_latent_split_whole(int64_t M, int64_t m_pad, int64_t r_pad, int dtype,
                                         int64_t row_steps, int n_cus);
// Bytes of the latent's fp32 partial tiles in `split` chunks.
int64_t prefill_latent_part_bytes(int64_t M, int64_t r_pad, int split);
// Workspace bytes the partial tiles of both splits may take for a member.
int64_t prefill_split_bytes(int64_t M, int64_t NB, int block_p, int64_t m_pad, int64_t r_pad,
                            int dtype, int n_cus);

// Row-kernel tiles (token rows × output features): narrow 128 × 64, tall
// 256 × 64 and short 64 × 64; a workgroup owns 64 / p block-rows.
// Block-rows per row-kernel workgroup (64/p).
int prefill_group(int64_t M, int64_t n_rows, int block_p, int n_cus);
// Token rows per row-kernel workgroup (64, 128 or 256) for that group size;
// lat_items: the latent's workgroups in the same launch.
int prefill_row_tile(int64_t M, int64_t n_rows, int group, int block_p, int n_cus, int dtype,
                     int64_t lat_items);
// Whether `tall` workgroups of the tall tile (2 a compute unit) finish before
// `narrow` workgroups of the narrow one (3 a compute unit, the latent's
// included); false while a test forces the tile.
bool prefill_rounds_prefer_tall(int64_t tall, int64_t narrow, int n_cus);
// The fused SLR linear in one launch: the latent GEMM's workgroups (`lat`, one per 64-token
// × 64-rank tile over all of in_features) first in the grid, then the row
// GEMM's (`rows`), whose low-rank steps wait for their token rows' latent
// tiles. dtype: SSL_F32, SSL_BF16 or SSL_F16; P ∈ {16, 32, 64}; G = 64/P.
hipError_t prefill_launch_fused(int dtype, int P, int G, const PfArgs& rows, const PfArgs& lat,
                                hipStream_t stream);
// The fused SLR linear with 2:4 S (32×32 blocks in the row kernel's layout,
// kNmPrefillBlockBytes each): latent, combine, then the row GEMM on
// v_smfmac_f32_16x16x64. dtype: SSL_BF16 or SSL_F16; G = 2.
hipError_t prefill_launch_fused_nm24(int dtype, const PfArgs& rows, const PfArgs& lat,
                                     hipStream_t stream);
constexpr int kNmPrefillBlockBytes = 32 * 2 * 16 + 32 * 4;
// The in-place op: the row GEMM only (rows.mode = PF_OP).
hipError_t prefill_launch_op(int dtype, int P, int G, const PfArgs& rows, hipStream_t stream);

}  // namespace ssl
