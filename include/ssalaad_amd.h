/*
 * ssalaad_amd.h — C ABI of the MI355X (gfx950) sparse-plus-low-rank linear library.
 *
 *   y = x · Bᵀ · Aᵀ  +  x · Sᵀ  +  b        (S block-sparse, BSR layout)
 *
 * Every entry point takes raw device pointers, sizes and a hipStream_t passed as
 * `void*`; none allocates device memory. Kernel entry points are asynchronous and
 * ordered on `stream`. Scratch is supplied by the caller in two parts:
 *   counters  int32 array sized by the *_counter_count query. It must be zero
 *             before the first call; every call that completes leaves it zero.
 *             Keep it for counters only (never alias it with data).
 *   workspace bytes sized by the *_workspace_size query (256-byte aligned); no
 *             initialisation needed. For ssl_slr_forward and its group, many-token
 *             calls with a small grid may run their row groups in parts whose fp32
 *             partial tiles take room the query includes; a workspace with less
 *             (but at least what the call needs without them) runs them whole.
 * Calls that share scratch must be ordered (same stream); concurrent calls on the
 * same scratch race.
 *
 * Return value: 0 (SSL_OK) or one of the ssl_status codes below. HIP launch
 * failures are reported as SSL_ERR_HIP; ssl_last_error() returns a message.
 *
 * Tensor conventions (all row-major, last dimension contiguous):
 *   x       [M, ldx]   activations; the first m columns are used
 *   out/y   [M, ldy]
 *   crow    [NB + 1]   int32 block-row pointer            (BSR crow_indices)
 *   col     [nnz]      int32 block-column index           (BSR col_indices)
 *   values  [nnz, q, p] block values, each block TRANSPOSED to (q, p) — the layout
 *                      the reference module stores in S_values
 *   active  [n_active] int32 block-rows that are updated, ascending
 *   A       [n_pad, r_pad], B [r_pad, m_pad]  low-rank factors, zero-padded
 *   bias    [n_pad]
 */
#ifndef SSALAAD_AMD_H
#define SSALAAD_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  SSL_OK = 0,
  SSL_ERR_INVALID = 1,     /* bad pointer, size or stride (maps to ValueError)   */
  SSL_ERR_UNSUPPORTED = 2, /* dtype / block shape without a kernel (TypeError)   */
  SSL_ERR_WORKSPACE = 3,   /* workspace missing or too small                     */
  SSL_ERR_HIP = 4,         /* HIP runtime error (RuntimeError)                   */
  SSL_ERR_CAPACITY = 5     /* caller-provided host array too small               */
} ssl_status;

typedef enum { SSL_F32 = 0, SSL_BF16 = 1, SSL_F16 = 2 } ssl_dtype;

/* Library version and last error message (thread-local, valid until next call). */
int ssl_version(void);
const char* ssl_last_error(void);

/* A status word in host memory that kernels can write (no reference
 * counterpart: the reference's kernels have no bounded waits to report). It
 * allocates 256 bytes of pinned, coherent host memory, zeroed, that every GPU
 * can address, and returns its host address and the device address kernels
 * take (pass it as ssl_slr_member.status). A workgroup that gives up a bounded
 * wait stores 1 into its first uint64, and the store is visible to the host
 * as soon as it lands, so a host can check the word before each call with a
 * plain read instead of a copy and a synchronisation. The memory lives until
 * the process ends; the host clears the word itself. This is the one call of
 * the library that allocates; it is made once per process or device, outside
 * any graph capture. */
int ssl_status_word_alloc(void** host_ptr, void** device_ptr);

/* Test hooks (host-side process-wide settings read at each launch; no
 * reference counterpart). They exist so that tests can reach paths that a
 * healthy device never takes, with every kernel still ending normally:
 *   SSL_DEBUG_PREFILL_TILE      0: the library picks the prefill row tile;
 *                               1: always the narrow tile (128 token rows ×
 *                               64 output features); 2: always the tall one
 *                               (256 × 64); 3: always the short one (64 × 64).
 *                               Any of them also sends fp32 calls of
 *                               ssl_prefill_min_rows() rows or more to the
 *                               prefill kernels whatever their size.
 *   SSL_DEBUG_WAIT_POLLS        polls before a bounded wait gives up (0: the
 *                               default of several seconds).
 *   SSL_DEBUG_WAIT_UNREACHABLE  nonzero: every wait of the fused kernel targets
 *                               a count no launch reaches, so each gives up
 *                               after its polls and reports it.
 *   SSL_DEBUG_PREFILL_SPLIT     0: the library decides whether a fused
 *                               prefill call splits its row groups' sparse
 *                               steps (and its latent's in_features) across
 *                               workgroups; 1: never; 2 to 4: every fused
 *                               prefill call splits its row groups in that
 *                               many parts (when the caller's workspace holds
 *                               the partial tiles).
 *   SSL_DEBUG_CHAIN_FRAG        0: the library decides whether a chained launch
 *                               of 32- or 64-wide blocks passes its stages'
 *                               inputs in fragment order (ssl_slr_stage.xf);
 *                               1: never (one-tile calls); 2: always.
 *   SSL_DEBUG_TOPK_GROUPS       0: ssl_block_topk picks its select; 1: one
 *                               workgroup; 2: many workgroups.
 * Not for concurrent use with calls on other threads. */
typedef enum {
  SSL_DEBUG_PREFILL_TILE = 0,
  SSL_DEBUG_WAIT_POLLS = 1,
  SSL_DEBUG_WAIT_UNREACHABLE = 2,
  SSL_DEBUG_PREFILL_SPLIT = 3,
  SSL_DEBUG_CHAIN_FRAG = 4,
  SSL_DEBUG_TOPK_GROUPS = 5
} ssl_debug_knob;
int ssl_debug_set(int32_t knob, int64_t value);

/* Device bounds checks (no reference counterpart): 1 in the library's checked
 * build (compiled with SSL_DEVICE_CHECKS=1, libssalaad_amd_checked.so), 0 in
 * the normal one. A checked build re-checks on the device every index the
 * kernels read from a plan, a column array or a prefill group, step or part
 * record; one outside what the call's plan can hold is dropped or clamped (the
 * kernel still ends normally) and recorded as bit 8 + code of the call's
 * status word (ssl_slr_member.status, or the plan's first exchange word):
 * code 0 a streaming plan entry, 1 a column index (negative, or, for the
 * in-place op, past x; the fused linear reads columns past in_features as
 * zeros), 2 a prefill group's
 * block-row, 3 a prefill step's x column or block, 4 a prefill part record.
 * Calls that pass no status word (the in-place op) record in a word of the
 * library's own, which ssl_debug_check_word returns and clears (synchronous;
 * always 0 in the normal build, -1 on a HIP error). */
int32_t ssl_device_checks(void);
int64_t ssl_debug_check_word(void);

/* -------------------------------------------------------------------------
 * Work plans (host side, integer only).
 *
 * A plan splits the work of one BSR matrix into workgroup chunks. Each block-row
 * owns its sparse blocks (cost q each) and `lr_units` low-rank units (cost 32
 * each, 32 ranks of A per unit). A row whose cost exceeds `target_cost` is split
 * into k chunks of nearly equal cost. Without low-rank units chunk j takes the
 * j-th consecutive share of the row's blocks; with them the row's last chunk
 * (its finaliser, listed after every other chunk of the table) takes all the
 * low-rank units and a smaller share of blocks. The k partial results are summed
 * in chunk order on the device, so long rows of skewed matrices are spread
 * across workgroups and results stay deterministic. `rows` lists the
 * block-rows that get chunks (NULL = every row 0..NB-1). target_cost <= 0 never
 * splits.
 *
 * Table layout: SSL_PLAN_STRIDE int32 per chunk:
 *   {row, blk_begin, blk_end, lr_begin, lr_end, seq, nseq, slot}
 * (blk_* index the BSR block arrays; lr_* count 32-rank units of the row).
 * Returns the chunk count in *n_chunks and the partial-sum slot count in *n_slots.
 * The structure is checked first (SSL_ERR_INVALID otherwise): crow starts at 0
 * and never decreases, each of the crow[NB] blocks has col in [0, NBK) (col may
 * be NULL only without blocks), and `rows` is strictly ascending in [0, NB).
 * The kernels index with these numbers unchecked, so callers build a plan from
 * the same crow/col they pass to the device.
 * ------------------------------------------------------------------------- */
#define SSL_PLAN_STRIDE 8
int ssl_plan_build(const int32_t* crow_host, const int32_t* col_host, int64_t NB, int64_t NBK,
                   const int32_t* rows_host, int64_t n_rows, int32_t block_q, int32_t lr_units,
                   int64_t target_cost, int32_t* table_out, int64_t table_capacity,
                   int64_t* n_chunks, int64_t* n_slots);

/* Prefill plan (host side, integer only): the row kernels used for calls with
 * many token rows give one workgroup `group` block-rows at once (group · p =
 * 64 output features) and walk the union of their block columns in steps of
 * step_cols columns (64 for 16-bit activations, 32 for fp32: 128 bytes of a
 * row either way), E = step_cols / p union entries per step, so each tile of
 * x feeds every block of that column in the group. Groups are consecutive runs
 * of `group` listed rows (`rows` NULL = every row 0..NB-1).
 *   groups  (2 + group) int32 per group:  {step_begin, step_end, row_0 .. row_{group-1}}
 *           (row −1: none; the last group may be short)
 *   steps   ssl_prefill_step_ints(p, group, step_cols) int32 per step:
 *           {mask, col_0 .. col_{E-1}, W[4][IB][E]}
 *           col_e: first x column of entry e (−1 past the last entry);
 *           W[w][i][e] = blk[e][(8·(w + 4i)) / p]: the BSR block index of that
 *           slot's row at entry e's column, or −1 (IB = group·p / 32: the row
 *           kernel's 4 waves each load IB runs of 8 weight rows per step, and
 *           each finds its block indices in one place);
 *           mask bit (h·group + g): slot g holds a block in half h (h = 0, 1)
 *           of the step's columns. Entries ascend by column; a column repeated
 *           within one row starts another entry. Padding words are −1.
 * Call once with NULL outputs for the counts. step_cols ∈ {32, 64}, p divides
 * step_cols and group · p = 64 (the row kernel's tiles;
 * ssl_prefill_step_ints is 0 otherwise). The structure is checked as for
 * ssl_plan_build. */
int32_t ssl_prefill_step_ints(int32_t block_p, int32_t group, int32_t step_cols);
/* Balanced K parts of a prefill plan's row groups (no reference counterpart:
 * the reference walks each block-row serially,
 * ssalaad/tilelang_sparse/addmm_inplace.py:74). A row workgroup runs its
 * group's sparse steps in a row, so with a skewed structure (per-row block
 * counts far from even) the longest group sets the time of a call whose row
 * workgroups all fit on the device at once. From the group table of
 * ssl_prefill_plan_build (n_groups records of 2 + group int32), this cuts every
 * group into parts of about the mean group's steps (at least 32, at most 16
 * parts a group), when the longest group holds more than twice that; else it
 * returns no records (*n_parts = 0). Records are 8 int32 each, in group order:
 * {group, step_begin, step_end, part, parts, first split part, 0, 0};
 * *split_parts counts the parts of the groups cut in more than one. Call with
 * NULL output for the counts. */
int ssl_prefill_parts_build(const int32_t* groups_host, int64_t n_groups, int32_t group,
                            int32_t* parts_out, int64_t parts_capacity, int64_t* n_parts,
                            int64_t* split_parts);
/* Workspace bytes the partial tiles of split_parts parts take in a call of M
 * token rows (fp32 tiles of up to 128 token rows × 64 output features). */
int64_t ssl_prefill_parts_bytes(int64_t M, int64_t split_parts);
int ssl_prefill_plan_build(const int32_t* crow_host, const int32_t* col_host, int64_t NB,
                           int64_t NBK, const int32_t* rows_host, int64_t n_rows, int32_t block_p,
                           int32_t group, int32_t step_cols, int32_t* groups_out,
                           int64_t groups_capacity, int32_t* steps_out, int64_t steps_capacity,
                           int64_t* n_groups, int64_t* n_steps);
/* Calls with at least this many token rows run the prefill kernels (16-bit
 * activations with 16/32/64 square blocks, fp32 with 16/32), which need a
 * prefill plan built with this group size for the call's M and row count
 * (n_rows: the rows the plans list; for a grouped call, all its linears' rows
 * together). ssl_prefill_step_cols gives the plan's step width for a dtype. */
int32_t ssl_prefill_step_cols(int32_t dtype);
int64_t ssl_prefill_min_rows(void);
int32_t ssl_prefill_group(int64_t M, int64_t n_rows, int32_t block_p, int32_t block_q);
/* 1 if a fused SLR call (ssl_slr_forward, ssl_slr_forward_group) with block
 * storage, M token rows and n_rows block-rows over all its linears takes the
 * prefill kernels (and so needs their plans), 0 if it streams. Only square
 * 16/32/64 blocks (fp32: 16/32) take them, from ssl_prefill_min_rows() rows:
 * 16-bit calls always, except calls of exactly that many rows (one token tile)
 * with at most 2048 output features (n_rows · block_p ≤ 2048), which stream;
 * fp32 calls when the grid of 64-row tiles, ceil(M / 64) · ceil(n_rows /
 * (64 / block_p)) workgroups, reaches the device's compute-unit count. A
 * forced row tile (SSL_DEBUG_PREFILL_TILE) sends every such call there. The
 * in-place op decides with ssl_bsr_addmm_takes_prefill instead. */
int32_t ssl_slr_takes_prefill(int64_t M, int64_t n_rows, int32_t block_p, int32_t block_q,
                              int32_t dtype);

/* -------------------------------------------------------------------------
 * In-place BSR addmm:  out[:, rows of active block-rows] += x · Sᵀ
 *
 * Replaces the TileLang op body
 *   ssalaad/tilelang_sparse/addmm_inplace.py:41-82 (_bsr_body) and :88-127
 *   (_tilelang_bsr_addmm_inplace_dense_impl), schema at :130-136,
 * and computes what the AVX2 kernel ssalaad/cpu_sparse/bsr_addmm_avx2.cpp:67-174
 * computes: for each planned block-row `by`, acc = out[:, by·p : by·p+p] in fp32,
 * plus Σ_blocks x[:, col·q : col·q+q] · values[blk]  (values blocks are (q, p)),
 * stored back in the out dtype. Block-rows without a chunk are not touched.
 * Blocks: p ∈ {16, 32, 48, 64} output features, q any multiple of 16 up to
 * 256 input features (square or not); dtype ∈ {f32, bf16, f16} for out, x and
 * values alike. `plan` is a device copy of a table from ssl_plan_build
 * (lr_units = 0). Calls for which ssl_bsr_addmm_takes_prefill(M, n_chunks, p, q,
 * dtype) is 1 (n_chunks: the plan's, its rows at M > 64) run the prefill kernel instead: they need `pf_groups`/`pf_steps`
 * (device copies from ssl_prefill_plan_build with the same rows and group =
 * pf_group = ssl_prefill_group(M, rows, p, q)) and `values_pq`, the block
 * values in (nnz, p, q) order (each block transposed); other calls may pass
 * NULL/0 there.
 * ------------------------------------------------------------------------- */
int32_t ssl_bsr_addmm_takes_prefill(int64_t M, int64_t n_rows, int32_t block_p,
                                    int32_t block_q, int32_t dtype);
int64_t ssl_bsr_addmm_workspace_size(int64_t M, int64_t NB, int32_t block_p,
                                     int64_t n_slots);
int64_t ssl_bsr_addmm_counter_count(int64_t M, int64_t NB);
int ssl_bsr_addmm_inplace(void* out, int64_t ldo, const void* x, int64_t ldx,
                          const int32_t* col, const void* values, int64_t nnz,
                          const int32_t* plan, int64_t n_chunks, int64_t n_slots,
                          const void* values_pq, const int32_t* pf_groups,
                          const int32_t* pf_steps,
                          int64_t pf_n_groups, int32_t pf_group, int64_t M, int64_t N,
                          int64_t K, int64_t NB, int32_t block_p, int32_t block_q,
                          int32_t dtype, int32_t* counters, int64_t n_counters,
                          void* workspace, int64_t workspace_bytes, void* stream);

/* -------------------------------------------------------------------------
 * Fused SLR linear:  y[M, n_pad] = x · Bᵀ · Aᵀ + x · Sᵀ + bias   (one launch)
 *
 * Replaces the forward of the reference module
 *   ssalaad/efficient/ls_linear.py:124-137 (_LRSLinearLRBlockCUDA.forward: two
 *   F.linear GEMMs :131, the BSR op :132-134, the bias add :41-44, :135-137) and
 *   ssalaad/efficient/ls_linear.py:50-51 (_LRSLinearLR, S = 0: pass nnz = 0).
 * The latent t = x·Bᵀ is rounded to the activation dtype, as F.linear does, then
 * t·Aᵀ, the sparse term and the bias are summed in fp32 and rounded once.
 * m ≤ ldx columns of x are read; A is [n_pad = NB·p, r_pad], B is [r_pad, m_pad]
 * with r_pad a multiple of 64 and m_pad ≥ m a multiple of 64; padding is zero.
 * `plan` comes from ssl_plan_build with lr_units = r_pad / 32 and rows = NULL;
 * `lr_wgs` counts the plan's chunks with low-rank units (lr_end > lr_begin).
 * `bias` may be NULL. y must hold M rows of n_pad columns (ldy ≥ n_pad).
 * `counters` (ssl_slr_counter_count int32) start at zero and are zero again when
 * the launch ends; they may be shared by calls ordered on one stream.
 * `exchange` (ssl_slr_exchange_size bytes, 256-byte aligned) belongs to one plan:
 * uint64 handshake words, zeroed when the plan is made, then advanced by every
 * call with that plan and never reset; calls with one plan must be ordered on
 * one stream, and the area must never be shared with another plan. Its first
 * uint64 is set to 1 if a workgroup gave up waiting (never expected; the host
 * may check it after synchronising). A zeroed area is always a valid state
 * (e.g. after growing it).
 * Calls for which ssl_slr_takes_prefill(M, NB, block_p, block_q, dtype) is 1
 * return SSL_ERR_INVALID before any launch: they need the prefill plans, which
 * only ssl_slr_forward_group takes (the pf_* fields of ssl_slr_member).
 * ------------------------------------------------------------------------- */
int64_t ssl_slr_workspace_size(int64_t M, int64_t NB, int32_t block_p, int64_t r_pad,
                               int64_t m_pad, int64_t n_slots, int32_t dtype);
int64_t ssl_slr_counter_count(int64_t M, int64_t NB);
int64_t ssl_slr_exchange_size(int64_t M, int64_t r_pad, int64_t m_pad, int32_t dtype);
int ssl_slr_forward(void* y, int64_t ldy, const void* x, int64_t ldx, const void* A,
                    const void* B, const void* bias, const int32_t* col,
                    const void* values, const int32_t* plan, int64_t n_chunks,
                    int64_t n_slots, int64_t lr_wgs, int64_t M, int64_t m, int64_t m_pad,
                    int64_t NB, int64_t r_pad, int32_t block_p, int32_t block_q,
                    int32_t dtype, int32_t* counters, int64_t n_counters, void* exchange,
                    int64_t exchange_bytes, void* workspace, int64_t workspace_bytes,
                    void* stream);

/* ssl_slr_forward with no caller scratch and no allocation. No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, hosts that forbid hipMalloc).
 * The counters, handshake words and workspace come from a file-scope device
 * array of ssl_slr_noalloc_scratch_bytes() (16 MiB) that each GPU the library
 * runs on holds until the process ends: at most 256 KiB of row counters, 512
 * KiB of handshake words and 15.25 MiB of workspace, as the *_counter_count,
 * *_exchange_size and *_workspace_size queries compute them for the call;
 * beyond that the call returns SSL_ERR_CAPACITY before any launch. Each call
 * first clears the counters and handshake words it uses (a fill kernel on
 * `stream`, then the fused launch), so calls with different plans may follow
 * one another; calls that overlap on one GPU (other streams or threads) race on
 * the shared array. A wait that gave up is recorded in the first handshake word
 * (cleared by the next call). Same arguments, limits and results as
 * ssl_slr_forward otherwise: calls for which ssl_slr_takes_prefill(M, NB,
 * block_p, block_q, dtype) is 1 need the prefill plans, which this entry point
 * does not take, and return SSL_ERR_INVALID before any launch. */
int64_t ssl_slr_noalloc_scratch_bytes(void);
int ssl_slr_forward_noalloc(void* y, int64_t ldy, const void* x, int64_t ldx, const void* A,
                            const void* B, const void* bias, const int32_t* col,
                            const void* values, const int32_t* plan, int64_t n_chunks,
                            int64_t n_slots, int64_t lr_wgs, int64_t M, int64_t m, int64_t m_pad,
                            int64_t NB, int64_t r_pad, int32_t block_p, int32_t block_q,
                            int32_t dtype, void* stream);

/* One linear of a fused call (the arguments of ssl_slr_forward that differ
 * between linears reading the same x). */
typedef struct ssl_slr_member {
  void* y;
  int64_t ldy;
  const void* A;
  const void* B;
  const void* bias;
  const int32_t* col;
  const void* values;
  const int32_t* plan;
  int64_t n_chunks;
  int64_t n_slots;
  int64_t lr_wgs;
  int64_t NB;
  int64_t r_pad;
  int32_t* counters;
  int64_t n_counters;
  void* exchange;
  int64_t exchange_bytes;
  void* workspace;
  int64_t workspace_bytes;
  /* prefill plan (ssl_prefill_plan_build with group = ssl_prefill_group(M,
   * rows of every linear of the call, p, q)): needed when
   * ssl_slr_takes_prefill is 1 for the call */
  const int32_t* pf_groups;
  const int32_t* pf_steps;
  int64_t pf_n_groups;
  int32_t pf_group;
  int64_t nnz;            /* stored blocks (length of col, first dim of values) */
  const void* values_pq;  /* for the prefill kernels: the block values in (nnz, p, q) order;
                           * 2:4 storage: the blocks in the prefill layout
                           * (ssl_nm24_prefill_block_bytes) */
  /* storage of `values`: SSL_S_BSR, (nnz, q, p) blocks (the reference module's
   * layout), or SSL_S_NM24, 2:4-sparse 32×32 blocks in the layout below
   * (replaces the semi-structured S of ssalaad/efficient/ls_linear.py:167-219) */
  int32_t s_format;
  /* where a workgroup that gave up waiting records it (uint64, set to 1;
   * device memory or the device address from ssl_status_word_alloc, never
   * cleared by the library). NULL: the first uint64 of `exchange`. Sharing one
   * word between every call lets a host check all of them at once. */
  uint64_t* status;
  /* optional, prefill kernels with block storage: the part table of the
   * prefill plan (a device copy of ssl_prefill_parts_build's records for the
   * same pf_groups), NULL for none. A call whose row groups would otherwise
   * run whole then gives each workgroup one record: the long groups of a
   * skewed structure run in parts of about the mean group's steps, summed in
   * part order by the last part to arrive. It needs ssl_prefill_parts_bytes(M,
   * pf_split_parts) more workspace bytes past ssl_slr_workspace_size's; with
   * less, or when the call splits every group evenly instead, the table is
   * not used. */
  const int32_t* pf_parts;
  int64_t pf_n_parts;
  int64_t pf_split_parts;
} ssl_slr_member;

typedef enum { SSL_S_BSR = 0, SSL_S_NM24 = 1 } ssl_s_format;

/* Bytes of one packed 2:4 block (32 input features × 32 output features):
 *   values [16][16][2] of the activation dtype: [c][i][s] = the i-th kept value,
 *          in increasing input feature order, of output column 2c + s (two kept
 *          values per group of four input features: group i / 2, slot i % 2);
 *   index  [16][8][2] bytes: [c][grp][s] = i0 | i1 << 2, the positions (0..3,
 *          i0 < i1) of the two kept values of group grp in output column 2c + s.
 * A group with fewer than two non-zeros keeps zeros at unused positions. */
int64_t ssl_nm24_block_bytes(void);

/* Bytes of one 2:4 block in the layout the prefill row kernel reads (the
 * operands of v_smfmac_f32_16x16x64), the same blocks in the same order:
 *   values [32][2][8] of the activation dtype: [j][h][t] = kept value 8h + t
 *          of output column j (input features 16h .. 16h + 15: four groups,
 *          two kept values each, group by group);
 *   index  [32] uint32: bits 16h + 4q .. 16h + 4q + 3 = i0 | i1 << 2 of
 *          group 4h + q of output column j.
 * Calls with ssl_nm24_takes_prefill(M, n_rows, dtype) = 1 pass these as the
 * member's values_pq, with a prefill plan (group 2, 64-column steps) over the
 * 2:4 block structure. */
int64_t ssl_nm24_prefill_block_bytes(void);
int32_t ssl_nm24_takes_prefill(int64_t M, int64_t n_rows, int32_t dtype);

/* Up to 4 SLR linears that read the same x (e.g. a layer's q, k and v
 * projections, or its gate and up projections) in ONE launch: each member is
 * computed exactly as ssl_slr_forward computes it (same rounding points), with
 * its own plan, counters, exchange area and workspace. Replaces nothing in the
 * reference (which calls each module on its own); it is the launch-count
 * reduction a decode step needs. All members share dtype and block size. */
int ssl_slr_forward_group(const void* x, int64_t ldx, int64_t M, int64_t m, int64_t m_pad,
                          int32_t block_p, int32_t block_q, int32_t dtype,
                          const ssl_slr_member* members, int32_t n_members, void* stream);

/* Chained launch: up to 4 dependent stages of grouped SLR linears (up to 8
 * linears in all) in ONE launch, e.g. a decoder layer's q,k,v -> o -> gate,up
 * -> down projections at decode. Stage 0 reads the launch's input x; every
 * later stage reads the output (y) of one member of an earlier stage, `src`,
 * as it is written inside the launch: its workgroups start their weight loads,
 * wait (bounded) until src has finished every output row tile of their token
 * tile, then read x device-coherently. Each member is computed as
 * ssl_slr_forward_group computes it for its stage's members alone (same plans
 * and rounding points); stage 0 also takes the same latent split, so its
 * outputs equal the grouped launch's bit for bit, while later stages compute
 * each latent tile over all of in_features in one workgroup (the fp32 sums of
 * t = x·Bᵀ then run in another order). Replaces nothing in the reference (its model calls
 * every module on its own, ssalaad/efficient/model.py:41-57); it removes the
 * kernel boundaries between a layer's projections, which dominate decode.
 *
 * Restrictions: bf16 or fp16; square 16/32/64 blocks or 2:4 storage; calls
 * the streaming kernel takes (for every stage, ssl_slr_takes_prefill /
 * ssl_nm24_takes_prefill is 0; otherwise SSL_ERR_UNSUPPORTED, and the caller
 * launches the stages one by one). A src member's output is stored
 * device-coherently and must lie within 2 GiB (M · ldy · element size).
 * Stage `sync` words: ssl_slr_chain_sync_count(M) int32, zero at rest, owned
 * by the stage; the launch returns them to zero (also after a wait that gave
 * up, which the members' status word reports). Calls that share sync words,
 * or any member's counters, exchange area or workspace, must be ordered on
 * one stream. */
#define SSL_MAX_CHAIN_STAGES 4
typedef struct ssl_slr_stage {
  const void* x;   /* stage 0: the launch's input; later stages: NULL or src's y */
  int64_t ldx;     /* stage 0: x's row stride (later stages use src's ldy) */
  int64_t m;       /* in_features of the stage's members (≤ src's NB · p) */
  int64_t m_pad;   /* in_features padded to a multiple of 64 (B's row stride) */
  int32_t first;   /* the stage's members: members[first .. first + count) */
  int32_t count;
  int32_t src;     /* later stages: index of the member whose output is x; -1 for stage 0 */
  int32_t* sync;   /* later stages: ssl_slr_chain_sync_count(M) zeroed int32 words,
                    * 256-byte aligned */
  int64_t n_sync;
  void* xf;        /* later stages of calls of 6 or more token rows with 32- or 64-wide
                    * blocks (ignored otherwise, may be NULL then): room for a second
                    * copy of src's output in MFMA-fragment order, which src writes and
                    * this stage reads (contiguous 1 KiB loads instead of 16 row
                    * segments): ssl_slr_chain_frag_bytes(M, src's NB · block_p) bytes,
                    * 256-byte aligned, no initial contents needed */
  int64_t xf_bytes;
} ssl_slr_stage;

int64_t ssl_slr_chain_sync_count(int64_t M);
/* Bytes of a fragment-order copy (ssl_slr_stage.xf) of an M-row output with
 * n_out features: 1 KiB per 16 token rows (in whole tiles of the call) and 32
 * features. No reference counterpart (a layout of this library's kernels). */
int64_t ssl_slr_chain_frag_bytes(int64_t M, int64_t n_out);
int ssl_slr_forward_chain(int64_t M, int32_t block_p, int32_t block_q, int32_t dtype,
                          const ssl_slr_stage* stages, int32_t n_stages,
                          const ssl_slr_member* members, int32_t n_members, void* stream);

/* A chained launch of many stages (up to SSL_MAX_CHAIN_TABLE linears and as
 * many stages, e.g. every projection of every layer of a model's decode step
 * in ONE launch, each layer's q,k,v a stage reading the previous layer's down
 * projection), described by a table in device memory instead of kernel
 * arguments. ssl_slr_chain_table_build checks the call exactly as
 * ssl_slr_forward_chain does and writes the table (ssl_slr_chain_table_bytes,
 * 16-byte aligned) into host memory; the caller copies it to device memory
 * once, and ssl_slr_chain_table_launch launches it (table_dev must hold a copy
 * of table_host). The table holds every pointer of the call (input, outputs,
 * weights, scratch): a launch recomputes the same call on whatever those
 * buffers hold, so it suits static-buffer decode loops and graph capture.
 * Extends ssl_slr_forward_chain; no reference counterpart. */
#define SSL_MAX_CHAIN_TABLE 256
int64_t ssl_slr_chain_table_bytes(void);
int ssl_slr_chain_table_build(int64_t M, int32_t block_p, int32_t block_q, int32_t dtype,
                              const ssl_slr_stage* stages, int32_t n_stages,
                              const ssl_slr_member* members, int32_t n_members, void* table,
                              int64_t table_bytes);
int ssl_slr_chain_table_launch(const void* table_host, const void* table_dev, void* stream);

/* -------------------------------------------------------------------------
 * Block projection (device): keep the n_keep blocks of largest Frobenius norm.
 * Replaces ssalaad/inference/egar.py:296-317 (_project_S), the sparse step of
 * the compression loop (called at egar.py:464):
 *   norms[b] = Σ_block v² with v the input as fp32   (M.float(), pow(2).sum)
 *   keep[b]  = 1 for the n_keep largest norms         (topk(n_keep, largest=True))
 *   out      = the input as fp32 where its block is kept, else 0
 * S is [NB·p, lds] in `dtype`; blocks are numbered row-major (b = by·NBK + bc).
 * n_keep is clamped to [0, NB·NBK] as the reference does. A NaN norm counts as
 * the largest (as in torch.topk). Equal norms are taken in ascending block
 * order: deterministic, where torch.topk leaves the order unspecified.
 * `norms` (NB·NBK fp32) and `keep` (NB·NBK bytes) are device arrays the call
 * fills; `out` ([NB·p, ldo] fp32) may be NULL to get the mask only.
 * `workspace` (ssl_block_topk_workspace_size(NB·NBK) bytes, 16-byte aligned,
 * no initial contents) holds the select's histograms and counts when many
 * workgroups share it; calls that share a workspace must be ordered.
 * ------------------------------------------------------------------------- */
int64_t ssl_block_topk_workspace_size(int64_t n_blocks);
int ssl_block_topk(const void* S, int64_t lds, int64_t NB, int64_t NBK, int32_t block_p,
                   int32_t block_q, int32_t dtype, int64_t n_keep, float* norms, uint8_t* keep,
                   float* out, int64_t ldo, void* workspace, int64_t workspace_bytes,
                   void* stream);

/* -------------------------------------------------------------------------
 * ssl_project_nm — N:M projection of a dense matrix.
 * Replaces ssalaad/inference/egar.py:284-292 (_project_S_nm), the sparse step
 * of the compression loop for N:M structure:
 *   in each run of nm_m consecutive entries of a row, keep the nm_n of
 *   largest magnitude (|R|.topk(nm_n)); out = R.float() · mask.
 * R is [n, ldr] in `dtype`; out is [n, ldo] fp32; keep (optional, [n, ldk]
 * bytes) receives the mask. A NaN magnitude counts as the largest (as in
 * torch.topk); equal magnitudes go to the lower index (torch.topk leaves
 * that order unspecified). Dropped entries are R·0 as the reference's
 * multiply leaves them (−0 for negative values, NaN for ±inf and NaN).
 * nm_m ∈ [1, 32], nm_n ∈ [0, nm_m], m a multiple of nm_m.
 * ------------------------------------------------------------------------- */
int ssl_project_nm(const void* R, int64_t ldr, int64_t n, int64_t m, int32_t nm_n, int32_t nm_m,
                   int32_t dtype, float* out, int64_t ldo, uint8_t* keep, int64_t ldk,
                   void* stream);

/* -------------------------------------------------------------------------
 * Dense → BSR encoder (device), the rule of ssalaad/efficient/artifact.py:20-37
 * (dense_to_bsr) followed by the module conversion of
 * ssalaad/efficient/ls_linear.py:89-97:
 *   a (p×q) block is kept iff the sum of |values| over the block is > 0, i.e. it
 *   holds no NaN and at least one non-zero; kept blocks are listed row-major.
 * Step 1 (ssl_bsr_encode_count) writes crow [NB+1] (int32), active_rows [NB]
 *   (ascending; entries past the count are unspecified) and the two totals
 *   totals[0] = nnz, totals[1] = number of active block-rows (int32, device).
 * Step 2 (ssl_bsr_encode_fill) writes col [nnz] (int32), values_bsr [nnz, p, q]
 *   (BSR layout; may be NULL) and values_t [nnz, q, p] (kernel layout; may be NULL).
 * S is [n, lds] row-major with n = NB·p and NBK·q ≤ lds columns used.
 * `flags` is a device scratch array of NB·NBK bytes shared by the two steps.
 * ------------------------------------------------------------------------- */
int ssl_bsr_encode_count(const void* S, int64_t lds, int64_t NB, int64_t NBK,
                         int32_t block_p, int32_t block_q, int32_t dtype, uint8_t* flags,
                         int32_t* crow, int32_t* active_rows, int32_t* totals,
                         void* stream);
int ssl_bsr_encode_fill(const void* S, int64_t lds, int64_t NB, int64_t NBK,
                        int32_t block_p, int32_t block_q, int32_t dtype,
                        const uint8_t* flags, const int32_t* crow, int32_t* col,
                        void* values_bsr, void* values_t, void* stream);

/* -------------------------------------------------------------------------
 * KV-cached decode step: the pieces of a LLaMA / Qwen3 decoder layer around
 * its SLR linears, for one new token per sequence. The reference has no
 * cached decode: its greedy generation recomputes the whole prefix with the
 * Hugging Face forward every step (ssalaad/inference/generate.py:1-26). These
 * calls reproduce that forward's per-token arithmetic (transformers'
 * LlamaDecoderLayer / Qwen3DecoderLayer) from a cache. Batch row b is
 * sequence slot b; `pos` (device int32 [rows]) is each row's position, which
 * must lie in [0, max_ctx). Caches are [slots, kv_heads, max_ctx, head_dim] in
 * the model dtype, 16-byte aligned.
 * ------------------------------------------------------------------------- */

/* h += delta (skipped when delta is NULL), rounded to the dtype; then
 * out = weight · (h · rsqrt(mean(h²) + eps)) with LlamaRMSNorm's rounding
 * points. h [rows, ldh] is updated in place (the residual stream). */
int ssl_add_rmsnorm(void* h, int64_t ldh, const void* delta, int64_t ldd, const void* weight,
                    void* out, int64_t ldo, int64_t rows, int64_t hidden, float eps,
                    int32_t dtype, void* stream);

/* The layer-0 input: h[row] = embed[tokens[row]] (embed [vocab, lde]; a token
 * outside [0, vocab) gives a zero row), then out = weight · norm(h) as above.
 * hidden at most 8192 for both calls. */
int ssl_embed_rmsnorm(const void* embed, int64_t lde, int64_t vocab, const int64_t* tokens,
                      void* h, int64_t ldh, const void* weight, void* out, int64_t ldo,
                      int64_t rows, int64_t hidden, float eps, int32_t dtype, void* stream);

/* Rotary embedding of q [rows, ldq] (heads·head_dim used) into q_out
 * [rows, heads, head_dim] and of k into k_cache at (row, head, pos[row]); v
 * is copied into v_cache at the same place. cos/sin tables are
 * [max_ctx, head_dim] in the dtype (the model's rotary embedding evaluated at
 * every position). q_norm / k_norm ([head_dim], may be NULL) apply Qwen3's
 * per-head RMSNorm first. head_dim even and at most 256. */
int ssl_rope_kv_append(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v,
                       int64_t ldv, const void* cos_table, const void* sin_table,
                       const void* q_norm, const void* k_norm, float eps, const int32_t* pos,
                       void* q_out, void* k_cache, void* v_cache, int64_t rows, int32_t heads,
                       int32_t kv_heads, int32_t head_dim, int64_t max_ctx, int32_t dtype,
                       void* stream);

/* out[row, h·head_dim + d] = softmax_j(q·k_j · scale) · v_j over positions
 * j ≤ pos[row] of the row's cache, with query head h reading key/value head
 * h / (heads / kv_heads). fp32 accumulation, one rounding at the store.
 * The context is cut into n_split slices (at most 256); the slice that
 * finishes last merges every slice's partial in the same launch.
 * ssl_decode_attention_splits proposes n_split for a batch; the workspace
 * (ssl_decode_attention_workspace_size bytes, 16-byte aligned) holds the
 * partials; `counters` (ssl_decode_attention_counter_count int32) must be zero
 * before the first call and every completed call leaves them zero. Calls that
 * share counters must be ordered. head_dim 64, 128 or 256; q [rows, heads,
 * head_dim]. */
int32_t ssl_decode_attention_splits(int64_t rows, int32_t heads, int32_t kv_heads,
                                    int64_t max_ctx);
int64_t ssl_decode_attention_workspace_size(int64_t rows, int32_t heads, int32_t head_dim,
                                            int32_t n_split);
int64_t ssl_decode_attention_counter_count(int64_t rows, int32_t heads, int32_t kv_heads);
int ssl_decode_attention(const void* q, const void* k_cache, const void* v_cache,
                         const int32_t* pos, void* out, int64_t ldo, int64_t rows, int32_t heads,
                         int32_t kv_heads, int32_t head_dim, int64_t max_ctx, float scale,
                         int32_t n_split, void* workspace, int64_t workspace_bytes,
                         int32_t* counters, int64_t n_counters, int32_t dtype, void* stream);

/* ssl_rope_kv_append followed by ssl_decode_attention in one launch, with the
 * same results: q, k, v are the projections of the new token ([rows, ld*],
 * 16-byte aligned rows), the new key is rotated and, with the value, written
 * into the caches at pos[row], and the attention reads that position from
 * registers. The roped q is not stored. Workspace, counters and splits as for
 * ssl_decode_attention; head_dim 64, 128 or 256. Replaces, for one decode
 * step, the rotary embedding, the cache update and sdpa of LlamaAttention
 * (transformers modeling_llama.py), as called by the reference's generation
 * loop (ssalaad/inference/generate.py:1-26). */
int ssl_decode_rope_attention(const void* q, int64_t ldq, const void* k, int64_t ldk,
                              const void* v, int64_t ldv, const void* cos_table,
                              const void* sin_table, const void* q_norm, const void* k_norm,
                              float eps, const int32_t* pos, void* k_cache, void* v_cache,
                              void* out, int64_t ldo, int64_t rows, int32_t heads,
                              int32_t kv_heads, int32_t head_dim, int64_t max_ctx, float scale,
                              int32_t n_split, void* workspace, int64_t workspace_bytes,
                              int32_t* counters, int64_t n_counters, int32_t dtype, void* stream);

/* out = silu(gate) · up (LlamaMLP's act_fn(gate_proj(x)) * up_proj(x)), silu
 * rounded to the dtype before the product. */
int ssl_silu_mul(const void* gate, int64_t ldg, const void* up, int64_t ldu, void* out,
                 int64_t ldo, int64_t rows, int64_t n, int32_t dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SSALAAD_AMD_H */
