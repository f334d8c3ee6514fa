// Host side of the streaming SLR / BSR kernels for gfx950: argument checks,
// scratch layout and launch set-up of the C-ABI entry points. The kernels are
// in stream_kernel.h, instantiated per dtype in stream_{bf16,f16,f32}.hip.

#include <string.h>

#include <vector>

#include "abi_internal.h"
#include "prefill.h"
#include "stream_kernel.h"

namespace ssl {

// ---------------------------------------------------------------------------
// Host-side launch plumbing
// ---------------------------------------------------------------------------
namespace {

hipError_t dispatch(int dtype, int mode, int sf, int P, int KE, int MT, const GroupArgs& a,
                    int64_t blocks, hipStream_t s) {
  switch (dtype) {
    case SSL_F32: return stream_launch<DT_F32>(mode, sf, P, KE, MT, a, blocks, s);
    case SSL_BF16: return stream_launch<DT_BF16>(mode, sf, P, KE, MT, a, blocks, s);
    case SSL_F16: return stream_launch<DT_F16>(mode, sf, P, KE, MT, a, blocks, s);
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

// Block shapes of the streaming kernel: p output features ∈ {16, 32, 48, 64}
// (the template's tile widths) and q input features any multiple of 16 up to 256
// (walked as K slabs at run time).
bool supported_block(int p, int q) {
  return (p == 16 || p == 32 || p == 48 || p == 64) && q >= 16 && q <= 256 && q % 16 == 0;
}
// Block shapes the prefill kernels take: square 16, 32 or 64 (fp32: 16 or 32,
// which divide its 32-column steps).
bool prefill_block(int p, int q, int dtype) {
  return p == q && (p == 16 || p == 32 || (p == 64 && dtype != SSL_F32));
}

// k elements per lane of the sparse MFMA fragments for q-deep blocks.
int stream_ke(int dtype, int q) { return (dtype != SSL_F32 && q % 32 == 0) ? 8 : 4; }

// The slab walk of blocks of q input features (SlrArgs' block fields).
void set_block_shape(SlrArgs& a, int dtype, int p, int q, int s_format) {
  const int eb = elem_bytes(dtype);
  const int km = 4 * stream_ke(dtype, q);
  a.q = q;
  if (s_format == SSL_S_NM24) {
    a.nks = 1;
    a.blk_bytes = kNmBlockBytes;
    a.slab_bytes = kNmBlockBytes;
  } else {
    a.nks = q / km;
    a.blk_bytes = p * q * eb;
    a.slab_bytes = km * p * eb;
  }
  a.nks_magic = a.nks > 1 ? (uint32_t)((((uint64_t)1 << 32) + a.nks - 1) / a.nks) : 0u;
}

// Slab indices stay exact through the high-multiply division (v·(nks − 1) < 2^32)
// and within int range.
bool slab_count_ok(int64_t nnz, int nks) {
  const int64_t v = nnz * nks;
  return v < 0x7fffffffLL && v * (nks > 1 ? nks - 1 : 1) < (1LL << 32);
}
bool supported_dtype(int dt) { return dt == SSL_F32 || dt == SSL_BF16 || dt == SSL_F16; }

// Scratch layout of one fused call. Row counters live in their own int32 array
// (zero at rest, never shared with data) and the handshake words in the plan's
// own uint64 array; the data workspace holds the latent partials, the final
// latent and the fp32 partial tiles of split rows (byte offsets).
struct Layout {
  int MT, MG;
  int n_rt, n_kc_max, ku_total;
  int64_t cnt_total;  // int32 counters: row counters [MG][NB], then (prefill) the
                      // latent tile counters' slots from index pf_cnt
  int64_t n_sync;     // u64 handshake words: status, then (2 + n_rt) per token tile
  int64_t fin_off;    // byte offset in the exchange area of the final-count copies
  int64_t x_total;    // exchange area bytes
  int64_t pf_cnt;     // first int32 counter of the prefill latent tile counters
  int64_t pf_rarrive; // first int32 counter of the prefill row parts' arrivals
  int64_t t_part, t_final, part_main;  // workspace byte offsets
  int64_t total_min;  // workspace bytes a call needs
  int64_t pf_split;   // then (prefill) the partial tiles of split calls
  int64_t total;      // workspace bytes with them (the size the query reports)
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
  // the prefill kernels' latent tile counters: per kPrefillLatentRows token
  // rows, kPfCntCopies slots of kPfCntStride int32 (the tiles written, and the
  // waiters that have passed), zero at rest like the row counters
  L.pf_cnt = align_up(L.cnt_total, kPfCntStride);
  L.pf_rarrive = L.pf_cnt;
  if (M >= kPrefillMinM) {
    L.pf_rarrive = L.pf_cnt + (int64_t)kPfCntCopies * kPfCntStride *
                                  ((M + kPrefillLatentRows - 1) / kPrefillLatentRows);
    // one arrival word per (64-row token tile, block-row) bounds the row parts'
    L.cnt_total = L.pf_rarrive + ((M + 63) / 64) * NB;
  }
  L.n_sync = 1 + (int64_t)L.MG * (2 + L.n_rt);
  L.fin_off = align_up(8 * L.n_sync, 256);
  L.x_total = L.fin_off + (L.n_rt > 0 ? 8LL * L.MG * kFinCopies * kFinSlotWords : 0);
  const int64_t rows = (int64_t)L.MG * 16 * L.MT;
  int64_t off = 0;
  L.t_part = off;
  if (L.n_kc_max > 1) off = align_up(off + 4 * (int64_t)L.n_kc_max * rows * r_pad, 256);
  L.t_final = off;
  off = align_up(off + (int64_t)elem_bytes(dtype) * rows * r_pad, 256);
  L.part_main = off;
  off = align_up(off + 4 * (int64_t)L.MG * n_slots * (16 * L.MT * p), 256);
  L.total_min = off;
  L.pf_split = off;
  L.total = align_up(off + prefill_split_bytes(M, NB, p, m_pad, r_pad, dtype, device_cus()), 256);
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

// Checks of one member of a fused call, and its scratch layout. Returns
// SSL_OK, or the status of the failure already recorded.
int check_member(int i, const ssl_slr_member& mb, int64_t M, int64_t m_pad, int block_p,
                 int block_q, int dtype, int s_format, Layout* L) {
  const int eb = elem_bytes(dtype);
  if (mb.NB < 0 || mb.r_pad < 0 || mb.n_chunks < 0 || mb.n_slots < 0 || mb.lr_wgs < 0)
    return fail(SSL_ERR_INVALID, "linear %d: negative size", i);
  if (mb.s_format != s_format)
    return fail(SSL_ERR_INVALID, "linear %d: all linears of a call share the sparse storage", i);
  if (mb.r_pad % 64) return fail(SSL_ERR_INVALID, "linear %d: r_pad must be a multiple of 64", i);
  if (mb.nnz < 0 || !slab_count_ok(mb.nnz, block_q / (4 * stream_ke(dtype, block_q))))
    return fail(SSL_ERR_UNSUPPORTED, "linear %d: too many blocks (%lld) for one call", i,
                (long long)mb.nnz);
  if (mb.NB == 0) {  // no output columns: nothing to launch for this linear
    *L = slr_layout(M, 0, block_p, 0, m_pad, 0, dtype);
    return SSL_OK;
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
  *L = slr_layout(M, mb.NB, block_p, mb.r_pad, m_pad, mb.n_slots, dtype);
  if (L->total > 0x7fffffffLL)
    return fail(SSL_ERR_UNSUPPORTED,
                "linear %d: workspace of %lld bytes exceeds 2 GiB; split the call by tokens", i,
                (long long)L->total);
  if (mb.workspace_bytes < L->total_min || !mb.workspace)
    return fail(SSL_ERR_WORKSPACE, "linear %d: workspace of %lld bytes needed", i,
                (long long)L->total_min);
  if (!aligned(mb.workspace, 256))
    return fail(SSL_ERR_WORKSPACE, "linear %d: workspace must be 256-byte aligned", i);
  if (mb.n_counters < L->cnt_total || !mb.counters)
    return fail(SSL_ERR_WORKSPACE, "linear %d: %lld zeroed counters needed", i,
                (long long)L->cnt_total);
  if (mb.exchange_bytes < L->x_total || !mb.exchange)
    return fail(SSL_ERR_WORKSPACE, "linear %d: exchange area of %lld bytes needed", i,
                (long long)L->x_total);
  if (!aligned(mb.exchange, 256))
    return fail(SSL_ERR_WORKSPACE, "linear %d: exchange area must be 256-byte aligned", i);
  return SSL_OK;
}

// The streaming kernel's arguments for one member (a latent split of n_kc
// chunks of ku_chunk units).
void fill_args(SlrArgs& a, const ssl_slr_member& mb, const Layout& L, const void* x, int64_t ldx,
               int64_t M, int64_t m, int64_t m_pad, int n_kc, int ku_chunk, int dtype,
               int block_p, int block_q, int s_format) {
  const DebugKnobs& knobs = debug_knobs();
  char* ws = (char*)mb.workspace;
  a.x = x; a.ldx = ldx; a.M = (int)M; a.m = (int)m;
  a.y = mb.y; a.ldy = mb.ldy; a.col = mb.col; a.values = mb.values; a.plan = mb.plan;
  a.n_chunks = (int)mb.n_chunks; a.NB = (int)mb.NB; a.nnz = (int)mb.nnz;
  a.A = mb.A; a.lda = mb.r_pad; a.bias = mb.bias;
  a.n_slots = mb.n_slots; a.part_main = (float*)(ws + L.part_main); a.cnt_main = mb.counters;
  a.B = mb.B; a.ldb = m_pad; a.t = ws + L.t_final; a.ldt = mb.r_pad;
  a.t_part = (float*)(ws + L.t_part);
  a.MG = L.MG; a.n_rt = L.n_rt; a.n_kc = n_kc; a.ku_total = L.ku_total;
  a.ku_chunk = ku_chunk;
  a.n_lat_wgs = (int)((int64_t)L.n_rt * n_kc * L.MG);
  a.sync = (u64*)mb.exchange; a.lr_wgs = (int)mb.lr_wgs; a.lat_weight = kLatentUnits / n_kc;
  a.fin = (u64*)((char*)mb.exchange + L.fin_off);
  a.tk_copies = mb.lr_wgs == mb.NB ? kFinCopies : 1;
  a.status = mb.status ? (u64*)mb.status : (u64*)mb.exchange;
  set_block_shape(a, dtype, block_p, block_q, s_format);
  a.wait_polls = knobs.wait_polls > 0 ? (int)knobs.wait_polls : kSpinLimit;
  // out of reach of any launch: tickets and counters advance far less per launch
  a.wait_bias = knobs.wait_unreachable ? (1 << 30) : 0;
  a.dep = nullptr; a.dep_need = 0; a.dep_waiters = 0; a.done = nullptr;
}

// K units (of 32 in_features) per latent chunk in a chained stage after the
// first: one batch of loads for each of the 8 waves.
constexpr int kChainLatentUnits = 64;
// Token rows from which a chained launch of 32- or 64-wide blocks passes the
// stages' inputs in fragment order (each wave reads a unit as one contiguous
// 1 KiB load). Below it the 16-row tiles are mostly padding, and the rows
// read by row segments (fewer bytes) were faster: LLaMA-1B layer stack at 2 /
// 4 / 6 token rows 2608 / 4977 / 7362 tok/s by rows, 2499 / 4963 / 7412 in
// fragment order (16 rows: 17.2 k by rows, 18.4 k in fragment order).
constexpr int64_t kChainFragMinM = 6;

// Whether a chained launch's later stages read fragment-order inputs.
bool chain_frag(int64_t M, int32_t block_p) {
  if (block_p != 32 && block_p != 64) return false;
  if (tile_mt(M) > 1) return true;  // taller tiles have only the fragment kernels
  const int64_t k = debug_knobs().chain_frag;
  if (k == 1) return false;
  if (k == 2) return true;
  return M >= kChainFragMinM;
}

// Checks a chained launch and fills its descriptor (c, zeroed by the caller,
// with room for NMAX members); c->grid = 0 when there is nothing to launch.
template <int NMAX>
int build_chain(int64_t M, int32_t block_p, int32_t block_q, int32_t dtype,
                const ssl_slr_stage* stages, int32_t n_stages, const ssl_slr_member* members,
                int32_t n_members, int max_stages, ChainDesc<NMAX>* c) {
  if (dtype != SSL_BF16 && dtype != SSL_F16)
    return fail(SSL_ERR_UNSUPPORTED, "chained launches take bf16 or fp16 activations");
  if (n_stages < 1 || n_stages > max_stages || !stages)
    return fail(SSL_ERR_INVALID, "a chained launch takes 1 to %d stages, got %d", max_stages,
                n_stages);
  if (n_members < 1 || n_members > NMAX || !members)
    return fail(SSL_ERR_INVALID, "a chained launch takes 1 to %d linears, got %d", NMAX,
                n_members);
  const int s_format = members[0].s_format;
  if (s_format == SSL_S_NM24) {
    if (block_p != kNmBlock || block_q != kNmBlock)
      return fail(SSL_ERR_UNSUPPORTED, "2:4 blocks are 32x32");
  } else if (s_format != SSL_S_BSR) {
    return fail(SSL_ERR_INVALID, "unknown sparse storage format %d", s_format);
  } else if (block_p != block_q || (block_p != 16 && block_p != 32 && block_p != 64)) {
    return fail(SSL_ERR_UNSUPPORTED, "chained launches take square blocks of 16, 32 or 64, got %dx%d",
                block_p, block_q);
  }
  if (M < 0) return fail(SSL_ERR_INVALID, "negative size");
  c->grid = 0;
  if (M == 0) return SSL_OK;
  if (M > 0x7fffffffLL) return fail(SSL_ERR_INVALID, "too many token rows");
  const int eb = elem_bytes(dtype);
  const int64_t n_sync = ssl_slr_chain_sync_count(M);

  // stages: contiguous member ranges in order; each later stage reads the
  // output of one member of an earlier stage, and a member feeds at most one
  std::vector<int> fed(n_members, 0);
  int next = 0;
  for (int s = 0; s < n_stages; ++s) {
    const ssl_slr_stage& st = stages[s];
    if (st.first != next || st.count < 1 || st.first + st.count > n_members)
      return fail(SSL_ERR_INVALID, "stage %d: its members must follow the previous stage's", s);
    next = st.first + st.count;
    if (st.m < 1 || st.m_pad % 64 || st.m_pad < st.m)
      return fail(SSL_ERR_INVALID, "stage %d: m >= 1 and m_pad a multiple of 64 and >= m", s);
    if (s == 0) {
      if (st.src != -1) return fail(SSL_ERR_INVALID, "stage 0 reads the launch's input (src -1)");
      if (!st.x || !aligned(st.x, 16) || st.ldx < st.m || (st.ldx * eb) % 16)
        return fail(SSL_ERR_INVALID, "x rows must be 16-byte aligned and at least m wide");
      continue;
    }
    if (st.src < 0 || st.src >= st.first)
      return fail(SSL_ERR_INVALID, "stage %d: src must be a member of an earlier stage", s);
    const ssl_slr_member& src = members[st.src];
    if (fed[st.src]++) return fail(SSL_ERR_INVALID, "stage %d: member %d already feeds a stage", s, st.src);
    if (src.NB * block_p < st.m)
      return fail(SSL_ERR_INVALID, "stage %d: in_features %lld exceed member %d's %lld outputs", s,
                  (long long)st.m, st.src, (long long)(src.NB * block_p));
    if (st.x && st.x != src.y)
      return fail(SSL_ERR_INVALID, "stage %d: x must be NULL (member %d's output)", s, st.src);
    if (!st.sync || st.n_sync < n_sync || !aligned(st.sync, 256))
      return fail(SSL_ERR_WORKSPACE, "stage %d: %lld zeroed sync words needed", s,
                  (long long)n_sync);
    if (M * src.ldy * eb > 0x7fffffffLL)
      return fail(SSL_ERR_UNSUPPORTED, "stage %d: its input is beyond 2 GiB; split the call by tokens", s);
    if (!st.xf && chain_frag(M, block_p))
      return fail(SSL_ERR_WORKSPACE, "stage %d: %lld token rows of 32- or 64-wide blocks need xf "
                  "(%lld bytes)", s, (long long)M,
                  (long long)ssl_slr_chain_frag_bytes(M, src.NB * block_p));
    if (st.xf) {
      const int64_t need = ssl_slr_chain_frag_bytes(M, src.NB * block_p);
      if (!aligned(st.xf, 256) || st.xf_bytes < need)
        return fail(SSL_ERR_WORKSPACE, "stage %d: xf must be 256-byte aligned with %lld bytes", s,
                    (long long)need);
      if (need > 0x7fffffffLL)
        return fail(SSL_ERR_UNSUPPORTED, "stage %d: its fragment copy is beyond 2 GiB", s);
    }
  }
  if (next != n_members) return fail(SSL_ERR_INVALID, "every member belongs to one stage");

  std::vector<Layout> L(n_members);
  int64_t wg = 0;
  int nseg = 0;
  int MT = tile_mt(M);
  for (int s = 0; s < n_stages; ++s) {
    const ssl_slr_stage& st = stages[s];
    const void* x = s == 0 ? st.x : members[st.src].y;
    const int64_t ldx = s == 0 ? st.ldx : members[st.src].ldy;
    int64_t n_stream = 0, rt_tiles = 0, rows = 0;
    for (int i = st.first; i < st.first + st.count; ++i) {
      const ssl_slr_member& mb = members[i];
      const int rc = check_member(i, mb, M, st.m_pad, block_p, block_q, dtype, s_format, &L[i]);
      if (rc != SSL_OK) return rc;
      n_stream += (mb.NB > 0 ? mb.n_chunks : 0) * L[i].MG;
      rt_tiles += (int64_t)L[i].n_rt * L[i].MG;
      rows += mb.NB;
    }
    if (s_format == SSL_S_NM24 ? ssl_nm24_takes_prefill(M, rows, dtype)
                               : ssl_slr_takes_prefill(M, rows, block_p, block_q, dtype))
      return fail(SSL_ERR_UNSUPPORTED,
                  "stage %d: a call of %lld token rows runs the prefill kernels; launch the "
                  "stages one by one", s, (long long)M);
    // Stage 0: the K split a grouped launch of its members would take (its
    // results equal ssl_slr_forward_group's bit for bit). Later stages: K
    // chunks of at most kChainLatentUnits units, one batch of loads per wave
    // (its B loads go out before the stage's input is ready), so a latent
    // over 2048 in_features is final without an exchange of partials:
    // measured 4-5% per step at 1 and 4 token rows against the standalone
    // split; the 5461-wide down projection takes three chunks (one chunk of
    // 350 KB of loads per workgroup took 6.4 µs).
    int n_kc = 1, ku_chunk = L[st.first].ku_total;
    if (s == 0) {
      latent_chunks(L[st.first], n_stream, rt_tiles, &n_kc, &ku_chunk);
    } else {
      n_kc = (L[st.first].ku_total + kChainLatentUnits - 1) / kChainLatentUnits;
      if (n_kc > L[st.first].n_kc_max) n_kc = L[st.first].n_kc_max;
      if (n_kc < 1) n_kc = 1;
      ku_chunk = (L[st.first].ku_total + n_kc - 1) / n_kc;
      n_kc = (L[st.first].ku_total + ku_chunk - 1) / ku_chunk;
    }
    // waiters of one token tile: every latent workgroup, then every row
    // workgroup of the stage's members, numbered in that order
    int waiters = 0;
    for (int i = st.first; i < st.first + st.count; ++i) {
      SlrArgs& a = c->m[i];
      fill_args(a, members[i], L[i], x, ldx, M, st.m, st.m_pad, n_kc, ku_chunk, dtype, block_p,
                block_q, s_format);
      c->seg_start[nseg] = (int)wg;
      c->seg_member[nseg] = i;
      c->seg_rows[nseg++] = 0;
      wg += (int64_t)L[i].n_rt * n_kc * L[i].MG;
      a.dep_lat_base = waiters;
      waiters += L[i].n_rt * n_kc;
    }
    for (int i = st.first; i < st.first + st.count; ++i) {
      const ssl_slr_member& mb = members[i];
      c->seg_start[nseg] = (int)wg;
      c->seg_member[nseg] = i;
      c->seg_rows[nseg++] = 1;
      wg += (mb.NB > 0 ? mb.n_chunks : 0) * L[i].MG;
      c->m[i].dep_row_base = waiters;
      waiters += mb.NB > 0 ? (int)mb.n_chunks : 0;
      if (wg > 0x7fffffffLL) return fail(SSL_ERR_INVALID, "grid too large");
    }
    if (s > 0 && waiters > 0) {
      // the stage waits for its source; the source counts its row tiles
      for (int i = st.first; i < st.first + st.count; ++i) {
        c->m[i].dep = st.sync;
        c->m[i].dep_need = (int)members[st.src].NB;
        c->m[i].dep_waiters = waiters;
      }
      c->m[st.src].done = st.sync;
      // the source's output also in fragment order (whole 32-column units per
      // row tile: 32- and 64-wide tiles)
      if (chain_frag(M, block_p)) {
        const int units = (int)(members[st.src].NB * block_p / 32);
        for (int i = st.first; i < st.first + st.count; ++i) {
          c->m[i].xf = st.xf;
          c->m[i].xf_units = units;
        }
        c->m[st.src].yf = st.xf;
        c->m[st.src].yf_units = units;
      }
    }
  }
  c->n_seg = nseg;
  c->seg_start[nseg] = (int)wg;
  c->grid = wg;
  c->M = (int)M;
  c->block_p = block_p;
  c->dtype = dtype;
  c->sf = s_format == SSL_S_NM24 ? SF_NM24 : SF_BSR;
  c->fr = chain_frag(M, block_p) ? 1 : 0;
  (void)MT;
  return SSL_OK;
}

template <int NMAX>
int launch_chain(const ChainDesc<NMAX>& c, const ChainArgs* a, const ChainTab* tab,
                 hipStream_t stream) {
  const int MT = tile_mt(c.M);
  hipError_t e = c.dtype == SSL_BF16
                     ? chain_launch<DT_BF16>(c.sf, c.block_p, MT, c.fr != 0, a, tab, c.grid, stream)
                     : chain_launch<DT_F16>(c.sf, c.block_p, MT, c.fr != 0, a, tab, c.grid, stream);
  return check_hip(e, "slr chained launch");
}


}  // namespace
}  // namespace ssl

using namespace ssl;

extern "C" {

int64_t ssl_prefill_min_rows(void) { return kPrefillMinM; }

// Which kernels a fused call with block storage takes: the prefill kernels
// from kPrefillMinM token rows for the square blocks they run (fp32: when
// their grid fills the device), except one-token-tile 16-bit calls with at
// most 2048 output features, where the streaming kernel (one weight pass per
// 64-row token tile) measured faster on MI355X.
int32_t ssl_slr_takes_prefill(int64_t M, int64_t n_rows, int32_t block_p, int32_t block_q,
                              int32_t dtype) {
  if (M < kPrefillMinM || !prefill_block(block_p, block_q, dtype)) return 0;
  if (dtype == SSL_F32) {
    // fp32 runs 16 times fewer MFMA flops per cycle: the tiled kernels win once
    // a grid of their short (64-row) tiles fills the device; smaller calls keep
    // the streaming kernel's finer split (LLaMA-60M at 2048 rows: 512×512 31.1
    // tiled vs 34.4 µs streaming, 512×1376 60.0 vs 59.7; the gate 1376×512 at
    // 1024 rows 31.7 vs 38.5, at 512 rows 25.3 vs 26.1). A forced row tile
    // (test hook) sends every such call to the tiled kernels.
    if (debug_knobs().prefill_group != 0) return 1;
    const int64_t items = ((M + 63) / 64) * ((n_rows + 64 / block_p - 1) / (64 / block_p));
    return items >= device_cus() ? 1 : 0;
  }
  if (debug_knobs().prefill_group != 0) return 1;  // a forced row tile (test hook)
  // The streaming kernel keeps only one-token-tile calls with at most 2048
  // output features: its finer K split wins there (2048×2048 and 2048×5461
  // with 32×32 blocks at 128 rows: 26.9 / 39.4 µs streaming against 28.8 /
  // 42.0). Everywhere else the tiled kernels, K parts included, win: 16×16
  // blocks 2.2-4.3× (11008×4096 at 128 / 256 / 512 rows 109 / 196 / 372 ->
  // 49 / 60 / 87 µs), 4096×11008 with 32×32 or 64×64 at 128 rows 82 / 64 ->
  // 46 / 44, 4096×4096 with 64×64 at 128 rows 34.3 -> 31.0.
  if (M <= kPrefillMinM && n_rows * block_p <= 2048) return 0;
  return 1;
}

int64_t ssl_prefill_parts_bytes(int64_t M, int64_t split_parts) {
  if (M <= 0 || split_parts <= 0) return 0;
  return align_up(split_parts * ((M + 127) / 128 * 128) * 64 * 4, 256);
}

int64_t ssl_nm24_block_bytes(void) { return kNmBlockBytes; }

int64_t ssl_nm24_prefill_block_bytes(void) { return kNmPrefillBlockBytes; }

// 2:4 calls take the prefill kernels (v_smfmac) from kPrefillMinM token rows.
int32_t ssl_nm24_takes_prefill(int64_t M, int64_t n_rows, int32_t dtype) {
  (void)n_rows;
  return (M >= kPrefillMinM && dtype != SSL_F32) ? 1 : 0;
}

int32_t ssl_prefill_step_cols(int32_t dtype) { return dtype == SSL_F32 ? 32 : 64; }

int32_t ssl_prefill_group(int64_t M, int64_t n_rows, int32_t block_p, int32_t block_q) {
  if (!(block_p == block_q && (block_p == 16 || block_p == 32 || block_p == 64))) return 1;
  return prefill_group(M, n_rows, block_p, device_cus());
}

int32_t ssl_bsr_addmm_takes_prefill(int64_t M, int64_t n_rows, int32_t block_p, int32_t block_q,
                                    int32_t dtype) {
  // fp32: only under a forced row tile (test hook); the streaming kernel's
  // finer split is the default for the op
  if (M < kPrefillMinM || !prefill_block(block_p, block_q, dtype)) return 0;
  if (debug_knobs().prefill_group != 0) return 1;
  if (dtype == SSL_F32) return 0;
  // One token tile whose grid of short (64-row) tiles would fill at most a
  // quarter of the CUs streams: the op's tiled kernel runs whole row groups (2048×5461
  // with 32×32 blocks at 128 rows: 22.8 µs streaming, 36.0 tiled; 4096×4096
  // and 4096×11008 with 64×64: 31.3 / 50.3 against 34.2 / 54.1), while
  // 11008×4096 with 64×64 (172 groups) and 16×16 blocks tile (36.4 against
  // 53.3, 51.5 against 109.4).
  if (M <= kPrefillMinM && block_p >= 32) {
    const int64_t per = 64 / block_p, groups = (n_rows + per - 1) / per;
    if (4 * groups <= device_cus()) return 0;
  }
  return 1;
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
                          const int32_t* pf_steps,
                          int64_t pf_n_groups, int32_t pf_group, int64_t M, int64_t N, int64_t K,
                          int64_t NB, int32_t block_p, int32_t block_q, int32_t dtype,
                          int32_t* counters, int64_t n_counters, void* workspace,
                          int64_t workspace_bytes, void* stream) {
  clear_error();
  if (!supported_dtype(dtype)) return fail(SSL_ERR_UNSUPPORTED, "unsupported dtype %d", dtype);
  if (!supported_block(block_p, block_q))
    return fail(SSL_ERR_UNSUPPORTED,
                "BSR kernel needs blocks of 16, 32, 48 or 64 output features and a multiple of "
                "16 (up to 256) input features, got %dx%d", block_p, block_q);
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

  if (nnz < 0 || !slab_count_ok(nnz, block_q / (4 * stream_ke(dtype, block_q))))
    return fail(SSL_ERR_UNSUPPORTED, "too many blocks (%lld) for one call", (long long)nnz);
  if (ssl_bsr_addmm_takes_prefill(M, n_chunks, block_p, block_q, dtype)) {
    if (!pf_groups || !pf_steps || pf_n_groups <= 0 || !values_pq)
      return fail(SSL_ERR_INVALID, "calls with %lld token rows need a prefill plan and (p, q) "
                  "ordered block values", (long long)M);
    if (pf_group != prefill_group(M, n_chunks, block_p, device_cus()))
      return fail(SSL_ERR_INVALID, "prefill plan built for group %d, this call needs %d", pf_group,
                  prefill_group(M, n_chunks, block_p, device_cus()));
    if (nnz < 0 || nnz * block_p * block_q * eb > 0x7fffffffLL)
      return fail(SSL_ERR_UNSUPPORTED, "block values beyond 2 GiB");
    if (M * ldx * eb > 0x7fffffffLL || M * ldo * eb > 0x7fffffffLL)
      return fail(SSL_ERR_UNSUPPORTED, "x or out beyond 2 GiB; split the call by tokens");
    PfArgs rows{};
    rows.x = x; rows.ldx = ldx; rows.M = (int)M; rows.m = (int)K; rows.m_pad = (int)K;
    rows.mode = PF_OP;
    rows.n = 1;
    rows.status = (uint64_t*)check_word_ptr();
    PfMember& pm = rows.mb[0];
    pm.y = out; pm.ldy = ldo; pm.values_pq = values_pq; pm.NB = (int)NB;
    pm.values_bytes = nnz * block_p * block_q * eb;
    pm.groups = pf_groups; pm.steps = pf_steps; pm.n_groups = (int)pf_n_groups;
    pm.ksplit = 1;  // the op's row kernel runs whole row groups
    rows.bm = prefill_row_tile(M, n_chunks, pf_group, block_p, device_cus(), dtype, 0);
    const int64_t T = (M + rows.bm - 1) / rows.bm;
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
  a.n_chunks = (int)n_chunks; a.NB = (int)NB; a.nnz = (int)nnz;
  a.n_slots = n_slots; a.part_main = (float*)workspace; a.cnt_main = counters;
  a.status = check_word_ptr();  // the op never waits; a checked build reports there
  set_block_shape(a, dtype, block_p, block_q, SSL_S_BSR);
  return check_hip(dispatch(dtype, MODE_OP, SF_BSR, block_p, stream_ke(dtype, block_q), MT, g,
                            n_chunks * MG, (hipStream_t)stream),
                   "bsr_addmm launch");
}

int64_t ssl_slr_counter_count(int64_t M, int64_t NB) {
  return slr_layout(M, NB, 16, 0, 64, 0, SSL_BF16).cnt_total;
}

int64_t ssl_slr_exchange_size(int64_t M, int64_t r_pad, int64_t m_pad, int32_t dtype) {
  (void)m_pad;
  (void)dtype;
  return slr_layout(M, 0, 16, r_pad, 64, 0, SSL_BF16).x_total;
}

int64_t ssl_slr_workspace_size(int64_t M, int64_t NB, int32_t block_p, int64_t r_pad,
                               int64_t m_pad, int64_t n_slots, int32_t dtype) {
  return slr_layout(M, NB, block_p, r_pad, m_pad, n_slots, dtype).total;
}
}  // extern "C"

namespace ssl {
// The workspace a call cannot do without (ssl_slr_workspace_size adds the room
// for the partial tiles of split prefill calls, which a smaller workspace
// forgoes).
int64_t slr_workspace_min(int64_t M, int64_t NB, int32_t block_p, int64_t r_pad, int64_t m_pad,
                          int64_t n_slots, int32_t dtype) {
  return slr_layout(M, NB, block_p, r_pad, m_pad, n_slots, dtype).total_min;
}
}  // namespace ssl

extern "C" {

int ssl_slr_forward_group(const void* x, int64_t ldx, int64_t M, int64_t m, int64_t m_pad,
                          int32_t block_p, int32_t block_q, int32_t dtype,
                          const ssl_slr_member* members, int32_t n_members, void* stream) {
  clear_error();
  if (!supported_dtype(dtype)) return fail(SSL_ERR_UNSUPPORTED, "unsupported dtype %d", dtype);
  if (!supported_block(block_p, block_q))
    return fail(SSL_ERR_UNSUPPORTED,
                "SLR kernel needs blocks of 16, 32, 48 or 64 output features and a multiple of "
                "16 (up to 256) input features, got %dx%d", block_p, block_q);
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
    const int rc = check_member(i, mb, M, m_pad, block_p, block_q, dtype, s_format, &L[i]);
    if (rc != SSL_OK) return rc;
    n_stream += (mb.NB > 0 ? mb.n_chunks : 0) * L[i].MG;
    rt_tiles += (int64_t)L[i].n_rt * L[i].MG;
  }
  if (n_stream == 0) return SSL_OK;

  int64_t call_rows = 0;
  for (int i = 0; i < n_members; ++i) call_rows += members[i].NB;
  const bool nm = s_format == SSL_S_NM24;
  if (nm ? ssl_nm24_takes_prefill(M, call_rows, dtype)
         : ssl_slr_takes_prefill(M, call_rows, block_p, block_q, dtype)) {
    // Many token rows: one launch
    // with the latent GEMM's workgroups first and the row GEMM's after them,
    // over groups of block-rows (2:4: on the structured-sparse MFMA); a row
    // workgroup's low-rank steps wait for its token rows' latent tiles.
    const int64_t blk_bytes = nm ? kNmPrefillBlockBytes : (int64_t)block_p * block_p * eb;
    const int cus = device_cus();
    PfArgs rows{}, lat{};
    if (M * ldx * eb > 0x7fffffffLL)
      return fail(SSL_ERR_UNSUPPORTED, "x beyond 2 GiB; split the call by tokens");
    rows.x = lat.x = x; rows.ldx = lat.ldx = ldx;
    rows.M = lat.M = (int)M; rows.m = lat.m = (int)m; rows.m_pad = lat.m_pad = (int)m_pad;
    rows.mode = PF_FUSED;
    rows.n = lat.n = n_members;
    rows.lbm = lat.lbm = kPrefillLatentRows;
    const DebugKnobs& knobs = debug_knobs();
    rows.polls = knobs.wait_polls > 0 ? (int)knobs.wait_polls : kSpinLimit;
    // out of reach of any launch: a latent tile adds 1 to its counter
    rows.wait_bias = knobs.wait_unreachable ? (1 << 30) : 0;
    rows.status = members[0].status ? members[0].status : (uint64_t*)members[0].exchange;
    const int64_t TL = (M + kPrefillLatentRows - 1) / kPrefillLatentRows;  // latent token tiles
    // one group size for the whole call, from all members' rows together
    int64_t total_rows = 0;
    for (int i = 0; i < n_members; ++i)
      if (members[i].NB > 0) total_rows += members[i].n_chunks;
    const int G = prefill_group(M, total_rows, block_p, cus);
    int64_t lat_wgs = 0;
    for (int i = 0; i < n_members; ++i)
      if (members[i].NB > 0 && members[i].r_pad > 0) lat_wgs += TL * (members[i].r_pad / 64);
    rows.bm = prefill_row_tile(M, total_rows, G, block_p, cus, dtype, lat_wgs);
    // K parts: when the row grid is small (prefill_row_split) and every
    // member's workspace holds the partial tiles
    int64_t items0 = 0, sp_steps = 0, n_grp = 0;
    for (int i = 0; i < n_members; ++i)
      if (members[i].NB > 0 && members[i].pf_n_groups > 0) {
        items0 += members[i].pf_n_groups * ((M + rows.bm - 1) / rows.bm);
        n_grp += members[i].pf_n_groups;
        sp_steps += members[i].nnz * block_p / ssl_prefill_step_cols(dtype);
      }
    int ksplit = prefill_row_split(items0, n_grp > 0 ? sp_steps / n_grp : 0,
                                   m_pad / ssl_prefill_step_cols(dtype), cus, rows.bm);
    for (int i = 0; i < n_members && ksplit > 1; ++i) {
      const ssl_slr_member& mb = members[i];
      if (mb.NB == 0) continue;
      const int64_t need = (int64_t)ksplit * mb.pf_n_groups * ((M + rows.bm - 1) / rows.bm) *
                           rows.bm * 64 * 4;
      if (mb.workspace_bytes < L[i].total || mb.r_pad / 64 > 64 ||
          need > prefill_split_bytes(M, mb.NB, block_p, m_pad, 0, dtype, cus))
        ksplit = 1;
    }
    // The split narrow grid, the latent's chunks included, against the tall
    // tile's: at most twice the CUs in parts plus up to 256 latent chunks can
    // overflow one round of 3 a CU on a device with fewer than 256 CUs.
    if (ksplit > 1 && rows.bm == 128 && knobs.prefill_split == 0) {
      int64_t tall = 0, narrow = 0;
      for (int i = 0; i < n_members; ++i) {
        const ssl_slr_member& mb = members[i];
        if (mb.NB == 0) continue;
        tall += mb.pf_n_groups * ((M + 255) / 256);
        narrow += mb.pf_n_groups * ((M + 127) / 128) * ksplit;
        if (mb.r_pad > 0)
          narrow += TL * (mb.r_pad / 64) * prefill_latent_split(M, m_pad, mb.r_pad, dtype).split;
      }
      if (prefill_rounds_prefer_tall(tall, narrow, cus)) {
        rows.bm = 256;
        ksplit = 1;
      }
    }
    // Part tables (skewed structures): when the groups run whole and the
    // tall grid takes at most two rounds of the device, a member whose part
    // table and partial tiles fit runs its long groups in parts. Partial
    // tiles are kept for the narrow and short tiles only, so a tall call
    // takes the narrow one.
    bool parts = false;
    if (ksplit == 1 && knobs.prefill_split == 0 && knobs.prefill_group != 2) {
      int64_t tall = 0;
      for (int i = 0; i < n_members; ++i)
        if (members[i].NB > 0) tall += members[i].pf_n_groups * ((M + 255) / 256);
      for (int i = 0; i < n_members && tall <= 4 * (int64_t)cus; ++i) {
        const ssl_slr_member& mb = members[i];
        if (mb.NB > 0 && mb.pf_parts && mb.pf_n_parts > 0 &&
            mb.workspace_bytes >= L[i].total + ssl_prefill_parts_bytes(M, mb.pf_split_parts))
          parts = true;
      }
      if (parts && rows.bm == 256) rows.bm = 128;
    }
    // Does the latent hold up rows that would otherwise start at once? Its
    // workgroups come first in the grid and each takes a row workgroup's slot
    // (LDS) until it ends: when the row grid fits one round of the device but
    // not beside the latent, the rows pushed out wait for the whole latent,
    // so it runs in short chunks (4096×11008 with Zipf 16×16 blocks at 50% and
    // 2048 tokens: 64 rows started after the 173-step latent, at 67 µs).
    bool lat_contends = false;
    if (ksplit == 1) {
      int64_t row_items = 0, lat_items = 0;
      for (int i = 0; i < n_members; ++i) {
        const ssl_slr_member& mb = members[i];
        if (mb.NB == 0) continue;
        const int64_t T = (M + rows.bm - 1) / rows.bm;
        const bool mp = parts && mb.pf_parts && mb.pf_n_parts > 0 &&
                        mb.workspace_bytes >= L[i].total + ssl_prefill_parts_bytes(M, mb.pf_split_parts);
        row_items += (mp ? mb.pf_n_parts : mb.pf_n_groups) * T;
        if (mb.r_pad > 0) lat_items += TL * (mb.r_pad / 64);
      }
      const int64_t slots = (rows.bm == 256 ? 2 : 3) * (int64_t)cus;
      lat_contends = row_items <= slots && row_items + lat_items > slots;
    }
    int64_t items = 0, litems = 0;
    for (int i = 0; i < n_members; ++i) {
      const ssl_slr_member& mb = members[i];
      PfMember& pm = rows.mb[i];
      rows.off[i] = (int)items;
      lat.off[i] = (int)litems;
      if (mb.NB == 0) continue;
      if (!mb.pf_groups || !mb.pf_steps || mb.pf_n_groups <= 0 || mb.pf_group != G ||
          (mb.nnz > 0 && !mb.values_pq))
        return fail(SSL_ERR_INVALID, "linear %d: calls with %lld token rows need a prefill plan "
                    "with group %d and %s", i, (long long)M, G,
                    nm ? "2:4 blocks in the prefill layout" : "(p, q) ordered block values");
      const int64_t T = (M + rows.bm - 1) / rows.bm;
      if (mb.nnz < 0 || mb.nnz * blk_bytes > 0x7fffffffLL ||
          mb.NB * block_p * mb.r_pad * eb > 0x7fffffffLL || M * mb.ldy * eb > 0x7fffffffLL ||
          (int64_t)mb.r_pad * m_pad * eb > 0x7fffffffLL)
        return fail(SSL_ERR_UNSUPPORTED, "linear %d: weights or output beyond 2 GiB", i);
      pm.y = mb.y; pm.ldy = mb.ldy; pm.A = mb.A; pm.lda = mb.r_pad; pm.NB = (int)mb.NB;
      pm.A_bytes = mb.NB * block_p * mb.r_pad * eb; pm.bias = mb.bias;
      pm.values_pq = mb.values_pq; pm.values_bytes = mb.nnz * blk_bytes;
      pm.groups = mb.pf_groups; pm.steps = mb.pf_steps; pm.n_groups = (int)mb.pf_n_groups;
      pm.B = mb.B; pm.ldb = m_pad;
      pm.t = (char*)mb.workspace + L[i].t_final; pm.ldt = mb.r_pad;
      pm.tcnt = mb.r_pad > 0 ? mb.counters + L[i].pf_cnt : nullptr;
      pm.r_pad = (int)mb.r_pad;
      // the row parts' tiles first in the member's split region, then the latent's
      const int64_t rows_bytes = prefill_split_bytes(M, mb.NB, block_p, m_pad, 0, dtype, cus);
      pm.ksplit = ksplit;
      pm.kchunk = 0;
      pm.kpart = (float*)((char*)mb.workspace + L[i].pf_split);
      pm.karrive = mb.counters + L[i].pf_rarrive;
      lat.mb[i] = pm;
      lat.mb[i].parts = nullptr;
      const int64_t lat_steps = m_pad / ssl_prefill_step_cols(dtype);
      PfLatentSplit ls{1, (int)lat_steps};
      if (ksplit > 1) {
        ls = prefill_latent_split(M, m_pad, mb.r_pad, dtype);
      } else if (mb.r_pad > 0) {
        // whole row groups: the latent splits when it is longer than their
        // sparse steps and the workspace holds its partial tiles
        const int64_t group_steps = mb.nnz * block_p / ssl_prefill_step_cols(dtype) /
                                    (mb.pf_n_groups > 0 ? mb.pf_n_groups : 1);
        ls = prefill_latent_split_whole(M, m_pad, mb.r_pad, dtype,
                                        lat_contends ? group_steps / 8 : group_steps, cus);
        if (ls.split > 1 && mb.workspace_bytes < L[i].pf_split + rows_bytes +
                                                     prefill_latent_part_bytes(M, mb.r_pad, ls.split))
          ls = PfLatentSplit{1, (int)lat_steps};
      }
      lat.mb[i].ksplit = ls.split;
      lat.mb[i].kchunk = ls.chunk;
      lat.mb[i].kpart = (float*)((char*)mb.workspace + L[i].pf_split + rows_bytes);
      if (parts && mb.pf_parts && mb.pf_n_parts > 0 &&
          mb.workspace_bytes >= L[i].total + ssl_prefill_parts_bytes(M, mb.pf_split_parts)) {
        if (mb.pf_n_parts < mb.pf_n_groups || mb.pf_split_parts < 0 ||
            mb.pf_split_parts > mb.pf_n_parts || mb.pf_n_parts > 0x7fffffffLL / 8)
          return fail(SSL_ERR_INVALID, "linear %d: part table sizes do not fit its plan", i);
        pm.parts = mb.pf_parts;
        pm.n_parts = (int)mb.pf_n_parts;
        pm.split_parts = (int)mb.pf_split_parts;
        pm.kpart = (float*)((char*)mb.workspace + L[i].total);
        items += mb.pf_n_parts * T;
      } else {
        items += mb.pf_n_groups * T * ksplit;
      }
      if (mb.r_pad > 0) litems += TL * (mb.r_pad / 64) * ls.split;
      if (items > 0x7fffffffLL / 8 || litems > 0x7fffffffLL) return fail(SSL_ERR_INVALID, "grid too large");
    }
    rows.off[n_members] = (int)items;
    lat.off[n_members] = (int)litems;
    rows.items = (int)items;
    lat.items = (int)litems;
    if (nm)
      return check_hip(prefill_launch_fused_nm24(dtype, rows, lat, (hipStream_t)stream),
                       "slr prefill launch (2:4)");
    return check_hip(prefill_launch_fused(dtype, block_p, G, rows, lat, (hipStream_t)stream),
                     "slr prefill launch");
  }

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
    fill_args(g.m[i], mb, L[i], x, ldx, M, m, m_pad, n_kc, ku_chunk, dtype, block_p, block_q,
              s_format);
  }
  g.lat_off[n_members] = (int)lat;
  g.str_off[n_members] = (int)str;
  g.lat_total = (int)lat;
  if (s_format == SSL_S_NM24)
    return check_hip(dispatch(dtype, MODE_FUSED, SF_NM24, kNmBlock, 8, L[0].MT, g, lat + str,
                              (hipStream_t)stream),
                     "slr launch (2:4)");
  return check_hip(dispatch(dtype, MODE_FUSED, SF_BSR, block_p, stream_ke(dtype, block_q), L[0].MT,
                            g, lat + str, (hipStream_t)stream),
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

int64_t ssl_slr_chain_sync_count(int64_t M) {
  if (M <= 0) return 0;
  const int MT = tile_mt(M);
  return (int64_t)kDepCopies * kDepSlotInts * ((M + 16 * MT - 1) / (16 * MT));
}

int64_t ssl_slr_chain_frag_bytes(int64_t M, int64_t n_out) {
  if (M <= 0 || n_out <= 0) return 0;
  const int MT = tile_mt(M);
  const int64_t tiles = (M + 16 * MT - 1) / (16 * MT) * MT;
  return tiles * ((n_out + 31) / 32) * 1024;
}

int ssl_slr_forward_chain(int64_t M, int32_t block_p, int32_t block_q, int32_t dtype,
                          const ssl_slr_stage* stages, int32_t n_stages,
                          const ssl_slr_member* members, int32_t n_members, void* stream) {
  clear_error();
  ChainArgs c{};
  if (int rc = build_chain<kMaxChain>(M, block_p, block_q, dtype, stages, n_stages, members,
                                      n_members, SSL_MAX_CHAIN_STAGES, &c))
    return rc;
  if (c.grid == 0) return SSL_OK;
  return launch_chain(c, &c, nullptr, (hipStream_t)stream);
}

int64_t ssl_slr_chain_table_bytes(void) { return (int64_t)sizeof(ChainTab); }

int ssl_slr_chain_table_build(int64_t M, int32_t block_p, int32_t block_q, int32_t dtype,
                              const ssl_slr_stage* stages, int32_t n_stages,
                              const ssl_slr_member* members, int32_t n_members, void* table,
                              int64_t table_bytes) {
  clear_error();
  if (!table || table_bytes < (int64_t)sizeof(ChainTab) || !aligned(table, 16))
    return fail(SSL_ERR_WORKSPACE, "a chain table needs %lld bytes, 16-byte aligned",
                (long long)sizeof(ChainTab));
  ChainTab* c = (ChainTab*)table;
  memset(c, 0, sizeof(ChainTab));
  return build_chain<kMaxChainTab>(M, block_p, block_q, dtype, stages, n_stages, members,
                                   n_members, kMaxChainTab, c);
}

int ssl_slr_chain_table_launch(const void* table_host, const void* table_dev, void* stream) {
  clear_error();
  if (!table_host || !table_dev || !aligned(table_dev, 16))
    return fail(SSL_ERR_INVALID, "a chain table launch needs the host table and its device copy "
                "(16-byte aligned)");
  const ChainTab& c = *(const ChainTab*)table_host;
  if (c.grid <= 0) return SSL_OK;
  if ((c.dtype != SSL_BF16 && c.dtype != SSL_F16) || c.M <= 0 || c.n_seg <= 0 ||
      c.n_seg > 2 * kMaxChainTab)
    return fail(SSL_ERR_INVALID, "not a chain table (build it with ssl_slr_chain_table_build)");
  return launch_chain(c, nullptr, (const ChainTab*)table_dev, (hipStream_t)stream);
}

}  // extern "C"
