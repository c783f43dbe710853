// Internal launch interface shared by the operator ABI (q3_ops.hip) and the
// model orchestration (q3_model.hip).  All pointers are device addresses;
// strides are in elements.  Launchers only enqueue work on `stream`.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q3 {

// ---- measurement hook ------------------------------------------------------
// When set (by the model's kernel timing), the decode launchers time their
// kernel with hipExtLaunchKernel start/stop events: the dispatch packet's own
// timestamps, no extra queue packets.
struct LaunchEvents {
  hipEvent_t start, stop;
};
extern thread_local const LaunchEvents *g_launch_events;

#define Q3_LAUNCH(kern, grid, block, shmem, stream, ...)                                      \
  do {                                                                                       \
    if (::q3::g_launch_events)                                                               \
      hipExtLaunchKernelGGL(kern, grid, block, shmem, stream, ::q3::g_launch_events->start,  \
                            ::q3::g_launch_events->stop, 0, __VA_ARGS__);                    \
    else                                                                                     \
      hipLaunchKernelGGL(kern, grid, block, shmem, stream, __VA_ARGS__);                     \
  } while (0)

// ---- row kernels: embedding gather, RMSNorm, per-group quantisation ----
struct RowArgs {
  int mode;  // 0: quant only (y = x), 1: rmsnorm, 2: embedding + rmsnorm
  int rows, cols;
  // input
  const float *x;
  int64_t ldx;
  const int8_t *table;  // mode 2: [V][cols] i8
  int64_t ldt;
  int64_t table_rows;   // mode 2: V (ids outside [0, V) read as a zero row)
  const float *tscale;  // mode 2: per-row scale, stride tss
  int64_t tss;
  const int32_t *ids;   // mode 2: ids, stride ids_stride
  int64_t ids_stride;
  const int32_t *ids_base_pos;  // mode 2 (optional): ids += *ids_base_pos
  float *x_out;         // mode 2: dequantised embedding rows (may be null)
  int64_t ldxo;
  // rmsnorm
  const float *w;
  int64_t w_stride;
  float inv;
  float *h;             // normalised rows (may be null)
  int64_t ldh;
  // quantisation (skipped when h8 == null)
  int8_t *h8;
  int64_t ldh8;
  float *hs;
  int64_t ldhs;
  int group;
};
hipError_t launch_rows(const RowArgs &a, hipStream_t s);

// ---- group GEMM --------------------------------------------------------
enum Epi : int {
  EPI_STORE = 0,   // out = D
  EPI_ADD = 1,     // add += D
  EPI_HEADQ = 2,   // per-128-column int8 quant (V)
  EPI_NRQ = 3,     // per-head RMSNorm + RoPE + int8 quant (Q, K)
  EPI_ARGMAX = 4,  // fold D into per-row (max, first index) keys
  EPI_SWIGLU = 5,  // gate/up pair -> f32 SwiGLU (decode GEMV only)
  EPI_SWIGLUQ = 6, // gate/up pair -> SwiGLU -> per-256-column int8 quant (tiled)
  EPI_QKV = 7,     // column segments with their own weights and HEADQ/NRQ epilogue (tiled)
};

// Destination of the HEADQ/NRQ int8 rows: either a dense [M][N] i8 view
// with [M][N/128] scales, or the paged KV pool (row m -> token pos0 + m).
struct QDest {
  int8_t *q8;
  int64_t ldq8;
  float *qs;
  int64_t ldqs;        // elements between rows of qs
  int64_t qs_col;      // elements between heads of qs
  // paged (used when table != null)
  const uint16_t *table;
  uint32_t page_tokens;
  int64_t page_bytes, row_bytes;             // i8 pages
  int64_t scale_page_bytes, scale_row_bytes; // f32 pages
  uint32_t pos0;
  const int32_t *pos_dev;  // optional: pos0 += *pos_dev
  // optional (paged): row m of a batch of independent sequences goes to
  // position row_pos[m] through its own table row_tables + m * ld_table
  const int32_t *row_pos;
  const uint16_t *row_tables;
  int64_t ld_table;
};

struct GemmArgs {
  int M, N, K, group;
  const int8_t *a;
  int64_t lda;
  const float *as;
  int64_t ldas;       // elements between rows of a_scale
  const int8_t *b;
  int64_t ldb;
  const float *bs;
  int64_t bs_stride;  // elements between consecutive b_scale entries
  // per-(row, K-group) B scales bs[n * bs_ld + g] when bs_ld > 0 (EPI_STORE
  // and EPI_ADD only); 0: one scale per row, bs[n * bs_stride]
  int64_t bs_ld;
  int epi;
  float *out;
  int64_t ldo;        // EPI_STORE / EPI_ADD target
  QDest qd;
  // EPI_NRQ
  const float *nw;
  int64_t nw_stride;
  const float *cos_t, *sin_t;  // [rows][64] at the rows' absolute positions
  int64_t ld_cs;
  const int32_t *cs_row_dev;   // optional: cos/sin row offset (device scalar)
  float inv_hd;
  // EPI_ARGMAX: one key per (row, column block of 128) at keys[m * keys_ld + blockIdx.x]
  unsigned long long *keys;
  int64_t keys_ld;
};
hipError_t launch_gemm(const GemmArgs &a, hipStream_t s);

// Finishes EPI_ARGMAX: reduces the nslots per-workgroup keys of each row
// and merges the winner into (best[m], bidx[m]) with the strict
// `best < value` rule (init != 0: start from -3e38 / 0 instead of the
// current contents); optionally writes the winning id to ids[*pos] (row 0),
// or, with ids_per_row, row m's id to ids_out[m].
hipError_t launch_argmax_finish(const unsigned long long *keys, int64_t keys_ld, int nslots,
                                int M, float *best,
                                int64_t best_stride, int32_t *bidx,
                                int64_t bidx_stride, int init, int32_t *ids_out,
                                const int32_t *pos_dev, int pos_add,
                                hipStream_t s, int ids_per_row = 0);

// ---- LDS-staged tiled group GEMM (prefill, M >= 64) ----------------------
// b1/bs1: the up matrix of EPI_SWIGLUQ (b0/bs0 gate).  Epilogues: STORE, ADD
// (out), HEADQ / NRQ (qd and the NRQ fields), SWIGLUQ (s8 / ss).
struct TileArgs {
  int M, N, K, group;
  const int8_t *a;
  int64_t lda;
  const float *as;
  int64_t ldas;
  const int8_t *b0, *b1;
  int64_t ldb;
  // b0 / b1 / seg[].b in the packed layout of launch_pack_b (stream kernel
  // only; ldb unused)
  int b_packed;
  const float *bs0, *bs1;
  int64_t bs_stride;
  int64_t bs_ld;  // GemmArgs::bs_ld (EPI_STORE / EPI_ADD)
  float *out;
  int64_t ldo;
  QDest qd;
  const float *nw;
  int64_t nw_stride;
  const float *cos_t, *sin_t;
  int64_t ld_cs;
  const int32_t *cs_row_dev;
  float inv_hd;
  const int32_t *cs_row_pos;  // optional: RoPE row of output row m = cs_row_pos[m]
  int8_t *s8;
  int64_t lds8;
  float *ss;
  int64_t ldss, ss_col;
  unsigned long long *keys;  // EPI_ARGMAX: [M][keys_ld], one key per 128-column tile
  int64_t keys_ld;
  // EPI_QKV: N = sum of the segments' widths (multiples of 128); segment i
  // covers columns [n0, n1) with its own weights b / scales bs (ldb and
  // bs_stride shared), destination qd, and, if norm, RMSNorm gains nw
  // (+ RoPE with the shared cos/sin rows) before the quant (else HEADQ).
  int nseg;
  struct Seg {
    int n0, n1;
    const int8_t *b;
    const float *bs;
    QDest qd;
    const float *nw;
    int norm;
  } seg[3];
};
bool gemm_tile_supported(const TileArgs &a, int epi);
hipError_t launch_gemm_tile(const TileArgs &a, int epi, hipStream_t s);
// Prefill shapes (M > 64, K = 1024..3072 in steps of 1024): the A tile in
// LDS, the weights streamed to registers (k_gemm_stream.hip).  Epilogues
// STORE, ADD, HEADQ, NRQ, QKV, SWIGLUQ.  launch_gemm_tile takes this path
// for the shapes it supports unless Q3_PREFILL_GEMM=tile.
bool gemm_stream_supported(const TileArgs &a, int epi);
hipError_t launch_gemm_stream(const TileArgs &a, int epi, hipStream_t s);
// Weights [N][K] (row stride ldb) in the layout the stream kernel reads with
// one contiguous 1 KiB load per MFMA operand fragment: fragment (16-row
// block nb, 64-byte k-slice s) at byte 1024 (nb * K / 64 + s), lane
// l = r + 16 q of it holding row 16 nb + r, bytes 64 s + 16 q .. + 15.
hipError_t launch_pack_b(const int8_t *b, int64_t ldb, int N, int K, int8_t *out, hipStream_t s);

// ---- fused gate/up GEMM + SwiGLU + per-256-column quant -----------------
struct GateUpArgs {
  int M, N, K, group;
  const int8_t *a;
  int64_t lda;
  const float *as;
  int64_t ldas;
  const int8_t *wg, *wu;
  int64_t ldw;
  const float *wgs, *wus;
  int64_t ws_stride;
  int8_t *s8;
  int64_t lds8;
  float *ss;
  int64_t ldss;
  int64_t ss_col;
};
hipError_t launch_gate_up(const GateUpArgs &a, hipStream_t s);

// ---- paged GQA attention -------------------------------------------------
// the merged launch's x exchange words (AttnArgs::xw): kXwCopies copies of
// the row, kXwStride words apart, each read by 1 / kXwCopies of the
// pollers (one copy's lines read by all of them are served one request at
// a time); kXwEmpty marks a word not yet stored
constexpr uint32_t kXwEmpty = 0xFFFFFFFFu;
constexpr int kXwCopies = 8;
constexpr int kXwStride = 1024 + 64;
constexpr int kXwWords = kXwCopies * kXwStride;

struct AttnArgs {
  int rows, heads, kv_heads;  // head_dim is 128
  uint32_t kv_len;
  const int32_t *kv_len_dev;  // optional: kv_len += *kv_len_dev
  int causal;
  float qk_scale;
  const int8_t *q8;
  int64_t ldq;
  const float *qs;
  int64_t ldqs;
  int64_t qs_col;
  const int8_t *k, *v;
  const float *ks, *vs;
  const uint16_t *table;
  uint32_t page_tokens;
  int64_t page_bytes, row_bytes, scale_page_bytes, scale_row_bytes;
  int8_t *o8;
  int64_t ldo;
  float *os;
  int64_t ldos;
  int64_t os_col;
  float *attn;   // optional f32 attention output [rows][heads*128]
  int64_t ld_attn;
  // decode kernel only: when fuse_heads != 0 the kernel first runs the head
  // epilogues of the new token (row 0 of fq/fk/fv, position kv_len - 1):
  // K norm+RoPE+quant and V quant into their page slots, Q norm+RoPE+quant
  // into q8/qs (which must then be writable).
  int fuse_heads;
  // with fuse_heads (or blk_page_n, below): the page ids of the first 32 key
  // blocks (blk_page[j] = table[32 j / page_tokens], j < min(32, blocks)) and of
  // the new token (table[(kv_len - 1) / page_tokens]), copied from the
  // caller's host mirror of the table, so that the first K/V addresses come
  // from kernel arguments instead of a table load.  With fuse_heads every
  // entry is set: those past the last block repeat its page (the kernel
  // reads its first chunk's entries without clamping them to the block
  // count, so the reads do not wait for kv_len)
  uint32_t blk_page[32];
  uint32_t new_page;
  const float *fq, *fk, *fv;
  const float *nq, *nk;
  const float *cos_row, *sin_row;
  float inv_hd;
  // decode kernel only: pf_wgs extra workgroups read these byte ranges once
  // (values discarded) while the attention workgroups run, so that the
  // kernels after it find their weights in the last-level cache
  int pf_n, pf_wgs;
  const int8_t *pf[12];
  int64_t pf_bytes[12];
  // decode kernel only, independent sequences: when row_pos != null the
  // launch covers `rows` sequences (one query row each): sequence r attends
  // over row_pos[r] + 1 keys through page table row_tables + r * ld_table, and
  // reads/writes row r of q8/qs/o8/os (kv_len and table are ignored)
  const int32_t *row_pos;
  const uint16_t *row_tables;
  int64_t ld_table;
  // decode kernel with fuse_heads only: the O projection's per-head group
  // partials (group = head, group_gemm.h:27-222 with ref_qwen3.py:145-158)
  //   opart[h * ld_opart + n] = RN(RN(f32(o8_h . wo[n][128h, 128h + 128))
  //                                   * wos[n]) * os_h),  n < o_rows
  // are written by head h's workgroup; the residual add sums them in head
  // order (GemvArgs::part).  wo: [o_rows][ldwo] int8.
  const int8_t *wo;
  const float *wos;
  int64_t ldwo;
  int o_rows;
  float *opart;
  int64_t ld_opart;
  // prefill kernel (optional): blk_page[j] is valid for j < blk_page_n <= 32
  // (else the table is read)
  int blk_page_n;
  // (last, so that the fields above keep their kernel-argument offsets)
  // fused b = 1 variant only: pf_kv_heads > 0 marks the last four ranges'
  // pf[] as the next attention's K pool, V pool, K scale pool and V scale
  // pool (their pf_bytes unused), whose logical pages 0 .. pf_pages - 1
  // (page ids from the device table pf_table; page and row strides as in
  // this call) are read into the L2 of the XCD that will read them: query
  // head h's workgroup is workgroup h of the grid's first row, which the
  // round-robin dispatch puts on XCD h % 8, so the prefetch workgroups on
  // XCD x read the HD-byte slices of the kv heads of the query heads
  // h = x (mod 8) (of pf_kv_heads) of every row of those pages, and their
  // scale rows.  Only the sequence's own pages are read, however the table
  // is fragmented.
  int pf_kv_heads;
  // fused Q|K|V + attention launch only (launch_qkv_attn): the projection's
  // outputs as 64-bit words ((1 << 32) | f32 bits) stored by the GEMV
  // workgroups and polled by the attention workgroups, which read them in
  // place of fq/fk/fv and write 0 back: [Q: heads][K: heads][V: heads] x 128
  // (K and V once per query head of their kv head, so that every word has
  // one reader).  3 * heads * 128 zero-initialised words.  A poll that gives
  // up (a lost workgroup: every wave still exits) sets *xerr to 1.
  unsigned long long *xin;
  uint32_t *xerr;
  // the prefetch's page table and page count (pf_kv_heads)
  const uint16_t *pf_table;
  int pf_pages;
  // merged launch (launch_down_qkv_attn): the residual row after the
  // previous layer's down projection as f32 bits (kXwWords: kXwCopies
  // copies), stored by the workgroup that computed each column and read by
  // all projection workgroups; 0xFFFFFFFF (kXwEmpty, a NaN no arithmetic
  // here produces from other inputs) before the launch, set by the launch
  // that follows (GemvArgs::clear)
  uint32_t *xw;
};
hipError_t launch_attention(const AttnArgs &a, hipStream_t s);
// the two multi-row kernels behind launch_attention: the phase-parallel one
// (default) and the block-order walk (Q3_PREFILL_ATTN=walk)
hipError_t launch_attn_prefill(const AttnArgs &a, hipStream_t s);
bool attn_prefill_supported(const AttnArgs &a);
hipError_t launch_attention_walk(const AttnArgs &a, hipStream_t s);

// ---- standalone per-head norm + RoPE + quant (f32 input) -----------------
struct NrqArgs {
  int rows, heads;
  const float *x;
  int64_t ldx;
  const float *nw;
  int64_t nw_stride;
  const float *cos_t, *sin_t;
  int64_t ld_cs;
  float inv_hd;
  int do_rope;
  int8_t *q8;
  int64_t ldq8;
  float *qs;
  int64_t ldqs, qs_col;
};
hipError_t launch_nrq_rows(const NrqArgs &a, hipStream_t s);

// ---- decode-shaped group GEMM (M <= 64) ---------------------------------
// One launch can cover up to three column ranges with their own weights and
// epilogue (fused Q/K/V).  No grid-wide synchronisation.  Prologues, O
// partials and the lm_head's column streaming take at most 16 rows.
enum Pro : int {
  PRO_NONE = 0,   // A operand int8 + scales from global memory
  PRO_NORM = 1,   // A = quant256(rmsnorm(x, w_pre))
  PRO_QUANT = 2,  // A = quant256(x)
  PRO_EMBED = 3,  // A = quant256(rmsnorm(emb[ids] * emb_s[ids], w_pre))
};
struct GemvSeg {
  int n0, n1;  // columns [n0, n1) of the launch
  int epi;     // EPI_STORE / EPI_ADD / EPI_ARGMAX / EPI_SWIGLU
  const int8_t *b, *b2;    // [n1-n0][K] rows (b2: up rows for EPI_SWIGLU)
  const float *bs, *bs2;   // per-row scales
  float *out;
  int64_t ldo;
};
struct GemvArgs {
  int M, K, group;
  const int8_t *a;  // PRO_NONE
  int64_t lda;
  const float *as;
  int64_t ldas;
  int pro;
  const float *x;   // PRO_NORM / PRO_QUANT rows (ldx); PRO_EMBED: x_out rows
  int64_t ldx;
  const float *w_pre;
  float inv_pre;
  const int8_t *emb;
  const float *emb_s;
  const int32_t *ids;
  int64_t vocab;
  float *x_out;     // PRO_EMBED: dequantised rows (written by workgroup 0)
  float *h_out;     // stage buffers written by workgroup 0 (may be null)
  int8_t *h8_out;
  float *hs_out;
  int nseg;
  GemvSeg seg[3];
  unsigned long long *keys;  // EPI_ARGMAX: [M][keys_ld] one key per workgroup
  int64_t keys_ld;
  // O projection partials of the decode attention (AttnArgs::opart), M = 1:
  // o = ((0 + part[0]) + part[1]) + ... + part[npart - 1] (1 <= npart <= 16,
  // row stride ld_part).  PRO_NORM normalises x + o instead of x; EPI_ADD
  // stores (dst + o) + out instead of dst + out (same columns as dst).
  const float *part;
  int npart;
  int64_t ld_part;
  // per-(row, K-group) B scales of segment 0 (PRO_NONE, EPI_STORE / EPI_ADD,
  // one segment): seg[0].bs[n * bs_ld + g]; 0: per-row scales
  int64_t bs_ld;
  // M = 1 whole-row launches: thread i of the grid writes kXwEmpty to
  // clear[i], i < nclear (the decode launch after a merged down + Q|K|V +
  // attention launch empties its x exchange words, which have many readers)
  uint32_t *clear;
  int nclear;
};
// (GemvArgs is read by every decode GEMV workgroup: fields added past its
// sixth 64-byte line of kernel arguments cost each workgroup a dependent
// scalar-cache miss, ~0.25 us, where the kernel reads them)
bool gemv_supported(int M, int K, int group);
// launch_gemv accepts GemvArgs::clear for a (the whole-row kernel runs it)
bool gemv_clear_supported(const GemvArgs &a);
// 17-64 rows (also 1-16): plain A operand, no partials, fewer than 65536 columns
bool gemv_rows_supported(int M, int K, int group, int ncols);
// whether launch_gemv takes per-(row, K-group) B scales for this launch
bool gemv_group_bscale_supported(const GemvArgs &a);
// key slots per row that an EPI_ARGMAX launch writes (keys_ld must cover it)
int gemv_argmax_slots(const GemvArgs &a);
hipError_t launch_gemv(const GemvArgs &a, hipStream_t s);

// Head epilogues of the Q/K/V projections from f32 rows: per (row, head)
// RMSNorm + RoPE + quant (Q, K) or quant (V) into dense or paged int8.
struct QkvHeadArgs {
  int M, q_heads, kv_heads;
  const float *q, *k, *v;
  int64_t ldq, ldk;
  QDest qd, kd, vd;
  const float *nq, *nk;
  const float *cos_q, *sin_q, *cos_k, *sin_k;  // rows at the rows' positions
  int64_t ld_cs;
  float inv_hd;
  // independent sequences (batched decode): row m is at position row_pos[m]
  // (its RoPE row, cos_q/sin_q = table origin) and its K/V go to slot
  // row_pos[m] of page table row_tables + m * ld_table (kd/vd give the pools)
  const int32_t *row_pos;
  const uint16_t *row_tables;
  int64_t ld_table;
};
hipError_t launch_qkv_heads(const QkvHeadArgs &a, hipStream_t s);

// ---- decode attention (one query row per head) ---------------------------
bool attn_decode_supported(const AttnArgs &a);
hipError_t launch_attn_decode(const AttnArgs &a, hipStream_t s);
// One launch for a decode token's Q|K|V projection (g: M = 1, K = 1024,
// group 256, three EPI_STORE segments Q | K | V, PRO_NORM or PRO_EMBED, as
// launch_gemv takes them) and its attention with the head epilogues and the
// O projection (a: fuse_heads, opart, one query row, a.xin set): the
// attention workgroups load their K/V blocks and prefetch while the GEMV
// workgroups (the rest of the grid) compute the projection, then take
// their head's Q/K/V from a.xin.  g still writes its f32 outputs.
bool qkv_attn_supported(const GemvArgs &g, const AttnArgs &a);
hipError_t launch_qkv_attn(const GemvArgs &g, const AttnArgs &a, hipStream_t s);
// the Qwen3-0.6B head configuration (16 query, 8 kv heads) takes kernels
// with the head counts as compile-time constants (the fused decode launches'
// role counts, the prefill attention's workgroup mapping); Q3_HEAD_CONSTS=0,
// read per launch, forces the generic kernels that read them
bool head_consts(int heads, int kv_heads);
// launch_qkv_attn with the previous layer's down projection in the same
// launch: d is that GEMV (M = 1, K = inter, group 256, PRO_QUANT of the
// SwiGLU row, one EPI_ADD segment into x with the O partials, d.part, in
// its epilogue, N = hidden), g's PRO_NORM reads the new x from a.xw.  The
// GEMV workgroups compute d's columns, store them to x and a.xw, wait for
// all of a.xw, then compute g; a.opart must not be d.part (the attention of
// this launch writes it while d reads the previous layer's).
bool down_qkv_attn_supported(const GemvArgs &d, const GemvArgs &g, const AttnArgs &a);
hipError_t launch_down_qkv_attn(const GemvArgs &d, const GemvArgs &g, const AttnArgs &a, hipStream_t s);

// ---- greedy pick over a logits row (main_big.cpp:300-322) ---------------
hipError_t launch_argmax_logits(const float *logits, int vocab,
                                int32_t *out_id, const int32_t *pos_dev,
                                int pos_add, hipStream_t s);

}  // namespace q3
