/*
 * q3ops.h — C ABI of the MI355X (gfx950) Qwen3 W8A8 forward path.
 *
 * This is the drop-in boundary for qwen3-tile-ops' operator surface.  Every
 * entry point mirrors one reference operator or orchestration function; the
 * comment above each declaration names the reference interface it replaces
 * (paths are relative to the reference repository root).
 *
 * Conventions
 *  - Only POD structs, plain pointers and scalars cross the boundary (the
 *    reference rule "only scalars and MatrixView cross op boundaries",
 *    kernels/qwen3.h:7-9, kernels/matrix.h:4-19).
 *  - Every `data` pointer in a view is a DEVICE address (hipMalloc'd memory
 *    on the current device).  Columns must be dense (col_bytes == element
 *    size); rows may be strided (row_bytes >= cols * element size).
 *  - `stream` is a hipStream_t passed as void* (NULL = default stream).  All
 *    ops are asynchronous and stream-ordered and none synchronises.  None
 *    allocates, except that the first call on a stream of
 *    q3_gemm_nt_group_argmax, or of q3_gemm_gate_up_swiglu_quant with at most
 *    64 rows, allocates that stream's 4 MiB workspace (kept until the
 *    process ends; calls on one stream share it in stream order).  The
 *    workspace is keyed by the hipStream_t value: a stream created after
 *    another was destroyed may get the same handle and then shares its
 *    workspace, so work still queued on a destroyed stream must finish
 *    first.  Under graph capture on a stream that has no workspace yet, the
 *    gate/up op takes its fused kernel instead (no workspace, no allocation),
 *    while q3_gemm_nt_group_argmax would allocate: call it once on the stream
 *    before capturing, or use q3_gemm_nt_group_argmax_noalloc.
 *  - Every function returns an int status: Q3_OK (0) or a negative Q3_ERR_*.
 *    The reference silently returns on unsupported shapes
 *    (kernels/group_gemm.h:47-49, kernels/lm_argmax.h:82); that behaviour is
 *    available through q3_set_silent_unsupported(1), which turns
 *    Q3_ERR_UNSUPPORTED into a no-op returning Q3_OK.
 *  - Numerics follow tools/ref_qwen3.py rounding point by rounding point:
 *    int8 x int8 products accumulate exactly in int32; every f32 operation is
 *    one IEEE round-to-nearest-even operation (no FMA contraction), and
 *    exp(x) = exp2(RN(x * 0x3FB8AA3B)) with glibc's exp2f semantics.
 */
#ifndef Q3OPS_H
#define Q3OPS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* MatrixView dtype codes: kernels/config.h:86-90 (i8=0 u8=1 i32=2 u32=3 f32=4). */
enum {
  Q3_DT_I8 = 0,
  Q3_DT_U8 = 1,
  Q3_DT_I32 = 2,
  Q3_DT_U32 = 3,
  Q3_DT_F32 = 4
};

/* Status codes. */
enum {
  Q3_OK = 0,
  Q3_ERR_ARG = -1,         /* NULL or inconsistent argument            */
  Q3_ERR_DTYPE = -2,       /* view dtype does not match the operand     */
  Q3_ERR_VIEW = -3,        /* view shape/stride inconsistent            */
  Q3_ERR_UNSUPPORTED = -4, /* shape the reference op also rejects       */
  Q3_ERR_HIP = -5,         /* a HIP runtime call failed                 */
  Q3_ERR_MODE = -6,        /* CTRL mode > 1 (main_big.cpp:346-348)      */
  Q3_ERR_RANGE = -7        /* position / page / token id out of range   */
};

/* Output form of the lm_head stage: main_big.cpp:142 (LmHeadOut). */
enum { Q3_LM_NONE = 0, Q3_LM_LOGITS = 1, Q3_LM_ARGMAX = 2 };

/* kernels/matrix.h:27-34 (MatrixView).  data is a device address.  A view
 * with rows == 0 may have data == NULL (an empty tensor); an operator whose
 * row count is 0 returns Q3_OK without launching or writing anything, as the
 * reference's row loops then do nothing. */
typedef struct q3_view {
  void *data;
  int32_t row_bytes;
  int32_t col_bytes;
  uint32_t rows;
  uint32_t cols;
  uint8_t dtype;
} q3_view;

/* kernels/kv_pages.h:13-24 (PagedKV).  k/v pages are
 * [page][page_tokens][row_bytes] i8, ks/vs are [page][page_tokens][kv_heads]
 * f32; table maps logical page -> physical page (device u16 array). */
typedef struct q3_paged_kv {
  void *k;
  void *v;
  void *ks;
  void *vs;
  const uint16_t *table;
  uint32_t page_tokens;
  uint32_t page_bytes;
  uint32_t row_bytes;
  uint32_t scale_page_bytes;
  uint32_t scale_row_bytes;
} q3_paged_kv;

/* Returns the previous setting.  1: unsupported shapes are a silent no-op
 * (reference behaviour), 0 (default): they return Q3_ERR_UNSUPPORTED. */
int q3_set_silent_unsupported(int on);

/* Human-readable name of a status code (static storage). */
const char *q3_status_str(int status);

/* ------------------------------------------------------------------------ */
/* Operators (one per reference op in the kernels/ headers)                */
/* ------------------------------------------------------------------------ */

/* kernels/embedding.h:99-168 embedding_rmsnorm_rows(table, scale, ids, tmp,
 * w, out, inv): tmp[r] = f32(table[ids[r]]) * scale[ids[r]];
 * out[r] = rmsnorm(tmp[r], w, inv).  table i8 [V][H], scale f32 [V][1],
 * ids i32 [rows][1], tmp/out f32 [rows][H], w f32 [H][1]. */
int q3_embedding_rmsnorm_rows(const q3_view *table, const q3_view *scale,
                              const q3_view *ids, const q3_view *tmp,
                              const q3_view *w, const q3_view *out, float inv,
                              void *stream);

/* kernels/rmsnorm.h:34-81 rmsnorm_rows(x, w, out, inv). */
int q3_rmsnorm_rows(const q3_view *x, const q3_view *w, const q3_view *out,
                    float inv, void *stream);

/* kernels/quant.h:89-138 quant_rows_heads(x, qi8, scale, group_cols):
 * per (row, group) scale = absmax * RN(1/127); q = sat127(rne(x / scale)). */
int q3_quant_rows_heads(const q3_view *x, const q3_view *qi8,
                        const q3_view *scale, uint32_t group_cols,
                        void *stream);

/* kernels/group_gemm.h:27-222 gemm_nt_group_store(a, a_scale, b, b_scale,
 * out, group_k, add, q8, qs, nw, cos, sin, inv_hd).
 *   D[m,n] = sum_g RN(RN(f32(I32_g[m,n]) * b_scale[n]) * a_scale[m,g]),
 *   summed in group order from +0.0f, where I32_g is the exact int32 dot
 *   product over K-group g.  a i8 [M][K], a_scale f32 [M][K/group_k],
 *   b i8 [N][K], b_scale f32 [N][1].  b_scale may instead be [N][K/group_k]
 *   (K/group_k > 1), one scale per weight row and K-group (BASELINE config 1's
 *   form; not in the reference): the term is then
 *   RN(RN(f32(I32_g[m,n]) * b_scale[n,g]) * a_scale[m,g]), and only the
 *   plain and residual stores accept it (other epilogues and the other GEMM
 *   ops return Q3_ERR_UNSUPPORTED).  Epilogue (same precedence as the
 *   reference): nw != NULL -> per-128-column head RMSNorm (gain nw, factor
 *   inv_hd), rotate-half RoPE with cos/sin rows [M][64], per-head int8 quant
 *   into q8 [M][N] / qs [M][N/128]; else q8 != NULL -> per-head int8 quant;
 *   else add != NULL -> add += D; else out = D.
 * Unlike the reference (rows <= 32, group_gemm.h:13,44) any M is accepted. */
int q3_gemm_nt_group_store(const q3_view *a, const q3_view *a_scale,
                           const q3_view *b, const q3_view *b_scale,
                           const q3_view *out, uint32_t group_k,
                           const q3_view *add, const q3_view *q8,
                           const q3_view *qs, const q3_view *nw,
                           const q3_view *cos, const q3_view *sin,
                           float inv_hd, void *stream);

/* Paged form of the K and V epilogues of gemm_nt_group_store as driven by
 * main_big.cpp:185-209: the per-head int8 rows and scales of token
 * pos0 + m are written to the page slot kv->table[(pos0+m)/page_tokens],
 * (pos0+m)%page_tokens of kv->k/kv->ks (is_v == 0, with norm/RoPE when nw
 * is non-NULL) or kv->v/kv->vs (is_v != 0).  Rows may cross pages (the
 * reference writes `rows` consecutive rows from one slot, which is only
 * valid inside one page, main_big.cpp:191-206). */
int q3_gemm_nt_group_kv_paged(const q3_view *a, const q3_view *a_scale,
                              const q3_view *b, const q3_view *b_scale,
                              uint32_t group_k, const q3_paged_kv *kv,
                              uint32_t pos0, int is_v, const q3_view *nw,
                              const q3_view *cos, const q3_view *sin,
                              float inv_hd, void *stream);

/* kernels/norm_rope_quant.h:88-111 norm_rope_quant_heads(x, w, cos, sin, q8,
 * scale, heads, inv_hd, do_rope): f32 x [rows][heads*128] -> q8/scale. */
int q3_norm_rope_quant_heads(const q3_view *x, const q3_view *w,
                             const q3_view *cos, const q3_view *sin,
                             const q3_view *q8, const q3_view *scale,
                             int heads, float inv_hd, int do_rope,
                             void *stream);

/* kernels/attention_gqa.h:549-572 attention_heads_gqa_tokscale_paged(q8,
 * q_scale, kv, kv_len, o8, os, heads, kv_heads, head_dim, causal,
 * qk_scale): per (head, row) online softmax over 32-key blocks with per-block
 * int8 P quantisation, then per-head int8 output quantisation.
 * q8 i8 [rows][heads*128], q_scale f32 [rows][heads], o8/os likewise.
 * head_dim must be 128 (the reference kernel is hd128-only). */
int q3_attention_heads_gqa_tokscale_paged(const q3_view *q8,
                                          const q3_view *q_scale,
                                          const q3_paged_kv *kv,
                                          uint32_t kv_len, const q3_view *o8,
                                          const q3_view *os, int heads,
                                          int kv_heads, int head_dim,
                                          int causal, float qk_scale,
                                          void *stream);

/* kernels/swiglu_quant.h:164-255 gemm_gate_up_swiglu_quant(a, a_scale, wg,
 * wgs, wu, wus, s8, ss, group_k): g/u as gemm_nt_group_store,
 * sw = RN(RN(g * RN(1/RN(exp(-g)+1))) * u), then per-256-column int8 quant
 * into s8 [M][I] / ss [M][I/256].  With M <= 64 (contiguous weight rows,
 * per-row weight scales, I < 65536, M * I * 4 bytes within the 4 MiB
 * workspace) the SwiGLU rows pass through the stream's workspace between a
 * GEMV over every CU and the quantisation; on a stream capturing a graph
 * that has no workspace yet it runs the fused kernel of larger M instead
 * (bit-identical results). */
int q3_gemm_gate_up_swiglu_quant(const q3_view *a, const q3_view *a_scale,
                                 const q3_view *wg, const q3_view *wgs,
                                 const q3_view *wu, const q3_view *wus,
                                 const q3_view *s8, const q3_view *ss,
                                 uint32_t group_k, void *stream);

/* kernels/lm_argmax.h:72-182 gemm_nt_group_argmax(a, a_scale, b, b_scale,
 * best, bidx, group_k): per row m, merges the logits row D[m,:] into the
 * running (best[m], bidx[m]) with the reference's strict `best < value`
 * rule, so the first index of the maximum wins and an initial best that is
 * not beaten is kept.  best f32 [M][1], bidx i32 [M][1] (read and written).
 * M <= 256.  The partial maxima between the GEMM and the final merge live in
 * a 4 MiB key workspace per (device, stream): the first call on a stream
 * allocates it (hipMalloc) and it is kept until the process ends, so calls
 * on different streams never share keys. */
int q3_gemm_nt_group_argmax(const q3_view *a, const q3_view *a_scale,
                            const q3_view *b, const q3_view *b_scale,
                            const q3_view *best, const q3_view *bidx,
                            uint32_t group_k, void *stream);

/* No counterpart in the reference.  q3_gemm_nt_group_argmax for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops
 * that forbid hipMalloc): same arguments, results and limits, but its keys
 * live in one fixed 4 MiB array of the library's device image (each device
 * holds its own copy until the process ends) and the call never allocates.
 * Shapes needing more than 2^19 keys (M x column blocks) are rejected with
 * Q3_ERR_UNSUPPORTED.  Every call on a device shares that device's array:
 * calls that overlap on one GPU (other streams, other host threads) race and
 * must be serialised by the caller. */
int q3_gemm_nt_group_argmax_noalloc(const q3_view *a, const q3_view *a_scale,
                                    const q3_view *b, const q3_view *b_scale,
                                    const q3_view *best, const q3_view *bidx,
                                    uint32_t group_k, void *stream);

/* main_big.cpp:300-322 argmax_logits: greedy pick over row 0 of logits
 * (per 32-column block, ordered-key comparison across blocks); the id is
 * written to *out_id (device i32). */
int q3_argmax_logits(const q3_view *logits, int32_t *out_id, void *stream);

/* ------------------------------------------------------------------------ */
/* Blob layout (tools/pqwf.py:95-273) and random-init writer                */
/* ------------------------------------------------------------------------ */

/* tools/pqwf.py:95-218 Layout: model shape plus every byte offset of the
 * blob.  Field names are the generated model_big.h constant names. */
typedef struct q3_layout {
  uint32_t hidden, layers, heads, kv_heads, head_dim, inter, vocab, seq,
      max_seq, half;
  int64_t kIDS, kCTRL, kX, kEMB, kLM, kNF, kCOS, kSIN;
  int64_t kLAYERW_BASE, kLAYERW_STRIDE;
  int64_t kLQ, kLQ_SCALE, kLK, kLK_SCALE, kLV, kLV_SCALE, kLO, kLO_SCALE;
  int64_t kLG, kLG_SCALE, kLU, kLU_SCALE, kLD, kLD_SCALE;
  int64_t kLAYERN_BASE, kLAYERN_STRIDE, kN1, kNQ, kNK, kN2;
  int64_t kLOGITS, kBLOCK_END;
  int64_t kH, kH8, kHS, kQ, kK, kV, kQ8, kK8, kV8, kQS, kKS, kVS;
  int64_t kATTN, kO, kO8, kOS, kG, kU, kSW, kS8, kSS, kARGF, kARGI;
  int64_t kKV_BASE, kKV_STRIDE, kKV_VOFF, kKV_SOFF, kSCRATCH_END;
} q3_layout;

/* tools/pqwf.py:137-218 Layout.compute. */
int q3_layout_compute(uint32_t hidden, uint32_t layers, uint32_t heads,
                      uint32_t kv_heads, uint32_t head_dim, uint32_t inter,
                      uint32_t vocab, uint32_t seq, uint32_t max_seq,
                      q3_layout *out);

/* tools/pqwf.py:251-273 Layout.header_text: writes the model_big.h text
 * (NUL-terminated) into buf; returns the length needed (excluding NUL). */
int q3_layout_header_text(const q3_layout *lay, char *buf, size_t cap);

/* Parameters of a deterministic random-init model (the offline stand-in for
 * tools/convert_pqwf.py:125-220, which needs the HF checkpoint).  Weights are
 * N(0, weight_std) f32 quantised per output row exactly like
 * tools/pqwf.py:72-89; norm gains are 1 + N(0, gain_std); RoPE tables follow
 * tools/convert_pqwf.py:46-52 (f64, rounded to f32); prompt ids are uniform in
 * [0, vocab) (or 100 + 10 i when ids_seed == 0, convert_pqwf.py:37-43). */
typedef struct q3_init_params {
  uint64_t weight_seed;
  uint64_t ids_seed;
  double weight_std;
  double gain_std;
  double rope_theta;
  int32_t n_prompt;
  int32_t n_gen;
  int32_t mode;
} q3_init_params;

/* Fills a HOST buffer of lay->kSCRATCH_END bytes (zeroed first).  Uses up to
 * `threads` host threads (0 = hardware concurrency).  Host only: no GPU. */
int q3_init_random_blob(const q3_layout *lay, const q3_init_params *p,
                        uint8_t *blob, int threads);

/* The generator behind q3_init_random_blob: out[i] = f32(mean + std * z_i)
 * with z_i the standard normal of (seed, stream, first + i).  Exported so
 * tests can rebuild any tensor's f32 values before quantisation. */
int q3_init_normal(uint64_t seed, uint64_t stream, uint64_t first, size_t n,
                   double mean, double std, float *out);

/* Stream id used by q3_init_random_blob for a tensor: layer < 0 addresses the
 * global tensors.  which: 0 emb, 1 lm, 2 nf, 3 wq, 4 wk, 5 wv, 6 wo, 7 wg,
 * 8 wu, 9 wd, 10 n1, 11 nq, 12 nk, 13 n2. */
uint64_t q3_init_stream_id(int layer, int which);

/* tools/pqwf.py:72-89 quantize_rows on host memory: w f32 [rows][cols] ->
 * q i8 [rows][cols], scale f32 [rows]. */
int q3_quantize_rows_host(const float *w, size_t rows, size_t cols, int8_t *q,
                          float *scale);

/* ------------------------------------------------------------------------ */
/* Model level: src/main_big.cpp                                            */
/* ------------------------------------------------------------------------ */

typedef struct q3_model q3_model;

/* main_big.cpp:55-136 make_model_views / make_layer_views over a DEVICE blob
 * of lay->kSCRATCH_END bytes laid out by tools/pqwf.py.  Allocates the page
 * table (reversed, main_big.cpp:168-171) and the fixed workspace once; no op
 * called through the handle allocates afterwards.  stream may be NULL. */
int q3_model_open(void *blob, const q3_layout *lay, void *stream,
                  q3_model **out);
/* (When the layout's seq exceeds 64 rows, open also copies every layer's
 * weights into a second device buffer in the matrix cores' fragment order,
 * for prefill chunks of more than 64 rows: about the size of the layer
 * weights, 0.44 GB at the Qwen3-0.6B shape; Q3_PACKED_WEIGHTS=0 at open, or
 * a failed allocation, keeps every read on the blob.  Decode and chunks of
 * up to 64 rows always read the blob.  The copy is a snapshot: after writing
 * new layer weights into the blob, call q3_model_repack before the next
 * forward.) */

/* Refreshes the packed weight copy from the blob's current layer weights
 * (a no-op without a copy).  Stream-ordered on the model's stream;
 * synchronises it.  No counterpart in the reference, whose ops read the
 * blob only. */
int q3_model_repack(q3_model *m);

/* Replaces the logical->physical page table (max_seq/32 entries, host
 * array).  Each entry must be < max_seq/32. */
int q3_model_set_page_table(q3_model *m, const uint16_t *table, uint32_t n);

/* main_big.cpp:145-296 forward_chunk(w, pos, rows, lm_out, optimize_tail):
 * rows <= seq tokens from ids[pos] through all layers; lm_out selects
 * Q3_LM_NONE / Q3_LM_LOGITS (logits row 0) / Q3_LM_ARGMAX (argf/argi). */
int q3_forward_chunk(q3_model *m, uint32_t pos, uint32_t rows, int lm_out,
                     int optimize_tail);

/* main_big.cpp:332-369 main(): reads CTRL = [n_prompt, n_gen, max_seq, mode]
 * from the blob, runs the chunked prefill and the greedy decode loop, and
 * writes each generated id to ids[pos] on the device.  Returns Q3_ERR_MODE
 * for mode > 1 (the reference returns 2). */
int q3_generate(q3_model *m);

/* Batched decode of n <= seq independent sequences: one
 * token each.  Replaces the reference's op-level batch path, per request:
 * paged_kv_scatter_batch (kernels/kv_pages.h) writes row r's K/V through its
 * own page table, paged attention (attention_gqa.h:549-572) runs per request
 * (tests/guest/paged_attn_multi.cpp), and every GEMM is row-independent.
 * Row r: token ids[r] (device) at position pos[r] (host), page table
 * tables + r * ld_table (host, logical -> physical page of the model's
 * pool); it attends over pos[r] + 1 keys, its K/V are written at pos[r],
 * and out_ids[r] (device) receives its greedy id.  Q3_ERR_RANGE if a
 * position or a page entry is out of range. */
int q3_decode_batch(q3_model *m, uint32_t n, const int32_t *ids, const int32_t *pos,
                    const uint16_t *tables, uint32_t ld_table, int32_t *out_ids);

/* Synchronises the model's stream and frees the handle's own allocations
 * (not the blob). */
int q3_model_close(q3_model *m);

/* The layout, device blob and stream the model was opened with (no
 * counterpart in the reference, whose model is a set of global views). */
int q3_model_info(const q3_model *m, q3_layout *lay, void **blob, void **stream);

/* A decode token's Q|K|V projection and attention share one launch
 * (Q3_DECODE_FUSE_QKV at open, default 1): bit 0 of *fused is set when
 * enabled.  With it, layer L's down projection runs in layer L + 1's
 * launch (Q3_DECODE_MERGE_DOWN at open, default 1): bit 1.  Their workgroups hand
 * the projection rows and the new residual row over in device memory with
 * bounded waits, and the merged launch's GEMV workgroups wait for each
 * other, so they must all be resident at once (another kernel holding most
 * CUs of the device meanwhile can starve them); *gave_up = 1 when, since
 * open, a wait ran out (its launch's results are wrong), else 0.
 * Synchronises the model's stream.  No counterpart in the reference (a
 * single hart). */
int q3_model_fused_status(q3_model *m, uint32_t *fused, uint32_t *gave_up);

/* ------------------------------------------------------------------------ */
/* Host engine: tools/engine.py:81-250 (PagePool, Scheduler, Engine.step)   */
/* ------------------------------------------------------------------------ */

/* Request states: tools/engine.py:15-19 (State). */
enum { Q3_REQ_WAITING = 0, Q3_REQ_PREFILL = 1, Q3_REQ_DECODE = 2, Q3_REQ_FINISHED = 3 };

/* A request record (tools/engine.py:33-59 Request: prompt length, n_fed,
 * len(generated), params.max_new, state, len(pages)). */
typedef struct q3_sched_req {
  uint32_t n_prompt, n_fed, n_gen, max_new;
  int32_t state;
  uint32_t n_pages;
} q3_sched_req;

/* One request's rows in a batch (tools/engine.py:62-70 BatchItem; `slot` is
 * the request's admission index, pos its n_fed when the batch was built). */
typedef struct q3_sched_item {
  int32_t slot;
  uint32_t row_start, rows, pos;
  int32_t prefill, needs_logits;
} q3_sched_item;

/* The scheduling core: a pool of num_pages physical pages of page_tokens
 * tokens (tools/engine.py:81-115: handed out from the top of a free stack,
 * returned to it) and the requests in admission order
 * (tools/engine.py:152-200).  Host memory only. */
typedef struct q3_sched q3_sched;
int q3_sched_create(uint32_t num_pages, uint32_t page_tokens, q3_sched **out);
int q3_sched_destroy(q3_sched *s);
/* Engine.add_request / Scheduler.add: a WAITING record; *slot = its index. */
int q3_sched_add(q3_sched *s, uint32_t n_prompt, uint32_t max_new, int32_t *slot);
int q3_sched_get(const q3_sched *s, int32_t slot, q3_sched_req *out);
/* Overwrites n_prompt, n_fed, n_gen, max_new and state (not the pages). */
int q3_sched_set(q3_sched *s, int32_t slot, const q3_sched_req *in);
/* The record's pages (logical order): *n = count, the first min(cap, *n)
 * copied to out (may be NULL). */
int q3_sched_pages(const q3_sched *s, int32_t slot, uint32_t *out, uint32_t cap, uint32_t *n);
/* The free stack, bottom to top (the next page handed out is the last). */
int q3_sched_free_pages(const q3_sched *s, uint32_t *out, uint32_t cap, uint32_t *n);
/* PagePool.alloc_page: *page = the top free page, or -1 when none is free.
 * With slot >= 0 it joins the record's pages; with slot == -1 it belongs to
 * no record and is never returned to the pool. */
int q3_sched_alloc_page(q3_sched *s, int32_t slot, int32_t *page);
/* PagePool.ensure: pages for the record's first n_tokens tokens; *ok = 0
 * when the pool runs dry (the pages found so far stay with the record). */
int q3_sched_ensure(q3_sched *s, int32_t slot, uint32_t n_tokens, int32_t *ok);
/* PagePool.release: the record's pages go back to the free stack. */
int q3_sched_release(q3_sched *s, int32_t slot);
/* Scheduler.finish: FINISHED, pages released (no-op when finished). */
int q3_sched_finish(q3_sched *s, int32_t slot);
/* Scheduler.build_batch: items in admission order (a prompt chunk of up to
 * 32 rows, or one decode row), at most max_rows rows; records at their
 * max_new are finished.  Q3_ERR_RANGE if more than cap items. */
int q3_sched_build(q3_sched *s, uint32_t max_rows, q3_sched_item *items, uint32_t cap,
                   uint32_t *n_items, uint32_t *total_rows);
/* The bookkeeping half of Engine.step after sampling: n_fed += rows; an
 * item with logits adds one generated id and finishes its request when
 * stop[i] != 0 or max_new is reached, else the request is DECODE; a prompt
 * chunk without logits leaves it PREFILL. */
int q3_sched_commit(q3_sched *s, const q3_sched_item *items, uint32_t n, const int32_t *stop);
/* Engine.step with an empty batch: finishes every request whose prompt is
 * fed and whose max_new is reached; *n_finished may be NULL. */
int q3_sched_finish_exhausted(q3_sched *s, uint32_t *n_finished);
/* The device side of a batch (the guest step): tokens holds each item's
 * row ids, concatenated in item order.  A prompt chunk, or a decode row
 * with on_device[i] == 0, runs q3_forward_chunk over the record's pages
 * (installed as the model's page table; its ids written to ids[pos..]) and,
 * when it needs logits, copies the vocab-wide logits row to
 * logits + i * ld_logits (host); decode rows with on_device[i] != 0 share
 * q3_decode_batch calls and receive their greedy id in out_ids[i] (-1 for
 * the others).  page_tokens must be 32 and every page within the model's
 * pool.  Synchronous. */
int q3_sched_run(q3_sched *s, q3_model *m, const q3_sched_item *items, uint32_t n,
                 const int32_t *tokens, const int32_t *on_device, int32_t *out_ids,
                 float *logits, uint64_t ld_logits);

/* ---- measurement (no counterpart in the reference) ------------------------
 * Decode kernel classes whose launches the model can time with HIP events on
 * its own stream (hipExtLaunchKernel start/stop events: the kernel's own
 * dispatch timestamps). */
enum {
  Q3_KT_ATTN_DECODE = 0, /* decode attention (+ fused head epilogues)     */
  Q3_KT_GEMV_QKV = 1,    /* Q|K|V projection, RMSNorm prologue            */
  Q3_KT_GEMV_O = 2,      /* O projection + residual                       */
  Q3_KT_GEMV_GATE_UP = 3,/* gate/up + SwiGLU, RMSNorm prologue            */
  Q3_KT_GEMV_DOWN = 4,   /* down projection + residual, quant prologue    */
  Q3_KT_LM_HEAD = 5,     /* lm_head GEMV (argmax mode)                    */
  Q3_KT_COUNT = 6
};

/* Enables event timing for the classes whose bit (1 << class) is set in
 * mask (0 disables).  Clears the accumulated times. */
int q3_model_set_kernel_timing(q3_model *m, uint32_t mask);

/* Synchronises the stream and returns the summed milliseconds and the
 * number of timed launches of one class since timing was enabled. */
int q3_model_kernel_time(q3_model *m, int kclass, double *total_ms, uint32_t *launches);

#ifdef __cplusplus
}
#endif

#endif /* Q3OPS_H */
