/*
 * oracle/ref_qwen3.h — CPU restatement of the reference's numpy mirror
 * tools/ref_qwen3.py (qwen3-tile-ops).
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product path (qwen3-tile-ops_amd/) never links, loads or calls it.
 *
 * Every function follows one function of tools/ref_qwen3.py rounding point
 * by rounding point (each definition cites the file:line it restates).  All
 * arrays are host memory, row-major and dense unless a stride is given.
 */
#ifndef ORC_REF_QWEN3_H
#define ORC_REF_QWEN3_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* f32 primitives (ref_qwen3.py:27-63) */
float orc_exp2f(float x);
float orc_exp_f32(float x);
void orc_exp_f32_array(const float *x, float *out, size_t n);
float orc_tree_sum(const float *v, int n);
float orc_tree_max(const float *v, int n);

/* quantisation (ref_qwen3.py:69-97) */
void orc_quant_with_scale(const float *x, int n, float scale, int8_t *out);
void orc_quant_rows_heads(const float *x, int rows, int cols, int group,
                          int8_t *out, float *scale);

/* kernels (ref_qwen3.py:103-296) */
void orc_gemm_nt_group(const int8_t *a8, const float *a_scale, int rows, int k,
                       const int8_t *w8, const float *w_scale, int n,
                       int group, float *out);
/* Per-(row, group) weight scales w_scale[n][k / group]. */
void orc_gemm_nt_group_bg(const int8_t *a8, const float *a_scale, int rows, int k,
                          const int8_t *w8, const float *w_scale, int n,
                          int group, float *out);
void orc_gemm_nt_group_i32(const int8_t *a8, int rows, int k,
                           const int8_t *w8, int n, int group, int32_t *out);
void orc_rmsnorm_rows(const float *x, int rows, int cols, int x_stride,
                      const float *w, float inv, float *out, int out_stride);
void orc_rope_head_hd(const float *x, int rows, int hd, int x_stride,
                      const float *cos_t, const float *sin_t, float *out,
                      int out_stride);
void orc_swiglu(const float *gate, const float *up, size_t n, float *out);
void orc_attention_head_blocks(const int8_t *q8, int q_stride,
                               const float *q_scale, int qs_stride,
                               const int8_t *k8, const float *k_scale,
                               const int8_t *v8, const float *v_scale,
                               int kv_stride, int kvs_stride, int q_rows,
                               int kv_len, int pos0, int causal,
                               float qk_scale, int hd, float *out,
                               int out_stride);
void orc_attention_heads_gqa_tokscale(const int8_t *q8, const float *q_scale,
                                      int rows, const int8_t *k8,
                                      const float *k_scale, const int8_t *v8,
                                      const float *v_scale, int kv_len,
                                      int heads, int kv_heads, int hd,
                                      int causal, float qk_scale, float *out);
void orc_embedding_rmsnorm(const int8_t *emb8, const float *emb_scale,
                           int hidden, const int32_t *ids, int rows,
                           const float *w, float inv, float *h, float *x);

/* model (ref_qwen3.py:302-490) */
typedef struct orc_layer {
  const int8_t *wq, *wk, *wv, *wo, *wg, *wu, *wd;
  const float *wq_s, *wk_s, *wv_s, *wo_s, *wg_s, *wu_s, *wd_s;
  const float *n1, *nq, *nk, *n2;
} orc_layer;

typedef struct orc_model {
  int hidden, heads, kv_heads, head_dim, inter, vocab, seq, max_seq, n_layers;
  const orc_layer *layers;
  const int8_t *emb8;
  const float *emb_s;
  const int8_t *lm8;
  const float *lm_s;
  const float *nf;
  const float *cos_t; /* [max_seq][head_dim/2] */
  const float *sin_t;
} orc_model;

/* Contiguous per-layer KV cache (ref_qwen3.py:344-363). */
typedef struct orc_cache {
  int8_t *k8; /* [max_seq][kv_heads*head_dim] */
  float *k_s; /* [max_seq][kv_heads] */
  int8_t *v8;
  float *v_s;
} orc_cache;

/* Last-layer stage record (ref_qwen3.py:428-434); any pointer may be NULL.
 * Each buffer holds `rows` rows of the stage's width. */
typedef struct orc_record {
  float *h;
  int8_t *h8;
  float *hs;
  float *q, *k, *v;
  int8_t *q8;
  float *qs;
  float *attn;
  int8_t *o8;
  float *os;
  float *o, *g, *u, *sw;
  int8_t *s8;
  float *ss;
  float *x;
  int32_t rows_written; /* rows of the last recorded forward */
} orc_record;

/* ref_qwen3.py:366-444 forward_chunk.  logits (may be NULL) receives the
 * [vocab] logits of the last row when want_logits != 0. */
int orc_forward_chunk(const orc_model *m, const int32_t *ids,
                      orc_cache *caches, int pos, int rows, int want_logits,
                      orc_record *rec, float *logits);

/* ref_qwen3.py:447-464 argmax_logits. */
int orc_argmax_logits(const float *logits, int vocab);

/* ref_qwen3.py:467-490 generate.  ids has n_prompt+n_gen entries (updated in
 * place with the generated ids); caches are zeroed first; last_logits
 * receives the final logits; generated receives n_gen ids.  rec (may be
 * NULL) is filled for every forward that produces logits, so it ends with
 * the last forward's last layer. */
int orc_generate(const orc_model *m, int32_t *ids, int n_prompt, int n_gen,
                 orc_cache *caches, orc_record *rec, float *last_logits,
                 int32_t *generated);

/* Number of OpenMP threads used (0 = leave the runtime default). */
void orc_set_threads(int n);
int orc_get_threads(void);

#ifdef __cplusplus
}
#endif

#endif
