/*
 * oracle/ref_qwen3.c — CPU restatement of tools/ref_qwen3.py.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product).  Built with
 * -ffp-contract=off so that every f32 expression below is exactly one IEEE
 * round-to-nearest-even operation, like the numpy mirror it restates.
 *
 * The only host-dependent primitive of the reference is np.exp2 on float32.
 * With numpy's AVX512 dispatch disabled it equals glibc 2.35 exp2f; that
 * function is restated here from its published algorithm (ARM
 * optimized-routines exp2f, adopted by glibc 2.28: 32-entry table of
 * 2^(i/32) and a degree-3 polynomial evaluated in double) and pinned against
 * glibc exp2f over every float in [-151, 129] by oracle/exp2_check.c, which
 * tests/test_oracle_prims.py runs.
 */
#include "ref_qwen3.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define F32_LOG2E_BITS 0x3FB8AA3Bu /* ref_qwen3.py:18 */

static float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static uint64_t f64_bits(double d) {
  uint64_t u;
  memcpy(&u, &d, 8);
  return u;
}
static double bits_f64(uint64_t u) {
  double d;
  memcpy(&d, &u, 8);
  return d;
}

static float kInv127(void) { return 1.0f / 127.0f; } /* ref_qwen3.py:19 */
#define EPS 1e-6f                                      /* ref_qwen3.py:20 */
#define FLT_MAX_F 3.402823466e38f                      /* ref_qwen3.py:21 */

void orc_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

int orc_get_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ---------------------------------------------------------------------- */
/* exp2f: T[i] = bits(RN_double(2^(i/32))) - (i << 47).                    */
/* ---------------------------------------------------------------------- */
static const uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full,
    0x3fef9301d0125b51ull, 0x3fef72b83c7d517bull, 0x3fef54873168b9aaull,
    0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, 0x3fef06fe0a31b715ull,
    0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull,
    0x3feea47eb03a5585ull, 0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull,
    0x3feea11473eb0187ull, 0x3feea589994cce13ull, 0x3feeace5422aa0dbull,
    0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull,
    0x3fef3720dcef9069ull, 0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full,
    0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

float orc_exp2f(float x) {
  const uint32_t ux = f32_bits(x);
  const uint32_t abstop = (ux >> 20) & 0x7ff;
  if (abstop >= (0x43000000u >> 20)) { /* |x| >= 128 or NaN/Inf */
    if (ux == 0xff800000u) return 0.0f;
    if (abstop >= (0x7f800000u >> 20)) return x + x;
    if (x > 0.0f) return bits_f32(0x7f800000u);
    if (x <= -150.0f) return 0.0f;
  }
  const double xd = (double)x;
  const double shift = 0x1.8p+52 / 32;
  volatile double kdv = xd + shift; /* keep the rounding-to-integer add */
  double kd = kdv;
  const uint64_t ki = f64_bits(kd);
  kd -= shift;
  const double r = xd - kd;
  uint64_t t = kExp2Tab[ki % 32];
  t += ki << 47;
  const double s = bits_f64(t);
  const double z = fma(0x1.c6af84b912394p-5, r, 0x1.ebfce50fac4f3p-3);
  const double r2 = r * r;
  double y = fma(0x1.62e42ff0c52d6p-1, r, 1.0);
  y = fma(z, r2, y);
  y = y * s;
  return (float)y;
}

/* ref_qwen3.py:27-29 exp_f32 = exp2(RN(x * log2e)). */
float orc_exp_f32(float x) {
  const float t = x * bits_f32(F32_LOG2E_BITS);
  return orc_exp2f(t);
}

void orc_exp_f32_array(const float *x, float *out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_exp_f32(x[i]);
}

/* ref_qwen3.py:32-38 rcp_f32 / rsqrt_f32. */
static float rcp_f32(float x) { return 1.0f / x; }
static float rsqrt_f32(float x) { return 1.0f / sqrtf(x); }

/* ref_qwen3.py:41-50 tree_reduce_rows: pairs (0,1),(2,3),... the odd tail
 * element is carried to the next level. */
float orc_tree_sum(const float *v, int n) {
  float buf[4096];
  if (n <= 0) return 0.0f;
  memcpy(buf, v, sizeof(float) * (size_t)n);
  while (n > 1) {
    int m = n / 2;
    for (int i = 0; i < m; ++i) buf[i] = buf[2 * i] + buf[2 * i + 1];
    if (n & 1) buf[m++] = buf[n - 1];
    n = m;
  }
  return buf[0];
}

/* ref_qwen3.py:57-58 tree_max_rows: where(b > a, b, a). */
float orc_tree_max(const float *v, int n) {
  float buf[4096];
  if (n <= 0) return -INFINITY;
  memcpy(buf, v, sizeof(float) * (size_t)n);
  while (n > 1) {
    int m = n / 2;
    for (int i = 0; i < m; ++i) {
      const float a = buf[2 * i], b = buf[2 * i + 1];
      buf[i] = (b > a) ? b : a;
    }
    if (n & 1) buf[m++] = buf[n - 1];
    n = m;
  }
  return buf[0];
}

/* ref_qwen3.py:61-63 row_absmax: tree max over |x|. */
static float row_absmax(const float *v, int n) {
  float buf[4096];
  for (int i = 0; i < n; ++i) buf[i] = fabsf(v[i]);
  return orc_tree_max(buf, n);
}

/* ref_qwen3.py:69-76 quant_with_scale: rne(x/scale), NaN -> 0, sat 127. */
void orc_quant_with_scale(const float *x, int n, float scale, int8_t *out) {
  for (int i = 0; i < n; ++i) {
    const float quot = x[i] / scale;
    float r = isnan(quot) ? 0.0f : rintf(quot);
    if (r < -127.0f) r = -127.0f;
    if (r > 127.0f) r = 127.0f;
    out[i] = (int8_t)r;
  }
}

/* np.max over |x| (ref_qwen3.py:81, 90-91). */
static float plain_absmax(const float *v, int n) {
  float m = 0.0f;
  int first = 1;
  for (int i = 0; i < n; ++i) {
    const float a = fabsf(v[i]);
    if (isnan(a)) return a;
    if (first || a > m) m = a;
    first = 0;
  }
  return m;
}

/* ref_qwen3.py:86-97 quant_rows_heads. */
void orc_quant_rows_heads(const float *x, int rows, int cols, int group,
                          int8_t *out, float *scale) {
  const int groups = cols / group;
  const float inv127 = kInv127();
  for (int r = 0; r < rows; ++r)
    for (int g = 0; g < groups; ++g) {
      const float *xs = x + (size_t)r * cols + (size_t)g * group;
      const float s = plain_absmax(xs, group) * inv127;
      scale[(size_t)r * groups + g] = s;
      orc_quant_with_scale(xs, group, s, out + (size_t)r * cols + (size_t)g * group);
    }
}

/* ref_qwen3.py:103-127 imatmul_nt: exact integer dot products. */
static int32_t idot(const int8_t *a, const int8_t *b, int n) {
  int32_t acc = 0;
  for (int i = 0; i < n; ++i) acc += (int32_t)a[i] * (int32_t)b[i];
  return acc;
}

/* Per-group int32 partials I32[m][g][n] (debug view of the group GEMM). */
void orc_gemm_nt_group_i32(const int8_t *a8, int rows, int k,
                           const int8_t *w8, int n, int group, int32_t *out) {
  const int groups = k / group;
#pragma omp parallel for schedule(static)
  for (int j = 0; j < n; ++j)
    for (int r = 0; r < rows; ++r)
      for (int g = 0; g < groups; ++g)
        out[((size_t)r * groups + g) * n + j] =
            idot(a8 + (size_t)r * k + (size_t)g * group,
                 w8 + (size_t)j * k + (size_t)g * group, group);
}

/* ref_qwen3.py:145-158 gemm_nt_group: per group
 *   part = RN(RN(f32(i32) * w_scale[n]) * a_scale[m, g]); out = RN(out + part)
 * accumulated in group order from +0.0f. */
void orc_gemm_nt_group(const int8_t *a8, const float *a_scale, int rows, int k,
                       const int8_t *w8, const float *w_scale, int n,
                       int group, float *out) {
  const int groups = k / group;
#pragma omp parallel for schedule(static)
  for (int j = 0; j < n; ++j) {
    const int8_t *wj = w8 + (size_t)j * k;
    for (int r = 0; r < rows; ++r) {
      const int8_t *ar = a8 + (size_t)r * k;
      float acc = 0.0f;
      for (int g = 0; g < groups; ++g) {
        const int32_t p = idot(ar + (size_t)g * group, wj + (size_t)g * group, group);
        float part = (float)p;
        part = part * w_scale[j];
        part = part * a_scale[(size_t)r * groups + g];
        acc = acc + part;
      }
      out[(size_t)r * n + j] = acc;
    }
  }
}

/* BASELINE config 1's per-(row, group) B scales: ref_qwen3.py:145-158 with
 * w_scale[n] replaced by w_scale[n][g] (row stride `groups`), i.e.
 *   part = RN(RN(f32(i32) * w_scale[n, g]) * a_scale[m, g]); out = RN(out + part)
 * in group order from +0.0f.  Not a reference function (the reference scales
 * weights per row only, group_gemm.h:98-101); pinned by what the arithmetic
 * fixes: equal group scales reduce it to orc_gemm_nt_group bit for bit, unit
 * scales to the integer sum, and tiny shapes to the f64 sum within rounding. */
void orc_gemm_nt_group_bg(const int8_t *a8, const float *a_scale, int rows, int k,
                          const int8_t *w8, const float *w_scale, int n,
                          int group, float *out) {
  const int groups = k / group;
#pragma omp parallel for schedule(static)
  for (int j = 0; j < n; ++j) {
    const int8_t *wj = w8 + (size_t)j * k;
    const float *wsj = w_scale + (size_t)j * groups;
    for (int r = 0; r < rows; ++r) {
      const int8_t *ar = a8 + (size_t)r * k;
      float acc = 0.0f;
      for (int g = 0; g < groups; ++g) {
        const int32_t p = idot(ar + (size_t)g * group, wj + (size_t)g * group, group);
        float part = (float)p;
        part = part * wsj[g];
        part = part * a_scale[(size_t)r * groups + g];
        acc = acc + part;
      }
      out[(size_t)r * n + j] = acc;
    }
  }
}

/* ref_qwen3.py:161-173 rmsnorm_from_values. */
void orc_rmsnorm_rows(const float *x, int rows, int cols, int x_stride,
                      const float *w, float inv, float *out, int out_stride) {
  for (int r = 0; r < rows; ++r) {
    const float *xr = x + (size_t)r * x_stride;
    float ss = 0.0f;
    for (int k = 0; k < cols; k += 32) {
      const int nb = (cols - k) < 32 ? (cols - k) : 32;
      float sq[32];
      for (int i = 0; i < nb; ++i) sq[i] = xr[k + i] * xr[k + i];
      ss = ss + orc_tree_sum(sq, nb);
    }
    ss = ss * inv;
    ss = ss + EPS;
    const float rinv = rsqrt_f32(ss);
    float *o = out + (size_t)r * out_stride;
    for (int c = 0; c < cols; ++c) {
      const float t = xr[c] * rinv;
      o[c] = t * w[c];
    }
  }
}

/* ref_qwen3.py:180-191 rope_head_hd (rotate-half). */
void orc_rope_head_hd(const float *x, int rows, int hd, int x_stride,
                      const float *cos_t, const float *sin_t, float *out,
                      int out_stride) {
  const int half = hd / 2;
  for (int r = 0; r < rows; ++r) {
    const float *xr = x + (size_t)r * x_stride;
    const float *c = cos_t + (size_t)r * half;
    const float *s = sin_t + (size_t)r * half;
    float tmp[512];
    for (int i = 0; i < half; ++i) {
      const float left = xr[i], right = xr[half + i];
      const float l = left * c[i];
      const float t = right * s[i];
      const float rr = left * s[i];
      const float t2 = right * c[i];
      tmp[i] = l - t;
      tmp[half + i] = rr + t2;
    }
    memcpy(out + (size_t)r * out_stride, tmp, sizeof(float) * (size_t)hd);
  }
}

/* ref_qwen3.py:194-200 swiglu. */
void orc_swiglu(const float *gate, const float *up, size_t n, float *out) {
  for (size_t i = 0; i < n; ++i) {
    float e = gate[i] * -1.0f;
    e = orc_exp_f32(e);
    e = e + 1.0f;
    e = rcp_f32(e);
    const float t = gate[i] * e;
    out[i] = t * up[i];
  }
}

/* ref_qwen3.py:210-266 attention_head_blocks: online softmax over 32-key
 * blocks; rows are independent.  q8/k8/v8 point at the head's first column;
 * q_scale/k_scale/v_scale at the head's scale column. */
void orc_attention_head_blocks(const int8_t *q8, int q_stride,
                               const float *q_scale, int qs_stride,
                               const int8_t *k8, const float *k_scale,
                               const int8_t *v8, const float *v_scale,
                               int kv_stride, int kvs_stride, int q_rows,
                               int kv_len, int pos0, int causal,
                               float qk_scale, int hd, float *out,
                               int out_stride) {
  const float inv127 = kInv127();
  int kv_end = kv_len;
  if (causal && pos0 + q_rows < kv_end) kv_end = pos0 + q_rows;
  for (int r = 0; r < q_rows; ++r) {
    const int8_t *qr = q8 + (size_t)r * q_stride;
    const float qs = q_scale[(size_t)r * qs_stride];
    float maximum = -FLT_MAX_F;
    float den = 0.0f;
    float res[512];
    for (int d = 0; d < hd; ++d) res[d] = 0.0f;
    for (int j = 0; j < kv_end; j += 32) {
      const int nc = (kv_len - j) < 32 ? (kv_len - j) : 32;
      float s[32], p[32];
      for (int c = 0; c < nc; ++c) {
        /* 1a-1b: S = q8.k8^T (i32), then ((f32 * k) * q) * qk */
        const int32_t acc = idot(qr, k8 + (size_t)(j + c) * kv_stride, hd);
        float v = (float)acc;
        v = v * k_scale[(size_t)(j + c) * kvs_stride];
        v = v * qs;
        v = v * qk_scale;
        /* 1c: causal mask keeps (col - row) <= pos0 - j */
        if (causal && (c - r) > (pos0 - j)) v = -INFINITY;
        s[c] = v;
      }
      /* 1d: running max + correction */
      float nmm = orc_tree_max(s, nc);
      /* np.maximum(nmm, maximum) */
      if (isnan(nmm) || isnan(maximum))
        nmm = NAN;
      else
        nmm = (maximum > nmm) ? maximum : nmm;
      const float corr = orc_exp_f32(maximum - nmm);
      den = den * corr;
      for (int d = 0; d < hd; ++d) res[d] = res[d] * corr;
      for (int c = 0; c < nc; ++c) p[c] = orc_exp_f32(s[c] - nmm);
      den = den + orc_tree_sum(p, nc);
      maximum = nmm;
      /* 1e: fold the V scale, quantise P */
      for (int c = 0; c < nc; ++c) p[c] = p[c] * v_scale[(size_t)(j + c) * kvs_stride];
      const float pmax = row_absmax(p, nc) * inv127;
      int8_t pq[32];
      orc_quant_with_scale(p, nc, pmax, pq);
      /* 1f: res += f32(P8 . V) * pmax */
      for (int d = 0; d < hd; ++d) {
        int32_t acc = 0;
        for (int c = 0; c < nc; ++c)
          acc += (int32_t)pq[c] * (int32_t)v8[(size_t)(j + c) * kv_stride + d];
        float part = (float)acc;
        part = part * pmax;
        res[d] = res[d] + part;
      }
    }
    den = rcp_f32(den);
    float *o = out + (size_t)r * out_stride;
    for (int d = 0; d < hd; ++d) o[d] = res[d] * den;
  }
}

/* ref_qwen3.py:269-289 attention_heads_gqa_tokscale. */
void orc_attention_heads_gqa_tokscale(const int8_t *q8, const float *q_scale,
                                      int rows, const int8_t *k8,
                                      const float *k_scale, const int8_t *v8,
                                      const float *v_scale, int kv_len,
                                      int heads, int kv_heads, int hd,
                                      int causal, float qk_scale, float *out) {
  const int group = heads / kv_heads;
  const int pos0 = causal ? kv_len - rows : 0;
  const int qw = heads * hd, kw = kv_heads * hd;
  const int nqb = (rows + 31) / 32;
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int h = 0; h < heads; ++h)
    for (int b = 0; b < nqb; ++b) {
      const int qi = b * 32;
      const int kv = h / group;
      const int nr = (rows - qi) < 32 ? (rows - qi) : 32;
      orc_attention_head_blocks(q8 + (size_t)qi * qw + (size_t)h * hd, qw,
                                q_scale + (size_t)qi * heads + h, heads,
                                k8 + (size_t)kv * hd, k_scale + kv,
                                v8 + (size_t)kv * hd, v_scale + kv, kw,
                                kv_heads, nr, kv_len, pos0 + qi, causal,
                                qk_scale, hd,
                                out + (size_t)qi * qw + (size_t)h * hd, qw);
    }
}

/* ref_qwen3.py:292-296 embedding_rmsnorm. */
void orc_embedding_rmsnorm(const int8_t *emb8, const float *emb_scale,
                           int hidden, const int32_t *ids, int rows,
                           const float *w, float inv, float *h, float *x) {
  for (int r = 0; r < rows; ++r) {
    const int id = ids[r];
    const int8_t *e = emb8 + (size_t)id * hidden;
    for (int c = 0; c < hidden; ++c) x[(size_t)r * hidden + c] = (float)e[c] * emb_scale[id];
  }
  orc_rmsnorm_rows(x, rows, hidden, hidden, w, inv, h, hidden);
}

/* ---------------------------------------------------------------------- */
/* model                                                                  */
/* ---------------------------------------------------------------------- */
static void *xmalloc(size_t n) {
  void *p = malloc(n ? n : 1);
  if (!p) abort();
  return p;
}

static void copy_rec_f(float *dst, const float *src, size_t n) {
  if (dst) memcpy(dst, src, n * sizeof(float));
}
static void copy_rec_i8(int8_t *dst, const int8_t *src, size_t n) {
  if (dst) memcpy(dst, src, n);
}

/* ref_qwen3.py:366-444 forward_chunk. */
int orc_forward_chunk(const orc_model *m, const int32_t *ids,
                      orc_cache *caches, int pos, int rows, int want_logits,
                      orc_record *rec, float *logits) {
  const int H = m->hidden, HD = m->head_dim;
  const int QW = m->heads * HD, KW = m->kv_heads * HD, I = m->inter;
  const int half = HD / 2;
  const float inv_h = 1.0f / (float)H;
  const float inv_hd = 1.0f / (float)HD;
  const float qk_scale = (float)(1.0 / sqrt((double)HD));
  if (rows <= 0 || pos < 0 || pos + rows > m->max_seq) return -1;

  const float *cos_p = m->cos_t + (size_t)pos * half;
  const float *sin_p = m->sin_t + (size_t)pos * half;
  const size_t R = (size_t)rows;

  float *x = xmalloc(R * H * 4), *h = xmalloc(R * H * 4);
  int8_t *h8 = xmalloc(R * H);
  float *hs = xmalloc(R * (H / 256) * 4);
  float *q = xmalloc(R * QW * 4), *k = xmalloc(R * KW * 4), *v = xmalloc(R * KW * 4);
  int8_t *q8 = xmalloc(R * QW), *k8 = xmalloc(R * KW), *v8 = xmalloc(R * KW);
  float *qs = xmalloc(R * m->heads * 4), *ks = xmalloc(R * m->kv_heads * 4);
  float *vs = xmalloc(R * m->kv_heads * 4);
  float *attn = xmalloc(R * QW * 4), *o = xmalloc(R * H * 4);
  int8_t *o8 = xmalloc(R * QW);
  float *os = xmalloc(R * m->heads * 4);
  float *g = xmalloc(R * I * 4), *u = xmalloc(R * I * 4), *sw = xmalloc(R * I * 4);
  int8_t *s8 = xmalloc(R * I);
  float *ss = xmalloc(R * (I / 256) * 4);

  /* layer 0 fuses the first rmsnorm into the embedding pass */
  orc_embedding_rmsnorm(m->emb8, m->emb_s, H, ids, rows, m->layers[0].n1, inv_h, h, x);
  for (int L = 0; L < m->n_layers; ++L) {
    const orc_layer *ly = &m->layers[L];
    orc_cache *c = &caches[L];
    if (L != 0) orc_rmsnorm_rows(x, rows, H, H, ly->n1, inv_h, h, H);
    orc_quant_rows_heads(h, rows, H, 256, h8, hs);
    orc_gemm_nt_group(h8, hs, rows, H, ly->wq, ly->wq_s, QW, 256, q);
    orc_gemm_nt_group(h8, hs, rows, H, ly->wk, ly->wk_s, KW, 256, k);
    orc_gemm_nt_group(h8, hs, rows, H, ly->wv, ly->wv_s, KW, 256, v);
    /* q/k norm + rope, per head (ref_qwen3.py:393-402) */
    for (int kvm = 0; kvm < m->kv_heads; ++kvm) {
      float *kh = k + (size_t)kvm * HD;
      orc_rmsnorm_rows(kh, rows, HD, KW, ly->nk, inv_hd, kh, KW);
      orc_rope_head_hd(kh, rows, HD, KW, cos_p, sin_p, kh, KW);
    }
    for (int hh = 0; hh < m->heads; ++hh) {
      float *qh = q + (size_t)hh * HD;
      orc_rmsnorm_rows(qh, rows, HD, QW, ly->nq, inv_hd, qh, QW);
      orc_rope_head_hd(qh, rows, HD, QW, cos_p, sin_p, qh, QW);
    }
    orc_quant_rows_heads(k, rows, KW, HD, k8, ks);
    orc_quant_rows_heads(v, rows, KW, HD, v8, vs);
    memcpy(c->k8 + (size_t)pos * KW, k8, R * KW);
    memcpy(c->k_s + (size_t)pos * m->kv_heads, ks, R * m->kv_heads * 4);
    memcpy(c->v8 + (size_t)pos * KW, v8, R * KW);
    memcpy(c->v_s + (size_t)pos * m->kv_heads, vs, R * m->kv_heads * 4);
    orc_quant_rows_heads(q, rows, QW, HD, q8, qs);
    const int kv_len = pos + rows;
    orc_attention_heads_gqa_tokscale(q8, qs, rows, c->k8, c->k_s, c->v8, c->v_s,
                                     kv_len, m->heads, m->kv_heads, HD, 1,
                                     qk_scale, attn);
    orc_quant_rows_heads(attn, rows, QW, HD, o8, os);
    orc_gemm_nt_group(o8, os, rows, QW, ly->wo, ly->wo_s, H, HD, o);
    for (size_t i = 0; i < R * H; ++i) x[i] = x[i] + o[i];

    orc_rmsnorm_rows(x, rows, H, H, ly->n2, inv_h, h, H);
    orc_quant_rows_heads(h, rows, H, 256, h8, hs);
    orc_gemm_nt_group(h8, hs, rows, H, ly->wg, ly->wg_s, I, 256, g);
    orc_gemm_nt_group(h8, hs, rows, H, ly->wu, ly->wu_s, I, 256, u);
    orc_swiglu(g, u, R * I, sw);
    orc_quant_rows_heads(sw, rows, I, 256, s8, ss);
    orc_gemm_nt_group(s8, ss, rows, I, ly->wd, ly->wd_s, H, 256, o);
    for (size_t i = 0; i < R * H; ++i) x[i] = x[i] + o[i];

    if (rec && L == m->n_layers - 1) { /* record.clear()+update: last layer */
      copy_rec_f(rec->h, h, R * H);
      copy_rec_i8(rec->h8, h8, R * H);
      copy_rec_f(rec->hs, hs, R * (H / 256));
      copy_rec_f(rec->q, q, R * QW);
      copy_rec_f(rec->k, k, R * KW);
      copy_rec_f(rec->v, v, R * KW);
      copy_rec_i8(rec->q8, q8, R * QW);
      copy_rec_f(rec->qs, qs, R * m->heads);
      copy_rec_f(rec->attn, attn, R * QW);
      copy_rec_i8(rec->o8, o8, R * QW);
      copy_rec_f(rec->os, os, R * m->heads);
      copy_rec_f(rec->o, o, R * H);
      copy_rec_f(rec->g, g, R * I);
      copy_rec_f(rec->u, u, R * I);
      copy_rec_f(rec->sw, sw, R * I);
      copy_rec_i8(rec->s8, s8, R * I);
      copy_rec_f(rec->ss, ss, R * (I / 256));
      copy_rec_f(rec->x, x, R * H);
      rec->rows_written = rows;
    }
  }

  if (want_logits) { /* ref_qwen3.py:436-443 */
    float *hl = xmalloc((size_t)H * 4);
    int8_t *h8l = xmalloc((size_t)H);
    float *hsl = xmalloc((size_t)(H / 256) * 4);
    orc_rmsnorm_rows(x + (size_t)(rows - 1) * H, 1, H, H, m->nf, inv_h, hl, H);
    orc_quant_rows_heads(hl, 1, H, 256, h8l, hsl);
    if (logits) orc_gemm_nt_group(h8l, hsl, 1, H, m->lm8, m->lm_s, m->vocab, 256, logits);
    free(hl);
    free(h8l);
    free(hsl);
  }
  free(x); free(h); free(h8); free(hs); free(q); free(k); free(v);
  free(q8); free(k8); free(v8); free(qs); free(ks); free(vs);
  free(attn); free(o); free(o8); free(os); free(g); free(u); free(sw);
  free(s8); free(ss);
  return 0;
}

/* ref_qwen3.py:447-464 argmax_logits: per 32-column block np.argmax (first
 * index of the maximum), blocks compared through the ordered f32 key. */
int orc_argmax_logits(const float *logits, int vocab) {
  int best = 0;
  uint32_t best_key = 0;
  int first = 1;
  for (int n = 0; n < vocab; n += 32) {
    const int nb = (vocab - n) < 32 ? (vocab - n) : 32;
    int idx = 0;
    for (int i = 1; i < nb; ++i) {
      const float a = logits[n + idx], b = logits[n + i];
      if (isnan(a)) break;             /* np.argmax stops at the first NaN */
      if (isnan(b) || b > a) idx = i;
    }
    const uint32_t bits = f32_bits(logits[n + idx]);
    const uint32_t key = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
    if (first || key > best_key) {
      best_key = key;
      best = n + idx;
      first = 0;
    }
  }
  return best;
}

/* ref_qwen3.py:467-490 generate. */
int orc_generate(const orc_model *m, int32_t *ids, int n_prompt, int n_gen,
                 orc_cache *caches, orc_record *rec, float *last_logits,
                 int32_t *generated) {
  const int KW = m->kv_heads * m->head_dim;
  for (int L = 0; L < m->n_layers; ++L) {
    memset(caches[L].k8, 0, (size_t)m->max_seq * KW);
    memset(caches[L].v8, 0, (size_t)m->max_seq * KW);
    memset(caches[L].k_s, 0, (size_t)m->max_seq * m->kv_heads * 4);
    memset(caches[L].v_s, 0, (size_t)m->max_seq * m->kv_heads * 4);
  }
  const int total = n_prompt + n_gen;
  int pos = 0, ngen = 0;
  float *logits = xmalloc((size_t)m->vocab * 4);
  int have = 0;
  while (pos < total) {
    const int rows = pos < n_prompt ? ((m->seq < n_prompt - pos) ? m->seq : n_prompt - pos) : 1;
    const int want = pos + rows >= n_prompt;
    if (orc_forward_chunk(m, ids + pos, caches, pos, rows, want, want ? rec : NULL,
                          logits) != 0) {
      free(logits);
      return -1;
    }
    if (want) have = 1;
    pos += rows;
    if (pos >= n_prompt && pos < total) {
      const int nxt = orc_argmax_logits(logits, m->vocab);
      ids[pos] = nxt;
      if (generated) generated[ngen] = nxt;
      ngen++;
    }
  }
  if (last_logits && have) memcpy(last_logits, logits, (size_t)m->vocab * 4);
  free(logits);
  return ngen;
}
