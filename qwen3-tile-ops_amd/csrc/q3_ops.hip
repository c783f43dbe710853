// C ABI of the operator surface (include/q3ops.h): argument validation and
// dispatch to the kernels.  Mirrors kernels/*.h one function per op.
#include <atomic>
#include <cstring>
#include <mutex>
#include <vector>

#include "q3_kernels.h"
#include "q3ops.h"

namespace {

std::atomic<int> g_silent{0};

inline int elem_size(uint8_t dt) { return (dt == Q3_DT_I8 || dt == Q3_DT_U8) ? 1 : 4; }

// A view with no data: NULL data on a view that has rows.  A 0-row view
// may carry NULL (a caller's empty tensor); the operators then do nothing
// for it, as the reference's row loops do.
inline bool no_data(const q3_view *v) { return !v->data && v->rows != 0; }

// A dense-column view of the given dtype with at least `cols` columns.
int check_view(const q3_view *v, uint8_t dt) {
  if (!v || no_data(v)) return Q3_ERR_ARG;
  if (v->dtype != dt) return Q3_ERR_DTYPE;
  const int es = elem_size(dt);
  if (v->col_bytes != es) return Q3_ERR_VIEW;
  if (v->rows > 1 && (v->row_bytes < static_cast<int64_t>(v->cols) * es || v->row_bytes % es != 0))
    return Q3_ERR_VIEW;
  return Q3_OK;
}

// A per-element vector [n][1] f32 (or a [1][n] row): returns its stride in
// elements via *stride.
int check_vec(const q3_view *v, uint32_t n, int64_t *stride) {
  if (!v || no_data(v)) return Q3_ERR_ARG;
  if (v->dtype != Q3_DT_F32) return Q3_ERR_DTYPE;
  if (v->rows >= n && v->cols >= 1) {
    if (v->row_bytes % 4 != 0 || (n > 1 && v->row_bytes < 4)) return Q3_ERR_VIEW;
    *stride = v->row_bytes / 4;
    return Q3_OK;
  }
  if (v->rows == 1 && v->cols >= n && v->col_bytes == 4) {
    *stride = 1;
    return Q3_OK;
  }
  return Q3_ERR_VIEW;
}

// An f32 scale matrix [rows][cols] whose columns may be strided
// (col_bytes a multiple of 4): at least `rows` x `cols`, and each row long
// enough for its last column.
int check_scales(const q3_view *v, uint32_t rows, uint32_t cols) {
  if (!v || no_data(v)) return Q3_ERR_ARG;
  if (v->dtype != Q3_DT_F32) return Q3_ERR_DTYPE;
  if (v->row_bytes % 4 || v->col_bytes % 4 || v->col_bytes <= 0) return Q3_ERR_VIEW;
  if (v->rows < rows || v->cols < cols) return Q3_ERR_VIEW;
  if (rows > 1 && cols > 0 &&
      v->row_bytes < static_cast<int64_t>(cols - 1) * v->col_bytes + 4)
    return Q3_ERR_VIEW;
  return Q3_OK;
}

inline int64_t ld(const q3_view *v) { return v->row_bytes / elem_size(v->dtype); }

int unsupported() { return g_silent.load() ? Q3_OK : Q3_ERR_UNSUPPORTED; }

int hip_status(hipError_t e) { return e == hipSuccess ? Q3_OK : Q3_ERR_HIP; }

#define Q3_TRY(expr)                 \
  do {                               \
    const int q3_rc_ = (expr);       \
    if (q3_rc_ != Q3_OK) return q3_rc_; \
  } while (0)

// Validates the common GEMM operands; fills the shape fields of g.  *skip:
// the caller returns the status without launching (an unsupported shape, or
// no rows: group_gemm.h:91's row loop then does nothing).
int gemm_common(const q3_view *a, const q3_view *a_scale, const q3_view *b,
                const q3_view *b_scale, uint32_t group_k, q3::GemmArgs &g,
                bool *skip) {
  *skip = false;
  Q3_TRY(check_view(a, Q3_DT_I8));
  Q3_TRY(check_view(b, Q3_DT_I8));
  if (!a_scale || no_data(a_scale) || !b_scale || no_data(b_scale)) return Q3_ERR_ARG;
  if (a_scale->dtype != Q3_DT_F32 || b_scale->dtype != Q3_DT_F32) return Q3_ERR_DTYPE;
  const uint32_t K = a->cols, N = b->rows, M = a->rows;
  if (b->cols != K) return Q3_ERR_VIEW;
  // group_gemm.h:47-49 rejects these; MFMA also needs 64-wide K steps.
  if (group_k == 0 || K % group_k != 0 || N % 128 != 0 || group_k % 64 != 0) {
    *skip = true;
    return unsupported();
  }
  if ((a->row_bytes % 16) || (b->row_bytes % 16) ||
      (reinterpret_cast<uintptr_t>(a->data) % 16) || (reinterpret_cast<uintptr_t>(b->data) % 16))
    return Q3_ERR_VIEW;
  if (a_scale->col_bytes != 4 || a_scale->row_bytes % 4 != 0) return Q3_ERR_VIEW;
  if (a_scale->rows < M || a_scale->cols < K / group_k) return Q3_ERR_VIEW;
  // b_scale [N][1] (one scale per weight row, the reference) or
  // [N][K / group_k] (one per weight row and K-group)
  int64_t bss = 1, bs_ld = 0;
  const uint32_t ng = K / group_k;
  if (ng > 1 && b_scale->cols == ng && b_scale->rows >= N) {
    Q3_TRY(check_scales(b_scale, N, ng));
    if (b_scale->col_bytes != 4) return Q3_ERR_VIEW;
    bs_ld = b_scale->row_bytes / 4;
  } else {
    Q3_TRY(check_vec(b_scale, N, &bss));
  }
  std::memset(&g, 0, sizeof(g));
  g.M = static_cast<int>(M);
  g.N = static_cast<int>(N);
  g.K = static_cast<int>(K);
  g.group = static_cast<int>(group_k);
  g.a = static_cast<const int8_t *>(a->data);
  g.lda = a->row_bytes;
  g.as = static_cast<const float *>(a_scale->data);
  g.ldas = a_scale->row_bytes / 4;
  g.b = static_cast<const int8_t *>(b->data);
  g.ldb = b->row_bytes;
  g.bs = static_cast<const float *>(b_scale->data);
  g.bs_stride = bss;
  g.bs_ld = bs_ld;
  *skip = M == 0;
  return Q3_OK;
}

// Decode-shaped STORE/ADD/ARGMAX GEMMs (up to 64 rows; more than 16 only
// below 65536 columns) go to the whole-chip GEMV kernel.
q3::GemvArgs to_gemv(const q3::GemmArgs &g);

bool use_gemv(const q3::GemmArgs &g) {
  const bool shape = g.M <= 16 ? q3::gemv_supported(g.M, g.K, g.group)
                               : q3::gemv_rows_supported(g.M, g.K, g.group, g.N);
  return shape && g.ldb == g.K && g.bs_stride == 1 &&
         (g.epi == q3::EPI_STORE || g.epi == q3::EPI_ADD || g.epi == q3::EPI_ARGMAX) &&
         (!g.bs_ld || q3::gemv_group_bscale_supported(to_gemv(g)));
}

q3::GemvArgs to_gemv(const q3::GemmArgs &g) {
  q3::GemvArgs v;
  std::memset(&v, 0, sizeof(v));
  v.M = g.M;
  v.K = g.K;
  v.group = g.group;
  v.a = g.a;
  v.lda = g.lda;
  v.as = g.as;
  v.ldas = g.ldas;
  v.pro = q3::PRO_NONE;
  v.nseg = 1;
  v.seg[0].n0 = 0;
  v.seg[0].n1 = g.N;
  v.seg[0].epi = g.epi;
  v.seg[0].b = g.b;
  v.seg[0].bs = g.bs;
  v.seg[0].out = g.out;
  v.seg[0].ldo = g.ldo;
  v.keys = g.keys;
  v.keys_ld = g.keys_ld;
  v.bs_ld = g.bs_ld;
  return v;
}

hipError_t launch_gemm_or_gemv(const q3::GemmArgs &g, hipStream_t s) {
  if (!use_gemv(g)) return q3::launch_gemm(g, s);
  return q3::launch_gemv(to_gemv(g), s);
}

// Per-workgroup argmax slots needed by launch_gemm_or_gemv for g.
int argmax_slots(const q3::GemmArgs &g) {
  if (use_gemv(g)) return q3::gemv_argmax_slots(to_gemv(g));
  return g.N / 128;
}

int nrq_common(const q3_view *nw, const q3_view *cos, const q3_view *sin,
               uint32_t rows, float inv_hd, q3::GemmArgs &g) {
  int64_t nws = 1;
  Q3_TRY(check_vec(nw, 128, &nws));
  Q3_TRY(check_view(cos, Q3_DT_F32));
  Q3_TRY(check_view(sin, Q3_DT_F32));
  if (cos->cols < 64 || sin->cols < 64 || cos->rows < rows || sin->rows < rows) return Q3_ERR_VIEW;
  if (cos->row_bytes != sin->row_bytes) return Q3_ERR_VIEW;
  g.nw = static_cast<const float *>(nw->data);
  g.nw_stride = nws;
  g.cos_t = static_cast<const float *>(cos->data);
  g.sin_t = static_cast<const float *>(sin->data);
  g.ld_cs = cos->row_bytes / 4;
  g.inv_hd = inv_hd;
  return Q3_OK;
}

int check_paged(const q3_paged_kv *kv) {
  if (!kv || !kv->k || !kv->v || !kv->ks || !kv->vs || !kv->table) return Q3_ERR_ARG;
  if (kv->page_tokens == 0 || kv->page_tokens % 32 != 0) return Q3_ERR_UNSUPPORTED;
  if (kv->page_bytes < kv->page_tokens * kv->row_bytes) return Q3_ERR_VIEW;
  if (kv->scale_page_bytes < kv->page_tokens * kv->scale_row_bytes) return Q3_ERR_VIEW;
  if (kv->row_bytes % 16 || kv->scale_row_bytes % 4) return Q3_ERR_VIEW;
  return Q3_OK;
}

// The per-(device, stream) workspace of the ops that need device memory
// between two launches (the argmax keys, the SwiGLU rows of a decode-shaped
// gate/up): allocated by the first such call on a stream, kept until the
// process ends.  Defined with the argmax entry points below.
constexpr int64_t kWorkspaceBytes = int64_t(8) << 19;  // 4 MiB
unsigned long long *stream_keys(hipStream_t s);
// The stream's workspace if it has one already, or if it may be allocated
// now (the stream is not capturing a graph); else null.
unsigned long long *stream_keys_if_free(hipStream_t s);

}  // namespace

extern "C" {

int q3_set_silent_unsupported(int on) { return g_silent.exchange(on ? 1 : 0); }

const char *q3_status_str(int s) {
  switch (s) {
    case Q3_OK: return "ok";
    case Q3_ERR_ARG: return "invalid argument";
    case Q3_ERR_DTYPE: return "dtype mismatch";
    case Q3_ERR_VIEW: return "inconsistent view shape or stride";
    case Q3_ERR_UNSUPPORTED: return "unsupported shape";
    case Q3_ERR_HIP: return "HIP runtime error";
    case Q3_ERR_MODE: return "unsupported CTRL mode";
    case Q3_ERR_RANGE: return "position, page or id out of range";
    default: return "unknown status";
  }
}

int q3_embedding_rmsnorm_rows(const q3_view *table, const q3_view *scale,
                              const q3_view *ids, const q3_view *tmp,
                              const q3_view *w, const q3_view *out, float inv,
                              void *stream) {
  Q3_TRY(check_view(table, Q3_DT_I8));
  Q3_TRY(check_view(tmp, Q3_DT_F32));
  Q3_TRY(check_view(out, Q3_DT_F32));
  if (!ids || no_data(ids)) return Q3_ERR_ARG;
  if (ids->dtype != Q3_DT_I32 && ids->dtype != Q3_DT_U32) return Q3_ERR_DTYPE;
  const uint32_t rows = ids->rows, cols = table->cols;
  if (tmp->cols < cols || out->cols < cols || tmp->rows < rows || out->rows < rows) return Q3_ERR_VIEW;
  int64_t tss = 1, ws = 1;
  Q3_TRY(check_vec(scale, table->rows, &tss));
  Q3_TRY(check_vec(w, cols, &ws));
  q3::RowArgs r{};
  r.mode = 2;
  r.rows = static_cast<int>(rows);
  r.cols = static_cast<int>(cols);
  r.table = static_cast<const int8_t *>(table->data);
  r.ldt = table->row_bytes;
  r.table_rows = table->rows;
  r.tscale = static_cast<const float *>(scale->data);
  r.tss = tss;
  r.ids = static_cast<const int32_t *>(ids->data);
  r.ids_stride = ids->row_bytes / 4 > 0 ? ids->row_bytes / 4 : 1;
  r.x_out = static_cast<float *>(tmp->data);
  r.ldxo = ld(tmp);
  r.w = static_cast<const float *>(w->data);
  r.w_stride = ws;
  r.inv = inv;
  r.h = static_cast<float *>(out->data);
  r.ldh = ld(out);
  return hip_status(q3::launch_rows(r, static_cast<hipStream_t>(stream)));
}

int q3_rmsnorm_rows(const q3_view *x, const q3_view *w, const q3_view *out,
                    float inv, void *stream) {
  Q3_TRY(check_view(x, Q3_DT_F32));
  Q3_TRY(check_view(out, Q3_DT_F32));
  if (out->rows < x->rows || out->cols < x->cols) return Q3_ERR_VIEW;
  int64_t ws = 1;
  Q3_TRY(check_vec(w, x->cols, &ws));
  q3::RowArgs r{};
  r.mode = 1;
  r.rows = static_cast<int>(x->rows);
  r.cols = static_cast<int>(x->cols);
  r.x = static_cast<const float *>(x->data);
  r.ldx = ld(x);
  r.w = static_cast<const float *>(w->data);
  r.w_stride = ws;
  r.inv = inv;
  r.h = static_cast<float *>(out->data);
  r.ldh = ld(out);
  return hip_status(q3::launch_rows(r, static_cast<hipStream_t>(stream)));
}

int q3_quant_rows_heads(const q3_view *x, const q3_view *qi8,
                        const q3_view *scale, uint32_t group_cols,
                        void *stream) {
  Q3_TRY(check_view(x, Q3_DT_F32));
  Q3_TRY(check_view(qi8, Q3_DT_I8));
  if (!scale || no_data(scale)) return Q3_ERR_ARG;
  if (scale->dtype != Q3_DT_F32) return Q3_ERR_DTYPE;
  if (group_cols == 0) return Q3_ERR_ARG;
  if (qi8->rows < x->rows || qi8->cols < x->cols) return Q3_ERR_VIEW;
  if (scale->col_bytes != 4 || scale->row_bytes % 4 != 0) return Q3_ERR_VIEW;
  if (scale->rows < x->rows || scale->cols < (x->cols + group_cols - 1) / group_cols) return Q3_ERR_VIEW;
  q3::RowArgs r{};
  r.mode = 0;
  r.rows = static_cast<int>(x->rows);
  r.cols = static_cast<int>(x->cols);
  r.x = static_cast<const float *>(x->data);
  r.ldx = ld(x);
  r.h8 = static_cast<int8_t *>(qi8->data);
  r.ldh8 = qi8->row_bytes;
  r.hs = static_cast<float *>(scale->data);
  r.ldhs = scale->row_bytes / 4;
  r.group = static_cast<int>(group_cols);
  return hip_status(q3::launch_rows(r, static_cast<hipStream_t>(stream)));
}

int q3_gemm_nt_group_store(const q3_view *a, const q3_view *a_scale,
                           const q3_view *b, const q3_view *b_scale,
                           const q3_view *out, uint32_t group_k,
                           const q3_view *add, const q3_view *q8,
                           const q3_view *qs, const q3_view *nw,
                           const q3_view *cos, const q3_view *sin,
                           float inv_hd, void *stream) {
  q3::GemmArgs g;
  bool skip = false;
  Q3_TRY(gemm_common(a, a_scale, b, b_scale, group_k, g, &skip));
  if (skip) return Q3_OK;
  // per-group B scales: the plain and residual stores
  if (g.bs_ld && (q8 || nw)) return unsupported();
  if (q8) {  // group_gemm.h:168-193 (nw selects norm+RoPE)
    Q3_TRY(check_view(q8, Q3_DT_I8));
    if (q8->rows < a->rows || q8->cols < b->rows) return Q3_ERR_VIEW;
    Q3_TRY(check_scales(qs, a->rows, b->rows / 128));
    g.qd.q8 = static_cast<int8_t *>(q8->data);
    g.qd.ldq8 = q8->row_bytes;
    g.qd.qs = static_cast<float *>(qs->data);
    g.qd.ldqs = qs->row_bytes / 4;
    g.qd.qs_col = qs->col_bytes / 4;
    if (nw) {
      g.epi = q3::EPI_NRQ;
      Q3_TRY(nrq_common(nw, cos, sin, a->rows, inv_hd, g));
    } else {
      g.epi = q3::EPI_HEADQ;
    }
  } else if (nw) {
    return Q3_ERR_ARG;  // the norm epilogue needs q8/qs
  } else if (add) {
    Q3_TRY(check_view(add, Q3_DT_F32));
    if (add->rows < a->rows || add->cols < b->rows) return Q3_ERR_VIEW;
    g.epi = q3::EPI_ADD;
    g.out = static_cast<float *>(add->data);
    g.ldo = ld(add);
  } else {
    Q3_TRY(check_view(out, Q3_DT_F32));
    if (out->rows < a->rows || out->cols < b->rows) return Q3_ERR_VIEW;
    g.epi = q3::EPI_STORE;
    g.out = static_cast<float *>(out->data);
    g.ldo = ld(out);
  }
  return hip_status(launch_gemm_or_gemv(g, static_cast<hipStream_t>(stream)));
}

int q3_gemm_nt_group_kv_paged(const q3_view *a, const q3_view *a_scale,
                              const q3_view *b, const q3_view *b_scale,
                              uint32_t group_k, const q3_paged_kv *kv,
                              uint32_t pos0, int is_v, const q3_view *nw,
                              const q3_view *cos, const q3_view *sin,
                              float inv_hd, void *stream) {
  q3::GemmArgs g;
  bool skip = false;
  Q3_TRY(gemm_common(a, a_scale, b, b_scale, group_k, g, &skip));
  if (skip) return Q3_OK;
  if (g.bs_ld) return unsupported();
  Q3_TRY(check_paged(kv));
  if (kv->row_bytes < b->rows || kv->scale_row_bytes < b->rows / 128 * 4) return Q3_ERR_VIEW;
  g.qd.q8 = static_cast<int8_t *>(is_v ? kv->v : kv->k);
  g.qd.qs = static_cast<float *>(is_v ? kv->vs : kv->ks);
  g.qd.table = kv->table;
  g.qd.page_tokens = kv->page_tokens;
  g.qd.page_bytes = kv->page_bytes;
  g.qd.row_bytes = kv->row_bytes;
  g.qd.scale_page_bytes = kv->scale_page_bytes;
  g.qd.scale_row_bytes = kv->scale_row_bytes;
  g.qd.pos0 = pos0;
  if (nw) {
    g.epi = q3::EPI_NRQ;
    Q3_TRY(nrq_common(nw, cos, sin, a->rows, inv_hd, g));
  } else {
    g.epi = q3::EPI_HEADQ;
  }
  return hip_status(q3::launch_gemm(g, static_cast<hipStream_t>(stream)));
}

int q3_norm_rope_quant_heads(const q3_view *x, const q3_view *w,
                             const q3_view *cos, const q3_view *sin,
                             const q3_view *q8, const q3_view *scale,
                             int heads, float inv_hd, int do_rope,
                             void *stream) {
  Q3_TRY(check_view(x, Q3_DT_F32));
  Q3_TRY(check_view(q8, Q3_DT_I8));
  if (heads <= 0 || x->cols != static_cast<uint32_t>(heads) * 128) return unsupported();
  if (q8->rows < x->rows || q8->cols < x->cols) return Q3_ERR_VIEW;
  Q3_TRY(check_scales(scale, x->rows, static_cast<uint32_t>(heads)));
  q3::NrqArgs r{};
  int64_t nws = 1;
  Q3_TRY(check_vec(w, 128, &nws));
  r.do_rope = do_rope;
  if (do_rope) {
    Q3_TRY(check_view(cos, Q3_DT_F32));
    Q3_TRY(check_view(sin, Q3_DT_F32));
    if (cos->cols < 64 || sin->cols < 64 || cos->rows < x->rows || sin->rows < x->rows ||
        cos->row_bytes != sin->row_bytes)
      return Q3_ERR_VIEW;
    r.cos_t = static_cast<const float *>(cos->data);
    r.sin_t = static_cast<const float *>(sin->data);
    r.ld_cs = cos->row_bytes / 4;
  } else {
    // rows are still addressed, but never read
    r.cos_t = r.sin_t = static_cast<const float *>(x->data);
    r.ld_cs = 0;
  }
  r.rows = static_cast<int>(x->rows);
  r.heads = heads;
  r.x = static_cast<const float *>(x->data);
  r.ldx = ld(x);
  r.nw = static_cast<const float *>(w->data);
  r.nw_stride = nws;
  r.inv_hd = inv_hd;
  r.q8 = static_cast<int8_t *>(q8->data);
  r.ldq8 = q8->row_bytes;
  r.qs = static_cast<float *>(scale->data);
  r.ldqs = scale->row_bytes / 4;
  r.qs_col = scale->col_bytes / 4;
  return hip_status(q3::launch_nrq_rows(r, static_cast<hipStream_t>(stream)));
}

int q3_attention_heads_gqa_tokscale_paged(const q3_view *q8,
                                          const q3_view *q_scale,
                                          const q3_paged_kv *kv,
                                          uint32_t kv_len, const q3_view *o8,
                                          const q3_view *os, int heads,
                                          int kv_heads, int head_dim,
                                          int causal, float qk_scale,
                                          void *stream) {
  Q3_TRY(check_view(q8, Q3_DT_I8));
  Q3_TRY(check_view(o8, Q3_DT_I8));
  Q3_TRY(check_paged(kv));
  if (!q_scale || no_data(q_scale) || !os || no_data(os)) return Q3_ERR_ARG;
  if (q_scale->dtype != Q3_DT_F32 || os->dtype != Q3_DT_F32) return Q3_ERR_DTYPE;
  if (head_dim != 128) return unsupported();
  if (heads <= 0 || kv_heads <= 0 || heads % kv_heads) return Q3_ERR_ARG;
  const uint32_t rows = q8->rows;
  if (q8->cols < static_cast<uint32_t>(heads) * 128 || o8->cols < q8->cols || o8->rows < rows)
    return Q3_ERR_VIEW;
  Q3_TRY(check_scales(q_scale, rows, static_cast<uint32_t>(heads)));
  Q3_TRY(check_scales(os, rows, static_cast<uint32_t>(heads)));
  if (causal && kv_len < rows) return Q3_ERR_RANGE;
  if (kv->row_bytes < static_cast<uint32_t>(kv_heads) * 128 ||
      kv->scale_row_bytes < static_cast<uint32_t>(kv_heads) * 4)
    return Q3_ERR_VIEW;
  if ((q8->row_bytes % 16) || (reinterpret_cast<uintptr_t>(q8->data) % 16)) return Q3_ERR_VIEW;
  q3::AttnArgs t{};
  t.rows = static_cast<int>(rows);
  t.heads = heads;
  t.kv_heads = kv_heads;
  t.kv_len = kv_len;
  t.causal = causal;
  t.qk_scale = qk_scale;
  t.q8 = static_cast<const int8_t *>(q8->data);
  t.ldq = q8->row_bytes;
  t.qs = static_cast<const float *>(q_scale->data);
  t.ldqs = q_scale->row_bytes / 4;
  t.qs_col = q_scale->col_bytes / 4;
  t.k = static_cast<const int8_t *>(kv->k);
  t.v = static_cast<const int8_t *>(kv->v);
  t.ks = static_cast<const float *>(kv->ks);
  t.vs = static_cast<const float *>(kv->vs);
  t.table = kv->table;
  t.page_tokens = kv->page_tokens;
  t.page_bytes = kv->page_bytes;
  t.row_bytes = kv->row_bytes;
  t.scale_page_bytes = kv->scale_page_bytes;
  t.scale_row_bytes = kv->scale_row_bytes;
  t.o8 = static_cast<int8_t *>(o8->data);
  t.ldo = o8->row_bytes;
  t.os = static_cast<float *>(os->data);
  t.ldos = os->row_bytes / 4;
  t.os_col = os->col_bytes / 4;
  if (q3::attn_decode_supported(t))
    return hip_status(q3::launch_attn_decode(t, static_cast<hipStream_t>(stream)));
  return hip_status(q3::launch_attention(t, static_cast<hipStream_t>(stream)));
}

int q3_gemm_gate_up_swiglu_quant(const q3_view *a, const q3_view *a_scale,
                                 const q3_view *wg, const q3_view *wgs,
                                 const q3_view *wu, const q3_view *wus,
                                 const q3_view *s8, const q3_view *ss,
                                 uint32_t group_k, void *stream) {
  q3::GemmArgs g;
  bool skip = false;
  Q3_TRY(gemm_common(a, a_scale, wg, wgs, group_k, g, &skip));
  if (skip) return Q3_OK;
  if (g.bs_ld) return unsupported();
  Q3_TRY(check_view(wu, Q3_DT_I8));
  if (wu->rows != wg->rows || wu->cols != wg->cols || wu->row_bytes != wg->row_bytes) return Q3_ERR_VIEW;
  if (reinterpret_cast<uintptr_t>(wu->data) % 16) return Q3_ERR_VIEW;
  int64_t wus_stride = 1;
  Q3_TRY(check_vec(wus, wu->rows, &wus_stride));
  if (wus_stride != g.bs_stride) return Q3_ERR_VIEW;
  Q3_TRY(check_view(s8, Q3_DT_I8));
  const uint32_t N = wg->rows;
  if (N % 256 != 0) return unsupported();  // swiglu_quant.h:197 (256-column groups)
  if (s8->rows < a->rows || s8->cols < N) return Q3_ERR_VIEW;
  Q3_TRY(check_scales(ss, a->rows, N / 256));
  q3::GateUpArgs u{};
  u.M = g.M;
  u.N = g.N;
  u.K = g.K;
  u.group = g.group;
  u.a = g.a;
  u.lda = g.lda;
  u.as = g.as;
  u.ldas = g.ldas;
  u.wg = g.b;
  u.wu = static_cast<const int8_t *>(wu->data);
  u.ldw = g.ldb;
  u.wgs = g.bs;
  u.wus = static_cast<const float *>(wus->data);
  u.ws_stride = g.bs_stride;
  u.s8 = static_cast<int8_t *>(s8->data);
  u.lds8 = s8->row_bytes;
  u.ss = static_cast<float *>(ss->data);
  u.ldss = ss->row_bytes / 4;
  u.ss_col = ss->col_bytes / 4;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  // decode shapes: the two-matrix GEMV (SwiGLU rows in f32, on every CU)
  // into the stream's workspace, then the per-256-column quantisation of
  // those rows (quant.h:89-138, the same arithmetic as swiglu_quant.h:197-231)
  if (u.ldw == u.K && u.ws_stride == 1 && u.ss_col == 1 && q3::gemv_rows_supported(u.M, u.K, u.group, u.N) &&
      static_cast<int64_t>(u.M) * u.N * 4 <= kWorkspaceBytes) {
    // (a stream capturing a graph without a workspace yet takes the fused
    // kernel below instead: no allocation inside a capture)
    float *tmp = reinterpret_cast<float *>(stream_keys_if_free(s));
    if (!tmp) return hip_status(q3::launch_gate_up(u, s));
    q3::GemvArgs v;
    std::memset(&v, 0, sizeof(v));
    v.M = u.M;
    v.K = u.K;
    v.group = u.group;
    v.a = u.a;
    v.lda = u.lda;
    v.as = u.as;
    v.ldas = u.ldas;
    v.pro = q3::PRO_NONE;
    v.nseg = 1;
    v.seg[0].n0 = 0;
    v.seg[0].n1 = u.N;
    v.seg[0].epi = q3::EPI_SWIGLU;
    v.seg[0].b = u.wg;
    v.seg[0].b2 = u.wu;
    v.seg[0].bs = u.wgs;
    v.seg[0].bs2 = u.wus;
    v.seg[0].out = tmp;
    v.seg[0].ldo = u.N;
    Q3_TRY(hip_status(q3::launch_gemv(v, s)));
    q3::RowArgs r{};
    r.mode = 0;
    r.rows = u.M;
    r.cols = u.N;
    r.x = tmp;
    r.ldx = u.N;
    r.h8 = u.s8;
    r.ldh8 = u.lds8;
    r.hs = u.ss;
    r.ldhs = u.ldss;
    r.group = 256;
    return hip_status(q3::launch_rows(r, s));
  }
  return hip_status(q3::launch_gate_up(u, s));
}

}  // extern "C"

// ---- lm_head + argmax: key workspaces --------------------------------------
// The argmax GEMM writes one 64-bit key per (row, column block) and
// argmax_finish_kernel merges them, so a call needs M * slots keys of device
// memory between its two launches.  Every key is written before it is read:
// nothing has to start at zero.
namespace {
constexpr int kMaxArgmaxRows = 256;
// 4 MiB of keys, e.g. 256 rows x 1187 lm_head blocks of 128 columns.
constexpr int64_t kArgmaxSlots = kWorkspaceBytes / 8;
constexpr int kMaxDevices = 64;

// q3_gemm_nt_group_argmax: one workspace per (device, stream), allocated by
// the first call on that stream and kept until the process ends, so calls on
// different streams never share keys.
struct StreamKeys {
  int dev;
  hipStream_t stream;
  unsigned long long *keys;
};
std::mutex g_stream_keys_mu;
std::vector<StreamKeys> g_stream_keys;

unsigned long long *stream_keys_impl(hipStream_t s, bool only_if_free) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lock(g_stream_keys_mu);
  for (const StreamKeys &e : g_stream_keys)
    if (e.dev == dev && e.stream == s) return e.keys;
  if (only_if_free) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return nullptr;
  }
  void *p = nullptr;
  if (hipMalloc(&p, sizeof(unsigned long long) * kArgmaxSlots) != hipSuccess) return nullptr;
  g_stream_keys.push_back({dev, s, static_cast<unsigned long long *>(p)});
  return static_cast<unsigned long long *>(p);
}

unsigned long long *stream_keys(hipStream_t s) { return stream_keys_impl(s, false); }
unsigned long long *stream_keys_if_free(hipStream_t s) { return stream_keys_impl(s, true); }

// q3_gemm_nt_group_argmax_noalloc: a fixed key array in the library's own
// device image (each device holds its own copy until the process ends).  In
// host code `scratch` names a host-side stand-in, never device memory: its
// device address comes from hipGetSymbolAddress, taken once per device with
// that device current, and only that address is handed to kernels.
constexpr int64_t kScratchSlots = int64_t(1) << 19;  // 4 MiB
static __device__ __align__(256) unsigned long long scratch[kScratchSlots];
std::mutex g_scratch_mu;
std::atomic<unsigned long long *> g_scratch_ptr[kMaxDevices];

unsigned long long *device_scratch(int *status) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    *status = Q3_ERR_HIP;
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    *status = Q3_ERR_UNSUPPORTED;
    return nullptr;
  }
  unsigned long long *p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p) return p;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
  if (!p) {
    void *addr = nullptr;
    if (hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)) != hipSuccess || !addr) {
      *status = Q3_ERR_HIP;
      return nullptr;
    }
    p = static_cast<unsigned long long *>(addr);
    g_scratch_ptr[dev].store(p, std::memory_order_release);
  }
  return p;
}

// Validation shared by both argmax entry points; fills g (EPI_ARGMAX) and
// the best/bidx strides.
int argmax_common(const q3_view *a, const q3_view *a_scale, const q3_view *b,
                  const q3_view *b_scale, const q3_view *best, const q3_view *bidx,
                  uint32_t group_k, q3::GemmArgs &g, int64_t *bst, int64_t *ist, bool *skip) {
  Q3_TRY(gemm_common(a, a_scale, b, b_scale, group_k, g, skip));
  if (*skip) return Q3_OK;
  if (g.bs_ld) {
    *skip = true;
    return unsupported();
  }
  if (!best || no_data(best) || !bidx || no_data(bidx)) return Q3_ERR_ARG;
  if (best->dtype != Q3_DT_F32) return Q3_ERR_DTYPE;
  if (bidx->dtype != Q3_DT_I32 && bidx->dtype != Q3_DT_U32) return Q3_ERR_DTYPE;
  Q3_TRY(check_vec(best, a->rows, bst));
  {
    // bidx has the same shape rules as best but an integer dtype
    q3_view tmp = *bidx;
    tmp.dtype = Q3_DT_F32;
    Q3_TRY(check_vec(&tmp, a->rows, ist));
  }
  if (a->rows > static_cast<uint32_t>(kMaxArgmaxRows)) {
    *skip = true;
    return unsupported();
  }
  g.epi = q3::EPI_ARGMAX;
  const int nslots = argmax_slots(g);
  if (static_cast<int64_t>(g.M) * nslots > kArgmaxSlots) {
    *skip = true;
    return unsupported();
  }
  g.keys_ld = nslots;
  return Q3_OK;
}

int argmax_launch(q3::GemmArgs &g, unsigned long long *keys, const q3_view *best, int64_t bst,
                  const q3_view *bidx, int64_t ist, hipStream_t s) {
  g.keys = keys;
  Q3_TRY(hip_status(launch_gemm_or_gemv(g, s)));
  const int nslots = static_cast<int>(g.keys_ld);
  return hip_status(q3::launch_argmax_finish(keys, nslots, nslots, g.M,
                                             static_cast<float *>(best->data), bst,
                                             static_cast<int32_t *>(bidx->data), ist, 0, nullptr,
                                             nullptr, 0, s));
}
}  // namespace

extern "C" int q3_gemm_nt_group_argmax(const q3_view *a, const q3_view *a_scale,
                                       const q3_view *b, const q3_view *b_scale,
                                       const q3_view *best, const q3_view *bidx,
                                       uint32_t group_k, void *stream) {
  q3::GemmArgs g;
  int64_t bst = 1, ist = 1;
  bool skip = false;
  Q3_TRY(argmax_common(a, a_scale, b, b_scale, best, bidx, group_k, g, &bst, &ist, &skip));
  if (skip) return Q3_OK;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  unsigned long long *keys = stream_keys(s);
  if (!keys) return Q3_ERR_HIP;
  return argmax_launch(g, keys, best, bst, bidx, ist, s);
}

extern "C" int q3_gemm_nt_group_argmax_noalloc(const q3_view *a, const q3_view *a_scale,
                                               const q3_view *b, const q3_view *b_scale,
                                               const q3_view *best, const q3_view *bidx,
                                               uint32_t group_k, void *stream) {
  q3::GemmArgs g;
  int64_t bst = 1, ist = 1;
  bool skip = false;
  Q3_TRY(argmax_common(a, a_scale, b, b_scale, best, bidx, group_k, g, &bst, &ist, &skip));
  if (skip) return Q3_OK;
  if (g.keys_ld * static_cast<int64_t>(g.M) > kScratchSlots) return unsupported();
  int status = Q3_OK;
  unsigned long long *keys = device_scratch(&status);
  if (!keys) return status;
  return argmax_launch(g, keys, best, bst, bidx, ist, static_cast<hipStream_t>(stream));
}

extern "C" int q3_argmax_logits(const q3_view *logits, int32_t *out_id, void *stream) {
  Q3_TRY(check_view(logits, Q3_DT_F32));
  if (!out_id) return Q3_ERR_ARG;
  if (logits->cols == 0) return Q3_ERR_VIEW;
  return hip_status(q3::launch_argmax_logits(static_cast<const float *>(logits->data),
                                             static_cast<int>(logits->cols), out_id, nullptr, 0,
                                             static_cast<hipStream_t>(stream)));
}
