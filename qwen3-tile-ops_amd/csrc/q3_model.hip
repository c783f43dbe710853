// Model orchestration over a device-resident PQWF blob.
//
//   src/main_big.cpp:55-136   make_model_views / make_layer_views
//   src/main_big.cpp:145-296  forward_chunk
//   src/main_big.cpp:332-369  main() greedy loop
//   tools/ref_qwen3.py:366-490 (the same semantics in numpy)
//
// Every buffer is an offset into the one device blob (tools/pqwf.py layout),
// so the device image after a run can be diffed stage by stage like the
// reference's blob dump.  The KV pool of each layer is paged with 32-token
// pages through a logical->physical page table (reversed by default, as in
// main_big.cpp:168-171); K/V rows are written by the projection GEMMs'
// epilogues straight into their page slots, one row at a time, so a chunk
// may start anywhere and span pages.  All work is enqueued on the model's
// stream; the generated ids are written on the device (no host round trip
// per token).
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <vector>

#include "q3_kernels.h"
#include "q3ops.h"

struct q3_model {
  uint8_t *blob;
  q3_layout lay;
  hipStream_t stream;
  uint16_t *ptab;              // device, max_seq / 32 entries
  std::vector<uint16_t> htab;  // host copy of the page table
  uint32_t n_pages;
  unsigned long long *keys;    // device argmax key (1 row)
  // argmax workspace: one key per lm_head column block (allocated at open)
  unsigned long long *keys_ws;
  int64_t keys_ld;
  // batched decode of independent sequences (q3_decode_batch): per-row
  // positions and page tables (device copies) and argmax key slots
  // bpos and btab share one device allocation (bstate): positions padded
  // to 256 bytes, then the tables, so one copy moves both
  uint8_t *bstate = nullptr;
  int32_t *bpos = nullptr;         // [seq]
  uint16_t *btab = nullptr;        // [seq][n_pages]
  size_t btab_off = 0;
  // pinned host staging of bstate, two slots: the host fills one while the
  // copy out of the other may still be pending on the stream
  uint8_t *bstage[2] = {nullptr, nullptr};
  hipEvent_t bstage_ev[2] = {nullptr, nullptr};
  bool bstage_used[2] = {false, false};
  uint32_t bstage_next = 0;
  unsigned long long *bkeys = nullptr;  // [seq][bkeys_ld]
  int64_t bkeys_ld = 0;
  float *bbest = nullptr;          // [seq] per-row argmax value
  // decode (b = 1): the O projection's per-head partials [2][heads][hidden],
  // written by the attention kernel, summed by the gate/up and down GEMVs;
  // layer L uses half L & 1 (its down projection can run in layer L + 1's
  // launch, whose attention writes the other half)
  float *opart = nullptr;
  // decode (b = 1): the Q|K|V projection in the attention's launch
  // (Q3_DECODE_FUSE_QKV, default 1), its exchange words and give-up flag
  // (AttnArgs::xin / xerr)
  bool qkvfuse = true;
  unsigned long long *xin = nullptr;
  uint32_t *xerr = nullptr;
  // decode (b = 1): layer L's down projection in layer L + 1's Q|K|V +
  // attention launch (Q3_DECODE_MERGE_DOWN, default 1: 0.625 against 0.632
  // ms/token), its new residual row as exchange words (AttnArgs::xw,
  // kXwWords), cleared by the gate/up launch of every b = 1 layer while
  // enabled.  Its GEMV workgroups wait for each other, so they need the
  // device's CUs (down_qkv_attn_supported checks the count)
  bool merge = true;
  uint32_t *xw = nullptr;
  // event timing of decode kernel classes (q3_model_set_kernel_timing)
  uint32_t kt_mask = 0;
  std::vector<hipEvent_t> kt_ev[Q3_KT_COUNT];  // start, end pairs
  uint32_t kt_used[Q3_KT_COUNT] = {};          // pairs recorded
  double kt_ms[Q3_KT_COUNT] = {};              // folded totals
  uint32_t kt_n[Q3_KT_COUNT] = {};
  // decode: workgroups that prefetch the next kernels' weights during the
  // attention kernel (Q3_DECODE_PREFETCH_WGS, default 176; 0 disables)
  int pf_wgs;
  // decode: O projection folded into the attention kernel
  // (Q3_DECODE_FUSE_OPROJ, default 1; 0 runs it as its own GEMV)
  bool ofuse = true;
  // q3_generate: the decode steps after the prefill chunks, captured as one
  // HIP graph on the model's stream and replayed while the generation they
  // were captured for (n_prompt, n_gen, mode, page table) is asked again
  // (Q3_DECODE_GRAPH, default 1; 0 launches them one by one)
  bool dgraph_on = true;
  hipGraphExec_t dgraph = nullptr;
  // prefill chunks of more than 64 rows: every layer's weights repacked at
  // open (q3::launch_pack_b) so that the stream GEMM reads each MFMA operand
  // fragment as one contiguous 1 KiB (Q3_PACKED_WEIGHTS=0: no copy)
  int8_t *packed = nullptr;
  int64_t pk_layer = 0;   // bytes per layer
  int64_t pk_off[7] = {}; // q, k, v, o, gate, up, down within a layer
  int32_t dg_key[3] = {-1, -1, -1};
  uint64_t tab_version = 0, dg_tab_version = ~0ull;
};

namespace q3 {
thread_local const LaunchEvents *g_launch_events = nullptr;
}  // namespace q3

namespace {

constexpr uint32_t kPageTokens = 32;
constexpr int kMaxGemvRows = 16;

int hip_status(hipError_t e) { return e == hipSuccess ? Q3_OK : Q3_ERR_HIP; }

#define Q3_TRY(expr)             \
  do {                           \
    const int rc_ = (expr);      \
    if (rc_ != Q3_OK) return rc_; \
  } while (0)

#define Q3_HIP(expr)                                      \
  do {                                                    \
    const hipError_t q3_e_ = (expr);                      \
    if (q3_e_ != hipSuccess) return Q3_ERR_HIP;           \
  } while (0)

template <class T>
T *at(const q3_model *m, int64_t off) {
  return reinterpret_cast<T *>(m->blob + off);
}

// Per-layer views (main_big.cpp:100-136).
struct LayerPtrs {
  const int8_t *wq, *wk, *wv, *wo, *wg, *wu, *wd;
  const int8_t *pq, *pk, *pv, *po, *pg, *pu, *pd;  // packed copies (null without)
  const float *wqs, *wks, *wvs, *wos, *wgs, *wus, *wds;
  const float *n1, *nq, *nk, *n2;
  int8_t *kc, *vc;
  float *kcs, *vcs;
};

LayerPtrs layer_ptrs(const q3_model *m, uint32_t L) {
  const q3_layout &y = m->lay;
  const int64_t w = static_cast<int64_t>(L) * y.kLAYERW_STRIDE;
  const int64_t n = static_cast<int64_t>(L) * y.kLAYERN_STRIDE;
  const int64_t kv = y.kKV_BASE + static_cast<int64_t>(L) * y.kKV_STRIDE;
  LayerPtrs p;
  p.wq = at<const int8_t>(m, y.kLQ + w);
  p.wk = at<const int8_t>(m, y.kLK + w);
  p.wv = at<const int8_t>(m, y.kLV + w);
  p.wo = at<const int8_t>(m, y.kLO + w);
  p.wg = at<const int8_t>(m, y.kLG + w);
  p.wu = at<const int8_t>(m, y.kLU + w);
  p.wd = at<const int8_t>(m, y.kLD + w);
  const int8_t *pl = m->packed ? m->packed + static_cast<int64_t>(L) * m->pk_layer : nullptr;
  const int8_t **pp[7] = {&p.pq, &p.pk, &p.pv, &p.po, &p.pg, &p.pu, &p.pd};
  for (int i = 0; i < 7; ++i) *pp[i] = pl ? pl + m->pk_off[i] : nullptr;
  p.wqs = at<const float>(m, y.kLQ_SCALE + w);
  p.wks = at<const float>(m, y.kLK_SCALE + w);
  p.wvs = at<const float>(m, y.kLV_SCALE + w);
  p.wos = at<const float>(m, y.kLO_SCALE + w);
  p.wgs = at<const float>(m, y.kLG_SCALE + w);
  p.wus = at<const float>(m, y.kLU_SCALE + w);
  p.wds = at<const float>(m, y.kLD_SCALE + w);
  p.n1 = at<const float>(m, y.kN1 + n);
  p.nq = at<const float>(m, y.kNQ + n);
  p.nk = at<const float>(m, y.kNK + n);
  p.n2 = at<const float>(m, y.kN2 + n);
  p.kc = at<int8_t>(m, kv);
  p.kcs = at<float>(m, kv + y.kKV_SOFF);
  p.vc = at<int8_t>(m, kv + y.kKV_VOFF);
  p.vcs = at<float>(m, kv + y.kKV_VOFF + y.kKV_SOFF);
  return p;
}

// Sums the recorded event pairs of class c into kt_ms and recycles them
// (synchronises the stream).
int kt_fold(q3_model *m, int c) {
  if (m->kt_used[c] == 0) return Q3_OK;
  Q3_HIP(hipStreamSynchronize(m->stream));
  for (uint32_t i = 0; i < m->kt_used[c]; ++i) {
    float ms = 0.0f;
    Q3_HIP(hipEventElapsedTime(&ms, m->kt_ev[c][2 * i], m->kt_ev[c][2 * i + 1]));
    m->kt_ms[c] += ms;
  }
  m->kt_n[c] += m->kt_used[c];
  m->kt_used[c] = 0;
  return Q3_OK;
}

// Times the one launch issued during its lifetime, when class c is being
// timed, through the launchers' hipExtLaunchKernel events.
class KTimer {
 public:
  KTimer(q3_model *m, int c) : m_(m), c_(c) {
    if (!(m->kt_mask & (1u << c))) return;
    constexpr uint32_t kMaxPairs = 2048;
    if (m->kt_used[c] == kMaxPairs && kt_fold(m, c) != Q3_OK) return;
    std::vector<hipEvent_t> &ev = m->kt_ev[c];
    while (ev.size() < 2 * (m->kt_used[c] + 1)) {
      hipEvent_t e;
      if (hipEventCreate(&e) != hipSuccess) return;
      ev.push_back(e);
    }
    pair_.start = ev[2 * m->kt_used[c]];
    pair_.stop = ev[2 * m->kt_used[c] + 1];
    q3::g_launch_events = &pair_;
    active_ = true;
  }
  ~KTimer() {
    if (!active_) return;
    q3::g_launch_events = nullptr;
    ++m_->kt_used[c_];
  }
  KTimer(const KTimer &) = delete;
  KTimer &operator=(const KTimer &) = delete;

 private:
  q3_model *m_;
  int c_;
  q3::LaunchEvents pair_{};
  bool active_ = false;
};

void set_paged(q3::QDest &d, const q3_model *m, int8_t *pool, float *spool, uint32_t pos0) {
  const q3_layout &y = m->lay;
  const int64_t KW = static_cast<int64_t>(y.kv_heads) * y.head_dim;
  d.q8 = pool;
  d.qs = spool;
  d.table = m->ptab;
  d.page_tokens = kPageTokens;
  d.page_bytes = kPageTokens * KW;
  d.row_bytes = KW;
  d.scale_page_bytes = kPageTokens * y.kv_heads * 4;
  d.scale_row_bytes = y.kv_heads * 4;
  d.pos0 = pos0;
}

// Row kernel over x rows [r0, r0+n): RMSNorm with gain w (or the embedding
// gather for layer 0) into h, then per-256 quant into h8/hs.
int norm_quant_rows(const q3_model *m, int mode, uint32_t pos, uint32_t r0, uint32_t n,
                    const float *w, float *x, float *h, int8_t *h8, float *hs) {
  const q3_layout &y = m->lay;
  const int64_t H = y.hidden;
  q3::RowArgs r{};
  r.mode = mode;
  r.rows = static_cast<int>(n);
  r.cols = static_cast<int>(H);
  r.x = x + r0 * H;
  r.ldx = H;
  if (mode == 2) {
    r.table = at<const int8_t>(m, y.kEMB);
    r.ldt = H;
    r.table_rows = y.vocab;
    r.tscale = at<const float>(m, y.kEMB + static_cast<int64_t>(y.vocab) * H);
    r.tss = 1;
    r.ids = at<const int32_t>(m, y.kIDS) + pos + r0;
    r.ids_stride = 1;
    r.x_out = x + r0 * H;
    r.ldxo = H;
  }
  r.w = w;
  r.w_stride = 1;
  r.inv = 1.0f / static_cast<float>(H);
  r.h = h + r0 * H;
  r.ldh = H;
  r.h8 = h8 + r0 * H;
  r.ldh8 = H;
  r.hs = hs + r0 * (H / 256);
  r.ldhs = H / 256;
  r.group = 256;
  return hip_status(q3::launch_rows(r, m->stream));
}

q3::GemmArgs gemm_args(int M, int N, int K, int group, const int8_t *a, const float *as,
                       const int8_t *b, const float *bs) {
  q3::GemmArgs g;
  std::memset(&g, 0, sizeof(g));
  g.M = M;
  g.N = N;
  g.K = K;
  g.group = group;
  g.a = a;
  g.lda = K;
  g.as = as;
  g.ldas = K / group;
  g.b = b;
  g.ldb = K;
  g.bs = bs;
  g.bs_stride = 1;
  return g;
}

// A residual GEMM (O, down) of a prefill chunk on the packed weights pb,
// when the stream kernel takes it: true and *rc = its status; false when
// the caller's row-major launch must run instead.
bool packed_add(const q3_model *m, const q3::GemmArgs &g, const int8_t *pb, hipStream_t s, int *rc) {
  if (!pb) return false;
  q3::TileArgs t{};
  t.M = g.M;
  t.N = g.N;
  t.K = g.K;
  t.group = g.group;
  t.a = g.a;
  t.lda = g.lda;
  t.as = g.as;
  t.ldas = g.ldas;
  t.b0 = pb;
  t.b_packed = 1;
  t.bs0 = g.bs;
  t.bs_stride = g.bs_stride;
  t.out = g.out;
  t.ldo = g.ldo;
  if (!q3::gemm_stream_supported(t, g.epi)) return false;
  *rc = q3::launch_gemm_stream(t, g.epi, s) == hipSuccess ? Q3_OK : Q3_ERR_HIP;
  return true;
}

q3::GemvArgs gemv_args(int M, int K, int group) {
  q3::GemvArgs v;
  std::memset(&v, 0, sizeof(v));
  v.M = M;
  v.K = K;
  v.group = group;
  return v;
}

q3::GemvSeg gemv_seg(int n0, int n1, int epi, const int8_t *b, const float *bs, float *out,
                     int64_t ldo) {
  q3::GemvSeg g;
  std::memset(&g, 0, sizeof(g));
  g.n0 = n0;
  g.n1 = n1;
  g.epi = epi;
  g.b = b;
  g.bs = bs;
  g.out = out;
  g.ldo = ldo;
  return g;
}

// True when a chunk of `rows` runs on the decode-shaped kernels.
bool small_path(const q3_layout &y, uint32_t rows) {
  const int H = static_cast<int>(y.hidden);
  const int QW = static_cast<int>(y.heads * y.head_dim);
  return rows <= static_cast<uint32_t>(kMaxGemvRows) && q3::gemv_supported(static_cast<int>(rows), H, 256) &&
         q3::gemv_supported(static_cast<int>(rows), QW, static_cast<int>(y.head_dim)) &&
         q3::gemv_supported(static_cast<int>(rows), static_cast<int>(y.inter), 256);
}

// main_big.cpp:264-295: final RMSNorm of the last row, lm_head, and either
// full logits (mode 1) or the fused argmax (mode 0).  Its stage buffers are
// the borrowed rows of main_big.cpp:268-272 (hl = o row 0, h8l = q8 row 0,
// hsl = qs row 0).
int lm_head(q3_model *m, uint32_t rows, int lm_out, int32_t *id_dst) {
  const q3_layout &y = m->lay;
  const hipStream_t s = m->stream;
  const int H = static_cast<int>(y.hidden), V = static_cast<int>(y.vocab);
  if (lm_out == Q3_LM_NONE) return Q3_OK;
  float *x = at<float>(m, y.kX);
  q3::GemvArgs g = gemv_args(1, H, 256);
  g.pro = q3::PRO_NORM;
  g.x = x + static_cast<int64_t>(rows - 1) * H;
  g.ldx = H;
  g.w_pre = at<const float>(m, y.kNF);
  g.inv_pre = 1.0f / static_cast<float>(H);
  g.h_out = at<float>(m, y.kO);
  g.h8_out = at<int8_t>(m, y.kQ8);
  g.hs_out = at<float>(m, y.kQS);
  g.nseg = 1;
  const int8_t *lm = at<const int8_t>(m, y.kLM);
  const float *lm_s = at<const float>(m, y.kLM + static_cast<int64_t>(V) * H);
  if (lm_out == Q3_LM_LOGITS) {
    float *logits = at<float>(m, y.kLOGITS);
    g.seg[0] = gemv_seg(0, V, q3::EPI_STORE, lm, lm_s, logits, V);
    Q3_HIP(q3::launch_gemv(g, s));
    if (id_dst) Q3_HIP(q3::launch_argmax_logits(logits, V, id_dst, nullptr, 0, s));
  } else {
    g.seg[0] = gemv_seg(0, V, q3::EPI_ARGMAX, lm, lm_s, nullptr, 0);
    g.keys = m->keys_ws;
    g.keys_ld = m->keys_ld;
    {
      KTimer kt(m, Q3_KT_LM_HEAD);
      Q3_HIP(q3::launch_gemv(g, s));
    }
    const int nslots = q3::gemv_argmax_slots(g);
    Q3_HIP(q3::launch_argmax_finish(m->keys_ws, m->keys_ld, nslots, 1, at<float>(m, y.kARGF), 1,
                                    at<int32_t>(m, y.kARGI), 1, /*init=*/1, id_dst, nullptr, 0, s));
  }
  return Q3_OK;
}

// main_big.cpp:145-296 for chunks of at most 16 rows: every GEMM is a
// whole-chip GEMV whose prologue builds its int8 operand from the f32 rows
// (embedding / RMSNorm / quant), and whose epilogue is a plain store, the
// residual add, SwiGLU or the argmax.
int forward_small(q3_model *m, uint32_t pos, uint32_t rows, int lm_out, int optimize_tail,
                  int32_t *id_dst) {
  const q3_layout &y = m->lay;
  const hipStream_t s = m->stream;
  const int H = static_cast<int>(y.hidden), HD = static_cast<int>(y.head_dim);
  const int QW = static_cast<int>(y.heads) * HD, KW = static_cast<int>(y.kv_heads) * HD;
  const int I = static_cast<int>(y.inter), V = static_cast<int>(y.vocab);
  const int HALF = static_cast<int>(y.half);
  const int R = static_cast<int>(rows);
  float *x = at<float>(m, y.kX);
  float *h = at<float>(m, y.kH);
  int8_t *h8 = at<int8_t>(m, y.kH8);
  float *hs = at<float>(m, y.kHS);
  float *q = at<float>(m, y.kQ);
  float *k = at<float>(m, y.kK);
  float *v = at<float>(m, y.kV);
  int8_t *q8 = at<int8_t>(m, y.kQ8);
  float *qs = at<float>(m, y.kQS);
  int8_t *o8 = at<int8_t>(m, y.kO8);
  float *os = at<float>(m, y.kOS);
  float *sw = at<float>(m, y.kSW);
  int8_t *s8 = at<int8_t>(m, y.kS8);
  float *ss = at<float>(m, y.kSS);
  const float *cos_t = at<const float>(m, y.kCOS);
  const float *sin_t = at<const float>(m, y.kSIN);
  const float inv_h = 1.0f / static_cast<float>(H);
  const float inv_hd = 1.0f / static_cast<float>(HD);
  const float qk_scale = static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(HD)));

  // layer L - 1's down projection when layer L's launch is to run it
  q3::GemvArgs pend;
  bool have_pend = false;
  for (uint32_t L = 0; L < y.layers; ++L) {
    const LayerPtrs lp = layer_ptrs(m, L);
    const bool is_last = (L + 1 == y.layers);
    float *op = m->opart + static_cast<int64_t>(L & 1) * y.heads * H;
    const bool do_tail = !is_last || lm_out != Q3_LM_NONE;
    const bool tail_last_row = optimize_tail && is_last;
    const uint32_t tr0 = tail_last_row ? rows - 1 : 0;
    const uint32_t tr = tail_last_row ? 1 : rows;
    const int M = static_cast<int>(tr);

    // Q | K | V projections; prologue = (embedding +) RMSNorm n1 + quant
    // (launched below: with the attention when one launch takes both)
    q3::GemvArgs gq;
    {
      q3::GemvArgs g = gemv_args(R, H, 256);
      if (L == 0) {
        g.pro = q3::PRO_EMBED;
        g.emb = at<const int8_t>(m, y.kEMB);
        g.emb_s = at<const float>(m, y.kEMB + static_cast<int64_t>(V) * H);
        g.ids = at<const int32_t>(m, y.kIDS) + pos;
        g.vocab = V;
        g.x_out = x;
      } else {
        g.pro = q3::PRO_NORM;
        g.x = x;
      }
      g.ldx = H;
      g.w_pre = lp.n1;
      g.inv_pre = inv_h;
      g.h_out = h;
      g.h8_out = h8;
      g.hs_out = hs;
      g.nseg = 3;
      g.seg[0] = gemv_seg(0, QW, q3::EPI_STORE, lp.wq, lp.wqs, q, QW);
      g.seg[1] = gemv_seg(QW, QW + KW, q3::EPI_STORE, lp.wk, lp.wks, k, KW);
      g.seg[2] = gemv_seg(QW + KW, QW + 2 * KW, q3::EPI_STORE, lp.wv, lp.wvs, v, KW);
      gq = g;
    }
    // paged GQA attention over kv_len = pos + rows keys
    q3::AttnArgs t{};
    t.rows = M;
    t.heads = static_cast<int>(y.heads);
    t.kv_heads = static_cast<int>(y.kv_heads);
    t.kv_len = pos + rows;
    t.causal = 1;
    t.qk_scale = qk_scale;
    t.q8 = q8 + static_cast<int64_t>(tr0) * QW;
    t.ldq = QW;
    t.qs = qs + static_cast<int64_t>(tr0) * y.heads;
    t.ldqs = y.heads;
    t.qs_col = 1;
    t.k = lp.kc;
    t.v = lp.vc;
    t.ks = lp.kcs;
    t.vs = lp.vcs;
    t.table = m->ptab;
    t.page_tokens = kPageTokens;
    t.page_bytes = static_cast<int64_t>(kPageTokens) * KW;
    t.row_bytes = KW;
    t.scale_page_bytes = static_cast<int64_t>(kPageTokens) * y.kv_heads * 4;
    t.scale_row_bytes = y.kv_heads * 4;
    // page ids of the first key blocks, from the host mirror of the table
    // (the prefill kernel reads them from its arguments; the fused decode
    // variant below sets the same entries)
    {
      const uint32_t nblk = std::min<uint32_t>(32, (pos + rows + 31) / 32);
      for (uint32_t j = 0; j < nblk; ++j) t.blk_page[j] = m->htab[j * 32 / kPageTokens];
      t.blk_page_n = static_cast<int>(nblk);
    }
    t.o8 = o8 + static_cast<int64_t>(tr0) * QW;
    t.ldo = QW;
    t.os = os + static_cast<int64_t>(tr0) * y.heads;
    t.ldos = y.heads;
    t.os_col = 1;
    // one decode token: the head epilogues run in the attention prologue,
    // and the O projection in its epilogue (per-head partials into opart)
    const bool fuse = do_tail && rows == 1 && q3::attn_decode_supported(t);
    bool ofuse = false;
    if (fuse) {
      q3::AttnArgs to = t;
      to.fuse_heads = 1;
      to.wo = lp.wo;
      to.wos = lp.wos;
      to.ldwo = QW;
      to.o_rows = H;
      to.opart = op;
      to.ld_opart = H;
      ofuse = m->ofuse && q3::attn_decode_supported(to);
    }
    if (fuse) {
      // page ids of the first key blocks and of the new token, from the
      // host mirror of the table
      const uint32_t kv_len = pos + rows;
      const uint32_t nblk = std::min<uint32_t>(32, (kv_len + 31) / 32);
      for (uint32_t j = 0; j < 32; ++j) t.blk_page[j] = m->htab[std::min(j, nblk - 1) * 32 / kPageTokens];
      t.new_page = m->htab[(kv_len - 1) / kPageTokens];
      if (ofuse) {
        t.wo = lp.wo;
        t.wos = lp.wos;
        t.ldwo = QW;
        t.o_rows = H;
        t.opart = op;
        t.ld_opart = H;
      }
      t.fuse_heads = 1;
      t.fq = q;
      t.fk = k;
      t.fv = v;
      t.nq = lp.nq;
      t.nk = lp.nk;
      t.cos_row = cos_t + static_cast<int64_t>(pos) * HALF;
      t.sin_row = sin_t + static_cast<int64_t>(pos) * HALF;
      t.inv_hd = inv_hd;
      // while the 16 attention workgroups run, idle CUs pull this layer's
      // O / gate / up / down weights and the next layer's Q / K / V weights
      // into the last-level cache
      const int64_t HH = static_cast<int64_t>(H);
      auto add_pf = [&t](const int8_t *p, int64_t bytes) {
        t.pf[t.pf_n] = p;
        t.pf_bytes[t.pf_n] = bytes;
        ++t.pf_n;
      };
      // (with the O projection fused, this layer's Wo is read by the
      // attention itself, so the next layer's is fetched instead)
      // (each matrix with the row scales that follow it in the blob, and
      // the norm gains of this layer and the next: the small operands every
      // workgroup of the next launches reads first)
      if (!ofuse) add_pf(lp.wo, HH * QW + 4 * HH);
      add_pf(lp.wg, static_cast<int64_t>(I) * H + 4 * I);
      add_pf(lp.wu, static_cast<int64_t>(I) * H + 4 * I);
      add_pf(lp.wd, HH * I + 4 * HH);
      add_pf(reinterpret_cast<const int8_t *>(lp.n1), y.kLAYERN_STRIDE * (is_last ? 1 : 2));
      if (!is_last) {
        const LayerPtrs nx = layer_ptrs(m, L + 1);
        add_pf(nx.wq, static_cast<int64_t>(QW) * H + 4 * QW);
        add_pf(nx.wk, static_cast<int64_t>(KW) * H + 4 * KW);
        add_pf(nx.wv, static_cast<int64_t>(KW) * H + 4 * KW);
        if (ofuse) add_pf(nx.wo, HH * QW + 4 * HH);
      }
      // the K/V pages (and scales) the next attention reads: the next
      // layer's, or layer 0's for the next token after the last layer; each
      // kv head's slices go to the L2 of the XCDs whose heads read them
      // (its own pages through the device table, whatever their order)
      {
        const LayerPtrs nx = layer_ptrs(m, is_last ? 0 : L + 1);
        const uint32_t len = std::min<uint32_t>(pos + rows + (is_last ? 1 : 0), y.max_seq);
        add_pf(nx.kc, 0);
        add_pf(nx.vc, 0);
        add_pf(reinterpret_cast<const int8_t *>(nx.kcs), 0);
        add_pf(reinterpret_cast<const int8_t *>(nx.vcs), 0);
        t.pf_table = m->ptab;
        t.pf_pages = static_cast<int>(std::min<uint32_t>((len + kPageTokens - 1) / kPageTokens, m->n_pages));
        t.pf_kv_heads = static_cast<int>(y.heads);
      }
      t.pf_wgs = m->pf_wgs;
      if (m->pf_wgs == 0) {
        t.pf_n = 0;
        t.pf_kv_heads = 0;
      }
    }
    bool qkvfuse = false;
    if (ofuse && m->qkvfuse) {
      t.xin = m->xin;
      t.xerr = m->xerr;
      qkvfuse = q3::qkv_attn_supported(gq, t);
      if (!qkvfuse) t.xin = nullptr, t.xerr = nullptr;
    }
    // gate/up + SwiGLU; prologue = RMSNorm n2 + quant (launched below); with
    // the down projection merged into the next launch it also clears the
    // exchange words of x
    q3::GemvArgs gu = gemv_args(M, H, 256);
    {
      q3::GemvArgs &g = gu;
      g.pro = q3::PRO_NORM;
      g.x = x + static_cast<int64_t>(tr0) * H;
      g.ldx = H;
      g.w_pre = lp.n2;
      g.inv_pre = inv_h;
      g.h_out = h + static_cast<int64_t>(tr0) * H;
      g.h8_out = h8 + static_cast<int64_t>(tr0) * H;
      g.hs_out = hs + static_cast<int64_t>(tr0) * (H / 256);
      g.nseg = 1;
      g.seg[0] = gemv_seg(0, I, q3::EPI_SWIGLU, lp.wg, lp.wgs, sw + static_cast<int64_t>(tr0) * I, I);
      g.seg[0].b2 = lp.wu;
      g.seg[0].bs2 = lp.wus;
      if (ofuse) {  // normalises x + O
        g.part = op;
        g.npart = static_cast<int>(y.heads);
        g.ld_part = H;
      }
      if (m->merge && rows == 1) {
        g.clear = m->xw;
        g.nclear = q3::kXwWords;
        if (!q3::gemv_clear_supported(g)) g.clear = nullptr, g.nclear = 0;
      }
    }
    // layer L - 1's down projection: in this launch when it can take it
    // (the gate/up launch after it clears x's words), else on its own first
    bool merged = false;
    if (have_pend) {
      if (qkvfuse && gu.clear) {
        t.xw = m->xw;
        merged = q3::down_qkv_attn_supported(pend, gq, t);
        if (!merged) t.xw = nullptr;
      }
      if (!merged) {
        KTimer kt(m, Q3_KT_GEMV_DOWN);
        Q3_HIP(q3::launch_gemv(pend, s));
      }
      have_pend = false;
    }
    if (!qkvfuse) {
      KTimer kt(m, Q3_KT_GEMV_QKV);
      Q3_HIP(q3::launch_gemv(gq, s));
    }
    if (!fuse) {
      // head epilogues: K (norm+RoPE+quant) and V (quant) of every row into
      // the page slots; Q (norm+RoPE+quant) of the tail rows
      q3::QkvHeadArgs e;
      std::memset(&e, 0, sizeof(e));
      e.kv_heads = static_cast<int>(y.kv_heads);
      e.k = k;
      e.v = v;
      e.ldq = QW;
      e.ldk = KW;
      set_paged(e.kd, m, lp.kc, lp.kcs, pos);
      set_paged(e.vd, m, lp.vc, lp.vcs, pos);
      e.nk = lp.nk;
      e.nq = lp.nq;
      e.cos_k = cos_t + static_cast<int64_t>(pos) * HALF;
      e.sin_k = sin_t + static_cast<int64_t>(pos) * HALF;
      e.ld_cs = HALF;
      e.inv_hd = inv_hd;
      e.qd.q8 = q8 + static_cast<int64_t>(tr0) * QW;
      e.qd.ldq8 = QW;
      e.qd.qs = qs + static_cast<int64_t>(tr0) * y.heads;
      e.qd.ldqs = y.heads;
      e.qd.qs_col = 1;
      e.cos_q = cos_t + static_cast<int64_t>(pos + tr0) * HALF;
      e.sin_q = sin_t + static_cast<int64_t>(pos + tr0) * HALF;
      if (do_tail && tr == rows) {
        e.M = R;
        e.q_heads = static_cast<int>(y.heads);
        e.q = q;
        Q3_HIP(q3::launch_qkv_heads(e, s));
      } else {
        e.M = R;
        e.q_heads = 0;
        Q3_HIP(q3::launch_qkv_heads(e, s));
        if (do_tail) {
          q3::QkvHeadArgs eq = e;
          eq.M = M;
          eq.q_heads = static_cast<int>(y.heads);
          eq.kv_heads = 0;
          eq.q = q + static_cast<int64_t>(tr0) * QW;
          Q3_HIP(q3::launch_qkv_heads(eq, s));
        }
      }
    }
    if (!do_tail) continue;
    if (merged) {
      KTimer kt(m, Q3_KT_ATTN_DECODE);
      Q3_HIP(q3::launch_down_qkv_attn(pend, gq, t, s));
    } else if (qkvfuse) {
      KTimer kt(m, Q3_KT_ATTN_DECODE);
      Q3_HIP(q3::launch_qkv_attn(gq, t, s));
    } else if (q3::attn_decode_supported(t)) {
      KTimer kt(m, Q3_KT_ATTN_DECODE);
      Q3_HIP(q3::launch_attn_decode(t, s));
    } else {
      Q3_HIP(q3::launch_attention(t, s));
    }
    float *xt = x + static_cast<int64_t>(tr0) * H;
    // O projection (group = head_dim) + residual (unless the attention
    // computed its partials: then the next two launches add them)
    if (!ofuse) {
      q3::GemvArgs g = gemv_args(M, QW, HD);
      g.a = o8 + static_cast<int64_t>(tr0) * QW;
      g.lda = QW;
      g.as = os + static_cast<int64_t>(tr0) * y.heads;
      g.ldas = y.heads;
      g.nseg = 1;
      g.seg[0] = gemv_seg(0, H, q3::EPI_ADD, lp.wo, lp.wos, xt, H);
      KTimer kt(m, Q3_KT_GEMV_O);
      Q3_HIP(q3::launch_gemv(g, s));
    }
    {
      KTimer kt(m, Q3_KT_GEMV_GATE_UP);
      Q3_HIP(q3::launch_gemv(gu, s));
    }
    // down projection + residual; prologue = per-256 quant of SwiGLU
    {
      q3::GemvArgs g = gemv_args(M, I, 256);
      g.pro = q3::PRO_QUANT;
      g.x = sw + static_cast<int64_t>(tr0) * I;
      g.ldx = I;
      g.h8_out = s8 + static_cast<int64_t>(tr0) * I;
      g.hs_out = ss + static_cast<int64_t>(tr0) * (I / 256);
      g.nseg = 1;
      g.seg[0] = gemv_seg(0, H, q3::EPI_ADD, lp.wd, lp.wds, xt, H);
      if (ofuse) {  // x = (x + O) + down
        g.part = op;
        g.npart = static_cast<int>(y.heads);
        g.ld_part = H;
      }
      if (!is_last && qkvfuse && gu.clear) {  // offered to the next layer's launch
        pend = g;
        have_pend = true;
      } else {
        KTimer kt(m, Q3_KT_GEMV_DOWN);
        Q3_HIP(q3::launch_gemv(g, s));
      }
    }
  }
  if (have_pend) {
    KTimer kt(m, Q3_KT_GEMV_DOWN);
    Q3_HIP(q3::launch_gemv(pend, s));
  }

  return lm_head(m, rows, lm_out, id_dst);
}

// V (quant) and K (norm + RoPE + quant) straight into the page slots and Q
// for the tail rows, with 128-column GEMM tiles (prefill-sized chunks).
int qkv_projections(q3_model *m, const LayerPtrs &lp, uint32_t pos, uint32_t rows, bool do_tail,
                    uint32_t tr0, uint32_t tr) {
  const q3_layout &y = m->lay;
  const hipStream_t s = m->stream;
  const int H = static_cast<int>(y.hidden), HD = static_cast<int>(y.head_dim);
  const int QW = static_cast<int>(y.heads) * HD, KW = static_cast<int>(y.kv_heads) * HD;
  const int HALF = static_cast<int>(y.half);
  int8_t *h8 = at<int8_t>(m, y.kH8);
  float *hs = at<float>(m, y.kHS);
  int8_t *q8 = at<int8_t>(m, y.kQ8);
  float *qs = at<float>(m, y.kQS);
  const float *cos_t = at<const float>(m, y.kCOS);
  const float *sin_t = at<const float>(m, y.kSIN);
  const float inv_hd = 1.0f / static_cast<float>(HD);
  if (do_tail && tr0 == 0 && tr == rows && rows <= 64 &&
      q3::gemv_rows_supported(static_cast<int>(rows), H, 256, QW + 2 * KW)) {
    // up to 64 rows: Q | K | V rows in f32 on the GEMV tiles, then the head
    // epilogues of every (row, head) (Q into q8/qs, K and V into the page
    // slots of positions pos + row)
    float *qf = at<float>(m, y.kQ), *kf = at<float>(m, y.kK), *vf = at<float>(m, y.kV);
    q3::GemvArgs g = gemv_args(static_cast<int>(rows), H, 256);
    g.a = h8;
    g.lda = H;
    g.as = hs;
    g.ldas = H / 256;
    g.nseg = 3;
    g.seg[0] = gemv_seg(0, QW, q3::EPI_STORE, lp.wq, lp.wqs, qf, QW);
    g.seg[1] = gemv_seg(QW, QW + KW, q3::EPI_STORE, lp.wk, lp.wks, kf, KW);
    g.seg[2] = gemv_seg(QW + KW, QW + 2 * KW, q3::EPI_STORE, lp.wv, lp.wvs, vf, KW);
    Q3_HIP(q3::launch_gemv(g, s));
    q3::QkvHeadArgs e;
    std::memset(&e, 0, sizeof(e));
    e.M = static_cast<int>(rows);
    e.q_heads = static_cast<int>(y.heads);
    e.kv_heads = static_cast<int>(y.kv_heads);
    e.q = qf;
    e.k = kf;
    e.v = vf;
    e.ldq = QW;
    e.ldk = KW;
    e.qd.q8 = q8;
    e.qd.ldq8 = QW;
    e.qd.qs = qs;
    e.qd.ldqs = y.heads;
    e.qd.qs_col = 1;
    set_paged(e.kd, m, lp.kc, lp.kcs, pos);
    set_paged(e.vd, m, lp.vc, lp.vcs, pos);
    e.nq = lp.nq;
    e.nk = lp.nk;
    e.cos_q = e.cos_k = cos_t + static_cast<int64_t>(pos) * HALF;
    e.sin_q = e.sin_k = sin_t + static_cast<int64_t>(pos) * HALF;
    e.ld_cs = HALF;
    e.inv_hd = inv_hd;
    return hip_status(q3::launch_qkv_heads(e, s));
  }
  if (do_tail && tr0 == 0 && tr == rows) {
    // Q | K | V as one launch (3x the workgroups of each alone), each column
    // segment with its own weights, epilogue and destination
    q3::TileArgs t{};
    t.M = static_cast<int>(rows);
    t.N = QW + 2 * KW;
    t.K = H;
    t.group = 256;
    t.a = h8;
    t.lda = H;
    t.as = hs;
    t.ldas = H / 256;
    t.ldb = H;
    t.bs_stride = 1;
    t.nw_stride = 1;
    t.cos_t = cos_t + static_cast<int64_t>(pos) * HALF;
    t.sin_t = sin_t + static_cast<int64_t>(pos) * HALF;
    t.ld_cs = HALF;
    t.inv_hd = inv_hd;
    t.nseg = 3;
    t.seg[0].n0 = 0;
    t.seg[0].n1 = QW;
    t.seg[0].b = lp.wq;
    t.seg[0].bs = lp.wqs;
    t.seg[0].qd.q8 = q8;
    t.seg[0].qd.ldq8 = QW;
    t.seg[0].qd.qs = qs;
    t.seg[0].qd.ldqs = y.heads;
    t.seg[0].qd.qs_col = 1;
    t.seg[0].nw = lp.nq;
    t.seg[0].norm = 1;
    t.seg[1].n0 = QW;
    t.seg[1].n1 = QW + KW;
    t.seg[1].b = lp.wk;
    t.seg[1].bs = lp.wks;
    set_paged(t.seg[1].qd, m, lp.kc, lp.kcs, pos);
    t.seg[1].nw = lp.nk;
    t.seg[1].norm = 1;
    t.seg[2].n0 = QW + KW;
    t.seg[2].n1 = QW + 2 * KW;
    t.seg[2].b = lp.wv;
    t.seg[2].bs = lp.wvs;
    set_paged(t.seg[2].qd, m, lp.vc, lp.vcs, pos);
    t.seg[2].norm = 0;
    if (lp.pq) {  // the packed weights, when the stream kernel takes the chunk
      q3::TileArgs tp = t;
      tp.b_packed = 1;
      tp.seg[0].b = lp.pq;
      tp.seg[1].b = lp.pk;
      tp.seg[2].b = lp.pv;
      if (q3::gemm_stream_supported(tp, q3::EPI_QKV)) return hip_status(q3::launch_gemm_stream(tp, q3::EPI_QKV, s));
    }
    if (q3::gemm_tile_supported(t, q3::EPI_QKV)) return hip_status(q3::launch_gemm_tile(t, q3::EPI_QKV, s));
  }
  {
    q3::GemmArgs g = gemm_args(static_cast<int>(rows), KW, H, 256, h8, hs, lp.wv, lp.wvs);
    g.epi = q3::EPI_HEADQ;
    set_paged(g.qd, m, lp.vc, lp.vcs, pos);
    Q3_HIP(q3::launch_gemm(g, s));
  }
  {
    q3::GemmArgs g = gemm_args(static_cast<int>(rows), KW, H, 256, h8, hs, lp.wk, lp.wks);
    g.epi = q3::EPI_NRQ;
    set_paged(g.qd, m, lp.kc, lp.kcs, pos);
    g.nw = lp.nk;
    g.nw_stride = 1;
    g.cos_t = cos_t + static_cast<int64_t>(pos) * HALF;
    g.sin_t = sin_t + static_cast<int64_t>(pos) * HALF;
    g.ld_cs = HALF;
    g.inv_hd = inv_hd;
    Q3_HIP(q3::launch_gemm(g, s));
  }
  if (do_tail) {
    q3::GemmArgs g = gemm_args(static_cast<int>(tr), QW, H, 256, h8 + static_cast<int64_t>(tr0) * H,
                               hs + static_cast<int64_t>(tr0) * (H / 256), lp.wq, lp.wqs);
    g.epi = q3::EPI_NRQ;
    g.qd.q8 = q8 + static_cast<int64_t>(tr0) * QW;
    g.qd.ldq8 = QW;
    g.qd.qs = qs + static_cast<int64_t>(tr0) * y.heads;
    g.qd.ldqs = y.heads;
    g.qd.qs_col = 1;
    g.nw = lp.nq;
    g.nw_stride = 1;
    g.cos_t = cos_t + static_cast<int64_t>(pos + tr0) * HALF;
    g.sin_t = sin_t + static_cast<int64_t>(pos + tr0) * HALF;
    g.ld_cs = HALF;
    g.inv_hd = inv_hd;
    Q3_HIP(q3::launch_gemm(g, s));
  }
  return Q3_OK;
}

// main_big.cpp:145-296.  id_dst (device, may be null) receives the greedy id
// of the last row when lm_out != Q3_LM_NONE.
int forward_chunk_impl(q3_model *m, uint32_t pos, uint32_t rows, int lm_out,
                       int optimize_tail, int32_t *id_dst) {
  const q3_layout &y = m->lay;
  if (rows == 0 || rows > y.seq || pos + rows > y.max_seq) return Q3_ERR_RANGE;
  if (lm_out < Q3_LM_NONE || lm_out > Q3_LM_ARGMAX) return Q3_ERR_ARG;
  if (small_path(y, rows)) return forward_small(m, pos, rows, lm_out, optimize_tail, id_dst);
  const int H = static_cast<int>(y.hidden), HD = static_cast<int>(y.head_dim);
  const int QW = static_cast<int>(y.heads) * HD, KW = static_cast<int>(y.kv_heads) * HD;
  const int I = static_cast<int>(y.inter);
  const hipStream_t s = m->stream;

  float *x = at<float>(m, y.kX);
  float *h = at<float>(m, y.kH);
  int8_t *h8 = at<int8_t>(m, y.kH8);
  float *hs = at<float>(m, y.kHS);
  int8_t *q8 = at<int8_t>(m, y.kQ8);
  float *qs = at<float>(m, y.kQS);
  int8_t *o8 = at<int8_t>(m, y.kO8);
  float *os = at<float>(m, y.kOS);
  int8_t *s8 = at<int8_t>(m, y.kS8);
  float *ss = at<float>(m, y.kSS);
  const float qk_scale = static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(HD)));

  // embedding + layer-0 RMSNorm (main_big.cpp:163-166), then its quant
  {
    const LayerPtrs l0 = layer_ptrs(m, 0);
    const int rc = norm_quant_rows(m, 2, pos, 0, rows, l0.n1, x, h, h8, hs);
    if (rc != Q3_OK) return rc;
  }

  for (uint32_t L = 0; L < y.layers; ++L) {
    const LayerPtrs lp = layer_ptrs(m, L);
    if (L != 0) {
      const int rc = norm_quant_rows(m, 1, pos, 0, rows, lp.n1, x, h, h8, hs);
      if (rc != Q3_OK) return rc;
    }
    // main_big.cpp:212-223: the last layer only needs the tail rows
    const bool is_last = (L + 1 == y.layers);
    const bool do_tail = !is_last || lm_out != Q3_LM_NONE;
    const bool tail_last_row = optimize_tail && is_last;
    const uint32_t tr0 = tail_last_row ? rows - 1 : 0;
    const uint32_t tr = tail_last_row ? 1 : rows;
    const int M = static_cast<int>(tr);

    // K (norm + RoPE + quant) and V (quant) straight into the page slots,
    // Q (norm + RoPE + quant) for the tail rows
    const int rc_qkv = qkv_projections(m, lp, pos, rows, do_tail, tr0, tr);
    if (rc_qkv != Q3_OK) return rc_qkv;
    if (!do_tail) continue;

    // paged GQA attention over kv_len = pos + rows keys
    {
      q3::AttnArgs t{};
      t.rows = M;
      t.heads = static_cast<int>(y.heads);
      t.kv_heads = static_cast<int>(y.kv_heads);
      t.kv_len = pos + rows;
      t.causal = 1;
      t.qk_scale = qk_scale;
      t.q8 = q8 + static_cast<int64_t>(tr0) * QW;
      t.ldq = QW;
      t.qs = qs + static_cast<int64_t>(tr0) * y.heads;
      t.ldqs = y.heads;
      t.qs_col = 1;
      t.k = lp.kc;
      t.v = lp.vc;
      t.ks = lp.kcs;
      t.vs = lp.vcs;
      t.table = m->ptab;
      t.page_tokens = kPageTokens;
      t.page_bytes = static_cast<int64_t>(kPageTokens) * KW;
      t.row_bytes = KW;
      t.scale_page_bytes = static_cast<int64_t>(kPageTokens) * y.kv_heads * 4;
      t.scale_row_bytes = y.kv_heads * 4;
      t.o8 = o8 + static_cast<int64_t>(tr0) * QW;
      t.ldo = QW;
      t.os = os + static_cast<int64_t>(tr0) * y.heads;
      t.ldos = y.heads;
      t.os_col = 1;
      if (q3::attn_decode_supported(t))
        Q3_HIP(q3::launch_attn_decode(t, s));
      else
        Q3_HIP(q3::launch_attention(t, s));
    }
    float *xt = x + static_cast<int64_t>(tr0) * H;
    // up to 64 rows: the GEMMs below on the GEMV tiles (the gate/up as
    // SwiGLU rows in f32, then their per-256-column quant)
    const bool gv = M <= 64 && q3::gemv_rows_supported(M, QW, HD, H) && q3::gemv_rows_supported(M, H, 256, I) &&
                    q3::gemv_rows_supported(M, I, 256, H);
    // O projection (group = head_dim) + residual into x
    if (gv) {
      q3::GemvArgs g = gemv_args(M, QW, HD);
      g.a = o8 + static_cast<int64_t>(tr0) * QW;
      g.lda = QW;
      g.as = os + static_cast<int64_t>(tr0) * y.heads;
      g.ldas = y.heads;
      g.nseg = 1;
      g.seg[0] = gemv_seg(0, H, q3::EPI_ADD, lp.wo, lp.wos, xt, H);
      Q3_HIP(q3::launch_gemv(g, s));
    } else {
      q3::GemmArgs g = gemm_args(M, H, QW, HD, o8 + static_cast<int64_t>(tr0) * QW,
                                 os + static_cast<int64_t>(tr0) * y.heads, lp.wo, lp.wos);
      g.epi = q3::EPI_ADD;
      g.out = xt;
      g.ldo = H;
      int rc = Q3_OK;
      if (packed_add(m, g, lp.po, s, &rc)) {
        if (rc != Q3_OK) return rc;
      } else {
        Q3_HIP(q3::launch_gemm(g, s));
      }
    }
    // post-attention RMSNorm + quant
    {
      const int rc = norm_quant_rows(m, 1, pos, tr0, tr, lp.n2, x, h, h8, hs);
      if (rc != Q3_OK) return rc;
    }
    // gate/up + SwiGLU + quant
    {
      q3::GateUpArgs u{};
      u.M = M;
      u.N = I;
      u.K = H;
      u.group = 256;
      u.a = h8 + static_cast<int64_t>(tr0) * H;
      u.lda = H;
      u.as = hs + static_cast<int64_t>(tr0) * (H / 256);
      u.ldas = H / 256;
      u.wg = lp.wg;
      u.wu = lp.wu;
      u.ldw = H;
      u.wgs = lp.wgs;
      u.wus = lp.wus;
      u.ws_stride = 1;
      u.s8 = s8 + static_cast<int64_t>(tr0) * I;
      u.lds8 = I;
      u.ss = ss + static_cast<int64_t>(tr0) * (I / 256);
      u.ldss = I / 256;
      u.ss_col = 1;
      q3::TileArgs t{};  // the packed weights, when the stream kernel takes the chunk
      t.M = M;
      t.N = I;
      t.K = H;
      t.group = 256;
      t.a = u.a;
      t.lda = H;
      t.as = u.as;
      t.ldas = H / 256;
      t.b0 = lp.pg;
      t.b1 = lp.pu;
      t.b_packed = 1;
      t.bs0 = lp.wgs;
      t.bs1 = lp.wus;
      t.bs_stride = 1;
      t.s8 = u.s8;
      t.lds8 = I;
      t.ss = u.ss;
      t.ldss = I / 256;
      t.ss_col = 1;
      if (gv) {
        float *swf = at<float>(m, y.kSW) + static_cast<int64_t>(tr0) * I;
        q3::GemvArgs g = gemv_args(M, H, 256);
        g.a = u.a;
        g.lda = H;
        g.as = u.as;
        g.ldas = H / 256;
        g.nseg = 1;
        g.seg[0] = gemv_seg(0, I, q3::EPI_SWIGLU, lp.wg, lp.wgs, swf, I);
        g.seg[0].b2 = lp.wu;
        g.seg[0].bs2 = lp.wus;
        Q3_HIP(q3::launch_gemv(g, s));
        q3::RowArgs r{};
        r.mode = 0;
        r.rows = M;
        r.cols = I;
        r.x = swf;
        r.ldx = I;
        r.h8 = u.s8;
        r.ldh8 = I;
        r.hs = u.ss;
        r.ldhs = I / 256;
        r.group = 256;
        Q3_HIP(q3::launch_rows(r, s));
      } else if (lp.pg && q3::gemm_stream_supported(t, q3::EPI_SWIGLUQ)) {
        Q3_HIP(q3::launch_gemm_stream(t, q3::EPI_SWIGLUQ, s));
      } else {
        Q3_HIP(q3::launch_gate_up(u, s));
      }
    }
    // down projection + residual into x
    if (gv) {
      q3::GemvArgs g = gemv_args(M, I, 256);
      g.a = s8 + static_cast<int64_t>(tr0) * I;
      g.lda = I;
      g.as = ss + static_cast<int64_t>(tr0) * (I / 256);
      g.ldas = I / 256;
      g.nseg = 1;
      g.seg[0] = gemv_seg(0, H, q3::EPI_ADD, lp.wd, lp.wds, xt, H);
      Q3_HIP(q3::launch_gemv(g, s));
    } else {
      q3::GemmArgs g = gemm_args(M, H, I, 256, s8 + static_cast<int64_t>(tr0) * I,
                                 ss + static_cast<int64_t>(tr0) * (I / 256), lp.wd, lp.wds);
      g.epi = q3::EPI_ADD;
      g.out = xt;
      g.ldo = H;
      int rc = Q3_OK;
      if (packed_add(m, g, lp.pd, s, &rc)) {
        if (rc != Q3_OK) return rc;
      } else {
        Q3_HIP(q3::launch_gemm(g, s));
      }
    }
  }

  return lm_head(m, rows, lm_out, id_dst);
}

}  // namespace

// The packed copy of every layer's seven weight matrices (q3::launch_pack_b
// layout), made once on the model's stream.
static int repack_weights(q3_model *m);

static int pack_weights(q3_model *m) {
  const q3_layout &y = m->lay;
  const int64_t H = y.hidden, QW = static_cast<int64_t>(y.heads) * y.head_dim;
  const int64_t KW = static_cast<int64_t>(y.kv_heads) * y.head_dim, I = y.inter;
  const int64_t rows[7] = {QW, KW, KW, H, I, I, H}, cols[7] = {H, H, H, QW, H, H, I};
  int64_t off = 0;
  for (int i = 0; i < 7; ++i) {
    if (rows[i] % 16 || cols[i] % 64) return Q3_OK;  // shapes the stream kernel never takes
    m->pk_off[i] = off;
    off += (rows[i] * cols[i] + 255) & ~int64_t(255);
  }
  m->pk_layer = off;
  if (hipMalloc(&m->packed, static_cast<size_t>(off) * y.layers) != hipSuccess) {
    // no room for the copy: prefill reads the row-major blob instead
    (void)hipGetLastError();
    m->packed = nullptr;
    return Q3_OK;
  }
  return repack_weights(m);
}

// The layer weights of the blob into the packed copy (fragment order).
static int repack_weights(q3_model *m) {
  const q3_layout &y = m->lay;
  const int64_t H = y.hidden, QW = static_cast<int64_t>(y.heads) * y.head_dim;
  const int64_t KW = static_cast<int64_t>(y.kv_heads) * y.head_dim, I = y.inter;
  const int64_t rows[7] = {QW, KW, KW, H, I, I, H}, cols[7] = {H, H, H, QW, H, H, I};
  const int64_t off = m->pk_layer;
  for (uint32_t L = 0; L < y.layers; ++L) {
    const int64_t w = static_cast<int64_t>(L) * y.kLAYERW_STRIDE;
    const int64_t src[7] = {y.kLQ, y.kLK, y.kLV, y.kLO, y.kLG, y.kLU, y.kLD};
    for (int i = 0; i < 7; ++i)
      Q3_HIP(q3::launch_pack_b(at<const int8_t>(m, src[i] + w), cols[i], static_cast<int>(rows[i]),
                               static_cast<int>(cols[i]), m->packed + L * off + m->pk_off[i], m->stream));
  }
  Q3_HIP(hipStreamSynchronize(m->stream));
  return Q3_OK;
}

extern "C" int q3_model_open(void *blob, const q3_layout *lay, void *stream, q3_model **out) {
  if (!blob || !lay || !out) return Q3_ERR_ARG;
  *out = nullptr;
  // Shapes the kernels are written for (hd128 heads, 256-column groups).
  if (lay->kv_heads == 0 || lay->heads == 0) return Q3_ERR_UNSUPPORTED;
  if (lay->head_dim != 128 || lay->hidden % 256 || lay->inter % 256 || lay->vocab % 128 ||
      lay->max_seq % kPageTokens || lay->heads % lay->kv_heads || lay->seq == 0)
    return Q3_ERR_UNSUPPORTED;
  if (lay->max_seq / kPageTokens > 65536) return Q3_ERR_UNSUPPORTED;
  q3_model *m = new (std::nothrow) q3_model();
  if (!m) return Q3_ERR_ARG;
  m->blob = static_cast<uint8_t *>(blob);
  m->lay = *lay;
  m->stream = static_cast<hipStream_t>(stream);
  m->n_pages = lay->max_seq / kPageTokens;
  m->keys_ld = lay->vocab / 16 + 64;  // one key per lm_head column block
  // (re-swept with the merged launch, ms/token, two runs each: 69 0.6225, 88 0.670, 104 0.619,
  // 120 0.6182, 136 0.6182, 152 0.6194, 176 0.6203, 240 0.619)
  m->pf_wgs = 120;
  if (const char *e = std::getenv("Q3_DECODE_PREFETCH_WGS")) m->pf_wgs = std::max(0, std::atoi(e));
  if (const char *e = std::getenv("Q3_DECODE_FUSE_OPROJ")) m->ofuse = std::atoi(e) != 0;
  if (const char *e = std::getenv("Q3_DECODE_GRAPH")) m->dgraph_on = std::atoi(e) != 0;
  if (const char *e = std::getenv("Q3_DECODE_FUSE_QKV")) m->qkvfuse = std::atoi(e) != 0;
  if (const char *e = std::getenv("Q3_DECODE_MERGE_DOWN")) m->merge = std::atoi(e) != 0;
  m->bkeys_ld = lay->vocab / 128 + 64;  // one key per 128-column block of the lm GEMM
  m->btab_off = (sizeof(int32_t) * lay->seq + 255) & ~size_t(255);
  const size_t bstate_bytes = m->btab_off + sizeof(uint16_t) * static_cast<size_t>(lay->seq) * m->n_pages;
  if (hipMalloc(&m->ptab, sizeof(uint16_t) * m->n_pages) != hipSuccess ||
      hipMalloc(&m->keys, sizeof(unsigned long long) * 8) != hipSuccess ||
      hipMalloc(&m->keys_ws, sizeof(unsigned long long) * m->keys_ld) != hipSuccess ||
      hipMalloc(&m->bstate, bstate_bytes) != hipSuccess ||
      hipHostMalloc(&m->bstage[0], bstate_bytes, hipHostMallocDefault) != hipSuccess ||
      hipHostMalloc(&m->bstage[1], bstate_bytes, hipHostMallocDefault) != hipSuccess ||
      hipEventCreateWithFlags(&m->bstage_ev[0], hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&m->bstage_ev[1], hipEventDisableTiming) != hipSuccess ||
      hipMalloc(&m->bkeys, sizeof(unsigned long long) * static_cast<size_t>(lay->seq) * m->bkeys_ld) !=
          hipSuccess ||
      hipMalloc(&m->bbest, sizeof(float) * lay->seq) != hipSuccess ||
      hipMalloc(&m->opart, sizeof(float) * 2 * lay->heads * lay->hidden) != hipSuccess) {
    q3_model_close(m);
    return Q3_ERR_HIP;
  }
  {
    const size_t xbytes = sizeof(unsigned long long) * 3 * lay->heads * lay->head_dim;
    const size_t wbytes = sizeof(uint32_t) * q3::kXwWords;
    if (hipMalloc(&m->xin, xbytes) != hipSuccess || hipMalloc(&m->xerr, sizeof(uint32_t)) != hipSuccess ||
        hipMalloc(&m->xw, wbytes) != hipSuccess || hipMemset(m->xin, 0, xbytes) != hipSuccess ||
        hipMemset(m->xw, 0xFF, wbytes) != hipSuccess || hipMemset(m->xerr, 0, sizeof(uint32_t)) != hipSuccess) {
      q3_model_close(m);
      return Q3_ERR_HIP;
    }
  }
  m->bpos = reinterpret_cast<int32_t *>(m->bstate);
  m->btab = reinterpret_cast<uint16_t *>(m->bstate + m->btab_off);
  std::vector<uint16_t> &tab = m->htab;
  tab.resize(m->n_pages);
  for (uint32_t p = 0; p < m->n_pages; ++p) tab[p] = static_cast<uint16_t>(m->n_pages - 1 - p);
  if (hipMemcpy(m->ptab, tab.data(), sizeof(uint16_t) * m->n_pages, hipMemcpyHostToDevice) !=
          hipSuccess ||
      hipMemset(m->keys, 0, sizeof(unsigned long long) * 8) != hipSuccess) {
    q3_model_close(m);
    return Q3_ERR_HIP;
  }
  const char *pk_env = std::getenv("Q3_PACKED_WEIGHTS");
  if (lay->seq > 64 && !(pk_env && std::atoi(pk_env) == 0)) {
    const int rc = pack_weights(m);
    if (rc != Q3_OK) {
      q3_model_close(m);
      return rc;
    }
  }
  *out = m;
  return Q3_OK;
}

// One decode step of n independent sequences (batched decode).  The
// reference's pieces for it are op-level: paged_kv_scatter_batch
// (kernels/kv_pages.h) writes each request's K/V row through its own page
// table, and paged attention runs per request (tests/guest/paged_attn_multi
// .cpp); every GEMM is row-independent, so the rows of different sequences
// share one launch.  Row r: token ids[r] (device) at position pos[r], pages
// tables[r * ld_table ...] (host arrays, validated here and staged through
// pinned memory to the model's device buffers, so the call does not wait for
// the stream); out_ids[r] (device) receives its greedy id.
extern "C" int q3_decode_batch(q3_model *m, uint32_t n, const int32_t *ids, const int32_t *pos,
                               const uint16_t *tables, uint32_t ld_table, int32_t *out_ids) {
  if (!m || !ids || !pos || !tables || !out_ids || n == 0) return Q3_ERR_ARG;
  const q3_layout &y = m->lay;
  if (n > y.seq) return Q3_ERR_RANGE;
  if (ld_table == 0 || ld_table > m->n_pages) return Q3_ERR_ARG;
  for (uint32_t r = 0; r < n; ++r) {
    if (pos[r] < 0 || static_cast<uint32_t>(pos[r]) >= y.max_seq) return Q3_ERR_RANGE;
    if (static_cast<uint32_t>(pos[r]) / kPageTokens >= ld_table) return Q3_ERR_RANGE;
    for (uint32_t i = 0; i <= static_cast<uint32_t>(pos[r]) / kPageTokens; ++i)
      if (tables[static_cast<size_t>(r) * ld_table + i] >= m->n_pages) return Q3_ERR_RANGE;
  }
  const hipStream_t s = m->stream;
  {
    const uint32_t slot = m->bstage_next;
    if (m->bstage_used[slot]) Q3_HIP(hipEventSynchronize(m->bstage_ev[slot]));
    uint8_t *st = m->bstage[slot];
    const size_t tab_bytes = sizeof(uint16_t) * static_cast<size_t>(n) * ld_table;
    std::memcpy(st, pos, sizeof(int32_t) * n);
    std::memcpy(st + m->btab_off, tables, tab_bytes);
    Q3_HIP(hipMemcpyAsync(m->bstate, st, m->btab_off + tab_bytes, hipMemcpyHostToDevice, s));
    Q3_HIP(hipEventRecord(m->bstage_ev[slot], s));
    m->bstage_used[slot] = true;
    m->bstage_next = slot ^ 1;
  }
  const int H = static_cast<int>(y.hidden), HD = static_cast<int>(y.head_dim);
  const int QW = static_cast<int>(y.heads) * HD, KW = static_cast<int>(y.kv_heads) * HD;
  const int I = static_cast<int>(y.inter), V = static_cast<int>(y.vocab);
  const int HALF = static_cast<int>(y.half);
  const int M = static_cast<int>(n);
  float *x = at<float>(m, y.kX);
  float *h = at<float>(m, y.kH);
  int8_t *h8 = at<int8_t>(m, y.kH8);
  float *hs = at<float>(m, y.kHS);
  int8_t *q8 = at<int8_t>(m, y.kQ8);
  float *qs = at<float>(m, y.kQS);
  int8_t *o8 = at<int8_t>(m, y.kO8);
  float *os = at<float>(m, y.kOS);
  int8_t *s8 = at<int8_t>(m, y.kS8);
  float *ss = at<float>(m, y.kSS);
  const float *cos_t = at<const float>(m, y.kCOS);
  const float *sin_t = at<const float>(m, y.kSIN);
  const float qk_scale = static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(HD)));

  auto rows = [&](int mode, const float *w) -> int {  // embedding/RMSNorm + quant of n rows
    q3::RowArgs r{};
    r.mode = mode;
    r.rows = M;
    r.cols = H;
    r.x = x;
    r.ldx = H;
    if (mode == 2) {
      r.table = at<const int8_t>(m, y.kEMB);
      r.ldt = H;
      r.table_rows = y.vocab;
      r.tscale = at<const float>(m, y.kEMB + static_cast<int64_t>(V) * H);
      r.tss = 1;
      r.ids = ids;
      r.ids_stride = 1;
      r.x_out = x;
      r.ldxo = H;
    }
    r.w = w;
    r.w_stride = 1;
    r.inv = 1.0f / static_cast<float>(H);
    r.h = h;
    r.ldh = H;
    r.h8 = h8;
    r.ldh8 = H;
    r.hs = hs;
    r.ldhs = H / 256;
    r.group = 256;
    return hip_status(q3::launch_rows(r, s));
  };
  Q3_TRY(rows(2, layer_ptrs(m, 0).n1));
  // up to 64 rows: the GEMMs run on the 16-column GEMV tiles (every CU
  // streams a slice of the weights; the rows come from L2), with the head
  // epilogues and the SwiGLU quantisation as launches of their own
  const bool gv = q3::gemv_rows_supported(M, H, 256, QW + 2 * KW) && q3::gemv_rows_supported(M, QW, HD, H) &&
                  q3::gemv_rows_supported(M, I, 256, H) && q3::gemv_rows_supported(M, H, 256, I);
  float *qf = at<float>(m, y.kQ), *kf = at<float>(m, y.kK), *vf = at<float>(m, y.kV);
  float *swf = at<float>(m, y.kSW);
  for (uint32_t L = 0; L < y.layers; ++L) {
    const LayerPtrs lp = layer_ptrs(m, L);
    if (L != 0) Q3_TRY(rows(1, lp.n1));
    if (gv) {
      // Q | K | V rows in f32, then the head epilogues of every (row, head):
      // Q (norm, RoPE, quant) into the dense q8/qs rows, K (norm, RoPE,
      // quant) and V (quant) into each row's page slot at its own position
      q3::GemvArgs g = gemv_args(M, H, 256);
      g.a = h8;
      g.lda = H;
      g.as = hs;
      g.ldas = H / 256;
      g.nseg = 3;
      g.seg[0] = gemv_seg(0, QW, q3::EPI_STORE, lp.wq, lp.wqs, qf, QW);
      g.seg[1] = gemv_seg(QW, QW + KW, q3::EPI_STORE, lp.wk, lp.wks, kf, KW);
      g.seg[2] = gemv_seg(QW + KW, QW + 2 * KW, q3::EPI_STORE, lp.wv, lp.wvs, vf, KW);
      Q3_HIP(q3::launch_gemv(g, s));
      q3::QkvHeadArgs e;
      std::memset(&e, 0, sizeof(e));
      e.M = M;
      e.q_heads = static_cast<int>(y.heads);
      e.kv_heads = static_cast<int>(y.kv_heads);
      e.q = qf;
      e.k = kf;
      e.v = vf;
      e.ldq = QW;
      e.ldk = KW;
      e.qd.q8 = q8;
      e.qd.ldq8 = QW;
      e.qd.qs = qs;
      e.qd.ldqs = y.heads;
      e.qd.qs_col = 1;
      set_paged(e.kd, m, lp.kc, lp.kcs, 0);
      set_paged(e.vd, m, lp.vc, lp.vcs, 0);
      e.nq = lp.nq;
      e.nk = lp.nk;
      e.cos_q = e.cos_k = cos_t;
      e.sin_q = e.sin_k = sin_t;
      e.ld_cs = HALF;
      e.inv_hd = 1.0f / static_cast<float>(HD);
      e.row_pos = m->bpos;
      e.row_tables = m->btab;
      e.ld_table = ld_table;
      Q3_HIP(q3::launch_qkv_heads(e, s));
    } else {
      // Q | K | V in one tile launch with the head epilogues, as above
      q3::TileArgs t{};
      t.M = M;
      t.N = QW + 2 * KW;
      t.K = H;
      t.group = 256;
      t.a = h8;
      t.lda = H;
      t.as = hs;
      t.ldas = H / 256;
      t.ldb = H;
      t.bs_stride = 1;
      t.nw_stride = 1;
      t.cos_t = cos_t;
      t.sin_t = sin_t;
      t.ld_cs = HALF;
      t.cs_row_pos = m->bpos;
      t.inv_hd = 1.0f / static_cast<float>(HD);
      t.nseg = 3;
      t.seg[0].n0 = 0;
      t.seg[0].n1 = QW;
      t.seg[0].b = lp.wq;
      t.seg[0].bs = lp.wqs;
      t.seg[0].qd.q8 = q8;
      t.seg[0].qd.ldq8 = QW;
      t.seg[0].qd.qs = qs;
      t.seg[0].qd.ldqs = y.heads;
      t.seg[0].qd.qs_col = 1;
      t.seg[0].nw = lp.nq;
      t.seg[0].norm = 1;
      t.seg[1].n0 = QW;
      t.seg[1].n1 = QW + KW;
      t.seg[1].b = lp.wk;
      t.seg[1].bs = lp.wks;
      set_paged(t.seg[1].qd, m, lp.kc, lp.kcs, 0);
      t.seg[1].nw = lp.nk;
      t.seg[1].norm = 1;
      t.seg[2].n0 = QW + KW;
      t.seg[2].n1 = QW + 2 * KW;
      t.seg[2].b = lp.wv;
      t.seg[2].bs = lp.wvs;
      set_paged(t.seg[2].qd, m, lp.vc, lp.vcs, 0);
      t.seg[2].norm = 0;
      for (int sg = 1; sg < 3; ++sg) {
        t.seg[sg].qd.table = nullptr;
        t.seg[sg].qd.row_pos = m->bpos;
        t.seg[sg].qd.row_tables = m->btab;
        t.seg[sg].qd.ld_table = ld_table;
      }
      if (!q3::gemm_tile_supported(t, q3::EPI_QKV)) return Q3_ERR_UNSUPPORTED;
      Q3_HIP(q3::launch_gemm_tile(t, q3::EPI_QKV, s));
    }
    {
      q3::AttnArgs t{};
      t.rows = M;
      t.heads = static_cast<int>(y.heads);
      t.kv_heads = static_cast<int>(y.kv_heads);
      t.causal = 1;
      t.qk_scale = qk_scale;
      t.q8 = q8;
      t.ldq = QW;
      t.qs = qs;
      t.ldqs = y.heads;
      t.qs_col = 1;
      t.k = lp.kc;
      t.v = lp.vc;
      t.ks = lp.kcs;
      t.vs = lp.vcs;
      t.table = m->btab;
      t.page_tokens = kPageTokens;
      t.page_bytes = static_cast<int64_t>(kPageTokens) * KW;
      t.row_bytes = KW;
      t.scale_page_bytes = static_cast<int64_t>(kPageTokens) * y.kv_heads * 4;
      t.scale_row_bytes = y.kv_heads * 4;
      t.o8 = o8;
      t.ldo = QW;
      t.os = os;
      t.ldos = y.heads;
      t.os_col = 1;
      t.row_pos = m->bpos;
      t.row_tables = m->btab;
      t.ld_table = ld_table;
      if (!q3::attn_decode_supported(t)) return Q3_ERR_UNSUPPORTED;
      KTimer kt(m, Q3_KT_ATTN_DECODE);
      Q3_HIP(q3::launch_attn_decode(t, s));
    }
    if (gv) {  // O projection + residual
      q3::GemvArgs g = gemv_args(M, QW, HD);
      g.a = o8;
      g.lda = QW;
      g.as = os;
      g.ldas = y.heads;
      g.nseg = 1;
      g.seg[0] = gemv_seg(0, H, q3::EPI_ADD, lp.wo, lp.wos, x, H);
      Q3_HIP(q3::launch_gemv(g, s));
    } else {
      q3::GemmArgs g = gemm_args(M, H, QW, HD, o8, os, lp.wo, lp.wos);
      g.ldas = y.heads;
      g.epi = q3::EPI_ADD;
      g.out = x;
      g.ldo = H;
      Q3_HIP(q3::launch_gemm(g, s));
    }
    Q3_TRY(rows(1, lp.n2));
    if (gv) {  // gate/up + SwiGLU (f32 rows), then the per-256-column quant
      q3::GemvArgs g = gemv_args(M, H, 256);
      g.a = h8;
      g.lda = H;
      g.as = hs;
      g.ldas = H / 256;
      g.nseg = 1;
      g.seg[0] = gemv_seg(0, I, q3::EPI_SWIGLU, lp.wg, lp.wgs, swf, I);
      g.seg[0].b2 = lp.wu;
      g.seg[0].bs2 = lp.wus;
      Q3_HIP(q3::launch_gemv(g, s));
      q3::RowArgs r{};
      r.mode = 0;
      r.rows = M;
      r.cols = I;
      r.x = swf;
      r.ldx = I;
      r.h8 = s8;
      r.ldh8 = I;
      r.hs = ss;
      r.ldhs = I / 256;
      r.group = 256;
      Q3_HIP(q3::launch_rows(r, s));
    } else {  // gate/up + SwiGLU + quant
      q3::GateUpArgs u;
      std::memset(&u, 0, sizeof(u));
      u.M = M;
      u.N = I;
      u.K = H;
      u.group = 256;
      u.a = h8;
      u.lda = H;
      u.as = hs;
      u.ldas = H / 256;
      u.wg = lp.wg;
      u.wu = lp.wu;
      u.ldw = H;
      u.wgs = lp.wgs;
      u.wus = lp.wus;
      u.ws_stride = 1;
      u.s8 = s8;
      u.lds8 = I;
      u.ss = ss;
      u.ldss = I / 256;
      u.ss_col = 1;
      Q3_HIP(q3::launch_gate_up(u, s));
    }
    if (gv) {  // down projection + residual
      q3::GemvArgs g = gemv_args(M, I, 256);
      g.a = s8;
      g.lda = I;
      g.as = ss;
      g.ldas = I / 256;
      g.nseg = 1;
      g.seg[0] = gemv_seg(0, H, q3::EPI_ADD, lp.wd, lp.wds, x, H);
      Q3_HIP(q3::launch_gemv(g, s));
    } else {
      q3::GemmArgs g = gemm_args(M, H, I, 256, s8, ss, lp.wd, lp.wds);
      g.epi = q3::EPI_ADD;
      g.out = x;
      g.ldo = H;
      Q3_HIP(q3::launch_gemm(g, s));
    }
  }
  // final RMSNorm + quant, lm_head argmax per row (main_big.cpp:264-290)
  Q3_TRY(rows(1, at<const float>(m, y.kNF)));
  {
    q3::GemmArgs g = gemm_args(M, V, H, 256, h8, hs, at<const int8_t>(m, y.kLM),
                               at<const float>(m, y.kLM + static_cast<int64_t>(V) * H));
    g.epi = q3::EPI_ARGMAX;
    g.keys = m->bkeys;
    g.keys_ld = m->bkeys_ld;
    Q3_HIP(q3::launch_gemm(g, s));
    Q3_HIP(q3::launch_argmax_finish(m->bkeys, m->bkeys_ld, V / 128, M, m->bbest, 1, out_ids, 1,
                                    /*init=*/1, out_ids, nullptr, 0, s, /*ids_per_row=*/1));
  }
  return Q3_OK;
}

extern "C" int q3_model_set_kernel_timing(q3_model *m, uint32_t mask) {
  if (!m) return Q3_ERR_ARG;
  if (mask >> Q3_KT_COUNT) return Q3_ERR_ARG;
  Q3_HIP(hipStreamSynchronize(m->stream));
  m->kt_mask = mask;
  for (int c = 0; c < Q3_KT_COUNT; ++c) {
    m->kt_used[c] = 0;
    m->kt_ms[c] = 0.0;
    m->kt_n[c] = 0;
  }
  return Q3_OK;
}

extern "C" int q3_model_kernel_time(q3_model *m, int kclass, double *total_ms, uint32_t *launches) {
  if (!m || kclass < 0 || kclass >= Q3_KT_COUNT || !total_ms || !launches) return Q3_ERR_ARG;
  const int rc = kt_fold(m, kclass);
  if (rc != Q3_OK) return rc;
  *total_ms = m->kt_ms[kclass];
  *launches = m->kt_n[kclass];
  return Q3_OK;
}

extern "C" int q3_model_repack(q3_model *m) {
  if (!m) return Q3_ERR_ARG;
  if (!m->packed) return Q3_OK;
  return repack_weights(m);
}

extern "C" int q3_model_fused_status(q3_model *m, uint32_t *fused, uint32_t *gave_up) {
  if (!m || !fused || !gave_up) return Q3_ERR_ARG;
  *fused = (m->qkvfuse ? 1u : 0u) | (m->qkvfuse && m->merge ? 2u : 0u);
  Q3_HIP(hipStreamSynchronize(m->stream));
  Q3_HIP(hipMemcpy(gave_up, m->xerr, sizeof(uint32_t), hipMemcpyDeviceToHost));
  return Q3_OK;
}

extern "C" int q3_model_set_page_table(q3_model *m, const uint16_t *table, uint32_t n) {
  if (!m || !table || n != m->n_pages) return Q3_ERR_ARG;
  for (uint32_t i = 0; i < n; ++i)
    if (table[i] >= m->n_pages) return Q3_ERR_RANGE;
  Q3_HIP(hipMemcpyAsync(m->ptab, table, sizeof(uint16_t) * n, hipMemcpyHostToDevice, m->stream));
  Q3_HIP(hipStreamSynchronize(m->stream));
  m->htab.assign(table, table + n);
  ++m->tab_version;
  return Q3_OK;
}

extern "C" int q3_model_info(const q3_model *m, q3_layout *lay, void **blob, void **stream) {
  if (!m) return Q3_ERR_ARG;
  if (lay) *lay = m->lay;
  if (blob) *blob = m->blob;
  if (stream) *stream = m->stream;
  return Q3_OK;
}

extern "C" int q3_forward_chunk(q3_model *m, uint32_t pos, uint32_t rows, int lm_out,
                                int optimize_tail) {
  if (!m) return Q3_ERR_ARG;
  return forward_chunk_impl(m, pos, rows, lm_out, optimize_tail, nullptr);
}

extern "C" int q3_generate(q3_model *m) {
  if (!m) return Q3_ERR_ARG;
  const q3_layout &y = m->lay;
  int32_t ctrl[4];
  Q3_HIP(hipMemcpyAsync(ctrl, m->blob + y.kCTRL, sizeof(ctrl), hipMemcpyDeviceToHost, m->stream));
  Q3_HIP(hipStreamSynchronize(m->stream));
  const int32_t n_prompt = ctrl[0], n_gen = ctrl[1], mode = ctrl[3];
  if (mode < 0 || mode > 1) return Q3_ERR_MODE;  // main_big.cpp:346-348
  if (n_prompt < 0 || n_gen < 0 || static_cast<int64_t>(n_prompt) + n_gen > y.max_seq)
    return Q3_ERR_RANGE;
  const bool fused = (mode == 0);
  const uint32_t total = static_cast<uint32_t>(n_prompt + n_gen);
  const uint32_t np = static_cast<uint32_t>(n_prompt);
  int32_t *ids = at<int32_t>(m, y.kIDS);
  // one forward of the loop: a prompt chunk, or a one-row decode step
  auto step = [&](uint32_t pos, uint32_t *next) {
    const uint32_t rows = (pos < np) ? ((np - pos < y.seq) ? np - pos : y.seq) : 1;
    const bool need_out = (pos + rows >= np);
    const int lm_out = need_out ? (fused ? Q3_LM_ARGMAX : Q3_LM_LOGITS) : Q3_LM_NONE;
    *next = pos + rows;
    // the id of the next token goes straight to ids[next] on the device
    int32_t *id_dst = (need_out && *next >= np && *next < total) ? ids + *next : nullptr;
    return forward_chunk_impl(m, pos, rows, lm_out, fused ? 1 : 0, id_dst);
  };
  // the decode steps run as one graph when the stream can capture (not the
  // null stream) and no launch is being timed
  const bool graph = m->dgraph_on && m->stream && m->kt_mask == 0 && total > np;
  uint32_t pos = 0;
  while (pos < total && !(graph && pos >= np)) {
    uint32_t next = 0;
    const int rc = step(pos, &next);
    if (rc != Q3_OK) return rc;
    pos = next;
  }
  if (pos >= total) return Q3_OK;
  const bool same = m->dgraph && m->dg_key[0] == n_prompt && m->dg_key[1] == n_gen &&
                    m->dg_key[2] == mode && m->dg_tab_version == m->tab_version;
  if (!same) {
    if (m->dgraph) (void)hipGraphExecDestroy(m->dgraph);
    m->dgraph = nullptr;
    Q3_HIP(hipStreamBeginCapture(m->stream, hipStreamCaptureModeRelaxed));
    int rc = Q3_OK;
    for (uint32_t p = pos; p < total && rc == Q3_OK;) {
      uint32_t next = 0;
      rc = step(p, &next);
      p = next;
    }
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(m->stream, &g);
    if (rc == Q3_OK && (e != hipSuccess || !g)) rc = Q3_ERR_HIP;
    if (rc == Q3_OK && hipGraphInstantiate(&m->dgraph, g, nullptr, nullptr, 0) != hipSuccess) {
      m->dgraph = nullptr;
      rc = Q3_ERR_HIP;
    }
    if (g) (void)hipGraphDestroy(g);
    if (rc != Q3_OK) return rc;
    m->dg_key[0] = n_prompt;
    m->dg_key[1] = n_gen;
    m->dg_key[2] = mode;
    m->dg_tab_version = m->tab_version;
  }
  Q3_HIP(hipGraphLaunch(m->dgraph, m->stream));
  return Q3_OK;
}

extern "C" int q3_model_close(q3_model *m) {
  if (!m) return Q3_ERR_ARG;
  int rc = Q3_OK;
  if (m->stream || m->ptab) {
    if (hipStreamSynchronize(m->stream) != hipSuccess) rc = Q3_ERR_HIP;
  }
  if (m->ptab) (void)hipFree(m->ptab);
  if (m->keys) (void)hipFree(m->keys);
  if (m->keys_ws) (void)hipFree(m->keys_ws);
  if (m->bstate) (void)hipFree(m->bstate);
  for (int i = 0; i < 2; ++i) {
    if (m->bstage[i]) (void)hipHostFree(m->bstage[i]);
    if (m->bstage_ev[i]) (void)hipEventDestroy(m->bstage_ev[i]);
  }
  if (m->bkeys) (void)hipFree(m->bkeys);
  if (m->bbest) (void)hipFree(m->bbest);
  if (m->opart) (void)hipFree(m->opart);
  if (m->xin) (void)hipFree(m->xin);
  if (m->xerr) (void)hipFree(m->xerr);
  if (m->xw) (void)hipFree(m->xw);
  if (m->dgraph) (void)hipGraphExecDestroy(m->dgraph);
  if (m->packed) (void)hipFree(m->packed);
  for (int c = 0; c < Q3_KT_COUNT; ++c)
    for (hipEvent_t e : m->kt_ev[c]) (void)hipEventDestroy(e);
  delete m;
  return rc;
}
