// Blob layout of the PQWF model image: byte offsets of every table, weight,
// activation buffer and KV-cache page pool.
//
// Restates tools/pqwf.py:95-273 (Layout.compute / header_text) so that a blob
// written here is byte-compatible with one written by tools/convert_pqwf.py
// and can be inspected with the reference's tools/compare.py.  The order and
// the sizes of the regions are part of the format, so they are kept exactly;
// the 64 KiB alignment of the activation area (pqwf.py:185) included.
#include <cstdio>
#include <cstring>
#include <string>

#include "q3ops.h"

namespace {

struct Placer {
  int64_t off = 0;
  int64_t place(int64_t size) {
    const int64_t at = off;
    off += size;
    return at;
  }
};

}  // namespace

extern "C" int q3_layout_compute(uint32_t hidden, uint32_t layers,
                                 uint32_t heads, uint32_t kv_heads,
                                 uint32_t head_dim, uint32_t inter,
                                 uint32_t vocab, uint32_t seq,
                                 uint32_t max_seq, q3_layout *o) {
  if (!o || hidden == 0 || layers == 0 || heads == 0 || kv_heads == 0 ||
      head_dim == 0 || inter == 0 || vocab == 0 || seq == 0 || max_seq == 0)
    return Q3_ERR_ARG;
  if (heads % kv_heads != 0 || head_dim % 2 != 0) return Q3_ERR_ARG;
  std::memset(o, 0, sizeof(*o));
  o->hidden = hidden;
  o->layers = layers;
  o->heads = heads;
  o->kv_heads = kv_heads;
  o->head_dim = head_dim;
  o->inter = inter;
  o->vocab = vocab;
  o->seq = seq;
  o->max_seq = max_seq;
  o->half = head_dim / 2;

  const int64_t H = hidden, L = layers, HD = head_dim, I = inter, V = vocab;
  const int64_t S = seq, MS = max_seq, HALF = head_dim / 2;
  const int64_t QW = int64_t(heads) * HD, KW = int64_t(kv_heads) * HD;
  const int64_t NH = heads, NKV = kv_heads;

  Placer p;
  o->kIDS = p.place(4 * MS);  // pqwf.py:147
  o->kCTRL = p.place(16);
  o->kX = p.place(4 * S * H);
  o->kEMB = p.place(V * H + 4 * V);
  o->kLM = p.place(V * H + 4 * V);
  o->kNF = p.place(4 * H);
  o->kCOS = p.place(4 * MS * HALF);
  o->kSIN = p.place(4 * MS * HALF);

  // One layer's weights; the block repeats with kLAYERW_STRIDE (pqwf.py:156-173).
  o->kLAYERW_BASE = p.off;
  const int64_t layer_start = p.off;
  o->kLQ = p.place(QW * H);
  o->kLQ_SCALE = p.place(4 * QW);
  o->kLK = p.place(KW * H);
  o->kLK_SCALE = p.place(4 * KW);
  o->kLV = p.place(KW * H);
  o->kLV_SCALE = p.place(4 * KW);
  o->kLO = p.place(H * QW);
  o->kLO_SCALE = p.place(4 * H);
  o->kLG = p.place(I * H);
  o->kLG_SCALE = p.place(4 * I);
  o->kLU = p.place(I * H);
  o->kLU_SCALE = p.place(4 * I);
  o->kLD = p.place(H * I);
  o->kLD_SCALE = p.place(4 * H);
  o->kLAYERW_STRIDE = p.off - layer_start;
  p.off = layer_start + L * o->kLAYERW_STRIDE;

  // Norm gains [n1 | nq | nk | n2] per layer (pqwf.py:121-122, 175-181).
  o->kLAYERN_BASE = p.off;
  o->kLAYERN_STRIDE = 4 * (H + HD + HD + H);
  p.off += L * o->kLAYERN_STRIDE;
  o->kN1 = o->kLAYERN_BASE;
  o->kNQ = o->kLAYERN_BASE + 4 * H;
  o->kNK = o->kNQ + 4 * HD;
  o->kN2 = o->kNK + 4 * HD;

  o->kLOGITS = p.place(4 * S * V);
  o->kBLOCK_END = p.off;
  p.off = (p.off + 0xFFFF) & ~int64_t(0xFFFF);  // pqwf.py:185

  o->kH = p.place(4 * S * H);
  o->kH8 = p.place(S * H);
  o->kHS = p.place(4 * S * (H / 256));
  o->kQ = p.place(4 * S * QW);
  o->kK = p.place(4 * S * KW);
  o->kV = p.place(4 * S * KW);
  o->kQ8 = p.place(S * QW);
  o->kK8 = p.place(S * KW);
  o->kV8 = p.place(S * KW);
  o->kQS = p.place(4 * S * NH);
  o->kKS = p.place(4 * S * NKV);
  o->kVS = p.place(4 * S * NKV);
  o->kATTN = p.place(4 * S * QW);
  o->kO = p.place(4 * S * H);
  o->kO8 = p.place(S * QW);
  o->kOS = p.place(4 * S * NH);
  o->kG = p.place(4 * S * I);
  o->kU = p.place(4 * S * I);
  o->kSW = p.place(4 * S * I);
  o->kS8 = p.place(S * I);
  o->kSS = p.place(4 * S * (I / 256));
  o->kARGF = p.place(256);
  o->kARGI = p.place(256);

  // Per-layer KV pool: [K rows][K scales][V rows][V scales] (pqwf.py:124-135).
  const int64_t kv_scale_off = MS * KW;
  const int64_t kv_scale_bytes = 4 * MS * NKV;
  o->kKV_BASE = p.off;
  o->kKV_SOFF = kv_scale_off;
  o->kKV_VOFF = kv_scale_off + kv_scale_bytes;
  o->kKV_STRIDE = 2 * (kv_scale_off + kv_scale_bytes);
  p.off += L * o->kKV_STRIDE;
  o->kSCRATCH_END = p.off;
  return Q3_OK;
}

extern "C" int q3_layout_header_text(const q3_layout *lay, char *buf,
                                     size_t cap) {
  if (!lay) return Q3_ERR_ARG;
  std::string s = "#pragma once\nnamespace mb {\n";
  auto ci = [&](const char *name, long v) {
    s += "inline constexpr int ";
    s += name;
    s += " = " + std::to_string(v) + ";\n";
  };
  auto cl = [&](const char *name, int64_t v) {
    s += "inline constexpr long ";
    s += name;
    s += " = " + std::to_string(static_cast<long long>(v)) + ";\n";
  };
  ci("kHidden", lay->hidden);
  ci("kLayers", lay->layers);
  ci("kHeads", lay->heads);
  ci("kKvHeads", lay->kv_heads);
  ci("kHeadDim", lay->head_dim);
  ci("kInter", lay->inter);
  ci("kVocab", lay->vocab);
  ci("kSeq", lay->seq);
  ci("kMaxSeq", lay->max_seq);
  ci("kHalf", lay->half);
#define Q3_HDR(name) cl(#name, lay->name)
  Q3_HDR(kIDS); Q3_HDR(kCTRL); Q3_HDR(kX); Q3_HDR(kEMB); Q3_HDR(kLM);
  Q3_HDR(kNF); Q3_HDR(kCOS); Q3_HDR(kSIN);
  Q3_HDR(kLAYERW_BASE); Q3_HDR(kLAYERW_STRIDE);
  Q3_HDR(kLQ); Q3_HDR(kLQ_SCALE); Q3_HDR(kLK); Q3_HDR(kLK_SCALE);
  Q3_HDR(kLV); Q3_HDR(kLV_SCALE); Q3_HDR(kLO); Q3_HDR(kLO_SCALE);
  Q3_HDR(kLG); Q3_HDR(kLG_SCALE); Q3_HDR(kLU); Q3_HDR(kLU_SCALE);
  Q3_HDR(kLD); Q3_HDR(kLD_SCALE);
  Q3_HDR(kLAYERN_BASE); Q3_HDR(kLAYERN_STRIDE);
  Q3_HDR(kN1); Q3_HDR(kNQ); Q3_HDR(kNK); Q3_HDR(kN2);
  Q3_HDR(kLOGITS); Q3_HDR(kBLOCK_END);
  Q3_HDR(kH); Q3_HDR(kH8); Q3_HDR(kHS); Q3_HDR(kQ); Q3_HDR(kK); Q3_HDR(kV);
  Q3_HDR(kQ8); Q3_HDR(kK8); Q3_HDR(kV8);
  Q3_HDR(kQS); Q3_HDR(kKS); Q3_HDR(kVS); Q3_HDR(kATTN); Q3_HDR(kO);
  Q3_HDR(kO8); Q3_HDR(kOS);
  Q3_HDR(kG); Q3_HDR(kU); Q3_HDR(kSW); Q3_HDR(kS8); Q3_HDR(kSS);
  Q3_HDR(kARGF); Q3_HDR(kARGI);
  Q3_HDR(kKV_BASE); Q3_HDR(kKV_STRIDE); Q3_HDR(kKV_VOFF); Q3_HDR(kKV_SOFF);
  Q3_HDR(kSCRATCH_END);
#undef Q3_HDR
  s += "}\n";
  if (buf && cap > 0) {
    const size_t n = s.size() < cap - 1 ? s.size() : cap - 1;
    std::memcpy(buf, s.data(), n);
    buf[n] = '\0';
  }
  return static_cast<int>(s.size());
}
