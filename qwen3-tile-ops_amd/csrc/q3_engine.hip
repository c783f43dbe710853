// Host scheduling core of the continuous-batching engine (the host engine of
// tools/engine.py:81-250, re-expressed over the device model):
//
//  * a pool of physical KV pages, handed out from the top of a free stack
//    and pushed back on release (the reference's assignment order), with a
//    per-page owner array instead of a used-set;
//  * request records in admission order (prompt length, tokens fed,
//    tokens generated, limit, state, page list);
//  * batch building: walk the records in order; a request still in its
//    prompt contributes one chunk of up to 32 rows, a decoding request one
//    row; a request whose pages cannot be found waits for a later batch; a
//    request at its limit is finished on the spot;
//  * commit: the sampled ids of a batch advance the records (a stop id or
//    the limit finishes a request and frees its pages);
//  * the device step: prefill chunks and rows whose logits the host needs
//    run q3_forward_chunk over the request's own page table; greedy decode
//    rows of a batch share q3_decode_batch launches (argmax on the device).
//
// Everything except q3_sched_run is host-only integer bookkeeping.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <new>
#include <vector>

#include "q3ops.h"

namespace {

constexpr uint32_t kChunkRows = 32;  // rows of one prefill chunk (tools/engine.py:175)
constexpr int32_t kNoOwner = -1;   // on the free stack
constexpr int32_t kDetached = -2;  // taken by q3_sched_alloc_page for no record

struct Record {
  uint32_t n_prompt = 0;
  uint32_t n_fed = 0;
  uint32_t n_gen = 0;
  uint32_t max_new = 0;
  int32_t state = Q3_REQ_WAITING;
  std::vector<uint32_t> pages;
};

}  // namespace

struct q3_sched {
  uint32_t num_pages = 0, page_tokens = 0;
  std::vector<uint32_t> free_stack;  // top = back
  std::vector<int32_t> owner;        // page -> slot, kNoOwner or kDetached
  std::vector<Record> recs;          // admission order; slot = index
  // device step scratch (q3_sched_run), allocated on first use
  int32_t *d_ids = nullptr, *d_out = nullptr;
  uint32_t d_cap = 0;
  std::vector<uint16_t> tab;         // one page table row (model's pool size)
};

namespace {

bool valid_slot(const q3_sched *s, int32_t slot) {
  return s && slot >= 0 && static_cast<size_t>(slot) < s->recs.size();
}

// Pages for the first n_tokens of the record; false when the pool runs dry
// (the pages found so far stay with the record).
bool cover(q3_sched *s, int32_t slot, uint32_t n_tokens) {
  Record &r = s->recs[slot];
  const size_t need = (static_cast<size_t>(n_tokens) + s->page_tokens - 1) / s->page_tokens;
  while (r.pages.size() < need) {
    if (s->free_stack.empty()) return false;
    const uint32_t p = s->free_stack.back();
    s->free_stack.pop_back();
    s->owner[p] = slot;
    r.pages.push_back(p);
  }
  return true;
}

void give_back(q3_sched *s, int32_t slot) {
  Record &r = s->recs[slot];
  for (uint32_t p : r.pages) {
    if (s->owner[p] != slot) continue;  // already returned
    s->owner[p] = kNoOwner;
    s->free_stack.push_back(p);
  }
  r.pages.clear();
}

void close_record(q3_sched *s, int32_t slot) {
  Record &r = s->recs[slot];
  if (r.state == Q3_REQ_FINISHED) return;
  r.state = Q3_REQ_FINISHED;
  give_back(s, slot);
}

}  // namespace

extern "C" {

int q3_sched_create(uint32_t num_pages, uint32_t page_tokens, q3_sched **out) {
  if (!out || page_tokens == 0) return Q3_ERR_ARG;
  *out = nullptr;
  q3_sched *s = new (std::nothrow) q3_sched();
  if (!s) return Q3_ERR_ARG;
  s->num_pages = num_pages;
  s->page_tokens = page_tokens;
  s->free_stack.resize(num_pages);
  for (uint32_t i = 0; i < num_pages; ++i) s->free_stack[i] = i;
  s->owner.assign(num_pages, kNoOwner);
  *out = s;
  return Q3_OK;
}

int q3_sched_destroy(q3_sched *s) {
  if (!s) return Q3_ERR_ARG;
  if (s->d_ids) (void)hipFree(s->d_ids);
  if (s->d_out) (void)hipFree(s->d_out);
  delete s;
  return Q3_OK;
}

int q3_sched_add(q3_sched *s, uint32_t n_prompt, uint32_t max_new, int32_t *slot) {
  if (!s || !slot) return Q3_ERR_ARG;
  Record r;
  r.n_prompt = n_prompt;
  r.max_new = max_new;
  s->recs.push_back(std::move(r));
  *slot = static_cast<int32_t>(s->recs.size() - 1);
  return Q3_OK;
}

int q3_sched_get(const q3_sched *s, int32_t slot, q3_sched_req *out) {
  if (!valid_slot(s, slot) || !out) return Q3_ERR_ARG;
  const Record &r = s->recs[slot];
  out->n_prompt = r.n_prompt;
  out->n_fed = r.n_fed;
  out->n_gen = r.n_gen;
  out->max_new = r.max_new;
  out->state = r.state;
  out->n_pages = static_cast<uint32_t>(r.pages.size());
  return Q3_OK;
}

int q3_sched_set(q3_sched *s, int32_t slot, const q3_sched_req *in) {
  if (!valid_slot(s, slot) || !in) return Q3_ERR_ARG;
  if (in->state < Q3_REQ_WAITING || in->state > Q3_REQ_FINISHED) return Q3_ERR_ARG;
  Record &r = s->recs[slot];
  r.n_prompt = in->n_prompt;
  r.n_fed = in->n_fed;
  r.n_gen = in->n_gen;
  r.max_new = in->max_new;
  r.state = in->state;
  return Q3_OK;
}

int q3_sched_pages(const q3_sched *s, int32_t slot, uint32_t *out, uint32_t cap, uint32_t *n) {
  if (!valid_slot(s, slot) || !n) return Q3_ERR_ARG;
  const Record &r = s->recs[slot];
  *n = static_cast<uint32_t>(r.pages.size());
  if (out) std::copy_n(r.pages.begin(), std::min<size_t>(cap, r.pages.size()), out);
  return Q3_OK;
}

int q3_sched_free_pages(const q3_sched *s, uint32_t *out, uint32_t cap, uint32_t *n) {
  if (!s || !n) return Q3_ERR_ARG;
  *n = static_cast<uint32_t>(s->free_stack.size());
  if (out) std::copy_n(s->free_stack.begin(), std::min<size_t>(cap, s->free_stack.size()), out);
  return Q3_OK;
}

int q3_sched_alloc_page(q3_sched *s, int32_t slot, int32_t *page) {
  if (!s || !page || (slot != -1 && !valid_slot(s, slot))) return Q3_ERR_ARG;
  *page = -1;
  if (s->free_stack.empty()) return Q3_OK;
  const uint32_t p = s->free_stack.back();
  s->free_stack.pop_back();
  s->owner[p] = slot >= 0 ? slot : kDetached;
  if (slot >= 0) s->recs[slot].pages.push_back(p);
  *page = static_cast<int32_t>(p);
  return Q3_OK;
}

int q3_sched_ensure(q3_sched *s, int32_t slot, uint32_t n_tokens, int32_t *ok) {
  if (!valid_slot(s, slot) || !ok) return Q3_ERR_ARG;
  *ok = cover(s, slot, n_tokens) ? 1 : 0;
  return Q3_OK;
}

int q3_sched_release(q3_sched *s, int32_t slot) {
  if (!valid_slot(s, slot)) return Q3_ERR_ARG;
  give_back(s, slot);
  return Q3_OK;
}

int q3_sched_finish(q3_sched *s, int32_t slot) {
  if (!valid_slot(s, slot)) return Q3_ERR_ARG;
  close_record(s, slot);
  return Q3_OK;
}

int q3_sched_build(q3_sched *s, uint32_t max_rows, q3_sched_item *items, uint32_t cap,
                   uint32_t *n_items, uint32_t *total_rows) {
  if (!s || !n_items || !total_rows || (cap && !items)) return Q3_ERR_ARG;
  uint32_t n = 0, rows = 0;
  for (size_t i = 0; i < s->recs.size(); ++i) {
    const int32_t slot = static_cast<int32_t>(i);
    Record &r = s->recs[i];
    if (r.state == Q3_REQ_FINISHED) continue;
    q3_sched_item it{};
    if (r.n_fed < r.n_prompt) {  // next prompt chunk
      if (rows >= max_rows) continue;
      const uint32_t chunk = std::min({kChunkRows, r.n_prompt - r.n_fed, max_rows - rows});
      if (!cover(s, slot, r.n_fed + chunk)) continue;
      it.prefill = 1;
      it.rows = chunk;
      it.needs_logits = (r.n_fed + chunk == r.n_prompt) ? 1 : 0;
    } else if (r.n_gen >= r.max_new) {  // nothing left to generate
      close_record(s, slot);
      continue;
    } else {  // one decode row: its last generated id
      if (rows >= max_rows || r.n_gen == 0 || !cover(s, slot, r.n_fed + 1)) continue;
      it.prefill = 0;
      it.rows = 1;
      it.needs_logits = 1;
    }
    if (n >= cap) return Q3_ERR_RANGE;
    it.slot = slot;
    it.row_start = rows;
    it.pos = r.n_fed;
    items[n++] = it;
    rows += it.rows;
  }
  *n_items = n;
  *total_rows = rows;
  return Q3_OK;
}

int q3_sched_commit(q3_sched *s, const q3_sched_item *items, uint32_t n, const int32_t *stop) {
  if (!s || (n && (!items || !stop))) return Q3_ERR_ARG;
  for (uint32_t i = 0; i < n; ++i)
    if (!valid_slot(s, items[i].slot)) return Q3_ERR_ARG;
  for (uint32_t i = 0; i < n; ++i) {
    Record &r = s->recs[items[i].slot];
    r.n_fed += items[i].rows;
    if (items[i].needs_logits) {
      ++r.n_gen;
      if (stop[i] || r.n_gen >= r.max_new)
        close_record(s, items[i].slot);
      else
        r.state = Q3_REQ_DECODE;
    } else if (r.n_fed < r.n_prompt) {
      r.state = Q3_REQ_PREFILL;
    }
  }
  return Q3_OK;
}

int q3_sched_finish_exhausted(q3_sched *s, uint32_t *n_finished) {
  if (!s) return Q3_ERR_ARG;
  uint32_t k = 0;
  for (size_t i = 0; i < s->recs.size(); ++i) {
    const Record &r = s->recs[i];
    if (r.state != Q3_REQ_FINISHED && r.n_fed >= r.n_prompt && r.n_gen >= r.max_new) {
      close_record(s, static_cast<int32_t>(i));
      ++k;
    }
  }
  if (n_finished) *n_finished = k;
  return Q3_OK;
}

int q3_sched_run(q3_sched *s, q3_model *m, const q3_sched_item *items, uint32_t n,
                 const int32_t *tokens, const int32_t *on_device, int32_t *out_ids,
                 float *logits, uint64_t ld_logits) {
  if (!s || !m || (n && (!items || !tokens || !on_device || !out_ids))) return Q3_ERR_ARG;
  q3_layout lay;
  void *blob_v = nullptr, *stream_v = nullptr;
  int rc = q3_model_info(m, &lay, &blob_v, &stream_v);
  if (rc != Q3_OK) return rc;
  uint8_t *blob = static_cast<uint8_t *>(blob_v);
  const hipStream_t st = static_cast<hipStream_t>(stream_v);
  const uint32_t slots = lay.max_seq / 32;
  if (s->page_tokens != 32 || s->num_pages > slots) return Q3_ERR_ARG;
  s->tab.assign(slots, 0);
  auto table_of = [&](const Record &r, uint16_t *dst) -> int {
    if (r.pages.size() > slots) return Q3_ERR_RANGE;
    std::fill(dst, dst + slots, uint16_t(0));
    for (size_t i = 0; i < r.pages.size(); ++i) {
      if (r.pages[i] >= slots) return Q3_ERR_RANGE;
      dst[i] = static_cast<uint16_t>(r.pages[i]);
    }
    return Q3_OK;
  };
  // items run as forward chunks (prefill, or the host samples their logits)
  size_t tok_off = 0;
  std::vector<uint32_t> greedy;
  std::vector<size_t> greedy_tok;
  for (uint32_t i = 0; i < n; ++i) {
    const q3_sched_item &it = items[i];
    if (!valid_slot(s, it.slot)) return Q3_ERR_ARG;
    const size_t off = tok_off;
    tok_off += it.rows;
    out_ids[i] = -1;
    if (!it.prefill && on_device[i]) {
      greedy.push_back(i);
      greedy_tok.push_back(off);
      continue;
    }
    if (it.rows > lay.seq || it.pos + it.rows > lay.max_seq) return Q3_ERR_RANGE;
    if ((rc = table_of(s->recs[it.slot], s->tab.data())) != Q3_OK) return rc;
    if ((rc = q3_model_set_page_table(m, s->tab.data(), slots)) != Q3_OK) return rc;
    if (hipMemcpyAsync(blob + lay.kIDS + 4 * static_cast<int64_t>(it.pos), tokens + off,
                       sizeof(int32_t) * it.rows, hipMemcpyHostToDevice, st) != hipSuccess)
      return Q3_ERR_HIP;
    const int lm = it.needs_logits ? Q3_LM_LOGITS : Q3_LM_NONE;
    if ((rc = q3_forward_chunk(m, it.pos, it.rows, lm, 1)) != Q3_OK) return rc;
    if (it.needs_logits) {
      if (!logits) return Q3_ERR_ARG;
      if (hipMemcpyAsync(logits + static_cast<uint64_t>(i) * ld_logits, blob + lay.kLOGITS,
                         sizeof(float) * lay.vocab, hipMemcpyDeviceToHost, st) != hipSuccess ||
          hipStreamSynchronize(st) != hipSuccess)
        return Q3_ERR_HIP;
    }
  }
  // greedy decode rows: q3_decode_batch, up to `seq` rows per call
  if (!greedy.empty()) {
    if (s->d_cap < lay.seq) {
      if (s->d_ids) (void)hipFree(s->d_ids);
      if (s->d_out) (void)hipFree(s->d_out);
      s->d_ids = s->d_out = nullptr;
      s->d_cap = 0;
      if (hipMalloc(&s->d_ids, sizeof(int32_t) * lay.seq) != hipSuccess ||
          hipMalloc(&s->d_out, sizeof(int32_t) * lay.seq) != hipSuccess)
        return Q3_ERR_HIP;
      s->d_cap = lay.seq;
    }
    std::vector<int32_t> ids, pos, got;
    std::vector<uint16_t> tables;
    for (size_t g0 = 0; g0 < greedy.size(); g0 += lay.seq) {
      const size_t cnt = std::min<size_t>(lay.seq, greedy.size() - g0);
      ids.resize(cnt);
      pos.resize(cnt);
      got.resize(cnt);
      tables.assign(cnt * slots, 0);
      for (size_t k = 0; k < cnt; ++k) {
        const q3_sched_item &it = items[greedy[g0 + k]];
        ids[k] = tokens[greedy_tok[g0 + k]];
        pos[k] = static_cast<int32_t>(it.pos);
        if ((rc = table_of(s->recs[it.slot], tables.data() + k * slots)) != Q3_OK) return rc;
      }
      if (hipMemcpyAsync(s->d_ids, ids.data(), sizeof(int32_t) * cnt, hipMemcpyHostToDevice, st) !=
          hipSuccess)
        return Q3_ERR_HIP;
      rc = q3_decode_batch(m, static_cast<uint32_t>(cnt), s->d_ids, pos.data(), tables.data(), slots,
                           s->d_out);
      if (rc != Q3_OK) return rc;
      if (hipMemcpyAsync(got.data(), s->d_out, sizeof(int32_t) * cnt, hipMemcpyDeviceToHost, st) !=
              hipSuccess ||
          hipStreamSynchronize(st) != hipSuccess)
        return Q3_ERR_HIP;
      for (size_t k = 0; k < cnt; ++k) out_ids[greedy[g0 + k]] = got[k];
    }
  }
  return hipStreamSynchronize(st) == hipSuccess ? Q3_OK : Q3_ERR_HIP;
}

}  // extern "C"
