// Decode attention (one query row per head) with the block recurrence of
// kernels/attention_gqa.h:404-547 / ref_qwen3.py:210-266, parallelised
// exactly.
//
// The reference walks 32-key blocks in order, carrying (maximum, den, res).
// Only the carried den/res updates are inherently sequential; everything
// else depends on the blocks plus the running maximum, and the running
// maximum is a prefix max of the per-block maxima.  So per chunk of up to
// CB = NW * BPW blocks:
//   phase 1 (parallel over blocks)  S_j = q8.k8^T (v_dot4_i32_i8, exact),
//                                   s = ((f32 S * ks) * qs) * qk, block max
//   phase 2 (a scan, one lane/block) nmm_j = max(nmm_{j-1}, max_j),
//                                   corr_j = exp(nmm_{j-1} - nmm_j)
//   phase 3 (parallel over blocks)  P = exp(s - nmm_j), psum_j = tree_sum(P),
//                                   P *= vs, pmax_j, P8, PV_j = f32(P8.V) * pmax_j
//   phase 4 (sequential per dim)    den = den*corr_j + psum_j,
//                                   res = res*corr_j + PV_j
// with the same rounding points as the reference, so the result is bit-equal
// to the sequential walk.  Chunks carry (maximum, den, res) like blocks do.
//
// A workgroup handles QPW query heads of one KV head (the kernel supports
// QPW = 1 and 2; with QPW = 1 the workgroups of a GQA pair each read the
// pair's K/V).  NW waves own blocks round-robin, BPW per chunk each.  The
// kernel is latency-bound, so its global loads are issued in the order they
// are needed (vector loads return in order): first the prologue's operands,
// then every K/V row and scale of the chunk; the exp table lives in LDS.
// The fused b = 1 variants and batches copy V into LDS stages and compute
// P8.V on the matrix cores (VMF below); the unfused b = 1 variant keeps V in
// registers from phase 1 to phase 3 (P8.V with v_dot4 on 4x4 byte-transposed
// V words).
//
// Optional prologue (decode fusion): the head epilogues of the new token's
// Q/K/V projection rows (kernels/norm_rope_quant.h:17-86 for Q and K,
// group_gemm.h:173-193 for V) run here, one wave per head.  They write the
// K/V page slot of position kv_len - 1 (one workgroup per KV head) and the Q
// int8 row for the record, and keep copies in LDS that the attention uses in
// place of the global K/V of that position.
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "q3_device.h"
#include "q3_gemv_pro.h"
#include "q3_kernels.h"

namespace q3 {
namespace {

constexpr int HD = 128;

// ---- P8.V on the matrix cores (the fused b = 1 variants) ----
// A block's V rows go from memory straight into an LDS stage, [32 keys][8 x
// 16 B] with 16-byte chunk c of key r at position c ^ vswz(r), so that the
// 8 keys a transposing read gathers fall on 8 different chunks.
typedef int v4i_d __attribute__((ext_vector_type(4)));
typedef int v2i_d __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2i_d *lds_v2i_ptr_d;
__device__ __forceinline__ int vswz(int key) { return (key & 3) | ((key >> 2) & 4); }

// 16 bytes per lane global -> LDS (lane l writes lds + 16 l), as inline
// assembly: the compiler does not count it among the loads in flight, so
// its waits for later loads only become stricter (loads complete in
// order), while its own global_load_lds would make it wait for every load
// before the next use of any.  A copy is issued in front of loads whose
// wait then covers it.
// (NT: a non-temporal read, for rows read once that no prefetch brought in)
template <bool NT = false>
__device__ __forceinline__ void lds_copy16(const void *src, const void *lds) {
  const uint32_t m0v =
      __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(to_lds(lds))));
  if constexpr (NT)
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src), "s"(m0v)
                 : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m0v)
                 : "memory", "m0");
}

// Byte position of key c's P8 in a block's 32-byte P8 row, so that lane L's
// 8 bytes at 8 (L / 16) are the keys 16 (j / 4) + 4 (L / 16) + j % 4,
// j = 0..7: the keys ds_read_b64_tr_b8 hands lane L of the V operand (in
// each 16-lane group, result lane i byte j is byte i % 8 of the 8 bytes
// addressed by source lane 2 j + i / 8).
__device__ __forceinline__ int p8_pos(int c) { return 8 * ((c & 15) >> 2) + (((c >> 4) << 2) | (c & 3)); }

__device__ __forceinline__ int sdot4(int a, int b, int c) {
  return __builtin_amdgcn_sdot4(a, b, c, false);
}

// The V words of one 32-key block as loaded (lane l: vw[cc] = the 4 int8
// values of dims d0..d0+3, d0 = 4 (l % 32), of key kh + cc, kh = 16 (l / 32))
// turned in place into 4x4 byte tiles transposed with v_perm_b32: afterwards
// vw[4 g + e] holds dim d0 + e of keys kh + 4 g .. kh + 4 g + 3, so that
// v_dot4_i32_i8 multiplies 4 keys at once.  It needs only the block's V, so
// the b = 1 kernel runs it for all but a wave's last block in phase 1, while
// that wave waits for its next block's K rows, instead of in the VALU-bound
// phase 3 (batches, bound by their loads, keep it in phase 3: 3.036 against
// 3.063 ms per config-4 step).
__device__ __forceinline__ void v_transpose(int (&vw)[16]) {
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const uint32_t w0 = vw[4 * g], w1 = vw[4 * g + 1], w2 = vw[4 * g + 2], w3 = vw[4 * g + 3];
    const uint32_t x01l = __builtin_amdgcn_perm(w1, w0, 0x06020400u);
    const uint32_t x01h = __builtin_amdgcn_perm(w1, w0, 0x07030501u);
    const uint32_t x23l = __builtin_amdgcn_perm(w3, w2, 0x06020400u);
    const uint32_t x23h = __builtin_amdgcn_perm(w3, w2, 0x07030501u);
    vw[4 * g] = static_cast<int>(__builtin_amdgcn_perm(x23l, x01l, 0x05040100u));
    vw[4 * g + 1] = static_cast<int>(__builtin_amdgcn_perm(x23h, x01h, 0x05040100u));
    vw[4 * g + 2] = static_cast<int>(__builtin_amdgcn_perm(x23l, x01l, 0x07060302u));
    vw[4 * g + 3] = static_cast<int>(__builtin_amdgcn_perm(x23h, x01h, 0x07060302u));
  }
}

// P8.V of one 32-key block for the lanes' layout of phase 3, on V words
// transposed by v_transpose: p8 of key c for head h sits in lane
// 32 (h + HB) + c, and acc[h][e] += sum over the lane's 16 keys of
// p8[h][key] * v[key][d0+e], exact in int32.  The P8 bytes of 4 consecutive
// keys are packed with DPP quad broadcasts.
template <int QPW, int HB = 0>
__device__ __forceinline__ void pv_dot(const int (&vt)[16], int p8, int lane, int (&acc)[QPW][4]) {
  const int b = p8 & 0xff;
  const int q0 = __builtin_amdgcn_mov_dpp(b, 0x00, 0xf, 0xf, false);  // quad lane 0
  const int q1 = __builtin_amdgcn_mov_dpp(b, 0x55, 0xf, 0xf, false);  // quad lane 1
  const int q2 = __builtin_amdgcn_mov_dpp(b, 0xaa, 0xf, 0xf, false);
  const int q3 = __builtin_amdgcn_mov_dpp(b, 0xff, 0xf, 0xf, false);
  const int packed = q0 | (q1 << 8) | (q2 << 16) | (q3 << 24);  // keys 4q..4q+3
  const bool upper = lane >= 32;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int r[4] = {vt[4 * g], vt[4 * g + 1], vt[4 * g + 2], vt[4 * g + 3]};
#pragma unroll
    for (int h = 0; h < QPW; ++h) {
      const int pa = __builtin_amdgcn_readlane(packed, 32 * (h + HB) + 4 * g);
      const int pb = __builtin_amdgcn_readlane(packed, 32 * (h + HB) + 16 + 4 * g);
      const int pk = upper ? pb : pa;
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[h][e] = sdot4(pk, r[e], acc[h][e]);
    }
  }
}

template <int QPW, int CB>
struct Smem {
  uint64_t tab[32];
  int8_t q8[QPW][HD];
  float qs[QPW];
  int8_t knew[HD], vnew[HD];
  float ksnew, vsnew;
  float s[QPW][CB * 32];  // scores of the chunk
  float bmax[QPW][CB];
  float corr[QPW][CB], psum[QPW][CB];
  float pv[QPW][CB][HD];  // f32(P8.V) * pmax per block
  float absmax[QPW][2];
  int8_t o8[HD];  // OFUSE: the head's quantised output and its scale
  float os;
};

// OFUSE: the O projection's row scales (shared by every head)
constexpr int kORowsMax = 1024;
template <bool OFUSE>
struct SmemO {
  float wos[OFUSE ? kORowsMax : 1];
};

// OFUSE (QPW = 1): the head's slice of the O projection weights, rows
// n = 96 i + tid / 8 (i < kOPieces), 16 bytes (columns 16 (tid % 8) ..) of
// the head's 128 per thread; up to kORowsMax rows.
constexpr int kOPieces = 11;
// pieces loaded after phase 1 of a chunk; the rest after its phase 3 (V rows
// consumed): all of them at once do not fit the register file
constexpr int kOPiecesEarly = 6;

// One step of an inclusive max-scan within rows of 16 lanes (DPP
// row_shr:D): lanes D.. of a row combine the value D lanes down, the first D
// keep their own (the disabled lanes of the move return the old value).
template <int D>
__device__ __forceinline__ float row_shr_max(float m) {
  const float o = __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(m), __float_as_int(m), 0x110 + D, 0xf, 0xf, false));
  return (o > m) ? o : m;
}

// The kernel arguments the first K/V loads depend on, read together and
// pinned in SGPRs in the fused variants: otherwise the K/V addresses wait on
// a chain of scalar-cache round trips (each read issued where it is first
// needed).
struct HotArgs {
  uint32_t kv_len, page_tokens, new_page;
  const int8_t *k, *v;
  const float *ks, *vs;
  int64_t page_bytes, row_bytes, scale_page_bytes, scale_row_bytes;
  const float *fq, *fk, *fv, *nq, *nk, *cos_row, *sin_row;
  const float *wos;
  int o_rows;
};

template <bool PIN, bool OFUSE>
__device__ __forceinline__ HotArgs hot_args(const AttnArgs &a) {
  HotArgs h;
  h.kv_len = a.kv_len;
  h.page_tokens = a.page_tokens;
  h.new_page = a.new_page;
  h.k = a.k;
  h.v = a.v;
  h.ks = a.ks;
  h.vs = a.vs;
  h.page_bytes = a.page_bytes;
  h.row_bytes = a.row_bytes;
  h.scale_page_bytes = a.scale_page_bytes;
  h.scale_row_bytes = a.scale_row_bytes;
  h.fq = a.fq;
  h.fk = a.fk;
  h.fv = a.fv;
  h.nq = a.nq;
  h.nk = a.nk;
  h.cos_row = a.cos_row;
  h.sin_row = a.sin_row;
  h.wos = OFUSE ? a.wos : nullptr;
  h.o_rows = OFUSE ? a.o_rows : 0;
  if constexpr (PIN) {
    h.kv_len = pin_sgpr(h.kv_len);
    h.page_tokens = pin_sgpr(h.page_tokens);
    h.new_page = pin_sgpr(h.new_page);
    h.k = pin_sgpr(h.k);
    h.v = pin_sgpr(h.v);
    h.ks = pin_sgpr(h.ks);
    h.vs = pin_sgpr(h.vs);
    h.page_bytes = pin_sgpr(h.page_bytes);
    h.row_bytes = pin_sgpr(h.row_bytes);
    h.scale_page_bytes = pin_sgpr(h.scale_page_bytes);
    h.scale_row_bytes = pin_sgpr(h.scale_row_bytes);
    h.fq = pin_sgpr(h.fq);
    h.fk = pin_sgpr(h.fk);
    h.fv = pin_sgpr(h.fv);
    h.nq = pin_sgpr(h.nq);
    h.nk = pin_sgpr(h.nk);
    h.cos_row = pin_sgpr(h.cos_row);
    h.sin_row = pin_sgpr(h.sin_row);
    if constexpr (OFUSE) {
      h.wos = pin_sgpr(h.wos);
      h.o_rows = pin_sgpr(h.o_rows);
    }
  }
  return h;
}

// Operands of the fused head epilogue of one wave (see fused_load).
struct FusedRegs {
  float t0, t1, w0, w1, c, s;
  uint32_t page;  // K/V waves of the writing workgroup: page of the new token
};

// wave 0: K head kvh, wave 1: V head kvh, waves 2..: query heads qh0 + h.
// Every wave issues the same six loads (waves past the heads repeat wave
// 0's, the V wave loads gains it does not use): with a fixed count the
// compiler's waits after them stay exact.
// POLL: the projection rows come from the exchange words instead (polled in
// the prologue, attn_poll_rows), so only the gains and RoPE rows load here.
template <int QPW, bool POLL = false>
__device__ __forceinline__ void fused_load(const HotArgs &a, int kvh, int qh0, int wave, int lane,
                                           FusedRegs &r) {
  const int w = wave < 2 + QPW ? wave : 0;
  if constexpr (!POLL) {
    const float *src = w == 0 ? a.fk + kvh * HD : w == 1 ? a.fv + kvh * HD : a.fq + (qh0 + w - 2) * HD;
    r.t0 = src[lane];
    r.t1 = src[lane + 64];
  }
  const float *nw = w == 0 ? a.nk : a.nq;
  r.w0 = nw[lane];
  r.w1 = nw[lane + 64];
  r.c = a.cos_row[lane];
  r.s = a.sin_row[lane];
  r.page = a.new_page;
}

template <int QPW, class SM>
__device__ void fused_compute(const AttnArgs &a, const HotArgs &h, SM &sm, FusedRegs r, int kvh, int qh0,
                              bool kv_writer, int wave, int lane) {
  if (wave >= 2 + QPW) return;
  const uint32_t t = h.kv_len - 1;  // the new token
  float t0 = r.t0, t1 = r.t1;
  if (wave != 1) head_norm_rope_regs(t0, t1, r.w0, r.w1, r.c, r.s, a.inv_hd, true);
  const float mx = max64(fmaxf(fabsf(t0), fabsf(t1)));
  const float scale = __fmul_rn(mx, inv127());
  const int8_t q0 = static_cast<int8_t>(quant1(t0, scale));
  const int8_t q1 = static_cast<int8_t>(quant1(t1, scale));
  int8_t *lrow;
  float *lsp;
  if (wave < 2) {
    lrow = wave == 0 ? sm.knew : sm.vnew;
    lsp = wave == 0 ? &sm.ksnew : &sm.vsnew;
    if (kv_writer) {
      const uint32_t page = r.page;
      const uint32_t slot = t % h.page_tokens;
      int8_t *row8 = const_cast<int8_t *>(wave == 0 ? h.k : h.v) + page * h.page_bytes +
                     slot * h.row_bytes + kvh * HD;
      float *sp = reinterpret_cast<float *>(reinterpret_cast<int8_t *>(const_cast<float *>(wave == 0 ? h.ks : h.vs)) +
                                            page * h.scale_page_bytes + slot * h.scale_row_bytes) + kvh;
      row8[lane] = q0;
      row8[lane + 64] = q1;
      if (lane == 0) *sp = scale;
    }
  } else {
    const int qh = qh0 + wave - 2;
    int8_t *row8 = const_cast<int8_t *>(a.q8) + qh * HD;
    row8[lane] = q0;
    row8[lane + 64] = q1;
    if (lane == 0) const_cast<float *>(a.qs)[qh * a.qs_col] = scale;
    lrow = sm.q8[wave - 2];
    lsp = &sm.qs[wave - 2];
  }
  lrow[lane] = q0;
  lrow[lane + 64] = q1;
  if (lane == 0) *lsp = scale;
}

// Workgroup w of the pf_wgs prefetch workgroups reads 16 B per thread from
// every (nthreads * 16)-byte chunk w, w + pf_wgs, ... of each range.  Four
// loads are in flight per thread; the values only feed an empty asm
// statement so that the loads are kept.  With pf_kv_heads, the last four
// ranges are the next attention's K/V pools and scale pools instead, read
// page by page through the page table (AttnArgs::pf_kv_heads): the
// workgroup has grid id first + w, on XCD (first + w) % 8, and the XCD's
// prefetch workgroups take whole pages in turn, reading of each the
// HD-byte slices of the XCD's nh query heads' kv heads (every slice for
// nh <= 2) in its K and V pool and its scale rows.
__device__ void prefetch_ranges(const AttnArgs &a, int w, int first) {
  const int nkv = a.pf_kv_heads > 0 ? 4 : 0;
  for (int r = 0; r < a.pf_n - nkv; ++r) {
    const int8_t *base = a.pf[r];
    const int64_t n16 = a.pf_bytes[r] / 16;
    int64_t i = static_cast<int64_t>(w) * blockDim.x + threadIdx.x;
    const int64_t stride = static_cast<int64_t>(a.pf_wgs) * blockDim.x;
    for (; i + 3 * stride < n16; i += 4 * stride) {
      const int4 v0 = reinterpret_cast<const int4 *>(base)[i];
      const int4 v1 = reinterpret_cast<const int4 *>(base)[i + stride];
      const int4 v2 = reinterpret_cast<const int4 *>(base)[i + 2 * stride];
      const int4 v3 = reinterpret_cast<const int4 *>(base)[i + 3 * stride];
      asm volatile("" ::"v"(v0.x), "v"(v1.x), "v"(v2.x), "v"(v3.x));
    }
    for (; i < n16; i += stride) {
      const int4 v0 = reinterpret_cast<const int4 *>(base)[i];
      asm volatile("" ::"v"(v0.x));
    }
  }
  if (nkv == 0 || a.pf_n < nkv || a.pf_pages <= 0) return;
  const int xcd = (first + w) % 8;
  const int w0 = ((xcd - first) % 8 + 8) % 8;  // first prefetch workgroup on this XCD
  const int nsub = (a.pf_wgs - w0 + 7) / 8;
  const int sub = (w - w0) / 8;
  const int nh = (a.pf_kv_heads - xcd + 7) / 8;
  const int grp = a.pf_kv_heads / a.kv_heads;
  if (nh <= 0 || grp <= 0) return;
  const int T = static_cast<int>(blockDim.x);
  const int t = static_cast<int>(threadIdx.x);
  // whole pages per workgroup (page sub, sub + nsub, ...): the page id is
  // read once per page; a page's K and V slices (page_tokens rows x nh
  // slices x 8 chunks of 16 bytes each) and its scale rows spread over the
  // threads
  const int per_page = static_cast<int>(a.page_tokens) * nh * 8;
  const int sp16 = static_cast<int>(a.scale_page_bytes / 16);
  const int8_t *kp = a.pf[a.pf_n - 4], *vp = a.pf[a.pf_n - 3];
  const int8_t *ksp = a.pf[a.pf_n - 2], *vsp = a.pf[a.pf_n - 1];
  for (int page = sub; page < a.pf_pages; page += nsub) {
    const int64_t phys = a.pf_table[page];
    for (int i = t; i < per_page; i += T) {
      const int row = i / (nh * 8), slice = (i >> 3) % nh;
      const int kvh = (xcd + 8 * slice) / grp;
      const int64_t off = phys * a.page_bytes + static_cast<int64_t>(row) * a.row_bytes + kvh * HD + 16 * (i & 7);
      const int4 v0 = *reinterpret_cast<const int4 *>(kp + off);
      const int4 v1 = *reinterpret_cast<const int4 *>(vp + off);
      asm volatile("" ::"v"(v0.x), "v"(v1.x));
    }
    for (int i = t; i < sp16; i += T) {
      const int64_t off = phys * a.scale_page_bytes + 16 * i;
      const int4 v0 = *reinterpret_cast<const int4 *>(ksp + off);
      const int4 v1 = *reinterpret_cast<const int4 *>(vsp + off);
      asm volatile("" ::"v"(v0.x), "v"(v1.x));
    }
  }
}

// POLL (fused Q|K|V + attention launch): the K, V and Q waves of the
// prologue take the new token's projection rows from AttnArgs::xin, polling
// until the GEMV workgroups of the same launch have stored them, and clear
// them for the next launch.  Every word has this one reader (xload /
// xstore, q3_device.h).

template <int QPW>
__device__ __forceinline__ void attn_poll_rows(const AttnArgs &a, int qh0, int wave, int lane, FusedRegs &r) {
  if (wave >= 2 + QPW) return;
  // wave 0: K, wave 1: V, waves 2..: Q, of query head qh0 + (wave - 2)
  const int sec = wave == 0 ? 1 : wave == 1 ? 2 : 0;
  const int qh = qh0 + (wave >= 2 ? wave - 2 : 0);
  unsigned long long *src = a.xin + (static_cast<int64_t>(sec) * a.heads + qh) * HD;
  unsigned long long w0 = 0, w1 = 0;
  for (int it = 0;; ++it) {
    w0 = xload(src + lane);
    w1 = xload(src + lane + 64);
    if (__all((w0 >> 32) == 1u && (w1 >> 32) == 1u)) break;
    if (it == kPollLimit) {
      if (lane == 0) __hip_atomic_store(a.xerr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
  }
  r.t0 = __uint_as_float(static_cast<uint32_t>(w0));
  r.t1 = __uint_as_float(static_cast<uint32_t>(w1));
  xstore(src + lane, 0ull);
  xstore(src + lane + 64, 0ull);
}

// FUSE: the head epilogues run in the prologue (a.fuse_heads); a template
// parameter rather than a branch so that both variants issue a fixed number
// of loads.  OFUSE (with FUSE, QPW = 1): the O projection partials of the
// head (AttnArgs::opart) are computed after the epilogue.  (bx, by): the
// workgroup's head group and sequence.
template <int QPW, int NW, int BPW, bool FUSE, bool OFUSE = false, bool POLL = false>
__device__ __forceinline__ void attn_decode_body(const AttnArgs &a, int bx, int by) {
  constexpr int CB = NW * BPW;
  static_assert(!OFUSE || (FUSE && QPW == 1), "O projection fusion: one head per workgroup");
  static_assert(!POLL || OFUSE, "polled projection rows: the fused b = 1 variant");
  __shared__ __align__(16) Smem<QPW, CB> sm;
  __shared__ __align__(16) SmemO<OFUSE> smo;
  // VMF (the fused b = 1 variants, one query head): V through LDS stages
  // and P8.V as v_mfma_i32_16x16x32_i8 with P8 (the query row, replicated
  // over the 16 rows) as A and the V rows of a 16-dim tile, read with
  // ds_read_b64_tr_b8, as B: integer sums, exact like the v_dot4 form.
  // (these launches hold one 12-wave workgroup per CU by registers, so the
  // stages' LDS does not cost residency)
  // Batches (QPW = 2) the same, with the two heads' P8 in the even and odd
  // A rows, so that one set of products serves both heads; their 48 KiB of
  // stages still let two 4-wave workgroups share a CU, as their registers
  // do.
  constexpr bool VMF = FUSE || QPW == 2;
  __shared__ __align__(16) int8_t vst[VMF ? NW * BPW * 4096 : 16];
  __shared__ __align__(16) int8_t p8s[VMF ? NW * BPW * 32 * QPW : 16];
  // workgroup barriers: POLL waits only for LDS (s_waitcnt lgkmcnt(0)), not
  // for every outstanding vector memory operation as __syncthreads does,
  // so that the O projection's weight pieces and the page-slot stores stay
  // in flight across phases that do not read them
  auto wg_barrier = []() {
    if constexpr (POLL)
      lds_barrier();
    else
      __syncthreads();
  };
  // FUSE: the first chunk's page ids (see pgs0 below), issued before the
  // hot arguments' reads so that both are in flight together
  uint32_t pre_pg[BPW];
  if constexpr (FUSE) {
#pragma unroll
    for (int i = 0; i < BPW; ++i) pre_pg[i] = a.blk_page[wave_id() + NW * i];
  }
  const HotArgs h = hot_args<FUSE, OFUSE>(a);
  // a batch of independent sequences: sequence blockIdx.y's length, pages
  // and rows of q8/qs/o8/os
  // Batches whose row count is a multiple of 8: workgroup i runs on XCD
  // i % 8 (round-robin dispatch), so the KV-head groups of one sequence are
  // given ids with equal residues and share that XCD's L2 (the per-row scale
  // sectors and page table lines they have in common).
  // (the fused b = 1 variants never have row_pos: no test of it there)
  const bool batch = !FUSE && a.row_pos;
  if (batch && (gridDim.y & 7) == 0) {
    const int nx = static_cast<int>(gridDim.x);
    const int id = bx + nx * by;
    const int slot = id >> 3;
    by = (id & 7) + 8 * (slot / nx);
    bx = slot % nx;
  }
  const int brow = batch ? by : 0;
  const uint16_t *table = batch ? a.row_tables + brow * a.ld_table : a.table;
  const int8_t *q8_row = a.q8 + brow * a.ldq;
  const float *qs_row = a.qs + brow * a.ldqs;
  int8_t *o8_row = a.o8 + brow * a.ldo;
  float *os_row = a.os + brow * a.ldos;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = wave_id();
  // query heads per kv head: 1 or 2 (attn_decode_supported), found with a
  // compare and applied with shifts (an integer division here would be
  // scheduled first and make the first batch of argument reads wait)
  const int gshift = a.heads == a.kv_heads ? 0 : 1;
  const int qh0 = bx * QPW;
  const int kvh = qh0 >> gshift;
  const bool kv_writer = (qh0 & ((1 << gshift) - 1)) == 0;
  const uint32_t kv_len = batch ? static_cast<uint32_t>(a.row_pos[brow]) + 1 : h.kv_len;
  // one query row: pos0 = kv_len - 1, so kv_end = kv_len and the causal mask
  // only removes keys >= kv_len (attention_gqa.h:454-458)
  const int pos0 = static_cast<int>(kv_len) - 1;
  const int kv_end = static_cast<int>(kv_len);
  const int nblocks = (kv_end + 31) / 32;
  // phase 1: load e of a block reads keys 8e .. 8e + 7 whole, lane l bytes
  // kb16 .. kb16 + 15 of key 8e + kg (one load instruction covers 8 full
  // 128-byte rows rather than 32 half rows); after the reduction lanes
  // 2m, 2m + 1 hold the score of key kcl
  const int kg = lane >> 3;
  const int kb16 = 16 * (lane & 7);
  const int kcl = 8 * ((lane >> 1) & 3) + kg;
  const int d0 = 4 * (lane & 31);   // phase 3: 4 dims per lane,
  const int kh = (lane >> 5) * 16;  //   16 keys per half-wave

  const int ph = tid / HD;  // phase-4 ownership: (head, dim)
  const int pd = tid % HD;
  float res = 0.0f, den = 0.0f;
  // the running max of each head across chunks, from -FLT_MAX (attention_gqa.h:418)
  float run0 = -3.402823466e38f, run1 = -3.402823466e38f;
  int qv[QPW][4];
  float qscale[QPW];

  // The exp table into LDS from immediates (no load to wait for; first
  // read in phase 3, after barriers), the first chunk's page ids, then the
  // prologue operands.
  // (with FUSE from the arguments: a wave-uniform index, scalar loads that
  // do not wait for kv_len, since the caller repeats the last block's page
  // in the entries past it; pinned, so that they are issued with the hot
  // arguments rather than after the exp table's branch below)
  static_assert(!FUSE || CB <= 32, "first chunk's page ids come from blk_page");
  uint32_t pgs0[BPW];
#pragma unroll
  for (int i = 0; i < BPW; ++i) {
    if constexpr (FUSE) {
      pgs0[i] = pin_sgpr(pre_pg[i]);
    } else {
      const int jblk = __builtin_amdgcn_readfirstlane(min(wave + NW * i, nblocks - 1));
      pgs0[i] = table[static_cast<uint32_t>(jblk * 32) / h.page_tokens];
    }
  }
  if (tid == 0) stage_exp2_table(sm.tab);
  FusedRegs fr{};
  int8_t q8a = 0, q8b = 0;
  float qsa = 0.0f;
  constexpr int kWosPerThread = (kORowsMax + NW * 64 - 1) / (NW * 64);
  float wosr[OFUSE ? kWosPerThread : 1];
  if constexpr (FUSE) {
    fused_load<QPW, POLL>(h, kvh, qh0, wave, lane, fr);
    if constexpr (OFUSE) {
#pragma unroll
      for (int i = 0; i < kWosPerThread; ++i) wosr[i] = h.wos[min(tid + i * NW * 64, h.o_rows - 1)];
    }
  } else {
    const int qh = qh0 + min(wave, QPW - 1);  // every wave loads (fixed count)
    q8a = q8_row[qh * HD + lane];
    q8b = q8_row[qh * HD + lane + 64];
    qsa = qs_row[qh * a.qs_col];
  }
  // keep this issue order (page ids, prologue operands, then the chunk's
  // K/V): the scheduler would otherwise wait for the page ids first
  __builtin_amdgcn_sched_barrier(0);

  // OFUSE: the head's O projection weight slice (see kOPieces) in registers,
  // used after the epilogue; the row scales go to LDS in the prologue.
  // Every chunk issues the loads once its K (then V) rows are consumed, so
  // that the registers are overwritten rather than carried from chunk to
  // chunk (a conditional load would keep them live across all chunks); in
  // all but the last chunk every lane reads the same 16 bytes.
  int4 wov[OFUSE ? kOPieces : 1];
  auto issue_wo = [&](int i0, int i1, bool live) {
    const int64_t col = live ? static_cast<int64_t>(qh0) * HD + 16 * (tid & 7) : 0;
#pragma unroll
    for (int i = i0; i < i1; ++i) {
      const int n = live ? min(i * NW * 8 + tid / 8, h.o_rows - 1) : 0;
      wov[i] = *reinterpret_cast<const int4 *>(a.wo + n * a.ldwo + col);
    }
  };

  // page ids of this wave's blocks in chunk b0 (for the first chunk they are
  // issued before the prologue operands, above)
  uint32_t pgs[BPW];
#pragma unroll
  for (int i = 0; i < BPW; ++i) pgs[i] = pgs0[i];
  auto load_pages = [&](int b0) {
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
      const int jblk = min(b0 + wave + NW * i, nblocks - 1);
      pgs[i] = table[static_cast<uint32_t>(jblk * 32) / h.page_tokens];
    }
  };

  // One chunk of up to CB blocks.  The first chunk is a separate instance
  // (FIRST) so that the prologue's arithmetic stays between the chunk's load
  // issues instead of being hoisted in front of all of them.
  auto chunk = [&](const int b0, auto first_tag) {
    constexpr bool FIRST = decltype(first_tag)::value;
    const int nb = min(CB, nblocks - b0);
    // ---- issue every load of this chunk ----
    // Page ids first, then K, V and scales with no condition around any load
    // (a block past the chunk reloads the last block, a key past kv_end the
    // last key of its block): vector loads complete in order, and with a
    // fixed count the compiler waits for exactly the loads a use needs
    // instead of for all of them.  The duplicates are never used: phase 1
    // masks keys >= kv_end to -inf, so their P, P8 and P8.V terms are 0.
    if constexpr (!FIRST) load_pages(b0);
    int kw[BPW][16], vw[BPW][16];
    float kscale[BPW], vscale[BPW];
    auto issue_block = [&](int i) {
      const int j = min(b0 + wave + NW * i, nblocks - 1) * 32;
      const int last = kv_end - 1 - j;  // >= 0: the block holds key kv_end - 1 or is full
      const uint32_t page = pgs[i];
      const uint32_t slot0 = static_cast<uint32_t>(j) % h.page_tokens;
      const int8_t *kb = h.k + page * h.page_bytes + slot0 * h.row_bytes + kvh * HD;
      const int8_t *vb = h.v + page * h.page_bytes + slot0 * h.row_bytes + kvh * HD;
      const int8_t *ksb = reinterpret_cast<const int8_t *>(h.ks) + page * h.scale_page_bytes +
                          slot0 * h.scale_row_bytes;
      const int8_t *vsb = reinterpret_cast<const int8_t *>(h.vs) + page * h.scale_page_bytes +
                          slot0 * h.scale_row_bytes;
      // VMF: the V rows into the wave's stage for block i, issued in front
      // of the K rows so that the wait for those (phase 1) covers them
      if constexpr (VMF) {
        int8_t *st = vst + (wave * BPW + i) * 4096;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 8 * e + (lane >> 3);
          lds_copy16<!FUSE>(vb + min(r, last) * h.row_bytes + 16 * ((lane & 7) ^ vswz(r)), st + 1024 * e);
        }
      }
      // Without the fused prologue (batches) the K/V rows are read once, by
      // one workgroup: non-temporal loads, so that they do not push the
      // scale and page-table lines the kv heads of a sequence share out of
      // L2 (config 4: 67.2 -> 65.2 us per launch).  The b = 1 variants read
      // rows their launch's prefetch workgroups brought into L2.
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int8_t *kp = kb + min(8 * e + kg, last) * h.row_bytes + kb16;
        if constexpr (!FUSE) {
          typedef int v4i_t __attribute__((ext_vector_type(4)));
          const v4i_t v = __builtin_nontemporal_load(reinterpret_cast<const v4i_t *>(kp));
          kw[i][4 * e] = v.x;
          kw[i][4 * e + 1] = v.y;
          kw[i][4 * e + 2] = v.z;
          kw[i][4 * e + 3] = v.w;
        } else {
          const int4 v = *reinterpret_cast<const int4 *>(kp);
          kw[i][4 * e] = v.x;
          kw[i][4 * e + 1] = v.y;
          kw[i][4 * e + 2] = v.z;
          kw[i][4 * e + 3] = v.w;
        }
      }
      kscale[i] = reinterpret_cast<const float *>(ksb + min(kcl, last) * h.scale_row_bytes)[kvh];
      if constexpr (!VMF) {
#pragma unroll
        for (int cc = 0; cc < 16; ++cc) {
          const int *vp = reinterpret_cast<const int *>(vb + min(kh + cc, last) * h.row_bytes + d0);
          if constexpr (!FUSE)
            vw[i][cc] = __builtin_nontemporal_load(vp);
          else
            vw[i][cc] = *vp;
        }
      }
      vscale[i] = reinterpret_cast<const float *>(vsb + min(lane & 31, last) * h.scale_row_bytes)[kvh];
    };
    // 22 loads per block: the last block is issued after the prologue, so
    // that the prologue does not stall on a full load counter (vmcnt holds
    // 63) waiting for the first block's data
    // (POLL: all of them, the prologue waits for the projection anyway)
    constexpr int NPRE = (FIRST && POLL) ? BPW : BPW - 1;
#pragma unroll
    for (int i = 0; i < NPRE; ++i) issue_block(i);
    if constexpr (FIRST) __builtin_amdgcn_sched_barrier(0);
    if constexpr (FIRST) {
      // ---- prologue (overlaps the loads above) ----
      if constexpr (POLL) attn_poll_rows<QPW>(a, qh0, wave, lane, fr);
      if constexpr (OFUSE) {
#pragma unroll
        for (int i = 0; i < kWosPerThread; ++i)
          if (tid + i * NW * 64 < kORowsMax) smo.wos[tid + i * NW * 64] = wosr[i];
      }
      if constexpr (FUSE) {
        fused_compute<QPW>(a, h, sm, fr, kvh, qh0, kv_writer, wave, lane);
      } else if (wave < QPW) {
        sm.q8[wave][lane] = q8a;
        sm.q8[wave][lane + 64] = q8b;
        if (lane == 0) sm.qs[wave] = qsa;
      }
      wg_barrier();
#pragma unroll
      for (int h = 0; h < QPW; ++h) {
        const int *qp = reinterpret_cast<const int *>(sm.q8[h] + kb16);
#pragma unroll
        for (int e = 0; e < 4; ++e) qv[h][e] = qp[e];
        qscale[h] = sm.qs[h];
      }
    }
    if constexpr (NPRE < BPW) issue_block(BPW - 1);
    // The new token (position kv_len - 1) comes from the prologue's LDS copy
    // (FUSE), patched into a block's K words just before its scores and into
    // its V words and scales just before their first use: the select reads
    // the loaded register, so a patch waits for that load, and one placed in
    // front of phase 1 made every wave wait for all of its chunk's loads
    // (the last block's V included) before its first score.
    auto patch_k = [&](int i, int j) {
      if constexpr (FUSE) {
        const int *kn = reinterpret_cast<const int *>(sm.knew + kb16);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (j + 8 * e + kg == pos0) {
#pragma unroll
            for (int t = 0; t < 4; ++t) kw[i][4 * e + t] = kn[t];
          }
        if (j + kcl == pos0) kscale[i] = sm.ksnew;
      }
    };
    auto patch_v = [&](int i, int j) {
      if constexpr (VMF && FUSE) {
        // the new token's row into the stage (its copy has completed: the
        // block's K rows, issued after it, have been waited for)
        const int r = pos0 - j;
        if (r >= 0 && r < 32 && lane < 32) {
          int8_t *dst = vst + (wave * BPW + i) * 4096 + r * HD;
          const int g = lane >> 2, q = lane & 3;
          *reinterpret_cast<int *>(dst + 16 * (g ^ vswz(r)) + 4 * q) =
              *reinterpret_cast<const int *>(sm.vnew + 16 * g + 4 * q);
        }
        if (j + (lane & 31) == pos0) vscale[i] = sm.vsnew;
      } else if constexpr (FUSE) {
#pragma unroll
        for (int cc = 0; cc < 16; ++cc)
          if (j + kh + cc == pos0) vw[i][cc] = *reinterpret_cast<const int *>(sm.vnew + d0);
        if (j + (lane & 31) == pos0) vscale[i] = sm.vsnew;
      }
    };
    // VMF: P8.V of the wave's block i (P8 bytes already in p8s) for the 128
    // dims, f32(sum) * pmh into sm.pv[0][jb]
    const int tr_key = 16 * (((lane & 15) >> 1) >> 2) + 4 * (lane >> 4) + (((lane & 15) >> 1) & 3);
    const int tr_base = tr_key * HD + 8 * (lane & 1);
    const int tr_sw = vswz(tr_key);
    // (QPW = 2: A row m carries head m % 2's P8, so result register q of a
    // lane holds head q % 2; pmh1 is head 1's pmax)
    auto pv_mfma = [&](int i, int jb, float pmh, float pmh1 = 0.0f) {
      const int8_t *st = vst + (wave * BPW + i) * 4096;
      const int hrow = QPW == 2 ? (lane & 1) : 0;
      const long av = *reinterpret_cast<const long *>(p8s + ((wave * BPW + i) * QPW + hrow) * 32 + 8 * (lane >> 4));
      const v4i_d z = {0, 0, 0, 0};
      v4i_d c[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const v2i_d bt =
            __builtin_amdgcn_ds_read_tr8_b64_v2i32(reinterpret_cast<lds_v2i_ptr_d>(to_lds(st + tr_base + ((t ^ tr_sw) << 4))));
        long bv;
        __builtin_memcpy(&bv, &bt, sizeof(bv));
        c[t] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bv, z, 0, 0, 0);
      }
      if (lane < 16) {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          sm.pv[0][jb][16 * t + lane] = __fmul_rn(static_cast<float>(c[t][0]), pmh);
          if constexpr (QPW == 2) sm.pv[QPW - 1][jb][16 * t + lane] = __fmul_rn(static_cast<float>(c[t][1]), pmh1);
        }
      }
    };
    // ---- phase 1: scores and block maxima ----
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
      const int jb = wave + NW * i;
      if (jb >= nb) continue;
      const int j = (b0 + jb) * 32;
      const bool valid = j + kcl < kv_end;
      patch_k(i, j);
#pragma unroll
      for (int h = 0; h < QPW; ++h) {
        int p[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          p[e] = 0;
#pragma unroll
          for (int t = 0; t < 4; ++t) p[e] = sdot4(qv[h][t], kw[i][4 * e + t], p[e]);
        }
        // exact int32 sums over the 8 lanes of a key, scattered over lane
        // bits 2, 1, 0: lane l keeps keys 8 (2 b2 + {0, 1}) + kg after bit
        // 2, key 8 (2 b2 + b1) + kg = kcl after bit 1
        const bool b2 = lane & 4, b1 = lane & 2;
        int k0 = b2 ? p[2] : p[0], k1 = b2 ? p[3] : p[1];
        k0 += lane_xor<4>(b2 ? p[0] : p[2]);
        k1 += lane_xor<4>(b2 ? p[1] : p[3]);
        int acc = b1 ? k1 : k0;
        acc += lane_xor<2>(b1 ? k0 : k1);
        acc += lane_xor<1>(acc);
        float s = -INFINITY;
        if (valid) {
          s = __fmul_rn(static_cast<float>(acc), kscale[i]);
          s = __fmul_rn(s, qscale[h]);
          s = __fmul_rn(s, a.qk_scale);
          if (kcl > pos0 - j) s = -INFINITY;  // (col - row) > pos0 - j, row 0
        }
        const float bm = max64(s);
        if ((lane & 1) == 0) sm.s[h][jb * 32 + kcl] = s;
        if (lane == 0) sm.bmax[h][jb] = bm;
      }
      if (FUSE && i < BPW - 1) {
        patch_v(i, j);
        if constexpr (!VMF) v_transpose(vw[i]);
      }
    }
    if constexpr (OFUSE) {
      __builtin_amdgcn_sched_barrier(0);
      issue_wo(0, kOPiecesEarly, b0 + CB >= nblocks);
      __builtin_amdgcn_sched_barrier(0);
    }
    wg_barrier();
    // ---- phase 2: prefix max (attention_gqa.h:476-477) ----
    // nmm_j = max(run, bmax_0, ..., bmax_j), prev_j = nmm_{j-1} (run for
    // j = 0): every wave scans the block maxima itself (lanes 32 h + j hold
    // head h's block j), in registers, so no barrier follows.  Scores are
    // never NaN or -0 (an exact zero dot product gives +0 after the positive
    // scales), so the select (a > b ? a : b) is an associative max and the
    // scan equals the reference's sequential walk.
    static_assert(CB <= 32, "phase 2 scans one block per lane");
    float nmm, prev;
    {
      const int hh = lane >> 5, cc = lane & 31;
      float m = (hh < QPW && cc < nb) ? sm.bmax[hh][cc] : -INFINITY;
      m = row_shr_max<1>(m);
      m = row_shr_max<2>(m);
      m = row_shr_max<4>(m);
      m = row_shr_max<8>(m);
      const float r15 = lane_read(m, 15), r47 = lane_read(m, 47);
      const float cross = (lane & 32) ? r47 : r15;
      if (lane & 16) m = (cross > m) ? cross : m;
      const float runh = hh ? run1 : run0;
      nmm = (runh > m) ? runh : m;
      const float up = __shfl_up(nmm, 1);
      prev = cc == 0 ? runh : up;
      run0 = lane_read(nmm, nb - 1);
      if constexpr (QPW > 1) run1 = lane_read(nmm, 32 + nb - 1);
      // corr_j = exp(nmm_{j-1} - nmm_j) of every block at once, in the last
      // wave (which owns the fewest blocks while the chunk is not full):
      // one exp per lane here instead of one per block in phase 3
      if (wave == NW - 1 && hh < QPW && cc < nb) sm.corr[hh][cc] = exp_f32_le0_tab(__fsub_rn(prev, nmm), sm.tab);
    }
    // ---- phase 3: P, P8 and P8.V per block ----
    // One head per workgroup and both of the wave's blocks in the chunk: their
    // P, psum, pmax and P8 side by side in the two half-waves (block i in
    // lanes 32 i ..), one exp and reduction chain for both; the phase is
    // VALU-bound on the SIMDs that hold two-block waves.
    bool paired = false;
    if constexpr (QPW == 1 && BPW == 2) {
      if (wave + NW < nb) {
        paired = true;
        const int c = lane & 31, hi = lane >> 5;
        const int jbl = wave + NW * hi;
        patch_v(1, (b0 + wave + NW) * 32);
        const float nm0 = lane_read(nmm, wave), nm1 = lane_read(nmm, wave + NW);
        const float nmb = hi ? nm1 : nm0;
        float p = 0.0f, pv = 0.0f;
        if ((b0 + jbl) * 32 + c < kv_end) {
          p = exp_f32_le0_tab(__fsub_rn(sm.s[0][jbl * 32 + c], nmb), sm.tab);
          pv = __fmul_rn(p, hi ? vscale[1] : vscale[0]);
        }
        const float psum = tree_sum32(p);
        const float pm = __fmul_rn(max32(pv), inv127());
        const int p8 = quant1(pv, pm);
        if (c == 0) sm.psum[0][jbl] = psum;
        if constexpr (VMF) {
          p8s[(wave * BPW + hi) * 32 * QPW + p8_pos(c)] = static_cast<int8_t>(p8);
          pv_mfma(0, wave, lane_bcast<0>(pm));
          pv_mfma(1, wave + NW, lane_bcast<32>(pm));
        } else {
          if constexpr (!FUSE) v_transpose(vw[0]);  // (FUSE: done in phase 1)
          v_transpose(vw[1]);
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            int acc[1][4] = {{0, 0, 0, 0}};
            if (i == 0)
              pv_dot<1, 0>(vw[0], p8, lane, acc);
            else
              pv_dot<1, 1>(vw[1], p8, lane, acc);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[0][e] += lane_xor<32>(acc[0][e]);
            const float pmh = i ? lane_bcast<32>(pm) : lane_bcast<0>(pm);
            if (lane < 32) {
              float4 o;
              o.x = __fmul_rn(static_cast<float>(acc[0][0]), pmh);
              o.y = __fmul_rn(static_cast<float>(acc[0][1]), pmh);
              o.z = __fmul_rn(static_cast<float>(acc[0][2]), pmh);
              o.w = __fmul_rn(static_cast<float>(acc[0][3]), pmh);
              *reinterpret_cast<float4 *>(&sm.pv[0][wave + NW * i][d0]) = o;
            }
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
      const int jb = wave + NW * i;
      if (paired || jb >= nb) continue;
      const int j = (b0 + jb) * 32;
      const int c = lane & 31;
      const bool valid = j + c < kv_end;
      if (i == BPW - 1) patch_v(i, j);  // (the others were patched in phase 1)
#pragma unroll
      for (int hp = 0; hp < QPW; hp += 2) {
        const int h = hp + (lane >> 5);
        const bool hok = h < QPW;
        // this block's nmm of the lane's head (lanes jb and 32 + jb)
        const float nm0 = lane_read(nmm, jb);
        const float nm1 = QPW > 1 ? lane_read(nmm, 32 + jb) : nm0;
        const float nmb = (lane & 32) ? nm1 : nm0;
        float p = 0.0f, pv = 0.0f;
        if (hok && valid) {
          p = exp_f32_le0_tab(__fsub_rn(sm.s[h][jb * 32 + c], nmb), sm.tab);
          pv = __fmul_rn(p, vscale[i]);
        }
        const float psum = tree_sum32(p);
        const float pm = __fmul_rn(max32(pv), inv127());
        const int p8 = hok ? quant1(pv, pm) : 0;
        if (hok && c == 0) sm.psum[h][jb] = psum;
        if constexpr (VMF) {
          if (hok) p8s[((wave * BPW + i) * QPW + h) * 32 + p8_pos(c)] = static_cast<int8_t>(p8);
          pv_mfma(i, jb, lane_bcast<0>(pm), lane_bcast<32>(pm));
          continue;
        }
        if (!FUSE || i == BPW - 1) v_transpose(vw[i]);
        int acc[2][4] = {{0, 0, 0, 0}, {0, 0, 0, 0}};
        pv_dot<(QPW > 1 ? 2 : 1)>(vw[i], p8, lane, reinterpret_cast<int(&)[(QPW > 1 ? 2 : 1)][4]>(acc));
#pragma unroll
        for (int s2 = 0; s2 < (QPW > 1 ? 2 : 1); ++s2)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[s2][e] += lane_xor<32>(acc[s2][e]);
        // lanes 0..31 own the result; pmax of head hp+s2 lives in lane 32*s2
        const float pm0 = lane_bcast<0>(pm), pm1 = lane_bcast<32>(pm);
        if (lane < 32) {
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) {
            const int hh = hp + s2;
            if (hh < QPW) {
              const float pmh = s2 ? pm1 : pm0;
              float4 o;
              o.x = __fmul_rn(static_cast<float>(acc[s2][0]), pmh);
              o.y = __fmul_rn(static_cast<float>(acc[s2][1]), pmh);
              o.z = __fmul_rn(static_cast<float>(acc[s2][2]), pmh);
              o.w = __fmul_rn(static_cast<float>(acc[s2][3]), pmh);
              *reinterpret_cast<float4 *>(&sm.pv[hh][jb][d0]) = o;
            }
          }
        }
      }
    }
    if constexpr (OFUSE) {
      __builtin_amdgcn_sched_barrier(0);
      issue_wo(kOPiecesEarly, kOPieces, b0 + CB >= nblocks);
      __builtin_amdgcn_sched_barrier(0);
    }
    wg_barrier();
    // ---- phase 4: the sequential den/res chain (attention_gqa.h:476-519) ----
    // Batches: operands of 8 blocks are read before their 8 chain steps
    // (entries past nb are read, in bounds, and not used); at b = 1 (up to
    // 24 blocks on 16 CUs) the plain loop measured faster (0.7175 against
    // 0.7229 ms/token).  No barrier follows: the LDS this reads (corr, psum,
    // pv) is next written in the next chunk's phase 3, behind that chunk's
    // first barrier, and the epilogue writes other arrays.
    if constexpr (FUSE) {
      if (tid < QPW * HD) {
        for (int jb = 0; jb < nb; ++jb) {
          const float corr = sm.corr[ph][jb];
          den = __fadd_rn(__fmul_rn(den, corr), sm.psum[ph][jb]);
          res = __fadd_rn(__fmul_rn(res, corr), sm.pv[ph][jb][pd]);
        }
      }
    } else if (tid < QPW * HD) {
      for (int j0 = 0; j0 < nb; j0 += 8) {
        float cr[8], ps[8], pw[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int jb = min(j0 + u, CB - 1);
          cr[u] = sm.corr[ph][jb];
          ps[u] = sm.psum[ph][jb];
          pw[u] = sm.pv[ph][jb][pd];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (j0 + u < nb) {
            den = __fadd_rn(__fmul_rn(den, cr[u]), ps[u]);
            res = __fadd_rn(__fmul_rn(res, cr[u]), pw[u]);
          }
        }
      }
    }
  };
  chunk(0, std::true_type{});
  for (int b0 = CB; b0 < nblocks; b0 += CB) chunk(b0, std::false_type{});


  // ---- epilogue: out = res * (1/den); per-head int8 quant (522-546) ----
  float out = 0.0f;
  if (tid < QPW * HD) {
    out = __fmul_rn(res, __fdiv_rn(1.0f, den));
    const float m = max64(fabsf(out));
    if (lane == 0) sm.absmax[ph][(tid % HD) / 64] = m;
  }
  wg_barrier();
  if (tid < QPW * HD) {
    const int qh = qh0 + ph;
    const float scale = __fmul_rn(fmaxf(sm.absmax[ph][0], sm.absmax[ph][1]), inv127());
    if (a.attn) a.attn[brow * a.ld_attn + qh * HD + pd] = out;
    const int8_t o8 = static_cast<int8_t>(quant1(out, scale));
    o8_row[qh * HD + pd] = o8;
    if (pd == 0) os_row[qh * a.os_col] = scale;
    if constexpr (OFUSE) {
      sm.o8[pd] = o8;
      if (pd == 0) sm.os = scale;
    }
  }
  if constexpr (OFUSE) {
    // O projection partials of this head: 8 lanes per row n, 16 columns
    // each (exact int32 dot products, summed across the 8 lanes), then the
    // two dequant roundings of the group GEMM
    wg_barrier();
    const int *op = reinterpret_cast<const int *>(sm.o8 + 16 * (tid & 7));
    const int o0 = op[0], o1 = op[1], o2 = op[2], o3 = op[3];
    const float osh = sm.os;
    float *dst = a.opart + static_cast<int64_t>(qh0) * a.ld_opart;
#pragma unroll
    for (int i = 0; i < kOPieces; ++i) {
      int acc = sdot4(wov[i].x, o0, 0);
      acc = sdot4(wov[i].y, o1, acc);
      acc = sdot4(wov[i].z, o2, acc);
      acc = sdot4(wov[i].w, o3, acc);
      acc += lane_xor<1>(acc);
      acc += lane_xor<2>(acc);
      acc += lane_xor<4>(acc);
      const int n = i * NW * 8 + tid / 8;
      if ((tid & 7) == 0 && n < h.o_rows) dst[n] = __fmul_rn(__fmul_rn(static_cast<float>(acc), smo.wos[n]), osh);
    }
  }
}

template <int QPW, int NW, int BPW, bool FUSE, bool OFUSE = false>
__global__ void __launch_bounds__(NW * 64) attn_decode_kernel(AttnArgs a) {
  // prefetch workgroups: grid rows y >= 1 of the fused (b = 1) variants, so
  // that telling them apart needs no kernel argument; else x >= heads / QPW
  if constexpr (FUSE) {
    if (blockIdx.y > 0) {
      const int w = static_cast<int>((blockIdx.y - 1) * gridDim.x + blockIdx.x);
      if (w < a.pf_wgs) prefetch_ranges(a, w, static_cast<int>(gridDim.x));
      return;
    }
  } else if (static_cast<int>(blockIdx.x) >= a.heads / QPW) {
    prefetch_ranges(a, static_cast<int>(blockIdx.x) - a.heads / QPW, a.heads / QPW);
    return;
  }
  attn_decode_body<QPW, NW, BPW, FUSE, OFUSE>(a, static_cast<int>(blockIdx.x), static_cast<int>(blockIdx.y));
}

// ---- one launch for a decode token's Q|K|V projection and attention -----
// A kernel boundary costs a launch (~1.6 us) plus the next kernel's first
// dependent loads (~1 us: its operands come from the other XCDs' writes),
// and the attention's K/V blocks then stream into 16 CUs behind them.  Here
// workgroups 0 .. heads - 1 are the b = 1 attention (as attn_decode_kernel
// <1, 12, 2, true, true>), the next gemv_wgs compute the projection (the
// whole-row GEMV of k_gemv.hip, 12 waves of kFusedR rows each), and the rest
// prefetch.  The attention workgroups issue their K/V loads at once and
// poll for their head's 384 projection values, which the GEMV workgroups
// store as exchange words (AttnArgs::xin) besides the f32 rows.  The
// producers never wait, so the launch completes whatever the dispatch order.
constexpr int kFusedWaves = 12;
constexpr int kFusedR = 2;  // projection rows per GEMV wave

// A GEMV wave's kFusedR projection rows: their segment, rows within it,
// scales and 1 KB weight rows (rows past N reload row N - 1, not stored).
struct QkvRows {
  int si, row0;
  int nr[kFusedR];
  float bsn[kFusedR];
  int4 w[kFusedR];
};

__device__ __forceinline__ void qkv_load_rows(const GemvArgs &a, int wg, int N, QkvRows &q) {
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  int s_n0[3];
  const int8_t *s_b[3];
  const float *s_bs[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    s_n0[i] = a.seg[i].n0;
    s_b[i] = a.seg[i].b;
    s_bs[i] = a.seg[i].bs;
  }
  q.row0 = (wg * kFusedWaves + wave) * kFusedR;
  q.si = (q.row0 >= s_n0[1] ? 1 : 0) + (q.row0 >= s_n0[2] ? 1 : 0);
  const int sg_n0 = q.si == 0 ? s_n0[0] : q.si == 1 ? s_n0[1] : s_n0[2];
  const int8_t *const sg_b = q.si == 0 ? s_b[0] : q.si == 1 ? s_b[1] : s_b[2];
  const float *const sg_bs = q.si == 0 ? s_bs[0] : q.si == 1 ? s_bs[1] : s_bs[2];
#pragma unroll
  for (int r = 0; r < kFusedR; ++r) {
    q.nr[r] = min(q.row0 + r, N - 1) - sg_n0;
    q.bsn[r] = sg_bs[q.nr[r]];
    q.w[r] = *reinterpret_cast<const int4 *>(sg_b + static_cast<int64_t>(q.nr[r]) * 1024 + 16 * lane);
  }
}

// The rows' dot products with the int8 A row in LDS (the whole-row GEMV's
// arithmetic), stored as f32 and as exchange words for the attention
// workgroups: Q once, K and V once per query head of their KV head.
__device__ __forceinline__ void qkv_store_rows(const GemvArgs &a, const AttnArgs &t, const QkvRows &q,
                                               const int8_t *a_lds, const float *as_lds, int N) {
  const int lane = threadIdx.x & 63;
  const GemvSeg &sg = a.seg[q.si];
  const int4 av = *reinterpret_cast<const int4 *>(a_lds + 16 * lane);
  const float asg = as_lds[lane >> 4];
  const int grp = t.heads == t.kv_heads ? 1 : 2;  // (attn_decode_supported: 1 or 2)
#pragma unroll
  for (int r = 0; r < kFusedR; ++r) {
    int acc = sdot4(q.w[r].x, av.x, 0);
    acc = sdot4(q.w[r].y, av.y, acc);
    acc = sdot4(q.w[r].z, av.z, acc);
    acc = sdot4(q.w[r].w, av.w, acc);
    acc += lane_xor<1>(acc);
    acc += lane_xor<2>(acc);
    acc += lane_xor<4>(acc);
    acc += lane_xor<8>(acc);
    // p_g = RN(RN(f32(I_g) * bs[n]) * as_g), summed in group order from +0
    const float p = __fmul_rn(__fmul_rn(static_cast<float>(acc), q.bsn[r]), asg);
    float out = 0.0f;
    out = __fadd_rn(out, lane_bcast<0>(p));
    out = __fadd_rn(out, lane_bcast<16>(p));
    out = __fadd_rn(out, lane_bcast<32>(p));
    out = __fadd_rn(out, lane_bcast<48>(p));
    if (lane == 0 && q.row0 + r < N) {
      sg.out[q.nr[r]] = out;
      const unsigned long long word = (1ull << 32) | __float_as_uint(out);
      if (q.si == 0) {
        xstore(t.xin + q.nr[r], word);
      } else {
        const int kvh = q.nr[r] / HD, d = q.nr[r] % HD;
        for (int c = 0; c < grp; ++c)
          xstore(t.xin + (static_cast<int64_t>(q.si) * t.heads + kvh * grp + c) * HD + d, word);
      }
    }
  }
}

template <int PRO>
__device__ __forceinline__ void qkv_gemv_role(const GemvArgs &a, const AttnArgs &t, int wg, int N) {
  __shared__ float blk[32];
  __shared__ __align__(16) int8_t a_lds[1024];
  __shared__ float as_lds[4];
  ProSrc ps = read_src<PRO, false>(a);
  pin_src<PRO, false>(ps);
  ProRow<1, 0> r0;
  pro_load_row<PRO, 1, 0, kFusedWaves>(a, ps, 0, r0);
  __builtin_amdgcn_sched_barrier(0);  // (issue order: prologue operands first)
  QkvRows q;
  qkv_load_rows(a, wg, N, q);
  __builtin_amdgcn_sched_barrier(0);
  pro_compute_row<PRO, 1, 0, kFusedWaves>(a, 0, r0, a_lds, as_lds, blk, wg == 0);  // ends with a barrier
  qkv_store_rows(a, t, q, a_lds, as_lds, N);
}

// The workgroup's role from its id and the role counts.  HEADS / KVH > 0:
// the counts are compile-time constants for that head configuration
// (heads workgroups, then the GEMV's ceil((heads + 2 kv_heads) * 128 /
// (kFusedWaves * kFusedR))), so no workgroup reads a kernel argument before
// its role's first batch of reads; each dependent argument read that misses
// the scalar cache costs ~0.25 us, and the GEMV's outputs are on the
// attention's critical path.  0: the counts are read from the arguments.
template <int HEADS, int KVH>
struct FusedRoles {
  static constexpr int kGemv = (HEADS + 2 * KVH) * HD / (kFusedWaves * kFusedR) +
                               ((HEADS + 2 * KVH) * HD % (kFusedWaves * kFusedR) != 0);
  __device__ static int heads(const AttnArgs &a) { return HEADS > 0 ? HEADS : a.heads; }
  __device__ static int gemv(int gemv_wgs) { return HEADS > 0 ? kGemv : gemv_wgs; }
};

template <int PRO, int HEADS, int KVH>
__global__ void __launch_bounds__(kFusedWaves * 64) qkv_attn_kernel(GemvArgs g, AttnArgs a, int gemv_wgs) {
  using Roles = FusedRoles<HEADS, KVH>;
  const int bx = static_cast<int>(blockIdx.x);
  const int heads = Roles::heads(a);
  if (bx < heads) {
    attn_decode_body<1, kFusedWaves, 2, true, true, true>(a, bx, 0);
    return;
  }
  const int gw = Roles::gemv(gemv_wgs);
  if (bx < heads + gw) {
    qkv_gemv_role<PRO>(g, a, bx - heads, g.seg[2].n1);
  } else {
    const int w = bx - heads - gw;
    if (w < a.pf_wgs) prefetch_ranges(a, w, heads + gw);
  }
}

// ---- the previous layer's down projection in the same launch ------------
// The G GEMV workgroups first finish the previous layer's MLP: waves 0..5
// of workgroup wg own down column n = wave * G + wg (n < N_down): the SwiGLU
// row quantised per 256 (d's PRO_QUANT prologue, K = 3072), its dot with
// the 3 KB weight row, then x[n] = (x[n] + O) + down with the O partials
// summed in head order, as the whole-row GEMV's EPI_ADD epilogue computes
// it.  Each column goes to x and, as f32 bits, to each copy of
// AttnArgs::xw.  After the workgroup's own stores, the last wave waits for
// all 1024 words of copy wg % kXwCopies (4 KB a round, 16 bytes a lane and
// load, all in flight before any check), puts the row into LDS and the
// workgroup continues as qkv_gemv_role with the new x.  kXwEmpty marks a
// word not yet stored: a NaN with every payload bit set, which the down
// epilogue produces only from such a NaN among its inputs (then the wait
// runs out and reports it).  Every GEMV workgroup waits for every other
// one, so all of them must be resident together (G + heads workgroups of
// one per CU: the launch checks G + heads <= CUs); the wait is bounded like
// the attention's.  The Q|K|V weights and the down operands are all
// requested before the first wait.
__device__ __forceinline__ void down_qkv_role(const GemvArgs &d, const GemvArgs &a, const AttnArgs &t, int wg,
                                              int G) {
  __shared__ float blk[32];
  __shared__ __align__(16) int8_t a_lds[3072];
  __shared__ float as_lds[12];
  __shared__ __align__(16) float x_lds[1024];
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int N = a.seg[2].n1;
  const int Nd = d.seg[0].n1;
  ProSrc dps = read_src<PRO_QUANT, true>(d);
  const int8_t *db = d.seg[0].b;
  const float *dbs = d.seg[0].bs;
  float *dx = d.seg[0].out;
  const float *gain = a.w_pre;
  pin_src<PRO_QUANT, true>(dps);
  // the SwiGLU row (waves w and w + 4, w + 8 load group set w & 3)
  ProRow<3, 0> rd;
  pro_load_row<PRO_QUANT, 3, 0, kFusedWaves>(d, dps, 0, rd);
  __builtin_amdgcn_sched_barrier(0);
  // this wave's down column: weights, scale, residual, O partials
  const int n = wave * G + wg;
  const bool down = n < Nd;
  const int nc = min(n, Nd - 1);
  int4 dw[3];
#pragma unroll
  for (int j = 0; j < 3; ++j) dw[j] = make_int4(0, 0, 0, 0);
  float dbsn = 0.0f, xn = 0.0f, pv = 0.0f;
  if (down) {
#pragma unroll
    for (int j = 0; j < 3; ++j)
      dw[j] = *reinterpret_cast<const int4 *>(db + static_cast<int64_t>(nc) * 3072 + 1024 * j + 16 * lane);
    dbsn = dbs[nc];
    xn = dx[nc];
    pv = dps.part[min(lane & 15, dps.npart - 1) * dps.ld_part + nc];
  }
  __builtin_amdgcn_sched_barrier(0);
  // the Q|K|V rows and the n1 gains of this wave's RMSNorm group
  QkvRows q;
  qkv_load_rows(a, wg, N, q);
  ProRow<1, 0> r0;
  r0.w[0] = *reinterpret_cast<const float4 *>(gain + (wave & 3) * 256 + 4 * lane);
  __builtin_amdgcn_sched_barrier(0);
  pro_compute_row<PRO_QUANT, 3, 0, kFusedWaves>(d, 0, rd, a_lds, as_lds, blk, wg == 0);  // ends with a barrier
  if (down) {
    float out = 0.0f;
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int4 av = *reinterpret_cast<const int4 *>(a_lds + 1024 * j + 16 * lane);
      const float asg = as_lds[4 * j + (lane >> 4)];
      int acc = sdot4(dw[j].x, av.x, 0);
      acc = sdot4(dw[j].y, av.y, acc);
      acc = sdot4(dw[j].z, av.z, acc);
      acc = sdot4(dw[j].w, av.w, acc);
      acc += lane_xor<1>(acc);
      acc += lane_xor<2>(acc);
      acc += lane_xor<4>(acc);
      acc += lane_xor<8>(acc);
      const float p = __fmul_rn(__fmul_rn(static_cast<float>(acc), dbsn), asg);
      out = __fadd_rn(out, lane_bcast<0>(p));
      out = __fadd_rn(out, lane_bcast<16>(p));
      out = __fadd_rn(out, lane_bcast<32>(p));
      out = __fadd_rn(out, lane_bcast<48>(p));
    }
    float o = 0.0f;  // the O projection, partials in head order
#pragma unroll
    for (int h = 0; h < kMaxPart; ++h)
      if (h < dps.npart) o = __fadd_rn(o, __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(pv), h)));
    const float v = __fadd_rn(__fadd_rn(xn, o), out);
    if (lane == 0) dx[n] = v;
    if (lane < kXwCopies)
      __hip_atomic_store(t.xw + lane * kXwStride + n, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  lds_barrier();  // (the first round of polls after the workgroup's own stores)
  if (wave == kFusedWaves - 1) {
    // columns 256 i + 4 lane .. + 3 are v[i]
    v4u32 v[4];
    for (int it = 0;; ++it) {
      xload_4k(t.xw + (wg % kXwCopies) * kXwStride, v[0], v[1], v[2], v[3]);
      bool ok = true;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        ok = ok && v[i].x != kXwEmpty && v[i].y != kXwEmpty && v[i].z != kXwEmpty && v[i].w != kXwEmpty;
      if (__all(ok)) break;
      if (it == kPollLimit) {
        if (lane == 0) __hip_atomic_store(t.xerr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<v4u32 *>(x_lds + 256 * i + 4 * lane) = v[i];
  }
  lds_barrier();
  if (wave < 4) r0.x[0] = *reinterpret_cast<const float4 *>(x_lds + wave * 256 + 4 * lane);
  // (the A row of the projection reuses a_lds: every wave read its down
  // operand before the prologue's first barrier)
  pro_compute_row<PRO_NORM, 1, 0, kFusedWaves>(a, 0, r0, a_lds, as_lds, blk, wg == 0);  // ends with a barrier
  qkv_store_rows(a, t, q, a_lds, as_lds, N);
}

template <int HEADS, int KVH>
__global__ void __launch_bounds__(kFusedWaves * 64) down_qkv_attn_kernel(GemvArgs d, GemvArgs g, AttnArgs a,
                                                                          int gemv_wgs) {
  using Roles = FusedRoles<HEADS, KVH>;
  const int bx = static_cast<int>(blockIdx.x);
  const int heads = Roles::heads(a);
  if (bx < heads) {
    attn_decode_body<1, kFusedWaves, 2, true, true, true>(a, bx, 0);
    return;
  }
  const int gw = Roles::gemv(gemv_wgs);
  if (bx < heads + gw) {
    down_qkv_role(d, g, a, bx - heads, gw);
  } else {
    const int w = bx - heads - gw;
    if (w < a.pf_wgs) prefetch_ranges(a, w, heads + gw);
  }
}

// One workgroup per query head (QPW = 1): 16 workgroups for the 16/8-head
// model instead of 8 halves the per-workgroup work, which matters more here
// than reading each KV head's rows twice.  8 waves x 3 blocks (768 keys per
// chunk) keep K and V of the chunk in registers without spilling.
// Independent sequences (row_pos set): one workgroup per KV head and
// sequence with both query heads of the group, so each K/V row is read once;
// the batch supplies the parallelism that b = 1 has to find in query heads.
hipError_t launch_decode_batch(const AttnArgs &a, hipStream_t s) {
  constexpr int QPW = 2, NW = 4, BPW = 3;
  Q3_LAUNCH((attn_decode_kernel<QPW, NW, BPW, false>), dim3(a.heads / QPW, a.rows), dim3(NW * 64), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_decode(const AttnArgs &a, hipStream_t s) {
  constexpr int QPW = 1, NW = 12, BPW = 2;
  static_assert(QPW * HD <= NW * 64, "phase 4 needs a thread per (head, dim)");
  const int extra = a.pf_n > 0 ? a.pf_wgs : 0;
  const int seqs = a.row_pos ? a.rows : 1;
  static_assert(kOPieces * NW * 8 >= kORowsMax, "O projection rows per workgroup");
  // fused: the prefetch workgroups are grid rows 1.. (ids after the heads')
  const int hx = a.heads / QPW;
  const dim3 fgrid(hx, 1 + (extra + hx - 1) / hx);
  if (a.fuse_heads && a.opart)
    Q3_LAUNCH((attn_decode_kernel<QPW, NW, BPW, true, true>), fgrid, dim3(NW * 64), 0, s, a);
  else if (a.fuse_heads)
    Q3_LAUNCH((attn_decode_kernel<QPW, NW, BPW, true>), fgrid, dim3(NW * 64), 0, s, a);
  else
    Q3_LAUNCH((attn_decode_kernel<QPW, NW, BPW, false>), dim3(a.heads / QPW + extra, seqs), dim3(NW * 64), 0, s, a);
  return hipGetLastError();
}

}  // namespace

bool attn_decode_supported(const AttnArgs &a) {
  const int grp = a.kv_heads > 0 ? a.heads / a.kv_heads : 0;
  auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  for (int r = 0; r < a.pf_n; ++r)
    if ((reinterpret_cast<uintptr_t>(a.pf[r]) & 15) != 0 || a.pf_bytes[r] < 0) return false;
  if (a.row_pos && (a.rows < 1 || a.rows > 65535 || a.fuse_heads || a.pf_n || !a.row_tables)) return false;
  if (a.pf_kv_heads > 0 &&
      (!a.fuse_heads || a.pf_n < 4 || a.kv_heads <= 0 || a.pf_kv_heads % a.kv_heads != 0 ||
       static_cast<int64_t>(a.kv_heads) * HD > a.row_bytes || !a.pf_table || a.pf_pages < 0 ||
       a.scale_page_bytes % 16 != 0 ||
       static_cast<int64_t>(a.page_tokens) * ((a.pf_kv_heads + 7) / 8) * 8 >= (int64_t{1} << 31) ||
       a.scale_page_bytes / 16 >= (int64_t{1} << 31)))
    return false;
  // O projection fusion: b = 1 with the head epilogues; rows of wo cover
  // every head's 128 columns and are 16-byte aligned
  if (a.opart && (!a.fuse_heads || a.row_pos || !a.wo || !a.wos || !al16(a.wo) || (a.ldwo % 16) != 0 ||
                  a.ldwo < static_cast<int64_t>(a.heads) * HD || a.o_rows < 1 || a.o_rows > kORowsMax ||
                  a.ld_opart < a.o_rows))
    return false;
  return (a.rows == 1 || a.row_pos) && a.causal && (grp == 1 || grp == 2) && a.kv_heads * grp == a.heads &&
         a.pf_n >= 0 && a.pf_n <= 12 && (a.pf_n == 0 || a.pf_wgs > 0) &&
         (a.row_bytes % 16) == 0 && (a.page_tokens % 32) == 0 && al16(a.k) && al16(a.v) &&
         al16(a.q8) && (a.scale_row_bytes % 4) == 0 && (a.kv_len >= 1 || a.row_pos) && !a.kv_len_dev &&
         (!a.row_pos || (a.ldq % 16) == 0);
}

namespace {
// the GEMV workgroups of the fused launches: kFusedR rows per wave
int qkv_gemv_wgs(const GemvArgs &g) {
  return (g.seg[2].n1 + kFusedWaves * kFusedR - 1) / (kFusedWaves * kFusedR);
}
}  // namespace

bool qkv_attn_supported(const GemvArgs &g, const AttnArgs &a) {
  if (g.M != 1 || g.K != 1024 || g.group != 256 || g.bs_ld || g.part || g.nseg != 3) return false;
  if (g.pro != PRO_NORM && g.pro != PRO_EMBED) return false;
  const int HW = a.heads * HD, KW = a.kv_heads * HD;
  if (g.seg[0].n0 != 0 || g.seg[0].n1 != HW || g.seg[1].n0 != HW || g.seg[1].n1 != HW + KW ||
      g.seg[2].n0 != HW + KW || g.seg[2].n1 != HW + 2 * KW)
    return false;
  for (int i = 0; i < 3; ++i)
    if (g.seg[i].epi != EPI_STORE || !g.seg[i].b || !g.seg[i].bs || !g.seg[i].out) return false;
  if (HW % kFusedR || KW % kFusedR) return false;
  // the attention: one query row, head epilogues and O projection fused,
  // one workgroup per query head (launch_decode's b = 1 variant)
  if (!a.xin || !a.xerr || !a.fuse_heads || !a.opart || a.row_pos || a.rows != 1 || a.heads % a.kv_heads) return false;
  return attn_decode_supported(a);
}

bool head_consts(int heads, int kv_heads) {
  if (heads != 16 || kv_heads != 8) return false;
  const char *e = std::getenv("Q3_HEAD_CONSTS");
  return !(e && std::strcmp(e, "0") == 0);
}

namespace {
bool fused_roles_const(const AttnArgs &a) { return head_consts(a.heads, a.kv_heads); }
}  // namespace

hipError_t launch_qkv_attn(const GemvArgs &g, const AttnArgs &a, hipStream_t s) {
  const int gw = qkv_gemv_wgs(g);
  const int extra = a.pf_n > 0 ? a.pf_wgs : 0;
  const dim3 grid(a.heads + gw + extra);
  const dim3 block(kFusedWaves * 64);
  const bool c = fused_roles_const(a);
  static_assert(FusedRoles<16, 8>::kGemv == (4096 + kFusedWaves * kFusedR - 1) / (kFusedWaves * kFusedR), "");
  if (g.pro == PRO_EMBED) {
    if (c)
      Q3_LAUNCH((qkv_attn_kernel<PRO_EMBED, 16, 8>), grid, block, 0, s, g, a, gw);
    else
      Q3_LAUNCH((qkv_attn_kernel<PRO_EMBED, 0, 0>), grid, block, 0, s, g, a, gw);
  } else {
    if (c)
      Q3_LAUNCH((qkv_attn_kernel<PRO_NORM, 16, 8>), grid, block, 0, s, g, a, gw);
    else
      Q3_LAUNCH((qkv_attn_kernel<PRO_NORM, 0, 0>), grid, block, 0, s, g, a, gw);
  }
  return hipGetLastError();
}

bool down_qkv_attn_supported(const GemvArgs &d, const GemvArgs &g, const AttnArgs &a) {
  if (g.pro != PRO_NORM || !a.xw || !qkv_attn_supported(g, a)) return false;
  auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const GemvSeg &s0 = d.seg[0];
  if (d.M != 1 || d.K != 3072 || d.group != 256 || d.bs_ld || d.pro != PRO_QUANT || d.nseg != 1 ||
      s0.epi != EPI_ADD || s0.n0 != 0 || !s0.b || !s0.bs || !s0.out)
    return false;
  // the down output is the row g normalises (K = 1024 = four 256-column
  // groups, one per polling wave), its partials are not the ones this
  // launch's attention writes
  if (s0.n1 != g.K || s0.out != g.x || !d.x || !al16(d.x) || !al16(g.w_pre) || !d.part || d.npart < 1 ||
      d.npart > kMaxPart || d.ld_part < s0.n1 || d.part == a.opart)
    return false;
  // every down column has a wave, and every GEMV workgroup is resident with
  // the attention's (one 12-wave workgroup per CU)
  const int gw = qkv_gemv_wgs(g);
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return false;
  return static_cast<int64_t>(gw) * kFusedWaves >= s0.n1 && a.heads + gw <= cus;
}

hipError_t launch_down_qkv_attn(const GemvArgs &d, const GemvArgs &g, const AttnArgs &a, hipStream_t s) {
  const int gw = qkv_gemv_wgs(g);
  const int extra = a.pf_n > 0 ? a.pf_wgs : 0;
  if (fused_roles_const(a))
    Q3_LAUNCH((down_qkv_attn_kernel<16, 8>), dim3(a.heads + gw + extra), dim3(kFusedWaves * 64), 0, s, d, g, a, gw);
  else
    Q3_LAUNCH((down_qkv_attn_kernel<0, 0>), dim3(a.heads + gw + extra), dim3(kFusedWaves * 64), 0, s, d, g, a, gw);
  return hipGetLastError();
}

hipError_t launch_attn_decode(const AttnArgs &a, hipStream_t s) {
  if (a.row_pos && a.heads == 2 * a.kv_heads) return launch_decode_batch(a, s);
  return launch_decode(a, s);
}

}  // namespace q3
