// Paged hd128 GQA attention for multi-row chunks (prefill), with the
// reference's block-quantised online softmax parallelised exactly.
//
//   kernels/attention_gqa.h:404-572 attention_heads_gqa_tokscale_paged /
//                                   attention_head_hd128_blocks_paged
//   ref_qwen3.py:210-289            attention_head_blocks / ..._gqa_tokscale
//
// The reference walks 32-key blocks j in order and carries, per query row,
// (maximum, den, res[128]):
//   s    = ((f32 S_j * ks) * qs) * qk, masked keys -inf, S_j = q8 . k8^T
//   nmm  = max(tree_max(s), maximum);  corr = exp(maximum - nmm)
//   P    = exp(s - nmm);  den = den * corr + tree_sum(P)
//   pv   = P * vs;  pmax = absmax(pv) * (1/127);  P8 = quant(pv, pmax)
//   res  = res * corr + f32(P8 . V_j) * pmax
// and ends with out = res * (1/den), quantised per head to int8.  Only the
// den/res updates depend on the previous block; the running maximum is a
// prefix max of the block maxima.  So per chunk of up to CB blocks (8 per
// query block of the workgroup):
//   phase 1 (one wave per block)    S_j, s, block maximum bm_j
//   phase 2 (every lane, tiny)      nmm_j = max(nmm_{j-1}, bm_j), in block order
//   phase 3 (one wave per block)    corr_j, P, psum_j, pv, pmax_j, P8_j
//   phase 4 (one wave per 16 dims)  res = res * corr_j + f32(P8_j . V_j) * pmax_j
//                                   and den = den * corr_j + psum_j, j in order
// with the reference's rounding points, so the result equals the one-block
// walk bit for bit.  Chunks carry (maximum, den, res) the way blocks do.
//
// Work: 8 waves per 16-row query block of one head.  The default workgroup
// holds one query block (74 KiB of LDS, two workgroups per CU) and the grid
// is ordered so that the two workgroups a CU usually receives, L and
// L + heads * floor(nqb / 2), take the causally complementary blocks
// nqb - 1 - qb and qb (the long one dispatched first).  The paired form (NI = 2, 16 waves) walks both blocks of a
// pair at once: A's key blocks are a prefix of B's, so each K/V block is
// copied once and serves both (two 16-column MFMA tiles) while A needs it.
// Wave w owns block w of a chunk in phases 1 and 3 and, in phase 4, 16 output
// dimensions (16 (w % 8)..+15) of item w / 8.  Step g runs phase 4 of chunk
// g - 1 and phase 1 of chunk g, barrier, phases 2-3 of chunk g (and the int8
// store of an item whose last chunk was g - 1), barrier.  Every wave copies
// its own block of the next chunk: V with global_load_lds into the other half
// of a two-chunk LDS ring, the K operand rows and ks | vs straight into
// registers.
//
// Layouts (lane = lc + 16 lg):
//   S^T_j = K_j . Q^T with v_mfma_i32_16x16x64_i8, keys as the M dimension:
//     lane holds s[kt][i] for key 16 kt + 4 lg + i, query row lc, so a
//     key reduction is 2 in-register levels, 2 lane swaps (lg) and the kt
//     pair, in the reference's pairwise-tree order.
//   P8_j stays in that lane order (byte m = 4 kt + i is key 16 kt + 4 lg + i)
//     as the B operand of (P8 . V)^T = V^T . P8^T (v_mfma_i32_16x16x32_i8);
//     the V^T operand carries the same key order and is read with
//     ds_read_b64_tr_b8 (gfx950's transposing LDS load: in each 16-lane
//     group, result lane i byte j is byte i & 7 of the 8 bytes addressed by
//     source lane 2 j + (i >> 3)), so no transposed copy of V is built, and
//     lane (lc, lg) receives row lc, dims 4 lg..4 lg + 3 of the wave's tile.
//   V stage  [32 keys][8 x 16 B], chunk c of key r at c ^ ((r & 3) | ((r >> 2) & 4)):
//     the 8 keys a transposing read gathers land on 8 different chunks.
#include <cstdlib>
#include <cstring>

#include "q3_device.h"
#include "q3_kernels.h"

namespace q3 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2i *lds_v2i_ptr;

constexpr int QB = 16;   // query rows per item
constexpr int KB = 32;   // keys per block (= reference block)
constexpr int HD = 128;

// NI query blocks per workgroup (2: the causal pair, 1: one block, two
// workgroups per CU); 8 waves per query block; wave w owns key block w of
// each chunk
template <int NI>
struct Cfg {
  static constexpr int NW = 8 * NI;
  static constexpr int CB = NW;       // key blocks per chunk
  static constexpr int LDB = CB + 4;  // row stride of the per-(row, block) arrays
};

template <int NI>
struct Lds {
  static constexpr int CB = Cfg<NI>::CB, LDB = Cfg<NI>::LDB;
  int8_t v[2][CB][KB * HD];    // V stages of two chunks
  uint64_t p8[NI][CB][64];     // P8 of each (item, block), in MFMA operand lane order
  float bm[NI][QB][LDB];       // block maxima [item][row][block]
  float corr[NI][QB][LDB], psum[NI][QB][LDB], pmax[NI][QB][LDB];
  float cmax[NI][QB][8];       // |out| maxima of each 16-dim tile
  uint64_t etab[32];
};
static_assert(sizeof(Lds<1>) <= 80 * 1024, "two single-block workgroups per CU");

__device__ __forceinline__ int vswz(int key) { return (key & 3) | ((key >> 2) & 4); }

__device__ __forceinline__ v4i zero4() {
  v4i z = {0, 0, 0, 0};
  return z;
}

// One query block of QB rows of head h.
struct Item {
  int qi, nr;      // first row, valid rows
  int pos0;        // position of row qi
  int nblk;        // key blocks walked
  bool extra;      // the reference's 32-row walk has more (fully masked) blocks
};

// The kernel arguments the first copies and Q loads depend on, read together
// at the top and pinned in SGPRs: read where first used, they form a chain of
// scalar-cache round trips (~0.25 us each on a miss) before the first load.
struct PreArgs {
  int rows, causal, blk_page_n;
  uint32_t kv_len, page_tokens;
  const int32_t *kv_len_dev;
  const uint16_t *table;
  const int8_t *k, *v;
  const float *ks, *vs;
  int64_t page_bytes, row_bytes, scale_page_bytes, scale_row_bytes;
  const int8_t *q8;
  int64_t ldq;
  const float *qs;
  int64_t ldqs, qs_col;
};

__device__ __forceinline__ PreArgs pre_args(const AttnArgs &a) {
  PreArgs p;
  p.rows = pin_sgpr(a.rows);
  p.causal = pin_sgpr(a.causal);
  p.blk_page_n = pin_sgpr(a.blk_page_n);
  p.kv_len = pin_sgpr(a.kv_len);
  p.page_tokens = pin_sgpr(a.page_tokens);
  p.kv_len_dev = pin_sgpr(a.kv_len_dev);
  p.table = pin_sgpr(a.table);
  p.k = pin_sgpr(a.k);
  p.v = pin_sgpr(a.v);
  p.ks = pin_sgpr(a.ks);
  p.vs = pin_sgpr(a.vs);
  p.page_bytes = pin_sgpr(a.page_bytes);
  p.row_bytes = pin_sgpr(a.row_bytes);
  p.scale_page_bytes = pin_sgpr(a.scale_page_bytes);
  p.scale_row_bytes = pin_sgpr(a.scale_row_bytes);
  p.q8 = pin_sgpr(a.q8);
  p.ldq = pin_sgpr(a.ldq);
  p.qs = pin_sgpr(a.qs);
  p.ldqs = pin_sgpr(a.ldqs);
  p.qs_col = pin_sgpr(a.qs_col);
  return p;
}

__device__ __forceinline__ Item make_item(const PreArgs &a, int qb, int kv_len) {
  Item it;
  it.qi = qb * QB;
  it.nr = min(QB, a.rows - it.qi);
  const int pg0 = a.causal ? kv_len - a.rows : 0;  // position of row 0
  it.pos0 = pg0 + it.qi;
  int kv_end = kv_len;
  if (a.causal) kv_end = min(kv_len, it.pos0 + it.nr);
  it.nblk = (kv_end + KB - 1) / KB;
  // ref_qwen3.py:281-288: 32-row query blocks, each walking up to its last row
  const int qi32 = it.qi & ~31;
  int kv_end32 = kv_len;
  if (a.causal) kv_end32 = min(kv_len, pg0 + qi32 + min(32, a.rows - qi32));
  it.extra = (kv_end32 + KB - 1) / KB > it.nblk;
  return it;
}

// quant_rcp (q3_device.h) for x >= 0 (P * vs): the NaN of 0 * inf goes to
// +0 through the max.
__device__ __forceinline__ int quant_rcp_pos(float x, double y) {
  float q = __double2float_rn(__dmul_rn(static_cast<double>(x), y));
  q = fmaxf(q, 0.0f);
  return static_cast<int>(fminf(rintf(q), 127.0f));
}

__device__ __forceinline__ uint32_t pack4(int b0, int b1, int b2, int b3) {
  return (static_cast<uint32_t>(b0) & 0xffu) | ((static_cast<uint32_t>(b1) & 0xffu) << 8) |
         ((static_cast<uint32_t>(b2) & 0xffu) << 16) | (static_cast<uint32_t>(b3) << 24);
}

// (the second bound is waves per SIMD: 16 waves per CU, two single-block
// workgroups or one pair, i.e. at most 128 VGPRs).  HEADS / KVH > 0: the
// head counts as compile-time constants (the grid is heads wide), so a
// workgroup finds its head and query block without reading an argument or
// dividing by one; each dependent kernel-argument read that misses the
// scalar cache costs ~0.25 us before the first copy.  0: read from a.
template <int NI, int HEADS = 0, int KVH = 0>
__global__ void __launch_bounds__(Cfg<NI>::NW * 64, 4) attn_prefill_kernel(AttnArgs a) {
  constexpr int CB = Cfg<NI>::CB;
  extern __shared__ __align__(16) int8_t smem[];
  Lds<NI> &L = *reinterpret_cast<Lds<NI> *>(smem);
  // LDS slot of item it (A = 0, B = 1; one slot when there is no A)
  auto sl = [](int it) { return NI == 2 ? it : 0; };

  // lane indices are re-read at every step (below): per-lane addresses
  // derived from them are recomputed, not hoisted out of the loop into
  // registers that would then spill
  int lane = threadIdx.x & 63;
  const int wave = wave_id();
  int lc = lane & 15;
  int lg = lane >> 4;
  // the first chunk's page id of this wave's block (used where the block is
  // below blk_page_n; read with the other arguments)
  static_assert(Cfg<NI>::CB <= 32, "first chunk's page ids come from blk_page");
  const uint32_t pg_arg0 = a.blk_page[wave];
  const PreArgs pa = pre_args(a);
  // XCD-aware order: workgroup L runs on XCD L % 8 and takes KV head
  // L % kv_heads, so the workgroups of one XCD share the K/V rows its L2 holds
  const int a_heads = HEADS > 0 ? HEADS : a.heads;
  const int a_kv_heads = HEADS > 0 ? KVH : a.kv_heads;
  const int group = a_heads / a_kv_heads;
  const int L_id = blockIdx.x + (HEADS > 0 ? HEADS : static_cast<int>(gridDim.x)) * blockIdx.y;
  const int nqb = (pa.rows + QB - 1) / QB;
  int kvh, h, qbA, qbB;
  if constexpr (NI == 2) {  // grid: heads x the pairs
    kvh = L_id % a_kv_heads;
    const int r_id = L_id / a_kv_heads;
    h = kvh * group + r_id % group;
    qbA = r_id / group;
    qbB = nqb - 1 - qbA;
  } else {  // grid: heads x nqb; workgroups L and L + heads * floor(nqb / 2)
            // (dispatched one round apart, so usually on one CU) take
            // complementary query blocks nqb - 1 - qb and qb of one head; the
            // long (late) query blocks are dispatched first, since the last
            // of them to end sets the launch
    const int half = nqb / 2 * a_heads;
    const int idx = L_id < half ? L_id : L_id - half;
    const int hs = idx % a_heads;
    kvh = hs % a_kv_heads;
    h = kvh * group + hs / a_kv_heads;
    qbB = L_id < half ? nqb - 1 - idx / a_heads : idx / a_heads;
    qbA = qbB;
  }
  int kv_len = static_cast<int>(pa.kv_len);
  if (pa.kv_len_dev) kv_len += *pa.kv_len_dev;
  const bool twoA = NI == 2 && qbB > qbA;  // item A exists (else B is the only item)
  const Item IA = make_item(pa, qbA, kv_len);
  const Item IB = make_item(pa, twoA ? qbB : qbA, kv_len);
  const int nA = twoA ? IA.nblk : 0;
  const int nB = IB.nblk;
  const int G = (nB + CB - 1) / CB;
  const int pt_shift = 31 - __builtin_clz(pa.page_tokens);  // page_tokens is a power of two
  // blocks of item `it` in chunk g
  auto nb_of = [&](int it, int g) { return max(0, min(CB, (it ? nB : nA) - g * CB)); };
  auto last_of = [&](int it, int g) { return (it ? nB : nA) > 0 && ((it ? nB : nA) - 1) / CB == g; };

  // ---- this wave's copies of its block of chunk g ----
  v4i kop[2][2];  // K operand rows of the wave's block: [kt][64-byte k-step]
  const int phys = lane & 7;
  // the page id of the wave's block of chunk g, held by lane 0: a kernel
  // argument for the first blk_page_n blocks, else a table load (per lane: a
  // wave-uniform load would be read into a scalar register at once, making
  // the wave wait there for every load issued before it, i.e. for the K/V
  // copies of the chunk before); users take it with pg()
  auto page_of = [&](int g) -> uint32_t {
    uint32_t p = 0;
    const int j = g * CB + wave;
    if (g < G && wave < nb_of(1, g)) {
      if (j < pa.blk_page_n)
        p = g == 0 ? pin_sgpr(pg_arg0) : a.blk_page[j];
      else if (lane == 0)
        p = pa.table[static_cast<uint32_t>(j * KB) >> pt_shift];
    }
    return p;
  };
  auto pg = [](uint32_t p) { return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(p), 0)); };
  // in-page offsets fit in 32 bits (checked on the host)
  const int rb = static_cast<int>(pa.row_bytes), srb = static_cast<int>(pa.scale_row_bytes);
  auto copy_v = [&](int g, uint32_t page) {
    if (g >= G || wave >= nb_of(1, g)) return;
    const int slot0 = ((g * CB + wave) * KB) & (pa.page_tokens - 1);
    const int8_t *vb = pa.v + static_cast<int64_t>(pg(page)) * pa.page_bytes + kvh * HD;
    int8_t *dst = L.v[g & 1][wave];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int key = 8 * t + (lane >> 3);
      const int off = (slot0 + key) * rb + ((phys ^ vswz(key)) << 4);
      __builtin_amdgcn_global_load_lds(const_cast<int8_t *>(vb + off), to_lds(dst + t * 1024), 16, 0, 0);
    }
  };
  auto load_k = [&](int g, uint32_t page) {
    if (g >= G || wave >= nb_of(1, g)) return;
    const int slot0 = ((g * CB + wave) * KB) & (pa.page_tokens - 1);
    const int8_t *kb = pa.k + static_cast<int64_t>(pg(page)) * pa.page_bytes + kvh * HD;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        kop[kt][ks] = *reinterpret_cast<const v4i *>(kb + ((slot0 + 16 * kt + lc) * rb + 64 * ks + 16 * lg));
  };
  // ks and vs of keys 16 kt + 4 lg + i of the wave's block, in registers
  // (not staged through LDS by global_load_lds: a DS read of memory that an
  // LDS DMA writes waits for every DMA in flight, i.e. for the next chunk's
  // V copies)
  float ksr[2][4], vsr[2][4];
  auto load_sc = [&](int g, uint32_t page) {
    if (g >= G || wave >= nb_of(1, g)) return;
    const int slot0 = ((g * CB + wave) * KB) & (pa.page_tokens - 1);
    const int64_t sp = static_cast<int64_t>(pg(page)) * pa.scale_page_bytes + kvh * 4;
    const int8_t *kb = reinterpret_cast<const int8_t *>(pa.ks) + sp;
    const int8_t *vb = reinterpret_cast<const int8_t *>(pa.vs) + sp;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int off = (slot0 + 16 * kt + 4 * lg + i) * srb;
        ksr[kt][i] = *reinterpret_cast<const float *>(kb + off);
        vsr[kt][i] = *reinterpret_cast<const float *>(vb + off);
      }
  };

  // ---- prologue: chunk 0 in flight, exp table, Q operands of both items ----
  uint32_t page = page_of(0);
  copy_v(0, page);
  load_k(0, page);
  load_sc(0, page);
  page = page_of(1);
  if (threadIdx.x == 0) stage_exp2_table(L.etab);
  // Q row lc of item A / B as the B operand, [item][64-byte k-step]; loaded
  // with each chunk's K rows so that it is not live through phases 3-4
  v4i qop[2][2];
  float qsv[2];
  auto load_q = [&](int g) {
    if (g >= G) return;
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const Item &I = it ? IB : IA;
      const bool ok = lc < I.nr && (it || twoA);
      const int8_t *q = pa.q8 + static_cast<int64_t>(I.qi + lc) * pa.ldq + h * HD + 16 * lg;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) qop[it][ks] = ok ? *reinterpret_cast<const v4i *>(q + 64 * ks) : zero4();
      qsv[it] = ok ? pa.qs[static_cast<int64_t>(I.qi + lc) * pa.ldqs + h * pa.qs_col] : 0.0f;
    }
  };
  load_q(0);
  // phase-4 role: item it4, dims 16 dt..16 dt + 15
  const int it4 = NI == 2 ? wave >> 3 : 1, dt = wave & 7;
  // transposing-read address of this lane inside a V stage, for dims 16 dt..+15
  int v_tr_off;
  {
    const int g4 = lane >> 4, jj = (lane & 15) >> 1, hh = lane & 1;
    const int key = 16 * (jj >> 2) + 4 * g4 + (jj & 3);
    v_tr_off = key * HD + ((dt ^ vswz(key)) << 4) + 8 * hh;
  }
  const float qk = a.qk_scale;
  float m_run[2] = {-3.402823466e38f, -3.402823466e38f};  // carried maxima of row lc
  float res[4] = {0.0f, 0.0f, 0.0f, 0.0f}, den = 0.0f;    // item it4, row lc, dims 16 dt + 4 lg + i
  float out[4];
  float s[2][2][4];  // [item][kt][i]

  for (int g = 0; g <= G; ++g) {
    asm volatile("" : "+v"(lane), "+v"(lc), "+v"(lg));
    // ---- phase 4 (chunk g - 1), item it4 ----
    bool ended = false;  // item it4's last chunk was g - 1
    if (g >= 1) {
      const int gp = g - 1;
      const int nbp = nb_of(it4, gp);
      const int8_t *vbase = &L.v[gp & 1][0][0];
      for (int b0 = 0; b0 < nbp; b0 += 4) {
        float4 c4, p4, s4;
        v2i vt[4];
        long pbv[4];
        const int8_t *vq = vbase + b0 * (KB * HD) + v_tr_off;
        if constexpr (NI == 1) {
          // Every LDS read of this phase is inline asm: the compiler makes a DS
          // read wait for every LDS DMA in flight (vmcnt 0) unless it can tell
          // the memory apart, and here chunk g's V copies (into the other half
          // of the ring) and K/Q/scale loads are in flight, which this phase
          // does not read and should run under.  What it reads: chunk g - 1's
          // V half, complete since that chunk's phase 1 (vmcnt 0) and its
          // barriers, and corr/pmax/psum/P8 from its phase 3, before B2(g - 1).
          // The reads complete at the lgkmcnt wait below, before B1(g), after
          // which chunk g + 1's copies overwrite this V half.
          // (one asm statement: the values exist only after its wait, and the
          // early-clobbered outputs keep the addresses intact until issued)
          auto la = [](const void *p) { return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p)); };
          asm volatile(
              "ds_read_b128 %0, %11\n\t"
              "ds_read_b128 %1, %12\n\t"
              "ds_read_b128 %2, %13\n\t"
              "ds_read_b64_tr_b8 %3, %14\n\t"
              "ds_read_b64_tr_b8 %4, %15\n\t"
              "ds_read_b64_tr_b8 %5, %16\n\t"
              "ds_read_b64_tr_b8 %6, %17\n\t"
              "ds_read_b64 %7, %18\n\t"
              "ds_read_b64 %8, %19\n\t"
              "ds_read_b64 %9, %20\n\t"
              "ds_read_b64 %10, %21\n\t"
              "s_waitcnt lgkmcnt(0)"
              : "=&v"(c4), "=&v"(p4), "=&v"(s4), "=&v"(vt[0]), "=&v"(vt[1]), "=&v"(vt[2]), "=&v"(vt[3]),
                "=&v"(pbv[0]), "=&v"(pbv[1]), "=&v"(pbv[2]), "=&v"(pbv[3])
              : "v"(la(&L.corr[sl(it4)][lc][b0])), "v"(la(&L.pmax[sl(it4)][lc][b0])),
                "v"(la(&L.psum[sl(it4)][lc][b0])), "v"(la(vq)), "v"(la(vq + KB * HD)), "v"(la(vq + 2 * KB * HD)),
                "v"(la(vq + 3 * KB * HD)), "v"(la(&L.p8[sl(it4)][b0][lane])), "v"(la(&L.p8[sl(it4)][b0 + 1][lane])),
                "v"(la(&L.p8[sl(it4)][b0 + 2][lane])), "v"(la(&L.p8[sl(it4)][b0 + 3][lane]))
              : "memory");
        } else {  // (16 waves: the asm form's outputs do not fit the registers)
          c4 = *reinterpret_cast<const float4 *>(&L.corr[sl(it4)][lc][b0]);
          p4 = *reinterpret_cast<const float4 *>(&L.pmax[sl(it4)][lc][b0]);
          s4 = *reinterpret_cast<const float4 *>(&L.psum[sl(it4)][lc][b0]);
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            vt[b] = __builtin_amdgcn_ds_read_tr8_b64_v2i32(reinterpret_cast<lds_v2i_ptr>(to_lds(vq + b * (KB * HD))));
            pbv[b] = static_cast<long>(L.p8[sl(it4)][b0 + b][lane]);
          }
        }
        const float crv[4] = {c4.x, c4.y, c4.z, c4.w};
        const float pmv[4] = {p4.x, p4.y, p4.z, p4.w};
        const float psv[4] = {s4.x, s4.y, s4.z, s4.w};
        v4i c[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          long va;
          __builtin_memcpy(&va, &vt[b], sizeof(va));
          c[b] = __builtin_amdgcn_mfma_i32_16x16x32_i8(va, pbv[b], zero4(), 0, 0, 0);
        }
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          if (b0 + b < nbp) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float part = __fmul_rn(static_cast<float>(c[b][i]), pmv[b]);
              res[i] = __fadd_rn(__fmul_rn(res[i], crv[b]), part);
            }
            den = __fadd_rn(__fmul_rn(den, crv[b]), psv[b]);
          }
        }
      }
      if (last_of(it4, gp)) {  // out = res * (1/den); |out| maximum of the tile's 16 dims
        ended = true;
        const bool extra = it4 ? IB.extra : IA.extra;
        const float rd = __fdiv_rn(1.0f, den);
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // a fully masked block adds +0 to res (turning -0 into +0)
          out[i] = __fmul_rn(extra ? __fadd_rn(res[i], 0.0f) : res[i], rd);
          mx = fmaxf(mx, fabsf(out[i]));
          res[i] = 0.0f;
        }
        den = 0.0f;
        LanePair pr = lane_pair16(__float_as_uint(mx));
        mx = fmaxf(__uint_as_float(pr.a), __uint_as_float(pr.b));
        pr = lane_pair32(__float_as_uint(mx));
        mx = fmaxf(__uint_as_float(pr.a), __uint_as_float(pr.b));
        if (lg == 0) L.cmax[sl(it4)][lc][dt] = mx;
      }
    }

    // ---- phase 1 (chunk g): S^T = K . Q^T for each item the block serves ----
    const int nbA = g < G ? nb_of(0, g) : 0, nbB = g < G ? nb_of(1, g) : 0;
    const int j = g * CB + wave;
    wait_vmcnt<0>();  // this wave's copies and K rows of chunk g
    if (wave < nbB) {
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        if (it == 1 || wave < nbA) {
          const Item &I = it ? IB : IA;
          const bool need_mask = j * KB + KB > kv_len || (a.causal && j * KB + KB - 1 > I.pos0);
          const int pos = I.pos0 + lc;
          float bmax = -INFINITY;
#pragma unroll
          for (int kt = 0; kt < 2; ++kt) {
            v4i acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(kop[kt][0], qop[it][0], zero4(), 0, 0, 0);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(kop[kt][1], qop[it][1], acc, 0, 0, 0);
            const float kv[4] = {ksr[kt][0], ksr[kt][1], ksr[kt][2], ksr[kt][3]};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              float x = static_cast<float>(acc[i]);
              x = __fmul_rn(x, kv[i]);
              x = __fmul_rn(x, qsv[it]);
              x = __fmul_rn(x, qk);
              if (need_mask) {
                const int key = j * KB + 16 * kt + 4 * lg + i;
                if (key >= kv_len || (a.causal && key > pos)) x = -INFINITY;
              }
              s[it][kt][i] = x;
              bmax = fmaxf(bmax, x);
            }
          }
          LanePair pr = lane_pair16(__float_as_uint(bmax));
          bmax = fmaxf(__uint_as_float(pr.a), __uint_as_float(pr.b));
          pr = lane_pair32(__float_as_uint(bmax));
          bmax = fmaxf(__uint_as_float(pr.a), __uint_as_float(pr.b));
          if (lg == 0) L.bm[sl(it)][lc][wave] = bmax;
        }
      }
    }
    lds_barrier();  // B1(g)

    // ---- int8 store of item it4 if it ended with chunk g - 1 ----
    if (ended) {
      const Item &E = it4 ? IB : IA;
      const float4 c0 = *reinterpret_cast<const float4 *>(&L.cmax[sl(it4)][lc][0]);
      const float4 c1 = *reinterpret_cast<const float4 *>(&L.cmax[sl(it4)][lc][4]);
      const float mx = fmaxf(fmaxf(fmaxf(c0.x, c0.y), fmaxf(c0.z, c0.w)), fmaxf(fmaxf(c1.x, c1.y), fmaxf(c1.z, c1.w)));
      const float scale = __fmul_rn(mx, inv127());
      const double y = rcp64(scale);
      if (lc < E.nr) {
        const int64_t row = E.qi + lc;
        const int col = h * HD + 16 * dt + 4 * lg;
        if (a.attn) {
          float *dst = a.attn + row * a.ld_attn + col;
#pragma unroll
          for (int i = 0; i < 4; ++i) dst[i] = out[i];
        }
        int8_t *o = a.o8 + row * a.ldo + col;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = static_cast<int8_t>(quant_rcp(out[i], y));
        if (dt == 0 && lg == 0) a.os[row * a.ldos + h * a.os_col] = scale;
      }
    }
    if (g == G) break;

    // ---- V rows of chunk g + 1 (V(g - 1)'s half was last read before B1(g)) ----
    copy_v(g + 1, page);

    // ---- phase 2: prefix max of the block maxima, per item, in block order ----
    // (each wave folds up to its own block; all blocks only when the item's
    // walk goes on into another chunk, which starts from the chunk's maximum)
    float m_prev[2], m_mine[2];
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int nb = it ? nbB : nbA;
      float m = g == 0 ? -3.402823466e38f : m_run[it];
      const bool carry = (it ? nB : nA) > (g + 1) * CB;
      const float *bmr = L.bm[sl(it)][lc];
#pragma unroll
      for (int b = 0; b < CB; ++b)
        if (b < min(wave, nb)) m = (m > bmr[b]) ? m : bmr[b];
      m_prev[it] = m_mine[it] = m;
      if (wave < nb) {
        m = (m > bmr[wave]) ? m : bmr[wave];
        m_mine[it] = m;
      }
      if (carry) {
#pragma unroll
        for (int b = 1; b < CB; ++b)
          if (b > wave && b < nb) m = (m > bmr[b]) ? m : bmr[b];
        m_run[it] = m;
      }
    }

    // ---- phase 3: corr, P, psum, P8 of this wave's block, per item ----
    if (wave < nbB) {
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        if (it == 1 || wave < nbA) {
          const float corr = exp_f32_le0_tab(__fsub_rn(m_prev[it], m_mine[it]), L.etab);
          float p[2][4];
#pragma unroll
          for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) p[kt][i] = exp_f32_le0_tab(__fsub_rn(s[it][kt][i], m_mine[it]), L.etab);
          // tree_sum over the 32 keys (key = 16 kt + 4 lg + i): bits 0-1 in
          // registers, bit 2 = lane bit 4, bit 3 = lane bit 5, bit 4 = kt
          float t[2];
#pragma unroll
          for (int kt = 0; kt < 2; ++kt) {
            const float a0 = __fadd_rn(p[kt][0], p[kt][1]);
            const float a1 = __fadd_rn(p[kt][2], p[kt][3]);
            float u = __fadd_rn(a0, a1);
            LanePair q = lane_pair16(__float_as_uint(u));
            u = __fadd_rn(__uint_as_float(q.a), __uint_as_float(q.b));
            q = lane_pair32(__float_as_uint(u));
            t[kt] = __fadd_rn(__uint_as_float(q.a), __uint_as_float(q.b));
          }
          const float psum = __fadd_rn(t[0], t[1]);
          // pv = P * vs (keys past kv_len: vs taken as 0, P is 0 there)
          float pmx = 0.0f;
#pragma unroll
          for (int kt = 0; kt < 2; ++kt) {
            const float vv[4] = {vsr[kt][0], vsr[kt][1], vsr[kt][2], vsr[kt][3]};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int key = j * KB + 16 * kt + 4 * lg + i;
              p[kt][i] = __fmul_rn(p[kt][i], key < kv_len ? vv[i] : 0.0f);
              pmx = fmaxf(pmx, p[kt][i]);
            }
          }
          LanePair pr = lane_pair16(__float_as_uint(pmx));
          pmx = fmaxf(__uint_as_float(pr.a), __uint_as_float(pr.b));
          pr = lane_pair32(__float_as_uint(pmx));
          pmx = fmaxf(__uint_as_float(pr.a), __uint_as_float(pr.b));
          const float pmax = __fmul_rn(pmx, inv127());
          const double y = rcp64(pmax);
          uint32_t w8[2];
          if (__builtin_amdgcn_ballot_w64(!(pmax >= 1.17549435e-38f)) == 0) {
            // every row's pmax is normal: x / pmax <= 127 * (1 + 2^-23) for
            // x <= absmax, so rne alone lands in [0, 127]
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
              int qv[4];
#pragma unroll
              for (int i = 0; i < 4; ++i)
                qv[i] = static_cast<int>(rintf(__double2float_rn(__dmul_rn(static_cast<double>(p[kt][i]), y))));
              w8[kt] = pack4(qv[0], qv[1], qv[2], qv[3]);
            }
          } else {
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
              w8[kt] = pack4(quant_rcp_pos(p[kt][0], y), quant_rcp_pos(p[kt][1], y), quant_rcp_pos(p[kt][2], y),
                             quant_rcp_pos(p[kt][3], y));
          }
          L.p8[sl(it)][wave][lane] = (static_cast<uint64_t>(w8[1]) << 32) | w8[0];
          if (lg == 0) {
            L.corr[sl(it)][lc][wave] = corr;
            L.psum[sl(it)][lc][wave] = psum;
            L.pmax[sl(it)][lc][wave] = pmax;
          }
        }
        __builtin_amdgcn_sched_barrier(0);  // one unit at a time: bounds the live exp chains
      }
    }
    // K rows, Q rows and ks | vs of chunk g + 1 (their registers were last
    // read above)
    load_k(g + 1, page);
    load_q(g + 1);
    load_sc(g + 1, page);
    page = page_of(g + 2);
    lds_barrier();  // B2(g)
  }
}

}  // namespace

bool attn_prefill_supported(const AttnArgs &a) {
  return a.blk_page_n >= 0 && a.blk_page_n <= 32 && a.page_tokens >= KB && (a.page_tokens & (a.page_tokens - 1)) == 0 && a.row_bytes % 16 == 0 &&
         a.row_bytes * a.page_tokens < (int64_t{1} << 31) && a.scale_row_bytes * a.page_tokens < (int64_t{1} << 31) &&
         a.kv_heads > 0 && a.heads % a.kv_heads == 0 && a.scale_row_bytes % 4 == 0 &&
         a.scale_page_bytes % 4 == 0;
}

hipError_t launch_attn_prefill(const AttnArgs &a, hipStream_t s) {
  if (a.rows <= 0) return hipSuccess;
  if (!attn_prefill_supported(a)) return hipErrorInvalidValue;
  // Q3_PREFILL_ATTN=pair: both blocks of a causal pair in one 16-wave
  // workgroup (a measured alternative; read at every launch)
  const char *ev = std::getenv("Q3_PREFILL_ATTN");
  const bool pair = ev && std::strcmp(ev, "pair") == 0;
  static bool attr_set[2] = {false, false};  // more than 64 KiB of dynamic LDS must be allowed once
  const int nqb = (a.rows + QB - 1) / QB;
  if (pair) {
    if (!attr_set[1]) {
      for (const void *f : {reinterpret_cast<const void *>(&attn_prefill_kernel<2, 16, 8>),
                            reinterpret_cast<const void *>(&attn_prefill_kernel<2, 0, 0>)}) {
        const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, sizeof(Lds<2>));
        if (e != hipSuccess) return e;
      }
      attr_set[1] = true;
    }
    if (head_consts(a.heads, a.kv_heads))
      Q3_LAUNCH((attn_prefill_kernel<2, 16, 8>), dim3(a.heads, (nqb + 1) / 2), dim3(Cfg<2>::NW * 64), sizeof(Lds<2>),
                s, a);
    else
      Q3_LAUNCH((attn_prefill_kernel<2, 0, 0>), dim3(a.heads, (nqb + 1) / 2), dim3(Cfg<2>::NW * 64), sizeof(Lds<2>),
                s, a);
  } else {
    if (!attr_set[0]) {
      for (const void *f : {reinterpret_cast<const void *>(&attn_prefill_kernel<1, 16, 8>),
                            reinterpret_cast<const void *>(&attn_prefill_kernel<1, 0, 0>)}) {
        const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, sizeof(Lds<1>));
        if (e != hipSuccess) return e;
      }
      attr_set[0] = true;
    }
    if (head_consts(a.heads, a.kv_heads))
      Q3_LAUNCH((attn_prefill_kernel<1, 16, 8>), dim3(a.heads, nqb), dim3(Cfg<1>::NW * 64), sizeof(Lds<1>), s, a);
    else
      Q3_LAUNCH((attn_prefill_kernel<1, 0, 0>), dim3(a.heads, nqb), dim3(Cfg<1>::NW * 64), sizeof(Lds<1>), s, a);
  }
  return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs &a, hipStream_t s) {
  // Q3_PREFILL_ATTN=walk: the block-order walk (k_attention.hip) even where
  // the phase-parallel kernel applies (read at every launch); page sizes the
  // latter does not take (not a power of two) always walk
  const char *ev = std::getenv("Q3_PREFILL_ATTN");
  const bool walk = ev && std::strcmp(ev, "walk") == 0;
  if (walk || !attn_prefill_supported(a)) return launch_attention_walk(a, s);
  return launch_attn_prefill(a, s);
}

}  // namespace q3
