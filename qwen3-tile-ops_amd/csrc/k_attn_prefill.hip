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
// prefix max of the block maxima.  So per chunk of up to CB = 8 blocks:
//   phase 1 (one wave per block)   S_j, s, block maximum bm_j
//   phase 2 (every lane, tiny)     nmm_j = max(nmm_{j-1}, bm_j), in block order
//   phase 3 (one wave per block)   corr_j, P, psum_j, pv, pmax_j, P8_j
//   phase 4 (one wave per 16 dims) res = res * corr_j + f32(P8_j . V_j) * pmax_j
//                                  for j in order (den likewise in wave 0)
// with the reference's rounding points, so the result equals the one-block
// walk bit for bit.  Chunks carry (maximum, den, res) the way blocks do.
//
// Work: a workgroup (8 waves) owns one query head and two 16-row query
// blocks qb and nqb - 1 - qb, walked one after the other, so that under the
// causal mask every workgroup has about the same number of key blocks.
// K/V stream through two halves of an LDS ring (one chunk each) with
// global_load_lds: a wave copies the block it computes in phases 1 and 3,
// and the copies of chunk g + 1 are issued while chunk g is in phases 3-4.
//
// Layouts (lane = lc + 16 lg):
//   S^T_j = K_j . Q^T with v_mfma_i32_16x16x64_i8, keys as the M dimension:
//     lane holds s[kt][i] for key 16 kt + 4 lg + i, query row lc, so a
//     key reduction is 2 in-register levels, 2 lane swaps (lg) and the kt
//     pair, in the reference's pairwise-tree order.
//   P8_j stays in that lane as the A operand of v_mfma_i32_16x16x32_i8
//     (byte m = 4 kt + i is key 16 kt + 4 lg + i); the V operand carries the
//     same key order and is read with ds_read_b64_tr_b8 (gfx950's transposing
//     LDS load: in each 16-lane group, result lane i byte j is byte i & 7 of
//     the 8 bytes addressed by source lane 2 j + (i >> 3)), so no transposed
//     copy of V is ever built.
//   K stage  [32 keys][8 x 16 B], chunk c of key r at c ^ (r & 7)
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

constexpr int NW = 8;    // waves per workgroup
constexpr int CB = 8;    // key blocks per chunk (one per wave in phases 1 and 3)
constexpr int QB = 16;   // query rows per item
constexpr int KB = 32;   // keys per block (= reference block)
constexpr int HD = 128;

struct Stage {
  int8_t k[KB * HD];
  int8_t v[KB * HD];
  float sc[2 * KB];  // ks[0..31] | vs[0..31]
};

struct Lds {
  Stage stg[2][CB];
  uint64_t p8[CB][64];  // P8 of each block of the chunk, in A-operand lane order
  float bm[QB][CB];     // block maxima [row][block]
  float corr[CB][QB], psum[CB][QB], pmax[CB][QB];
  float cmax[QB][NW];   // output absmax of each wave's 16 dims
  float rd[QB];         // 1 / den
  uint64_t etab[32];
};

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

__device__ __forceinline__ Item make_item(const AttnArgs &a, int qb, int kv_len) {
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

// quant(x, scale) = sat127(rne(RN(x / scale))) (ref_qwen3.py:69-76) with
// y = RN64(1 / scale): RN32(x * y in f64) = RN32(x / scale), since a quotient
// of two f32 is never an f32 rounding midpoint and stays at least 2^-50 (relative)
// away from every midpoint, while x * y is within 2^-52 of x / scale.  Quotients
// where the f32 rounding is not the normal one (subnormal: rne gives 0 either
// way; overflow: both saturate) and scale = 0 (y = inf, 0 * inf = NaN -> 0,
// x * inf = inf -> 127) give the same int8 as the division.
__device__ __forceinline__ int quant_rcp(float x, double y) {
  const float q = __double2float_rn(__dmul_rn(static_cast<double>(x), y));
  float r = (q != q) ? 0.0f : rintf(q);
  r = fminf(127.0f, fmaxf(-127.0f, r));
  return static_cast<int>(r);
}

__device__ __forceinline__ uint32_t pack4(int b0, int b1, int b2, int b3) {
  return (static_cast<uint32_t>(b0) & 0xffu) | ((static_cast<uint32_t>(b1) & 0xffu) << 8) |
         ((static_cast<uint32_t>(b2) & 0xffu) << 16) | (static_cast<uint32_t>(b3) << 24);
}

__global__ void __launch_bounds__(NW * 64) attn_prefill_kernel(AttnArgs a) {
  extern __shared__ __align__(16) int8_t smem[];
  Lds &L = *reinterpret_cast<Lds *>(smem);

  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int lc = lane & 15;
  const int lg = lane >> 4;
  const int h = blockIdx.x;
  const int kvh = h / (a.heads / a.kv_heads);
  int kv_len = static_cast<int>(a.kv_len);
  if (a.kv_len_dev) kv_len += *a.kv_len_dev;
  const int nqb = (a.rows + QB - 1) / QB;
  const int qbA = blockIdx.y, qbB = nqb - 1 - static_cast<int>(blockIdx.y);
  const int n_items = qbB > qbA ? 2 : 1;
  const Item itA = make_item(a, qbA, kv_len);
  const Item itB = make_item(a, n_items > 1 ? qbB : qbA, kv_len);
  const int nchA = (itA.nblk + CB - 1) / CB;
  const int nch = nchA + (n_items > 1 ? (itB.nblk + CB - 1) / CB : 0);

  // chunk g -> (item, first block, blocks)
  auto chunk_item = [&](int g) { return g < nchA ? 0 : 1; };
  auto chunk_cb = [&](int g) { return (g < nchA ? g : g - nchA) * CB; };
  auto chunk_nb = [&](int g) {
    const int nb = (g < nchA ? itA.nblk : itB.nblk) - chunk_cb(g);
    return min(CB, nb);
  };
  // page id of the block this wave copies in chunk g (uniform)
  auto page_of = [&](int g) -> uint32_t {
    if (g >= nch || wave >= chunk_nb(g)) return 0;
    const uint32_t key0 = static_cast<uint32_t>((chunk_cb(g) + wave) * KB);
    return a.table[key0 / a.page_tokens];
  };
  // copies of this wave's block of chunk g: 4 x K, 4 x V, 1 x scales
  auto issue = [&](int g, uint32_t page) {
    if (g >= nch || wave >= chunk_nb(g)) return;
    Stage &st = L.stg[g & 1][wave];
    const uint32_t slot0 = static_cast<uint32_t>((chunk_cb(g) + wave) * KB) % a.page_tokens;
    const int8_t *kb = a.k + page * a.page_bytes + slot0 * a.row_bytes + kvh * HD;
    const int8_t *vb = a.v + page * a.page_bytes + slot0 * a.row_bytes + kvh * HD;
    const int phys = lane & 7;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int key = 8 * t + (lane >> 3);
      const int8_t *kp = kb + key * a.row_bytes + (phys ^ (key & 7)) * 16;
      const int8_t *vp = vb + key * a.row_bytes + (phys ^ vswz(key)) * 16;
      __builtin_amdgcn_global_load_lds(const_cast<int8_t *>(kp), to_lds(st.k + t * 1024), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(const_cast<int8_t *>(vp), to_lds(st.v + t * 1024), 16, 0, 0);
    }
    const float *sbase = lane < 32 ? a.ks : a.vs;
    const int8_t *sp = reinterpret_cast<const int8_t *>(sbase) + page * a.scale_page_bytes +
                       (slot0 + (lane & 31)) * a.scale_row_bytes + kvh * 4;
    __builtin_amdgcn_global_load_lds(const_cast<int8_t *>(sp), to_lds(st.sc), 4, 0, 0);
  };

  // ---- prologue: first chunk's copies, Q operands of both items ----
  uint32_t pg_next = page_of(1);
  issue(0, page_of(0));
  if (threadIdx.x == 0) stage_exp2_table(L.etab);
  v4i qA[2], qB[2];
  float qsA, qsB;
  {
    const int8_t *q = a.q8 + h * HD + 16 * lg;
    const int rA = itA.qi + lc, rB = itB.qi + lc;
    const bool okA = lc < itA.nr, okB = lc < itB.nr;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      qA[ks] = okA ? *reinterpret_cast<const v4i *>(q + static_cast<int64_t>(rA) * a.ldq + 64 * ks) : zero4();
      qB[ks] = okB ? *reinterpret_cast<const v4i *>(q + static_cast<int64_t>(rB) * a.ldq + 64 * ks) : zero4();
    }
    qsA = okA ? a.qs[static_cast<int64_t>(rA) * a.ldqs + h * a.qs_col] : 0.0f;
    qsB = okB ? a.qs[static_cast<int64_t>(rB) * a.ldqs + h * a.qs_col] : 0.0f;
  }

  // transposing-read address of this lane inside a V stage, for dims 16 wave..+15
  int v_tr_off;
  {
    const int g4 = lane >> 4, jj = (lane & 15) >> 1, hh = lane & 1;
    const int key = 16 * (jj >> 2) + 4 * g4 + (jj & 3);
    v_tr_off = key * HD + ((wave ^ vswz(key)) << 4) + 8 * hh;
  }

  const float qk = a.qk_scale;
  float m_run = -3.402823466e38f;  // carried maximum of row lc
  float res[4], den[4];           // rows 4 lg + i, dim 16 wave + lc
#pragma unroll
  for (int i = 0; i < 4; ++i) res[i] = den[i] = 0.0f;

  for (int g = 0; g < nch; ++g) {
    const int it = chunk_item(g);
    const Item &I = it ? itB : itA;
    const int cb = chunk_cb(g);
    const int nb = chunk_nb(g);
    const bool mine = wave < nb;  // this wave owns block cb + wave
    const int j = cb + wave;
    Stage &st = L.stg[g & 1][wave];
    wait_vmcnt<0>();  // this wave's copies of chunk g (the next chunk is not issued yet)

    // ---- phase 1: S^T = K . Q^T, scaled and masked, block maximum ----
    float s[2][4];
    if (mine) {
      const v4i q0 = it ? qB[0] : qA[0];
      const v4i q1 = it ? qB[1] : qA[1];
      const float qs = it ? qsB : qsA;
      v4i acc[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const int key = 16 * kt + lc;
        const v4i k0 = *reinterpret_cast<const v4i *>(st.k + key * HD + ((lg) ^ (key & 7)) * 16);
        const v4i k1 = *reinterpret_cast<const v4i *>(st.k + key * HD + ((4 + lg) ^ (key & 7)) * 16);
        acc[kt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(k0, q0, zero4(), 0, 0, 0);
        acc[kt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(k1, q1, acc[kt], 0, 0, 0);
      }
      const bool need_mask = j * KB + KB > kv_len || (a.causal && j * KB + KB - 1 > I.pos0);
      const int pos = I.pos0 + lc;
      float bmax = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const float4 ksc = *reinterpret_cast<const float4 *>(&st.sc[16 * kt + 4 * lg]);
        const float kv[4] = {ksc.x, ksc.y, ksc.z, ksc.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float x = static_cast<float>(acc[kt][i]);
          x = __fmul_rn(x, kv[i]);
          x = __fmul_rn(x, qs);
          x = __fmul_rn(x, qk);
          if (need_mask) {
            const int key = j * KB + 16 * kt + 4 * lg + i;
            if (key >= kv_len || (a.causal && key > pos)) x = -INFINITY;
          }
          s[kt][i] = x;
          bmax = fmaxf(bmax, x);
        }
      }
      LanePair pr = lane_pair16(__float_as_uint(bmax));
      bmax = fmaxf(__uint_as_float(pr.a), __uint_as_float(pr.b));
      pr = lane_pair32(__float_as_uint(bmax));
      bmax = fmaxf(__uint_as_float(pr.a), __uint_as_float(pr.b));
      if (lg == 0) L.bm[lc][wave] = bmax;
    }
    lds_barrier();

    // ---- copies of chunk g + 1 (its half was last read in chunk g - 1) ----
    issue(g + 1, pg_next);
    pg_next = page_of(g + 2);

    // ---- phase 2: prefix max of the block maxima in block order ----
    float m_prev = m_run, m_mine = m_run;
    {
      const float4 b0 = *reinterpret_cast<const float4 *>(&L.bm[lc][0]);
      const float4 b1 = *reinterpret_cast<const float4 *>(&L.bm[lc][4]);
      const float bmv[CB] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
      float m = m_run;
#pragma unroll
      for (int b = 0; b < CB; ++b) {
        if (b < nb) {
          const float nm = (m > bmv[b]) ? m : bmv[b];
          if (b == wave) {
            m_prev = m;
            m_mine = nm;
          }
          m = nm;
        }
      }
      m_run = m;
    }

    // ---- phase 3: corr, P, psum, P8 of this wave's block ----
    if (mine) {
      const float corr = exp_f32_le0_tab(__fsub_rn(m_prev, m_mine), L.etab);
      float p[2][4];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) p[kt][i] = exp_f32_le0_tab(__fsub_rn(s[kt][i], m_mine), L.etab);
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
        const float4 vsc = *reinterpret_cast<const float4 *>(&st.sc[KB + 16 * kt + 4 * lg]);
        const float vv[4] = {vsc.x, vsc.y, vsc.z, vsc.w};
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
      const double y = __ddiv_rn(1.0, static_cast<double>(pmax));
      uint32_t w8[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
        w8[kt] = pack4(quant_rcp(p[kt][0], y), quant_rcp(p[kt][1], y), quant_rcp(p[kt][2], y),
                       quant_rcp(p[kt][3], y));
      L.p8[wave][lane] = (static_cast<uint64_t>(w8[1]) << 32) | w8[0];
      if (lg == 0) {
        L.corr[wave][lc] = corr;
        L.psum[wave][lc] = psum;
        L.pmax[wave][lc] = pmax;
      }
    }
    lds_barrier();

    // ---- phase 4: res = res * corr_j + f32(P8_j . V_j) * pmax_j, j in order ----
    {
      const int8_t *vbase = &L.stg[g & 1][0].v[0];
#pragma unroll
      for (int b = 0; b < CB; ++b) {
        if (b < nb) {
          const long pa = static_cast<long>(L.p8[b][lane]);
          const v2i vt = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
              reinterpret_cast<lds_v2i_ptr>(to_lds(vbase + b * sizeof(Stage) + v_tr_off)));
          long vb;
          __builtin_memcpy(&vb, &vt, sizeof(vb));
          const v4i c = __builtin_amdgcn_mfma_i32_16x16x32_i8(pa, vb, zero4(), 0, 0, 0);
          const float4 cr = *reinterpret_cast<const float4 *>(&L.corr[b][4 * lg]);
          const float4 pm = *reinterpret_cast<const float4 *>(&L.pmax[b][4 * lg]);
          const float crv[4] = {cr.x, cr.y, cr.z, cr.w};
          const float pmv[4] = {pm.x, pm.y, pm.z, pm.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float part = __fmul_rn(static_cast<float>(c[i]), pmv[i]);
            res[i] = __fadd_rn(__fmul_rn(res[i], crv[i]), part);
          }
          if (wave == 0) {
            const float4 ps = *reinterpret_cast<const float4 *>(&L.psum[b][4 * lg]);
            const float psv[4] = {ps.x, ps.y, ps.z, ps.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) den[i] = __fadd_rn(__fmul_rn(den[i], crv[i]), psv[i]);
          }
        }
      }
    }

    // ---- end of an item: out = res * (1/den), per-head int8 quantisation ----
    const bool item_end = (g + 1 == nch) || (chunk_item(g + 1) != it);
    if (item_end) {
      if (wave == 0 && lc == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) L.rd[4 * lg + i] = __fdiv_rn(1.0f, den[i]);
      }
      lds_barrier();
      const float4 rd4 = *reinterpret_cast<const float4 *>(&L.rd[4 * lg]);
      const float rdv[4] = {rd4.x, rd4.y, rd4.z, rd4.w};
      float out[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // a fully masked block adds +0 to res (turning -0 into +0)
        const float r = I.extra ? __fadd_rn(res[i], 0.0f) : res[i];
        out[i] = __fmul_rn(r, rdv[i]);
        float m = fabsf(out[i]);
        m = fmaxf(m, lane_xor<1>(m));
        m = fmaxf(m, lane_xor<2>(m));
        m = fmaxf(m, lane_xor<4>(m));
        m = fmaxf(m, lane_xor<8>(m));
        if (lc == 0) L.cmax[4 * lg + i][wave] = m;
      }
      lds_barrier();
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * lg + i;
        const float4 c0 = *reinterpret_cast<const float4 *>(&L.cmax[r][0]);
        const float4 c1 = *reinterpret_cast<const float4 *>(&L.cmax[r][4]);
        const float mx = fmaxf(fmaxf(fmaxf(c0.x, c0.y), fmaxf(c0.z, c0.w)), fmaxf(fmaxf(c1.x, c1.y), fmaxf(c1.z, c1.w)));
        if (r < I.nr) {
          const int64_t row = I.qi + r;
          const int col = h * HD + 16 * wave + lc;
          if (a.attn) a.attn[row * a.ld_attn + col] = out[i];
          const float scale = __fmul_rn(mx, inv127());
          a.o8[row * a.ldo + col] = static_cast<int8_t>(quant1(out[i], scale));
          if (wave == 0 && lc == 0) a.os[row * a.ldos + h * a.os_col] = scale;
        }
        res[i] = den[i] = 0.0f;
      }
      m_run = -3.402823466e38f;
    }
  }
}

}  // namespace

bool attn_prefill_supported(const AttnArgs &a) {
  return a.page_tokens % KB == 0 && a.row_bytes % 16 == 0 && a.kv_heads > 0 && a.heads % a.kv_heads == 0 &&
         a.scale_row_bytes % 4 == 0 && a.scale_page_bytes % 4 == 0;
}

hipError_t launch_attn_prefill(const AttnArgs &a, hipStream_t s) {
  if (a.rows <= 0) return hipSuccess;
  if (!attn_prefill_supported(a)) return hipErrorInvalidValue;
  static bool attr_set = false;  // more than 64 KiB of dynamic LDS must be allowed once
  if (!attr_set) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&attn_prefill_kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, sizeof(Lds));
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int nqb = (a.rows + QB - 1) / QB;
  const dim3 grid(a.heads, (nqb + 1) / 2);
  Q3_LAUNCH(attn_prefill_kernel, grid, dim3(NW * 64), sizeof(Lds), s, a);
  return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs &a, hipStream_t s) {
  static const bool walk = [] {
    const char *e = std::getenv("Q3_PREFILL_ATTN");
    return e && std::strcmp(e, "walk") == 0;
  }();
  if (walk || !attn_prefill_supported(a)) return launch_attention_walk(a, s);
  return launch_attn_prefill(a, s);
}

}  // namespace q3
