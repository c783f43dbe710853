// Paged hd128 GQA attention with the reference's block-quantised online
// softmax (prefill and any multi-row chunk).
//
//   kernels/attention_gqa.h:404-572 attention_heads_gqa_tokscale_paged /
//                                   attention_head_hd128_blocks_paged
//   ref_qwen3.py:210-289            attention_head_blocks / ..._gqa_tokscale
//
// Per (head, 32-row query block) and per 32-key block j, in key order:
//   S   = q8 . k8^T (int32, exact)            -> ((f32 S * ks) * qs) * qk
//   mask keys with (col - row) > pos0 - j     -> -inf
//   nmm = max(tree_max(S), maximum); corr = exp(maximum - nmm)
//   den = den * corr; res = res * corr; P = exp(S - nmm); den += tree_sum(P)
//   P  *= vs; pmax = absmax(P) * (1/127); P8 = quant(P, pmax)
//   res += f32(P8 . V) * pmax
// then out = res * (1/den) and per-head int8 quantisation of out.
//
// Workgroup = 4 waves on one (head, 16-row query block).  The key blocks are
// walked in pairs and streamed through NS LDS stages with global_load_lds
// copies issued two pairs ahead, so a pair's K, V and scales are resident
// when its turn comes.  Within a pair the scores (waves 0-1: first block,
// waves 2-3: second), the softmax chains and the P8.V products of the two
// blocks run side by side; the carried state (maximum, den, res) is updated
// block by block in the reference's order, the second block starting from
// the first block's maximum, so the result equals the one-block walk (an
// odd last block is walked alone).  The blocks' page ids are read once into
// LDS.
//   K stage  [32 keys][128] int8, 16-byte chunks XOR-swizzled by key so the
//            MFMA operand reads of 16 keys spread over the LDS banks
//   V stage  [32 keys][128] int8, transposed per block into vt [dim][key]
//            (rows padded to 80 bytes) with 4x4 byte transposes (v_perm_b32)
//   scales   ks[32] | vs[32] f32 of the block's keys for this KV head
// S (16x32) and P8.V (16x128) use v_mfma_i32_16x16x64_i8; the 32-key K
// operand of P8.V is zero-padded to 64.  The softmax step gives each
// half-wave one query row, so the block's tree sum is a 32-lane butterfly
// (equal to the reference's pairwise tree, with +0 padding for a partial
// last block); a wave's 2 rows x 2 blocks run side by side.  The work of a
// workgroup is VALU-issue bound (one wave per SIMD), and the causal
// critical path is the last query block, which walks every key block: 16
// rows per workgroup halve that path against 32 (twice the workgroups, two
// per CU).
#include "q3_device.h"
#include "q3_kernels.h"

namespace q3 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i zero4() {
  v4i z = {0, 0, 0, 0};
  return z;
}

constexpr int QB = 16;    // query rows per workgroup
constexpr int KB = 32;    // keys per block (= reference block)
constexpr int HD = 128;
constexpr int LDO = HD + 4;
constexpr int NS = 6;     // LDS stages (copies run NS - 2 blocks ahead of a pair)
constexpr int PGW = 512;  // page ids held in LDS at a time (blocks)
// vt row stride: 64 key bytes + 16 bytes of padding, so that the transpose's
// dword writes of 16 consecutive dims fall in different LDS banks (a 64-byte
// stride puts them all in one) while rows stay 16-byte aligned for the MFMA
// operand reads
constexpr int VTS = 80;

struct Stage {
  int8_t k[KB * HD];
  int8_t v[KB * HD];
  float sc[2 * KB];  // ks[0..31], vs[32..63]
};

// Copies of key block b (its page id in pg) into stage st.  Every wave
// copies a quarter of K and of V (one 16-byte global_load_lds each); wave 0
// also copies the 64 scales (one 4-byte global_load_lds).
__device__ __forceinline__ void issue_block(const AttnArgs &a, Stage &st, uint32_t page, int b,
                                            int kvh, int tid, int wave, int lane) {
  const uint32_t slot0 = static_cast<uint32_t>(b * KB) % a.page_tokens;
  const int key = tid >> 3;
  const int chunk = (tid & 7) ^ (key & 7);
  const int8_t *kp = a.k + page * a.page_bytes + (slot0 + key) * a.row_bytes + kvh * HD + chunk * 16;
  const int8_t *vp = a.v + page * a.page_bytes + (slot0 + key) * a.row_bytes + kvh * HD + (tid & 7) * 16;
  __builtin_amdgcn_global_load_lds(const_cast<int8_t *>(kp), to_lds(st.k + wave * 1024), 16, 0, 0);
  __builtin_amdgcn_global_load_lds(const_cast<int8_t *>(vp), to_lds(st.v + wave * 1024), 16, 0, 0);
  if (wave == 0) {
    const int c = lane & 31;
    const float *sbase = lane < 32 ? a.ks : a.vs;
    const int8_t *sp = reinterpret_cast<const int8_t *>(sbase) + page * a.scale_page_bytes +
                       (slot0 + c) * a.scale_row_bytes + kvh * 4;
    __builtin_amdgcn_global_load_lds(const_cast<int8_t *>(sp), to_lds(st.sc), 4, 0, 0);
  }
}

__global__ void __launch_bounds__(256) attention_kernel(AttnArgs a) {
  __shared__ __align__(16) Stage stg[NS];
  __shared__ int32_t s_i32[2][QB][KB + 1];
  __shared__ __align__(16) int8_t p8[2][QB][64];   // [block of the pair][row][key], keys 32..63 = 0
  __shared__ __align__(16) int8_t vt[2][HD][VTS];  // [block of the pair][dim][key], keys 32..63 = 0
  __shared__ float row_max[QB], row_den[QB], row_corr[2][QB], row_pmax[2][QB], row_qs[QB];
  __shared__ uint64_t etab[32];
  __shared__ uint32_t pg[PGW];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = wave_id();
  const int lr = lane & 15;
  const int lg = lane >> 4;
  const int h = blockIdx.x;
  const int qi = blockIdx.y * QB;
  const int group = a.heads / a.kv_heads;
  const int kvh = h / group;
  uint32_t kv_len = a.kv_len;
  if (a.kv_len_dev) kv_len += static_cast<uint32_t>(*a.kv_len_dev);
  const int nr = min(QB, a.rows - qi);
  const int pos0 = a.causal ? static_cast<int>(kv_len) - a.rows + qi : 0;
  int kv_end = static_cast<int>(kv_len);
  if (a.causal && pos0 + nr < kv_end) kv_end = pos0 + nr;
  const int nblk = (kv_end + KB - 1) / KB;
  const uint32_t ppb = a.page_tokens / KB;  // blocks per page

  // ---- prologue: page ids, exp table, row state, Q fragments ----
  for (int b = tid; b < min(nblk, PGW); b += 256) pg[b] = a.table[static_cast<uint32_t>(b) / ppb];
  if (tid == 0) stage_exp2_table(etab);
  for (int i = tid; i < 2 * QB * 32; i += 256) p8[i / (QB * 32)][(i / 32) % QB][32 + i % 32] = 0;
  for (int i = tid; i < 2 * HD * 32; i += 256) vt[i / (HD * 32)][(i / 32) % HD][32 + i % 32] = 0;
  if (tid < QB) {
    row_max[tid] = -3.402823466e38f;
    row_den[tid] = 0.0f;
    row_qs[tid] = tid < nr ? a.qs[static_cast<int64_t>(qi + tid) * a.ldqs + h * a.qs_col] : 0.0f;
  }
  // Q operand for S: wave w -> block w / 2 of the pair, key n-tile w % 2
  const int s_nt = wave & 1;
  const int s_blk = wave >> 1;
  v4i qa[2];
  {
    const int r = lr;
    for (int ks = 0; ks < 2; ++ks)
      qa[ks] = r < nr ? *reinterpret_cast<const v4i *>(a.q8 + static_cast<int64_t>(qi + r) * a.ldq + h * HD +
                                                       ks * 64 + lg * 16)
                      : zero4();
  }
  // Q fragments complete before the copies start, so the loop's waits only
  // count copies (the compiler would otherwise wait for everything at the
  // first use of qa inside the loop)
  wait_vmcnt<0>();
  __syncthreads();
  for (int b = 0; b < NS - 2 && b < nblk; ++b) issue_block(a, stg[b], pg[b], b, kvh, tid, wave, lane);

  float res[2][4];
  for (int nt = 0; nt < 2; ++nt)
    for (int i = 0; i < 4; ++i) res[nt][i] = 0.0f;

  // page ids of the next PGW blocks (contexts over PGW blocks)
  auto refresh_pages = [&](int bi) {
    for (int b = bi + tid; b < min(nblk, bi + PGW); b += 256) pg[b % PGW] = a.table[static_cast<uint32_t>(b) / ppb];
    __syncthreads();
  };

  // Key blocks in pairs (jb, jb + 1): the pair's scores, softmax chains and
  // P8.V products are computed side by side; the carried state (maximum,
  // den, res) is updated block jb first, then block jb + 1, with the
  // reference's operations, so the result equals the one-block walk.
  for (int jb = 0; jb < nblk; jb += 2) {
    const bool hasB = jb + 1 < nblk;  // uniform
    Stage &sa = stg[jb % NS];
    Stage &sb = stg[(jb + 1) % NS];
    // ---- copies of blocks jb + NS - 2 and jb + NS - 1 (their stages were ----
    // ---- last read by the previous pair)                                 ----
    const int bi = jb + NS - 2;  // even (jb and NS are), so only bi can start a page-id window
    if (bi < nblk && (bi % PGW) == 0) refresh_pages(bi);
    if (bi + 1 < nblk) {
      issue_block(a, stg[bi % NS], pg[bi % PGW], bi, kvh, tid, wave, lane);
      issue_block(a, stg[(bi + 1) % NS], pg[(bi + 1) % PGW], bi + 1, kvh, tid, wave, lane);
      // blocks jb + 2 .. jb + NS - 1 may stay in flight
      if (wave == 0)
        wait_vmcnt<3 * (NS - 2)>();
      else
        wait_vmcnt<2 * (NS - 2)>();
    } else {
      if (bi < nblk) issue_block(a, stg[bi % NS], pg[bi % PGW], bi, kvh, tid, wave, lane);
      wait_vmcnt<0>();
    }
    lds_barrier();

    // ---- S = q8 . k8^T: waves 0, 1 block jb; waves 2, 3 block jb + 1 ----
    // (without a block jb + 1 they read a stale stage; those rows are masked)
    {
      const Stage &st = s_blk ? sb : sa;
      const int key = s_nt * 16 + lr;
      v4i c = zero4();
      for (int ks = 0; ks < 2; ++ks) {
        const int chunk = (ks * 4 + lg) ^ (key & 7);
        const v4i kb = *reinterpret_cast<const v4i *>(st.k + key * HD + chunk * 16);
        c = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa[ks], kb, c, 0, 0, 0);
      }
      for (int i = 0; i < 4; ++i) s_i32[s_blk][lg * 4 + i][s_nt * 16 + lr] = c[i];
    }
    // ---- V blocks -> vt [dim][key]: thread = 4 keys x 4 dims of each ----
    for (int blk = 0; blk < (hasB ? 2 : 1); ++blk) {
      const Stage &st = blk ? sb : sa;
      const int kq = tid >> 5;        // keys 4kq..4kq+3
      const int dq = tid & 31;        // dims 4dq..4dq+3
      const uint32_t w0 = *reinterpret_cast<const uint32_t *>(st.v + (4 * kq + 0) * HD + 4 * dq);
      const uint32_t w1 = *reinterpret_cast<const uint32_t *>(st.v + (4 * kq + 1) * HD + 4 * dq);
      const uint32_t w2 = *reinterpret_cast<const uint32_t *>(st.v + (4 * kq + 2) * HD + 4 * dq);
      const uint32_t w3 = *reinterpret_cast<const uint32_t *>(st.v + (4 * kq + 3) * HD + 4 * dq);
      const uint32_t x01l = __builtin_amdgcn_perm(w1, w0, 0x06020400u);
      const uint32_t x01h = __builtin_amdgcn_perm(w1, w0, 0x07030501u);
      const uint32_t x23l = __builtin_amdgcn_perm(w3, w2, 0x06020400u);
      const uint32_t x23h = __builtin_amdgcn_perm(w3, w2, 0x07030501u);
      *reinterpret_cast<uint32_t *>(&vt[blk][4 * dq + 0][4 * kq]) = __builtin_amdgcn_perm(x23l, x01l, 0x05040100u);
      *reinterpret_cast<uint32_t *>(&vt[blk][4 * dq + 1][4 * kq]) = __builtin_amdgcn_perm(x23h, x01h, 0x05040100u);
      *reinterpret_cast<uint32_t *>(&vt[blk][4 * dq + 2][4 * kq]) = __builtin_amdgcn_perm(x23l, x01l, 0x07060302u);
      *reinterpret_cast<uint32_t *>(&vt[blk][4 * dq + 3][4 * kq]) = __builtin_amdgcn_perm(x23h, x01h, 0x07060302u);
    }
    lds_barrier();

    // ---- online softmax: a half-wave per query row, a wave's 4 rows and ----
    // ---- the pair's two blocks side by side (independent chains        ----
    // ---- interleave); block jb + 1 starts from block jb's maximum       ----
    {
      const int c = lane & 31;
      const int jA = jb * KB, jB = jA + KB;
      const bool kvA = c < min(KB, static_cast<int>(kv_len) - jA);
      const bool kvB = hasB && c < min(KB, static_cast<int>(kv_len) - jB);
      const float kscA = sa.sc[c], kscB = sb.sc[c];
      const float vscA = kvA ? sa.sc[KB + c] : 0.0f;  // keys past kv_len: P = 0, P*vs = 0
      const float vscB = kvB ? sb.sc[KB + c] : 0.0f;
      constexpr int NP = QB / 8;  // rows per half-wave
      int rr[NP];
      float svA[NP], svB[NP], mold[NP];
#pragma unroll
      for (int pass = 0; pass < NP; ++pass) {
        const int r = wave * (2 * NP) + pass * 2 + (lane >> 5);
        rr[pass] = r;
        // read unconditionally (r, c < 32), select afterwards
        float x = static_cast<float>(s_i32[0][r][c]);
        x = __fmul_rn(x, kscA);
        x = __fmul_rn(x, row_qs[r]);
        x = __fmul_rn(x, a.qk_scale);
        const bool mA = !kvA || r >= nr || (a.causal && (c - r) > (pos0 - jA));
        svA[pass] = mA ? -INFINITY : x;
        float y = static_cast<float>(s_i32[1][r][c]);
        y = __fmul_rn(y, kscB);
        y = __fmul_rn(y, row_qs[r]);
        y = __fmul_rn(y, a.qk_scale);
        const bool mB = !kvB || r >= nr || (a.causal && (c - r) > (pos0 - jB));
        svB[pass] = mB ? -INFINITY : y;
        mold[pass] = row_max[r];
      }
      float nmA[NP], nmB[NP], crA[NP], crB[NP], pA[NP], pB[NP], psA[NP], psB[NP], pvA[NP], pvB[NP], pmA[NP],
          pmB[NP];
#pragma unroll
      for (int pass = 0; pass < NP; ++pass) {
        const float bmA = max32(svA[pass]);
        const float bmB = max32(svB[pass]);
        nmA[pass] = (mold[pass] > bmA) ? mold[pass] : bmA;
        nmB[pass] = (nmA[pass] > bmB) ? nmA[pass] : bmB;
      }
#pragma unroll
      for (int pass = 0; pass < NP; ++pass) {
        crA[pass] = exp_f32_le0_tab(__fsub_rn(mold[pass], nmA[pass]), etab);
        crB[pass] = exp_f32_le0_tab(__fsub_rn(nmA[pass], nmB[pass]), etab);
        // masked and missing keys hold -inf: exp gives exactly +0
        pA[pass] = exp_f32_le0_tab(__fsub_rn(svA[pass], nmA[pass]), etab);
        pB[pass] = exp_f32_le0_tab(__fsub_rn(svB[pass], nmB[pass]), etab);
      }
#pragma unroll
      for (int pass = 0; pass < NP; ++pass) {
        psA[pass] = tree_sum32(pA[pass]);
        psB[pass] = tree_sum32(pB[pass]);
        pvA[pass] = __fmul_rn(pA[pass], vscA);
        pvB[pass] = __fmul_rn(pB[pass], vscB);
      }
#pragma unroll
      for (int pass = 0; pass < NP; ++pass) {
        pmA[pass] = __fmul_rn(max32(pvA[pass]), inv127());
        pmB[pass] = __fmul_rn(max32(pvB[pass]), inv127());
      }
#pragma unroll
      for (int pass = 0; pass < NP; ++pass) {
        const int r = rr[pass];
        if (r < nr) {  // whole half-wave agrees on r
          p8[0][r][c] = static_cast<int8_t>(quant1(pvA[pass], pmA[pass]));
          if (hasB) p8[1][r][c] = static_cast<int8_t>(quant1(pvB[pass], pmB[pass]));
          if (c == 0) {
            float den = __fadd_rn(__fmul_rn(row_den[r], crA[pass]), psA[pass]);
            if (hasB) den = __fadd_rn(__fmul_rn(den, crB[pass]), psB[pass]);
            row_den[r] = den;
            row_max[r] = hasB ? nmB[pass] : nmA[pass];
            row_corr[0][r] = crA[pass];
            row_pmax[0][r] = pmA[pass];
            row_corr[1][r] = crB[pass];
            row_pmax[1][r] = pmB[pass];
          }
        }
      }
    }
    lds_barrier();

    // ---- res = res * corr + f32(P8 . V) * pmax, block jb then jb + 1 ----
    for (int blk = 0; blk < (hasB ? 2 : 1); ++blk) {
      const v4i pa = *reinterpret_cast<const v4i *>(&p8[blk][lr][lg * 16]);
      v4i vb[2];
      for (int nt = 0; nt < 2; ++nt)
        vb[nt] = *reinterpret_cast<const v4i *>(&vt[blk][wave * 32 + nt * 16 + lr][lg * 16]);
      for (int nt = 0; nt < 2; ++nt) {
        const v4i c = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa, vb[nt], zero4(), 0, 0, 0);
        for (int i = 0; i < 4; ++i) {
          const int r = lg * 4 + i;  // rows >= nr are never stored
          const float part = __fmul_rn(static_cast<float>(c[i]), row_pmax[blk][r]);
          res[nt][i] = __fadd_rn(__fmul_rn(res[nt][i], row_corr[blk][r]), part);
        }
      }
    }
    lds_barrier();  // s_i32, vt, p8, row state and the pair's stages are rewritten next
  }

  // ---- out = res * (1/den), then per-head int8 quantisation ----
  float(*otile)[LDO] = reinterpret_cast<float(*)[LDO]>(&stg[0]);  // stages are free now
  static_assert(sizeof(float) * QB * LDO <= sizeof(Stage) * NS, "otile fits in the stages");
  for (int nt = 0; nt < 2; ++nt)
    for (int i = 0; i < 4; ++i) {
      const int r = lg * 4 + i;
      if (r < nr) {
        const float rd = __fdiv_rn(1.0f, row_den[r]);
        otile[r][wave * 32 + nt * 16 + lr] = __fmul_rn(res[nt][i], rd);
      }
    }
  __syncthreads();
  for (int r = wave; r < nr; r += 4) {
    const float t0 = otile[r][lane], t1 = otile[r][lane + 64];
    if (a.attn) {
      float *dst = a.attn + static_cast<int64_t>(qi + r) * a.ld_attn + h * HD;
      dst[lane] = t0;
      dst[lane + 64] = t1;
    }
    const float mx = max64(fmaxf(fabsf(t0), fabsf(t1)));
    const float scale = __fmul_rn(mx, inv127());
    int8_t *o = a.o8 + static_cast<int64_t>(qi + r) * a.ldo + h * HD;
    o[lane] = static_cast<int8_t>(quant1(t0, scale));
    o[lane + 64] = static_cast<int8_t>(quant1(t1, scale));
    if (lane == 0) a.os[static_cast<int64_t>(qi + r) * a.ldos + h * a.os_col] = scale;
  }
}

}  // namespace

hipError_t launch_attention_walk(const AttnArgs &a, hipStream_t s) {
  if (a.rows <= 0) return hipSuccess;
  // the stage copies address whole 32-key blocks inside one page
  if (a.page_tokens % KB || a.row_bytes % 16 || a.kv_heads <= 0 || a.heads % a.kv_heads ||
      (a.scale_row_bytes % 4))
    return hipErrorInvalidValue;
  const dim3 grid(a.heads, (a.rows + QB - 1) / QB);
  hipLaunchKernelGGL(attention_kernel, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace q3
