// Paged hd128 GQA attention with the reference's block-quantised online
// softmax.
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
// Workgroup = 4 waves.  S (32x32) and P8.V (32x128) use
// v_mfma_i32_16x16x64_i8; the 32-key K operand of P8.V is zero-padded to
// 64.  The softmax step gives each half-wave one query row, so the block's
// tree sum is a 32-lane butterfly (equal to the reference's pairwise tree,
// with +0 padding for a partial last block).
#include "q3_device.h"
#include "q3_kernels.h"

namespace q3 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i zero4() {
  v4i z = {0, 0, 0, 0};
  return z;
}

constexpr int QB = 32;    // query rows per workgroup
constexpr int KB = 32;    // keys per block (= reference block)
constexpr int HD = 128;
constexpr int LDO = HD + 4;

__global__ void __launch_bounds__(256) attention_kernel(AttnArgs a) {
  __shared__ int32_t s_i32[QB][KB + 1];
  __shared__ __align__(16) int8_t p8[QB][64];     // [row][key], keys 32..63 = 0
  __shared__ __align__(16) int8_t vt[HD][64];     // [dim][key], keys 32..63 = 0
  __shared__ float row_max[QB], row_den[QB], row_corr[QB], row_pmax[QB];
  __shared__ float otile[QB][LDO];

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

  // zero the K padding of the P8 and V^T tiles once
  for (int i = tid; i < QB * 32; i += 256) p8[i / 32][32 + i % 32] = 0;
  for (int i = tid; i < HD * 32; i += 256) vt[i / 32][32 + i % 32] = 0;
  if (tid < QB) {
    row_max[tid] = -3.402823466e38f;
    row_den[tid] = 0.0f;
  }

  // Q operand for S: wave w -> m-tile (w >> 1), n-tile (w & 1)
  const int s_mt = wave >> 1, s_nt = wave & 1;
  v4i qa[2];
  {
    const int r = s_mt * 16 + lr;
    for (int ks = 0; ks < 2; ++ks)
      qa[ks] = (r < nr) ? *reinterpret_cast<const v4i *>(
                              a.q8 + static_cast<int64_t>(qi + r) * a.ldq + h * HD + ks * 64 + lg * 16)
                        : zero4();
  }

  float res[2][2][4];
  for (int mt = 0; mt < 2; ++mt)
    for (int nt = 0; nt < 2; ++nt)
      for (int i = 0; i < 4; ++i) res[mt][nt][i] = 0.0f;

  for (int j = 0; j < kv_end; j += KB) {
    const uint32_t page = a.table[static_cast<uint32_t>(j) / a.page_tokens];
    const uint32_t slot0 = static_cast<uint32_t>(j) % a.page_tokens;
    const int8_t *kbase = a.k + page * a.page_bytes + slot0 * a.row_bytes + kvh * HD;
    const int8_t *vbase = a.v + page * a.page_bytes + slot0 * a.row_bytes + kvh * HD;
    const float *ksb = reinterpret_cast<const float *>(
        reinterpret_cast<const int8_t *>(a.ks) + page * a.scale_page_bytes + slot0 * a.scale_row_bytes);
    const float *vsb = reinterpret_cast<const float *>(
        reinterpret_cast<const int8_t *>(a.vs) + page * a.scale_page_bytes + slot0 * a.scale_row_bytes);
    const int nvalid = min(KB, static_cast<int>(kv_len) - j);

    // ---- S = q8 . k8^T ----
    {
      const int key = s_nt * 16 + lr;
      v4i c = zero4();
      for (int ks = 0; ks < 2; ++ks) {
        const v4i kb = (key < nvalid)
                           ? *reinterpret_cast<const v4i *>(kbase + key * a.row_bytes + ks * 64 + lg * 16)
                           : zero4();
        c = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa[ks], kb, c, 0, 0, 0);
      }
      for (int i = 0; i < 4; ++i) s_i32[s_mt * 16 + lg * 4 + i][s_nt * 16 + lr] = c[i];
    }
    // ---- V block -> LDS, transposed to [dim][key] ----
    {
      const int key = tid >> 3;        // 0..31
      const int d0 = (tid & 7) * 16;   // 0..112
      v4i vv = zero4();
      if (key < nvalid) vv = *reinterpret_cast<const v4i *>(vbase + key * a.row_bytes + d0);
      const int8_t *vb = reinterpret_cast<const int8_t *>(&vv);
      for (int d = 0; d < 16; ++d) vt[d0 + d][key] = vb[d];
    }
    __syncthreads();

    // ---- online softmax, one query row per half-wave ----
    for (int pass = 0; pass < 4; ++pass) {
      const int r = wave * 8 + pass * 2 + (lane >> 5);
      const int c = lane & 31;
      if (r < nr) {  // whole half-wave agrees on r
        const bool kvalid = c < nvalid;
        float s = -INFINITY;
        if (kvalid) {
          s = static_cast<float>(s_i32[r][c]);
          s = __fmul_rn(s, ksb[c * (a.scale_row_bytes / 4) + kvh]);
          s = __fmul_rn(s, a.qs[static_cast<int64_t>(qi + r) * a.ldqs + h * a.qs_col]);
          s = __fmul_rn(s, a.qk_scale);
          if (a.causal && (c - r) > (pos0 - j)) s = -INFINITY;
        }
        const float bmax = max32(s);
        const float mold = row_max[r];
        const float nmm = (mold > bmax) ? mold : bmax;
        const float corr = exp_f32(__fsub_rn(mold, nmm));
        const float p = kvalid ? exp_f32(__fsub_rn(s, nmm)) : 0.0f;
        const float psum = tree_sum32(p);
        float pv = 0.0f;
        if (kvalid) pv = __fmul_rn(p, vsb[c * (a.scale_row_bytes / 4) + kvh]);
        const float pm = __fmul_rn(max32(pv), inv127());
        p8[r][c] = static_cast<int8_t>(quant1(pv, pm));
        if (c == 0) {
          row_den[r] = __fadd_rn(__fmul_rn(row_den[r], corr), psum);
          row_max[r] = nmm;
          row_corr[r] = corr;
          row_pmax[r] = pm;
        }
      }
    }
    __syncthreads();

    // ---- res = res * corr + f32(P8 . V) * pmax ----
    {
      v4i pa[2], vb[2];
      for (int mt = 0; mt < 2; ++mt) pa[mt] = *reinterpret_cast<const v4i *>(&p8[mt * 16 + lr][lg * 16]);
      for (int nt = 0; nt < 2; ++nt)
        vb[nt] = *reinterpret_cast<const v4i *>(&vt[wave * 32 + nt * 16 + lr][lg * 16]);
      for (int mt = 0; mt < 2; ++mt)
        for (int nt = 0; nt < 2; ++nt) {
          const v4i c = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa[mt], vb[nt], zero4(), 0, 0, 0);
          for (int i = 0; i < 4; ++i) {
            const int r = mt * 16 + lg * 4 + i;
            if (r < nr) {
              const float part = __fmul_rn(static_cast<float>(c[i]), row_pmax[r]);
              res[mt][nt][i] = __fadd_rn(__fmul_rn(res[mt][nt][i], row_corr[r]), part);
            }
          }
        }
    }
    __syncthreads();
  }

  // ---- out = res * (1/den), then per-head int8 quantisation ----
  for (int mt = 0; mt < 2; ++mt)
    for (int nt = 0; nt < 2; ++nt)
      for (int i = 0; i < 4; ++i) {
        const int r = mt * 16 + lg * 4 + i;
        if (r < nr) {
          const float rd = __fdiv_rn(1.0f, row_den[r]);
          otile[r][wave * 32 + nt * 16 + lr] = __fmul_rn(res[mt][nt][i], rd);
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

hipError_t launch_attention(const AttnArgs &a, hipStream_t s) {
  if (a.rows <= 0) return hipSuccess;
  const dim3 grid(a.heads, (a.rows + QB - 1) / QB);
  hipLaunchKernelGGL(attention_kernel, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace q3
