// Decode attention (one query row per head) with the block recurrence of
// kernels/attention_gqa.h:404-547 / ref_qwen3.py:210-266, parallelised
// exactly.
//
// The reference walks 32-key blocks in order, carrying (maximum, den, res).
// Only the carried den/res updates are inherently sequential; everything
// else depends on the blocks plus the running maximum, and the running
// maximum is a prefix max of the per-block maxima.  So per chunk of up to
// 24 blocks (768 keys):
//   phase 1 (parallel over blocks)  S_j = q8.k8^T (v_dot4_i32_i8, exact),
//                                   s = ((f32 S * ks) * qs) * qk, block max
//   phase 2 (sequential, tiny)      nmm_j = max(nmm_{j-1}, max_j)
//   phase 3 (parallel over blocks)  corr_j = exp(nmm_{j-1} - nmm_j),
//                                   P = exp(s - nmm_j), psum_j = tree_sum(P),
//                                   P *= vs, pmax_j, P8, PV_j = f32(P8.V) * pmax_j
//   phase 4 (sequential per dim)    den = den*corr_j + psum_j,
//                                   res = res*corr_j + PV_j
// with the same rounding points as the reference, so the result is bit-equal
// to the sequential walk.  Chunks carry (maximum, den, res) like blocks do.
//
// One workgroup per KV head handles its GRP (1 or 2) query heads (GQA), so
// K and V are read once per token per KV head.  8 waves own blocks
// round-robin (at most 3 per chunk each).  The kernel is latency-bound, so
// every global load of a chunk (page-table entries, K and V rows, their
// scales) is issued before any of it is used, V stays in registers from
// phase 1 to phase 3, and the exp table lives in LDS.
//
// Optional prologue (decode fusion): the head epilogues of the new token's
// Q/K/V projection rows (kernels/norm_rope_quant.h:17-86 for Q and K,
// group_gemm.h:173-193 for V) run here, one wave per head.  They write the
// K/V page slot of position kv_len - 1 and the Q int8 row for the record,
// and keep copies in LDS that the attention uses in place of re-reading
// global memory (the first chunk's loads are already in flight by then).
#include "q3_device.h"
#include "q3_kernels.h"

namespace q3 {
namespace {

constexpr int HD = 128;
constexpr int CB = 24;         // blocks per chunk (768 keys)
constexpr int NW = 8;          // waves per workgroup
constexpr int BPW = CB / NW;   // blocks per wave per chunk

__device__ __forceinline__ int sdot4(int a, int b, int c) {
  return __builtin_amdgcn_sdot4(a, b, c, false);
}

template <int GRP>
struct Smem {
  uint64_t tab[32];
  int8_t q8[GRP][HD];
  float qs[GRP];
  int8_t knew[HD], vnew[HD];
  float ksnew, vsnew;
  float s[GRP][CB * 32];  // scores of the chunk
  float bmax[GRP][CB];
  float prev[GRP][CB], nmm[GRP][CB];
  float corr[GRP][CB], psum[GRP][CB];
  float pv[GRP][CB][HD];  // f32(P8.V) * pmax per block
  float run[GRP];
  float absmax[GRP][2];
};

template <int GRP>
__device__ void fused_heads(const AttnArgs &a, Smem<GRP> &sm, int kvh, int wave, int lane) {
  // wave 0: K head kvh, wave 1: V head kvh, waves 2..: Q heads kvh*GRP + h
  if (wave >= 2 + GRP) return;
  const uint32_t t = a.kv_len - 1;  // the new token
  const float *src;
  if (wave == 0)
    src = a.fk + kvh * HD;
  else if (wave == 1)
    src = a.fv + kvh * HD;
  else
    src = a.fq + (kvh * GRP + wave - 2) * HD;
  float t0 = src[lane], t1 = src[lane + 64];
  if (wave != 1)
    head_norm_rope(t0, t1, lane, wave == 0 ? a.nk : a.nq, 1, a.cos_row, a.sin_row, a.inv_hd, true);
  const float mx = max64(fmaxf(fabsf(t0), fabsf(t1)));
  const float scale = __fmul_rn(mx, inv127());
  const int8_t q0 = static_cast<int8_t>(quant1(t0, scale));
  const int8_t q1 = static_cast<int8_t>(quant1(t1, scale));
  int8_t *row8;
  float *sp;
  int8_t *lrow;
  float *lsp;
  if (wave < 2) {
    const uint32_t page = a.table[t / a.page_tokens];
    const uint32_t slot = t % a.page_tokens;
    row8 = const_cast<int8_t *>(wave == 0 ? a.k : a.v) + page * a.page_bytes + slot * a.row_bytes +
           kvh * HD;
    sp = reinterpret_cast<float *>(reinterpret_cast<int8_t *>(const_cast<float *>(wave == 0 ? a.ks : a.vs)) +
                                   page * a.scale_page_bytes + slot * a.scale_row_bytes) + kvh;
    lrow = wave == 0 ? sm.knew : sm.vnew;
    lsp = wave == 0 ? &sm.ksnew : &sm.vsnew;
  } else {
    const int h = wave - 2;
    const int qh = kvh * GRP + h;
    row8 = const_cast<int8_t *>(a.q8) + qh * HD;
    sp = const_cast<float *>(a.qs) + qh * a.qs_col;
    lrow = sm.q8[h];
    lsp = &sm.qs[h];
  }
  row8[lane] = q0;
  row8[lane + 64] = q1;
  lrow[lane] = q0;
  lrow[lane + 64] = q1;
  if (lane == 0) {
    *sp = scale;
    *lsp = scale;
  }
}

template <int GRP>
__global__ void __launch_bounds__(NW * 64) attn_decode_kernel(AttnArgs a) {
  __shared__ __align__(16) Smem<GRP> sm;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int kvh = blockIdx.x;
  const uint32_t kv_len = a.kv_len;
  // one query row: pos0 = kv_len - 1, so kv_end = kv_len and the causal mask
  // only removes keys >= kv_len (attention_gqa.h:454-458)
  const int pos0 = static_cast<int>(kv_len) - 1;
  const int kv_end = static_cast<int>(kv_len);
  const int nblocks = (kv_end + 31) / 32;
  const int sr = static_cast<int>(a.scale_row_bytes / 4);
  const int half = lane & 1;   // phase 1: lane pair (2c, 2c+1) on key c,
  const int kc = lane >> 1;    //   lane parity picks dims [0,64) / [64,128)
  const int d0 = 4 * (lane & 31);   // phase 3: 4 dims per lane,
  const int kh = (lane >> 5) * 16;  //   16 keys per half-wave

  const int ph = tid / HD;  // phase-4 ownership: (head, dim)
  const int pd = tid % HD;
  float res = 0.0f, den = 0.0f;
  int qv[GRP][16];
  float qscale[GRP];

  for (int b0 = 0; b0 < nblocks; b0 += CB) {
    const int nb = min(CB, nblocks - b0);
    // ---- issue every load of this chunk ----
    int kw[BPW][16], vw[BPW][16];
    float kscale[BPW], vscale[BPW];
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
      const int jb = wave + NW * i;
      kscale[i] = 0.0f;
      vscale[i] = 0.0f;
#pragma unroll
      for (int e = 0; e < 16; ++e) kw[i][e] = vw[i][e] = 0;
      if (jb >= nb) continue;
      const int j = (b0 + jb) * 32;
      const uint32_t page = a.table[static_cast<uint32_t>(j) / a.page_tokens];
      const uint32_t slot0 = static_cast<uint32_t>(j) % a.page_tokens;
      const int8_t *kb = a.k + page * a.page_bytes + slot0 * a.row_bytes + kvh * HD;
      const int8_t *vb = a.v + page * a.page_bytes + slot0 * a.row_bytes + kvh * HD;
      const int8_t *ksb = reinterpret_cast<const int8_t *>(a.ks) + page * a.scale_page_bytes +
                          slot0 * a.scale_row_bytes;
      const int8_t *vsb = reinterpret_cast<const int8_t *>(a.vs) + page * a.scale_page_bytes +
                          slot0 * a.scale_row_bytes;
      if (j + kc < kv_end) {
        const int4 *kp = reinterpret_cast<const int4 *>(kb + kc * a.row_bytes + half * 64);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int4 v = kp[e];
          kw[i][4 * e] = v.x;
          kw[i][4 * e + 1] = v.y;
          kw[i][4 * e + 2] = v.z;
          kw[i][4 * e + 3] = v.w;
        }
        kscale[i] = reinterpret_cast<const float *>(ksb + kc * a.scale_row_bytes)[kvh];
      }
#pragma unroll
      for (int cc = 0; cc < 16; ++cc)
        if (j + kh + cc < kv_end)
          vw[i][cc] = *reinterpret_cast<const int *>(vb + (kh + cc) * a.row_bytes + d0);
      if (j + (lane & 31) < kv_end)
        vscale[i] = reinterpret_cast<const float *>(vsb + (lane & 31) * a.scale_row_bytes)[kvh];
    }
    if (b0 == 0) {
      // ---- prologue (overlaps the loads above) ----
      if (tid < 32) sm.tab[tid] = kExp2Tab[tid];
      if (tid < GRP) sm.run[tid] = -3.402823466e38f;
      if (a.fuse_heads) {
        fused_heads<GRP>(a, sm, kvh, wave, lane);
      } else if (wave < GRP) {
        const int qh = kvh * GRP + wave;
        sm.q8[wave][lane] = a.q8[qh * HD + lane];
        sm.q8[wave][lane + 64] = a.q8[qh * HD + lane + 64];
        if (lane == 0) sm.qs[wave] = a.qs[qh * a.qs_col];
      }
      __syncthreads();
#pragma unroll
      for (int h = 0; h < GRP; ++h) {
        const int *qp = reinterpret_cast<const int *>(sm.q8[h] + half * 64);
#pragma unroll
        for (int e = 0; e < 16; ++e) qv[h][e] = qp[e];
        qscale[h] = sm.qs[h];
      }
    }
    // the new token (position kv_len - 1) comes from the prologue's LDS copy
    if (a.fuse_heads) {
#pragma unroll
      for (int i = 0; i < BPW; ++i) {
        const int j = (b0 + wave + NW * i) * 32;
        if (wave + NW * i >= nb) continue;
        if (j + kc == pos0) {
          const int *kn = reinterpret_cast<const int *>(sm.knew + half * 64);
#pragma unroll
          for (int e = 0; e < 16; ++e) kw[i][e] = kn[e];
          kscale[i] = sm.ksnew;
        }
#pragma unroll
        for (int cc = 0; cc < 16; ++cc)
          if (j + kh + cc == pos0) vw[i][cc] = *reinterpret_cast<const int *>(sm.vnew + d0);
        if (j + (lane & 31) == pos0) vscale[i] = sm.vsnew;
      }
    }
    // ---- phase 1: scores and block maxima ----
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
      const int jb = wave + NW * i;
      if (jb >= nb) continue;
      const int j = (b0 + jb) * 32;
      const bool valid = j + kc < kv_end;
#pragma unroll
      for (int h = 0; h < GRP; ++h) {
        int acc = 0;
#pragma unroll
        for (int e = 0; e < 16; ++e) acc = sdot4(qv[h][e], kw[i][e], acc);
        acc += __shfl_xor(acc, 1);  // exact int32: both halves of the key
        float s = -INFINITY;
        if (valid) {
          s = __fmul_rn(static_cast<float>(acc), kscale[i]);
          s = __fmul_rn(s, qscale[h]);
          s = __fmul_rn(s, a.qk_scale);
          if (kc > pos0 - j) s = -INFINITY;  // (col - row) > pos0 - j, row 0
        }
        const float bm = max64(s);
        if (half == 0) sm.s[h][jb * 32 + kc] = s;
        if (lane == 0) sm.bmax[h][jb] = bm;
      }
    }
    __syncthreads();
    // ---- phase 2: prefix max (attention_gqa.h:476-477) ----
    if (tid < GRP) {
      float run = sm.run[tid];
      for (int jb = 0; jb < nb; ++jb) {
        const float bm = sm.bmax[tid][jb];
        const float nmm = (run > bm) ? run : bm;
        sm.prev[tid][jb] = run;
        sm.nmm[tid][jb] = nmm;
        run = nmm;
      }
      sm.run[tid] = run;
    }
    __syncthreads();
    // ---- phase 3: P, P8 and P8.V per block ----
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
      const int jb = wave + NW * i;
      if (jb >= nb) continue;
      const int j = (b0 + jb) * 32;
      const int c = lane & 31;
      const bool valid = j + c < kv_end;
#pragma unroll
      for (int hp = 0; hp < GRP; hp += 2) {
        const int h = hp + (lane >> 5);
        const bool hok = h < GRP;
        float p = 0.0f, pv = 0.0f;
        if (hok && valid) {
          p = exp_f32_tab(__fsub_rn(sm.s[h][jb * 32 + c], sm.nmm[h][jb]), sm.tab);
          pv = __fmul_rn(p, vscale[i]);
        }
        const float psum = tree_sum32(p);
        const float pm = __fmul_rn(max32(pv), inv127());
        const int p8 = hok ? quant1(pv, pm) : 0;
        if (hok && c == 0) {
          sm.psum[h][jb] = psum;
          sm.corr[h][jb] = exp_f32_tab(__fsub_rn(sm.prev[h][jb], sm.nmm[h][jb]), sm.tab);
        }
        int acc[2][4] = {{0, 0, 0, 0}, {0, 0, 0, 0}};
#pragma unroll
        for (int cc = 0; cc < 16; ++cc) {
          const int key = kh + cc;
          const int pa = __shfl(p8, key);       // head hp, key `key`
          const int pb = __shfl(p8, 32 + key);  // head hp+1, key `key`
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int ve = static_cast<int>(static_cast<int8_t>(vw[i][cc] >> (8 * e)));
            acc[0][e] += pa * ve;
            acc[1][e] += pb * ve;
          }
        }
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[s2][e] += __shfl_xor(acc[s2][e], 32);
        // lanes 0..31 own the result; pmax of head hp+s2 lives in lane 32*s2
        const float pm0 = __shfl(pm, 0), pm1 = __shfl(pm, 32);
        if (lane < 32) {
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) {
            const int hh = hp + s2;
            if (hh < GRP) {
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
    __syncthreads();
    // ---- phase 4: the sequential den/res chain (attention_gqa.h:476-519) ----
    if (tid < GRP * HD) {
      for (int jb = 0; jb < nb; ++jb) {
        const float corr = sm.corr[ph][jb];
        den = __fadd_rn(__fmul_rn(den, corr), sm.psum[ph][jb]);
        res = __fadd_rn(__fmul_rn(res, corr), sm.pv[ph][jb][pd]);
      }
    }
    __syncthreads();
  }

  // ---- epilogue: out = res * (1/den); per-head int8 quant (522-546) ----
  float out = 0.0f;
  if (tid < GRP * HD) {
    out = __fmul_rn(res, __fdiv_rn(1.0f, den));
    const float m = max64(fabsf(out));
    if (lane == 0) sm.absmax[ph][(tid % HD) / 64] = m;
  }
  __syncthreads();
  if (tid < GRP * HD) {
    const int qh = kvh * GRP + ph;
    const float scale = __fmul_rn(fmaxf(sm.absmax[ph][0], sm.absmax[ph][1]), inv127());
    if (a.attn) a.attn[qh * HD + pd] = out;
    a.o8[qh * HD + pd] = static_cast<int8_t>(quant1(out, scale));
    if (pd == 0) a.os[qh * a.os_col] = scale;
  }
}

}  // namespace

bool attn_decode_supported(const AttnArgs &a) {
  const int grp = a.kv_heads > 0 ? a.heads / a.kv_heads : 0;
  auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  return a.rows == 1 && a.causal && (grp == 1 || grp == 2) && a.kv_heads * grp == a.heads &&
         (a.row_bytes % 16) == 0 && (a.page_tokens % 32) == 0 && al16(a.k) && al16(a.v) &&
         al16(a.q8) && (a.scale_row_bytes % 4) == 0 && a.kv_len >= 1 && !a.kv_len_dev;
}

hipError_t launch_attn_decode(const AttnArgs &a, hipStream_t s) {
  const int grp = a.heads / a.kv_heads;
  const dim3 grid(a.kv_heads, 1);
  if (grp == 1)
    hipLaunchKernelGGL(attn_decode_kernel<1>, grid, dim3(NW * 64), 0, s, a);
  else
    hipLaunchKernelGGL(attn_decode_kernel<2>, grid, dim3(NW * 64), 0, s, a);
  return hipGetLastError();
}

}  // namespace q3
