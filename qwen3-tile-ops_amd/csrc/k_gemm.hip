// Per-K-group int8 GEMM on the gfx950 matrix cores, with the reference's
// fused epilogues.
//
//   kernels/group_gemm.h:27-222  gemm_nt_group_store
//   ref_qwen3.py:145-158         gemm_nt_group
//   kernels/norm_rope_quant.h:17-86 (Q/K epilogue), group_gemm.h:173-193 (V)
//   kernels/lm_argmax.h:72-182   gemm_nt_group_argmax
//
// D[m,n] = sum over K-groups g, in order, of RN(RN(f32(I_g[m,n]) * bs[n]) *
// as[m,g]), starting from +0.0f; I_g is the exact int32 dot product of the
// group, computed with v_mfma_i32_16x16x64_i8 (exact, order-free).
//
// Work decomposition: a workgroup of 4 waves owns a 16*MT x 128 output tile
// (128 columns = one attention head, so the per-head epilogues stay inside
// the workgroup); each wave owns 32 columns (two 16x16 MFMA tiles) for all
// 16*MT rows.  MFMA operand layout (16x16x64, wave64): lane l supplies row
// (l % 16) of A and column (l % 16) of B, with 16 consecutive k values
// starting at 16 * (l / 16); the int32 result of lane l is rows
// 4 * (l / 16) + i, i = 0..3, of column l % 16.
#include "q3_device.h"
#include "q3_kernels.h"

namespace q3 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int BN = 128;
constexpr int LDT = BN + 4;  // LDS tile row pitch (floats)

__device__ __forceinline__ v4i load16(const int8_t *p) {
  return *reinterpret_cast<const v4i *>(p);
}

__device__ __forceinline__ v4i zero4() {
  v4i z = {0, 0, 0, 0};
  return z;
}

// Row destination of the int8 head output (dense view or paged KV slot).
__device__ __forceinline__ void qdest_row(const QDest &d, int m, int head,
                                          int8_t **row8, float **scale) {
  if (d.table) {
    uint32_t t = d.pos0 + static_cast<uint32_t>(m);
    if (d.pos_dev) t += static_cast<uint32_t>(*d.pos_dev);
    const uint32_t page = d.table[t / d.page_tokens];
    const uint32_t slot = t % d.page_tokens;
    *row8 = d.q8 + page * d.page_bytes + slot * d.row_bytes + head * 128;
    *scale = reinterpret_cast<float *>(reinterpret_cast<int8_t *>(d.qs) +
                                       page * d.scale_page_bytes +
                                       slot * d.scale_row_bytes) + head;
  } else {
    *row8 = d.q8 + static_cast<int64_t>(m) * d.ldq8 + head * 128;
    *scale = d.qs + static_cast<int64_t>(m) * d.ldqs + head * d.qs_col;
  }
}

template <int MT, int EPI>
__global__ void __launch_bounds__(256) gemm_group_kernel(GemmArgs a) {
  constexpr int BM = 16 * MT;
  __shared__ float tile[(EPI >= EPI_HEADQ) ? BM * LDT : 1];

  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int lr = lane & 15;
  const int lg = lane >> 4;
  const int m0 = blockIdx.y * BM;
  const int n_blk = blockIdx.x * BN;
  const int nw0 = n_blk + wave * 32;
  const int M = a.M;

  float acc[MT][2][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[mt][nt][i] = 0.0f;

  const int8_t *arow[MT];
  bool avalid[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int r = m0 + mt * 16 + lr;
    avalid[mt] = r < M;
    arow[mt] = a.a + static_cast<int64_t>(avalid[mt] ? r : 0) * a.lda + lg * 16;
  }
  const int8_t *brow[2];
  float bscale[2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int n = nw0 + nt * 16 + lr;
    brow[nt] = a.b + static_cast<int64_t>(n) * a.ldb + lg * 16;
    bscale[nt] = a.bs_ld ? 0.0f : a.bs[static_cast<int64_t>(n) * a.bs_stride];
  }

  const int G = a.group;
  const int ngroups = a.K / G;
  for (int g = 0; g < ngroups; ++g) {
    v4i c[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      c[mt][0] = zero4();
      c[mt][1] = zero4();
    }
    for (int kk = 0; kk < G; kk += 64) {
      const int k = g * G + kk;
      v4i av[MT], bv[2];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) av[mt] = avalid[mt] ? load16(arow[mt] + k) : zero4();
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) bv[nt] = load16(brow[nt] + k);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
          c[mt][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[mt], bv[nt], c[mt][nt], 0, 0, 0);
    }
    // per-group dequant and ordered f32 accumulation
    float bsg[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
      bsg[nt] = a.bs_ld ? a.bs[static_cast<int64_t>(nw0 + nt * 16 + lr) * a.bs_ld + g] : bscale[nt];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = m0 + mt * 16 + lg * 4 + i;
        const float asv = (r < M) ? a.as[static_cast<int64_t>(r) * a.ldas + g] : 0.0f;
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          float p = __fmul_rn(static_cast<float>(c[mt][nt][i]), bsg[nt]);
          p = __fmul_rn(p, asv);
          acc[mt][nt][i] = __fadd_rn(acc[mt][nt][i], p);
        }
      }
  }

  if constexpr (EPI == EPI_STORE || EPI == EPI_ADD) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = m0 + mt * 16 + lg * 4 + i;
        if (r >= M) continue;
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          const int n = nw0 + nt * 16 + lr;
          float *dst = a.out + static_cast<int64_t>(r) * a.ldo + n;
          if constexpr (EPI == EPI_ADD)
            *dst = __fadd_rn(*dst, acc[mt][nt][i]);
          else
            *dst = acc[mt][nt][i];
        }
      }
    return;
  } else {
    // stage the f32 tile in LDS so each wave can walk whole rows
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
          tile[(mt * 16 + lg * 4 + i) * LDT + wave * 32 + nt * 16 + lr] = acc[mt][nt][i];
    __syncthreads();

    const int head = n_blk / 128;
    for (int rr = wave; rr < BM; rr += 4) {
      const int m = m0 + rr;
      if (m >= M) break;
      float t0 = tile[rr * LDT + lane];
      float t1 = tile[rr * LDT + lane + 64];
      if constexpr (EPI == EPI_ARGMAX) {
        const uint32_t k0 = ordered_key(t0), k1 = ordered_key(t1);
        unsigned long long best =
            (static_cast<unsigned long long>(k0) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(n_blk + lane));
        const unsigned long long other =
            (static_cast<unsigned long long>(k1) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(n_blk + lane + 64));
        best = other > best ? other : best;
#pragma unroll
        for (int s = 1; s < 64; s <<= 1) {
          const unsigned long long o = lane_xor_u64(best, s);
          best = o > best ? o : best;
        }
        if (lane == 0) a.keys[static_cast<int64_t>(m) * a.keys_ld + blockIdx.x] = best;
        continue;
      } else {
        if constexpr (EPI == EPI_NRQ) {
          int64_t crow = m;
          if (a.cs_row_dev) crow += *a.cs_row_dev;
          head_norm_rope(t0, t1, lane, a.nw, a.nw_stride, a.cos_t + crow * a.ld_cs,
                         a.sin_t + crow * a.ld_cs, a.inv_hd, true);
        }
        const float mx = max64(fmaxf(fabsf(t0), fabsf(t1)));
        const float scale = __fmul_rn(mx, inv127());
        int8_t *row8;
        float *sp;
        qdest_row(a.qd, m, head, &row8, &sp);
        row8[lane] = static_cast<int8_t>(quant1(t0, scale));
        row8[lane + 64] = static_cast<int8_t>(quant1(t1, scale));
        if (lane == 0) *sp = scale;
      }
    }
  }
}

template <int EPI>
hipError_t launch_epi(const GemmArgs &a, hipStream_t s) {
  const int nblk = a.N / BN;
  if (a.M <= 16) {
    hipLaunchKernelGGL((gemm_group_kernel<1, EPI>), dim3(nblk, 1), dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL((gemm_group_kernel<2, EPI>), dim3(nblk, (a.M + 31) / 32), dim3(256), 0, s, a);
  }
  return hipGetLastError();
}

// One workgroup per row: maximum of the row's per-workgroup keys, then the
// strict `best < value` merge (lm_argmax.h:58-66).
__global__ void __launch_bounds__(256) argmax_finish_kernel(const unsigned long long *keys,
                                                            int64_t keys_ld, int nslots, float *best,
                                                            int64_t best_stride, int32_t *bidx,
                                                            int64_t bidx_stride, int init,
                                                            int32_t *ids_out,
                                                            const int32_t *pos_dev, int pos_add,
                                                            int ids_per_row) {
  __shared__ unsigned long long red[4];
  const int m = blockIdx.x;
  unsigned long long key = 0ull;
  for (int i = threadIdx.x; i < nslots; i += 256) {
    const unsigned long long k = keys[static_cast<int64_t>(m) * keys_ld + i];
    key = k > key ? k : key;
  }
#pragma unroll
  for (int s = 1; s < 64; s <<= 1) {
    const unsigned long long o = lane_xor_u64(key, s);
    key = o > key ? o : key;
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = key;
  __syncthreads();
  if (threadIdx.x != 0) return;
  key = red[0];
  for (int w = 1; w < 4; ++w) key = red[w] > key ? red[w] : key;
  // main_big.cpp:281-290 starts the fused argmax from best = -3e38, bidx = 0
  float b = init ? -3.0e38f : best[m * best_stride];
  int32_t bi = init ? 0 : bidx[m * bidx_stride];
  if (key != 0ull) {
    const float v = key_value(static_cast<uint32_t>(key >> 32));
    const int32_t idx = static_cast<int32_t>(0xFFFFFFFFu - static_cast<uint32_t>(key));
    if (b < v) {  // lm_argmax.h:58-66: mask = best < tmax
      b = v;
      bi = idx;
    }
  }
  best[m * best_stride] = b;
  bidx[m * bidx_stride] = bi;
  if (ids_out && ids_per_row) {
    ids_out[m] = bi;
  } else if (ids_out && m == 0) {
    const int p = (pos_dev ? *pos_dev : 0) + pos_add;
    ids_out[p] = bi;
  }
}

// main_big.cpp:300-322: per 32-column block first argmax (float compare),
// blocks compared through the ordered key, earliest block wins ties.
__global__ void __launch_bounds__(64) argmax_logits_kernel(const float *logits, int vocab,
                                                           int32_t *out_id,
                                                           const int32_t *pos_dev,
                                                           int pos_add) {
  const int lane = threadIdx.x;
  const int nblocks = (vocab + 31) / 32;
  unsigned long long best = 0ull;  // (key << 32) | (0xFFFFFFFF - block)
  int best_idx = 0;
  bool have = false;
  for (int b = lane; b < nblocks; b += 64) {
    const int n0 = b * 32;
    const int nb = min(32, vocab - n0);
    int idx = 0;
    float mv = logits[n0];
    for (int i = 1; i < nb; ++i) {
      const float v = logits[n0 + i];
      if (mv != mv) break;
      if (v != v || v > mv) {
        mv = v;
        idx = i;
      }
    }
    const uint32_t bits = f32_bits(mv);
    const uint32_t key = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
    const unsigned long long k =
        (static_cast<unsigned long long>(key) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(b));
    if (!have || k > best) {
      best = k;
      best_idx = n0 + idx;
      have = true;
    }
  }
  // wave reduction of (best, best_idx); lanes without blocks hold key 0
#pragma unroll
  for (int s = 1; s < 64; s <<= 1) {
    const unsigned long long o = lane_xor_u64(best, s);
    const int oi = static_cast<int>(lane_xor_m(static_cast<uint32_t>(best_idx), s));
    if (o > best) {
      best = o;
      best_idx = oi;
    }
  }
  if (lane == 0) {
    const int p = (pos_dev ? *pos_dev : 0) + pos_add;
    out_id[p] = best_idx;
  }
}

}  // namespace

hipError_t launch_gemm(const GemmArgs &a, hipStream_t s) {
  if (a.M <= 0) return hipSuccess;
  if (a.bs_ld && a.epi != EPI_STORE && a.epi != EPI_ADD) return hipErrorInvalidValue;
  // prefill shapes and batches of sequences: the LDS-staged tile kernel
  // (ARGMAX over at most 64 rows, so that one row tile reads the weights once)
  if (a.M > 16 && (a.epi != EPI_ARGMAX || a.M <= 64)) {
    TileArgs t{};
    t.M = a.M;
    t.N = a.N;
    t.K = a.K;
    t.group = a.group;
    t.a = a.a;
    t.lda = a.lda;
    t.as = a.as;
    t.ldas = a.ldas;
    t.b0 = a.b;
    t.ldb = a.ldb;
    t.bs0 = a.bs;
    t.bs_stride = a.bs_stride;
    t.bs_ld = a.bs_ld;
    t.out = a.out;
    t.ldo = a.ldo;
    t.qd = a.qd;
    t.nw = a.nw;
    t.nw_stride = a.nw_stride;
    t.cos_t = a.cos_t;
    t.sin_t = a.sin_t;
    t.ld_cs = a.ld_cs;
    t.cs_row_dev = a.cs_row_dev;
    t.inv_hd = a.inv_hd;
    t.keys = a.keys;
    t.keys_ld = a.keys_ld;
    if (gemm_tile_supported(t, a.epi)) return launch_gemm_tile(t, a.epi, s);
  }
  switch (a.epi) {
    case EPI_STORE: return launch_epi<EPI_STORE>(a, s);
    case EPI_ADD: return launch_epi<EPI_ADD>(a, s);
    case EPI_HEADQ: return launch_epi<EPI_HEADQ>(a, s);
    case EPI_NRQ: return launch_epi<EPI_NRQ>(a, s);
    case EPI_ARGMAX: return launch_epi<EPI_ARGMAX>(a, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_argmax_finish(const unsigned long long *keys, int64_t keys_ld, int nslots,
                                int M, float *best, int64_t best_stride, int32_t *bidx,
                                int64_t bidx_stride, int init, int32_t *ids_out,
                                const int32_t *pos_dev, int pos_add, hipStream_t s,
                                int ids_per_row) {
  if (M <= 0) return hipSuccess;
  hipLaunchKernelGGL(argmax_finish_kernel, dim3(M), dim3(256), 0, s, keys, keys_ld, nslots, best,
                     best_stride, bidx, bidx_stride, init, ids_out, pos_dev, pos_add, ids_per_row);
  return hipGetLastError();
}

hipError_t launch_argmax_logits(const float *logits, int vocab, int32_t *out_id,
                                const int32_t *pos_dev, int pos_add, hipStream_t s) {
  hipLaunchKernelGGL(argmax_logits_kernel, dim3(1), dim3(64), 0, s, logits, vocab, out_id,
                     pos_dev, pos_add);
  return hipGetLastError();
}

}  // namespace q3
