// Fused gate/up GEMM + SwiGLU + per-256-column int8 quantisation.
//
//   kernels/swiglu_quant.h:105-255 gemm_gate_up_swiglu_quant
//   ref_qwen3.py:421-424 (g, u, sw, s8/ss) and :194-200 (swiglu)
//
// A workgroup owns a 16*MT x 256 tile of the output (one quantisation group)
// and computes both the gate and the up GEMM for it, sharing the A operand.
// Each wave owns 64 columns (four 16x16 MFMA tiles per matrix).  The gate and
// up values of an element land in the same lane, so SwiGLU is applied in
// registers; the tile then goes through LDS for the row-wise group quant.
#include "q3_device.h"
#include "q3_kernels.h"

namespace q3 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int BN = 256;
constexpr int LDT = BN + 4;

__device__ __forceinline__ v4i load16(const int8_t *p) {
  return *reinterpret_cast<const v4i *>(p);
}
__device__ __forceinline__ v4i zero4() {
  v4i z = {0, 0, 0, 0};
  return z;
}

// ref_qwen3.py:194-200: e = exp(-g); e = e + 1; e = 1/e; out = (g * e) * u.
__device__ __forceinline__ float swiglu1(float g, float u) {
  float e = __fmul_rn(g, -1.0f);
  e = exp_f32(e);
  e = __fadd_rn(e, 1.0f);
  e = __fdiv_rn(1.0f, e);
  return __fmul_rn(__fmul_rn(g, e), u);
}

template <int MT>
__global__ void __launch_bounds__(256) gate_up_kernel(GateUpArgs a) {
  constexpr int BM = 16 * MT;
  __shared__ float tile[BM * LDT];

  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int lr = lane & 15;
  const int lg = lane >> 4;
  const int m0 = blockIdx.y * BM;
  const int n_blk = blockIdx.x * BN;
  const int nw0 = n_blk + wave * 64;
  const int M = a.M;

  float accg[MT][4][4], accu[MT][4][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        accg[mt][nt][i] = 0.0f;
        accu[mt][nt][i] = 0.0f;
      }

  const int8_t *arow[MT];
  bool avalid[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int r = m0 + mt * 16 + lr;
    avalid[mt] = r < M;
    arow[mt] = a.a + static_cast<int64_t>(avalid[mt] ? r : 0) * a.lda + lg * 16;
  }
  float gsc[4], usc[4];
  int64_t boff[4];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int n = nw0 + nt * 16 + lr;
    boff[nt] = static_cast<int64_t>(n) * a.ldw + lg * 16;
    gsc[nt] = a.wgs[static_cast<int64_t>(n) * a.ws_stride];
    usc[nt] = a.wus[static_cast<int64_t>(n) * a.ws_stride];
  }

  const int G = a.group;
  const int ngroups = a.K / G;
  for (int g = 0; g < ngroups; ++g) {
    v4i cg[MT][4], cu[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        cg[mt][nt] = zero4();
        cu[mt][nt] = zero4();
      }
    for (int kk = 0; kk < G; kk += 64) {
      const int k = g * G + kk;
      v4i av[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) av[mt] = avalid[mt] ? load16(arow[mt] + k) : zero4();
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const v4i bg = load16(a.wg + boff[nt] + k);
        const v4i bu = load16(a.wu + boff[nt] + k);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          cg[mt][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[mt], bg, cg[mt][nt], 0, 0, 0);
          cu[mt][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[mt], bu, cu[mt][nt], 0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = m0 + mt * 16 + lg * 4 + i;
        const float asv = (r < M) ? a.as[static_cast<int64_t>(r) * a.ldas + g] : 0.0f;
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
          float pg = __fmul_rn(static_cast<float>(cg[mt][nt][i]), gsc[nt]);
          pg = __fmul_rn(pg, asv);
          accg[mt][nt][i] = __fadd_rn(accg[mt][nt][i], pg);
          float pu = __fmul_rn(static_cast<float>(cu[mt][nt][i]), usc[nt]);
          pu = __fmul_rn(pu, asv);
          accu[mt][nt][i] = __fadd_rn(accu[mt][nt][i], pu);
        }
      }
  }

#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
        tile[(mt * 16 + lg * 4 + i) * LDT + wave * 64 + nt * 16 + lr] =
            swiglu1(accg[mt][nt][i], accu[mt][nt][i]);
  __syncthreads();

  const int grp = n_blk / 256;
  for (int rr = wave; rr < BM; rr += 4) {
    const int m = m0 + rr;
    if (m >= M) break;
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = tile[rr * LDT + lane + 64 * j];
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) mx = fmaxf(mx, fabsf(v[j]));
    mx = max64(mx);
    const float scale = __fmul_rn(mx, inv127());
    int8_t *dst = a.s8 + static_cast<int64_t>(m) * a.lds8 + n_blk;
#pragma unroll
    for (int j = 0; j < 4; ++j) dst[lane + 64 * j] = static_cast<int8_t>(quant1(v[j], scale));
    if (lane == 0) a.ss[static_cast<int64_t>(m) * a.ldss + grp * a.ss_col] = scale;
  }
}

}  // namespace

hipError_t launch_gate_up(const GateUpArgs &a, hipStream_t s) {
  if (a.M <= 0) return hipSuccess;
  if (a.M > 16) {  // prefill shapes: the LDS-staged tile kernel
    TileArgs t{};
    t.M = a.M;
    t.N = a.N;
    t.K = a.K;
    t.group = a.group;
    t.a = a.a;
    t.lda = a.lda;
    t.as = a.as;
    t.ldas = a.ldas;
    t.b0 = a.wg;
    t.b1 = a.wu;
    t.ldb = a.ldw;
    t.bs0 = a.wgs;
    t.bs1 = a.wus;
    t.bs_stride = a.ws_stride;
    t.s8 = a.s8;
    t.lds8 = a.lds8;
    t.ss = a.ss;
    t.ldss = a.ldss;
    t.ss_col = a.ss_col;
    if (gemm_tile_supported(t, EPI_SWIGLUQ)) return launch_gemm_tile(t, EPI_SWIGLUQ, s);
  }
  const int nblk = a.N / BN;
  if (a.M <= 16) {
    hipLaunchKernelGGL(gate_up_kernel<1>, dim3(nblk, 1), dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL(gate_up_kernel<2>, dim3(nblk, (a.M + 31) / 32), dim3(256), 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace q3
