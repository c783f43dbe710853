// Prefill-shaped per-group int8 GEMM (M >= 64): LDS-staged MFMA tiles.
//
// Arithmetic of kernels/group_gemm.h:27-222 / ref_qwen3.py:145-158, with the
// epilogues of group_gemm.h:173-214 (V quant, residual add),
// norm_rope_quant.h:17-86 (Q/K) and swiglu_quant.h:164-255 (gate/up):
//   D[m,n] = sum over K-groups g, in order from +0.0f, of
//            RN(RN(f32(I_g[m,n]) * bs[n]) * as[m,g])
// where I_g is the exact int32 dot product of group g
// (v_mfma_i32_16x16x64_i8).
//
// Decomposition: a workgroup of NW waves (8: two per SIMD, so that one
// wave's dequantisation and address work overlaps the other's MFMAs) owns a
// BM x BN output tile (for the gate/up kernel: BN output columns of both
// matrices).  Waves are arranged WGM (rows) x NW/WGM (columns).  Operand tiles of each KS-byte k-step are
// copied global -> LDS with global_load_lds_dwordx4 (the copy needs no
// registers), STAGES steps in flight, and each wave reads its MFMA fragments
// (KS / 64 slices per step) from LDS with ds_read_b128.  The copy of one
// k-step is (BM + NMAT*BN) * KS / 1024 instructions of 1 KiB; lane i of an
// instruction writes LDS bytes [16 i, 16 i + 16), so the layout is chosen
// through the global address each lane reads: LDS row r keeps its 16-byte
// chunk c in slot c ^ ((r / RPC) % CH) (CH chunks per row, RPC rows per
// 256-byte bank cycle), which spreads the 16 rows of a fragment read over
// all banks.  Steps are coarse (KS = 128 or 256 B: one barrier per 2-4 MFMA
// k-slices) because a k-step's fixed cost (barrier, LDS latency) is
// comparable to a 64-byte step's MFMA work; the copies of step t + STAGES - 1
// are issued right after step t's barrier, into the stage step t - 1 read.
//
// The per-group dequantisation (one thread per output element, groups in
// order) costs 4 VALU operations per element and group (cvt, two RN
// multiplies, add): as much issue time as the group's MFMAs at g = 256 and
// twice as much at g = 128.  The int32 group sums are therefore double
// buffered by group parity: group g is dequantised after the first MFMAs of
// group g + 1 are issued, so the two run side by side instead of
// MFMA -> dequant -> MFMA on one set of registers.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <type_traits>
#include <utility>

#include "q3_device.h"
#include "q3_epi.h"
#include "q3_kernels.h"

namespace q3 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
__device__ __forceinline__ v4i zero4() {
  v4i z = {0, 0, 0, 0};
  return z;
}

template <int BM, int BN, int WGM, int NMAT, int STAGES, int KS>
struct TileShape {
  static constexpr int NW = 8;                         // waves per workgroup
  static constexpr int NTHR = 64 * NW;
  static constexpr int WGN = NW / WGM;
  static constexpr int WM = BM / WGM, WN = BN / WGN;  // wave tile (output columns)
  static constexpr int MT = WM / 16, NT = WN / 16;
  static constexpr int BROWS = NMAT * BN;              // B rows per k-step
  static constexpr int STAGE = (BM + BROWS) * KS;      // bytes per k-step
  static constexpr int INSTR = STAGE / 1024;           // 1 KiB copies per k-step
  static constexpr int IPW_HI = (INSTR + NW - 1) / NW; // copies per wave: waves below
  static constexpr int IPW_LO = INSTR / NW;            //   INSTR % NW issue one more
  static constexpr int CH = KS / 16;                   // 16-byte chunks per LDS row
  static constexpr int RPI = 1024 / KS;                // rows per copy instruction
  static constexpr int RPC = KS >= 256 ? 1 : 256 / KS; // rows per 256-byte bank cycle
  static constexpr int SLICES = KS / 64;               // MFMA k-slices per step
  static constexpr int LDT = BN + 4;                   // f32 epilogue tile pitch
  static_assert(WGM * WGN == NW, "wave grid");
  static_assert(WM % 16 == 0 && WN % 16 == 0, "16x16 MFMA tiles");
  static_assert(KS == 64 || KS == 128 || KS == 256, "k-step bytes");
  static_assert(BM % RPI == 0, "copies do not straddle A and B");
  static_assert(IPW_HI * (STAGES - 1) < 64, "vmcnt range");
  __device__ static int swz(int r, int c) { return c ^ ((r / RPC) & (CH - 1)); }
};

// BSG: per-(row, K-group) B scales bs0[n * bs_ld + g] (staged in LDS with
// the A scales) instead of one scale per weight row.
template <int BM, int BN, int WGM, int NMAT, int STAGES, int KS, int EPI, int GROUP, bool BSG>
__global__ void __launch_bounds__(512) gemm_tile_kernel(TileArgs a) {
  using S = TileShape<BM, BN, WGM, NMAT, STAGES, KS>;
  constexpr int MT = S::MT, NT = S::NT;
  extern __shared__ __align__(16) int8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int wm = wave % WGM;
  const int wn = wave / WGM;
  const int lr = lane & 15;
  const int lg = lane >> 4;
  const int m0 = blockIdx.y * BM;
  const int n0 = blockIdx.x * BN;
  // the tile's column segment (EPI_QKV: Q, K or V; else the single matrix):
  // its weights, scales, first column within them, destination and norm
  const int8_t *B0 = a.b0;
  const float *BS0 = a.bs0;
  int nb = n0;
  QDest qd = a.qd;
  const float *nw = a.nw;
  bool do_norm = EPI == EPI_NRQ;
  if constexpr (EPI == EPI_QKV) {
    int si = 0;
    for (int i = 1; i < a.nseg; ++i)
      if (n0 >= a.seg[i].n0) si = i;
    B0 = a.seg[si].b;
    BS0 = a.seg[si].bs;
    nb = n0 - a.seg[si].n0;
    qd = a.seg[si].qd;
    nw = a.seg[si].nw;
    do_norm = a.seg[si].norm != 0;
  }
  const int M = a.M;
  const int T = a.K / KS;            // k-steps
  const int ngroups = a.K / a.group;
  float *as_lds = reinterpret_cast<float *>(smem + STAGES * S::STAGE);  // [BM][ngroups]
  float *bs_lds = as_lds + BM * ngroups;                                 // BSG: [BN][ngroups]
  uint64_t *tab = reinterpret_cast<uint64_t *>(bs_lds + (BSG ? BN * ngroups : 0));  // exp table (SwiGLU)

  // k-step t -> stage s; instruction j copies LDS rows [RPI j, RPI (j + 1))
  auto issue = [&](int t, int s) {
    int8_t *st = smem + s * S::STAGE;
#pragma unroll
    for (int q = 0; q < S::IPW_HI; ++q) {
      const int j = wave + S::NW * q;
      if (j >= S::INSTR) break;  // wave-uniform
      const int r = S::RPI * j + lane / S::CH;
      const int c = S::swz(r, lane % S::CH);
      const int8_t *src;
      if (S::RPI * j < BM) {
        const int row = min(m0 + r, M - 1);
        src = a.a + static_cast<int64_t>(row) * a.lda + t * KS + 16 * c;
      } else {
        const int rb = r - BM;
        const int8_t *bm = (NMAT == 2 && rb >= BN) ? a.b1 : B0;
        src = bm + static_cast<int64_t>(nb + rb % BN) * a.ldb + t * KS + 16 * c;
      }
      __builtin_amdgcn_global_load_lds(const_cast<int8_t *>(src), to_lds(st + 1024 * j), 16, 0, 0);
    }
  };

  // A scales of the tile's rows (all groups) and the per-column B scales
  for (int i = threadIdx.x; i < BM * ngroups; i += S::NTHR) {
    const int r = i / ngroups, g = i % ngroups;
    as_lds[i] = (m0 + r < M) ? a.as[static_cast<int64_t>(m0 + r) * a.ldas + g] : 0.0f;
  }
  if (EPI == EPI_SWIGLUQ && threadIdx.x == 0) stage_exp2_table(tab);
  float bsv[NMAT][NT];
  if constexpr (BSG) {
    static_assert(!BSG || NMAT == 1, "per-group B scales: one weight matrix");
    for (int i = threadIdx.x; i < BN * ngroups; i += S::NTHR)
      bs_lds[i] = BS0[static_cast<int64_t>(nb + i / ngroups) * a.bs_ld + i % ngroups];
  } else {
#pragma unroll
    for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const float *bs = mi == 0 ? BS0 : a.bs1;
        bsv[mi][nt] = bs[static_cast<int64_t>(nb + wn * S::WN + nt * 16 + lr) * a.bs_stride];
      }
  }

  // scales first, then the first STAGES-1 copies: vector loads complete in
  // order, so waiting for the scales does not wait for the copies
#pragma unroll
  for (int p = 0; p < STAGES - 1; ++p)
    if (p < T) issue(p, p);

  float acc[NMAT][MT][NT][4];
#pragma unroll
  for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[mi][mt][nt][i] = 0.0f;

  // Exact int32 group sums, double-buffered by group parity (GROUP > 0):
  // group g is dequantised (and its buffer cleared) right after the first
  // MFMAs of group g + 1 are issued, so its VALU work runs while they
  // execute (the two buffers share no register).  GROUP == 0 (group size
  // known only at run time): one buffer, dequantised as soon as the group's
  // last slice is done.
  v4i c[2][NMAT][MT][NT];
#pragma unroll
  for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) c[0][mi][mt][nt] = c[1][mi][mt][nt] = zero4();

  // acc += RN(RN(f32(c) * bs[n]) * as[m][g]) (groups in ascending order),
  // then c = 0 for the buffer's next group
  auto dequant = [&](auto PAR, int g) {
    constexpr int b = decltype(PAR)::value;
    if constexpr (BSG) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) bsv[0][nt] = bs_lds[(wn * S::WN + nt * 16 + lr) * ngroups + g];
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float asv = as_lds[(wm * S::WM + mt * 16 + lg * 4 + i) * ngroups + g];
#pragma unroll
        for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            const float p = __fmul_rn(__fmul_rn(static_cast<float>(c[b][mi][mt][nt][i]), bsv[mi][nt]), asv);
            acc[mi][mt][nt][i] = __fadd_rn(acc[mi][mt][nt][i], p);
          }
      }
#pragma unroll
    for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) c[b][mi][mt][nt] = zero4();
  };

  constexpr int SPG = GROUP > 0 ? GROUP / 64 : 1;        // k-slices per group
  constexpr bool WHOLE = GROUP > 0 && SPG >= S::SLICES;  // a group is whole steps
  // One k-step.  WHOLE: every slice goes to buffer PAR (the group's parity)
  // and gfirst marks the group's first step; otherwise a step holds an even
  // number of groups and the buffer follows the slice.  Stage t % STAGES is
  // refilled STAGES - 1 steps later, by the copies issued after the barrier
  // of step t + 1, when every wave is past step t.
  auto step = [&](int t, auto PAR, bool gfirst) {
    if (t + STAGES - 2 < T) {
      // steps t+1 .. t+STAGES-2 of this wave may stay in flight
      if (wave < S::INSTR % S::NW || S::INSTR % S::NW == 0)
        wait_vmcnt<S::IPW_HI * (STAGES - 2)>();
      else
        wait_vmcnt<S::IPW_LO * (STAGES - 2)>();
    } else {
      wait_vmcnt<0>();
    }
    lds_barrier();
    if (t + STAGES - 1 < T) issue(t + STAGES - 1, (t + STAGES - 1) % STAGES);
    const int8_t *st = smem + (t % STAGES) * S::STAGE;
    static_for<S::SLICES>([&](auto KK) {
      constexpr int kk = decltype(KK)::value;
      v4i af[MT], bf[NMAT][NT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int r = wm * S::WM + mt * 16 + lr;
        af[mt] = *reinterpret_cast<const v4i *>(st + r * KS + 16 * S::swz(r, 4 * kk + lg));
      }
#pragma unroll
      for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const int r = BM + mi * BN + wn * S::WN + nt * 16 + lr;
          bf[mi][nt] = *reinterpret_cast<const v4i *>(st + r * KS + 16 * S::swz(r, 4 * kk + lg));
        }
      const int slice = t * S::SLICES + kk;
      constexpr int par = GROUP == 0 ? 0 : WHOLE ? decltype(PAR)::value : (kk / SPG) & 1;
#pragma unroll
      for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
            c[par][mi][mt][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[mt], bf[mi][nt], c[par][mi][mt][nt], 0, 0, 0);
      if constexpr (GROUP == 0) {
        const int spg = a.group / 64;
        if ((slice + 1) % spg == 0) dequant(std::integral_constant<int, 0>{}, slice / spg);
      } else if constexpr (WHOLE) {
        if (kk == 0 && gfirst && slice > 0) dequant(std::integral_constant<int, par ^ 1>{}, slice / SPG - 1);
      } else if constexpr (kk % SPG == 0) {
        if (slice > 0) dequant(std::integral_constant<int, par ^ 1>{}, slice / SPG - 1);
      }
    });
  };

  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  if constexpr (WHOLE) {
    constexpr int SPS = SPG / S::SLICES;  // k-steps per group
    int t = 0;
    for (int g = 0; g < ngroups; g += 2) {
      for (int q = 0; q < SPS; ++q, ++t) step(t, P0{}, q == 0);
      if (g + 1 < ngroups)
        for (int q = 0; q < SPS; ++q, ++t) step(t, P1{}, q == 0);
    }
  } else {
    for (int t = 0; t < T; ++t) step(t, P0{}, false);
  }
  if constexpr (GROUP > 0) {  // the last group
    if ((ngroups - 1) & 1)
      dequant(P1{}, ngroups - 1);
    else
      dequant(P0{}, ngroups - 1);
  }
  __syncthreads();

  if constexpr (EPI == EPI_STORE || EPI == EPI_ADD) {
    // EPI_ADD: every residual element of the lane is loaded before the first
    // store (a load after a store to the same array would wait for it, one
    // memory latency per element); rows past M read row M - 1, unused.
    // The residual and result are read and written once: non-temporal
    // accesses, so that their 8 M N bytes do not push the A and B tiles
    // other workgroups re-read out of L2 (config 1, M = 2048: Q 16.8 ->
    // 15.7 us, K+V 10.9 -> 10.4 us; gate+up at M = 512 14.2 -> 13.7 us).
    float xr[MT][4][NT];
    if constexpr (EPI == EPI_ADD) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = min(m0 + wm * S::WM + mt * 16 + lg * 4 + i, M - 1);
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
            xr[mt][i][nt] = __builtin_nontemporal_load(&a.out[static_cast<int64_t>(m) * a.ldo + n0 + wn * S::WN + nt * 16 + lr]);
        }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = m0 + wm * S::WM + mt * 16 + lg * 4 + i;
        if (m >= M) continue;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          float *dst = a.out + static_cast<int64_t>(m) * a.ldo + n0 + wn * S::WN + nt * 16 + lr;
          if constexpr (EPI == EPI_ADD)
            __builtin_nontemporal_store(__fadd_rn(xr[mt][i][nt], acc[0][mt][nt][i]), dst);
          else
            __builtin_nontemporal_store(acc[0][mt][nt][i], dst);
        }
      }
  } else {
    // f32 tile through LDS (the stages are free now) so a wave can walk rows
    float *tile = reinterpret_cast<float *>(smem);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          float v = acc[0][mt][nt][i];
          if constexpr (EPI == EPI_SWIGLUQ) v = swiglu_tab(acc[0][mt][nt][i], acc[NMAT - 1][mt][nt][i], tab);
          tile[(wm * S::WM + mt * 16 + lg * 4 + i) * S::LDT + wn * S::WN + nt * 16 + lr] = v;
        }
    __syncthreads();
    if constexpr (EPI == EPI_HEADQ || EPI == EPI_NRQ || EPI == EPI_QKV) {
      // group_gemm.h:173-193 / norm_rope_quant.h:17-86 per (row, head).
      // Pass 1 loads every operand of the wave's rows (gains, cos/sin rows,
      // destination slots through the page table) as independent loads
      // issued together; pass 2 computes and stores.  Walking rows with
      // their loads inside would wait for a chain of dependent loads per
      // row.  Rows past M load row M - 1's operands and store nothing.
      static_assert(BN == 128, "one head (128 columns) per tile");
      constexpr int RPW = (BM + S::NW - 1) / S::NW;  // rows per wave
      float w0 = 0.0f, w1 = 0.0f, cr[RPW], sr[RPW];
      int8_t *row8[RPW];
      float *sp[RPW];
      int64_t cs_off = 0;
      if (do_norm) {
        w0 = nw[static_cast<int64_t>(lane) * a.nw_stride];
        w1 = nw[static_cast<int64_t>(lane + 64) * a.nw_stride];
        if (a.cs_row_dev) cs_off = *a.cs_row_dev;
      }
#pragma unroll
      for (int q = 0; q < RPW; ++q) {
        const int mm = min(m0 + min(wave + S::NW * q, BM - 1), M - 1);
        cr[q] = sr[q] = 0.0f;
        if (do_norm) {
          const int64_t crow = a.cs_row_pos ? static_cast<int64_t>(a.cs_row_pos[mm]) : mm + cs_off;
          cr[q] = a.cos_t[crow * a.ld_cs + lane];
          sr[q] = a.sin_t[crow * a.ld_cs + lane];
        }
        qdest_row(qd, mm, nb / 128, &row8[q], &sp[q]);
      }
      // every row is computed (a row past M holds zeros: finite, unused)
      // and only the stores are predicated, so the rows' independent
      // reduction chains can interleave
#pragma unroll
      for (int q = 0; q < RPW; ++q) {
        const int rr = min(wave + S::NW * q, BM - 1);
        const bool store = wave + S::NW * q < BM && m0 + rr < M;
        float t0 = tile[rr * S::LDT + lane];
        float t1 = tile[rr * S::LDT + lane + 64];
        if (do_norm) head_norm_rope_regs(t0, t1, w0, w1, cr[q], sr[q], a.inv_hd, true);
        const float mx = max64(fmaxf(fabsf(t0), fabsf(t1)));
        const float scale = __fmul_rn(mx, inv127());
        const int8_t q0 = static_cast<int8_t>(quant1(t0, scale));
        const int8_t q1 = static_cast<int8_t>(quant1(t1, scale));
        if (store) {
          row8[q][lane] = q0;
          row8[q][lane + 64] = q1;
          if (lane == 0) *sp[q] = scale;
        }
      }
    } else {
    for (int rr = wave; rr < BM; rr += S::NW) {
      const int m = m0 + rr;
      if (m >= M) break;
      if constexpr (EPI == EPI_ARGMAX) {
        // lm_argmax.h:72-182: the row's (max, first column) over the tile's
        // 128 columns as one 64-bit key; the finish kernel takes the max
        // over the tiles
        static_assert(EPI != EPI_ARGMAX || BN == 128, "one key per 128 columns");
        const float t0 = tile[rr * S::LDT + lane];
        const float t1 = tile[rr * S::LDT + lane + 64];
        unsigned long long best = (static_cast<unsigned long long>(ordered_key(t0)) << 32) |
                                  (0xFFFFFFFFu - static_cast<uint32_t>(n0 + lane));
        const unsigned long long other = (static_cast<unsigned long long>(ordered_key(t1)) << 32) |
                                         (0xFFFFFFFFu - static_cast<uint32_t>(n0 + lane + 64));
        best = other > best ? other : best;
#pragma unroll
        for (int sft = 1; sft < 64; sft <<= 1) {
          const unsigned long long o = lane_xor_u64(best, sft);
          best = o > best ? o : best;
        }
        if (lane == 0) a.keys[static_cast<int64_t>(m) * a.keys_ld + blockIdx.x] = best;
      } else if constexpr (EPI == EPI_SWIGLUQ) {
        // swiglu_quant.h:195-231: per 256-column group absmax * (1/127)
        static_assert(EPI != EPI_SWIGLUQ || BN % 256 == 0, "whole quantisation groups");
#pragma unroll
        for (int q = 0; q < BN / 256; ++q) {
          float v[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) v[j] = tile[rr * S::LDT + q * 256 + lane + 64 * j];
          float mx = 0.0f;
#pragma unroll
          for (int j = 0; j < 4; ++j) mx = fmaxf(mx, fabsf(v[j]));
          mx = max64(mx);
          const float scale = __fmul_rn(mx, inv127());
          int8_t *dst = a.s8 + static_cast<int64_t>(m) * a.lds8 + n0 + q * 256;
#pragma unroll
          for (int j = 0; j < 4; ++j) dst[lane + 64 * j] = static_cast<int8_t>(quant1(v[j], scale));
          if (lane == 0) a.ss[static_cast<int64_t>(m) * a.ldss + ((n0 + q * 256) / 256) * a.ss_col] = scale;
        }
      }
    }
    }  // EPI_ARGMAX / EPI_SWIGLUQ
  }
}

template <int BM, int BN, int WGM, int NMAT, int STAGES, int KS, int EPI, int GROUP, bool BSG>
hipError_t launch_shape(const TileArgs &a, hipStream_t s) {
  using S = TileShape<BM, BN, WGM, NMAT, STAGES, KS>;
  if (a.K % KS) return hipErrorInvalidValue;
  const int ngroups = a.K / a.group;
  size_t lds = static_cast<size_t>(STAGES) * S::STAGE + sizeof(float) * (BM + (BSG ? BN : 0)) * ngroups +
               32 * sizeof(uint64_t);
  if (EPI != EPI_STORE && EPI != EPI_ADD)
    lds = std::max(lds, sizeof(float) * BM * S::LDT);
  if (lds > 160 * 1024) return hipErrorInvalidValue;
  static bool attr_set = false;  // more than 64 KiB of dynamic LDS must be allowed once
  if (!attr_set) {
    const hipError_t e =
        hipFuncSetAttribute(reinterpret_cast<const void *>(&gemm_tile_kernel<BM, BN, WGM, NMAT, STAGES, KS, EPI, GROUP, BSG>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const dim3 grid(a.N / BN, (a.M + BM - 1) / BM);
  Q3_LAUNCH((gemm_tile_kernel<BM, BN, WGM, NMAT, STAGES, KS, EPI, GROUP, BSG>), grid, dim3(S::NTHR), lds, s, a);
  return hipGetLastError();
}

// The group size as a template argument where the model uses it (256, and
// 128 for the O projection), so that the group-sum buffers alternate at
// compile time; any other group size takes the run-time path.
template <int BM, int BN, int WGM, int NMAT, int STAGES, int KS, int EPI, bool BSG = false>
hipError_t launch_tile(const TileArgs &a, hipStream_t s) {
  if (a.group == 256) return launch_shape<BM, BN, WGM, NMAT, STAGES, KS, EPI, 256, BSG>(a, s);
  if (a.group == 128) return launch_shape<BM, BN, WGM, NMAT, STAGES, KS, EPI, 128, BSG>(a, s);
  return launch_shape<BM, BN, WGM, NMAT, STAGES, KS, EPI, 0, BSG>(a, s);
}

}  // namespace

bool gemm_tile_supported(const TileArgs &a, int epi) {
  if (a.M < 1 || a.K % 256 || a.group % 64 || a.K % a.group || a.N <= 0) return false;
  if (a.K / a.group > 64) return false;
  auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (!al16(a.a) || (epi != EPI_QKV && !al16(a.b0)) || (a.lda % 16) || (a.ldb % 16)) return false;
  if (epi == EPI_SWIGLUQ) return a.N % 256 == 0 && a.b1 && al16(a.b1);
  return a.N % 128 == 0;
}

hipError_t launch_gemm_tile(const TileArgs &a, int epi, hipStream_t s) {
  if (a.M <= 0) return hipSuccess;
  // Q3_PREFILL_GEMM=tile: the LDS-staged tile kernel for row-major weights
  // even where the stream kernel applies (read at every launch)
  const char *ev = std::getenv("Q3_PREFILL_GEMM");
  const bool stream_ok = !(ev && std::strcmp(ev, "tile") == 0);
  // Plain and residual stores on row-major weights with at least 256 tiles
  // of 64 x 128 (config 1's M = 2048 rows, gate+up at M = 512): those tiles
  // (8 waves of 32 x 32, three 128-byte k-steps in flight) beat the stream
  // kernel's 32-row tiles, whose weight bytes serve half the rows and whose
  // gathered 16-row x 64-byte weight loads stream slower than the tile
  // kernel's whole 128-byte row pieces: 1.5-1.7x at M = 2048 on every
  // config-1 shape (sweep of 11 tile shapes; the stream kernel stays ahead
  // on the smaller grids).
  if ((epi == EPI_STORE || epi == EPI_ADD) && !a.b_packed && a.M > 64 && gemm_tile_supported(a, epi) &&
      static_cast<int64_t>((a.M + 63) / 64) * (a.N / 128) >= 256) {
    if (a.bs_ld)
      return epi == EPI_STORE ? launch_tile<64, 128, 2, 1, 3, 128, EPI_STORE, true>(a, s)
                              : launch_tile<64, 128, 2, 1, 3, 128, EPI_ADD, true>(a, s);
    return epi == EPI_STORE ? launch_tile<64, 128, 2, 1, 3, 128, EPI_STORE>(a, s)
                            : launch_tile<64, 128, 2, 1, 3, 128, EPI_ADD>(a, s);
  }
  // gate/up + SwiGLU + quant on row-major weights: this kernel's 32 x 256
  // tiles of both matrices (whole 128-byte row pieces through LDS) beat the
  // stream kernel's gathered weight loads (op level, M = 512: 16.3 against
  // 21.3 us; M = 2048: 44.0 against 59.7 us)
  if (epi == EPI_SWIGLUQ && !a.b_packed && gemm_tile_supported(a, epi))
    return launch_tile<32, 256, 1, 2, 2, 128, EPI_SWIGLUQ>(a, s);
  if ((stream_ok || a.b_packed) && gemm_stream_supported(a, epi)) return launch_gemm_stream(a, epi, s);
  if (a.b_packed) return hipErrorInvalidValue;  // only the stream kernel reads packed weights
  if (!gemm_tile_supported(a, epi)) return hipErrorInvalidValue;
  if (a.bs_ld) {  // per-(row, K-group) B scales: plain and residual stores only
    if (epi != EPI_STORE && epi != EPI_ADD) return hipErrorInvalidValue;
    if (a.M <= 64)
      return epi == EPI_STORE ? launch_tile<64, 32, 4, 1, 3, 256, EPI_STORE, true>(a, s)
                              : launch_tile<64, 32, 4, 1, 3, 256, EPI_ADD, true>(a, s);
    return epi == EPI_STORE ? launch_tile<64, 128, 2, 1, 3, 128, EPI_STORE, true>(a, s)
                            : launch_tile<32, 64, 2, 1, 6, 256, EPI_ADD, true>(a, s);
  }
  // a batch of sequences (M <= 64): 32-column tiles, for 4x the workgroups
  if (a.M <= 64 && (epi == EPI_STORE || epi == EPI_ADD)) {
    if (epi == EPI_STORE) return launch_tile<64, 32, 4, 1, 3, 256, EPI_STORE>(a, s);
    return launch_tile<64, 32, 4, 1, 3, 256, EPI_ADD>(a, s);
  }
  switch (epi) {
    case EPI_STORE: return launch_tile<64, 128, 2, 1, 3, 128, EPI_STORE>(a, s);
    case EPI_ADD: return launch_tile<32, 64, 2, 1, 6, 256, EPI_ADD>(a, s);
    case EPI_HEADQ: return launch_tile<32, 128, 2, 1, 3, 128, EPI_HEADQ>(a, s);
    case EPI_NRQ: return launch_tile<32, 128, 2, 1, 3, 128, EPI_NRQ>(a, s);
    case EPI_QKV:
      if (a.nseg < 1 || a.nseg > 3 || a.seg[0].n0 != 0 || a.seg[a.nseg - 1].n1 != a.N) return hipErrorInvalidValue;
      for (int i = 0; i < a.nseg; ++i)
        if (a.seg[i].n0 % 128 || a.seg[i].n1 % 128 || a.seg[i].n1 <= a.seg[i].n0 ||
            (i > 0 && a.seg[i].n0 != a.seg[i - 1].n1) || (reinterpret_cast<uintptr_t>(a.seg[i].b) & 15))
          return hipErrorInvalidValue;
      return launch_tile<32, 128, 2, 1, 3, 128, EPI_QKV>(a, s);
    case EPI_SWIGLUQ: return launch_tile<32, 256, 1, 2, 2, 128, EPI_SWIGLUQ>(a, s);
    case EPI_ARGMAX:  // rows of a batch of sequences (M <= 64): the weights are read once
      if (!a.keys || a.keys_ld < a.N / 128) return hipErrorInvalidValue;
      return launch_tile<64, 128, 2, 1, 3, 256, EPI_ARGMAX>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace q3
