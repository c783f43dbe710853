// Decode-shaped group GEMM ("GEMV", M <= 64 rows) across the whole chip.
//
// Arithmetic of k_gemm.hip (kernels/group_gemm.h:27-222,
// ref_qwen3.py:145-158): per K-group an exact int32 MFMA partial, dequant
// RN(RN(f32(I) * bs[n]) * as[m,g]), groups summed in order from +0.0f.
//
// Decomposition: a workgroup owns 16*NT output columns and its 4 waves split
// the K-groups round-robin; each wave issues all of its weight loads before
// its MFMAs and parks its dequantised per-group tiles in LDS; then one
// (row, column) per thread adds the groups in order.  Workgroups never wait
// for each other: there are no grid-wide dependencies, fences or contended
// atomics in this kernel.  Batches of 17-64 rows (independent sequences
// decoding together) run either as MT = 2 or 4 tiles of 16 rows over the
// same weight registers (each weight byte loaded once per workgroup) or as
// one 16-row tile per workgroup in grid rows (each weight byte loaded once
// per grid row, a quarter of A per workgroup); dispatch_rows picks per
// launch width.  The A operand comes from L2.
//
// Prologue (consumer-side quantisation): instead of reading a pre-quantised
// int8 A operand, the workgroup may build it in LDS from f32 rows
//   PRO_NORM   RMSNorm with gain w (rmsnorm.h:34-81) then per-256 quant
//   PRO_EMBED  embedding gather + dequant (embedding.h:99-168), then as NORM
//   PRO_QUANT  per-256 quant only (quant.h:89-138)
// with the reference's exact rounding points; workgroup 0 also stores the
// stage buffers (x, h, h8, hs) the reference writes.
//
// Epilogues: STORE, ADD (residual, group_gemm.h:194-214), SWIGLU (gate and up
// rows of the same columns, swiglu_quant.h:195-231, stored as f32 for the
// next prologue) and ARGMAX (lm_argmax.h:55-67: one (max, first index) key
// per workgroup and row into a slot array, reduced by argmax_finish).
#include <algorithm>

#include "q3_device.h"
#include "q3_epi.h"
#include "q3_kernels.h"
#include "q3_gemv_pro.h"

namespace q3 {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i zero4() {
  v4i z = {0, 0, 0, 0};
  return z;
}

// The O projection partials (GemvArgs::part, M = 1, at most kMaxPart):
// PART = kPartPro adds them in the PRO_NORM prologue, PART = kPartEpi in the
// EPI_ADD epilogue.
constexpr int kPartPro = 1, kPartEpi = 2;
// BSG: per-(row, K-group) B scales seg[0].bs[n * bs_ld + g], loaded with
// the other scales before the weight stream (PRO_NONE, one matrix).
// MT row tiles of 16 (MT > 1: plain A operand, rows past M computed on row
// M - 1's data and not stored), their A fragments loaded AB tiles at a time.
template <int GPW, int KSTEPS, int NT, int NMAT, int PRO, int PART, bool BSG = false, int MT = 1, int AB = MT>
__global__ void __launch_bounds__(256) gemv_kernel(GemvArgs a) {
  static_assert(PART == 0 || NT == 1, "partials: one item column per thread");
  static_assert(!BSG || (NMAT == 1 && PRO == PRO_NONE && PART == 0), "per-group B scales: plain GEMV");
  static_assert(MT == 1 || (PRO == PRO_NONE && PART == 0 && NT == 1), "row tiles: plain A operand");
  static_assert(AB >= 1 && MT % AB == 0, "A fragment batches");
  constexpr int NPRO = PART == kPartPro ? kMaxPart : 0;
  constexpr int NEPI = PART == kPartEpi ? kMaxPart : 0;
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int NB = 16 * NT;       // columns per workgroup
  constexpr int PP = NB + 1;        // partial-tile pitch
  constexpr int MR = 16 * MT;       // rows per workgroup
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int lr = lane & 15;
  const int lg = lane >> 4;
  // grid row y: rows [row0, row0 + M) of the launch (plain A operand)
  const int row0 = static_cast<int>(blockIdx.y) * MR;
  const int M = min(MR, a.M - row0);
  const int K = a.K;
  const int G = a.group;
  const int ngroups = K / G;
  const int n_blk = blockIdx.x * NB;
  // The workgroup's segment: the fields the weight stream needs are
  // selected from all three segments' fields, read at once (a search loop or
  // an indexed read would make each kernel-argument read wait for the one
  // before it); the epilogue's fields are read by index later, in the shadow
  // of the weight loads.
  // (pin_sgpr: the value exists in SGPRs here, so the compiler can neither
  // turn the selects back into selected addresses nor delay the reads)
  // (all reads first, then the pins: one wait for the whole batch)
  ProSrc ps = read_src<PRO, PART != 0>(a);
  int nseg = a.nseg;
  int s_n0[3];
  const int8_t *s_b[3], *s_b2[3];
  const float *s_bs[3], *s_bs2[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    s_n0[i] = a.seg[i].n0;
    s_b[i] = a.seg[i].b;
    s_bs[i] = a.seg[i].bs;
    s_b2[i] = NMAT == 2 ? a.seg[i].b2 : s_b[i];
    s_bs2[i] = NMAT == 2 ? a.seg[i].bs2 : s_bs[i];
  }
  pin_src<PRO, PART != 0>(ps);
  if constexpr (PRO == PRO_NONE) {
    ps.a += static_cast<int64_t>(row0) * ps.lda;
    ps.as += static_cast<int64_t>(row0) * ps.ldas;
  }
  nseg = pin_sgpr(nseg);
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    s_n0[i] = pin_sgpr(s_n0[i]);
    s_b[i] = pin_sgpr(s_b[i]);
    s_bs[i] = pin_sgpr(s_bs[i]);
    if constexpr (NMAT == 2) {
      s_b2[i] = pin_sgpr(s_b2[i]);
      s_bs2[i] = pin_sgpr(s_bs2[i]);
    }
  }
  const int si = (nseg > 1 && n_blk >= s_n0[1] ? 1 : 0) + (nseg > 2 && n_blk >= s_n0[2] ? 1 : 0);
  auto pick = [&](const auto (&v)[3]) { return si == 0 ? v[0] : si == 1 ? v[1] : v[2]; };
  const int sg_n0 = pick(s_n0);
  const int8_t *const sg_b = pick(s_b);
  const int8_t *const sg_b2 = pick(s_b2);
  const float *const sg_bs = pick(s_bs);
  const float *const sg_bs2 = pick(s_bs2);
  const GemvSeg &sg = a.seg[si];

  // LDS: partials [NMAT][ngroups][MR][PP] f32, then (prologue) A [M][K] i8
  // and its scales [M][K/256] f32 and 32 block sums
  float *part = reinterpret_cast<float *>(smem);
  const int part_floats = NMAT * ngroups * MR * PP;
  int8_t *a_lds = reinterpret_cast<int8_t *>(part + part_floats);
  float *as_lds = reinterpret_cast<float *>(a_lds + ((M * K + 15) & ~15));
  float *blk = as_lds + M * (K / 256);
  __shared__ uint64_t exptab[32];
  constexpr int QW = GPW * KSTEPS / 4;  // 256-column groups per wave

  // row 0's prologue operands and the exp table, then the weight stream
  // (see ProRow).  The weight loads are unconditional (a wave past the last
  // group reloads that group and never uses it): vector loads complete in
  // order, and with a fixed count after the prologue operands the compiler
  // waits for those operands alone (vmcnt(#weight loads)) instead of for
  // everything.
  ProRow<QW, NPRO> r0;
  if constexpr (PRO != PRO_NONE) pro_load_row<PRO, QW, NPRO>(a, ps, 0, r0);
  __builtin_amdgcn_sched_barrier(0);  // (issue order: prologue operands first)
  // EPI_ADD with partials: those of the thread's item column, before the
  // weights (the column j = it % NB is the same for every item it of the
  // thread since 256 is a multiple of NB)
  float pe[NEPI > 0 ? NEPI : 1];
  if constexpr (NEPI > 0) {
    const float *pc = ps.part + (n_blk - sg_n0 + static_cast<int>(threadIdx.x) % NB);
#pragma unroll
    for (int h = 0; h < NEPI; ++h) pe[h] = pc[min(h, ps.npart - 1) * ps.ld_part];
  }
  __builtin_amdgcn_sched_barrier(0);
  // A operand rows and scales of the unfused path (the first AB row tiles),
  // also before the weights.  With row tiles the A scales of all MR rows go
  // through LDS instead (asg[r][g], rows past M hold row M - 1's): a few
  // loads per thread rather than 4 per (tile, group) and lane, which would
  // overrun the 63 loads that vmcnt can count in flight.
  const bool avalid = lr < M;
  v4i av[AB][GPW][KSTEPS];
  float asv[AB][GPW][4];
  float *asg = part + part_floats;
  constexpr int NSG = MT > 1 ? (MR * 4 * GPW + 255) / 256 : 1;  // staged scales per thread
  float sgv[NSG];
  if constexpr (MT > 1) {
#pragma unroll
    for (int k = 0; k < NSG; ++k) {
      const int e = min(static_cast<int>(threadIdx.x) + 256 * k, MR * ngroups - 1);
      const int m = min(e / ngroups, M - 1);
      sgv[k] = ps.as[static_cast<int64_t>(m) * ps.ldas + e % ngroups];
    }
  }
  // row tiles t0 .. t0 + AB - 1; with one tile, rows past M are zeros
  auto load_a = [&](int t0) {
#pragma unroll
    for (int tb = 0; tb < AB; ++tb) {
      const int r = 16 * (t0 + tb) + lr;
      const bool ok = r < M;
      const int8_t *arow = ps.a + static_cast<int64_t>(MT == 1 ? (ok ? r : 0) : min(r, M - 1)) * ps.lda + lg * 16;
#pragma unroll
      for (int gi = 0; gi < GPW; ++gi) {
        const int g = min(wave + 4 * gi, ngroups - 1);
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
          const v4i v = *reinterpret_cast<const v4i *>(arow + g * G + ks * 64);
          av[tb][gi][ks] = (MT > 1 || ok) ? v : zero4();
        }
        if constexpr (MT == 1) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int m = min(16 * (t0 + tb) + lg * 4 + i, M - 1);
            asv[tb][gi][i] = ps.as[static_cast<int64_t>(m) * ps.ldas + g];
          }
        }
      }
    }
  };
  if constexpr (PRO == PRO_NONE) load_a(0);
  // the weight rows' scales, then the weights
  float bsv[NMAT][NT];
  float bsg[BSG ? GPW : 1][NT];
  if constexpr (BSG) {
    const int64_t bs_ld = a.bs_ld;
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi) {
      const int g = min(wave + 4 * gi, ngroups - 1);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        bsg[gi][nt] = sg_bs[static_cast<int64_t>(n_blk - sg_n0 + nt * 16 + lr) * bs_ld + g];
    }
  } else {
#pragma unroll
    for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) bsv[mi][nt] = (mi == 0 ? sg_bs : sg_bs2)[n_blk - sg_n0 + nt * 16 + lr];
  }
  v4i bv[NMAT][NT][GPW][KSTEPS];
#pragma unroll
  for (int gi = 0; gi < GPW; ++gi) {
    const int g = min(wave + 4 * gi, ngroups - 1);
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      const int k = g * G + ks * 64 + lg * 16;
#pragma unroll
      for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const int8_t *b = (mi == 0 ? sg_b : sg_b2) +
                            static_cast<int64_t>(n_blk - sg_n0 + nt * 16 + lr) * K;
          bv[mi][nt][gi][ks] = *reinterpret_cast<const v4i *>(b + k);
        }
    }
  }
  // the exp table from immediates (a load here would be issued after the
  // weights and waited for with them); first read after barriers
  // keep every load above issued before the prologue's arithmetic (the
  // scheduler would otherwise start it first and wait for its operands
  // before issuing the weights)
  __builtin_amdgcn_sched_barrier(0);
  if (NMAT == 2 && threadIdx.x == 0) stage_exp2_table(exptab);
  // EPI_ADD over row tiles: the residual value of each of the thread's MT
  // items (see the ordered sums below), loaded now so that the sums do not
  // wait for one load per item (the store of an item would otherwise hold
  // back the next item's load)
  float basev[MT];
  if constexpr (MT > 1) {
    if (sg.epi == EPI_ADD) {
#pragma unroll
      for (int k = 0; k < MT; ++k) {
        const int it = static_cast<int>(threadIdx.x) + 256 * k;
        const int m = min(it / NB, M - 1);
        basev[k] = sg.out[static_cast<int64_t>(row0 + m) * sg.ldo + (n_blk - sg_n0 + it % NB)];
      }
    }
  }

  if constexpr (PRO != PRO_NONE) {
    pro_compute_row<PRO, QW, NPRO>(a, 0, r0, a_lds, as_lds, blk, blockIdx.x == 0);
    for (int m = 1; m < M; ++m) {
      ProRow<QW, 0> r;
      pro_load_row<PRO, QW, 0>(a, ps, m, r);
      pro_compute_row<PRO, QW, 0>(a, m, r, a_lds, as_lds, blk, blockIdx.x == 0);
    }
    const int8_t *arow = a_lds + (avalid ? lr : 0) * K + lg * 16;
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi) {
      const int g = min(wave + 4 * gi, ngroups - 1);
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks)
        av[0][gi][ks] = avalid ? *reinterpret_cast<const v4i *>(arow + g * G + ks * 64) : zero4();
#pragma unroll
      for (int i = 0; i < 4; ++i) asv[0][gi][i] = as_lds[min(lg * 4 + i, M - 1) * (K / 256) + g];
    }
  }
  if constexpr (MT > 1) {
#pragma unroll
    for (int k = 0; k < NSG; ++k)
      asg[min(static_cast<int>(threadIdx.x) + 256 * k, MR * ngroups - 1)] = sgv[k];
    lds_barrier();
  }
  // MFMAs of row tiles t0 .. t0 + AB - 1, dequantised group tiles into LDS
  auto compute = [&](int t0) {
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi) {
      const int g = wave + 4 * gi;
      if (g >= ngroups) break;
#pragma unroll
      for (int tb = 0; tb < AB; ++tb) {
        float asv_[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (MT > 1)
            asv_[i] = asg[(16 * (t0 + tb) + lg * 4 + i) * ngroups + g];
          else
            asv_[i] = lg * 4 + i < M ? asv[tb][gi][i] : 0.0f;
        }
#pragma unroll
        for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            v4i acc = zero4();
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks)
              acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[tb][gi][ks], bv[mi][nt][gi][ks], acc, 0, 0, 0);
            float *pt = part + ((mi * ngroups + g) * MR + 16 * (t0 + tb)) * PP + nt * 16 + lr;
            const float bsc = BSG ? bsg[BSG ? gi : 0][nt] : bsv[mi][nt];
#pragma unroll
            for (int i = 0; i < 4; ++i)
              pt[(lg * 4 + i) * PP] = __fmul_rn(__fmul_rn(static_cast<float>(acc[i]), bsc), asv_[i]);
          }
      }
    }
  };
  compute(0);
  // later batches of row tiles: their A fragments into the same registers
#pragma unroll
  for (int t0 = AB; t0 < MT; t0 += AB) {
    load_a(t0);
    compute(t0);
  }
  __syncthreads();

  // ordered group sums: item = (row m, column j); MR*NB items over 256 threads
  static_assert((MR * NB) % 256 == 0 && (MT == 1 || MR * NB == 256 * MT), "items per thread");
#pragma unroll
  for (int k = 0; k < MR * NB / 256; ++k) {
    const int it = static_cast<int>(threadIdx.x) + 256 * k;
    const int m = it / NB;
    const int j = it % NB;
    float out = 0.0f, out2 = 0.0f;
    for (int g = 0; g < ngroups; ++g) {
      out = __fadd_rn(out, part[(g * MR + m) * PP + j]);
      if (NMAT == 2) out2 = __fadd_rn(out2, part[((ngroups + g) * MR + m) * PP + j]);
    }
    const int ncol = n_blk - sg_n0 + j;
    if (sg.epi == EPI_ARGMAX) {
      unsigned long long key = 0ull;
      if (m < M)
        key = (static_cast<unsigned long long>(ordered_key(out)) << 32) |
              (0xFFFFFFFFu - static_cast<uint32_t>(ncol));
      // NB consecutive threads share a row when NB <= 64 (wave-aligned)
#pragma unroll
      for (int s = 1; s < NB && s < 64; s <<= 1) {
        const unsigned long long o = lane_xor_u64(key, s);
        key = o > key ? o : key;
      }
      if (m < M && j == 0) a.keys[static_cast<int64_t>(row0 + m) * a.keys_ld + blockIdx.x] = key;
      continue;
    }
    if (m >= M) continue;
    float *dst = sg.out + static_cast<int64_t>(row0 + m) * sg.ldo + ncol;
    if (sg.epi == EPI_ADD) {
      float base = MT > 1 ? basev[k] : *dst;
      if constexpr (NEPI > 0) {
        float o = 0.0f;  // the O projection, partials in head order
#pragma unroll
        for (int h = 0; h < NEPI; ++h)
          if (h < ps.npart) o = __fadd_rn(o, pe[h]);
        base = __fadd_rn(base, o);
      }
      *dst = __fadd_rn(base, out);
    } else if (sg.epi == EPI_SWIGLU)
      *dst = swiglu_tab(out, out2, exptab);
    else
      *dst = out;
  }
}

// Column-streaming variant for very wide single-segment launches (the
// lm_head): a fixed grid walks 16*NT-column tiles t = blockIdx.x,
// t + gridDim.x, ...  The A operand is built once per workgroup, the next
// tile's weights are loaded (unconditionally, clamped to the last tile, so
// that the loads stay in flight with a static count) while the current tile
// is reduced, and EPI_ARGMAX keeps one running key per row, written to slot
// blockIdx.x at the end.  Items (row m, column j) map to threads so that a
// row's NB = 64 columns are one wave.
template <int GPW, int KSTEPS, int NT, int PRO>
__global__ void __launch_bounds__(256) gemv_stream_kernel(GemvArgs a, int ntiles) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int NB = 16 * NT;
  constexpr int PP = NB + 1;
  constexpr int QW = GPW * KSTEPS / 4;
  static_assert(NB == 64, "argmax reduction assumes one wave per row");
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int lr = lane & 15;
  const int lg = lane >> 4;
  const int M = a.M;
  const int K = a.K;
  const int G = a.group;
  const int ngroups = K / G;
  const GemvSeg &sg = a.seg[0];
  float *part = reinterpret_cast<float *>(smem);
  int8_t *a_lds = reinterpret_cast<int8_t *>(part + ngroups * 16 * PP);
  float *as_lds = reinterpret_cast<float *>(a_lds + ((M * K + 15) & ~15));
  float *blk = as_lds + M * (K / 256);

  ProSrc ps = read_src<PRO, false>(a);
  pin_src<PRO, false>(ps);
  ProRow<QW, 0> r0;
  if constexpr (PRO != PRO_NONE) pro_load_row<PRO, QW, 0>(a, ps, 0, r0);

  // a tile's column scales, then its weights: issued together one tile
  // ahead, so that using tile t waits only for loads issued before tile
  // t + 1's (vector loads complete in order)
  auto load_tile = [&](v4i (&bv)[NT][GPW][KSTEPS], float (&bsv)[NT], int t) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) bsv[nt] = sg.bs[t * NB + nt * 16 + lr];
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi) {
      const int g = min(wave + 4 * gi, ngroups - 1);
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) {
        const int k = g * G + ks * 64 + lg * 16;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const int8_t *b = sg.b + static_cast<int64_t>(t * NB + nt * 16 + lr) * K;
          bv[nt][gi][ks] = *reinterpret_cast<const v4i *>(b + k);
        }
      }
    }
  };
  // A operand rows and scales of the unfused path are loaded before the
  // first tile (so that waiting for them does not wait for the tile)
  v4i av[GPW][KSTEPS];
  float asv[GPW][4];
  if constexpr (PRO == PRO_NONE) {
    const int8_t *arow = ps.a + static_cast<int64_t>(lr < M ? lr : 0) * ps.lda + lg * 16;
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi) {
      const int g = min(wave + 4 * gi, ngroups - 1);
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks)
        av[gi][ks] = lr < M ? *reinterpret_cast<const v4i *>(arow + g * G + ks * 64) : zero4();
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = lg * 4 + i;
        asv[gi][i] = m < M ? ps.as[static_cast<int64_t>(m) * ps.ldas + g] : 0.0f;
      }
    }
  }
  const int step = static_cast<int>(gridDim.x);
  int t = blockIdx.x;
  v4i b0[NT][GPW][KSTEPS], b1[NT][GPW][KSTEPS];
  float s0[NT], s1[NT];
  load_tile(b0, s0, t);
  __builtin_amdgcn_sched_barrier(0);

  if constexpr (PRO != PRO_NONE) {
    pro_compute_row<PRO, QW, 0>(a, 0, r0, a_lds, as_lds, blk, blockIdx.x == 0);
    for (int m = 1; m < M; ++m) {
      ProRow<QW, 0> r;
      pro_load_row<PRO, QW, 0>(a, ps, m, r);
      pro_compute_row<PRO, QW, 0>(a, m, r, a_lds, as_lds, blk, blockIdx.x == 0);
    }
    const int8_t *arow = a_lds + (lr < M ? lr : 0) * K + lg * 16;
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi) {
      const int g = wave + 4 * gi;
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks)
        av[gi][ks] = (g < ngroups && lr < M) ? *reinterpret_cast<const v4i *>(arow + g * G + ks * 64) : zero4();
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = lg * 4 + i;
        asv[gi][i] = (g < ngroups && m < M) ? as_lds[m * (K / 256) + g] : 0.0f;
      }
    }
  }

  unsigned long long best[4] = {0ull, 0ull, 0ull, 0ull};  // items tid + 256 k
  // one tile: MFMAs, per-group dequant into LDS, ordered group sums
  auto tile = [&](const v4i (&bv)[NT][GPW][KSTEPS], const float (&bsv)[NT], int tt) {
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi) {
      const int g = wave + 4 * gi;
      if (g >= ngroups) break;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        v4i acc = zero4();
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks)
          acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[gi][ks], bv[nt][gi][ks], acc, 0, 0, 0);
        float *pt = part + (g * 16) * PP + nt * 16 + lr;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          pt[(lg * 4 + i) * PP] = __fmul_rn(__fmul_rn(static_cast<float>(acc[i]), bsv[nt]), asv[gi][i]);
      }
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int it = threadIdx.x + 256 * kk;
      if (it >= M * NB) break;
      const int m = it / NB;
      const int j = it % NB;
      float out = 0.0f;
      for (int g = 0; g < ngroups; ++g) out = __fadd_rn(out, part[(g * 16 + m) * PP + j]);
      const int ncol = tt * NB + j;
      if (sg.epi == EPI_ARGMAX) {
        const unsigned long long key = (static_cast<unsigned long long>(ordered_key(out)) << 32) |
                                       (0xFFFFFFFFu - static_cast<uint32_t>(ncol));
        best[kk] = key > best[kk] ? key : best[kk];
      } else {
        sg.out[static_cast<int64_t>(m) * sg.ldo + ncol] = out;
      }
    }
    __syncthreads();  // part is rewritten by the next tile
  };
  // two register sets in turn, the next tile's loads in flight during each
  // tile (no register copy between tiles, which would wait for them)
  while (t < ntiles) {
    load_tile(b1, s1, min(t + step, ntiles - 1));
    tile(b0, s0, t);
    t += step;
    if (t >= ntiles) break;
    load_tile(b0, s0, min(t + step, ntiles - 1));
    tile(b1, s1, t);
    t += step;
  }
  if (sg.epi == EPI_ARGMAX) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int it = threadIdx.x + 256 * kk;
      if (it >= M * NB) break;  // wave-uniform: M * NB is a multiple of 64
      unsigned long long key = best[kk];
#pragma unroll
      for (int sft = 1; sft < 64; sft <<= 1) {
        const unsigned long long o = lane_xor_u64(key, sft);
        key = o > key ? o : key;
      }
      if (lane == 0) a.keys[static_cast<int64_t>(it / NB) * a.keys_ld + blockIdx.x] = key;
    }
  }
}

// M = 1 (decode, and the last row of a prefill chunk): the lm_head GEMV on
// v_dot4 instead of MFMA tiles.  The MFMA operand layout makes every load
// instruction gather 16 weight rows x 64 B at a 1 KB stride, and that
// pattern alone streams at ~4.2 TB/s on this GPU, against ~6.3 TB/s for
// contiguous 16-byte-per-lane reads (probe); with one activation row the
// MFMA's other 15 rows are idle anyway.  Here a wave reads whole 1 KB
// weight rows, lane l holding k = 16 l .. 16 l + 15, R rows per step with
// the next step's loads in flight, as non-temporal loads: each row is read
// once per launch, and the 156 MB of lm_head rows would otherwise displace
// the last-level cache's lines the next launches read (decode lm_head 27.4
// -> 26.2 us, 0.619 -> 0.618 ms/token).  Per row: v_dot4 partials (exact int32),
// the 16 lanes of each 256-column group summed with DPP (exact), then the
// group GEMM's arithmetic (kernels/lm_argmax.h:72-182, ref_qwen3.py:145-158):
// p_g = RN(RN(f32(I_g) * bs[n]) * as_g), out = (((0 + p_0) + p_1) + p_2) + p_3.
// One argmax key per workgroup, as the tile kernels write.
__device__ __forceinline__ int sdot4(int x, int y, int acc) { return __builtin_amdgcn_sdot4(x, y, acc, false); }

template <int PRO, int R>
__global__ void __launch_bounds__(256) gemv_row_kernel(GemvArgs a, int N) {
  __shared__ float blk[32];
  __shared__ __align__(16) int8_t a_lds[1024];
  __shared__ float as_lds[4];
  __shared__ unsigned long long wkey[4];
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const GemvSeg &sg = a.seg[0];

  ProSrc ps = read_src<PRO, false>(a);
  pin_src<PRO, false>(ps);
  ProRow<1, 0> r0;
  if constexpr (PRO != PRO_NONE) pro_load_row<PRO, 1, 0>(a, ps, 0, r0);

  // rows of a wave's step: R consecutive rows; a workgroup step covers 4 R
  // (N is a multiple of 64, so every wave of a workgroup runs the same steps)
  const int stride = static_cast<int>(gridDim.x) * 4 * R;
  int b = (static_cast<int>(blockIdx.x) * 4 + wave) * R;
  auto load = [&](int4 (&w)[R], float (&bs)[R], int b0) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int n = min(b0 + r, N - 1);  // past N: reloaded, never used
      bs[r] = sg.bs[n];
      const v4i v = __builtin_nontemporal_load(reinterpret_cast<const v4i *>(sg.b + static_cast<int64_t>(n) * 1024 + 16 * lane));
      w[r] = make_int4(v.x, v.y, v.z, v.w);
    }
  };
  int4 w0[R], w1[R];
  float bs0[R], bs1[R];
  load(w0, bs0, b);
  __builtin_amdgcn_sched_barrier(0);

  // the activation's 16 bytes at k = 16 lane and the lane's group scale
  int4 av;
  float asg;
  if constexpr (PRO == PRO_NONE) {
    av = *reinterpret_cast<const int4 *>(ps.a + 16 * lane);
    asg = ps.as[lane / 16];
  } else {
    pro_compute_row<PRO, 1, 0>(a, 0, r0, a_lds, as_lds, blk, blockIdx.x == 0);  // ends with a barrier
    av = *reinterpret_cast<const int4 *>(a_lds + 16 * lane);
    asg = as_lds[lane / 16];
  }

  unsigned long long best = 0ull;
  auto rows = [&](const int4 (&w)[R], const float (&bs)[R], int b0) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      int acc = sdot4(w[r].x, av.x, 0);
      acc = sdot4(w[r].y, av.y, acc);
      acc = sdot4(w[r].z, av.z, acc);
      acc = sdot4(w[r].w, av.w, acc);
      acc += lane_xor<1>(acc);
      acc += lane_xor<2>(acc);
      acc += lane_xor<4>(acc);
      acc += lane_xor<8>(acc);
      const float p = __fmul_rn(__fmul_rn(static_cast<float>(acc), bs[r]), asg);
      float out = 0.0f;
      out = __fadd_rn(out, lane_bcast<0>(p));
      out = __fadd_rn(out, lane_bcast<16>(p));
      out = __fadd_rn(out, lane_bcast<32>(p));
      out = __fadd_rn(out, lane_bcast<48>(p));
      const int n = b0 + r;
      if (n < N) {
        if (sg.epi == EPI_ARGMAX) {
          const unsigned long long key = (static_cast<unsigned long long>(ordered_key(out)) << 32) |
                                         (0xFFFFFFFFu - static_cast<uint32_t>(n));
          best = key > best ? key : best;
        } else if (lane == 0) {
          sg.out[n] = out;
        }
      }
    }
  };
  while (b < N) {
    load(w1, bs1, b + stride);
    rows(w0, bs0, b);
    b += stride;
    if (b >= N) break;
    load(w0, bs0, b + stride);
    rows(w1, bs1, b);
    b += stride;
  }
  if (sg.epi == EPI_ARGMAX) {
    if (lane == 0) wkey[wave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
      unsigned long long k = wkey[0];
#pragma unroll
      for (int i = 1; i < 4; ++i) k = wkey[i] > k ? wkey[i] : k;
      a.keys[blockIdx.x] = k;
    }
  }
}

// M = 1 on whole weight rows (the decode Q|K|V, gate/up and down launches,
// K = 1024 KB): R rows per wave, lane l holding bytes k = 1024 j + 16 l ..
// + 15 of a row (contiguous 1 KB per load instruction) instead of the MFMA
// operand layout's 16 rows x 64 B per instruction, on N / (4 R) workgroups.
// The prologue builds the int8 A row in LDS as gemv_kernel's does (PRO,
// with the O partials when NP > 0).  Per row: v_dot4 partials (exact
// int32), the 16 lanes of each 256-column group g = 4 j + l / 16 summed
// with DPP (exact), then the group GEMM's arithmetic p_g = RN(RN(f32(I_g) *
// bs[n]) * as_g), out = (((0 + p_0) + p_1) + ...) in ascending g, in
// registers.  Epilogues as gemv_kernel's: STORE, SWIGLU (NMAT = 2: gate and
// up rows of the same column) and ADD (dst = (dst + o) + out, o the O
// partials summed in head order when NEPI > 0).  A wave's rows lie in one
// segment (segment boundaries are multiples of 4 R).
template <int PRO, int KB, int NMAT, int R, int NP, int NEPI>
__global__ void __launch_bounds__(256) gemv_wr_kernel(GemvArgs a, int N) {
  __shared__ float blk[32];
  __shared__ __align__(16) int8_t a_lds[1024 * KB];
  __shared__ float as_lds[4 * KB];
  __shared__ uint64_t exptab[32];
  static_assert(NP == 0 || NEPI == 0, "partials: prologue or epilogue");
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  ProSrc ps = read_src<PRO, (NP + NEPI) != 0>(a);
  // the segment fields the weight loads need, selected from all three
  int nseg = a.nseg;
  int s_n0[3];
  const int8_t *s_b[3], *s_b2[3];
  const float *s_bs[3], *s_bs2[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    s_n0[i] = a.seg[i].n0;
    s_b[i] = a.seg[i].b;
    s_bs[i] = a.seg[i].bs;
    s_b2[i] = NMAT == 2 ? a.seg[i].b2 : s_b[i];
    s_bs2[i] = NMAT == 2 ? a.seg[i].bs2 : s_bs[i];
  }
  pin_src<PRO, (NP + NEPI) != 0>(ps);
  ProRow<KB, NP> r0;
  pro_load_row<PRO, KB, NP>(a, ps, 0, r0);
  __builtin_amdgcn_sched_barrier(0);  // (issue order: prologue operands first)
  const int row0 = (static_cast<int>(blockIdx.x) * 4 + wave) * R;
  const int si = (nseg > 1 && row0 >= s_n0[1] ? 1 : 0) + (nseg > 2 && row0 >= s_n0[2] ? 1 : 0);
  auto pick = [&](const auto (&v)[3]) { return si == 0 ? v[0] : si == 1 ? v[1] : v[2]; };
  const int sg_n0 = pick(s_n0);
  const int8_t *const sg_b = pick(s_b);
  const int8_t *const sg_b2 = pick(s_b2);
  const float *const sg_bs = pick(s_bs);
  const float *const sg_bs2 = pick(s_bs2);
  // the rows' scales and weights (rows past N reload row N - 1, unused),
  // and for the residual epilogue its operands
  int nr[R];
  float bsn[NMAT][R];
  int4 w[NMAT][R][KB];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    nr[r] = min(row0 + r, N - 1) - sg_n0;  // row within the segment
#pragma unroll
    for (int mi = 0; mi < NMAT; ++mi) {
      bsn[mi][r] = (mi == 0 ? sg_bs : sg_bs2)[nr[r]];
#pragma unroll
      for (int j = 0; j < KB; ++j)
        w[mi][r][j] = *reinterpret_cast<const int4 *>((mi == 0 ? sg_b : sg_b2) +
                                                      static_cast<int64_t>(nr[r]) * (1024 * KB) + 1024 * j + 16 * lane);
    }
  }
  float pv[R];
  if constexpr (NEPI > 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) pv[r] = ps.part[min(lane & 15, ps.npart - 1) * ps.ld_part + sg_n0 + nr[r]];
  }
  __builtin_amdgcn_sched_barrier(0);
  if (NMAT == 2 && threadIdx.x == 0) stage_exp2_table(exptab);
  pro_compute_row<PRO, KB, NP>(a, 0, r0, a_lds, as_lds, blk, blockIdx.x == 0);  // ends with a barrier
  const GemvSeg &sg = a.seg[si];
  int4 av[KB];
  float asg[KB];
#pragma unroll
  for (int j = 0; j < KB; ++j) {
    av[j] = *reinterpret_cast<const int4 *>(a_lds + 1024 * j + 16 * lane);
    asg[j] = as_lds[4 * j + (lane >> 4)];
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float out[NMAT];
#pragma unroll
    for (int mi = 0; mi < NMAT; ++mi) {
      out[mi] = 0.0f;
#pragma unroll
      for (int j = 0; j < KB; ++j) {
        int acc = sdot4(w[mi][r][j].x, av[j].x, 0);
        acc = sdot4(w[mi][r][j].y, av[j].y, acc);
        acc = sdot4(w[mi][r][j].z, av[j].z, acc);
        acc = sdot4(w[mi][r][j].w, av[j].w, acc);
        acc += lane_xor<1>(acc);
        acc += lane_xor<2>(acc);
        acc += lane_xor<4>(acc);
        acc += lane_xor<8>(acc);
        const float p = __fmul_rn(__fmul_rn(static_cast<float>(acc), bsn[mi][r]), asg[j]);
        out[mi] = __fadd_rn(out[mi], lane_bcast<0>(p));
        out[mi] = __fadd_rn(out[mi], lane_bcast<16>(p));
        out[mi] = __fadd_rn(out[mi], lane_bcast<32>(p));
        out[mi] = __fadd_rn(out[mi], lane_bcast<48>(p));
      }
    }
    float *dst = sg.out + nr[r];
    float v = out[0];
    if (sg.epi == EPI_ADD) {
      float base = *dst;
      if constexpr (NEPI > 0) {
        float o = 0.0f;  // the O projection, partials in head order
#pragma unroll
        for (int h = 0; h < NEPI; ++h)
          if (h < ps.npart) o = __fadd_rn(o, __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(pv[r]), h)));
        base = __fadd_rn(base, o);
      }
      v = __fadd_rn(base, out[0]);
    } else if (NMAT == 2 && sg.epi == EPI_SWIGLU) {
      v = swiglu_tab(out[0], out[NMAT - 1], exptab);
    }
    if (lane == 0 && row0 + r < N) *dst = v;
  }
  if (a.clear) {
    // (256 = the block size; blockDim.x would be one more argument read)
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < a.nclear) a.clear[i] = kXwEmpty;
  }
}

// Per (row, head) wave: the head epilogues of the Q/K/V projections
// (kernels/norm_rope_quant.h:17-86, group_gemm.h:173-193), from f32 rows.
__global__ void __launch_bounds__(256) qkv_heads_kernel(QkvHeadArgs a) {
  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x * 4 + wave_id();
  const int nh = a.q_heads + 2 * a.kv_heads;
  if (item >= a.M * nh) return;
  const int m = item / nh;
  const int h = item % nh;
  const float *src;
  QDest d;
  int head;
  bool nrq;
  const float *nw;
  const float *cs;
  const float *sn;
  if (h < a.q_heads) {
    src = a.q + static_cast<int64_t>(m) * a.ldq + h * 128;
    d = a.qd;
    head = h;
    nrq = true;
    nw = a.nq;
    cs = a.cos_q;
    sn = a.sin_q;
  } else if (h < a.q_heads + a.kv_heads) {
    head = h - a.q_heads;
    src = a.k + static_cast<int64_t>(m) * a.ldk + head * 128;
    d = a.kd;
    nrq = true;
    nw = a.nk;
    cs = a.cos_k;
    sn = a.sin_k;
  } else {
    head = h - a.q_heads - a.kv_heads;
    src = a.v + static_cast<int64_t>(m) * a.ldk + head * 128;
    d = a.vd;
    nrq = false;
    nw = nullptr;
    cs = sn = nullptr;
  }
  float t0 = src[lane], t1 = src[lane + 64];
  const int64_t csrow = a.row_pos ? static_cast<int64_t>(a.row_pos[m]) : m;
  if (nrq)
    head_norm_rope(t0, t1, lane, nw, 1, cs + csrow * a.ld_cs, sn + csrow * a.ld_cs, a.inv_hd, true);
  const float mx = max64(fmaxf(fabsf(t0), fabsf(t1)));
  const float scale = __fmul_rn(mx, inv127());
  int8_t *row8;
  float *sp;
  if (d.table) {
    const bool batched = a.row_pos && h >= a.q_heads;  // K/V of independent sequences
    const uint32_t t = batched ? static_cast<uint32_t>(a.row_pos[m]) : d.pos0 + static_cast<uint32_t>(m);
    const uint16_t *table = batched ? a.row_tables + m * a.ld_table : d.table;
    const uint32_t page = table[t / d.page_tokens];
    const uint32_t slot = t % d.page_tokens;
    row8 = d.q8 + page * d.page_bytes + slot * d.row_bytes + head * 128;
    sp = reinterpret_cast<float *>(reinterpret_cast<int8_t *>(d.qs) + page * d.scale_page_bytes +
                                   slot * d.scale_row_bytes) + head;
  } else {
    row8 = d.q8 + static_cast<int64_t>(m) * d.ldq8 + head * 128;
    sp = d.qs + static_cast<int64_t>(m) * d.ldqs + head * d.qs_col;
  }
  row8[lane] = static_cast<int8_t>(quant1(t0, scale));
  row8[lane + 64] = static_cast<int8_t>(quant1(t1, scale));
  if (lane == 0) *sp = scale;
}

template <int GPW, int KSTEPS, int NT, int NMAT, int PRO, int PART, bool BSG = false, int MT = 1, int AB = MT>
hipError_t launch_t(const GemvArgs &a, int ncols, hipStream_t s, int ry = 1) {
  constexpr int NB = 16 * NT;
  // the prologue gives each wave GPW * KSTEPS / 4 groups of 256 columns
  if (PRO != PRO_NONE && a.K != 256 * GPW * KSTEPS) return hipErrorInvalidValue;
  if (a.M > 16 * MT * ry || (ry > 1 && PRO != PRO_NONE)) return hipErrorInvalidValue;
  const int ngroups = a.K / a.group;
  if (MT > 1 && ngroups != 4 * GPW) return hipErrorInvalidValue;  // the scale staging covers 4 * GPW groups
  size_t lds = sizeof(float) * NMAT * ngroups * 16 * MT * (NB + 1);
  if (MT > 1) lds += sizeof(float) * 16 * MT * ngroups;  // the staged A scales
  if (PRO != PRO_NONE)
    lds += ((a.M * a.K + 15) & ~15) + sizeof(float) * (a.M * (a.K / 256) + a.K / 32);
  // dynamic LDS beyond 64 KiB (row tiles) must be allowed once; the kernel's
  // static LDS (the exp table) counts against the same 160 KiB
  constexpr size_t kMaxDyn = 159 * 1024;
  if (lds > (MT > 1 ? kMaxDyn : 65536)) return hipErrorInvalidValue;
  if constexpr (MT > 1) {
    static bool attr_set = false;
    if (!attr_set) {
      const hipError_t e = hipFuncSetAttribute(
          reinterpret_cast<const void *>(&gemv_kernel<GPW, KSTEPS, NT, NMAT, PRO, PART, BSG, MT, AB>),
          hipFuncAttributeMaxDynamicSharedMemorySize, kMaxDyn);
      if (e != hipSuccess) return e;
      attr_set = true;
    }
  }
  Q3_LAUNCH((gemv_kernel<GPW, KSTEPS, NT, NMAT, PRO, PART, BSG, MT, AB>), dim3(ncols / NB, ry), dim3(256), lds, s, a);
  return hipGetLastError();
}

// 17-64 rows (plain A operand, 16-column tiles).  A workgroup streams its
// weights and every row of A it covers, and a CU has only so many cache
// lines in flight, so the rows are split between workgroups (grid rows)
// until the grid holds about two workgroups per CU: narrow launches (O,
// down: 64 column tiles) run one 16-row tile per workgroup, wide ones
// (Q|K|V, gate/up at 64 rows) 2 row tiles over the same weight registers
// (4 when even 2 would exceed that grid).  With three groups per wave
// (K = 3072) the A fragments of 4 tiles come in two batches so that they
// and the weights fit the register file.
template <int NMAT, bool BSG>
hipError_t dispatch_rows(const GemvArgs &a, int ncols, hipStream_t s) {
  constexpr int kMaxWgs = 512;  // fewest row tiles per workgroup that keep the grid within this
  const int cb = ncols / 16;
  const int r1 = (a.M + 15) / 16, r2 = (a.M + 31) / 32;
  const int mt = cb * r1 <= kMaxWgs ? 1 : cb * r2 <= kMaxWgs ? 2 : 4;
#define Q3_ROWS(GPW, KS)                                                                               \
  return mt == 1 ? launch_t<GPW, KS, 1, NMAT, PRO_NONE, 0, BSG>(a, ncols, s, r1)                       \
         : mt == 2 ? launch_t<GPW, KS, 1, NMAT, PRO_NONE, 0, BSG, 2, 2>(a, ncols, s, r2)               \
                : launch_t<GPW, KS, 1, NMAT, PRO_NONE, 0, BSG, 4, (GPW * KS > 8 ? 2 : 4)>(a, ncols, s, 1)
  if (a.K == 1024 && a.group == 256) Q3_ROWS(1, 4);
  if (a.K == 1024 && a.group == 128) Q3_ROWS(2, 2);
  if (a.K == 2048 && a.group == 128) Q3_ROWS(4, 2);
  if (a.K == 2048 && a.group == 256) Q3_ROWS(2, 4);
  if (a.K == 3072 && a.group == 256) Q3_ROWS(3, 4);
#undef Q3_ROWS
  return hipErrorInvalidValue;
}

// The prologue kinds (a template parameter, so that no branch on a kernel
// argument precedes the first loads) are built for K = 1024, 2048 and 3072
// with group 256 and 16-column tiles.
template <int NMAT, int PRO, int PART>
hipError_t dispatch_pro(const GemvArgs &a, int ncols, hipStream_t s) {
  if (a.group != 256) return hipErrorInvalidValue;
  if (a.K == 1024) return launch_t<1, 4, 1, NMAT, PRO, PART>(a, ncols, s);
  if (a.K == 2048) return launch_t<2, 4, 1, NMAT, PRO, PART>(a, ncols, s);
  if (a.K == 3072) return launch_t<3, 4, 1, NMAT, PRO, PART>(a, ncols, s);
  return hipErrorInvalidValue;
}

template <int NT, int NMAT>
hipError_t dispatch_k(const GemvArgs &a, int ncols, hipStream_t s) {
  if constexpr (NMAT == 1) {
    if (a.bs_ld) {  // per-(row, K-group) B scales
      if (a.K == 1024 && a.group == 256) return launch_t<1, 4, NT, 1, PRO_NONE, 0, true>(a, ncols, s);
      if (a.K == 1024 && a.group == 128) return launch_t<2, 2, NT, 1, PRO_NONE, 0, true>(a, ncols, s);
      if (a.K == 2048 && a.group == 128) return launch_t<4, 2, NT, 1, PRO_NONE, 0, true>(a, ncols, s);
      if (a.K == 2048 && a.group == 256) return launch_t<2, 4, NT, 1, PRO_NONE, 0, true>(a, ncols, s);
      if (a.K == 3072 && a.group == 256) return launch_t<3, 4, NT, 1, PRO_NONE, 0, true>(a, ncols, s);
      return hipErrorInvalidValue;
    }
  }
  if (a.pro == PRO_NONE) {
    if (a.K == 1024 && a.group == 256) return launch_t<1, 4, NT, NMAT, PRO_NONE, 0>(a, ncols, s);
    if (a.K == 1024 && a.group == 128) return launch_t<2, 2, NT, NMAT, PRO_NONE, 0>(a, ncols, s);
    if (a.K == 2048 && a.group == 128) return launch_t<4, 2, NT, NMAT, PRO_NONE, 0>(a, ncols, s);
    if (a.K == 2048 && a.group == 256) return launch_t<2, 4, NT, NMAT, PRO_NONE, 0>(a, ncols, s);
    if (a.K == 3072 && a.group == 256) return launch_t<3, 4, NT, NMAT, PRO_NONE, 0>(a, ncols, s);
    return hipErrorInvalidValue;
  }
  if constexpr (NT == 1) {
    if (a.pro == PRO_NORM) return dispatch_pro<NMAT, PRO_NORM, 0>(a, ncols, s);
    if (a.pro == PRO_EMBED) return dispatch_pro<NMAT, PRO_EMBED, 0>(a, ncols, s);
    if (a.pro == PRO_QUANT) return dispatch_pro<NMAT, PRO_QUANT, 0>(a, ncols, s);
  }
  return hipErrorInvalidValue;
}

// With O projection partials (decode): the gate/up launch (PRO_NORM with
// SWIGLU, K = hidden) and the down launch (EPI_ADD, K = intermediate),
// group 256.
template <int NMAT>
hipError_t dispatch_part(const GemvArgs &a, int ncols, hipStream_t s) {
  if (a.M != 1 || a.npart < 1 || a.npart > kMaxPart || a.nseg != 1 || a.group != 256) return hipErrorInvalidValue;
  const bool pro = a.pro == PRO_NORM, epi = a.seg[0].epi == EPI_ADD;
  if (pro == epi || a.ld_part < (pro ? a.K : ncols) ||
      (reinterpret_cast<uintptr_t>(a.part) & 15) != 0 || (a.ld_part % 4) != 0)
    return hipErrorInvalidValue;
  if constexpr (NMAT == 2) {
    if (pro && a.K == 1024) return launch_t<1, 4, 1, NMAT, PRO_NORM, kPartPro>(a, ncols, s);
  } else {
    if (epi && a.K == 3072 && a.pro == PRO_QUANT) {
      return launch_t<3, 4, 1, NMAT, PRO_QUANT, kPartEpi>(a, ncols, s);
    }
  }
  return hipErrorInvalidValue;
}

// One row with a prologue (the decode launches): the whole-row kernel, R
// rows per wave so that each launch has N / (4 R) = 256 workgroups for the
// model's shapes: Q|K|V (K = 1024, 4 rows), gate/up (two matrices, 3 rows),
// down (K = 3072, 1 row).  Returns false where it does not apply.
template <int PRO, int KB, int NMAT, int R, int NP, int NEPI>
hipError_t launch_wr(const GemvArgs &a, int ncols, hipStream_t s) {
  Q3_LAUNCH((gemv_wr_kernel<PRO, KB, NMAT, R, NP, NEPI>), dim3(ncols / (4 * R)), dim3(256), 0, s, a, ncols);
  return hipGetLastError();
}

// R for the whole-row kernel, or 0 where it does not apply
int wr_rows(const GemvArgs &a, int ncols) {
  if (a.M != 1 || a.group != 256 || a.bs_ld || a.pro == PRO_NONE) return 0;
  const int epi = a.seg[0].epi;
  const bool two = epi == EPI_SWIGLU;
  int R;
  if (two) {
    if (a.K != 1024 || a.pro != PRO_NORM || a.nseg != 1) return 0;
    R = 3;
  } else if (a.K == 3072) {
    if (a.pro != PRO_QUANT || a.nseg != 1 || epi != EPI_ADD) return 0;
    R = 1;
  } else if (a.K == 1024) {
    if (a.pro != PRO_NORM && a.pro != PRO_EMBED) return 0;
    R = 2;  // Q|K|V: 512 workgroups (0.7138 -> 0.7108 ms/token against 4 columns per wave)
  } else {
    return 0;
  }
  if (ncols % (4 * R)) return 0;
  if (a.clear && (a.nclear < 0 || static_cast<int64_t>(a.nclear) > static_cast<int64_t>(ncols / (4 * R)) * 256))
    return 0;
  for (int i = 0; i < a.nseg; ++i) {
    const int e = a.seg[i].epi;
    if (a.seg[i].n0 % (4 * R) || (two != (e == EPI_SWIGLU)) || (e != EPI_STORE && e != EPI_ADD && e != EPI_SWIGLU))
      return 0;
  }
  if (a.part) {  // O partials: gate/up's prologue or down's epilogue, as dispatch_part takes them
    const bool pro = a.pro == PRO_NORM;
    if (a.npart < 1 || a.npart > kMaxPart || a.nseg != 1 || pro != two || (!pro && epi != EPI_ADD) ||
        a.ld_part < (pro ? a.K : ncols) || (reinterpret_cast<uintptr_t>(a.part) & 15) != 0 || (a.ld_part % 4) != 0)
      return 0;
  }
  return R;
}

bool wr_launch(const GemvArgs &a, int ncols, hipStream_t s, hipError_t *err) {
  if (!wr_rows(a, ncols)) return false;
  const bool two = a.seg[0].epi == EPI_SWIGLU;
  const bool part = a.part != nullptr;
  if (two)
    *err = part ? launch_wr<PRO_NORM, 1, 2, 3, kMaxPart, 0>(a, ncols, s) : launch_wr<PRO_NORM, 1, 2, 3, 0, 0>(a, ncols, s);
  else if (a.K == 3072)
    *err = part ? launch_wr<PRO_QUANT, 3, 1, 1, 0, kMaxPart>(a, ncols, s) : launch_wr<PRO_QUANT, 3, 1, 1, 0, 0>(a, ncols, s);
  else
    *err = a.pro == PRO_NORM ? launch_wr<PRO_NORM, 1, 1, 2, 0, 0>(a, ncols, s)
                             : launch_wr<PRO_EMBED, 1, 1, 2, 0, 0>(a, ncols, s);
  return true;
}

}  // namespace

bool gemv_supported(int M, int K, int group) {
  if (M < 1 || M > 16) return false;
  return (K == 1024 && (group == 256 || group == 128)) || (K == 2048 && (group == 128 || group == 256)) ||
         (K == 3072 && group == 256);
}

bool gemv_rows_supported(int M, int K, int group, int ncols) {
  return M >= 1 && M <= 64 && ncols < 65536 && gemv_supported(1, K, group);
}

namespace {

int ncols_of(const GemvArgs &a) {
  int ncols = 0;
  for (int i = 0; i < a.nseg; ++i) ncols = a.seg[i].n1;
  return ncols;
}

// Launches that take the column-streaming kernel: one wide segment
// (lm_head: 151936 columns) of STORE or ARGMAX over K = 1024, group 256.
bool use_stream(const GemvArgs &a) {
  const int epi = a.seg[0].epi;
  return a.nseg == 1 && ncols_of(a) >= 65536 && ncols_of(a) % 64 == 0 && a.K == 1024 && a.group == 256 &&
         (epi == EPI_ARGMAX || epi == EPI_STORE);
}

int stream_grid(int ntiles) {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      cus = n;
    else
      cus = 256;
  }
  return std::min(ntiles, 2 * cus);
}

}  // namespace

bool gemv_group_bscale_supported(const GemvArgs &a) {
  const int epi = a.seg[0].epi;
  return a.pro == PRO_NONE && a.nseg == 1 && !a.part && (epi == EPI_STORE || epi == EPI_ADD) &&
         !use_stream(a) && (a.M <= 16 ? gemv_supported(a.M, a.K, a.group)
                                      : gemv_rows_supported(a.M, a.K, a.group, ncols_of(a)));
}

bool gemv_clear_supported(const GemvArgs &a) {
  return a.M == 1 && a.pro != PRO_NONE && a.K % 1024 == 0 && !use_stream(a) && wr_rows(a, ncols_of(a)) > 0;
}

int gemv_argmax_slots(const GemvArgs &a) {
  const int ncols = ncols_of(a);
  if (use_stream(a)) return stream_grid(ncols / 64);
  return ncols / (ncols >= 65536 ? 64 : 16);
}

hipError_t launch_gemv(const GemvArgs &a, hipStream_t s) {
  if (a.M <= 0) return hipSuccess;
  if (a.clear && !gemv_clear_supported(a)) return hipErrorInvalidValue;
  if (a.bs_ld && !gemv_group_bscale_supported(a)) return hipErrorInvalidValue;
  if (a.pro != PRO_NONE && (a.K % 1024 != 0 || a.M > 16)) return hipErrorInvalidValue;
  const int ncols = ncols_of(a);
  if (use_stream(a) && a.M == 1) {  // one row: whole-row v_dot4 streaming
    const dim3 grid(stream_grid(ncols / 64));
    constexpr int R = 4;
    switch (a.pro) {
      case PRO_NONE: Q3_LAUNCH((gemv_row_kernel<PRO_NONE, R>), grid, dim3(256), 0, s, a, ncols); break;
      case PRO_NORM: Q3_LAUNCH((gemv_row_kernel<PRO_NORM, R>), grid, dim3(256), 0, s, a, ncols); break;
      case PRO_EMBED: Q3_LAUNCH((gemv_row_kernel<PRO_EMBED, R>), grid, dim3(256), 0, s, a, ncols); break;
      case PRO_QUANT: Q3_LAUNCH((gemv_row_kernel<PRO_QUANT, R>), grid, dim3(256), 0, s, a, ncols); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  if (use_stream(a)) {
    if (a.M > 16) return hipErrorInvalidValue;
    const int ntiles = ncols / 64;
    const size_t lds = sizeof(float) * 4 * 16 * 65 +
                       (a.pro != PRO_NONE ? ((a.M * a.K + 15) & ~15) + sizeof(float) * (a.M * 4 + 32) : 0);
    const dim3 grid(stream_grid(ntiles));
    switch (a.pro) {
      case PRO_NONE: Q3_LAUNCH((gemv_stream_kernel<1, 4, 4, PRO_NONE>), grid, dim3(256), lds, s, a, ntiles); break;
      case PRO_NORM: Q3_LAUNCH((gemv_stream_kernel<1, 4, 4, PRO_NORM>), grid, dim3(256), lds, s, a, ntiles); break;
      case PRO_EMBED: Q3_LAUNCH((gemv_stream_kernel<1, 4, 4, PRO_EMBED>), grid, dim3(256), lds, s, a, ntiles); break;
      case PRO_QUANT: Q3_LAUNCH((gemv_stream_kernel<1, 4, 4, PRO_QUANT>), grid, dim3(256), lds, s, a, ntiles); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  {
    hipError_t err = hipSuccess;
    if (wr_launch(a, ncols, s, &err)) return err;
  }
  const bool two = a.seg[0].epi == EPI_SWIGLU;
  if (a.M > 16) {  // a batch of rows: plain A operand, no partials, 16-column tiles
    if (a.pro != PRO_NONE || a.part || !gemv_rows_supported(a.M, a.K, a.group, ncols)) return hipErrorInvalidValue;
    if (two) return dispatch_rows<2, false>(a, ncols, s);
    return a.bs_ld ? dispatch_rows<1, true>(a, ncols, s) : dispatch_rows<1, false>(a, ncols, s);
  }
  if (a.part) return two ? dispatch_part<2>(a, ncols, s) : dispatch_part<1>(a, ncols, s);
  if (two) return dispatch_k<1, 2>(a, ncols, s);
  if (ncols >= 65536) return dispatch_k<4, 1>(a, ncols, s);
  return dispatch_k<1, 1>(a, ncols, s);
}

hipError_t launch_qkv_heads(const QkvHeadArgs &a, hipStream_t s) {
  const int items = a.M * (a.q_heads + 2 * a.kv_heads);
  if (items <= 0) return hipSuccess;
  hipLaunchKernelGGL(qkv_heads_kernel, dim3((items + 3) / 4), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace q3
