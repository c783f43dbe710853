// Prefill-sized per-group int8 GEMM (M > 64), weights streamed to registers.
//
// Arithmetic of kernels/group_gemm.h:27-222 / ref_qwen3.py:145-158, with the
// epilogues of group_gemm.h:173-214 (V quant, residual add),
// norm_rope_quant.h:17-86 (Q/K) and swiglu_quant.h:164-255 (gate/up):
//   D[m,n] = sum over K-groups g, in order from +0.0f, of
//            RN(RN(f32(I_g[m,n]) * bs[n]) * as[m,g])
// (bs[n][g] with per-group B scales), I_g the exact int32 dot product of
// group g (v_mfma_i32_16x16x64_i8).
//
// Decomposition.  A workgroup of NW waves owns a BM x BN output tile (for
// gate/up: BN columns of both matrices, i.e. whole 256-column quantisation
// groups of the SwiGLU output).  The A rows of the tile (BM x K int8, shared
// by every wave) and the scales are copied global -> LDS once, with
// global_load_lds (no registers), 16-byte chunks XOR-swizzled by row so that
// a fragment read of 16 rows hits every LDS bank; one barrier follows.
// Each wave owns NT * 16 columns of each matrix and streams those weight rows
// straight into registers: a ring of D k-slices (64 bytes of K each) is kept
// in flight, the slice in use being consumed by the MFMAs while the next D - 1
// arrive.  No wave ever waits for another wave inside the main loop, so there
// is no per-step barrier, and a CU keeps NW * D * NT * NMAT KiB of weights in
// flight (128 KiB for gate/up), enough to cover last-level-cache latency.
//
// Per-group dequantisation: 4 VALU operations per output element and group
// (cvt, two RN multiplies, add).  The int32 group sums are double buffered by
// group parity: group g is dequantised right after the first MFMAs of group
// g + 1 are issued, so the VALU work of one group overlaps the MFMAs of the
// next.
//
// Tile order: workgroup i runs on XCD i % 8 (round-robin dispatch); the tiles
// are numbered so that consecutive tiles share a column block (the same
// weight rows) and each XCD takes a contiguous run of them, so a weight tile
// is read from HBM once per XCD and then from that XCD's L2.
#include <algorithm>

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

// NWN waves across the columns times KP partitions of K (NW = NWN * KP).
template <int BM, int NWN, int KP, int NT, int NMAT, int D, int KB>
struct StreamShape {
  static constexpr int NW = NWN * KP;
  static constexpr int NTHR = NW * 64;
  static constexpr int MT = BM / 16;         // 16-row MFMA tiles per wave
  static constexpr int WN = NT * 16;         // columns per wave (per matrix)
  static constexpr int BN = NWN * WN;        // columns per workgroup (per matrix)
  static constexpr int K = 1024 * KB;
  static constexpr int SLICES = K / 64;      // MFMA k-slices
  static constexpr int SW = SLICES / KP;     // k-slices per wave
  static constexpr int LPS = NMAT * NT;      // weight loads (1 KiB per wave) per slice
  static constexpr int A_INSTR = BM * K / 1024;  // A copy instructions (1 KiB each)
  static constexpr int LDT = BN + 4;         // f32 epilogue tile pitch
  static_assert(BM % 16 == 0 && A_INSTR % NW == 0, "A copies: whole instructions per wave");
  static_assert(D >= 2 && (D - 1) * LPS < 64, "vmcnt range");
};

// Tile i of a column-major order (consecutive tiles share a column block),
// with XCD x = id % 8 taking the x-th contiguous run of tiles.
__device__ __forceinline__ void xcd_tile(int id, int total, int tiles_m, int *n_tile, int *m_tile) {
  const int q = total / 8, r = total % 8;
  const int x = id % 8, k = id / 8;
  const int u = x * q + min(x, r) + k;
  *n_tile = u / tiles_m;
  *m_tile = u % tiles_m;
}

// LDS address of A row r, 16-byte chunk c (chunks XOR-swizzled by row).
__device__ __forceinline__ int a_off(int r, int c, int K) { return r * K + 16 * (c ^ (r & 7)); }

template <int BM, int NWN, int KP, int NT, int NMAT, int D, int KB, int EPI, int GROUP, bool BSG>
__global__ void __launch_bounds__(NWN * KP * 64) gemm_stream_kernel(TileArgs a) {
  using S = StreamShape<BM, NWN, KP, NT, NMAT, D, KB>;
  constexpr int MT = S::MT, K = S::K, NW = S::NW;
  constexpr int NG = K / GROUP;              // K-groups
  constexpr int SPG = GROUP / 64;            // slices per group
  // one loop iteration covers BODY slices (whole groups, an even number of
  // them, and a whole number of ring turns)
  constexpr int BODY = D > 2 * SPG ? D : 2 * SPG;
  constexpr int GPB = BODY / SPG;
  static_assert(BODY % D == 0 && BODY % (2 * SPG) == 0 && (KP > 1 || NG % GPB == 0), "loop body");
  constexpr int GPP = NG / KP;               // groups per K partition
  static_assert(NG % KP == 0 && (KP == 1 || NMAT == 1), "K partitions");
  static_assert(KP == 1 || EPI == EPI_STORE || EPI == EPI_ADD, "K partitions: plain epilogues");
  static_assert(!BSG || (NMAT == 1 && (EPI == EPI_STORE || EPI == EPI_ADD)), "per-group B scales");
  extern __shared__ __align__(16) int8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int wn = wave % NWN;                 // column block of the wave
  const int kp = wave / NWN;                 // its K partition
  const int s0 = kp * S::SW;                 // its first k-slice
  const int lr = lane & 15;
  const int lg = lane >> 4;
  const int M = a.M;
  const int tiles_m = (M + BM - 1) / BM;
  int n_tile, m_tile;
  xcd_tile(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x), tiles_m, &n_tile, &m_tile);
  const int m0 = m_tile * BM;
  const int n0 = n_tile * S::BN;
  // the tile's column segment (EPI_QKV: Q, K or V; else the single matrix)
  const int8_t *B0 = a.b0;
  const float *BS0 = a.bs0;
  int nb = n0;
  QDest qd = a.qd;
  const float *nw = a.nw;
  bool do_norm = EPI == EPI_NRQ;
  if constexpr (EPI == EPI_QKV) {
    // every segment's fields are kernel arguments at fixed offsets: select
    // among them rather than index, so no argument load waits on another
    const int si = (a.nseg > 1 && n0 >= a.seg[1].n0) + (a.nseg > 2 && n0 >= a.seg[2].n0);
    const auto &s0g = a.seg[0], &s1g = a.seg[1], &s2g = a.seg[2];
    B0 = si == 2 ? s2g.b : si == 1 ? s1g.b : s0g.b;
    BS0 = si == 2 ? s2g.bs : si == 1 ? s1g.bs : s0g.bs;
    nb = n0 - (si == 2 ? s2g.n0 : si == 1 ? s1g.n0 : s0g.n0);
    qd = si == 2 ? s2g.qd : si == 1 ? s1g.qd : s0g.qd;
    nw = si == 2 ? s2g.nw : si == 1 ? s1g.nw : s0g.nw;
    do_norm = (si == 2 ? s2g.norm : si == 1 ? s1g.norm : s0g.norm) != 0;
  }
  // LDS: exp table | A scales [BM][NG] | B scales [BN][NG] (BSG) | A tile [BM][K];
  // after the main loop the f32 epilogue tile overlays everything past the table
  uint64_t *tab = reinterpret_cast<uint64_t *>(smem);
  float *as_lds = reinterpret_cast<float *>(smem + 256);
  float *bs_lds = as_lds + BM * NG;
  int8_t *a_lds = reinterpret_cast<int8_t *>(bs_lds + (BSG ? S::BN * NG : 0));
  float *tile = as_lds;

  // 0. the epilogue's global operands first: issued before every copy and
  //    weight load, they complete first, so the main loop's vmcnt counts are
  //    unchanged and their latency hides behind the weight stream.  EPI_ADD:
  //    the residual elements of the lane (last K partition; rows past M read
  //    row M - 1 and store nothing).  Head epilogues: gains, cos/sin rows and
  //    page ids of the wave's rows (rows past M: row M - 1's).
  float xr[MT][4][NT];
  if constexpr (EPI == EPI_ADD) {
    if (kp == KP - 1) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = min(m0 + mt * 16 + lg * 4 + i, M - 1);
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
            xr[mt][i][nt] = a.out[static_cast<int64_t>(m) * a.ldo + n0 + wn * S::WN + nt * 16 + lr];
        }
    }
  }
  constexpr bool HEADS = EPI == EPI_HEADQ || EPI == EPI_NRQ || EPI == EPI_QKV;
  constexpr int RPW = (BM + NW - 1) / NW;  // head epilogue rows per wave
  // loads that depend on another global load (device-side positions, per-row
  // tables) wait for the epilogue; only independent ones are issued here
  const bool pre_cs = do_norm && !a.cs_row_pos && !a.cs_row_dev;
  const bool pre_pg = qd.table && !qd.pos_dev && !qd.row_pos;
  float hw0 = 0.0f, hw1 = 0.0f, hcr[RPW], hsr[RPW];
  // pre_pg: lane q < RPW holds the page id of the wave's row q (a per-lane
  // value, so nothing waits for it before the epilogue reads it)
  uint32_t hpg = 0;
  if constexpr (HEADS) {
    if (do_norm) {
      hw0 = nw[static_cast<int64_t>(lane) * a.nw_stride];
      hw1 = nw[static_cast<int64_t>(lane + 64) * a.nw_stride];
    }
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
      const int mm = min(m0 + min(wave + NW * q, BM - 1), M - 1);
      hcr[q] = hsr[q] = 0.0f;
      if (pre_cs) {
        hcr[q] = a.cos_t[static_cast<int64_t>(mm) * a.ld_cs + lane];
        hsr[q] = a.sin_t[static_cast<int64_t>(mm) * a.ld_cs + lane];
      }
    }
    if (pre_pg && lane < RPW) {
      const int mm = min(m0 + min(wave + NW * lane, BM - 1), M - 1);
      hpg = qd.table[(qd.pos0 + static_cast<uint32_t>(mm)) / qd.page_tokens];
    }
  }

  // 1. scales and the A tile -> LDS.  Instruction j of the A copy fills LDS
  //    bytes [1024 j, 1024 j + 1024) of the tile: row r = j / KB, chunks
  //    c0 .. c0 + 63 with c0 = 64 (j % KB); lane i writes physical chunk
  //    c0 + i, which holds logical chunk (c0 + i) ^ (r & 7).  Rows past M
  //    copy row M - 1 (computed, never stored).
  if (wave == 0) {
    for (int e0 = 0; e0 < BM * NG; e0 += 64) {
      const int e = min(e0 + lane, BM * NG - 1);
      const int r = e / NG, g = e % NG;
      const float *src = a.as + static_cast<int64_t>(min(m0 + r, M - 1)) * a.ldas + g;
      __builtin_amdgcn_global_load_lds(const_cast<float *>(src), to_lds(as_lds + e0), 4, 0, 0);
    }
    if constexpr (BSG) {
      for (int e0 = 0; e0 < S::BN * NG; e0 += 64) {
        const int e = min(e0 + lane, S::BN * NG - 1);
        const int c = e / NG, g = e % NG;
        const float *src = BS0 + static_cast<int64_t>(nb + c) * a.bs_ld + g;
        __builtin_amdgcn_global_load_lds(const_cast<float *>(src), to_lds(bs_lds + e0), 4, 0, 0);
      }
    }
  }
#pragma unroll
  for (int q = 0; q < S::A_INSTR / NW; ++q) {
    const int j = wave + NW * q;
    const int r = j / KB;
    const int c0 = 64 * (j % KB);
    const int c = (c0 + lane) ^ (r & 7);
    const int8_t *src = a.a + static_cast<int64_t>(min(m0 + r, M - 1)) * a.lda + 16 * c;
    __builtin_amdgcn_global_load_lds(const_cast<int8_t *>(src), to_lds(a_lds + 1024 * j), 16, 0, 0);
  }
  if (EPI == EPI_SWIGLUQ && threadIdx.x == 0) stage_exp2_table(tab);
  // keep every copy above issued before the weight loads below: the wait
  // before the first barrier counts on the copies being the older loads
  __builtin_amdgcn_sched_barrier(0);

  // 2. per-row B scales (registers), then the first D slices of the weights
  float bsv[NMAT][NT];
  if constexpr (!BSG) {
#pragma unroll
    for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const float *bs = mi == 0 ? BS0 : a.bs1;
        bsv[mi][nt] = bs[static_cast<int64_t>(nb + wn * S::WN + nt * 16 + lr) * a.bs_stride];
      }
  }
  // a fragment (16 weight rows x 64 bytes of K) per lane load: row-major
  // weights give lane (lr, lg) row lr, bytes 16 lg of the slice (16 rows at
  // the row stride); packed weights hold each fragment as 1 KiB, lane order
  const int8_t *brow[NMAT][NT];
  const int64_t sstride = a.b_packed ? 1024 : 64;
#pragma unroll
  for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int8_t *bm = mi == 0 ? B0 : a.b1;
      const int64_t col = nb + wn * S::WN + nt * 16;
      brow[mi][nt] = a.b_packed ? bm + ((col / 16) * S::SLICES + s0) * 1024 + 16 * lane
                                : bm + (col + lr) * a.ldb + 64 * s0 + 16 * lg;
    }
  v4i ring[D][NMAT][NT];
  auto issue = [&](auto SLOT, int s) {
    constexpr int slot = decltype(SLOT)::value;
    const int64_t k = sstride * min(s, S::SW - 1);  // past the end: re-read the last slice (unused)
#pragma unroll
    for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        ring[slot][mi][nt] = *reinterpret_cast<const v4i *>(brow[mi][nt] + k);
  };
  static_for<D>([&](auto J) { issue(J, decltype(J)::value); });

  float acc[NMAT][MT][NT][4];
#pragma unroll
  for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[mi][mt][nt][i] = 0.0f;
  v4i c[2][NMAT][MT][NT];
#pragma unroll
  for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) c[0][mi][mt][nt] = c[1][mi][mt][nt] = zero4();

  // every wave's A and scale copies are in LDS once slice 0 has arrived
  // (loads complete in order and the copies were issued first)
  wait_vmcnt<(D - 1) * S::LPS>();
  lds_barrier();

  // acc += RN(RN(f32(c) * bs) * as[m][g]); then c = 0 for the buffer's next group
  auto dequant = [&](auto PAR, int g) {
    constexpr int b = decltype(PAR)::value;
    if constexpr (BSG) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) bsv[0][nt] = bs_lds[(wn * S::WN + nt * 16 + lr) * NG + g];
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float asv = as_lds[(mt * 16 + lg * 4 + i) * NG + g];
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

  // the slice s of this wave: MFMAs on it from ring slot `slot` into
  // buffer `par`, then (ISSUE) slice s + D into that slot.  AFTER: slices
  // issued after this one (D - 1, fewer near the end, where no slice past
  // the wave's last is issued: a wave cannot finish, nor pass a barrier,
  // before every load it issued has returned)
  auto slice = [&](auto SLOT, auto PAR, auto AFTER, auto ISSUE, int s) {
    constexpr int slot = decltype(SLOT)::value;
    constexpr int par = decltype(PAR)::value;
    constexpr int after = decltype(AFTER)::value;
    wait_vmcnt<after * S::LPS>();
    v4i af[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      af[mt] = *reinterpret_cast<const v4i *>(a_lds + a_off(mt * 16 + lr, 4 * (s0 + s) + lg, K));
#pragma unroll
    for (int mi = 0; mi < NMAT; ++mi)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          c[par][mi][mt][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[mt], ring[slot][mi][nt],
                                                                       c[par][mi][mt][nt], 0, 0, 0);
    if constexpr (decltype(ISSUE)::value) issue(std::integral_constant<int, slot>{}, s + D);
  };

  if constexpr (KP == 1) {
    // 3. main loop, GPB groups per iteration; group g accumulates in buffer
    //    g & 1, and slice s of the kernel lives in ring slot s % D; the last
    //    iteration (LAST) issues no slice past the end
    auto body = [&](auto LAST, int g0) {
      static_for<BODY>([&](auto J) {
        constexpr int j = decltype(J)::value;
        constexpr bool last = decltype(LAST)::value;
        constexpr int after = last ? (D - 1 < BODY - 1 - j ? D - 1 : BODY - 1 - j) : D - 1;
        slice(std::integral_constant<int, j % D>{}, std::integral_constant<int, (j / SPG) & 1>{},
              std::integral_constant<int, after>{}, std::integral_constant<bool, !last || j + D < BODY>{},
              g0 * SPG + j);
        // at a group's first slice: the previous group, whose MFMAs are all
        // issued, is dequantised while these run
        if constexpr (j % SPG == 0) {
          const int g = g0 + j / SPG;
          if (g > 0) dequant(std::integral_constant<int, ((j / SPG) & 1) ^ 1>{}, g - 1);
        }
      });
    };
#pragma unroll 1
    for (int g0 = 0; g0 < NG - GPB; g0 += GPB) body(std::false_type{}, g0);
    body(std::true_type{}, NG - GPB);
    dequant(std::integral_constant<int, (NG - 1) & 1>{}, NG - 1);
  } else {
    // 3'. K partitions: the wave's GPP groups, each dequantised into a
    //     partial of its own (p = RN(RN(f32(I_g) * bs) * as)); then the
    //     partitions' partials are summed in group order: partition t adds
    //     its groups to the running sum partition t - 1 left in LDS
    float part[GPP][MT][NT][4];
    static_for<GPP>([&](auto GI) {
      constexpr int gi = decltype(GI)::value;
      static_for<SPG>([&](auto J) {
        constexpr int j = gi * SPG + decltype(J)::value;
        constexpr int after = D - 1 < S::SW - 1 - j ? D - 1 : S::SW - 1 - j;
        slice(std::integral_constant<int, j % D>{}, std::integral_constant<int, 0>{},
              std::integral_constant<int, after>{}, std::integral_constant<bool, (j + D < S::SW)>{}, j);
      });
      dequant(std::integral_constant<int, 0>{}, kp * GPP + gi);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            part[gi][mt][nt][i] = acc[0][mt][nt][i];
            acc[0][mt][nt][i] = 0.0f;
          }
    });
    float *chain = reinterpret_cast<float *>(a_lds + BM * K);  // [BM][LDT]
    static_for<KP>([&](auto T) {
      constexpr int t = decltype(T)::value;
      if (kp == t) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              float v = 0.0f;
              if constexpr (t > 0) v = chain[(mt * 16 + lg * 4 + i) * S::LDT + wn * S::WN + nt * 16 + lr];
#pragma unroll
              for (int gi = 0; gi < GPP; ++gi) v = __fadd_rn(v, part[gi][mt][nt][i]);
              if constexpr (t + 1 < KP)
                chain[(mt * 16 + lg * 4 + i) * S::LDT + wn * S::WN + nt * 16 + lr] = v;
              else
                acc[0][mt][nt][i] = v;
            }
      }
      if constexpr (t + 1 < KP) __syncthreads();
    });
  }

  // 4. epilogues
  if constexpr (EPI == EPI_STORE || EPI == EPI_ADD) {
    if (kp != KP - 1) return;  // the last K partition holds the sums
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = m0 + mt * 16 + lg * 4 + i;
        if (m >= M) continue;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          float *dst = a.out + static_cast<int64_t>(m) * a.ldo + n0 + wn * S::WN + nt * 16 + lr;
          if constexpr (EPI == EPI_ADD)
            *dst = __fadd_rn(xr[mt][i][nt], acc[0][mt][nt][i]);
          else
            *dst = acc[0][mt][nt][i];
        }
      }
  } else {
    // f32 tile through LDS so that a wave can walk whole rows
    __syncthreads();
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          float v = acc[0][mt][nt][i];
          if constexpr (EPI == EPI_SWIGLUQ) v = swiglu_tab(acc[0][mt][nt][i], acc[NMAT - 1][mt][nt][i], tab);
          tile[(mt * 16 + lg * 4 + i) * S::LDT + wn * S::WN + nt * 16 + lr] = v;
        }
    __syncthreads();
    if constexpr (EPI == EPI_HEADQ || EPI == EPI_NRQ || EPI == EPI_QKV) {
      // group_gemm.h:173-193 / norm_rope_quant.h:17-86 per (row, head), on
      // the operands loaded at the start (step 0) where they were independent
      // of other loads; rows past M store nothing
      static_assert(S::BN == 128, "one head (128 columns) per tile");
#pragma unroll
      for (int q = 0; q < RPW; ++q) {
        const int rr = min(wave + NW * q, BM - 1);
        const bool store = wave + NW * q < BM && m0 + rr < M;
        const int mm = min(m0 + rr, M - 1);
        int8_t *row8;
        float *sp;
        if (pre_pg)
          qdest_slot(qd, __builtin_amdgcn_readlane(hpg, q), qd.pos0 + static_cast<uint32_t>(mm), nb / 128, &row8,
                     &sp);
        else
          qdest_row(qd, mm, nb / 128, &row8, &sp);
        if (do_norm && !pre_cs) {
          const int64_t crow = a.cs_row_pos ? static_cast<int64_t>(a.cs_row_pos[mm])
                                            : mm + static_cast<int64_t>(a.cs_row_dev ? *a.cs_row_dev : 0);
          hcr[q] = a.cos_t[crow * a.ld_cs + lane];
          hsr[q] = a.sin_t[crow * a.ld_cs + lane];
        }
        float t0 = tile[rr * S::LDT + lane];
        float t1 = tile[rr * S::LDT + lane + 64];
        if (do_norm) head_norm_rope_regs(t0, t1, hw0, hw1, hcr[q], hsr[q], a.inv_hd, true);
        const float mx = max64(fmaxf(fabsf(t0), fabsf(t1)));
        const float scale = __fmul_rn(mx, inv127());
        const double y = rcp64(scale);
        const int8_t q0 = static_cast<int8_t>(quant_rcp(t0, y));
        const int8_t q1 = static_cast<int8_t>(quant_rcp(t1, y));
        if (store) {
          row8[lane] = q0;
          row8[lane + 64] = q1;
          if (lane == 0) *sp = scale;
        }
      }
    } else if constexpr (EPI == EPI_SWIGLUQ) {
      // swiglu_quant.h:195-231: per 256-column group absmax * (1/127)
      static_assert(S::BN % 256 == 0, "whole quantisation groups");
      for (int rr = wave; rr < BM; rr += NW) {
        const int m = m0 + rr;
        if (m >= M) break;
#pragma unroll
        for (int q = 0; q < S::BN / 256; ++q) {
          float v[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) v[j] = tile[rr * S::LDT + q * 256 + lane + 64 * j];
          float mx = 0.0f;
#pragma unroll
          for (int j = 0; j < 4; ++j) mx = fmaxf(mx, fabsf(v[j]));
          mx = max64(mx);
          const float scale = __fmul_rn(mx, inv127());
          const double y = rcp64(scale);
          int8_t *dst = a.s8 + static_cast<int64_t>(m) * a.lds8 + n0 + q * 256;
#pragma unroll
          for (int j = 0; j < 4; ++j) dst[lane + 64 * j] = static_cast<int8_t>(quant_rcp(v[j], y));
          if (lane == 0) a.ss[static_cast<int64_t>(m) * a.ldss + ((n0 + q * 256) / 256) * a.ss_col] = scale;
        }
      }
    }
  }
}

template <int BM, int NWN, int KP, int NT, int NMAT, int D, int KB, int EPI, int GROUP, bool BSG>
hipError_t launch_one(const TileArgs &a, hipStream_t s) {
  using S = StreamShape<BM, NWN, KP, NT, NMAT, D, KB>;
  constexpr int NG = S::K / GROUP;
  size_t lds = 256 + sizeof(float) * (BM + (BSG ? S::BN : 0)) * NG + static_cast<size_t>(BM) * S::K;
  if (KP > 1) lds += sizeof(float) * BM * S::LDT;  // the partitions' running sums
  if (EPI != EPI_STORE && EPI != EPI_ADD) lds = std::max(lds, 256 + sizeof(float) * BM * S::LDT);
  if (lds > 160 * 1024) return hipErrorInvalidValue;
  static bool attr_set = false;  // more than 64 KiB of dynamic LDS must be allowed once
  if (!attr_set) {
    const hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void *>(&gemm_stream_kernel<BM, NWN, KP, NT, NMAT, D, KB, EPI, GROUP, BSG>),
        hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int tiles = (a.N / S::BN) * ((a.M + BM - 1) / BM);
  Q3_LAUNCH((gemm_stream_kernel<BM, NWN, KP, NT, NMAT, D, KB, EPI, GROUP, BSG>), dim3(tiles), dim3(S::NTHR), lds,
            s, a);
  return hipGetLastError();
}

template <int BM, int NWN, int KP, int NT, int NMAT, int D, int EPI, bool BSG>
hipError_t launch_k(const TileArgs &a, hipStream_t s) {
  const int kb = a.K / 1024;
  if (a.group == 256) {
    if (kb == 1) return launch_one<BM, NWN, KP, NT, NMAT, D, 1, EPI, 256, BSG>(a, s);
    if (kb == 2) return launch_one<BM, NWN, KP, NT, NMAT, D, 2, EPI, 256, BSG>(a, s);
    if (kb == 3) return launch_one<BM, NWN, KP, NT, NMAT, D, 3, EPI, 256, BSG>(a, s);
  } else if (a.group == 128) {
    if (kb == 1) return launch_one<BM, NWN, KP, NT, NMAT, D, 1, EPI, 128, BSG>(a, s);
    if (kb == 2) return launch_one<BM, NWN, KP, NT, NMAT, D, 2, EPI, 128, BSG>(a, s);
    if (kb == 3) return launch_one<BM, NWN, KP, NT, NMAT, D, 3, EPI, 128, BSG>(a, s);
  }
  return hipErrorInvalidValue;
}

// STORE / ADD: 16 waves per workgroup, as 8 column blocks x 2 K partitions
// (128-column tiles) when those give at least one workgroup per CU, else
// 4 column blocks x 4 K partitions (64-column tiles).
template <int EPI, bool BSG>
hipError_t launch_plain(const TileArgs &a, hipStream_t s) {
  const int tiles_m = (a.M + 31) / 32;
  if (a.N % 128 == 0 && (a.N / 128) * tiles_m >= 256) return launch_k<32, 8, 2, 1, 1, 8, EPI, BSG>(a, s);
  return launch_k<32, 4, 4, 1, 1, 4, EPI, BSG>(a, s);
}

// One thread per 16-byte chunk of the packed matrix: chunk p = (fragment
// f, lane l), fragment f = (16-row block nb, k-slice s) = nb * S + s.
__global__ void __launch_bounds__(256) pack_b_kernel(const int8_t *b, int64_t ldb, int N, int K,
                                                      int8_t *out) {
  const int S = K / 64;
  const int64_t total = static_cast<int64_t>(N / 16) * S * 64;
  const int64_t p = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (p >= total) return;
  const int l = static_cast<int>(p % 64);
  const int64_t f = p / 64;
  const int s = static_cast<int>(f % S);
  const int64_t nb = f / S;
  const v4i v = *reinterpret_cast<const v4i *>(b + (nb * 16 + (l & 15)) * ldb + 64 * s + 16 * (l >> 4));
  *reinterpret_cast<v4i *>(out + 16 * p) = v;
}

}  // namespace

hipError_t launch_pack_b(const int8_t *b, int64_t ldb, int N, int K, int8_t *out, hipStream_t s) {
  if (N % 16 || K % 64 || ldb < K || (ldb % 16) || (reinterpret_cast<uintptr_t>(b) & 15) ||
      (reinterpret_cast<uintptr_t>(out) & 15))
    return hipErrorInvalidValue;
  const int64_t chunks = static_cast<int64_t>(N / 16) * (K / 64) * 64;
  if (chunks == 0) return hipSuccess;
  hipLaunchKernelGGL(pack_b_kernel, dim3(static_cast<unsigned>((chunks + 255) / 256)), dim3(256), 0, s, b, ldb,
                     N, K, out);
  return hipGetLastError();
}

bool gemm_stream_supported(const TileArgs &a, int epi) {
  if (a.M <= 64 || a.K % 1024 || a.K > 3072 || (a.group != 256 && a.group != 128)) return false;
  auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (!al16(a.a) || (a.lda % 16) || (!a.b_packed && (a.ldb % 16))) return false;
  if (epi != EPI_QKV && !al16(a.b0)) return false;
  switch (epi) {
    case EPI_STORE:
    case EPI_ADD: return a.N % 64 == 0;
    case EPI_HEADQ:
    case EPI_NRQ: return !a.bs_ld && a.N % 128 == 0;
    case EPI_QKV: return !a.bs_ld && a.N % 128 == 0;
    case EPI_SWIGLUQ: return !a.bs_ld && a.N % 256 == 0 && a.b1 && al16(a.b1);
    default: return false;
  }
}

hipError_t launch_gemm_stream(const TileArgs &a, int epi, hipStream_t s) {
  if (!gemm_stream_supported(a, epi)) return hipErrorInvalidValue;
  switch (epi) {
    case EPI_STORE: return a.bs_ld ? launch_plain<EPI_STORE, true>(a, s) : launch_plain<EPI_STORE, false>(a, s);
    case EPI_ADD: return a.bs_ld ? launch_plain<EPI_ADD, true>(a, s) : launch_plain<EPI_ADD, false>(a, s);
    case EPI_HEADQ: return launch_k<32, 8, 1, 1, 1, 16, EPI_HEADQ, false>(a, s);
    case EPI_NRQ: return launch_k<32, 8, 1, 1, 1, 16, EPI_NRQ, false>(a, s);
    case EPI_QKV:
      if (a.nseg < 1 || a.nseg > 3 || a.seg[0].n0 != 0 || a.seg[a.nseg - 1].n1 != a.N) return hipErrorInvalidValue;
      for (int i = 0; i < a.nseg; ++i)
        if (a.seg[i].n0 % 128 || a.seg[i].n1 % 128 || a.seg[i].n1 <= a.seg[i].n0 ||
            (i > 0 && a.seg[i].n0 != a.seg[i - 1].n1) || (reinterpret_cast<uintptr_t>(a.seg[i].b) & 15))
          return hipErrorInvalidValue;
      return launch_k<32, 8, 1, 1, 1, 16, EPI_QKV, false>(a, s);
    case EPI_SWIGLUQ: return launch_k<32, 16, 1, 1, 2, 4, EPI_SWIGLUQ, false>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace q3
