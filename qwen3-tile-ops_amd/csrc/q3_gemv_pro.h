// Consumer-side operand prologue of the decode GEMVs: the int8 A operand
// of M rows built in LDS from f32 rows (RMSNorm + per-256 quant, the
// embedding gather, or quant alone), with the reference's rounding points.
// Shared by k_gemv.hip and the fused Q|K|V + attention kernel
// (k_attn_decode.hip), which runs it in 12-wave workgroups: waves 4.. load
// the same operands as wave (w & 3) (a fixed load count) and skip the
// arithmetic, but reach every barrier.
#pragma once

#include "q3_device.h"
#include "q3_kernels.h"

namespace q3 {
namespace {

// the most O projection partials (query heads) a decode GEMV adds
constexpr int kMaxPart = 16;

// The prologue builds the int8 A operand of M rows (K = 1024*QW columns,
// 256-column groups) in LDS.  Thread layout: wave w owns groups w, w+4, ...
// (QW of them); lane l owns columns 4l..4l+3 of a group, so a 32-column
// RMSNorm block is 8 lanes (the reference's pairwise tree: in-thread pairs,
// then xor 1/2/4), and a quantisation group is one wave.
//
// A row's global operands are loaded into registers in one go
// (pro_load_row) before any of them is used.  The kernel loads row 0 before
// it issues the weight stream: vector loads return in order, so operands
// requested after the weights would wait for all of them.
template <int QW, int NP>
struct ProRow {
  float4 x[QW];     // f32 row (PRO_NORM / PRO_QUANT)
  float4 w[QW];     // RMSNorm gain (PRO_NORM / PRO_EMBED)
  uint32_t e[QW];   // four int8 embedding values (PRO_EMBED)
  float esc;        // embedding row scale
  float4 p[QW][NP > 0 ? NP : 1];  // O projection partials (GemvArgs::part)
  int npart;
};

// The kernel arguments the first loads depend on (prologue sources, O
// partials, the unfused A operand), read together at the top of the kernel
// and pinned in SGPRs (pin_src): each read waiting for the one before costs
// a scalar-cache round trip.
struct ProSrc {
  const float *x;
  int64_t ldx;
  const float *w;
  const int8_t *emb;
  const float *emb_s;
  const int32_t *ids;
  int64_t vocab;
  const float *part;
  int npart;
  int64_t ld_part;
  const int8_t *a;
  int64_t lda;
  const float *as;
  int64_t ldas;
};

template <int PRO, bool PART>
__device__ __forceinline__ ProSrc read_src(const GemvArgs &a) {
  ProSrc p{};
  if constexpr (PRO == PRO_EMBED) {
    p.emb = a.emb;
    p.emb_s = a.emb_s;
    p.ids = a.ids;
    p.vocab = a.vocab;
  } else if constexpr (PRO != PRO_NONE) {
    p.x = a.x;
    p.ldx = a.ldx;
  } else {
    p.a = a.a;
    p.lda = a.lda;
    p.as = a.as;
    p.ldas = a.ldas;
  }
  if constexpr (PRO == PRO_NORM || PRO == PRO_EMBED) p.w = a.w_pre;
  if constexpr (PART) {
    p.part = a.part;
    p.npart = a.npart;
    p.ld_part = a.ld_part;
  }
  return p;
}

template <int PRO, bool PART>
__device__ __forceinline__ void pin_src(ProSrc &p) {
  if constexpr (PRO == PRO_EMBED) {
    p.emb = pin_sgpr(p.emb);
    p.emb_s = pin_sgpr(p.emb_s);
    p.ids = pin_sgpr(p.ids);
    p.vocab = pin_sgpr(p.vocab);
  } else if constexpr (PRO != PRO_NONE) {
    p.x = pin_sgpr(p.x);
    p.ldx = pin_sgpr(p.ldx);
  } else {
    p.a = pin_sgpr(p.a);
    p.lda = pin_sgpr(p.lda);
    p.as = pin_sgpr(p.as);
    p.ldas = pin_sgpr(p.ldas);
  }
  if constexpr (PRO == PRO_NORM || PRO == PRO_EMBED) p.w = pin_sgpr(p.w);
  if constexpr (PART) {
    p.part = pin_sgpr(p.part);
    p.npart = pin_sgpr(p.npart);
    p.ld_part = pin_sgpr(p.ld_part);
  }
}

template <int PRO, int QW, int NP, int NWV = 4>
__device__ __forceinline__ void pro_load_row(const GemvArgs &a, const ProSrc &ps, int m, ProRow<QW, NP> &r) {
  const int lane = threadIdx.x & 63;
  const int wave = NWV == 4 ? wave_id() : (wave_id() & 3);
  const int K = a.K;
  if constexpr (PRO == PRO_EMBED) {
    const int32_t id = ps.ids[m];
    const bool ok = id >= 0 && id < ps.vocab;  // out-of-range ids embed to zero
    r.esc = ok ? ps.emb_s[id] : 0.0f;
#pragma unroll
    for (int q = 0; q < QW; ++q) {
      const int c = (wave + 4 * q) * 256 + 4 * lane;
      r.e[q] = ok ? *reinterpret_cast<const uint32_t *>(ps.emb + static_cast<int64_t>(id) * K + c) : 0u;
    }
  } else {
#pragma unroll
    for (int q = 0; q < QW; ++q) {
      const int c = (wave + 4 * q) * 256 + 4 * lane;
      r.x[q] = *reinterpret_cast<const float4 *>(ps.x + static_cast<int64_t>(m) * ps.ldx + c);
    }
    // the O projection partials (row 0 only; every row of the fixed count is
    // loaded, rows past npart repeat the last one and are not added)
    if constexpr (NP > 0) {
      {
#pragma unroll
        for (int q = 0; q < QW; ++q) {
          const int c = (wave + 4 * q) * 256 + 4 * lane;
#pragma unroll
          for (int h = 0; h < NP; ++h)
            r.p[q][h] = *reinterpret_cast<const float4 *>(ps.part + min(h, ps.npart - 1) * ps.ld_part + c);
        }
        r.npart = ps.npart;
      }
    }
  }
  if constexpr (PRO != PRO_QUANT) {
#pragma unroll
    for (int q = 0; q < QW; ++q)
      r.w[q] = *reinterpret_cast<const float4 *>(ps.w + (wave + 4 * q) * 256 + 4 * lane);
  }
}

// NWV: waves per workgroup (4, or 12 in the fused decode kernel).  The
// barriers wait for LDS only (lds_barrier), not for every outstanding
// vector load as __syncthreads does: the weight rows the kernel issued
// after the row's operands keep arriving while the prologue computes, and
// each wave's own loads are waited for where their registers are used.
// Nothing global that one wave stores here is read by another.
template <int PRO, int QW, int NP, int NWV = 4>
__device__ void pro_compute_row(const GemvArgs &a, int m, const ProRow<QW, NP> &r, int8_t *a_lds,
                                float *as_lds, float *blk, bool stage_writer) {
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int K = a.K;
  constexpr int ngr = 4 * QW;
  const bool act = NWV == 4 || wave < 4;  // the waves that own groups
  const bool write_stage = stage_writer && act;
  float v[QW][4] = {};
  if (act) {
#pragma unroll
  for (int q = 0; q < QW; ++q) {
    const int c = (wave + 4 * q) * 256 + 4 * lane;
    if constexpr (PRO == PRO_EMBED) {
      const uint32_t e = r.e[q];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        v[q][i] = __fmul_rn(static_cast<float>(static_cast<int8_t>(e >> (8 * i))), r.esc);
      if (write_stage && a.x_out)
        *reinterpret_cast<float4 *>(a.x_out + static_cast<int64_t>(m) * a.ldx + c) =
            make_float4(v[q][0], v[q][1], v[q][2], v[q][3]);
    } else {
      v[q][0] = r.x[q].x;
      v[q][1] = r.x[q].y;
      v[q][2] = r.x[q].z;
      v[q][3] = r.x[q].w;
      if constexpr (NP > 0) {
        // residual of the O projection: x + (((0 + p0) + p1) + ...), the
        // partials summed in head order like the group GEMM's groups
        {
          float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int h = 0; h < NP; ++h) {
            if (h < r.npart) {
              o[0] = __fadd_rn(o[0], r.p[q][h].x);
              o[1] = __fadd_rn(o[1], r.p[q][h].y);
              o[2] = __fadd_rn(o[2], r.p[q][h].z);
              o[3] = __fadd_rn(o[3], r.p[q][h].w);
            }
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) v[q][i] = __fadd_rn(v[q][i], o[i]);
        }
      }
    }
  }
  }
  if constexpr (PRO != PRO_QUANT) {
    if (act) {
#pragma unroll
    for (int q = 0; q < QW; ++q) {
      float s = __fadd_rn(__fadd_rn(__fmul_rn(v[q][0], v[q][0]), __fmul_rn(v[q][1], v[q][1])),
                          __fadd_rn(__fmul_rn(v[q][2], v[q][2]), __fmul_rn(v[q][3], v[q][3])));
      s = __fadd_rn(s, lane_xor<1>(s));
      s = __fadd_rn(s, lane_xor<2>(s));
      s = __fadd_rn(s, lane_xor<4>(s));
      if ((lane & 7) == 0) blk[(wave + 4 * q) * 8 + (lane >> 3)] = s;
    }
    }
    lds_barrier();
    if (act) {
    float ss = 0.0f;
#pragma unroll
    for (int b = 0; b < 8 * ngr; ++b) ss = __fadd_rn(ss, blk[b]);
    const float rinv = rms_factor(ss, a.inv_pre);
#pragma unroll
    for (int q = 0; q < QW; ++q) {
      const float w4[4] = {r.w[q].x, r.w[q].y, r.w[q].z, r.w[q].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) v[q][i] = __fmul_rn(__fmul_rn(v[q][i], rinv), w4[i]);
      if (write_stage && a.h_out)
        *reinterpret_cast<float4 *>(a.h_out + static_cast<int64_t>(m) * K + (wave + 4 * q) * 256 + 4 * lane) =
            make_float4(v[q][0], v[q][1], v[q][2], v[q][3]);
    }
    }
  }
  if (act) {
#pragma unroll
  for (int q = 0; q < QW; ++q) {
    const int g = wave + 4 * q;
    const int c = g * 256 + 4 * lane;
    float mx = fmaxf(fmaxf(fabsf(v[q][0]), fabsf(v[q][1])), fmaxf(fabsf(v[q][2]), fabsf(v[q][3])));
    mx = max64(mx);
    const float scale = __fmul_rn(mx, inv127());
    char4 qv;
    qv.x = static_cast<signed char>(quant1(v[q][0], scale));
    qv.y = static_cast<signed char>(quant1(v[q][1], scale));
    qv.z = static_cast<signed char>(quant1(v[q][2], scale));
    qv.w = static_cast<signed char>(quant1(v[q][3], scale));
    *reinterpret_cast<char4 *>(a_lds + m * K + c) = qv;
    if (lane == 0) as_lds[m * ngr + g] = scale;
    if (write_stage) {
      if (a.h8_out) *reinterpret_cast<char4 *>(a.h8_out + static_cast<int64_t>(m) * K + c) = qv;
      if (a.hs_out && lane == 0) a.hs_out[static_cast<int64_t>(m) * ngr + g] = scale;
    }
  }
  }
  lds_barrier();  // blk is reused by the next row; A is complete
}

}  // namespace
}  // namespace q3
