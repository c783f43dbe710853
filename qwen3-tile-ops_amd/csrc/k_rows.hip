// Row kernels: embedding gather + dequant, RMSNorm, per-group int8 quant.
//
//   mode 2  kernels/embedding.h:99-168 embedding_rmsnorm_rows
//           (ref_qwen3.py:292-296): x = f32(emb8[id]) * emb_s[id]
//   mode 1  kernels/rmsnorm.h:34-81 rmsnorm_rows (ref_qwen3.py:161-177)
//   quant   kernels/quant.h:89-138 quant_rows_heads (ref_qwen3.py:86-97),
//           fused behind modes 1/2 or alone (mode 0)
//
// One wave64 per row.  Columns are visited 64 at a time: lanes 0-31 hold
// 32-column block 2i and lanes 32-63 block 2i+1, so the per-block tree sum
// is a 5-level butterfly inside each half-wave and the block sums are then
// added strictly in column order, exactly like the reference's
// `ss = ss + tree_sum(block**2)` loop.  The row is re-read (L1/L2 resident)
// instead of held in registers so any width works.
#include "q3_device.h"
#include "q3_kernels.h"

namespace q3 {
namespace {

__device__ __forceinline__ float load_x(const RowArgs &a, int row, int c,
                                        int32_t id) {
  if (a.mode == 2) {
    if (id < 0 || id >= a.table_rows) return 0.0f;
    const float e = static_cast<float>(a.table[static_cast<int64_t>(id) * a.ldt + c]);
    return __fmul_rn(e, a.tscale[static_cast<int64_t>(id) * a.tss]);
  }
  return a.x[static_cast<int64_t>(row) * a.ldx + c];
}

__global__ void __launch_bounds__(256) rows_kernel(RowArgs a) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  int32_t id = 0;
  if (a.mode == 2) {
    int64_t base = 0;
    if (a.ids_base_pos) base = *a.ids_base_pos;
    id = a.ids[(base + row) * a.ids_stride];
  }
  const int cols = a.cols;

  float rinv = 1.0f;
  if (a.mode != 0) {
    // pass 1: ordered block sums of squares (and the embedding write-out)
    float ss = 0.0f;
    const int nblk = (cols + 31) / 32;
    for (int c0 = 0; c0 < cols; c0 += 64) {
      const int c = c0 + lane;
      float v = 0.0f;
      if (c < cols) {
        v = load_x(a, row, c, id);
        if (a.mode == 2 && a.x_out) a.x_out[static_cast<int64_t>(row) * a.ldxo + c] = v;
      }
      const float bsum = tree_sum32(__fmul_rn(v, v));
      const float b_lo = lane_bcast<0>(bsum);
      const float b_hi = lane_bcast<32>(bsum);
      ss = __fadd_rn(ss, b_lo);
      if ((c0 >> 5) + 1 < nblk) ss = __fadd_rn(ss, b_hi);
    }
    rinv = rms_factor(ss, a.inv);
    // pass 2: h = (x * rinv) * w
    if (a.h) {
      for (int c = lane; c < cols; c += 64) {
        const float v = load_x(a, row, c, id);
        const float y = __fmul_rn(__fmul_rn(v, rinv), a.w[static_cast<int64_t>(c) * a.w_stride]);
        a.h[static_cast<int64_t>(row) * a.ldh + c] = y;
      }
    }
  }
  if (!a.h8) return;
  // per-group quantisation of y (= x in mode 0)
  const int G = a.group;
  for (int g0 = 0, gi = 0; g0 < cols; g0 += G, ++gi) {
    const int g1 = min(cols, g0 + G);
    float m = 0.0f;
    for (int c = g0 + lane; c < g1; c += 64) {
      float y = load_x(a, row, c, id);
      if (a.mode != 0)
        y = __fmul_rn(__fmul_rn(y, rinv), a.w[static_cast<int64_t>(c) * a.w_stride]);
      m = fmaxf(m, fabsf(y));
    }
    m = max64(m);
    const float scale = __fmul_rn(m, inv127());
    if (lane == 0) a.hs[static_cast<int64_t>(row) * a.ldhs + gi] = scale;
    for (int c = g0 + lane; c < g1; c += 64) {
      float y = load_x(a, row, c, id);
      if (a.mode != 0)
        y = __fmul_rn(__fmul_rn(y, rinv), a.w[static_cast<int64_t>(c) * a.w_stride]);
      a.h8[static_cast<int64_t>(row) * a.ldh8 + c] = static_cast<int8_t>(quant1(y, scale));
    }
  }
}

// kernels/norm_rope_quant.h:88-111 norm_rope_quant_heads: one wave per
// (row, head) of an f32 [rows][heads*128] input.
__global__ void __launch_bounds__(256) nrq_rows_kernel(NrqArgs a) {
  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= a.rows * a.heads) return;
  const int row = item / a.heads, head = item % a.heads;
  const float *xr = a.x + static_cast<int64_t>(row) * a.ldx + head * 128;
  float t0 = xr[lane], t1 = xr[lane + 64];
  head_norm_rope(t0, t1, lane, a.nw, a.nw_stride, a.cos_t + static_cast<int64_t>(row) * a.ld_cs,
                 a.sin_t + static_cast<int64_t>(row) * a.ld_cs, a.inv_hd, a.do_rope != 0);
  const float mx = max64(fmaxf(fabsf(t0), fabsf(t1)));
  const float scale = __fmul_rn(mx, inv127());
  int8_t *q = a.q8 + static_cast<int64_t>(row) * a.ldq8 + head * 128;
  q[lane] = static_cast<int8_t>(quant1(t0, scale));
  q[lane + 64] = static_cast<int8_t>(quant1(t1, scale));
  if (lane == 0) a.qs[static_cast<int64_t>(row) * a.ldqs + head * a.qs_col] = scale;
}

// Register-resident variant for 1024-wide rows with 256-column groups (the
// model's hidden size): one 256-thread workgroup per row, thread t owns
// columns 4t..4t+3.  The 32-column block tree is: pairs inside the thread,
// then xor-1/2/4 butterflies over the block's 8 threads (the reference's
// adjacent-pair tree, level by level); the 32 block sums are then added in
// column order by every thread from LDS.  A 256-column quant group is
// exactly one wave.
__global__ void __launch_bounds__(256) rows1024_kernel(RowArgs a) {
  __shared__ float bsum[32];
  const int row = blockIdx.x;
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int c0 = 4 * t;
  // the gains do not depend on the row: issued first, their latency overlaps
  // the row's load and the sum of squares
  float w[4];
  if (a.mode != 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = a.w[static_cast<int64_t>(c0 + i) * a.w_stride];
  }
  float v[4];
  if (a.mode == 2) {
    int64_t base = 0;
    if (a.ids_base_pos) base = *a.ids_base_pos;
    const int32_t id = a.ids[(base + row) * a.ids_stride];
    if (id >= 0 && id < a.table_rows) {
      const char4 e = *reinterpret_cast<const char4 *>(a.table + static_cast<int64_t>(id) * a.ldt + c0);
      const float sc = a.tscale[static_cast<int64_t>(id) * a.tss];
      v[0] = __fmul_rn(static_cast<float>(e.x), sc);
      v[1] = __fmul_rn(static_cast<float>(e.y), sc);
      v[2] = __fmul_rn(static_cast<float>(e.z), sc);
      v[3] = __fmul_rn(static_cast<float>(e.w), sc);
    } else {
      v[0] = v[1] = v[2] = v[3] = 0.0f;
    }
    if (a.x_out)
      *reinterpret_cast<float4 *>(a.x_out + static_cast<int64_t>(row) * a.ldxo + c0) =
          make_float4(v[0], v[1], v[2], v[3]);
  } else {
    const float4 x = *reinterpret_cast<const float4 *>(a.x + static_cast<int64_t>(row) * a.ldx + c0);
    v[0] = x.x;
    v[1] = x.y;
    v[2] = x.z;
    v[3] = x.w;
  }
  if (a.mode != 0) {
    float s = __fadd_rn(__fadd_rn(__fmul_rn(v[0], v[0]), __fmul_rn(v[1], v[1])),
                        __fadd_rn(__fmul_rn(v[2], v[2]), __fmul_rn(v[3], v[3])));
    s = __fadd_rn(s, lane_xor<1>(s));
    s = __fadd_rn(s, lane_xor<2>(s));
    s = __fadd_rn(s, lane_xor<4>(s));
    if ((t & 7) == 0) bsum[t >> 3] = s;
    __syncthreads();
    float ss = 0.0f;
#pragma unroll
    for (int b = 0; b < 32; ++b) ss = __fadd_rn(ss, bsum[b]);
    const float rinv = rms_factor(ss, a.inv);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      v[i] = __fmul_rn(__fmul_rn(v[i], rinv), w[i]);
    if (a.h)
      *reinterpret_cast<float4 *>(a.h + static_cast<int64_t>(row) * a.ldh + c0) =
          make_float4(v[0], v[1], v[2], v[3]);
  }
  if (!a.h8) return;
  float m = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  m = max64(m);
  const float scale = __fmul_rn(m, inv127());
  const double y = rcp64(scale);
  char4 q;
  q.x = static_cast<signed char>(quant_rcp(v[0], y));
  q.y = static_cast<signed char>(quant_rcp(v[1], y));
  q.z = static_cast<signed char>(quant_rcp(v[2], y));
  q.w = static_cast<signed char>(quant_rcp(v[3], y));
  *reinterpret_cast<char4 *>(a.h8 + static_cast<int64_t>(row) * a.ldh8 + c0) = q;
  if (lane == 0) a.hs[static_cast<int64_t>(row) * a.ldhs + (t >> 6)] = scale;
}

// Quantisation alone (mode 0) of rows whose width is a multiple of 256 with
// 256-column groups: one wave per (row, group), lane l owns columns 4l..4l+3
// of the group (the arithmetic of rows1024_kernel's quantisation).
__global__ void __launch_bounds__(256) quant_groups_kernel(RowArgs a, int ngroups) {
  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= a.rows * ngroups) return;
  const int row = item / ngroups, g = item % ngroups;
  const int c0 = 256 * g + 4 * lane;
  const float4 x = *reinterpret_cast<const float4 *>(a.x + static_cast<int64_t>(row) * a.ldx + c0);
  float m = fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w)));
  m = max64(m);
  const float scale = __fmul_rn(m, inv127());
  const double y = rcp64(scale);
  char4 q;
  q.x = static_cast<signed char>(quant_rcp(x.x, y));
  q.y = static_cast<signed char>(quant_rcp(x.y, y));
  q.z = static_cast<signed char>(quant_rcp(x.z, y));
  q.w = static_cast<signed char>(quant_rcp(x.w, y));
  *reinterpret_cast<char4 *>(a.h8 + static_cast<int64_t>(row) * a.ldh8 + c0) = q;
  if (lane == 0) a.hs[static_cast<int64_t>(row) * a.ldhs + g] = scale;
}

bool quant_groups_ok(const RowArgs &a) {
  auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  return a.mode == 0 && a.h8 && a.group == 256 && a.cols % 256 == 0 && (a.ldx & 3) == 0 && al16(a.x) &&
         (a.ldh8 & 3) == 0 && (reinterpret_cast<uintptr_t>(a.h8) & 3) == 0;
}

bool rows1024_ok(const RowArgs &a) {
  auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (a.cols != 1024) return false;
  if (a.h8 && (a.group != 256 || (a.ldh8 & 3) || !al16(a.h8))) return false;
  if (a.mode == 2) {
    if ((a.ldt & 3) || (reinterpret_cast<uintptr_t>(a.table) & 3)) return false;
    if (a.x_out && ((a.ldxo & 3) || !al16(a.x_out))) return false;
  } else if ((a.ldx & 3) || !al16(a.x)) {
    return false;
  }
  if (a.h && ((a.ldh & 3) || !al16(a.h))) return false;
  return true;
}

}  // namespace

hipError_t launch_nrq_rows(const NrqArgs &a, hipStream_t s) {
  const int items = a.rows * a.heads;
  if (items <= 0) return hipSuccess;
  hipLaunchKernelGGL(nrq_rows_kernel, dim3((items + 3) / 4), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_rows(const RowArgs &a, hipStream_t s) {
  if (a.rows <= 0) return hipSuccess;
  if (quant_groups_ok(a)) {
    const int ngroups = a.cols / 256;
    const int64_t items = static_cast<int64_t>(a.rows) * ngroups;
    hipLaunchKernelGGL(quant_groups_kernel, dim3(static_cast<unsigned>((items + 3) / 4)), dim3(256), 0, s, a,
                       ngroups);
    return hipGetLastError();
  }
  if (rows1024_ok(a)) {
    hipLaunchKernelGGL(rows1024_kernel, dim3(a.rows), dim3(256), 0, s, a);
    return hipGetLastError();
  }
  const dim3 grid((a.rows + 3) / 4);
  hipLaunchKernelGGL(rows_kernel, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace q3
