// Device helpers shared by the GEMM kernels' epilogues: SwiGLU with the
// staged exp2 table, the destination of an int8 head row (dense rows or a
// paged K/V slot), and a compile-time loop.
#pragma once

#include <type_traits>
#include <utility>

#include "q3_device.h"
#include "q3_kernels.h"

namespace q3 {

// ref_qwen3.py:194-200: e = exp(-g); e = e + 1; e = 1/e; out = (g * e) * u
// (exp table staged in LDS by stage_exp2_table).
__device__ __forceinline__ float swiglu_tab(float g, float u, const uint64_t *tab) {
  float e = __fmul_rn(g, -1.0f);
  e = exp_f32_tab(e, tab);
  e = __fadd_rn(e, 1.0f);
  e = __fdiv_rn(1.0f, e);
  return __fmul_rn(__fmul_rn(g, e), u);
}

// Slot pointers of token position t in page `page` of a paged K/V pool,
// head `head`.
__device__ __forceinline__ void qdest_slot(const QDest &d, uint32_t page, uint32_t t, int head, int8_t **row8,
                                           float **scale) {
  const uint32_t slot = t % d.page_tokens;
  *row8 = d.q8 + page * d.page_bytes + slot * d.row_bytes + head * 128;
  *scale = reinterpret_cast<float *>(reinterpret_cast<int8_t *>(d.qs) + page * d.scale_page_bytes +
                                     slot * d.scale_row_bytes) + head;
}

// Row destination of the int8 head output of row m, head `head`: a dense
// [rows][heads * 128] view, or the page slot of token pos0 + m (or
// row_pos[m] through that row's own table) of a paged K/V pool.
__device__ __forceinline__ void qdest_row(const QDest &d, int m, int head, int8_t **row8, float **scale) {
  if (d.table || d.row_pos) {
    uint32_t t = d.pos0 + static_cast<uint32_t>(m);
    if (d.pos_dev) t += static_cast<uint32_t>(*d.pos_dev);
    const uint16_t *table = d.table;
    if (d.row_pos) {
      t = static_cast<uint32_t>(d.row_pos[m]);
      table = d.row_tables + m * d.ld_table;
    }
    qdest_slot(d, table[t / d.page_tokens], t, head, row8, scale);
  } else {
    *row8 = d.q8 + static_cast<int64_t>(m) * d.ldq8 + head * 128;
    *scale = d.qs + static_cast<int64_t>(m) * d.ldqs + head * d.qs_col;
  }
}

// f(std::integral_constant<int, 0>{}), ..., f(std::integral_constant<int, N - 1>{})
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

}  // namespace q3
