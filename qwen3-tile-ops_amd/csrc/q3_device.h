// Device-side numeric primitives shared by every kernel (gfx950, wave64).
//
// The arithmetic contract is tools/ref_qwen3.py:17-97: every f32 operation
// is a single IEEE round-to-nearest-even operation (this file is compiled
// with -ffp-contract=off, so no expression below fuses into an FMA), and
//   exp(x)   = exp2f(RN(x * 0x3FB8AA3B))            (ref_qwen3.py:27-29)
//   rcp(x)   = 1 / x, rsqrt(x) = 1 / sqrt(x)         (ref_qwen3.py:32-38)
//   quant(x) = sat127(rne(x / scale)), NaN -> 0      (ref_qwen3.py:69-76)
//   scale    = absmax * RN(1/127)                    (ref_qwen3.py:79-97)
//
// exp2f reproduces glibc's exp2f (the function numpy's float32 exp2 reduces
// to when its AVX512 dispatch is disabled) from the published algorithm of
// ARM optimized-routines exp2f, which glibc adopted in 2.28: x = k/32 + r,
// 2^(k/32) from a 32-entry table (the table entries are the doubles nearest
// 2^(i/32), stored minus i<<47 so the exponent can be added as an integer),
// and 2^r from a degree-3 polynomial in double precision.  The same
// algorithm in the CPU oracle is compared against glibc exp2f on every
// float in [-151, 129].
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q3 {

constexpr int kWave = 64;

// Index of the calling wave within its workgroup as a wave-uniform (scalar)
// value.  The compiler cannot prove threadIdx.x / 64 uniform by itself; it
// would then keep per-lane copies of anything selected by the wave index
// (argument pointers included) instead of scalar registers.
__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
}

__device__ __forceinline__ float bits_f32(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t f32_bits(float f) { return __float_as_uint(f); }

__constant__ static const uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full,
    0x3fef9301d0125b51ull, 0x3fef72b83c7d517bull, 0x3fef54873168b9aaull,
    0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, 0x3fef06fe0a31b715ull,
    0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull,
    0x3feea47eb03a5585ull, 0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull,
    0x3feea11473eb0187ull, 0x3feea589994cce13ull, 0x3feeace5422aa0dbull,
    0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull,
    0x3fef3720dcef9069ull, 0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full,
    0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

// glibc-compatible exp2f (see the header comment).
__device__ __forceinline__ float exp2f_glibc(float x) {
  const uint32_t ux = f32_bits(x);
  const uint32_t abstop = (ux >> 20) & 0x7ffu;
  if (abstop >= (0x43000000u >> 20)) {  // |x| >= 128, Inf or NaN
    if (ux == 0xff800000u) return 0.0f;
    if (abstop >= (0x7f800000u >> 20)) return x + x;
    if (x > 0.0f) return bits_f32(0x7f800000u);
    if (x <= -150.0f) return 0.0f;
  }
  const double xd = static_cast<double>(x);
  const double shift = 0x1.8p+52 / 32;
  double kd = __dadd_rn(xd, shift);
  const uint64_t ki = static_cast<uint64_t>(__double_as_longlong(kd));
  kd = __dsub_rn(kd, shift);
  const double r = __dsub_rn(xd, kd);
  uint64_t t = kExp2Tab[ki & 31u];
  t += ki << 47;
  const double s = __longlong_as_double(static_cast<long long>(t));
  const double z = __fma_rn(0x1.c6af84b912394p-5, r, 0x1.ebfce50fac4f3p-3);
  const double r2 = __dmul_rn(r, r);
  double y = __fma_rn(0x1.62e42ff0c52d6p-1, r, 1.0);
  y = __fma_rn(z, r2, y);
  y = __dmul_rn(y, s);
  return __double2float_rn(y);
}

// ref_qwen3.py:27-29.
__device__ __forceinline__ float exp_f32(float x) {
  return exp2f_glibc(__fmul_rn(x, bits_f32(0x3FB8AA3Bu)));
}

// Same function with the 32-entry table read from `tab` (a copy of kExp2Tab
// staged in LDS by the caller), so a latency-critical loop does not wait on
// a global-memory table lookup per call.
__device__ __forceinline__ float exp2f_glibc_tab(float x, const uint64_t *tab) {
  const uint32_t ux = f32_bits(x);
  const uint32_t abstop = (ux >> 20) & 0x7ffu;
  if (abstop >= (0x43000000u >> 20)) {
    if (ux == 0xff800000u) return 0.0f;
    if (abstop >= (0x7f800000u >> 20)) return x + x;
    if (x > 0.0f) return bits_f32(0x7f800000u);
    if (x <= -150.0f) return 0.0f;
  }
  const double xd = static_cast<double>(x);
  const double shift = 0x1.8p+52 / 32;
  double kd = __dadd_rn(xd, shift);
  const uint64_t ki = static_cast<uint64_t>(__double_as_longlong(kd));
  kd = __dsub_rn(kd, shift);
  const double r = __dsub_rn(xd, kd);
  uint64_t t = tab[ki & 31u];
  t += ki << 47;
  const double s = __longlong_as_double(static_cast<long long>(t));
  const double z = __fma_rn(0x1.c6af84b912394p-5, r, 0x1.ebfce50fac4f3p-3);
  const double r2 = __dmul_rn(r, r);
  double y = __fma_rn(0x1.62e42ff0c52d6p-1, r, 1.0);
  y = __fma_rn(z, r2, y);
  y = __dmul_rn(y, s);
  return __double2float_rn(y);
}

__device__ __forceinline__ float exp_f32_tab(float x, const uint64_t *tab) {
  return exp2f_glibc_tab(__fmul_rn(x, bits_f32(0x3FB8AA3Bu)), tab);
}

__device__ __forceinline__ float inv127() { return 1.0f / 127.0f; }

// ref_qwen3.py:69-76: one element of aquant with an external scale.
__device__ __forceinline__ int quant1(float x, float scale) {
  const float q = __fdiv_rn(x, scale);
  float r = (q != q) ? 0.0f : rintf(q);
  r = fminf(127.0f, fmaxf(-127.0f, r));
  return static_cast<int>(r);
}

// ---- wave reductions --------------------------------------------------
// Pairwise tree over 32 consecutive lanes: level k adds lanes i and i^2^k.
// For 32 leaves this is exactly ref_qwen3.py:41-50's tree (pairs (0,1),
// (2,3), ...); for n < 32 leaves padded with +0.0 it equals the reference's
// carry-the-odd-element tree because a carried node only ever meets +0.0.
__device__ __forceinline__ float tree_sum32(float v) {
  v = __fadd_rn(v, __shfl_xor(v, 1));
  v = __fadd_rn(v, __shfl_xor(v, 2));
  v = __fadd_rn(v, __shfl_xor(v, 4));
  v = __fadd_rn(v, __shfl_xor(v, 8));
  v = __fadd_rn(v, __shfl_xor(v, 16));
  return v;
}

// max is exact in any order (NaN-free inputs).
__device__ __forceinline__ float max32(float v) {
  v = fmaxf(v, __shfl_xor(v, 1));
  v = fmaxf(v, __shfl_xor(v, 2));
  v = fmaxf(v, __shfl_xor(v, 4));
  v = fmaxf(v, __shfl_xor(v, 8));
  v = fmaxf(v, __shfl_xor(v, 16));
  return v;
}

__device__ __forceinline__ float max64(float v) {
  v = max32(v);
  return fmaxf(v, __shfl_xor(v, 32));
}

// RMSNorm factor from the ordered 32-column block sums (ref_qwen3.py:161-170):
// ss = (((0 + b0) + b1) + ...) * inv + eps, then 1 / sqrt(ss).
// sqrt here must be the correctly rounded one: __builtin_sqrtf lowers to
// v_sqrt_f32 plus an FMA residual correction, whereas HIP's __fsqrt_rn is
// the bare approximate v_sqrt_f32 unless OCML_BASIC_ROUNDED_OPERATIONS is
// defined.
__device__ __forceinline__ float sqrt_rn(float x) { return __builtin_sqrtf(x); }

__device__ __forceinline__ float rms_factor(float ss, float inv) {
  ss = __fmul_rn(ss, inv);
  ss = __fadd_rn(ss, 1e-6f);
  return __fdiv_rn(1.0f, sqrt_rn(ss));
}

// One 128-wide head row held by a wave as t0 = x[lane], t1 = x[lane + 64]:
// per-head RMSNorm (kernels/norm_rope_quant.h:27-40, ref_qwen3.py:396/401)
// followed by rotate-half RoPE (norm_rope_quant.h:42-65,
// ref_qwen3.py:180-191).  Block sums: lanes 0-31 of t0 are columns 0-31,
// lanes 32-63 columns 32-63, t1 likewise for 64-127, added in column order.
// Operands in registers: gains w0 = nw[lane], w1 = nw[lane + 64], and the
// RoPE row's c = cos[lane], s = sin[lane].
__device__ __forceinline__ void head_norm_rope_regs(float &t0, float &t1, float w0, float w1,
                                                    float c, float s, float inv_hd, bool do_rope) {
  const float sa = tree_sum32(__fmul_rn(t0, t0));
  const float sb = tree_sum32(__fmul_rn(t1, t1));
  float ss = 0.0f;
  ss = __fadd_rn(ss, __shfl(sa, 0));
  ss = __fadd_rn(ss, __shfl(sa, 32));
  ss = __fadd_rn(ss, __shfl(sb, 0));
  ss = __fadd_rn(ss, __shfl(sb, 32));
  const float rinv = rms_factor(ss, inv_hd);
  const float y0 = __fmul_rn(__fmul_rn(t0, rinv), w0);
  const float y1 = __fmul_rn(__fmul_rn(t1, rinv), w1);
  if (do_rope) {
    t0 = __fsub_rn(__fmul_rn(y0, c), __fmul_rn(y1, s));
    t1 = __fadd_rn(__fmul_rn(y0, s), __fmul_rn(y1, c));
  } else {
    t0 = y0;
    t1 = y1;
  }
}

__device__ __forceinline__ void head_norm_rope(float &t0, float &t1, int lane,
                                               const float *nw, int64_t nw_stride,
                                               const float *cos_row, const float *sin_row,
                                               float inv_hd, bool do_rope) {
  const float w0 = nw[static_cast<int64_t>(lane) * nw_stride];
  const float w1 = nw[static_cast<int64_t>(lane + 64) * nw_stride];
  const float c = do_rope ? cos_row[lane] : 0.0f;
  const float s = do_rope ? sin_row[lane] : 0.0f;
  head_norm_rope_regs(t0, t1, w0, w1, c, s, inv_hd, do_rope);
}

}  // namespace q3
