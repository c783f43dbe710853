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
// The value in SGPRs at this point (an empty asm that takes and returns it):
// kernel-argument reads pinned this way are issued together at the top
// instead of one after another where each is first used.
template <class T>
__device__ __forceinline__ T pin_sgpr(T v) {
  asm volatile("" : "+s"(v));
  return v;
}
// Pointers (kernel arguments point to global memory): the address goes
// through the asm as an integer and comes back as a global-address-space
// pointer, so that loads through it stay global loads (a plain pinned
// pointer would lose its address space and become flat loads, which wait
// on both counters).
template <class T>
__device__ __forceinline__ T *pin_sgpr(T *p) {
  uint64_t v = reinterpret_cast<uint64_t>(p);
  asm volatile("" : "+s"(v));
  typedef __attribute__((address_space(1))) T *global_ptr;
  return (T *)(global_ptr)v;
}

__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
}

// Ordered 32-bit key of an f32 (main_big.cpp:314), with -0 folded into +0 so
// that equal values compare equal, as the reference's float `<` does.  With
// (0xFFFFFFFF - column) in the low half, the largest 64-bit key is the
// first column holding the maximum (lm_argmax.h:58-66).
__device__ __forceinline__ uint32_t ordered_key(float v) {
  uint32_t b = __float_as_uint(v);
  if (b == 0x80000000u) b = 0u;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
// the value an ordered key stands for
__device__ __forceinline__ float key_value(uint32_t k) {
  const uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(b);
}

// ---- words handed between workgroups of one launch ----------------------
// Relaxed agent-scope atomics compile to global loads and stores with the
// sc1 cache policy and no cache writeback or invalidate: a store becomes
// visible to loads of that policy on every XCD, with no fence.  A word
// carries its own "stored" mark (a value that cannot be empty), so a reader
// polls it until the mark appears, with every load of a round in flight
// before the check, and gives up after kPollLimit rounds (the launch then
// reports it through a flag; no wait is unbounded).
constexpr int kPollLimit = 1 << 17;  // about 60 ms of round trips

__device__ __forceinline__ unsigned long long xload(const unsigned long long *p) {
  return __hip_atomic_load(const_cast<unsigned long long *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void xstore(unsigned long long *p, unsigned long long v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 16 bytes a lane at p + 16 lane + {0, 1, 2, 3} KB with the cache policy of
// xload (sc1), all four in flight, then a wait for them.  Inline assembly:
// the compiler treats its buffer-load builtins as plain reads and hoists them
// out of a polling loop.
typedef unsigned v4u32 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void xload_4k(const uint32_t *p, v4u32 &a, v4u32 &b, v4u32 &c, v4u32 &d) {
  asm volatile(
      "global_load_dwordx4 %0, %4, off sc1\n\t"
      "global_load_dwordx4 %1, %4, off offset:1024 sc1\n\t"
      "global_load_dwordx4 %2, %4, off offset:2048 sc1\n\t"
      "global_load_dwordx4 %3, %4, off offset:3072 sc1\n\t"
      "s_waitcnt vmcnt(0)"
      : "=&v"(a), "=&v"(b), "=&v"(c), "=&v"(d)
      : "v"(p + 4 * (threadIdx.x & 63))
      : "memory");
}

// ---- LDS staging ------------------------------------------------------
// Generic pointer to an LDS object as the address-space-3 pointer that
// __builtin_amdgcn_global_load_lds takes (through an integer so that the
// host pass of the same source also compiles).
typedef __attribute__((address_space(3))) void *lds_void_ptr;

__device__ __forceinline__ lds_void_ptr to_lds(const void *p) {
  return reinterpret_cast<lds_void_ptr>(reinterpret_cast<uintptr_t>(p));
}

// s_waitcnt vmcnt(N), the other counters untouched (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier for pipelined loops: LDS operations of this wave
// complete (lgkmcnt), then s_barrier.  __syncthreads() would also wait for
// every outstanding vector load (vmcnt(0)), i.e. for the copies of later
// steps that are meant to stay in flight; each wave instead waits for its
// own copies of the current step with wait_vmcnt before this barrier.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ float bits_f32(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t f32_bits(float f) { return __float_as_uint(f); }

#define Q3_EXP2_TAB_VALUES \
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, \
    0x3fef9301d0125b51ull, 0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, \
    0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, 0x3fef06fe0a31b715ull, \
    0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, \
    0x3feea47eb03a5585ull, 0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, \
    0x3feea11473eb0187ull, 0x3feea589994cce13ull, 0x3feeace5422aa0dbull, \
    0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, \
    0x3fef3720dcef9069ull, 0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, \
    0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull

__constant__ static const uint64_t kExp2Tab[32] = {Q3_EXP2_TAB_VALUES};
// The same values as an ordinary constant (not host-writable like a
// __constant__ symbol), so that copies with constant indices fold into
// immediates.
constexpr uint64_t kExp2Vals[32] = {Q3_EXP2_TAB_VALUES};

// One thread writes the table to dst (LDS) from immediates: no load, so
// nothing waits on it (the first reader comes after a barrier).
__device__ __forceinline__ void stage_exp2_table(uint64_t *dst) {
#pragma unroll
  for (int i = 0; i < 32; ++i) dst[i] = kExp2Vals[i];
}

// Special cases of exp2f (|x| >= 128, Inf, NaN) as selects over the result
// of the main path, which is computed for every input: no branch, so
// independent exp chains interleave.  For -150 < x <= -128 (subnormal
// results) the main path's value is kept, as in glibc.
__device__ __forceinline__ float exp2f_special(float x, float y) {
  const uint32_t ux = f32_bits(x);
  const uint32_t abstop = (ux >> 20) & 0x7ffu;
  float sp = y;
  sp = (x <= -150.0f) ? 0.0f : sp;
  sp = (x > 0.0f) ? bits_f32(0x7f800000u) : sp;
  sp = (abstop >= (0x7f800000u >> 20)) ? x + x : sp;
  sp = (ux == 0xff800000u) ? 0.0f : sp;
  return (abstop >= (0x43000000u >> 20)) ? sp : y;
}

// Main path of glibc's exp2f for a table entry read by `tab_at`.
template <class TabAt>
__device__ __forceinline__ float exp2f_glibc_main(float x, TabAt tab_at) {
  const double xd = static_cast<double>(x);
  const double shift = 0x1.8p+52 / 32;
  double kd = __dadd_rn(xd, shift);
  const uint64_t ki = static_cast<uint64_t>(__double_as_longlong(kd));
  kd = __dsub_rn(kd, shift);
  const double r = __dsub_rn(xd, kd);
  uint64_t t = tab_at(static_cast<uint32_t>(ki & 31u));
  t += ki << 47;
  const double s = __longlong_as_double(static_cast<long long>(t));
  const double z = __fma_rn(0x1.c6af84b912394p-5, r, 0x1.ebfce50fac4f3p-3);
  const double r2 = __dmul_rn(r, r);
  double y = __fma_rn(0x1.62e42ff0c52d6p-1, r, 1.0);
  y = __fma_rn(z, r2, y);
  y = __dmul_rn(y, s);
  return __double2float_rn(y);
}

// glibc-compatible exp2f (see the header comment).  For |x| >= 128 the main
// path's table index and exponent are meaningless but harmless (integer and
// f64 arithmetic only); exp2f_special then picks the glibc result.
__device__ __forceinline__ float exp2f_glibc(float x) {
  const float y = exp2f_glibc_main(x, [](uint32_t i) { return kExp2Tab[i]; });
  return exp2f_special(x, y);
}

// ref_qwen3.py:27-29.
__device__ __forceinline__ float exp_f32(float x) {
  return exp2f_glibc(__fmul_rn(x, bits_f32(0x3FB8AA3Bu)));
}

// Same function with the 32-entry table read from `tab` (a copy of kExp2Tab
// staged in LDS by the caller), so a latency-critical loop does not wait on
// a global-memory table lookup per call.
__device__ __forceinline__ float exp2f_glibc_tab(float x, const uint64_t *tab) {
  const float y = exp2f_glibc_main(x, [tab](uint32_t i) { return tab[i]; });
  return exp2f_special(x, y);
}

__device__ __forceinline__ float exp_f32_tab(float x, const uint64_t *tab) {
  return exp2f_glibc_tab(__fmul_rn(x, bits_f32(0x3FB8AA3Bu)), tab);
}

// exp_f32_tab for x <= 0 or x = -inf (softmax arguments s - max): of
// exp2f's special cases only "x2 <= -150 -> +0" can occur (x2 = x*log2(e)
// <= 0; -inf included); -150 < x2 < -128 takes the main path in glibc too.
__device__ __forceinline__ float exp_f32_le0_tab(float x, const uint64_t *tab) {
  const float x2 = __fmul_rn(x, bits_f32(0x3FB8AA3Bu));
  const float y = exp2f_glibc_main(x2, [tab](uint32_t i) { return tab[i]; });
  return (x2 <= -150.0f) ? 0.0f : y;
}

__device__ __forceinline__ float inv127() { return 1.0f / 127.0f; }

// ref_qwen3.py:69-76: one element of aquant with an external scale.
__device__ __forceinline__ int quant1(float x, float scale) {
  const float q = __fdiv_rn(x, scale);
  float r = (q != q) ? 0.0f : rintf(q);
  r = fminf(127.0f, fmaxf(-127.0f, r));
  return static_cast<int>(r);
}

// quant1(x, scale) with y = rcp64(scale) = RN64(1 / scale), one f64 multiply
// per element instead of an f32 division: RN32(x * y) = RN32(x / scale),
// since a quotient of two f32 is never an f32 rounding midpoint and stays at
// least 2^-50 (relative) away from every midpoint, while x * y is within
// 2^-52 of x / scale.  Quotients where the f32 rounding is not the normal
// one (subnormal: rne gives 0 either way; overflow: both saturate) and
// scale = 0 (y = inf: 0 * inf = NaN -> 0, x * inf = +-inf -> +-127) give the
// same int8 as the division.
__device__ __forceinline__ double rcp64(float scale) { return __ddiv_rn(1.0, static_cast<double>(scale)); }
__device__ __forceinline__ int quant_rcp(float x, double y) {
  const float q = __double2float_rn(__dmul_rn(static_cast<double>(x), y));
  float r = (q != q) ? 0.0f : rintf(q);
  r = fminf(127.0f, fmaxf(-127.0f, r));
  return static_cast<int>(r);
}

// ---- lane exchanges in VALU (no LDS round trip) -----------------------
// lane_xor<M>(x): lane i receives x of lane i ^ M.  M = 1, 2: DPP quad_perm;
// M = 4: quad_perm [3,2,1,0] then row_half_mirror (i -> (i ^ 3) ^ 7);
// M = 8: DPP row_ror:8; M = 16, 32: v_permlane16_swap / v_permlane32_swap,
// which return the register with its odd/even 16- (32-) lane halves
// exchanged, split over two results: a lane in an odd half finds its
// partner in the first result, a lane in an even half in the second.
// Every lane gets exactly its partner's value, as with ds_swizzle /
// ds_bpermute, so reductions built on it add the same operands in the same
// order.  The DPP controls used read no lane outside its row, so bound_ctrl
// changes no value; it is set so that the compiler can fold the move into
// the instruction that uses it.
template <int M>
__device__ __forceinline__ uint32_t lane_xor(uint32_t x) {
  const int v = static_cast<int>(x);
  if constexpr (M == 1) {
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(v, 0xB1, 0xf, 0xf, true));
  } else if constexpr (M == 2) {
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(v, 0x4E, 0xf, 0xf, true));
  } else if constexpr (M == 4) {
    const int t = __builtin_amdgcn_mov_dpp(v, 0x1B, 0xf, 0xf, true);
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(t, 0x141, 0xf, 0xf, true));
  } else if constexpr (M == 8) {
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(v, 0x128, 0xf, 0xf, true));
  } else if constexpr (M == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return (__lane_id() & 16) ? r[0] : r[1];
  } else {
    static_assert(M == 32, "lane_xor: M is a power of two below 64");
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return (__lane_id() & 32) ? r[0] : r[1];
  }
}

template <int M>
__device__ __forceinline__ float lane_xor(float x) {
  return __uint_as_float(lane_xor<M>(__float_as_uint(x)));
}

template <int M>
__device__ __forceinline__ int lane_xor(int x) {
  return static_cast<int>(lane_xor<M>(static_cast<uint32_t>(x)));
}

// Same with the distance as a value; every call site sits in a fully
// unrolled loop, so m is a constant there and one case remains.
__device__ __forceinline__ uint32_t lane_xor_m(uint32_t x, int m) {
  switch (m) {
    case 1: return lane_xor<1>(x);
    case 2: return lane_xor<2>(x);
    case 4: return lane_xor<4>(x);
    case 8: return lane_xor<8>(x);
    case 16: return lane_xor<16>(x);
    case 32: return lane_xor<32>(x);
    default: return static_cast<uint32_t>(__shfl_xor(static_cast<int>(x), m));
  }
}

__device__ __forceinline__ unsigned long long lane_xor_u64(unsigned long long v, int m) {
  const uint32_t lo = lane_xor_m(static_cast<uint32_t>(v), m);
  const uint32_t hi = lane_xor_m(static_cast<uint32_t>(v >> 32), m);
  return (static_cast<unsigned long long>(hi) << 32) | lo;
}

// {x_i, x_(i^16)} (resp. i^32) at every lane i, in an order that depends on
// the lane: for a commutative combine (f32 add, max, integer add) the result
// equals combine(x, lane_xor<16>(x)) bit for bit, without the select.
struct LanePair {
  uint32_t a, b;
};

__device__ __forceinline__ LanePair lane_pair16(uint32_t x) {
  const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  return {r[0], r[1]};
}

__device__ __forceinline__ LanePair lane_pair32(uint32_t x) {
  const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return {r[0], r[1]};
}

// Value of lane L (a constant) in every lane.
template <int L>
__device__ __forceinline__ float lane_bcast(float x) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), L));
}

// Value of lane l (wave-uniform, a runtime value) in every lane.
__device__ __forceinline__ float lane_read(float x, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
}

// ---- wave reductions --------------------------------------------------
// Pairwise tree over 32 consecutive lanes: level k adds lanes i and i^2^k.
// For 32 leaves this is exactly ref_qwen3.py:41-50's tree (pairs (0,1),
// (2,3), ...); for n < 32 leaves padded with +0.0 it equals the reference's
// carry-the-odd-element tree because a carried node only ever meets +0.0.
__device__ __forceinline__ float tree_sum32(float v) {
  v = __fadd_rn(v, lane_xor<1>(v));
  v = __fadd_rn(v, lane_xor<2>(v));
  v = __fadd_rn(v, lane_xor<4>(v));
  v = __fadd_rn(v, lane_xor<8>(v));
  const LanePair p = lane_pair16(__float_as_uint(v));
  return __fadd_rn(__uint_as_float(p.a), __uint_as_float(p.b));
}

// max is exact in any order (NaN-free inputs).
__device__ __forceinline__ float max32(float v) {
  v = fmaxf(v, lane_xor<1>(v));
  v = fmaxf(v, lane_xor<2>(v));
  v = fmaxf(v, lane_xor<4>(v));
  v = fmaxf(v, lane_xor<8>(v));
  const LanePair p = lane_pair16(__float_as_uint(v));
  return fmaxf(__uint_as_float(p.a), __uint_as_float(p.b));
}

__device__ __forceinline__ float max64(float v) {
  v = max32(v);
  const LanePair p = lane_pair32(__float_as_uint(v));
  return fmaxf(__uint_as_float(p.a), __uint_as_float(p.b));
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
  ss = __fadd_rn(ss, lane_bcast<0>(sa));
  ss = __fadd_rn(ss, lane_bcast<32>(sa));
  ss = __fadd_rn(ss, lane_bcast<0>(sb));
  ss = __fadd_rn(ss, lane_bcast<32>(sb));
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
