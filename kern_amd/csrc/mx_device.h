// Device-side element codecs and helpers shared by the gfx950 kernels.
//
// The arithmetic here is integer-exact and matches the CPU oracle bit for bit:
//   * e2m1: sign = bit 3, magnitude table {0, .5, 1, 1.5, 2, 3, 4, 6}   (tools/trtllm-bmm/probe.py:24-31)
//   * e8m0: 2^(c-127), 255 = NaN                                         (crates/kern-manifest/src/values.rs:18-24)
//   * e4m3fn: round-to-nearest-even, saturating to +-448, NaN -> 0x7f|sign
//   * MXFP8 block scale: clamp(floor(log2 amax) - 8 + 127, 0, 254)       (probe.py:38-43 floor rule)
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));

#define KERN_DEV static __device__ __forceinline__

// A wave's LDS writes made visible to its own lanes' later LDS reads of other lanes' data (a wave writes a
// region of its own and reads it back in another lane order). LDS instructions of one wave execute in
// order, so this costs no instruction; it states the cross-lane dependence to the compiler (a wavefront-
// scope release/acquire pair around a wave barrier), which may otherwise treat the accesses as unordered.
#define WAVE_LDS_SYNC()                                 \
  do {                                                  \
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront"); \
    __builtin_amdgcn_wave_barrier();                    \
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront"); \
  } while (0)

KERN_DEV float bf16_bits_to_f32(uint32_t b16) { return __uint_as_float(b16 << 16); }

// round-to-nearest-even f32 -> bf16 bits (NaN stays a quiet NaN)
KERN_DEV uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// bf16 bits of a (low half) and b (high half), round to nearest even, through V_CVT_PK_BF16_F32: the same
// bits as f32_to_bf16_bits for every input (NaN comes back quiet with the sign and top payload bits)
KERN_DEV uint32_t bf16x2_hw(float a, float b) {
  const v2f v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, v2bf));
}

// MXFP8 scale code for a block whose largest |bits| is amax: floor(log2 amax) - 8 + 127 clamped to [0, 254] for
// a finite amax, 255 for a non-finite one (amax_bits >= 0x7f800000). A normal amax has floor(log2) = E - 127 for
// its exponent field E <= 254, so the code is E - 8; a subnormal or zero amax (E = 0) gives a negative code,
// clamped to 0, like E <= 8. (The two forms agree on all 2^31 values of |bits|: an exhaustive host check.)
KERN_DEV uint32_t mx_scale_code(uint32_t amax_bits) {
  const uint32_t E = amax_bits >> 23;
  return E >= 255u ? 255u : (E > 8u ? E - 8u : 0u);
}

// two e4m3fn codes (low byte = a) of f32 values through the hardware converter: RNE, saturating to +-448
// by clamping first, NaN -> 0x7f|sign. Each code is bit-identical to an integer round-to-nearest-even
// encoder of the value (the CPU oracle's), checked on gfx950 over all bf16 values at shifts -20..126.
KERN_DEV uint32_t e4m3_hw2(float a, float b) {
  const float ca = __builtin_fminf(__builtin_fmaxf(a, -448.0f), 448.0f);
  const float cb = __builtin_fminf(__builtin_fmaxf(b, -448.0f), 448.0f);
  uint32_t r = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(ca, cb, 0, false) & 0xffffu;
  if (__builtin_isnan(a)) r = (r & 0xff00u) | ((__float_as_uint(a) >> 24) & 0x80u) | 0x7fu;
  if (__builtin_isnan(b)) r = (r & 0x00ffu) | ((((__float_as_uint(b) >> 24) & 0x80u) | 0x7fu) << 8);
  return r;
}

// four MXFP8 element codes of the bf16 pairs in dwords w0, w1 (low half first) under block scale code
// sc: e4m3(x * 2^(127 - sc)), or 0x7f|sign for a non-finite block (sc == 255). The power-of-two
// scaling is exact (ldexp) for every element that does not round to zero.
KERN_DEV uint32_t mx_pack4(uint32_t w0, uint32_t w1, uint32_t sc) {
  if (sc == 255u) {
    return (((w0 >> 8) & 0x80u) | 0x7fu) | ((((w0 >> 24) & 0x80u) | 0x7fu) << 8) |
           ((((w1 >> 8) & 0x80u) | 0x7fu) << 16) | ((((w1 >> 24) & 0x80u) | 0x7fu) << 24);
  }
  const int sh = 127 - (int)sc;
  const float a = __builtin_ldexpf(__uint_as_float(w0 << 16), sh);
  const float b = __builtin_ldexpf(__uint_as_float(w0 & 0xffff0000u), sh);
  const float c = __builtin_ldexpf(__uint_as_float(w1 << 16), sh);
  const float d = __builtin_ldexpf(__uint_as_float(w1 & 0xffff0000u), sh);
  int r = __builtin_amdgcn_cvt_pk_fp8_f32(__builtin_fminf(__builtin_fmaxf(a, -448.0f), 448.0f),
                                          __builtin_fminf(__builtin_fmaxf(b, -448.0f), 448.0f), 0, false);
  r = __builtin_amdgcn_cvt_pk_fp8_f32(__builtin_fminf(__builtin_fmaxf(c, -448.0f), 448.0f),
                                      __builtin_fminf(__builtin_fmaxf(d, -448.0f), 448.0f), r, true);
  return (uint32_t)r;
}

// two MXFP8 element codes (low byte = a) of f32 values in a block with scale code sc: e4m3(v * 2^(127-sc))
// through the hardware converter, or 0x7f|sign when the block is non-finite (sc == 255)
KERN_DEV uint32_t mx_code2(float a, float b, uint32_t sc) {
  if (sc == 255u)
    return (((__float_as_uint(a) >> 24) & 0x80u) | 0x7fu) | ((((__float_as_uint(b) >> 24) & 0x80u) | 0x7fu) << 8);
  const int sh = 127 - (int)sc;
  return e4m3_hw2(__builtin_ldexpf(a, sh), __builtin_ldexpf(b, sh));
}

// max of v over lanes l, l ^ 16, l ^ 32 and l ^ 48 (the four 16-lane rows of the wave), by the two
// row-swapping moves (V_PERMLANE32_SWAP, V_PERMLANE16_SWAP): no LDS round trip
KERN_DEV uint32_t max_over_rows(uint32_t v) {
  const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  v = max((uint32_t)p[0], (uint32_t)p[1]);
  const auto q = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return max((uint32_t)q[0], (uint32_t)q[1]);
}

// mx_code2 of the four pairs of one lane's share of a block, with one test of the block's scale code: every
// element of a block with sc < 255 is finite (the largest |bits| is below 0x7f800000), so the conversions
// need no NaN handling; a non-finite block (sc == 255) gets 0x7f|sign for every element. Same codes as
// mx_code2 pair by pair.
KERN_DEV void mx_code2x4(const float (&h)[4][2], uint32_t sc, uint32_t (&o)[4]) {
  const int sh = 127 - (int)sc;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float a = __builtin_fminf(__builtin_fmaxf(__builtin_ldexpf(h[r][0], sh), -448.0f), 448.0f);
    const float b = __builtin_fminf(__builtin_fmaxf(__builtin_ldexpf(h[r][1], sh), -448.0f), 448.0f);
    o[r] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xffffu;
  }
  if (sc == 255u) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      o[r] = (((__float_as_uint(h[r][0]) >> 24) & 0x80u) | 0x7fu) |
             ((((__float_as_uint(h[r][1]) >> 24) & 0x80u) | 0x7fu) << 8);
  }
}

// alpha * tanh(x / alpha) as num / den = a P(a^2) / Q(a^2), a = x clamped to [-8 alpha, 8 alpha] (past 8,
// tanh is 1 to within 2.3e-7): tanh(y) ~ y p(y^2) / q(y^2) with p of degree 3 and q of degree 4 (q(0) = 1), a
// minimax fit of the relative error made for this kernel (linear programming on a dense grid of [0, 8] with
// Loeb reweighting; 1.7e-7 in exact arithmetic, 4.0e-7 with an f32 evaluation). Its coefficients are scaled
// once per expert (SituCoef: the coefficient of y^2k times alpha^-2k, so P(a^2) = p(y^2) for a = alpha y):
// no multiply by 1/alpha, and the alpha of alpha * tanh cancels the 1/alpha of y. Seven FMAs and no
// transcendental, so that SiTU-GLU below needs one exponential and one reciprocal in all. The clamp
// propagates NaN.
struct SituCoef {
  float p1, p2, p3, q1, q2, q3, q4, c;  // wave-uniform (kept in SGPRs)
};
KERN_DEV float uniform_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
}
KERN_DEV SituCoef situ_coef(float alpha) {
  const float ia = 1.0f / alpha, i2 = ia * ia;
  SituCoef C;
  float sc = i2;
  C.p1 = uniform_f32(1.292369813e-01f * sc), C.q1 = uniform_f32(4.625690877e-01f * sc);
  sc *= i2;
  C.p2 = uniform_f32(2.948877867e-03f * sc), C.q2 = uniform_f32(2.380688488e-02f * sc);
  sc *= i2;
  C.p3 = uniform_f32(1.140421136e-05f * sc), C.q3 = uniform_f32(2.383597312e-04f * sc);
  sc *= i2;
  C.q4 = uniform_f32(2.451302805e-07f * sc);
  C.c = uniform_f32(8.0f * alpha);
  return C;
}
KERN_DEV void tanh_pq_clamped(float a, const SituCoef& C, float& num, float& den) {
  const float s = a * a;
  float p = __builtin_fmaf(s, C.p3, C.p2);
  p = __builtin_fmaf(p, s, C.p1);
  p = __builtin_fmaf(p, s, 9.999998808e-01f);
  float q = __builtin_fmaf(s, C.q4, C.q3);
  q = __builtin_fmaf(q, s, C.q2);
  q = __builtin_fmaf(q, s, C.q1);
  q = __builtin_fmaf(q, s, 1.0f);
  num = a * p;
  den = q;
}
KERN_DEV void tanh_pq(float x, const SituCoef& C, float& num, float& den) {
  tanh_pq_clamped(__builtin_elementwise_minimum(__builtin_elementwise_maximum(x, -C.c), C.c), C, num, den);
}

// SiTU-GLU (tools/trtllm-bmm/probe.py:23, :46-47) of gate g and up u, alpha * tanh(g / alpha) * sigmoid(g) *
// beta * tanh(u / beta), with G = situ_coef(alpha) and U = situ_coef(beta), as one fraction:
// na * nb / (da * db * (1 + exp(-g))) with alpha * tanh = na / da and beta * tanh = nb / db from tanh_pq. One
// exponential and one hardware reciprocal, no divides. Where exp(-g) or the denominator overflows (g below
// about -76, sigmoid(g) < 1e-33) the value is 0; NaN in g or u gives NaN.
KERN_DEV float situ_fast(float g, float u, const SituCoef& G, const SituCoef& U) {
  float na, da, nb, db;
  // the gate's clamp need not keep a NaN (V_MED3_F32, one instruction): exp(-g) carries it into the result
  tanh_pq_clamped(__builtin_amdgcn_fmed3f(g, -G.c, G.c), G, na, da);
  tanh_pq(u, U, nb, db);
  const float d = da * db;
  return (na * nb) * __builtin_amdgcn_rcpf(__builtin_fmaf(d, __expf(-g), d));
}

// The scale operand of V_CVT_SCALEF32_PK_BF16_FP4 for e8m0 code `code`: the instruction reads only the
// operand's exponent field as an e8m0 code, so the bare field (code << 23) converts exactly as
// e8m0_to_f32(code) does, codes 0 and 255 included (all 256 codes x 256 byte patterns x 4 selects compared
// on the device).
KERN_DEV float fp4_cvt_scale(uint32_t code) { return __uint_as_float(code << 23); }

// f32 value 2^(code-127) (code 0 is the subnormal 2^-127, 255 is NaN)
KERN_DEV float e8m0_to_f32(uint32_t code) {
  const uint32_t b = code == 0u ? 0x00400000u : (code == 255u ? 0x7fc00000u : code << 23);  // selects, no branches
  return __uint_as_float(b);
}

// splitmix64 i-th draw of a stream (crates/kern-test/src/workload.rs:18-24)
KERN_DEV uint64_t splitmix64_at(uint64_t seed, uint64_t i) {
  uint64_t z = seed + (i + 1ull) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
