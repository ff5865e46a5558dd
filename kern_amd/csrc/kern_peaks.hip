// Roofline probes for bench.py's `peaks` leg: the sustained rate of the scaled MFMA in each operand format
// the path uses, and the HBM streaming-read rate. A code object of its own (kern_peaks.hsaco), loaded through
// the module layer of the C ABI; nothing on the product path launches it.
//
//   kern_peak_mfma16_<a>_<b>: every wave multiplies 64x64 tiles over K in steps of 128 on
//     V_MFMA_SCALE_F32_16X16X128_F8F6F4 (16 instructions a step, 16 independent accumulators), alternating
//     two operand sets of random bytes (codes that are not NaN), e8m0 scales 1.0. FLOPs = waves * steps *
//     2 * 64 * 64 * 128.
//   kern_peak_mfma32_<a>_<b>: the same tiles on V_MFMA_SCALE_F32_32X32X64_F8F6F4 (8 instructions a step).
//   kern_peak_stream: reads n16 16-byte words once (non-temporal loads, four in flight per lane, grid
//     stride) and folds them into one word per lane, stored only when it equals a fixed value.
//   kern_peak_empty: nothing (the cost of a dispatch).
//
// And a check of a hardware conversion the product kernels rely on:
//   kern_probe_bf16_cvt: for every f32 bit pattern u in [lo, lo + n), the hardware bf16 packing
//     (bf16x2_hw, V_CVT_PK_BF16_F32) against the software round-to-nearest-even (f32_to_bf16_bits), on u and
//     on u with its sign flipped; counts the mismatches into out[0] and leaves one mismatching input in out[1].
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mx_device.h"

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));

// operand bytes: random, with the e4m3 NaN codes (0x7f, 0xff) turned into 0x7e / 0xfe
static __device__ __forceinline__ int no_nan(int v) {
  const unsigned u = (unsigned)v;
  const unsigned nan = (((u & 0x7f7f7f7fu) + 0x01010101u) & 0x80808080u);  // byte is x7f -> its top bit set
  return (int)(u ^ (nan >> 7));
}

template <int CBSZ, int BLGP>
static __device__ void mfma16_loop(const int* __restrict__ src, float* __restrict__ out, int steps) {
  const int lane = threadIdx.x & 63;
  v8i a[2][4], b[2][4];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        a[s][i][j] = no_nan(src[((s * 4 + i) * 8 + j) * 64 + lane]);
        b[s][i][j] = no_nan(src[4096 + ((s * 4 + i) * 8 + j) * 64 + lane]);
      }
  v4f acc[4][4] = {};
  const int one = 0x7f7f7f7f;
  for (int t = 0; t < steps; t += 2) {
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[s][i], b[s][j], acc[i][j], CBSZ, BLGP, 0,
                                                                        one, 0, one);
  }
  float r = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) r += acc[i][j][0] + acc[i][j][1] + acc[i][j][2] + acc[i][j][3];
  if (r == 1.2345f) out[0] = r;
}

template <int CBSZ, int BLGP>
static __device__ void mfma32_loop(const int* __restrict__ src, float* __restrict__ out, int steps) {
  const int lane = threadIdx.x & 63;
  v8i a[2][4], b[2][4];  // [set][tile * 2 + k half]
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        a[s][i][j] = no_nan(src[((s * 4 + i) * 8 + j) * 64 + lane]);
        b[s][i][j] = no_nan(src[4096 + ((s * 4 + i) * 8 + j) * 64 + lane]);
      }
  v16f acc[2][2] = {};
  const int one = 0x7f7f7f7f;
  for (int t = 0; t < steps; t += 2) {
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[s][i * 2 + kh], b[s][j * 2 + kh], acc[i][j],
                                                                        CBSZ, BLGP, 0, one, 0, one);
  }
  float r = 0.f;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) r += acc[i][j][e];
  if (r == 1.2345f) out[0] = r;
}

// CBSZ / BLGP format codes of the F8F6F4 MFMA: 0 = fp8 e4m3, 4 = fp4 e2m1 (A = first operand)
#define PEAK_MFMA(NAME, CB, BL)                                                                                 \
  extern "C" __global__ __launch_bounds__(256) void kern_peak_mfma16_##NAME(const int* src, float* out, int steps) { \
    mfma16_loop<CB, BL>(src, out, steps);                                                                      \
  }                                                                                                            \
  extern "C" __global__ __launch_bounds__(256) void kern_peak_mfma32_##NAME(const int* src, float* out, int steps) { \
    mfma32_loop<CB, BL>(src, out, steps);                                                                      \
  }
PEAK_MFMA(fp8_fp8, 0, 0)
PEAK_MFMA(fp4_fp8, 4, 0)
PEAK_MFMA(fp4_fp4, 4, 4)
#undef PEAK_MFMA

extern "C" __global__ __launch_bounds__(256) void kern_peak_stream(const v4u* __restrict__ src, int64_t n16,
                                                                   unsigned* __restrict__ out) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  v4u acc = {0u, 0u, 0u, 0u};
  int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const v4u v0 = __builtin_nontemporal_load(src + i);
    const v4u v1 = __builtin_nontemporal_load(src + i + stride);
    const v4u v2 = __builtin_nontemporal_load(src + i + 2 * stride);
    const v4u v3 = __builtin_nontemporal_load(src + i + 3 * stride);
    acc ^= v0 ^ v1 ^ v2 ^ v3;
  }
  for (; i < n16; i += stride) acc ^= __builtin_nontemporal_load(src + i);
  const unsigned r = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (r == 0x9e3779b9u) out[0] = r;  // a data-dependent store keeps the loads (harmless if it ever happens)
}

extern "C" __global__ void kern_peak_empty(int* out) { (void)out; }

// The GEMVs' fp4 -> bf16 conversion scale (fp4_cvt_scale: the bare e8m0 exponent field) against the f32 value
// e8m0_to_f32 of the same code: thread (code = blockIdx.x, byte = threadIdx.x) converts a dword holding the
// byte in each position under both, all four byte selects; mismatches are counted in out[0], the last one's
// (code << 8 | byte) in out[1]. Grid 256, block 256.
typedef __bf16 v2bf16_t __attribute__((ext_vector_type(2)));
extern "C" __global__ __launch_bounds__(256) void kern_probe_fp4_scale(uint32_t* out) {
  const uint32_t code = blockIdx.x, b = threadIdx.x;
  const uint32_t w = b | (((b * 0x9E3779B9u) >> 8) & 0xffffff00u);
  const float s_val = e8m0_to_f32(code), s_fld = fp4_cvt_scale(code);
  uint32_t bad = 0;
#pragma unroll
  for (int sel = 0; sel < 4; ++sel) {
    const uint32_t ws = sel == 0 ? w : (sel == 1 ? ((w << 8) | b) : (sel == 2 ? ((w << 16) | (b << 8) | b) : (w << 24) | (b * 0x010101u)));
    const v2bf16_t x0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(ws, s_val, 0), y0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(ws, s_fld, 0);
    const v2bf16_t x1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(ws, s_val, 1), y1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(ws, s_fld, 1);
    const v2bf16_t x2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(ws, s_val, 2), y2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(ws, s_fld, 2);
    const v2bf16_t x3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(ws, s_val, 3), y3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(ws, s_fld, 3);
    bad += (__builtin_bit_cast(uint32_t, x0) != __builtin_bit_cast(uint32_t, y0)) +
           (__builtin_bit_cast(uint32_t, x1) != __builtin_bit_cast(uint32_t, y1)) +
           (__builtin_bit_cast(uint32_t, x2) != __builtin_bit_cast(uint32_t, y2)) +
           (__builtin_bit_cast(uint32_t, x3) != __builtin_bit_cast(uint32_t, y3));
  }
  if (bad) {
    atomicAdd(out, bad);
    out[1] = (code << 8) | b;
  }
}

extern "C" __global__ __launch_bounds__(256) void kern_probe_bf16_cvt(uint32_t lo, uint32_t n, uint32_t* out) {
  uint32_t bad = 0, which = 0;
  const uint64_t stride = (uint64_t)gridDim.x * 256u;
  for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < n; i += stride) {
    const uint32_t u = lo + (uint32_t)i, v = u ^ 0x80000000u;
    const uint32_t hw = bf16x2_hw(__uint_as_float(u), __uint_as_float(v));
    const uint32_t sw = f32_to_bf16_bits(__uint_as_float(u)) | (f32_to_bf16_bits(__uint_as_float(v)) << 16);
    if (hw != sw) ++bad, which = u;
  }
  if (bad) {
    atomicAdd(out, bad);
    out[1] = which;
  }
}
