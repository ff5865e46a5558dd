// gfx950 kernels of the MXFP4 matmul path. Built into one code object (kern_mx.hsaco) whose entries
// take flat kernel arguments in the order of their manifest launch `params`; the C ABI in capi.cpp
// launches them with hipModuleLaunchKernel from that sha256-pinned object.
//
// Data layouts in HBM (all byte offsets; E experts, m weight rows, K reduction length):
//   raw MXFP4 weights   u8 [E][m][K/2], element 2j in the low nibble        (probe.py:28)
//   raw scales          u8 [E][m][K/32] e8m0                                 (probe.py:31)
//   repacked weights    per expert, 1 KiB fragment ((R/16)*(K/128) + k/128); lane L = 16*((k%128)/32) + R%16
//                       owns the 16 bytes at L*16 = k in [128*kt + 32*(L/16), +32) of row R: exactly the
//                       fp4 A-operand of V_MFMA_SCALE_F32_16X16X128_F8F6F4 for lane L.
//   repacked scales     per expert, 256 B fragment ((R/16)*(K/512) + k/512); lane L owns a dword whose byte j
//                       is the scale of row R, k-block 16*kg + 4*j + L/16 (MFMA scale operand, OPSEL = j).
//   gated (FC1) rows    repacked row R holds raw row: quad (R%16)/4 of group R/16 is gate n, gate n+1, up n,
//                       up n+1 (n = 8*(R/16) + 2*((R%16)/4)); gate = rows [m/2, m) (w1), up = [0, m/2) (w3).
//   activations         e4m3 u8 [rows][K], scales linear u8 [rows][K/32] or R128c4 (cublas.rs:396-400)
#include "mx_device.h"

template <int V>
struct IC { static constexpr int value = V; };

// ====================================================================================== quantizer
// op moe_quant (fixtures/k3/head.json:25057): in bf16 x[T][K], out u8 q[T][K], out u8 sf[T][K/32], i32 T,
// launch i32 K. Two lanes per 32-element block, 16 elements (two 16-byte loads) per lane, so a wave-wide
// load covers 1 KiB of contiguous input and each 16-byte store 1 KiB of output; the block amax is
// reduced over the lane pair with DPP. A workgroup covers 4096 elements: grid ceil(T*K / 4096), block 256.
// Lane p of the launch (p even on even lanes) takes elements [16p, 16p + 16).
KERN_DEV void quant_bf16_lane(const uint16_t* __restrict__ x, uint8_t* __restrict__ q, uint8_t* __restrict__ sf, int T,
                              int K, int64_t p) {
  // a lane takes 16 adjacent elements (half a 32-element block), a lane pair one block: one cross-lane step
  // for the block's amax, one 16-byte store. (8 elements per lane, four lanes per block, two chunks per
  // lane: 3% slower at config 3's activations; more than one pair per lane was slower still.)
  const int64_t np = (int64_t)T * (K >> 4);
  // a lane pair is in or out of range together (K % 32 == 0: np is even)
  if (p >= np) return;
  // default-policy loads: at [4096, 7168], non-temporal ones took 16.5 us against 15.5 us over eight rotating
  // inputs (none resident in the Infinity Cache) and 16.3 against 14.1 us on one input. The weight streams of
  // the GEMVs and skinny MoE tiles are the other way round: non-temporal is 4-15% faster there.
  const v4u v0 = reinterpret_cast<const v4u*>(x)[2 * p];
  const v4u v1 = reinterpret_cast<const v4u*>(x)[2 * p + 1];
  uint32_t amax = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    amax = max(amax, max((v0[j] << 16) & 0x7fffffffu, v0[j] & 0x7fff0000u));
    amax = max(amax, max((v1[j] << 16) & 0x7fffffffu, v1[j] & 0x7fff0000u));
  }
  amax = max(amax, (uint32_t)__builtin_amdgcn_mov_dpp((int)amax, 0xB1, 0xF, 0xF, false));  // lane ^ 1
  const uint32_t sc = mx_scale_code(amax);
  v4u out;
  out[0] = mx_pack4(v0[0], v0[1], sc);
  out[1] = mx_pack4(v0[2], v0[3], sc);
  out[2] = mx_pack4(v1[0], v1[1], sc);
  out[3] = mx_pack4(v1[2], v1[3], sc);
  reinterpret_cast<v4u*>(q)[p] = out;
  if ((threadIdx.x & 1) == 0) sf[p >> 1] = (uint8_t)sc;  // p and the lane have the same parity
}
extern "C" __global__ __launch_bounds__(256) void kern_mx_quant_bf16(const uint16_t* __restrict__ x,
                                                                     uint8_t* __restrict__ q,
                                                                     uint8_t* __restrict__ sf, int T, int K) {
  quant_bf16_lane(x, q, sf, T, K, (int64_t)blockIdx.x * 256 + threadIdx.x);
}

// f32 -> MXFP8 with the codec of the FC1 epilogue (mx_scale_code of the block's largest |bits|, then
// mx_code2 pairs): in f32 x[T][K], out u8 q[T][K], out u8 sf[T][K/32], i32 T, i32 K (K % 32 == 0). Four
// lanes per 32-element block, eight elements (two 16-byte loads) per lane; the block amax is reduced over
// the four lanes. Grid ceil(T*K / 2048), block 256.
extern "C" __global__ __launch_bounds__(256) void kern_mx_quant_f32(const float* __restrict__ x,
                                                                    uint8_t* __restrict__ q,
                                                                    uint8_t* __restrict__ sf, int T, int K) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;  // 8-element piece
  const int64_t np = (int64_t)T * (K >> 3);
  // the four lanes of a block are in or out of range together (K % 32 == 0: np is a multiple of 4)
  if (p >= np) return;
  const v4u v0 = reinterpret_cast<const v4u*>(x)[2 * p];
  const v4u v1 = reinterpret_cast<const v4u*>(x)[2 * p + 1];
  uint32_t amax = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) amax = max(amax, max(v0[j] & 0x7fffffffu, v1[j] & 0x7fffffffu));
  amax = max(amax, (uint32_t)__shfl_xor((int)amax, 1));
  amax = max(amax, (uint32_t)__shfl_xor((int)amax, 2));
  const uint32_t sc = mx_scale_code(amax);
  const uint32_t c0 = mx_code2(__uint_as_float(v0[0]), __uint_as_float(v0[1]), sc);
  const uint32_t c1 = mx_code2(__uint_as_float(v0[2]), __uint_as_float(v0[3]), sc);
  const uint32_t c2 = mx_code2(__uint_as_float(v1[0]), __uint_as_float(v1[1]), sc);
  const uint32_t c3 = mx_code2(__uint_as_float(v1[2]), __uint_as_float(v1[3]), sc);
  reinterpret_cast<uint2*>(q)[p] = make_uint2(c0 | (c1 << 16), c2 | (c3 << 16));
  if ((threadIdx.x & 3) == 0) sf[p >> 2] = (uint8_t)sc;
}

// ====================================================================================== repack
// derive op k3_moe_w_shuffle (head.json:26358): in u8 raw, out u8 shuffled, i32 rows, i32 row_bytes,
// i32 gated; launch prepends i32 E. One thread per 16-byte lane slot of the output; grid
// E*rows*row_bytes/16/256, block 256.
KERN_DEV int64_t w_src_row(int64_t R, int64_t rows, int gated) {
  if (!gated) return R;
  int64_t j = R & 3;
  int64_t n = 8 * (R >> 4) + 2 * ((R & 15) >> 2) + (j & 1);
  return j < 2 ? (rows >> 1) + n : n;
}

extern "C" __global__ __launch_bounds__(256) void kern_mx_w_shuffle(const uint8_t* __restrict__ raw,
                                                                    uint8_t* __restrict__ out, int E, int rows,
                                                                    int row_bytes, int gated) {
  const int64_t slot = (int64_t)blockIdx.x * 256 + threadIdx.x;  // 16-byte output slot
  const int64_t KT = row_bytes / 64;
  const int64_t per_e = (int64_t)rows * row_bytes / 16;
  if (slot >= per_e * E) return;
  const int64_t e = slot / per_e;
  const int64_t s = slot - e * per_e;
  const int64_t frag = s >> 6, L = s & 63;
  const int64_t rg = frag / KT, kt = frag - rg * KT;
  const int64_t R = rg * 16 + (L & 15);
  const int64_t src = (e * rows + w_src_row(R, rows, gated)) * row_bytes + kt * 64 + (L >> 4) * 16;
  const v4u val = *reinterpret_cast<const v4u*>(raw + src);
  reinterpret_cast<v4u*>(out)[slot] = val;
}

// derive op k3_moe_sf_shuffle (head.json:26413): in u8 raw, out u8 shuffled, i32 rows, i32 sf_cols,
// i32 gated; launch prepends i32 E. One thread per output dword; grid E*rows*sf_cols/4/256, block 256.
extern "C" __global__ __launch_bounds__(256) void kern_mx_sf_shuffle(const uint8_t* __restrict__ raw,
                                                                     uint8_t* __restrict__ out, int E, int rows,
                                                                     int sf_cols, int gated) {
  const int64_t d = (int64_t)blockIdx.x * 256 + threadIdx.x;  // output dword
  const int64_t KG = sf_cols / 16;
  const int64_t per_e = (int64_t)rows * sf_cols / 4;
  if (d >= per_e * E) return;
  const int64_t e = d / per_e;
  const int64_t s = d - e * per_e;
  const int64_t frag = s >> 6, L = s & 63;
  const int64_t rg = frag / KG, kg = frag - rg * KG;
  const int64_t R = rg * 16 + (L & 15);
  const uint8_t* src = raw + (e * rows + w_src_row(R, rows, gated)) * sf_cols + kg * 16 + (L >> 4);
  uint32_t v = (uint32_t)src[0] | ((uint32_t)src[4] << 8) | ((uint32_t)src[8] << 16) | ((uint32_t)src[12] << 24);
  reinterpret_cast<uint32_t*>(out)[d] = v;
}

// LDS and global address spaces (operands of the direct global->LDS loads)
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glob_void_t;

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding: vmcnt[3:0] | expcnt 7 << 4 |
// lgkmcnt 15 << 8 | vmcnt[5:4] << 14)
#define WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | 0x70 | 0xF00 | (((n) >> 4) << 14))
// s_waitcnt lgkmcnt(0) with vmcnt and expcnt left alone
#define WAIT_LGKMCNT0 __builtin_amdgcn_s_waitcnt(0xC07F)

// ====================================================================================== decode GEMV
// op mxfp4_gemv_bf16 (new; the W4A16 decode, M <= 16 tokens): in bf16 x[M][K], in u8 w (repacked,
// non-gated) [N][K/2], in u8 w_sf (repacked), out bf16 y[M][N], i32 M, launch i32 N, i32 K, i32 nb, i32 sb.
// Grid N/16, block 256, dynamic LDS M*(sb*1024 + 16) + K/2 bytes: one 16-row group per workgroup. Wave w
// takes the 128-wide k-tiles kt = 4i + w (equal shares; its scale is byte w of each scale dword of the
// group). x is consumed in slices of sb k-tiles per wave (sb divides K/512, M*sb <= 16), weights in rounds
// of nb fragments per wave (nb divides sb). Each slice of x, and with the first slice the row group's
// whole scale block, goes from memory straight into LDS (buffer loads to LDS, no registers); the round's
// weight fragments are requested behind them in straight-line code, so waiting for the LDS data leaves
// the weights in flight, and each fragment is multiplied as soon as it lands. At M = 1, K = 7168 one
// slice covers the row group and the weights come in two rounds of 7 KiB per wave.
// fp4 is decoded with its scale by V_CVT_SCALEF32_PK_BF16_FP4 and multiplied on V_MFMA_F32_16X16X32_BF16
// (tokens are the 16 B columns; columns >= M are computed and dropped); the four partial sums meet in LDS.

// 16 bytes per lane from a buffer straight into LDS at `lds_wave_base + 16 * lane` (wave-uniform base);
// offsets past the buffer's end read zeros
KERN_DEV void dma16_buf(__amdgpu_buffer_rsrc_t r, int voffset, void* lds_wave_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds_wave_base, 16, voffset, 0, 0, 0);
}

template <int NB>
KERN_DEV v4f gemv_rows(__amdgpu_buffer_rsrc_t xr, __amdgpu_buffer_rsrc_t wr_, __amdgpu_buffer_rsrc_t sr_, uint16_t* xs,
                       int M, int K, int nk, int sb, int lane, int c, int grp, int wave, bool live) {
  const int row = sb * 512 + 8;  // LDS row stride in bf16 (16 B pad)
  const int per_tok = 64 * sb;   // 16-byte pieces of one token's slice: a multiple of 64
  const int pieces = M * per_tok;         // <= 1024: at most four requests per wave
  const int spieces = (K >> 9) * 16;      // 16-byte pieces of the row group's scales (<= 512)
  uint8_t* ss = reinterpret_cast<uint8_t*>(xs + M * row);  // the row group's scales, as stored in HBM
  // lanes of absent tokens (c >= M) read token 0's row: an MFMA output column depends on its own B
  // column only, and the columns of absent tokens are never stored
  const uint16_t* xl = xs + (live ? c : 0) * row + wave * 128 + grp * 32;
  // this wave's scale byte (k-tile 4*kg + wave) in the dword of this lane at k group kg
  const uint8_t* sl = ss + lane * 4 + wave;
  const int wv = (wave * 64 + lane) * 16;  // this lane's byte in a 4 KiB group of four fragments
  v4f acc[2] = {};  // two chains, so consecutive MFMAs do not wait on each other
  for (int s0 = 0; s0 < nk; s0 += sb) {
    if (s0) __syncthreads();  // every wave's reads of the previous slice are done
    // x[:, 512*s0 .. 512*(s0+sb)) and (first slice) the scales go from memory straight into LDS:
    // request r of this wave moves pieces 256r + 64*wave + lane (all of one token: piece q is token
    // q / per_tok, column (q % per_tok)*8)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int q0 = 256 * r + 64 * wave;
      if (q0 < pieces) {
        const int t = q0 / per_tok, col0 = (q0 - t * per_tok) * 8;
        dma16_buf(xr, (t * K + s0 * 512 + col0 + lane * 8) * 2, xs + t * row + col0);
      }
    }
    if (s0 == 0) {
      // per lane: the scale region holds exactly spieces pieces (K/2 bytes), which need not fill a
      // wave's request, and lanes past it must not write LDS beyond the region
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int q0 = 256 * r + 64 * wave;
        if (q0 + lane < spieces) dma16_buf(sr_, (q0 + lane) * 16, ss + q0 * 16);
      }
    }
    for (int i0 = s0; i0 < s0 + sb; i0 += NB) {
      // weights after x and the scales, so that their wait below leaves the weights in flight; the
      // scheduling barriers keep the issue order as written
      __builtin_amdgcn_sched_barrier(0);
      v4u wv4[NB];
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        wv4[u] = __builtin_amdgcn_raw_buffer_load_b128(wr_, wv, (i0 + u) * 4096, 2);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (i0 == s0) {
        WAIT_VMCNT(NB);  // this wave's requests into LDS have landed (only the weights may be in flight)
        __syncthreads();  // ... and every wave's
      }
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        const float s = fp4_cvt_scale(sl[(i0 + u) * 256]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // A: 8 fp4 of this lane's row, k = 32*grp + 8*j .. +8 of the tile (dword j of the lane's slot)
          const uint32_t wd = wv4[u][j];
          v2bf p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, s, 0);
          v2bf p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, s, 1);
          v2bf p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, s, 2);
          v2bf p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, s, 3);
          v8bf a = {p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
          const v4u xb = *reinterpret_cast<const v4u*>(xl + (i0 - s0 + u) * 512 + j * 8);
          acc[j & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(v8bf, xb), acc[j & 1], 0, 0, 0);
        }
      }
    }
  }
  return acc[0] + acc[1];
}

extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(5))) void kern_mx_gemv_bf16(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ w, const uint8_t* __restrict__ wsf,
    uint16_t* __restrict__ y, int M, int N, int K, int nb, int sb) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];  // [M][sb*512 + 8], then the scales
  __shared__ v4f red[4][64];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rg = blockIdx.x;
  const int KT = K >> 7, KG = K >> 9;
  const int nk = KT >> 2;  // k-tiles of every wave (K % 512 == 0)
  const int c = lane & 15, grp = lane >> 4;
  const bool live = c < M;
  // buffer resources: this row group's fragments and scales, and x (out-of-range reads return zero)
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, M * K * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t wr_ =
      __builtin_amdgcn_make_buffer_rsrc((void*)(w + (int64_t)rg * KT * 1024), (short)0, KT * 1024, 0x00020000);
  const __amdgpu_buffer_rsrc_t sr_ =
      __builtin_amdgcn_make_buffer_rsrc((void*)(wsf + (int64_t)rg * KG * 256), (short)0, KG * 256, 0x00020000);
  v4f acc;
  switch (nb) {
    case 7: acc = gemv_rows<7>(xr, wr_, sr_, xs, M, K, nk, sb, lane, c, grp, wave, live); break;
    case 4: acc = gemv_rows<4>(xr, wr_, sr_, xs, M, K, nk, sb, lane, c, grp, wave, live); break;
    case 2: acc = gemv_rows<2>(xr, wr_, sr_, xs, M, K, nk, sb, lane, c, grp, wave, live); break;
    default: acc = gemv_rows<1>(xr, wr_, sr_, xs, M, K, nk, sb, lane, c, grp, wave, live); break;
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    v4f s = red[0][lane] + red[1][lane] + red[2][lane] + red[3][lane];
    if (live) {
      // lane (c, grp) holds rows 4*grp + i of the group for token c
      const int n0 = rg * 16 + grp * 4;
      uint32_t lo = f32_to_bf16_bits(s[0]) | (f32_to_bf16_bits(s[1]) << 16);
      uint32_t hi = f32_to_bf16_bits(s[2]) | (f32_to_bf16_bits(s[3]) << 16);
      uint2* dst = reinterpret_cast<uint2*>(y + (int64_t)c * N + n0);
      *dst = make_uint2(lo, hi);
    }
  }
}

// ---------------------------------------------------------------- decode GEMV, M <= 2: one row group per workgroup
// Same operand mapping as above (fp4 rows decoded by V_CVT_SCALEF32_PK_BF16_FP4 into the A operand of
// V_MFMA_F32_16X16X32_BF16, tokens in the B columns). One workgroup of four waves per 16-row group, so
// all N/16 workgroups are resident at once (18 waves per CU at N = 18432). Wave w owns the 512-wide k
// groups [w*KG/4, (w+1)*KG/4) of its row group, contiguous, so that
//   * its slice of x (1 KiB per token and k group) goes into a wave-private LDS region with one
//     buffer->LDS request per KiB, and no workgroup barrier precedes the first multiply;
//   * one scale dword per k group (the lane's dword of the group's 256 B scale fragment) carries the
//     scales of all four k-tiles of the group;
//   * its weight fragments are one contiguous run, streamed four ahead with non-temporal loads.
// Fewer fragments in flight per wave ran faster than more (4: 12.7 us, 14: 13.6 us at N = 18432,
// K = 7168); with 18 waves per CU, four in flight already keep HBM saturated.
// The four partial sums meet in LDS at the end. LDS: 4 * ceil(KG/4) * M KiB (dynamic) + 4 KiB.
extern "C" __global__ __launch_bounds__(256) void kern_mx_gemv_bf16_rg(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ w, const uint8_t* __restrict__ wsf,
    uint16_t* __restrict__ y, int M, int N, int K, int gmax) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xg[];  // [wave][gmax][M][512]
  __shared__ v4f red[4][64];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rg = blockIdx.x;
  const int KG = K >> 9, KT = K >> 7;
  const int g0 = (wave * KG) >> 2, ng = (((wave + 1) * KG) >> 2) - g0;
  const int c = lane & 15, kq = lane >> 4;
  uint16_t* xw = xg + wave * gmax * M * 512;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, M * K * 2, 0x00020000);
  for (int g = 0; g < ng; ++g)
    for (int t = 0; t < M; ++t) dma16_buf(xr, (t * K + (g0 + g) * 512) * 2 + lane * 16, xw + (g * M + t) * 512);
  __builtin_amdgcn_sched_barrier(0);
  const __amdgpu_buffer_rsrc_t sr =
      __builtin_amdgcn_make_buffer_rsrc((void*)(wsf + ((int64_t)rg * KG + g0) * 256), (short)0, ng * 256, 0x00020000);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(w + ((int64_t)rg * KT + 4 * g0) * 1024), (short)0, ng * 4096, 0x00020000);
  // lanes of absent tokens (c >= M) read token 0's x: an MFMA output column depends on its own B column
  // only, and the columns of absent tokens are never stored
  // only the lanes of present tokens (c < M) read x: the B columns of absent tokens are never stored, and
  // an MFMA output column depends on its own B column only, so their registers may hold anything
  const bool xlive = c < M;
  const uint16_t* xl = xw + c * 512 + 32 * kq;
  v4u xb[4] = {};
  v4f acc[2] = {};
  if (ng > 0) {
    uint32_t sc = __builtin_amdgcn_raw_buffer_load_b32(sr, lane * 4, 0, 2);
    v4u b[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      b[u] = __builtin_amdgcn_raw_buffer_load_b128(wr, u * 1024 + lane * 16, 0, 2);
      __builtin_amdgcn_sched_barrier(0);
    }
    WAIT_VMCNT(5);  // requests complete in order: the x slice has landed, the scale and weights may not have
    // the next group's requests are issued unconditionally (past the last group they point beyond the
    // buffer and read zeros without touching memory): with a branch around them the compiler's wait
    // counts would have to assume none were issued and drain every request before each group's last
    // fragment
    for (int g = 0; g < ng; ++g) {
      const int nx = g + 1 < ng ? 0 : 0x40000000;
      const uint32_t sc_next = __builtin_amdgcn_raw_buffer_load_b32(sr, nx + (g + 1) * 256 + lane * 4, 0, 2);
      __builtin_amdgcn_sched_barrier(0);
      const uint16_t* xk = xl + g * M * 512;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float s = fp4_cvt_scale((sc >> (8 * u)) & 0xffu);
        if (xlive) {
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) xb[jj] = *reinterpret_cast<const v4u*>(xk + u * 128 + jj * 8);
        }
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const uint32_t wd = b[u][jj];
          v2bf p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, s, 0);
          v2bf p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, s, 1);
          v2bf p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, s, 2);
          v2bf p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, s, 3);
          v8bf a = {p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
          acc[jj & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(v8bf, xb[jj]), acc[jj & 1], 0, 0, 0);
        }
        b[u] = __builtin_amdgcn_raw_buffer_load_b128(wr, nx + (4 * (g + 1) + u) * 1024 + lane * 16, 0, 2);
        __builtin_amdgcn_sched_barrier(0);
      }
      sc = sc_next;
    }
  }
  red[wave][lane] = acc[0] + acc[1];
  __syncthreads();
  if (wave == 0) {
    const v4f s = red[0][lane] + red[1][lane] + red[2][lane] + red[3][lane];
    if (c < M) {
      // lane (c, kq) holds rows 4*kq + i of the group for token c
      const int n0 = rg * 16 + kq * 4;
      const uint32_t lo = f32_to_bf16_bits(s[0]) | (f32_to_bf16_bits(s[1]) << 16);
      const uint32_t hi = f32_to_bf16_bits(s[2]) | (f32_to_bf16_bits(s[3]) << 16);
      *reinterpret_cast<uint2*>(y + (int64_t)c * N + n0) = make_uint2(lo, hi);
    }
  }
}

// --------------------------------------------- decode GEMV at fixed K: the same, fully unrolled
// Taken (kern_mxfp4_gemv_bf16) for K = 512 * NKT while the x slices, 2*M*K bytes of dynamic LDS, fit in
// 144 KiB, at M <= 3 or at any M <= 16 while N <= 8192; with the static ssc and red arrays (at most 5 KiB)
// the workgroup stays below the 160 KiB of LDS.
// For K = 512 * NKT with NKT in {2, 4, 8, 14, 16} each wave owns exactly NKT consecutive k-tiles (k-tile
// ranges, not whole 512-wide groups) and its loop is unrolled, so the weight stream has no requests past
// its end and no branches around them: every request is one the compiler's wait counts can see, and an
// extra request per wave costs measurably (one unneeded 256 B scale fragment per wave: +0.8 us at N =
// 18432). The wave's scale fragments (those its k-tiles touch, at most five) go into LDS with one
// buffer->LDS request beside its x slice; each k-tile reads its scale byte from there.
template <int NKT>
KERN_DEV void gemv_rows_fixed(const uint16_t* __restrict__ x, const uint8_t* __restrict__ w,
                              const uint8_t* __restrict__ wsf, uint16_t* __restrict__ y, int M, int N, int K) {
  constexpr int NSMAX = (NKT + 6) / 4;
  extern __shared__ __attribute__((aligned(16))) uint16_t xg[];  // [wave][M][NKT * 128]
  __shared__ v4f red[4][64];
  __shared__ __attribute__((aligned(16))) uint32_t ssc[4][NSMAX * 64];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rg = blockIdx.x;
  const int KG = K >> 9, KT = K >> 7;
  const int kt0 = wave * NKT, kgA = kt0 >> 2;
  const int ns = ((kt0 + NKT - 1) >> 2) - kgA + 1;  // scale fragments the wave's k-tiles touch
  const int c = lane & 15, kq = lane >> 4;
  uint16_t* xw = xg + wave * M * NKT * 128;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, M * K * 2, 0x00020000);
  for (int t = 0; t < M; ++t) {
#pragma unroll
    for (int p = 0; p < NKT * 16; p += 64)
      if (p + lane < NKT * 16) dma16_buf(xr, (t * K + 128 * kt0 + (p + lane) * 8) * 2, xw + t * NKT * 128 + p * 8);
  }
  const __amdgpu_buffer_rsrc_t sr =
      __builtin_amdgcn_make_buffer_rsrc((void*)(wsf + (int64_t)rg * KG * 256), (short)0, KG * 256, 0x00020000);
  if (lane < ns * 16) __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (lds_void_t*)&ssc[wave][0], 16, kgA * 256 + lane * 16, 0, 0, 2);
  __builtin_amdgcn_sched_barrier(0);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(w + ((int64_t)rg * KT + kt0) * 1024), (short)0, NKT * 1024, 0x00020000);
  constexpr int D = NKT < 4 ? NKT : 4;
  v4u buf[D];
#pragma unroll
  for (int i = 0; i < D; ++i) {
    buf[i] = __builtin_amdgcn_raw_buffer_load_b128(wr, i * 1024 + lane * 16, 0, 2);
    __builtin_amdgcn_sched_barrier(0);
  }
  // requests complete in order: once at most the D weight requests are outstanding, the x slice and the
  // scale fragments are in LDS (the compiler does not track these buffer->LDS writes into dynamic LDS)
  WAIT_VMCNT(D);
  const bool xlive = c < M;
  const uint16_t* xl = xw + c * NKT * 128 + 32 * kq;
  // this lane's scale dwords of the wave's k groups, read from LDS once (a byte read per fragment cost
  // LDS time like a 16-byte read: 12.5 -> 12.4 us at config 2); fragment i's dword is number
  // ((kt0 % 4) + i) / 4, one of two known at compile time
  uint32_t sdw[NSMAX];
#pragma unroll
  for (int j = 0; j < NSMAX; ++j) sdw[j] = j < ns ? ssc[wave][j * 64 + lane] : 0u;
  const int ph = kt0 & 3;
  v4u xb[4] = {};
  v4f acc[2] = {};
#pragma unroll
  for (int i = 0; i < NKT; ++i) {
    const v4u wv = buf[i % D];
    const int kt = kt0 + i;
    const uint32_t dw = ((ph + i) >> 2) == (i >> 2) ? sdw[i >> 2] : sdw[(i >> 2) + 1];
    const float s = fp4_cvt_scale((dw >> (8 * (kt & 3))) & 255u);
    if (xlive) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) xb[jj] = *reinterpret_cast<const v4u*>(xl + i * 128 + jj * 8);
    }
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const uint32_t wd = wv[jj];
      v2bf p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, s, 0);
      v2bf p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, s, 1);
      v2bf p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, s, 2);
      v2bf p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, s, 3);
      v8bf a = {p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
      acc[jj & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(v8bf, xb[jj]), acc[jj & 1], 0, 0, 0);
    }
    if (i + D < NKT) buf[i % D] = __builtin_amdgcn_raw_buffer_load_b128(wr, (i + D) * 1024 + lane * 16, 0, 2);
    __builtin_amdgcn_sched_barrier(0);
  }
  red[wave][lane] = acc[0] + acc[1];
  __syncthreads();
  if (wave == 0) {
    const v4f s = red[0][lane] + red[1][lane] + red[2][lane] + red[3][lane];
    if (c < M) {
      const int n0 = rg * 16 + kq * 4;
      const uint32_t lo = f32_to_bf16_bits(s[0]) | (f32_to_bf16_bits(s[1]) << 16);
      const uint32_t hi = f32_to_bf16_bits(s[2]) | (f32_to_bf16_bits(s[3]) << 16);
      *reinterpret_cast<uint2*>(y + (int64_t)c * N + n0) = make_uint2(lo, hi);
    }
  }
}

#define GEMV_ROWS_FIXED(NKT)                                                                                   \
  extern "C" __global__ __launch_bounds__(256) void kern_mx_gemv_bf16_r##NKT(                                   \
      const uint16_t* __restrict__ x, const uint8_t* __restrict__ w, const uint8_t* __restrict__ wsf,          \
      uint16_t* __restrict__ y, int M, int N, int K) {                                                         \
    gemv_rows_fixed<NKT>(x, w, wsf, y, M, N, K);                                                            \
  }
GEMV_ROWS_FIXED(2)
GEMV_ROWS_FIXED(4)
GEMV_ROWS_FIXED(8)
GEMV_ROWS_FIXED(14)
GEMV_ROWS_FIXED(16)
#undef GEMV_ROWS_FIXED

// ------------------------------------------------- decode GEMV, 2 < M <= 16: persistent, x held in registers
// A grid of about 256 workgroups of 8 waves. Workgroup b owns the 8-row half groups [b*hb, (b+1)*hb)
// (hb = 9 at N = 18432: 72 rows, the same share for every CU), which touch at most five 16-row groups;
// the half group it shares with a neighbour is loaded with the other half's lanes pointed past the
// buffer (they read zeros) and only its own rows are stored. Wave w owns k-tiles [w*KTW, (w+1)*KTW)
// (K = 1024*KTW) of every row group and walks them k-tile by k-tile, each across its row groups, so x
// is read once per workgroup instead of once per row group (59 MB of L2 reads at M = 16 against 264 MB)
// and only one k-tile of x is held: the next k-tile's x is requested as a k-tile starts (fetching all
// of x up front stalls the weight stream behind it: 17.2 against 15.3 us at M = 16, N = 18432).
// x is requested row-contiguous (16 lanes a 256-byte row) and passes through 4 KiB of LDS of the wave's
// own, written as loaded and read back in the MFMA's operand pieces: requested straight in those pieces,
// each request gathered 16 rows' 16-byte pieces at a 64-byte stride (M = 16: 15.4 against 14.6-15.0 us
// at N = 18432, 12.5 against 10.5 at N = 7168, K = 8192).
// Fragments stream six ahead. The eight partial sums meet in LDS.
template <int KTW>
KERN_DEV void gemv_persistent(const uint16_t* __restrict__ x, const uint8_t* __restrict__ w,
                              const uint8_t* __restrict__ wsf, uint16_t* __restrict__ y, int M, int N, int K, int hb) {
  constexpr int NG = 5, D = 6, TOT = NG * KTW;
  __shared__ v4f red[8][NG][64];
  __shared__ __attribute__((aligned(16))) uint8_t xst[8][4096];  // per wave, one k-tile of x (16 rows x 256 B)
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int KT = K >> 7, KG = K >> 9;
  const int H = N >> 3;
  const int h0 = blockIdx.x * hb, h1 = min(h0 + hb, H);
  const int g0 = h0 >> 1, ng = ((h1 + 1) >> 1) - g0;  // row groups touched: [g0, g0 + ng), ng <= NG
  const int c = lane & 15, kq = lane >> 4, r = lane & 15;
  const int kt0 = wave * KTW, kgA = kt0 >> 2;
  // x: lane (c, kq) holds x[c][128*kt + 32*kq .. +32] for each of its k-tiles (absent tokens: zeros)
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, M * K * 2, 0x00020000);
  // request p of a k-tile loads rows 4p .. 4p+3, 16 lanes a row and 16 B a lane (row-contiguous); absent
  // tokens read zeros, and requests with no present token are not sent (their LDS rows keep stale bytes,
  // which reach only the MFMA columns of absent tokens, never stored: M = 4, 13.3 -> 12.8 us)
  int xso[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int row = 4 * p + (lane >> 4);
    xso[p] = row < M ? (row * K + 128 * kt0) * 2 + (lane & 15) * 16 : 0x40000000;
  }
  v4u xl[4], xv[4];
  auto load_x = [&](int j) {
#pragma unroll
    for (int p = 0; p < 4; ++p)
      if (4 * p < M) xl[p] = __builtin_amdgcn_raw_buffer_load_b128(xr, xso[p] + 256 * j, 0, 0);
  };
  load_x(0);
  // scale dwords of k groups kgA .. kgA + 2 (KTW <= 8 consecutive k-tiles span at most three groups)
  const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(wsf + (int64_t)g0 * KG * 256), (short)0, ng * KG * 256, 0x00020000);
  constexpr int NS = (KTW + 6) / 4;
  uint32_t sdw[NG][NS];
#pragma unroll
  for (int g = 0; g < NG; ++g)
#pragma unroll
    for (int t = 0; t < NS; ++t) {
      const int kg = kgA + t;
      sdw[g][t] = __builtin_amdgcn_raw_buffer_load_b32(
          sr, (g < ng && kg < KG) ? (g * KG + kg) * 256 + lane * 4 : 0x40000000, 0, 2);
    }
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(w + (int64_t)g0 * KT * 1024), (short)0, ng * KT * 1024, 0x00020000);
  // item i = j*NG + g is fragment (g0 + g, kt0 + j); rows outside the owned half groups read zeros
  auto woff = [&](int i) -> int {
    const int g = i % NG, half = (g0 + g) * 2 + (r >> 3);
    return (g < ng && half >= h0 && half < h1) ? (g * KT + kt0 + i / NG) * 1024 + lane * 16 : 0x40000000;
  };
  v4u buf[D];
#pragma unroll
  for (int i = 0; i < D; ++i) {
    if (i < TOT) buf[i] = __builtin_amdgcn_raw_buffer_load_b128(wr, woff(i), 0, 2);
    __builtin_amdgcn_sched_barrier(0);
  }
  v4f acc[NG][2] = {};
#pragma unroll
  for (int i = 0; i < TOT; ++i) {
    const int g = i % NG, j = i / NG, kt = kt0 + j;
    if (g == 0) {
      // x of k-tile j through the wave's LDS: written as loaded, 16-byte chunk h of row r at h ^ r (the 16
      // rows' reads of one chunk then hit distinct banks), read back as operand pieces
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const int row = 4 * p + (lane >> 4);
        if (4 * p < M) *reinterpret_cast<v4u*>(&xst[wave][row * 256 + (((lane & 15) ^ row) << 4)]) = xl[p];
      }
      WAVE_LDS_SYNC();
#pragma unroll
      for (int q = 0; q < 4; ++q)
        xv[q] = *reinterpret_cast<const v4u*>(&xst[wave][c * 256 + (((4 * kq + q) ^ c) << 4)]);
      if (j + 1 < KTW) load_x(j + 1);
    }
    const v4u wv = buf[i % D];
    // row groups past the workgroup's share were loaded as zeros (requests keep one fixed order); their
    // conversions and products are skipped (a uniform branch). Every share holds row group 0, and testing
    // it at compile time keeps the compiler from sinking item 0's request into the branch behind a full wait.
    if (g == 0 || g < ng) {
      const float s = fp4_cvt_scale((sdw[g][(kt >> 2) - kgA] >> (8 * (kt & 3))) & 0xffu);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const uint32_t wd = wv[jj];
        v2bf p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, s, 0);
        v2bf p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, s, 1);
        v2bf p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, s, 2);
        v2bf p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, s, 3);
        v8bf a = {p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
        acc[g][jj & 1] =
            __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(v8bf, xv[jj]), acc[g][jj & 1], 0, 0, 0);
      }
    }
    if (i + D < TOT) buf[i % D] = __builtin_amdgcn_raw_buffer_load_b128(wr, woff(i + D), 0, 2);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int g = 0; g < NG; ++g) red[wave][g][lane] = acc[g][0] + acc[g][1];
  __syncthreads();
  for (int g = wave; g < ng; g += 8) {
    v4f s = red[0][g][lane];
#pragma unroll
    for (int v = 1; v < 8; ++v) s += red[v][g][lane];
    const int half = (g0 + g) * 2 + (kq >> 1);
    if (c < M && half >= h0 && half < h1) {
      const int n0 = (g0 + g) * 16 + kq * 4;
      const uint32_t lo = f32_to_bf16_bits(s[0]) | (f32_to_bf16_bits(s[1]) << 16);
      const uint32_t hi = f32_to_bf16_bits(s[2]) | (f32_to_bf16_bits(s[3]) << 16);
      *reinterpret_cast<uint2*>(y + (int64_t)c * N + n0) = make_uint2(lo, hi);
    }
  }
}

#define GEMV_PERSISTENT(KTW)                                                                                   \
  extern "C" __global__ __launch_bounds__(512) void kern_mx_gemv_bf16_p##KTW(                                   \
      const uint16_t* __restrict__ x, const uint8_t* __restrict__ w, const uint8_t* __restrict__ wsf,          \
      uint16_t* __restrict__ y, int M, int N, int K, int hb) {                                                 \
    gemv_persistent<KTW>(x, w, wsf, y, M, N, K, hb);                                                           \
  }
GEMV_PERSISTENT(1)
GEMV_PERSISTENT(2)
GEMV_PERSISTENT(4)
GEMV_PERSISTENT(7)
GEMV_PERSISTENT(8)
#undef GEMV_PERSISTENT

// ------------------------------------- dense MXFP4 x MXFP8 -> bf16 at M <= 64 tokens: the persistent walk
// The tiled GEMM gives a small batch one workgroup per 256 weight rows (36 at N = 9216, which read the
// weights at about 1.2 TB/s). This kernel walks the weights as gemv_persistent does (about 256 workgroups
// of 8 waves, hb <= 9 half groups each, wave w owning k-tiles [w*KTW, (w+1)*KTW) of K = 1024*KTW, k-tile
// by k-tile across the row groups, fragments four ahead) and multiplies them in their fp4 form on the
// block-scaled MFMA against the MXFP8 activations of four 16-token groups. Lane (c, q) of group tg takes
// token 16*tg + c's bytes [16q, 16q + 16) and [64 + 16q, +16) of the k-tile (the 8-bit operand layout of
// V_MFMA_SCALE_F32_16X16X128_F8F6F4) and its k block q's scale byte, both through the wave's LDS: the
// k-tile's rows are requested row-contiguous one k-tile ahead, and the scale bytes of the wave's k groups
// once. Requested straight in operand pieces, each request gathered 16 rows (M = 64, N = 9216: 25.8
// against 17.0 us). Both scale operands arrive shifted to byte 0 (OPSEL 0). The eight partial sums meet
// in LDS one token group at a time; dbg (if not null) receives the f32 sums the bf16 values round.
template <int KTW>
KERN_DEV void gemm_skinny_bf16(const uint8_t* __restrict__ w, const uint8_t* __restrict__ wsf,
                               const uint8_t* __restrict__ xq, const uint8_t* __restrict__ xsf,
                               uint16_t* __restrict__ y, float* __restrict__ dbg, int M, int N, int K, int hb) {
  constexpr int NG = 5, D = 4, TOT = NG * KTW, TG = 4;
  constexpr int NS = (KTW + 6) / 4;  // k groups a wave's k-tiles touch (KTW <= 8: at most three)
  __shared__ v4f red[8][NG][64];
  __shared__ __attribute__((aligned(16))) uint8_t xst[8][8192];      // per wave: one k-tile of 64 token rows
  __shared__ __attribute__((aligned(16))) uint8_t sst[8][NS][1024];  // per wave: 64 rows' 16 scale bytes a k group
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int KT = K >> 7, KG = K >> 9, KB = K >> 5;
  const int H = N >> 3;
  const int h0 = blockIdx.x * hb, h1 = min(h0 + hb, H);
  const int g0 = h0 >> 1, ng = ((h1 + 1) >> 1) - g0;  // row groups touched: [g0, g0 + ng), ng <= NG
  const int c = lane & 15, q = lane >> 4, r = lane & 15;
  const int kt0 = wave * KTW, kgA = kt0 >> 2;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)xq, (short)0, M * K, 0x00020000);
  const __amdgpu_buffer_rsrc_t xsr = __builtin_amdgcn_make_buffer_rsrc((void*)xsf, (short)0, M * KB, 0x00020000);
  // activations are requested row-contiguous: request p of a k-tile loads token rows 8p .. 8p+7, 8 lanes a
  // 128-byte row; they pass through the wave's LDS (16-byte chunk h of row r at h ^ ((r >> 1) & 7)) and are
  // read back as operand pieces. Scale bytes: the wave's NS k groups, one 16-byte request per row each,
  // staged once. Absent tokens and k groups read zeros; requests with no present token are not sent (their
  // LDS rows reach only the MFMA columns of absent tokens, never stored).
  int xo[8];
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const int row = 8 * p + (lane >> 3);
    xo[p] = row < M ? row * K + 128 * kt0 + 16 * (lane & 7) : 0x40000000;
  }
  v4u xl[8];
  auto load_x = [&](int j) {
#pragma unroll
    for (int p = 0; p < 8; ++p)
      if (8 * p < M) xl[p] = __builtin_amdgcn_raw_buffer_load_b128(xr, xo[p] + 128 * j, 0, 0);
  };
  {
    v4u sl[NS];
#pragma unroll
    for (int t = 0; t < NS; ++t)
      sl[t] = __builtin_amdgcn_raw_buffer_load_b128(xsr, (lane < M && kgA + t < KG) ? lane * KB + 16 * (kgA + t)
                                                                                      : 0x40000000, 0, 0);
#pragma unroll
    for (int t = 0; t < NS; ++t) *reinterpret_cast<v4u*>(&sst[wave][t][lane * 16]) = sl[t];
    WAVE_LDS_SYNC();
  }
  load_x(0);
  v4u xa[TG], xb[TG];
  // weight-scale dwords of k groups kgA .. kgA + 2 (KTW <= 8 consecutive k-tiles span at most three groups)
  const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(wsf + (int64_t)g0 * KG * 256), (short)0, ng * KG * 256, 0x00020000);
  uint32_t sdw[NG][NS];
#pragma unroll
  for (int g = 0; g < NG; ++g)
#pragma unroll
    for (int t = 0; t < NS; ++t) {
      const int kg = kgA + t;
      sdw[g][t] = __builtin_amdgcn_raw_buffer_load_b32(
          sr, (g < ng && kg < KG) ? (g * KG + kg) * 256 + lane * 4 : 0x40000000, 0, 2);
    }
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(w + (int64_t)g0 * KT * 1024), (short)0, ng * KT * 1024, 0x00020000);
  // item i = j*NG + g is fragment (g0 + g, kt0 + j); rows outside the owned half groups read zeros
  auto woff = [&](int i) -> int {
    const int g = i % NG, half = (g0 + g) * 2 + (r >> 3);
    return (g < ng && half >= h0 && half < h1) ? (g * KT + kt0 + i / NG) * 1024 + lane * 16 : 0x40000000;
  };
  v4u buf[D];
#pragma unroll
  for (int i = 0; i < D; ++i) {
    if (i < TOT) buf[i] = __builtin_amdgcn_raw_buffer_load_b128(wr, woff(i), 0, 2);
    __builtin_amdgcn_sched_barrier(0);
  }
  v4f acc[NG][TG] = {};
#pragma unroll
  for (int i = 0; i < TOT; ++i) {
    const int g = i % NG, j = i / NG, kt = kt0 + j;
    uint32_t xs[TG];
    if (g == 0) {
#pragma unroll
      for (int p = 0; p < 8; ++p) {
        const int row = 8 * p + (lane >> 3);
        if (8 * p < M) *reinterpret_cast<v4u*>(&xst[wave][row * 128 + (((lane & 7) ^ ((row >> 1) & 7)) << 4)]) = xl[p];
      }
      WAVE_LDS_SYNC();
#pragma unroll
      for (int tg = 0; tg < TG; ++tg) {
        const int row = 16 * tg + c, sw = (row >> 1) & 7;
        xa[tg] = *reinterpret_cast<const v4u*>(&xst[wave][row * 128 + ((q ^ sw) << 4)]);
        xb[tg] = *reinterpret_cast<const v4u*>(&xst[wave][row * 128 + (((q + 4) ^ sw) << 4)]);
      }
      if (j + 1 < KTW) load_x(j + 1);
    }
#pragma unroll
    for (int tg = 0; tg < TG; ++tg)
      xs[tg] = *reinterpret_cast<const uint32_t*>(&sst[wave][(kt >> 2) - kgA][(16 * tg + c) * 16 + 4 * (kt & 3)]);
    const v4u wv = buf[i % D];
    if (g == 0 || g < ng) {
      const int sw = (int)(sdw[g][(kt >> 2) - kgA] >> (8 * (kt & 3)));
      const v8i a = {(int)wv[0], (int)wv[1], (int)wv[2], (int)wv[3], 0, 0, 0, 0};
#pragma unroll
      for (int tg = 0; tg < TG; ++tg) {
        if (16 * tg >= M) break;  // token groups with no token (uniform)
        const v4u lo = xa[tg], hi = xb[tg];
        const v8i b = {(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        const int sx = (int)(xs[tg] >> (8 * q));
        acc[g][tg] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, acc[g][tg], 4, 0, 0, sw, 0, sx);
      }
    }
    if (i + D < TOT) buf[i % D] = __builtin_amdgcn_raw_buffer_load_b128(wr, woff(i + D), 0, 2);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int tg = 0; tg < TG; ++tg) {
    if (16 * tg >= M) break;
#pragma unroll
    for (int g = 0; g < NG; ++g) red[wave][g][lane] = acc[g][tg];
    __syncthreads();
    for (int g = wave; g < ng; g += 8) {
      v4f s = red[0][g][lane];
#pragma unroll
      for (int v = 1; v < 8; ++v) s += red[v][g][lane];
      const int half = (g0 + g) * 2 + (q >> 1), t = 16 * tg + c;
      if (t < M && half >= h0 && half < h1) {
        const int64_t o = (int64_t)t * N + (g0 + g) * 16 + q * 4;
        const uint32_t lo = f32_to_bf16_bits(s[0]) | (f32_to_bf16_bits(s[1]) << 16);
        const uint32_t hi = f32_to_bf16_bits(s[2]) | (f32_to_bf16_bits(s[3]) << 16);
        *reinterpret_cast<uint2*>(y + o) = make_uint2(lo, hi);
        if (dbg) *reinterpret_cast<v4f*>(dbg + o) = s;
      }
    }
    __syncthreads();
  }
}

#define GEMM_SKINNY(KTW)                                                                                       \
  extern "C" __global__ __launch_bounds__(512) void kern_mx_gemm_bf16_s##KTW(                                   \
      const uint8_t* __restrict__ w, const uint8_t* __restrict__ wsf, const uint8_t* __restrict__ xq,          \
      const uint8_t* __restrict__ xsf, uint16_t* __restrict__ y, float* __restrict__ dbg, int M, int N, int K, \
      int hb) {                                                                                                \
    gemm_skinny_bf16<KTW>(w, wsf, xq, xsf, y, dbg, M, N, K, hb);                                               \
  }
GEMM_SKINNY(1)
GEMM_SKINNY(2)
GEMM_SKINNY(4)
GEMM_SKINNY(7)
GEMM_SKINNY(8)
#undef GEMM_SKINNY

// ====================================================================================== block-scaled GEMM
// One workgroup computes a 128-row (token/slot) x 256-row (weight) tile with 8 waves (two per SIMD) in a
// 2x4 grid; each wave owns 64 x 64 = 4 x 4 tiles of V_MFMA_SCALE_F32_16X16X128_F8F6F4 (A = fp4 weights,
// B = e4m3 activations, e8m0 scales in-instruction). K advances in 128-wide k-tiles through a four-stage
// LDS ring filled by direct global->LDS loads (GLOBAL_LOAD_LDS_DWORDX4), up to four tiles ahead of the
// MFMAs. Each k-step multiplies half of its tile, meets the other waves at the step's one barrier,
// refills the stage it has just finished reading, reads the next tile's operands and multiplies the
// other half while those reads land; the second wave of each SIMD fills the first one's stalls.
//   W stage: 16 fragments of 1 KiB, copied verbatim (the repacked layout is the MFMA operand layout);
//   X stage: 128 rows x 128 B, 16-byte chunk j of row t stored at t*128 + ((j ^ ((t>>1)&7)) << 4) so that
//      the fragment reads (16 rows, one chunk each) touch distinct bank groups; the permutation is
//      applied on the global side, each lane fetching the chunk that belongs at its LDS position;
//   scales once per 512 of K (two slots): W fragments verbatim, X as dwords [k-tile][row].
enum { MODE_FC2 = 0, MODE_FC1 = 1, MODE_PT = 2, MODE_DENSE_BF16 = 3 };
// MoE slots with at most this many rows take the skinny path (one 16-row token subtile). FC2's weight rows
// are short (K = intermediate size), and there the ring already wins from 9 rows on.
template <int MODE>
constexpr int skinny_rows() { return MODE == MODE_FC1 ? 16 : 8; }

struct BmmArgs {
  const uint8_t* a;      // repacked weights [E][m][k/2]
  const uint8_t* sf_a;   // repacked scales
  const uint8_t* b;      // e4m3 activations
  const uint8_t* sf_b;   // activation scales
  void* c;               // output
  uint8_t* sf_c;         // FC1 output scales (R128c4)
  const int* route_map;  // FC1 gather
  const float* alpha;
  const float* beta;
  const int* num_non_exiting;
  const int* cta_batch;
  const int* cta_limit;
  const float* d_scale;  // PT
  float* dbg;            // optional f32 debug output
  int m, k, rows;        // rows: dense M
  int max_slots;         // MoE: capacity of the slot tables (cta_batch / cta_limit entries)
  int sf_b_r128c4;
};

#define BT 128
#define BN 256
#define LDS_W (BN * 64)
#define LDS_X (BT * 128)
#define LDS_SW (16 * 256)
#define LDS_SX (4 * BT * 4)


// 16 bytes per lane from global memory straight into LDS at `lds_wave_base + 16 * lane` (wave-uniform base),
// GLOBAL_LOAD_LDS_DWORDX4 with the LDS address in M0. Written as inline assembly so that the compiler does
// not track these loads into LDS: every read of the ring waits for them explicitly (WAIT_VMCNT with the
// count of requests sent since, then a barrier), and the compiler's own alias tracking could not tell the
// ring's slots apart and added waits for every load in flight. M0 holds nothing else in the kernels that use
// these (no other instruction there reads it).
// The LDS address of a generic pointer into LDS is its low 32 bits (the shared aperture sits in the high
// half): taken that way, with no address-space cast, and so no null check on each request.
KERN_DEV uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)p; }
// The requests take a wave-uniform base in an SGPR pair and a per-lane 32-bit byte offset (the instructions'
// SADDR form): the per-lane address needs no 64-bit add per request, and a k step moves the base once for all
// of a wave's requests into that buffer. dma16s moves 16 bytes per lane, dma4s 4 bytes per lane (to
// `lds_wave_base + 4 * lane`).
KERN_DEV uint64_t uniform_ptr(const void* p) {
  const uint64_t b = (uint64_t)(uintptr_t)p;
  // readfirstlane returns an int: each half goes through uint32_t, so the low half is not sign-extended
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
  return ((uint64_t)hi << 32) | (uint64_t)lo;
}
KERN_DEV void dma16s(const void* base, uint32_t voff, void* lds_wave_base) {
  const uint32_t lds = __builtin_amdgcn_readfirstlane(lds_addr(lds_wave_base));
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(uniform_ptr(base)),
               "s"(lds)
               : "memory", "m0");
}
KERN_DEV void dma4s(const void* base, uint32_t voff, void* lds_wave_base) {
  const uint32_t lds = __builtin_amdgcn_readfirstlane(lds_addr(lds_wave_base));
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(uniform_ptr(base)),
               "s"(lds)
               : "memory", "m0");
}

// The LDS ring: four tile stages of each operand, two scale slots of each kind.
struct BmmLds {
  uint8_t* w[4];
  uint8_t* x[4];
  uint8_t* sw;   // two weight-scale slots of LDS_SW bytes (one k group each)
  uint8_t* sx;   // two activation-scale slots of LDS_SX bytes
  uint8_t* stg;  // 2 KiB per wave, outside the ring: the epilogue's staging
};

// The tile's epilogue (every mode): lane (c, g) of accumulator (ts, rs) of wave (wt, wn) holds weight
// rows nx*BN + wn*64 + 16*rs + 4*g + i for tile row wt*64 + 16*ts + c; rows at or past `valid` are not
// stored.
// STAGED (the LDS ring's tiles): each wave writes its output rows into its own 2 KiB of LDS (`stg`, outside
// the ring, so that the next tile's first requests can land in the ring meanwhile), then stores them back
// row by row, 16 bytes a lane, so that each store instruction covers whole row segments (128 B a row for
// bf16, 64 for e4m3, 32 for FC1's e4m3 half): written straight from the accumulators, every store
// instruction touches 16 rows with 32 bytes (or fewer) each, and at K3's full 128-row slots those scattered
// pieces took 3-6 us per tile, as long as a fifth of the k-loop. The staged stores are buffer stores whose
// range ends at the tile's last live row, so that rows past it are dropped by the hardware rather than
// branched around: every wave sends the same number of stores per tile (epi_stores), and the next tile's
// first wait can count them.
template <int MODE>
constexpr int epi_stores() { return MODE == MODE_FC1 ? 2 + 4 : (MODE == MODE_PT ? 4 : 8); }
template <int MODE, bool STAGED>
KERN_DEV void bmm_epilogue(const BmmArgs& A, const v4f (&acc)[4][4], int wt, int wn, int nx, int row0, int valid,
                           int expert, int lane, uint8_t* stg = nullptr) {
  const int m = A.m;
  const int c = lane & 15, g = lane >> 4;
  const int wrow0 = nx * BN + wn * 64;  // first weight row of this wave
  if (MODE == MODE_FC2 || MODE == MODE_DENSE_BF16) {
    uint16_t* C = reinterpret_cast<uint16_t*>(A.c);
    if (A.dbg) {
#pragma unroll
      for (int ts = 0; ts < 4; ++ts) {
        const int t = wt * 64 + ts * 16 + c;
        if (t < valid) {
#pragma unroll
          for (int rs = 0; rs < 4; ++rs)
            *reinterpret_cast<v4f*>(A.dbg + (int64_t)(row0 + t) * m + wrow0 + rs * 16 + g * 4) = acc[ts][rs];
        }
      }
    }
    if (STAGED) {
      // one 16-row subtile at a time: row r (128 B, 64 bf16) at r * 128, 16-byte unit k at ((k ^ (r & 7)) << 4),
      // the unit's two 8-byte halves swapped in rows 8..15, so that the 16 lanes of each g write 16 distinct
      // bank pairs (rows r and r + 8 would otherwise share them)
      const int rr = lane >> 3, k = lane & 7;
      const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(C + (int64_t)row0 * m), (short)0, max(valid, 0) * m * 2, 0x00020000);
#pragma unroll
      for (int ts = 0; ts < 4; ++ts) {
#pragma unroll
        for (int rs = 0; rs < 4; ++rs) {
          const v4f v = acc[ts][rs];
          const int kw = 2 * rs + (g >> 1);
          *reinterpret_cast<uint2*>(stg + c * 128 + ((kw ^ (c & 7)) << 4) + 8 * ((g & 1) ^ (c >> 3))) =
              make_uint2(bf16x2_hw(v[0], v[1]), bf16x2_hw(v[2], v[3]));
        }
        WAVE_LDS_SYNC();
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int r = 8 * h + rr;
          v4u d = *reinterpret_cast<const v4u*>(stg + r * 128 + ((k ^ (r & 7)) << 4));
          if (h) d = d.zwxy;
          const int t = wt * 64 + 16 * ts + r;
          // FC2's rows are read again only by the finalize's gather: non-temporal stores (config 4: FC2 363 ->
          // 359 us); the dense GEMM's output keeps the default policy
          __builtin_amdgcn_raw_buffer_store_b128(d, cr, (t * m + wrow0 + 8 * k) * 2, 0, MODE == MODE_FC2 ? 2 : 0);
        }
      }
    } else {
#pragma unroll
      for (int ts = 0; ts < 4; ++ts) {
        const int t = wt * 64 + ts * 16 + c;
        if (t < valid) {
          const int64_t p = row0 + t;
#pragma unroll
          for (int rs = 0; rs < 4; ++rs) {
            const int n = wrow0 + rs * 16 + g * 4;
            const v4f v = acc[ts][rs];
            *reinterpret_cast<uint2*>(C + p * m + n) = make_uint2(bf16x2_hw(v[0], v[1]), bf16x2_hw(v[2], v[3]));
          }
        }
      }
    }
  } else if (MODE == MODE_PT) {
    uint8_t* C = reinterpret_cast<uint8_t*>(A.c);
    const float ds = A.d_scale[0];
    if (A.dbg) {
#pragma unroll
      for (int ts = 0; ts < 4; ++ts) {
        const int t = wt * 64 + ts * 16 + c;
        if (t < valid) {
#pragma unroll
          for (int rs = 0; rs < 4; ++rs)
            *reinterpret_cast<v4f*>(A.dbg + (int64_t)(row0 + t) * m + wrow0 + rs * 16 + g * 4) = acc[ts][rs];
        }
      }
    }
    if (STAGED) {
      // two 16-row subtiles at a time, subtile ts at (ts & 1) * 1024: row r (64 B, 64 e4m3) at r * 64, 16-byte
      // unit k at ((k ^ ((r >> 1) & 3)) << 4), the unit's two 8-byte halves swapped in rows 8..15: the 32 lanes
      // of each half-wave then write 32 distinct banks
      const int rr = lane >> 2, k = lane & 3;
      const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(C + (int64_t)row0 * m), (short)0, max(valid, 0) * m, 0x00020000);
#pragma unroll
      for (int q = 0; q < 2; ++q) {
#pragma unroll
        for (int ts = 2 * q; ts < 2 * q + 2; ++ts) {
#pragma unroll
          for (int rs = 0; rs < 4; ++rs) {
            const v4f v = acc[ts][rs];
            *reinterpret_cast<uint32_t*>(stg + (ts & 1) * 1024 + c * 64 + ((rs ^ ((c >> 1) & 3)) << 4) +
                                         4 * (g ^ ((c >> 2) & 2))) =
                e4m3_hw2(v[0] * ds, v[1] * ds) | (e4m3_hw2(v[2] * ds, v[3] * ds) << 16);
          }
        }
        WAVE_LDS_SYNC();
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          v4u d = *reinterpret_cast<const v4u*>(stg + j * 1024 + rr * 64 + ((k ^ ((rr >> 1) & 3)) << 4));
          if (rr >= 8) d = d.zwxy;
          const int t = wt * 64 + 16 * (2 * q + j) + rr;
          __builtin_amdgcn_raw_buffer_store_b128(d, cr, t * m + wrow0 + 16 * k, 0, 0);
        }
      }
    } else {
#pragma unroll
      for (int ts = 0; ts < 4; ++ts) {
        const int t = wt * 64 + ts * 16 + c;
        if (t < valid) {
          const int64_t p = row0 + t;
#pragma unroll
          for (int rs = 0; rs < 4; ++rs) {
            const int n = wrow0 + rs * 16 + g * 4;
            const v4f v = acc[ts][rs];
            const uint32_t o = e4m3_hw2(v[0] * ds, v[1] * ds) | (e4m3_hw2(v[2] * ds, v[3] * ds) << 16);
            *reinterpret_cast<uint32_t*>(C + p * m + n) = o;
          }
        }
      }
    }
  } else {  // MODE_FC1: gated SiTU-GLU, e4m3 + ue8m0 block-32 (R128c4) output
    uint8_t* C = reinterpret_cast<uint8_t*>(A.c);
    const int half = m >> 1;
    const float al = A.alpha[expert], be = A.beta[expert];
    const SituCoef G = situ_coef(al), U = situ_coef(be);  // SiTU's per-expert coefficient sets
    // the wave's 64 interleaved gate/up rows give 32 output columns: one MXFP8 block
    const int ncol0 = (nx * BN + wn * 64) >> 1;
    const int blk = ncol0 >> 5;
    // sf_c: R128c4 over the tables' max_slots * 128 rows
    const __amdgpu_buffer_rsrc_t sfr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)A.sf_c, (short)0, A.max_slots * ((((half >> 5) + 3) >> 2) * 512), 0x00020000);
    // a ring tile's row0 is its slot's first row, a multiple of 128: row p = row0 + t has p >> 7 = row0 >> 7
    // and p & 127 = t, so its R128c4 byte is at sf_base + (t & 31) * 16 + (t >> 5) * 4
    const int sf_base = 512 * ((row0 >> 7) * ((((half >> 5) + 3) >> 2)) + (blk >> 2)) + (blk & 3);
#pragma unroll
    for (int ts = 0; ts < 4; ++ts) {
      const int t = wt * 64 + ts * 16 + c;
      const bool ok = t < valid;
      const int64_t p = row0 + t;
      uint32_t sc = 0;
      // a 16-row subtile with no live row (a wave-uniform test) needs no SiTU and no codes: its staging rows
      // are past the tile's live ones, which are never stored, and its sf_c store below is dropped
      if (wt * 64 + ts * 16 < valid) {
        // h for 4 subtiles x 2 columns; columns ncol0 + 8*rs + 2*g + {0,1}
        float h[4][2];
#pragma unroll
        for (int rs = 0; rs < 4; ++rs) {
          const v4f v = acc[ts][rs];
#pragma unroll
          for (int i = 0; i < 2; ++i) h[rs][i] = situ_fast(v[i], v[i + 2], G, U);
        }
        if (ok && A.dbg) {
#pragma unroll
          for (int rs = 0; rs < 4; ++rs)
#pragma unroll
            for (int i = 0; i < 2; ++i) {
              const int n = ncol0 + 8 * rs + 2 * g + i;
              A.dbg[(p * 3 + 0) * half + n] = acc[ts][rs][i];
              A.dbg[(p * 3 + 1) * half + n] = acc[ts][rs][i + 2];
              A.dbg[(p * 3 + 2) * half + n] = h[rs][i];
            }
        }
        // the largest |h| of the lane (IEEE maximum of magnitudes: NaN-propagating, and for other values the
        // same bits as the largest |bits|), then of the block
        float fm = __builtin_fabsf(h[0][0]);
#pragma unroll
        for (int rs = 0; rs < 4; ++rs)
#pragma unroll
          for (int i = 0; i < 2; ++i) fm = __builtin_elementwise_maximum(fm, __builtin_fabsf(h[rs][i]));
        sc = mx_scale_code(max_over_rows(__float_as_uint(fm)));
        uint32_t o[4];
        mx_code2x4(h, sc, o);
        if (STAGED) {
          // wave row r (32 B: the wave's MXFP8 block of the row) at r * 32
          uint8_t* pc = stg + (16 * ts + c) * 32 + 2 * g;
#pragma unroll
          for (int rs = 0; rs < 4; ++rs) *reinterpret_cast<uint16_t*>(pc + 8 * rs) = (uint16_t)o[rs];
        } else if (ok) {
#pragma unroll
          for (int rs = 0; rs < 4; ++rs)
            *reinterpret_cast<uint16_t*>(C + p * half + ncol0 + 8 * rs + 2 * g) = (uint16_t)o[rs];
          if (g == 0) {
            const int64_t kb4 = ((half >> 5) + 3) >> 2;
            const int64_t off =
                512 * ((p >> 7) * kb4 + (blk >> 2)) + (p & 31) * 16 + ((p & 127) >> 5) * 4 + (blk & 3);
            A.sf_c[off] = (uint8_t)sc;
          }
        }
      }
      if (STAGED) {
        // one byte store per subtile from every lane, the lanes other than g = 0 and the rows past the
        // tile's live ones pointed past the end of sf_c (dropped)
        const int off = sf_base + (t & 31) * 16 + (t >> 5) * 4;
        __builtin_amdgcn_raw_buffer_store_b8((uint8_t)sc, sfr, ok && g == 0 ? off : 0x7fffff00, 0, 0);
      }
    }
    if (STAGED) {
      WAVE_LDS_SYNC();
      const int rr = lane >> 1, k = lane & 1;
      const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(C + (int64_t)row0 * half), (short)0, max(valid, 0) * half, 0x00020000);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const v4u d = *reinterpret_cast<const v4u*>(stg + (32 * j + rr) * 32 + 16 * k);
        const int t = wt * 64 + 32 * j + rr;
        __builtin_amdgcn_raw_buffer_store_b128(d, cr, t * half + ncol0 + 16 * k, 0, 0);
      }
    }
  }
}

// The hardware hands workgroups to the 8 XCDs round robin (workgroup lin = x + gridDim.x * y to XCD
// lin % 8), each XCD with its own L2.
// Dense grids (every tile live): workgroup -> (weight tile nx of gx, 128-row block), re-linearized so that
// each XCD takes a contiguous run of tiles.
KERN_DEV void tile_of(int gx, int& nx, int& slot) {
  const int total = gridDim.x * gridDim.y;
  int lin = blockIdx.x + gridDim.x * blockIdx.y;
  if ((total & 7) == 0) lin = (lin & 7) * (total >> 3) + (lin >> 3);
  nx = lin % gx;
  slot = lin / gx;
}
// MoE tile i of workgroup `owner` -> (weight tile nx of gx, slot) among the S live slots. The workgroup
// runs on XCD x = owner % 8 (the hardware deals workgroups to the XCDs round robin; G is a multiple of 8),
// as CU c = owner / 8 of the XCD's G/8. XCD x takes the contiguous slots [S*x/8, S*(x+1)/8), so that the
// slots of one expert (consecutive in the tables) share one L2 and its weights stream from HBM about once,
// not once per XCD (dealing slot s to XCD s % 8 spread a prefill expert's ~10 slots over all eight L2s).
// The XCD's CUs walk its tiles in order li = c + (G/8) i, grouped MOE_BS slots at a time; within a group,
// MOE_BW weight tiles at a time, slot by slot: the G/8 tiles the XCD runs at once share MOE_BS activation
// tiles and MOE_BW weight tiles through its L2. False when the workgroup has no tile i (li is past the
// XCD's tiles, and so is every later i).
#ifndef MOE_BS
#define MOE_BS 2
#endif
#ifndef MOE_BW
#define MOE_BW 16
#endif
KERN_DEV bool moe_tile(int owner, int i, int S, int gx, int G, int& nx, int& slot) {
  const int x = owner & 7, per = G >> 3;
  const int s0 = (S * x) >> 3, ns = ((S * (x + 1)) >> 3) - s0;
  const int li = (owner >> 3) + per * i;
  if (li >= ns * gx) return false;
  const int grp = li / (MOE_BS * gx), t = li - grp * (MOE_BS * gx);
  const int bs = min(MOE_BS, ns - grp * MOE_BS);  // slots of this group (the last may have fewer)
  const int full = gx / MOE_BW;                   // whole blocks of MOE_BW weight tiles
  int nb, r, w;
  if (t < full * bs * MOE_BW) {
    nb = t / (bs * MOE_BW), r = t - nb * (bs * MOE_BW), w = MOE_BW;
  } else {
    nb = full, r = t - full * bs * MOE_BW, w = gx - full * MOE_BW;
  }
  slot = s0 + grp * MOE_BS + r / w;
  nx = nb * MOE_BW + r % w;
  return true;
}

// One 128-row (slot or token block) x 256-row (weights) tile on the LDS ring: ring_tile (where its requests
// read from), ring_prologue (a first tile's first requests) and ring_kloop (the multiplies).
// Two wave groups take turns (ping-pong): group 0 (waves 0-3, token rows 0-63) brings in the weight tiles,
// group 1 (waves 4-7, rows 64-127) the activation tiles; waves w and w+4 share a SIMD. Every k-tile t has two
// half-steps separated by workgroup barriers: in the first, group 0 multiplies tile t while group 1 requests
// activations three tiles ahead and reads tile t's operands; in the second, group 1 multiplies tile t while
// group 0 requests weights four tiles ahead and reads tile t+1's operands. Each SIMD's matrix core thus
// always has one wave's MFMAs queued while the other wave's loads are in flight.
// Chaining: in a persistent workgroup the requests that run past a tile's last k-tile are the next tile's
// first ones (its k-tiles 0..3 of weights, 0..2 of activations, and the scales of its first k group), sent
// during the last four k-steps exactly as in the middle of a tile, so that the next tile starts with its
// first k-tiles landed: no separate first requests, nothing re-read. Every wave fills only its own pieces of
// the ring (group 0 wave gw the weight fragments gw + 4r and their scale rows, group 1 wave gw the activation
// blocks gw + 4r and scale rows 4h + gw), and one wave's requests land in the order it sends them.
struct RingTile {
  const uint8_t* wbase;  // weight fragment 0, k-tile 0 of the tile (uniform)
  const uint8_t* sbase;  // its scale dwords (uniform)
  int xtok[4];           // group 1: activation row (token) of request r (this lane's row)
  int stok[2];           // group 1: activation row of scale request h
  int nx, expert, row0, valid;
};

// live 32-row activation blocks of a tile (group 1's requests per k-tile)
KERN_DEV int ring_nxr(int valid) { return min(4, max(1, (valid + 31) >> 5)); }

template <int MODE>
KERN_DEV RingTile ring_tile(const BmmArgs& A, int nx, int expert, int row0, int valid) {
  // the wave index through readfirstlane (uniform); the thread index through an opaque copy, so that the
  // lane-only values are derived anew for each tile (hoisted out of the persistent loop they stayed live
  // across tiles, were spilled, and were reloaded behind full memory waits in every tile)
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int lane = tid & 63, gw = __builtin_amdgcn_readfirstlane(tid >> 6) & 3;
  const int K = A.k, KT = K >> 7, KG = K >> 9, m = A.m;
  RingTile T;
  T.nx = nx, T.expert = expert, T.row0 = row0, T.valid = valid;
  const int rg0 = (nx * BN) >> 4;  // first 16-row group of this tile
  T.wbase = A.a + (int64_t)expert * m * (K >> 1) + ((int64_t)rg0 * KT) * 1024;
  T.sbase = A.sf_a + (int64_t)expert * m * (K >> 5) + ((int64_t)rg0 * KG) * 256;
  // token (activation row) of tile row t; rows past the slot's last valid row read row/token 0 (their
  // accumulators are never stored)
  // (FC1: the route_map entry is read for every row, live or not, in bounds as the tables hold max_slots *
  // 128 rows: a fixed number of loads, which the next k-loop's first wait counts)
  auto token_of = [&](int t) -> int {
    const int v = MODE == MODE_FC1 ? A.route_map[row0 + t] : row0 + t;
    return t >= valid ? 0 : v;
  };
#pragma unroll
  for (int r = 0; r < 4; ++r) T.xtok[r] = token_of(32 * r + 8 * gw + (lane >> 3));
#pragma unroll
  for (int h = 0; h < 2; ++h) T.stok[h] = token_of(16 * (4 * h + gw) + (lane >> 2));
  return T;
}

// Requests (lane: this thread's lane, from the caller's opaque copy of the thread index).
// Group 0: weight tile kt (4 requests), weight-scale group kg (4). Group 1: activation tile kt (NXR requests,
// the 32-row blocks that hold live rows) and activation-scale group kg (NXS: the live 64-row halves); LDS
// rows of blocks not requested keep stale data that no wave reads (a wave reads the rows of its live 16-row
// subtiles only), so a ring of 17-32-row slots issues 5 requests per k-tile instead of 8.
KERN_DEV void ring_req_w(const RingTile& T, int KT, int gw, int lane, int kt, uint8_t* sW) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int f = r * 4 + gw;  // fragment (16-row group) 0..15
    dma16s(T.wbase + (int64_t)kt * 1024, (uint32_t)(f * KT * 1024 + lane * 16), sW + f * 1024);
  }
}
KERN_DEV void ring_req_ws(const RingTile& T, int KG, int gw, int lane, int kg, uint8_t* sSW) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int f = r * 4 + gw;
    dma4s(T.sbase + (int64_t)kg * 256, (uint32_t)(f * KG * 256 + lane * 4), sSW + f * 256);
  }
}
// Activation requests read through per-tile sources: xs[r], this lane's 16 bytes of request r at k-tile 0,
// and sxs[h], its scale dword of request h at k group 0 (ring_xsrc). Request r fills LDS rows
// 32r + 8*gw + lane/8, 16-byte position lane%8, with chunk (lane%8) ^ ((row/2)%8) of the row's k-tile (the X
// stage's swizzle). Scale dwords of a k group are gathered into LDS as [tile row][k-tile of the group] (16
// bytes a row): request h fills rows 16*(4h + gw) + lane/4, k-tile lane % 4, so that the multiplying waves
// read a row's four k-tiles in one 16-byte read per group (a k-tile's scale dword holds the row's four
// 32-wide k blocks). Scale rows: linear [T][K/32], or R128c4 (one 512-byte tile per 128 rows x 4 k blocks).
struct RingXSrc {
  const uint8_t* xb;   // the activations (uniform)
  const uint8_t* sxb;  // their scales (uniform)
  uint32_t xs[4];      // byte offsets from xb and sxb (the activation buffers stay below 4 GiB)
  uint32_t sxs[2];
};
KERN_DEV RingXSrc ring_xsrc(const BmmArgs& A, const RingTile& T, int gw, int lane) {
  RingXSrc S;
  const int K = A.k;
  S.xb = A.b, S.sxb = A.sf_b;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = 32 * r + 8 * gw + (lane >> 3);
    S.xs[r] = (uint32_t)T.xtok[r] * (uint32_t)K + (((lane & 7) ^ ((t >> 1) & 7)) << 4);
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t srow = (uint32_t)T.stok[h];
    S.sxs[h] = A.sf_b_r128c4 ? 512u * ((srow >> 7) * (uint32_t)(K >> 7) + (lane & 3)) + (srow & 31) * 16 +
                                   ((srow & 127) >> 5) * 4
                             : srow * (uint32_t)(K >> 5) + (lane & 3) * 4;
  }
  return S;
}
template <int NXR>
KERN_DEV void ring_req_x(const RingXSrc& S, int gw, int kt, uint8_t* sX) {
#pragma unroll
  for (int r = 0; r < NXR; ++r) dma16s(S.xb + (int64_t)kt * 128, S.xs[r], sX + (r * 4 + gw) * 1024);
}
// k group kg of the scale rows: 4 k-tiles on, 16 bytes (linear) or four 512-byte tiles (R128c4)
template <int NXR>
KERN_DEV void ring_req_xs(const BmmArgs& A, const RingXSrc& S, int gw, int kg, uint8_t* sSX) {
  constexpr int NXS = NXR > 2 ? 2 : 1;
  const int64_t step = A.sf_b_r128c4 ? 2048 : 16;
#pragma unroll
  for (int h = 0; h < NXS; ++h) dma4s(S.sxb + kg * step, S.sxs[h], sSX + 256 * (4 * h + gw));
}

// A first tile's first requests (a tile no earlier tile chained to): group 0 the weight scales of k group 0
// and weight tiles 0..3, group 1 the activation scales and activation tiles 0..2, as the last k-steps of a
// chained tile send them. Nothing waits here: ring_kloop does. Every wave has passed the previous tile's last
// barrier (or there is none).
template <int MODE>
KERN_DEV void ring_prologue(const BmmArgs& A, const BmmLds& L, const RingTile& T) {
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), gw = wave & 3;
  const int K = A.k, KT = K >> 7, KG = K >> 9;
  if (wave < 4) {
    ring_req_ws(T, KG, gw, lane, 0, L.sw);
    ring_req_w(T, KT, gw, lane, 0, L.w[0]);
    ring_req_w(T, KT, gw, lane, 1, L.w[1]);
    ring_req_w(T, KT, gw, lane, 2, L.w[2]);
    ring_req_w(T, KT, gw, lane, 3, L.w[3]);
  } else {
    const RingXSrc S = ring_xsrc(A, T, gw, lane);
    auto go = [&](auto NXRc) {
      constexpr int NXR = decltype(NXRc)::value;
      ring_req_xs<NXR>(A, S, gw, 0, L.sx);
      ring_req_x<NXR>(S, gw, 0, L.x[0]);
      ring_req_x<NXR>(S, gw, 1, L.x[1]);
      ring_req_x<NXR>(S, gw, 2, L.x[2]);
    };
    switch (ring_nxr(T.valid)) {
      case 1: go(IC<1>{}); break;
      case 2: go(IC<2>{}); break;
      case 3: go(IC<3>{}); break;
      default: go(IC<4>{}); break;
    }
  }
}

// The tile's multiplies: acc = this wave's 64 x 64 block. The tile's first requests are out (ring_prologue,
// or the tile before chained to it, sending all four activation blocks and both scale halves). K group g's
// scales live in slot g % 2. The last four k-steps send Tn's first requests, with Tn's k group 0 scales into
// slot 0 as well: with an odd number of k groups that is the slot of T's last group, whose scales every wave
// has read into registers by then (group 0 at the k-step before the group, group 1 at its first). Without
// `chain` (Tn is T) they re-read T's last k-tile and scale group instead, so that the counts, and the waits,
// are the same. Ends with every wave past the tile's last barrier (no wave reads the ring after it); the
// last requests may still be in flight.
// first: no epilogue ran since the tile's first requests (ring_prologue); otherwise the tile before's
// epilogue stores (epi_stores) and, in FC1, Tn's route_map loads (ring_tile: 6) were sent after them.
template <int MODE>
KERN_DEV void ring_kloop(const BmmArgs& A, const BmmLds& L, const RingTile& T, const RingTile& Tn, bool chain,
                         bool first, v4f (&acc)[4][4]) {
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wt = wave >> 2, wn = wave & 3;  // token half, weight quarter
  const int grp = wt, gw = wn;
  const int K = A.k, KT = K >> 7, KG = K >> 9;
  const int valid = T.valid;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};

  // number of live 16-row token subtiles for this wave
  const int live_ts = min(4, max(0, (valid - wt * 64 + 15) >> 4));
  const int c = lane & 15, g = lane >> 4;
  const RingXSrc S = ring_xsrc(A, T, gw, lane);
  // past T's last k group: Tn's k group 0, or T's last again
  const int wn_kg = chain ? 0 : KG - 1;
  // the scale slots of k group kg
  auto sw_slot = [&](int kg) -> uint8_t* { return L.sw + (kg & 1) * LDS_SW; };
  auto sx_slot = [&](int kg) -> uint8_t* { return L.sx + (kg & 1) * LDS_SX; };

  auto run = [&](auto NTSc, auto NXRc) {
    constexpr int NTS = decltype(NTSc)::value;  // live token subtiles of this wave (uniform)
    constexpr int NXR = decltype(NXRc)::value;  // live 32-row activation blocks (group 1's requests)
    constexpr int NXS = NXR > 2 ? 2 : 1;        // activation-scale requests per k group
    // k-tile 0 and the scales of k group 0 have landed once only tiles 1..3 (1..2 for activations; 4
    // requests each when chained, NXR after ring_prologue) and whatever this wave sent after them are
    // outstanding: Tn's route_map loads (FC1) and, unless first, the tile before's epilogue stores
    constexpr int R = MODE == MODE_FC1 ? 6 : 0, ST = epi_stores<MODE>();
    if (grp == 0) {
      if (first)
        WAIT_VMCNT(12 + R);
      else
        WAIT_VMCNT(12 + R + ST);
    } else {
      if (first)
        WAIT_VMCNT(2 * NXR + R);
      else
        WAIT_VMCNT(8 + R + ST);
    }
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    v4i wa[4];         // W operands of the tile in hand
    v8i xb[4];         // X operands, per token subtile
    v4u sxq[4];        // X scale dwords of the current k group (k-tile j in sxq[ts][j])
    uint32_t swd[4];   // weight-scale dwords of the current k group
    // operands of the tile in stage st (k-tile jt of its group; weight scales too when jt == 0)
    auto read_tile = [&](const uint8_t* sW, const uint8_t* sX, const uint8_t* sSW, const uint8_t* sSX, int jt,
                         bool with_sw) {
#pragma unroll
      for (int rs = 0; rs < 4; ++rs) wa[rs] = *reinterpret_cast<const v4i*>(sW + (wn * 4 + rs) * 1024 + lane * 16);
      if (with_sw) {
#pragma unroll
        for (int rs = 0; rs < 4; ++rs) swd[rs] = reinterpret_cast<const uint32_t*>(sSW + (wn * 4 + rs) * 256)[lane];
      }
#pragma unroll
      for (int ts = 0; ts < NTS; ++ts) {
        const int t = wt * 64 + ts * 16 + c;
        const uint8_t* xr = sX + t * 128;
        const int sw = (t >> 1) & 7;
        const v4i x0 = *reinterpret_cast<const v4i*>(xr + ((g ^ sw) << 4));
        const v4i x1 = *reinterpret_cast<const v4i*>(xr + (((g + 4) ^ sw) << 4));
        xb[ts] = (v8i){x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
        // the row's scale dwords for the group's four k-tiles, at its first
        if (jt == 0) sxq[ts] = *reinterpret_cast<const v4u*>(sSX + t * 16);
      }
    };
    auto mfmas = [&](auto Jt) {
      constexpr int jt = decltype(Jt)::value;  // k-tile within the group: scale byte of the weights
#pragma unroll
      for (int ts = 0; ts < NTS; ++ts) {
        const uint32_t sxb = sxq[ts][jt] >> (8 * g);  // this lane's k block's byte, in byte 0
#pragma unroll
        for (int rs = 0; rs < 4; ++rs) {
          const v8i wb = {wa[rs][0], wa[rs][1], wa[rs][2], wa[rs][3], 0, 0, 0, 0};
          acc[ts][rs] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wb, xb[ts], acc[ts][rs], 4, 0, jt,
                                                                          (int)swd[rs], 0, (int)sxb);
        }
      }
    };
    // k-tile kt (= 4 kg + jt) lives in stage jt, its k group's scales in slot kg % 2. LAST: the tile's last
    // k group, whose requests four (three) k-tiles ahead are past the end.
    auto step0 = [&](int kt, auto Jc, auto LASTc) {  // group 0
      constexpr int jt = decltype(Jc)::value;
      constexpr bool LAST = decltype(LASTc)::value;
      const int kg = kt >> 2;
      // first half-step: multiply tile kt (operands read in the previous half-step)
      mfmas(IC<jt>{});
      __builtin_amdgcn_sched_barrier(0);
      // this wave's weights of tile kt+1 have landed once only the requests sent after them are
      // outstanding: tiles kt+2, kt+3 (4 each) and, for jt = 1, 2, the next group's scales (4). At the last
      // k-tile there is nothing left to read.
      if (!LAST || jt < 3) WAIT_VMCNT(8 + ((jt == 1 || jt == 2) ? 4 : 0));
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      // second half-step: stage jt is read by both groups; refill it with weight tile kt+4 (the next
      // group's weight scales first), then read tile kt+1
      if (!LAST) {
        if (jt == 0) ring_req_ws(T, KG, gw, lane, kg + 1, sw_slot(kg + 1));
        ring_req_w(T, KT, gw, lane, kt + 4, L.w[jt]);
      } else {
        if (jt == 0) ring_req_ws(Tn, KG, gw, lane, wn_kg, L.sw);
        ring_req_w(Tn, KT, gw, lane, chain ? jt : KT - 1, L.w[jt]);
      }
      if (!LAST || jt < 3)
        read_tile(L.w[(jt + 1) & 3], L.x[(jt + 1) & 3], sw_slot((kt + 1) >> 2), sx_slot((kt + 1) >> 2), (jt + 1) & 3,
                  jt == 3);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
    };
    auto step1 = [&](int kt, auto Jc, auto LASTc) {  // group 1
      constexpr int jt = decltype(Jc)::value;
      constexpr bool LAST = decltype(LASTc)::value;
      const int kg = kt >> 2;
      // first half-step: activation tile kt+3 into stage (jt+3)%4 (the next group's activation scales
      // first when kt+3 starts it), then this tile's operands, complete before the barrier because
      // group 0 refills the stage next. In the last group, tile kt+3 is past the end from jt = 1 on: Tn's
      // tile jt-1 with all four blocks and both scale halves (Tn's live rows are not this tile's).
      if (!LAST || jt == 0) {
        if (!LAST && jt == 1) ring_req_xs<NXR>(A, S, gw, kg + 1, sx_slot(kg + 1));
        ring_req_x<NXR>(S, gw, kt + 3, L.x[(jt + 3) & 3]);
      } else {
        const RingXSrc Sn = ring_xsrc(A, Tn, gw, lane);
        if (jt == 1) ring_req_xs<4>(A, Sn, gw, wn_kg, L.sx);
        ring_req_x<4>(Sn, gw, chain ? jt - 1 : KT - 1, L.x[(jt + 3) & 3]);
      }
      read_tile(L.w[jt], L.x[jt], sw_slot(kg), sx_slot(kg), jt, jt == 0);
      WAIT_LGKMCNT0;
      // this wave's activations of tile kt+1 have landed once only the requests sent after them are
      // outstanding: tiles kt+2, kt+3 (NXR each) and, for jt = 1, 2, the next group's scales (NXS); in the
      // last group the requests past the end are 4 blocks and 2 scale halves
      if (!LAST)
        WAIT_VMCNT(2 * NXR + ((jt == 1 || jt == 2) ? NXS : 0));
      else if (jt < 3)
        WAIT_VMCNT(jt == 0 ? 2 * NXR : (jt == 1 ? NXR + 6 : 10));
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      // second half-step: multiply tile kt
      mfmas(IC<jt>{});
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
    };
    // k groups 0 .. KG-2 (no request past the end), then the last one
    constexpr auto N = IC<0>{};
    constexpr auto Y = IC<1>{};
    const int kt_last = KT - 4;
    if (grp == 0) {
      read_tile(L.w[0], L.x[0], sw_slot(0), sx_slot(0), 0, true);
      for (int kt = 0; kt < kt_last; kt += 4) {
        step0(kt, IC<0>{}, N); step0(kt + 1, IC<1>{}, N); step0(kt + 2, IC<2>{}, N); step0(kt + 3, IC<3>{}, N);
      }
      step0(kt_last, IC<0>{}, Y); step0(kt_last + 1, IC<1>{}, Y);
      step0(kt_last + 2, IC<2>{}, Y); step0(kt_last + 3, IC<3>{}, Y);
    } else {
      for (int kt = 0; kt < kt_last; kt += 4) {
        step1(kt, IC<0>{}, N); step1(kt + 1, IC<1>{}, N); step1(kt + 2, IC<2>{}, N); step1(kt + 3, IC<3>{}, N);
      }
      step1(kt_last, IC<0>{}, Y); step1(kt_last + 1, IC<1>{}, Y);
      step1(kt_last + 2, IC<2>{}, Y); step1(kt_last + 3, IC<3>{}, Y);
    }
  };
  // group 0 (weights, token rows 0-63) by its live subtiles; group 1 (activations, rows 64-127) by its live
  // subtiles and the live 32-row blocks it requests, which valid fixes together: 1-32 rows (0, 1),
  // 33-64 (0, 2), 65-80 (1, 3), 81-96 (2, 3), 97-112 (3, 4), 113-128 (4, 4)
  if (grp == 0) {
    switch (live_ts) {
      case 4: run(IC<4>{}, IC<4>{}); break;
      case 3: run(IC<3>{}, IC<4>{}); break;
      case 2: run(IC<2>{}, IC<4>{}); break;
      case 1: run(IC<1>{}, IC<4>{}); break;
      default: run(IC<0>{}, IC<4>{}); break;
    }
  } else {
    switch (ring_nxr(valid) * 8 + live_ts) {
      case 1 * 8 + 0: run(IC<0>{}, IC<1>{}); break;
      case 2 * 8 + 0: run(IC<0>{}, IC<2>{}); break;
      case 3 * 8 + 1: run(IC<1>{}, IC<3>{}); break;
      case 3 * 8 + 2: run(IC<2>{}, IC<3>{}); break;
      case 4 * 8 + 3: run(IC<3>{}, IC<4>{}); break;
      default: run(IC<4>{}, IC<4>{}); break;  // 113-128 rows (and any count past a full tile)
    }
  }
}

// The epilogue of a ring tile, staged through the wave's 2 KiB of `stg`.
template <int MODE>
KERN_DEV void ring_epilogue(const BmmArgs& A, const RingTile& T, const v4f (&acc)[4][4], uint8_t* stg) {
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));  // lane values derived per tile (see ring_tile)
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  bmm_epilogue<MODE, true>(A, acc, wave >> 2, wave & 3, T.nx, T.row0, T.valid, T.expert, lane, stg + wave * 2048);
}

// Dense modes: one tile per workgroup, grid [m/256, ceil(rows/128)].
template <int MODE>
KERN_DEV void bmm_tile(const BmmArgs& A, const BmmLds& L) {
  int nx, blk;
  tile_of(A.m / BN, nx, blk);
  const int row0 = blk * BT;
  if (row0 >= A.rows) return;
  const RingTile T = ring_tile<MODE>(A, nx, 0, row0, min(A.rows, row0 + BT) - row0);
  ring_prologue<MODE>(A, L, T);
  v4f acc[4][4];
  ring_kloop<MODE>(A, L, T, T, false, true, acc);
  ring_epilogue<MODE>(A, T, acc, L.stg);
  // the last (clamped) requests land before the workgroup's LDS is released
  WAIT_VMCNT(0);
}

// the LDS ring of one GEMM workgroup: 4 x (16 + 16) KiB tile stages + 2 x (4 + 2) KiB scale slots = 140 KiB,
// and 2 KiB per wave for staging the epilogue's stores (16 KiB)
#define BMM_LDS_DECL(L)                                                                                  \
  __shared__ __attribute__((aligned(1024))) uint8_t w0_[LDS_W], w1_[LDS_W], w2_[LDS_W], w3_[LDS_W];          \
  __shared__ __attribute__((aligned(1024))) uint8_t x0_[LDS_X], x1_[LDS_X], x2_[LDS_X], x3_[LDS_X];          \
  __shared__ __attribute__((aligned(1024))) uint8_t sw_[2 * LDS_SW], sx_[2 * LDS_SX];                      \
  __shared__ __attribute__((aligned(1024))) uint8_t stg_[8 * 2048];                                          \
  BmmLds L = {{w0_, w1_, w2_, w3_}, {x0_, x1_, x2_, x3_}, sw_, sx_, stg_}

// Skinny slots (at most skinny_rows routed rows, e.g. an expert's share of a decode batch): nothing to
// share through LDS, so no ring and no barrier. Four waves (one half of the workgroup) take a 256-row weight
// tile of the slot: each wave streams its own four weight fragments (rows 64*w .. +64) over all of K, with
// the slot's one or two 16-row activation subtiles, straight into registers, three k-tiles ahead,
// multiplying each k-tile as it lands. The two halves of the workgroup work through their own tiles
// independently, so one half's start and end overlap the other's streaming.
template <int MODE, int NTS>
KERN_DEV void skinny_tile(const BmmArgs& A, int nx, int expert, int row0, int valid, int hw, int lane) {
  // lane-only addresses derived anew in each tile (an opaque copy of the lane index), as in ring_tile
  asm volatile("" : "+v"(lane));
  const int K = A.k, KT = K >> 7, KG = K >> 9, m = A.m;
  const int c = lane & 15, g = lane >> 4;
  const int rg0 = (nx * BN) >> 4;
  // wave-uniform bases with 32-bit per-lane offsets (the activations stay below 4 GiB): each load is a
  // uniform base plus a k step in SGPRs and one VGPR offset, with no 64-bit address arithmetic per lane
  const uint8_t* wbase = A.a + (int64_t)expert * m * (K >> 1) + ((int64_t)(rg0 + 4 * hw) * KT) * 1024;
  const uint8_t* sbase = A.sf_a + (int64_t)expert * m * (K >> 5) + ((int64_t)(rg0 + 4 * hw) * KG) * 256;
  const uint32_t wl = (uint32_t)lane * 16u, sl = (uint32_t)lane * 4u;
  // buffer resources over the tile's weights and scales and over the activations, with the full 4 GiB
  // range (every offset stays inside its buffer); the k step goes in the instruction's scalar offset
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc((void*)wbase, (short)0, -1, 0x00020000);
  const __amdgpu_buffer_rsrc_t swr = __builtin_amdgcn_make_buffer_rsrc((void*)sbase, (short)0, -1, 0x00020000);
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)A.b, (short)0, -1, 0x00020000);
  const __amdgpu_buffer_rsrc_t sxr = __builtin_amdgcn_make_buffer_rsrc((void*)A.sf_b, (short)0, -1, 0x00020000);
  // this lane's activation row in each 16-row subtile: rows past the slot read the slot's first row and
  // are never stored
  uint32_t xo[NTS > 0 ? NTS : 1], sxo[NTS > 0 ? NTS : 1];
  const int sx_kstep = A.sf_b_r128c4 ? 512 : 4;
#pragma unroll
  for (int ts = 0; ts < NTS; ++ts) {
    const int t = ts * 16 + c < valid ? ts * 16 + c : 0;
    const uint32_t xrow = MODE == MODE_FC1 ? (uint32_t)A.route_map[row0 + t] : (uint32_t)(row0 + t);
    xo[ts] = xrow * (uint32_t)K + 16u * g;
    sxo[ts] = A.sf_b_r128c4 ? 512u * ((xrow >> 7) * (uint32_t)(K >> 7)) + (xrow & 31) * 16 + ((xrow & 127) >> 5) * 4 + g
                            : xrow * (uint32_t)(K >> 5) + g;
  }
  v4f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};
  // register stages: k-tile kt lives in stage kt % 4; the weight-scale dwords of k group kt / 4 in
  // slot (kt / 4) % 2, read by the MFMA's byte select (kt % 4)
  v4i wq[4][4], xq[4][NTS][2];
  uint32_t sxq[4][NTS], swq[2][4];
  // k-tile kt, S = kt % 8 (clamped: the prefetches past the end re-read the last tile, never multiplied)
  auto load = [&](int kt, auto Sc) {
    constexpr int S = decltype(Sc)::value, st = S & 3, sg = S >> 2;
    kt = min(kt, KT - 1);
    if (st == 0) {
#pragma unroll
      for (int f = 0; f < 4; ++f)
        swq[sg][f] = __builtin_amdgcn_raw_buffer_load_b32(swr, f * KG * 256 + sl, (kt >> 2) * 256, 0);
    }
#pragma unroll
    for (int f = 0; f < 4; ++f)  // weights are read once: non-temporal
      wq[st][f] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(wr, f * KT * 1024 + wl, kt * 1024, 2));
#pragma unroll
    for (int ts = 0; ts < NTS; ++ts) {
      // the B operand's two 16-byte chunks of the k-tile, g and g + 4 (the layout the MFMA reads)
      xq[st][ts][0] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(xr, xo[ts], kt * 128, 0));
      xq[st][ts][1] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(xr, xo[ts] + 64, kt * 128, 0));
      sxq[st][ts] = __builtin_amdgcn_raw_buffer_load_b8(sxr, sxo[ts], kt * sx_kstep, 0);
    }
  };
  auto compute = [&](auto Sc) {
    constexpr int S = decltype(Sc)::value, st = S & 3, sg = S >> 2;
#pragma unroll
    for (int ts = 0; ts < NTS; ++ts) {
      const v8i xb = {xq[st][ts][0][0], xq[st][ts][0][1], xq[st][ts][0][2], xq[st][ts][0][3],
                      xq[st][ts][1][0], xq[st][ts][1][1], xq[st][ts][1][2], xq[st][ts][1][3]};
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        const v8i wb = {wq[st][f][0], wq[st][f][1], wq[st][f][2], wq[st][f][3], 0, 0, 0, 0};
        acc[ts][f] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wb, xb, acc[ts][f], 4, 0, st, (int)swq[sg][f],
                                                                       0, (int)sxq[st][ts]);
      }
    }
  };
  // the scheduler barriers keep every stage's loads where they are written: sunk towards their use, they
  // would make each multiply wait for nearly all loads in flight
#define SKB __builtin_amdgcn_sched_barrier(0)
  load(0, IC<0>{}); SKB;
  load(1, IC<1>{}); SKB;
  load(2, IC<2>{}); SKB;
  int k0 = 0;
  for (; k0 + 8 <= KT; k0 += 8) {
    load(k0 + 3, IC<3>{}); SKB; compute(IC<0>{}); SKB;
    load(k0 + 4, IC<4>{}); SKB; compute(IC<1>{}); SKB;
    load(k0 + 5, IC<5>{}); SKB; compute(IC<2>{}); SKB;
    load(k0 + 6, IC<6>{}); SKB; compute(IC<3>{}); SKB;
    load(k0 + 7, IC<7>{}); SKB; compute(IC<4>{}); SKB;
    load(k0 + 8, IC<0>{}); SKB; compute(IC<5>{}); SKB;
    load(k0 + 9, IC<1>{}); SKB; compute(IC<6>{}); SKB;
    load(k0 + 10, IC<2>{}); SKB; compute(IC<7>{}); SKB;
  }
  if (k0 < KT) {  // K % 1024 == 512: one k group left, tiles k0 .. k0+2 already requested
    load(k0 + 3, IC<3>{}); SKB;
    compute(IC<0>{}); SKB; compute(IC<1>{}); SKB; compute(IC<2>{}); SKB; compute(IC<3>{}); SKB;
  }
#undef SKB
  bmm_epilogue<MODE, false>(A, acc, 0, hw, nx, row0, valid, expert, lane);
}

// The MoE ops (moe_fc1 / moe_fc2): a persistent grid of one workgroup per CU. Workgroup b owns the 256-row
// weight tiles moe_tile(b, i) (i = 0, 1, ..; gx = m/256 weight tiles per slot) of the live slots: those of
// slots of more than skinny_rows rows run on the LDS ring with all 8 waves. The tiles of small slots run in
// quarters (64 rows, one wave each, no LDS) that the eight waves take one each. In a launch with at most
// G/2 live tiles (a decode batch: T = 1 gives 128 FC1 tiles, which whole would leave half the CUs idle),
// quarter o of a small tile owned by workgroup b' runs on workgroup b' + o*G/4, so that the few tiles
// spread over every CU; otherwise a small tile's quarters all run on its owner. A pass classifies 128
// candidate tiles of each owner (b alone, or b, b - G/4, b - G/2, b - 3G/4; one per thread, one
// cta_limit read each) and compacts them into two LDS lists. The owners are congruent mod 8 (one XCD), and
// an owner's tile i exists only while i is below its share of the XCD's tiles: the pass whose last
// candidate of the smallest owner has none is the last. Both kinds of work share one launch, so a batch
// that mixes small and large slots has one tail, and slots past num_non_exiting cost nothing.
template <int MODE>
KERN_DEV void bmm_moe(const BmmArgs& A, const BmmLds& L, int* list, int* lexp, int* lval, int* wcnt) {
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // the live slots, never more than the tables hold (a corrupt count cannot send reads past them)
  const int nne = min(A.num_non_exiting[0], A.max_slots);
  const int gx = A.m >> 8, G = gridDim.x;
  constexpr int kSkinny = skinny_rows<MODE>();
  if (gx > 512) return;  // the tile lists hold nx < 512 (the host rejects m > 131072)
  // quarter owners: b - o*G/4 (mod G) for o = 0..3 when the launch has at most G/2 live tiles (and G/4 is
  // a multiple of 8), else b for all four quarters. Spreading the small tiles of larger launches cost
  // more than it gained: config 4's FC1 (4096 tiles, half of them small) took 853 us against 712 us with
  // each small tile's four quarters streaming together on its owner's CU (sharing the activation rows
  // and DRAM pages), and a T = 1 FC2 (224 tiles) 17.8 us against 15.7 us; a T = 1 FC1 (128 tiles) gains,
  // 27.7 us against 31.1 us.
  const bool spread = (G & 31) == 0 && 2 * nne * gx <= G;
  const int Q = G >> 2;
  // the owner of quarter o's tiles (this workgroup itself when not spreading)
  auto owner = [&](int o) { return spread ? (int)(((unsigned)blockIdx.x + (unsigned)(G - o * Q)) % (unsigned)G)
                                          : (int)blockIdx.x; };
  int bmin = owner(0);
  for (int o = 1; o < 4; ++o) bmin = min(bmin, owner(o));
  for (int base = 0;; base += 128) {
    // thread (o, j): candidate j of quarter o's owner; a small tile there gives this workgroup quarter o.
    // These lane values are derived anew in each pass from an opaque copy of the thread index: hoisted out
    // of the loop they stay live across the tiles, which need every register, and were spilled to scratch
    // and reloaded behind full memory waits in every pass.
    int tp = tid;
    asm volatile("" : "+v"(tp));
    const int o = tp >> 7, j = tp & 127;
    int nx, slot;
    const bool any = moe_tile(owner(o), base + j, nne, gx, G, nx, slot);
    const int v = any ? A.cta_limit[slot] - slot * BT : 0;
    const int ex = o == 0 && v > kSkinny ? A.cta_batch[slot] : 0;
    const bool ring = o == 0 && v > kSkinny, skin = v > 0 && v <= kSkinny;
    __syncthreads();  // the previous pass's work is done with the lists and the LDS
    const unsigned long long br = __ballot(ring), bs = __ballot(skin);
    if (lane == 0) wcnt[wave] = __popcll(br), wcnt[8 + wave] = __popcll(bs);
    __syncthreads();
    int pr = 0, ps = 0, nr = 0, ns = 0;
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      pr += w < wave ? wcnt[w] : 0;
      ps += w < wave ? wcnt[8 + w] : 0;
      nr += wcnt[w];
      ns += wcnt[8 + w];
    }
    const unsigned long long below = (1ull << (tp & 63)) - 1ull;
    if (ring) {  // at most 128: o == 0 only
      const int at = pr + __popcll(br & below);
      list[at] = slot * 512 + nx;  // decoded here once (m <= 512 * 256, checked on the host)
      lexp[at] = ex;
      lval[at] = v;
    }
    if (spread) {
      if (skin) list[128 + ps + __popcll(bs & below)] = (slot * 512 + nx) * 4 + o;
    } else {
      // all four thread groups classify the same tiles: quarter o of the r-th small tile goes to 4r + o,
      // so that waves 0-3 take one tile's quarters together and waves 4-7 the next one's
      const int r = ((wave & 1) ? wcnt[8 + wave - 1] : 0) + __popcll(bs & below);
      if (skin) list[128 + 4 * r + o] = (slot * 512 + nx) * 4 + o;
      ns = 4 * (wcnt[8] + wcnt[9]);
    }
    // the pass's last candidate of the smallest owner (the first CU of the XCD among the owners) lies past
    // the XCD's tiles: no later pass has work for any owner
    const bool last = !moe_tile(bmin, base + 127, nne, gx, G, nx, slot);
    __syncthreads();
    // the ring tiles, chained: each tile's last k-steps send the next one's first requests (ring_kloop)
    if (nr > 0) {
      RingTile T = ring_tile<MODE>(A, list[0] & 511, lexp[0], (list[0] >> 9) * BT, lval[0]);
      ring_prologue<MODE>(A, L, T);
      for (int e = 0; e < nr; ++e) {
        // the next tile (this one again after the last, so that its loads are sent all the same)
        const bool chain = e + 1 < nr;
        const int en = chain ? e + 1 : e;
        const int code = list[en];
        const RingTile Tn = ring_tile<MODE>(A, code & 511, lexp[en], (code >> 9) * BT, lval[en]);
        // Tn's loads (FC1's route_map) stay before the k-loop's first wait, which counts them
        asm volatile("" ::: "memory");
        v4f acc[4][4];
        ring_kloop<MODE>(A, L, T, Tn, chain, e == 0, acc);
        ring_epilogue<MODE>(A, T, acc, L.stg);
        T = Tn;
      }
      // the last tile's (clamped) requests land before the ring is used again or the LDS released
      WAIT_VMCNT(0);
    }
    for (int e = wave; e < ns; e += 8) {
      const int code = list[128 + e], q = code & 3;
      nx = (code >> 2) & 511, slot = code >> 11;
      const int row0 = slot * BT, expert = A.cta_batch[slot], valid = A.cta_limit[slot] - row0;
      if (kSkinny <= 16 || valid <= 16)
        skinny_tile<MODE, 1>(A, nx, expert, row0, valid, q, lane);
      else
        skinny_tile<MODE, (kSkinny + 15) / 16>(A, nx, expert, row0, valid, q, lane);
    }
    if (last) break;
  }
}

// Shader-clock probe, compiled only with -DKERN_CLOCK_PROBE (kern_amd/build.py writes that build to
// kern_amd/lib/kern_mx_clock.hsaco, a code object of its own beside the product's; bench.py loads it to read
// the clock the ring GEMMs run at). There, the dbg argument of kern_mx_gemm_e4m3, kern_mx_bmm_fc1 and
// kern_mx_bmm_fc2 receives no debug values but four u64 per workgroup: s_memtime (shader clock cycles) and
// s_memrealtime (a constant 100 MHz) at the workgroup's start and end. Without the macro, nothing changes.
#ifdef KERN_CLOCK_PROBE
#define CLOCK_PROBE_BEGIN()                                                  \
  const uint64_t ck_t0 = __builtin_amdgcn_s_memtime(), ck_r0 = __builtin_amdgcn_s_memrealtime()
// The end stamps follow a barrier, so they mark the workgroup's last wave, not wave 0's. Where waves run
// apart (the persistent MoE kernels' small-tile quarters), the older of the two waves that share a SIMD
// issues first and can end up to 200 us before the other: FC1 at T = 64 measured wave 0's span at 326 us,
// the last waves' at 506 us, and the launch at 514 us.
#define CLOCK_PROBE_END(buf)                                                                          \
  do {                                                                                                \
    __syncthreads();                                                                                  \
    const uint64_t ck_t1 = __builtin_amdgcn_s_memtime(), ck_r1 = __builtin_amdgcn_s_memrealtime();    \
    if ((buf) && threadIdx.x == 0) {                                                                  \
      uint64_t* o = reinterpret_cast<uint64_t*>(buf) + 4 * (blockIdx.x + gridDim.x * blockIdx.y);     \
      o[0] = ck_t0, o[1] = ck_t1, o[2] = ck_r0, o[3] = ck_r1;                                         \
    }                                                                                                 \
  } while (0)
#define PROBE_DBG(d) nullptr
#else
#define CLOCK_PROBE_BEGIN() (void)0
#define CLOCK_PROBE_END(buf) (void)0
#define PROBE_DBG(d) (d)
#endif

// op trtllm_bmm_bf16_mxe2m1_mxe4m3 (moe_fc2, head.json:25683; interface trtllm_bmm.py:19-27):
// a, sf_a, b, sf_b (R128c4 when sf_b_r128c4), c bf16 [padded][m], num_non_exiting, total_padded,
// cta_batch, cta_limit; launch adds i32 m, i32 k, i32 max_slots (the tables' capacity), i32 sf_b_r128c4,
// f32* dbg (may be null). Persistent: grid [G, 1, 1] with G a multiple of 8 (one workgroup per CU: 256),
// block 512 (bmm_moe).
extern "C" __global__ __launch_bounds__(512) void kern_mx_bmm_fc2(
    const uint8_t* a, const uint8_t* sf_a, const uint8_t* b, const uint8_t* sf_b, uint16_t* c,
    const int* num_non_exiting, const int* total_padded, const int* cta_batch, const int* cta_limit, int m, int k,
    int max_slots, int sf_b_r128c4, float* dbg) {
  BMM_LDS_DECL(L);
  BmmArgs A = {};
  A.a = a; A.sf_a = sf_a; A.b = b; A.sf_b = sf_b; A.c = c;
  A.num_non_exiting = num_non_exiting; A.cta_batch = cta_batch; A.cta_limit = cta_limit;
  A.m = m; A.k = k; A.max_slots = max_slots; A.sf_b_r128c4 = sf_b_r128c4; A.dbg = PROBE_DBG(dbg);
  (void)total_padded;
  // the pass's ring tiles (their expert and live rows beside them), then its small-tile quarters
  __shared__ int list[128 + 512], lexp[128], lval[128], wcnt[16];
  CLOCK_PROBE_BEGIN();
  bmm_moe<MODE_FC2>(A, L, list, lexp, lval, wcnt);
  CLOCK_PROBE_END(dbg);
}

// op trtllm_bmm_mxe4m3_mxe2m1_mxe4m3 (moe_fc1, head.json:25459): a, sf_a, b, sf_b (linear [T][k/32]),
// c u8 [padded][m/2], sf_c u8 R128c4, route_map, alpha, beta, num_non_exiting, total_padded, cta_batch,
// cta_limit; launch adds i32 m, i32 k, i32 max_slots, f32* dbg. Persistent grid [G, 1, 1] as moe_fc2, block
// 512.
extern "C" __global__ __launch_bounds__(512) void kern_mx_bmm_fc1(
    const uint8_t* a, const uint8_t* sf_a, const uint8_t* b, const uint8_t* sf_b, uint8_t* c, uint8_t* sf_c,
    const int* route_map, const float* alpha, const float* beta, const int* num_non_exiting,
    const int* total_padded, const int* cta_batch, const int* cta_limit, int m, int k, int max_slots, float* dbg) {
  BMM_LDS_DECL(L);
  BmmArgs A = {};
  A.a = a; A.sf_a = sf_a; A.b = b; A.sf_b = sf_b; A.c = c; A.sf_c = sf_c; A.route_map = route_map;
  A.alpha = alpha; A.beta = beta;
  A.num_non_exiting = num_non_exiting; A.cta_batch = cta_batch; A.cta_limit = cta_limit;
  A.m = m; A.k = k; A.max_slots = max_slots; A.sf_b_r128c4 = 0; A.dbg = PROBE_DBG(dbg);
  (void)total_padded;
  // the pass's ring tiles (their expert and live rows beside them), then its small-tile quarters
  __shared__ int list[128 + 512], lexp[128], lval[128], wcnt[16];
  CLOCK_PROBE_BEGIN();
  bmm_moe<MODE_FC1>(A, L, list, lexp, lval, wcnt);
  CLOCK_PROBE_END(dbg);
}

// Dense e4m3-output mode of the FC1 family (the prefill GEMM, one batch): c[t][n] = e4m3(acc * d_scale[0]).
// a, sf_a, b [M][k], sf_b linear, c u8 [M][m], d_scale f32[1], i32 M; launch adds i32 m, i32 k, f32* dbg.
// Grid [m/256, ceil(M/128), 1], block 512.
extern "C" __global__ __launch_bounds__(512) void kern_mx_gemm_e4m3(const uint8_t* a, const uint8_t* sf_a,
                                                                    const uint8_t* b, const uint8_t* sf_b,
                                                                    uint8_t* c, const float* d_scale, int M, int m,
                                                                    int k, float* dbg) {
  BMM_LDS_DECL(L);
  BmmArgs A = {};
  A.a = a; A.sf_a = sf_a; A.b = b; A.sf_b = sf_b; A.c = c; A.d_scale = d_scale;
  A.m = m; A.k = k; A.rows = M; A.sf_b_r128c4 = 0; A.dbg = PROBE_DBG(dbg);
  CLOCK_PROBE_BEGIN();
  bmm_tile<MODE_PT>(A, L);
  CLOCK_PROBE_END(dbg);
}

// Dense bf16-output mode of the FC2 family (one batch, no routing tables).
extern "C" __global__ __launch_bounds__(512) void kern_mx_gemm_bf16(const uint8_t* a, const uint8_t* sf_a,
                                                                    const uint8_t* b, const uint8_t* sf_b,
                                                                    uint16_t* c, int M, int m, int k, float* dbg) {
  BMM_LDS_DECL(L);
  BmmArgs A = {};
  A.a = a; A.sf_a = sf_a; A.b = b; A.sf_b = sf_b; A.c = c;
  A.m = m; A.k = k; A.rows = M; A.sf_b_r128c4 = 0; A.dbg = dbg;
  bmm_tile<MODE_DENSE_BF16>(A, L);
}

// ====================================================================================== MXFP8 x MXFP8 GEMM
// extern:cublaslt_mxfp8_tn (crates/kern-runtime/src/cublas.rs:387-400): row-major C[m][n] (bf16, row stride
// ldc) = sum_k deq(A)[m][k] * deq(W)[n][k]; A [m][k] and W [n][k] e4m3, each with an e8m0 scale per 32
// elements of K in the 128x4 tiled layout (rows padded to 128, k blocks to 4; block (r/128, b/4) at
// 512 (r/128 * ceil(K/128) + b/4), entry (r, b) at (r%32)*16 + (r%128/32)*4 + b%4). K % 32 == 0.
//
// One workgroup of 8 waves (two per SIMD) computes a 128 (m) x 256 (n) tile, wave (wm, wn) = 64 x 64 in a
// 2 x 4 grid, on V_MFMA_SCALE_F32_16X16X128_F8F6F4 with W as the A operand and A as the B operand (so each
// lane ends with four consecutive n of one m). Both operands go from memory straight into LDS (buffer
// loads: reads past an operand's end return zeros; rows past m or n read the last valid row and are
// never stored), 16-byte chunk j of row t at t*128 + ((j ^ ((t>>1)&7)) << 4), through a three-stage ring
// two k-tiles ahead of the MFMAs with one workgroup barrier per k-tile. Each stage is its own __shared__
// variable and the loop is unrolled by three, so that the compiler's wait counts for a stage's reads
// do not include the requests still landing in the other stages (with one runtime-selected buffer pair
// it waited for every request before each tile's reads, and loads never overlapped the MFMAs).
// Every wave issues the same seven requests per k-tile: two 1 KiB pieces of the A tile, four of the W
// tile and 48 dwords of the tile's three 512-byte scale blocks (A's, W's two), so one count fits all.
// In the last k-tile, when K % 128 != 0, the chunks past K are zeroed in registers and the scale bytes
// of k blocks past K read as 1.0.
// Buffer -> LDS requests written as inline asm, for kern_mx_gemm_mxfp8 only: the compiler does not see
// them as LDS writes, so it adds no wait of its own before the tile's LDS reads (its alias analysis
// could not tell the stage being read from the stages still filling and waited for every request). The
// kernel orders them itself: explicit request counts and a barrier per k-tile, and it issues no other
// vector-memory loads that the compiler would count. M0 carries the wave's LDS base; nothing else in
// that kernel uses M0 (checked in its code object).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
KERN_DEV void lds_dma16(__amdgpu_buffer_rsrc_t r, int voff, const void* lds_wave_base) {
  const uint32_t m0v = lds_addr(lds_wave_base);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0v), "v"(voff), "s"(r)
               : "memory", "m0");
}
// the same with the k step's byte offset in soffset (an SGPR, wave-uniform): no per-lane add per request
KERN_DEV void lds_dma16so(__amdgpu_buffer_rsrc_t r, int voff, int soff, const void* lds_wave_base) {
  const uint32_t m0v = lds_addr(lds_wave_base);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(m0v), "v"(voff), "s"(r),
               "s"(soff)
               : "memory", "m0");
}
KERN_DEV void lds_dma4(__amdgpu_buffer_rsrc_t r, int voff, const void* lds_wave_base) {
  const uint32_t m0v = lds_addr(lds_wave_base);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds" ::"s"(m0v), "v"(voff), "s"(r)
               : "memory", "m0");
}
#pragma clang diagnostic pop

#define G8_XT 16384                  // A tile: 128 rows x 128 B
#define G8_WT 32768                  // W tile: 256 rows x 128 B
#define G8_STAGE (G8_XT + G8_WT + 2048)  // + scale blocks: A's, then W's two, and 512 B of pad

extern "C" __global__ __launch_bounds__(512) void kern_mx_gemm_mxfp8(const uint8_t* __restrict__ a,
                                                                     const uint8_t* __restrict__ w,
                                                                     uint16_t* __restrict__ c,
                                                                     const uint8_t* __restrict__ a_sf,
                                                                     const uint8_t* __restrict__ w_sf, int M, int N,
                                                                     int K, int ldc) {
  __shared__ __attribute__((aligned(1024))) uint8_t st0[G8_STAGE], st1[G8_STAGE], st2[G8_STAGE];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  // tile: each XCD takes a contiguous run of the (m, n) tiles (as tile_of)
  const int gxn = gridDim.x, total = gridDim.x * gridDim.y;
  int lin = blockIdx.x + gxn * blockIdx.y;
  if ((total & 7) == 0) lin = (lin & 7) * (total >> 3) + (lin >> 3);
  const int m0 = (lin / gxn) * 128, n0 = (lin % gxn) * 256;
  const int KT = (K + 127) >> 7, KB = K >> 5, kb4 = (KB + 3) >> 2;
  const int mt = (M + 127) >> 7, nt = (N + 127) >> 7;
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*)a, (short)0, M * K, 0x00020000);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)w, (short)0, N * K, 0x00020000);
  // this lane's source row and 16-byte chunk for request r of each operand (rows 64r + 8*wave + lane/8)
  int offa[2], offw[4];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int t = 64 * r + 8 * wave + (lane >> 3);
    offa[r] = min(m0 + t, M - 1) * K + (((lane & 7) ^ ((t >> 1) & 7)) << 4);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = 64 * r + 8 * wave + (lane >> 3);
    offw[r] = min(n0 + t, N - 1) * K + (((lane & 7) ^ ((t >> 1) & 7)) << 4);
  }
  // scale dword d = 64 * wave + lane: d < 128 from A's 512-byte block of the k-tile, then W's two blocks
  // (a block past the last 128 rows of W re-reads the last one: its rows are never stored); waves 6 and
  // 7 re-read A's first dword into the pad, so that every lane of every wave issues the same request
  // (a wave reads one array: waves 0-1 A's, 2-5 W's, 6-7 A's again, so its buffer resource is uniform)
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc((void*)a_sf, (short)0, mt * kb4 * 512, 0x00020000);
  const __amdgpu_buffer_rsrc_t rsw = __builtin_amdgcn_make_buffer_rsrc((void*)w_sf, (short)0, nt * kb4 * 512, 0x00020000);
  const bool s_w = wave >= 2 && wave < 6;
  const __amdgpu_buffer_rsrc_t rs = s_w ? rsw : rsa;
  const int soff = wave < 2 ? ((m0 >> 7) * kb4) * 512 + (64 * wave + lane) * 4
                   : s_w    ? (min((n0 >> 7) + ((wave - 2) >> 1), nt - 1) * kb4) * 512 + (((wave - 2) & 1) * 64 + lane) * 4
                            : ((m0 >> 7) * kb4) * 512;
  // this lane's chunk within each k-tile (the same for all of its requests: 64r + 8*wave keeps t/2 % 8)
  const int jb = ((lane & 7) ^ (((8 * wave + (lane >> 3)) >> 1) & 7)) << 4;
  auto dma_tile = [&](int kt, uint8_t* stg) {
    kt = min(kt, KT - 1);  // requests past the last tile re-read it into a stage that is never multiplied
    // chunks past K (a partial last k-tile) read from past the buffer's end: zeros, so the MFMAs need
    // no masks. The offsets pass through an empty asm so that no copy of them is kept per step.
    int oa[2] = {offa[0], offa[1]}, ow[4] = {offw[0], offw[1], offw[2], offw[3]};
    asm volatile("" : "+v"(oa[0]), "+v"(oa[1]), "+v"(ow[0]), "+v"(ow[1]), "+v"(ow[2]), "+v"(ow[3]));
    if (kt * 128 + 128 <= K) {
      // a whole k-tile (wave-uniform test): the k step's offset goes in soffset
      int so = __builtin_amdgcn_readfirstlane(kt * 128);
      asm volatile("" : "+s"(so));
#pragma unroll
      for (int r = 0; r < 2; ++r) lds_dma16so(ra, oa[r], so, stg + (r * 8 + wave) * 1024);
#pragma unroll
      for (int r = 0; r < 4; ++r) lds_dma16so(rw, ow[r], so, stg + G8_XT + (r * 8 + wave) * 1024);
    } else {
      const bool in_k = kt * 128 + jb < K;  // 0xFFFFFFF0 lies past any operand (they are below 2 GiB)
#pragma unroll
      for (int r = 0; r < 2; ++r) lds_dma16(ra, in_k ? oa[r] + kt * 128 : (int)0xFFFFFFF0u, stg + (r * 8 + wave) * 1024);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        lds_dma16(rw, in_k ? ow[r] + kt * 128 : (int)0xFFFFFFF0u, stg + G8_XT + (r * 8 + wave) * 1024);
    }
    lds_dma4(rs, soff + kt * 512, stg + G8_XT + G8_WT + wave * 256);
  };

  v4f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};

  auto tile = [&](const uint8_t* stg, bool last) {
    // operands: n subtiles (A operand, from W), then the m subtiles (B operand, from A) in two halves,
    // each multiplied as it lands (fewer operand registers live at once)
    v8i wo[4], ao[2];
    uint32_t sw_[4], sa_[2];
    const uint8_t* sc = stg + G8_XT + G8_WT;
    // the lane coordinates pass through an empty asm, so that the LDS addresses derived from them are
    // computed here, per tile, instead of being hoisted out of the loop for every copy of the unrolled
    // steps (which ran out of registers)
    int cl = lane & 15, g = lane >> 4;
    asm volatile("" : "+v"(cl), "+v"(g));
    const int kr = K & 127;  // valid bytes of a partial last tile (its chunks past K are zeros)
    const bool vs = !last || kr == 0 || 32 * g < kr;  // this lane's k block lies within K
    // Scales (R128c4: row t's four k blocks are one dword at (t & 31) * 16 + ((t & 127) >> 5) * 4 of its
    // 128-row block). The 16 bytes at (t & 31) * 16 hold the dwords of rows t, t + 32, t + 64 and t + 96, so
    // one 16-byte read per subtile pair fetches the dwords of subtiles q and q + 2 (the lane keeps the half
    // of its 64-row group), and the lane takes its k block's byte by a shift. Lanes that differ only in their
    // k block read the same 16 bytes, and each group of 16 lanes reads 256 contiguous bytes: no bank
    // conflicts. (Two 8-byte reads, which the compiler paired into one ds_read2_b64 of two rows 256 bytes
    // apart, put both halves of every lane on the same banks: a sixth of the LDS cycles were conflicts.
    // A read per byte cost the LDS as much as a 16-byte read, and conflicted too.)
    const int sh = 8 * g;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const v4u d = *reinterpret_cast<const v4u*>(sc + 512 + (wn >> 1) * 512 + (q * 16 + cl) * 16);
      const uint32_t lo = (wn & 1) ? d[2] : d[0], hi = (wn & 1) ? d[3] : d[1];
      sw_[q] = vs ? (lo >> sh) & 255u : 127u;
      sw_[q + 2] = vs ? (hi >> sh) & 255u : 127u;
    }
    uint32_t sa4[2][2];  // [half][subtile]: rows wm*64 + (2h + q)*16 + cl
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const v4u d = *reinterpret_cast<const v4u*>(sc + (q * 16 + cl) * 16);
      const uint32_t lo = wm ? d[2] : d[0], hi = wm ? d[3] : d[1];
      sa4[0][q] = vs ? (lo >> sh) & 255u : 127u;
      sa4[1][q] = vs ? (hi >> sh) & 255u : 127u;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int t = wn * 64 + q * 16 + cl;
      const uint8_t* row = stg + G8_XT + t * 128;
      const int sw = (t >> 1) & 7;
      v4i x0 = *reinterpret_cast<const v4i*>(row + ((g ^ sw) << 4));
      v4i x1 = *reinterpret_cast<const v4i*>(row + (((g + 4) ^ sw) << 4));
      wo[q] = (v8i){x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int t = wm * 64 + (2 * h + q) * 16 + cl;
        const uint8_t* row = stg + t * 128;
        const int sw = (t >> 1) & 7;
        v4i x0 = *reinterpret_cast<const v4i*>(row + ((g ^ sw) << 4));
        v4i x1 = *reinterpret_cast<const v4i*>(row + (((g + 4) ^ sw) << 4));
        ao[q] = (v8i){x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
        sa_[q] = sa4[h][q];
      }
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[2 * h + q][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wo[j], ao[q], acc[2 * h + q][j], 0, 0, 0,
                                                                                (int)sw_[j], 0, (int)sa_[q]);
    }
  };
  // k-tile kt: its requests landed for this wave once only tile kt+1's seven are outstanding; after the
  // barrier every wave's have, and every wave is done reading tile kt-1, whose stage takes tile kt+2
  // The loop runs in threes; past the last k-tile a step still waits, meets the barrier and issues its
  // (clamped) requests, so that every path has the same request counts, and skips only the multiply.
  auto step = [&](int kt, uint8_t* cur, uint8_t* refill) {
    __builtin_amdgcn_sched_barrier(0);
    WAIT_VMCNT(7);
    // a bare barrier: __syncthreads() would add a workgroup fence, which waits for every request in
    // flight (tile kt+1's too). The previous tile's LDS reads are complete: its MFMAs consumed them.
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    dma_tile(kt + 2, refill);
    if (kt < KT) tile(cur, kt == KT - 1);
    __builtin_amdgcn_sched_barrier(0);
  };
  dma_tile(0, st0);
  dma_tile(1, st1);
  for (int kt = 0; kt < KT; kt += 3) {
    step(kt, st0, st2);
    step(kt + 1, st1, st0);
    step(kt + 2, st2, st1);
  }
  WAIT_VMCNT(0);  // the clamped re-reads land before the workgroup's LDS is released

  // lane (cl, g) of tile (i, j) holds n = n0 + wn*64 + 16j + 4g + (0..3) for m = m0 + wm*64 + 16i + cl
  const int cl = lane & 15, g = lane >> 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + wm * 64 + 16 * i + cl;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + wn * 64 + 16 * j + 4 * g;
      if (n >= N) continue;
      const v4f v = acc[i][j];
      uint16_t* dst = c + (int64_t)m * ldc + n;
      if (n + 3 < N && ((((uintptr_t)dst) & 7) == 0)) {
        const uint32_t lo = f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16);
        const uint32_t hi = f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16);
        *reinterpret_cast<uint2*>(dst) = make_uint2(lo, hi);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (n + e < N) dst[e] = (uint16_t)f32_to_bf16_bits(v[e]);
      }
    }
  }
}

// ====================================================================================== routing
// op moe_routing (head.json:25117): in i32 topk_idx[T][topk]; out counts [2E], cta_batch, cta_limit,
// num_non_exiting[1], total_padded[1], route_map, exp2perm [T*topk]; launch adds i32 T, i32 topk,
// i32 local_start, i32 E_local (<= 512). Rows of one expert in ascending expanded index, each expert padded
// to 128-row CTA slots (tables as tools/kernels/abi/trtllm_bmm.py:19-27). A stable counting sort with no
// serial step: each wave owns a contiguous segment of the expanded indices. (1) Each wave counts its
// segment per expert (LDS atomics). (2) Per expert, the counts become the wave's first row of the expert
// (exclusive prefixes over the waves on top of the expert's first slot, the slot counts an exclusive scan
// over the experts). (3) Each wave walks its segment again, 64 indices at a time: the lanes holding expert
// e OR their lane bits into a per-wave 64-bit mask, so a lane's rank among the lower lanes of its expert is
// a popcount; the lowest such lane then advances the wave's next row of e and clears the mask (one wave's
// LDS operations execute in program order). kern_mx_routing does it all in one workgroup of 1024 threads;
// kern_mx_routing_count/_scan/_rank split large batches over chunks of several workgroups.
#define ROUTE_EMAX 512
KERN_DEV int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int u = __shfl_up(v, d);
    if (lane >= d) v += u;
  }
  return v;
}

// the local expert of expanded index i, or -1 when it is not local
KERN_DEV int route_expert(const int* __restrict__ topk_idx, int i, int local_start, int E) {
  const int e = topk_idx[i] - local_start;
  return e >= 0 && e < E ? e : -1;
}

// phase (1) for one wave's segment [i_begin, i_end): wb[e] += the segment's indices of expert e
KERN_DEV void route_count_wave(const int* __restrict__ topk_idx, int i_begin, int i_end, int local_start, int E,
                               int* wb, int lane) {
  for (int i = i_begin + lane; i < i_end; i += 64) {
    const int e = route_expert(topk_idx, i, local_start, E);
    if (e >= 0) atomicAdd(&wb[e], 1);
  }
}

// phase (3) for one wave's segment: wb[e] holds the segment's first row of expert e, wm[e] is zero (and is
// again on return)
KERN_DEV void route_rank_wave(const int* __restrict__ topk_idx, int* __restrict__ route_map,
                              int* __restrict__ exp2perm, int i_begin, int i_end, int topk, int local_start, int E,
                              int* wb, unsigned long long* wm, int lane) {
  for (int i0 = i_begin; i0 < i_end; i0 += 64) {
    const int i = i0 + lane;
    const int e = i < i_end ? route_expert(topk_idx, i, local_start, E) : -1;
    if (e >= 0) atomicOr(&wm[e], 1ull << lane);
    if (e >= 0) {
      const unsigned long long m = wm[e];
      const int rank = __popcll(m & ((1ull << lane) - 1ull));
      const int p = wb[e] + rank;
      exp2perm[i] = p;
      route_map[p] = i / topk;
      if (rank == 0) {  // the expert's lowest lane, after every lane of the group has read the mask
        wb[e] += __popcll(m);
        wm[e] = 0ull;
      }
    } else if (i < i_end) {
      exp2perm[i] = -1;
    }
  }
}

KERN_DEV void routing_block(const int* __restrict__ topk_idx, int* __restrict__ counts, int* __restrict__ cta_batch,
                           int* __restrict__ cta_limit, int* __restrict__ num_non_exiting,
                           int* __restrict__ total_padded, int* __restrict__ route_map, int* __restrict__ exp2perm,
                           int T, int topk, int local_start, int E_local) {
  __shared__ int wbase[16 * ROUTE_EMAX];                 // [wave][expert]: count, then the wave's next row
  __shared__ unsigned long long wmask[16 * ROUTE_EMAX];  // [wave][expert]: lanes holding the expert
  __shared__ int wsum[16];
  __shared__ int total_slots;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = T * topk, E = E_local;
  const int seg = (n + 16 * 64 - 1) / (16 * 64) * 64;  // indices per wave, a multiple of 64
  const int i_begin = wave * seg, i_end = min(n, i_begin + seg);
  int* wb = wbase + wave * E;
  unsigned long long* wm = wmask + wave * E;
  for (int q = lane; q < E; q += 64) wb[q] = 0, wm[q] = 0ull;
  // (1) per-wave counts (the wave's own table: the clears above came first in program order)
  route_count_wave(topk_idx, i_begin, i_end, local_start, E, wb, lane);
  __syncthreads();
  // (2) per expert: exclusive prefix over the waves, total count and slot count
  int cnt = 0, ns = 0;
  if (tid < E) {
    for (int w = 0; w < 16; ++w) {
      const int c = wbase[w * E + tid];
      wbase[w * E + tid] = cnt;
      cnt += c;
    }
    ns = (cnt + 127) >> 7;
  }
  // exclusive scan of the slot counts over the experts (E <= 512: waves 0..7)
  const int incl = wave_incl_scan(ns, lane);
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  if (tid == 0) {
    int s = 0;
    for (int w = 0; w < 16; ++w) {
      const int v = wsum[w];
      wsum[w] = s;
      s += v;
    }
    total_slots = s;
    num_non_exiting[0] = s;
    total_padded[0] = s * 128;
  }
  __syncthreads();
  if (tid < E) {
    const int o = wsum[wave] + incl - ns;
    for (int w = 0; w < 16; ++w) wbase[w * E + tid] += o * 128;  // wave w's first row of expert tid
    counts[tid] = cnt;
    counts[E + tid] = o;
    for (int s2 = 0; s2 < ns; ++s2) {
      cta_batch[o + s2] = tid;
      cta_limit[o + s2] = min((o + s2 + 1) * 128, o * 128 + cnt);
    }
  }
  const int S = total_slots;
  for (int p = tid; p < S * 128; p += 1024) route_map[p] = -1;
  __syncthreads();  // the first rows are complete, and every padding row is written before the rows that fill it
  // (3) stable ranks, 64 indices of the wave's segment at a time
  route_rank_wave(topk_idx, route_map, exp2perm, i_begin, i_end, topk, local_start, E, wb, wm, lane);
}

extern "C" __global__ __launch_bounds__(1024) void kern_mx_routing(
    const int* __restrict__ topk_idx, int* __restrict__ counts, int* __restrict__ cta_batch,
    int* __restrict__ cta_limit, int* __restrict__ num_non_exiting, int* __restrict__ total_padded,
    int* __restrict__ route_map, int* __restrict__ exp2perm, int T, int topk, int local_start, int E_local) {
  routing_block(topk_idx, counts, cta_batch, cta_limit, num_non_exiting, total_padded, route_map, exp2perm, T, topk,
                local_start, E_local);
}

// moe_quant and moe_routing in one launch (they are independent): workgroup 0 builds the routing tables
// (kern_mx_routing's block), workgroups 1.. quantize (kern_mx_quant_bf16's lanes, 1024 per workgroup). For
// decode-sized batches, where each of the two launches is mostly launch and memory latency. Grid
// 1 + ceil(T*K/16 / 1024), block 1024.
extern "C" __global__ __launch_bounds__(1024) void kern_mx_quant_routing(
    const uint16_t* __restrict__ x, uint8_t* __restrict__ q, uint8_t* __restrict__ sf, int K,
    const int* __restrict__ topk_idx, int* __restrict__ counts, int* __restrict__ cta_batch,
    int* __restrict__ cta_limit, int* __restrict__ num_non_exiting, int* __restrict__ total_padded,
    int* __restrict__ route_map, int* __restrict__ exp2perm, int T, int topk, int local_start, int E_local) {
  if (blockIdx.x == 0) {
    routing_block(topk_idx, counts, cta_batch, cta_limit, num_non_exiting, total_padded, route_map, exp2perm, T, topk,
                  local_start, E_local);
    return;
  }
  quant_bf16_lane(x, q, sf, T, K, (int64_t)(blockIdx.x - 1) * 1024 + threadIdx.x);
}

// moe_routing for large batches in three launches, with kern_mx_routing's tables bit for bit. The n = T*topk
// expanded indices split into G = min(64, ceil(n / 4096)) chunks of CH = floor(n / G) rounded down to 64
// indices, the last chunk taking the rest; for n >= 4096 every chunk holds at least 1984 > E indices.
// (count) workgroup g counts its chunk per expert and parks the counts in exp2perm[g*CH + e], the first E
// entries of its own chunk. (scan) one workgroup turns the G x E counts into the slot tables and, per
// chunk and expert, the chunk's first row of the expert, written back in the same places; it also writes
// the padding rows of route_map. (rank) workgroup g reads its chunk's E first rows, then ranks the chunk
// as kern_mx_routing's block ranks its segments (16 waves) and overwrites the parked entries with the
// chunk's own exp2perm. No chunk reads another chunk's exp2perm range, so the rank workgroups do not race.
// All three take kern_mx_routing's arguments; grid [G] for count and rank, [1] for scan, block 1024.
// The host takes this path for n >= 4096 only.
#define ROUTE_CHUNK 4096
#define ROUTE_GMAX 64
KERN_DEV int route_chunks(int n) { return min(ROUTE_GMAX, max(1, (n + ROUTE_CHUNK - 1) / ROUTE_CHUNK)); }
KERN_DEV int route_chunk_len(int n, int G) { return (n / G) & ~63; }

extern "C" __global__ __launch_bounds__(1024) void kern_mx_routing_count(
    const int* __restrict__ topk_idx, int* __restrict__ counts, int* __restrict__ cta_batch,
    int* __restrict__ cta_limit, int* __restrict__ num_non_exiting, int* __restrict__ total_padded,
    int* __restrict__ route_map, int* __restrict__ exp2perm, int T, int topk, int local_start, int E_local) {
  __shared__ int h[ROUTE_EMAX];
  const int tid = threadIdx.x, n = T * topk, E = E_local, G = route_chunks(n), g = blockIdx.x;
  if (g >= G) return;
  const int CH = route_chunk_len(n, G), b = g * CH, end = g == G - 1 ? n : b + CH;
  if (tid < E) h[tid] = 0;
  __syncthreads();
  for (int i = b + tid; i < end; i += 1024) {
    const int e = route_expert(topk_idx, i, local_start, E);
    if (e >= 0) atomicAdd(&h[e], 1);
  }
  __syncthreads();
  if (tid < E && b + tid < end) exp2perm[b + tid] = h[tid];
}

extern "C" __global__ __launch_bounds__(1024) void kern_mx_routing_scan(
    const int* __restrict__ topk_idx, int* __restrict__ counts, int* __restrict__ cta_batch,
    int* __restrict__ cta_limit, int* __restrict__ num_non_exiting, int* __restrict__ total_padded,
    int* __restrict__ route_map, int* __restrict__ exp2perm, int T, int topk, int local_start, int E_local) {
  __shared__ int h[ROUTE_GMAX * ROUTE_EMAX];  // [chunk][expert]: count, then the chunk's first row (128 KiB)
  __shared__ int off[ROUTE_EMAX], cnt_e[ROUTE_EMAX];
  __shared__ int wsum[16];
  __shared__ int total_slots;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = T * topk, E = E_local, G = route_chunks(n), CH = route_chunk_len(n, G);
  for (int q = tid; q < G * E; q += 1024) {
    const int g = q / E, i = g * CH + (q - g * E);
    h[q] = i < n ? exp2perm[i] : 0;
  }
  __syncthreads();
  // per expert: exclusive prefix over the chunks (eight loads before their stores), total and slot count
  int cnt = 0, ns = 0;
  if (tid < E) {
    for (int g0 = 0; g0 < G; g0 += 8) {
      int c[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) c[j] = g0 + j < G ? h[(g0 + j) * E + tid] : 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (g0 + j < G) h[(g0 + j) * E + tid] = cnt;
        cnt += c[j];
      }
    }
    ns = (cnt + 127) >> 7;
  }
  // exclusive scan of the slot counts over the experts (E <= 512: waves 0..7)
  const int incl = wave_incl_scan(ns, lane);
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  if (tid == 0) {
    int s = 0;
    for (int w = 0; w < 16; ++w) {
      const int v = wsum[w];
      wsum[w] = s;
      s += v;
    }
    total_slots = s;
    num_non_exiting[0] = s;
    total_padded[0] = s * 128;
  }
  __syncthreads();
  if (tid < E) {
    const int o = wsum[wave] + incl - ns;
    off[tid] = o;
    cnt_e[tid] = cnt;
    counts[tid] = cnt;
    counts[E + tid] = o;
  }
  __syncthreads();
  const int S = total_slots;
  // slot tables, a thread per slot: the slot's expert is the last with off[e] <= s (an expert without
  // slots shares its off with the next one, and the last expert's off + slots is S > s)
  for (int s = tid; s < S; s += 1024) {
    int lo = 0, hi = E - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (off[mid] <= s) lo = mid;
      else hi = mid - 1;
    }
    cta_batch[s] = lo;
    cta_limit[s] = min((s + 1) * 128, off[lo] * 128 + cnt_e[lo]);
  }
  // padding rows, a wave per expert: rows past the count in the expert's last slot
  for (int e = wave; e < E; e += 16) {
    const int p0 = off[e] * 128 + cnt_e[e], p1 = (off[e] + ((cnt_e[e] + 127) >> 7)) * 128;
    for (int p = p0 + lane; p < p1; p += 64) route_map[p] = -1;
  }
  // per chunk and expert: the first row, parked where the count was
  for (int q = tid; q < G * E; q += 1024) {
    const int g = q / E, e = q - g * E, i = g * CH + e;
    if (i < n) exp2perm[i] = off[e] * 128 + h[q];
  }
}

extern "C" __global__ __launch_bounds__(1024) void kern_mx_routing_rank(
    const int* __restrict__ topk_idx, int* __restrict__ counts, int* __restrict__ cta_batch,
    int* __restrict__ cta_limit, int* __restrict__ num_non_exiting, int* __restrict__ total_padded,
    int* __restrict__ route_map, int* __restrict__ exp2perm, int T, int topk, int local_start, int E_local) {
  __shared__ int wbase[16 * ROUTE_EMAX];                 // [wave][expert]: count, then the wave's next row
  __shared__ unsigned long long wmask[16 * ROUTE_EMAX];  // [wave][expert]: lanes holding the expert
  __shared__ int first[ROUTE_EMAX];                      // the chunk's first row of each expert
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = T * topk, E = E_local, G = route_chunks(n), g = blockIdx.x;
  if (g >= G) return;
  const int CH = route_chunk_len(n, G), b = g * CH, end = g == G - 1 ? n : b + CH;
  if (tid < E) first[tid] = b + tid < end ? exp2perm[b + tid] : 0;
  const int seg = (end - b + 16 * 64 - 1) / (16 * 64) * 64;  // indices per wave, a multiple of 64
  const int i_begin = b + wave * seg, i_end = min(end, i_begin + seg);
  int* wb = wbase + wave * E;
  unsigned long long* wm = wmask + wave * E;
  for (int q = lane; q < E; q += 64) wb[q] = 0, wm[q] = 0ull;
  route_count_wave(topk_idx, i_begin, i_end, local_start, E, wb, lane);
  __syncthreads();  // every parked first row is read before any exp2perm store of the chunk; counts complete
  if (tid < E) {
    int r = first[tid];
    for (int w = 0; w < 16; ++w) {
      const int c = wbase[w * E + tid];
      wbase[w * E + tid] = r;
      r += c;
    }
  }
  __syncthreads();
  route_rank_wave(topk_idx, route_map, exp2perm, i_begin, i_end, topk, local_start, E, wb, wm, lane);
}


// ====================================================================================== MoE glue
// silu_mul (tools/kernels-src/silu_mul.cu:1-5): out[t][i] = bf16(bf16(g / (1 + exp(-g))) * u), g = in[t][i],
// u = in[t][d + i]; in [tokens][2d], out [tokens][d] (bf16). Same ABI as the reference kernel: (out, in, d),
// grid [tokens, ceil(d / 2048)], block 256, eight consecutive elements per thread (one 16-byte load per
// operand); d % 8 == 0. SiLU in f32 with an IEEE divide, rounded to bf16; the product of two bf16 values
// is exact in f32 and rounded once.
extern "C" __global__ __launch_bounds__(256) void kern_silu_mul_bf16(uint16_t* __restrict__ out,
                                                                     const uint16_t* __restrict__ in, int d) {
  const int64_t t = blockIdx.x;
  const int i = (blockIdx.y * 256 + threadIdx.x) * 8;
  if (i >= d) return;
  const v4u gv = *reinterpret_cast<const v4u*>(in + t * 2 * d + i);
  const v4u uv = *reinterpret_cast<const v4u*>(in + t * 2 * d + d + i);
  v4u ov;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t o = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float g = bf16_bits_to_f32((gv[j] >> (16 * h)) & 0xffffu);
      const float u = bf16_bits_to_f32((uv[j] >> (16 * h)) & 0xffffu);
      const float sl = bf16_bits_to_f32(f32_to_bf16_bits(g / (1.0f + expf(-g))));
      o |= f32_to_bf16_bits(sl * u) << (16 * h);
    }
    ov[j] = o;
  }
  *reinterpret_cast<v4u*>(out + t * d + i) = ov;
}

// MoE finalize: y[t] = sum_j w[t][j] * fc2_out[exp2perm[t*topk + j]] over the token's routed rows in j order
// (f32 fused multiply-adds; rows of non-local experts, exp2perm < 0, add nothing), the combine of
// tools/trtllm-bmm/probe.py:100-110 (index_add of weighted FC2 rows). moe_finalize_rms (head.json: module
// k3_prefill_glue, entry kern_k3g_finalize_rms) then writes out[t] = bf16(y * (1 / sqrt(mean(y^2) + eps)) *
// gamma), the plain finalize out[t] = bf16(y). One workgroup of 256 threads per token, eight consecutive
// columns per thread and chunk; H % 8 == 0 and, with the norm, H <= 8192 (the row stays in registers
// between the two passes).
// the combined row y of one 8-column chunk of token t
KERN_DEV void moe_combine_chunk(const uint16_t* __restrict__ fc2_out, const int* __restrict__ exp2perm,
                                const float* __restrict__ topk_w, int t, int H, int topk, int chunk, float acc[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  // eight routed rows at a time: all eight loads in flight before the first multiply, then the products
  // added in routing order (j = 0, 1, ..), skipping rows that are not local
  for (int j0 = 0; j0 < topk; j0 += 8) {
    v4u xv[8];
    float w[8];
    bool ok[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const int j = j0 + jj;
      const int row = j < topk ? exp2perm[(int64_t)t * topk + j] : -1;
      w[jj] = j < topk ? topk_w[(int64_t)t * topk + j] : 0.f;
      ok[jj] = row >= 0;
      xv[jj] = ok[jj] ? *reinterpret_cast<const v4u*>(fc2_out + (int64_t)row * H + chunk * 8) : (v4u){0, 0, 0, 0};
    }
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      if (!ok[jj]) continue;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        acc[e] = __builtin_fmaf(w[jj], bf16_bits_to_f32((xv[jj][e >> 1] >> (16 * (e & 1))) & 0xffffu), acc[e]);
    }
  }
}

// moe_combine_chunk for the Q chunks c0 + 256 q of one thread at once (chunks >= nchunks are skipped):
// the rows of all Q chunks are in flight together; per chunk the sum is the same as moe_combine_chunk's
template <int Q>
KERN_DEV void moe_combine_chunks(const uint16_t* __restrict__ fc2_out, const int* __restrict__ exp2perm,
                                 const float* __restrict__ topk_w, int t, int H, int topk, int c0, int nchunks,
                                 float acc[Q][8]) {
#pragma unroll
  for (int q = 0; q < Q; ++q)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[q][e] = 0.f;
  for (int j0 = 0; j0 < topk; j0 += 8) {
    v4u xv[Q][8];
    float w[8];
    bool ok[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const int j = j0 + jj;
      const int row = j < topk ? exp2perm[(int64_t)t * topk + j] : -1;
      w[jj] = j < topk ? topk_w[(int64_t)t * topk + j] : 0.f;
      ok[jj] = row >= 0;
#pragma unroll
      for (int q = 0; q < Q; ++q) {
        const int c = c0 + 256 * q;
        xv[q][jj] = ok[jj] && c < nchunks ? *reinterpret_cast<const v4u*>(fc2_out + (int64_t)row * H + c * 8)
                                          : (v4u){0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      if (!ok[jj]) continue;
#pragma unroll
      for (int q = 0; q < Q; ++q)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          acc[q][e] = __builtin_fmaf(w[jj], bf16_bits_to_f32((xv[q][jj][e >> 1] >> (16 * (e & 1))) & 0xffffu), acc[q][e]);
    }
  }
}

KERN_DEV v4u bf16x8(const float v[8]) {
  v4u o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = f32_to_bf16_bits(v[2 * e]) | (f32_to_bf16_bits(v[2 * e + 1]) << 16);
  return o;
}

// op moe_finalize_rms (head.json, call l1.finalize): in bf16 fc2_out [padded][H], in i32 exp2perm [T*topk],
// in f32 topk_weight [T][topk], in bf16 gamma [H], out bf16 out [T][H], i32 T; launch adds i32 H, i32 topk,
// f32 eps. Grid [T], block = the row's H/8 chunks rounded up to a multiple of 64 (at most 1024: H <= 8192):
// one chunk per thread, whose eight routed rows are in flight together. A token's whole row in one pass of
// small threads: at config 4's T = 512 and at T = 2048 this ran 6% shorter than 256 threads of four chunks
// each (185 registers a thread allowed two such workgroups per CU, 52 allow the CU's share of the token rows).
// A launch with fewer threads (any multiple of 64) is still correct: its threads take chunks tid,
// tid + blockDim, .. twice, once for the row's sum of squares and once for the output, reading the routed
// rows twice.
extern "C" __global__ __launch_bounds__(1024) void kern_mx_moe_finalize_rms(
    const uint16_t* __restrict__ fc2_out, const int* __restrict__ exp2perm, const float* __restrict__ topk_w,
    const uint16_t* __restrict__ gamma, uint16_t* __restrict__ out, int T, int H, int topk, float eps) {
  __shared__ float red[16];
  (void)T;
  const int t = blockIdx.x, tid = threadIdx.x, chunks = H >> 3, nt = blockDim.x, nw = nt >> 6;
  const bool whole = chunks <= nt;  // one chunk per thread at most (uniform)
  const bool live = tid < chunks;
  // gamma's chunk first: its load overlaps the routed rows' instead of following the reduction
  const v4u gm = whole && live ? *reinterpret_cast<const v4u*>(gamma + tid * 8) : (v4u){0, 0, 0, 0};
  float y[1][8];
  float ss = 0.f;
  if (whole) {
    moe_combine_chunks<1>(fc2_out, exp2perm, topk_w, t, H, topk, tid, chunks, y);
    if (live) {
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(y[0][e], y[0][e], ss);
    }
  } else {
    for (int c = tid; c < chunks; c += nt) {
      moe_combine_chunks<1>(fc2_out, exp2perm, topk_w, t, H, topk, c, chunks, y);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(y[0][e], y[0][e], ss);
    }
  }
  // sum of squares over the row: wave reduction, then the waves in LDS, in wave order
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
  for (int w = 0; w < nw; ++w) tot += red[w];
  const float r = 1.0f / sqrtf(tot / (float)H + eps);
  auto put = [&](int c, const v4u& g) {
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = y[0][e] * r * bf16_bits_to_f32((g[e >> 1] >> (16 * (e & 1))) & 0xffffu);
    *reinterpret_cast<v4u*>(out + (int64_t)t * H + c * 8) = bf16x8(v);
  };
  if (whole) {
    if (live) put(tid, gm);
  } else {
    for (int c = tid; c < chunks; c += nt) {
      moe_combine_chunks<1>(fc2_out, exp2perm, topk_w, t, H, topk, c, chunks, y);
      put(c, *reinterpret_cast<const v4u*>(gamma + c * 8));
    }
  }
}

// MoE finalize without the norm (the combine flashinfer's do_finalize returns, probe.py:85-110):
// fc2_out, exp2perm, topk_weight, out bf16 [T][H], i32 T; launch adds i32 H, i32 topk. Grid [T], block 256.
extern "C" __global__ __launch_bounds__(256) void kern_mx_moe_finalize(const uint16_t* __restrict__ fc2_out,
                                                                       const int* __restrict__ exp2perm,
                                                                       const float* __restrict__ topk_w,
                                                                       uint16_t* __restrict__ out, int T, int H,
                                                                       int topk) {
  (void)T;
  const int t = blockIdx.x;
  for (int c = threadIdx.x; c < (H >> 3); c += 256) {
    float v[8];
    moe_combine_chunk(fc2_out, exp2perm, topk_w, t, H, topk, c, v);
    *reinterpret_cast<v4u*>(out + (int64_t)t * H + c * 8) = bf16x8(v);
  }
}

// ====================================================================================== weight_prep
// The derived tables a manifest's `once` program computes after load (tools/kernels-src/weight_prep.cu:1-20).
// The entry names, argument lists and the one-thread-per-element mapping (i = block * blockDim + thread,
// nothing past n) are the reference's, so the once-program launches (literal grids) run unchanged.

// out[i] = f32(w[i]) + 1 (GemmaRMSNorm's weight + 1)
extern "C" __global__ void kern_weight_p1_bf16_f32(const uint16_t* __restrict__ w, float* __restrict__ out, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = bf16_bits_to_f32(w[i]) + 1.0f;
}

// out[i] = f32(w[i])
extern "C" __global__ void kern_cast_bf16_f32(const uint16_t* __restrict__ w, float* __restrict__ out, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = bf16_bits_to_f32(w[i]);
}

// RoPE cache: inv = 1 / base^(2j / (2 half)), angle = r * inv (f32), cos/sin rounded to bf16 at
// [r * stride + j] for r < rows, j < half. Grid.x = rows, a thread per column (block >= half).
extern "C" __global__ void kern_rope_table_bf16(uint16_t* __restrict__ cos_t, uint16_t* __restrict__ sin_t, int rows,
                                                int half, int stride, float base) {
  const int j = threadIdx.x, r = blockIdx.x;
  if (j >= half || r >= rows) return;
  const float inv = 1.0f / powf(base, (float)(2 * j) / (float)(2 * half));
  const float angle = (float)r * inv;
  cos_t[(int64_t)r * stride + j] = (uint16_t)f32_to_bf16_bits(cosf(angle));
  sin_t[(int64_t)r * stride + j] = (uint16_t)f32_to_bf16_bits(sinf(angle));
}

extern "C" __global__ void kern_fill_f32(float* __restrict__ p, int n, float v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

extern "C" __global__ void kern_fill_i32(int* __restrict__ p, int n, int v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

extern "C" __global__ void kern_fill_i64(int64_t* __restrict__ p, int n, int64_t v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

extern "C" __global__ void kern_fill_u8(uint8_t* __restrict__ p, int n, int v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = (uint8_t)v;
}

// the bf16 fill of K3's k3_weight_prep module (fixtures/k3/head.json op fill_bf16): p[i] = bf16(v), RNE
extern "C" __global__ void kern_fill_bf16(uint16_t* __restrict__ p, int n, float v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = (uint16_t)f32_to_bf16_bits(v);
}

// p[i * stride] = start + i * step
extern "C" __global__ void kern_iota_i32(int* __restrict__ p, int n, int start, int step, int stride) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[(int64_t)i * stride] = start + i * step;
}

// ====================================================================================== workload fills
// Synthetic seeded inputs (splitmix64 stream, crates/kern-test/src/workload.rs:11-26):
// out[i] = lo + draw_i % span.
extern "C" __global__ __launch_bounds__(256) void kern_mx_fill_random_u8(uint8_t* __restrict__ out, int64_t n,
                                                                         uint64_t seed, int lo, int span) {
  int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 16;
  if (i >= n) return;
  if (i + 16 <= n) {
    v4u v;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      uint32_t d = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b)
        d |= (uint32_t)((lo + (int)(splitmix64_at(seed, i + 4 * w + b) % (uint64_t)span)) & 0xff) << (8 * b);
      v[w] = d;
    }
    *reinterpret_cast<v4u*>(out + i) = v;
  } else {
    for (int64_t j = i; j < n; ++j) out[j] = (uint8_t)(lo + (int)(splitmix64_at(seed, j) % (uint64_t)span));
  }
}
