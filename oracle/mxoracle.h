/* CPU oracle for the MXFP4 matmul path — TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of the arithmetic of kern's quantized matmul path, used by tests/,
 * by __graft_entry__.smoke() and by bench.py's cpu_baseline leg as the checker. Nothing in the
 * product (kern_amd/) links, loads or calls it; the product fails loudly when its HIP library is
 * missing instead of falling back here.
 *
 * Every function names the reference file:line it restates. Where the reference's arithmetic lives
 * outside its tree (flashinfer-cubin 0.6.18 / FlashInfer 0.6.18: mxfp8_quantize, shuffle_matrix_a,
 * routing kernels), the function states our own definition and how it is pinned instead.
 *
 * Pinning (what checks each function, besides GPU parity):
 *   codecs ........ exhaustive KATs (all 16 e2m1 / 256 e4m3 / 256 e8m0 codes) + brute-force nearest
 *                   search over every finite e4m3 value for the encoder (tests/test_oracle_codecs.py)
 *   quantizer ..... closed-form cases (power-of-two amax, 448 saturation, zero, subnormal, NaN/Inf)
 *                   + committed golden vectors (tests/golden/) + an independent numpy restatement
 *   repack ........ bijection / inverse round trip, GEMM(repacked) == GEMM(raw), hand fixtures
 *   GEMMs ......... closed-form permutation KAT in the style of kern-runtime/tests/mxfp8_gemm.rs:40-95
 *                   + float64 numpy matmul on the dequantized operands
 *   routing ....... invariants (each routed row exactly once, slots cover rows, totals consistent)
 *                   + brute-force stable sort
 */
#ifndef MXORACLE_H
#define MXORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- splitmix64 (crates/kern-test/src/workload.rs:11-26) ---- */
uint64_t mxo_splitmix64_next(uint64_t* state);
/* The i-th draw of a splitmix64 stream seeded with `seed` (0-based), computed directly. */
uint64_t mxo_splitmix64_at(uint64_t seed, uint64_t i);
/* N(0,1) from draws 2i and 2i+1: u1 = (d0>>11)*2^-53, u2 = (d1>>11)*2^-53,
 * z = sqrt(-2 ln(1-u1)) * cos(2*pi*u2). */
double mxo_normal_at(uint64_t seed, uint64_t i);

/* ---- element codecs ---- */
float mxo_e2m1_decode(uint8_t nibble);              /* tools/trtllm-bmm/probe.py:24-31 */
float mxo_e8m0_decode(uint8_t code);                /* crates/kern-manifest/src/values.rs:18-24 */
uint8_t mxo_e8m0_encode(double v);                  /* values.rs:115-135 */
float mxo_e4m3_decode(uint8_t code);                /* values.rs:81-89 */
uint8_t mxo_e4m3_encode_values_rs(double v);        /* values.rs:91-113 (half away from zero) */
/* Round-to-nearest-even, saturating e4m3fn encode of f32 bits scaled by 2^shift, computed exactly
 * in integers: the element rule of our MXFP8 quantizer. NaN -> 0x7f|sign, +-Inf -> +-448. */
uint8_t mxo_e4m3_encode_rne(uint32_t f32_bits, int shift);
float mxo_bf16_to_f32(uint16_t b);
uint16_t mxo_f32_to_bf16(float f);                  /* round to nearest even, NaN stays quiet NaN */

/* ---- bf16 -> MXFP8 quantizer (op moe_quant, fixtures/k3/head.json:25057; rule of
 * tools/trtllm-bmm/probe.py:38-43): per 32-element block, scale code
 * clamp(floor(log2 amax) - 8 + 127, 0, 254) (amax 0 -> code 0), codes = RNE-saturating e4m3 of
 * x / 2^(code-127); a block holding NaN/Inf gets scale 255 and codes 0x7f|sign.
 * x: bf16 [T, K]; q: u8 [T, K]; sf: u8 [T, K/32] row-major (linear). */
void mxo_quant_mxfp8(const uint16_t* x, int64_t T, int64_t K, uint8_t* q, uint8_t* sf);
/* The same rule for one block of 32 f32 values; writes 32 codes, returns the scale code. */
uint8_t mxo_quant_block32_f32(const float* v, uint8_t* q);

/* ---- weight repack (derive ops k3_moe_w_shuffle / k3_moe_sf_shuffle, head.json:26358, :26413) ----
 * raw w: u8 [E][rows][row_bytes] (K = 2*row_bytes, element 2j in the low nibble, probe.py:28);
 * raw sf: u8 [E][rows][sf_cols] (sf_cols = K/32).
 * Repacked row R of an expert holds raw row mxo_w_src_row(R, rows, gated): for gated (FC1 [up; gate]
 * rows, K3 binds w3 then w1, head.json:1161) each 4-row quad is gate n, gate n+1, up n, up n+1 with
 * n = 8*(R/16) + 2*((R%16)/4); otherwise the identity.
 * w layout: per expert, 1 KiB fragments ((R/16)*(K/128) + k/128), inside it lane
 * L = 16*((k%128)/32) + R%16 owns 16 bytes at L*16 holding k = 128*kt + 32*(L/16) .. +32.
 * sf layout: per expert, 256-byte fragments ((R/16)*(K/512) + k/512), lane L = 16*g + R%16 owns the
 * dword at L*4 whose byte j is the scale of row R, k-block 16*(k/512) + 4*j + g.
 * Requires rows % 16 == 0 and K % 512 == 0. Sizes are unchanged by the repack. */
int64_t mxo_w_src_row(int64_t R, int64_t rows, int gated);
int64_t mxo_w_offset(int64_t R, int64_t kbyte, int64_t rows, int64_t row_bytes); /* within one expert */
int64_t mxo_sf_offset(int64_t R, int64_t kblock, int64_t rows, int64_t sf_cols); /* within one expert */
void mxo_w_shuffle(const uint8_t* raw, uint8_t* out, int64_t E, int64_t rows, int64_t row_bytes, int gated);
void mxo_w_unshuffle(const uint8_t* in, uint8_t* raw, int64_t E, int64_t rows, int64_t row_bytes, int gated);
void mxo_sf_shuffle(const uint8_t* raw, uint8_t* out, int64_t E, int64_t rows, int64_t sf_cols, int gated);
void mxo_sf_unshuffle(const uint8_t* in, uint8_t* raw, int64_t E, int64_t rows, int64_t sf_cols, int gated);

/* ---- R128c4 scale layout (crates/kern-runtime/src/cublas.rs:396-400): rows padded to 128, k-blocks
 * to 4; entry (r, b) at 512*(r/128 * ceil(kblocks/4) + b/4) + (r%32)*16 + (r%128/32)*4 + b%4. */
int64_t mxo_r128c4_offset(int64_t r, int64_t b, int64_t kblocks);
int64_t mxo_r128c4_size(int64_t rows, int64_t kblocks);

/* ---- dequantization (probe.py:27-35) ---- */
/* raw (unrepacked) MXFP4 [N][K/2] + sf [N][K/32] -> f32 [N][K] */
void mxo_deq_fp4(const uint8_t* w, const uint8_t* sf, int64_t N, int64_t K, float* out);
/* e4m3 [T][K] + linear sf [T][K/32] -> f32 [T][K] */
void mxo_deq_fp8(const uint8_t* q, const uint8_t* sf, int64_t T, int64_t K, float* out);

/* ---- GEMM reference: C[t][n] = sum_k X[t][k] * W[n][k], f32 accumulation in ascending k ----
 * (the product of trtllm_bmm_* with one batch; row-major TN as cublas.rs:387-400) */
void mxo_gemm_f32(const float* X, const float* W, int64_t T, int64_t N, int64_t K, float* C, int nthreads);

/* W4A16 decode GEMV reference: y[t][n] = bf16( sum_k bf16(x[t][k]) * deq(W)[n][k] ), f32 accumulation,
 * with W given raw (unrepacked). */
void mxo_gemv_w4a16(const uint16_t* x, const uint8_t* w, const uint8_t* sf, int64_t M, int64_t N, int64_t K,
                    uint16_t* y, float* y_f32, int nthreads);

/* ---- activations ---- */
/* situ(g, u) = alpha*tanh(g/alpha)*sigmoid(g) * beta*tanh(u/beta)   (probe.py:23, :46-47) */
float mxo_situ(float g, float u, float alpha, float beta);
/* out[t][i] = bf16(bf16(g/(1+exp(-g))) * u), g = in[t][i], u = in[t][d+i]  (tools/kernels-src/silu_mul.cu:1-5) */
void mxo_silu_mul_bf16(const uint16_t* in, int64_t T, int64_t d, uint16_t* out);

/* Linear [rows][kblocks] scales gathered from the 128x4 tiled layout (cublas.rs:396-400). */
void mxo_r128c4_gather(const uint8_t* tiled, int64_t rows, int64_t kblocks, uint8_t* linear);

/* RoPE cache of weight_prep.cu: cos/sin[r*stride + j] = bf16(cos/sin(f32(r) * (1 / base^(2j/(2 half))))) */
void mxo_rope_table(uint16_t* cos_t, uint16_t* sin_t, int64_t rows, int64_t half, int64_t stride, float base);

/* MoE finalize: y[t] = sum_j w[t][j] * fc2[e2p[t*topk+j]] (j ascending, f32 FMAs, e2p < 0 skipped)
 * (tools/trtllm-bmm/probe.py:100-110); gamma == NULL: out = bf16(y), else out = bf16(y / sqrt(mean(y^2) +
 * eps) * gamma) (op moe_finalize_rms; parity unpinned: the reference kernel's source is absent). */
void mxo_moe_finalize(const uint16_t* fc2, const int32_t* e2p, const float* w, const uint16_t* gamma, int64_t T,
                      int64_t H, int topk, float eps, uint16_t* out);

/* ---- routing tables (tools/kernels/abi/trtllm_bmm.py:19-27, :50-60; op moe_routing head.json:25117) ----
 * topk_idx: i32 [T][topk] global expert ids. Local experts are [local_start, local_start+E_local).
 * Expanded index i = t*topk + j. For local expert e: counts[e] = rows routed to it; it owns
 * ceil(counts[e]/tile) consecutive CTA slots starting at slot_off[e] (exclusive scan in e order).
 * Rows of one expert are ordered by ascending expanded index. perm(i) = tile*slot_off[e] + rank.
 * Outputs: counts [2*E_local] (counts, then slot offsets); cta_batch/cta_limit [>= slots];
 * num_non_exiting[0] = slots; total_padded[0] = slots*tile; route_map [slots*tile] permuted row ->
 * token (-1 in padding); exp2perm [T*topk] expanded index -> permuted row (-1 if not local).
 * cta_limit[s] = min((s+1)*tile, tile*slot_off[e] + counts[e]) (one past the last valid row). */
void mxo_routing(const int32_t* topk_idx, int64_t T, int topk, int local_start, int E_local, int tile,
                 int32_t* counts, int32_t* cta_batch, int32_t* cta_limit, int32_t* num_non_exiting,
                 int32_t* total_padded, int32_t* route_map, int32_t* exp2perm);
/* Slot capacity the routing can need: min(E, T*k) + (T*k - min(E, T*k)) / tile (trtllm_bmm.py:50-55). */
int64_t mxo_max_ctas(int64_t tokens, int topk, int experts, int tile);

/* ---- grouped GEMM references over the routing tables (repacked weights, as the device reads them) ----
 * FC2 (trtllm_bmm_bf16_mxe2m1_mxe4m3, trtllm_bmm.py:19-27): for slot s < num_non_exiting, expert
 * e = cta_batch[s], rows p in [s*tile, cta_limit[s]): c[p][n] = bf16(sum_k deq(b)[p][k] * deq(a_e)[n][k]).
 * b is e4m3 [rows][k] with R128c4 scales over rows (sf_b_r128c4=1) or linear [rows][k/32].
 * acc_out (optional, may be NULL): f32 [rows][m] pre-rounding accumulators. */
void mxo_fc2(const uint8_t* a, const uint8_t* sf_a, const uint8_t* b, const uint8_t* sf_b, int sf_b_r128c4,
             int64_t rows_b, uint16_t* c, float* acc_out, const int32_t* num_non_exiting,
             const int32_t* cta_batch, const int32_t* cta_limit, int64_t m, int64_t k, int tile, int nthreads);
/* FC1 (trtllm_bmm_mxe4m3_mxe2m1_mxe4m3, gated SiTU-GLU, e4m3 out + ue8m0 block-32 R128c4 sf_c):
 * rows p of slot s gather b row route_map[p] (linear sf_b [T][k/32]); g/u are the gate/up
 * accumulators of output column n (m/2 columns); h = situ(g, u, alpha[e], beta[e]); c[p][:] and
 * sf_c = mxo_quant_block32_f32 over each 32 columns of h; sf_c in R128c4 over padded rows.
 * dbg (optional): f32 [padded][3][m/2] = gate acc, up acc, h. */
void mxo_fc1(const uint8_t* a, const uint8_t* sf_a, const uint8_t* b, const uint8_t* sf_b, uint8_t* c,
             uint8_t* sf_c, int64_t padded_rows, const int32_t* route_map, const float* alpha, const float* beta,
             float* dbg, const int32_t* num_non_exiting, const int32_t* cta_batch, const int32_t* cta_limit,
             int64_t m, int64_t k, int tile, int nthreads);
/* Dense e4m3-out mode (no gate): c[t][n] = e4m3_rne_sat(acc[t][n] * d_scale), acc over repacked
 * a [n][k] and linear-scaled b [t][k]; acc_out (optional) f32 [T][m]. */
void mxo_gemm_e4m3_pt(const uint8_t* a, const uint8_t* sf_a, const uint8_t* b, const uint8_t* sf_b, int64_t T,
                      int64_t m, int64_t k, float d_scale, uint8_t* c, float* acc_out, int nthreads);
/* RNE-saturating e4m3 of an f32 value (the per-tensor epilogue's cast), scalar and array forms. */
uint8_t mxo_e4m3_from_f32(float v);
void mxo_e4m3_from_f32_array(const float* v, int64_t n, uint8_t* out);
/* mxo_quant_block32_f32 over consecutive blocks of 32: codes q[32*nblocks], scales sf[nblocks]. */
void mxo_quant_blocks_f32(const float* v, int64_t nblocks, uint8_t* q, uint8_t* sf);

#ifdef __cplusplus
}
#endif
#endif
