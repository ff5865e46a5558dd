/* kern_amd — the C ABI of the MI355X-native MXFP4 matmul path.
 *
 * Two layers, both plain C (pointers, sizes, a hipStream_t passed as void*):
 *
 *  1. Module layer: the thin host->HIP layer that kern's runtime calls in place of its CUDA driver
 *     calls. It loads a SHA-256-pinned gfx950 code object, resolves entries, checks a launch's
 *     kernel-argument layout against the code object's own metadata, launches, and captures /
 *     replays hipGraphs.
 *  2. Op layer: one entry point per manifest op of the path, same parameter order and meaning as the
 *     op's `params` (fixtures/k3/head.json), plus the launch scalars the manifest launch supplies.
 *     Each entry point validates shapes on the host, then launches its kernel through layer 1 from
 *     the library's own pinned code object (kern_mx.hsaco).
 *
 * Every function returns KERN_OK (0) or a kern_status; kern_last_error() gives the message for the
 * calling thread. Device pointers must be on the device current on the calling thread. Calls are
 * asynchronous on `stream` (NULL = the null stream).
 */
#ifndef KERN_AMD_H
#define KERN_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes, grouped by who acts, as crates/kern-runtime/src/error.rs:5-67 groups its Error. */
typedef enum kern_status {
  KERN_OK = 0,
  KERN_ERR_MANIFEST = 1,        /* manifest inconsistency found past verification (error.rs:7-11) */
  KERN_ERR_KERNEL_ARTIFACT = 2, /* code object missing/unreadable, sha256 mismatch, param layout (error.rs:13-17) */
  KERN_ERR_WEIGHT_ARTIFACT = 3, /* weight bytes not as the op needs them (error.rs:19-23) */
  KERN_ERR_API = 4,             /* caller broke the contract: bad shape, null pointer, unknown name (error.rs:25-30) */
  KERN_ERR_DOMAIN = 6,          /* an input value outside the op's domain (error.rs:38-42) */
  KERN_ERR_CALL = 7,            /* one launch of a program failed; message carries the call context (error.rs:44-51) */
  KERN_ERR_HIP = 8              /* a HIP runtime call failed (error.rs:53-55, the CUDA variant) */
} kern_status;

/* Message of the last failed call on this thread ("" if none). */
const char* kern_last_error(void);

/* ------------------------------------------------------------------------------------------------
 * Module layer (replaces kern-runtime's CUDA driver calls)
 * ------------------------------------------------------------------------------------------------ */
typedef struct kern_module_s* kern_module;
typedef struct kern_function_s* kern_function;
typedef struct kern_graph_s* kern_graph;

/* Lower-case hex SHA-256 of `len` bytes into out[65]. (cubin.rs:62-109 pins modules by this digest) */
int kern_sha256_hex(const void* data, size_t len, char out[65]);

/* Load a code object image on the current device after checking its SHA-256 against `sha256_hex`
 * (64 hex chars; NULL skips the check). Replaces cuModuleLoadData in cubin.rs:226-263 and the
 * pinning of cubin.rs:70-109. */
int kern_module_load(const void* image, size_t len, const char* sha256_hex, kern_module* out);
int kern_module_unload(kern_module mod);

/* Resolve an entry (cuModuleGetFunction, compile.rs:313-445). */
int kern_module_function(kern_module mod, const char* entry, kern_function* out);

/* Explicit kernel-argument sizes of an entry, read from the code object's AMDGPU metadata (our own
 * build), in order: the analog of cuFuncGetParamInfo used by the ABI check in compile.rs:385-415.
 * Writes up to `cap` sizes; *n gets the count. */
int kern_function_param_sizes(kern_function fn, uint32_t* sizes, int cap, int* n);

/* Their byte offsets in the kernel-argument segment, from the same metadata. */
int kern_function_param_offsets(kern_function fn, uint32_t* offsets, int cap, int* n);

/* The same sizes read from a code object image in host memory, without a device (a manifest's
 * launches can be checked against an artifact before any GPU is touched). */
int kern_code_object_param_sizes(const void* image, size_t len, const char* entry, uint32_t* sizes, int cap,
                                 int* n);

/* The ABI check itself: KERN_ERR_KERNEL_ARTIFACT unless the entry's explicit arguments are exactly
 * `n` arguments of the given byte sizes (pointer 8, i32/f32 4, i64 8, bytes<n> n). */
int kern_function_check_params(kern_function fn, const uint32_t* sizes, int n);

/* Launch with a packed kernel-argument buffer laid out per the AMDGPU kernarg ABI (each argument at
 * its natural alignment). Replaces cuLaunchKernelEx (exec.rs:726-821). */
int kern_launch(kern_function fn, const uint32_t grid[3], const uint32_t block[3], uint32_t shared_bytes,
                void* stream, const void* kernargs, size_t kernargs_size);

/* hipGraph capture of everything enqueued on `stream` between begin and end, then replay
 * (exec.rs:489-548 record, :644-654 enqueue_captured). */
int kern_graph_begin(void* stream);
int kern_graph_end(void* stream, kern_graph* out);
int kern_graph_launch(kern_graph g, void* stream);
int kern_graph_destroy(kern_graph g);

/* Free a handle from kern_module_function (its kernel stays in the module). */
int kern_function_release(kern_function fn);

/* ------------------------------------------------------------------------------------------------
 * Manifest-op layer: one kern manifest op, run from its own JSON with its `impl` pointed at a module
 * loaded here. The op object is the value of one `ops` entry (crates/kern-manifest/src/types.rs:970-1040):
 * {"params": [...], "impl": {"launches": [{"module", "entry", "params"?, "block", "grid", "shared_mem"?,
 * "when"?, "args"?}, ...]}}, with grids and shared_mem as Expr trees over manifest vars
 * (types.rs:1517-1576), args as LaunchArg (types.rs:1174-1191) and packs of Fields (types.rs:1193-1260).
 * This is the module-swap of candidate::splice (crates/kern-manifest/src/candidate.rs:1-26): the op's
 * params and every call stay as they are; only `impl` names this module.
 * ------------------------------------------------------------------------------------------------ */
typedef struct kern_op_s* kern_op;

/* Parse and check an op (the checks of verify.rs:655-700: arg count, forwarded params matching their
 * launch params in kind and dtype, no writes through `in` params, no reads of `out` params before a
 * launch wrote them, packs filling exactly their bytes<n>), resolve each launch's entry in `mod`, which
 * the manifest's `modules` table names `module_name`, and check its params against the code object's
 * kernel-argument sizes (compile.rs:385-415). Extern launches, scratch buffers, rank args, TMA
 * descriptors, clusters and programmatic dependent launch have no gfx950 counterpart here:
 * KERN_ERR_MANIFEST. So is a launch of one of kern_mx's entries with a block other than the one its mapping
 * of threads to work is written for (the message names it; kern_op_plan and kern_op_verify refuse it too). */
int kern_op_create(const char* op_json, const char* module_name, kern_module mod, kern_op* out);
int kern_op_destroy(kern_op op);
int kern_op_num_params(kern_op op);   /* -1 for a null op */
int kern_op_num_launches(kern_op op);

/* Run the op's launches in order on `stream` (exec.rs:726-821), each only while its `when` holds.
 * params[i] is interface param i: a device address for a buffer, otherwise the scalar's bits in the
 * low bytes (i32 and f32 4, u8 1, i64 8). var_names/var_values bind the manifest vars the grids,
 * shared_mem, `when` and pack fields read. An unknown var, a grid beyond the launch limits or a failed
 * launch is KERN_ERR_CALL with the launch's context (compile.rs:725, exec.rs:707). */
int kern_op_launch(kern_op op, const uint64_t* params, int nparams, const char* const* var_names,
                   const uint64_t* var_values, int nvars, void* stream);

/* Host-only: parse an op's JSON and run the create-time checks that need no code object (the verifier's,
 * verify.rs:655-700): KERN_OK or KERN_ERR_MANIFEST with the reason. */
int kern_op_verify(const char* op_json);

/* Host-only: what kern_op_launch would do for one launch of an op (no device, no code object), for
 * checking a manifest against this ABI without a GPU: grid, block, dynamic LDS bytes and the
 * kernel-argument image (each argument at its natural alignment, bytes<n> aligned to n when n is 1, 2, 4
 * or 8 and to 8 otherwise, size rounded up to 8; kern_op_launch places arguments at the code object's
 * own offsets, which agree with this for every entry of kern_mx).
 * *skip = 1 when the launch's `when` does not hold (nothing else is written then). */
int kern_op_plan(const char* op_json, int launch_index, const uint64_t* params, int nparams,
                 const char* const* var_names, const uint64_t* var_values, int nvars, uint32_t grid[3],
                 uint32_t block[3], uint32_t* shared_bytes, void* kernargs, size_t cap, size_t* kernargs_size,
                 int* skip);

/* candidate::splice (crates/kern-manifest/src/candidate.rs:152-185): put a Candidate {modules, ops}
 * (candidate.rs:34-44; a manifest's `modules` and `ops` sections, each op under the name and with the params
 * of the op it replaces) into a manifest. Refused with KERN_ERR_MANIFEST, every reason listed ("candidate does
 * not fit: ..."), when an op is not in the manifest, its params differ from the manifest's, or one of its
 * launches names a module in neither; otherwise the candidate's modules are taken in (renamed
 * `<name>@<sha256[0:8]>` where the manifest pins other bytes under the name, candidate.rs:116-131), its ops
 * replace the manifest's with their launches renamed to match, and modules nothing launches are dropped. The
 * rest of the manifest is carried over as the same text. Writes the spliced manifest (NUL-terminated) to
 * out[cap] and its length (without the NUL) to *out_len; out NULL queries the length. The result is then
 * verified by kern_rt_check / kern_rt_load, as splice ends with verify(). */
int kern_candidate_splice(const char* manifest_json, const char* candidate_json, char* out, size_t cap,
                          size_t* out_len);

/* Building candidates (candidate.rs:83-113, :231-300). Each writes a Candidate {modules, ops} (JSON,
 * NUL-terminated; modules and ops in name order) to out[cap] and its length to *out_len; out NULL queries the
 * length. Misfits are KERN_ERR_MANIFEST with every reason listed ("candidate does not fit: ...").
 * kern_candidate_of (Candidate::of, :84-87): the manifest's own implementation of the n_ops ops named, with
 * the modules they launch; an op the manifest lacks is left out.
 * kern_candidate_only (Candidate::only, :89-97): the same cut of a candidate.
 * kern_candidate_join (Candidate::join, :99-113): n candidates as one; an op two of them implement is refused
 * ("op `X` is implemented twice"), and a module name two of them give to other bytes stays with the first and
 * is renamed <name>@<sha256[0:8]> in the others.
 * kern_candidate_tile (tile, :231-300): one implementation of `op` from n pieces, piece i running
 * pieces[i].candidate_json's implementation while `var` is in [min, max] (an end whose has_ flag is 0 is
 * open): each launch is narrowed to the piece's range (its own `when` on `var` intersected with it; dropped
 * when the two miss; refused when conditioned on another var; a lower end of 1 is no bound), modules are
 * adopted as by join, and a scratch name an earlier piece gives another dtype or shape becomes <name>@<i>,
 * in the piece's launch args too. Ranges are the caller's: overlapping pieces both run there, and a value no
 * piece covers runs nothing. Refused when no launch of any piece runs in its range. */
typedef struct kern_candidate_piece {
  const char* candidate_json;
  int32_t has_min, has_max;
  uint64_t min, max;
} kern_candidate_piece;
int kern_candidate_of(const char* manifest_json, const char* const* ops, int n_ops, char* out, size_t cap,
                      size_t* out_len);
int kern_candidate_only(const char* candidate_json, const char* const* ops, int n_ops, char* out, size_t cap,
                        size_t* out_len);
int kern_candidate_join(const char* const* candidates, int n, char* out, size_t cap, size_t* out_len);
int kern_candidate_tile(const char* op, const char* var, const kern_candidate_piece* pieces, int n, char* out,
                        size_t cap, size_t* out_len);

/* ------------------------------------------------------------------------------------------------
 * Program runtime (kern_amd/csrc/runtime.cpp): a kern manifest's buffers, modules, ops and programs,
 * run by program name with var values, as crates/kern-runtime's Runtime (src/lib.rs:137-236) runs them.
 * One runtime per device, one stream per runtime; every call binds the runtime's device on the calling
 * thread first (lib.rs:21-23) and calls on one runtime are serialized; graph capture is serialized
 * process-wide (exec.rs:435-440). The runtime owns every device allocation (compile.rs:289-307).
 * Served manifest subset: vars, buffers of kind input / output / inout / weight / source / workspace /
 * carry on the device, modules by file under kernels_dir pinned by sha256, ops whose launches name one
 * module, programs of one lane with `graph` / `derive`. States, topology, peers, exported or host-placed
 * buffers and extra lanes are KERN_ERR_MANIFEST. A buffer's checkpoint `bind` and a program's `batch` are
 * carried, not acted on: weights and sources are the caller's bytes (kern_rt_load_weight), vars the
 * caller's values.
 * ------------------------------------------------------------------------------------------------ */

typedef struct kern_runtime_s* kern_runtime;

/* Runtime::load (load.rs:44-72): parse and verify the manifest, load each module from kernels_dir (file
 * = the module's `source`, checked against its `sha256`), create its ops, allocate and zero every buffer
 * at its vars' maxima, and give input buffers pinned staging. */
int kern_rt_load(const char* manifest_json, const char* kernels_dir, int gpu, kern_runtime* out);
int kern_rt_destroy(kern_runtime rt);
/* The same parse and verification on the host: module files are read and their sha256 checked, ops
 * verified (kern_op_verify), nothing is created on a device. */
int kern_rt_check(const char* manifest_json, const char* kernels_dir);

/* Runtime::write_input / read_output (lib.rs:288-330): len bytes from the start of an input / inout
 * buffer (through its pinned staging) or an output / inout buffer; len <= the buffer's bytes. */
int kern_rt_write_input(kern_runtime rt, const char* name, const void* data, size_t len);
int kern_rt_read_output(kern_runtime rt, const char* name, void* data, size_t len);
/* Harness access to any buffer (harness.rs:30-69). */
int kern_rt_write_buffer(kern_runtime rt, const char* name, size_t offset, const void* data, size_t len);
int kern_rt_read_buffer(kern_runtime rt, const char* name, size_t offset, void* data, size_t len);
/* A weight or source buffer's bytes, whole (what load_weights binds from a checkpoint, load.rs:336). */
int kern_rt_load_weight(kern_runtime rt, const char* name, const void* data, size_t len);
/* Run every derive program once, in manifest order, then free the source buffers (derive.rs:72-78).
 * Required before any other program runs when the manifest has derive programs. */
int kern_rt_derive(kern_runtime rt);

/* Runtime::run (exec.rs:409-448): issue the program as its manifest says (a `graph` program through its
 * hipGraph, captured at these var values on first use), then synchronize. var_names / var_values bind
 * manifest vars (each <= its max). A failed launch is KERN_ERR_CALL with "program `p` call #i (label, op
 * `o`): op launch #j (entry): ..." (compile.rs:725, exec.rs:707). */
int kern_rt_run(kern_runtime rt, const char* program, const char* const* var_names, const uint64_t* var_values,
                int nvars);
/* Runtime::capture / run_captured (exec.rs:489-548, :636-654): capture the program at these var values
 * (replacing an earlier graph at the same values); replay a captured graph and synchronize. */
int kern_rt_capture(kern_runtime rt, const char* program, const char* const* var_names, const uint64_t* var_values,
                    int nvars);
int kern_rt_run_captured(kern_runtime rt, const char* program, const char* const* var_names,
                         const uint64_t* var_values, int nvars);
/* Runtime::time_captured (harness.rs:252-266): the median milliseconds of one replay over iters back-to-back
 * replays, an event between each. */
int kern_rt_time_captured(kern_runtime rt, const char* program, const char* const* var_names,
                          const uint64_t* var_values, int nvars, int iters, float* ms_per_iter);
/* Runtime::run_range (harness.rs:186-207): calls [lo, hi) of a (non-derive) program, issued eagerly, then
 * synchronize. A range outside 0..calls is KERN_ERR_API. */
int kern_rt_run_range(kern_runtime rt, const char* program, const char* const* var_names, const uint64_t* var_values,
                      int nvars, int lo, int hi);
/* Runtime::time_range (harness.rs:209-250): ms_per_call[i] = the GPU milliseconds of call lo + i, issued
 * eagerly between events, minimum over iters runs of just calls [lo, hi) (a launch gap counts towards the call
 * after it, as in the reference). ms_per_call holds hi - lo floats. */
int kern_rt_time_range(kern_runtime rt, const char* program, const char* const* var_names, const uint64_t* var_values,
                       int nvars, int lo, int hi, int iters, float* ms_per_call);
int kern_rt_synchronize(kern_runtime rt);
/* A buffer's device address and bytes (Runtime::buffer_sizes, lib.rs:243). */
int kern_rt_buffer(kern_runtime rt, const char* name, void** device_ptr, size_t* bytes);

/* ------------------------------------------------------------------------------------------------
 * Op layer. The library loads its code object kern_mx.hsaco (next to libkern_amd.so unless
 * kern_init names another path) on first use per device and checks the SHA-256 it was built with.
 * ------------------------------------------------------------------------------------------------ */

/* Optional explicit init: path of kern_mx.hsaco (NULL = next to the library). */
int kern_init(const char* code_object_path);
/* SHA-256 the library pins its code object to (64 hex chars). */
const char* kern_code_object_sha256(void);
/* The library's own module (kern_mx.hsaco, pinned) on the current device, loaded on first use; owned
 * by the library. This is the module a manifest binds as `kern_mx` for kern_op_create. */
int kern_mx_module(kern_module* out);

/* moe_quant (fixtures/k3/head.json:25057; rule tools/trtllm-bmm/probe.py:38-43):
 * in bf16 x[T][K], out u8 q[T][K] (e4m3), out u8 sf[T][K/32] (ue8m0, linear), i32 T; launch i32 K.
 * Per 32-block: scale = clamp(floor(log2 amax) - 8 + 127, 0, 254), codes RNE-saturating e4m3.
 * K % 32 == 0. */
int kern_moe_quant(const void* x, void* q, void* sf, int32_t tokens, int32_t K, void* stream);

/* f32 -> MXFP8 with the FC1 epilogue's codec (the MXFP8 output stage of trtllm_bmm_mxe4m3_mxe2m1_mxe4m3,
 * head.json:25459, whose sf_c rule is probe.py:38-43's): in f32 x[T][K], out u8 q[T][K] (e4m3), out u8
 * sf[T][K/32] (ue8m0, linear); same scale and element rules as kern_moe_quant, applied to f32 values
 * (an f32 subnormal or a value between bf16 neighbours is encoded from its exact value). K % 32 == 0. */
int kern_mxfp8_quant_f32(const float* x, void* q, void* sf, int32_t tokens, int32_t K, void* stream);

/* k3_moe_w_shuffle (head.json:26358; derive program head.json:28670): in u8 raw [E][rows][row_bytes],
 * out u8 repacked (same size), i32 rows, i32 row_bytes, i32 gated; launch i32 E.
 * rows % 16 == 0, row_bytes % 256 == 0 (K % 512 == 0). */
int kern_moe_w_shuffle(const void* raw, void* out, int32_t experts, int32_t rows, int32_t row_bytes,
                       int32_t gated, void* stream);

/* k3_moe_sf_shuffle (head.json:26413): in u8 raw [E][rows][sf_cols], out u8 repacked, i32 rows,
 * i32 sf_cols, i32 gated; launch i32 E. rows % 16 == 0, sf_cols % 16 == 0. */
int kern_moe_sf_shuffle(const void* raw, void* out, int32_t experts, int32_t rows, int32_t sf_cols,
                        int32_t gated, void* stream);

/* moe_routing (head.json:25117; tables of tools/kernels/abi/trtllm_bmm.py:19-27, :50-60):
 * in i32 topk_idx[tokens][topk] -> out counts[2*local_experts], cta_batch[ctas], cta_limit[ctas],
 * num_non_exiting[1], total_padded[1], route_map[ctas*128], exp2perm[tokens*topk].
 * ctas = local_experts + ceil(tokens*topk/128) bounds the slots. local_experts <= 512,
 * tokens*topk + 128*local_experts <= INT32_MAX (the padded rows are i32). At tokens = 0 the tables still
 * come out (no live slots) and topk_idx / exp2perm may be null. One launch below 16384 expanded ids, else
 * three (min(64, ceil(ids/4096)) workgroups; exp2perm holds per-chunk counts between them), all on `stream`. */
int kern_moe_routing(const int32_t* topk_idx, int32_t* counts, int32_t* cta_batch, int32_t* cta_limit,
                     int32_t* num_non_exiting, int32_t* total_padded, int32_t* route_map, int32_t* exp2perm,
                     int32_t tokens, int32_t topk, int32_t local_start, int32_t local_experts, void* stream);

/* moe_quant and moe_routing in one call: the outputs of kern_moe_quant(x, q, sf, tokens, K) and of
 * kern_moe_routing(topk_idx, ..., tokens, topk, local_start, local_experts), bit for bit, with the same
 * argument rules. No counterpart in the reference, which runs the two ops (head.json:25057, :25117) as
 * two launches: for callers that run both back to back on the same tokens, such as a decode step, where
 * each launch is mostly launch and memory latency. One launch when the quantizer needs at most 255
 * workgroups of 1024 lanes (tokens * K <= 4,177,920), else the two launches. */
int kern_moe_quant_routing(const void* x, void* q, void* sf, int32_t tokens, int32_t K, const int32_t* topk_idx,
                           int32_t* counts, int32_t* cta_batch, int32_t* cta_limit, int32_t* num_non_exiting,
                           int32_t* total_padded, int32_t* route_map, int32_t* exp2perm, int32_t topk,
                           int32_t local_start, int32_t local_experts, void* stream);

/* trtllm_bmm_bf16_mxe2m1_mxe4m3 = moe_fc2 (head.json:25683; interface trtllm_bmm.py:19-27):
 * a u8 [E][m][k/2] repacked MXFP4, sf_a repacked, b u8 [rows][k] e4m3, sf_b (R128c4 over rows when
 * sf_b_r128c4, else linear [rows][k/32]), c bf16 [rows][m], num_non_exiting, total_padded, cta_batch,
 * cta_limit; launch: m, k, ctas (grid.y, the manifest's E + ceil(tokens*topk/128)), and dbg (NULL or
 * f32 [rows][m] pre-rounding accumulators). m % 256 == 0, k % 512 == 0; the activations (ctas * 128
 * rows of k bytes) below 4 GiB, as the kernel addresses them by 32-bit offsets (KERN_ERR_API otherwise). */
int kern_trtllm_bmm_bf16_mxe2m1_mxe4m3(const void* a, const void* sf_a, const void* b, const void* sf_b, void* c,
                                       const int32_t* num_non_exiting, const int32_t* total_padded,
                                       const int32_t* cta_batch, const int32_t* cta_limit, int32_t m, int32_t k,
                                       int32_t ctas, int32_t sf_b_r128c4, float* dbg, void* stream);

/* trtllm_bmm_mxe4m3_mxe2m1_mxe4m3 = moe_fc1 (head.json:25459): a (gated repack), sf_a, b u8 [T][k]
 * e4m3, sf_b linear [T][k/32], c u8 [rows][m/2] e4m3, sf_c u8 R128c4 over rows x (m/2)/32, route_map,
 * alpha f32[E], beta f32[E], num_non_exiting, total_padded, cta_batch, cta_limit; launch m, k, ctas,
 * dbg (NULL or f32 [rows][3][m/2] = gate acc, up acc, SiTU-GLU value). m % 256 == 0, k % 512 == 0, and
 * T * k below 2^32 (the kernel addresses the activations by 32-bit offsets; T is not passed, so this one
 * is the caller's to keep: T < 599,186 tokens at k = 7168). */
int kern_trtllm_bmm_mxe4m3_mxe2m1_mxe4m3(const void* a, const void* sf_a, const void* b, const void* sf_b, void* c,
                                         void* sf_c, const int32_t* route_map, const float* alpha,
                                         const float* beta, const int32_t* num_non_exiting,
                                         const int32_t* total_padded, const int32_t* cta_batch,
                                         const int32_t* cta_limit, int32_t m, int32_t k, int32_t ctas, float* dbg,
                                         void* stream);

/* Dense e4m3-output mode of the FC1 family (no gate, per-tensor output scale), the prefill GEMM:
 * c[t][n] = e4m3_rne_sat(acc[t][n] * d_scale[0]); a/sf_a repacked [m][k], b u8 [M][k], sf_b linear,
 * c u8 [M][m], d_scale f32[1] on the device; dbg NULL or f32 [M][m]. M * k below 2^32. */
int kern_mxfp4_gemm_e4m3(const void* a, const void* sf_a, const void* b, const void* sf_b, void* c,
                         const float* d_scale, int32_t M, int32_t m, int32_t k, float* dbg, void* stream);

/* Dense bf16-output mode of the FC2 family: c bf16 [M][m]. M * k below 2^32. */
int kern_mxfp4_gemm_bf16(const void* a, const void* sf_a, const void* b, const void* sf_b, void* c, int32_t M,
                         int32_t m, int32_t k, float* dbg, void* stream);

/* mxfp4_gemv_bf16 (new op; the W4A16 decode, no reference counterpart): in bf16 x[M][K], in u8 w
 * repacked [N][K/2], in u8 w_sf repacked, out bf16 y[M][N], i32 M (1..16); launch N, K.
 * N % 16 == 0, K % 512 == 0, K <= 16384. */
int kern_mxfp4_gemv_bf16(const void* x, const void* w, const void* w_sf, void* y, int32_t M, int32_t N, int32_t K,
                         void* stream);

/* extern:cublaslt_mxfp8_tn (crates/kern-runtime/src/cublas.rs:387-400; args [a, w, c, a_scale, w_scale, m,
 * n, k, ldc]): c bf16 [m][ldc] = sum_k deq(a)[m][k] * deq(w)[n][k], a [m][k] and w [n][k] e4m3, scales
 * e8m0 per 32 of K in the 128x4 tiled layout (rows padded to 128, k blocks to 4). k % 32 == 0,
 * ldc >= n, operands below 2 GiB. f32 accumulation, bf16 RNE out. */
int kern_mxfp8_gemm_bf16(const void* a, const void* w, void* c, const void* a_sf, const void* w_sf, int32_t m,
                         int32_t n, int32_t k, int32_t ldc, void* stream);

/* silu_mul (tools/kernels-src/silu_mul.cu:1-36, kernel ABI (out, in, d), grid [tokens, ceil(d/2048)]):
 * out bf16 [tokens][d] = bf16(bf16(g / (1 + exp(-g))) * u), g = in[t][i], u = in[t][d + i], in bf16
 * [tokens][2d]. d % 8 == 0. */
int kern_silu_mul(void* out, const void* in, int32_t tokens, int32_t d, void* stream);

/* moe_finalize_rms (fixtures/k3/head.json op moe_finalize_rms, call l1.finalize: fc2_out, exp2perm,
 * topk_weight, gamma, out, tokens; the launch adds H, topk and eps): y[t] = sum_j topk_weight[t][j] *
 * fc2_out[exp2perm[t*topk + j]] in j order with f32 FMAs (exp2perm < 0: a non-local expert, skipped),
 * the combine of tools/trtllm-bmm/probe.py:100-110; out[t] = bf16(y / sqrt(mean(y^2) + eps) * gamma).
 * 0 < H <= 8192, H % 8 == 0. The reference kernel's source is not in its tree: the norm's eps and weight
 * convention are this build's. */
int kern_moe_finalize_rms(const void* fc2_out, const int32_t* exp2perm, const float* topk_weight, const void* gamma,
                          void* out, int32_t tokens, int32_t H, int32_t topk, float eps, void* stream);

/* The same combine without the norm: out[t] = bf16(y) (flashinfer's do_finalize, probe.py:85-110). */
int kern_moe_finalize(const void* fc2_out, const int32_t* exp2perm, const float* topk_weight, void* out,
                      int32_t tokens, int32_t H, int32_t topk, void* stream);

/* weight_prep family (tools/kernels-src/weight_prep.cu:1-70): the derived tables a manifest's `once`
 * program builds after load; same entries and one-thread-per-element mapping as the reference's module,
 * here launched with 256-thread workgroups over n elements.
 *   weight_p1_bf16_f32: out[i] = f32(w[i]) + 1      cast_bf16_f32: out[i] = f32(w[i])
 *   rope_table_bf16:    cos/sin[r*stride + j] = bf16(cos/sin(r / base^(2j/(2 half)))), r < rows, j < half
 *   fill_{f32,i32,i64,u8,bf16}: p[i] = v (bf16: RNE of v; fill_bf16 is K3's k3_weight_prep entry)
 *   iota_i32:           p[i*stride] = start + i*step */
int kern_weight_p1_bf16_f32(const void* w, float* out, int32_t n, void* stream);
int kern_cast_bf16_f32(const void* w, float* out, int32_t n, void* stream);
int kern_rope_table_bf16(void* cos_t, void* sin_t, int32_t rows, int32_t half, int32_t stride, float base,
                         void* stream);
int kern_fill_f32(float* p, int32_t n, float v, void* stream);
int kern_fill_i32(int32_t* p, int32_t n, int32_t v, void* stream);
int kern_fill_i64(int64_t* p, int32_t n, int64_t v, void* stream);
int kern_fill_u8(uint8_t* p, int32_t n, int32_t v, void* stream);
int kern_fill_bf16(void* p, int32_t n, float v, void* stream);
int kern_iota_i32(int32_t* p, int32_t n, int32_t start, int32_t step, int32_t stride, void* stream);

/* Seeded synthetic bytes: out[i] = lo + splitmix64_i(seed) % span (crates/kern-test/src/workload.rs:11-26). */
int kern_fill_random_u8(void* out, int64_t n, uint64_t seed, int32_t lo, int32_t span, void* stream);

#ifdef __cplusplus
}
#endif
#endif
