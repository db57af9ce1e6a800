/* q36moe -- MI355X (gfx950) W4A8 mixture-of-experts layer, C ABI.
 *
 * Drop-in for the MoE FFN of the q36 engine: router logits in, combined
 * hidden state out.  Plain pointers and sizes only; every device pointer is
 * a HIP device allocation owned by the caller unless stated otherwise, and
 * every stream is a hipStream_t passed as void*.
 *
 * Reference interfaces replaced (file:line in the q36 tree):
 *   q36moe_weights_upload  <- upload() MXFP4 expert branch, q36_engine.cu:196-228
 *                             (GGUF block_mxfp4 [E][M][K/32], q36.h:112-114)
 *   q36moe_weights_upload_typed
 *                          <- upload() with its Q5_K / Q6_K expert branch,
 *                             q36_engine.cu:229-252 (requantised to q8_0-split,
 *                             h_q8_row :73-86); the down projection of such
 *                             experts runs as k_gemm_expert_i8 (:2526-2618)
 *                             after k_quant_q8b (:2627-2640)
 *   q36moe_requant_q8      <- that branch's host repack, one matrix
 *   q36moe_ctx_create      <- MoE scratch allocated in q36_engine_create,
 *                             q36_engine.cu:1467-1512 (no allocation in forward)
 *   q36moe_forward         <- moe_ffn, q36_engine.cu:1592-1654 (decode) and
 *                             pf_moe_block, q36_engine.cu:3423-3472 (prefill),
 *                             starting after the router matvec
 *   q36moe_router_topk     <- k_router_topk, q36_ops.cuh:397-431
 *   q36moe_router_logits   <- the router matvec at the top of moe_ffn,
 *                             k_matvec_f32_row (q36_engine.cu:1602,
 *                             q36_ops.cuh:331-342), and pf_gemm's fp16
 *                             tensor-core GEMM for prefill (q36_engine.cu:3427,
 *                             :3403-3414)
 *   q36moe_quant_e4m3      <- k_quant_e4m3, q36_engine.cu:2411-2428
 *   q36moe_ctx_copy_tap    <- the Q36_DEBUG routing dumps, q36_engine.cu:1648-1653
 *   q36moe_probe_mfma      <- the block-scaled MMA calibration harness,
 *                             test_mma_bs.cu:46-69
 *
 * Errors are returned, never exit(): 0 ok, Q36MOE_EINVAL for bad arguments,
 * Q36MOE_ENOMEM for failed allocations, Q36MOE_EHIP for a HIP runtime error
 * (the reference prints and exits instead, q36_engine.cu:45).
 */
#ifndef Q36MOE_H
#define Q36MOE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define Q36MOE_OK       0
#define Q36MOE_EINVAL (-22)
#define Q36MOE_ENOMEM (-12)
#define Q36MOE_EHIP   (-1000)
#define Q36MOE_EIO    (-5)    /* the file could not be opened or mapped */
#define Q36MOE_ENOENT (-2)    /* no such tensor / metadata key          */

/* activation / output element formats */
#define Q36MOE_FMT_F32  0
#define Q36MOE_FMT_BF16 1

/* debug taps (q36moe_ctx_copy_tap) */
#define Q36MOE_TAP_TOPK_IDX  0  /* int32 [T][k]                         */
#define Q36MOE_TAP_TOPK_W    1  /* f32   [T][k]                         */
#define Q36MOE_TAP_XQ        2  /* u8    [T][d_model]  e4m3             */
#define Q36MOE_TAP_XS        3  /* u8    [T][d_model/32] E8M0           */
#define Q36MOE_TAP_EOFF      4  /* int32 [n_expert+1] sorted offsets    */
#define Q36MOE_TAP_PERM      5  /* int32 [T*k] entry id per sorted slot */
#define Q36MOE_TAP_POS       6  /* int32 [T*k] sorted slot per entry    */
#define Q36MOE_TAP_HQ        7  /* u8    [T*k+T][d_ff] e4m3 SwiGLU rows
                                   (int8 for q8_0-split down matrices)  */
#define Q36MOE_TAP_HS        8  /* u8    [T*k+T][d_ff/32] E8M0          */
#define Q36MOE_TAP_DNW       9  /* f32   [T*k+T][d_model] w * down rows
                                   (staged as f16 with a power-of-two
                                   scale per 16 columns; widened here);
                                   rows in sorted order, or in entry
                                   order (t*k+s, then n+t for the shared
                                   expert) when last_path is 3 and
                                   T*k <= 4096 (tiles found in-kernel) */
#define Q36MOE_TAP_HSF      10  /* f32   [T*k+T][d_ff/32] int8 h scales
                                   (q8_0-split down; HQ then holds int8) */
#define Q36MOE_TAP_XQ8      11  /* i8    [T][d_model] int8 x of a q8_0-split
                                   shared expert (sorted path)           */
#define Q36MOE_TAP_XSF      12  /* f32   [T][d_model/32] its scales      */

typedef struct q36moe_weights q36moe_weights;
typedef struct q36moe_ctx q36moe_ctx;

/* Library version string and the number of bytes one expert occupies on
 * the device (gate+up+down, nibbles + E8M0). */
const char *q36moe_version(void);
size_t q36moe_expert_bytes(int d_model, int d_ff);

/* Upload one layer's expert weights given as host GGUF block_mxfp4 arrays:
 * gate/up [n_expert][d_ff][d_model/32], down [n_expert][d_model][d_ff/32]
 * (17-byte blocks).  sh_* are the dense shared expert (same block layout,
 * one matrix each, d_ff_sh rows) or all NULL with d_ff_sh = 0.  The blocks
 * are repacked into the device fragment layout inside this call.
 * Constraints: d_model and d_ff multiples of 512, d_ff_sh 0 or == d_ff,
 * 1 <= n_expert <= 256.  E8M0 bytes of 255 (NaN in OCP MX) -> EINVAL. */
int q36moe_weights_upload(const void *gate, const void *up, const void *down,
                          const void *sh_gate, const void *sh_up, const void *sh_down,
                          int n_expert, int d_model, int d_ff, int d_ff_sh,
                          q36moe_weights **out);

/* As q36moe_weights_upload, with the routed down projection and the shared
 * expert in any of the reference's expert types.  down_type is the ggml type
 * of `down` -- 39 MXFP4 (the call above), 13 Q5_K, 14 Q6_K (super-blocks of
 * 256, so d_ff % 256 == 0) or 8 Q8_0 -- as [n_expert][d_model][row blocks];
 * sh_type the type of all three shared matrices (the release file's are
 * Q8_0).  A Q5_K / Q6_K matrix is dequantised and requantised on the host to
 * int8 codes with one f16 scale per 32 (the reference's q8_0-split layout),
 * a Q8_0 one is split as it is.  Activations feeding such a matrix are
 * quantised per 32 to int8 with an fp32 scale (d = amax/127; h for a
 * q8_0-split down, and x for a q8_0-split shared expert) and the product runs
 * on int8 MFMA, each 32-block's integer dot product scaled by both scales.
 * A q8_0-split shared expert refuses q36moe_forward_q8 (its x must be the
 * unquantised input): EINVAL. */
int q36moe_weights_upload_typed(const void *gate, const void *up, const void *down, int down_type,
                                const void *sh_gate, const void *sh_up, const void *sh_down, int sh_type,
                                int n_expert, int d_model, int d_ff, int d_ff_sh,
                                q36moe_weights **out);
/* ggml type of the routed down projection of w as uploaded (39 or 8), and
 * of its shared expert (39, 8, or 0 without one). */
int q36moe_weights_down_type(const q36moe_weights *w);
int q36moe_weights_shared_type(const q36moe_weights *w);

/* Allocate a weight set on the device without filling it; the caller fills
 * the packed buffers returned by q36moe_weights_device_ptrs (e.g. with
 * random bytes for synthetic benchmarks).  Packed layout per matrix:
 * [M*K/2 nibble bytes][M*K/32 E8M0 bytes]; per expert stride for gate/up/down
 * is the matrix size. */
int q36moe_weights_alloc(int n_expert, int d_model, int d_ff, int d_ff_sh,
                         q36moe_weights **out);
/* Device addresses of the packed matrices.  gate_bytes / down_bytes are one
 * routed gate (= up) / down matrix, the per-expert stride; a shared matrix
 * is gate_bytes in MXFP4, or d_model*d_ff*17/16 when
 * q36moe_weights_shared_type gives Q8_0 (int8 codes + f16 per 32). */
int q36moe_weights_device_ptrs(const q36moe_weights *w, void **gate, void **up,
                               void **down, void **sh_gate, void **sh_up,
                               void **sh_down, size_t *gate_bytes, size_t *down_bytes);
void q36moe_weights_free(q36moe_weights *w);

/* Fill every packed matrix of w on the device with seeded synthetic MXFP4
 * data: E2M1 codes uniform over the 16 values, E8M0 exponent bytes uniform
 * in [127+exp_lo, 127+exp_hi] (a counter-based hash of seed and byte index,
 * so the same seed gives the same bytes).  For benchmarks that need many
 * distinct layers resident in HBM. */
int q36moe_weights_fill_synthetic(q36moe_weights *w, uint64_t seed, int exp_lo, int exp_hi,
                                  void *stream);

/* Host-side repack of one [M][K] GGUF block_mxfp4 matrix into the packed
 * device layout (and back).  Pure host code; used by upload and by tests. */
int q36moe_pack_mxfp4(const void *gguf_blocks, int M, int K, void *packed);
int q36moe_unpack_mxfp4(const void *packed, int M, int K, void *gguf_blocks);

/* Host-side: one [M][K] matrix of GGUF blocks of ggml_type (8 Q8_0, 13
 * Q5_K, 14 Q6_K) to the q8_0-split layout: codes [M][K] int8 and f16
 * scales [M][K/32] (bit patterns), value = scale * code.  Q5_K / Q6_K are
 * dequantised exactly as q36_dequant.cuh:128-165 and requantised per 32
 * with d = amax/127 rounded to f16 and codes rint(v * (1/d)) clamped to
 * [-128, 127] (h_q8_row, q36_engine.cu:73-86). */
int q36moe_requant_q8(int ggml_type, const void *src, int M, int K, int8_t *codes, uint16_t *scales);
/* Host-side repack of a q8_0-split matrix into the packed device layout
 * (M*K code bytes then M*K/16 scale bytes), and back.  An inf/NaN scale
 * -> EINVAL.  M % 16 == 0, K % 64 == 0. */
int q36moe_pack_q8(const int8_t *codes, const uint16_t *scales, int M, int K, void *packed);
int q36moe_unpack_q8(const void *packed, int M, int K, int8_t *codes, uint16_t *scales);

/* Context: per-stream scratch for up to max_tokens tokens.  All scratch is
 * allocated here; q36moe_forward allocates nothing. */
int q36moe_ctx_create(int max_tokens, int n_expert, int d_model, int d_ff,
                      int top_k, void *stream, q36moe_ctx **out);
int q36moe_ctx_set_stream(q36moe_ctx *c, void *stream);
void q36moe_ctx_free(q36moe_ctx *c);

/* The MoE layer.  x [T][d_model] (f32 or bf16, row stride d_model),
 * logits [T][ld_logits] f32 (first n_expert columns used), shg the
 * shared-expert gate logits or NULL: token t's at shg[t * ld_shg] (ld_shg 0
 * means 1; the reference's batched decode keeps it as column 256 of each
 * 257-wide router row, q36_engine.cu:2092-2095, which is shg = logits + 256,
 * ld_shg = 257), out [T][d_model] (f32 or bf16).
 * out[t] = sum_s w[t][s] * E_{idx[t][s]}(x[t]) + sigmoid(shg[t*ld_shg]) * S(x[t]),
 * E(x) = down . q8(silu(gate . q8(x)) * up . q8(x)), q8 = per-32 E8M0 +
 * e4m3 quantisation, w = top-k softmax weights renormalised, times scale.
 * A matrix uploaded in the q8_0-split layout (q36moe_weights_upload_typed)
 * takes its activation quantised per 32 to int8 + fp32 scale instead.
 * Asynchronous on the context stream; T = 0 is a no-op. */
int q36moe_forward(q36moe_ctx *c, const q36moe_weights *w,
                   const void *x, int x_fmt, const float *logits, int ld_logits,
                   const float *shg, int ld_shg, int T, float scale, void *out, int out_fmt);

/* q36moe_forward without a context and without allocating anything: the
 * scratch is a static device array in the library (8 MiB per GPU it runs
 * on, held until the process ends), so a caller that cannot allocate -- code
 * under HIP graph capture, a tight serving loop, a harness that forbids
 * hipMalloc -- can still run the layer.  No counterpart in the reference
 * (its engine allocates once at create time).  Same arguments and result as
 * q36moe_forward on a context with top_k and the automatic path, for T <=
 * 64 tokens (larger T: EINVAL); asynchronous on `stream`.  Every call on a
 * GPU shares that GPU's array: calls that overlap on one GPU (two streams,
 * two threads) race and must be serialised by the caller.  No tap or replay
 * reads this scratch. */
int q36moe_forward_noalloc(const q36moe_weights *w, const void *x, int x_fmt, const float *logits, int ld_logits,
                           const float *shg, int ld_shg, int T, int top_k, float scale, void *out, int out_fmt,
                           void *stream);

/* Stage entry points (device pointers, asynchronous on `stream`). */
int q36moe_router_topk(const float *logits, int T, int n_expert, int ld, int k,
                       float scale, int renorm, int32_t *idx, float *wt, void *stream);
/* Router logits: logits[t][r] = w[r] . x[t] for r < n_expert (row stride
 * ld); with n_rows == n_expert + 1 the last row is the shared-expert gate
 * and goes to shg[t].  w [n_rows][d_model] f32 (device), x [T][d_model]
 * f32|bf16, d_model == 2048.  mode 1: fp32 products and sums (the decode
 * matvec); 2: w and x rounded to fp16, fp32 accumulation (the prefill
 * GEMM); 0: mode 1 for T <= 16, else 2. */
int q36moe_router_logits(const float *w, int n_rows, int n_expert, const void *x, int x_fmt, int T,
                         int d_model, int mode, float *logits, int ld, float *shg, void *stream);

int q36moe_quant_e4m3(const void *x, int x_fmt, int T, int K,
                      uint8_t *xq, uint8_t *xs, void *stream);

/* The producer of the MoE input in one pass: residual add, RMSNorm and the
 * per-32 E8M0 + e4m3 quantisation (replaces k_add_rmsnorm + k_quant_e4m3,
 * q36_engine.cu:696-706 and :2411-2428; k_rmsnorm_b, :3230-3240, when a is
 * NULL).  For each token t (rows of d_model == 2048 f32, device pointers):
 *   if a: h[t] += a[t] (written back);  y[t] = h[t] * rsqrt(mean(h[t]^2) + eps) * w
 * y [T][d_model] f32 is written when non-NULL (the router input); xq
 * [T][d_model] e4m3 and xs [T][d_model/32] E8M0 when non-NULL (the MoE input
 * of q36moe_forward_q8).  Asynchronous on `stream`. */
int q36moe_add_rmsnorm_quant(float *h, const float *a, const float *w, int T, int d_model,
                             float eps, float *y, uint8_t *xq, uint8_t *xs, void *stream);

/* q36moe_forward on activations already quantised by
 * q36moe_add_rmsnorm_quant (or q36moe_quant_e4m3): xq [T][d_model] e4m3,
 * xs [T][d_model/32] E8M0, device pointers that must stay valid until the
 * forward has run (and while its XQ/XS taps are read).  Same result as
 * q36moe_forward on the x they were quantised from.  EINVAL with shg for a
 * q8_0-split shared expert (it quantises the unquantised x itself). */
int q36moe_forward_q8(q36moe_ctx *c, const q36moe_weights *w, const uint8_t *xq, const uint8_t *xs,
                      const float *logits, int ld_logits, const float *shg, int ld_shg, int T,
                      float scale, void *out, int out_fmt);

/* Execution path of q36moe_forward.  The sorted path (route + sort + grouped
 * expert GEMMs + combine) serves any T, with fat tiles (up to 160 rows per
 * expert tile, weights staged through LDS) or skinny tiles (up to 32 rows,
 * weights streamed straight into registers); the direct path (no sort,
 * slots combined in registers) serves T <= 16 as two kernels (gate/up, then
 * down).  Skinny tiles run either as one kernel per tile (gate/up, h kept
 * in LDS, down) or as separate gate/up and down kernels; the one-kernel
 * form needs MXFP4 down and shared-expert matrices.  mode 0 picks the
 * direct path for T <= 16, skinny tiles (one kernel per tile where it
 * applies) while T*k <= 8*n_expert (16*n_expert when the one-kernel form
 * applies) and fat tiles above; 1 forces sorted with
 * fat tiles, 4 sorted with skinny tiles as two kernels, 5 sorted with
 * skinny tiles in one kernel per tile (two kernels for an int8 down or
 * shared expert), 2 direct (EINVAL from forward when T > 16).  Mode 3 (a
 * one-kernel decode variant, measured slower) no longer exists: EINVAL.
 * last_path: 0 sorted (fat), 1 direct, 2 sorted (skinny, two kernels),
 * 3 sorted (skinny, one kernel per tile).  With the
 * direct path the PERM/POS taps are the identity (rows in entry order) and
 * the EOFF/DNW taps are unavailable. */
int q36moe_ctx_set_path(q36moe_ctx *c, int mode);
int q36moe_ctx_last_path(const q36moe_ctx *c);

/* Synchronises the context stream; Q36MOE_EHIP if it reports an error. */
int q36moe_ctx_check(q36moe_ctx *c);

/* Copy one internal buffer of the last forward into dst (device pointer,
 * at most `bytes`); *written receives the byte count. */
int q36moe_ctx_copy_tap(q36moe_ctx *c, int tap, void *dst, size_t bytes, size_t *written);

/* Per-stage timing of forward: when enabled, forward records HIP events
 * around each kernel on the context stream and synchronises at its end;
 * q36moe_ctx_stage_times adds up milliseconds per stage since the last
 * reset (n_stages entries, names via q36moe_stage_name). */
int q36moe_ctx_set_timing(q36moe_ctx *c, int on);
int q36moe_ctx_stage_times(q36moe_ctx *c, double *ms, int *calls, int n_stages, int reset);
const char *q36moe_stage_name(int stage);
int q36moe_num_stages(void);

/* Launch again, on the context stream and without synchronising, the
 * kernels of one stage of the last forward (same inputs, tokens and path)
 * with the weights w.  Bracketing many replays over rotating weight sets
 * with two events gives a kernel's average duration without per-launch
 * event overhead.  The stage's outputs are rewritten; call forward again
 * before reading results.  w must have the formats (MXFP4 / q8_0-split
 * down and shared expert) of the last forward's weights, else EINVAL.  No
 * counterpart in the reference (profiling aid). */
int q36moe_ctx_replay(q36moe_ctx *c, const q36moe_weights *w, int stage);

/* GGUF v3 ingest (replaces gguf_open, gguf.c, and bind_moe + upload,
 * q36_model.c:54-77 and q36_engine.cu:196-228, for the MoE tensors).  The
 * file is mapped read-only and its header, metadata and tensor directory
 * parsed; tensor data is never copied by the reader.  Errors: Q36MOE_EIO
 * (open/map), Q36MOE_EINVAL (not GGUF v3, malformed, or a tensor past the
 * end of the file), Q36MOE_ENOENT (no such tensor or key). */
typedef struct q36moe_gguf q36moe_gguf;
int q36moe_gguf_open(const char *path, q36moe_gguf **out);
void q36moe_gguf_close(q36moe_gguf *g);
int q36moe_gguf_info(const q36moe_gguf *g, uint32_t *version, uint64_t *n_tensors, uint64_t *n_kv,
                     uint32_t *alignment, uint64_t *data_offset);
/* Tensor by exact name: ggml type id, n_dims, dims[4] (dims[0] innermost,
 * unused dims 1), absolute file offset, host pointer into the mapping and
 * byte size (0 for a type without a known block size).  Any out pointer
 * may be NULL. */
int q36moe_gguf_tensor(const q36moe_gguf *g, const char *name, uint32_t *ggml_type, uint32_t *n_dims,
                       uint64_t *dims, uint64_t *file_offset, const void **data, uint64_t *nbytes);
int q36moe_gguf_u32(const q36moe_gguf *g, const char *key, uint32_t *out);
/* Uploads block `layer`'s experts: blk.N.ffn_{gate,up,down}_exps.weight of
 * ggml dims [d_model][d_ff][E] / [d_ff][d_model][E]; gate and up MXFP4
 * (ggml type 39), down MXFP4, Q5_K, Q6_K or Q8_0 (as
 * q36moe_weights_upload_typed); with with_shared, also
 * blk.N.ffn_{gate,up,down}_shexp.weight, all three of one type: MXFP4,
 * Q8_0 (the release file's), Q5_K or Q6_K. */
int q36moe_weights_from_gguf(const q36moe_gguf *g, int layer, int with_shared, q36moe_weights **out);
/* The router rows of block `layer` as host f32 for q36moe_router_logits:
 * blk.N.ffn_gate_inp.weight [n_expert][d_model] (F32 or BF16, widened
 * exactly) and, when present, blk.N.ffn_gate_inp_shexp.weight as row
 * n_expert.  dst holds dst_floats floats (EINVAL if the rows do not fit);
 * *n_rows and *d_model receive the shape written. */
int q36moe_router_from_gguf(const q36moe_gguf *g, int layer, float *dst, size_t dst_floats, int *n_rows,
                            int *d_model);

/* One v_mfma_scale_f32_16x16x128_f8f6f4 on caller-packed operands:
 * a, b: 64 lanes x 32 bytes; sa, sb: 64 lane scale dwords (byte 0 used);
 * fmt_a / fmt_b: 0 e4m3, 1 e5m2, 2 e2m3, 3 e3m2, 4 e2m1; c: 64 x 4 floats. */
int q36moe_probe_mfma(const void *a, const void *b, const uint32_t *sa,
                      const uint32_t *sb, int fmt_a, int fmt_b, float *c, void *stream);

/* One v_mfma_scale_f32_32x32x64_f8f6f4 with A e2m1 and B e4m3 on
 * caller-packed operands (the 32x32 tile the fat gate/up uses): a, b: 64
 * lanes x 32 bytes; sa, sb: 64 lane scale dwords (byte 0 used); c: 64 x 16
 * floats.  Calibration harness, like q36moe_probe_mfma. */
int q36moe_probe_mfma32(const void *a, const void *b, const uint32_t *sa, const uint32_t *sb, float *c,
                        void *stream);

#ifdef __cplusplus
}
#endif
#endif
