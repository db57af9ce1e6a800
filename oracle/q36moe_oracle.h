/* CPU oracle for the W4A8 MoE layer -- TEST INFRASTRUCTURE ONLY.
 *
 * This header and q36moe_oracle.c restate, in plain C, the arithmetic of the
 * q36 engine's MoE FFN path (router top-k, MXFP4 dequant, FP8 activation
 * quantiser, expert dispatch, SwiGLU expert GEMMs, weighted combine).  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it, and only as the checker; the product path (q36_amd/, libq36moe.so)
 * never calls into it.
 *
 * Every function cites the reference file:line whose behaviour it follows.
 */
#ifndef Q36MOE_ORACLE_H
#define Q36MOE_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar formats ---------------------------------------------------- */
double or_e8m0(uint8_t e);                 /* 2^(e-127) (e=255 -> 2^128)    */
double or_e2m1(uint8_t code);              /* OCP E2M1 value of a nibble    */
float  or_e4m3_decode(uint8_t b);          /* OCP E4M3FN -> float (NaN 0x7f) */
uint8_t or_e4m3_encode(float v);           /* RNE, satfinite, NaN -> 0x7f   */
int    or_quant_exp(float amax);           /* e2 of the per-32 quantiser    */

/* ---- block formats ----------------------------------------------------- */
/* One GGUF block_mxfp4 (17 B: e, qs[16]) -> 32 floats (fp32 products). */
void or_deq_mxfp4_block(const uint8_t *blk17, float *out32);
/* n values (multiple of 32) of a row of GGUF blocks -> float. */
void or_deq_mxfp4_row(const uint8_t *blocks, int n, float *out);

/* ---- activation quantiser (k_quant_e4m3) ------------------------------- */
void or_quant_e4m3(const float *X, int T, int K, uint8_t *Xq, uint8_t *Xs);
void or_dequant_e4m3(const uint8_t *Xq, const uint8_t *Xs, int T, int K, double *Xd);

/* ---- router (k_router_topk) -------------------------------------------- */
/* idx[T][k], wt[T][k].  Weights in double: exp(l-m)/sum_all, then
 * renormalised over the k selected and multiplied by scale. */
void or_router_topk(const float *logits, int T, int n_expert, int ld, int k,
                    float scale, int renorm, int32_t *idx, double *wt);

/* ---- dispatch: deterministic stable counting sort ---------------------- */
/* entries i = t*k+s with expert idx[i]; outputs
 *   off[n_expert+1]  exclusive prefix of per-expert counts
 *   perm[T*k]        entry id at each sorted position (expert asc, id asc)
 *   pos[T*k]         sorted position of each entry (inverse of perm)   */
void or_sort(const int32_t *idx, int n_entries, int n_expert,
             int32_t *off, int32_t *perm, int32_t *pos);

/* ---- GEMV over GGUF MXFP4 rows x FP8 activation (config 1 CPU path) ---- */
/* y[M] = W[M][K] . x  with W dequantised per row and fp32 accumulation. */
void or_gemv_mxfp4_f32(const uint8_t *W, int M, int K,
                       const uint8_t *xq, const uint8_t *xs, float *y);
void or_gemv_mxfp4_f32_mt(const uint8_t *W, int M, int K,
                          const uint8_t *xq, const uint8_t *xs, float *y,
                          int nthreads);

/* ---- Q8 formats (requantised expert layout) ---------------------------- */
uint16_t or_f16_encode(float f);           /* IEEE binary16, RNE            */
float  or_f16_decode(uint16_t h);
void or_deq_q8_0_block(const uint8_t *b34, float *out32);
void or_deq_q5_K_block(const uint8_t *b176, float *out256);
void or_deq_q6_K_block(const uint8_t *b210, float *out256);
/* ggml type 8 / 13 / 14 / 39; -1 for another type or a ragged n */
int  or_deq_row(uint32_t type, const void *blocks, int n, float *out);
void or_requant_q8_row(const float *x, int K, int8_t *qs, uint16_t *ds);
int  or_requant_q8(uint32_t type, const void *src, int M, int K, int8_t *qs, uint16_t *ds);
void or_quant_q8b(const float *x, int K, int8_t *q, float *d);
void or_expert_down_q8(const int8_t *qs, const uint16_t *ds, int D, int FF, const double *h, double *y);
/* h = silu(gate . x) * (up . x) in double over q8_0-split gate/up [FF][D] */
void or_expert_h_q8(const int8_t *gq, const uint16_t *gd, const int8_t *uq, const uint16_t *ud, int D, int FF,
                    const double *x, double *h);

/* ---- the whole layer --------------------------------------------------- */
typedef struct {
    const uint8_t *gate, *up, *down;          /* GGUF blocks [E][M][K/32]   */
    const uint8_t *sh_gate, *sh_up, *sh_down; /* GGUF blocks [M][K/32] or 0 */
    int n_expert, d_model, d_ff, d_ff_sh;
    /* routed down in the q8_0-split layout instead of `down` (NULL = MXFP4):
     * codes [E][d_model][d_ff] int8, f16 scales [E][d_model][d_ff/32] */
    const int8_t *down_q8;
    const uint16_t *down_q8d;
    /* shared expert in the q8_0-split layout instead of sh_* (NULL = MXFP4,
     * the release file's Q8_0 _shexp tensors): codes gate/up
     * [d_ff_sh][d_model], down [d_model][d_ff_sh], f16 scales per 32.  Its
     * activations are quantised per 32 to int8 + fp32 scale (k_quant_q8b),
     * x and h alike, as pf_gemm does for split-Q8 weights
     * (q36_engine.cu:3403-3406, :3464-3469). */
    const int8_t *sh_gate_q8, *sh_up_q8, *sh_down_q8;
    const uint16_t *sh_gate_q8d, *sh_up_q8d, *sh_down_q8d;
} or_weights;

/* act_mode 0: W4A8 -- x and h quantised exactly as the product does
 *             (per-32 E8M0 + e4m3), h rounded to fp32 before quantising.
 * act_mode 1: W4A32 -- activations kept unquantised (the reference decode
 *             path, q36_engine.cu:1610-1618), for drift reporting.
 * act_mode 2: the reference's prefill numerics -- x per-32 e4m3, h kept in
 *             f32 and rounded to fp16 for the MXFP4 down (k_gemm_expert_tc,
 *             q36_engine.cu:3459-3462), for drift reporting.
 * Computes the rows listed in `tokens` (n_tok of them; NULL = 0..T-1) and
 * writes out[n_tok][d_model] in double.  shg may be NULL (no shared expert
 * contribution).                                                         */
void or_moe_forward(const or_weights *w, const float *x, const float *logits,
                    int ld_logits, const float *shg, int T, int k,
                    float scale, int act_mode, const int32_t *tokens,
                    int n_tok, double *out);

/* Stage restatements used for staged parity:
 *   or_expert_h:    h = silu(gate . x) * (up . x) in double (before any fp32
 *                   rounding or quantisation), x given dequantised, gate/up
 *                   GGUF blocks [FF][D/32]      (q36_engine.cu:1610-1615)
 *   or_expert_down: y = down . h, down [D][FF/32], h dequantised
 *                   (q36_engine.cu:1616-1618)                              */
void or_expert_h(const uint8_t *gate, const uint8_t *up, int D, int FF,
                 const double *x, double *h);
void or_expert_down(const uint8_t *down, int D, int FF, const double *h, double *y);

/* fp32-accumulation layer forward used as the timed CPU baseline; same
 * semantics as act_mode 0 but every dot product accumulates in float. */
void or_moe_forward_f32(const or_weights *w, const float *x, const float *logits,
                        int ld_logits, const float *shg, int T, int k,
                        float scale, float *out, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
