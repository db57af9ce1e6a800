/* CPU oracle for the W4A8 MoE layer -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the q36 engine's MoE FFN arithmetic, used by
 * tests/ (as the checker), __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg.  The product library never links or calls it.
 *
 * Pinning (what checks each function against something other than itself):
 *   or_e8m0 / or_e2m1 / or_deq_mxfp4_*  -- the reference's own known answers
 *       (test_dequant.c:51-61) and, exhaustively over all 16 codes x 256
 *       exponents, the reference's q36_deq_mxfp4 compiled from its own
 *       header (oracle/Makefile -> oracle/_ref/).
 *   or_e4m3_encode / or_e4m3_decode     -- OCP FP8 closed forms (all 256
 *       codes, every tie), and torch.float8_e4m3fn as an independent
 *       library routine.
 *   or_quant_exp / or_quant_e4m3        -- closed form of
 *       q36_engine.cu:2421-2427 plus invariants (minimal scale, |q|<=448).
 *   or_router_topk                      -- brute-force sort by
 *       (logit desc, index asc) and fp64 softmax.
 *   or_sort                             -- brute force + bijection /
 *       histogram / scan invariants.
 *   or_f16_encode / or_f16_decode       -- numpy float16 (an independent
 *       library routine) over every f16 pattern and every rounding tie.
 *   or_deq_q8_0 / _q5_K / _q6_K         -- the reference's own q36_deq_row
 *       compiled from its header (oracle/_ref/), bit-exact on random
 *       blocks, plus hand-computed single-element cases.
 *   or_requant_q8_row / or_quant_q8b    -- closed forms of
 *       q36_engine.cu:73-86 and :2627-2640 plus invariants (|q| <= 127 /
 *       128, the block maximum maps to +-127, numpy rint / float16).
 *   or_gemv_* / or_moe_forward          -- fp64 brute force on tiny shapes
 *       and closed forms (rank-1 weights, single non-zero block, linearity
 *       in the routing weights).
 */
#include "q36moe_oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------------- */
/* Scalars                                                                 */
/* ---------------------------------------------------------------------- */

/* E8M0 scale 2^(e-127).  The reference stores it halved next to a doubled
 * E2M1 table (q36_dequant.cuh:84-103: e8m0_half(e)=2^(e-128), e<2 handled
 * as fp32 denormals); the product table*half equals E2M1*2^(e-127) for all
 * e in 0..254.  e=255 gives 2^128 here as in ggml (OCP calls it NaN). */
double or_e8m0(uint8_t e) { return ldexp(1.0, (int)e - 127); }

/* OCP E2M1: bit3 sign, bits2:1 exponent (bias 1), bit0 mantissa.
 * Values {0,.5,1,1.5,2,3,4,6}; the reference's doubled table
 * {0,1,2,3,4,6,8,12} (q36_dequant.cuh:84-88) is twice this. */
double or_e2m1(uint8_t c) {
    static const double mag[8] = {0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0};
    double v = mag[c & 7];
    return (c & 8) ? -v : v;
}

/* OCP E4M3FN decode: bias 7, no inf, S.1111.111 = NaN. */
float or_e4m3_decode(uint8_t b) {
    int s = b >> 7, e = (b >> 3) & 15, m = b & 7;
    float v;
    if (e == 15 && m == 7) return NAN;
    if (e == 0) v = ldexpf((float)m, -9);
    else        v = ldexpf((float)(8 + m), e - 10);
    return s ? -v : v;
}

/* OCP E4M3FN encode, round-to-nearest-even, saturating to +-448 (the
 * __NV_SATFINITE conversion the reference's __nv_fp8_e4m3 constructor
 * performs, q36_engine.cu:2426).  NaN -> 0x7f (sign kept). */
uint8_t or_e4m3_encode(float v) {
    uint32_t u; memcpy(&u, &v, 4);
    uint8_t sign = (uint8_t)((u >> 31) << 7);
    uint32_t a = u & 0x7fffffffu;
    /* NaN -> 0x7f whatever its sign: a NaN computed from inf * 0 has a
     * platform-dependent sign bit */
    if (a > 0x7f800000u) return 0x7f;
    if (a >= 0x43e00000u) return sign | 0x7e;          /* >= 448 */
    if (a < 0x3c800000u) {                            /* < 2^-6: subnormal */
        float f; memcpy(&f, &a, 4);
        float q = rintf(f * 512.0f);                  /* units of 2^-9, RNE */
        return sign | (uint8_t)q;                     /* q==8 -> 0x08 = 2^-6 */
    }
    int e = (int)(a >> 23) - 127;                     /* -6 .. 8 */
    uint32_t m = a & 0x7fffffu;
    uint32_t r = ((uint32_t)(e + 7) << 3) | (m >> 20);
    uint32_t rb = (m >> 19) & 1u, sticky = m & 0x7ffffu, lsb = r & 1u;
    if (rb && (sticky || lsb)) r++;
    if (r > 0x7e) r = 0x7e;
    return sign | (uint8_t)r;
}

/* Exponent of the per-32 activation scale: e2 = ceil(log2(amax/448)),
 * clamped to [-127,127], -127 for an all-zero block
 * (q36_engine.cu:2421-2423).  The quotient is the fp32 a/448 of the
 * reference; its ceil(log2) is taken exactly from the binary exponent
 * (a correctly rounded log2f can round 2^n(1+2^-23) down to n: that case
 * differs by one scale step and is pinned in tests). */
int or_quant_exp(float amax) {
    if (!(amax > 0.0f)) return -127;
    /* an infinite amax: ceil(log2(inf)) converts to the largest int in the
     * reference's saturating float-to-int conversion, then clamps to 127 */
    if (amax > 3.40282347e38f) return 127;
    float q = amax / 448.0f;
    int ex;
    float f = frexpf(q, &ex);                         /* q = f*2^ex, f in [.5,1) */
    int e2 = (f == 0.5f) ? ex - 1 : ex;
    if (e2 < -127) e2 = -127;
    if (e2 > 127) e2 = 127;
    return e2;
}

/* 2^-e2 built from exponent bits as in q36_engine.cu:2424-2426 (e2=127
 * yields 0.0 there, kept here). */
static float inv_scale(int e2) {
    uint32_t bits = (uint32_t)(127 - e2) << 23;
    float f; memcpy(&f, &bits, 4);
    return f;
}

/* ---------------------------------------------------------------------- */
/* MXFP4 blocks                                                            */
/* ---------------------------------------------------------------------- */

/* Element order of q36_deq_mxfp4 (q36_dequant.cuh:106-113): element j is the
 * low nibble of qs[j], element j+16 the high nibble. */
void or_deq_mxfp4_block(const uint8_t *blk, float *out) {
    double d = or_e8m0(blk[0]);
    for (int j = 0; j < 16; j++) {
        out[j]      = (float)(or_e2m1(blk[1 + j] & 15) * d);
        out[j + 16] = (float)(or_e2m1(blk[1 + j] >> 4) * d);
    }
}

void or_deq_mxfp4_row(const uint8_t *blocks, int n, float *out) {
    for (int b = 0; b < n / 32; b++) or_deq_mxfp4_block(blocks + 17 * b, out + 32 * b);
}

/* ---------------------------------------------------------------------- */
/* Activation quantiser: q36_engine.cu:2411-2428 (k_quant_e4m3)            */
/* ---------------------------------------------------------------------- */
void or_quant_e4m3(const float *X, int T, int K, uint8_t *Xq, uint8_t *Xs) {
    int nb = K / 32;
    for (int t = 0; t < T; t++)
        for (int b = 0; b < nb; b++) {
            const float *v = X + (size_t)t * K + b * 32;
            float a = 0.0f;
            for (int j = 0; j < 32; j++) a = fmaxf(a, fabsf(v[j]));
            int e2 = or_quant_exp(a);
            float mul = inv_scale(e2);
            for (int j = 0; j < 32; j++)
                Xq[(size_t)t * K + b * 32 + j] = or_e4m3_encode(v[j] * mul);
            Xs[(size_t)t * nb + b] = (uint8_t)(127 + e2);
        }
}

void or_dequant_e4m3(const uint8_t *Xq, const uint8_t *Xs, int T, int K, double *Xd) {
    int nb = K / 32;
    for (int t = 0; t < T; t++)
        for (int k = 0; k < K; k++)
            Xd[(size_t)t * K + k] = (double)or_e4m3_decode(Xq[(size_t)t * K + k]) *
                                    or_e8m0(Xs[(size_t)t * nb + k / 32]);
}

/* ---------------------------------------------------------------------- */
/* Router: q36_ops.cuh:397-431 (k_router_topk)                             */
/* ---------------------------------------------------------------------- */
/* k rounds of argmax with ties to the lower expert index (:416-423); the
 * weight of a pick is exp(l-m)/sum_all (:424), then renormalised over the
 * picks and multiplied by scale (:428-430).  Doubles throughout. */
void or_router_topk(const float *logits, int T, int n_expert, int ld, int k,
                    float scale, int renorm, int32_t *idx, double *wt) {
    char *taken = (char *)malloc((size_t)n_expert);
    for (int t = 0; t < T; t++) {
        const float *l = logits + (size_t)t * ld;
        double m = -1e30;
        for (int j = 0; j < n_expert; j++) if (l[j] > m) m = l[j];
        double s = 0.0;
        for (int j = 0; j < n_expert; j++) s += exp((double)l[j] - m);
        memset(taken, 0, (size_t)n_expert);
        double ws = 0.0;
        for (int r = 0; r < k; r++) {
            int bj = -1; float bv = 0.0f;
            for (int j = 0; j < n_expert; j++) {
                if (taken[j]) continue;
                if (bj < 0 || l[j] > bv) { bv = l[j]; bj = j; }
            }
            taken[bj] = 1;
            idx[(size_t)t * k + r] = bj;
            wt[(size_t)t * k + r] = exp((double)bv - m) / s;
            ws += wt[(size_t)t * k + r];
        }
        for (int r = 0; r < k; r++)
            wt[(size_t)t * k + r] = renorm ? wt[(size_t)t * k + r] / ws * scale
                                           : wt[(size_t)t * k + r] * scale;
    }
    free(taken);
}

/* ---------------------------------------------------------------------- */
/* Dispatch: the reference buckets entry ids t*8+s per expert with an       */
/* atomic counter (q36_engine.cu:3387-3392), so order inside a bucket is     */
/* unspecified; this build fixes it to ascending entry id.                  */
/* ---------------------------------------------------------------------- */
void or_sort(const int32_t *idx, int n, int n_expert,
             int32_t *off, int32_t *perm, int32_t *pos) {
    for (int e = 0; e <= n_expert; e++) off[e] = 0;
    for (int i = 0; i < n; i++) off[idx[i] + 1]++;
    for (int e = 0; e < n_expert; e++) off[e + 1] += off[e];
    int32_t *fill = (int32_t *)malloc(sizeof(int32_t) * (size_t)(n_expert + 1));
    memcpy(fill, off, sizeof(int32_t) * (size_t)(n_expert + 1));
    for (int i = 0; i < n; i++) {
        int p = fill[idx[i]]++;
        perm[p] = i;
        pos[i] = p;
    }
    free(fill);
}

/* ---------------------------------------------------------------------- */
/* Config-1 CPU path: dequant + GEMV, fp32 accumulation.  The dequant is    */
/* q36_deq_mxfp4 (q36_dequant.cuh:106-113) per row; the row dot follows     */
/* the per-block order of dot_mxfp4_split (q36_ops.cuh:153-167).            */
/* ---------------------------------------------------------------------- */
static void gemv_rows(const uint8_t *W, int r0, int r1, int K,
                      const float *x, float *y) {
    float wr[32];
    int nb = K / 32;
    for (int r = r0; r < r1; r++) {
        float acc = 0.0f;
        const uint8_t *row = W + (size_t)r * nb * 17;
        for (int b = 0; b < nb; b++) {
            or_deq_mxfp4_block(row + 17 * b, wr);
            float s = 0.0f;
            for (int j = 0; j < 32; j++) s += wr[j] * x[b * 32 + j];
            acc += s;
        }
        y[r] = acc;
    }
}

static float *deq_x(const uint8_t *xq, const uint8_t *xs, int K) {
    float *x = (float *)malloc(sizeof(float) * (size_t)K);
    for (int k = 0; k < K; k++)
        x[k] = or_e4m3_decode(xq[k]) * (float)or_e8m0(xs[k / 32]);
    return x;
}

void or_gemv_mxfp4_f32(const uint8_t *W, int M, int K,
                       const uint8_t *xq, const uint8_t *xs, float *y) {
    float *x = deq_x(xq, xs, K);
    gemv_rows(W, 0, M, K, x, y);
    free(x);
}

void or_gemv_mxfp4_f32_mt(const uint8_t *W, int M, int K,
                          const uint8_t *xq, const uint8_t *xs, float *y,
                          int nthreads) {
    float *x = deq_x(xq, xs, K);
#ifdef _OPENMP
    #pragma omp parallel num_threads(nthreads)
    {
        int nt = omp_get_num_threads(), id = omp_get_thread_num();
        int r0 = (int)((long)M * id / nt), r1 = (int)((long)M * (id + 1) / nt);
        gemv_rows(W, r0, r1, K, x, y);
    }
#else
    (void)nthreads;
    gemv_rows(W, 0, M, K, x, y);
#endif
    free(x);
}

/* ---------------------------------------------------------------------- */
/* Whole layer                                                             */
/* ---------------------------------------------------------------------- */
/* ---------------------------------------------------------------------- */
/* Q8 formats: the reference's requantised expert layout (q8_0-split)      */
/* ---------------------------------------------------------------------- */

/* IEEE binary16 from float, round to nearest even, overflow to inf (the
 * __float2half conversion of the reference's h_f16, q36_engine.cu:69-71). */
uint16_t or_f16_encode(float f) {
    uint32_t u; memcpy(&u, &f, 4);
    uint32_t sign = (u >> 16) & 0x8000u, a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);           /* NaN */
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);          /* >= 65520 -> inf */
    if (a < 0x38800000u) {                                            /* below 2^-14: subnormal */
        float q = fabsf(f) * 16777216.0f;                              /* units of 2^-24 (exact) */
        return (uint16_t)(sign | (uint32_t)rintf(q));
    }
    uint32_t r = ((a >> 13) - (112u << 10));                           /* rebias 127 -> 15 */
    uint32_t rem = a & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return (uint16_t)(sign | r);
}

float or_f16_decode(uint16_t h) {
    int s = h >> 15, e = (h >> 10) & 31, m = h & 1023;
    float v;
    if (e == 31) v = m ? NAN : INFINITY;
    else if (e == 0) v = ldexpf((float)m, -24);
    else v = ldexpf((float)(1024 + m), e - 25);
    return s ? -v : v;
}

/* Q8_0 block (34 B: f16 d, 32 int8): d * q  (q36_dequant.cuh:116-119). */
void or_deq_q8_0_block(const uint8_t *b, float *out) {
    uint16_t dh; memcpy(&dh, b, 2);
    float d = or_f16_decode(dh);
    for (int j = 0; j < 32; j++) out[j] = d * (float)(int8_t)b[2 + j];
}

/* 6-bit scale / min of sub-block j of a Q5_K super-block (q36_dequant.cuh:
 * 121-126, ggml get_scale_min_k4): sub-blocks 0-3 take the low 6 bits of
 * bytes j and j+4; 4-7 take a nibble of byte j+4 and the top two bits of
 * bytes j-4 (scale) and j (min). */
static void k4_scale_min(int j, const uint8_t *q, int *sc, int *mn) {
    if (j < 4) {
        *sc = q[j] & 63;
        *mn = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 15) | ((q[j - 4] >> 6) << 4);
        *mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* Q5_K super-block (176 B: f16 d, f16 dmin, scales[12], qh[32], qs[128]),
 * 256 values (q36_dequant.cuh:128-142).  Value i = 64c + 32h + l (chunk c,
 * half h): 5-bit q = nibble h of qs[32c + l] | bit (2c + h) of qh[l] << 4;
 * y = (d*sc) * q - (dmin*mn) for sub-block 2c + h. */
void or_deq_q5_K_block(const uint8_t *b, float *out) {
    uint16_t dh, mh; memcpy(&dh, b, 2); memcpy(&mh, b + 2, 2);
    const float d = or_f16_decode(dh), dmin = or_f16_decode(mh);
    const uint8_t *sc = b + 4, *qh = b + 16, *qs = b + 48;
    for (int c = 0; c < 4; c++)
        for (int h = 0; h < 2; h++) {
            int s, m;
            k4_scale_min(2 * c + h, sc, &s, &m);
            const float d1 = d * (float)s, m1 = dmin * (float)m;
            for (int l = 0; l < 32; l++) {
                int q = (h ? qs[32 * c + l] >> 4 : qs[32 * c + l] & 15) |
                        (((qh[l] >> (2 * c + h)) & 1) << 4);
                float t = d1 * (float)q;   /* product, then difference: no fused multiply-add */
                out[64 * c + 32 * h + l] = t - m1;
            }
        }
}

/* Q6_K super-block (210 B: ql[128], qh[64], int8 scales[16], f16 d), 256
 * values (q36_dequant.cuh:144-165).  Half n (128 values), quarter g, lane l:
 * 6-bit q = nibble (g >= 2) of ql[64n + 32(g & 1) + l] | bits 2g..2g+1 of
 * qh[32n + l] << 4, minus 32; y = d * sc[8n + 2g + l/16] * q. */
void or_deq_q6_K_block(const uint8_t *b, float *out) {
    const uint8_t *ql = b, *qh = b + 128;
    const int8_t *sc = (const int8_t *)(b + 192);
    uint16_t dh; memcpy(&dh, b + 208, 2);
    const float d = or_f16_decode(dh);
    for (int n = 0; n < 2; n++)
        for (int g = 0; g < 4; g++)
            for (int l = 0; l < 32; l++) {
                int lo = ql[64 * n + 32 * (g & 1) + l];
                lo = g >= 2 ? lo >> 4 : lo & 15;
                int q = (lo | (((qh[32 * n + l] >> (2 * g)) & 3) << 4)) - 32;
                float t = d * (float)sc[8 * n + 2 * g + l / 16];
                out[128 * n + 32 * g + l] = t * (float)q;
            }
}

int or_deq_row(uint32_t type, const void *blocks, int n, float *out) {
    const uint8_t *p = (const uint8_t *)blocks;
    switch (type) {
        case 8:  if (n % 32) return -1; for (int i = 0; i < n / 32; i++) or_deq_q8_0_block(p + 34 * i, out + 32 * i); return 0;
        case 13: if (n % 256) return -1; for (int i = 0; i < n / 256; i++) or_deq_q5_K_block(p + 176 * i, out + 256 * i); return 0;
        case 14: if (n % 256) return -1; for (int i = 0; i < n / 256; i++) or_deq_q6_K_block(p + 210 * i, out + 256 * i); return 0;
        case 39: if (n % 32) return -1; or_deq_mxfp4_row(p, n, out); return 0;
        default: return -1;
    }
}

/* h_q8_row (q36_engine.cu:73-86): per 32 values d = amax/127 (fp32),
 * stored as f16; q = rint(v * (1/d)) with 1/d from the fp32 d, clamped to
 * [-128, 127]. */
void or_requant_q8_row(const float *x, int K, int8_t *qs, uint16_t *ds) {
    for (int b = 0; b < K / 32; b++) {
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) { float v = fabsf(x[32 * b + j]); if (v > amax) amax = v; }
        const float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
        ds[b] = or_f16_encode(d);
        for (int j = 0; j < 32; j++) {
            long q = lrintf(x[32 * b + j] * id);
            qs[32 * b + j] = (int8_t)(q > 127 ? 127 : q < -128 ? -128 : q);
        }
    }
}

/* One expert matrix of M rows x K from GGUF blocks of `type` to the
 * q8_0-split layout (codes [M][K], f16 scales [M][K/32]).  Q5_K / Q6_K are
 * dequantised and requantised as the reference's upload does
 * (q36_engine.cu:229-252); Q8_0 blocks are split as they are. */
int or_requant_q8(uint32_t type, const void *src, int M, int K, int8_t *qs, uint16_t *ds) {
    size_t rb;
    if (type == 13) rb = (size_t)K / 256 * 176;
    else if (type == 14) rb = (size_t)K / 256 * 210;
    else if (type == 8) rb = (size_t)K / 32 * 34;
    else return -1;
    if (K % (type == 8 ? 32 : 256)) return -1;
    float *row = (float *)malloc(sizeof(float) * (size_t)K);
    for (int r = 0; r < M; r++) {
        const uint8_t *p = (const uint8_t *)src + rb * r;
        if (type == 8) {
            for (int b = 0; b < K / 32; b++) {
                memcpy(&ds[(size_t)r * (K / 32) + b], p + 34 * b, 2);
                memcpy(&qs[(size_t)r * K + 32 * b], p + 34 * b + 2, 32);
            }
        } else {
            or_deq_row(type, p, K, row);
            or_requant_q8_row(row, K, qs + (size_t)r * K, ds + (size_t)r * (K / 32));
        }
    }
    free(row);
    return 0;
}

/* k_quant_q8b (q36_engine.cu:2627-2640): per 32 values d = amax/127,
 * q = rint(v * 127/amax) clamped to [-127, 127] (0 for an all-zero block).
 * The reference divides with CUDA's fast __fdividef; this is the IEEE
 * quotient. */
void or_quant_q8b(const float *x, int K, int8_t *q, float *d) {
    for (int b = 0; b < K / 32; b++) {
        float a = 0.0f;
        for (int j = 0; j < 32; j++) a = fmaxf(a, fabsf(x[32 * b + j]));
        const float id = a > 0.0f ? 127.0f / a : 0.0f;
        d[b] = a / 127.0f;
        for (int j = 0; j < 32; j++) {
            long v = lrintf(x[32 * b + j] * id);
            q[32 * b + j] = (int8_t)(v > 127 ? 127 : v < -127 ? -127 : v);
        }
    }
}

/* y[r] = sum_b f16(ds[r][b]) * sum_j qs[r][32b+j] * h[32b+j] over q8_0-split
 * rows, h in double (the down GEMV of the requantised layout,
 * q36_engine.cu:736-741). */
static void mv_q8_d(const int8_t *qs, const uint16_t *ds, int M, int K, const double *h, double *y) {
    for (int r = 0; r < M; r++) {
        double acc = 0.0;
        for (int b = 0; b < K / 32; b++) {
            double p = 0.0;
            for (int j = 0; j < 32; j++) p += (double)qs[(size_t)r * K + 32 * b + j] * h[32 * b + j];
            acc += (double)or_f16_decode(ds[(size_t)r * (K / 32) + b]) * p;
        }
        y[r] = acc;
    }
}

void or_expert_down_q8(const int8_t *qs, const uint16_t *ds, int D, int FF, const double *h, double *y) {
    mv_q8_d(qs, ds, D, FF, h, y);
}

static double silu_d(double g) { return g / (1.0 + exp(-g)); }
static double sigm_d(double g) { return 1.0 / (1.0 + exp(-g)); }

/* y[M] = W[M][K] . x  (GGUF MXFP4 rows, double accumulation). */
static void mv_d(const uint8_t *W, int M, int K, const double *x, double *y) {
    int nb = K / 32;
    float wr[32];
    for (int r = 0; r < M; r++) {
        const uint8_t *row = W + (size_t)r * nb * 17;
        double acc = 0.0;
        for (int b = 0; b < nb; b++) {
            or_deq_mxfp4_block(row + 17 * b, wr);
            for (int j = 0; j < 32; j++) acc += (double)wr[j] * x[b * 32 + j];
        }
        y[r] = acc;
    }
}

/* Quantise a float row with the activation rule, return dequantised doubles. */
static void quant_roundtrip(const float *v, int K, double *out) {
    uint8_t *q = (uint8_t *)malloc((size_t)K), *s = (uint8_t *)malloc((size_t)K / 32);
    or_quant_e4m3(v, 1, K, q, s);
    or_dequant_e4m3(q, s, 1, K, out);
    free(q); free(s);
}

/* One SwiGLU expert: out = down . q(silu(gate.x) * up.x), following
 * k_expert_gemv2 -> k_silu_mul_slots -> k_expert_gemv
 * (q36_engine.cu:1610-1618) with the activation quantisation of the
 * W4A8 prefill path (q36_engine.cu:2411-2428, :3437-3441) applied to x and
 * to the SwiGLU output when act_mode==0.  act_mode 1 keeps x and h
 * unquantised (the reference's decode matvecs, W4A32); act_mode 2 is the
 * reference's own prefill numerics: x per-32 e4m3 (k_quant_e4m3 ->
 * k_gemm_expert_mma), h kept in f32 by k_silu_mul and rounded to fp16 by the
 * MXFP4 down's fp16 tensor-core GEMM (k_gemm_expert_tc with x_by_entry,
 * q36_engine.cu:3459-3462). */
static void expert_d(const uint8_t *g, const uint8_t *u, const uint8_t *d,
                     const int8_t *dq, const uint16_t *dd,
                     int D, int FF, const double *xin, int act_mode, double *out) {
    double *gv = (double *)malloc(sizeof(double) * (size_t)FF);
    double *uv = (double *)malloc(sizeof(double) * (size_t)FF);
    double *hd = (double *)malloc(sizeof(double) * (size_t)FF);
    float *hf = (float *)malloc(sizeof(float) * (size_t)FF);
    mv_d(g, FF, D, xin, gv);
    mv_d(u, FF, D, xin, uv);
    for (int f = 0; f < FF; f++) hf[f] = (float)(silu_d(gv[f]) * uv[f]);
    if (dq) {
        /* q8_0-split down (the reference's requantised Q5_K / Q6_K experts):
         * h quantised per 32 to int8 with an fp32 scale (k_quant_q8b ->
         * k_gemm_expert_i8, q36_engine.cu:3452-3458) under act_mode 0 */
        if (act_mode == 0) {
            int8_t *q = (int8_t *)malloc((size_t)FF);
            float *hs = (float *)malloc(sizeof(float) * (size_t)FF / 32);
            or_quant_q8b(hf, FF, q, hs);
            for (int f = 0; f < FF; f++) hd[f] = (double)q[f] * (double)hs[f / 32];
            free(q); free(hs);
        } else {
            for (int f = 0; f < FF; f++) hd[f] = hf[f];
        }
        mv_q8_d(dq, dd, D, FF, hd, out);
    } else {
        if (act_mode == 0) quant_roundtrip(hf, FF, hd);
        else if (act_mode == 2) for (int f = 0; f < FF; f++) hd[f] = or_f16_decode(or_f16_encode(hf[f]));
        else for (int f = 0; f < FF; f++) hd[f] = hf[f];
        mv_d(d, D, FF, hd, out);
    }
    free(gv); free(uv); free(hd); free(hf);
}

/* Shared expert of split-Q8 matrices (pf_gemm wtype 0, q36_engine.cu:
 * 3403-3406, used for the shared expert at :3464-3469): x quantised per 32
 * by k_quant_q8b, int8 gate/up, SwiGLU in fp32, h quantised the same way,
 * int8 down; act_mode 1 keeps x and h unquantised (the decode matvecs,
 * :1627-1629). */
static void expert_q8_d(const or_weights *w, int D, int FF, const float *x, int act_mode, double *out) {
    double *xd = (double *)malloc(sizeof(double) * (size_t)D);
    double *g = (double *)malloc(sizeof(double) * (size_t)FF);
    double *u = (double *)malloc(sizeof(double) * (size_t)FF);
    double *hd = (double *)malloc(sizeof(double) * (size_t)FF);
    float *hf = (float *)malloc(sizeof(float) * (size_t)FF);
    int K = D > FF ? D : FF;
    int8_t *q = (int8_t *)malloc((size_t)K);
    float *sc = (float *)malloc(sizeof(float) * (size_t)K / 32);
    if (act_mode == 0) {
        or_quant_q8b(x, D, q, sc);
        for (int j = 0; j < D; j++) xd[j] = (double)q[j] * (double)sc[j / 32];
    } else {
        for (int j = 0; j < D; j++) xd[j] = x[j];
    }
    mv_q8_d(w->sh_gate_q8, w->sh_gate_q8d, FF, D, xd, g);
    mv_q8_d(w->sh_up_q8, w->sh_up_q8d, FF, D, xd, u);
    for (int f = 0; f < FF; f++) hf[f] = (float)(silu_d(g[f]) * u[f]);
    if (act_mode == 0) {
        or_quant_q8b(hf, FF, q, sc);
        for (int f = 0; f < FF; f++) hd[f] = (double)q[f] * (double)sc[f / 32];
    } else {
        for (int f = 0; f < FF; f++) hd[f] = hf[f];
    }
    mv_q8_d(w->sh_down_q8, w->sh_down_q8d, D, FF, hd, out);
    free(xd); free(g); free(u); free(hd); free(hf); free(q); free(sc);
}

void or_expert_h_q8(const int8_t *gq, const uint16_t *gd, const int8_t *uq, const uint16_t *ud, int D, int FF,
                    const double *x, double *h) {
    double *u = (double *)malloc(sizeof(double) * (size_t)FF);
    mv_q8_d(gq, gd, FF, D, x, h);
    mv_q8_d(uq, ud, FF, D, x, u);
    for (int f = 0; f < FF; f++) h[f] = silu_d(h[f]) * u[f];
    free(u);
}

void or_expert_h(const uint8_t *gate, const uint8_t *up, int D, int FF,
                 const double *x, double *h) {
    double *u = (double *)malloc(sizeof(double) * (size_t)FF);
    mv_d(gate, FF, D, x, h);
    mv_d(up, FF, D, x, u);
    for (int f = 0; f < FF; f++) h[f] = silu_d(h[f]) * u[f];
    free(u);
}

void or_expert_down(const uint8_t *down, int D, int FF, const double *h, double *y) {
    mv_d(down, D, FF, h, y);
}

void or_moe_forward(const or_weights *w, const float *x, const float *logits,
                    int ld_logits, const float *shg, int T, int k,
                    float scale, int act_mode, const int32_t *tokens,
                    int n_tok, double *out) {
    int D = w->d_model, FF = w->d_ff, E = w->n_expert;
    size_t es = (size_t)FF * (D / 32) * 17;   /* gate/up bytes per expert */
    size_t ds = (size_t)D * (FF / 32) * 17;   /* down bytes per expert */
    if (!tokens) n_tok = T;
    /* tokens are independent: the parallel loop changes no arithmetic */
    #pragma omp parallel for schedule(dynamic, 1)
    for (int i = 0; i < n_tok; i++) {
        double *xd = (double *)malloc(sizeof(double) * (size_t)D);
        double *y = (double *)malloc(sizeof(double) * (size_t)D);
        int32_t idx[64];
        double wt[64];
        int t = tokens ? tokens[i] : i;
        const float *xt = x + (size_t)t * D;
        if (act_mode == 0 || act_mode == 2) quant_roundtrip(xt, D, xd);
        else for (int j = 0; j < D; j++) xd[j] = xt[j];
        or_router_topk(logits + (size_t)t * ld_logits, 1, E, ld_logits, k, scale, 1, idx, wt);
        double *o = out + (size_t)i * D;
        for (int j = 0; j < D; j++) o[j] = 0.0;
        /* sum over slots in top-k order, then the gated shared expert
         * (k_moe_combine, q36_engine.cu:784-791; k_moe_combine_pf :3393-3401) */
        for (int s = 0; s < k; s++) {
            int e = idx[s];
            expert_d(w->gate + es * e, w->up + es * e, w->down ? w->down + ds * e : 0,
                     w->down_q8 ? w->down_q8 + (size_t)D * FF * e : 0,
                     w->down_q8 ? w->down_q8d + (size_t)D * (FF / 32) * e : 0, D, FF, xd, act_mode, y);
            for (int j = 0; j < D; j++) o[j] += wt[s] * y[j];
        }
        if (shg && w->sh_gate_q8) {
            expert_q8_d(w, D, w->d_ff_sh, xt, act_mode, y);
            double gsh = sigm_d((double)shg[t]);
            for (int j = 0; j < D; j++) o[j] += gsh * y[j];
        } else if (shg && w->sh_gate) {
            expert_d(w->sh_gate, w->sh_up, w->sh_down, 0, 0, D, w->d_ff_sh, xd, act_mode, y);
            double gsh = sigm_d((double)shg[t]);
            for (int j = 0; j < D; j++) o[j] += gsh * y[j];
        }
        free(xd); free(y);
    }
}

/* ---------------------------------------------------------------------- */
/* fp32 layer forward: the timed CPU baseline.                             */
/* ---------------------------------------------------------------------- */
static void mv_f(const uint8_t *W, int M, int K, const float *x, float *y,
                 int nthreads) {
#ifdef _OPENMP
    #pragma omp parallel num_threads(nthreads)
    {
        int nt = omp_get_num_threads(), id = omp_get_thread_num();
        int r0 = (int)((long)M * id / nt), r1 = (int)((long)M * (id + 1) / nt);
        gemv_rows(W, r0, r1, K, x, y);
    }
#else
    (void)nthreads;
    gemv_rows(W, 0, M, K, x, y);
#endif
}

static void quant_roundtrip_f(const float *v, int K, float *out) {
    uint8_t *q = (uint8_t *)malloc((size_t)K), *s = (uint8_t *)malloc((size_t)K / 32);
    or_quant_e4m3(v, 1, K, q, s);
    for (int j = 0; j < K; j++) out[j] = or_e4m3_decode(q[j]) * (float)or_e8m0(s[j / 32]);
    free(q); free(s);
}

void or_moe_forward_f32(const or_weights *w, const float *x, const float *logits,
                        int ld_logits, const float *shg, int T, int k,
                        float scale, float *out, int nthreads) {
    if (!w->down) return;   /* MXFP4 down only (the timed baseline's format) */
    int D = w->d_model, FF = w->d_ff, E = w->n_expert;
    int FFm = FF > w->d_ff_sh ? FF : w->d_ff_sh;
    size_t es = (size_t)FF * (D / 32) * 17, ds = (size_t)D * (FF / 32) * 17;
    float *xf = (float *)malloc(sizeof(float) * (size_t)D);
    float *g = (float *)malloc(sizeof(float) * (size_t)FFm);
    float *u = (float *)malloc(sizeof(float) * (size_t)FFm);
    float *h = (float *)malloc(sizeof(float) * (size_t)FFm);
    float *y = (float *)malloc(sizeof(float) * (size_t)D);
    int32_t *idx = (int32_t *)malloc(sizeof(int32_t) * (size_t)k);
    double *wt = (double *)malloc(sizeof(double) * (size_t)k);
    for (int t = 0; t < T; t++) {
        quant_roundtrip_f(x + (size_t)t * D, D, xf);
        or_router_topk(logits + (size_t)t * ld_logits, 1, E, ld_logits, k, scale, 1, idx, wt);
        float *o = out + (size_t)t * D;
        for (int j = 0; j < D; j++) o[j] = 0.0f;
        int nexp = k + ((shg && w->sh_gate) ? 1 : 0);
        for (int s = 0; s < nexp; s++) {
            const uint8_t *G, *U, *Dn; int F; float ws;
            if (s < k) {
                int e = idx[s];
                G = w->gate + es * e; U = w->up + es * e; Dn = w->down + ds * e;
                F = FF; ws = (float)wt[s];
            } else {
                G = w->sh_gate; U = w->sh_up; Dn = w->sh_down; F = w->d_ff_sh;
                ws = 1.0f / (1.0f + expf(-shg[t]));
            }
            mv_f(G, F, D, xf, g, nthreads);
            mv_f(U, F, D, xf, u, nthreads);
            for (int f = 0; f < F; f++) h[f] = g[f] / (1.0f + expf(-g[f])) * u[f];
            quant_roundtrip_f(h, F, h);
            mv_f(Dn, D, F, h, y, nthreads);
            for (int j = 0; j < D; j++) o[j] += ws * y[j];
        }
    }
    free(xf); free(g); free(u); free(h); free(y); free(idx); free(wt);
}
