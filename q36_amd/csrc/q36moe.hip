// q36moe: W4A8 (MXFP4 weight x FP8-e4m3 activation) mixture-of-experts
// layer for MI355X (gfx950).  Kernels + the C ABI declared in q36moe.h.
//
// One forward runs on the context stream with no host synchronisation.
// Direct path (decode, T <= 16):
//   k_direct_gateup  (entry, 16 or 32 rows): every wave routes the token
//              (softmax top-k, q36_ops.cuh:397-431), quantises its quarter of
//              x (per-32 E8M0 + e4m3, q36_engine.cu:2411-2428), gate and up on
//              v_mfma_scale_f32_16x16x128_f8f6f4, SwiGLU rows in fp32.
//   k_direct_down    (token, 16 output rows): a wave per slot quantises its h
//              row and multiplies it by the down tile; the slots are summed in
//              slot order with the gated shared expert (q36_engine.cu:784-791).
// Sorted path (any T):
//   k_route    routing + x quantisation per token, per-block expert counts
//              and in-block ranks; k_colscan / k_scatter: the stable counting
//              sort (the deterministic k_moe_dispatch, q36_engine.cu:3387-3392)
//              and the ragged tile list.
//   k_skinny_gateup (tiles <= 32 rows) or k_gateup_dma (<= 160 rows, A and B
//              staged in LDS by direct-to-LDS loads): gate/up + SwiGLU +
//              quantisation of h in sorted order (q36_engine.cu:3436-3450).
//   k_down_lds down rows x staged h, scaled by the routing weight
//              (q36_engine.cu:3451-3463); k_combine: the weighted sum back in
//              token order (q36_engine.cu:3393-3401).
// q8_0-split matrices (the reference's requantised k-quant experts and its
// Q8_0 shared expert) run on int8 MFMA with per-32 scales: down_q8_tile in
// k_down_lds<true>, the Q8 branches of k_direct_down<true> and
// k_direct_gateup<true, *>, and the shared gate/up body (k_shared_gateup_q8,
// or the leading workgroups of k_gateup_dma).  In front of the boundary:
// k_router_f32 / k_router_f16 (router logits) and k_add_rmsnorm_quant (the
// residual + RMSNorm + quantisation producer).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <atomic>
#include <mutex>
#include <new>
#include <thread>
#include <type_traits>
#include <vector>

#include "q36moe.h"

typedef int v8i __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));

namespace {

constexpr int kMaxExperts = 256;
constexpr int kMaxTopK = 8;
constexpr int kRouteTPB = 16;      // most tokens per k_route workgroup (one wavefront each)
constexpr int kRouteTPBSmall = 4;  // tokens per workgroup for small batches (T <= kRouteSmallT)
constexpr int kRouteSmallT = 512;
constexpr int kRouteD = 2048;     // d_model of k_route (the q36 shape, q36.h:78-84)
constexpr int kDirectMaxT = 16;    // largest batch routed to the direct (unsorted) path
constexpr int kDirect2Tiles = 8;   // direct gate/up: two row tiles per workgroup from this batch on
// Cache policy of weight loads that are read once: non-temporal.  +6% in a
// stream probe; the one-kernel skinny path at decode32 went 52.7 -> 48.3 us,
// decode1 10.2 -> 9.8, prefill4096 217 -> 212.5.
constexpr int kNt = 2;

// ---------------------------------------------------------------------------
// scalar formats
// ---------------------------------------------------------------------------

// OCP E4M3FN, round-to-nearest-even, saturating at +-448, NaN -> 0x7f
// (whatever its sign).
__device__ __forceinline__ uint32_t e4m3_encode(float v) {
    const uint32_t u = __float_as_uint(v);
    const uint32_t sign = (u >> 24) & 0x80u;
    const uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return 0x7fu;
    if (a >= 0x43e00000u) return sign | 0x7eu;
    if (a < 0x3c800000u) {
        const float q = __builtin_rintf(__uint_as_float(a) * 512.0f);
        return sign | (uint32_t)q;
    }
    uint32_t r = (((a >> 23) - 120u) << 3) | ((a >> 20) & 7u);
    const uint32_t rb = (a >> 19) & 1u, sticky = a & 0x7ffffu;
    r += rb & ((sticky != 0u) | (r & 1u));
    return sign | (r > 0x7eu ? 0x7eu : r);
}

// Four scaled values to e4m3 bytes (first value in the low byte).  The
// hardware conversion (v_cvt_pk_fp8_f32: OCP E4M3FN, round to nearest even)
// equals e4m3_encode for every finite |v| <= 448 -- all the per-32
// quantiser produces from a finite block -- as an exhaustive run over all
// 2^32 fp32 patterns showed; NaN and infinities, where the hardware neither
// saturates nor canonicalises NaN, go through e4m3_encode.
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
    const bool fin = __builtin_isfinite(a) & __builtin_isfinite(b) & __builtin_isfinite(c) &
                     __builtin_isfinite(d);
    if (__builtin_expect(fin, 1)) {
        int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
        w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
        return (uint32_t)w;
    }
    return e4m3_encode(a) | (e4m3_encode(b) << 8) | (e4m3_encode(c) << 16) | (e4m3_encode(d) << 24);
}

// e2 = ceil(log2(amax/448)) from the binary exponent of the fp32 quotient,
// clamped to [-127, 127]; -127 for an all-zero block.
__device__ __forceinline__ int quant_exp(float amax) {
    // amax = 1.m * 2^E with amax / 448 a normal float: the quotient is
    // (1.m / 1.75) * 2^(E-8), and 1.m / 1.75 lies in [0.57, 1] or in
    // (1 + 0.57 * 2^-23, 1.143) -- never within rounding of a power of two --
    // so e2 = E - 8, plus 1 when 1.m > 1.75, equals the division's result
    const uint32_t ub = __float_as_uint(amax), bexp = ub >> 23;   // sign 0 for amax > 0
    if (bexp >= 10u && bexp <= 254u) return (int)bexp - 135 + ((ub & 0x7fffffu) > 0x600000u ? 1 : 0);
    if (!(amax > 0.0f)) return -127;
    // an infinite amax: the reference's ceil(log2(inf)) saturates in its
    // float-to-int conversion and clamps to 127 (scale 0: finite codes 0,
    // the infinite element NaN)
    if (amax > 3.40282347e38f) return 127;
    const float q = amax / 448.0f;
    int ex;
    const float f = frexpf(q, &ex);
    int e2 = (f == 0.5f) ? ex - 1 : ex;
    e2 = e2 < -127 ? -127 : e2;
    return e2 > 127 ? 127 : e2;
}

// 2^-e2 assembled from exponent bits (0.0 for e2 = 127, as in the reference).
__device__ __forceinline__ float inv_scale(int e2) {
    return __uint_as_float((uint32_t)(127 - e2) << 23);
}

__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// g * sigmoid(g) on the hardware exp2 and reciprocal (about 2 ulp; h is
// quantised to e4m3 right after, whose step is 2^-3 relative)
__device__ __forceinline__ float silu(float g) {
    return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * 1.44269504088896341f));
}

// v_mfma_scale_f32_16x16x128_f8f6f4, A = E2M1 (cbsz 4), B = E4M3 (blgp 0).
// Operand layout on gfx950 (measured with q36moe_probe_mfma):
//   A (E2M1, 4 VGPRs): lane L = row L%16, 32 consecutive K 32*(L/16).. with
//       element j in nibble j (low nibble first).
//   B (E4M3, 8 VGPRs): lane L = column L%16; bytes 0-15 hold K 16q..16q+15,
//       bytes 16-31 hold K 64+16q..64+16q+15, q = L/16.
//   scales: byte 0 of sa / sb; K block kb (K 32kb..32kb+31) is scaled by the
//       values of lane group kb (A: lane row+16kb, B: lane col+16kb).
//   C: lane L holds rows 4*(L/16)+i, i = 0..3, of column L%16.
//
// Scale operands are never computed by VALU right before the MFMA: the A
// scale dword is used as loaded with the byte picked by op_sel (SEL), the B
// scale comes from an LDS byte load.  A VALU-shifted scale register issued
// two wait states before v_mfma_scale was read stale on gfx950 (inf/NaN
// from garbage E8M0 bytes).
template <int SEL, int SELB = 0>
__device__ __forceinline__ v4f mfma_f4xf8(const v8i &a, const v8i &b, const v4f &c,
                                          int sa, int sb) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 4, 0, SEL, sa, SELB, sb);
}

template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

// ---------------------------------------------------------------------------
// routing + activation quantisation
// ---------------------------------------------------------------------------

// Order-preserving key of a float logit (larger value -> larger key); NaN
// maps to 0 so it is never picked (the reference's `v > best` never takes
// a NaN either).
__device__ __forceinline__ uint32_t logit_key(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (u & 0x7fffffffu) > 0x7f800000u ? 0u : k;   // selects, no branch
}

// Top-k routing of one token by one wavefront, without k serial rounds of
// cross-lane argmax:
//   1. a lower bound B on the k-th largest key: the minimum of the maxima of
//      eight disjoint 8-lane groups (eight distinct keys are >= B, so at least
//      k <= 8 keys clear it);
//   2. the keys >= B (the candidates; about 2k for N(0,1) logits) are packed
//      into LDS in ascending index order (mbcnt prefix);
//   3. each candidate's rank under (value desc, index asc) -- the order of
//      the reference's k rounds of warp argmax with ties to the lower index
//      (q36_ops.cuh:409-427) -- is counted against the other candidates
//      (a key below B cannot outrank one at or above it); ranks < k are the
//      picks and the rank is the slot;
//   4. lane r < k owns pick r; its weight is exp(l_r - max) / sum_q exp(l_q -
//      max) * scale, the reference's exp(l-m)/sum_all renormalised over the
//      picks (q36_ops.cuh:424-430), in which the full denominator cancels;
//      the sum runs in slot order as the reference's renormalisation does.
// `lds` is kRouteLds words private to the wave (16-byte aligned): [0,8) pick
// keys, [8,16) pick indices, then up to 256 (key, index) candidates and 16
// zero pads.
constexpr int kRouteLds = 2 * kMaxTopK + 2 * (kMaxExperts + 16);

struct Pick {
    int idx;     // expert index of pick `lane` (lanes < k)
    int slot;    // its rank in (value desc, index asc) order (== lane)
    float w;     // renormalised weight times scale
};

// exp(x) on the hardware exp2 (v_exp_f32), about 1 ulp; routing weights only.
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

__device__ __forceinline__ float key_val(uint32_t kk) {
    return __uint_as_float((kk & 0x80000000u) ? (kk & 0x7fffffffu) : ~kk);
}

// max of a over the 4 lanes of its quad (lanes 4j..4j+3), in every lane:
// DPP quad permutes (xor 1, xor 2) instead of two LDS shuffles.
__device__ __forceinline__ float max_quad(float a) {
    a = fmaxf(a, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0xB1, 0xf, 0xf, false)));
    return fmaxf(a, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x4E, 0xf, 0xf, false)));
}

// max of a over lanes l, l^16, l^32, l^48, in every lane: v_permlane16_swap
// / v_permlane32_swap put the two rows (halves) of each pair side by side
// in two registers -- VALU work, where a shuffle is an LDS round trip
// (ds_bpermute).  Same result as fmaxf with __shfl_xor 16 then 32 (fmaxf is
// commutative, NaN included).
__device__ __forceinline__ float max_rows4(float a) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(a), false, false);
    a = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(a), false, false);
    return fmaxf(__uint_as_float(t[0]), __uint_as_float(t[1]));
}

// max over each aligned group of 8 lanes, in every lane of the group
__device__ __forceinline__ uint32_t group8_max(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xf, 0xf, false));   // quad xor 1
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xf, 0xf, false));   // quad xor 2
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xf, 0xf, false));  // half-row mirror
    return v;
}

// Steps 1-3: the picks' keys go to lds[0, k) and their indices to
// lds[kMaxTopK, kMaxTopK + k), in slot order.  Returns, in every lane, the
// expert index of slot `want` (wave-uniform; -1 for none), taken from the
// ranking lanes by ballot so a caller that needs one slot does not wait for
// the pick writes.  The writes are made visible by route_sync().
// The token's logits, lane + 64j.  The four loads are unconditional and
// independent (a guarded load would be sunk into a branch and waited on one
// at a time).
__device__ __forceinline__ void route_load(const float *__restrict__ l, int E, float (&lv)[4]) {
    const int lane = __lane_id();
#pragma unroll
    for (int j = 0; j < 4; j++) lv[j] = l[min(lane + 64 * j, E - 1)];
}

__device__ __forceinline__ int route_rank(const float (&lv)[4], int E, int k, uint32_t *lds, int want) {
    const int lane = __lane_id();
    uint32_t key[4];
    bool ok[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        ok[j] = lane + 64 * j < E;
        // an index past E reads as NaN (key 0); selecting the input rather
        // than the key keeps the load outside any branch
        key[j] = logit_key(ok[j] ? lv[j] : __uint_as_float(0x7fffffffu));
    }
    // 1. bound: min over the 8 group maxima (a group with no valid key gives 0)
    uint32_t lm = max(max(key[0], key[1]), max(key[2], key[3]));
    const uint32_t gm = group8_max(lm);
    uint32_t bnd = __builtin_amdgcn_readlane(gm, 0);
#pragma unroll
    for (int g = 1; g < 8; g++) bnd = min(bnd, (uint32_t)__builtin_amdgcn_readlane(gm, 8 * g));
    // 2. pack the candidates (index order) as 64-bit order values
    //    key << 32 | ~index: larger key first, then lower index
    uint64_t *cand = reinterpret_cast<uint64_t *>(lds + 2 * kMaxTopK);
    int nc = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const bool c = ok[j] && key[j] >= bnd;
        const uint64_t sel = __ballot(c);
        const int pos = nc + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(sel >> 32),
                                                            __builtin_amdgcn_mbcnt_lo((uint32_t)sel, 0u));
        if (c) cand[pos] = ((uint64_t)key[j] << 32) | (uint32_t)~(uint32_t)(lane + 64 * j);
        nc += __popcll(sel);
    }
    // padded to a multiple of 16 with 0, which outranks nothing
    if (lane < 16) cand[nc + lane] = 0ull;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // 3. rank each candidate; ranks below k are the picks, 16 candidates
    //    read per pass (32 per pass measured the same).
    int e = 0;
    for (int c0 = 0; c0 < nc; c0 += 64) {
        const int ci = c0 + lane;
        const uint64_t mo = cand[ci < nc ? ci : 0];
        int r = 0;
        for (int d = 0; d < nc; d += 16) {
            uint64_t o[16];
#pragma unroll
            for (int u = 0; u < 16; u++) o[u] = cand[d + u];
#pragma unroll
            for (int u = 0; u < 16; u++) r += o[u] > mo;
        }
        const bool pick = ci < nc && r < k;
        if (pick) {
            lds[r] = (uint32_t)(mo >> 32);
            lds[kMaxTopK + r] = ~(uint32_t)mo;
        }
        const uint64_t m = __ballot(pick && r == want);
        if (m) e = (int)~(uint32_t)__builtin_amdgcn_readlane((uint32_t)mo, __builtin_ctzll(m));
    }
    return e;
}

__device__ __forceinline__ void route_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Step 4, after route_sync(): the weight of slot `slot` (any lane may ask
// for any slot < k).  All eight pick keys are read at once; slots >= k add
// an exact 0 so the sum runs over slots 0..k-1 in order.
__device__ __forceinline__ float route_weight(const uint32_t *lds, int k, float scale, int slot) {
    const uint4 a = *reinterpret_cast<const uint4 *>(lds);
    const uint4 b = *reinterpret_cast<const uint4 *>(lds + 4);
    const uint32_t kk[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    const float vmax = key_val(kk[0]);
    float wsum = 0.0f;
    uint32_t mine = kk[0];
#pragma unroll
    for (int q = 0; q < kMaxTopK; q++) {
        const float t = fast_exp(key_val(kk[q]) - vmax);
        wsum += q < k ? t : 0.0f;
        mine = q == slot ? kk[q] : mine;
    }
    return fast_exp(key_val(mine) - vmax) * __builtin_amdgcn_rcpf(wsum) * scale;
}

__device__ __forceinline__ Pick route_pick(const float (&lv)[4], int E, int k, float scale, uint32_t *lds) {
    const int lane = __lane_id();
    route_rank(lv, E, k, lds, -1);
    route_sync();
    const int me = lane < k ? lane : 0;
    Pick P;
    P.idx = (int)lds[kMaxTopK + me];
    P.slot = me;
    P.w = route_weight(lds, k, scale, me);
    return P;
}

// One wavefront routes one token (k_router_topk, q36_ops.cuh:397-431) and
// writes idx/wt in slot order.  renorm = 0 gives the plain softmax
// probabilities exp(l - max) / sum_all times scale instead.
__device__ void route_token(const float *__restrict__ l, int E, int k, float scale, int renorm,
                            int32_t *idx, float *wt, int *lds_ent, uint32_t *lds) {
    float lv[4];
    route_load(l, E, lv);
    const Pick P = route_pick(lv, E, k, scale, lds);
    const int lane = __lane_id();
    float w = P.w;
    if (!renorm) {
        float vmax = -INFINITY;
#pragma unroll
        for (int q = 0; q < kMaxTopK; q++)
            if (q < k) vmax = fmaxf(vmax, key_val(lds[q]));
        float denom = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int e = lane + 64 * j;
            denom += e < E ? expf(l[e] - vmax) : 0.0f;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) denom += __shfl_xor(denom, o, 64);
        w = expf(key_val(lds[lane < k ? lane : 0]) - vmax) / denom * scale;
    }
    if (lane < k) {
        idx[P.slot] = P.idx;
        wt[P.slot] = w;
        if (lds_ent) lds_ent[P.slot] = P.idx;
    }
}

// Quantise one 32-element block (per-32 E8M0 + e4m3), q36_engine.cu:2411-2428.
__device__ __forceinline__ void quant_block32(const void *__restrict__ x, int x_fmt,
                                              size_t off, uint8_t *__restrict__ q,
                                              uint8_t *__restrict__ s) {
    float v[32];
    if (x_fmt == Q36MOE_FMT_F32) {
        const float4 *p = reinterpret_cast<const float4 *>(static_cast<const float *>(x) + off);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 t = p[i];
            v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
        }
    } else {
        const uint4 *p = reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(x) + off);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint4 t = p[i];
            const uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                v[8 * i + 2 * j] = __uint_as_float(w[j] << 16);
                v[8 * i + 2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
            }
        }
    }
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) a = fmaxf(a, fabsf(v[i]));
    const int e2 = quant_exp(a);
    const float mul = inv_scale(e2);
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
        w[i] = e4m3x4(v[4 * i] * mul, v[4 * i + 1] * mul, v[4 * i + 2] * mul, v[4 * i + 3] * mul);
    uint4 *qo = reinterpret_cast<uint4 *>(q);
    qo[0] = make_uint4(w[0], w[1], w[2], w[3]);
    qo[1] = make_uint4(w[4], w[5], w[6], w[7]);
    *s = (uint8_t)(127 + e2);
}

// Quantise 8 consecutive values held by one lane; lanes 4j..4j+3 form one
// 32-value block (amax via two xor-shuffles).  Writes 8 e4m3 bytes and,
// from the first lane of the block, the E8M0 byte.
__device__ __forceinline__ uint8_t quant8_lane(const float (&v)[8], int lane, uint8_t *q, uint8_t *sc) {
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) a = fmaxf(a, fabsf(v[i]));
    a = max_quad(a);
    const int e2 = quant_exp(a);
    const float mul = inv_scale(e2);
    const uint32_t w0 = e4m3x4(v[0] * mul, v[1] * mul, v[2] * mul, v[3] * mul);
    const uint32_t w1 = e4m3x4(v[4] * mul, v[5] * mul, v[6] * mul, v[7] * mul);
    *reinterpret_cast<uint2 *>(q) = make_uint2(w0, w1);
    if ((lane & 3) == 0) *sc = (uint8_t)(127 + e2);
    return (uint8_t)(127 + e2);
}

// 8 activations as raw bits, then widened to float: split so the load can be
// issued early (before routing) without the conversion waiting on it there.
// activations handed over already quantised (q36moe_forward_q8): x is the
// e4m3 codes [T][D], xs_in the E8M0 scales [T][D/32]
constexpr int kFmtE4M3 = 2;

struct X8 {
    u32x4 a, b;
};
__device__ __forceinline__ X8 load8_raw(const void *x, int fmt, size_t off) {
    X8 r;
    if (fmt == kFmtE4M3) {
        const uint2 v = *reinterpret_cast<const uint2 *>(static_cast<const uint8_t *>(x) + off);
        r.a = u32x4{v.x, v.y, 0u, 0u};
        r.b = u32x4{0u, 0u, 0u, 0u};
    } else if (fmt == Q36MOE_FMT_F32) {
        const u32x4 *p = reinterpret_cast<const u32x4 *>(static_cast<const float *>(x) + off);
        r.a = p[0];
        r.b = p[1];
    } else {
        r.a = *reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(x) + off);
        r.b = u32x4{0u, 0u, 0u, 0u};   // unused (no copy of r.a: that would wait on the load)
    }
    return r;
}
__device__ __forceinline__ void cvt8(const X8 &r, int fmt, float (&v)[8]) {
    if (fmt == Q36MOE_FMT_F32) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[j] = __uint_as_float(r.a[j]);
            v[4 + j] = __uint_as_float(r.b[j]);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[2 * j] = __uint_as_float(r.a[j] << 16);
            v[2 * j + 1] = __uint_as_float(r.a[j] & 0xffff0000u);
        }
    }
}
__device__ __forceinline__ void load8(const void *x, int fmt, size_t off, float (&v)[8]) {
    cvt8(load8_raw(x, fmt, off), fmt, v);
}

// The per-32 int8 quantiser of h for a q8_0-split down (k_quant_q8b,
// q36_engine.cu:2627-2640): d = amax/127, code = rint(v * 127/amax) clamped
// to [-127, 127], all zero for an all-zero block.
__device__ __forceinline__ float q8b_inv(float amax) { return amax > 0.0f ? 127.0f / amax : 0.0f; }
__device__ __forceinline__ uint32_t q8b4(float a, float b, float c, float d, float inv) {
    auto one = [inv](float v) {
        const float r = fminf(fmaxf(__builtin_rintf(v * inv), -127.0f), 127.0f);
        return (uint32_t)((int)r & 255);
    };
    return one(a) | (one(b) << 8) | (one(c) << 16) | (one(d) << 24);
}

// f16 bit patterns (low / high half of a dword) to float
__device__ __forceinline__ float f16lo(uint32_t d) { return (float)__builtin_bit_cast(_Float16, (uint16_t)d); }
__device__ __forceinline__ float f16hi(uint32_t d) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(d >> 16)); }

// Scaling an int8 block result without an integer-to-float convert: the
// MFMA accumulates onto kQ8Bias (the fp32 bits of 1.5 * 2^23), so its i32
// result r = kQ8Bias + ci reads as the fp32 value 12582912 + ci exactly
// (|ci| <= 32 * 128 * 128 < 2^22).  A weight scale w is an f16 value, so
// 12582912 * w is exact in fp32 and fma(r, w, -12582912 * w) = round(ci * w),
// one rounding, as convert-then-multiply has.  The block then costs two fmas
// per output (this and the one applying the activation scale) once
// -12582912 * w is at hand.
constexpr int kQ8Bias = 0x4B400000;
constexpr float kQ8BiasF = 12582912.0f;
__device__ __forceinline__ float q8_scaled(int r, float w, float nwb) { return fmaf(__int_as_float(r), w, nwb); }

struct RouteArgs {
    const float *logits; int ld; int T; int E; int k; float scale;
    const void *x; int x_fmt; int D; int nb;
    int32_t *idx; float *wt; uint8_t *xq; uint8_t *xs; uint8_t *xs2;
    int32_t *blk_cnt; int32_t *rank;
    const uint8_t *xs_in;     // scales of pre-quantised x (x_fmt kFmtE4M3)
    int8_t *xq8; float *xsf;  // int8 x + fp32 scales per 32 for a q8_0-split shared expert, or null
    int counts;               // write blk_cnt / rank (0: the one-kernel skinny path sorts itself)
};

// One wavefront per token, TPB tokens per workgroup: top-k routing,
// FP8 quantisation of x (8 values per lane, 4 lanes per 32-block), then the
// block's per-expert counts (expert-major, blk_cnt[e][block]) and each
// entry's rank among the block's earlier entries of the same expert (the
// stable order of the sort), from a per-expert mask of the block's tokens.
// Small batches use 4 tokens per workgroup to spread the quantisation over
// more CUs; large ones 16, which keeps the per-block count table short.
// FP8 quantisation of values 512c .. 512c+511 of token t's x (8 per lane,
// 4 lanes per 32-block): codes, E8M0 scales in both layouts, and the int8 x
// of a q8_0-split shared expert when A.xq8 is set.
template <int XF>
__device__ __forceinline__ void route_quant_pass(const RouteArgs &A, int t, int c, const X8 &xr, int lane) {
    const int nb32 = A.D / 32;
    const size_t o = (size_t)t * A.D + c * 512 + lane * 8;
    const int b = c * 16 + (lane >> 2);
    float v[8];
    cvt8(xr, XF, v);
    const uint8_t sb = quant8_lane(v, lane, A.xq + o, A.xs + (size_t)t * nb32 + b);
    // lane-group-major copy for the grouped GEMM: [t][b % 4][b / 4]
    if ((lane & 3) == 0) A.xs2[(size_t)t * nb32 + (b & 3) * (nb32 / 4) + (b >> 2)] = sb;
    if (A.xq8) {   // the q8_0-split shared expert's int8 x (k_quant_q8b)
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) a = fmaxf(a, fabsf(v[i]));
        a = max_quad(a);
        const float inv = q8b_inv(a);
        *reinterpret_cast<uint2 *>(A.xq8 + o) =
            make_uint2(q8b4(v[0], v[1], v[2], v[3], inv), q8b4(v[4], v[5], v[6], v[7], inv));
        if ((lane & 3) == 0) A.xsf[(size_t)t * nb32 + b] = a / 127.0f;
    }
}

// XF: the x format (A.x_fmt), fixed at compile time so the loads and their
// waits are branch-free.
template <int TPB, int XF>
__global__ __launch_bounds__(64 * TPB) void k_route(RouteArgs A) {
    __shared__ uint32_t tmask[kMaxExperts];
    __shared__ int ent[TPB * kMaxTopK];
    __shared__ __align__(16) uint32_t rlds[TPB][kRouteLds];
    static_assert(TPB <= 32, "token mask");
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t0 = blockIdx.x * TPB;
    const int nb32 = A.D / 32;
    if (A.counts) {   // uniform
        for (int e = threadIdx.x; e < A.E; e += 64 * TPB) tmask[e] = 0u;
        __syncthreads();
    }
    const int t = t0 + wave;
    if (t < A.T) {
        // x of the token (kRouteD values, 8 per lane per pass), then the
        // logits.  Each pass is quantised as soon as its x is in and the
        // routing comes last: at large T every CU's loads are queued behind
        // the whole x stream, so routing first would leave the SIMDs idle
        // until the logits (the last bytes to arrive) were in.
        constexpr bool preq = XF == kFmtE4M3;
        X8 xr[kRouteD / 512];
        if constexpr (!preq) {
#pragma unroll
            for (int c = 0; c < kRouteD / 512; c++) xr[c] = load8_raw(A.x, XF, (size_t)t * A.D + c * 512 + lane * 8);
        }
        float lv[4];
        route_load(A.logits + (size_t)t * A.ld, A.E, lv);
        if constexpr (preq) {
            // codes stay where the caller put them; only the lane-group-major
            // copy of the scales is made for the grouped GEMM
            for (int b = lane; b < nb32; b += 64)
                A.xs2[(size_t)t * nb32 + (b & 3) * (nb32 / 4) + (b >> 2)] = A.xs_in[(size_t)t * nb32 + b];
        } else {
#pragma unroll
        for (int c = 0; c < kRouteD / 512; c++) route_quant_pass<XF>(A, t, c, xr[c], lane);
        }
        const Pick P = route_pick(lv, A.E, A.k, A.scale, rlds[wave]);
        if (lane < A.k) {
            A.idx[(size_t)t * A.k + lane] = P.idx;
            A.wt[(size_t)t * A.k + lane] = P.w;
            if (A.counts) {
                ent[wave * A.k + lane] = P.idx;
                atomicOr(&tmask[P.idx], 1u << wave);
            }
        }
    }
    if (!A.counts) return;
    __syncthreads();
    const int ntok = min(TPB, A.T - t0);
    if (threadIdx.x < ntok * A.k) {
        const int tl = threadIdx.x / A.k;
        const int e = ent[threadIdx.x];
        A.rank[(size_t)t0 * A.k + threadIdx.x] = __popc(tmask[e] & ((1u << tl) - 1u));
    }
    for (int e = threadIdx.x; e < A.E; e += 64 * TPB)
        A.blk_cnt[(size_t)e * A.nb + blockIdx.x] = __popc(tmask[e]);
}

// k_route without the per-block counts (the one-kernel skinny path sorts
// itself), one token per workgroup: wave w < 4 quantises values 512w ..
// 512w+511 and wave 4 routes, so the routing chain (logits load, ranking,
// stores) runs beside the quantisation instead of after a pass of it.
constexpr int kRouteTokW = kRouteD / 512 + 1;
template <int XF>
__global__ __launch_bounds__(64 * kRouteTokW) void k_route_tok(RouteArgs A) {
    __shared__ __align__(16) uint32_t rlds[kRouteLds];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int t = blockIdx.x;
    constexpr bool preq = XF == kFmtE4M3;
    constexpr int RW = kRouteTokW - 1;   // the routing wave
    if (wave == RW) {
        float lv[4];
        route_load(A.logits + (size_t)t * A.ld, A.E, lv);
        const Pick P = route_pick(lv, A.E, A.k, A.scale, rlds);
        if (lane < A.k) {
            A.idx[(size_t)t * A.k + lane] = P.idx;
            A.wt[(size_t)t * A.k + lane] = P.w;
        }
        return;
    }
    if constexpr (preq) {
        const int nb32 = A.D / 32;
        for (int b = threadIdx.x; b < nb32; b += 64 * RW)
            A.xs2[(size_t)t * nb32 + (b & 3) * (nb32 / 4) + (b >> 2)] = A.xs_in[(size_t)t * nb32 + b];
    } else {
        const X8 xr = load8_raw(A.x, XF, (size_t)t * A.D + wave * 512 + lane * 8);
        route_quant_pass<XF>(A, t, wave, xr, lane);
    }
}

template <int TPB>
static void launch_route_tpb(int nb, hipStream_t s, const RouteArgs &ra) {
    switch (ra.x_fmt) {
        case Q36MOE_FMT_F32:
            hipLaunchKernelGGL((k_route<TPB, Q36MOE_FMT_F32>), dim3(nb), dim3(64 * TPB), 0, s, ra);
            break;
        case Q36MOE_FMT_BF16:
            hipLaunchKernelGGL((k_route<TPB, Q36MOE_FMT_BF16>), dim3(nb), dim3(64 * TPB), 0, s, ra);
            break;
        default:
            hipLaunchKernelGGL((k_route<TPB, kFmtE4M3>), dim3(nb), dim3(64 * TPB), 0, s, ra);
            break;
    }
}

static void launch_route(bool large, int nb, hipStream_t s, const RouteArgs &ra) {
    if (!ra.counts) {
        switch (ra.x_fmt) {
            case Q36MOE_FMT_F32:
                hipLaunchKernelGGL(k_route_tok<Q36MOE_FMT_F32>, dim3(ra.T), dim3(64 * kRouteTokW), 0, s, ra);
                break;
            case Q36MOE_FMT_BF16:
                hipLaunchKernelGGL(k_route_tok<Q36MOE_FMT_BF16>, dim3(ra.T), dim3(64 * kRouteTokW), 0, s, ra);
                break;
            default:
                hipLaunchKernelGGL(k_route_tok<kFmtE4M3>, dim3(ra.T), dim3(64 * kRouteTokW), 0, s, ra);
                break;
        }
        return;
    }
    if (large) launch_route_tpb<kRouteTPB>(nb, s, ra);
    else launch_route_tpb<kRouteTPBSmall>(nb, s, ra);
}

__global__ __launch_bounds__(256) void k_topk(const float *logits, int T, int E, int ld, int k,
                                             float scale, int renorm, int32_t *idx, float *wt) {
    __shared__ __align__(16) uint32_t rlds[4][kRouteLds];
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;
    route_token(logits + (size_t)t * ld, E, k, scale, renorm, idx + (size_t)t * k, wt + (size_t)t * k,
                nullptr, rlds[threadIdx.x >> 6]);
}

__global__ __launch_bounds__(256) void k_quant(const void *x, int x_fmt, int T, int K,
                                              uint8_t *xq, uint8_t *xs) {
    const long nblk = (long)T * (K / 32);
    const long b = (long)blockIdx.x * 256 + threadIdx.x;
    if (b >= nblk) return;
    quant_block32(x, x_fmt, (size_t)b * 32, xq + (size_t)b * 32, xs + b);
}

// ---------------------------------------------------------------------------
// sort: offsets, stable scatter, tile list
// ---------------------------------------------------------------------------
struct ScanArgs {
    const int32_t *blk_cnt; int nb; int tpb; int inline_cols; int E; int T; int k;
    const int32_t *idx; const float *wt; const int32_t *rank; const float *shg; int ld_shg;
    int tn;      // rows per routed tile
    int tn_sh;   // rows per shared-expert tile
    int32_t *blk_off; int32_t *tot; int32_t *e_off; int32_t *perm; int32_t *pos;
    int32_t *row_tok; float *row_w; int4 *tiles; int32_t *ntiles;
};

// Column scans: for each expert, the exclusive prefix of its per-block counts
// (blk_off[e][b]) and its total.  kColExp experts per workgroup, 256 / kColExp
// threads per expert, each summing a contiguous run of blocks.
constexpr int kColExp = 8;
constexpr int kScanInlineBlocks = 64;   // k_scatter does the column scan itself up to this many blocks
__global__ __launch_bounds__(256) void k_colscan(ScanArgs A) {
    constexpr int NP = 256 / kColExp;              // partitions per expert: one half-wave
    static_assert(NP == 32, "one expert per half-wave");
    constexpr int CH = 8;                          // counts held in registers per thread
    const int lane = threadIdx.x & 63;
    const int el = threadIdx.x / NP, pi = threadIdx.x % NP;
    const int e = blockIdx.x * kColExp + el;
    const bool ok = e < A.E;
    const int chunk = (A.nb + NP - 1) / NP;
    const int b0 = pi * chunk, b1 = min(A.nb, b0 + chunk);
    const int32_t *cnt = A.blk_cnt + (size_t)e * A.nb;
    // all of a thread's counts are loaded at once (one memory round trip)
    int v[CH], sum = 0;
    if (chunk <= CH) {
#pragma unroll
        for (int j = 0; j < CH; j++) {
            v[j] = ok && b0 + j < b1 ? cnt[b0 + j] : 0;
            sum += v[j];
        }
    } else if (ok) {
        for (int b = b0; b < b1; b++) sum += cnt[b];
    }
    // inclusive scan over the expert's 32 lanes: row_shr 1/2/4/8 inside each
    // 16-lane row, then row_bcast15 adds row 0's (row 2's) total to row 1 (3)
    int inc = sum;
    inc += __builtin_amdgcn_update_dpp(0, inc, 0x111, 0xf, 0xf, false);
    inc += __builtin_amdgcn_update_dpp(0, inc, 0x112, 0xf, 0xf, false);
    inc += __builtin_amdgcn_update_dpp(0, inc, 0x114, 0xf, 0xf, false);
    inc += __builtin_amdgcn_update_dpp(0, inc, 0x118, 0xf, 0xf, false);
    inc += __builtin_amdgcn_update_dpp(0, inc, 0x142, 0xa, 0xf, false);
    const int total = __shfl(inc, (lane & 32) | 31, 64);
    if (!ok) return;
    int run = inc - sum;
    if (chunk <= CH) {
#pragma unroll
        for (int j = 0; j < CH; j++)
            if (b0 + j < b1) {
                A.blk_off[(size_t)e * A.nb + b0 + j] = run;
                run += v[j];
            }
    } else {
        for (int b = b0; b < b1; b++) {
            const int c = cnt[b];
            A.blk_off[(size_t)e * A.nb + b] = run;
            run += c;
        }
    }
    if (pi == 0) A.tot[e] = total;
}

// Exclusive scan of v[0..n) (n <= 256) by one wavefront into out (LDS).
__device__ __forceinline__ void wave_scan256(const int *v, int n, int *out, int *total) {
    const int lane = __lane_id();
    int a[4], s = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        a[j] = (4 * lane + j < n) ? v[4 * lane + j] : 0;
        s += a[j];
    }
    // inclusive scan over the wave: row_shr 1/2/4/8 within each 16-lane row
    // (lanes without a source add 0), then the rows' totals by row_bcast15
    // (rows 1, 3) and row_bcast31 (rows 2, 3) -- DPP moves, not LDS shuffles
    int inc = s;
    inc += __builtin_amdgcn_update_dpp(0, inc, 0x111, 0xf, 0xf, false);
    inc += __builtin_amdgcn_update_dpp(0, inc, 0x112, 0xf, 0xf, false);
    inc += __builtin_amdgcn_update_dpp(0, inc, 0x114, 0xf, 0xf, false);
    inc += __builtin_amdgcn_update_dpp(0, inc, 0x118, 0xf, 0xf, false);
    inc += __builtin_amdgcn_update_dpp(0, inc, 0x142, 0xa, 0xf, false);
    inc += __builtin_amdgcn_update_dpp(0, inc, 0x143, 0xc, 0xf, false);
    int run = inc - s;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        if (4 * lane + j < n) out[4 * lane + j] = run;
        run += a[j];
    }
    if (lane == 63 && total) *total = inc;
}

// Scatter of one route block's entries to their sorted slots: expert offsets
// from the totals (wave scan in LDS), then p = off[e] + blk_off[e][b] + rank.
// Block 0 also writes the offsets and the ragged tile list.  This is the
// deterministic replacement of the reference's atomic bucketing
// (k_moe_dispatch, q36_engine.cu:3387-3392): entry ids t*k+s ascend inside
// each expert.
// With few routing blocks (inline_cols) each workgroup also does the column
// scan itself -- every expert's counts over all blocks, a few KiB -- and
// k_colscan is not launched.
__global__ __launch_bounds__(256) void k_scatter(ScanArgs A) {
    __shared__ int tot[kMaxExperts], off[kMaxExperts + 1], ntile[kMaxExperts], toff[kMaxExperts + 1];
    __shared__ int boff[kMaxExperts];
    const int tid = threadIdx.x, b = blockIdx.x;
    // this thread's first entry and shared-gate logit are loaded up front,
    // in flight with the totals and offsets
    const int n = A.T * A.k;
    const int i0 = b * A.tpb * A.k, i1 = min(n, i0 + A.tpb * A.k);
    const int ia = i0 + tid;
    int ea = 0, ra = 0;
    float wa = 0.0f;
    if (ia < i1) {
        ea = A.idx[ia];
        ra = A.rank[ia];
        wa = A.wt[ia];
    }
    const int ts = b * A.tpb + tid, ts1 = min(A.T, (b + 1) * A.tpb);
    float sga = 0.0f;
    if (A.shg && ts < ts1) sga = A.shg[(size_t)ts * A.ld_shg];
    for (int e = tid; e < A.E; e += 256) {
        if (A.inline_cols) {
            const int32_t *cnt = A.blk_cnt + (size_t)e * A.nb;
            int run = 0, mine = 0;
            for (int bb = 0; bb < A.nb; bb++) {
                if (bb == b) mine = run;
                run += cnt[bb];
            }
            tot[e] = run;
            boff[e] = mine;
        } else {
            tot[e] = A.tot[e];
            boff[e] = A.blk_off[(size_t)e * A.nb + b];
        }
        ntile[e] = (tot[e] + A.tn - 1) / A.tn;
    }
    __syncthreads();
    if (tid < 64) wave_scan256(tot, A.E, off, &off[A.E]);
    else if (tid < 128) wave_scan256(ntile, A.E, toff, &toff[A.E]);
    __syncthreads();
    auto place = [&](int i, int e, int r, float w) {
        const int p = off[e] + boff[e] + r;
        A.perm[p] = i;
        A.pos[i] = p;
        A.row_tok[p] = i / A.k;
        A.row_w[p] = w;
    };
    if (ia < i1) place(ia, ea, ra, wa);
    for (int i = ia + 256; i < i1; i += 256) place(i, A.idx[i], A.rank[i], A.wt[i]);
    if (A.shg) {
        for (int t = ts; t < ts1; t += 256) {
            const float g = t == ts ? sga : A.shg[(size_t)t * A.ld_shg];
            A.row_tok[n + t] = t;
            A.row_w[n + t] = 1.0f / (1.0f + expf(-g));
        }
    }
    if (b == 0) {
        for (int e = tid; e <= A.E; e += 256) A.e_off[e] = off[e];
        // routed tiles in ascending column-tile count (expert order within a
        // count): the kernels walk the list backwards, so the largest tiles
        // start first and the small ones fill the tail.  Thread e counts its
        // expert's tiles per count; each wave scans its 64 experts for all
        // counts at once (DPP), and the wave totals give the offsets.
        constexpr int NBK = 10;   // column tiles of the largest (fat) tile
        static_assert(kMaxExperts <= 256, "one expert per thread");
        __shared__ int wtot[4][NBK];
        const int e = tid, lane = tid & 63, wv = tid >> 6;
        int c[NBK], inc[NBK];
#pragma unroll
        for (int k2 = 0; k2 < NBK; k2++) c[k2] = 0;
        if (e < A.E)
            for (int j = 0; j < ntile[e]; j++) {
                const int rows = min(A.tn, tot[e] - j * A.tn);
                const int k2 = (rows + 15) / 16 - 1;
#pragma unroll
                for (int k3 = 0; k3 < NBK; k3++) c[k3] += k3 == k2 ? 1 : 0;
            }
#pragma unroll
        for (int k2 = 0; k2 < NBK; k2++) {
            int v = c[k2];
            v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);
            v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);
            v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);
            v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);
            v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);
            v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);
            inc[k2] = v;
            if (lane == 63) wtot[wv][k2] = v;
        }
        __syncthreads();
        if (e < A.E) {
            int pos[NBK], base = 0;
#pragma unroll
            for (int k2 = 0; k2 < NBK; k2++) {
                int before = 0, all = 0;
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    before += w < wv ? wtot[w][k2] : 0;
                    all += wtot[w][k2];
                }
                pos[k2] = base + before + inc[k2] - c[k2];
                base += all;
            }
            for (int j = 0; j < ntile[e]; j++) {
                const int p0 = off[e] + j * A.tn;
                const int rows = min(A.tn, tot[e] - j * A.tn);
                const int k2 = (rows + 15) / 16 - 1;
                int pp = 0;
#pragma unroll
                for (int k3 = 0; k3 < NBK; k3++)
                    if (k3 == k2) pp = pos[k3]++;
                A.tiles[pp] = make_int4(e, p0, p0 + rows, 0);
            }
        }
        const int nsh = A.shg ? (A.T + A.tn_sh - 1) / A.tn_sh : 0;
        for (int j = tid; j < nsh; j += 256) {
            const int p0 = n + j * A.tn_sh;
            A.tiles[toff[A.E] + j] = make_int4(A.E, p0, min(p0 + A.tn_sh, n + A.T), 0);
        }
        if (tid == 0) *A.ntiles = toff[A.E] + nsh;
    }
}

// ---------------------------------------------------------------------------
// grouped expert GEMM on scaled MFMA
// ---------------------------------------------------------------------------

struct GemmArgs {
    const uint8_t *wa, *wb;   // routed experts: gate/up (GATEUP) or down (DOWN)
    const uint8_t *sa, *sb;   // shared expert matrices (tile.x == E)
    size_t wstride;           // bytes per expert matrix
    int E, M;                 // routed experts, rows per matrix
    const int4 *tiles; const int32_t *ntiles;
    const uint8_t *bq;        // B rows: x by token (GATEUP) / h by sorted slot (DOWN)
    const uint8_t *bs2;       // their E8M0 scales, lane-group-major [row][4][K/128]
    const int32_t *row_tok; const float *row_w;
    uint8_t *hq, *hs, *hs2;   // GATEUP output rows (sorted slot): h, natural and lane-major scales
    uint16_t *dnh;            // DOWN output rows (sorted slot), weighted, as f16 [row][ldo]
    uint8_t *dne;             // with one exponent byte per 16 columns [row][ldo / 16]
    int ldo;                  // output row length
    // q8_0-split routed down: GATEUP writes the routed rows of h as int8
    // with fp32 scales (hsf [row][ldo/32]); DOWN reads them from bsf
    int hq8;
    float *hsf; const float *bsf;
    // q8_0-split shared expert: its tiles are skipped by the MXFP4 gate/up
    // kernels (k_shared_gateup_q8 computes its rows from the int8 x) and run
    // down_q8_tile in DOWN
    int shq8;
    const int8_t *xq8; const float *xsf;   // int8 x [T][K] + fp32 scales [T][K/32]
    int T, nrouted;                        // tokens; routed rows (shared row of token t = nrouted + t)
    int sh_wgs;                            // k_gateup_dma: leading workgroups that run the shared body
};

// Quantise and store one lane's share of a 32-row block of h for sorted row
// p: h[r][i] is row ffb + 16r + 4q + i (the MFMA result layout of two row
// tiles); lanes q = 0..3 of a column hold the block.  E8M0 + e4m3 for an
// MXFP4 down, int8 + fp32 scale when q8 is set.
__device__ __forceinline__ void store_h_block(const GemmArgs &A, bool q8, int p, bool valid, int ffb,
                                              int q, int lane, const float (&h)[2][4]) {
    float amax = 0.0f;
#pragma unroll
    for (int r = 0; r < 2; r++)
#pragma unroll
        for (int i = 0; i < 4; i++) amax = fmaxf(amax, fabsf(h[r][i]));
    amax = max_rows4(amax);
    const int b = ffb / 32, nb = A.ldo / 32;
    if (q8) {
        const float inv = q8b_inv(amax);
        if (valid) {
#pragma unroll
            for (int r = 0; r < 2; r++)
                *reinterpret_cast<uint32_t *>(A.hq + (size_t)p * A.ldo + ffb + r * 16 + 4 * q) =
                    q8b4(h[r][0], h[r][1], h[r][2], h[r][3], inv);
            if (lane < 16) A.hsf[(size_t)p * nb + b] = amax / 127.0f;
        }
        return;
    }
    const int e2 = quant_exp(amax);
    const float mul = inv_scale(e2);
    if (valid) {
#pragma unroll
        for (int r = 0; r < 2; r++)
            *reinterpret_cast<uint32_t *>(A.hq + (size_t)p * A.ldo + ffb + r * 16 + 4 * q) =
                e4m3x4(h[r][0] * mul, h[r][1] * mul, h[r][2] * mul, h[r][3] * mul);
        if (lane < 16) {
            A.hs[(size_t)p * nb + b] = (uint8_t)(127 + e2);
            A.hs2[(size_t)p * nb + (b & 3) * (nb / 4) + (b >> 2)] = (uint8_t)(127 + e2);
        }
    }
}

// op_sel byte of both scale dwords (A and B hold 4 K-steps each), fixed once
// the K loop is unrolled.  `sel` must be a compile-time constant or
// wave-uniform as the compiler sees it (readfirstlane): a per-lane value
// turns the switch into EXEC-masked branches around the MFMAs, which gave
// wrong results on gfx950.
__device__ __forceinline__ v4f mfma_sel(int sel, const v8i &a, const v8i &b, const v4f &c, int sa, int sb) {
    switch (sel & 3) {
        case 0: return mfma_f4xf8<0, 0>(a, b, c, sa, sb);
        case 1: return mfma_f4xf8<1, 1>(a, b, c, sa, sb);
        case 2: return mfma_f4xf8<2, 2>(a, b, c, sa, sb);
        default: return mfma_f4xf8<3, 3>(a, b, c, sa, sb);
    }
}

// ---------------------------------------------------------------------------
// fat gate/up: A and B staged in LDS by direct-to-LDS loads
// ---------------------------------------------------------------------------
// Workgroup = (expert tile of up to kGdTok rows, 64 rows of gate and the same
// 64 rows of up), 4 waves, two workgroups per CU: while one waits at its
// per-step barrier the other keeps the matrix pipes busy.  Per K-step of 128
// the workgroup stages 8 A tiles (8 KiB of E2M1 fragments, contiguous in the
// packed layout) and the tile's B rows (128 B of each e4m3 x row) with
// buffer_load_dwordx4 ... lds: the data goes from L2 to LDS without passing
// through VGPRs, and 8 lanes cover one 128-byte x row.  A streams from HBM
// with three stages (two K-steps in flight); B mostly hits L2 and has two.
// Waves form a 2 x 2 grid: wave w computes gate and up tiles 2(w&1)..+1
// against column tiles (w>>1) + 2j.  B rows sit in LDS as 256-byte lines of
// two rows with the 16-byte slot index XORed by the line index, so the 16
// lanes of a fragment read hit 16 distinct bank groups.
constexpr int kGdTok = 160;                      // rows per fat tile (10 column tiles)
static_assert(kGdTok / 16 <= 10, "k_scatter orders tiles by column-tile count, 1..10");

// Direct-to-LDS loads are issued in their buffer (MUBUF) form, not as
// global_load_lds: the global form is a FLAT instruction that may access
// LDS, and while one is outstanding the compiler's wait counting treats the
// LDS counter as out of order, so every later LDS fragment read was waited
// on with lgkmcnt(0) (all reads of the step) instead of the count of reads
// issued after it.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dma_src(const void *base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, 0x7ffffffe, 0x00020000);
}
template <int AUX = 0>
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t off, void *lds) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16, off, 0, 0, AUX);
}

// Barrier for the staging pipeline.  A fence-based barrier would make the
// compiler wait for every outstanding direct-to-LDS load (they count as LDS
// writes), including the stages still meant to be in flight; here the wait
// for the stage about to be read is wait_vm's, and this wave's LDS reads of
// the previous stage are complete before any wave passes the barrier and
// restages that slot.
// 16-byte load with the non-temporal hint (weights read once)
__device__ __forceinline__ u32x4 ldg_nt16(const void *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}

// Workgroup barrier for LDS data only: __syncthreads() also waits for every
// outstanding global load (vmcnt(0)), which drains prefetched weights.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
__device__ __forceinline__ void dma_barrier() {
    // the scheduler may move MFMAs across an asm barrier: pin them (and all
    // else) to their step, or every step's fragments stay live at once.
    // The wait is the builtin (lgkmcnt(0) only), not inline asm: the
    // compiler's wait counting does not see inside asm, so after an asm
    // wait it still counted earlier scalar loads as outstanding and put a
    // full lgkmcnt(0) before the first fragment use of every step.
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xC07F);   // gfx9 encoding: vmcnt 63, expcnt 7, lgkmcnt 0
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
}

// byte offset of (row r, 16-byte chunk c) in a B stage
__device__ __forceinline__ int gd_boff(int r, int c) {
    const int m = r >> 1;
    return m * 256 + ((((r & 1) << 3) | c) ^ (m & 7)) * 16;
}

namespace gdma {
constexpr int RT = 4, W = 4, TOK = kGdTok;
static_assert(TOK == 16 * 2 * 5, "column tiles per wave: at most 5 (the largest body instantiated)");
constexpr int STA = 4, STB = 2;   // A stage of step kt: kt % 4, static inside a 4-step group
struct Lds {
    __align__(16) uint8_t a[STA][2 * RT * 1024];
    __align__(16) uint8_t b[STB][TOK * 128];
    __align__(16) uint8_t sc[2 * RT * 1024];
};
static_assert(sizeof(Lds) * 2 <= 160 * 1024, "two workgroups per CU");

// The K loop runs as 4 groups of 4 steps: 3 iterations of a runtime loop
// whose body has no conditions (stage slots are the step within the group,
// every load is issued unconditionally), then the last group as a static
// copy that stops the staging.  x row groups: the tile's column tiles need
// 4*NJ groups of 8 rows at most, NJ per wave (rows past the tile repeat its
// last row); a wave with fewer column tiles than its neighbours still
// covers its groups (groups w + 4i, i < NJ, reach past 2*ntt - 1).
template <int NJ>
__device__ __forceinline__ void body(const GemmArgs &A, Lds &L, const uint8_t *Wg, const uint8_t *Wu,
                                     int mt0, int p0, int p1, bool hq8) {
    constexpr int KD = 2048, NKT = KD / 128;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15, q = lane >> 4;
    const int wa = wave & 1, wt = wave >> 1;
    const int ntok = p1 - p0;
    // A: wave w stages gate tile mt0+w and up tile mt0+w; B: row groups
    // w + 4i (8 rows each) holding rows of the tile.  Sources are a uniform
    // base plus a 32-bit per-lane offset (the saddr form of the load).
    const uint32_t aoff = (uint32_t)(mt0 + wave) * NKT * 1024 + lane * 16;
    constexpr int NBI = NJ > 0 ? NJ : 1;
    uint32_t boff[NBI];
#pragma unroll
    for (int i = 0; i < NBI; i++) {
        const int m = 4 * (wave + W * i) + (lane >> 4);
        const int s = (lane & 15) ^ (m & 7);
        const int r = min(2 * m + (s >> 3), ntok - 1);
        boff[i] = (uint32_t)A.row_tok[p0 + r] * KD + (s & 7) * 16;
    }
    const __amdgpu_buffer_rsrc_t rg = dma_src(Wg), ru = dma_src(Wu), rb = dma_src(A.bq);
    auto issue_a = [&](int kt, int slot) {
        dma16<kNt>(rg, aoff + kt * 1024, &L.a[slot][wave * 1024]);
        dma16<kNt>(ru, aoff + kt * 1024, &L.a[slot][(RT + wave) * 1024]);
    };
    auto issue_b = [&](int kt, int slot) {
#pragma unroll
        for (int i = 0; i < NBI; i++) dma16(rb, boff[i] + kt * 128, &L.b[slot][(wave + W * i) * 1024]);
    };
    const uint32_t nib = (uint32_t)512 * KD / 2;
    dma16(rg, nib + ((uint32_t)(mt0 + wave) * 64 + lane) * 16, &L.sc[wave * 1024]);
    dma16(ru, nib + ((uint32_t)(mt0 + wave) * 64 + lane) * 16, &L.sc[(RT + wave) * 1024]);
    constexpr int NJ1 = NJ > 0 ? NJ : 1;
    u32x4 sb[NJ1];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int r = min(16 * (wt + 2 * j) + n, ntok - 1);
        sb[j] = *reinterpret_cast<const u32x4 *>(A.bs2 + (size_t)A.row_tok[p0 + r] * (KD / 32) + q * 16);
    }
    // step kt issues B(kt+1) then A(kt+3) after its barrier (A's slot kt+3
    // is the one step kt-1 read; three steps cover the HBM latency of the
    // weights, two did not: with A staged two steps ahead the kernel took
    // 88 us, 66 without A's loads at all); when step kt needs B(kt), only
    // A(kt+2) was issued after it
    issue_a(0, 0);
    issue_b(0, 0);
    issue_a(1, 1);
    issue_a(2, 2);

    v4f acc[4][NJ1];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[a][j] = v4f{0.f, 0.f, 0.f, 0.f};
    uint32_t sa[4];
    uint32_t sbg[NJ1];
    auto group = [&](int g, auto LASTC) {
        constexpr bool LAST = decltype(LASTC)::value;
#pragma unroll
        for (int j = 0; j < NJ; j++) sbg[j] = (g & 2) ? ((g & 1) ? sb[j][3] : sb[j][2]) : ((g & 1) ? sb[j][1] : sb[j][0]);
        static_for<0, 4>([&](auto S) {
            constexpr int st = decltype(S)::value;
            const int kt = 4 * g + st;
            // pin the previous step's MFMAs before the barrier: the compiler
            // would otherwise sink them to the end and keep every step's
            // fragments live at once
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int j = 0; j < NJ; j++) asm volatile("" : "+v"(acc[a][j]));
            // the last steps issue no A after their B: wait for everything
            if constexpr (LAST && st >= 2) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            else asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
            dma_barrier();
            // restage the slots read in the previous step (free: every wave
            // has passed this barrier) before this step's MFMAs
            if constexpr (!(LAST && st == 3)) issue_b(kt + 1, (st + 1) & 1);
            if constexpr (!(LAST && st >= 1)) issue_a(kt + 3, (st + 3) & 3);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (st == 0) {
#pragma unroll
                for (int a = 0; a < 4; a++) {
                    const int slot = (a < 2 ? 0 : RT) + 2 * wa + (a & 1);
                    sa[a] = *reinterpret_cast<const uint32_t *>(&L.sc[slot * 1024 + lane * 16 + 4 * g]);
                }
            }
            // A fragments first (4, held for the step), then column tile j's
            // B fragment is read while the MFMAs of tiles j-2 and j-1 run
            // (LDS latency under load is longer than one tile's 4 MFMAs)
            u32x4 af[4];
#pragma unroll
            for (int a = 0; a < 4; a++) {
                const int slot = (a < 2 ? 0 : RT) + 2 * wa + (a & 1);
                af[a] = *reinterpret_cast<const u32x4 *>(&L.a[st][slot * 1024 + lane * 16]);
            }
            auto read_b = [&](int j) {
                const int r = 16 * (wt + 2 * j) + n;
                const u32x4 b0 = *reinterpret_cast<const u32x4 *>(&L.b[st & 1][gd_boff(r, q)]);
                const u32x4 b1 = *reinterpret_cast<const u32x4 *>(&L.b[st & 1][gd_boff(r, 4 + q)]);
                return v8i{(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
            };
            v8i bq[NJ1 + 1];
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                if (j == 0) bq[0] = read_b(0);
                if (j == 0 && NJ > 1) bq[1] = read_b(1);
                if (j + 2 < NJ) bq[j + 2] = read_b(j + 2);
#pragma unroll
                for (int a = 0; a < 4; a++) {
                    const v8i av = v8i{(int)af[a][0], (int)af[a][1], (int)af[a][2], (int)af[a][3], 0, 0, 0, 0};
                    acc[a][j] = mfma_f4xf8<st, st>(av, bq[j], acc[a][j], (int)sa[a], (int)sbg[j]);
                }
            }
            if constexpr (NJ > 0) {
                __builtin_amdgcn_sched_group_barrier(0x100, 4 + 2 + (NJ > 1 ? 2 : 0) + (st == 0 ? 4 : 0), 0);
#pragma unroll
                for (int j = 0; j < NJ; j++) {
                    if (j + 2 < NJ) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
                }
            }
        });
    };
#pragma unroll 1
    for (int g = 0; g < NKT / 4 - 1; g++) group(g, std::false_type{});
    group(NKT / 4 - 1, std::true_type{});

    // SwiGLU of gate tile i and up tile i (i = 0, 1: one 32-row h block)
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int p = p0 + 16 * (wt + 2 * j) + n;
        float h[2][4];
#pragma unroll
        for (int r = 0; r < 2; r++)
#pragma unroll
            for (int i = 0; i < 4; i++) h[r][i] = silu(acc[r][j][i]) * acc[2 + r][j][i];
        store_h_block(A, hq8, p, p < p1, (mt0 + 2 * wa) * 16, q, lane, h);
    }
}
}  // namespace gdma

// ---------------------------------------------------------------------------
// shared expert gate/up with q8_0-split matrices (sorted path)
// ---------------------------------------------------------------------------
// The reference runs a split-Q8 shared expert through pf_gemm's int8 path
// (q36_engine.cu:3403-3406, :3464-3469): x quantised per 32 to int8 with an
// fp32 scale, int8 MMA per 32-block with both scales applied.  Workgroup =
// (256 tokens, a 32-row block of gate and the same 32 rows of up); wave w
// takes tokens 64w..64w+63 (4 column tiles) against the 4 row tiles over all
// of K = 2048, so each weight fragment loaded feeds 4 MFMAs (the weights,
// 2 MiB for gate + up, stay in L2).  Each block's integer result is scaled
// and added in fp32.  The epilogue is the routed kernels': SwiGLU and the
// int8 quantisation of h into the token's shared row.
constexpr int kShCt = 4;                 // column tiles per wave
constexpr int kShTok = 4 * 16 * kShCt;   // tokens per workgroup
constexpr int kShRb = 512 / 32;          // 32-row blocks of d_ff

// Operands of one K-pair (two 32-blocks) of the shared gate/up body.
struct ShKp {
    u32x4 af[4], sf[4];      // weight codes and f16 scales of the 4 row tiles
    uint2 bx[kShCt][2];      // x codes of the column tiles, both blocks
    float2 dh[kShCt];        // their fp32 scales
};

// Workgroup (token block tb, 32-row block rb) of the shared gate/up.
__device__ __forceinline__ void shared_gateup_q8_body(const GemmArgs &A, int tb, int rb) {
    constexpr int KD = 2048, NKP = KD / 64, NKB = KD / 32, MF = 512;
    const int tid = threadIdx.x, lane = tid & 63, q = lane >> 4, n = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t0 = tb * kShTok + wave * 16 * kShCt;   // this wave's first token
    const int mt0 = rb * 2;                            // first row tile of the 32-row block
    if (t0 >= A.T) return;                             // wave-uniform; no barrier follows
    const int8_t *xr[kShCt];
    const float *xs[kShCt];
#pragma unroll
    for (int j = 0; j < kShCt; j++) {
        // padding columns repeat the last token; never stored
        const int t = min(t0 + 16 * j + n, A.T - 1);
        xr[j] = A.xq8 + (size_t)t * KD;
        xs[j] = A.xsf + (size_t)t * NKB;
    }
    auto load = [&](int kp, ShKp &o) {
#pragma unroll
        for (int a = 0; a < 4; a++) {
            const uint8_t *W = a < 2 ? A.sa : A.sb;
            const int mt = mt0 + (a & 1);
            o.af[a] = *reinterpret_cast<const u32x4 *>(W + ((size_t)mt * NKP + kp) * 1024 + lane * 16);
            o.sf[a] = *reinterpret_cast<const u32x4 *>(W + (size_t)MF * KD + (((size_t)mt * 4 + q) * NKB + 2 * kp) * 8);
        }
        // x K 64kp + 8q..+7 (block 2kp) and 64kp + 32 + 8q..+7 (block 2kp+1)
#pragma unroll
        for (int j = 0; j < kShCt; j++) {
            o.bx[j][0] = *reinterpret_cast<const uint2 *>(xr[j] + 64 * kp + 8 * q);
            o.bx[j][1] = *reinterpret_cast<const uint2 *>(xr[j] + 64 * kp + 32 + 8 * q);
            o.dh[j] = *reinterpret_cast<const float2 *>(xs[j] + 2 * kp);
        }
    };
    v4f acc[4][kShCt];   // gate mt0, mt0+1, up mt0, mt0+1 x column tiles
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int j = 0; j < kShCt; j++) acc[a][j] = v4f{0.f, 0.f, 0.f, 0.f};
    ShKp cur, nxt;
    load(0, cur);
#pragma unroll 1
    for (int kp = 0; kp < NKP; kp++) {
        if (kp + 1 < NKP) load(kp + 1, nxt);   // in flight while this pair computes
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int a = 0; a < 4; a++) {
                const long av = (long)(((uint64_t)cur.af[a][2 * h + 1] << 32) | cur.af[a][2 * h]);
                const uint32_t s01 = cur.sf[a][2 * h], s23 = cur.sf[a][2 * h + 1];
                const float w[4] = {f16lo(s01), f16hi(s01), f16lo(s23), f16hi(s23)};
                float nw[4];
#pragma unroll
                for (int i = 0; i < 4; i++) nw[i] = -kQ8BiasF * w[i];
#pragma unroll
                for (int j = 0; j < kShCt; j++) {
                    const long b = (long)(((uint64_t)cur.bx[j][h].y << 32) | cur.bx[j][h].x);
                    const v4i ci = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, b, v4i{kQ8Bias, kQ8Bias, kQ8Bias, kQ8Bias}, 0, 0, 0);
                    const float dhh = h ? cur.dh[j].y : cur.dh[j].x;
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[a][j][i] = fmaf(q8_scaled(ci[i], w[i], nw[i]), dhh, acc[a][j][i]);
                }
            }
        cur = nxt;
    }
#pragma unroll
    for (int j = 0; j < kShCt; j++) {
        float h[2][4];
#pragma unroll
        for (int r = 0; r < 2; r++)
#pragma unroll
            for (int i = 0; i < 4; i++) h[r][i] = silu(acc[r][j][i]) * acc[2 + r][j][i];
        const int t = t0 + 16 * j + n;
        store_h_block(A, true, A.nrouted + t, t < A.T, mt0 * 16, q, lane, h);
    }
}

// Stand-alone launch (skinny-tile layers); fat-tile layers run the same
// body in k_gateup_dma's first workgroups, beside the routed tiles.
__global__ __launch_bounds__(256) void k_shared_gateup_q8(GemmArgs A) {
    shared_gateup_q8_body(A, blockIdx.x, blockIdx.y);
}

__global__ __launch_bounds__(256, 2) void k_gateup_dma(GemmArgs A) {
    __shared__ gdma::Lds L;
    constexpr int NRB = 512 / (16 * gdma::RT);
    // a q8_0-split shared expert's workgroups come first (a multiple of 8,
    // so the XCD of each routed workgroup is unchanged) and run beside the
    // routed tiles
    const int bid = (int)blockIdx.x - A.sh_wgs;
    if (bid < 0) {
        shared_gateup_q8_body(A, (int)blockIdx.x / kShRb, (int)blockIdx.x % kShRb);
        return;
    }
    // tiles in reverse list order: k_scatter lists the routed tiles in
    // ascending size and the shared expert's (full) tiles last, so the
    // largest start first and the smallest fill the tail.  The down kernel
    // walks the same order.  Reversing alone: mixed 236.3 -> 232.0 us; the
    // size order on top: prefill4096 206.8 -> 202.8, mixed 222.7 -> 221.0
    // (another box).
    const int xcd = bid & 7, jx = bid >> 3;
    const int ngrp = (*A.ntiles + 7) >> 3, grp = jx / NRB;
    if (grp >= ngrp) return;
    const int ti = 8 * (ngrp - 1 - grp) + xcd;
    const int mt0 = (jx % NRB) * gdma::RT;
    if (ti >= *A.ntiles) return;
    const int4 tile = A.tiles[ti];
    const int e = tile.x, p0 = tile.y, p1 = tile.z;
    if (e == A.E && A.shq8) return;      // k_shared_gateup_q8's rows
    const uint8_t *Wg = e < A.E ? A.wa + (size_t)e * A.wstride : A.sa;
    const uint8_t *Wu = e < A.E ? A.wb + (size_t)e * A.wstride : A.sb;
    const int ntt = (p1 - p0 + 15) >> 4;
    const int wt = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) >> 1;   // uniform: the switch below is a scalar branch
    const bool hq8 = A.hq8 && e < A.E;   // the shared expert's down stays MXFP4
    const int nj = ntt > wt ? (ntt - wt + 1) >> 1 : 0;
    switch (nj) {
        case 0: gdma::body<0>(A, L, Wg, Wu, mt0, p0, p1, hq8); break;
        case 1: gdma::body<1>(A, L, Wg, Wu, mt0, p0, p1, hq8); break;
        case 2: gdma::body<2>(A, L, Wg, Wu, mt0, p0, p1, hq8); break;
        case 3: gdma::body<3>(A, L, Wg, Wu, mt0, p0, p1, hq8); break;
        case 4: gdma::body<4>(A, L, Wg, Wu, mt0, p0, p1, hq8); break;
        default: gdma::body<5>(A, L, Wg, Wu, mt0, p0, p1, hq8); break;
    }
}

// ---------------------------------------------------------------------------
// router logits (the matvec in front of the MoE step)
// ---------------------------------------------------------------------------
// logits[t][r] = W[r] . x[t] for r < n_expert; row n_expert (when present)
// is the shared-expert gate, written to shg[t].  Two numerics, as the
// reference has two paths:
//   k_router_f32: fp32 products and sums, one wavefront per row (decode:
//     k_matvec_f32_row, q36_ops.cuh:331-342); the row stays in registers
//     while every token's dot product is formed.
//   k_router_f16: W and x rounded to fp16 (RNE), fp32 accumulation on
//     v_mfma_f32_16x16x32_f16 (prefill: pf_gemm's fp16 tensor-core path,
//     q36_engine.cu:3403-3414, 2365-2384).
constexpr int kRtD = 2048;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__global__ __launch_bounds__(64) void k_router_f32(const float *__restrict__ W, int n_expert,
                                                   const void *__restrict__ x, int x_fmt, int T,
                                                   float *__restrict__ logits, int ld,
                                                   float *__restrict__ shg) {
    const int r = blockIdx.x, lane = threadIdx.x;
    const float *w = W + (size_t)r * kRtD;
    float4 wv[8];
#pragma unroll
    for (int j = 0; j < 8; j++) wv[j] = *reinterpret_cast<const float4 *>(w + (j * 64 + lane) * 4);
    for (int t = 0; t < T; t++) {
        float xv[32];
        if (x_fmt == Q36MOE_FMT_F32) {
            const float *xt = static_cast<const float *>(x) + (size_t)t * kRtD;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float4 v = *reinterpret_cast<const float4 *>(xt + (j * 64 + lane) * 4);
                xv[4 * j] = v.x; xv[4 * j + 1] = v.y; xv[4 * j + 2] = v.z; xv[4 * j + 3] = v.w;
            }
        } else {
            const uint16_t *xt = static_cast<const uint16_t *>(x) + (size_t)t * kRtD;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const uint2 v = *reinterpret_cast<const uint2 *>(xt + (j * 64 + lane) * 4);
                xv[4 * j] = __uint_as_float(v.x << 16); xv[4 * j + 1] = __uint_as_float(v.x & 0xffff0000u);
                xv[4 * j + 2] = __uint_as_float(v.y << 16); xv[4 * j + 3] = __uint_as_float(v.y & 0xffff0000u);
            }
        }
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            acc = fmaf(wv[j].x, xv[4 * j], acc);
            acc = fmaf(wv[j].y, xv[4 * j + 1], acc);
            acc = fmaf(wv[j].z, xv[4 * j + 2], acc);
            acc = fmaf(wv[j].w, xv[4 * j + 3], acc);
        }
        acc = wave_sum(acc);
        if (lane == 0) {
            if (r < n_expert) logits[(size_t)t * ld + r] = acc;
            else shg[t] = acc;
        }
    }
}

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// 8 consecutive activations of token row `t` from K offset k, rounded to fp16
__device__ __forceinline__ f16x8 x8_f16(const void *x, int x_fmt, size_t off) {
    float v[8];
    load8(x, x_fmt, off, v);
    f16x8 h;
#pragma unroll
    for (int i = 0; i < 8; i++) h[i] = (_Float16)v[i];
    return h;
}

// workgroup = 64 router rows x 64 tokens; wave w owns tokens 16w..16w+15
// and all 4 row tiles.  v_mfma_f32_16x16x32_f16 operands: lane L holds row
// (A) or column (B) L%16 and K elements 8(L/16)..8(L/16)+7.
__global__ __launch_bounds__(256) void k_router_f16(const float *__restrict__ W, int n_rows, int n_expert,
                                                    const void *__restrict__ x, int x_fmt, int T,
                                                    float *__restrict__ logits, int ld,
                                                    float *__restrict__ shg) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), n = lane & 15, g = lane >> 4;
    const int r0 = blockIdx.x * 64, t0 = blockIdx.y * 64 + wave * 16;
    const int tok = min(t0 + n, T - 1);                  // padding columns repeat the last token
    int rows[4];
#pragma unroll
    for (int i = 0; i < 4; i++) rows[i] = min(r0 + 16 * i + n, n_rows - 1);
    v4f acc[4];
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = v4f{0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < kRtD; k0 += 32) {
        const f16x8 b = x8_f16(x, x_fmt, (size_t)tok * kRtD + k0 + 8 * g);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float *wr = W + (size_t)rows[i] * kRtD + k0 + 8 * g;
            const float4 w0 = *reinterpret_cast<const float4 *>(wr);
            const float4 w1 = *reinterpret_cast<const float4 *>(wr + 4);
            const f16x8 a = f16x8{(_Float16)w0.x, (_Float16)w0.y, (_Float16)w0.z, (_Float16)w0.w,
                                  (_Float16)w1.x, (_Float16)w1.y, (_Float16)w1.z, (_Float16)w1.w};
            acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[i], 0, 0, 0);
        }
    }
    // C: lane L holds rows 4(L/16)+j of token column L%16
    const int t = t0 + n;
    if (t >= T) return;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = r0 + 16 * i + 4 * g + j;
            if (r < n_expert) logits[(size_t)t * ld + r] = acc[i][j];
            else if (r < n_rows) shg[t] = acc[i][j];
        }
}

// ---------------------------------------------------------------------------
// the producer of the MoE input: residual add + RMSNorm + quantisation
// ---------------------------------------------------------------------------
// One token row per workgroup, 4 waves x 512 values, 8 per lane (the lane
// layout of quant8_lane, so each 32-block is quantised by 4 lanes of one
// wave straight from registers).  h += a is written back; the sum of
// squares is fp32 per lane, a wave butterfly, then the 4 wave sums in
// wave order; y = h * rsqrt(mean + eps) * w (k_add_rmsnorm,
// q36_engine.cu:696-706) goes to y and / or to e4m3 + E8M0.
__global__ __launch_bounds__(256) void k_add_rmsnorm_quant(float *__restrict__ h, const float *__restrict__ a,
                                                          const float *__restrict__ w, float eps,
                                                          float *__restrict__ y, uint8_t *__restrict__ xq,
                                                          uint8_t *__restrict__ xs) {
    __shared__ float part[4];
    const int t = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const size_t o = (size_t)t * kRtD + wave * 512 + lane * 8;
    const float4 h0 = *reinterpret_cast<const float4 *>(h + o), h1 = *reinterpret_cast<const float4 *>(h + o + 4);
    const float4 g0 = *reinterpret_cast<const float4 *>(w + wave * 512 + lane * 8);
    const float4 g1 = *reinterpret_cast<const float4 *>(w + wave * 512 + lane * 8 + 4);
    float v[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
    const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
    if (a) {
        const float4 a0 = *reinterpret_cast<const float4 *>(a + o), a1 = *reinterpret_cast<const float4 *>(a + o + 4);
        v[0] += a0.x; v[1] += a0.y; v[2] += a0.z; v[3] += a0.w;
        v[4] += a1.x; v[5] += a1.y; v[6] += a1.z; v[7] += a1.w;
        *reinterpret_cast<float4 *>(h + o) = make_float4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<float4 *>(h + o + 4) = make_float4(v[4], v[5], v[6], v[7]);
    }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) ss = fmaf(v[i], v[i], ss);
    ss = wave_sum(ss);
    if (lane == 0) part[wave] = ss;
    __syncthreads();
    const float r = rsqrtf((part[0] + part[1] + part[2] + part[3]) / (float)kRtD + eps);
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = v[i] * r * g[i];
    if (y) {
        *reinterpret_cast<float4 *>(y + o) = make_float4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<float4 *>(y + o + 4) = make_float4(v[4], v[5], v[6], v[7]);
    }
    if (xq) quant8_lane(v, lane, xq + o, xs + (size_t)t * (kRtD / 32) + wave * 16 + (lane >> 2));
}

// ---------------------------------------------------------------------------
// skinny gate/up: tiles of at most 32 rows (few rows per expert)
// ---------------------------------------------------------------------------
// With a handful of rows per expert the grouped GEMM is a weight stream.
// Every wave keeps its A (E2M1 fragments) in its own registers, loaded all at
// once straight from HBM, with no LDS staging of A; B rows (e4m3) come from
// L2 into registers.  Workgroup = (tile, 32-row block of gate and up); the 8
// waves split K into 8 x 256, partial sums meet in LDS in wave order, then
// SwiGLU and the per-32 quantisation of h (one block per row).  The down
// projection of skinny tiles runs in k_down_lds, as for fat tiles.
constexpr int kSkTok = 32;     // rows per skinny tile (two 16-row column tiles)
constexpr int kSkinnyRows = 8; // auto mode: skinny while T*k <= kSkinnyRows * n_expert
constexpr int kSxFusedRows = 16; // ... and to kSxFusedRows * n_expert on the one-kernel skinny path
constexpr int kSkW = 8;        // waves per workgroup

template <int NJ>
__device__ __forceinline__ void skinny_gateup(const GemmArgs &A, const uint8_t *Wg, const uint8_t *Wu,
                                              int mt0, int p0, int p1, float (*red)[4][64][4], bool hq8) {
    constexpr int KD = 2048, NKT = KD / 128;
    // the wave index is made wave-uniform for the compiler: the MFMA op_sel
    // below depends on it and must be chosen by scalar branches
    const int tid = threadIdx.x, lane = tid & 63, q = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const size_t nib = (size_t)512 * KD / 2;
    // this wave's K-steps: 2w and 2w+1 (one scale dword group, op_sel 2w%4 and +1)
    const int kt0 = 2 * wave, g = kt0 >> 2;
    u32x4 af[4][2];
    uint32_t sa[4];
#pragma unroll
    for (int a = 0; a < 4; a++) {
        const uint8_t *W = a < 2 ? Wg : Wu;
        const int mt = mt0 + (a & 1);
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++)
            af[a][s2] = *reinterpret_cast<const u32x4 *>(W + ((size_t)mt * NKT + kt0 + s2) * 1024 + lane * 16);
        sa[a] = *reinterpret_cast<const uint32_t *>(W + nib + ((size_t)mt * 64 + lane) * NKT + 4 * g);
    }
    u32x4 bf[NJ][2][2];
    uint32_t sb[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int p = p0 + j * 16 + (lane & 15);
        const int r = A.row_tok[p < p1 ? p : p0];
        const uint8_t *bp = A.bq + (size_t)r * KD + q * 16;
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++) {
            bf[j][s2][0] = *reinterpret_cast<const u32x4 *>(bp + (kt0 + s2) * 128);
            bf[j][s2][1] = *reinterpret_cast<const u32x4 *>(bp + (kt0 + s2) * 128 + 64);
        }
        sb[j] = *reinterpret_cast<const uint32_t *>(A.bs2 + (size_t)r * (KD / 32) + q * NKT + 4 * g);
    }
    v4f acc[4][NJ];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[a][j] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s2 = 0; s2 < 2; s2++)
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const u32x4 b0 = bf[j][s2][0], b1 = bf[j][s2][1];
            const v8i bv = v8i{(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
#pragma unroll
            for (int a = 0; a < 4; a++) {
                const u32x4 f = af[a][s2];
                const v8i av = v8i{(int)f[0], (int)f[1], (int)f[2], (int)f[3], 0, 0, 0, 0};
                acc[a][j] = mfma_sel((kt0 + s2) & 3, av, bv, acc[a][j], (int)sa[a], (int)sb[j]);
            }
        }
    // column tiles one at a time through one 32 KiB LDS slab (more
    // workgroups per CU than a slab per column tile would allow)
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        if (j > 0) __syncthreads();      // wave 0 has read column tile j-1
#pragma unroll
        for (int a = 0; a < 4; a++) *reinterpret_cast<v4f *>(&red[wave][a][lane][0]) = acc[a][j];
        __syncthreads();
        if (wave != 0) continue;
        // wave 0 finishes column tile j: sums over the 8 K-slices in wave order
        const int p = p0 + j * 16 + (lane & 15);
        float h[2][4];
#pragma unroll
        for (int r = 0; r < 2; r++) {
            v4f gs = *reinterpret_cast<const v4f *>(&red[0][r][lane][0]);
            v4f us = *reinterpret_cast<const v4f *>(&red[0][2 + r][lane][0]);
#pragma unroll
            for (int w = 1; w < kSkW; w++) {
                gs += *reinterpret_cast<const v4f *>(&red[w][r][lane][0]);
                us += *reinterpret_cast<const v4f *>(&red[w][2 + r][lane][0]);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) h[r][i] = silu(gs[i]) * us[i];
        }
        store_h_block(A, hq8, p, p < p1, mt0 * 16, q, lane, h);
    }
}

// XCD-major order: the 16 row blocks of one tile run back to back on one XCD.
__global__ __launch_bounds__(64 * kSkW) void k_skinny_gateup(GemmArgs A) {
    constexpr int NRB = 16;
    __shared__ __align__(16) float red[kSkW][4][64][4];
    const int xcd = blockIdx.x & 7, jx = blockIdx.x >> 3;
    const int ti = 8 * (jx / NRB) + xcd, rb = jx % NRB;
    if (ti >= *A.ntiles) return;
    const int4 tile = A.tiles[ti];
    const int e = tile.x, p0 = tile.y, p1 = tile.z;
    const int nj = (p1 - p0 + 15) >> 4;
    const uint8_t *Wg = e < A.E ? A.wa + (size_t)e * A.wstride : A.sa;
    const uint8_t *Wu = e < A.E ? A.wb + (size_t)e * A.wstride : A.sb;
    if (e == A.E && A.shq8) return;      // k_shared_gateup_q8's rows
    const bool hq8 = A.hq8 && e < A.E;   // shared rows: an MXFP4 down
    if (nj <= 1) skinny_gateup<1>(A, Wg, Wu, rb * 2, p0, p1, red, hq8);
    else skinny_gateup<2>(A, Wg, Wu, rb * 2, p0, p1, red, hq8);
}

// ---------------------------------------------------------------------------
// down projection for fat tiles: B (h rows) staged once in LDS, A in registers
// ---------------------------------------------------------------------------
// K = d_ff = 512 is short, so the whole B operand of up to 128 rows fits in
// LDS (128 x 512 B) and every wave keeps its A -- 4 row tiles x all of K --
// in registers for the workgroup's lifetime.  One barrier after staging;
// then each wave walks the 16-row column tiles, reading each B fragment once
// for 4 MFMAs, and stores the finished column tile (x routing weight) before
// the next: no accumulator outlives its column tile.
//   workgroup = (tile, 256 output rows), 4 waves of 4 row tiles each; tiles
//   longer than 128 rows are staged in chunks of 128.
constexpr int kDlW = 4;                  // waves
constexpr int kDlRT = 4;                 // row tiles per wave
constexpr int kDlRows = 128;             // B rows staged per chunk

// Staging of a weighted down row: f16 with a power-of-two scale per 16
// columns.  The 16 columns of group g of row p are held by lanes q = 0..3 of
// one MFMA column, 4 each; their maximum |v| has the biased fp32 exponent eb
// (clamped to [15, 254]; 255 keeps inf / NaN), the group is stored as
// v * 2^(141 - eb) (exact: a power of two), every value of which is below
// 2^15 < 65504, rounded to f16 (RNE, relative error <= 2^-11), with eb in
// dne; the combine multiplies back by 2^(eb - 141).  Half the bytes of an
// f32 staging (which the reference uses, q36_engine.cu:3451-3463) for a
// rounding of 2^-11 of each staged value.
__device__ __forceinline__ void store_dn16(const GemmArgs &A, int p, int g, int q, bool valid, float v0, float v1,
                                           float v2, float v3) {
    float a = fmaxf(fmaxf(fabsf(v0), fabsf(v1)), fmaxf(fabsf(v2), fabsf(v3)));
    a = max_rows4(a);
    uint32_t eb = (__float_as_uint(a) >> 23) & 0xffu;
    eb = eb == 255u ? 255u : eb < 15u ? 15u : eb > 254u ? 254u : eb;
    const float mul = __uint_as_float((268u - eb) << 23);
    if (valid) {
        const uint32_t lo = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(v0 * mul)) |
                            ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(v1 * mul)) << 16);
        const uint32_t hi = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(v2 * mul)) |
                            ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(v3 * mul)) << 16);
        *reinterpret_cast<uint2 *>(A.dnh + (size_t)p * A.ldo + g * 16 + 4 * q) = make_uint2(lo, hi);
        if (q == 0) A.dne[(size_t)p * (A.ldo / 16) + g] = (uint8_t)eb;
    }
}

// store_dn16 for the 4 row tiles mt0 .. mt0+3 (64 columns) of one MFMA
// column tile at once: one maximum and one exponent for all 64 (written to
// each of the 4 groups' exponent bytes), and the routing weight w folded into
// the scale multiply.  f16 holds every value within 2^-29 of the group
// maximum at full relative precision, so the wider group rounds the same.
__device__ __forceinline__ void store_dn16x4(const GemmArgs &A, int p, int mt0, int q, bool valid, const v4f (&c)[4],
                                             float w) {
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++)
        a = fmaxf(a, fmaxf(fmaxf(fabsf(c[i][0]), fabsf(c[i][1])), fmaxf(fabsf(c[i][2]), fabsf(c[i][3]))));
    a = max_rows4(a);
    a *= fabsf(w);
    uint32_t eb = (__float_as_uint(a) >> 23) & 0xffu;
    eb = eb == 255u ? 255u : eb < 15u ? 15u : eb > 254u ? 254u : eb;
    const float wm = w * __uint_as_float((268u - eb) << 23);
    if (valid) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t lo = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(c[i][0] * wm)) |
                                ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(c[i][1] * wm)) << 16);
            const uint32_t hi = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(c[i][2] * wm)) |
                                ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(c[i][3] * wm)) << 16);
            *reinterpret_cast<uint2 *>(A.dnh + (size_t)p * A.ldo + (mt0 + i) * 16 + 4 * q) = make_uint2(lo, hi);
        }
        if (q == 0) *reinterpret_cast<uint32_t *>(A.dne + (size_t)p * (A.ldo / 16) + mt0) = eb * 0x01010101u;
    }
}

// byte offset of (row r, 16-byte chunk c) of a staged h row: rows of 512 B,
// chunk index XORed (low 4 bits) with the row, so the 16 rows of a fragment
// read fall in 16 distinct bank groups
__device__ __forceinline__ int dl_boff(int r, int c) { return r * 512 + ((c & 16) | ((c ^ r) & 15)) * 16; }

// Stage h rows c0 .. c0+nr (sorted order, 512 B each) into sb with
// direct-to-LDS loads, all in flight at once: wave w loads row pairs w + 4u
// (1 KiB each, lane-contiguous in LDS, chunk order of dl_boff).
__device__ __forceinline__ void stage_h_rows(const uint8_t *bq, int c0, int nr, uint8_t *sb) {
    constexpr int KD = 512;
    const int lane = threadIdx.x & 63;
    const int npair = __builtin_amdgcn_readfirstlane((nr + 1) >> 1);
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const __amdgpu_buffer_rsrc_t rq = dma_src(bq);
#pragma unroll
    for (int u = 0; u < kDlRows / 2 / kDlW; u++) {
        const int pr = wv + kDlW * u;
        if (pr < npair) {
            const int r = 2 * pr + (lane >> 5), ph = lane & 31;
            const int c = (ph & 16) | ((ph ^ r) & 15);       // logical chunk in this slot
            dma16(rq, (uint32_t)(c0 + min(r, nr - 1)) * KD + c * 16, &sb[pr * 1024]);
        }
    }
}

// Row stride of the staged fp32 h scales: 20 floats, so the 16 rows of a
// fragment read (16 B each) start in 16 distinct bank groups.
constexpr int kDlSfStride = 20;

// Down projection of one routed tile whose expert is in the q8_0-split
// layout (k_gemm_expert_i8, q36_engine.cu:2526-2618): int8 h rows with fp32
// scales against int8 weights with f16 scales.  Each 32-block is one
// v_mfma_i32_16x16x32_i8 whose exact integer result is scaled by the
// weight row's f16 scale times the h row's fp32 scale and accumulated in
// fp32 (two fmas per output and block, q8_scaled).  The wave's 4 row tiles
// run as 4 passes over the staged B (codes and fp32 scales of one row tile
// are 160 VGPRs); B is staged once per chunk, as in the MXFP4 body.  Each
// pass is software-pipelined by one block: a block's scaling overlaps the
// next block's MFMA.
__device__ __forceinline__ void down_q8_tile(const GemmArgs &A, const uint8_t *W, int p0, int p1, int rb, uint8_t *sb,
                                             float (*ssf)[kDlSfStride], float *ws) {
    constexpr int KD = 512, NKP = KD / 64, NKB = KD / 32;
    const int tid = threadIdx.x, lane = tid & 63, q = lane >> 4, n = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint8_t *Wsc = W + (size_t)2048 * KD;   // f16 scales after the codes
    const int mt0 = (rb * kDlW + wave) * kDlRT;
    for (int c0 = p0; c0 < p1; c0 += kDlRows) {
        const int nr = min(kDlRows, p1 - c0);
        if (c0 != p0) __syncthreads();   // previous chunk fully read
        stage_h_rows(A.bq, c0, nr, sb);
        for (int c = tid; c < nr; c += 64 * kDlW) {
            const float4 *src = reinterpret_cast<const float4 *>(A.bsf + (size_t)(c0 + c) * NKB);
#pragma unroll
            for (int u = 0; u < 4; u++) *reinterpret_cast<float4 *>(&ssf[c][4 * u]) = src[u];
            ws[c] = A.row_w[c0 + c];
        }
        __syncthreads();
        const int ntt = (nr + 15) >> 4;
#pragma unroll 1
        for (int ps = 0; ps < kDlRT; ps++) {
            const int mt = mt0 + ps;
            u32x4 ac[NKP];
            float dw[NKB][4];   // f16 scales of rows 4q..4q+3, widened once per pass
            float ndw[NKB][4];  // -12582912 * dw (exact)
#pragma unroll
            for (int kp = 0; kp < NKP; kp++) {
                ac[kp] = *reinterpret_cast<const u32x4 *>(W + ((size_t)mt * NKP + kp) * 1024 + lane * 16);
                const u32x4 sv = *reinterpret_cast<const u32x4 *>(Wsc + (((size_t)mt * 4 + q) * NKB + 2 * kp) * 8);
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    dw[2 * kp + h][0] = f16lo(sv[2 * h]);
                    dw[2 * kp + h][1] = f16hi(sv[2 * h]);
                    dw[2 * kp + h][2] = f16lo(sv[2 * h + 1]);
                    dw[2 * kp + h][3] = f16hi(sv[2 * h + 1]);
#pragma unroll
                    for (int i = 0; i < 4; i++) ndw[2 * kp + h][i] = -kQ8BiasF * dw[2 * kp + h][i];
                }
            }
            for (int j = 0; j < ntt; j++) {
                // padding columns read row 0 of the chunk; never stored
                const int r = j * 16 + n < nr ? j * 16 + n : 0;
                float dh[NKB];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const float4 v = *reinterpret_cast<const float4 *>(&ssf[r][4 * u]);
                    dh[4 * u] = v.x; dh[4 * u + 1] = v.y; dh[4 * u + 2] = v.z; dh[4 * u + 3] = v.w;
                }
                // all 16 B fragments read up front (one LDS latency per column
                // tile): lane (column n, group q) holds h K 32kb + 8q..+7 =
                // half q&1 of chunk 2kb + q/2
                uint2 bv[NKB];
#pragma unroll
                for (int kb = 0; kb < NKB; kb++)
                    bv[kb] = *reinterpret_cast<const uint2 *>(&sb[dl_boff(r, 2 * kb + (q >> 1)) + (q & 1) * 8]);
                v4f acc = {0.f, 0.f, 0.f, 0.f};
                v4i prev;
#pragma unroll
                for (int kb = 0; kb < NKB; kb++) {
                    const long b = (long)(((uint64_t)bv[kb].y << 32) | bv[kb].x);
                    const u32x4 f = ac[kb >> 1];
                    const long a = (kb & 1) ? (long)(((uint64_t)f[3] << 32) | f[2]) : (long)(((uint64_t)f[1] << 32) | f[0]);
                    const v4i ci = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, v4i{kQ8Bias, kQ8Bias, kQ8Bias, kQ8Bias}, 0, 0, 0);
                    if (kb > 0) {   // the previous block, while this one's MFMA runs
#pragma unroll
                        for (int i = 0; i < 4; i++)
                            acc[i] = fmaf(q8_scaled(prev[i], dw[kb - 1][i], ndw[kb - 1][i]), dh[kb - 1], acc[i]);
                    }
                    prev = ci;
                    // one block per scheduling group: left alone, the compiler
                    // issues every block's MFMA first and holds all the results
                    asm volatile("" : "+v"(acc));
                    __builtin_amdgcn_sched_barrier(0);
                }
#pragma unroll
                for (int i = 0; i < 4; i++)
                    acc[i] = fmaf(q8_scaled(prev[i], dw[NKB - 1][i], ndw[NKB - 1][i]), dh[NKB - 1], acc[i]);
                {
                    const float w = ws[r];
                    store_dn16(A, c0 + j * 16 + n, mt, q, j * 16 + n < nr, acc[0] * w, acc[1] * w, acc[2] * w,
                               acc[3] * w);
                }
            }
        }
    }
}

// Q8: tiles whose down matrix is q8_0-split (routed: hq8, shared: shq8)
// take down_q8_tile; the others, and every tile of an MXFP4 layer, the
// body below.
template <bool Q8>
__global__ __launch_bounds__(64 * kDlW, Q8 ? 2 : 1) void k_down_lds(GemmArgs A) {
    constexpr int KD = 512, NKT = KD / 128, NRB = 2048 / (16 * kDlRT * kDlW);
    __shared__ __align__(16) uint8_t sb[kDlRows * 512];
    __shared__ uint32_t ss[kDlRows][4];       // B scale dwords: [row][lane group]
    __shared__ float ws[kDlRows];             // routing weight of each row
    __shared__ __align__(16) float ssf[Q8 ? kDlRows : 1][kDlSfStride];   // int8 h scales
    const int xcd = blockIdx.x & 7, jx = blockIdx.x >> 3;
    // tiles in reverse list order, as in k_gateup_dma
    const int ngrp = (*A.ntiles + 7) >> 3, grp = jx / NRB;
    if (grp >= ngrp) return;
    const int ti = 8 * (ngrp - 1 - grp) + xcd, rb = jx % NRB;
    if (ti >= *A.ntiles) return;
    const int4 tile = A.tiles[ti];
    const int e = __builtin_amdgcn_readfirstlane(tile.x), p0 = tile.y, p1 = tile.z;
    if constexpr (Q8) {
        if (e < A.E ? A.hq8 : A.shq8) {
            down_q8_tile(A, e < A.E ? A.wa + (size_t)e * A.wstride : A.sa, p0, p1, rb, sb, ssf, ws);
            return;
        }
    }
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), q = lane >> 4, n = lane & 15;
    const uint8_t *W = e < A.E ? A.wa + (size_t)e * A.wstride : A.sa;
    const size_t nib = (size_t)2048 * KD / 2;
    // this wave's A: row tiles mt0 + i, all 4 K-steps
    const int mt0 = (rb * kDlW + wave) * kDlRT;
    u32x4 af[kDlRT][NKT];
    uint32_t sa[kDlRT];
#pragma unroll
    for (int i = 0; i < kDlRT; i++) {
#pragma unroll
        for (int kt = 0; kt < NKT; kt++)
            af[i][kt] = ldg_nt16(W + ((size_t)(mt0 + i) * NKT + kt) * 1024 + lane * 16);
        sa[i] = *reinterpret_cast<const uint32_t *>(W + nib + ((size_t)(mt0 + i) * 64 + lane) * NKT);
    }
    for (int c0 = p0; c0 < p1; c0 += kDlRows) {
        const int nr = min(kDlRows, p1 - c0);
        if (c0 != p0) __syncthreads();   // previous chunk fully read
        // stage rows c0 .. c0+nr of h (contiguous in sorted order), then
        // their lane-group-major scale dwords and routing weights
        stage_h_rows(A.bq, c0, nr, sb);
        for (int c = tid; c < nr; c += 64 * kDlW) {
            *reinterpret_cast<u32x4 *>(&ss[c][0]) = *reinterpret_cast<const u32x4 *>(A.bs2 + (size_t)(c0 + c) * 16);
            ws[c] = A.row_w[c0 + c];
        }
        __syncthreads();
        const int ntt = (nr + 15) >> 4;
        for (int j = 0; j < ntt; j++) {
            // padding columns read row 0 of the chunk; never stored
            const int r = j * 16 + n < nr ? j * 16 + n : 0;
            v8i bv[NKT];
#pragma unroll
            for (int kt = 0; kt < NKT; kt++) {
                const u32x4 b0 = *reinterpret_cast<const u32x4 *>(&sb[dl_boff(r, 8 * kt + q)]);
                const u32x4 b1 = *reinterpret_cast<const u32x4 *>(&sb[dl_boff(r, 8 * kt + 4 + q)]);
                bv[kt] = v8i{(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
            }
            const uint32_t sbw = ss[r][q];
            v4f acc[kDlRT];
#pragma unroll
            for (int i = 0; i < kDlRT; i++) acc[i] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kt = 0; kt < NKT; kt++)
#pragma unroll
                for (int i = 0; i < kDlRT; i++) {
                    const u32x4 f = af[i][kt];
                    const v8i av = v8i{(int)f[0], (int)f[1], (int)f[2], (int)f[3], 0, 0, 0, 0};
                    acc[i] = mfma_sel(kt, av, bv[kt], acc[i], (int)sa[i], (int)sbw);
                }
            store_dn16x4(A, c0 + j * 16 + n, mt0, q, j * 16 + n < nr, acc, ws[r]);
        }
    }
}

// ---------------------------------------------------------------------------
// skinny tiles: the whole expert in one workgroup
// ---------------------------------------------------------------------------
// Workgroup = one skinny tile (expert e, sorted rows p0..p1: at most 16 when
// the kernel finds its tiles itself, 32 from k_scatter):
// gate/up over all 512 rows of gate and up, SwiGLU and the e4m3
// quantisation of h into LDS, then the down projection over all 2048 output
// rows, staged weighted exactly as k_down_lds stages them.  h makes no round
// trip through HBM between two launches, and one expert's down weights
// stream while other workgroups are still in their gate/up.
//   8 waves; wave w owns gate and up row tiles 4w..4w+3 (h rows 64w..64w+63,
//   two quantisation blocks, one after the other) and down row tiles
//   16w..16w+15.  Each step loads 8 KiB per wave, contiguous in the packed
//   layout, two steps ahead into three register buffers: 16 gate/up steps
//   (8 per h block), then 8 down steps, all unrolled.  With one workgroup
//   per CU a CU keeps ~128 KiB in flight; loads into VGPRs held HBM near
//   its read rate from 150 CUs, where direct-to-LDS staging topped out near
//   28 GB/s per CU.  The kernel is bound by the weight stream (without its
//   MFMAs it takes as long), and the stream by the length of the runs it
//   reads: RT row tiles x 8/RT K-steps per step measured 51 / 53 / 60 us at
//   decode32 for RT = 1 / 2 / 4 (8 / 4 / 2 KiB runs); 16 KiB steps (one
//   whole row tile) 51.6.  RT = 1 is used, although each B fragment read
//   from LDS then feeds only NJ MFMAs.  An expert with a single tile loads
//   its weights non-temporal (NT).  The kernel serves up to 512 tokens at
//   256 experts, where its tiles still fit one workgroup per CU.
//   x rows of the tile sit in LDS (2 KiB each, 16-byte chunk index XORed in
//   its low 4 bits with the row, so a fragment read's 16 rows hit 16 bank
//   groups); h rows in the dl_boff layout of k_down_lds.
constexpr int kSxW = 8;
constexpr int kSxRT = 1;   // row tiles per gate/up step
constexpr int kBufFlags = 0x00020000;   // buffer resource word 3 (raw, 32-bit data format)
struct SxLds {
    __align__(16) uint8_t x[kSkTok * 2048];
    __align__(16) uint8_t h[kSkTok * 512];
    uint32_t hs[kSkTok][4];   // h scale dwords by lane group (lane-group-major order)
    float ws[kSkTok];         // routing weight of each row
    int tok[kSkTok];          // token of each row (rows past the tile repeat its last)
    int ent[kSkTok];          // staging row of each row's down output (see dn_store)
    // tile discovery: per-expert counts, their exclusive prefixes, tiles per
    // expert and theirs, per-wave counts, the tile found
    int cnt[kMaxExperts], off[kMaxExperts + 1], ntl[kMaxExperts], toff[kMaxExperts + 1];
    int wsum[kSxW];
    int sel;
};

// Tile discovery for k_skinny_expert (in place of k_scatter): every
// workgroup counts the routed entries per expert from the top-k indices,
// scans the counts into offsets and tiles of tn rows, finds its own tile and
// gathers that tile's entries in entry order -- the stable sorted order of
// k_scatter, so perm / pos / e_off come out identical.  At most
// kSxDiscoverMax routed entries (kSxEnt per thread).
constexpr int kSxEnt = 8;
constexpr int kSxDiscoverMax = kSxEnt * 64 * kSxW;
constexpr int kSxTok = 16;   // rows per discovered tile while T*k <= 4 * E; kSkTok above
struct SxArgs {
    const int32_t *idx; const float *wt;   // top-k routing of each entry
    const float *shg; int ld_shg;          // shared-gate logits (shared tiles), or null
    int32_t *perm, *pos, *e_off;           // sorted order out (taps; pos feeds the combine)
    int T, k, E;
    int discover;                          // 0: tiles from k_scatter
    int tn;                                // rows per discovered tile (<= kSkTok)
};

__device__ __forceinline__ int sx_off(int r, int c) { return r * 2048 + ((c & ~15) | ((c ^ r) & 15)) * 16; }

template <int NJ, int RT, bool NT, class Prep>
__device__ __forceinline__ void skinny_expert(const GemmArgs &G, const GemmArgs &Dn, int e, int p0, int p1,
                                              SxLds &L, Prep &&prep) {
    // RT row tiles per gate/up step, 8 / RT consecutive K-steps of each
    static_assert(RT == 1 || RT == 2 || RT == 4, "row tiles per step");
    constexpr int RD = RT == 4 ? 4 : 2;   // down row tiles per step (K = 4 K-steps)
    constexpr int KG = 2048, NKG = KG / 128, KD = 512, NKD = KD / 128;
    constexpr int NSG = 16, NSD = 8;   // gate/up and down steps
    const int tid = threadIdx.x, lane = tid & 63, q = lane >> 4, n = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nr = p1 - p0;
    const uint8_t *Wg = e < G.E ? G.wa + (size_t)e * G.wstride : G.sa;
    const uint8_t *Wu = e < G.E ? G.wb + (size_t)e * G.wstride : G.sb;
    const uint8_t *Wd = e < Dn.E ? Dn.wa + (size_t)e * Dn.wstride : Dn.sa;
    const int nibg = 512 * KG / 2, nibd = 2048 * KD / 2;
    const uint32_t lo16 = (uint32_t)lane * 16;
    // Buffer loads: one offset VGPR (the lane's) for every load, the
    // fragment's offset in an SGPR; with plain pointers the compiler keeps a
    // 64-bit address per fragment live across the unrolled steps.
    const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc((void *)Wg, (short)0, (int)G.wstride, kBufFlags);
    const __amdgpu_buffer_rsrc_t ru = __builtin_amdgcn_make_buffer_rsrc((void *)Wu, (short)0, (int)G.wstride, kBufFlags);
    const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc((void *)Wd, (short)0, (int)Dn.wstride, kBufFlags);
    // A step's operands: 8 weight fragments -- RT row tiles x 8/RT
    // consecutive K-steps (contiguous in the packed layout) -- and the row
    // tiles' scale dwords (byte kt & 3 of dword kt >> 2 in gate/up, byte kd
    // in down).  Gate/up: h block s >> 3, its row tiles a = 0..3 (gate rr0,
    // up rr0, gate rr1, up rr1; rr = row tile within the block) in groups of
    // RT, each group over the 16 K-steps.  Down: pass d >> 1 over row
    // tiles 16w + 4 pass .. +3 in two steps (RD row tiles, 8/RD K-steps).
    struct Step { u32x4 f[8]; uint32_t sc[4]; };
    auto load = [&](auto S, Step &b) {
        constexpr int st = decltype(S)::value;
        if constexpr (st < NSG) {
            constexpr int blk = st >> 3, m = st & 7, KS = 8 / RT;
            constexpr int a0 = (m / (16 / KS)) * RT, kt0 = (m % (16 / KS)) * KS;
#pragma unroll
            for (int ai = 0; ai < RT; ai++) {
                const int a = a0 + ai;
                const __amdgpu_buffer_rsrc_t r = (a & 1) ? ru : rg;
                const int mt = 4 * wave + 2 * blk + (a >> 1);
#pragma unroll
                for (int k = 0; k < KS; k++)
                    b.f[KS * ai + k] = __builtin_amdgcn_raw_buffer_load_b128(r, lo16, (mt * NKG + kt0 + k) * 1024, NT ? kNt : 0);
                if constexpr (KS <= 4)
                    b.sc[ai] = __builtin_amdgcn_raw_buffer_load_b32(r, lo16, nibg + mt * 1024 + 4 * (kt0 >> 2), 0);
                else {
                    b.sc[2 * ai] = __builtin_amdgcn_raw_buffer_load_b32(r, lo16, nibg + mt * 1024 + 4 * (kt0 >> 2), 0);
                    b.sc[2 * ai + 1] = __builtin_amdgcn_raw_buffer_load_b32(r, lo16, nibg + mt * 1024 + 4 * (kt0 >> 2) + 4, 0);
                }
            }
        } else {
            constexpr int d = st - NSG, KS = 8 / RD, ps = d >> 1, g = d & 1;
#pragma unroll
            for (int ai = 0; ai < RD; ai++) {
                const int mt = 16 * wave + 4 * ps + (RD == 4 ? ai : 2 * g + ai);
#pragma unroll
                for (int k = 0; k < KS; k++)
                    b.f[KS * ai + k] = __builtin_amdgcn_raw_buffer_load_b128(
                        rd, lo16, (mt * NKD + (RD == 4 ? 2 * g : 0) + k) * 1024, NT ? kNt : 0);
                b.sc[ai] = __builtin_amdgcn_raw_buffer_load_b32(rd, (uint32_t)lane * 4, nibd + mt * 256, 0);
            }
        }
    };
    // Prologue, in this order (sched barriers keep it): weight step 0; the
    // tile's rows (prep); the x rows of the tile (L.tok: rows past the tile
    // repeat its last row, never stored) and their B scales; weight step 1.  Waiting for the x
    // rows (loads complete in order) then leaves step 1 in flight.
    Step bs[3];   // three step buffers, loads two steps ahead of the MFMAs
    load(std::integral_constant<int, 0>{}, bs[0]);
    __builtin_amdgcn_sched_barrier(0);
    prep();   // the tile's rows into L.tok / L.ws, while step 0 is in flight
    __builtin_amdgcn_sched_barrier(0);
    const int xr_r = tid >> 4, xr_c = tid & 15;
    u32x4 xv[8];
    {
        const int tok = L.tok[xr_r];
        const uint8_t *xr = G.bq + (size_t)tok * KG;
#pragma unroll
        for (int u = 0; u < 8; u++) xv[u] = *reinterpret_cast<const u32x4 *>(xr + (xr_c + 16 * u) * 16);
    }
    u32x4 sb[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int tok = L.tok[16 * j + n];
        sb[j] = *reinterpret_cast<const u32x4 *>(G.bs2 + (size_t)tok * (KG / 32) + q * 16);
    }
    __builtin_amdgcn_sched_barrier(0);
    load(std::integral_constant<int, 1>{}, bs[1]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 8; u++) *reinterpret_cast<u32x4 *>(&L.x[sx_off(xr_r, xr_c + 16 * u)]) = xv[u];
    lds_barrier();

    v4f acc[4][NJ];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[a][j] = v4f{0.f, 0.f, 0.f, 0.f};
    // LDS byte offsets of this lane's B fragment halves (hh = 0: K 16q..,
    // hh = 1: K 64+16q..) for K-steps of parity par, column tile 0: the
    // swizzled chunk's low 4 bits depend only on (par, hh, q) ^ n, so K-step
    // kt adds (kt >> 1) * 256 and column tile j adds j rows (immediates)
    int xo[2][2], ho[2][2];
#pragma unroll
    for (int par = 0; par < 2; par++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            const int lo = ((8 * par + 4 * hh + q) ^ n) & 15;
            xo[par][hh] = n * 2048 + lo * 16;   // = sx_off(n, 8 * par + 4 * hh + q)
            ho[par][hh] = n * 512 + lo * 16;    // = dl_boff(n, 8 * par + 4 * hh + q)
        }
    // B fragment of K-step kt (x) or kd (h) for column tile j
    auto xfrag = [&](int kt, int j) {
        const int o = j * 16 * 2048 + (kt >> 1) * 256;
        const u32x4 b0 = *reinterpret_cast<const u32x4 *>(&L.x[xo[kt & 1][0] + o]);
        const u32x4 b1 = *reinterpret_cast<const u32x4 *>(&L.x[xo[kt & 1][1] + o]);
        return v8i{(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
    };
    auto hfrag = [&](int kd, int j) {
        const int o = j * 16 * 512 + (kd >> 1) * 256;
        const u32x4 b0 = *reinterpret_cast<const u32x4 *>(&L.h[ho[kd & 1][0] + o]);
        const u32x4 b1 = *reinterpret_cast<const u32x4 *>(&L.h[ho[kd & 1][1] + o]);
        return v8i{(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
    };
    // per K-step of the step: its B fragment (read once) against the RT row
    // tiles
    auto gu_step = [&](auto S, const Step &b) {
        constexpr int st = decltype(S)::value, m = st & 7, KS = 8 / RT;
        constexpr int a0 = (m / (16 / KS)) * RT, kt0 = (m % (16 / KS)) * KS;
        static_for<0, KS>([&](auto K) {
            constexpr int k = decltype(K)::value, kt = kt0 + k, sel = kt & 3;
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const v8i bv = xfrag(kt, j);
#pragma unroll
                for (int ai = 0; ai < RT; ai++) {
                    const u32x4 fr = b.f[KS * ai + k];
                    const v8i av = v8i{(int)fr[0], (int)fr[1], (int)fr[2], (int)fr[3], 0, 0, 0, 0};
                    const int sa = KS <= 4 ? (int)b.sc[ai] : (int)b.sc[2 * ai + (k >> 2)];
                    acc[a0 + ai][j] = mfma_f4xf8<sel, sel>(av, bv, acc[a0 + ai][j], sa, (int)sb[j][kt >> 2]);
                }
            }
        });
    };
    uint32_t hsv[NJ];   // h scale dword of this lane's column in each column tile
    auto dn_step = [&](auto S, const Step &b) {
        constexpr int d = decltype(S)::value - NSG, KS = 8 / RD, g = d & 1;
        constexpr int a0 = RD == 4 ? 0 : 2 * g, kd0 = RD == 4 ? 2 * g : 0;
        static_for<0, KS>([&](auto K) {
            constexpr int k = decltype(K)::value, kd = kd0 + k;
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const v8i bv = hfrag(kd, j);
#pragma unroll
                for (int ai = 0; ai < RD; ai++) {
                    const u32x4 fr = b.f[KS * ai + k];
                    const v8i av = v8i{(int)fr[0], (int)fr[1], (int)fr[2], (int)fr[3], 0, 0, 0, 0};
                    acc[a0 + ai][j] = mfma_f4xf8<kd, kd>(av, bv, acc[a0 + ai][j], (int)b.sc[ai], (int)hsv[j]);
                }
            }
        });
    };
    // SwiGLU of h block 2w+blk: gate row tiles 4w+2blk+rr in acc[2rr], up in
    // acc[2rr+1]
    auto swiglu = [&](int blk) {
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int r = 16 * j + n, p = p0 + r;
            const bool valid = r < nr;
            float h[2][4];
#pragma unroll
            for (int rr = 0; rr < 2; rr++)
#pragma unroll
                for (int i = 0; i < 4; i++) h[rr][i] = silu(acc[2 * rr][j][i]) * acc[2 * rr + 1][j][i];
            float amax = 0.0f;
#pragma unroll
            for (int rr = 0; rr < 2; rr++)
#pragma unroll
                for (int i = 0; i < 4; i++) amax = fmaxf(amax, fabsf(h[rr][i]));
            amax = max_rows4(amax);
            const int e2 = quant_exp(amax);
            const float mul = inv_scale(e2);
            const int ffb = 64 * wave + 32 * blk, b = ffb / 32;
#pragma unroll
            for (int rr = 0; rr < 2; rr++) {
                const uint32_t c = e4m3x4(h[rr][0] * mul, h[rr][1] * mul, h[rr][2] * mul, h[rr][3] * mul);
                *reinterpret_cast<uint32_t *>(&L.h[dl_boff(r, (ffb >> 4) + rr) + 4 * q]) = c;
                if (valid) *reinterpret_cast<uint32_t *>(G.hq + (size_t)p * KD + ffb + 16 * rr + 4 * q) = c;
            }
            if (q == 0) {
                reinterpret_cast<uint8_t *>(L.hs[r])[(b & 3) * 4 + (b >> 2)] = (uint8_t)(127 + e2);
                if (valid) {
                    G.hs[(size_t)p * (KD / 32) + b] = (uint8_t)(127 + e2);
                    G.hs2[(size_t)p * (KD / 32) + (b & 3) * 4 + (b >> 2)] = (uint8_t)(127 + e2);
                }
            }
#pragma unroll
            for (int a = 0; a < 4; a++) acc[a][j] = v4f{0.f, 0.f, 0.f, 0.f};
        }
    };
    // down row tiles mt0 .. mt0+3 finished (acc[0..3]): weight, stage as
    // f16 + exponent, clear
    auto dn_store = [&](int mt0) {
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int r = 16 * j + n;
            const v4f c4[4] = {acc[0][j], acc[1][j], acc[2][j], acc[3][j]};
            store_dn16x4(Dn, L.ent[r], mt0, q, r < nr, c4, L.ws[r]);
#pragma unroll
            for (int i = 0; i < 4; i++) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
        }
    };
    static_for<0, NSG + NSD>([&](auto S) {
        constexpr int st = decltype(S)::value;
        auto &ac = acc;   // named here: an asm operand alone does not capture it
        // one step per scheduling region: otherwise later steps' loads are
        // hoisted and every step's fragments are live at once
        __builtin_amdgcn_sched_barrier(0);
        // issue step st+2 into the buffer step st-1 used, then compute step st
        if constexpr (st + 2 < NSG + NSD) load(std::integral_constant<int, st + 2>{}, bs[(st + 2) % 3]);
        // order inside the step: the next step's loads first, then per
        // K-step and column tile its B fragment read and 4 MFMAs
        if constexpr (st + 2 < NSG + NSD) {
            constexpr int nl = st + 2 < NSG ? 8 + (RT == 1 ? 2 : RT) : 8 + RD;
            __builtin_amdgcn_sched_group_barrier(0x020, nl, 0);
        }
        // B fragment i+1 is read before the MFMAs of fragment i issue
        constexpr int rts = st < NSG ? RT : RD, nfr = 8 / rts * NJ;
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
        for (int i = 0; i < nfr; i++) {
            if (i + 1 < nfr) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, rts, 0);
        }
        if constexpr (st < NSG) {
            gu_step(S, bs[st % 3]);
            if constexpr ((st & 7) == 7) swiglu(st >> 3);
            if constexpr (st == NSG - 1) {
                lds_barrier();   // every wave's h rows in LDS
#pragma unroll
                for (int j = 0; j < NJ; j++) hsv[j] = L.hs[16 * j + n][q];
            }
        } else {
            dn_step(S, bs[st % 3]);
            // two steps per pass of 4 row tiles
            if constexpr (((st - NSG) & 1) == 1) dn_store(16 * wave + 4 * ((st - NSG) >> 1));
        }
        // pin this step's MFMAs here: without a use the compiler sinks them
        // to the end and keeps every step's fragments live
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int j = 0; j < NJ; j++) asm volatile("" : "+v"(ac[a][j]));
    });
}

// Finds this workgroup's tile (expert e, sorted rows p0..p1) from the top-k
// indices; false past the last tile.  ev / wv keep this thread's entries
// for sx_gather.
__device__ bool sx_find(const SxArgs &X, SxLds &L, int ti, int &e_out, int &p0_out, int &p1_out, int (&ev)[kSxEnt],
                        float (&wv)[kSxEnt]) {
    const int tid = threadIdx.x, wave = tid >> 6;
    const int n = X.T * X.k, E = X.E;
    for (int e = tid; e < E; e += 64 * kSxW) L.cnt[e] = 0;
#pragma unroll
    for (int u = 0; u < kSxEnt; u++) {
        const int i = tid + 64 * kSxW * u;
        ev[u] = i < n ? X.idx[i] : -1;
        wv[u] = i < n ? X.wt[i] : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kSxEnt; u++)
        if (ev[u] >= 0) atomicAdd(&L.cnt[ev[u]], 1);
    __syncthreads();
    const int tn = X.tn;
    for (int e = tid; e < E; e += 64 * kSxW) L.ntl[e] = (L.cnt[e] + tn - 1) / tn;
    __syncthreads();
    if (wave == 0) wave_scan256(L.cnt, E, L.off, &L.off[E]);
    else if (wave == 1) wave_scan256(L.ntl, E, L.toff, &L.toff[E]);
    __syncthreads();
    const int nrt = L.toff[E];
    const int nsh = X.shg ? (X.T + tn - 1) / tn : 0;
    if (ti >= nrt + nsh) return false;
    if (ti == 0)
        for (int e = tid; e <= E; e += 64 * kSxW) X.e_off[e] = L.off[e];
    int e, p0, p1;
    if (ti < nrt) {
        for (int ee = tid; ee < E; ee += 64 * kSxW)
            if (L.ntl[ee] > 0 && ti >= L.toff[ee] && ti < L.toff[ee] + L.ntl[ee]) L.sel = ee;
        __syncthreads();
        e = __builtin_amdgcn_readfirstlane(L.sel);
        p0 = L.off[e] + (ti - L.toff[e]) * tn;
        p1 = min(p0 + tn, L.off[e] + L.cnt[e]);
    } else {   // shared-expert rows
        e = E;
        p0 = n + (ti - nrt) * tn;
        p1 = min(n + X.T, p0 + tn);
    }
    e_out = e;
    p0_out = __builtin_amdgcn_readfirstlane(p0);
    p1_out = __builtin_amdgcn_readfirstlane(p1);
    return true;
}

// Fills L.tok / L.ws with the rows of the tile sx_find found and writes
// their pos / perm.  It runs while the first weight step is in flight, so
// its barriers wait on LDS only.
__device__ void sx_gather(const SxArgs &X, SxLds &L, int e, int p0, int p1, const int (&ev)[kSxEnt],
                          const float (&wv)[kSxEnt]) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = X.T * X.k;
    if (e < X.E) {
        const int rank0 = p0 - L.off[e];
        // ranks of the expert's entries in entry order, 512 entries a round
        int base = 0;
#pragma unroll
        for (int u = 0; u < kSxEnt; u++) {
            if (64 * kSxW * u >= n) break;   // uniform
            const bool f = ev[u] == e;
            const uint64_t m = __ballot(f);
            if (lane == 0) L.wsum[wave] = __popcll(m);
            lds_barrier();
            int pre = 0, tot = 0;
#pragma unroll
            for (int w = 0; w < kSxW; w++) {
                pre += w < wave ? L.wsum[w] : 0;
                tot += L.wsum[w];
            }
            const int rank = base + pre +
                             (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
            if (f && rank >= rank0 && rank < rank0 + (p1 - p0)) {
                const int r = rank - rank0, i = tid + 64 * kSxW * u;
                L.tok[r] = i / X.k;
                L.ws[r] = wv[u];
                L.ent[r] = i;   // staged in entry order: the combine needs no pos
                X.pos[i] = p0 + r;
                X.perm[p0 + r] = i;
            }
            base += tot;
            lds_barrier();   // wsum is rewritten next round
        }
    } else {   // shared-expert rows: token order
        const int r0 = p0 - n;
        if (tid < p1 - p0) {
            const int t = r0 + tid;
            L.tok[tid] = t;
            L.ws[tid] = 1.0f / (1.0f + expf(-X.shg[(size_t)t * X.ld_shg]));
            L.ent[tid] = n + t;
        }
        lds_barrier();
    }
    const int nr = p1 - p0;
    if (tid >= nr && tid < kSkTok) L.tok[tid] = L.tok[nr - 1];
    lds_barrier();
}

__global__ __launch_bounds__(64 * kSxW) void k_skinny_expert(GemmArgs G, GemmArgs Dn, SxArgs X) {
    __shared__ SxLds L;
    const int ti = blockIdx.x;
    int e, p0, p1;
    if (X.discover) {
        int ev[kSxEnt];
        float wv[kSxEnt];
        if (!sx_find(X, L, ti, e, p0, p1, ev, wv)) return;
        auto prep = [&]() { sx_gather(X, L, e, p0, p1, ev, wv); };
        // an expert with one tile streams its weights once (non-temporal);
        // the tiles of a popular expert and of the shared expert reread
        // them, from L2 when they run close together
        const bool once = e < X.E && L.ntl[e] == 1;
        if (p1 - p0 <= 16) {
            if (once) skinny_expert<1, kSxRT, true>(G, Dn, e, p0, p1, L, prep);
            else skinny_expert<1, kSxRT, false>(G, Dn, e, p0, p1, L, prep);
        } else {
            skinny_expert<2, kSxRT, false>(G, Dn, e, p0, p1, L, prep);
        }
    } else {
        if (ti >= *G.ntiles) return;
        const int4 tile = G.tiles[ti];
        e = __builtin_amdgcn_readfirstlane(tile.x);
        p0 = __builtin_amdgcn_readfirstlane(tile.y);
        p1 = __builtin_amdgcn_readfirstlane(tile.z);
        auto prep = [&]() {
            if (threadIdx.x < kSkTok) {
                const int r = min((int)threadIdx.x, p1 - p0 - 1);
                L.tok[threadIdx.x] = G.row_tok[p0 + r];
                L.ws[threadIdx.x] = G.row_w[p0 + r];
                L.ent[threadIdx.x] = p0 + r;   // sorted order (the combine reads pos)
            }
            __syncthreads();
        };
        if (p1 - p0 <= 16) skinny_expert<1, kSxRT, false>(G, Dn, e, p0, p1, L, prep);
        else skinny_expert<2, kSxRT, false>(G, Dn, e, p0, p1, L, prep);
    }
}

// ---------------------------------------------------------------------------
// direct path for small batches (decode): no sort, two kernels
// ---------------------------------------------------------------------------
struct DirectArgs {
    const float *logits; int ld; int T; int E; int k; float scale;
    const void *x; int x_fmt;
    const float *shg; int ld_shg;               // shared-gate logit of token t: shg[t * ld_shg]
    const uint8_t *gate, *up, *down;            // routed experts (packed)
    const uint8_t *sh_gate, *sh_up, *sh_down;   // shared expert (packed) or null
    size_t wstride;                             // bytes per packed matrix
    int32_t *idx; float *wt;                    // routing of each entry
    int32_t *pos; int32_t *perm;                // identity maps (entry order)
    uint8_t *xq; uint8_t *xs;                   // quantised x (tap)
    float *hf;                                  // [entries][FF] fp32 SwiGLU rows
    uint8_t *hq; uint8_t *hs;                   // quantised h (tap)
    void *out; int out_fmt;
    const uint8_t *xs_in;                       // scales of pre-quantised x (x_fmt kFmtE4M3)
    size_t dn_wstride;                          // bytes per routed down matrix
    int dn_q8;                                  // routed down is q8_0-split
    float *hsf;                                 // int8 h scales (tap, q8_0-split down)
    int sh_q8;                                  // shared expert is q8_0-split
};

constexpr int kDD = 2048;   // d_model of the instantiated kernels

// Weight loads of the direct kernels: non-temporal while batches are small
// (each expert's bytes read once), cached from kDirectCachedT tokens, where
// entries sharing an expert reread its tiles (decode16: 128 entries over ~101
// experts).  Measured: T = 9 / 10 / 12 / 14 / 16 with cached loads 27.1 /
// 28.2 / 31.7 / 36.5 / 38.9 us against 26.6 / 28.0 / 31.9 / 36.9 / 39.9
// non-temporal.
constexpr int kDirectCachedT = 12;
// (a template parameter: a per-call select of the two loads measured 0.7 us
// slower at decode8, where only the non-temporal one runs)
template <bool CACHED>
__device__ __forceinline__ u32x4 direct_ld16(const void *p) {
    if constexpr (CACHED) return *reinterpret_cast<const u32x4 *>(p);
    else return ldg_nt16(p);
}
constexpr int kDF = 512;    // d_ff

// Entry i (token t, slot s; or the shared expert of token t for i >= T*k)
// x 16 rows of gate and up.  Wave w reduces K range [512w, 512w+512): it
// quantises exactly that range of x into LDS, so no cross-wave exchange is
// needed before the MFMAs.  Partial sums meet in LDS in wave order.
struct DirectGateupLds {
    __align__(16) uint8_t sx[kDD + 32];   // + 32 zero bytes
    uint8_t sxs[kDD / 32];
    float sxf[kDD / 32];                  // int8 x scales (q8_0-split shared expert)
    float red[4][2][32];                  // per wave: gate / up partial sums of up to 2 row tiles
    __align__(16) uint32_t rlds[4][kRouteLds];
};

// Shared-expert entry of the direct path when its matrices are q8_0-split
// (pf_gemm's int8 path, q36_engine.cu:3403-3406): wave w quantises x K
// [512w, 512w+512) per 32 to int8 + fp32 scale into LDS and runs its 16
// blocks against 16 rows of gate and up (int8 MFMA, each block scaled by
// both scales); partial sums meet in LDS in wave order as in the MXFP4 body.
__device__ __forceinline__ void direct_shared_q8(const DirectArgs &A, int t, int i, int ft, DirectGateupLds &L_) {
    constexpr int NKP = kDD / 64, NKB = kDD / 32;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int q = lane >> 4;
    const bool col0 = (lane & 15) == 0;
    int8_t *sx = reinterpret_cast<int8_t *>(L_.sx);
    float *sxf = L_.sxf;
    const X8 xr = load8_raw(A.x, A.x_fmt, (size_t)t * kDD + wave * 512 + lane * 8);
    // this wave's 8 K-pairs of the gate and up row tile ft
    u32x4 ag[8], au[8], sg[8], su[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
        const int kp = wave * 8 + u;
        ag[u] = *reinterpret_cast<const u32x4 *>(A.sh_gate + ((size_t)ft * NKP + kp) * 1024 + lane * 16);
        au[u] = *reinterpret_cast<const u32x4 *>(A.sh_up + ((size_t)ft * NKP + kp) * 1024 + lane * 16);
        const size_t so = (size_t)kDF * kDD + (((size_t)ft * 4 + q) * NKB + 2 * kp) * 8;
        sg[u] = *reinterpret_cast<const u32x4 *>(A.sh_gate + so);
        su[u] = *reinterpret_cast<const u32x4 *>(A.sh_up + so);
    }
    float v[8];
    cvt8(xr, A.x_fmt, v);
    float amax = 0.0f;
#pragma unroll
    for (int u = 0; u < 8; u++) amax = fmaxf(amax, fabsf(v[u]));
    amax = max_quad(amax);
    const float inv = q8b_inv(amax);
    *reinterpret_cast<uint2 *>(sx + wave * 512 + lane * 8) =
        make_uint2(q8b4(v[0], v[1], v[2], v[3], inv), q8b4(v[4], v[5], v[6], v[7], inv));
    if ((lane & 3) == 0) sxf[wave * 16 + (lane >> 2)] = amax / 127.0f;
    if (threadIdx.x < 8) reinterpret_cast<uint32_t *>(L_.sx + kDD)[threadIdx.x] = 0u;
    __syncthreads();
    v4f cg = {0.f, 0.f, 0.f, 0.f}, cu = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 8; u++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int kb = 2 * (wave * 8 + u) + h;
            // column 0 is the token; lanes of other columns read zeros
            const uint2 bv = *reinterpret_cast<const uint2 *>(col0 ? sx + kb * 32 + 8 * q : sx + kDD);
            const long b = (long)(((uint64_t)bv.y << 32) | bv.x);
            const float dh = sxf[kb];
            const long a0 = (long)(((uint64_t)ag[u][2 * h + 1] << 32) | ag[u][2 * h]);
            const long a1 = (long)(((uint64_t)au[u][2 * h + 1] << 32) | au[u][2 * h]);
            const v4i bias = {kQ8Bias, kQ8Bias, kQ8Bias, kQ8Bias};
            const v4i gi = __builtin_amdgcn_mfma_i32_16x16x32_i8(a0, b, bias, 0, 0, 0);
            const v4i ui = __builtin_amdgcn_mfma_i32_16x16x32_i8(a1, b, bias, 0, 0, 0);
            const uint32_t g01 = sg[u][2 * h], g23 = sg[u][2 * h + 1];
            const uint32_t u01 = su[u][2 * h], u23 = su[u][2 * h + 1];
            const float wg[4] = {f16lo(g01), f16hi(g01), f16lo(g23), f16hi(g23)};
            const float wu[4] = {f16lo(u01), f16hi(u01), f16lo(u23), f16hi(u23)};
#pragma unroll
            for (int r = 0; r < 4; r++) {
                cg[r] = fmaf(q8_scaled(gi[r], wg[r], -kQ8BiasF * wg[r]), dh, cg[r]);
                cu[r] = fmaf(q8_scaled(ui[r], wu[r], -kQ8BiasF * wu[r]), dh, cu[r]);
            }
            // one block per scheduling group (otherwise all 32 MFMA results
            // are held at once)
            asm volatile("" : "+v"(cg), "+v"(cu));
            __builtin_amdgcn_sched_barrier(0);
        }
    if (col0) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            L_.red[wave][0][4 * q + r] = cg[r];
            L_.red[wave][1][4 * q + r] = cu[r];
        }
    }
    __syncthreads();
    if (wave == 0 && lane < 16) {
        const float g = L_.red[0][0][lane] + L_.red[1][0][lane] + L_.red[2][0][lane] + L_.red[3][0][lane];
        const float u = L_.red[0][1][lane] + L_.red[1][1][lane] + L_.red[2][1][lane] + L_.red[3][1][lane];
        A.hf[(size_t)i * kDF + ft * 16 + lane] = silu(g) * u;
    }
}

// NFT row tiles ft0 .. ft0+NFT-1 per workgroup: one routing and NFT tiles'
// weight loads in flight.  Measured (gate/up us, one tile / two): T=2 7.2 /
// 7.5, T=4 9.8 / 10.0, T=8 16.5 / 15.5, T=16 27.4 / 25.6; four tiles at
// T=16 25.7.
template <bool SHQ8 = false, int NFT = 1, bool CACHED = false>
__device__ __forceinline__ void direct_gateup_body(const DirectArgs &A, int i, int ft0,
                                                   DirectGateupLds &L_) {
    static_assert(NFT == 1 || NFT == 2, "row tiles per workgroup");
    if constexpr (SHQ8) {   // workgroup-uniform: the shared expert's entries
        const int nr0 = A.T * A.k;
        if (i >= nr0) {
#pragma unroll
            for (int u = 0; u < NFT; u++) direct_shared_q8(A, i - nr0, i, ft0 + u, L_);
            return;
        }
    }
    uint8_t *sx = L_.sx;
    uint8_t *sxs = L_.sxs;
    auto &red = L_.red;
    auto &rlds = L_.rlds;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int nr = A.T * A.k;
    const bool routed = i < nr;
    const int t = routed ? i / A.k : i - nr;
    const int s = routed ? i % A.k : 0;

    // issue this wave's x loads first (512 values, 8 per lane), then the
    // logits (the other order measured 0.2 us slower at decode batch 1)
    const X8 xr = load8_raw(A.x, A.x_fmt, (size_t)t * kDD + wave * 512 + lane * 8);
    float lv[4];
    if (routed) route_load(A.logits + (size_t)t * A.ld, A.E, lv);

    int e = A.E;
    float wgt = 0.0f;
    if (routed) {
        // every wave routes the token (no barrier needed to share the result)
        // the expert index comes straight from the ranking lanes; the weight
        // (a further LDS round trip) is read after the weight loads issue
        e = route_rank(lv, A.E, A.k, rlds[wave], s);
    } else {
        wgt = 1.0f / (1.0f + expf(-A.shg[(size_t)t * A.ld_shg]));
    }
    const uint8_t *Wg = (e < A.E) ? A.gate + (size_t)e * A.wstride : A.sh_gate;
    const uint8_t *Wu = (e < A.E) ? A.up + (size_t)e * A.wstride : A.sh_up;
    const size_t nib = (size_t)kDF * kDD / 2;
    uint4 ag[NFT][4], au[NFT][4];
    int sag[NFT], sau[NFT];
#pragma unroll
    for (int u = 0; u < NFT; u++) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const size_t o = ((size_t)(ft0 + u) * (kDD / 128) + wave * 4 + j) * 1024 + (size_t)lane * 16;
            { const u32x4 t = direct_ld16<CACHED>(Wg + o); ag[u][j] = make_uint4(t[0], t[1], t[2], t[3]); }
            { const u32x4 t = direct_ld16<CACHED>(Wu + o); au[u][j] = make_uint4(t[0], t[1], t[2], t[3]); }
        }
        const size_t so = nib + ((size_t)(ft0 + u) * 64 + lane) * (kDD / 128) + wave * 4;
        sag[u] = *reinterpret_cast<const int *>(Wg + so);
        sau[u] = *reinterpret_cast<const int *>(Wu + so);
    }
    if (routed) {
        route_sync();
        wgt = route_weight(rlds[wave], A.k, A.scale, s);
    }

    if (A.x_fmt == kFmtE4M3) {
        *reinterpret_cast<uint2 *>(sx + wave * 512 + lane * 8) = make_uint2(xr.a[0], xr.a[1]);
        if ((lane & 3) == 0) sxs[wave * 16 + (lane >> 2)] = A.xs_in[(size_t)t * (kDD / 32) + wave * 16 + (lane >> 2)];
    } else {
        float xv[8];
        cvt8(xr, A.x_fmt, xv);
        quant8_lane(xv, lane, sx + wave * 512 + lane * 8, sxs + wave * 16 + (lane >> 2));
    }
    if (threadIdx.x < 8) reinterpret_cast<uint32_t *>(sx + kDD)[threadIdx.x] = 0u;
    __syncthreads();

    // B fragment: column 0 is the token; lanes of other columns read zeros
    const int q = lane >> 4;
    const bool col0 = (lane & 15) == 0;
    v4f cg[NFT], cu[NFT];
#pragma unroll
    for (int u = 0; u < NFT; u++) cg[u] = cu[u] = v4f{0.f, 0.f, 0.f, 0.f};
    static_for<0, 4>([&](auto J) {
        constexpr int j = decltype(J)::value;
        const int kt = wave * 4 + j;
        const uint8_t *b0p = col0 ? sx + kt * 128 + 16 * q : sx + kDD;
        const uint8_t *b1p = col0 ? sx + kt * 128 + 64 + 16 * q : sx + kDD + 16;
        const uint4 b0 = *reinterpret_cast<const uint4 *>(b0p);
        const uint4 b1 = *reinterpret_cast<const uint4 *>(b1p);
        const v8i b = v8i{(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w,
                          (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
        const int sb = sxs[kt * 4 + q];
#pragma unroll
        for (int u = 0; u < NFT; u++) {
            const v8i a0 = v8i{(int)ag[u][j].x, (int)ag[u][j].y, (int)ag[u][j].z, (int)ag[u][j].w, 0, 0, 0, 0};
            const v8i a1 = v8i{(int)au[u][j].x, (int)au[u][j].y, (int)au[u][j].z, (int)au[u][j].w, 0, 0, 0, 0};
            cg[u] = mfma_f4xf8<j>(a0, b, cg[u], sag[u], sb);
            cu[u] = mfma_f4xf8<j>(a1, b, cu[u], sau[u], sb);
        }
    });
    if (col0) {
#pragma unroll
        for (int u = 0; u < NFT; u++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                red[wave][0][16 * u + 4 * q + r] = cg[u][r];
                red[wave][1][16 * u + 4 * q + r] = cu[u][r];
            }
    }
    __syncthreads();
    if (wave == 0 && lane < 16 * NFT) {
        const int ft = ft0 + (lane >> 4), lr = lane & 15;
        const float g = red[0][0][lane] + red[1][0][lane] + red[2][0][lane] + red[3][0][lane];
        const float u = red[0][1][lane] + red[1][1][lane] + red[2][1][lane] + red[3][1][lane];
        A.hf[(size_t)i * kDF + ft * 16 + lr] = silu(g) * u;
    }
    if (ft0 == 0) {
        if (threadIdx.x == 0 && routed) {
            A.idx[i] = e;
            A.wt[i] = wgt;
            A.pos[i] = i;
            A.perm[i] = i;
        }
        if (routed && s == 0) {    // quantised x of token t (tap)
            for (int c = threadIdx.x; c < kDD / 16; c += 256)
                *reinterpret_cast<uint4 *>(A.xq + (size_t)t * kDD + c * 16) =
                    *reinterpret_cast<const uint4 *>(sx + c * 16);
            if (threadIdx.x < kDD / 32) A.xs[(size_t)t * (kDD / 32) + threadIdx.x] = sxs[threadIdx.x];
        }
    }
}

template <bool SHQ8, int NFT, bool CACHED = false>
__global__ __launch_bounds__(256) void k_direct_gateup(DirectArgs A) {
    __shared__ DirectGateupLds L_;
    direct_gateup_body<SHQ8, NFT, CACHED>(A, blockIdx.x, blockIdx.y * NFT, L_);
}

// Token t x 16 output rows; wave s handles slot s (wave k: shared expert):
// quantises its SwiGLU row, multiplies by the 16x512 down tile, scales by
// the routing weight; wave 0 adds the slots in order (k_moe_combine order,
// q36_engine.cu:784-791) and writes the output rows.  Q8: waves whose down
// matrix is q8_0-split (the routed slots with dn_q8, the shared expert with
// sh_q8) quantise h per 32 to int8 with an fp32 scale (k_quant_q8b) and run
// each 32-block as one int8 MFMA scaled by both scales (k_gemm_expert_i8).
template <bool Q8, bool CACHED = false>
__global__ __launch_bounds__(576) void k_direct_down(DirectArgs A) {
    __shared__ __align__(16) uint8_t sh[kMaxTopK + 1][kDF + 32];
    __shared__ uint8_t shs[kMaxTopK + 1][kDF / 32];
    __shared__ float shf[Q8 ? kMaxTopK + 1 : 1][kDF / 32];
    __shared__ float red[kMaxTopK + 1][16];
    const int rt = blockIdx.x, t = blockIdx.y;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int nslot = blockDim.x >> 6;
    const int nr = A.T * A.k;
    const bool routed = wave < A.k;
    const bool wq8 = Q8 && (routed ? A.dn_q8 : A.sh_q8);   // wave-uniform: selects the MFMA kind
    const int i = routed ? t * A.k + wave : nr + t;
    const int e = routed ? A.idx[i] : A.E;
    const float wgt = routed ? A.wt[i] : 1.0f / (1.0f + expf(-A.shg[(size_t)t * A.ld_shg]));
    const int q = lane >> 4;
    const bool col0 = (lane & 15) == 0;
    constexpr int NKP = kDF / 64, NKB = kDF / 32;
    float hv[8];
    load8(A.hf, Q36MOE_FMT_F32, (size_t)i * kDF + lane * 8, hv);
    // phase 1: this wave's down tile into registers, its h row quantised into LDS
    u32x4 ac[NKP], as[NKP];   // q8_0-split: codes and f16 scales
    uint4 a[4];               // MXFP4: E2M1 fragments and the scale dword
    int sa = 0;
    if (wq8) {
        const uint8_t *W = routed ? A.down + (size_t)e * A.dn_wstride : A.sh_down;
        const uint8_t *Wsc = W + (size_t)kDD * kDF;
#pragma unroll
        for (int kp = 0; kp < NKP; kp++) {
            ac[kp] = *reinterpret_cast<const u32x4 *>(W + ((size_t)rt * NKP + kp) * 1024 + lane * 16);
            as[kp] = *reinterpret_cast<const u32x4 *>(Wsc + (((size_t)rt * 4 + q) * NKB + 2 * kp) * 8);
        }
        // lanes 4j..4j+3 hold block j
        float amax = 0.0f;
#pragma unroll
        for (int u = 0; u < 8; u++) amax = fmaxf(amax, fabsf(hv[u]));
        amax = max_quad(amax);
        const float inv = q8b_inv(amax);
        const uint2 hc = make_uint2(q8b4(hv[0], hv[1], hv[2], hv[3], inv), q8b4(hv[4], hv[5], hv[6], hv[7], inv));
        *reinterpret_cast<uint2 *>(&sh[wave][lane * 8]) = hc;
        if ((lane & 3) == 0) shf[wave][lane >> 2] = amax / 127.0f;
        if (rt == 0) {   // quantised h (tap)
            *reinterpret_cast<uint2 *>(A.hq + (size_t)i * kDF + lane * 8) = hc;
            if ((lane & 3) == 0) A.hsf[(size_t)i * (kDF / 32) + (lane >> 2)] = amax / 127.0f;
        }
    } else {
        const uint8_t *W = (e < A.E) ? A.down + (size_t)e * A.dn_wstride : A.sh_down;
        const size_t nib = (size_t)kDD * kDF / 2;
#pragma unroll
        for (int j = 0; j < 4; j++)
            { const u32x4 t = direct_ld16<CACHED>(W + ((size_t)rt * 4 + j) * 1024 + (size_t)lane * 16); a[j] = make_uint4(t[0], t[1], t[2], t[3]); }
        sa = *reinterpret_cast<const int *>(W + nib + ((size_t)rt * 64 + lane) * 4);
        quant8_lane(hv, lane, &sh[wave][lane * 8], &shs[wave][lane >> 2]);
        if (rt == 0) {   // quantised h (tap)
            *reinterpret_cast<uint2 *>(A.hq + (size_t)i * kDF + lane * 8) =
                *reinterpret_cast<const uint2 *>(&sh[wave][lane * 8]);
            if ((lane & 3) == 0) A.hs[(size_t)i * (kDF / 32) + (lane >> 2)] = shs[wave][lane >> 2];
        }
    }
    if (lane < 8) reinterpret_cast<uint32_t *>(&sh[wave][kDF])[lane] = 0u;
    __syncthreads();
    // phase 2: column 0 is the entry's h row; lanes of other columns read zeros
    v4f c = {0.f, 0.f, 0.f, 0.f};
    if (wq8) {
#pragma unroll
        for (int kb = 0; kb < NKB; kb++) {
            const uint2 bv = *reinterpret_cast<const uint2 *>(col0 ? &sh[wave][kb * 32 + 8 * q] : &sh[wave][kDF]);
            const long b = (long)(((uint64_t)bv.y << 32) | bv.x);
            const u32x4 f = ac[kb >> 1];
            const long av = (kb & 1) ? (long)(((uint64_t)f[3] << 32) | f[2]) : (long)(((uint64_t)f[1] << 32) | f[0]);
            const v4i ci = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, b, v4i{kQ8Bias, kQ8Bias, kQ8Bias, kQ8Bias}, 0, 0, 0);
            const float dh = shf[wave][kb];
            const u32x4 sv = as[kb >> 1];
            const uint32_t s01 = (kb & 1) ? sv[2] : sv[0], s23 = (kb & 1) ? sv[3] : sv[1];
            const float w[4] = {f16lo(s01), f16hi(s01), f16lo(s23), f16hi(s23)};
#pragma unroll
            for (int r = 0; r < 4; r++) c[r] = fmaf(q8_scaled(ci[r], w[r], -kQ8BiasF * w[r]), dh, c[r]);
        }
    } else {
        static_for<0, 4>([&](auto J) {
            constexpr int j = decltype(J)::value;
            const uint8_t *b0p = col0 ? &sh[wave][j * 128 + 16 * q] : &sh[wave][kDF];
            const uint8_t *b1p = col0 ? &sh[wave][j * 128 + 64 + 16 * q] : &sh[wave][kDF + 16];
            const uint4 b0 = *reinterpret_cast<const uint4 *>(b0p);
            const uint4 b1 = *reinterpret_cast<const uint4 *>(b1p);
            const v8i b = v8i{(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w,
                              (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
            const int sb = shs[wave][j * 4 + q];
            const v8i av = v8i{(int)a[j].x, (int)a[j].y, (int)a[j].z, (int)a[j].w, 0, 0, 0, 0};
            c = mfma_f4xf8<j>(av, b, c, sa, sb);
        });
    }
    if (col0) {
#pragma unroll
        for (int r = 0; r < 4; r++) red[wave][4 * q + r] = c[r] * wgt;
    }
    __syncthreads();
    if (wave == 0 && lane < 16) {
        float acc = 0.0f;
        for (int sl = 0; sl < nslot; sl++) acc += red[sl][lane];
        const size_t o = (size_t)t * kDD + rt * 16 + lane;
        if (A.out_fmt == Q36MOE_FMT_F32) static_cast<float *>(A.out)[o] = acc;
        else static_cast<uint16_t *>(A.out)[o] = (uint16_t)f32_to_bf16(acc);
    }
}

// ---------------------------------------------------------------------------
// combine
// ---------------------------------------------------------------------------
// 4 staged values of row p from column j (f16 + exponent per 16 columns)
__device__ __forceinline__ float4 load_dn16(const uint16_t *__restrict__ dnh, const uint8_t *__restrict__ dne,
                                            int D, size_t p, int j) {
    const uint2 h = *reinterpret_cast<const uint2 *>(dnh + p * D + j);
    const float sc = __uint_as_float(((uint32_t)dne[p * (D / 16) + (j >> 4)] - 14u) << 23);
    return make_float4(f16lo(h.x) * sc, f16hi(h.x) * sc, f16lo(h.y) * sc, f16hi(h.y) * sc);
}

// Combine: token t's weighted rows summed in slot order (then the shared
// row), 8 columns per thread; every slot's load is issued before the first
// add, so a token costs one round trip after its slot positions.  Block
// (t, column block of 8 * blockDim.x).
__global__ __launch_bounds__(256) void k_combine(const uint16_t *__restrict__ dnh, const uint8_t *__restrict__ dne,
                                                const int32_t *__restrict__ pos, int T, int k,
                                                int D, int has_sh, void *out, int out_fmt) {
    const int t = blockIdx.x;
    const int j = (blockIdx.y * blockDim.x + threadIdx.x) * 8;
    if (j >= D) return;
    const int n = T * k;
    uint4 hv[kMaxTopK + 1];
    uint32_t ev[kMaxTopK + 1];
    const int ns = k + (has_sh ? 1 : 0);
#pragma unroll
    for (int s = 0; s < kMaxTopK + 1; s++) {
        if (s < ns) {
            // pos null: rows staged in entry order (the one-kernel path with
            // its tiles found in-kernel), so no dependent load of pos
            const size_t p = s < k ? (pos ? (size_t)pos[(size_t)t * k + s] : (size_t)t * k + s) : (size_t)(n + t);
            hv[s] = *reinterpret_cast<const uint4 *>(dnh + p * D + j);
            ev[s] = dne[p * (D / 16) + (j >> 4)];
        }
    }
    float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < kMaxTopK + 1; s++) {
        if (s < ns) {
            const float sc = __uint_as_float((ev[s] - 14u) << 23);
            const uint32_t w[4] = {hv[s].x, hv[s].y, hv[s].z, hv[s].w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                a[2 * i] += f16lo(w[i]) * sc;
                a[2 * i + 1] += f16hi(w[i]) * sc;
            }
        }
    }
    if (out_fmt == Q36MOE_FMT_F32) {
        float4 *o = reinterpret_cast<float4 *>(static_cast<float *>(out) + (size_t)t * D + j);
        o[0] = make_float4(a[0], a[1], a[2], a[3]);
        o[1] = make_float4(a[4], a[5], a[6], a[7]);
    } else {
        uint4 o;
        o.x = f32_to_bf16(a[0]) | (f32_to_bf16(a[1]) << 16);
        o.y = f32_to_bf16(a[2]) | (f32_to_bf16(a[3]) << 16);
        o.z = f32_to_bf16(a[4]) | (f32_to_bf16(a[5]) << 16);
        o.w = f32_to_bf16(a[6]) | (f32_to_bf16(a[7]) << 16);
        *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(out) + (size_t)t * D + j) = o;
    }
}

// The staged down rows widened to f32 (the DNW debug tap).
__global__ __launch_bounds__(256) void k_dn16_expand(const uint16_t *__restrict__ dnh, const uint8_t *__restrict__ dne,
                                                    int D, float *__restrict__ dst) {
    const size_t p = blockIdx.x;
    for (int j = threadIdx.x * 4; j < D; j += 256 * 4)
        *reinterpret_cast<float4 *>(dst + p * D + j) = load_dn16(dnh, dne, D, p, j);
}

// ---------------------------------------------------------------------------
// synthetic weights (benchmarks)
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// Region [0, nib) gets uniform bytes, [nib, nib + scl) exponent bytes in
// [lo, lo + span); 16 bytes per thread.
__global__ __launch_bounds__(256) void k_fill(uint8_t *dst, size_t nib, size_t scl, uint64_t seed,
                                             int lo, int span) {
    const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 16;
    if (i >= nib + scl) return;
    const uint64_t a = mix64(seed ^ (i * 0x9e3779b97f4a7c15ull));
    const uint64_t b = mix64(a ^ 0x632be59bd9b4e019ull);
    uint8_t v[16];
    for (int j = 0; j < 16; j++) {
        const uint8_t r = (uint8_t)((j < 8 ? a : b) >> (8 * (j & 7)));
        v[j] = (i + j < nib) ? r : (uint8_t)(lo + (int)(((uint32_t)r * (uint32_t)span) >> 8));
    }
    *reinterpret_cast<uint4 *>(dst + i) = *reinterpret_cast<const uint4 *>(v);
}

// ---------------------------------------------------------------------------
// calibration probe: one scaled MFMA on caller-packed lane operands
// ---------------------------------------------------------------------------
template <int FA, int FB>
__global__ void k_probe(const v8i *a, const v8i *b, const uint32_t *sa, const uint32_t *sb,
                        v4f *c) {
    const int l = threadIdx.x;
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[l], b[l], acc, FA, FB, 0,
                                                           (int)sa[l], 0, (int)sb[l]);
    c[l] = acc;
}

// v_mfma_scale_f32_32x32x64_f8f6f4 with the same lane data: 16 results per
// lane, c[l * 16 + i]
typedef float v16f __attribute__((ext_vector_type(16)));
__global__ void k_probe32(const v8i *a, const v8i *b, const uint32_t *sa, const uint32_t *sb, v16f *c) {
    const int l = threadIdx.x;
    v16f acc = {};
    acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[l], b[l], acc, 4, 0, 0, (int)sa[l], 0, (int)sb[l]);
    c[l] = acc;
}

template <int FA>
hipError_t launch_probe_b(int fb, const v8i *a, const v8i *b, const uint32_t *sa,
                          const uint32_t *sb, v4f *c, hipStream_t s) {
    switch (fb) {
        case 0: hipLaunchKernelGGL((k_probe<FA, 0>), dim3(1), dim3(64), 0, s, a, b, sa, sb, c); break;
        case 1: hipLaunchKernelGGL((k_probe<FA, 1>), dim3(1), dim3(64), 0, s, a, b, sa, sb, c); break;
        case 2: hipLaunchKernelGGL((k_probe<FA, 2>), dim3(1), dim3(64), 0, s, a, b, sa, sb, c); break;
        case 3: hipLaunchKernelGGL((k_probe<FA, 3>), dim3(1), dim3(64), 0, s, a, b, sa, sb, c); break;
        default: hipLaunchKernelGGL((k_probe<FA, 4>), dim3(1), dim3(64), 0, s, a, b, sa, sb, c); break;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
enum Stage { ST_ROUTE = 0, ST_SCAN, ST_GATEUP, ST_DOWN, ST_COMBINE, ST_COUNT };
const char *const kStageNames[ST_COUNT] = {"route", "scan", "gateup", "down", "combine"};

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace

struct q36moe_weights {
    int E, D, FF, FFsh;
    uint8_t *gate, *up, *down;       // [E][packed matrix]
    uint8_t *sh_gate, *sh_up, *sh_down;
    size_t gu_bytes, dn_bytes;       // one packed matrix
    int dn_q8;                       // routed down in the packed q8_0-split layout
    int sh_q8;                       // shared expert (all three matrices) q8_0-split
    size_t sh_gu_bytes, sh_dn_bytes; // one packed shared matrix
    void *base;                      // single device allocation
};

// Kernel arguments of the last forward; the weights are bound per launch so
// a stage can be replayed over other weight sets (q36moe_ctx_replay).
struct Plan {
    int T, has_sh, direct, skinny, fused, tiles, nb;
    RouteArgs ra;
    ScanArgs sa;
    GemmArgs ga, da;
    SxArgs sx;
    DirectArgs di;
    const void *out; int out_fmt;
};

// Device scratch of one forward for up to max_T tokens, carved from one
// base address (a context's allocation, or the library's static array for
// q36moe_forward_noalloc).  No kernel relies on its contents at entry.
struct Scratch {
    int max_T, E, D, FF, K;
    int nb_max;
    size_t tile_cap;
    int32_t *topk_idx; float *topk_w; int32_t *rank;
    uint8_t *xq, *xs, *xs2;
    int32_t *blk_cnt, *blk_off, *tot, *e_off, *perm, *pos, *row_tok;
    float *row_w;
    int4 *tiles; int32_t *ntiles;
    uint8_t *hq, *hs, *hs2;
    float *hsf;                     // fp32 scales of int8 h rows (q8_0-split down)
    int8_t *xq8; float *xsf;        // int8 x + fp32 scales (q8_0-split shared expert, sorted path)
    uint16_t *dnh; uint8_t *dne;    // staged weighted down rows: f16 [rows][D] + exponent per 16 columns
    float *hf;                      // direct path: fp32 SwiGLU rows
};

struct q36moe_ctx {
    int dev;
    hipStream_t stream;
    Scratch s;
    void *base;
    const uint8_t *tap_xq, *tap_xs;   // where the last forward's quantised x is
    int path_mode;                  // 0 auto, 1 sorted (fat tiles), 2 direct, 4 sorted (skinny tiles, two
                                    // kernels), 5 sorted (skinny tiles, one kernel per tile)
    int last_T, last_sh, last_path;
    int timing;
    Plan *plan;                     // kernel arguments of the last forward
    hipEvent_t ev[ST_COUNT + 1];
    double ms[ST_COUNT];
    int calls[ST_COUNT];
    ~q36moe_ctx() { delete plan; }
};

namespace {

int hip_rc(hipError_t e) { return e == hipSuccess ? Q36MOE_OK : Q36MOE_EHIP; }

// ggml type ids of the expert formats (q36.h:133-141)
constexpr int kTypeQ8_0 = 8, kTypeQ5_K = 13, kTypeQ6_K = 14, kTypeMXFP4 = 39;

bool dims_ok(int E, int D, int FF) {
    return E >= 1 && E <= kMaxExperts && D > 0 && FF > 0 && D % 512 == 0 && FF % 512 == 0;
}

int alloc_weights(int E, int D, int FF, int FFsh, int dn_q8, int sh_q8, q36moe_weights **out) {
    if (!out || !dims_ok(E, D, FF) || !(FFsh == 0 || FFsh == FF)) return Q36MOE_EINVAL;
    q36moe_weights *w = new (std::nothrow) q36moe_weights();
    if (!w) return Q36MOE_ENOMEM;
    w->E = E; w->D = D; w->FF = FF; w->FFsh = FFsh; w->dn_q8 = dn_q8; w->sh_q8 = FFsh ? sh_q8 : 0;
    const size_t m = (size_t)D * FF;
    w->gu_bytes = m / 2 + m / 32;
    const size_t q8_bytes = m + m / 16;               // int8 codes + f16 per 32
    w->dn_bytes = dn_q8 ? q8_bytes : w->gu_bytes;
    w->sh_gu_bytes = w->sh_dn_bytes = w->sh_q8 ? q8_bytes : w->gu_bytes;
    const size_t routed = align256(w->gu_bytes * E), routed_dn = align256(w->dn_bytes * E);
    const size_t sh_gu = align256(w->sh_gu_bytes), sh_dn = align256(w->sh_dn_bytes);
    const size_t total = 2 * routed + routed_dn + (FFsh ? 2 * sh_gu + sh_dn : 0);
    if (hipMalloc(&w->base, total) != hipSuccess) {
        delete w;
        return Q36MOE_ENOMEM;
    }
    uint8_t *p = static_cast<uint8_t *>(w->base);
    w->gate = p; w->up = p + routed; w->down = p + 2 * routed;
    if (FFsh) {
        uint8_t *q = p + 2 * routed + routed_dn;
        w->sh_gate = q; w->sh_up = q + sh_gu; w->sh_down = q + 2 * sh_gu;
    } else {
        w->sh_gate = w->sh_up = w->sh_down = nullptr;
    }
    *out = w;
    return Q36MOE_OK;
}

// Bytes per row of a matrix of row length K in ggml type t (blocks of 32,
// super-blocks of 256); 0 for a type no expert matrix may have here.
size_t type_row_bytes(int t, int K) {
    if (t == kTypeMXFP4 && K % 32 == 0) return (size_t)(K / 32) * 17;
    if (t == kTypeQ8_0 && K % 32 == 0) return (size_t)(K / 32) * 34;
    if (t == kTypeQ5_K && K % 256 == 0) return (size_t)(K / 256) * 176;
    if (t == kTypeQ6_K && K % 256 == 0) return (size_t)(K / 256) * 210;
    return 0;
}


// Lays out the scratch of one forward for up to max_T tokens from `base`
// (or only sizes it when base is null); returns the bytes it spans.
size_t carve_scratch(uint8_t *base, int max_T, int E, int D, int FF, int K, Scratch *S) {
    Scratch z{};
    Scratch &c = S ? *S : z;
    c.max_T = max_T; c.E = E; c.D = D; c.FF = FF; c.K = K;
    c.nb_max = (max_T + kRouteTPBSmall - 1) / kRouteTPBSmall;
    const size_t n = (size_t)max_T * K;
    const size_t rows = n + max_T;            // routed entries + shared rows
    c.tile_cap = n / 16 + (size_t)(n < (size_t)E ? n : E) + (max_T + 15) / 16 + 16;
    size_t off = 0;
    auto take = [&off](size_t bytes) { size_t o = off; off = align256(off + bytes); return o; };
    const size_t o_idx = take(n * 4), o_w = take(n * 4), o_rank = take(n * 4);
    const size_t o_xq = take((size_t)max_T * D), o_xs = take((size_t)max_T * D / 32);
    const size_t o_xs2 = take((size_t)max_T * D / 32);
    const size_t o_bc = take((size_t)c.nb_max * E * 4), o_bo = take((size_t)c.nb_max * E * 4);
    const size_t o_tot = take((size_t)E * 4);
    const size_t o_eo = take((size_t)(E + 1) * 4), o_perm = take(n * 4), o_pos = take(n * 4);
    const size_t o_rt = take(rows * 4), o_rw = take(rows * 4);
    const size_t o_tiles = take(c.tile_cap * 16), o_nt = take(4);
    const size_t o_hq = take(rows * FF), o_hs = take(rows * FF / 32), o_hs2 = take(rows * FF / 32);
    const size_t o_hsf = take(rows * FF / 32 * 4);
    const size_t o_xq8 = take((size_t)max_T * D), o_xsf = take((size_t)max_T * D / 32 * 4);
    const size_t o_dnh = take(rows * D * 2), o_dne = take(rows * D / 16);
    const size_t direct_rows = (size_t)(max_T < kDirectMaxT ? max_T : kDirectMaxT) * (K + 1);
    const size_t o_hf = take(direct_rows * FF * 4);
    if (!base) return off;
    uint8_t *b = base;
    c.topk_idx = reinterpret_cast<int32_t *>(b + o_idx);
    c.topk_w = reinterpret_cast<float *>(b + o_w);
    c.rank = reinterpret_cast<int32_t *>(b + o_rank);
    c.xq = b + o_xq; c.xs = b + o_xs; c.xs2 = b + o_xs2;
    c.blk_cnt = reinterpret_cast<int32_t *>(b + o_bc);
    c.blk_off = reinterpret_cast<int32_t *>(b + o_bo);
    c.tot = reinterpret_cast<int32_t *>(b + o_tot);
    c.e_off = reinterpret_cast<int32_t *>(b + o_eo);
    c.perm = reinterpret_cast<int32_t *>(b + o_perm);
    c.pos = reinterpret_cast<int32_t *>(b + o_pos);
    c.row_tok = reinterpret_cast<int32_t *>(b + o_rt);
    c.row_w = reinterpret_cast<float *>(b + o_rw);
    c.tiles = reinterpret_cast<int4 *>(b + o_tiles);
    c.ntiles = reinterpret_cast<int32_t *>(b + o_nt);
    c.hq = b + o_hq; c.hs = b + o_hs; c.hs2 = b + o_hs2;
    c.hsf = reinterpret_cast<float *>(b + o_hsf);
    c.xq8 = reinterpret_cast<int8_t *>(b + o_xq8);
    c.xsf = reinterpret_cast<float *>(b + o_xsf);
    c.dnh = reinterpret_cast<uint16_t *>(b + o_dnh);
    c.dne = b + o_dne;
    c.hf = reinterpret_cast<float *>(b + o_hf);
    return off;
}

// Scratch of q36moe_forward_noalloc: one static array per GPU, sized for
// kNoAllocMaxT tokens of the q36 shape (256 experts, top-8, d_model 2048,
// d_ff 512: about 5.7 MB of the 8 MiB).  In host code `scratch` names a
// host-side stand-in, not device memory: the device address of each GPU's
// copy is looked up once per device (hipGetSymbolAddress, with that device
// current) and only that address is handed to kernels.
constexpr int kNoAllocMaxT = 64;
constexpr size_t kNoAllocBytes = (size_t)8 << 20;
constexpr int kNoAllocMaxDev = 64;
__device__ __align__(256) uint8_t scratch[kNoAllocBytes];

std::mutex g_noalloc_mu;
uint8_t *g_noalloc_ptr[kNoAllocMaxDev];

// Device address of this GPU's scratch array (looked up on first use).
int noalloc_scratch(uint8_t **out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return Q36MOE_EHIP;
    if (dev < 0 || dev >= kNoAllocMaxDev) return Q36MOE_EINVAL;
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (!g_noalloc_ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return Q36MOE_EHIP;
        g_noalloc_ptr[dev] = static_cast<uint8_t *>(p);
    }
    *out = g_noalloc_ptr[dev];
    return Q36MOE_OK;
}

}  // namespace

extern "C" {

const char *q36moe_version(void) { return "q36moe 0.1 gfx950"; }

int q36moe_weights_alloc(int n_expert, int d_model, int d_ff, int d_ff_sh, q36moe_weights **out) {
    return alloc_weights(n_expert, d_model, d_ff, d_ff_sh, 0, 0, out);
}

int q36moe_weights_upload(const void *gate, const void *up, const void *down, const void *sh_gate,
                          const void *sh_up, const void *sh_down, int n_expert, int d_model,
                          int d_ff, int d_ff_sh, q36moe_weights **out) {
    return q36moe_weights_upload_typed(gate, up, down, kTypeMXFP4, sh_gate, sh_up, sh_down, kTypeMXFP4, n_expert,
                                       d_model, d_ff, d_ff_sh, out);
}

int q36moe_weights_upload_typed(const void *gate, const void *up, const void *down, int down_type,
                                const void *sh_gate, const void *sh_up, const void *sh_down, int sh_type,
                                int n_expert, int d_model, int d_ff, int d_ff_sh, q36moe_weights **out) {
    if (!gate || !up || !down || !out) return Q36MOE_EINVAL;
    if (d_ff_sh && (!sh_gate || !sh_up || !sh_down)) return Q36MOE_EINVAL;
    const size_t dn_row = type_row_bytes(down_type, d_ff);
    if (!dn_row) return Q36MOE_EINVAL;
    if (d_ff_sh && (!type_row_bytes(sh_type, d_model) || !type_row_bytes(sh_type, d_ff))) return Q36MOE_EINVAL;
    const int dn_q8 = down_type != kTypeMXFP4, sh_q8 = d_ff_sh && sh_type != kTypeMXFP4;
    q36moe_weights *w = nullptr;
    int rc = alloc_weights(n_expert, d_model, d_ff, d_ff_sh, dn_q8, sh_q8, &w);
    if (rc) return rc;
    const size_t gu_src = (size_t)d_ff * (d_model / 32) * 17;
    const size_t dn_src = (size_t)d_model * dn_row;
    const int sh_t = d_ff_sh ? sh_type : kTypeMXFP4;
    // (src, src stride, dst, dst stride, M, K, count, ggml type)
    struct Job { const uint8_t *src; size_t src_stride; uint8_t *dst; size_t dst_stride; int M, K, n, type; };
    const Job jobs[6] = {
        {static_cast<const uint8_t *>(gate), gu_src, w->gate, w->gu_bytes, d_ff, d_model, n_expert, kTypeMXFP4},
        {static_cast<const uint8_t *>(up), gu_src, w->up, w->gu_bytes, d_ff, d_model, n_expert, kTypeMXFP4},
        {static_cast<const uint8_t *>(down), dn_src, w->down, w->dn_bytes, d_model, d_ff, n_expert, down_type},
        {static_cast<const uint8_t *>(sh_gate), 0, w->sh_gate, w->sh_gu_bytes, d_ff, d_model, d_ff_sh ? 1 : 0, sh_t},
        {static_cast<const uint8_t *>(sh_up), 0, w->sh_up, w->sh_gu_bytes, d_ff, d_model, d_ff_sh ? 1 : 0, sh_t},
        {static_cast<const uint8_t *>(sh_down), 0, w->sh_down, w->sh_dn_bytes, d_model, d_ff, d_ff_sh ? 1 : 0, sh_t},
    };
    // each matrix set is repacked on host threads (experts split across
    // them, as the reference's upload does with OpenMP) into one staging
    // buffer, then copied in one transfer
    const unsigned hw = std::thread::hardware_concurrency();
    const int nth = (int)(hw == 0 ? 1 : hw > 16 ? 16 : hw);
    for (const Job &j : jobs) {
        if (rc || j.n == 0) continue;
        uint8_t *stage = static_cast<uint8_t *>(malloc(j.dst_stride * j.n));
        if (!stage) { rc = Q36MOE_ENOMEM; break; }
        std::atomic<int> err{0};
        auto work = [&](int tid) noexcept {
            const bool q8 = j.type != kTypeMXFP4;
            std::vector<int8_t> codes;
            std::vector<uint16_t> scales;
            try {
                codes.resize(q8 ? (size_t)j.M * j.K : 0);
                scales.resize(q8 ? (size_t)j.M * j.K / 32 : 0);
            } catch (...) {
                err.store(Q36MOE_ENOMEM);
                return;
            }
            for (int e = tid; e < j.n; e += nth) {
                int r;
                if (q8) {
                    r = q36moe_requant_q8(j.type, j.src + j.src_stride * e, j.M, j.K, codes.data(), scales.data());
                    if (r == 0) r = q36moe_pack_q8(codes.data(), scales.data(), j.M, j.K, stage + j.dst_stride * e);
                } else {
                    r = q36moe_pack_mxfp4(j.src + j.src_stride * e, j.M, j.K, stage + j.dst_stride * e);
                }
                if (r) err.store(r);
            }
        };
        const int nt = j.n < nth ? j.n : nth;
        std::vector<std::thread> pool;
        try {
            for (int t = 1; t < nt; t++) pool.emplace_back(work, t);
        } catch (...) {
            // threads that could not be started: their share runs here
            for (int t = (int)pool.size() + 1; t < nt; t++) work(t);
        }
        work(0);
        for (auto &t : pool) t.join();
        rc = err.load();
        if (rc == 0) rc = hip_rc(hipMemcpy(j.dst, stage, j.dst_stride * j.n, hipMemcpyHostToDevice));
        free(stage);
    }
    if (rc) {
        q36moe_weights_free(w);
        return rc;
    }
    *out = w;
    return Q36MOE_OK;
}

int q36moe_weights_fill_synthetic(q36moe_weights *w, uint64_t seed, int exp_lo, int exp_hi,
                                  void *stream) {
    if (!w || exp_lo > exp_hi || exp_lo < -127 || exp_hi > 127) return Q36MOE_EINVAL;
    if (w->dn_q8 || w->sh_q8) return Q36MOE_EINVAL;   // MXFP4 sets only
    hipStream_t s = static_cast<hipStream_t>(stream);
    const size_t m = (size_t)w->D * w->FF, nib = m / 2, scl = m / 32;
    uint8_t *mats[3] = {w->gate, w->up, w->down};
    uint64_t salt = 1;
    for (int k = 0; k < 3; k++)
        for (int e = 0; e < w->E; e++, salt++) {
            hipLaunchKernelGGL(k_fill, dim3((unsigned)((nib + scl) / 16 / 256 + 1)), dim3(256), 0, s,
                               mats[k] + w->gu_bytes * e, nib, scl, seed * 0x100000001b3ull + salt,
                               127 + exp_lo, exp_hi - exp_lo + 1);
        }
    if (w->FFsh) {
        uint8_t *sh[3] = {w->sh_gate, w->sh_up, w->sh_down};
        for (int k = 0; k < 3; k++, salt++)
            hipLaunchKernelGGL(k_fill, dim3((unsigned)((nib + scl) / 16 / 256 + 1)), dim3(256), 0, s,
                               sh[k], nib, scl, seed * 0x100000001b3ull + salt, 127 + exp_lo,
                               exp_hi - exp_lo + 1);
    }
    return hip_rc(hipGetLastError());
}

int q36moe_weights_device_ptrs(const q36moe_weights *w, void **gate, void **up, void **down,
                               void **sh_gate, void **sh_up, void **sh_down, size_t *gate_bytes,
                               size_t *down_bytes) {
    if (!w) return Q36MOE_EINVAL;
    if (gate) *gate = w->gate;
    if (up) *up = w->up;
    if (down) *down = w->down;
    if (sh_gate) *sh_gate = w->sh_gate;
    if (sh_up) *sh_up = w->sh_up;
    if (sh_down) *sh_down = w->sh_down;
    if (gate_bytes) *gate_bytes = w->gu_bytes;
    if (down_bytes) *down_bytes = w->dn_bytes;
    return Q36MOE_OK;
}

int q36moe_weights_down_type(const q36moe_weights *w) {
    if (!w) return Q36MOE_EINVAL;
    return w->dn_q8 ? kTypeQ8_0 : kTypeMXFP4;
}

int q36moe_weights_shared_type(const q36moe_weights *w) {
    if (!w) return Q36MOE_EINVAL;
    if (!w->FFsh) return 0;
    return w->sh_q8 ? kTypeQ8_0 : kTypeMXFP4;
}

void q36moe_weights_free(q36moe_weights *w) {
    if (!w) return;
    if (w->base) (void)hipFree(w->base);
    delete w;
}

int q36moe_ctx_create(int max_tokens, int n_expert, int d_model, int d_ff, int top_k, void *stream,
                      q36moe_ctx **out) {
    if (!out || max_tokens < 1 || !dims_ok(n_expert, d_model, d_ff) || top_k < 1 ||
        top_k > kMaxTopK || top_k > n_expert)
        return Q36MOE_EINVAL;
    q36moe_ctx *c = new (std::nothrow) q36moe_ctx();
    if (!c) return Q36MOE_ENOMEM;
    c->plan = new (std::nothrow) Plan();
    if (!c->plan) {
        delete c;
        return Q36MOE_ENOMEM;
    }
    if (hipGetDevice(&c->dev) != hipSuccess) {
        delete c;
        return Q36MOE_EHIP;
    }
    c->stream = static_cast<hipStream_t>(stream);
    const size_t bytes = carve_scratch(nullptr, max_tokens, n_expert, d_model, d_ff, top_k, nullptr);
    if (hipMalloc(&c->base, bytes) != hipSuccess) {
        delete c;
        return Q36MOE_ENOMEM;
    }
    carve_scratch(static_cast<uint8_t *>(c->base), max_tokens, n_expert, d_model, d_ff, top_k, &c->s);
    c->tap_xq = c->s.xq; c->tap_xs = c->s.xs;
    for (int i = 0; i <= ST_COUNT; i++) {
        if (hipEventCreate(&c->ev[i]) != hipSuccess) {
            for (int j = 0; j < i; j++) (void)hipEventDestroy(c->ev[j]);
            (void)hipFree(c->base);
            delete c;
            return Q36MOE_EHIP;
        }
    }
    *out = c;
    return Q36MOE_OK;
}

int q36moe_ctx_set_stream(q36moe_ctx *c, void *stream) {
    if (!c) return Q36MOE_EINVAL;
    c->stream = static_cast<hipStream_t>(stream);
    return Q36MOE_OK;
}

void q36moe_ctx_free(q36moe_ctx *c) {
    if (!c) return;
    for (int i = 0; i <= ST_COUNT; i++) (void)hipEventDestroy(c->ev[i]);
    if (c->base) (void)hipFree(c->base);
    delete c;
}

static void bind_weights(Plan &P, const q36moe_weights *w) {
    P.ga.wa = w->gate; P.ga.wb = w->up; P.ga.sa = w->sh_gate; P.ga.sb = w->sh_up;
    P.ga.wstride = w->gu_bytes;
    P.da.wa = w->down; P.da.wb = nullptr; P.da.sa = w->sh_down; P.da.sb = nullptr;
    P.da.wstride = w->dn_bytes;
    P.ga.hq8 = P.da.hq8 = w->dn_q8;
    P.ga.shq8 = P.da.shq8 = P.has_sh && w->sh_q8;
    P.di.gate = w->gate; P.di.up = w->up; P.di.down = w->down;
    P.di.sh_gate = w->sh_gate; P.di.sh_up = w->sh_up; P.di.sh_down = P.has_sh ? w->sh_down : nullptr;
    P.di.wstride = w->gu_bytes;
    P.di.dn_wstride = w->dn_bytes;
    P.di.dn_q8 = w->dn_q8;
    P.di.sh_q8 = P.has_sh && w->sh_q8;
}

// Launches the kernels of one stage (direct path: ST_GATEUP is the routing +
// gate/up kernel, ST_DOWN the down + combine kernel; its other stages are
// empty).
static void launch_stage(const Scratch &c, const Plan &P, int st, hipStream_t s) {
    const int T = P.T, K = c.K, D = c.D, FF = c.FF;
    if (P.direct) {
        const int n = T * K + (P.has_sh ? T : 0);
        if (st == ST_GATEUP) {
            // two row tiles per workgroup from kDirect2Tiles tokens on (one
            // routing and twice the loads in flight per workgroup; below
            // that, more workgroups spread a small batch better)
            static_assert(kDirectCachedT >= kDirect2Tiles, "cached loads only in the two-tile kernels");
            if (T >= kDirectCachedT) {
                if (P.di.sh_q8)
                    hipLaunchKernelGGL((k_direct_gateup<true, 2, true>), dim3(n, FF / 32), dim3(256), 0, s, P.di);
                else
                    hipLaunchKernelGGL((k_direct_gateup<false, 2, true>), dim3(n, FF / 32), dim3(256), 0, s, P.di);
            } else if (T >= kDirect2Tiles) {
                if (P.di.sh_q8)
                    hipLaunchKernelGGL((k_direct_gateup<true, 2>), dim3(n, FF / 32), dim3(256), 0, s, P.di);
                else
                    hipLaunchKernelGGL((k_direct_gateup<false, 2>), dim3(n, FF / 32), dim3(256), 0, s, P.di);
            } else {
                if (P.di.sh_q8)
                    hipLaunchKernelGGL((k_direct_gateup<true, 1>), dim3(n, FF / 16), dim3(256), 0, s, P.di);
                else
                    hipLaunchKernelGGL((k_direct_gateup<false, 1>), dim3(n, FF / 16), dim3(256), 0, s, P.di);
            }
        } else if (st == ST_DOWN) {
            const bool q8 = P.di.dn_q8 || P.di.sh_q8, cached = T >= kDirectCachedT;
            const dim3 g(D / 16, T), b(64 * (K + P.has_sh));
            if (q8 && cached) hipLaunchKernelGGL((k_direct_down<true, true>), g, b, 0, s, P.di);
            else if (q8) hipLaunchKernelGGL((k_direct_down<true, false>), g, b, 0, s, P.di);
            else if (cached) hipLaunchKernelGGL((k_direct_down<false, true>), g, b, 0, s, P.di);
            else hipLaunchKernelGGL((k_direct_down<false, false>), g, b, 0, s, P.di);
        }
        return;
    }
    switch (st) {
        case ST_ROUTE:
            launch_route(P.sa.tpb == kRouteTPB, P.nb, s, P.ra);
            break;
        case ST_SCAN:
            if (P.fused && P.sx.discover) break;   // k_skinny_expert finds its own tile
            if (!P.sa.inline_cols)
                hipLaunchKernelGGL(k_colscan, dim3((c.E + kColExp - 1) / kColExp), dim3(256), 0, s, P.sa);
            hipLaunchKernelGGL(k_scatter, dim3(P.nb), dim3(256), 0, s, P.sa);
            break;
        case ST_GATEUP:
            if (P.fused) {
                hipLaunchKernelGGL(k_skinny_expert, dim3(P.tiles), dim3(64 * kSxW), 0, s, P.ga, P.da, P.sx);
            } else if (P.skinny) {
                hipLaunchKernelGGL(k_skinny_gateup, dim3(P.tiles * 16), dim3(64 * kSkW), 0, s, P.ga);
                if (P.ga.shq8)
                    hipLaunchKernelGGL(k_shared_gateup_q8, dim3((T + kShTok - 1) / kShTok, kShRb), dim3(256), 0, s,
                                       P.ga);
            } else
                hipLaunchKernelGGL(k_gateup_dma, dim3(P.tiles * (FF / (16 * gdma::RT)) + P.ga.sh_wgs),
                                   dim3(64 * gdma::W), 0, s, P.ga);
            break;
        case ST_DOWN:
            if (P.fused) break;   // in k_skinny_expert
            if (P.da.hq8 || P.da.shq8)
                hipLaunchKernelGGL(k_down_lds<true>, dim3(P.tiles * (D / (16 * kDlRT * kDlW))), dim3(64 * kDlW), 0, s,
                                   P.da);
            else
                hipLaunchKernelGGL(k_down_lds<false>, dim3(P.tiles * (D / (16 * kDlRT * kDlW))), dim3(64 * kDlW), 0,
                                   s, P.da);
            break;
        case ST_COMBINE:
            // small batches: 64-thread blocks, so the work spreads over more CUs
            hipLaunchKernelGGL(k_combine, dim3(T, T < 256 ? D / 512 : D / 2048), dim3(T < 256 ? 64 : 256), 0, s, c.dnh,
                               c.dne, P.fused && P.sx.discover ? nullptr : c.pos, T, K, D, P.has_sh,
                               const_cast<void *>(P.out), P.out_fmt);
            break;
        default: break;
    }
}

int q36moe_ctx_replay(q36moe_ctx *c, const q36moe_weights *w, int stage) {
    if (!c || !w || stage < 0 || stage >= ST_COUNT) return Q36MOE_EINVAL;
    if (c->last_T <= 0) return Q36MOE_EINVAL;
    if (w->E != c->s.E || w->D != c->s.D || w->FF != c->s.FF) return Q36MOE_EINVAL;
    if (c->plan->has_sh && !w->sh_gate) return Q36MOE_EINVAL;
    // the plan's h quantisation matches the down format it was made for
    if ((c->plan->direct ? c->plan->di.dn_q8 : c->plan->da.hq8) != w->dn_q8) return Q36MOE_EINVAL;
    if ((c->plan->direct ? c->plan->di.sh_q8 : c->plan->da.shq8) != (c->plan->has_sh && w->sh_q8))
        return Q36MOE_EINVAL;
    Plan P = *c->plan;
    bind_weights(P, w);
    launch_stage(c->s, P, stage, c->stream);
    return hipGetLastError() == hipSuccess ? Q36MOE_OK : Q36MOE_EHIP;
}

// Plans one forward on scratch c and launches its kernels on stream s
// (events ev[0..ST_COUNT] around the stages when ev is non-null).
// x_fmt: Q36MOE_FMT_F32 / _BF16, or kFmtE4M3 with x the codes and xs_in the
// scales of already quantised activations.
static int launch_forward(const Scratch &c, Plan &P, int pm, const q36moe_weights *w, const void *x, int x_fmt,
                          const uint8_t *xs_in, const float *logits, int ld_logits, const float *shg,
                          int ld_shg, int T, float scale, void *out, int out_fmt, hipStream_t s,
                          hipEvent_t *ev) {
    if (!w || T < 0 || T > c.max_T) return Q36MOE_EINVAL;
    if (w->E != c.E || w->D != c.D || w->FF != c.FF) return Q36MOE_EINVAL;
    if (out_fmt != Q36MOE_FMT_F32 && out_fmt != Q36MOE_FMT_BF16) return Q36MOE_EINVAL;
    // kernels are instantiated for the q36 shape (q36.h:78-84)
    if (c.D != 2048 || c.FF != 512) return Q36MOE_EINVAL;
    if (T == 0) return Q36MOE_OK;
    if (!x || !logits || !out || ld_logits < c.E) return Q36MOE_EINVAL;
    if (x_fmt == kFmtE4M3 && !xs_in) return Q36MOE_EINVAL;
    if (shg && !w->sh_gate) return Q36MOE_EINVAL;
    if (ld_shg < 0) return Q36MOE_EINVAL;
    if (ld_shg == 0) ld_shg = 1;
    const int has_sh = shg != nullptr;
    const int E = c.E, D = c.D, FF = c.FF, K = c.K;
    const int n = T * K;
    const int tpb = T <= kRouteSmallT ? kRouteTPBSmall : kRouteTPB;
    const int nb = (T + tpb - 1) / tpb;

    const bool direct = pm == 2 ? (T <= kDirectMaxT) : (pm == 1 || pm == 4 || pm == 5) ? false : (T <= kDirectMaxT);
    if (pm == 2 && !direct) return Q36MOE_EINVAL;
    const bool shq8 = has_sh && w->sh_q8;
    // a q8_0-split shared expert quantises x itself (int8 + fp32 per 32):
    // pre-quantised e4m3 input cannot feed it
    if (shq8 && x_fmt == kFmtE4M3) return Q36MOE_EINVAL;
    // sorted path: skinny tiles (<= 32 rows) while the average expert has at
    // most kSkinnyRows rows, else fat tiles of up to kGdTok rows
    // the one-kernel skinny path (every matrix MXFP4) serves twice the rows
    // per expert: it beat fat tiles up to 512 tokens (T=384: 96 vs 103 us)
    const bool fusable = !w->dn_q8 && !shq8;
    const size_t skinny_rows = (size_t)(fusable ? kSxFusedRows : kSkinnyRows) * E;
    const bool skinny = pm == 4 || pm == 5 || (pm == 0 && (size_t)n <= skinny_rows);
    // skinny tiles in one kernel per tile (k_skinny_expert) when every
    // matrix is MXFP4; the int8 down or shared expert keeps two kernels
    const bool fused = skinny && pm != 4 && fusable;
    const int tn = skinny ? kSkTok : kGdTok;
    // a q8_0-split shared expert's down is VALU-heavy: its rows go in small
    // tiles so the work spreads over many workgroups instead of trailing
    const int tn_sh = shq8 ? kSkTok : tn;
    int tiles = n / tn + (n < E ? n : E) + (has_sh ? (T + tn_sh - 1) / tn_sh : 0);
    tiles = (tiles + 7) & ~7;   // whole groups of 8 for the XCD-major tile order

    P = Plan{};
    P.T = T; P.has_sh = has_sh; P.direct = direct; P.skinny = skinny; P.fused = fused;
    P.tiles = tiles; P.nb = nb; P.out = out; P.out_fmt = out_fmt;
    if (direct) {
        P.di = DirectArgs{logits, ld_logits, T, E, K, scale, x, x_fmt, shg, ld_shg,
                          nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0,
                          c.topk_idx, c.topk_w, c.pos, c.perm, c.xq, c.xs, c.hf,
                          c.hq, c.hs, out, out_fmt, xs_in, 0, 0, c.hsf};
    } else {
        P.ra = RouteArgs{logits, ld_logits, T, E, K, scale, x, x_fmt, D, nb,
                         c.topk_idx, c.topk_w, c.xq, c.xs, c.xs2, c.blk_cnt, c.rank, xs_in, nullptr, nullptr, 1};
        P.sa = ScanArgs{c.blk_cnt, nb, tpb, nb <= kScanInlineBlocks ? 1 : 0, E, T, K, c.topk_idx, c.topk_w, c.rank,
                        shg, ld_shg, tn, tn_sh, c.blk_off, c.tot, c.e_off, c.perm, c.pos, c.row_tok, c.row_w,
                        c.tiles, c.ntiles};
        GemmArgs &ga = P.ga;
        ga.E = E; ga.M = FF;
        ga.tiles = c.tiles; ga.ntiles = c.ntiles;
        // pre-quantised codes are read where the caller left them
        ga.bq = x_fmt == kFmtE4M3 ? static_cast<const uint8_t *>(x) : c.xq;
        ga.bs2 = c.xs2; ga.row_tok = c.row_tok; ga.row_w = c.row_w;
        ga.hq = c.hq; ga.hs = c.hs; ga.hs2 = c.hs2; ga.ldo = FF;
        ga.hsf = c.hsf;
        ga.xq8 = c.xq8; ga.xsf = c.xsf; ga.T = T; ga.nrouted = n;
        ga.sh_wgs = shq8 && !skinny ? (T + kShTok - 1) / kShTok * kShRb : 0;
        GemmArgs &da = P.da;
        da = ga;
        da.M = D;
        da.bq = c.hq; da.bs2 = c.hs2; da.dnh = c.dnh; da.dne = c.dne; da.ldo = D;
        da.bsf = c.hsf;
        // discovered tiles: 16 rows while the average expert has at most 4
        // (T <= 128 at 256 experts, top-8), else 32: a second column tile
        // rather than a second stream of the same weights, and no more tiles
        // than CUs (T=256: 100.5 -> 85.5 us)
        const int stn = (size_t)n <= (size_t)4 * E ? kSxTok : kSkTok;
        P.sx = SxArgs{c.topk_idx, c.topk_w, shg, ld_shg, c.perm, c.pos, c.e_off, T, K, E,
                      fused && n <= kSxDiscoverMax ? 1 : 0, stn};
        if (P.sx.discover) {   // grid for tiles of stn rows; no counts for a scatter
            P.ra.counts = 0;
            int t = n / stn + (n < E ? n : E) + (has_sh ? (T + stn - 1) / stn : 0);
            P.tiles = (t + 7) & ~7;
        }
    }
    bind_weights(P, w);
    if (!direct && shq8) {   // k_route also writes the int8 x the shared expert reads
        P.ra.xq8 = c.xq8;
        P.ra.xsf = c.xsf;
    }
    for (int st = 0; st < ST_COUNT; st++) {
        if (ev) (void)hipEventRecord(ev[st], s);
        launch_stage(c, P, st, s);
    }
    if (ev) (void)hipEventRecord(ev[ST_COUNT], s);
    return hipGetLastError() == hipSuccess ? Q36MOE_OK : Q36MOE_EHIP;
}

static int forward_impl(q36moe_ctx *c, const q36moe_weights *w, const void *x, int x_fmt,
                        const uint8_t *xs_in, const float *logits, int ld_logits, const float *shg,
                        int ld_shg, int T, float scale, void *out, int out_fmt) {
    if (!c) return Q36MOE_EINVAL;
    Plan P;
    const int rc = launch_forward(c->s, P, c->path_mode, w, x, x_fmt, xs_in, logits, ld_logits, shg, ld_shg, T,
                                  scale, out, out_fmt, c->stream, c->timing ? c->ev : nullptr);
    if (rc || T == 0) return rc;
    *c->plan = P;
    c->last_T = T;
    c->last_sh = P.has_sh;
    c->last_path = P.direct ? 1 : P.fused ? 3 : P.skinny ? 2 : 0;
    // the sorted path reads pre-quantised codes in place; the direct path
    // copies every token's codes into the context
    const bool in_place = !P.direct && x_fmt == kFmtE4M3;
    c->tap_xq = in_place ? static_cast<const uint8_t *>(x) : c->s.xq;
    c->tap_xs = in_place ? xs_in : c->s.xs;
    if (c->timing) {
        if (hipEventSynchronize(c->ev[ST_COUNT]) != hipSuccess) return Q36MOE_EHIP;
        for (int st = 0; st < ST_COUNT; st++) {
            float ms = 0.f;
            if (hipEventElapsedTime(&ms, c->ev[st], c->ev[st + 1]) != hipSuccess) return Q36MOE_EHIP;
            c->ms[st] += ms;
            c->calls[st]++;
        }
    }
    return Q36MOE_OK;
}

int q36moe_forward(q36moe_ctx *c, const q36moe_weights *w, const void *x, int x_fmt,
                   const float *logits, int ld_logits, const float *shg, int ld_shg, int T, float scale,
                   void *out, int out_fmt) {
    if (x_fmt != Q36MOE_FMT_F32 && x_fmt != Q36MOE_FMT_BF16) return Q36MOE_EINVAL;
    return forward_impl(c, w, x, x_fmt, nullptr, logits, ld_logits, shg, ld_shg, T, scale, out, out_fmt);
}

int q36moe_forward_noalloc(const q36moe_weights *w, const void *x, int x_fmt, const float *logits, int ld_logits,
                           const float *shg, int ld_shg, int T, int top_k, float scale, void *out, int out_fmt,
                           void *stream) {
    if (!w || x_fmt < Q36MOE_FMT_F32 || x_fmt > Q36MOE_FMT_BF16) return Q36MOE_EINVAL;
    if (T < 0 || T > kNoAllocMaxT || top_k < 1 || top_k > kMaxTopK || top_k > w->E) return Q36MOE_EINVAL;
    if (carve_scratch(nullptr, kNoAllocMaxT, w->E, w->D, w->FF, top_k, nullptr) > kNoAllocBytes)
        return Q36MOE_EINVAL;
    if (T == 0) return Q36MOE_OK;
    uint8_t *base = nullptr;
    const int rc = noalloc_scratch(&base);
    if (rc) return rc;
    Scratch S;
    carve_scratch(base, kNoAllocMaxT, w->E, w->D, w->FF, top_k, &S);
    Plan P;
    return launch_forward(S, P, 0, w, x, x_fmt, nullptr, logits, ld_logits, shg, ld_shg, T, scale, out, out_fmt,
                          static_cast<hipStream_t>(stream), nullptr);
}

int q36moe_forward_q8(q36moe_ctx *c, const q36moe_weights *w, const uint8_t *xq, const uint8_t *xs,
                      const float *logits, int ld_logits, const float *shg, int ld_shg, int T, float scale,
                      void *out, int out_fmt) {
    if (T > 0 && !xs) return Q36MOE_EINVAL;
    return forward_impl(c, w, xq, kFmtE4M3, xs, logits, ld_logits, shg, ld_shg, T, scale, out, out_fmt);
}

int q36moe_router_topk(const float *logits, int T, int n_expert, int ld, int k, float scale,
                       int renorm, int32_t *idx, float *wt, void *stream) {
    if (T < 0 || n_expert < 1 || n_expert > kMaxExperts || ld < n_expert || k < 1 ||
        k > kMaxTopK || k > n_expert)
        return Q36MOE_EINVAL;
    if (T == 0) return Q36MOE_OK;
    if (!logits || !idx || !wt) return Q36MOE_EINVAL;
    hipLaunchKernelGGL(k_topk, dim3((T + 3) / 4), dim3(256), 0, static_cast<hipStream_t>(stream),
                       logits, T, n_expert, ld, k, scale, renorm, idx, wt);
    return hip_rc(hipGetLastError());
}

int q36moe_router_logits(const float *w, int n_rows, int n_expert, const void *x, int x_fmt, int T,
                          int d_model, int mode, float *logits, int ld, float *shg, void *stream) {
    if (T < 0 || d_model != kRtD || n_expert < 1 || n_rows < n_expert || n_rows > n_expert + 1 ||
        ld < n_expert || mode < 0 || mode > 2 || (x_fmt != Q36MOE_FMT_F32 && x_fmt != Q36MOE_FMT_BF16))
        return Q36MOE_EINVAL;
    if (T == 0) return Q36MOE_OK;
    if (!w || !x || !logits || (n_rows > n_expert && !shg)) return Q36MOE_EINVAL;
    const bool f16 = mode == 2 || (mode == 0 && T > kDirectMaxT);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (f16)
        hipLaunchKernelGGL(k_router_f16, dim3((n_rows + 63) / 64, (T + 63) / 64), dim3(256), 0, s, w, n_rows,
                           n_expert, x, x_fmt, T, logits, ld, shg);
    else
        hipLaunchKernelGGL(k_router_f32, dim3(n_rows), dim3(64), 0, s, w, n_expert, x, x_fmt, T, logits, ld,
                           shg);
    return hip_rc(hipGetLastError());
}

int q36moe_add_rmsnorm_quant(float *h, const float *a, const float *w, int T, int d_model,
                             float eps, float *y, uint8_t *xq, uint8_t *xs, void *stream) {
    if (T < 0 || d_model != kRtD || !(eps >= 0.0f) || (!xq) != (!xs)) return Q36MOE_EINVAL;
    if (T == 0) return Q36MOE_OK;
    if (!h || !w || (!y && !xq)) return Q36MOE_EINVAL;
    hipLaunchKernelGGL(k_add_rmsnorm_quant, dim3(T), dim3(256), 0, static_cast<hipStream_t>(stream), h, a, w,
                       eps, y, xq, xs);
    return hip_rc(hipGetLastError());
}

int q36moe_quant_e4m3(const void *x, int x_fmt, int T, int K, uint8_t *xq, uint8_t *xs,
                      void *stream) {
    if (T < 0 || K <= 0 || K % 32 != 0 || (x_fmt != Q36MOE_FMT_F32 && x_fmt != Q36MOE_FMT_BF16))
        return Q36MOE_EINVAL;
    if (T == 0) return Q36MOE_OK;
    if (!x || !xq || !xs) return Q36MOE_EINVAL;
    const long nblk = (long)T * (K / 32);
    hipLaunchKernelGGL(k_quant, dim3((unsigned)((nblk + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), x, x_fmt, T, K, xq, xs);
    return hip_rc(hipGetLastError());
}

int q36moe_ctx_copy_tap(q36moe_ctx *c, int tap, void *dst, size_t bytes, size_t *written) {
    if (!c || !dst) return Q36MOE_EINVAL;
    const size_t T = (size_t)c->last_T, n = T * c->s.K, rows = n + (c->last_sh ? T : 0);
    const void *src = nullptr;
    size_t sz = 0;
    switch (tap) {
        case Q36MOE_TAP_TOPK_IDX: src = c->s.topk_idx; sz = n * 4; break;
        case Q36MOE_TAP_TOPK_W: src = c->s.topk_w; sz = n * 4; break;
        case Q36MOE_TAP_XQ: src = c->tap_xq; sz = T * c->s.D; break;
        case Q36MOE_TAP_XS: src = c->tap_xs; sz = T * c->s.D / 32; break;
        case Q36MOE_TAP_EOFF:
            if (c->last_path == 1) return Q36MOE_EINVAL;   // the direct path does not sort
            src = c->s.e_off; sz = (size_t)(c->s.E + 1) * 4; break;
        case Q36MOE_TAP_PERM: src = c->s.perm; sz = n * 4; break;
        case Q36MOE_TAP_POS: src = c->s.pos; sz = n * 4; break;
        case Q36MOE_TAP_HQ: src = c->s.hq; sz = rows * c->s.FF; break;
        case Q36MOE_TAP_HS: src = c->s.hs; sz = rows * c->s.FF / 32; break;
        case Q36MOE_TAP_HSF: src = c->s.hsf; sz = rows * c->s.FF / 32 * 4; break;
        case Q36MOE_TAP_XQ8:
            if (c->last_path == 1) return Q36MOE_EINVAL;   // quantised in LDS only
            src = c->s.xq8; sz = T * c->s.D; break;
        case Q36MOE_TAP_XSF:
            if (c->last_path == 1) return Q36MOE_EINVAL;
            src = c->s.xsf; sz = T * c->s.D / 32 * 4; break;
        case Q36MOE_TAP_DNW:
            if (c->last_path == 1) return Q36MOE_EINVAL;   // combined in registers
            sz = rows * c->s.D * 4;
            if (bytes < sz) return Q36MOE_EINVAL;
            if (written) *written = sz;
            hipLaunchKernelGGL(k_dn16_expand, dim3((unsigned)rows), dim3(256), 0, c->stream, c->s.dnh, c->s.dne,
                               c->s.D, static_cast<float *>(dst));
            return hip_rc(hipGetLastError());
        default: return Q36MOE_EINVAL;
    }
    if (bytes < sz) return Q36MOE_EINVAL;
    if (written) *written = sz;
    if (sz == 0) return Q36MOE_OK;
    return hip_rc(hipMemcpyAsync(dst, src, sz, hipMemcpyDeviceToDevice, c->stream));
}

int q36moe_ctx_set_path(q36moe_ctx *c, int mode) {
    if (!c || mode < 0 || mode > 5 || mode == 3) return Q36MOE_EINVAL;
    c->path_mode = mode;
    return Q36MOE_OK;
}

int q36moe_ctx_last_path(const q36moe_ctx *c) { return c ? c->last_path : Q36MOE_EINVAL; }

int q36moe_ctx_check(q36moe_ctx *c) {
    if (!c) return Q36MOE_EINVAL;
    return hip_rc(hipStreamSynchronize(c->stream));
}

int q36moe_ctx_set_timing(q36moe_ctx *c, int on) {
    if (!c) return Q36MOE_EINVAL;
    c->timing = on ? 1 : 0;
    return Q36MOE_OK;
}

int q36moe_ctx_stage_times(q36moe_ctx *c, double *ms, int *calls, int n_stages, int reset) {
    if (!c || n_stages < 0) return Q36MOE_EINVAL;
    for (int i = 0; i < n_stages && i < ST_COUNT; i++) {
        if (ms) ms[i] = c->ms[i];
        if (calls) calls[i] = c->calls[i];
    }
    if (reset)
        for (int i = 0; i < ST_COUNT; i++) {
            c->ms[i] = 0.0;
            c->calls[i] = 0;
        }
    return Q36MOE_OK;
}

const char *q36moe_stage_name(int stage) {
    return (stage >= 0 && stage < ST_COUNT) ? kStageNames[stage] : nullptr;
}

int q36moe_num_stages(void) { return ST_COUNT; }

int q36moe_probe_mfma(const void *a, const void *b, const uint32_t *sa, const uint32_t *sb,
                      int fmt_a, int fmt_b, float *c, void *stream) {
    if (!a || !b || !sa || !sb || !c || fmt_a < 0 || fmt_a > 4 || fmt_b < 0 || fmt_b > 4)
        return Q36MOE_EINVAL;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const v8i *av = static_cast<const v8i *>(a);
    const v8i *bv = static_cast<const v8i *>(b);
    v4f *cv = reinterpret_cast<v4f *>(c);
    hipError_t e;
    switch (fmt_a) {
        case 0: e = launch_probe_b<0>(fmt_b, av, bv, sa, sb, cv, s); break;
        case 1: e = launch_probe_b<1>(fmt_b, av, bv, sa, sb, cv, s); break;
        case 2: e = launch_probe_b<2>(fmt_b, av, bv, sa, sb, cv, s); break;
        case 3: e = launch_probe_b<3>(fmt_b, av, bv, sa, sb, cv, s); break;
        default: e = launch_probe_b<4>(fmt_b, av, bv, sa, sb, cv, s); break;
    }
    return hip_rc(e);
}

int q36moe_probe_mfma32(const void *a, const void *b, const uint32_t *sa, const uint32_t *sb, float *c,
                        void *stream) {
    if (!a || !b || !sa || !sb || !c) return Q36MOE_EINVAL;
    hipLaunchKernelGGL(k_probe32, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream),
                       static_cast<const v8i *>(a), static_cast<const v8i *>(b), sa, sb, reinterpret_cast<v16f *>(c));
    return hip_rc(hipGetLastError());
}

}  // extern "C"
