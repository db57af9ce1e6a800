// Host-side repack of GGUF MXFP4 matrices into the gfx950 fragment layout.
//
// GGUF block_mxfp4 (q36.h:112-114): 17 bytes = E8M0 exponent + 16 bytes of
// nibbles; element j of the block is the low nibble of qs[j], element j+16
// the high nibble (q36_dequant.cuh:106-113).  The reference re-lays experts
// as [nibbles M*K/2][scales M*K/32] per expert (q36_engine.cu:205-227); this
// build keeps that split but orders both regions by MFMA fragment:
//
//   nibbles: tiles of 16 rows x 128 K (1024 B), tile (mt, kt) at
//            (mt*(K/128) + kt)*1024; lane L of a wave owns bytes L*16..+16 =
//            row mt*16 + L%16, K-block kb = kt*4 + L/16, packed as
//            consecutive pairs (byte j = code[2j] | code[2j+1] << 4), the
//            operand order of v_mfma_scale_f32_16x16x128_f8f6f4 for E2M1.
//   scales:  at M*K/2; byte (mt*64 + L)*(K/128) + kt is the E8M0 of that
//            same (row, K-block), so one lane reads all scales of its row
//            tile with a single contiguous K/128-byte load.
//
// A wave therefore streams 1 KB of contiguous nibbles per K-step of 128.
#include "q36moe.h"

#include <cmath>
#include <cstring>

namespace {

inline bool dims_ok(int M, int K) {
    return M > 0 && K > 0 && M % 16 == 0 && K % 512 == 0;
}

}  // namespace

extern "C" int q36moe_pack_mxfp4(const void *gguf_blocks, int M, int K, void *packed) {
    if (!gguf_blocks || !packed || !dims_ok(M, K)) return Q36MOE_EINVAL;
    const uint8_t *src = static_cast<const uint8_t *>(gguf_blocks);
    uint8_t *nib = static_cast<uint8_t *>(packed);
    uint8_t *scl = nib + (size_t)M * K / 2;
    const int nkb = K / 32, nkt = K / 128;
    int bad = 0;
    for (int r = 0; r < M; r++) {
        const int mt = r / 16, rl = r % 16;
        for (int kb = 0; kb < nkb; kb++) {
            const uint8_t *blk = src + ((size_t)r * nkb + kb) * 17;
            if (blk[0] == 255) bad = 1;
            uint8_t code[32];
            for (int j = 0; j < 16; j++) {
                code[j] = blk[1 + j] & 15;
                code[j + 16] = blk[1 + j] >> 4;
            }
            const int kt = kb / 4, lane = rl + 16 * (kb % 4);
            uint8_t *d = nib + ((size_t)mt * nkt + kt) * 1024 + (size_t)lane * 16;
            for (int j = 0; j < 16; j++) d[j] = (uint8_t)(code[2 * j] | (code[2 * j + 1] << 4));
            scl[((size_t)mt * 64 + lane) * nkt + kt] = blk[0];
        }
    }
    return bad ? Q36MOE_EINVAL : Q36MOE_OK;
}

extern "C" int q36moe_unpack_mxfp4(const void *packed, int M, int K, void *gguf_blocks) {
    if (!gguf_blocks || !packed || !dims_ok(M, K)) return Q36MOE_EINVAL;
    const uint8_t *nib = static_cast<const uint8_t *>(packed);
    const uint8_t *scl = nib + (size_t)M * K / 2;
    uint8_t *dst = static_cast<uint8_t *>(gguf_blocks);
    const int nkb = K / 32, nkt = K / 128;
    for (int r = 0; r < M; r++) {
        const int mt = r / 16, rl = r % 16;
        for (int kb = 0; kb < nkb; kb++) {
            const int kt = kb / 4, lane = rl + 16 * (kb % 4);
            const uint8_t *s = nib + ((size_t)mt * nkt + kt) * 1024 + (size_t)lane * 16;
            uint8_t code[32];
            for (int j = 0; j < 16; j++) {
                code[2 * j] = s[j] & 15;
                code[2 * j + 1] = s[j] >> 4;
            }
            uint8_t *blk = dst + ((size_t)r * nkb + kb) * 17;
            blk[0] = scl[((size_t)mt * 64 + lane) * nkt + kt];
            for (int j = 0; j < 16; j++) blk[1 + j] = (uint8_t)(code[j] | (code[j + 16] << 4));
        }
    }
    return Q36MOE_OK;
}

extern "C" size_t q36moe_expert_bytes(int d_model, int d_ff) {
    const size_t m = (size_t)d_model * d_ff;
    return 3 * (m / 2 + m / 32);
}

// ---------------------------------------------------------------------------
// q8_0-split expert matrices (the reference's requantised Q5_K / Q6_K
// experts, q36_engine.cu:229-252)
// ---------------------------------------------------------------------------
//
// Logical layout (as the reference keeps it on the device): int8 codes
// [M][K] and one f16 scale per 32 codes [M][K/32]; value = f16 * code.
//
// Packed (this build's device layout), ordered for v_mfma_i32_16x16x32_i8:
//   codes:  tiles of 16 rows x 64 K (1024 B), tile (mt, kp) at
//           (mt*(K/64) + kp)*1024; lane L owns bytes L*16..+16 = row
//           mt*16 + L%16: bytes 0-7 are K 64kp + 8(L/16)..+7 (block 2kp),
//           bytes 8-15 the same 8 K of block 2kp+1 -- the A operand of two
//           MFMAs (lane L: row L%16, K 8(L/16)..+7 of one 32-block).
//   scales: f16 at byte M*K; lane group q = L/16 of row tile mt holds the
//           scales of rows mt*16 + 4q + i (i = 0..3), the rows its MFMA
//           results cover: half ((mt*4 + q)*(K/32) + kb)*4 + i.
namespace {

inline bool q8_dims_ok(int M, int K) { return M > 0 && K > 0 && M % 16 == 0 && K % 64 == 0; }

inline float f16_to_f32(uint16_t h) {
    _Float16 v;
    std::memcpy(&v, &h, 2);
    return (float)v;
}

inline uint16_t f32_to_f16(float f) {   // round to nearest even (IEEE conversion)
    const _Float16 v = (_Float16)f;
    uint16_t h;
    std::memcpy(&h, &v, 2);
    return h;
}

// Q5_K super-block -> 256 floats.  Sub-block s (32 values) of chunk c = s/2
// reads the low (s even) or high nibble of qs[32c + l], bit s of qh[l] as
// the fifth bit, and a 6-bit scale and min packed in scales[12]: bytes 0-3
// and 4-7 hold scale/min of sub-blocks 0-3 in their low 6 bits, bytes 8-11
// the low nibbles of sub-blocks 4-7 whose top two bits sit in bits 6-7 of
// bytes 0-3 (scale) and 4-7 (min).  y = (d*scale)*q - dmin*min.
void deq_q5k(const uint8_t *b, float *y) {
    uint16_t hd, hm;
    std::memcpy(&hd, b, 2);
    std::memcpy(&hm, b + 2, 2);
    const float d = f16_to_f32(hd), dmin = f16_to_f32(hm);
    const uint8_t *sm = b + 4, *qh = b + 16, *qs = b + 48;
    for (int s = 0; s < 8; s++) {
        int sc, mn;
        if (s < 4) {
            sc = sm[s] & 63;
            mn = sm[s + 4] & 63;
        } else {
            sc = (sm[s + 4] & 15) | ((sm[s - 4] >> 6) << 4);
            mn = (sm[s + 4] >> 4) | ((sm[s] >> 6) << 4);
        }
        const float ds = d * (float)sc, ms = dmin * (float)mn;
        const uint8_t *lo = qs + 32 * (s >> 1);
        for (int l = 0; l < 32; l++) {
            const int q = ((s & 1) ? lo[l] >> 4 : lo[l] & 15) + (((qh[l] >> s) & 1) ? 16 : 0);
            const float p = ds * (float)q;   // separate multiply and subtract, no fma
            y[32 * s + l] = p - ms;
        }
    }
}

// Q6_K super-block -> 256 floats.  Value v = 128n + 32g + l: the low four
// bits are nibble g/2 of ql[64n + 32(g%2) + l], bits 4-5 are bits 2g..2g+1
// of qh[32n + l]; q - 32 scaled by d * scales[8n + 2g + l/16].
void deq_q6k(const uint8_t *b, float *y) {
    const uint8_t *ql = b, *qh = b + 128;
    const int8_t *sc = reinterpret_cast<const int8_t *>(b + 192);
    uint16_t hd;
    std::memcpy(&hd, b + 208, 2);
    const float d = f16_to_f32(hd);
    for (int v = 0; v < 256; v++) {
        const int n = v >> 7, g = (v >> 5) & 3, l = v & 31;
        const int byte = ql[64 * n + 32 * (g & 1) + l];
        const int q = ((g >> 1) ? byte >> 4 : byte & 15) | (((qh[32 * n + l] >> (2 * g)) & 3) << 4);
        const float ds = d * (float)sc[8 * n + 2 * g + l / 16];
        y[v] = ds * (float)(q - 32);
    }
}

}  // namespace

extern "C" int q36moe_requant_q8(int ggml_type, const void *src, int M, int K, int8_t *codes,
                                 uint16_t *scales) {
    if (!src || !codes || !scales || M <= 0 || K <= 0) return Q36MOE_EINVAL;
    const uint8_t *p = static_cast<const uint8_t *>(src);
    const int nkb = K / 32;
    if (ggml_type == 8) {   // Q8_0: already 32 codes + f16 scale per block
        if (K % 32) return Q36MOE_EINVAL;
        for (size_t b = 0; b < (size_t)M * nkb; b++) {
            std::memcpy(&scales[b], p + 34 * b, 2);
            std::memcpy(codes + 32 * b, p + 34 * b + 2, 32);
        }
        return Q36MOE_OK;
    }
    if ((ggml_type != 13 && ggml_type != 14) || K % 256) return Q36MOE_EINVAL;
    const size_t sb = ggml_type == 13 ? 176 : 210, row_bytes = (size_t)K / 256 * sb;
    float y[256];
    for (int r = 0; r < M; r++)
        for (int s = 0; s < K / 256; s++) {
            const uint8_t *blk = p + (size_t)r * row_bytes + s * sb;
            if (ggml_type == 13) deq_q5k(blk, y);
            else deq_q6k(blk, y);
            // per 32: d = amax/127 kept as f16, codes rint(v / d) from the
            // fp32 d, clamped to int8 (h_q8_row, q36_engine.cu:73-86)
            for (int j = 0; j < 8; j++) {
                const float *v = y + 32 * j;
                float amax = 0.0f;
                for (int i = 0; i < 32; i++) amax = std::fabs(v[i]) > amax ? std::fabs(v[i]) : amax;
                const float dq = amax / 127.0f, inv = dq != 0.0f ? 1.0f / dq : 0.0f;
                const size_t b = (size_t)r * nkb + s * 8 + j;
                scales[b] = f32_to_f16(dq);
                for (int i = 0; i < 32; i++) {
                    const long q = std::lrint(v[i] * inv);
                    codes[32 * b + i] = (int8_t)(q > 127 ? 127 : q < -128 ? -128 : q);
                }
            }
        }
    return Q36MOE_OK;
}

extern "C" int q36moe_pack_q8(const int8_t *codes, const uint16_t *scales, int M, int K, void *packed) {
    if (!codes || !scales || !packed || !q8_dims_ok(M, K)) return Q36MOE_EINVAL;
    uint8_t *cd = static_cast<uint8_t *>(packed);
    uint16_t *sd = reinterpret_cast<uint16_t *>(cd + (size_t)M * K);
    const int nkp = K / 64, nkb = K / 32;
    for (int r = 0; r < M; r++) {
        const int mt = r / 16, rl = r % 16;
        for (int kb = 0; kb < nkb; kb++) {
            const uint16_t s = scales[(size_t)r * nkb + kb];
            if ((s & 0x7c00u) == 0x7c00u) return Q36MOE_EINVAL;   // inf / NaN scale
            for (int q = 0; q < 4; q++) {
                const int lane = rl + 16 * q;
                uint8_t *d = cd + ((size_t)mt * nkp + kb / 2) * 1024 + (size_t)lane * 16 + (kb & 1) * 8;
                std::memcpy(d, codes + (size_t)r * K + 32 * kb + 8 * q, 8);
            }
            sd[(((size_t)mt * 4 + rl / 4) * nkb + kb) * 4 + rl % 4] = s;
        }
    }
    return Q36MOE_OK;
}

extern "C" int q36moe_unpack_q8(const void *packed, int M, int K, int8_t *codes, uint16_t *scales) {
    if (!codes || !scales || !packed || !q8_dims_ok(M, K)) return Q36MOE_EINVAL;
    const uint8_t *cd = static_cast<const uint8_t *>(packed);
    const uint16_t *sd = reinterpret_cast<const uint16_t *>(cd + (size_t)M * K);
    const int nkp = K / 64, nkb = K / 32;
    for (int r = 0; r < M; r++) {
        const int mt = r / 16, rl = r % 16;
        for (int kb = 0; kb < nkb; kb++) {
            for (int q = 0; q < 4; q++) {
                const int lane = rl + 16 * q;
                std::memcpy(codes + (size_t)r * K + 32 * kb + 8 * q,
                            cd + ((size_t)mt * nkp + kb / 2) * 1024 + (size_t)lane * 16 + (kb & 1) * 8, 8);
            }
            scales[(size_t)r * nkb + kb] = sd[(((size_t)mt * 4 + rl / 4) * nkb + kb) * 4 + rl % 4];
        }
    }
    return Q36MOE_OK;
}
