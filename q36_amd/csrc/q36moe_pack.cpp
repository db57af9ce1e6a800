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
