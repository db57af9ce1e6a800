/* Exports the reference's own MXFP4 dequant (q36_dequant.cuh, compiled as C
 * straight from /root/reference by oracle/Makefile) so tests can check the
 * oracle's restatement against it.  TEST INFRASTRUCTURE ONLY; the output
 * goes to oracle/_ref/ and is never part of the product. */
#include "q36.h"
#include "q36_dequant.cuh"

void ref_deq_mxfp4(const uint8_t *blk17, float *out32) {
    q36_deq_mxfp4((const block_mxfp4 *)blk17, out32);
}
float ref_e8m0_half(uint8_t e) { return q36_e8m0_half(e); }
void ref_deq_row_mxfp4(const uint8_t *blocks, int n, float *out) {
    q36_deq_row(Q36_GGML_MXFP4, blocks, n, out);
}
int ref_sizeof_block_mxfp4(void) { return (int)sizeof(block_mxfp4); }
/* any type q36_deq_row handles (Q8_0, MXFP4, Q5_K, Q6_K, F32) */
void ref_deq_row(uint32_t type, const void *blocks, int n, float *out) {
    q36_deq_row(type, blocks, n, out);
}
float ref_fp16(uint16_t h) { return q36_fp16(h); }
