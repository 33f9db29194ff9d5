/* Test-only translation unit: exports two functions that are static in the
 * reference, subn_fwht_quant and subn_rot_f32 (src/forward_kda.c:43-135), so
 * the oracle's restatement of them can be checked bit for bit.  It compiles
 * the reference's forward_kda.c where it lies under the reference tree (the
 * include path, oracle/ref.mk) and adds two wrappers; nothing of the
 * reference is copied.  Linked into oracle/_ref/libl98ref_subn.so with the
 * reference's other objects in place of forward_kda.o.  Never part of the
 * product. */
#include "forward_kda.c"

void l98ref_subn_fwht_quant(const float *x, int n, int blk, int gw, int8_t *q, float *s) {
    /* the fixed-point scratch: the scaled row, then its transform */
    int32_t *scr = (int32_t *)malloc(sizeof(int32_t) * 2 * (size_t)n);
    if (!scr) return;
    subn_fwht_quant(x, n, blk, gw, q, s, scr);
    free(scr);
}

void l98ref_subn_rot_f32(float *x, int n, int blk) { subn_rot_f32(x, n, blk); }
