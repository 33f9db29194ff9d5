/* Float powf/sinf/cosf restating the reference's own float routines, and the
 * RoPE table built from them (see mathf.c). */
#ifndef L98_MATHF_H
#define L98_MATHF_H
#ifdef __cplusplus
extern "C" {
#endif
float l98_powf(float x, float y);
float l98_sinf(float x);
float l98_cosf(float x);
void l98_rope_table(float *cs, int seq_len, int rot, float theta);
#ifdef __cplusplus
}
#endif
#endif
