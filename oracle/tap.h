/* Intermediate-value recorder for the tap build of the reference engine
 * (oracle/ref.mk target `tap`).  Test infrastructure only. */
#ifndef L98_TAP_H
#define L98_TAP_H
void l98_tap(const char *tag, int layer, const float *p, int n);
#endif
