/*
 * ref_q4k_decode.c -- exports the reference's own C decode header
 * (lxdde/ports/nouveau/q4k_decode.h, the twin of sosomodel::dequant that the
 * reference's CUDA kernels and its hostcheck compile) as plain symbols, so the
 * tests can check the oracle against it.  TEST INFRASTRUCTURE ONLY.
 *
 * Built by oracle/Makefile straight from /root/reference into oracle/_ref/;
 * nothing of the header is copied here.  REF_Q4K_DECODE_H is set on the
 * compiler command line to the header's path under /root/reference.
 */
#include REF_Q4K_DECODE_H

float ref_q4k_f16(unsigned short bits) { return q4k_f16(bits); }
void ref_q4k_scale_min(const unsigned char *scales, int j, unsigned char *sc, unsigned char *m)
{
    q4k_scale_min(scales, j, sc, m);
}
float ref_q4k_dot_sub(const unsigned char *blk, int j, const float *x) { return q4k_dot_sub(blk, j, x); }
float ref_q4k_dot_block(const unsigned char *blk, const float *x) { return q4k_dot_block(blk, x); }
float ref_q80_dot_block(const unsigned char *blk, const float *x) { return q80_dot_block(blk, x); }
