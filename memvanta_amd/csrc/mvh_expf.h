/*
 * mvh_expf.h -- binary32 exp computed exactly as the host C library's expf
 * (glibc 2.35, x86-64, FMA code path), which the reference calls through
 * std::exp(float) in its softmax and SwiGLU (src/llama_model.cpp:248,249,256,257).
 *
 * Method (the published table-driven algorithm glibc uses): in double
 * precision, x*32/ln2 = k + r with round-to-nearest k (via the 1.5*2^52 shift)
 * and |r| <= 1/2; 2^(k/32) comes from a 32-entry table of 2^(i/32) with the
 * exponent bits of k added; 2^(r/32) from a cubic; one final rounding to
 * float.  The table entries are the correctly rounded doubles of 2^(i/32)
 * minus (i << 47), derived independently; the coefficients are those of the
 * library.  A host build of this exact code agrees with glibc's expf on every
 * non-NaN binary32 input (tests/test_expf_restatement.py).
 *
 * Plain C99/C++ (host or HIP device: define MVH_EXPF_QUAL, and MVH_EXPF_TABLE
 * as a device-memory declaration, before including).
 */
#ifndef MVH_EXPF_H
#define MVH_EXPF_H
#include <stdint.h>
#include <string.h>

#ifndef MVH_EXPF_QUAL
#define MVH_EXPF_QUAL static inline
#endif

/* bits of round(2^(i/32)) - (i << 47), i = 0..31.  A table in memory: in
 * device code a switch over a lane-dependent index compiles to a branch tree
 * that a wave walks once per distinct index. */
#ifndef MVH_EXPF_TABLE
#define MVH_EXPF_TABLE static const
#endif
MVH_EXPF_TABLE uint64_t mvh_expf_table[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull,
    0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull,
    0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull,
    0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull,
    0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull,
    0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull,
    0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull,
    0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full,
    0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

MVH_EXPF_QUAL uint64_t mvh_expf_tab(uint32_t i) { return mvh_expf_table[i & 31u]; }

/* tab != NULL: the 32 entries of mvh_expf_tab (a GPU kernel keeps them in
 * LDS, so the lookup is not a global-memory round trip). */
MVH_EXPF_QUAL float mvh_expf_tabbed(float x, const uint64_t* tab) {
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    uint32_t ux;
    memcpy(&ux, &x, 4);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) { /* |x| >= 88 or nan */
        if (ux == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8u) return x + x;
        if (x > 0x1.62e42ep6f) return __builtin_inff();
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_n, xd, shift);
    uint64_t ki;
    memcpy(&ki, &kd, 8);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    uint64_t t = tab ? tab[ki % 32] : mvh_expf_tab((uint32_t)(ki % 32));
    t += ki << 47;
    double s;
    memcpy(&s, &t, 8);
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

MVH_EXPF_QUAL float mvh_expf(float x) { return mvh_expf_tabbed(x, 0); }

#endif
