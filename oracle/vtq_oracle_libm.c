/*
 * vtq_oracle_libm.c -- TEST INFRASTRUCTURE (the checker; never linked into
 * the product).
 *
 * Single-precision functions of the Rust crate `libm = "0.2"` (Cargo.toml:23)
 * that the reference's forward step calls: expf (forward_quantized.rs:559,
 * :934), powf/cosf/sinf (:423-426, :438-441, :453-456) and sqrtf (:486,
 * ops/rms_norm.rs:102).  The crate is absent from /root/reference; it ports
 * the FreeBSD msun routines (e_expf.c in its musl restructuring, e_powf.c,
 * s_sinf.c / s_cosf.c with k_sinf.c, k_cosf.c, e_rem_pio2f.c,
 * k_rem_pio2.c), whose published algorithms are restated here.  Pinned as a
 * whole by the reference's PINNED_TRANSCENDENTAL BLAKE3 hash
 * (tests/transcendental_determinism.rs:14-63).
 *
 * Compiled with -ffp-contract=off: every operation is one IEEE operation in
 * the stated precision (float, or double where the algorithm uses double).
 *
 * Upstream notices.  The algorithms and their constants come from FreeBSD
 * msun by way of musl and the Rust `libm` crate, which carry these grants:
 *
 *   FreeBSD msun (e_expf.c, e_powf.c, s_sinf.c, s_cosf.c, k_sinf.c,
 *   k_cosf.c, e_rem_pio2f.c, k_rem_pio2.c):
 *     Copyright (C) 1993 by Sun Microsystems, Inc. All rights reserved.
 *     Developed at SunPro, a Sun Microsystems, Inc. business.
 *     Permission to use, copy, modify, and distribute this
 *     software is freely granted, provided that this notice
 *     is preserved.
 *   (The float versions: conversion to float by Ian Lance Taylor, Cygnus
 *   Support; optimisations by Bruce D. Evans.)
 *
 *   musl libc (the restructured expf and scalbnf), MIT licence:
 *     Copyright (c) 2005-2020 Rich Felker, et al.
 *     Permission is hereby granted, free of charge, to any person obtaining
 *     a copy of this software and associated documentation files (the
 *     "Software"), to deal in the Software without restriction, including
 *     without limitation the rights to use, copy, modify, merge, publish,
 *     distribute, sublicense, and/or sell copies of the Software, and to
 *     permit persons to whom the Software is furnished to do so, subject to
 *     the following conditions:
 *     The above copyright notice and this permission notice shall be
 *     included in all copies or substantial portions of the Software.
 *     THE SOFTWARE IS PROVIDED "AS IS", WITHOUT WARRANTY OF ANY KIND,
 *     EXPRESS OR IMPLIED, INCLUDING BUT NOT LIMITED TO THE WARRANTIES OF
 *     MERCHANTABILITY, FITNESS FOR A PARTICULAR PURPOSE AND NONINFRINGEMENT.
 *     IN NO EVENT SHALL THE AUTHORS OR COPYRIGHT HOLDERS BE LIABLE FOR ANY
 *     CLAIM, DAMAGES OR OTHER LIABILITY, WHETHER IN AN ACTION OF CONTRACT,
 *     TORT OR OTHERWISE, ARISING FROM, OUT OF OR IN CONNECTION WITH THE
 *     SOFTWARE OR THE USE OR OTHER DEALINGS IN THE SOFTWARE.
 *
 *   The Rust `libm` crate (the port the reference calls) is distributed
 *   under the MIT licence above (Copyright (c) 2018 Jorge Aparicio) or
 *   Apache-2.0.
 */
#include "vtq_oracle_e2e.h"

#include <math.h>
#include <string.h>

static uint32_t fbits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static float bitsf(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static double bitsd(uint64_t u) {
    double d;
    memcpy(&d, &u, 8);
    return d;
}

/* x * 2^n with the musl splitting of large |n| (scalbnf.c). */
static float scalbnf_(float x, int n) {
    if (n > 127) {
        x *= 0x1p127f;
        n -= 127;
        if (n > 127) {
            x *= 0x1p127f;
            n -= 127;
            if (n > 127) n = 127;
        }
    } else if (n < -126) {
        x *= 0x1p-126f * 0x1p24f;
        n += 126 - 24;
        if (n < -126) {
            x *= 0x1p-126f * 0x1p24f;
            n += 126 - 24;
            if (n < -126) n = -126;
        }
    }
    return x * bitsf((uint32_t)(0x7f + n) << 23);
}

static double scalbn_(double x, int n) {
    if (n > 1023) {
        x *= 0x1p1023;
        n -= 1023;
        if (n > 1023) {
            x *= 0x1p1023;
            n -= 1023;
            if (n > 1023) n = 1023;
        }
    } else if (n < -1022) {
        x *= 0x1p-1022 * 0x1p53;
        n += 1022 - 53;
        if (n < -1022) {
            x *= 0x1p-1022 * 0x1p53;
            n += 1022 - 53;
            if (n < -1022) n = -1022;
        }
    }
    return x * bitsd((uint64_t)(0x3ff + n) << 52);
}

/* ---- expf: k = round(x/ln2), r = x - k*ln2 (hi/lo), rational
 * approximation of exp(r) on [-ln2/2, ln2/2], scaled by 2^k. ---- */
float vtqo_expf(float x) {
    const float half[2] = {0.5f, -0.5f};
    const float ln2hi = bitsf(0x3f317200), ln2lo = bitsf(0x35bfbe8e), invln2 = bitsf(0x3fb8aa3b);
    const float P1 = bitsf(0x3e2aaa8f), P2 = bitsf(0xbb355215);
    uint32_t hx = fbits(x);
    const int sign = (int)(hx >> 31);
    hx &= 0x7fffffff;
    if (hx >= 0x42aeac50) {       /* |x| >= 87.33655 or NaN */
        if (hx > 0x7f800000) return x;
        if (hx >= 0x42b17218 && !sign) return x * 0x1p127f;  /* overflow */
        if (sign && hx >= 0x42cff1b5) return 0.0f;          /* x <= -103.972084 */
    }
    int k;
    float hi, lo;
    if (hx > 0x3eb17218) {        /* |x| > ln2/2 */
        if (hx > 0x3f851592)      /* |x| > 1.5 ln2 */
            k = (int)(invln2 * x + half[sign]);
        else
            k = 1 - sign - sign;
        const float kf = (float)k;
        hi = x - kf * ln2hi;
        lo = kf * ln2lo;
        x = hi - lo;
    } else if (hx > 0x39000000) { /* |x| > 2^-14 */
        k = 0;
        hi = x;
        lo = 0.0f;
    } else {
        return 1.0f + x;
    }
    const float xx = x * x;
    const float c = x - xx * (P1 + xx * P2);
    const float y = 1.0f + (x * c / (2.0f - c) - lo + hi);
    return k == 0 ? y : scalbnf_(y, k);
}

float vtqo_sqrtf(float x) { return sqrtf(x); }

/* ---- powf: log2|x| in extra precision (split into 12-bit heads and tails),
 * times y, then 2^(result) by a rational approximation. ---- */
float vtqo_powf(float x, float y) {
    const float bp[2] = {1.0f, 1.5f};
    const float dp_h[2] = {0.0f, bitsf(0x3f15c000)};
    const float dp_l[2] = {0.0f, bitsf(0x35d1cfdc)};
    const float two24 = bitsf(0x4b800000), huge = 1.0e30f, tiny = 1.0e-30f;
    const float L1 = bitsf(0x3f19999a), L2 = bitsf(0x3edb6db7), L3 = bitsf(0x3eaaaaab), L4 = bitsf(0x3e8ba305),
                L5 = bitsf(0x3e6c3255), L6 = bitsf(0x3e53f142);
    const float P1 = bitsf(0x3e2aaaab), P2 = bitsf(0xbb360b61), P3 = bitsf(0x388ab355), P4 = bitsf(0xb5ddea0e),
                P5 = bitsf(0x3331bb4c);
    const float lg2 = bitsf(0x3f317218), lg2_h = bitsf(0x3f317200), lg2_l = bitsf(0x35bfbe8c);
    const float ovt = 4.2995665694e-08f;
    const float cp = bitsf(0x3f76384f), cp_h = bitsf(0x3f764000), cp_l = bitsf(0xb8f623c6);
    const float ivln2 = bitsf(0x3fb8aa3b), ivln2_h = bitsf(0x3fb8aa00), ivln2_l = bitsf(0x36eca570);

    float z, ax, z_h, z_l, p_h, p_l, y1, t1, t2, r, s, sn, t, u, v, w;
    int32_t i, j, k, yisint, n, is;
    const int32_t hx = (int32_t)fbits(x), hy = (int32_t)fbits(y);
    int32_t ix = hx & 0x7fffffff;
    const int32_t iy = hy & 0x7fffffff;

    if (iy == 0) return 1.0f;                        /* x**0 = 1, even if x is NaN */
    if (hx == 0x3f800000) return 1.0f;               /* 1**y = 1, even if y is NaN */
    if (ix > 0x7f800000 || iy > 0x7f800000) return x + y;

    /* yisint: 0 not an integer, 1 odd, 2 even (only needed for x < 0) */
    yisint = 0;
    if (hx < 0) {
        if (iy >= 0x4b800000) {
            yisint = 2;
        } else if (iy >= 0x3f800000) {
            k = (iy >> 23) - 0x7f;
            j = iy >> (23 - k);
            if ((j << (23 - k)) == iy) yisint = 2 - (j & 1);
        }
    }
    if (iy == 0x7f800000) {  /* y = +-inf */
        if (ix == 0x3f800000) return 1.0f;
        if (ix > 0x3f800000) return hy >= 0 ? y : 0.0f;
        return hy >= 0 ? 0.0f : -y;
    }
    if (iy == 0x3f800000) return hy >= 0 ? x : 1.0f / x;  /* y = +-1 */
    if (hy == 0x40000000) return x * x;                   /* y = 2 */
    if (hy == 0x3f000000 && hx >= 0) return sqrtf(x);     /* y = 0.5 */

    ax = fabsf(x);
    if (ix == 0x7f800000 || ix == 0 || ix == 0x3f800000) {  /* x = +-0, +-inf, +-1 */
        z = ax;
        if (hy < 0) z = 1.0f / z;
        if (hx < 0) {
            if (((ix - 0x3f800000) | yisint) == 0)
                z = (z - z) / (z - z);
            else if (yisint == 1)
                z = -z;
        }
        return z;
    }
    sn = 1.0f;
    if (hx < 0) {
        if (yisint == 0) return (x - x) / (x - x);
        if (yisint == 1) sn = -1.0f;
    }

    if (iy > 0x4d000000) {  /* |y| > 2^27 */
        if (ix < 0x3f7ffff8) return hy < 0 ? sn * huge * huge : sn * tiny * tiny;
        if (ix > 0x3f800007) return hy > 0 ? sn * huge * huge : sn * tiny * tiny;
        t = ax - 1.0f;
        w = (t * t) * (0.5f - t * (0.333333333333f - t * 0.25f));
        u = ivln2_h * t;
        v = t * ivln2_l - w * ivln2;
        t1 = u + v;
        is = (int32_t)fbits(t1);
        t1 = bitsf((uint32_t)is & 0xfffff000u);
        t2 = v - (t1 - u);
    } else {
        float s2, s_h, s_l, t_h, t_l;
        n = 0;
        if (ix < 0x00800000) {  /* subnormal x */
            ax *= two24;
            n -= 24;
            ix = (int32_t)fbits(ax);
        }
        n += (ix >> 23) - 0x7f;
        j = ix & 0x007fffff;
        ix = j | 0x3f800000;
        if (j <= 0x1cc471) {
            k = 0;  /* |x| < sqrt(3/2) */
        } else if (j < 0x5db3d7) {
            k = 1;  /* |x| < sqrt(3) */
        } else {
            k = 0;
            n += 1;
            ix -= 0x00800000;
        }
        ax = bitsf((uint32_t)ix);
        /* s = (x-1)/(x+1) or (x-1.5)/(x+1.5), as s_h + s_l */
        u = ax - bp[k];
        v = 1.0f / (ax + bp[k]);
        s = u * v;
        s_h = bitsf(fbits(s) & 0xfffff000u);
        is = (int32_t)((((uint32_t)ix >> 1) & 0xfffff000u) | 0x20000000u);
        t_h = bitsf((uint32_t)is + 0x00400000u + ((uint32_t)k << 21));
        t_l = ax - (t_h - bp[k]);
        s_l = v * ((u - s_h * t_h) - s_h * t_l);
        /* log(ax) */
        s2 = s * s;
        r = s2 * s2 * (L1 + s2 * (L2 + s2 * (L3 + s2 * (L4 + s2 * (L5 + s2 * L6)))));
        r += s_l * (s_h + s);
        s2 = s_h * s_h;
        t_h = 3.0f + s2 + r;
        t_h = bitsf(fbits(t_h) & 0xfffff000u);
        t_l = r - ((t_h - 3.0f) - s2);
        u = s_h * t_h;
        v = s_l * t_h + t_l * s;
        p_h = u + v;
        p_h = bitsf(fbits(p_h) & 0xfffff000u);
        p_l = v - (p_h - u);
        z_h = cp_h * p_h;
        z_l = cp_l * p_h + p_l * cp + dp_l[k];
        t = (float)n;
        t1 = ((z_h + z_l) + dp_h[k]) + t;
        t1 = bitsf(fbits(t1) & 0xfffff000u);
        t2 = z_l - (((t1 - t) - dp_h[k]) - z_h);
    }

    /* (y1 + y2) * (t1 + t2) */
    y1 = bitsf(fbits(y) & 0xfffff000u);
    p_l = (y - y1) * t1 + y * t2;
    p_h = y1 * t1;
    z = p_l + p_h;
    j = (int32_t)fbits(z);
    if (j > 0x43000000) {  /* z > 128 */
        return sn * huge * huge;
    } else if (j == 0x43000000) {
        if (p_l + ovt > z - p_h) return sn * huge * huge;
    } else if ((j & 0x7fffffff) > 0x43160000) {  /* z < -150 */
        return sn * tiny * tiny;
    } else if ((uint32_t)j == 0xc3160000u && p_l <= z - p_h) {
        return sn * tiny * tiny;
    }

    /* 2^(p_h + p_l) */
    i = j & 0x7fffffff;
    k = (i >> 23) - 0x7f;
    n = 0;
    if (i > 0x3f000000) {  /* |z| > 0.5: n = [z + 0.5] */
        n = j + (0x00800000 >> (k + 1));
        k = ((n & 0x7fffffff) >> 23) - 0x7f;
        t = bitsf((uint32_t)n & ~(0x007fffffu >> k));
        n = ((n & 0x007fffff) | 0x00800000) >> (23 - k);
        if (j < 0) n = -n;
        p_h -= t;
    }
    t = p_l + p_h;
    t = bitsf(fbits(t) & 0xffff8000u);
    u = t * lg2_h;
    v = (p_l - (t - p_h)) * lg2 + t * lg2_l;
    z = u + v;
    w = v - (z - u);
    t = z * z;
    t1 = z - t * (P1 + t * (P2 + t * (P3 + t * (P4 + t * P5))));
    r = (z * t1) / (t1 - 2.0f) - (w + z * w);
    z = 1.0f - (r - z);
    j = (int32_t)fbits(z);
    j += (int32_t)((uint32_t)n << 23);
    if ((j >> 23) <= 0)
        z = scalbnf_(z, n);
    else
        z = bitsf((uint32_t)j);
    return sn * z;
}

/* ---- sin/cos kernels on [-pi/4, pi/4] in double ---- */
static float sindf_(double x) {
    const double S1 = bitsd(0xbfc5555554cbac77ull), S2 = bitsd(0x3f811110896efbb2ull),
                 S3 = bitsd(0xbf2a00f9e2cae774ull), S4 = bitsd(0x3ec6cd878c3b46a7ull);
    const double z = x * x, w = z * z, r = S3 + z * S4, s = z * x;
    return (float)((x + s * (S1 + z * S2)) + s * w * r);
}
static float cosdf_(double x) {
    const double C0 = bitsd(0xbfdffffffd0c5e81ull), C1 = bitsd(0x3fa55553e1053a42ull),
                 C2 = bitsd(0xbf56c087e80f1e27ull), C3 = bitsd(0x3ef99342e0ee5069ull);
    const double z = x * x, w = z * z, r = C2 + z * C3;
    return (float)(((1.0 + z * C0) + w * C1) + (w * z) * r);
}

/* Payne-Hanek reduction for huge arguments (k_rem_pio2.c), single input
 * word, precision 0 (24 bits): only what rem_pio2f's large path needs. */
static const int32_t ipio2_[] = {0xA2F983, 0x6E4E44, 0x1529FC, 0x2757D1, 0xF534DD, 0xC0DB62, 0x95993C,
                                 0x439041, 0xFE5163, 0xABDEBB, 0xC561B7, 0x246E3A, 0x424DD2, 0xE00649,
                                 0x2EEA09, 0xD1921C, 0xFE1DEB, 0x1CB129, 0xA73EE8, 0x8235F5, 0x2EBB44,
                                 0x84E99C, 0x7026B4, 0x5F7E41, 0x3991D6, 0x398353, 0x39F49C, 0x845F8B,
                                 0xBDF928, 0x3B1FF8, 0x97FFDE, 0x05980F, 0xEF2F11, 0x8B5A0A, 0x6D1F6D,
                                 0x367ECF, 0x27CB09, 0xB74F46, 0x3F669E, 0x5FEA2D, 0x7527BA, 0xC7EBE5,
                                 0xF17B3D, 0x0739F7, 0x8A5292, 0xEA6BFB, 0x5FB11F, 0x8D5D08, 0x560330,
                                 0x46FC7B, 0x6BABF0, 0xCFBC20, 0x9AF436, 0x1DA9E3, 0x91615E, 0xE61B08,
                                 0x659985, 0x5F14A0, 0x68408D, 0xFFD880, 0x4D7327, 0x310606, 0x1556CA,
                                 0x73A8C9, 0x60E27B, 0xC08C6B};
static const uint64_t pio2_bits_[] = {0x3FF921FB40000000ull, 0x3E74442D00000000ull, 0x3CF8469880000000ull,
                                      0x3B78CC5160000000ull, 0x39F01B8380000000ull, 0x387A252040000000ull,
                                      0x36E3822280000000ull, 0x3569F31D00000000ull};

static int rem_pio2_large_(const double* x, double* y, int e0) {
    const int jk = 3, jp = 3, jx = 0;  /* prec 0, one input word */
    int32_t jz, jv, carry, n, iq[20], i, j, k, m, q0, ih;
    double z, fw, f[20], fq[20], q[20];
    double PIo2[8];
    for (i = 0; i < 8; i++) PIo2[i] = bitsd(pio2_bits_[i]);

    jv = (e0 - 3) / 24;
    if (jv < 0) jv = 0;
    q0 = e0 - 24 * (jv + 1);
    j = jv - jx;
    m = jx + jk;
    for (i = 0; i <= m; i++, j++) f[i] = j < 0 ? 0.0 : (double)ipio2_[j];
    for (i = 0; i <= jk; i++) {
        for (j = 0, fw = 0.0; j <= jx; j++) fw += x[j] * f[jx + i - j];
        q[i] = fw;
    }
    jz = jk;
recompute:
    for (i = 0, j = jz, z = q[jz]; j > 0; i++, j--) {
        fw = (double)(int32_t)(0x1p-24 * z);
        iq[i] = (int32_t)(z - 0x1p24 * fw);
        z = q[j - 1] + fw;
    }
    z = scalbn_(z, q0);
    z -= 8.0 * floor(z * 0.125);
    n = (int32_t)z;
    z -= (double)n;
    ih = 0;
    if (q0 > 0) {
        i = iq[jz - 1] >> (24 - q0);
        n += i;
        iq[jz - 1] -= i << (24 - q0);
        ih = iq[jz - 1] >> (23 - q0);
    } else if (q0 == 0) {
        ih = iq[jz - 1] >> 23;
    } else if (z >= 0.5) {
        ih = 2;
    }
    if (ih > 0) {
        n += 1;
        carry = 0;
        for (i = 0; i < jz; i++) {
            j = iq[i];
            if (carry == 0) {
                if (j != 0) {
                    carry = 1;
                    iq[i] = 0x1000000 - j;
                }
            } else {
                iq[i] = 0xffffff - j;
            }
        }
        if (q0 > 0) {
            switch (q0) {
            case 1: iq[jz - 1] &= 0x7fffff; break;
            case 2: iq[jz - 1] &= 0x3fffff; break;
            }
        }
        if (ih == 2) {
            z = 1.0 - z;
            if (carry != 0) z -= scalbn_(1.0, q0);
        }
    }
    if (z == 0) {
        j = 0;
        for (i = jz - 1; i >= jk; i--) j |= iq[i];
        if (j == 0) {
            for (k = 1; iq[jk - k] == 0; k++) {
            }
            for (i = jz + 1; i <= jz + k; i++) {
                f[jx + i] = (double)ipio2_[jv + i];
                for (j = 0, fw = 0.0; j <= jx; j++) fw += x[j] * f[jx + i - j];
                q[i] = fw;
            }
            jz += k;
            goto recompute;
        }
    }
    if (z == 0.0) {
        jz -= 1;
        q0 -= 24;
        while (iq[jz] == 0) {
            jz--;
            q0 -= 24;
        }
    } else {
        z = scalbn_(z, -q0);
        if (z >= 0x1p24) {
            fw = (double)(int32_t)(0x1p-24 * z);
            iq[jz] = (int32_t)(z - 0x1p24 * fw);
            jz += 1;
            q0 += 24;
            iq[jz] = (int32_t)fw;
        } else {
            iq[jz] = (int32_t)z;
        }
    }
    fw = scalbn_(1.0, q0);
    for (i = jz; i >= 0; i--) {
        q[i] = fw * (double)iq[i];
        fw *= 0x1p-24;
    }
    for (i = jz; i >= 0; i--) {
        for (fw = 0.0, k = 0; k <= jp && k <= jz - i; k++) fw += PIo2[k] * q[i + k];
        fq[jz - i] = fw;
    }
    fw = 0.0;
    for (i = jz; i >= 0; i--) fw += fq[i];
    y[0] = ih == 0 ? fw : -fw;
    return n & 7;
}

/* x = n*pi/2 + y, |y| <~ pi/4 (e_rem_pio2f.c, round-to-nearest form) */
static int rem_pio2f_(float x, double* y) {
    const double toint = 1.5 / 2.22044604925031308085e-16;
    const double invpio2 = bitsd(0x3FE45F306DC9C883ull), pio2_1 = bitsd(0x3FF921FB50000000ull),
                 pio2_1t = bitsd(0x3E5110B4611A6263ull);
    const uint32_t ix = fbits(x) & 0x7fffffff;
    if (ix < 0x4dc90fdb) {  /* |x| ~< 2^28 * pi/2 */
        const double fn = (double)x * invpio2 + toint - toint;
        *y = (double)x - fn * pio2_1 - fn * pio2_1t;
        return (int32_t)fn;
    }
    if (ix >= 0x7f800000) {
        *y = (double)(x - x);
        return 0;
    }
    const int sign = (int)(fbits(x) >> 31);
    const int e0 = (int)(ix >> 23) - (0x7f + 23);
    const double tx = (double)bitsf(ix - ((uint32_t)e0 << 23));
    double ty;
    const int n = rem_pio2_large_(&tx, &ty, e0);
    if (sign) {
        *y = -ty;
        return -n;
    }
    *y = ty;
    return n;
}

static const uint64_t pio2m_[4] = {0x3FF921FB54442D18ull, 0x400921FB54442D18ull, 0x4012D97C7F3321D2ull,
                                   0x401921FB54442D18ull};

float vtqo_sinf(float x) {
    const double s1 = bitsd(pio2m_[0]), s2 = bitsd(pio2m_[1]), s3 = bitsd(pio2m_[2]), s4 = bitsd(pio2m_[3]);
    const double xd = (double)x;
    uint32_t ix = fbits(x);
    const int sign = (int)(ix >> 31);
    ix &= 0x7fffffff;
    if (ix <= 0x3f490fda) {       /* |x| ~<= pi/4 */
        if (ix < 0x39800000) return x;  /* |x| < 2^-12 */
        return sindf_(xd);
    }
    if (ix <= 0x407b53d1) {       /* |x| ~<= 5pi/4 */
        if (ix <= 0x4016cbe3) {   /* |x| ~<= 3pi/4 */
            if (sign) return -cosdf_(xd + s1);
            return cosdf_(xd - s1);
        }
        return sindf_(sign ? -(xd + s2) : -(xd - s2));
    }
    if (ix <= 0x40e231d5) {       /* |x| ~<= 9pi/4 */
        if (ix <= 0x40afeddf) {   /* |x| ~<= 7pi/4 */
            if (sign) return cosdf_(xd + s3);
            return -cosdf_(xd - s3);
        }
        return sindf_(sign ? xd + s4 : xd - s4);
    }
    if (ix >= 0x7f800000) return x - x;
    double y;
    const int n = rem_pio2f_(x, &y);
    switch (n & 3) {
    case 0: return sindf_(y);
    case 1: return cosdf_(y);
    case 2: return sindf_(-y);
    default: return -cosdf_(y);
    }
}

float vtqo_cosf(float x) {
    const double c1 = bitsd(pio2m_[0]), c2 = bitsd(pio2m_[1]), c3 = bitsd(pio2m_[2]), c4 = bitsd(pio2m_[3]);
    const double xd = (double)x;
    uint32_t ix = fbits(x);
    const int sign = (int)(ix >> 31);
    ix &= 0x7fffffff;
    if (ix <= 0x3f490fda) {       /* |x| ~<= pi/4 */
        if (ix < 0x39800000) return 1.0f;  /* |x| < 2^-12 */
        return cosdf_(xd);
    }
    if (ix <= 0x407b53d1) {       /* |x| ~<= 5pi/4 */
        if (ix > 0x4016cbe3)      /* |x| ~> 3pi/4 */
            return -cosdf_(sign ? xd + c2 : xd - c2);
        if (sign) return sindf_(xd + c1);
        return sindf_(c1 - xd);
    }
    if (ix <= 0x40e231d5) {       /* |x| ~<= 9pi/4 */
        if (ix > 0x40afeddf)      /* |x| ~> 7pi/4 */
            return cosdf_(sign ? xd + c4 : xd - c4);
        if (sign) return sindf_(-xd - c3);
        return sindf_(xd - c3);
    }
    if (ix >= 0x7f800000) return x - x;
    double y;
    const int n = rem_pio2f_(x, &y);
    switch (n & 3) {
    case 0: return cosdf_(y);
    case 1: return sindf_(-y);
    case 2: return -cosdf_(y);
    default: return sindf_(y);
    }
}
