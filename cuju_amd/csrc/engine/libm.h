// SPDX-License-Identifier: LGPL-2.1-or-later AND MIT AND SunPro
// Restates the GNU C Library 2.39's math routines: sin, cos, acos and asinf from the GNU C Library
// (Copyright (C) 2001-2024 Free Software Foundation, Inc.; Copyright (C) 1993 Sun Microsystems, Inc.;
// LGPL 2.1 or later), sinf, cosf, powf and pow from Arm Optimized Routines (Copyright (c) 2017-2020
// Arm Limited; MIT), atanf, atan2f and acosf from fdlibm (Copyright (C) 1993 Sun Microsystems, Inc.:
// Developed at SunPro, a Sun Microsystems, Inc. business. Permission to use, copy, modify, and
// distribute this software is freely granted, provided that this notice is preserved); see NOTICE.
// The math routines GRF calls, computed as glibc 2.39 computes them on x86-64 with FMA, so results
// agree to the last bit on the host and on gfx950. Each routine follows the published algorithm
// named above it; "fused" steps are the contractions of glibc's FMA build and are written as
// explicit fma, everything else is unfused. Parity with the reference ports
// (include/cuju/libm/*.h) is checked exhaustively for the unary float functions and on sampled
// and special inputs for the rest.
#pragma once

#include <cmath>

#include "hd.h"
#include "libm_data.h"

namespace eng {
namespace libm {

HD double Fma(double a, double b, double c) { return fma(a, b, c); }

// ---- sinf / cosf: Arm Optimized Routines sinf.c/cosf.c (glibc flt-32 s_sinf.c) -------------------
// Reference: include/cuju/libm/sincosf.h:61-212.

struct SinCosCoeffs {
    double sign[4];
    double hpi_inv, hpi, c0, c1, s1, c2, s2, c3, s3, c4;
};

// The tables the float routines index with a per-lane value. On the device each workgroup reads
// them from its LDS, where StageMathTables copies them before any engine code runs; the host
// reads the constant tables.
#if ENG_DEVICE
__shared__ uint64_t gLdsSinCosfCoefficients[28];
__shared__ uint64_t gLdsPowfLog2Table[32];
__shared__ uint64_t gLdsExp2fTable[32];
#endif
#if defined(__HIPCC__)
// Every thread of the workgroup calls it at the start of a kernel.
__device__ inline void StageMathTables() {
#if ENG_DEVICE
    for (int i = threadIdx.x; i < 32; i += blockDim.x) {
        gLdsPowfLog2Table[i] = kPowfLog2Table[i];
        gLdsExp2fTable[i] = kExp2fTable[i];
        if (i < 28) gLdsSinCosfCoefficients[i] = kSinCosfCoefficients[i];
    }
    __syncthreads();
#endif
}
#endif
#if ENG_DEVICE
#define LIBM_SINCOSF_TABLE gLdsSinCosfCoefficients
#define LIBM_POWF_LOG2_TABLE gLdsPowfLog2Table
#define LIBM_EXP2F_TABLE gLdsExp2fTable
#else
#define LIBM_SINCOSF_TABLE kSinCosfCoefficients
#define LIBM_POWF_LOG2_TABLE kPowfLog2Table
#define LIBM_EXP2F_TABLE kExp2fTable
#endif

HD SinCosCoeffs LoadSinCos(int set) {
    SinCosCoeffs k;
    const uint64_t *t = LIBM_SINCOSF_TABLE + 14 * set;
    k.sign[0] = DoubleOf(t[0]);
    k.sign[1] = DoubleOf(t[1]);
    k.sign[2] = DoubleOf(t[2]);
    k.sign[3] = DoubleOf(t[3]);
    k.hpi_inv = DoubleOf(t[4]);
    k.hpi = DoubleOf(t[5]);
    k.c0 = DoubleOf(t[6]);
    k.c1 = DoubleOf(t[7]);
    k.s1 = DoubleOf(t[8]);
    k.c2 = DoubleOf(t[9]);
    k.s2 = DoubleOf(t[10]);
    k.c3 = DoubleOf(t[11]);
    k.s3 = DoubleOf(t[12]);
    k.c4 = DoubleOf(t[13]);
    return k;
}

// sign[j] for j in 0..3, selected rather than indexed.
HD double SignOf(const SinCosCoeffs &k, int j) {
    return j == 0 ? k.sign[0] : j == 1 ? k.sign[1] : j == 2 ? k.sign[2] : k.sign[3];
}

// Exponent and top 3 mantissa bits of |x|.
HD uint32_t Top12f(float x) { return (BitsOf(x) >> 20) & 0x7ff; }

// |x| < 120: x - n*pi/2 with n = round(x * 2/pi) computed on a 2^24 fixed-point scale.
HD double ReduceFast(double x, const SinCosCoeffs &k, int *n) {
    double r = x * k.hpi_inv;
    int q = ((int32_t)r + 0x800000) >> 24;
    *n = q;
    return Fma(-(double)q, k.hpi, x);
}

// Payne-Hanek reduction of a finite |x| >= 120 with 4/pi held in 32-bit windows.
HDN double ReduceLarge(uint32_t xi, int *np) {
    const uint32_t *arr = &kFourOverPiBits[(xi >> 26) & 15];
    int shift = (xi >> 23) & 7;
    xi = ((xi & 0xffffff) | 0x800000) << shift;
    uint64_t r0 = (uint32_t)(xi * arr[0]);
    uint64_t r1 = (uint64_t)xi * arr[4];
    uint64_t r2 = (uint64_t)xi * arr[8];
    r0 = (r2 >> 32) | (r0 << 32);
    r0 += r1;
    uint64_t n = (r0 + (1ULL << 61)) >> 62;
    r0 -= n << 62;
    *np = (int)n;
    return (double)(int64_t)r0 * 0x1.921FB54442D18p-62;
}

// Sine polynomial for even n, cosine polynomial for odd n, on the reduced argument.
HD float SinCosPoly(double x, double x2, const SinCosCoeffs &k, int n) {
    if ((n & 1) == 0) {
        double x3 = x * x2;
        double s1 = Fma(x2, k.s3, k.s2);
        double x7 = x3 * x2;
        double s = Fma(x3, k.s1, x);
        return (float)Fma(x7, s1, s);
    }
    double x4 = x2 * x2;
    double c2 = Fma(x2, k.c4, k.c3);
    double c1 = Fma(x2, k.c1, k.c0);
    double x6 = x4 * x2;
    double c = Fma(x4, k.c2, c1);
    return (float)Fma(x6, c2, c);
}

struct SinCos {
    float s, c;
};

// Shared reduction of sinf and cosf: returns false for |x| < pi/4 (no reduction).
HD bool SinCosReduce(float y, double *xr, double *sgn, int *n, int *set) {
    uint32_t top = Top12f(y);
    *set = 0;
    if (top < Top12f(0x1.921FB6p-1f)) return false;
    SinCosCoeffs k0 = LoadSinCos(0);
    if (top < Top12f(120.0f)) {
        *xr = ReduceFast((double)y, k0, n);
        *sgn = SignOf(k0, *n & 3);
        *set = (*n & 2) ? 1 : 0;
    } else {
        uint32_t b = BitsOf(y);
        int s = b >> 31;
        *xr = ReduceLarge(b, n);
        *sgn = SignOf(k0, (*n + s) & 3);
        *set = ((*n + s) & 2) ? 1 : 0;
    }
    return true;
}

HD float sinf(float y) {
    uint32_t top = Top12f(y);
    if (top >= Top12f(INFINITY)) return (y - y) / (y - y);
    if (top < Top12f(0x1.921FB6p-1f)) {
        if (top < Top12f(0x1p-12f)) return y;
        double x = y;
        return SinCosPoly(x, x * x, LoadSinCos(0), 0);
    }
    double x, s;
    int n, set;
    SinCosReduce(y, &x, &s, &n, &set);
    return SinCosPoly(x * s, x * x, LoadSinCos(set), n);
}

HD float cosf(float y) {
    uint32_t top = Top12f(y);
    if (top >= Top12f(INFINITY)) return (y - y) / (y - y);
    if (top < Top12f(0x1.921FB6p-1f)) {
        if (top < Top12f(0x1p-12f)) return 1.0f;
        double x = y;
        return SinCosPoly(x, x * x, LoadSinCos(0), 1);
    }
    double x, s;
    int n, set;
    SinCosReduce(y, &x, &s, &n, &set);
    return SinCosPoly(x * s, x * x, LoadSinCos(set), n ^ 1);
}

// sinf and cosf of one argument sharing the reduction; each result equals the single function's.
HD SinCos sincosf(float y) {
    ENG_SCOPE(50);
    uint32_t top = Top12f(y);
    if (top >= Top12f(INFINITY)) {
        float v = (y - y) / (y - y);
        return SinCos{v, v};
    }
    if (top < Top12f(0x1.921FB6p-1f)) {
        if (top < Top12f(0x1p-12f)) return SinCos{y, 1.0f};
        double x = y;
        SinCosCoeffs k = LoadSinCos(0);
        return SinCos{SinCosPoly(x, x * x, k, 0), SinCosPoly(x, x * x, k, 1)};
    }
    double x, s;
    int n, set;
    SinCosReduce(y, &x, &s, &n, &set);
    SinCosCoeffs k = LoadSinCos(set);
    double xs = x * s, x2 = x * x;
    return SinCos{SinCosPoly(xs, x2, k, n), SinCosPoly(xs, x2, k, n ^ 1)};
}

// ---- powf: Arm Optimized Routines powf.c (glibc flt-32 e_powf.c), log2 N=16, exp2 N=32 ----------
// Reference: include/cuju/libm/powf.h:93-198.

HD double Powf_Log2(uint32_t ix) {
    uint32_t tmp = ix - 0x3f330000;
    int i = (tmp >> 19) % 16;
    uint32_t top = tmp & 0xff800000;
    uint32_t iz = ix - top;
    int k = (int32_t)top >> 23;
    double invc = DoubleOf(LIBM_POWF_LOG2_TABLE[2 * i]);
    double logc = DoubleOf(LIBM_POWF_LOG2_TABLE[2 * i + 1]);
    double z = (double)FloatOf(iz);
    double A0 = DoubleOf(kPowfLog2Poly[0]), A1 = DoubleOf(kPowfLog2Poly[1]),
           A2 = DoubleOf(kPowfLog2Poly[2]), A3 = DoubleOf(kPowfLog2Poly[3]),
           A4 = DoubleOf(kPowfLog2Poly[4]);
    double r = Fma(z, invc, -1.0);
    double y0 = logc + (double)k;
    double r2 = r * r;
    double y = Fma(A0, r, A1);
    double p = Fma(A2, r, A3);
    double r4 = r2 * r2;
    double q = Fma(A4, r, y0);
    q = Fma(p, r2, q);
    y = Fma(y, r4, q);
    return y;
}

HD float Powf_Exp2(double xd, uint32_t sign_bias) {
    const double SHIFT = 0x1.8p+52 / 32;
    double kd = xd + SHIFT;
    uint64_t ki = BitsOf(kd);
    kd -= SHIFT;
    double r = xd - kd;
    uint64_t t = LIBM_EXP2F_TABLE[ki % 32];
    uint64_t ski = ki + sign_bias;
    t += ski << (52 - 5);
    double s = DoubleOf(t);
    double C0 = DoubleOf(kExp2fPoly[0]), C1 = DoubleOf(kExp2fPoly[1]), C2 = DoubleOf(kExp2fPoly[2]);
    double z = Fma(C0, r, C1);
    double r2 = r * r;
    double y = Fma(C2, r, 1.0);
    y = Fma(z, r2, y);
    y = y * s;
    return (float)y;
}

// 0: not an integer, 1: odd integer, 2: even integer.
HD int Powf_CheckInt(uint32_t iy) {
    int e = iy >> 23 & 0xff;
    if (e < 0x7f) return 0;
    if (e > 0x7f + 23) return 2;
    if (iy & ((1u << (0x7f + 23 - e)) - 1)) return 0;
    if (iy & (1u << (0x7f + 23 - e))) return 1;
    return 2;
}
HD bool Powf_ZeroInfNan(uint32_t i) { return 2 * i - 1 >= 2u * 0x7f800000 - 1; }
HD bool SignalingF(float x) {
    uint32_t i = BitsOf(x);
    return 2 * (i ^ 0x00400000) > 2u * 0x7fc00000;
}

HD float powf(float x, float y) {
    ENG_SCOPE(49);
    uint32_t sign_bias = 0;
    uint32_t ix = BitsOf(x), iy = BitsOf(y);
    if (ix - 0x00800000 >= 0x7f800000 - 0x00800000 || Powf_ZeroInfNan(iy)) {
        if (Powf_ZeroInfNan(iy)) {
            if (2 * iy == 0) return SignalingF(x) ? x + y : 1.0f;
            if (ix == 0x3f800000) return SignalingF(y) ? x + y : 1.0f;
            if (2 * ix > 2u * 0x7f800000 || 2 * iy > 2u * 0x7f800000) return x + y;
            if (2 * ix == 2 * 0x3f800000) return 1.0f;
            if ((2 * ix < 2 * 0x3f800000) == !(iy & 0x80000000)) return 0.0f;
            return y * y;
        }
        if (Powf_ZeroInfNan(ix)) {
            float x2 = x * x;
            if ((ix & 0x80000000) && Powf_CheckInt(iy) == 1) {
                x2 = -x2;
                sign_bias = 1;
            }
            if (2 * ix == 0 && (iy & 0x80000000)) {
                float zero = 0.0f;
                return (sign_bias ? -1.0f : 1.0f) / zero;
            }
            return (iy & 0x80000000) ? 1 / x2 : x2;
        }
        if (ix & 0x80000000) {
            int yint = Powf_CheckInt(iy);
            if (yint == 0) return (x - x) / (x - x);
            if (yint == 1) sign_bias = 1u << 16;
            ix &= 0x7fffffff;
        }
        if (ix < 0x00800000) {
            ix = BitsOf(x * 0x1p23f);
            ix &= 0x7fffffff;
            ix -= 23u << 23;
        }
    }
    double logx = Powf_Log2(ix);
    double ylogx = (double)y * logx;
    if ((BitsOf(ylogx) >> 47 & 0xffff) >= BitsOf(126.0) >> 47) {
        float s = sign_bias ? -1.0f : 1.0f;
        if (ylogx > 0x1.fffffffd1d571p+6) return (s * 0x1p97f) * 0x1p97f;
        if (ylogx <= -150.0) return (s * 0x1p-95f) * 0x1p-95f;
        if (ylogx < -149.0) return (s * 0x1.4p-75f) * 0x1.4p-75f;
    }
    return Powf_Exp2(ylogx, sign_bias);
}

// powf for an exponent that is positive and not an odd integer: a base of +-0 gives 0, 1 gives 1.
HD float PowfPos(float x, float y) {
    if (x == 0.0f) return 0.0f;
    if (x == 1.0f) return 1.0f;
    return powf(x, y);
}

// ---- pow (double): Arm Optimized Routines pow.c (glibc dbl-64 e_pow.c), N=128 ---------------------
// Reference: include/cuju/libm/pow.h:447-651.

HD uint32_t Top12d(double x) { return (uint32_t)(BitsOf(x) >> 52); }

HD double Pow_Log(uint64_t ix, double *tail) {
    uint64_t tmp = ix - 0x3fe6955500000000ull;
    int i = (int)((tmp >> 45) % 128);
    int k = (int)((int64_t)tmp >> 52);
    uint64_t iz = ix - (tmp & 0xfffull << 52);
    double z = DoubleOf(iz);
    double kd = (double)k;
    double invc = DoubleOf(kPowLogTable[3 * i]);
    double logc = DoubleOf(kPowLogTable[3 * i + 1]);
    double logctail = DoubleOf(kPowLogTable[3 * i + 2]);
    const double Ln2hi = 0x1.62e42fefa3800p-1, Ln2lo = 0x1.ef35793c76730p-45;
    double A[7];
    for (int j = 0; j < 7; j++) A[j] = DoubleOf(kPowLogPoly[j]);
    double r = Fma(z, invc, -1.0);
    double t1 = Fma(kd, Ln2hi, logc);
    double t2 = t1 + r;
    double lo1 = Fma(kd, Ln2lo, logctail);
    double lo2 = t1 - t2 + r;
    double ar = A[0] * r;
    double ar2 = r * ar;
    double ar3 = r * ar2;
    double hi = t2 + ar2;
    double lo3 = Fma(ar, r, -ar2);
    double lo4 = t2 - hi + ar2;
    double p56 = Fma(r, A[6], A[5]);
    double p34 = Fma(ar2, p56, Fma(r, A[4], A[3]));
    double p12 = Fma(ar2, p34, Fma(r, A[2], A[1]));
    double lo = Fma(ar3, p12, lo1 + lo2 + lo3 + lo4);
    double y = hi + lo;
    *tail = hi - y + lo;
    return y;
}

HD double Pow_Oflow(uint32_t sign) { return (sign ? -0x1p769 : 0x1p769) * 0x1p769; }
HD double Pow_Uflow(uint32_t sign) { return (sign ? -0x1p-767 : 0x1p-767) * 0x1p-767; }

HDN double Pow_SpecialCase(double tmp, uint64_t sbits, uint64_t ki) {
    if ((ki & 0x80000000) == 0) {
        sbits -= 1009ull << 52;
        double scale = DoubleOf(sbits);
        return 0x1p1009 * Fma(scale, tmp, scale);
    }
    sbits += 1022ull << 52;
    double scale = DoubleOf(sbits);
    double st = scale * tmp;
    double y = scale + st;
    if (fabs(y) < 1.0) {
        double one = y < 0.0 ? -1.0 : 1.0;
        double lo = scale - y + st;
        double hi = one + y;
        lo = one - hi + y + lo;
        y = (hi + lo) - one;
        if (y == 0.0) y = DoubleOf(sbits & 0x8000000000000000ull);
    }
    return 0x1p-1022 * y;
}

HD double Pow_Exp(double x, double xtail, uint32_t sign_bias) {
    uint32_t abstop = Top12d(x) & 0x7ff;
    if (abstop - Top12d(0x1p-54) >= Top12d(512.0) - Top12d(0x1p-54)) {
        if (abstop - Top12d(0x1p-54) >= 0x80000000) {
            double one = 1.0 + x;
            return sign_bias ? -one : one;
        }
        if (abstop >= Top12d(1024.0)) {
            if (BitsOf(x) >> 63) return Pow_Uflow(sign_bias);
            return Pow_Oflow(sign_bias);
        }
        abstop = 0;
    }
    const double InvLn2N = 0x1.71547652b82fep0 * 128, Shift = 0x1.8p52;
    const double NegLn2hiN = -0x1.62e42fefa0000p-8, NegLn2loN = -0x1.cf79abc9e3b3ap-47;
    double kd = Fma(InvLn2N, x, Shift);
    uint64_t ki = BitsOf(kd);
    kd -= Shift;
    double r = Fma(kd, NegLn2loN, Fma(kd, NegLn2hiN, x));
    r += xtail;
    uint64_t idx = 2 * (ki % 128);
    uint64_t top = (ki + sign_bias) << 45;
    double tail = DoubleOf(kPowExpTable[idx]);
    uint64_t sbits = kPowExpTable[idx + 1] + top;
    double C0 = DoubleOf(kPowExpPoly[0]), C1 = DoubleOf(kPowExpPoly[1]),
           C2 = DoubleOf(kPowExpPoly[2]), C3 = DoubleOf(kPowExpPoly[3]);
    double r2 = r * r;
    double tmp = Fma(Fma(r, C3, C2), r2 * r2, Fma(Fma(r, C1, C0), r2, tail + r));
    if (abstop == 0) return Pow_SpecialCase(tmp, sbits, ki);
    double scale = DoubleOf(sbits);
    return Fma(scale, tmp, scale);
}

HD int Pow_CheckInt(uint64_t iy) {
    int e = iy >> 52 & 0x7ff;
    if (e < 0x3ff) return 0;
    if (e > 0x3ff + 52) return 2;
    if (iy & ((1ull << (0x3ff + 52 - e)) - 1)) return 0;
    if (iy & (1ull << (0x3ff + 52 - e))) return 1;
    return 2;
}
HD bool Pow_ZeroInfNan(uint64_t i) { return 2 * i - 1 >= 2 * BitsOf((double)INFINITY) - 1; }
HD bool SignalingD(double x) {
    uint64_t i = BitsOf(x);
    return 2 * (i ^ 0x0008000000000000ull) > 2 * 0x7ff8000000000000ull;
}

HDN double pow(double x, double y) {
    uint32_t sign_bias = 0;
    uint64_t ix = BitsOf(x), iy = BitsOf(y);
    uint32_t topx = Top12d(x), topy = Top12d(y);
    if (topx - 0x001 >= 0x7ff - 0x001 || (topy & 0x7ff) - 0x3be >= 0x43e - 0x3be) {
        if (Pow_ZeroInfNan(iy)) {
            if (2 * iy == 0) return SignalingD(x) ? x + y : 1.0;
            if (ix == BitsOf(1.0)) return SignalingD(y) ? x + y : 1.0;
            if (2 * ix > 2 * BitsOf((double)INFINITY) || 2 * iy > 2 * BitsOf((double)INFINITY))
                return x + y;
            if (2 * ix == 2 * BitsOf(1.0)) return 1.0;
            if ((2 * ix < 2 * BitsOf(1.0)) == !(iy >> 63)) return 0.0;
            return y * y;
        }
        if (Pow_ZeroInfNan(ix)) {
            double x2 = x * x;
            if ((ix >> 63) && Pow_CheckInt(iy) == 1) x2 = -x2;
            return (iy >> 63) ? 1 / x2 : x2;
        }
        if (ix >> 63) {
            int yint = Pow_CheckInt(iy);
            if (yint == 0) return (x - x) / (x - x);
            if (yint == 1) sign_bias = 0x800 << 7;
            ix &= 0x7fffffffffffffffull;
            topx &= 0x7ff;
        }
        if ((topy & 0x7ff) - 0x3be >= 0x43e - 0x3be) {
            if (ix == BitsOf(1.0)) return 1.0;
            if ((topy & 0x7ff) < 0x3be) return ix > BitsOf(1.0) ? 1.0 + y : 1.0 - y;
            return (ix > BitsOf(1.0)) == (topy < 0x800) ? Pow_Oflow(0) : Pow_Uflow(0);
        }
        if (topx == 0) {
            ix = BitsOf(x * 0x1p52);
            ix &= 0x7fffffffffffffffull;
            ix -= 52ull << 52;
        }
    }
    double lo;
    double hi = Pow_Log(ix, &lo);
    double ehi = y * hi;
    double elo = Fma(y, lo, Fma(y, hi, -ehi));
    return Pow_Exp(ehi, elo, sign_bias);
}

// ---- acosf / atanf / atan2f: FreeBSD msun e_acosf.c, s_atanf.c, e_atan2f.c (glibc thresholds) ----
// Reference: include/cuju/libm/inverse_trigonometric_float.h:32-272. Plain float arithmetic.

HD float RationalAcos(float z) {
    const float pS0 = 1.6666667163e-01f, pS1 = -3.2556581497e-01f, pS2 = 2.0121252537e-01f,
                pS3 = -4.0055535734e-02f, pS4 = 7.9153501429e-04f, pS5 = 3.4793309169e-05f,
                qS1 = -2.4033949375e+00f, qS2 = 2.0209457874e+00f, qS3 = -6.8828397989e-01f,
                qS4 = 7.7038154006e-02f;
    float p = z * (pS0 + z * (pS1 + z * (pS2 + z * (pS3 + z * (pS4 + z * pS5)))));
    float q = 1.0f + z * (qS1 + z * (qS2 + z * (qS3 + z * qS4)));
    return p / q;
}

HD float acosf(float x) {
    const float pi = 3.1415925026e+00f, pio2_hi = 1.5707962513e+00f, pio2_lo = 7.5497894159e-08f;
    int32_t hx = (int32_t)BitsOf(x), ix = hx & 0x7fffffff;
    if (ix == 0x3f800000) {
        if (hx > 0) return 0.0f;
        return pi + 2.0f * pio2_lo;
    }
    if (ix > 0x3f800000) return (x - x) / (x - x);
    if (ix < 0x3f000000) {
        if (ix <= 0x32800000) return pio2_hi + pio2_lo;
        float z = x * x;
        float r = RationalAcos(z);
        return pio2_hi - (x - (pio2_lo - x * r));
    }
    if (hx < 0) {
        float z = (1.0f + x) * 0.5f;
        float s = sqrtf(z);
        float r = RationalAcos(z);
        float w = r * s - pio2_lo;
        return pi - 2.0f * (s + w);
    }
    float z = (1.0f - x) * 0.5f;
    float s = sqrtf(z);
    float df = FloatOf(BitsOf(s) & 0xfffff000);
    float c = (z - df * df) / (s + df);
    float r = RationalAcos(z);
    float w = r * s + c;
    return 2.0f * (df + w);
}

HDN float asinf(float x);

HD float atanf(float x) {
    const float atanhi[4] = {4.6364760399e-01f, 7.8539812565e-01f, 9.8279368877e-01f,
                             1.5707962513e+00f};
    const float atanlo[4] = {5.0121582440e-09f, 3.7748947079e-08f, 3.4473217170e-08f,
                             7.5497894159e-08f};
    const float aT[11] = {3.3333334327e-01f,  -2.0000000298e-01f, 1.4285714924e-01f,
                          -1.1111110449e-01f, 9.0908870101e-02f,  -7.6918758452e-02f,
                          6.6610731184e-02f,  -5.8335702866e-02f, 4.9768779427e-02f,
                          -3.6531571299e-02f, 1.6285819933e-02f};
    int32_t hx = (int32_t)BitsOf(x), ix = hx & 0x7fffffff;
    if (ix >= 0x4c000000) {
        if (ix > 0x7f800000) return x + x;
        if (hx > 0) return atanhi[3] + atanlo[3];
        return -atanhi[3] - atanlo[3];
    }
    if (ix < 0x31000000 && 1.0e30f + x > 1.0f) return x;
    // fdlibm's four argument reductions, (2|x| - 1) / (2 + |x|), (|x| - 1) / (|x| + 1),
    // (|x| - 1.5) / (1 + 1.5|x|) and -1 / |x|, as one selected quotient: the same operations on
    // each lane, so lanes in different ranges share one division.
    const bool reduced = ix >= 0x3ee00000;
    const int id = ix < 0x3f300000 ? 0 : ix < 0x3f980000 ? 1 : ix < 0x401c0000 ? 2 : 3;
    const float ax = fabsf(x);
    const float num = id == 0 ? 2.0f * ax - 1.0f : id == 1 ? ax - 1.0f : id == 2 ? ax - 1.5f : -1.0f;
    const float den = id == 0 ? 2.0f + ax : id == 1 ? ax + 1.0f : id == 2 ? 1.0f + 1.5f * ax : ax;
    if (reduced) x = num / den;
    float z = x * x;
    float w = z * z;
    float s1 = z * (aT[0] + w * (aT[2] + w * (aT[4] + w * (aT[6] + w * (aT[8] + w * aT[10])))));
    float s2 = w * (aT[1] + w * (aT[3] + w * (aT[5] + w * (aT[7] + w * aT[9]))));
    if (!reduced) return x - x * (s1 + s2);
    const float hi = id == 0 ? atanhi[0] : id == 1 ? atanhi[1] : id == 2 ? atanhi[2] : atanhi[3];
    const float lo = id == 0 ? atanlo[0] : id == 1 ? atanlo[1] : id == 2 ? atanlo[2] : atanlo[3];
    z = hi - ((x * (s1 + s2) - lo) - x);
    return (hx < 0) ? -z : z;
}

HD float atan2f(float y, float x) {
    ENG_SCOPE(51);
    const float tiny = 1.0e-30f, pi_o_4 = 7.8539818525e-01f, pi_o_2 = 1.5707963705e+00f,
                pi = 3.1415927410e+00f, pi_lo = -8.7422776573e-08f;
    int32_t hx = (int32_t)BitsOf(x), hy = (int32_t)BitsOf(y);
    int32_t ix = hx & 0x7fffffff, iy = hy & 0x7fffffff;
    if (ix > 0x7f800000 || iy > 0x7f800000) return x + y;
    if (hx == 0x3f800000) return atanf(y);
    int m = ((hy >> 31) & 1) | ((hx >> 30) & 2);
    if (iy == 0) {
        switch (m) {
            case 0:
            case 1:
                return y;
            case 2:
                return pi + tiny;
            default:
                return -pi - tiny;
        }
    }
    if (ix == 0) return (hy < 0) ? -pi_o_2 - tiny : pi_o_2 + tiny;
    if (ix == 0x7f800000) {
        if (iy == 0x7f800000) {
            switch (m) {
                case 0:
                    return pi_o_4 + tiny;
                case 1:
                    return -pi_o_4 - tiny;
                case 2:
                    return 3.0f * pi_o_4 + tiny;
                default:
                    return -3.0f * pi_o_4 - tiny;
            }
        }
        switch (m) {
            case 0:
                return 0.0f;
            case 1:
                return -0.0f;
            case 2:
                return pi + tiny;
            default:
                return -pi - tiny;
        }
    }
    if (iy == 0x7f800000) return (hy < 0) ? -pi_o_2 - tiny : pi_o_2 + tiny;
    int32_t k = (iy - ix) >> 23;
    float z;
    if (k > 60)
        z = pi_o_2 + 0.5f * pi_lo;
    else if (hx < 0 && k < -60)
        z = 0.0f;
    else
        z = atanf(fabsf(y / x));
    // The quadrant, selected rather than branched.
    const float zl = z - pi_lo;
    return m == 0 ? z : m == 1 ? FloatOf(BitsOf(z) ^ 0x80000000u) : m == 2 ? pi - zl : zl - pi;
}

// ---- asinf: glibc 2.39 flt-32 e_asinf.c ----------------------------------------------------------
// Reference: include/cuju/libm/asinf.h:40-95.
HD float asinf(float x) {
    const float pio2_hi = 1.57079637050628662109375f, pio2_lo = -4.37113900018624283e-8f,
                pio4_hi = 0.785398185253143310546875f, p0 = 1.666675248e-1f, p1 = 7.495297643e-2f,
                p2 = 4.547037598e-2f, p3 = 2.417951451e-2f, p4 = 4.216630880e-2f;
    int32_t hx = (int32_t)BitsOf(x), ix = hx & 0x7fffffff;
    if (ix == 0x3f800000) return x * pio2_hi + x * pio2_lo;
    if (ix > 0x3f800000) return (x - x) / (x - x);
    if (ix < 0x3f000000) {
        if (ix < 0x32000000) {
            if (1.000e+30f + x > 1.0f) return x;
        } else {
            float t = x * x;
            float w = t * (p0 + t * (p1 + t * (p2 + t * (p3 + t * p4))));
            return x + x * w;
        }
    }
    float w = 1.0f - fabsf(x);
    float t = w * 0.5f;
    float p = t * (p0 + t * (p1 + t * (p2 + t * (p3 + t * p4))));
    float s = sqrtf(t);
    if (ix >= 0x3F79999A) {
        t = pio2_hi - (2.0f * (s + s * p) - pio2_lo);
    } else {
        w = FloatOf(BitsOf(s) & 0xfffff000);
        float c = (t - w * w) / (s + w);
        float r = p;
        p = 2.0f * s * r - (pio2_lo - 2.0f * c);
        float q = pio4_hi - 2.0f * w;
        t = pio4_hi - (p - q);
    }
    return hx > 0 ? t : -t;
}

// ---- sin / cos (double): glibc 2.39 dbl-64 s_sin.c (IBM), branred.c ------------------------------
// Reference: include/cuju/libm/sin_double.h:30-266.

namespace trig {
constexpr double s1 = -0x1.5555555555555p-3, s2 = 0x1.1111111110ECEp-7, s3 = -0x1.A01A019DB08B8p-13,
                 s4 = 0x1.71DE27B9A7ED9p-19, s5 = -0x1.ADDFFC2FCDF59p-26;
constexpr double big = 0x1.8000000000000p45;
constexpr double hp0 = 0x1.921FB54442D18p0, hp1 = 0x1.1A62633145C07p-54;
constexpr double mp1 = 0x1.921FB58000000p0, mp2 = -0x1.DDE973C000000p-27,
                 pp3 = -0x1.CB3B398000000p-55, pp4 = -0x1.d747f23e32ed7p-83;
constexpr double hpinv = 0x1.45F306DC9C883p-1, toint = 0x1.8000000000000p52;
constexpr double sn3 = -0x1.5555555555515p-3, sn5 = 0x1.11110e829872fp-7, cs2 = 0x1.0000000000000p-1,
                 cs4 = -0x1.5555555555535p-5, cs6 = 0x1.6c16bedd9e239p-10;
}  // namespace trig

HD int TabIndex(double u) { return (int)(uint32_t)BitsOf(u) << 2; }

HD double DoCos(double x, double dx) {
    using namespace trig;
    if (x < 0) dx = -dx;
    double u = big + fabs(x);
    x = fabs(x) - (u - big) + dx;
    double xx = x * x;
    double s = Fma(x * xx, Fma(xx, sn5, sn3), x);
    double c = xx * Fma(xx, Fma(xx, cs6, cs4), cs2);
    int k = TabIndex(u);
    double sn = DoubleOf(kSinCosTab[k]), ssn = DoubleOf(kSinCosTab[k + 1]),
           cs = DoubleOf(kSinCosTab[k + 2]), ccs = DoubleOf(kSinCosTab[k + 3]);
    double cor = Fma(-s, sn, Fma(-c, cs, Fma(-s, ssn, ccs)));
    return cs + cor;
}

HD double DoSin(double x, double dx) {
    using namespace trig;
    double xold = x;
    if (fabs(x) < 0.126) {
        double t = x * x;
        double p = Fma(t, Fma(t, Fma(t, Fma(t, s5, s4), s3), s2), s1);
        double cor = Fma(t, Fma(p, x, -(0.5 * dx)), dx);
        return x + cor;
    }
    if (x <= 0) dx = -dx;
    double u = big + fabs(x);
    x = fabs(x) - (u - big);
    double xx = x * x;
    double s = x + Fma(x * xx, Fma(xx, sn5, sn3), dx);
    double c = Fma(x, dx, xx * Fma(xx, Fma(xx, cs6, cs4), cs2));
    int k = TabIndex(u);
    double sn = DoubleOf(kSinCosTab[k]), ssn = DoubleOf(kSinCosTab[k + 1]),
           cs = DoubleOf(kSinCosTab[k + 2]), ccs = DoubleOf(kSinCosTab[k + 3]);
    double cor = Fma(s, cs, Fma(-c, sn, Fma(s, ccs, ssn)));
    return copysign(sn + cor, xold);
}

HD int ReduceSinCos(double x, double *a, double *da) {
    using namespace trig;
    double t = Fma(x, hpinv, toint);
    double xn = t - toint;
    double y = Fma(-xn, mp2, Fma(-xn, mp1, x));
    int n = (int)(uint32_t)BitsOf(t) & 3;
    double b = Fma(-xn, pp3, y);
    double db = Fma(-xn, pp3, y - b);
    double r = Fma(-xn, pp4, b);
    db = db + Fma(-xn, pp4, b - r);
    *a = r;
    *da = db;
    return n;
}

HD double DoSinCos(double a, double da, int n) {
    double r = (n & 1) ? DoCos(a, da) : DoSin(a, da);
    return (n & 2) ? -r : r;
}

// One half of branred's split argument times 2/pi, in base-2^24 digits (unfused, as glibc builds it).
HD void BranredPart(double x, double *f, double *ft, double *s) {
    const double t576 = 0x1p576, tm24 = 0x1p-24, big = 0x1.8p52, big1 = 0x1.8p54;
    double b[6], t, sum = 0, bb;
    int k = (int)((BitsOf(x) >> 52) & 2047);
    k = (k - 450) / 24;
    if (k < 0) k = 0;
    double gor = DoubleOf(BitsOf(t576) - ((uint64_t)(k * 24) << 52));
    for (int i = 0; i < 6; i++) {
        b[i] = x * DoubleOf(kTwoOverPi24[k + i]) * gor;
        gor *= tm24;
    }
    for (int i = 0; i < 3; i++) {
        t = (b[i] + big) - big;
        sum += t;
        b[i] -= t;
    }
    double s1 = 0;
    for (int i = 5; i >= 0; i--) s1 += b[i];
    bb = (((((b[0] - s1) + b[1]) + b[2]) + b[3]) + b[4]) + b[5];
    t = (s1 + big) - big;
    sum += t;
    s1 -= t;
    double b1 = s1 + bb;
    bb = (s1 - b1) + bb;
    t = (sum + big1) - big1;
    sum -= t;
    *f = b1;
    *ft = bb;
    *s = sum;
}

HDN int Branred(double x, double *a, double *aa) {
    const double tm600 = 0x1p-600, split = 134217729.0;
    const double hp0 = 0x1.921FB54442D18p0, hp1 = 0x1.1A62633145C07p-54;
    const double mp1 = 0x1.921FB58000000p0, mp2 = -0x1.DDE9740000000p-27;
    x *= tm600;
    double t = x * split;
    double x1 = t - (t - x);
    double x2 = x - x1;
    double b1, bb1, sum1, b2, bb2, sum2;
    BranredPart(x1, &b1, &bb1, &sum1);
    BranredPart(x2, &b2, &bb2, &sum2);
    double sum = sum1 + sum2;
    double b = b1 + b2;
    double bb = (fabs(b1) > fabs(b2)) ? (b1 - b) + b2 : (b2 - b) + b1;
    if (b > 0.5) {
        b -= 1.0;
        sum += 1.0;
    } else if (b < -0.5) {
        b += 1.0;
        sum -= 1.0;
    }
    double s = b + (bb + bb1 + bb2);
    t = ((b - s) + bb) + (bb1 + bb2);
    b = s * split;
    double t1 = b - (b - s);
    double t2 = s - t1;
    b = s * hp0;
    bb = (((t1 * mp1 - b) + t1 * mp2) + t2 * mp1) + ((t2 * mp2 + s * hp1) + t * hp0);
    s = b + bb;
    t = (b - s) + bb;
    *a = s;
    *aa = t;
    return ((int)sum) & 3;
}

HDN double sin(double x) {
    using namespace trig;
    int32_t k = (int32_t)(BitsOf(x) >> 32) & 0x7fffffff;
    if (k < 0x3e500000) return x;
    if (k < 0x3feb6000) return DoSin(x, 0);
    if (k < 0x400368fd) {
        double t = hp0 - fabs(x);
        return copysign(DoCos(t, hp1), x);
    }
    double a, da;
    if (k < 0x419921FB) {
        int n = ReduceSinCos(x, &a, &da);
        return DoSinCos(a, da, n);
    }
    if (k < 0x7ff00000) {
        int n = Branred(x, &a, &da);
        return DoSinCos(a, da, n);
    }
    return x / x;
}

HDN double cos(double x) {
    using namespace trig;
    int32_t k = (int32_t)(BitsOf(x) >> 32) & 0x7fffffff;
    if (k < 0x3e400000) return 1.0;
    if (k < 0x3feb6000) return DoCos(x, 0);
    if (k < 0x400368fd) {
        double y = hp0 - fabs(x);
        double a = y + hp1;
        double da = (y - a) + hp1;
        return DoSin(a, da);
    }
    double a, da;
    if (k < 0x419921FB) {
        int n = ReduceSinCos(x, &a, &da);
        return DoSinCos(a, da, n + 1);
    }
    if (k < 0x7ff00000) {
        int n = Branred(x, &a, &da);
        return DoSinCos(a, da, n + 1);
    }
    return x / x;
}

// ---- acos (double): glibc 2.39 dbl-64 e_asin.c (IBM) ---------------------------------------------
// Reference: include/cuju/libm/acos_double.h:29-143.

namespace arc {
constexpr double hp0 = 0x1.921FB54442D18p0, hp1 = 0x1.1A62633145C07p-54;
constexpr double d2 = 0x1.55555555554f9p-3, d3 = 0x1.333333336127dp-4, d4 = 0x1.6db6dae42c0e4p-5,
                 d5 = 0x1.f1c7e04f4ad99p-6, d6 = 0x1.6e442c822d419p-6, d7 = 0x1.292d80f453c72p-6;
constexpr double rt0 = 0x1.fffffffecc1ddp-1, rt1 = 0x1.fffffff757304p-2, rt2 = 0x1.800496769c91ap-2,
                 rt3 = 0x1.4006318d1dab9p-2;
constexpr double t27 = 134217728.0;
}  // namespace arc

HD double AsinSeries(double t) {
    using namespace arc;
    return Fma(Fma(Fma(Fma(Fma(t, d7, d6), t, d5), t, d4), t, d3), t, d2);
}

// Table expansions for 0.125 <= |x| < 0.96875: point, linear term, terms to `last`, a constant,
// then the arc sine of the point.
HD double AcosTable(int n, int last, double x, int32_t m) {
    using namespace arc;
    const uint64_t *T = kAsinCosTab;
    double xx = (m > 0) ? x - DoubleOf(T[n]) : -x - DoubleOf(T[n]);
    double p = DoubleOf(T[n + last]);
    for (int j = last - 1; j >= 2; j--) p = Fma(p, xx, DoubleOf(T[n + j]));
    double s = Fma(xx * xx, p, DoubleOf(T[n + last + 1]));
    double lo = Fma(DoubleOf(T[n + 1]), xx, s);
    double hi = (m > 0) ? (hp0 - DoubleOf(T[n + last + 2])) : (hp0 + DoubleOf(T[n + last + 2]));
    lo = (m > 0) ? (hp1 - lo) : (hp1 + lo);
    return hi + lo;
}

HDN double acos(double x) {
    using namespace arc;
    uint64_t bits = BitsOf(x);
    int32_t m = (int32_t)(bits >> 32);
    int32_t k = 0x7fffffff & m;
    if (k < 0x3c880000) return hp0;
    if (k < 0x3fc00000) {
        double x2 = x * x;
        double r = hp0 - x;
        double cor = Fma(-AsinSeries(x2), x * x2, ((hp0 - r) - x) + hp1);
        return r + cor;
    }
    if (k < 0x3fe00000) {
        int n = (k < 0x3fd00000) ? 11 * ((k & 0x000fffff) >> 15) : 11 * ((k & 0x000fffff) >> 14) + 352;
        return AcosTable(n, 6, x, m);
    }
    if (k < 0x3fe80000) return AcosTable(1056 + ((k & 0x000fe000) >> 11) * 3, 7, x, m);
    if (k < 0x3fed8000) return AcosTable(992 + ((k & 0x000fe000) >> 13) * 13, 8, x, m);
    if (k < 0x3fee8000) return AcosTable(884 + ((k & 0x000fe000) >> 13) * 14, 9, x, m);
    if (k < 0x3fef0000) return AcosTable(768 + ((k & 0x000fe000) >> 13) * 15, 10, x, m);
    if (k < 0x3ff00000) {
        double z = 0.5 * ((m > 0) ? (1.0 - x) : (1.0 + x));
        int32_t zw = (int32_t)(BitsOf(z) >> 32);
        // inroot seed times 2^(511 - exponent bits / 2), the power of two built directly.
        double pw = DoubleOf((uint64_t)(0x3ff + (511 - (zw >> 21))) << 52);
        double r = DoubleOf(kInverseRootSeeds[(zw & 0x001fffff) >> 14]) * pw;
        double t = Fma(-(r * r), z, 1.0);
        r = r * Fma(Fma(Fma(t, rt3, rt2), t, rt1), t, rt0);
        double c = r * z;
        double refine = Fma(-(r * 0.5), c, 1.5);
        double hi = Fma(-c, t27, Fma(c, t27, c));
        double lo = Fma(-hi, hi, z) / Fma(refine, c, hi);
        double p = AsinSeries(z) * z;
        double prod = p * (hi + lo);
        if (m < 0) {
            double cor = (hp1 - lo) - prod;
            double d = hp0 - hi;
            double res = d + cor;
            return res + res;
        }
        double cor = lo + prod;
        double res = hi + cor;
        return res + res;
    }
    if (k == 0x3ff00000 && (uint32_t)bits == 0) return (m > 0) ? 0 : 2.0 * hp0;
    return (x - x) / (x - x);
}

HD void sincos(double x, double *s, double *c) {
    *s = sin(x);
    *c = cos(x);
}

// The routines by code, for the checks of tests (the host build's debugging entry points and the
// device's): float 0 sinf, 1 cosf, 2 powf(x, y), 3 atan2f(x, y), 4 atanf, 5 acosf, 6 asinf,
// 7 and 8 the sine and cosine of sincosf; double 0 sin, 1 cos, 2 pow(x, y), 3 acos, 4 and 5 the
// sine and cosine of sincos.
HD float EvaluateFloat(int which, float x, float y) {
    switch (which) {
        case 0: return sinf(x);
        case 1: return cosf(x);
        case 2: return powf(x, y);
        case 3: return atan2f(x, y);
        case 4: return atanf(x);
        case 5: return acosf(x);
        case 6: return asinf(x);
        case 7: return sincosf(x).s;
        default: return sincosf(x).c;
    }
}
HD double EvaluateDouble(int which, double x, double y) {
    double s = 0, c = 0;
    switch (which) {
        case 0: return sin(x);
        case 1: return cos(x);
        case 2: return pow(x, y);
        case 3: return acos(x);
        case 4: sincos(x, &s, &c); return s;
        default: sincos(x, &s, &c); return c;
    }
}

}  // namespace libm
}  // namespace eng
