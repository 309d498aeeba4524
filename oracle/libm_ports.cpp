// Test infrastructure: the reference's ports of glibc 2.39's math routines
// (include/cuju/libm/*.h, header-only), compiled from where they lie under the reference tree by
// oracle/Makefile into oracle/_ref/liblibm_ports.so. Tests and the golden-vector script evaluate
// them over input ranges and arrays; nothing of the product links them.
//
//   float codes: 0 sinf, 1 cosf, 2 powf(x, y), 3 atan2f(x, y) (x is the numerator), 4 atanf,
//                5 acosf, 6 asinf, 7 sincosf's sine, 8 sincosf's cosine
//   double codes: 0 sin, 1 cos, 2 pow(x, y), 3 acos, 4 sincos's sine, 5 sincos's cosine
#include <cstdint>
#include <cstring>

#include "cuju/libm/acos_double.h"
#include "cuju/libm/asinf.h"
#include "cuju/libm/inverse_trigonometric_float.h"
#include "cuju/libm/pow.h"
#include "cuju/libm/powf.h"
#include "cuju/libm/sin_double.h"
#include "cuju/libm/sincos_double.h"
#include "cuju/libm/sincosf.h"

namespace {
float Float(int which, float x, float y) {
    namespace m = cuju::libm;
    switch (which) {
        case 0: return m::sinf(x);
        case 1: return m::cosf(x);
        case 2: return m::powf(x, y);
        case 3: return m::atan2f(x, y);
        case 4: return m::atanf(x);
        case 5: return m::acosf(x);
        case 6: return m::asinf(x);
        case 7: return m::sincosf(x).sine;
        default: return m::sincosf(x).cosine;
    }
}
double Double(int which, double x, double y) {
    namespace m = cuju::libm;
    double s = 0, c = 0;
    switch (which) {
        case 0: return m::sin(x);
        case 1: return m::cos(x);
        case 2: return m::pow(x, y);
        case 3: return m::acos(x);
        case 4: m::sincos(x, &s, &c); return s;
        default: m::sincos(x, &s, &c); return c;
    }
}
}  // namespace

extern "C" {
__attribute__((visibility("default"))) void oracle_libm_float_range(int which, uint32_t first, long long count, float *out) {
    for (long long i = 0; i < count; i++) {
        const uint32_t bits = first + (uint32_t)i;
        float x;
        memcpy(&x, &bits, 4);
        out[i] = Float(which, x, 0.0f);
    }
}
__attribute__((visibility("default"))) void oracle_libm_float(int which, const float *x, const float *y, float *out, long long count) {
    for (long long i = 0; i < count; i++) out[i] = Float(which, x[i], y[i]);
}
__attribute__((visibility("default"))) void oracle_libm_double(int which, const double *x, const double *y, double *out, long long count) {
    for (long long i = 0; i < count; i++) out[i] = Double(which, x[i], y[i]);
}
}
