// Compilation model of the engine: every simulation function is compiled for gfx950 (the product,
// one wave64 per match) and for the host (a diff tool for tests). Floating point follows IEEE 754
// with no contraction (-ffp-contract=off), correctly rounded division and square root, and
// subnormals kept; any other mode changes the bits the match depends on.
#pragma once

#include <cstdint>
#include <cstring>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#endif

#if defined(__FAST_MATH__)
#error "the engine needs IEEE 754 semantics, without fast math"
#endif

#if defined(__HIPCC__)
#define HD __host__ __device__ inline
#define HDN __host__ __device__ __attribute__((noinline)) inline
#else
#define HD inline
#define HDN inline
#endif

#if defined(__HIP_DEVICE_COMPILE__)
#define ENG_DEVICE 1
// Read-only numeric data: one copy in device global memory (the scalar cache serves it).
#define CUJU_DATA(T, name, n) __device__ static const T name[n]
#else
#define ENG_DEVICE 0
#define CUJU_DATA(T, name, n) static const T name[n]
#endif

// A timing hook at the top of each stage of the tick (`ENG_SCOPE(stage number)`). It expands to
// nothing unless a profiling build defines it before this header.
#ifndef ENG_SCOPE
#define ENG_SCOPE(stage)
#endif

namespace eng {

// A path GRF leaves undefined. The host aborts the call with an exception; the device raises the
// match's error word and the batch reports it at the next synchronization.
HD void Unsupported(const char *reason);

HD uint32_t BitsOf(float v) {
    uint32_t b;
    memcpy(&b, &v, 4);
    return b;
}
HD bool SignBit(float v) { return (BitsOf(v) >> 31) != 0; }
HD float FloatOf(uint32_t b) {
    float v;
    memcpy(&v, &b, 4);
    return v;
}
HD uint64_t BitsOf(double v) {
    uint64_t b;
    memcpy(&b, &v, 8);
    return b;
}
HD double DoubleOf(uint64_t b) {
    double v;
    memcpy(&v, &b, 8);
    return v;
}

// Whether `x` holds in any lane of the wavefront that executes the call (the lanes of a wavefront
// run different matches). The host runs one match at a time, so there it is `x`. Being a
// wavefront-wide operation, a call is a point where those lanes meet: none passes it before all
// have reached it.
HD bool AnyLane(bool x) {
#if ENG_DEVICE
    return __builtin_amdgcn_ballot_w64(x) != 0;
#else
    return x;
#endif
}

// x86-64 float-to-integer conversions (cvttss2si / cvttsd2si), which GRF's build performs. NaN and
// out-of-range inputs give the "integer indefinite" value where a GPU conversion would saturate.
HD int32_t TruncToInt32(float v) {
    if (!(v >= -2147483648.0f && v < 2147483648.0f)) return INT32_MIN;
    return (int32_t)v;
}
HD int32_t TruncToInt32(double v) {
    if (!(v > -2147483649.0 && v < 2147483648.0)) return INT32_MIN;
    return (int32_t)v;
}
// float -> unsigned goes through a 64-bit signed conversion on x86-64; the low word is kept.
HD uint32_t TruncToUint32(float v) {
    if (!(v >= -9223372036854775808.0f && v < 9223372036854775808.0f)) return 0u;
    return (uint32_t)(uint64_t)(int64_t)v;
}

}  // namespace eng
