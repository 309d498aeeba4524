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

// ---- the lanes of one match ------------------------------------------------------------------------
// On the device a match runs on a group of kGroupLanes adjacent lanes of a wavefront. Every lane
// of the group runs the match's sequential code with the same data, so the group never diverges
// there and its loads and stores of one address merge. Loops whose iterations are independent split
// their iterations over the group ("rank" = the lane's place in it) and combine the results in
// iteration order, so a match computes exactly what one lane alone would. The host runs a match
// on one lane.
#ifndef ENG_GROUP_LANES
#define ENG_GROUP_LANES 4
#endif
#if ENG_DEVICE
constexpr int kGroupLanes = ENG_GROUP_LANES;
static_assert(kGroupLanes == 1 || kGroupLanes == 2 || kGroupLanes == 4 || kGroupLanes == 8 || kGroupLanes == 16 ||
                  kGroupLanes == 32 || kGroupLanes == 64,
              "a group is a power of two of lanes within a wavefront");
#else
constexpr int kGroupLanes = 1;
#endif
// Groups never exceed a wavefront.
constexpr int kMaxGroupLanes = 64;
// A set of the lanes of a match: bit r for the lane of rank r.
using LaneMask = uint64_t;
// The lanes of rank below r (r < 64), and of rank r and below.
HD LaneMask LanesBelow(int r) { return ((LaneMask)1 << r) - 1u; }
HD LaneMask LanesThrough(int r) { return r >= 63 ? ~(LaneMask)0 : ((LaneMask)1 << (r + 1)) - 1u; }

HD int LaneId() {
#if ENG_DEVICE
    return (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
#else
    return 0;
#endif
}
HD int GroupRank() { return LaneId() & (kGroupLanes - 1); }
// Bit r: `x` in the group's lane of rank r. Every lane of the group must make the call.
HD LaneMask GroupBallot(bool x) {
#if ENG_DEVICE
    const uint64_t all = __builtin_amdgcn_ballot_w64(x);
    if constexpr (kGroupLanes == 64) return all;
    else return (all >> (LaneId() & ~(kGroupLanes - 1))) & (((LaneMask)1 << kGroupLanes) - 1u);
#else
    return x ? 1u : 0u;
#endif
}
HD int PopCount(uint64_t x) {
#if ENG_DEVICE
    return __builtin_popcountll(x);
#else
    int n = 0;
    for (; x; x &= x - 1) n++;
    return n;
#endif
}
// The lowest set bit of a nonzero mask.
HD int LowestBit(uint64_t x) {
#if ENG_DEVICE
    return __builtin_ctzll(x);
#else
    int i = 0;
    while (!(x & 1u)) {
        x >>= 1;
        i++;
    }
    return i;
#endif
}
// The value of the group's lane of rank `rank`. Every lane of the group must make the call.
HD uint32_t GroupShuffle(uint32_t v, int rank) {
#if ENG_DEVICE
    const int src = (LaneId() & ~(kGroupLanes - 1)) + rank;
    return (uint32_t)__builtin_amdgcn_ds_bpermute(src << 2, (int)v);
#else
    (void)rank;
    return v;
#endif
}
HD int32_t GroupShuffle(int32_t v, int rank) { return (int32_t)GroupShuffle((uint32_t)v, rank); }
HD bool GroupShuffle(bool v, int rank) { return GroupShuffle((uint32_t)v, rank) != 0; }
HD float GroupShuffle(float v, int rank) {
    uint32_t b;
    memcpy(&b, &v, 4);
    b = GroupShuffle(b, rank);
    float r;
    memcpy(&r, &b, 4);
    return r;
}
HD double GroupShuffle(double v, int rank) {
    uint64_t b;
    memcpy(&b, &v, 8);
    const uint32_t lo = GroupShuffle((uint32_t)b, rank), hi = GroupShuffle((uint32_t)(b >> 32), rank);
    b = ((uint64_t)hi << 32) | lo;
    double r;
    memcpy(&r, &b, 8);
    return r;
}
// Orders the group's memory operations: what a lane stored before the call is what every lane of
// the group loads after it (one wavefront's memory operations complete in order).
HD void GroupSync() {
#if ENG_DEVICE
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
#endif
}
// dst[i] = src[i] for i below `count`, for arrays that do not overlap; the lanes of the match take
// `Run` entries each per round. Every lane of the match calls it; it ends synchronized.
template <int Run, class T>
HD void GroupCopy(T *dst, const T *src, int count) {
    for (int base = GroupRank() * Run; base < count; base += Run * kGroupLanes) {
        T v[Run];
        for (int j = 0; j < Run; j++)
            if (base + j < count) v[j] = src[base + j];
        for (int j = 0; j < Run; j++)
            if (base + j < count) dst[base + j] = v[j];
    }
    GroupSync();
}
// a[i] = a[i + 1] for i from 0 to count - 1, as a loop in increasing i leaves it. The lanes of the
// match copy `Run` entries each per round, every read of a round before its writes (a lane's first
// entry overwrites the last one the lane before it reads), so the reads of a round overlap in
// flight instead of following one another. Every lane of the match calls it.
template <int Run, class T>
HD void GroupShiftDown(T *a, int count) {
    for (int base = 0; base < count; base += Run * kGroupLanes) {
        const int first = base + GroupRank() * Run;
        T v[Run];
        for (int j = 0; j < Run; j++)
            if (first + j < count) v[j] = a[first + j + 1];
        GroupSync();
        for (int j = 0; j < Run; j++)
            if (first + j < count) a[first + j] = v[j];
        GroupSync();
    }
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
