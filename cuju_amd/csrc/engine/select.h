// SPDX-License-Identifier: Apache-2.0
// Restates game logic of cuju (Copyright 2026 The cuju Authors), a reimplementation of Google
// Research Football (Copyright 2019 Google LLC); see NOTICE.
// Animation selection of players and officials: a crude filter over the animation table, stable
// sorts by similarity keys, and the physics plan of the chosen animation.
// Semantics: include/cuju/simulation/select_animation.h:37-2795 (every expression keeps GRF's
// operation order, precision and conversions). Candidate lists, plans and sort keys live in the
// match's Scratch block.
#pragma once

#include "anim.h"
#include "ball.h"

namespace eng {

enum SelectResult { kSelectFalse = 0, kSelectTrue = 1, kSelectUnsupported = 2 };

// A candidate list in scratch memory.
struct AList {
    int16_t *e;
    int32_t count;
    HD int size() const { return count; }
    HD bool empty() const { return count == 0; }
    HD int16_t &operator[](int i) { return e[i]; }
    HD int16_t operator[](int i) const { return e[i]; }
    HD void push_back(int v) {
        if (count >= kMaxAnimations) Fatal("a fixed-capacity list outgrows its capacity");
        else e[count++] = (int16_t)v;
    }
};
// A planned position list in scratch memory.
struct PList {
    Vec3 *e;
    int32_t count;
    HD int size() const { return count; }
    HD Vec3 &operator[](int i) { return e[i]; }
    HD const Vec3 &operator[](int i) const { return e[i]; }
};

HD int VelocityRank(int v, bool dribbleAsWalk = false) {
    int id = 0;
    switch (v) {
        case kVelIdle:
            id = 0;
            break;
        case kVelDribble:
            id = 1;
            break;
        case kVelWalk:
            id = 2;
            break;
        case kVelSprint:
            id = 3;
            break;
    }
    if (dribbleAsWalk && id > 1) id--;
    return id;
}

// A zero vector gives NaN components.
HD void NormalizeTo(Vec3 &v, float len) {
    float f = len / sqrtf(v.Dot(v));
    v.v[0] *= f;
    v.v[1] *= f;
    v.v[2] *= f;
}
HD Vec3 NormalizedTo(const Vec3 &v, float len) {
    Vec3 r = v;
    NormalizeTo(r, len);
    return r;
}
HD void NormalizeMaximum(Vec3 &v, float len) {
    if (v.Length() > len) {
        v.Normalize();
        v *= len;
    }
}
HD Vec3 NormalizedMaximum(const Vec3 &v, float len) {
    if (v.Length() > len) return v.Normalized(0) * len;
    return v;
}

// `Vec3(0,-1,0).Rotated2D(a)` for the preferred angles {0, +-0.111pi, +-0.25pi, +-0.5pi, +-0.75pi,
// +-0.999pi}, each angle a double product with PI rounded to float (the vector itself for 0).
HD Vec3 PreferredDirection(int i) {
    switch (i) {
        case 0:
            return Vec3(0, -1, 0);
        case 1:
            return Vec3(0x1.5de48ap-2f, -0x1.e12f08p-1f, 0);
        case 2:
            return Vec3(-0x1.5de48ap-2f, -0x1.e12f08p-1f, 0);
        case 3:
            return Vec3(0x1.6a09e6p-1f, -0x1.6a09e6p-1f, 0);
        case 4:
            return Vec3(-0x1.6a09e6p-1f, -0x1.6a09e6p-1f, 0);
        case 5:
            return Vec3(1, 0x1.777a5cp-25f, 0);
        case 6:
            return Vec3(-1, 0x1.777a5cp-25f, 0);
        case 7:
            return Vec3(0x1.6a09e6p-1f, 0x1.6a09e6p-1f, 0);
        case 8:
            return Vec3(-0x1.6a09e6p-1f, 0x1.6a09e6p-1f, 0);
        case 9:
            return Vec3(0x1.9bc4e4p-9f, 0x1.ffff5ap-1f, 0);
        default:
            return Vec3(-0x1.9bc4e4p-9f, 0x1.ffff5ap-1f, 0);
    }
}
HD float PreferredAngle(int i) {
    const double f[11] = {0, 0.111, -0.111, 0.25, -0.25, 0.5, -0.5, 0.75, -0.75, 0.999, -0.999};
    return (float)(f[i] * (double)PI);
}
HDN Vec3 SnapToPreferredDirection(const Vec3 &src) {
    float best = -1.0f;
    Vec3 bv;
    for (int i = 0; i < 11; i++) {
        Vec3 cnd = PreferredDirection(i);
        float d = cnd.Dot(src);
        if (d > best) {
            best = d;
            bv = cnd;
        }
    }
    return bv;
}
HDN float SnapToPreferredAngle(float a) {
    float bestDiff = 10000.0, bv = 0;
    for (int i = 0; i < 11; i++) {
        float d = fabsf(PreferredAngle(i) - a);
        if (d < bestDiff) {
            bestDiff = d;
            bv = PreferredAngle(i);
        }
    }
    return bv;
}
HDN float SnapToBodyAngle(float a) {
    const double f[5] = {0, 0.25, -0.25, 0.75, -0.75};
    float bestDiff = 10000.0, bv = 0;
    for (int i = 0; i < 5; i++) {
        float cnd = (float)(f[i] * (double)PI);
        float d = fabsf(cnd - a);
        if (d < bestDiff) {
            bestDiff = d;
            bv = cnd;
        }
    }
    return bv;
}

HD float CorneringBias(const Vec3 &cur, const Vec3 &desired, float velExp, float bias) {
    float angle = desired.Normalized(cur).Angle2D(cur);
    float cb = libm::sinf(fabsf(angle) - 0.5f * PI) * 0.5f + 0.5f;
    float vb = libm::powf(Clamp(cur.Length() / (kSprintVelocity - 0.5f), 0.0f, 1.0f), velExp);
    return vb * cb * bias;
}

HD float StretchSprint(float v, float inMax, float targetMax) {
    if (v < kWalkSprintSwitch) return v;
    float part = v - kWalkSprintSwitch;
    float oldL = inMax - kWalkSprintSwitch, newL = targetMax - kWalkSprintSwitch;
    return kWalkSprintSwitch + part * (newL / oldL);
}

HD Vec3 FootReachOffset(float velocity, float bodyAngleRel, float height) {
    float distance = 0.34f + velocity * kDefaultTouchOffsetMs * 0.001f * 1.0f;
    Vec3 fwd(0, -distance * 0.8f, 0);
    float ba = bodyAngleRel;
    if (velocity < kIdleDribbleSwitch) ba = 0;
    Vec3 angled = Vec3(0, -distance * 0.2f, 0).Rotated2D(ba);
    return (fwd + angled) * (1.0f - Clamp((height - 0.11f) / 4.0f, 0.0f, 0.5f));
}

// Stable sort of `list` by precomputed keys (doubles hold float and int keys exactly, so `<` on
// them orders as on the original type). Any stable sort of a strict weak order without NaN gives
// GRF's std::stable_sort order.
HDN void StableSortByKeys(const Ctx &c, AList &list) {
    ENG_SCOPE(33);
    const int n = list.count;
    double *keys = c.ws->keys;
    int16_t *a = c.ws->order[0], *b = c.ws->order[1];
#if !ENG_DEVICE
    for (int i = 0; i < n; i++)
        if (keys[i] != keys[i]) Fatal("an animation sort key is NaN");
#endif
    // Bottom-up merge sort; the merges of one pass are independent, so the lanes of the match take
    // them in turn.
    for (int i = GroupRank(); i < n; i += kGroupLanes) a[i] = (int16_t)i;
    GroupSync();
    for (int width = 1; width < n; width *= 2) {
        for (int lo = GroupRank() * 2 * width; lo < n; lo += kGroupLanes * 2 * width) {
            int mid = lo + width < n ? lo + width : n, hi = lo + 2 * width < n ? lo + 2 * width : n;
            int l = lo, r = mid, o = lo;
            while (l < mid && r < hi) b[o++] = (keys[a[r]] < keys[a[l]]) ? a[r++] : a[l++];
            while (l < mid) b[o++] = a[l++];
            while (r < hi) b[o++] = a[r++];
        }
        GroupSync();
        int16_t *t = a;
        a = b;
        b = t;
    }
    // `a` holds the order; gather through `b`.
    for (int i = GroupRank(); i < n; i += kGroupLanes) b[i] = list.e[a[i]];
    GroupSync();
    for (int i = GroupRank(); i < n; i += kGroupLanes) list.e[i] = b[i];
    GroupSync();
}

constexpr int kMaxChainKeys = 8;
HD bool ChainPrecedes(const double *l, const double *r, int k) {
    for (int i = 0; i < k; i++) {
        if (l[i] < r[i]) return true;
        if (r[i] < l[i]) return false;
    }
    return false;
}

struct CrudeQuery {
    bool byFunctionType = false;
    int functionType = 0;
    bool heedForcedFoot = false;
    int strongFoot = 1;
    bool bySide = false;
    Vec3 lookAtVectorRelative;
    bool allowLastDitch = false;
    bool byIncomingVelocity = false, incomingVelocityStrict = false, incomingVelocityNoDribbleToIdle = false,
         incomingVelocityNoDribbleToSprint = false, incomingVelocityForceLinearity = false;
    int incomingVelocity = 0;
    bool byOutgoingVelocity = false;
    int outgoingVelocity = 0;
    bool byPickupBall = false, pickupBall = true;
    bool byIncomingBodyDirection = false;
    Vec3 incomingBodyDirection;
    bool incomingBodyDirectionStrict = false, incomingBodyDirectionForceLinearity = false;
    bool byIncomingBallDirection = false;
    Vec3 incomingBallDirection;
    bool byOutgoingBallDirection = false;
    Vec3 outgoingBallDirection;
    bool byTripType = false;
    int tripType = 0;
    int32_t incomingSpecialState = kStrEmpty, incomingRetainState = kStrEmpty;
    float specialVar1 = 0, specialVar2 = 0;
};

HDN bool CheckFunctionType(int at, int fn) {
    switch (fn) {
        case kFnMovement:
            return at == kAtMovement;
        case kFnBallControl:
            return at == kAtBallControl;
        case kFnTrap:
            return at == kAtTrap;
        case kFnShortPass:
            return at == kAtShortPass;
        case kFnLongPass:
            return at == kAtLongPass;
        case kFnHighPass:
            return at == kAtHighPass;
        case kFnShot:
            return at == kAtShot;
        case kFnDeflect:
            return at == kAtDeflect;
        case kFnCatch:
            return at == kAtCatch;
        case kFnInterfere:
            return at == kAtInterfere;
        case kFnTrip:
            return at == kAtTrip;
        case kFnSliding:
            return at == kAtSliding;
        case kFnSpecial:
            return at == kAtSpecial;
        default:
            return false;
    }
}

// |ALLOWED[i].Angle2D(ALLOWED[j])| / PI at 6i + j.
HD float AllowedBodyDirectionKey(int i, int j) {
    const float t[36] = {0x0p+0f,   0x1p-2f, 0x1p-2f, 0x1.8p-1f, 0x1.8p-1f, 0x0p+0f, 0x1p-2f,   0x0p+0f,
                         0x1p-1f,   0x1p-1f, 0x1p+0f, 0x1p+0f,   0x1p-2f,   0x1p-1f, 0x0p+0f,   0x1p+0f,
                         0x1p-1f,   0x0p+0f, 0x1.8p-1f, 0x1p-1f, 0x1p+0f,   0x0p+0f, 0x1p-1f,   0x0p+0f,
                         0x1.8p-1f, 0x1p+0f, 0x1p-1f, 0x1p-1f,   0x0p+0f,   0x0p+0f, 0x0p+0f,   0x1p+0f,
                         0x0p+0f,   0x0p+0f, 0x0p+0f, 0x0p+0f};
    return t[6 * i + j];
}
// |FixAngle(ALLOWED[i].Angle2D())| and |Vec3(0,-1,0).Angle2D(ALLOWED[i])|.
HD float AllowedBodyFixAbsolute(int i) {
    const float t[6] = {0x0p+0f, 0x1.921fbp-1f, 0x1.921fcp-1f, 0x1.2d97c8p+1f, 0x1.2d97c8p+1f, 0x1.921fb6p+0f};
    return t[i];
}
HD float AllowedBodyIdleAbsolute(int i) {
    const float t[6] = {0x0p+0f, 0x1.921fb6p-1f, 0x1.921fb6p-1f, 0x1.2d97c8p+1f, 0x1.2d97c8p+1f, 0x0p+0f};
    return t[i];
}
// Bit for bit; a loaded state may hold a body direction outside the table.
HD int AllowedBodyDirectionEntry(const Vec3 &d) {
    for (int i = 0; i < 6; i++) {
        Vec3 a = AllowedBodyDir(i);
        if (BitsOf(d.v[0]) == BitsOf(a.v[0]) && BitsOf(d.v[1]) == BitsOf(a.v[1]) && BitsOf(d.v[2]) == BitsOf(a.v[2]))
            return i;
    }
    return -1;
}

// The incoming-velocity test of the crude selection that GRF's selection sets for each function
// type (humanoid_base.cpp, SelectAnimation): strict for movement and ball control, otherwise
// lenient, with the dribble, sprint and linearity refinements of passes, shots and the rest.
struct VelocityRule {
    bool strict = false, noDribbleToIdle = false, noDribbleToSprint = false, forceLinearity = false;
};
HD VelocityRule FunctionVelocityRule(int fn) {
    VelocityRule r;
    if (fn == kFnMovement || fn == kFnBallControl) {
        r.strict = true;
    } else if (fn != kFnDeflect) {
        r.noDribbleToSprint = true;
        if (fn != kFnShortPass && fn != kFnLongPass && fn != kFnHighPass && fn != kFnShot) {
            r.forceLinearity = true;
            r.noDribbleToIdle = true;
        }
    }
    return r;
}
HD bool VelocityRuleOf(const CrudeQuery &q, const VelocityRule &r) {
    return q.incomingVelocityStrict == r.strict && q.incomingVelocityNoDribbleToIdle == r.noDribbleToIdle &&
           q.incomingVelocityNoDribbleToSprint == r.noDribbleToSprint && q.incomingVelocityForceLinearity == r.forceLinearity;
}
// The incoming-velocity test of one animation (`q.byIncomingVelocity` set).
HD bool IncomingVelocityPasses(const CrudeQuery &q, float incomingVelocity, float outgoingVelocity) {
    int aIn = VelocityCat(incomingVelocity);
    if (!q.incomingVelocityStrict) {
        if (q.incomingVelocityNoDribbleToIdle && aIn == kVelIdle && q.incomingVelocity == kVelDribble) return false;
        if (aIn == kVelIdle && q.incomingVelocity == kVelWalk) return false;
        if (aIn == kVelIdle && q.incomingVelocity == kVelSprint) return false;
        if (aIn == kVelDribble && q.incomingVelocity == kVelIdle) return false;
        if (aIn == kVelWalk && q.incomingVelocity == kVelIdle) return false;
        if (aIn == kVelSprint && q.incomingVelocity == kVelIdle) return false;
        if (q.incomingVelocityNoDribbleToSprint && aIn == kVelSprint && q.incomingVelocity == kVelDribble) return false;
        if (q.incomingVelocityForceLinearity) {
            float ain = RangeVelocity(incomingVelocity), aout = RangeVelocity(outgoingVelocity);
            float qin = VelocityFloat(q.incomingVelocity);
            if (VelocityCat(ain) == kVelDribble) ain = kWalkVelocity;
            if (VelocityCat(aout) == kVelDribble) aout = kWalkVelocity;
            if (VelocityCat(qin) == kVelDribble) qin = kWalkVelocity;
            float upper = (qin < aout) ? aout : qin;
            float lower = (aout < qin) ? aout : qin;
            if (ain > upper) return false;
            if (ain < lower) return false;
        }
    } else if (aIn != q.incomingVelocity) {
        return false;
    }
    return true;
}
// The canonical query of a function type's velocity rule, which the prefiltered record lists
// (Tables::crudeVelocity) were built with.
HD CrudeQuery VelocityRuleQuery(int fn, int incomingVelocity) {
    CrudeQuery q;
    const VelocityRule r = FunctionVelocityRule(fn);
    q.byIncomingVelocity = true;
    q.incomingVelocity = incomingVelocity;
    q.incomingVelocityStrict = r.strict;
    q.incomingVelocityNoDribbleToIdle = r.noDribbleToIdle;
    q.incomingVelocityNoDribbleToSprint = r.noDribbleToSprint;
    q.incomingVelocityForceLinearity = r.forceLinearity;
    return q;
}

// The incoming-body-direction test that GRF's selection sets for each function type: strict for
// movement; otherwise lenient, with the linearity refinement except for deflections and ball
// control.
struct BodyRule {
    bool strict = false, forceLinearity = false;
};
HD BodyRule FunctionBodyRule(int fn) {
    BodyRule r;
    if (fn != kFnMovement) r.forceLinearity = fn != kFnDeflect ? fn != kFnBallControl : false;
    else r.strict = true;
    return r;
}
// The incoming-body-direction test of one animation, for a query body direction given by its
// absolute angles and either its allowed-direction entry (`entry` >= 0) or the direction itself.
HD bool IncomingBodyPasses(const BodyRule &rule, int entry, const Vec3 &direction, float queryInBodyFixAbs,
                           float queryIdleBodyAbs, const CrudeRecord &r) {
    const float margin = 0.06f * PI;
    if (VelocityCat(r.incomingVelocity) != kVelIdle) {
        if (r.inBodyFixAbsolute > queryInBodyFixAbs + margin) return false;
        // Selected with constant indices, so a record copied into registers stays there.
        float entryAngle = r.incomingBodyAngles[0];
        for (int i = 1; i < 6; i++)
            if (entry == i) entryAngle = r.incomingBodyAngles[i];
        const float qOff = entry >= 0 ? entryAngle : r.incomingBodyDirection.Angle2D(direction);
        if (rule.strict) {
            if (fabsf(qOff) > margin) return false;
        } else {
            if (fabsf(qOff) > 0.5f * PI + margin) return false;
        }
        if (rule.forceLinearity) {
            float bt = r.bodyTurnAngle;
            if ((bt > margin && qOff > margin) || (bt < -margin && qOff < -margin)) return false;
            if (fabsf(bt) + fabsf(qOff) > PI + margin) return false;
        }
    } else {
        if (rule.strict) {
            if (queryIdleBodyAbs > margin) return false;
        } else {
            if (queryIdleBodyAbs > 0.25f * PI + margin) return false;
        }
    }
    return true;
}
// Allowed body-direction entries of a query (AllowedBodyDirectionEntry), which index the
// body-prefiltered record lists (Tables::crudeBody).
constexpr int kBodyEntries = 6;

HDN void FilterAnimations(const Ctx &c, const CrudeQuery &query, AList &out) {
    ENG_SCOPE(28);
    // The query, the tables' bounds and the list held in registers across the list's stores.
    const CrudeQuery q = query;
    const Tables &T = *c.t;
    const float maxIncomingBallDeviation = T.maxIncomingBallDeviation.value();
    const float maxOutgoingBallDeviation = T.maxOutgoingBallDeviation.value();
    int16_t *const kept = out.e;
    int count = 0;
    const float margin = 0.06f * PI;
    Vec3 fenced;
    float queryInToFence = 0.0f;
    if (q.bySide) {
        fenced = q.lookAtVectorRelative.Rotated2D(PI);
        queryInToFence = fenced.Angle2D(q.incomingBodyDirection);
    }
    const bool byBody = q.byIncomingBodyDirection && !(q.byIncomingVelocity && q.incomingVelocity == kVelIdle);
    const int queryBodyEntry = byBody ? AllowedBodyDirectionEntry(q.incomingBodyDirection) : -1;
    float queryInBodyFixAbs = 0.0f, queryIdleBodyAbs = 0.0f;
    if (queryBodyEntry >= 0) {
        queryInBodyFixAbs = AllowedBodyFixAbsolute(queryBodyEntry);
        queryIdleBodyAbs = AllowedBodyIdleAbsolute(queryBodyEntry);
    } else if (byBody) {
        queryInBodyFixAbs = fabsf(FixAngle(q.incomingBodyDirection.Angle2D()));
        queryIdleBodyAbs = fabsf(Vec3(0, -1, 0).Angle2D(q.incomingBodyDirection));
    }
    const int16_t *list = nullptr;
    int n = T.animCount;
    if (q.byFunctionType && q.functionType >= 0 && q.functionType < kFunctionSlots) {
        list = T.fnAnims + T.fnOffset[q.functionType];
        n = T.fnOffset[q.functionType + 1] - T.fnOffset[q.functionType];
    }
    const bool qInBallNonzero = q.incomingBallDirection.Length() != 0.0f;
    Vec3 qInBallAdapted = q.incomingBallDirection;
    qInBallAdapted.v[2] *= 0.4f;
    if (qInBallNonzero) qInBallAdapted.Normalize();
    const Vec3 qOut2D = q.outgoingBallDirection.Get2D();
    const bool qOutNull = fabsf(qOut2D.v[0]) < 0.000001f && fabsf(qOut2D.v[1]) < 0.000001f && fabsf(qOut2D.v[2]) < 0.000001f;
    const Vec3 qOutNormalized = qOutNull ? Vec3(0) : qOut2D.Normalized(Vec3(0));
    // Each animation passes or fails on its own, so the lanes of the match test consecutive ones
    // and append the passing ones in list order.
    bool velocityTested = false, bodyTested = false;
    BodyRule bodyRule;
    bodyRule.strict = q.incomingBodyDirectionStrict;
    bodyRule.forceLinearity = q.incomingBodyDirectionForceLinearity;
    auto accepts = [&](const CrudeRecord &r) -> bool {
        const int at = r.animationType;
        if (q.byFunctionType && !list && !CheckFunctionType(at, q.functionType)) return false;
        if (q.byIncomingVelocity && !velocityTested && !IncomingVelocityPasses(q, r.incomingVelocity, r.outgoingVelocity))
            return false;
        if (q.byOutgoingVelocity && VelocityCat(r.outgoingVelocity) != q.outgoingVelocity) return false;
        if (q.bySide) {
            const Vec3 &aIn = r.incomingBodyDirection;
            const Vec3 &aOut = r.outDirectionRotated;
            const float turn = r.turnAngle;
            if (fabsf(turn) > 0.06f * PI) {
                int aSide = (turn > 0) ? 0 : 1;
                float aInToFence = fenced.Angle2D(aIn);
                float fenceToOut = aOut.Angle2D(fenced);
                int aInToFenceSide = (aInToFence > 0) ? 0 : 1;
                int qInToFenceSide = (queryInToFence > 0) ? 0 : 1;
                int fenceToOutSide = (fenceToOut > 0) ? 0 : 1;
                if (aInToFenceSide == aSide && fenceToOutSide == aSide && fabsf(aInToFence + fenceToOut) < PI) return false;
                // GRF: adds the side number 0 or 1 to an angle in radians.
                if (qInToFenceSide == aSide && fenceToOutSide == aSide && fabsf((float)qInToFenceSide + fenceToOut) < PI)
                    return false;
            }
        }
        const bool retains = r.flags & 1;
        if (q.byPickupBall) {
            if ((!retains && q.pickupBall) || (retains && !q.pickupBall)) return false;
        }
        if (!q.allowLastDitch && (r.flags & 2)) return false;
        if (byBody && !bodyTested &&
            !IncomingBodyPasses(bodyRule, queryBodyEntry, q.incomingBodyDirection, queryInBodyFixAbs, queryIdleBodyAbs, r))
            return false;
        if (q.byIncomingBallDirection && (r.flags & 4) && qInBallNonzero) {
            float ang = fabsf(qInBallAdapted.Angle2D(r.inBallAdapted));
            float maxDev = r.incomingMaxDeviation;
            if (maxDev == 0.0f) {
                maxDev = maxIncomingBallDeviation;
                if (at == kAtDeflect) maxDev = 0.4f * PI;
            }
            if (ang > maxDev) return false;
        }
        if (q.byOutgoingBallDirection) {
            const Vec3 &abd = r.ballDirectionNormalized;
            float ang = qOutNull && (r.flags & 8) ? 0.0f : fabsf((qOutNull ? abd : qOutNormalized).Angle2D(abd));
            float maxDev = r.outgoingMaxDeviation;
            if ((double)maxDev == 0.0) maxDev = maxOutgoingBallDeviation;
            if (ang > maxDev) return false;
        }
        if (q.incomingSpecialState != r.incomingSpecialState) return false;
        if ((q.functionType == kFnDeflect ||
             ((q.incomingRetainState != kStrEmpty) != (r.incomingRetainState != kStrEmpty))) &&
            q.incomingRetainState != r.incomingRetainState)
            return false;
        if (q.specialVar1 != r.specialVar1) return false;
        if (q.specialVar2 != r.specialVar2) return false;
        if (q.byTripType && r.tripTypeRounded != q.tripType) return false;
        if (q.heedForcedFoot && r.forcedFootWhich != 0) {
            int foot = (r.flags & 16) ? 0 : 1;
            if (r.currentFoot == 0) foot = foot == 0 ? 1 : 0;
            if (r.forcedFootWhich == 1 && q.strongFoot != foot) return false;
            if (r.forcedFootWhich == 2 && q.strongFoot == foot) return false;
        }
        return true;
    };
    const CrudeRecord *records = list ? T.crude + T.fnOffset[q.functionType] : T.crudeByIndex;
    // A query with its function type's velocity rule reads the animations of that type that pass
    // the velocity test, prefiltered in list order.
    if (list && q.byIncomingVelocity && q.incomingVelocity >= kVelIdle && q.incomingVelocity <= kVelSprint &&
        VelocityRuleOf(q, FunctionVelocityRule(q.functionType))) {
        const int slot = q.functionType * 4 + q.incomingVelocity;
        records = T.crudeVelocity + T.crudeVelocityOffset[slot];
        n = T.crudeVelocityOffset[slot + 1] - T.crudeVelocityOffset[slot];
        velocityTested = true;
        // With its function type's body rule and an allowed body direction too, the list is
        // prefiltered by the body test as well.
        const BodyRule canonical = FunctionBodyRule(q.functionType);
        if (q.byIncomingBodyDirection && queryBodyEntry >= 0 && canonical.strict == bodyRule.strict &&
            canonical.forceLinearity == bodyRule.forceLinearity) {
            const int body = slot * kBodyEntries + queryBodyEntry;
            records = T.crudeBody + T.crudeBodyOffset[body];
            n = T.crudeBodyOffset[body + 1] - T.crudeBodyOffset[body];
            bodyTested = true;
        }
    }
    for (int k0 = 0; k0 < n; k0 += kGroupLanes) {
        const int k = k0 + GroupRank();
        // The whole record at once, field by field into registers: the tests read its fields
        // one after another.
        const bool keep = k < n && accepts(records[k]);
        const LaneMask passed = GroupBallot(keep);
        if (keep) kept[count + PopCount(passed & LanesBelow(GroupRank()))] = records[k].index;
        count += PopCount(passed);
    }
    out.count = count;
    GroupSync();
}

// The crude query of IdleMovementAnimation: movement from idle to idle.
HD CrudeQuery IdleMovementQuery() {
    CrudeQuery q;
    q.byFunctionType = true;
    q.functionType = kFnMovement;
    q.byIncomingVelocity = true;
    q.incomingVelocity = kVelIdle;
    q.byOutgoingVelocity = true;
    q.outgoingVelocity = kVelIdle;
    return q;
}

// Directions relative to the humanoid's angle; velocities are categories.
struct Predicates {
    int desiredFoot = 0;
    int incomingVelocity = 0;
    Vec3 relDesiredDirection;
    float corneringBias = 0.0f;
    int desiredVelocity = 0;
    Vec3 relIncomingBodyDirection;
    Vec3 lookAt;  // world coordinates
    Vec3 relDesiredTripDirection;
    float idle = 0.0f;
};

HD float MovementSimilarityOf(const Vec3 &outDir, const Vec3 &outMov, const Vec3 &relDesired, int desiredVel, float cb) {
    Vec3 dm = relDesired * VelocityFloat(desiredVel);
    dm = dm * (1.0f - cb);
    float v = (dm - outMov).Length();
    v -= fabsf(relDesired.Dot(outDir)) * 4.0f;
    return v;
}

HDN float DirectionSimilarityRating(const Anim &a, const Predicates &p, const Vec3 &relLookAt) {
    Vec3 relBody = (relLookAt - a.translation).Normalized(Vec3(0, -1, 0));
    float maxSmuggle = 0.1f * PI;
    float outAngle = a.outgoingDirection.Rotated2D(Clamp(p.relDesiredDirection.Angle2D(a.outgoingDirection), -maxSmuggle, maxSmuggle))
                         .Angle2D(Vec3(0, -1, 0));
    Vec3 predicted = a.outgoingBodyDirection.Rotated2D(outAngle);
    float r = fabsf(predicted.Angle2D(relBody));
    r += fabsf(a.outgoingBodyAngle.value()) * 0.05f;
    return r;
}
HD float KeyIdle(const Anim &a, const Predicates &p) { return fabsf(a.idleLevel - p.idle); }
HD int KeyFoot(const Anim &a, const Predicates &p) {
    int r = 1;
    if (a.currentFoot == p.desiredFoot) r = 0;
    if (VelocityCat(a.incomingVelocity) == kVelIdle) r = 0;
    return r;
}
HD float KeyIncomingVelocity(const Anim &a, const Predicates &p) {
    int cur = VelocityRank(p.incomingVelocity);
    int in = VelocityRank(VelocityCat(a.incomingVelocity));
    float r = fabsf(Clamp((float)(in - cur), -3, 3));
    int out = VelocityRank(VelocityCat(a.outgoingVelocity));
    if (in > (cur > out ? cur : out)) r += 0.5f;
    if (in < (cur < out ? cur : out)) r += 0.5f;
    return r;
}

// The search compares Length; the result is GetDistance.
HDN float ClosestOpponentDistance(const World &w, int p) {
    const int opp = 1 - w.playerTeamID[p];
    const Vec3 pos = Sp(w, p).position;
    float best = 10000;
    int bi = -1;
    for (int o = 0; o < w.match.playerCount; o++) {
        if (w.playerTeamID[o] != opp || !w.roster.active[o]) continue;
        float d = (Sp(w, o).position - pos).Length();
        if (d < best) {
            best = d;
            bi = o;
        }
    }
    if (bi < 0) {
        Fatal("a player has no active opponent");
        return 0;
    }
    return GetDistance(Sp(w, bi).position, pos);
}

// Curve(NormalizedClamp(10 * frame, 0, 160), 1) for frames clamped to 0..16.
HD float PhysicsCurvedTime(int frame) {
    int f = frame < 0 ? 0 : frame > 16 ? 16 : frame;
    return Curve(NormalizedClamp((float)(10 * f), 0, 160), 1.0f);
}

HD float LineClosestToPoint(const Vec3 &s, const Vec3 &e, const Vec3 &p) {
    if (s == e) return 0.0f;
    float ld = (e - s).Length();
    if (ld < 0.000001f) return 0.0f;
    return ((p.v[0] - s.v[0]) * (e.v[0] - s.v[0]) + (p.v[1] - s.v[1]) * (e.v[1] - s.v[1])) / (ld * ld);
}

HDN int StringToFunctionType(int at) {
    switch (at) {
        case kAtMovement:
            return kFnMovement;
        case kAtBallControl:
            return kFnBallControl;
        case kAtTrap:
            return kFnTrap;
        case kAtShortPass:
            return kFnShortPass;
        case kAtLongPass:
            return kFnLongPass;
        case kAtHighPass:
            return kFnHighPass;
        case kAtShot:
            return kFnShot;
        case kAtDeflect:
            return kFnDeflect;
        case kAtCatch:
            return kFnCatch;
        case kAtInterfere:
            return kFnInterfere;
        case kAtTrip:
            return kFnTrip;
        case kAtSliding:
            return kFnSliding;
        case kAtSpecial:
            return kFnSpecial;
    }
    return kFnNone;
}

HD Vec3 OutgoingMovementOf(const PList &p) {
    if (p.count < 2) return Vec3(0);
    return (p[p.count - 1] - p[p.count - 2]) * 100.0f;
}

// ---- movement plans ------------------------------------------------------------------------------
// A selected animation's positions, frame by frame (10 ms apart) from where the humanoid stands: the
// animation's own movement, stretched to the player's top speed, turned toward the desired
// direction and blended with it by the physics share, is what a carried velocity chases; the
// velocity's turn, change and gain per frame are bounded. Every expression keeps GRF's operation
// order (humanoid_base.cpp, CalculatePhysicsVector).

// How much of the animation's outgoing movement replaces the desired one: all for touches,
// deflections, specials and animations into or out of a special state, half for trips, none for
// ball control, traps, interference, sliding and untouched movement.
HD float OutgoingSwitch(int at, bool touch, bool special) {
    if (special) return 1.0f;
    switch (at) {
        case kAtBallControl:
        case kAtTrap:
        case kAtInterfere:
        case kAtSliding:
            return 0.0f;
        case kAtDeflect:
        case kAtSpecial:
            return 1.0f;
        case kAtTrip:
            return 0.5f;
        default:
            return touch ? 1.0f : 0.0f;
    }
}
// How much of the plan follows physics rather than the animation's own movement: none for short
// and high passes, shots, deflections, specials and animations from a special state; half for
// interference and trips of type one (none for other trips); all otherwise.
HD float PhysicsShare(int at, bool tripTypeIsOne, bool fromSpecial) {
    if (fromSpecial) return 0.0f;
    switch (at) {
        case kAtShortPass:
        case kAtHighPass:
        case kAtShot:
        case kAtDeflect:
        case kAtSpecial:
            return 0.0f;
        case kAtInterfere:
            return 0.5f;
        case kAtTrip:
            return tripTypeIsOne ? 0.5f : 0.0f;
        default:
            return 1.0f;
    }
}
// The most the plan turns the animation toward the desired direction: when the animation already
// turns that way (over), when it turns the other way (under), and when it runs straight.
struct TurnCaps {
    float under, over, straight;
};
HD TurnCaps PlanTurnCaps(bool touch, bool sliding, const Vec3 &carried, const Vec3 &outgoing, float ballControl) {
    if (sliding) return {0.5f * PI, 0.5f * PI, 0.5f * PI};
    if (!touch) return {0.125f * PI, 0.125f * PI, 0.125f * PI};
    // A touch turns less the faster the humanoid moves through it and the worse its ball control.
    float bonus = 1.0f - libm::PowfPos(NormalizedClamp((carried + outgoing).Length() * 0.5f, 0, kSprintVelocity), 0.8f) * 0.8f;
    bonus *= 0.6f + 0.4f * ballControl;
    return {0.2f * PI * bonus, 0.0f, 0.1f * PI * bonus};
}
// The turn the plan reaches by its last frame: from the animation's outgoing movement (its
// outgoing direction when that is idle) to the desired movement (the desired body direction when
// that is idle), within the caps; none when they lie more than a quarter turn apart, sliding aside.
HD float PlanSteer(int at, const TurnCaps &caps, const Vec3 &outgoing, const Vec3 &outgoingFacing, const Vec3 &desired,
                   const Vec3 &desiredBody, const Vec3 &facing) {
    const Vec3 from = VelocityCat(outgoing.Length()) == kVelIdle ? outgoingFacing : outgoing.Normalized(0);
    const Vec3 to = VelocityCat(desired.Length()) == kVelIdle ? desiredBody : desired.Normalized(0);
    const float wanted = to.Angle2D(from);
    if (!(fabsf(wanted) <= 0.5f * PI || at == kAtSliding)) return 0.0f;
    const float animationTurn = from.Angle2D(facing);
    float cap = caps.straight;
    if (fabsf(animationTurn) > 0.06f * PI) cap = SignSide(wanted) == SignSide(animationTurn) ? caps.over : caps.under;
    return Clamp(wanted, -cap, cap);
}
// The time warp of the animation: at progress p the plan reads animation frame effFrames * p^lag.
// Movement and ball control under physics lag by the player's agility and the animation's
// difficulty (at least 0.7 before a touch), blended toward no warp by the physics share.
struct FrameLag {
    float beforeTouch = 1.0f, afterTouch = 1.0f;
};
HD FrameLag PlanFrameLag(int at, float physicsBias, bool touch, float agility, float difficulty) {
    FrameLag lag;
    if (!(physicsBias > 0.0f && (at == kAtBallControl || at == kAtMovement))) return lag;
    float e = 1.4f - 0.5f * 0.8f;
    e *= 1.2f - agility * 0.4f;
    if (touch) e += -0.1f + Clamp(difficulty * 0.4f, 0.0f, 0.5f);
    else e += -0.2f + Clamp(difficulty * 0.2f, 0.0f, 0.2f);
    e = Clamp(e, 0.25f, 4.0f);
    lag.beforeTouch = (touch ? MaxF(e, 0.7f) : e) * physicsBias + 1.0f * (1.0f - physicsBias);
    lag.afterTouch = e * physicsBias + 1.0f * (1.0f - physicsBias);
    return lag;
}
constexpr float kFrameSeconds = 10 / 1000.0f;

struct MovementPlanner {
    // The plan's constants.
    int at = 0, touchFrame = 0, effFrames = 0, settleFrom = 0, posCount = 0;
    bool touch = false, outgoingIdle = false;
    libm::SinCos turn{};
    float agility = 0, accel = 0, physicsBias = 0, steer = 0, difficultyPenalty = 0, powerFactor = 0, maxVel = 0,
          playerMaxVel = 0, desiredVel = 0;
    FrameLag lag;
    Vec3 desiredDir, outgoingTurned;
    const Vec3 *smoothed = nullptr;  // the animation's smoothed movement, when tabulated
    const Vec3 *positions = nullptr;
    // What carries from frame to frame.
    Vec3 velocity, position;

    HD float Progress(int frame) const { return (frame * 10 + 10) / (float)((effFrames + 1) * 10); }
    // The animation's movement at the warped frame, on the pitch.
    HD Vec3 AnimationMovement(int frame, float progress) const {
        const float e = touch && frame < touchFrame ? lag.beforeTouch : lag.afterTouch;
        const float warped = e == 1.0f ? progress : libm::powf(progress, e);
        const uint32_t animFrame = TruncToUint32(effFrames * warped);
        return RotatedBy(smoothed && animFrame < (uint32_t)posCount ? smoothed[animFrame]
                                                                      : MovementAtFrame(positions, posCount, animFrame, 1),
                         turn);
    }
    // Movement, ball control and traps above the walk-sprint switch stretch to the player's top
    // speed when it is higher.
    HD void Stretch(Vec3 &movement, float &speed) const {
        if (!(speed > kWalkSprintSwitch && (at == kAtMovement || at == kAtBallControl || at == kAtTrap))) return;
        if (!(maxVel > speed)) return;
        speed = StretchSprint(speed, kAnimSprintVelocity, maxVel);
        movement = movement.Normalized(0) * speed;
    }
    // The terms of a frame that the carried velocity leaves alone: the animation's movement on the
    // pitch, stretched to the top speed, its direction and lean toward the desired direction, and
    // the sine and cosine of the frame's share of the steer.
    HD PlanFrame Ahead(int frame) const {
        PlanFrame a;
        const float progress = Progress(frame);
        a.raw = AnimationMovement(frame, progress);
        Vec3 stretched = a.raw;
        a.stretchedSpeed = a.raw.Length();
        Stretch(stretched, a.stretchedSpeed);
        a.lean = MaxF(0.0f, NormalizedMaximum(stretched, 1.0f).Dot(desiredDir));
        a.unit = stretched.Normalized(0);
        const float rotation = steer * progress;
        a.rc = 1.0f;
        a.rs = rotation;
        // Below 2^-12 the sine is the argument and the cosine 1, by the test of sinf/cosf.
        if (!(libm::Top12f(rotation) < libm::Top12f(0x1p-12f))) {
            const libm::SinCos t = libm::sincosf(rotation);
            a.rc = t.c;
            a.rs = t.s;
        }
        return a;
    }
    // What the carried velocity chases this frame: the desired speed held near the stretched
    // animation speed (down by 1.2 or 1.6 m/s; up by the carried excess, fading over the animation
    // and with the angle to the desired direction), along the stretched movement turned by the
    // frame's share of the steer, blended with the raw movement by the physics share.
    HD Vec3 Target(const PlanFrame &a, float progress, float carriedSpeed) const {
        float faster = 0.0f;
        if (carriedSpeed > a.stretchedSpeed) faster = MinF(1.0f - progress, MaxF(0.0f, carriedSpeed - a.stretchedSpeed));
        if (faster > 0) faster *= a.lean;
        if (at == kAtSliding) faster = 100;
        const float slower = touch ? 1.2f : 1.6f;
        const float speed = Clamp(desiredVel, a.stretchedSpeed - slower, a.stretchedSpeed + faster);
        const Vec3 turned = RotatedCS(a.unit * speed, a.rc, a.rs);
        return turned * physicsBias + a.raw * (1.0f - physicsBias);
    }
    // A turn sharper than the agility allows per frame (less at speed, more without a touch) sheds
    // carried speed in proportion to the excess.
    HD void BoundTurn(Vec3 &change, float carriedSpeed) const {
        const Vec3 next = velocity + change;
        if (!(carriedSpeed > kIdleDribbleSwitch && next.Length() > kIdleDribbleSwitch)) return;
        const Vec3 nextDir = next.Normalized(), carriedDir = velocity.Normalized();
        float perFrame = 1.0f * kFrameSeconds;
        perFrame *= (0.7f + 0.3f * agility);
        if (!touch) perFrame *= 1.5f;
        const float limit = perFrame * PI / (NormalizedClamp(carriedSpeed, 0, kSprintVelocity) + 0.01f);
        const float corner = fabsf(nextDir.Angle2D(carriedDir));
        if (corner > limit) change += -velocity * Clamp((corner - limit) / PI * 3.0f, 0.0f, 1.0f);
    }
    // The change per frame is capped by speed (movement less so), the frame's place on the
    // acceleration curve and the humanoid's power.
    HD void BoundChange(Vec3 &change, float carriedSpeed, int frame) const {
        float cap = at == kAtSliding ? 0.1f : at == kAtTrip ? 0.03f * 0.7f : 0.03f;
        const float fast = libm::PowfPos(NormalizedClamp(carriedSpeed, 0, kSprintVelocity), 1.5f);
        const float curved = at == kAtMovement ? fast * 0.4f : fast;
        cap *= (1.0f - curved) + curved * PhysicsCurvedTime(frame);
        cap *= 1.2f - fast * 0.4f;
        cap *= powerFactor;
        NormalizeMaximum(change, MinF(change.Length(), cap * 10));
    }
    // Above the idle-dribble switch the speed gained per frame is capped by the player's
    // acceleration, less in the air (near top speed) and for difficult animations.
    HD void BoundGain(Vec3 &change, float carriedSpeed) const {
        if (at == kAtSliding || at == kAtDeflect) return;
        const Vec3 next = velocity + change;
        const float nextSpeed = next.Length();
        if (!(nextSpeed > kIdleDribbleSwitch)) return;
        const float power = 11.0f * (1.0f - difficultyPenalty * 0.4f);
        const float air = Clamp(
            libm::PowfPos(Clamp((carriedSpeed - kIdleDribbleSwitch) / (playerMaxVel - kIdleDribbleSwitch), 0.0f, 1.0f), 1.8f), 0.0f,
            1.0f);
        Vec3 gain;
        if (nextSpeed > carriedSpeed) gain = next.Normalized(0) * (nextSpeed - carriedSpeed);
        const float gained = gain.Length();
        const float most = power * (1.0f - air) * (accel * 0.3f + 0.7f) * kFrameSeconds;
        if (gained > most) change = change - gain * (1.0f - most / gained);
    }
    // Over the last two frames the velocity settles into the animation's outgoing category: zero
    // for an idle end, the outgoing direction at dribble speed for a moving end that came out idle.
    HD Vec3 Settle(const Vec3 &v, int frame) const {
        if (frame < settleFrom) return v;
        const bool idle = VelocityCat(v.Length()) == kVelIdle;
        if (outgoingIdle && !idle) return Vec3(0);
        if (!outgoingIdle && idle) return NormalizedTo(outgoingTurned, kDribbleVelocity);
        return v;
    }
    // One frame, from its terms computed ahead: the new position.
    HD Vec3 Step(int frame, const PlanFrame &a) {
        const float progress = Progress(frame);
        const float carriedSpeed = velocity.Length();
        Vec3 change = Target(a, progress, carriedSpeed) - velocity;
        BoundTurn(change, carriedSpeed);
        BoundChange(change, carriedSpeed, frame);
        BoundGain(change, carriedSpeed);
        velocity = Settle(velocity + change, frame);
        position += velocity * kFrameSeconds;
        return position;
    }
};

// ---- ball reach ----------------------------------------------------------------------------------
// GRF's test of a touch at a ball key (humanoid_base.cpp, GetBestCheatableAnimationID and its
// distance advantage): the ball must lie within a radius of a point a little behind the
// animation's ball, measured in a frame that stretches the axis across the incoming movement.

// The humanoid's movement through a candidate: incoming, at the touch and outgoing (relative to
// its body), the outgoing angle and the animation's frame count.
struct ReachMotion {
    Vec3 in, touch, out;
    float outAngle;
    int frames;
};
// The factor on the bare radius: larger when the body (a foot's 10 cm ahead) is near the
// animation's ball and near the ball, and when the humanoid moves slowly.
HD float ReachGrowth(const ReachMotion &m, const Vec3 &body, const Vec3 &foot, const Vec3 &animBall, const Vec3 &ball) {
    const float inSpeed = m.in.Length(), outSpeed = m.out.Length();
    const float meanSpeed = (m.in + m.out).Length() * 0.5f;
    const float gainPerSecond = (outSpeed - inSpeed) / (m.frames * 0.01f);
    const Vec3 toe = body + foot.Normalized(0) * 0.1f;
    const float nearAnimBall = 1.0f - Curve(NormalizedClamp((toe - animBall).Length(), 0.0f, 0.7f), 0.7f);
    const float nearBall = 1.0f - Curve(NormalizedClamp((toe - ball).Length(), 0.0f, 0.7f), 0.4f);
    const float slow = 1.0f - NormalizedClamp(meanSpeed, kIdleVelocity, kSprintVelocity);
    const float steady = 1.0f - NormalizedClamp(gainPerSecond / 20.0f, -1.0f, 1.0f);
    return 1.0f + 1.0f * nearAnimBall + 0.6f * nearBall + 0.8f * nearAnimBall * nearBall + 0.0f * steady + 1.0f * slow;
}
// The offset of the measuring point from the animation's ball: against the humanoid's weighted
// movement (mostly outgoing), longer the faster it moves and the more its outgoing direction
// points forward.
HD Vec3 BehindBall(const ReachMotion &m, const Vec3 &outDir) {
    const Vec3 back = -(m.in * 0.1f + m.touch * 0.2f + m.out * 0.7f);
    Vec3 behind = back.Normalized(0) * libm::PowfPos(NormalizedClamp(back.Length(), 0, kSprintVelocity), 0.5f);
    float forward = Vec3(0, -1, 0).Dot(outDir);
    forward = 0.5f + Clamp(forward * 0.5f + 0.5f, 0.0f, 1.0f) * 0.5f;
    behind *= forward;
    return behind;
}
// Whether `ball` (2D, relative to the body's start) is within reach of `animBall` for a bare
// radius and a cheat margin.
HD bool BallWithinReach(const ReachMotion &m, const Vec3 &body, const Vec3 &foot, const Vec3 &animBall, const Vec3 &ball,
                        float radiusFactor, float cheat) {
    const float cheatFactor = 0.5f, cheatBonus = 0.02f;
    float radius = radiusFactor;
    radius *= ReachGrowth(m, body, foot, animBall, ball);
    const Vec3 outDir = VelocityCat(m.out.Length()) == kVelIdle ? Vec3(0, -1, 0).Rotated2D(m.outAngle) : m.out.Normalized();
    const Vec3 behind = BehindBall(m, outDir);
    // Across the incoming movement the offset stretches by 1/0.6 standing to 1/0.3 at a sprint,
    // and the radius by the root of that.
    Vec3 offset = ball - animBall;
    const float toStraight = Vec3(0, -1, 0).Angle2D(m.in.Normalized(outDir));
    offset.Rotate2D(toStraight);
    const float lateral = 0.6f - 0.3f * libm::PowfPos(NormalizedClamp(m.in.Length(), kIdleVelocity, kSprintVelocity), 0.7f);
    offset.v[0] /= lateral;
    radius *= libm::powf(1.0f / lateral, 0.5f);
    offset.Rotate2D(-toStraight);
    const Vec3 center = animBall + behind * (radius + (cheat * 0.6f)) * cheatFactor;
    return !(GetDistance(animBall + offset, center) > (radius + cheat) * cheatFactor + cheatBonus);
}
// The bare radius and cheat margin at a key: 0.3 m less the key's distance from the animation's
// own touch frame, wider for deflections, interference, passes and shots (which also cheat), much
// narrower for sliding, and narrower for ball control and traps when a pass or shot is preferred.
struct TouchReach {
    float radius, cheat;
};
HD TouchReach KeyReach(int fn, float awkward, bool preferPassAndShot) {
    TouchReach r{0.3f * (1.0f - awkward), 0.0f};
    switch (fn) {
        case kFnDeflect:
            r.radius *= 1.8f;
            r.cheat = 0.4f;
            break;
        case kFnSliding:
            r.radius *= 0.2f;
            break;
        case kFnInterfere:
            r.radius *= 1.4f;
            r.cheat = 0.2f;
            break;
        case kFnShortPass:
        case kFnLongPass:
        case kFnHighPass:
        case kFnShot:
            r.radius *= 1.3f;
            r.cheat = 0.15f;
            break;
        case kFnTrap:
        case kFnBallControl:
            if (preferPassAndShot) r.radius *= 0.3f;
            break;
        default:
            break;
    }
    r.cheat *= 1.0f - awkward;
    return r;
}
// What one touch search reads, fixed for its candidates.
struct TouchSearch {
    MentalBallView mental;
    const Vec3 *predictions;
    bool flip, retainerIsMe, preferPassAndShot, useDesiredMovement;
    int fn;
    libm::SinCos back;  // turns pitch directions into the body's frame
    Vec3 inMov, position, desiredMovement, desiredBodyRel;
    float height, ballControl;
    uint64_t now;
    HD TouchSearch(const World &w, int mentalImage, int humanoid, int function, const libm::SinCos &backTurn, const Vec3 &movement,
                   const Vec3 &at, float bodyHeight, float control, bool prefer, bool useDesired, const Vec3 &desired,
                   const Vec3 &desiredBody)
        : mental(w, mentalImage),
          predictions(w.match.ball.predictions),
          flip(w.match.ball.lazyFlip),
          retainerIsMe(w.match.ballRetainer == humanoid),
          preferPassAndShot(prefer),
          useDesiredMovement(useDesired),
          fn(function),
          back(backTurn),
          inMov(RotatedBy(movement, backTurn)),
          position(at),
          desiredMovement(desired),
          desiredBodyRel(desiredBody),
          height(bodyHeight),
          ballControl(control),
          now(w.match.actualTimeMs) {}
};
// The height gap between the ball and the animation's ball at a key, eased for low balls and a
// base animation's low ball, doubled and more for a ball far overhead; none for the retainer.
HD float TouchHeightMiss(const TouchSearch &ts, bool baseAnimation, float animZ, float ballZ) {
    float miss = fabsf(ballZ - animZ);
    miss *= 1.0f - Clamp((float)(((double)animZ - 0.11) * (double)0.3f), 0.0f, 0.2f);
    miss *= 1.0f - Clamp((float)(((double)ballZ - 0.11) * (double)0.4f), 0.0f, 0.3f);
    if (ballZ > 1.8f && ballZ > animZ + 0.12f) miss *= 2.0f;
    if (ballZ > 2.6f && ballZ > animZ + 0.08f) miss *= 20.0f;
    if (ts.fn == kFnDeflect) miss *= 0.8f;
    if (ts.retainerIsMe) miss = 0.0f;
    if (ballZ < 0.5f && baseAnimation) miss = MaxF(miss - 0.15f, 0.0f);
    return miss;
}
struct TouchProbe {
    bool reaches = false;
    Vec3 smuggle;  // from the animation's ball to the ball, 2D
};

struct Selector {
    World &w;
    const Ctx &c;
    int hi;  // humanoid index: a player, or playerCount + official
    Predicates pred;
    struct TurnCache {
        bool valid = false;
        uint32_t bits = 0;
        libm::SinCos t{};
    } fwd, back;

    HD Selector(World &world, const Ctx &ctx, int index) : w(world), c(ctx), hi(index) {}

    HD static libm::SinCos Cached(TurnCache &tc, float angle, float arg) {
        uint32_t b = BitsOf(angle);
        if (!tc.valid || tc.bits != b) {
            tc.t = libm::sincosf(arg);
            tc.bits = b;
            tc.valid = true;
        }
        return tc.t;
    }
    HD libm::SinCos Turn(float a) { return Cached(fwd, a, a); }
    HD libm::SinCos BackTurn(float a) { return Cached(back, a, -a); }

    HD bool Official() const { return hi >= w.match.playerCount; }
    HD Player &P() { return w.match.players[hi]; }
    HD Humanoid &H() { return Official() ? w.match.officials[hi - w.match.playerCount].humanoid : P().base.humanoid; }
    HD SpatialState &S() { return H().spatial; }
    HD const Anim &A(int i) const { return c.t->anims[i]; }
    HD const AnimDerived &D(int i) const { return c.t->derived[i]; }
    HD int MentalImg() { return MentalImageIndex(w, H().mentalImageTime); }
    HD Vec3 MentalBallAt(int ms) { return MentalBallPrediction(w, MentalImg(), ms); }
    HD float Statistic(int s) { return Official() ? c.sd->data[hi].stats[s] : GetStatistic(w, c, hi, s); }
    HD float BaseLastTouchBias(int decayMs) {
        uint64_t last = Official() ? w.match.officials[hi - w.match.playerCount].lastTouchTimeMs : P().base.lastTouchTimeMs;
        if (decayMs > 0) return 1.0f - Clamp((float)(w.match.actualTimeMs - last) / (float)decayMs, 0.0f, 1.0f);
        return 0.0f;
    }
    HD Vec3 RelativeLookAt() { return RotatedBy(pred.lookAt - S().position, BackTurn(S().angle.value())); }

    HD float MovementSimilarityKey(int i) {
        const SelectionRecord &r = c.t->selection[i];
        return MovementSimilarityOf(r.preferredOutgoingDirection, r.preferredOutgoingMovement, pred.relDesiredDirection,
                                    pred.desiredVelocity, pred.corneringBias);
    }
    HD int IncomingBodyDirectionQuery() { return BodyDirectionIndex(pred.relIncomingBodyDirection); }
    HD float IncomingBodyDirectionKey(int i, int q) {
        float r = AllowedBodyDirectionKey(c.t->selection[i].incomingBodyIndex, q);
        if (VelocityCat(A(i).incomingVelocity) == kVelIdle) r = 0;
        return r;
    }
    HD float PreferredOutgoingAngle(int i) { return c.t->selection[i].preferredOutgoingAngle; }
    HD float LookAngle(int i) { return c.t->selection[i].lookAngle; }
    HD Vec3 SmoothedMovement(int i, uint32_t frame) {
        const Anim &a = A(i);
        int32_t first = c.t->selection[i].smoothedFirst;
        if (first >= 0 && frame < (uint32_t)a.posCount) return c.t->smoothed[first + frame];
        return MovementAtFrame(c.t->positions + a.posFirst, a.posCount, frame, 1);
    }

    HD void SetMovementSimilarityPredicate(const Vec3 &relDesired, int desiredVel) {
        pred.relDesiredDirection = relDesired;
        pred.desiredVelocity = desiredVel;
        pred.corneringBias = CorneringBias(Vec3(0, -1.0f * S().floatVelocity, 0),
                                                           relDesired * VelocityFloat(desiredVel), 1.0f, 0.9f);
    }

    // Keys are computed into scratch, then a stable sort permutes the list.
    template <class KeyFn>
    HD void Sort(AList &l, KeyFn key) {
        if (l.count < 2) return;
        for (int i = GroupRank(); i < l.count; i += kGroupLanes) c.ws->keys[i] = (double)key((int)l[i]);
        GroupSync();
        StableSortByKeys(c, l);
    }
    HD void SortBaseAnimation(AList &l) {
        Sort(l, [&](int i) { return A(i).baseAnimation ? 0 : 1; });
    }
    // The position of the element that a stable sort of `l` by `key`, followed (with `byBase`) by
    // the stable sort by base animation, puts first: the smallest (base key, key), the earliest on
    // ties. The lanes of the match scan every fourth element and combine their bests.
    template <class KeyFn>
    HD int StableFirst(const AList &l, KeyFn key, bool byBase) {
        double bestKey = 0, bestBase = 0;
        int best = -1;
        for (int i = GroupRank(); i < l.count; i += kGroupLanes) {
            const double k = (double)key((int)l[i]);
            const double b = byBase ? (A(l[i]).baseAnimation ? 0 : 1) : 0;
#if !ENG_DEVICE
            if (k != k) Fatal("an animation sort key is NaN");
#endif
            if (best < 0 || b < bestBase || (b == bestBase && k < bestKey)) {
                best = i;
                bestKey = k;
                bestBase = b;
            }
        }
        for (int r = 1; r < kGroupLanes; r++) {
            const int other = GroupShuffle((int32_t)best, r);
            const double ok = GroupShuffle(bestKey, r), ob = GroupShuffle(bestBase, r);
            if (other >= 0 && (best < 0 || ob < bestBase || (ob == bestBase && (ok < bestKey || (ok == bestKey && other < best))))) {
                best = other;
                bestKey = ok;
                bestBase = ob;
            }
        }
        // Every lane now holds the group's first; lane 0's combination is taken for all.
        return GroupShuffle((int32_t)best, 0);
    }
    // Keeps, in order, the elements of `l` for which `keep` holds (the lanes of the match test
    // consecutive elements and compact the list in place).
    template <class KeepFn>
    HD void KeepInOrder(AList &l, KeepFn keep) {
        int kept = 0;
        for (int k0 = 0; k0 < l.count; k0 += kGroupLanes) {
            const int k = k0 + GroupRank();
            const int16_t e = k < l.count ? l[k] : 0;
            const bool ok = k < l.count && keep((int)e);
            const LaneMask mask = GroupBallot(ok);
            GroupSync();
            if (ok) l.e[kept + PopCount(mask & LanesBelow(GroupRank()))] = e;
            kept += PopCount(mask);
            GroupSync();
        }
        l.count = kept;
    }
    // The first element after a chain of stable sorts: the smallest key tuple, the earliest on ties.
    template <class KeysFn>
    HD int FirstOfSortChain(const AList &l, int keyCount, KeysFn keys) {
        ENG_SCOPE(34);
        if (l.count < 2) return l[0];
        // The first element with the least keys. The lanes of the match each take every
        // kGroupLanes-th element, keeping their first least, and combine in element order: the
        // same element for keys that order totally. A NaN key (which the host build rejects)
        // takes the sequential scan.
        int best = -1;
        double bk[kMaxChainKeys];
        bool nan = false;
        for (int e = GroupRank(); e < l.count; e += kGroupLanes) {
            double k[kMaxChainKeys];
            keys((int)l[e], k);
            for (int j = 0; j < keyCount; j++)
                if (k[j] != k[j]) nan = true;
#if !ENG_DEVICE
            if (nan) Fatal("an animation sort key is NaN");
#endif
            if (best < 0 || ChainPrecedes(k, bk, keyCount)) {
                best = e;
                for (int j = 0; j < keyCount; j++) bk[j] = k[j];
            }
        }
        if (GroupBallot(nan)) {
            best = -1;
            for (int e = 0; e < l.count; e++) {
                double k[kMaxChainKeys];
                keys((int)l[e], k);
                if (best < 0 || ChainPrecedes(k, bk, keyCount)) {
                    best = e;
                    for (int j = 0; j < keyCount; j++) bk[j] = k[j];
                }
            }
            return l[best];
        }
        int winner = -1;
        double wk[kMaxChainKeys];
        for (int r = 0; r < kGroupLanes; r++) {
            const int e = GroupShuffle((int32_t)best, r);
            if (e < 0) continue;
            double k[kMaxChainKeys];
            for (int j = 0; j < keyCount; j++) k[j] = GroupShuffle(bk[j], r);
            if (winner < 0 || ChainPrecedes(k, wk, keyCount) || (!ChainPrecedes(wk, k, keyCount) && e < winner)) {
                winner = e;
                for (int j = 0; j < keyCount; j++) wk[j] = k[j];
            }
        }
        return l[winner];
    }

    HD bool AllowLastDitch(bool withPossessionAmount = true) {
        if (withPossessionAmount && TeamOfPlayer(w, hi).teamPossessionAmount < 1.0f) return true;
        return ((int)P().timeToBallOptimisticMs * 1.7f + 800 < (float)(int)P().timeToBallMs);
    }
    HD bool HighOrBouncyBall() {
        const Ball &b = w.match.ball;
        float hn = BallPredict(b, 10).v[2], ht = BallPredict(b, kDefaultTouchOffsetMs).v[2];
        float bounce = fabsf(b.momentum.v[2]);
        if (hn > 0.3f || ht > 0.3f) return true;
        if (bounce > 1.0f) return true;
        return false;
    }

    HDN void KeepNearestQuadrant(AList &l, const PlayerCommand &cmd, bool strict, float allowedAngle = 0,
                                         int allowedVelocitySteps = 0, int forcedQuadrant = -1) {
        ENG_SCOPE(32);
        if (l.empty()) return;
        int bestQ = forcedQuadrant;
        auto keeps = [&](int ai) {
            const Anim &a = A(ai);
            if (strict) return a.quadrantID == bestQ;
            const Quadrant &bq = c.t->quadrants[bestQ];
            const Quadrant &qd = c.t->quadrants[a.quadrantID];
            bool keep = true;
            if (!a.lastDitch) {
                int dv = VelocityRank(qd.velocity, true) - VelocityRank(bq.velocity, true);
                if ((dv < 0 ? -dv : dv) > allowedVelocitySteps) keep = false;
            }
            if (fabsf(qd.angle.value() - bq.angle.value()) > allowedAngle) keep = false;
            return keep;
        };
        if (bestQ == -1) {
            // GRF sorts by similarity (then base animation), takes the first element's quadrant
            // and keeps the sorted elements near it. The first element passes its own test and the
            // test depends on the element alone, so filtering first and sorting the kept ones
            // gives the same list.
            auto key = [&](int i) { return MovementSimilarityKey(i); };
            const bool byBase = strict && cmd.desiredFunctionType != kFnMovement;
            bestQ = A(l[StableFirst(l, key, byBase)]).quadrantID;
            KeepInOrder(l, keeps);
            Sort(l, key);
            if (byBase) SortBaseAnimation(l);
            return;
        }
        int kept = 1;
        for (int k = 1; k < l.count; k++)
            if (keeps(l[k])) l[kept++] = l[k];
        l.count = kept;
    }

    HDN void KeepNearestLook(AList &l, const PlayerCommand &cmd, bool strict, float allowedAngle = 0) {
        ENG_SCOPE(32);
        if (l.empty()) return;
        Vec3 relLookAt;
        if (l.count > 1) relLookAt = RelativeLookAt();
        // As in KeepNearestQuadrant: the first element of GRF's sorted list passes its
        // own test, so the kept elements are filtered first and sorted after.
        auto key = [&](int i) { return DirectionSimilarityRating(A(i), pred, relLookAt); };
        const bool byBase = strict && cmd.desiredFunctionType != kFnMovement;
        const float bestLook = LookAngle(l[StableFirst(l, key, byBase)]);
        const float allowed = strict ? 0.06f * PI : allowedAngle;
        KeepInOrder(l, [&](int ai) { return fabsf(LookAngle(ai) - bestLook) <= allowed; });
        Sort(l, key);
        if (byBase) SortBaseAnimation(l);
    }

    HDN int IdleMovementAnimation() {
        // The crude selection of IdleMovementQuery, made once from the tables; only read here.
        const AList l{const_cast<int16_t *>(c.t->idleMovement), c.t->idleMovementCount};
        pred.idle = 1;
        pred.relIncomingBodyDirection = Vec3(0, -1, 0);
        pred.incomingVelocity = kVelIdle;
        SetMovementSimilarityPredicate(Vec3(0, -1, 0), kVelIdle);
        pred.lookAt = S().position + RotatedBy(Vec3(0, -10, 0), Turn(S().angle.value()));
        Vec3 relLookAt;
        int qi = 0;
        if (l.count > 1) {
            relLookAt = RelativeLookAt();
            qi = IncomingBodyDirectionQuery();
        }
        return FirstOfSortChain(l, 5, [&](int i, double *k) {
            k[0] = MovementSimilarityKey(i);
            k[1] = DirectionSimilarityRating(A(i), pred, relLookAt);
            k[2] = KeyIncomingVelocity(A(i), pred);
            k[3] = IncomingBodyDirectionKey(i, qi);
            k[4] = KeyIdle(A(i), pred);
        });
    }

    // The movement plan of animation `ai` into `out` (see MovementPlanner); returns the velocity it
    // ends with and sets `rotationOffset`, the turn the plan adds to the animation's outgoing angle.
    // `together`: every lane of the match makes this call with the same arguments, and they share
    // the frames' terms; otherwise a lane plans alone.
    HDN Vec3 PlanMovement(int ai, bool useDesiredMovement, const Vec3 &desiredMovement, const Vec3 &desiredBodyRel, PList &out,
                          float &rotationOffset, bool together) {
        ENG_SCOPE(38);
        const Anim &a = A(ai);
        const AnimDerived &d = D(ai);
        const SpatialState &s = S();
        const float angle = s.angle.value();
        MovementPlanner plan;
        plan.at = a.animationType;
        plan.touchFrame = d.touchFrame;
        plan.touch = d.touchFrame > 0;
        plan.turn = Turn(angle);
        plan.agility = Statistic(kStatAgility);
        plan.accel = Statistic(kStatAcceleration);
        const bool special = a.incomingSpecialState != kStrEmpty || a.outgoingSpecialState != kStrEmpty;
        // The velocity carried into the animation: the humanoid's own (the animation's incoming
        // velocity takes no part in it).
        const float incomingSwitch = 0.0f;
        const Vec3 animIn = RotatedBy(Vec3(0, -1, 0), plan.turn) * RangeVelocity(a.incomingVelocity);
        plan.velocity = animIn * incomingSwitch + s.movement * (1.0f - incomingSwitch);
        const Vec3 predOut = RotatedBy(a.outgoingMovement, plan.turn);
        const float outgoingSwitch = OutgoingSwitch(plan.at, plan.touch, special);
        const Vec3 asked = useDesiredMovement ? desiredMovement : predOut;
        const Vec3 desired = predOut * outgoingSwitch + asked * (1.0f - outgoingSwitch);
        plan.playerMaxVel = GetMaximumVelocity(*c.sd, hi);
        plan.maxVel = plan.touch ? plan.playerMaxVel * 0.92f : plan.playerMaxVel;
        const float difficulty = d.difficultyFactor;
        plan.difficultyPenalty = libm::PowfPos(
            Clamp((difficulty - 0.0f) * (1.0f - (plan.agility * 0.2f + plan.accel * 0.2f)) * 2.0f, 0.0f, 1.0f), 0.7f);
        plan.powerFactor = 1.0f - Clamp(libm::PowfPos(BaseLastTouchBias(1000), 0.8f) * (0.8f - Statistic(kStatDribble) * 0.3f), 0.0f, 0.4f);
        plan.powerFactor *= 1.0f - Clamp(H().decayingPositionOffset.Length() * (10.0f - Statistic(kStatBalance) * 5.0f) - 0.1f,
                                         0.0f, 0.3f);
        plan.physicsBias = PhysicsShare(plan.at, d.tripTypeIsOne, a.incomingSpecialState != kStrEmpty);
        const TurnCaps caps = PlanTurnCaps(plan.touch, plan.at == kAtSliding, plan.velocity, predOut,
                                           plan.touch ? Statistic(kStatBallControl) : 0.0f);
        plan.steer = plan.physicsBias > 0.0f ? PlanSteer(plan.at, caps, predOut, RotatedBy(a.outgoingDirection, plan.turn), desired,
                                                         RotatedBy(desiredBodyRel, plan.turn), s.directionVec)
                                             : 0.0f;
        plan.lag = PlanFrameLag(plan.at, plan.physicsBias, plan.touch, plan.agility, difficulty);
        plan.desiredVel = desired.Length();
        plan.desiredDir = desired.Normalized(0);
        if (a.frameCount > kAnimPositions) Fatal("a fixed-capacity list outgrows its capacity");
        plan.effFrames = a.frameCount - 1;
        plan.settleFrom = a.frameCount - 2;
        plan.outgoingIdle = VelocityCat(a.outgoingVelocity) == kVelIdle;
        plan.outgoingTurned = RotatedBy(a.outgoingMovement, plan.turn);
        const int32_t smoothedFirst = c.t->selection[ai].smoothedFirst;
        plan.smoothed = smoothedFirst >= 0 ? c.t->smoothed + smoothedFirst : nullptr;
        plan.positions = c.t->positions + a.posFirst;
        plan.posCount = a.posCount;
        Vec3 *const frames = out.e;
        const int frameCount = a.frameCount;
        if (together) {
            // The lanes of the match compute the frames' terms ahead; the carried velocity then
            // runs through them in order.
            PlanFrame *const ahead = c.ws->planFrames;
            for (int frame = GroupRank(); frame < frameCount; frame += kGroupLanes) ahead[frame] = plan.Ahead(frame);
            GroupSync();
            for (int frame = 0; frame < frameCount; frame++) frames[frame] = plan.Step(frame, ahead[frame]);
        } else {
            for (int frame = 0; frame < frameCount; frame++) frames[frame] = plan.Step(frame, plan.Ahead(frame));
        }
        out.count = frameCount > 0 ? frameCount : 0;
        if (!plan.outgoingIdle && VelocityCat(plan.velocity.Length()) != kVelIdle)
            rotationOffset = RotatedBy(plan.velocity, BackTurn(angle)).Angle2D(a.outgoingMovement);
        else
            rotationOffset = plan.steer * plan.physicsBias;
        return plan.velocity;
    }

    // Whether ball control needs a touch: when the command asks to move (above the idle-dribble
    // switch), the ball moves faster than 2 m/s, the animation turns more than an eighth turn, or
    // the humanoid's movement (its own blended with the animation's) and the ball's (as seen 240
    // to 250 ms ahead) differ by 2 m/s or more, in speed beyond -1.4 to 0.7 m/s, or, for an
    // animation that leaves moving, in direction.
    HDN bool BallControlNeedsTouch(int ai, const PlayerCommand &cmd) {
        const Anim &a = A(ai);
        const SpatialState &s = S();
        if (cmd.desiredVelocityFloat > kIdleDribbleSwitch || fabsf(w.match.ball.momentum.Length()) > 2.0f) return true;
        if (fabsf(a.outgoingAngle.value()) > 0.125f * PI) return true;
        Vec3 mine = RotatedBy(a.outgoingMovement, Turn(s.angle.value())) * 0.3f + s.movement * 0.7f;
        const float blendedSpeed = mine.Length();
        mine.Normalize(s.directionVec);
        mine *= s.movement.Length() * 0.8f + blendedSpeed * 0.2f;
        const Vec3 ball = (MentalBallAt(250).Get2D() - MentalBallAt(240).Get2D()) * 100;
        if ((double)(mine - ball).Length() >= 2.0) return true;
        const float speedGap = mine.Length() - ball.Length();
        if ((double)speedGap < -1.4 || (double)speedGap >= 0.7) return true;
        return VelocityCat(a.outgoingVelocity) != kVelIdle &&
               (double)mine.Normalized(s.directionVec).Dot(ball.Normalized(s.directionVec)) < 0.975;
    }

    // Where, and facing which way, the running animation ends: its last planned position (its
    // own translation once the plan has run out) plus the smuggles; its outgoing angle plus the
    // end rotation smuggle.
    HDN void PredictedPose(Vec3 &position, float &angle) {
        ENG_SCOPE(22);
        const AnimationState &cur = H().anim;
        const Anim &a = A(cur.anim);
        const SpatialState &s = S();
        const Vec3 travel = (uint32_t)cur.positions.count > (uint32_t)cur.frameNum ? cur.positions[a.frameCount - 1]
                                                                                   : a.translation.Get2D().Rotated2D(s.angle.value());
        position = s.position + travel + cur.actionSmuggle + cur.actionSmuggleSustain + cur.movementSmuggle;
        angle = ModulateIntoRange(-PI, PI, s.angle.value() + a.outgoingAngle.value() + cur.rotationSmuggleEnd.value());
    }

    HD int DesiredTimeToBallMs() {
        return TruncToInt32(Clamp((float)P().desiredTimeToBallMs, (float)(int)P().timeToBallMs, 1000000.0f));
    }

    // Whether the player steers its running animation toward the ball: the designated player of
    // the match and of its team, in play, with no set piece, retainer, touch, special state or
    // trip other than of type one.
    HD bool SteersTowardBall() {
        const AnimationState &cur = H().anim;
        const Anim &a = A(cur.anim);
        const MatchState &m = w.match;
        if (m.designatedPossessionPlayer != hi || TeamOfPlayer(w, hi).designatedTeamPossessionPlayer != hi) return false;
        if (!m.inPlay || m.inSetPiece || m.ballRetainer != -1 || cur.touchFrame != -1) return false;
        if (a.incomingSpecialState != kStrEmpty || a.outgoingSpecialState != kStrEmpty) return false;
        return !(cur.functionType == kFnTrip && !D(cur.anim).tripTypeIsOne);
    }
    // The movement smuggle: the shift that brings the foot of the animation's end pose onto the
    // ball when it arrives (the later of the animation's touch time and the player's time to the
    // ball), toward the ball's path when the player does not have it; none when the ball arrives
    // too late (250 ms after the touch, 2 s for an animation that ends idle), barely moves or
    // would speed the humanoid past the dribble-walk switch. At most 1.6 m/s over the animation,
    // less 6 cm.
    HDN Vec3 MovementSmuggle() {
        if (!SteersTowardBall()) return Vec3(0);
        AnimationState &cur = H().anim;
        const Anim &a = A(cur.anim);
        uint32_t ballDue = (uint32_t)(int)P().timeToBallMs;
        if (DesiredTimeToBallMs() > (int)ballDue) ballDue = (uint32_t)DesiredTimeToBallMs();
        const uint32_t animMs = (uint32_t)a.frameCount * 10, touchMs = animMs + kDefaultTouchOffsetMs;
        const uint32_t arrival = touchMs > ballDue ? touchMs : ballDue;
        const uint32_t latest = VelocityCat(a.outgoingVelocity) == kVelIdle ? 2000u : 250u + kDefaultTouchOffsetMs;
        if (arrival - touchMs > latest) return Vec3(0);
        const Vec3 outgoing = OutgoingMovementOf(PList{cur.positions.e, cur.positions.count});
        Vec3 endPosition;
        float endAngle;
        PredictedPose(endPosition, endAngle);
        const Vec3 ballThen = MentalBallAt((int)arrival);
        const Vec3 foot =
            endPosition + FootReachOffset(outgoing.Length(), a.outgoingBodyAngle.value(), ballThen.v[2]).Rotated2D(endAngle);
        Vec3 gap;
        if (P().hasPossession) {
            gap = ballThen.Get2D() - foot;
        } else {
            const Vec3 from = MentalBallAt(0).Get2D(), to = ballThen.Get2D();
            if ((from - to).Length() < 0.5f) return Vec3(0);
            gap = (from + (to - from) * LineClosestToPoint(from, to, foot)) - foot;
        }
        const Vec3 result = outgoing + gap / (animMs * 0.001f);
        if (result.Length() > outgoing.Length() && result.Length() > kDribbleWalkSwitch) return Vec3(0);
        NormalizeMaximum(gap, 1.6f * ((a.frameCount - 1) * 0.01f));
        return gap.Normalized(0) * MaxF(0.0f, gap.Length() - 0.06f);
    }

    HD float LastTouchBiasAt(int decayMs, uint64_t t) {
        uint64_t at = t;
        if (t == 0) at = w.match.actualTimeMs;
        if (decayMs > 0) return 1.0f - Clamp((float)(at - P().base.lastTouchTimeMs) / (float)decayMs, 0.0f, 1.0f);
        return 0.0f;
    }

    // Whether the ball, `frame` frames ahead on the match's own prediction, is on the pitch (with
    // the line's width and the ball's radius).
    HD static bool BallOnPitchAt(const Vec3 *predictions, bool flip, int frame) {
        Vec3 at = BallPredictRaw(predictions, frame * 10);
        if (flip) at.Mirror();
        return !(fabsf(at.v[0]) > kPitchHalfLength + kLineHalfWidth + 0.11f || fabsf(at.v[1]) > kPitchHalfWidth + kLineHalfWidth + 0.11f);
    }

    // One candidate of the touch search: its movement plan into `plan`, then its ball keys from the
    // middle one down, then up from the one after the middle; true with the first key whose ball
    // the body reaches (TouchProbe).
    HDN bool TryTouchAnimation(const TouchSearch &ts, int ai, PList &plan, float &rotSmuggle, float &predAngle, Vec3 &outMov,
                               Vec3 &smuggle, int &touchFrame) {
        const Anim &a = A(ai);
        PlanMovement(ai, ts.useDesiredMovement, ts.desiredMovement, ts.desiredBodyRel, plan, rotSmuggle, false);
        predAngle = ModulateIntoRange(-PI, PI, a.outgoingAngle.value() + rotSmuggle);
        outMov = RotatedBy(OutgoingMovementOf(plan), ts.back);
        const int total = a.footballCount, middle = total / 2;
        for (int tn = 0; tn < total; tn++) {
            const FootballKey &key = c.t->football[a.footballFirst + (tn <= middle ? middle - tn : tn)];
            if (!ts.retainerIsMe && !BallOnPitchAt(ts.predictions, ts.flip, key.frame)) continue;
            const TouchProbe probe = ProbeKey(ts, a, D(ai).touchFrame, key, plan, outMov, predAngle);
            if (probe.reaches) {
                smuggle = probe.smuggle;
                touchFrame = key.frame;
                return true;
            }
        }
        return false;
    }

    // A ball key of a candidate against the ball: the body at the key's frame of the plan, the
    // animation's ball there (scaled to the player's height), the mental ball moved along its path
    // to the point nearest it. The key fails on the height gap (TouchHeightMiss); otherwise the ball
    // must lie within the reach (TouchReach) of the animation's ball (BallWithinReach).
    HD TouchProbe ProbeKey(const TouchSearch &ts, const Anim &a, int defaultTouchFrame, const FootballKey &key, const PList &plan,
                           const Vec3 &outMov, float predAngle) {
        const int tf = key.frame;
        const Vec3 touchMov = RotatedBy(MovementAtFrame(plan.e, plan.count, tf, 0), ts.back);
        const Vec3 ballNow = ts.mental.At(tf * 10);
        const Vec3 ballMov = RotatedBy((ts.mental.At(tf * 10 + 10) - ballNow) * 100.0f, ts.back);
        const Vec3 ballAt = RotatedBy(ballNow - ts.position, ts.back);
        const Vec3 touchPos = RotatedBy(plan[tf], ts.back);
        Quat bodyOrientation;
        Vec3 bodyOrigin;
        float bodyAngle;
        GetKeyFrameZ(c, a, kBpPlayer, tf, bodyOrientation, bodyOrigin, bodyAngle);
        Vec3 animBall = (key.position - bodyOrigin) + touchPos;
        animBall.v[2] = key.position.v[2] * (ts.height / kDefaultPlayerHeight);
        // The ball's path from 6 ms before the key to 3 ms after, at its point nearest the
        // animation's ball.
        const Vec3 before = ballAt - ballMov * 0.006f, after = ballAt + ballMov * 0.003f;
        const Vec3 ball = before + (after - before) * Clamp(LineClosestToPoint(before, after, animBall), 0.0f, 1.0f);
        TouchProbe probe;
        probe.smuggle = (ball - animBall).Get2D();
        if (!(TouchHeightMiss(ts, a.baseAnimation, animBall.v[2], ball.v[2]) < 0.22f)) return probe;
        const int offTouch = defaultTouchFrame - tf;
        float awkward = NormalizedClamp((float)(offTouch < 0 ? -offTouch : offTouch), 0.0f, 4.0f);
        awkward = awkward * awkward * 0.5f;
        float late = libm::powf(tf / 24.0f, 0.7f);
        if (late > 1.0f) late = 1.0f + ((late - 1.0f) * 0.5f);
        TouchReach reach = KeyReach(ts.fn, awkward, ts.preferPassAndShot);
        const float touchSpeed = touchMov.Length();
        Vec3 foot = FootReachOffset(touchSpeed, bodyAngle, ball.v[2]);
        if (VelocityCat(touchSpeed) != kVelIdle) foot.Rotate2D(FixAngle(touchMov.Normalized(Vec3(0, -1, 0)).Angle2D()));
        // Right after the player's last touch the reach shrinks (less with good ball control).
        const float sinceTouch = Curve(LastTouchBiasAt(600, ts.now + (uint64_t)(int64_t)(tf * 10)), 1.0f);
        if (sinceTouch > 0.0f) {
            const float f = 1.0f - sinceTouch * 0.97f * (1.0f - ts.ballControl * 0.1f);
            reach.radius *= f;
            reach.cheat *= f;
        }
        Vec3 body = touchPos;
        body.v[2] = 0;
        const ReachMotion motion{ts.inMov, touchMov, outMov, predAngle, a.frameCount};
        probe.reaches = BallWithinReach(motion, body, foot, animBall.Get2D(), ball.Get2D(), reach.radius * late, reach.cheat) ||
                        ts.retainerIsMe;
        return probe;
    }

    // GRF's touch search over `sorted` (humanoid_base.cpp, GetBestCheatableAnimationID): the first
    // candidate, in list order, whose plan brings a ball key to the ball. Returns it (-1 for none)
    // with its plan, touch frame and position, the smuggle that moves the body onto the ball and
    // the plan's rotation offset.
    HDN int FindTouchAnimation(const AList &sorted, bool useDesiredMovement, const Vec3 &desiredDir, float desiredVel,
                               const Vec3 &desiredBodyRel, PList &positions, int &touchFrameOut, Vec3 &touchPosOut,
                               Vec3 &actionSmuggleOut, float &rotationSmuggleOut, bool preferPassAndShot = false) {
        ENG_SCOPE(31);
        const MatchState &m = w.match;
        const SpatialState &s = S();
        const float angle = s.angle.value();
        if (m.ballRetainer != -1 && m.ballRetainer != hi) return -1;
        // What the keys read of the match, which the evaluations leave unchanged.
        const TouchSearch ts(w, MentalImg(), hi, StringToFunctionType(A(sorted[0]).animationType), BackTurn(angle),
                             s.movement, s.position, c.sd->data[hi].height, Statistic(kStatBallControl), preferPassAndShot,
                             useDesiredMovement, desiredDir * desiredVel, desiredBodyRel);
        // A candidate passes only at a key where the ball is on the pitch and passes the height
        // test. The plan moves the ball's height at a key only between its heights just before
        // and just after the key, so a key whose ball height lies far enough from that span fails
        // the test whatever the plan. The lanes keep, in list order, the candidates with a key
        // that may pass; the others fail without a plan. The bound's factors are the smallest the
        // test can apply, with margins over the rounding.
        auto mayPass = [&](int ai) -> bool {
            if (ts.retainerIsMe) return true;
            const Anim &a = A(ai);
            for (int key = 0; key < a.footballCount; key++) {
                const FootballKey &fk = c.t->football[a.footballFirst + key];
                const int tf = fk.frame;
                if (!BallOnPitchAt(ts.predictions, ts.flip, tf)) continue;
                const float m0 = ts.mental.At(tf * 10).v[2], m1 = ts.mental.At(tf * 10 + 10).v[2];
                const float z = m0 - ts.position.v[2], dzdt = (m1 - m0) * 100.0f;
                const float zBefore = z - dzdt * 0.006f, zAfter = z + dzdt * 0.003f;
                const float slack = (fabsf(zBefore) + fabsf(zAfter)) * 1e-5f + 1e-6f;
                const float lo = MinF(zBefore, zAfter) - slack, hi = MaxF(zBefore, zAfter) + slack;
                const float az = fk.position.v[2] * (ts.height / kDefaultPlayerHeight);
                const float gap = az < lo ? lo - az : az > hi ? az - hi : 0.0f;
                float bound = gap * (1.0f - Clamp((float)(((double)az - 0.11) * (double)0.3f), 0.0f, 0.2f)) * 0.69f;
                if (ts.fn == kFnDeflect) bound *= 0.8f;
                if (a.baseAnimation && lo < 0.5f) bound -= 0.15f;
                if (!(bound > 0.2201f)) return true;
            }
            return false;
        };
        AList candidates{c.ws->lists[2], 0};
        for (int k0 = 0; k0 < sorted.count; k0 += kGroupLanes) {
            const int k = k0 + GroupRank();
            const bool keep = k < sorted.count && mayPass(sorted[k]);
            const LaneMask kept = GroupBallot(keep);
            if (keep) candidates.e[candidates.count + PopCount(kept & LanesBelow(GroupRank()))] = sorted[k];
            candidates.count += PopCount(kept);
        }
        GroupSync();
        // The lanes of the match evaluate consecutive candidates; the earliest that passes wins.
        // Without one the caller reads neither the plan nor the rotation.
        int best = -1;
        float rotSmuggle = 0, predAngle = 0;
        Vec3 outMov, smuggle;
        positions.count = 0;
        for (int e0 = 0; e0 < candidates.count && best < 0; e0 += kGroupLanes) {
            const int entry = e0 + GroupRank();
            PList mine{kGroupLanes == 1 ? positions.e : c.ws->lanePlans[GroupRank()], 0};
            float rot = 0, pa = 0;
            Vec3 ao, sm;
            int tf = 0;
            const bool ok = entry < candidates.count && TryTouchAnimation(ts, candidates[entry], mine, rot, pa, ao, sm, tf);
            const LaneMask passed = GroupBallot(ok);
            if (!passed) continue;
            const int from = LowestBit(passed);
            rotSmuggle = GroupShuffle(rot, from);
            const int count = GroupShuffle((int32_t)mine.count, from);
            best = candidates[e0 + from];
            predAngle = GroupShuffle(pa, from);
            outMov = GroupShuffle(ao, from);
            smuggle = GroupShuffle(sm, from);
            touchFrameOut = GroupShuffle((int32_t)tf, from);
            if (kGroupLanes > 1) {
                GroupSync();
                const Vec3 *src = c.ws->lanePlans[from];
                for (int i = GroupRank(); i < count; i += kGroupLanes) positions.e[i] = src[i];
                GroupSync();
            }
            positions.count = count;
        }
        if (best >= 0) {
            touchPosOut = MentalBallAt(touchFrameOut * 10);
            actionSmuggleOut = ShapeActionSmuggle(ts, RotatedBy(smuggle, Turn(angle)), touchPosOut.v[2], angle + predAngle,
                                                  outMov.Length(), touchFrameOut);
        }
        rotationSmuggleOut = rotSmuggle;
        return best;
    }

    // The smuggle that moves the body onto the ball through the touch: the gap less a discard
    // (more for ball control, less for a high ball) and 2 cm (more for interference), never more
    // than the gap less 20 cm, none for the ball's retainer; along the outgoing direction it only
    // shortens, by at most what a slow, late touch allows; less near an opponent.
    HD Vec3 ShapeActionSmuggle(const TouchSearch &ts, const Vec3 &gap, float ballHeight, float outgoingAngle, float outSpeed,
                               int touchFrame) {
        float keep = 1.0f - 0.4f * (ts.fn != kFnBallControl ? 0.8f : 1.0f) * (ballHeight > 0.5f ? 0.7f : 1.0f) *
                                (ballHeight > 1.0f ? 0.7f : 1.0f);
        float length = Clamp(gap.Length() - (0.02f + (ts.fn == kFnInterfere ? 0.1f : 0.0f)), 0.0f, (float)100.0);
        length *= keep;
        length = MinF(length, gap.Length() - 0.2f);
        if (ts.retainerIsMe) length = 0.0f;
        Vec3 smuggle = gap.Normalized(0) * length;
        smuggle.Rotate2D(-outgoingAngle);
        float forward = 0.25f * (1.0f - libm::powf(NormalizedClamp(outSpeed, kIdleVelocity, kSprintVelocity - 2.0f), 0.6f)) *
                        (touchFrame * 0.1f);
        if (ts.fn != kFnBallControl && ts.fn != kFnTrap) forward += 0.1f;
        if (smuggle.v[1] < 0.0f) smuggle.v[1] = Clamp(smuggle.v[1] + 0.02f, -forward, 0.0f);
        smuggle.Rotate2D(outgoingAngle);
        return smuggle * (0.7f + 0.3f * NormalizedClamp(ClosestOpponentDistance(w, hi), 0.6f, 1.2f));
    }

    HD void InstallAnimation(int sel, int fn, int interrupt, int touchFrame, const Vec3 &touchPos, float rotScale,
                             float rotSmuggleEnd, const Vec3 &actionSmuggle, const PList &positions, const PlayerCommand &cmd) {
        Humanoid &h = H();
        AnimationState &cur = h.anim;
        SpatialState &s = S();
        h.prevAnimFrameNum = cur.frameNum;
        h.prevAnimFunctionType = cur.functionType;
        const Anim &next = A(sel);
        cur.anim = sel;
        cur.id = sel;
        cur.functionType = fn;
        cur.frameNum = 0;
        cur.touchFrame = touchFrame;
        cur.originatingInterrupt = interrupt;
        cur.touchPos = touchPos;
        const float maxRot = 0.25f * PI;
        cur.rotationSmuggleBegin.set(
            Clamp(ModulateIntoRange(-PI, PI, s.relBodyAngleNonQuantized.value() - next.incomingBodyAngle.value()) * 1.0f,
                  -maxRot * rotScale, maxRot * rotScale));
        cur.rotationSmuggleEnd.set(rotSmuggleEnd);
        cur.rotationSmuggleOffset.set(0);
        cur.actionSmuggle = actionSmuggle;
        cur.actionSmuggleOffset = Vec3(0);
        cur.actionSmuggleSustain = Vec3(0);
        cur.actionSmuggleSustainOffset = Vec3(0);
        cur.movementSmuggle = Vec3(0);
        cur.movementSmuggleOffset = Vec3(0);
        cur.incomingMovement = s.movement;
        cur.outgoingMovement = OutgoingMovementOf(positions);
        // The plan fits the list: both hold kAnimPositions entries.
        GroupCopy<4>(cur.positions.e, positions.e, positions.count);
        cur.positions.count = positions.count;
        cur.positionOffset = Vec3(0);
        cur.originatingCommand = cmd;
    }

    HD void ApplyOutgoingState(int interrupt) {
        AnimationState &cur = H().anim;
        SpatialState &s = S();
        if (interrupt != kIntReQueue || cur.frameNum > 12) {
            const Anim &a = A(cur.anim);
            s.foot = a.outgoingFoot;
            if (a.outgoingSpecialState != kStrEmpty) {
                s.floatVelocity = 0;
                s.velocityCat = kVelIdle;
                s.movement = Vec3(0);
            }
        }
    }

    // The crude query of an official's command: strict incoming velocity and body direction.
    HD CrudeQuery OfficialQuery(const PlayerCommand &cmd, int fn) {
        const SpatialState &s = S();
        CrudeQuery q;
        q.byFunctionType = true;
        q.functionType = fn;
        q.byIncomingVelocity = true;
        q.incomingVelocity = s.velocityCat;
        q.incomingVelocityStrict = true;
        q.incomingVelocityForceLinearity = true;
        q.byIncomingBodyDirection = true;
        q.incomingBodyDirection = s.relBodyDirectionVec;
        q.incomingBodyDirectionStrict = true;
        q.incomingBodyDirectionForceLinearity = true;
        FinishQuery(q, cmd, fn, w.match.ballRetainer == hi);
        return q;
    }

    // An official's animation for a command (GRF's HumanoidBase::SelectAnimation): for movement,
    // trips and specials, the first candidate of the query by the ranking, with its movement plan;
    // other function types select nothing.
    HDN SelectResult SelectOfficialAnimation(const PlayerCommand &cmd, int interrupt) {
        AnimationState &cur = H().anim;
        const SpatialState &s = S();
        const int fn = cmd.desiredFunctionType;
        ApplyOutgoingState(interrupt);
        const float angle = s.angle.value();
        AList l{c.ws->lists[0], 0};
        FilterAnimations(c, OfficialQuery(cmd, fn), l);
        if (l.empty()) {
            if (fn != kFnMovement) return kSelectFalse;
            l.push_back(IdleMovementAnimation());
        }
        if (cmd.useDesiredMovement) {
            SetMovementSimilarityPredicate(RotatedBy(cmd.desiredDirection, BackTurn(angle)), VelocityCat(cmd.desiredVelocityFloat));
            pred.lookAt = cmd.desiredLookAt;
            if (fn == kFnMovement) {
                KeepNearestQuadrant(l, cmd, true);
                if (cmd.useDesiredLookAt) KeepNearestLook(l, cmd, true);
            } else {
                Sort(l, [&](int i) { return MovementSimilarityKey(i); });
            }
        }
        pred.idle = 1;
        pred.desiredFoot = s.foot;
        pred.relIncomingBodyDirection = s.relBodyDirectionVec;
        pred.incomingVelocity = s.velocityCat;
        if (cmd.useDesiredTripDirection) pred.relDesiredTripDirection = RotatedBy(cmd.desiredTripDirection, BackTurn(angle));
        if (l.empty() || !(fn == kFnMovement || fn == kFnTrip || fn == kFnSpecial)) return kSelectFalse;
        const int sel = FirstOfChain(l, fn, cmd.useDesiredTripDirection, 4, false);
        Vec3 lookRel = Vec3(0, -1, 0);
        if (cmd.useDesiredLookAt)
            lookRel = (RotatedBy((cmd.desiredLookAt - s.position).Get2D(), BackTurn(angle)) - A(sel).translation).Normalized(Vec3(0, -1, 0));
        PList plan{c.ws->plans[0], 0};
        float rotation = 0;
        PlanMovement(sel, cmd.useDesiredMovement, cmd.desiredDirection * cmd.desiredVelocityFloat, lookRel, plan, rotation, true);
        if (interrupt == kIntReQueue && cur.positions.count > 1 && plan.count > 1 && RestartsCurrent(sel, fn, 0.20f * PI, false))
            return kSelectFalse;
        InstallAnimation(sel, fn, interrupt, -1, Vec3(), 1.0f, rotation, Vec3(), plan, cmd);
        return kSelectTrue;
    }

    // Whether the ball is out of a touch's range (function types other than movement, trips,
    // specials and sliding): more than 10 m away in 200 ms; more than 2 m away at the touch and
    // further from where the humanoid will be then than it is now; or, for the non-retainer and
    // all but deflections, seen more than 2 m from where it will be a second ahead.
    HD bool BallOutOfTouchRange(int fn, bool retainerIsMe) {
        const SpatialState &s = S();
        const bool needsBall = fn != kFnMovement && fn != kFnTrip && fn != kFnSpecial && fn != kFnSliding;
        if (!needsBall) return false;
        if ((MentalBallAt(200).Get2D() - s.position).Length() > 10.0f) return true;
        const Vec3 atTouch = MentalBallAt(kDefaultTouchOffsetMs).Get2D();
        const Vec3 humanoidThen = s.position + s.movement * (float)kDefaultTouchOffsetMs * (float)0.001;
        if ((atTouch - s.position).Length() > 2.0f && (atTouch - humanoidThen).Length() > (MentalBallAt(0).Get2D() - s.position).Length())
            return true;
        return fn != kFnDeflect && !retainerIsMe && (MentalBallAt(1000) - BallPredict(w.match.ball, 1000)).Length() > 2.0f;
    }

    // GRF's rules for a command that arrives while an animation runs (a requeue): true when the
    // running animation stays. Movement never replaces another function; a running movement stays
    // for a player with the ball or far (12 m) from the designated player, in its last 6 frames or
    // while requeues are delayed; ball control stays after frame 8 or while delayed, and against a
    // trap; a trap stays within 6 frames of its touch or while delayed. Any of them stays for the
    // command it came from (within 1.5 m/s) and, in a movement, ball control or trap, for a
    // command close to what it already plans; movement stays against ball control just after a
    // kick of the player's own ball, unless the velocity changes by 1 m/s or more.
    HD bool RequeueKeepsCurrent(const PlayerCommand &cmd, int fn) {
        const Player &player = P();
        const Humanoid &h = H();
        const AnimationState &cur = h.anim;
        const SpatialState &s = S();
        const MatchState &m = w.match;
        const int running = cur.functionType;
        const bool delayed = h.requeueDelayFrames > 0;
        const bool runningMovement = running == kFnMovement, runningControl = running == kFnBallControl, runningTrap = running == kFnTrap;
        if (fn == kFnMovement) {
            if (!runningMovement) return true;
            const float focus = (Sp(w, m.designatedPossessionPlayer).position - s.position).Length();
            if (player.hasPossession || focus > 12.0f || cur.frameNum + 6 > A(cur.anim).frameCount - 1 || delayed) return true;
        }
        if (runningControl && fn == kFnBallControl && (cur.frameNum > 8 || delayed)) return true;
        if (runningControl && fn == kFnTrap) return true;
        if (runningTrap && (fn == kFnTrap || fn == kFnBallControl) && (cur.frameNum + 6 > cur.touchFrame || delayed)) return true;
        const Vec3 asked = cmd.desiredDirection * cmd.desiredVelocityFloat;
        const PlayerCommand &origin = cur.originatingCommand;
        if (origin.desiredFunctionType == fn && ((origin.desiredDirection * origin.desiredVelocityFloat) - asked).Length() < 1.5f)
            return true;
        const bool continues = (runningMovement && fn == kFnMovement) || (runningControl && fn == kFnBallControl) ||
                               (runningTrap && (fn == kFnBallControl || fn == kFnTrap));
        if (continues) {
            const Vec3 planned = cur.outgoingMovement - cur.incomingMovement;
            const Vec3 wanted = asked - s.movement;
            const float agreement = wanted.Dot(planned), gap = GetDistance(wanted, planned);
            if ((agreement > 0.0f && gap < 4.0f) || agreement > 0.8f || gap < 2.0f) return true;
        }
        const bool justKicked = m.actualTimeMs - player.base.lastTouchTimeMs < 600 && player.base.lastTouchType == kTouchKicked;
        return runningMovement && fn == kFnBallControl && justKicked && player.hasPossession && (s.movement - asked).Length() < 1.0f;
    }

    // The crude query of a player's command: the function type (long passes as short ones), the
    // ball direction it asks for, the incoming velocity (dribble as walk beyond movement; idle out
    // of a special state) and body direction under the function type's rules, the side the player
    // looks to, pickup, the incoming ball direction of traps, interference and deflections, last
    // ditch, trip type, and the special and retain states it comes from.
    HD CrudeQuery CommandQuery(const PlayerCommand &cmd, int fn, bool retainerIsMe) {
        const AnimationState &cur = H().anim;
        const SpatialState &s = S();
        const Anim &current = A(cur.anim);
        const libm::SinCos back = BackTurn(s.angle.value());
        CrudeQuery q;
        q.byFunctionType = true;
        q.functionType = fn == kFnLongPass ? kFnShortPass : fn;
        if (cmd.touchInfo.desiredPower != 0.0f) {
            q.byOutgoingBallDirection = true;
            q.outgoingBallDirection = RotatedBy(cmd.touchInfo.desiredDirection, back);
        }
        const VelocityRule velocity = FunctionVelocityRule(q.functionType);
        q.byIncomingVelocity = true;
        q.incomingVelocity = s.velocityCat;
        if (q.functionType != kFnMovement && q.incomingVelocity == kVelDribble) q.incomingVelocity = kVelWalk;
        q.incomingVelocityStrict = velocity.strict;
        q.incomingVelocityNoDribbleToIdle = velocity.noDribbleToIdle;
        q.incomingVelocityNoDribbleToSprint = velocity.noDribbleToSprint;
        q.incomingVelocityForceLinearity = velocity.forceLinearity;
        const BodyRule body = FunctionBodyRule(q.functionType);
        q.byIncomingBodyDirection = true;
        q.incomingBodyDirection = s.relBodyDirectionVec;
        q.incomingBodyDirectionStrict = body.strict;
        q.incomingBodyDirectionForceLinearity = body.forceLinearity;
        if (cmd.useDesiredLookAt && current.outgoingSpecialState == kStrEmpty && !retainerIsMe) {
            q.bySide = true;
            q.lookAtVectorRelative = RotatedBy((cmd.desiredLookAt - s.position).Normalized(s.directionVec), back);
        }
        if (cmd.onlyDeflectAnimationsThatPickupBall) {
            q.byPickupBall = true;
            q.pickupBall = true;
        }
        if (fn == kFnTrap || fn == kFnInterfere || fn == kFnDeflect) {
            q.byIncomingBallDirection = true;
            q.incomingBallDirection = RotatedBy(MentalBallAt(180) - MentalBallAt(120), back).Normalized(Vec3(0));
        }
        q.allowLastDitch = AllowLastDitch();
        FinishQuery(q, cmd, fn, retainerIsMe);
        return q;
    }
    // What every query takes from the command and the running animation: trip type, the special
    // and retain states it comes from, the special variables; idle velocity out of a special state.
    HD void FinishQuery(CrudeQuery &q, const PlayerCommand &cmd, int fn, bool retainerIsMe) {
        const AnimationState &cur = H().anim;
        const Anim &current = A(cur.anim);
        if (fn == kFnTrip) {
            q.byTripType = true;
            q.tripType = cmd.tripType;
        }
        q.incomingSpecialState = current.outgoingSpecialState;
        if (retainerIsMe) q.incomingRetainState = D(cur.anim).outgoingRetainRawValue;
        if (cmd.useSpecialVar1) q.specialVar1 = (float)cmd.specialVar1;
        if (cmd.useSpecialVar2) q.specialVar2 = (float)cmd.specialVar2;
        if (current.outgoingSpecialState != kStrEmpty) q.incomingVelocity = kVelIdle;
    }

    // Narrows the candidates to the desired movement and look (the keep-best filters) for
    // movement, ball control, traps and interference; false when a trap's best candidate leaves
    // too far from the desired movement. Each filter is one call site, so matches of a wavefront
    // that select for different function types run it together; per environment they run in
    // GRF's order (body direction first for ball control only).
    HD bool NarrowToDesired(AList &l, const PlayerCommand &cmd, int fn, bool allowLastDitch) {
        const SpatialState &s = S();
        SetMovementSimilarityPredicate(RotatedBy(cmd.desiredDirection, BackTurn(s.angle.value())), VelocityCat(cmd.desiredVelocityFloat));
        pred.lookAt = cmd.desiredLookAt;
        const bool keeps = fn == kFnMovement || fn == kFnBallControl || fn == kFnTrap || fn == kFnInterfere;
        bool strict = true;
        float allowed = 0.0f;
        int velocitySteps = 0;
        if (fn == kFnBallControl) {
            strict = !AllowLastDitch();
            allowed = 0.0f * PI;
        } else if (fn == kFnTrap) {
            strict = !(AllowLastDitch(false) || HighOrBouncyBall());
            allowed = 0.3f * PI;
            velocitySteps = 2;
        } else if (fn == kFnInterfere) {
            strict = cmd.strictMovement == kStrictTrue;
            allowed = 0.3f * PI;
            velocitySteps = 1;
        }
        if (fn == kFnBallControl && cmd.useDesiredLookAt) KeepNearestLook(l, cmd, strict, allowed);
        if (keeps) KeepNearestQuadrant(l, cmd, strict, allowed, velocitySteps, -1);
        if (keeps && fn != kFnBallControl && cmd.useDesiredLookAt) KeepNearestLook(l, cmd, strict, allowed);
        if (fn == kFnTrap && !HighOrBouncyBall() && !allowLastDitch) return TrapLeavesTowardDesired(l[0], cmd);
        return true;
    }
    // A trap's best candidate must leave within 0.375 pi of the desired direction and near the
    // desired movement (within walking speed ahead, sprinting speed behind, plus 0.5 m/s).
    HD bool TrapLeavesTowardDesired(int best, const PlayerCommand &cmd) {
        const SpatialState &s = S();
        const float angle = s.angle.value();
        const Anim &a = A(best);
        const Vec3 leaving = RotatedBy(a.outgoingMovement, Turn(angle));
        const float ahead = cmd.desiredDirection.Dot(s.directionVec);
        if (fabsf(RotatedBy(a.outgoingDirection, Turn(angle)).Angle2D(cmd.desiredDirection)) > 0.375f * PI) return false;
        const float gap = (leaving - cmd.desiredDirection * cmd.desiredVelocityFloat).Length();
        return !((gap > kWalkVelocity + 0.5f && ahead > 0.0f) || (gap > kSprintVelocity + 0.5f && ahead <= 0.0f));
    }
    // The idle level a player's candidates are ranked by: 1 at a set piece or with the ball more
    // than 16 m away in 200 ms, else 2 out of play and 0 in play.
    HD int IdleLevel() {
        const MatchState &m = w.match;
        if (m.inSetPiece) return 1;
        if ((BallPredict(m.ball, 200) - S().position).Length() > 16.0f) return 1;
        return m.inPlay ? 0 : 2;
    }
    // The sort keys of a candidate of a movement, trip or special, which take only the first of
    // GRF's chain of stable sorts: base animation (all but movement), trip direction (with one),
    // incoming velocity, body direction, foot, idle level and priority, most significant first.
    HD int FirstOfChain(const AList &l, int fn, bool byTrip, int keyCount, bool withPriority) {
        const bool byBase = fn != kFnMovement;
        const int qi = l.count > 1 ? IncomingBodyDirectionQuery() : 0;
        return FirstOfSortChain(l, keyCount + byTrip + byBase, [&](int i, double *k) {
            int n = 0;
            if (byBase) k[n++] = A(i).baseAnimation ? 0 : 1;
            if (byTrip) k[n++] = -D(i).bumpDirection.Dot(pred.relDesiredTripDirection);
            k[n++] = KeyIncomingVelocity(A(i), pred);
            k[n++] = IncomingBodyDirectionKey(i, qi);
            k[n++] = KeyFoot(A(i), pred);
            k[n++] = KeyIdle(A(i), pred);
            if (withPriority) k[n++] = D(i).priorityAbsolute;
        });
    }
    // GRF's chain of stable sorts of a touch's candidates, least significant first: priority, idle
    // level, foot, body direction (all but ball control), incoming velocity, trip direction, base
    // animation; deflections that retain the ball to the front.
    HD void OrderTouchCandidates(AList &l, const PlayerCommand &cmd, int fn) {
        Sort(l, [&](int i) { return D(i).priorityAbsolute; });
        Sort(l, [&](int i) { return KeyIdle(A(i), pred); });
        Sort(l, [&](int i) { return KeyFoot(A(i), pred); });
        if (fn != kFnBallControl) {
            const int qi = l.count > 1 ? IncomingBodyDirectionQuery() : 0;
            Sort(l, [&](int i) { return IncomingBodyDirectionKey(i, qi); });
        }
        Sort(l, [&](int i) { return KeyIncomingVelocity(A(i), pred); });
        if (cmd.useDesiredTripDirection) Sort(l, [&](int i) { return -D(i).bumpDirection.Dot(pred.relDesiredTripDirection); });
        if (fn != kFnMovement) SortBaseAnimation(l);
    }
    // Whether a requeued selection would only restart what runs: the same function type with the
    // same outgoing quadrant (a moving animation) or, both idle, preferred outgoing angles within
    // `idleTolerance`.
    HD bool RestartsCurrent(int sel, int fn, float idleTolerance, bool bothIdle) {
        const AnimationState &cur = H().anim;
        const Anim &current = A(cur.anim), &next = A(sel);
        const bool currentIdle = VelocityCat(current.outgoingVelocity) == kVelIdle;
        const bool idleAsWell = !bothIdle || VelocityCat(next.outgoingVelocity) == kVelIdle;
        return cur.functionType == fn &&
               ((!currentIdle && current.quadrantID == next.quadrantID) ||
                ((currentIdle && idleAsWell) && fabsf(PreferredOutgoingAngle(cur.anim) - PreferredOutgoingAngle(sel)) < idleTolerance));
    }

    // A player's animation for a command (GRF's HumanoidBase::SelectAnimation for players): the
    // candidates of the command's query, narrowed to the desired movement and ranked; a movement,
    // trip or special takes the first by the ranking, a touch the first whose plan reaches the
    // ball (sliding falls back to its first), then the plan is installed. kSelectFalse when none
    // fits or a requeue keeps what runs.
    HDN SelectResult SelectPlayerAnimation(const PlayerCommand &cmd, int interrupt, bool preferPassAndShot) {
        ENG_SCOPE(14);
        AnimationState &cur = H().anim;
        const SpatialState &s = S();
        const int fn = cmd.desiredFunctionType;
        const bool retainerIsMe = w.match.ballRetainer == hi;
        if (BallOutOfTouchRange(fn, retainerIsMe)) return kSelectFalse;
        if (interrupt == kIntReQueue) {
            if (w.match.designatedPossessionPlayer < 0) return kSelectUnsupported;
            if (RequeueKeepsCurrent(cmd, fn)) return kSelectFalse;
        }
        ApplyOutgoingState(interrupt);
        const float angle = s.angle.value();
        const CrudeQuery q = CommandQuery(cmd, fn, retainerIsMe);
        AList l{c.ws->lists[0], 0};
        FilterAnimations(c, q, l);
        if (l.empty()) {
            if (fn != kFnMovement) return kSelectFalse;
            l.push_back(IdleMovementAnimation());
        }
        if (cmd.useDesiredMovement && !NarrowToDesired(l, cmd, fn, q.allowLastDitch)) return kSelectFalse;
        // The predicates of the ranking, set in GRF's order: idle level, foot, body direction
        // (all but ball control), incoming velocity, trip direction.
        pred.idle = (float)IdleLevel();
        pred.desiredFoot = s.foot;
        if (fn != kFnBallControl) pred.relIncomingBodyDirection = s.relBodyDirectionVec;
        pred.incomingVelocity = s.velocityCat;
        if (cmd.useDesiredTripDirection) pred.relDesiredTripDirection = RotatedBy(cmd.desiredTripDirection, BackTurn(angle));
        const bool firstOnly = fn == kFnMovement || fn == kFnTrip || fn == kFnSpecial;
        if (!firstOnly) OrderTouchCandidates(l, cmd, fn);
        if (fn == kFnDeflect) Sort(l, [&](int i) { return D(i).outgoingRetainRaw ? 0 : 1; });
        if (l.empty() && fn == kFnMovement) l.push_back(IdleMovementAnimation());
        Vec3 lookRel = Vec3(0, -1, 0);
        if (cmd.useDesiredLookAt)
            lookRel = RotatedBy((cmd.desiredLookAt - (s.position + s.movement * 0.1f)).Normalized(Vec3(0, -1, 0)), BackTurn(angle));
        // The touch search and the movement plan, one call site each, so that matches selecting
        // for different function types run them together.
        int sel = -1, touchFrame = -1;
        PList plan{c.ws->plans[0], 0};
        Vec3 touchPos, smuggle;
        float rotation = 0;
        bool search = false, prefer = false, physics = false;
        if (firstOnly) {
            sel = FirstOfChain(l, fn, cmd.useDesiredTripDirection, 5, true);
            physics = true;
        } else if (fn == kFnBallControl) {
            search = BallControlNeedsTouch(l[0], cmd);
            prefer = preferPassAndShot;
        } else if (fn == kFnTrap || fn == kFnInterfere || fn == kFnDeflect) {
            search = true;
            prefer = preferPassAndShot;
        } else if (fn == kFnShortPass || fn == kFnLongPass || fn == kFnHighPass || fn == kFnShot || fn == kFnSliding) {
            search = true;
        }
        if (search)
            sel = FindTouchAnimation(l, cmd.useDesiredMovement, cmd.desiredDirection, cmd.desiredVelocityFloat, lookRel, plan,
                                     touchFrame, touchPos, smuggle, rotation, prefer);
        if (fn == kFnSliding && sel == -1 && !l.empty()) {
            sel = l[0];
            physics = true;
        }
        if (physics) {
            ENG_SCOPE(48);
            PlanMovement(sel, cmd.useDesiredMovement, cmd.desiredDirection * cmd.desiredVelocityFloat, lookRel, plan, rotation, true);
        }
        if (interrupt == kIntReQueue && sel != -1 && cur.positions.count > 1 && plan.count > 1 && RestartsCurrent(sel, fn, 0.06f * PI, true))
            sel = -1;
        if (sel == -1) return kSelectFalse;
        InstallAnimation(sel, fn, interrupt, touchFrame, touchPos, fn == kFnMovement ? 1.0f : 0.5f, rotation, smuggle, plan, cmd);
        cur.movementSmuggle = MovementSmuggle();
        cur.movementSmuggleOffset = Vec3(0);
        return kSelectTrue;
    }
};

}  // namespace eng
