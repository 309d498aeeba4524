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

HD int GetVelocityID(int v, bool dribbleAsWalk = false) {
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
HDN Vec3 ForceIntoPreferredDirectionVector(const Vec3 &src) {
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
HDN float ForceIntoPreferredDirectionAngle(float a) {
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
HDN float ForceIntoAllowedBodyDirectionAngle(float a) {
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

HD float CalculateBiasForFastCornering(const Vec3 &cur, const Vec3 &desired, float velExp, float bias) {
    float angle = desired.Normalized(cur).Angle2D(cur);
    float cb = libm::sinf(fabsf(angle) - 0.5f * PI) * 0.5f + 0.5f;
    float vb = libm::powf(Clamp(cur.Length() / (kSprintVelocity - 0.5f), 0.0f, 1.0f), velExp);
    return vb * cb * bias;
}

HD float StretchSprintTo(float v, float inMax, float targetMax) {
    if (v < kWalkSprintSwitch) return v;
    float part = v - kWalkSprintSwitch;
    float oldL = inMax - kWalkSprintSwitch, newL = targetMax - kWalkSprintSwitch;
    return kWalkSprintSwitch + part * (newL / oldL);
}

HD Vec3 GetFrontOfFootOffsetRelative(float velocity, float bodyAngleRel, float height) {
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

HDN void CrudeSelection(const Ctx &c, const CrudeQuery &query, AList &out) {
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

// The crude query of GetIdleMovementAnimationID: movement from idle to idle.
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
    int cur = GetVelocityID(p.incomingVelocity);
    int in = GetVelocityID(VelocityCat(a.incomingVelocity));
    float r = fabsf(Clamp((float)(in - cur), -3, 3));
    int out = GetVelocityID(VelocityCat(a.outgoingVelocity));
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
    HD int IncomingBodyDirectionQuery() { return ForceIntoAllowedBodyDirectionIndex(pred.relIncomingBodyDirection); }
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
        pred.corneringBias = CalculateBiasForFastCornering(Vec3(0, -1.0f * S().floatVelocity, 0),
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

    HDN void KeepBestDirectionAnimations(AList &l, const PlayerCommand &cmd, bool strict, float allowedAngle = 0,
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
                int dv = GetVelocityID(qd.velocity, true) - GetVelocityID(bq.velocity, true);
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

    HDN void KeepBestBodyDirectionAnimations(AList &l, const PlayerCommand &cmd, bool strict, float allowedAngle = 0) {
        ENG_SCOPE(32);
        if (l.empty()) return;
        Vec3 relLookAt;
        if (l.count > 1) relLookAt = RelativeLookAt();
        // As in KeepBestDirectionAnimations: the first element of GRF's sorted list passes its
        // own test, so the kept elements are filtered first and sorted after.
        auto key = [&](int i) { return DirectionSimilarityRating(A(i), pred, relLookAt); };
        const bool byBase = strict && cmd.desiredFunctionType != kFnMovement;
        const float bestLook = LookAngle(l[StableFirst(l, key, byBase)]);
        const float allowed = strict ? 0.06f * PI : allowedAngle;
        KeepInOrder(l, [&](int ai) { return fabsf(LookAngle(ai) - bestLook) <= allowed; });
        Sort(l, key);
        if (byBase) SortBaseAnimation(l);
    }

    HDN int GetIdleMovementAnimationID() {
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

    HDN Vec3 CalculatePhysicsVector(int ai, bool useDesiredMovement, const Vec3 &desiredMovement, bool useDesiredBody,
                                    const Vec3 &desiredBodyRel, PList &out, float &rotationOffset) {
        ENG_SCOPE(38);
        (void)useDesiredBody;
        const Anim &a = A(ai);
        const AnimDerived &d = D(ai);
        SpatialState &s = S();
        const float angle = s.angle.value();
        const libm::SinCos turn = Turn(angle);
        out.count = 0;
        int touchFrame = d.touchFrame;
        bool touch = (touchFrame > 0);
        float agility = Statistic(kStatAgility), accel = Statistic(kStatAcceleration), dribble = Statistic(kStatDribble);
        float inSwitch = 0.0f, outSwitch = 0.0f;
        const int at = a.animationType;
        if (at == kAtBallControl) outSwitch = 0.0f;
        else if (at == kAtTrap) outSwitch = 0.0f;
        else if (at == kAtInterfere) outSwitch = 0.0f;
        else if (at == kAtDeflect) outSwitch = 1.0f;
        else if (at == kAtSliding) outSwitch = 0.0f;
        else if (at == kAtSpecial) outSwitch = 1.0f;
        else if (at == kAtTrip) outSwitch = 0.5f;
        else if (touch) outSwitch = 1.0f;
        if (a.incomingSpecialState != kStrEmpty || a.outgoingSpecialState != kStrEmpty) outSwitch = 1.0f;
        Vec3 animIn = RotatedBy(Vec3(0, -1, 0), turn) * RangeVelocity(a.incomingVelocity);
        Vec3 adaptedCur = animIn * inSwitch + s.movement * (1.0f - inSwitch);
        Vec3 predOut = RotatedBy(a.outgoingMovement, turn);
        Vec3 velDesired = useDesiredMovement ? desiredMovement : predOut;
        Vec3 adaptedDesired = predOut * outSwitch + velDesired * (1.0f - outSwitch);
        const float playerMaxVel = GetMaximumVelocity(*c.sd, hi);
        float maxVel = playerMaxVel;
        if (touch) maxVel *= 0.92f;
        const int stepMs = 10;
        float difficulty = d.difficultyFactor;
        float difficultyPenalty =
            libm::PowfPos(Clamp((difficulty - 0.0f) * (1.0f - (agility * 0.2f + accel * 0.2f)) * 2.0f, 0.0f, 1.0f), 0.7f);
        float powerFactor = 1.0f - Clamp(libm::PowfPos(BaseLastTouchBias(1000), 0.8f) * (0.8f - dribble * 0.3f), 0.0f, 0.4f);
        powerFactor *= 1.0f - Clamp(H().decayingPositionOffset.Length() * (10.0f - Statistic(kStatBalance) * 5.0f) - 0.1f,
                                    0.0f, 0.3f);
        Vec3 temporal = adaptedCur;
        Vec3 curPos;
        float physicsBias = 1.0f;
        float maxUnder = 0.125f * PI, maxOver = 0.125f * PI, maxStraight = 0.125f * PI;
        if (touch) {
            float bonus = 1.0f - libm::PowfPos(NormalizedClamp((adaptedCur + predOut).Length() * 0.5f, 0, kSprintVelocity), 0.8f) * 0.8f;
            bonus *= 0.6f + 0.4f * Statistic(kStatBallControl);
            maxUnder = 0.2f * PI * bonus;
            maxOver = 0;
            maxStraight = 0.1f * PI * bonus;
        }
        if (at == kAtSliding) maxUnder = maxOver = maxStraight = 0.5f * PI;
        if (at == kAtMovement) physicsBias *= 1.0f;
        if (at == kAtBallControl) physicsBias *= 1.0f;
        if (at == kAtTrap) physicsBias *= 1.0f;
        if (at == kAtShortPass) physicsBias *= 0.0f;
        if (at == kAtHighPass) physicsBias *= 0.0f;
        if (at == kAtShot) physicsBias *= 0.0f;
        if (at == kAtInterfere) physicsBias *= 0.5f;
        if (at == kAtDeflect) physicsBias *= 0.0f;
        if (at == kAtSliding) physicsBias *= 1.0f;
        if (at == kAtTrip) physicsBias *= d.tripTypeIsOne ? 0.5f : 0.0f;
        if (at == kAtSpecial) physicsBias *= 0.0f;
        if (a.incomingSpecialState != kStrEmpty) physicsBias *= 0.0f;
        const float accelMul = 0.5f + 0.5f;
        float capped = 0;
        if (physicsBias > 0.0f) {
            Vec3 animOut = predOut.Normalized(0);
            if (VelocityCat(predOut.Length()) == kVelIdle) animOut = RotatedBy(a.outgoingDirection, turn);
            Vec3 desiredVec = adaptedDesired.Normalized(0);
            if (VelocityCat(adaptedDesired.Length()) == kVelIdle) desiredVec = RotatedBy(desiredBodyRel, turn);
            float toDesired = desiredVec.Angle2D(animOut);
            if (fabsf(toDesired) <= 0.5f * PI || at == kAtSliding) {
                float change = animOut.Angle2D(s.directionVec);
                if (fabsf(change) > 0.06f * PI) {
                    int sign = SignSide(change);
                    if (SignSide(toDesired) == sign) capped = Clamp(toDesired, -maxOver, maxOver);
                    else capped = Clamp(toDesired, -maxUnder, maxUnder);
                } else {
                    capped = Clamp(toDesired, -maxStraight, maxStraight);
                }
            }
        }
        const int effFrames = a.frameCount - 1;
        const float adaptedDesiredVel = adaptedDesired.Length();
        const Vec3 adaptedDesiredDir = adaptedDesired.Normalized(0);
        if (a.frameCount > kAnimPositions) Fatal("a fixed-capacity list outgrows its capacity");
        // The frames read only these values of the animation, held in registers across the
        // plan's stores.
        const int frameCount = a.frameCount, lastFramesMs = (a.frameCount - 2) * 10;
        const bool outgoingIdle = VelocityCat(a.outgoingVelocity) == kVelIdle;
        const Vec3 outgoingTurned = RotatedBy(a.outgoingMovement, turn);
        const int32_t smoothedFirst = c.t->selection[ai].smoothedFirst;
        const Vec3 *const smoothed = c.t->smoothed + (smoothedFirst >= 0 ? smoothedFirst : 0);
        const Vec3 *const animPositions = c.t->positions + a.posFirst;
        const int posCount = a.posCount;
        Vec3 *const plan = out.e;
        for (int frame = 0; frame < frameCount; frame++) {
            const int tms = frame * stepMs;
            float frameBias = (tms + 10) / (float)((effFrames + 1) * 10);
            // The frame's part independent of the carried movement.
            float lagExp = 1.0f;
            if (physicsBias > 0.0f && (at == kAtBallControl || at == kAtMovement)) {
                lagExp = 1.4f - 0.5f * 0.8f;
                lagExp *= 1.2f - agility * 0.4f;
                if (touch) lagExp += -0.1f + Clamp(difficulty * 0.4f, 0.0f, 0.5f);
                else lagExp += -0.2f + Clamp(difficulty * 0.2f, 0.0f, 0.2f);
                lagExp = Clamp(lagExp, 0.25f, 4.0f);
                if (touch && tms < touchFrame * 10) lagExp = MaxF(lagExp, 0.7f);
                lagExp = lagExp * physicsBias + 1.0f * (1.0f - physicsBias);
            }
            float adaptedFrameBias = lagExp == 1.0f ? frameBias : libm::powf(frameBias, lagExp);
            const uint32_t animFrame = TruncToUint32(effFrames * adaptedFrameBias);
            Vec3 animMov = RotatedBy(smoothedFirst >= 0 && animFrame < (uint32_t)posCount
                                         ? smoothed[animFrame]
                                         : MovementAtFrame(animPositions, posCount, animFrame, 1),
                                     turn);
            float animVel = animMov.Length();
            Vec3 adaptedAnimMov = animMov;
            float adaptedAnimVel = animVel;
            if (animVel > kWalkSprintSwitch && (at == kAtMovement || at == kAtBallControl || at == kAtTrap)) {
                if (maxVel > animVel) {
                    adaptedAnimVel = StretchSprintTo(animVel, kAnimSprintVelocity, maxVel);
                    adaptedAnimMov = adaptedAnimMov.Normalized(0) * adaptedAnimVel;
                }
            }
            const Vec3 normMax = NormalizedMaximum(adaptedAnimMov, 1.0f);
            const Vec3 normAdapted = adaptedAnimMov.Normalized(0);
            const float rotation = capped * frameBias;
            float rc, rs;
            // Below 2^-12 the sine is the argument and the cosine 1, by the test of sinf/cosf.
            if (libm::Top12f(rotation) < libm::Top12f(0x1p-12f)) {
                rc = 1.0f;
                rs = rotation;
            } else {
                libm::SinCos ft = libm::sincosf(rotation);
                rc = ft.c;
                rs = ft.s;
            }
            const float curvedTime = PhysicsCurvedTime(frame);
            // The part carried from frame to frame.
            float maxSlower = touch ? 1.2f : 1.6f;
            float maxFaster = 0.0f;
            const float tLen = temporal.Length();
            if (tLen > adaptedAnimVel) maxFaster = MinF(0.0f + 1.0f * (1.0f - frameBias), MaxF(maxFaster, tLen - adaptedAnimVel));
            if (maxFaster > 0) maxFaster *= MaxF(0.0f, normMax.Dot(adaptedDesiredDir));
            if (at == kAtSliding) maxFaster = 100;
            adaptedAnimVel = Clamp(adaptedDesiredVel, adaptedAnimVel - maxSlower, adaptedAnimVel + maxFaster);
            adaptedAnimMov = normAdapted * adaptedAnimVel;
            Vec3 result = RotatedCS(adaptedAnimMov, rc, rs);
            result = result * physicsBias + animMov * (1.0f - physicsBias);
            Vec3 toDesired = (result - temporal);
            float penaltyBreak = 0.0f;
            {
                Vec3 predicted = temporal + toDesired;
                float startVel = kIdleDribbleSwitch;
                if (tLen > startVel && predicted.Length() > startVel) {
                    const Vec3 pd = predicted.Normalized(), td = temporal.Normalized();
                    float maf = 1.0f * (stepMs / 1000.0f);
                    maf *= (0.7f + 0.3f * agility);
                    if (!touch) maf *= 1.5f;
                    float maxAngle = maf * PI;
                    float vf = NormalizedClamp(tLen, 0, kSprintVelocity);
                    maxAngle = maxAngle / (vf + 0.01f);
                    float corner = pd.Angle2D(td);
                    if (fabsf(corner) > maxAngle) {
                        float over = fabsf(corner) - maxAngle;
                        toDesired += -temporal * Clamp(over / PI * 3.0f, 0.0f, 1.0f);
                    }
                }
            }
            {
                float maxChange = 0.03f;
                if (at == kAtTrip) maxChange *= 0.7f;
                if (at == kAtSliding) maxChange = 0.1f;
                float vf = libm::PowfPos(NormalizedClamp(tLen, 0, kSprintVelocity), 1.5f);
                float fsf = vf;
                if (at == kAtMovement) fsf *= 0.4f;
                maxChange *= (1.0f - fsf) + fsf * curvedTime;
                maxChange *= 1.2f - vf * 0.4f;
                maxChange *= 0.75f + 0.5f * 0.5f;
                maxChange *= powerFactor;
                float dl = toDesired.Length();
                float maxAdd = maxChange * stepMs;
                NormalizeMaximum(toDesired, MinF(dl, maxAdd));
            }
            if (at != kAtSliding && at != kAtDeflect) {
                float velExp = 1.8f;
                float accPower = 11.0f * accelMul;
                float falloff = kIdleDribbleSwitch;
                const float nextLen = (temporal + toDesired).Length();
                if (nextLen > falloff) {
                    accPower *= 1.0f - difficultyPenalty * 0.4f;
                    float air = Clamp(libm::PowfPos(Clamp((tLen - falloff) / (playerMaxVel - falloff), 0.0f, 1.0f), velExp), 0.0f, 1.0f);
                    Vec3 fwdv;
                    if (nextLen > tLen) {
                        Vec3 dest = temporal + toDesired;
                        float acc = nextLen - tLen;
                        fwdv = dest.Normalized(0) * acc;
                    }
                    float add = fwdv.Length();
                    float maxAccPerSec = accPower * (1.0f - air) * (accel * 0.3f + 0.7f);
                    float maxAccAdd = maxAccPerSec * (stepMs / 1000.0f);
                    if (add > maxAccAdd) {
                        float remaining = maxAccAdd / add;
                        toDesired = toDesired - fwdv * (1.0f - remaining);
                    }
                }
            }
            Vec3 tmp = temporal + toDesired;
            if (tms >= lastFramesMs) {
                if (outgoingIdle && VelocityCat(tmp.Length()) != kVelIdle)
                    tmp = Vec3(0);
                else if (!outgoingIdle && VelocityCat(tmp.Length()) == kVelIdle)
                    tmp = NormalizedTo(outgoingTurned, kDribbleVelocity);
            }
            temporal = tmp;
            if (tms >= lastFramesMs) penaltyBreak = 0.0f;
            curPos += temporal * (1.0f - penaltyBreak) * (stepMs / 1000.0f);
            plan[frame] = curPos;
        }
        out.count = a.frameCount > 0 ? a.frameCount : 0;
        Vec3 resulting = temporal;
        if (VelocityCat(a.outgoingVelocity) != kVelIdle && VelocityCat(resulting.Length()) != kVelIdle)
            rotationOffset = RotatedBy(resulting, BackTurn(angle)).Angle2D(a.outgoingMovement);
        else
            rotationOffset = capped * physicsBias;
        return resulting;
    }

    HDN bool NeedTouch(int ai, const PlayerCommand &cmd) {
        const Anim &a = A(ai);
        SpatialState &s = S();
        // GRF: never true, a bool as float is idle, kept as written.
        if (VelocityCat((float)(a.outgoingVelocity != (float)kVelIdle)) != kVelIdle) return true;
        if (cmd.desiredVelocityFloat > kIdleDribbleSwitch) return true;
        if (fabsf(w.match.ball.momentum.Length()) > 2.0f) return true;
        Vec3 am = RotatedBy(a.outgoingMovement, Turn(s.angle.value())) * 0.3f + s.movement * 0.7f;
        float av = am.Length();
        am.Normalize(s.directionVec);
        am *= s.movement.Length() * 0.8f + av * 0.2f;
        Vec3 bm = (MentalBallAt(250).Get2D() - MentalBallAt(240).Get2D()) * 100;
        if (fabsf(a.outgoingAngle.value()) > 0.125f * PI) return true;
        float dd = (am - bm).Length();
        if ((double)dd >= 2.0) return true;
        float vd = am.Length() - bm.Length();
        if ((double)vd < -1.4 || (double)vd >= 0.7) return true;
        if (VelocityCat(a.outgoingVelocity) != kVelIdle) {
            float ad = am.Normalized(s.directionVec).Dot(bm.Normalized(s.directionVec));
            if ((double)ad < 0.975) return true;
        }
        return false;
    }

    HDN void CalculatePredictedSituation(Vec3 &predPos, float &predAngle) {
        ENG_SCOPE(22);
        AnimationState &cur = H().anim;
        const Anim &a = A(cur.anim);
        SpatialState &s = S();
        if ((uint32_t)cur.positions.count > (uint32_t)cur.frameNum)
            predPos = s.position + cur.positions[a.frameCount - 1] + cur.actionSmuggle + cur.actionSmuggleSustain + cur.movementSmuggle;
        else
            predPos = s.position + a.translation.Get2D().Rotated2D(s.angle.value()) + cur.actionSmuggle + cur.actionSmuggleSustain +
                      cur.movementSmuggle;
        predAngle = s.angle.value() + a.outgoingAngle.value() + cur.rotationSmuggleEnd.value();
        predAngle = ModulateIntoRange(-PI, PI, predAngle);
    }

    HD int DesiredTimeToBallMs() {
        return TruncToInt32(Clamp((float)P().desiredTimeToBallMs, (float)(int)P().timeToBallMs, 1000000.0f));
    }

    HDN Vec3 CalculateMovementSmuggle() {
        AnimationState &cur = H().anim;
        const Anim &a = A(cur.anim);
        const MatchState &m = w.match;
        if (TeamOfPlayer(w, hi).designatedTeamPossessionPlayer != hi || m.designatedPossessionPlayer != hi ||
            cur.touchFrame != -1 || (cur.functionType == kFnTrip && !D(cur.anim).tripTypeIsOne) ||
            a.incomingSpecialState != kStrEmpty || a.outgoingSpecialState != kStrEmpty || !m.inPlay || m.inSetPiece ||
            m.ballRetainer != -1)
            return Vec3(0);
        Vec3 toDesired;
        uint32_t ttb = (uint32_t)(int)P().timeToBallMs;
        if (DesiredTimeToBallMs() > (int)ttb) ttb = (uint32_t)DesiredTimeToBallMs();
        uint32_t animMs = (uint32_t)a.frameCount * 10;
        uint32_t future = animMs + kDefaultTouchOffsetMs > ttb ? animMs + kDefaultTouchOffsetMs : ttb;
        Vec3 predOut = OutgoingMovementOf(PList{cur.positions.e, cur.positions.count});
        Vec3 predPos;
        float predAngle;
        CalculatePredictedSituation(predPos, predAngle);
        Vec3 ballPos = MentalBallAt((int)future);
        float bh = ballPos.v[2];
        Vec3 foot = GetFrontOfFootOffsetRelative(predOut.Length(), a.outgoingBodyAngle.value(), bh).Rotated2D(predAngle);
        Vec3 desiredBall = predPos + foot;
        if (!P().hasPossession) {
            Vec3 bs = MentalBallAt(0).Get2D(), be = MentalBallAt((int)future).Get2D();
            if ((bs - be).Length() < 0.5f) return Vec3(0);
            float fraction = 0.0f;
            if (!(bs == be)) {
                float ld = (be - bs).Length();
                if (!(ld < 0.000001f))
                    fraction = ((desiredBall.v[0] - bs.v[0]) * (be.v[0] - bs.v[0]) + (desiredBall.v[1] - bs.v[1]) * (be.v[1] - bs.v[1])) /
                               (ld * ld);
            }
            Vec3 closest = bs + (be - bs) * fraction;
            toDesired = closest - desiredBall;
        } else {
            toDesired = ballPos.Get2D() - desiredBall;
        }
        uint32_t maxEffectMs = 250 + kDefaultTouchOffsetMs;
        if (VelocityCat(a.outgoingVelocity) == kVelIdle) maxEffectMs = 2000;
        float maxEffectVel = kDribbleWalkSwitch, maxSmugglePerSec = 1.6f;
        if (future - (animMs + kDefaultTouchOffsetMs) > maxEffectMs) return Vec3(0);
        Vec3 toDesiredMov = toDesired / (animMs * 0.001f);
        Vec3 resulting = predOut + toDesiredMov;
        float pv = predOut.Length(), rv = resulting.Length();
        if (rv > pv && rv > maxEffectVel) return Vec3(0);
        NormalizeMaximum(toDesired, maxSmugglePerSec * ((a.frameCount - 1) * 0.01f));
        toDesired = toDesired.Normalized(0) * MaxF(0.0f, toDesired.Length() - 0.06f);
        return toDesired;
    }

    HD float LastTouchBiasAt(int decayMs, uint64_t t) {
        uint64_t at = t;
        if (t == 0) at = w.match.actualTimeMs;
        if (decayMs > 0) return 1.0f - Clamp((float)(at - P().base.lastTouchTimeMs) / (float)decayMs, 0.0f, 1.0f);
        return 0.0f;
    }

    HDN static float BodyBallDistanceAdvantage(const Anim &a, const Vec3 &touchMov, const Vec3 &inMov, const Vec3 &outMov,
                                               float outAngle, const Vec3 &bodyPos, const Vec3 &footOff,
                                               const Vec3 &animBall2D, const Vec3 &actualBall2D, float radiusFactor,
                                               float radiusCheat) {
        const float cheatFactor = 0.5f, cheatBonus = 0.02f;
        float inV = inMov.Length(), outV = outMov.Length();
        float avgV = (inMov + outMov).Length() * 0.5f;
        float vChange = outV - inV;
        float vChangePerSec = vChange / (a.frameCount * 0.01f);
        float bodyAnimBall = 1.0f - Curve(NormalizedClamp(((bodyPos + footOff.Normalized(0) * 0.1f) - animBall2D).Length(), 0.0f, 0.7f), 0.7f);
        float bodyActualBall =
            1.0f - Curve(NormalizedClamp(((bodyPos + footOff.Normalized(0) * 0.1f) - actualBall2D).Length(), 0.0f, 0.7f), 0.4f);
        float velBonus = 1.0f - NormalizedClamp(avgV, kIdleVelocity, kSprintVelocity);
        float velChangeBonus = 1.0f - NormalizedClamp(vChangePerSec / 20.0f, -1.0f, 1.0f);
        float radius = radiusFactor;
        radius *= 1.0f + 1.0f * bodyAnimBall + 0.6f * bodyActualBall + 0.8f * bodyAnimBall * bodyActualBall +
                  0.0f * velChangeBonus + 1.0f * velBonus;
        float effCheat = radiusCheat;
        Vec3 outDir;
        if (VelocityCat(outMov.Length()) == kVelIdle) outDir = Vec3(0, -1, 0).Rotated2D(outAngle);
        else outDir = outMov.Normalized();
        Vec3 behindU = -(inMov * 0.1f + touchMov * 0.2f + outMov * 0.7f);
        Vec3 behind = behindU.Normalized(0) * libm::PowfPos(NormalizedClamp(behindU.Length(), 0, kSprintVelocity), 0.5f);
        float dot = Vec3(0, -1, 0).Dot(outDir);
        dot = 0.5f + Clamp(dot * 0.5f + 0.5f, 0.0f, 1.0f) * 0.5f;
        behind *= dot;
        Vec3 a2b = actualBall2D - animBall2D;
        {
            Vec3 su = inMov;
            Vec3 sv = su.Normalized(outDir);
            float toStraight = Vec3(0, -1, 0).Angle2D(sv);
            a2b.Rotate2D(toStraight);
            float lateral = 0.6f - 0.3f * libm::PowfPos(NormalizedClamp(su.Length(), kIdleVelocity, kSprintVelocity), 0.7f);
            a2b.v[0] /= lateral;
            radius *= libm::powf(1.0f / lateral, 0.5f);
            a2b.Rotate2D(-toStraight);
        }
        Vec3 adaptedActual = animBall2D + a2b;
        Vec3 behindCenter = animBall2D + behind * (radius + (effCheat * 0.6f)) * cheatFactor;
        float allowed = (radius + effCheat) * cheatFactor + cheatBonus;
        return GetDistance(adaptedActual, behindCenter) > allowed ? 0.0f : 1.0f;
    }

    HDN int GetBestCheatableAnimationID(const AList &sorted, bool useDesiredMovement, const Vec3 &desiredDir, float desiredVel,
                                        bool useDesiredBody, const Vec3 &desiredBodyRel, PList &positions, int &touchFrameOut,
                                        Vec3 &touchPosOut, Vec3 &actionSmuggleOut, float &rotationSmuggleOut,
                                        bool preferPassAndShot = false) {
        ENG_SCOPE(31);
        const MatchState &m = w.match;
        SpatialState &s = S();
        const float angle = s.angle.value();
        const bool retainerIsMe = m.ballRetainer == hi;
        if (m.ballRetainer != -1 && !retainerIsMe) return -1;
        const libm::SinCos bk = BackTurn(angle);
        Vec3 inMov = RotatedBy(s.movement, bk);
        int best = -1;
        Vec3 bestSmuggle2D;
        Vec3 desiredMovement = desiredDir * desiredVel;
        float height = c.sd->data[hi].height;
        const int fn = StringToFunctionType(A(sorted[0]).animationType);
        float tmpRotSmuggle = 0, predAngle = 0;
        Vec3 adaptedOut;
        bool found = false;
        // What the keys read of the match, which the evaluations leave unchanged.
        const MentalBallView mental(w, MentalImg());
        const Vec3 position = s.position;
        const Vec3 *const ballPredictions = m.ball.predictions;
        const bool ballFlip = m.ball.lazyFlip;
        const FootballKey *const footballKeys = c.t->football;
        const float ballControl = Statistic(kStatBallControl);
        const uint64_t now = m.actualTimeMs;
        // One candidate: its physics plan into `plan`, then its ball keys from the middle one down,
        // then up; true with the touch at the first key the body reaches.
        auto evaluate = [&](int ai, PList &plan, float &rotSmuggle, float &predAngleOut, Vec3 &adaptedOutOut, Vec3 &smuggleOut,
                            int &touchFrame) -> bool {
            bool hit = false;
            const Anim &a = A(ai);
            bool isBase = a.baseAnimation;
            CalculatePhysicsVector(ai, useDesiredMovement, desiredMovement, useDesiredBody, desiredBodyRel, plan, rotSmuggle);
            predAngleOut = a.outgoingAngle.value() + rotSmuggle;
            predAngleOut = ModulateIntoRange(-PI, PI, predAngleOut);
            const float predAngle = predAngleOut;
            PList &positions = plan;
            Vec3 outMov = RotatedBy(OutgoingMovementOf(positions), bk);
            adaptedOutOut = outMov;
            const Vec3 adaptedOut = outMov;
            const int total = a.footballCount;
            int defaultTouchFrame = D(ai).touchFrame;
            for (int tn = 0; tn < total && !hit; tn++) {
                const int key = tn <= total / 2 ? total / 2 - tn : tn;
                const FootballKey &fk = footballKeys[a.footballFirst + key];
                Vec3 animBall = fk.position;
                int tf = fk.frame;
                if (!retainerIsMe) {
                    Vec3 abs = BallPredictRaw(ballPredictions, tf * 10);
                    if (ballFlip) abs.Mirror();
                    if (fabsf(abs.v[0]) > kPitchHalfLength + kLineHalfWidth + 0.11f ||
                        fabsf(abs.v[1]) > kPitchHalfWidth + kLineHalfWidth + 0.11f)
                        continue;
                }
                Vec3 touchMov = RotatedBy(MovementAtFrame(positions.e, positions.count, tf, 0), bk);
                Vec3 ballPos = mental.At(tf * 10);
                Vec3 ballMov = (mental.At(tf * 10 + 10) - ballPos) * 100.0f;
                ballPos = RotatedBy(ballPos - position, bk);
                ballMov = RotatedBy(ballMov, bk);
                const Vec3 touchPos = RotatedBy(positions[tf], bk);
                Vec3 bodyPos = touchPos;
                bodyPos.v[2] = 0;
                Quat abr;
                Vec3 abp;
                float z;
                GetKeyFrameZ(c, a, kBpPlayer, tf, abr, abp, z);
                float abh = animBall.v[2];
                animBall = (animBall - abp) + touchPos;
                animBall.v[2] = abh * (height / kDefaultPlayerHeight);
                {
                    Vec3 before = ballPos - ballMov * 0.006f, after = ballPos + ballMov * 0.003f;
                    float fr = Clamp(LineClosestToPoint(before, after, animBall), 0.0f, 1.0f);
                    ballPos = before + (after - before) * fr;
                }
                Vec3 smuggle3D = ballPos - animBall;
                Vec3 smuggle2D = smuggle3D.Get2D();
                float dz = fabsf(smuggle3D.v[2]);
                dz *= 1.0f - Clamp((float)(((double)animBall.v[2] - 0.11) * (double)0.3f), 0.0f, 0.2f);
                dz *= 1.0f - Clamp((float)(((double)ballPos.v[2] - 0.11) * (double)0.4f), 0.0f, 0.3f);
                if (ballPos.v[2] > 1.8f && ballPos.v[2] > animBall.v[2] + 0.12f) dz *= 2.0f;
                if (ballPos.v[2] > 2.6f && ballPos.v[2] > animBall.v[2] + 0.08f) dz *= 20.0f;
                if (fn == kFnDeflect) dz *= 0.8f;
                if (retainerIsMe) dz = 0.0f;
                if (ballPos.v[2] < 0.5f && isBase) dz = MaxF(dz - 0.15f, 0.0f);
                if (dz < 0.22f) {
                    int dtf = defaultTouchFrame - tf;
                    float awk = NormalizedClamp((float)(dtf < 0 ? -dtf : dtf), 0.0f, 4.0f);
                    awk = awk * awk * 0.5f;
                    float tff = tf / 24.0f;
                    tff = libm::powf(tff, 0.7f);
                    if (tff > 1.0f) tff = 1.0f + ((tff - 1.0f) * 0.5f);
                    float cheatOff = 0.0f;
                    float rf = 0.3f * (1.0f - awk);
                    if (fn == kFnDeflect) {
                        rf *= 1.8f;
                        cheatOff += 0.4f;
                    }
                    if (fn == kFnSliding) {
                        rf *= 0.2f;
                        cheatOff = 0.0f;
                    }
                    if (fn == kFnInterfere) {
                        rf *= 1.4f;
                        cheatOff += 0.2f;
                    }
                    if (fn == kFnShortPass || fn == kFnLongPass || fn == kFnHighPass || fn == kFnShot) {
                        rf *= 1.3f;
                        cheatOff += 0.15f;
                    }
                    if ((fn == kFnTrap || fn == kFnBallControl) && preferPassAndShot) rf *= 0.3f;
                    cheatOff *= (1.0f - awk);
                    float tv = touchMov.Length();
                    Vec3 foot = GetFrontOfFootOffsetRelative(tv, z, ballPos.v[2]);
                    if (VelocityCat(tv) != kVelIdle) foot.Rotate2D(FixAngle(touchMov.Normalized(Vec3(0, -1, 0)).Angle2D()));
                    float ltb = Curve(LastTouchBiasAt(600, now + (uint64_t)(int64_t)(tf * 10)), 1.0f);
                    if (ltb > 0.0f) {
                        float f = 1.0f - ltb * 0.97f * (1.0f - ballControl * 0.1f);
                        rf *= f;
                        cheatOff *= f;
                    }
                    float adv = BodyBallDistanceAdvantage(a, touchMov, inMov, adaptedOut, predAngle, bodyPos, foot, animBall.Get2D(),
                                                          ballPos.Get2D(), rf * tff, cheatOff);
                    if (adv >= 1.0f || retainerIsMe) {
                        hit = true;
                        smuggleOut = smuggle2D;
                        touchFrame = tf;
                    }
                }
            }
            return hit;
        };
        // A candidate passes only at a key where the ball is on the pitch and passes the height
        // test (dz < 0.22). The plan moves the ball's height at a key only between its heights just
        // before and just after the key, so a key whose ball height lies far enough from that span
        // fails the test whatever the plan. The lanes keep, in list order, the candidates with a
        // key that may pass; the others fail without a plan. The bound's factors are the smallest
        // the test can apply, with margins over the rounding.
        auto mayPass = [&](int ai) -> bool {
            if (retainerIsMe) return true;
            const Anim &a = A(ai);
            for (int key = 0; key < a.footballCount; key++) {
                const FootballKey &fk = footballKeys[a.footballFirst + key];
                const int tf = fk.frame;
                Vec3 abs = BallPredictRaw(ballPredictions, tf * 10);
                if (ballFlip) abs.Mirror();
                if (fabsf(abs.v[0]) > kPitchHalfLength + kLineHalfWidth + 0.11f ||
                    fabsf(abs.v[1]) > kPitchHalfWidth + kLineHalfWidth + 0.11f)
                    continue;
                const float m0 = mental.At(tf * 10).v[2], m1 = mental.At(tf * 10 + 10).v[2];
                const float z = m0 - position.v[2], dzdt = (m1 - m0) * 100.0f;
                const float zBefore = z - dzdt * 0.006f, zAfter = z + dzdt * 0.003f;
                const float slack = (fabsf(zBefore) + fabsf(zAfter)) * 1e-5f + 1e-6f;
                const float lo = MinF(zBefore, zAfter) - slack, hi = MaxF(zBefore, zAfter) + slack;
                const float az = fk.position.v[2] * (height / kDefaultPlayerHeight);
                const float gap = az < lo ? lo - az : az > hi ? az - hi : 0.0f;
                float bound = gap * (1.0f - Clamp((float)(((double)az - 0.11) * (double)0.3f), 0.0f, 0.2f)) * 0.69f;
                if (fn == kFnDeflect) bound *= 0.8f;
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
        positions.count = 0;
        for (int e0 = 0; e0 < candidates.count && !found; e0 += kGroupLanes) {
            const int entry = e0 + GroupRank();
            PList mine{kGroupLanes == 1 ? positions.e : c.ws->lanePlans[GroupRank()], 0};
            float rot = 0, pa = 0;
            Vec3 ao, sm;
            int tf = 0;
            const bool ok = entry < candidates.count && evaluate(candidates[entry], mine, rot, pa, ao, sm, tf);
            const LaneMask passed = GroupBallot(ok);
            if (!passed) continue;
            const int from = LowestBit(passed);
            tmpRotSmuggle = GroupShuffle(rot, from);
            const int count = GroupShuffle((int32_t)mine.count, from);
            found = true;
            best = candidates[e0 + from];
            predAngle = GroupShuffle(pa, from);
            adaptedOut = GroupShuffle(ao, from);
            bestSmuggle2D = GroupShuffle(sm, from);
            touchFrameOut = GroupShuffle((int32_t)tf, from);
            if (kGroupLanes > 1) {
                GroupSync();
                const Vec3 *src = c.ws->lanePlans[from];
                for (int i = GroupRank(); i < count; i += kGroupLanes) positions.e[i] = src[i];
                GroupSync();
            }
            positions.count = count;
        }
        if (found) {
            touchPosOut = MentalBallAt(touchFrameOut * 10);
            actionSmuggleOut = RotatedBy(bestSmuggle2D, Turn(angle));
            float sd = actionSmuggleOut.Length();
            float discard = 0.4f;
            if (fn != kFnBallControl) discard *= 0.8f;
            if (touchPosOut.v[2] > 0.5f) discard *= 0.7f;
            if (touchPosOut.v[2] > 1.0f) discard *= 0.7f;
            float discardBonus = 0.0f;
            if (fn == kFnInterfere) discardBonus += 0.1f;
            sd = Clamp(sd - (0.02f + discardBonus), 0.0f, (float)100.0);
            sd *= 1.0f - discard;
            sd = MinF(sd, actionSmuggleOut.Length() - 0.2f);
            if (retainerIsMe) sd = 0.0f;
            actionSmuggleOut = actionSmuggleOut.Normalized(0) * sd;
            {
                float toStraight = angle + predAngle;
                actionSmuggleOut.Rotate2D(-toStraight);
                float shorten = 0.02f;
                float allowFwd = 0.25f *
                                 (1.0f - libm::powf(NormalizedClamp(adaptedOut.Length(), kIdleVelocity, kSprintVelocity - 2.0f), 0.6f)) *
                                 (touchFrameOut * 0.1f);
                if (fn != kFnBallControl && fn != kFnTrap) allowFwd += 0.1f;
                if (actionSmuggleOut.v[1] < 0.0f) actionSmuggleOut.v[1] = Clamp(actionSmuggleOut.v[1] + shorten, -allowFwd, 0.0f);
                actionSmuggleOut.Rotate2D(toStraight);
            }
            actionSmuggleOut *= 0.7f + 0.3f * NormalizedClamp(ClosestOpponentDistance(w, hi), 0.6f, 1.2f);
        }
        rotationSmuggleOut = tmpRotSmuggle;
        return best;
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

    HDN SelectResult BaseSelectAnimation(const PlayerCommand &cmd, int interrupt) {
        AnimationState &cur = H().anim;
        SpatialState &s = S();
        const int fn = cmd.desiredFunctionType;
        ApplyOutgoingState(interrupt);
        const Anim &current = A(cur.anim);
        const float angle = s.angle.value();
        CrudeQuery q;
        q.byFunctionType = true;
        q.functionType = fn;
        q.byIncomingVelocity = true;
        q.incomingVelocity = s.velocityCat;
        q.incomingVelocityStrict = true;
        q.byIncomingBodyDirection = true;
        q.incomingBodyDirectionStrict = true;
        q.incomingBodyDirection = s.relBodyDirectionVec;
        q.incomingVelocityForceLinearity = true;
        q.incomingBodyDirectionForceLinearity = true;
        if (fn == kFnTrip) {
            q.byTripType = true;
            q.tripType = cmd.tripType;
        }
        q.incomingSpecialState = current.outgoingSpecialState;
        if (w.match.ballRetainer == hi) q.incomingRetainState = D(cur.anim).outgoingRetainRawValue;
        if (cmd.useSpecialVar1) q.specialVar1 = (float)cmd.specialVar1;
        if (cmd.useSpecialVar2) q.specialVar2 = (float)cmd.specialVar2;
        if (current.outgoingSpecialState != kStrEmpty) q.incomingVelocity = kVelIdle;
        AList l{c.ws->lists[0], 0};
        CrudeSelection(c, q, l);
        if (l.empty()) {
            if (fn == kFnMovement) l.push_back(GetIdleMovementAnimationID());
            else return kSelectFalse;
        }
        if (cmd.useDesiredMovement) {
            Vec3 rel = RotatedBy(cmd.desiredDirection, BackTurn(angle));
            SetMovementSimilarityPredicate(rel, VelocityCat(cmd.desiredVelocityFloat));
            pred.lookAt = cmd.desiredLookAt;
            if (fn == kFnMovement) {
                KeepBestDirectionAnimations(l, cmd, true);
                if (cmd.useDesiredLookAt) KeepBestBodyDirectionAnimations(l, cmd, true);
            } else {
                Sort(l, [&](int i) { return MovementSimilarityKey(i); });
            }
        }
        pred.idle = 1;
        pred.desiredFoot = s.foot;
        pred.relIncomingBodyDirection = s.relBodyDirectionVec;
        pred.incomingVelocity = s.velocityCat;
        if (cmd.useDesiredTripDirection) pred.relDesiredTripDirection = RotatedBy(cmd.desiredTripDirection, BackTurn(angle));
        int sel = -1;
        PList plan{c.ws->plans[0], 0};
        float rotSmuggle = 0;
        if (l.empty()) return kSelectFalse;
        const bool byTrip = cmd.useDesiredTripDirection, byBase = fn != kFnMovement;
        const int qi = l.count > 1 ? IncomingBodyDirectionQuery() : 0;
        const int first = FirstOfSortChain(l, 4 + byTrip + byBase, [&](int i, double *k) {
            int n = 0;
            if (byBase) k[n++] = A(i).baseAnimation ? 0 : 1;
            if (byTrip) k[n++] = -D(i).bumpDirection.Dot(pred.relDesiredTripDirection);
            k[n++] = KeyIncomingVelocity(A(i), pred);
            k[n++] = IncomingBodyDirectionKey(i, qi);
            k[n++] = KeyFoot(A(i), pred);
            k[n++] = KeyIdle(A(i), pred);
        });
        if (fn == kFnMovement || fn == kFnTrip || fn == kFnSpecial) {
            sel = first;
            const Anim &na = A(sel);
            Vec3 dm = cmd.desiredDirection * cmd.desiredVelocityFloat;
            Vec3 dbr = Vec3(0, -1, 0);
            if (cmd.useDesiredLookAt)
                dbr = (RotatedBy((cmd.desiredLookAt - s.position).Get2D(), BackTurn(angle)) - na.translation).Normalized(Vec3(0, -1, 0));
            CalculatePhysicsVector(sel, cmd.useDesiredMovement, dm, cmd.useDesiredLookAt, dbr, plan, rotSmuggle);
        }
        if (interrupt == kIntReQueue && sel != -1 && cur.positions.count > 1 && plan.count > 1) {
            const Anim &sa = A(sel);
            bool curIdle = VelocityCat(current.outgoingVelocity) == kVelIdle;
            if (cur.functionType == fn && ((!curIdle && current.quadrantID == sa.quadrantID) ||
                                           (curIdle && fabsf(PreferredOutgoingAngle(cur.anim) - PreferredOutgoingAngle(sel)) < 0.20f * PI)))
                sel = -1;
        }
        if (sel == -1) return kSelectFalse;
        InstallAnimation(sel, fn, interrupt, -1, Vec3(), 1.0f, rotSmuggle, Vec3(), plan, cmd);
        return kSelectTrue;
    }

    HDN SelectResult SelectAnimation(const PlayerCommand &cmd, int interrupt, bool preferPassAndShot) {
        ENG_SCOPE(14);
        Player &player = P();
        Humanoid &h = H();
        AnimationState &cur = h.anim;
        SpatialState &s = S();
        const MatchState &m = w.match;
        const int fn = cmd.desiredFunctionType;
        const bool retainerIsMe = m.ballRetainer == hi;
        if (fn != kFnMovement && fn != kFnTrip && fn != kFnSpecial && fn != kFnSliding) {
            if ((MentalBallAt(200).Get2D() - s.position).Length() > 10.0f) return kSelectFalse;
            if ((MentalBallAt(kDefaultTouchOffsetMs).Get2D() - s.position).Length() > 2.0f &&
                (MentalBallAt(kDefaultTouchOffsetMs).Get2D() - (s.position + s.movement * (float)kDefaultTouchOffsetMs * (float)0.001)).Length() >
                    (MentalBallAt(0).Get2D() - s.position).Length())
                return kSelectFalse;
        }
        if (fn != kFnMovement && fn != kFnTrip && fn != kFnSpecial && fn != kFnSliding && fn != kFnDeflect && !retainerIsMe) {
            if ((MentalBallAt(1000) - BallPredict(m.ball, 1000)).Length() > 2.0f) return kSelectFalse;
        }
        if (interrupt == kIntReQueue) {
            if (m.designatedPossessionPlayer < 0) return kSelectUnsupported;
            float focus = (Sp(w, m.designatedPossessionPlayer).position - s.position).Length();
            const int cf = cur.functionType;
            const int eff = A(cur.anim).frameCount - 1;
            if (cf != kFnMovement && fn == kFnMovement) return kSelectFalse;
            if (cf == kFnMovement && fn == kFnMovement && (player.hasPossession || focus > 12.0f)) return kSelectFalse;
            if (cf == kFnMovement && fn == kFnMovement && cur.frameNum + 6 > eff) return kSelectFalse;
            if (cf == kFnMovement && fn == kFnMovement && h.requeueDelayFrames > 0) return kSelectFalse;
            if (cf == kFnBallControl && fn == kFnBallControl && (cur.frameNum > 8 || h.requeueDelayFrames > 0)) return kSelectFalse;
            if (cf == kFnBallControl && fn == kFnTrap) return kSelectFalse;
            if (cf == kFnTrap && fn == kFnTrap && (cur.frameNum + 6 > cur.touchFrame || h.requeueDelayFrames > 0)) return kSelectFalse;
            if (cf == kFnTrap && fn == kFnBallControl && (cur.frameNum + 6 > cur.touchFrame || h.requeueDelayFrames > 0))
                return kSelectFalse;
            const PlayerCommand &oc = cur.originatingCommand;
            if (oc.desiredFunctionType == fn &&
                ((oc.desiredDirection * oc.desiredVelocityFloat) - (cmd.desiredDirection * cmd.desiredVelocityFloat)).Length() < 1.5f)
                return kSelectFalse;
            if ((cf == kFnMovement && fn == kFnMovement) || (cf == kFnBallControl && fn == kFnBallControl) ||
                (cf == kFnTrap && fn == kFnBallControl) || (cf == kFnTrap && fn == kFnTrap)) {
                Vec3 planned = cur.outgoingMovement - cur.incomingMovement;
                Vec3 desired = (cmd.desiredDirection * cmd.desiredVelocityFloat) - s.movement;
                if ((desired.Dot(planned) > 0.0f && GetDistance(desired, planned) < 4.0f) || desired.Dot(planned) > 0.8f ||
                    GetDistance(desired, planned) < 2.0f)
                    return kSelectFalse;
            }
            if (cf == kFnMovement && fn == kFnBallControl &&
                (m.actualTimeMs - player.base.lastTouchTimeMs < 600 && player.base.lastTouchType == kTouchKicked) && player.hasPossession) {
                float change = (s.movement - (cmd.desiredDirection * cmd.desiredVelocityFloat)).Length();
                if (change < 1.0f) return kSelectFalse;
            }
        }
        ApplyOutgoingState(interrupt);
        const Anim &current = A(cur.anim);
        const float angle = s.angle.value();
        CrudeQuery q;
        q.byFunctionType = true;
        q.functionType = fn;
        if (q.functionType == kFnLongPass) q.functionType = kFnShortPass;
        if (cmd.touchInfo.desiredPower != 0.0f) {
            q.byOutgoingBallDirection = true;
            q.outgoingBallDirection = RotatedBy(cmd.touchInfo.desiredDirection, BackTurn(angle));
        }
        q.byIncomingVelocity = true;
        q.incomingVelocity = s.velocityCat;
        if (q.functionType != kFnMovement && q.incomingVelocity == kVelDribble) q.incomingVelocity = kVelWalk;
        {
            const VelocityRule rule = FunctionVelocityRule(q.functionType);
            q.incomingVelocityStrict = rule.strict;
            q.incomingVelocityNoDribbleToIdle = rule.noDribbleToIdle;
            q.incomingVelocityNoDribbleToSprint = rule.noDribbleToSprint;
            q.incomingVelocityForceLinearity = rule.forceLinearity;
        }
        q.byIncomingBodyDirection = true;
        q.incomingBodyDirection = s.relBodyDirectionVec;
        {
            const BodyRule rule = FunctionBodyRule(q.functionType);
            q.incomingBodyDirectionStrict = rule.strict;
            q.incomingBodyDirectionForceLinearity = rule.forceLinearity;
        }
        q.bySide = false;
        if (cmd.useDesiredLookAt && (current.outgoingSpecialState == kStrEmpty) && !retainerIsMe) {
            Vec3 look = (cmd.desiredLookAt - s.position).Normalized(s.directionVec);
            q.lookAtVectorRelative = RotatedBy(look, BackTurn(angle));
            q.bySide = true;
        }
        if (cmd.onlyDeflectAnimationsThatPickupBall) {
            q.byPickupBall = true;
            q.pickupBall = true;
        }
        if (fn == kFnTrap || fn == kFnInterfere || fn == kFnDeflect) {
            q.byIncomingBallDirection = true;
            q.incomingBallDirection = RotatedBy(MentalBallAt(180) - MentalBallAt(120), BackTurn(angle)).Normalized(Vec3(0));
        }
        q.allowLastDitch = AllowLastDitch();
        if (fn == kFnTrip) {
            q.byTripType = true;
            q.tripType = cmd.tripType;
        }
        q.incomingSpecialState = current.outgoingSpecialState;
        if (retainerIsMe) q.incomingRetainState = D(cur.anim).outgoingRetainRawValue;
        if (cmd.useSpecialVar1) q.specialVar1 = (float)cmd.specialVar1;
        if (cmd.useSpecialVar2) q.specialVar2 = (float)cmd.specialVar2;
        if (current.outgoingSpecialState != kStrEmpty) q.incomingVelocity = kVelIdle;
        AList l{c.ws->lists[0], 0};
        CrudeSelection(c, q, l);
        if (l.empty()) {
            if (fn == kFnMovement) l.push_back(GetIdleMovementAnimationID());
            else return kSelectFalse;
        }
        if (cmd.useDesiredMovement) {
            Vec3 rel = RotatedBy(cmd.desiredDirection, BackTurn(angle));
            SetMovementSimilarityPredicate(rel, VelocityCat(cmd.desiredVelocityFloat));
            pred.lookAt = cmd.desiredLookAt;
            // The keep-best filters of each function type, as one call site per filter: matches of
            // a wavefront that select for different function types run each filter together. Per
            // environment the filters run in GRF's order (body direction first for ball control
            // only).
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
            if (fn == kFnBallControl && cmd.useDesiredLookAt) KeepBestBodyDirectionAnimations(l, cmd, strict, allowed);
            if (keeps) KeepBestDirectionAnimations(l, cmd, strict, allowed, velocitySteps, -1);
            if (keeps && fn != kFnBallControl && cmd.useDesiredLookAt) KeepBestBodyDirectionAnimations(l, cmd, strict, allowed);
            if (fn == kFnTrap && !HighOrBouncyBall() && q.allowLastDitch == false) {
                Vec3 dm = cmd.desiredDirection * cmd.desiredVelocityFloat;
                const Anim &ba = A(l[0]);
                Vec3 bestOut = RotatedBy(ba.outgoingMovement, Turn(angle));
                float cdd = cmd.desiredDirection.Dot(s.directionVec);
                bool allow = true;
                float ad = fabsf(RotatedBy(ba.outgoingDirection, Turn(angle)).Angle2D(cmd.desiredDirection));
                if (ad > 0.375f * PI) allow = false;
                Vec3 diff = bestOut - dm;
                if ((diff.Length() > kWalkVelocity + 0.5f && cdd > 0.0f) || (diff.Length() > kSprintVelocity + 0.5f && cdd <= 0.0f))
                    allow = false;
                if (!allow) return kSelectFalse;
            }
        }
        // A movement, trip or special needs only the first of the sort chain.
        const bool firstOnly = fn == kFnMovement || fn == kFnTrip || fn == kFnSpecial;
        if (!firstOnly) Sort(l, [&](int i) { return D(i).priorityAbsolute; });
        int idleLevel = 0;
        if (!m.inPlay) idleLevel = 2;
        if (m.inSetPiece) idleLevel = 1;
        else if ((BallPredict(m.ball, 200) - s.position).Length() > 16.0f) idleLevel = 1;
        pred.idle = (float)idleLevel;
        if (!firstOnly) Sort(l, [&](int i) { return KeyIdle(A(i), pred); });
        pred.desiredFoot = s.foot;
        if (!firstOnly) Sort(l, [&](int i) { return KeyFoot(A(i), pred); });
        if (fn != kFnBallControl) {
            pred.relIncomingBodyDirection = s.relBodyDirectionVec;
            if (!firstOnly) {
                const int qi = l.count > 1 ? IncomingBodyDirectionQuery() : 0;
                Sort(l, [&](int i) { return IncomingBodyDirectionKey(i, qi); });
            }
        }
        pred.incomingVelocity = s.velocityCat;
        if (!firstOnly) Sort(l, [&](int i) { return KeyIncomingVelocity(A(i), pred); });
        if (cmd.useDesiredTripDirection) {
            pred.relDesiredTripDirection = RotatedBy(cmd.desiredTripDirection, BackTurn(angle));
            if (!firstOnly) Sort(l, [&](int i) { return -D(i).bumpDirection.Dot(pred.relDesiredTripDirection); });
        }
        if (fn != kFnMovement && !firstOnly) SortBaseAnimation(l);
        if (fn == kFnDeflect) Sort(l, [&](int i) { return D(i).outgoingRetainRaw ? 0 : 1; });
        int sel = -1;
        PList plan{c.ws->plans[0], 0};
        int tmpTouchFrame = -1;
        Vec3 tmpTouchPos, tmpSmuggle;
        float tmpRot = 0;
        if (l.empty() && fn == kFnMovement) l.push_back(GetIdleMovementAnimationID());
        Vec3 dbr = Vec3(0, -1, 0);
        if (cmd.useDesiredLookAt)
            dbr = RotatedBy((cmd.desiredLookAt - (s.position + s.movement * 0.1f)).Normalized(Vec3(0, -1, 0)), BackTurn(angle));
        // The candidate search of the touch function types and the physics plan of the others, as
        // one call site each, so that matches selecting for different function types run them
        // together.
        bool cheat = false, prefer = false, physics = false;
        if (firstOnly) {
            const bool byTrip = cmd.useDesiredTripDirection, byBase = fn != kFnMovement;
            const int qi = l.count > 1 ? IncomingBodyDirectionQuery() : 0;
            sel = FirstOfSortChain(l, 5 + byTrip + byBase, [&](int i, double *k) {
                int n = 0;
                if (byBase) k[n++] = A(i).baseAnimation ? 0 : 1;
                if (byTrip) k[n++] = -D(i).bumpDirection.Dot(pred.relDesiredTripDirection);
                k[n++] = KeyIncomingVelocity(A(i), pred);
                k[n++] = IncomingBodyDirectionKey(i, qi);
                k[n++] = KeyFoot(A(i), pred);
                k[n++] = KeyIdle(A(i), pred);
                k[n++] = D(i).priorityAbsolute;
            });
            physics = true;
        } else if (fn == kFnBallControl) {
            cheat = NeedTouch(l[0], cmd);
            prefer = preferPassAndShot;
        } else if (fn == kFnTrap || fn == kFnInterfere || fn == kFnDeflect) {
            cheat = true;
            prefer = preferPassAndShot;
        } else if (fn == kFnShortPass || fn == kFnLongPass || fn == kFnHighPass || fn == kFnShot || fn == kFnSliding) {
            cheat = true;
        }
        if (cheat)
            sel = GetBestCheatableAnimationID(l, cmd.useDesiredMovement, cmd.desiredDirection, cmd.desiredVelocityFloat,
                                              cmd.useDesiredLookAt, dbr, plan, tmpTouchFrame, tmpTouchPos, tmpSmuggle, tmpRot,
                                              prefer);
        if (fn == kFnSliding && sel == -1 && !l.empty()) {
            sel = l[0];
            physics = true;
        }
        if (physics) {
            ENG_SCOPE(48);
            Vec3 dm = cmd.desiredDirection * cmd.desiredVelocityFloat;
            CalculatePhysicsVector(sel, cmd.useDesiredMovement, dm, cmd.useDesiredLookAt, dbr, plan, tmpRot);
        }
        if (interrupt == kIntReQueue && sel != -1 && cur.positions.count > 1 && plan.count > 1) {
            const Anim &sa = A(sel);
            bool curIdle = VelocityCat(current.outgoingVelocity) == kVelIdle;
            bool selIdle = VelocityCat(sa.outgoingVelocity) == kVelIdle;
            if (cur.functionType == fn &&
                ((!curIdle && current.quadrantID == sa.quadrantID) ||
                 ((curIdle && selIdle) && fabsf(PreferredOutgoingAngle(cur.anim) - PreferredOutgoingAngle(sel)) < 0.06f * PI)))
                sel = -1;
        }
        if (sel == -1) return kSelectFalse;
        const float rotScale = fn == kFnMovement ? 1.0f : 0.5f;
        InstallAnimation(sel, fn, interrupt, tmpTouchFrame, tmpTouchPos, rotScale, tmpRot, tmpSmuggle, plan, cmd);
        cur.movementSmuggle = CalculateMovementSmuggle();
        cur.movementSmuggleOffset = Vec3(0);
        return kSelectTrue;
    }
};

}  // namespace eng
