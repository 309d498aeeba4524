// SPDX-License-Identifier: Apache-2.0
// Restates game logic of cuju (Copyright 2026 The cuju Authors), a reimplementation of Google
// Research Football (Copyright 2019 Google LLC); see NOTICE.
// Ball flight, the earliest reach times of players, and player possession.
// Semantics: include/cuju/ball.h:23-348 (prediction), include/cuju/ai_time.h:97-239 (time needed,
// the device form), include/cuju/possession.h:35-123 (scan),
// include/cuju/simulation/player_possession.h:15-126, include/cuju/simulation/ball_touch.h:17-143.
#pragma once

#include "world.h"

namespace eng {

struct BallSpatial {
    Vec3 momentum;
    Quat rotationPerMs;
};

// The cached ticks' shift: entries 2..399 take entries 3..400, as the ticks copy them one after
// another in increasing order.
HD void ShiftPredictions(Ball &ball) { GroupShiftDown<4>(ball.predictions + 2, 398); }

// Entry k of `predictions` is the position after 10k ms. When the first step lands where the last
// tick predicted, the predictions shift down one entry instead, at most `validPredictions` times.
HD bool SameBits(const Vec3 &a, const Vec3 &b) {
    return BitsOf(a.v[0]) == BitsOf(b.v[0]) && BitsOf(a.v[1]) == BitsOf(b.v[1]) && BitsOf(a.v[2]) == BitsOf(b.v[2]);
}
HD bool SameBits(const Quat &a, const Quat &b) {
    return BitsOf(a.q[0]) == BitsOf(b.q[0]) && BitsOf(a.q[1]) == BitsOf(b.q[1]) && BitsOf(a.q[2]) == BitsOf(b.q[2]) &&
           BitsOf(a.q[3]) == BitsOf(b.q[3]);
}

// A ball in flight stepped 10 ms at a time: the state that carries from one step to the next, and
// the stages of a step in the order GRF applies them (the Land, RubGrass, HitFrame, PushNet, Roll
// and Swerve of one step, then the position moves by the momentum). GRF's constants, SI units.
struct BallFlight {
    static constexpr float kDt = 0.01f, kRadius = 0.11f, kGrassHeight = 0.025f;
    static constexpr float kGravity = -9.81f, kDrag = 0.015f, kBounce = 0.62f, kLinearBounce = 0.06f;
    static constexpr float kFriction = 0.04f, kLinearFriction = 1.6f;
    static constexpr float kPostRadius = 0.07f, kPostAbsorb = 0.8f;
    static constexpr float kNetExponent = 2.6f, kNetPower = 1.8f, kNetAbsorb = 0.95f;

    Vec3 pos, mom;
    Quat rot;
    // The Euler angles of `rot`, computed at their first use after `rot` changes.
    Vec3 angles;
    bool anglesKnown = false;

    HD Vec3 Angles() {
        if (!anglesKnown) {
            rot.Angles(angles.v[0], angles.v[1], angles.v[2]);
            anglesKnown = true;
        }
        return angles;
    }
    HD bool InGrass() const { return pos.v[2] < kRadius + kGrassHeight; }

    // How deep the ball sits in the grass (0 to 1, before it lands on the ground) and how hard the
    // landing was.
    struct Contact {
        float grass, impact;
    };
    // Gravity and air drag, then the ground: a falling ball bounces back up, losing speed, and the
    // ball never sinks below its radius.
    HD Contact Land() {
        Contact c{0.0f, 0.0f};
        mom.v[2] = mom.v[2] + kGravity * kDt;
        const float speed = mom.Length();
        const float dragged = speed - kDrag * (speed * speed) * kDt;
        mom = mom.Normalized(0) * dragged;
        const float depth = Clamp(1.0f - ((pos.v[2] - 0.11f) / kGrassHeight), 0.0f, 1.0f);
        c.grass = libm::PowfPos(depth, 0.7f);
        if (pos.v[2] < 0.11f) {
            if (mom.v[2] < 0.0f) {
                c.impact = NormalizedClamp(-mom.v[2] - 0.5f, 0.0f, 12.0f);
                mom.v[2] = -mom.v[2] * kBounce;
                const float up = mom.v[2] - kLinearBounce;
                mom.v[2] = up > 0.0f ? up : 0.0f;
            }
            pos.v[2] = 0.11f;
        }
        return c;
    }
    // Rolling friction of the grass on the horizontal momentum.
    HD void RubGrass(const Contact &c) {
        const float rub = (kFriction * c.grass);
        Vec3 flat = mom.Get2D();
        const float speed = flat.Length();
        float slowed = speed - rub * (speed * speed) * kDt;
        slowed = Clamp(slowed - (kLinearFriction * c.grass * kDt), 0.0f, 100000.0f);
        flat.Normalize(Vec3(0));
        flat *= slowed;
        mom.v[0] = flat.v[0];
        mom.v[1] = flat.v[1];
    }
    // A ball touching a post bounces off it around the post, one touching the crossbar around the
    // bar, each keeping 80% of the speed it had across it.
    HD void HitFrame() {
        const float reach = kRadius + kPostRadius;
        if (pos.v[2] < kGoalHeight + kRadius + kPostRadius &&
            (pos.Get2D().Absolute() - Vec3(kPitchHalfLength, kGoalHalfWidth, 0)).Length() < reach) {
            const Vec3 post(pos.v[0] < 0 ? -kPitchHalfLength : kPitchHalfLength, pos.v[1] < 0 ? -kGoalHalfWidth : kGoalHalfWidth, 0);
            const Vec3 away = (pos.Get2D() - post).Normalized(pos.v[0] < 0 ? Vec3(1, 0, 0) : Vec3(-1, 0, 0));
            const float z = pos.v[2];
            pos = post + away * (kPostRadius + kRadius);
            pos.v[2] = z;
            mom = (mom.Get2D().Normalized(away) + (away * 1.1f)).Normalized() * mom.Get2D().Length() * kPostAbsorb +
                  (Vec3(0, 0, 1) * mom.v[2]);
        }
        const Vec3 side = pos * Vec3(1, 0, 1);
        if ((side.Absolute() - Vec3(kPitchHalfLength, 0, kGoalHeight)).Length() < reach &&
            fabsf(pos.v[1]) < kGoalHalfWidth + kRadius + kPostRadius) {
            const Vec3 bar = pos.v[0] < 0 ? Vec3(-kPitchHalfLength, 0, kGoalHeight) : Vec3(kPitchHalfLength, 0, kGoalHeight);
            const Vec3 away = (side - bar).Normalized(pos.v[0] < 0 ? Vec3(0, 0, 1) : Vec3(0, 0, -1));
            const float y = pos.v[1];
            pos = bar + away * (kPostRadius + kRadius);
            pos.v[1] = y;
            const Vec3 across = mom * Vec3(1, 0, 1);
            mom = (across.Normalized(away) + (away * 1.1f)).Normalized() * across.Length() * kPostAbsorb + (Vec3(0, 1, 0) * mom.v[1]);
        }
    }
    // Inside the goal, past the line, the side nettings, the back netting and the roof push the
    // ball back in. Returns whether a netting touched it.
    HD bool PushNet(bool inGoal) {
        if (!inGoal) return false;
        const float sign = 1;  // the nettings push a ball in the goal back toward the pitch
        const bool behind = fabsf(pos.v[0]) > kPitchHalfLength + 0.11f;
        if (!behind) return false;
        const bool beforeBack = fabsf(pos.v[0]) < kPitchHalfLength + kGoalDepth - 0.11f;
        const bool below = pos.v[2] < kGoalHeight + 0.11f;
        const bool between = fabsf(pos.v[1]) < kGoalHalfWidth - 0.11f;
        bool touched = false;
        if (!between) {
            const float reach = Clamp(fabsf(fabsf(pos.v[1]) - kGoalHalfWidth), 0, 1);
            const float push = libm::powf(reach, kNetExponent) * -SignSide(pos.v[1]) * sign;
            const float tension = Clamp((fabsf(mom.v[0]) - kPitchHalfLength) * 2.0f, 0.0f, 1.0f);
            const float power = kNetPower + (1.0f - tension) * 3.0f;
            mom.v[1] = mom.v[1] * kNetAbsorb + push * power * (100 * kDt);
            touched = true;
        }
        if (!beforeBack) {
            const float reach = Clamp(fabsf(fabsf(pos.v[0]) - (kPitchHalfLength + kGoalDepth)), 0, 1);
            const float push = libm::powf(reach, kNetExponent) * -SignSide(pos.v[0]) * sign;
            mom.v[0] = mom.v[0] * kNetAbsorb + push * kNetPower * (100 * kDt);
            touched = true;
        }
        if (!below) {
            const float reach = Clamp(fabsf(fabsf(pos.v[2]) - kGoalHeight), 0, 1);
            const float push = libm::powf(reach, kNetExponent) * -sign;
            const float tension = Clamp((fabsf(mom.v[0]) - kPitchHalfLength) * 2.0f, 0.0f, 1.0f);
            const float power = kNetPower + (1.0f - tension) * 3.0f;
            mom.v[2] = mom.v[2] * kNetAbsorb + push * power * (100 * kDt);
            touched = true;
        }
        return touched;
    }
    // A ball on the grass turns toward rolling without slipping, the turn per ms bounded by the
    // grass (more after a hard landing), and its momentum leans toward the rolling speed.
    HD void Roll(const Contact &c) {
        const float spinX = mom.v[1] / kRadius, spinY = mom.v[0] / kRadius;
        Quat rx, ry;
        rx.SetAngleAxis(Clamp(spinX * 0.001f, -PI * 0.49f, PI * 0.49f), Vec3(-1, 0, 0));
        ry.SetAngleAxis(Clamp(spinY * 0.001f, -PI * 0.49f, PI * 0.49f), Vec3(0, 1, 0));
        const Quat rolling = rx * ry;
        Quat toRolling = rot.RotationTo(rolling).Normalized();
        const float change = fabsf(toRolling.RotationAngle(Quat::Identity())) * 1000.0f;
        float bound = 1.0f * PI * c.grass;
        if (c.impact > 0.0f) bound += 4.0f * PI;
        float share = 1.0f;
        if (change > bound) share = bound / change;
        if (share < 1.0f) toRolling = toRolling.RotationMultipliedBy(share);
        const Quat turned = toRolling * rot;
        const Vec3 a = Angles();
        const float x = -a.v[0], y = a.v[1];
        const float rollX = y * kRadius * 1000.0f, rollY = x * kRadius * 1000.0f;
        float lean = 0.01f;
        lean *= c.grass;
        if (c.impact > 0.0f) lean += 0.5f * c.impact;
        lean = Clamp(lean, 0.0f, 1.0f);
        mom.v[0] = mom.v[0] * (1.0f - lean) + rollX * lean;
        mom.v[1] = mom.v[1] * (1.0f - lean) + rollY * lean;
        rot = turned;
        anglesKnown = false;
    }
    // The Magnus force of the spin bends the momentum, strongest at middling speeds.
    HD void Swerve() {
        Vec3 spin = Angles();
        spin *= 10.0f;
        float strength = NormalizedClamp(mom.Length(), 0.0f, 70.0f);
        strength = libm::PowfPos(libm::sinf(strength * PI * 0.94f), 2.6f);
        const Vec3 along = mom.Normalized(0) * strength * 30.0f;
        const Vec3 bend = along.Cross(-spin) * 1.0f;
        mom += bend * kDt;
    }
};

// The prediction is a function of the ball's position, orientation, momentum and rotation and of
// whether it is in the goal. When those match the last full prediction bit for bit, its first step
// lands on entry 1; unless the cached path applies, the full path would write exactly what the
// arrays already hold, so only its other results are restored.
HDN BallSpatial BallCalculatePrediction(Ball &ball, bool ballIsInGoal) {
    ENG_SCOPE(37);
    if (ball.memoValid && ball.memoInGoal == ballIsInGoal && SameBits(ball.memoPosition, ball.positionBuffer) &&
        SameBits(ball.memoMomentum, ball.momentum) && SameBits(ball.memoOrientation, ball.orientationBuffer) &&
        SameBits(ball.memoRotation, ball.rotationPerMs) &&
        !(ball.validPredictions > 0 && ball.predictions[2] == ball.predictions[1])) {
        ball.validPredictions = kCachedPredictions;
        ball.touchesNet = ball.memoTouchesNet;
        BallSpatial out;
        out.momentum = ball.memoOutMomentum;
        out.rotationPerMs = ball.memoOutRotation;
        return out;
    }
    const Vec3 inPosition = ball.positionBuffer, inMomentum = ball.momentum;
    const Quat inOrientation = ball.orientationBuffer, inRotation = ball.rotationPerMs;
    BallFlight f;
    f.pos = ball.positionBuffer;
    f.mom = ball.momentum;
    f.rot = ball.rotationPerMs;
    Quat orientation = ball.orientationBuffer;
    BallSpatial out;
    ball.predictions[0] = f.pos;
    ball.touchesNet = false;
    bool useCache = false;
    for (uint32_t t = 10; t < kBallPredictionSpanMs + kCachedPredictions * 10; t += 10) {
        if (useCache) {
            // GRF: the last shift reads predictions[400], which no tick writes.
            ShiftPredictions(ball);
            break;
        }
        const bool first = t == 10;
        const BallFlight::Contact contact = f.Land();
        if (f.InGrass()) f.RubGrass(contact);
        // GRF: the posts, the crossbar and the netting act on the first step only.
        if (first) {
            f.HitFrame();
            if (f.PushNet(ballIsInGoal)) ball.touchesNet = true;
        }
        if (f.InGrass()) f.Roll(contact);
        f.Swerve();
        f.pos += f.mom * BallFlight::kDt;
        if (first) {
            Vec3 turn = f.Angles();
            turn *= BallFlight::kDt / 0.001f;
            Quat step;
            step.SetAngles(turn.v[0], turn.v[1], turn.v[2]);
            orientation = step * orientation;
            out.momentum = f.mom;
            out.rotationPerMs = f.rot;
            ball.orientationPrediction = orientation;
            if (ball.validPredictions > 0 && ball.predictions[2] == f.pos) {
                ball.validPredictions--;
                useCache = true;
            } else {
                ball.validPredictions = kCachedPredictions;
            }
        }
        ball.predictions[t / 10] = f.pos;
    }
    ball.memoValid = !useCache;
    if (!useCache) {
        ball.memoInGoal = ballIsInGoal;
        ball.memoTouchesNet = ball.touchesNet;
        ball.memoPosition = inPosition;
        ball.memoMomentum = inMomentum;
        ball.memoOrientation = inOrientation;
        ball.memoRotation = inRotation;
        ball.memoOutMomentum = out.momentum;
        ball.memoOutRotation = out.rotationPerMs;
    }
    return out;
}

HD void BallRecalculatePrediction(World &w) {
    BallMaterialize(w.match.ball);
    BallCalculatePrediction(w.match.ball, w.match.ballIsInGoal);
}

HDN void BallProcess(Ball &b, bool inGoal) {
    ENG_SCOPE(7);
    BallMaterialize(b);
    BallSpatial s = BallCalculatePrediction(b, inGoal);
    b.momentum = s.momentum;
    b.rotationPerMs = s.rotationPerMs;
    b.positionBuffer = BallPredictRaw(b.predictions, 10);
    b.orientationBuffer = b.orientationPrediction;
    auto &h = b.positionHistory;
    if (h.count < (int)kBallHistorySize) {
        h.push_back(b.positionBuffer);
    } else {
        GroupShiftDown<4>(h.e, h.count - 1);
        h[h.count - 1] = b.positionBuffer;
    }
}

// `clamp((float)(10 k) / (float)700, 0, 1)`, computed in float once per step index. The device
// divides by a reciprocal product and one fused correction, which rounds exactly as the division
// for every step index below 200 (the walks end at 70).
HD float TimeNeededBias(uint32_t step) {
#if ENG_DEVICE
    const float x = (float)(step * 10), r = 1.0f / 700.0f;
    const float q = x * r;
    return Clamp(fmaf(fmaf(-q, 700.0f, x), r, q), 0, 1);
#else
    return Clamp((float)(step * 10) / (float)700, 0, 1);
#endif
}

struct TimeNeeded {
    uint32_t usual = 0, optimistic = 0;
};

HD uint32_t DirectTimeMs(const Vec3 &pos, const Vec3 &mov, const Vec3 &target, float maxVel) {
    return (uint32_t)TruncToInt32(roundf((target - (pos + mov * 0.2f)).Length() / (maxVel * 0.75f) * 1000));
}

// Velocities in m/s; `maxTime` is UINT32_MAX for no limit.
HD TimeNeeded GetTimeNeededMs(const Vec3 &pos, const Vec3 &mov, const Vec3 &target, float maxVel,
                               bool precise, uint32_t maxTime) {
    ENG_SCOPE(36);
    TimeNeeded r;
    if ((pos - target).Length() > (precise ? 48.0f : 16.0f)) {
        r.usual = DirectTimeMs(pos, mov, target, maxVel);
        r.optimistic = r.usual - 200;
        return r;
    }
    Vec3 cur = pos, cm = mov;
    if (cm.Length() > kIdleDribbleSwitch) {
        cur += cm.Normalized() * 0.1f;
        cur += cm * 0.01f;
    } else {
        cur += (target - pos).Normalized(0) * 0.1f;
    }
    uint32_t time = 0;
    const uint32_t step = 10;
    float usualR = 0.28f, optR = 0.9f, resultingUsualR = usualR;
    bool foundOpt = false;
    float amv = maxVel * 0.94f;
    for (uint32_t k = 0;; k++) {
        float bias = TimeNeededBias(k);  // k = time / step
        if (bias >= 1.0f) {
            float rem = Clamp((target - cur).Length() - usualR, 0.0f, 100000.0f);
            r.usual = TruncToUint32((float)time + (rem / amv) * 1000);
            resultingUsualR = usualR + rem;
            if (!foundOpt) {
                float ro = Clamp((target - cur).Length() - optR, 0.0f, 100000.0f);
                r.optimistic = TruncToUint32((float)time + (ro / amv) * 1000);
            }
            break;
        }
        cm.v[0] = mov.v[0] * (1.0f - bias);
        cm.v[1] = mov.v[1] * (1.0f - bias);
        cur.v[0] += cm.v[0] * step * 0.001f;
        cur.v[1] += cm.v[1] * step * 0.001f;
        usualR += amv * bias * step * 0.001f;
        optR += amv * bias * step * 0.001f;
        float d2 = (target - cur).SquaredLength();
        if ((d2 < optR * optR || (maxTime != (uint32_t)-1 && time > maxTime)) && !foundOpt) {
            r.optimistic = time;
            foundOpt = true;
        }
        if (d2 < usualR * usualR || (maxTime != (uint32_t)-1 && time > maxTime)) {
            resultingUsualR = usualR;
            r.usual = time;
            break;
        }
        time += step;
    }
    if (maxTime != (uint32_t)-1 && time > maxTime) {
        uint32_t def = DirectTimeMs(pos, mov, target, maxVel), ext = (time + 100) * 2;
        r.usual = def > ext ? def : ext;
        if (!foundOpt) r.optimistic = r.usual;
        return r;
    }
    if (r.usual == 0) {
        r.usual = (uint32_t)TruncToInt32(roundf(Clamp((target - pos).Length() / resultingUsualR, 0.0f, 1.0f) * 10));
        r.optimistic = r.usual;
    }
    return r;
}

// GetTimeNeededMs split in two for a player whose movement exceeds the idle threshold: the walk,
// which every target shares, and the search along it for one target. The search gives the same
// result as GetTimeNeededMs. With `cooperative` the lanes of the match (all running the same
// sequential code) test consecutive steps of the walk together.
HD bool TimeWalkApplies(const Vec3 &mov) { return mov.Length() > kIdleDribbleSwitch; }
HDN void BuildTimeWalk(TimeWalk &wk, const Vec3 &pos, const Vec3 &mov, float maxVel) {
    Vec3 cur = pos, cm = mov;
    cur += cm.Normalized() * 0.1f;
    cur += cm * 0.01f;
    wk.z = cur.v[2];
    const uint32_t step = 10;
    float usualR = 0.28f, optR = 0.9f;
    const float amv = maxVel * 0.94f;
    for (int k = 0; k < kTimeWalkSteps; k++) {
        const float bias = TimeNeededBias((uint32_t)k);
        cm.v[0] = mov.v[0] * (1.0f - bias);
        cm.v[1] = mov.v[1] * (1.0f - bias);
        cur.v[0] += cm.v[0] * step * 0.001f;
        cur.v[1] += cm.v[1] * step * 0.001f;
        usualR += amv * bias * step * 0.001f;
        optR += amv * bias * step * 0.001f;
        wk.x[k] = cur.v[0];
        wk.y[k] = cur.v[1];
        wk.usual[k] = usualR;
        wk.optimistic[k] = optR;
        wk.usualSquared[k] = usualR * usualR;
        wk.optimisticSquared[k] = optR * optR;
    }
}
HDN TimeNeeded WalkTimeNeeded(const TimeWalk &wk, const Vec3 &pos, const Vec3 &mov, const Vec3 &target, float maxVel,
                              bool precise, uint32_t maxTime, bool cooperative) {
    TimeNeeded r;
    if ((pos - target).Length() > (precise ? 48.0f : 16.0f)) {
        r.usual = DirectTimeMs(pos, mov, target, maxVel);
        r.optimistic = r.usual - 200;
        return r;
    }
    const bool limited = maxTime != (uint32_t)-1;
    const int stride = cooperative ? kGroupLanes : 1, rank = cooperative ? GroupRank() : 0;
    int reach = -1, optimistic = -1;
    for (int k0 = 0; k0 < kTimeWalkSteps && reach < 0; k0 += stride) {
        const int k = k0 + rank;
        bool u = false, o = false;
        if (k < kTimeWalkSteps) {
            const bool late = limited && (uint32_t)(k * 10) > maxTime;
            const Vec3 cur(wk.x[k], wk.y[k], wk.z);
            const float d2 = (target - cur).SquaredLength();
            o = d2 < wk.optimisticSquared[k] || late;
            u = d2 < wk.usualSquared[k] || late;
        }
        const LaneMask um = cooperative ? GroupBallot(u) : (LaneMask)u;
        LaneMask om = cooperative ? GroupBallot(o) : (LaneMask)o;
        if (um) {
            reach = k0 + LowestBit(um);
            om &= LanesThrough(LowestBit(um));  // the optimistic test comes first within a step
        }
        if (optimistic < 0 && om) optimistic = k0 + LowestBit(om);
    }
    const bool foundOpt = optimistic >= 0;
    if (foundOpt) r.optimistic = (uint32_t)(optimistic * 10);
    uint32_t time;
    float resultingUsualR;
    if (reach >= 0) {
        time = (uint32_t)(reach * 10);
        resultingUsualR = wk.usual[reach];
        r.usual = time;
    } else {
        // The bias reaches 1 at 700 ms; the rest of the way runs at 94% of the maximum velocity.
        time = (uint32_t)(kTimeWalkSteps * 10);
        const int last = kTimeWalkSteps - 1;
        const Vec3 cur(wk.x[last], wk.y[last], wk.z);
        const float amv = maxVel * 0.94f;
        float rem = Clamp((target - cur).Length() - wk.usual[last], 0.0f, 100000.0f);
        r.usual = TruncToUint32((float)time + (rem / amv) * 1000);
        resultingUsualR = wk.usual[last] + rem;
        if (!foundOpt) {
            float ro = Clamp((target - cur).Length() - wk.optimistic[last], 0.0f, 100000.0f);
            r.optimistic = TruncToUint32((float)time + (ro / amv) * 1000);
        }
    }
    if (limited && time > maxTime) {
        uint32_t def = DirectTimeMs(pos, mov, target, maxVel), ext = (time + 100) * 2;
        r.usual = def > ext ? def : ext;
        if (!foundOpt) r.optimistic = r.usual;
        return r;
    }
    if (r.usual == 0) {
        r.usual = (uint32_t)TruncToInt32(roundf(Clamp((target - pos).Length() / resultingUsualR, 0.0f, 1.0f) * 10));
        r.optimistic = r.usual;
    }
    return r;
}

// GetTimeNeededMs for the targets of one player (position, movement and velocity fixed), with a
// shortcut for targets the walk cannot reach (ai_time.h:133). Over its 70 steps the walk moves at
// most 0.355 |movement| (in the plane) from where it starts, and its optimistic radius grows to
// at most 0.9 + 0.345 amv. A target farther from the start than their sum, with a margin over the
// rounding of the walk, fails every step's test. Its result then follows from the step at which
// the walk stops: one step past the time limit, or the end of the bias at 700 ms. The radii there
// are the same for every target, and so is the position for a moving player; an idle player
// starts a tenth of a metre towards the target, so its position is walked per target, without
// the tests. Every other target runs GetTimeNeededMs itself, so the results are GetTimeNeededMs's.
struct TimeNeededScan {
    Vec3 pos, mov, start, end;
    float maxVel, amv, reach, endUsual = 0, endOptimistic = 0;
    bool moving, ended = false;

    HD TimeNeededScan(const Vec3 &p, const Vec3 &m, float velocity) : pos(p), mov(m), maxVel(velocity) {
        amv = maxVel * 0.94f;
        moving = mov.Length() > kIdleDribbleSwitch;
        start = pos;
        if (moving) {
            start += mov.Normalized() * 0.1f;
            start += mov * 0.01f;
        }
        reach = (sqrtf(mov.v[0] * mov.v[0] + mov.v[1] * mov.v[1]) * 0.36f + 0.9f + 0.35f * amv) * 1.001f + 0.01f;
    }
    // The position after the 70 steps from `from`, as GetTimeNeededMs steps it.
    HD Vec3 WalkFrom(const Vec3 &from) const {
        Vec3 cur = from;
        const uint32_t step = 10;
        for (uint32_t k = 0; k < kTimeWalkSteps; k++) {
            const float bias = TimeNeededBias(k);
            const float cx = mov.v[0] * (1.0f - bias), cy = mov.v[1] * (1.0f - bias);
            cur.v[0] += cx * step * 0.001f;
            cur.v[1] += cy * step * 0.001f;
        }
        return cur;
    }
    // The radii after the 70 steps, and a moving player's position.
    HD void WalkToEnd() {
        float usualR = 0.28f, optR = 0.9f;
        const uint32_t step = 10;
        for (uint32_t k = 0; k < kTimeWalkSteps; k++) {
            const float bias = TimeNeededBias(k);
            usualR += amv * bias * step * 0.001f;
            optR += amv * bias * step * 0.001f;
        }
        endUsual = usualR;
        endOptimistic = optR;
        if (moving) end = WalkFrom(start);
        ended = true;
    }
    // True with the result in `r` for a target the walk cannot reach; false for a far target (the
    // direct estimate) and for one within reach.
    HD bool Unreachable(const Vec3 &target, bool precise, uint32_t maxTime, TimeNeeded &r) {
        if ((pos - target).Length() > (precise ? 48.0f : 16.0f)) return false;
        const Vec3 from = moving ? start : pos + (target - pos).Normalized(0) * 0.1f;
        const float margin = (fabsf(from.v[0]) + fabsf(from.v[1])) * 1e-5f;
        if (!((target - from).Length() > reach + margin)) return false;
        const bool limited = maxTime != (uint32_t)-1;
        if (limited && maxTime < (kTimeWalkSteps - 1) * 10) {
            // Stopped by the limit one step past it, the optimistic time found there.
            const uint32_t time = (maxTime / 10 + 1) * 10;
            const uint32_t def = DirectTimeMs(pos, mov, target, maxVel), ext = (time + 100) * 2;
            r.optimistic = time;
            r.usual = def > ext ? def : ext;
            return true;
        }
        if (!ended) WalkToEnd();
        const uint32_t time = kTimeWalkSteps * 10;
        const float d = (target - (moving ? end : WalkFrom(from))).Length();
        const float rem = Clamp(d - endUsual, 0.0f, 100000.0f), ro = Clamp(d - endOptimistic, 0.0f, 100000.0f);
        r.usual = TruncToUint32((float)time + (rem / amv) * 1000);
        r.optimistic = TruncToUint32((float)time + (ro / amv) * 1000);
        if (limited && time > maxTime) {
            const uint32_t def = DirectTimeMs(pos, mov, target, maxVel), ext = (time + 100) * 2;
            r.usual = def > ext ? def : ext;
            r.optimistic = r.usual;
        }
        return true;
    }
    HD TimeNeeded Get(const Vec3 &target, bool precise, uint32_t maxTime) {
        TimeNeeded r;
        if (Unreachable(target, precise, maxTime, r)) return r;
        return GetTimeNeededMs(pos, mov, target, maxVel, precise, maxTime);
    }
};

struct ScanResult {
    uint32_t timeToBall, timeToBallOptimistic;
};

HD Vec3 PredFlip(const Vec3 *pred, bool flip, int ms) {
    Vec3 v = BallPredictRaw(pred, ms);
    if (flip) v.Mirror();
    return v;
}

// GRF's earliest time to the ball over the 3 s of predictions. It visits points of the prediction
// from `start` at a stride of the ball's distance (10 to 500 ms) until the walk reaches one in its
// usual time, then goes back to the point before and steps 10 ms at a time to the first that is
// reached; the optimistic time is the first visited point reached optimistically. Points above
// 1.5 m count as unreached.
//
// Here `lanes` lanes of the match share one scan (this one is `lane`): the points before the
// refinement follow from the prediction alone, so every lane walks them and each evaluates the
// walk at its own point of a round of `lanes`; the lowest reached point of a round ends the coarse
// part, and the refinement's 10 ms points are shared the same way. What the scan visits, and so
// its result, is the same for any number of lanes.
HDN ScanResult SharedPossessionScan(const Vec3 *pred, bool flip, const Vec3 &pos, const Vec3 &mov, float maxVel,
                                    bool precise, uint32_t start, int lane, int lanes) {
    ENG_SCOPE(35);
    ScanResult s;
    {
        uint32_t latest = kBallPredictionSpanMs;
        uint32_t direct = TruncToUint32(roundf(
            (PredFlip(pred, flip, kBallPredictionSpanMs - 10).Get2D() - (pos + mov * 0.2f)).Length() /
            (maxVel * 0.75f) * 1000));
        s.timeToBall = latest > direct ? latest : direct;
    }
    s.timeToBallOptimistic = s.timeToBall;
    TimeNeededScan times(pos, mov, maxVel);
    const int base = GroupRank() - lane;
    const LaneMask mine = lanes >= 64 ? ~(LaneMask)0 : (((LaneMask)1 << lanes) - 1u);
    // This lane's point: whether the walk reaches it usually and optimistically (never above 1.5 m).
    auto evaluate = [&](uint32_t ms, bool &usual, bool &optimistic) {
        usual = optimistic = false;
        const Vec3 at = PredFlip(pred, flip, (int)ms);
        if (!(at.v[2] < 1.5f)) return;
        const TimeNeeded r = times.Get(at.Get2D(), precise, ms);
        usual = r.usual <= ms;
        optimistic = r.optimistic <= ms;
    };
    // The round's lowest usual hit, or -1; the optimistic time takes the lowest optimistic hit up
    // to it (the points of a round rise with the lane).
    auto settle = [&](bool usual, bool optimistic, uint32_t ms) {
        const LaneMask hits = (GroupBallot(usual) >> base) & mine;
        LaneMask opts = (GroupBallot(optimistic) >> base) & mine;
        if (hits) opts &= LanesThrough(LowestBit(hits));
        if (opts) {
            const uint32_t o = GroupShuffle(ms, base + LowestBit(opts));
            if (o < s.timeToBallOptimistic) s.timeToBallOptimistic = o;
        }
        return hits ? LowestBit(hits) : -1;
    };
    uint32_t ms = start, prev = 0, from = 0, to = 0;
    bool reached = false;
    while (!reached && ms < kBallPredictionSpanMs) {
        uint32_t myMs = 0, myPrev = 0;
        bool here = false;
        for (int t = 0; t < lanes && ms < kBallPredictionSpanMs; t++) {
            if (t == lane) {
                myMs = ms;
                myPrev = prev;
                here = true;
            }
            const float dist = (pos - PredFlip(pred, flip, (int)ms).Get2D()).Length() + 0.2f;
            const uint32_t toGo = (uint32_t)TruncToInt32(roundf((dist / 50.0f) * 1000.0f));
            uint32_t stepMs = TruncToUint32(Clamp((float)toGo, 10, 500));
            stepMs = (stepMs / 10) * 10;
            prev = ms;
            ms += stepMs;
        }
        bool usual = false, optimistic = false;
        if (here) evaluate(myMs, usual, optimistic);
        const int hit = settle(usual, optimistic, myMs);
        if (hit >= 0) {
            from = GroupShuffle(myPrev, base + hit);
            to = GroupShuffle(myMs, base + hit);
            reached = true;
        }
    }
    if (!reached) return s;
    // The refinement reaches `to` at the latest, where the coarse part already did.
    for (uint32_t r0 = from + 10; r0 <= to; r0 += 10 * (uint32_t)lanes) {
        const uint32_t myMs = r0 + 10 * (uint32_t)lane;
        bool usual = false, optimistic = false;
        if (myMs <= to) evaluate(myMs, usual, optimistic);
        const int hit = settle(usual, optimistic, myMs);
        if (hit >= 0) {
            s.timeToBall = r0 + 10 * (uint32_t)hit;
            return s;
        }
    }
    s.timeToBall = to;
    return s;
}

// The same scan on one lane, point after point.
HDN ScanResult PossessionScan(const Vec3 *pred, bool flip, const Vec3 &pos, const Vec3 &mov, float maxVel,
                              bool precise, uint32_t start) {
    ENG_SCOPE(35);
    ScanResult s;
    {
        uint32_t latest = kBallPredictionSpanMs;
        uint32_t direct = TruncToUint32(roundf(
            (PredFlip(pred, flip, kBallPredictionSpanMs - 10).Get2D() - (pos + mov * 0.2f)).Length() /
            (maxVel * 0.75f) * 1000));
        s.timeToBall = latest > direct ? latest : direct;
    }
    s.timeToBallOptimistic = s.timeToBall;
    bool refine = false;
    uint32_t stepMs = 10, prev = 0;
    TimeNeededScan times(pos, mov, maxVel);
    for (uint32_t ms = start; ms < kBallPredictionSpanMs; ms += stepMs) {
        if (PredFlip(pred, flip, ms).v[2] < 1.5f) {
            const Vec3 target = PredFlip(pred, flip, ms).Get2D();
            TimeNeeded r = times.Get(target, precise, ms);
            if (r.optimistic <= ms && ms < s.timeToBallOptimistic) s.timeToBallOptimistic = ms;
            if (r.usual <= ms) {
                if (!refine) {
                    ms = prev;
                    stepMs = 10;
                    refine = true;
                } else {
                    s.timeToBall = ms;
                    break;
                }
            }
        }
        if (!refine) {
            float dist = (pos - PredFlip(pred, flip, ms).Get2D()).Length() + 0.2f;
            uint32_t toGo = (uint32_t)TruncToInt32(roundf((dist / 50.0f) * 1000.0f));
            stepMs = TruncToUint32(Clamp((float)toGo, 10, 500));
            stepMs = (stepMs / 10) * 10;
        } else {
            stepMs = 10;
        }
        prev = ms;
    }
    return s;
}

HDN bool HasPossession(const World &w, int p) {
    const Ball &b = w.match.ball;
    const SpatialState &s = Sp(w, p);
    if ((double)(s.position - BallPredict(b, 0)).Length() > 5.0) return false;
    if ((double)fabsf(BallPredict(b, 0).v[2]) > 0.5) return false;
    bool distOk = true;
    Vec3 center = s.position + s.movement * 0.05f + s.directionVec * 0.1f;
    if ((BallPredict(b, 0).Get2D() - center).Length() > 1.0f) distOk = false;
    bool movOk = true;
    Vec3 bm = (BallPredict(b, 10) - BallPredict(b, 0)) * 100.0f;
    if ((bm - s.movement).Length() > 6.0f) movOk = false;
    return distOk && movOk;
}

HD bool IsPassOrShot(int f) { return f == kFnShortPass || f == kFnLongPass || f == kFnHighPass || f == kFnShot; }

HDN void PlayerUpdatePossessionStatistics(World &w, const StaticData &sd, int p, int lane = 0, int lanes = 1) {
    Player &ps = w.match.players[p];
    const Humanoid &h = ps.base.humanoid;
    const Ball &b = w.match.ball;
    const Team &team = TeamOfPlayer(w, p);
    const Team &opp = OpponentTeamOfPlayer(w, p);
    const Vec3 pos = h.spatial.position, mov = h.spatial.movement;
    const float maxVel = GetMaximumVelocity(sd, p);
    ps.timeToBallPreviousMs = ps.timeToBallMs;
    uint32_t start = 0;
    const bool touchPending = h.anim.frameNum < h.anim.touchFrame;
    if (IsPassOrShot(h.anim.functionType) && !touchPending) start = 500;
    bool precise = team.designatedTeamPossessionPlayer == p;
    // The host build runs the shared scan with one lane, so its tests check that scan's order.
    const ScanResult s = lanes > 1 || !ENG_DEVICE
                             ? SharedPossessionScan(b.predictions, b.lazyFlip, pos, mov, maxVel, precise, start, lane, lanes)
                             : PossessionScan(b.predictions, b.lazyFlip, pos, mov, maxVel, precise, start);
    ps.timeToBallMs = s.timeToBall;
    ps.timeToBallOptimisticMs = s.timeToBallOptimistic;
    if (h.anim.touchFrame != -1 && touchPending) {
        uint32_t at = (uint32_t)((h.anim.touchFrame - h.anim.frameNum) * 10);
        if (at < ps.timeToBallMs) ps.timeToBallMs = at;
        ps.timeToBallOptimisticMs = ps.timeToBallMs;
    }
    if (ps.timeToBallMs < kDefaultTouchOffsetMs) {
        ps.timeToBallMs = TruncToUint32(
            NormalizedClamp(((pos + mov * (float)(kDefaultTouchOffsetMs * 0.001)) - BallPredict(b, kDefaultTouchOffsetMs).Get2D()).Length(),
                            0.0f, 0.6f) *
            kDefaultTouchOffsetMs);
        ps.timeToBallOptimisticMs = ps.timeToBallMs;
    }
    if (IsPassOrShot(h.anim.functionType) && !touchPending) ps.hasPossession = false;
    else ps.hasPossession = HasPossession(w, p);
    ps.hasBestPossession = ps.hasPossession && opp.timeToBallMs > (int32_t)ps.timeToBallMs;
    ps.hasUniquePossession = ps.hasPossession && !opp.hasPossession;
    if (w.match.ballRetainer == p) {
        ps.timeToBallMs = 1;
        ps.timeToBallOptimisticMs = 1;
        ps.desiredTimeToBallMs = (int32_t)ps.timeToBallMs;
        ps.hasPossession = ps.hasBestPossession = ps.hasUniquePossession = true;
    } else if (w.match.ballRetainer != -1) {
        ps.hasPossession = ps.hasBestPossession = ps.hasUniquePossession = false;
    }
    w.roster.timeToBallMs[p] = ps.timeToBallMs;
}

HDN void TeamUpdatePossessionStatistics(World &w, const Ctx &c, int teamID) {
    ENG_SCOPE(16);
    // A player's statistics read only the ball, the opposing team and its own fields, so the lanes
    // of the match take the players in turn, one a lane in whole rounds. The players left after
    // the whole rounds, when the group has at least two lanes for each, get as many lanes each as
    // the group holds, which share the player's scan (they write the same results).
    const PlayerList players = TeamActivePlayers(w, teamID);
    const int whole = players.count - players.count % kGroupLanes;
    const int rest = players.count - whole;
    const int share = rest > 0 && kGroupLanes >= 2 * rest ? kGroupLanes / rest : 1;
    const int single = share == 1 ? players.count : whole;
    for (int i = GroupRank(); i < single; i += kGroupLanes) PlayerUpdatePossessionStatistics(w, *c.sd, players[i]);
    if (share > 1 && GroupRank() < share * rest)
        PlayerUpdatePossessionStatistics(w, *c.sd, players[whole + GroupRank() / share], GroupRank() % share, share);
    GroupSync();
    // The team's summary over its active players in state order, kept in registers and stored once.
    bool hasPossession = false;
    int timeToBall = 100000;
    for (int i = 0; i < players.count; i++) {
        if (w.match.players[players[i]].hasPossession) hasPossession = true;
        const int t = (int)w.roster.timeToBallMs[players[i]];
        if (t < timeToBall) timeToBall = t;
    }
    Team &t = TeamByID(w, teamID);
    t.hasPossession = hasPossession;
    t.timeToBallMs = timeToBall;
}

HDN void BallTouch(World &w, const Ctx &c, const Vec3 &target) {
    Ball &b = w.match.ball;
    b.validPredictions = 0;
    if (b.positionBuffer.v[2] < 0.11f) b.positionBuffer.v[2] = 0.11f;
    b.momentum = target;
    // GRF: the predictions run twice, and each run changes the count of valid cached ones. The
    // second run starts from the same ball, so its first step lands on the first run's entry 1:
    // unless that equals entry 2 (the cached path, which shifts), it recomputes exactly what the
    // first run left, and is skipped.
    BallRecalculatePrediction(w);
    if (b.validPredictions > 0 && b.predictions[2] == b.predictions[1]) BallRecalculatePrediction(w);
    if (w.match.mentalImages.count > 0) {
        MentalImage &m = w.match.mentalImages[0];
        m.ballPredictions.count = kBallPredictionSpanMs / 10;
        GroupCopy<4>(m.ballPredictions.e, b.predictions, (int)(kBallPredictionSpanMs / 10));
        m.lazyFlip = b.lazyFlip;
    }
    TeamUpdatePossessionStatistics(w, c, w.FirstTeamID());
    TeamUpdatePossessionStatistics(w, c, 1 - w.FirstTeamID());
}

// With `predict` false the predictions stay as they are, for a caller whose next step recomputes
// every output of the prediction before anything reads it.
HD void BallSetRotation(World &w, float x, float y, float z, float bias = 1.0f, bool predict = true) {
    Quat rx, ry, rz;
    rx.SetAngleAxis(Clamp(x * 0.001f, -PI * 0.49f, PI * 0.49f), Vec3(-1, 0, 0));
    ry.SetAngleAxis(Clamp(y * 0.001f, -PI * 0.49f, PI * 0.49f), Vec3(0, 1, 0));
    rz.SetAngleAxis(Clamp(z * 0.001f, -PI * 0.49f, PI * 0.49f), Vec3(0, 0, 1));
    Quat tmp = rx * ry * rz;
    Ball &b = w.match.ball;
    b.rotationPerMs = b.rotationPerMs.Slerp(bias, tmp);
    if (predict) BallRecalculatePrediction(w);
}

HD void BallSetPosition(World &w, const Vec3 &target) {
    Ball &b = w.match.ball;
    b.validPredictions = 0;
    b.positionBuffer = target;
    b.momentum = Vec3(0);
    BallSetRotation(w, 0, 0, 0, 1.0f);
    b.positionHistory.count = 0;
}

}  // namespace eng
