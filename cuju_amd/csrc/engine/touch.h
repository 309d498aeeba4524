// SPDX-License-Identifier: Apache-2.0
// Restates game logic of cuju (Copyright 2026 The cuju Authors), a reimplementation of Google
// Research Football (Copyright 2019 Google LLC); see NOTICE.
// Touch vectors (the ball momentum a touch gives) and pass/shot aiming.
// Semantics: include/cuju/simulation/touch.h:15-400 (results depend on the number and order of the
// RNG draws), include/cuju/simulation/ai_functions.h:27-190.
#pragma once

#include "control.h"
#include "select.h"

namespace eng {

HD float ControllerFloatVelocity(World &w, int p) {
    if (ExternalControllerActive(w, p)) return HumanGetFloatVelocity(w, p);
    return w.match.players[p].controller.lastDesiredVelocity;
}

HDN void GetDifficultyFactors(World &w, const Ctx &c, int p, const Vec3 &posOffset, float &distF, float &heightF,
                              float &ballMovF) {
    const Ball &b = w.match.ball;
    const SpatialState &s = Sp(w, p);
    distF = heightF = ballMovF = 0.0f;
    float posPenalty = NormalizedClamp(posOffset.Length(), 0.0f, 0.1f) * 2.0f;
    float velPenalty = libm::powf(NormalizedClamp((s.movement - b.momentum).Length(), 10.0f, 50.0f), 1.5f) * 5.0f;
    float nd = NormalizedClamp(((s.position + s.directionVec * 0.2f) - BallPredict(b, 0).Get2D()).Length(), 0.7f, 1.3f);
    float farPenalty = nd * nd * 2.0f;
    distF += posPenalty * 2.0f;
    distF += velPenalty;
    distF += farPenalty * 4.0f;
    heightF += posPenalty * 0.5f;
    heightF += velPenalty * 2.0f;
    heightF += farPenalty;
    const int teamID = w.playerTeamID[p];
    if (w.match.lastTouchTeamID != teamID) {
        int lt = TeamByID(w, 1 - teamID).lastTouchPlayer;
        if (lt >= 0) {
            int decay = TruncToInt32(1000 - GetStatistic(w, c, p, kStatReaction) * 500);
            float pen = libm::powf(GetLastTouchBias(w, lt, decay), 0.6f) * 5.0f;
            distF += pen;
            heightF += pen;
            ballMovF += pen * 0.1f;
        }
    }
    ballMovF = Clamp(ballMovF, 0.0f, 0.9f);
    float skill = (1.0f - GetStatistic(w, c, p, kStatBallControl) * 0.5f) * RandomInRange(w, 0.5f, 1.0f);
    distF *= skill;
    heightF *= skill;
    ballMovF *= skill;
    distF = Clamp(distF, 0.0f, 1.0f);
    heightF = Clamp(heightF, 0.0f, 1.0f);
    ballMovF = Clamp(ballMovF, 0.0f, 1.0f);
}

HDN bool GetBallControlVector(World &w, const Ctx &c, int p, const Vec3 &nextStartPos, float nextStartAngle,
                              float nextBodyAngle, const Vec3 &outMov, const AnimationState &cur, int frameNum,
                              const SpatialState &s, float &xRot, float &yRot, Vec3 &touch, float extraFoot = 0.0f) {
    const Ball &b = w.match.ball;
    const Player &ps = w.match.players[p];
    const Anim &a = c.A(cur.anim);
    const PlayerCommand &oc = cur.originatingCommand;
    auto Stat = [&](int st) { return GetStatistic(w, c, p, st); };
    float physicsBias = 0.7f;
    if (!ps.hasPossession) physicsBias = 0.9f;
    if (VelocityCat(a.outgoingVelocity) == kVelIdle) physicsBias = 1.0f;
    float explosiveness = 0.6f;
    float maxOverdrive = 1.0f * explosiveness;
    if (oc.desiredVelocityFloat < kDribbleWalkSwitch) maxOverdrive = 0.0f;
    if (oc.desiredVelocityFloat > kWalkSprintSwitch) maxOverdrive = 2.0f * explosiveness;
    float curDirF = s.directionVec.Dot(oc.desiredDirection) * 0.5f + 0.5f;
    float nextDirF = Vec3(0, -1, 0).Rotated2D(nextStartAngle).Dot(oc.desiredDirection) * 0.5f + 0.5f;
    float dotF = Clamp(MinF(curDirF, nextDirF), 0.0f, 1.0f);
    maxOverdrive *= dotF;
    if (VelocityCat(a.outgoingVelocity) == kVelIdle) maxOverdrive = 0.0f;
    float ob = 0.7f;
    float cv = ControllerFloatVelocity(w, p);
    Vec3 dm = oc.desiredDirection * (oc.desiredVelocityFloat * ob + cv * (1.0f - ob));
    if (dm.Length() > kWalkSprintSwitch)
        dm = dm.Normalized(0) * StretchSprint(dm.Length(), kSprintVelocity, GetMaximumVelocity(*c.sd, p));
    float vel = Clamp(dm.Length(), outMov.Length(), outMov.Length() + maxOverdrive);
    dm = dm.Normalized(Vec3(0, -1, 0).Rotated2D(nextStartAngle)) * vel;
    Vec3 pm = Vec3(0, -1, 0).Rotated2D(nextStartAngle) * vel;
    float dv = dm.Length(), pv = pm.Length();
    Vec3 relFoot = FootReachOffset(pv, nextBodyAngle - s.angle.value(), BallPredict(b, 0).v[2]);
    float annoyVel = Curve(NormalizedClamp(a.outgoingVelocity, kIdleVelocity, kSprintVelocity), 0.7f);
    float annoy = (1.0f - NormalizedClamp(ClosestOpponentDistance(w, p), 0.5f, 1.5f)) *
                  (1.0f - (Stat(kStatCalmness) * 0.5f + Stat(kStatBalance) * 0.3f)) * annoyVel;
    Vec3 foot = Vec3(0, -1, 0).Rotated2D(nextBodyAngle) * (relFoot.Length() + extraFoot + annoy * 3.0f);
    float hf = NormalizedClamp(BallPredict(b, 0).v[2], 0.5f, 1.0f) * 0.5f;
    foot += relFoot * hf * 0.5f + s.bodyDirectionVec * hf * 0.5f;
    Vec3 dPlanned = nextStartPos, pPlanned = nextStartPos;
    float dvf = NormalizedClamp(dv, 0.0f, kSprintVelocity);
    float dDelay = dvf * dvf * 0.60f + 0.25f;
    float pvf = NormalizedClamp(pv, 0.0f, kSprintVelocity);
    float pDelay = pvf * pvf * 0.60f + 0.25f;
    dPlanned += dm * dDelay + foot;
    pPlanned += pm * pDelay + foot;
    Vec3 planned = pPlanned * physicsBias + dPlanned * (1.0f - physicsBias);
    Vec3 toPlanned = planned - BallPredict(b, 0).Get2D();
    float timeToGo = (((a.frameCount - 1) - frameNum) * 10) * 0.001f;
    timeToGo += pDelay * physicsBias + dDelay * (1.0f - physicsBias);
    timeToGo += kDefaultTouchOffsetMs * 0.001f;
    float divisor = timeToGo * (0.38f + 0.02f * Stat(kStatDribble));
    divisor *= 1.1f;
    float power = libm::powf((toPlanned.Length() / divisor), 0.7f);
    Vec3 direction = toPlanned.Normalized(Vec3(0, -1, 0).Rotated2D(nextBodyAngle));
    float height = Clamp(0.1f + 1.5f * libm::powf(power / 10.0f, 1.6f), 0.0f, 1.5f);
    float pmul = 1.2f - (Stat(kStatBallControl) * 0.03f);
    float vb = NormalizedClamp(vel, kWalkVelocity, kSprintVelocity - 0.8f);
    pmul = 1.0f * (1.0f - vb) + pmul * vb;
    touch = direction * power * pmul + Vec3(0, 0, height);
    float backspin = 30.0f;
    float tv = touch.Length();
    float vf = libm::powf(NormalizedClamp(touch.Length(), 0.0f, 10.0f), 0.7f);
    Vec3 spin = (foot.Normalized(0) * 0.6f + touch.Normalized(0) * 0.4f).Normalized(0);
    xRot = spin.v[1] * ((2 * PI * tv) - (backspin * vf));
    yRot = spin.v[0] * ((2 * PI * tv) - (backspin * vf));
    return true;
}

HDN bool GetTrapVector(World &w, const Ctx &c, int p, const Vec3 &nsp, float nsa, float nba, const Vec3 &outMov,
                       const AnimationState &cur, int frameNum, const SpatialState &s, const Vec3 &posOffset, float &xRot,
                       float &yRot, Vec3 &result) {
    float df, hf, bmf;
    GetDifficultyFactors(w, c, p, posOffset, df, hf, bmf);
    Vec3 bc;
    if (!GetBallControlVector(w, c, p, nsp, nsa, nba, outMov, cur, frameNum, s, xRot, yRot, bc, df)) return false;
    const Vec3 bm = w.match.ball.momentum;
    bc.v[2] += bm.v[2] * hf * 1.0f + hf * 4.0f;
    result = bc * (1.0f - bmf) + bm * bmf;
    return true;
}

HDN Vec3 GetShotVector(World &w, const Ctx &c, int p, const AnimationState &cur, const SpatialState &s, const Vec3 &posOffset,
                       float &xRot, float &yRot, float &zRot) {
    const Anim &a = c.A(cur.anim);
    const AnimDerived &d = c.D(cur.anim);
    const PlayerCommand &oc = cur.originatingCommand;
    const Vec3 bm = w.match.ball.momentum;
    auto Stat = [&](int st) { return GetStatistic(w, c, p, st); };
    Vec3 touchMov = MovementAtFrame(c.t->positions + a.posFirst, a.posCount, cur.frameNum, 0).Rotated2D(s.angle.value());
    Vec3 touchDir = touchMov.Normalized(s.directionVec);
    float touchVel = touchMov.Length();
    if (VelocityCat(touchVel) == kVelIdle) touchDir = s.directionVec;
    float ideal = 0.2f * PI;
    float neg = fabsf(touchDir.Angle2D(oc.touchInfo.desiredDirection.Rotated2D(-ideal)));
    float pos = fabsf(touchDir.Angle2D(oc.touchInfo.desiredDirection.Rotated2D(ideal)));
    float angle = (pos < neg) ? pos : neg;
    float dirF = Clamp(angle / PI, 0.0f, 1.0f);
    dirF = Curve(1.0f - dirF, 0.8f);
    float pdPower = libm::powf(dirF, 0.8f);
    float pvPower = libm::powf(NormalizedClamp(touchVel, 0.0f, kSprintVelocity), 0.3f);
    float poPower = 1.0f - NormalizedClamp(posOffset.Length(), 0.0f, 0.1f);
    float powerF = 1.0f * (0.7f + pdPower * 0.3f) * (0.7f + pvPower * 0.3f) * (0.4f + poPower * 0.6f);
    powerF = Clamp(powerF, 0.0f, 1.0f);
    float adaptedDesired = 45.0f * (0.7f + libm::powf(oc.touchInfo.desiredPower, 0.5f) * 0.3f);
    float animMaxPower = d.touchMaxPowerFactor;
    if (animMaxPower == 0.0f) animMaxPower = 1.0f;
    float power = Clamp(powerF * adaptedDesired, 0.0f, (32.0f + Stat(kStatShotPower) * 13.0f) * (0.2f + animMaxPower * 0.8f));
    float pmbm = (touchMov - bm).Length();
    pmbm = NormalizedClamp(pmbm, 0.0f, 10.0f);
    power *= 1.0f + pmbm * 0.2f;
    float pdEasy = libm::powf(dirF, 0.8f);
    float pvEasy = 1.0f - NormalizedClamp(fabsf(touchVel - kDribbleVelocity), 0.0f, 4.0f);
    float poEasy = 1.0f - NormalizedClamp(posOffset.Length(), 0.0f, 0.1f);
    float pmbmEasy = 1.0f - pmbm * (0.5f - Stat(kStatVolley) * 0.3f);
    float powerEasy = 1.0f - NormalizedClamp(power, 30.0f, 100.0f);
    powerEasy = Curve(powerEasy, 1.0f);
    float easy = 1.0f * (0.4f + pdEasy * 0.6f) * (0.7f + pvEasy * 0.3f) * (0.3f + poEasy * 0.7f) * (0.6f + pmbmEasy * 0.4f) *
                 (0.6f + powerEasy * 0.4f);
    float difficulty = Clamp(1.0f - easy, 0.0f, 1.0f);
    Vec3 desiredShot = (oc.touchInfo.desiredDirection.Get2D() + Vec3(0, 0, 0.05f)).Normalized() * power;
    Vec3 worst = oc.touchInfo.desiredDirection.Get2D();
    float lag = difficulty * 0.8f;
    worst = (touchDir * lag + worst * (1.0f - lag)).Normalized(0);
    // GRF: the arguments evaluate right to left, so the components draw z, then y, then x.
    float rz = RandomInRange(w, -1, 1);
    float ry = RandomInRange(w, -1, 1);
    float rx = RandomInRange(w, -1, 1);
    worst = worst + (Vec3(rx, ry, rz) * 0.5f * difficulty);
    worst.Normalize();
    float worstH = Curve(libm::powf(difficulty, 0.7f), 0.7f) * 0.7f;
    float worstP = power * (1.0f - libm::powf(difficulty, 0.7f) * 0.5f);
    Vec3 worstShot = (worst + Vec3(0, 0, worstH)).Normalized() * worstP;
    float wf = RandomInRange(w, 0.0f, 1.0f);
    wf = libm::powf(wf, Stat(kStatShot) * 0.7f);
    Vec3 shot = desiredShot * (1.0f - wf) + worstShot * wf;
    float rcf = 0.3f + wf * 0.7f;
    float pcf = 0.7f;
    xRot = -oc.touchInfo.desiredDirection.v[1] * 20.0f + (RandomInRange(w, -20, 20) * rcf);
    yRot = -oc.touchInfo.desiredDirection.v[0] * 20.0f + (RandomInRange(w, -20, 20) * rcf);
    float bta = s.bodyDirectionVec.Angle2D(shot) / PI;
    if (fabsf(bta) > 0.5f) bta = (1.0f - fabsf(bta)) * SignSide(bta);
    bta *= 2.0f;
    float amount = bta * 0.25f;
    shot.Rotate2D(amount * (0.4f + 0.6f * NormalizedClamp(shot.Length(), 0.0f, 70.0f)));
    zRot = amount * -420 + (RandomInRange(w, -20, 20) * pcf);
    return shot;
}

HDN Vec3 GetBestPossibleTouch(World &w, const Ctx &c, int p, const Vec3 &desired, int fn) {
    Humanoid &h = Hum(w, p);
    const AnimationState &cur = h.anim;
    const AnimDerived &d = c.D(cur.anim);
    const Vec3 bm = w.match.ball.momentum;
    float maxBase = 30.0f;
    if (fn == kFnHighPass) maxBase = 42.0f;
    Vec3 r = desired;
    float mpf = d.touchMaxPowerFactor;
    if (mpf == 0.0f) mpf = 1.0f;
    mpf = mpf * 0.7f + 0.3f;
    float maxPower = maxBase * mpf * (1.0f - Clamp(h.decayingPositionOffset.Length() * 2.5f, 0.0f, 0.25f));
    maxPower += bm.Length() * 0.5f;
    if (r.Length() > maxPower) {
        float missing = r.Length() - maxPower;
        r = r.Normalized(0) * maxPower;
        r.v[2] += Clamp(missing, 0.0f, 10.0f) * 0.25f;
    }
    float diff = d.touchDifficultyFactor;
    if (fn == kFnShortPass || fn == kFnLongPass) diff *= (1.0f - GetStatistic(w, c, p, kStatShortPass) * 0.5f);
    if (fn == kFnHighPass) diff *= (1.0f - GetStatistic(w, c, p, kStatHighPass) * 0.5f);
    float df, hf, bmf;
    GetDifficultyFactors(w, c, p, h.decayingPositionOffset, df, hf, bmf);
    float randomRot = df * 0.15f + hf * 0.15f + bmf * 0.3f + diff * 0.5f;
    Vec3 abd = d.ballDirection.Rotated2D(h.startAngle.value() + cur.rotationSmuggleOffset.value());
    if (abd.Length() > 0.01f) {
        float bias = Clamp(randomRot * 1.5f, 0.0f, 1.0f);
        Vec3 native = abd.Normalized(r).Get2D() * r.Length() + r * Vec3(0, 0, 1);
        r = r * (1.0f - bias) + native * bias;
    } else {
        float capped = (0.5f < randomRot) ? 0.5f : randomRot;
        float rot = RandomInRange(w, -0.5f * PI, 0.5f * PI) * capped;
        r.Rotate2D(rot);
    }
    r *= 1.0f - df * 0.3f;
    r.v[2] += df * 1.5f;
    r.v[2] += bm.v[2] * hf * 0.5f + hf * 1.0f;
    r = r * (1.0f - bmf) + bm * bmf;
    r.v[2] += diff * 5.0f * RandomInRange(w, 0.2f, 1.0f);
    return r;
}

// ---- pass and shot aiming ----------------------------------------------------------------------
HDN void GetAutoPass(int passType, const Vec3 &v, Vec3 &dir, float &power) {
    float heightOffset = 0.11f, powerFactor = 1.8f, distExp = 1.4f;
    if (passType == kFnHighPass) {
        heightOffset = 0.45f - NormalizedClamp(v.Length(), 0.0f, 60.0f) * 0.15f;
        powerFactor = 1.15f;
        distExp = 1.4f;
    }
    dir = (v.Normalized(0) + Vec3(0, 0, heightOffset)).Normalized(0);
    power = libm::powf(NormalizedClamp(v.Length(), 0.0f, 60.0f), distExp) * powerFactor;
}

HDN void GetPass(const World &w, int p, int passType, const Vec3 &inDir, float inPower, float autoDirBias, float autoPowerBias,
                 Vec3 &outDir, float &outPower, int &target, int forcedTarget = -1) {
    const SpatialState &s = Sp(w, p);
    const AnimationState &cur = Hum(w, p).anim;
    const int teamID = w.playerTeamID[p];
    bool fullAutoDir = false, fullAutoPower = false;
    if (ExternalControllerActive(w, p)) fullAutoDir = fullAutoPower = true;
    float adb = autoDirBias, apb = autoPowerBias;
    Vec3 ppos = s.position + s.movement.Normalized(0) * 0.2f;
    if (cur.touchFrame != -1) ppos = cur.touchPos.Get2D();
    Vec3 manual = ppos + inDir * Clamp(inPower * 60.0f, 1.0f, 100.0f);
    PlayerList players = TeamActivePlayers(w, teamID);
    if (players.size() < 2) {
        outDir = s.directionVec;
        outPower = 1.0f;
        target = p;
        fullAutoDir = fullAutoPower = false;
        adb = apb = 0.0f;
    }
    int best = p;
    Vec3 autoT = manual;
    if (forcedTarget >= 0) {
        best = forcedTarget;
        const SpatialState &fs = Sp(w, forcedTarget);
        float dur = 0.3f + (fs.position - ppos).Length() * 0.05f;
        dur = libm::powf(Clamp(dur, 0.0f, 1.0f), 0.7f) * 0.7f;
        autoT = fs.position + fs.movement * dur;
    } else {
        float bestRating = 10000;
        autoT = ppos;
        for (int tm : players) {
            if (tm == p) continue;
            const SpatialState &ts = Sp(w, tm);
            float dur = 0.3f + (ts.position - ppos).Length() * 0.05f;
            dur = libm::powf(Clamp(dur, 0.0f, 1.0f), 0.7f) * 0.7f;
            Vec3 tp = ts.position + ts.movement * dur;
            float dr = libm::powf(NormalizedClamp((tp - manual).Length(), 0.0f, 70.0f), 0.8f) * 0.8f;
            float ar = fabsf((tp - ppos).Normalized(0).Angle2D(inDir) / (1.0f * PI)) * 1.0f;
            if (dr + ar < bestRating) {
                bestRating = dr + ar;
                best = tm;
                autoT = tp;
            }
        }
    }
    target = best;
    Vec3 autoRel = autoT - ppos, manualRel = manual - ppos;
    if (forcedTarget >= 0 || (fullAutoDir && fullAutoPower)) {
        adb = 1.0;
        apb = 1.0;
    } else {
        float maxDist = 50.0f;
        // The subtraction from 1 runs in double and rounds once.
        float distF = (float)(1.0 - (double)libm::powf(Clamp((autoRel - manualRel).Length() / maxDist, 0.0f, 1.0f), 1.5f));
        float prox = libm::powf(1.0f - NormalizedClamp((ppos - autoT).Length(), 0.0f, 12.0f), 0.5f);
        if (fullAutoDir) {
            adb = 1.0f;
        } else {
            adb *= distF;
            adb = libm::powf(adb, 1.0f - prox * 0.9f);
        }
        if (fullAutoPower) {
            apb = 1.0f;
        } else {
            apb *= distF;
            apb = Clamp((float)((double)apb * (1.0 + (double)prox)), 0.0f, 1.0f);
        }
    }
    if (passType == kFnLongPass) {
        float td = autoRel.Length() * adb + manualRel.Length() * (1.0f - adb);
        Vec3 off = Vec3(-TeamDynamicSide(w, teamID) * td * 0.2f, 0, 0);
        autoRel += off;
        manualRel += off;
    }
    Vec3 res = (autoRel.Normalized(0) * adb + manualRel.Normalized(0) * (1.0f - adb)).Normalized(manual);
    res *= float(autoRel.Length() * apb + manualRel.Length() * (1.0f - apb));
    GetAutoPass(passType, res, outDir, outPower);
}

HDN Vec3 GetShotDirection(const World &w, int p, const Vec3 &inDir, float autoDirBias) {
    const SpatialState &s = Sp(w, p);
    const int side = TeamDynamicSide(w, w.playerTeamID[p]);
    Vec3 goal = Vec3(side * -kPitchHalfLength, 0, 0);
    Vec3 toGoal = (goal - (s.position + s.movement * 0.12f)).Normalized(0);
    float rel = toGoal.Angle2D(inDir);
    float sf = Clamp((rel / PI) / 0.5f, -1.0f, 1.0f);
    sf = libm::powf(fabsf(sf), 0.7f) * SignSide(sf);
    goal.v[1] = sf * kGoalHalfWidth * 0.9f * side;
    Vec3 autoDir = (goal - (s.position + s.movement * 0.12f)).Normalized(0);
    return (inDir * (1.0f - autoDirBias) + autoDir * autoDirBias).Normalized(inDir);
}

}  // namespace eng
