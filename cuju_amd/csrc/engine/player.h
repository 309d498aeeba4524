// SPDX-License-Identifier: Apache-2.0
// Restates game logic of cuju (Copyright 2026 The cuju Authors), a reimplementation of Google
// Research Football (Copyright 2019 Google LLC); see NOTICE.
// The controllers of the players (reaction times, situation ratings, the gamer's buttons) and the
// tick of a player's humanoid (next frame, next animation, ball touches, smuggles).
// Semantics: include/cuju/simulation/player_controller.h:15-248,
// include/cuju/simulation/humanoid_process.h:87-681.
#pragma once

#include "referee.h"
#include "control.h"
#include "touch.h"

namespace eng {

// Defined with the team AI and the player AI.
HDN void TeamApplyAttackingRun(World &w, const Ctx &c, int teamID, int manualPlayer);
HDN bool PlayerRequestCommand(World &w, const Ctx &c, int p, CommandQueue &q);

// Reaction times in ms.
HD int BaseReactionTime(const World &w, const Ctx &c, int p) {
    return TruncToInt32(roundf(80.0f - GetStatistic(w, c, p, kStatReaction) * 40.0f));
}
HD int PlayerControllerReactionTime(const World &w, const Ctx &c, int p) {
    return TruncToInt32((float)BaseReactionTime(w, c, p) + (1.0f - TeamDifficulty(w, w.playerTeamID[p])) * 100);
}
HD void ElizaControllerProcess(World &w, const Ctx &c, int p) {
    Player &ps = w.match.players[p];
    int rt = PlayerControllerReactionTime(w, c, p);
    if (MatchLastTouchPlayer(w) == p && ps.base.lastTouchType != kTouchAccidental) rt = 0;
    ps.controller.base.mentalImageTime = rt;
}
HD PlayerControllerState &ActiveControllerBase(World &w, int p) {
    if (ExternalControllerActive(w, p)) return HumanGamerOf(w, p).controller.base;
    return w.match.players[p].controller.base;
}

// 1 for open space around `focus`, falling as opponents can reach it within the time.
HDN float CalculateFreeSpace(const World &w, int k, int teamID, const Vec3 &focus, float safeDistance, float futureS) {
    float situation = 0.0f;
    ImageList opp;
    MentalTeamPlayerImages(w, k, 1 - teamID, opp);
    for (int i = 0; i < opp.count; i++) {
        PlayerImagePos &o = opp[i];
        if (o.role == kRoleGoalkeeper) continue;
        o.position = o.position + o.movement * 0.2f;
        Vec3 toFocus = (focus - o.position).Normalized(0) * kSprintVelocity * Clamp(futureS - 0.2f, 0.0f, 1000.0f);
        if (toFocus.Length() > (focus - o.position).Length()) toFocus = focus - o.position;
        o.position += toFocus;
        situation += 1.0f - Clamp((o.position - focus).Length(), 0, safeDistance) / safeDistance;
    }
    return 1.0f - NormalizedClamp(situation, 0.0f, 2.5f);
}
HDN void CalculateTacticalSituation(World &w, int p) {
    Player &ps = w.match.players[p];
    const SpatialState &s = ps.base.humanoid.spatial;
    const int t = w.playerTeamID[p];
    const int side = TeamDynamicSide(w, t);
    const int k = MentalImageIndex(w, ActiveControllerBase(w, p).mentalImageTime);
    float ts = 0.5f;
    Vec3 check = s.position + Vec3(-side, 0, 0) * kSprintVelocity * ts;
    ps.tactical.forwardSpaceRating = CalculateFreeSpace(w, k, t, check, 5.0f, ts);
    ts = 0.1f;
    check = s.position + s.movement * ts;
    ps.tactical.spaceRating = CalculateFreeSpace(w, k, t, check, 5.0f, ts);
    ps.tactical.forwardRating =
        1.0f - Clamp((Vec3(kPitchHalfLength * -side, 0, 0) - s.position).Length() / (kPitchHalfLength * 2.0f), 0.0f, 1.0f);
    ps.tactical.forwardRating = libm::powf(ps.tactical.forwardRating, 1.5f);
}
HD bool TeamHasUniquePossession(const World &w, int teamID) {
    return TeamByID(w, teamID).hasPossession && !TeamByID(w, 1 - teamID).hasPossession;
}
HDN void ControllerCalculateSituation(World &w, int p, PlayerControllerState &ctl) {
    const MatchState &m = w.match;
    const Player &ps = m.players[p];
    const int t = w.playerTeamID[p];
    const Team &team = TeamByID(w, t), &opp = TeamByID(w, 1 - t);
    ctl.hasPossession = ps.hasPossession;
    ctl.hasUniquePossession = ps.hasUniquePossession;
    ctl.teamHasPossession = team.hasPossession;
    ctl.teamHasUniquePossession = TeamHasUniquePossession(w, t);
    ctl.oppTeamHasPossession = opp.hasPossession;
    ctl.oppTeamHasUniquePossession = TeamHasUniquePossession(w, 1 - t);
    ctl.hasBestChanceOfPossession = team.designatedTeamPossessionPlayer == p;
    ctl.teamHasBestPossession = m.bestPossessionTeam == TeamSlot(w, t);
    ctl.possessionAmount = (float)(opp.timeToBallMs + 200) / (float)(ctl.timeNeededMs + 200);
    ctl.teamPossessionAmount = team.teamPossessionAmount;
    ctl.fadingTeamPossessionAmount = team.fadingTeamPossessionAmount;
    if (ctl.hasBestChanceOfPossession) {
        float d = NormalizedClamp((BallPredict(m.ball, 300).Get2D() - ps.base.humanoid.spatial.position).Length(), 2.0f, 14.0f);
        // A product in place of GRF's power of 2.0f gives the same float for every input.
        float db = d * d;
        ctl.fadingTeamPossessionAmount = ctl.fadingTeamPossessionAmount * db + ctl.teamPossessionAmount * (1.0f - db);
    }
    ctl.oppTimeNeededToGetToBall = opp.timeToBallMs;
    ctl.hasBestPossession = ctl.hasPossession && ctl.possessionAmount >= 1.0f;
}

// The gamer's buttons arm an action (1 defensive, 2 a pass or shot whose gauge grows while held).
HDN bool HumanControllerProcess(World &w, const Ctx &c, int p) {
    MatchState &m = w.match;
    HumanControllerState &hc = HumanGamerOf(w, p).controller;
    PlayerControllerState &ctl = hc.base;
    const bool *b = hc.keyboard.buttons;
    // GRF: a gamer reacts with the base reaction time, without the team difficulty.
    int rt = BaseReactionTime(w, c, p);
    if (MatchLastTouchPlayer(w) == p && m.players[p].base.lastTouchType != kTouchAccidental) rt = 0;
    ctl.mentalImageTime = rt;
    Vec3 dir;
    float unused = 0.0f;
    HumanGetKeyboardInput(w, p, dir, unused);
    hc.previousDirection = dir;
    hc.steadyDirection = dir;
    hc.lastSteadyDirectionSnapshotTimeMs = (int32_t)m.actualTimeMs;
    ControllerCalculateSituation(w, p, ctl);
    const int t = w.playerTeamID[p];
    const TeamAI &ai = TeamByID(w, t).ai;
    if (hc.actionMode == 0 && (!m.inSetPiece || ai.taker == p)) {
        float ctx = ctl.possessionAmount - 1.0f;
        if (m.designatedPossessionPlayer == p) {
            ctx = 1.0f;
        } else {
            if (b[kBtnShortPass]) ctx += 0.15f;
            if (b[kBtnLongPass]) ctx += 0.15f;
            if (b[kBtnShot]) ctx += 0.15f;
            if (b[kBtnPressure]) ctx -= 0.15f;
            if (b[kBtnSliding]) ctx -= 0.15f;
            if (b[kBtnTeamPressure]) ctx -= 0.15f;
            if (BallPredict(m.ball, 0).v[2] > 1.5f) ctx += 0.2f;
        }
        // GRF: a held button reads as a fresh press every tick; the last armed button wins.
        if (ctx < 0.0f) {
            if (!m.inSetPiece) {
                const int order[4] = {kBtnPressure, kBtnSliding, kBtnTeamPressure, kBtnKeeperRush};
                for (int i = 0; i < 4; i++)
                    if (b[order[i]]) {
                        hc.actionMode = 1;
                        hc.actionButton = order[i];
                    }
            }
        } else {
            bool allowHigh = true, allowShot = true;
            if (ai.taker == p && ai.setPieceType == kModeThrowIn) allowHigh = allowShot = false;
            if (b[kBtnShortPass]) {
                hc.actionMode = 2;
                hc.actionButton = kBtnShortPass;
            }
            if (b[kBtnLongPass]) {
                hc.actionMode = 2;
                hc.actionButton = kBtnLongPass;
            }
            if (b[kBtnHighPass] && allowHigh) {
                hc.actionMode = 2;
                hc.actionButton = kBtnHighPass;
            }
            if (b[kBtnShot] && allowShot) {
                hc.actionMode = 2;
                hc.actionButton = kBtnShot;
            }
        }
    }
    if (hc.actionMode == 2) {
        if (b[hc.actionButton]) {
            hc.gaugeMs += 10;
            hc.gaugeMs = (int)Clamp((float)hc.gaugeMs, 10, 1000);
            hc.actionBufferTimeMs = 0;
        } else {
            hc.actionBufferTimeMs += 10;
        }
    }
    if (b[kBtnSwitch] && ctl.hasPossession) TeamApplyAttackingRun(w, c, t, -1);
    return true;
}

// ---- the humanoid tick of a player ------------------------------------------------------------------

// Whether a player may drop its animation for a fresh command this tick (GRF's requeue).
HDN bool MayRequeue(World &w, const Ctx &c, int p, const Anim &a, int k) {
    const Player &ps = w.match.players[p];
    const Humanoid &h = ps.base.humanoid;
    const AnimationState &cur = h.anim;
    const int t = w.playerTeamID[p];
    const Team &team = TeamByID(w, t);
    float actionDistance = ((h.spatial.position + h.spatial.movement * 0.1f) - BallPredict(w.match.ball, 100).Get2D()).Length();
    const uint64_t second = TeamSlot(w, t) == 1 ? 1 : 0;
    const uint64_t now = w.match.actualTimeMs;
    bool frameOk = false;
    // Players closer to the action requeue more often; the second team is phase-shifted.
    if (w.match.designatedPossessionPlayer == p && actionDistance < 3.0f) frameOk = ((now + second * 10) % 20) == 0;
    else if (w.match.designatedPossessionPlayer == p) frameOk = ((now + second * 10) % 30) == 0;
    else if (team.designatedTeamPossessionPlayer == p) frameOk = ((now + second * 20) % 40) == 0;
    else if (actionDistance < 5.0f) frameOk = ((now + second * 20) % 50) == 0;
    else if (actionDistance < 10.0f) frameOk = ((now + second * 40) % 80) == 0;
    if (!frameOk) return false;
    float ballDistance = (MentalBallPrediction(w, k, 500).Get2D() - h.spatial.position).Length();
    const bool touchPending = cur.frameNum < cur.touchFrame;
    return ((cur.functionType == kFnMovement && !ps.hasPossession && ballDistance < 16.0f) ||
            (cur.functionType == kFnMovement && ps.hasPossession) || (cur.functionType == kFnTrap && touchPending) ||
            (cur.functionType == kFnBallControl && touchPending)) &&
           a.incomingSpecialState == kStrEmpty && a.outgoingSpecialState == kStrEmpty;
}

// Touch of a pass: the command's plan, refined towards a fresh pass decision within 0.15 pi.
HDN bool PassTouch(World &w, const Ctx &c, int p, const AnimationState &cur, Vec3 &touch, float &zRot) {
    const Humanoid &h = Hum(w, p);
    const TouchInformation &ti = cur.originatingCommand.touchInfo;
    Vec3 dir = ti.desiredDirection;
    float power = ti.desiredPower;
    int target = ti.targetPlayer;
    Vec3 inDir = ti.inputDirection;
    if (ExternalControllerActive(w, p)) inDir = HumanGetDirection(w, p);
    Vec3 tDir = dir;
    float tPower = power;
    int tTarget = -1;
    AimPass(w, p, cur.originatingCommand.desiredFunctionType, inDir, ti.inputPower, ti.autoDirectionBias, ti.autoPowerBias, tDir,
            tPower, tTarget, ti.forcedTargetPlayer);
    const float maxDev = 0.15f * PI;
    float diff = tDir.Get2D().Angle2D(dir.Get2D());
    if (fabsf(diff) <= maxDev) {
        dir = tDir;
        power = tPower;
        target = tTarget;
    } else if (fabsf(diff) < 2.0f * maxDev) {
        float cd = Clamp(diff, -maxDev, maxDev);
        dir = dir.Rotated2D(cd);
        if (tTarget != target) {
            float rb = NormalizedClamp(fabsf(cd), 0.0f, fabsf(diff));
            power = power * (1.0f - rb) + tPower * rb;
            target = tTarget;
        } else {
            power = tPower;
        }
    }
    if (target >= 0 && !TeamSelectPlayer(w, c, w.playerTeamID[p], target)) return false;
    touch = dir * 36 * (power + 0.3f);
    touch = AttainableTouch(w, c, p, touch, cur.functionType);
    float amount = CurlAmount(h.spatial.bodyDirectionVec, touch);
    if (cur.functionType == kFnHighPass) amount *= 0.2f;
    CurlKick(touch, amount);
    zRot = amount * -340;
    return true;
}

// The touch of the ball at the animation's touch frame, by function type.
HDN bool AnimationTouch(World &w, const Ctx &c, int p, const Anim &a, const AnimDerived &d, float bumpy) {
    Player &ps = w.match.players[p];
    Humanoid &h = ps.base.humanoid;
    AnimationState &cur = h.anim;
    const int t = w.playerTeamID[p];
    const Vec3 bm = w.match.ball.momentum;
    const float nba = h.startAngle.value() + a.outgoingAngle.value() + a.outgoingBodyAngle.value() + cur.rotationSmuggleEnd.value();
    PList pl{cur.positions.e, cur.positions.count};
    const Vec3 outMov = OutgoingMovementOf(pl);
    const int fn = cur.functionType;
    const bool knockOn = (cur.originatingCommand.modifier & kModifierKnockOn) != 0;
    // Each function type computes the ball's new momentum and spin; the touch, the spin and the
    // last touch then have one call site each, so that matches of a wavefront touching the ball
    // in different ways run the ball's new prediction together. Per environment the calls and
    // their order are GRF's.
    Vec3 tv;
    bool touch = true, rotate = true;
    float rx = 0, ry = 0, rz = 0, bias = 1.0f;
    int touchType = d.touchType;
    if (fn == kFnTrap || (fn == kFnBallControl && !ps.hasPossession)) {
        const Kick k = TrapKick(w, c, p, h, nba, outMov);
        tv = k.momentum;
        rx = k.xRot;
        ry = k.yRot;
        if (knockOn) tv *= 1.35f;
        tv = tv * (1.0f - bumpy) + bm * bumpy;
        bias = 0.5f * (1.0f - bumpy);
    } else if (fn == kFnBallControl) {
        const Kick k = BallControlKick(w, c, p, h, nba, outMov);
        tv = k.momentum;
        rx = k.xRot;
        ry = k.yRot;
        if (knockOn) tv *= 1.35f;
        tv = tv * (1.0f - bumpy) + bm * bumpy;
        bias = 0.6f * (1.0f - bumpy);
    } else if (fn == kFnInterfere) {
        const Kick k = TrapKick(w, c, p, h, nba, outMov);
        rx = k.xRot;
        ry = k.yRot;
        tv = k.momentum * 0.5f + (BallPredict(w.match.ball, 0).Get2D() - h.spatial.position).Normalized() * 4.0f +
             Vec3(0, 0, RandomInRange(w, 0.5f, 1.5f));
        tv = tv * (1.0f - bumpy) + bm * bumpy;
        // GRF passes the bias as the z rotation here, with the default bias of 1.
        rz = 0.3f * (1.0f - bumpy);
        touchType = kTouchAccidental;
    } else if (fn == kFnSliding) {
        tv = d.ballDirection.Rotated2D(h.spatial.angle.value());
        tv = tv * 6.0f + w.match.ball.momentum * -0.28f;
        tv += Vec3(0, 0, 6);
        tv = tv * (1.0f - bumpy) + bm * bumpy;
        rotate = false;
        touchType = kTouchAccidental;
    } else if (fn == kFnShortPass || fn == kFnLongPass || fn == kFnHighPass) {
        if (!PassTouch(w, c, p, cur, tv, rz)) return false;
        tv = tv * (1.0f - bumpy) + bm * bumpy;
        float forwardness = fn == kFnHighPass ? -1.3f : 3.5f;
        float tl = Clamp(tv.Length(), 0.0, 15.0);
        rx = tv.Normalized(0).v[1] * (tl * forwardness);
        ry = tv.Normalized(0).v[0] * (tl * forwardness);
        bias = 0.9f * (1.0f - bumpy);
    } else if (fn == kFnShot) {
        // GRF computes a shot direction here and discards it; the call has no side effects.
        tv = ShotKick(w, c, p, cur, h.spatial, h.decayingPositionOffset, rx, ry, rz);
        tv = tv * (1.0f - bumpy) + bm * bumpy;
        bias = 0.7f * (1.0f - bumpy);
    } else if (fn == kFnDeflect) {
        bool canRetain = d.outgoingRetainRawValue != kStrEmpty && w.match.ballRetainer == -1;
        float velDiff = NormalizedClamp((w.match.ball.momentum - h.spatial.movement).Length(), 0.0f, 40.0f);
        float reactDiff = 0.0f;
        int ltp = TeamByID(w, 1 - t).lastTouchPlayer;
        if (ltp >= 0)
            reactDiff = libm::powf(
                GetLastTouchBias(w, ltp, TruncToInt32(1200 - GetStatistic(w, c, p, kStatReaction) * 400)), 0.6f);
        if ((1.0f - velDiff) * (1.0f - reactDiff) < 0.3f) canRetain = false;
        if (canRetain) {
            w.match.ballRetainer = p;
            touch = rotate = false;
        } else {
            Vec3 bmov = w.match.ball.momentum.Get2D();
            Vec3 pmov = h.spatial.movement;
            float lateral = RandomInRange(w, -1, 1);
            tv = (-bmov * 0.1f + pmov * 2.0f + Vec3(-TeamDynamicSide(w, t), 0, 0) * 4.0f + Vec3(0, lateral, 0)).Normalized(0) *
                 (bmov.Length() * 0.3f + pmov.Length() * 2.5f);
            tv.v[2] += 1.2f;
            tv = tv * (1.0f - bumpy) + bm * bumpy;
            bias = 0.2f * (1.0f - bumpy);
        }
        touchType = kTouchAccidental;
    } else {
        return true;
    }
    if (touch) BallTouch(w, c, tv);
    if (rotate) BallSetRotation(w, rx, ry, rz, bias);
    return TeamSetLastTouchPlayer(w, c, p, touchType);
}

// A humanoid's tick (humanoid_process.h:89-681) in three parts: the frame advance that decides
// whether the animation is interrupted, the interruption (command request and animation
// selection, the expensive part), and the rest. Run in that order they are the whole tick; the
// team loop lets the matches of a wavefront meet at the interruption.
HDN void HumanoidProcessBegin(World &w, const Ctx &c, int p) {
    ENG_SCOPE(12);
    Player &ps = w.match.players[p];
    Humanoid &h = ps.base.humanoid;
    AnimationState &cur = h.anim;
    const int t = w.playerTeamID[p];
    const int k = MentalImageIndex(w, h.mentalImageTime);
    h.decayingPositionOffset *= 0.95f;
    if ((double)h.decayingPositionOffset.Length() < 0.005) h.decayingPositionOffset = Vec3(0);
    h.decayingDifficultyFactor = Clamp(h.decayingDifficultyFactor - 0.002f, 0.0f, 1.0f);
    h.mentalImageTime = w.match.lastTouchTeamID == t ? 0 : GetReactionTimeMs(w, c, p);
    CalculateSpatialState(c, h);
    h.spatial.positionOffsetMovement = Vec3(0);
    cur.frameNum++;
    h.prevAnimFrameNum++;
    {
        const Anim &a = c.A(cur.anim);
        if (cur.frameNum == a.frameCount - 1 && h.interruptAnim == kIntNone) h.interruptAnim = kIntSwitch;
        if (h.interruptAnim == kIntNone && MayRequeue(w, c, p, a, k)) h.interruptAnim = kIntReQueue;
    }
}
HDN bool HumanoidProcessInterrupt(World &w, const Ctx &c, int p) {
    Humanoid &h = w.match.players[p].base.humanoid;
    AnimationState &cur = h.anim;
    {
        ENG_SCOPE(30);
        CommandQueue &q = c.ws->commands;
        q.clear();
        if (h.interruptAnim == kIntTrip && h.tripType != 0) {
            AddTripCommandToQueue(h, q, h.tripType);
            h.tripType = 0;
            q.push_back(GetBasicMovementCommand(h, h.spatial.floatVelocity));
        } else {
            if (!PlayerRequestCommand(w, c, p, q)) return false;
        }
        bool found = false, preferPassAndShot = false;
        for (int i = 0; i < q.count; i++) {
            if (IsPassOrShot(q[i].desiredFunctionType)) preferPassAndShot = true;
            Selector sel(w, c, p);
            SelectResult r = sel.SelectPlayerAnimation(q[i], h.interruptAnim, preferPassAndShot);
            if (r == kSelectUnsupported) return false;
            found = r == kSelectTrue;
            if (found) break;
        }
        if (h.interruptAnim == kIntSwitch && !found) {
            Fatal("no animation applies to the humanoid");
            return false;
        }
        if (found) {
            h.startPos = h.spatial.position;
            h.startAngle = h.spatial.angle;
            {
                Selector sel(w, c, p);
                Vec3 np;
                float na;
                sel.PredictedPose(np, na);
                h.nextStartPos = np;
                h.nextStartAngle.set(na);
            }
            h.applyBuf.anim = cur.anim;
            h.applyBuf.smooth = true;
            const int fn = cur.functionType;
            h.applyBuf.smoothFactor =
                (h.interruptAnim == kIntSwitch && h.prevAnimFunctionType == kFnMovement && fn == kFnMovement) ? 0.0f : 1.0f;
            if (fn == kFnShot || fn == kFnShortPass || fn == kFnHighPass || fn == kFnDeflect || fn == kFnSliding ||
                fn == kFnBallControl || fn == kFnTrap)
                h.applyBuf.smoothFactor = 0.8f;
            float diff = c.D(cur.anim).difficultyFactor;
            if (diff > h.decayingDifficultyFactor) h.decayingDifficultyFactor = diff;
            if (h.interruptAnim == kIntReQueue && h.prevAnimFunctionType == fn) h.requeueDelayFrames = 22;
        }
    }
    return true;
}
HDN bool HumanoidProcessEnd(World &w, const Ctx &c, int p) {
    Player &ps = w.match.players[p];
    Humanoid &h = ps.base.humanoid;
    AnimationState &cur = h.anim;
    const int t = w.playerTeamID[p];
    const Ball &ball = w.match.ball;
    h.requeueDelayFrames = h.requeueDelayFrames - 1 > 0 ? h.requeueDelayFrames - 1 : 0;
    h.interruptAnim = kIntNone;
    const Anim &a = c.A(cur.anim);
    {
        float now = (BallPredict(ball, 0).Get2D() - h.spatial.position).Length();
        float future = (BallPredict(ball, 200).Get2D() - (h.spatial.position + h.spatial.movement * 0.2f)).Length();
        float ltb = GetLastTouchBias(w, p, 1500);
        float oltb = TeamLastTouchBias(w, 1 - t, 240);
        if (p == w.match.designatedPossessionPlayer &&
            ((ltb <= 0.01f && oltb <= 0.01f && cur.functionType == kFnMovement && now < 0.6f && future > 0.65f && future > now) ||
             (ltb <= 0.7f && ps.hasPossession && cur.functionType == kFnTrip && now < 0.4f)) &&
            BallPredict(ball, 0).v[2] < 1.6f)
            ps.triggerControlledBallCollision = true;
    }
    bool controlled = ps.triggerControlledBallCollision;
    if (controlled) ps.triggerControlledBallCollision = false;
    const AnimDerived &d = c.D(cur.anim);
    if (controlled && cur.touchFrame == -1) {
        Vec3 bm = w.match.ball.momentum;
        float nba = h.startAngle.value() + a.outgoingAngle.value() + a.outgoingBodyAngle.value() + cur.rotationSmuggleEnd.value();
        PList pl{cur.positions.e, cur.positions.count};
        const Kick k = TrapKick(w, c, p, h, nba, OutgoingMovementOf(pl));
        const float xr = k.xRot, yr = k.yRot;
        Vec3 tv = k.momentum;
        if (cur.originatingCommand.modifier & kModifierKnockOn) tv *= 1.35f;
        const float bumpy = 0.0f;
        tv = tv * (1.0f - bumpy) + bm * bumpy;
        BallTouch(w, c, tv);
        BallSetRotation(w, xr, yr, 0, 0.2f * (1.0f - bumpy));
        if (!TeamSetLastTouchPlayer(w, c, p, d.touchType)) return false;
    }
    if (cur.touchFrame == cur.frameNum) {
        Vec3 desiredBall;
        for (int i = 0; i < a.footballCount; i++) {
            const FootballKey &fk = c.t->football[a.footballFirst + i];
            if (fk.frame == cur.touchFrame) desiredBall = fk.position;
        }
        float touchable = 0.4f;
        float full = (BallPredict(w.match.ball, 0) - (cur.touchPos + cur.positionOffset)).Length();
        if (a.incomingRetainState != kStrEmpty) {
            full = 0.0f;
            touchable = 1.0f;
        }
        float bumpy = full / touchable;
        bumpy = Clamp(bumpy - 0.001f, 0.0f, 1.0f);
        bumpy = Curve(bumpy, 1.0f);
        bumpy = Curve(bumpy, 0.5f);
        if (full < touchable && fabsf(desiredBall.v[2] - BallPredict(w.match.ball, 0).v[2]) < 1.0f)
            if (!AnimationTouch(w, c, p, a, d, bumpy)) return false;
    }
    if (w.match.ballRetainer == p) {
        if ((cur.touchFrame <= cur.frameNum && d.outgoingRetainRawValue != kStrEmpty) ||
            (cur.touchFrame > cur.frameNum && a.incomingRetainState != kStrEmpty) ||
            (d.incomingRetainRawValue != kStrEmpty && d.outgoingRetainRawValue != kStrEmpty)) {
            int bp = -1;
            if (d.outgoingRetainRawValue != kStrEmpty) bp = d.outgoingRetainBodyPart;
            if (bp < 0 && d.incomingRetainRawValue != kStrEmpty) bp = d.incomingRetainBodyPart;
            if (bp < 0) {
                Fatal("an animation that retains the ball names no body part");
                return false;
            }
            const Skeleton &sk = c.skeletons[p];
            Derived der[kHumanoidNodes];
            DeriveNodes(sk, h.nodes, der);
            const Derived &node = der[sk.nodeMap[bp]];
            BallTouch(w, c, Vec3(0));
            // BallSetPosition predicts again from its own position before anything reads the
            // predictions, so this rotation's prediction is left out.
            BallSetRotation(w, 0, 0, 0, 1.0f, false);
            BallSetPosition(w, node.position + node.rotation * Vec3(0, 0, -0.36f));
            if (!TeamSetLastTouchPlayer(w, c, p, kTouchNonKicked)) return false;
        } else {
            w.match.ballRetainer = -1;
        }
    }
    const int frames = a.frameCount - 1;
    // Smuggles spread the planned offsets over the frames, weighted by a raised cosine.
    if (cur.touchFrame != -1 && cur.frameNum <= cur.touchFrame) {
        float v = libm::cosf((cur.frameNum / (float)(cur.touchFrame + 1) - 0.5f) * PI * 2.0f) + 1.0f;
        v = v * 0.1f + 0.9f;
        h.spatial.actionSmuggleMovement = (cur.actionSmuggle / (float)(cur.touchFrame + 1)) * v * 100.0f;
        cur.actionSmuggleOffset += h.spatial.actionSmuggleMovement / 100.0f;
    } else {
        h.spatial.actionSmuggleMovement = Vec3(0);
    }
    if (cur.touchFrame == -1 && cur.frameNum <= frames) {
        float v = libm::cosf((cur.frameNum / (float)(frames + 1) - 0.5f) * PI * 2.0f) + 1.0f;
        v = v * 0.1f + 0.9f;
        h.spatial.movementSmuggleMovement = (cur.movementSmuggle / (float)(frames + 1)) * v * 100.0f;
        cur.movementSmuggleOffset += h.spatial.movementSmuggleMovement / 100.0f;
    } else {
        h.spatial.movementSmuggleMovement = Vec3(0);
    }
    const int beginFrames = 16;
    int cap = beginFrames < frames + 1 ? beginFrames : frames + 1;
    float capped = MinF(1.0f, (cur.frameNum + 1) / (float)cap);
    float beginBias = capped, endBias = capped;
    if (cur.touchFrame != -1) {
        int capT = beginFrames < cur.touchFrame + 1 ? beginFrames : cur.touchFrame + 1;
        beginBias = MinF(1.0f, (cur.frameNum + 1) / (float)capT);
        endBias = cur.frameNum > cur.touchFrame ? (cur.frameNum - cur.touchFrame) / (float)(frames - cur.touchFrame) : 0.0f;
    }
    cur.rotationSmuggleOffset.set(cur.rotationSmuggleBegin.value() * (1.0f - beginBias) + cur.rotationSmuggleEnd.value() * endBias);
    if (w.match.ballRetainer == p && Formation(w, c, p).role == kRoleGoalkeeper && !w.match.inSetPiece && w.match.inPlay) {
        // A keeper holding the ball is kept inside the box.
        const int side = TeamDynamicSide(w, t);
        const Vec3 bn = BallPredict(w.match.ball, 0);
        if (bn.v[1] > 20.05f) OffsetPosition(w, p, Vec3(0, Clamp(20.05f - bn.v[1], -0.5f, 0.5f), 0) * 0.3f);
        if (bn.v[1] < -20.05f) OffsetPosition(w, p, Vec3(0, Clamp(-20.05f - bn.v[1], -0.5f, 0.5f), 0) * 0.3f);
        if (bn.v[0] * -side > -kPitchHalfLength + 16.4f)
            OffsetPosition(w, p, Vec3(Clamp((-kPitchHalfLength + 16.4f) - bn.v[0] * -side, -0.5f, 0.5f), 0, 0) * -side * 0.3f);
        if (bn.v[0] * -side < -kPitchHalfLength + 0.1f)
            OffsetPosition(w, p, Vec3(Clamp((-kPitchHalfLength + 0.1f) - bn.v[0] * -side, -0.5f, 0.5f), 0, 0) * -side * 0.4f);
    }
    h.applyBuf.frameNum = cur.frameNum;
    if ((uint32_t)cur.positions.count > (uint32_t)cur.frameNum) {
        h.applyBuf.position = h.startPos + cur.positions[cur.frameNum] + cur.actionSmuggleOffset +
                              cur.actionSmuggleSustainOffset + cur.movementSmuggleOffset;
        h.applyBuf.orientation.set(h.startAngle.value() + cur.rotationSmuggleOffset.value());
        h.applyBuf.noPos = true;
    } else {
        h.applyBuf.position = h.startPos + cur.actionSmuggleOffset + cur.actionSmuggleSustainOffset + cur.movementSmuggleOffset;
        h.applyBuf.orientation = h.startAngle;
        h.applyBuf.noPos = false;
    }
    for (int i = 0; i < kBodyParts; i++) h.applyBuf.offsets[i] = h.offsets[i];
    return true;
}

}  // namespace eng
