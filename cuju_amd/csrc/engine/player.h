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

// How much the gamer's buttons lean toward attacking: the player's possession amount less 1 (1
// for the designated player), plus 0.15 for each pass or shot button held, less 0.15 for each
// pressure or sliding button, plus 0.2 for a ball above 1.5 m.
HD float AttackLean(const World &w, int p, const PlayerControllerState &ctl, const bool *b) {
    if (w.match.designatedPossessionPlayer == p) return 1.0f;
    float lean = ctl.possessionAmount - 1.0f;
    if (b[kBtnShortPass]) lean += 0.15f;
    if (b[kBtnLongPass]) lean += 0.15f;
    if (b[kBtnShot]) lean += 0.15f;
    if (b[kBtnPressure]) lean -= 0.15f;
    if (b[kBtnSliding]) lean -= 0.15f;
    if (b[kBtnTeamPressure]) lean -= 0.15f;
    if (BallPredict(w.match.ball, 0).v[2] > 1.5f) lean += 0.2f;
    return lean;
}
// With no action armed (and, at a set piece, only for the taker) the buttons arm one: leaning to
// defence, the last held of pressure, sliding, team pressure and keeper rush (not at a set
// piece), as action 1; otherwise the last held of short pass, long pass, high pass and shot (a
// throw-in's taker neither lofts nor shoots), as action 2. GRF reads a held button as a fresh
// press every tick.
HD void ArmGamerAction(World &w, int p, HumanControllerState &hc) {
    const MatchState &m = w.match;
    const TeamAI &ai = TeamByID(w, w.playerTeamID[p]).ai;
    const bool *b = hc.keyboard.buttons;
    if (!(hc.actionMode == 0 && (!m.inSetPiece || ai.taker == p))) return;
    auto arm = [&](int mode, int button) {
        hc.actionMode = mode;
        hc.actionButton = button;
    };
    if (AttackLean(w, p, hc.base, b) < 0.0f) {
        if (m.inSetPiece) return;
        const int defensive[4] = {kBtnPressure, kBtnSliding, kBtnTeamPressure, kBtnKeeperRush};
        for (int i = 0; i < 4; i++)
            if (b[defensive[i]]) arm(1, defensive[i]);
        return;
    }
    const bool throwIn = ai.taker == p && ai.setPieceType == kModeThrowIn;
    if (b[kBtnShortPass]) arm(2, kBtnShortPass);
    if (b[kBtnLongPass]) arm(2, kBtnLongPass);
    if (b[kBtnHighPass] && !throwIn) arm(2, kBtnHighPass);
    if (b[kBtnShot] && !throwIn) arm(2, kBtnShot);
}
// A gamer-controlled player's controller tick: the reaction time (the base one, without the team
// difficulty; none right after its own touch), the steady direction, the situation, the armed
// action and, for a pass or shot, its gauge (10 ms a tick while held, 10 to 1000 ms) or the time
// since release. The switch button with the ball starts an attacking run.
HDN bool HumanControllerProcess(World &w, const Ctx &c, int p) {
    MatchState &m = w.match;
    HumanControllerState &hc = HumanGamerOf(w, p).controller;
    PlayerControllerState &ctl = hc.base;
    const bool *b = hc.keyboard.buttons;
    int reaction = BaseReactionTime(w, c, p);
    if (MatchLastTouchPlayer(w) == p && m.players[p].base.lastTouchType != kTouchAccidental) reaction = 0;
    ctl.mentalImageTime = reaction;
    Vec3 dir;
    float unused = 0.0f;
    HumanGetKeyboardInput(w, p, dir, unused);
    hc.previousDirection = dir;
    hc.steadyDirection = dir;
    hc.lastSteadyDirectionSnapshotTimeMs = (int32_t)m.actualTimeMs;
    ControllerCalculateSituation(w, p, ctl);
    ArmGamerAction(w, p, hc);
    if (hc.actionMode == 2) {
        if (b[hc.actionButton]) {
            hc.gaugeMs += 10;
            hc.gaugeMs = (int)Clamp((float)hc.gaugeMs, 10, 1000);
            hc.actionBufferTimeMs = 0;
        } else {
            hc.actionBufferTimeMs += 10;
        }
    }
    if (b[kBtnSwitch] && ctl.hasPossession) TeamApplyAttackingRun(w, c, w.playerTeamID[p], -1);
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

// A pass's aim: direction, power and receiver.
struct PassAim {
    Vec3 dir;
    float power;
    int target;
};
// The command's pass aim moved toward a fresh one taken at the touch (the gamer's current
// direction for a gamer's player): the fresh aim within 0.15 pi of the planned direction; up to
// 0.3 pi, the planned direction turned by 0.15 pi toward it, with the fresh power (blended by the
// turn's share for a new receiver); beyond that, the plan.
HD PassAim RefinePassAim(World &w, int p, const AnimationState &cur) {
    const TouchInformation &ti = cur.originatingCommand.touchInfo;
    PassAim plan{ti.desiredDirection, ti.desiredPower, ti.targetPlayer};
    const Vec3 input = ExternalControllerActive(w, p) ? HumanGetDirection(w, p) : ti.inputDirection;
    PassAim fresh{plan.dir, plan.power, -1};
    AimPass(w, p, cur.originatingCommand.desiredFunctionType, input, ti.inputPower, ti.autoDirectionBias, ti.autoPowerBias,
            fresh.dir, fresh.power, fresh.target, ti.forcedTargetPlayer);
    const float maxTurn = 0.15f * PI;
    const float turn = fresh.dir.Get2D().Angle2D(plan.dir.Get2D());
    if (fabsf(turn) <= maxTurn) return fresh;
    if (!(fabsf(turn) < 2.0f * maxTurn)) return plan;
    const float applied = Clamp(turn, -maxTurn, maxTurn);
    plan.dir = plan.dir.Rotated2D(applied);
    if (fresh.target != plan.target) {
        const float share = NormalizedClamp(fabsf(applied), 0.0f, fabsf(turn));
        plan.power = plan.power * (1.0f - share) + fresh.power * share;
        plan.target = fresh.target;
    } else {
        plan.power = fresh.power;
    }
    return plan;
}
// A pass's touch: the refined aim's receiver selected (when there is one), 36 m/s per unit of
// power plus 0.3, made attainable, and curled away from the body (a fifth as much for a high
// pass), with the matching z spin.
HDN bool PassTouch(World &w, const Ctx &c, int p, const AnimationState &cur, Vec3 &touch, float &zRot) {
    const Humanoid &h = Hum(w, p);
    const PassAim aim = RefinePassAim(w, p, cur);
    if (aim.target >= 0 && !TeamSelectPlayer(w, c, w.playerTeamID[p], aim.target)) return false;
    touch = aim.dir * 36 * (aim.power + 0.3f);
    touch = AttainableTouch(w, c, p, touch, cur.functionType);
    float amount = CurlAmount(h.spatial.bodyDirectionVec, touch);
    if (cur.functionType == kFnHighPass) amount *= 0.2f;
    CurlKick(touch, amount);
    zRot = amount * -340;
    return true;
}

// What a touch does to the ball: its momentum (already blended with the incoming momentum by the
// touch's bumpiness), the spin and its bias, whether the ball is touched and spun at all, and the
// touch type recorded.
struct TouchOutcome {
    Vec3 momentum;
    float rx = 0, ry = 0, rz = 0, bias = 1.0f;
    bool touch = true, rotate = true;
    int type = 0;
};
// The angle the body faces after the animation: its start angle, outgoing angle and outgoing
// body angle plus the end rotation smuggle.
HD float NextBodyAngle(const Humanoid &h, const Anim &a) {
    return h.startAngle.value() + a.outgoingAngle.value() + a.outgoingBodyAngle.value() + h.anim.rotationSmuggleEnd.value();
}
// A deflection retains the ball when the animation can and nobody retains it, unless the ball
// comes fast (to 40 m/s relative) and just off an opponent (slower with reaction): then it goes
// upfield, mostly along the humanoid's movement, with a lateral draw, lifted 1.2 m/s.
HD void DeflectionOutcome(World &w, const Ctx &c, int p, const AnimDerived &d, TouchOutcome &o) {
    const Humanoid &h = Hum(w, p);
    const int t = w.playerTeamID[p];
    bool retain = d.outgoingRetainRawValue != kStrEmpty && w.match.ballRetainer == -1;
    const float fast = NormalizedClamp((w.match.ball.momentum - h.spatial.movement).Length(), 0.0f, 40.0f);
    float surprise = 0.0f;
    const int last = TeamByID(w, 1 - t).lastTouchPlayer;
    if (last >= 0) surprise = libm::powf(GetLastTouchBias(w, last, TruncToInt32(1200 - GetStatistic(w, c, p, kStatReaction) * 400)), 0.6f);
    if ((1.0f - fast) * (1.0f - surprise) < 0.3f) retain = false;
    o.type = kTouchAccidental;
    if (retain) {
        w.match.ballRetainer = p;
        o.touch = o.rotate = false;
        return;
    }
    const Vec3 ball = w.match.ball.momentum.Get2D(), own = h.spatial.movement;
    const float lateral = RandomInRange(w, -1, 1);
    o.momentum = (-ball * 0.1f + own * 2.0f + Vec3(-TeamDynamicSide(w, t), 0, 0) * 4.0f + Vec3(0, lateral, 0)).Normalized(0) *
                 (ball.Length() * 0.3f + own.Length() * 2.5f);
    o.momentum.v[2] += 1.2f;
}
// The touch of the ball at the animation's touch frame, by function type: traps (and ball
// control off the ball) and ball control kick toward a planned point (knock-ons 35% harder);
// interference halves a trap's kick and knocks the ball 4 m/s away from the body with a lift
// draw; sliding kicks along the animation's ball direction; passes and shots aim; deflections may
// retain. Every momentum but a retained ball's blends with the incoming one by the bumpiness.
// The touch, the spin and the record have one call site each, so that matches of a wavefront
// touching the ball in different ways run the ball's new prediction together; per environment the
// calls and their order are GRF's.
HDN bool AnimationTouch(World &w, const Ctx &c, int p, const Anim &a, const AnimDerived &d, float bumpy) {
    Player &ps = w.match.players[p];
    Humanoid &h = ps.base.humanoid;
    const AnimationState &cur = h.anim;
    const Vec3 incoming = w.match.ball.momentum;
    const float nextBody = NextBodyAngle(h, a);
    const Vec3 outMov = OutgoingMovementOf(PList{h.anim.positions.e, h.anim.positions.count});
    const int fn = cur.functionType;
    const bool knockOn = (cur.originatingCommand.modifier & kModifierKnockOn) != 0;
    TouchOutcome o;
    o.type = d.touchType;
    if (fn == kFnTrap || fn == kFnBallControl || fn == kFnInterfere) {
        const bool trap = fn != kFnBallControl || !ps.hasPossession;
        const Kick k = trap ? TrapKick(w, c, p, h, nextBody, outMov) : BallControlKick(w, c, p, h, nextBody, outMov);
        o.rx = k.xRot;
        o.ry = k.yRot;
        if (fn == kFnInterfere) {
            o.momentum = k.momentum * 0.5f + (BallPredict(w.match.ball, 0).Get2D() - h.spatial.position).Normalized() * 4.0f +
                         Vec3(0, 0, RandomInRange(w, 0.5f, 1.5f));
            // GRF passes the bias as the z rotation here, with the default bias of 1.
            o.rz = 0.3f * (1.0f - bumpy);
            o.type = kTouchAccidental;
        } else {
            o.momentum = k.momentum;
            if (knockOn) o.momentum *= 1.35f;
            o.bias = (trap ? 0.5f : 0.6f) * (1.0f - bumpy);
        }
    } else if (fn == kFnSliding) {
        o.momentum = d.ballDirection.Rotated2D(h.spatial.angle.value());
        o.momentum = o.momentum * 6.0f + w.match.ball.momentum * -0.28f;
        o.momentum += Vec3(0, 0, 6);
        o.rotate = false;
        o.type = kTouchAccidental;
    } else if (fn == kFnShortPass || fn == kFnLongPass || fn == kFnHighPass) {
        if (!PassTouch(w, c, p, cur, o.momentum, o.rz)) return false;
    } else if (fn == kFnShot) {
        // GRF computes a shot direction here and discards it; the call has no side effects.
        o.momentum = ShotKick(w, c, p, cur, h.spatial, h.decayingPositionOffset, o.rx, o.ry, o.rz);
        o.bias = 0.7f * (1.0f - bumpy);
    } else if (fn == kFnDeflect) {
        DeflectionOutcome(w, c, p, d, o);
        if (o.touch) o.bias = 0.2f * (1.0f - bumpy);
    } else {
        return true;
    }
    if (o.touch) o.momentum = o.momentum * (1.0f - bumpy) + incoming * bumpy;
    if (fn == kFnShortPass || fn == kFnLongPass || fn == kFnHighPass) {
        // Passes spin forward (high passes back) by their speed, up to 15 m/s.
        const float forwardness = fn == kFnHighPass ? -1.3f : 3.5f;
        const float speed = Clamp(o.momentum.Length(), 0.0, 15.0);
        o.rx = o.momentum.Normalized(0).v[1] * (speed * forwardness);
        o.ry = o.momentum.Normalized(0).v[0] * (speed * forwardness);
        o.bias = 0.9f * (1.0f - bumpy);
    }
    if (o.touch) BallTouch(w, c, o.momentum);
    if (o.rotate) BallSetRotation(w, o.rx, o.ry, o.rz, o.bias);
    return TeamSetLastTouchPlayer(w, c, p, o.type);
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
    h.spatial = c.ws->spatialAhead[p];
    h.prevPosition2D = h.spatial.position;
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
// Whether the ball runs into the designated player's feet unplayed: in a movement, nobody having
// touched it for 1.5 s (the opponents for 240 ms), within 0.6 m now and moving away (over 0.65 m
// in 200 ms); or in a trip with the ball, touched within the last 70% of 1.5 s, within 0.4 m. The
// ball must be below 1.6 m.
HD bool BallRunsIntoFeet(World &w, int p) {
    const Player &ps = w.match.players[p];
    const Humanoid &h = ps.base.humanoid;
    const Ball &ball = w.match.ball;
    const float now = (BallPredict(ball, 0).Get2D() - h.spatial.position).Length();
    const float soon = (BallPredict(ball, 200).Get2D() - (h.spatial.position + h.spatial.movement * 0.2f)).Length();
    const float own = GetLastTouchBias(w, p, 1500), theirs = TeamLastTouchBias(w, 1 - w.playerTeamID[p], 240);
    const int fn = h.anim.functionType;
    const bool running = own <= 0.01f && theirs <= 0.01f && fn == kFnMovement && now < 0.6f && soon > 0.65f && soon > now;
    const bool tripping = own <= 0.7f && ps.hasPossession && fn == kFnTrip && now < 0.4f;
    return p == w.match.designatedPossessionPlayer && (running || tripping) && BallPredict(ball, 0).v[2] < 1.6f;
}
// A controlled collision (the feet met the ball, or the body did for the designated player)
// outside a touch animation traps the ball, with a fifth of the spin.
HD bool ControlledCollision(World &w, const Ctx &c, int p, const Anim &a, const AnimDerived &d) {
    Humanoid &h = Hum(w, p);
    const AnimationState &cur = h.anim;
    const Vec3 incoming = w.match.ball.momentum;
    const Kick k = TrapKick(w, c, p, h, NextBodyAngle(h, a), OutgoingMovementOf(PList{h.anim.positions.e, h.anim.positions.count}));
    Vec3 momentum = k.momentum;
    if (cur.originatingCommand.modifier & kModifierKnockOn) momentum *= 1.35f;
    const float bumpy = 0.0f;
    momentum = momentum * (1.0f - bumpy) + incoming * bumpy;
    BallTouch(w, c, momentum);
    BallSetRotation(w, k.xRot, k.yRot, 0, 0.2f * (1.0f - bumpy));
    return TeamSetLastTouchPlayer(w, c, p, d.touchType);
}
// At the animation's touch frame the ball is touched when it lies within 0.4 m of the planned
// touch position (always for an animation that comes retaining it) and within 1 m of the
// animation's ball height; the bumpiness is how far off it lies, curved twice.
HD bool TouchAtTouchFrame(World &w, const Ctx &c, int p, const Anim &a, const AnimDerived &d) {
    const AnimationState &cur = Hum(w, p).anim;
    float animationBallHeight = 0;
    for (int i = 0; i < a.footballCount; i++) {
        const FootballKey &fk = c.t->football[a.footballFirst + i];
        if (fk.frame == cur.touchFrame) animationBallHeight = fk.position.v[2];
    }
    float reach = 0.4f;
    float off = (BallPredict(w.match.ball, 0) - (cur.touchPos + cur.positionOffset)).Length();
    if (a.incomingRetainState != kStrEmpty) {
        off = 0.0f;
        reach = 1.0f;
    }
    float bumpy = Clamp(off / reach - 0.001f, 0.0f, 1.0f);
    bumpy = Curve(bumpy, 1.0f);
    bumpy = Curve(bumpy, 0.5f);
    if (!(off < reach && fabsf(animationBallHeight - BallPredict(w.match.ball, 0).v[2]) < 1.0f)) return true;
    return AnimationTouch(w, c, p, a, d, bumpy);
}
// A retainer keeps the ball while its animation holds it (after the touch with an outgoing retain
// state, before it with an incoming one, or throughout with both): the ball sits 0.36 m below the
// holding body part, still, touched without a kick. Otherwise it lets go.
HD bool CarryRetainedBall(World &w, const Ctx &c, int p, const Anim &a, const AnimDerived &d) {
    Humanoid &h = Hum(w, p);
    const AnimationState &cur = h.anim;
    const bool holdsOut = d.outgoingRetainRawValue != kStrEmpty, holdsIn = d.incomingRetainRawValue != kStrEmpty;
    const bool holding = (cur.touchFrame <= cur.frameNum && holdsOut) || (cur.touchFrame > cur.frameNum && a.incomingRetainState != kStrEmpty) ||
                         (holdsIn && holdsOut);
    if (!holding) {
        w.match.ballRetainer = -1;
        return true;
    }
    int part = holdsOut ? d.outgoingRetainBodyPart : -1;
    if (part < 0 && holdsIn) part = d.incomingRetainBodyPart;
    if (part < 0) {
        Fatal("an animation that retains the ball names no body part");
        return false;
    }
    const Skeleton &sk = c.skeletons[p];
    Transform der[kHumanoidNodes];
    WorldTransforms(sk, h.nodes, der);
    const Transform &node = der[sk.nodeMap[part]];
    BallTouch(w, c, Vec3(0));
    // BallSetPosition predicts again from its own position before anything reads the
    // predictions, so this rotation's prediction is left out.
    BallSetRotation(w, 0, 0, 0, 1.0f, false);
    BallSetPosition(w, node.position + node.rotation * Vec3(0, 0, -0.36f));
    return TeamSetLastTouchPlayer(w, c, p, kTouchNonKicked);
}
// One frame's share of a smuggle spread over `span` frames, weighted by a raised cosine (0.9 to
// 1.1 times the mean): the movement it adds (per second) and the offset it accumulates.
HD void SmuggleStep(const Vec3 &total, int frame, int span, Vec3 &movement, Vec3 &offset) {
    float weight = libm::cosf((frame / (float)span - 0.5f) * PI * 2.0f) + 1.0f;
    weight = weight * 0.1f + 0.9f;
    movement = (total / (float)span) * weight * 100.0f;
    offset += movement / 100.0f;
}
// The rotation smuggle fades from its begin value over the first 16 frames (to the touch, when it
// comes sooner) and toward its end value over the animation (after the touch, for one with a
// touch).
HD float RotationSmuggleAt(const AnimationState &cur, int frames) {
    const int beginFrames = 16;
    const int cap = beginFrames < frames + 1 ? beginFrames : frames + 1;
    float beginBias = MinF(1.0f, (cur.frameNum + 1) / (float)cap), endBias = beginBias;
    if (cur.touchFrame != -1) {
        const int capTouch = beginFrames < cur.touchFrame + 1 ? beginFrames : cur.touchFrame + 1;
        beginBias = MinF(1.0f, (cur.frameNum + 1) / (float)capTouch);
        endBias = cur.frameNum > cur.touchFrame ? (cur.frameNum - cur.touchFrame) / (float)(frames - cur.touchFrame) : 0.0f;
    }
    return cur.rotationSmuggleBegin.value() * (1.0f - beginBias) + cur.rotationSmuggleEnd.value() * endBias;
}
// A goalkeeper holding the ball in open play steps back inside its box: toward 20.05 m across
// (30% of the excess a tick), 16.4 m out (30%) and 0.1 m in from the goal line (40%), at most
// half a metre of excess each.
HD void KeepKeeperInBox(World &w, int p) {
    const int side = TeamDynamicSide(w, w.playerTeamID[p]);
    const Vec3 ball = BallPredict(w.match.ball, 0);
    if (ball.v[1] > 20.05f) OffsetPosition(w, p, Vec3(0, Clamp(20.05f - ball.v[1], -0.5f, 0.5f), 0) * 0.3f);
    if (ball.v[1] < -20.05f) OffsetPosition(w, p, Vec3(0, Clamp(-20.05f - ball.v[1], -0.5f, 0.5f), 0) * 0.3f);
    if (ball.v[0] * -side > -kPitchHalfLength + 16.4f)
        OffsetPosition(w, p, Vec3(Clamp((-kPitchHalfLength + 16.4f) - ball.v[0] * -side, -0.5f, 0.5f), 0, 0) * -side * 0.3f);
    if (ball.v[0] * -side < -kPitchHalfLength + 0.1f)
        OffsetPosition(w, p, Vec3(Clamp((-kPitchHalfLength + 0.1f) - ball.v[0] * -side, -0.5f, 0.5f), 0, 0) * -side * 0.4f);
}
// The pose the frame applies: the planned position (while the plan lasts) plus the smuggle
// offsets, the start angle turned by the rotation smuggle, and the pose offsets.
HD void FillApplyBuffer(Humanoid &h) {
    const AnimationState &cur = h.anim;
    h.applyBuf.frameNum = cur.frameNum;
    if ((uint32_t)cur.positions.count > (uint32_t)cur.frameNum) {
        h.applyBuf.position =
            h.startPos + cur.positions[cur.frameNum] + cur.actionSmuggleOffset + cur.actionSmuggleSustainOffset + cur.movementSmuggleOffset;
        h.applyBuf.orientation.set(h.startAngle.value() + cur.rotationSmuggleOffset.value());
        h.applyBuf.noPos = true;
    } else {
        h.applyBuf.position = h.startPos + cur.actionSmuggleOffset + cur.actionSmuggleSustainOffset + cur.movementSmuggleOffset;
        h.applyBuf.orientation = h.startAngle;
        h.applyBuf.noPos = false;
    }
    for (int i = 0; i < kBodyParts; i++) h.applyBuf.offsets[i] = h.offsets[i];
}
// The rest of a humanoid's tick: controlled collisions, the touch, the retained ball, the
// smuggles of the frame, the keeper's box and the apply buffer.
HDN bool HumanoidProcessEnd(World &w, const Ctx &c, int p) {
    Player &ps = w.match.players[p];
    Humanoid &h = ps.base.humanoid;
    AnimationState &cur = h.anim;
    h.requeueDelayFrames = h.requeueDelayFrames - 1 > 0 ? h.requeueDelayFrames - 1 : 0;
    h.interruptAnim = kIntNone;
    const Anim &a = c.A(cur.anim);
    const AnimDerived &d = c.D(cur.anim);
    if (BallRunsIntoFeet(w, p)) ps.triggerControlledBallCollision = true;
    const bool controlled = ps.triggerControlledBallCollision;
    if (controlled) ps.triggerControlledBallCollision = false;
    if (controlled && cur.touchFrame == -1 && !ControlledCollision(w, c, p, a, d)) return false;
    if (cur.touchFrame == cur.frameNum && !TouchAtTouchFrame(w, c, p, a, d)) return false;
    if (w.match.ballRetainer == p && !CarryRetainedBall(w, c, p, a, d)) return false;
    const int frames = a.frameCount - 1;
    if (cur.touchFrame != -1 && cur.frameNum <= cur.touchFrame)
        SmuggleStep(cur.actionSmuggle, cur.frameNum, cur.touchFrame + 1, h.spatial.actionSmuggleMovement, cur.actionSmuggleOffset);
    else
        h.spatial.actionSmuggleMovement = Vec3(0);
    if (cur.touchFrame == -1 && cur.frameNum <= frames)
        SmuggleStep(cur.movementSmuggle, cur.frameNum, frames + 1, h.spatial.movementSmuggleMovement, cur.movementSmuggleOffset);
    else
        h.spatial.movementSmuggleMovement = Vec3(0);
    cur.rotationSmuggleOffset.set(RotationSmuggleAt(cur, frames));
    if (w.match.ballRetainer == p && Formation(w, c, p).role == kRoleGoalkeeper && !w.match.inSetPiece && w.match.inPlay)
        KeepKeeperInBox(w, p);
    FillApplyBuffer(h);
    return true;
}

}  // namespace eng
