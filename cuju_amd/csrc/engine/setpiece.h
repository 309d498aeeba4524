// SPDX-License-Identifier: Apache-2.0
// Restates game logic of cuju (Copyright 2026 The cuju Authors), a reimplementation of Google
// Research Football (Copyright 2019 Google LLC); see NOTICE.
// The reset of the world for a set piece, the placement of the players for it and sending-offs.
// The placement keeps every conversion between double and float of GRF's arithmetic.
// Semantics: include/cuju/simulation/reset.h:15-721.
#pragma once

#include "team.h"

namespace eng {

constexpr int kFootRight = 1;

HDN bool LeftTeamOwnsBall(const World &w) {
    const Scenario &s = w.scenario;
    float l = 1000000, r = 1000000;
    for (int i = 0; i < s.leftTeamSize; i++) l = MinF(l, (s.leftTeam[i].startPosition - s.ballPosition).Length());
    for (int i = 0; i < s.rightTeamSize; i++) r = MinF(r, (s.rightTeam[i].startPosition - s.ballPosition).Length());
    return l < r;
}
// Humanoid index: players first, then the officials.
HD Humanoid &AnyHumanoid(World &w, int hi) {
    const int pc = w.match.playerCount;
    return hi < pc ? w.match.players[hi].base.humanoid : w.match.officials[hi - pc].humanoid;
}

// Places a humanoid at `pos` facing `focus`, idling at a random frame of the idle animation.
HDN bool HumanoidResetPosition(World &w, const Ctx &c, int hi, const Vec3 &pos, const Vec3 &focus) {
    Humanoid &h = AnyHumanoid(w, hi);
    SpatialState &s = h.spatial;
    h.startPos = pos;
    h.startAngle.set(FixAngle((focus - pos).Normalized(Vec3(0, -1, 0)).Angle2D()));
    h.nextStartPos = h.startPos;
    h.nextStartAngle = h.startAngle;
    h.prevPosition2D = h.startPos;
    s.position = h.startPos;
    s.angle = h.startAngle;
    s.directionVec = Vec3(0, -1, 0).Rotated2D(h.startAngle.value());
    s.floatVelocity = 0;
    s.actualMovement = s.physicsMovement = s.animationMovement = s.movement = Vec3(0);
    s.actionSmuggleMovement = s.movementSmuggleMovement = s.positionOffsetMovement = Vec3(0);
    s.relBodyAngleNonQuantized.set(0);
    s.velocityCat = kVelIdle;
    s.relBodyDirectionVec = Vec3(0, -1, 0);
    s.relBodyAngle.set(0);
    s.bodyDirectionVec = Vec3(0, -1, 0);
    s.bodyAngle.set(0);
    s.foot = kFootRight;
    Selector sel(w, c, hi);
    const int idle = sel.GetIdleMovementAnimationID();
    const Anim &ia = c.A(idle);
    AnimationState &cur = h.anim;
    cur.id = idle;
    cur.anim = idle;
    if (ia.posCount > cur.positions.kCapacity) Unsupported("a state list outgrows its capacity");
    const int copied = ia.posCount < cur.positions.kCapacity ? ia.posCount : cur.positions.kCapacity;
    GroupCopy<4>(cur.positions.e, c.t->positions + ia.posFirst, copied);
    cur.positions.count = copied;
    // GRF: the frame draws below the effective frame count, one less than the frame count.
    cur.frameNum = TruncToInt32(RandomInRange(w, 0, (float)(ia.frameCount - 1 - 1)));
    cur.touchFrame = -1;
    cur.originatingInterrupt = kIntNone;
    cur.actionSmuggle = cur.actionSmuggleOffset = cur.actionSmuggleSustain = cur.actionSmuggleSustainOffset = Vec3(0);
    cur.movementSmuggle = cur.movementSmuggleOffset = Vec3(0);
    cur.rotationSmuggleBegin.set(0);
    cur.rotationSmuggleEnd.set(0);
    cur.rotationSmuggleOffset.set(0);
    cur.functionType = kFnMovement;
    cur.incomingMovement = cur.outgoingMovement = cur.positionOffset = Vec3(0);
    h.prevAnimFrameNum = 0;
    h.prevAnimFunctionType = kFnMovement;
    h.nodes[0].position = h.startPos;
    h.applyBuf.anim = cur.anim;
    h.applyBuf.smooth = false;
    h.applyBuf.smoothFactor = 0.0f;
    h.applyBuf.position = h.startPos;
    h.applyBuf.orientation = h.startAngle;
    // The offsets of the apply buffer keep their values.
    h.interruptAnim = kIntNone;
    h.tripType = 0;
    h.decayingPositionOffset = Vec3(0);
    h.decayingDifficultyFactor = 0.0f;
    h.movementHistory.count = 0;
    h.requeueDelayFrames = 0;
    h.tripDirection = Vec3(0);
    const Skeleton &sk = c.skeletons[hi];
    for (int bp = 0; bp < kBodyParts - 1; bp++) h.nodes[sk.nodeMap[bp]].rotation = Quat();
    return true;
}

// The throw-in taker's idle animation that holds the ball at the right elbow.
HDN bool HumanoidSelectRetainAnimation(World &w, const Ctx &c, int hi) {
    Humanoid &h = AnyHumanoid(w, hi);
    Selector sel(w, c, hi);
    CrudeQuery q;
    q.byFunctionType = true;
    q.functionType = kFnMovement;
    q.byIncomingVelocity = true;
    q.incomingVelocity = kVelIdle;
    q.byOutgoingVelocity = true;
    q.outgoingVelocity = kVelIdle;
    q.incomingRetainState = kStrRightElbow;
    AList l{c.ws->lists[0], 0};
    CrudeSelection(c, q, l);
    if (l.empty()) return Fail("no animation retains the ball for the restart");
    sel.SetMovementSimilarityPredicate(Vec3(0, -1, 0), kVelIdle);
    sel.Sort(l, [&](int i) { return sel.MovementSimilarityKey(i); });
    h.startAngle.set(FixAngle((Vec3(0) - h.startPos).Angle2D()));
    AnimationState &cur = h.anim;
    cur.positions.count = 0;
    cur.anim = l[0];
    cur.id = l[0];
    cur.frameNum = 0;
    cur.touchFrame = -1;
    cur.actionSmuggle = cur.actionSmuggleOffset = cur.actionSmuggleSustain = cur.actionSmuggleSustainOffset = Vec3(0);
    cur.movementSmuggle = cur.movementSmuggleOffset = Vec3(0);
    cur.rotationSmuggleBegin.set(0);
    cur.rotationSmuggleEnd.set(0);
    cur.rotationSmuggleOffset.set(0);
    cur.functionType = kFnMovement;
    h.applyBuf.anim = cur.anim;
    h.applyBuf.smooth = false;
    h.applyBuf.position = h.startPos;
    h.applyBuf.orientation = h.startAngle;
    w.match.ballRetainer = hi;
    return true;
}

HDN bool PlayerBaseResetSituation(World &w, const Ctx &c, int hi, const Vec3 &focus) {
    const int pc = w.match.playerCount;
    PersonBase &b = hi < pc ? w.match.players[hi].base : w.match.officials[hi - pc];
    b.positionHistoryPerSecond.count = 0;
    b.lastTouchTimeMs = 0;
    b.lastTouchType = kTouchNone;
    if (b.isActive) {
        b.humanoid.mentalImageTime = 0;
        Vec3 pos = b.humanoid.spatial.position;
        if (!HumanoidResetPosition(w, c, hi, pos, focus)) return false;
    }
    if (hi < pc) {
        if (ExternalControllerActive(w, hi)) {
            HumanControllerReset(w, b.externalController);
        } else {
            w.match.players[hi].controller.lastDesiredDirection = Vec3(0);
            w.match.players[hi].controller.lastDesiredVelocity = 0;
        }
    }
    return true;
}
HDN bool PlayerResetSituation(World &w, const Ctx &c, int p, const Vec3 &focus) {
    if (!PlayerBaseResetSituation(w, c, p, focus)) return false;
    Player &ps = w.match.players[p];
    ps.hasPossession = ps.hasBestPossession = ps.hasUniquePossession = false;
    ps.possessionDurationMs = 0;
    ps.timeToBallMs = 1000;
    ps.timeToBallOptimisticMs = 1000;
    ps.desiredTimeToBallMs = 0;
    ps.manMarking = -1;
    ps.triggerControlledBallCollision = false;
    ps.tactical.forwardSpaceRating = 0;
    ps.tactical.toGoalSpaceRating = 0;
    ps.tactical.spaceRating = 0;
    return true;
}
HD void TeamAIReset(TeamAI &ai) {
    ai.taker = -1;
    ai.setPieceType = kModeNormal;
    ai.offsideTrapX = 0;
    ai.endApplyAttackingRunMs = 0;
    ai.attackingRunPlayer = -1;
    ai.endApplyTeamPressureMs = 0;
    ai.teamPressurePlayer = -1;
    ai.endApplyKeeperRushMs = 0;
    ai.teamHasPossession = ai.teamHasUniquePossession = false;
    ai.oppTeamHasPossession = ai.oppTeamHasUniquePossession = false;
    ai.teamHasBestPossession = false;
    ai.teamPossessionAmount = 1.0f;
    ai.fadingTeamPossessionAmount = 1.0f;
    ai.timeNeededToGetToBall = 100;
    ai.oppTimeNeededToGetToBall = 100;
}
HDN bool TeamResetSituation(World &w, const Ctx &c, int teamID, const Vec3 &focus) {
    Team &t = TeamByID(w, teamID);
    t.timeToBallMs = 100;
    t.hasPossession = false;
    t.teamPossessionAmount = 1.0f;
    t.fadingTeamPossessionAmount = 1.0f;
    t.lastTouchPlayer = -1;
    PlayerList ps = TeamAllPlayers(w, teamID);
    if (ps.empty()) {
        Fatal("a team has no players");
        return false;
    }
    t.designatedTeamPossessionPlayer = ps[0];
    for (int i = 0; i < ps.count; i++)
        if (w.match.players[ps[i]].base.isActive && !PlayerResetSituation(w, c, ps[i], focus)) return false;
    TeamAIReset(t.ai);
    return true;
}
HD void BallResetSituation(Ball &b, const Vec3 &focus) {
    // Materializing keeps the frame of the stored predictions.
    BallMaterialize(b);
    b.momentum = Vec3(0);
    b.rotationPerMs = Quat();
    for (int i = 0; i < kBallPredictionSpanMs / 10; i++) b.predictions[i] = focus + Vec3(0, 0, 0.11f);
    b.memoValid = false;
    b.orientationPrediction = Quat();
    b.positionHistory.count = 0;
    b.positionBuffer = focus + Vec3(0, 0, 0.11f);
    b.validPredictions = 0;
    b.orientationBuffer = Quat();
    b.touchesNet = false;
}
HDN bool MatchResetSituation(World &w, const Ctx &c, const Vec3 &focus) {
    MatchState &m = w.match;
    m.cameraPosition.count = 0;
    m.ballRetainer = -1;
    m.ballIsInGoal = false;
    m.goalScored = false;
    m.mentalImages.count = 0;
    for (int i = 0; i < 4; i++) m.lastTouchTeamIDs[i] = -1;
    m.lastTouchTeamID = -1;
    m.lastGoalScorer = -1;
    m.bestPossessionTeam = -1;
    m.possessionSideHistory.count = 0;
    m.lastBodyBallCollisionTimeMs = 0;
    BallResetSituation(m.ball, focus);
    const int first = w.FirstTeamID();
    if (!TeamResetSituation(w, c, first, focus)) return false;
    if (!TeamResetSituation(w, c, 1 - first, focus)) return false;
    // The referee is the first official.
    return PlayerBaseResetSituation(w, c, m.playerCount + 0, focus);
}

// Places a team for a set piece and names its taker.
HDN bool TeamAIPrepareSetPiece(World &w, const Ctx &c, int teamID, int setPiece, int otherTeamID, int kickoffTeamID,
                               int takerTeamID) {
    MatchState &m = w.match;
    Team &team = TeamByID(w, teamID);
    TeamAI &ai = team.ai;
    const int side = TeamDynamicSide(w, teamID);
    auto flatBall = [&]() { return BallPredict(m.ball, 0).Get2D(); };
    auto reset = [&](int p, const Vec3 &pos, const Vec3 &focus) { return HumanoidResetPosition(w, c, p, pos, focus); };
    auto F = [](double v) { return (float)v; };
    ai.setPieceType = setPiece;
    if (setPiece == kModeNormal) return true;
    PlayerList ps = TeamActivePlayers(w, teamID);
    for (int i = 0; i < ps.count;) {
        Vec3 focus = flatBall();
        if (Formation(w, c, ps[i]).role == kRoleGoalkeeper) {
            if (setPiece == kModeKickOff) focus.v[0] = focus.v[1] = 0;
            if (!reset(ps[i], Vec3((float)((double)(kPitchHalfLength * side) * 0.98), 0, 0), focus)) return false;
            for (int j = i; j + 1 < ps.count; j++) ps[j] = ps[j + 1];
            ps.count--;
        } else {
            i++;
        }
    }
    const bool taker = takerTeamID == teamID;
    // GRF passes a double here, which rounds to float.
    team.fadingTeamPossessionAmount = taker ? 1.5f : 0.5f;
    const double ds = side, hl = kPitchHalfLength, hw = kPitchHalfWidth;
    switch (setPiece) {
        case kModeKickOff:
            for (int i = 0; i < ps.count; i++) {
                const Vec3 &fp = Formation(w, c, ps[i]).position;
                Vec3 bp = fp * Vec3(F((double)(-side * kPitchHalfLength) * 0.6), F((double)(-side * kPitchHalfWidth) * 0.6), 0);
                bp.v[1] += RandomInRange(w, -2.0f, 2.0f);
                bp.v[0] = F(bp.v[0] * 0.5);
                bp.v[0] = F(bp.v[0] + (hl * 0.2) * ds);
                if ((double)(bp.v[0] * side) < 0.5) bp.v[0] = F(0.5 * ds);
                if ((double)bp.Length() < 9.4) {
                    bp.Normalize(Vec3(side, 0, 0));
                    bp *= 9.4f;
                }
                if (!reset(ps[i], bp, flatBall())) return false;
                // GRF re-places the two players nearest the centre after every placement.
                if (taker) {
                    PlayerList r = GetClosestPlayers(w, c, teamID, Vec3(0), false, 2);
                    for (int k = 0; k < r.count; k++)
                        if (!reset(r[k], Vec3(0, F((double)k * 1.4 * ds), 0), flatBall())) return false;
                }
            }
            break;
        case kModeGoalKick:
            for (int i = 0; i < ps.count; i++) {
                float back, front;
                if (taker) {
                    back = F((double)(side * kPitchHalfLength) * 0.5);
                    front = F((double)(-side * kPitchHalfLength) * 0.2);
                } else {
                    back = F((double)(side * kPitchHalfLength) * 0.4);
                    front = F((double)(-side * kPitchHalfLength) * 0.1);
                }
                Vec3 bp = GetAdaptedFormationPosition(w, c, ps[i], back, front, F(-hw * 0.7), F(hw * 0.7), 0, 0, 0, 0, Vec3(0), 0, 0,
                                                      0, false);
                if (!reset(ps[i], bp, flatBall())) return false;
            }
            break;
        case kModeCorner:
            for (int i = 0; i < ps.count; i++) {
                float back, front, xf, xfs, yf, yfs, mf, mfs;
                Vec3 ball = flatBall();
                if (taker) {
                    back = F((double)(-side * kPitchHalfLength) * 0.2);
                    front = F((double)(-side * kPitchHalfLength) * 0.96);
                    xf = F(front * 0.85);
                    xfs = 0.7f;
                    yf = ball.v[1] * 0.1f;
                    yfs = 0.7f;
                    mf = 0.9f;
                    mfs = 0.5f;
                } else {
                    back = F((double)(side * kPitchHalfLength) * 0.98);
                    front = F((double)(side * kPitchHalfLength) * 0.5);
                    xf = F(back * 0.94);
                    xfs = 0.8f;
                    yf = ball.v[1] * 0.1f;
                    yfs = 0.9f;
                    mf = 0.1f;
                    mfs = 0.7f;
                }
                Vec3 bp = GetAdaptedFormationPosition(w, c, ps[i], back, front, F(-hw * 0.6), F(hw * 0.6), xf, xfs, yf, yfs,
                                                      Vec3(ball.v[0] * 0.95f, ball.v[1] * 0.1f, 0), 0.9f, mf, mfs, false);
                if (!reset(ps[i], bp, flatBall())) return false;
            }
            break;
        case kModeThrowIn:
            for (int i = 0; i < ps.count; i++) {
                float back, front, xf, xfs, yf, yfs;
                Vec3 ball = flatBall();
                const float L = kPitchHalfLength;
                back = Clamp(ball.v[0] + 30 * side, -L, L);
                if (taker) {
                    front = Clamp(ball.v[0] + 20 * -side, -L, L);
                    xf = Clamp(ball.v[0] + 4 * -side, -L, L);
                    xfs = F(0.4);
                    yf = F(ball.v[1] * 0.996);
                    yfs = F(0.6);
                } else {
                    front = Clamp(ball.v[0] + 15 * -side, -L, L);
                    xf = Clamp(ball.v[0] + 16 * side, -L, L);
                    xfs = F(0.2);
                    yf = F(ball.v[1] * 0.95);
                    yfs = F(0.5);
                }
                float low = -kPitchHalfWidth * 0.75f + ball.v[1] * 0.25f;
                float high = kPitchHalfWidth * 0.75f + ball.v[1] * 0.25f;
                Vec3 bp = GetAdaptedFormationPosition(w, c, ps[i], back, front, low, high, xf, xfs, yf, yfs, ball, F(0.7), 0, 0, false);
                if (!reset(ps[i], bp, flatBall())) return false;
            }
            break;
        case kModeFreeKick: {
            for (int i = 0; i < ps.count; i++) {
                float back, front, xf, xfs, yf, yfs;
                Vec3 ball = flatBall();
                const float L = kPitchHalfLength;
                const float shw = side * kPitchHalfLength;
                float xo = F((double)Clamp((ball.v[0] * -side) / L, F(-1.0), F(1.0)) * 0.5 + 0.5);
                if (taker) {
                    back = Clamp(F((double)shw * (0.7 - (double)xo * 0.7)), -L, L);
                    front = Clamp(F((double)shw * (-0.3 - (double)xo * 0.7)), -L, L);
                    xf = Clamp(ball.v[0] + 10 * -side, -L, L);
                    xfs = F(0.5 + (double)xo * 0.2);
                    yf = F(ball.v[1] * 0.4);
                    yfs = F(0.6 + (double)xo * 0.2);
                } else {
                    back = Clamp(F((double)shw * (1.0 - (double)xo * 0.6)), -L, L);
                    front = Clamp(F((double)shw * (0.5 - (double)xo * 0.8)), -L, L);
                    xf = Clamp(ball.v[0] + 20 * side, -L, L);
                    xfs = F(0.6 - (double)xo * 0.4);
                    yf = F(ball.v[1] * 0.2);
                    yfs = F(0.8 - (double)xo * 0.4);
                }
                Vec3 bp = GetAdaptedFormationPosition(w, c, ps[i], back, front, F(-hw * 0.7), F(hw * 0.7), xf, xfs, yf, yfs, ball, F(0.4),
                                                      0, 0, false);
                // The wall keeps 9.15 m.
                if (!taker && (double)(bp - flatBall()).Length() < 9.15) bp = flatBall() + (bp - flatBall()).Normalized() * 9.15f;
                if (!reset(ps[i], bp, flatBall())) return false;
            }
            if (!taker && (double)(flatBall() - Vec3(side * kPitchHalfLength, 0, 0)).Length() < 40.0) {
                PlayerList r = GetClosestPlayers(w, c, teamID, flatBall(), false, 3);
                for (int k = 0; k < r.count; k++) {
                    Vec3 toGoal = (Vec3(side * kPitchHalfLength, 0, 0) - flatBall()).Normalized(0);
                    toGoal += Vec3(0, F(1.0 - (double)k), 0) * F(0.07);
                    toGoal.Normalize();
                    if (!reset(r[k], flatBall() + toGoal * 9.15f, flatBall())) return false;
                }
            }
            break;
        }
        case kModePenalty:
            for (int i = 0; i < ps.count; i++) {
                float back, front, xf, xfs, yf, yfs;
                Vec3 ball = flatBall();
                const float L = kPitchHalfLength;
                if (taker) {
                    back = Clamp(ball.v[0] + 50 * side, -L, L);
                    front = Clamp(ball.v[0] + 10 * -side, -L, L);
                    xf = ball.v[0];
                    xfs = F(0.6);
                    yf = F(0.0);
                    yfs = F(0.8);
                } else {
                    back = Clamp(ball.v[0] + 11 * side, -L, L);
                    front = Clamp(ball.v[0] + 20 * -side, -L, L);
                    xf = ball.v[0];
                    xfs = F(1.0);
                    yf = F(0.0);
                    yfs = F(1.0);
                }
                Vec3 bp = GetAdaptedFormationPosition(w, c, ps[i], back, front, F(-hw * 0.8), F(hw * 0.8), xf, xfs, yf, yfs, Vec3(0), 0, 0,
                                                      0, false);
                int ps_ = (BallPredict(m.ball, 0).v[0] < 0) ? -1 : 1;
                if ((double)(bp.v[0] * ps_) > hl - 16.5 - 0.5) bp.v[0] = F((hl - 16.5 - 0.5) * ps_);
                if ((double)(bp - flatBall()).Length() < 9.15 + 0.5) bp = flatBall() + (bp - flatBall()).Normalized() * F(9.15 + 0.5);
                if (!reset(ps[i], bp, flatBall())) return false;
            }
            break;
        default:
            for (int i = 0; i < ps.count; i++) {
                Vec3 bp = Formation(w, c, ps[i]).position *
                          Vec3(F((double)(-side * kPitchHalfLength) * 0.7), F((double)(-side * kPitchHalfWidth) * 0.7), 0);
                if (!reset(ps[i], bp, flatBall())) return false;
            }
            break;
    }
    if (setPiece == kModeKickOff) {
        PlayerList formationPlayers = TeamAllPlayers(w, teamID);
        PlayerList toPlace = TeamAllPlayers(w, teamID);
        // GRF: after the start, a kickoff to the team that did not own the ball at the start swaps
        // the start positions of the two teams when they are of equal size.
        if (m.matchTimeMs > 0 && TeamAllPlayers(w, otherTeamID).size() == formationPlayers.size() &&
            (LeftTeamOwnsBall(w) ^ (kickoffTeamID == 0)))
            formationPlayers = TeamAllPlayers(w, otherTeamID);
        for (int i = 0; i < formationPlayers.count; i++) {
            if (!m.players[toPlace[i]].base.isActive) continue;
            Vec3 bp = Formation(w, c, formationPlayers[i]).startPosition * Vec3(-side * kPitchHalfLength, -side * kPitchHalfWidth, 0);
            if (!reset(toPlace[i], bp, flatBall())) return false;
        }
    }
    if (taker) {
        Vec3 ball = flatBall();
        PlayerList closest = GetClosestPlayers(w, c, teamID, flatBall(), false, 2);
        if (closest.empty()) return Fail("the set piece has no taker");
        ai.taker = closest[0];
        if (setPiece == kModeKickOff) {
            // The kickoff taker keeps its formation position.
        } else if (setPiece == kModeThrowIn) {
            if (!reset(closest[0], ball + flatBall().Normalized(Vec3(0, -side, 0)) * 0.3f, ball)) return false;
        } else if (setPiece == kModeFreeKick) {
            if (!reset(ai.taker, ball + Vec3(side, 0, 0) * 2.3f, ball)) return false;
        } else {
            if (!reset(ai.taker, ball + flatBall().Normalized(Vec3(0, -side, 0)) * 2.3f, ball)) return false;
        }
        if (setPiece == kModeThrowIn && !HumanoidSelectRetainAnimation(w, c, ai.taker)) return false;
        if (setPiece == kModePenalty && !reset(ai.taker, ball + Vec3(side, 0, 0) * 3.0f, ball)) return false;
    } else {
        ai.taker = -1;
    }
    return true;
}

HDN bool PlayerSendOff(World &w, const Ctx &c, int p) {
    MatchState &m = w.match;
    Player &ps = m.players[p];
    const int t = w.playerTeamID[p];
    RandomInRange(w, 0, 3);  // GRF: the referee's message draws once.
    auto here = [&]() { return ps.base.humanoid.spatial.position; };
    if (!PlayerResetSituation(w, c, p, here())) return false;
    if (ps.base.externalController >= 0) {
        Team &team = TeamByID(w, t);
        for (int g = 0; g < team.gamers.count; g++) {
            if (team.gamers[g].selectedPlayer != p) continue;
            int other = GetClosestPlayer(w, c, t, here(), true, p, true);
            team.mainSelectedPlayer = other;
            HumanGamerSetSelectedPlayer(w, GlobalGamerIndex(w, t, g), other);
        }
    }
    // GRF: the deactivation resets the player a second time.
    if (!PlayerResetSituation(w, c, p, here())) return false;
    ps.base.isActive = false;
    ps.base.externalController = -1;
    TeamByID(w, t).designatedTeamPossessionPlayer = GetClosestPlayer(w, c, t, BallPredict(m.ball, 0).Get2D(), false);
    if (Formation(w, c, p).role == kRoleGoalkeeper) {
        int first = -1;
        for (int q = 0; q < m.playerCount && first < 0; q++)
            if (w.playerTeamID[q] == t && m.players[q].base.isActive) first = q;
        if (first < 0) {
            Fatal("the sending-off leaves no active player");
            return false;
        }
        w.formationOverride[first] = (int8_t)(1 + FormationSource(w, p));
    }
    return true;
}

HDN bool RefereePrepareSetPiece(World &w, const Ctx &c, int setPiece) {
    Referee &ref = w.match.referee;
    RefereeBuffer &b = ref.buffer;
    if (setPiece == kModeFreeKick) {
        b.restartPos.v[0] = Clamp(b.restartPos.v[0], (float)(-0.95 * kPitchHalfLength), (float)(0.95 * kPitchHalfLength));
        b.restartPos.v[1] = Clamp(b.restartPos.v[1], (float)(-0.95 * kPitchHalfWidth), (float)(0.95 * kPitchHalfWidth));
    }
    if (!MatchResetSituation(w, c, w.scenario.reverseTeamProcessing ? -b.restartPos : b.restartPos)) return false;
    const int first = w.FirstTeamID(), second = 1 - first;
    // The buffer stores the kickoff team as its slot.
    const int spTeam = b.setPieceTeam == 0 ? first : second;
    if (!TeamAIPrepareSetPiece(w, c, first, setPiece, second, spTeam, b.teamID)) return false;
    if (!TeamAIPrepareSetPiece(w, c, second, setPiece, first, spTeam, b.teamID)) return false;
    b.taker = TeamByID(w, b.teamID).ai.taker;
    ref.offsidePlayers.count = 0;
    return true;
}

}  // namespace eng
