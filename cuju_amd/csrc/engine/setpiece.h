// SPDX-License-Identifier: Apache-2.0
// Restates game logic of cuju (Copyright 2026 The cuju Authors), a reimplementation of Google
// Research Football (Copyright 2019 Google LLC); see NOTICE.
// Restarts: the match brought back to a set piece, each team placed for it, and a player sent off.
// Semantics: include/cuju/simulation/reset.h:15-721. Every conversion between double and float of
// GRF's placement arithmetic is kept as GRF performs it. The organisation is this engine's own: a
// stance value for a humanoid standing still, a placement rule per restart that one loop applies,
// and the restarts of persons, teams, ball and match as value resets.
#pragma once

#include "team.h"

namespace eng {

constexpr int kFootRight = 1;

// ---- a humanoid standing still ---------------------------------------------------------------------

// A place and the angle that faces a point from it (GRF's angle of the look direction, the -y axis
// at angle 0), with the direction vector of that angle.
struct Stance {
    Vec3 at;
    Radian angle;
    Vec3 facing;
};
HD Stance StanceFacing(const Vec3 &at, const Vec3 &focus) {
    Stance s{};
    s.at = at;
    s.angle.set(FixAngle((focus - at).Normalized(Vec3(0, -1, 0)).Angle2D()));
    s.facing = Vec3(0, -1, 0).Rotated2D(s.angle.value());
    return s;
}

// The spatial state of a humanoid idling in a stance: no movement of any kind, the body straight
// ahead, the right foot leading. The non-quantized relative body direction keeps its value.
HD void StandStill(SpatialState &s, const Stance &st) {
    const Vec3 ahead(0, -1, 0);
    s.position = st.at;
    s.angle = st.angle;
    s.directionVec = st.facing;
    s.velocityCat = kVelIdle;
    s.floatVelocity = 0;
    Vec3 *const moves[] = {&s.actualMovement,        &s.physicsMovement,         &s.animationMovement,
                           &s.movement,              &s.actionSmuggleMovement,   &s.movementSmuggleMovement,
                           &s.positionOffsetMovement};
    for (Vec3 *m : moves) *m = Vec3(0);
    s.bodyAngle.set(0);
    s.relBodyAngle.set(0);
    s.relBodyAngleNonQuantized.set(0);
    s.bodyDirectionVec = ahead;
    s.relBodyDirectionVec = ahead;
    s.foot = kFootRight;
}

// An animation starting afresh carries no smuggled action, movement or rotation.
HD void DropSmuggles(AnimationState &a) {
    Vec3 *const offsets[] = {&a.actionSmuggle,    &a.actionSmuggleOffset, &a.actionSmuggleSustain,
                             &a.actionSmuggleSustainOffset, &a.movementSmuggle, &a.movementSmuggleOffset};
    for (Vec3 *v : offsets) *v = Vec3(0);
    a.rotationSmuggleBegin.set(0);
    a.rotationSmuggleEnd.set(0);
    a.rotationSmuggleOffset.set(0);
}

// Humanoid index: the players first, then the officials.
HD Humanoid &HumanoidAt(World &w, int hi) {
    const int players = w.match.playerCount;
    return hi < players ? w.match.players[hi].base.humanoid : w.match.officials[hi - players].humanoid;
}

// Puts a humanoid at `pos` facing `focus`, idling at a random frame of the idle animation it
// selects from there: the stance first, which the selection reads, then the animation, the apply
// buffer and the nodes.
HDN bool PlaceHumanoid(World &w, const Ctx &c, int hi, const Vec3 &pos, const Vec3 &focus) {
    Humanoid &h = HumanoidAt(w, hi);
    const Stance st = StanceFacing(pos, focus);
    h.startPos = h.nextStartPos = h.prevPosition2D = st.at;
    h.startAngle = h.nextStartAngle = st.angle;
    StandStill(h.spatial, st);

    Selector sel(w, c, hi);
    const int idle = sel.IdleMovementAnimation();
    const Anim &ia = c.A(idle);
    AnimationState &a = h.anim;
    if (ia.posCount > a.positions.kCapacity) Unsupported("a state list outgrows its capacity");
    const int planned = ia.posCount < a.positions.kCapacity ? ia.posCount : a.positions.kCapacity;
    GroupCopy<4>(a.positions.e, c.t->positions + ia.posFirst, planned);
    a.positions.count = planned;
    a.anim = a.id = idle;
    // GRF: the frame draws below the effective frame count, one less than the frame count.
    a.frameNum = TruncToInt32(RandomInRange(w, 0, (float)(ia.frameCount - 1 - 1)));
    a.touchFrame = -1;
    a.functionType = kFnMovement;
    a.originatingInterrupt = kIntNone;
    DropSmuggles(a);
    a.incomingMovement = a.outgoingMovement = a.positionOffset = Vec3(0);

    h.prevAnimFrameNum = 0;
    h.prevAnimFunctionType = kFnMovement;
    h.interruptAnim = kIntNone;
    h.requeueDelayFrames = 0;
    h.tripType = 0;
    h.tripDirection = h.decayingPositionOffset = Vec3(0);
    h.decayingDifficultyFactor = 0.0f;
    h.movementHistory.count = 0;
    // The apply buffer restarts without smoothing; its body-part offsets keep their values.
    AnimApplyBuffer &buf = h.applyBuf;
    buf.anim = a.anim;
    buf.smooth = false;
    buf.smoothFactor = 0.0f;
    buf.position = st.at;
    buf.orientation = st.angle;
    h.nodes[0].position = st.at;
    const Skeleton &sk = c.skeletons[hi];
    for (int bp = 0; bp + 1 < kBodyParts; bp++) h.nodes[sk.nodeMap[bp]].rotation = Quat();
    return true;
}

// The throw-in taker holds the ball: the idle animation whose start retains it at the right elbow
// and moves most like standing still, facing the centre spot.
HDN bool HoldBallForThrowIn(World &w, const Ctx &c, int hi) {
    CrudeQuery hold;
    hold.byFunctionType = true;
    hold.functionType = kFnMovement;
    hold.byIncomingVelocity = hold.byOutgoingVelocity = true;
    hold.incomingVelocity = hold.outgoingVelocity = kVelIdle;
    hold.incomingRetainState = kStrRightElbow;
    AList found{c.ws->lists[0], 0};
    FilterAnimations(c, hold, found);
    if (found.empty()) return Fail("no animation retains the ball for the restart");
    Selector sel(w, c, hi);
    sel.SetMovementSimilarityPredicate(Vec3(0, -1, 0), kVelIdle);
    sel.Sort(found, [&](int i) { return sel.MovementSimilarityKey(i); });
    const int anim = found[0];

    Humanoid &h = HumanoidAt(w, hi);
    h.startAngle.set(FixAngle((Vec3(0) - h.startPos).Angle2D()));
    AnimationState &a = h.anim;
    a.anim = a.id = anim;
    a.frameNum = 0;
    a.touchFrame = -1;
    a.functionType = kFnMovement;
    a.positions.count = 0;
    DropSmuggles(a);
    AnimApplyBuffer &buf = h.applyBuf;
    buf.anim = anim;
    buf.smooth = false;
    buf.position = h.startPos;
    buf.orientation = h.startAngle;
    w.match.ballRetainer = hi;
    return true;
}

// ---- restarting persons, teams, the ball and the match ------------------------------------------------

// A player or official at a restart: its touch record and history cleared and, when active, placed
// where it stands facing `focus`; a player's controller forgets its last wish.
HDN bool RestartPerson(World &w, const Ctx &c, int hi, const Vec3 &focus) {
    const int players = w.match.playerCount;
    const bool isPlayer = hi < players;
    PersonBase &b = isPlayer ? w.match.players[hi].base : w.match.officials[hi - players];
    b.lastTouchTimeMs = 0;
    b.lastTouchType = kTouchNone;
    b.positionHistoryPerSecond.count = 0;
    if (b.isActive) {
        b.humanoid.mentalImageTime = 0;
        const Vec3 where = b.humanoid.spatial.position;
        if (!PlaceHumanoid(w, c, hi, where, focus)) return false;
    }
    if (!isPlayer) return true;
    if (ExternalControllerActive(w, hi)) {
        HumanControllerReset(w, b.externalController);
    } else {
        AIControllerState &ai = w.match.players[hi].controller;
        ai.lastDesiredDirection = Vec3(0);
        ai.lastDesiredVelocity = 0;
    }
    return true;
}
// A player at a restart: the person's restart, then no possession, a second to the ball and no
// marking or space ratings (the forward rating stays).
HDN bool RestartPlayer(World &w, const Ctx &c, int p, const Vec3 &focus) {
    if (!RestartPerson(w, c, p, focus)) return false;
    Player &ps = w.match.players[p];
    ps.hasPossession = ps.hasBestPossession = ps.hasUniquePossession = false;
    ps.triggerControlledBallCollision = false;
    ps.possessionDurationMs = 0;
    ps.desiredTimeToBallMs = 0;
    ps.timeToBallMs = ps.timeToBallOptimisticMs = 1000;
    w.roster.timeToBallMs[p] = 1000;
    ps.manMarking = -1;
    ps.tactical.forwardSpaceRating = ps.tactical.toGoalSpaceRating = ps.tactical.spaceRating = 0;
    return true;
}
// A team's AI with no restart under way, no plan running and an even possession picture.
HD void ClearTeamPlan(TeamAI &ai) {
    ai.setPieceType = kModeNormal;
    ai.taker = ai.attackingRunPlayer = ai.teamPressurePlayer = -1;
    ai.endApplyAttackingRunMs = ai.endApplyTeamPressureMs = ai.endApplyKeeperRushMs = 0;
    ai.offsideTrapX = 0;
    ai.teamHasPossession = ai.teamHasUniquePossession = ai.teamHasBestPossession = false;
    ai.oppTeamHasPossession = ai.oppTeamHasUniquePossession = false;
    ai.teamPossessionAmount = ai.fadingTeamPossessionAmount = 1.0f;
    ai.timeNeededToGetToBall = ai.oppTimeNeededToGetToBall = 100;
}
HDN bool RestartTeam(World &w, const Ctx &c, int teamID, const Vec3 &focus) {
    Team &t = TeamByID(w, teamID);
    t.hasPossession = false;
    t.timeToBallMs = 100;
    t.teamPossessionAmount = t.fadingTeamPossessionAmount = 1.0f;
    t.lastTouchPlayer = -1;
    const PlayerList all = TeamAllPlayers(w, teamID);
    if (all.empty()) {
        Fatal("a team has no players");
        return false;
    }
    t.designatedTeamPossessionPlayer = all[0];
    for (int i = 0; i < all.count; i++)
        if (w.roster.active[all[i]] && !RestartPlayer(w, c, all[i], focus)) return false;
    ClearTeamPlan(t.ai);
    return true;
}
// The ball lying still at `focus`, 11 cm up, every prediction there. Materializing first keeps the
// frame of the stored predictions.
HD void RestBall(Ball &b, const Vec3 &focus) {
    BallMaterialize(b);
    const Vec3 lying = focus + Vec3(0, 0, 0.11f);
    b.momentum = Vec3(0);
    b.rotationPerMs = b.orientationPrediction = b.orientationBuffer = Quat();
    b.positionBuffer = lying;
    for (int i = 0; i < kBallPredictionSpanMs / 10; i++) b.predictions[i] = lying;
    b.validPredictions = 0;
    b.positionHistory.count = 0;
    b.touchesNet = false;
    b.memoValid = false;
}
HDN bool RestartMatch(World &w, const Ctx &c, const Vec3 &focus) {
    MatchState &m = w.match;
    m.ballRetainer = m.lastTouchTeamID = m.lastGoalScorer = m.bestPossessionTeam = -1;
    for (int &t : m.lastTouchTeamIDs) t = -1;
    m.ballIsInGoal = m.goalScored = false;
    m.lastBodyBallCollisionTimeMs = 0;
    m.mentalImages.count = m.possessionSideHistory.count = m.cameraPosition.count = 0;
    RestBall(m.ball, focus);
    const int first = w.FirstTeamID();
    if (!RestartTeam(w, c, first, focus) || !RestartTeam(w, c, 1 - first, focus)) return false;
    // The referee is the first official.
    return RestartPerson(w, c, m.playerCount, focus);
}

// ---- placing a team for a restart -----------------------------------------------------------------

HD float ToFloat(double v) { return (float)v; }

// Where the outfield players of a team go for a goal kick, corner, throw-in, free kick or penalty:
// the placement of their formation positions, for the team that takes the restart or the one that
// defends it. `side` is the team's side of the pitch and `ball` the ball on the ground.
HD Placement PlacementRule(int setPiece, bool taking, int side, const Vec3 &ball) {
    const double hw = kPitchHalfWidth;
    const float L = kPitchHalfLength, own = side * kPitchHalfLength, theirs = -side * kPitchHalfLength;
    auto onPitch = [&](float x) { return Clamp(x, -L, L); };
    Placement r{};
    switch (setPiece) {
        case kModeGoalKick:
            r.back = ToFloat((double)own * (taking ? 0.5 : 0.4));
            r.front = ToFloat((double)theirs * (taking ? 0.2 : 0.1));
            r.low = ToFloat(-hw * 0.7);
            r.high = ToFloat(hw * 0.7);
            r.microFocus = Vec3(0);
            break;
        case kModeCorner:
            if (taking) {
                r.back = ToFloat((double)theirs * 0.2);
                r.front = ToFloat((double)theirs * 0.96);
                r.xFocus = ToFloat(r.front * 0.85);
            } else {
                r.back = ToFloat((double)own * 0.98);
                r.front = ToFloat((double)own * 0.5);
                r.xFocus = ToFloat(r.back * 0.94);
            }
            r.low = ToFloat(-hw * 0.6);
            r.high = ToFloat(hw * 0.6);
            r.xFocusStrength = taking ? 0.7f : 0.8f;
            r.yFocus = ball.v[1] * 0.1f;
            r.yFocusStrength = taking ? 0.7f : 0.9f;
            r.microFocus = Vec3(ball.v[0] * 0.95f, ball.v[1] * 0.1f, 0);
            r.microFocusStrength = 0.9f;
            r.midFocus = taking ? 0.9f : 0.1f;
            r.midFocusStrength = taking ? 0.5f : 0.7f;
            break;
        case kModeThrowIn:
            r.back = onPitch(ball.v[0] + 30 * side);
            r.front = onPitch(ball.v[0] + (taking ? 20 : 15) * -side);
            r.xFocus = taking ? onPitch(ball.v[0] + 4 * -side) : onPitch(ball.v[0] + 16 * side);
            r.xFocusStrength = ToFloat(taking ? 0.4 : 0.2);
            r.yFocus = ToFloat(ball.v[1] * (taking ? 0.996 : 0.95));
            r.yFocusStrength = ToFloat(taking ? 0.6 : 0.5);
            r.low = -kPitchHalfWidth * 0.75f + ball.v[1] * 0.25f;
            r.high = kPitchHalfWidth * 0.75f + ball.v[1] * 0.25f;
            r.microFocus = ball;
            r.microFocusStrength = ToFloat(0.7);
            break;
        case kModeFreeKick: {
            // How far up the pitch the kick is, 0 at the team's own line to 1 at the opponent's.
            const double up = (double)ToFloat((double)Clamp((ball.v[0] * -side) / L, ToFloat(-1.0), ToFloat(1.0)) * 0.5 + 0.5);
            if (taking) {
                r.back = onPitch(ToFloat((double)own * (0.7 - up * 0.7)));
                r.front = onPitch(ToFloat((double)own * (-0.3 - up * 0.7)));
                r.xFocus = onPitch(ball.v[0] + 10 * -side);
                r.xFocusStrength = ToFloat(0.5 + up * 0.2);
                r.yFocus = ToFloat(ball.v[1] * 0.4);
                r.yFocusStrength = ToFloat(0.6 + up * 0.2);
            } else {
                r.back = onPitch(ToFloat((double)own * (1.0 - up * 0.6)));
                r.front = onPitch(ToFloat((double)own * (0.5 - up * 0.8)));
                r.xFocus = onPitch(ball.v[0] + 20 * side);
                r.xFocusStrength = ToFloat(0.6 - up * 0.4);
                r.yFocus = ToFloat(ball.v[1] * 0.2);
                r.yFocusStrength = ToFloat(0.8 - up * 0.4);
            }
            r.low = ToFloat(-hw * 0.7);
            r.high = ToFloat(hw * 0.7);
            r.microFocus = ball;
            r.microFocusStrength = ToFloat(0.4);
            break;
        }
        case kModePenalty:
            r.back = onPitch(ball.v[0] + (taking ? 50 : 11) * side);
            r.front = onPitch(ball.v[0] + (taking ? 10 : 20) * -side);
            r.xFocus = ball.v[0];
            r.xFocusStrength = ToFloat(taking ? 0.6 : 1.0);
            r.yFocus = ToFloat(0.0);
            r.yFocusStrength = ToFloat(taking ? 0.8 : 1.0);
            r.low = ToFloat(-hw * 0.8);
            r.high = ToFloat(hw * 0.8);
            r.microFocus = Vec3(0);
            break;
    }
    return r;
}
HD bool HasPlacementRule(int setPiece) {
    return setPiece == kModeGoalKick || setPiece == kModeCorner || setPiece == kModeThrowIn || setPiece == kModeFreeKick ||
           setPiece == kModePenalty;
}

// Keeps `bp` at least `gap` metres from the ball on the ground, along the line from the ball.
HD Vec3 KeepOff(const Vec3 &bp, const Vec3 &ball, float gap) { return ball + (bp - ball).Normalized() * gap; }

// The kickoff spots: the formation pulled into the team's half, a random sideways step, at least
// 0.5 m behind the line and outside the centre circle; the taking team's two players nearest the
// centre spot go onto it again after every placement.
HDN bool PlaceForKickOff(World &w, const Ctx &c, int teamID, bool taking, const PlayerList &outfield, const Vec3 &ball) {
    const int side = TeamDynamicSide(w, teamID);
    const double ds = side, hl = kPitchHalfLength;
    const Vec3 scale(ToFloat((double)(-side * kPitchHalfLength) * 0.6), ToFloat((double)(-side * kPitchHalfWidth) * 0.6), 0);
    for (int i = 0; i < outfield.count; i++) {
        Vec3 bp = Formation(w, c, outfield[i]).position * scale;
        bp.v[1] += RandomInRange(w, -2.0f, 2.0f);
        bp.v[0] = ToFloat(bp.v[0] * 0.5);
        bp.v[0] = ToFloat(bp.v[0] + (hl * 0.2) * ds);
        if ((double)(bp.v[0] * side) < 0.5) bp.v[0] = ToFloat(0.5 * ds);
        if ((double)bp.Length() < 9.4) {
            bp.Normalize(Vec3(side, 0, 0));
            bp *= 9.4f;
        }
        if (!PlaceHumanoid(w, c, outfield[i], bp, ball)) return false;
        if (!taking) continue;
        const PlayerList centre = GetClosestPlayers(w, c, teamID, Vec3(0), false, 2);
        for (int k = 0; k < centre.count; k++)
            if (!PlaceHumanoid(w, c, centre[k], Vec3(0, ToFloat((double)k * 1.4 * ds), 0), ball)) return false;
    }
    return true;
}

// The outfield players by the restart's placement rule, then a defending wall 9.15 m from a free
// kick (three players between the ball and the goal when it is within 40 m) and, at a penalty,
// everyone outside the box and 9.65 m from the spot.
HDN bool PlaceByRule(World &w, const Ctx &c, int teamID, int setPiece, bool taking, const PlayerList &outfield, const Vec3 &ball) {
    const int side = TeamDynamicSide(w, teamID);
    const Placement r = PlacementRule(setPiece, taking, side, ball);
    const double hl = kPitchHalfLength;
    const int penaltyEnd = (ball.v[0] < 0) ? -1 : 1;
    for (int i = 0; i < outfield.count; i++) {
        Vec3 bp = PlaceInFormation(w, c, outfield[i], r, false);
        if (setPiece == kModeFreeKick && !taking && (double)(bp - ball).Length() < 9.15) bp = KeepOff(bp, ball, 9.15f);
        if (setPiece == kModePenalty) {
            if ((double)(bp.v[0] * penaltyEnd) > hl - 16.5 - 0.5) bp.v[0] = ToFloat((hl - 16.5 - 0.5) * penaltyEnd);
            if ((double)(bp - ball).Length() < 9.15 + 0.5) bp = KeepOff(bp, ball, ToFloat(9.15 + 0.5));
        }
        if (!PlaceHumanoid(w, c, outfield[i], bp, ball)) return false;
    }
    const Vec3 goal(side * kPitchHalfLength, 0, 0);
    if (setPiece == kModeFreeKick && !taking && (double)(ball - goal).Length() < 40.0) {
        const PlayerList wall = GetClosestPlayers(w, c, teamID, ball, false, 3);
        for (int k = 0; k < wall.count; k++) {
            Vec3 toGoal = (goal - ball).Normalized(0);
            toGoal += Vec3(0, ToFloat(1.0 - (double)k), 0) * ToFloat(0.07);
            toGoal.Normalize();
            if (!PlaceHumanoid(w, c, wall[k], ball + toGoal * 9.15f, ball)) return false;
        }
    }
    return true;
}

// The taking team's nearest player to the ball takes the restart: it stays put at a kickoff, stands
// 0.3 m off the ball holding it at a throw-in, 2.3 m behind it otherwise, 3 m behind at a penalty.
HDN bool PlaceTaker(World &w, const Ctx &c, int teamID, int setPiece, const Vec3 &ball) {
    TeamAI &ai = TeamByID(w, teamID).ai;
    const int side = TeamDynamicSide(w, teamID);
    const PlayerList nearest = GetClosestPlayers(w, c, teamID, ball, false, 2);
    if (nearest.empty()) return Fail("the set piece has no taker");
    const int taker = ai.taker = nearest[0];
    // The direction of the ball from the centre spot (down the touchline's normal at the spot).
    const Vec3 outward = ball.Normalized(Vec3(0, -side, 0));
    switch (setPiece) {
        case kModeKickOff:
            return true;
        case kModeThrowIn:
            return PlaceHumanoid(w, c, taker, ball + outward * 0.3f, ball) && HoldBallForThrowIn(w, c, taker);
        case kModeFreeKick:
            return PlaceHumanoid(w, c, taker, ball + Vec3(side, 0, 0) * 2.3f, ball);
        default:
            if (!PlaceHumanoid(w, c, taker, ball + outward * 2.3f, ball)) return false;
            return setPiece != kModePenalty || PlaceHumanoid(w, c, taker, ball + Vec3(side, 0, 0) * 3.0f, ball);
    }
}

// Whether the left team's nearest starting player stands nearer the ball's starting spot than the
// right team's.
HD float NearestStart(const FormationEntry *team, int size, const Vec3 &ball) {
    float nearest = 1000000;
    for (int i = 0; i < size; i++) nearest = MinF(nearest, (team[i].startPosition - ball).Length());
    return nearest;
}
HDN bool LeftTeamStartsNearerBall(const World &w) {
    const Scenario &s = w.scenario;
    return NearestStart(s.leftTeam, s.leftTeamSize, s.ballPosition) < NearestStart(s.rightTeam, s.rightTeamSize, s.ballPosition);
}

// A team's placement for a restart: its goalkeepers on their line, its outfield players by the
// restart, at a kickoff everyone back to the starting formation (the two teams' swapped when GRF
// swaps them), then the taker.
HDN bool PlaceTeam(World &w, const Ctx &c, int teamID, int setPiece, int otherTeamID, int kickoffTeamID, int takerTeamID) {
    MatchState &m = w.match;
    Team &team = TeamByID(w, teamID);
    team.ai.setPieceType = setPiece;
    if (setPiece == kModeNormal) return true;
    const int side = TeamDynamicSide(w, teamID);
    const bool taking = takerTeamID == teamID;
    const Vec3 ball = BallPredict(m.ball, 0).Get2D();

    const PlayerList active = TeamActivePlayers(w, teamID);
    PlayerList outfield;
    const Vec3 goalLine((float)((double)(kPitchHalfLength * side) * 0.98), 0, 0);
    for (int i = 0; i < active.count; i++) {
        if (Formation(w, c, active[i]).role != kRoleGoalkeeper) {
            outfield.push_back(active[i]);
            continue;
        }
        Vec3 facing = ball;
        if (setPiece == kModeKickOff) facing.v[0] = facing.v[1] = 0;
        if (!PlaceHumanoid(w, c, active[i], goalLine, facing)) return false;
    }
    // GRF passes a double here, which rounds to float.
    team.fadingTeamPossessionAmount = taking ? 1.5f : 0.5f;

    bool placed;
    if (setPiece == kModeKickOff) {
        placed = PlaceForKickOff(w, c, teamID, taking, outfield, ball);
    } else if (HasPlacementRule(setPiece)) {
        placed = PlaceByRule(w, c, teamID, setPiece, taking, outfield, ball);
    } else {
        const Vec3 scale(ToFloat((double)(-side * kPitchHalfLength) * 0.7), ToFloat((double)(-side * kPitchHalfWidth) * 0.7), 0);
        placed = true;
        for (int i = 0; i < outfield.count && placed; i++)
            placed = PlaceHumanoid(w, c, outfield[i], Formation(w, c, outfield[i]).position * scale, ball);
    }
    if (!placed) return false;

    if (setPiece == kModeKickOff) {
        // GRF: after the start, a kickoff to the team that did not own the ball at the start swaps
        // the start positions of two teams of equal size.
        const PlayerList own = TeamAllPlayers(w, teamID);
        const bool swap = m.matchTimeMs > 0 && TeamAllPlayers(w, otherTeamID).size() == own.size() &&
                          (LeftTeamStartsNearerBall(w) ^ (kickoffTeamID == 0));
        const PlayerList spots = swap ? TeamAllPlayers(w, otherTeamID) : own;
        const Vec3 scale(-side * kPitchHalfLength, -side * kPitchHalfWidth, 0);
        for (int i = 0; i < spots.count; i++) {
            if (!w.roster.active[own[i]]) continue;
            if (!PlaceHumanoid(w, c, own[i], Formation(w, c, spots[i]).startPosition * scale, ball)) return false;
        }
    }
    if (!taking) {
        team.ai.taker = -1;
        return true;
    }
    return PlaceTaker(w, c, teamID, setPiece, ball);
}

// ---- sending a player off ---------------------------------------------------------------------------

// GRF's red card: the referee's message draws once; the player is restarted where it stands (its
// gamers move to the nearest selectable team mate), restarted again, deactivated and released; the
// team's designated player is the one nearest the ball, and a keeper's formation entry passes to
// the team's first remaining player.
HDN bool SendOff(World &w, const Ctx &c, int p) {
    MatchState &m = w.match;
    Player &ps = m.players[p];
    const int t = w.playerTeamID[p];
    RandomInRange(w, 0, 3);
    auto standing = [&]() { return ps.base.humanoid.spatial.position; };
    if (!RestartPlayer(w, c, p, standing())) return false;
    if (ps.base.externalController >= 0) {
        Team &team = TeamByID(w, t);
        for (int g = 0; g < team.gamers.count; g++) {
            if (team.gamers[g].selectedPlayer != p) continue;
            const int mate = GetClosestPlayer(w, c, t, standing(), true, p, true);
            team.mainSelectedPlayer = mate;
            HumanGamerSetSelectedPlayer(w, GlobalGamerIndex(w, t, g), mate);
        }
    }
    if (!RestartPlayer(w, c, p, standing())) return false;
    ps.base.isActive = false;
    w.roster.active[p] = false;
    ps.base.externalController = -1;
    TeamByID(w, t).designatedTeamPossessionPlayer = GetClosestPlayer(w, c, t, BallPredict(m.ball, 0).Get2D(), false);
    if (Formation(w, c, p).role != kRoleGoalkeeper) return true;
    for (int q = 0; q < m.playerCount; q++)
        if (w.playerTeamID[q] == t && w.roster.active[q]) {
            w.formationOverride[q] = (int8_t)(1 + FormationSource(w, p));
            return true;
        }
    Fatal("the sending-off leaves no active player");
    return false;
}

// The referee's restart: a free kick's spot kept inside 95% of the pitch, the match restarted
// around the spot (in the rest frame), both teams placed in processing order, the taker recorded.
HDN bool RefereeRestart(World &w, const Ctx &c, int setPiece) {
    Referee &ref = w.match.referee;
    RefereeBuffer &b = ref.buffer;
    if (setPiece == kModeFreeKick) {
        b.restartPos.v[0] = Clamp(b.restartPos.v[0], (float)(-0.95 * kPitchHalfLength), (float)(0.95 * kPitchHalfLength));
        b.restartPos.v[1] = Clamp(b.restartPos.v[1], (float)(-0.95 * kPitchHalfWidth), (float)(0.95 * kPitchHalfWidth));
    }
    if (!RestartMatch(w, c, w.scenario.reverseTeamProcessing ? -b.restartPos : b.restartPos)) return false;
    const int first = w.FirstTeamID(), second = 1 - first;
    // The buffer stores the kickoff team as its slot.
    const int kickoffTeam = b.setPieceTeam == 0 ? first : second;
    if (!PlaceTeam(w, c, first, setPiece, second, kickoffTeam, b.teamID)) return false;
    if (!PlaceTeam(w, c, second, setPiece, first, kickoffTeam, b.teamID)) return false;
    b.taker = TeamByID(w, b.teamID).ai.taker;
    ref.offsidePlayers.count = 0;
    return true;
}

}  // namespace eng
