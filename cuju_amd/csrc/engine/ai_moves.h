// SPDX-License-Identifier: Apache-2.0
// Restates game logic of cuju (Copyright 2026 The cuju Authors), a reimplementation of Google
// Research Football (Copyright 2019 Google LLC); see NOTICE.
// The player AI, first half: the state it reads, the defensive component, the ball commands and
// the movement towards the ball, the formation and the support positions.
// Semantics: include/cuju/simulation/ai_controller.h:418-1620.
#pragma once

#include "ai.h"

namespace eng {

struct AIBase {
    World &w;
    const Ctx &c;
    const int p;
    MatchState &m;
    Player &ps;
    AIControllerState *eliza;  // null under a gamer
    PlayerControllerState &ctl;
    const int teamID, oppID, side;  // `side`: the sign of x of the own goal
    int k = 0;                      // mental image
    CommandQueue &q;

    HD AIBase(World &world, const Ctx &ctx, int player, CommandQueue &queue, PlayerControllerState &controller,
              AIControllerState *e)
        : w(world),
          c(ctx),
          p(player),
          m(world.match),
          ps(world.match.players[player]),
          eliza(e),
          ctl(controller),
          teamID(world.playerTeamID[player]),
          oppID(1 - world.playerTeamID[player]),
          side(TeamDynamicSide(world, world.playerTeamID[player])),
          q(queue) {}

    HD Vec3 Pos(int o) const { return Sp(w, o).position; }
    HD Vec3 Mov(int o) const { return Sp(w, o).movement; }
    HD Vec3 Dir(int o) const { return Sp(w, o).directionVec; }
    HD Vec3 Pos() const { return Pos(p); }
    HD Vec3 Mov() const { return Mov(p); }
    HD Vec3 Dir() const { return Dir(p); }
    HD float FloatVelocity() const { return PlayerFloatVelocity(w, p); }
    HD float Stat(int s) const { return GetStatistic(w, c, p, s); }
    HD int StaticRole(int o) const { return Formation(w, c, o).role; }
    HD int DynamicRole() const { return ps.dynamicFormationEntry.role; }
    HD const Team &Own() const { return TeamByID(w, teamID); }
    HD const Team &Opp() const { return TeamByID(w, oppID); }
    HD const TeamAI &AI() const { return Own().ai; }
    HD Vec3 MentalBall(int ms) const { return MentalBallPrediction(w, k, ms); }
    HD Vec3 BallAt(int ms) const { return BallPredict(m.ball, ms); }

    // How likely the player is to win a duel for the ball with the opponents' designated player
    // (both 0.1 s ahead): 1 when the opponent stands between it and the ball seen 100 ms ahead
    // facing away, 0 when the player is between.
    HD float CouldWinABallDuelLikeliness() const {
        const int o = Opp().designatedTeamPossessionPlayer;
        const Vec3 opponent = Pos(o) + Mov(o) * 0.1f;
        const Vec3 toOpponent = opponent - (Pos() + Mov() * 0.1f);
        const Vec3 opponentToBall = MentalBall(100).Get2D() - (Pos(o) + Mov(o) * 0.1f);
        const float behind = toOpponent.Normalized(0).Dot(opponentToBall.Normalized(0)) * 0.5f + 0.5f;
        return (1.0f - behind);
    }

    // The shooting point of an opponent (as the player saw it a reaction time ago, 0.5 s ahead):
    // on its way to the team's goal, 24 m out for the designated player and 8 m for others (at
    // least 0.4 m from where it is), held to the offside trap. Returns its distance from the
    // opponent in `reach`.
    HD Vec3 ShootingPoint(int o, const Vec3 &goal, float &reach) const {
        const PlayerImage oi = MentalPlayerImage(w, MentalImageIndex(w, PlayerControllerReactionTime(w, c, p)), o);
        const Vec3 op = oi.position + oi.movement * 0.5f;
        const float range = o == m.designatedPossessionPlayer ? 24.0f : 8.0f;
        reach = Clamp((goal - op).Length() - range, 0.4f, kPitchHalfLength);
        Vec3 point = op + (goal - op).Normalized(0) * reach;
        const float trapX = AI().offsideTrapX;
        if (point.v[0] * side > trapX * side) {
            const Line toGoal(op, goal);
            const Line trap(Vec3(trapX, -kPitchHalfWidth, 0), Vec3(trapX, kPitchHalfWidth, 0));
            point = toGoal.IntersectionPoint(trap);
            reach = (point - op).Length();
        }
        return point;
    }
    // Moves `desired` toward defending the marked (or forced) opponent, by `bias`, in open play
    // for outfield players: to within the opponent's reach of its shooting point less a 4 m
    // buffer, then goalside by 70% of however far the player (0.14 s ahead) is beyond that reach.
    HDN void AddDefensiveComponent(Vec3 &desired, float bias, int forcedOpp = -1) const {
        const int o = forcedOpp < 0 ? ps.manMarking : forcedOpp;
        if (!(m.inPlay && !m.inSetPiece && StaticRole(p) != kRoleGoalkeeper)) return;
        if (o < 0) return;
        const float buffer = 4.0f;
        const Vec3 goal = Vec3(kPitchHalfLength * side, 0, 0);
        float reach = 0;
        const Vec3 point = ShootingPoint(o, goal, reach);
        Vec3 defend = desired;
        const Vec3 toPoint = point - desired;
        const float toPointLength = toPoint.Length();
        const float slack = toPointLength - (reach - buffer);
        if (slack > 0.0f) defend = desired + toPoint.Normalized(0) * Clamp(slack, 0.0f, toPointLength);
        const float late = (point - (Pos() + Mov() * 0.14f)).Length() - reach;
        if (late > 0.0f) defend += (goal - defend).Normalized(0) * late * 0.7f;
        desired = desired * (1.0f - bias) + defend * bias;
    }
    // Where to stand against opponent `o` (as the player sees it): on its line to the team's goal
    // where the perpendicular bisector of the player and the opponent crosses it (within the
    // line), plus a tenth of a sprint second and `distance` toward goal and its movement 0.14 s on.
    HDN Vec3 GetDefendPosition(int o, float distance = 0.0f) const {
        const PlayerImage oi = MentalPlayerImage(w, k, o);
        const Vec3 goal = Vec3(kPitchHalfLength * side, 0, 0);
        const Vec3 op = oi.position;
        const Vec3 home = goal - op;
        const Line toGoal(op, goal);
        const Line between(Pos(), op);
        const Vec3 mid = between.pts[0] * 0.5f + between.pts[1] * 0.5f;
        const Line bisector(mid, mid + (between.pts[0] - mid).Rotated2D((float)(0.5 * (double)PI)));
        float along = 0.0f;
        toGoal.IntersectionPoint(bisector, along);
        along = Clamp(along, 0.0f, 1.0f);
        Vec3 stand = toGoal.pts[0] + (toGoal.pts[1] - toGoal.pts[0]) * along;
        stand += (home.Normalized(0) * kSprintVelocity * 0.1f) + (oi.movement * 0.14f) + (home.Normalized(0) * distance);
        return stand;
    }

    // ---- commands ----
    // The ball in the goalkeeper's reach for a save: within 10 m beyond the optimization
    // threshold in 400 ms, free, in its penalty box in 160 ms (compared in double), and not a
    // teammate's kick (a back pass).
    HD bool BallSaveable() const {
        if (GetDistance(BallAt(400), Pos()) > kBallDistanceOptimizeThreshold + 10.0f) return false;
        if (m.lastTouchTeamID == teamID && MatchLastTouchPlayer(w) != p && m.lastTouchTeamIDs[kTouchKicked] == teamID) return false;
        if (m.ballRetainer >= 0) return false;
        const Vec3 ball = BallAt(160);
        return !(fabsf(ball.v[1]) > 20.05f) && !((double)(ball.v[0] * -side) > -(double)kPitchHalfLength + 16.4);
    }
    // A goalkeeper's deflection (only those that pick the ball up, on request) of a saveable ball.
    HDN void KeeperDeflectCommand(bool onlyPickup) {
        if (StaticRole(p) != kRoleGoalkeeper || !BallSaveable()) return;
        PlayerCommand cmd = DefaultPlayerCommand();
        cmd.desiredFunctionType = kFnDeflect;
        if (onlyPickup) cmd.onlyDeflectAnimationsThatPickupBall = true;
        q.push_back(cmd);
    }
    // Waiting at a set piece: standing, facing on; looking at the ball, or, for the retainer,
    // along its input.
    HDN void SetPieceCommand() {
        PlayerCommand cmd = DefaultPlayerCommand();
        cmd.useDesiredMovement = true;
        cmd.useDesiredLookAt = true;
        cmd.desiredDirection = Dir();
        cmd.desiredVelocityFloat = kIdleVelocity;
        cmd.desiredLookAt = m.ballRetainer == p ? Pos() + ctl.inputDirection * 10.0f : BallAt(0).Get2D();
        q.push_back(cmd);
    }
    // ---- touch commands: each a guard, then a command from the input ----
    // The ball free and near (within the optimization threshold of where it will be in 200 ms).
    HD bool BallFreeAndNear() const { return !(GetDistance(BallAt(200), Pos()) > kBallDistanceOptimizeThreshold) && m.ballRetainer < 0; }
    // A command of `fn` along the input (snapped to 8 directions with no bias when `snap`), at the
    // input's speed; an idle input turns to the opponents' goal on request.
    HD PlayerCommand InputCommand(int fn, bool snap, bool idleTurnToGoal) const {
        PlayerCommand cmd = DefaultPlayerCommand();
        cmd.desiredFunctionType = fn;
        cmd.useDesiredMovement = true;
        cmd.desiredDirection = ctl.inputDirection;
        if (snap) QuantizeDirection(cmd.desiredDirection, kQuantizedDirectionBias);
        cmd.desiredVelocityFloat = ctl.inputVelocityFloat;
        if (VelocityCat(cmd.desiredVelocityFloat) == kVelIdle && idleTurnToGoal) cmd.desiredDirection = Vec3(-side, 0, 0);
        return cmd;
    }
    // Ball control: for the match's designated player, or the team's one likely enough (25%) to win
    // the duel; off the ball and not in last ditch, only for a ball neither rising nor falling and
    // not running faster than 15 m/s relative to the player. A sprinting dribbler's sticky run
    // turns at most an eighth turn; a walking or dribbling player asked to dribble can keep its
    // body direction, walking.
    HDN void BallControlCommand(bool idleTurnToGoal = false, bool knockOn = false, bool stickyRun = false,
                                bool keepBodyDirection = false) {
        if (!BallFreeAndNear()) return;
        if (!ps.hasPossession && !AllowLastDitchOf(w, p)) {
            const float strictnessInverse = 3.0f;
            if (fabsf(m.ball.momentum.v[2]) > 5.0f * strictnessInverse) return;
            if ((m.ball.momentum.Get2D() - Mov()).Length() > 5.0f * strictnessInverse) return;
        }
        if (!(m.designatedPossessionPlayer == p || (Own().designatedTeamPossessionPlayer == p && CouldWinABallDuelLikeliness() >= 0.25f)))
            return;
        PlayerCommand cmd = InputCommand(kFnBallControl, true, idleTurnToGoal);
        if (knockOn) cmd.modifier |= kModifierKnockOn;
        if (stickyRun && ctl.hasPossession && ctl.hasBestPossession && cmd.desiredVelocityFloat > kWalkSprintSwitch &&
            FloatVelocity() > kDribbleWalkSwitch) {
            const float turn = cmd.desiredDirection.Angle2D(Dir());
            if (fabsf(turn) > 0.125f * PI && fabsf(turn) < 0.7f * PI) {
                if (turn > 0) cmd.desiredDirection = Dir().Rotated2D(0.125f * PI);
                if (turn < 0) cmd.desiredDirection = Dir().Rotated2D(0.125f * -PI);
            }
        }
        cmd.useDesiredLookAt = true;
        const int moving = Sp(w, p).velocityCat;
        if (keepBodyDirection && (moving == kVelWalk || moving == kVelDribble) && VelocityCat(cmd.desiredVelocityFloat) == kVelDribble) {
            cmd.desiredVelocityFloat = kWalkVelocity;
            cmd.desiredLookAt = Pos() + Dir() * 10.0f;
        } else {
            cmd.desiredLookAt = Pos() + Mov() * 0.2f + cmd.desiredDirection * 10.0f;
        }
        q.push_back(cmd);
    }
    // A trap of a ball moving at least 2 m/s that the player does not hold: for the match's
    // designated player, or the team's one that reaches the ball within a second while the
    // opponents need 400 ms more, do not hold it and are half likely to lose the duel. An AI
    // goalkeeper traps facing upfield, standing.
    HDN void TrapCommand(bool idleTurnToGoal = false, bool knockOn = false) {
        if (m.ball.momentum.Get2D().Length() < 2.0f || !BallFreeAndNear() || ctl.hasPossession) return;
        if (!(m.designatedPossessionPlayer == p ||
              (Own().designatedTeamPossessionPlayer == p && ps.timeToBallOptimisticMs < 1000 && ctl.oppTimeNeededToGetToBall > 400 &&
               !ctl.oppTeamHasPossession && CouldWinABallDuelLikeliness() >= 0.5f)))
            return;
        PlayerCommand cmd = InputCommand(kFnTrap, true, false);
        if (StaticRole(p) == kRoleGoalkeeper && !ExternalControllerActive(w, p)) {
            cmd.desiredDirection = Vec3(-side, 0, 0);
            cmd.desiredVelocityFloat = kIdleVelocity;
        }
        if (VelocityCat(cmd.desiredVelocityFloat) == kVelIdle && idleTurnToGoal) cmd.desiredDirection = Vec3(-side, 0, 0);
        if (knockOn) cmd.modifier |= kModifierKnockOn;
        cmd.useDesiredLookAt = true;
        cmd.desiredLookAt = Pos() + Mov() * 0.3f + cmd.desiredDirection * 10.0f;
        q.push_back(cmd);
    }
    // Interference when the team is not best placed: by any means (loosely), or strictly when at
    // least 20% likely to win the duel.
    HDN void InterfereCommand(bool byAnyMeans) {
        if (!BallFreeAndNear() || ctl.teamHasBestPossession) return;
        if (!byAnyMeans && CouldWinABallDuelLikeliness() < 0.2f) return;
        PlayerCommand cmd = InputCommand(kFnInterfere, false, false);
        cmd.strictMovement = byAnyMeans ? kStrictFalse : kStrictTrue;
        q.push_back(cmd);
    }
    // A sliding tackle, only without gamers in the team: the opponents hold the ball, the team is
    // badly placed (possession under 0.6) and the player, not the designated one, 70% likely to
    // win the duel, with the ball 0.7 to 1.6 m from where it will be in 200 ms (the opponents
    // needing more than 260 ms to it), or 0.6 to 1.8 m from it while their player winds up a shot.
    // It sprints at the ball, led by the opponent's movement.
    HDN void SlidingCommand() {
        if (HumanGamerCount(Own()) != 0 || m.ballRetainer >= 0 || CouldWinABallDuelLikeliness() < 0.7f) return;
        if (!(!ctl.teamHasBestPossession && ctl.possessionAmount < 0.6f && m.designatedPossessionPlayer != p && ctl.oppTeamHasPossession))
            return;
        const int o = ctl.opponentPlayer;
        const Vec3 ball = MentalBallPrediction(w, MentalImageIndex(w, 20), 200);
        const Vec3 ahead = Pos() + Mov() * (float)0.2;
        const float gap = (ahead - ball).Length();
        const AnimationState &oa = Hum(w, o).anim;
        const bool loose = gap > 0.7f && gap < 1.6f && ctl.oppTimeNeededToGetToBall > 260;
        const bool shooting = gap > 0.6f && gap < 1.8f && oa.functionType == kFnShot && oa.frameNum < oa.touchFrame;
        if (!(loose || shooting)) return;
        PlayerCommand cmd = DefaultPlayerCommand();
        cmd.desiredFunctionType = kFnSliding;
        cmd.useDesiredMovement = true;
        cmd.desiredDirection = ((ball.Get2D() + Mov(o) * 0.2f) - ahead).Normalized(Vec3(-side, 0, 0));
        cmd.desiredVelocityFloat = kSprintVelocity;
        cmd.useDesiredLookAt = true;
        cmd.desiredLookAt = Pos() + Mov() * 0.1f + cmd.desiredDirection * 10.0f;
        q.push_back(cmd);
    }

    // ---- movement towards the ball ----
    // Staying on a held ball: toward where it will be at the touch (250 ms plus the touch offset
    // ahead), blending back to the player's own direction within 0.4 m (to the 0.5), looking that
    // way; the speed the distance at the AI's rate, or, from dribbling speed on, the desired speed
    // held up to 8 m/s above it and eased 10% toward (90% up to) the nearest velocity category.
    // Returns the player's time to the ball.
    HDN unsigned BallControlMovement(float desiredVel, Vec3 &bestDir, float &bestVel, Vec3 &bestLookAt) const {
        ENG_SCOPE(47);
        const Vec3 toBall = MentalBall((int)(250 + kDefaultTouchOffsetMs)).Get2D() - Pos();
        const float dist = toBall.Length();
        const float toward = dist < 0.4f ? libm::powf(NormalizedClamp(dist, 0.2f, 0.4f), 0.5f) : 1.0f;
        bestDir = toBall.Normalized(Dir()) * toward + Dir() * (1.0f - toward);
        bestDir.Normalize(Dir());
        bestVel = dist * kDistanceToVelocity;
        // GRF: a velocity not below the dribble velocity, NaN included, takes the clamp.
        if (!(bestVel < kDribbleVelocity)) {
            bestVel = Clamp(desiredVel, bestVel, bestVel + 8.0f);
            if (RangeVelocity(bestVel) < bestVel) bestVel = bestVel * 0.9f + RangeVelocity(bestVel) * 0.1f;
            if (RangeVelocity(bestVel) > bestVel) bestVel = bestVel * 0.1f + RangeVelocity(bestVel) * 0.9f;
        }
        bestLookAt = Pos() + bestDir * 10.0f;
        return ps.timeToBallMs;
    }

    // The desired direction snapped to the nearest of 16 directions in the frame of the ball's
    // path (the path from now to a second ahead as the x axis).
    HD Vec3 SnapInBallFrame(const Vec3 &desiredDir) const {
        const Vec3 along = (MentalBall(0).Get2D() - MentalBall(1000).Get2D()).Normalized(desiredDir);
        const float frame = along.Angle2D();
        Vec3 inFrame = desiredDir.Rotated2D(-frame);
        const int directions = 16;
        float a = inFrame.Angle2D();
        a /= PI * 2.0f;
        a = roundf(a * directions);
        a /= directions;
        a *= PI * 2.0f;
        const float bias = 1.0f;
        inFrame = (inFrame * (1.0f - bias) + (Vec3(1, 0, 0).Rotated2D(a) * bias)).Normalized(inFrame);
        return inFrame.Rotated2D(frame);
    }
    // How an interception point suits the chase: the movement toward it against the desired
    // movement (40%) and direction (60%), its time (within 5 s), its distance from the point of the
    // ball's path nearest the player (within two sprint seconds) and the last desired time to the
    // ball, by the weights.
    struct InterceptWeights {
        float movement, time, perpendicular, previous;
    };
    HD float InterceptRating(const InterceptWeights &wt, const Vec3 &target, unsigned t, const Vec3 &desiredDir, const Vec3 &desiredMov,
                             const Vec3 &nearestOnPath, int previousDesired, int timeToBall) const {
        const Vec3 pp = Pos();
        const float speed = Clamp((target - pp).Length() * kDistanceToVelocity, kIdleVelocity, kSprintVelocity);
        const Vec3 toward = (target - pp).Normalized(0) * speed;
        float movement = 1.0f - NormalizedClamp((desiredMov - toward).Length(), 0.0f, kSprintVelocity);
        const float direction = 1.0f - NormalizedClamp(fabsf(desiredDir.Angle2D(toward.Normalized(desiredDir))), 0.0f, 0.5f * PI);
        movement = movement * 0.4f + direction * 0.6f;
        const float time = 1.0f - NormalizedClamp((float)t, 0, 5000);
        const float perpendicular = 1.0f - NormalizedClamp((nearestOnPath - target).Length(), 0, 2.0f * kSprintVelocity);
        float previous = 0.0f;
        if (previousDesired >= timeToBall) {
            const int diff = previousDesired - timeToBall;
            previous = 1.0f - (diff < 0 ? -diff : diff) / 500.0f;
        }
        return movement * wt.movement + time * wt.time + perpendicular * wt.perpendicular + previous * wt.previous;
    }
    // Where to look while chasing: along the desired direction when the interception is within
    // 100 ms or the chase is idle, else the desired direction held within the sector between the
    // ball and the chase direction; at most a quarter turn off the ball, 10 m out.
    HD Vec3 ChaseLookAt(int bestTime, float bestVel, const Vec3 &desiredDir, const Vec3 &chaseDir) const {
        const Vec3 pp = Pos();
        const Vec3 ball = (MentalBall(20).Get2D() - pp).Normalized(desiredDir);
        Vec3 look = desiredDir;
        if (!(bestTime < 100) && VelocityCat(bestVel) != kVelIdle) look = GetClamped2D(desiredDir, ball, chaseDir);
        return pp + ball.Rotated2D(Clamp(look.Angle2D(ball) * 1.0f, -0.25f * PI, 0.25f * PI)) * 10.0f;
    }

    // GRF's chase of a loose ball: from the player's time to the ball on, the points of the
    // mental ball's path below 1 m (stepping by a twentieth of the slack, 10 to 100 ms) that the
    // player reaches in time, rated by how they suit the desired movement (or, with haste, by
    // time); a point off the pitch, or one reached while the ball comes toward the player or far
    // earlier than its time to the ball, ends the scan. Returns the chosen time (the span's end
    // without one), with the direction, speed and look-at of the chase.
    HDN unsigned ToBallMovement(const Vec3 &desiredDir, float desiredVel, Vec3 &bestDir, float &bestVel, Vec3 &bestLookAt,
                                float haste) const {
        ENG_SCOPE(39);
        const Vec3 pp = Pos();
        const float maxVel = GetMaximumVelocity(*c.sd, p);
        InterceptWeights weights{1.0f, 0.0f, 0.1f, 0.0f};
        if (haste > 0.0f) weights = {0.0f, 1.0f, 0.0f, 0.0f};
        const Line path(MentalBall(0).Get2D(), MentalBall(1000).Get2D());
        float along = 0;
        path.DistanceToPoint(pp, along);
        const Vec3 nearestOnPath = path.pts[0] + (path.pts[1] - path.pts[0]) * along;
        const Vec3 snapped = SnapInBallFrame(desiredDir);
        const Vec3 desiredMov = snapped * desiredVel;
        float bestRating = -10000.0f;
        int bestNeeded = -10, bestTime = -10;
        const uint32_t ttb = ps.timeToBallMs;
        unsigned start = TruncToUint32(Clamp((float)ttb, 40, (float)(kBallPredictionSpanMs - 10)));
        const Vec3 first = MentalBall((int)start);
        if (fabsf(first.v[0]) > kPitchHalfLength - 0.2f || fabsf(first.v[1]) > kPitchHalfWidth - 0.2f) start = 80;
        const int previousDesired = ps.desiredTimeToBallMs;
        const Vec3 ballHeading = ((MentalBall((int)(ttb + 10)) - MentalBall((int)ttb)).Get2D() * 100.0f).Normalized(snapped);
        unsigned step = 1;
        const Vec3 mov = Mov();
        const bool walks = TimeWalkApplies(mov);
        TimeWalk &walk = c.ws->walk;
        bool built = false;
        const MentalBallView mental(w, k);
        TimeNeededScan scan(pp, mov, maxVel);
        for (unsigned t = start; t < (unsigned)kBallPredictionSpanMs; t += 10 * step) {
            Vec3 target = mental.At((int)t);
            bool last = fabsf(target.v[0]) > kPitchHalfLength - 0.2f || fabsf(target.v[1]) > kPitchHalfWidth - 0.2f;
            if (!last && target.v[2] >= 1.0f) continue;
            target = target.Get2D();
            TimeNeeded tn;
            if (!scan.Unreachable(target, true, t, tn)) {
                if (walks && !built) {
                    BuildTimeWalk(walk, pp, mov, maxVel);
                    GroupSync();
                    built = true;
                }
                tn = walks ? WalkTimeNeeded(walk, pp, mov, target, maxVel, true, t, true) : GetTimeNeededMs(pp, mov, target, maxVel, true, t);
            }
            const unsigned needed = tn.usual;
            int next = TruncToInt32(roundf((float)(int)(needed - t) * 0.05f)) - 5;
            next = next < 1 ? 1 : next;
            next = 10 < next ? 10 : next;
            step = (unsigned)next;
            if (needed <= t) {
                if (Clamp((float)ttb / (float)t, 0.0f, 1.0f) < 0.35f) last = true;
                if ((target - pp).Normalized(0).Dot(ballHeading) > 0.0f) last = true;
                const float rating = InterceptRating(weights, target, t, snapped, desiredMov, nearestOnPath, previousDesired, (int)ttb);
                if (rating > bestRating || (last && bestTime == -10)) {
                    bestRating = rating;
                    bestTime = (int)t;
                    bestNeeded = (int)needed;
                }
            }
            if (last) {
                if (bestTime == -10) bestTime = bestNeeded = (int)t;
                break;
            }
        }
        if (bestTime == -10) bestTime = bestNeeded = kBallPredictionSpanMs - 10;
        bestDir = (MentalBall(bestTime).Get2D() - pp).Normalized(Dir());
        bestVel = Clamp(((float)bestNeeded / (float)bestTime) * maxVel, kIdleVelocity, kSprintVelocity);
        if (bestTime > 250) bestVel = bestVel * 0.97f + FloatVelocity() * 0.03f;
        bestLookAt = ChaseLookAt(bestTime, bestVel, snapped, bestDir);
        return (unsigned)bestTime;
    }

    // Where a player moving by its input looks: turned from its direction toward the ball in
    // 40 ms (half a metre ahead of it), fully when slow, 30% less (to the 0.5, then the 0.7) at a
    // sprint.
    HD Vec3 InputLook(const Vec3 &manualDir) const {
        const float slow =
            1.0f - libm::powf(NormalizedClamp(MinF(ctl.inputVelocityFloat, FloatVelocity()), kIdleDribbleSwitch, kSprintVelocity), 0.5f) *
                       0.3f;
        Vec3 focus = MentalBall(40).Get2D();
        focus += Dir() * 0.5f;
        const float toFocus = (focus - Pos()).Normalized(manualDir).Angle2D(manualDir);
        return manualDir.Rotated2D(toFocus * libm::powf(slow, 0.7f));
    }
    // Whether the player goes for the ball: forced; the match's designated player; or the team's
    // designated player with its team holding the ball (possession over 0.5 after a recent touch
    // of its own or with the opponents off it, over 0.99, or its own best possession).
    HD bool GoesForBall(bool forceMagnet) const {
        const int teamDesignated = Own().designatedTeamPossessionPlayer;
        const float poss = ctl.possessionAmount;
        return forceMagnet || m.designatedPossessionPlayer == p ||
               ((GetLastTouchBias(w, p, 2000) > 0.01f && poss > 0.5f) && teamDesignated == p) ||
               ((!ctl.oppTeamHasPossession && poss > 0.5f) && teamDesignated == p) || (poss > 0.99f && teamDesignated == p) ||
               (ctl.hasBestPossession && teamDesignated == p);
    }
    // How much a chase that is not the match's designated player's overrides the input: by a
    // recent own touch (within 1.7 s of the ball, to the 0.4) and the chase's agreement with the
    // input (to the 0.5); for a gamer's player with the opponents off the ball, at least the
    // magnet of agreement or a recent switch, by possession and less toward the own half; all of
    // it when forced.
    HD float ChaseOverride(const Vec3 &chaseDir, const Vec3 &manualDir, float ownHalf, bool forceMagnet) const {
        float agree = 1.0f - Clamp(fabsf(chaseDir.Angle2D(manualDir)) / PI, 0.0f, 1.0f);
        agree = agree * 0.5f + 0.5f;
        float bias = 0.0f;
        if (GetLastTouchBias(w, p, 2000) > 0.01f && ps.timeToBallMs < 1700)
            bias = libm::powf(GetLastTouchBias(w, p, 2000), 0.4f) * libm::powf(agree, 0.5f);
        if (!ctl.oppTeamHasPossession && ps.base.externalController >= 0) {
            float magnet = MaxF(Curve(agree, 0.8f), libm::powf(GetLastSwitchBias(w, ctl), 0.5f));
            magnet *= 1.0f - ownHalf;
            bias = Clamp(libm::powf((MaxF(ctl.possessionAmount, 0.5f) - 0.5f) * 2.0f, 0.5f) * magnet, bias, 1.0f);
        }
        if (forceMagnet) bias = 1.0f;
        return bias;
    }
    // The team's designated player against an opponent on the ball: a gamer's player is pulled
    // (30% of a recent switch, less toward the own half) toward shadowing the opponent (near it:
    // its movement) or hunting it (further: a point 30% of the way from it to the goal).
    HD float ShadowOpponent(float ownHalf, Vec3 &autoDir, float &autoVel, Vec3 &autoLook) const {
        const int lookMs = 40;
        const PlayerImage oi = MentalPlayerImage(w, k, ctl.opponentPlayer);
        const Vec3 op = oi.position + oi.movement * 0.14f + oi.directionVector * 0.6f;
        const Vec3 oppToGoal = (Vec3(kPitchHalfLength * side, 0, 0) - op).Normalized(0);
        const float radius = 5.0f;
        const Vec3 front = op + (oppToGoal * radius * 0.7f);
        const float actionBias = 1.0f - Curve(NormalizedClamp((Pos() - front).Length(), 0.0f, radius), 0.7f);
        float bias;
        if (ExternalControllerActive(w, p)) bias = actionBias * 0.0f + GetLastSwitchBias(w, ctl) * 0.3f;
        else bias = actionBias * 0.0f;
        bias *= 1.0f - ownHalf;
        if (!(bias > 0.0f)) return bias;
        const float apart = (op - Pos()).Length();
        const float shadow = libm::powf(1.0f - Curve(NormalizedClamp(apart, 0.0f, 7.0f), 0.7f), 1.2f);
        const Vec3 shadowDir = oi.movement.Normalized(ctl.inputDirection);
        const float shadowVel = VelocityFloat(oi.velocity);
        const Vec3 shadowLook = (MentalBall(lookMs).Get2D() - Pos()).Normalized(0);
        const Vec3 huntMov = (op + oppToGoal * apart * 0.3f) - Pos();
        const Vec3 huntDir = huntMov.Normalized(ctl.inputDirection);
        const float huntVel = Clamp(huntMov.Length() * kDistanceToVelocity, kIdleVelocity, kSprintVelocity);
        const Vec3 huntLook = (MentalBall(lookMs).Get2D() - Pos()).Normalized(0);
        autoDir = (shadowDir * shadow + huntDir * (1.0f - shadow)).Normalized(ctl.inputDirection);
        autoVel = Clamp(shadowVel * shadow + huntVel * (1.0f - shadow), kIdleVelocity, kSprintVelocity);
        autoLook = ((shadowLook * shadow + huntLook * (1.0f - shadow))).Normalized(0);
        return bias;
    }
    // A movement command: the input (direction snapped to 8 directions with no bias, its speed)
    // blended with an automatic movement by its override: the ball control or chase of a player
    // going for the ball (a retainer keeps its input), or the shadowing of the opponent on the
    // ball. Below the idle-dribble switch the player faces where it looks.
    HDN void MovementCommand(bool forceMagnet, bool extraHaste) {
        ENG_SCOPE(40);
        Vec3 manualDir = ctl.inputDirection;
        QuantizeDirection(manualDir, kQuantizedDirectionBias);
        const float manualVel = ctl.inputVelocityFloat;
        Vec3 autoDir = manualDir, autoLook = InputLook(manualDir);
        float autoVel = manualVel, autoBias = 0.0f;
        ps.desiredTimeToBallMs = 0;
        const float ownHalf = NormalizedClamp(ctl.inputDirection.Dot(Vec3(side, 0, 0)), -1.0f, 1.0f);
        if (m.ballRetainer == p) {
            autoBias = 0.0f;
        } else if (GoesForBall(forceMagnet)) {
            Vec3 lookAt;
            if (ctl.hasBestPossession) {
                ps.desiredTimeToBallMs = (int)BallControlMovement(ctl.inputVelocityFloat, autoDir, autoVel, lookAt);
            } else {
                const float haste = (extraHaste || forceMagnet || ctl.possessionAmount < 1.1f) ? 1.0f : 0.0f;
                ps.desiredTimeToBallMs = (int)ToBallMovement(manualDir, ctl.inputVelocityFloat, autoDir, autoVel, lookAt, haste);
            }
            autoLook = (lookAt - Pos()).Normalized(0);
            autoBias = 1.0f;
            if (!ctl.hasBestPossession && m.designatedPossessionPlayer != p) autoBias = ChaseOverride(autoDir, manualDir, ownHalf, forceMagnet);
        } else if (w.playerTeamID[m.designatedPossessionPlayer] != teamID && Own().designatedTeamPossessionPlayer == p) {
            autoBias = ShadowOpponent(ownHalf, autoDir, autoVel, autoLook);
        }
        const Vec3 res = (manualDir * manualVel) * (1.0f - autoBias) + (autoDir * autoVel) * autoBias;
        PlayerCommand cmd = DefaultPlayerCommand();
        cmd.useDesiredMovement = true;
        cmd.useDesiredLookAt = true;
        cmd.desiredDirection = res.Normalized(manualDir);
        cmd.desiredVelocityFloat = Clamp(res.Length(), kIdleVelocity, kSprintVelocity);
        if (cmd.desiredVelocityFloat < kIdleDribbleSwitch) cmd.desiredDirection = autoLook;
        cmd.desiredLookAt = Pos() + autoLook * 10.0f;
        q.push_back(cmd);
    }

    // How lazy a player is, 0 to 1: by its distance from the opponents' designated player (lazy
    // from 20 m, fully at 65 m, both nearer when tired), half of it always and half by role (the
    // mindset, inverted as the team holds the ball).
    HD float Laziness() const {
        const float fresh = ps.base.fatigueFactorInverse;
        const float from = 20.0f * (fresh * 0.8f + 0.2f), to = 65.0f * (fresh * 0.5f + 0.5f);
        const float away = (Pos() - Pos(Opp().designatedTeamPossessionPlayer)).Length();
        const float holding = Clamp(ctl.fadingTeamPossessionAmount - 0.5f, 0.0f, 1.0f);
        const float mind = GetMindSet(DynamicRole());
        const float byRole = mind + holding * (1.0f - mind * 2.0f);
        return NormalizedClamp(away, from, to) * (0.5f + byRole * 0.5f);
    }
    // GRF's lazy velocity: a desired speed beyond a sprint counts a tenth of the excess; a lazy
    // player slows (not below dribbling when it asked for that) and, after running a lot in the
    // last 10 s (less with work rate), stays below a share of a sprint.
    HDN float GetLazyVelocity(float desiredVel) const {
        float v = desiredVel;
        if (v > kSprintVelocity) v = kSprintVelocity + (v - kSprintVelocity) * 0.1f;
        const float lazy = Laziness();
        float r = v * (1.0f - lazy);
        if (desiredVel >= kDribbleVelocity && r < kDribbleVelocity) r = kDribbleVelocity;
        float breath = 1.0f - NormalizedClamp(PlayerAverageVelocity(w, p, 10), kIdleVelocity, kSprintVelocity);
        breath = libm::powf(breath, 0.8f - Stat(kStatWorkRate) * 0.2f);
        breath = Clamp(breath * 1.2f, 0.0f, 1.0f);
        breath = breath * lazy + 1.0f * (1.0f - lazy);
        return MinF(r, kSprintVelocity * breath);
    }

    // ---- support positions: a force field around the formation place ----
    // How strongly opponents push a supporting player away: 0.3, times 2.2 for full and centre
    // backs, 2 for defensive midfielders, 1.6 for midfielders, 1.2 for attacking midfielders.
    HD float OpponentRepelWeight() const {
        float weight = 0.3f * 1.0f;
        switch (DynamicRole()) {
            case kRoleCentreBack:
            case kRoleLeftBack:
            case kRoleRightBack: weight *= 2.2f; break;
            case kRoleDefensiveMid: weight *= 2.0f; break;
            case kRoleCentralMid:
            case kRoleLeftMid:
            case kRoleRightMid: weight *= 1.6f; break;
            case kRoleAttackingMid: weight *= 1.2f; break;
            case kRoleCentreForward: weight *= 1.0f; break;
            default: break;
        }
        return weight;
    }
    // The anchor: the formation place moved upfield, 3.6 to 12 m by mindset for the forward
    // support player, else up to 22 m (to the 1.5 of the mindset) the nearer the player is to
    // the lane 8 m across from the carrier; pulling harder the further the player is from it.
    HD ForceSpot SupportAnchor(const Vec3 &base, float mind, const Vec3 &cur, const Vec3 &carrier) const {
        ForceSpot s;
        s.origin = base;
        if (p == AI().forwardSupportPlayer) {
            s.origin.v[0] += -side * (0.3f + 0.7f * mind) * 12.0f;
        } else {
            float amount = 22.0f;
            const float laneY = -SignSide(carrier.v[1]) * 8.0f;
            amount *= Curve(1.0f - NormalizedClamp(fabsf(laneY - cur.v[1]), 0.0f, 30.0f), 1.0f);
            s.origin.v[0] += -side * libm::powf(mind, 1.5f) * amount;
        }
        s.power = 1.0f * 0.7f;
        s.power *= 0.3f + 0.7f * NormalizedClamp((s.origin - cur).Length(), 0.0f, 20.0f);
        return s;
    }
    // GRF's support position (the forces in GRF's order): the anchor; a run toward the opponents'
    // goal line; the 3 opponents nearest a point near the carrier pushing away (from 2 m beyond
    // them, away from the carrier; softer and wider on a run); with the ball well held, the 6
    // nearest teammates; with it held better still, the ball's path 200 to 650 ms ahead; and for
    // players other than the carrier, a flock ring around it (attract to 21 m, repel within 12 m).
    // The result stays onside (8 cm) and on the pitch.
    HDN Vec3 GetSupportPositionForceField(const Vec3 &base, bool makeRun) const {
        ENG_SCOPE(41);
        const int designated = Own().designatedTeamPossessionPlayer;
        const Vec3 cur = Pos() + Mov() * 0.1f;
        const Vec3 carrier = Pos(designated) + Mov(designated) * 0.1f;
        const float mind = GetMindSet(DynamicRole());
        const float opponentWeight = OpponentRepelWeight(), mateWeight = 0.4f * 1.0f, ballWeight = 1.0f * 1.0f,
                    runWeight = 1.0f * 1.0f, flockWeight = 0.45f * 1.0f, webScale = 0.75f;
        const float offsideX = GetOffsideLine(w, k, oppID, 240);
        ForceField &ff = c.ws->forceField;
        ff.clear();
        ff.push_back(SupportAnchor(base, mind, cur, carrier));
        if (makeRun) ff.push_back(MakeSpot(Vec3(-side * kPitchHalfLength, cur.v[1] * 0.5f, 0.0f), kAttract, kDecayConstant, 2.0f * runWeight));
        // GRF adds 0.7 to every coordinate of the focus here.
        const PlayerList opponents = GetClosestPlayers(w, c, oppID, carrier * 0.3f + cur + 0.7f, false, 3);
        for (int i = 0; i < opponents.count; i++) {
            const PlayerImage oi = MentalPlayerImage(w, k, opponents[i]);
            const Vec3 at = oi.position + oi.movement * 0.1f;
            ForceSpot s = MakeSpot(at + (at - carrier).Normalized(0) * 2.0f, kRepel, kDecayVariable, 1.0f * opponentWeight, 5.0f, 0.7f);
            if (makeRun) {
                s.scale = 2.0f;
                s.power *= 0.5f;
            }
            ff.push_back(s);
        }
        if (Own().fadingTeamPossessionAmount >= 1.02f) {
            const PlayerList mates = GetClosestPlayers(w, c, teamID, cur, false, 6);
            for (int i = 0; i < mates.count; i++) {
                if (mates[i] == p) continue;
                const PlayerImage mi = MentalPlayerImage(w, k, mates[i]);
                ff.push_back(MakeSpot(mi.position + mi.movement * 0.1f, kRepel, kDecayVariable, 1.0f * mateWeight, 14.0f * webScale, 1.0f));
            }
        }
        if (p != designated && Own().fadingTeamPossessionAmount >= 1.06f) {
            const int times[4] = {200, 350, 500, 650};
            for (int i = 0; i < 4; i++)
                ff.push_back(MakeSpot(MentalBall(times[i]).Get2D(), kRepel, kDecayVariable, 1.0f * ballWeight, 2.0f, 0.5f));
        }
        if (p != designated) {
            ff.push_back(MakeSpot(carrier, kAttract, kDecayVariable, 1.0f * flockWeight, 28.0f * webScale, 1.0f));
            ff.push_back(MakeSpot(carrier, kRepel, kDecayVariable, 1.0f * flockWeight, 16.0f * webScale, 1.0f));
        }
        Vec3 r = cur + GetForceFieldMovement(ff, cur, 7);
        const float margin = 0.08f;
        if (r.v[0] * -side > (offsideX * -side) - margin) r.v[0] = offsideX - (margin * -side);
        r.v[0] = Clamp(r.v[0], -kPitchHalfLength, kPitchHalfLength);
        r.v[1] = Clamp(r.v[1], -kPitchHalfWidth, kPitchHalfWidth);
        return r;
    }

    // The field strategy of each line (defence, midfield, attack): how much of the static
    // formation place a player far from the ball keeps, the range of fading possession over
    // which it moves to support, above which share of support it may make a run, and the base of
    // its defensive pull.
    enum StrategyKind { kDefense, kMidfield, kOffense };
    struct LineStrategy {
        float staticShare, attackLow, attackHigh, runThreshold, defensiveBase;
    };
    HD static LineStrategy LineStrategyOf(int kind) {
        switch (kind) {
            case kDefense: return {1.0f, 0.2f, 0.9f, 0.0f, 1.9f};
            case kMidfield: return {0.9f, 0.1f, 0.7f, 0.9f, 1.5f};
            default: return {0.8f, 0.1f, 0.6f, 0.7f, 1.3f};
        }
    }
    // Where a player of a line goes: its static formation place blended into its dynamic one as
    // the match's designated player comes within 15 to 20 m; moved toward its support position as
    // the team holds the ball (a run when it is the team's runner); pulled to defend its man by
    // the line's base less its mindset and the possession; inside the offside trap except for
    // attackers. Its speed is the distance at the AI's distance-to-velocity rate, made lazy.
    HDN void FieldStrategyRequestInput(int kind, Vec3 &dir, float &vel) const {
        const LineStrategy line = LineStrategyOf(kind);
        const FormationHistory history = FormationHistoryOf(w, p);
        const Vec3 fixed = TeamAdaptedFormationPosition(w, c, p, false, history);
        const Vec3 dynamic = TeamAdaptedFormationPosition(w, c, p, true, history);
        const float far = NormalizedClamp(GetDistance(Pos(), Pos(m.designatedPossessionPlayer)), 15.0f, 20.0f);
        const float keep = Curve(line.staticShare * far, 1.0f);
        Vec3 desired = fixed * keep + dynamic * (1.0f - keep);
        const float attack = NormalizedClamp((ctl.fadingTeamPossessionAmount - 0.5f) * 1.0f, line.attackLow, line.attackHigh);
        const bool run = kind != kDefense && attack > line.runThreshold && AI().endApplyAttackingRunMs > m.actualTimeMs &&
                         AI().attackingRunPlayer == p;
        desired = desired * (1.0f - attack) + GetSupportPositionForceField(desired, run) * attack;
        const float mind = GetMindSet(DynamicRole());
        AddDefensiveComponent(desired, libm::powf(Clamp(line.defensiveBase - mind - ctl.fadingTeamPossessionAmount, 0.0f, 1.0f), 0.7f));
        if (kind != kOffense) TeamApplyOffsideTrap(w, teamID, desired);
        dir = (desired - Pos()).Normalized(Dir());
        vel = Clamp(GetLazyVelocity((desired - Pos()).Length() * kDistanceToVelocity), 0, kSprintVelocity);
    }

    // Whether the ball is bound for the keeper's goal, kept in the controller with where it will
    // cross the goal line: the ball 4 s ahead is beyond the goal line, the keeper is within 32 m
    // of the ball 250 ms ahead, and the ball's path (now to 800 ms ahead) crosses the goal line
    // within 3.7 m of the centre, widened by the keeper's panic (1.02, up to 1.52 as its
    // defensive positioning and vision fall).
    HDN bool BallBoundForGoal() {
        const float panic = 1.02f + (1.0f - (Stat(kStatDefensivePositioning) * 0.6f + Stat(kStatVision) * 0.4f)) * 0.5f;
        bool bound = false;
        float crossY = 0;
        if (MentalBall(4000).v[0] * side > kPitchHalfLength && (Pos() - MentalBall(250)).Length() < 32.0f) {
            const Line path(MentalBall(0).Get2D(), MentalBall(800).Get2D());
            const Line goalLine(Vec3(kPitchHalfLength * side, -kPitchHalfWidth, 0), Vec3(kPitchHalfLength * side, kPitchHalfWidth, 0));
            const float y = path.IntersectionPoint(goalLine).Get2D().v[1];
            bound = !((double)fabsf(y) > 3.7 * (double)panic);
            if (bound) crossY = y;
        }
        eliza->ballBoundForGoal = bound;
        eliza->ballBoundForGoalY = crossY;
        return bound;
    }

    // How far an opponent is from a shot, scaled down close to goal.
    HD float ToThreshold(const Vec3 &goal, const Vec3 &from, float threshold) const {
        float d = (goal - from).Length();
        return Clamp(d - threshold * NormalizedClamp(d, 0.0f, threshold * 2.0f), 0.0f, kPitchHalfLength);
    }
    // How far the keeper comes off its line, 0 to 1: 30% with the ball well held (fading
    // possession 1 to 1.5); without it, all the way when the opponent on the ball will reach its
    // shooting point (20 m out, less near goal) before any teammate reaches it, unless a second
    // attacker's shooting point (24 m) is as badly covered. `path` starts where the attack comes
    // from (the opponent 0.32 s ahead, blended with the ball).
    HD float KeeperRush(const Vec3 &ball, const Vec3 &goal, Line &path) const {
        float rush = 0.3f;
        rush *= NormalizedClamp(ctl.fadingTeamPossessionAmount, 1.0f, 1.5f);
        if (!(ctl.fadingTeamPossessionAmount < 1.0f)) return rush;
        const int o = Opp().designatedTeamPossessionPlayer;
        const Vec3 op = Pos(o) + Mov(o) * 0.32f;
        if (m.players[o].hasPossession == false) path.pts[0] = op * 0.6f + ball * 0.4f;
        else path.pts[0] = op * 0.4f + ball * 0.6f;
        const float oppThreshold = ToThreshold(goal, op, 20.0f);
        const Vec3 shootingPoint = op + (goal - op).Normalized(0) * oppThreshold;
        const int mate = GetClosestPlayer(w, c, teamID, shootingPoint, false, p);
        float mateThreshold = 99999;
        if (mate >= 0) mateThreshold = (shootingPoint - (Pos(mate) + Mov(mate) * 0.24f)).Length();
        if (!(mateThreshold > oppThreshold + 1.0f)) return rush;
        const int helper = GetClosestPlayer(w, c, oppID, goal, false, o);
        if (helper < 0) return 1.0f;
        const Vec3 hp = Pos(helper) + Mov(helper) * 0.32f;
        const float helperThreshold = ToThreshold(goal, hp, 24.0f);
        const Vec3 helperPoint = hp + (goal - hp).Normalized(0) * helperThreshold;
        const int mateHelper = GetClosestPlayer(w, c, teamID, helperPoint, false, p);
        float mateHelperThreshold = 99999;
        if (mateHelper >= 0) mateHelperThreshold = (helperPoint - (Pos(mateHelper) + Mov(mateHelper) * 0.24f)).Length();
        float second = 0.0f;
        if (mateHelperThreshold > helperThreshold) second = NormalizedClamp(mateHelperThreshold - helperThreshold, 0.0f, 2.0f);
        float ratio = 1.0f - NormalizedClamp(helperThreshold / (oppThreshold + 0.0001f), 1.0f, 1.5f);
        ratio *= 0.7f;
        return Clamp(1.0f - (second * ratio), 0.0f, 1.0f);
    }
    // The keeper covering its goal from a ball in its half: on the bisector of the angle the posts
    // make from the ball (met 0.7 m inside the goal line, within the posts), out from there by
    // the rush (at least 0.7 m) toward where the attack comes from; walking once in front of its
    // target near that line.
    HD Vec3 KeeperCover(const Vec3 &ball, const Vec3 &goal, float &maxVel) const {
        const Vec3 post1 = Vec3(kPitchHalfLength * side, 3.7f, 0) - ball;
        const Vec3 post2 = Vec3(kPitchHalfLength * side, -3.7f, 0) - ball;
        const Vec3 middle = post1.Rotated2D(post2.Angle2D(post1) * 0.5f).Normalized(Vec3(side, 0, 0));
        Line path(ball, ball + middle);
        const Line inside(Vec3((kPitchHalfLength - 0.7f) * side, -kPitchHalfWidth, 0), Vec3((kPitchHalfLength - 0.7f) * side, kPitchHalfWidth, 0));
        Vec3 onLine = path.IntersectionPoint(inside).Get2D();
        onLine.v[1] = Clamp(onLine.v[1], -3.7f, 3.7f);
        path.pts[1] = onLine;
        float rush = KeeperRush(ball, goal, path);
        if (AI().endApplyKeeperRushMs > m.actualTimeMs) rush = 1.0f;
        const float out = Clamp(MaxF(path.Length() - 0.5f, 0.0f) * rush, 0.7f, kPitchHalfLength);
        Vec3 target = path.pts[1] + (path.pts[0] - path.pts[1]).Normalized(0) * out;
        float along = 0.0f;
        const float fromPath = path.DistanceToPoint(Pos(), along);
        if ((target - goal).Length() < (Pos() - goal).Length() && fromPath < 1.0f && along > 0.0f) maxVel = kWalkVelocity;
        target.v[0] = Clamp(target.v[0], -kPitchHalfLength + 0.2f, kPitchHalfLength - 0.2f);
        return target;
    }
    // The keeper against a ball bound for goal: onto the ball's line to where it crosses the goal
    // line (0.4 m short), at the point nearest the keeper; at the crossing itself when the ball
    // will pass the keeper above 2.5 m.
    HD Vec3 KeeperSave() const {
        Line path;
        path.pts[0] = MentalBall(10).Get2D();
        Vec3 crossing = Vec3(kPitchHalfLength * side, eliza->ballBoundForGoalY, 0);
        crossing += (path.pts[0] - crossing).Normalized(0) * 0.4f;
        path.pts[1] = crossing;
        float keeperAt = 0.0f;
        path.DistanceToPoint(Pos() + Mov() * 0.05f, keeperAt);
        float secondAt = 0.0f;
        path.DistanceToPoint(MentalBall(1010).Get2D(), secondAt);
        if ((double)secondAt > 1e-4 && (double)MentalBall(TruncToInt32(10 + 1000 * (keeperAt / secondAt))).v[2] > 2.5) return crossing;
        keeperAt = Clamp(keeperAt, 0.0f, 1.0f);
        Vec3 target = path.pts[0] + (path.pts[1] - path.pts[0]) * keeperAt;
        target.v[2] = 0.0f;
        target.v[0] = Clamp(target.v[0], -kPitchHalfLength + 0.2f, kPitchHalfLength - 0.2f);
        return target;
    }
    // The goalkeeper's movement: 10 m off its goal line by default; with the ball (600 ms plus a
    // fifth of its time to it ahead) in its half, covering the goal or saving a ball bound for it.
    HDN void GoalieRequestInput(Vec3 &dir, float &vel) {
        ENG_SCOPE(46);
        const Vec3 ball = MentalBall(TruncToInt32(600 + (float)ps.timeToBallMs * 0.2f)).Get2D();
        const Vec3 goal = Vec3(kPitchHalfLength * side, 0, 0);
        Vec3 target = Vec3((kPitchHalfLength - 10.0f) * side, 0, 0);
        float maxVel = kSprintVelocity;
        if (ball.v[0] * side > 0) {
            target = BallBoundForGoal() ? KeeperSave() : KeeperCover(ball, goal, maxVel);
        }
        dir = target - Pos();
        vel = Clamp(dir.Length() * kDistanceToVelocity, kIdleVelocity, maxVel);
        dir.Normalize(Dir());
    }

    // ---- passes ----
    // How much an opponent (0.2 s ahead) threatens a ball on its way from `origin` to `target`,
    // 0 to 1: the seconds the ball needs to reach the opponent's point of the line (0.7 s plus
    // 0.03 times the distance to that point times its fraction of the way, 2.5 s more past the
    // middle of a high pass; divided by the ball-speed factor) against the seconds the opponent
    // needs to reach the line at a sprint, with half a second of slack. Opponents behind the
    // passer or 20% past the target do not count, nor those under a high pass's flight (20% to
    // 65% of the way).
    HD float InterceptThreat(const Vec3 &origin, const Vec3 &target, const Line &line, int passType, const PlayerImagePos &opp,
                             float ballVelMul) const {
        const float secondScale = 1.0f;
        const Vec3 at = opp.position + opp.movement * 0.2f;
        float along = 0.0f;
        const float away = line.DistanceToPoint(at, along);
        if (!(along >= 0.0f && along <= 1.0f + 0.2f)) return 0.0f;
        if (passType == kFnHighPass && !(along < 0.2f || along > 0.65f)) return 0.0f;
        const float onLine = Clamp(along, 0.0f, 1.0f);
        const Vec3 meet = origin * (1.0f - onLine) + target * onLine;
        const float opponentSeconds = (away + 1.0f) / kSprintVelocity;
        const float lofted = (passType == kFnHighPass && along > 0.5f) ? 2.5f : 0.0f;
        float ballSeconds = 0.7f + (meet - origin).Length() * along * 0.03f + lofted;
        ballSeconds *= 1.0f / ballVelMul;
        return Clamp(ballSeconds - opponentSeconds + (secondScale * 0.5f), 0.0f, secondScale);
    }
    // The odds of a pass (or, with a ball-speed factor, a shot) to `target` from 0.12 s ahead:
    // 1 less the summed threats (a high pass starts at 0.4), clamped.
    HDN float PassingOdds(const Vec3 &target, int passType, const ImageList &opps, float ballVelMul = 1.0f) const {
        ENG_SCOPE(42);
        const float secondScale = 1.0f;
        const Vec3 origin = Pos() + Mov() * 0.12f;
        const Line line(origin, target);
        float danger = 0.0f;
        for (int i = 0; i < opps.count; i++) danger += InterceptThreat(origin, target, line, passType, opps[i], ballVelMul);
        if (passType == kFnHighPass) danger += 0.4f;
        danger = NormalizedClamp(danger, 0.0f, secondScale);
        return 1.0f - danger;
    }
    // The odds of a pass to teammate `target` where it will be (0.7 s plus 3% a metre ahead, at
    // most half a second; a long pass 20% further upfield); no high pass under 10 m.
    HDN float PassingOddsTo(int target, int passType, const ImageList &opps) const {
        const float d = (Pos(target) - Pos()).Length();
        if (passType == kFnHighPass && d < 10.0f) return 0.0f;
        Vec3 at = Pos(target) + Mov(target) * Clamp(0.7f + d * 0.03f, 0.0f, 0.5f);
        if (passType == kFnLongPass) at += Vec3(-side * d * 0.2f, 0, 0);
        return PassingOdds(at, passType, opps);
    }
    // A fully automatic pass of `passType` to teammate `target`.
    HDN void AddPass(int target, int passType) {
        PlayerCommand cmd = DefaultPlayerCommand();
        cmd.desiredFunctionType = passType;
        TouchInformation &t = cmd.touchInfo;
        t.targetPlayer = -1;
        t.forcedTargetPlayer = target;
        t.inputDirection = Vec3(0);
        t.inputPower = 0;
        t.autoDirectionBias = 1.0f;
        t.autoPowerBias = 1.0f;
        AimPass(w, p, passType, t.inputDirection, t.inputPower, t.autoDirectionBias, t.autoPowerBias, t.desiredDirection,
                t.desiredPower, t.targetPlayer, t.forcedTargetPlayer);
        q.push_back(cmd);
    }
    // A panic clearance away from the own goal: the facing direction (its x squeezed to 80%)
    // turned upfield and toward the touchline it faces, lifted 0.3; offered as a high pass (power
    // 0.7), a shot (0.6) and a long pass (0.8), fully manual.
    HDN void AddPanicPass() {
        const int flank = SignSide(Dir().v[1]);
        Vec3 away = ((Dir() * Vec3(0.8f, 1.0f, 0.0f)).Normalized() + Vec3(-side * 0.7f, flank * 0.5f, 0)).Normalized(0) + Vec3(0, 0, 0.3f);
        away.Normalize(Dir());
        PlayerCommand cmd = DefaultPlayerCommand();
        cmd.touchInfo.inputDirection = away;
        cmd.touchInfo.desiredDirection = away;
        cmd.touchInfo.autoDirectionBias = 0.0f;
        cmd.touchInfo.autoPowerBias = 0.0f;
        const struct {
            int type;
            float power;
        } clearances[3] = {{kFnHighPass, 0.7f}, {kFnShot, 0.6f}, {kFnLongPass, 0.8f}};
        for (const auto &option : clearances) {
            cmd.desiredFunctionType = option.type;
            cmd.touchInfo.inputPower = option.power;
            cmd.touchInfo.desiredPower = option.power;
            q.push_back(cmd);
        }
    }
    // The dribble: a force field around where the player will be in 0.25 s, pushed by the 5
    // nearest opponents (0.25 s ahead, within 10 m), the near touchline and goal line (5 m beyond
    // them, within 20 m), and pulled to the opponents' goal (its y following the player's, less
    // near the goal line and by the center magnet) by the offensiveness (0.7 plus small shares of
    // the dribble setting and the mindset). The speed is the pull at the AI's rate, snapped to a
    // velocity category.
    HDN void BestDribbleMovement(Vec3 &desiredDir, float &desiredVel) const {
        ENG_SCOPE(43);
        const Vec3 at = Pos(), mov = Mov();
        const float offense = 0.7f + kDribbleOffensiveness * 0.05f + GetMindSet(DynamicRole()) * 0.05f;
        const float powerMul = 1.0f, futureS = 0.25f;
        const PlayerList opponents = GetClosestPlayers(w, c, oppID, at, false, 5);
        ForceField &ff = c.ws->forceField;
        ff.clear();
        const float nearGoalLine = NormalizedClamp(fabsf(at.v[0]) / kPitchHalfLength, 0.0f, 1.0f);
        float central = 1.0f - nearGoalLine * nearGoalLine;
        central *= 0.5f;
        const Vec3 goal = Vec3(-side * kPitchHalfLength, at.v[1] * (1.0f - kDribbleCenterMagnet) * central, 0);
        for (int i = 0; i < opponents.count; i++) {
            const PlayerImage oi = MentalPlayerImage(w, k, opponents[i]);
            ff.push_back(MakeSpot(oi.position + oi.movement * futureS, kRepel, kDecayVariable, 2.0f * powerMul, 10.0f, 1.0f));
        }
        ff.push_back(MakeSpot(Vec3(at.v[0], (kPitchHalfWidth + 5.0f) * SignSide(at.v[1]), 0), kRepel, kDecayVariable, 4.0f * powerMul, 20.0f, 0.7f));
        ff.push_back(MakeSpot(Vec3((kPitchHalfLength + 5.0f) * SignSide(at.v[0]), at.v[1], 0), kRepel, kDecayVariable, 4.0f * powerMul, 20.0f, 0.7f));
        ff.push_back(MakeSpot(goal, kAttract, kDecayConstant, offense * powerMul));
        const Vec3 pull = GetForceFieldMovement(ff, at + mov * futureS, 1.0f);
        desiredDir = pull.Normalized(Dir());
        desiredVel = RangeVelocity(Clamp(pull.Length() * kDistanceToVelocity, kIdleVelocity, kSprintVelocity));
    }
};

}  // namespace eng
