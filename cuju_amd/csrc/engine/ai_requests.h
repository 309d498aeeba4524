// SPDX-License-Identifier: Apache-2.0
// Restates game logic of cuju (Copyright 2026 The cuju Authors), a reimplementation of Google
// Research Football (Copyright 2019 Google LLC); see NOTICE.
// The player AI, second half: decisions on the ball, celebrations, set pieces, the command queue of
// a player without a gamer and of a gamer's player.
// Semantics: include/cuju/simulation/ai_controller.h:1620-2494.
#pragma once

#include "ai_moves.h"

namespace eng {

struct AIController : AIBase {
    using AIBase::AIBase;

    HD float Random(float lo, float hi) { return RandomInRange(w, lo, hi); }

    HD float TacticalRating(const Player &pl, float fsw, float sw, float fw, float total) const {
        const auto &t = pl.tactical;
        return (t.forwardSpaceRating * fsw + t.spaceRating * sw + t.forwardRating * fw) / total;
    }

    // The weights of the tactical rating a player on the ball compares with its teammates':
    // forward space 0.4, space 0.3 and forwardness 2 to 8 by the role's mindset.
    struct PassWeights {
        float forwardSpace, space, forward, total;
    };
    HD PassWeights PassWeightsOf(float mind) const {
        PassWeights pw;
        pw.forwardSpace = 0.4f;
        pw.space = 0.3f;
        pw.forward = 2.0f + mind * 6.0f;
        pw.total = pw.forwardSpace + pw.space + pw.forward;
        return pw;
    }
    // The teammate best worth a pass and the pass's type: one rated better than the passer (by 6%
    // less the mindset's share; a goalkeeper at 70%), by the rating gain (weighted 1 to 11 by the
    // mindset) and the best odds of a short, long or high pass, less how hard a one-touch pass is;
    // above a threshold and minimum odds that fall as possession lasts. -1 for none.
    HD int BestPassTarget(float mind, const ImageList &opps, float oneTouchIsHard, float longPossession, int &passType,
                          float &passOdds) const {
        const PassWeights pw = PassWeightsOf(mind);
        const float improvement = 0.06f * (1.0f - mind);
        const float gainWeight = 1.0f + (mind * mind) * 10.0f, oddsWeight = 1.0f;
        const float minimum = 0.2f * (1.0f - mind) - longPossession * 0.1f;
        const float threshold = 0.1f - longPossession * 0.05f;
        const float own = TacticalRating(ps, pw.forwardSpace, pw.space, pw.forward, pw.total);
        const PlayerList mates = TeamActivePlayers(w, teamID);
        float bestTotal = 0.0f;
        int best = -1;
        passType = kFnShortPass;
        passOdds = 0.0f;
        for (int i = 0; i < mates.count; i++) {
            const int mate = mates[i];
            if (mate == p) continue;
            float rating = TacticalRating(m.players[mate], pw.forwardSpace, pw.space, pw.forward, pw.total);
            if (StaticRole(mate) == kRoleGoalkeeper) rating *= 0.7f;
            if (!(rating > own + improvement)) continue;
            const float shortOdds = PassingOddsTo(mate, kFnShortPass, opps);
            const float longOdds = PassingOddsTo(mate, kFnLongPass, opps);
            const float highOdds = PassingOddsTo(mate, kFnHighPass, opps);
            float odds = highOdds;
            int type = kFnHighPass;
            if (shortOdds >= longOdds && shortOdds >= highOdds) {
                odds = shortOdds;
                type = kFnShortPass;
            } else if (longOdds >= highOdds) {
                odds = longOdds;
                type = kFnLongPass;
            }
            float total = (rating - own) * gainWeight + odds * oddsWeight - oneTouchIsHard;
            total /= gainWeight + oddsWeight;
            if (total > bestTotal && total > threshold && odds > minimum) {
                bestTotal = total;
                best = mate;
                passOdds = odds;
                passType = type;
            }
        }
        return best;
    }
    // A defensive player (mindset below 0.25) near its own goal (2 to 16 m) clears in a panic when
    // no pass is good enough for the danger and its possession is shaky; a goalkeeper clears when
    // its possession is below 3.
    HD void ConsiderClearance(float mind, int bestPlayer, float bestOdds) {
        if (!(mind < 0.25f)) return;
        const float panic = 1.0f - mind * 2.0f;
        const float nearGoal = 1.0f - NormalizedClamp((Pos() - Vec3(kPitchHalfLength * side, 0, 0)).Length(), 2.0f, 16.0f);
        if (DynamicRole() != kRoleGoalkeeper) {
            if ((bestPlayer < 0 || bestOdds < panic * nearGoal) && ctl.possessionAmount < 0.9f + panic * nearGoal * 0.8f) AddPanicPass();
        } else if (ctl.possessionAmount < 3.0f) {
            AddPanicPass();
        }
    }
    // Near the ideal shooting spot (7 m out, within 16 m) the player shoots at the best of the
    // goal's centre and the posts' insides (odds to the 0.5) when they and a draw of up to 0.5
    // pass 0.5: at that point, scattered by a draw (less with the shot statistic), leaning 30%
    // against its running direction by speed, with a drawn power (stronger further out).
    HD void ConsiderShot(const ImageList &opps, float rawVel) {
        const float goalDistance = NormalizedClamp((Vec3(kPitchHalfLength * -side, 0, 0) - Pos()).Length(), 0.0f, 32.0f);
        const float ideal = Curve(1.0f - NormalizedClamp((Vec3((kPitchHalfLength - 7.0f) * -side, 0, 0) - Pos()).Length(), 0.0f, 16.0f), 1.0f);
        if (!(ideal > 0.1f)) return;
        const float gx = (kPitchHalfLength + 1.0f) * -side;
        const float low = PassingOdds(Vec3(gx, -3.6f, 0), kFnShot, opps, 3.0f);
        const float center = PassingOdds(Vec3(gx, 0.0f, 0), kFnShot, opps, 3.0f);
        const float high = PassingOdds(Vec3(gx, 3.6f, 0), kFnShot, opps, 3.0f);
        float odds = center, y = 0.0f;
        if (low > odds) {
            odds = low;
            y = -3.5f;
        }
        if (high > odds) {
            odds = high;
            y = 3.5f;
        }
        if (!(libm::powf(odds, 0.5f) + Random(0.0f, 0.5f) > 0.5f)) return;
        PlayerCommand cmd = DefaultPlayerCommand();
        cmd.desiredFunctionType = kFnShot;
        cmd.desiredVelocityFloat = rawVel;
        const float shot = Stat(kStatShot);
        const float aimY = y + Random(-1.0f + shot, 1.0f - shot);
        TouchInformation &t = cmd.touchInfo;
        t.desiredDirection = (Vec3(gx, aimY, 0) - (Pos() + Mov() * 0.2f)).Normalized(Vec3(-side, 0, 0));
        t.desiredDirection = (t.desiredDirection * 0.7f + -Dir() * (FloatVelocity() / kSprintVelocity) * 0.3f).Normalized();
        t.autoDirectionBias = 1.0f;
        t.desiredPower = Random(0.7f * (0.6f + goalDistance * 0.4f), 1.0f * (0.6f + goalDistance * 0.4f));
        q.push_back(cmd);
    }
    // The commands of a player on the ball: a panic clearance, a pass to the best-placed teammate,
    // a shot, and a dribble direction from a force field.
    HDN void GetOnTheBallCommands(Vec3 &rawDir, float &rawVel) {
        ENG_SCOPE(44);
        const float ballGap = NormalizedClamp((m.ball.momentum - Mov()).Length(), 0.0f, 10.0f);
        const float oneTouchIsHard = ballGap - Stat(kStatShortPass) * ballGap * 0.8f;
        ImageList opps;
        MentalTeamPlayerImages(w, k, oppID, opps);
        const float held = NormalizedClamp((float)ps.possessionDurationMs, 0, 5000);
        const float mind = GetMindSet(DynamicRole());
        int passType = kFnShortPass;
        float passOdds = 0.0f;
        const int target = BestPassTarget(mind, opps, oneTouchIsHard, held * held, passType, passOdds);
        ConsiderClearance(mind, target, passOdds);
        if (target >= 0) AddPass(target, passType);
        ConsiderShot(opps, rawVel);
        BestDribbleMovement(rawDir, rawVel);
    }

    // ---- celebrations ----
    // After a goal the scoring team runs to the corner on the ball's end and the scorer's flank
    // (a quarter of the distance per second), the scorer sprinting, teammates within 20 m
    // joining the scorer (half the distance per second) and looking its way; the conceding team
    // stands (type 2). Two to four seconds after play stopped each plays its celebration.
    struct Celebration {
        Vec3 dir, look;
        float vel;
        int type, scorer;  // type 1 scored, 2 conceded; scorer 2 for the scorer itself
    };
    HD Celebration CelebrationOf() const {
        const int xSide = (BallAt(0).Get2D().v[0] > 0) ? 1 : -1;
        const int last = Own().lastTouchPlayer;
        const int ySide = last >= 0 ? ((Pos(last).v[1] > 0) ? 1 : -1) : side;
        const Vec3 corner = Vec3(kPitchHalfLength * xSide, kPitchHalfWidth * ySide, 0);
        Celebration c{(corner - Pos()).Normalized(), Pos() + Dir() * 1000, ClampVelocity((corner - Pos()).Length() / 4.0f), 1, 1};
        if (m.lastGoalTeam != TeamSlot(w, teamID)) {
            c.type = 2;
            c.vel = kIdleVelocity;
            return c;
        }
        if (last == p) {
            c.scorer = 2;
            c.vel = kSprintVelocity;
        } else if (last >= 0) {
            const Vec3 at = Pos(last);
            if ((at - Pos()).Length() < 20) {
                c.dir = ((at * 0.5f + at * 0.5f) - Pos()).Normalized();
                c.vel = ClampVelocity((float)((double)(at - Pos()).Length() / 2.0));
            } else {
                c.vel = kIdleVelocity;
            }
            c.look = Pos() + Dir(last) * 100;
        }
        return c;
    }
    HDN void AddCelebration() {
        const Celebration c = CelebrationOf();
        const uint64_t stop = m.referee.buffer.stopTime;
        if (m.actualTimeMs - stop > 2000 && m.actualTimeMs - stop < 4000) {
            PlayerCommand cmd = DefaultPlayerCommand();
            cmd.desiredFunctionType = kFnSpecial;
            cmd.useSpecialVar1 = true;
            cmd.specialVar1 = c.type;
            cmd.useSpecialVar2 = true;
            cmd.specialVar2 = c.scorer;
            q.push_back(cmd);
        }
        PlayerCommand cmd = DefaultPlayerCommand();
        cmd.useDesiredMovement = true;
        cmd.desiredDirection = c.dir;
        cmd.desiredVelocityFloat = c.vel;
        cmd.useDesiredLookAt = true;
        cmd.desiredLookAt = c.look;
        q.push_back(cmd);
    }

    // ---- restarts ----
    // The penalty taker shoots at a drawn point up to 5 m from the goal's centre with a drawn
    // power. Returns the shot's direction.
    HD Vec3 PenaltyShot() {
        PlayerCommand action = DefaultPlayerCommand();
        action.desiredFunctionType = kFnShot;
        TouchInformation &t = action.touchInfo;
        const float y = Random(-5, 5);
        t.desiredDirection = (Vec3(-side * kPitchHalfLength, y, 0) - Pos()).Normalized(Vec3(-side, 0, 0));
        t.desiredPower = Random(0.4f, 1.0f);
        q.push_back(action);
        return t.desiredDirection;
    }
    // Where a restart's pass goes, by draws: a goal kick, 60% of the time without gamers, lofted
    // 20% upfield across the pitch, else short to the taker's x; a kick-off a metre ahead; a free
    // kick, half the time, lofted into the box, else 10 m upfield; a corner, 70% of the time,
    // lofted to the far post area (1% to 13% out, GRF's draws y first), else to 80% upfield; a
    // throw-in at the taker; a goalkeeper holding the ball lofts it upfield to a teammate who has
    // 10 m of space (or after 4 s), or waits. Returns false when the keeper waits.
    HD bool RestartPassTarget(int type, PlayerCommand &action, Vec3 &target) {
        TouchInformation &t = action.touchInfo;
        switch (type) {
            case kModeGoalKick:
                if (Random(0.0f, 1.0f) > 0.4f && HumanGamerCount(Own()) == 0) {
                    action.desiredFunctionType = kFnHighPass;
                    target = Vec3((kPitchHalfLength * -side) * 0.2f, Random(-kPitchHalfWidth, kPitchHalfWidth), 0.0f);
                } else {
                    target = Vec3(Pos().v[0] * 0.9f, Random(-kPitchHalfWidth, kPitchHalfWidth), 0.0f);
                }
                return true;
            case kModeKickOff:
                target = Pos() + Dir() * 1.0f;
                return true;
            case kModeFreeKick:
                if (Random(0.0f, 1.0f) > 0.5f) {
                    action.desiredFunctionType = kFnHighPass;
                    target = Vec3(kPitchHalfLength * -side, Random(-10.0f, 10.0f), 0.0f);
                } else {
                    const float y = Random(-10.0f, 10.0f);
                    target = Pos() + Vec3(-side * 10.0f, y, 0.0f);
                }
                return true;
            case kModeCorner:
                if (Random(0.0f, 1.0f) > 0.3f) {
                    action.desiredFunctionType = kFnHighPass;
                    const float y = Random(-10.0f, 10.0f);
                    const float x = Random(0.0f, 0.12f);
                    target = Vec3((kPitchHalfLength * -side) * (0.99f - x), y, 0.0f);
                } else {
                    target = Vec3((kPitchHalfLength * -side) * 0.8f, Pos().v[1] * 0.8f, 0.0f);
                }
                return true;
            case kModeThrowIn:
                target = Pos();
                return true;
            default:
                break;
        }
        if (m.ballRetainer != p) return true;
        action.desiredFunctionType = kFnHighPass;
        target = Vec3(kPitchHalfLength * side, Random(-kPitchHalfWidth, kPitchHalfWidth), 0.0f);
        const int mate = GetClosestPlayer(w, c, teamID, target, false, p);
        if (mate < 0) return true;
        const int marker = GetClosestPlayer(w, c, oppID, Pos(mate), false, -1);
        if (marker < 0) return true;
        if (((Pos(marker) + Mov(marker) * 0.1f) - Pos(mate)).Length() > 10.0f || ps.possessionDurationMs > 4000) {
            t.forcedTargetPlayer = mate;
            return true;
        }
        return false;
    }
    // The commands of a set piece's taker (or the ball's retainer): the restart's shot or pass to
    // the teammate nearest its target, then a movement: toward the ball at walking pace, or, for
    // the retainer, facing its pass (or the centre) standing.
    HDN void SetPieceCommands() {
        const int type = AI().setPieceType;
        Vec3 passDir;
        if (type == kModePenalty) {
            passDir = PenaltyShot();
        } else {
            PlayerCommand action = DefaultPlayerCommand();
            TouchInformation &t = action.touchInfo;
            action.desiredFunctionType = kFnShortPass;
            t.inputDirection = Dir();
            t.inputPower = 0.5f;
            t.autoDirectionBias = 1.0f;
            t.autoPowerBias = 1.0f;
            t.forcedTargetPlayer = -1;
            Vec3 target;
            if (RestartPassTarget(type, action, target)) {
                if (t.forcedTargetPlayer < 0) t.forcedTargetPlayer = GetClosestPlayer(w, c, teamID, target, false, p);
                AimPass(w, p, action.desiredFunctionType, t.inputDirection, t.inputPower, t.autoDirectionBias, t.autoPowerBias,
                        t.desiredDirection, t.desiredPower, t.targetPlayer, t.forcedTargetPlayer);
                q.push_back(action);
            }
            passDir = t.desiredDirection;
        }
        PlayerCommand cmd = DefaultPlayerCommand();
        cmd.useDesiredMovement = true;
        cmd.useDesiredLookAt = true;
        if (m.ballRetainer != p) {
            BallControlMovement(kWalkVelocity, cmd.desiredDirection, cmd.desiredVelocityFloat, cmd.desiredLookAt);
        } else {
            cmd.desiredDirection = (passDir.Length() > 0.0f) ? passDir.Get2D().Normalized(Dir()) : (Vec3(0) - Pos()).Normalized(Dir());
            cmd.desiredVelocityFloat = kIdleVelocity;
            cmd.desiredLookAt = Pos() + cmd.desiredDirection * 10.0f;
        }
        q.push_back(cmd);
    }

    // The command out of open play, when there is one: celebrating after a goal, watching the
    // referee show a card (from a second after play stopped until the restart is prepared), and,
    // out of play or for a lazy player, drifting toward the centre (60% its own direction) at
    // 95% of its speed less a draw of up to 3.2 m/s, looking at the ball. True when one was given.
    HD bool StoppageCommand(bool lazy) {
        const RefereeBuffer &rb = m.referee.buffer;
        if (!m.inPlay && m.goalScored) {
            AddCelebration();
            return true;
        }
        const bool card = m.referee.foul.foulType == 2 || m.referee.foul.foulType == 3;
        PlayerCommand cmd = DefaultPlayerCommand();
        cmd.useDesiredMovement = true;
        cmd.useDesiredLookAt = true;
        if (!m.inPlay && rb.active && card && rb.stopTime < m.actualTimeMs - 1000 && rb.prepareTime > m.actualTimeMs) {
            cmd.desiredDirection = Dir();
            cmd.desiredVelocityFloat = kIdleVelocity;
            cmd.desiredLookAt = m.officials[0].humanoid.spatial.position;
            q.push_back(cmd);
            return true;
        }
        if (m.inPlay && !lazy) return false;
        cmd.desiredDirection = (Dir() * 0.6f + (Vec3(0) - Pos()).Normalized(Dir()) * 0.4f).Normalized(Dir());
        cmd.desiredVelocityFloat = ClampVelocity(FloatVelocity() * 0.95f - Random(0.0f, 3.2f));
        cmd.desiredLookAt = Pos() + (BallAt(0).Get2D() - Pos()).Normalized(cmd.desiredDirection) * 10.0f;
        q.push_back(cmd);
        return true;
    }
    // How a player off the ball presses the opponents' designated player: under team pressure, it
    // faces its own goal and stands; else, with the opponents best placed, no man to mark and the
    // opponent within the hunting distance (10 to 20 m by mindset, shorter when tired or for an
    // easy team), the team's designated player (with possession over 0.8) goes for the ball in
    // haste, and one of the two nearest to the opponent moves to its defending position when it
    // is out of line.
    HD void PressOpponent(bool &forceMagnet, bool &extraHaste) {
        const int o = Opp().designatedTeamPossessionPlayer;
        const float mind = GetMindSet(DynamicRole());
        float hunt = 10.0f + (1.0f - mind) * 10.0f;
        hunt *= 0.5f * ps.base.fatigueFactorInverse +
                0.5f * (1.0f - NormalizedClamp(PlayerAverageVelocity(w, p, 10), kIdleVelocity, kSprintVelocity));
        hunt *= 0.3f + TeamDifficulty(w, teamID) * 0.7f;
        if (forceMagnet) {
            ctl.inputDirection = Vec3(side * kPitchHalfLength, 0, 0) - Pos();
            ctl.inputVelocityFloat = kIdleVelocity;
            ctl.inputDirection.Normalize(Dir());
            return;
        }
        if (!(!ctl.teamHasBestPossession && ps.manMarking < 0 && ((Pos(o) + Mov(o) * 0.12f) - (Pos() + Mov() * 0.04f)).Length() < hunt))
            return;
        if (p == Own().designatedTeamPossessionPlayer && ctl.possessionAmount > 0.8f) {
            forceMagnet = true;
            extraHaste = true;
        }
        const PlayerList nearest = GetClosestPlayers(w, c, teamID, Pos(o) + Mov(o) * 0.1f, false, 2);
        bool near = false;
        for (int i = 0; i < nearest.count && !near; i++) near = nearest[i] == p;
        if (!near) return;
        const Vec3 defend = GetDefendPosition(o);
        if (!NeedDefendingMovement(side, Pos(), defend)) return;
        ctl.inputDirection = (defend - Pos()).Normalized(ctl.inputDirection);
        ctl.inputVelocityFloat = Clamp((defend - Pos()).Length() * kDistanceToVelocity, 0.0f, kSprintVelocity);
        forceMagnet = true;
    }

    // The part a player without a gamer plays in open play: the keeper keeps goal; an outfield
    // player off the ball keeps its line's place; the designated player plays the ball when its
    // team has no gamer, or it has a gamer's controller that is not active. (A ball retainer was
    // handled as a restart before.)
    enum OpenPlayPart { kNoPart, kLinePart, kBallPart, kKeeperPart };
    HD int OpenPlayPartOf(int role) const {
        if (!m.inPlay || m.inSetPiece) return kNoPart;
        if (role == kRoleGoalkeeper) return kKeeperPart;
        if (m.designatedPossessionPlayer != p) return kLinePart;
        const bool unattended = HumanGamerCount(Own()) == 0 || (!ExternalControllerActive(w, p) && ps.base.externalController >= 0);
        return unattended ? kBallPart : kNoPart;
    }
    // The line an outfield role keeps: backs defend, the five midfield roles hold the middle, the
    // centre-forward attacks.
    HD static int LineOfRole(int role) {
        switch (role) {
            case kRoleLeftBack:
            case kRoleCentreBack:
            case kRoleRightBack: return kDefense;
            case kRoleCentreForward: return kOffense;
            default: return kMidfield;
        }
    }
    // The keeper's part: its own movement, which replaces the movement command when the ball is
    // bound for goal or another player is designated (the return value), and a deflection unless
    // it holds the ball uniquely with possession 3.4 or more (pickups only when nothing is bound
    // for goal and the possession passes 1.3).
    HD bool KeeperPart(Vec3 &dir, float &vel) {
        const bool bound = BallBoundForGoal();
        GoalieRequestInput(dir, vel);
        if (!ctl.hasUniquePossession || ctl.possessionAmount < 3.4f) KeeperDeflectCommand(!bound && ctl.possessionAmount > 1.3f);
        return bound || p != m.designatedPossessionPlayer;
    }
    // The team's pressure order names this player, still running, while the opponents hold the
    // ball better; never the designated player or the keeper.
    HD bool PressureOrdered(int role) const {
        return m.inPlay && !m.inSetPiece && (AI().endApplyTeamPressureMs > m.actualTimeMs && AI().teamPressurePlayer == p) &&
               !ctl.teamHasBestPossession && m.designatedPossessionPlayer != p && role != kRoleGoalkeeper;
    }
    // Moving by the player's own choice: along `dir` at `vel`, looking 10 m toward the ball 40 ms
    // ahead.
    HD void OwnMovement(const Vec3 &dir, float vel) {
        PlayerCommand cmd = DefaultPlayerCommand();
        cmd.useDesiredMovement = true;
        cmd.desiredDirection = dir;
        cmd.desiredVelocityFloat = vel;
        cmd.useDesiredLookAt = true;
        cmd.desiredLookAt = Pos() + (MentalBall(40).Get2D() - Pos()).Normalized(0) * 10.0f;
        q.push_back(cmd);
    }

    // The request of a player without a gamer: the situation and the opponent on the ball, then
    // a stoppage command or the restart when there is one; in open play its part's input (one
    // call site per part, so that the matches of a wavefront whose players differ in role run it
    // together), the touch commands, and the movement command (pressing first), or the keeper's
    // own movement.
    HDN bool RequestCommand() {
        if (m.designatedPossessionPlayer < 0) return Fail("the AI controller finds no designated possession player");
        if (Own().designatedTeamPossessionPlayer < 0 || Opp().designatedTeamPossessionPlayer < 0)
            return Fail("the AI controller finds no designated team possession player");
        k = MentalImageIndex(w, ctl.mentalImageTime);
        ctl.lastSwitchTimeDurationMs = 0;
        ctl.lastSwitchTimeMs = 0;
        ps.desiredTimeToBallMs = 0;
        ControllerCalculateSituation(w, p, ctl);
        ctl.opponentPlayer = TeamBestPossessionPlayer(w, oppID);
        ctl.timeNeededMs = (float)ps.timeToBallMs;
        // GRF: laziness is fixed at creation from the player's own static entry.
        if (StoppageCommand(c.sd->formation[p].lazy)) return true;
        if ((m.inSetPiece && AI().taker == p) || m.ballRetainer == p) {
            SetPieceCommands();
            return true;
        }
        const int role = StaticRole(p);
        const int part = OpenPlayPartOf(role);
        Vec3 input = Dir(), own = Dir();
        float inputVel = kIdleVelocity, ownVel = kIdleVelocity;
        bool ownMovement = false;
        bool onTheBall = part == kBallPart && ps.timeToBallMs < 1000;
        if (part == kKeeperPart) {
            ownMovement = KeeperPart(own, ownVel);
            onTheBall = ps.timeToBallMs < 1000 && m.designatedPossessionPlayer == p;
        }
        if (part == kLinePart) FieldStrategyRequestInput(LineOfRole(role), input, inputVel);
        if (onTheBall) GetOnTheBallCommands(input, inputVel);
        bool forceMagnet = PressureOrdered(role), extraHaste = false;
        ctl.inputDirection = input;
        ctl.inputVelocityFloat = inputVel;
        eliza->lastDesiredDirection = input.Length() != 0 ? input : Dir();
        eliza->lastDesiredVelocity = inputVel;
        const bool openPlay = m.inPlay && !m.inSetPiece;
        if (openPlay) {
            BallControlCommand();
            TrapCommand();
            InterfereCommand(false);
            SlidingCommand();
        }
        if (ownMovement || !openPlay) {
            OwnMovement(own, ownVel);
            return true;
        }
        if (p != m.designatedPossessionPlayer) PressOpponent(forceMagnet, extraHaste);
        ctl.inputVelocityFloat = RangeVelocity(ctl.inputVelocityFloat);
        MovementCommand(forceMagnet, extraHaste);
        return true;
    }
};

HDN void TeamApplyTeamPressure(World &w, const Ctx &c, int teamID) {
    TeamAI &ai = TeamByID(w, teamID).ai;
    ai.endApplyTeamPressureMs = w.match.actualTimeMs + 500;
    int o = TeamBestPossessionPlayer(w, 1 - teamID);
    const SpatialState &os = Sp(w, o);
    Vec3 op = os.position + os.movement * 0.24f;
    ai.teamPressurePlayer =
        GetClosestPlayer(w, c, teamID, op + Vec3(TeamDynamicSide(w, teamID) * 1.0f, 0, 0), true, TeamGoalie(w, c, teamID));
    if (ai.teamPressurePlayer >= 0) w.match.players[ai.teamPressurePlayer].manMarking = o;
}
HD void TeamApplyKeeperRush(World &w, int teamID) { TeamByID(w, teamID).ai.endApplyKeeperRushMs = w.match.actualTimeMs + 300; }

// ---- a gamer's player ------------------------------------------------------------------------------
// A gamer's armed action expires: a pass or shot once its touch has happened, when the shot or
// high-pass gauge is overridden by the short-pass button outside set pieces, after 2 s without
// release, when the player's time to the ball grows by 700 ms, or in an interference; a defensive
// action once its tackle has happened or after a second.
HD void ExpireGamerAction(const MatchState &m, const Player &ps, const AnimationState &cur, HumanControllerState &hc) {
    const bool *b = hc.keyboard.buttons;
    const int fn = cur.functionType;
    const bool touched = !(cur.frameNum < cur.touchFrame);
    bool expired = false;
    if (hc.actionMode == 2) {
        expired = (IsPassOrShot(fn) && touched) ||
                  (!m.inSetPiece && b[kBtnShortPass] && (hc.actionButton == kBtnShot || hc.actionButton == kBtnHighPass)) ||
                  (!m.inSetPiece && (hc.actionBufferTimeMs > 2000 || ps.timeToBallMs > ps.timeToBallPreviousMs + 700 || fn == kFnInterfere));
    } else if (hc.actionMode == 1) {
        expired = ((fn == kFnSliding || fn == kFnInterfere) && touched) || hc.actionBufferTimeMs > 1000;
    }
    if (!expired) return;
    hc.actionMode = 0;
    hc.gaugeMs = 0;
    hc.actionBufferTimeMs = 0;
}
// A pass of a gamer's: the stick's direction at a power from the gauge (to the pass type's
// exponent) with the default gameplay settings' auto biases.
HD void GamerPass(World &w, int p, const PlayerControllerState &ctl, int type, float gauge, CommandQueue &q) {
    const float exponent = type == kFnShortPass ? 0.7f : type == kFnLongPass ? 0.65f : 0.55f;
    PlayerCommand cmd = DefaultPlayerCommand();
    cmd.desiredFunctionType = type;
    TouchInformation &ti = cmd.touchInfo;
    ti.inputDirection = ctl.inputDirection;
    ti.inputPower = Clamp(libm::powf(gauge, exponent), 0.01f, 1.0f);
    ti.autoDirectionBias = type == kFnShortPass ? 0.4f : 0.2f;
    ti.autoPowerBias = type == kFnHighPass ? 0.5f : 0.7f;
    AimPass(w, p, type, ti.inputDirection, ti.inputPower, ti.autoDirectionBias, ti.autoPowerBias, ti.desiredDirection, ti.desiredPower,
            ti.targetPlayer, -1);
    q.push_back(cmd);
}
// A pass or shot armed by a gamer goes out when its button is released, held past half a second,
// or (off the ball, outside set pieces) once it has been released before; its gauge runs from
// 60 ms to a second. A kick-off taker passes short to the nearest teammate ahead whatever the
// button; passes share one call site, so that matches of a wavefront passing in different ways
// run the pass search together.
HD void ReleaseGamerAction(World &w, const Ctx &c, int p, AIController &ai, HumanControllerState &hc, CommandQueue &q) {
    const MatchState &m = w.match;
    const bool *b = hc.keyboard.buttons;
    const int t = w.playerTeamID[p];
    const TeamAI &tai = TeamByID(w, t).ai;
    const PlayerControllerState &ctl = hc.base;
    if (!(!b[hc.actionButton] || (b[hc.actionButton] && hc.gaugeMs > 500) ||
          (!m.players[p].hasPossession && !m.inSetPiece && hc.actionBufferTimeMs > 0)))
        return;
    const int baseMs = 60;
    float gauge = (float)(hc.gaugeMs - baseMs) * (1.0f / float(1000 - baseMs));
    gauge = Clamp(gauge, 0.0f, 1.0f);
    if (m.inSetPiece && tai.taker == p && tai.setPieceType == kModeKickOff) {
        PlayerCommand cmd = DefaultPlayerCommand();
        cmd.desiredFunctionType = kFnShortPass;
        TouchInformation &ti = cmd.touchInfo;
        ti.autoDirectionBias = 1.0f;
        ti.autoPowerBias = 1.0f;
        ti.inputDirection = ai.Dir();
        ti.inputPower = 0.1f;
        ti.forcedTargetPlayer = GetClosestPlayer(w, c, t, ai.Pos() + ai.Dir() * 1.0f, false, p);
        AimPass(w, p, cmd.desiredFunctionType, ti.inputDirection, ti.inputPower, ti.autoDirectionBias, ti.autoPowerBias,
                ti.desiredDirection, ti.desiredPower, ti.targetPlayer, ti.forcedTargetPlayer);
        q.push_back(cmd);
    } else if (hc.actionButton == kBtnShortPass || hc.actionButton == kBtnLongPass || hc.actionButton == kBtnHighPass) {
        const int type = hc.actionButton == kBtnShortPass ? kFnShortPass : hc.actionButton == kBtnLongPass ? kFnLongPass : kFnHighPass;
        GamerPass(w, p, ctl, type, gauge, q);
    } else if (hc.actionButton == kBtnShot) {
        PlayerCommand cmd = DefaultPlayerCommand();
        cmd.desiredFunctionType = kFnShot;
        cmd.desiredVelocityFloat = ctl.inputVelocityFloat;
        cmd.touchInfo.inputDirection = ctl.inputDirection;
        cmd.touchInfo.autoDirectionBias = 1.0f;
        cmd.touchInfo.desiredDirection = AimShot(w, p, cmd.touchInfo.inputDirection, cmd.touchInfo.autoDirectionBias);
        cmd.touchInfo.desiredPower = Clamp(libm::powf(gauge, 0.6f), 0.01f, 1.0f);
        q.push_back(cmd);
    }
}
// A defensive action lasts while its button is held: a sliding tackle along the stick, team
// pressure, or the keeper's rush; released, it ends.
HD void HoldDefensiveAction(World &w, const Ctx &c, int p, AIController &ai, HumanControllerState &hc, CommandQueue &q) {
    const int t = w.playerTeamID[p];
    if (!hc.keyboard.buttons[hc.actionButton]) {
        hc.actionMode = 0;
        return;
    }
    if (hc.actionButton == kBtnSliding) {
        PlayerCommand cmd = DefaultPlayerCommand();
        cmd.desiredFunctionType = kFnSliding;
        cmd.useDesiredMovement = true;
        cmd.desiredDirection = hc.base.inputDirection;
        cmd.desiredVelocityFloat = hc.base.inputVelocityFloat;
        cmd.useDesiredLookAt = true;
        cmd.desiredLookAt = ai.Pos() + ai.Mov() * 0.1f + cmd.desiredDirection * 10.0f;
        q.push_back(cmd);
    }
    if (hc.actionButton == kBtnTeamPressure) TeamApplyTeamPressure(w, c, t);
    if (hc.actionButton == kBtnKeeperRush) TeamApplyKeeperRush(w, t);
}
// In open play a gamer's player controls and traps along the stick's steady direction (dribble
// turns an idle touch to goal, dribble with sprint knocks on); with a pass or shot armed it
// does so along its own direction at a speed that falls the more the stick points away, then
// interferes when pressure is held.
HD void GamerTouchCommands(World &w, int p, AIController &ai, HumanControllerState &hc) {
    const bool *b = hc.keyboard.buttons;
    PlayerControllerState &ctl = hc.base;
    const bool idleTurn = b[kBtnDribble];
    const bool knockOn = b[kBtnDribble] && b[kBtnSprint];
    const Vec3 savedDir = ctl.inputDirection;
    const float savedVel = ctl.inputVelocityFloat;
    if (hc.actionMode == 2) {
        float along = ai.Dir().Dot(ctl.inputDirection) * 0.5f + 0.5f;
        if (along < 0) along = 0;
        if (Sp(w, p).velocityCat != kVelIdle)
            ctl.inputDirection = (ai.Dir() * 1.0f + ctl.inputDirection * 0.0f).Normalized(ctl.inputDirection);
        along = libm::powf(along, 1.5f);
        along = along * 0.8f + 0.2f;
        along *= 0.9f;
        ctl.inputVelocityFloat = ai.FloatVelocity() * along;
    }
    ai.BallControlCommand(idleTurn, knockOn, true, false);
    ai.TrapCommand(idleTurn, knockOn);
    if (hc.actionMode == 2) {
        ctl.inputDirection = savedDir;
        ctl.inputVelocityFloat = savedVel;
    }
    ai.InterfereCommand(b[kBtnPressure]);
}
// The commands of a gamer's player (GRF's human controller with the default gameplay settings):
// the armed action expires, goes out or holds; at a set piece the taker (until its pass goes)
// and the others wait in position; otherwise the touch commands and a movement, forced toward
// the ball by pressure or an armed pass or shot. Without the magnet the movement follows the
// stick, facing the ball half a second ahead; dribble with sprint off the ball follows it too.
HDN bool HumanRequestCommand(World &w, const Ctx &c, int p, CommandQueue &q) {
    ENG_SCOPE(45);
    HumanControllerState &hc = HumanGamerOf(w, p).controller;
    PlayerControllerState &ctl = hc.base;
    AIController ai(w, c, p, q, ctl, nullptr);
    MatchState &m = w.match;
    Player &ps = m.players[p];
    const int t = w.playerTeamID[p];
    const TeamAI &tai = TeamByID(w, t).ai;
    const bool *b = hc.keyboard.buttons;
    ai.k = MentalImageIndex(w, ctl.mentalImageTime);
    ps.desiredTimeToBallMs = 0;
    ctl.opponentPlayer = TeamBestPossessionPlayer(w, 1 - t);
    ctl.timeNeededMs = (float)ps.timeToBallMs;
    Vec3 rawDir;
    float rawVel = 0;
    HumanGetKeyboardInput(w, p, rawDir, rawVel);
    ctl.inputDirection = rawDir;
    ctl.inputVelocityFloat = rawVel;
    ExpireGamerAction(m, ps, Hum(w, p).anim, hc);
    if (hc.actionMode == 2) ReleaseGamerAction(w, c, p, ai, hc, q);
    else if (hc.actionMode == 1) HoldDefensiveAction(w, c, p, ai, hc, q);
    const bool takerWaits = tai.taker == p && (hc.actionMode != 2 || (hc.actionMode == 2 && b[hc.actionButton]) || m.ballRetainer == p);
    if (m.inSetPiece && (takerWaits || (tai.taker != p && m.ballRetainer < 0))) {
        ai.SetPieceCommand();
        return true;
    }
    const Vec3 unsteady = ctl.inputDirection;
    ctl.inputDirection = hc.steadyDirection;
    if (m.inPlay && !m.inSetPiece) GamerTouchCommands(w, p, ai, hc);
    const bool urge = (hc.actionMode != 2 && b[kBtnPressure]) || hc.actionMode == 2;
    ai.MovementCommand(urge, urge);
    if (!q.empty()) {
        PlayerCommand &cmd = q.back();
        if (!w.scenario.useMagnet) {
            cmd.desiredDirection = ctl.inputDirection;
            cmd.desiredVelocityFloat = ctl.inputVelocityFloat;
            if (cmd.desiredVelocityFloat < kIdleDribbleSwitch) cmd.desiredDirection = (ai.MentalBall(500).Get2D() - ai.Pos()).Normalized(ctl.inputDirection);
            cmd.desiredLookAt = ai.MentalBall(500).Get2D();
        }
        if (m.inPlay && !m.inSetPiece && b[kBtnDribble] && b[kBtnSprint] && !ctl.hasBestPossession) {
            cmd.desiredDirection = ctl.inputDirection;
            cmd.desiredVelocityFloat = ctl.inputVelocityFloat;
        }
    }
    ctl.inputDirection = unsteady;
    return true;
}

HDN bool PlayerRequestCommand(World &w, const Ctx &c, int p, CommandQueue &q) {
    ENG_SCOPE(13);
    if (ExternalControllerActive(w, p)) return HumanRequestCommand(w, c, p, q);
    AIControllerState &e = w.match.players[p].controller;
    AIController ai(w, c, p, q, e.base, &e);
    return ai.RequestCommand();
}

}  // namespace eng
