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

    // Pass to the best-placed team mate, a panic clearance near the own goal, a shot when placed
    // for one, and a dribble direction from a force field.
    HDN void GetOnTheBallCommands(Vec3 &rawDir, float &rawVel) {
        ENG_SCOPE(44);
        float movDiff = NormalizedClamp((m.ball.momentum - Mov()).Length(), 0.0f, 10.0f);
        float oneTouchIsHard = movDiff - Stat(kStatShortPass) * movDiff * 0.8f;
        ImageList opps;
        MentalTeamPlayerImages(w, k, oppID, opps);
        float ptf = NormalizedClamp((float)ps.possessionDurationMs, 0, 5000);
        float longPossession = ptf * ptf;
        const float mind = GetMindSet(DynamicRole());
        const float fsw = 0.4f, sw = 0.3f;
        float fw = 2.0f + mind * 6.0f;
        float totalTactical = fsw + sw + fw;
        float improvement = 0.06f * (1.0f - mind);
        float diffW = 1.0f + (mind * mind) * 10.0f;
        const float passW = 1.0f;
        float passMinimum = 0.2f * (1.0f - mind) - longPossession * 0.1f;
        float totalPassW = diffW + passW;
        float passThreshold = 0.1f - longPossession * 0.05f;
        float rating = TacticalRating(ps, fsw, sw, fw, totalTactical);
        PlayerList mates = TeamActivePlayers(w, teamID);
        float bestTotal = 0.0f, bestPassRating = 0.0f;
        int bestPlayer = -1, bestPassType = kFnShortPass;
        for (int i = 0; i < mates.count; i++) {
            const int mate = mates[i];
            if (mate == p) continue;
            float mr = TacticalRating(m.players[mate], fsw, sw, fw, totalTactical);
            if (StaticRole(mate) == kRoleGoalkeeper) mr *= 0.7f;
            if (!(mr > rating + improvement)) continue;
            float diff = mr - rating;
            float oShort = PassingOddsTo(mate, kFnShortPass, opps);
            float oLong = PassingOddsTo(mate, kFnLongPass, opps);
            float oHigh = PassingOddsTo(mate, kFnHighPass, opps);
            float pr;
            int pt;
            if (oShort >= oLong && oShort >= oHigh) {
                pr = oShort;
                pt = kFnShortPass;
            } else if (oLong >= oHigh) {
                pr = oLong;
                pt = kFnLongPass;
            } else {
                pr = oHigh;
                pt = kFnHighPass;
            }
            float total = diff * diffW + pr * passW - oneTouchIsHard;
            total /= totalPassW;
            if (total > bestTotal && total > passThreshold && pr > passMinimum) {
                bestTotal = total;
                bestPlayer = mate;
                bestPassRating = pr;
                bestPassType = pt;
            }
        }
        if (mind < 0.25f) {
            float panic = 1.0f - mind * 2.0f;
            float goalCloseness = 1.0f - NormalizedClamp((Pos() - Vec3(kPitchHalfLength * side, 0, 0)).Length(), 2.0f, 16.0f);
            if (DynamicRole() != kRoleGoalkeeper) {
                if ((bestPlayer < 0 || bestPassRating < panic * goalCloseness) &&
                    ctl.possessionAmount < 0.9f + panic * goalCloseness * 0.8f)
                    AddPanicPass();
            } else if (ctl.possessionAmount < 3.0f) {
                AddPanicPass();
            }
        }
        if (bestPlayer >= 0) AddPass(bestPlayer, bestPassType);
        float goalDistance = NormalizedClamp((Vec3(kPitchHalfLength * -side, 0, 0) - Pos()).Length(), 0.0f, 32.0f);
        float ideal = 1.0f - NormalizedClamp((Vec3((kPitchHalfLength - 7.0f) * -side, 0, 0) - Pos()).Length(), 0.0f, 16.0f);
        ideal = Curve(ideal, 1.0f);
        if (ideal > 0.1f) {
            const float gx = (kPitchHalfLength + 1.0f) * -side;
            float low = PassingOdds(Vec3(gx, -3.6f, 0), kFnShot, opps, 3.0f);
            float center = PassingOdds(Vec3(gx, 0.0f, 0), kFnShot, opps, 3.0f);
            float high = PassingOdds(Vec3(gx, 3.6f, 0), kFnShot, opps, 3.0f);
            float odds = center, y = 0.0f;
            if (low > odds) {
                odds = low;
                y = -3.5f;
            }
            if (high > odds) {
                odds = high;
                y = 3.5f;
            }
            odds = libm::powf(odds, 0.5f);
            if (odds + Random(0.0f, 0.5f) > 0.5f) {
                PlayerCommand cmd = DefaultPlayerCommand();
                cmd.desiredFunctionType = kFnShot;
                cmd.desiredVelocityFloat = rawVel;
                const float shot = Stat(kStatShot);
                float ry = y + Random(-1.0f + shot, 1.0f - shot);
                TouchInformation &t = cmd.touchInfo;
                t.desiredDirection = (Vec3(gx, ry, 0) - (Pos() + Mov() * 0.2f)).Normalized(Vec3(-side, 0, 0));
                t.desiredDirection = (t.desiredDirection * 0.7f + -Dir() * (FloatVelocity() / kSprintVelocity) * 0.3f).Normalized();
                t.autoDirectionBias = 1.0f;
                t.desiredPower = Random(0.7f * (0.6f + goalDistance * 0.4f), 1.0f * (0.6f + goalDistance * 0.4f));
                q.push_back(cmd);
            }
        }
        BestDribbleMovement(rawDir, rawVel);
    }

    HDN void AddCelebration() {
        int xSide = (BallAt(0).Get2D().v[0] > 0) ? 1 : -1;
        int ySide = side;
        const int ltp = Own().lastTouchPlayer;
        if (ltp >= 0) ySide = (Pos(ltp).v[1] > 0) ? 1 : -1;
        Vec3 cp = Vec3(kPitchHalfLength * xSide, kPitchHalfWidth * ySide, 0);
        Vec3 dd = (cp - Pos()).Normalized();
        float dv = ClampVelocity((cp - Pos()).Length() / 4.0f);
        Vec3 look = Pos() + Dir() * 1000;
        int type = 1;
        if (m.lastGoalTeam != TeamSlot(w, teamID)) {
            type = 2;
            dv = kIdleVelocity;
        }
        int madeGoal = 1;
        if (type == 1) {
            if (ltp == p) {
                madeGoal = 2;
                dv = kSprintVelocity;
            } else if (ltp >= 0) {
                if ((Pos(ltp) - Pos()).Length() < 20) {
                    cp = Pos(ltp);
                    dd = ((Pos(ltp) * 0.5f + cp * 0.5f) - Pos()).Normalized();
                    dv = ClampVelocity((float)((double)(Pos(ltp) - Pos()).Length() / 2.0));
                } else {
                    dv = kIdleVelocity;
                }
                look = Pos() + Dir(ltp) * 100;
            }
        }
        const uint64_t stop = m.referee.buffer.stopTime;
        if (m.actualTimeMs - stop > 2000 && m.actualTimeMs - stop < 4000) {
            PlayerCommand cmd = DefaultPlayerCommand();
            cmd.desiredFunctionType = kFnSpecial;
            cmd.useSpecialVar1 = true;
            cmd.specialVar1 = type;
            cmd.useSpecialVar2 = true;
            cmd.specialVar2 = madeGoal;
            q.push_back(cmd);
        }
        PlayerCommand cmd = DefaultPlayerCommand();
        cmd.useDesiredMovement = true;
        cmd.desiredDirection = dd;
        cmd.desiredVelocityFloat = dv;
        cmd.useDesiredLookAt = true;
        cmd.desiredLookAt = look;
        q.push_back(cmd);
    }

    HDN void SetPieceCommands() {
        const int type = AI().setPieceType;
        PlayerCommand action = DefaultPlayerCommand();
        TouchInformation &t = action.touchInfo;
        if (type == kModePenalty) {
            action.desiredFunctionType = kFnShot;
            float ry = Random(-5, 5);
            t.desiredDirection = (Vec3(-side * kPitchHalfLength, ry, 0) - Pos()).Normalized(Vec3(-side, 0, 0));
            t.desiredPower = Random(0.4f, 1.0f);
            q.push_back(action);
        } else {
            action.desiredFunctionType = kFnShortPass;
            t.inputDirection = Dir();
            t.inputPower = 0.5f;
            t.autoDirectionBias = 1.0f;
            t.autoPowerBias = 1.0f;
            t.forcedTargetPlayer = -1;
            Vec3 target;
            bool doCommand = true;
            if (type == kModeGoalKick) {
                if (Random(0.0f, 1.0f) > 0.4f && HumanGamerCount(Own()) == 0) {
                    action.desiredFunctionType = kFnHighPass;
                    float ry = Random(-kPitchHalfWidth, kPitchHalfWidth);
                    target = Vec3((kPitchHalfLength * -side) * 0.2f, ry, 0.0f);
                } else {
                    float ry = Random(-kPitchHalfWidth, kPitchHalfWidth);
                    target = Vec3(Pos().v[0] * 0.9f, ry, 0.0f);
                }
            } else if (type == kModeKickOff) {
                target = Pos() + Dir() * 1.0f;
            } else if (type == kModeFreeKick) {
                if (Random(0.0f, 1.0f) > 0.5f) {
                    action.desiredFunctionType = kFnHighPass;
                    float ry = Random(-10.0f, 10.0f);
                    target = Vec3(kPitchHalfLength * -side, ry, 0.0f);
                } else {
                    float ry = Random(-10.0f, 10.0f);
                    target = Pos() + Vec3(-side * 10.0f, ry, 0.0f);
                }
            } else if (type == kModeCorner) {
                if (Random(0.0f, 1.0f) > 0.3f) {
                    action.desiredFunctionType = kFnHighPass;
                    // GRF: arguments evaluate right to left, so y draws first.
                    float ry = Random(-10.0f, 10.0f);
                    float rx = Random(0.0f, 0.12f);
                    target = Vec3((kPitchHalfLength * -side) * (0.99f - rx), ry, 0.0f);
                } else {
                    target = Vec3((kPitchHalfLength * -side) * 0.8f, Pos().v[1] * 0.8f, 0.0f);
                }
            } else if (type == kModeThrowIn) {
                target = Pos();
            } else if (m.ballRetainer == p) {
                action.desiredFunctionType = kFnHighPass;
                float ry = Random(-kPitchHalfWidth, kPitchHalfWidth);
                target = Vec3(kPitchHalfLength * side, ry, 0.0f);
                int tp = GetClosestPlayer(w, c, teamID, target, false, p);
                if (tp >= 0) {
                    int co = GetClosestPlayer(w, c, oppID, Pos(tp), false, -1);
                    if (co >= 0) {
                        if (((Pos(co) + Mov(co) * 0.1f) - Pos(tp)).Length() > 10.0f || ps.possessionDurationMs > 4000)
                            t.forcedTargetPlayer = tp;
                        else
                            doCommand = false;
                    }
                }
            }
            if (doCommand) {
                if (t.forcedTargetPlayer < 0) t.forcedTargetPlayer = GetClosestPlayer(w, c, teamID, target, false, p);
                AimPass(w, p, action.desiredFunctionType, t.inputDirection, t.inputPower, t.autoDirectionBias, t.autoPowerBias,
                        t.desiredDirection, t.desiredPower, t.targetPlayer, t.forcedTargetPlayer);
                q.push_back(action);
            }
        }
        PlayerCommand cmd = DefaultPlayerCommand();
        cmd.useDesiredMovement = true;
        cmd.useDesiredLookAt = true;
        if (m.ballRetainer != p) {
            BallControlMovement(kWalkVelocity, cmd.desiredDirection, cmd.desiredVelocityFloat, cmd.desiredLookAt);
        } else {
            cmd.desiredDirection = (t.desiredDirection.Length() > 0.0f) ? t.desiredDirection.Get2D().Normalized(Dir())
                                                                       : (Vec3(0) - Pos()).Normalized(Dir());
            cmd.desiredVelocityFloat = kIdleVelocity;
            cmd.desiredLookAt = Pos() + cmd.desiredDirection * 10.0f;
        }
        q.push_back(cmd);
    }

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
        Vec3 rawDir = Dir();
        float rawVel = kIdleVelocity;
        Vec3 manualDir = Dir();
        float manualVel = kIdleVelocity;
        bool manual = false, extraHaste = false;
        // GRF: laziness is fixed at creation from the player's own static entry.
        const bool lazy = c.sd->formation[p].lazy;
        const int role = StaticRole(p);
        const RefereeBuffer &rb = m.referee.buffer;
        if (!m.inPlay && m.goalScored) {
            AddCelebration();
            return true;
        }
        if (!m.inPlay && rb.active && (m.referee.foul.foulType == 2 || m.referee.foul.foulType == 3) &&
            rb.stopTime < m.actualTimeMs - 1000 && rb.prepareTime > m.actualTimeMs) {
            // Everyone watches the referee show the card.
            PlayerCommand cmd = DefaultPlayerCommand();
            cmd.useDesiredMovement = true;
            cmd.useDesiredLookAt = true;
            cmd.desiredDirection = Dir();
            cmd.desiredVelocityFloat = kIdleVelocity;
            cmd.desiredLookAt = m.officials[0].humanoid.spatial.position;
            q.push_back(cmd);
            return true;
        }
        if (!m.inPlay || lazy) {
            PlayerCommand cmd = DefaultPlayerCommand();
            cmd.useDesiredMovement = true;
            cmd.desiredDirection = (Dir() * 0.6f + (Vec3(0) - Pos()).Normalized(Dir()) * 0.4f).Normalized(Dir());
            cmd.desiredVelocityFloat = ClampVelocity(FloatVelocity() * 0.95f - Random(0.0f, 3.2f));
            cmd.useDesiredLookAt = true;
            cmd.desiredLookAt = Pos() + (BallAt(0).Get2D() - Pos()).Normalized(cmd.desiredDirection) * 10.0f;
            q.push_back(cmd);
            return true;
        }
        if ((m.inSetPiece && AI().taker == p) || m.ballRetainer == p) {
            SetPieceCommands();
            return true;
        }
        // The field strategy of each line and the on-the-ball commands each have one call site, so
        // that matches of a wavefront whose players differ in role or situation run them together;
        // per environment the calls and their order are GRF's.
        int strategy = -1;
        bool onTheBall = false;
        if (m.inPlay && !m.inSetPiece && m.ballRetainer != p && m.designatedPossessionPlayer != p && role != kRoleGoalkeeper) {
            if (role == kRoleLeftBack || role == kRoleCentreBack || role == kRoleRightBack)
                strategy = kDefense;
            else if (role == kRoleDefensiveMid || role == kRoleLeftMid || role == kRoleCentralMid || role == kRoleRightMid ||
                     role == kRoleAttackingMid)
                strategy = kMidfield;
            else if (role == kRoleCentreForward)
                strategy = kOffense;
        } else if (m.inPlay && !m.inSetPiece && m.designatedPossessionPlayer == p &&
                   (HumanGamerCount(Own()) == 0 || (!ExternalControllerActive(w, p) && ps.base.externalController >= 0)) &&
                   role != kRoleGoalkeeper) {
            onTheBall = ps.timeToBallMs < 1000;
            extraHaste = false;
        } else if (m.inPlay && !m.inSetPiece && role == kRoleGoalkeeper) {
            CalculateIfBallIsBoundForGoal();
            const bool bound = eliza->ballBoundForGoal;
            if (bound) manual = true;
            if (p != m.designatedPossessionPlayer) manual = true;
            GoalieRequestInput(manualDir, manualVel);
            if (!ctl.hasUniquePossession || ctl.possessionAmount < 3.4f)
                KeeperDeflectCommand(!bound && ctl.possessionAmount > 1.3f);
            onTheBall = ps.timeToBallMs < 1000 && m.designatedPossessionPlayer == p;
        }
        if (strategy >= 0) FieldStrategyRequestInput(strategy, rawDir, rawVel);
        if (onTheBall) GetOnTheBallCommands(rawDir, rawVel);
        bool forceMagnet = m.inPlay && !m.inSetPiece && (AI().endApplyTeamPressureMs > m.actualTimeMs && AI().teamPressurePlayer == p) &&
                           !ctl.teamHasBestPossession && m.designatedPossessionPlayer != p && role != kRoleGoalkeeper;
        ctl.inputDirection = rawDir;
        ctl.inputVelocityFloat = rawVel;
        eliza->lastDesiredDirection = rawDir.Length() != 0 ? rawDir : Dir();
        eliza->lastDesiredVelocity = rawVel;
        if (m.inPlay && !m.inSetPiece) {
            BallControlCommand();
            TrapCommand();
            InterfereCommand(false);
            SlidingCommand();
        }
        if (!manual && m.inPlay && !m.inSetPiece) {
            const int o = Opp().designatedTeamPossessionPlayer;
            if (p != m.designatedPossessionPlayer) {
                float mind = GetMindSet(DynamicRole());
                float hunt = 10.0f + (1.0f - mind) * 10.0f;
                hunt *= 0.5f * ps.base.fatigueFactorInverse +
                        0.5f * (1.0f - NormalizedClamp(PlayerAverageVelocity(w, p, 10), kIdleVelocity, kSprintVelocity));
                hunt *= 0.3f + TeamDifficulty(w, teamID) * 0.7f;
                if (forceMagnet) {
                    ctl.inputDirection = Vec3(side * kPitchHalfLength, 0, 0) - Pos();
                    ctl.inputVelocityFloat = kIdleVelocity;
                    ctl.inputDirection.Normalize(Dir());
                } else if (!ctl.teamHasBestPossession && ps.manMarking < 0 &&
                           ((Pos(o) + Mov(o) * 0.12f) - (Pos() + Mov() * 0.04f)).Length() < hunt) {
                    if (p == Own().designatedTeamPossessionPlayer && ctl.possessionAmount > 0.8f) {
                        forceMagnet = true;
                        extraHaste = true;
                    }
                    PlayerList closest = GetClosestPlayers(w, c, teamID, Pos(o) + Mov(o) * 0.1f, false, 2);
                    bool close = false;
                    for (int i = 0; i < closest.count; i++)
                        if (closest[i] == p) {
                            close = true;
                            break;
                        }
                    if (close) {
                        Vec3 dp = GetDefendPosition(o);
                        if (NeedDefendingMovement(side, Pos(), dp)) {
                            ctl.inputDirection = (dp - Pos()).Normalized(ctl.inputDirection);
                            ctl.inputVelocityFloat = Clamp((dp - Pos()).Length() * kDistanceToVelocity, 0.0f, kSprintVelocity);
                            forceMagnet = true;
                        }
                    }
                }
            }
            ctl.inputVelocityFloat = RangeVelocity(ctl.inputVelocityFloat);
            MovementCommand(forceMagnet, extraHaste);
        } else {
            PlayerCommand cmd = DefaultPlayerCommand();
            cmd.useDesiredMovement = true;
            cmd.desiredDirection = manualDir;
            cmd.desiredVelocityFloat = manualVel;
            cmd.useDesiredLookAt = true;
            cmd.desiredLookAt = Pos() + (MentalBall(40).Get2D() - Pos()).Normalized(0) * 10.0f;
            q.push_back(cmd);
        }
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

// The commands of a gamer's player: the armed action, then ball control, trap, interference and a
// movement that follows the stick (steady direction) with the default gameplay settings.
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
    auto resetAction = [&]() {
        hc.actionMode = 0;
        hc.gaugeMs = 0;
        hc.actionBufferTimeMs = 0;
    };
    ai.k = MentalImageIndex(w, ctl.mentalImageTime);
    ps.desiredTimeToBallMs = 0;
    ctl.opponentPlayer = TeamBestPossessionPlayer(w, 1 - t);
    ctl.timeNeededMs = (float)ps.timeToBallMs;
    Vec3 rawDir;
    float rawVel = 0;
    HumanGetKeyboardInput(w, p, rawDir, rawVel);
    ctl.inputDirection = rawDir;
    ctl.inputVelocityFloat = rawVel;
    const AnimationState &cur = Hum(w, p).anim;
    const int fn = cur.functionType;
    const bool touchPending = cur.frameNum < cur.touchFrame;
    if (hc.actionMode == 2 && IsPassOrShot(fn) && !touchPending) resetAction();
    if (hc.actionMode == 1 && (fn == kFnSliding || fn == kFnInterfere) && !touchPending) resetAction();
    if (hc.actionMode == 2 && hc.actionButton == kBtnShot && b[kBtnShortPass] && !m.inSetPiece) resetAction();
    if (hc.actionMode == 2 && hc.actionButton == kBtnHighPass && b[kBtnShortPass] && !m.inSetPiece) resetAction();
    if (hc.actionMode == 2 && !m.inSetPiece &&
        (hc.actionBufferTimeMs > 2000 || ps.timeToBallMs > ps.timeToBallPreviousMs + 700 || fn == kFnInterfere))
        resetAction();
    if (hc.actionMode == 1 && hc.actionBufferTimeMs > 1000) resetAction();
    if (hc.actionMode == 2) {
        if (!b[hc.actionButton] || (b[hc.actionButton] && hc.gaugeMs > 500) ||
            (!ps.hasPossession && !m.inSetPiece && hc.actionBufferTimeMs > 0)) {
            const int baseMs = 60;
            float gauge = (float)(hc.gaugeMs - baseMs) * (1.0f / float(1000 - baseMs));
            gauge = Clamp(gauge, 0.0f, 1.0f);
            auto pass = [&](int type, float exponent, float autoDir, float autoPower) {
                PlayerCommand cmd = DefaultPlayerCommand();
                cmd.desiredFunctionType = type;
                TouchInformation &ti = cmd.touchInfo;
                ti.inputDirection = ctl.inputDirection;
                ti.inputPower = Clamp(libm::powf(gauge, exponent), 0.01f, 1.0f);
                ti.autoDirectionBias = autoDir;
                ti.autoPowerBias = autoPower;
                AimPass(w, p, type, ti.inputDirection, ti.inputPower, ti.autoDirectionBias, ti.autoPowerBias, ti.desiredDirection,
                        ti.desiredPower, ti.targetPlayer, -1);
                q.push_back(cmd);
            };
            // GRF: the exponents and biases are the default gameplay settings.
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
                // One call site for the three passes, so that matches of a wavefront passing in
                // different ways run the pass search together.
                const int type = hc.actionButton == kBtnShortPass ? kFnShortPass
                                 : hc.actionButton == kBtnLongPass ? kFnLongPass
                                                                   : kFnHighPass;
                const float exponent = type == kFnShortPass ? 0.7f : type == kFnLongPass ? 0.65f : 0.55f;
                const float autoDir = type == kFnShortPass ? 0.4f : 0.2f;
                const float autoPower = type == kFnHighPass ? 0.5f : 0.7f;
                pass(type, exponent, autoDir, autoPower);
            } else if (hc.actionButton == kBtnShot) {
                PlayerCommand cmd = DefaultPlayerCommand();
                cmd.desiredFunctionType = kFnShot;
                cmd.desiredVelocityFloat = ctl.inputVelocityFloat;
                cmd.touchInfo.inputDirection = ctl.inputDirection;
                cmd.touchInfo.autoDirectionBias = 1.0f;
                cmd.touchInfo.desiredDirection =
                    AimShot(w, p, cmd.touchInfo.inputDirection, cmd.touchInfo.autoDirectionBias);
                cmd.touchInfo.desiredPower = Clamp(libm::powf(gauge, 0.6f), 0.01f, 1.0f);
                q.push_back(cmd);
            }
        }
    } else if (hc.actionMode == 1) {
        if (b[hc.actionButton]) {
            if (hc.actionButton == kBtnSliding) {
                PlayerCommand cmd = DefaultPlayerCommand();
                cmd.desiredFunctionType = kFnSliding;
                cmd.useDesiredMovement = true;
                cmd.desiredDirection = ctl.inputDirection;
                cmd.desiredVelocityFloat = ctl.inputVelocityFloat;
                cmd.useDesiredLookAt = true;
                cmd.desiredLookAt = ai.Pos() + ai.Mov() * 0.1f + cmd.desiredDirection * 10.0f;
                q.push_back(cmd);
            }
            if (hc.actionButton == kBtnTeamPressure) TeamApplyTeamPressure(w, c, t);
            if (hc.actionButton == kBtnKeeperRush) TeamApplyKeeperRush(w, t);
        } else {
            hc.actionMode = 0;
        }
    }
    if ((m.inSetPiece && tai.taker == p && (hc.actionMode != 2 || (hc.actionMode == 2 && b[hc.actionButton]) || m.ballRetainer == p)) ||
        (m.inSetPiece && tai.taker != p && m.ballRetainer < 0)) {
        ai.SetPieceCommand();
        return true;
    }
    Vec3 savedNonsteady = ctl.inputDirection;
    ctl.inputDirection = hc.steadyDirection;
    if (m.inPlay && !m.inSetPiece) {
        bool idleTurn = b[kBtnDribble];
        bool knockOn = b[kBtnDribble] && b[kBtnSprint];
        Vec3 savedDir = ctl.inputDirection;
        float savedVel = ctl.inputVelocityFloat;
        if (hc.actionMode == 2) {
            float dot = ai.Dir().Dot(ctl.inputDirection) * 0.5f + 0.5f;
            if (dot < 0) dot = 0;
            if (Sp(w, p).velocityCat != kVelIdle)
                ctl.inputDirection = (ai.Dir() * 1.0f + ctl.inputDirection * 0.0f).Normalized(ctl.inputDirection);
            dot = libm::powf(dot, 1.5f);
            dot = dot * 0.8f + 0.2f;
            dot *= 0.9f;
            ctl.inputVelocityFloat = ai.FloatVelocity() * dot;
        }
        ai.BallControlCommand(idleTurn, knockOn, true, false);
        ai.TrapCommand(idleTurn, knockOn);
        if (hc.actionMode == 2) {
            ctl.inputDirection = savedDir;
            ctl.inputVelocityFloat = savedVel;
        }
        ai.InterfereCommand(b[kBtnPressure]);
    }
    bool forceMagnet = false, extraHaste = false;
    if ((hc.actionMode != 2 && b[kBtnPressure]) || hc.actionMode == 2) forceMagnet = extraHaste = true;
    ai.MovementCommand(forceMagnet, extraHaste);
    if (!q.empty()) {
        PlayerCommand &cmd = q.back();
        if (!w.scenario.useMagnet) {
            cmd.desiredDirection = ctl.inputDirection;
            cmd.desiredVelocityFloat = ctl.inputVelocityFloat;
            if (cmd.desiredVelocityFloat < kIdleDribbleSwitch)
                cmd.desiredDirection = (ai.MentalBall(500).Get2D() - ai.Pos()).Normalized(ctl.inputDirection);
            cmd.desiredLookAt = ai.MentalBall(500).Get2D();
        }
        if (m.inPlay && !m.inSetPiece && b[kBtnDribble] && b[kBtnSprint] && !ctl.hasBestPossession) {
            cmd.desiredDirection = ctl.inputDirection;
            cmd.desiredVelocityFloat = ctl.inputVelocityFloat;
        }
    }
    ctl.inputDirection = savedNonsteady;
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
