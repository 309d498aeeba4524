// SPDX-License-Identifier: Apache-2.0
// Restates game logic of cuju (Copyright 2026 The cuju Authors), a reimplementation of Google
// Research Football (Copyright 2019 Google LLC); see NOTICE.
// The referee (half time, balls out of play, fouls, offside, the start of each set piece), the
// collisions of the ball with the players and of the players with each other, and the record of a
// touch. Semantics: include/cuju/simulation/referee.h:15-353,
// include/cuju/simulation/collisions.h:17-608, include/cuju/simulation/ball_touch.h:128-141.
#pragma once

#include "officials.h"

namespace eng {

// Defined with the set pieces.
HDN bool LeftTeamStartsNearerBall(const World &w);
HDN bool RefereeRestart(World &w, const Ctx &c, int setPiece);

enum MatchPhase { kPreMatch, kFirstHalf, kSecondHalf };

// GRF: the team processed first counts as the last to touch before any touch.
HD int MatchLastTouchTeam(const World &w) {
    return w.match.lastTouchTeamID != -1 ? w.match.lastTouchTeamID : w.FirstTeamID();
}
HD int MatchLastTouchPlayer(const World &w) { return TeamByID(w, MatchLastTouchTeam(w)).lastTouchPlayer; }
HD int StaticSide(int teamID) { return teamID == 0 ? -1 : 1; }

// The position in the fixed frame of the pitch, in which team 0 starts on side -1.
HD Vec3 PitchPosition(const World &w, int p) {
    Vec3 pos = Sp(w, p).position;
    const int t = w.playerTeamID[p];
    const int side = w.flags.teamSide[t];
    if (!(t == 0 ? side == -1 : side == 1)) pos.Mirror();
    return pos;
}

// Advances the clocks by `ms`; the match clock runs at the scenario's pace while in play.
HDN void BumpActualTime(World &w, const Ctx &c, uint64_t ms) {
    MatchState &m = w.match;
    if (m.inPlay) m.matchTimeMs = (uint64_t)((float)m.matchTimeMs + ms * (1.0f / c.sd->matchDurationFactor));
    m.actualTimeMs += ms;
    if (m.goalScored) m.goalScoredTimer += ms;
    else m.goalScoredTimer = 0;
    if (m.inPlay && !m.inSetPiece) {
        // Stored relative to the team processed first; clamps keep std::max/min's tie operand.
        const float sign = w.FirstTeamID() == 1 ? -1.0f : 1.0f;
        float poss = m.possessionLastMinute * sign;
        const int t = w.playerTeamID[m.designatedPossessionPlayer] == 0 ? 0 : 1;
        const float delta = 0.001f * ms;
        if (t == 0) {
            float moved = poss - delta;
            poss = (moved < -60.0f) ? -60.0f : moved;
        } else {
            float moved = poss + delta;
            poss = (60.0f < moved) ? 60.0f : moved;
        }
        m.possessionLastMinute = poss * sign;
    }
}
HD void MatchSetMatchPhase(World &w, int phase) {
    w.match.matchPhase = phase;
    for (int p = 0; p < w.match.playerCount; p++) {
        PersonBase &b = w.match.players[p].base;
        if (!b.isActive) continue;
        b.fatigueFactorInverse = Clamp(b.fatigueFactorInverse + 1.0f, 0.01f, 1.0f);
    }
}
HD void ResetFoul(Foul &f) {
    f.foulPlayer = -1;
    f.foulType = 0;
    f.advantage = false;
    f.foulTime = 0;
    f.hasBeenProcessed = true;
}
// GRF without referee animations: the clock skips the wait of a stoppage at once.
HDN void RefereeStop(World &w, const Ctx &c, int setPiece, uint64_t extraPrepareMs = 0) {
    MatchState &m = w.match;
    RefereeBuffer &b = m.referee.buffer;
    m.inPlay = false;
    b.desiredSetPiece = setPiece;
    b.stopTime = m.actualTimeMs;
    b.prepareTime = m.actualTimeMs + 2000;
    BumpActualTime(w, c, 1900);
    if (extraPrepareMs) {
        b.prepareTime += extraPrepareMs;
        BumpActualTime(w, c, extraPrepareMs);
    }
    b.startTime = b.prepareTime + 2000;
}
// True when the foul stops play.
HDN bool RefereeCheckFoul(World &w, const Ctx &c) {
    MatchState &m = w.match;
    Referee &ref = m.referee;
    Foul &f = ref.foul;
    bool penalty = false;
    // The penalty area, 16.5 m deep and 20.15 m to each side, compared in double.
    if (f.foulType != 0 && (double)fabsf(f.foulPosition.v[1]) < 20.15 - (double)kLineHalfWidth &&
        (double)(f.foulPosition.v[0] * -StaticSide(w.playerTeamID[f.foulVictim])) >
            (double)kPitchHalfLength - 16.5 + (double)kLineHalfWidth)
        penalty = true;
    if (f.advantage) {
        if (penalty) {
            f.advantage = false;
        } else if (m.actualTimeMs - 600 > f.foulTime) {
            if (m.actualTimeMs - 3000 > f.foulTime) {
                f.foulPlayer = -1;
                f.foulType = 0;
            } else if (TeamByID(w, w.playerTeamID[f.foulVictim]).fadingTeamPossessionAmount < 1.0) {
                f.advantage = false;
            }
        }
    }
    if (f.foulType != 0 && !f.advantage && !f.hasBeenProcessed) {
        RefereeBuffer &b = ref.buffer;
        const uint64_t extra = f.foulType >= 2 ? 10000 : 0;
        if (!penalty) {
            RefereeStop(w, c, kModeFreeKick, extra);
            b.restartPos = f.foulPosition;
        } else {
            RefereeStop(w, c, kModePenalty, extra);
            b.restartPos = Vec3((float)(((double)kPitchHalfLength - 11.0) * StaticSide(w.playerTeamID[f.foulPlayer])), 0, 0);
        }
        b.teamID = w.playerTeamID[f.foulVictim];
        b.active = true;
        Player &off = m.players[f.foulPlayer];
        // 2 is a yellow card, 3 a red one.
        if (f.foulType == 2) {
            off.cards++;
            off.cardEffectiveTimeMs = m.actualTimeMs + 6000;
        }
        if (f.foulType == 3) {
            off.cards += 3;
            off.cardEffectiveTimeMs = m.actualTimeMs + 6000;
        }
        f.hasBeenProcessed = true;
        return true;
    }
    return false;
}

HDN bool RefereeProcess(World &w, const Ctx &c) {
    ENG_SCOPE(6);
    MatchState &m = w.match;
    Referee &ref = m.referee;
    RefereeBuffer &b = ref.buffer;
    Foul &f = ref.foul;
    const Scenario &sc = w.scenario;
    if (m.inPlay && !m.inSetPiece) {
        Vec3 bp = BallPredict(m.ball, 0);
        // GRF: half time is an `int` product that wraps; after a wrap to a negative product the
        // unsigned comparison never comes true.
        const int64_t halfTime = (int32_t)((uint32_t)1800 * (uint32_t)sc.secondHalf);
        if (m.matchTimeMs >= (uint64_t)halfTime && m.matchPhase == kFirstHalf) {
            m.inPlay = false;
            b.desiredSetPiece = kModeKickOff;
            b.stopTime = m.actualTimeMs;
            b.prepareTime = b.stopTime + 100;
            b.startTime = b.prepareTime + 200;
            b.restartPos = sc.ballPosition;
            b.active = true;
            b.endPhase = true;
            b.teamID = LeftTeamStartsNearerBall(w) ? 1 : 0;
            b.setPieceTeam = TeamSlot(w, b.teamID);
            b.taker = -1;
            ResetFoul(f);
            MatchSetMatchPhase(w, kSecondHalf);
        }
        if (sc.reverseTeamProcessing) bp.Mirror();
        if ((double)fabsf(bp.v[0]) > (double)(kPitchHalfLength + kLineHalfWidth) + 0.11 || m.goalScored) {
            f.advantage = false;
            bool isFoul = false;
            if (!m.goalScored) isFoul = RefereeCheckFoul(w, c);
            else f.foulType = 0;
            if (!isFoul) {
                m.inPlay = false;
                const int lastTeam = MatchLastTouchTeam(w);
                const int lastSide = StaticSide(lastTeam);
                if (m.goalScored) {
                    b.desiredSetPiece = kModeKickOff;
                    b.stopTime = m.actualTimeMs;
                    b.prepareTime = m.actualTimeMs + 500;
                    BumpActualTime(w, c, 400);
                    b.startTime = b.prepareTime + 500;
                    b.restartPos = Vec3(0, 0, 0);
                    b.teamID = w.FirstTeamID();
                    // `lastGoalTeam` is a slot; the other slot kicks off.
                    b.setPieceTeam = 1 - m.lastGoalTeam;
                } else if ((bp.v[0] > 0 && lastSide > 0) || (bp.v[0] < 0 && lastSide < 0)) {
                    RefereeStop(w, c, kModeCorner);
                    b.restartPos = Vec3(kPitchHalfLength * lastSide, bp.v[1] > 0 ? kPitchHalfWidth : -kPitchHalfWidth, 0);
                    b.teamID = 1 - lastTeam;
                } else {
                    RefereeStop(w, c, kModeGoalKick);
                    b.restartPos = Vec3((float)((double)kPitchHalfLength * 0.92 * -lastSide), 0, 0);
                    b.teamID = 1 - lastTeam;
                }
                b.active = true;
            }
        }
        if (ref.afterSetPieceRelaxTimeMs == 0 &&
            (double)fabsf(bp.v[1]) > (double)(kPitchHalfWidth + kLineHalfWidth) + 0.11) {
            f.advantage = false;
            if (!RefereeCheckFoul(w, c)) {
                m.inPlay = false;
                b.teamID = 1 - MatchLastTouchTeam(w);
                RefereeStop(w, c, kModeThrowIn);
                b.restartPos.v[0] = Clamp(bp.v[0], -kPitchHalfLength + 0.6f, kPitchHalfLength - 0.6f);
                if (bp.v[1] > 0) b.restartPos.v[1] = kPitchHalfWidth;
                if (bp.v[1] <= 0) b.restartPos.v[1] = -kPitchHalfWidth;
                b.restartPos.v[2] = 0;
                b.active = true;
            }
        }
        RefereeCheckFoul(w, c);
    } else if (!m.inPlay && !m.inSetPiece && b.active) {
        if (b.prepareTime == m.actualTimeMs) {
            if (b.endPhase) {
                if (m.matchPhase == kPreMatch) MatchSetMatchPhase(w, kFirstHalf);
                b.endPhase = false;
            }
            Rng{w.rng}.Seed(sc.gameEngineRandomSeed);
            if (!RefereeRestart(w, c, b.desiredSetPiece)) return false;
        }
        if (b.startTime == m.actualTimeMs) {
            m.inPlay = true;
            m.inSetPiece = true;
        }
    }
    if (m.inSetPiece) {
        bool taken = b.desiredSetPiece == kModeKickOff;
        if (!taken) {
            if (b.taker < 0) return Fail("the set piece has no taker");
            const AnimationState &ta = Hum(w, b.taker).anim;
            taken = ta.touchFrame != -1 && !(ta.frameNum < ta.touchFrame);
        }
        if (taken) {
            b.active = false;
            m.inSetPiece = false;
            TeamByID(w, 0).ai.setPieceType = kModeNormal;
            TeamByID(w, 1).ai.setPieceType = kModeNormal;
            ref.afterSetPieceRelaxTimeMs = 400;
            f.foulPlayer = -1;
            f.foulType = 0;
            if (m.matchPhase == kPreMatch) MatchSetMatchPhase(w, kFirstHalf);
        }
    }
    if (ref.afterSetPieceRelaxTimeMs > 0) ref.afterSetPieceRelaxTimeMs -= 10;
    return true;
}

// Offside records of a touch: players of the touching team beyond the defenders' line at the touch.
HDN bool RefereeBallTouched(World &w, const Ctx &c) {
    MatchState &m = w.match;
    Referee &ref = m.referee;
    RefereeBuffer &b = ref.buffer;
    if (!w.scenario.offsides) return true;
    const int lt = m.lastTouchTeamID;
    if (lt == -1) return true;
    if (m.inPlay && !m.inSetPiece && !b.active && TeamActivePlayers(w, 1 - lt).size() > 1) {
        const int owner = MatchLastTouchPlayer(w);
        for (int i = 0; i < ref.offsidePlayers.count; i++) {
            if (ref.offsidePlayers[i] != owner) continue;
            ref.foul.advantage = false;
            if (!RefereeCheckFoul(w, c)) {
                RefereeStop(w, c, kModeFreeKick);
                b.restartPos = PitchPosition(w, owner);
                b.teamID = 1 - lt;
                b.active = true;
            }
        }
    }
    ref.offsidePlayers.count = 0;
    if (m.inPlay && (!b.active || (b.desiredSetPiece != kModeThrowIn && b.desiredSetPiece != kModeCorner))) {
        // GRF: a fresh image, so the defenders and the ball enter as they are this tick.
        ImageList im;
        PlayerList def = TeamActivePlayers(w, 1 - lt);
        for (int i = 0; i < def.count; i++) {
            const SpatialState &s = Sp(w, def[i]);
            im.push_back(PlayerImagePos{s.position, s.movement, m.players[def[i]].dynamicFormationEntry.role});
        }
        const int side = TeamDynamicSide(w, lt);
        float line = OffsideLineFromImages(im, BallPredict(m.ball, 0), TeamDynamicSide(w, 1 - lt), 0);
        const int toucher = TeamByID(w, lt).lastTouchPlayer;
        PlayerList att = TeamActivePlayers(w, lt);
        for (int i = 0; i < att.count; i++) {
            if (att[i] == toucher) continue;
            if (Sp(w, att[i]).position.v[0] * side < line * side) ref.offsidePlayers.push_back(att[i]);
        }
    }
    return true;
}

HD bool TeamSetLastTouchPlayer(World &w, const Ctx &c, int p, int touchType) {
    const int t = w.playerTeamID[p];
    TeamByID(w, t).lastTouchPlayer = p;
    Player &ps = w.match.players[p];
    ps.base.lastTouchTimeMs = w.match.actualTimeMs;
    ps.base.lastTouchType = touchType;
    w.match.lastTouchTeamIDs[touchType] = t;
    w.match.lastTouchTeamID = t;
    return RefereeBallTouched(w, c);
}

// ---- collisions --------------------------------------------------------------------------------------
HD PlayerList PlayersInProcessingOrder(const World &w) {
    PlayerList ps = TeamActivePlayers(w, w.FirstTeamID());
    PlayerList o = TeamActivePlayers(w, 1 - w.FirstTeamID());
    for (int i = 0; i < o.count; i++) ps.push_back(o[i]);
    return ps;
}

HDN bool CheckBallCollisions(World &w, const Ctx &c) {
    ENG_SCOPE(5);
    MatchState &m = w.match;
    if (m.actualTimeMs <= (uint64_t)(uint32_t)(m.lastBodyBallCollisionTimeMs + 150)) return true;
    PlayerList ps = PlayersInProcessingOrder(w);
    Vec3 bounce;
    float bias = 0.0;
    int bounces = 0;
    for (int pi = 0; pi < ps.count; pi++) {
        const int p = ps[pi];
        const int t = w.playerTeamID[p];
        float oppBias = TeamLastTouchBias(w, 1 - t, 200);
        float ownBias = GetLastTouchBias(w, p, 200);
        if (!(ownBias <= 0.01f && oppBias > 0.01f)) continue;
        Player &pl = m.players[p];
        const Humanoid &h = pl.base.humanoid;
        const int fn = h.anim.functionType;
        bool collisionAnim = fn == kFnMovement || fn == kFnTrip || fn == kFnSliding || fn == kFnInterfere || fn == kFnDeflect;
        bool onlyUnexpected = fn == kFnInterfere || fn == kFnDeflect;
        bool unexpected = false;
        if (onlyUnexpected) {
            int k = MentalImageIndex(w, GetReactionTimeMs(w, c, p) + h.anim.frameNum * 10);
            if ((MentalBallPrediction(w, k, 1000) - BallPredict(m.ball, 1000)).Length() > 0.5f) unexpected = true;
        }
        if (!(collisionAnim && !pl.hasUniquePossession && onlyUnexpected == unexpected)) continue;
        float sizeOffset = -0.1f;
        if (!pl.hasPossession) sizeOffset += 0.03f;
        else sizeOffset -= 0.03f;
        if (fn == kFnSliding || fn == kFnInterfere) sizeOffset += 0.1f;
        if (fn == kFnDeflect) sizeOffset += 0.2f;
        if (!(((h.spatial.position + Vec3(0, 0, 0.8f)) - BallPredict(m.ball, 0)).Length() < 2.5f)) continue;
        const Skeleton &sk = c.skeletons[p];
        Derived der[kHumanoidNodes];
        DeriveNodes(sk, h.nodes, der);
        for (int n = 0; n < sk.nodeCount; n++) {
            for (int g = 0; g < sk.nodes[n].geometryCount; g++) {
                WorldGeometry wg = GeometryWorld(sk.nodes[n].geometries[g], der[n]);
                float radius = 0.11f + sizeOffset;
                if (!wg.box.Intersects(BallPredict(m.ball, 0), radius)) continue;
                if (p == TeamByID(w, t).designatedTeamPossessionPlayer && MatchLastTouchBias(w, 200) < 0.01f) {
                    pl.triggerControlledBallCollision = true;
                } else {
                    float mb = oppBias * 0.8f + 0.2f;
                    bounce += (BallPredict(m.ball, 0) - wg.position).Normalized(Vec3(0)) * mb + h.spatial.movement * (1.0f - mb);
                    bounces++;
                    if (!TeamSetLastTouchPlayer(w, c, p, kTouchAccidental)) return false;
                    Vec3 center = wg.box.Center();
                    bias += (1.0f - Clamp(((BallPredict(m.ball, 0) - center).Length() - radius) / wg.box.Radius(), 0.0f, 1.0f)) *
                                0.9f +
                            0.1f;
                }
            }
        }
    }
    if (bias > 0.0f) {
        bounce /= Vec3(bounces * 1.0f);
        bounce.v[2] *= 0.6f;
        bounce.Normalize();
        Vec3 cur = m.ball.momentum;
        Vec3 full = (bounce * 6.0f) + (bounce * cur.Length() * 0.6f) + (cur * -0.2f);
        bias = Clamp(bias, 0.0f, 1.0f);
        bias = bias * 0.5f + 0.5f;
        Vec3 res = full * bias + cur * (1.0f - bias);
        if (res.Length() > cur.Length()) res = res.Normalized(0) * cur.Length();
        res *= 0.7f;
        BallTouch(w, c, res);
        // GRF: the arguments evaluate right to left: z, then y, then x.
        float rz = RandomInRange(w, -30, 30);
        float ry = RandomInRange(w, -30, 30);
        float rx = RandomInRange(w, -30, 30);
        BallSetRotation(w, rx, ry, rz, 0.5f * bias);
        m.lastBodyBallCollisionTimeMs = (uint32_t)m.actualTimeMs;
    }
    return true;
}

HDN void RefereeTripNotice(World &w, int tripped, int tripping, int tackleType) {
    MatchState &m = w.match;
    Referee &ref = m.referee;
    if (ref.buffer.active) return;
    const Humanoid &hd = Hum(w, tripped), &hg = Hum(w, tripping);
    const int td = w.playerTeamID[tripped], tg = w.playerTeamID[tripping];
    Foul &f = ref.foul;
    if (tackleType == 2) {
        if ((double)TeamByID(w, td).fadingTeamPossessionAmount > 1.1 &&
            (hg.anim.functionType == kFnInterfere || hg.anim.functionType == kFnSliding) &&
            (double)(hd.spatial.position - BallPredict(m.ball, 0).Get2D()).Length() < 2.0 && tg != td) {
            f.foulType = 1;
            f.advantage = true;
            f.foulPlayer = tripping;
            f.foulVictim = tripped;
            f.foulTime = m.actualTimeMs;
            f.foulPosition = PitchPosition(w, tripped);
            f.hasBeenProcessed = false;
        }
    } else if (tackleType == 3 && (tripping != f.foulPlayer || f.foulType == 0)) {
        if (m.actualTimeMs - m.players[tripping].base.lastTouchTimeMs > 600 && hg.anim.functionType == kFnSliding &&
            tg != td && (double)(BallPredict(m.ball, 0) - hd.spatial.position).Length() < 8.0) {
            float severity = 1.0;
            if (hg.anim.touchFrame != -1) {
                // The frame difference divides in double, the clamp takes floats, the power is double.
                const int tf = hg.anim.touchFrame, cf = hg.anim.frameNum;
                float timing = Clamp((float)(fabs((double)(tf - cf)) / tf), 0.0, 1.0);
                severity = (float)(libm::pow((double)timing, 0.7) * 0.5);
                severity = (float)(severity +
                                   NormalizedClamp((BallPredict(m.ball, 0) - hg.anim.touchPos).Length(), 0.0, 2.0) * 0.5);
            }
            // GRF: `dot * 0.5 + 0.5` adds as one double term.
            severity = (float)(severity +
                               ((hd.spatial.position - hg.spatial.position).Normalized(0).Dot(hd.spatial.directionVec) * 0.5 + 0.5));
            if ((double)severity > 1.0) {
                f.foulType = 1;
                f.advantage = false;
                f.foulPlayer = tripping;
                f.foulVictim = tripped;
                f.foulTime = m.actualTimeMs;
                f.foulPosition = PitchPosition(w, tripped);
                f.hasBeenProcessed = false;
                if ((double)severity > 1.4) f.foulType = 2;
                if ((double)severity > 2.0) f.foulType = 3;
            }
        }
    }
}

HDN void TripMe(World &w, const Ctx &c, int p, const Vec3 &tripVector, int tripType) {
    if (w.match.ballRetainer == p) return;
    Humanoid &h = Hum(w, p);
    const Anim &a = c.A(h.anim.anim);
    if (a.incomingSpecialState != kStrEmpty || a.outgoingSpecialState != kStrEmpty) return;
    if (h.interruptAnim == kIntNone &&
        (h.anim.functionType != kFnTrip || (c.D(h.anim.anim).tripTypeIsOne && tripType > 1)) &&
        h.anim.functionType != kFnSliding) {
        h.interruptAnim = kIntTrip;
        h.tripDirection = tripVector;
        h.tripType = tripType;
    }
}


HD bool BoxesIntersect(const Aabb &a, const Aabb &o) {
    return (o.lo.v[0] < a.hi.v[0] && o.lo.v[1] < a.hi.v[1] && o.lo.v[2] < a.hi.v[2]) &&
           (o.hi.v[0] > a.lo.v[0] && o.hi.v[1] > a.lo.v[1] && o.hi.v[2] > a.lo.v[2]);
}
HDN void PlayerGeometries(const World &w, const Ctx &c, int p, PlayerGeometryList &out) {
    const Skeleton &sk = c.skeletons[p];
    Derived der[kHumanoidNodes];
    DeriveNodes(sk, Hum(w, p).nodes, der);
    out.clear();
    for (int n = 0; n < sk.nodeCount; n++)
        for (int g = 0; g < sk.nodes[n].geometryCount; g++) {
            const SkelGeometry &sg = sk.nodes[n].geometries[g];
            out.push_back(PlayerGeometry{sg.footOrLowerLeg, GeometryWorld(sg, der[n])});
        }
}

HDN void CheckHumanoidCollision(World &w, const Ctx &c, int p1, int p2, PlayerBounceList &b1, PlayerBounceList &b2) {
    MatchState &m = w.match;
    const float distanceFactor = 0.72f;
    const float bounceRadius = 0.5f * distanceFactor;
    const float similarRadius = 0.8f * distanceFactor;
    const float similarExponent = 0.2f;
    const float similarForceFactor = 0.25f;
    auto S = [&](int p) -> const SpatialState & { return Sp(w, p); };
    auto stat = [&](int p, int s) { return GetStatistic(w, c, p, s); };
    auto fnOf = [&](int p) { return Hum(w, p).anim.functionType; };
    auto touchPending = [&](int p) { return Hum(w, p).anim.frameNum < Hum(w, p).anim.touchFrame; };
    auto designated = [&](int p) { return TeamByID(w, w.playerTeamID[p]).designatedTeamPossessionPlayer; };
    const Vec3 pos1 = S(p1).position, pos2 = S(p2).position;
    float dist = (pos1 - pos2).Length();
    float bounceBias = 0.0f;
    Vec3 bv;
    float back1 = 0.5f, back2 = 0.5f;
    if (dist < bounceRadius * 2.0f || dist < (bounceRadius + similarRadius) * 2.0f) {
        bv = (pos1 - pos2).Normalized(Vec3(0, -1, 0));
        Vec3 face1 = S(p1).directionVec.Rotated2D(S(p1).relBodyAngle.value() * 0.7f);
        Vec3 face2 = S(p2).directionVec.Rotated2D(S(p2).relBodyAngle.value() * 0.7f);
        back1 = Clamp(face1.Dot(bv) * 0.5f + 0.5f, 0.0f, 1.0f);
        back2 = Clamp(face2.Dot(-bv) * 0.5f + 0.5f, 0.0f, 1.0f);
        auto ballDistanceDifference = [&]() {
            float d1 = (BallPredict(m.ball, 10).Get2D() - S(p1).position).Length();
            float d2 = (BallPredict(m.ball, 10).Get2D() - S(p2).position).Length();
            float c2 = MinF(d2, 1.2f), c1 = MinF(d1, 1.2f);
            return Clamp(c2 - c1, -0.6f, 0.6f) * 1.0f;
        };
        if (dist < bounceRadius * 2.0f) {
            bounceBias += back1 * 0.8f;
            bounceBias -= back2 * 0.8f;
            float v1 = PlayerFloatVelocity(w, p1), v2 = PlayerFloatVelocity(w, p2);
            bounceBias -= Clamp(((v1 - v2) / kSprintVelocity) * 0.2f, -0.2f, 0.2f);
            if (touchPending(p1) && fnOf(p1) == kFnInterfere) bounceBias += 0.1f + 0.4f * stat(p1, kStatStandingTackle);
            if (touchPending(p1) && fnOf(p1) == kFnSliding) bounceBias += 0.1f + 0.4f * stat(p1, kStatSlidingTackle);
            if (touchPending(p2) && fnOf(p2) == kFnInterfere) bounceBias -= 0.1f + 0.4f * stat(p2, kStatStandingTackle);
            if (touchPending(p2) && fnOf(p2) == kFnSliding) bounceBias -= 0.1f + 0.4f * stat(p2, kStatSlidingTackle);
            if (p1 == m.designatedPossessionPlayer) bounceBias += 0.4f;
            if (p2 == m.designatedPossessionPlayer) bounceBias -= 0.4f;
            if (p1 == designated(p1) && p2 == designated(p2)) bounceBias += ballDistanceDifference();
            bounceBias += stat(p1, kStatBalance) * 1.0f;
            bounceBias -= stat(p2, kStatBalance) * 1.0f;
            bounceBias = Clamp(bounceBias, -1.0f, 1.0f);
            bounceBias *= 0.5f;
            float nb = bounceBias * 0.5f + 0.5f;
            Vec3 off1 = (pos1 - pos2).Normalized(0) * (bounceRadius - dist * 0.5f) * (1.0f - nb) * 2.0f;
            Vec3 off2 = (pos2 - pos1).Normalized(0) * (bounceRadius - dist * 0.5f) * nb * 2.0f;
            // The player on the ball is pushed aside towards the nearer of his two flanks.
            if (m.designatedPossessionPlayer == p2 && m.players[p2].hasPossession) {
                Vec3 l = pos2 + S(p2).directionVec.Rotated2D(0.3f * PI) * bounceRadius * 2;
                Vec3 r = pos2 + S(p2).directionVec.Rotated2D(-0.3f * PI) * bounceRadius * 2;
                Vec3 near = (pos1 - l).Length() < (pos1 - r).Length() ? l : r;
                off1 += NormalizedMaximum(near - pos1, 0.01f) * stat(p1, kStatBalance) * 0.3f;
            } else if (m.designatedPossessionPlayer == p1 && m.players[p1].hasPossession) {
                Vec3 l = pos1 + S(p1).directionVec.Rotated2D(0.3f * PI) * bounceRadius * 2;
                Vec3 r = pos1 + S(p1).directionVec.Rotated2D(-0.3f * PI) * bounceRadius * 2;
                Vec3 near = (pos2 - l).Length() < (pos2 - r).Length() ? l : r;
                off2 += NormalizedMaximum(near - pos2, 0.01f) * stat(p2, kStatBalance) * 0.3f;
            }
            NormalizeMaximum(off1, kSprintVelocity * 0.01f);
            NormalizeMaximum(off2, kSprintVelocity * 0.01f);
            OffsetPosition(w, p1, off1);
            OffsetPosition(w, p2, off2);
        }
        float similarBias = 0.0f;
        if (similarForceFactor > 0.0f && dist < (bounceRadius + similarRadius) * 2.0f) {
            float gap = dist - bounceRadius * 2.0f;
            float shell = (0.0f < gap) ? gap : 0.0f;
            similarBias += back1 * 0.8f;
            similarBias -= back2 * 0.8f;
            float v1 = PlayerFloatVelocity(w, p1), v2 = PlayerFloatVelocity(w, p2);
            similarBias -= Clamp(((v1 - v2) / kSprintVelocity) * 0.2f, -0.2f, 0.2f);
            if (p1 == m.designatedPossessionPlayer) similarBias += 0.6f;
            if (p2 == m.designatedPossessionPlayer) similarBias -= 0.6f;
            if (p1 == designated(p1) && p2 == designated(p2)) similarBias += ballDistanceDifference();
            similarBias += stat(p1, kStatBalance) * 1.0f;
            similarBias -= stat(p2, kStatBalance) * 1.0f;
            similarBias = Clamp(similarBias, -1.0f, 1.0f);
            similarBias *= 0.9f;
            float force = Clamp(1.0f - (shell / (similarRadius * 2.0f)), 0.0f, 1.0f);
            force = libm::powf(force, similarExponent);
            force *= similarForceFactor;
            float ns = similarBias * 0.5f + 0.5f;
            b1.push_back(PlayerBounce{p2, force * (1.0f - ns)});
            b2.push_back(PlayerBounce{p1, force * ns});
        }
        if (dist < bounceRadius * 2.0f) {
            float s1 = 0.0f, s2 = 0.0f;
            s1 += (1.0f - back1) * 1.0f;
            s2 += (1.0f - back2) * 1.0f;
            float v1 = PlayerFloatVelocity(w, p1), v2 = PlayerFloatVelocity(w, p2);
            s1 += NormalizedClamp(v1, kIdleVelocity, kSprintVelocity) * 1.0f;
            s2 += NormalizedClamp(v2, kIdleVelocity, kSprintVelocity) * 1.0f;
            if (m.players[p1].hasBestPossession) s1 += 1.0f;
            if (m.players[p2].hasBestPossession) s2 += 1.0f;
            const float balanceWeight = 3.0f;
            s1 += (1.0f - stat(p1, kStatBalance) * 1.0f) * balanceWeight;
            s2 += (1.0f - stat(p2, kStatBalance) * 1.0f) * balanceWeight;
            s1 += Clamp(Hum(w, p1).decayingPositionOffset.Length() * 10.0f, 0.0f, 1.0f);
            s2 += Clamp(Hum(w, p2).decayingPositionOffset.Length() * 10.0f, 0.0f, 1.0f);
            const float penetrationWeight = 6.0f;
            float pen = ((S(p1).position + S(p1).movement * 0.03f) - (S(p2).position + S(p2).movement * 0.03f)).Length();
            s1 += libm::powf(1.0f - NormalizedClamp(pen, 0.0f, bounceRadius * 2.0f), 0.4f) * penetrationWeight;
            s2 += libm::powf(1.0f - NormalizedClamp(pen, 0.0f, bounceRadius * 2.0f), 0.4f) * penetrationWeight;
            float d1 = (BallPredict(m.ball, 10).Get2D() - S(p1).position).Length();
            float d2 = (BallPredict(m.ball, 10).Get2D() - S(p2).position).Length();
            s1 += 1.0f - NormalizedClamp(d1, 0.0f, 0.7f);
            s2 += 1.0f - NormalizedClamp(d2, 0.0f, 0.7f);
            s1 /= 5.0f + balanceWeight + penetrationWeight;
            s2 /= 5.0f + balanceWeight + penetrationWeight;
            const float t0 = 0.38f, t1 = 0.48f, t2 = 0.58f;
            if (s1 > t0) {
                int tt = 0;
                if (s1 > t1) tt = 1;
                if (s1 > t2) tt = 2;
                if (tt > 0) {
                    TripMe(w, c, p1, (S(p1).movement * 0.1f + S(p2).movement * 0.06f + bv * 1.0f).Normalized(bv), tt);
                    RefereeTripNotice(w, p1, p2, tt);
                }
            }
            if (s2 > t0) {
                int tt = 0;
                if (s2 > t1) tt = 1;
                if (s2 > t2) tt = 2;
                if (tt > 0) {
                    TripMe(w, c, p2, (S(p2).movement * 0.1f + S(p1).movement * 0.06f - bv * 1.0f).Normalized(-bv), tt);
                    RefereeTripNotice(w, p2, p1, tt);
                }
            }
        }
    }
    auto frameOf = [&](int p) { return Hum(w, p).anim.frameNum; };
    auto framesOf = [&](int p) { return c.A(Hum(w, p).anim.anim).frameCount; };
    int tackle = 0;
    if ((fnOf(p1) == kFnSliding || fnOf(p1) == kFnInterfere) && frameOf(p1) > 5 && frameOf(p1) < 28) tackle += 1;
    if ((fnOf(p2) == kFnSliding || fnOf(p2) == kFnInterfere) && frameOf(p2) > 5 && frameOf(p2) < 28) tackle += 2;
    if (dist < 2.0f && tackle > 0 && tackle < 3) {
        const int tackler = tackle == 1 ? p1 : p2, victim = tackle == 1 ? p2 : p1;
        PlayerGeometryList &tg = c.ws->tackleGeometry[0], &vg = c.ws->tackleGeometry[1];
        PlayerGeometries(w, c, tackler, tg);
        PlayerGeometries(w, c, victim, vg);
        for (int i = 0; i < tg.count; i++) {
            Aabb box = tg[i].wg.box;
            box.lo += 0.1f;
            box.hi -= Vec3(0.1f);
            for (int j = 0; j < vg.count; j++) {
                if (!vg[j].footOrLowerLeg) continue;
                if (BoxesIntersect(box, vg[j].wg.box)) {
                    if (frameOf(tackler) > 10 && frameOf(tackler) < framesOf(tackler) - 6) {
                        int tt = fnOf(tackler) == kFnInterfere ? 1 : 3;
                        TripMe(w, c, victim, S(victim).directionVec, tt);
                        RefereeTripNotice(w, victim, tackler, tt);
                    }
                    break;
                }
            }
        }
    }
}

HDN bool CheckHumanoidCollisions(World &w, const Ctx &c) {
    ENG_SCOPE(17);
    PlayerList ps = PlayersInProcessingOrder(w);
    PlayerBounceList *const bounces = c.ws->bounces;
    for (int i = 0; i < ps.count; i++) bounces[i].clear();
    // A pair farther apart than both contact radii changes nothing, so only near pairs make the
    // call; the test is the one the pair's own check starts with, on the same values.
    const float bounceRadius = 0.5f * 0.72f, similarRadius = 0.8f * 0.72f;
    // The pairs read the positions from a copy gathered once, not from each player's spatial state
    // (one cache line per player, read again for every pair); a call moves only its two players,
    // whose copies it refreshes.
    Vec3 at[kPlayers];
    for (int i = 0; i < ps.count; i++) at[i] = Sp(w, ps[i]).position;
    for (int i = 0; i + 1 < ps.count; i++) {
        for (int j = i + 1; j < ps.count; j++) {
            const float dist = (at[i] - at[j]).Length();
            if (dist < bounceRadius * 2.0f || dist < (bounceRadius + similarRadius) * 2.0f) {
                CheckHumanoidCollision(w, c, ps[i], ps[j], bounces[i], bounces[j]);
                at[i] = Sp(w, ps[i]).position;
                at[j] = Sp(w, ps[j]).position;
            }
        }
    }
    for (int i = 0; i < ps.count; i++) {
        float total = 0.0f;
        for (int k = 0; k < bounces[i].count; k++) total += bounces[i][k].force;
        if (total > 0.0f) {
            Vec3 v;
            for (int k = 0; k < bounces[i].count; k++) {
                const PlayerBounce &b = bounces[i][k];
                v += (Sp(w, b.opponent).movement - Sp(w, ps[i]).movement) * b.force * (b.force / total);
            }
            OffsetPosition(w, ps[i], v * 0.01f * 1.0f);
        }
    }
    return true;
}

}  // namespace eng
