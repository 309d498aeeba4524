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
// ---- fouls -------------------------------------------------------------------------------------
// Whether the foul lies in the penalty area of the victim's opponents: 16.5 m deep and 20.15 m to
// each side of the centre line, the line's half width inside (compared in double).
HD bool FoulInPenaltyArea(const World &w, const Foul &f) {
    return f.foulType != 0 && (double)fabsf(f.foulPosition.v[1]) < 20.15 - (double)kLineHalfWidth &&
           (double)(f.foulPosition.v[0] * -StaticSide(w.playerTeamID[f.foulVictim])) >
               (double)kPitchHalfLength - 16.5 + (double)kLineHalfWidth;
}
// An advantage ends in the penalty area at once; 600 ms after the foul, when the victim's team no
// longer holds the ball; and 3 s after it the foul is forgotten.
HD void ReviewAdvantage(World &w, Foul &f, bool penalty) {
    const uint64_t now = w.match.actualTimeMs;
    if (!f.advantage) return;
    if (penalty) {
        f.advantage = false;
        return;
    }
    if (!(now - 600 > f.foulTime)) return;
    if (now - 3000 > f.foulTime) {
        f.foulPlayer = -1;
        f.foulType = 0;
    } else if (TeamByID(w, w.playerTeamID[f.foulVictim]).fadingTeamPossessionAmount < 1.0) {
        f.advantage = false;
    }
}
// A foul that stops play: a free kick where it happened or a penalty 11 m out (cards add 10 s to
// the stoppage) for the victim's team; a yellow card (type 2) adds one card, a red one (type 3)
// three, taking effect after 6 s.
HD void AwardFoul(World &w, const Ctx &c, Foul &f, bool penalty) {
    MatchState &m = w.match;
    RefereeBuffer &b = m.referee.buffer;
    const uint64_t extra = f.foulType >= 2 ? 10000 : 0;
    if (penalty) {
        RefereeStop(w, c, kModePenalty, extra);
        b.restartPos = Vec3((float)(((double)kPitchHalfLength - 11.0) * StaticSide(w.playerTeamID[f.foulPlayer])), 0, 0);
    } else {
        RefereeStop(w, c, kModeFreeKick, extra);
        b.restartPos = f.foulPosition;
    }
    b.teamID = w.playerTeamID[f.foulVictim];
    b.active = true;
    Player &offender = m.players[f.foulPlayer];
    if (f.foulType == 2 || f.foulType == 3) {
        offender.cards += f.foulType == 2 ? 1 : 3;
        offender.cardEffectiveTimeMs = m.actualTimeMs + 6000;
    }
    f.hasBeenProcessed = true;
}
// The referee's look at the pending foul: the advantage reviewed, then a foul without advantage
// not yet processed is awarded. True when it stops play.
HDN bool RefereeCheckFoul(World &w, const Ctx &c) {
    Foul &f = w.match.referee.foul;
    const bool penalty = FoulInPenaltyArea(w, f);
    ReviewAdvantage(w, f, penalty);
    if (f.foulType == 0 || f.advantage || f.hasBeenProcessed) return false;
    AwardFoul(w, c, f, penalty);
    return true;
}

// ---- the referee's tick -------------------------------------------------------------------------
// At half time (the match clock passing 1800 times the scenario's second-half value: GRF's `int`
// product, which wraps; after a wrap to a negative product the unsigned comparison never comes
// true) play stops for a kick-off by the team that did not start nearer the ball, with the foul
// cleared, and the second half begins.
HD void CheckHalfTime(World &w) {
    MatchState &m = w.match;
    RefereeBuffer &b = m.referee.buffer;
    const Scenario &sc = w.scenario;
    const int64_t halfTime = (int32_t)((uint32_t)1800 * (uint32_t)sc.secondHalf);
    if (!(m.matchTimeMs >= (uint64_t)halfTime && m.matchPhase == kFirstHalf)) return;
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
    ResetFoul(m.referee.foul);
    MatchSetMatchPhase(w, kSecondHalf);
}
// The ball beyond a goal line (`ball` on the fixed pitch, the ball's radius past the line) or a
// goal: unless a pending foul stops play first (none after a goal), a kick-off by the slot that
// conceded (after 400 ms; 500 ms to prepare, 500 more to start), a corner on the ball's side for
// the team that did not touch it last when that team's own goal line was crossed, else a goal
// kick 92% of the way out.
HD void CheckGoalLine(World &w, const Ctx &c, const Vec3 &ball) {
    MatchState &m = w.match;
    Referee &ref = m.referee;
    RefereeBuffer &b = ref.buffer;
    if (!((double)fabsf(ball.v[0]) > (double)(kPitchHalfLength + kLineHalfWidth) + 0.11 || m.goalScored)) return;
    ref.foul.advantage = false;
    if (m.goalScored) ref.foul.foulType = 0;
    else if (RefereeCheckFoul(w, c)) return;
    m.inPlay = false;
    const int lastTeam = MatchLastTouchTeam(w), lastSide = StaticSide(lastTeam);
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
    } else if ((ball.v[0] > 0 && lastSide > 0) || (ball.v[0] < 0 && lastSide < 0)) {
        RefereeStop(w, c, kModeCorner);
        b.restartPos = Vec3(kPitchHalfLength * lastSide, ball.v[1] > 0 ? kPitchHalfWidth : -kPitchHalfWidth, 0);
        b.teamID = 1 - lastTeam;
    } else {
        RefereeStop(w, c, kModeGoalKick);
        b.restartPos = Vec3((float)((double)kPitchHalfLength * 0.92 * -lastSide), 0, 0);
        b.teamID = 1 - lastTeam;
    }
    b.active = true;
}
// The ball beyond a touchline outside the relaxation after a set piece: unless a pending foul
// stops play first, a throw-in where it went out (0.6 m inside the goal lines) for the team that
// did not touch it last.
HD void CheckTouchLine(World &w, const Ctx &c, const Vec3 &ball) {
    MatchState &m = w.match;
    Referee &ref = m.referee;
    RefereeBuffer &b = ref.buffer;
    if (!(ref.afterSetPieceRelaxTimeMs == 0 && (double)fabsf(ball.v[1]) > (double)(kPitchHalfWidth + kLineHalfWidth) + 0.11)) return;
    ref.foul.advantage = false;
    if (RefereeCheckFoul(w, c)) return;
    m.inPlay = false;
    b.teamID = 1 - MatchLastTouchTeam(w);
    RefereeStop(w, c, kModeThrowIn);
    b.restartPos.v[0] = Clamp(ball.v[0], -kPitchHalfLength + 0.6f, kPitchHalfLength - 0.6f);
    b.restartPos.v[1] = ball.v[1] > 0 ? kPitchHalfWidth : -kPitchHalfWidth;
    b.restartPos.v[2] = 0;
    b.active = true;
}
// A set piece ends when it is taken: a kick-off at once, any other when its taker's animation
// reaches its touch. The teams return to normal play, the referee relaxes the touchlines for
// 400 ms and forgets the foul. False for a set piece without a taker.
HD bool EndSetPieceWhenTaken(World &w) {
    MatchState &m = w.match;
    Referee &ref = m.referee;
    RefereeBuffer &b = ref.buffer;
    bool taken = b.desiredSetPiece == kModeKickOff;
    if (!taken) {
        if (b.taker < 0) return Fail("the set piece has no taker");
        const AnimationState &ta = Hum(w, b.taker).anim;
        taken = ta.touchFrame != -1 && !(ta.frameNum < ta.touchFrame);
    }
    if (!taken) return true;
    b.active = false;
    m.inSetPiece = false;
    TeamByID(w, 0).ai.setPieceType = kModeNormal;
    TeamByID(w, 1).ai.setPieceType = kModeNormal;
    ref.afterSetPieceRelaxTimeMs = 400;
    ref.foul.foulPlayer = -1;
    ref.foul.foulType = 0;
    if (m.matchPhase == kPreMatch) MatchSetMatchPhase(w, kFirstHalf);
    return true;
}

// The referee's tick. In open play: half time, the goal line, the touchline, the pending foul.
// During a stoppage: the set piece is prepared at its preparation time (the world RNG reseeded;
// the first half begins at the match's opening kick-off) and play resumes, as a set piece, at its
// start time. Then a set piece in progress may end, and the relaxation runs down.
HDN bool RefereeProcess(World &w, const Ctx &c) {
    ENG_SCOPE(6);
    MatchState &m = w.match;
    Referee &ref = m.referee;
    RefereeBuffer &b = ref.buffer;
    if (m.inPlay && !m.inSetPiece) {
        Vec3 ball = BallPredict(m.ball, 0);
        CheckHalfTime(w);
        if (w.scenario.reverseTeamProcessing) ball.Mirror();
        CheckGoalLine(w, c, ball);
        CheckTouchLine(w, c, ball);
        RefereeCheckFoul(w, c);
    } else if (!m.inPlay && !m.inSetPiece && b.active) {
        if (b.prepareTime == m.actualTimeMs) {
            if (b.endPhase) {
                if (m.matchPhase == kPreMatch) MatchSetMatchPhase(w, kFirstHalf);
                b.endPhase = false;
            }
            Rng{w.rng}.Seed(w.scenario.gameEngineRandomSeed);
            if (!RefereeRestart(w, c, b.desiredSetPiece)) return false;
        }
        if (b.startTime == m.actualTimeMs) {
            m.inPlay = true;
            m.inSetPiece = true;
        }
    }
    if (m.inSetPiece && !EndSetPieceWhenTaken(w)) return false;
    if (ref.afterSetPieceRelaxTimeMs > 0) ref.afterSetPieceRelaxTimeMs -= 10;
    return true;
}

// ---- offside -----------------------------------------------------------------------------------
// A touch by a player recorded offside at its team's previous touch (in open play, no stoppage
// pending, more than one defender) gives the defending team a free kick where it stands, unless
// a pending foul stops play first.
HD void PunishOffside(World &w, const Ctx &c, int attackers) {
    MatchState &m = w.match;
    Referee &ref = m.referee;
    RefereeBuffer &b = ref.buffer;
    if (!(m.inPlay && !m.inSetPiece && !b.active && TeamActivePlayers(w, 1 - attackers).size() > 1)) return;
    const int owner = MatchLastTouchPlayer(w);
    for (int i = 0; i < ref.offsidePlayers.count; i++) {
        if (ref.offsidePlayers[i] != owner) continue;
        ref.foul.advantage = false;
        if (RefereeCheckFoul(w, c)) continue;
        RefereeStop(w, c, kModeFreeKick);
        b.restartPos = PitchPosition(w, owner);
        b.teamID = 1 - attackers;
        b.active = true;
    }
}
// The players of the touching team, the toucher aside, beyond the defenders' offside line at the
// touch (from the defenders and the ball as they are this tick, as GRF takes a fresh image), in
// play unless a throw-in or corner is pending.
HD void RecordOffsidePositions(World &w, int attackers) {
    MatchState &m = w.match;
    Referee &ref = m.referee;
    const RefereeBuffer &b = ref.buffer;
    ref.offsidePlayers.count = 0;
    if (!(m.inPlay && (!b.active || (b.desiredSetPiece != kModeThrowIn && b.desiredSetPiece != kModeCorner)))) return;
    ImageList defenders;
    const PlayerList def = TeamActivePlayers(w, 1 - attackers);
    for (int i = 0; i < def.count; i++) {
        const SpatialState &s = Sp(w, def[i]);
        defenders.push_back(PlayerImagePos{s.position, s.movement, m.players[def[i]].dynamicFormationEntry.role});
    }
    const int side = TeamDynamicSide(w, attackers);
    const float line = OffsideLineFromImages(defenders, BallPredict(m.ball, 0), TeamDynamicSide(w, 1 - attackers), 0);
    const int toucher = TeamByID(w, attackers).lastTouchPlayer;
    const PlayerList att = TeamActivePlayers(w, attackers);
    for (int i = 0; i < att.count; i++)
        if (att[i] != toucher && Sp(w, att[i]).position.v[0] * side < line * side) ref.offsidePlayers.push_back(att[i]);
}
// The referee's part of a touch, with offsides on: punish a touch by a player recorded offside,
// then record the offside positions at this touch.
HDN bool RefereeBallTouched(World &w, const Ctx &c) {
    if (!w.scenario.offsides) return true;
    const int attackers = w.match.lastTouchTeamID;
    if (attackers == -1) return true;
    PunishOffside(w, c, attackers);
    RecordOffsidePositions(w, attackers);
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

// Whether player p's body may deflect the ball this tick: the opponents touched it within 200 ms
// and p did not; p is in a movement, trip, sliding, interference or deflection (the last two only
// when the ball surprises it: the ball a second ahead, as p saw it its reaction time and frame
// ago, lies more than 0.5 m from where it will be); and p does not alone hold the ball.
// `opponentBias`: how recently the opponents touched it.
HD bool BodyMayDeflect(World &w, const Ctx &c, int p, float &opponentBias) {
    const MatchState &m = w.match;
    opponentBias = TeamLastTouchBias(w, 1 - w.playerTeamID[p], 200);
    const float ownBias = GetLastTouchBias(w, p, 200);
    if (!(ownBias <= 0.01f && opponentBias > 0.01f)) return false;
    const Player &pl = m.players[p];
    const Humanoid &h = pl.base.humanoid;
    const int fn = h.anim.functionType;
    const bool bodyAnimation = fn == kFnMovement || fn == kFnTrip || fn == kFnSliding || fn == kFnInterfere || fn == kFnDeflect;
    const bool onlySurprised = fn == kFnInterfere || fn == kFnDeflect;
    bool surprised = false;
    if (onlySurprised) {
        const int k = MentalImageIndex(w, GetReactionTimeMs(w, c, p) + h.anim.frameNum * 10);
        surprised = (MentalBallPrediction(w, k, 1000) - BallPredict(m.ball, 1000)).Length() > 0.5f;
    }
    return bodyAnimation && !pl.hasUniquePossession && onlySurprised == surprised;
}
// The margin by which p's body parts reach past the ball's radius: 0.1 m less, 0.03 m more off
// the ball (0.03 m less on it), 0.1 m more in a tackle, 0.2 m more in a deflection.
HD float BodyReach(const Player &pl) {
    const int fn = pl.base.humanoid.anim.functionType;
    float reach = -0.1f;
    if (!pl.hasPossession) reach += 0.03f;
    else reach -= 0.03f;
    if (fn == kFnSliding || fn == kFnInterfere) reach += 0.1f;
    if (fn == kFnDeflect) reach += 0.2f;
    return reach;
}
// The ball after bodies deflected it: along the mean bounce direction (its height at 60%), at
// 6 m/s plus 60% of its speed less a fifth of its momentum, blended with its momentum by the
// summed contact depth (half to all of it), never faster than it came, at 70%; spun by three
// draws (GRF evaluates the arguments right to left: z, then y, then x).
HD void DeflectBall(World &w, const Ctx &c, Vec3 bounce, int bounces, float depth) {
    MatchState &m = w.match;
    bounce /= Vec3(bounces * 1.0f);
    bounce.v[2] *= 0.6f;
    bounce.Normalize();
    const Vec3 cur = m.ball.momentum;
    const Vec3 full = (bounce * 6.0f) + (bounce * cur.Length() * 0.6f) + (cur * -0.2f);
    const float bias = Clamp(depth, 0.0f, 1.0f) * 0.5f + 0.5f;
    Vec3 res = full * bias + cur * (1.0f - bias);
    if (res.Length() > cur.Length()) res = res.Normalized(0) * cur.Length();
    res *= 0.7f;
    BallTouch(w, c, res);
    const float rz = RandomInRange(w, -30, 30);
    const float ry = RandomInRange(w, -30, 30);
    const float rx = RandomInRange(w, -30, 30);
    BallSetRotation(w, rx, ry, rz, 0.5f * bias);
    m.lastBodyBallCollisionTimeMs = (uint32_t)m.actualTimeMs;
}
// The ball against the players' bodies, at most every 150 ms, players in processing order. A
// body part of a player that may deflect it (within 2.5 m of its chest) touching the ball makes
// the team's designated player, when nobody touched the ball within 200 ms, control it;
// otherwise it records an accidental touch and adds a bounce (away from the part, blended with
// the player's movement by how recently the opponents touched) and a contact depth.
HDN bool CheckBallCollisions(World &w, const Ctx &c) {
    ENG_SCOPE(5);
    MatchState &m = w.match;
    if (m.actualTimeMs <= (uint64_t)(uint32_t)(m.lastBodyBallCollisionTimeMs + 150)) return true;
    const PlayerList ps = PlayersInProcessingOrder(w);
    Vec3 bounce;
    float depth = 0.0;
    int bounces = 0;
    for (int pi = 0; pi < ps.count; pi++) {
        const int p = ps[pi];
        float opponentBias = 0;
        if (!BodyMayDeflect(w, c, p, opponentBias)) continue;
        Player &pl = m.players[p];
        const Humanoid &h = pl.base.humanoid;
        const float reach = BodyReach(pl);
        if (!(((h.spatial.position + Vec3(0, 0, 0.8f)) - BallPredict(m.ball, 0)).Length() < 2.5f)) continue;
        const Skeleton &sk = c.skeletons[p];
        Transform der[kHumanoidNodes];
        WorldTransforms(sk, h.nodes, der);
        for (int n = 0; n < sk.nodeCount; n++) {
            for (int g = 0; g < sk.nodes[n].geometryCount; g++) {
                const WorldGeometry part = PlacedGeometry(sk.nodes[n].geometries[g], der[n]);
                const float radius = 0.11f + reach;
                const Vec3 ball = BallPredict(m.ball, 0);
                if (!part.box.Intersects(ball, radius)) continue;
                if (p == TeamByID(w, w.playerTeamID[p]).designatedTeamPossessionPlayer && MatchLastTouchBias(w, 200) < 0.01f) {
                    pl.triggerControlledBallCollision = true;
                    continue;
                }
                const float own = opponentBias * 0.8f + 0.2f;
                bounce += (ball - part.position).Normalized(Vec3(0)) * own + h.spatial.movement * (1.0f - own);
                bounces++;
                if (!TeamSetLastTouchPlayer(w, c, p, kTouchAccidental)) return false;
                depth += (1.0f - Clamp(((BallPredict(m.ball, 0) - part.box.Center()).Length() - radius) / part.box.Radius(), 0.0f, 1.0f)) *
                             0.9f +
                         0.1f;
            }
        }
    }
    if (depth > 0.0f) DeflectBall(w, c, bounce, bounces, depth);
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
    Transform der[kHumanoidNodes];
    WorldTransforms(sk, Hum(w, p).nodes, der);
    out.clear();
    for (int n = 0; n < sk.nodeCount; n++)
        for (int g = 0; g < sk.nodes[n].geometryCount; g++) {
            const SkelGeometry &sg = sk.nodes[n].geometries[g];
            out.push_back(PlayerGeometry{sg.footOrLowerLeg, PlacedGeometry(sg, der[n])});
        }
}

// ---- player contacts ------------------------------------------------------------------------------
// Two players whose bodies (0.36 m each) touch push apart and may trip; within the wider shell
// (0.576 m more each) they drag on each other's movement; and a tackle's legs may catch the other
// player's feet within 2 m. GRF's collisions.h: the float operations and their order are its own.
constexpr float kContactBody = 0.5f * 0.72f, kContactShell = 0.8f * 0.72f, kTackleReach = 2.0f;

struct Contact {
    int p1, p2;
    Vec3 pos1, pos2;  // where they stood before the contact moved them
    float dist;
    Vec3 away;  // from p2 toward p1, 2D
    float back1, back2;  // how much each turns its back to the other, 0 to 1
};
HD Contact MakeContact(const World &w, int p1, int p2) {
    Contact k;
    k.p1 = p1;
    k.p2 = p2;
    const SpatialState &s1 = Sp(w, p1), &s2 = Sp(w, p2);
    k.pos1 = s1.position;
    k.pos2 = s2.position;
    k.dist = (k.pos1 - k.pos2).Length();
    k.back1 = k.back2 = 0.5f;
    if (k.dist < kContactBody * 2.0f || k.dist < (kContactBody + kContactShell) * 2.0f) {
        k.away = (k.pos1 - k.pos2).Normalized(Vec3(0, -1, 0));
        const Vec3 face1 = s1.directionVec.Rotated2D(s1.relBodyAngle.value() * 0.7f);
        const Vec3 face2 = s2.directionVec.Rotated2D(s2.relBodyAngle.value() * 0.7f);
        k.back1 = Clamp(face1.Dot(k.away) * 0.5f + 0.5f, 0.0f, 1.0f);
        k.back2 = Clamp(face2.Dot(-k.away) * 0.5f + 0.5f, 0.0f, 1.0f);
    }
    return k;
}
// Which way a contact leans, from -1 (p2 wins) to 1 (p1 wins): the back turned, relative speed,
// (for a push) a tackle before its touch, being the match's designated player (`designatedWeight`),
// between two designated players nearness to the ball (up to 0.6 m), and balance.
HD float ContactLean(World &w, const Ctx &c, const Contact &k, float designatedWeight, bool withTackles) {
    const MatchState &m = w.match;
    auto stat = [&](int p, int s) { return GetStatistic(w, c, p, s); };
    auto tackling = [&](int p, int fn) {
        const AnimationState &a = Hum(w, p).anim;
        return a.frameNum < a.touchFrame && a.functionType == fn;
    };
    auto designated = [&](int p) { return TeamByID(w, w.playerTeamID[p]).designatedTeamPossessionPlayer == p; };
    float lean = 0.0f;
    lean += k.back1 * 0.8f;
    lean -= k.back2 * 0.8f;
    lean -= Clamp(((PlayerFloatVelocity(w, k.p1) - PlayerFloatVelocity(w, k.p2)) / kSprintVelocity) * 0.2f, -0.2f, 0.2f);
    if (withTackles) {
        if (tackling(k.p1, kFnInterfere)) lean += 0.1f + 0.4f * stat(k.p1, kStatStandingTackle);
        if (tackling(k.p1, kFnSliding)) lean += 0.1f + 0.4f * stat(k.p1, kStatSlidingTackle);
        if (tackling(k.p2, kFnInterfere)) lean -= 0.1f + 0.4f * stat(k.p2, kStatStandingTackle);
        if (tackling(k.p2, kFnSliding)) lean -= 0.1f + 0.4f * stat(k.p2, kStatSlidingTackle);
    }
    if (k.p1 == m.designatedPossessionPlayer) lean += designatedWeight;
    if (k.p2 == m.designatedPossessionPlayer) lean -= designatedWeight;
    if (designated(k.p1) && designated(k.p2)) {
        const float d1 = (BallPredict(m.ball, 10).Get2D() - Sp(w, k.p1).position).Length();
        const float d2 = (BallPredict(m.ball, 10).Get2D() - Sp(w, k.p2).position).Length();
        lean += Clamp(MinF(d2, 1.2f) - MinF(d1, 1.2f), -0.6f, 0.6f) * 1.0f;
    }
    lean += stat(k.p1, kStatBalance) * 1.0f;
    lean -= stat(k.p2, kStatBalance) * 1.0f;
    return Clamp(lean, -1.0f, 1.0f);
}
// The shove that moves `other` (at `otherPos`) toward the nearer flank of `carrier`, the player
// on the ball, 0.3 pi off its direction: at most 1 cm, scaled by the other's balance.
HD Vec3 ShoveToFlank(World &w, const Ctx &c, int carrier, const Vec3 &carrierPos, int other, const Vec3 &otherPos) {
    const Vec3 dir = Sp(w, carrier).directionVec;
    const Vec3 left = carrierPos + dir.Rotated2D(0.3f * PI) * kContactBody * 2;
    const Vec3 right = carrierPos + dir.Rotated2D(-0.3f * PI) * kContactBody * 2;
    const Vec3 flank = (otherPos - left).Length() < (otherPos - right).Length() ? left : right;
    return NormalizedMaximum(flank - otherPos, 0.01f) * GetStatistic(w, c, other, kStatBalance) * 0.3f;
}
// Bodies that overlap push apart by the overlap, shared by the lean; the player on the ball is
// shoved aside; each moves at most a sprint's 10 ms.
HD void PushApart(World &w, const Ctx &c, const Contact &k) {
    const MatchState &m = w.match;
    const float lean = ContactLean(w, c, k, 0.4f, true) * 0.5f;
    const float share = lean * 0.5f + 0.5f;
    Vec3 off1 = (k.pos1 - k.pos2).Normalized(0) * (kContactBody - k.dist * 0.5f) * (1.0f - share) * 2.0f;
    Vec3 off2 = (k.pos2 - k.pos1).Normalized(0) * (kContactBody - k.dist * 0.5f) * share * 2.0f;
    if (m.designatedPossessionPlayer == k.p2 && m.players[k.p2].hasPossession)
        off1 += ShoveToFlank(w, c, k.p2, k.pos2, k.p1, k.pos1);
    else if (m.designatedPossessionPlayer == k.p1 && m.players[k.p1].hasPossession)
        off2 += ShoveToFlank(w, c, k.p1, k.pos1, k.p2, k.pos2);
    NormalizeMaximum(off1, kSprintVelocity * 0.01f);
    NormalizeMaximum(off2, kSprintVelocity * 0.01f);
    OffsetPosition(w, k.p1, off1);
    OffsetPosition(w, k.p2, off2);
}
// Within the shell each drags on the other's movement: a force that fades across the shell (to
// the 0.2, at a quarter), split by the lean.
HD void Drag(World &w, const Ctx &c, const Contact &k, PlayerBounceList &b1, PlayerBounceList &b2) {
    const float gap = k.dist - kContactBody * 2.0f;
    const float shell = (0.0f < gap) ? gap : 0.0f;
    const float lean = ContactLean(w, c, k, 0.6f, false) * 0.9f;
    float force = Clamp(1.0f - (shell / (kContactShell * 2.0f)), 0.0f, 1.0f);
    force = libm::powf(force, 0.2f);
    force *= 0.25f;
    const float share = lean * 0.5f + 0.5f;
    b1.push_back(PlayerBounce{k.p2, force * (1.0f - share)});
    b2.push_back(PlayerBounce{k.p1, force * share});
}
// A player's chance of tripping in a push, 0 to 1: its back turned, its speed, being best placed
// for the ball, poor balance (weight 3), its own position offset, how deep the two overlap 30 ms
// ahead (weight 6) and the ball within 0.7 m.
HD float TripScore(World &w, const Ctx &c, int p, float back, float penetration, float bodyReach) {
    const float balanceWeight = 3.0f, penetrationWeight = 6.0f;
    float score = 0.0f;
    score += (1.0f - back) * 1.0f;
    score += NormalizedClamp(PlayerFloatVelocity(w, p), kIdleVelocity, kSprintVelocity) * 1.0f;
    if (w.match.players[p].hasBestPossession) score += 1.0f;
    score += (1.0f - GetStatistic(w, c, p, kStatBalance) * 1.0f) * balanceWeight;
    score += Clamp(Hum(w, p).decayingPositionOffset.Length() * 10.0f, 0.0f, 1.0f);
    score += libm::powf(1.0f - NormalizedClamp(penetration, 0.0f, bodyReach), 0.4f) * penetrationWeight;
    score += 1.0f - NormalizedClamp((BallPredict(w.match.ball, 10).Get2D() - Sp(w, p).position).Length(), 0.0f, 0.7f);
    score /= 5.0f + balanceWeight + penetrationWeight;
    return score;
}
// The trip a score brings: none up to 0.48, type 1 to 0.58, type 2 above.
HD int TripTypeOf(float score) {
    if (!(score > 0.38f)) return 0;
    int type = 0;
    if (score > 0.48f) type = 1;
    if (score > 0.58f) type = 2;
    return type;
}
// After a push each player may trip, away from the other along a blend of the two movements,
// and the referee notes it.
HD void TripInPush(World &w, const Ctx &c, const Contact &k) {
    const SpatialState &s1 = Sp(w, k.p1), &s2 = Sp(w, k.p2);
    const float penetration = ((s1.position + s1.movement * 0.03f) - (s2.position + s2.movement * 0.03f)).Length();
    const float score1 = TripScore(w, c, k.p1, k.back1, penetration, kContactBody * 2.0f);
    const float score2 = TripScore(w, c, k.p2, k.back2, penetration, kContactBody * 2.0f);
    const int type1 = TripTypeOf(score1), type2 = TripTypeOf(score2);
    if (type1 > 0) {
        TripMe(w, c, k.p1, (Sp(w, k.p1).movement * 0.1f + Sp(w, k.p2).movement * 0.06f + k.away * 1.0f).Normalized(k.away), type1);
        RefereeTripNotice(w, k.p1, k.p2, type1);
    }
    if (type2 > 0) {
        TripMe(w, c, k.p2, (Sp(w, k.p2).movement * 0.1f + Sp(w, k.p1).movement * 0.06f - k.away * 1.0f).Normalized(-k.away), type2);
        RefereeTripNotice(w, k.p2, k.p1, type2);
    }
}
// Within 2 m, one (and only one) player between frames 6 and 27 of a sliding or standing tackle
// may catch the other's feet: a tackle part (shrunk by 10 cm) overlapping a foot or lower leg,
// between the tackle's frame 11 and its sixth frame from the end, trips the other (type 1 for a
// standing tackle, 3 for a sliding one) along its own direction.
HD void TackleContact(World &w, const Ctx &c, int p1, int p2, float dist) {
    auto tackling = [&](int p) {
        const AnimationState &a = Hum(w, p).anim;
        return (a.functionType == kFnSliding || a.functionType == kFnInterfere) && a.frameNum > 5 && a.frameNum < 28;
    };
    const int tackle = (tackling(p1) ? 1 : 0) + (tackling(p2) ? 2 : 0);
    if (!(dist < kTackleReach && tackle > 0 && tackle < 3)) return;
    const int tackler = tackle == 1 ? p1 : p2, victim = tackle == 1 ? p2 : p1;
    PlayerGeometryList &tg = c.ws->tackleGeometry[0], &vg = c.ws->tackleGeometry[1];
    PlayerGeometries(w, c, tackler, tg);
    PlayerGeometries(w, c, victim, vg);
    for (int i = 0; i < tg.count; i++) {
        Aabb box = tg[i].wg.box;
        box.lo += 0.1f;
        box.hi -= Vec3(0.1f);
        for (int j = 0; j < vg.count; j++) {
            if (!vg[j].footOrLowerLeg || !BoxesIntersect(box, vg[j].wg.box)) continue;
            const AnimationState &ta = Hum(w, tackler).anim;
            if (ta.frameNum > 10 && ta.frameNum < c.A(ta.anim).frameCount - 6) {
                const int type = ta.functionType == kFnInterfere ? 1 : 3;
                TripMe(w, c, victim, Sp(w, victim).directionVec, type);
                RefereeTripNotice(w, victim, tackler, type);
            }
            break;
        }
    }
}
// One pair's contact, in GRF's order: push apart, drag, trips in the push, then the tackle.
HDN void CheckHumanoidCollision(World &w, const Ctx &c, int p1, int p2, PlayerBounceList &b1, PlayerBounceList &b2) {
    const Contact k = MakeContact(w, p1, p2);
    if (k.dist < kContactBody * 2.0f) PushApart(w, c, k);
    if (k.dist < (kContactBody + kContactShell) * 2.0f) Drag(w, c, k, b1, b2);
    if (k.dist < kContactBody * 2.0f) TripInPush(w, c, k);
    TackleContact(w, c, p1, p2, k.dist);
}

HDN bool CheckHumanoidCollisions(World &w, const Ctx &c) {
    ENG_SCOPE(17);
    PlayerList ps = PlayersInProcessingOrder(w);
    PlayerBounceList *const bounces = c.ws->bounces;
    for (int i = 0; i < ps.count; i++) bounces[i].clear();
    // A pair at least the tackle reach apart (2 m, beyond both contact radii) changes nothing, so
    // only nearer pairs make the call; the distance is the one the pair's own check computes.
    static_assert((kContactBody + kContactShell) * 2.0f < kTackleReach, "the tackle reach bounds every contact");
    // The pairs read the positions from a copy gathered once, not from each player's spatial state
    // (one cache line per player, read again for every pair); a call moves only its two players,
    // whose copies it refreshes.
    Vec3 at[kPlayers];
    for (int i = 0; i < ps.count; i++) at[i] = Sp(w, ps[i]).position;
    for (int i = 0; i + 1 < ps.count; i++) {
        for (int j = i + 1; j < ps.count; j++) {
            if ((at[i] - at[j]).Length() < kTackleReach) {
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
