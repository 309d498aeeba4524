// SPDX-License-Identifier: Apache-2.0
// Restates game logic of cuju (Copyright 2026 The cuju Authors), a reimplementation of Google
// Research Football (Copyright 2019 Google LLC); see NOTICE.
// Team queries the player AI and the team AI share: lines, tactic properties, the closest players,
// the goalkeeper, the best possession player, gamer switch targets, and the pose offsets of a
// player. Semantics: include/cuju/simulation/ai_controller.h:43-87 (Line),
// include/cuju/real_to_string.h:17-53, include/cuju/simulation/team_process.h:20-130,
// include/cuju/simulation/geometry_offsets.h:13-200.
#pragma once

#include "player.h"

namespace eng {

// A 2D segment from pts[0] to pts[1] (z ignored).
struct Line {
    Vec3 pts[2];
    HD Line() {}
    HD Line(const Vec3 &a, const Vec3 &b) {
        pts[0] = a;
        pts[1] = b;
    }
    HD float Length() const { return (pts[0] - pts[1]).Length(); }
    // The parameter along the segment of the projection of `pt`.
    HD float ClosestToPoint(const Vec3 &pt) const {
        if (pts[0] == pts[1]) return 0.0f;
        float d = (pts[1] - pts[0]).Length();
        if (d < 0.000001f) return 0.0f;
        return ((pt.v[0] - pts[0].v[0]) * (pts[1].v[0] - pts[0].v[0]) + (pt.v[1] - pts[0].v[1]) * (pts[1].v[1] - pts[0].v[1])) /
               (d * d);
    }
    HD float DistanceToPoint(const Vec3 &pt, float &f) const {
        f = ClosestToPoint(pt);
        Vec3 is;
        is.v[0] = pts[0].v[0] + f * (pts[1].v[0] - pts[0].v[0]);
        is.v[1] = pts[0].v[1] + f * (pts[1].v[1] - pts[0].v[1]);
        return (is - pt).Length();
    }
    // The intersection with the infinite line through `l`; `f` is its parameter on this segment.
    HD Vec3 IntersectionPoint(const Line &l, float &f) const {
        const Vec3 &a = l.pts[0], &b = l.pts[1];
        float div = (b.v[1] - a.v[1]) * (pts[1].v[0] - pts[0].v[0]) - (b.v[0] - a.v[0]) * (pts[1].v[1] - pts[0].v[1]);
        if (div == 0.0f) return pts[0];
        f = ((b.v[0] - a.v[0]) * (pts[0].v[1] - a.v[1]) - (b.v[1] - a.v[1]) * (pts[0].v[0] - a.v[0])) / (div);
        return pts[0] + (pts[1] - pts[0]) * f;
    }
    HD Vec3 IntersectionPoint(const Line &l) const {
        float f = 0.0f;
        return IntersectionPoint(l, f);
    }
};

// GRF stores some settings as "%f" text and reads them back with atof. The text holds the value
// rounded to six decimals (ties to even) and atof returns the nearest double, which for the
// magnitudes used here (below 2^33) is the quotient N / 1e6 of that rounded integer.
HDN float RoundTripSixDecimals(float v) {
    const uint32_t bits = BitsOf(v);
    const uint32_t biased = (bits >> 23) & 0xff;
    if (biased == 0xff) return v;
    uint64_t mant = bits & 0x7fffff;
    int e;
    if (biased == 0) {
        e = -149;
    } else {
        mant |= 0x800000;
        e = (int)biased - 150;
    }
    // |v| * 1e6 = mant * 1e6 * 2^e, with mant * 1e6 < 2^44.
    const uint64_t scaled = mant * 1000000ull;
    uint64_t n;
    if (e >= 0) {
        n = scaled << e;
    } else if (-e >= 64) {
        n = 0;
    } else {
        const int s = -e;
        n = scaled >> s;
        const uint64_t rest = scaled - (n << s);
        const uint64_t half = 1ull << (s - 1);
        if (rest > half || (rest == half && (n & 1))) n++;
    }
    const float r = (float)((double)n / 1e6);
    return (bits >> 31) ? -r : r;
}

HD float PropertiesGetReal(const Tactics &t, int id, float fallback = 0) {
    return ((t.present >> id) & 1) ? t.value[id] : fallback;
}
HD void PropertiesSet(Tactics &t, int id, float value) {
    t.present |= 1u << id;
    t.value[id] = RoundTripSixDecimals(value);
}

// The closest active players of a team to `pos`, nearest first, ties in state order: the first
// `count` of a stable insertion sort by distance. Every player's tests and position load together
// (the slots past the match's players are in the arrays; the controller and formation tests, which
// index other tables, run only for the team's active players), and the sort runs in registers: an
// insertion lands after the last kept entry it is not nearer than, where the shifting scan stops,
// NaN distances included. A team holds at most kTeamPlayers players.
HDN PlayerList GetClosestPlayers(const World &w, const Ctx &c, int teamID, const Vec3 &pos, bool onlyAI, unsigned count = 3,
                                 bool onlySelectable = false) {
    float dist[kTeamPlayers];
    int who[kTeamPlayers], n = 0;
    const int players = w.match.playerCount;
#pragma unroll
    for (int p = 0; p < kPlayers; p++) {
        bool in = (p < players) & (w.playerTeamID[p] == teamID) & w.roster.active[p];
        const float d = (Sp(w, p).position - pos).Length();
        if (in && !((!onlyAI || !ExternalControllerActive(w, p)) && (!onlySelectable || Formation(w, c, p).controllable))) in = false;
        if (!in) continue;
        if (n >= kTeamPlayers) {
            Fatal("a team holds more players than a team has");
            break;
        }
        int at = 0;
#pragma unroll
        for (int s = 0; s < kTeamPlayers; s++)
            if (s < n && !(d < dist[s])) at = s + 1;
#pragma unroll
        for (int s = kTeamPlayers - 1; s > 0; s--)
            if (s > at && s <= n) {
                dist[s] = dist[s - 1];
                who[s] = who[s - 1];
            }
#pragma unroll
        for (int s = 0; s < kTeamPlayers; s++)
            if (s == at) {
                dist[s] = d;
                who[s] = p;
            }
        n++;
    }
    PlayerList r;
#pragma unroll
    for (int i = 0; i < kTeamPlayers; i++)
        if ((unsigned)i < count && i < n) r.push_back(who[i]);
    return r;
}
HD int TeamGoalie(const World &w, const Ctx &c, int teamID) {
    for (int p = 0; p < w.match.playerCount; p++)
        if (w.playerTeamID[p] == teamID && w.roster.active[p] && Formation(w, c, p).role == kRoleGoalkeeper) return p;
    return -1;
}
// The active player of a team with the least time to the ball, the first in state order on ties.
// Every player's tests and time load together, without an early exit.
HDN int TeamBestPossessionPlayer(const World &w, int teamID) {
    int best = 10000000, bp = -1;
    const int players = w.match.playerCount;
#pragma unroll
    for (int p = 0; p < kPlayers; p++) {
        const bool in = (p < players) & (w.playerTeamID[p] == teamID) & w.roster.active[p];
        const int t = (int)w.roster.timeToBallMs[p];
        if (in && t < best) {
            best = t;
            bp = p;
        }
    }
    return bp;
}
// True unless every team with agents has exactly one agent per controllable player.
HD bool DynamicPlayerSelection(const World &w) {
    const Scenario &s = w.scenario;
    int l = 0, r = 0;
    for (int i = 0; i < s.leftTeamSize; i++) l += s.leftTeam[i].controllable ? 1 : 0;
    for (int i = 0; i < s.rightTeamSize; i++) r += s.rightTeam[i].controllable ? 1 : 0;
    return !((l == s.leftAgents || s.leftAgents == 0) && (r == s.rightAgents || s.rightAgents == 0));
}
// Where a gamer's switch looks for a player: the middle of the designated player and the ball in
// 100 ms, its width squeezed to 80%; from there 4 m back toward the team's goal (and a fifth of
// the way to the team's designated player) when defending, 8 m upfield when attacking, blended by
// how much the team holds the ball.
HD Vec3 SwitchFocus(const World &w, int teamID) {
    const MatchState &m = w.match;
    const Team &t = TeamByID(w, teamID);
    const int side = TeamDynamicSide(w, teamID);
    const Vec3 action = Sp(w, m.designatedPossessionPlayer).position * 0.5f + BallPredict(m.ball, 100).Get2D() * 0.5f;
    const Vec3 squeezed = action * Vec3(1.0f, 0.8f, 0.0f);
    const Vec3 defending = (squeezed + Vec3(side * 4.0f, 0.0f, 0.0f)) * 0.8f + Sp(w, t.designatedTeamPossessionPlayer).position * 0.2f;
    const Vec3 attacking = squeezed + Vec3(-side * 8.0f, 0.0f, 0.0f);
    float attack = t.fadingTeamPossessionAmount - 0.5f;
    attack = attack * 0.2f + Clamp(t.teamPossessionAmount - 0.5f, 0.0f, 1.0f) * 0.8f;
    attack = Clamp((float)((double)(attack - 0.5f) * 2.0 + 0.5), 0.0f, 1.0f);
    attack = Clamp(libm::powf(attack, 1.5f), 0.0f, 1.0f);
    return defending * (1.0f - attack) + attacking * attack;
}
// How far a humanoid will be from `goal` half a second ahead.
HD float GoalDistanceAhead(const SpatialState &s, const Vec3 &goal) { return (goal - (s.position + s.movement * 0.5f)).Length(); }
// The player a gamer's switch goes to (-1 for none): of the 8 AI-controlled players nearest the
// switch focus, goalkeepers aside, the nearest; while an opponent is the designated player, the
// first of them that will be at most a metre (plus a tenth of the opponent's distance, up to 3 m)
// further from the team's goal than the opponent.
HDN int SwitchTargetPlayer(const World &w, const Ctx &c, int teamID) {
    const int designated = w.match.designatedPossessionPlayer;
    const PlayerList nearest = GetClosestPlayers(w, c, teamID, SwitchFocus(w, teamID), true, 8);
    PlayerList field;
    for (int i = 0; i < nearest.count; i++)
        if (Formation(w, c, nearest[i]).role != kRoleGoalkeeper) field.push_back(nearest[i]);
    if (field.empty()) return -1;
    if (w.playerTeamID[designated] == teamID) return field[0];
    const Vec3 goal = Vec3(TeamDynamicSide(w, teamID) * kPitchHalfLength, 0.0f, 0.0f);
    const float opponent = GoalDistanceAhead(Sp(w, designated), goal);
    const float tooLate = 1.0f;
    for (int i = 0; i < field.count; i++)
        if (GoalDistanceAhead(Sp(w, field[i]), goal) < opponent + tooLate + Clamp(opponent * 0.1f, 0.0f, 3.0f)) return field[i];
    return field[0];
}

// ---- pose offsets ------------------------------------------------------------------------------------
// A humanoid's pose offsets bend body parts from the animation's pose (a bias toward an
// orientation per part). In play, off the ball and moving, the legs bend, the upper body turns to
// the ball and an arm fends off a close opponent alongside. The offsets are GRF's
// (geometry_offsets.h); the orientations are built the same way.
HD void SetOffset(Humanoid &h, int bp, float bias, const Quat &q) {
    h.offsets[bp].bias = bias;
    h.offsets[bp].orientation = q;
}
HD Quat AngleAxis(float angle, const Vec3 &axis) {
    Quat q;
    q.SetAngleAxis(angle, axis);
    return q;
}
// The legs bend as far as the humanoid moves slower than its animation (to a tenth of it; above
// 7 m/s it may run 10% faster), by up to `influence`.
HD void BendLegs(Humanoid &h, float influence) {
    const SpatialState &s = h.spatial;
    const float actual = s.actualMovement.Length();
    const float slower = Clamp((actual + 0.2f) / (s.animationMovement.Length() + 0.2f), 0.1f, 1.0f + (actual > 7.0f ? (float)0.1 : 0.0f));
    const float bend = 0.8f;
    const float bias = (1.0f - slower) * influence;
    const Quat knee = AngleAxis(0.3f * PI * bend, Vec3(1, 0, 0)), ankle = AngleAxis(-0.1f * PI * bend, Vec3(1, 0, 0));
    SetOffset(h, kBpLeftThigh, bias, AngleAxis(-0.15f * PI * bend, Vec3(1, 0.06, -0.12).Normalized()));
    SetOffset(h, kBpRightThigh, bias, AngleAxis(-0.15f * PI * bend, Vec3(1, -0.06, 0.12).Normalized()));
    SetOffset(h, kBpLeftKnee, bias, knee);
    SetOffset(h, kBpRightKnee, bias, knee);
    SetOffset(h, kBpLeftAnkle, bias, ankle);
    SetOffset(h, kBpRightAnkle, bias, ankle);
}
// The upper body (30%) and the head (70%) turn toward the ball as the humanoid sees it, beyond a
// 0.05 pi dead zone, by up to `influence`: less the further it has to turn, for a ball within
// 1.6 m and at speed.
HD void TurnTowardBall(World &w, Humanoid &h, float influence) {
    const SpatialState &s = h.spatial;
    const Vec3 toBall = (MentalBallPrediction(w, MentalImageIndex(w, h.mentalImageTime), 10).Get2D() - s.position).Normalized(s.directionVec);
    float turn = toBall.Angle2D(s.relBodyDirectionVecNonQuantized.Rotated2D(s.angle.value()));
    turn = Clamp(fabsf(turn) - 0.05f * PI, 0.0f, PI) * SignSide(turn);
    float bias = Clamp(libm::powf(1.0f - fabsf(turn / PI), 0.3f) * influence, 0.0f, 1.0f);
    const float ballDistance = GetDistance(BallPredict(w.match.ball, 100).Get2D(), s.position);
    const float falloff = 1.6f;
    if (ballDistance < falloff) bias *= NormalizedClamp(ballDistance, falloff * 0.4f, falloff);
    const float fast = NormalizedClamp(s.floatVelocity, kIdleVelocity, kSprintVelocity - 0.5f);
    bias *= 1.0f - fast * fast * 0.3f;
    Quat middle = AngleAxis(turn, Vec3(0, 0, 1));
    middle.Normalize();
    SetOffset(h, kBpMiddle, bias * 0.3f, middle);
    Quat head = AngleAxis(turn, Vec3(0, 0, 1));
    head.Normalize();
    SetOffset(h, kBpNeck, bias * 0.7f, head);
}
// The opponent quickest to the ball, within 1.4 m and running the same way, is fended off with the
// arm on its side: raised and bent out when it is behind (0.6 to 0.85 pi off the body), raised
// and bent forward when alongside (0.2 to 0.6 pi), held low ahead (within 0.2 rad: GRF's bound is
// in radians there). Angle bounds compare in double.
HD void FendOff(World &w, Humanoid &h, int p, float influence) {
    const SpatialState &s = h.spatial;
    const int o = TeamBestPossessionPlayer(w, 1 - w.playerTeamID[p]);
    if (o < 0) {
        Fatal("a player has no active opponent");
        return;
    }
    const SpatialState &os = Sp(w, o);
    if (!((double)(os.position - s.position).Length() < 1.4 && (double)os.directionVec.Dot(s.directionVec) > 0.0)) return;
    const Vec3 body = Vec3(0, -1, 0).Rotated2D(s.angle.value()).Rotated2D(s.relBodyAngle.value());
    const float toOpponent = body.Angle2D((os.position - s.position).Normalized(body));
    const double off = fabsf(toOpponent), dpi = (double)PI;
    const bool right = toOpponent > 0;
    const int shoulder = right ? kBpRightShoulder : kBpLeftShoulder, elbow = right ? kBpRightElbow : kBpLeftElbow;
    const float raise = (float)((right ? 0.4 : -0.4) * dpi);
    if (off > 0.6 * dpi && off < 0.85 * dpi) {
        SetOffset(h, shoulder, 0.8f * influence, AngleAxis(raise, Vec3(0, 1, 0)).Normalized());
        SetOffset(h, elbow, 0.7f * influence, AngleAxis(0, Vec3(0, 1, 0)).Normalized());
        SetOffset(h, kBpMiddle, 0.3f * influence, AngleAxis(0.2f * PI, Vec3(1, 0, 0)).Normalized());
    }
    if (off > 0.2 * dpi && off <= 0.6 * dpi) {
        SetOffset(h, shoulder, 0.7f * influence, AngleAxis(raise, Vec3(0, 1, 0)).Normalized());
        SetOffset(h, elbow, 0.8f * influence, AngleAxis((float)(-0.5 * dpi), Vec3(1, 0, 0)).Normalized());
    }
    if (off < 0.2) {
        SetOffset(h, shoulder, 0.6f * influence, AngleAxis((float)(-0.4 * dpi), Vec3(1, 0, 0)).Normalized());
        SetOffset(h, elbow, 0.8f * influence, AngleAxis((float)(-0.2 * dpi), Vec3(1, 0, 0)).Normalized());
    }
}
// Player p's pose offsets for the tick: cleared, then, in play without holding the ball and
// moving, the legs, the upper body (off the ball) and the arms.
HDN void PoseOffsets(World &w, int p) {
    Humanoid &h = Hum(w, p);
    const Quat identity(0, 0, 0, 1);
    for (int bp = kBpMiddle; bp <= kBpBody; bp++) SetOffset(h, bp, 0.0, identity);
    if (!(w.match.inPlay && w.match.ballRetainer != p) || h.anim.functionType != kFnMovement) return;
    BendLegs(h, 0.7f);
    if (!w.match.players[p].hasPossession) TurnTowardBall(w, h, 0.5f);
    FendOff(w, h, p, 0.9f);
}

}  // namespace eng
