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
HDN int GetBestSwitchTargetPlayer(const World &w, const Ctx &c, int teamID) {
    const MatchState &m = w.match;
    const Team &t = TeamByID(w, teamID);
    const int side = TeamDynamicSide(w, teamID);
    Vec3 action = Sp(w, m.designatedPossessionPlayer).position * 0.5f + BallPredict(m.ball, 100).Get2D() * 0.5f;
    Vec3 def = (action * Vec3(1.0f, 0.8f, 0.0f)) + Vec3(side * 4.0f, 0.0f, 0.0f);
    Vec3 off = (action * Vec3(1.0f, 0.8f, 0.0f)) + Vec3(-side * 8.0f, 0.0f, 0.0f);
    def = def * 0.8f + Sp(w, t.designatedTeamPossessionPlayer).position * 0.2f;
    float ob = t.fadingTeamPossessionAmount - 0.5f;
    ob = ob * 0.2f + Clamp(t.teamPossessionAmount - 0.5f, 0.0f, 1.0f) * 0.8f;
    ob = Clamp((float)((double)(ob - 0.5f) * 2.0 + 0.5), 0.0f, 1.0f);
    ob = Clamp(libm::powf(ob, 1.5f), 0.0f, 1.0f);
    Vec3 res = def * (1.0f - ob) + off * ob;
    PlayerList cand = GetClosestPlayers(w, c, teamID, res, true, 8);
    PlayerList kept;
    for (int i = 0; i < cand.count; i++)
        if (Formation(w, c, cand[i]).role != kRoleGoalkeeper) kept.push_back(cand[i]);
    if (kept.empty()) return -1;
    int best = 0;
    const float tooLate = 1.0f;
    const int d = m.designatedPossessionPlayer;
    if (w.playerTeamID[d] != teamID) {
        const SpatialState &os = Sp(w, d);
        Vec3 goal = Vec3(side * kPitchHalfLength, 0.0f, 0.0f);
        float og = (goal - (os.position + os.movement * 0.5f)).Length();
        for (int i = 0; i < kept.count; i++) {
            const SpatialState &ms = Sp(w, kept[i]);
            float mg = (goal - (ms.position + ms.movement * 0.5f)).Length();
            if (mg < og + tooLate + Clamp(og * 0.1f, 0.0f, 3.0f)) {
                best = i;
                break;
            }
        }
    }
    return kept[best];
}

// ---- pose offsets ------------------------------------------------------------------------------------
HD void SetOffset(Humanoid &h, int bp, float bias, const Quat &q) {
    h.offsets[bp].bias = bias;
    h.offsets[bp].orientation = q;
}
HD Quat AngleAxis(float angle, const Vec3 &axis) {
    Quat q;
    q.SetAngleAxis(angle, axis);
    return q;
}
// Legs bend to the true velocity, the upper body turns to the ball, the arms fend off a close
// opponent alongside.
HDN void CalculateGeometryOffsets(World &w, int p) {
    Humanoid &h = Hum(w, p);
    const SpatialState &s = h.spatial;
    const Quat identity(0, 0, 0, 1);
    for (int bp = kBpMiddle; bp <= kBpBody; bp++) SetOffset(h, bp, 0.0, identity);
    const float legsInfluence = 0.7f, bodyInfluence = 0.5f, armsInfluence = 0.9f;
    if (!(w.match.inPlay && w.match.ballRetainer != p)) return;
    if (h.anim.functionType != kFnMovement) return;
    {
        float actual = s.actualMovement.Length();
        float anim = s.animationMovement.Length();
        float vf = (actual + 0.2f) / (anim + 0.2f);
        float allowFaster = 0.0f;
        if (s.actualMovement.Length() > 7.0f) allowFaster = (float)((double)allowFaster + 0.1);
        vf = Clamp(vf, 0.1f, 1.0f + allowFaster);
        const float bend = 0.8f;
        Quat leftHip = AngleAxis(-0.15f * PI * bend, Vec3(1, 0.06, -0.12).Normalized());
        Quat rightHip = AngleAxis(-0.15f * PI * bend, Vec3(1, -0.06, 0.12).Normalized());
        Quat knee = AngleAxis(0.3f * PI * bend, Vec3(1, 0, 0));
        Quat ankle = AngleAxis(-0.1f * PI * bend, Vec3(1, 0, 0));
        float legBias = (1.0f - vf) * legsInfluence;
        SetOffset(h, kBpLeftThigh, legBias, leftHip);
        SetOffset(h, kBpRightThigh, legBias, rightHip);
        SetOffset(h, kBpLeftKnee, legBias, knee);
        SetOffset(h, kBpRightKnee, legBias, knee);
        SetOffset(h, kBpLeftAnkle, legBias, ankle);
        SetOffset(h, kBpRightAnkle, legBias, ankle);
    }
    if (!w.match.players[p].hasPossession) {
        Vec3 toBall = (MentalBallPrediction(w, MentalImageIndex(w, h.mentalImageTime), 10).Get2D() - s.position)
                          .Normalized(s.directionVec);
        float a = toBall.Angle2D(s.relBodyDirectionVecNonQuantized.Rotated2D(s.angle.value()));
        a = Clamp(fabsf(a) - 0.05f * PI, 0.0f, PI) * SignSide(a);
        float lb = libm::powf(1.0f - fabsf(a / PI), 0.3f);
        lb = Clamp(lb * bodyInfluence, 0.0f, 1.0f);
        float bd = GetDistance(BallPredict(w.match.ball, 100).Get2D(), s.position);
        const float falloff = 1.6f;
        if (bd < falloff) lb *= NormalizedClamp(bd, falloff * 0.4f, falloff);
        float vfr = NormalizedClamp(s.floatVelocity, kIdleVelocity, kSprintVelocity - 0.5f);
        lb *= 1.0f - vfr * vfr * 0.3f;
        Quat middle = AngleAxis(a, Vec3(0, 0, 1));
        middle.Normalize();
        SetOffset(h, kBpMiddle, lb * 0.3f, middle);
        Quat head = AngleAxis(a, Vec3(0, 0, 1));
        head.Normalize();
        SetOffset(h, kBpNeck, lb * 0.7f, head);
    }
    const int o = TeamBestPossessionPlayer(w, 1 - w.playerTeamID[p]);
    if (o < 0) {
        Fatal("a player has no active opponent");
        return;
    }
    const SpatialState &os = Sp(w, o);
    if (!((double)(os.position - s.position).Length() < 1.4 && (double)os.directionVec.Dot(s.directionVec) > 0.0)) return;
    Vec3 base = Vec3(0, -1, 0).Rotated2D(s.angle.value()).Rotated2D(s.relBodyAngle.value());
    Vec3 ov = os.position - s.position;
    float a = base.Angle2D(ov.Normalized(base));
    // The angle bounds compare in double.
    const double aa = fabsf(a);
    const double dpi = (double)PI;
    const bool right = a > 0;
    const int shoulderPart = right ? kBpRightShoulder : kBpLeftShoulder;
    const int elbowPart = right ? kBpRightElbow : kBpLeftElbow;
    const float shoulderAngle = (float)((right ? 0.4 : -0.4) * dpi);
    if (aa > 0.6 * dpi && aa < 0.85 * dpi) {
        SetOffset(h, shoulderPart, 0.8f * armsInfluence, AngleAxis(shoulderAngle, Vec3(0, 1, 0)).Normalized());
        SetOffset(h, elbowPart, 0.7f * armsInfluence, AngleAxis(0, Vec3(0, 1, 0)).Normalized());
        SetOffset(h, kBpMiddle, 0.3f * armsInfluence, AngleAxis(0.2f * PI, Vec3(1, 0, 0)).Normalized());
    }
    if (aa > 0.2 * dpi && aa <= 0.6 * dpi) {
        SetOffset(h, shoulderPart, 0.7f * armsInfluence, AngleAxis(shoulderAngle, Vec3(0, 1, 0)).Normalized());
        SetOffset(h, elbowPart, 0.8f * armsInfluence, AngleAxis((float)(-0.5 * dpi), Vec3(1, 0, 0)).Normalized());
    }
    // GRF: this bound is 0.2 radians, not 0.2 pi.
    if (aa < 0.2) {
        SetOffset(h, shoulderPart, 0.6f * armsInfluence, AngleAxis((float)(-0.4 * dpi), Vec3(1, 0, 0)).Normalized());
        SetOffset(h, elbowPart, 0.8f * armsInfluence, AngleAxis((float)(-0.2 * dpi), Vec3(1, 0, 0)).Normalized());
    }
}

}  // namespace eng
