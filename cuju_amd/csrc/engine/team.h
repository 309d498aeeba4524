// SPDX-License-Identifier: Apache-2.0
// Restates game logic of cuju (Copyright 2026 The cuju Authors), a reimplementation of Google
// Research Football (Copyright 2019 Google LLC); see NOTICE.
// The team AI (tactics, offside trap, danger ranking, attacking runs, dynamic roles, man marking)
// and the tick of a team (possession amounts, players, gamer switches, designated player).
// Semantics: include/cuju/simulation/team_ai.h:15-533, include/cuju/simulation/team_process.h:134-312.
#pragma once

#include "ai_requests.h"

namespace eng {

// Defined with the set pieces.
HDN bool SendOff(World &w, const Ctx &c, int p);

// Goals and the possession of the last minute are stored in processing order; these take IDs.
HD int MatchGoalCount(const World &w, int teamID) { return w.match.goalCount[teamID == w.FirstTeamID() ? 0 : 1]; }
HD float MatchPossessionLastMinute(const World &w) {
    return w.FirstTeamID() == 1 ? -w.match.possessionLastMinute : w.match.possessionLastMinute;
}

// GRF's user tactics, shared by every team, in the alphabetical order of their names; a negative
// id marks the two dribble settings, which the update skips.
struct UserTactic {
    int32_t id;
    float value, modifierMultiplier;
};
constexpr int kUserTactics = 12;
HD UserTactic UserTacticAt(int i) {
    switch (i) {
        case 0: return {-1, 0.72f, 0.0f};
        case 1: return {-1, 0.5f, 0.0f};
        case 2: return {kDefenseDepth, 0.3f, 0.1f};
        case 3: return {kDefenseMicroFocusStrength, 0.96f, 0.15f};
        case 4: return {kDefenseMidfieldFocus, 0.96f, 0.3f};
        case 5: return {kDefenseSideFocusStrength, 0.16f, 0.1f};
        case 6: return {kDefenseWidth, 0.7f, 0.1f};
        case 7: return {kOffenseDepth, 0.34f, 0.1f};
        case 8: return {kOffenseMicroFocusStrength, 0.92f, 0.15f};
        case 9: return {kOffenseMidfieldFocus, 0.88f, 0.3f};
        case 10: return {kOffenseSideFocusStrength, 0.88f, 0.1f};
        default: return {kOffenseWidth, 0.74f, 0.1f};
    }
}
HDN void TeamUpdateTactics(World &w, int teamID) {
    TeamAI &ai = TeamByID(w, teamID).ai;
    const MatchState &m = w.match;
    int goals = MatchGoalCount(w, teamID), oppGoals = MatchGoalCount(w, 1 - teamID);
    ai.liveTactics = ai.baseTactics;
    float goalFactor = Clamp((float)(0.5 + (double)((oppGoals - goals) * 0.25f)), 0.0f, 1.0f);
    float timeFactor = 0.5f + 0.5f * Clamp((float)m.matchTimeMs / 6300000.0f, 0.0f, 1.0f);
    float offenseBias = Clamp(0.5f + (goalFactor - 0.5f) * (timeFactor * 1.0f), 0.0f, 1.0f);
    float pf = MatchPossessionLastMinute(w) / 60.0f;
    float recent = teamID == 0 ? (float)(0.5 - (double)(pf * 0.5f)) : (float)(0.5 + (double)(pf * 0.5f));
    ai.offensivenessBias = offenseBias * 0.5f + recent * 0.5f;
    for (int i = 0; i < kUserTactics; i++) {
        const UserTactic ut = UserTacticAt(i);
        // A stored tactic passes through six-decimal text.
        float mul = ut.modifierMultiplier == 0.0f ? 0.0f : RoundTripSixDecimals(ut.modifierMultiplier);
        float offset = (RoundTripSixDecimals(ut.value) - 0.5f) * 2.0f * mul;
        float base = ut.id < 0 ? -1.0f : PropertiesGetReal(ai.baseTactics, ut.id, -1.0f);
        if (base >= 0.0f) PropertiesSet(ai.liveTactics, ut.id, Clamp(base + offset, 0.0f, 1.0f));
    }
}
// The closest player without a gamer to a point 26 m ahead of the team's possession player.
HD int SelectAttackingRunPlayer(const World &w, const Ctx &c, int teamID) {
    int pp = TeamByID(w, teamID).designatedTeamPossessionPlayer;
    Vec3 focus = Sp(w, pp).position + Vec3(-TeamDynamicSide(w, teamID) * 26.0f, 0, 0);
    return GetClosestPlayer(w, c, teamID, focus, true, pp);
}
HDN void TeamApplyAttackingRun(World &w, const Ctx &c, int teamID, int manualPlayer) {
    TeamAI &ai = TeamByID(w, teamID).ai;
    ai.endApplyAttackingRunMs = w.match.actualTimeMs + 4000;
    ai.attackingRunPlayer = manualPlayer >= 0 ? manualPlayer : SelectAttackingRunPlayer(w, c, teamID);
}

// What the team AI copies of the match each tick: who has the ball, the possession amounts and
// both teams' times to the ball.
HD void RefreshTeamView(World &w, int teamID) {
    const MatchState &m = w.match;
    const Team &team = TeamByID(w, teamID), &opp = TeamByID(w, 1 - teamID);
    TeamAI &ai = TeamByID(w, teamID).ai;
    ai.teamHasPossession = team.hasPossession;
    ai.teamHasUniquePossession = TeamHasUniquePossession(w, teamID);
    ai.oppTeamHasPossession = opp.hasPossession;
    ai.oppTeamHasUniquePossession = TeamHasUniquePossession(w, 1 - teamID);
    ai.teamHasBestPossession = m.bestPossessionTeam == TeamSlot(w, teamID);
    ai.teamPossessionAmount = team.teamPossessionAmount;
    ai.fadingTeamPossessionAmount = team.fadingTeamPossessionAmount;
    ai.timeNeededToGetToBall = team.timeToBallMs;
    ai.oppTimeNeededToGetToBall = opp.timeToBallMs;
}
// The x of the team's offside trap: the deepest (toward the team's own goal) of a line 30 to 50 m
// out from goal (nearer the more offensive the team), the ball pushed 20 to 30 m back when far
// out, the ball in 700 ms, the opponents' designated player 4 m goalside (tested 0.15 s ahead,
// placed 0.1 s ahead) and the offside line less 4 m of slack. False without an opponent
// designated player.
HD bool OffsideTrapLine(World &w, int teamID, float &x) {
    const MatchState &m = w.match;
    const TeamAI &ai = TeamByID(w, teamID).ai;
    const int side = TeamDynamicSide(w, teamID);
    const float offensive = ai.offensivenessBias;
    const float startDistance = 30.0f + 20.0f * offensive, forceDistance = 6.0f;
    float deepest = (kPitchHalfLength - startDistance) * side;
    const float push = 20.0f + 10.0f * (1.0f - offensive);
    float ball = BallPredict(m.ball, 0).v[0] * side;
    ball += push * (1.0f - NormalizedClamp(ball, kPitchHalfLength - startDistance - push, kPitchHalfLength - forceDistance));
    ball *= side;
    if (ball * side > deepest * side) deepest = ball;
    if (BallPredict(m.ball, 700).v[0] * side > deepest * side) deepest = BallPredict(m.ball, 700).v[0];
    const int carrier = TeamByID(w, 1 - teamID).designatedTeamPossessionPlayer;
    if (carrier < 0) return false;
    const SpatialState &cs = Sp(w, carrier);
    const float caution = 4.0f * side;
    if ((cs.position.v[0] + cs.movement.v[0] * 0.15f + caution) * side > deepest * side)
        deepest = cs.position.v[0] + cs.movement.v[0] * 0.1f + caution;
    const float offside = GetOffsideLine(w, MentalImageIndex(w, 0), teamID);
    const float slack = 4.0f;
    if (offside * side - slack > deepest * side) deepest = offside - slack * side;
    x = deepest;
    return true;
}
// The opponents by danger, most dangerous first (ties in state order, GRF's insertion sort below
// 17 elements): nearness to a point 2 m out from the team's goal line, a fifth of the way to the
// ball in 100 ms, scaled to 95%, and 5% more for their designated player.
HD void RankOpponentsByDanger(World &w, int teamID) {
    const MatchState &m = w.match;
    const Team &opp = TeamByID(w, 1 - teamID);
    TeamAI &ai = TeamByID(w, teamID).ai;
    const int side = TeamDynamicSide(w, teamID);
    const PlayerList opponents = TeamActivePlayers(w, 1 - teamID);
    Vec3 danger = Vec3((float)(((double)kPitchHalfLength - 2.0) * side), 0, 0);
    danger = danger * 0.8f + BallPredict(m.ball, 100).Get2D() * 0.2f;
    ai.tacticalOpponents.count = 0;
    for (int i = 0; i < opponents.count; i++) {
        TacticalOpponent e;
        e.player = opponents[i];
        e.dangerFactor = (1.0f - NormalizedClamp((Sp(w, opponents[i]).position - danger).Length(), 0, kPitchHalfLength * 2));
        e.dangerFactor *= 0.95f;
        if (opponents[i] == opp.designatedTeamPossessionPlayer) e.dangerFactor += 0.05f;
        int at = ai.tacticalOpponents.count;
        ai.tacticalOpponents.push_back(e);
        for (; at > 0 && e.dangerFactor > ai.tacticalOpponents[at - 1].dangerFactor; at--)
            ai.tacticalOpponents[at] = ai.tacticalOpponents[at - 1];
        ai.tacticalOpponents[at] = e;
    }
}
// Every half second, with the team best placed for the ball, at most one gamer and no run on, an
// attacking run starts when the runner is near the designated player (within 40 m, to the 0.5)
// and finds space 10 m ahead of it (the 4 nearest opponents within 15 m crowd it).
HD void ConsiderAttackingRun(World &w, const Ctx &c, int teamID) {
    const MatchState &m = w.match;
    const Team &team = TeamByID(w, teamID);
    if (!(m.actualTimeMs % 500 == 0 && team.ai.endApplyAttackingRunMs <= m.actualTimeMs && HumanGamerCount(team) < 2 &&
          m.bestPossessionTeam == TeamSlot(w, teamID)))
        return;
    const int runner = SelectAttackingRunPlayer(w, c, teamID);
    if (runner < 0) return;
    const Vec3 at = Sp(w, runner).position;
    const float near = libm::powf(1.0f - NormalizedClamp((at - Sp(w, team.designatedTeamPossessionPlayer).position).Length(), 0, 40), 0.5f);
    const Vec3 spot = at * Vec3(1.0f, 0.8f, 0.0f) + Vec3(TeamDynamicSide(w, teamID) * 10.0f, 0, 0);
    const PlayerList crowd = GetClosestPlayers(w, c, 1 - teamID, spot, false, 4);
    float space = 1.0f;
    for (int i = 0; i < crowd.count; i++)
        space -= libm::powf(Curve(1.0f - NormalizedClamp((Sp(w, crowd[i]).position - spot).Length(), 0, 15), 1.0f), 0.5f) * 0.3f;
    if (near * space >= 0.5f) TeamApplyAttackingRun(w, c, teamID, -1);
}

// The team AI's tick: tactics each second, the view of the match, the offside trap, the danger
// ranking, attacking runs and, every 1.5 s, the forward support player (the nearest to a point
// 1.5 m upfield of the designated player).
HDN bool TeamAIProcess(World &w, const Ctx &c, int teamID) {
    ENG_SCOPE(10);
    const MatchState &m = w.match;
    TeamAI &ai = TeamByID(w, teamID).ai;
    if (m.actualTimeMs % 1000 == 0) TeamUpdateTactics(w, teamID);
    RefreshTeamView(w, teamID);
    float trap = 0;
    if (!OffsideTrapLine(w, teamID, trap)) return Fail("the team AI finds no opponent possession player");
    ai.offsideTrapX = trap;
    RankOpponentsByDanger(w, teamID);
    ConsiderAttackingRun(w, c, teamID);
    if (m.actualTimeMs % 1500 == 0) {
        const int d = TeamByID(w, teamID).designatedTeamPossessionPlayer;
        const Vec3 ahead = Sp(w, d).position * Vec3(1.0f, 1.0f, 0.0f) + Vec3(-TeamDynamicSide(w, teamID) * 1.5f, 0, 0);
        ai.forwardSupportPlayer = GetClosestPlayer(w, c, teamID, ahead, false, d);
    }
    return true;
}

// ---- dynamic roles: an integer assignment problem (GRF's libhungarian) -----------------------------
constexpr int kHungarianMax = kTeamPlayers;
// Reduces `cost` (size x size, row-major) in place and returns the total cost, or -1 when the
// reduced costs fail to prove the assignment optimal. `colOfRow` is written only on success.
// The steps follow the published Hungarian method of libhungarian so ties resolve alike.
HDN int HungarianSolve(int *cost, int n, int *colOfRow) {
    const int kInf = 0x7FFFFFFF;
    auto C = [&](int r, int c) -> int & { return cost[r * n + c]; };
    int col_of[kHungarianMax], unchosen[kHungarianMax], rowDec[kHungarianMax], slackRow[kHungarianMax],
        rowOf[kHungarianMax], parent[kHungarianMax], colInc[kHungarianMax], slack[kHungarianMax];
    for (int i = 0; i < n; i++) col_of[i] = unchosen[i] = rowDec[i] = slackRow[i] = rowOf[i] = parent[i] = colInc[i] = slack[i] = 0;
    int total = 0, r = 0, c = 0, t = 0, q = 0, unmatched = 0, s = 0;
    for (c = 0; c < n; c++) {
        s = C(0, c);
        for (r = 1; r < n; r++)
            if (C(r, c) < s) s = C(r, c);
        total += s;
        if (s != 0)
            for (r = 0; r < n; r++) C(r, c) -= s;
    }
    for (c = 0; c < n; c++) {
        rowOf[c] = -1;
        parent[c] = -1;
        colInc[c] = 0;
        slack[c] = kInf;
    }
    for (r = 0; r < n; r++) {
        s = C(r, 0);
        for (c = 1; c < n; c++)
            if (C(r, c) < s) s = C(r, c);
        rowDec[r] = s;
        bool matched = false;
        for (c = 0; c < n; c++)
            if (s == C(r, c) && rowOf[c] < 0) {
                col_of[r] = c;
                rowOf[c] = r;
                matched = true;
                break;
            }
        if (!matched) {
            col_of[r] = -1;
            unchosen[t++] = r;
        }
    }
    if (t != 0) {
        unmatched = t;
        for (;;) {
            // Grow the alternating tree until an unmatched column is reached.
            q = 0;
            bool breakthrough = false;
            while (!breakthrough) {
                while (q < t && !breakthrough) {
                    r = unchosen[q];
                    s = rowDec[r];
                    for (c = 0; c < n; c++) {
                        if (!slack[c]) continue;
                        int del = C(r, c) - s + colInc[c];
                        if (del < slack[c]) {
                            if (del == 0) {
                                if (rowOf[c] < 0) {
                                    breakthrough = true;
                                    break;
                                }
                                slack[c] = 0;
                                parent[c] = r;
                                unchosen[t++] = rowOf[c];
                            } else {
                                slack[c] = del;
                                slackRow[c] = r;
                            }
                        }
                    }
                    if (!breakthrough) q++;
                }
                if (breakthrough) break;
                s = kInf;
                for (c = 0; c < n; c++)
                    if (slack[c] && slack[c] < s) s = slack[c];
                for (q = 0; q < t; q++) rowDec[unchosen[q]] += s;
                for (c = 0; c < n; c++) {
                    if (slack[c]) {
                        slack[c] -= s;
                        if (slack[c] == 0) {
                            r = slackRow[c];
                            if (rowOf[c] < 0) {
                                for (int j = c + 1; j < n; j++)
                                    if (slack[j] == 0) colInc[j] += s;
                                breakthrough = true;
                                break;
                            }
                            parent[c] = r;
                            unchosen[t++] = rowOf[c];
                        }
                    } else {
                        colInc[c] += s;
                    }
                }
            }
            // Augment along the tree from (r, c).
            for (;;) {
                int j = col_of[r];
                col_of[r] = c;
                rowOf[c] = r;
                if (j < 0) break;
                r = parent[j];
                c = j;
            }
            if (--unmatched == 0) break;
            t = 0;
            for (c = 0; c < n; c++) {
                parent[c] = -1;
                slack[c] = kInf;
            }
            for (r = 0; r < n; r++)
                if (col_of[r] < 0) unchosen[t++] = r;
        }
    }
    for (r = 0; r < n; r++)
        for (c = 0; c < n; c++)
            if (C(r, c) < rowDec[r] - colInc[c]) return -1;
    for (r = 0; r < n; r++) {
        c = col_of[r];
        if (c < 0 || C(r, c) != rowDec[r] - colInc[c]) return -1;
    }
    r = 0;
    for (c = 0; c < n; c++)
        if (colInc[c]) r++;
    if (r > n) return -1;
    for (int i = 0; i < n; i++) colOfRow[i] = col_of[i];
    for (int i = 0; i < n; i++) total += rowDec[i];
    for (int i = 0; i < n; i++) total -= colInc[i];
    return total;
}

// Assigns the outfield formation slots to the players nearest them: costs are decimeters, and
// pairs beyond a growing cutoff cost 50000 until an assignment stays under it.
HDN bool TeamCalculateDynamicRoles(World &w, const Ctx &c, int teamID) {
    ENG_SCOPE(26);
    PlayerList all = TeamActivePlayers(w, teamID);
    PlayerList ps;
    if (!all.empty()) {
        // GRF: removes the first goalkeeper; only one listed first is supported.
        if (Formation(w, c, all[0]).role != kRoleGoalkeeper) return Fail("the dynamic roles need the goalkeeper first");
        for (int i = 1; i < all.count; i++) ps.push_back(all[i]);
    }
    const unsigned n = (unsigned)ps.count;
    Vec3 slots[kTeamPlayers];
    for (unsigned s = 0; s < n; s++) slots[s] = TeamAdaptedFormationPosition(w, c, ps[s], false);
    auto cost = [&](unsigned pi, unsigned si) {
        Vec3 pp = Sp(w, ps[pi]).position + Sp(w, ps[pi]).movement * 0.5f;
        return TruncToInt32(roundf((pp - slots[si]).Length() * 10));
    };
    int costs[kTeamPlayers * kTeamPlayers], sorted[kTeamPlayers * kTeamPlayers];
    int count = 0;
    for (unsigned pi = 0; pi < n; pi++)
        for (unsigned si = 0; si < n; si++) sorted[count++] = costs[pi * n + si] = cost(pi, si);
    for (int u = 1; u < count; u++)
        for (int s = u; s > 0 && sorted[s] < sorted[s - 1]; s--) {
            int x = sorted[s];
            sorted[s] = sorted[s - 1];
            sorted[s - 1] = x;
        }
    // GRF tries the cutoffs n, n + 5, ... in turn and keeps the first assignment that succeeds.
    // Each solve is independent of the others, so the lanes of the match solve consecutive
    // cutoffs together and the lowest that succeeds wins.
    const int cutoffs = (unsigned)count > n ? (int)(((unsigned)count - 1 - n) / 5 + 1) : 0;
    for (int c0 = 0; c0 < cutoffs; c0 += kGroupLanes) {
        const int ci = c0 + GroupRank();
        int colOfRow[kTeamPlayers];
        bool ok = false;
        if (ci < cutoffs) {
            const unsigned cutoff = n + 5 * (unsigned)ci;
            // A row is a formation slot, a column a player.
            int m[kTeamPlayers * kTeamPlayers];
            for (unsigned pi = 0; pi < n; pi++)
                for (unsigned si = 0; si < n; si++) {
                    int e = costs[pi * n + si];
                    if (e >= sorted[cutoff]) e = 50000;
                    m[pi + si * n] = e;
                }
            const int total = HungarianSolve(m, (int)n, colOfRow);
            ok = total != -1 && (total < 50000 || cutoff >= (unsigned)count - 5);
        }
        const LaneMask solved = GroupBallot(ok);
        if (!solved) continue;
        const int from = LowestBit(solved);
        int chosen[kTeamPlayers];
        for (unsigned si = 0; si < n; si++) chosen[si] = GroupShuffle((int32_t)colOfRow[si], from);
        for (unsigned pi = 0; pi < n; pi++)
            for (unsigned si = 0; si < n; si++)
                if (chosen[si] == (int)pi) {
                    const StaticFormation &f = Formation(w, c, ps[si]);
                    FormationEntry &e = w.match.players[ps[pi]].dynamicFormationEntry;
                    e.role = f.role;
                    e.position = f.position;
                    e.startPosition = f.startPosition;
                    e.lazy = f.lazy;
                    e.controllable = f.controllable;
                }
        break;
    }
    return true;
}

// How well player `p` marks opponent `o` (both 0.1 s ahead): the marker stands on a line across
// its way to the team's goal (half a metre behind it, 4 to 14 m each way); the opponent should be
// on the far side of that line, 2 m from it, and across from its middle. The quality loses up to
// half for distance from the line (to 60 m, to the 0.5) and half for distance from the middle
// (to the 0.5); an opponent on the near side counts 60%; a fifth is nearness (to the pitch's
// length).
HDN float MarkingQuality(const World &w, int teamID, int p, int o) {
    const int side = TeamDynamicSide(w, teamID);
    const SpatialState &ms = Sp(w, p), &os = Sp(w, o);
    const Vec3 opponent = os.position + os.movement * 0.1f, marker = ms.position + ms.movement * 0.1f;
    const Vec3 toGoal = Vec3(kPitchHalfLength * side, 0, 0) - marker;
    const float reach = Clamp((toGoal).Length(), 4.0f, 14.0f);
    const Vec3 home = toGoal.Normalized(Vec3(side, 0, 0));
    const Vec3 behind = -home * 0.5f;
    const Line across(marker + behind + home.Rotated2D((float)(-0.5 * (double)PI)) * reach,
                      marker + behind + home.Rotated2D((float)(0.5 * (double)PI)) * reach);
    const Vec3 &a = across.pts[0], &b = across.pts[1];
    const bool farSide = ((b.v[0] - a.v[0]) * (opponent.v[1] - a.v[1]) - (b.v[1] - a.v[1]) * (opponent.v[0] - a.v[0])) > 0;
    float along = 0.0f;
    const float fromLine = across.DistanceToPoint(opponent, along);
    const float offLine = libm::powf(NormalizedClamp(farSide ? fabsf(fromLine - 2.0f) : fromLine, 0.0f, 60.0f), 0.5f);
    const float offMiddle = libm::powf(Clamp(fabsf(along * 2.0f - 1.0f), 0.0f, 1.0f), 0.5f);
    float quality = 1.0f;
    quality -= offLine * 0.5f;
    quality -= offMiddle * 0.5f;
    quality = Clamp(quality, 0.0f, 1.0f);
    if (!farSide) quality *= 0.6f;
    const float nearness = (1.0f - NormalizedClamp((marker - opponent).Length(), 0.0f, kPitchHalfLength * 2.0f));
    return quality * 0.8f + nearness * 0.2f;
}
// The three most dangerous opponents get the best-placed outfield marker each, in danger order.
HDN bool TeamCalculateManMarking(World &w, const Ctx &c, int teamID) {
    ENG_SCOPE(27);
    const int marked = 3;
    const TeamAI &ai = TeamByID(w, teamID).ai;
    PlayerList ps = TeamActivePlayers(w, teamID);
    for (int i = 0; i < ps.count; i++) w.match.players[ps[i]].manMarking = -1;
    const int mc = ai.tacticalOpponents.count < marked ? ai.tacticalOpponents.count : marked;
    for (int rank = 0; rank < mc; rank++) {
        int best = -1, bestIndex = 0;
        float bestQ = -1.0f;
        const int o = ai.tacticalOpponents[rank].player;
        for (int i = 0; i < ps.count; i++) {
            if (Formation(w, c, ps[i]).role == kRoleGoalkeeper) continue;
            float qv = MarkingQuality(w, teamID, ps[i], o);
            if (qv > bestQ) {
                best = ps[i];
                bestQ = qv;
                bestIndex = i;
            }
        }
        if (best >= 0) {
            w.match.players[best].manMarking = o;
            for (int i = bestIndex; i + 1 < ps.count; i++) ps[i] = ps[i + 1];
            ps.count--;
        }
        if (ps.empty()) break;
    }
    return true;
}

// ---- the tick of a team -----------------------------------------------------------------------------
// A player's tick (team_process.h, PlayerProcess) around its humanoid's: the part before the
// humanoid's interruption, which returns the position the fatigue measures from, and the part after.
HDN bool PlayerProcessBegin(World &w, const Ctx &c, int p, Vec3 &before) {
    ENG_SCOPE(11);
    MatchState &m = w.match;
    Player &ps = m.players[p];
    ps.desiredTimeToBallMs = (ps.desiredTimeToBallMs - 10 < 0) ? 0 : ps.desiredTimeToBallMs - 10;
    if (ExternalControllerActive(w, p) && !HumanControllerProcess(w, c, p)) return false;
    ElizaControllerProcess(w, c, p);
    if (m.inPlay) {
        if (m.actualTimeMs % 1000 == 0) ps.base.positionHistoryPerSecond.push_back(ps.base.humanoid.spatial.position);
        if (ps.hasPossession) ps.possessionDurationMs += 10;
        else ps.possessionDurationMs = 0;
        if ((m.actualTimeMs + (uint64_t)(c.sd->stableID[p] * 10)) % 100 == 0) CalculateTacticalSituation(w, p);
    }
    before = ps.base.humanoid.spatial.position;
    HumanoidProcessBegin(w, c, p);
    return true;
}
HDN bool PlayerProcessEnd(World &w, const Ctx &c, int p, const Vec3 &before) {
    MatchState &m = w.match;
    Player &ps = m.players[p];
    if (!HumanoidProcessEnd(w, c, p)) return false;
    if (m.inPlay) {
        float d = (ps.base.humanoid.spatial.position - before).Length();
        // GRF: the raw statistic, without the difficulty and fatigue scaling.
        const float stamina = c.sd->data[p].stats[kStatStamina];
        ps.base.fatigueFactorInverse -= d * 0.00003f * (2.0f - stamina) * (1.0f / c.sd->matchDurationFactor);
        ps.base.fatigueFactorInverse = Clamp(ps.base.fatigueFactorInverse, 0.01f, 1.0f);
    }
    if (ps.cards > 1 && ps.cardEffectiveTimeMs <= m.actualTimeMs && TeamActivePlayers(w, w.playerTeamID[p]).size() > 1)
        return SendOff(w, c, p);
    return true;
}

// The team's possession amount: the opponents' time to the ball over its own (1.5 s added to
// each), and a fading amount that follows it (clamped to 0.5..1.5) at most 0.005 a tick. Out of
// play, at a set piece or with a retainer both are 1.5 for the team with (or best placed for) the
// ball and 0.5 for the other.
HD void UpdatePossessionAmounts(World &w, int teamID) {
    const MatchState &m = w.match;
    Team &t = TeamByID(w, teamID);
    const Team &opp = TeamByID(w, 1 - teamID);
    t.teamPossessionAmount = (float)(opp.timeToBallMs + 1500) / (float)(t.timeToBallMs + 1500);
    const float fading = t.fadingTeamPossessionAmount * 0.995f + Clamp(t.teamPossessionAmount, 0.5f, 1.5f) * 0.005f;
    t.fadingTeamPossessionAmount += Clamp(fading - t.fadingTeamPossessionAmount, -0.005f, 0.005f);
    if (m.inPlay && !m.inSetPiece && m.ballRetainer == -1) return;
    const bool ours = m.ballRetainer != -1 ? w.playerTeamID[m.ballRetainer] == teamID : m.bestPossessionTeam == TeamSlot(w, teamID);
    t.fadingTeamPossessionAmount = t.teamPossessionAmount = ours ? 1.5f : 0.5f;
}

// In play, a gamer's held switch button (GRF reads a held switch as a fresh press every tick)
// moves it off a player that does not alone hold the ball, unless it is already on the team's
// best and designated player with the team holding the ball: to the designated player, else the
// best one, when the team is best placed and no gamer holds them; else to the switch target. Never
// to the goalkeeper or an uncontrollable player. Out of play, from the third second, gamers with
// dynamic selection let go of their players. False on a switch with no selected player.
HD bool HonourSwitchButtons(World &w, const Ctx &c, int teamID) {
    MatchState &m = w.match;
    Team &t = TeamByID(w, teamID);
    if (!m.inPlay) {
        if (m.actualTimeMs < 2000) return true;
        if (DynamicPlayerSelection(w))
            for (int g = 0; g < t.gamers.count; g++)
                if (t.gamers[g].selectedPlayer >= 0) HumanGamerSetSelectedPlayer(w, GlobalGamerIndex(w, teamID, g), -1);
        t.mainSelectedPlayer = -1;
        return true;
    }
    for (int g = 0; g < t.gamers.count; g++) {
        const int selected = t.gamers[g].selectedPlayer, best = TeamBestPossessionPlayer(w, teamID);
        const bool settled = selected == best && selected == t.designatedTeamPossessionPlayer && !(t.teamPossessionAmount < 1.0f);
        if (!t.gamers[g].controller.keyboard.buttons[kBtnSwitch] || settled) continue;
        if (selected < 0) return Fail("the switch of a gamer that controls no player");
        if (m.players[selected].hasUniquePossession) continue;
        const bool bestPlaced = m.bestPossessionTeam == TeamSlot(w, teamID);
        int target;
        if (m.players[t.designatedTeamPossessionPlayer].base.externalController < 0 && bestPlaced) {
            target = t.designatedTeamPossessionPlayer;
        } else if (m.players[best].base.externalController < 0 && bestPlaced) {
            target = best;
        } else {
            target = SwitchTargetPlayer(w, c, teamID);
            if (target >= 0 && m.players[target].base.externalController >= 0) target = -1;
        }
        if (target == TeamGoalie(w, c, teamID)) target = -1;
        if (target >= 0 && Formation(w, c, target).controllable) {
            t.mainSelectedPlayer = target;
            HumanGamerSetSelectedPlayer(w, GlobalGamerIndex(w, teamID, g), target);
        }
    }
    return true;
}

// The team's designated player becomes its best one (the quickest to the ball) when that is
// clearly quicker: the ratio of their times (500 ms added to each) below 0.8, halved for a best
// player on the ball and doubled for a designated one, 20% easier for a gamer's best player and
// harder for a gamer's designated one, and harder for an AI best player while the designated one
// beats the opponents by more than 100 ms.
HD void ReconsiderDesignatedPlayer(World &w, int teamID) {
    const MatchState &m = w.match;
    Team &t = TeamByID(w, teamID);
    const int designated = t.designatedTeamPossessionPlayer, best = TeamBestPossessionPlayer(w, teamID);
    if (designated == best) return;
    const int current = (int)w.roster.timeToBallMs[designated];
    float ratio = (float)((int)w.roster.timeToBallMs[best] + 500) / (float)(current + 500);
    if (m.players[best].hasPossession) ratio *= 0.5f;
    if (m.players[designated].hasPossession) ratio /= 0.5f;
    if (ExternalControllerActive(w, best)) ratio *= 0.8f;
    if (ExternalControllerActive(w, designated)) ratio /= 0.8f;
    if (!ExternalControllerActive(w, best) && current < TeamByID(w, 1 - teamID).timeToBallMs - 100) {
        ratio += 0.2f;
        ratio *= 1.2f;
    }
    if (ratio < 0.8f) t.designatedTeamPossessionPlayer = best;
}

// A team's tick: possession amounts, gamers' automatic selection, the team AI with dynamic roles
// and man marking (staggered between the teams), its players, gamer switches and the designated
// player.
// Each active player's spatial state for the tick, on the group's lanes at once: it reads the
// player's own animation and last position only, which no other player's tick changes, so each
// player's turn takes it from the match's scratch block instead of computing it in order.
HDN void SpatialStatesAhead(World &w, const Ctx &c, int teamID) {
    const PlayerList ahead = TeamActivePlayers(w, teamID);
    for (int i = GroupRank(); i < ahead.count; i += kGroupLanes)
        c.ws->spatialAhead[ahead[i]] = NextSpatialState(c, Hum(w, ahead[i]));
    GroupSync();
}
HDN bool TeamProcess(World &w, const Ctx &c, int teamID) {
    ENG_SCOPE(25);
    MatchState &m = w.match;
    UpdatePossessionAmounts(w, teamID);
    TeamHumanGamersSelectAnyone(w, c, teamID);
    if (m.inPlay && !m.inSetPiece) {
        if (!TeamAIProcess(w, c, teamID)) return false;
        uint64_t off = teamID == (1 - w.FirstTeamID()) ? 200 : 0;
        if ((m.actualTimeMs + off) % 400 == 0 && !TeamCalculateDynamicRoles(w, c, teamID)) return false;
        if ((m.actualTimeMs + off + 100) % 400 == 0 && !TeamCalculateManMarking(w, c, teamID)) return false;
    }
    SpatialStatesAhead(w, c, teamID);
    // The active players of the team in state order, each checked when its turn comes. A match
    // whose next humanoid needs a new animation stops there until every match of the wavefront has
    // stopped or finished, so that the interruptions run together; each match still processes
    // its players in order.
    auto next = [&](int from) {
        while (from < m.playerCount && !(w.playerTeamID[from] == teamID && w.roster.active[from])) from++;
        return from;
    };
    int p = next(0);
    bool interrupted = false;
    Vec3 before;
    for (;;) {
        while (!interrupted && p < m.playerCount) {
            if (!PlayerProcessBegin(w, c, p, before)) return false;
            interrupted = Hum(w, p).interruptAnim != kIntNone;
            if (interrupted) break;
            if (!PlayerProcessEnd(w, c, p, before)) return false;
            p = next(p + 1);
        }
        if (!AnyLane(interrupted)) break;
        if (interrupted) {
            if (!HumanoidProcessInterrupt(w, c, p) || !PlayerProcessEnd(w, c, p, before)) return false;
            interrupted = false;
            p = next(p + 1);
        }
    }
    if (!HonourSwitchButtons(w, c, teamID)) return false;
    ReconsiderDesignatedPlayer(w, teamID);
    return true;
}

}  // namespace eng
