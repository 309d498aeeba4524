// SPDX-License-Identifier: Apache-2.0
// Restates game logic of cuju (Copyright 2026 The cuju Authors), a reimplementation of Google
// Research Football (Copyright 2019 Google LLC); see NOTICE.
// The built-in player AI: formation positions, the offside trap, the commands of a player without a
// gamer and of a gamer's player. Expressions with a double literal run in double, as in GRF.
// Semantics: include/cuju/simulation/ai_controller.h:16-2494.
#pragma once

#include "team_base.h"

namespace eng {

HD float GetMindSet(int role) {
    switch (role) {
        case kRoleGoalkeeper:
        case kRoleCentreBack: return 0.0f;
        case kRoleLeftBack:
        case kRoleRightBack:
        case kRoleDefensiveMid: return 0.25f;
        case kRoleAttackingMid: return 0.75f;
        case kRoleCentreForward: return 1.0f;
        default: return 0.5f;
    }
}
HD float ClampVelocity(float v) {
    if (v < 0) return 0;
    if (v > kSprintVelocity) return kSprintVelocity;
    return v;
}

// Gets the point at `self` clamped into the angular sector from `first` to `second`.
HDN Vec3 GetClamped2D(const Vec3 &self, const Vec3 &first, const Vec3 &second) {
    int dir = SignSide(second.Angle2D(first));
    float a1 = self.Angle2D(first), a2 = self.Angle2D(second);
    if (SignSide(a1) != dir || SignSide(a2) == dir) return fabsf(a1) < fabsf(a2) ? first : second;
    return self;
}
HDN void QuantizeDirection(Vec3 &in, float bias) {
    Vec3 n = in.Normalized(0);
    const int directions = 8;
    float a = n.Angle2D();
    a /= PI * 2.0f;
    a = roundf(a * directions);
    a /= directions;
    a *= PI * 2.0f;
    in = (n * (1.0f - bias) + (Vec3(1, 0, 0).Rotated2D(a) * bias)).Normalized(n) * in.Length();
}
constexpr float kQuantizedDirectionBias = 0.0f;
HD bool NeedDefendingMovement(int side, const Vec3 &pos, const Vec3 &target) {
    float deep = MaxF((target.v[0] - pos.v[0]) * -side, 0.0f);
    float wide = fabsf(target.v[1] - pos.v[1]);
    deep -= 0.5f;
    return wide > deep * 0.8f;
}
// GRF: a player missing from the mental image gets the image's first entry.
// The first entry of player `p` is found eight entries at a time: a batch's player numbers load
// together, and the lowest matching index wins.
HDN PlayerImage MentalPlayerImage(const World &w, int k, int p) {
    const MentalImage &mi = w.match.mentalImages[k];
    const int age = (int)(w.match.actualTimeMs - (uint64_t)mi.timeStampMs);
    const int count = mi.players.count;
    int found = -1;
    for (int first = 0; first < count && found < 0; first += 8) {
        int ids[8];
#pragma unroll
        for (int j = 0; j < 8; j++) ids[j] = mi.players[first + j < count ? first + j : count - 1].player;
#pragma unroll
        for (int j = 7; j >= 0; j--)
            if (first + j < count && ids[j] == p) found = first + j;
    }
    if (found >= 0) {
        const PlayerImage im = MentalImageEntry(w, mi, found);
        PlayerImage r = im;
        const SpatialState &s = Sp(w, im.player);
        r.position = im.position + im.movement * (float)age * 0.001f;
        r.position = r.position.EnforceMaximumDeviation(s.position, mi.maxDistanceDeviation);
        r.movement = r.movement.EnforceMaximumDeviation(s.movement, mi.maxMovementDeviation);
        return r;
    }
    return count > 0 ? MentalImageEntry(w, mi, 0) : mi.players[0];
}
HDN float PlayerAverageVelocity(const World &w, int p, float periodS) {
    const auto &hist = w.match.players[p].base.positionHistoryPerSecond;
    unsigned n = hist.count;
    if (n == 0) return 0;
    Vec3 prev;
    float total = 0;
    unsigned k = 0;
    while (k <= (unsigned)periodS) {
        Vec3 pos = hist[n - 1 - k];
        if (k > 0) total += (pos - prev).Length();
        k++;
        if (n - k == 0) break;
        prev = pos;
    }
    return total / periodS;
}
HD bool AllowLastDitchOf(const World &w, int p, bool withPossessionAmount = true) {
    const Player &ps = w.match.players[p];
    if (withPossessionAmount && TeamByID(w, w.playerTeamID[p]).teamPossessionAmount < 1.0f) return true;
    return (float)ps.timeToBallOptimisticMs * 1.7f + 800 < (float)ps.timeToBallMs;
}
// The mean of the newest min(count, ms / 10 + 1) possession sides, summed newest first. The
// entries load in batches of 16 (indexes clamped into the history) so that a batch waits for
// memory once; the additions keep their order.
HD float AveragePossessionSide(const World &w, unsigned ms) {
    const auto &h = w.match.possessionSideHistory;
    const unsigned cap = ms / 10 + 1;
    const int k = (unsigned)h.count < cap ? h.count : (int)cap;
    float total = 0;
    for (int first = 0; first < k; first += 16) {
        float batch[16];
#pragma unroll
        for (int j = 0; j < 16; j++) batch[j] = h[h.count - 1 - (first + j < k ? first + j : k - 1)];
#pragma unroll
        for (int j = 0; j < 16; j++) {
            if (first + j >= k) break;
            total += batch[j];
        }
    }
    if (k > 0) total /= (float)k;
    return total;
}

// GRF: every team shares these two dribble settings.
constexpr float kDribbleOffensiveness = 0.5f;
constexpr float kDribbleCenterMagnet = 0.72f;
// Role-specific shifts of a tactic value.
HDN float Mixup(float base, int id, int role) {
    float v = -100.0f;
    if (role == kRoleCentreBack && id == kOffenseWidth) v = 0.2f;
    if (role == kRoleLeftBack || role == kRoleRightBack) {
        if (id == kDefenseOwnHalf) v = -0.075f;
        if (id == kOffenseWidth) v = 0.2f;
        if (id == kOffenseOwnHalf) v = -0.1f;
    }
    if (role == kRoleLeftMid || role == kRoleRightMid) {
        if (id == kDefenseOwnHalf) v = -0.05f;
        if (id == kOffenseOwnHalf) v = -0.1f;
    }
    if ((role == kRoleAttackingMid || role == kRoleCentreForward) && id == kDefenseDepth) v = 0.125f;
    if (v > -100.0f) return Clamp(base + v, 0.0f, 1.0f);
    return base;
}

// ---- formation positions -------------------------------------------------------------------------
// A player's place comes from its formation position (x and y in [-1, 1]) mapped into a block of
// the pitch (`back` to `front` along x, `low` to `high` across) and pulled toward focus points.
// The restarts set the block and foci by rule; in play the team's tactics and the ball set them.
struct Placement {
    float back, front, low, high;
    float xFocus, xFocusStrength, yFocus, yFocusStrength;
    Vec3 microFocus;
    float microFocusStrength;
    float midFocus, midFocusStrength;
};
// Formation x squeezed toward a midfield line (`focus` in 0..1 across the formation's length),
// most for the middle of the formation (none beyond 1/1.2 of its half length).
HD float StretchTowardMidfield(float x, float focus, float strength) {
    const float line = focus * 2.0f - 1.0f;
    float stretch = Clamp(1.0f - fabsf(x * 1.2f), 0.0f, 1.0f);
    stretch = Curve(stretch, 1.0f);
    stretch *= strength;
    return x * (1.0f - stretch) + line * stretch;
}
// The pull toward the x focus: up to `strength`, easing (a cosine, to the 0.8 in double) with
// nearness over the block's length.
HD float PullTowardX(float x, const Placement &r) {
    float bias = 1.0f - Clamp(fabsf(r.xFocus - x) / fabsf(r.back - r.front), 0.0f, 1.0f);
    bias = -libm::cosf(bias * PI) * 0.5f + 0.5f;
    bias = (float)libm::pow((double)bias, 0.8);
    bias *= r.xFocusStrength;
    return x * (1.0f - bias) + r.xFocus * bias;
}
// The pull toward the y focus: up to `strength`, by nearness over the block's width, more for a
// focus far from the centre line.
HD float PullTowardY(float y, const Placement &r) {
    float bias = 1.0f - Clamp(fabsf(r.yFocus - y) / fabsf(r.high - r.low), 0.0f, 1.0f);
    bias *= 0.2f + 0.8f * fabsf(r.yFocus) / kPitchHalfWidth;
    bias *= r.yFocusStrength;
    return y * (1.0f - bias) + r.yFocus * bias;
}
// The pull toward the micro focus of the block position `unpulled`, within 50 m (across distance
// counted at 80%): falling with distance (curved), with a bump of 0.1 around 15% of the range; the
// focus keeps 60% of its y and takes 40% of the player's.
HD Vec3 PullTowardMicro(const Vec3 &pos, const Vec3 &unpulled, const Placement &r) {
    const float yInfluence = 0.2f, yPosition = 0.4f;
    const float reach = ((r.microFocus - unpulled) * Vec3(1, 1.0f - yInfluence, 0)).Length() / 50.0f;
    if (!(reach < 1.0f)) return pos;
    float bias = 1.0f;
    bias *= 1.0f - reach;
    bias = Curve(bias, 0.3f);
    const float peakAt = 0.15f, peakWidth = 0.25f, peakHeight = 0.1f;
    bias += (1.0f - NormalizedClamp(fabsf(reach - peakAt), 0.0f, peakWidth)) * peakHeight;
    bias = Clamp(bias, 0.0f, 1.0f);
    bias *= r.microFocusStrength;
    const Vec3 focus = r.microFocus * Vec3(1, 1.0f - yPosition, 1) + pos * Vec3(0, yPosition, 0);
    return pos * (1.0f - bias) + focus * (bias);
}
// Player p's place by a placement: its static (or dynamic) formation position squeezed toward
// the midfield line, mapped into the block (y mirrored for the side), then pulled toward the x, y
// and micro foci.
HDN Vec3 PlaceInFormation(const World &w, const Ctx &c, int p, const Placement &r, bool dynamic) {
    const int side = TeamDynamicSide(w, w.playerTeamID[p]);
    Vec3 pos = dynamic ? w.match.players[p].dynamicFormationEntry.position : Formation(w, c, p).position;
    if (r.midFocusStrength > 0.0f) pos.v[0] = StretchTowardMidfield(pos.v[0], r.midFocus, r.midFocusStrength);
    pos.v[0] = r.back + (pos.v[0] * 0.5f + 0.5f) * (r.front - r.back);
    pos.v[1] = r.low + (pos.v[1] * -side * 0.5f + 0.5f) * (r.high - r.low);
    const Vec3 unpulled = pos;
    if (r.xFocusStrength > 0.0f) pos.v[0] = PullTowardX(pos.v[0], r);
    if (r.yFocusStrength > 0.0f) pos.v[1] = PullTowardY(pos.v[1], r);
    if (r.microFocusStrength > 0.0f) pos = PullTowardMicro(pos, unpulled, r);
    return pos;
}

// What a player's formation position reads of the match's history: four averages of the ball's
// positions, over durations that shorten as the player nears the possession player, from one pass
// over the history, and the average possession side over 6 s. A player's static and dynamic
// formation positions read the same ones.
struct FormationHistory {
    Vec3 ball[4];
    float possessionSide;
};
HDN FormationHistory FormationHistoryOf(const World &w, int p) {
    const Vec3 focal = Sp(w, w.match.designatedPossessionPlayer).position;
    const float urgency = 1.0f - NormalizedClamp((focal - Sp(w, p).position).Length(), 2.0f, 30.0f);
    const unsigned durations[4] = {TruncToUint32(3500 * (1.0f - urgency * 0.7f)), TruncToUint32(4000 * (1.0f - urgency * 0.5f)),
                                   3000, 2000};
    FormationHistory h;
    BallAveragePositions(w, durations, h.ball);
    h.possessionSide = AveragePossessionSide(w, 6000);
    return h;
}

// The tactic values a role plays to (GRF's live tactics with the role's mixups): depth, width,
// own-half offset, midfield focus and strengths, offensive and defensive. The side focus strengths
// lean by the role's mindset and the team's offensiveness.
struct RoleTactics {
    float offDepth, defDepth, offWidth, defWidth, offOwnHalf, defOwnHalf, offMid, defMid, offMidS, defMidS, offSideS, defSideS,
        offMicroS, defMicroS;
};
HD RoleTactics RoleTacticsOf(const TeamAI &ai, int role) {
    auto T = [&](int id) { return Mixup(PropertiesGetReal(ai.liveTactics, id), id, role); };
    RoleTactics t;
    t.offDepth = T(kOffenseDepth);
    t.defDepth = T(kDefenseDepth);
    t.offWidth = T(kOffenseWidth);
    t.defWidth = T(kDefenseWidth);
    t.offOwnHalf = T(kOffenseOwnHalf);
    t.defOwnHalf = T(kDefenseOwnHalf);
    t.offMid = T(kOffenseMidfieldFocus);
    t.defMid = T(kDefenseMidfieldFocus);
    t.offMidS = T(kOffenseMidfieldFocusStrength);
    t.defMidS = T(kDefenseMidfieldFocusStrength);
    t.offSideS = T(kOffenseSideFocusStrength);
    t.defSideS = T(kDefenseSideFocusStrength);
    t.offMicroS = T(kOffenseMicroFocusStrength);
    t.defMicroS = T(kDefenseMicroFocusStrength);
    const double mind = GetMindSet(role);
    t.offSideS = (float)((double)t.offSideS + (-0.5 + mind) * (double)0.2f);
    t.defSideS = (float)((double)t.defSideS + (0.5 - mind) * (double)0.2f);
    const float ob = ai.offensivenessBias;
    t.offSideS = Clamp(t.offSideS + -0.3f + (ob) * 0.3f, 0.0f, 1.0f);
    t.defSideS = Clamp(t.defSideS + -0.3f + (1.0f - ob) * 0.3f, 0.0f, 1.0f);
    return t;
}
// How offensively the team sets up, 0 to 1: its fading possession (0.8 to 1.2 maps to 0 to 1),
// blended (up to 60%, at even possession) with how far upfield the ball has been (within 70% of
// the half length), shifted by the team's offensiveness.
HD float AttackShare(const TeamAI &ai, float ballX, int side) {
    const float possession = NormalizedClamp(ai.fadingTeamPossessionAmount - 0.5f, 0.3f, 0.7f);
    const float upfield = NormalizedClamp(((ballX / kPitchHalfLength) * -side), -0.7f, 0.7f);
    float blend = 1.0f - fabsf(possession * 2.0f - 1.0f);
    blend *= 0.6f;
    const float share = possession * (1.0f - blend) + upfield * blend;
    return Clamp(share + (ai.offensivenessBias - 0.5f) * 0.3f, 0.0f, 1.0f);
}
// The block a team plays in: centred on the ball's averages (x shifted toward the possession side
// and by the own-half offset; y), squeezed toward the centre by the depth and width it spans
// (95% and 90% fit), never behind the offside trap.
HD void TeamBlock(const TeamAI &ai, const RoleTactics &t, float share, int side, float ballX, float ballY, float possessionSide,
                  Placement &r) {
    const float depth = ai.depth * (t.offDepth * share + t.defDepth * (1.0f - share));
    const float width = ai.width * (t.offWidth * share + t.defWidth * (1.0f - share));
    const float offsetX =
        kPitchHalfLength * side * ((t.offOwnHalf * 2.0f - 1.0f) * share + (t.defOwnHalf * 2.0f - 1.0f) * (1.0f - share));
    const float sideStrength = (t.offSideS * share + t.defSideS * (1.0f - share));
    const float sideX = 0.2f * (share * 2.0f - 1.0f) * -side * kPitchHalfLength + 0.8f * -possessionSide * kPitchHalfLength;
    float centerX = Clamp((ballX * (1.0f - sideStrength) + sideX * sideStrength) + offsetX, -kPitchHalfLength, kPitchHalfLength);
    float centerY = Clamp(ballY, -kPitchHalfWidth, kPitchHalfWidth);
    const float fitDepth = 0.95f, fitWidth = 0.9f;
    centerX *= ((1.0f - depth) / 1.0f) * fitDepth + (1.0f - fitDepth);
    centerY *= ((1.0f - width) / 1.0f) * fitWidth + (1.0f - fitWidth);
    r.back = centerX - depth * kPitchHalfLength * -side;
    r.front = centerX + depth * kPitchHalfLength * -side;
    r.low = centerY - width * kPitchHalfWidth;
    r.high = centerY + width * kPitchHalfWidth;
    if (r.back * side > ai.offsideTrapX * side) r.back = Clamp(ai.offsideTrapX, -kPitchHalfLength, kPitchHalfLength);
}
// The micro focus around the play (`focal`): a metre upfield when attacking, 2 m goalside (no
// deeper than the block's back) when defending, its y at 90%; its strength scaled by how far
// upfield (attacking) or back (defending) the ball has been.
HD void TeamMicroFocus(const RoleTactics &t, float share, int side, float ballX, const Vec3 &focal, Placement &r) {
    const Vec3 defensive = Vec3(Clamp(focal.v[0] + side * 2.0f, -kPitchHalfLength, r.back * side), focal.v[1] * 0.9f, 0);
    r.microFocus = (Vec3(Clamp(focal.v[0] - side * 1.0f, -kPitchHalfLength, kPitchHalfLength), focal.v[1] * 0.9f, 0)) * share +
                   (defensive) * (1.0f - share);
    const float strength = (t.offMicroS * share + t.defMicroS * (1.0f - share));
    float upfield = NormalizedClamp((ballX / kPitchHalfLength) * -side, -0.7f, 0.7f);
    upfield = upfield * 0.7f + 0.3f;
    const float automatic = (libm::powf(upfield, 0.8f) * share + (libm::powf(1.0f - upfield, 0.6f)) * (1.0f - share));
    r.microFocusStrength = strength * (0.2f + 0.8f * automatic);
}

// Player p's place in open play (GRF's adapted formation position): the role's tactics and the
// team's attack share set the block around the ball's recent averages, a y focus on the ball
// (stronger attacking), the micro focus around the play (the 3 s ball average attacking; the 2 s
// average halfway to the designated player defending), and a midfield focus from the tactics
// (70%) and the ball (30%). Clamped to the pitch.
HDN Vec3 TeamAdaptedFormationPosition(const World &w, const Ctx &c, int p, bool dynamic, const FormationHistory &history) {
    const int side = TeamDynamicSide(w, w.playerTeamID[p]);
    const TeamAI &ai = TeamByID(w, w.playerTeamID[p]).ai;
    const MatchState &m = w.match;
    const int role = dynamic ? m.players[p].dynamicFormationEntry.role : Formation(w, c, p).role;
    const float ballX = history.ball[0].v[0], ballY = history.ball[1].v[1];
    const RoleTactics t = RoleTacticsOf(ai, role);
    const float share = AttackShare(ai, ballX, side);
    const Vec3 designated = Sp(w, m.designatedPossessionPlayer).position;
    const Vec3 focal =
        (history.ball[2].Get2D() * 1.0f + designated * 0.0f) * share + (history.ball[3].Get2D() * 0.5f + designated * 0.5f) * (1.0f - share);
    Placement r{};
    TeamBlock(ai, t, share, side, ballX, ballY, history.possessionSide, r);
    r.xFocus = 0.0f;
    r.xFocusStrength = 0.0f;
    r.yFocus = ballY * 1.0f;
    r.yFocusStrength = 0.5f * share + 0.2f * (1.0f - share);
    TeamMicroFocus(t, share, side, ballX, focal, r);
    const float manualMid = (t.offMid * share + t.defMid * (1.0f - share));
    const float autoMid = NormalizedClamp((ballX / kPitchHalfLength) * -side, -0.8f, 0.8f);
    r.midFocus = manualMid * 0.7f + autoMid * 0.3f;
    r.midFocusStrength = (t.offMidS * share + t.defMidS * (1.0f - share));
    Vec3 place = PlaceInFormation(w, c, p, r, dynamic);
    place.v[0] = Clamp(place.v[0], -kPitchHalfLength, kPitchHalfLength);
    place.v[1] = Clamp(place.v[1], -kPitchHalfWidth, kPitchHalfWidth);
    return place;
}
HD Vec3 TeamAdaptedFormationPosition(const World &w, const Ctx &c, int p, bool dynamic) {
    return TeamAdaptedFormationPosition(w, c, p, dynamic, FormationHistoryOf(w, p));
}

// Pulls a position in front of the trap line back into a 4 m band around it.
HDN void TeamApplyOffsideTrap(const World &w, int teamID, Vec3 &pos) {
    const int side = TeamDynamicSide(w, teamID);
    const float trap = TeamByID(w, teamID).ai.offsideTrapX;
    const float half = 2.0f;
    float ax = pos.v[0] * side, at = trap * side;
    if (ax > at - half) {
        float front = at - half;
        float f = Clamp((ax - front) / (half * 2.0f), 0.0f, 1.0f);
        pos.v[0] = (front + half * f) * side;
    }
}

}  // namespace eng
