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

// The formation position (normalized to [-1, 1]) mapped into the team's current block and pulled
// towards the focus points.
HDN Vec3 GetAdaptedFormationPosition(const World &w, const Ctx &c, int p, float backX, float frontX, float lowY, float highY,
                                     float xFocus, float xFocusStrength, float yFocus, float yFocusStrength,
                                     const Vec3 &microFocus, float microFocusStrength, float midFocus,
                                     float midFocusStrength, bool dynamic) {
    int side = TeamDynamicSide(w, w.playerTeamID[p]);
    Vec3 pos = dynamic ? w.match.players[p].dynamicFormationEntry.position : Formation(w, c, p).position;
    if (midFocusStrength > 0.0f) {
        float factor = midFocus * 2.0f - 1.0f;
        float stretch = Clamp(1.0f - fabsf(pos.v[0] * 1.2f), 0.0f, 1.0f);
        stretch = Curve(stretch, 1.0f);
        stretch *= midFocusStrength;
        pos.v[0] = pos.v[0] * (1.0f - stretch) + factor * stretch;
    }
    float xl = frontX - backX;
    pos.v[0] = backX + (pos.v[0] * 0.5f + 0.5f) * xl;
    float yl = highY - lowY;
    pos.v[1] = lowY + (pos.v[1] * -side * 0.5f + 0.5f) * yl;
    Vec3 pure = pos;
    if (xFocusStrength > 0.0f) {
        float bias = 1.0f - Clamp(fabsf(xFocus - pos.v[0]) / fabsf(backX - frontX), 0.0f, 1.0f);
        bias = -libm::cosf(bias * PI) * 0.5f + 0.5f;
        bias = (float)libm::pow((double)bias, 0.8);
        bias *= xFocusStrength;
        pos.v[0] = pos.v[0] * (1.0f - bias) + xFocus * bias;
    }
    if (yFocusStrength > 0.0f) {
        float d = Clamp(fabsf(yFocus - pos.v[1]) / fabsf(highY - lowY), 0.0f, 1.0f);
        float bias = 1.0f - d;
        bias *= 0.2f + 0.8f * fabsf(yFocus) / kPitchHalfWidth;
        bias *= yFocusStrength;
        pos.v[1] = pos.v[1] * (1.0f - bias) + yFocus * bias;
    }
    if (microFocusStrength > 0.0f) {
        const float yInfluence = 0.2f, yPosition = 0.4f;
        float fd = ((microFocus - pure) * Vec3(1, 1.0f - yInfluence, 0)).Length() / 50.0f;
        if (fd < 1.0f) {
            float mb = 1.0f;
            mb *= 1.0f - fd;
            mb = Curve(mb, 0.3f);
            const float peakAt = 0.15f, peakWidth = 0.25f, peakHeight = 0.1f;
            mb += (1.0f - NormalizedClamp(fabsf(fd - peakAt), 0.0f, peakWidth)) * peakHeight;
            mb = Clamp(mb, 0.0f, 1.0f);
            mb *= microFocusStrength;
            Vec3 mfp = microFocus * Vec3(1, 1.0f - yPosition, 1) + pos * Vec3(0, yPosition, 0);
            pos = pos * (1.0f - mb) + mfp * (mb);
        }
    }
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

HDN Vec3 TeamAdaptedFormationPosition(const World &w, const Ctx &c, int p, bool dynamic, const FormationHistory &history) {
    const int t = w.playerTeamID[p];
    const int side = TeamDynamicSide(w, t);
    const TeamAI &ai = TeamByID(w, t).ai;
    const Tactics &tac = ai.liveTactics;
    const MatchState &m = w.match;
    int role = dynamic ? m.players[p].dynamicFormationEntry.role : Formation(w, c, p).role;
    Vec3 focal = Sp(w, m.designatedPossessionPlayer).position;
    const Vec3 *const averages = history.ball;
    float ballX = averages[0].v[0];
    float ballY = averages[1].v[1];
    auto T = [&](int id) { return Mixup(PropertiesGetReal(tac, id), id, role); };
    float offDepth = T(kOffenseDepth), defDepth = T(kDefenseDepth);
    float offWidth = T(kOffenseWidth), defWidth = T(kDefenseWidth);
    float offOwnHalf = T(kOffenseOwnHalf), defOwnHalf = T(kDefenseOwnHalf);
    float offMid = T(kOffenseMidfieldFocus), defMid = T(kDefenseMidfieldFocus);
    float offMidS = T(kOffenseMidfieldFocusStrength), defMidS = T(kDefenseMidfieldFocusStrength);
    float offSideS = T(kOffenseSideFocusStrength), defSideS = T(kDefenseSideFocusStrength);
    float offMicroS = T(kOffenseMicroFocusStrength), defMicroS = T(kDefenseMicroFocusStrength);
    const double mind = GetMindSet(role);
    offSideS = (float)((double)offSideS + (-0.5 + mind) * (double)0.2f);
    defSideS = (float)((double)defSideS + (0.5 - mind) * (double)0.2f);
    const float ob = ai.offensivenessBias;
    offSideS = Clamp(offSideS + -0.3f + (ob) * 0.3f, 0.0f, 1.0f);
    defSideS = Clamp(defSideS + -0.3f + (1.0f - ob) * 0.3f, 0.0f, 1.0f);
    float possAmount = NormalizedClamp(ai.fadingTeamPossessionAmount - 0.5f, 0.3f, 0.7f);
    float ballBias = NormalizedClamp(((ballX / kPitchHalfLength) * -side), -0.7f, 0.7f);
    float bbb = 1.0f - fabsf(possAmount * 2.0f - 1.0f);
    bbb *= 0.6f;
    float pb = possAmount * (1.0f - bbb) + ballBias * bbb;
    pb = Clamp(pb + (ob - 0.5f) * 0.3f, 0.0f, 1.0f);
    focal = (averages[2].Get2D() * 1.0f + focal * 0.0f) * pb + (averages[3].Get2D() * 0.5f + focal * 0.5f) * (1.0f - pb);
    float depth = ai.depth * (offDepth * pb + defDepth * (1.0f - pb));
    float width = ai.width * (offWidth * pb + defWidth * (1.0f - pb));
    float offsetX = kPitchHalfLength * side * ((offOwnHalf * 2.0f - 1.0f) * pb + (defOwnHalf * 2.0f - 1.0f) * (1.0f - pb));
    float sideS = (offSideS * pb + defSideS * (1.0f - pb));
    float sideFocus = pb * 2.0f - 1.0f;
    float sideX = 0.2f * sideFocus * -side * kPitchHalfLength + 0.8f * -history.possessionSide * kPitchHalfLength;
    float centerX = Clamp((ballX * (1.0f - sideS) + sideX * sideS) + offsetX, -kPitchHalfLength, kPitchHalfLength);
    float centerY = Clamp(ballY, -kPitchHalfWidth, kPitchHalfWidth);
    const float fitDepth = 0.95f, fitWidth = 0.9f;
    centerX *= ((1.0f - depth) / 1.0f) * fitDepth + (1.0f - fitDepth);
    centerY *= ((1.0f - width) / 1.0f) * fitWidth + (1.0f - fitWidth);
    float backX = centerX - depth * kPitchHalfLength * -side;
    float frontX = centerX + depth * kPitchHalfLength * -side;
    float lowY = centerY - width * kPitchHalfWidth;
    float highY = centerY + width * kPitchHalfWidth;
    if (backX * side > ai.offsideTrapX * side) backX = Clamp(ai.offsideTrapX, -kPitchHalfLength, kPitchHalfLength);
    float yFocus = ballY * 1.0f;
    float yFocusS = 0.5f * pb + 0.2f * (1.0f - pb);
    Vec3 micro = focal;
    Vec3 defensive = Vec3(Clamp(micro.v[0] + side * 2.0f, -kPitchHalfLength, backX * side), micro.v[1] * 0.9f, 0);
    micro = (Vec3(Clamp(micro.v[0] - side * 1.0f, -kPitchHalfLength, kPitchHalfLength), micro.v[1] * 0.9f, 0)) * pb +
            (defensive) * (1.0f - pb);
    float microS = (offMicroS * pb + defMicroS * (1.0f - pb));
    float msb = NormalizedClamp((ballX / kPitchHalfLength) * -side, -0.7f, 0.7f);
    msb = msb * 0.7f + 0.3f;
    float autoMicro = (libm::powf(msb, 0.8f) * pb + (libm::powf(1.0f - msb, 0.6f)) * (1.0f - pb));
    microS = microS * (0.2f + 0.8f * autoMicro);
    float manualMid = (offMid * pb + defMid * (1.0f - pb));
    float autoMid = NormalizedClamp((ballX / kPitchHalfLength) * -side, -0.8f, 0.8f);
    float midFocus = manualMid * 0.7f + autoMid * 0.3f;
    float midS = (offMidS * pb + defMidS * (1.0f - pb));
    Vec3 d = GetAdaptedFormationPosition(w, c, p, backX, frontX, lowY, highY, 0.0f, 0.0f, yFocus, yFocusS, micro, microS,
                                         midFocus, midS, dynamic);
    d.v[0] = Clamp(d.v[0], -kPitchHalfLength, kPitchHalfLength);
    d.v[1] = Clamp(d.v[1], -kPitchHalfWidth, kPitchHalfWidth);
    return d;
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
