// SPDX-License-Identifier: Apache-2.0
// Restates game logic of cuju (Copyright 2026 The cuju Authors), a reimplementation of Google
// Research Football (Copyright 2019 Google LLC); see NOTICE.
// Player commands, the force fields and offside lines that the AI shares with the officials, and
// the tick of the referee and the two linesmen.
// Semantics: include/cuju/simulation/humanoid_process.h:18-83 (commands),
// include/cuju/simulation/officials.h:17-398.
#pragma once

#include "select.h"

namespace eng {

constexpr int kModifierKnockOn = 1;

HD PlayerCommand DefaultPlayerCommand() {
    PlayerCommand c{};
    c.desiredFunctionType = kFnMovement;
    c.desiredVelocityFloat = kIdleVelocity;
    c.strictMovement = kStrictDynamic;
    c.tripType = 1;
    c.touchInfo.targetPlayer = -1;
    c.touchInfo.forcedTargetPlayer = -1;
    return c;
}
HD PlayerCommand GetTripCommand(const Humanoid &h, const Vec3 &tripVector, int tripType) {
    PlayerCommand c = DefaultPlayerCommand();
    c.desiredFunctionType = kFnTrip;
    c.useDesiredTripDirection = true;
    c.desiredTripDirection = tripVector;
    c.desiredVelocityFloat = h.spatial.floatVelocity;
    c.useTripType = true;
    c.tripType = tripType;
    return c;
}
// Type 1 queues itself; 2 and 3 queue themselves, the other of the two, then type 1.
HD void AddTripCommandToQueue(const Humanoid &h, CommandQueue &q, int tripType) {
    q.push_back(GetTripCommand(h, h.tripDirection, tripType));
    if (tripType != 1) {
        q.push_back(GetTripCommand(h, h.tripDirection, tripType == 3 ? 2 : 3));
        q.push_back(GetTripCommand(h, h.tripDirection, 1));
    }
}
HD PlayerCommand GetBasicMovementCommand(const Humanoid &h, float velocity) {
    PlayerCommand c = DefaultPlayerCommand();
    c.useDesiredMovement = true;
    c.useDesiredLookAt = true;
    c.desiredDirection = h.spatial.directionVec;
    c.desiredVelocityFloat = velocity;
    c.desiredLookAt = h.spatial.position + c.desiredDirection * 10.0f;
    return c;
}

// ---- force fields -----------------------------------------------------------------------------------
constexpr float kDistanceToVelocity = 2.6f;
constexpr float kBallDistanceOptimizeThreshold = 10.0f;

HD ForceSpot MakeSpot(const Vec3 &origin, int magnet, int decay, float power, float scale = 0.0f,
                      float exponent = 1.0f) {
    ForceSpot s;
    s.origin = origin;
    s.magnet = magnet;
    s.decay = decay;
    s.power = power;
    s.scale = scale;
    s.exponent = exponent;
    return s;
}

// Sums run in spot order.
HDN Vec3 GetForceFieldMovement(const ForceField &field, const Vec3 &pos, float dampingDistance = 10) {
    Vec3 sum;
    float force = 0.0f;
    for (int i = 0; i < field.count; i++) {
        const ForceSpot &s = field[i];
        float d = (s.origin - pos).Length();
        float intensity = 1.0f;
        if (s.decay != kDecayConstant) {
            intensity = Clamp(1.0f - d / s.scale, 0.0f, 1.0f);
            if (s.exponent != 1.0f) intensity = libm::powf(intensity, s.exponent);
        }
        if (intensity > 0.0f) {
            Vec3 rel = s.origin - pos;
            rel.Normalize(0);
            if (s.magnet == kRepel) rel = -rel;
            else if (d < dampingDistance) rel *= d / dampingDistance;
            float f = s.power * intensity;
            sum += rel * f;
            force += f;
        }
    }
    if (force == 0.0f) return Vec3(0);
    return (sum / force) * kSprintVelocity;
}

// ---- mental images and offside lines ------------------------------------------------------------------
struct PlayerImagePos {
    Vec3 position, movement;
    int32_t role;
};
using ImageList = Small<PlayerImagePos, kPlayers>;

// The images of one team in the mental image's order, extrapolated to now and held within the
// image's deviation limits of the true state.
HDN void MentalTeamPlayerImages(const World &w, int k, int teamID, ImageList &out) {
    const MentalImage &mi = w.match.mentalImages[k];
    const int age = (int)(w.match.actualTimeMs - (uint64_t)mi.timeStampMs);
    out.clear();
    for (int i = 0; i < mi.players.count; i++) {
        const PlayerImage im = MentalImageEntry(w, mi, i);
        if (!w.roster.active[im.player] || w.playerTeamID[im.player] != teamID) continue;
        const SpatialState &s = Sp(w, im.player);
        Vec3 pos = im.position + im.movement * (float)age * 0.001f;
        PlayerImagePos e;
        e.position = pos.EnforceMaximumDeviation(s.position, mi.maxDistanceDeviation);
        e.movement = im.movement.EnforceMaximumDeviation(s.movement, mi.maxMovementDeviation);
        e.role = im.role;
        out.push_back(e);
    }
}
// Moves the images along x by `futureMs` in place. The deepest image is skipped (the keeper's
// place), the next deepest or the ball sets the line, which stays in the opponent half.
HDN float OffsideLineFromImages(ImageList &im, const Vec3 &ball, int side, unsigned futureMs) {
    int ignored = 0;
    for (int i = 0; i < im.count; i++) {
        im[i].position.v[0] += im[i].movement.v[0] * futureMs * 0.001f;
        if (im[i].position.v[0] * side > im[ignored].position.v[0] * side) ignored = i;
    }
    Vec3 deepest;
    for (int i = 0; i < im.count; i++)
        if (im[i].position.v[0] * side > deepest.v[0] * side && i != ignored) deepest = im[i].position;
    float line = deepest.v[0];
    if (ball.v[0] * side > line * side) line = ball.v[0];
    if (line * side < 0) line = 0;
    return Clamp(line, -kPitchHalfLength, kPitchHalfLength);
}
HDN float GetOffsideLine(const World &w, int k, int teamID, unsigned futureMs = 0) {
    ImageList im;
    MentalTeamPlayerImages(w, k, teamID, im);
    return OffsideLineFromImages(im, MentalBallPrediction(w, k, 0), TeamDynamicSide(w, teamID), futureMs);
}
// Mean of the last positions of the ball, newest first, about one entry per 10 ms.
// The averages of the ball's last positions over several durations, from one pass: a duration of
// d ms averages the newest min(count, d / 10 + 1) entries of the history, each mirrored when the
// ball's frame is, summed newest first; an empty history gives the ball's position. Every average
// is a prefix of the same running sum, so one pass records each at its length. The entries load
// in batches of 8 (indexes clamped into the history), so a batch waits for memory once; the
// additions keep their order.
template <int N>
HD void BallAveragePositions(const World &w, const unsigned (&durationsMs)[N], Vec3 (&out)[N]) {
    const Ball &b = w.match.ball;
    const int count = b.positionHistory.count;
    const Vec3 *const history = b.positionHistory.e;
    const bool flip = b.lazyFlip;
    // Fully unrolled over the N averages, so the lengths and sums stay in registers.
    int lengths[N];
    int longest = 0;
#pragma unroll
    for (int i = 0; i < N; i++) {
        const unsigned cap = durationsMs[i] / 10 + 1;
        lengths[i] = (unsigned)count < cap ? count : (int)cap;
        longest = lengths[i] > longest ? lengths[i] : longest;
    }
    Vec3 sum, sums[N];
    for (int first = 0; first < longest; first += 8) {
        Vec3 batch[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int k = first + j < longest ? first + j : longest - 1;
            batch[j] = history[count - 1 - k];
        }
        // Only a batch that holds the end of an average records sums.
        bool records = false;
#pragma unroll
        for (int i = 0; i < N; i++) records |= lengths[i] > first && lengths[i] <= first + 8;
        if (!records) {
#pragma unroll
            for (int j = 0; j < 8; j++) {
                Vec3 p = batch[j];
                if (flip) p.Mirror();
                sum += p;
            }
            continue;
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            if (first + j >= longest) break;
            Vec3 p = batch[j];
            if (flip) p.Mirror();
            sum += p;
#pragma unroll
            for (int i = 0; i < N; i++)
                if (lengths[i] == first + j + 1) sums[i] = sum;
        }
    }
#pragma unroll
    for (int i = 0; i < N; i++) {
        if (lengths[i] > 0) {
            out[i] = sums[i];
            out[i] /= Vec3((float)lengths[i]);
        } else {
            out[i] = BallPredict(b, 0);
        }
    }
}
HDN Vec3 BallAveragePosition(const World &w, unsigned durationMs) {
    const unsigned durations[1] = {durationMs};
    Vec3 avg[1];
    BallAveragePositions(w, durations, avg);
    return avg[0];
}

// ---- officials ---------------------------------------------------------------------------------------
// The officials' decisions are GRF's (include/cuju/simulation/officials.h); their organisation here
// (a command toward a target, one function per duty, the humanoid tick in stages) is this engine's.

// A command to move toward `target` at `velocity`, looking at `lookAt`; the direction falls back to
// the humanoid's own when the target is where it stands.
HD PlayerCommand HeadFor(const SpatialState &s, const Vec3 &target, float velocity, const Vec3 &lookAt) {
    PlayerCommand c = DefaultPlayerCommand();
    c.useDesiredMovement = true;
    c.useDesiredLookAt = true;
    c.desiredDirection = (target - s.position).Normalized(s.directionVec);
    c.desiredVelocityFloat = velocity;
    c.desiredLookAt = lookAt;
    return c;
}

// The referee books the player of a foul that earns a card: walks to two metres of the offender,
// then shows the card (special animation 3) and stands facing the offender.
HD void RefereeBooksOffender(const World &w, const SpatialState &s, CommandQueue &q) {
    const Vec3 pos = s.position;
    const Vec3 offender = Sp(w, w.match.referee.foul.foulPlayer).position;
    const Vec3 spot = offender + (pos - offender).Normalized(0) * (float)2.0;
    if ((double)(pos - spot).Length() > 2.0) {
        q.push_back(HeadFor(s, spot, RangeVelocity((spot - pos).Length() * 1.0f), offender));
        return;
    }
    PlayerCommand card = DefaultPlayerCommand();
    card.desiredFunctionType = kFnSpecial;
    card.useSpecialVar1 = true;
    card.specialVar1 = 3;
    q.push_back(card);
    q.push_back(HeadFor(s, spot, kIdleVelocity, offender));
}

// Otherwise the referee keeps near the recent play: drawn toward 60% of the ball's mean position
// over two seconds, pushed off where the ball will be in 200 ms and off every player's place in
// 400 ms, looking where the ball will be in 60 ms.
HD void RefereeFollowsPlay(const World &w, const Ctx &ctx, const SpatialState &s, CommandQueue &q) {
    const MatchState &m = w.match;
    const Vec3 pos = s.position;
    ForceField &field = ctx.ws->forceField;
    field.clear();
    field.push_back(MakeSpot(BallAveragePosition(w, 2000).Get2D() * 0.6f, kAttract, kDecayConstant, 0.5f));
    field.push_back(MakeSpot(BallPredict(m.ball, 200).Get2D(), kRepel, kDecayVariable, 0.5f, 10.0f));
    const int first = w.FirstTeamID();
    for (int k = 0; k < 2; k++) {
        const PlayerList players = TeamActivePlayers(w, k == 0 ? first : 1 - first);
        for (int i = 0; i < players.count; i++) {
            const SpatialState &p = Sp(w, players[i]);
            field.push_back(MakeSpot(p.position + p.movement * 0.4f, kRepel, kDecayVariable, 0.5f, 10.0f));
        }
    }
    const Vec3 target = pos + GetForceFieldMovement(field, pos);
    const float velocity = Clamp((target - pos).Length() * kDistanceToVelocity * 0.5f, kIdleVelocity, kSprintVelocity);
    q.push_back(HeadFor(s, target, velocity, BallPredict(m.ball, 60).Get2D()));
}

// A linesman runs along his touchline level with the offside line of the team defending his half,
// 0.8 m outside the pitch, looking across it.
HD void LinesmanFollowsLine(const World &w, const SpatialState &s, CommandQueue &q) {
    const Vec3 pos = s.position;
    const int latest = MentalImageIndex(w, 0);
    const bool lowerTouchline = pos.v[1] < 0;
    const float line = GetOffsideLine(w, latest, lowerTouchline ? 1 : 0);
    const Vec3 target(line, lowerTouchline ? -(kPitchHalfWidth + 0.8f) : kPitchHalfWidth + 0.8f, 0);
    q.push_back(HeadFor(s, target, RangeVelocity((target - pos).Length() * kDistanceToVelocity), Vec3(target.v[0], 0, 0)));
}

HDN void RefereeRequestCommand(World &w, const Ctx &ctx, int official, CommandQueue &q) {
    const MatchState &m = w.match;
    const SpatialState &s = m.officials[official].humanoid.spatial;
    if (official != 0) {
        LinesmanFollowsLine(w, s, q);
        return;
    }
    const Referee &ref = m.referee;
    const bool booking = ref.buffer.active && (ref.foul.foulType == 2 || ref.foul.foulType == 3) &&
                         ref.buffer.prepareTime > m.actualTimeMs + 5000;
    if (booking) RefereeBooksOffender(w, s, q);
    else RefereeFollowsPlay(w, ctx, s, q);
}

// An interrupted official takes the first command whose animation it finds, and starts that
// animation from where it stands, smoothed (less when it merely switches).
HDN bool OfficialInterrupt(World &w, const Ctx &c, int official) {
    const int hi = w.match.playerCount + official;
    Humanoid &h = w.match.officials[official].humanoid;
    CommandQueue &q = c.ws->commands;
    q.clear();
    if (h.interruptAnim == kIntTrip && h.tripType != 0) {
        AddTripCommandToQueue(h, q, h.tripType);
        h.tripType = 0;
        q.push_back(GetBasicMovementCommand(h, h.spatial.floatVelocity));
    } else {
        RefereeRequestCommand(w, c, official, q);
    }
    bool found = false;
    for (int i = 0; i < q.count && !found; i++) {
        Selector sel(w, c, hi);
        const SelectResult r = sel.SelectOfficialAnimation(q[i], h.interruptAnim);
        if (r == kSelectUnsupported) return false;
        found = r == kSelectTrue;
    }
    if (!found) return true;
    AnimationState &cur = h.anim;
    h.startPos = h.spatial.position;
    h.startAngle = h.spatial.angle;
    {
        Selector sel(w, c, hi);
        Vec3 nextPos;
        float nextAngle;
        sel.PredictedPose(nextPos, nextAngle);
        h.nextStartPos = nextPos;
        h.nextStartAngle.set(nextAngle);
    }
    h.applyBuf.anim = cur.anim;
    h.applyBuf.smooth = true;
    h.applyBuf.smoothFactor = (h.interruptAnim == kIntSwitch) ? 0.6f : 1.0f;
    const float difficulty = c.D(cur.anim).difficultyFactor;
    if (difficulty > h.decayingDifficultyFactor) h.decayingDifficultyFactor = difficulty;
    if (h.interruptAnim == kIntReQueue && h.prevAnimFunctionType == cur.functionType) h.requeueDelayFrames = 32;
    return true;
}

// The apply buffer of an official's frame: its start plus the smuggled offsets, plus the frame's
// planned position when the animation plans one (then the frame keeps the root in place).
HD void OfficialFillApplyBuffer(const Ctx &c, Humanoid &h) {
    AnimationState &cur = h.anim;
    const Anim &a = c.A(cur.anim);
    const float through = (cur.frameNum + 1) / (float)((a.frameCount - 1) + 1);
    cur.rotationSmuggleOffset.set(cur.rotationSmuggleBegin.value() * (1.0f - through) + cur.rotationSmuggleEnd.value() * through);
    AnimApplyBuffer &buf = h.applyBuf;
    buf.frameNum = cur.frameNum;
    // The start, then the smuggles, then the frame position, in that order of addition.
    const Vec3 base = h.startPos + cur.actionSmuggleOffset + cur.actionSmuggleSustainOffset + cur.movementSmuggleOffset;
    const bool planned = (uint32_t)cur.positions.count > (uint32_t)cur.frameNum;
    if (planned) {
        buf.position = base + cur.positions[cur.frameNum];
        buf.orientation.set(h.startAngle.value() + cur.rotationSmuggleOffset.value());
    } else {
        buf.position = base;
        buf.orientation = h.startAngle;
    }
    buf.noPos = planned;
    for (int i = 0; i < kBodyParts; i++) buf.offsets[i] = h.offsets[i];
}

// The tick of an official's humanoid: the player's tick without touches, smuggles or requeues.
HDN bool OfficialHumanoidProcess(World &w, const Ctx &c, int official) {
    Humanoid &h = w.match.officials[official].humanoid;
    AnimationState &cur = h.anim;
    // The offset from the last collision and the difficulty of the last animation fade.
    h.decayingPositionOffset *= 0.95f;
    if ((double)h.decayingPositionOffset.Length() < 0.005) h.decayingPositionOffset = Vec3(0);
    h.decayingDifficultyFactor = Clamp(h.decayingDifficultyFactor - 0.002f, 0.0f, 1.0f);
    h.spatial = c.ws->spatialAhead[kPlayers + official];
    h.prevPosition2D = h.spatial.position;
    h.spatial.positionOffsetMovement = Vec3(0);
    cur.frameNum++;
    h.prevAnimFrameNum++;
    // The last frame of an animation interrupts it.
    if (cur.frameNum == c.A(cur.anim).frameCount - 1 && h.interruptAnim == kIntNone) h.interruptAnim = kIntSwitch;
    if (h.interruptAnim != kIntNone && !OfficialInterrupt(w, c, official)) return false;
    h.requeueDelayFrames = (int)Clamp((float)(h.requeueDelayFrames - 1), 0, 10000);
    h.interruptAnim = kIntNone;
    OfficialFillApplyBuffer(c, h);
    return true;
}
HDN bool OfficialsProcess(World &w, const Ctx &c) {
    ENG_SCOPE(15);
    // The three spatial states for the tick at once, as a team's players' are: each reads its own
    // official's animation and last position, which the others' ticks leave alone.
    for (int o = GroupRank(); o < 3; o += kGroupLanes)
        c.ws->spatialAhead[kPlayers + o] = NextSpatialState(c, w.match.officials[o].humanoid);
    GroupSync();
    for (int o = 0; o < 3; o++)
        if (!OfficialHumanoidProcess(w, c, o)) return false;
    return true;
}

}  // namespace eng
