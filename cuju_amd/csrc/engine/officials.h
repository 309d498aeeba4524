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
HDN void RefereeRequestCommand(World &w, const Ctx &ctx, int official, CommandQueue &q) {
    const MatchState &m = w.match;
    const SpatialState &s = m.officials[official].humanoid.spatial;
    const Vec3 pos = s.position;
    if (official == 0) {
        const Referee &ref = m.referee;
        if (ref.buffer.active && (ref.foul.foulType == 2 || ref.foul.foulType == 3) &&
            ref.buffer.prepareTime > m.actualTimeMs + 5000) {
            // Walk to two meters of the offender, then show the card (special variable 3).
            const Vec3 off = Sp(w, ref.foul.foulPlayer).position;
            Vec3 target = off + (pos - off).Normalized(0) * (float)2.0;
            if ((double)(pos - target).Length() > 2.0) {
                PlayerCommand c = DefaultPlayerCommand();
                c.useDesiredMovement = true;
                c.useDesiredLookAt = true;
                c.desiredDirection = (target - pos).Normalized(s.directionVec);
                c.desiredVelocityFloat = RangeVelocity((target - pos).Length() * 1.0f);
                c.desiredLookAt = off;
                q.push_back(c);
            } else {
                PlayerCommand c = DefaultPlayerCommand();
                c.desiredFunctionType = kFnSpecial;
                c.useSpecialVar1 = true;
                c.specialVar1 = 3;
                q.push_back(c);
                PlayerCommand f = DefaultPlayerCommand();
                f.useDesiredMovement = true;
                f.useDesiredLookAt = true;
                f.desiredDirection = (target - pos).Normalized(s.directionVec);
                f.desiredVelocityFloat = kIdleVelocity;
                f.desiredLookAt = off;
                q.push_back(f);
            }
        } else {
            PlayerCommand c = DefaultPlayerCommand();
            c.useDesiredMovement = true;
            c.useDesiredLookAt = true;
            ForceField &field = ctx.ws->forceField;
            field.clear();
            field.push_back(MakeSpot(BallAveragePosition(w, 2000).Get2D() * 0.6f, kAttract, kDecayConstant, 0.5f));
            field.push_back(MakeSpot(BallPredict(m.ball, 200).Get2D(), kRepel, kDecayVariable, 0.5f, 10.0f));
            const int first = w.FirstTeamID();
            for (int t = 0; t < 2; t++) {
                PlayerList ps = TeamActivePlayers(w, t == 0 ? first : 1 - first);
                for (int i = 0; i < ps.count; i++) {
                    const SpatialState &ps_s = Sp(w, ps[i]);
                    field.push_back(MakeSpot(ps_s.position + ps_s.movement * 0.4f, kRepel, kDecayVariable, 0.5f, 10.0f));
                }
            }
            Vec3 target = pos + GetForceFieldMovement(field, pos);
            c.desiredDirection = (target - pos).Normalized(s.directionVec);
            c.desiredVelocityFloat =
                Clamp((target - pos).Length() * kDistanceToVelocity * 0.5f, kIdleVelocity, kSprintVelocity);
            c.desiredLookAt = BallPredict(m.ball, 60).Get2D();
            q.push_back(c);
        }
    } else {
        // A linesman follows the offside line of the team whose half he runs along.
        PlayerCommand c = DefaultPlayerCommand();
        c.useDesiredMovement = true;
        c.useDesiredLookAt = true;
        const int latest = MentalImageIndex(w, 0);
        float line;
        Vec3 target;
        if (pos.v[1] < 0) {
            line = GetOffsideLine(w, latest, 1);
            target = Vec3(line, -(kPitchHalfWidth + 0.8f), 0);
        } else {
            line = GetOffsideLine(w, latest, 0);
            target = Vec3(line, kPitchHalfWidth + 0.8f, 0);
        }
        c.desiredDirection = (target - pos).Normalized(s.directionVec);
        c.desiredVelocityFloat = RangeVelocity((target - pos).Length() * kDistanceToVelocity);
        c.desiredLookAt = Vec3(target.v[0], 0, 0);
        q.push_back(c);
    }
}

// The tick of an official's humanoid: the player tick without touches, smuggles or requeues.
HDN bool OfficialHumanoidProcess(World &w, const Ctx &c, int official) {
    const int hi = w.match.playerCount + official;
    Humanoid &h = w.match.officials[official].humanoid;
    AnimationState &cur = h.anim;
    h.decayingPositionOffset *= 0.95f;
    if ((double)h.decayingPositionOffset.Length() < 0.005) h.decayingPositionOffset = Vec3(0);
    h.decayingDifficultyFactor = Clamp(h.decayingDifficultyFactor - 0.002f, 0.0f, 1.0f);
    CalculateSpatialState(c, h);
    h.spatial.positionOffsetMovement = Vec3(0);
    cur.frameNum++;
    h.prevAnimFrameNum++;
    if (cur.frameNum == c.A(cur.anim).frameCount - 1 && h.interruptAnim == kIntNone) h.interruptAnim = kIntSwitch;
    if (h.interruptAnim != kIntNone) {
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
        for (int i = 0; i < q.count; i++) {
            Selector sel(w, c, hi);
            SelectResult r = sel.BaseSelectAnimation(q[i], h.interruptAnim);
            if (r == kSelectUnsupported) return false;
            found = r == kSelectTrue;
            if (found) break;
        }
        if (found) {
            h.startPos = h.spatial.position;
            h.startAngle = h.spatial.angle;
            {
                Selector sel(w, c, hi);
                Vec3 np;
                float na;
                sel.CalculatePredictedSituation(np, na);
                h.nextStartPos = np;
                h.nextStartAngle.set(na);
            }
            h.applyBuf.anim = cur.anim;
            h.applyBuf.smooth = true;
            h.applyBuf.smoothFactor = (h.interruptAnim == kIntSwitch) ? 0.6f : 1.0f;
            float diff = c.D(cur.anim).difficultyFactor;
            if (diff > h.decayingDifficultyFactor) h.decayingDifficultyFactor = diff;
            if (h.interruptAnim == kIntReQueue && h.prevAnimFunctionType == cur.functionType) h.requeueDelayFrames = 32;
        }
    }
    h.requeueDelayFrames = (int)Clamp((float)(h.requeueDelayFrames - 1), 0, 10000);
    h.interruptAnim = kIntNone;
    const Anim &a = c.A(cur.anim);
    float fb = (cur.frameNum + 1) / (float)((a.frameCount - 1) + 1);
    cur.rotationSmuggleOffset.set(cur.rotationSmuggleBegin.value() * (1.0f - fb) + cur.rotationSmuggleEnd.value() * fb);
    h.applyBuf.frameNum = cur.frameNum;
    // Official: start + smuggles + frame position, in that order of addition.
    Vec3 base = h.startPos + cur.actionSmuggleOffset + cur.actionSmuggleSustainOffset + cur.movementSmuggleOffset;
    if ((uint32_t)cur.positions.count > (uint32_t)cur.frameNum) {
        h.applyBuf.position = base + cur.positions[cur.frameNum];
        h.applyBuf.orientation.set(h.startAngle.value() + cur.rotationSmuggleOffset.value());
        h.applyBuf.noPos = true;
    } else {
        h.applyBuf.position = base;
        h.applyBuf.orientation = h.startAngle;
        h.applyBuf.noPos = false;
    }
    for (int i = 0; i < kBodyParts; i++) h.applyBuf.offsets[i] = h.offsets[i];
    return true;
}
HDN bool OfficialsProcess(World &w, const Ctx &c) {
    ENG_SCOPE(15);
    for (int o = 0; o < 3; o++)
        if (!OfficialHumanoidProcess(w, c, o)) return false;
    return true;
}

}  // namespace eng
