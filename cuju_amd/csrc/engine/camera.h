// SPDX-License-Identifier: Apache-2.0
// Restates game logic of cuju (Copyright 2026 The cuju Authors), a reimplementation of Google
// Research Football (Copyright 2019 Google LLC); see NOTICE.
// GRF's in-game camera. It never affects play, but its pose is part of the state and its shake
// draws two numbers a tick from the world RNG. Semantics: include/cuju/simulation/camera.h:15-170.
#pragma once

#include "world.h"

namespace eng {

HD float CameraWeight(int index, int count) {
    const float size = count;
    float w = libm::sinf((index / size - 0.3f) * 1.4f * PI) * 0.5f + 0.5f;
    w *= libm::powf(1.0f - index / size, 0.3f);
    return w;
}

// GRF updates the camera with team 1 mirrored. Of what the update reads, the mirror changes only
// the positions of team 1's players (x and y negated) and team 1's side (negated), so it reads
// those through `position` and `side` instead of mirroring the team there and back.
HDN void UpdateInGameCamera(World &w, const Ctx &c) {
    MatchState &m = w.match;
    const int first = w.FirstTeamID(), second = 1 - first;
    auto position = [&](int p) {
        Vec3 v = Sp(w, p).position;
        if (w.playerTeamID[p] == 1) v.Mirror();
        return v;
    };
    auto side = [&](int t) { return t == 1 ? -TeamDynamicSide(w, t) : TeamDynamicSide(w, t); };
    const float fovDefault = 0.4f, zoomDefault = 0.5f, heightDefault = 0.3f, angleDefault = 0.0f;
    float fov = 0.5f + fovDefault * 0.5f;
    float zoom = zoomDefault;
    float height = heightDefault * 1.5f;
    float playerBias = 0.6f;
    const SpatialState &ds = Sp(w, m.designatedPossessionPlayer);
    Vec3 bp = BallPredict(m.ball, 0) * (1.0f - playerBias) + position(m.designatedPossessionPlayer) * playerBias;
    bp += ds.directionVec * 1.0f;
    bp += Vec3(((TeamByID(w, first).fadingTeamPossessionAmount - 1.0f) * -side(first) +
                (TeamByID(w, second).fadingTeamPossessionAmount - 1.0f) * -side(second)) *
                   4.0f,
               0, 0);
    bp.v[2] *= 0.1f;
    float maxW = (float)((double)(kPitchHalfLength * 0.84f) * (1.0 / (double)(zoom + 0.01f)));
    float maxH = (float)((double)(kPitchHalfWidth * 0.60f) * (1.0 / (double)(zoom + 0.01f)) * (double)(height * 0.75f + 0.25f));
    if (fabsf(bp.v[0]) > maxW) bp.v[0] = maxW * SignSide(bp.v[0]);
    if (fabsf(bp.v[1]) > maxH) bp.v[1] = maxH * SignSide(bp.v[1]);
    // GRF: the arguments evaluate right to left, so the shake draws y before x.
    float ry = RandomInRange(w, -0.1f, 0.1f);
    float rx = RandomInRange(w, -0.1f, 0.1f);
    Vec3 shudder = Vec3(rx, ry, 0) * (m.ball.momentum.Length() * 0.8f + 6.0f);
    shudder *= 0.2f;
    auto &cp = m.cameraPosition;
    Vec3 add = bp + shudder * ((float)cp.count / (float)kCameraHistory);
    if (cp.count == kCameraHistory) {
        GroupShiftDown<4>(cp.e, cp.count - 1);
        cp[cp.count - 1] = add;
    } else {
        cp.push_back(add);
    }
    Vec3 avg;
    float n = 0;
    const int pc = cp.count;
    const float *table = c.t->cameraWeights + pc * (pc - 1) / 2;
    // The sums run in order; the entries load eight at a time, so their loads overlap in flight.
    constexpr int kChunk = 8;
    for (int i0 = 0; i0 < pc; i0 += kChunk) {
        float wt[kChunk];
        Vec3 at[kChunk];
        for (int j = 0; j < kChunk; j++)
            if (i0 + j < pc) {
                wt[j] = table[i0 + j];
                at[j] = cp[i0 + j];
            }
        for (int j = 0; j < kChunk; j++)
            if (i0 + j < pc) {
                avg += at[j] * wt[j];
                n += wt[j];
            }
    }
    avg /= Vec3(n);
    float angleFactor = 1.0f - angleDefault * 0.4f;
    if (!m.goalScored || (m.goalScored && m.goalScoredTimer < 1000)) {
        zoom = (0.6f + zoom * 1.0f) * (1.0f / fov);
        height = 4.0f + height * 10;
        float distRot = avg.v[1] / 800.0f;
        m.cameraOrientation.SetAngleAxis(distRot + (0.42f - height * 0.01f) * PI, Vec3(1, 0, 0));
        m.cameraNodeOrientation.SetAngleAxis((-avg.v[0] / kPitchHalfLength) * (1.0f - angleFactor) * 0.25f * PI * 1.24f,
                                             Vec3(0, 0, 1));
        m.cameraNodePosition =
            avg * Vec3(1.0f * (1.0f - angleDefault * 0.2f) * (1.0f - zoomDefault * 0.3f), 0.9f - zoomDefault * 0.3f, 0.2f) +
            Vec3(0, -41.4f - (fovDefault * 3.7f) + libm::powf(height, 1.2f) * 0.46f, 10.0f + height) * zoom;
        m.cameraFov = (fov * 28.0f) - (m.cameraNodePosition.v[1] / 30.0f);
        m.cameraNearCap = m.cameraNodePosition.v[2];
        m.cameraFarCap = 200;
    } else {
        Vec3 target = BallPredict(m.ball, 0).Get2D();
        if (m.lastGoalScorer >= 0) target = position(m.lastGoalScorer);
        float rot = (float)m.goalScoredTimer * 0.0005f;
        m.cameraOrientation.SetAngleAxis(0.45f * PI, Vec3(1, 0, 0));
        m.cameraNodeOrientation.SetAngleAxis(rot, Vec3(0, 0, 1));
        m.cameraNodePosition = target + Vec3(0, -1, 0).Rotated2D(rot) * 15.0f + Vec3(0, 0, 3);
        m.cameraFov = 35.0f;
        m.cameraNearCap = 1;
        m.cameraFarCap = 220;
    }
}

// The camera works on the unmirrored pitch: GRF mirrors team 1 around its update, which
// UpdateInGameCamera reads in place.
HDN void UpdateCamera(World &w, const Ctx &c) {
    ENG_SCOPE(19);
    MatchState &m = w.match;
    if (m.autoUpdateInGameCamera) UpdateInGameCamera(w, c);
    const unsigned zoomTime = 2000, startTime = 0;
    if (m.actualTimeMs < zoomTime + startTime) {
        Quat init(0, 0, 0, 1);
        init.SetAngleAxis(0.0f * PI, Vec3(1, 0, 0));
        Quat heading(0, 0, 0, 1);
        init = heading * init;
        Vec3 initPos = Vec3(0.0f, 0.0f, 60.0);
        int elapsed = TruncToInt32(Clamp((float)(m.actualTimeMs - startTime), 0, zoomTime));
        float bias = elapsed / (float)(zoomTime);
        bias *= PI;
        bias = libm::sinf(bias - 0.5f * PI) * -0.5f + 0.5f;
        m.cameraOrientation = m.cameraOrientation.Slerp(bias, Quat(0, 0, 0, 1));
        m.cameraNodeOrientation = m.cameraNodeOrientation.Slerp(bias, init);
        m.cameraNodePosition = m.cameraNodePosition * (1.0f - bias) + initPos * bias;
        m.cameraFov = m.cameraFov * (1.0f - bias) + 40 * bias;
        m.cameraNearCap = m.cameraNearCap * (1.0f - bias) + 2.0f * bias;
    }
}

}  // namespace eng
