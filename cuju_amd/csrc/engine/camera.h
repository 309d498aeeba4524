// SPDX-License-Identifier: Apache-2.0
// Restates game logic of cuju (Copyright 2026 The cuju Authors), a reimplementation of Google
// Research Football (Copyright 2019 Google LLC); see NOTICE.
// GRF's in-game camera. It never affects play, but its pose is part of the state and its shake
// draws two numbers a tick from the world RNG. Semantics: include/cuju/simulation/camera.h:15-170.
// The float operations and the two draws are GRF's; the organisation (an aim point, a shake, a
// weighted history, and the poses that follow play, circle a scorer or zoom in at the start) is
// this engine's own.
#pragma once

#include "world.h"

namespace eng {

// The weight of entry `index` of a history of `count` positions (the host tabulates it).
HD float CameraWeight(int index, int count) {
    const float size = count;
    float w = libm::sinf((index / size - 0.3f) * 1.4f * PI) * 0.5f + 0.5f;
    w *= libm::powf(1.0f - index / size, 0.3f);
    return w;
}

// GRF's camera settings: field of view, zoom, height and angle, each from 0 to 1.
struct CameraSettings {
    static constexpr float kFov = 0.4f, kZoom = 0.5f, kHeight = 0.3f, kAngle = 0.0f;
};

// GRF updates the camera with team 1 mirrored. Of what the update reads, the mirror changes only
// the positions of team 1's players (x and y negated) and team 1's side (negated), so the camera
// reads those through these two instead of mirroring the team there and back.
HD Vec3 CameraPlayerPosition(const World &w, int p) {
    Vec3 v = Sp(w, p).position;
    if (w.playerTeamID[p] == 1) v.Mirror();
    return v;
}
HD int CameraTeamSide(const World &w, int t) { return t == 1 ? -TeamDynamicSide(w, t) : TeamDynamicSide(w, t); }

// Where the camera aims: between the ball and the designated player (60% the player), a metre
// ahead of the player, pushed toward the goal of the team that is losing possession, flattened,
// and kept within a box that the zoom and height set.
HD Vec3 CameraAim(const World &w) {
    const MatchState &m = w.match;
    const float towardPlayer = 0.6f;
    const int dp = m.designatedPossessionPlayer;
    Vec3 aim = BallPredict(m.ball, 0) * (1.0f - towardPlayer) + CameraPlayerPosition(w, dp) * towardPlayer;
    aim += Sp(w, dp).directionVec * 1.0f;
    const int first = w.FirstTeamID(), second = 1 - first;
    const float push = (TeamByID(w, first).fadingTeamPossessionAmount - 1.0f) * -CameraTeamSide(w, first) +
                       (TeamByID(w, second).fadingTeamPossessionAmount - 1.0f) * -CameraTeamSide(w, second);
    aim += Vec3(push * 4.0f, 0, 0);
    aim.v[2] *= 0.1f;
    const float zoom = CameraSettings::kZoom, height = CameraSettings::kHeight * 1.5f;
    const float halfW = (float)((double)(kPitchHalfLength * 0.84f) * (1.0 / (double)(zoom + 0.01f)));
    const float halfH = (float)((double)(kPitchHalfWidth * 0.60f) * (1.0 / (double)(zoom + 0.01f)) * (double)(height * 0.75f + 0.25f));
    if (fabsf(aim.v[0]) > halfW) aim.v[0] = halfW * SignSide(aim.v[0]);
    if (fabsf(aim.v[1]) > halfH) aim.v[1] = halfH * SignSide(aim.v[1]);
    return aim;
}

// The shake, stronger the faster the ball: GRF evaluates the two draws right to left, y first.
HD Vec3 CameraShake(World &w) {
    const float y = RandomInRange(w, -0.1f, 0.1f);
    const float x = RandomInRange(w, -0.1f, 0.1f);
    Vec3 shake = Vec3(x, y, 0) * (w.match.ball.momentum.Length() * 0.8f + 6.0f);
    shake *= 0.2f;
    return shake;
}

// The camera's position history gets the aim point with the shake scaled by the history's length;
// a full history drops its oldest entry.
HD void RecordCameraAim(MatchState &m, const Vec3 &aim, const Vec3 &shake) {
    auto &history = m.cameraPosition;
    const Vec3 entry = aim + shake * ((float)history.count / (float)kCameraHistory);
    if (history.count < kCameraHistory) {
        history.push_back(entry);
        return;
    }
    GroupShiftDown<4>(history.e, history.count - 1);
    history[history.count - 1] = entry;
}

// The history's weighted mean, with the weights of its length. The sums run in entry order; the
// entries load eight at a time, so their loads overlap in flight.
HD Vec3 CameraHistoryMean(const MatchState &m, const Ctx &c) {
    const auto &history = m.cameraPosition;
    const int count = history.count;
    const float *weights = c.t->cameraWeights + count * (count - 1) / 2;
    Vec3 sum;
    float total = 0;
    constexpr int kChunk = 8;
    for (int i0 = 0; i0 < count; i0 += kChunk) {
        float wt[kChunk];
        Vec3 at[kChunk];
        for (int j = 0; j < kChunk; j++)
            if (i0 + j < count) {
                wt[j] = weights[i0 + j];
                at[j] = history[i0 + j];
            }
        for (int j = 0; j < kChunk; j++)
            if (i0 + j < count) {
                sum += at[j] * wt[j];
                total += wt[j];
            }
    }
    sum /= Vec3(total);
    return sum;
}

// In play (and for the first second after a goal) the camera looks down on the mean aim point
// from the side, tilted and lifted by its settings.
HD void CameraFollowPlay(MatchState &m, const Vec3 &mean) {
    using S = CameraSettings;
    const float fov = 0.5f + S::kFov * 0.5f;
    const float zoom = (0.6f + S::kZoom * 1.0f) * (1.0f / fov);
    const float height = 4.0f + (S::kHeight * 1.5f) * 10;
    const float angleFactor = 1.0f - S::kAngle * 0.4f;
    m.cameraOrientation.SetAngleAxis(mean.v[1] / 800.0f + (0.42f - height * 0.01f) * PI, Vec3(1, 0, 0));
    m.cameraNodeOrientation.SetAngleAxis((-mean.v[0] / kPitchHalfLength) * (1.0f - angleFactor) * 0.25f * PI * 1.24f,
                                         Vec3(0, 0, 1));
    m.cameraNodePosition =
        mean * Vec3(1.0f * (1.0f - S::kAngle * 0.2f) * (1.0f - S::kZoom * 0.3f), 0.9f - S::kZoom * 0.3f, 0.2f) +
        Vec3(0, -41.4f - (S::kFov * 3.7f) + libm::powf(height, 1.2f) * 0.46f, 10.0f + height) * zoom;
    m.cameraFov = (fov * 28.0f) - (m.cameraNodePosition.v[1] / 30.0f);
    m.cameraNearCap = m.cameraNodePosition.v[2];
    m.cameraFarCap = 200;
}

// After a goal the camera circles the scorer (or the ball) 15 m out and 3 m up.
HD void CameraCircleScorer(const World &w, MatchState &m) {
    Vec3 target = BallPredict(m.ball, 0).Get2D();
    if (m.lastGoalScorer >= 0) target = CameraPlayerPosition(w, m.lastGoalScorer);
    const float turn = (float)m.goalScoredTimer * 0.0005f;
    m.cameraOrientation.SetAngleAxis(0.45f * PI, Vec3(1, 0, 0));
    m.cameraNodeOrientation.SetAngleAxis(turn, Vec3(0, 0, 1));
    m.cameraNodePosition = target + Vec3(0, -1, 0).Rotated2D(turn) * 15.0f + Vec3(0, 0, 3);
    m.cameraFov = 35.0f;
    m.cameraNearCap = 1;
    m.cameraFarCap = 220;
}

// For the first two seconds the camera eases in from straight above the centre spot, 60 m up.
HD void CameraIntro(MatchState &m) {
    const unsigned zoomTime = 2000, startTime = 0;
    if (m.actualTimeMs >= zoomTime + startTime) return;
    Quat above(0, 0, 0, 1);
    above.SetAngleAxis(0.0f * PI, Vec3(1, 0, 0));
    above = Quat(0, 0, 0, 1) * above;
    const Vec3 overhead(0.0f, 0.0f, 60.0);
    const int elapsed = TruncToInt32(Clamp((float)(m.actualTimeMs - startTime), 0, zoomTime));
    float ease = elapsed / (float)(zoomTime);
    ease *= PI;
    ease = libm::sinf(ease - 0.5f * PI) * -0.5f + 0.5f;
    m.cameraOrientation = m.cameraOrientation.Slerp(ease, Quat(0, 0, 0, 1));
    m.cameraNodeOrientation = m.cameraNodeOrientation.Slerp(ease, above);
    m.cameraNodePosition = m.cameraNodePosition * (1.0f - ease) + overhead * ease;
    m.cameraFov = m.cameraFov * (1.0f - ease) + 40 * ease;
    m.cameraNearCap = m.cameraNearCap * (1.0f - ease) + 2.0f * ease;
}

// While the referee shows a card (from a second after play stopped until the restart is prepared)
// the camera leaves play and frames the referee from 10 m away (zoom 1.5) and 3 m up; after that
// it follows play again. A change of mode clears the aim history. GRF also holds the restart back
// while the referee's card animation runs: prepared a second later, started two seconds after
// that. `mirrored`: the match is in a frame that mirrors the referee's position.
HD void CameraOnCard(World &w, bool mirrored) {
    MatchState &m = w.match;
    Referee &ref = m.referee;
    const bool card = ref.foul.foulType == 2 || ref.foul.foulType == 3;
    if (!(ref.buffer.active && card && ref.buffer.stopTime < m.actualTimeMs - 1000)) return;
    const bool follow = !(ref.buffer.prepareTime > m.actualTimeMs);
    if (follow != m.autoUpdateInGameCamera) {
        m.cameraPosition.count = 0;
        m.autoUpdateInGameCamera = follow;
    }
    if (follow) return;
    Humanoid &referee = m.officials[0].humanoid;
    Vec3 at = referee.spatial.position;
    if (mirrored) at.Mirror();
    const Vec3 target = at + Vec3(0, 0, 0.8f);
    const float zoom = 1.5f;
    m.cameraOrientation.SetAngleAxis(0.4f * PI, Vec3(1, 0, 0));
    m.cameraNodeOrientation.SetAngleAxis((float)((double)target.Angle2D() + 1.5 * (double)PI), Vec3(0, 0, 1));
    m.cameraNodePosition = target - target.Get2D().Normalized(Vec3(0, -1, 0)) * 10 * (1.0f / zoom) + Vec3(0, 0, 3);
    m.cameraFov = 60.0f;
    m.cameraNearCap = 1;
    m.cameraFarCap = 220;
    if (referee.anim.functionType == kFnSpecial && ref.buffer.active) {
        ref.buffer.prepareTime = m.actualTimeMs + 1000;
        ref.buffer.startTime = ref.buffer.prepareTime + 2000;
    }
}

// The camera's tick, on the unmirrored pitch (team 1 read mirrored in place).
HDN void UpdateCamera(World &w, const Ctx &c) {
    ENG_SCOPE(19);
    MatchState &m = w.match;
    if (m.autoUpdateInGameCamera) {
        const Vec3 aim = CameraAim(w);
        RecordCameraAim(m, aim, CameraShake(w));
        const Vec3 mean = CameraHistoryMean(m, c);
        if (!m.goalScored || (m.goalScored && m.goalScoredTimer < 1000)) CameraFollowPlay(m, mean);
        else CameraCircleScorer(w, m);
    }
    CameraIntro(m);
}

}  // namespace eng
