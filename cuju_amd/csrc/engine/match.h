// SPDX-License-Identifier: Apache-2.0
// Restates game logic of cuju (Copyright 2026 The cuju Authors), a reimplementation of Google
// Research Football (Copyright 2019 Google LLC); see NOTICE.
// One tick of a match: each stage runs in the frame it expects, between two MirrorMatch calls.
// Semantics: include/cuju/simulation/match_process.h:17-374.
#pragma once

#include "setpiece.h"
#include "camera.h"

namespace eng {

// Slot 0 holds the newest of at most three mental images. The images hold what a frame change
// mirrors, so a team that the current frame holds mirrored from the rest frame (`mirrored`, by
// team ID) stores its direction negated too: a frame change negates a humanoid's position and
// movement but leaves its direction alone.
HDN void PushMentalImage(World &w, const bool (&mirrored)[2]) {
    ENG_SCOPE(8);
    MatchState &m = w.match;
    const int n = m.mentalImages.count < 3 ? m.mentalImages.count + 1 : 3;
    for (int i = n - 1; i > 0; i--) {
        m.mentalImages[i] = m.mentalImages[i - 1];
        w.flags.mentalBallMirrored[i] = w.flags.mentalBallMirrored[i - 1];
    }
    MentalImage &mi = m.mentalImages[0];
    memset(&mi, 0, sizeof(MentalImage));
    mi.timeStampMs = (uint32_t)m.actualTimeMs;
    mi.maxDistanceDeviation = 2.5f;
    mi.maxMovementDeviation = kWalkVelocity;
    for (int slot = 0; slot < 2; slot++) {
        PlayerList ps = TeamActivePlayers(w, slot == 0 ? w.FirstTeamID() : 1 - w.FirstTeamID());
        for (int i = 0; i < ps.count; i++) {
            const SpatialState &s = Sp(w, ps[i]);
            PlayerImage im{};
            im.player = ps[i];
            im.position = s.position;
            im.directionVector = s.directionVec;
            if (mirrored[w.playerTeamID[ps[i]]]) im.directionVector.Mirror();
            im.velocity = s.velocityCat;
            im.movement = s.movement;
            im.role = m.players[ps[i]].dynamicFormationEntry.role;
            mi.players.push_back(im);
        }
    }
    const int np = kBallPredictionSpanMs / 10;
    mi.ballPredictions.count = np;
    GroupCopy<4>(mi.ballPredictions.e, m.ball.predictions, np);
    mi.lazyFlip = m.ball.lazyFlip;
    w.flags.mentalBallMirrored[0] = false;
    m.mentalImages.count = n;
}

HDN void CalculateBestPossessionTeamID(World &w) {
    MatchState &m = w.match;
    if (m.ballRetainer != -1) {
        m.bestPossessionTeam = TeamSlot(w, w.playerTeamID[m.ballRetainer]);
        return;
    }
    const int first = w.FirstTeamID();
    int a = TeamByID(w, first).timeToBallMs, b = TeamByID(w, 1 - first).timeToBallMs;
    m.bestPossessionTeam = a < b ? TeamSlot(w, first) : a > b ? TeamSlot(w, 1 - first) : -1;
}

// ---- goals ---------------------------------------------------------------------------------------
// GRF counts a goal when the ball's path over the tick crosses the goal plane (the goal line moved
// out by the line's half width and the ball's radius) inside the mouth, which it splits into two
// triangles. The crossing point's parameters along the path and within a triangle compare in
// double.

// Where the segment from `from` to `to` crosses the plane through `on` with normal `normal`, as a
// fraction of the segment strictly between 0 and 1; false when it runs parallel or misses.
HD bool SegmentCrossesPlane(const Vec3 &on, const Vec3 &normal, const Vec3 &from, const Vec3 &to, Vec3 &at) {
    const Vec3 path = to - from;
    const float along = normal.Dot(path);
    if (fabsf(along) < 0.000001f) return false;
    const float r = -normal.Dot(from - on) / along;
    if ((double)r <= 0.0 || (double)r >= 1.0) return false;
    at = from + path * r;
    return true;
}
// Whether a point of a triangle's plane lies inside it: its barycentric coordinates along the
// edges from corner 0, each at least 0 and summing to at most 1.
HD bool InsideTriangle(const Vec3 (&corner)[3], const Vec3 &point) {
    const Vec3 e1 = corner[1] - corner[0], e2 = corner[2] - corner[0], rel = point - corner[0];
    const float uu = e1.Dot(e1), uv = e1.Dot(e2), vv = e2.Dot(e2);
    const float wu = rel.Dot(e1), wv = rel.Dot(e2);
    const float d = uv * uv - uu * vv;
    const float s = (uv * wv - vv * wu) / d;
    if ((double)s < 0.0 || (double)s > 1.0) return false;
    const float t = (uv * wu - uu * wv) / d;
    return !((double)t < 0.0 || (double)(s + t) > 1.0);
}
HD bool PathThroughTriangle(const Vec3 (&corner)[3], const Vec3 &normal, const Vec3 &from, const Vec3 &to) {
    Vec3 at;
    return SegmentCrossesPlane(corner[0], normal, from, to, at) && InsideTriangle(corner, at);
}
// Whether the ball went into the goal at `side` this tick, from `before`: it must end near the
// goal line, and a ball that started wide of the posts beyond the line does not count.
HDN bool BallEnteredGoal(const World &w, int side, const Vec3 &before) {
    const Ball &b = w.match.ball;
    if ((double)fabsf(BallPredict(b, 10).v[0]) < (double)kPitchHalfLength - 1.0) return false;
    const Vec3 after = BallPredict(b, 0);
    const float x = (kPitchHalfLength + kLineHalfWidth + 0.11f) * side;
    const Vec3 normal(-side, 0, 0);
    const Vec3 lower[3] = {Vec3(x, 3.7f, 0), Vec3(x, -3.7f, 0), Vec3(x, 3.7f, 2.5f)};
    const Vec3 upper[3] = {Vec3(x, -3.7f, 0), Vec3(x, -3.7f, 2.5f), Vec3(x, 3.7f, 2.5f)};
    const bool crossed = PathThroughTriangle(lower, normal, before, after) || PathThroughTriangle(upper, normal, before, after);
    if ((double)fabsf(before.v[1]) > 3.7 && (double)fabsf(before.v[0]) > (double)(kPitchHalfLength - kLineHalfWidth) - 0.11)
        return false;
    return crossed;
}
// A goal for team `scorer`: it changes its tactics, and the scorer is the last toucher of the
// scoring team, or of the other team for an own goal (one whose last touches of both kinds were
// not the scoring team's).
HD void RecordGoal(World &w, int first, int scorer) {
    MatchState &m = w.match;
    m.goalCount[scorer == first ? 0 : 1] += 1;
    m.goalScored = true;
    m.lastGoalTeam = TeamSlot(w, scorer);
    TeamUpdateTactics(w, scorer);
    const int team = m.lastGoalTeam == 0 ? first : 1 - first;
    const bool own = !(m.lastTouchTeamIDs[kTouchKicked] == team || m.lastTouchTeamIDs[kTouchNonKicked] == team);
    m.lastGoalScorer = TeamByID(w, own ? 1 - team : team).lastTouchPlayer;
}

// The designated possession player after the possession choice: the retainer; else, when one team
// is quicker to the ball, its designated player once it is at least 15% quicker (10 ms added to
// both times) than the current one; else the designated player of the current one's team.
HD void HandOverDesignation(World &w, int first) {
    MatchState &m = w.match;
    if (m.ballRetainer != -1) {
        m.designatedPossessionPlayer = m.ballRetainer;
        return;
    }
    if (m.bestPossessionTeam == -1) {
        m.designatedPossessionPlayer = TeamByID(w, w.playerTeamID[m.designatedPossessionPlayer]).designatedTeamPossessionPlayer;
        return;
    }
    const int candidate = TeamByID(w, m.bestPossessionTeam == 0 ? first : 1 - first).designatedTeamPossessionPlayer;
    if (candidate == m.designatedPossessionPlayer) return;
    const uint32_t current = w.roster.timeToBallMs[m.designatedPossessionPlayer], quicker = w.roster.timeToBallMs[candidate];
    if ((float)(quicker + 10) / (float)(current + 10) < 0.85f) m.designatedPossessionPlayer = candidate;
}

// The last six seconds of which side holds the ball (each team's fading possession less a half,
// signed by its side), one entry a tick while a team is best placed.
HD void RecordPossessionSide(World &w) {
    MatchState &m = w.match;
    float side = 0;
    side += (TeamByID(w, 0).fadingTeamPossessionAmount - 0.5f) * TeamDynamicSide(w, 0);
    side += (TeamByID(w, 1).fadingTeamPossessionAmount - 0.5f) * TeamDynamicSide(w, 1);
    auto &history = m.possessionSideHistory;
    if (history.count < 600) {
        history.push_back(side);
        return;
    }
    GroupShiftDown<8>(history.e, history.count - 1);
    history[history.count - 1] = side;
}

// False when the tick ends early: while play waits for a restart (the clock still advances), or
// on an unsupported path, which also clears `ok`.
HDN bool MatchProcess(World &w, const Ctx &c, bool &ok) {
    ENG_SCOPE(4);
    MatchState &m = w.match;
    ok = true;
    const bool rev = w.scenario.reverseTeamProcessing;
    const int first = w.FirstTeamID(), second = 1 - first;
    // Between the set piece's preparation and its start a tick only advances the clocks: the
    // referee touches nothing that a team frame changes, so the frame changes around it, which
    // cancel exactly, are left out.
    {
        const RefereeBuffer &rb = m.referee.buffer;
        if (!m.inPlay && !m.inSetPiece && rb.active && rb.prepareTime + 10 < m.actualTimeMs && rb.startTime != m.actualTimeMs) {
            if (!RefereeProcess(w, c)) return ok = false;
            BumpActualTime(w, c, 10);
            return false;
        }
    }
    MirrorMatch(w, rev, !rev, rev);
    if (m.inPlay && !CheckBallCollisions(w, c)) return ok = false;
    if (!RefereeProcess(w, c)) return ok = false;
    Vec3 prevBall = BallPredict(m.ball, 0);
    if (!m.inPlay && m.referee.buffer.prepareTime + 10 < m.actualTimeMs) {
        MirrorMatch(w, rev, !rev, rev);
        BumpActualTime(w, c, 10);
        return false;
    }
    // GRF returns to the rest frame here, moves the ball alone for its flight, pushes the mental
    // image and updates the switches. The collision frame already holds the ball where the flight
    // expects it; the image takes the collision frame's players, their directions mirrored like
    // their positions (PushMentalImage); and the switches read times, IDs and controllers only. So
    // the three run in the collision frame, and one frame change leads to the first team's.
    BallProcess(m.ball, m.ballIsInGoal);
    if (m.mentalImages.count == 0 || m.actualTimeMs % 100 == 0) {
        const bool mirrored[2] = {rev, !rev};
        PushMentalImage(w, mirrored);
    }
    if (!TeamUpdateSwitch(w, c, first)) return ok = false;
    if (!TeamUpdateSwitch(w, c, second)) return ok = false;
    MirrorMatch(w, rev != (first == 1), !rev != (first == 0), rev != (first == 1));
    if (!TeamProcess(w, c, first)) return ok = false;
    MirrorMatch(w, true, true, true);
    if (!TeamProcess(w, c, second)) return ok = false;
    // Two frame changes in a row make one: each mirror is its own inverse on disjoint state, so a
    // flag of the pair is the exclusive or of the two.
    MirrorMatch(w, (first == 0) != rev, (first == 1) != !rev, (first == 0) != rev);
    if (!OfficialsProcess(w, c)) return ok = false;
    // A team's possession statistics read its own players and the ball, and other teams' times
    // only. Each runs with its team and the ball where GRF has them (the team in its own frame, the
    // ball in that team's), leaving the other team where it is, which takes two team mirrors
    // fewer than moving the whole match.
    {
        bool m0 = rev, m1 = !rev, mb = rev;  // the collision frame, relative to the rest frame
        auto frame = [&](bool t0, bool t1, bool ball) {
            MirrorMatch(w, m0 != t0, m1 != t1, mb != ball);
            m0 = t0;
            m1 = t1;
            mb = ball;
        };
        frame(first == 0 ? false : m0, first == 1 ? false : m1, first == 1);
        TeamUpdatePossessionStatistics(w, c, first);
        frame(second == 0 ? false : m0, second == 1 ? false : m1, second == 1);
        TeamUpdatePossessionStatistics(w, c, second);
        // The possession choice reads times and IDs only, so the return to the collision frame
        // waits for it.
        CalculateBestPossessionTeamID(w);
        HandOverDesignation(w, first);
        frame(rev, !rev, rev);
    }
    if (!CheckHumanoidCollisions(w, c)) return ok = false;
    BumpActualTime(w, c, 10);
    // A goal counts into the goal of the team whose side it is: the other team scores.
    const bool intoFirst = m.inPlay && BallEnteredGoal(w, TeamDynamicSide(w, first), prevBall);
    const bool intoSecond = m.inPlay && BallEnteredGoal(w, TeamDynamicSide(w, second), prevBall);
    m.ballIsInGoal |= intoFirst || intoSecond;
    MirrorMatch(w, rev, !rev, rev);
    if (m.inPlay && (intoFirst || intoSecond)) RecordGoal(w, first, intoFirst ? second : first);
    if (m.inPlay && m.bestPossessionTeam != -1) RecordPossessionSide(w);
    CameraOnCard(w, rev);
    return true;
}

HDN void PlayerPreparePutBuffers(World &w, int p) {
    PoseOffsets(w, p);
    Player &ps = w.match.players[p];
    const Team &t = TeamByID(w, w.playerTeamID[p]);
    const bool ext = ExternalControllerActive(w, p);
    ps.bufferNameCaptionShowCondition = ext;
    int gamers = 0;
    for (int g = 0; g < t.gamers.count; g++)
        if (!t.gamers[g].controller.keyboard.disabled) gamers++;
    if (gamers == 0) ps.bufferNameCaptionShowCondition = t.designatedTeamPossessionPlayer == p;
    int color = 5;
    const HumanGamer *gm = nullptr;
    if (ps.base.externalController >= 0) {
        gm = &GamerByGlobal(w, ps.base.externalController);
        color = gm->keyboardIndex % 6;
    }
    const float colors[6][3] = {{100, 140, 255}, {100, 255, 140}, {255, 110, 110}, {255, 255, 60}, {200, 80, 200}, {200, 200, 200}};
    ps.bufferPlayerColor = Vec3(colors[color][0], colors[color][1], colors[color][2]);
    if (ext && gm->controller.actionMode == 2)
        ps.bufferPlayerColor = ps.bufferPlayerColor * (libm::sinf(w.match.actualTimeMs * 0.02f) * 0.3f + 0.7f);
}
HDN void MatchPreparePutBuffers(World &w) {
    ENG_SCOPE(20);
    const int first = w.FirstTeamID(), second = 1 - first;
    // A player's buffers and pose offsets are its own, and the rest of the match is only read, so
    // the lanes of the match take a team's players in turn.
    MirrorMatch(w, false, false, first == 1);
    PlayerList a = TeamActivePlayers(w, first);
    for (int i = GroupRank(); i < a.count; i += kGroupLanes) PlayerPreparePutBuffers(w, a[i]);
    GroupSync();
    MirrorMatch(w, false, false, true);
    PlayerList b = TeamActivePlayers(w, second);
    for (int i = GroupRank(); i < b.count; i += kGroupLanes) PlayerPreparePutBuffers(w, b[i]);
    GroupSync();
    MirrorMatch(w, false, false, first == 0);
}
HDN void MatchFetchPutBuffers(World &w, const Ctx &c) {
    ENG_SCOPE(21);
    const int first = w.FirstTeamID();
    const Skeleton *skels[kPlayers + 3];
    Humanoid *hums[kPlayers + 3];
    int n = 0;
    for (int t = 0; t < 2; t++) {
        PlayerList ps = TeamActivePlayers(w, t == 0 ? first : 1 - first);
        for (int i = 0; i < ps.count; i++) {
            skels[n] = &c.skeletons[ps[i]];
            hums[n++] = &w.match.players[ps[i]].base.humanoid;
        }
    }
    for (int o = 0; o < 3; o++) {
        skels[n] = &c.skeletons[w.match.playerCount + o];
        hums[n++] = &w.match.officials[o].humanoid;
    }
    FetchPutBuffers(c, skels, hums, n);
}
// One 10 ms tick of the game.
HDN bool GameTick(World &w, const Ctx &c) {
#if !ENG_DEVICE
    HostTicks()++;
#endif
    bool ok;
    bool process = MatchProcess(w, c, ok);
    if (!ok) return false;
    UpdateCamera(w, c);
    if (process) {
        MatchPreparePutBuffers(w);
        MatchFetchPutBuffers(w, c);
    }
#if !ENG_DEVICE
    // The host build checks the roster against the fields it copies after every tick.
    if (!RosterMatches(w)) {
        Unsupported("the roster differs from the players");
        return false;
    }
#endif
    return true;
}

}  // namespace eng
