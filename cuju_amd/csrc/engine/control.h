// SPDX-License-Identifier: Apache-2.0
// Restates game logic of cuju (Copyright 2026 The cuju Authors), a reimplementation of Google
// Research Football (Copyright 2019 Google LLC); see NOTICE.
// Keyboard input of the gamers (agents), and which player each gamer controls.
// Semantics: include/cuju/simulation/human_controller.h:11-117,
// include/cuju/simulation/team_select.h:13-207, include/cuju/batch/agent_setup.h:15-70.
#pragma once

#include "world.h"

namespace eng {

enum Button {
    kBtnLongPass,
    kBtnHighPass,
    kBtnShortPass,
    kBtnShot,
    kBtnKeeperRush,
    kBtnSliding,
    kBtnPressure,
    kBtnTeamPressure,
    kBtnSwitch,
    kBtnSprint,
    kBtnDribble,
    kBtnCount
};
constexpr float kStickDeadzone = 0.75f;
constexpr int kTeamControllers = 11;

HD HumanGamer &HumanGamerOf(World &w, int p) { return GamerByGlobal(w, w.match.players[p].base.externalController); }
// The keyboard stores its direction times its mirror sign and reports it the same way.
HD Vec3 KeyboardDirection(const KeyboardState &k) { return k.direction; }

HD float GetLastSwitchBias(World &w, PlayerControllerState &c) {
    if (!w.match.inPlay || w.match.inSetPiece) c.lastSwitchTimeMs = (uint64_t)(int64_t)-10000;
    if (c.lastSwitchTimeDurationMs > 0)
        return 1.0f - Clamp((w.match.actualTimeMs - c.lastSwitchTimeMs) / (float)c.lastSwitchTimeDurationMs, 0.0f, 1.0f);
    return 0.0f;
}

// A stick held outward at a touchline or goal line is cut to zero in that axis (GRF clamps with
// std::min(0, x) or std::max(0, x); the expression never gives -0).
HD Vec3 StickInsidePitch(Vec3 stick, const Vec3 &pos) {
    float &x = stick.v[0], &y = stick.v[1];
    if (pos.v[0] > kPitchHalfLength) x = ((x < 0.0f) ? x : 0.0f) + 0.0f;
    if (pos.v[0] < -kPitchHalfLength) x = (0.0f < x) ? x : 0.0f;
    if (pos.v[1] > kPitchHalfWidth) y = ((y < 0.0f) ? y : 0.0f) + 0.0f;
    if (pos.v[1] < -kPitchHalfWidth) y = (0.0f < y) ? y : 0.0f;
    return stick;
}
// The velocity the held buttons ask for: sprint, then dribble, then standing to switch with the
// ball, else walking.
HD float ButtonVelocity(const World &w, const bool *buttons, int p) {
    if (buttons[kBtnSprint]) return kSprintVelocity;
    if (buttons[kBtnDribble]) return kDribbleVelocity;
    if (buttons[kBtnSwitch] && w.match.designatedPossessionPlayer == p) return kIdleVelocity;
    return kWalkVelocity;
}
// The player's own movement, fading out over the moments after a switch to it, blends into what the
// gamer asks for.
HD void BlendAfterSwitch(World &w, int p, PlayerControllerState &base, Vec3 &dir, float &vel) {
    if (!(GetLastSwitchBias(w, base) > 0.0f)) return;
    const float influence = 0.5f;
    const float fading = libm::powf(GetLastSwitchBias(w, base), 0.7f);
    const Vec3 own = Sp(w, p).directionVec * PlayerFloatVelocity(w, p);
    const Vec3 asked = dir * vel;
    const Vec3 blend = own * fading * influence + asked * (1.0f - fading * influence);
    dir = blend.Normalized(dir);
    vel = blend.Length();
}
// What a gamer's keyboard asks of player `p`: a direction and a velocity. A stick inside the dead
// zone keeps the player's direction, idle.
HDN void HumanGetKeyboardInput(World &w, int p, Vec3 &dir, float &vel) {
    HumanControllerState &hc = HumanGamerOf(w, p).controller;
    const SpatialState &s = Sp(w, p);
    dir = StickInsidePitch(KeyboardDirection(hc.keyboard), s.position);
    if (dir.Length() < kStickDeadzone) {
        dir = s.directionVec;
        vel = kIdleVelocity;
    } else {
        vel = ButtonVelocity(w, hc.keyboard.buttons, p);
        dir.Normalize();
    }
    BlendAfterSwitch(w, p, hc.base, dir, vel);
}
HD float HumanGetFloatVelocity(World &w, int p) {
    Vec3 d;
    float v = 0;
    HumanGetKeyboardInput(w, p, d, v);
    return v;
}
HD Vec3 HumanGetDirection(World &w, int p) { return KeyboardDirection(HumanGamerOf(w, p).controller.keyboard).Normalized(Sp(w, p).directionVec); }

// GRF: sprint, dribble and the defensive buttons are sticky; the others release.
HD void ReleaseNonStickyButtons(KeyboardState &k) {
    const int bs[6] = {kBtnLongPass, kBtnHighPass, kBtnShortPass, kBtnShot, kBtnSliding, kBtnSwitch};
    for (int b : bs) k.buttons[b] = false;
}
HD void KeyboardReleaseNonStickyButtons(World &w, int g) {
    ReleaseNonStickyButtons(GamerByGlobal(w, g).controller.keyboard);
    ReleaseNonStickyButtons(w.match.secondKeyboardCopies[g]);
}

HDN void HumanControllerReset(World &w, int g) {
    HumanControllerState &c = GamerByGlobal(w, g).controller;
    c.actionMode = 0;
    c.gaugeMs = 0;
    c.actionButton = kBtnShortPass;
    c.actionBufferTimeMs = 0;
    c.base.lastSwitchTimeMs = (uint64_t)(int64_t)-10000;
    c.base.lastSwitchTimeDurationMs = 300;
    c.lastSteadyDirectionSnapshotTimeMs = 0;
    c.steadyDirection = Vec3(0, -1, 0);
    c.previousDirection = Vec3(0, -1, 0);
    c.base.fadingTeamPossessionAmount = 1.0;
    KeyboardReleaseNonStickyButtons(w, g);
}
HD void HumanControllerSetPlayer(World &w, int g, int p) {
    HumanControllerState &c = GamerByGlobal(w, g).controller;
    c.base.lastSwitchTimeMs = w.match.actualTimeMs;
    c.base.player = p;
    // The state stores a team as its slot.
    c.base.team = TeamSlot(w, w.playerTeamID[p]);
    c.base.opponentTeam = TeamSlot(w, 1 - w.playerTeamID[p]);
}
// `g` is a global gamer index, or -1 to hand the player back to the AI.
HD void SetExternalController(World &w, int p, int g) {
    Player &ps = w.match.players[p];
    ps.base.externalController = g;
    if (g >= 0) {
        HumanControllerReset(w, g);
        HumanControllerSetPlayer(w, g, p);
    } else {
        ps.controller.lastDesiredDirection = Vec3(0);
        ps.controller.lastDesiredVelocity = 0;
    }
}
HDN void HumanGamerSetSelectedPlayer(World &w, int g, int p) {
    HumanGamer &gm = GamerByGlobal(w, g);
    if (p >= 0 && w.match.players[p].base.externalController >= 0) return;
    if (gm.selectedPlayer >= 0) {
        if (gm.selectedPlayer == p) return;
        SetExternalController(w, gm.selectedPlayer, -1);
    }
    if (p >= 0) {
        gm.selectedPlayer = p;
        SetExternalController(w, p, g);
    } else {
        gm.selectedPlayer = -1;
    }
}
// The gamer first in the team's switch order goes to the back of it.
HD void RotateSwitchOrder(Team &t) {
    auto &order = t.switchPriority;
    const int front = order[0];
    for (int i = 0; i + 1 < order.count; i++) order[i] = order[i + 1];
    order[order.count - 1] = front;
}
// A selectable player becomes the team's main selection and, when no gamer holds it, the player of
// the gamer first in the switch order (who then goes to the back); it is the designated player.
HDN bool TeamSelectPlayer(World &w, const Ctx &c, int teamID, int p) {
    Team &t = TeamByID(w, teamID);
    if (Formation(w, c, p).controllable) {
        t.mainSelectedPlayer = p;
        if (w.match.players[p].base.externalController < 0 && t.gamers.count > 0) {
            HumanGamerSetSelectedPlayer(w, GlobalGamerIndex(w, teamID, t.switchPriority[0]), p);
            RotateSwitchOrder(t);
        }
    }
    t.designatedTeamPossessionPlayer = p;
    return true;
}
// A tie keeps the player first in the state.
HDN int GetClosestPlayer(const World &w, const Ctx &c, int teamID, const Vec3 &pos, bool onlyAI, int except = -1,
                         bool onlySelectable = false) {
    float best = 10000;
    int bp = -1;
    const int players = w.match.playerCount;
    // Every player's tests and position load together, without an early exit; the controller and
    // formation tests run only for candidates.
#pragma unroll
    for (int p = 0; p < kPlayers; p++) {
        const bool in = (p < players) & (w.playerTeamID[p] == teamID) & w.roster.active[p] & (p != except);
        const float d = (Sp(w, p).position - pos).Length();
        if (in && d < best) {
            if ((!onlyAI || !ExternalControllerActive(w, p)) && (!onlySelectable || Formation(w, c, p).controllable)) {
                best = d;
                bp = p;
            }
        }
    }
    return bp;
}
// A time in ms: the shortest of the players that enabled gamers control, or 10000.
HD int HumanControlledToBallTime(const World &w, int teamID) {
    const Team &t = TeamByID(w, teamID);
    int best = 10000;
    for (int g = 0; g < t.gamers.count; g++) {
        const HumanGamer &gm = t.gamers[g];
        if (gm.selectedPlayer >= 0 && !gm.controller.keyboard.disabled) {
            int tt = (int)w.roster.timeToBallMs[gm.selectedPlayer];
            best = (tt < best) ? tt : best;
        }
    }
    return best;
}
// GRF's automatic switching while in play: the gamer on the match's designated player yields the
// front of the switch order; the team's designated outfield player goes to a gamer when it is
// three times quicker to the ball than every controlled player, or when it alone has the ball (or
// a set piece is on). Each test reads the designated player anew.
HDN bool TeamUpdateSwitch(World &w, const Ctx &c, int teamID) {
    ENG_SCOPE(9);
    MatchState &m = w.match;
    Team &t = TeamByID(w, teamID);
    if (!m.inPlay || t.gamers.count == 0) return true;
    if (t.gamers.count > 1 && t.gamers[t.switchPriority[0]].selectedPlayer == m.designatedPossessionPlayer) RotateSwitchOrder(t);
    auto freeOutfield = [&](int d) { return !ExternalControllerActive(w, d) && Formation(w, c, d).role != kRoleGoalkeeper; };
    int d = t.designatedTeamPossessionPlayer;
    if (!ExternalControllerActive(w, d) && 3 * (int)w.roster.timeToBallMs[d] < HumanControlledToBallTime(w, teamID) &&
        Formation(w, c, d).role != kRoleGoalkeeper && !TeamSelectPlayer(w, c, teamID, d))
        return false;
    d = t.designatedTeamPossessionPlayer;
    if (freeOutfield(d) && (m.players[d].hasUniquePossession || m.inSetPiece) && !TeamSelectPlayer(w, c, teamID, d)) return false;
    return true;
}
HDN void TeamHumanGamersSelectAnyone(World &w, const Ctx &c, int teamID) {
    MatchState &m = w.match;
    if (!m.inPlay) return;
    Team &t = TeamByID(w, teamID);
    if (t.mainSelectedPlayer == -1)
        t.mainSelectedPlayer = GetClosestPlayer(w, c, teamID, BallPredict(m.ball, 0).Get2D(), true, -1, true);
    for (int g = 0; g < t.gamers.count; g++) {
        if (t.gamers[g].selectedPlayer == -1) {
            int p = GetClosestPlayer(w, c, teamID, BallPredict(m.ball, 0).Get2D(), true, -1, true);
            if (p >= 0) HumanGamerSetSelectedPlayer(w, GlobalGamerIndex(w, teamID, g), p);
        }
    }
}

}  // namespace eng
