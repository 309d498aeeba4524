// SPDX-License-Identifier: Apache-2.0
// Restates game logic of cuju (Copyright 2026 The cuju Authors), a reimplementation of Google
// Research Football (Copyright 2019 Google LLC); see NOTICE.
// The scenario builder: the agentless `l0_r0` bundle ("CUJASSET1") of a GRF scenario, built on the
// host from a description of what the scenario file sets (include/cuju/assets/scenario_builder.h,
// src/scenario_api.h). It runs this engine's own reset and kick-off ticks, so a bundle it writes
// is the bundle the batch loads.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace eng {
namespace host {

// One `AddPlayer` call, in environment coordinates; `role` is GRF's `e_PlayerRole` (0 to 9).
struct ScenarioPlayer {
    double x = 0, y = 0;
    int32_t role = 0;
    bool lazy = false, controllable = true;
};

// What a scenario file builds for one parity of the episode number, with GRF's `ScenarioConfig`
// defaults. An empty team is refused: the Python side adds GRF's lazy goalkeeper first.
struct ScenarioDescription {
    double ballX = 0, ballY = 0;
    std::vector<ScenarioPlayer> leftTeam, rightTeam;
    bool useMagnet = true, offsides = true, realTime = false;
    double leftTeamDifficulty = 1.0, rightTeamDifficulty = 0.6;
    bool deterministic = false, endOnScore = false, endOnPossessionChange = false, endOnOutOfPlay = false;
    int32_t gameDuration = 3000, secondHalf = 999999999;
    bool controlAllPlayers = false;
    uint32_t gameEngineRandomSeed = 42;
};

// The bundle bytes of the even (`parity[0]`) and odd episodes of a scenario named `name`, with
// the animation tables at `animations`. Throws std::invalid_argument for a description GRF
// refuses and std::runtime_error for one the simulation cannot start.
std::string BuildScenarioBundle(const std::string &name, const ScenarioDescription (&parity)[2], const std::string &animations);

}  // namespace host
}  // namespace eng
