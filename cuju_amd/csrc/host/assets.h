// SPDX-License-Identifier: Apache-2.0
// Restates game logic of cuju (Copyright 2026 The cuju Authors), a reimplementation of Google
// Research Football (Copyright 2019 Google LLC); see NOTICE.
// Host-side construction of everything a match reads besides its world: the animation tables and
// their derived records, the skeletons and static data of each scenario variant, the reset
// templates of a bundle with any agent counts, and the codec between GRF's state bytes and a
// World. These run once at creation (and at get_state) and never in the step.
#pragma once

#include <memory>
#include <string>
#include <vector>

#include "../engine/codec.h"
#include "../engine/episode.h"

namespace eng {
namespace host {

std::string ReadFile(const std::string &path);

// The animation tables of `animations.bin` ("CUJANIM1"), flattened into index ranges, with the
// per-frame interpolation tables and every record the selection reads, as one host copy.
struct AnimationTables {
    std::vector<Anim> anims;
    std::vector<NodeAnim> nodes;
    std::vector<KeyFrame> keys;
    std::vector<InterpEntry> interp;
    std::vector<MiddleEntry> middle;
    std::vector<FootballKey> football;
    std::vector<Vec3> positions;
    std::vector<Quadrant> quadrants;
    Radian maxIncomingBallDeviation{}, maxOutgoingBallDeviation{};
    std::vector<AnimDerived> derived;
    std::vector<SelectionRecord> selection;
    std::vector<Vec3> smoothed;  // parallels `positions`
    std::vector<int16_t> fnAnims;
    std::vector<int32_t> fnOffset;
    std::vector<CrudeRecord> crude, crudeByIndex, crudeVelocity, crudeBody;
    std::vector<int32_t> crudeVelocityOffset, crudeBodyOffset;
    std::vector<float> cameraWeights;
    std::vector<int16_t> idleMovement;  // the crude selection of the idle query
    // Tables whose pointers index the vectors above.
    Tables View() const;
};
std::unique_ptr<AnimationTables> LoadAnimationTables(const std::string &path);

// The sections of a bundle variant: the skeletons ("CUJHUM1") and the static data (the
// PlayerData of every entry, then FORM, MDUR and SIDS).
std::vector<Skeleton> ParseSkeletons(const std::string &bytes);
StaticData ParseStatic(const std::string &bytes);

// One team order and episode parity of a bundle.
struct Variant {
    int reverse = 0, parity = 0;
    int freeControllerCount = 0;  // the keyboards no gamer owns, which saving needs
    StaticData staticData{};
    std::unique_ptr<World> world;  // after a reset, in the rest frame
    std::string scenario;          // scenario bytes without seed and difficulties
    std::vector<Skeleton> skeletons;
};
// A `.cjb` bundle ("CUJASSET1"): a scenario, its agent counts and four variants indexed by
// reverse * 2 + parity.
struct Bundle {
    std::string scenario;
    int leftAgents = 0, rightAgents = 0;
    Variant variants[4];
};
// `left`/`right` of -1 keep the bundle's agents.
std::unique_ptr<Bundle> LoadBundle(const std::string &path, int left = -1, int right = -1);

// The state codec. The count of free controllers is not in the bytes, so the first load finds
// it and later loads try it first.
struct StateCodec {
    int freeControllerCount = -1;
    int animationCount = -1;
    bool Load(const std::string &bytes, World &w);
    std::string Save(World &w, std::vector<codec::SchemaEntry> *schema = nullptr);
    // `mirror` names the call frame: bit 0 mirrors team 0, bit 1 team 1, bit 2 the ball.
    bool LoadFrame(const std::string &bytes, int mirror, World &w);
    std::string SaveFrame(World &w, int mirror, std::vector<codec::SchemaEntry> *schema = nullptr);
};
void ResetWorld(World &w);
// The scenario bytes of a world without the per-episode seed and the batch-set difficulties.
std::string ScenarioKey(const World &w);
// Gives a rest-frame template `left` and `right` agents as GRF's reset does.
void SetupAgents(World &w, const StaticData &sd, int left, int right, const std::string &bundle);

}  // namespace host
}  // namespace eng
