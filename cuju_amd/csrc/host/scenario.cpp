// SPDX-License-Identifier: Apache-2.0
// Restates game logic of cuju (Copyright 2026 The cuju Authors), a reimplementation of Google
// Research Football (Copyright 2019 Google LLC); see NOTICE.
// The scenario builder (include/cuju/assets/scenario_builder.h:570-784). A variant's template is
// the state GRF's `GameEnv::reset` leaves before the ticks that bring the match into play: every
// field below is what GRF's constructors set, then this engine's reset from the template draws
// the idle frames, the officials' skin and the lighting. The skeletons of a variant hold the pose
// after the kick-off ticks. The bundle layout is the one LoadBundle reads.
#include "scenario.h"

#include <cmath>
#include <cstring>
#include <memory>
#include <stdexcept>

#include "assets.h"

namespace eng {
namespace host {
namespace {

struct GrfNode {
    const char *name;
    int32_t parent, localMode;
    float position[3];
    const char *geometry;
    int32_t geometryLocalMode;
    float geometryValues[16];
};
#include "grf_persons.inc"

// GRF: a `TeamData` holds 11 formation slots and 11 persons; a larger team crashes GRF.
constexpr int kScenarioTeamPlayers = 11;
constexpr int kPlayerRoles = 10;
// GRF: `PlayerData::PlayerData()` of the officials.
constexpr float kOfficialStatistic = (float)0.6, kOfficialHeight = 1.8f;

// GRF: the formation slots of `TeamData` (x, y as `atof` reads them) and their roles: GK, LB,
// CB, CB, RB, CM, CM, CM, LM, CF, RM.
constexpr double kSlotShape[kScenarioTeamPlayers][2] = {{-1.0, 0.0},  {-0.7, 0.75}, {-1.0, 0.25}, {-1.0, -0.25},
                                                        {-0.7, -0.75}, {0.0, 0.5},  {-0.2, 0.0},  {0.0, -0.5},
                                                        {0.6, 0.75},   {1.0, 0.0},  {0.6, -0.75}};
constexpr int32_t kSlotRole[kScenarioTeamPlayers] = {0, 2, 1, 1, 3, 5, 5, 5, 6, 9, 7};

// GRF: `GetDefaultRolePosition`, by `e_PlayerRole`.
Vec3 RoleAnchor(int32_t role) {
    static const float anchor[kPlayerRoles][2] = {{-1.0f, 0.0f}, {-1.0f, 0.0f}, {-0.8f, 0.8f}, {-0.8f, -0.8f}, {-0.5f, 0.0f},
                                                  {0.0f, 0.0f},  {0.0f, 1.0f},  {0.0f, -1.0f}, {0.5f, 0.0f},  {1.0f, 0.0f}};
    if (role < 0 || role >= kPlayerRoles) return Vec3(0, 0, 0);
    return Vec3(anchor[role][0], anchor[role][1], 0);
}

// GRF: the tactics the `TeamAIController` constructor sets, in TacticId order: the base ones and
// the live ones (the base mixed with `TeamData`'s). GRF keeps "%f" texts, read back as floats.
constexpr double kBaseTactics[kTacticKeys] = {0.75, 0.8, 0.5, 0.35, 0.54, 0.4, 0.8, 0.9, 0.7, 0.6, 0.35, 0.52, 0.1, 0.9};
constexpr double kLiveTactics[kTacticKeys] = {0.71, 0.938, 0.776, 0.35, 0.54, 0.332, 0.84, 0.868, 0.826, 0.828, 0.35, 0.52, 0.176, 0.948};

// GRF: `clamp` returns an in-range value itself, so a zero keeps its sign.
float GrfClamp(float value, float lo, float hi) {
    if (lo > value) return lo;
    if (hi < value) return hi;
    return value;
}

// GRF: `FormationEntry(x, y, ...)` scales the scenario's y into formation units.
constexpr float kFormationYScale = -2.36f;

FormationEntry EntryOf(const ScenarioPlayer &p) {
    FormationEntry e{};
    e.role = p.role;
    e.position = Vec3((float)p.x, (float)p.y * kFormationYScale, 0);
    e.startPosition = e.position;
    e.lazy = p.lazy;
    e.controllable = p.controllable;
    return e;
}

// GRF: `TeamData::TeamData` spreads the fixed slots (shape blended with the role anchor) and
// pushes apart outfield spots closer than 0.5, at most 10 rounds. The scenario then sets each
// spot's role, start position and flags by index, so a spot follows the player's index.
std::vector<FormationEntry> SpreadFormation(const std::vector<ScenarioPlayer> &team) {
    const int n = (int)team.size();
    std::vector<FormationEntry> spots(n);
    for (int i = 0; i < n; i++) {
        spots[i] = FormationEntry{};
        spots[i].role = kSlotRole[i];
        const Vec3 shape((float)kSlotShape[i][0], (float)kSlotShape[i][1], 0);
        spots[i].position = shape * 0.6f + RoleAnchor(spots[i].role) * 0.4f;
    }
    const float spacing = 0.5f;
    bool moved = true;
    for (int round = 0; moved && round < 10; round++) {
        std::vector<Vec3> push(n, Vec3(0, 0, 0));
        moved = false;
        for (int a = 0; a + 1 < n; a++) {
            if (spots[a].role == kRoleGoalkeeper) continue;
            for (int b = a + 1; b < n; b++) {
                if (spots[b].role == kRoleGoalkeeper) continue;
                const Vec3 gap = spots[a].position - spots[b].position;
                if (!(gap.Length() < spacing)) continue;
                moved = true;
                const float closeness = 1.0f - (gap.Length() / spacing);
                push[a] += gap.Normalized(Vec3(0, 1, 0)) * spacing * closeness * 0.5f;
                push[b] -= gap.Normalized(Vec3(0, 1, 0)) * spacing * closeness * 0.5f;
            }
        }
        if (!moved) break;
        for (int i = 0; i < n; i++) {
            spots[i].position += push[i];
            spots[i].position.v[0] = GrfClamp(spots[i].position.v[0], -1, 1);
            spots[i].position.v[1] = GrfClamp(spots[i].position.v[1], -1, 1);
        }
    }
    for (int i = 0; i < n; i++) {
        const FormationEntry own = EntryOf(team[i]);
        spots[i].startPosition = own.startPosition;
        spots[i].lazy = own.lazy;
        spots[i].role = own.role;
        spots[i].controllable = own.controllable;
    }
    return spots;
}

void CheckTeams(const ScenarioDescription &d) {
    for (int side = 0; side < 2; side++) {
        const std::vector<ScenarioPlayer> &team = side ? d.rightTeam : d.leftTeam;
        const std::string name = side ? "right" : "left";
        if (team.empty()) throw std::invalid_argument("the " + name + " team is empty; the scenario module adds its goalkeeper");
        if ((int)team.size() > kScenarioTeamPlayers)
            throw std::invalid_argument("the " + name + " team has " + std::to_string(team.size()) + " players, more than the 11 that GRF holds");
        if ((int)team.size() > kTeamPlayers)
            throw std::invalid_argument("the " + name + " team has " + std::to_string(team.size()) + " players, more than the " +
                                        std::to_string(kTeamPlayers) + " of this build");
        for (const ScenarioPlayer &p : team)
            if (p.role < 0 || p.role >= kPlayerRoles)
                throw std::invalid_argument("expected a player role from 0 to 9, found " + std::to_string(p.role));
        // GRF: the dynamic-role pass seeks the goalkeeper without advancing, so a team whose first
        // player is not one hangs GRF once the match is in open play.
        if (team.front().role != kRoleGoalkeeper)
            throw std::invalid_argument("the first player of the " + name + " team is not a goalkeeper, which hangs GRF once the match is in open play");
    }
}

class Bytes {
public:
    template <class T>
    void Put(const T &v) {
        out_.append(reinterpret_cast<const char *>(&v), sizeof(T));
    }
    void Text(const std::string &s) {
        Put((int32_t)s.size());
        out_ += s;
    }
    void Raw(const std::string &s) { out_ += s; }
    std::string &str() { return out_; }

private:
    std::string out_;
};

// Players in state order, then the three officials; FORM, MDUR and SIDS as ParseStatic reads them.
std::string StaticSection(const std::vector<FormationEntry> &spots, const std::vector<int> &person, int32_t officialSkin) {
    Bytes b;
    const int players = (int)spots.size();
    b.Put((int32_t)(players + 3));
    for (int e = 0; e < players + 3; e++) {
        PlayerData d{};
        if (e < players) {
            const float *row = kPersonValues[person[e]];
            for (int s = 0; s < kStatistics; s++) d.stats[s] = row[s];
            d.velocityStat = row[kStatistics];
            d.height = row[kStatistics + 1];
            d.skinColor = kPersonSkin[person[e]];
        } else {
            for (float &s : d.stats) s = kOfficialStatistic;
            d.velocityStat = kOfficialStatistic;
            d.height = kOfficialHeight;
            d.skinColor = officialSkin;
        }
        b.Put(d);
    }
    b.Raw("FORM");
    for (const FormationEntry &f : spots) {
        b.Put(f.role);
        b.Put(f.position);
        b.Put(f.startPosition);
        b.Put((uint8_t)f.lazy);
        b.Put((uint8_t)f.controllable);
    }
    b.Raw("MDUR");
    b.Put(kMatchDurationFactor);
    b.Raw("SIDS");
    // GRF: stable IDs follow creation order, which is state order with the officials last.
    for (int32_t e = 0; e < players + 3; e++) b.Put(e);
    return b.str();
}

// GRF: `player.object` as `HumanoidBase::ResetPosition` leaves its bones; the root sits at the
// origin with the file's rotation (a -0 z).
NodeState TemplateNode(int k) {
    NodeState n{};
    const GrfNode &g = kSkeletonNodes[k];
    n.position = k == 0 ? Vec3(0, 0, 0) : Vec3(g.position[0], g.position[1], g.position[2]);
    n.rotation = k == 0 ? Quat(0, 0, -0.0f, 1) : Quat(0, 0, 0, 1);
    n.scale = Vec3(1);
    n.localMode = g.localMode;
    return n;
}

// One CUJHUM1 record per humanoid: its node values with GRF's names and geometry.
std::string SkeletonSection(const std::vector<const NodeState *> &humanoids) {
    Bytes b;
    b.Raw("CUJHUM1");
    b.Put((int32_t)humanoids.size());
    for (const NodeState *nodes : humanoids) {
        for (int part = 0; part < kBodyParts; part++) b.Put(kSkeletonNodeMap[part]);
        b.Put((int32_t)kHumanoidNodes);
        for (int k = 0; k < kHumanoidNodes; k++) {
            const GrfNode &g = kSkeletonNodes[k];
            b.Text(g.name);
            b.Put(g.parent);
            b.Put(nodes[k].localMode);
            b.Put(nodes[k].position);
            b.Put(nodes[k].rotation);
            b.Put(nodes[k].scale);
            b.Put((int32_t)(g.geometry ? 1 : 0));
            if (!g.geometry) continue;
            b.Text(g.geometry);
            b.Put(g.geometryLocalMode);
            for (float v : g.geometryValues) b.Put(v);
        }
    }
    return b.str();
}

// GRF: a humanoid after the `HumanoidBase` constructor, whose default command chose the idle
// animation.
Humanoid FreshHumanoid() {
    Humanoid h{};
    for (int k = 0; k < kHumanoidNodes; k++) h.nodes[k] = TemplateNode(k);
    PlayerCommand &cmd = h.anim.originatingCommand;
    cmd.desiredFunctionType = kFnMovement;
    cmd.strictMovement = kStrictDynamic;
    cmd.touchInfo.targetPlayer = -1;
    cmd.touchInfo.forcedTargetPlayer = -1;
    cmd.tripType = 1;
    return h;
}

// GRF: `PlayerController::Reset` and `SetPlayer`.
PlayerControllerState FreshController(int player, int teamSlot) {
    PlayerControllerState s{};
    s.player = player;
    s.inputDirection = Vec3(0, -1, 0);
    s.team = teamSlot;
    s.opponentTeam = 1 - teamSlot;
    s.opponentPlayer = -1;
    s.lastSwitchTimeMs = (uint64_t)(int64_t)-10000;  // GRF stores -10000 in an unsigned field
    s.possessionAmount = 0.9f;
    s.teamPossessionAmount = 1.0f;
    s.fadingTeamPossessionAmount = 1.0f;
    s.oppTimeNeededToGetToBall = 100;
    return s;
}

Tactics TacticsOf(const double (&values)[kTacticKeys]) {
    Tactics t{};
    t.present = (1u << kTacticKeys) - 1;
    for (int k = 0; k < kTacticKeys; k++) t.value[k] = (float)values[k];
    return t;
}

float DrawInRange(uint8_t *rng, float lo, float hi) {
    Rng g{rng};
    const float stretch = hi - lo;
    return lo + g.Uniform() * stretch;
}

struct BuiltVariant {
    std::string staticData, state, skeletons;
};

BuiltVariant BuildVariant(const ScenarioDescription &d, bool reverse, const AnimationTables &tables) {
    CheckTeams(d);
    // Value-initialized, as GRF's objects start: zeros, with every quaternion the identity.
    auto world = std::make_unique<World>();
    World &w = *world;
    w.flags.teamSide[0] = w.flags.teamSide[1] = -1;
    Scenario &sc = w.scenario;
    MatchState &m = w.match;

    // 1000 + reverse seeds the shipped bundles; a deterministic scenario keeps its own seed.
    const uint32_t seed = d.deterministic ? d.gameEngineRandomSeed : 1000u + (reverse ? 1u : 0u);

    // GRF: `GameEnv::reset` runs with the game running and the step at -1; the generator draws
    // `uniform_real<float>(0, 1)`.
    w.gameState = kRunning;
    w.waitingForGameCount = 0;
    w.step = -1;
    const float range[2] = {0.0f, 1.0f};
    memcpy(w.rng + 2504, range, sizeof(range));

    // GRF: `GameEnv::setConfig` scales the ball position in double.
    sc.ballPosition = Vec3((float)((double)(float)d.ballX * 54.4), (float)((double)(float)d.ballY * -83.6), 0);
    sc.leftTeamSize = (int32_t)d.leftTeam.size();
    sc.rightTeamSize = (int32_t)d.rightTeam.size();
    sc.leftAgents = sc.rightAgents = 0;
    sc.useMagnet = d.useMagnet;
    sc.offsides = d.offsides;
    sc.leftDifficulty = (float)d.leftTeamDifficulty;
    sc.rightDifficulty = (float)d.rightTeamDifficulty;
    sc.deterministic = d.deterministic;
    sc.endOnScore = d.endOnScore;
    sc.endOnPossessionChange = d.endOnPossessionChange;
    sc.endOnOutOfPlay = d.endOnOutOfPlay;
    sc.gameDuration = d.gameDuration;
    sc.secondHalf = d.secondHalf;
    sc.controlAllPlayers = d.controlAllPlayers;
    sc.realTime = d.realTime;
    sc.gameEngineRandomSeed = seed;
    sc.reverseTeamProcessing = reverse;
    for (int p = 0; p < sc.leftTeamSize; p++) sc.leftTeam[p] = EntryOf(d.leftTeam[p]);
    for (int p = 0; p < sc.rightTeamSize; p++) sc.rightTeam[p] = EntryOf(d.rightTeam[p]);

    // Slot 0 holds the team processed first: the right team when reversed.
    m.firstTeam = 0;
    m.secondTeam = 1;
    m.playerCount = sc.leftTeamSize + sc.rightTeamSize;
    const int firstTeamID = reverse ? 1 : 0;
    const std::vector<ScenarioPlayer> *bySlot[2] = {firstTeamID == 0 ? &d.leftTeam : &d.rightTeam,
                                                    firstTeamID == 0 ? &d.rightTeam : &d.leftTeam};
    std::vector<FormationEntry> spots;
    std::vector<int> person;
    for (int slot = 0; slot < 2; slot++) {
        const std::vector<FormationEntry> team = SpreadFormation(*bySlot[slot]);
        for (int i = 0; i < (int)team.size(); i++) {
            spots.push_back(team[i]);
            person.push_back(i);
        }
    }

    // GRF: `Player::Player`, `Player::Activate` and `Player::ResetSituation`, first team first.
    const int firstSize = (int)bySlot[0]->size();
    for (int p = 0; p < m.playerCount; p++) {
        Player &pl = m.players[p];
        pl.base.isActive = true;
        pl.base.humanoid = FreshHumanoid();
        pl.controller.base = FreshController(p, p < firstSize ? 0 : 1);
        pl.base.externalController = -1;
        pl.base.lastTouchType = kTouchNone;
        pl.base.fatigueFactorInverse = 1.0f;
        pl.manMarking = -1;
        pl.dynamicFormationEntry = spots[p];
        pl.timeToBallMs = pl.timeToBallOptimisticMs = pl.timeToBallPreviousMs = 1000;
    }
    for (PersonBase &o : m.officials) {
        o.isActive = true;
        o.humanoid = FreshHumanoid();
        o.externalController = -1;
        o.lastTouchType = kTouchNone;
        o.fatigueFactorInverse = 1.0f;
    }
    // GRF: the `Team` and `TeamAIController` constructors.
    for (Team &t : m.teams) {
        t.timeToBallMs = 100;
        t.teamPossessionAmount = 1.0f;
        t.fadingTeamPossessionAmount = 1.0f;
        TeamAI &ai = t.ai;
        ai.taker = -1;
        ai.setPieceType = kModeNormal;
        ai.baseTactics = TacticsOf(kBaseTactics);
        ai.liveTactics = TacticsOf(kLiveTactics);
        ai.offensivenessBias = 0.5f;
        ai.depth = 0.45f;
        ai.width = 0.95f;
        ai.attackingRunPlayer = ai.teamPressurePlayer = ai.forwardSupportPlayer = -1;
        t.lastTouchPlayer = -1;
        t.mainSelectedPlayer = -1;
    }
    // The possession time is stored negated while the right team comes first, so it starts at -0.
    m.goalCount[0] = m.goalCount[1] = 0;
    m.possessionLastMinute = reverse ? -0.0f : 0.0f;
    // GRF: one keyboard per possible gamer, disabled and unmirrored while no gamer owns it.
    m.freeControllerCount = 2 * kTeamPlayers;
    for (int k = 0; k < m.freeControllerCount; k++) {
        KeyboardState &kb = m.freeControllers[k];
        kb = KeyboardState{};
        kb.mirror = 1.0f;
        kb.direction = Vec3(0);
        kb.disabled = true;
    }
    // GRF: `Ball::Ball` predicts the flight of a ball at rest at the origin.
    BallCalculatePrediction(m.ball, false);
    m.lastGoalTeam = m.lastGoalScorer = -1;
    for (int32_t &id : m.lastTouchTeamIDs) id = -1;
    m.lastTouchTeamID = -1;
    m.bestPossessionTeam = -1;
    m.designatedPossessionPlayer = 0;
    m.ballRetainer = -1;
    m.possessionSideHistoryMaxTimeMs = 6000;
    m.autoUpdateInGameCamera = true;
    // The referee prepares the first team's kick-off, in the frame of the rest.
    RefereeBuffer &rb = m.referee.buffer;
    rb.active = true;
    rb.desiredSetPiece = kModeKickOff;
    rb.teamID = firstTeamID;
    rb.setPieceTeam = 0;
    rb.startTime = 2000;
    rb.restartPos = sc.ballPosition;
    rb.taker = -1;
    rb.endPhase = true;
    m.referee.foul.foulPlayer = m.referee.foul.foulVictim = -1;
    m.referee.foul.hasBeenProcessed = true;

    // GRF: each player resets its position twice before the officials draw their skin colour.
    uint8_t skinRng[sizeof(w.rng)];
    memcpy(skinRng, w.rng, sizeof(skinRng));
    Rng{skinRng}.Seed(seed);
    for (int draw = 0; draw < 2 * m.playerCount; draw++) DrawInRange(skinRng, 0, 1);
    const int32_t officialSkin = (int32_t)std::round(DrawInRange(skinRng, 1, 4));

    BuiltVariant out;
    out.staticData = StaticSection(spots, person, officialSkin);
    const StaticData sd = ParseStatic(out.staticData);
    // GRF scales only the rendered mesh by the height, so every humanoid has one skeleton.
    std::vector<NodeState> pose(kHumanoidNodes);
    for (int k = 0; k < kHumanoidNodes; k++) pose[k] = TemplateNode(k);
    const std::vector<const NodeState *> poses(m.playerCount + 3, pose.data());
    const std::vector<Skeleton> skeletons = ParseSkeletons(SkeletonSection(poses));
    const Tables view = tables.View();
    auto scratch = std::make_unique<Scratch>();
    Ctx c{};
    c.t = &view;
    c.sd = &sd;
    c.skeletons = skeletons.data();
    c.ticksPerStep = 10;
    c.ws = scratch.get();

    // GRF: creating the match draws the idle frames, the officials' skin and the lighting.
    InitializePlayerTeams(w);
    if (!ResetFromTemplate(w, c, seed)) throw std::runtime_error("the simulation does not support the creation of this scenario");
    // GRF: `Team::AddHumanGamers` takes each team's player closest to the ball at the origin.
    for (int teamID = 0; teamID < 2; teamID++)
        TeamByID(w, teamID).designatedTeamPossessionPlayer = GetClosestPlayer(w, c, teamID, BallPredict(m.ball, 0).Get2D(), false);

    StateCodec codec;
    codec.freeControllerCount = m.freeControllerCount;
    out.state = codec.SaveFrame(w, 0);

    // The skeletons record the pose after the ticks into play; the simulation reads the state.
    auto played = std::make_unique<World>(w);
    auto core = std::make_unique<EnvCore>();
    memset(core.get(), 0, sizeof(EnvCore));
    if (!SettleAfterReset(*played, c, *core))
        throw std::runtime_error("the simulation does not support the ticks that bring this scenario into play");
    std::vector<const NodeState *> nodes;
    for (int p = 0; p < m.playerCount; p++) nodes.push_back(played->match.players[p].base.humanoid.nodes);
    for (int o = 0; o < 3; o++) nodes.push_back(played->match.officials[o].humanoid.nodes);
    out.skeletons = SkeletonSection(nodes);
    return out;
}

}  // namespace

std::string BuildScenarioBundle(const std::string &name, const ScenarioDescription (&parity)[2], const std::string &animations) {
    if (parity[0].leftTeam.size() != parity[1].leftTeam.size() || parity[0].rightTeam.size() != parity[1].rightTeam.size())
        throw std::invalid_argument("the team sizes depend on the parity of the episode, which a bundle does not support");
    const std::unique_ptr<AnimationTables> tables = LoadAnimationTables(animations);
    Bytes b;
    b.Raw("CUJASSET1");
    b.Text(name);
    b.Put((int32_t)0);  // left agents
    b.Put((int32_t)0);  // right agents
    b.Put((int32_t)4);  // variants
    for (int reverse = 0; reverse < 2; reverse++)
        for (int p = 0; p < 2; p++) {
            const BuiltVariant v = BuildVariant(parity[p], reverse != 0, *tables);
            b.Put((int32_t)reverse);
            b.Put((int32_t)p);
            for (const std::string *part : {&v.staticData, &v.state, &v.skeletons}) {
                b.Put((uint32_t)part->size());
                b.Raw(*part);
            }
        }
    return b.str();
}

}  // namespace host
}  // namespace eng
