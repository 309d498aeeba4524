// SPDX-License-Identifier: Apache-2.0
// Restates game logic of cuju (Copyright 2026 The cuju Authors), a reimplementation of Google
// Research Football (Copyright 2019 Google LLC); see NOTICE.
// The match of one environment: GRF's serialized engine objects (their fields are GRF's state
// format, include/cuju/state/environment_state.h:91-882) plus the frame bookkeeping a state omits.
// Each struct lists its fields in GRF's byte order and visits them in that order, so one routine
// loads and saves a state. A pointer is an int32 index, -1 for null.
#pragma once

#include "vec.h"

namespace eng {

#ifndef CUJU_TEAM_PLAYERS
#define CUJU_TEAM_PLAYERS 11
#endif
constexpr int kTeamPlayers = CUJU_TEAM_PLAYERS;
constexpr int kPlayers = 2 * kTeamPlayers;
constexpr int kAnimPositions = 320;  // frames of the longest animation, rounded up
constexpr int kBodyParts = 14;
constexpr int kHumanoidNodes = 14;
constexpr int kControllers = 32;
constexpr int kMatchKeyboards = 22;
constexpr int kTacticKeys = 14;

// A list whose count and elements a state stores; capacity is fixed.
template <class T, int N>
struct List {
    static constexpr int kCapacity = N;
    int32_t count = 0;
    T e[N];
    HD T &operator[](int i) { return e[i]; }
    HD const T &operator[](int i) const { return e[i]; }
    HD void push_back(const T &x) {
        if (count >= N) Unsupported("a state list outgrows its capacity");
        else e[count++] = x;
    }
    HD T *begin() { return e; }
    HD T *end() { return e + count; }
    HD const T *begin() const { return e; }
    HD const T *end() const { return e + count; }
};

// GRF's radian: the true angle is `angle - PI` when `rotated` (a mirror flips the flag).
struct Radian {
    float angle;
    bool rotated;
    uint8_t pad[3];
    HD float value() const { return rotated ? angle - PI : angle; }
    HD void set(float v) {
        angle = v;
        rotated = false;
    }
};
static_assert(sizeof(Radian) == 8, "radian layout");

// ---- humanoid -------------------------------------------------------------------------------------

struct BiasedOffset {
    Quat orientation;
    float bias;
};
struct MovementHistoryEntry {
    Vec3 position;
    Quat orientation;
    int32_t timeDifferenceMs;
    int32_t nodeName;
};
struct NodeState {
    Vec3 position;
    Quat rotation;
    Vec3 scale;
    int32_t localMode;
};
struct TouchInformation {
    Vec3 inputDirection;
    float inputPower, autoDirectionBias, autoPowerBias;
    Vec3 desiredDirection;
    float desiredPower;
    int32_t targetPlayer, forcedTargetPlayer;
};
struct PlayerCommand {
    int32_t desiredFunctionType;
    bool useDesiredMovement;
    Vec3 desiredDirection;
    int32_t strictMovement;
    float desiredVelocityFloat;
    bool useDesiredLookAt;
    Vec3 desiredLookAt;
    bool useTouchInformation;
    TouchInformation touchInfo;
    bool onlyDeflectAnimationsThatPickupBall, useTripType;
    int32_t tripType;
    bool useDesiredTripDirection;
    Vec3 desiredTripDirection;
    bool useSpecialVar1;
    int32_t specialVar1;
    bool useSpecialVar2;
    int32_t specialVar2;
    int32_t modifier;
};
struct FormationEntry {
    int32_t role;
    Vec3 position, startPosition;
    bool lazy, controllable;
};
struct PlayerImage {
    Vec3 position, directionVector, movement;
    int32_t player;
    int32_t velocity, role;
};
struct AnimationState {
    int32_t anim;
    int32_t id, frameNum, functionType, originatingInterrupt;
    Vec3 actionSmuggle, actionSmuggleOffset, actionSmuggleSustain, actionSmuggleSustainOffset,
        movementSmuggle, movementSmuggleOffset;
    Radian rotationSmuggleBegin, rotationSmuggleEnd;
    Radian rotationSmuggleOffset;
    int32_t touchFrame;
    Vec3 touchPos, incomingMovement, outgoingMovement, positionOffset;
    PlayerCommand originatingCommand;
    List<Vec3, kAnimPositions> positions;
};
struct AnimApplyBuffer {
    int32_t anim;
    int32_t frameNum;
    bool smooth;
    float smoothFactor;
    bool noPos;
    Vec3 position;
    Radian orientation;
    BiasedOffset offsets[kBodyParts];
};
struct SpatialState {
    Vec3 position;
    Radian angle;
    Vec3 directionVec;
    int32_t velocityCat;
    float floatVelocity;
    Vec3 actualMovement, physicsMovement, animationMovement, movement, actionSmuggleMovement,
        movementSmuggleMovement, positionOffsetMovement;
    Radian bodyAngle;
    Vec3 bodyDirectionVec;
    Radian relBodyAngleNonQuantized, relBodyAngle;
    Vec3 relBodyDirectionVec, relBodyDirectionVecNonQuantized;
    int32_t foot;
};
// In the order of use: the spatial state and the small fields, the nodes, the apply buffer, the
// animation (its planned positions last), the movement history.
struct Humanoid {
    SpatialState spatial;
    int32_t prevAnimFrameNum, prevAnimFunctionType;
    Vec3 startPos;
    Radian startAngle;
    Vec3 nextStartPos;
    Radian nextStartAngle;
    Vec3 prevPosition2D;
    int32_t interruptAnim, requeueDelayFrames, tripType;
    Vec3 tripDirection, decayingPositionOffset;
    float decayingDifficultyFactor;
    int32_t mentalImageTime;
    NodeState nodes[kHumanoidNodes];
    AnimApplyBuffer applyBuf;
    BiasedOffset offsets[kBodyParts];
    AnimationState anim;
    List<MovementHistoryEntry, 32> movementHistory;
};

// ---- controllers ----------------------------------------------------------------------------------

struct PlayerControllerState {
    int32_t player;
    Vec3 inputDirection;
    float inputVelocityFloat;
    int32_t team, opponentTeam;
    int32_t opponentPlayer;
    float timeNeededMs;
    int32_t mentalImageTime;
    uint64_t lastSwitchTimeMs;
    uint32_t lastSwitchTimeDurationMs;
    bool hasPossession, hasUniquePossession, teamHasPossession, teamHasUniquePossession,
        oppTeamHasPossession, oppTeamHasUniquePossession, hasBestPossession, teamHasBestPossession;
    float possessionAmount, teamPossessionAmount, fadingTeamPossessionAmount;
    int32_t oppTimeNeededToGetToBall;
    bool hasBestChanceOfPossession;
};
struct AIControllerState {
    PlayerControllerState base;
    bool ballBoundForGoal;
    float ballBoundForGoalY;
    Vec3 lastDesiredDirection;
    float lastDesiredVelocity;
};
struct KeyboardState {
    float mirror;
    Vec3 direction;  // stored times `mirror`
    bool disabled;
    bool buttons[11];
};
struct HumanControllerState {
    PlayerControllerState base;
    KeyboardState keyboard;
    int32_t actionMode, actionButton, actionBufferTimeMs, gaugeMs;
    Vec3 previousDirection, steadyDirection;
    int32_t lastSteadyDirectionSnapshotTimeMs;
};
struct HumanGamer {
    int32_t selectedPlayer;
    int32_t team;
    int32_t keyboardIndex;
    HumanControllerState controller;
};

// The part of a player an official shares.
struct PersonBase {
    bool isActive;
    int32_t externalController;
    uint64_t lastTouchTimeMs;
    int32_t lastTouchType;
    float fatigueFactorInverse;
    Humanoid humanoid;
    List<Vec3, 512> positionHistoryPerSecond;
};
struct TacticalSituation {
    float forwardSpaceRating, toGoalSpaceRating, spaceRating, forwardRating;
};
// The player's own small fields first, then its controller and its person.
struct Player {
    int32_t manMarking;
    FormationEntry dynamicFormationEntry;
    bool hasPossession, hasBestPossession, hasUniquePossession;
    int32_t possessionDurationMs;
    uint32_t timeToBallMs, timeToBallOptimisticMs, timeToBallPreviousMs;
    bool triggerControlledBallCollision;
    TacticalSituation tactical;
    bool bufferNameCaptionShowCondition;
    Vec3 bufferPlayerColor;
    int32_t desiredTimeToBallMs, cards;
    uint64_t cardEffectiveTimeMs;
    AIControllerState controller;  // stored only while active
    PersonBase base;
};

// ---- teams ----------------------------------------------------------------------------------------

// GRF stores tactics as a map of 14 keys to "%f" texts; the float of each text is kept.
enum TacticId {
    kDefenseDepth,
    kDefenseMicroFocusStrength,
    kDefenseMidfieldFocus,
    kDefenseMidfieldFocusStrength,
    kDefenseOwnHalf,
    kDefenseSideFocusStrength,
    kDefenseWidth,
    kOffenseDepth,
    kOffenseMicroFocusStrength,
    kOffenseMidfieldFocus,
    kOffenseMidfieldFocusStrength,
    kOffenseOwnHalf,
    kOffenseSideFocusStrength,
    kOffenseWidth
};
struct Tactics {
    uint32_t present;
    float value[kTacticKeys];
};
struct TacticalOpponent {
    int32_t player;
    float dangerFactor;
};
struct TeamAI {
    int32_t taker;
    int32_t setPieceType;
    Tactics baseTactics, liveTactics;
    float offensivenessBias;
    bool teamHasPossession, teamHasUniquePossession, oppTeamHasPossession,
        oppTeamHasUniquePossession, teamHasBestPossession;
    float teamPossessionAmount, fadingTeamPossessionAmount;
    int32_t timeNeededToGetToBall, oppTimeNeededToGetToBall;
    float depth, width, offsideTrapX;
    uint64_t endApplyAttackingRunMs;
    int32_t attackingRunPlayer;
    uint64_t endApplyTeamPressureMs;
    int32_t teamPressurePlayer;
    uint64_t endApplyKeeperRushMs;
    int32_t forwardSupportPlayer;
    List<TacticalOpponent, kTeamPlayers> tacticalOpponents;
};
struct Team {
    bool hasPossession;
    int32_t timeToBallMs;
    int32_t designatedTeamPossessionPlayer;
    float teamPossessionAmount, fadingTeamPossessionAmount;
    int32_t lastTouchPlayer, mainSelectedPlayer;
    TeamAI ai;
    List<int32_t, kTeamPlayers> switchPriority;
    List<HumanGamer, kTeamPlayers> gamers;
};

struct MentalImage {
    uint32_t timeStampMs;
    float maxDistanceDeviation, maxMovementDeviation;
    List<PlayerImage, kPlayers> players;
    List<Vec3, 320> ballPredictions;
    bool lazyFlip;  // not in the state: the predictions hold negated x and y
    // Not in the state: the player images of team t hold negated x and y when lazyTeamFlip[t].
    bool lazyTeamFlip[2];
};

// The scalars first, then the prediction and history arrays.
struct Ball {
    Vec3 momentum;
    Quat rotationPerMs;
    int32_t validPredictions;
    Quat orientationPrediction;
    Vec3 positionBuffer;
    Quat orientationBuffer;
    bool touchesNet;
    bool lazyFlip;  // not in the state: predictions and history hold negated x and y
    // Not in the state: the inputs and first-step results of the last full prediction, which a
    // prediction from the same inputs recomputes bit for bit. Every other write of `predictions`
    // clears `memoValid`.
    bool memoValid, memoInGoal, memoTouchesNet;
    Vec3 memoPosition, memoMomentum, memoOutMomentum;
    Quat memoOrientation, memoRotation, memoOutRotation;
    Vec3 predictions[401];
    List<Vec3, 402> positionHistory;
};

struct RefereeBuffer {
    bool active;
    int32_t desiredSetPiece;
    int32_t teamID;
    int32_t setPieceTeam;
    uint64_t stopTime, prepareTime, startTime;
    Vec3 restartPos;
    int32_t taker;
    bool endPhase;
};
struct Foul {
    int32_t foulPlayer, foulVictim;
    int32_t foulType;
    bool advantage;
    uint64_t foulTime;
    Vec3 foulPosition;
    bool hasBeenProcessed;
};
struct Referee {
    RefereeBuffer buffer;
    int32_t afterSetPieceRelaxTimeMs;
    List<int32_t, kTeamPlayers> offsidePlayers;
    Foul foul;
};

// Members up to `controlAllPlayers` are constant over an episode.
struct Scenario {
    Vec3 ballPosition;
    int32_t leftTeamSize, rightTeamSize, leftAgents, rightAgents;
    bool useMagnet, offsides;
    float leftDifficulty, rightDifficulty;
    bool deterministic, endOnScore, endOnPossessionChange, endOnOutOfPlay;
    int32_t gameDuration, secondHalf;  // steps
    bool controlAllPlayers;
    bool realTime;
    uint32_t gameEngineRandomSeed;
    bool reverseTeamProcessing;  // the second team plays from the left
    FormationEntry leftTeam[kTeamPlayers], rightTeam[kTeamPlayers];
};

// The scalars first, then the teams, the ball and the referee, then the large arrays.
struct MatchState {
    int32_t firstTeam, secondTeam;
    int32_t playerCount;
    int32_t goalCount[2];
    float possessionLastMinute;
    uint64_t matchTimeMs, actualTimeMs, goalScoredTimer;
    int32_t matchPhase;
    bool inPlay, inSetPiece, goalScored, ballIsInGoal;
    int32_t lastGoalTeam;
    int32_t lastGoalScorer;
    int32_t lastTouchTeamIDs[4];
    int32_t lastTouchTeamID;
    int32_t bestPossessionTeam;
    int32_t designatedPossessionPlayer;
    int32_t ballRetainer;
    uint32_t possessionSideHistoryMaxTimeMs;
    uint32_t lastBodyBallCollisionTimeMs;
    int32_t freeControllerCount;
    bool autoUpdateInGameCamera;
    float cameraFov, cameraNearCap, cameraFarCap;
    Quat cameraOrientation, cameraNodeOrientation;
    Vec3 cameraNodePosition;
    Team teams[2];  // teams[0] is processed first
    Ball ball;
    Referee referee;
    List<MentalImage, 4> mentalImages;
    Player players[kPlayers];
    PersonBase officials[3];  // referee, two linesmen
    KeyboardState secondKeyboardCopies[kControllers];
    KeyboardState freeControllers[kControllers];
    List<float, 600> possessionSideHistory;
    List<Vec3, 160> cameraPosition;
};

// Frames between ticks: each team in its own frame (side -1, unmirrored), the ball in team 0's.
struct FrameFlags {
    bool teamMirrored[2];
    int32_t teamSide[2];
    bool ballMirrored;
    bool humanoidMirrored[kPlayers];
    bool mentalBallMirrored[4];
};

// Copies of the per-player fields that scans over a team read for every player, side by side so
// that a scan touches two cache lines instead of one line per player (a Player spans 13 KB). The
// engine writes each copy where it writes the field (SetPlayerActive, SetPlayerTimeToBall); a load
// of a state fills them (InitializePlayerTeams).
struct Roster {
    bool active[kPlayers];              // players[p].base.isActive
    uint32_t timeToBallMs[kPlayers];    // players[p].timeToBallMs
};

// The members are in the order of their use, the small and often read first, so that a match's
// hot scalars share a few cache lines; the state codec visits them in GRF's order by name.
struct World {
    int32_t gameState;
    int32_t waitingForGameCount;
    int32_t step;
    // Not in a state.
    FrameFlags flags;
    int32_t playerTeamID[kPlayers];
    // 0: the player's own formation entry; else 1 + the player whose entry it uses.
    int8_t formationOverride[kPlayers];
    Roster roster;
    // The state.
    Scenario scenario;
    MatchState match;
    uint8_t rng[2512];
    HD int FirstTeamID() const { return match.firstTeam ^ (scenario.reverseTeamProcessing ? 1 : 0); }
};

}  // namespace eng
