// SPDX-License-Identifier: Apache-2.0
// Restates game logic of cuju (Copyright 2026 The cuju Authors), a reimplementation of Google
// Research Football (Copyright 2019 Google LLC); see NOTICE.
// Read-only tables of the simulation, laid out as flat arrays addressed by index so one host build
// step produces them and a single copy moves them to HBM (every span is an index range, not a
// pointer). Semantics follow include/cuju/animation/animation_data.h:21-155,
// include/cuju/animation/animation_derived.h:54-98, include/cuju/animation/skeleton.h:17-45,
// include/cuju/simulation/static_data.h:17-60 and the selection records of
// include/cuju/simulation/select_animation.h:431-533.
#pragma once

#include "state.h"

namespace eng {

// ---- enumerations (GRF's; a state stores them as integers) ----------------------------------------
enum Velocity { kVelIdle, kVelDribble, kVelWalk, kVelSprint };
enum FunctionType {
    kFnNone,
    kFnMovement,
    kFnBallControl,
    kFnTrap,
    kFnShortPass,
    kFnLongPass,
    kFnHighPass,
    kFnHeader,
    kFnShot,
    kFnDeflect,
    kFnCatch,
    kFnInterfere,
    kFnTrip,
    kFnSliding,
    kFnSpecial
};
enum TouchType { kTouchKicked, kTouchNonKicked, kTouchAccidental, kTouchNone };
enum Role {
    kRoleGoalkeeper,
    kRoleCentreBack,
    kRoleLeftBack,
    kRoleRightBack,
    kRoleDefensiveMid,
    kRoleCentralMid,
    kRoleLeftMid,
    kRoleRightMid,
    kRoleAttackingMid,
    kRoleCentreForward
};
enum GameMode { kModeNormal, kModeKickOff, kModeGoalKick, kModeFreeKick, kModeCorner, kModeThrowIn, kModePenalty };
enum StrictMovement { kStrictFalse, kStrictTrue, kStrictDynamic };
enum BodyPart {
    kBpMiddle,
    kBpNeck,
    kBpLeftThigh,
    kBpRightThigh,
    kBpLeftKnee,
    kBpRightKnee,
    kBpLeftAnkle,
    kBpRightAnkle,
    kBpLeftShoulder,
    kBpRightShoulder,
    kBpLeftElbow,
    kBpRightElbow,
    kBpBody,
    kBpPlayer
};
enum Interrupt {
    kIntNone,
    kIntSwitch,
    kIntSliding,
    kIntBump,
    kIntTrip,
    kIntCheat,
    kIntCancel,
    kIntReQueue
};
// Animation type strings (GRF's e_AnimationString).
enum AnimType {
    kAtEmpty = 0,
    kAtType = 5,
    kAtTrap = 6,
    kAtDeflect = 7,
    kAtInterfere = 8,
    kAtTrip = 9,
    kAtShortPass = 10,
    kAtLongPass = 11,
    kAtShot = 12,
    kAtSliding = 13,
    kAtMovement = 14,
    kAtSpecial = 15,
    kAtBallControl = 16,
    kAtHighPass = 17,
    kAtCatch = 18
};
enum StateString { kStrEmpty, kStrLayBack, kStrLayFront, kStrLeftElbow, kStrRightElbow };
enum Statistic {
    kStatBalance,
    kStatReaction,
    kStatAcceleration,
    kStatVelocity,
    kStatStamina,
    kStatAgility,
    kStatShotPower,
    kStatStandingTackle,
    kStatSlidingTackle,
    kStatBallControl,
    kStatDribble,
    kStatShortPass,
    kStatHighPass,
    kStatHeader,
    kStatShot,
    kStatVolley,
    kStatCalmness,
    kStatWorkRate,
    kStatResilience,
    kStatDefensivePositioning,
    kStatOffensivePositioning,
    kStatVision
};
constexpr int kStatistics = 22;

// ---- static data of a scenario variant -------------------------------------------------------------
struct PlayerData {
    float stats[kStatistics];
    float velocityStat;
    float height;
    int32_t skinColor;
};
struct StaticFormation {
    int32_t role;
    Vec3 position, startPosition;
    bool lazy, controllable;
};
constexpr int kStaticEntries = kPlayers + 3;
// Players in state order, then the referee and two linesmen.
struct StaticData {
    int32_t count;
    PlayerData data[kStaticEntries];
    StaticFormation formation[kStaticEntries];
    float matchDurationFactor;
    int32_t stableID[kStaticEntries];
};

// ---- skeleton -------------------------------------------------------------------------------------
constexpr int kLocalRelative = 0, kLocalAbsolute = 1;
struct SkelGeometry {
    bool footOrLowerLeg;
    int32_t localMode;
    Vec3 position;
    Quat rotation;
    Vec3 scale;
    Vec3 boxMin, boxMax;  // mesh space
};
struct SkelNode {
    int32_t parent;
    int32_t localMode;
    Vec3 position;
    Quat rotation;
    Vec3 scale;
    int32_t geometryCount;
    SkelGeometry geometries[2];
};
struct Skeleton {
    int32_t nodeMap[kBodyParts];
    int32_t nodeCount;
    SkelNode nodes[kHumanoidNodes];  // pre-order
};

// ---- animations -----------------------------------------------------------------------------------
struct KeyFrame {
    int32_t frame;
    Quat orientation;
    Vec3 position;
};
struct InterpEntry {
    Quat orientation;
    Vec3 position;
    float angleZ;  // yaw of `orientation` by Quat::Angles
};
struct MiddleEntry {
    Quat orientation;
    Vec3 position;
    Quat normalized;
    bool normalizedKeepsZeros;  // squared length in [1e-6, 2): normalizing keeps every zero
};
struct NodeAnim {
    int32_t bodyPart;
    int32_t keyFirst, keyCount;
    // Frame f (0..frameCount+1) of the node is entry interpFirst + f * interpStride of interp[] and
    // middle[]: an animation's nodes lie side by side frame after frame, so the nodes of a pose
    // share cache lines.
    int32_t interpFirst;
    int32_t interpFrames;  // frameCount + 2
    int32_t interpStride;  // the animation's node count
};
struct FootballKey {
    int32_t frame;
    Quat orientation;
    Vec3 position;
    float power;
};
struct Anim {
    int32_t frameCount, currentFoot, animationType;
    Vec3 translation, incomingMovement;
    float incomingVelocity;
    Vec3 outgoingMovement, outgoingDirection, incomingBodyDirection, outgoingBodyDirection;
    float outgoingVelocity;
    Radian outgoingAngle, incomingBodyAngle, outgoingBodyAngle;
    int32_t outgoingFoot;
    float idleLevel;
    int32_t quadrantID;
    float specialVar1, specialVar2;
    bool lastDitch, baseAnimation;
    int32_t outgoingSpecialState, incomingRetainState, incomingSpecialState;
    int32_t nodeFirst, nodeCount;
    int8_t nodeOfBodyPart[kBodyParts];  // the node that moves each body part, -1 for none
    bool hasFootball;
    int32_t footballFirst, footballCount;
    bool hasPositions;
    int32_t posFirst, posCount;
};
struct Quadrant {
    int32_t id;
    Vec3 position;
    int32_t velocity;
    Radian angle;
};
// Values GRF parses from each animation's text variables at every use, parsed once on the host.
struct AnimDerived {
    double priorityAbsolute;
    int32_t touchFrame;
    float difficultyFactor;
    bool tripTypeIsOne;
    int32_t tripTypeRounded;
    Vec3 bumpDirection, incomingBallDirection, ballDirection;
    float incomingMaxDeviation, outgoingMaxDeviation;
    bool outgoingRetainRaw;
    int32_t outgoingRetainRawValue, incomingRetainRawValue;
    int32_t outgoingRetainBodyPart, incomingRetainBodyPart;
    int32_t forcedFootWhich;  // 0 none, 1 strong, 2 weak
    bool touchFootLeft;
    int32_t touchType;  // 0 kicked (foot or lower leg), 1 non-kicked
    float touchMaxPowerFactor, touchDifficultyFactor;
    // Animation-only terms of the crude selection, computed with the same functions.
    Vec3 crudeOutDirectionRotated;
    float crudeTurnAngle, crudeInBodyFixAbsolute;
    Vec3 crudeOutBodyDirection;
    bool crudeInBallNonzero;
    Vec3 crudeInBallAdapted, crudeBallDirectionNormalized;
};
// Per-animation terms of the selection sorts, computed on the host with the same expressions.
struct SelectionRecord {
    float incomingBodyAngles[6];
    float bodyTurnAngle;
    int32_t incomingBodyIndex;
    Vec3 preferredOutgoingDirection, preferredOutgoingMovement;
    float preferredOutgoingAngle;
    float lookAngle;
    int32_t smoothedFirst;  // into smoothed[], -1 below two positions
    bool ballDirectionFinite;
};
// Every term the crude selection reads of one animation, copied from Anim, AnimDerived and
// SelectionRecord into one 128-byte line: the filter tests hundreds of animations per query, and
// one line each is what it moves. `flags`: bit 0 outgoing retain, 1 last ditch, 2 nonzero
// incoming ball direction, 3 finite outgoing ball direction, 4 touching foot left.
struct alignas(128) CrudeRecord {
    Vec3 incomingBodyDirection, outDirectionRotated, inBallAdapted, ballDirectionNormalized;
    float incomingVelocity, outgoingVelocity, turnAngle, inBodyFixAbsolute;
    float incomingBodyAngles[6];
    float bodyTurnAngle;
    float incomingMaxDeviation, outgoingMaxDeviation, specialVar1, specialVar2;
    int16_t index, animationType, incomingSpecialState, incomingRetainState, tripTypeRounded;
    int8_t forcedFootWhich, currentFoot;
    uint8_t flags;
};
static_assert(sizeof(CrudeRecord) == 128, "one crude record per cache line");
constexpr int kFunctionSlots = 16;
constexpr int kMaxAnimations = 1536;  // the tables hold 1452
constexpr int kCameraHistory = 150;
constexpr int kCameraWeights = kCameraHistory * (kCameraHistory + 1) / 2;

struct Tables {
    const Anim *anims;
    int32_t animCount;
    const NodeAnim *nodes;
    const KeyFrame *keys;
    const InterpEntry *interp;
    const MiddleEntry *middle;
    const FootballKey *football;
    const Vec3 *positions;
    const Quadrant *quadrants;
    int32_t quadrantCount;
    Radian maxIncomingBallDeviation, maxOutgoingBallDeviation;
    const AnimDerived *derived;
    const SelectionRecord *selection;
    const Vec3 *smoothed;
    const int16_t *fnAnims;   // animations accepted per function type, ascending
    const int32_t *fnOffset;  // kFunctionSlots + 1 entries
    const CrudeRecord *crude;         // parallel to fnAnims
    const CrudeRecord *crudeByIndex;  // one per animation
    // Per function type and incoming velocity (slot fn * 4 + velocity), the records of the type
    // that pass its velocity rule, in list order; kFunctionSlots * 4 + 1 offsets.
    const CrudeRecord *crudeVelocity;
    const int32_t *crudeVelocityOffset;
    // The same lists prefiltered by the body rule of the function type for each allowed body
    // direction (slot (fn * 4 + velocity) * 6 + entry); kFunctionSlots * 4 * 6 + 1 offsets.
    const CrudeRecord *crudeBody;
    const int32_t *crudeBodyOffset;
    const float *cameraWeights;
    // The crude selection of idle movement in and out (IdleMovementAnimation), which reads
    // only the tables: one list for every call.
    const int16_t *idleMovement;
    int32_t idleMovementCount;
};

// The walk that GRF's time-to-target estimate takes from a moving player (ai_time.h:170-200):
// position, reach and optimistic reach after each 10 ms step while the acceleration bias grows
// below 1. It depends on the player's position, movement and speed, not on the target.
constexpr int kTimeWalkSteps = 70;
struct TimeWalk {
    float z;  // the walk moves in x and y only
    float x[kTimeWalkSteps], y[kTimeWalkSteps];
    float usual[kTimeWalkSteps], optimistic[kTimeWalkSteps];
    float usualSquared[kTimeWalkSteps], optimisticSquared[kTimeWalkSteps];
};
HD void Fatal(const char *reason);

// A small inline list (GRF's std::vector uses), capacity fixed.
template <class T, int N>
struct Small {
    int32_t count = 0;
    T e[N];
    HD int size() const { return count; }
    HD bool empty() const { return count == 0; }
    HD void clear() { count = 0; }
    HD void push_back(const T &x) {
        if (count >= N) Fatal("a fixed-capacity list outgrows its capacity");
        else e[count++] = x;
    }
    HD T &operator[](int i) { return e[i]; }
    HD const T &operator[](int i) const { return e[i]; }
    HD T *begin() { return e; }
    HD T *end() { return e + count; }
    HD const T *begin() const { return e; }
    HD const T *end() const { return e + count; }
    HD T &back() { return e[count - 1]; }
};
struct Aabb {
    Vec3 lo, hi;
    // GRF: the maximum starts at FLT_MIN / 100, just above zero, which collisions depend on.
    HD void Reset() {
        const float smallest = 1.17549435e-38f / 100, largest = 3.40282347e+38f / 100;
        lo = Vec3(largest, largest, largest);
        hi = Vec3(smallest, smallest, smallest);
    }
    // Grows the box to hold `p`, axis by axis (a zero bound keeps the sign it was first set with).
    HD void Hold(const Vec3 &p) {
        for (int k = 0; k < 3; k++) {
            if (p.v[k] < lo.v[k]) lo.v[k] = p.v[k];
            if (p.v[k] > hi.v[k]) hi.v[k] = p.v[k];
        }
    }
    // The box that holds this one turned by `r`: its eight corners turned, taken x fastest, then y,
    // then z.
    HDN Aabb Rotated(const Quat &r) const {
        Aabb b;
        b.Reset();
        for (int i = 0; i < 8; i++) b.Hold(r * Vec3((i & 1 ? hi : lo).v[0], (i & 2 ? hi : lo).v[1], (i & 4 ? hi : lo).v[2]));
        return b;
    }
    HD Aabb Translated(const Vec3 &o) const {
        Aabb b = *this;
        b.lo += o;
        b.hi += o;
        return b;
    }
    HDN bool Intersects(const Vec3 &center, float radius) const {
        float d2 = 0;
        for (int k = 0; k < 3; k++) {
            if (center.v[k] < lo.v[k]) {
                float d = center.v[k] - lo.v[k];
                d2 += d * d;
            } else if (center.v[k] > hi.v[k]) {
                float d = center.v[k] - hi.v[k];
                d2 += d * d;
            }
        }
        return d2 <= radius * radius;
    }
    // Each coordinate divides by 2 in double and rounds to float.
    HD Vec3 Center() const {
        float x = (lo.v[0] + hi.v[0]) / 2.0, y = (lo.v[1] + hi.v[1]) / 2.0, z = (lo.v[2] + hi.v[2]) / 2.0;
        return Vec3(x, y, z);
    }
    // Squares and roots in double (std::pow(float, int)), rounded to float twice.
    HD float Radius() const {
        float x = hi.v[0] - lo.v[0], y = hi.v[1] - lo.v[1], z = hi.v[2] - lo.v[2];
        float l = (float)sqrt((double)x * x + (double)y * y);
        return (float)(sqrt((double)l * l + (double)z * z) / 2.0);
    }
};
struct WorldGeometry {
    Aabb box;
    Vec3 position;
};
struct PlayerGeometry {
    bool footOrLowerLeg;
    WorldGeometry wg;
};
using PlayerGeometryList = Small<PlayerGeometry, kHumanoidNodes * 2>;

// Lists that the match's sequential code fills and reads within one call: an interruption's
// command queue, one force field of the AI or the referee, the bounces of the collision pass and
// the geometry of a tackler and its victim.
constexpr int kMaxCommands = 16;
using CommandQueue = Small<PlayerCommand, kMaxCommands>;
enum MagnetType { kAttract, kRepel };
enum DecayType { kDecayConstant, kDecayVariable };
struct ForceSpot {
    Vec3 origin;
    int32_t magnet = kAttract;
    int32_t decay = kDecayConstant;
    float exponent = 1.0f;
    float power = 0.0f;
    float scale = 0.0f;
};
using ForceField = Small<ForceSpot, 64>;
struct PlayerBounce {
    int32_t opponent;
    float force;
};
using PlayerBounceList = Small<PlayerBounce, kPlayers>;

// Lanes of one match with a plan of their own in the candidate search.
constexpr int kPlanLanes = kMaxGroupLanes;
static_assert(kGroupLanes <= kPlanLanes, "every lane of a match needs a candidate plan");

// A frame's terms of a movement plan that do not depend on the velocity it carries.
struct PlanFrame {
    Vec3 raw, unit;
    float stretchedSpeed, lean, rc, rs;
};

// Per-match working memory: the animation selection's candidate lists, planned positions, sort keys
// and one candidate plan per lane of the match, and the lists above. One block per environment in
// HBM, which every lane of the match addresses, in place of large per-lane stack arrays: the lanes
// run the code that fills the lists with the same data, so one copy serves the match. Each list is
// cleared where its use begins; none is live across a call that uses the same list.
struct Scratch {
    CommandQueue commands;
    ForceField forceField;
    PlayerBounceList bounces[kPlayers];
    PlayerGeometryList tackleGeometry[2];
    int16_t lists[3][kMaxAnimations];
    int32_t listCount[3];
    Vec3 plans[2][kAnimPositions];
    Vec3 lanePlans[kPlanLanes][kAnimPositions];
    TimeWalk walk;  // the match's sequential code
    double keys[kMaxAnimations];
    int16_t order[2][kMaxAnimations];
    SpatialState spatialAhead[kPlayers + 3];  // spatial states computed ahead: the players', then the officials'
    PlanFrame planFrames[kAnimPositions];     // a movement plan's frame terms, computed ahead
};

// Everything a match reads besides its world: the shared tables, its variant's static data and
// its scratch block.
struct Ctx {
    const Tables *t;
    const StaticData *sd;
    const Skeleton *skeletons;  // players then officials
    int32_t ticksPerStep;
    Scratch *ws;
    HD const Anim &A(int i) const { return t->anims[i]; }
    HD const AnimDerived &D(int i) const { return t->derived[i]; }
};

}  // namespace eng
