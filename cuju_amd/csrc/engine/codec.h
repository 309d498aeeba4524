// SPDX-License-Identifier: Apache-2.0
// Restates game logic of cuju (Copyright 2026 The cuju Authors), a reimplementation of Google
// Research Football (Copyright 2019 Google LLC); see NOTICE.
// Host-side codec between GRF's state bytes and a World. GRF's format is the raw little-endian
// bytes of each field, in the engine's object order (the order of
// src/environment_state.cpp:11-100 and include/cuju/state/environment_state.h), lists as an int32
// count then the elements. One visitor serves load and save, so a load followed by a save gives the
// input bytes back. A schema mode records each field's byte position and path for diffing.
#pragma once

#include <cstdio>
#include <cstdlib>
#include <stdexcept>
#include <string>
#include <vector>

#include "state.h"

namespace eng {
namespace codec {

struct SchemaEntry {
    size_t position;
    int size;
    std::string path;
};

class Archive {
public:
    explicit Archive(const std::string *input) : in_(input) {}
    bool loading() const { return in_ != nullptr; }
    const std::string &bytes() const { return out_; }
    size_t position() const { return pos_; }
    bool atEnd() const { return in_ && pos_ == in_->size(); }
    std::vector<SchemaEntry> *schema = nullptr;
    // Pointer fields seen during a load, checked against their collections afterwards.
    struct Pointer {
        int32_t value;
        int kind;
    };
    std::vector<Pointer> pointers;

    void push(const char *name) {
        if (schema) scope_.push_back(name);
    }
    void push(const char *name, int index) {
        if (schema) scope_.push_back(std::string(name) + "[" + std::to_string(index) + "]");
    }
    void pop() {
        if (schema) scope_.pop_back();
    }

    template <class T>
    void raw(T &v, const char *name) {
        if (schema) {
            std::string path;
            for (auto &s : scope_) path += s + ".";
            schema->push_back({pos_, (int)sizeof(T), path + name});
        }
        if (in_) {
            if (pos_ + sizeof(T) > in_->size()) throw std::runtime_error(std::string("state too short at ") + name);
            memcpy(&v, in_->data() + pos_, sizeof(T));
        } else {
            out_.append(reinterpret_cast<const char *>(&v), sizeof(T));
        }
        pos_ += sizeof(T);
    }
    enum { kPlayer, kTeam, kGamer, kKeyboard, kAnimation, kKinds };
    void ptr(int32_t &v, int kind, const char *name) {
        raw(v, name);
        if (in_) pointers.push_back({v, kind});
    }
    void str(std::string &s) {
        int32_t n = (int32_t)s.size();
        raw(n, "length");
        if (in_) {
            if (n < 0 || (size_t)n > in_->size() - pos_) throw std::runtime_error("state too short at a string");
            s.assign(in_->data() + pos_, n);
        } else {
            out_.append(s);
        }
        pos_ += n;
    }
    template <class T, int N, class F>
    void list(List<T, N> &l, const char *name, F each) {
        raw(l.count, name);
        if (l.count < 0 || l.count > N)
            throw std::runtime_error(std::string("capacity exceeded: ") + name);
        for (int i = 0; i < l.count; i++) {
            push(name, i);
            each(l.e[i]);
            pop();
        }
    }

private:
    const std::string *in_;
    std::string out_;
    size_t pos_ = 0;
    std::vector<std::string> scope_;
};

#define F(x) a.raw(x, #x)
#define P(x, k) a.ptr(x, Archive::k, #x)

inline void V(Archive &a, Radian &r, const char *n) { a.raw(r, n); }

inline void V(Archive &a, PlayerCommand &c) {
    F(c.desiredFunctionType);
    F(c.useDesiredMovement);
    F(c.desiredDirection);
    F(c.strictMovement);
    F(c.desiredVelocityFloat);
    F(c.useDesiredLookAt);
    F(c.desiredLookAt);
    F(c.useTouchInformation);
    TouchInformation &t = c.touchInfo;
    F(t.inputDirection);
    F(t.inputPower);
    F(t.autoDirectionBias);
    F(t.autoPowerBias);
    F(t.desiredDirection);
    F(t.desiredPower);
    P(t.targetPlayer, kPlayer);
    P(t.forcedTargetPlayer, kPlayer);
    F(c.onlyDeflectAnimationsThatPickupBall);
    F(c.useTripType);
    F(c.tripType);
    F(c.useDesiredTripDirection);
    F(c.desiredTripDirection);
    F(c.useSpecialVar1);
    F(c.specialVar1);
    F(c.useSpecialVar2);
    F(c.specialVar2);
    F(c.modifier);
}

inline void V(Archive &a, FormationEntry &f) {
    F(f.role);
    F(f.position);
    F(f.startPosition);
    F(f.lazy);
    F(f.controllable);
}

inline void V(Archive &a, BiasedOffset (&o)[kBodyParts]) {
    for (int i = 0; i < kBodyParts; i++) {
        a.push("offsets", i);
        F(o[i].orientation);
        F(o[i].bias);
        a.pop();
    }
}

inline void V(Archive &a, Humanoid &h) {
    for (int n = 0; n < kHumanoidNodes; n++) {
        a.push("nodes", n);
        F(h.nodes[n].position);
        F(h.nodes[n].rotation);
        F(h.nodes[n].scale);
        F(h.nodes[n].localMode);
        a.pop();
    }
    a.push("applyBuf");
    P(h.applyBuf.anim, kAnimation);
    F(h.applyBuf.frameNum);
    F(h.applyBuf.smooth);
    F(h.applyBuf.smoothFactor);
    F(h.applyBuf.noPos);
    F(h.applyBuf.position);
    F(h.applyBuf.orientation);
    V(a, h.applyBuf.offsets);
    a.pop();
    V(a, h.offsets);
    a.push("anim");
    AnimationState &s = h.anim;
    P(s.anim, kAnimation);
    F(s.id);
    F(s.frameNum);
    F(s.functionType);
    F(s.originatingInterrupt);
    F(s.actionSmuggle);
    F(s.actionSmuggleOffset);
    F(s.actionSmuggleSustain);
    F(s.actionSmuggleSustainOffset);
    F(s.movementSmuggle);
    F(s.movementSmuggleOffset);
    F(s.rotationSmuggleBegin);
    F(s.rotationSmuggleEnd);
    F(s.rotationSmuggleOffset);
    F(s.touchFrame);
    F(s.touchPos);
    F(s.incomingMovement);
    F(s.outgoingMovement);
    F(s.positionOffset);
    a.push("originatingCommand");
    V(a, s.originatingCommand);
    a.pop();
    a.list(s.positions, "positions", [&](Vec3 &p) { a.raw(p, "p"); });
    a.pop();
    F(h.prevAnimFrameNum);
    F(h.prevAnimFunctionType);
    F(h.startPos);
    F(h.startAngle);
    F(h.nextStartPos);
    F(h.nextStartAngle);
    a.push("spatial");
    SpatialState &p = h.spatial;
    F(p.position);
    F(p.angle);
    F(p.directionVec);
    F(p.velocityCat);
    F(p.floatVelocity);
    F(p.actualMovement);
    F(p.physicsMovement);
    F(p.animationMovement);
    F(p.movement);
    F(p.actionSmuggleMovement);
    F(p.movementSmuggleMovement);
    F(p.positionOffsetMovement);
    F(p.bodyAngle);
    F(p.bodyDirectionVec);
    F(p.relBodyAngleNonQuantized);
    F(p.relBodyAngle);
    F(p.relBodyDirectionVec);
    F(p.relBodyDirectionVecNonQuantized);
    F(p.foot);
    a.pop();
    F(h.prevPosition2D);
    F(h.interruptAnim);
    F(h.requeueDelayFrames);
    F(h.tripType);
    F(h.tripDirection);
    F(h.decayingPositionOffset);
    F(h.decayingDifficultyFactor);
    a.list(h.movementHistory, "movementHistory", [&](MovementHistoryEntry &m) {
        a.raw(m.position, "position");
        a.raw(m.orientation, "orientation");
        a.raw(m.timeDifferenceMs, "timeDifferenceMs");
        a.raw(m.nodeName, "nodeName");
    });
    F(h.mentalImageTime);
}

inline void V(Archive &a, PlayerControllerState &c) {
    P(c.player, kPlayer);
    F(c.inputDirection);
    F(c.inputVelocityFloat);
    P(c.team, kTeam);
    P(c.opponentTeam, kTeam);
    P(c.opponentPlayer, kPlayer);
    F(c.timeNeededMs);
    F(c.mentalImageTime);
    F(c.lastSwitchTimeMs);
    F(c.lastSwitchTimeDurationMs);
    F(c.hasPossession);
    F(c.hasUniquePossession);
    F(c.teamHasPossession);
    F(c.teamHasUniquePossession);
    F(c.oppTeamHasPossession);
    F(c.oppTeamHasUniquePossession);
    F(c.hasBestPossession);
    F(c.teamHasBestPossession);
    F(c.possessionAmount);
    F(c.teamPossessionAmount);
    F(c.fadingTeamPossessionAmount);
    F(c.oppTimeNeededToGetToBall);
    F(c.hasBestChanceOfPossession);
}

inline void V(Archive &a, KeyboardState &k) {
    F(k.mirror);
    F(k.direction);
    F(k.disabled);
    for (int b = 0; b < 11; b++) a.raw(k.buttons[b], "buttons");
}

// isActive, humanoid, [controller], externalController, ... as GRF interleaves them.
template <class C>
inline void VPerson(Archive &a, PersonBase &b, C controller) {
    F(b.isActive);
    a.push("humanoid");
    V(a, b.humanoid);
    a.pop();
    controller();
    P(b.externalController, kGamer);
    F(b.lastTouchTimeMs);
    F(b.lastTouchType);
    F(b.fatigueFactorInverse);
    a.list(b.positionHistoryPerSecond, "positionHistoryPerSecond", [&](Vec3 &v) { a.raw(v, "v"); });
}

inline void V(Archive &a, Player &p) {
    VPerson(a, p.base, [&] {
        if (!p.base.isActive) return;
        a.push("controller");
        V(a, p.controller.base);
        F(p.controller.ballBoundForGoal);
        F(p.controller.ballBoundForGoalY);
        F(p.controller.lastDesiredDirection);
        F(p.controller.lastDesiredVelocity);
        a.pop();
    });
    P(p.manMarking, kPlayer);
    V(a, p.dynamicFormationEntry);
    F(p.hasPossession);
    F(p.hasBestPossession);
    F(p.hasUniquePossession);
    F(p.possessionDurationMs);
    F(p.timeToBallMs);
    F(p.timeToBallOptimisticMs);
    F(p.timeToBallPreviousMs);
    F(p.triggerControlledBallCollision);
    F(p.tactical.forwardSpaceRating);
    F(p.tactical.toGoalSpaceRating);
    F(p.tactical.spaceRating);
    F(p.tactical.forwardRating);
    F(p.bufferNameCaptionShowCondition);
    F(p.bufferPlayerColor);
    F(p.desiredTimeToBallMs);
    F(p.cards);
    F(p.cardEffectiveTimeMs);
}

inline const char *TacticKey(int id) {
    static const char *const keys[kTacticKeys] = {
        "position_defense_depth_factor",           "position_defense_microfocus_strength",
        "position_defense_midfieldfocus",          "position_defense_midfieldfocus_strength",
        "position_defense_ownhalf_factor",         "position_defense_sidefocus_strength",
        "position_defense_width_factor",           "position_offense_depth_factor",
        "position_offense_microfocus_strength",    "position_offense_midfieldfocus",
        "position_offense_midfieldfocus_strength", "position_offense_ownhalf_factor",
        "position_offense_sidefocus_strength",     "position_offense_width_factor"};
    return keys[id];
}

// A map of keys to "%f" texts in key order; each text must reproduce itself from its float.
inline void V(Archive &a, Tactics &t) {
    int32_t n = 0;
    for (int i = 0; i < kTacticKeys; i++) n += (t.present >> i) & 1;
    a.raw(n, "properties");
    if (a.loading()) {
        if (n < 0 || n > kTacticKeys) throw std::runtime_error("properties: unexpected size");
        t.present = 0;
        for (int e = 0; e < n; e++) {
            std::string key, text;
            a.str(key);
            a.str(text);
            int id = 0;
            while (id < kTacticKeys && key != TacticKey(id)) id++;
            if (id == kTacticKeys) throw std::runtime_error("properties: unknown key " + key);
            char buf[32];
            snprintf(buf, sizeof(buf), "%f", (double)(float)atof(text.c_str()));
            if (text != buf) throw std::runtime_error("properties: value does not round-trip");
            t.present |= 1u << id;
            t.value[id] = (float)atof(text.c_str());
        }
    } else {
        for (int id = 0; id < kTacticKeys; id++) {
            if (!((t.present >> id) & 1)) continue;
            std::string key = TacticKey(id);
            char buf[32];
            snprintf(buf, sizeof(buf), "%f", (double)t.value[id]);
            std::string text = buf;
            a.str(key);
            a.str(text);
        }
    }
}

inline void V(Archive &a, Team &t) {
    F(t.hasPossession);
    F(t.timeToBallMs);
    P(t.designatedTeamPossessionPlayer, kPlayer);
    F(t.teamPossessionAmount);
    F(t.fadingTeamPossessionAmount);
    a.push("ai");
    TeamAI &c = t.ai;
    P(c.taker, kPlayer);
    F(c.setPieceType);
    V(a, c.baseTactics);
    V(a, c.liveTactics);
    F(c.offensivenessBias);
    F(c.teamHasPossession);
    F(c.teamHasUniquePossession);
    F(c.oppTeamHasPossession);
    F(c.oppTeamHasUniquePossession);
    F(c.teamHasBestPossession);
    F(c.teamPossessionAmount);
    F(c.fadingTeamPossessionAmount);
    F(c.timeNeededToGetToBall);
    F(c.oppTimeNeededToGetToBall);
    F(c.depth);
    F(c.width);
    F(c.offsideTrapX);
    F(c.endApplyAttackingRunMs);
    P(c.attackingRunPlayer, kPlayer);
    F(c.endApplyTeamPressureMs);
    P(c.teamPressurePlayer, kPlayer);
    F(c.endApplyKeeperRushMs);
    P(c.forwardSupportPlayer, kPlayer);
    a.list(c.tacticalOpponents, "tacticalOpponents", [&](TacticalOpponent &o) {
        a.ptr(o.player, Archive::kPlayer, "player");
        a.raw(o.dangerFactor, "dangerFactor");
    });
    a.pop();
    a.list(t.gamers, "gamers", [&](HumanGamer &g) {
        P(g.selectedPlayer, kPlayer);
        P(g.team, kTeam);
        P(g.keyboardIndex, kKeyboard);
        V(a, g.controller.base);
        V(a, g.controller.keyboard);
        F(g.controller.actionMode);
        F(g.controller.actionButton);
        F(g.controller.actionBufferTimeMs);
        F(g.controller.gaugeMs);
        F(g.controller.previousDirection);
        F(g.controller.steadyDirection);
        F(g.controller.lastSteadyDirectionSnapshotTimeMs);
    });
    a.list(t.switchPriority, "switchPriority", [&](int32_t &p) { a.raw(p, "p"); });
    P(t.lastTouchPlayer, kPlayer);
    P(t.mainSelectedPlayer, kPlayer);
}

inline void V(Archive &a, Scenario &s) {
    F(s.ballPosition);
    F(s.leftTeamSize);
    F(s.rightTeamSize);
    if (s.leftTeamSize < 0 || s.rightTeamSize < 0 || s.leftTeamSize > kTeamPlayers ||
        s.rightTeamSize > kTeamPlayers)
        throw std::runtime_error("the state holds a team size out of range");
    F(s.leftAgents);
    F(s.rightAgents);
    F(s.useMagnet);
    F(s.offsides);
    F(s.leftDifficulty);
    F(s.rightDifficulty);
    F(s.deterministic);
    F(s.endOnScore);
    F(s.endOnPossessionChange);
    F(s.endOnOutOfPlay);
    F(s.gameDuration);
    F(s.secondHalf);
    F(s.controlAllPlayers);
    F(s.realTime);
    F(s.gameEngineRandomSeed);
    F(s.reverseTeamProcessing);
    for (int i = 0; i < s.leftTeamSize; i++) {
        a.push("leftTeam", i);
        V(a, s.leftTeam[i]);
        a.pop();
    }
    for (int i = 0; i < s.rightTeamSize; i++) {
        a.push("rightTeam", i);
        V(a, s.rightTeam[i]);
        a.pop();
    }
}

inline void VScenarioHead(Archive &a, World &w) {
    F(w.gameState);
    F(w.waitingForGameCount);
    for (int i = 0; i < 2512; i++) a.raw(w.rng[i], "rng");
    a.push("scenario");
    V(a, w.scenario);
    a.pop();
}

inline void VWorld(Archive &a, World &w, int freeControllerCount) {
    VScenarioHead(a, w);
    MatchState &m = w.match;
    m.playerCount = w.scenario.leftTeamSize + w.scenario.rightTeamSize;
    if (w.scenario.leftTeamSize < 0 || w.scenario.rightTeamSize < 0 || m.playerCount > kPlayers)
        throw std::runtime_error("the state holds more players than a match holds");
    F(w.step);
    a.push("match");
    F(m.firstTeam);
    F(m.secondTeam);
    a.list(m.mentalImages, "mentalImages", [&](MentalImage &im) {
        a.raw(im.timeStampMs, "timeStampMs");
        a.raw(im.maxDistanceDeviation, "maxDistanceDeviation");
        a.raw(im.maxMovementDeviation, "maxMovementDeviation");
        a.list(im.players, "players", [&](PlayerImage &p) {
            a.raw(p.position, "position");
            a.raw(p.directionVector, "directionVector");
            a.raw(p.movement, "movement");
            a.ptr(p.player, Archive::kPlayer, "player");
            a.raw(p.velocity, "velocity");
            a.raw(p.role, "role");
        });
        a.list(im.ballPredictions, "ballPredictions", [&](Vec3 &v) { a.raw(v, "v"); });
    });
    for (int t = 0; t < 2; t++) {
        a.push("teams", t);
        V(a, m.teams[t]);
        a.pop();
    }
    for (int p = 0; p < m.playerCount; p++) {
        a.push("players", p);
        V(a, m.players[p]);
        a.pop();
    }
    F(m.goalCount[0]);
    F(m.goalCount[1]);
    F(m.possessionLastMinute);
    for (int o = 0; o < 3; o++) {
        a.push("officials", o);
        VPerson(a, m.officials[o], [] {});
        a.pop();
    }
    const int keyboards = m.teams[0].gamers.count + m.teams[1].gamers.count;
    if (keyboards > kControllers) throw std::runtime_error("too many keyboards");
    for (int k = 0; k < keyboards; k++) {
        a.push("secondKeyboardCopies", k);
        V(a, m.secondKeyboardCopies[k]);
        a.pop();
    }
    m.freeControllerCount = freeControllerCount;
    for (int k = 0; k < freeControllerCount; k++) {
        a.push("freeControllers", k);
        V(a, m.freeControllers[k]);
        a.pop();
    }
    a.push("ball");
    Ball &b = m.ball;
    F(b.momentum);
    F(b.rotationPerMs);
    for (int i = 0; i < 401; i++) a.raw(b.predictions[i], "predictions");
    F(b.validPredictions);
    F(b.orientationPrediction);
    a.list(b.positionHistory, "positionHistory", [&](Vec3 &v) { a.raw(v, "v"); });
    F(b.positionBuffer);
    F(b.orientationBuffer);
    F(b.touchesNet);
    a.pop();
    F(m.matchTimeMs);
    F(m.actualTimeMs);
    F(m.goalScoredTimer);
    F(m.matchPhase);
    F(m.inPlay);
    F(m.inSetPiece);
    F(m.goalScored);
    F(m.ballIsInGoal);
    P(m.lastGoalTeam, kTeam);
    P(m.lastGoalScorer, kPlayer);
    for (int i = 0; i < 4; i++) a.raw(m.lastTouchTeamIDs[i], "lastTouchTeamIDs");
    F(m.lastTouchTeamID);
    P(m.bestPossessionTeam, kTeam);
    P(m.designatedPossessionPlayer, kPlayer);
    P(m.ballRetainer, kPlayer);
    F(m.possessionSideHistoryMaxTimeMs);
    a.list(m.possessionSideHistory, "possessionSideHistory", [&](float &v) { a.raw(v, "v"); });
    F(m.autoUpdateInGameCamera);
    F(m.cameraOrientation);
    F(m.cameraNodeOrientation);
    F(m.cameraNodePosition);
    F(m.cameraFov);
    F(m.cameraNearCap);
    F(m.cameraFarCap);
    a.list(m.cameraPosition, "cameraPosition", [&](Vec3 &v) { a.raw(v, "v"); });
    F(m.lastBodyBallCollisionTimeMs);
    a.push("referee");
    Referee &r = m.referee;
    F(r.buffer.active);
    F(r.buffer.desiredSetPiece);
    F(r.buffer.teamID);
    P(r.buffer.setPieceTeam, kTeam);
    F(r.buffer.stopTime);
    F(r.buffer.prepareTime);
    F(r.buffer.startTime);
    F(r.buffer.restartPos);
    P(r.buffer.taker, kPlayer);
    F(r.buffer.endPhase);
    F(r.afterSetPieceRelaxTimeMs);
    a.list(r.offsidePlayers, "offsidePlayers", [&](int32_t &v) { a.raw(v, "v"); });
    P(r.foul.foulPlayer, kPlayer);
    P(r.foul.foulVictim, kPlayer);
    F(r.foul.foulType);
    F(r.foul.advantage);
    F(r.foul.foulTime);
    F(r.foul.foulPosition);
    F(r.foul.hasBeenProcessed);
    a.pop();
    a.pop();
}

#undef F
#undef P

}  // namespace codec
}  // namespace eng
