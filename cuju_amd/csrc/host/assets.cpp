// SPDX-License-Identifier: Apache-2.0
// Restates game logic of cuju (Copyright 2026 The cuju Authors), a reimplementation of Google
// Research Football (Copyright 2019 Google LLC); see NOTICE.
// Host loaders. Formats: include/cuju/animation/animation_data.h:210-307 (CUJANIM1),
// include/cuju/animation/skeleton.h:41-85 (CUJHUM1), include/cuju/simulation/static_data.h:72-105,
// include/cuju/batch/batch_core.h:660-752 (CUJASSET1). Derived values:
// include/cuju/animation/animation_derived.h:102-166, include/cuju/animation/keyframes.h:126-160,
// include/cuju/batch/tables.h:25-90 and the record builders of
// include/cuju/simulation/select_animation.h:449-565. Codec: include/cuju/simulation/state_io.h,
// agents: include/cuju/batch/agent_setup.h:15-164.
#include "assets.h"

#include <cmath>
#include <cstdlib>
#include <fstream>
#include <map>
#include <sstream>
#include <stdexcept>

namespace eng {

// Host fault hooks of the engine.
const char *&FailReason() {
    thread_local const char *reason = "";
    return reason;
}
void FatalHost(const char *message) { throw std::runtime_error(std::string("engine: ") + message); }

namespace host {

std::string ReadFile(const std::string &path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open " + path);
    std::stringstream s;
    s << f.rdbuf();
    return s.str();
}

namespace {

// Little-endian cursor over a byte string.
class Reader {
public:
    Reader(const std::string &b, const char *what, size_t at) : b_(b), what_(what), at_(at) {}
    template <class T>
    T get() {
        if (at_ + sizeof(T) > b_.size()) throw std::runtime_error(std::string(what_) + " end early");
        T v;
        memcpy(&v, b_.data() + at_, sizeof(T));
        at_ += sizeof(T);
        return v;
    }
    std::string str() {
        const int32_t n = get<int32_t>();
        if (n < 0 || at_ + (size_t)n > b_.size()) throw std::runtime_error(std::string("a string of ") + what_ + " runs past the end");
        std::string s = b_.substr(at_, n);
        at_ += n;
        return s;
    }
    bool end() const { return at_ == b_.size(); }

private:
    const std::string &b_;
    const char *what_;
    size_t at_;
};

int StateStringId(const std::string &s) {
    static const char *const known[5] = {"", "lay_back", "lay_front", "left_elbow", "right_elbow"};
    for (int i = 0; i < 5; i++)
        if (s == known[i]) return i;
    throw std::runtime_error("unknown state string `" + s + "` in the animation tables");
}
int BodyPartId(const std::string &s) {
    static const char *const names[14] = {"middle",     "neck",          "left_thigh",     "right_thigh", "left_knee",
                                          "right_knee", "left_ankle",    "right_ankle",    "left_shoulder",
                                          "right_shoulder", "left_elbow", "right_elbow", "body", "player"};
    for (int i = 0; i < 14; i++)
        if (s == names[i]) return i;
    return -1;
}
// "x,y,z" with the C library's atof per component, missing components 0.
Vec3 ParseVector(const std::string &s) {
    Vec3 r(0.0f);
    if (s.empty()) return r;
    std::vector<std::string> tok;
    size_t start = s.find_first_not_of(',');
    while (start != std::string::npos) {
        size_t end = s.find_first_of(',', start);
        tok.push_back(s.substr(start, end == std::string::npos ? std::string::npos : end - start));
        start = end == std::string::npos ? end : s.find_first_not_of(',', end);
    }
    if (tok.empty()) throw std::runtime_error("an empty vector in the animation variables");
    for (size_t i = 0; i < tok.size() && i < 3; i++) r.v[i] = (float)atof(tok[i].c_str());
    return r;
}

struct Parsed {
    std::vector<std::map<std::string, std::string>> variables;
};

void ParseAnimations(const std::string &bytes, AnimationTables &t, Parsed &p) {
    if (bytes.compare(0, 8, "CUJANIM1") != 0) throw std::runtime_error("expected the animation tables");
    Reader r(bytes, "the animation tables", 8);
    const int32_t n = r.get<int32_t>();
    if (n < 0 || n > kMaxAnimations) throw std::runtime_error("too many animations");
    t.anims.resize(n);
    p.variables.resize(n);
    for (int i = 0; i < n; i++) {
        Anim &a = t.anims[i];
        r.str();  // name
        a.frameCount = r.get<int32_t>();
        a.currentFoot = r.get<int32_t>();
        a.animationType = r.get<int32_t>();
        a.translation = r.get<Vec3>();
        a.incomingMovement = r.get<Vec3>();
        a.incomingVelocity = r.get<float>();
        a.outgoingMovement = r.get<Vec3>();
        a.outgoingDirection = r.get<Vec3>();
        a.incomingBodyDirection = r.get<Vec3>();
        a.outgoingBodyDirection = r.get<Vec3>();
        a.outgoingVelocity = r.get<float>();
        a.outgoingAngle = r.get<Radian>();
        a.incomingBodyAngle = r.get<Radian>();
        a.outgoingBodyAngle = r.get<Radian>();
        a.outgoingFoot = r.get<int32_t>();
        a.idleLevel = r.get<float>();
        a.quadrantID = r.get<int32_t>();
        a.specialVar1 = r.get<float>();
        a.specialVar2 = r.get<float>();
        a.lastDitch = r.get<uint8_t>() != 0;
        a.baseAnimation = r.get<uint8_t>() != 0;
        a.outgoingSpecialState = StateStringId(r.str());
        a.incomingRetainState = StateStringId(r.str());
        a.incomingSpecialState = StateStringId(r.str());
        const int32_t vars = r.get<int32_t>();
        for (int v = 0; v < vars; v++) {
            std::string k = r.str();
            p.variables[i][k] = r.str();
        }
        const int32_t nodes = r.get<int32_t>();
        a.nodeFirst = (int32_t)t.nodes.size();
        a.nodeCount = nodes;
        for (int b = 0; b < kBodyParts; b++) a.nodeOfBodyPart[b] = -1;
        for (int k = 0; k < nodes; k++) {
            NodeAnim na{};
            na.bodyPart = r.get<int32_t>();
            if (na.bodyPart < 0 || na.bodyPart >= kBodyParts) throw std::runtime_error("bad body part in the animation tables");
            for (int e = a.nodeFirst; e < (int)t.nodes.size(); e++)
                if (t.nodes[e].bodyPart == na.bodyPart) throw std::runtime_error("an animation repeats a body part");
            a.nodeOfBodyPart[na.bodyPart] = (int8_t)k;
            const int32_t keys = r.get<int32_t>();
            na.keyFirst = (int32_t)t.keys.size();
            na.keyCount = keys;
            for (int q = 0; q < keys; q++) {
                KeyFrame kf;
                kf.frame = r.get<int32_t>();
                kf.orientation = r.get<Quat>();
                kf.position = r.get<Vec3>();
                t.keys.push_back(kf);
            }
            t.nodes.push_back(na);
        }
        a.hasFootball = r.get<int32_t>() != 0;
        a.footballFirst = (int32_t)t.football.size();
        a.footballCount = 0;
        if (a.hasFootball) {
            const int32_t fk = r.get<int32_t>();
            a.footballCount = fk;
            for (int q = 0; q < fk; q++) {
                FootballKey f;
                f.frame = r.get<int32_t>();
                f.orientation = r.get<Quat>();
                f.position = r.get<Vec3>();
                f.power = r.get<float>();
                t.football.push_back(f);
            }
        }
        const int32_t pc = r.get<int32_t>();
        a.hasPositions = pc >= 0;
        a.posFirst = (int32_t)t.positions.size();
        a.posCount = pc > 0 ? pc : 0;
        if (a.posCount > kAnimPositions) throw std::runtime_error("an animation holds too many positions");
        for (int q = 0; q < pc; q++) t.positions.push_back(r.get<Vec3>());
    }
    const int32_t nq = r.get<int32_t>();
    t.quadrants.resize(nq);
    for (Quadrant &q : t.quadrants) {
        q.id = r.get<int32_t>();
        q.position = r.get<Vec3>();
        q.velocity = r.get<int32_t>();
        q.angle = r.get<Radian>();
    }
    t.maxIncomingBallDeviation = r.get<Radian>();
    t.maxOutgoingBallDeviation = r.get<Radian>();
    if (!r.end()) throw std::runtime_error("the animation tables hold bytes after their end");
}

// The poses of frames 0..frameCount+1 of every node, and the halfway blends between them.
void BuildInterpolation(AnimationTables &t) {
    size_t total = 0;
    for (const Anim &a : t.anims) total += (size_t)a.nodeCount * (a.frameCount + 2);
    t.interp.assign(total, InterpEntry{});
    t.middle.assign(total, MiddleEntry{});
    size_t base = 0;
    for (const Anim &a : t.anims) {
        const int frames = a.frameCount + 2, stride = a.nodeCount;
        for (int k = 0; k < a.nodeCount; k++) {
            NodeAnim &na = t.nodes[a.nodeFirst + k];
            const size_t off = base + (size_t)k;
            for (int f = 0; f < frames; f++) {
                InterpEntry &e = t.interp[off + (size_t)f * stride];
                ComputeInterpolated(a, t.keys.data() + na.keyFirst, na.keyCount, f, e.orientation, e.position);
                float x, y;
                e.orientation.Angles(x, y, e.angleZ);
            }
            for (int f = 0; f + 1 < frames; f++) {
                const InterpEntry &at = t.interp[off + (size_t)f * stride], &nx = t.interp[off + (size_t)(f + 1) * stride];
                MiddleEntry &m = t.middle[off + (size_t)f * stride];
                BlendFrames(at.orientation, at.position, nx.orientation, nx.position, 0.5f, m.orientation, m.position);
                m.normalized = m.orientation.Normalized();
                const float sq = m.orientation.SquaredMagnitude();
                m.normalizedKeepsZeros = sq >= 0.000001f && sq < 2.0f;
            }
            na.interpFirst = (int32_t)off;
            na.interpFrames = frames;
            na.interpStride = stride;
        }
        base += (size_t)a.nodeCount * frames;
    }
}

// Values GRF parses from the text variables at every use; the host's atof/atoi parse them once.
void BuildDerived(AnimationTables &t, const Parsed &p) {
    t.derived.resize(t.anims.size());
    for (size_t i = 0; i < t.anims.size(); i++) {
        auto var = [&](const char *k) {
            auto it = p.variables[i].find(k);
            return it == p.variables[i].end() ? std::string() : it->second;
        };
        const Anim &a = t.anims[i];
        AnimDerived &d = t.derived[i];
        d.priorityAbsolute = fabs(atof(var("priority").c_str()));
        d.touchFrame = atoi(var("touchframe").c_str());
        d.difficultyFactor = (float)atof(var("animdifficultyfactor").c_str());
        d.tripTypeIsOne = var("triptype") == "1";
        d.tripTypeRounded = (int)round(atof(var("triptype").c_str()));
        d.bumpDirection = ParseVector(var("bumpdirection"));
        d.incomingBallDirection = ParseVector(var("incomingballdirection"));
        d.ballDirection = ParseVector(var("balldirection"));
        d.incomingMaxDeviation = (float)fabs(atof(var("incomingballdirection_maxdeviation").c_str()) * PI);
        d.outgoingMaxDeviation = (float)fabs(atof(var("outgoingballdirection_maxdeviation").c_str()) * PI);
        const std::string outRetain = var("outgoing_retain_state"), inRetain = var("incoming_retain_state");
        d.outgoingRetainRawValue = StateStringId(outRetain);
        d.outgoingRetainRaw = !outRetain.empty();
        d.incomingRetainRawValue = StateStringId(inRetain);
        d.outgoingRetainBodyPart = outRetain.empty() ? -1 : BodyPartId(outRetain);
        d.incomingRetainBodyPart = inRetain.empty() ? -1 : BodyPartId(inRetain);
        const std::string forced = var("forcedfoot");
        d.forcedFootWhich = forced == "strong" ? 1 : forced == "weak" ? 2 : 0;
        d.touchFootLeft = var("touchfoot") == "left";
        const std::string touchPart = var("touch_bodypart");
        d.touchType = (touchPart.find("foot") != std::string::npos || touchPart.find("lowerleg") != std::string::npos) ? 0 : 1;
        d.touchMaxPowerFactor = (float)atof(var("touch_maxpowerfactor").c_str());
        d.touchDifficultyFactor = (float)atof(var("touch_difficultyfactor").c_str());
        d.crudeOutDirectionRotated = a.outgoingDirection.Rotated2D(a.outgoingBodyAngle.value());
        d.crudeTurnAngle = d.crudeOutDirectionRotated.Angle2D(a.incomingBodyDirection);
        d.crudeInBodyFixAbsolute = fabsf(FixAngle(a.incomingBodyDirection.Angle2D()));
        d.crudeOutBodyDirection = Vec3(0, -1, 0).Rotated2D(a.outgoingBodyAngle.value() + a.outgoingAngle.value());
        d.crudeInBallNonzero = d.incomingBallDirection.Length() != 0.0f;
        d.crudeInBallAdapted = d.incomingBallDirection;
        d.crudeInBallAdapted.v[2] *= 0.4f;
        if (d.crudeInBallNonzero) d.crudeInBallAdapted.Normalize();
        d.crudeBallDirectionNormalized = d.ballDirection;
        d.crudeBallDirectionNormalized.Normalize(Vec3(0));
    }
}

void BuildSelection(AnimationTables &t) {
    t.selection.resize(t.anims.size());
    t.smoothed.assign(t.positions.size(), Vec3());
    for (size_t i = 0; i < t.anims.size(); i++) {
        const Anim &a = t.anims[i];
        const AnimDerived &d = t.derived[i];
        SelectionRecord &s = t.selection[i];
        s = SelectionRecord{};
        for (int k = 0; k < 6; k++) s.incomingBodyAngles[k] = a.incomingBodyDirection.Angle2D(AllowedBodyDir(k));
        s.bodyTurnAngle = a.incomingBodyDirection.Angle2D(d.crudeOutBodyDirection);
        s.incomingBodyIndex = BodyDirectionIndex(a.incomingBodyDirection);
        s.preferredOutgoingDirection = SnapToPreferredDirection(a.outgoingDirection);
        s.preferredOutgoingMovement = s.preferredOutgoingDirection * RangeVelocity(a.outgoingVelocity);
        s.preferredOutgoingAngle = SnapToPreferredAngle(a.outgoingAngle.value());
        s.lookAngle = SnapToBodyAngle(a.outgoingBodyAngle.value()) + s.preferredOutgoingAngle;
        s.smoothedFirst = a.posCount >= 2 ? a.posFirst : -1;
        const Vec3 &bd = d.crudeBallDirectionNormalized;
        s.ballDirectionFinite = std::isfinite(bd.v[0]) && std::isfinite(bd.v[1]) && std::isfinite(bd.v[2]);
        if (s.smoothedFirst >= 0)
            for (uint32_t f = 0; f < (uint32_t)a.posCount; f++)
                t.smoothed[a.posFirst + f] = MovementAtFrame(t.positions.data() + a.posFirst, a.posCount, f, 1);
    }
    t.fnAnims.clear();
    t.fnOffset.assign(kFunctionSlots + 1, 0);
    for (int fn = 0; fn < kFunctionSlots; fn++) {
        t.fnOffset[fn] = (int32_t)t.fnAnims.size();
        for (int i = 0; i < (int)t.anims.size(); i++)
            if (CheckFunctionType(t.anims[i].animationType, fn)) t.fnAnims.push_back((int16_t)i);
    }
    t.fnOffset[kFunctionSlots] = (int32_t)t.fnAnims.size();
    auto small = [](int v, int lo, int hi, const char *what) {
        if (v < lo || v > hi) throw std::runtime_error(std::string("animation tables: a crude record cannot hold ") + what);
        return v;
    };
    t.crudeByIndex.assign(t.anims.size(), CrudeRecord{});
    for (size_t i = 0; i < t.anims.size(); i++) {
        const Anim &a = t.anims[i];
        const AnimDerived &d = t.derived[i];
        const SelectionRecord &sr = t.selection[i];
        CrudeRecord &r = t.crudeByIndex[i];
        r.incomingBodyDirection = a.incomingBodyDirection;
        r.outDirectionRotated = d.crudeOutDirectionRotated;
        r.inBallAdapted = d.crudeInBallAdapted;
        r.ballDirectionNormalized = d.crudeBallDirectionNormalized;
        r.incomingVelocity = a.incomingVelocity;
        r.outgoingVelocity = a.outgoingVelocity;
        r.turnAngle = d.crudeTurnAngle;
        r.inBodyFixAbsolute = d.crudeInBodyFixAbsolute;
        for (int j = 0; j < 6; j++) r.incomingBodyAngles[j] = sr.incomingBodyAngles[j];
        r.bodyTurnAngle = sr.bodyTurnAngle;
        r.incomingMaxDeviation = d.incomingMaxDeviation;
        r.outgoingMaxDeviation = d.outgoingMaxDeviation;
        r.specialVar1 = a.specialVar1;
        r.specialVar2 = a.specialVar2;
        r.index = (int16_t)small((int)i, 0, 32767, "the animation index");
        r.animationType = (int16_t)small(a.animationType, -32768, 32767, "the animation type");
        r.incomingSpecialState = (int16_t)small(a.incomingSpecialState, -32768, 32767, "the special state");
        r.incomingRetainState = (int16_t)small(a.incomingRetainState, -32768, 32767, "the retain state");
        r.tripTypeRounded = (int16_t)small(d.tripTypeRounded, -32768, 32767, "the trip type");
        r.forcedFootWhich = (int8_t)small(d.forcedFootWhich, -128, 127, "the forced foot");
        r.currentFoot = (int8_t)small(a.currentFoot, -128, 127, "the current foot");
        r.flags = (uint8_t)((d.outgoingRetainRaw ? 1 : 0) | (a.lastDitch ? 2 : 0) | (d.crudeInBallNonzero ? 4 : 0) |
                            (sr.ballDirectionFinite ? 8 : 0) | (d.touchFootLeft ? 16 : 0));
    }
    t.crude.clear();
    for (int16_t i : t.fnAnims) t.crude.push_back(t.crudeByIndex[i]);
    t.crudeVelocity.clear();
    t.crudeVelocityOffset.assign(kFunctionSlots * 4 + 1, 0);
    for (int fn = 0; fn < kFunctionSlots; fn++)
        for (int v = kVelIdle; v <= kVelSprint; v++) {
            t.crudeVelocityOffset[fn * 4 + v] = (int32_t)t.crudeVelocity.size();
            const CrudeQuery q = VelocityRuleQuery(fn, v);
            for (int j = t.fnOffset[fn]; j < t.fnOffset[fn + 1]; j++)
                if (IncomingVelocityPasses(q, t.crude[j].incomingVelocity, t.crude[j].outgoingVelocity))
                    t.crudeVelocity.push_back(t.crude[j]);
        }
    t.crudeVelocityOffset[kFunctionSlots * 4] = (int32_t)t.crudeVelocity.size();
    t.crudeBody.clear();
    t.crudeBodyOffset.assign(kFunctionSlots * 4 * kBodyEntries + 1, 0);
    for (int slot = 0; slot < kFunctionSlots * 4; slot++) {
        const int fn = slot / 4, v = slot % 4;
        const BodyRule rule = FunctionBodyRule(fn);
        for (int e = 0; e < kBodyEntries; e++) {
            t.crudeBodyOffset[slot * kBodyEntries + e] = (int32_t)t.crudeBody.size();
            for (int j = t.crudeVelocityOffset[slot]; j < t.crudeVelocityOffset[slot + 1]; j++) {
                const CrudeRecord &r = t.crudeVelocity[j];
                // An idle query velocity turns the body test off (FilterAnimations, byBody).
                if (v == kVelIdle || IncomingBodyPasses(rule, e, AllowedBodyDir(e), AllowedBodyFixAbsolute(e),
                                                        AllowedBodyIdleAbsolute(e), r))
                    t.crudeBody.push_back(r);
            }
        }
    }
    t.crudeBodyOffset[kFunctionSlots * 4 * kBodyEntries] = (int32_t)t.crudeBody.size();
    t.cameraWeights.assign(kCameraWeights, 0.0f);
    for (int n = 1; n <= kCameraHistory; n++)
        for (int i = 0; i < n; i++) t.cameraWeights[n * (n - 1) / 2 + i] = CameraWeight(i, n);
}

}  // namespace

std::vector<Skeleton> ParseSkeletons(const std::string &bytes) {
    if (bytes.compare(0, 7, "CUJHUM1") != 0) throw std::runtime_error("expected the skeletons of a bundle");
    Reader r(bytes, "the skeletons", 7);
    const int32_t n = r.get<int32_t>();
    if (n < 0 || n > kStaticEntries) throw std::runtime_error("too many skeletons");
    std::vector<Skeleton> out(n);
    for (Skeleton &s : out) {
        memset(&s, 0, sizeof(Skeleton));
        for (int b = 0; b < kBodyParts; b++) s.nodeMap[b] = r.get<int32_t>();
        s.nodeCount = r.get<int32_t>();
        if (s.nodeCount < 0 || s.nodeCount > kHumanoidNodes) throw std::runtime_error("too many skeleton nodes");
        for (int k = 0; k < s.nodeCount; k++) {
            SkelNode &node = s.nodes[k];
            r.str();
            node.parent = r.get<int32_t>();
            node.localMode = r.get<int32_t>();
            node.position = r.get<Vec3>();
            node.rotation = r.get<Quat>();
            node.scale = r.get<Vec3>();
            node.geometryCount = r.get<int32_t>();
            if (node.geometryCount < 0 || node.geometryCount > 2) throw std::runtime_error("too many geometries");
            for (int g = 0; g < node.geometryCount; g++) {
                SkelGeometry &geo = node.geometries[g];
                const std::string name = r.str();
                geo.footOrLowerLeg = name == "left_foot" || name == "right_foot" || name == "left_lowerleg" || name == "right_lowerleg";
                geo.localMode = r.get<int32_t>();
                geo.position = r.get<Vec3>();
                geo.rotation = r.get<Quat>();
                geo.scale = r.get<Vec3>();
                geo.boxMin = r.get<Vec3>();
                geo.boxMax = r.get<Vec3>();
            }
        }
        for (int b = 0; b < kBodyParts; b++)
            if (s.nodeMap[b] < -1 || s.nodeMap[b] >= s.nodeCount) throw std::runtime_error("a skeleton maps a body part outside its nodes");
    }
    if (!r.end()) throw std::runtime_error("the skeletons hold bytes after their end");
    return out;
}

// An int32 count, the PlayerData of each entry (players in state order, then the three
// officials), then sections FORM (each player's formation), MDUR and SIDS.
StaticData ParseStatic(const std::string &b) {
    static_assert(sizeof(PlayerData) == 100, "player data layout");
    StaticData sd;
    memset(&sd, 0, sizeof(sd));
    sd.matchDurationFactor = 0x1.c5d638p-5f;
    if (b.size() < 4) throw std::runtime_error("static data: too short");
    memcpy(&sd.count, b.data(), 4);
    size_t off = 4 + (size_t)sd.count * sizeof(PlayerData);
    if (sd.count < 3 || sd.count > kStaticEntries || b.size() < off) throw std::runtime_error("static data: bad size");
    memcpy(sd.data, b.data() + 4, sd.count * sizeof(PlayerData));
    const int players = sd.count - 3;
    const size_t entry = 4 + 12 + 12 + 1 + 1;
    if (b.compare(off, 4, "FORM") != 0 || b.size() < off + 4 + players * entry) throw std::runtime_error("static data: bad formation section");
    off += 4;
    for (int p = 0; p < players; p++) {
        StaticFormation &f = sd.formation[p];
        memcpy(&f.role, &b[off], 4);
        memcpy(&f.position, &b[off + 4], 12);
        memcpy(&f.startPosition, &b[off + 16], 12);
        f.lazy = b[off + 28] != 0;
        f.controllable = b[off + 29] != 0;
        off += entry;
    }
    if (b.compare(off, 4, "MDUR") != 0 || b.size() < off + 8) throw std::runtime_error("static data: bad duration section");
    memcpy(&sd.matchDurationFactor, &b[off + 4], 4);
    off += 8;
    if (b.compare(off, 4, "SIDS") != 0 || b.size() != off + 4 + (size_t)sd.count * 4) throw std::runtime_error("static data: bad stable ID section");
    memcpy(sd.stableID, &b[off + 4], (size_t)sd.count * 4);
    return sd;
}

std::string ScenarioKey(const World &w) {
    Scenario s = w.scenario;
    s.gameEngineRandomSeed = 0;
    s.leftDifficulty = 0;
    s.rightDifficulty = 0;
    codec::Archive a(nullptr);
    codec::V(a, s);
    return a.bytes();
}


Tables AnimationTables::View() const {
    Tables t{};
    t.anims = anims.data();
    t.animCount = (int32_t)anims.size();
    t.nodes = nodes.data();
    t.keys = keys.data();
    t.interp = interp.data();
    t.middle = middle.data();
    t.football = football.data();
    t.positions = positions.data();
    t.quadrants = quadrants.data();
    t.quadrantCount = (int32_t)quadrants.size();
    t.maxIncomingBallDeviation = maxIncomingBallDeviation;
    t.maxOutgoingBallDeviation = maxOutgoingBallDeviation;
    t.derived = derived.data();
    t.selection = selection.data();
    t.smoothed = smoothed.data();
    t.fnAnims = fnAnims.data();
    t.fnOffset = fnOffset.data();
    t.crude = crude.data();
    t.crudeByIndex = crudeByIndex.data();
    t.crudeVelocity = crudeVelocity.data();
    t.crudeVelocityOffset = crudeVelocityOffset.data();
    t.crudeBody = crudeBody.data();
    t.crudeBodyOffset = crudeBodyOffset.data();
    t.cameraWeights = cameraWeights.data();
    t.idleMovement = idleMovement.data();
    t.idleMovementCount = (int32_t)idleMovement.size();
    return t;
}

std::unique_ptr<AnimationTables> LoadAnimationTables(const std::string &path) {
    auto t = std::make_unique<AnimationTables>();
    Parsed p;
    ParseAnimations(ReadFile(path), *t, p);
    BuildInterpolation(*t);
    BuildDerived(*t, p);
    BuildSelection(*t);
    {
        // The idle-movement candidates: the idle query has fixed inputs, so its crude selection
        // runs once here instead of at every idle request.
        const Tables view = t->View();
        auto scratch = std::make_unique<Scratch>();
        Ctx c{};
        c.t = &view;
        c.ws = scratch.get();
        AList idle{scratch->lists[1], 0};
        FilterAnimations(c, IdleMovementQuery(), idle);
        if (idle.count < 1) throw std::invalid_argument("expected animations of idle movement");
        t->idleMovement.assign(idle.e, idle.e + idle.count);
    }
    return t;
}

void ResetWorld(World &w) {
    memset(static_cast<void *>(&w), 0, sizeof(World));
    w.flags.teamSide[0] = w.flags.teamSide[1] = -1;
}

bool StateCodec::Load(const std::string &bytes, World &w) {
    auto tryLoad = [&](int fc) {
        try {
            codec::Archive a(&bytes);
            codec::VWorld(a, w, fc);
            if (!a.atEnd()) return false;
            const MatchState &m = w.match;
            const int sizes[codec::Archive::kKinds] = {m.playerCount, 2, m.teams[0].gamers.count + m.teams[1].gamers.count,
                                                       kMatchKeyboards, animationCount};
            for (const auto &p : a.pointers)
                if (sizes[p.kind] >= 0 && (p.value < -1 || p.value >= sizes[p.kind])) return false;
            return true;
        } catch (const std::exception &) {
            return false;
        }
    };
    if (freeControllerCount >= 0 && tryLoad(freeControllerCount)) return true;
    for (int fc = 0; fc <= kControllers; fc++) {
        ResetWorld(w);
        if (tryLoad(fc)) {
            freeControllerCount = fc;
            return true;
        }
    }
    return false;
}
std::string StateCodec::Save(World &w, std::vector<codec::SchemaEntry> *schema) {
    BallMaterialize(w.match.ball);
    for (int i = 0; i < w.match.mentalImages.count; i++) MentalMaterialize(w, w.match.mentalImages[i]);
    codec::Archive a(nullptr);
    a.schema = schema;
    codec::VWorld(a, w, freeControllerCount);
    return a.bytes();
}
bool StateCodec::LoadFrame(const std::string &bytes, int mirror, World &w) {
    ResetWorld(w);
    if (!Load(bytes, w)) return false;
    InitializePlayerTeams(w);
    CanonicalToRest(w);
    MirrorMatch(w, mirror & 1, mirror & 2, mirror & 4);
    return true;
}
std::string StateCodec::SaveFrame(World &w, int mirror, std::vector<codec::SchemaEntry> *schema) {
    MirrorMatch(w, mirror & 1, mirror & 2, mirror & 4);
    RestToCanonical(w);
    std::string b = Save(w, schema);
    CanonicalToRest(w);
    MirrorMatch(w, mirror & 1, mirror & 2, mirror & 4);
    return b;
}

namespace {
// GRF: a reset disables and releases every keyboard and sets its mirror (-1 for a right agent);
// the stored direction is times the mirror, so mirror -1 stores -0.
KeyboardState ResetKeyboard(float mirror) {
    KeyboardState k{};
    k.mirror = mirror;
    k.direction = Vec3(0, 0, 0) * mirror;
    k.disabled = true;
    return k;
}
// A newly built gamer without a player (PlayerController::Reset, then HumanController::Reset).
HumanGamer NewHumanGamer(int slot, int keyboard, float mirror) {
    HumanGamer g;
    memset(&g, 0, sizeof(g));
    g.selectedPlayer = -1;
    g.team = slot;
    g.keyboardIndex = keyboard;
    PlayerControllerState &b = g.controller.base;
    b.player = b.team = b.opponentTeam = b.opponentPlayer = -1;
    b.inputDirection = Vec3(0, -1, 0);
    b.possessionAmount = 0.9f;
    b.teamPossessionAmount = 1.0f;
    b.oppTimeNeededToGetToBall = 100;
    b.lastSwitchTimeMs = (uint64_t)(int64_t)-10000;
    b.lastSwitchTimeDurationMs = 300;
    b.fadingTeamPossessionAmount = 1.0f;
    HumanControllerState &c = g.controller;
    c.keyboard = ResetKeyboard(mirror);
    c.actionButton = kBtnShortPass;
    c.previousDirection = Vec3(0, -1, 0);
    c.steadyDirection = Vec3(0, -1, 0);
    return g;
}
}  // namespace

void SetupAgents(World &w, const StaticData &sd, int left, int right, const std::string &bundle) {
    Scenario &sc = w.scenario;
    MatchState &m = w.match;
    auto check = [&](const char *side, int agents, int players) {
        if (agents < 0 || agents > players)
            throw std::invalid_argument("expected from 0 to " + std::to_string(players) + " " + side + " agents for " + bundle +
                                        ", found " + std::to_string(agents));
    };
    check("left", left, sc.leftTeamSize);
    check("right", right, sc.rightTeamSize);
    if (left + right > kMatchKeyboards) throw std::invalid_argument("too many agents for " + bundle);
    // Remove every gamer: no gamers also means no main selected player.
    sc.leftAgents = sc.rightAgents = 0;
    for (Team &t : m.teams) {
        t.gamers.count = 0;
        t.switchPriority.count = 0;
        t.mainSelectedPlayer = -1;
    }
    for (int p = 0; p < m.playerCount; p++) m.players[p].base.externalController = -1;
    m.freeControllerCount = kMatchKeyboards;
    for (int k = 0; k < kMatchKeyboards; k++) m.freeControllers[k] = ResetKeyboard(1.0f);
    sc.leftAgents = left;
    sc.rightAgents = right;
    const int agents[2] = {left, right};
    for (int t = 0; t < 2; t++) {
        Team &team = TeamByID(w, t);
        team.gamers.count = agents[t];
        team.switchPriority.count = agents[t];
        for (int g = 0; g < agents[t]; g++) team.switchPriority[g] = g;
    }
    for (int t = 0; t < 2; t++) {
        // GRF: both teams still face side -1 at the controller setup, so right keyboards mirror.
        const float mirror = t == 1 && TeamDynamicSide(w, 1) == -1 ? -1.0f : 1.0f;
        for (int g = 0; g < agents[t]; g++) {
            const int gi = GlobalGamerIndex(w, t, g);
            HumanGamer &h = GamerByGlobal(w, gi);
            h = NewHumanGamer(TeamSlot(w, t), g + (t ? kTeamControllers : 0), mirror);
            m.secondKeyboardCopies[gi] = h.controller.keyboard;
        }
    }
    m.freeControllerCount = kMatchKeyboards - left - right;
    // GRF: the gamers take the active controllable players closest to the ball (at the origin
    // with the players on their formation spots), the closest as the main selected player, then
    // assigned in stable-ID order.
    Ctx c{};
    c.sd = &sd;
    for (int t = 0; t < 2; t++) {
        if (agents[t] == 0) continue;
        const Vec3 ball = BallPredict(m.ball, 0).Get2D();
        PlayerList ps = GetClosestPlayers(w, c, t, ball, true, (unsigned)agents[t], true);
        if (ps.empty()) continue;
        TeamByID(w, t).mainSelectedPlayer = ps[0];
        for (int i = 1; i < ps.count; i++)
            for (int j = i; j > 0 && sd.stableID[ps[j]] < sd.stableID[ps[j - 1]]; j--) {
                int x = ps[j];
                ps[j] = ps[j - 1];
                ps[j - 1] = x;
            }
        for (int g = 0; g < ps.count; g++) HumanGamerSetSelectedPlayer(w, GlobalGamerIndex(w, t, g), ps[g]);
    }
}

std::unique_ptr<Bundle> LoadBundle(const std::string &path, int left, int right) {
    const std::string bytes = ReadFile(path);
    size_t off = 0;
    auto need = [&](size_t n) {
        if (off + n > bytes.size()) throw std::runtime_error("asset bundle truncated: " + path);
    };
    auto integer = [&]() {
        need(4);
        int32_t v;
        memcpy(&v, bytes.data() + off, 4);
        off += 4;
        return v;
    };
    auto blob = [&]() {
        const uint32_t n = (uint32_t)integer();
        need(n);
        std::string s = bytes.substr(off, n);
        off += n;
        return s;
    };
    if (bytes.compare(0, 9, "CUJASSET1") != 0) throw std::runtime_error("not an asset bundle: " + path);
    off = 9;
    auto b = std::make_unique<Bundle>();
    b->scenario = blob();
    b->leftAgents = integer();
    b->rightAgents = integer();
    if (integer() != 4) throw std::runtime_error("asset bundle: expected 4 variants");
    const int l = left == -1 ? b->leftAgents : left, r = right == -1 ? b->rightAgents : right;
    const bool setup = l != b->leftAgents || r != b->rightAgents;
    StateCodec codec;
    for (int i = 0; i < 4; i++) {
        const int reverse = integer(), parity = integer();
        if ((reverse != 0 && reverse != 1) || (parity != 0 && parity != 1)) throw std::runtime_error("asset bundle: bad variant");
        Variant &v = b->variants[reverse * 2 + parity];
        v.reverse = reverse;
        v.parity = parity;
        v.staticData = ParseStatic(blob());
        v.world = std::make_unique<World>();
        if (!codec.LoadFrame(blob(), 0, *v.world)) throw std::runtime_error("asset bundle: bad reset state in " + path);
        v.freeControllerCount = codec.freeControllerCount;
        if (setup) {
            SetupAgents(*v.world, v.staticData, l, r, path);
            v.freeControllerCount = v.world->match.freeControllerCount;
        }
        v.scenario = ScenarioKey(*v.world);
        v.skeletons = ParseSkeletons(blob());
        if ((int)v.skeletons.size() != v.staticData.count) throw std::runtime_error("asset bundle: skeleton count mismatch in " + path);
        if (v.world->match.playerCount + 3 != v.staticData.count) throw std::runtime_error("asset bundle: static data does not match the players");
    }
    for (const Variant &v : b->variants)
        if (!v.world) throw std::runtime_error("asset bundle: missing variant");
    b->leftAgents = l;
    b->rightAgents = r;
    return b;
}

}  // namespace host
}  // namespace eng
