// The debugging library: the same C ABI with the engine on host threads. Tests load it to follow
// a match tick by tick; the package never loads it.
#include "runtime.h"

#include <algorithm>
#include <stdexcept>
#include <thread>

namespace eng {
namespace host {
// ---- the host device: the engine on host threads -------------------------------------------------------
namespace {
class HostDevice : public Device {
public:
    explicit HostDevice(int threads) {
        threads_ = threads > 0 ? threads : (int)std::max(1u, std::thread::hardware_concurrency());
    }
    const char *Name() const override { return "host"; }
    bool HostMemory() const override { return true; }
    void *Allocate(size_t n) override {
        void *p = calloc(1, n);
        if (!p) throw std::bad_alloc();
        return p;
    }
    void Release(void *p) override { free(p); }
    void ToDevice(void *d, const void *s, size_t n) override { memcpy(d, s, n); }
    void ToHost(void *d, const void *s, size_t n) override { memcpy(d, s, n); }
    void ToDeviceAsync(void *d, const void *s, size_t n, void *) override { memcpy(d, s, n); }
    void Fill(void *d, int v, size_t n) override { memset(d, v, n); }
    void Synchronize(void *) override {}
    void CheckFault() override {
        if (!fault_.empty()) {
            std::string f = fault_;
            fault_.clear();
            throw std::runtime_error(f);
        }
    }
    int Threads() const override { return threads_; }
    void Reset(const Batch &b, const uint8_t *mask, const int64_t *seeds, const int32_t *reverse, void *) override {
        ForEach(b.count, [&](int e) {
            if (mask && !mask[e]) return true;
            return ResetAndWriteEnvironment(b, e, seeds, reverse);
        });
    }
    void Step(const Batch &b, const int32_t *actions, void *) override {
        stepTicks_.assign(b.count, 0);
        ForEach(b.count, [&](int e) {
            const long long before = HostTicks();
            const bool ok = StepEnvironment(b, e, actions);
            stepTicks_[e] = HostTicks() - before;
            return ok;
        });
    }
    // The ticks each environment ran in the last step, its auto-reset's included.
    const std::vector<long long> &StepTicks() const { return stepTicks_; }
    void Outputs(const Batch &b, int env, void *) override { WriteEnvironmentOutputs(b, env, false); }

private:
    template <class F>
    void ForEach(int count, F body) {
        const int workers = std::min(threads_, count);
        std::vector<std::string> faults(workers);
        auto run = [&](int w) {
            for (int e = w; e < count; e += workers) {
                try {
                    FailReason() = "";
                    if (!body(e)) {
                        faults[w] = "environment " + std::to_string(e) + " reached a path that GRF leaves undefined: " + FailReason();
                        return;
                    }
                } catch (const std::exception &ex) {
                    faults[w] = "environment " + std::to_string(e) + ": " + ex.what();
                    return;
                }
            }
        };
        if (workers == 1) {
            run(0);
        } else {
            std::vector<std::thread> pool;
            for (int w = 0; w < workers; w++) pool.emplace_back(run, w);
            for (auto &t : pool) t.join();
        }
        for (auto &f : faults)
            if (!f.empty() && fault_.empty()) fault_ = f;
    }
    int threads_;
    std::string fault_;
    std::vector<long long> stepTicks_;
};
}  // namespace

// The ticks each environment ran in the batch's last step: GRF's step ticks until play, so a
// stoppage makes one environment step run many more than the ticks per step.
extern "C" __attribute__((visibility("default"))) int cuju_debug_step_ticks(void *environment, long long *out) {
    auto *device = dynamic_cast<HostDevice *>(&static_cast<BatchRuntime *>(environment)->Dev());
    if (!device) return -1;
    const std::vector<long long> &ticks = device->StepTicks();
    std::copy(ticks.begin(), ticks.end(), out);
    return (int)ticks.size();
}

std::unique_ptr<Device> MakeLibraryDevice(int threads, int) { return std::make_unique<HostDevice>(threads); }
extern const char *const kBackendName = "host";
extern const bool kLibraryHostMemory = true;
}  // namespace host
}  // namespace eng

#include <cmath>
#include <cstring>
#include <sstream>

// The field layout of a state, one line per field: byte position, size and path. Tests use it to
// name the first field where two states differ.
extern "C" __attribute__((visibility("default"))) const char *cuju_debug_state_schema(const char *bytes, unsigned long long size) {
    thread_local std::string text;
    try {
        std::string in(bytes, size);
        auto w = std::make_unique<eng::World>();
        eng::host::StateCodec codec;
        if (!codec.Load(in, *w)) return nullptr;
        std::vector<eng::codec::SchemaEntry> schema;
        codec.Save(*w, &schema);
        std::ostringstream o;
        for (const auto &e : schema) o << e.position << ' ' << e.size << ' ' << e.path << '\n';
        text = o.str();
        return text.c_str();
    } catch (...) {
        return nullptr;
    }
}

// The first `count` episode seeds that environment `index` of a batch with `seed` draws.
extern "C" __attribute__((visibility("default"))) void cuju_debug_episode_seeds(unsigned long long seed, unsigned int index, int count,
                                                                                  unsigned int *out) {
    auto g = std::make_unique<eng::EpisodeGenerator>();
    eng::SeedEpisodeGenerator(*g, seed, index);
    for (int i = 0; i < count; i++) out[i] = eng::DrawEpisodeSeed(*g);
}

// The world generator seeded with `seed`: `count` raw words, then `count` uniform floats in
// [low, high) from a second generator of the same seed.
extern "C" __attribute__((visibility("default"))) void cuju_debug_world_rng(unsigned int seed, int count, float low, float high,
                                                                              unsigned int *words, float *uniforms) {
    uint8_t bytes[sizeof(eng::World::rng)];
    eng::Rng g{bytes};
    g.Seed(seed);
    for (int i = 0; i < count; i++) words[i] = g.Next();
    g.Seed(seed);
    g.Store(eng::Rng::kLowAt, low);
    g.Store(eng::Rng::kHighAt, high);
    for (int i = 0; i < count; i++) uniforms[i] = g.Uniform();
}

// GRF's time-to-target estimate for `count` cases: directly, along the shared walk, and by the
// possession scan's shortcut (usual and optimistic times of each, direct first); tests compare them.
extern "C" __attribute__((visibility("default"))) void cuju_debug_time_needed(const float *cases, int count, unsigned int *out) {
    auto walk = std::make_unique<eng::TimeWalk>();
    std::unique_ptr<eng::TimeNeededScan> scan;
    for (int i = 0; i < count; i++) {
        const float *q = cases + (size_t)i * 12;
        const eng::Vec3 pos(q[0], q[1], q[2]), mov(q[3], q[4], q[5]), target(q[6], q[7], q[8]);
        const float maxVel = q[9];
        const bool precise = q[10] != 0.0f;
        const uint32_t maxTime = q[11] < 0 ? (uint32_t)-1 : (uint32_t)q[11];
        const eng::TimeNeeded a = eng::GetTimeNeededMs(pos, mov, target, maxVel, precise, maxTime);
        eng::TimeNeeded b = a;
        if (eng::TimeWalkApplies(mov)) {
            eng::BuildTimeWalk(*walk, pos, mov, maxVel);
            b = eng::WalkTimeNeeded(*walk, pos, mov, target, maxVel, precise, maxTime, false);
        }
        // Consecutive cases of one player share a scan, as the targets of a possession scan do.
        if (!scan || !(scan->pos == pos) || !(scan->mov == mov) || scan->maxVel != maxVel)
            scan = std::make_unique<eng::TimeNeededScan>(pos, mov, maxVel);
        const eng::TimeNeeded c = scan->Get(target, precise, maxTime);
        out[(size_t)i * 6 + 0] = a.usual;
        out[(size_t)i * 6 + 1] = a.optimistic;
        out[(size_t)i * 6 + 2] = b.usual;
        out[(size_t)i * 6 + 3] = b.optimistic;
        out[(size_t)i * 6 + 4] = c.usual;
        out[(size_t)i * 6 + 5] = c.optimistic;
    }
}

// The bytes of one environment's blocks in device memory: World, EnvCore, EnvSlot and Scratch. The
// engine's structs have the same layout on the host and the device.
extern "C" __attribute__((visibility("default"))) void cuju_debug_layout(unsigned long long *out) {
    out[0] = sizeof(eng::World);
    out[1] = sizeof(eng::EnvCore);
    out[2] = sizeof(eng::EnvSlot);
    out[3] = sizeof(eng::Scratch);
}
// The engine's math routines for tests, by the codes of eng::libm::EvaluateFloat and
// EvaluateDouble: on arrays, and on the consecutive float bit patterns from `first`.
extern "C" __attribute__((visibility("default"))) void cuju_debug_libm(int which, const float *x, const float *y, float *out,
                                                                         long long count) {
    for (long long i = 0; i < count; i++) out[i] = eng::libm::EvaluateFloat(which, x[i], y[i]);
}
extern "C" __attribute__((visibility("default"))) void cuju_debug_libm_range(int which, uint32_t first, long long count, float *out) {
    for (long long i = 0; i < count; i++) out[i] = eng::libm::EvaluateFloat(which, eng::FloatOf(first + (uint32_t)i), 0.0f);
}
extern "C" __attribute__((visibility("default"))) void cuju_debug_libm_double(int which, const double *x, const double *y,
                                                                                double *out, long long count) {
    for (long long i = 0; i < count; i++) out[i] = eng::libm::EvaluateDouble(which, x[i], y[i]);
}

// The description a scenario builder needs to rebuild a bundle's variant (reverse 0, `parity`),
// read back from its template: the flags, difficulties and player entries as stored, and for
// each coordinate the float whose scaling gives the stored value (any one does: the builder
// reads the description only through that scaling). Tests rebuild the shipped bundles from it.
#include "../../../include/cuju_amd.h"
namespace {
template <class F>
float Preimage(float stored, double estimate, F scale) {
    auto same = [&](float f) {
        const float v = scale(f);
        return memcmp(&v, &stored, sizeof(float)) == 0;
    };
    float up = (float)estimate, down = up;
    if (same(up)) return up;
    for (int k = 0; k < 32; k++) {
        up = nextafterf(up, INFINITY);
        if (same(up)) return up;
        down = nextafterf(down, -INFINITY);
        if (same(down)) return down;
    }
    throw std::runtime_error("no float scales to the stored coordinate");
}
}  // namespace
extern "C" __attribute__((visibility("default"))) int cuju_debug_bundle_description(const char *path, int parity, cuju_scenario_description *out,
                                                                                      cuju_scenario_player *left, cuju_scenario_player *right) {
    try {
        const auto bundle = eng::host::LoadBundle(path);
        const eng::Scenario &s = bundle->variants[parity & 1].world->scenario;
        memset(out, 0, sizeof(*out));
        out->version = CUJU_SCENARIO_VERSION;
        out->ball_x = Preimage(s.ballPosition.v[0], s.ballPosition.v[0] / 54.4, [](float f) { return (float)((double)f * 54.4); });
        out->ball_y = Preimage(s.ballPosition.v[1], s.ballPosition.v[1] / -83.6, [](float f) { return (float)((double)f * -83.6); });
        for (int side = 0; side < 2; side++) {
            const eng::FormationEntry *team = side ? s.rightTeam : s.leftTeam;
            const int n = side ? s.rightTeamSize : s.leftTeamSize;
            cuju_scenario_player *players = side ? right : left;
            for (int p = 0; p < n; p++) {
                const eng::Vec3 &at = team[p].startPosition;
                players[p].x = at.v[0];
                players[p].y = Preimage(at.v[1], (double)at.v[1] / -2.36, [](float f) { return f * -2.36f; });
                players[p].role = team[p].role;
                players[p].lazy = team[p].lazy;
                players[p].controllable = team[p].controllable;
            }
            (side ? out->right_size : out->left_size) = n;
        }
        out->left_team = left;
        out->right_team = right;
        out->use_magnet = s.useMagnet;
        out->offsides = s.offsides;
        out->real_time = s.realTime;
        out->left_team_difficulty = s.leftDifficulty;
        out->right_team_difficulty = s.rightDifficulty;
        out->deterministic = s.deterministic;
        out->end_episode_on_score = s.endOnScore;
        out->end_episode_on_possession_change = s.endOnPossessionChange;
        out->end_episode_on_out_of_play = s.endOnOutOfPlay;
        out->game_duration = s.gameDuration;
        out->second_half = s.secondHalf;
        out->control_all_players = s.controlAllPlayers;
        out->game_engine_random_seed = s.deterministic ? s.gameEngineRandomSeed : 42;
        return 0;
    } catch (...) {
        return -1;
    }
}
