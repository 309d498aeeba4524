// The C ABI over the batch runtime: the entry points of the reference's src/environment_api.h
// (cited per function in include/cuju_amd.h) with its argument meaning and error convention:
// -1 or null with a per-thread message, -2 for an action out of range.
#include <algorithm>
#include <cstring>
#include <fstream>
#include <exception>
#include <stdexcept>
#include <string>

#include "../../../include/cuju_amd.h"
#include "runtime.h"
#include "scenario.h"

namespace eng {
namespace host {
// Defined by each library: its device and backend name.
std::unique_ptr<Device> MakeLibraryDevice(int threads, int environments);
extern const char *const kBackendName;
// Whether the library's device keeps the batch in host memory (the host debugging build).
extern const bool kLibraryHostMemory;
}  // namespace host
}  // namespace eng

using eng::host::BatchRuntime;

namespace {
// The calling thread's last failure, and the bytes of the last state it read.
thread_local std::string lastError;
thread_local std::string stateBytes;

BatchRuntime *Of(void *e) { return static_cast<BatchRuntime *>(e); }

// Runs `body` and turns what it throws into the error convention: the message is kept for
// cuju_last_error, and the call returns `failed`. An action index out of range
// (std::out_of_range) returns `outOfRange` where the entry point reports it apart.
template <class R, class Body>
R Guarded(R failed, Body body, R outOfRange) {
    try {
        return body();
    } catch (const std::out_of_range &e) {
        lastError = e.what();
        return outOfRange;
    } catch (const std::exception &e) {
        lastError = e.what();
        return failed;
    }
}
// 0, or -1 on failure.
template <class Body>
int Status(Body body) {
    return Guarded(-1, [&] {
        body();
        return 0;
    }, -1);
}

void Require(bool holds, const char *what) {
    if (!holds) throw std::invalid_argument(what);
}
std::string Found(const char *expected, long long wanted, long long found) {
    return std::string(expected) + std::to_string(wanted) + ", found " + std::to_string(found);
}

// The runtime's configuration from the ABI's, checked as the reference checks it.
eng::host::Configuration ConfigurationOf(const struct cuju_configuration *s) {
    Require(s != nullptr, "expected a configuration");
    if (s->version != CUJU_CONFIGURATION_VERSION)
        throw std::invalid_argument(Found("expected the configuration version ", CUJU_CONFIGURATION_VERSION, s->version));
    if (s->environment_count < 1)
        throw std::invalid_argument("expected at least one environment, found " + std::to_string(s->environment_count));
    Require(!s->allocate == !s->release, "expected both allocate and release, or neither");
    const int n = s->environment_count;
    eng::host::Configuration c;
    c.assets.assign(s->assets, s->assets + s->asset_count);
    if (s->assignment) c.assignment.assign(s->assignment, s->assignment + n);
    if (s->fixed_seeds) c.fixedSeeds.assign(s->fixed_seeds, s->fixed_seeds + n);
    if (s->agent_counts) c.agentCounts.assign(s->agent_counts, s->agent_counts + 2 * s->asset_count);
    c.animations = s->animations ? s->animations : "";
    c.count = n;
    c.seed = s->seed;
    c.actionSet = s->action_set;
    c.observation = s->observation;
    c.checkpoints = s->checkpoints != 0;
    c.numpyLegacy = s->numpy_legacy != 0;
    c.autoReset = s->auto_reset != 0;
    c.threads = s->threads;
    c.allocate = s->allocate;
    c.release = s->release;
    c.allocatorContext = s->allocator_context;
    c.ticksPerStep = s->ticks_per_step;
    c.smmWidth = s->smm_width;
    c.smmHeight = s->smm_height;
    c.stack = s->stack;
    c.episodeNumber = s->episode_number;
    // A larger value fails the range check rather than wrapping.
    c.firstIndex = (int64_t)std::min<unsigned long long>(s->first_index, 1ULL << 62);
    return c;
}

// One parity's scenario from the ABI's description.
eng::host::ScenarioDescription ScenarioOf(const cuju_scenario_description &s) {
    if (s.version != CUJU_SCENARIO_VERSION)
        throw std::invalid_argument(Found("expected the scenario description version ", CUJU_SCENARIO_VERSION, s.version));
    Require(s.left_size >= 0 && s.right_size >= 0, "expected team sizes of zero or more");
    Require((s.left_size == 0 || s.left_team) && (s.right_size == 0 || s.right_team), "expected the players of each team");
    eng::host::ScenarioDescription d;
    d.ballX = s.ball_x;
    d.ballY = s.ball_y;
    auto team = [](const cuju_scenario_player *players, int count) {
        std::vector<eng::host::ScenarioPlayer> out;
        for (const cuju_scenario_player *p = players; p < players + count; p++)
            out.push_back({p->x, p->y, p->role, p->lazy != 0, p->controllable != 0});
        return out;
    };
    d.leftTeam = team(s.left_team, s.left_size);
    d.rightTeam = team(s.right_team, s.right_size);
    d.useMagnet = s.use_magnet != 0;
    d.offsides = s.offsides != 0;
    d.realTime = s.real_time != 0;
    d.deterministic = s.deterministic != 0;
    d.endOnScore = s.end_episode_on_score != 0;
    d.endOnPossessionChange = s.end_episode_on_possession_change != 0;
    d.endOnOutOfPlay = s.end_episode_on_out_of_play != 0;
    d.controlAllPlayers = s.control_all_players != 0;
    d.leftTeamDifficulty = s.left_team_difficulty;
    d.rightTeamDifficulty = s.right_team_difficulty;
    d.gameDuration = s.game_duration;
    d.secondHalf = s.second_half;
    d.gameEngineRandomSeed = s.game_engine_random_seed;
    return d;
}

void WriteFile(const char *path, const std::string &bytes) {
    std::ofstream file(path, std::ios::binary);
    if (file) file.write(bytes.data(), (std::streamsize)bytes.size());
    if (!file) throw std::runtime_error(std::string("cannot write ") + path);
}
}  // namespace

#pragma GCC visibility push(default)
extern "C" {

const char *cuju_last_error(void) { return lastError.c_str(); }
const char *cuju_backend(void) { return eng::host::kBackendName; }

void *cuju_environment_create(const struct cuju_configuration *s) {
    lastError.clear();
    return Guarded<void *>(nullptr, [&]() -> void * {
        const eng::host::Configuration c = ConfigurationOf(s);
        return new BatchRuntime(c, eng::host::MakeLibraryDevice(s->threads, c.count));
    }, nullptr);
}
int cuju_memory_estimate(const struct cuju_configuration *settings, unsigned long long *bytes) {
    lastError.clear();
    return Status([&] {
        eng::host::Configuration c = ConfigurationOf(settings);
        // The estimate takes nothing from the caller's allocator.
        c.allocate = nullptr;
        c.release = nullptr;
        *bytes = BatchRuntime(c, eng::host::MakeSizingDevice(eng::host::kLibraryHostMemory)).MemoryBytes();
    });
}
int cuju_local_memory_bytes(unsigned long long *bytes) {
    *bytes = 0;
    return 0;
}
unsigned long long cuju_environment_memory_bytes(void *e) { return Of(e)->MemoryBytes(); }
void cuju_environment_destroy(void *e) { delete Of(e); }
int cuju_environment_count(void *e) { return Of(e)->Count(); }
int cuju_environment_threads(void *e) { return Of(e)->Dev().Threads(); }
int cuju_environment_geometry(void *e, int *lanes) { return Of(e)->Dev().Geometry(lanes); }
int cuju_environment_agents(void *e, int *left, int *right) {
    const BatchRuntime &b = *Of(e);
    for (int i = 0; i < b.Count(); i++) {
        if (left) left[i] = b.LeftAgents(i);
        if (right) right[i] = b.RightAgents(i);
    }
    return b.Agents();
}
int cuju_environment_players(void *e, int *left, int *right) {
    const BatchRuntime &b = *Of(e);
    for (int i = 0; i < b.Count(); i++) {
        if (left) left[i] = b.LeftPlayers(i);
        if (right) right[i] = b.RightPlayers(i);
    }
    return b.Players();
}
int cuju_environment_set_difficulty(void *e, const float *difficulty) {
    return Status([&] { Of(e)->SetDifficulty(difficulty); });
}
void cuju_environment_difficulty(void *e, float *difficulty) {
    const BatchRuntime &b = *Of(e);
    for (int i = 0; i < 2 * b.Count(); i++) difficulty[i] = b.Difficulty(i / 2, i % 2);
}
int cuju_environment_reset(void *e, const unsigned int *seeds, const int *reverse, void *stream) {
    return Status([&] { Of(e)->Reset(seeds, reverse, stream); });
}
int cuju_environment_reset_masked(void *e, const unsigned char *mask, int mask_on_device, const int64_t *seeds, const int *reverse,
                                  void *stream, int synchronize) {
    return Status([&] {
        Of(e)->ResetMasked(mask, mask_on_device != 0, seeds, reverse, stream);
        if (synchronize) Of(e)->Synchronize(stream);
    });
}
int cuju_environment_reset_done(void *e, void *stream) {
    return Status([&] { Of(e)->ResetDone(stream); });
}
int cuju_environment_step(void *e, const int *actions, int on_device, void *stream, int synchronize) {
    return Guarded(-1, [&] {
        Of(e)->Step(actions, on_device != 0, stream, synchronize != 0);
        return 0;
    }, -2);
}
int cuju_environment_step_no_alloc(void *e, const int *actions, void *stream) {
    return Status([&] { Of(e)->StepWithStaticScratch(actions, stream); });
}
int cuju_environment_step_async(void *e, const int *actions, int on_device, void *stream) {
    return cuju_environment_step(e, actions, on_device, stream, 0);
}
int cuju_environment_step_wait(void *) { return 0; }
int cuju_environment_synchronize(void *e, void *stream) {
    return Status([&] { Of(e)->Synchronize(stream); });
}
const char *cuju_environment_get_state(void *e, int index, unsigned long long *size, int *episode) {
    return Guarded<const char *>(nullptr, [&]() -> const char * {
        stateBytes = Of(e)->GetState(index, episode);
        *size = stateBytes.size();
        return stateBytes.data();
    }, nullptr);
}
int cuju_environment_set_state(void *e, int index, const char *bytes, unsigned long long size, const int *episode) {
    return Status([&] {
        Require(bytes && episode, "expected state bytes and the episode values");
        Of(e)->SetState(index, std::string(bytes, size), episode[0], episode[1], episode[2], episode + 3);
    });
}
int cuju_environment_set_stack(void *e, int index, const char *name, const void *frames, unsigned long long size) {
    return Status([&] {
        Require(frames != nullptr, "expected frames");
        Of(e)->SetStack(index, name ? name : "", frames, size);
    });
}
const char *cuju_environment_raw_field(void *e, int field, int *type, int *dimensions, unsigned long long *offset) {
    if (!e || !type || !dimensions || !offset) return nullptr;
    return Of(e)->RawField(field, type, dimensions, offset);
}
void *cuju_environment_buffer(void *e, const char *name) {
    const std::string wanted = name ? name : "";
    void *p = Of(e)->Buffer(wanted);
    if (!p) lastError = "no buffer named " + (name ? wanted : std::string("(null)"));
    return p;
}
int cuju_environment_episode(void *e, int index, long long *values, float *difficulty) {
    return Status([&] {
        Require(values != nullptr, "expected room for the episode values");
        Of(e)->Episode(index, values, difficulty);
    });
}
const char *cuju_environment_scenario(void *e, int bundle) { return Of(e)->ScenarioName(bundle); }
int cuju_scenario_build_bundle(const struct cuju_scenario_description *even, const struct cuju_scenario_description *odd,
                               const char *name, const char *animations, const char *out) {
    return Status([&] {
        Require(even && odd && name && animations && out, "expected two descriptions, a name and two paths");
        const eng::host::ScenarioDescription parity[2] = {ScenarioOf(*even), ScenarioOf(*odd)};
        WriteFile(out, eng::host::BuildScenarioBundle(name, parity, animations));
    });
}

}  // extern "C"
#pragma GCC visibility pop
