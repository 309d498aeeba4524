// The C ABI over the batch runtime: the entry points of the reference's src/environment_api.h
// (cited per function in include/cuju_amd.h) with its argument meaning and error convention:
// -1 or null with a per-thread message, -2 for an action out of range.
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
thread_local std::string lastError;
thread_local std::string stateBytes;
int Fail(const std::exception &e) {
    lastError = e.what();
    return -1;
}
BatchRuntime *Of(void *e) { return static_cast<BatchRuntime *>(e); }

eng::host::Configuration ConfigurationOf(const struct cuju_configuration *s) {
    if (!s) throw std::invalid_argument("expected a configuration");
    if (s->version != CUJU_CONFIGURATION_VERSION)
        throw std::invalid_argument("expected the configuration version " + std::to_string(CUJU_CONFIGURATION_VERSION) + ", found " +
                                    std::to_string(s->version));
    if (s->environment_count < 1) throw std::invalid_argument("expected at least one environment, found " + std::to_string(s->environment_count));
    if (!s->allocate != !s->release) throw std::invalid_argument("expected both allocate and release, or neither");
    eng::host::Configuration c;
    for (int i = 0; i < s->asset_count; i++) c.assets.push_back(s->assets[i]);
    if (s->assignment) c.assignment.assign(s->assignment, s->assignment + s->environment_count);
    c.animations = s->animations ? s->animations : "";
    c.count = s->environment_count;
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
    if (s->fixed_seeds) c.fixedSeeds.assign(s->fixed_seeds, s->fixed_seeds + s->environment_count);
    if (s->agent_counts) c.agentCounts.assign(s->agent_counts, s->agent_counts + 2 * s->asset_count);
    c.episodeNumber = s->episode_number;
    // A larger value fails the range check rather than wrapping.
    c.firstIndex = (int64_t)(s->first_index < (1ULL << 62) ? s->first_index : (1ULL << 62));
    return c;
}
}  // namespace

#pragma GCC visibility push(default)
extern "C" {

const char *cuju_last_error(void) { return lastError.c_str(); }
const char *cuju_backend(void) { return eng::host::kBackendName; }

void *cuju_environment_create(const struct cuju_configuration *s) {
    try {
        lastError.clear();
        const eng::host::Configuration c = ConfigurationOf(s);
        return new BatchRuntime(c, eng::host::MakeLibraryDevice(s->threads, c.count));
    } catch (const std::exception &e) {
        Fail(e);
        return nullptr;
    }
}

int cuju_memory_estimate(const struct cuju_configuration *settings, unsigned long long *bytes) {
    try {
        lastError.clear();
        eng::host::Configuration c = ConfigurationOf(settings);
        // The estimate takes nothing from the caller's allocator.
        c.allocate = nullptr;
        c.release = nullptr;
        BatchRuntime sized(c, eng::host::MakeSizingDevice(eng::host::kLibraryHostMemory));
        *bytes = sized.MemoryBytes();
        return 0;
    } catch (const std::exception &e) {
        return Fail(e);
    }
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
    BatchRuntime *b = Of(e);
    for (int i = 0; i < b->Count(); i++) {
        if (left) left[i] = b->LeftAgents(i);
        if (right) right[i] = b->RightAgents(i);
    }
    return b->Agents();
}
int cuju_environment_players(void *e, int *left, int *right) {
    BatchRuntime *b = Of(e);
    for (int i = 0; i < b->Count(); i++) {
        if (left) left[i] = b->LeftPlayers(i);
        if (right) right[i] = b->RightPlayers(i);
    }
    return b->Players();
}
int cuju_environment_set_difficulty(void *e, const float *difficulty) {
    try {
        Of(e)->SetDifficulty(difficulty);
        return 0;
    } catch (const std::exception &ex) {
        return Fail(ex);
    }
}
void cuju_environment_difficulty(void *e, float *difficulty) {
    BatchRuntime *b = Of(e);
    for (int i = 0; i < b->Count(); i++)
        for (int s = 0; s < 2; s++) difficulty[i * 2 + s] = b->Difficulty(i, s);
}
int cuju_environment_reset(void *e, const unsigned int *seeds, const int *reverse, void *stream) {
    try {
        Of(e)->Reset(seeds, reverse, stream);
        return 0;
    } catch (const std::exception &ex) {
        return Fail(ex);
    }
}
int cuju_environment_reset_masked(void *e, const unsigned char *mask, int mask_on_device, const int64_t *seeds, const int *reverse,
                                  void *stream, int synchronize) {
    try {
        Of(e)->ResetMasked(mask, mask_on_device != 0, seeds, reverse, stream);
        if (synchronize) Of(e)->Synchronize(stream);
        return 0;
    } catch (const std::exception &ex) {
        return Fail(ex);
    }
}
int cuju_environment_reset_done(void *e, void *stream) {
    try {
        Of(e)->ResetDone(stream);
        return 0;
    } catch (const std::exception &ex) {
        return Fail(ex);
    }
}
int cuju_environment_step(void *e, const int *actions, int on_device, void *stream, int synchronize) {
    try {
        Of(e)->Step(actions, on_device != 0, stream, synchronize != 0);
        return 0;
    } catch (const std::out_of_range &ex) {
        Fail(ex);
        return -2;
    } catch (const std::exception &ex) {
        return Fail(ex);
    }
}
int cuju_environment_step_no_alloc(void *e, const int *actions, void *stream) {
    try {
        Of(e)->StepWithStaticScratch(actions, stream);
        return 0;
    } catch (const std::exception &ex) {
        return Fail(ex);
    }
}
int cuju_environment_step_async(void *e, const int *actions, int on_device, void *stream) {
    return cuju_environment_step(e, actions, on_device, stream, 0);
}
int cuju_environment_step_wait(void *e) {
    (void)e;
    return 0;
}
int cuju_environment_synchronize(void *e, void *stream) {
    try {
        Of(e)->Synchronize(stream);
        return 0;
    } catch (const std::exception &ex) {
        return Fail(ex);
    }
}
const char *cuju_environment_get_state(void *e, int index, unsigned long long *size, int *episode) {
    try {
        stateBytes = Of(e)->GetState(index, episode);
        *size = stateBytes.size();
        return stateBytes.data();
    } catch (const std::exception &ex) {
        Fail(ex);
        return nullptr;
    }
}
int cuju_environment_set_state(void *e, int index, const char *bytes, unsigned long long size, const int *episode) {
    try {
        if (!bytes || !episode) throw std::invalid_argument("expected state bytes and the episode values");
        Of(e)->SetState(index, std::string(bytes, size), episode[0], episode[1], episode[2], episode + 3);
        return 0;
    } catch (const std::exception &ex) {
        return Fail(ex);
    }
}
int cuju_environment_set_stack(void *e, int index, const char *name, const void *frames, unsigned long long size) {
    try {
        if (!frames) throw std::invalid_argument("expected frames");
        Of(e)->SetStack(index, name ? name : "", frames, size);
        return 0;
    } catch (const std::exception &ex) {
        return Fail(ex);
    }
}
const char *cuju_environment_raw_field(void *e, int field, int *type, int *dimensions, unsigned long long *offset) {
    if (!e || !type || !dimensions || !offset) return nullptr;
    return Of(e)->RawField(field, type, dimensions, offset);
}
void *cuju_environment_buffer(void *e, const char *name) {
    void *p = Of(e)->Buffer(name ? name : "");
    if (!p) lastError = std::string("no buffer named ") + (name ? name : "(null)");
    return p;
}

int cuju_environment_episode(void *e, int index, long long *values, float *difficulty) {
    try {
        if (!values) throw std::invalid_argument("expected room for the episode values");
        Of(e)->Episode(index, values, difficulty);
        return 0;
    } catch (const std::exception &ex) {
        return Fail(ex);
    }
}
const char *cuju_environment_scenario(void *e, int bundle) { return Of(e)->ScenarioName(bundle); }
int cuju_scenario_build_bundle(const struct cuju_scenario_description *even, const struct cuju_scenario_description *odd,
                               const char *name, const char *animations, const char *out) {
    try {
        if (!even || !odd || !name || !animations || !out) throw std::invalid_argument("expected two descriptions, a name and two paths");
        const cuju_scenario_description *sources[2] = {even, odd};
        eng::host::ScenarioDescription parity[2];
        for (int i = 0; i < 2; i++) {
            const cuju_scenario_description &s = *sources[i];
            if (s.version != CUJU_SCENARIO_VERSION)
                throw std::invalid_argument("expected the scenario description version " + std::to_string(CUJU_SCENARIO_VERSION) +
                                            ", found " + std::to_string(s.version));
            if (s.left_size < 0 || s.right_size < 0) throw std::invalid_argument("expected team sizes of zero or more");
            if ((s.left_size > 0 && !s.left_team) || (s.right_size > 0 && !s.right_team)) throw std::invalid_argument("expected the players of each team");
            eng::host::ScenarioDescription &d = parity[i];
            d.ballX = s.ball_x;
            d.ballY = s.ball_y;
            for (int side = 0; side < 2; side++) {
                const cuju_scenario_player *players = side ? s.right_team : s.left_team;
                std::vector<eng::host::ScenarioPlayer> &team = side ? d.rightTeam : d.leftTeam;
                for (int p = 0, n = side ? s.right_size : s.left_size; p < n; p++)
                    team.push_back({players[p].x, players[p].y, players[p].role, players[p].lazy != 0, players[p].controllable != 0});
            }
            d.useMagnet = s.use_magnet != 0;
            d.offsides = s.offsides != 0;
            d.realTime = s.real_time != 0;
            d.leftTeamDifficulty = s.left_team_difficulty;
            d.rightTeamDifficulty = s.right_team_difficulty;
            d.deterministic = s.deterministic != 0;
            d.endOnScore = s.end_episode_on_score != 0;
            d.endOnPossessionChange = s.end_episode_on_possession_change != 0;
            d.endOnOutOfPlay = s.end_episode_on_out_of_play != 0;
            d.gameDuration = s.game_duration;
            d.secondHalf = s.second_half;
            d.controlAllPlayers = s.control_all_players != 0;
            d.gameEngineRandomSeed = s.game_engine_random_seed;
        }
        const std::string bundle = eng::host::BuildScenarioBundle(name, parity, animations);
        std::ofstream file(out, std::ios::binary);
        if (!file) throw std::runtime_error(std::string("cannot write ") + out);
        file.write(bundle.data(), (std::streamsize)bundle.size());
        if (!file) throw std::runtime_error(std::string("cannot write ") + out);
        return 0;
    } catch (const std::exception &ex) {
        return Fail(ex);
    }
}

}  // extern "C"
#pragma GCC visibility pop
