// The batch runtime. Semantics: include/cuju/batch/batch_environment.h:36-230 (creation and
// checks), :254-330 (resets and steps), :384-395 (state export).
#include "runtime.h"

#include <algorithm>
#include <stdexcept>

namespace eng {
namespace host {

BatchRuntime::BatchRuntime(const Configuration &cfg, std::unique_ptr<Device> device) : cfg_(cfg), dev_(std::move(device)) {
    try {
        if ((cfg.observation & kObsSimple115) && (cfg.observation & kObsSimple115v2))
            throw std::invalid_argument("simple115 and simple115v2 are exclusive");
        if ((cfg.observation & kObsSmm) && (cfg.smmWidth < 1 || cfg.smmHeight < 1))
            throw std::invalid_argument("expected an SMM of at least 1 by 1, found " + std::to_string(cfg.smmWidth) + " by " +
                                        std::to_string(cfg.smmHeight));
        if (!(cfg.observation & (kObsSimple115 | kObsSimple115v2 | kObsSmm | kObsRaw)))
            throw std::invalid_argument("expected at least one representation");
        if (cfg.assets.empty()) throw std::invalid_argument("expected an asset bundle");
        if (cfg.count < 1) throw std::invalid_argument("expected at least one environment, found " + std::to_string(cfg.count));
        if (cfg.ticksPerStep < 1) throw std::invalid_argument("expected at least one tick in a step");
        if (!cfg.fixedSeeds.empty()) {
            if ((int)cfg.fixedSeeds.size() != cfg.count) throw std::invalid_argument("expected one fixed seed for each environment");
            for (int64_t s : cfg.fixedSeeds)
                if (s < -1 || s > 4294967295LL) throw std::invalid_argument("expected a fixed seed from 0 to 4294967295, found " + std::to_string(s));
        }
        if (cfg.firstIndex < 0 || cfg.firstIndex + cfg.count > (int64_t(1) << 32))
            throw std::invalid_argument("expected a first index from 0 to 2**32 minus the environment count");
        if (cfg.episodeNumber < 0) throw std::invalid_argument("expected an episode number of at least 0");
        if (cfg.stack != 1 && cfg.stack != 4) throw std::invalid_argument("expected a stack of 1 or 4 observations, found " + std::to_string(cfg.stack));
        if (cfg.actionSet < 0 || cfg.actionSet > 2) throw std::invalid_argument("expected an action set from 0 to 2");
        const int count = cfg.count;
        std::vector<int32_t> assignment = cfg.assignment;
        if (assignment.empty()) assignment.assign(count, 0);
        if ((int)assignment.size() != count) throw std::invalid_argument("expected one bundle for each environment");
        for (int32_t a : assignment)
            if (a < 0 || a >= (int)cfg.assets.size()) throw std::invalid_argument("expected a bundle from 0 to " + std::to_string(cfg.assets.size() - 1) + ", found " + std::to_string(a));
        if (!cfg.agentCounts.empty() && cfg.agentCounts.size() != 2 * cfg.assets.size())
            throw std::invalid_argument("expected a left and a right agent count for each bundle");
        for (size_t i = 0; i < cfg.assets.size(); i++) {
            const int l = cfg.agentCounts.empty() ? -1 : cfg.agentCounts[2 * i];
            const int r = cfg.agentCounts.empty() ? -1 : cfg.agentCounts[2 * i + 1];
            bundles_.push_back(LoadBundle(cfg.assets[i], l, r));
        }
        tables_ = LoadAnimationTables(cfg.animations);
        for (const Anim &a : tables_->anims)
            if (a.frameCount > kAnimPositions) throw std::invalid_argument("expected animations of at most 320 frames");

        // Shared tables: one device copy, addressed through a device Tables record.
        const AnimationTables &T = *tables_;
        Tables dt = T.View();
        dt.anims = Upload(T.anims);
        dt.nodes = Upload(T.nodes);
        dt.keys = Upload(T.keys);
        dt.interp = Upload(T.interp);
        dt.middle = Upload(T.middle);
        dt.football = Upload(T.football);
        dt.positions = Upload(T.positions);
        dt.quadrants = Upload(T.quadrants);
        dt.derived = Upload(T.derived);
        dt.selection = Upload(T.selection);
        dt.smoothed = Upload(T.smoothed);
        dt.fnAnims = Upload(T.fnAnims);
        dt.fnOffset = Upload(T.fnOffset);
        dt.crude = Upload(T.crude);
        dt.crudeByIndex = Upload(T.crudeByIndex);
        dt.crudeVelocity = Upload(T.crudeVelocity);
        dt.crudeVelocityOffset = Upload(T.crudeVelocityOffset);
        dt.crudeBody = Upload(T.crudeBody);
        dt.crudeBodyOffset = Upload(T.crudeBodyOffset);
        dt.cameraWeights = Upload(T.cameraWeights);
        dt.idleMovement = Upload(T.idleMovement);
        dt.idleMovementCount = (int32_t)T.idleMovement.size();
        const Tables *dTables = Upload(&dt, 1);

        std::vector<Ctx> contexts;
        std::vector<const World *> templates;
        int agents = 0;
        for (const auto &bundle : bundles_) {
            if (bundle->leftAgents < 0 || bundle->rightAgents < 0 || bundle->leftAgents + bundle->rightAgents > kMaxAgents)
                throw std::runtime_error("expected at most 22 agents in a bundle");
            agents = std::max(agents, bundle->leftAgents + bundle->rightAgents);
            for (const Variant &v : bundle->variants) {
                Ctx c{};
                c.t = dTables;
                c.sd = Upload(&v.staticData, 1);
                c.skeletons = Upload(v.skeletons);
                c.ticksPerStep = cfg.ticksPerStep;
                c.ws = nullptr;
                contexts.push_back(c);
                templates.push_back(Upload(v.world.get(), 1));
                const Scenario &sc = v.world->scenario;
                players_ = std::max({players_, sc.leftTeamSize, sc.rightTeamSize});
                if (sc.controlAllPlayers && DynamicPlayerSelection(*v.world))
                    throw std::invalid_argument("a scenario with control_all_players needs 0 or all of the controllable players of a side as agents");
                // The per-second position history of a player holds 512 entries.
                const int64_t seconds = (int64_t)sc.gameDuration * cfg.ticksPerStep / 100 + 1;
                if (seconds > 512) throw std::invalid_argument("a match longer than the position history of a player");
            }
        }
        b_.contexts = Upload(contexts);
        b_.templates = Upload(templates);
        b_.count = count;
        b_.agents = agents;
        b_.actionSet = cfg.actionSet;
        b_.observation = cfg.observation;
        b_.checkpoints = cfg.checkpoints;
        b_.numpyLegacy = cfg.numpyLegacy;
        b_.autoReset = cfg.autoReset;
        b_.stack = cfg.stack;
        b_.worlds = Alloc<World>(count);
        b_.cores = Alloc<EnvCore>(count);
        b_.slots = Alloc<EnvSlot>(count);
        b_.scratch = Alloc<Scratch>(count);
        b_.reward = Alloc<float>((size_t)count * agents);
        b_.done = Alloc<uint8_t>(count);
        b_.scoreReward = Alloc<int32_t>(count);
        if (cfg.observation & (kObsSimple115 | kObsSimple115v2)) {
            b_.simple115 = Alloc<float>((size_t)count * agents * kSimple115 * cfg.stack);
            b_.finalSimple115 = Alloc<float>((size_t)count * agents * kSimple115 * cfg.stack);
        }
        b_.smmWidth = cfg.smmWidth;
        b_.smmHeight = cfg.smmHeight;
        if (cfg.observation & kObsSmm) {
            const size_t maps = (size_t)count * agents * cfg.smmWidth * cfg.smmHeight * kSmmLayers * cfg.stack;
            const size_t rows = (size_t)count * agents * kSmmMarkRow * cfg.stack;
            b_.smm = Alloc<uint8_t>(maps);
            b_.finalSmm = Alloc<uint8_t>(maps);
            b_.smmMarks = Alloc<int32_t>(rows);
            b_.finalSmmMarks = Alloc<int32_t>(rows);
        }
        if (cfg.observation & kObsRaw) {
            b_.rawLayout = MakeRawLayout((size_t)count * agents, players_, StickyActionCount(cfg.actionSet));
            b_.raw = Alloc<uint8_t>(b_.rawLayout.bytes);
            b_.finalRaw = Alloc<uint8_t>(b_.rawLayout.bytes);
        }
        b_.teamDifficulty = nullptr;
        if (!dev_->HostMemory()) actions_ = Alloc<int32_t>((size_t)count * agents);
        seeds_ = Alloc<int64_t>(count);
        reverse_ = Alloc<int32_t>(count);
        mask_ = Alloc<uint8_t>(count);
        slots_.resize(count);
        std::vector<uint8_t> agentMask((size_t)count * agents, 0);
        for (int e = 0; e < count; e++) {
            EnvSlot &s = slots_[e];
            memset(&s, 0, sizeof(EnvSlot));
            SeedEpisodeGenerator(s.gen, cfg.seed, (uint32_t)(cfg.firstIndex + e));
            s.fixedSeed = cfg.fixedSeeds.empty() ? -1 : cfg.fixedSeeds[e];
            s.episodeOffset = cfg.episodeNumber;
            s.bundle = assignment[e];
            s.leftAgents = bundles_[s.bundle]->leftAgents;
            s.rightAgents = bundles_[s.bundle]->rightAgents;
            for (int a = 0; a < s.leftAgents + s.rightAgents; a++) agentMask[(size_t)e * agents + a] = 1;
        }
        dev_->ToDevice(b_.slots, slots_.data(), sizeof(EnvSlot) * count);
        agentMask_ = Upload(agentMask);
        started_.assign(count, false);
        unstarted_ = count;
    } catch (...) {
        for (void *p : owned_) {
            if (UsesCallerAllocator()) cfg_.release(p, cfg_.allocatorContext);
            else dev_->Release(p);
        }
        owned_.clear();
        throw;
    }
}

BatchRuntime::~BatchRuntime() {
    // Blocks go back to a caller's allocator, which may hand them out at once, so every stream that
    // may still run this batch's work (a caller's non-blocking stream among them) must be idle.
    try {
        dev_->SynchronizeAll();
    } catch (...) {
    }
    for (void *p : owned_) {
        if (UsesCallerAllocator()) cfg_.release(p, cfg_.allocatorContext);
        else dev_->Release(p);
    }
}

bool BatchRuntime::UsesCallerAllocator() const { return cfg_.allocate != nullptr && !dev_->HostMemory(); }

void *BatchRuntime::AllocateBytes(size_t bytes) {
    void *p = nullptr;
    if (UsesCallerAllocator()) {
        p = cfg_.allocate(bytes, cfg_.allocatorContext);
        if (!p) throw std::runtime_error("the allocator of the configuration has no " + std::to_string(bytes) + " bytes of device memory");
        owned_.push_back(p);
        dev_->Fill(p, 0, bytes);
    } else {
        p = dev_->Allocate(bytes);
        owned_.push_back(p);
    }
    allocated_ += bytes;
    return p;
}

namespace {
class SizingDevice : public Device {
public:
    explicit SizingDevice(bool hostMemory) : hostMemory_(hostMemory) {}
    const char *Name() const override { return "sizing"; }
    // As the library's own device: a device in host memory stages no actions.
    bool HostMemory() const override { return hostMemory_; }
    // Every block is the same placeholder: nothing reads or writes it.
    void *Allocate(size_t) override { return &placeholder_; }
    void Release(void *) override {}
    void ToDevice(void *, const void *, size_t) override {}
    void ToHost(void *, const void *, size_t) override { throw std::logic_error("a sizing device holds no data"); }
    void ToDeviceAsync(void *, const void *, size_t, void *) override {}
    void Fill(void *, int, size_t) override {}
    void Synchronize(void *) override {}
    void Reset(const Batch &, const uint8_t *, const int64_t *, const int32_t *, void *) override {}
    void Step(const Batch &, const int32_t *, void *) override {}
    void Outputs(const Batch &, int, void *) override {}
    void CheckFault() override {}

private:
    bool hostMemory_;
    alignas(256) unsigned char placeholder_[256] = {};
};
}  // namespace

std::unique_ptr<Device> MakeSizingDevice(bool hostMemory) { return std::make_unique<SizingDevice>(hostMemory); }

int BatchRuntime::LeftPlayers(int env) const { return VariantAt(slots_[env].bundle * 4).world->scenario.leftTeamSize; }
int BatchRuntime::RightPlayers(int env) const { return VariantAt(slots_[env].bundle * 4).world->scenario.rightTeamSize; }

void BatchRuntime::CheckStarted() const {
    if (unstarted_ > 0) throw std::logic_error("expected a reset of the batch, or a state for every environment, before its first step");
}
void BatchRuntime::CheckEnvironment(int env) const {
    if (env < 0 || env >= b_.count)
        throw std::invalid_argument("expected an environment from 0 to " + std::to_string(b_.count - 1) + ", found " + std::to_string(env));
}

void BatchRuntime::Reset(const uint32_t *seeds, const int32_t *reverse, void *stream) {
    const int n = b_.count;
    const int64_t *ds = nullptr;
    const int32_t *dr = nullptr;
    if (seeds) {
        std::vector<int64_t> wide(seeds, seeds + n);
        dev_->ToDevice(seeds_, wide.data(), sizeof(int64_t) * n);
        ds = seeds_;
    }
    if (reverse) {
        for (int e = 0; e < n; e++)
            if (reverse[e] != 0 && reverse[e] != 1) throw std::invalid_argument("the reverse flag of environment " + std::to_string(e) + " is not 0 or 1");
        dev_->ToDevice(reverse_, reverse, sizeof(int32_t) * n);
        dr = reverse_;
    }
    dev_->Reset(b_, nullptr, ds, dr, stream);
    dev_->Synchronize(stream);
    dev_->CheckFault();
    started_.assign(n, true);
    unstarted_ = 0;
}

void BatchRuntime::ResetMasked(const uint8_t *mask, bool maskOnDevice, const int64_t *seeds, const int32_t *reverse, void *stream) {
    const int n = b_.count;
    if (seeds)
        for (int e = 0; e < n; e++)
            if (seeds[e] < -1 || seeds[e] > 4294967295LL)
                throw std::invalid_argument("expected seeds from 0 to 4294967295, or -1 to draw, found " + std::to_string(seeds[e]) +
                                            " for environment " + std::to_string(e));
    if (reverse)
        for (int e = 0; e < n; e++)
            if (reverse[e] != 0 && reverse[e] != 1) throw std::invalid_argument("the reverse flag of environment " + std::to_string(e) + " is not 0 or 1");
    // Host arrays are copied on the stream before the launch reads them; the call waits for those
    // copies, so the caller may free its arrays on return.
    const uint8_t *dm = mask;
    if (mask && !maskOnDevice) {
        dev_->ToDeviceAsync(mask_, mask, n, stream);
        dm = mask_;
    }
    const int64_t *ds = nullptr;
    const int32_t *dr = nullptr;
    if (seeds) {
        dev_->ToDeviceAsync(seeds_, seeds, sizeof(int64_t) * n, stream);
        ds = seeds_;
    }
    if (reverse) {
        dev_->ToDeviceAsync(reverse_, reverse, sizeof(int32_t) * n, stream);
        dr = reverse_;
    }
    if (unstarted_ > 0) {
        std::vector<uint8_t> started(n, 1);
        if (mask && maskOnDevice && !dev_->HostMemory()) {
            dev_->Synchronize(stream);
            dev_->ToHost(started.data(), mask, n);
        } else if (mask) {
            started.assign(mask, mask + n);
        }
        for (int e = 0; e < n; e++)
            if (started[e] && !started_[e]) {
                started_[e] = true;
                unstarted_--;
            }
    }
    dev_->Reset(b_, dm, ds, dr, stream);
    if ((mask && !maskOnDevice) || seeds || reverse) dev_->Synchronize(stream);
}

void BatchRuntime::ResetDone(void *stream) {
    CheckStarted();
    dev_->Reset(b_, b_.done, nullptr, nullptr, stream);
}

void BatchRuntime::Step(const int32_t *actions, bool onDevice, void *stream, bool synchronize) {
    CheckStarted();
    const int n = ActionSetSize(b_.actionSet);
    if (!onDevice || dev_->HostMemory()) {
        // GRF: an action indexes a Python list, which raises outside [-n, n).
        for (int e = 0; e < b_.count; e++) {
            const int32_t *row = actions + (size_t)e * b_.agents;
            for (int a = 0; a < slots_[e].leftAgents + slots_[e].rightAgents; a++)
                if (row[a] < -n || row[a] >= n)
                    throw std::out_of_range("expected action indices from " + std::to_string(-n) + " to " + std::to_string(n - 1) +
                                            ", found " + std::to_string(row[a]));
        }
    }
    const int32_t *da = actions;
    if (!onDevice && !dev_->HostMemory()) {
        dev_->ToDeviceAsync(actions_, actions, sizeof(int32_t) * b_.count * b_.agents, stream);
        da = actions_;
    }
    dev_->Step(b_, da, stream);
    if (synchronize || (!onDevice && !dev_->HostMemory())) {
        dev_->Synchronize(stream);
        dev_->CheckFault();
    }
}

void BatchRuntime::StepWithStaticScratch(const int32_t *actions, void *stream) {
    CheckStarted();
    int capacity = 0;
    Scratch *scratch = dev_->StaticScratch(&capacity);
    if (!scratch) throw std::logic_error("expected a device with a static scratch array for a step that allocates nothing");
    if (b_.count > capacity)
        throw std::invalid_argument("expected at most " + std::to_string(capacity) +
                                    " environments for a step that allocates nothing, found " + std::to_string(b_.count));
    Batch b = b_;
    b.scratch = scratch;
    dev_->Step(b, actions, stream);
}

void BatchRuntime::Synchronize(void *stream) {
    dev_->Synchronize(stream);
    dev_->CheckFault();
}

void BatchRuntime::SetDifficulty(const float *difficulty) {
    const size_t n = (size_t)b_.count * 2;
    for (size_t i = 0; i < n; i++)
        if (!(difficulty[i] <= 1)) throw std::invalid_argument("expected a difficulty from 0 to 1, found " + std::to_string(difficulty[i]));
    if (!b_.teamDifficulty) b_.teamDifficulty = Alloc<float>(n);
    dev_->ToDevice(const_cast<float *>(b_.teamDifficulty), difficulty, n * sizeof(float));
    hostDifficulty_.assign(difficulty, difficulty + n);
}

float BatchRuntime::Difficulty(int env, int side) const {
    if (!hostDifficulty_.empty() && hostDifficulty_[env * 2 + side] >= 0.0f) return hostDifficulty_[env * 2 + side];
    // GRF: episode_number is the episode before the first, so its parity is the first's.
    const Scenario &sc = VariantAt(slots_[env].bundle * 4 + (cfg_.episodeNumber & 1)).world->scenario;
    return side == 0 ? sc.leftDifficulty : sc.rightDifficulty;
}

void BatchRuntime::Episode(int env, long long *values, float *difficulty) {
    CheckEnvironment(env);
    dev_->Synchronize(nullptr);
    dev_->CheckFault();
    auto slot = std::make_unique<EnvSlot>();
    dev_->ToHost(slot.get(), b_.slots + env, sizeof(EnvSlot));
    auto obs = std::make_unique<Observation>();
    dev_->ToHost(obs.get(), &b_.cores[env].obs, sizeof(Observation));
    // The variant without reverse processing orders the teams as the observation does.
    const Scenario &sc = VariantAt(slot->bundle * 4).world->scenario;
    const long long out[17] = {slot->seed, slot->reverse, slot->episode, slot->episodeOffset, slot->bundle, obs->step,
                               slot->fixedSeed, sc.deterministic, cfg_.ticksPerStep, slot->leftAgents, slot->rightAgents,
                               sc.leftTeamSize, sc.rightTeamSize, obs->team[0].designatedPlayer, obs->team[1].designatedPlayer,
                               slot->finalDesignated[0], slot->finalDesignated[1]};
    memcpy(values, out, sizeof(out));
    if (difficulty) {
        dev_->ToHost(&difficulty[0], &b_.worlds[env].scenario.leftDifficulty, sizeof(float));
        dev_->ToHost(&difficulty[1], &b_.worlds[env].scenario.rightDifficulty, sizeof(float));
        const Scenario &own = VariantAt(slot->variant).world->scenario;
        difficulty[2] = own.leftDifficulty;
        difficulty[3] = own.rightDifficulty;
    }
}

const char *BatchRuntime::ScenarioName(int bundle) const {
    if (bundle < 0 || bundle >= (int)bundles_.size()) return nullptr;
    return bundles_[bundle]->scenario.c_str();
}

std::string BatchRuntime::GetState(int env, int *episode) {
    CheckEnvironment(env);
    dev_->Synchronize(nullptr);
    dev_->CheckFault();
    auto w = std::make_unique<World>();
    auto core = std::make_unique<EnvCore>();
    auto slot = std::make_unique<EnvSlot>();
    dev_->ToHost(w.get(), b_.worlds + env, sizeof(World));
    dev_->ToHost(core.get(), b_.cores + env, sizeof(EnvCore));
    dev_->ToHost(slot.get(), b_.slots + env, sizeof(EnvSlot));
    StateCodec codec;
    codec.freeControllerCount = VariantAt(slot->variant).freeControllerCount;
    std::string bytes = codec.SaveFrame(*w, 0);
    if (episode) {
        episode[0] = core->prevScoreDiff;
        episode[1] = core->prevGameMode;
        episode[2] = core->prevBallOwnedTeam;
        for (int a = 0; a < b_.agents; a++) episode[3 + a] = slot->collected[a];
    }
    return bytes;
}

void BatchRuntime::SetState(int env, const std::string &bytes, int prevScoreDiff, int prevGameMode, int prevBallOwnedTeam,
                            const int32_t *collected) {
    CheckEnvironment(env);
    dev_->Synchronize(nullptr);
    dev_->CheckFault();
    auto w = std::make_unique<World>();
    StateCodec codec;
    codec.animationCount = (int)tables_->anims.size();
    const int bundle = slots_[env].bundle;
    if (!codec.LoadFrame(bytes, 0, *w)) throw std::invalid_argument("expected the bytes of a state, found bytes that do not load");
    // GRF compares scenarios without `real_time`, so the bundle's stands in for the comparison.
    const bool realTime = w->scenario.realTime;
    w->scenario.realTime = bundles_[bundle]->variants[0].world->scenario.realTime;
    const std::string key = ScenarioKey(*w);
    int index = 0;
    while (index < 4 && bundles_[bundle]->variants[index].scenario != key) index++;
    if (index == 4) throw std::invalid_argument("expected a state of the scenario of the environment, found another");
    w->scenario.realTime = realTime;
    // An environment continues a state only under the difficulties it plays.
    const Scenario &expected = bundles_[bundle]->variants[index].world->scenario;
    float want[2] = {expected.leftDifficulty, expected.rightDifficulty};
    for (int side = 0; side < 2; side++)
        if (!hostDifficulty_.empty() && hostDifficulty_[env * 2 + side] >= 0.0f) want[side] = hostDifficulty_[env * 2 + side];
    if (memcmp(&w->scenario.leftDifficulty, &want[0], 4) != 0 || memcmp(&w->scenario.rightDifficulty, &want[1], 4) != 0)
        throw std::invalid_argument("expected a state of the difficulties of the environment, " + std::to_string(want[0]) + " and " +
                                    std::to_string(want[1]) + ", found " + std::to_string(w->scenario.leftDifficulty) + " and " +
                                    std::to_string(w->scenario.rightDifficulty));
    const int variant = bundle * 4 + index;
    const Variant &v = VariantAt(variant);
    const Tables hostTables = tables_->View();
    Ctx c{};
    c.t = &hostTables;
    c.sd = &v.staticData;
    c.skeletons = v.skeletons.data();
    c.ticksPerStep = cfg_.ticksPerStep;
    auto core = std::make_unique<EnvCore>();
    memset(core.get(), 0, sizeof(EnvCore));
    core->prevScoreDiff = prevScoreDiff;
    core->prevGameMode = prevGameMode;
    core->prevBallOwnedTeam = prevBallOwnedTeam;
    Observe(*w, c, core->obs);
    auto slot = std::make_unique<EnvSlot>();
    dev_->ToHost(slot.get(), b_.slots + env, sizeof(EnvSlot));
    slot->variant = variant;
    const int agents = slot->leftAgents + slot->rightAgents;
    for (int a = 0; a < kMaxAgents; a++) slot->collected[a] = collected && a < agents ? collected[a] : 0;
    for (int a = 0; a < agents; a++) {
        const bool left = a < slot->leftAgents;
        StickyActions(*w, b_.actionSet, left, left ? a : a - slot->leftAgents, slot->sticky[a]);
    }
    // A sent-off keeper's replacement lives outside the state bytes, so it carries over.
    dev_->ToHost(w->formationOverride, b_.worlds[env].formationOverride, sizeof(w->formationOverride));
    dev_->ToDevice(b_.worlds + env, w.get(), sizeof(World));
    dev_->ToDevice(b_.cores + env, core.get(), sizeof(EnvCore));
    dev_->ToDevice(b_.slots + env, slot.get(), sizeof(EnvSlot));
    dev_->Fill(b_.reward + (size_t)env * b_.agents, 0, sizeof(float) * b_.agents);
    dev_->Fill(b_.done + env, 0, 1);
    dev_->Fill(b_.scoreReward + env, 0, sizeof(int32_t));
    dev_->Outputs(b_, env, nullptr);
    dev_->Synchronize(nullptr);
    dev_->CheckFault();
    if (!started_[env]) {
        started_[env] = true;
        unstarted_--;
    }
}

void BatchRuntime::SetStack(int env, const std::string &name, const void *frames, size_t bytes) {
    CheckEnvironment(env);
    if (b_.stack < 2) throw std::invalid_argument("expected a batch that stacks its observations");
    const size_t agents = (size_t)(slots_[env].leftAgents + slots_[env].rightAgents);
    auto checkBytes = [&](size_t expected) {
        if (bytes != expected)
            throw std::invalid_argument("expected a stack of " + std::to_string(expected) + " bytes for the agents of environment " +
                                        std::to_string(env) + ", found " + std::to_string(bytes));
    };
    if (name == "simple115" && b_.simple115) {
        const size_t width = (size_t)kSimple115 * b_.stack;
        checkBytes(agents * width * sizeof(float));
        dev_->Synchronize(nullptr);
        dev_->ToDevice(b_.simple115 + (size_t)env * b_.agents * width, frames, bytes);
        return;
    }
    if (name != "smm" || !b_.smm) throw std::invalid_argument("expected the stack simple115 or smm of the batch, found " + name);
    // A minimap is zero but for its marks, and each frame keeps the list of its marks so that the
    // next step erases exactly them: rebuild those lists from the cells of 255.
    const size_t cells = (size_t)b_.smmWidth * b_.smmHeight * kSmmLayers;  // marks of one frame
    const size_t agentBytes = cells * b_.stack;
    checkBytes(agents * agentBytes);
    const uint8_t *in = static_cast<const uint8_t *>(frames);
    const int rowsPerAgent = kSmmMarkRow * b_.stack;
    std::vector<int32_t> marks(agents * rowsPerAgent, 0);
    for (size_t a = 0; a < agents; a++)
        for (int f = 0; f < b_.stack; f++) {
            int32_t *row = marks.data() + a * rowsPerAgent + f * kSmmMarkRow;
            for (size_t m = 0; m < cells; m++) {
                const uint8_t v = in[a * agentBytes + (m / kSmmLayers) * kSmmLayers * b_.stack + kSmmLayers * f + m % kSmmLayers];
                if (v == 0) continue;
                if (v != 255 || row[0] == kSmmMarks)
                    throw std::invalid_argument("expected a minimap of GRF, zeros and at most " + std::to_string(kSmmMarks) +
                                                " cells of 255 a frame, found a cell of " + std::to_string(v));
                row[1 + row[0]++] = (int32_t)m;
            }
        }
    dev_->Synchronize(nullptr);
    dev_->ToDevice(b_.smm + (size_t)env * b_.agents * agentBytes, frames, bytes);
    dev_->ToDevice(b_.smmMarks + (size_t)env * b_.agents * rowsPerAgent, marks.data(), marks.size() * sizeof(int32_t));
}

// GRF's raw keys, in the order of the arrays (observation.py).
static const char *const kRawFieldNames[kRawFields] = {
    "ball", "ball_direction", "ball_rotation", "ball_owned_team", "ball_owned_player",
    "left_team", "left_team_direction", "left_team_tired_factor", "left_team_yellow_card", "left_team_active", "left_team_roles",
    "right_team", "right_team_direction", "right_team_tired_factor", "right_team_yellow_card", "right_team_active", "right_team_roles",
    "score", "steps_left", "game_mode", "active", "designated", "sticky_actions"};

RawLayout MakeRawLayout(size_t outputs, int players, int sticky) {
    RawLayout L{};
    L.players = players;
    L.sticky = sticky;
    auto set = [&](int field, int type, int d0, int d1) {
        L.type[field] = type;
        L.shape[field][0] = d0;
        L.shape[field][1] = d1;
        L.elements[field] = (d0 ? d0 : 1) * (d1 ? d1 : 1);
    };
    for (int f : {kRawBall, kRawBallDirection, kRawBallRotation}) set(f, kRawFloat32, 3, 0);
    set(kRawBallOwnedTeam, kRawInt32, 0, 0);
    set(kRawBallOwnedPlayer, kRawInt32, 0, 0);
    for (int base : {kRawLeftTeam, kRawRightTeam}) {
        set(base, kRawFloat32, players, 2);
        set(base + 1, kRawFloat32, players, 2);
        set(base + 2, kRawFloat32, players, 0);
        set(base + 3, kRawBool, players, 0);
        set(base + 4, kRawBool, players, 0);
        set(base + 5, kRawInt32, players, 0);
    }
    set(kRawScore, kRawInt32, 2, 0);
    for (int f : {kRawStepsLeft, kRawGameMode, kRawActive, kRawDesignated}) set(f, kRawInt32, 0, 0);
    set(kRawStickyActions, kRawUint8, sticky, 0);
    uint64_t offset = 0;
    for (int f = 0; f < kRawFields; f++) {
        L.offset[f] = offset;
        offset += (outputs * L.elements[f] * RawTypeBytes(L.type[f]) + 255) / 256 * 256;
    }
    L.bytes = offset;
    return L;
}

const char *BatchRuntime::RawField(int field, int *type, int *dimensions, unsigned long long *offset) const {
    if (!b_.raw || field < 0 || field >= kRawFields) return nullptr;
    *type = b_.rawLayout.type[field];
    dimensions[0] = b_.rawLayout.shape[field][0];
    dimensions[1] = b_.rawLayout.shape[field][1];
    *offset = b_.rawLayout.offset[field];
    return kRawFieldNames[field];
}

void *BatchRuntime::Buffer(const std::string &name) {
    if (name == "simple115") return b_.simple115;
    if (name == "final_simple115") return b_.finalSimple115;
    if (name == "smm") return b_.smm;
    if (name == "final_smm") return b_.finalSmm;
    if (name == "raw") return b_.raw;
    if (name == "final_raw") return b_.finalRaw;
    if (name == "reward") return b_.reward;
    if (name == "done") return b_.done;
    if (name == "score_reward") return b_.scoreReward;
    if (name == "agent_mask") return agentMask_;
    return nullptr;
}


}  // namespace host
}  // namespace eng
