// The batch runtime behind the C ABI: creation from bundles and animation tables, the buffers in
// device memory, resets, steps and state export. The work on the environments runs on a
// `Device`: the HIP device for the product, or the host (a debugging build of the same engine
// code that tests use to locate a divergence tick by tick).
// Semantics: include/cuju/batch/batch_environment.h:30-621, src/environment_api.h.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "assets.h"

namespace eng {
namespace host {

class Device {
public:
    virtual ~Device() = default;
    virtual const char *Name() const = 0;
    // True when device memory is host memory.
    virtual bool HostMemory() const = 0;
    // Zero-filled memory.
    virtual void *Allocate(size_t bytes) = 0;
    virtual void Release(void *p) = 0;
    virtual void ToDevice(void *dst, const void *src, size_t bytes) = 0;
    virtual void ToHost(void *dst, const void *src, size_t bytes) = 0;
    virtual void ToDeviceAsync(void *dst, const void *src, size_t bytes, void *stream) = 0;
    virtual void Fill(void *dst, int value, size_t bytes) = 0;
    virtual void Synchronize(void *stream) = 0;
    // Waits for all work on the device, whichever stream it was enqueued on.
    virtual void SynchronizeAll() { Synchronize(nullptr); }
    // Resets every environment whose mask byte is nonzero (all when `mask` is null). Arrays are in
    // device memory.
    virtual void Reset(const Batch &b, const uint8_t *mask, const int64_t *seeds, const int32_t *reverse, void *stream) = 0;
    virtual void Step(const Batch &b, const int32_t *actions, void *stream) = 0;
    // Writes the outputs of environment `env` after a reset or a loaded state.
    virtual void Outputs(const Batch &b, int env, void *stream) = 0;
    // Throws when a launch since the last check reached an undefined path.
    virtual void CheckFault() = 0;
    virtual int Threads() const { return 0; }
    // Environments per wavefront, and in `lanes` the lanes of each (1 and 1 off the GPU).
    virtual int Geometry(int *lanes) const {
        *lanes = 1;
        return 1;
    }
    // The device's own scratch array for a step that allocates nothing, and the environments it
    // holds; null when the device has none.
    virtual Scratch *StaticScratch(int *environments) {
        *environments = 0;
        return nullptr;
    }
};

struct Configuration {
    std::vector<std::string> assets;
    std::vector<int32_t> assignment;
    std::string animations;
    int count = 1;
    uint64_t seed = 0;
    int actionSet = 0;
    int observation = kObsSimple115v2;
    bool checkpoints = false, numpyLegacy = true, autoReset = true;
    int threads = 0;
    int ticksPerStep = 10;
    int smmWidth = 96, smmHeight = 72;
    int stack = 1;
    std::vector<int64_t> fixedSeeds;
    std::vector<int32_t> agentCounts;
    int episodeNumber = 0;
    int64_t firstIndex = 0;
    // Device memory from the caller's allocator (src/environment_api.h:81-86): `allocate` returns
    // null when it has none, and `release` gets each block back once the device is idle. Null
    // takes the device's own allocation.
    void *(*allocate)(size_t bytes, void *context) = nullptr;
    void (*release)(void *pointer, void *context) = nullptr;
    void *allocatorContext = nullptr;
};

// A device that holds no memory and runs nothing: a batch created on it checks its configuration,
// loads its bundles and tables on the host and counts the bytes it would allocate on a HIP device
// (src/environment_api.h:148-152, the reference's EstimateMemory).
// A device that allocates placeholders only, to size a batch: `hostMemory` as the library's device.
std::unique_ptr<Device> MakeSizingDevice(bool hostMemory);

// The raw arrays of `outputs` agent views in one buffer, each at a multiple of 256 bytes.
RawLayout MakeRawLayout(size_t outputs, int players, int sticky);

class BatchRuntime {
public:
    BatchRuntime(const Configuration &cfg, std::unique_ptr<Device> device);
    ~BatchRuntime();
    BatchRuntime(const BatchRuntime &) = delete;
    BatchRuntime &operator=(const BatchRuntime &) = delete;

    int Count() const { return b_.count; }
    int Agents() const { return b_.agents; }
    int LeftAgents(int env) const { return slots_[env].leftAgents; }
    int RightAgents(int env) const { return slots_[env].rightAgents; }
    int Players() const { return players_; }
    int LeftPlayers(int env) const;
    int RightPlayers(int env) const;
    size_t MemoryBytes() const { return allocated_; }
    Device &Dev() { return *dev_; }
    const Batch &Buffers() const { return b_; }

    void Reset(const uint32_t *seeds, const int32_t *reverse, void *stream);
    void ResetMasked(const uint8_t *mask, bool maskOnDevice, const int64_t *seeds, const int32_t *reverse, void *stream);
    void ResetDone(void *stream);
    void Step(const int32_t *actions, bool onDevice, void *stream, bool synchronize);
    // A step on device actions whose working memory is the device's static scratch array instead
    // of the batch's: it allocates nothing and waits for nothing.
    void StepWithStaticScratch(const int32_t *actions, void *stream);
    void Synchronize(void *stream);
    void SetDifficulty(const float *difficulty);
    float Difficulty(int env, int side) const;
    // The engine bytes of one environment; `episode` gets the score difference, game mode and
    // ball-owning team after the last step, then each agent's checkpoints.
    std::string GetState(int env, int *episode);
    // Loads engine bytes of GRF's state into environment `env` and writes its outputs; the reward
    // is 0 and done clear until the next step. `collected` may be null.
    void SetState(int env, const std::string &bytes, int prevScoreDiff, int prevGameMode, int prevBallOwnedTeam,
                  const int32_t *collected);
    // Writes the observation stack of environment `env`: `[agents][115 * stack]` floats, oldest
    // frame first.
    void SetStack(int env, const std::string &name, const void *frames, size_t bytes);
    // The current episode of environment `env`, synchronously: 17 values (seed, team order,
    // resets so far, episode_number, bundle, last observation's step, fixed seed or -1,
    // deterministic, ticks per step, agents, players and designated players per side, now and at
    // the last episode end) and, unless null, the played then the scenario's difficulties.
    void Episode(int env, long long *values, float *difficulty);
    // The scenario name bundle `bundle` records, or null past the last bundle.
    const char *ScenarioName(int bundle) const;
    // The buffer of an output name, or null.
    void *Buffer(const std::string &name);
    // Raw array `field`: its name, element type, the two dimensions after the agent axis (0 when
    // absent) and its byte offset into `raw` and `final_raw`; null past the last or without raw.
    const char *RawField(int field, int *type, int *dimensions, unsigned long long *offset) const;

private:
    // Zero-filled device memory, from the caller's allocator when the configuration names one.
    void *AllocateBytes(size_t bytes);
    bool UsesCallerAllocator() const;
    template <class T>
    T *Alloc(size_t n) {
        return static_cast<T *>(AllocateBytes(sizeof(T) * (n ? n : 1)));
    }
    template <class T>
    T *Upload(const T *src, size_t n) {
        T *d = Alloc<T>(n);
        if (n) dev_->ToDevice(d, src, sizeof(T) * n);
        return d;
    }
    template <class T>
    T *Upload(const std::vector<T> &v) {
        return Upload(v.data(), v.size());
    }
    const Variant &VariantAt(int v) const { return bundles_[v / 4]->variants[v % 4]; }
    void CheckStarted() const;
    void CheckEnvironment(int env) const;

    Configuration cfg_;
    std::unique_ptr<Device> dev_;
    std::vector<void *> owned_;
    size_t allocated_ = 0;
    std::vector<std::unique_ptr<Bundle>> bundles_;
    std::unique_ptr<AnimationTables> tables_;
    std::vector<EnvSlot> slots_;  // as created: bundles and agent counts
    std::vector<float> hostDifficulty_;
    std::vector<bool> started_;
    int unstarted_ = 0;
    int players_ = 0;
    Batch b_{};
    uint8_t *agentMask_ = nullptr;
    int32_t *actions_ = nullptr;
    int64_t *seeds_ = nullptr;
    int32_t *reverse_ = nullptr;
    uint8_t *mask_ = nullptr;
};

}  // namespace host
}  // namespace eng
