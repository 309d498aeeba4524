// The MI355X device of the batch runtime: device memory, copies and the kernels (reset, step and
// the outputs of one environment).
//
// Geometry. Each environment runs on a group of ENG_GROUP_LANES adjacent lanes (engine/hd.h), and a
// workgroup of one wavefront holds `matches_` environments. A step's cost is the wavefront's: its
// matches' divergent control flow runs one path after another (16 identical matches step in a
// quarter of the time of 16 ordinary ones), and a match's own sequential chain of dependent loads
// sets a floor that wider groups lower, since the loops of independent iterations split over the
// group. This file is compiled once per group width (2, 4, 8, 16, 32 and 64 lanes), each copy with its own
// kernels, fault words and device class.
//
// Occupancy. The step kernel is bounded to the registers of two wavefronts per SIMD (256 VGPRs,
// none spilled to AGPRs: -mllvm -amdgpu-spill-vgpr-to-agpr=0), so two wavefronts share each SIMD
// and each hides the other's memory latency; unbounded, the kernel takes 256 VGPRs and 58 AGPRs,
// one wavefront per SIMD. MakeLibraryDevice (the copy built with ENG_PRIMARY_VARIANT) picks the
// geometry per batch: as many matches per wavefront as fill every SIMD with two wavefronts, at most
// 32, and the widest group those matches leave room for. Measured on gfx950, ms per step after 100
// steps, one wavefront per SIMD against two: 4,096 environments of 11-a-side 118.5 at 16 lanes x 4
// matches against 103.6 at 16 x 2; 8,192 of 11-a-side self-play 172.4 at 8 x 8 against 144.4 at
// 16 x 4; 16,384 of 11-a-side 258.6 at 4 x 16 against 206.1 at 8 x 8 (205.6 at 8 x 6 with three
// wavefronts per SIMD); 32,768 of the mixed batch 342.8 at 2 x 32 against 245.2 at 4 x 16. The
// bound itself costs nothing: 257.7 at 4 x 16 with one wavefront per SIMD. 64 environments of
// 5-a-side take 20.6 at 16 x 1 either way.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "host/runtime.h"

#ifndef ENG_DEVICE_FACTORY
#error "each build of the device names its factory (ENG_DEVICE_FACTORY)"
#endif

namespace eng {
namespace host {
std::unique_ptr<Device> ENG_DEVICE_FACTORY(int matches);
// The static scratch array of the step that allocates nothing, on the current device (defined by
// the primary build, which owns the array).
Scratch *StaticScratchOfCurrentDevice(int *environments);
}  // namespace host
}  // namespace eng

namespace {

__device__ int32_t gFaultEnvironment;

// A workgroup is one wavefront. The launch geometry is host code, where the engine's own
// eng::kGroupLanes is the host's single lane, so it reads the device group size from the macro
// both compilation passes share.
constexpr int kWaveLanes = 64;
// Wavefronts each SIMD must be able to hold, which bounds the registers of a lane.
#ifndef ENG_WAVES_PER_SIMD
#define ENG_WAVES_PER_SIMD 2
#endif
constexpr int kDeviceGroupLanes = ENG_GROUP_LANES;
constexpr int kMaxMatches = kWaveLanes / kDeviceGroupLanes;
#if defined(__HIP_DEVICE_COMPILE__)
static_assert(eng::kGroupLanes == kDeviceGroupLanes, "the launch and the engine agree on the lanes of a match");
#endif

__device__ void RecordFault(int env) {
    if (eng::gEngineFault == 0) eng::gEngineFault = 1;
    atomicMin(&gFaultEnvironment, env);
}

__device__ int MatchIndex() { return (int)(blockIdx.x * (blockDim.x / kDeviceGroupLanes) + threadIdx.x / kDeviceGroupLanes); }

// The batch description, the kernels' first argument, read where the launch placed it: at the
// start of the kernel argument segment. A reference to the by-value parameter itself would make
// every lane copy its 752 bytes onto its stack first.
__device__ const eng::Batch &LaunchBatch() {
#if defined(__HIP_DEVICE_COMPILE__)
    // A constant-segment address is the same number as a generic one.
    return *reinterpret_cast<const eng::Batch *>((uintptr_t)__builtin_amdgcn_kernarg_segment_ptr());
#else
    return *static_cast<const eng::Batch *>(nullptr);
#endif
}

__global__ void __launch_bounds__(kWaveLanes, ENG_WAVES_PER_SIMD) ResetKernel(eng::Batch, const uint8_t *mask, const int64_t *seeds,
                                                                      const int32_t *reverse) {
    const eng::Batch &b = LaunchBatch();
    eng::libm::StageMathTables();
    const int env = MatchIndex();
    if (env >= b.count) return;
    if (mask && !mask[env]) return;
    if (!eng::ResetAndWriteEnvironment(b, env, seeds, reverse)) RecordFault(env);
}

__global__ void __launch_bounds__(kWaveLanes, ENG_WAVES_PER_SIMD) StepKernel(eng::Batch, const int32_t *actions) {
    const eng::Batch &b = LaunchBatch();
    eng::libm::StageMathTables();
    const int env = MatchIndex();
    if (env >= b.count) return;
    if (!eng::StepEnvironment(b, env, actions)) RecordFault(env);
}

__global__ void __launch_bounds__(kDeviceGroupLanes) OutputKernel(eng::Batch, int env) {
    const eng::Batch &b = LaunchBatch();
    eng::libm::StageMathTables();
    eng::WriteEnvironmentOutputs(b, env, false);
}

void Check(hipError_t e, const char *what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

class HipDevice : public eng::host::Device {
public:
    explicit HipDevice(int matches) : matches_(std::max(1, std::min(kMaxMatches, matches))) {
        int n = 0;
        Check(hipGetDeviceCount(&n), "hipGetDeviceCount");
        if (n < 1) throw std::runtime_error("no HIP device");
        ClearFault();
        // The batch is created with its device current: look the static scratch up now, so the
        // step that allocates nothing makes no runtime call besides its launch.
        staticScratch_ = eng::host::StaticScratchOfCurrentDevice(&staticScratchEnvironments_);
    }
    const char *Name() const override { return "hip"; }
    bool HostMemory() const override { return false; }
    void *Allocate(size_t n) override {
        void *p = nullptr;
        Check(hipMalloc(&p, n), "hipMalloc");
        Check(hipMemset(p, 0, n), "hipMemset");
        return p;
    }
    void Release(void *p) override { (void)hipFree(p); }
    void ToDevice(void *d, const void *s, size_t n) override { Check(hipMemcpy(d, s, n, hipMemcpyHostToDevice), "hipMemcpy"); }
    void ToHost(void *d, const void *s, size_t n) override { Check(hipMemcpy(d, s, n, hipMemcpyDeviceToHost), "hipMemcpy"); }
    void ToDeviceAsync(void *d, const void *s, size_t n, void *stream) override {
        Check(hipMemcpyAsync(d, s, n, hipMemcpyHostToDevice, static_cast<hipStream_t>(stream)), "hipMemcpyAsync");
    }
    void Fill(void *d, int v, size_t n) override { Check(hipMemset(d, v, n), "hipMemset"); }
    void Synchronize(void *stream) override { Check(hipStreamSynchronize(static_cast<hipStream_t>(stream)), "hipStreamSynchronize"); }
    void SynchronizeAll() override { Check(hipDeviceSynchronize(), "hipDeviceSynchronize"); }
    void Reset(const eng::Batch &b, const uint8_t *mask, const int64_t *seeds, const int32_t *reverse, void *stream) override {
        const int blocks = (b.count + matches_ - 1) / matches_;
        hipLaunchKernelGGL(ResetKernel, dim3(blocks), dim3(matches_ * kDeviceGroupLanes), 0, static_cast<hipStream_t>(stream), b,
                           mask, seeds, reverse);
        Check(hipGetLastError(), "reset launch");
    }
    void Step(const eng::Batch &b, const int32_t *actions, void *stream) override {
        const int blocks = (b.count + matches_ - 1) / matches_;
        hipLaunchKernelGGL(StepKernel, dim3(blocks), dim3(matches_ * kDeviceGroupLanes), 0, static_cast<hipStream_t>(stream), b,
                           actions);
        Check(hipGetLastError(), "step launch");
    }
    void Outputs(const eng::Batch &b, int env, void *stream) override {
        if (env < 0 || env >= b.count) throw std::out_of_range("no environment " + std::to_string(env));
        hipLaunchKernelGGL(OutputKernel, dim3(1), dim3(kDeviceGroupLanes), 0, static_cast<hipStream_t>(stream), b, env);
        Check(hipGetLastError(), "output launch");
    }
    eng::Scratch *StaticScratch(int *environments) override {
        *environments = staticScratch_ ? staticScratchEnvironments_ : 0;
        return staticScratch_;
    }
    void CheckFault() override {
        uint32_t fault = 0;
        int32_t env = 0;
        Check(hipMemcpyFromSymbol(&fault, HIP_SYMBOL(eng::gEngineFault), sizeof(fault)), "hipMemcpyFromSymbol");
        if (!fault) return;
        Check(hipMemcpyFromSymbol(&env, HIP_SYMBOL(gFaultEnvironment), sizeof(env)), "hipMemcpyFromSymbol");
        ClearFault();
        throw std::runtime_error("environment " + std::to_string(env) + (fault == 2 ? " reached a state that no match reaches" : " reached a path that GRF leaves undefined"));
    }
    int Geometry(int *lanes) const override {
        *lanes = kDeviceGroupLanes;
        return matches_;
    }

private:
    int matches_;
    eng::Scratch *staticScratch_ = nullptr;
    int staticScratchEnvironments_ = 0;
    void ClearFault() {
        const uint32_t zero = 0;
        const int32_t none = 0x7fffffff;
        Check(hipMemcpyToSymbol(HIP_SYMBOL(eng::gEngineFault), &zero, sizeof(zero)), "hipMemcpyToSymbol");
        Check(hipMemcpyToSymbol(HIP_SYMBOL(gFaultEnvironment), &none, sizeof(none)), "hipMemcpyToSymbol");
    }
};

}  // namespace

namespace eng {
namespace host {
std::unique_ptr<Device> ENG_DEVICE_FACTORY(int matches) { return std::make_unique<HipDevice>(matches); }
}  // namespace host
}  // namespace eng

#if ENG_PRIMARY_VARIANT
namespace {

// The math routines over an index range, for the checks of tests: consecutive float bit patterns
// from `first` (kind 0), float arrays (kind 1) or double arrays (kind 2). Every lane reads the
// tables from its workgroup's LDS, as the step does.
constexpr int kLibmThreads = 256;
__global__ void __launch_bounds__(kLibmThreads) LibmKernel(int kind, int which, uint32_t first, long long count, const void *x,
                                                            const void *y, void *out) {
    eng::libm::StageMathTables();
    const long long stride = (long long)gridDim.x * blockDim.x;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
        if (kind == 0) {
            static_cast<float *>(out)[i] = eng::libm::EvaluateFloat(which, eng::FloatOf(first + (uint32_t)i), 0.0f);
        } else if (kind == 1) {
            static_cast<float *>(out)[i] =
                eng::libm::EvaluateFloat(which, static_cast<const float *>(x)[i], static_cast<const float *>(y)[i]);
        } else {
            static_cast<double *>(out)[i] =
                eng::libm::EvaluateDouble(which, static_cast<const double *>(x)[i], static_cast<const double *>(y)[i]);
        }
    }
}

// The working memory of the step that allocates nothing (cuju_environment_step_no_alloc): the
// per-environment Scratch blocks of at most kStaticScratchEnvironments environments, one copy on
// each GPU for the life of the process. Every such call on a GPU shares it: calls that overlap on
// one GPU race. Nothing in it needs to start at zero, since the step builds every list, plan, key
// array and time walk before reading it.
constexpr int kStaticScratchEnvironments = 64;
static __device__ __align__(256) unsigned char scratch[kStaticScratchEnvironments * sizeof(eng::Scratch)];

// The device address of `scratch` on each GPU. In host code the array's name stands in for the
// symbol only; its address on a device comes from hipGetSymbolAddress with that device current.
std::mutex gScratchMutex;
std::vector<void *> gScratchAddress;

}  // namespace

namespace eng {
namespace host {

Scratch *StaticScratchOfCurrentDevice(int *environments) {
    *environments = 0;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) {
        // Leave no error behind for the next launch check to report as its own.
        (void)hipGetLastError();
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(gScratchMutex);
    if ((int)gScratchAddress.size() <= device) gScratchAddress.resize(device + 1, nullptr);
    if (!gScratchAddress[device]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
        gScratchAddress[device] = p;
    }
    *environments = kStaticScratchEnvironments;
    return static_cast<Scratch *>(gScratchAddress[device]);
}

std::unique_ptr<Device> MakeHipDevice2(int matches);
std::unique_ptr<Device> MakeHipDevice4(int matches);
std::unique_ptr<Device> MakeHipDevice8(int matches);
std::unique_ptr<Device> MakeHipDevice16(int matches);
std::unique_ptr<Device> MakeHipDevice32(int matches);
std::unique_ptr<Device> MakeHipDevice64(int matches);

// Two wavefronts for each SIMD where the batch allows it: the matches of a wavefront are the
// environments over the wavefront slots, 1 to 32, and the group is the widest of 64, 32, 16, 8, 4
// or 2 lanes that those matches leave room for in 64 (measured on an MI355X: one match of 64 lanes
// steps 64 environments of 5-a-side in 17.7 ms at the median against 18.5 at 16 lanes; two of 32
// step 4,096 of 11-a-side in 88.5 ms against 90.4 at 2 x 16). CUJU_AMD_MATCHES sets the matches of
// a wavefront instead.
std::unique_ptr<Device> MakeLibraryDevice(int, int environments) {
    int device = 0, units = 0;
    Check(hipGetDevice(&device), "hipGetDevice");
    Check(hipDeviceGetAttribute(&units, hipDeviceAttributeMultiprocessorCount, device), "hipDeviceGetAttribute");
    const int slots = std::max(1, 4 * units * ENG_WAVES_PER_SIMD);
    int matches = (std::max(1, environments) + slots - 1) / slots;
    if (const char *v = getenv("CUJU_AMD_MATCHES")) matches = atoi(v);
    matches = std::max(1, std::min(32, matches));
    // CUJU_AMD_LANES sets the lanes of a match (2 to 64), and with it at most 64 / lanes matches.
    if (const char *v = getenv("CUJU_AMD_LANES")) {
        switch (atoi(v)) {
        case 64: return MakeHipDevice64(1);
        case 32: return MakeHipDevice32(std::min(matches, 2));
        case 16: return MakeHipDevice16(std::min(matches, 4));
        case 8: return MakeHipDevice8(std::min(matches, 8));
        case 4: return MakeHipDevice4(std::min(matches, 16));
        case 2: return MakeHipDevice2(matches);
        default: throw std::invalid_argument("CUJU_AMD_LANES must be 2, 4, 8, 16, 32 or 64");
        }
    }
    if (matches == 1) return MakeHipDevice64(1);
    if (matches == 2) return MakeHipDevice32(2);
    if (matches <= 4) return MakeHipDevice16(matches);
    if (matches <= 8) return MakeHipDevice8(matches);
    if (matches <= 16) return MakeHipDevice4(matches);
    return MakeHipDevice2(matches);
}

// torch names a HIP device "cuda" on ROCm; the reference binding compares this name with the
// device type it was asked for (python/cuju/_batch/library.py:217-222).
extern const char *const kBackendName = "cuda";
extern const bool kLibraryHostMemory = false;

}  // namespace host
}  // namespace eng

extern "C" __attribute__((visibility("default"))) int cuju_debug_libm_device(int kind, int which, unsigned int first,
                                                                            long long count, const void *x, const void *y,
                                                                            void *out, void *stream) {
    if (kind < 0 || kind > 2 || which < 0 || which > (kind == 2 ? 5 : 8) || count < 0 || !out || (kind != 0 && (!x || !y)))
        return -1;
    if (count == 0) return 0;
    const long long blocks = std::min<long long>((count + kLibmThreads - 1) / kLibmThreads, 8192);
    hipLaunchKernelGGL(LibmKernel, dim3((unsigned)blocks), dim3(kLibmThreads), 0, static_cast<hipStream_t>(stream), kind, which,
                       first, count, x, y, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
#endif
