// The MI355X device of the batch runtime: device memory, copies and the kernels (reset, step and
// the outputs of one environment). Each environment runs on a group of kGroupLanes adjacent lanes
// (engine/hd.h), and a workgroup (one wavefront) holds `matches_` environments. A match is a long
// chain of dependent loads with data-dependent branches: one match per wavefront leaves the latency
// of each load exposed, while many matches per wavefront serialize on divergence. With one lane
// per match, 16 per wavefront measured best on gfx950 for the 11-a-side scenarios (1: 9.1k,
// 4: 16.9k, 16: 33.5k, 64: 22.9k env-steps/s at 16,384 environments, early steps); groups of four
// lanes fill the wavefront with the same 16 matches.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "host/runtime.h"

namespace eng {
__device__ uint32_t gEngineFault;
}  // namespace eng

namespace {

__device__ int32_t gFaultEnvironment;

// A workgroup is one wavefront. The launch geometry is host code, where the engine's own
// eng::kGroupLanes is the host's single lane, so it reads the device group size from the macro
// both compilation passes share.
constexpr int kWaveLanes = 64;
// Wavefronts each SIMD must be able to hold, which bounds the registers of a lane.
#ifndef ENG_WAVES_PER_SIMD
#define ENG_WAVES_PER_SIMD 1
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

__global__ void __launch_bounds__(kWaveLanes, ENG_WAVES_PER_SIMD) ResetKernel(eng::Batch b, const uint8_t *mask, const int64_t *seeds,
                                                                      const int32_t *reverse) {
    eng::libm::StageMathTables();
    const int env = MatchIndex();
    if (env >= b.count) return;
    if (mask && !mask[env]) return;
    if (!eng::ResetAndWriteEnvironment(b, env, seeds, reverse)) RecordFault(env);
}

__global__ void __launch_bounds__(kWaveLanes, ENG_WAVES_PER_SIMD) StepKernel(eng::Batch b, const int32_t *actions) {
    eng::libm::StageMathTables();
    const int env = MatchIndex();
    if (env >= b.count) return;
    if (!eng::StepEnvironment(b, env, actions)) RecordFault(env);
}

__global__ void __launch_bounds__(kDeviceGroupLanes) OutputKernel(eng::Batch b, int env) {
    eng::libm::StageMathTables();
    eng::WriteEnvironmentOutputs(b, env, false);
}

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

void Check(hipError_t e, const char *what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// The working memory of the step that allocates nothing (cuju_environment_step_no_alloc): the
// per-environment Scratch blocks of at most kStaticScratchEnvironments environments, 4.3 MB, one
// copy on each GPU for the life of the process. Every such call on a GPU shares it: calls that
// overlap on one GPU race. Nothing in it needs to start at zero, since the step builds every
// list, plan, key array and time walk before reading it.
constexpr int kStaticScratchEnvironments = 64;
static __device__ __align__(256) unsigned char scratch[kStaticScratchEnvironments * sizeof(eng::Scratch)];

// The device address of `scratch` on each GPU. In host code the array's name stands in for the
// symbol only; its address on a device comes from hipGetSymbolAddress with that device current.
std::mutex gScratchMutex;
std::vector<void *> gScratchAddress;

void *StaticScratchOfCurrentDevice() {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> lock(gScratchMutex);
    if ((int)gScratchAddress.size() <= device) gScratchAddress.resize(device + 1, nullptr);
    if (!gScratchAddress[device]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
        gScratchAddress[device] = p;
    }
    return gScratchAddress[device];
}

class HipDevice : public eng::host::Device {
public:
    HipDevice() {
        // Environments per workgroup, 1 to 64 / kGroupLanes.
        if (const char *v = getenv("CUJU_AMD_MATCHES")) matches_ = std::max(1, std::min(kMaxMatches, atoi(v)));
        int n = 0;
        Check(hipGetDeviceCount(&n), "hipGetDeviceCount");
        if (n < 1) throw std::runtime_error("no HIP device");
        ClearFault();
        // The batch is created with its device current: look the static scratch up now, so the
        // step that allocates nothing makes no runtime call besides its launch.
        staticScratch_ = static_cast<eng::Scratch *>(StaticScratchOfCurrentDevice());
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
        *environments = staticScratch_ ? kStaticScratchEnvironments : 0;
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

private:
    int matches_ = kMaxMatches < 16 ? kMaxMatches : 16;
    eng::Scratch *staticScratch_ = nullptr;
    void ClearFault() {
        const uint32_t zero = 0;
        const int32_t none = 0x7fffffff;
        Check(hipMemcpyToSymbol(HIP_SYMBOL(eng::gEngineFault), &zero, sizeof(zero)), "hipMemcpyToSymbol");
        Check(hipMemcpyToSymbol(HIP_SYMBOL(gFaultEnvironment), &none, sizeof(none)), "hipMemcpyToSymbol");
    }
};

}  // namespace

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

namespace eng {
namespace host {
std::unique_ptr<Device> MakeLibraryDevice(int) { return std::make_unique<HipDevice>(); }
// torch names a HIP device "cuda" on ROCm; the reference binding compares this name with the
// device type it was asked for (python/cuju/_batch/library.py:217-222).
extern const char *const kBackendName = "cuda";
}  // namespace host
}  // namespace eng
