// flint_bench: times Flint's kernels through the C ABI against the vendor
// libraries on one MI355X and writes a "flint-bench/1" JSON log (the
// reference's harness, ref bench/main.cpp:1-122, bench/harness.cpp:157-313,
// bench/report.cpp:488; its command line is in cli.cpp).
//
// Benchmarks:
//   copy  flint_copy against hipMemcpyAsync, bytes compared bit for bit.
//   mma   the v_mfma_f32_32x32x16_f16 ceiling loop (mfma_kernel.h), one-sided,
//         its exactly known result checked by the kernel itself.
//   gemm  flint_gemm_{nt,nn,tn} and the fused epilogues against rocBLAS
//         (rocblas_gemm_ex) or, with an epilogue, hipBLASLt's BIAS,
//         GELU_AUX_BIAS and DGELU epilogues; outputs compared numerically.
//
// Protocol per case: a time-based warm-up alternating the sides and doubling
// each side's batch until it takes half a sample; a two-pass calibration that
// sizes each side's sample to sample_ms; then interleaved rounds, Flint first
// on even valid rounds, each launch using the next of `rotation_sets` buffer
// sets, enough of them that together they exceed 4x the 256 MiB Infinity Cache,
// so no launch finds its operands cached. Times are hipEvent pairs around a
// batch of launches on one stream. The ratio is baseline time / Flint time.
//
// monitor.h samples clocks, power, temperature and throttling through amd-smi:
// each timed sample carries the statistics of the window it ran in, a round is
// discarded when another process appeared on the GPU or a sample fell short of
// 0.9 x sample_ms, and the compute fraction is also given at the window's mean
// clock. Without amd-smi access those statistics are null. A run refuses to
// start while other processes hold the GPU, unless --allow-busy.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>
#include <hipblaslt/hipblaslt-ext.hpp>
#include <rocblas/rocblas.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <ctime>
#include <filesystem>
#include <functional>
#include <optional>
#include <sstream>
#include <string>
#include <unistd.h>
#include <vector>

#include "cli.h"
#include "flint/flint.h"
#include "mfma_kernel.h"
#include "monitor.h"

namespace fb {
namespace {

// flint.h declares its stream type as the reference does; the value is this
// harness's hipStream_t.
inline flint_stream as_flint(hipStream_t s) { return reinterpret_cast<flint_stream>(s); }

// ---------------------------------------------------------------- errors

struct Failure : std::runtime_error {
    using std::runtime_error::runtime_error;
};

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw Failure(std::string(what) + ": " + hipGetErrorString(e));
}

void flint_check(flint_status s, const char* what) {
    if (s != FLINT_OK) throw Failure(std::string(what) + ": " + flint_status_string(s) + ": " + flint_last_error());
}

const char* blas_status_name(hipblasStatus_t s) {
    switch (s) {
    case HIPBLAS_STATUS_SUCCESS: return "HIPBLAS_STATUS_SUCCESS";
    case HIPBLAS_STATUS_NOT_INITIALIZED: return "HIPBLAS_STATUS_NOT_INITIALIZED";
    case HIPBLAS_STATUS_ALLOC_FAILED: return "HIPBLAS_STATUS_ALLOC_FAILED";
    case HIPBLAS_STATUS_INVALID_VALUE: return "HIPBLAS_STATUS_INVALID_VALUE";
    case HIPBLAS_STATUS_MAPPING_ERROR: return "HIPBLAS_STATUS_MAPPING_ERROR";
    case HIPBLAS_STATUS_EXECUTION_FAILED: return "HIPBLAS_STATUS_EXECUTION_FAILED";
    case HIPBLAS_STATUS_INTERNAL_ERROR: return "HIPBLAS_STATUS_INTERNAL_ERROR";
    case HIPBLAS_STATUS_NOT_SUPPORTED: return "HIPBLAS_STATUS_NOT_SUPPORTED";
    case HIPBLAS_STATUS_ARCH_MISMATCH: return "HIPBLAS_STATUS_ARCH_MISMATCH";
    case HIPBLAS_STATUS_INVALID_ENUM: return "HIPBLAS_STATUS_INVALID_ENUM";
    default: return "HIPBLAS_STATUS_UNKNOWN";
    }
}

void lt_check(hipblasStatus_t s, const char* what) {
    if (s != HIPBLAS_STATUS_SUCCESS) throw Failure(std::string(what) + ": " + blas_status_name(s));
}

void roc_check(rocblas_status s, const char* what) {
    if (s != rocblas_status_success) throw Failure(std::string(what) + ": " + rocblas_status_to_string(s));
}

// ---------------------------------------------------------------- device

constexpr double kMiB = 1024.0 * 1024.0;
constexpr unsigned long long kInfinityCache = 256ull << 20;   // MI355X's last-level cache
constexpr double kRatedBandwidthGBs = 8000.0;                 // MI355X HBM3E, published
// HBM3E transfers per reported memory clock: the device reports 2,000 MHz on
// an 8,192-bit bus, and 4 x 2,000 MHz x 1,024 B = 8.19 TB/s is the part's
// published 8 TB/s (the reference's GDDR formula takes 2).
constexpr double kTransfersPerMemClock = 4.0;
constexpr double kPeakFlopPerCuPerClock = 4096.0;             // dense FP16 MFMA, gfx950

struct DeviceInfo {
    std::string name, arch, compute_capability;
    int cu_count = 0;
    double rated_clock_mhz = 0, memory_clock_mhz = 0;
    int bus_width = 0;
    unsigned long long total_bytes = 0, l2_per_xcd_bytes = 0, llc_bytes = kInfinityCache;
};

DeviceInfo device_info() {
    hipDeviceProp_t p;
    hip_check(hipGetDeviceProperties(&p, 0), "hipGetDeviceProperties");
    DeviceInfo d;
    d.arch = p.gcnArchName;
    // The marketing name comes from the driver's ID table, which a box may
    // lack; the architecture then names the device.
    d.name = p.name[0] ? std::string(p.name) : "AMD " + d.arch.substr(0, d.arch.find(':'));
    d.compute_capability = std::to_string(p.major) + "." + std::to_string(p.minor);
    d.cu_count = p.multiProcessorCount;
    d.rated_clock_mhz = p.clockRate / 1000.0;
    d.memory_clock_mhz = p.memoryClockRate / 1000.0;
    d.bus_width = p.memoryBusWidth;
    d.total_bytes = p.totalGlobalMem;
    d.l2_per_xcd_bytes = p.l2CacheSize;
    return d;
}

// Buffer sets of bytes_per_set whose total exceeds 4x the last-level cache.
int rotation_sets(const DeviceInfo& d, double bytes_per_set) {
    const double cache = double(std::max<unsigned long long>(d.llc_bytes, d.l2_per_xcd_bytes));
    return int(std::floor(4.0 * cache / std::max(bytes_per_set, 1.0))) + 1;
}

std::string size_label(unsigned long long bytes) {
    const unsigned long long mib = 1ull << 20;
    if (bytes % mib == 0) return std::to_string(bytes / mib) + " MiB";
    return std::to_string(bytes) + " B";
}

// ---------------------------------------------------------------- fills

// A 32-bit mix of (seed, index) into [-1, 1).
__device__ inline float unit_noise(unsigned seed, unsigned long long i) {
    unsigned long long z = i * 0x9E3779B97F4A7C15ull + seed * 0xD1B54A32D192ED03ull + 1;
    z ^= z >> 31;
    z *= 0xBF58476D1CE4E5B9ull;
    z ^= z >> 29;
    return float(unsigned(z >> 40)) * (2.0f / 16777216.0f) - 1.0f;
}

__global__ void fill_f16(_Float16* p, unsigned long long count, unsigned seed, float scale) {
    for (unsigned long long i = blockIdx.x * 256ull + threadIdx.x; i < count; i += gridDim.x * 256ull)
        p[i] = _Float16(scale * unit_noise(seed, i));
}

__global__ void fill_f32(float* p, unsigned long long count, unsigned seed, float scale) {
    for (unsigned long long i = blockIdx.x * 256ull + threadIdx.x; i < count; i += gridDim.x * 256ull)
        p[i] = scale * unit_noise(seed, i);
}

__global__ void fill_bytes(unsigned char* p, unsigned long long count, unsigned seed) {
    for (unsigned long long i = blockIdx.x * 256ull + threadIdx.x; i < count; i += gridDim.x * 256ull)
        p[i] = (unsigned char)(unit_noise(seed, i) * 127.0f + 128.0f);
}

void fill_half(void* p, unsigned long long count, unsigned seed, float scale, hipStream_t s) {
    hipLaunchKernelGGL(fill_f16, dim3(4096), dim3(256), 0, s, static_cast<_Float16*>(p), count, seed, scale);
    hip_check(hipGetLastError(), "fill_f16");
}

void fill_float(void* p, unsigned long long count, unsigned seed, float scale, hipStream_t s) {
    hipLaunchKernelGGL(fill_f32, dim3(4096), dim3(256), 0, s, static_cast<float*>(p), count, seed, scale);
    hip_check(hipGetLastError(), "fill_f32");
}

// ---------------------------------------------------------------- memory

struct DeviceBuffer {
    void* ptr = nullptr;
    size_t bytes = 0;
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t n) : bytes(n) {
        if (n) hip_check(hipMalloc(&ptr, n), "hipMalloc");
    }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&& o) noexcept : ptr(o.ptr), bytes(o.bytes) { o.ptr = nullptr; }
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
        std::swap(ptr, o.ptr);
        std::swap(bytes, o.bytes);
        return *this;
    }
    ~DeviceBuffer() {
        if (ptr) (void)hipFree(ptr);
    }
    char* at(size_t offset) const { return static_cast<char*>(ptr) + offset; }
};

size_t round256(size_t n) { return (n + 255) / 256 * 256; }

// ---------------------------------------------------------------- timing

// Enqueues `count` launches on `stream`; launch i, counted from `first`, uses
// buffer set i % rotation_sets. Throws on failure.
using Launcher = std::function<void(hipStream_t, long long first, long long count)>;

struct EventTimer {
    hipEvent_t a = nullptr, b = nullptr;
    EventTimer() {
        hip_check(hipEventCreate(&a), "hipEventCreate");
        hip_check(hipEventCreate(&b), "hipEventCreate");
    }
    ~EventTimer() {
        (void)hipEventDestroy(a);
        (void)hipEventDestroy(b);
    }
    double time(const Launcher& launch, hipStream_t s, long long first, long long count) {
        hip_check(hipEventRecord(a, s), "hipEventRecord");
        launch(s, first, count);
        hip_check(hipEventRecord(b, s), "hipEventRecord");
        hip_check(hipEventSynchronize(b), "hipEventSynchronize");
        float ms = 0;
        hip_check(hipEventElapsedTime(&ms, a, b), "hipEventElapsedTime");
        return ms;
    }
};

double median(std::vector<double> v) {
    if (v.empty()) return 0;
    std::sort(v.begin(), v.end());
    const size_t n = v.size();
    return n % 2 ? v[n / 2] : 0.5 * (v[n / 2 - 1] + v[n / 2]);
}

struct Sample {
    long long launches = 0;
    double ms_per_launch = 0, sample_ms = 0;
    std::optional<WindowStats> stats;
};

struct Round {
    bool flint_first = true, valid = true;
    Sample flint, baseline;
    double ratio = 0;
    std::string discard_reason;
};

struct Side {
    long long launches_per_sample = 0;
    double min_sample_ms = 0, ms_per_launch = 0, gbs = 0, rated_fraction = 0, tflops = 0,
           rated_compute_fraction = 0;
    std::optional<double> clock_adjusted_fraction, clock_adjusted_compute_fraction;
    std::optional<WindowStats> stats;   // the valid samples' windows, merged by time
};

struct OutputCheck {
    double rel_l2 = 0, max_abs = 0, max_abs_baseline = 0;
    unsigned long long nonfinite = 0;
    bool deterministic = false;
};

struct Candidate {
    int index = 0;
    long long solution_index = -1;
    unsigned long long workspace_bytes = 0;
    double waves_count = 0;
    std::string status;
    std::optional<double> ms_per_launch;
};

struct BaselineAlgorithm {
    LtAlgo selection = LtAlgo::Fastest;
    int used = 0;
    std::vector<Candidate> candidates;
};

struct CaseSpec {
    std::string benchmark, label, layout, epilogue, baseline_name;
    unsigned long long size_bytes = 0;
    double bytes_moved = 0, flops = 0, peak_flop_per_cu_per_clock = 0;
    int rotation_sets = 1;
    Launcher flint, reference;   // reference empty: one-sided
};

struct CaseResult {
    CaseSpec spec;
    bool one_sided = false;
    double warmup_seconds = 0;
    std::vector<Round> rounds;
    int valid_rounds = 0;
    bool enough_rounds = false, outputs_match = false;
    double ratio_median = 0, ratio_min = 0, ratio_max = 0;
    Side flint, baseline;
    std::optional<OutputCheck> output_check, pre_check;
    std::optional<BaselineAlgorithm> baseline_algorithm;
    bool ok() const { return enough_rounds && outputs_match; }
};

constexpr double kShortestSample = 0.9;   // of sample_ms, for a round to count

Side summarize(long long launches, const std::vector<const Sample*>& samples, const CaseSpec& spec,
               const DeviceInfo& d) {
    Side side;
    side.launches_per_sample = launches;
    if (samples.empty()) return side;
    std::vector<double> per_launch;
    side.min_sample_ms = samples[0]->sample_ms;
    for (const Sample* s : samples) {
        per_launch.push_back(s->ms_per_launch);
        side.min_sample_ms = std::min(side.min_sample_ms, s->sample_ms);
    }
    side.ms_per_launch = median(per_launch);
    if (samples[0]->stats) {
        // Means are weighted by the seconds of the windows that hold a
        // reading; a window without one adds its time and counts only.
        WindowStats m;
        double sm = 0, mem = 0, pw = 0, act = 0, cap = 0, thm = 0, read_seconds = 0;
        for (const Sample* s : samples) {
            const WindowStats& w = *s->stats;
            m.seconds += w.seconds;
            m.samples += w.samples;
            m.failed_reads += w.failed_reads;
            m.temp_c_max = std::max(m.temp_c_max, w.temp_c_max);
            m.new_process = m.new_process || w.new_process;
            if (w.samples == 0) continue;
            read_seconds += w.seconds;
            sm += w.sm_mhz * w.seconds, mem += w.mem_mhz * w.seconds, pw += w.power_w * w.seconds;
            act += w.activity * w.seconds, cap += w.power_cap_share * w.seconds, thm += w.thermal_share * w.seconds;
        }
        if (read_seconds > 0) {
            m.sm_mhz = sm / read_seconds, m.mem_mhz = mem / read_seconds, m.power_w = pw / read_seconds;
            m.activity = act / read_seconds, m.power_cap_share = cap / read_seconds;
            m.thermal_share = thm / read_seconds;
        }
        side.stats = m;
    }
    if (spec.bytes_moved > 0) {
        side.gbs = spec.bytes_moved / (side.ms_per_launch * 1e-3) / 1e9;
        side.rated_fraction = side.gbs / kRatedBandwidthGBs;
        // Against the bandwidth at the memory clock the monitor read (ref
        // bench/harness.cpp:80-85).
        if (side.stats && side.stats->mem_mhz > 0 && d.bus_width > 0)
            side.clock_adjusted_fraction =
                side.gbs / (kTransfersPerMemClock * side.stats->mem_mhz * 1e6 * (d.bus_width / 8) / 1e9);
    }
    if (spec.flops > 0) {
        side.tflops = spec.flops / (side.ms_per_launch * 1e-3) / 1e12;
        const double peak = spec.peak_flop_per_cu_per_clock * d.cu_count * d.rated_clock_mhz * 1e6 / 1e12;
        if (peak > 0) side.rated_compute_fraction = side.tflops / peak;
        if (side.stats && side.stats->sm_mhz > 0)
            side.clock_adjusted_compute_fraction =
                side.tflops / (spec.peak_flop_per_cu_per_clock * d.cu_count * side.stats->sm_mhz * 1e6 / 1e12);
    }
    return side;
}

CaseResult run_case(const CaseSpec& spec, const DeviceInfo& d, const Options& o, hipStream_t stream, Monitor& mon) {
    CaseResult r;
    r.spec = spec;
    hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    EventTimer timer;
    const Launcher* sides[2] = {&spec.flint, &spec.reference};
    r.one_sided = !spec.reference;
    const int n_sides = r.one_sided ? 1 : 2;
    long long next = 0;   // rotation index of the next launch, across samples

    const auto t0 = std::chrono::steady_clock::now();
    auto elapsed = [&] { return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count(); };
    long long counts[2] = {1, 1};
    double per_launch[2] = {0, 0};
    do {
        for (int i = 0; i < n_sides; ++i) {
            const double ms = timer.time(*sides[i], stream, next, counts[i]);
            next += counts[i];
            per_launch[i] = std::max(ms, 1e-3) / counts[i];
            if (ms < o.sample_ms / 2) counts[i] *= 2;
        }
    } while (elapsed() < o.warmup_seconds);

    long long launches[2] = {1, 1};
    for (int i = 0; i < n_sides; ++i) {
        for (int pass = 0; pass < 2; ++pass) {
            launches[i] = std::max(1LL, (long long)std::ceil(o.sample_ms * 1.05 / per_launch[i]));
            const double ms = timer.time(*sides[i], stream, next, launches[i]);
            next += launches[i];
            per_launch[i] = std::max(ms, 1e-3) / launches[i];
        }
    }
    r.warmup_seconds = elapsed();

    const bool monitored = mon.available();
    double begin[2] = {0, 0}, end[2] = {0, 0};
    int others = -1;
    auto sample = [&](int side) {
        Sample s;
        s.launches = launches[side];
        begin[side] = mon.now();
        s.sample_ms = timer.time(*sides[side], stream, next, s.launches);
        end[side] = mon.now();
        next += s.launches;
        s.ms_per_launch = s.sample_ms / s.launches;
        if (s.sample_ms < o.sample_ms)   // grow later samples back past sample_ms
            launches[side] = (long long)std::ceil(s.launches * o.sample_ms * 1.05 / std::max(s.sample_ms, 1e-3));
        return s;
    };

    for (int i = 0; i < o.max_rounds && r.valid_rounds < o.rounds; ++i) {
        Round round;
        round.flint_first = r.one_sided || r.valid_rounds % 2 == 0;
        if (monitored) {
            mon.forget_before(mon.now() - 1.0);
            others = mon.other_processes();
        }
        if (r.one_sided) {
            round.flint = sample(0);
        } else if (round.flint_first) {
            round.flint = sample(0);
            round.baseline = sample(1);
        } else {
            round.baseline = sample(1);
            round.flint = sample(0);
        }
        if (!r.one_sided) round.ratio = round.baseline.ms_per_launch / round.flint.ms_per_launch;
        if (monitored) {
            const int others_now = mon.other_processes();
            round.flint.stats = mon.window(begin[0], end[0], others, others_now);
            if (!r.one_sided) round.baseline.stats = mon.window(begin[1], end[1], others, others_now);
        }
        for (int side = 0; side < n_sides && round.valid; ++side) {
            const Sample& s = side == 0 ? round.flint : round.baseline;
            if (s.stats && s.stats->new_process) {
                round.valid = false;
                round.discard_reason = "another process used the GPU";
            } else if (s.sample_ms < kShortestSample * o.sample_ms) {
                round.valid = false;
                round.discard_reason = "a sample ran " + std::to_string(s.sample_ms) +
                                       " ms, short of the protocol's floor";
            }
        }
        r.valid_rounds += round.valid ? 1 : 0;
        r.rounds.push_back(round);
    }
    r.enough_rounds = r.valid_rounds >= o.rounds;

    std::vector<double> ratios;
    std::vector<const Sample*> fs, bs;
    for (const Round& round : r.rounds) {
        if (!round.valid) continue;
        ratios.push_back(round.ratio);
        fs.push_back(&round.flint);
        bs.push_back(&round.baseline);
    }
    if (!r.one_sided && !ratios.empty()) {
        r.ratio_median = median(ratios);
        r.ratio_min = *std::min_element(ratios.begin(), ratios.end());
        r.ratio_max = *std::max_element(ratios.begin(), ratios.end());
    }
    r.flint = summarize(launches[0], fs, spec, d);
    if (!r.one_sided) r.baseline = summarize(launches[1], bs, spec, d);
    return r;
}

// ---------------------------------------------------------------- copy

CaseResult copy_case(unsigned long long bytes, const DeviceInfo& d, const Options& o, hipStream_t s, Monitor& mon) {
    const size_t stride = round256(bytes);
    CaseSpec spec;
    spec.benchmark = "copy";
    spec.label = size_label(bytes);
    spec.baseline_name = "hipMemcpyAsync";
    spec.size_bytes = bytes;
    spec.bytes_moved = 2.0 * double(bytes);
    spec.rotation_sets = rotation_sets(d, 2.0 * double(stride));
    const int sets = spec.rotation_sets;
    DeviceBuffer src(stride * sets), dst(stride * sets);
    hipLaunchKernelGGL(fill_bytes, dim3(4096), dim3(256), 0, s, static_cast<unsigned char*>(src.ptr),
                       (unsigned long long)src.bytes, 7u);
    hip_check(hipGetLastError(), "fill_bytes");
    spec.flint = [&, stride, sets, bytes](hipStream_t st, long long first, long long count) {
        for (long long i = first; i < first + count; ++i) {
            const size_t off = stride * size_t(i % sets);
            flint_check(flint_copy(dst.at(off), src.at(off), bytes, as_flint(st)), "flint_copy");
        }
    };
    spec.reference = [&, stride, sets, bytes](hipStream_t st, long long first, long long count) {
        for (long long i = first; i < first + count; ++i) {
            const size_t off = stride * size_t(i % sets);
            hip_check(hipMemcpyAsync(dst.at(off), src.at(off), bytes, hipMemcpyDeviceToDevice, st),
                      "hipMemcpyAsync");
        }
    };
    CaseResult r = run_case(spec, d, o, s, mon);

    // Output check: each side's copy of set 0 equals the source, bit for bit.
    std::vector<unsigned char> want(bytes), got(bytes);
    hip_check(hipMemcpy(want.data(), src.ptr, bytes, hipMemcpyDeviceToHost), "hipMemcpy");
    bool match = true;
    for (int side = 0; side < 2; ++side) {
        hip_check(hipMemsetAsync(dst.ptr, 0xA5 + side, bytes, s), "hipMemsetAsync");
        if (side == 0) flint_check(flint_copy(dst.ptr, src.ptr, bytes, as_flint(s)), "flint_copy");
        else hip_check(hipMemcpyAsync(dst.ptr, src.ptr, bytes, hipMemcpyDeviceToDevice, s), "hipMemcpyAsync");
        hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
        hip_check(hipMemcpy(got.data(), dst.ptr, bytes, hipMemcpyDeviceToHost), "hipMemcpy");
        match = match && std::memcmp(want.data(), got.data(), bytes) == 0;
    }
    r.outputs_match = match;
    r.spec.flint = nullptr;
    r.spec.reference = nullptr;
    return r;
}

// ---------------------------------------------------------------- mma

CaseResult mma_case(int chains, const DeviceInfo& d, const Options& o, hipStream_t s, Monitor& mon) {
    const int blocks_per_cu = 2;   // 8 waves per CU: two per SIMD
    const int blocks = blocks_per_cu * d.cu_count;
    const int iters = kMfmaPerWave / chains;
    CaseSpec spec;
    spec.benchmark = "mma";
    spec.label = "mfma 32x32x16 f16->f32, " + std::to_string(chains) + " chains, " + std::to_string(blocks_per_cu) +
                 " blocks/CU";
    spec.flops = mfma_loop_flops(blocks, iters, chains);
    spec.peak_flop_per_cu_per_clock = kPeakFlopPerCuPerClock;
    DeviceBuffer bad(sizeof(int));
    hip_check(hipMemsetAsync(bad.ptr, 0, sizeof(int), s), "hipMemsetAsync");
    int* flag = static_cast<int*>(bad.ptr);
    spec.flint = [=](hipStream_t st, long long, long long count) {
        for (long long i = 0; i < count; ++i)
            hip_check(launch_mfma_loop(chains, blocks, flag, iters, st), "mfma_loop");
    };
    CaseResult r = run_case(spec, d, o, s, mon);
    int wrong = 0;
    hip_check(hipMemcpy(&wrong, bad.ptr, sizeof(int), hipMemcpyDeviceToHost), "hipMemcpy");
    r.outputs_match = wrong == 0;
    r.spec.flint = nullptr;
    return r;
}

// ---------------------------------------------------------------- gemm

struct Host16 {
    static double get(const void* p, size_t i) { return double(static_cast<const _Float16*>(p)[i]); }
};
struct Host32 {
    static double get(const void* p, size_t i) { return double(static_cast<const float*>(p)[i]); }
};

// Flint's output (two runs, a and a2) against the baseline's (b), count values.
OutputCheck compare(const std::vector<unsigned char>& a, const std::vector<unsigned char>& a2,
                    const std::vector<unsigned char>& b, size_t count, bool fp32) {
    OutputCheck c;
    c.deterministic = a == a2;
    double diff2 = 0, base2 = 0;
    for (size_t i = 0; i < count; ++i) {
        const double x = fp32 ? Host32::get(a.data(), i) : Host16::get(a.data(), i);
        const double y = fp32 ? Host32::get(b.data(), i) : Host16::get(b.data(), i);
        if (!std::isfinite(x) || !std::isfinite(y)) {
            c.nonfinite += !std::isfinite(x) + !std::isfinite(y);
            continue;
        }
        diff2 += (x - y) * (x - y);
        base2 += y * y;
        c.max_abs = std::max(c.max_abs, std::fabs(x - y));
        c.max_abs_baseline = std::max(c.max_abs_baseline, std::fabs(y));
    }
    c.rel_l2 = base2 > 0 ? std::sqrt(diff2 / base2) : (diff2 > 0 ? INFINITY : 0);
    return c;
}

bool check_passes(const OutputCheck& c) {
    return c.deterministic && c.nonfinite == 0 && c.rel_l2 <= 1.0 / 1024.0 && c.max_abs_baseline > 0;
}

struct LtContext {
    hipblasLtHandle_t handle = nullptr;
    rocblas_handle roc = nullptr;
    DeviceBuffer workspace{64ull << 20};
    LtContext() {
        lt_check(hipblasLtCreate(&handle), "hipblasLtCreate");
        roc_check(rocblas_create_handle(&roc), "rocblas_create_handle");
    }
    ~LtContext() {
        if (handle) (void)hipblasLtDestroy(handle);
        if (roc) (void)rocblas_destroy_handle(roc);
    }
};

// A hipBLASLt matmul in column-major terms: D (rows x cols) = op(A) op(B).
struct LtPlan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr, dl = nullptr;
    std::vector<hipblasLtMatmulHeuristicResult_t> heuristics;
    ~LtPlan() {
        if (desc) (void)hipblasLtMatmulDescDestroy(desc);
        for (auto l : {a, b, c, dl})
            if (l) (void)hipblasLtMatrixLayoutDestroy(l);
    }
};

template <class T>
void set_attr(hipblasLtMatmulDesc_t desc, hipblasLtMatmulDescAttributes_t attr, const T& value) {
    lt_check(hipblasLtMatmulDescSetAttribute(desc, attr, &value, sizeof(value)), "hipblasLtMatmulDescSetAttribute");
}

CaseResult gemm_case(const Shape& sh, Layout layout, Epilogue ep, const DeviceInfo& d, const Options& o,
                     hipStream_t s, LtContext& lt, Monitor& mon) {
    const size_t m = size_t(sh.m), n = size_t(sh.n), k = size_t(sh.k);
    const bool tn = layout == Layout::TN, residual = ep == Epilogue::BiasResidual;
    const bool has_pre = ep == Epilogue::BiasGelu || ep == Epilogue::DGelu;
    const bool has_bias = ep == Epilogue::Bias || ep == Epilogue::BiasGelu || residual;
    const bool y32 = tn || residual;
    const size_t x_bytes = 2 * m * k, w_bytes = 2 * n * k, y_bytes = m * n * (y32 ? 4 : 2);
    const size_t pre_bytes = has_pre ? 2 * m * n : 0, res_bytes = residual ? 4 * m * n : 0,
                 bias_bytes = has_bias ? 4 * n : 0;

    CaseSpec spec;
    spec.benchmark = "gemm";
    spec.label = sh.label;
    spec.layout = layout_name(layout);
    spec.epilogue = epilogue_name(ep);
    spec.baseline_name = ep == Epilogue::None       ? "rocBLAS"
                         : ep == Epilogue::DGelu    ? "hipBLASLt DGELU"
                         : residual                 ? "hipBLASLt, residual in C"
                                                    : "hipBLASLt, FP32 bias";
    spec.size_bytes = x_bytes + w_bytes + y_bytes + pre_bytes + res_bytes + bias_bytes;
    spec.flops = 2.0 * double(m) * double(n) * double(k);
    spec.peak_flop_per_cu_per_clock = kPeakFlopPerCuPerClock;
    spec.rotation_sets = rotation_sets(d, double(spec.size_bytes));
    const int sets = spec.rotation_sets;

    // One allocation per operand, `sets` copies at 256-byte strides. A bias-gelu
    // case's pre is an output; dgelu's is an input.
    const size_t sx = round256(x_bytes), sw = round256(w_bytes), sy = round256(y_bytes), sp = round256(pre_bytes),
                 sr = round256(res_bytes), sb = round256(bias_bytes);
    DeviceBuffer X(sx * sets), W(sw * sets), Y(sy * sets), P(sp * sets), R(sr * sets), B(sb * sets);
    fill_half(X.ptr, X.bytes / 2, 11, 1.0f, s);
    fill_half(W.ptr, W.bytes / 2, 12, residual || has_bias ? 0.02f * 1.7320508f : 1.0f, s);
    if (y32) fill_float(Y.ptr, Y.bytes / 4, 13, 1.0f, s);
    if (ep == Epilogue::DGelu) fill_half(P.ptr, P.bytes / 2, 14, 3.0f, s);
    if (residual) fill_float(R.ptr, R.bytes / 4, 15, 1.0f, s);
    if (has_bias) fill_float(B.ptr, B.bytes / 4, 16, 0.02f * 1.7320508f, s);

    size_t tn_ws = 0;
    if (tn) flint_check(flint_gemm_tn_workspace(m, n, k, &tn_ws), "flint_gemm_tn_workspace");
    DeviceBuffer tn_workspace(tn_ws);

    // Flint's call into set i's buffers (y, pre at the given addresses).
    auto flint_call = [&, m, n, k](int i, void* y, void* pre, bool accumulate, hipStream_t st) {
        const void* x = X.at(sx * i);
        const void* w = W.at(sw * i);
        const void* bias = B.at(sb * i);
        switch (layout) {
        case Layout::TN:
            flint_check(flint_gemm_tn(y, x, w, m, n, k, accumulate ? 1 : 0, tn_workspace.ptr, tn_ws, as_flint(st)),
                        "flint_gemm_tn");
            return;
        case Layout::NN:
            if (ep == Epilogue::DGelu) flint_check(flint_gemm_nn_dgelu(y, x, w, pre, m, n, k, as_flint(st)), "flint_gemm_nn_dgelu");
            else flint_check(flint_gemm_nn(y, x, w, m, n, k, as_flint(st)), "flint_gemm_nn");
            return;
        case Layout::NT: break;
        }
        switch (ep) {
        case Epilogue::Bias: flint_check(flint_gemm_nt_bias(y, x, w, bias, m, n, k, as_flint(st)), "flint_gemm_nt_bias"); return;
        case Epilogue::BiasGelu:
            flint_check(flint_gemm_nt_bias_gelu(y, pre, x, w, bias, m, n, k, as_flint(st)), "flint_gemm_nt_bias_gelu");
            return;
        case Epilogue::BiasResidual:
            flint_check(flint_gemm_nt_bias_residual(y, x, w, bias, R.at(sr * i), m, n, k, as_flint(st)),
                        "flint_gemm_nt_bias_residual");
            return;
        default: flint_check(flint_gemm_nt(y, x, w, m, n, k, as_flint(st)), "flint_gemm_nt"); return;
        }
    };

    // The baseline. Row-major y (m x n) is column-major y^T (n x m), so every
    // product is computed transposed: nt y^T = w x^T, nn y^T = w^T x^T,
    // tn y^T = w^T x.
    const hipblasOperation_t op_a = layout == Layout::NT ? HIPBLAS_OP_T : HIPBLAS_OP_N;
    const hipblasOperation_t op_b = layout == Layout::TN ? HIPBLAS_OP_T : HIPBLAS_OP_N;
    const int64_t lda = layout == Layout::NT ? int64_t(k) : int64_t(n);
    const int64_t ldb = layout == Layout::TN ? int64_t(m) : int64_t(k);
    LtPlan plan;
    BaselineAlgorithm algorithm;
    algorithm.selection = o.lt_algo;
    const float one = 1.0f, zero = 0.0f;

    auto lt_call = [&](const hipblasLtMatmulAlgo_t* algo, int i, void* y, void* pre, hipStream_t st) {
        if (pre) set_attr(plan.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE_AUX_POINTER, pre);
        const void* c = residual ? static_cast<const void*>(R.at(sr * i)) : static_cast<const void*>(y);
        if (has_bias) set_attr(plan.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, static_cast<const void*>(B.at(sb * i)));
        return hipblasLtMatmul(lt.handle, plan.desc, &one, W.at(sw * i), plan.a, X.at(sx * i), plan.b,
                               residual ? &one : &zero, c, plan.c, y, plan.dl, algo, lt.workspace.ptr,
                               lt.workspace.bytes, st);
    };
    auto roc_call = [&, m, n, k](int i, void* y, bool accumulate, hipStream_t st) {
        roc_check(rocblas_set_stream(lt.roc, st), "rocblas_set_stream");
        const rocblas_operation ta = op_a == HIPBLAS_OP_T ? rocblas_operation_transpose : rocblas_operation_none;
        const rocblas_operation tb = op_b == HIPBLAS_OP_T ? rocblas_operation_transpose : rocblas_operation_none;
        const rocblas_datatype out_t = y32 ? rocblas_datatype_f32_r : rocblas_datatype_f16_r;
        roc_check(rocblas_gemm_ex(lt.roc, ta, tb, rocblas_int(n), rocblas_int(m), rocblas_int(k), &one, W.at(sw * i),
                                  rocblas_datatype_f16_r, rocblas_int(lda), X.at(sx * i), rocblas_datatype_f16_r,
                                  rocblas_int(ldb), accumulate ? &one : &zero, y, out_t, rocblas_int(n), y, out_t,
                                  rocblas_int(n), rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0),
                  "rocblas_gemm_ex");
    };

    if (ep != Epilogue::None) {
        lt_check(hipblasLtMatmulDescCreate(&plan.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F), "hipblasLtMatmulDescCreate");
        set_attr(plan.desc, HIPBLASLT_MATMUL_DESC_TRANSA, int32_t(op_a));
        set_attr(plan.desc, HIPBLASLT_MATMUL_DESC_TRANSB, int32_t(op_b));
        const hipblasLtEpilogue_t e = ep == Epilogue::BiasGelu ? HIPBLASLT_EPILOGUE_GELU_AUX_BIAS
                                      : ep == Epilogue::DGelu  ? HIPBLASLT_EPILOGUE_DGELU
                                                               : HIPBLASLT_EPILOGUE_BIAS;
        set_attr(plan.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, uint32_t(e));
        if (has_bias) {
            set_attr(plan.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, int32_t(HIP_R_32F));
            set_attr(plan.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, static_cast<const void*>(B.ptr));
        }
        if (has_pre) {
            set_attr(plan.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE_AUX_POINTER, static_cast<void*>(P.ptr));
            set_attr(plan.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE_AUX_LD, int64_t(n));
            set_attr(plan.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE_AUX_DATA_TYPE, int32_t(HIP_R_16F));
        }
        const hipDataType out_t = y32 ? HIP_R_32F : HIP_R_16F;
        // Stored shapes (rows x cols, column-major) of A = w and B = x.
        const uint64_t a_rows = op_a == HIPBLAS_OP_T ? k : n, a_cols = op_a == HIPBLAS_OP_T ? n : k;
        const uint64_t b_rows = op_b == HIPBLAS_OP_T ? m : k, b_cols = op_b == HIPBLAS_OP_T ? k : m;
        lt_check(hipblasLtMatrixLayoutCreate(&plan.a, HIP_R_16F, a_rows, a_cols, lda), "hipblasLtMatrixLayoutCreate");
        lt_check(hipblasLtMatrixLayoutCreate(&plan.b, HIP_R_16F, b_rows, b_cols, ldb), "hipblasLtMatrixLayoutCreate");
        lt_check(hipblasLtMatrixLayoutCreate(&plan.c, out_t, n, m, n), "hipblasLtMatrixLayoutCreate");
        lt_check(hipblasLtMatrixLayoutCreate(&plan.dl, out_t, n, m, n), "hipblasLtMatrixLayoutCreate");
        hipblasLtMatmulPreference_t pref = nullptr;
        lt_check(hipblasLtMatmulPreferenceCreate(&pref), "hipblasLtMatmulPreferenceCreate");
        const uint64_t ws = lt.workspace.bytes;
        lt_check(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws)),
                 "hipblasLtMatmulPreferenceSetAttribute");
        plan.heuristics.resize(8);
        int returned = 0;
        const hipblasStatus_t hs = hipblasLtMatmulAlgoGetHeuristic(lt.handle, plan.desc, plan.a, plan.b, plan.c,
                                                                   plan.dl, pref, 8, plan.heuristics.data(), &returned);
        (void)hipblasLtMatmulPreferenceDestroy(pref);
        lt_check(hs, "hipblasLtMatmulAlgoGetHeuristic");
        plan.heuristics.resize(size_t(std::max(returned, 0)));
        if (plan.heuristics.empty()) throw Failure("hipBLASLt offers no algorithm for " + sh.label);

        // Each candidate: a few short samples on set 0, median per launch.
        EventTimer timer;
        for (size_t c = 0; c < plan.heuristics.size(); ++c) {
            Candidate cand;
            cand.index = int(c);
            cand.solution_index = hipblaslt_ext::getIndexFromAlgo(plan.heuristics[c].algo);
            cand.workspace_bytes = plan.heuristics[c].workspaceSize;
            cand.waves_count = plan.heuristics[c].wavesCount;
            const hipblasStatus_t st = lt_call(&plan.heuristics[c].algo, 0, Y.ptr, P.ptr, s);
            cand.status = blas_status_name(st);
            if (st == HIPBLAS_STATUS_SUCCESS) {
                hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
                const hipblasLtMatmulAlgo_t* algo = &plan.heuristics[c].algo;
                Launcher once = [&, algo](hipStream_t st2, long long first, long long count) {
                    for (long long i = first; i < first + count; ++i) {
                        const int set = int(i % sets);
                        lt_check(lt_call(algo, set, Y.at(sy * set), has_pre ? P.at(sp * set) : nullptr, st2),
                                 "hipblasLtMatmul");
                    }
                };
                double per = timer.time(once, s, 0, 1);
                const long long count = std::max(1LL, (long long)std::ceil(std::min(5.0, o.sample_ms) / std::max(per, 1e-3)));
                std::vector<double> times;
                for (int rep = 0; rep < 3; ++rep) times.push_back(timer.time(once, s, rep * count, count) / count);
                cand.ms_per_launch = median(times);
            }
            algorithm.candidates.push_back(cand);
        }
        int used = -1;
        for (const Candidate& c : algorithm.candidates) {
            if (!c.ms_per_launch) continue;
            if (used < 0 || (o.lt_algo == LtAlgo::Fastest && *c.ms_per_launch < *algorithm.candidates[used].ms_per_launch))
                used = c.index;
            if (o.lt_algo == LtAlgo::First) break;
        }
        if (used < 0) throw Failure("no hipBLASLt algorithm launched for " + sh.label);
        if (o.lt_algo == LtAlgo::First && algorithm.candidates[0].ms_per_launch) used = 0;
        algorithm.used = used;
    }
    const hipblasLtMatmulAlgo_t* chosen = ep != Epilogue::None ? &plan.heuristics[size_t(algorithm.used)].algo : nullptr;

    spec.flint = [&, sets](hipStream_t st, long long first, long long count) {
        for (long long i = first; i < first + count; ++i) {
            const int set = int(i % sets);
            flint_call(set, Y.at(sy * set), has_pre ? P.at(sp * set) : nullptr, true, st);
        }
    };
    spec.reference = [&, sets, chosen](hipStream_t st, long long first, long long count) {
        for (long long i = first; i < first + count; ++i) {
            const int set = int(i % sets);
            if (chosen) lt_check(lt_call(chosen, set, Y.at(sy * set), has_pre ? P.at(sp * set) : nullptr, st), "hipblasLtMatmul");
            else roc_call(set, Y.at(sy * set), tn, st);
        }
    };
    CaseResult r = run_case(spec, d, o, s, mon);
    if (ep != Epilogue::None) r.baseline_algorithm = algorithm;

    // Output check on set 0: Flint twice into differently poisoned outputs, the
    // baseline once (not accumulating: tn starts from zero on both sides).
    DeviceBuffer y1(y_bytes), y2(y_bytes), yb(y_bytes), p1(pre_bytes), p2(pre_bytes), pb(pre_bytes);
    const bool pre_out = ep == Epilogue::BiasGelu;
    hip_check(hipMemsetAsync(y1.ptr, 0xFF, y_bytes, s), "hipMemsetAsync");
    hip_check(hipMemsetAsync(y2.ptr, 0x7C, y_bytes, s), "hipMemsetAsync");
    hip_check(hipMemsetAsync(yb.ptr, 0x00, y_bytes, s), "hipMemsetAsync");
    if (pre_out) {
        hip_check(hipMemsetAsync(p1.ptr, 0xFF, pre_bytes, s), "hipMemsetAsync");
        hip_check(hipMemsetAsync(p2.ptr, 0x7C, pre_bytes, s), "hipMemsetAsync");
    }
    void* pre_in = ep == Epilogue::DGelu ? static_cast<void*>(P.ptr) : nullptr;
    flint_call(0, y1.ptr, pre_out ? p1.ptr : pre_in, false, s);
    flint_call(0, y2.ptr, pre_out ? p2.ptr : pre_in, false, s);
    if (chosen) lt_check(lt_call(chosen, 0, yb.ptr, pre_out ? pb.ptr : pre_in, s), "hipblasLtMatmul");
    else roc_call(0, yb.ptr, false, s);
    hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
    auto host = [](const DeviceBuffer& b) {
        std::vector<unsigned char> v(b.bytes);
        if (b.bytes) hip_check(hipMemcpy(v.data(), b.ptr, b.bytes, hipMemcpyDeviceToHost), "hipMemcpy");
        return v;
    };
    r.output_check = compare(host(y1), host(y2), host(yb), m * n, y32);
    bool match = check_passes(*r.output_check);
    if (pre_out) {
        r.pre_check = compare(host(p1), host(p2), host(pb), m * n, false);
        match = match && check_passes(*r.pre_check);
    }
    r.outputs_match = match;
    r.spec.flint = nullptr;
    r.spec.reference = nullptr;
    return r;
}

// ---------------------------------------------------------------- JSON

struct Json {
    std::ostringstream out;
    std::vector<bool> first{true};
    void sep() {
        if (!first.back()) out << ", ";
        first.back() = false;
    }
    static std::string quote(const std::string& s) {
        std::string q = "\"";
        for (char c : s) {
            if (c == '"' || c == '\\') q += '\\', q += c;
            else if ((unsigned char)c < 0x20) {
                char buf[8];
                std::snprintf(buf, sizeof buf, "\\u%04x", c);
                q += buf;
            } else q += c;
        }
        return q + "\"";
    }
    void key(const char* k) {
        sep();
        out << quote(k) << ": ";
    }
    void open(char c) {
        out << c;
        first.push_back(true);
    }
    void close(char c) {
        out << c;
        first.pop_back();
    }
    void begin_obj(const char* k) { key(k), open('{'); }
    void begin_arr(const char* k) { key(k), open('['); }
    void item_obj() { sep(), open('{'); }
    void num(const char* k, double v) {
        key(k);
        if (std::isfinite(v)) {
            char buf[32];
            std::snprintf(buf, sizeof buf, "%.17g", v);
            out << buf;
        } else {
            out << "null";
        }
    }
    void integer(const char* k, long long v) { key(k), out << v; }
    void str(const char* k, const std::string& v) { key(k), out << quote(v); }
    void boolean(const char* k, bool v) { key(k), out << (v ? "true" : "false"); }
    void null(const char* k) { key(k), out << "null"; }
    void str_or_null(const char* k, const std::string& v) { v.empty() ? null(k) : str(k, v); }
};

void write_stats(Json& j, const std::optional<WindowStats>& w) {
    if (!w) return j.null("stats");
    j.begin_obj("stats");
    j.num("seconds", w->seconds);
    j.integer("samples", w->samples);
    j.integer("failed_reads", w->failed_reads);
    // Without a reading the means are unknown, not zero.
    const char* means[] = {"sm_mhz", "mem_mhz", "power_w", "gfx_activity_percent", "temp_c_max",
                           "power_cap_share", "thermal_share"};
    const double values[] = {w->sm_mhz, w->mem_mhz, w->power_w, w->activity, w->temp_c_max,
                             w->power_cap_share, w->thermal_share};
    for (int i = 0; i < 7; ++i) {
        if (w->samples > 0) j.num(means[i], values[i]);
        else j.null(means[i]);
    }
    j.boolean("new_process", w->new_process);
    j.close('}');
}

void write_sample(Json& j, const char* k, const Sample& s) {
    j.begin_obj(k);
    j.integer("launches", s.launches);
    j.num("ms_per_launch", s.ms_per_launch);
    j.num("sample_ms", s.sample_ms);
    write_stats(j, s.stats);
    j.close('}');
}

void write_side(Json& j, const char* k, const Side& s) {
    j.begin_obj(k);
    j.integer("launches_per_sample", s.launches_per_sample);
    j.num("min_sample_ms", s.min_sample_ms);
    j.num("ms_per_launch", s.ms_per_launch);
    j.num("gbs", s.gbs);
    j.num("rated_fraction", s.rated_fraction);
    if (s.clock_adjusted_fraction) j.num("clock_adjusted_fraction", *s.clock_adjusted_fraction);
    else j.null("clock_adjusted_fraction");
    j.num("tflops", s.tflops);
    j.num("rated_compute_fraction", s.rated_compute_fraction);
    if (s.clock_adjusted_compute_fraction) j.num("clock_adjusted_compute_fraction", *s.clock_adjusted_compute_fraction);
    else j.null("clock_adjusted_compute_fraction");
    write_stats(j, s.stats);
    j.close('}');
}

void write_check(Json& j, const char* k, const std::optional<OutputCheck>& c) {
    if (!c) return j.null(k);
    j.begin_obj(k);
    j.num("rel_l2", c->rel_l2);
    j.num("max_abs", c->max_abs);
    j.num("max_abs_baseline", c->max_abs_baseline);
    j.integer("nonfinite", (long long)c->nonfinite);
    j.boolean("deterministic", c->deterministic);
    j.close('}');
}

void write_case(Json& j, const CaseResult& r) {
    j.item_obj();
    j.str("benchmark", r.spec.benchmark);
    j.str("label", r.spec.label);
    j.str_or_null("layout", r.spec.layout);
    j.str_or_null("epilogue", r.spec.epilogue);
    j.str_or_null("baseline_name", r.spec.baseline_name);
    j.integer("size_bytes", (long long)r.spec.size_bytes);
    j.num("bytes_moved", r.spec.bytes_moved);
    j.num("flops", r.spec.flops);
    j.num("peak_flop_per_cu_per_clock", r.spec.peak_flop_per_cu_per_clock);
    j.integer("rotation_sets", r.spec.rotation_sets);
    j.boolean("one_sided", r.one_sided);
    j.num("warmup_seconds", r.warmup_seconds);
    j.boolean("ok", r.ok());
    j.boolean("outputs_match", r.outputs_match);
    write_check(j, "output_check", r.output_check);
    write_check(j, "pre_check", r.pre_check);
    if (r.baseline_algorithm) {
        const BaselineAlgorithm& a = *r.baseline_algorithm;
        j.begin_obj("baseline_algorithm");
        j.str("selection", lt_algo_name(a.selection));
        j.integer("used", a.used);
        j.begin_arr("candidates");
        for (const Candidate& c : a.candidates) {
            j.item_obj();
            j.integer("index", c.index);
            j.integer("solution_index", c.solution_index);
            j.integer("workspace_bytes", (long long)c.workspace_bytes);
            j.num("waves_count", c.waves_count);
            j.str("status", c.status);
            if (c.ms_per_launch) j.num("ms_per_launch", *c.ms_per_launch);
            else j.null("ms_per_launch");
            j.close('}');
        }
        j.close(']');
        j.close('}');
    } else {
        j.null("baseline_algorithm");
    }
    j.integer("valid_rounds", r.valid_rounds);
    j.boolean("enough_rounds", r.enough_rounds);
    if (r.one_sided) {
        j.null("ratio");
    } else {
        j.begin_obj("ratio");
        j.num("median", r.ratio_median);
        j.num("min", r.ratio_min);
        j.num("max", r.ratio_max);
        j.close('}');
    }
    write_side(j, "flint", r.flint);
    if (r.one_sided) j.null("baseline");
    else write_side(j, "baseline", r.baseline);
    j.begin_arr("rounds");
    for (const Round& round : r.rounds) {
        j.item_obj();
        j.boolean("flint_first", round.flint_first);
        j.boolean("valid", round.valid);
        j.str_or_null("discard_reason", round.discard_reason);
        write_sample(j, "flint", round.flint);
        if (r.one_sided) {
            j.null("baseline");
            j.null("ratio");
        } else {
            write_sample(j, "baseline", round.baseline);
            j.num("ratio", round.ratio);
        }
        j.close('}');
    }
    j.close(']');
    j.close('}');
}

std::string run_text(const std::string& cmd) {
    std::string text;
    FILE* f = popen(cmd.c_str(), "r");
    if (!f) return text;
    char buf[256];
    while (std::fgets(buf, sizeof buf, f)) text += buf;
    if (pclose(f) != 0) return "";
    while (!text.empty() && (text.back() == '\n' || text.back() == '\r')) text.pop_back();
    return text;
}

std::filesystem::path exe_dir() {
    std::error_code ec;
    const auto p = std::filesystem::read_symlink("/proc/self/exe", ec);
    return ec ? std::filesystem::current_path() : p.parent_path();
}

std::string utc_now(const char* format) {
    const std::time_t t = std::time(nullptr);
    std::tm tm{};
    gmtime_r(&t, &tm);
    char buf[64];
    std::strftime(buf, sizeof buf, format, &tm);
    return buf;
}

struct AtStart {
    bool monitored = false;
    int other_processes = -1, utilization_percent = -1;
};

std::string report(const Command& c, const DeviceInfo& d, const std::vector<CaseResult>& cases, const AtStart& at) {
    // The repository root is three levels above build/release/bin.
    const std::string root = (exe_dir() / ".." / ".." / "..").lexically_normal().string();
    std::string sha = run_text("git -C '" + root + "' rev-parse HEAD 2>/dev/null");
    const std::string dirty = sha.empty() ? "" : run_text("git -C '" + root + "' status --porcelain 2>/dev/null");
    // A copy of the tree without its .git (a build shipped to another machine)
    // can name its commit through FLINT_GIT_SHA; it is then taken as clean.
    const char* env_sha = std::getenv("FLINT_GIT_SHA");
    if (sha.empty() && env_sha && *env_sha) sha = env_sha;
    Json j;
    j.open('{');
    j.str("schema", "flint-bench/1");
    j.str("benchmark", benchmark_name(c.benchmark));
    j.boolean("quick", c.options.quick);
    j.boolean("standard_protocol", standard_protocol(c.options));
    j.begin_arr("args");
    for (const std::string& a : c.args) j.sep(), j.out << Json::quote(a);
    j.close(']');
    j.begin_obj("git");
    j.str("sha", sha.empty() ? "unknown" : sha);
    j.boolean("dirty", !dirty.empty());
    j.close('}');
    j.str("timestamp_utc", utc_now("%Y-%m-%dT%H:%M:%SZ"));
    j.begin_obj("device");
    j.str("name", d.name);
    j.str("arch", d.arch);
    j.str("compute_capability", d.compute_capability);
    j.integer("cu_count", d.cu_count);
    j.num("rated_sm_clock_mhz", d.rated_clock_mhz);
    j.num("memory_clock_mhz", d.memory_clock_mhz);
    j.integer("bus_width_bits", d.bus_width);
    j.num("rated_bandwidth_gbs", kRatedBandwidthGBs);
    j.num("peak_fp16_tflops", kPeakFlopPerCuPerClock * d.cu_count * d.rated_clock_mhz * 1e6 / 1e12);
    j.integer("total_bytes", (long long)d.total_bytes);
    j.integer("l2_per_xcd_bytes", (long long)d.l2_per_xcd_bytes);
    j.integer("l2_bytes", (long long)d.llc_bytes);
    j.close('}');
    j.begin_obj("options");
    j.num("warmup_seconds", c.options.warmup_seconds);
    j.num("sample_ms", c.options.sample_ms);
    j.integer("rounds", c.options.rounds);
    j.integer("max_rounds", c.options.max_rounds);
    j.boolean("allow_busy", c.options.allow_busy);
    j.boolean("quick", c.options.quick);
    j.str("lt_algo", lt_algo_name(c.options.lt_algo));
    j.close('}');
    j.begin_obj("gpu_at_start");
    j.boolean("process_detection", at.other_processes >= 0);
    if (at.other_processes >= 0) j.integer("other_processes", at.other_processes);
    else j.null("other_processes");
    if (at.utilization_percent >= 0) j.integer("utilization_percent", at.utilization_percent);
    else j.null("utilization_percent");
    j.close('}');
    j.str("monitor", at.monitored ? "amd-smi gpu metrics, ~10 ms samples" : "unavailable: amd-smi could not open the device");
    j.begin_arr("cases");
    for (const CaseResult& r : cases) write_case(j, r);
    j.close(']');
    j.close('}');
    return j.out.str() + "\n";
}

void print_case(const CaseResult& r) {
    std::string name = r.spec.benchmark;
    if (!r.spec.layout.empty()) {
        name += " " + r.spec.layout;
        if (r.spec.epilogue != "none") name += "+" + r.spec.epilogue;
    }
    name += " " + r.spec.label;
    std::printf("%-44s flint %9.4f ms", name.c_str(), r.flint.ms_per_launch);
    if (r.spec.flops > 0) std::printf(" %8.1f TFLOP/s (%5.1f%%)", r.flint.tflops, 100 * r.flint.rated_compute_fraction);
    if (r.spec.bytes_moved > 0) std::printf(" %8.1f GB/s (%5.1f%%)", r.flint.gbs, 100 * r.flint.rated_fraction);
    if (!r.one_sided) {
        std::printf(" | %s %9.4f ms", r.spec.baseline_name.c_str(), r.baseline.ms_per_launch);
        if (r.spec.flops > 0) std::printf(" %8.1f TFLOP/s", r.baseline.tflops);
        if (r.spec.bytes_moved > 0) std::printf(" %8.1f GB/s", r.baseline.gbs);
        std::printf(" | ratio %.3f [%.3f, %.3f]", r.ratio_median, r.ratio_min, r.ratio_max);
    }
    std::printf(" %s\n", r.ok() ? "ok" : r.outputs_match ? "TOO FEW ROUNDS" : "OUTPUT MISMATCH");
    std::fflush(stdout);
}

int run(const Command& c) {
    const DeviceInfo d = device_info();
    Monitor mon;
    AtStart at;
    at.monitored = mon.available();
    at.other_processes = mon.other_processes();
    at.utilization_percent = mon.utilization_percent();
    if (at.other_processes > 0) {
        const std::string what = "the GPU is busy: " + std::to_string(at.other_processes) +
                                 " other process(es) hold it; run with --allow-busy to measure anyway";
        if (!c.options.allow_busy) throw Failure(what);
        std::fprintf(stderr, "flint_bench: warning: %s\n", what.c_str());
    }
    hipStream_t s = nullptr;
    hip_check(hipStreamCreate(&s), "hipStreamCreate");
    std::vector<CaseResult> cases;
    std::optional<LtContext> lt;
    if (c.benchmark == Benchmark::Gemm) lt.emplace();
    if (c.benchmark == Benchmark::Copy)
        for (unsigned long long bytes : c.sizes) cases.push_back(copy_case(bytes, d, c.options, s, mon)), print_case(cases.back());
    if (c.benchmark == Benchmark::Mma)
        for (int chains : c.chains) cases.push_back(mma_case(chains, d, c.options, s, mon)), print_case(cases.back());
    if (c.benchmark == Benchmark::Gemm)
        for (const Shape& sh : c.shapes)
            cases.push_back(gemm_case(sh, c.layout, c.epilogue, d, c.options, s, *lt, mon)), print_case(cases.back());
    hip_check(hipStreamDestroy(s), "hipStreamDestroy");

    std::filesystem::path out = c.out;
    if (out.empty()) {
        std::string gpu = d.name;
        for (char& ch : gpu)
            if (!std::isalnum((unsigned char)ch)) ch = '-';
        out = exe_dir() / ".." / "bench-results" /
              (std::string(benchmark_name(c.benchmark)) + "-" + gpu + "-" + utc_now("%Y%m%dT%H%M%SZ") + ".json");
    }
    if (out.has_parent_path()) std::filesystem::create_directories(out.parent_path());
    const std::string text = report(c, d, cases, at);
    FILE* f = std::fopen(out.string().c_str(), "wb");
    if (!f || std::fwrite(text.data(), 1, text.size(), f) != text.size() || std::fclose(f) != 0)
        throw Failure("cannot write " + out.string());
    std::printf("wrote %s\n", out.string().c_str());
    bool all_ok = true;
    for (const CaseResult& r : cases) all_ok = all_ok && r.ok();
    return all_ok ? 0 : 1;
}

}  // namespace
}  // namespace fb

int main(int argc, char** argv) {
    fb::Command c;
    try {
        c = fb::parse(argc, argv);
    } catch (const fb::UsageError& e) {
        std::fprintf(stderr, "flint_bench: %s\nrun 'flint_bench --help' for the options\n", e.what());
        return 2;
    }
    if (c.help) {
        std::fputs(fb::usage().c_str(), stdout);
        return 0;
    }
    try {
        return fb::run(c);
    } catch (const std::exception& e) {
        std::fprintf(stderr, "flint_bench: error: %s\n", e.what());
        return 1;
    }
}
