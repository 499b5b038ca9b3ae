// flint_bench's device monitor (the counterpart of the reference's NVML
// monitor, ref bench/monitor.h:1-123): a thread samples the GPU's metrics
// table through amd-smi every ~10 ms, and each timed sample is judged by the
// window of samples taken while it ran.
//
// Per sample: the graphics clock (mean over the XCDs' current clocks), the
// memory clock, socket power, the hotspot temperature, graphics activity, and
// the firmware's accumulated power-cap (PPT) and socket-thermal residencies,
// whose growth over a window, divided by the growth of its accumulation
// counter, is the share of the window spent throttled. Processes other than
// this one on the GPU are listed before and after each round.
//
// The monitor is optional: when amd-smi cannot open the device (no driver
// interface, no permission), `available()` is false and callers report null
// statistics instead.
#pragma once

#include <amd_smi/amdsmi.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdio>
#include <mutex>
#include <optional>
#include <string>
#include <thread>
#include <unistd.h>
#include <vector>

namespace fb {

struct WindowStats {
    double seconds = 0;
    long long samples = 0, failed_reads = 0;
    double sm_mhz = 0, mem_mhz = 0, power_w = 0, activity = 0;   // means over the window
    double temp_c_max = 0;
    double power_cap_share = 0, thermal_share = 0;               // of the window, from the residencies
    bool new_process = false;                                    // another process appeared
};

class Monitor {
public:
    Monitor() {
        if (amdsmi_init(AMDSMI_INIT_AMD_GPUS) != AMDSMI_STATUS_SUCCESS) return;
        initialised_ = true;
        if (!find_device()) return;
        t0_ = std::chrono::steady_clock::now();
        thread_ = std::thread([this] { loop(); });
    }
    ~Monitor() {
        stop_ = true;
        if (thread_.joinable()) thread_.join();
        if (initialised_) (void)amdsmi_shut_down();
    }
    Monitor(const Monitor&) = delete;
    Monitor& operator=(const Monitor&) = delete;

    bool available() const { return thread_.joinable(); }
    double now() const { return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0_).count(); }

    // Processes other than this one that hold the GPU; -1 when unknown.
    int other_processes() const {
        if (!handle_) return -1;
        uint32_t n = 64;
        std::vector<amdsmi_proc_info_t> list(n);
        if (amdsmi_get_gpu_process_list(handle_, &n, list.data()) != AMDSMI_STATUS_SUCCESS) return -1;
        int others = 0;
        for (uint32_t i = 0; i < std::min<uint32_t>(n, uint32_t(list.size())); ++i)
            others += list[i].pid != amdsmi_process_handle_t(getpid());
        return others;
    }

    // Graphics activity now, in percent; -1 when unknown.
    int utilization_percent() {
        amdsmi_gpu_metrics_t m;
        if (!handle_ || amdsmi_get_gpu_metrics_info(handle_, &m) != AMDSMI_STATUS_SUCCESS) return -1;
        return m.average_gfx_activity == 0xFFFF ? -1 : int(m.average_gfx_activity);
    }

    // The window [begin, end]; others_at_begin and others_now are
    // other_processes() before and after it.
    WindowStats window(double begin, double end, int others_at_begin, int others_now) {
        WindowStats w;
        w.seconds = end - begin;
        std::lock_guard<std::mutex> lock(mutex_);
        const Sample* first = nullptr;
        const Sample* last = nullptr;
        for (const Sample& s : samples_) {
            if (s.t < begin || s.t > end) continue;
            if (!s.ok) {
                ++w.failed_reads;
                continue;
            }
            ++w.samples;
            w.sm_mhz += s.gfx_mhz;
            w.mem_mhz += s.mem_mhz;
            w.power_w += s.power_w;
            w.activity += s.activity;
            w.temp_c_max = std::max(w.temp_c_max, s.temp_c);
            if (!first) first = &s;
            last = &s;
        }
        // A window shorter than the ~10 ms between readings may hold none:
        // it then takes the last good reading before it, the one in effect
        // when it began (ref bench/monitor.cpp:242-246 holds that reading
        // the same way), so every window of a running monitor has a clock.
        if (w.samples == 0) {
            const Sample* held = nullptr;
            for (const Sample& s : samples_)
                if (s.ok && s.t < begin) held = &s;
            if (held) {
                w.samples = 1;
                w.sm_mhz = held->gfx_mhz;
                w.mem_mhz = held->mem_mhz;
                w.power_w = held->power_w;
                w.activity = held->activity;
                w.temp_c_max = held->temp_c;
            }
        }
        if (w.samples) {
            w.sm_mhz /= w.samples;
            w.mem_mhz /= w.samples;
            w.power_w /= w.samples;
            w.activity /= w.samples;
        }
        if (first && last && last->acc > first->acc) {
            const double span = double(last->acc - first->acc);
            w.power_cap_share = double(last->ppt - first->ppt) / span;
            w.thermal_share = double(last->thm - first->thm) / span;
        }
        w.new_process = others_at_begin >= 0 && others_now > others_at_begin;
        return w;
    }

    // Drops the samples taken before t (no later window will start earlier),
    // except the last good one, which a window without readings of its own
    // holds over.
    void forget_before(double t) {
        std::lock_guard<std::mutex> lock(mutex_);
        auto end = std::find_if(samples_.begin(), samples_.end(),
                                [&](const Sample& s) { return s.t >= t; });
        auto keep = end;
        for (auto it = samples_.begin(); it != end; ++it)
            if (it->ok) keep = it;
        samples_.erase(samples_.begin(), keep == end ? end : keep);
    }

private:
    struct Sample {
        double t = 0;
        bool ok = false;
        double gfx_mhz = 0, mem_mhz = 0, power_w = 0, temp_c = 0, activity = 0;
        uint64_t acc = 0, ppt = 0, thm = 0;
    };

    // The amd-smi device whose PCI address is HIP device 0's.
    bool find_device() {
        char bus[64] = {};
        if (hipDeviceGetPCIBusId(bus, sizeof bus, 0) != hipSuccess) return false;
        unsigned domain = 0, b = 0, d = 0, f = 0;
        if (std::sscanf(bus, "%x:%x:%x.%x", &domain, &b, &d, &f) != 4) return false;
        uint32_t sockets = 0;
        if (amdsmi_get_socket_handles(&sockets, nullptr) != AMDSMI_STATUS_SUCCESS || sockets == 0) return false;
        std::vector<amdsmi_socket_handle> socket_list(sockets);
        if (amdsmi_get_socket_handles(&sockets, socket_list.data()) != AMDSMI_STATUS_SUCCESS) return false;
        for (amdsmi_socket_handle sock : socket_list) {
            uint32_t count = 0;
            if (amdsmi_get_processor_handles(sock, &count, nullptr) != AMDSMI_STATUS_SUCCESS || count == 0) continue;
            std::vector<amdsmi_processor_handle> procs(count);
            if (amdsmi_get_processor_handles(sock, &count, procs.data()) != AMDSMI_STATUS_SUCCESS) continue;
            for (amdsmi_processor_handle p : procs) {
                amdsmi_bdf_t bdf;
                if (amdsmi_get_gpu_device_bdf(p, &bdf) != AMDSMI_STATUS_SUCCESS) continue;
                if (bdf.domain_number == domain && bdf.bus_number == b && bdf.device_number == d &&
                    bdf.function_number == f) {
                    handle_ = p;
                    return true;
                }
            }
        }
        return false;
    }

    Sample read() const {
        Sample s;
        s.t = now();
        amdsmi_gpu_metrics_t m;
        if (amdsmi_get_gpu_metrics_info(handle_, &m) != AMDSMI_STATUS_SUCCESS) return s;
        double sum = 0;
        int n = 0;
        for (int i = 0; i < AMDSMI_MAX_NUM_GFX_CLKS; ++i)
            if (m.current_gfxclks[i] != 0 && m.current_gfxclks[i] != 0xFFFF) sum += m.current_gfxclks[i], ++n;
        if (n) s.gfx_mhz = sum / n;
        else if (m.current_gfxclk != 0xFFFF) s.gfx_mhz = m.current_gfxclk;
        else s.gfx_mhz = m.average_gfxclk_frequency;
        s.mem_mhz = m.current_uclk != 0xFFFF ? m.current_uclk : m.average_uclk_frequency;
        s.power_w = m.current_socket_power != 0xFFFF ? m.current_socket_power : m.average_socket_power;
        s.temp_c = m.temperature_hotspot != 0xFFFF ? m.temperature_hotspot : 0;
        s.activity = m.average_gfx_activity != 0xFFFF ? m.average_gfx_activity : 0;
        s.acc = m.accumulation_counter;
        s.ppt = m.ppt_residency_acc;
        s.thm = m.socket_thm_residency_acc;
        s.ok = s.gfx_mhz > 0 && s.gfx_mhz < 0xFFFF;
        return s;
    }

    void loop() {
        while (!stop_) {
            const Sample s = read();
            {
                std::lock_guard<std::mutex> lock(mutex_);
                samples_.push_back(s);
            }
            std::this_thread::sleep_for(std::chrono::milliseconds(10));
        }
    }

    bool initialised_ = false;
    amdsmi_processor_handle handle_ = nullptr;
    std::chrono::steady_clock::time_point t0_ = std::chrono::steady_clock::now();
    std::atomic<bool> stop_{false};
    std::mutex mutex_;
    std::vector<Sample> samples_;
    std::thread thread_;
};

}  // namespace fb
