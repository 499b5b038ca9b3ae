// flint_bench's command line: the benchmark, its cases and the measurement
// protocol's options. Mirrors the reference's option set and error messages
// (ref bench/cli.h:1-56, bench/cli.cpp:222-516); parsing needs no GPU.
#pragma once

#include <stdexcept>
#include <string>
#include <vector>

namespace fb {

// A command-line mistake: main prints "flint_bench: <what>" and exits 2.
struct UsageError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

enum class Benchmark { None, Copy, Mma, Gemm };
enum class Layout { NT, NN, TN };
enum class Epilogue { None, Bias, BiasGelu, BiasResidual, DGelu };
enum class LtAlgo { Fastest, First };

struct Shape {
    long long m = 0, n = 0, k = 0;
    std::string label;   // as typed, "8192x768x768"
};

struct Options {
    double warmup_seconds = 1.5;
    double sample_ms = 100;
    int rounds = 10;
    int max_rounds = 30;
    bool allow_busy = false;
    bool quick = false;
    LtAlgo lt_algo = LtAlgo::Fastest;
};

struct Command {
    Benchmark benchmark = Benchmark::None;
    bool help = false;
    std::vector<unsigned long long> sizes;   // copy
    std::vector<int> chains;                 // mma
    Layout layout = Layout::NT;              // gemm
    Epilogue epilogue = Epilogue::None;      // gemm
    std::vector<Shape> shapes;               // gemm
    Options options;
    std::string out;                         // empty: the default path
    std::vector<std::string> args;           // argv[1:] without --out and its path
};

// Parses argv; throws UsageError. A command with help set runs nothing.
Command parse(int argc, char** argv);

std::string usage();

const char* benchmark_name(Benchmark b);
const char* layout_name(Layout l);
const char* epilogue_name(Epilogue e);
const char* lt_algo_name(LtAlgo a);

// Whether the options meet the published protocol: at least 10 rounds, a 1 s
// warm-up and 100 ms samples, outside --quick (ref bench/harness.h:178).
bool standard_protocol(const Options& o);

}  // namespace fb
