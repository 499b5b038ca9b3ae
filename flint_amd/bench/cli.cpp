// flint_bench's command-line parser. The option names, defaults and error
// texts are the reference's interface (ref bench/cli.cpp:222-444; the help
// text below is this harness's own), so scripts and tests written against it read the same; the case
// lists name the same GPT-2 124M shapes at 8,192 tokens.
#include "cli.h"

#include <cctype>
#include <cerrno>
#include <cstdlib>
#include <map>

namespace fb {
namespace {

constexpr long long kMaxMN = 8388480;   // flint_gemm_*: m and n up to this
constexpr long long kMaxK = 65536;

[[noreturn]] void fail(const std::string& what) { throw UsageError(what); }

std::vector<std::string> split(const std::string& text) {
    std::vector<std::string> items;
    size_t start = 0;
    for (;;) {
        const size_t comma = text.find(',', start);
        items.push_back(text.substr(start, comma == std::string::npos ? std::string::npos : comma - start));
        if (comma == std::string::npos) return items;
        start = comma + 1;
    }
}

bool all_digits(const std::string& s) {
    if (s.empty()) return false;
    for (char c : s)
        if (!std::isdigit(static_cast<unsigned char>(c))) return false;
    return true;
}

// Digits only, at most 18 of them (so the value fits a long long).
bool parse_count(const std::string& s, long long& value) {
    if (!all_digits(s) || s.size() > 18) return false;
    value = std::atoll(s.c_str());
    return true;
}

int parse_int(const std::string& option, const std::string& text) {
    long long v = 0;
    if (!parse_count(text, v)) fail(option + ": not an integer: '" + text + "'");
    if (v < 1 || v > 1000000) fail(option + ": must be between 1 and 1000000: '" + text + "'");
    return static_cast<int>(v);
}

double parse_double(const std::string& option, const std::string& text) {
    errno = 0;
    char* end = nullptr;
    const double v = std::strtod(text.c_str(), &end);
    if (text.empty() || end != text.c_str() + text.size() || errno != 0 || !(v == v))
        fail(option + ": not a number: '" + text + "'");
    return v;
}

std::vector<unsigned long long> parse_sizes(const std::string& text) {
    std::vector<unsigned long long> sizes;
    for (const std::string& item : split(text)) {
        std::string digits = item;
        unsigned long long scale = 1;
        if (!digits.empty()) {
            const char suffix = digits.back();
            if (suffix == 'K' || suffix == 'M' || suffix == 'G') {
                scale = suffix == 'K' ? 1ull << 10 : suffix == 'M' ? 1ull << 20 : 1ull << 30;
                digits.pop_back();
            }
        }
        long long v = 0;
        if (!parse_count(digits, v)) fail("--sizes: not a size: '" + item + "'");
        if (v == 0) fail("--sizes: sizes must be positive: '" + item + "'");
        if (static_cast<unsigned long long>(v) > (64ull << 30) / scale)
            fail("--sizes: size too large: '" + item + "'");
        sizes.push_back(static_cast<unsigned long long>(v) * scale);
    }
    return sizes;
}

std::vector<int> parse_chains(const std::string& text) {
    std::vector<int> chains;
    for (const std::string& item : split(text)) {
        if (item != "4" && item != "8" && item != "16") fail("--chains: must be 4, 8 or 16: '" + item + "'");
        chains.push_back(std::atoi(item.c_str()));
    }
    return chains;
}

Shape parse_shape(const std::string& item, Layout layout, Epilogue epilogue) {
    const std::string bad = "--shapes: not a shape MxNxK of positive integers: '" + item + "'";
    const size_t x1 = item.find('x');
    const size_t x2 = x1 == std::string::npos ? x1 : item.find('x', x1 + 1);
    if (x2 == std::string::npos || item.find('x', x2 + 1) != std::string::npos) fail(bad);
    Shape s;
    s.label = item;
    if (!parse_count(item.substr(0, x1), s.m) || !parse_count(item.substr(x1 + 1, x2 - x1 - 1), s.n) ||
        !parse_count(item.substr(x2 + 1), s.k))
        fail(bad);
    if (s.m == 0 || s.n == 0 || s.k == 0) fail("--shapes: dimensions must be positive: '" + item + "'");
    if (s.m > kMaxMN || s.n > kMaxMN || s.k > kMaxK)
        fail("--shapes: past the limits (M up to " + std::to_string(kMaxMN) + ", N up to " +
             std::to_string(kMaxMN) + ", K up to " + std::to_string(kMaxK) + "): '" + item + "'");
    if (layout != Layout::TN && s.k % 8 != 0) fail("--shapes: K must be a multiple of 8: '" + item + "'");
    if (layout == Layout::NN && s.n % 8 != 0)
        fail("--shapes: N must be a multiple of 8 with --layout nn: '" + item + "'");
    if (layout == Layout::TN && s.m % 8 != 0)
        fail("--shapes: M must be a multiple of 8 with --layout tn: '" + item + "'");
    if (layout == Layout::TN && s.n % 8 != 0)
        fail("--shapes: N must be a multiple of 8 with --layout tn: '" + item + "'");
    if (epilogue == Epilogue::BiasGelu && s.n % 8 != 0)
        fail("--shapes: N must be a multiple of 8 with --epilogue bias-gelu: '" + item + "'");
    if (epilogue == Epilogue::BiasResidual && s.n % 2 != 0)
        fail("--shapes: N must be even with --epilogue bias-residual: '" + item + "'");
    return s;
}

// The GPT-2 124M layers at 8,192 tokens (C = 768, MLP 3072, qkv 2304, vocab
// padded to 50304), per layout and epilogue.
std::string default_shapes(Layout layout, Epilogue epilogue) {
    switch (epilogue) {
    case Epilogue::Bias: return "8192x2304x768,8192x768x768,8192x3072x768,8192x768x3072";
    case Epilogue::BiasGelu: return "8192x3072x768";
    case Epilogue::BiasResidual: return "8192x768x768,8192x768x3072";
    case Epilogue::DGelu: return "8192x3072x768";
    case Epilogue::None: break;
    }
    switch (layout) {
    case Layout::NN: return "8192x768x2304,8192x768x768,8192x768x3072,8192x3072x768,8192x768x50304";
    case Layout::TN: return "2304x768x8192,768x768x8192,3072x768x8192,768x3072x8192,50304x768x8192";
    case Layout::NT: break;
    }
    return "8192x2304x768,8192x768x768,8192x3072x768,8192x768x3072,8192x50304x768";
}

}  // namespace

const char* benchmark_name(Benchmark b) {
    switch (b) {
    case Benchmark::Copy: return "copy";
    case Benchmark::Mma: return "mma";
    case Benchmark::Gemm: return "gemm";
    case Benchmark::None: break;
    }
    return "";
}

const char* layout_name(Layout l) { return l == Layout::NT ? "nt" : l == Layout::NN ? "nn" : "tn"; }

const char* epilogue_name(Epilogue e) {
    switch (e) {
    case Epilogue::Bias: return "bias";
    case Epilogue::BiasGelu: return "bias-gelu";
    case Epilogue::BiasResidual: return "bias-residual";
    case Epilogue::DGelu: return "dgelu";
    case Epilogue::None: break;
    }
    return "none";
}

const char* lt_algo_name(LtAlgo a) { return a == LtAlgo::First ? "first" : "fastest"; }

bool standard_protocol(const Options& o) {
    return !o.quick && o.rounds >= 10 && o.warmup_seconds >= 1.0 && o.sample_ms >= 100;
}

Command parse(int argc, char** argv) {
    Command c;
    std::vector<std::string> all;
    for (int i = 1; i < argc; ++i) all.push_back(argv[i]);
    // The log records the arguments without --out and its path, so that no
    // local path reaches it.
    for (size_t i = 0; i < all.size(); ++i) {
        if (all[i] == "--out") {
            ++i;
            continue;
        }
        if (all[i].rfind("--out=", 0) == 0) continue;
        c.args.push_back(all[i]);
    }

    // Options as given; their meaning is settled once the benchmark is known.
    std::map<std::string, std::string> given;
    std::string benchmark;
    bool have_benchmark = false;
    static const char* kValued[] = {"--sizes", "--chains", "--layout", "--epilogue", "--lt-algo", "--shapes",
                                    "--rounds", "--max-rounds", "--warmup", "--sample-ms", "--out"};
    static const char* kFlags[] = {"--allow-busy", "--quick", "--help"};
    for (size_t i = 0; i < all.size(); ++i) {
        const std::string& arg = all[i];
        if (arg.rfind("--", 0) != 0) {
            if (have_benchmark) fail("unexpected argument: " + arg);
            benchmark = arg;
            have_benchmark = true;
            continue;
        }
        const size_t eq = arg.find('=');
        const std::string name = arg.substr(0, eq);
        bool valued = false, flag = false;
        for (const char* v : kValued) valued = valued || name == v;
        for (const char* f : kFlags) flag = flag || name == f;
        if (!valued && !flag) fail("unknown option: " + name);
        if (flag) {
            if (eq != std::string::npos) fail(name + " takes no value");
            given[name] = "";
            continue;
        }
        std::string value;
        if (eq != std::string::npos) {
            value = arg.substr(eq + 1);
        } else {
            if (i + 1 >= all.size()) fail(name + " needs a value");
            value = all[++i];
        }
        given[name] = value;
    }
    c.help = given.count("--help") != 0;

    auto has = [&](const char* name) { return given.count(name) != 0; };
    // Values first, so a bad value is named before a misplaced option.
    if (has("--layout")) {
        const std::string& v = given["--layout"];
        if (v == "nt") c.layout = Layout::NT;
        else if (v == "nn") c.layout = Layout::NN;
        else if (v == "tn") c.layout = Layout::TN;
        else fail("--layout: must be nt, nn or tn: '" + v + "'");
    }
    if (has("--epilogue")) {
        const std::string& v = given["--epilogue"];
        if (v == "none") c.epilogue = Epilogue::None;
        else if (v == "bias") c.epilogue = Epilogue::Bias;
        else if (v == "bias-gelu") c.epilogue = Epilogue::BiasGelu;
        else if (v == "bias-residual") c.epilogue = Epilogue::BiasResidual;
        else if (v == "dgelu") c.epilogue = Epilogue::DGelu;
        else fail("--epilogue: must be none, bias, bias-gelu, bias-residual or dgelu: '" + v + "'");
    }
    if (has("--lt-algo")) {
        const std::string& v = given["--lt-algo"];
        if (v == "fastest") c.options.lt_algo = LtAlgo::Fastest;
        else if (v == "first") c.options.lt_algo = LtAlgo::First;
        else fail("--lt-algo: must be fastest or first: '" + v + "'");
    }
    c.options.quick = has("--quick");
    c.options.allow_busy = has("--allow-busy");
    if (c.options.quick) {
        c.options.warmup_seconds = 0.2;
        c.options.sample_ms = 10;
        c.options.rounds = 3;
        c.options.max_rounds = 6;
    }
    if (has("--rounds")) c.options.rounds = parse_int("--rounds", given["--rounds"]);
    if (has("--max-rounds")) {
        c.options.max_rounds = parse_int("--max-rounds", given["--max-rounds"]);
    } else if (has("--rounds")) {
        c.options.max_rounds = c.options.rounds > 30 ? 3 * c.options.rounds : 30;
    }
    if (has("--warmup")) {
        c.options.warmup_seconds = parse_double("--warmup", given["--warmup"]);
        if (c.options.warmup_seconds < 0) fail("--warmup: must not be negative: '" + given["--warmup"] + "'");
    }
    if (has("--sample-ms")) {
        c.options.sample_ms = parse_double("--sample-ms", given["--sample-ms"]);
        if (!(c.options.sample_ms > 0)) fail("--sample-ms: must be positive: '" + given["--sample-ms"] + "'");
    }
    if (has("--out")) {
        c.out = given["--out"];
        if (c.out.empty()) fail("--out: empty path");
    }

    if (!have_benchmark) {
        if (c.help) return c;
        fail("no benchmark given");
    }
    if (benchmark == "copy") c.benchmark = Benchmark::Copy;
    else if (benchmark == "mma") c.benchmark = Benchmark::Mma;
    else if (benchmark == "gemm") c.benchmark = Benchmark::Gemm;
    else fail("unknown benchmark: " + benchmark);

    const bool copy = c.benchmark == Benchmark::Copy, mma = c.benchmark == Benchmark::Mma,
               gemm = c.benchmark == Benchmark::Gemm;
    if (has("--sizes") && !copy) fail("--sizes applies to copy only");
    if (has("--chains") && !mma) fail("--chains applies to mma only");
    if (has("--shapes") && !gemm) fail("--shapes applies to gemm only");
    if (has("--layout") && !gemm) fail("--layout applies to gemm only");
    if (has("--epilogue") && !gemm) fail("--epilogue applies to gemm only");
    if (has("--lt-algo") && !gemm) fail("--lt-algo applies to gemm only");
    if (c.options.max_rounds < c.options.rounds)
        fail("--max-rounds: " + std::to_string(c.options.max_rounds) + " is below --rounds " +
             std::to_string(c.options.rounds));

    if (copy) c.sizes = parse_sizes(has("--sizes") ? given["--sizes"] : "1M,16M,256M");
    if (mma) c.chains = parse_chains(has("--chains") ? given["--chains"] : "4,8,16");
    if (gemm) {
        if (c.epilogue == Epilogue::DGelu && c.layout != Layout::NN) fail("--epilogue dgelu needs --layout nn");
        if (c.epilogue != Epilogue::None && c.epilogue != Epilogue::DGelu && c.layout != Layout::NT)
            fail(std::string("--epilogue ") + epilogue_name(c.epilogue) + " needs --layout nt");
        const std::string list = has("--shapes") ? given["--shapes"] : default_shapes(c.layout, c.epilogue);
        for (const std::string& item : split(list)) c.shapes.push_back(parse_shape(item, c.layout, c.epilogue));
    }
    return c;
}

std::string usage() {
    return "usage: flint_bench <benchmark> [options]\n"
           "\n"
           "Times libflint on this GPU against a vendor baseline and writes a\n"
           "flint-bench/1 JSON log. Options take their value as --name VALUE or\n"
           "--name=VALUE.\n"
           "\n"
           "Benchmarks\n"
           "  copy    bytes moved by flint_copy; baseline hipMemcpyAsync (device to device)\n"
           "  mma     one-sided: a loop of v_mfma_f32_32x32x16_f16 (FP16 in, FP32 sums),\n"
           "          as a fraction of the dense FP16 matrix-core peak\n"
           "  gemm    flint_gemm_nt / _nn / _tn and the fused epilogues; baseline\n"
           "          rocBLAS gemm_ex for plain products, hipBLASLt for epilogues\n"
           "\n"
           "copy\n"
           "  --sizes LIST      byte counts separated by commas; a K, M or G suffix means\n"
           "                    KiB, MiB or GiB. Default 1M,16M,256M\n"
           "mma\n"
           "  --chains LIST     accumulator chains per wave, each 4, 8 or 16. Default 4,8,16\n"
           "gemm\n"
           "  --layout nt|nn|tn which operand is transposed. nt: y[M,N] = x[M,K] w[N,K]^T;\n"
           "                    nn: y = x w with w[K,N]; tn: FP32 y[M,N] += x[K,M]^T w[K,N]\n"
           "                    (timed accumulating). Default nt\n"
           "  --epilogue none|bias|bias-gelu|bias-residual|dgelu\n"
           "                    work fused after the product. With --layout nt only:\n"
           "                      bias           + one FP32 value per column, then round\n"
           "                                     (hipBLASLt BIAS)\n"
           "                      bias-gelu      as bias, then GELU, keeping the pre-GELU\n"
           "                                     values too (hipBLASLt GELU_AUX_BIAS)\n"
           "                      bias-residual  as bias, plus an FP32 residual, into FP32 y\n"
           "                                     (hipBLASLt bias, residual as C, beta 1)\n"
           "                    With --layout nn only:\n"
           "                      dgelu          times GELU'(pre) at a stored FP16 pre\n"
           "                                     (hipBLASLt DGELU)\n"
           "                    Default none\n"
           "  --lt-algo fastest|first\n"
           "                    hipBLASLt baseline for epilogue cases: `fastest` times up\n"
           "                    to 8 heuristic candidates on the case's own buffers and keeps\n"
           "                    the quickest (default); `first` takes the heuristic's top\n"
           "                    pick. Every candidate's time is logged\n"
           "  --shapes LIST     MxNxK items separated by commas. Limits: M, N <= 8388480,\n"
           "                    K <= 65536. nt, nn: K % 8 == 0; nn and bias-gelu: N % 8 == 0;\n"
           "                    bias-residual: N even; tn: M % 8 == 0 and N % 8 == 0, any K.\n"
           "                    Defaults are GPT-2 124M at 8192 tokens:\n"
           "                      nt  8192x2304x768,8192x768x768,8192x3072x768,\n"
           "                          8192x768x3072,8192x50304x768 (bias: all but the\n"
           "                          logits; bias-gelu: 8192x3072x768; bias-residual:\n"
           "                          8192x768x768 and 8192x768x3072)\n"
           "                      nn  8192x768x2304,8192x768x768,8192x768x3072,\n"
           "                          8192x3072x768,8192x768x50304 (dgelu: 8192x3072x768)\n"
           "                      tn  2304x768x8192,768x768x8192,3072x768x8192,\n"
           "                          768x3072x8192,50304x768x8192\n"
           "\n"
           "Protocol\n"
           "  --rounds N        valid interleaved rounds a case needs (default 10)\n"
           "  --max-rounds N    give up after this many rounds (default 30; 3 x --rounds\n"
           "                    when that is larger)\n"
           "  --warmup SECONDS  untimed launches first, per case (default 1.5)\n"
           "  --sample-ms MS    minimum length of one timed sample (default 100)\n"
           "  --quick           test-sized protocol whose numbers are not results:\n"
           "                    --warmup 0.2 --sample-ms 10 --rounds 3 --max-rounds 6,\n"
           "                    each overridable\n"
           "  --allow-busy      do not refuse to start while other processes use the GPU\n"
           "  --out PATH        where the JSON goes (default: a file in bench-results/ next\n"
           "                    to the binary, named for benchmark, GPU and start time)\n"
           "  --help            print this and exit\n";
}

}  // namespace fb
