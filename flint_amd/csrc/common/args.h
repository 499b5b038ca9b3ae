// Argument checking for the C-ABI entry points.
//
// An entry point describes its device buffers as Spans and runs a Checker
// chain over them and its sizes. Each link of the chain runs only while every
// earlier link has passed; the first failing link writes the entry point's
// message ("<function>: <what>") for flint_last_error and the chain's status
// becomes FLINT_ERROR_INVALID_ARGUMENT. The order of the links is the order in
// which the reference reports problems, and the message texts are its texts
// (its tests match both), so each entry point spells its chain out in that
// order.
#pragma once

#include <cstddef>
#include <cstdint>
#include <initializer_list>

#include "common/common.h"

namespace flint {

// One device buffer of a call: its parameter name, its address and the bytes
// the call reads or writes there.
struct Span {
    const char* name;
    const void* at;
    size_t bytes;

    uintptr_t begin() const { return reinterpret_cast<uintptr_t>(at); }
    bool null() const { return at == nullptr; }
    bool aligned() const { return begin() % 16 == 0; }
    // [at, at + bytes) does not wrap past the top of the address space.
    bool in_space() const { return bytes <= UINTPTR_MAX - begin(); }
    bool meets(const Span& o) const {
        return begin() < o.begin() + o.bytes && o.begin() < begin() + bytes;
    }
};

class Checker {
public:
    explicit Checker(const char* function) : function_(function) {}

    // Fails with "<function>: <format...>" unless `ok`.
    Checker& require(bool ok, const char* format, ...) __attribute__((__format__(__printf__, 3, 4)));

    // Operand checks grouped by kind: every span is tested for null, then
    // every span for alignment, then every span for wrap. (The GEMM entry
    // points report problems in this order.)
    Checker& operands(std::initializer_list<Span> spans);

    // Buffer checks span by span: null, alignment and wrap of the first span,
    // then of the second, and so on; then no span among the first `outputs`
    // may overlap a span listed after it ("a and b overlap", in list order).
    Checker& buffers(const Span* spans, size_t count, size_t outputs);
    Checker& buffers(std::initializer_list<Span> spans, size_t outputs) {
        return buffers(spans.begin(), spans.size(), outputs);
    }

    // "<first> and <other> overlap" for the first `other` that meets `first`.
    Checker& apart(const Span& first, std::initializer_list<Span> others);

    // A caller-provided workspace of at least `needed` bytes (checked only
    // when needed > 0): "needs N bytes of workspace, given M" (M = 0 for a
    // null workspace), then its alignment and wrap.
    Checker& workspace(const void* at, size_t given, size_t needed);

    bool ok() const { return status_ == FLINT_OK; }
    flint_status status() const { return status_; }

private:
    Checker& one(const Span& s, int kind);

    const char* function_;
    flint_status status_ = FLINT_OK;
};

}  // namespace flint
