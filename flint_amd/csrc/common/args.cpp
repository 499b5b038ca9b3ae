#include "common/args.h"

#include <cstdarg>
#include <cstdio>

namespace flint {

namespace {

enum Kind { kNull, kAlign, kWrap };

const char* const kKindText[] = {"is null", "is not 16-byte aligned",
                                 "runs past the end of the address space"};

bool passes(const Span& s, int kind) {
    switch (kind) {
    case kNull: return !s.null();
    case kAlign: return s.aligned();
    default: return s.in_space();
    }
}

}  // namespace

Checker& Checker::require(bool ok, const char* format, ...) {
    if (!this->ok() || ok) return *this;
    char what[448];
    va_list args;
    va_start(args, format);
    std::vsnprintf(what, sizeof what, format, args);
    va_end(args);
    status_ = fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: %s", function_, what);
    return *this;
}

Checker& Checker::one(const Span& s, int kind) {
    return require(passes(s, kind), "%s %s", s.name, kKindText[kind]);
}

Checker& Checker::operands(std::initializer_list<Span> spans) {
    for (int kind : {kNull, kAlign, kWrap})
        for (const Span& s : spans) one(s, kind);
    return *this;
}

Checker& Checker::buffers(const Span* spans, size_t count, size_t outputs) {
    for (size_t i = 0; i < count; ++i)
        for (int kind : {kNull, kAlign, kWrap}) one(spans[i], kind);
    for (size_t i = 0; i < outputs && i < count; ++i)
        for (size_t j = i + 1; j < count; ++j)
            require(!spans[i].meets(spans[j]), "%s and %s overlap", spans[i].name, spans[j].name);
    return *this;
}

Checker& Checker::apart(const Span& first, std::initializer_list<Span> others) {
    for (const Span& o : others) require(!first.meets(o), "%s and %s overlap", first.name, o.name);
    return *this;
}

Checker& Checker::workspace(const void* at, size_t given, size_t needed) {
    if (needed == 0) return *this;
    require(at != nullptr && given >= needed, "needs %zu bytes of workspace, given %zu", needed,
            at == nullptr ? size_t{0} : given);
    const Span ws{"workspace", at, needed};
    return one(ws, kAlign).one(ws, kWrap);
}

}  // namespace flint
