// C-ABI entry points of the data-movement functions: copy, FP32 -> FP16,
// heads split / merge and the embedding's passes. Each is a Checker chain and
// one launcher call; limits, check order and message texts are the
// reference's interface (ref src/api/copy.cpp:6-28, convert.cpp:6-29,
// heads.cpp:10-78, embedding.cpp:11-134).
#include <cstdint>

#include "common/args.h"
#include "kernels/kernels.h"

namespace {

using flint::Checker;
using flint::Span;

flint_status move_heads(bool split, void* y, const void* x, size_t batches, size_t length,
                        size_t heads, size_t head_width, size_t row_width, size_t first,
                        flint_stream stream) {
    Checker c(split ? "flint_heads_split" : "flint_heads_merge");
    c.require(row_width != 0 && row_width % 8 == 0 && row_width <= flint::kHeadsMaxRowWidth,
              "row_width (%zu) must be a multiple of 8 from 8 to %zu", row_width,
              flint::kHeadsMaxRowWidth)
        .require(head_width != 0 && head_width % 8 == 0,
                 "head_width (%zu) must be a positive multiple of 8", head_width)
        .require(first % 8 == 0, "first (%zu) must be a multiple of 8", first)
        .require(heads != 0, "heads must be positive");
    // Evaluated only once head_width is known to be nonzero.
    if (c.ok())
        c.require(heads <= row_width / head_width && first <= row_width - heads * head_width,
                  "%zu heads of %zu columns from column %zu run past row_width (%zu)", heads,
                  head_width, first, row_width);
    c.require(length == 0 || batches <= flint::kHeadsMaxRows / length,
              "batches (%zu) x length (%zu) can be up to %zu rows", batches, length,
              flint::kHeadsMaxRows);
    if (!c.ok() || batches == 0 || length == 0) return c.status();
    const size_t rows = batches * length;
    const size_t wide = rows * row_width * 2;            // the [rows][row_width] side
    const size_t narrow = rows * heads * head_width * 2;  // the per-head side
    if (!c.buffers({{"y", y, split ? narrow : wide}, {"x", x, split ? wide : narrow}}, 1).ok())
        return c.status();
    FLINT_HIP_CHECK(flint::launch_heads(y, x, batches, length, heads, head_width, row_width, first,
                                        !split, flint::to_hip(stream)));
    return FLINT_OK;
}

// The embedding backward's limits: its scatter sums run in the bias
// gradient's column chunks, and the positions' sums over sequences too.
Checker& embedding_backward_sizes(Checker& c, size_t sequences, size_t length, size_t vocab,
                                  size_t width) {
    c.require(width != 0 && width % 8 == 0 && width <= flint::kEmbeddingBackwardMaxWidth,
              "width (%zu) must be a multiple of 8 from 8 to %zu", width,
              flint::kEmbeddingBackwardMaxWidth)
        .require(vocab != 0 && vocab <= flint::kEmbeddingMaxVocab, "vocab (%zu) must be from 1 to %zu",
                 vocab, flint::kEmbeddingMaxVocab);
    if (!c.ok()) return c;
    const size_t max_length = flint::kEmbeddingBackwardMaxPositionValues / width;
    c.require(length != 0 && length <= max_length,
              "length (%zu) must be from 1 to %zu, so that length x width (%zu) is at most %zu",
              length, max_length, width, flint::kEmbeddingBackwardMaxPositionValues);
    if (!c.ok()) return c;
    const size_t max_sequences = flint::kEmbeddingBackwardMaxRows / length;
    return c.require(sequences != 0 && sequences <= max_sequences,
                     "sequences (%zu) must be from 1 to %zu, so that sequences x length is at "
                     "most %zu rows",
                     sequences, max_sequences, flint::kEmbeddingBackwardMaxRows);
}

}  // namespace

extern "C" {

FLINT_API flint_status flint_copy(void* dst, const void* src, size_t bytes, flint_stream stream) {
    if (bytes == 0) return FLINT_OK;
    Checker c("flint_copy");
    const Span d{"dst", dst, bytes}, s{"src", src, bytes};
    // Byte copies take any alignment; the wrap message names the size.
    c.require(!d.null(), "dst is null")
        .require(!s.null(), "src is null")
        .require(d.in_space() && s.in_space(), "%zu bytes run past the end of the address space",
                 bytes)
        .apart(d, {s});
    if (!c.ok()) return c.status();
    FLINT_HIP_CHECK(flint::launch_copy(dst, src, bytes, flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_fp32_to_fp16(void* y, const void* x, size_t count,
                                          flint_stream stream) {
    constexpr size_t kMax = SIZE_MAX / 4;
    Checker c("flint_fp32_to_fp16");
    if (!c.require(count <= kMax, "count (%zu) can be up to %zu", count, kMax).ok() || count == 0)
        return c.status();
    if (!c.buffers({{"y", y, count * 2}, {"x", x, count * 4}}, 1).ok()) return c.status();
    FLINT_HIP_CHECK(flint::launch_fp32_to_fp16(y, x, count, flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_heads_split(void* y, const void* x, size_t batches, size_t length,
                                         size_t heads, size_t head_width, size_t row_width,
                                         size_t first, flint_stream stream) {
    return move_heads(true, y, x, batches, length, heads, head_width, row_width, first, stream);
}

FLINT_API flint_status flint_heads_merge(void* y, const void* x, size_t batches, size_t length,
                                         size_t heads, size_t head_width, size_t row_width,
                                         size_t first, flint_stream stream) {
    return move_heads(false, y, x, batches, length, heads, head_width, row_width, first, stream);
}

FLINT_API flint_status flint_embedding_forward(void* x, const void* tokens, const void* wte,
                                               const void* wpe, size_t sequences, size_t length,
                                               size_t vocab, size_t width, flint_stream stream) {
    Checker c("flint_embedding_forward");
    c.require(width != 0 && width % 8 == 0 && width <= flint::kEmbeddingMaxWidth,
              "width (%zu) must be a multiple of 8 from 8 to %zu", width, flint::kEmbeddingMaxWidth)
        .require(vocab != 0 && vocab <= flint::kEmbeddingMaxVocab, "vocab (%zu) must be from 1 to %zu",
                 vocab, flint::kEmbeddingMaxVocab)
        .require(length == 0 || sequences <= flint::kEmbeddingMaxRows / length,
                 "sequences (%zu) x length (%zu) can be up to %zu rows", sequences, length,
                 flint::kEmbeddingMaxRows);
    if (!c.ok() || sequences == 0 || length == 0) return c.status();
    const size_t rows = sequences * length;
    c.buffers({{"x", x, rows * width * 4},
               {"tokens", tokens, rows * 2},
               {"wte", wte, vocab * width * 4},
               {"wpe", wpe, length * width * 4}},
              1);
    if (!c.ok()) return c.status();
    FLINT_HIP_CHECK(flint::launch_embedding_forward(x, tokens, wte, wpe, rows, length, width,
                                                    flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_embedding_backward(void* dwte, void* dwpe, const void* dx,
                                                const void* tokens, size_t sequences,
                                                size_t length, size_t vocab, size_t width,
                                                int accumulate_wte, int accumulate_wpe,
                                                void* workspace, size_t workspace_bytes,
                                                flint_stream stream) {
    Checker c("flint_embedding_backward");
    if (!embedding_backward_sizes(c, sequences, length, vocab, width).ok()) return c.status();
    const size_t needed = flint::embedding_backward_workspace(sequences, length, vocab, width);
    const size_t rows = sequences * length;
    c.require(workspace_bytes >= needed, "needs %zu bytes of workspace, given %zu", needed,
              workspace_bytes)
        .buffers({{"dwte", dwte, vocab * width * 4},
                  {"dwpe", dwpe, length * width * 4},
                  {"workspace", workspace, needed},
                  {"dx", dx, rows * width * 4},
                  {"tokens", tokens, rows * 2}},
                 3);
    if (!c.ok()) return c.status();
    FLINT_HIP_CHECK(flint::launch_embedding_backward(dwte, dwpe, dx, tokens, sequences, length,
                                                     vocab, width, accumulate_wte != 0,
                                                     accumulate_wpe != 0, workspace,
                                                     flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_embedding_backward_workspace(size_t sequences, size_t length,
                                                          size_t vocab, size_t width,
                                                          size_t* bytes) {
    Checker c("flint_embedding_backward_workspace");
    c.require(bytes != nullptr, "bytes is null");
    if (!embedding_backward_sizes(c, sequences, length, vocab, width).ok()) return c.status();
    *bytes = flint::embedding_backward_workspace(sequences, length, vocab, width);
    return FLINT_OK;
}

}  // extern "C"
