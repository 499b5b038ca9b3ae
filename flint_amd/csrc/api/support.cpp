// C-ABI entry points of the data-movement functions: copy, FP32 -> FP16,
// heads split / merge and the embedding's passes. Checks and message text
// follow the reference's src/api/copy.cpp:6-28, convert.cpp:6-29,
// heads.cpp:10-78 and embedding.cpp:11-134.
#include <cstdint>
#include <iterator>

#include "common/common.h"
#include "kernels/kernels.h"

using flint::fail;

namespace {

flint_status move_heads(bool split, void* y, const void* x, size_t batches, size_t length,
                        size_t heads, size_t head_width, size_t row_width, size_t first,
                        flint_stream stream) {
    const char* name = split ? "flint_heads_split" : "flint_heads_merge";
    if (row_width == 0 || row_width % 8 != 0 || row_width > flint::kHeadsMaxRowWidth) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT,
                    "%s: row_width (%zu) must be a multiple of 8 from 8 to %zu", name, row_width,
                    flint::kHeadsMaxRowWidth);
    }
    if (head_width == 0 || head_width % 8 != 0) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT,
                    "%s: head_width (%zu) must be a positive multiple of 8", name, head_width);
    }
    if (first % 8 != 0) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: first (%zu) must be a multiple of 8", name,
                    first);
    }
    if (heads == 0) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: heads must be positive", name);
    }
    if (heads > row_width / head_width || first > row_width - heads * head_width) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT,
                    "%s: %zu heads of %zu columns from column %zu run past row_width (%zu)", name,
                    heads, head_width, first, row_width);
    }
    if (length != 0 && batches > flint::kHeadsMaxRows / length) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT,
                    "%s: batches (%zu) x length (%zu) can be up to %zu rows", name, batches,
                    length, flint::kHeadsMaxRows);
    }
    if (batches == 0 || length == 0) return FLINT_OK;
    const size_t rows = batches * length;
    const size_t rows_bytes = rows * row_width * 2;
    const size_t heads_bytes = rows * heads * head_width * 2;
    const flint::Buffer buffers[] = {
        {"y", y, split ? heads_bytes : rows_bytes},
        {"x", x, split ? rows_bytes : heads_bytes},
    };
    if (flint_status s = flint::check_buffers(name, buffers, std::size(buffers), 1); s != FLINT_OK) {
        return s;
    }
    FLINT_HIP_CHECK(flint::launch_heads(y, x, batches, length, heads, head_width, row_width, first,
                                        !split, flint::to_hip(stream)));
    return FLINT_OK;
}

flint_status check_embedding_backward_dims(const char* name, size_t sequences, size_t length,
                                           size_t vocab, size_t width) {
    if (width == 0 || width % 8 != 0 || width > flint::kEmbeddingBackwardMaxWidth) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT,
                    "%s: width (%zu) must be a multiple of 8 from 8 to %zu", name, width,
                    flint::kEmbeddingBackwardMaxWidth);
    }
    if (vocab == 0 || vocab > flint::kEmbeddingMaxVocab) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: vocab (%zu) must be from 1 to %zu", name,
                    vocab, flint::kEmbeddingMaxVocab);
    }
    if (length == 0 || length > flint::kEmbeddingBackwardMaxPositionValues / width) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT,
                    "%s: length (%zu) must be from 1 to %zu, so that length x width (%zu) is at "
                    "most %zu",
                    name, length, flint::kEmbeddingBackwardMaxPositionValues / width, width,
                    flint::kEmbeddingBackwardMaxPositionValues);
    }
    if (sequences == 0 || sequences > flint::kEmbeddingBackwardMaxRows / length) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT,
                    "%s: sequences (%zu) must be from 1 to %zu, so that sequences x length is at "
                    "most %zu rows",
                    name, sequences, flint::kEmbeddingBackwardMaxRows / length,
                    flint::kEmbeddingBackwardMaxRows);
    }
    return FLINT_OK;
}

}  // namespace

extern "C" {

FLINT_API flint_status flint_copy(void* dst, const void* src, size_t bytes, flint_stream stream) {
    if (bytes == 0) return FLINT_OK;
    if (dst == nullptr) return fail(FLINT_ERROR_INVALID_ARGUMENT, "flint_copy: dst is null");
    if (src == nullptr) return fail(FLINT_ERROR_INVALID_ARGUMENT, "flint_copy: src is null");
    const uintptr_t d = reinterpret_cast<uintptr_t>(dst);
    const uintptr_t s = reinterpret_cast<uintptr_t>(src);
    if (bytes > UINTPTR_MAX - d || bytes > UINTPTR_MAX - s) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT,
                    "flint_copy: %zu bytes run past the end of the address space", bytes);
    }
    if (d < s + bytes && s < d + bytes) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "flint_copy: dst and src overlap");
    }
    FLINT_HIP_CHECK(flint::launch_copy(dst, src, bytes, flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_fp32_to_fp16(void* y, const void* x, size_t count,
                                          flint_stream stream) {
    constexpr const char* name = "flint_fp32_to_fp16";
    constexpr size_t kMax = SIZE_MAX / 4;
    if (count > kMax) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: count (%zu) can be up to %zu", name, count,
                    kMax);
    }
    if (count == 0) return FLINT_OK;
    const flint::Buffer buffers[] = {{"y", y, count * 2}, {"x", x, count * 4}};
    if (flint_status s = flint::check_buffers(name, buffers, std::size(buffers), 1); s != FLINT_OK) {
        return s;
    }
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
    constexpr const char* name = "flint_embedding_forward";
    if (width == 0 || width % 8 != 0 || width > flint::kEmbeddingMaxWidth) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT,
                    "%s: width (%zu) must be a multiple of 8 from 8 to %zu", name, width,
                    flint::kEmbeddingMaxWidth);
    }
    if (vocab == 0 || vocab > flint::kEmbeddingMaxVocab) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: vocab (%zu) must be from 1 to %zu", name,
                    vocab, flint::kEmbeddingMaxVocab);
    }
    if (length != 0 && sequences > flint::kEmbeddingMaxRows / length) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT,
                    "%s: sequences (%zu) x length (%zu) can be up to %zu rows", name, sequences,
                    length, flint::kEmbeddingMaxRows);
    }
    if (sequences == 0 || length == 0) return FLINT_OK;
    const size_t rows = sequences * length;
    const flint::Buffer buffers[] = {
        {"x", x, rows * width * 4},
        {"tokens", tokens, rows * 2},
        {"wte", wte, vocab * width * 4},
        {"wpe", wpe, length * width * 4},
    };
    if (flint_status s = flint::check_buffers(name, buffers, std::size(buffers), 1); s != FLINT_OK) {
        return s;
    }
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
    constexpr const char* name = "flint_embedding_backward";
    if (flint_status s = check_embedding_backward_dims(name, sequences, length, vocab, width);
        s != FLINT_OK) {
        return s;
    }
    const size_t needed = flint::embedding_backward_workspace(sequences, length, vocab, width);
    if (workspace_bytes < needed) {
        return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: needs %zu bytes of workspace, given %zu",
                    name, needed, workspace_bytes);
    }
    const size_t rows = sequences * length;
    const flint::Buffer buffers[] = {
        {"dwte", dwte, vocab * width * 4},
        {"dwpe", dwpe, length * width * 4},
        {"workspace", workspace, needed},
        {"dx", dx, rows * width * 4},
        {"tokens", tokens, rows * 2},
    };
    if (flint_status s = flint::check_buffers(name, buffers, std::size(buffers), 3); s != FLINT_OK) {
        return s;
    }
    FLINT_HIP_CHECK(flint::launch_embedding_backward(dwte, dwpe, dx, tokens, sequences, length,
                                                     vocab, width, accumulate_wte != 0,
                                                     accumulate_wpe != 0, workspace,
                                                     flint::to_hip(stream)));
    return FLINT_OK;
}

FLINT_API flint_status flint_embedding_backward_workspace(size_t sequences, size_t length,
                                                          size_t vocab, size_t width,
                                                          size_t* bytes) {
    constexpr const char* name = "flint_embedding_backward_workspace";
    if (bytes == nullptr) return fail(FLINT_ERROR_INVALID_ARGUMENT, "%s: bytes is null", name);
    if (flint_status s = check_embedding_backward_dims(name, sequences, length, vocab, width);
        s != FLINT_OK) {
        return s;
    }
    *bytes = flint::embedding_backward_workspace(sequences, length, vocab, width);
    return FLINT_OK;
}

}  // extern "C"
