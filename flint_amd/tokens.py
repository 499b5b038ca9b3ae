"""FLINTTOK token files: the on-disk input of the training step.

Format (ref scripts/fineweb.py:29-37; everything little-endian): a 64-byte
header, then `count` uint16 tokens with no padding, so the file is exactly
64 + 2 * count bytes.

    bytes  0-7   magic b"FLINTTOK"
    bytes  8-11  uint32 version = 1
    bytes 12-15  uint32 tokenizer id = 1 (tiktoken "gpt2": 50,257 tokens,
                 <|endoftext|> = 50256)
    bytes 16-23  uint64 token count
    bytes 24-63  zero

`write_token_file` writes one; `TokenFile` memory-maps one after checking every
header field and the size rule; `TokenFile.batch` cuts `sequences` rows of
`length` tokens starting at a token offset into the uint16 `tokens` and
`targets` (the next token) that flint_gpt2_forward takes (the ABI's token type,
ref include/flint/flint.h:511-523), the layout of the reference's training loop
(B x T tokens, targets shifted by one).
`DataLoader` walks a list of shards in order, batch after batch, moving to the
next shard when fewer than B*T+1 tokens remain in the current one.
"""

import hashlib
import os
import struct
from pathlib import Path

import numpy as np

MAGIC = b"FLINTTOK"
VERSION = 1
TOKENIZER_GPT2 = 1
VOCAB = 50257
HEADER_BYTES = 64
_HEADER = struct.Struct("<8sIIQ40x")


class TokenFileError(ValueError):
    pass


def header_bytes(count, version=VERSION, tokenizer=TOKENIZER_GPT2):
    return _HEADER.pack(MAGIC, version, tokenizer, count)


def write_token_file(path, tokens):
    """Writes integer tokens (values below 65,536) as a token file, atomically
    (a temporary file renamed into place, removed on failure), and returns the
    sha256 of the whole file."""
    arr = np.asarray(tokens)
    if arr.ndim != 1:
        raise TokenFileError("tokens must be one-dimensional")
    if arr.size and (arr.min() < 0 or arr.max() >= 1 << 16):
        raise TokenFileError("a token does not fit in uint16")
    data = np.ascontiguousarray(arr, dtype="<u2").tobytes()
    header = header_bytes(arr.size)
    path = Path(path)
    tmp = path.with_name(path.name + ".tmp")
    try:
        with open(tmp, "wb") as f:
            f.write(header)
            f.write(data)
        os.replace(tmp, path)
    except BaseException:
        tmp.unlink(missing_ok=True)
        raise
    return hashlib.sha256(header + data).hexdigest()


class TokenFile:
    """A checked, memory-mapped FLINTTOK file."""

    def __init__(self, path):
        self.path = Path(path)
        size = self.path.stat().st_size
        if size < HEADER_BYTES:
            raise TokenFileError(f"{self.path}: {size} bytes, shorter than the 64-byte header")
        with open(self.path, "rb") as f:
            raw = f.read(HEADER_BYTES)
        magic, version, tokenizer, count = _HEADER.unpack(raw)
        if magic != MAGIC:
            raise TokenFileError(f"{self.path}: bad magic {magic!r}")
        if version != VERSION:
            raise TokenFileError(f"{self.path}: version {version}, expected {VERSION}")
        if tokenizer != TOKENIZER_GPT2:
            raise TokenFileError(f"{self.path}: tokenizer id {tokenizer}, expected {TOKENIZER_GPT2}")
        if any(raw[24:]):
            raise TokenFileError(f"{self.path}: header bytes 24-63 are not zero")
        if size != HEADER_BYTES + 2 * count:
            raise TokenFileError(f"{self.path}: {size} bytes, but the header's count {count} needs "
                                 f"{HEADER_BYTES + 2 * count}")
        self.count = count
        self.tokens = (np.memmap(self.path, dtype="<u2", mode="r", offset=HEADER_BYTES, shape=(count,))
                       if count else np.zeros(0, "<u2"))

    def batch(self, offset, sequences, length):
        """uint16 (tokens, targets), each sequences x length and C-contiguous,
        from tokens [offset, offset + sequences * length + 1): the arrays can be
        copied to the device as they are and handed to flint_gpt2_forward."""
        need = sequences * length + 1
        if offset < 0 or offset + need > self.count:
            raise TokenFileError(f"{self.path}: a batch of {need} tokens at {offset} runs past {self.count}")
        chunk = np.asarray(self.tokens[offset:offset + need], dtype=np.uint16)
        if chunk.size and chunk.max() >= VOCAB:
            raise TokenFileError(f"{self.path}: token {int(chunk.max())} is outside the GPT-2 vocabulary")
        return (np.ascontiguousarray(chunk[:-1].reshape(sequences, length)),
                np.ascontiguousarray(chunk[1:].reshape(sequences, length)))


class DataLoader:
    """Consecutive batches over shards in order; each batch advances by
    sequences * length tokens (the last target overlaps the next batch's
    first token), and a shard too short for the next batch is left for the
    next one."""

    def __init__(self, paths, sequences, length):
        self.files = [TokenFile(p) for p in paths]
        if not self.files:
            raise TokenFileError("no token files")
        self.sequences, self.length = sequences, length
        if all(f.count < sequences * length + 1 for f in self.files):
            raise TokenFileError("no shard holds one batch")
        self.shard, self.offset = 0, 0

    def next_batch(self):
        need = self.sequences * self.length + 1
        while self.offset + need > self.files[self.shard].count:
            self.shard = (self.shard + 1) % len(self.files)
            self.offset = 0
        out = self.files[self.shard].batch(self.offset, self.sequences, self.length)
        self.offset += self.sequences * self.length
        return out
