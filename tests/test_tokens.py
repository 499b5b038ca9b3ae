"""FLINTTOK token files and the batch loader (flint_amd/tokens.py), on the CPU.
The file-format cases mirror the reference's tests/test_fineweb.py:160-233:
header round trip, wider integer inputs, the empty file, nine corruptions that
must be refused, and an atomic write; then the batches the GPT-2 step takes."""

import hashlib

import numpy as np
import pytest

from flint_amd.tokens import DataLoader, TokenFile, TokenFileError, write_token_file


def test_header_round_trip(tmp_path):
    path = tmp_path / "tokens.bin"
    tokens = np.array([50256, 0, 1, 65535, 12345], dtype=np.uint16)
    sha = write_token_file(path, tokens)
    raw = path.read_bytes()
    assert raw[:8] == b"FLINTTOK"
    assert int.from_bytes(raw[8:12], "little") == 1 and int.from_bytes(raw[12:16], "little") == 1
    assert int.from_bytes(raw[16:24], "little") == 5 and raw[24:64] == bytes(40)
    assert raw[64:] == tokens.astype("<u2").tobytes() and len(raw) == 64 + 2 * 5
    assert sha == hashlib.sha256(raw).hexdigest()
    f = TokenFile(path)
    assert f.count == 5 and f.tokens.dtype == np.dtype("<u2") and np.array_equal(f.tokens, tokens)
    assert not list(tmp_path.glob("*.tmp"))


def test_wider_integer_arrays_are_converted_when_they_fit(tmp_path):
    write_token_file(tmp_path / "a.bin", np.array([1, 50256], dtype=np.int64))
    assert TokenFile(tmp_path / "a.bin").tokens.tolist() == [1, 50256]
    with pytest.raises(ValueError):
        write_token_file(tmp_path / "b.bin", np.array([70000], dtype=np.int64))
    assert not (tmp_path / "b.bin").exists() and not list(tmp_path.glob("*.tmp"))


def test_an_empty_token_file_round_trips(tmp_path):
    write_token_file(tmp_path / "empty.bin", np.empty(0, dtype=np.uint16))
    assert (tmp_path / "empty.bin").stat().st_size == 64
    assert TokenFile(tmp_path / "empty.bin").count == 0


def corrupt(mutate):
    def apply(path):
        raw = bytearray(path.read_bytes())
        result = mutate(raw)
        path.write_bytes(bytes(result if result is not None else raw))
    return apply


BAD_FILES = {
    "magic": corrupt(lambda b: b.__setitem__(0, ord("X"))),
    "version": corrupt(lambda b: b.__setitem__(8, 2)),
    "tokenizer id": corrupt(lambda b: b.__setitem__(12, 7)),
    "reserved bytes": corrupt(lambda b: b.__setitem__(40, 1)),
    "count too big": corrupt(lambda b: b.__setitem__(16, 9)),
    "count too small": corrupt(lambda b: b.__setitem__(16, 2)),
    "truncated": corrupt(lambda b: b[:-1]),
    "extra byte": corrupt(lambda b: b + b"\0"),
    "shorter than the header": corrupt(lambda b: b[:30]),
}


@pytest.mark.parametrize("case", sorted(BAD_FILES))
def test_bad_token_files_are_rejected(tmp_path, case):
    path = tmp_path / "tokens.bin"
    write_token_file(path, np.arange(5, dtype=np.uint16))
    BAD_FILES[case](path)
    with pytest.raises(TokenFileError):
        TokenFile(path)


def test_batches_are_rows_of_the_stream_with_targets_shifted_by_one(tmp_path):
    stream = np.arange(1000) % 50257
    write_token_file(tmp_path / "s.bin", stream)
    tokens, targets = TokenFile(tmp_path / "s.bin").batch(offset=17, sequences=4, length=32)
    assert tokens.dtype == np.int32 and tokens.shape == (4, 32) and targets.shape == (4, 32)
    assert np.array_equal(tokens.ravel(), stream[17:17 + 128])
    assert np.array_equal(targets.ravel(), stream[18:18 + 128])
    with pytest.raises(TokenFileError, match="runs past"):
        TokenFile(tmp_path / "s.bin").batch(offset=1000 - 128, sequences=4, length=32)


def test_tokens_outside_the_vocabulary_are_refused_at_batch_time(tmp_path):
    write_token_file(tmp_path / "v.bin", np.array([1, 2, 60000, 3, 4]))
    with pytest.raises(TokenFileError, match="vocabulary"):
        TokenFile(tmp_path / "v.bin").batch(0, 1, 4)


def test_loader_walks_shards_in_order_and_skips_short_tails(tmp_path):
    a = np.arange(0, 300)
    b = np.arange(1000, 1100)            # shorter than one batch of 2 x 64 + 1
    c = np.arange(2000, 2400)
    paths = []
    for name, arr in (("a", a), ("b", b), ("c", c)):
        write_token_file(tmp_path / f"{name}.bin", arr)
        paths.append(tmp_path / f"{name}.bin")
    loader = DataLoader(paths, sequences=2, length=64)
    starts = [int(loader.next_batch()[0][0, 0]) for _ in range(6)]
    # a holds batches at 0 and 128 (the next needs tokens up to 385); b is too
    # short; c holds 2000, 2128, 2256; then back to a.
    assert starts == [0, 128, 2000, 2128, 2256, 0]
