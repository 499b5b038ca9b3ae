"""FLINTTOK token files and the batch loader (flint_amd/tokens.py), on the CPU.

The format is the reference's (ref scripts/fineweb.py:29-37): a 64-byte
little-endian header (magic, version 1, tokenizer id 1, uint64 count, 40 zero
bytes) and then `count` uint16 tokens. The cases below are built from that
field list: every file the reader must refuse is made by changing exactly one
field (or the length) of a good file, and round trips are checked as a
property over random token arrays of every small length."""

import hashlib
import struct

import numpy as np
import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

from flint_amd import tokens as tk

FIELDS = struct.Struct("<8sIIQ")          # the header's leading fields; 40 zero bytes follow


def good_file(tmp_path, values, name="t.bin"):
    path = tmp_path / name
    tk.write_token_file(path, np.asarray(values))
    return path


def parse(raw):
    magic, version, tokenizer, count = FIELDS.unpack_from(raw)
    return {"magic": magic, "version": version, "tokenizer": tokenizer, "count": count,
            "reserved": raw[FIELDS.size:64], "payload": raw[64:]}


@settings(max_examples=60, deadline=None)
@given(st.lists(st.integers(0, 65535), max_size=300))
def test_written_files_parse_back_field_by_field(tmp_path_factory, values):
    path = tmp_path_factory.mktemp("rt") / "x.bin"
    digest = tk.write_token_file(path, np.array(values, dtype=np.int64))
    raw = path.read_bytes()
    got = parse(raw)
    assert (got["magic"], got["version"], got["tokenizer"]) == (b"FLINTTOK", 1, 1)
    assert got["count"] == len(values) and got["reserved"] == b"\0" * 40
    assert got["payload"] == struct.pack(f"<{len(values)}H", *values)
    assert digest == hashlib.sha256(raw).hexdigest()
    f = tk.TokenFile(path)
    assert f.count == len(values) and f.tokens.dtype == np.dtype("<u2")
    assert f.tokens.tolist() == values
    assert [p.name for p in path.parent.iterdir()] == ["x.bin"]   # no temporary left


def test_the_writer_refuses_what_uint16_cannot_hold_and_leaves_nothing(tmp_path):
    for bad in (np.array([65536]), np.array([-1, 3]), np.zeros((2, 2), np.uint16)):
        with pytest.raises(tk.TokenFileError):
            tk.write_token_file(tmp_path / "bad.bin", bad)
    assert list(tmp_path.iterdir()) == []


# Each entry turns the bytes of a good 5-token file into a file the reader must
# refuse, by one change: (what changes, function of the good bytes).
def _field(offset, fmt, value):
    def change(raw):
        out = bytearray(raw)
        struct.pack_into(fmt, out, offset, value)
        return bytes(out)
    return change


REFUSED = [
    ("magic", _field(0, "<8s", b"FLINTTOC")),
    ("version 0", _field(8, "<I", 0)),
    ("version 2", _field(8, "<I", 2)),
    ("tokenizer id", _field(12, "<I", 2)),
    ("count one more than the payload", _field(16, "<Q", 6)),
    ("count one less than the payload", _field(16, "<Q", 4)),
    ("count near 2^64", _field(16, "<Q", (1 << 64) - 1)),
    ("first reserved byte", _field(24, "<B", 1)),
    ("last reserved byte", _field(63, "<B", 0x80)),
    ("payload one byte short", lambda raw: raw[:-1]),
    ("payload one byte long", lambda raw: raw + b"\x07"),
    ("header only, count 5", lambda raw: raw[:64]),
    ("shorter than the header", lambda raw: raw[:63]),
    ("empty file", lambda raw: b""),
]


@pytest.mark.parametrize("what,change", REFUSED, ids=[r[0] for r in REFUSED])
def test_a_file_with_one_field_wrong_is_refused(tmp_path, what, change):
    path = good_file(tmp_path, [3, 1, 4, 1, 5])
    path.write_bytes(change(path.read_bytes()))
    with pytest.raises(tk.TokenFileError):
        tk.TokenFile(path)


def test_every_refusal_case_starts_from_a_file_the_reader_accepts(tmp_path):
    path = good_file(tmp_path, [3, 1, 4, 1, 5])
    assert tk.TokenFile(path).tokens.tolist() == [3, 1, 4, 1, 5]


def test_a_batch_is_the_abis_uint16_rows_with_targets_one_token_later(tmp_path):
    stream = (np.arange(2000) * 7919) % tk.VOCAB
    path = good_file(tmp_path, stream)
    tokens, targets = tk.TokenFile(path).batch(offset=33, sequences=3, length=40)
    for a in (tokens, targets):
        assert a.dtype == np.uint16 and a.shape == (3, 40) and a.flags["C_CONTIGUOUS"]
        # Two bytes per token, as flint_gpt2_forward reads them.
        assert a.nbytes == 3 * 40 * 2
    assert np.array_equal(tokens.reshape(-1), stream[33:153])
    assert np.array_equal(targets.reshape(-1), stream[34:154])
    # The last usable offset and the first one that runs past the end.
    tk.TokenFile(path).batch(offset=2000 - 121, sequences=3, length=40)
    with pytest.raises(tk.TokenFileError, match="runs past"):
        tk.TokenFile(path).batch(offset=2000 - 120, sequences=3, length=40)


def test_tokens_beyond_the_vocabulary_are_refused_when_batched(tmp_path):
    path = good_file(tmp_path, [0, tk.VOCAB - 1, 5, tk.VOCAB, 9])
    tk.TokenFile(path).batch(0, 1, 2)            # reads 0, 50256, 5; 50257 is never read
    with pytest.raises(tk.TokenFileError, match="vocabulary"):
        tk.TokenFile(path).batch(1, 1, 2)


def test_the_loader_visits_shards_in_order_and_passes_over_short_ones(tmp_path):
    sizes = {"s0": 300, "s1": 100, "s2": 400}    # s1 is shorter than 2 x 64 + 1 tokens
    paths = []
    for i, (name, size) in enumerate(sizes.items()):
        paths.append(good_file(tmp_path, 1000 * i + np.arange(size), name + ".bin"))
    loader = tk.DataLoader(paths, sequences=2, length=64)
    first = [int(loader.next_batch()[0][0, 0]) for _ in range(6)]
    # s0 holds batches starting at 0 and 128 (a third needs tokens up to 384);
    # s2 holds three; then the walk starts over at s0.
    assert first == [0, 128, 2000, 2128, 2256, 0]
    with pytest.raises(tk.TokenFileError):
        tk.DataLoader([paths[1]], sequences=2, length=64)
