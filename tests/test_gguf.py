"""GGUF index reading (charlotte_hip_matmul_gguf_*), on the host.

Follows the reference's own tests of its reader, over its own fixture files
(tests/fixtures/gguf/*.gguf, copied to tests/golden/gguf/ as data):
  tests/gguf_malformed_test.cpp:34-70 — each malformed file fails with its
    own named error; every truncation of a valid file fails cleanly;
  tests/gguf_parse_test.cpp:30-155 — the valid file's tensors, lookup by
    name, absolute aligned offsets inside the file, a declared alignment, a
    64-byte name.
Beyond them: the reference's matmul fixture read alike by the library and by
an independent Python reader (tests/support/gguf_fixture.py), byte for byte.
"""

import os

import numpy as np
import pytest

from tests.support.oracle_lib import Q4_0, Q6_K

HERE = os.path.dirname(os.path.abspath(__file__))
GGUF = os.path.join(HERE, "golden", "gguf")


def _path(name):
    return os.path.join(GGUF, name + ".gguf")


def _error(name):
    from charlotte_amd import matmul as mm

    with pytest.raises(mm.GgufError) as e:
        mm.GgufFile(_path(name))
    assert e.value.status == mm.Status.BAD_FILE
    return e.value.read_error


MALFORMED = {
    "bad_magic": "BadMagic",
    "bad_version": "UnsupportedVersion",
    "truncated_header": "ShortRead",
    "tensor_count_too_large": "CountTooLarge",
    # Claims five keys; what follows is zero padding, read as an empty key.
    "metadata_count_lies": "EmptyKey",
    "negative_dimension": "NegativeDimension",
    "unknown_tensor_type": "UnknownTensorType",
    "not_block_aligned": "RowNotWholeBlocks",
    "duplicate_tensor_name": "DuplicateTensorName",
    "duplicate_tensor_name_apart": "DuplicateTensorName",
    "nested_array": "NestedArray",
    "unknown_value_type": "UnknownValueType",
    "offset_past_eof": "TensorDataOutOfBounds",
    "data_truncated": "TensorDataOutOfBounds",
    "offset_overflow": "OffsetOverflow",
    "alignment_wrong_type": "BadAlignment",
    "alignment_not_power_of_two": "BadAlignment",
    "misaligned_tensor_offset": "MisalignedTensorData",
    "overlapping_tensor_data": "OverlappingTensorData",
    "empty_metadata_key": "EmptyKey",
    "duplicate_metadata_key": "DuplicateMetadataKey",
    "tensor_name_65_bytes": "TensorNameTooLong",
}


@pytest.mark.parametrize("name", sorted(MALFORMED))
def test_malformed_files_fail_with_their_own_named_error(name):
    assert _error(name).name == MALFORMED[name]


def test_an_empty_file_fails_rather_than_reading_anything():
    from charlotte_amd import matmul as mm

    with pytest.raises(mm.GgufError) as e:
        mm.GgufFile(data=b"")
    assert e.value.read_error == mm.ReadError.ShortRead


def test_every_truncation_of_a_valid_file_fails():
    from charlotte_amd import matmul as mm

    whole = open(_path("valid"), "rb").read()
    mm.GgufFile(data=whole).close()
    accepted = 0
    for cut in range(len(whole)):
        try:
            mm.GgufFile(data=whole[:cut]).close()
            accepted += 1
        except mm.GgufError as e:
            assert e.read_error != mm.ReadError.Ok
    # A cut inside the last tensor's padding still holds every tensor's bytes;
    # one that loses any of them is refused.
    last = max(t.offset + t.bytes for t in mm.GgufFile(data=whole).tensors)
    assert accepted == len(whole) - last


def test_a_missing_file_is_an_io_error():
    from charlotte_amd import matmul as mm

    with pytest.raises(mm.GgufError) as e:
        mm.GgufFile(os.path.join(GGUF, "does_not_exist.gguf"))
    assert e.value.status == mm.Status.IO_ERROR


def test_the_valid_file_yields_its_tensors():
    from charlotte_amd import matmul as mm

    f = mm.GgufFile(_path("valid"))
    assert [t.name for t in f.tensors] == ["token_embd.weight", "output_norm.weight"]
    embd, norm = f.tensors
    assert embd.gguf_type == Q4_0 and embd.dimensions == (64, 2) and embd.element_count == 128
    assert embd.bytes == 72  # 4 blocks of 18 bytes
    assert norm.gguf_type == 0 and norm.element_count == 4 and norm.bytes == 16
    assert f.find("output_norm.weight") == 1 and f.find("does.not.exist") == -1
    size = os.path.getsize(_path("valid"))
    for t in f.tensors:
        assert t.offset % 32 == 0 and t.offset + t.bytes <= size
    f.close()


def test_a_declared_alignment_is_honoured_and_a_64_byte_name_accepted():
    from charlotte_amd import matmul as mm

    f = mm.GgufFile(_path("alignment_64"))
    assert len(f.tensors) == 2 and all(t.offset % 64 == 0 for t in f.tensors)
    assert f.tensors[1].offset - f.tensors[0].offset == 64
    g = mm.GgufFile(_path("tensor_name_64_bytes"))
    assert len(g.tensors) == 1 and len(g.tensors[0].name) == 64


def test_the_matmul_fixture_reads_as_an_independent_reader_reads_it(fixture_tensors):
    from charlotte_amd import matmul as mm

    f = mm.GgufFile(os.path.join(HERE, "golden", "matmul_rows.gguf"))
    assert [t.name for t in f.tensors] == list(fixture_tensors)
    for t in f.tensors:
        want = fixture_tensors[t.name]
        assert t.gguf_type == want.type and t.dimensions == tuple(want.dims)
        assert f.data(t) == want.data


@pytest.mark.parametrize("name,gtype", [("embedding_q4_0", Q4_0), ("embedding_q6_k", Q6_K), ("q6_k_tensor", Q6_K)])
def test_quantized_fixtures_lay_out_as_the_oracle_does(oracle, name, gtype):
    """A tensor read from a file lays out (host side) to the oracle's bytes."""
    from charlotte_amd import matmul as mm

    f = mm.GgufFile(_path(name))
    t = next(t for t in f.tensors if t.gguf_type == gtype)
    stored = f.data(t)
    blocks = t.element_count // (32 if gtype == Q4_0 else 256)
    got = np.frombuffer(mm.lay_out(gtype, stored, blocks), np.uint8)
    assert (got == oracle.lay_out(gtype, stored)).all()
