"""The checkpoint record format (xfold/params.py:40-91) and the loader: a known-answer byte
string, round trips over the dtypes and layouts the reference's own tests use
(tests/test_params_runtime.py:17-31 of the reference: a transposed float32 matrix, a float16
scalar, uint8), cut-short records, checkpoints split over files with a record crossing the
split, and the zstd case without the optional module."""

import io
import struct

import numpy as np
import pytest
import torch

from xfold_cpu_amd.params import ConcatenatedFiles, RecordError, encode_record, load_params, read_records


def test_known_answer_record():
    """scope 'ab', name 'w', float32 [2] = (1, -2), spelled out byte by byte."""
    want = bytes.fromhex(
        "02000000" "01000000" "07000000" "01000000" "08000000"      # '<5i' lengths, ndim, data bytes
        "6162" "77" "666c6f61743332"                                 # 'ab', 'w', 'float32'
        "02000000"                                                   # shape (2,)
        "0000803f" "000000c0")                                       # 1.0, -2.0
    assert encode_record("ab", "w", np.array([1.0, -2.0], dtype=np.float32)) == want
    [(scope, name, t)] = list(read_records(io.BytesIO(want)))
    assert (scope, name) == ("ab", "w")
    assert t.dtype == torch.float32 and t.tolist() == [1.0, -2.0]


def test_round_trip_dtypes_shapes_and_several_records():
    arrays = (np.arange(15, dtype=np.float32).reshape(3, 5).T, np.array(3, dtype=np.float16),
              np.arange(16, dtype=np.uint8))
    payload = b"".join(encode_record("scope", str(i), a) for i, a in enumerate(arrays))
    payload += encode_record("scope", "bf", torch.tensor([[1.5, -0.25]], dtype=torch.bfloat16))
    payload += encode_record("scope", "empty", torch.zeros(0, 4))
    got = list(read_records(io.BytesIO(payload)))
    assert [(s, n) for s, n, _ in got] == [("scope", "0"), ("scope", "1"), ("scope", "2"), ("scope", "bf"),
                                           ("scope", "empty")]
    assert got[4][2].shape == (0, 4)
    for (_, _, t), a in zip(got, arrays):
        torch.testing.assert_close(t, torch.from_numpy(a.copy()), rtol=0, atol=0)
    assert got[3][2].dtype == torch.bfloat16 and got[3][2].tolist() == [[1.5, -0.25]]


def test_cut_short_records_fail_clearly():
    record = encode_record("scope", "weight", np.ones((3, 5), dtype=np.float32))
    for cut in (record[:7], record[:-1], record[:30]):
        with pytest.raises(RecordError):
            list(read_records(io.BytesIO(cut)))
    assert list(read_records(io.BytesIO(b""))) == []


def test_inconsistent_header_is_rejected():
    record = bytearray(encode_record("s", "w", np.ones(4, dtype=np.float32)))
    struct.pack_into("<i", record, 16, 12)                # data length 12 for 4 floats
    with pytest.raises(RecordError):
        list(read_records(io.BytesIO(bytes(record[:-4]))))


def test_checkpoint_split_over_files(tmp_path):
    records = [encode_record("scope", "w", np.arange(30, dtype=np.float32)),
               encode_record("other", "b", np.arange(6, dtype=np.uint8).reshape(2, 3))]
    blob = b"".join(records)
    cuts = [0, 5, 50, len(records[0]) + 3, len(blob)]          # a header and payloads cross parts
    paths = []
    for i in range(len(cuts) - 1):
        p = tmp_path / f"part{i}.bin"
        p.write_bytes(blob[cuts[i]:cuts[i + 1]])
        paths.append(p)
    with ConcatenatedFiles(paths) as raw:
        assert raw.read() == blob
    params = load_params(paths)
    assert sorted(params) == ["other/b", "scope/w"]
    torch.testing.assert_close(params["scope/w"], torch.arange(30, dtype=torch.float32), rtol=0, atol=0)
    assert params["other/b"].tolist() == [[0, 1, 2], [3, 4, 5]]


def test_compressed_checkpoint_without_zstandard(tmp_path):
    try:
        import zstandard  # noqa: F401
        pytest.skip("zstandard is installed here")
    except ImportError:
        pass
    p = tmp_path / "af3.bin.zst"
    p.write_bytes(b"\x28\xb5\x2f\xfd" + b"\x00" * 16)
    with pytest.raises(RecordError, match="zstd"):
        load_params(p)
