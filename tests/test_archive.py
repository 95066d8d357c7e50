"""The .cact archive reader (rn_archive_*) on synthetic archives written by
tests/cact_writer.py from docs/format.md — host code, no device needed.

The reference's archive tests (crates/cact/tests/whistle_archive.rs) read the
real model files, which are not in the reference tree; the geometry they assert
(vocab 8199, d_model 512, 8 layers, engram orders [2, 3] at sites [3, 7], a
28-level codebook, 681 records) is written into a synthetic header here and read
back."""
import numpy as np
import pytest

import rustyneedle_amd as rn
from cact_writer import write

HALF, SINGLE, CODEBOOK, RAW = 1, 2, 3, 4


def _whistle_like():
    cb = rn.synthetic_codebook(128)
    half = np.arange(12, dtype=np.float16).tobytes()
    single = np.arange(5, dtype=np.float32).tobytes()
    blob = rn.synthetic_codebook_blob(16, 200, 128, 2, seed=1).tobytes()
    tensors = [(HALF, (3, 4), half, 0, 0), (CODEBOOK, (16, 200), blob, 128, 2), (SINGLE, (5,), single, 0, 0)]
    tensors += [(RAW, (7,), bytes(range(7)), 0, 0)] * 678  # 681 records in all
    return write(tensors, cb, rope_theta=500000.0, vocab=8199, d_model=512, num_layers=8, num_heads=8,
                 num_kv_heads=2, global_mask_lo=0b101, global_mask_hi=1, engram_orders=(2, 3),
                 engram_sites=(3, 7)), cb, blob


def test_geometry_records_and_bytes():
    data, cb, blob = _whistle_like()
    a = rn.Archive(data=data)
    g = a.geometry()
    assert (g["vocab"], g["d_model"], g["num_layers"], g["codebook_len"], g["tensor_count"]) == (8199, 512, 8, 28, 681)
    assert g["engram_orders"] == [2, 3] and g["engram_sites"] == [3, 7]
    assert g["global_layers"] == (1 << 32) | 0b101 and g["num_kv_heads"] == 2
    assert g["rope_theta"] == np.float32(500000.0)
    assert np.array_equal(a.codebook(), cb)
    r = a.record(1)
    assert (r["kind"], r["shape"], r["group_size"], r["bits"], r["nbytes"]) == (CODEBOOK, [16, 200], 128, 2, len(blob))
    assert r["offset"] % 64 == 0
    assert a.tensor_bytes(1).tobytes() == blob
    assert np.array_equal(a.tensor_bytes(0).view(np.float16), np.arange(12, dtype=np.float16))
    assert a.record(2)["shape"] == [5]
    with pytest.raises(rn.RnError):
        a.record(681)


def test_open_from_a_file(tmp_path):
    data, _, blob = _whistle_like()
    path = tmp_path / "model.cact"
    path.write_bytes(data)
    a = rn.Archive(str(path))
    assert a.tensor_bytes(1).tobytes() == blob
    with pytest.raises(rn.RnError, match="No such file"):
        rn.Archive(str(tmp_path / "missing.cact"))


def _error(data: bytes) -> str:
    with pytest.raises(rn.RnError) as e:
        rn.Archive(data=data)
    return str(e.value)


def test_format_errors_carry_the_reference_messages():
    cb = rn.synthetic_codebook(128)
    good = write([(HALF, (4,), np.zeros(4, np.float16).tobytes(), 0, 0)], cb)
    assert "format tag 0x12345678" in _error(b"\x78\x56\x34\x12" + good[4:])
    assert "truncated inside the header" in _error(good[:100])
    assert "truncated inside the codebook" in _error(good[:196 + 40])
    assert "truncated inside the tensor directory" in _error(good[:196 + 112 + 20])
    bad_kind = bytearray(good)
    bad_kind[196 + 112] = 9
    assert "unknown tensor element kind 9" in _error(bytes(bad_kind))
    outside = write([(HALF, (4,), np.zeros(4, np.float16).tobytes(), 0, 0)], cb)
    assert "lies outside the archive" in _error(outside[:-64] if len(outside) > 320 else outside[:300])
    odd = bytearray(good)
    off = 196 + 112 + 20  # the record's offset field
    odd[off:off + 8] = (int.from_bytes(odd[off:off + 8], "little") + 1).to_bytes(8, "little")
    assert "not aligned to its element width" in _error(bytes(odd))
    many = bytearray(good)
    many[196 - 4 - 64 - 4 - 20:196 - 4 - 64 - 4 - 16] = (5).to_bytes(4, "little")  # engram order count
    assert "order or site count" in _error(bytes(many))


def test_matrix_from_a_non_codebook_record_is_refused():
    data, _, _ = _whistle_like()
    a = rn.Archive(data=data)
    with pytest.raises(rn.RnError, match="not codebook-quantised"):
        a.matrix(0)
