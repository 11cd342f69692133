"""CPU checks of the safetensors shard index (Shards::open / find / read_raw, safetensors.rs:215-488):
offsets, shapes and bytes across several shards, file-name order, and the reference's header
checks (safetensors.rs:769-800 and the header-length guard at :270-276)."""
import json

import numpy as np
import pytest

from helpers import write_safetensors


def _shards(d):
    import rabbit_amd as R
    return R.Shards(str(d))


def test_index_across_shards_and_exact_bytes(tmp_path, rbt_lib):
    rng = np.random.default_rng(0)
    a = rng.integers(0, 256, 1000, dtype=np.uint8)
    b = rng.standard_normal((3, 5)).astype(np.float32)
    c = rng.integers(0, 256, 77, dtype=np.uint8)
    # file-name order: model-00001 before model-00002 (written in the other order on purpose)
    write_safetensors(tmp_path / "model-00002-of-00002.safetensors", [("c.weight", "U8", [7, 11], c.tobytes())])
    write_safetensors(tmp_path / "model-00001-of-00002.safetensors",
                      [("a.weight", "U8", [10, 100], a.tobytes()), ("b", "F32", [3, 5], b.tobytes())],
                      metadata={"format": "pt", "note": 'x"y'})
    (tmp_path / "config.json").write_text("{}")  # not a shard
    sh = _shards(tmp_path)
    assert len(sh) == 3
    ia, ib, ic = sh.find("a.weight"), sh.find("b"), sh.find("c.weight")
    assert (ia["file_index"], ib["file_index"], ic["file_index"]) == (0, 0, 1)
    assert ia["shape"] == [10, 100] and ia["dtype"] == "U8" and ia["nbytes"] == 1000
    assert ib["shape"] == [3, 5] and ib["dtype"] == "F32" and ib["nbytes"] == 60
    assert ib["offset"] == ia["offset"] + 1000
    assert np.array_equal(sh.read("a.weight"), a)
    assert np.array_equal(sh.read("b").view(np.float32).reshape(3, 5), b)
    assert np.array_equal(sh.read("c.weight"), c)
    assert np.array_equal(sh.read_range("a.weight", 990, 10), a[990:])


def test_later_shard_wins_a_repeated_name(tmp_path, rbt_lib):
    # HashMap::insert over shards in file-name order (safetensors.rs:334)
    write_safetensors(tmp_path / "a.safetensors", [("t", "U8", [2], b"\x01\x02")])
    write_safetensors(tmp_path / "b.safetensors", [("t", "U8", [3], b"\x07\x08\x09")])
    sh = _shards(tmp_path)
    assert len(sh) == 1 and list(sh.read("t")) == [7, 8, 9]


def test_header_escapes_whitespace_and_shape_filtering(tmp_path, rbt_lib):
    # a JSON header written by hand: escapes in names, spaces, a float and a negative shape entry
    # (the reference keeps only the u64 entries: filter_map(as_u64))
    hdr = ('{ "__metadata__" : {"k": [1, 2.5, {"z": null}]},\n'
           ' "caf\\u00e9.w\\"q" : {"dtype":"U8", "shape":[2, -1, 3.5, 4], "data_offsets":[0, 8]} }').encode()
    write_safetensors(tmp_path / "m.safetensors", [], raw_header=hdr)
    with open(tmp_path / "m.safetensors", "ab") as f:
        f.write(bytes(range(8)))
    sh = _shards(tmp_path)
    info = sh.find('café.w"q')
    assert info["shape"] == [2, 4] and info["nbytes"] == 8
    assert list(sh.read('café.w"q')) == list(range(8))


def _bad(tmp_path, hdr_obj=None, raw=None, data=b"\x00" * 16):
    import rabbit_amd as R
    hb = raw if raw is not None else json.dumps(hdr_obj).encode()
    with open(tmp_path / "bad.safetensors", "wb") as f:
        f.write(len(hb).to_bytes(8, "little"))
        f.write(hb)
        f.write(data)
    with pytest.raises(R.RbtError) as ei:
        R.Shards(str(tmp_path))
    return ei.value


def test_rejects_end_before_start(tmp_path, rbt_lib):
    # safetensors.rs:769-782
    e = _bad(tmp_path, {"a": {"dtype": "F32", "shape": [1], "data_offsets": [4, 0]}})
    assert e.status == -8 and "precedes start" in str(e)


def test_rejects_end_past_end_of_file(tmp_path, rbt_lib):
    # safetensors.rs:785-800
    e = _bad(tmp_path, {"a": {"dtype": "F32", "shape": [1024], "data_offsets": [0, 4096]}})
    assert e.status == -8 and "extends past end of file" in str(e)


def test_rejects_header_longer_than_file(tmp_path, rbt_lib):
    import rabbit_amd as R
    with open(tmp_path / "x.safetensors", "wb") as f:
        f.write((1 << 40).to_bytes(8, "little"))
        f.write(b"{}")
    with pytest.raises(R.RbtError) as ei:
        R.Shards(str(tmp_path))
    assert ei.value.status == -8 and "exceeds file size" in str(ei.value)


@pytest.mark.parametrize("meta,what", [
    ({"dtype": "F64", "shape": [1], "data_offsets": [0, 8]}, "unknown dtype"),
    ({"dtype": "U8", "shape": [1], "data_offsets": [0, 1, 2]}, "must have 2 elements"),
    ({"dtype": "U8", "shape": [1], "data_offsets": [-1, 1]}, "is not a u64"),
    ({"shape": [1], "data_offsets": [0, 1]}, "missing dtype"),
    ({"dtype": "U8", "data_offsets": [0, 1]}, "missing shape"),
])
def test_rejects_malformed_entries(tmp_path, rbt_lib, meta, what):
    e = _bad(tmp_path, {"a": meta})
    assert e.status == -8 and what in str(e)


def test_rejects_bad_json_and_reports_missing_tensors(tmp_path, rbt_lib):
    import rabbit_amd as R
    e = _bad(tmp_path, raw=b'{"a": {"dtype": "U8", ')
    assert e.status == -8 and "header json" in str(e)
    (tmp_path / "bad.safetensors").unlink()
    write_safetensors(tmp_path / "ok.safetensors", [("t", "U8", [1], b"\x05")])
    sh = R.Shards(str(tmp_path))
    with pytest.raises(R.RbtError) as ei:
        sh.find("nope")
    assert ei.value.status == -7 and "missing tensor: nope" in str(ei.value)
    with pytest.raises(R.RbtError) as ei:
        sh.read_range("t", 1, 1)
    assert ei.value.status == -2
