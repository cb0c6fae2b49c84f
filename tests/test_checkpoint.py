"""Checkpoint reader (safetensors.rs) on the CPU: files written by the
safetensors library read back bit for bit through the C ABI, the shard
discovery and precedence of MultiSafetensors::open / find, and the header
validation that turns malformed files into errors."""
import json
import os
import struct

import numpy as np
import pytest

from conftest import rng


def _ck():
    from qwenasr_amd.model import Checkpoint
    return Checkpoint


def raw_file(path, header, data=b""):
    h = header if isinstance(header, bytes) else json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + data)
    return path


def test_reader_matches_safetensors_library(tmp_path):
    import torch
    from safetensors.torch import save_file
    r = rng(11)
    src = {
        "f32": torch.from_numpy(r.normal(0, 1, (3, 5)).astype(np.float32)),
        "bf16": torch.from_numpy(r.normal(0, 1, (4, 8)).astype(np.float32)).to(torch.bfloat16),
        "f16": torch.from_numpy(r.normal(0, 1, (7,)).astype(np.float16)),
        "i64": torch.arange(-3, 9, dtype=torch.int64).reshape(2, 2, 3),
        "i32": torch.tensor([1, -2, 3], dtype=torch.int32),
        "bool": torch.tensor([True, False, True]),
        "scalar": torch.tensor(2.5, dtype=torch.float32),
        "empty": torch.zeros((0, 3), dtype=torch.float32),
        "name with spaces/é": torch.ones(2, dtype=torch.float32),
    }
    save_file(src, str(tmp_path / "x.safetensors"), metadata={"format": "pt", "note": "a\"b"})
    ck = _ck()(tmp_path / "x.safetensors", file=True)
    assert sorted(ck.names()) == sorted(src)
    assert ck.n_shards == 1
    for n, t in src.items():
        got = ck.array(n)
        if t.dtype == torch.bfloat16:
            want = t.view(torch.int16).numpy().view(np.uint16)
            assert ck.find(n)[0] == 3
        else:
            want = t.numpy()
        assert got.shape == tuple(t.shape), n
        assert got.dtype == want.dtype and got.tobytes() == want.tobytes(), n
    from qwenasr_amd import QasrError
    with pytest.raises(QasrError):
        ck.find("absent")
    ck.close()


def test_shards_and_precedence(tmp_path):
    from qwenasr_amd import QasrError
    from qwenasr_amd.synth import SynthDecoder, decoder_tensors, write_checkpoint
    cfg = dict(n_layers=2, hidden=64, n_heads=2, n_kv_heads=1, head_dim=128, intermediate=128, vocab=32,
               eps=1e-6, theta=1e6)
    tens = decoder_tensors(SynthDecoder(cfg, seed=3))
    d = tmp_path / "m"
    write_checkpoint(str(d), tens, shards=3)
    Checkpoint = _ck()
    ck = Checkpoint(d)
    assert ck.n_shards == 3 and sorted(ck.names()) == sorted(tens)
    for n, (a, _) in tens.items():
        assert ck.array(n).tobytes() == np.ascontiguousarray(a).tobytes(), n
    ck.close()
    # a name in two shards: the first shard in name order wins (find, safetensors.rs:254-262)
    import torch
    from safetensors.torch import save_file
    save_file({"dup": torch.zeros(4)}, str(d / "model-00000-extra.safetensors"))
    save_file({"dup": torch.ones(4)}, str(d / "model-zzz.safetensors"))
    ck = Checkpoint(d)
    assert ck.n_shards == 5 and (ck.array("dup") == 0).all()
    ck.close()
    # model.safetensors, when it opens, is the whole checkpoint
    save_file({"only": torch.ones(2)}, str(d / "model.safetensors"))
    ck = Checkpoint(d)
    assert ck.n_shards == 1 and ck.names() == ["only"]
    ck.close()
    # ... and when it does not open, the shards are read instead
    (d / "model.safetensors").write_bytes(b"not a checkpoint")
    ck = Checkpoint(d)
    assert ck.n_shards == 5
    ck.close()
    # files that are not model-*.safetensors are ignored; none at all is an error
    e = tmp_path / "empty"
    e.mkdir()
    save_file({"x": torch.ones(1)}, str(e / "weights.safetensors"))
    with pytest.raises(QasrError, match="no safetensors"):
        Checkpoint(e)


BAD_HEADERS = [
    ("not a JSON object", b"[1, 2]"),
    ("truncated", b'{"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]'),
    ("offsets past the data", {"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}),
    ("offsets disagree with the shape", {"a": {"dtype": "F32", "shape": [3], "data_offsets": [0, 4]}}),
    ("decreasing offsets", {"a": {"dtype": "U8", "shape": [1], "data_offsets": [4, 0]}}),
    ("missing offsets", {"a": {"dtype": "F32", "shape": [1]}}),
    ("float in shape", b'{"a": {"dtype": "F32", "shape": [1.0], "data_offsets": [0, 4]}}'),
    ("leading zero", b'{"a": {"dtype": "F32", "shape": [01], "data_offsets": [0, 4]}}'),
    ("negative dimension", {"a": {"dtype": "F32", "shape": [-1], "data_offsets": [0, 4]}}),
    ("trailing bytes", b'{"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}} x'),
    ("not UTF-8", b'{"\xff": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}}'),
    ("lone surrogate", b'{"\\ud800": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}}'),
    ("bad escape", b'{"\\q": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}}'),
]


@pytest.mark.parametrize("what,header", BAD_HEADERS, ids=[b[0] for b in BAD_HEADERS])
def test_malformed_headers_are_errors(tmp_path, what, header):
    from qwenasr_amd import QasrError
    p = raw_file(tmp_path / "bad.safetensors", header, b"\0" * 4)
    with pytest.raises(QasrError, match="bad.safetensors"):
        _ck()(p, file=True)


def test_short_and_oversized_files(tmp_path):
    from qwenasr_amd import QasrError
    (tmp_path / "short.safetensors").write_bytes(b"\x01\x02")
    with pytest.raises(QasrError, match="shorter than 8"):
        _ck()(tmp_path / "short.safetensors", file=True)
    (tmp_path / "big.safetensors").write_bytes(struct.pack("<Q", 1000) + b"{}")
    with pytest.raises(QasrError, match="header length"):
        _ck()(tmp_path / "big.safetensors", file=True)
    with pytest.raises(QasrError, match="cannot open"):
        _ck()(tmp_path / "absent.safetensors", file=True)


def test_header_escapes_metadata_and_unknown_fields(tmp_path):
    hdr = (b'{"__metadata__": {"k": ["nested", {"x": [1, 2.5e3, true, null]}]},'
           b' "a\\u00e9\\ud83d\\ude00\\n\\"": {"dtype": "I32", "shape": [2], "data_offsets": [0, 8], "extra": {"z": 1}},'
           b' "u8": {"dtype": "U8", "shape": [3], "data_offsets": [8, 11]},'
           b' "dup": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]},'
           b' "dup": {"dtype": "F32", "shape": [1], "data_offsets": [4, 8]}}')
    data = np.array([7, -9], np.int32).tobytes() + b"\x01\x02\x03"
    p = raw_file(tmp_path / "e.safetensors", hdr, data)
    ck = _ck()(p, file=True)
    name = "aé\U0001F600\n\""
    assert sorted(ck.names()) == sorted([name, "u8", "dup"])
    assert ck.array(name).tolist() == [7, -9]
    dt, shape, _, nbytes = ck.find("u8")                   # a dtype the reference does not know: kept, untyped
    assert dt == 0 and shape == (3,) and nbytes == 3
    assert ck.array("dup").view(np.int32).tolist() == [-9]    # a repeated name: the last entry wins
    ck.close()


def test_mutated_headers_never_escape_the_data(tmp_path):
    """Seeded byte mutations of a valid header (replace, delete, insert, a
    wrong header length, a short data region): every file is either rejected
    with an error or opens with tensors that lie wholly inside its data region
    (the data bytes are 128..167, so a tensor's bytes name their own offset)."""
    import random
    from qwenasr_amd import QasrError
    hdr = json.dumps({"__metadata__": {"format": "pt"},
                      "a": {"dtype": "F32", "shape": [2, 3], "data_offsets": [0, 24]},
                      "b": {"dtype": "BF16", "shape": [4], "data_offsets": [24, 32]},
                      "c": {"dtype": "I64", "shape": [1], "data_offsets": [32, 40]}}).encode()
    data = bytes(range(128, 168))
    alphabet = b'{}[]",:0123456789-+.eE \\u"tfnaFBI'
    r = random.Random(5)
    p = tmp_path / "m.safetensors"
    opened = 0
    for _ in range(1500):
        hh = bytearray(hdr)
        for _ in range(r.randint(1, 3)):
            k, i = r.randrange(4), r.randrange(len(hh) + 1)
            if k == 0 and i < len(hh):
                hh[i] = r.choice(alphabet)
            elif k == 1 and i < len(hh):
                del hh[i]
            elif k == 2:
                hh[i:i] = bytes([r.choice(alphabet)])
            else:
                hh[i:i] = bytes([r.randrange(256)])
        dd = data[:r.choice([40, 40, 40, 39, 24, 0])]
        hl = len(hh) if r.random() < 0.9 else r.randrange(len(hh) + 16)
        p.write_bytes(struct.pack("<Q", hl) + bytes(hh) + dd)
        try:
            ck = _ck()(p, file=True)
        except QasrError:
            continue
        opened += 1
        for n in ck.names():
            dt, shape, _, nbytes = ck.find(n)
            raw = ck.array(n).view(np.uint8).reshape(-1)
            assert raw.size == nbytes and nbytes <= len(dd), n
            if dt != 0:
                assert nbytes == int(np.prod(shape, dtype=np.int64)) * ck.array(n).dtype.itemsize, n
            if nbytes:
                o = int(raw[0]) - 128
                assert 0 <= o and raw.tobytes() == dd[o:o + nbytes], n
        ck.close()
    assert opened > 0
