"""The reference's model file, format v4 (model_serialization.hpp:36-52, 150-300,
380-503; keyvalue_record.hpp:20-200), written and read by the GPT session.

Pinned by an independent Python parser of the bytes written from the layout
the reference documents (header, spec record, matrices, tokenizer), by a save
/ load round trip, and by the reference's load errors (bad magic, other
versions, other precision, shape mismatch, truncation)."""
import struct

import numpy as np
import pytest

import nnengine

CFG = dict(vocab_size=40, d_model=16, seq_len=8, num_heads=2, d_ff=24, num_layers=2, pos_enc="alibi")
SPEC_ORDER = ["type", "layer_dims", "d_model", "num_heads", "d_ff", "num_layers", "patch_size", "vocab_size",
              "seq_len", "pos_encoding", "activation", "norm_type"]


def _session(eng, seed=0, cfg=CFG):
    g = eng.gpt(**cfg)
    rng = np.random.default_rng(seed)
    g.set_params([rng.normal(0, 0.1, s).astype(np.float32) for s in g.param_shapes()])
    return g


def _parse(raw):
    off = 0

    def take(fmt):
        nonlocal off
        v = struct.unpack_from("<" + fmt, raw, off)
        off += struct.calcsize("<" + fmt)
        return v if len(v) > 1 else v[0]
    magic, version, prec = raw[:4], take("xxxxI"), take("B")
    spec_len = take("Q")
    end = off + spec_len
    count = take("I")
    fields = []
    for _ in range(count):
        klen = take("I")
        key = raw[off:off + klen].decode()
        off += klen
        typ, vlen = take("B"), take("I")
        val = raw[off:off + vlen]
        off += vlen
        fields.append((key, typ, val))
    assert off == end
    return magic, version, prec, fields, off


def test_file_bytes_follow_the_reference_layout(cpu, tmp_path):
    g = _session(cpu)
    path = str(tmp_path / "m.nnm")
    tok = b'{"model":"bpe","vocab":[]}'
    g.save(path, tok)
    raw = open(path, "rb").read()
    magic, version, prec, fields, off = _parse(raw)
    assert magic == b"NNNN" and version == 4 and prec == 0
    assert [k for k, _, _ in fields] == SPEC_ORDER
    vals = {k: (t, v) for k, t, v in fields}
    assert vals["layer_dims"] == (2, b"")
    u = {k: struct.unpack("<Q", v)[0] for k, (t, v) in vals.items() if t == 0}
    assert u == dict(type=3, d_model=16, num_heads=2, d_ff=24, num_layers=2, patch_size=0, vocab_size=40,
                     seq_len=8, pos_encoding=2, activation=1, norm_type=1)
    for p in g.params():
        r, c = struct.unpack_from("<QQ", raw, off)
        off += 16
        assert (r, c) == p.shape
        got = np.frombuffer(raw, dtype="<f4", count=r * c, offset=off).reshape(r, c)
        off += 4 * r * c
        assert np.array_equal(got, p)
    (tlen,) = struct.unpack_from("<Q", raw, off)
    off += 8
    assert raw[off:off + tlen] == tok and off + tlen == len(raw)


def test_round_trip(cpu, tmp_path):
    a, b = _session(cpu, 1), _session(cpu, 2)
    path = str(tmp_path / "m.nnm")
    a.save(path)
    assert b.load(path) == b""
    for x, y in zip(a.params(), b.params()):
        assert np.array_equal(x, y)


def test_load_errors(cpu, tmp_path):
    g = _session(cpu)
    path = tmp_path / "m.nnm"
    g.save(str(path), b"tok")
    good = path.read_bytes()

    def bad(raw):
        p = tmp_path / "bad.nnm"
        p.write_bytes(raw)
        with pytest.raises(nnengine.EngineError):
            _session(cpu).load(str(p))
    bad(b"MMMM" + good[4:])                                   # magic
    bad(good[:4] + struct.pack("<I", 3) + good[8:])           # older format
    bad(good[:4] + struct.pack("<I", 5) + good[8:])           # newer format
    bad(good[:8] + b"\x01" + good[9:])                        # f64 file
    bad(good[:len(good) - 10])                                # truncated
    other = dict(CFG, d_model=32)
    with pytest.raises(nnengine.EngineError):
        cpu.gpt(**other).load(str(path))                      # shape mismatch
