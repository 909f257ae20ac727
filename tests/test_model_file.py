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


def _with_spec_field(raw, key, value):
    """The file bytes with one u64 spec field replaced (same length, so every offset holds)."""
    kb = key.encode()
    i = raw.index(struct.pack("<I", len(kb)) + kb + b"\x00" + struct.pack("<I", 8))
    j = i + 4 + len(kb) + 1 + 4
    return raw[:j] + struct.pack("<Q", value) + raw[j + 8:]


@pytest.mark.parametrize("key,value", [("num_heads", 4), ("seq_len", 16), ("pos_encoding", 1), ("activation", 0),
                                       ("norm_type", 0), ("type", 1)])
def test_load_rejects_another_spec(cpu, tmp_path, key, value):
    """A file whose spec describes another model with the same matrix shapes (other head count, context,
    position encoding, activation, norm, model type) does not load: the reference builds the model from
    the file's spec (text_train.cpp:940-952), a session's model is fixed, so the specs must agree. The
    type check is build_gpt_model_from_spec's (domain_gpt.hpp:90-92): type GPT, or ALiBi positions."""
    cfg = dict(CFG, pos_enc="learned") if key == "type" else CFG
    g = _session(cpu, cfg=cfg)
    path = tmp_path / "m.nnm"
    g.save(str(path))
    p = tmp_path / "other.nnm"
    p.write_bytes(_with_spec_field(path.read_bytes(), key, value))
    with pytest.raises(nnengine.EngineError, match="type|" + key):
        _session(cpu, cfg=cfg).load(str(p))
    # the unchanged file loads, and an ALiBi file may carry the legacy ALiBi_GPT type (4)
    _session(cpu, cfg=cfg).load(str(path))
    if cfg["pos_enc"] == "alibi":
        q = tmp_path / "legacy.nnm"
        q.write_bytes(_with_spec_field(path.read_bytes(), "type", 4))
        _session(cpu).load(str(q))


def test_load_restarts_the_optimizer(cpu, tmp_path):
    """After load the AdamW moments and step count start afresh, as an optimizer created after
    load_model does (text_train.cpp:952 then 966): one step after loading into a session that has
    trained equals one step of a fresh session that loaded the same file."""
    rng = np.random.default_rng(5)
    toks = rng.integers(0, CFG["vocab_size"], size=(CFG["seq_len"] + 1, 2))
    batch = (toks[:-1].astype(np.float32), toks[1:].T.reshape(-1))
    path = str(tmp_path / "m.nnm")
    _session(cpu, 1).save(path)
    used = _session(cpu, 2)
    for _ in range(3):
        used.load_batch(*batch)
        used.train_step()
    used.load(path)
    fresh = _session(cpu, 3)
    fresh.load(path)
    for g in (used, fresh):
        g.load_batch(*batch)
        g.train_step()
    for x, y in zip(used.params(), fresh.params()):
        assert np.array_equal(x, y)
