"""Model files (format v4) move between the HIP engine and the oracle in both
directions with every parameter bit-identical."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CFG = dict(vocab_size=64, d_model=32, seq_len=16, num_heads=4, d_ff=48, num_layers=2, pos_enc="learned")


def _session(eng, seed):
    g = eng.gpt(**CFG)
    rng = np.random.default_rng(seed)
    g.set_params([rng.normal(0, 0.1, s).astype(np.float32) for s in g.param_shapes()])
    return g


def test_interchange(hip, cpu, tmp_path):
    for src, dst in ((hip, cpu), (cpu, hip)):
        a, b = _session(src, 3), _session(dst, 4)
        path = str(tmp_path / "m.nnm")
        a.save(path, b"tokenizer")
        assert b.load(path) == b"tokenizer"
        for x, y in zip(a.params(), b.params()):
            assert np.array_equal(x, y)
