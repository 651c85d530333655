"""The oracle reproduces the committed golden vectors bit for bit."""
import os

import numpy as np

from oracle import oracle as O
from tests.golden.make_golden import digest, inputs

HERE = os.path.join(os.path.dirname(__file__), "golden")


def test_granite_cfg1_fixture():
    gold = np.load(os.path.join(HERE, "granite_cfg1.npz"))
    q, k, v = inputs(int(gold["seed"]))
    assert digest(q, k, v) == str(gold["input_sha256"]), "numpy generator drift: regenerate inputs"
    cache = O.KvCache(512)
    cps = list(gold["checkpoints"])
    for p in range(512):
        out = O.granite_attention_decode(q[p], k[p], v[p], p, cache)
        if p in cps:
            assert np.array_equal(out, gold["outputs"][cps.index(p)]), p
