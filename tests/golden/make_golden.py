"""Writes tests/golden/granite_cfg1.npz from the oracle (oracle/qx_oracle.c).

Config 1 of the benchmark plan: one Granite attention layer, seeded
q [1024] / k [512] / v [512] ~ N(0,1) fp32 per step (numpy PCG64,
standard_normal(dtype=float32), drawn as three [512, n] blocks in the order
q, k, v), positions 0..511 appended into an fp32 cache of capacity 512.
Stored: the [1024] outputs at the reference parity checkpoints
{0,1,7,31,63,127,255,511} (tools/qx-bench/src/main.rs:10925-11079) and a
sha256 of the inputs so generator drift is detected.

The reference implementation is Rust and cannot run here; these vectors pin
the oracle against regressions and are the GPU parity target.
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402

SEED = 20261201
CHECKPOINTS = [0, 1, 7, 31, 63, 127, 255, 511]


def inputs(seed=SEED, positions=512):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((positions, 1024), dtype=np.float32)
    k = rng.standard_normal((positions, 512), dtype=np.float32)
    v = rng.standard_normal((positions, 512), dtype=np.float32)
    return q, k, v


def digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def main():
    q, k, v = inputs()
    cache = O.KvCache(512)
    outs = []
    for p in range(512):
        out = O.granite_attention_decode(q[p], k[p], v[p], p, cache)
        if p in CHECKPOINTS:
            outs.append(out)
    np.savez_compressed(os.path.join(HERE, "granite_cfg1.npz"), seed=np.int64(SEED),
                        checkpoints=np.array(CHECKPOINTS, np.int64), outputs=np.stack(outs),
                        input_sha256=np.array(digest(q, k, v)))
    print("wrote granite_cfg1.npz")


if __name__ == "__main__":
    main()
