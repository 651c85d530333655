"""Oracle pins for the KV / state commitment hashing (oracle/qx_oracle_hash.c).

BLAKE3 is the `blake3` crate 1.8.7 (Cargo.lock:656-659, not vendored); the
commitment framing is crates/qx-commit/src/{hash.rs,state.rs,merkle.rs,execution.rs}.
Pins: the BLAKE3 project's published test vectors (test_vectors.json of the
BLAKE3 specification repository: input byte i is i mod 251) for 0, 1, 1023
and 1024 bytes, so one to sixteen 64-byte blocks of a chunk, with the
partial last block; and the reference's own protocol golden vectors
(crates/qx-commit/tests/golden_vectors.rs:66-190), which run kv_leaf_hash_v1,
state_hash_v1 and BLAKE3 Merkle parents on one-chunk trees.  SHA-256 leaves
of those vectors come from hashlib.  Trees of several 256-byte chunks (token
rows above 256 bytes) are built from these pinned primitives in state.rs's
order (crates/qx-commit/src/state.rs:313-348); no reference vector covers a
multi-chunk tree itself.
"""
import hashlib
import struct

import pytest

from oracle import oracle as O


def sha_domain(domain: bytes, fields) -> bytes:
    """hash_domain(Sha256V1, ...), crates/qx-commit/src/hash.rs:41-50."""
    h = hashlib.sha256(domain)
    for f in fields:
        h.update(len(f).to_bytes(8, "little"))
        h.update(f)
    return h.digest()


def b3_merkle_pair(tree_domain: bytes, left: bytes, right: bytes) -> bytes:
    """MerkleTree::new over two leaves (crates/qx-commit/src/merkle.rs:5-12, 69-99)."""
    return O.hash_domain_b3(O.D_MERKLE, [tree_domain, left, right])


def f32_bytes(values):
    return b"".join(struct.pack("<f", v) for v in values)


# BLAKE3 test_vectors.json: (input length, first 32 bytes of the hash)
BLAKE3_PUBLISHED = [
    (0, "af1349b9f5f9a1a6a0404dea36dcc9499bcb25c9adc112b7cc9a93cae41f3262"),
    (1, "2d3adedff11b61f14c886e35afa036736dcd87a74d27b5c1510225d0f592e213"),
    (1023, "10108970eeda3eb932baac1428c7a2163b0e924c9a9e25b35bba72b28f70bd11"),
    (1024, "42214739f095a406f3fc83deb889744ac00df831c10daa55189b5d121c855af7"),
]


@pytest.mark.parametrize("n,digest", BLAKE3_PUBLISHED)
def test_blake3_published_vectors(n, digest):
    assert O.blake3(bytes(i % 251 for i in range(n))).hex() == digest


def test_blake3_single_chunk_limit():
    # the commitment scheme never hashes more than one 1024-byte chunk at once
    with pytest.raises(RuntimeError, match="input rejected"):
        O.blake3(bytes(1025))


def test_reference_protocol_golden_vectors():
    kv_leaf = O.kv_leaf_hash_v1(2, 9, f32_bytes([1.0, -2.0, 0.5, -0.0]), f32_bytes([3.0, 4.0, -5.0, 6.0]))
    assert kv_leaf.hex() == "3516c5116950fd510fd4c2c65b63454c29739d9030e3a83e1944391137b8dac1"
    kv_root = b3_merkle_pair(O.D_KV, kv_leaf, sha_domain(O.D_KV, [b"other-kv-leaf"]))
    assert kv_root.hex() == "ac3cb8d1ef765a4b2e71c4adc61921ab2105650d8a3685e445df7c27afbd3c6c"
    # CheckpointV1::hash (crates/qx-commit/src/execution.rs:33-53)
    residual = O.state_hash_v1(f32_bytes([0.25, -1.5]))
    canonical = bytes([0x11] * 32) + (9).to_bytes(4, "little") + (2).to_bytes(2, "little") + residual + kv_root
    checkpoint = O.hash_domain_b3(O.D_CHECKPOINT, [canonical])
    assert checkpoint.hex() == "73eabcfc5497772b03f0473ae0054c66a93b5b83b877ba3e5f5640dfa8b1a826"
    token_root = b3_merkle_pair(b"QX:TOKEN:V1", checkpoint, sha_domain(O.D_CHECKPOINT, [b"other"]))
    assert token_root.hex() == "a4fe82012dbe3226056e3292f4c8aaa86ca00056f3200b329f3a4a8fb39f1203"
    # TokenResultV1::hash (execution.rs:69-90): job, token 9, root, predicted 42, count 2
    tr = bytes([0x11] * 32) + (9).to_bytes(4, "little") + token_root + (42).to_bytes(4, "little") + \
        (2).to_bytes(4, "little")
    token_result = O.hash_domain_b3(b"QX:TOKEN:RESULT:V1", [tr])
    assert token_result.hex() == "ac0f9c304fcee19fb42743cbf0458a778dc706255736cc62f5c84625c50d2d6a"
    job_root = b3_merkle_pair(b"QX:JOB:V1", token_result, sha_domain(b"QX:TOKEN:V1", [b"other-token"]))
    assert job_root.hex() == "ae1dc5b1f6871042973bbb1585da16264b7247a030e6d31e648c51a55040dca2"


def test_chunk_boundaries_and_coordinates_are_committed():
    # crates/qx-commit/src/state.rs:372-386
    assert O.state_hash_v1(bytes([7] * 257)) != O.state_hash_v1(bytes([7] * 256))
    key, value = bytes([1] * 256), bytes([2] * 256)
    assert O.kv_leaf_hash_v1(1, 2, key, value) != O.kv_leaf_hash_v1(2, 2, key, value)


def test_empty_commitment_input_is_rejected():
    # chunk_tree_hash: "state commitment input must not be empty" (state.rs:219-223)
    with pytest.raises(RuntimeError):
        O.state_hash_v1(b"")


def test_single_chunk_tree_is_the_chunk_leaf():
    """A tree of one chunk is its leaf, hash_domain(leaf domain, [u32 0, bytes])."""
    data = bytes(range(200))
    leaf = O.hash_domain_b3(O.D_KV_KEY_CHUNK, [(0).to_bytes(4, "little"), data])
    assert O.chunk_tree_hash(data, 256, O.D_KV_KEY_CHUNK, O.D_KV_KEY_TREE) == leaf


def test_verification_digest_layout():
    """kernels/verification_hash.metal:349-522 on the oracle: genesis = (state
    root, zeros); checkpoint layers carry a state root, the others zeros; every
    layer carries kv_leaf_hash_v1 of its rows."""
    layers, stride, interval = 3, 512, 2
    res = bytes((i * 7 + 3) & 0xFF for i in range((layers + 1) * stride))
    krows = [bytes((i + 31 * l) & 0xFF for i in range(1024)) for l in range(layers)]
    vrows = [bytes((3 * i + 17 * l) & 0xFF for i in range(1024)) for l in range(layers)]
    out = O.verification_hashes(res, stride, krows, vrows, 77, layers, interval)
    assert out[0:32] == O.state_hash_v1(res[:stride]) and out[32:64] == bytes(32)
    for p in range(1, layers + 1):
        layer = p - 1
        d = out[64 * p:64 * p + 64]
        ckpt = (layer + 1) % interval == 0 or layer + 1 == layers
        assert d[:32] == (O.state_hash_v1(res[p * stride:(p + 1) * stride]) if ckpt else bytes(32))
        assert d[32:] == O.kv_leaf_hash_v1(layer, 77, krows[layer], vrows[layer])


def test_batched_leaves_equal_single_leaves_and_are_thread_safe():
    """qxo_kv_leaf_hashes (the CPU baseline's loop) equals kv_leaf_hash_v1 row
    by row, also when four threads hash at once (the chunk tree's node
    scratch is per thread)."""
    import concurrent.futures as cf

    import numpy as np

    g = np.random.default_rng(12)
    keys = g.integers(0, 256, (24, 1024), dtype=np.uint8)
    values = g.integers(0, 256, (24, 2048), dtype=np.uint8)
    got = O.kv_leaf_hashes(3, 100, keys, values)
    for i in range(24):
        assert bytes(got[i]) == O.kv_leaf_hash_v1(3, 100 + i, keys[i].tobytes(), values[i].tobytes())
    with cf.ThreadPoolExecutor(4) as ex:
        outs = list(ex.map(lambda _: O.kv_leaf_hashes(3, 100, keys, values), range(16)))
    assert all(np.array_equal(o, got) for o in outs)
