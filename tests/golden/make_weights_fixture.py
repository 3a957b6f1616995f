"""Builds the serialised-weight fixtures of tests/golden/ from the format's definition
(include/rocket_weights_io.h) with numpy alone, independently of the library:

    weights_int4_g32.rktw   int4 group-wise weight N=64 K=128 group=32, with its fp32 scales
    weights_int8_pc.rktw    int8 per-channel weight N=32 K=64, no scales

Run `python tests/golden/make_weights_fixture.py` to rewrite them; the tests regenerate the
bytes and compare, so the committed files pin the format.
"""
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def xxh64(data: bytes) -> int:
    """XXH64 with seed 0, from the independent `xxhash` package."""
    import xxhash
    return xxhash.xxh64(data, seed=0).intdigest()


def pack_int4(B):
    """int4 values [N, K] -> the device layout: per 8 values of K one little-endian word whose
    byte j holds value 8d+j in the high nibble and 8d+4+j in the low nibble."""
    N, K = B.shape
    v = (B.astype(np.int16) & 0xF).astype(np.uint8).reshape(N, K // 8, 2, 4)
    return ((v[:, :, 0, :] << 4) | v[:, :, 1, :]).astype(np.uint8).tobytes()


def serialise(kind, N, K, group, M, codes: bytes, scales=None) -> bytes:
    sb = b"" if scales is None else np.ascontiguousarray(scales, "<f4").tobytes()
    head = b"RKTW" + struct.pack("<7I", 1, kind, 1 if scales is not None else 0, N, K, group, M)
    head += struct.pack("<3Q", len(codes), len(sb), xxh64(codes + sb))
    head += struct.pack("<Q", xxh64(head))
    assert len(head) == 64
    return head + codes + sb


def int4_fixture():
    rng = np.random.default_rng(0x52545457)
    N, K, group, M = 64, 128, 32, 4
    B = rng.integers(-8, 8, (N, K)).astype(np.int8)
    scales = rng.uniform(0.005, 0.02, (N, K // group)).astype(np.float32)
    return B, scales, serialise(2, N, K, group, M, pack_int4(B), scales)


def int8_fixture():
    rng = np.random.default_rng(0x52545458)
    N, K, M = 32, 64, 8
    B = rng.integers(-128, 128, (N, K)).astype(np.int8)
    return B, serialise(1, N, K, 0, M, B.tobytes())


if __name__ == "__main__":
    with open(os.path.join(HERE, "weights_int4_g32.rktw"), "wb") as f:
        f.write(int4_fixture()[2])
    with open(os.path.join(HERE, "weights_int8_pc.rktw"), "wb") as f:
        f.write(int8_fixture()[1])
