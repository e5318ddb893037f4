"""Pins for oracle.walsh_format: a hand-worked vector and round trips."""
import numpy as np

from oracle import walsh_format as wf


def test_hand_worked_vector():
    # values 0, +1, -1, 0, 0, 0, 0, 0, +1 -> mask bits at 1, 2, 8 (LSB first):
    # bytes 0b00000110 = 6, 0b00000001 = 1; signs of the non-zeros +, -, + ->
    # bits 1, 0, 1 = 0b101 = 5
    codes = np.array([0, 1, -1, 0, 0, 0, 0, 0, 1], np.int8)
    bm, sg, nnz = wf.encode_codes(codes)
    assert bm.tolist() == [6, 1] and sg.tolist() == [5] and nnz == 3
    assert np.array_equal(wf.decode_codes(bm, sg, (9,), 3), codes)


def test_round_trip_and_num_nonzero_cut():
    rng = np.random.default_rng(0)
    for shape in ((32, 16, 16), (8, 5, 7), (1,), (3, 43)):
        codes = rng.integers(-1, 2, size=shape).astype(np.int8)
        bm, sg, nnz = wf.encode_codes(codes)
        assert len(bm) == (codes.size + 7) // 8 and len(sg) == (nnz + 7) // 8
        assert np.array_equal(wf.decode_codes(bm, sg, shape, nnz), codes)
    # a num_nonzero below the mask's count leaves the later non-zeros at 0
    codes = np.array([1, -1, 1, 1], np.int8)
    bm, sg, _ = wf.encode_codes(codes)
    assert wf.decode_codes(bm, sg, (4,), 2).tolist() == [1, -1, 0, 0]


# ------------------------------------------------- files written by the reference
import json  # noqa: E402
import os  # noqa: E402
import struct  # noqa: E402

import pytest  # noqa: E402

from oracle import ternary as otern  # noqa: E402

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
_DT = {0: np.int8, 1: np.int32, 2: np.float16, 3: np.float32}


def walk_walsh(path):
    """(config, {name: (marker, payload)}) of a .walsh v4 file, parsed with
    struct alone (the chunk layout of compress.py:146-355)."""
    with open(path, "rb") as f:
        b = f.read()
    pos = 0

    def take(n):
        nonlocal pos
        v = b[pos:pos + n]
        assert len(v) == n, "truncated"
        pos += n
        return v

    def u(fmt):
        return struct.unpack("<" + fmt, take(struct.calcsize(fmt)))[0]

    def array():
        code, nd = u("B"), u("B")
        shape = tuple(u("I") for _ in range(nd))
        dt = np.dtype(_DT[code])
        return np.frombuffer(take(int(np.prod(shape)) * dt.itemsize), dt).reshape(shape)
    assert take(4) == b"SPIN" and u("H") == 4
    config = json.loads(take(u("I")).decode())
    chunks = {}
    while True:
        m = take(1)
        if m == b"E" and b[pos:pos + 3] == b"ND!":
            pos += 3
            break
        name = take(u("H")).decode()
        if m in (b"E", b"A"):
            chunks[name] = (m, (u("f"), array()))
        elif m == b"B":
            shape = tuple(u("I") for _ in range(u("B")))
            nnz = u("I")
            bm = np.frombuffer(take(u("I")), np.uint8)
            sg = np.frombuffer(take(u("I")), np.uint8)
            chunks[name] = (m, (shape, nnz, bm, sg))
        else:
            chunks[name] = (m, array())
    assert pos == len(b)
    return config, chunks


@pytest.mark.parametrize("algebra", ["hadamard", "octonion"])
def test_reference_written_walsh_file(algebra):
    """tests/golden/tiny_<algebra>.walsh was written by the reference's
    compress_model (compress.py:121-358) from the tensors kept in
    walsh_files.npz.  The oracle's decoder reads the reference's ternary
    bytes back to the absmean codes of the latents (physics.py:24-29), the
    float16 entries are the latents rounded to float16, the int8 embedding
    is round(W / scale) with scale = max|W| / 127, the tied output weight is
    left out, and the mHC-free checkpoint has no chunk the reader skips."""
    path = os.path.join(GOLDEN, f"tiny_{algebra}.walsh")
    if not os.path.exists(path):
        pytest.skip("fixture not present")
    with np.load(os.path.join(GOLDEN, "walsh_files.npz"), allow_pickle=False) as z:
        sd = {k.split("/", 1)[1]: z[k] for k in z.files if k.startswith(algebra + "/")}
    config, chunks = walk_walsh(path)
    assert config["algebra"] == algebra and config["n_embd"] == 64
    assert "output.weight" not in chunks
    kinds = {}
    for name, (m, payload) in chunks.items():
        kinds[m] = kinds.get(m, 0) + 1
        if m == b"B":
            shape, nnz, bm, sg = payload
            w = sd[name]
            assert tuple(w.shape) == shape
            codes = otern.ternary_codes(w, otern.absmean_gamma(w))
            assert nnz == int((codes != 0).sum())
            assert np.array_equal(wf.decode_codes(bm, sg, shape, nnz), codes), name
        elif m == b"E":
            scale, q = payload
            w = sd[name]
            assert scale == np.float32(np.abs(w).max() / 127.0)
            assert np.array_equal(q, np.clip(np.round(w / np.float32(scale)), -127, 127).astype(np.int8))
        elif m == b"R":
            c = sd[name]
            assert np.array_equal(payload, np.stack([c.real, c.imag], -1).astype(np.float32))
        else:
            assert payload.dtype == np.float16
            assert np.array_equal(payload, sd[name].astype(np.float16)), name
    assert kinds[b"B"] == 7 and kinds[b"E"] == 1 and kinds[b"R"] == 1
    if algebra == "hadamard":
        assert kinds[b"L"] == 7 and kinds[b"H"] == 1 and kinds[b"h"] == 1
