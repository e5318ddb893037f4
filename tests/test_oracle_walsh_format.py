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
