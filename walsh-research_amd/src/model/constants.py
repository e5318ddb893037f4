"""Cayley-Dickson octonion tables (src/model/constants.py:13-52).

y_i = sum_j SIGN_TABLE[i][j] * x_j @ W[WEIGHT_IDX[i][j]]^T, the octonion
product x*w; WEIGHT_IDX[i][j] = i XOR j.  (The reference file also holds
backward tables that nothing uses and that are not the transposes these
forward tables imply; they are not reproduced.)
"""

SIGN_TABLE = [
    [+1, -1, -1, -1, -1, -1, -1, -1],
    [+1, +1, +1, -1, +1, -1, -1, +1],
    [+1, -1, +1, +1, +1, +1, -1, -1],
    [+1, +1, -1, +1, +1, -1, +1, -1],
    [+1, -1, -1, -1, +1, +1, +1, +1],
    [+1, +1, -1, +1, -1, +1, -1, +1],
    [+1, +1, +1, -1, -1, +1, +1, -1],
    [+1, -1, +1, +1, -1, -1, +1, +1],
]

WEIGHT_IDX = [[i ^ j for j in range(8)] for i in range(8)]
