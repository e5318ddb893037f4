"""Oracle: Cayley-Dickson octonion ternary linear layer.

Test infrastructure only (see ``oracle/__init__.py``).

The layer (``src/model/physics.py:66-82``) maps 8 input parts x_j
[M, in_o] to 8 output parts
    y_i = beta * sum_j S[i][j] * x_j @ W[idx[i][j]]^T ,
with the sign table S and index table idx of ``src/model/constants.py:13-52``
(idx[i][j] = i XOR j).  The tables are typed in below as data; the oracle
tests re-derive them from a Cayley-Dickson doubling of the quaternions.
"""
import numpy as np

# src/model/constants.py:13-31 (rows = output part i, columns = input part j)
SIGN_TABLE = np.array([
    [+1, -1, -1, -1, -1, -1, -1, -1],
    [+1, +1, +1, -1, +1, -1, -1, +1],
    [+1, -1, +1, +1, +1, +1, -1, -1],
    [+1, +1, -1, +1, +1, -1, +1, -1],
    [+1, -1, -1, -1, +1, +1, +1, +1],
    [+1, +1, -1, +1, -1, +1, -1, +1],
    [+1, +1, +1, -1, -1, +1, +1, -1],
    [+1, -1, +1, +1, -1, -1, +1, +1],
], dtype=np.int8)

# src/model/constants.py:34-52
WEIGHT_IDX = np.array([[i ^ j for j in range(8)] for i in range(8)], dtype=np.int8)


def octonion_linear_f64(x_parts, codes, beta) -> np.ndarray:
    """Float64 forward.  x_parts [8, M, in_o], codes [8, out_o, in_o],
    beta [out_o] broadcast over all 8 parts (``physics.py:63-64, 81-82``).
    Returns [8, M, out_o]."""
    x = np.asarray(x_parts, dtype=np.float64)
    w = np.asarray(codes, dtype=np.float64)
    y = np.zeros((8, x.shape[1], w.shape[1]))
    for i in range(8):
        for j in range(8):
            y[i] += SIGN_TABLE[i, j] * (x[j] @ w[WEIGHT_IDX[i, j]].T)
    return y * np.asarray(beta, np.float64)


def bf16_round(a) -> np.ndarray:
    """Round float32 values to bfloat16 (ties to even), returned as float32."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    nan = np.isnan(a)
    if nan.any():
        out = out.copy()
        out[nan] = np.nan
    return out


def octonion_linear_gpu_semantics(x_parts, codes, beta) -> np.ndarray:
    """What the reference GPU path returns: inputs cast to bf16 in-kernel,
    float32 accumulation, the sum rounded to bf16 (``cayley_dickson_cuda.py:
    402, 411, 421``), then multiplied by beta in bf16 arithmetic
    (``:668``, bf16 tensor times float32 parameter promotes to float32 and
    the caller keeps that dtype).  Computed here in float64 on the
    bf16-rounded inputs, with the stated roundings."""
    xb = bf16_round(x_parts).astype(np.float64)
    acc = octonion_linear_f64(xb, codes, np.ones(np.asarray(codes).shape[1]))
    yb = bf16_round(acc.astype(np.float32)).astype(np.float64)
    return yb * np.asarray(beta, np.float64)


def dense_matrix(codes, beta) -> np.ndarray:
    """The layer as a dense [8*out_o, 8*in_o] matrix: block (i, j) is
    beta * S[i][j] * W[i^j] (rows: output part-major, columns: input
    part-major, matching ``chassis.py:426`` splits)."""
    w = np.asarray(codes, dtype=np.float64)
    out_o, in_o = w.shape[1], w.shape[2]
    A = np.zeros((8 * out_o, 8 * in_o))
    for i in range(8):
        for j in range(8):
            A[i * out_o:(i + 1) * out_o, j * in_o:(j + 1) * in_o] = SIGN_TABLE[i, j] * w[WEIGHT_IDX[i, j]]
    return np.asarray(beta, np.float64).reshape(1, -1).repeat(8, 0).reshape(-1)[:, None] * A


def octonion_linear_bwd_f64(x_parts, codes, beta, gy_parts, latent=None):
    """Float64 gradients of ``octonion_linear_f64`` for output gradients gy
    [8, M, out_o]: the exact transpose of the forward's block structure (what
    CayleyDicksonFunction.backward computes, ``cayley_dickson_cuda.py:500-567``)
    and the STE of physics.quantize_ternary (``physics.py:48-50``): the weight
    gradient is zero where the latent weight lies outside [-1.5, 1.5].

    Returns (dx [8, M, in_o], dW [8, out_o, in_o], dbeta [out_o]).
    """
    x = np.asarray(x_parts, dtype=np.float64)
    w = np.asarray(codes, dtype=np.float64)
    gy = np.asarray(gy_parts, dtype=np.float64)
    b = np.asarray(beta, np.float64)
    g = gy * b
    dx = np.zeros_like(x)
    dW = np.zeros_like(w)
    dbeta = np.zeros(w.shape[1])
    for i in range(8):
        ypre = np.zeros(gy.shape[1:])
        for j in range(8):
            k = WEIGHT_IDX[i, j]
            s = SIGN_TABLE[i, j]
            dx[j] += s * (g[i] @ w[k])
            dW[k] += s * (g[i].T @ x[j])
            ypre += s * (x[j] @ w[k].T)
        dbeta += (gy[i] * ypre).sum(0)
    if latent is not None:
        lat = np.asarray(latent, np.float64)
        dW = dW * ((lat >= -1.5) & (lat <= 1.5))
    return dx, dW, dbeta
