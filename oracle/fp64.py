"""Float64 brute-force forms of the hot-path math, written from the equations.

TEST INFRASTRUCTURE ONLY (see oracle/qwen36_cpu.py).  These loops share no
code with qwen36_cpu.py: they are the independent check that pins it.  Each
function states the equation it evaluates; sizes are kept small by the tests.
"""

from __future__ import annotations

import math

import numpy as np


def rope_tables(position: int, rope_dim: int = 64, theta: float = 1e7) -> tuple[np.ndarray, np.ndarray]:
    """cos/sin of position * theta^(-2i/d), i < d/2, duplicated over both halves."""
    half = rope_dim // 2
    ang = np.array([position * theta ** (-(2.0 * i) / rope_dim) for i in range(half)], dtype=np.float64)
    ang = np.concatenate([ang, ang])
    return np.cos(ang), np.sin(ang)


def apply_rope(x: np.ndarray, position: int, rope_dim: int = 64, theta: float = 1e7) -> np.ndarray:
    """Rotate pairs (i, i + d/2) of the first rope_dim dims by angle position*theta^(-2i/d)."""
    x = np.asarray(x, dtype=np.float64)
    out = x.copy()
    half = rope_dim // 2
    for i in range(half):
        a = position * theta ** (-(2.0 * i) / rope_dim)
        c, s = math.cos(a), math.sin(a)
        x1, x2 = x[..., i], x[..., i + half]
        out[..., i] = x1 * c - x2 * s
        out[..., i + half] = x2 * c + x1 * s
    return out


def l2norm(x: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    return x / np.sqrt((x * x).sum(axis=-1, keepdims=True) + eps)


def conv_step(prev3: np.ndarray, x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """SiLU(w[c,0] x_{t-3} + w[c,1] x_{t-2} + w[c,2] x_{t-1} + w[c,3] x_t) per channel.

    prev3 [C, 3] holds x_{t-3}, x_{t-2}, x_{t-1}; x [C]; w [C, 4].
    """
    acc = np.zeros(x.shape[0], dtype=np.float64)
    for c in range(x.shape[0]):
        hist = [prev3[c, 0], prev3[c, 1], prev3[c, 2], x[c]]
        acc[c] = sum(float(w[c, j]) * float(hist[j]) for j in range(4))
    return acc / (1.0 + np.exp(-acc))


def delta_step(S: np.ndarray, q: np.ndarray, k: np.ndarray, v: np.ndarray, beta: float, g: float):
    """One gated delta-rule step for one head, element by element.

    S [dk, dv]; q, k already normalised (q scaled).  Returns (o [dv], S_new).
        S' = exp(g) S ; r_j = sum_i S'[i,j] k_i ; d_j = beta (v_j - r_j)
        S_new[i,j] = S'[i,j] + k_i d_j ; o_j = sum_i S_new[i,j] q_i
    """
    dk, dv = S.shape
    Sp = np.exp(g) * S.astype(np.float64)
    r = np.zeros(dv)
    for j in range(dv):
        for i in range(dk):
            r[j] += Sp[i, j] * k[i]
    d = beta * (v - r)
    Sn = Sp.copy()
    for i in range(dk):
        for j in range(dv):
            Sn[i, j] += k[i] * d[j]
    o = np.zeros(dv)
    for j in range(dv):
        for i in range(dk):
            o[j] += Sn[i, j] * q[i]
    return o, Sn


def attention(q: np.ndarray, K: np.ndarray, V: np.ndarray, scale: float) -> np.ndarray:
    """softmax(q K^T * scale) V for one head: q [d], K, V [T, d]."""
    s = np.array([scale * float(np.dot(q, K[t])) for t in range(K.shape[0])], dtype=np.float64)
    m = s.max()
    p = np.exp(s - m)
    p /= p.sum()
    return (p[:, None] * V.astype(np.float64)).sum(axis=0)


def sigmoid(x: np.ndarray) -> np.ndarray:
    return 1.0 / (1.0 + np.exp(-np.asarray(x, dtype=np.float64)))


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """Per row of n elements: y_d = x_d / sqrt(sum_e x_e^2 / n + eps) * (1 + w_d)."""
    x = np.asarray(x, dtype=np.float64)
    flat = x.reshape(-1, x.shape[-1])
    out = np.empty_like(flat)
    n = flat.shape[1]
    for r in range(flat.shape[0]):
        ms = sum(float(v) * float(v) for v in flat[r]) / n
        scale = 1.0 / math.sqrt(ms + eps)
        for d in range(n):
            out[r, d] = flat[r, d] * scale * (1.0 + float(w[d]))
    return out.reshape(x.shape)


def gated_rmsnorm(x: np.ndarray, z: np.ndarray, w: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """Per row of n elements: y_d = w_d * x_d / sqrt(sum_e x_e^2 / n + eps) * z_d / (1 + exp(-z_d))."""
    x = np.asarray(x, dtype=np.float64)
    zf = np.asarray(z, dtype=np.float64).reshape(-1, x.shape[-1])
    flat = x.reshape(-1, x.shape[-1])
    out = np.empty_like(flat)
    n = flat.shape[1]
    for r in range(flat.shape[0]):
        ms = sum(float(v) * float(v) for v in flat[r]) / n
        scale = 1.0 / math.sqrt(ms + eps)
        for d in range(n):
            zd = zf[r, d]
            out[r, d] = float(w[d]) * flat[r, d] * scale * zd / (1.0 + math.exp(-zd))
    return out.reshape(x.shape)


def e4m3fn_value(byte: int) -> float:
    """OCP float8 e4m3fn: sign, 4 exponent bits (bias 7), 3 mantissa bits; subnormals; NaN at S.1111.111; no inf."""
    sign = -1.0 if byte & 0x80 else 1.0
    e, m = (byte >> 3) & 0xF, byte & 0x7
    if e == 0xF and m == 0x7:
        return math.nan
    if e == 0:
        return sign * (m / 8.0) * 2.0 ** -6
    return sign * (1.0 + m / 8.0) * 2.0 ** (e - 7)


def dequant_fp8(w_bytes: np.ndarray, scale: np.ndarray, block: int = 128) -> np.ndarray:
    """w[r][c] * scale[r // block][c // block], element by element in float64."""
    rows, cols = w_bytes.shape
    out = np.empty((rows, cols), dtype=np.float64)
    for r in range(rows):
        for c in range(cols):
            out[r, c] = e4m3fn_value(int(w_bytes[r, c])) * float(scale[r // block, c // block])
    return out
