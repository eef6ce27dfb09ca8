"""float64 closed forms of the path's ops (for the checks that pin the oracle
and for long-row comparisons)."""
import numpy as np


def layernorm(x, n, gamma=None, beta=None, eps=1e-5):
    x = np.asarray(x, np.float64).reshape(-1, n)
    m = x.mean(axis=1, keepdims=True)
    y = (x - m) / np.sqrt(((x - m) ** 2).mean(axis=1, keepdims=True) + eps)
    if gamma is not None:
        y = y * np.asarray(gamma, np.float64)
        if beta is not None:
            y = y + np.asarray(beta, np.float64)
    return y.ravel()


def rmsnorm(x, cols, w=None, w_len=None, eps=1e-6):
    x = np.asarray(x, np.float64).reshape(-1, cols)
    y = x / np.sqrt((x ** 2).mean(axis=1, keepdims=True) + eps)
    if w is not None:
        k = min(cols, len(w) if w_len is None else w_len)
        y[:, :k] *= np.asarray(w, np.float64)[:k]
    return y


def softmax(x, mode=0):
    x = np.asarray(x, np.float64)
    x = x.reshape(1, -1) if x.ndim == 1 else x
    with np.errstate(invalid="ignore", over="ignore"):
        m = x.max(axis=1, keepdims=True)
        e = np.exp(x - m)
        s = e.sum(axis=1, keepdims=True)
        if mode == 0:
            return e / (s + 1e-9)
        if mode == 1:
            return e / s
        return (x - m) - np.log(s)


def layernorm_bwd(x, dy, n, gamma=None, eps=1e-5):
    """float64 dL/dx, dL/dgamma, dL/dbeta of y = xhat*gamma + beta over
    groups of n (the sums over groups not yet added onto anything)."""
    x = np.asarray(x, np.float64).reshape(-1, n)
    dy = np.asarray(dy, np.float64).reshape(-1, n)
    g = 1.0 if gamma is None else np.asarray(gamma, np.float64)
    m = x.mean(axis=1, keepdims=True)
    inv = 1.0 / np.sqrt(((x - m) ** 2).mean(axis=1, keepdims=True) + eps)
    xh = (x - m) * inv
    dxh = dy * g
    s1 = dxh.mean(axis=1, keepdims=True)
    s2 = (dxh * xh).mean(axis=1, keepdims=True)
    dx = inv * (dxh - s1 - xh * s2)
    # Magnitude of the terms whose difference dx is (the reference forms
    # inv/n * (n*dxh - sum - xhat*sum2) in float32): its rounding error scales
    # with this, not with the possibly cancelled dx.
    dx_scale = inv * (np.abs(dxh) + np.abs(s1) + np.abs(xh * s2))
    return dx.ravel(), (dy * xh).sum(axis=0), dy.sum(axis=0), (np.abs(dy * xh).sum(axis=0), np.abs(dy).sum(axis=0)), \
        dx_scale.ravel()


def dgelu(x):
    k = np.sqrt(np.float64(np.float32(2.0) / np.float32(3.14159265359)))
    x = np.asarray(x, np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        t = np.tanh(k * (x + 0.044715 * x ** 3))
        return 0.5 * (1 + t) + 0.5 * x * (1 - t * t) * k * (1 + 3 * 0.044715 * x * x)


def dsilu(x):
    x = np.asarray(x, np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        s = 1 / (1 + np.exp(-x))
        return s + x * s * (1 - s)
