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
