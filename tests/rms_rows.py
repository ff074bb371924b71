"""Rows on which the order of gemm::rms_norm's sum of squares matters.

gemm::rms_norm (src/Gemm.cpp:197-207) adds the exact double squares in element
order; the GPU kernels add them in a thread-strided tree (256 threads, thread t
adding elements t, t + 256, ... in order, a 64-lane butterfly per wave, then
(w0 + w1) + (w2 + w3)).  The two double sums can differ in their last bits, and
the float inverse 1 / sqrt(sum / n + eps) with them when it lies near a float
rounding boundary.  adversarial_rows() builds such rows for n = 2048: one large
element x0, 2046 copies of s = 2^-22 whose squares (2^-44) are each below half
an ulp of x0^2 (so the in-order sum drops every one of them, while the tree adds
them among themselves first and keeps them), and one element x1 chosen so that
a float rounding midpoint of the inverse lies between the two sums' inverses.
"""
import numpy as np

N = 2048


def tree_sum(x: np.ndarray) -> float:
    """The kernels' order (float64, IEEE, as the GPU's double adds)."""
    d = np.asarray(x, np.float32).astype(np.float64)
    sq = np.zeros(256)
    for u in range(len(d) // 256):
        sq = sq + d[u * 256:(u + 1) * 256] ** 2
    w = sq.reshape(4, 64)
    for o in (32, 16, 8, 4, 2, 1):
        w = w + w[:, np.arange(64) ^ o]
    w = w[:, 0]
    return float((w[0] + w[1]) + (w[2] + w[3]))


def seq_sum(x: np.ndarray) -> float:
    """gemm::rms_norm's order."""
    s = 0.0
    for v in np.asarray(x, np.float32).astype(np.float64):
        s = s + v * v
    return s


def inverse(total: float, n: int, eps: np.float32) -> np.float32:
    return np.float32(1.0 / np.sqrt(np.float64(total) / n + np.float64(eps)))


def adversarial_rows(count: int, eps: float = 1e-6, seed: int = 5) -> np.ndarray:
    """`count` rows of N floats whose tree and in-order inverses differ."""
    eps = np.float32(eps)
    rng = np.random.default_rng(seed)
    s = np.float32(2.0 ** -22)
    rows = []
    while len(rows) < count:
        x0 = np.float32(rng.uniform(32.5, 45.0))
        s0 = np.float64(x0) ** 2
        f = np.float32(1.0 / np.sqrt(s0 / N + np.float64(eps)))
        for nb in (np.nextafter(f, np.float32(0)), np.nextafter(f, np.float32(np.inf))):
            m = (np.longdouble(f) + np.longdouble(nb)) / 2          # a rounding boundary of the inverse
            sm = np.longdouble(N) * (1 / (m * m) - np.longdouble(eps))
            x = np.full(N, s, np.float32)
            x[0] = x0
            kept = tree_sum(x) - seq_sum(x)                        # what only the tree keeps
            need = sm - np.longdouble(s0) - np.longdouble(kept) / 2
            if need <= 0 or need > s0 / 256:
                continue
            x[1] = np.float32(np.sqrt(np.float64(need)))
            if inverse(tree_sum(x), N, eps) != inverse(seq_sum(x), N, eps):
                rows.append(x)
                break
    return np.stack(rows[:count])
