"""Seeded synthetic inputs shared by the tests (numpy PCG64 streams)."""
import numpy as np


def weights(n, k, seed, std=0.02):
    """N(0, std) float32 weights [n, k]."""
    return np.random.default_rng(seed).standard_normal((n, k), dtype=np.float32) * np.float32(std)


def activations(m, k, seed, outlier_frac=0.001, outlier=20.0):
    """N(0,1) float32 activations [m, k]; ceil(frac*k) distinct positions per row set to +-outlier."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k), dtype=np.float32)
    if outlier_frac and k:
        cnt = int(np.ceil(outlier_frac * k))
        for i in range(m):
            pos = rng.choice(k, size=cnt, replace=False)
            x[i, pos] = np.where(rng.random(cnt) < 0.5, -outlier, outlier).astype(np.float32)
    return x


def random_codes(n, k, seed, p_zero=0.31, p3=0.0):
    """Packed bytes with i.i.d. codes: 0 w.p. p_zero, 3 w.p. p3, else +1/-1."""
    rng = np.random.default_rng(seed)
    u = rng.random(n * k)
    codes = np.where(u < p_zero, 0, np.where(u < p_zero + p3, 3, np.where(rng.random(n * k) < 0.5, 1, 2)))
    return pack_codes(codes.astype(np.uint8))


def pack_codes(codes):
    """Flat 2-bit codes -> packed bytes (element e in byte e//4 at bits 2*(e%4))."""
    codes = np.asarray(codes, np.uint8).reshape(-1)
    pad = (-codes.size) % 4
    c = np.concatenate([codes, np.zeros(pad, np.uint8)]).reshape(-1, 4)
    return (c[:, 0] | (c[:, 1] << 2) | (c[:, 2] << 4) | (c[:, 3] << 6)).astype(np.uint8)


def ternary(data, numel):
    """Packed bytes -> int8 ternary values t = (c&1) - (c>>1), by numpy bit ops."""
    b = np.asarray(data, np.uint8)
    codes = np.stack([(b >> (2 * i)) & 3 for i in range(4)], axis=1).reshape(-1)[:numel]
    return ((codes & 1).astype(np.int8) - (codes >> 1).astype(np.int8)).astype(np.int8)


def rvq_bases(w, nb):
    """The reference converter's residual ternary decomposition (quantize_adaptive_basis,
    tools/conversion/convert_llama_v2.py:28-72), restated in numpy to produce test
    weights of the multi-base format: scale = mean|R| (1.0 below 1e-9), t =
    clamp(round_half_even(R / scale), -1, 1), R -= t * scale.  -> (t [nb, n, k] int8,
    scales [nb] float32)."""
    r = np.asarray(w, np.float32).copy()
    ts, ss = [], []
    for _ in range(nb):
        s = np.float32(np.abs(r, dtype=np.float32).mean(dtype=np.float64))
        if s < 1e-9:
            s = np.float32(1.0)
        t = np.clip(np.round(r / s), -1, 1).astype(np.int8)
        r = (r - t.astype(np.float32) * s).astype(np.float32)
        ts.append(t)
        ss.append(s)
    return np.stack(ts), np.array(ss, np.float32)


def pack_interleaved_2bit(t):
    """pack_2bit (convert_llama_v2.py:111-151): ternary [nb, n, k] -> [n, k/4, nb] bytes,
    codes (v + 3) % 3 (-1 -> 2), column 4c + j at bits 2j."""
    nb, n, k = t.shape
    codes = ((t.astype(np.int16) + 3) % 3).astype(np.uint8)       # [nb, n, k]
    c = codes.transpose(1, 2, 0).reshape(n, k // 4, 4, nb)          # [n, k/4, 4, nb]
    return np.ascontiguousarray(c[:, :, 0] | (c[:, :, 1] << 2) | (c[:, :, 2] << 4) | (c[:, :, 3] << 6), np.uint8)
