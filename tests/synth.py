"""Deterministic synthetic sampler inputs for the tests.

Only integer hashing and IEEE float32/float64 +, -, *, / are used (no libm
transcendental), so the same seed gives the same bits on every x86-64 host and
numpy build.  The shapes follow the workloads the sampler is measured on:
Gaussian rows with outliers (Qwen2.5-7B single stream), Gaussian rows with a
per-row offset (GPT-2 batched), Zipf-shaped rows over a per-row permutation
(Qwen2.5-7B batched top-k/top-p) and sparse allow masks with a shared bias
(constrained decoding).
"""
import numpy as np

_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_GOLD = np.uint64(0x9E3779B97F4A7C15)


def splitmix(x):
    """splitmix64 finaliser on a uint64 array (wrapping arithmetic)."""
    with np.errstate(over="ignore"):
        z = (x + _GOLD).astype(np.uint64)
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def hashes(seed, stream, n):
    with np.errstate(over="ignore"):
        base = np.uint64((seed * 0x100000001B3 + stream * 0x9E3779B1) & 0xFFFFFFFFFFFFFFFF)
        return splitmix(np.arange(n, dtype=np.uint64) + splitmix(np.array([base], np.uint64))[0])


def uniform(seed, stream, n):
    """float32 in [0, 1) with 24 random bits."""
    h = hashes(seed, stream, n)
    return ((h >> np.uint64(40)).astype(np.float32) * np.float32(2.0 ** -24)).astype(np.float32)


def normal(seed, stream, n):
    """Irwin-Hall(4) scaled to unit variance: symmetric, bell-shaped, bounded."""
    s = (uniform(seed, stream, n) + uniform(seed, stream + 1, n)
         + uniform(seed, stream + 2, n) + uniform(seed, stream + 3, n))
    return ((s - np.float32(2.0)) * np.float32(1.7320508)).astype(np.float32)


def ints(seed, stream, n, lo, hi):
    h = hashes(seed, stream, n)
    return ((h % np.uint64(hi - lo)).astype(np.int64) + lo).astype(np.int32)


def ln_approx(r):
    """Natural log of positive float64 values using only frexp and +,-,*,/
    (atanh series on the mantissa); accurate to ~1e-12, deterministic."""
    m, e = np.frexp(np.asarray(r, dtype=np.float64))  # r = m * 2**e, m in [0.5,1)
    m = m * 2.0
    e = e - 1
    t = (m - 1.0) / (m + 1.0)
    t2 = t * t
    s = np.zeros_like(t)
    for k in range(19, 0, -2):
        s = s * t2 + 1.0 / k
    return 2.0 * t * s + e * 0.6931471805599453


def gaussian_rows(seed, B, V, sigma, offset_range=0.0, outliers=0, outlier_value=12.0):
    x = np.empty((B, V), np.float32)
    for b in range(B):
        row = normal(seed + 7919 * b, 0, V) * np.float32(sigma)
        if offset_range:
            off = (uniform(seed + 7919 * b, 10, 1)[0] * np.float32(2.0) - np.float32(1.0)) * np.float32(offset_range)
            row = (row + off).astype(np.float32)
        if outliers:
            idx = ints(seed + 7919 * b, 20, outliers, 0, V)
            row[idx] = np.float32(outlier_value)
        x[b] = row
    return x


def zipf_rows(seed, B, V, slope=1.1, noise=0.3):
    x = np.empty((B, V), np.float32)
    lnr = ln_approx(np.arange(1, V + 1, dtype=np.float64))
    for b in range(B):
        perm = np.argsort(hashes(seed + 104729 * b, 30, V), kind="stable")
        base = (-slope * lnr[perm]).astype(np.float32)
        x[b] = (base + normal(seed + 104729 * b, 40, V) * np.float32(noise)).astype(np.float32)
    return x


def history(seed, B, n, V, with_invalid=False):
    h = ints(seed, 50, B * n, 0, V).reshape(B, n)
    if with_invalid and n >= 4:
        h[:, 1] = -1
        h[:, 3] = V + 5
    return h


def allow_bits(seed, B, V, p_allow):
    words = (V + 31) // 32
    u = uniform(seed, 60, B * words * 32).reshape(B, words * 32)
    bits = (u < np.float32(p_allow))
    bits[:, V:] = False
    packed = np.zeros((B, words), np.uint32)
    for j in range(32):
        packed |= bits[:, j::32].astype(np.uint32) << np.uint32(j)
    return packed


def sparse_bias(seed, V, nnz, sigma):
    b = np.zeros(V, np.float32)
    idx = np.argsort(hashes(seed, 70, V), kind="stable")[:nnz]
    b[idx] = normal(seed, 80, nnz) * np.float32(sigma)
    return b


def digest(a):
    """64-bit hash of the raw bytes (position-mixed splitmix words), used to
    check that regenerated fixture inputs are bit-identical."""
    data = np.ascontiguousarray(a).reshape(-1).view(np.uint8)
    pad = (-len(data)) % 8
    if pad:
        data = np.concatenate([data, np.zeros(pad, np.uint8)])
    words = data.view(np.uint64)
    with np.errstate(over="ignore"):
        chunk = splitmix(words ^ splitmix(np.arange(len(words), dtype=np.uint64)))
        acc = np.bitwise_xor.reduce(chunk) ^ np.uint64(len(words))
        return int(splitmix(np.array([acc], np.uint64))[0])


def make_row(kind, seed, V):
    """One float32 row of a named shape (used by the golden fixtures)."""
    if kind == "gauss":
        return gaussian_rows(seed, 1, V, 2.5)[0]
    if kind == "outliers":  # N(0, 2.5^2) + 8 tokens at exactly +12
        return gaussian_rows(seed, 1, V, 2.5, outliers=min(8, V))[0]
    if kind == "gauss_offset":
        return gaussian_rows(seed, 1, V, 3.0, offset_range=5.0)[0]
    if kind == "zipf":
        return zipf_rows(seed, 1, V)[0]
    if kind == "ties":  # values on a 0.5 grid: many exact ties at the threshold
        g = normal(seed, 0, V) * np.float32(2.0)
        return (np.floor(g) * np.float32(0.5)).astype(np.float32)
    if kind == "const":
        return np.full(V, np.float32(0.25), np.float32)
    if kind == "neginf":  # mostly -inf, a few finite values
        x = normal(seed, 0, V) * np.float32(2.5)
        keep = uniform(seed, 90, V) < np.float32(0.03)
        x[~keep] = -np.inf
        return x.astype(np.float32)
    if kind == "allneginf":
        return np.full(V, -np.inf, np.float32)
    if kind == "ascending":
        return np.sort(normal(seed, 0, V) * np.float32(2.5)).astype(np.float32)
    if kind == "descending":
        return np.sort(normal(seed, 0, V) * np.float32(2.5))[::-1].astype(np.float32).copy()
    if kind == "signed_zero":  # +-0 and small values around the threshold
        x = np.floor(normal(seed, 0, V)).astype(np.float32) * np.float32(0.0)
        x[::3] = -0.0
        x[::7] = np.float32(1.0)
        return x.astype(np.float32)
    if kind == "huge":  # magnitudes near the fp32 range
        return (normal(seed, 0, V) * np.float32(1e37)).astype(np.float32)
    # Rows a diverging model produces.  A nan compares false with everything,
    # so where it sits decides what the reference's heap and argmax do.
    qnan, neg_qnan = _bits_f32(0x7FC00000), _bits_f32(0xFFC00000)
    if kind == "nan_first":  # id 0 is nan: the greedy scan keeps id 0
        x = normal(seed, 0, V) * np.float32(2.5)
        x[0] = qnan
        return x.astype(np.float32)
    if kind == "nan_early":  # nans among the first ids: they enter the heap while it fills
        x = normal(seed, 0, V) * np.float32(2.5)
        x[1:12:3] = qnan
        x[2:12:5] = neg_qnan
        return x.astype(np.float32)
    if kind == "nan_late":  # one nan after the heap has filled, next to the largest values
        x = normal(seed, 0, V) * np.float32(2.5)
        if V > 1:
            x[V // 2] = qnan
            x[min(V - 1, V // 2 + 1)] = np.float32(9.0)
        return x.astype(np.float32)
    if kind == "nan_sparse":  # ~2 % nans of both signs, spread over the row
        x = normal(seed, 0, V) * np.float32(2.5)
        u = uniform(seed, 91, V)
        x[u < np.float32(0.01)] = qnan
        x[(u >= np.float32(0.01)) & (u < np.float32(0.02))] = neg_qnan
        return x.astype(np.float32)
    if kind == "nan_all":
        return np.full(V, qnan, np.float32)
    if kind == "inf_mix":  # a few +inf (ties at the top) and -inf
        x = normal(seed, 0, V) * np.float32(2.5)
        u = uniform(seed, 92, V)
        x[u < np.float32(0.002)] = np.inf
        x[(u >= np.float32(0.002)) & (u < np.float32(0.05))] = -np.inf
        return x.astype(np.float32)
    if kind == "nan_inf":  # nan, +inf and -inf together
        x = make_row("inf_mix", seed, V)
        x[uniform(seed, 93, V) < np.float32(0.01)] = qnan
        return x.astype(np.float32)
    raise ValueError(kind)


def quantize_special_rows():
    """Activation rows with nans and infinities at the places the AVX2 build
    treats differently: a lane's last 8-chunk (its nan survives the lane
    maximum), earlier chunks (it does not), the scalar tail, and rows made of
    them."""
    rows = []
    qnan, inf = np.float32(np.nan), np.float32(np.inf)
    for n in (7, 8, 37, 256, 3584):
        base = (normal(8100 + n, 0, n) * np.float32(3.0)).astype(np.float32)
        n8 = n & ~7
        places = {0, n // 2, n - 1}
        if n8:
            places |= {n8 - 1, n8 - 8, max(0, n8 - 9)}
        for pos in sorted(places):
            for val in (qnan, -qnan, inf, -inf):
                x = base.copy()
                x[pos] = val
                rows.append(x)
        x = base.copy()
        x[::5] = qnan
        rows.append(x)
        rows.append(np.full(n, qnan, np.float32))
        rows.append(np.full(n, inf, np.float32))
        x = base.copy()
        x[n // 3] = inf
        x[n - 1] = qnan
        rows.append(x)
    return rows


def _bits_f32(bits):
    return np.array([bits], np.uint32).view(np.float32)[0]
