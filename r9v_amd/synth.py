"""Seeded synthetic inputs for the quantized-weight path (bench and tests).

The stream is SplitMix64 (crates/r9v-common/src/rng.rs:79-85) used in counter
mode: value i of the stream seeded by `seed` is mix(seed + (i + 1) * GAMMA),
which equals the i-th SplitMix64 output and vectorises in numpy.  Gaussians
are Box-Muller in f64 from two 53-bit uniforms, rounded once to the target
dtype.  Per-config seeds are xxh3_64("r9vx|<config>|<case>").

Weight blocks follow the GGUF wire formats.  Every bit of a Q4_K block other
than d/dmin, and every bit of an IQ4_XS block other than d, belongs to exactly
one uniformly distributed field (4-bit quants, 6-bit sub-scales/mins), so those
bytes are uniform random bytes; d (and dmin) are f16(|N(0, sigma)|).
"""
from __future__ import annotations

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)

# weight schemes by their SchemeId codes (as r9v_amd.ffi)
Q4_K = 3
IQ4_XS = 15
Q6_K = 11
Q8_0 = 5
IQ3_S = 17
BLOCK_BYTES = {Q4_K: 144, IQ4_XS: 136, Q6_K: 210, Q8_0: 34, IQ3_S: 110}
BLOCK_LEN = {Q4_K: 256, IQ4_XS: 256, Q6_K: 256, Q8_0: 32, IQ3_S: 256}
D_OFFSET = {Q4_K: 0, IQ4_XS: 0, Q6_K: 208, Q8_0: 0, IQ3_S: 0}  # byte offset of each block's f16 d


def seed_for(config: str, case: str = "") -> int:
    import xxhash

    return xxhash.xxh3_64_intdigest(f"r9vx|{config}|{case}".encode())


def splitmix64(seed: int, n: int, start: int = 0) -> np.ndarray:
    """Values start..start+n-1 of the SplitMix64 stream seeded by `seed`."""
    with np.errstate(over="ignore"):
        i = np.arange(start + 1, start + n + 1, dtype=np.uint64)
        z = np.uint64(seed) + i * GAMMA
        z = (z ^ (z >> np.uint64(30))) * M1
        z = (z ^ (z >> np.uint64(27))) * M2
        return z ^ (z >> np.uint64(31))


def random_bytes(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint8)
    chunk = 1 << 24  # u64 words per chunk
    words = (n + 7) // 8
    for w0 in range(0, words, chunk):
        w1 = min(words, w0 + chunk)
        b = splitmix64(seed, w1 - w0, start=w0).view(np.uint8)
        lo, hi = w0 * 8, min(n, w1 * 8)
        out[lo:hi] = b[: hi - lo]
    return out


def uniform01(seed: int, n: int, start: int = 0) -> np.ndarray:
    return (splitmix64(seed, n, start) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))


def normal(seed: int, n: int, sigma: float = 1.0, mean: float = 0.0) -> np.ndarray:
    """f64 N(mean, sigma^2), Box-Muller over consecutive uniform pairs."""
    m = (n + 1) // 2
    u = uniform01(seed, 2 * m)
    u1 = 1.0 - u[0::2]  # (0, 1]
    u2 = u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * m, dtype=np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return z[:n] * sigma + mean


def to_bf16_bits(v: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bits, round-to-nearest-even (crates/r9v-t0/src/dtype.rs:102-111)."""
    f = np.ascontiguousarray(v, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    lsb = (u >> np.uint64(16)) & np.uint64(1)
    r = ((u + np.uint64(0x7FFF) + lsb) >> np.uint64(16)).astype(np.uint16)
    nan = np.isnan(f)
    if nan.any():
        r[nan] = ((u[nan] >> np.uint64(16)) | np.uint64(0x40)).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def normal_bf16(seed: int, shape, sigma: float = 1.0) -> np.ndarray:
    """bf16 bits (uint16) of N(0, sigma^2): f64 -> f32 -> bf16 RNE."""
    n = int(np.prod(shape))
    return to_bf16_bits(normal(seed, n, sigma).astype(np.float32)).reshape(shape)


def normal_f32(seed: int, shape, sigma: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    return normal(seed, n, sigma).astype(np.float32).reshape(shape)


def half_normal_f16_bits(seed: int, n: int, sigma: float) -> np.ndarray:
    return np.abs(normal(seed, n, sigma)).astype(np.float16).view(np.uint16)


def quant_weights(scheme: int, seed: int, rows: int, k: int) -> np.ndarray:
    """GGUF wire blocks for a [rows, k] weight: uint8 [rows, k/block_len*block_bytes].
    Every byte is seeded-random except each block's f16 d (and Q4_K's dmin),
    which is |N(0, 0.02)| (|N(0, 0.01)| for dmin)."""
    bl, bb = BLOCK_LEN[scheme], BLOCK_BYTES[scheme]
    if k % bl:
        raise ValueError(f"k must be a multiple of {bl}")
    nblocks = rows * (k // bl)
    blk = random_bytes(seed, nblocks * bb).reshape(nblocks, bb)
    d = half_normal_f16_bits(seed ^ 0xD1D1D1D1D1D1D1D1, nblocks, 0.02)
    o = D_OFFSET[scheme]
    blk[:, o:o + 2] = d.view(np.uint8).reshape(nblocks, 2)
    if scheme == Q4_K:
        dmin = half_normal_f16_bits(seed ^ 0x3C3C3C3C3C3C3C3C, nblocks, 0.01)
        blk[:, 2:4] = dmin.view(np.uint8).reshape(nblocks, 2)
    return blk.reshape(rows, (k // bl) * bb)


def zipf_logits(seed: int, t: int, e: int, s: float = 1.1) -> np.ndarray:
    """Router logits N(0,1) + ln p_rank(e), p_r ~ (r+1)^-s over a seeded expert
    permutation (Zipf-skewed popularity), f32 [t, e]."""
    perm_keys = splitmix64(seed ^ 0x5EED5EED, e)
    rank = np.empty(e, dtype=np.int64)
    rank[np.argsort(perm_keys, kind="stable")] = np.arange(e)
    p = (rank + 1.0) ** (-s)
    p = p / p.sum()
    base = normal(seed, t * e).reshape(t, e)
    return (base + np.log(p)[None, :]).astype(np.float32)
