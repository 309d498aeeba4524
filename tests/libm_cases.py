"""Inputs and checksums of the math-routine checks (the glibc 2.39 routines the step calls).

* The unary float routines (sinf, cosf, atanf, acosf, asinf) are checked exhaustively: all 2**32
  bit patterns, in 256 blocks of 2**24 consecutive patterns. A block's digest is SHA-256 over its
  outputs; the routine's checksum is SHA-256 over the 256 block digests in order.
* The others are checked on fixed samples: powf and atan2f on pairs, sincosf on floats, and the
  double routines sin, cos, pow, acos and sincos. A sample holds a grid of special values (zeros of
  both signs, infinities, NaN, subnormals, the extremes, values next to 1, integers and
  half-integers), one random pair for every combination of the two exponents (floats) or 64
  random mantissas for every exponent (doubles), uniformly random bit patterns, and uniform draws
  from the ranges the step feeds them. Its checksum is SHA-256 over the outputs.

Outputs are hashed as little-endian bits with every NaN made the default quiet NaN: the routines
keep a NaN's class, not its payload or sign, which the device makes canonical. Samples come from
SplitMix64 over the sample index, so every machine builds the same inputs.
"""

from __future__ import annotations

import concurrent.futures
import hashlib

import numpy as np

UNARY_FLOAT = {'sinf': 0, 'cosf': 1, 'atanf': 4, 'acosf': 5, 'asinf': 6}
SAMPLED_FLOAT = {'powf': 2, 'atan2f': 3, 'sincosf_sin': 7, 'sincosf_cos': 8}
SAMPLED_DOUBLE = {'sin': 0, 'cos': 1, 'pow': 2, 'acos': 3, 'sincos_sin': 4, 'sincos_cos': 5}
BLOCK = 1 << 24
BLOCKS = 256


def _splitmix(index, stream):
    with np.errstate(over='ignore'):
        x = np.asarray(index, dtype=np.uint64) + np.uint64(stream) * np.uint64(0x9E3779B97F4A7C15)
        x = x * np.uint64(0xD1B54A32D192ED03) + np.uint64(0x632BE59BD9B4E019)
        x ^= x >> np.uint64(30)
        x *= np.uint64(0xBF58476D1CE4E5B9)
        x ^= x >> np.uint64(27)
        x *= np.uint64(0x94D049BB133111EB)
        x ^= x >> np.uint64(31)
    return x


def _uniform(n, stream, low, high, dtype):
    u = (_splitmix(np.arange(n), stream) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))
    return (low + (high - low) * u).astype(dtype)


FLOAT_SPECIALS = np.array(
    [0.0, -0.0, 1.0, -1.0, 0.5, -0.5, 2.0, -2.0, 3.0, -3.0, 1.5, -1.5, np.inf, -np.inf, np.nan,
     np.float32(1.4e-45), -np.float32(1.4e-45), np.float32(1.1754942e-38), np.float32(1.17549435e-38),
     np.finfo(np.float32).max, -np.finfo(np.float32).max, np.nextafter(np.float32(1), np.float32(2)),
     np.nextafter(np.float32(1), np.float32(0)), 1e-20, 1e20, 100.5, -100.5, 3.1415927, -3.1415927, 1.5707964,
     1e5, 1e9, 126.0, -149.0, 128.0, 0.70710677], dtype=np.float32)
DOUBLE_SPECIALS = np.array(
    [0.0, -0.0, 1.0, -1.0, 0.5, -0.5, 2.0, -2.0, 3.0, -3.0, 1.5, -1.5, np.inf, -np.inf, np.nan, 5e-324, -5e-324,
     2.2250738585072009e-308, 2.2250738585072014e-308, np.finfo(np.float64).max, -np.finfo(np.float64).max,
     np.nextafter(1.0, 2.0), np.nextafter(1.0, 0.0), 1e-20, 1e20, 100.5, -100.5, np.pi, -np.pi, np.pi / 2,
     105414350.0, 2.0 ** 27, 1e22, 1e300, 1023.0, -1074.0, 1024.0, 0.7071067811865476, 0.99999999, -0.99999999],
    dtype=np.float64)


def float_pairs(name):
    """The (x, y) float32 sample of a sampled float routine (y is unused by the unary ones)."""
    grid_x, grid_y = np.meshgrid(FLOAT_SPECIALS, FLOAT_SPECIALS, indexing='ij')
    e = np.arange(256, dtype=np.uint64)
    ex, ey = np.meshgrid(e, e, indexing='ij')
    m = _splitmix(np.arange(ex.size), 1)
    bx = ((m & np.uint64(0x807FFFFF)) | (ex.reshape(-1) << np.uint64(23))).astype(np.uint32)
    by = (((m >> np.uint64(32)) & np.uint64(0x807FFFFF)) | (ey.reshape(-1) << np.uint64(23))).astype(np.uint32)
    n = 1 << 20
    rx = (_splitmix(np.arange(n), 2) >> np.uint64(32)).astype(np.uint32)
    ry = (_splitmix(np.arange(n), 3) >> np.uint64(32)).astype(np.uint32)
    if name == 'powf':
        ux, uy = _uniform(n, 4, 0.0, 64.0, np.float32), _uniform(n, 5, -8.0, 8.0, np.float32)
    elif name == 'atan2f':
        ux, uy = _uniform(n, 4, -100.0, 100.0, np.float32), _uniform(n, 5, -100.0, 100.0, np.float32)
    else:
        ux, uy = _uniform(n, 4, -40.0, 40.0, np.float32), np.zeros(n, np.float32)
    x = np.concatenate([grid_x.reshape(-1), bx.view(np.float32), rx.view(np.float32), ux])
    y = np.concatenate([grid_y.reshape(-1), by.view(np.float32), ry.view(np.float32), uy])
    return np.ascontiguousarray(x, dtype=np.float32), np.ascontiguousarray(y, dtype=np.float32)


def double_pairs(name):
    """The (x, y) float64 sample of a double routine (y is unused by the unary ones)."""
    grid_x, grid_y = np.meshgrid(DOUBLE_SPECIALS, DOUBLE_SPECIALS, indexing='ij')
    e = np.repeat(np.arange(2048, dtype=np.uint64), 64)
    m = _splitmix(np.arange(e.size), 11)
    bx = ((m & np.uint64(0x800FFFFFFFFFFFFF)) | (e << np.uint64(52))).view(np.float64)
    by = ((_splitmix(np.arange(e.size), 12) & np.uint64(0x800FFFFFFFFFFFFF)) |
          (np.roll(e, 777) << np.uint64(52))).view(np.float64)
    n = 1 << 19
    rx = _splitmix(np.arange(n), 13).view(np.float64)
    ry = _splitmix(np.arange(n), 14).view(np.float64)
    if name == 'pow':
        ux, uy = _uniform(n, 15, 0.0, 100.0, np.float64), _uniform(n, 16, -10.0, 10.0, np.float64)
    elif name == 'acos':
        ux, uy = _uniform(n, 15, -1.0, 1.0, np.float64), np.zeros(n)
    else:
        ux = np.concatenate([_uniform(n // 2, 15, -10.0, 10.0, np.float64),
                             _uniform(n - n // 2, 16, 1e5, 1e12, np.float64)])
        uy = np.zeros(n)
    x = np.concatenate([grid_x.reshape(-1), bx, rx, ux])
    y = np.concatenate([grid_y.reshape(-1), by, ry, uy])
    return np.ascontiguousarray(x, dtype=np.float64), np.ascontiguousarray(y, dtype=np.float64)


def canonical(out):
    """Outputs with every NaN made the default quiet NaN, as bytes."""
    out = np.array(out, copy=True)
    nan = np.isnan(out)
    bits = out.view(np.uint32 if out.dtype == np.float32 else np.uint64)
    bits[nan] = 0x7FC00000 if out.dtype == np.float32 else 0x7FF8000000000000
    return bits.tobytes()


def sample_digest(out):
    return hashlib.sha256(canonical(out)).hexdigest()


def exhaustive_digest(fill, threads=8):
    """The checksum of a unary float routine over all 2**32 inputs. `fill(first, out)` writes the
    outputs of the len(out) consecutive patterns from `first` into the float32 array `out`; it
    must release the GIL (ctypes calls do) so that blocks run in parallel."""
    def block(b):
        out = np.empty(BLOCK, dtype=np.float32)
        fill(b * BLOCK, out)
        return hashlib.sha256(canonical(out)).digest()

    with concurrent.futures.ThreadPoolExecutor(max_workers=threads) as pool:
        digests = list(pool.map(block, range(BLOCKS)))
    return hashlib.sha256(b''.join(digests)).hexdigest()


def block_digests_to_checksum(digests):
    return hashlib.sha256(b''.join(digests)).hexdigest()
