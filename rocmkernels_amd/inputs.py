"""Seeded synthetic inputs for tests and benchmarks.

Two generators:

* ``normal(seed, shape)``: iid N(0, 1) float32 from a counter-based splitmix64 stream and the Box-Muller
  transform in double precision. Portable and vectorised; used for the benchmark configurations
  (seeds Q 101, K 102, V 103, dO 104, lengths 105).
* ``reference_uniform(seed, count)``: the values the reference's tests draw on Linux with libstdc++,
  ``std::mt19937(seed)`` feeding ``std::uniform_real_distribution<float>(-1, 1)``
  (ROCmKernels.Tests/TestSupport.hpp:11-21). libstdc++'s generate_canonical<float, 24> uses one 32-bit draw:
  u = float(x) / 2^32 (clamped below 1), value = u * 2 - 1 in float. MSVC's distribution differs, so these are
  the reference test inputs as a Linux build of the reference would see them.
"""
import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_MIX1 = np.uint64(0xBF58476D1CE4E5B9)
_MIX2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed, count, offset=0):
    """Outputs offset+1 .. offset+count of splitmix64 seeded with ``seed`` (state advances by the golden gamma)."""
    index = np.arange(offset + 1, offset + count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + index * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _MIX1
        z = (z ^ (z >> np.uint64(27))) * _MIX2
    return z ^ (z >> np.uint64(31))


def _unit(bits):
    """53-bit uniform double in [0, 1)."""
    return (bits >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def normal(seed, shape):
    """iid N(0,1) float32 array of ``shape``: element 2i is r*cos(2*pi*u2), 2i+1 is r*sin(2*pi*u2) of pair i."""
    count = int(np.prod(shape))
    pairs = (count + 1) // 2
    bits = splitmix64(seed, 2 * pairs)
    u1 = _unit(bits[0::2]) + (1.0 / 9007199254740992.0)  # (0, 1]: log stays finite
    u2 = _unit(bits[1::2])
    radius = np.sqrt(-2.0 * np.log(u1))
    angle = 2.0 * np.pi * u2
    values = np.empty(2 * pairs, dtype=np.float64)
    values[0::2] = radius * np.cos(angle)
    values[1::2] = radius * np.sin(angle)
    return values[:count].astype(np.float32).reshape(shape)


def uniform_int(seed, count, low, high):
    """``count`` integers uniform in [low, high] (inclusive)."""
    u = _unit(splitmix64(seed, count))
    return (low + np.floor(u * (high - low + 1))).astype(np.int64)


class MT19937:
    """std::mt19937 (32-bit Mersenne Twister, init_genrand seeding)."""

    def __init__(self, seed):
        state = [seed & 0xFFFFFFFF]
        for i in range(1, 624):
            previous = state[-1]
            state.append((1812433253 * (previous ^ (previous >> 30)) + i) & 0xFFFFFFFF)
        self._state = state
        self._index = 624

    def _twist(self):
        s = self._state
        for i in range(624):
            y = (s[i] & 0x80000000) | (s[(i + 1) % 624] & 0x7FFFFFFF)
            s[i] = s[(i + 397) % 624] ^ (y >> 1) ^ (0x9908B0DF if y & 1 else 0)
        self._index = 0

    def __call__(self):
        if self._index >= 624:
            self._twist()
        y = self._state[self._index]
        self._index += 1
        y ^= y >> 11
        y ^= (y << 7) & 0x9D2C5680
        y ^= (y << 15) & 0xEFC60000
        y ^= y >> 18
        return y


def reference_uniform(seed, count, low=-1.0, high=1.0):
    """``count`` float32 values of libstdc++ uniform_real_distribution<float>(low, high) over std::mt19937(seed)."""
    generator = MT19937(seed)
    raw = np.array([generator() for _ in range(count)], dtype=np.uint64)
    u = raw.astype(np.float32) / np.float32(4294967296.0)
    u = np.where(u >= np.float32(1.0), np.nextafter(np.float32(1.0), np.float32(0.0)), u).astype(np.float32)
    return (u * (np.float32(high) - np.float32(low)) + np.float32(low)).astype(np.float32)
