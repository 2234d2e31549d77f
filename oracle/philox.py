"""CPU oracle of the in-kernel Gaussian noise (fdp_noise_key, include/flashdp_hip.h).

TEST INFRASTRUCTURE ONLY.  Only ``tests/`` and ``__graft_entry__.smoke()`` may
import this module, as the checker of the noise the kernels draw.

The reference draws its DP noise with ``torch.normal`` / ``torch.randn``
(flashdp/layers/linear.py:74-80, flashdp/layers/layernorm.py:140-155): any
standard-normal stream is equivalent for the mechanism, so the build draws its
own inside the kernels and this module restates that stream exactly:

  philox4x32_10  Philox4x32-10 of Salmon, Moraes, Dror, Shaw, "Parallel random
                 numbers: as easy as 1, 2, 3" (SC 2011).  Pinned by the
                 published known-answer vectors of the Random123 distribution
                 (tests/test_oracle.py).
  normals        element e of output `stream`: block offset + e // 4 with
                 counter {lo, hi, stream, 0} and key {lo(seed), hi(seed)}; words
                 (w0, w1) and (w2, w3) -> two normals each by Box-Muller, the
                 radius from the 32-bit uniform (w0 + 0.5) / 2^32 (|z| <= 6.76)
                 and the angle from the 24-bit uniform ((w1 >> 8) + 0.5) / 2^24.
                 Pinned statistically (moments, tails, independence of
                 neighbouring elements and streams) in tests/test_oracle.py.
"""
from __future__ import annotations

import numpy as np

M0, M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
W0, W1 = np.uint32(0x9E3779B9), np.uint32(0xBB67AE85)
_MASK = np.uint64(0xFFFFFFFF)


def philox4x32_10(ctr, key):
    """ctr: uint32 array [..., 4]; key: uint32 array [..., 2] (broadcast) -> [..., 4]."""
    c = np.asarray(ctr, dtype=np.uint32)
    k = np.broadcast_to(np.asarray(key, dtype=np.uint32), c.shape[:-1] + (2,)).copy()
    c0, c1, c2, c3 = (c[..., i].astype(np.uint64) for i in range(4))
    k0, k1 = k[..., 0].astype(np.uint32), k[..., 1].astype(np.uint32)
    for r in range(10):
        if r > 0:
            k0 = (k0 + W0).astype(np.uint32)
            k1 = (k1 + W1).astype(np.uint32)
        p0 = M0 * c0
        p1 = M1 * c2
        hi0, lo0 = p0 >> np.uint64(32), p0 & _MASK
        hi1, lo1 = p1 >> np.uint64(32), p1 & _MASK
        c0, c1, c2, c3 = (hi1 ^ c1 ^ k0.astype(np.uint64)), lo1, (hi0 ^ c3 ^ k1.astype(np.uint64)), lo0
    return np.stack([c0, c1, c2, c3], axis=-1).astype(np.uint32)


def _uniform24(w):
    return ((w >> np.uint32(8)).astype(np.float64) + 0.5) / float(1 << 24)


def _uniform32(w):
    return (w.astype(np.float64) + 0.5) / float(1 << 32)


def normals(n: int, seed: int, offset: int = 0, stream: int = 0) -> np.ndarray:
    """The first n normals (float64) of the in-kernel draw with key (seed, offset)
    for output `stream`."""
    nblk = (n + 3) // 4
    q = np.arange(nblk, dtype=np.uint64) + np.uint64(offset)
    ctr = np.zeros((nblk, 4), dtype=np.uint32)
    ctr[:, 0] = (q & _MASK).astype(np.uint32)
    ctr[:, 1] = (q >> np.uint64(32)).astype(np.uint32)
    ctr[:, 2] = np.uint32(stream)
    seed = int(seed) & (2**64 - 1)
    key = np.array([seed & 0xFFFFFFFF, seed >> 32], dtype=np.uint32)
    w = philox4x32_10(ctr, key)
    out = np.empty((nblk, 4), dtype=np.float64)
    for a, b, j in ((0, 1, 0), (2, 3, 2)):
        r = np.sqrt(-2.0 * np.log(_uniform32(w[:, a])))
        th = 2.0 * np.pi * _uniform24(w[:, b])
        out[:, j] = r * np.cos(th)
        out[:, j + 1] = r * np.sin(th)
    return out.reshape(-1)[:n]
