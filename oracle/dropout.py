"""Attention-dropout keep mask (test infrastructure; see oracle/__init__.py).

The reference applies dropout to the attention probabilities in training:
``memory_efficient_attention(..., p=self.dropout_p if self.training else 0)``
and SDPA's ``dropout_p`` (esa/mha.py:76,82), flash_attn_varlen_func's
``dropout_p`` (esa/mha_flash_varlen.py:177-184): out = (P o Z / (1 - p)) V for
a random keep mask Z with P(Z = 1) = 1 - p.  Those libraries draw Z from
their own generators, so no run reproduces the reference's Z; this build
defines Z as a counter-based hash of (seed, head, query token, key token),
restated here from its definition in the C ABI (include/esa_hip.h):

  keep(q, k, h) = half(fmix32(row(q, h) ^ col(k)), k mod 2) >= thr
  row(q, h)     = fmix32(s0 ^ fmix32(q * heads + h))
  col(k)        = fmix32(s1 ^ fmix32(floor(k / 2)))
  half(x, 0) = x mod 2^16, half(x, 1) = floor(x / 2^16)
  s0 = seed & 0xFFFFFFFF, s1 = (seed >> 32) ^ 0x9E3779B9
  thr = min(floor(float32(p) * 2^16 + 0.5), 2^16 - 1); kept values scale by
  inv_keep = 2^16 / (2^16 - thr), the inverse of the exact keep rate

(the keys 2i and 2i + 1 share one hash and take its low and high 16 bits).

fmix32 is the 32-bit finalizer of MurmurHash3 (Austin Appleby, SMHasher,
public domain): h ^= h >> 16; h *= 0x85EBCA6B; h ^= h >> 13; h *= 0xC2B2AE35;
h ^= h >> 16.  ``murmurhash3_x86_32`` below is the whole published hash for
4-byte keys built on it, so the finalizer is pinned against an independent
implementation (scikit-learn's ``murmurhash3_32``).
"""
from __future__ import annotations

import numpy as np

_M32 = np.uint32(0xFFFFFFFF)


def fmix32(h):
    """MurmurHash3's 32-bit finalizer, elementwise over uint32 values."""
    h = np.asarray(h, dtype=np.uint32).copy()
    with np.errstate(over="ignore"):
        h ^= h >> np.uint32(16)
        h *= np.uint32(0x85EBCA6B)
        h ^= h >> np.uint32(13)
        h *= np.uint32(0xC2B2AE35)
        h ^= h >> np.uint32(16)
    return h


def _rotl32(x, r):
    return (x << np.uint32(r)) | (x >> np.uint32(32 - r))


def murmurhash3_x86_32(keys, seed: int):
    """MurmurHash3_x86_32 of each 4-byte little-endian key (one block, no tail), uint32 results."""
    k = np.asarray(keys).astype(np.int64).astype(np.uint32)
    with np.errstate(over="ignore"):
        k = k * np.uint32(0xCC9E2D51)
        k = _rotl32(k, 15)
        k = k * np.uint32(0x1B873593)
        h = np.full(k.shape, seed & 0xFFFFFFFF, dtype=np.uint32) ^ k
        h = _rotl32(h, 13)
        h = h * np.uint32(5) + np.uint32(0xE6546B64)
        h ^= np.uint32(4)   # the key length
    return fmix32(h)


def params(p: float, seed: int):
    """(s0, s1, thr, inv_keep) as the library derives them from (dropout_p, seed); p is a float32 argument."""
    p32 = float(np.float32(p))
    seed = int(seed) & ((1 << 64) - 1)
    s0 = np.uint32(seed & 0xFFFFFFFF)
    s1 = np.uint32(((seed >> 32) & 0xFFFFFFFF) ^ 0x9E3779B9)
    t = p32 * 65536.0 + 0.5
    thr = np.uint32(65535) if t >= 65535.0 else np.uint32(int(t))
    inv_keep = float(np.float32(65536.0 / (65536.0 - float(thr))))
    return s0, s1, thr, inv_keep


def row_keys(seed: int, heads: int, q_idx, head: int):
    s0 = params(0.0, seed)[0]
    qi = np.asarray(q_idx, dtype=np.int64)
    with np.errstate(over="ignore"):
        lin = (qi.astype(np.uint32) * np.uint32(heads) + np.uint32(head)).astype(np.uint32)
    return fmix32(s0 ^ fmix32(lin))


def col_keys(seed: int, k_idx):
    """The column key of each key token: shared by the pair {2i, 2i + 1}."""
    s1 = params(0.0, seed)[1]
    return fmix32(s1 ^ fmix32((np.asarray(k_idx, dtype=np.int64) >> 1).astype(np.uint32)))


def _half(bits, k_idx):
    """Key k's 16 bits of its pair's hash: the low half for even k, the high half for odd k."""
    sh = ((np.asarray(k_idx, dtype=np.int64) & 1) * 16).astype(np.uint32)
    return (bits >> sh) & np.uint32(0xFFFF)


def keep_pairs(p: float, seed: int, heads: int, q_idx, k_idx):
    """Bool [heads, n]: Z of the pairs (q_idx[i], k_idx[i]) (global token indices) in every head."""
    _, _, thr, _ = params(p, seed)
    c = col_keys(seed, k_idx)
    return np.stack([_half(fmix32(row_keys(seed, heads, q_idx, h) ^ c), k_idx) >= thr for h in range(heads)])


def keep_mask(p: float, seed: int, heads: int, q_idx, k_idx, head_lo: int = 0, head_hi: int | None = None):
    """Bool [head_hi - head_lo, len(q_idx), len(k_idx)]: Z for the global query / key token indices given."""
    _, _, thr, _ = params(p, seed)
    head_hi = heads if head_hi is None else head_hi
    c = col_keys(seed, k_idx)
    kk = np.asarray(k_idx, dtype=np.int64)[None, :]
    out = np.empty((head_hi - head_lo, len(q_idx), len(c)), dtype=bool)
    for i, h in enumerate(range(head_lo, head_hi)):
        r = row_keys(seed, heads, q_idx, h)
        out[i] = _half(fmix32(r[:, None] ^ c[None, :]), kk) >= thr
    return out
