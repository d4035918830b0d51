"""The attention-dropout oracle, pinned on the CPU.

- fmix32 (MurmurHash3's finalizer) inside the whole MurmurHash3_x86_32 equals scikit-learn's murmurhash3_32,
  an independent implementation, on random 4-byte keys and seeds (a wrong constant or shift fails it), and the
  hash's published test vectors hold.
- The keep mask: rate 1 - p within binomial bounds; no correlation between neighbouring queries, keys (a key
  pair {2i, 2i + 1} shares one hash, its halves), heads, seeds, and the four entries of random 2x2 blocks are
  jointly independent (the per-element hash mixes a row key with a column key by xor, which a weak finalizer
  would leave visible there).
- Attention with dropout: p = 0 is the plain oracle; the mean over many seeds of the dropped output tends to
  the undropped output (the 1 / (1 - p) scale and the mask on the probabilities); the analytic backward equals
  torch.autograd through a dense fp64 forward on the same materialised mask.
"""
import math

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import dropout as D


def test_fmix32_inside_murmurhash3_matches_scikit_learn():
    sk = pytest.importorskip("sklearn.utils")
    rng = np.random.default_rng(0)
    keys = rng.integers(-2 ** 31, 2 ** 31, size=400, dtype=np.int64)
    for seed in (0, 1, 0x9747B28C, 2 ** 31 + 5, 2 ** 32 - 1):
        ref = np.array([sk.murmurhash3_32(int(k), seed, positive=True) for k in keys], dtype=np.uint64)
        assert np.array_equal(D.murmurhash3_x86_32(keys, seed).astype(np.uint64), ref), seed


def test_murmurhash3_published_vectors():
    """The test vectors published for MurmurHash3_x86_32: the empty key (the hash is then fmix32(seed) alone)
    with seeds 0, 1 and 2^32 - 1, and the 4-byte keys 00 00 00 00, "test" and "aaaa"."""
    for seed, want in ((0, 0x00000000), (1, 0x514E28B7), (0xFFFFFFFF, 0x81F16F39)):
        assert int(D.fmix32(np.uint32(seed))) == want
    for key, seed, want in ((b"\0\0\0\0", 0, 0x2362F9DE), (b"test", 0, 0xBA6BD213), (b"test", 0x9747B28C, 0x704B81DC),
                            (b"aaaa", 0x9747B28C, 0x5A97808A)):
        k = np.array([int.from_bytes(key, "little")], dtype=np.int64)
        assert int(D.murmurhash3_x86_32(k, seed)[0]) == want, key


def test_params_threshold_and_scale():
    assert D.params(0.0, 5)[2] == 0 and D.params(0.0, 5)[3] == 1.0   # keep everything, unscaled
    assert D.params(0.5, 5)[2] == 2 ** 15 and D.params(0.5, 5)[3] == 2.0
    assert D.params(np.nextafter(np.float32(1), np.float32(0)), 5)[2] == 2 ** 16 - 1   # capped: one value in 2^16 kept
    assert D.params(0.08, 5)[2] == 5243                                   # round(0.08 * 2^16)
    assert D.params(0.08, 5)[3] == pytest.approx(65536 / (65536 - 5243), rel=1e-7)
    assert abs(D.params(0.08, 5)[3] * 0.92 - 1) < 3e-5                   # p quantised to 2^-16
    s0, s1, _, _ = D.params(0.1, (7 << 32) | 9)
    assert (int(s0), int(s1)) == (9, 7 ^ 0x9E3779B9)


@pytest.mark.parametrize("p", [0.05, 0.08, 0.5, 0.9])
def test_keep_rate_within_binomial_bounds(p):
    z = D.keep_mask(p, 20260101, 4, np.arange(700), np.arange(900))
    n = z.size
    sigma = math.sqrt(p * (1 - p) / n)
    assert abs(z.mean() - (1 - p)) < 5 * sigma


def _corr(a, b):
    a, b = a.astype(np.float64).ravel(), b.astype(np.float64).ravel()
    return float(np.corrcoef(a, b)[0, 1])


def test_mask_has_no_visible_structure():
    p, seed, heads = 0.5, 99, 4
    z = D.keep_mask(p, seed, heads, np.arange(600), np.arange(600))
    n = z[:, 1:, :].size
    bound = 5 / math.sqrt(n)
    assert abs(_corr(z[:, 1:, :], z[:, :-1, :])) < bound     # neighbouring queries
    assert abs(_corr(z[:, :, 1:], z[:, :, :-1])) < bound     # neighbouring keys
    assert abs(_corr(z[1:], z[:-1])) < 5 / math.sqrt(z[1:].size)   # neighbouring heads
    z2 = D.keep_mask(p, seed + 1, heads, np.arange(600), np.arange(600))
    assert abs(_corr(z, z2)) < 5 / math.sqrt(z.size)            # neighbouring seeds
    # the transpose is not the same mask (row and column keys differ)
    assert abs(_corr(z[0], z[0].T)) < 5 / math.sqrt(z[0].size)
    # 2x2 blocks (q1, q2) x (k1, k2): all four kept with probability (1 - p)^4, and the xor of the four is
    # unbiased -- the combination a per-element xor of row and column keys could correlate
    rng = np.random.default_rng(3)
    qa, qb = rng.integers(0, 600, 200000), rng.integers(0, 600, 200000)
    ka, kb = rng.integers(0, 600, 200000), rng.integers(0, 600, 200000)
    ok = (qa != qb) & (ka != kb)
    b4 = np.stack([z[0, qa, ka], z[0, qa, kb], z[0, qb, ka], z[0, qb, kb]])[:, ok]
    m = b4.shape[1]
    all4 = b4.all(0).mean()
    assert abs(all4 - 0.0625) < 5 * math.sqrt(0.0625 * 0.9375 / m)
    parity = np.bitwise_xor.reduce(b4, axis=0).mean()
    assert abs(parity - 0.5) < 5 * math.sqrt(0.25 / m)


def _seg_inputs(seed, tq, tk, h, d):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(tq, h, d, generator=g, dtype=torch.float64), torch.randn(tk, h, d, generator=g,
            dtype=torch.float64), torch.randn(tk, h, d, generator=g, dtype=torch.float64),
            torch.randn(tq, h, d, generator=g, dtype=torch.float64))


def test_p_zero_is_the_plain_oracle():
    q, k, v, g = _seg_inputs(1, 50, 50, 3, 16)
    cu = np.array([0, 20, 50])
    out0, lse0 = OA.varlen_attention(q, k, v, cu, cu, 0.25)
    out1, lse1 = OA.varlen_attention(q, k, v, cu, cu, 0.25, dropout=(0.0, 77))
    assert torch.equal(out0, out1) and torch.equal(lse0, lse1)
    for a, b in zip(OA.varlen_attention_bwd(g, q, k, v, cu, cu, 0.25),
                    OA.varlen_attention_bwd(g, q, k, v, cu, cu, 0.25, dropout=(0.0, 77))):
        assert torch.equal(a, b)


def test_mean_over_seeds_tends_to_the_undropped_output():
    """E_Z[(P o Z / (1 - p)) V] = P V: averaged over 400 seeds the dropped output is within 6 standard errors
    of the undropped one (the per-element variance estimated from the draws)."""
    q, k, v, _ = _seg_inputs(2, 12, 12, 2, 16)
    cu = np.array([0, 12])
    ref, lse_ref = OA.varlen_attention(q, k, v, cu, cu, 0.5)
    draws = torch.stack([OA.varlen_attention(q, k, v, cu, cu, 0.5, dropout=(0.3, s))[0] for s in range(400)])
    mean, se = draws.mean(0), draws.std(0) / math.sqrt(draws.shape[0])
    assert bool(((mean - ref).abs() <= 6 * se + 1e-12).all())
    # and a single draw differs from it (the mask is applied)
    assert not torch.allclose(draws[0], ref)
    assert torch.equal(OA.varlen_attention(q, k, v, cu, cu, 0.5, dropout=(0.3, 5))[1], lse_ref)


@pytest.mark.parametrize("mask", ["none", "node"])
def test_backward_equals_autograd_through_the_dense_forward(mask):
    """The analytic dropout backward (dS = P (dP W - D)) against autograd of out = (softmax(S) o W) V on the
    same materialised W = Z / (1 - p), per segment, with and without a node mask."""
    p, seed, h, d = 0.2, 4242, 3, 16
    lengths = [9, 14]
    cu = np.concatenate([[0], np.cumsum(lengths)])
    t = int(cu[-1])
    q, k, v, g = _seg_inputs(3, t, t, h, d)
    adj = None
    if mask == "node":
        rng = np.random.default_rng(5)
        rows, cols = [], []
        for b in range(len(lengths)):
            s, e = int(cu[b]), int(cu[b + 1])
            for i in range(s, e):
                js = sorted(set(rng.integers(s, e, size=4).tolist()))
                rows.append(js)
        indptr = np.concatenate([[0], np.cumsum([len(r) for r in rows])])
        adj = (indptr, np.array([j for r in rows for j in r]))
    dq, dk, dv = OA.varlen_attention_bwd(g, q, k, v, cu, cu, 0.3, adj=adj, dropout=(p, seed))
    out, _ = OA.varlen_attention(q, k, v, cu, cu, 0.3, adj=adj, dropout=(p, seed))
    qa, ka, va = (x.clone().requires_grad_(True) for x in (q, k, v))
    inv = D.params(p, seed)[3]
    outs = []
    for b in range(len(lengths)):
        s, e = int(cu[b]), int(cu[b + 1])
        sc = torch.einsum("ihd,jhd->hij", qa[s:e], ka[s:e]) * 0.3
        if adj is not None:
            m = torch.zeros(e - s, e - s, dtype=torch.bool)
            for i in range(s, e):
                for j in adj[1][adj[0][i]:adj[0][i + 1]]:
                    m[i - s, j - s] = True
            sc = sc.masked_fill(~m, float("-inf"))
        pr = torch.softmax(sc, -1)
        w = torch.as_tensor(D.keep_mask(p, seed, h, np.arange(s, e), np.arange(s, e))).double() * inv
        outs.append(torch.einsum("hij,jhd->ihd", pr * w, va[s:e]))
    dense = torch.cat(outs)
    assert torch.allclose(dense, out, atol=1e-12)
    dense.backward(g)
    for got, ref in ((dq, qa.grad), (dk, ka.grad), (dv, va.grad)):
        assert torch.allclose(got, ref, atol=1e-11)


def test_pair_path_and_global_ids_agree_with_the_segment_path():
    """masked_attention_pairs (the gathers the module oracle differentiates) with dropout equals varlen_attention
    with dropout under a node mask; a subset of the batch given its global token ids reproduces the full batch's
    rows (the mask hashes global indices)."""
    p, seed, h, d = 0.3, 31337, 2, 16
    lengths = [11, 17, 6]
    cu = np.concatenate([[0], np.cumsum(lengths)])
    t = int(cu[-1])
    q, k, v, _ = _seg_inputs(8, t, t, h, d)
    rng = np.random.default_rng(2)
    rows = []
    for b in range(len(lengths)):
        s, e = int(cu[b]), int(cu[b + 1])
        rows += [sorted(set(rng.integers(s, e, size=3).tolist())) for _ in range(s, e)]
    indptr = np.concatenate([[0], np.cumsum([len(r) for r in rows])])
    adj = (indptr, np.array([j for r in rows for j in r]))
    full, _ = OA.varlen_attention(q, k, v, cu, cu, 0.4, adj=adj, dropout=(p, seed))
    pairs = OA.masked_attention_pairs(q, k, v, cu, cu, 0.4, adj=adj, dropout=(p, seed))
    assert torch.allclose(pairs, full, atol=1e-12)
    # graph 1 alone, renumbered from 0, with its global ids
    s, e = int(cu[1]), int(cu[2])
    sub_rows = rows[s:e]
    sub_ptr = np.concatenate([[0], np.cumsum([len(r) for r in sub_rows])])
    sub_adj = (sub_ptr, np.array([j - s for r in sub_rows for j in r]))
    ids = np.arange(s, e)
    sub, _ = OA.varlen_attention(q[s:e], k[s:e], v[s:e], [0, e - s], [0, e - s], 0.4, adj=sub_adj,
                                 dropout=(p, seed, ids, ids))
    assert torch.allclose(sub, full[s:e], atol=1e-12)
    sub_pairs = OA.masked_attention_pairs(q[s:e], k[s:e], v[s:e], [0, e - s], [0, e - s], 0.4, adj=sub_adj,
                                          dropout=(p, seed, ids, ids))
    assert torch.allclose(sub_pairs, full[s:e], atol=1e-12)


@pytest.mark.parametrize("p", [0.08, 0.5])
def test_key_pair_halves_are_independent(p):
    """Keys 2i and 2i + 1 take the low and high 16 bits of one hash: their keep decisions are uncorrelated and
    both are kept at rate (1 - p)^2, within 5 sigma."""
    z = D.keep_mask(p, 20260102, 2, np.arange(1500), np.arange(1200))
    even, odd = z[:, :, 0::2], z[:, :, 1::2]
    n = even.size
    assert abs(_corr(even, odd)) < 5 / math.sqrt(n)
    q = (1 - p) ** 2
    assert abs((even & odd).mean() - q) < 5 * math.sqrt(q * (1 - q) / n)
