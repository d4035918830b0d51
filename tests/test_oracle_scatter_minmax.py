"""The scatter_min / scatter_max oracle (torch_scatter's semantics), pinned on the CPU.

- The vectorised restatement equals the literal sequential loop of torch_scatter's CPU update (strict
  comparison from numeric_limits::max() / lowest(), ascending index, untouched outputs 0 with arg =
  src.size(0)) bit for bit, on inputs full of ties, NaN, +-inf, the float32 maximum, -0 and dropped indices.
- Values: on finite inputs they equal torch's own scatter_reduce('amin' / 'amax', include_self=False), an
  independent implementation, wherever a node has an edge (and 0 where it has none).
- Args: brute force -- arg[n] is the smallest edge id of node n whose value equals out[n].
- Known answer: the scatter_max example of torch_scatter's documentation (two rows of five values).
"""
import numpy as np
import pytest
import torch

from oracle import edges as E


def _cases(seed, n_cases):
    rng = np.random.default_rng(seed)
    for _ in range(n_cases):
        e, n, f = int(rng.integers(0, 50)), int(rng.integers(1, 14)), int(rng.integers(1, 4))
        y = rng.integers(-3, 4, size=(e, f)).astype(np.float32)   # small integers: many ties
        u = rng.random((e, f))
        y[u < 0.05] = np.nan
        y[(u >= 0.05) & (u < 0.08)] = np.inf
        y[(u >= 0.08) & (u < 0.11)] = -np.inf
        y[(u >= 0.11) & (u < 0.14)] = np.finfo(np.float32).max
        y[(u >= 0.14) & (u < 0.17)] = -0.0
        yield y, rng.integers(-1, n + 1, size=e), n


@pytest.mark.parametrize("maximum", [False, True])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_vectorised_equals_the_sequential_update(maximum, dtype):
    for y, idx, n in _cases(1, 250):
        a_out, a_arg = E.scatter_minmax_loop(y, idx, n, maximum, dtype)
        b_out, b_arg = E.scatter_minmax(y, idx, n, maximum, dtype)
        assert np.array_equal(a_arg, b_arg)
        assert np.array_equal(a_out.view(np.uint32), b_out.view(np.uint32))


@pytest.mark.parametrize("maximum", [False, True])
def test_values_equal_torch_scatter_reduce_and_args_brute_force(maximum):
    rng = np.random.default_rng(2)
    e, n, f = 4000, 700, 3
    y = rng.integers(-50, 50, size=(e, f)).astype(np.float32) / 4   # ties
    idx = rng.integers(0, n, size=e)
    out, arg = E.scatter_minmax(y, idx, n, maximum)
    ref = torch.zeros(n, f).scatter_reduce(0, torch.as_tensor(idx).unsqueeze(1).expand(e, f), torch.as_tensor(y),
                                           "amax" if maximum else "amin", include_self=False)
    assert np.array_equal(out, ref.numpy())   # nodes without edges keep the zeros on both sides
    has = np.bincount(idx, minlength=n) > 0
    for node in range(n):
        for c in range(f):
            if not has[node]:
                assert arg[node, c] == e and out[node, c] == 0
                continue
            es = np.nonzero((idx == node) & (y[:, c] == out[node, c]))[0]
            assert arg[node, c] == es.min()


def test_values_beyond_the_start_and_nan_never_win():
    """torch_scatter starts a minimum at numeric_limits::max(): +inf and the maximum itself never replace
    it, so a node with only such values (or NaN) gives 0 and arg = E, like a node with no edges."""
    fmax = np.finfo(np.float32).max
    y = np.array([np.inf, fmax, np.nan, 5.0, np.inf], np.float32)
    idx = np.array([0, 0, 1, 2, 2])
    out, arg = E.scatter_minmax_loop(y, idx, 4)
    assert out[:, 0].tolist() == [0.0, 0.0, 5.0, 0.0] and arg[:, 0].tolist() == [5, 5, 3, 5]
    out, arg = E.scatter_minmax_loop(-y, idx, 4, maximum=True)
    assert out[:, 0].tolist() == [0.0, 0.0, -5.0, 0.0] and arg[:, 0].tolist() == [5, 5, 3, 5]
    # bfloat16's largest finite value is its start: a bf16 value at it never wins either
    bmax = np.float32(np.uint32(0x7F7F0000).view(np.float32))
    out, arg = E.scatter_minmax_loop(np.array([bmax, 1.0], np.float32), np.array([0, 1]), 2, dtype="bfloat16")
    assert out[:, 0].tolist() == [0.0, 1.0] and arg[:, 0].tolist() == [2, 1]


def test_documented_scatter_max_example():
    """torch_scatter's documentation: src = [[2, 0, 1, 4, 3], [0, 2, 1, 3, 4]], index = [[4, 5, 4, 2, 3],
    [0, 0, 2, 2, 1]], scatter_max(src, index, dim=-1) gives out = [[0, 0, 4, 3, 2, 0], [2, 4, 3, 0, 0, 0]]
    and argmax = [[5, 5, 3, 4, 0, 1], [1, 4, 3, 5, 5, 5]] (each row is a 1-D scatter over 6 outputs)."""
    src = [[2, 0, 1, 4, 3], [0, 2, 1, 3, 4]]
    index = [[4, 5, 4, 2, 3], [0, 0, 2, 2, 1]]
    want_out = [[0, 0, 4, 3, 2, 0], [2, 4, 3, 0, 0, 0]]
    want_arg = [[5, 5, 3, 4, 0, 1], [1, 4, 3, 5, 5, 5]]
    for s, i, wo, wa in zip(src, index, want_out, want_arg):
        for fn in (E.scatter_minmax_loop, E.scatter_minmax):
            out, arg = fn(np.array(s, np.float32), np.array(i), 6, maximum=True)
            assert out[:, 0].tolist() == wo and arg[:, 0].tolist() == wa
