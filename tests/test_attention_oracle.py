"""The attention oracle pinned on the CPU: torch's scaled_dot_product_attention in fp64 and
closed forms; and the host wrapper's argument checks (no GPU call)."""
import numpy as np
import pytest
import torch

import oracle


def _rand(rng, *shape):
    return rng.standard_normal(shape)


def test_attention_matches_torch_sdpa():
    rng = np.random.default_rng(0)
    h, d = 3, 16
    cu_q, cu_kv = [0, 5, 5, 17, 40], [0, 9, 20, 20, 61]
    q, k, v = _rand(rng, 40, h, d), _rand(rng, 61, h, d), _rand(rng, 61, h, d)
    got = oracle.attention(q, k, v, cu_q, cu_kv)
    for b in range(4):
        q0, q1, k0, k1 = cu_q[b], cu_q[b + 1], cu_kv[b], cu_kv[b + 1]
        if q1 == q0:
            continue
        if k1 == k0:  # no keys: zeros (attention.ts:57)
            assert not got[q0:q1].any()
            continue
        t = torch.nn.functional.scaled_dot_product_attention(
            torch.from_numpy(q[q0:q1]).transpose(0, 1), torch.from_numpy(k[k0:k1]).transpose(0, 1),
            torch.from_numpy(v[k0:k1]).transpose(0, 1)).transpose(0, 1).numpy()
        np.testing.assert_allclose(got[q0:q1], t, rtol=1e-12, atol=1e-12)
    # explicit scale and row subset
    sub = oracle.attention(q, k, v, cu_q, cu_kv, scale=0.3, rows=[1, 20])
    full = oracle.attention(q, k, v, cu_q, cu_kv, scale=0.3)
    np.testing.assert_allclose(sub[[1, 20]], full[[1, 20]], rtol=1e-13)
    assert not sub[[0, 2, 19, 21]].any()


def test_attention_closed_forms():
    rng = np.random.default_rng(1)
    h, d, n = 2, 8, 13
    q, k = _rand(rng, n, h, d), _rand(rng, n, h, d)
    row = _rand(rng, 1, h, d)
    v_const = np.repeat(row, n, axis=0)
    np.testing.assert_allclose(oracle.attention(q, k, v_const, [0, n], [0, n]),
                               np.repeat(row, n, axis=0), rtol=1e-12)
    v = _rand(rng, n, h, d)
    zero_q = oracle.attention(np.zeros_like(q), k, v, [0, n], [0, n])
    np.testing.assert_allclose(zero_q, np.repeat(v.mean(0, keepdims=True), n, 0), rtol=1e-12)
    one = oracle.attention(q, k[:1], v[:1], [0, n], [0, 1])
    np.testing.assert_allclose(one, np.repeat(v[:1], n, 0), rtol=1e-12)
    perm = rng.permutation(n)
    np.testing.assert_allclose(oracle.attention(q, k[perm], v[perm], [0, n], [0, n]),
                               oracle.attention(q, k, v, [0, n], [0, n]), rtol=1e-12)
    # a planted mistake (no scale) must be caught by the torch comparison's values
    wrong = oracle.attention(q, k, v, [0, n], [0, n], scale=1.0)
    assert not np.allclose(wrong, oracle.attention(q, k, v, [0, n], [0, n]))


def test_wrapper_rejects_cpu_tensors(pkg):
    x = torch.zeros(4, 2, 64)
    with pytest.raises(pkg.TscError):
        pkg.sparse_attention(x, x, x, [0, 4])
