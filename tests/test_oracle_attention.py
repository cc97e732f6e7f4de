"""Oracle of the attention consumer (decode attention over the gathered
workspace) pinned by closed forms: equal scores average V, one dominant key
selects its value row, a single key returns its value, key order does not
matter, the output is linear in V and a shift of every score changes nothing."""
import sys
from pathlib import Path

import numpy as np

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
from oracle import v1 as O  # noqa: E402


def _inputs(seed, B=3, S=50, Hq=4, Hkv=1, D=128):
    g = np.random.default_rng(seed)
    return (g.standard_normal((B, Hq, D)), g.standard_normal((B, S, Hkv, D)), g.standard_normal((B, S, Hkv, D)))


def test_equal_scores_average_values():
    q, k, v = _inputs(1)
    out = O.decode_attention(np.zeros_like(q), k, v, 0.1)
    assert np.allclose(out, v.mean(axis=1)[:, None, 0, :].repeat(4, 1))


def test_dominant_key_and_single_key():
    q, k, v = _inputs(2)
    k[:, 17, 0] = 40 * q[:, 0]  # key 17 aligned with head 0: its score exceeds the others by thousands
    out = O.decode_attention(q, k, v, 1.0)
    assert np.allclose(out[:, 0], v[:, 17, 0], atol=1e-12)
    one = O.decode_attention(q, k[:, :1], v[:, :1], 1.0)
    assert np.allclose(one, v[:, :1, 0].repeat(4, 1))
    lens = np.array([1, 0, 50])
    part = O.decode_attention(q, k, v, 1.0, lens)
    assert np.allclose(part[0], v[0, 0, 0][None].repeat(4, 0)) and (part[1] == 0).all()


def test_key_order_linearity_and_shift():
    q, k, v = _inputs(3, Hq=8, Hkv=2)
    base = O.decode_attention(q, k, v, 0.088)
    perm = np.random.default_rng(3).permutation(k.shape[1])
    assert np.allclose(O.decode_attention(q, k[:, perm], v[:, perm], 0.088), base)
    assert np.allclose(O.decode_attention(q, k, 2 * v + 3, 0.088), 2 * base + 3)
    # a key component orthogonal to every query adds the same amount to all scores of a head
    q2 = q.copy()
    q2[..., -1] = 1.0
    k2 = k.copy()
    k2[..., -1] = 0.0
    shifted = k2.copy()
    shifted[..., -1] = 5.0  # every score of every head rises by 5 * scale
    assert np.allclose(O.decode_attention(q2, shifted, v, 0.088), O.decode_attention(q2, k2, v, 0.088))


def test_wrapper_rejects_options_it_does_not_implement():
    # host logic only (the checks run before any device call)
    import importlib
    import pytest
    import torch
    A = importlib.import_module("10_20_amd.attention")
    q = torch.zeros((1, 1, 4, 128), dtype=torch.bfloat16)
    kv = torch.zeros((1, 8, 1, 128), dtype=torch.bfloat16)
    for kw in ({"window_size": (64, 0)}, {"softcap": 30.0}, {"block_table": kv}, {"return_softmax_lse": True},
               {"k": kv}):
        with pytest.raises(NotImplementedError):
            A.flash_attn_with_kvcache(q, kv, kv, **kw)
    with pytest.raises(ValueError):  # host tensors: the operator needs the GPU
        A.flash_attn_with_kvcache(q, kv, kv, rotary_interleaved=True, num_splits=4)
