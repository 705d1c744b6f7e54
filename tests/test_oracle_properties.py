"""Property tests of the oracle's split-softmax path (hypothesis, CPU).

The LSE merge (restated from src/core/resident_kv_store.py:2497-2509) must
give the full softmax attention for ANY split of the keys into segments, in
any number and of any (ragged) size, including one-token segments and
segments whose scores sit far below the others (weights that underflow).
Checked against the float64 brute force.
"""
import numpy as np
import torch
from hypothesis import given, settings, strategies as st

from oracle import attention as oa


@st.composite
def split_case(draw):
    length = draw(st.integers(1, 300))
    hkv = draw(st.sampled_from([1, 2, 4]))
    g = draw(st.sampled_from([1, 3, 7]))
    d = draw(st.sampled_from([8, 32, 64]))
    cuts = sorted(set(draw(st.lists(st.integers(1, max(1, length - 1)), max_size=12))))
    cuts = [c for c in cuts if 0 < c < length]
    scale = draw(st.sampled_from([0.125, 1.0, 3.0, -0.5]))
    seed = draw(st.integers(0, 2 ** 31 - 1))
    shift = draw(st.sampled_from([0.0, 30.0]))  # one segment's keys far off the rest
    return length, hkv, g, d, cuts, scale, seed, shift


@settings(max_examples=60, deadline=None, derandomize=True)
@given(split_case())
def test_lse_merge_of_any_split_is_full_softmax(c):
    length, hkv, g, d, cuts, scale, seed, shift = c
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(hkv * g, d, generator=gen)
    k = torch.randn(length, hkv, d, generator=gen)
    v = torch.randn(length, hkv, d, generator=gen)
    if shift and cuts:
        k[:cuts[0]] += shift / d ** 0.5  # scores of the first segment move by ~shift
    bounds = [0, *cuts, length]
    parts = [oa.partial_attend(q, k[a:b], v[a:b], scale) for a, b in zip(bounds, bounds[1:])]
    got = oa.lse_merge(parts).numpy()
    ref = oa.brute_attention_fp64(q.numpy(), k.numpy(), v.numpy(), scale)
    np.testing.assert_allclose(got, ref, atol=2e-5, rtol=1e-4)
