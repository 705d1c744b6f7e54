"""Property test of paged decode (hypothesis, GPU): random ragged batches
through every schedule the op offers - the automatic choice, single pass,
split-K at several partition sizes and the balanced split at random wave
counts - each against the fp32 oracle. Contexts include 0, lengths below a
partition, lengths that are not multiples of the block size, and pools whose
unused slots hold NaN (a read outside a context shows in the output)."""
import pytest
import torch
from hypothesis import given, settings, strategies as st

from oracle import attention as oa
from tests.helpers import assert_attention_close
from tests.test_gpu_decode import case, run_decode

pytestmark = pytest.mark.gpu


@st.composite
def batch(draw):
    hkv = draw(st.sampled_from([1, 2, 4, 8]))
    g = draw(st.sampled_from([1, 2, 4, 7, 8]))
    d = draw(st.sampled_from([64, 128]))
    bs = draw(st.sampled_from([8, 16, 32]))
    ctx = draw(st.lists(st.one_of(st.just(0), st.integers(1, 40), st.integers(41, 1200)),
                        min_size=1, max_size=6))
    dtype = draw(st.sampled_from([torch.float16, torch.bfloat16]))
    partition = draw(st.sampled_from([32, 64, 512]))
    waves = draw(st.integers(1, 1500))
    seed = draw(st.integers(0, 10 ** 6))
    return hkv, g, d, bs, ctx, dtype, partition, waves, seed


@settings(max_examples=40, deadline=None, derandomize=True)
@given(batch())
def test_ragged_batches_every_schedule(c):
    hkv, g, d, bs, ctx, dtype, partition, waves, seed = c
    if max(ctx) == 0:
        ctx = ctx + [1]
    hq = hkv * g
    print(f"ragged hkv={hkv} g={g} d={d} bs={bs} ctx={ctx} {dtype} P={partition} W={waves}",
          flush=True)
    q, k, v, tables, scale = case(seed, ctx, hq, hkv, d, bs, dtype)
    ref = oa.paged_decode(q, k, v, tables, ctx, scale)
    for p, w in ((None, 0), (0, 0), (partition, 0), (None, waves)):
        got = run_decode(q, k, v, tables, ctx, scale, partition_size=p, num_waves=w)
        assert_attention_close(got, ref, what=f"P={p} W={w}")
