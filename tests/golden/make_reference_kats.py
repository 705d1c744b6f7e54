"""Writes reference_kats.json: the known answers the reference's own tests
pin for the paged-attention path, with their provenance.

Nothing from the reference is imported or run. The block tables follow from
the LIFO free stack of src/core/memory_manager.py:49,69 with the exact calls
the tests make; the attention value is the closed form of the data the test
writes (K = V = t at token t, q = ones), evaluated with math.fsum.

    python tests/golden/make_reference_kats.py
"""
import json
import math
import os


def closed_form_test_kernels(head_dim: int, tokens: int) -> float:
    # score_t = (q . k_t) / sqrt(D) = D*t/sqrt(D) = sqrt(D)*t; out = sum t w_t / sum w_t
    s = [math.sqrt(head_dim) * t for t in range(tokens)]
    m = max(s)
    w = [math.exp(x - m) for x in s]
    return math.fsum(t * wt for t, wt in zip(range(tokens), w)) / math.fsum(w)


kats = {
    "test_kernels_append": {
        "source": "tests/test_kernels.py:14-63",
        "num_blocks": 16, "block_size": 4, "num_heads": 2, "head_dim": 8,
        "calls": "allocate(req_1, 0); append_slot x5",
        "context_len": 5,
        "block_table": [15, 14],
        "k_equals_v_equals_token_index": True,
        "query": "ones",
        "scale": 1.0 / math.sqrt(8),
        "expected_output_every_element": closed_form_test_kernels(8, 5),
    },
    "verify_attention_load_initial_kv": {
        "source": "tests/verify_attention.py:35-58,77",
        "num_blocks": 10, "block_size": 4, "num_heads": 4, "head_dim": 16,
        "calls": "load_initial_kv(req_1, 5 tokens); write_new_kv x1",
        "context_len_after_load": 5,
        "block_table_after_load": [9, 8],
        "context_len_after_append": 6,
        "block_table_after_append": [9, 8],
    },
    "verify_attention_kernel_vs_ref": {
        "source": "tests/verify_attention.py:88-136",
        "num_blocks": 100, "block_size": 16, "num_heads": 4, "head_dim": 32,
        "dtype": "float16",
        "calls": "allocate(rid, 0); write_new_kv(rid, k, v) x50 with one fixed (k, v)",
        "context_len": 50,
        "block_table": [99, 98, 97, 96],
        "expected_output": "v (50 identical keys give a uniform softmax)",
        "atol": 1e-2, "rtol": 1e-2,
    },
}

if __name__ == "__main__":
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_kats.json")
    with open(path, "w") as f:
        json.dump(kats, f, indent=2, sort_keys=True)
        f.write("\n")
    print(path)
