"""Writes the known-answer fixtures in this folder.

The expected values are written out by hand or from closed forms (no
oracle, no reference code is run): they are the independent pins the
oracle and the HIP library are both checked against.
Run: python tests/golden/make_golden.py
"""
import json
import math
from pathlib import Path

HERE = Path(__file__).resolve().parent


def metadata():
    page_table = [
        [10, 11, 12, 13, 14, 15],
        [20, 21, 22, 23, 24, 25],
        [30, 31, 32, 33, 34, 35],
    ]
    return {
        # build_decode_indices_kernel (src/attention/flashinfer_backend.cu:43-70):
        # row r of the output run comes from page_table[table_indices[r], :len];
        # columns past the table width read 0; bad rows leave the run untouched (0 here).
        "build_indices": [
            {"page_table": page_table, "table_indices": [2, 0], "kv_indptr": [0, 3, 5],
             "expected": [30, 31, 32, 10, 11]},
            {"page_table": page_table, "table_indices": [1], "kv_indptr": [0, 8],
             "expected": [20, 21, 22, 23, 24, 25, 0, 0]},
            {"page_table": page_table, "table_indices": [5, 1, -1], "kv_indptr": [0, 2, 3, 4],
             "expected": [0, 0, 20, 0]},
            {"page_table": page_table, "table_indices": [0, 1], "kv_indptr": [0, 0, 2],
             "expected": [20, 21]},
        ],
        # gather_int32_2d_kernel (src/kernels/token_pool.cu:31-49)
        "gather_int32_2d": [
            {"table": page_table, "req": [0, 2, 1, 3, 0, -1], "pos": [5, 0, 3, 0, 6, 1],
             "expected": [15, 30, 23, 0, 0, 0]},
        ],
        # write_token_pool_kernel (src/kernels/token_pool.cu:10-29)
        "write_token_pool": [
            {"pool": [[0, 0, 0], [0, 0, 0]], "req": [1, 0, 2, 1, -1], "pos": [2, 0, 0, 3, 1],
             "tok": [7, 8, 9, 10, 11], "expected": [[8, 0, 0], [0, 0, 7]]},
        ],
        # CacheManager::pages_to_tokens (src/scheduler/prefill.cc:103-119): a page is
        # identified by its first slot; its tokens are page + i.
        "pages_to_tokens": [
            {"page_starts": [32, 0, 16], "page_size": 16,
             "expected": list(range(32, 48)) + list(range(0, 16)) + list(range(16, 32))},
            {"page_starts": [5, 3], "page_size": 1, "expected": [5, 3]},
        ],
    }


def attention():
    cases = []
    # Case 1: uniform scores, 2 new tokens on a 1-token prefix (qo 2, kv 3).
    # Bottom-right alignment: query 0 sees kv 0..1, query 1 sees kv 0..2.
    cases.append({
        "head_dim": 4, "sm_scale": 1.0,
        "q": [[1, 0, 0, 0], [0, 1, 0, 0]],
        "k": [[0, 0, 0, 0]] * 3,
        "v": [[1, 0, 0, 0], [0, 1, 0, 0], [0, 0, 1, 0]],
        "indices": [0, 1, 2], "qo_indptr": [0, 2], "kv_indptr": [0, 3],
        "expected": [[0.5, 0.5, 0, 0], [1 / 3, 1 / 3, 1 / 3, 0]],
    })
    # Case 2: two kv tokens with scores a and 0, a = bf16(ln 2) = 0.69140625:
    # weights e^a/(e^a+1), 1/(e^a+1); V rows 3 e0 and 3 e1.
    a = 0.69140625
    w0 = math.exp(a) / (math.exp(a) + 1)
    cases.append({
        "head_dim": 4, "sm_scale": 1.0,
        "q": [[a, 0, 0, 0]],
        "k": [[1, 0, 0, 0], [0, 0, 0, 0]],
        "v": [[3, 0, 0, 0], [0, 3, 0, 0]],
        "indices": [0, 1], "qo_indptr": [0, 1], "kv_indptr": [0, 2],
        "expected": [[3 * w0, 3 * (1 - w0), 0, 0]],
    })
    # Case 3: indices permute pool slots; two requests, no prefix (qo == kv).
    # Request 0 (slots 2, 0): query 0 sees slot 2 only -> v[2]; query 1 sees both
    # with equal scores -> (v[2] + v[0]) / 2. Request 1 (slot 1): v[1].
    cases.append({
        "head_dim": 4, "sm_scale": 1.0,
        "q": [[0, 0, 0, 0]] * 3,
        "k": [[1, 1, 1, 1]] * 3,
        "v": [[2, 0, 0, 0], [0, 0, 0, 5], [0, 4, 0, 0]],
        "indices": [2, 0, 1], "qo_indptr": [0, 2, 3], "kv_indptr": [0, 2, 3],
        "expected": [[0, 4, 0, 0], [1, 2, 0, 0], [0, 0, 0, 5]],
    })
    return {"cases": cases}


if __name__ == "__main__":
    (HERE / "metadata_kat.json").write_text(json.dumps(metadata(), indent=1) + "\n")
    (HERE / "attention_kat.json").write_text(json.dumps(attention(), indent=1) + "\n")
    print("wrote", HERE)
