"""The synthetic 27B model's tensor plan against the reference's index of the real Q4_K_M file
(tests/golden/gguf/gguf_index.json, copied from the reference's tests/fixtures/, used there by
tests/gguf_index.rs:16,79): the same 866 tensor names, ggml types and shapes, so the benchmark model has the real
file's byte mix (docs/data/q4km_type_breakdown.txt: Q4_K 249, Q6_K 97, Q8_0 24, Q5_K 32, Q4_0 8, F32 456)."""
import collections
import json
import os

import aqueduct as aq

HERE = os.path.dirname(os.path.abspath(__file__))
TYPE_ID = {"F32": 0, "Q4_0": 2, "Q8_0": 8, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14}


def index():
    return json.load(open(os.path.join(HERE, "golden", "gguf", "gguf_index.json")))


def test_27b_plan_equals_the_real_files_tensor_index():
    idx = index()
    assert idx["n_tensors"] == len(idx["tensors"]) == 866
    want = {}
    for t in idx["tensors"]:
        rows, cols = (t["shape_numpy_order"] + [1])[:2] if len(t["shape_numpy_order"]) == 2 else \
            (1, t["shape_numpy_order"][0])
        want[t["name"]] = (t["ggml_type_id"], rows, cols)
    plan = aq.model_plan(aq.config_27b(), aq.MIX_Q4_K_M, 1)
    got = {name: (sp.ggml_type, sp.rows, sp.cols) for name, sp in plan}
    assert len(got) == len(plan) == 866
    missing, extra = sorted(set(want) - set(got)), sorted(set(got) - set(want))
    assert not missing and not extra, f"missing {missing[:5]}, extra {extra[:5]}"
    diff = [(n, got[n], want[n]) for n in want if got[n] != want[n]]
    assert not diff, f"{len(diff)} tensors differ, e.g. {diff[:5]}"
    counts = collections.Counter(t for t, _, _ in got.values())
    assert counts == {TYPE_ID["Q4_K"]: 249, TYPE_ID["Q6_K"]: 97, TYPE_ID["Q8_0"]: 24, TYPE_ID["Q5_K"]: 32,
                      TYPE_ID["Q4_0"]: 8, TYPE_ID["F32"]: 456}


def test_27b_plan_bytes_equal_the_real_files_tensor_bytes():
    idx = index()
    by = {t["name"]: t["byte_size"] for t in idx["tensors"]}
    plan = aq.model_plan(aq.config_27b(), aq.MIX_Q4_K_M, 1)
    tot = 0
    for name, sp in plan:
        nb = sp.rows * aq.row_bytes(sp.ggml_type, sp.cols)
        assert nb == by[name], name
        tot += nb
    assert tot == sum(by.values())
