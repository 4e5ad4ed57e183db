"""The oracle against the committed golden fixtures (tests/golden/, written by
tests/golden/make_golden.py): dequantised values and GEMV outputs bit for bit,
and the tiny model's greedy tokens and per-step logits summary.  CPU only."""
import json
import os

import numpy as np
import pytest

from dotllm_amd import synth
from oracle import oracle as O

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
from golden.make_golden import TYPES  # noqa: E402


@pytest.mark.parametrize("name", list(TYPES))
def test_dequant_golden(name):
    z = np.load(os.path.join(HERE, "dequant.npz"))
    out = O.dequantize(z[name + "_src"], TYPES[name], 4, 512)
    assert np.array_equal(out.view(np.uint32), z[name + "_out"].view(np.uint32))


@pytest.mark.parametrize("name", list(TYPES))
def test_gemv_golden(name):
    z = np.load(os.path.join(HERE, "gemv.npz"))
    y = O.matmul(z[name + "_x"], z[name + "_w"], TYPES[name], 256, 32)
    assert np.array_equal(y, z[name + "_y"])


def test_tiny_greedy_golden():
    with open(os.path.join(HERE, "tiny_greedy.json")) as f:
        g = json.load(f)
    img = synth.build_image("tiny", seed=g["weights_seed"])
    assert synth.prompt(32000, 16, seed=g["prompt_seed"]) == g["prompt"]
    m = O.Model(img, kv_fp16=False)
    toks, logits = m.generate(g["prompt"], len(g["tokens"]), return_logits=True)
    m.close()
    assert toks == g["tokens"]
    for row, st in zip(logits, g["steps"]):
        assert [int(i) for i in np.argsort(row)[::-1][:5]] == st["top5"]
        np.testing.assert_allclose(row[st["top5"]], st["top5_logits"], rtol=0, atol=0)
        assert abs(float(np.sum(row, dtype=np.float64)) - st["sum"]) <= 1e-9 * max(1.0, abs(st["sum"]))
        assert abs(float(np.sum(row.astype(np.float64) ** 2)) - st["sumsq"]) <= 1e-9 * st["sumsq"]


def test_device_floors_within_reordering_range():
    """The greedy regression floors of the full-size GPU runs (MIN_SAME in
    tests/test_gpu_long.py: how far the device was measured to keep the
    reference's tokens) against how far the oracle itself keeps them when
    only its summation order changes (order_prefix.json, written by
    tests/golden/order_prefix.py from the same fixtures): every floor is at
    least the shortest of the reorderings, so the device departs no earlier
    than some valid reordering of the reference's arithmetic; and each
    recorded prefix length is what the recorded tokens give against the
    fixture's."""
    from test_gpu_long import MIN_SAME
    d = json.load(open(os.path.join(HERE, "order_prefix.json")))
    assert set(d) <= set(MIN_SAME)
    for key, r in d.items():
        assert MIN_SAME[key] >= min(r["identical"]), (key, MIN_SAME[key], r["identical"])
        ref = np.load(os.path.join(HERE, f"long_{key}.npz"))["tokens"].tolist()
        for o, toks in r["tokens"].items():
            same = next((i for i, (a, b) in enumerate(zip(toks, ref)) if a != b), len(ref))
            assert same == r["identical"][r["orders"].index(int(o))], (key, o)
