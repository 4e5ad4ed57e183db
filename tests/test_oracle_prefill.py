"""The oracle's batched prompt path and its reduction-order variant (CPU).

orc_prefill computes the expected values for long prompts.  It must be the
sequential loop (N ProcessToken calls, InferenceEngine.cs:84-88) bit for bit:
the same operations per token in the same order, only scheduled differently.
These tests pin that against orc_process_token for every accumulation form the
reference's MatMul has (scalar sequential K-quant sums, 8-lane sums with a
horizontal sum, Q3_K's own association), GQA and MHA, fp16 and fp32 KV, a
prompt split over two calls and one that crosses the 512-token chunk.

orc_set_order(1..3) is the same computation in three other valid fp32
summation orders; the long fixtures use them to measure how far summation
order alone moves the logits.  Each must change results (or it measures
nothing), stay at fp32 rounding size on a shallow model, and leave the
reference order untouched.
"""
import json
import os

import numpy as np
import pytest

from dotllm_amd import F16, F32, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, byte_count, synth
from dotllm_amd._lib import Q2_K, Q3_K
from oracle import oracle as O

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

# d (and dmin) offsets of each K-quant / block type, to keep the scales finite
SCALES = {Q4_0: (32, 18, (0,)), Q8_0: (32, 34, (0,)), Q2_K: (256, 84, (0, 2)), Q3_K: (256, 110, (0,)),
          Q4_K: (256, 144, (0, 2)), Q5_K: (256, 176, (0, 2)), Q6_K: (256, 210, (208,))}


def blocks(t, rows, cols, rng):
    if t == F32:
        return rng.normal(0, 0.5, size=rows * cols).astype(np.float32).view(np.uint8)
    if t == F16:
        return rng.normal(0, 0.5, size=rows * cols).astype(np.float16).view(np.uint8)
    b = rng.integers(0, 256, size=rows * byte_count(t, cols), dtype=np.uint8)
    be, bb, offs = SCALES[t]
    h = rng.uniform(-0.1, 0.1, size=(rows * cols // be, len(offs))).astype(np.float16).view(np.uint8)
    bv = b.reshape(-1, bb)
    for j, off in enumerate(offs):
        bv[:, off:off + 2] = h.reshape(-1, len(offs), 2)[:, j]
    return b


@pytest.fixture(autouse=True)
def _order0():
    O.set_order(0)
    yield
    O.set_order(0)


@pytest.mark.parametrize("t", [Q4_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, F16, F32])
def test_batched_matmul_is_single_row_matmul(t):
    """Every activation row through the batched path equals its own
    single-row MatMul (TO:60-90) bit for bit, for every weight type, including
    odd row and token counts (partial blocks of 8 rows and 64 tokens)."""
    rng = np.random.default_rng(t)
    K, N, R = 512, 27, 70
    w = blocks(t, N, K, rng)
    a = rng.normal(0, 1, size=(R, K)).astype(np.float32)
    got = O.matmul_rows(a, w, t, K, N)
    for r in range(R):
        want = O.matmul(a[r], w, t, K, N)
        assert np.array_equal(got[r].view(np.uint32), want.view(np.uint32)), r


MINI_Q4KM = dict(arch="llama", hidden=512, layers=2, heads=8, kv_heads=2, head_dim=64, ffn=1024, vocab=1000,
                 rope_base=10000.0, context=700, mix="q4_k_m")
MINI_PHI3 = dict(arch="phi3", hidden=512, layers=2, heads=4, kv_heads=4, head_dim=96, ffn=768, vocab=1000,
                 rope_base=10000.0, context=700, mix="phi3")
MODELS = {"tiny": ("tiny", None), "small5": ("small5", None), "mini_q4km": ("x", MINI_Q4KM),
          "mini_phi3": ("x", MINI_PHI3)}


@pytest.mark.parametrize("kv_fp16", [False, True])
@pytest.mark.parametrize("model", list(MODELS))
def test_prefill_is_the_sequential_loop(model, kv_fp16):
    """A 40-token prompt as two batched calls (15 + 25 tokens) leaves the KV
    cache of every layer and position and the last logits bitwise equal to 40
    sequential ProcessToken calls: Q8_0 (MHA, head_dim 64), Q5_K + Q6_K
    (query groups of 2, head_dim 128), Q4_K + Q6_K (groups of 4), Q6_K + Q8_0
    (MHA, head_dim 96)."""
    name, spec = MODELS[model]
    img = synth.build_image(name, seed=5, spec=spec)
    vocab = (spec or synth.SPECS[name])["vocab"]
    toks = synth.prompt(vocab, 40, seed=3)
    seq = O.Model(img, kv_fp16=kv_fp16, context=64)
    bat = O.Model(img, kv_fp16=kv_fp16, context=64)
    for i, t in enumerate(toks):
        ls = seq.process_token(t, i)
    bat.prefill(toks[:15], 0)
    lb = bat.prefill(toks[15:], 15)
    assert np.array_equal(ls.view(np.uint32), lb.view(np.uint32))
    for layer in range(seq.config.layers):
        for pos in range(40):
            ks, vs = seq.kv_read(layer, pos)
            kb, vb = bat.kv_read(layer, pos)
            assert np.array_equal(ks.view(np.uint32), kb.view(np.uint32)), (layer, pos)
            assert np.array_equal(vs.view(np.uint32), vb.view(np.uint32)), (layer, pos)
    # decoding continues from the batched state exactly as from the sequential one
    assert np.array_equal(seq.process_token(7, 40).view(np.uint32), bat.process_token(7, 40).view(np.uint32))
    seq.close()
    bat.close()


def test_prefill_across_the_chunk_boundary(tiny_image):
    """530 tokens: one 512-token chunk and a second of 18, bitwise the loop."""
    toks = synth.prompt(32000, 530, seed=11)
    seq = O.Model(tiny_image, kv_fp16=False, context=544)
    bat = O.Model(tiny_image, kv_fp16=False, context=544)
    O.set_threads(8)
    try:
        for i, t in enumerate(toks):
            ls = seq.process_token(t, i)
        lb = bat.prefill(toks, 0)
    finally:
        O.set_threads(1)
    assert np.array_equal(ls.view(np.uint32), lb.view(np.uint32))
    for layer in (0, 3):
        for pos in (0, 511, 512, 529):
            assert np.array_equal(np.concatenate(seq.kv_read(layer, pos)), np.concatenate(bat.kv_read(layer, pos)))


@pytest.mark.parametrize("order", [1, 2, 3])
def test_other_orders_are_reorderings(tiny_image, order):
    """Each other order moves the logits (so it measures something), by fp32
    rounding size on the 4-layer model, and differently from the others;
    dequantisation (no reductions) is unchanged; the reference order afterwards
    reproduces the earlier results bit for bit; an order outside 1..3 is the
    reference's."""
    toks = synth.prompt(32000, 24, seed=4)
    m0 = O.Model(tiny_image, kv_fp16=False)
    l0 = m0.prefill(toks, 0)
    outs = {}
    try:
        for o in (1, 2, 3):
            O.set_order(o)
            outs[o] = O.Model(tiny_image, kv_fp16=False).prefill(toks, 0)
        w = blocks(Q4_K, 4, 512, np.random.default_rng(0))
        O.set_order(order)
        d1 = O.dequantize(w, Q4_K, 4, 512)
        O.set_order(7)
        l7 = O.Model(tiny_image, kv_fp16=False).prefill(toks, 0)
    finally:
        O.set_order(0)
    d0 = O.dequantize(w, Q4_K, 4, 512)
    assert np.array_equal(d0.view(np.uint32), d1.view(np.uint32))
    diff = float(np.max(np.abs(outs[order] - l0)))
    assert 0 < diff < 1e-4, diff
    for o in (1, 2, 3):
        if o != order:
            assert not np.array_equal(outs[o].view(np.uint32), outs[order].view(np.uint32))
    assert np.array_equal(l7.view(np.uint32), l0.view(np.uint32))
    again = O.Model(tiny_image, kv_fp16=False).prefill(toks, 0)
    assert np.array_equal(again.view(np.uint32), l0.view(np.uint32))


def _long(key):
    path = os.path.join(HERE, f"long_{key}.npz")
    if not os.path.exists(path):
        pytest.skip(f"{path} not written yet (tests/golden/make_golden.py long {key})")
    z = np.load(path)
    return z, json.loads(str(z["meta"]))


@pytest.mark.parametrize("key", ["c3", "c3h", "c4", "c5", "c5h", "7b64h", "7b64"])
def test_long_fixture_consistent(key):
    """tests/golden/long_<config>.npz: the prompt comes from its seed, the
    model is the stated init, each token is the argmax of its step's stored
    logits (top 256 descending, ties by index, gap = top1 - top2), the sampled
    indices are the generator's, and at the steps whose whole vector is kept
    the top, sampled, mean and RMS entries are that vector's; floors
    non-negative, KV samples finite."""
    from golden.make_golden import INIT, LONG, sample_indices
    z, meta = _long(key)
    name = meta["model"]
    assert meta["init"] == INIT and LONG[key][0] == name and LONG[key][3] == meta["kv_fp16"]
    vocab = synth.SPECS[name]["vocab"]
    assert synth.prompt(vocab, meta["n_prompt"], seed=meta["prompt_seed"]) == z["prompt"].tolist()
    n = meta["n_gen"]
    assert z["tokens"].shape == (n,) and z["top_idx"].shape == (n, 256) and z["floor"].shape == (n,)
    assert np.array_equal(z["sample_idx"], sample_indices(vocab))
    assert z["sample_val"].shape == (n, z["sample_idx"].size)
    assert np.array_equal(z["top_idx"][:, 0], z["tokens"])
    assert np.all(np.diff(z["top_val"], axis=1) <= 0)
    np.testing.assert_allclose(z["gap"], z["top_val"][:, 0] - z["top_val"][:, 1], rtol=0, atol=1e-6)
    assert np.all(z["rms"] >= np.abs(z["mean"])) and np.all(z["floor"] >= 0)
    assert meta["floor_orders"] == [1, 2, 3] and z["floor_by_order"].shape == (n, 3)
    assert np.array_equal(z["floor"], z["floor_by_order"].max(axis=1))
    assert z["full_steps"].tolist() == sorted({0, n - 1})
    for s, row in zip(z["full_steps"], z["full_val"]):
        assert row.shape == (vocab,)
        assert np.array_equal(row[z["top_idx"][s]], z["top_val"][s])
        assert np.array_equal(row[z["sample_idx"]], z["sample_val"][s])
        assert int(np.argmax(row)) == z["tokens"][s]
        r64 = row.astype(np.float64)
        assert r64.mean() == z["mean"][s] and np.sqrt(np.mean(r64 * r64)) == z["rms"][s]
    assert np.all(np.isfinite(z["k"])) and np.all(np.isfinite(z["v"]))


@pytest.mark.parametrize("order", [0, 2])
def test_fused_qkv_is_the_separate_product(order):
    """QkvLayout.Fused (IE:321-332): one MatMul over blk.N.attn_qkv.weight, its
    output split into q, k, v.  Every output row of MatMul is its own dot
    product (TO:60-90), so on the same weights the fused model is the separate
    one bit for bit, in the step, in the batched prompt path and in a
    reordered summation; tiny's matrices are all Q8_0, so the fused image holds
    exactly the separate image's Q, K, V bytes."""
    sep = synth.build_image("tiny", seed=11)
    fus = synth.build_image("tiny", seed=11, fused_qkv=True)
    ms, mf = O.Model(sep), O.Model(fus)
    try:
        O.set_order(order)
        p = synth.prompt(ms.config.vocab, 9, seed=4)
        a, b = ms.prefill(p, 0), mf.prefill(p, 0)
        assert np.array_equal(a, b)
        t = int(np.argmax(a))
        for s in range(5):
            a, b = ms.process_token(t, len(p) + s), mf.process_token(t, len(p) + s)
            assert np.array_equal(a, b), s
            t = int(np.argmax(a))
        for layer in (0, 3):
            for pos in (0, len(p) + 2):
                ka, va = ms.kv_read(layer, pos)
                kb, vb = mf.kv_read(layer, pos)
                assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    finally:
        O.set_order(0)
        ms.close()
        mf.close()


def test_fused_qkv_rows_are_the_three_tensors():
    """The synthetic fused tensor is attn_q, attn_k, attn_v's bytes in that
    order (what the device's row-range views and the equality above assume),
    and the GGUF config reports the fused layout (ArchitectureResolver.cs:145-146)."""
    from dotllm_amd.engine import LoadedModel
    sep = LoadedModel.load(synth.build_image("tiny", seed=11))
    fus = LoadedModel.load(synth.build_image("tiny", seed=11, fused_qkv=True))
    assert fus.config.qkv_fused and not sep.config.qkv_fused
    for layer in (0, 1):
        f = fus.tensor(f"blk.{layer}.attn_qkv.weight")
        parts = [sep.tensor(f"blk.{layer}.attn_{x}.weight") for x in "qkv"]
        assert f.rows == sum(t.rows for t in parts) and f.cols == parts[0].cols
        assert np.array_equal(np.asarray(f.data).reshape(-1),
                              np.concatenate([np.asarray(t.data).reshape(-1) for t in parts]))
