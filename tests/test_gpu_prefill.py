"""Parity of the batched (MFMA) prompt path against the oracle.

The reference has no batched path: a prompt is N sequential ProcessToken calls
(InferenceEngine.cs:84-88) and only the KV cache and the last token's logits
are observable.  So the batched GEMM is checked against the oracle's MatMul
with several activation rows (TO:92-111, the dequant-row loop) at the GEMV bar,
and whole prompts against N sequential oracle steps: the KV cache of every
position and the last token's logits at the decode path's logit bars.
"""
import numpy as np
import pytest

from dotllm_amd import Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, byte_count, synth
from dotllm_amd.engine import InferenceEngine, LoadedModel
from oracle import oracle as O
from oracle_pair import KV_MARGIN, OraclePair

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-3      # the spec's GEMV bar
FP32_LEVEL = 2e-5    # what the two-plane fp16 activations and exact block integers give
LOGIT_TOL = 2e-2
KV_MIN = 2e-3        # relative KV bound floor: a few fp16 ulps (the fp16 cache's granularity)
NEAR_TIE = 1e-2


def row_rel_err(y, ref):
    """max over rows of max|y_r - ref_r| / max|ref_r| (rows of ref that are all zero must match exactly)."""
    worst = 0.0
    for yr, rr in zip(y, ref):
        m = float(np.max(np.abs(rr)))
        d = float(np.max(np.abs(yr.astype(np.float64) - rr)))
        if m == 0.0:
            assert d == 0.0
            continue
        worst = max(worst, d / m)
    return worst


def random_blocks(t, rows, cols, seed):
    """Random block bytes with finite fp16 scale fields: every q, sc and m value occurs."""
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, size=rows * byte_count(t, cols), dtype=np.uint8)
    bb = {Q4_K: 144, Q5_K: 176, Q6_K: 210, Q8_0: 34, Q4_0: 18}[t]
    blocks = b.reshape(-1, bb)
    halves = rng.uniform(-2, 2, size=(blocks.shape[0], 2)).astype(np.float16).view(np.uint8)
    if t in (Q4_K, Q5_K):
        blocks[:, 0:4] = halves.reshape(-1, 4)
    elif t == Q6_K:
        blocks[:, 208:210] = halves[:, :2]
    else:
        blocks[:, 0:2] = halves[:, :2]
    return b


SHAPES = [(2, 128, 256), (37, 96, 512), (130, 200, 1024), (257, 384, 2048)]


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K, Q8_0, Q4_0])
@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("kind", ["quantized", "random"])
def test_batched_matmul(hip, t, m, n, k, kind):
    """MatMul with aRows = m: ragged token and row counts, rows of a spanning 1e-3..1e3 and a zero row."""
    rng = np.random.default_rng(m * 7 + n + k)
    if kind == "quantized":
        w = synth.quantize(t, rng.normal(0, 0.02, size=(n, k)).astype(np.float32))
    else:
        w = random_blocks(t, n, k, m + n)
    a = rng.normal(0, 1, size=(m, k)).astype(np.float32)
    a *= (10.0 ** rng.uniform(-3, 3, size=(m, 1))).astype(np.float32)
    a[m // 2] = 0.0
    ref = O.matmul(a, w, t, k, n, result_len=m * n).reshape(m, n)
    y = np.zeros(m * n, dtype=np.float32)
    hip.mat_mul(a.reshape(-1), w, y, t, k, n)
    err = row_rel_err(y.reshape(m, n), ref)
    assert err <= GEMV_TOL
    assert err <= FP32_LEVEL, err


def test_batched_matmul_resident_weight(hip):
    """The weightKey path with several rows: the resident copy feeds the GEMM."""
    n, k, m = 256, 1024, 64
    w = synth.quantize(Q4_K, np.random.default_rng(4).normal(0, 0.02, size=(n, k)).astype(np.float32))
    a = np.random.default_rng(5).normal(0, 1, size=(m, k)).astype(np.float32)
    y1 = np.zeros(m * n, dtype=np.float32)
    hip.mat_mul(a.reshape(-1), w, y1, Q4_K, k, n, weight_key="pf.test.weight")
    y2 = np.zeros(m * n, dtype=np.float32)
    hip.mat_mul(a.reshape(-1), None, y2, Q4_K, k, n, weight_key="pf.test.weight")
    hip.release_weight("pf.test.weight")
    assert np.array_equal(y1, y2)
    ref = O.matmul(a, w, Q4_K, k, n, result_len=m * n)
    assert row_rel_err(y1.reshape(m, n), ref.reshape(m, n)) <= FP32_LEVEL


@pytest.fixture(scope="module")
def oracle_threads():
    O.set_threads(16)
    yield
    O.set_threads(1)


def _kv_err(eng, pair, layer, n):
    """max over positions of |K - K_ref|, |V - V_ref| relative to max |K_ref|, |V_ref|
    of the layer, and the same for the oracle's other-order runs (the floor)."""
    ek = ev = mk = mv = fk = fv = 0.0
    for pos in range(n):
        k, v = eng.kv_read(layer, pos)
        rk, rv = pair.m0.kv_read(layer, pos)
        ek, ev = max(ek, float(np.max(np.abs(k - rk)))), max(ev, float(np.max(np.abs(v - rv))))
        for ok, ov in pair.kv_alt_reads(layer, pos):
            fk, fv = max(fk, float(np.max(np.abs(ok - rk)))), max(fv, float(np.max(np.abs(ov - rv))))
        mk, mv = max(mk, float(np.max(np.abs(rk)))), max(mv, float(np.max(np.abs(rv))))
    return max(ek / mk, ev / mv), max(fk / mk, fv / mv)


def _prompt_check(hip, img, prompt, ctx, kv_fp16, layers, split=None):
    """The batched prompt against the oracle's sequential loop (tests/oracle_pair.py;
    its batched path is bitwise that loop): last logits within max(2e-2, FLOOR_MARGIN x the
    oracle's summation-order floor), KV of every position of the sampled layers
    within max(2e-3, KV_MARGIN x the other orders' largest relative difference), and the next
    decode step from the batched cache within the same logit bound."""
    pair = OraclePair(img, kv_fp16, ctx)
    rl = pair.prefill(prompt, 0)
    eng = InferenceEngine(LoadedModel.load(img), hip, kv_fp16=kv_fp16, context=ctx)
    if split:
        eng.prefill(prompt[:split], 0)
        gl, am = eng.prefill(prompt[split:], split)
    else:
        gl, am = eng.prefill(prompt, 0)
    err = float(np.max(np.abs(gl - rl)))
    top2 = np.sort(rl)[-2:]
    kv = [_kv_err(eng, pair, layer, len(prompt)) for layer in layers]
    # decoding continues from the batched cache as from the sequential one
    nxt = int(np.argmax(rl))
    dl = eng.process_token(nxt, len(prompt))
    rdl = pair.step(nxt, len(prompt))
    bound, tie_at = pair.bounds()
    print(f"prompt {len(prompt)} kv_fp16={kv_fp16}: max |dlogit| {err:.3e} (bound {bound[0]:.3e}), "
          f"KV rel err / floor per layer {[('%.1e' % e, '%.1e' % f) for e, f in kv]}")
    assert err <= bound[0]
    if top2[1] - top2[0] >= tie_at[0]:
        assert am == nxt
    for e, f in kv:
        assert e <= max(KV_MIN, KV_MARGIN * f), (e, f)
    assert float(np.max(np.abs(dl - rdl))) <= bound[1]
    pair.close()
    eng.dispose()


@pytest.mark.parametrize("kv_fp16", [True, False])
def test_prefill_tiny_multi_tile(hip, tiny_image, kv_fp16):
    """tiny Q8_0, MHA head_dim 64: 200 tokens = 2 token tiles, 4 key tiles.
    Every projection launch has under 128 tiles, so Q, K, V and O run in 8 K
    parts and down (44 steps) in 4, summed by the next kernel."""
    prompt = synth.prompt(32000, 200, seed=17)
    _prompt_check(hip, tiny_image, prompt, 256, kv_fp16, [0, 3])


def test_prefill_tiny_no_split(hip, tiny_image, monkeypatch):
    """The same prompt with the K split turned off: every projection one
    launch walking all of K, ragged token and row tiles."""
    monkeypatch.setenv("LLMDOT_HIP_PF_NO_SPLIT", "1")
    prompt = synth.prompt(32000, 200, seed=17)
    _prompt_check(hip, tiny_image, prompt, 256, True, [0, 3])


@pytest.mark.parametrize("kv_fp16,split", [(True, None), (False, None), (True, 1500)])
def test_prefill_tiny_long(hip, tiny_image, kv_fp16, split):
    """2000 tokens through the batched path (one 2048-token chunk: 16 query
    tiles, the heaviest dispatched first, long key loops), and the same prompt
    as two calls with the second at pos0 = 1500, against 2000 oracle steps."""
    img = synth.build_image("tiny", seed=1234, context=2100)
    prompt = synth.prompt(32000, 2000, seed=23)
    _prompt_check(hip, img, prompt, 2100, kv_fp16, [0, 3], split=split)


def test_prefill_tiny_two_calls(hip, tiny_image):
    """A prompt split over two prefill calls (second at pos0 = 77): cached keys plus the chunk."""
    prompt = synth.prompt(32000, 150, seed=18)
    _prompt_check(hip, tiny_image, prompt, 256, True, [0, 3], split=77)


def test_prefill_tiny_small_chunks(hip, tiny_image, monkeypatch):
    """Chunks of 64 tokens (the chunk loop) reproduce the single-chunk result."""
    monkeypatch.setenv("LLMDOT_HIP_PREFILL_CHUNK", "64")
    prompt = synth.prompt(32000, 150, seed=19)
    _prompt_check(hip, tiny_image, prompt, 256, True, [0, 3])


def test_prefill_llama1b(hip, oracle_threads):
    """1B shape, Q4_K_M mix (Q4_K + Q6_K attn_v/head), GQA 32/8, head_dim 64."""
    img = synth.build_image("llama1b", seed=1234, context=96)
    prompt = synth.prompt(128256, 80, seed=7)
    for kv_fp16 in (False, True):
        _prompt_check(hip, img, prompt, 96, kv_fp16, [0, 15])


def test_prefill_small5(hip, oracle_threads):
    """Q5_K_M mix (Q5_K GEMMs on the batched path), GQA 8/4, head_dim 128."""
    img = synth.build_image("small5", seed=1234, context=96)
    prompt = synth.prompt(32000, 80, seed=7)
    for kv_fp16 in (False, True):
        _prompt_check(hip, img, prompt, 96, kv_fp16, [0, 3])


def test_prefill_phi3mini(hip, oracle_threads):
    """Phi-3-mini shape: Q6_K/Q8_0, MHA, head_dim 96."""
    img = synth.build_image("phi3mini", seed=1234, context=32)
    prompt = synth.prompt(32064, 20, seed=7)
    _prompt_check(hip, img, prompt, 32, True, [0, 31])


def test_prefill_mistral7b(hip, oracle_threads):
    """7B shape, Q4_K_M mix, GQA 32/8, head_dim 128."""
    img = synth.build_image("mistral7b", seed=1234, context=32)
    prompt = synth.prompt(32000, 12, seed=7)
    _prompt_check(hip, img, prompt, 32, True, [0, 31])


def test_prefill_64_token_tiles_bit_identical(hip, monkeypatch):
    """1B shape, 1024-token prompt: Q, O and down have 128 tiles of 128 tokens,
    which run as 64-token tiles (Q STORE, O and down ADD into the residual),
    with Q4_K, Q6_K and the min term.  Every output's sum runs in the same
    order as with 128-token tiles, so the last logits and the KV cache must
    be bit-identical with the 64-token tiles turned off."""
    n, ctx = 1024, 1040
    img = synth.build_image("llama1b", seed=1234, context=ctx)
    prompt = synth.prompt(128256, n, seed=29)
    runs = []
    for off in (False, True):
        if off:
            monkeypatch.setenv("LLMDOT_HIP_PF_TM64", "0")
        else:
            monkeypatch.delenv("LLMDOT_HIP_PF_TM64", raising=False)
        eng = InferenceEngine(LoadedModel.load(img), hip, kv_fp16=True, context=ctx)
        try:
            logits, am = eng.prefill(prompt, 0)
            kv = [eng.kv_read(layer, pos) for layer in (0, 7, 15) for pos in (0, 511, 1023)]
        finally:
            eng.dispose()
        runs.append((np.array(logits, copy=True), am, kv))
    (l0, a0, kv0), (l1, a1, kv1) = runs
    assert a0 == a1
    assert np.array_equal(l0, l1), float(np.max(np.abs(l0 - l1)))
    for (k0, v0), (k1, v1) in zip(kv0, kv1):
        assert np.array_equal(k0, k1) and np.array_equal(v0, v1)


def test_prefill_qk_pair_bit_identical(hip, monkeypatch):
    """Phi-3-mini shape (Q and K Q8_0, V Q6_K), 1024-token prompt: Q and K
    (24 row tiles each) run as one launch of 48 row tiles instead of two side
    by side.  Each output's sum runs in the same order either way, so the last
    logits and the KV cache must be bit-identical with the pair turned off."""
    n, ctx = 1024, 1040
    img = synth.build_image("phi3mini", seed=1234, context=ctx)
    prompt = synth.prompt(32064, n, seed=31)
    runs = []
    for off in (False, True):
        if off:
            monkeypatch.setenv("LLMDOT_HIP_PF_QK_PAIR", "0")
        else:
            monkeypatch.delenv("LLMDOT_HIP_PF_QK_PAIR", raising=False)
        eng = InferenceEngine(LoadedModel.load(img), hip, kv_fp16=True, context=ctx)
        try:
            logits, am = eng.prefill(prompt, 0)
            kv = [eng.kv_read(layer, pos) for layer in (0, 15, 31) for pos in (0, 511, 1023)]
        finally:
            eng.dispose()
        runs.append((np.array(logits, copy=True), am, kv))
    (l0, a0, kv0), (l1, a1, kv1) = runs
    assert a0 == a1
    assert np.array_equal(l0, l1), float(np.max(np.abs(l0 - l1)))
    for (k0, v0), (k1, v1) in zip(kv0, kv1):
        assert np.array_equal(k0, k1) and np.array_equal(v0, v1)


@pytest.mark.parametrize("t", [Q8_0, Q4_0])
@pytest.mark.parametrize("k", [96, 160])
def test_batched_matmul_short_k(hip, t, k):
    """32-element block formats with K not a multiple of 128: Q8_0 stages 4
    blocks at a time, so the last stage of each row holds 1 or 3 blocks plus
    bytes past the row (read, never used)."""
    m, n = 130, 200
    rng = np.random.default_rng(k + t)
    w = synth.quantize(t, rng.normal(0, 0.02, size=(n, k)).astype(np.float32))
    a = rng.normal(0, 1, size=(m, k)).astype(np.float32)
    ref = O.matmul(a, w, t, k, n, result_len=m * n).reshape(m, n)
    y = np.zeros(m * n, dtype=np.float32)
    hip.mat_mul(a.reshape(-1), w, y, t, k, n)
    err = row_rel_err(y.reshape(m, n), ref)
    assert err <= FP32_LEVEL, err


@pytest.mark.parametrize("window,split", [(40, None), (100, None), (100, 150), (40, 70)])
def test_prefill_tiny_sliding_window(hip, window, split):
    """SlidingWindow (IE:385-387) in the batched prompt (fp16 KV, the MFMA
    attention): each query attends from its window's start, the Softmax's
    vector lanes counted from there, and a query block starts at the key tile
    of its first query's window.  300 tokens (5 query tiles whose windows start
    in different key tiles), also as two calls (the second at pos0 = split,
    its windows reaching into the cache), against the oracle's loop."""
    img = synth.build_image("tiny", seed=1234, context=400, sliding_window=window)
    prompt = synth.prompt(32000, 300, seed=29)
    _prompt_check(hip, img, prompt, 400, True, [0, 3], split=split)


def test_prefill_small5_sliding_window(hip, oracle_threads):
    """A window of 30 with query groups of 2 (Q5_K_M mix): 80 tokens, fp16 KV."""
    img = synth.build_image("small5", seed=1234, context=96, sliding_window=30)
    _prompt_check(hip, img, synth.prompt(32000, 80, seed=7), 96, True, [0, 3])


@pytest.mark.parametrize("kv_fp16", [True, False])
def test_prefill_qk_norm(hip, oracle_threads, kv_fp16):
    """Per-head Q/K norms (IE:354-373) in the batched prompt: each head's row
    normed in the RoPE/KV pass before its rotation; tiny (MHA) 200 tokens and
    small5 (query groups of 2, fused Q/K/V) 80 tokens, against the oracle."""
    img = synth.build_image("tiny", seed=1234, context=256, qk_norm=True)
    _prompt_check(hip, img, synth.prompt(32000, 200, seed=31), 256, kv_fp16, [0, 3])
    img = synth.build_image("small5", seed=1234, context=96, qk_norm=True, fused_qkv=True)
    _prompt_check(hip, img, synth.prompt(32000, 80, seed=7), 96, kv_fp16, [0, 3])
