"""Writes the golden fixtures under tests/golden/ from the oracle.

The reference (C#/.NET) cannot run here, so end-to-end outputs are pinned by
the oracle's own outputs on seeded synthetic inputs; these fixtures freeze
them, so a later change to the oracle or to the synthetic generator that moves
a result shows up as a test failure.

  python tests/golden/make_golden.py

Outputs (small, committed):
  dequant.npz     per type: 4 rows x 512 columns of random block bytes (finite
                  fp16 scales) and their dequantised values
  gemv.npz        per type: a 32 x 256 weight, an input vector and W x
  tiny_greedy.json  tiny Q8_0 model (seed 1234), 16-token prompt (seed 7):
                  32 greedy tokens and, per step, the top-5 logits and the
                  logits' sum and sum of squares

  python tests/golden/make_golden.py long KEY     (KEY below; 5-60 minutes each)

  long_<KEY>.npz  the full-size workloads and the 7B greedy-64 runs, from the
                  oracle's batched prompt path (orc_prefill, bitwise the
                  sequential loop) with greedy decoding after it; every model
                  is the seeded synthetic image with N(0, 0.02) on every matrix:
                    c3     llama1b,   512-token prompt + 256 tokens, fp32 KV
                    c3h    llama1b,   512-token prompt + 256 tokens, fp16 KV
                    c4     mistral7b, 2048-token prompt + 64 tokens, fp16 KV
                    c5     phi3mini,  2048-token prompt + 256 tokens, fp32 KV
                    c5h    phi3mini,  2048-token prompt + 256 tokens, fp16 KV
                    7b64h  mistral7b, 16-token prompt + 64 tokens, fp16 KV
                    7b64   mistral7b, 16-token prompt + 64 tokens, fp32 KV
                  per step: the top-256 logits, the logits at 4096 fixed
                  indices (sample_indices), the top-2 gap, the logits' mean and
                  root mean square; the whole logits vector at the first and
                  last step; the KV rows of a few (layer, position) pairs; and
                  per step the floor: max |logit difference| over the whole
                  vector between the oracle in the reference's reduction order
                  and in each of three other valid fp32 orders
                  (orc_set_order(1..3)), teacher-forced on the same tokens, the
                  largest of the three (each kept in floor_by_order) -- what
                  summation order alone moves the results by
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from dotllm_amd import F16, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, byte_count, synth  # noqa: E402
from oracle import oracle as O  # noqa: E402

TYPES = {"q4_0": Q4_0, "q8_0": Q8_0, "q4_k": Q4_K, "q5_k": Q5_K, "q6_k": Q6_K, "f16": F16}
SCALE_FIELDS = {Q4_0: (32, 18, [0]), Q8_0: (32, 34, [0]), Q4_K: (256, 144, [0, 2]),
                Q5_K: (256, 176, [0, 2]), Q6_K: (256, 210, [208])}


def random_blocks(t, rows, cols, seed):
    """Random bytes with every fp16 scale field set to a finite value."""
    rng = np.random.default_rng(seed)
    if t == F16:
        return rng.normal(0, 1, size=rows * cols).astype(np.float16).view(np.uint8)
    b = rng.integers(0, 256, size=rows * byte_count(t, cols), dtype=np.uint8)
    be, bb, offs = SCALE_FIELDS[t]
    nblk = rows * cols // be
    for off in offs:
        h = rng.uniform(-2, 2, size=nblk).astype(np.float16).view(np.uint8).reshape(nblk, 2)
        for i in range(nblk):
            b[i * bb + off:i * bb + off + 2] = h[i]
    return b


def main():
    deq, gemv = {}, {}
    for name, t in TYPES.items():
        src = random_blocks(t, 4, 512, 11)
        deq[name + "_src"] = src
        deq[name + "_out"] = O.dequantize(src, t, 4, 512)
        rng = np.random.default_rng(21)
        w = synth.quantize(t, rng.normal(0, 0.05, size=(32, 256)).astype(np.float32))
        x = rng.normal(0, 1, size=256).astype(np.float32)
        gemv[name + "_w"] = w
        gemv[name + "_x"] = x
        gemv[name + "_y"] = O.matmul(x, w, t, 256, 32)
    np.savez_compressed(os.path.join(HERE, "dequant.npz"), **deq)
    np.savez_compressed(os.path.join(HERE, "gemv.npz"), **gemv)

    img = synth.build_image("tiny", seed=1234)
    prompt = synth.prompt(32000, 16, seed=7)
    m = O.Model(img, kv_fp16=False)
    toks, logits = m.generate(prompt, 32, return_logits=True)
    m.close()
    steps = []
    for row in logits:
        top = np.argsort(row)[::-1][:5]
        steps.append({"top5": [int(i) for i in top], "top5_logits": [float(row[i]) for i in top],
                      "sum": float(np.sum(row, dtype=np.float64)),
                      "sumsq": float(np.sum(row.astype(np.float64) ** 2))})
    with open(os.path.join(HERE, "tiny_greedy.json"), "w") as f:
        json.dump({"model": "tiny", "weights_seed": 1234, "prompt_seed": 7, "prompt": [int(t) for t in prompt],
                   "tokens": [int(t) for t in toks], "steps": steps}, f, indent=1)
    print("wrote dequant.npz, gemv.npz, tiny_greedy.json")


def image_fingerprint(img) -> str:
    """SHA-256 over 4 KiB taken every 4 MiB of the image, plus its length."""
    import hashlib
    b = np.asarray(img, dtype=np.uint8).reshape(-1)
    h = hashlib.sha256(str(b.size).encode())
    for off in range(0, b.size, 4 << 20):
        h.update(b[off:off + 4096].tobytes())
    return h.hexdigest()


N_TOP = 256        # logits kept per step: the oracle's top N_TOP ...
N_SAMPLE = 4096    # ... and N_SAMPLE at fixed indices drawn once per vocabulary
INIT = "N(0, 0.02) on every matrix (scaled_init=False), RMSNorm weights 1.0"


def sample_indices(vocab, seed=97):
    """The N_SAMPLE vocabulary indices every step of a fixture stores (sorted)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    return np.sort(rng.choice(vocab, size=min(N_SAMPLE, vocab), replace=False)).astype(np.int32)


def step_stats(row):
    """Top-N_TOP indices and values (descending, ties by index), top-2 gap, mean and RMS of one logits row."""
    top = np.argsort(-row, kind="stable")[:N_TOP]
    r64 = row.astype(np.float64)
    return top, row[top], float(row[top[0]] - row[top[1]]), float(r64.mean()), float(np.sqrt(np.mean(r64 * r64)))


LONG = {
    # name: (model, prompt tokens, generated tokens, fp16 KV, KV sample layers, KV sample positions)
    "c3": ("llama1b", 512, 256, False, (0, 7, 15), (0, 1, 255, 511, 700)),
    "c3h": ("llama1b", 512, 256, True, (0, 7, 15), (0, 1, 255, 511, 700)),
    "c4": ("mistral7b", 2048, 64, True, (0, 15, 31), (0, 1, 1023, 2047, 2100)),
    "c5": ("phi3mini", 2048, 256, False, (0, 15, 31), (0, 1, 1023, 2047, 2250)),
    "c5h": ("phi3mini", 2048, 256, True, (0, 15, 31), (0, 1, 1023, 2047, 2250)),
    "7b64h": ("mistral7b", 16, 64, True, (0, 15, 31), (0, 15, 16, 50, 78)),
    "7b64": ("mistral7b", 16, 64, False, (0, 15, 31), (0, 15, 16, 50, 78)),
}


ALT_ORDERS = (1, 2, 3)   # the other valid fp32 orders the floor is taken over (oracle.h)


def long_run(key):
    """Greedy run of one workload in the reference's order, and the same tokens
    teacher-forced through the oracle in each of ALT_ORDERS for the floor."""
    import time
    name, n_prompt, n_gen, kv_fp16, layers, positions = LONG[key]
    ctx = n_prompt + n_gen + 8
    img = synth.build_image(name, seed=1234, context=ctx)
    vocab = synth.SPECS[name]["vocab"]
    prompt = synth.prompt(vocab, n_prompt, seed=7)
    sidx = sample_indices(vocab)
    O.set_threads(int(os.environ.get("ORACLE_THREADS", os.cpu_count() or 1)))
    orders = (0,) + ALT_ORDERS
    ms = [O.Model(img, kv_fp16=kv_fp16, context=ctx) for _ in orders]
    t0 = time.time()

    def run(tokens, pos0):
        out = []
        try:
            for o, m in zip(orders, ms):
                O.set_order(o)
                out.append(m.prefill(tokens, pos0))
        finally:
            O.set_order(0)
        return out

    ls = run(prompt, 0)
    print(f"{key}: prompt of {n_prompt} in {time.time() - t0:.0f}s", flush=True)
    full_steps = sorted({0, n_gen - 1})
    toks, tidx, tval, sval, gap, mean, rms, floor, full, forders = [], [], [], [], [], [], [], [], [], []
    for s in range(n_gen):
        l0 = ls[0]
        ti, tv, g, mu, r = step_stats(l0)
        tok = O.argmax(l0)
        assert tok == int(ti[0])
        toks.append(tok); tidx.append(ti); tval.append(tv); sval.append(l0[sidx]); gap.append(g)
        mean.append(mu); rms.append(r)
        fo = [float(np.max(np.abs(lk - l0))) for lk in ls[1:]]
        forders.append(fo)
        floor.append(max(fo))
        if s in full_steps:
            full.append(l0.copy())
        if s + 1 < n_gen:
            ls = run([tok], n_prompt + s)
        if s % 16 == 15:
            print(f"{key}: step {s + 1}/{n_gen}, floor so far {max(floor):.3e}, {time.time() - t0:.0f}s", flush=True)
    kv = {}
    for part in ("k", "v"):
        kv[part] = np.zeros((len(layers), len(positions), ms[0].config.kv_heads * ms[0].config.head_dim), np.float32)
        kv[part + "_floor"] = np.zeros((len(layers), len(positions)), np.float32)
    for i, l in enumerate(layers):
        for j, p in enumerate(positions):
            k0, v0 = ms[0].kv_read(l, p)
            kv["k"][i, j], kv["v"][i, j] = k0, v0
            for m in ms[1:]:
                k1, v1 = m.kv_read(l, p)
                kv["k_floor"][i, j] = max(kv["k_floor"][i, j], np.max(np.abs(k1 - k0)))
                kv["v_floor"][i, j] = max(kv["v_floor"][i, j], np.max(np.abs(v1 - v0)))
    for m in ms:
        m.close()
    meta = dict(config=key, model=name, weights_seed=1234, prompt_seed=7, n_prompt=n_prompt, n_gen=n_gen,
                kv_fp16=kv_fp16, image_context=ctx, image_fingerprint=image_fingerprint(img), init=INIT,
                n_top=N_TOP, n_sample=int(sidx.size), sample_seed=97, floor_orders=list(ALT_ORDERS))
    np.savez_compressed(os.path.join(HERE, f"long_{key}.npz"), meta=np.array(json.dumps(meta)),
                        prompt=np.asarray(prompt, np.int32), tokens=np.asarray(toks, np.int32),
                        top_idx=np.asarray(tidx, np.int32), top_val=np.asarray(tval, np.float32),
                        sample_idx=sidx, sample_val=np.asarray(sval, np.float32),
                        full_steps=np.asarray(full_steps, np.int32), full_val=np.asarray(full, np.float32),
                        gap=np.asarray(gap), mean=np.asarray(mean), rms=np.asarray(rms), floor=np.asarray(floor),
                        floor_by_order=np.asarray(forders),
                        kv_layers=np.asarray(layers, np.int32), kv_positions=np.asarray(positions, np.int32), **kv)
    print(f"wrote long_{key}.npz in {time.time() - t0:.0f}s; max floor {max(floor):.3e}", flush=True)


if __name__ == "__main__":
    if len(sys.argv) == 3 and sys.argv[1] == "long":
        long_run(sys.argv[2])
    else:
        main()
