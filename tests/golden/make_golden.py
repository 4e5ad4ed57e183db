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

  python tests/golden/make_golden.py mistral7b    (about 20 minutes on 8 cores)
  python tests/golden/make_golden.py floor7b      (adds the order-1 floor to it)
  python tests/golden/make_golden.py long c3|c4|c5   (10-40 minutes each)

  mistral7b_greedy64.json  7B-shape Q4_K_M model (seed 1234), 16-token prompt
                  (seed 7), with fp16 and with fp32 KV: 64 greedy tokens and,
                  per step, the top-16 logits, the top-2 gap, and the logits'
                  mean and root mean square; plus a fingerprint of the image
                  (floor7b adds, per step, the order-1 floor described below)

  long_<config>.npz  the full-size workloads, from the oracle's batched prompt
                  path (orc_prefill, bitwise the sequential loop) with greedy
                  decoding after it:
                    c3  llama1b,   512-token prompt + 256 tokens, fp32 KV
                    c4  mistral7b, 2048-token prompt + 16 tokens, fp16 KV
                    c5  phi3mini,  2048-token prompt + 256 tokens, fp32 KV
                  per step: the top-16 logits, the top-2 gap, the logits' mean
                  and root mean square; the KV rows of a few (layer, position)
                  pairs; and per step the floor: max |logit difference| between
                  the oracle in the reference's reduction order and in another
                  valid fp32 order (orc_set_order(1)), teacher-forced on the same
                  tokens -- what summation order alone moves the results by
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


def mistral7b_greedy64():
    img = synth.build_image("mistral7b", seed=1234, context=96)
    prompt = synth.prompt(32000, 16, seed=7)
    O.set_threads(os.cpu_count() or 1)
    runs = []
    for kv_fp16 in (True, False):
        m = O.Model(img, kv_fp16=kv_fp16, context=96)
        toks, logits = m.generate(prompt, 64, return_logits=True)
        m.close()
        steps = []
        for row in logits:
            top = np.argsort(row)[::-1][:16]
            r64 = row.astype(np.float64)
            steps.append({"top16": [int(i) for i in top], "top16_logits": [float(row[i]) for i in top],
                          "gap": float(row[top[0]] - row[top[1]]), "mean": float(r64.mean()),
                          "rms": float(np.sqrt(np.mean(r64 * r64)))})
        runs.append({"kv_fp16": kv_fp16, "tokens": [int(t) for t in toks], "steps": steps})
        print(f"kv_fp16={kv_fp16}: {len(toks)} tokens", flush=True)
    with open(os.path.join(HERE, "mistral7b_greedy64.json"), "w") as f:
        json.dump({"model": "mistral7b", "weights_seed": 1234, "image_context": 96, "prompt_seed": 7,
                   "prompt": [int(t) for t in prompt], "image_fingerprint": image_fingerprint(img),
                   "runs": runs}, f, indent=1)
    print("wrote mistral7b_greedy64.json")


def step_stats(row):
    """Top-16 indices and values (descending), top-2 gap, mean and RMS of one logits row."""
    top = np.argsort(row, kind="stable")[::-1][:16]
    r64 = row.astype(np.float64)
    return top, row[top], float(row[top[0]] - row[top[1]]), float(r64.mean()), float(np.sqrt(np.mean(r64 * r64)))


LONG = {
    # name: (model, prompt tokens, generated tokens, fp16 KV, KV sample layers, KV sample positions)
    "c3": ("llama1b", 512, 256, False, (0, 7, 15), (0, 1, 255, 511, 700)),
    "c4": ("mistral7b", 2048, 16, True, (0, 15, 31), (0, 1, 1023, 2047, 2060)),
    "c5": ("phi3mini", 2048, 256, False, (0, 15, 31), (0, 1, 1023, 2047, 2250)),
}


def long_run(key):
    """Greedy run of one full-size workload in the reference's order, and the
    same tokens teacher-forced through the order-1 oracle for the floor."""
    import time
    name, n_prompt, n_gen, kv_fp16, layers, positions = LONG[key]
    ctx = n_prompt + n_gen + 8
    img = synth.build_image(name, seed=1234, context=ctx)
    vocab = synth.SPECS[name]["vocab"]
    prompt = synth.prompt(vocab, n_prompt, seed=7)
    O.set_threads(int(os.environ.get("ORACLE_THREADS", os.cpu_count() or 1)))
    m0 = O.Model(img, kv_fp16=kv_fp16, context=ctx)
    m1 = O.Model(img, kv_fp16=kv_fp16, context=ctx)
    t0 = time.time()
    O.set_order(0)
    l0 = m0.prefill(prompt, 0)
    O.set_order(1)
    l1 = m1.prefill(prompt, 0)
    O.set_order(0)
    print(f"{key}: prompt of {n_prompt} in {time.time() - t0:.0f}s", flush=True)
    toks, tidx, tval, gap, mean, rms, floor = [], [], [], [], [], [], []
    for s in range(n_gen):
        ti, tv, g, mu, r = step_stats(l0)
        tok = O.argmax(l0)
        assert tok == int(ti[0])
        toks.append(tok); tidx.append(ti); tval.append(tv); gap.append(g); mean.append(mu); rms.append(r)
        floor.append(float(np.max(np.abs(l1 - l0))))
        if s + 1 < n_gen:
            O.set_order(0)
            l0 = m0.prefill([tok], n_prompt + s)
            O.set_order(1)
            l1 = m1.prefill([tok], n_prompt + s)
            O.set_order(0)
        if s % 16 == 15:
            print(f"{key}: step {s + 1}/{n_gen}, floor so far {max(floor):.3e}, {time.time() - t0:.0f}s", flush=True)
    kv = {}
    for part in ("k", "v"):
        kv[part] = np.zeros((len(layers), len(positions), m0.config.kv_heads * m0.config.head_dim), np.float32)
        kv[part + "_floor"] = np.zeros((len(layers), len(positions)), np.float32)
    for i, l in enumerate(layers):
        for j, p in enumerate(positions):
            k0, v0 = m0.kv_read(l, p)
            k1, v1 = m1.kv_read(l, p)
            kv["k"][i, j], kv["v"][i, j] = k0, v0
            kv["k_floor"][i, j] = np.max(np.abs(k1 - k0))
            kv["v_floor"][i, j] = np.max(np.abs(v1 - v0))
    m0.close(); m1.close()
    meta = dict(config=key, model=name, weights_seed=1234, prompt_seed=7, n_prompt=n_prompt, n_gen=n_gen,
                kv_fp16=kv_fp16, image_context=ctx, image_fingerprint=image_fingerprint(img))
    np.savez_compressed(os.path.join(HERE, f"long_{key}.npz"), meta=np.array(json.dumps(meta)),
                        prompt=np.asarray(prompt, np.int32), tokens=np.asarray(toks, np.int32),
                        top_idx=np.asarray(tidx, np.int32), top_val=np.asarray(tval, np.float32),
                        gap=np.asarray(gap), mean=np.asarray(mean), rms=np.asarray(rms), floor=np.asarray(floor),
                        kv_layers=np.asarray(layers, np.int32), kv_positions=np.asarray(positions, np.int32), **kv)
    print(f"wrote long_{key}.npz in {time.time() - t0:.0f}s; max floor {max(floor):.3e}", flush=True)


def floor7b():
    """Adds to mistral7b_greedy64.json, per step of each run, the order-1 floor:
    the reference-order logits are recomputed through orc_prefill (and must
    equal the fixture's bit for bit), the order-1 logits on the same tokens."""
    path = os.path.join(HERE, "mistral7b_greedy64.json")
    with open(path) as f:
        g = json.load(f)
    img = synth.build_image(g["model"], seed=g["weights_seed"], context=g["image_context"])
    assert image_fingerprint(img) == g["image_fingerprint"]
    O.set_threads(int(os.environ.get("ORACLE_THREADS", os.cpu_count() or 1)))
    prompt = g["prompt"]
    for run in g["runs"]:
        m0 = O.Model(img, kv_fp16=run["kv_fp16"], context=g["image_context"])
        m1 = O.Model(img, kv_fp16=run["kv_fp16"], context=g["image_context"])
        O.set_order(0)
        l0 = m0.prefill(prompt, 0)
        O.set_order(1)
        l1 = m1.prefill(prompt, 0)
        O.set_order(0)
        for s, st in enumerate(run["steps"]):
            top = st["top16"]
            assert [int(i) for i in np.argsort(l0, kind="stable")[::-1][:16]] == top
            assert np.array_equal(l0[top], np.asarray(st["top16_logits"], np.float32)), s
            st["floor"] = float(np.max(np.abs(l1 - l0)))
            if s + 1 < len(run["steps"]):
                tok = run["tokens"][s]
                O.set_order(0)
                l0 = m0.prefill([tok], len(prompt) + s)
                O.set_order(1)
                l1 = m1.prefill([tok], len(prompt) + s)
                O.set_order(0)
        m0.close(); m1.close()
        print(f"kv_fp16={run['kv_fp16']}: max floor {max(st['floor'] for st in run['steps']):.3e}", flush=True)
    with open(path, "w") as f:
        json.dump(g, f, indent=1)
    print("updated mistral7b_greedy64.json")


if __name__ == "__main__":
    if sys.argv[1:] == ["mistral7b"]:
        mistral7b_greedy64()
    elif sys.argv[1:] == ["floor7b"]:
        floor7b()
    elif len(sys.argv) == 3 and sys.argv[1] == "long":
        long_run(sys.argv[2])
    else:
        main()
