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

  mistral7b_greedy64.json  7B-shape Q4_K_M model (seed 1234), 16-token prompt
                  (seed 7), with fp16 and with fp32 KV: 64 greedy tokens and,
                  per step, the top-16 logits, the top-2 gap, and the logits'
                  mean and root mean square; plus a fingerprint of the image
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


if __name__ == "__main__":
    if sys.argv[1:] == ["mistral7b"]:
        mistral7b_greedy64()
    else:
        main()
