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


if __name__ == "__main__":
    main()
