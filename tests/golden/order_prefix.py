"""How far a valid reordering keeps the reference order's greedy tokens.

For the frozen greedy runs (long_<KEY>.npz, written by make_golden.py), runs the
oracle free in each of its three other valid fp32 summation orders
(orc_set_order(1..3)) from the same prompt, and records for each order the
number of leading generated tokens identical to the reference order's.  The
oracle in another order is as valid an implementation of the reference's
arithmetic as any: where it departs early, identity of the whole greedy
sequence is not a property that summation order preserves on that workload.

  python tests/golden/order_prefix.py KEY [KEY ...]   (keys of make_golden.LONG)

Writes (merging with earlier keys) tests/golden/order_prefix.json:
  {KEY: {"orders": [1, 2, 3], "identical": [n1, n2, n3], "n_gen": N,
         "tokens": {order: [...]}}}
"""
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

from dotllm_amd import synth  # noqa: E402
from golden.make_golden import ALT_ORDERS, LONG, image_fingerprint  # noqa: E402
from oracle import oracle as O  # noqa: E402

OUT = os.path.join(HERE, "order_prefix.json")


def free_run(key):
    z = np.load(os.path.join(HERE, f"long_{key}.npz"))
    meta = json.loads(str(z["meta"]))
    name, n_prompt, n_gen, kv_fp16 = LONG[key][:4]
    img = synth.build_image(meta["model"], seed=meta["weights_seed"], context=meta["image_context"])
    assert image_fingerprint(img) == meta["image_fingerprint"], "the synthetic generator changed"
    prompt = z["prompt"].tolist()
    ref = z["tokens"].tolist()
    O.set_threads(int(os.environ.get("ORACLE_THREADS", os.cpu_count() or 1)))
    out = {"orders": list(ALT_ORDERS), "identical": [], "n_gen": n_gen, "tokens": {}}
    t0 = time.time()
    for o in ALT_ORDERS:
        m = O.Model(img, kv_fp16=kv_fp16, context=meta["image_context"])
        try:
            O.set_order(o)
            toks = [O.argmax(m.prefill(prompt, 0))]
            for s in range(1, n_gen):
                toks.append(O.argmax(m.prefill([toks[-1]], n_prompt + s - 1)))
        finally:
            O.set_order(0)
            m.close()
        same = next((i for i, (a, b) in enumerate(zip(toks, ref)) if a != b), n_gen)
        out["identical"].append(same)
        out["tokens"][str(o)] = [int(t) for t in toks]
        print(f"{key}: order {o} identical to the reference order for {same} of {n_gen} tokens "
              f"({time.time() - t0:.0f}s)", flush=True)
    return out


def main(keys):
    res = json.load(open(OUT)) if os.path.exists(OUT) else {}
    for k in keys:
        res[k] = free_run(k)
        with open(OUT, "w") as f:
            json.dump(res, f, indent=1)


if __name__ == "__main__":
    main(sys.argv[1:])
