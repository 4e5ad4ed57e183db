"""The oracle's decode-step composition against an independent fp64 NumPy
forward written from the reference source (CPU).

The oracle's parts are pinned one by one (dequantisation bit for bit,
ExpApprox, RmsNorm, RoPE, GEMV in tests/test_oracle.py); this pins how
orc_process_token puts them together: ProcessToken and the LLaMA-like layer
(src/Llmdot.Core/Inference/InferenceEngine.cs:134-146, 184-196), the attention
(IE:304-450: RoPE per head with the precomputed frequencies IE:57-72, KV slots,
q head h reading kv head h / (H / Hkv), scaled scores, Softmax, the value sum),
the SwiGLU FFN (IE:452-476) and the final norm and LM head (IE:575-602).

The forward below is NumPy in float64, sharing nothing with the oracle but the
pinned dequantised weights and the pinned ExpApprox (restated vectorised and
checked against the oracle's).  It follows the reference's structure where the
structure decides the result: ExpApprox on the vector lanes (the first
8 floor(n / 8) elements) and exp on the tail in Softmax and SiLU; float32
rotation angles.  A plausible slip in the oracle -- kv head h % Hkv instead of
h / group, a missing residual, the norm on the wrong tensor, the rotation pair
(i, i + 1) instead of (i, i + half) -- moves the logits by far more than the
bound, which only fp32 rounding must meet.
"""
import numpy as np
import pytest

from dotllm_amd import gguf, synth
from oracle import oracle as O

TOL = 1e-4


def exp_approx(x):
    """VectorMath.ExpApproxVector (VM:137-166) lane by lane in float32."""
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        c = np.minimum(np.maximum(x, np.float32(-87.3)), np.float32(88.4))
        k = np.trunc(c * np.float32(1.4426950408889634) + np.float32(0.5)).astype(np.int32)
        kf = k.astype(np.float32)
        y = (c - kf * np.float32(0.693145751953125)) - kf * np.float32(1.42860677e-6)
        q = (y * y) * np.float32(0.5)
        p = (((np.float32(1) + y) + q) + ((q * y) * np.float32(0.3333333))) + (((q * y) * y) * np.float32(0.2))
        r = p * ((k + 127).astype(np.uint32) << 23).view(np.float32)
    r = np.where(x < np.float32(-87.3), np.float32(0), r)
    return np.where(x > np.float32(88.4), np.float32(np.inf), r)


def lanes_then_tail(n):
    """Elements computed on Vector<float> lanes: the first 8 floor(n / 8)."""
    return np.arange(n) < (n // 8) * 8


class Forward:
    def __init__(self, img, context):
        g = gguf.read(img)
        self.cfg = cfg = gguf.resolve(g)
        self.g = g
        self.W = {}
        for t in g.tensors:
            if t.data is None:
                continue
            w = O.dequantize(t.data, t.ggml_type, t.rows, t.cols).astype(np.float64)
            self.W[t.name] = w.reshape(t.rows, t.cols) if t.rows > 1 else w
        H, Hkv, hd = cfg.head_count, cfg.head_count_kv, cfg.head_dim
        rot = cfg.rope_dimension_count or hd
        half = rot // 2
        # PrecomputeRopeFrequencies (IE:57-72), in float32 as the reference
        i = np.arange(half, dtype=np.float32)
        self.freq = np.float32(1) / np.power(np.float32(cfg.rope_freq_base), np.float32(2) * i / np.float32(rot),
                                             dtype=np.float32)
        self.half, self.H, self.Hkv, self.hd = half, H, Hkv, hd
        L = cfg.layer_count
        self.K = np.zeros((L, context, Hkv, hd))
        self.V = np.zeros((L, context, Hkv, hd))

    def norm(self, x, w):
        return w * x / np.sqrt(np.mean(x * x) + self.cfg.norm_epsilon)

    def rope(self, x, pos):
        a = (np.float32(pos) * self.freq).astype(np.float64)   # the angle in float32, then cos/sin
        c, s = np.cos(a), np.sin(a)
        h = self.half
        x = x.copy()
        x0, x1 = x[..., :h].copy(), x[..., h:2 * h].copy()
        x[..., :h] = x0 * c - x1 * s
        x[..., h:2 * h] = x0 * s + x1 * c
        return x

    def softmax(self, s):
        e = s - s.max()
        vec = lanes_then_tail(len(s))
        e = np.where(vec, exp_approx(e.astype(np.float32)).astype(np.float64), np.exp(e))
        return e / e.sum()

    def silu(self, g):
        vec = lanes_then_tail(len(g))
        d = np.where(vec, exp_approx((-g).astype(np.float32)).astype(np.float64), np.exp(-g))
        return g / (1 + d)

    def step(self, token, pos):
        W, H, Hkv, hd = self.W, self.H, self.Hkv, self.hd
        group = H // Hkv
        x = W["token_embd.weight"][token].copy()
        for l in range(self.cfg.layer_count):
            p = f"blk.{l}."
            h = self.norm(x, W[p + "attn_norm.weight"])
            if p + "attn_qkv.weight" in W:   # fused (IE:321-332): one product, split Q | K | V
                f = W[p + "attn_qkv.weight"] @ h
                q, k, v = f[:H * hd], f[H * hd:(H + Hkv) * hd], f[(H + Hkv) * hd:]
            else:
                q, k, v = W[p + "attn_q.weight"] @ h, W[p + "attn_k.weight"] @ h, W[p + "attn_v.weight"] @ h
            q, k, v = q.reshape(H, hd), k.reshape(Hkv, hd), v.reshape(Hkv, hd)
            # per-head RmsNorm of q and k before RoPE (IE:354-373)
            if p + "attn_q_norm.weight" in W:
                q = np.stack([self.norm(r, W[p + "attn_q_norm.weight"]) for r in q])
            if p + "attn_k_norm.weight" in W:
                k = np.stack([self.norm(r, W[p + "attn_k_norm.weight"]) for r in k])
            q, k = self.rope(q, pos), self.rope(k, pos)
            self.K[l, pos], self.V[l, pos] = k, v
            # SlidingWindow (IE:385-387): the last W positions only
            w = self.cfg.sliding_window
            lo = max(0, pos + 1 - w) if w > 0 else 0
            out = np.zeros((H, hd))
            for hh in range(H):
                kv = hh // group
                sc = self.K[l, lo:pos + 1, kv] @ q[hh] * (1.0 / np.sqrt(hd))
                out[hh] = self.softmax(sc) @ self.V[l, lo:pos + 1, kv]
            x = x + W[p + "attn_output.weight"] @ out.reshape(-1)
            h2 = self.norm(x, W[p + "ffn_norm.weight"])
            a = self.silu(W[p + "ffn_gate.weight"] @ h2) * (W[p + "ffn_up.weight"] @ h2)
            x = x + W[p + "ffn_down.weight"] @ a
        hf = self.norm(x, W["output_norm.weight"])
        out_w = W["output.weight"] if "output.weight" in W else W["token_embd.weight"]
        return out_w @ hf


def test_exp_approx_restatement_matches_oracle():
    xs = np.concatenate([np.linspace(-100, 100, 20001), np.random.default_rng(0).normal(0, 10, 20000)]).astype(np.float32)
    mine = exp_approx(xs)
    theirs = np.array([O.exp_approx(float(v)) for v in xs], dtype=np.float32)
    assert np.array_equal(mine.view(np.uint32), theirs.view(np.uint32))


GQA4 = dict(arch="llama", hidden=512, layers=2, heads=8, kv_heads=2, head_dim=64, ffn=1024, vocab=2000,
            rope_base=500000.0, context=64, mix="q4_k_m")


@pytest.mark.parametrize("name,spec,opts", [("tiny", None, {}), ("small5", None, {}), ("gqa4", GQA4, {}),
                                            ("gqa4", GQA4, dict(qk_norm=True)),
                                            ("small5", None, dict(fused_qkv=True, qk_norm=True)),
                                            ("tiny", None, dict(sliding_window=5))])
def test_process_token_composition(name, spec, opts):
    """16 teacher-forced steps of a random token stream: the oracle's logits
    within 1e-4 of the fp64 forward at every step (MHA head_dim 64 Q8_0;
    query groups of 2 with head_dim 128 and Q5_K/Q6_K; groups of 4 with
    Q4_K/Q6_K and theta 500000; per-head Q/K norms, alone and with fused Q/K/V;
    a sliding window of 5 positions, so 11 of the 16 steps attend to a window
    whose vector lanes start inside the cache)."""
    img = synth.build_image(name if spec is None else "x", seed=31, spec=spec, **opts)
    fw = Forward(img, 32)
    m = O.Model(img, kv_fp16=False, context=32)
    toks = synth.prompt(fw.cfg.vocab_size, 16, seed=5)
    errs = []
    for pos, t in enumerate(toks):
        ref = fw.step(t, pos)
        got = m.process_token(t, pos)
        errs.append(float(np.max(np.abs(got - ref))))
    m.close()
    print(f"{name}: oracle vs fp64 forward, max |dlogit| per step up to {max(errs):.2e}")
    assert max(errs) <= TOL, errs


def test_composition_check_catches_a_gqa_slip():
    """The same comparison with the forward's kv head mapping changed to
    h % Hkv (a plausible slip for grouped queries) fails by orders of
    magnitude: the check above would see such a slip in the oracle."""
    spec = dict(arch="llama", hidden=512, layers=2, heads=8, kv_heads=2, head_dim=64, ffn=1024, vocab=2000,
                rope_base=10000.0, context=64, mix="q4_k_m")
    img = synth.build_image("x", seed=31, spec=spec)

    class Slipped(Forward):
        def step(self, token, pos):
            H, Hkv = self.H, self.Hkv
            W, hd = self.W, self.hd
            x = W["token_embd.weight"][token].copy()
            for l in range(self.cfg.layer_count):
                p = f"blk.{l}."
                h = self.norm(x, W[p + "attn_norm.weight"])
                q = self.rope((W[p + "attn_q.weight"] @ h).reshape(H, hd), pos)
                k = self.rope((W[p + "attn_k.weight"] @ h).reshape(Hkv, hd), pos)
                v = (W[p + "attn_v.weight"] @ h).reshape(Hkv, hd)
                self.K[l, pos], self.V[l, pos] = k, v
                out = np.zeros((H, hd))
                for hh in range(H):
                    kv = hh % Hkv
                    sc = self.K[l, :pos + 1, kv] @ q[hh] * (1.0 / np.sqrt(hd))
                    out[hh] = self.softmax(sc) @ self.V[l, :pos + 1, kv]
                x = x + W[p + "attn_output.weight"] @ out.reshape(-1)
                h2 = self.norm(x, W[p + "ffn_norm.weight"])
                a = self.silu(W[p + "ffn_gate.weight"] @ h2) * (W[p + "ffn_up.weight"] @ h2)
                x = x + W[p + "ffn_down.weight"] @ a
            return W["output.weight"] @ self.norm(x, W["output_norm.weight"])

    fw = Slipped(img, 32)
    m = O.Model(img, kv_fp16=False, context=32)
    errs = [float(np.max(np.abs(m.process_token(t, pos) - fw.step(t, pos))))
            for pos, t in enumerate(synth.prompt(2000, 8, seed=5))]
    m.close()
    assert max(errs) > 100 * TOL, errs
