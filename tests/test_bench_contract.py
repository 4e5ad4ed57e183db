"""The bench's host-side contract, without a GPU: the one-GPU refusal, the
counter-traffic figure tied to the GEMV source it measured, the prefill FLOP
count and the dominant kernel's label per workload."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402
from dotllm_amd import synth  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout.strip() == ""


def test_traffic_figure_matches_the_current_gemv_source():
    value, note = bench.measured_traffic("mistral7b")
    assert value is not None, note
    assert bench.gemv_source_hash() in note
    # bytes per gate/up launch: within 2% above the algorithmic bytes (no re-reads)
    algorithmic = 2 * 14336 * (4096 // 256) * 144 + 4096 * 4 + 4096 // 8 * 4 + 14336 * 4
    assert algorithmic <= value <= 1.02 * algorithmic


def test_traffic_refused_for_another_gemv_build(tmp_path, monkeypatch):
    src = tmp_path / "gemv.hip"
    src.write_bytes(open(bench.GEMV_SOURCE, "rb").read() + b"\n// changed\n")
    monkeypatch.setattr(bench, "GEMV_SOURCE", str(src))
    value, note = bench.measured_traffic("mistral7b")
    assert value is None and note.startswith("stale")


def test_traffic_only_for_the_profiled_workload():
    value, note = bench.measured_traffic("phi3mini")
    assert value is None and "no counter profile" in note


@pytest.mark.parametrize("name", ["llama1b", "mistral7b", "phi3mini"])
def test_prefill_flops_count(name):
    """2 x (Q, K, V, O, gate, up, down parameters) per token, the causal
    attention (QK^T and PV over n^2 / 2 pairs, two multiply-adds each, per q
    head and layer) and one LM head, counted here from the shapes."""
    s = synth.SPECS[name]
    n = 512
    per_layer = (s["hidden"] * s["heads"] * s["head_dim"] * 2 + s["hidden"] * s["kv_heads"] * s["head_dim"] * 2
                 + 3 * s["hidden"] * s["ffn"])
    want = 2 * per_layer * s["layers"] * n + 2 * (2 * s["head_dim"] * n * n / 2) * s["heads"] * s["layers"] \
        + 2 * s["hidden"] * s["vocab"]
    assert bench.prefill_flops(s, n) == pytest.approx(want, rel=1e-12)


def test_dominant_kernel_label_follows_the_weights():
    labels = {}
    for name in ("mistral7b", "phi3mini"):
        spec = synth.SPECS[name]
        t = {v: k.upper() for k, v in synth.QUANT_NAMES.items()}[synth.tensor_type(spec["mix"], "blk.0.ffn_gate.weight")]
        labels[name] = t
    assert labels == {"mistral7b": "Q4_K", "phi3mini": "Q8_0"}
    src = open(os.path.join(ROOT, "bench.py")).read()
    assert "gemv_kernel<{ffn_type}, SWIGLU, RmsNorm>" in src


def test_every_synthetic_mix_has_a_workload_label():
    """The workload label names the model's real weight mix (the Phi-3-mini
    shape is Q6_K/Q8_0, not Q4_K_M)."""
    for name, spec in synth.SPECS.items():
        assert spec["mix"] in bench.MIX_LABELS, name
    assert bench.MIX_LABELS[synth.SPECS["phi3mini"]["mix"]] == "Q6_K/Q8_0"
    assert bench.MIX_LABELS[synth.SPECS["mistral7b"]["mix"]] == "Q4_K_M"
