"""The C# package (dotllm_amd/csharp) against the C ABI and the reference's
interface, checked as text (no .NET SDK in this image, so it is not compiled
here):

* Native/HipNative.cs declares every function of include/llmdot_hip.h with the
  same name and parameter count;
* HipBackend implements every member of IComputeBackend
  (src/Llmdot.Core/Inference/Backends/IComputeBackend.cs:7-29: 20 methods, two
  of them overloaded twice, plus IDisposable.Dispose) with the interface's
  parameter counts;
* the patches are unified diffs of the files they name.
"""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CS = os.path.join(ROOT, "dotllm_amd", "csharp")

# IComputeBackend members: name -> parameter counts of its overloads
ICOMPUTE = {"MatMul": [7], "MatMulF32": [6], "RmsNorm": [4], "LayerNorm": [5], "ApplyRoPE": [6, 5],
            "Softmax": [2], "Silu": [2], "SiluInPlace": [1], "Gelu": [2], "GeluScalar": [1], "Add": [2, 3],
            "Scale": [3, 2], "Mul": [3], "Softcap": [2], "Conv1D": [5], "DequantizeToFloat": [5], "ArgMax": [1],
            "Dispose": [0]}


def _params(arglist: str) -> int:
    a = arglist.strip()
    if not a:
        return 0
    depth, n = 0, 1
    for ch in a:
        if ch in "<([":
            depth += 1
        elif ch in ">)]":
            depth -= 1
        elif ch == "," and depth == 0:
            n += 1
    return n


def header_functions():
    text = open(os.path.join(ROOT, "include", "llmdot_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"^\s*(?:const char\*|int32_t)\s+(llmdot_hip_\w+)\s*\(([^;]*?)\)\s*;", text, re.M | re.S):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if args in ("", "void") else _params(args)
    return out


def test_native_declares_every_c_function():
    decl = open(os.path.join(CS, "Llmdot.Hip", "Native", "HipNative.cs")).read()
    found = {m.group(1): _params(m.group(2))
             for m in re.finditer(r"static extern \w+ (llmdot_hip_\w+)\(([^)]*)\);", decl)}
    want = header_functions()
    assert len(want) == 50
    assert found == want


def test_backend_implements_every_interface_member():
    src = open(os.path.join(CS, "Llmdot.Hip", "HipBackend.cs")).read()
    assert re.search(r"class HipBackend : IComputeBackend, IDeviceDecodeBackend", src)
    got = {}
    for m in re.finditer(r"^\s*public (?:[\w<>?\[\], ()]+ )?(\w+)\(([^)]*)\)", src, re.M):
        got.setdefault(m.group(1), []).append(_params(m.group(2)))
    for name, counts in ICOMPUTE.items():
        assert sorted(got.get(name, [])) == sorted(counts), name


def test_patches_are_unified_diffs():
    pd = os.path.join(CS, "patches")
    files = sorted(os.listdir(pd))
    assert files == ["0001-core-device-decoder-hook.patch", "0002-backend-factory-hip.patch"]
    touched = []
    for f in files:
        text = open(os.path.join(pd, f)).read()
        touched += re.findall(r"^\+\+\+ b/(\S+)", text, re.M)
        assert re.search(r"^@@ -\d+(,\d+)? \+\d+(,\d+)? @@", text, re.M)
    assert touched == ["src/Llmdot.Core/Properties/AssemblyInfo.cs",
                       "src/Llmdot.Core/Inference/Backends/IDeviceDecodeBackend.cs",
                       "src/Llmdot.Core/Inference/InferenceEngine.cs",
                       "src/Llmdot.Extensions.AI/BackendFactory.cs",
                       "src/Llmdot.Extensions.AI/Llmdot.Extensions.AI.csproj"]
