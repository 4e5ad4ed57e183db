"""Measurement helpers: the streaming probe (llmdot_hip_stream_bench) and the
counter calibration run.

  python3 -m dotllm_amd.measure calibrate   # 3 reads + 3 writes of 256 MiB (run under
                                            # rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)
  python3 -m dotllm_amd.measure peak        # streaming read / write bandwidth
  python3 -m dotllm_amd.measure gemv        # isolated Q4_K / Q6_K GEMVs at the 7B shapes,
                                            # weights cycled through >= 512 MB of copies
  python3 -m dotllm_amd.measure prefill-gemm   # batched Q4_K GEMM 2048 x 14336 x 4096 (MatMul
                                               # with 2048 activation rows), 3 calls
"""
from __future__ import annotations

import ctypes as C
import sys

from ._lib import check, lib
from .backend import HipBackend


def stream_bench(backend: HipBackend, nbytes: int, mode: int, iters: int) -> float:
    """Milliseconds for `iters` launches reading (mode 0) or writing (mode 1) nbytes."""
    ms = C.c_float(0)
    check(lib().llmdot_hip_stream_bench(backend.handle, int(nbytes), int(mode), int(iters), C.byref(ms)))
    return ms.value


def stream_peak_gbps(backend: HipBackend, nbytes: int = 1 << 30, iters: int = 10) -> dict:
    """Practical streaming bandwidth (GB/s) of one read and one write pass over nbytes."""
    out = {}
    for mode, name in ((0, "read"), (1, "write")):
        ms = stream_bench(backend, nbytes, mode, iters)
        out[name] = nbytes * iters / (ms * 1e-3) / 1e9
    return out


# (type, rows, cols, copies): Q4_K 4096x4096, 14336x4096, 4096x14336, the
# 7B gate+up pair as one 28672x4096 matrix, Q+K (5120x4096), and the Q6_K
# LM head and attn_v; copies chosen so every pass reads >= 512 MB (twice the
# 256 MB MALL, so no launch finds its weights there).
GEMV_SHAPES = [(12, 4096, 4096, 55), (12, 14336, 4096, 16), (12, 4096, 14336, 16), (12, 28672, 4096, 8),
               (12, 5120, 4096, 44), (14, 32000, 4096, 5), (14, 1024, 4096, 150)]


def gemv_bench(backend: HipBackend, iters: int = 200) -> list:
    """Isolated GEMV timing through llmdot_hip_time_gemv (STORE, fp32 x)."""
    import numpy as np
    from . import synth
    from ._lib import byte_count
    rng = np.random.default_rng(0)
    h = backend.handle
    out = []
    for t, rows, cols, ncopy in GEMV_SHAPES:
        w = synth.quantize(t, rng.normal(0, 0.02, size=(rows, cols)).astype(np.float32))
        assert w.nbytes == rows * byte_count(t, cols)
        ptrs = []
        try:
            for _ in range(ncopy):
                p = C.c_void_p()
                check(lib().llmdot_hip_device_alloc(h, w.nbytes, C.byref(p)))
                ptrs.append(p)
                check(lib().llmdot_hip_memcpy_h2d(h, p, w.ctypes.data_as(C.c_void_p), w.nbytes))
            x = rng.normal(0, 1, size=cols).astype(np.float32)
            dx, dy = C.c_void_p(), C.c_void_p()
            check(lib().llmdot_hip_device_alloc(h, x.nbytes, C.byref(dx)))
            ptrs.append(dx)
            check(lib().llmdot_hip_device_alloc(h, rows * 4, C.byref(dy)))
            ptrs.append(dy)
            check(lib().llmdot_hip_memcpy_h2d(h, dx, x.ctypes.data_as(C.c_void_p), x.nbytes))
            arr = (C.c_void_p * ncopy)(*[p.value for p in ptrs[:ncopy]])
            ms = C.c_float()
            check(lib().llmdot_hip_time_gemv(h, t, arr, ncopy, dx, dy, rows, cols, 20, C.byref(ms)))
            check(lib().llmdot_hip_time_gemv(h, t, arr, ncopy, dx, dy, rows, cols, iters, C.byref(ms)))
            us = ms.value * 1000.0 / iters
            nbytes = w.nbytes + 4 * (cols + rows)
            out.append({"type": "Q4_K" if t == 12 else "Q6_K", "rows": rows, "cols": cols, "us": us,
                        "bytes": nbytes, "gbps": nbytes / us / 1e3})
        finally:
            for p in ptrs:
                lib().llmdot_hip_device_free(h, p)
    return out


def main(argv) -> int:
    cmd = argv[1] if len(argv) > 1 else "peak"
    be = HipBackend(0)
    try:
        if cmd == "calibrate":
            n = 256 << 20
            for mode, name in ((0, "read"), (1, "write")):
                ms = stream_bench(be, n, mode, 3)
                print(f"{name}: 3 launches of {n} bytes, {3 * n / (ms * 1e-3) / 1e9:.0f} GB/s")
        elif cmd == "gemv":
            for r in gemv_bench(be):
                print(f"{r['type']} {r['rows']}x{r['cols']}: {r['us']:.2f} us/launch, {r['bytes'] / 1e6:.2f} MB, "
                      f"{r['gbps']:.0f} GB/s ({100 * r['gbps'] / 8000:.1f}% of 8 TB/s)")
        elif cmd == "prefill-gemm":
            import numpy as np
            from . import Q4_K, synth
            m, n, k = 2048, 14336, 4096
            rng = np.random.default_rng(0)
            w = synth.quantize(Q4_K, rng.normal(0, 0.02, size=(n, k)).astype(np.float32))
            a = rng.normal(0, 1, size=(m, k)).astype(np.float32)
            y = np.zeros(m * n, dtype=np.float32)
            for _ in range(3):
                be.mat_mul(a.reshape(-1), w, y, Q4_K, k, n, weight_key="measure.prefill_gemm")
            be.release_weight("measure.prefill_gemm")
            print(f"Q4_K GEMM {m}x{n}x{k}: 3 calls, {2.0 * m * n * k / 1e12:.3f} TFLOP each")
        elif cmd == "peak":
            for k, v in stream_peak_gbps(be).items():
                print(f"stream {k}: {v:.0f} GB/s")
        else:
            print(__doc__)
            return 2
    finally:
        be.dispose()
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
