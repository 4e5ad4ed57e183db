"""Measurement helpers: the streaming probe (llmdot_hip_stream_bench) and the
counter calibration run.

  python3 -m dotllm_amd.measure calibrate   # 3 reads + 3 writes of 256 MiB (run under
                                            # rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)
  python3 -m dotllm_amd.measure peak        # streaming read / write bandwidth
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


def main(argv) -> int:
    cmd = argv[1] if len(argv) > 1 else "peak"
    be = HipBackend(0)
    try:
        if cmd == "calibrate":
            n = 256 << 20
            for mode, name in ((0, "read"), (1, "write")):
                ms = stream_bench(be, n, mode, 3)
                print(f"{name}: 3 launches of {n} bytes, {3 * n / (ms * 1e-3) / 1e9:.0f} GB/s")
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
